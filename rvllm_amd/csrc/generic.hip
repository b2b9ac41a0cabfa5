// generic.hip - paged attention for the shapes the tuned kernels do not
// take: any head_dim up to 1024, any block size, f16 or f32 cells, any
// number of query rows per sequence. It computes what rvllm's CPU path
// computes for one layer: the padded gather of each sequence's keys
// through its block table, batch_mask and gqa_attention (src/model.rs:
// 346-415, 628-644), here straight over the paged cache.
//
// Row i of sequence b sits at position p = pos_offset[b] + i (decode: the
// one row at read_num[b] - 1) and sees key j iff j < read_num[b], j <= p
// and, with a window, j + window > p: a contiguous range [lo, hi). A row
// that sees no key gets zeros. Keys behind a block id outside the pool are
// skipped (never read).
//
// One wave per (query head, row, sequence). Scores go through LDS in
// chunks of 256 keys, each lane scoring its keys over the whole head
// dimension; then each lane accumulates its own head_dim elements over the
// chunk's probabilities (an online softmax across chunks). Arithmetic is
// f32 throughout: cells are widened exactly, products and sums are f32.
// This is the correctness path for unusual shapes, not a tuned kernel.
#include "pool.h"

#include <cmath>

using rvkv_detail::fail;
using rvkv_detail::hip_fail;

namespace {

constexpr int kChunk = 256;      // keys per LDS chunk
constexpr int kMaxHd = 1024;

struct GenericArgs {
  const float *q;
  float *out;
  const void *kc, *vc;        // this layer's K and V tensors
  const uint32_t *tables;     // [batch][max_blocks]
  const uint32_t *pos_offset; // [batch] or NULL (decode: p = read_num - 1)
  const uint32_t *read_num;   // [batch]
  uint64_t block_stride;      // cells per block (all KV heads)
  uint64_t head_stride;       // cells per (block, KV head)
  uint32_t hd, bs, max_blocks, num_blocks, n_heads, group, q_len;
  uint32_t ctx_cap;           // keys readable through a table row
  float scale;
  int32_t window;
};

template <typename Cell>
__device__ __forceinline__ float cell(const Cell *p, uint64_t i) {
  return (float)p[i];
}

template <typename Cell, int PER>
__global__ void __launch_bounds__(64) generic_attn_kernel(GenericArgs a) {
  __shared__ float qs[kMaxHd];
  __shared__ float ps[kChunk];
  __shared__ uint64_t rows[kChunk];  // cell offset of each key's row, or ~0
  const int lane = threadIdx.x;
  const uint32_t h = blockIdx.x, i = blockIdx.y, b = blockIdx.z;
  const uint32_t kvh = h / a.group;
  const Cell *kc = static_cast<const Cell *>(a.kc);
  const Cell *vc = static_cast<const Cell *>(a.vc);

  const uint32_t rn = min(a.read_num[b], a.ctx_cap);
  // Position of the row; hi/lo bound the keys it sees.
  const uint64_t p = a.pos_offset ? (uint64_t)a.pos_offset[b] + i
                                  : (uint64_t)rn - 1;  // rn 0: sees nothing
  const uint32_t hi = a.pos_offset ? (uint32_t)min<uint64_t>(rn, p + 1) : rn;
  uint32_t lo = 0;
  if (a.window > 0 && p + 1 > (uint64_t)a.window)
    lo = (uint32_t)(p + 1 - (uint64_t)a.window);

  const size_t qrow = (((size_t)b * a.q_len + i) * a.n_heads + h) * a.hd;
  for (uint32_t d = lane; d < a.hd; d += 64) qs[d] = a.q[qrow + d] * a.scale;
  __syncthreads();

  float acc[PER];
#pragma unroll
  for (int r = 0; r < PER; ++r) acc[r] = 0.f;
  float m = -INFINITY, l = 0.f;
  const uint32_t *table = a.tables + (size_t)b * a.max_blocks;

  for (uint32_t c0 = lo; c0 < hi; c0 += kChunk) {
    const uint32_t n = min((uint32_t)kChunk, hi - c0);
    // Scores of this chunk's keys, four per lane.
    float cmax = -INFINITY;
    for (uint32_t k = lane; k < n; k += 64) {
      const uint32_t j = c0 + k;
      const uint32_t blk = table[j / a.bs];
      float s = -INFINITY;
      uint64_t row = ~0ull;
      if (blk < a.num_blocks) {
        row = (uint64_t)blk * a.block_stride + (uint64_t)kvh * a.head_stride +
              (uint64_t)(j % a.bs) * a.hd;
        float x = 0.f;
        for (uint32_t d = 0; d < a.hd; ++d) x = fmaf(qs[d], cell(kc, row + d), x);
        s = x;
      }
      ps[k] = s;
      rows[k] = row;
      cmax = fmaxf(cmax, s);
    }
    for (int off = 32; off > 0; off >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off));
    const float mn = fmaxf(m, cmax);
    if (mn == -INFINITY) {  // nothing readable yet
      __syncthreads();
      continue;
    }
    const float corr = expf(m - mn);  // m = -inf: 0
    float lsum = 0.f;
    for (uint32_t k = lane; k < n; k += 64) {
      const float e = expf(ps[k] - mn);  // skipped keys: 0
      ps[k] = e;
      lsum += e;
    }
    for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off);
    l = l * corr + lsum;
    m = mn;
#pragma unroll
    for (int r = 0; r < PER; ++r) acc[r] *= corr;
    __syncthreads();
    // P.V: lane owns head_dim elements lane, lane + 64, ...
    for (uint32_t k = 0; k < n; ++k) {
      const float pk = ps[k];
      const uint64_t row = rows[k];
      if (row == ~0ull || pk == 0.f) continue;  // (uniform) never read
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        const uint32_t d = lane + 64 * r;
        if (d < a.hd) acc[r] = fmaf(pk, cell(vc, row + d), acc[r]);
      }
    }
    __syncthreads();
  }

  float *o = a.out + qrow;
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const uint32_t d = lane + 64 * r;
    if (d < a.hd) o[d] = l > 0.f ? acc[r] / l : 0.f;
  }
}

template <typename Cell>
void launch_generic(const GenericArgs &a, dim3 grid, hipStream_t st) {
  const uint32_t per = (a.hd + 63) / 64;
  if (per <= 1)
    hipLaunchKernelGGL((generic_attn_kernel<Cell, 1>), grid, dim3(64), 0, st, a);
  else if (per <= 2)
    hipLaunchKernelGGL((generic_attn_kernel<Cell, 2>), grid, dim3(64), 0, st, a);
  else if (per <= 4)
    hipLaunchKernelGGL((generic_attn_kernel<Cell, 4>), grid, dim3(64), 0, st, a);
  else if (per <= 8)
    hipLaunchKernelGGL((generic_attn_kernel<Cell, 8>), grid, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((generic_attn_kernel<Cell, 16>), grid, dim3(64), 0, st, a);
}

}  // namespace

namespace rvkv_detail {

bool generic_head_dim_ok(uint32_t hd) { return hd >= 1 && hd <= kMaxHd; }

int generic_attention(const char *op, const rvkv_pool *pool, uint32_t layer,
                      const float *q, const uint32_t *tables,
                      uint32_t max_blocks, const uint32_t *pos_offset,
                      const uint32_t *read_num, uint32_t batch,
                      uint32_t q_len, uint32_t n_heads, uint32_t ctx_cap,
                      float scale, int32_t window, float *out) {
  if (batch == 0 || q_len == 0) return RVKV_OK;
  if (!generic_head_dim_ok(pool->head_dim))
    return fail(RVKV_EUNSUPPORTED, op, "head_dim must be at most 1024");
  if (batch > 65535 || q_len > 65535 || n_heads > 0x7fffffffu)
    return fail(RVKV_EUNSUPPORTED, op, "batch or q_len too large");
  GenericArgs a{};
  a.q = q;
  a.out = out;
  a.kc = pool->tensor(layer, 0);
  a.vc = pool->tensor(layer, 1);
  a.tables = tables;
  a.pos_offset = pos_offset;
  a.read_num = read_num;
  a.block_stride = pool->block_elems;
  a.head_stride = (uint64_t)pool->block_size * pool->head_dim;
  a.hd = pool->head_dim;
  a.bs = pool->block_size;
  a.max_blocks = max_blocks;
  a.num_blocks = pool->num_blocks;
  a.n_heads = n_heads;
  a.group = n_heads / pool->n_kv;
  a.q_len = q_len;
  const uint64_t cap = (uint64_t)max_blocks * pool->block_size;
  a.ctx_cap = (uint32_t)(cap < ctx_cap ? cap : ctx_cap);
  a.scale = scale;
  a.window = window;
  const dim3 grid(n_heads, q_len, batch);
  if (pool->f32())
    launch_generic<float>(a, grid, pool->stream);
  else
    launch_generic<_Float16>(a, grid, pool->stream);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

}  // namespace rvkv_detail
