// rvkv.hip - MI355X (gfx950) paged KV cache: append, gather, copy-on-write
// block copy and paged GQA decode attention, behind the C ABI of
// include/rvkv.h. Hand-written HIP for CDNA4 (wave64, DPP, fdot2).
//
// Physical cache layout, per layer and per K/V tensor, f16:
//   [num_blocks][n_kv_heads][block_size][head_dim]
// One (block, head) tile is a contiguous block_size*head_dim run, so a
// wavefront reading one KV head of a sequence streams whole 2 KiB+ runs
// (bs 16, hd 64) with 128-bit lane loads. rvllm's logical layout
// [num_blocks, block_size, n_kv_heads, head_dim] (src/kv_storage.rs:7) is
// what gather/read_blocks expose.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "pool.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace rvkv_detail {
int fail(int code, const char *op, const char *reason) {
  g_last_error = std::string(op) + ": " + reason;
  return code;
}

int hip_fail(const char *op, hipError_t e) {
  g_last_error = std::string(op) + ": " + hipGetErrorString(e);
  return RVKV_EHIP;
}
}  // namespace rvkv_detail

using rvkv_detail::fail;
using rvkv_detail::hip_fail;

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2 as_h2(uint32_t x) {
  return __builtin_bit_cast(h2, x);
}
__device__ __forceinline__ uint32_t as_u32(h2 x) {
  return __builtin_bit_cast(uint32_t, x);
}

// 16-byte loads and stores with the non-temporal hint, for bytes that are
// read or written once (K/V streamed by a decode, rows moved by an append,
// a gather or a copy): on this part a plain streaming read of a decode
// launch's size runs ~5 % faster with it, a copy ~6 %. Stores use it only
// where a wave writes whole contiguous runs (attn_prep and the f32 gather,
// whose lanes write two separate halves, measured slower with it).
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
// A wave-uniform word read through the constant address space, so it is a
// scalar load (the kernels also store to global memory, and through a plain
// pointer the compiler may use vector loads). Only for inputs no kernel of
// the launch writes.
__device__ __forceinline__ uint32_t sload(const uint32_t *p) {
  typedef const __attribute__((address_space(4))) uint32_t cu32;
  return *(cu32 *)(uintptr_t)p;
}
__device__ __forceinline__ uint4 sload4(const uint4 *p) {
  typedef const __attribute__((address_space(4))) uint32_t cu32;
  cu32 *q = (cu32 *)(uintptr_t)p;
  return make_uint4(q[0], q[1], q[2], q[3]);
}

__device__ __forceinline__ uint4 load_nt16(const void *p) {
  const u32x4v x = __builtin_nontemporal_load(static_cast<const u32x4v *>(p));
  return make_uint4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ float4 load_nt16f(const void *p) {
  const f32x4v x = __builtin_nontemporal_load(static_cast<const f32x4v *>(p));
  return make_float4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ void store_nt16(void *p, uint4 v) {
  __builtin_nontemporal_store(u32x4v{v.x, v.y, v.z, v.w},
                              static_cast<u32x4v *>(p));
}
__device__ __forceinline__ void store_nt16f(void *p, float4 v) {
  __builtin_nontemporal_store(f32x4v{v.x, v.y, v.z, v.w},
                              static_cast<f32x4v *>(p));
}

}  // namespace


// ---------------------------------------------------------------------------
// KV append. One thread per VW contiguous elements of one (token, head)
// row; VW = 8 (16-byte f16 store) when head_dim % 8 == 0.
// Replaces kv_write.cu (one thread per f32 scalar, 32-bit indices).
// ---------------------------------------------------------------------------
template <int VW, bool SRC_F32>
__global__ void __launch_bounds__(256)
    append_kernel(const void *__restrict__ k, const void *__restrict__ v,
                  const uint32_t *__restrict__ slot_block,
                  const uint32_t *__restrict__ slot_off,
                  uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                  uint32_t n_tokens, uint32_t n_kv, uint32_t hd, uint32_t bs,
                  uint32_t num_blocks, uint64_t src_layer_stride = 0,
                  uint64_t cache_layer_stride = 0, uint32_t tok_group = 1) {
  // blockIdx.y selects a layer (rvkv_append_layers): the source rows and the
  // cache tensors move by their per-layer strides; one layer otherwise.
  if (blockIdx.y) {
    const uint64_t sl = (uint64_t)blockIdx.y * src_layer_stride;
    if constexpr (SRC_F32) {
      k = static_cast<const float *>(k) + sl;
      v = static_cast<const float *>(v) + sl;
    } else {
      k = static_cast<const uint16_t *>(k) + sl;
      v = static_cast<const uint16_t *>(v) + sl;
    }
    kc += (uint64_t)blockIdx.y * cache_layer_stride;
    vc += (uint64_t)blockIdx.y * cache_layer_stride;
  }
  const uint32_t vec_per_row = hd / VW;
  const uint32_t per_token = n_kv * vec_per_row;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t token, head, d;
  if (tok_group <= 1) {
    if (i >= (uint64_t)n_tokens * per_token) return;
    token = (uint32_t)(i / per_token);
    const uint32_t j = (uint32_t)(i - (uint64_t)token * per_token);
    head = j / vec_per_row;
    d = (j - head * vec_per_row) * VW;
  } else {
    // Head-major inside groups of tok_group tokens: consecutive lanes write
    // consecutive rows of one head's tile.
    const uint32_t per_group = tok_group * per_token;
    const uint64_t g = i / per_group;
    const uint32_t w = (uint32_t)(i - g * per_group);
    head = w / (tok_group * vec_per_row);
    const uint32_t r = w - head * (tok_group * vec_per_row);
    const uint32_t t = r / vec_per_row;
    d = (r - t * vec_per_row) * VW;
    const uint64_t tok = g * tok_group + t;
    if (tok >= n_tokens) return;
    token = (uint32_t)tok;
  }
  const uint32_t blk = slot_block[token];
  const uint32_t off = slot_off[token];
  if (blk >= num_blocks || off >= bs) return;  // out-of-range slot: skipped
  const size_t src = (size_t)token * n_kv * hd + (size_t)head * hd + d;
  const size_t dst =
      (((size_t)blk * n_kv + head) * bs + off) * (size_t)hd + d;
  if constexpr (VW == 8) {
    uint4 ko, vo;
    if constexpr (SRC_F32) {
      const float4 *ks = reinterpret_cast<const float4 *>(
          static_cast<const float *>(k) + src);
      const float4 *vs = reinterpret_cast<const float4 *>(
          static_cast<const float *>(v) + src);
      const float4 k0 = load_nt16f(ks), k1 = load_nt16f(ks + 1);
      const float4 v0 = load_nt16f(vs), v1 = load_nt16f(vs + 1);
      // f32 -> f16 round-to-nearest-even (v_cvt_f16_f32, default mode).
      ko.x = as_u32(h2{(_Float16)k0.x, (_Float16)k0.y});
      ko.y = as_u32(h2{(_Float16)k0.z, (_Float16)k0.w});
      ko.z = as_u32(h2{(_Float16)k1.x, (_Float16)k1.y});
      ko.w = as_u32(h2{(_Float16)k1.z, (_Float16)k1.w});
      vo.x = as_u32(h2{(_Float16)v0.x, (_Float16)v0.y});
      vo.y = as_u32(h2{(_Float16)v0.z, (_Float16)v0.w});
      vo.z = as_u32(h2{(_Float16)v1.x, (_Float16)v1.y});
      vo.w = as_u32(h2{(_Float16)v1.z, (_Float16)v1.w});
    } else {
      ko = load_nt16(static_cast<const uint16_t *>(k) + src);
      vo = load_nt16(static_cast<const uint16_t *>(v) + src);
    }
    store_nt16(kc + dst, ko);
    store_nt16(vc + dst, vo);
  } else {
    if constexpr (SRC_F32) {
      kc[dst] = __builtin_bit_cast(
          uint16_t, (_Float16)(static_cast<const float *>(k)[src]));
      vc[dst] = __builtin_bit_cast(
          uint16_t, (_Float16)(static_cast<const float *>(v)[src]));
    } else {
      kc[dst] = static_cast<const uint16_t *>(k)[src];
      vc[dst] = static_cast<const uint16_t *>(v)[src];
    }
  }
}

// f16 rows appended to an f32 cache: every f16 value is exact in f32.
__global__ void __launch_bounds__(256)
    append_widen_kernel(const uint16_t *__restrict__ k,
                        const uint16_t *__restrict__ v,
                        const uint32_t *__restrict__ slot_block,
                        const uint32_t *__restrict__ slot_off,
                        float *__restrict__ kc, float *__restrict__ vc,
                        uint32_t n_tokens, uint32_t n_kv, uint32_t hd,
                        uint32_t bs, uint32_t num_blocks) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t per_token = (uint64_t)n_kv * hd;
  if (i >= n_tokens * per_token) return;
  const uint32_t token = (uint32_t)(i / per_token);
  const uint32_t j = (uint32_t)(i - token * per_token);  // head * hd + d
  const uint32_t blk = slot_block[token], off = slot_off[token];
  if (blk >= num_blocks || off >= bs) return;
  const uint32_t head = j / hd, d = j - head * hd;
  const size_t dst = (((size_t)blk * n_kv + head) * bs + off) * hd + d;
  kc[dst] = (float)__builtin_bit_cast(_Float16, k[i]);
  vc[dst] = (float)__builtin_bit_cast(_Float16, v[i]);
}

// ---------------------------------------------------------------------------
// Block-table gather into rvllm's padded [batch, n_kv, ctx_len, hd].
// Replaces kv_gather.cu. One thread per VW output elements.
// ---------------------------------------------------------------------------
template <int VW, bool OUT_F32>
__global__ void __launch_bounds__(256)
    gather_kernel(const uint16_t *__restrict__ kc,
                  const uint16_t *__restrict__ vc,
                  const uint32_t *__restrict__ block_idx, void *__restrict__ ok,
                  void *__restrict__ ov, uint32_t batch, uint32_t max_blocks,
                  uint32_t ctx_len, uint32_t n_kv, uint32_t hd, uint32_t bs,
                  uint32_t num_blocks) {
  const uint32_t vec_per_row = hd / VW;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t rows = (uint64_t)batch * n_kv * ctx_len;
  if (i >= rows * vec_per_row) return;
  const uint64_t row = i / vec_per_row;  // (b, head, pos)
  const uint32_t d = (uint32_t)(i - row * vec_per_row) * VW;
  const uint32_t pos = (uint32_t)(row % ctx_len);
  const uint64_t bh = row / ctx_len;
  const uint32_t head = (uint32_t)(bh % n_kv);
  const uint32_t b = (uint32_t)(bh / n_kv);
  const uint32_t blk = block_idx[(size_t)b * max_blocks + pos / bs];
  const size_t dst = row * hd + d;
  const bool ok_blk = blk < num_blocks;
  const size_t src =
      (((size_t)(ok_blk ? blk : 0) * n_kv + head) * bs + pos % bs) * hd + d;
  if constexpr (VW == 8) {
    // (plain loads: the padded layout re-reads a sequence's last block for
    // every padding position, and those re-reads hit in L2)
    uint4 kr = ok_blk ? *reinterpret_cast<const uint4 *>(kc + src)
                      : make_uint4(0, 0, 0, 0);
    uint4 vr = ok_blk ? *reinterpret_cast<const uint4 *>(vc + src)
                      : make_uint4(0, 0, 0, 0);
    if constexpr (OUT_F32) {
      float *kf = static_cast<float *>(ok) + dst;
      float *vf = static_cast<float *>(ov) + dst;
      const uint32_t kw[4] = {kr.x, kr.y, kr.z, kr.w};
      const uint32_t vw[4] = {vr.x, vr.y, vr.z, vr.w};
      float ko[8], vo[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h2 kh = as_h2(kw[e]), vh = as_h2(vw[e]);
        ko[2 * e] = (float)kh.x;
        ko[2 * e + 1] = (float)kh.y;
        vo[2 * e] = (float)vh.x;
        vo[2 * e + 1] = (float)vh.y;
      }
      // (plain stores: each lane writes two 16-byte halves of a 32-byte
      // run, and non-temporal stores of such partial lines measured 37 %
      // slower)
      reinterpret_cast<float4 *>(kf)[0] = make_float4(ko[0], ko[1], ko[2], ko[3]);
      reinterpret_cast<float4 *>(kf)[1] = make_float4(ko[4], ko[5], ko[6], ko[7]);
      reinterpret_cast<float4 *>(vf)[0] = make_float4(vo[0], vo[1], vo[2], vo[3]);
      reinterpret_cast<float4 *>(vf)[1] = make_float4(vo[4], vo[5], vo[6], vo[7]);
    } else {
      store_nt16(static_cast<uint16_t *>(ok) + dst, kr);
      store_nt16(static_cast<uint16_t *>(ov) + dst, vr);
    }
  } else {
    uint16_t kr = ok_blk ? kc[src] : 0, vr = ok_blk ? vc[src] : 0;
    if constexpr (OUT_F32) {
      static_cast<float *>(ok)[dst] = (float)__builtin_bit_cast(_Float16, kr);
      static_cast<float *>(ov)[dst] = (float)__builtin_bit_cast(_Float16, vr);
    } else {
      static_cast<uint16_t *>(ok)[dst] = kr;
      static_cast<uint16_t *>(ov)[dst] = vr;
    }
  }
}

// ---------------------------------------------------------------------------
// Attention prep + append. Per (row, head slot) - slots are the
// n_heads q heads, then the n_kv k heads, then the n_kv v heads - T threads
// each hold PPT rotate-half pairs (j, j + HD/2): optional bias, optional
// per-head RMS norm (q and k; sum of squares reduced over the T lanes), RoPE
// with this row's cos/sin (q and k), then q to q_out (f32) and k/v rounded
// to f16 into the row's slot. Mirrors src/model.rs:600-639; the Metal
// attn_prep (attention.metal:8-88) is the reference's own fused version.
// Products and sums are kept unfused (no FMA contraction), as the CPU path
// computes them.
struct PrepArgs {
  const float *q_in, *k_in, *v_in;
  const float *q_bias, *k_bias, *v_bias, *q_norm, *k_norm;
  const float *cos_t, *sin_t;
  const uint32_t *slot_block, *slot_off;
  float *q_out;
  uint16_t *kc, *vc;
  uint32_t rows, n_heads, n_kv, num_blocks, bs;
  uint32_t q_stride, kv_stride;  // elements between consecutive input rows
  uint32_t hd;                   // (read by the generic kernel)
  float eps;
};

__device__ __forceinline__ void ld8(const float *p, float *x) {
  const float4 a = *reinterpret_cast<const float4 *>(p);
  const float4 b = *reinterpret_cast<const float4 *>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ void st8(float *p, const float *x) {
  *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4 *>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
}
__device__ __forceinline__ uint32_t h2bits(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}
__device__ __forceinline__ void st8h(uint16_t *p, const float *x) {
  *reinterpret_cast<uint4 *>(p) = make_uint4(
      h2bits(x[0], x[1]), h2bits(x[2], x[3]), h2bits(x[4], x[5]),
      h2bits(x[6], x[7]));
}

// One item = one (row, head slot): slots [0, n_heads) are q heads, then the
// n_kv k heads, then the n_kv v heads. Each lane owns 8 consecutive
// rotate-half pairs (d, d + HD/2), so every access is 16 bytes wide; the
// T = HD/16 lanes of an item reduce the RMS sum of squares by xor shuffles.
// Element arithmetic is the reference's, unfused (contract off): bias add,
// x / rms * w, then x0*c - x1*s and x0*s + x1*c.
template <int HD>
__global__ void __launch_bounds__(256) attn_prep_kernel(PrepArgs a) {
#pragma clang fp contract(off)
  constexpr int HALF = HD / 2;
  constexpr int V = 8;
  constexpr int T = HALF / V;  // lanes per item: 2, 4, 8, 16
  const uint32_t n_slots = a.n_heads + 2 * a.n_kv;
  const uint32_t item = blockIdx.x * (256 / T) + threadIdx.x / T;
  if (item >= a.rows * n_slots) return;  // whole items exit together
  const int j = (threadIdx.x % T) * V;
  const uint32_t row = item / n_slots;
  const uint32_t slot = item - row * n_slots;
  const bool is_q = slot < a.n_heads;
  const bool is_v = slot >= a.n_heads + a.n_kv;
  const uint32_t hh = is_q ? slot : (is_v ? slot - a.n_heads - a.n_kv
                                          : slot - a.n_heads);
  const float *src = is_q ? a.q_in + (size_t)row * a.q_stride + hh * HD
                          : (is_v ? a.v_in : a.k_in) +
                                (size_t)row * a.kv_stride + hh * HD;
  float x0[V], x1[V];
  ld8(src + j, x0);
  ld8(src + j + HALF, x1);
  const float *bias = is_q ? a.q_bias : (is_v ? a.v_bias : a.k_bias);
  if (bias) {
    float b0[V], b1[V];
    ld8(bias + (size_t)hh * HD + j, b0);
    ld8(bias + (size_t)hh * HD + j + HALF, b1);
#pragma unroll
    for (int p = 0; p < V; ++p) {
      x0[p] = x0[p] + b0[p];
      x1[p] = x1[p] + b1[p];
    }
  }
  const uint32_t blk = a.slot_block[row], off = a.slot_off[row];
  const bool slot_ok = blk < a.num_blocks && off < a.bs;
  const size_t dst = (((size_t)blk * a.n_kv + hh) * a.bs + off) * HD;
  if (is_v) {
    if (slot_ok) {
      st8h(a.vc + dst + j, x0);
      st8h(a.vc + dst + j + HALF, x1);
    }
    return;
  }
  const float *w = is_q ? a.q_norm : a.k_norm;
  if (w) {  // uniform over the T lanes of this item
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < V; ++p) ss = ss + (x0[p] * x0[p] + x1[p] * x1[p]);
#pragma unroll
    for (int o = T / 2; o >= 1; o >>= 1) ss = ss + __shfl_xor(ss, o, T);
    const float rms = sqrtf(ss / (float)HD + a.eps);
    float w0[V], w1[V];
    ld8(w + j, w0);
    ld8(w + j + HALF, w1);
#pragma unroll
    for (int p = 0; p < V; ++p) {
      x0[p] = (x0[p] / rms) * w0[p];
      x1[p] = (x1[p] / rms) * w1[p];
    }
  }
  float c[V], sn[V];
  ld8(a.cos_t + (size_t)row * HALF + j, c);
  ld8(a.sin_t + (size_t)row * HALF + j, sn);
  float r0[V], r1[V];
#pragma unroll
  for (int p = 0; p < V; ++p) {
    r0[p] = x0[p] * c[p] - x1[p] * sn[p];
    r1[p] = x0[p] * sn[p] + x1[p] * c[p];
  }
  if (is_q) {
    float *o = a.q_out + ((size_t)row * a.n_heads + hh) * HD;
    st8(o + j, r0);
    st8(o + j + HALF, r1);
  } else if (slot_ok) {
    st8h(a.kc + dst + j, r0);
    st8h(a.kc + dst + j + HALF, r1);
  }
}

// attn_prep for the shapes attn_prep_kernel does not take (an even head_dim
// other than 32/64/128/256, or f32 cells): one wave per (row, head slot),
// lane i owning the rotate-half pairs (p, p + hd/2) for p = i, i + 64, ...;
// the same element arithmetic, the RMS sum reduced over the wave.
template <typename Cell>
__global__ void __launch_bounds__(64) attn_prep_generic_kernel(PrepArgs a) {
#pragma clang fp contract(off)
  const uint32_t n_slots = a.n_heads + 2 * a.n_kv;
  const uint32_t item = blockIdx.x;
  const uint32_t row = item / n_slots;
  const uint32_t slot = item - row * n_slots;
  const uint32_t HD = a.hd, HALF = HD / 2;
  const uint32_t lane = threadIdx.x;
  const bool is_q = slot < a.n_heads;
  const bool is_v = slot >= a.n_heads + a.n_kv;
  const uint32_t hh = is_q ? slot : (is_v ? slot - a.n_heads - a.n_kv
                                          : slot - a.n_heads);
  const float *src = is_q ? a.q_in + (size_t)row * a.q_stride + (size_t)hh * HD
                          : (is_v ? a.v_in : a.k_in) +
                                (size_t)row * a.kv_stride + (size_t)hh * HD;
  const float *bias = is_q ? a.q_bias : (is_v ? a.v_bias : a.k_bias);
  const float *bh = bias ? bias + (size_t)hh * HD : nullptr;
  const uint32_t blk = a.slot_block[row], off = a.slot_off[row];
  const bool slot_ok = blk < a.num_blocks && off < a.bs;
  const size_t dst = (((size_t)blk * a.n_kv + hh) * a.bs + off) * HD;
  Cell *kc = reinterpret_cast<Cell *>(a.kc);
  Cell *vc = reinterpret_cast<Cell *>(a.vc);
  const float *w = is_v ? nullptr : (is_q ? a.q_norm : a.k_norm);
  float rms = 1.f;
  if (w) {  // (uniform over the wave)
    float ss = 0.f;
    for (uint32_t p = lane; p < HALF; p += 64) {
      const float x0 = bh ? src[p] + bh[p] : src[p];
      const float x1 = bh ? src[p + HALF] + bh[p + HALF] : src[p + HALF];
      ss = ss + (x0 * x0 + x1 * x1);
    }
    for (int o = 32; o >= 1; o >>= 1) ss = ss + __shfl_xor(ss, o);
    rms = sqrtf(ss / (float)HD + a.eps);
  }
  for (uint32_t p = lane; p < HALF; p += 64) {
    float x0 = bh ? src[p] + bh[p] : src[p];
    float x1 = bh ? src[p + HALF] + bh[p + HALF] : src[p + HALF];
    if (is_v) {
      if (slot_ok) {
        vc[dst + p] = (Cell)x0;
        vc[dst + p + HALF] = (Cell)x1;
      }
      continue;
    }
    if (w) {
      x0 = (x0 / rms) * w[p];
      x1 = (x1 / rms) * w[p + HALF];
    }
    const float c = a.cos_t[(size_t)row * HALF + p];
    const float sn = a.sin_t[(size_t)row * HALF + p];
    const float r0 = x0 * c - x1 * sn;
    const float r1 = x0 * sn + x1 * c;
    if (is_q) {
      float *o = a.q_out + ((size_t)row * a.n_heads + hh) * HD;
      o[p] = r0;
      o[p + HALF] = r1;
    } else if (slot_ok) {
      kc[dst + p] = (Cell)r0;
      kc[dst + p + HALF] = (Cell)r1;
    }
  }
}

// ---------------------------------------------------------------------------
// Copy-on-write block copy, every layer, K and V. grid.y = pair,
// grid.z = tensor (2 * n_layers); threads stride over the block's 16-byte
// (or 2-byte) words.
// ---------------------------------------------------------------------------
template <typename W>
__global__ void __launch_bounds__(256)
    copy_blocks_kernel(uint16_t *__restrict__ base,
                       const uint32_t *__restrict__ src,
                       const uint32_t *__restrict__ dst, size_t tensor_elems,
                       size_t block_elems, uint32_t num_blocks) {
  const uint32_t s = sload(src + blockIdx.y), d = sload(dst + blockIdx.y);
  if (s >= num_blocks || d >= num_blocks) return;
  uint16_t *t = base + (size_t)blockIdx.z * tensor_elems;
  const W *from = reinterpret_cast<const W *>(t + (size_t)s * block_elems);
  W *to = reinterpret_cast<W *>(t + (size_t)d * block_elems);
  const size_t words = block_elems * 2 / sizeof(W);
  for (size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x; w < words;
       w += (size_t)gridDim.x * blockDim.x) {
    if constexpr (sizeof(W) == 16)
      store_nt16(to + w, load_nt16(from + w));
    else
      to[w] = from[w];
  }
}

// Logical [n, bs, n_kv, hd] view of listed blocks (test/inspection path).
__global__ void __launch_bounds__(256)
    read_blocks_kernel(const uint16_t *__restrict__ t,
                       const uint32_t *__restrict__ ids, uint32_t n,
                       uint16_t *__restrict__ out, uint32_t bs, uint32_t n_kv,
                       uint32_t hd, uint32_t num_blocks) {
  const size_t per_block = (size_t)bs * n_kv * hd;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= per_block * n) return;
  const uint32_t bi = (uint32_t)(i / per_block);
  const size_t r = i - (size_t)bi * per_block;  // (slot, head, d) logical
  const uint32_t d = (uint32_t)(r % hd);
  const uint32_t head = (uint32_t)((r / hd) % n_kv);
  const uint32_t slot = (uint32_t)(r / ((size_t)hd * n_kv));
  const uint32_t blk = ids[bi];
  out[i] = blk < num_blocks
               ? t[(((size_t)blk * n_kv + head) * bs + slot) * hd + d]
               : (uint16_t)0;
}

// FNV-1a 64 over the logical little-endian bytes of each listed block.
__global__ void __launch_bounds__(64)
    checksum_kernel(const uint16_t *__restrict__ t,
                    const uint32_t *__restrict__ ids, uint32_t n,
                    uint64_t *__restrict__ out, uint32_t bs, uint32_t n_kv,
                    uint32_t hd, uint32_t num_blocks) {
  const uint32_t bi = blockIdx.x * blockDim.x + threadIdx.x;
  if (bi >= n) return;
  const uint32_t blk = ids[bi];
  uint64_t h = 0xcbf29ce484222325ull;
  if (blk < num_blocks) {
    for (uint32_t slot = 0; slot < bs; ++slot)
      for (uint32_t head = 0; head < n_kv; ++head) {
        const uint16_t *row =
            t + (((size_t)blk * n_kv + head) * bs + slot) * hd;
        for (uint32_t d = 0; d < hd; ++d) {
          h = (h ^ (row[d] & 0xffu)) * 0x100000001b3ull;
          h = (h ^ (row[d] >> 8)) * 0x100000001b3ull;
        }
      }
  }
  out[bi] = h;
}

// ---------------------------------------------------------------------------
// Paged GQA decode attention.
//
// Work unit: one wavefront per (sequence, KV head, query sub-group of <= 8
// heads, context partition of P tokens). The wave streams its partition's
// K and V straight through the block table:
//   * a K/V row of head_dim f16 is R = head_dim/8 lanes x 16 bytes, so one
//     wave-wide load covers RPL = 64/R consecutive tokens of ONE block
//     (block_size is a power of two >= RPL): the block id is wave-uniform
//     and lives in an SGPR, every lane issues one 128-bit load;
//   * each group of R lanes ("row group") owns every RPL-th token and keeps
//     its own online-softmax state (running max m, sum l, acc[8] per head)
//     in registers, so the P.V update needs no cross-lane traffic;
//   * q.k: v_dot2_f32_f16 (f16 products, f32 accumulate) over the lane's 8
//     elements, then a DPP butterfly (quad_perm, row_half_mirror,
//     row_mirror) sums the R lanes of the row;
//   * P.V: probabilities rounded to f16 (the running sum l uses the same
//     rounded values, so the normalisation stays consistent), paired over
//     two tokens and fed to v_dot2_f32_f16 against V re-paired with
//     v_perm_b32;
//   * at the end the RPL row groups merge with cross-lane shuffles and the
//     partial (m, l, acc) goes to the workspace, or - when the whole
//     context fits one partition - the normalised output goes straight to
//     `out`.
// Scores are kept in the log2 domain (q pre-scaled by scale*log2(e)) and
// exponentiated with v_exp_f32.
// A second kernel merges the partitions of each (sequence, query head).
// ---------------------------------------------------------------------------
struct DecodeArgs {
  const uint16_t *kc;
  const uint16_t *vc;
  const float *q;
  float *out;
  const uint32_t *tables;
  const uint32_t *ctx_lens;
  // Partial results of split sequences, indexed by (slot * n_heads + head):
  // acc [slots][n_heads][hd], (m, l) [slots][n_heads][2].
  float *ws_acc;
  float *ws_ml;
  // Planned mode: work items {seq, first token, end token, slot} (slot
  // kNoSlot = the item is the whole visible context: write the output) and
  // reduction rows {seq, first slot, slot count, 0}. NULL: uniform mode,
  // where grid.x = partition and slot = seq * n_parts + partition.
  const uint4 *items;
  const uint4 *reds;
  // Fused append (rvkv_decode_step): this step's K/V row of every sequence
  // ([batch, n_kv, hd], f32 or f16) and its slot; NULL for a plain decode.
  const void *new_k;
  const void *new_v;
  const uint32_t *new_blk;
  const uint32_t *new_off;
  int32_t new_f32;
  uint32_t block_size;
  uint64_t block_stride;  // elements per block (all heads)
  uint32_t head_stride;   // elements per (block, head) tile
  uint32_t max_blocks, num_blocks, n_kv, n_heads, group, n_sub;
  uint32_t bs_log2, part_tokens, n_parts, ctx_cap;
  uint32_t hd;  // the cache's head_dim (the kernels' HD is it rounded up)
  uint32_t f32cache;  // cells are f32 (decode_f32_kernel) instead of f16
  float qscale;
  int32_t window;
  // Host-side launch hint (not read by the kernels): average context
  // tokens per workgroup.
  uint32_t avg_tokens;
  // Host-side launch hint: tokens of the longest workgroup.
  uint32_t max_tokens;
  // Host-side: the shape runs the generic kernel (generic.hip).
  uint32_t generic;
};

constexpr uint32_t kNoSlot = 0xFFFFFFFFu;

// A plan item whose seq field has this bit is a shared-prefix group item
// (matrix-core decode only); the other bits locate its member list.
constexpr uint32_t kGroupItem = 0x80000000u;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                         0xF, 0xF, false));
}

// Sum over the R lanes of a row group (R in {2, 4, 8, 16, 32}); every lane of
// the group ends with the total.
template <int R>
__device__ __forceinline__ float row_group_sum(float x) {
  x += dpp<0xB1>(x);  // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (R >= 4) x += dpp<0x4E>(x);  // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (R >= 8) x += dpp<0x141>(x);  // row_half_mirror: 8-lane total
  if constexpr (R >= 16) x += dpp<0x140>(x);  // row_mirror: 16-lane total
  if constexpr (R >= 32) {
    // lane ^ 16: v_permlane16_swap of x with itself leaves rows (0, 2) of x
    // in element 0 and rows (1, 3) in element 1 of every lane, in the VALU
    // (no LDS round trip as for a swizzle).
    const auto r = __builtin_amdgcn_permlane16_swap(
        __builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
        false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    x = __uint_as_float(r0) + __uint_as_float(r1);
  }
  return x;
}

constexpr float kNegBig = -1.0e30f;  // finite "minus infinity" for m

// Zero bytes covering one wave-wide load (64 lanes x 16 B, two loads per
// row at most): the V source of masked keys.
__device__ __align__(16) uint4 g_zero_rows[128];

// Eight f16 of a row at byte address p whose first element is e0 of a
// row of hd elements (RAGGED rows: any head_dim, 2-byte aligned): elements
// at or past hd read as zero.
__device__ __forceinline__ uint4 load_row8(const char *p, uint32_t e0,
                                           uint32_t hd) {
  const uint16_t *q = reinterpret_cast<const uint16_t *>(p);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = e0 + 2 * i < hd ? q[2 * i] : 0u;
    const uint32_t hi = e0 + 2 * i + 1 < hd ? q[2 * i + 1] : 0u;
    w[i] = lo | (hi << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
// The appended row's elements e0..e0+7 (f32 source rounded to f16
// nearest-even, or f16 bits), zero past hd.
__device__ __forceinline__ uint4 new_row8(const void *src, bool f32,
                                          size_t row, uint32_t e0,
                                          uint32_t hd) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint16_t v[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t e = e0 + 2 * i + k;
      if (e >= hd) {
        v[k] = 0;
      } else if (f32) {
        v[k] = __builtin_bit_cast(
            uint16_t, (_Float16) static_cast<const float *>(src)[row + e]);
      } else {
        v[k] = static_cast<const uint16_t *>(src)[row + e];
      }
    }
    w[i] = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ void store_row8(uint16_t *p, uint4 x, uint32_t e0,
                                           uint32_t hd) {
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (e0 + i < hd) p[i] = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
}

// q.k over the lane's NL*8 elements. q is carried as an f16 pair (hi, lo)
// with hi + lo = q to ~2^-22 relative, so the score keeps q's f32 precision
// while every product stays an exact f16 x f16 fdot2 with f32 accumulation
// (K is f16 in the cache, so nothing else is rounded).
template <int NL>
__device__ __forceinline__ float qk_dot(const h2 (&qh)[NL][4],
                                        const h2 (&ql)[NL][4],
                                        const uint4 (&k)[NL]) {
  float d = 0.f;
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    d = __builtin_amdgcn_fdot2(ql[j][0], as_h2(k[j].x), d, false);
    d = __builtin_amdgcn_fdot2(ql[j][1], as_h2(k[j].y), d, false);
    d = __builtin_amdgcn_fdot2(ql[j][2], as_h2(k[j].z), d, false);
    d = __builtin_amdgcn_fdot2(ql[j][3], as_h2(k[j].w), d, false);
  }
#pragma unroll
  for (int j = 0; j < NL; ++j) {
    d = __builtin_amdgcn_fdot2(qh[j][0], as_h2(k[j].x), d, false);
    d = __builtin_amdgcn_fdot2(qh[j][1], as_h2(k[j].y), d, false);
    d = __builtin_amdgcn_fdot2(qh[j][2], as_h2(k[j].z), d, false);
    d = __builtin_amdgcn_fdot2(qh[j][3], as_h2(k[j].w), d, false);
  }
  return d;
}

// Splits x*sc into f16 hi + lo: hi = the f32 product rounded toward zero to
// f16 (one intrinsic, so every use sees the same value; a plain conversion
// may be fused with the product and rounded differently at different uses)
// and lo = the residual of the exact product (fma) rounded to f16.
__device__ __forceinline__ void split_f16(float x0, float x1, float sc, h2 &hi,
                                          h2 &lo) {
  hi = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x0 * sc, x1 * sc));
  lo = h2{(_Float16)__builtin_fmaf(x0, sc, -(float)hi[0]),
          (_Float16)__builtin_fmaf(x1, sc, -(float)hi[1])};
}

// Online-softmax state of one row group for GT query heads: running max m
// (log2 domain), running sum l and acc over the lane's NL*8 elements.
template <int GT, int NL>
struct SoftmaxState {
  float m[GT], l[GT], acc[GT][NL * 8];
};

// One chunk of U wave-wide loads (U*RPL tokens): scores, online softmax
// update and P.V. MASKED handles partial chunks (keys outside [lo, t1) or
// unreadable blocks get probability 0); full chunks skip every test.
// Masked keys are excluded twice: their score becomes -inf (probability 0)
// and, in the caller, their V row is loaded from g_zero_rows instead of the
// cache, so whatever the slot holds (an inf from an overflowing append,
// another sequence's data behind an unreadable block id) never meets a
// zero probability as 0 * inf.
template <int R, int GT, int U, int NL, bool MASKED>
__device__ __forceinline__ void decode_chunk(SoftmaxState<GT, NL> &st,
                                             const h2 (&qh)[GT][NL][4],
                                             const h2 (&ql)[GT][NL][4],
                                             const uint4 (&kr)[U][NL],
                                             const uint4 (&vr)[U][NL],
                                             uint32_t tok0, uint32_t lo,
                                             uint32_t t1, uint32_t okmask,
                                             uint32_t newtok) {
  constexpr int RPL = 64 / R;
  float s[U][GT];
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      s[u][g] = row_group_sum<R>(qk_dot<NL>(qh[g], ql[g], kr[u]));
    }
    if constexpr (MASKED) {
      const uint32_t tok = tok0 + u * RPL;
      // (newtok, the key appended by a fused decode step, is folded in
      // separately from registers.)
      const bool valid =
          ((okmask >> u) & 1u) && tok >= lo && tok < t1 && tok != newtok;
#pragma unroll
      for (int g = 0; g < GT; ++g)
        s[u][g] = valid ? s[u][g] : -__builtin_inff();
    }
  }

  h2 pp[U / 2][GT];  // f16 probabilities, paired over tokens (u, u+1)
  const h2 ones = h2{(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    float mx = st.m[g];
#pragma unroll
    for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u][g]);
    const float corr = __builtin_amdgcn_exp2f(st.m[g] - mx);
    st.m[g] = mx;
    float lsum = st.l[g] * corr;
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      pp[u / 2][g] = h2{(_Float16)__builtin_amdgcn_exp2f(s[u][g] - mx),
                        (_Float16)__builtin_amdgcn_exp2f(s[u + 1][g] - mx)};
      // The sum uses the same rounded probabilities the P.V product does.
      lsum = __builtin_amdgcn_fdot2(pp[u / 2][g], ones, lsum, false);
    }
    st.l[g] = lsum;
#pragma unroll
    for (int e = 0; e < NL * 8; ++e) st.acc[g][e] *= corr;
  }

#pragma unroll
  for (int u = 0; u < U; u += 2) {
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t a0[4] = {vr[u][j].x, vr[u][j].y, vr[u][j].z, vr[u][j].w};
      const uint32_t a1[4] = {vr[u + 1][j].x, vr[u + 1][j].y,
                              vr[u + 1][j].z, vr[u + 1][j].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // (V[u][2w], V[u+1][2w]) and (V[u][2w+1], V[u+1][2w+1])
        const h2 lo2 = as_h2(__builtin_amdgcn_perm(a1[w], a0[w], 0x05040100u));
        const h2 hi2 = as_h2(__builtin_amdgcn_perm(a1[w], a0[w], 0x07060302u));
#pragma unroll
        for (int g = 0; g < GT; ++g) {
          float &x0 = st.acc[g][j * 8 + 2 * w];
          float &x1 = st.acc[g][j * 8 + 2 * w + 1];
          x0 = __builtin_amdgcn_fdot2(pp[u / 2][g], lo2, x0, false);
          x1 = __builtin_amdgcn_fdot2(pp[u / 2][g], hi2, x1, false);
        }
      }
    }
  }
}

// Lane mapping: a K/V row of HD f16 is R = HD/(8*NL) lanes; lane c of a
// row group holds elements (j*R + c)*8 .. +7 for j < NL, so load j of a
// wave covers bytes [j*R*16, (j+1)*R*16) of RPL = 64/R consecutive rows:
// every wave-wide load instruction reads whole contiguous runs.
// Decode kernel: one workgroup of W = blockDim.x/64 wavefronts per
// (sequence, KV head, query sub-group, context partition). The waves take
// the partition's chunks of TC tokens round-robin (wave w: chunks w, w+W,
// ...), so the W waves of a workgroup stream neighbouring tiles together.
// Each wave keeps per-row-group online-softmax state in registers, merges
// its row groups with cross-lane shuffles, then the W wave results merge
// through LDS. A workgroup covering the whole context writes the
// normalised output; otherwise it writes its partial (m, l, acc) and the
// reduction kernel merges the partitions.
template <int HD, int GT, int U, int NL, bool RAGGED>
__global__ void __launch_bounds__(256) decode_part_kernel(
    const uint4 *p_items, const uint32_t *p_tables, const uint32_t *p_ctx,
    uint32_t p_mb, uint32_t p_bs, uint32_t p_pt, DecodeArgs a) {
  // (The start-up chain's inputs come as leading arguments, which the
  // build preloads into SGPRs: no argument load before the first table
  // read. a holds the same values.)
  constexpr int R = HD / (8 * NL);  // lanes per K/V row
  constexpr int RPL = 64 / R;       // rows (tokens) per wave-wide load
  constexpr int TC = U * RPL;       // tokens per chunk
  static_assert(U % 2 == 0, "tokens are paired for the P.V dot2");
  static_assert(R >= 2 && R <= 32, "row must span 2..32 lanes");
  extern __shared__ float lds[];  // [W][GT][HD + 2]

  const int lane = threadIdx.x & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler keep it
  // (and every block id / address derived from it) in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int rg = lane / R;
  const int c = lane % R;
  uint32_t b, t0, tend, slot;
  // (KV head, query sub-group)
  uint32_t hy = blockIdx.y;
  if (p_items) {  // planned: one work item per grid.x
    const uint4 it = sload4(p_items + blockIdx.x);
    b = it.x;
    t0 = it.y;
    tend = it.z;
    slot = it.w;
  } else {  // uniform: fixed-size partitions of every sequence
    b = blockIdx.z;
    t0 = blockIdx.x * p_pt;
    tend = t0 + p_pt;
    slot = a.n_parts > 1 ? b * a.n_parts + blockIdx.x : kNoSlot;
    // Workgroups go to the XCDs round robin by linear id, and with one
    // partition the id is hy + gridDim.y * b. With a batch of whole eights,
    // renumber so a sequence's heads are consecutive workgroups of one XCD:
    // its L2 then asks for all the heads' tiles of each block back to back
    // (Qwen3-0.6B 256 x 4096: 647.2 -> 642.6 us a layer, three alternating
    // runs each). Otherwise rotate hy by the sequence, so each XCD serves
    // every head, not one fixed head's tiles of each block.
    if (gridDim.x == 1 && gridDim.z % 8 == 0) {
      const uint32_t L = blockIdx.y + gridDim.y * blockIdx.z;
      const uint32_t xcd = L % 8, idx = L / 8;
      b = (idx / gridDim.y) * 8 + xcd;
      hy = idx % gridDim.y;
    } else {
      hy = (hy + b) % gridDim.y;
    }
  }
  const uint32_t kvh = hy / a.n_sub;
  const uint32_t sub = hy - kvh * a.n_sub;
  const uint32_t h0 = kvh * a.group + sub * GT;
  const uint32_t ng = min((uint32_t)GT, a.group - sub * GT);
  // Block ids are wave-uniform: read through the constant address space so
  // they are scalar loads into SGPRs (a plain pointer may be reloaded with
  // vector loads, since the kernel also stores to global memory).
  typedef const __attribute__((address_space(4))) uint32_t cu32;
  cu32 *table = (cu32 *)(uintptr_t)(p_tables + (size_t)b * p_mb);
  const uint32_t first = t0 + (uint32_t)wave * TC;  // this wave's 1st chunk

  // The first block ids depend only on the partition: their scalar loads go
  // out together with the ctx_len load (clamped to the table for now).
  const uint32_t mb1 = p_mb - 1;
  uint32_t ids[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    ids[u] = table[min((first + u * RPL) >> p_bs, mb1)];

  // Row length in elements: HD, or (RAGGED) the cache's head_dim, whose
  // lanes past its end hold zeros.
  const uint32_t hdr = RAGGED ? a.hd : HD;
  // q rows of the GT heads (this lane's elements) are loaded up front too.
  float4 qraw[GT][NL][2];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const uint32_t hg = h0 + ((uint32_t)g < ng ? g : 0);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t e0 = (j * R + c) * 8;
      const float *qe = a.q + ((size_t)b * a.n_heads + hg) * hdr + e0;
      if constexpr (RAGGED) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = e0 + i < hdr ? qe[i] : 0.f;
        qraw[g][j][0] = make_float4(x[0], x[1], x[2], x[3]);
        qraw[g][j][1] = make_float4(x[4], x[5], x[6], x[7]);
      } else {
        const float4 *qp = reinterpret_cast<const float4 *>(qe);
        qraw[g][j][0] = qp[0];
        qraw[g][j][1] = qp[1];
      }
    }
  }

  uint32_t ctx = sload(p_ctx + b);
  ctx = min(ctx, a.ctx_cap);
  const uint32_t lo =
      (a.window > 0 && ctx > (uint32_t)a.window) ? ctx - (uint32_t)a.window : 0;
  const uint32_t t1 = min(tend, ctx);
  // A sequence that one partition covers writes its output directly.
  if (!p_items && ctx <= p_pt) slot = kNoSlot;

  if (t0 >= t1) {
    // Past the end of this sequence (the reduction never reads it). An
    // empty sequence (ctx_len 0) gets a zero row from its first partition.
    if (ctx == 0 && t0 == 0 && wave == 0 && rg == 0)
      for (uint32_t g = 0; g < ng; ++g)
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          const uint32_t e0 = (j * R + c) * 8;
          float *oe = a.out + ((size_t)b * a.n_heads + h0 + g) * hdr + e0;
          if constexpr (RAGGED) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
              if (e0 + i < hdr) oe[i] = 0.f;
          } else {
            float4 *o = reinterpret_cast<float4 *>(oe);
            o[0] = make_float4(0.f, 0.f, 0.f, 0.f);
            o[1] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
    return;
  }

  SoftmaxState<GT, NL> st;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    st.m[g] = kNegBig;
    st.l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < NL * 8; ++e) st.acc[g][e] = 0.f;
  }

  // Fused append (rvkv_decode_step): position ctx-1 holds the key appended
  // this step; the workgroup whose range contains it stores the row and
  // folds it in from registers after the main loop.
  const uint32_t newtok = (a.new_k != nullptr && ctx - 1 >= t0 && ctx - 1 < t1)
                              ? ctx - 1
                              : 0xFFFFFFFFu;

  // Chunks are TC tokens from the partition start, taken round-robin by the
  // W waves; the window's lower edge skips whole rounds below it.
  const uint32_t base =
      t0 + (lo > t0 ? (lo - t0) / (TC * W) * (TC * W) : 0);
  const uint32_t start = base + (uint32_t)wave * TC;
  if (start < t1) {
    // q for the GT heads, this lane's elements, pre-scaled, as f16 hi/lo
    // pairs.
    h2 qh[GT][NL][4], ql[GT][NL][4];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const float sc = a.qscale;
        const float4 x0 = qraw[g][j][0], x1 = qraw[g][j][1];
        split_f16(x0.x, x0.y, sc, qh[g][j][0], ql[g][j][0]);
        split_f16(x0.z, x0.w, sc, qh[g][j][1], ql[g][j][1]);
        split_f16(x1.x, x1.y, sc, qh[g][j][2], ql[g][j][2]);
        split_f16(x1.z, x1.w, sc, qh[g][j][3], ql[g][j][3]);
      }
    }

    const uint32_t bs_mask = (1u << p_bs) - 1u;
    const uint32_t last_blk = (ctx - 1) >> p_bs;
    // Byte offsets: the uniform part (block, head, first row of the load)
    // is scalar; the per-lane part is a constant 32-bit offset.
    const char *kbase = reinterpret_cast<const char *>(a.kc) +
                        (size_t)kvh * a.head_stride * 2;
    const char *vbase = reinterpret_cast<const char *>(a.vc) +
                        (size_t)kvh * a.head_stride * 2;
    const uint32_t lane_off = (uint32_t)(rg * hdr * 2 + c * 16);
    const uint64_t blk_bytes = a.block_stride * 2;
    if (start != first || last_blk < ((first + TC - 1) >> p_bs)) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        ids[u] = table[min((start + u * RPL) >> p_bs, last_blk)];
    }

    const char *zero_v = reinterpret_cast<const char *>(g_zero_rows) + lane_off;
    // Issues one chunk's K/V loads into (kr, vr) from block ids `cid`;
    // reports its readable-block mask and whether it is full (no key
    // masked). In a partial chunk, the rows of masked keys are loaded from
    // the zero rows (in the cache) instead of HBM.
    auto issue = [&](uint4 (&kr)[U][NL], uint4 (&vr)[U][NL],
                     const uint32_t (&cid)[U], uint32_t ch, uint32_t &okmask,
                     bool &full) {
      okmask = 0;
#pragma unroll
      for (int u = 0; u < U; ++u)
        okmask |= (uint32_t)(cid[u] < a.num_blocks) << u;
      // The chunk holding this step's appended key takes the masked path,
      // which leaves that key out.
      const bool has_new = newtok >= ch && newtok < ch + TC;
      full = !has_new && ch >= lo && ch + TC <= t1 &&
             okmask == (1u << U) - 1u;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t tb = ch + u * RPL;  // first token of this load
        const bool ok = (okmask >> u) & 1u;
        const uint64_t uoff = (uint64_t)(ok ? cid[u] : 0u) * blk_bytes +
                              (uint64_t)(tb & bs_mask) * (hdr * 2);
        const char *kp = kbase + uoff + lane_off;
        const char *vp = vbase + uoff + lane_off;
        if (!full) {  // (wave-uniform)
          // Rows of masked keys are not read from the cache at all.
          const uint32_t tok = tb + rg;
          const bool valid = ok && tok >= lo && tok < t1 && tok != newtok;
          vp = valid ? vp : zero_v;
          kp = valid ? kp : zero_v;
        }
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          if constexpr (RAGGED) {
            kr[u][j] = load_row8(kp + j * R * 16, (j * R + c) * 8, hdr);
            vr[u][j] = load_row8(vp + j * R * 16, (j * R + c) * 8, hdr);
          } else {
            kr[u][j] = load_nt16(kp + j * R * 16);
            vr[u][j] = load_nt16(vp + j * R * 16);
          }
        }
      }
    };
    auto fetch_ids = [&](uint32_t (&cid)[U], uint32_t ch) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        cid[u] = table[min((ch + u * RPL) >> p_bs, last_blk)];
    };
    auto consume = [&](uint4 (&kr)[U][NL], uint4 (&vr)[U][NL], uint32_t ch,
                       uint32_t okmask, bool full) {
      if (full)
        decode_chunk<R, GT, U, NL, false>(st, qh, ql, kr, vr, ch + rg, lo, t1,
                                          okmask, newtok);
      else
        decode_chunk<R, GT, U, NL, true>(st, qh, ql, kr, vr, ch + rg, lo, t1,
                                         okmask, newtok);
    };
    const uint32_t stride = (uint32_t)W * TC;
    for (uint32_t ch = start; ch < t1; ch += stride) {
      uint4 kr[U][NL], vr[U][NL];
      uint32_t okmask;
      bool full;
      issue(kr, vr, ids, ch, okmask, full);
      // Block ids of this wave's next chunk: scalar loads one chunk ahead.
      fetch_ids(ids, ch + stride);
      consume(kr, vr, ch, okmask, full);
    }

    if (newtok != 0xFFFFFFFFu && wave == 0) {
      // The appended row: round to f16 exactly like append_kernel, store it
      // (sub-group 0, row group 0), and add it to row group 0's softmax
      // state as one more key.
      uint4 nk[NL], nv[NL];
      const size_t src = ((size_t)b * a.n_kv + kvh) * hdr;
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const uint32_t e0 = (j * R + c) * 8;
        if (RAGGED) {
          nk[j] = new_row8(a.new_k, a.new_f32, src, e0, hdr);
          nv[j] = new_row8(a.new_v, a.new_f32, src, e0, hdr);
        } else if (a.new_f32) {
          const float4 *kp = reinterpret_cast<const float4 *>(
              static_cast<const float *>(a.new_k) + src + e0);
          const float4 *vp = reinterpret_cast<const float4 *>(
              static_cast<const float *>(a.new_v) + src + e0);
          const float4 k0 = kp[0], k1 = kp[1], v0 = vp[0], v1 = vp[1];
          nk[j].x = as_u32(h2{(_Float16)k0.x, (_Float16)k0.y});
          nk[j].y = as_u32(h2{(_Float16)k0.z, (_Float16)k0.w});
          nk[j].z = as_u32(h2{(_Float16)k1.x, (_Float16)k1.y});
          nk[j].w = as_u32(h2{(_Float16)k1.z, (_Float16)k1.w});
          nv[j].x = as_u32(h2{(_Float16)v0.x, (_Float16)v0.y});
          nv[j].y = as_u32(h2{(_Float16)v0.z, (_Float16)v0.w});
          nv[j].z = as_u32(h2{(_Float16)v1.x, (_Float16)v1.y});
          nv[j].w = as_u32(h2{(_Float16)v1.z, (_Float16)v1.w});
        } else {
          nk[j] = *reinterpret_cast<const uint4 *>(
              static_cast<const uint16_t *>(a.new_k) + src + e0);
          nv[j] = *reinterpret_cast<const uint4 *>(
              static_cast<const uint16_t *>(a.new_v) + src + e0);
        }
      }
      if (sub == 0 && rg == 0) {
        const uint32_t blk = a.new_blk[b], off = a.new_off[b];
        if (blk < a.num_blocks && off < a.block_size) {
          const size_t dst =
              ((size_t)blk * a.n_kv + kvh) * a.head_stride + (size_t)off * hdr;
          uint16_t *kc = const_cast<uint16_t *>(a.kc);
          uint16_t *vc = const_cast<uint16_t *>(a.vc);
#pragma unroll
          for (int j = 0; j < NL; ++j) {
            const uint32_t e0 = (j * R + c) * 8;
            if constexpr (RAGGED) {
              store_row8(kc + dst + e0, nk[j], e0, hdr);
              store_row8(vc + dst + e0, nv[j], e0, hdr);
            } else {
              *reinterpret_cast<uint4 *>(kc + dst + e0) = nk[j];
              *reinterpret_cast<uint4 *>(vc + dst + e0) = nv[j];
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        const float d = row_group_sum<R>(qk_dot<NL>(qh[g], ql[g], nk));
        if (rg == 0) {
          const float mx = fmaxf(st.m[g], d);
          const float corr = __builtin_amdgcn_exp2f(st.m[g] - mx);
          const _Float16 p = (_Float16)__builtin_amdgcn_exp2f(d - mx);
          st.m[g] = mx;
          st.l[g] = st.l[g] * corr + (float)p;
#pragma unroll
          for (int j = 0; j < NL; ++j) {
            const uint32_t w4[4] = {nv[j].x, nv[j].y, nv[j].z, nv[j].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const h2 vv = as_h2(w4[w]);
              float &x0 = st.acc[g][j * 8 + 2 * w];
              float &x1 = st.acc[g][j * 8 + 2 * w + 1];
              x0 = x0 * corr + (float)p * (float)vv.x;
              x1 = x1 * corr + (float)p * (float)vv.y;
            }
          }
        }
      }
    }

    // Merge the RPL row groups of the wave (lanes c, c+R, c+2R, ...).
#pragma unroll
    for (int g = 0; g < GT; ++g) {
#pragma unroll
      for (int off = R; off < 64; off <<= 1) {
        const float mo = __shfl_xor(st.m[g], off);
        const float lo_ = __shfl_xor(st.l[g], off);
        const float mx = fmaxf(st.m[g], mo);
        const float ws = __builtin_amdgcn_exp2f(st.m[g] - mx);
        const float wo = __builtin_amdgcn_exp2f(mo - mx);
        st.l[g] = st.l[g] * ws + lo_ * wo;
#pragma unroll
        for (int e = 0; e < NL * 8; ++e) {
          const float ao = __shfl_xor(st.acc[g][e], off);
          st.acc[g][e] = st.acc[g][e] * ws + ao * wo;
        }
        st.m[g] = mx;
      }
    }
  }

  // Merge the W waves through LDS: wave w stores (m, l) of each head and
  // its accumulator row; then every thread finishes 4 consecutive elements
  // of one head's output at a time.
  float *ml_s = lds;                                  // [W][GT][2]
  float *acc_s = lds + ((W * GT * 2 + 3) & ~3);       // [W][GT][HD]
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (c == 0) {
        ml_s[(wave * GT + g) * 2] = st.m[g];
        ml_s[(wave * GT + g) * 2 + 1] = st.l[g];
      }
      float4 *r = reinterpret_cast<float4 *>(acc_s + (size_t)(wave * GT + g) * HD);
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const float *x = &st.acc[g][j * 8];
        r[(j * R + c) * 2] = make_float4(x[0], x[1], x[2], x[3]);
        r[(j * R + c) * 2 + 1] = make_float4(x[4], x[5], x[6], x[7]);
      }
    }
  }
  __syncthreads();

  for (int i = threadIdx.x; i < GT * HD / 4; i += blockDim.x) {
    const int g = i / (HD / 4), d = (i - g * (HD / 4)) * 4;
    if ((uint32_t)g >= ng) break;
    float M = kNegBig;
    for (int w = 0; w < W; ++w) M = fmaxf(M, ml_s[(w * GT + g) * 2]);
    float L = 0.f;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = 0; w < W; ++w) {
      const float wt = __builtin_amdgcn_exp2f(ml_s[(w * GT + g) * 2] - M);
      L += ml_s[(w * GT + g) * 2 + 1] * wt;
      const float4 v =
          *reinterpret_cast<const float4 *>(acc_s + (size_t)(w * GT + g) * HD + d);
      x.x += v.x * wt;
      x.y += v.y * wt;
      x.z += v.z * wt;
      x.w += v.w * wt;
    }
    if (slot == kNoSlot) {
      float *o = a.out + ((size_t)b * a.n_heads + h0 + g) * hdr + d;
      // (L is 0 only if every key in range sat behind an unreadable block
      // id: zeros, as for a sequence with nothing to attend to.)
      const float y[4] = {L > 0.f ? x.x / L : 0.f, L > 0.f ? x.y / L : 0.f,
                          L > 0.f ? x.z / L : 0.f, L > 0.f ? x.w / L : 0.f};
      if (!RAGGED) {
        *reinterpret_cast<float4 *>(o) = make_float4(y[0], y[1], y[2], y[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((uint32_t)(d + e) < hdr) o[e] = y[e];
      }
    } else {
      const size_t idx = (size_t)slot * a.n_heads + h0 + g;
      *reinterpret_cast<float4 *>(a.ws_acc + idx * HD + d) = x;
      if (d == 0) {
        a.ws_ml[idx * 2] = M;
        a.ws_ml[idx * 2 + 1] = L;
      }
    }
  }
}

// Decode over an f32 cache (rvllm's own cache dtype): the layout, work
// split, partials and merges of decode_part_kernel, with f32 cells and f32
// arithmetic throughout (q.k and p.v as f32 fmas, probabilities in f32).
// A lane loads 4 cells (16 bytes) per row and load, NL loads per row: R =
// HD / (4 NL) lanes per row, RPL = 64 / R rows per wave-wide load. Masked
// keys load zero rows, as in the f16 kernel.
template <int HD, int GT>
__global__ void __launch_bounds__(256) decode_f32_kernel(DecodeArgs a) {
  constexpr int NL = HD >= 256 ? 2 : 1;
  constexpr int R = HD / (4 * NL);
  constexpr int RPL = 64 / R;
  constexpr int U = 4;
  constexpr int TC = U * RPL;
  static_assert(R >= 2 && R <= 32, "row must span 2..32 lanes");
  extern __shared__ float lds[];  // [W][GT][HD + 2]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int rg = lane / R, c = lane % R;
  uint32_t b, t0, tend, slot;
  uint32_t hy = blockIdx.y;
  if (a.items) {
    const uint4 it = sload4(a.items + blockIdx.x);
    b = it.x;
    t0 = it.y;
    tend = it.z;
    slot = it.w;
  } else {
    b = blockIdx.z;
    t0 = blockIdx.x * a.part_tokens;
    tend = t0 + a.part_tokens;
    slot = a.n_parts > 1 ? b * a.n_parts + blockIdx.x : kNoSlot;
    hy = (hy + b) % gridDim.y;  // (as in the f16 kernel: heads over XCDs)
  }
  const uint32_t kvh = hy / a.n_sub;
  const uint32_t sub = hy - kvh * a.n_sub;
  const uint32_t h0 = kvh * a.group + sub * GT;
  const uint32_t ng = min((uint32_t)GT, a.group - sub * GT);
  typedef const __attribute__((address_space(4))) uint32_t cu32;
  cu32 *table = (cu32 *)(uintptr_t)(a.tables + (size_t)b * a.max_blocks);

  float4 q[GT][NL];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const uint32_t hg = h0 + ((uint32_t)g < ng ? g : 0);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      float4 x = *reinterpret_cast<const float4 *>(
          a.q + ((size_t)b * a.n_heads + hg) * HD + (j * R + c) * 4);
      q[g][j] = make_float4(x.x * a.qscale, x.y * a.qscale, x.z * a.qscale,
                            x.w * a.qscale);
    }
  }
  uint32_t ctx = min(sload(a.ctx_lens + b), a.ctx_cap);
  const uint32_t lo =
      (a.window > 0 && ctx > (uint32_t)a.window) ? ctx - (uint32_t)a.window : 0;
  const uint32_t t1 = min(tend, ctx);
  if (!a.items && ctx <= a.part_tokens) slot = kNoSlot;
  if (t0 >= t1) {
    if (ctx == 0 && t0 == 0 && wave == 0 && rg == 0)
      for (uint32_t g = 0; g < ng; ++g)
#pragma unroll
        for (int j = 0; j < NL; ++j)
          *reinterpret_cast<float4 *>(a.out + ((size_t)b * a.n_heads + h0 + g) *
                                                  HD + (j * R + c) * 4) =
              make_float4(0.f, 0.f, 0.f, 0.f);
    return;
  }

  float m[GT], l[GT], acc[GT][NL * 4];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < NL * 4; ++e) acc[g][e] = 0.f;
  }
  const uint32_t first = t0 + (uint32_t)wave * TC;
  const uint32_t stride = (uint32_t)W * TC;
  const uint32_t skip = lo > t0 ? (lo - t0) / stride * stride : 0;
  const uint32_t bs_mask = (1u << a.bs_log2) - 1u;
  const uint32_t last_blk = (ctx - 1) >> a.bs_log2;
  const char *kbase =
      reinterpret_cast<const char *>(a.kc) + (size_t)kvh * a.head_stride * 4;
  const char *vbase =
      reinterpret_cast<const char *>(a.vc) + (size_t)kvh * a.head_stride * 4;
  const uint32_t lane_off = (uint32_t)(rg * HD * 4 + c * 16);
  const char *zero_v = reinterpret_cast<const char *>(g_zero_rows) + lane_off;
  const uint64_t blk_bytes = a.block_stride * 4;
  // Fused append (rvkv_decode_step): position ctx - 1 holds the row appended
  // this step; the workgroup whose range holds it skips that key in the
  // loop, stores the row and folds it in from registers afterwards.
  const uint32_t newtok = (a.new_k != nullptr && ctx - 1 >= t0 && ctx - 1 < t1)
                              ? ctx - 1
                              : 0xFFFFFFFFu;
  for (uint32_t ch = first + skip; ch < t1; ch += stride) {
    float4 kr[U][NL], vr[U][NL];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t tb = ch + u * RPL;
      const uint32_t id = table[min(tb >> a.bs_log2, last_blk)];
      const uint32_t tok = tb + rg;
      valid[u] = id < a.num_blocks && tok >= lo && tok < t1 && tok != newtok;
      const char *row = (uint64_t)(id < a.num_blocks ? id : 0u) * blk_bytes +
                        (uint64_t)(tb & bs_mask) * (HD * 4) + lane_off + kbase;
      const char *kp = valid[u] ? row : zero_v;
      const char *vp = valid[u] ? row - kbase + vbase : zero_v;
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        const uint4 kb = load_nt16(kp + j * R * 16);
        const uint4 vb = load_nt16(vp + j * R * 16);
        kr[u][j] = make_float4(__uint_as_float(kb.x), __uint_as_float(kb.y),
                               __uint_as_float(kb.z), __uint_as_float(kb.w));
        vr[u][j] = make_float4(__uint_as_float(vb.x), __uint_as_float(vb.y),
                               __uint_as_float(vb.z), __uint_as_float(vb.w));
      }
    }
    // Keep the chunk's loads issued together ahead of the math (without
    // this fence the scheduler may pair each load with its first use).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float s[U];
      float mx = m[g];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float d = 0.f;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          d = __builtin_fmaf(q[g][j].x, kr[u][j].x, d);
          d = __builtin_fmaf(q[g][j].y, kr[u][j].y, d);
          d = __builtin_fmaf(q[g][j].z, kr[u][j].z, d);
          d = __builtin_fmaf(q[g][j].w, kr[u][j].w, d);
        }
        d = row_group_sum<R>(d);
        s[u] = valid[u] ? d : -__builtin_inff();
        mx = fmaxf(mx, s[u]);
      }
      const float corr = __builtin_amdgcn_exp2f(m[g] - mx);
      m[g] = mx;
      l[g] *= corr;
#pragma unroll
      for (int e = 0; e < NL * 4; ++e) acc[g][e] *= corr;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float pu = __builtin_amdgcn_exp2f(s[u] - mx);
        l[g] += pu;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          acc[g][j * 4 + 0] = __builtin_fmaf(pu, vr[u][j].x, acc[g][j * 4 + 0]);
          acc[g][j * 4 + 1] = __builtin_fmaf(pu, vr[u][j].y, acc[g][j * 4 + 1]);
          acc[g][j * 4 + 2] = __builtin_fmaf(pu, vr[u][j].z, acc[g][j * 4 + 2]);
          acc[g][j * 4 + 3] = __builtin_fmaf(pu, vr[u][j].w, acc[g][j * 4 + 3]);
        }
      }
    }
  }
  if (newtok != 0xFFFFFFFFu && wave == 0) {
    // The appended row (f32 source copied, f16 widened exactly, as the
    // append does): stored by sub-group 0's row group 0, and one more key
    // of row group 0's softmax state.
    float4 nk[NL], nv[NL];
    const size_t src = ((size_t)b * a.n_kv + kvh) * HD;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const uint32_t e0 = (j * R + c) * 4;
      if (a.new_f32) {
        nk[j] = *reinterpret_cast<const float4 *>(
            static_cast<const float *>(a.new_k) + src + e0);
        nv[j] = *reinterpret_cast<const float4 *>(
            static_cast<const float *>(a.new_v) + src + e0);
      } else {
        const uint2 kh = *reinterpret_cast<const uint2 *>(
            static_cast<const uint16_t *>(a.new_k) + src + e0);
        const uint2 vh = *reinterpret_cast<const uint2 *>(
            static_cast<const uint16_t *>(a.new_v) + src + e0);
        const h2 k01 = as_h2(kh.x), k23 = as_h2(kh.y);
        const h2 v01 = as_h2(vh.x), v23 = as_h2(vh.y);
        nk[j] = make_float4((float)k01.x, (float)k01.y, (float)k23.x,
                            (float)k23.y);
        nv[j] = make_float4((float)v01.x, (float)v01.y, (float)v23.x,
                            (float)v23.y);
      }
    }
    if (sub == 0 && rg == 0) {
      const uint32_t nb = a.new_blk[b], no = a.new_off[b];
      if (nb < a.num_blocks && no < a.block_size) {
        const size_t dst = (size_t)nb * a.block_stride +
                           (size_t)kvh * a.head_stride + (size_t)no * HD;
        float *kc = reinterpret_cast<float *>(const_cast<uint16_t *>(a.kc));
        float *vc = reinterpret_cast<float *>(const_cast<uint16_t *>(a.vc));
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          const uint32_t e0 = (j * R + c) * 4;
          *reinterpret_cast<float4 *>(kc + dst + e0) = nk[j];
          *reinterpret_cast<float4 *>(vc + dst + e0) = nv[j];
        }
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < NL; ++j) {
        d = __builtin_fmaf(q[g][j].x, nk[j].x, d);
        d = __builtin_fmaf(q[g][j].y, nk[j].y, d);
        d = __builtin_fmaf(q[g][j].z, nk[j].z, d);
        d = __builtin_fmaf(q[g][j].w, nk[j].w, d);
      }
      d = row_group_sum<R>(d);
      if (rg == 0) {
        const float mx = fmaxf(m[g], d);
        const float corr = __builtin_amdgcn_exp2f(m[g] - mx);
        const float p = __builtin_amdgcn_exp2f(d - mx);
        m[g] = mx;
        l[g] = l[g] * corr + p;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          acc[g][j * 4 + 0] = __builtin_fmaf(p, nv[j].x, acc[g][j * 4 + 0] * corr);
          acc[g][j * 4 + 1] = __builtin_fmaf(p, nv[j].y, acc[g][j * 4 + 1] * corr);
          acc[g][j * 4 + 2] = __builtin_fmaf(p, nv[j].z, acc[g][j * 4 + 2] * corr);
          acc[g][j * 4 + 3] = __builtin_fmaf(p, nv[j].w, acc[g][j * 4 + 3] * corr);
        }
      }
    }
  }
  // Merge the row groups of the wave, then the waves through LDS.
#pragma unroll
  for (int g = 0; g < GT; ++g) {
#pragma unroll
    for (int off = R; off < 64; off <<= 1) {
      const float mo = __shfl_xor(m[g], off);
      const float lo_ = __shfl_xor(l[g], off);
      const float mx = fmaxf(m[g], mo);
      const float ws = __builtin_amdgcn_exp2f(m[g] - mx);
      const float wo = __builtin_amdgcn_exp2f(mo - mx);
      l[g] = l[g] * ws + lo_ * wo;
#pragma unroll
      for (int e = 0; e < NL * 4; ++e) {
        const float ao = __shfl_xor(acc[g][e], off);
        acc[g][e] = acc[g][e] * ws + ao * wo;
      }
      m[g] = mx;
    }
  }
  constexpr int ROW = HD + 2;
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float *r = lds + ((size_t)wave * GT + g) * ROW;
      if (c == 0) {
        r[0] = m[g];
        r[1] = l[g];
      }
#pragma unroll
      for (int j = 0; j < NL; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) r[2 + (j * R + c) * 4 + e] = acc[g][j * 4 + e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < GT * HD; i += blockDim.x) {
    const int g = i / HD, d = i - g * HD;
    if ((uint32_t)g >= ng) break;
    float M = kNegBig;
    for (int w = 0; w < W; ++w) M = fmaxf(M, lds[((size_t)w * GT + g) * ROW]);
    float L = 0.f, x = 0.f;
    for (int w = 0; w < W; ++w) {
      const float *r = lds + ((size_t)w * GT + g) * ROW;
      const float wt = __builtin_amdgcn_exp2f(r[0] - M);
      L += r[1] * wt;
      x += r[2 + d] * wt;
    }
    if (slot == kNoSlot) {
      a.out[((size_t)b * a.n_heads + h0 + g) * HD + d] = L > 0.f ? x / L : 0.f;
    } else {
      const size_t idx = (size_t)slot * a.n_heads + h0 + g;
      a.ws_acc[idx * HD + d] = x;
      if (d == 0) {
        a.ws_ml[idx * 2] = M;
        a.ws_ml[idx * 2 + 1] = L;
      }
    }
  }
}

// Reduction pass (only for sequences split over several partitions): one
// wave per (sequence, query head) merges its partitions: M = max m_i,
// out = sum_i 2^(m_i - M) acc_i / sum_i 2^(m_i - M) l_i. Partitions that saw
// no visible key carry l = 0 and are skipped.
template <int HD>
__global__ void __launch_bounds__(64) decode_reduce_kernel(
    const uint4 *p_reds, const float *p_ml, const float *p_acc,
    uint32_t p_nh, DecodeArgs a) {
  // (Leading arguments preloaded into SGPRs by the build; a holds the same
  // values.)
  constexpr int EPL = HD / 64 > 0 ? HD / 64 : 1;  // elements per lane
  const uint32_t h = blockIdx.x;
  const int lane = threadIdx.x;
  uint32_t b, slot0, np;
  if (p_reds) {
    // The row is wave-uniform: scalar loads (constant address space).
    typedef const __attribute__((address_space(4))) uint32_t cu32;
    cu32 *r = (cu32 *)(uintptr_t)(p_reds + blockIdx.y);
    b = r[0];
    slot0 = r[1];
    np = r[2];
  } else {
    b = blockIdx.y;
    const uint32_t ctx = min(sload(a.ctx_lens + b), a.ctx_cap);
    if (ctx <= a.part_tokens) return;  // written directly
    slot0 = b * a.n_parts;
    np = (ctx + a.part_tokens - 1) / a.part_tokens;
  }
  const float *ml = p_ml + ((size_t)slot0 * p_nh + h) * 2;
  const size_t ml_step = (size_t)p_nh * 2;
  const float *accp = p_acc + ((size_t)slot0 * p_nh + h) * HD;
  const size_t acc_step = (size_t)p_nh * HD;
  const size_t hrow = (size_t)b * p_nh + h;
  if (np <= 8) {
    // Few partitions (the common case): every (m, l) pair (uniform loads)
    // and every partial row are fetched at once, one round trip in all.
    float m[8], l[8], x[8][EPL];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool live = (uint32_t)k < np;
      m[k] = live ? ml[k * ml_step] : kNegBig;
      l[k] = live ? ml[k * ml_step + 1] : 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = lane * EPL + e;
        x[k][e] = live && d < HD ? accp[k * acc_step + d] : 0.f;
      }
    }
    float M = kNegBig;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (l[k] != 0.f) M = fmaxf(M, m[k]);
    float acc[EPL], L = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // (l = 0: a partition that saw no visible key stays out)
      const float w = l[k] != 0.f ? __builtin_amdgcn_exp2f(m[k] - M) : 0.f;
      L += l[k] * w;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] += w != 0.f ? w * x[k][e] : 0.f;
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int d = lane * EPL + e;
      if ((uint32_t)d < a.hd) a.out[hrow * a.hd + d] = acc[e] * inv;
    }
    return;
  }
  // Lane i holds partition c + i's (m, l) for the 64-partition chunk at c;
  // M comes first, then every partial is weighted by 2^(m_i - M): the loads
  // of different partitions are independent, so they are all in flight at
  // once instead of one round trip per partition.
  float M = kNegBig;
  for (uint32_t c = 0; c < np; c += 64) {
    const uint32_t p = c + lane;
    if (p < np && ml[p * ml_step + 1] != 0.f) M = fmaxf(M, ml[p * ml_step]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  float L = 0.f;
  for (uint32_t c = 0; c < np; c += 64) {
    const uint32_t p = c + lane;
    float w = 0.f;
    if (p < np) {
      const float lp = ml[p * ml_step + 1];
      // (l = 0: a partition that saw no visible key)
      if (lp != 0.f) w = __builtin_amdgcn_exp2f(ml[p * ml_step] - M);
      L += lp * w;
    }
    const uint32_t n = min(np - c, 64u);
    // Eight partitions per pass: their loads all issue before any is used.
    auto add = [&](uint32_t i, const float (&x)[EPL]) {
      const float wi =
          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), i));
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        acc[e] += wi != 0.f ? wi * x[e] : 0.f;  // skipped partials stay out
    };
    auto fetch = [&](uint32_t i, float (&x)[EPL]) {
      const float *src = accp + (size_t)(c + i) * acc_step;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = lane * EPL + e;
        x[e] = d < HD ? src[d] : 0.f;
      }
    };
    uint32_t i = 0;
    for (; i + 8 <= n; i += 8) {
      float x[8][EPL];
#pragma unroll
      for (int k = 0; k < 8; ++k) fetch(i + k, x[k]);
#pragma unroll
      for (int k = 0; k < 8; ++k) add(i + k, x[k]);
    }
    for (; i < n; ++i) {
      float x[EPL];
      fetch(i, x);
      add(i, x);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) L += __shfl_xor(L, o);
  const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int d = lane * EPL + e;
    if ((uint32_t)d < a.hd) a.out[hrow * a.hd + d] = acc[e] * inv;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
namespace {

constexpr int kSupportedHd[] = {32, 64, 128, 256};

bool hd_supported(uint32_t hd) {
  for (int x : kSupportedHd)
    if ((uint32_t)x == hd) return true;
  return false;
}

// The decode kernels' HD for a cache head_dim: the smallest of 32, 64, 128,
// 256 that holds it (0 past 256). Rows shorter than HD read element by
// element, their missing lanes as zeros.
uint32_t decode_hd(uint32_t hd) {
  for (int x : kSupportedHd)
    if (hd <= (uint32_t)x) return (uint32_t)x;
  return 0;
}

uint32_t ilog2(uint32_t x) {
  uint32_t r = 0;
  while ((1u << r) < x) ++r;
  return r;
}

uint32_t div_up(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Query heads one wave serves: group split into sub-groups of <= 8.
void subgroups(uint32_t group, uint32_t *n_sub, uint32_t *gt) {
  *n_sub = div_up(group, 8);
  *gt = div_up(group, *n_sub);
}

// Tokens per context partition: the smallest power of two >= 256 for which
// the grid has at most ~8192 partition waves (32 per CU on 256 CUs), so long
// contexts keep enough waves in flight without a large reduction.
// Tuning overrides (RVKV_DECODE_PART_TOKENS, RVKV_DECODE_UNROLL); 0 = auto.
uint32_t env_u32(const char *name) {
  const char *v = getenv(name);
  return v ? (uint32_t)strtoul(v, nullptr, 10) : 0u;
}

// The matrix-core decode without a plan: waves a partition (its keys split
// over them, merged in the workgroup) and partition size. Four waves a
// partition below 2048 (sequence, KV head) pairs (as for plan items), then
// as many partitions as it takes for ~2048 waves, the chip's two a SIMD;
// at most 4096 keys a partition, so one long sequence does not set the
// launch's tail alone. (Llama-3.2-1B's shape: 64 x 2048 as one partition
// of four waves 47.4-47.8 us a layer, of two 49.2-49.8, two one-wave
// partitions and the reduction 50.5-50.8, one wave 62.6; 256 x 4096 one
// wave a sequence, 326 us.) RVKV_DECODE_KSPLIT=1|2|4 overrides; it is read
// at every call, so a test can take each width (each call sizes and checks
// its workspace against the same reading).
uint32_t mfma_uniform_parts(uint64_t pairs, uint32_t max_ctx,
                            uint32_t *ksplit) {
  const uint32_t forced_k = env_u32("RVKV_DECODE_KSPLIT");
  *ksplit = forced_k == 1 || forced_k == 2 || forced_k == 4
                ? forced_k
                : (pairs >= 2048 ? 1u : 4u);
  const uint64_t items = pairs * *ksplit;
  const uint64_t parts = items >= 2048 ? 1 : (2048 + items - 1) / items;
  const uint64_t per = (max_ctx + parts - 1) / parts;
  uint32_t P = 256;
  while (P < per && P < 4096) P <<= 1;
  return P;
}

uint32_t partition_tokens(const rvkv_pool *p, uint32_t batch, uint32_t n_heads,
                          uint32_t max_ctx) {
  static const uint32_t forced = env_u32("RVKV_DECODE_PART_TOKENS");
  if (forced >= 256 && forced % 256 == 0) return forced;
  if (rvkv_detail::mfma_decode_wanted(p, n_heads)) {
    uint32_t ksplit;
    return mfma_uniform_parts((uint64_t)batch * p->n_kv, max_ctx, &ksplit);
  }
  uint32_t group = n_heads / (p->n_kv ? p->n_kv : 1);
  uint32_t n_sub, gt;
  subgroups(group ? group : 1, &n_sub, &gt);
  const uint64_t pairs = (uint64_t)batch * p->n_kv * n_sub;
  // Enough workgroups for two per CU (256 CUs); a whole context per
  // workgroup whenever the batch alone provides that many.
  const uint64_t want = 512;
  const uint64_t parts = pairs >= want ? 1 : (want + pairs - 1) / pairs;
  const uint64_t per = (max_ctx + parts - 1) / parts;
  uint32_t P = 256;
  while (P < per && P < (1u << 30)) P <<= 1;
  return P;
}

// Short items: even the longest workgroup has under 192 context tokens.
bool short_items(uint64_t workgroups, uint32_t max_tokens) {
  return workgroups < 2048 && max_tokens < 192;
}

// Wavefronts per decode workgroup: four (the waves of a workgroup split its
// context) unless the grid alone already has >= 2048 workgroups (8 per CU).
// Short items with groups of up to four heads keep four waves, each with
// two loads per chunk (120 VGPRs at head_dim 256: every wave of churn's
// 1024-workgroup launch resident at once); larger groups take two waves of
// four loads (fewer waves each doing more chunks beat more waves each
// paying the start-up and merge when not all fit: churn's final launch
// 23.0 vs 26.2 us at four loads). A launch that still holds some long
// items keeps four waves of four or eight loads: its time is set by them
// (churn's 200-step run 1.9 -> 2.4 TB/s against deciding on the average).
// RVKV_DECODE_WAVES overrides.
uint32_t decode_waves(uint64_t workgroups, uint32_t max_tokens, int gt) {
  static const uint32_t forced = env_u32("RVKV_DECODE_WAVES");
  if (forced >= 1 && forced <= 4) return forced;
  if (workgroups >= 2048) return 1;
  return short_items(workgroups, max_tokens) && gt > 4 ? 2 : 4;
}

struct WsLayout {
  size_t acc_off, ml_off, bytes;
  uint32_t n_parts;
};

// Shapes the tuned decode kernels take: head_dim up to 256 (run at 32, 64,
// 128 or 256, rounded up; an f32 cache needs it exact) and power-of-two
// blocks of at least 512 / that many tokens. Every other shape runs the
// generic kernel.
bool decode_tuned(const rvkv_pool *p) {
  const uint32_t hdp = decode_hd(p->head_dim), bs = p->block_size;
  if (hdp == 0 || (p->f32() && hdp != p->head_dim)) return false;
  return (bs & (bs - 1)) == 0 && bs >= 512 / hdp;
}

WsLayout ws_layout(const rvkv_pool *p, uint32_t batch, uint32_t n_heads,
                   uint32_t max_ctx) {
  WsLayout w{};
  if (!decode_tuned(p)) {  // the generic kernel needs no workspace
    w.n_parts = 1;
    return w;
  }
  const uint32_t P = partition_tokens(p, batch, n_heads, max_ctx);
  w.n_parts = div_up(max_ctx ? max_ctx : 1, P);
  if (w.n_parts <= 1) return w;  // direct write, no workspace
  const size_t slots = (size_t)batch * n_heads * w.n_parts;
  w.acc_off = 0;
  w.ml_off = (slots * decode_hd(p->head_dim) * 4 + 255) & ~(size_t)255;
  w.bytes = w.ml_off + ((slots * 2 * 4 + 255) & ~(size_t)255);
  return w;
}

template <int HD, int GT>
void launch_decode(const DecodeArgs &a, dim3 grid, hipStream_t st) {
  static const uint32_t forced_u = env_u32("RVKV_DECODE_UNROLL");
  static const uint32_t forced_w = env_u32("RVKV_DECODE_WAVES");
  const uint64_t wgs = (uint64_t)grid.x * grid.y * grid.z;
  uint32_t W = decode_waves(wgs, a.max_tokens, GT);
  // Eight loads per chunk pay off for 512-byte rows, for large groups in
  // single-wave workgroups, and for long items when every wave of the
  // launch fits at two per SIMD in workgroups of several waves (<= 2048
  // waves; Llama 64 x 2048 on this kernel: 63.0 -> 64.8 % of 8 TB/s); two
  // for short items with groups of up to four (with four waves a
  // workgroup, above); otherwise four keep more waves resident (Qwen3-0.6B
  // 256 x 4096, 2048 one-wave workgroups: 640.1 us a layer at four, 642.0
  // at eight).
  const bool u8 =
      forced_u ? forced_u == 8
               : ((HD >= 256 && a.avg_tokens >= 512) || (GT >= 5 && W == 1) ||
                  (GT <= 4 && a.avg_tokens >= 512 && W > 1 &&
                   wgs * W <= 2048));
  const bool u2 = forced_u ? forced_u == 2
                           : GT <= 4 && short_items(wgs, a.max_tokens);
  // Eight-load kernels hold two waves a SIMD (2048 on the chip): with
  // 513-1024 uniform workgroups, two waves each keep the launch one
  // generation long (gemma-3 1024 x 1024: 183.3 -> 180.5 us a layer). (A
  // plan's ragged items keep four: churn's long-item phase was no faster.)
  if (!forced_w && !a.items && u8 && W == 4 && wgs > 512 && wgs <= 1024)
    W = 2;
  // (m, l) pairs rounded up to 16 bytes, then the accumulator rows; at
  // least the f32 kernel's W * GT * (HD + 2) floats.
  const size_t lds =
      (((size_t)W * GT * 2 + 3) / 4 * 4 + (size_t)W * GT * HD) * sizeof(float);
  if (a.f32cache)
    hipLaunchKernelGGL((decode_f32_kernel<HD, GT>), grid, dim3(64 * W), lds, st,
                       a);
  else if (a.hd != HD)  // a head_dim below HD: rows read element by element
    hipLaunchKernelGGL((decode_part_kernel<HD, GT, 4, 1, true>), grid,
                       dim3(64 * W), lds, st, a.items, a.tables,
                       a.ctx_lens, a.max_blocks, a.bs_log2, a.part_tokens, a);
  else if (u8)
    hipLaunchKernelGGL((decode_part_kernel<HD, GT, 8, 1, false>), grid,
                       dim3(64 * W), lds, st, a.items, a.tables,
                       a.ctx_lens, a.max_blocks, a.bs_log2, a.part_tokens, a);
  else if (u2)
    hipLaunchKernelGGL((decode_part_kernel<HD, GT, 2, 1, false>), grid,
                       dim3(64 * W), lds, st, a.items, a.tables,
                       a.ctx_lens, a.max_blocks, a.bs_log2, a.part_tokens, a);
  else
    hipLaunchKernelGGL((decode_part_kernel<HD, GT, 4, 1, false>), grid,
                       dim3(64 * W), lds, st, a.items, a.tables,
                       a.ctx_lens, a.max_blocks, a.bs_log2, a.part_tokens, a);
}

template <int HD>
void dispatch_gt(uint32_t gt, const DecodeArgs &a, dim3 grid, hipStream_t st) {
  switch (gt) {
    case 1: launch_decode<HD, 1>(a, grid, st); break;
    case 2: launch_decode<HD, 2>(a, grid, st); break;
    case 3: launch_decode<HD, 3>(a, grid, st); break;
    case 4: launch_decode<HD, 4>(a, grid, st); break;
    case 5: launch_decode<HD, 5>(a, grid, st); break;
    case 6: launch_decode<HD, 6>(a, grid, st); break;
    case 7: launch_decode<HD, 7>(a, grid, st); break;
    default: launch_decode<HD, 8>(a, grid, st); break;
  }
}

uint32_t grid_1d(uint64_t threads, uint32_t block) {
  return (uint32_t)((threads + block - 1) / block);
}

}  // namespace

extern "C" {

const char *rvkv_last_error(void) { return g_last_error.c_str(); }

int rvkv_pool_create(uint32_t n_layers, uint32_t num_blocks,
                     uint32_t block_size, uint32_t n_kv_heads,
                     uint32_t head_dim, rvkv_dtype cache_dtype,
                     rvkv_stream stream, rvkv_pool **out) {
  const char *op = "pool_create";
  if (!out) return fail(RVKV_EINVAL, op, "out is NULL");
  *out = nullptr;
  if (n_layers == 0 || num_blocks == 0 || block_size == 0 || n_kv_heads == 0 ||
      head_dim == 0)
    return fail(RVKV_EINVAL, op,
                "n_layers/num_blocks/block_size/n_kv_heads/head_dim must be "
                "positive");
  if (cache_dtype != RVKV_F16 && cache_dtype != RVKV_F32)
    return fail(RVKV_EINVAL, op, "cache dtype must be F16 or F32");
  rvkv_pool *p = new rvkv_pool();
  p->n_layers = n_layers;
  p->num_blocks = num_blocks;
  p->block_size = block_size;
  p->n_kv = n_kv_heads;
  p->head_dim = head_dim;
  p->elem_bytes = cache_dtype == RVKV_F32 ? 4 : 2;
  p->hd16 = head_dim * p->elem_bytes / 2;
  p->stream = static_cast<hipStream_t>(stream);
  p->block_elems = (size_t)n_kv_heads * block_size * head_dim;
  p->tensor_elems = p->block_elems * num_blocks;
  p->block16 = p->block_elems * p->elem_bytes / 2;
  p->tensor16 = p->tensor_elems * p->elem_bytes / 2;
  hipError_t e = hipGetDevice(&p->device);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(op, e);
  }
  const size_t bytes = p->tensor16 * 2 * 2 * n_layers;
  e = hipMalloc(&p->base, bytes);
  if (e != hipSuccess) {
    delete p;
    (void)hipGetLastError();
    return fail(RVKV_ENOMEM, op, "hipMalloc of the pool failed");
  }
  e = hipMemsetAsync(p->base, 0, bytes, p->stream);
  if (e != hipSuccess) {
    (void)hipFree(p->base);
    delete p;
    return hip_fail(op, e);
  }
  *out = p;
  return RVKV_OK;
}

void rvkv_pool_destroy(rvkv_pool *pool) {
  if (!pool) return;
  (void)hipStreamSynchronize(pool->stream);
  (void)hipFree(pool->base);
  delete pool;
}

size_t rvkv_pool_bytes(const rvkv_pool *pool) {
  return pool ? pool->tensor16 * 4 * pool->n_layers : 0;
}

int rvkv_pool_set_stream(rvkv_pool *pool, rvkv_stream stream) {
  if (!pool) return fail(RVKV_EINVAL, "pool_set_stream", "pool is NULL");
  pool->stream = static_cast<hipStream_t>(stream);
  return RVKV_OK;
}

namespace {
// Tokens per head-major lane group of the append (RVKV_APPEND_GROUP, read
// once; 1 = token-major). Head-major groups of 4 measured 3-6 % faster
// than token-major for f32 rows (Qwen3 prefill append), neutral for f16.
uint32_t append_tok_group(uint32_t n_tokens) {
  static const uint32_t g = [] {
    const char *e = getenv("RVKV_APPEND_GROUP");
    const long v = e ? strtol(e, nullptr, 10) : 4;
    return (uint32_t)(v >= 1 && v <= 64 ? v : 1);
  }();
  return n_tokens >= g ? g : 1;
}
}  // namespace

int rvkv_append(rvkv_pool *pool, uint32_t layer, const void *k, const void *v,
                rvkv_dtype src_dtype, const uint32_t *slot_block,
                const uint32_t *slot_off, uint32_t n_tokens) {
  const char *op = "kv_write";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers)
    return fail(RVKV_EINVAL, op, "layer out of range");
  if (n_tokens == 0) return fail(RVKV_EINVAL, op, "k/v len is 0");
  if (!k || !v || !slot_block || !slot_off)
    return fail(RVKV_EINVAL, op, "NULL k/v/block_ids/offsets");
  if (src_dtype != RVKV_F16 && src_dtype != RVKV_F32)
    return fail(RVKV_EINVAL, op, "src dtype must be F16 or F32");
  uint16_t *kc = pool->tensor(layer, 0), *vc = pool->tensor(layer, 1);
  if (pool->f32() && src_dtype == RVKV_F16) {
    // f16 rows into an f32 cache: widened exactly, one thread per cell.
    const uint64_t cells = (uint64_t)n_tokens * pool->n_kv * pool->head_dim;
    hipLaunchKernelGGL(append_widen_kernel, dim3(grid_1d(cells, 256)),
                       dim3(256), 0, pool->stream,
                       static_cast<const uint16_t *>(k),
                       static_cast<const uint16_t *>(v), slot_block, slot_off,
                       reinterpret_cast<float *>(kc),
                       reinterpret_cast<float *>(vc), n_tokens, pool->n_kv,
                       pool->head_dim, pool->block_size, pool->num_blocks);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
  }
  // f32 rows into an f32 cache are copied bit for bit: the same kernel as
  // an f16 copy, over 16-bit words (hd16 of them per row).
  const bool f32_copy = pool->f32();
  if (f32_copy) src_dtype = RVKV_F16;
  const uint32_t hd = pool->hd16;
  const bool v8 = hd % 8 == 0;
  if (v8 && src_dtype == RVKV_F32 &&
      ((uintptr_t)k % 16 || (uintptr_t)v % 16))
    return fail(RVKV_EINVAL, op, "f32 k/v must be 16-byte aligned");
  if (v8 && src_dtype == RVKV_F16 && ((uintptr_t)k % 16 || (uintptr_t)v % 16))
    return fail(RVKV_EINVAL, op,
                f32_copy ? "f32 k/v must be 16-byte aligned"
                         : "f16 k/v must be 16-byte aligned");
  const uint32_t tg = v8 ? append_tok_group(n_tokens) : 1;
  const uint64_t threads =
      (uint64_t)((n_tokens + tg - 1) / tg) * tg * pool->n_kv *
      (v8 ? hd / 8 : hd);
  const dim3 grid(grid_1d(threads, 256));
  if (v8) {
    if (src_dtype == RVKV_F32)
      hipLaunchKernelGGL((append_kernel<8, true>), grid, dim3(256), 0,
                         pool->stream, k, v, slot_block, slot_off, kc, vc,
                         n_tokens, pool->n_kv, hd, pool->block_size,
                         pool->num_blocks, 0, 0, tg);
    else
      hipLaunchKernelGGL((append_kernel<8, false>), grid, dim3(256), 0,
                         pool->stream, k, v, slot_block, slot_off, kc, vc,
                         n_tokens, pool->n_kv, hd, pool->block_size,
                         pool->num_blocks, 0, 0, tg);
  } else {
    if (src_dtype == RVKV_F32)
      hipLaunchKernelGGL((append_kernel<1, true>), grid, dim3(256), 0,
                         pool->stream, k, v, slot_block, slot_off, kc, vc,
                         n_tokens, pool->n_kv, hd, pool->block_size,
                         pool->num_blocks);
    else
      hipLaunchKernelGGL((append_kernel<1, false>), grid, dim3(256), 0,
                         pool->stream, k, v, slot_block, slot_off, kc, vc,
                         n_tokens, pool->n_kv, hd, pool->block_size,
                         pool->num_blocks);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

int rvkv_append_layers(rvkv_pool *pool, uint32_t layer0, uint32_t n_layers,
                       const void *k, const void *v, rvkv_dtype src_dtype,
                       uint64_t src_layer_stride, const uint32_t *slot_block,
                       const uint32_t *slot_off, uint32_t n_tokens) {
  const char *op = "kv_write";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (n_layers == 0 || layer0 >= pool->n_layers ||
      n_layers > pool->n_layers - layer0)
    return fail(RVKV_EINVAL, op, "layer range out of range");
  if (n_layers > 65535) return fail(RVKV_EUNSUPPORTED, op, "too many layers");
  if (n_tokens == 0) return fail(RVKV_EINVAL, op, "k/v len is 0");
  if (!k || !v || !slot_block || !slot_off)
    return fail(RVKV_EINVAL, op, "NULL k/v/block_ids/offsets");
  if (src_dtype != RVKV_F16 && src_dtype != RVKV_F32)
    return fail(RVKV_EINVAL, op, "src dtype must be F16 or F32");
  if (src_layer_stride <
      (uint64_t)n_tokens * pool->n_kv * pool->head_dim && n_layers > 1)
    return fail(RVKV_EINVAL, op,
                "src_layer_stride is shorter than one layer's rows");
  const uint32_t src_bytes = src_dtype == RVKV_F32 ? 4 : 2;
  const uint32_t hd = pool->hd16;
  const bool one_launch = !pool->f32() && hd % 8 == 0;
  if (!one_launch) {
    // f32 cells and head_dim % 8 != 0: one rvkv_append per layer.
    for (uint32_t l = 0; l < n_layers; ++l) {
      const size_t sl = (size_t)l * src_layer_stride * src_bytes;
      int rc = rvkv_append(pool, layer0 + l, static_cast<const char *>(k) + sl,
                           static_cast<const char *>(v) + sl, src_dtype,
                           slot_block, slot_off, n_tokens);
      if (rc) return rc;
    }
    return RVKV_OK;
  }
  if ((uintptr_t)k % 16 || (uintptr_t)v % 16 ||
      (src_layer_stride * src_bytes) % 16)
    return fail(RVKV_EINVAL, op,
                "k/v and the layer stride must be 16-byte aligned");
  uint16_t *kc = pool->tensor(layer0, 0), *vc = pool->tensor(layer0, 1);
  const uint64_t cache_stride = 2 * (uint64_t)pool->tensor16;
  const uint32_t tg = append_tok_group(n_tokens);
  const uint64_t threads =
      (uint64_t)((n_tokens + tg - 1) / tg) * tg * pool->n_kv * (hd / 8);
  const dim3 grid(grid_1d(threads, 256), n_layers);
  if (src_dtype == RVKV_F32)
    hipLaunchKernelGGL((append_kernel<8, true>), grid, dim3(256), 0,
                       pool->stream, k, v, slot_block, slot_off, kc, vc,
                       n_tokens, pool->n_kv, hd, pool->block_size,
                       pool->num_blocks, src_layer_stride, cache_stride, tg);
  else
    hipLaunchKernelGGL((append_kernel<8, false>), grid, dim3(256), 0,
                       pool->stream, k, v, slot_block, slot_off, kc, vc,
                       n_tokens, pool->n_kv, hd, pool->block_size,
                       pool->num_blocks, src_layer_stride, cache_stride, tg);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

int rvkv_gather(const rvkv_pool *pool, uint32_t layer,
                const uint32_t *block_idx, uint32_t batch, uint32_t max_blocks,
                uint32_t ctx_len, void *out_k, void *out_v,
                rvkv_dtype out_dtype) {
  const char *op = "kv_gather";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers)
    return fail(RVKV_EINVAL, op, "layer out of range");
  if (batch == 0 || max_blocks == 0 || ctx_len == 0)
    return fail(RVKV_EINVAL, op,
                "batch/max_blocks/ctx_len/block_size/n_kv_heads/head_dim must "
                "be positive");
  if ((uint64_t)ctx_len > (uint64_t)max_blocks * pool->block_size)
    return fail(RVKV_EINVAL, op,
                "ctx_len must not exceed max_blocks * block_size");
  if (!block_idx || !out_k || !out_v)
    return fail(RVKV_EINVAL, op, "NULL block_idx/out_k/out_v");
  if (out_dtype != RVKV_F16 && out_dtype != RVKV_F32)
    return fail(RVKV_EINVAL, op, "out dtype must be F16 or F32");
  if (pool->f32()) {
    // An f32 cache gathers into f32 only, bit for bit: the raw-copy kernel
    // over 16-bit words.
    if (out_dtype != RVKV_F32)
      return fail(RVKV_EUNSUPPORTED, op, "an f32 cache gathers into F32 only");
    out_dtype = RVKV_F16;
  }
  const uint32_t hd = pool->hd16;
  const bool v8 = hd % 8 == 0 && (uintptr_t)out_k % 16 == 0 &&
                  (uintptr_t)out_v % 16 == 0;
  const uint64_t rows = (uint64_t)batch * pool->n_kv * ctx_len;
  const dim3 grid(grid_1d(rows * (v8 ? hd / 8 : hd), 256));
  const uint16_t *kc = pool->tensor(layer, 0), *vc = pool->tensor(layer, 1);
#define RVKV_GATHER(VW, F32)                                                  \
  hipLaunchKernelGGL((gather_kernel<VW, F32>), grid, dim3(256), 0,            \
                     pool->stream, kc, vc, block_idx, out_k, out_v, batch,    \
                     max_blocks, ctx_len, pool->n_kv, hd, pool->block_size,   \
                     pool->num_blocks)
  if (v8) {
    if (out_dtype == RVKV_F32) RVKV_GATHER(8, true);
    else RVKV_GATHER(8, false);
  } else {
    if (out_dtype == RVKV_F32) RVKV_GATHER(1, true);
    else RVKV_GATHER(1, false);
  }
#undef RVKV_GATHER
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

uint32_t rvkv_decode_partition_tokens(const rvkv_pool *pool, uint32_t batch,
                                      uint32_t n_heads, uint32_t max_ctx_len) {
  if (!pool) return 0;
  return partition_tokens(pool, batch, n_heads, max_ctx_len);
}

size_t rvkv_decode_workspace_bytes(const rvkv_pool *pool, uint32_t batch,
                                   uint32_t n_heads, uint32_t max_ctx_len) {
  if (!pool) return 0;
  return ws_layout(pool, batch, n_heads, max_ctx_len).bytes;
}

}  // extern "C"

namespace {

// Checks what every decode entry point needs and fills the common part of
// DecodeArgs; returns 0 or an error code (message already set).
int prepare_decode(const char *op, const rvkv_pool *pool, uint32_t layer,
                   const float *q, const uint32_t *block_tables,
                   const uint32_t *ctx_lens, uint32_t max_blocks,
                   uint32_t n_heads, uint32_t max_ctx_len, float scale,
                   int32_t window, float *out, DecodeArgs *a, uint32_t *gt) {
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers)
    return fail(RVKV_EINVAL, op, "layer out of range");
  if (max_blocks == 0) return fail(RVKV_EINVAL, op, "max_blocks must be positive");
  if (n_heads == 0 || n_heads % pool->n_kv != 0)
    return fail(RVKV_EINVAL, op,
                "n_heads must be a positive multiple of n_kv_heads");
  const bool generic = !decode_tuned(pool);
  if (generic && !rvkv_detail::generic_head_dim_ok(pool->head_dim))
    return fail(RVKV_EUNSUPPORTED, op, "head_dim must be at most 1024");
  const uint32_t bs = pool->block_size;
  if (!q || !block_tables || !ctx_lens || !out)
    return fail(RVKV_EINVAL, op, "NULL q/block_tables/ctx_lens/out");
  if ((uintptr_t)q % 16 || (uintptr_t)out % 16)
    return fail(RVKV_EINVAL, op, "q and out must be 16-byte aligned");
  const uint32_t group = n_heads / pool->n_kv;
  uint32_t n_sub;
  subgroups(group, &n_sub, gt);
  if ((uint64_t)pool->n_kv * n_sub > 65535)
    return fail(RVKV_EUNSUPPORTED, op, "head count too large");
  if (max_ctx_len == 0) max_ctx_len = 1;
  const uint64_t cap64 = (uint64_t)max_blocks * bs;
  *a = DecodeArgs{};
  a->kc = pool->tensor(layer, 0);
  a->vc = pool->tensor(layer, 1);
  a->q = q;
  a->out = out;
  a->tables = block_tables;
  a->ctx_lens = ctx_lens;
  a->block_stride = pool->block_elems;
  a->head_stride = bs * pool->head_dim;
  a->hd = pool->head_dim;
  a->f32cache = pool->f32() ? 1u : 0u;
  a->block_size = bs;
  a->max_blocks = max_blocks;
  a->num_blocks = pool->num_blocks;
  a->n_kv = pool->n_kv;
  a->n_heads = n_heads;
  a->group = group;
  a->n_sub = n_sub;
  a->bs_log2 = ilog2(bs);
  a->ctx_cap = (uint32_t)(cap64 < max_ctx_len ? cap64 : max_ctx_len);
  a->qscale = scale * 1.4426950408889634f;  // log2(e)
  a->window = window;
  a->generic = generic ? 1u : 0u;
  return RVKV_OK;
}

// The generic kernel over the decode's arguments (one row per sequence).
int decode_generic(const char *op, const rvkv_pool *pool, uint32_t layer,
                   const DecodeArgs &a, uint32_t batch, float scale) {
  return rvkv_detail::generic_attention(
      op, pool, layer, a.q, a.tables, a.max_blocks, nullptr, a.ctx_lens,
      batch, 1, a.n_heads, a.ctx_cap, scale, a.window, a.out);
}

int check_ws(const char *op, void *ws, size_t ws_bytes, size_t need) {
  if (need == 0) return RVKV_OK;
  if (!ws) return fail(RVKV_EINVAL, op, "workspace is NULL");
  if (ws_bytes < need)
    return fail(RVKV_EINVAL, op, "workspace smaller than the required bytes");
  if ((uintptr_t)ws % 256)
    return fail(RVKV_EINVAL, op, "workspace must be 256-byte aligned");
  return RVKV_OK;
}

// Launches the partition kernel on `grid` and, when some sequence is split,
// the reduction kernel on `rgrid`.
int launch_decode_pair(const char *op, const DecodeArgs &a, uint32_t hd,
                       uint32_t gt, dim3 grid, dim3 rgrid, bool reduce,
                       hipStream_t st) {
  switch (hd) {
    case 32: dispatch_gt<32>(gt, a, grid, st); break;
    case 64: dispatch_gt<64>(gt, a, grid, st); break;
    case 128: dispatch_gt<128>(gt, a, grid, st); break;
    default: dispatch_gt<256>(gt, a, grid, st); break;
  }
  if (reduce) {
    switch (hd) {
      case 32: hipLaunchKernelGGL(decode_reduce_kernel<32>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
      case 64: hipLaunchKernelGGL(decode_reduce_kernel<64>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
      case 128: hipLaunchKernelGGL(decode_reduce_kernel<128>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
      default: hipLaunchKernelGGL(decode_reduce_kernel<256>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
    }
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

int launch_reduce(const char *op, const DecodeArgs &a, uint32_t hd,
                  dim3 rgrid, hipStream_t st) {
  switch (hd) {
    case 32: hipLaunchKernelGGL(decode_reduce_kernel<32>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
    case 64: hipLaunchKernelGGL(decode_reduce_kernel<64>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
    case 128: hipLaunchKernelGGL(decode_reduce_kernel<128>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
    default: hipLaunchKernelGGL(decode_reduce_kernel<256>, rgrid, dim3(64), 0, st, a.reds, a.ws_ml, a.ws_acc, a.n_heads, a); break;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

}  // namespace

struct rvkv_decode_plan;

namespace {
int planned_mfma(const char *op, const rvkv_pool *pool,
                 const rvkv_decode_plan *plan, uint32_t layer,
                 const DecodeArgs &a, uint32_t max_blocks, float scale);
}  // namespace

struct rvkv_decode_plan {
  const rvkv_pool *pool;
  uint32_t batch, n_heads, n_kv, head_dim, max_ctx;
  int32_t window;
  uint32_t part_tokens, n_items, n_reds, n_slots, avg_tokens = 0,
      max_tokens = 0;
  uint4 *d_buf = nullptr;   // items, reduction rows, group lists (device)
  // Pinned staging copies of the same, used in turn: an update waits only
  // for the upload kNStage updates back, so the host can build a few steps
  // ahead of the device (stream order protects d_buf).
  static constexpr int kNStage = 3;
  uint4 *h_buf[kNStage] = {};
  hipEvent_t uploaded[kNStage] = {};  // upload from h_buf[i] done
  int next = 0;             // staging buffer the next update fills
  size_t cap = 0;           // entries every buffer holds
  size_t acc_off, ml_off, ws_bytes;
};

namespace {

// Waves a plan item on the matrix cores (its keys split over them, merged
// in the workgroup): four while the launch has under 2048 workgroups, one
// from 2048 on (Qwen2.5 ragged, ~1500 workgroups: 74.7 -> 70.8 us a layer;
// Llama-3.2-1B 64 x 2048, 512: 50.9 -> 48.1 us; 256 x 4096, 2048: one wave
// 327 us, four 335). RVKV_DECODE_PLAN_KSPLIT=1|2|4 overrides; it is read at
// every launch (the split needs no workspace), so a test can take each width.
uint32_t planned_ksplit(const rvkv_decode_plan *plan) {
  const uint32_t k = env_u32("RVKV_DECODE_PLAN_KSPLIT");
  if (k == 1 || k == 2 || k == 4) return k;
  return (uint64_t)plan->n_items * plan->n_kv >= 2048 ? 1u : 4u;
}

// A planned decode on the matrix cores (large GQA groups): the plan's work
// items through the prefill kernel in decode mode, which writes the output
// of whole-context items and the partials of split ones; then the same
// reduction pass as the VALU decode.
int planned_mfma(const char *op, const rvkv_pool *pool,
                 const rvkv_decode_plan *plan, uint32_t layer,
                 const DecodeArgs &a, uint32_t max_blocks, float scale) {
  int rc = rvkv_detail::mfma_decode(
      pool, layer, a.q, a.tables, a.ctx_lens, max_blocks, plan->n_heads,
      scale, plan->window, a.items, plan->n_items, a.ws_acc, a.ws_ml, a.out,
      a.new_k, a.new_v, a.new_blk, a.new_off, a.new_f32,
      reinterpret_cast<const uint32_t *>(plan->d_buf + plan->n_items +
                                         plan->n_reds),
      0, 0, 0xFFFFFFFFu, planned_ksplit(plan));
  if (rc || plan->n_reds == 0) return rc;
  return launch_reduce(op, a, decode_hd(pool->head_dim),
                       dim3(plan->n_heads, plan->n_reds),
                       pool->stream);
}

// (Re)builds the work list of `pl` for these context lengths and uploads it
// on the pool's stream. Device-side ordering after earlier decodes comes from
// the stream; the pinned staging buffer is reused once the previous upload
// has completed.
int plan_build(rvkv_decode_plan *pl, const uint32_t *ctx_lens_host,
               uint32_t batch, const uint32_t *tables_host = nullptr,
               uint32_t max_blocks = 0) {
  const char *op = "decode_plan";
  const rvkv_pool *pool = pl->pool;
  uint32_t n_sub, gt;
  subgroups(pl->n_heads / pool->n_kv, &n_sub, &gt);
  const uint64_t n_hy = (uint64_t)pool->n_kv * n_sub;
  const int32_t window = pl->window;
  // Visible tokens per sequence: [lo_b, ctx_b), lo_b from the window.
  uint64_t total = 0;
  uint32_t max_ctx = 1;
  for (uint32_t b = 0; b < batch; ++b) {
    const uint32_t n = ctx_lens_host[b];
    const uint32_t lo = (window > 0 && n > (uint32_t)window) ? n - window : 0;
    total += n - lo;
    if (n > max_ctx) max_ctx = n;
  }
  // Tokens per work item: about one sequence, but at least enough that the
  // grid has <= ~1024 workgroups and at most what keeps >= ~256 of them.
  // (The matrix-core decode splits an item's keys over four waves when
  // the launch has under 2048 workgroups, see planned_ksplit; with one
  // wave an item, items a quarter as long measured best for Qwen2.5.)
  const bool mfma = rvkv_detail::mfma_decode_wanted(pool, pl->n_heads);
  static const uint32_t forced_div = env_u32("RVKV_DECODE_PLAN_DIV");
  const double per = forced_div ? (double)forced_div : 1.0;
  const double avg = (double)total / batch / per;
  const double lo_p = (double)total * n_hy / (1024.0 * per);
  const double hi_p = (double)total * n_hy / (256.0 * per);
  double want = avg < lo_p ? lo_p : avg;
  if (want > hi_p) want = hi_p;
  // Item boundaries: multiples of 256 tokens on the matrix-core decode
  // (its 32/64-key tiles and block-id prefetch assume them); on the VALU
  // decode multiples of 64 (any multiple of a wave-wide load's tokens
  // works), and items down to 128 tokens, so that in a batch of mostly short
  // sequences a few long ones are cut into items near the typical length
  // instead of setting the launch's tail (RVKV_DECODE_PLAN_GRAN = 64 or 256
  // overrides the VALU granule).
  static const uint32_t forced_gran = env_u32("RVKV_DECODE_PLAN_GRAN");
  const uint32_t gran =
      mfma ? 256u : (forced_gran == 64 || forced_gran == 256 ? forced_gran
                                                             : 64u);
  uint32_t P = gran == 256 ? 256 : 128;
  while (P < want && P < (1u << 30)) P <<= 1;

  // Items of at most P tokens over [start, n), with 1/8 slack (1/2 on the
  // matrix-core decode) so a range just past a multiple of P does not get a
  // sliver item; split evenly on gran-token boundaries. Returns the count and
  // the step. (Qwen2.5 ragged, P = 2048: slack 1/2 69.2-69.6 us a layer
  // against 69.5-71.4 at 1/8, 73.0-73.4 at 3/4 and 73.5-73.6 at 1.)
  // VALU decode: a sequence up to four times the average length (and up to
  // 2P, within the >= ~256-workgroup bound) stays one item. Splitting it
  // costs the reduction launch, and a moderately long item that starts
  // first (longest first) finishes in the launch's tail, when the bandwidth
  // is its own; the few long survivors of a churning batch are still cut
  // into items near the typical length.
  const uint32_t whole_max =
      mfma ? 0u
           : (uint32_t)std::min(std::min(4.0 * (double)total / batch, hi_p),
                                2.0 * P);
  auto split = [&](uint32_t start, uint32_t n, uint32_t *step_out) {
    const uint32_t span = n - start;
    if (span <= whole_max) {
      *step_out = span;
      return 1u;
    }
    uint32_t k = div_up(span, P + (mfma ? P / 2 : P / 8));
    const uint32_t step = (div_up(span, k) + gran - 1) / gran * gran;
    *step_out = step;
    return div_up(span, step);
  };

  // Shared-prefix groups (matrix-core decode, host tables, no window): the
  // sequences whose tables open with the same blocks are taken up to S at a
  // time (S * group query rows fill one 32-row matrix tile), longest first;
  // a group reads the blocks all its members share, [0, T), once for all of
  // them, and each member reads only [T, n) on its own. T is a multiple of
  // 256 below every member's appended position (n - 1), so a group never
  // holds a key this step writes. Each member's partial of a group range is
  // one more partition of that member for the reduction.
  const uint32_t group = pl->n_heads / pool->n_kv;
  std::vector<uint32_t> gstart(batch, 0xFFFFFFFFu);  // own-range start
  std::vector<uint32_t> gidx(batch, 0xFFFFFFFFu);    // group of a member
  struct Group {
    uint32_t T;
    std::vector<uint32_t> mem;
  };
  std::vector<Group> groups;
  static const uint32_t no_groups = env_u32("RVKV_DECODE_NO_GROUPS");
  if (mfma && tables_host && window <= 0 && group <= 16 && max_blocks &&
      !no_groups) {
    const uint32_t S = std::min<uint32_t>(32 / group, 8);
    const uint32_t lg = ilog2(pool->block_size);
    std::vector<std::pair<uint32_t, uint32_t>> cand;  // (first block, b)
    for (uint32_t b = 0; b < batch; ++b)
      if (ctx_lens_host[b] > 256u)
        cand.push_back({tables_host[(size_t)b * max_blocks], b});
    std::sort(cand.begin(), cand.end(), [&](const auto &x, const auto &y) {
      if (x.first != y.first) return x.first < y.first;
      if (ctx_lens_host[x.second] != ctx_lens_host[y.second])
        return ctx_lens_host[x.second] > ctx_lens_host[y.second];
      return x.second < y.second;
    });
    for (size_t i = 0; i < cand.size();) {
      size_t j = i;
      while (j < cand.size() && cand[j].first == cand[i].first) ++j;
      for (size_t c = i; c + 1 < j; c += S) {
        const size_t e = std::min(j, c + S);
        if (e - c < 2) break;
        uint32_t min_n = 0xFFFFFFFFu;
        for (size_t m = c; m < e; ++m)
          min_n = std::min(min_n, ctx_lens_host[cand[m].second]);
        // Blocks every member has at the same place, below min_n - 1.
        const uint32_t lim =
            std::min<uint32_t>((min_n - 1) >> lg, max_blocks);
        const uint32_t *t0 = tables_host + (size_t)cand[c].second * max_blocks;
        uint32_t common = 0;
        while (common < lim) {
          bool same = true;
          for (size_t m = c + 1; m < e && same; ++m)
            same = tables_host[(size_t)cand[m].second * max_blocks + common] ==
                   t0[common];
          if (!same) break;
          ++common;
        }
        const uint32_t T =
            std::min<uint32_t>(common << lg, min_n - 1) & ~255u;
        if (T < 256) continue;
        Group g{T, {}};
        for (size_t m = c; m < e; ++m) {
          g.mem.push_back(cand[m].second);
          gstart[cand[m].second] = T;
          gidx[cand[m].second] = (uint32_t)groups.size();
        }
        groups.push_back(std::move(g));
      }
      i = j;
    }
  }

  std::vector<uint4> items, reds;
  items.reserve(batch);
  uint32_t slots = 0;
  // First slot of each grouped member (its group partials come first).
  std::vector<uint32_t> mslot(batch, 0);
  std::vector<uint32_t> gpieces(groups.size(), 0), gstep(groups.size(), 0);
  for (size_t g = 0; g < groups.size(); ++g)
    gpieces[g] = split(0, groups[g].T, &gstep[g]);
  for (uint32_t b = 0; b < batch; ++b) {
    const uint32_t n = ctx_lens_host[b];
    if (n == 0) {  // zero row
      items.push_back(make_uint4(b, 0, 0, kNoSlot));
      continue;
    }
    const uint32_t lo = (window > 0 && n > (uint32_t)window) ? n - window : 0;
    const bool grouped = gidx[b] != 0xFFFFFFFFu;
    const uint32_t start = grouped ? gstart[b] : lo / gran * gran;
    const uint32_t pre = grouped ? gpieces[gidx[b]] : 0;
    uint32_t step;
    const uint32_t k = split(start, n, &step);
    if (k == 1 && pre == 0) {
      items.push_back(make_uint4(b, start, n, kNoSlot));
      continue;
    }
    mslot[b] = slots;
    for (uint32_t i = 0; i < k; ++i) {
      const uint32_t t0 = start + i * step;
      items.push_back(make_uint4(b, t0, t0 + step < n ? t0 + step : n,
                                 slots + pre + i));
    }
    reds.push_back(make_uint4(b, slots, pre + k, 0));
    slots += pre + k;
  }
  // Group items: {kGroupItem | word offset of the member list, t0, t1, 0};
  // list = n, then the members' sequences, then their slots for this piece.
  std::vector<uint32_t> glist;
  for (size_t g = 0; g < groups.size(); ++g) {
    const Group &G = groups[g];
    for (uint32_t i = 0; i < gpieces[g]; ++i) {
      const uint32_t t0 = i * gstep[g];
      const uint32_t t1 = std::min(t0 + gstep[g], G.T);
      items.push_back(make_uint4(kGroupItem | (uint32_t)glist.size(), t0, t1,
                                 0));
      glist.push_back((uint32_t)G.mem.size());
      for (uint32_t m : G.mem) glist.push_back(m);
      for (uint32_t m : G.mem) glist.push_back(mslot[m] + i);
    }
  }
  while (glist.size() % 4) glist.push_back(0);
  // Longest items first: the short tail fills in behind them. With the
  // block tables, items of one length are further ordered by the first
  // block they read, so the items of sequences that share prefix blocks
  // run back to back: consecutive workgroups go round-robin over the XCDs,
  // and each XCD's sharers then find those blocks in its L2 instead of
  // reading them from HBM once per sharer.
  if (tables_host) {
    // Items whose first block also starts another item form a group, placed
    // by its longest member; inside a group, longest first.
    const uint32_t lg = ilog2(pool->block_size);
    std::vector<uint32_t> fb(items.size());
    std::vector<std::pair<uint32_t, uint32_t>> by_block(items.size());
    for (size_t i = 0; i < items.size(); ++i) {
      const uint32_t bi = items[i].y >> lg;
      const uint32_t sq = items[i].x & kGroupItem
                              ? glist[(items[i].x & ~kGroupItem) + 1]
                              : items[i].x;
      fb[i] = bi < max_blocks ? tables_host[(size_t)sq * max_blocks + bi]
                              : 0xFFFFFFFFu;
      by_block[i] = {fb[i], items[i].z - items[i].y};
    }
    std::sort(by_block.begin(), by_block.end());
    std::vector<uint32_t> key(items.size());  // the group's longest item
    std::vector<uint32_t> grouped(items.size());
    for (size_t i = 0; i < items.size(); ++i) {
      const auto lo_it = std::lower_bound(
          by_block.begin(), by_block.end(), std::make_pair(fb[i], 0u));
      const auto hi_it = std::upper_bound(
          by_block.begin(), by_block.end(),
          std::make_pair(fb[i], 0xFFFFFFFFu));
      grouped[i] = (hi_it - lo_it) > 1;
      key[i] = (hi_it - 1)->second;
    }
    std::vector<uint32_t> order(items.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (uint32_t)i;
    std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
      const uint32_t lx = grouped[x] ? key[x] : items[x].z - items[x].y;
      const uint32_t ly = grouped[y] ? key[y] : items[y].z - items[y].y;
      if (lx != ly) return lx > ly;
      if (fb[x] != fb[y]) return fb[x] < fb[y];
      return (items[x].z - items[x].y) > (items[y].z - items[y].y);
    });
    std::vector<uint4> sorted(items.size());
    for (size_t i = 0; i < order.size(); ++i) sorted[i] = items[order[i]];
    items.swap(sorted);
    // Shared-prefix group items read the same blocks: the items of one
    // prefix go 8 grid positions apart, so (workgroups going to the XCDs
    // round robin by linear id) they run on one XCD, close together in
    // time, and each prefix block is fetched into that XCD's L2 once
    // instead of once per XCD; different prefixes take different XCDs.
    // (RVKV_DECODE_GROUP_XCD=0: plain order.)
    static const char *gx = getenv("RVKV_DECODE_GROUP_XCD");
    std::vector<std::vector<uint4>> lane(8);
    std::vector<uint4> rest;
    std::vector<std::pair<uint32_t, uint32_t>> prefix;  // (first block, lane)
    size_t first_g = items.size(), n_g = 0;
    for (size_t i = 0; i < items.size(); ++i) {
      if (!(items[i].x & kGroupItem)) {
        rest.push_back(items[i]);
        continue;
      }
      if (n_g++ == 0) first_g = i;
      // A prefix is named by the first block its first member's table holds.
      const uint32_t sq = glist[(items[i].x & ~kGroupItem) + 1];
      const uint32_t key = tables_host[(size_t)sq * max_blocks];
      size_t k = 0;
      while (k < prefix.size() && prefix[k].first != key) ++k;
      if (k == prefix.size()) prefix.push_back({key, (uint32_t)(k % 8)});
      lane[prefix[k].second].push_back(items[i]);
    }
    const size_t n = items.size();
    size_t span = 0;  // positions the longest lane needs
    for (int l = 0; l < 8; ++l)
      if (!lane[l].empty()) span = std::max(span, l + 8 * (lane[l].size() - 1) + 1);
    if (!(gx && gx[0] == '0') && n_g > 1 && span <= n) {
      size_t p0 = first_g & ~(size_t)7;
      while (p0 + span > n) p0 -= 8;
      std::vector<char> taken(n, 0);
      for (int l = 0; l < 8; ++l)
        for (size_t j = 0; j < lane[l].size(); ++j) {
          items[p0 + l + 8 * j] = lane[l][j];
          taken[p0 + l + 8 * j] = 1;
        }
      size_t r = 0;
      for (size_t i = 0; i < n; ++i)
        if (!taken[i]) items[i] = rest[r++];
    }
  } else {
    std::stable_sort(items.begin(), items.end(),
                     [](const uint4 &x, const uint4 &y) {
                       return (x.z - x.y) > (y.z - y.y);
                     });
  }
  const size_t need = items.size() + reds.size() + glist.size() / 4;
  hipError_t e = hipSuccess;
  const int si = pl->next;
  if (pl->uploaded[si]) e = hipEventSynchronize(pl->uploaded[si]);
  if (e == hipSuccess && need > pl->cap) {
    // Growing (rare: the first build reserves room for two items per
    // sequence): the old device list may still be read by queued decodes.
    if (pl->d_buf) e = hipStreamSynchronize(pool->stream);
    if (e == hipSuccess && pl->d_buf) e = hipFree(pl->d_buf);
    for (int i = 0; i < rvkv_decode_plan::kNStage; ++i) {
      if (e == hipSuccess && pl->h_buf[i]) e = hipHostFree(pl->h_buf[i]);
      pl->h_buf[i] = nullptr;
    }
    pl->d_buf = nullptr;
    pl->cap = 0;
    const size_t cap =
        std::max<size_t>(need + need / 4 + 16, 2 * (size_t)batch + 64);
    if (e == hipSuccess) e = hipMalloc(&pl->d_buf, cap * sizeof(uint4));
    for (int i = 0; i < rvkv_decode_plan::kNStage; ++i)
      if (e == hipSuccess)
        e = hipHostMalloc(&pl->h_buf[i], cap * sizeof(uint4));
    if (e == hipSuccess) pl->cap = cap;
  }
  if (e == hipSuccess && !pl->uploaded[si])
    e = hipEventCreateWithFlags(&pl->uploaded[si], hipEventDisableTiming);
  if (e != hipSuccess) return hip_fail(op, e);
  uint4 *h = pl->h_buf[si];
  std::copy(items.begin(), items.end(), h);
  std::copy(reds.begin(), reds.end(), h + items.size());
  std::memcpy(h + items.size() + reds.size(), glist.data(),
              glist.size() * sizeof(uint32_t));
  e = hipMemcpyAsync(pl->d_buf, h, need * sizeof(uint4),
                     hipMemcpyHostToDevice, pool->stream);
  if (e == hipSuccess) e = hipEventRecord(pl->uploaded[si], pool->stream);
  if (e != hipSuccess) return hip_fail(op, e);
  pl->next = (si + 1) % rvkv_decode_plan::kNStage;

  pl->batch = batch;
  pl->max_ctx = max_ctx;
  pl->part_tokens = P;
  pl->avg_tokens = items.empty() ? 0u : (uint32_t)(total / items.size());
  pl->max_tokens = 0;
  for (const uint4 &it : items)
    pl->max_tokens = std::max(pl->max_tokens, it.z > it.y ? it.z - it.y : 0u);
  pl->n_items = (uint32_t)items.size();
  pl->n_reds = (uint32_t)reds.size();
  pl->n_slots = slots;
  const size_t ent = (size_t)slots * pl->n_heads;
  pl->acc_off = 0;
  pl->ml_off = (ent * decode_hd(pool->head_dim) * 4 + 255) & ~(size_t)255;
  pl->ws_bytes = slots && decode_tuned(pool)
                     ? pl->ml_off + ((ent * 2 * 4 + 255) & ~(size_t)255)
                     : 0;
  return RVKV_OK;
}

int plan_check_args(const char *op, const rvkv_pool *pool,
                    const uint32_t *ctx_lens_host, uint32_t batch,
                    uint32_t n_heads) {
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (batch == 0 || !ctx_lens_host)
    return fail(RVKV_EINVAL, op, "batch must be positive, ctx_lens non-NULL");
  if (batch > 65535) return fail(RVKV_EUNSUPPORTED, op, "batch too large");
  if (n_heads == 0 || n_heads % pool->n_kv != 0)
    return fail(RVKV_EINVAL, op,
                "n_heads must be a positive multiple of n_kv_heads");
  return RVKV_OK;
}

}  // namespace

// Decode partials of rvkv_paged_decode_noalloc: one array per GPU, for the
// life of the process. Host code never uses this name as an address (it
// is a host-side stand-in); scratch_device_ptr() returns the device's copy.
// 8 MiB holds the partials of every uniform decode up to head_dim 256 with
// up to 4 query heads per KV head (at most ~1024*G partial rows, each
// (head_dim + 2) floats), any batch.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];
// Cross-stream ordering of the scratch array: the stream of the last call
// that used it and an event recorded on that stream after its launches.
// A call on another stream waits on that event first, so calls on
// different streams of one device serialise on the array instead of
// overwriting each other's partials.
hipEvent_t g_scratch_done[kMaxDevices];
hipStream_t g_scratch_stream[kMaxDevices];
bool g_scratch_used[kMaxDevices];

// Device `dev`'s copy of `scratch`, looked up once per device (with that
// device current; the caller's current device is restored).
int scratch_device_ptr(const char *op, int dev, void **out) {
  if (dev < 0 || dev >= kMaxDevices)
    return fail(RVKV_EUNSUPPORTED, op, "device index too large");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(op, e);
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return hip_fail(op, e);
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    hipEvent_t ev = nullptr;
    if (e == hipSuccess)
      e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess) return hip_fail(op, e);
    if (!ptr) return fail(RVKV_EHIP, op, "scratch has no device address");
    g_scratch_ptr[dev] = ptr;
    g_scratch_done[dev] = ev;
  }
  *out = g_scratch_ptr[dev];
  return RVKV_OK;
}

// Orders this call's use of device `dev`'s scratch array after the last
// call's when that one ran on another stream (the caller holds
// g_scratch_mu from here until scratch_release, so calls from several
// threads take the array one at a time). A stream under graph capture
// is not ordered (an event recorded outside the capture cannot be waited
// on inside it): a captured graph's replays race with calls on other
// streams, as the header states.
int scratch_acquire(const char *op, int dev, hipStream_t stream,
                    bool *capturing) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cs);
  if (e != hipSuccess) return hip_fail(op, e);
  *capturing = cs != hipStreamCaptureStatusNone;
  if (*capturing) return RVKV_OK;
  if (g_scratch_used[dev] && g_scratch_stream[dev] != stream &&
      (e = hipStreamWaitEvent(stream, g_scratch_done[dev], 0)) != hipSuccess)
    return hip_fail(op, e);
  return RVKV_OK;
}

// Records the end of this call's launches on `stream` for the next caller.
int scratch_release(const char *op, int dev, hipStream_t stream) {
  hipError_t e = hipEventRecord(g_scratch_done[dev], stream);
  if (e != hipSuccess) return hip_fail(op, e);
  g_scratch_stream[dev] = stream;
  g_scratch_used[dev] = true;
  return RVKV_OK;
}

int paged_decode_ws(const char *op, const rvkv_pool *pool, uint32_t layer,
                    const float *q, const uint32_t *block_tables,
                    const uint32_t *ctx_lens, uint32_t batch,
                    uint32_t max_blocks, uint32_t n_heads,
                    uint32_t max_ctx_len, float scale, int32_t window,
                    float *out, void *ws, size_t ws_bytes, bool no_alloc);

// A decode without a plan on the matrix cores: a.n_parts uniform
// partitions of a.part_tokens keys a sequence (one wave each), then the
// uniform reduction pass when some sequence spans several.
int uniform_mfma(const char *op, const rvkv_pool *pool, uint32_t layer,
                 const DecodeArgs &a, uint32_t batch, float scale) {
  uint32_t ksplit = 1;
  static const uint32_t forced = env_u32("RVKV_DECODE_PART_TOKENS");
  if (!forced)
    mfma_uniform_parts((uint64_t)batch * pool->n_kv, a.ctx_cap, &ksplit);
  int rc = rvkv_detail::mfma_decode(
      pool, layer, a.q, a.tables, a.ctx_lens, a.max_blocks, a.n_heads, scale,
      a.window, nullptr, batch * a.n_parts, a.ws_acc, a.ws_ml, a.out,
      a.new_k, a.new_v, a.new_blk, a.new_off, a.new_f32 != 0, nullptr,
      a.n_parts, a.part_tokens, a.ctx_cap, ksplit);
  if (rc || a.n_parts <= 1) return rc;
  return launch_reduce(op, a, decode_hd(pool->head_dim),
                       dim3(a.n_heads, batch), pool->stream);
}

}  // namespace

extern "C" {

int rvkv_paged_decode(const rvkv_pool *pool, uint32_t layer, const float *q,
                      const uint32_t *block_tables, const uint32_t *ctx_lens,
                      uint32_t batch, uint32_t max_blocks, uint32_t n_heads,
                      uint32_t max_ctx_len, float scale, int32_t window,
                      float *out, void *ws, size_t ws_bytes) {
  return paged_decode_ws("paged_decode", pool, layer, q, block_tables,
                         ctx_lens, batch, max_blocks, n_heads, max_ctx_len,
                         scale, window, out, ws, ws_bytes, false);
}

int rvkv_paged_decode_noalloc(const rvkv_pool *pool, uint32_t layer,
                              const float *q, const uint32_t *block_tables,
                              const uint32_t *ctx_lens, uint32_t batch,
                              uint32_t max_blocks, uint32_t n_heads,
                              uint32_t max_ctx_len, float scale,
                              int32_t window, float *out) {
  return paged_decode_ws("paged_decode_noalloc", pool, layer, q,
                         block_tables, ctx_lens, batch, max_blocks, n_heads,
                         max_ctx_len, scale, window, out, nullptr, 0, true);
}

}  // extern "C"

namespace {

int paged_decode_ws(const char *op, const rvkv_pool *pool, uint32_t layer,
                    const float *q, const uint32_t *block_tables,
                    const uint32_t *ctx_lens, uint32_t batch,
                    uint32_t max_blocks, uint32_t n_heads,
                    uint32_t max_ctx_len, float scale, int32_t window,
                    float *out, void *ws, size_t ws_bytes, bool no_alloc) {
  if (pool && batch == 0) return RVKV_OK;
  DecodeArgs a;
  uint32_t gt;
  int rc = prepare_decode(op, pool, layer, q, block_tables, ctx_lens,
                          max_blocks, n_heads, max_ctx_len, scale, window,
                          out, &a, &gt);
  if (rc) return rc;
  if (batch > 65535) return fail(RVKV_EUNSUPPORTED, op, "batch too large");
  if (a.generic) return decode_generic(op, pool, layer, a, batch, scale);
  if (max_ctx_len == 0) max_ctx_len = 1;
  const WsLayout w = ws_layout(pool, batch, n_heads, max_ctx_len);
  if (no_alloc && w.bytes > 0) {
    // The partials go to this device's static scratch array: no
    // allocation, and nothing in it needs clearing (every partial the
    // reduction reads is written by this call's first launch).
    if (w.bytes > kScratchBytes)
      return fail(RVKV_EUNSUPPORTED, op,
                  "decode partials exceed the 8 MiB scratch; use "
                  "rvkv_paged_decode with a workspace");
    if ((rc = scratch_device_ptr(op, pool->device, &ws))) return rc;
    ws_bytes = kScratchBytes;
  }
  if ((rc = check_ws(op, ws, ws_bytes, w.bytes))) return rc;
  a.ws_acc = w.n_parts > 1 ? (float *)((char *)ws + w.acc_off) : nullptr;
  a.ws_ml = w.n_parts > 1 ? (float *)((char *)ws + w.ml_off) : nullptr;
  a.part_tokens = partition_tokens(pool, batch, n_heads, max_ctx_len);
  a.n_parts = w.n_parts;
  a.avg_tokens = a.part_tokens < max_ctx_len ? a.part_tokens : max_ctx_len;
  a.max_tokens = a.avg_tokens;
  const dim3 grid(w.n_parts, pool->n_kv * a.n_sub, batch);
  const bool ordered = no_alloc && w.bytes > 0;
  bool capturing = false;
  std::unique_lock<std::mutex> lock(g_scratch_mu, std::defer_lock);
  if (ordered) lock.lock();
  if (ordered &&
      (rc = scratch_acquire(op, pool->device, pool->stream, &capturing)))
    return rc;
  rc = rvkv_detail::mfma_decode_wanted(pool, n_heads)
           ? uniform_mfma(op, pool, layer, a, batch, scale)
           : launch_decode_pair(op, a, decode_hd(pool->head_dim), gt, grid,
                                dim3(n_heads, batch), w.n_parts > 1,
                                pool->stream);
  if (rc == RVKV_OK && ordered && !capturing)
    rc = scratch_release(op, pool->device, pool->stream);
  return rc;
}

}  // namespace

extern "C" {

int rvkv_decode_plan_create(const rvkv_pool *pool,
                            const uint32_t *ctx_lens_host, uint32_t batch,
                            uint32_t n_heads, int32_t window,
                            rvkv_decode_plan **out) {
  const char *op = "decode_plan";
  if (!out) return fail(RVKV_EINVAL, op, "out is NULL");
  *out = nullptr;
  int rc = plan_check_args(op, pool, ctx_lens_host, batch, n_heads);
  if (rc) return rc;
  rvkv_decode_plan *pl = new rvkv_decode_plan();
  pl->pool = pool;
  pl->n_heads = n_heads;
  pl->n_kv = pool->n_kv;
  pl->head_dim = pool->head_dim;
  pl->window = window;
  if ((rc = plan_build(pl, ctx_lens_host, batch))) {
    rvkv_decode_plan_destroy(pl);
    return rc;
  }
  *out = pl;
  return RVKV_OK;
}

int rvkv_decode_plan_update(rvkv_decode_plan *plan,
                            const uint32_t *ctx_lens_host, uint32_t batch) {
  return rvkv_decode_plan_update_tables(plan, ctx_lens_host, nullptr, 0,
                                        batch);
}

int rvkv_decode_plan_update_tables(rvkv_decode_plan *plan,
                                   const uint32_t *ctx_lens_host,
                                   const uint32_t *tables_host,
                                   uint32_t max_blocks, uint32_t batch) {
  const char *op = "decode_plan";
  if (!plan) return fail(RVKV_EINVAL, op, "plan is NULL");
  int rc = plan_check_args(op, plan->pool, ctx_lens_host, batch,
                           plan->n_heads);
  if (rc) return rc;
  if (tables_host && max_blocks == 0)
    return fail(RVKV_EINVAL, op, "max_blocks must be positive with tables");
  return plan_build(plan, ctx_lens_host, batch, tables_host, max_blocks);
}

void rvkv_decode_plan_destroy(rvkv_decode_plan *plan) {
  if (!plan) return;
  // Decodes queued with this plan may still read its device list.
  (void)hipStreamSynchronize(plan->pool->stream);
  for (int i = 0; i < rvkv_decode_plan::kNStage; ++i) {
    if (plan->uploaded[i]) (void)hipEventDestroy(plan->uploaded[i]);
    if (plan->h_buf[i]) (void)hipHostFree(plan->h_buf[i]);
  }
  if (plan->d_buf) (void)hipFree(plan->d_buf);
  delete plan;
}

size_t rvkv_decode_plan_workspace_bytes(const rvkv_decode_plan *plan) {
  return plan ? plan->ws_bytes : 0;
}

uint32_t rvkv_decode_plan_items(const rvkv_decode_plan *plan) {
  return plan ? plan->n_items : 0;
}

int rvkv_paged_decode_planned(const rvkv_pool *pool,
                              const rvkv_decode_plan *plan, uint32_t layer,
                              const float *q, const uint32_t *block_tables,
                              const uint32_t *ctx_lens, uint32_t max_blocks,
                              float scale, float *out, void *ws,
                              size_t ws_bytes) {
  const char *op = "paged_decode";
  if (!plan) return fail(RVKV_EINVAL, op, "plan is NULL");
  if (pool && (plan->n_kv != pool->n_kv || plan->head_dim != pool->head_dim))
    return fail(RVKV_EINVAL, op, "plan was built for another pool shape");
  DecodeArgs a;
  uint32_t gt;
  int rc = prepare_decode(op, pool, layer, q, block_tables, ctx_lens,
                          max_blocks, plan->n_heads, plan->max_ctx, scale,
                          plan->window, out, &a, &gt);
  if (rc) return rc;
  if (a.generic) return decode_generic(op, pool, layer, a, plan->batch, scale);
  if ((rc = check_ws(op, ws, ws_bytes, plan->ws_bytes))) return rc;
  a.ws_acc = plan->n_slots ? (float *)((char *)ws + plan->acc_off) : nullptr;
  a.ws_ml = plan->n_slots ? (float *)((char *)ws + plan->ml_off) : nullptr;
  a.items = plan->d_buf;
  a.reds = plan->d_buf + plan->n_items;
  a.part_tokens = plan->part_tokens;
  a.avg_tokens = plan->avg_tokens;
  a.max_tokens = plan->max_tokens;
  a.n_parts = 1;
  if (rvkv_detail::mfma_decode_wanted(pool, plan->n_heads))
    return planned_mfma(op, pool, plan, layer, a, max_blocks, scale);
  const dim3 grid(plan->n_items, pool->n_kv * a.n_sub, 1);
  return launch_decode_pair(op, a, decode_hd(pool->head_dim), gt, grid,
                            dim3(plan->n_heads, plan->n_reds ? plan->n_reds : 1),
                            plan->n_reds > 0, pool->stream);
}

int rvkv_decode_step(rvkv_pool *pool, const rvkv_decode_plan *plan,
                     uint32_t layer, const void *k, const void *v,
                     rvkv_dtype src_dtype, const uint32_t *slot_block,
                     const uint32_t *slot_off, const float *q,
                     const uint32_t *block_tables, const uint32_t *ctx_lens,
                     uint32_t batch, uint32_t max_blocks, uint32_t n_heads,
                     uint32_t max_ctx_len, float scale, int32_t window,
                     float *out, void *ws, size_t ws_bytes) {
  const char *op = "decode_step";
  if (!k || !v || !slot_block || !slot_off)
    return fail(RVKV_EINVAL, op, "NULL k/v/block_ids/offsets");
  if (src_dtype != RVKV_F16 && src_dtype != RVKV_F32)
    return fail(RVKV_EINVAL, op, "src dtype must be F16 or F32");
  if ((uintptr_t)k % 16 || (uintptr_t)v % 16)
    return fail(RVKV_EINVAL, op, "k/v must be 16-byte aligned");
  if (plan) {
    if (plan->batch != batch)
      return fail(RVKV_EINVAL, op, "batch differs from the plan's");
    if (plan->n_heads != n_heads || plan->window != window)
      return fail(RVKV_EINVAL, op, "n_heads/window differ from the plan's");
  }
  if (pool && batch == 0) return RVKV_OK;
  DecodeArgs a;
  uint32_t gt;
  int rc = prepare_decode(op, pool, layer, q, block_tables, ctx_lens,
                          max_blocks, n_heads,
                          plan ? plan->max_ctx : max_ctx_len, scale, window,
                          out, &a, &gt);
  if (rc) return rc;
  if (a.generic) {
    // The generic kernel: the append and the decode as two launches on the
    // stream. Every check runs before the append, so a refused call leaves
    // the cache unchanged.
    if (plan) {
      if (plan->n_kv != pool->n_kv || plan->head_dim != pool->head_dim)
        return fail(RVKV_EINVAL, op, "plan was built for another pool shape");
    } else if (batch > 65535) {
      return fail(RVKV_EUNSUPPORTED, op, "batch too large");
    }
    if ((rc = rvkv_append(pool, layer, k, v, src_dtype, slot_block, slot_off,
                          batch)))
      return rc;
    return decode_generic(op, pool, layer, a, batch, scale);
  } else {
    a.new_k = k;
    a.new_v = v;
    a.new_blk = slot_block;
    a.new_off = slot_off;
    a.new_f32 = src_dtype == RVKV_F32;
  }
  if (plan) {
    if (plan->n_kv != pool->n_kv || plan->head_dim != pool->head_dim)
      return fail(RVKV_EINVAL, op, "plan was built for another pool shape");
    if ((rc = check_ws(op, ws, ws_bytes, plan->ws_bytes))) return rc;
    a.ws_acc = plan->n_slots ? (float *)((char *)ws + plan->acc_off) : nullptr;
    a.ws_ml = plan->n_slots ? (float *)((char *)ws + plan->ml_off) : nullptr;
    a.items = plan->d_buf;
    a.reds = plan->d_buf + plan->n_items;
    a.part_tokens = plan->part_tokens;
    a.avg_tokens = plan->avg_tokens;
    a.max_tokens = plan->max_tokens;
    a.n_parts = 1;
    if (rvkv_detail::mfma_decode_wanted(pool, n_heads))
      return planned_mfma(op, pool, plan, layer, a, max_blocks, scale);
    const dim3 grid(plan->n_items, pool->n_kv * a.n_sub, 1);
    return launch_decode_pair(
        op, a, decode_hd(pool->head_dim), gt, grid,
        dim3(plan->n_heads, plan->n_reds ? plan->n_reds : 1),
        plan->n_reds > 0, pool->stream);
  }
  if (batch > 65535) return fail(RVKV_EUNSUPPORTED, op, "batch too large");
  if (max_ctx_len == 0) max_ctx_len = 1;
  const WsLayout w = ws_layout(pool, batch, n_heads, max_ctx_len);
  if ((rc = check_ws(op, ws, ws_bytes, w.bytes))) return rc;
  a.ws_acc = w.n_parts > 1 ? (float *)((char *)ws + w.acc_off) : nullptr;
  a.ws_ml = w.n_parts > 1 ? (float *)((char *)ws + w.ml_off) : nullptr;
  a.part_tokens = partition_tokens(pool, batch, n_heads, max_ctx_len);
  a.n_parts = w.n_parts;
  a.avg_tokens = a.part_tokens < max_ctx_len ? a.part_tokens : max_ctx_len;
  a.max_tokens = a.avg_tokens;
  if (rvkv_detail::mfma_decode_wanted(pool, n_heads))
    return uniform_mfma(op, pool, layer, a, batch, scale);
  const dim3 grid(w.n_parts, pool->n_kv * a.n_sub, batch);
  return launch_decode_pair(op, a, decode_hd(pool->head_dim), gt, grid,
                            dim3(n_heads, batch), w.n_parts > 1, pool->stream);
}

}  // extern "C"

namespace {

// Shared by the split (q, k, v) and the fused (qkv) entry points; q and
// k/v rows are q_stride / kv_stride floats apart.
int attn_prep_impl(rvkv_pool *pool, uint32_t layer, const float *q_in,
                   const float *k_in, const float *v_in, uint32_t q_stride,
                   uint32_t kv_stride, uint32_t rows, uint32_t n_heads,
                   const float *q_bias, const float *k_bias,
                   const float *v_bias, const float *q_norm,
                   const float *k_norm, float eps, const float *cos_t,
                   const float *sin_t, const uint32_t *slot_block,
                   const uint32_t *slot_off, float *q_out) {
  const char *op = "attn_prep";
  const uint32_t hd = pool->head_dim;
  PrepArgs a{};
  a.q_in = q_in;
  a.k_in = k_in;
  a.v_in = v_in;
  a.q_bias = q_bias;
  a.k_bias = k_bias;
  a.v_bias = v_bias;
  a.q_norm = q_norm;
  a.k_norm = k_norm;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.slot_block = slot_block;
  a.slot_off = slot_off;
  a.q_out = q_out;
  a.kc = pool->tensor(layer, 0);
  a.vc = pool->tensor(layer, 1);
  a.rows = rows;
  a.n_heads = n_heads;
  a.n_kv = pool->n_kv;
  a.num_blocks = pool->num_blocks;
  a.bs = pool->block_size;
  a.q_stride = q_stride;
  a.kv_stride = kv_stride;
  a.hd = hd;
  a.eps = eps;
  for (const void *p : {(const void *)q_in, (const void *)k_in,
                        (const void *)v_in, (const void *)q_bias,
                        (const void *)k_bias, (const void *)v_bias,
                        (const void *)q_norm, (const void *)k_norm,
                        (const void *)cos_t, (const void *)sin_t,
                        (const void *)q_out})
    if ((uintptr_t)p % 16)
      return fail(RVKV_EINVAL, op, "float buffers must be 16-byte aligned");
  const uint64_t items = (uint64_t)rows * (n_heads + 2 * pool->n_kv);
  if (items > 0xffffffffull)
    return fail(RVKV_EUNSUPPORTED, op, "too many rows for one launch");
  if (pool->f32() || !hd_supported(hd)) {
    if (items > 0x7fffffffull)
      return fail(RVKV_EUNSUPPORTED, op, "too many rows for one launch");
    const dim3 grid((uint32_t)items);
    if (pool->f32())
      hipLaunchKernelGGL(attn_prep_generic_kernel<float>, grid, dim3(64), 0,
                         pool->stream, a);
    else
      hipLaunchKernelGGL(attn_prep_generic_kernel<_Float16>, grid, dim3(64),
                         0, pool->stream, a);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
  }
  const uint32_t per_block = 256 / (hd / 16);
  const dim3 grid((uint32_t)((items + per_block - 1) / per_block));
  switch (hd) {
    case 32: hipLaunchKernelGGL(attn_prep_kernel<32>, grid, dim3(256), 0, pool->stream, a); break;
    case 64: hipLaunchKernelGGL(attn_prep_kernel<64>, grid, dim3(256), 0, pool->stream, a); break;
    case 128: hipLaunchKernelGGL(attn_prep_kernel<128>, grid, dim3(256), 0, pool->stream, a); break;
    default: hipLaunchKernelGGL(attn_prep_kernel<256>, grid, dim3(256), 0, pool->stream, a); break;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

// Validation common to both entry points; 1 = proceed, 0 = nothing to do,
// < 0 = error code.
int attn_prep_check(rvkv_pool *pool, uint32_t layer, uint32_t rows,
                    uint32_t n_heads) {
  const char *op = "attn_prep";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers)
    return fail(RVKV_EINVAL, op, "layer out of range");
  if (rows == 0) return 0;
  if (n_heads == 0 || n_heads % pool->n_kv != 0)
    return fail(RVKV_EINVAL, op,
                "n_heads must be a positive multiple of n_kv_heads");
  if (pool->head_dim % 2 != 0 || pool->head_dim > 1024)
    return fail(RVKV_EUNSUPPORTED, op,
                "head_dim must be even and at most 1024");
  return 1;
}

}  // namespace

extern "C" {

int rvkv_attn_prep(rvkv_pool *pool, uint32_t layer, const float *q_in,
                   const float *k_in, const float *v_in, uint32_t rows,
                   uint32_t n_heads, const float *q_bias, const float *k_bias,
                   const float *v_bias, const float *q_norm,
                   const float *k_norm, float eps, const float *cos_t,
                   const float *sin_t, const uint32_t *slot_block,
                   const uint32_t *slot_off, float *q_out) {
  const int rc = attn_prep_check(pool, layer, rows, n_heads);
  if (rc <= 0) return rc;
  if (!q_in || !k_in || !v_in || !cos_t || !sin_t || !slot_block ||
      !slot_off || !q_out)
    return fail(RVKV_EINVAL, "attn_prep",
                "NULL q/k/v/cos/sin/block_ids/offsets/q_out");
  const uint32_t hd = pool->head_dim;
  return attn_prep_impl(pool, layer, q_in, k_in, v_in, n_heads * hd,
                        pool->n_kv * hd, rows, n_heads, q_bias, k_bias,
                        v_bias, q_norm, k_norm, eps, cos_t, sin_t,
                        slot_block, slot_off, q_out);
}

int rvkv_attn_prep_qkv(rvkv_pool *pool, uint32_t layer, const float *qkv,
                       uint32_t rows, uint32_t n_heads, const float *bias,
                       const float *q_norm, const float *k_norm, float eps,
                       const float *cos_t, const float *sin_t,
                       const uint32_t *block_ids, const uint32_t *offsets,
                       float *q_out) {
  const int rc = attn_prep_check(pool, layer, rows, n_heads);
  if (rc <= 0) return rc;
  if (!qkv || !cos_t || !sin_t || !block_ids || !offsets || !q_out)
    return fail(RVKV_EINVAL, "attn_prep",
                "NULL qkv/cos/sin/block_ids/offsets/q_out");
  const uint32_t hd = pool->head_dim, kv = pool->n_kv;
  const uint32_t width = (n_heads + 2 * kv) * hd;  // the QKV width
  return attn_prep_impl(
      pool, layer, qkv, qkv + (size_t)n_heads * hd,
      qkv + (size_t)(n_heads + kv) * hd, width, width, rows, n_heads, bias,
      bias ? bias + (size_t)n_heads * hd : nullptr,
      bias ? bias + (size_t)(n_heads + kv) * hd : nullptr, q_norm, k_norm,
      eps, cos_t, sin_t, block_ids, offsets, q_out);
}

int rvkv_copy_blocks(rvkv_pool *pool, const uint32_t *src, const uint32_t *dst,
                     uint32_t n) {
  const char *op = "copy_blocks";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (n == 0) return RVKV_OK;
  if (!src || !dst) return fail(RVKV_EINVAL, op, "NULL src/dst");
  if (n > 65535) return fail(RVKV_EUNSUPPORTED, op, "at most 65535 pairs per call");
  const size_t bytes = pool->block16 * 2;
  const bool w16 = bytes % 16 == 0;
  const size_t words = w16 ? bytes / 16 : bytes / 2;
  uint32_t gx = grid_1d(words, 256);
  if (gx > 64) gx = 64;
  const dim3 grid(gx, n, 2 * pool->n_layers);
  if (w16)
    hipLaunchKernelGGL(copy_blocks_kernel<uint4>, grid, dim3(256), 0,
                       pool->stream, pool->base, src, dst, pool->tensor16,
                       pool->block16, pool->num_blocks);
  else
    hipLaunchKernelGGL(copy_blocks_kernel<uint16_t>, grid, dim3(256), 0,
                       pool->stream, pool->base, src, dst, pool->tensor16,
                       pool->block16, pool->num_blocks);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

int rvkv_read_blocks(const rvkv_pool *pool, uint32_t layer, uint32_t which,
                     const uint32_t *block_ids, uint32_t n, void *out) {
  const char *op = "read_blocks";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers || which > 1)
    return fail(RVKV_EINVAL, op, "layer or which out of range");
  if (n == 0) return RVKV_OK;
  if (!block_ids || !out) return fail(RVKV_EINVAL, op, "NULL block_ids/out");
  const dim3 grid(grid_1d((uint64_t)pool->block16 * n, 256));
  hipLaunchKernelGGL(read_blocks_kernel, grid, dim3(256), 0, pool->stream,
                     pool->tensor(layer, which), block_ids, n,
                     static_cast<uint16_t *>(out), pool->block_size,
                     pool->n_kv, pool->hd16, pool->num_blocks);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

int rvkv_block_checksums(const rvkv_pool *pool, uint32_t layer,
                         uint32_t which, const uint32_t *block_ids, uint32_t n,
                         uint64_t *out) {
  const char *op = "block_checksums";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers || which > 1)
    return fail(RVKV_EINVAL, op, "layer or which out of range");
  if (n == 0) return RVKV_OK;
  if (!block_ids || !out) return fail(RVKV_EINVAL, op, "NULL block_ids/out");
  hipLaunchKernelGGL(checksum_kernel, dim3(grid_1d(n, 64)), dim3(64), 0,
                     pool->stream, pool->tensor(layer, which), block_ids, n,
                     out, pool->block_size, pool->n_kv, pool->hd16,
                     pool->num_blocks);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

}  // extern "C"
