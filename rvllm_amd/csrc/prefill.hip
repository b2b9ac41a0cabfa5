// prefill.hip - paged prefill / chunked-prefill attention (q_len >= 1 query
// rows per sequence, causal, optional sliding window) straight over the
// paged f16 cache, on the gfx950 matrix cores.
//
// What it computes is rvllm's prefill attention: gather the sequence's keys
// through its block table, add batch_mask and run gqa_attention
// (src/model.rs:346-415, called at src/model.rs:628-644; the CUDA backend's
// kv_gather + cuBLAS scores + mask + softmax + apply, src/cuda/model.rs:
// 528-569). Row i of sequence b sits at position p = pos_offset[b] + i and
// sees key j iff j < read_num_tokens[b], j <= p and (window > 0) j + window
// > p. A row that sees no key gets zeros.
//
// Work split: one workgroup = (sequence, KV head, tile of 128 query rows),
// four wave64s of 32 rows each. The rows of a KV head are the GQA group
// folded into the query axis, row r = (query qi = r / G, head g = r % G), so
// every key/value tile read from HBM serves G heads * 128/G positions.
// Keys stream in tiles of 64 through LDS; the next tile's global loads are
// in flight while the current one is computed. At head_dim 256 a workgroup
// is eight waves in four pairs; the two waves of a pair hold the same 32
// rows and one half of the head dimension each (tiles of 32 keys).
//
// Matrix layout (v_mfma_f32_32x32x16_f16, f32 accumulate):
//   S^T = K . Q^T   (M = 32 keys, N = 32 query rows, K = 16 of head_dim)
//   O^T = V^T . P^T (M = 32 of head_dim, N = 32 query rows, K = 16 keys)
// With S transposed every lane holds ONE query row (lane % 32) and 16 keys
// of each 32-key sub-tile, so the online-softmax max/sum is in-lane plus one
// exchange with lane ^ 32, and the probabilities feed the P.V product from
// registers. The K rows are fed to the S product in a permuted order
// sigma(m) chosen so that accumulator register j of lane-half h holds key
// 16*(j/8) + 8*h + j%8: that is exactly the k-slot order the P^T operand
// needs (8 consecutive keys per lane-half), so no lane shuffles are needed.
// V is the one operand read across its rows (8 keys of one d column); it is
// staged transposed in LDS, Vt[d][key], so that read is one 16-byte load.
//
// q is pre-scaled by scale*log2(e) and split into f16 hi + lo parts, each
// multiplied with K on the matrix cores (so scores keep q's f32 precision);
// probabilities are rounded to f16 and the row sum adds the rounded values,
// so numerator and denominator see the same weights. Products are exact in
// f32; sums are f32.
#include "pool.h"

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <type_traits>

using rvkv_detail::fail;
using rvkv_detail::hip_fail;

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A 16-byte K/V load; NT: with the non-temporal hint, for bytes read once
// (the decode mode), where it reads ~5 % faster; prefill tiles are re-read
// by a head's other query tiles through the L2 and load normally.
template <bool NT>
__device__ __forceinline__ u32x4 ld16(const char *p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  else
    return *reinterpret_cast<const u32x4 *>(p);
}
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));

// Four f16 of an LDS column, transposed across the 16-lane group.
__device__ __forceinline__ v4h tr_read(const uint16_t *p) {
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s *)(p));
  return __builtin_bit_cast(v4h, r);
}

// Keys per tile: 64, or 32 at head_dim 256 (one 32-key sub-tile keeps the
// S accumulators and the tile's load registers within the register file).
// (32 also for one-wave decode workgroups, whose single wave loads the
// whole tile.)
template <int HD, int WAVES>
constexpr int tile_keys() {
  return HD >= 256 || WAVES == 1 ? 32 : 64;
}
constexpr int kWaveRows = 32;  // query rows per wave
// V in LDS: row-major like K, read transposed (ds_read_b64_tr_b16) for the
// P.V product, or stored transposed. Row-major measured 1.4-2.6 % faster at
// head_dim 64 (prefill and the decode mode); transposed was as fast or up to
// 2.4 % faster at 128 and 256, where the P.V product issues more V reads.
constexpr bool v_rowmajor(int hd) { return hd <= 64; }
// Tiles staged by LDS DMA (buffer_load_dwordx4 / global_load_lds_dwordx4
// with the LDS flag: each lane's 16 bytes go from memory straight into LDS,
// no staging registers and no LDS stores):
// head_dim 64 and 128 in 4-wave workgroups. Without staging registers two
// such workgroups fit on a CU at 128, each with its own barrier, so the two
// waves of a SIMD are not held in the same phase (one's softmax can overlap
// the other's matrix work). Rows are unpadded (a lane writes 16 consecutive
// bytes of the wave's 1 KiB); chunk c of row r sits in slot c ^ swz(r).
template <int HD, int WAVES>
constexpr bool dma_tiles() { return (HD == 64 || HD == 128) && WAVES == 4; }
// The slot swizzle (LDS serves 64 banks of 4 bytes, 256 bytes, per cycle).
// A K fragment read (16 lanes, rows 0-15 of one chunk column) and a
// transposing V read (32 lanes, rows 4j..4j+3, four consecutive chunks)
// must each meet 16 different 16-byte bank groups.
// 256-byte rows (head_dim 128, 16 chunks): the two 2-bit halves of r % 16
// swapped. 128-byte rows (64, 8 chunks; two rows a bank cycle, told apart
// by bit 0 of r): bit 1 of r to bit 2 of the slot, bits 2-3 to bits 0-1.
template <int HD>
__device__ __forceinline__ uint32_t swz(uint32_t r) {
  if constexpr (HD == 128)
    return ((r & 3u) << 2) | ((r >> 2) & 3u);
  else
    return (((r >> 1) & 1u) << 2) | ((r >> 2) & 3u);
}
// At head_dim 256 the two waves of a pair share 32 query rows: each holds
// half of the head dimension of Q and O (the S product's two halves are
// added through LDS), so a wave's O and Q fit two waves per SIMD.
constexpr bool split_dims(int hd) { return hd >= 256; }
template <int HD, int WAVES>
constexpr int block_rows() {
  return kWaveRows * (split_dims(HD) ? WAVES / 2 : WAVES);
}
constexpr float kNegBig = -1.0e30f;      // finite start value of the row max

struct PrefillArgs {
  const float *q;  // [batch * q_len, n_heads, hd]
  float *out;      // same shape
  const uint16_t *kc, *vc;
  const uint32_t *tables;  // [batch, max_blocks]
  const uint32_t *pos_offset, *read_num;
  uint64_t block_stride;  // elements per block (all heads)
  uint32_t head_stride;   // elements per (block, head) tile
  uint32_t q_len, max_blocks, num_blocks, n_heads, group, bs_log2;
  uint32_t batch, n_kv;
  uint32_t rows;     // group * q_len rows per (sequence, KV head)
  uint32_t n_tiles;  // ceil(rows / rows per workgroup)
  float qscale;      // scale * log2(e)
  int32_t window;
  // Decode mode (q_len 1 at position read_num - 1) over a decode plan's
  // work items {seq, first key, end key, slot}: slot kNoSlot writes the
  // output; otherwise the unnormalised partial (acc, m, l) goes to ws_acc /
  // ws_ml [slot][n_heads] for the decode reduction pass. NULL: prefill.
  const uint4 *items;
  // Shared-prefix group items (seq field | kGroupItem): word offset of a
  // list {n, n sequences, n slots}; the group's n * group query rows share
  // the item's key range, whose blocks all members' tables hold alike.
  const uint32_t *groups;
  // Decode mode without a plan (items NULL, dec_parts > 0): grid.x =
  // sequence * dec_parts + partition, each partition dec_part_tokens keys
  // (slot = sequence * dec_parts + partition when the sequence spans more
  // than one, else the output is written), read counts capped at
  // dec_ctx_cap, as the VALU decode's uniform mode does.
  uint32_t dec_parts, dec_part_tokens, dec_ctx_cap;
  float *ws_acc, *ws_ml;
  // Fused append (decode mode): this step's K/V row of every sequence
  // ([batch, n_kv, hd], f32 or f16) goes to slot (new_blk[b], new_off[b])
  // and is the key at position ctx - 1; the work item holding that key
  // stores the row and uses it from registers. NULL: no append.
  const void *new_k, *new_v;
  const uint32_t *new_blk, *new_off;
  bool new_f32;
};

constexpr uint32_t kNoSlot = 0xFFFFFFFFu;
// 1 KiB of zeros: under LDS DMA the rows of keys that are not read (past
// the range, unreadable blocks) are loaded from here, so their V is 0 in
// LDS (masked keys get probability 0, and 0 * stale V must stay 0).
__device__ __align__(16) uint4 g_pf_zero[64];
// Buffer resource of one (block, head) tile for the DMA loads: byte range
// (the lane offsets stay below it) and word 3 (32-bit data format, the
// value raw buffer accesses use on this architecture).
constexpr int kRsrcBytes = 0x7fffffff;
constexpr int kRsrcWord3 = 0x00020000;

// One LDS DMA instruction by buffer load: lane l's 16 bytes at base + off
// go to lds + 16 l. base and lds are wave-uniform (a descriptor in scalar
// registers, M0); only the 32-bit offset is per lane.
__device__ __forceinline__ void dma16(const char *base, uint32_t off,
                                      unsigned char *lds) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      (void *)base, (short)0, kRsrcBytes, kRsrcWord3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void *)lds, 16, off, 0, 0, 0);
}
constexpr uint32_t kGroupItem = 0x80000000u;

template <int HD, int WAVES>
struct Lds {
  static constexpr int BN = tile_keys<HD, WAVES>();
  static constexpr bool DMA = dma_tiles<HD, WAVES>();
  // K row stride in halves (16 B pad; unpadded and swizzled under DMA)
  static constexpr int KS = DMA ? HD : HD + 8;
  // Row-major V stride: 32 halves of pad. The transposing reads of P.V
  // (four keys x four dims per 16 lanes) met 0.33 bank conflicts per LDS
  // access with 8, 16 or 24 halves of pad (Llama prefill, 17 M conflict
  // cycles a launch) and none with 32.
  static constexpr int VRS = DMA ? HD : HD + 32;
  static constexpr size_t k_bytes = (size_t)BN * KS * 2;
  static constexpr int VS = BN + 8;  // Vt row stride in halves (transposed)
  static constexpr size_t v_bytes =
      v_rowmajor(HD) || DMA ? (size_t)BN * VRS * 2 : (size_t)HD * VS * 2;
  // Workgroups of several waves double-buffer the tile, so one barrier a
  // tile both publishes it and retires the buffer the next tile overwrites
  // (a one-wave workgroup orders its own LDS accesses).
  static constexpr int NBUF = WAVES > 1 ? 2 : 1;
  static constexpr size_t buf = (k_bytes + v_bytes + BN + 15) / 16 * 16;
  // Split head dimension: one f32 S^T tile per wave for its partner.
  static constexpr size_t x_bytes =
      split_dims(HD) ? (size_t)WAVES * 64 * BN / 2 * 4 : 0;
  static constexpr size_t bytes = NBUF * buf + x_bytes;  // + key flags
};

// max(a, b, c): the compiler fuses it into one v_max3_f32 (it knows MFMA
// results need no NaN quieting). Not inline assembly: the compiler must see
// the read of the MFMA accumulators to insert the wait states the hardware
// requires between an MFMA's write of a register and a VALU read of it.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
}

// Lanes i and i ^ 32 combined: v_permlane32_swap of v with itself leaves
// the lower half's value in element 0 and the upper half's in element 1 of
// every lane, in the VALU (no LDS round trip as for a bpermute).
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false,
                                                  false);
  const uint32_t r0 = r[0], r1 = r[1];
  return vmax3(__uint_as_float(r0), __uint_as_float(r1), __uint_as_float(r1));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false,
                                                  false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __uint_as_float(r0) + __uint_as_float(r1);
}

// Eight elements of an appended K or V row as f16, rounded to nearest even
// from an f32 source exactly as the append kernel does.
__device__ __forceinline__ u32x4 new_row_chunk(const void *src, bool f32,
                                               size_t elem) {
  u32x4 r;
  if (f32) {
    const float4 *p =
        reinterpret_cast<const float4 *>(static_cast<const float *>(src) + elem);
    const float4 x = p[0], y = p[1];
    auto pk = [](float lo, float hi) {
      const _Float16 l = (_Float16)lo, h = (_Float16)hi;
      return (uint32_t)__builtin_bit_cast(uint16_t, l) |
             ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
    };
    r[0] = pk(x.x, x.y);
    r[1] = pk(x.z, x.w);
    r[2] = pk(y.x, y.y);
    r[3] = pk(y.z, y.w);
  } else {
    r = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(src) +
                                         elem);
  }
  return r;
}

__device__ __forceinline__ uint32_t lo_bound(uint32_t p, int32_t window) {
  return (window > 0 && p + 1 > (uint32_t)window) ? p + 1 - (uint32_t)window
                                                  : 0u;
}

// WAVES wave64s per workgroup (4 or 8, 32 query rows each); the K/V tile
// loads and LDS stores are shared among them, so more waves halve each
// wave's share of that work. Registers are bounded for 8 resident waves per
// CU at head_dim 128 and 256 (<= 256 a lane, so the O accumulators stay in
// arch VGPRs; at 256 only because each wave holds half of O and Q), 12
// below: two or more waves per SIMD overlap one's softmax with another's
// matrix work. (With all of O and Q in one wave, head_dim 256 ran one wave
// per SIMD, its S product serialised on LDS reads: 18 % slower. 128-key
// tiles at head_dim 64 were measured 7-9 % slower than 64.)
template <int HD, int WAVES, int KSPLIT = 1>
__global__ void __launch_bounds__(
    64 * WAVES * KSPLIT,
    // (a one-wave workgroup may share a SIMD with others: 2 bounds the
    // registers to two waves per SIMD)
    WAVES == 1 ? 2 : (HD <= 64 ? 12 : 8) / WAVES)
    prefill_kernel(PrefillArgs a) {
  constexpr int NTH = 64 * WAVES;  // threads per workgroup
  constexpr bool SPLIT = split_dims(HD);
  static_assert(!SPLIT || (WAVES % 2 == 0 && WAVES > 1), "wave pairs");
  constexpr int kBM = block_rows<HD, WAVES>();
  using LD = Lds<HD, WAVES>;
  constexpr int KS = LD::KS, VS = LD::VS, BN = LD::BN, VRS = LD::VRS;
  constexpr bool DMA = LD::DMA;
  constexpr bool TRV = v_rowmajor(HD) || DMA;
  constexpr int NT = BN / 32;                 // 32-key sub-tiles per tile
  // This wave's share of the head dimension: all of it, or one half.
  constexpr int KC = HD / 16 / (SPLIT ? 2 : 1);  // MFMA k-steps of S
  constexpr int DT = HD / 32 / (SPLIT ? 2 : 1);  // 32-row tiles of O^T
  constexpr int CPR = HD / 8;                 // 16-byte chunks per key row
  constexpr int CHK = BN * CPR / NTH;         // K chunks per thread per tile
  static_assert(CHK >= 1 && BN * CPR % NTH == 0, "tile/thread mismatch");
  static_assert(!DMA || ((CPR == 8 || CPR == 16) && !SPLIT && WAVES > 1),
                "DMA tiles: 8 or 16 chunks a row");
  extern __shared__ __align__(16) unsigned char smem_all[];
  // Decode items split over KSPLIT waves by keys (one-wave workgroups
  // only): each wave runs the one-wave loop over its share of the item's
  // keys in its own LDS region, and the waves' softmax states merge at the
  // end through LDS. tid is the thread's index within its wave then.
  static_assert(KSPLIT == 1 || WAVES == 1, "key split: one-wave items");
  const uint32_t kwave =
      KSPLIT > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0u;
  unsigned char *const smem = smem_all + kwave * LD::bytes;
  // Barriers among the threads that share one LDS region: the workgroup,
  // or with KSPLIT the wave (whose LDS accesses execute in order).
  auto region_sync = [&]() {
    if constexpr (KSPLIT > 1) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
      __syncthreads();
    }
  };
  auto region_or = [&](int x) {
    if constexpr (KSPLIT > 1)
      return __builtin_amdgcn_ballot_w64(x != 0) != 0;
    else
      return __syncthreads_or(x) != 0;
  };

  // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs
  // (each with its own L2), so workgroup w runs on XCD w % 8. Renumber so
  // each XCD gets a contiguous range of logical ids, in which the query
  // tiles of one (sequence, KV head) are adjacent: they re-read the same
  // K/V, which then stays in that XCD's L2. Within a head, long (late)
  // rows go first.
  uint32_t tile, kvh, b, item_lo = 0, item_hi = 0xFFFFFFFFu, slot = kNoSlot;
  // Group item: member list (n, sequences, slots); its first member's
  // table serves every member over the item's range.
  const uint32_t *gl = nullptr;
  uint32_t n_mem = 0;
  if (a.items) {  // decode items: grid (items, n_kv), plan order kept
    typedef const __attribute__((address_space(4))) uint32_t cu32;
    cu32 *itp = (cu32 *)(uintptr_t)(a.items + blockIdx.x);  // scalar loads
    const uint4 it = make_uint4(itp[0], itp[1], itp[2], itp[3]);
    b = it.x;
    item_lo = it.y;
    item_hi = it.z;
    slot = it.w;
    kvh = blockIdx.y;
    tile = 0;
    if (b & kGroupItem) {
      gl = a.groups + (b & ~kGroupItem);
      n_mem = gl[0];
      b = gl[1];
    }
  } else if (a.dec_parts) {  // uniform decode partitions
    b = blockIdx.x / a.dec_parts;
    const uint32_t part = blockIdx.x - b * a.dec_parts;
    item_lo = part * a.dec_part_tokens;
    item_hi = item_lo + a.dec_part_tokens;
    slot = a.dec_parts > 1 ? blockIdx.x : kNoSlot;
    kvh = blockIdx.y;
    if (a.dec_parts == 1 && gridDim.x % 8 == 0) {
      // One partition a sequence and a batch of whole eights: a sequence's
      // KV heads as consecutive workgroups of one XCD (linear id round robin
      // over the 8), as the VALU decode does (Llama-3.2-1B 256 x 4096:
      // 326.5 -> 325.9 us a layer).
      const uint32_t L = blockIdx.x + gridDim.x * blockIdx.y;
      const uint32_t xcd = L % 8, idx = L / 8;
      b = (idx / gridDim.y) * 8 + xcd;
      kvh = idx % gridDim.y;
    }
    tile = 0;
  } else {
    const uint32_t n_wg = a.n_tiles * a.n_kv * a.batch;
    const uint32_t w = blockIdx.x, xcd = w % 8, idx = w / 8;
    const uint32_t per = n_wg / 8, rem = n_wg % 8;
    const uint32_t logical =
        xcd < rem ? xcd * (per + 1) + idx
                  : rem * (per + 1) + (xcd - rem) * per + idx;
    tile = a.n_tiles - 1 - logical % a.n_tiles;
    kvh = (logical / a.n_tiles) % a.n_kv;
    b = logical / a.n_tiles / a.n_kv;
  }
  const int tid = KSPLIT > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Row group of the wave, and the half of the head dimension it holds.
  const uint32_t rgrp = SPLIT ? wave >> 1 : wave;
  const uint32_t dh = SPLIT ? wave & 1u : 0u;
  const int lane = tid & 63, hl = lane >> 5, ln = lane & 31;
  const uint32_t bs_mask = (1u << a.bs_log2) - 1u;

  // Decode: the one query row sits at position read_num - 1 (an empty
  // sequence wraps to 2^32 - 1 and sees no key).
  // (b is uniform: the per-sequence words come by scalar loads)
  typedef const __attribute__((address_space(4))) uint32_t cu32s;
  const bool decode = a.items || a.dec_parts;
  const uint32_t rn = a.dec_parts
                          ? min(*(cu32s *)(uintptr_t)(a.read_num + b),
                                a.dec_ctx_cap)
                          : *(cu32s *)(uintptr_t)(a.read_num + b);
  const uint32_t off =
      decode ? rn - 1u : *(cu32s *)(uintptr_t)(a.pos_offset + b);
  const uint32_t cap = a.max_blocks << a.bs_log2;
  const uint32_t ctx = min(rn, cap);
  if (a.dec_parts) {
    // One partition covers the sequence: its output is written directly
    // (the reduction skips it). A partition past the sequence's end has
    // nothing to do (the reduction never reads it); an empty sequence gets
    // its zero row from partition 0.
    if (ctx <= a.dec_part_tokens) slot = kNoSlot;
    if (item_lo >= ctx && item_lo > 0) return;
  }
  if constexpr (KSPLIT > 1) {
    // This wave's share of the item's keys, in whole tiles (item_lo is a
    // multiple of 256); a wave with none keeps an empty range.
    const uint32_t hi0 = min(item_hi, ctx);
    const uint32_t len = hi0 > item_lo ? hi0 - item_lo : 0u;
    const uint32_t sub = (len + KSPLIT * BN - 1) / (KSPLIT * BN) * BN;
    const uint32_t lo_w = min(item_lo + kwave * sub, max(hi0, item_lo));
    item_hi = min(lo_w + sub, max(hi0, item_lo));
    item_lo = lo_w;
  }
  const uint32_t *table = a.tables + (size_t)b * a.max_blocks;

  // Query rows of this (sequence, KV head): group * q_len, or a group
  // item's members' rows (each member one decode row per head).
  const uint32_t rows = gl ? n_mem * a.group : a.rows;
  // Key range any row of the workgroup sees, in whole tiles. (A group
  // item's range ends below every member's position, so ctx and off bound
  // none of it.)
  const uint32_t r_first = tile * kBM;
  const uint32_t r_last = min(r_first + kBM, rows) - 1u;
  const uint32_t k_end = min(min(ctx, off + r_last / a.group + 1u), item_hi);
  // (item_lo is a multiple of 256, so of BN)
  const uint32_t k_begin = max(
      lo_bound(off + r_first / a.group, a.window) & ~(uint32_t)(BN - 1),
      item_lo);

  // The same for this wave's 32 rows (wave-uniform).
  const uint32_t rw0 = r_first + rgrp * kWaveRows;
  const bool wave_live = rw0 < rows;
  const uint32_t rw1 = min(rw0 + kWaveRows, rows) - 1u;
  const uint32_t w_end =
      wave_live ? min(min(ctx, off + rw1 / a.group + 1u), item_hi) : 0u;
  const uint32_t w_begin = lo_bound(off + rw0 / a.group, a.window);
  // Keys every row of the wave sees: [w_lo_max, w_hi_min).
  const uint32_t w_hi_min =
      wave_live ? min(min(ctx, off + rw0 / a.group + 1u), item_hi) : 0u;
  const uint32_t w_lo_max = lo_bound(off + rw1 / a.group, a.window);

  // This lane's query row.
  const uint32_t r = rw0 + ln;
  const bool row_ok = r < rows;
  const uint32_t ri = row_ok ? r / a.group : 0u;
  const uint32_t head = kvh * a.group + (row_ok ? r - ri * a.group : 0u);
  // A group item's row ri / group is member ri's one decode row.
  const uint32_t qi = gl ? 0u : ri;
  const uint32_t bq = gl && row_ok ? gl[1 + ri] : b;
  const uint32_t my_slot = gl ? (row_ok ? gl[1 + n_mem + ri] : kNoSlot) : slot;
  const uint32_t p = off + qi;
  const uint32_t row_hi = row_ok ? min(min(ctx, p + 1u), item_hi) : 0u;
  const uint32_t row_lo = max(lo_bound(p, a.window), item_lo);
  const size_t qrow = ((size_t)bq * a.q_len + qi) * a.n_heads + head;
  // The appended key (fused decode step) when this item holds it.
  const uint32_t newtok =
      (a.new_k && ctx >= 1u && ctx - 1u >= item_lo && ctx - 1u < item_hi)
          ? ctx - 1u
          : 0xFFFFFFFFu;

  // q pre-scaled, as f16 hi + lo (lo = the rounding residual of hi): the S
  // product runs once on each, so scores keep q's f32 precision.
  half8 qf[KC], ql[KC];
  {
    const float *qp = a.q + qrow * HD + dh * (KC * 16);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int d0 = kc * 16 + hl * 8;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
      if (row_ok) {
        x = *reinterpret_cast<const float4 *>(qp + d0);
        y = *reinterpret_cast<const float4 *>(qp + d0 + 4);
      }
      const float xs[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        // hi: the f32 product rounded toward zero to f16 (one intrinsic,
        // so every use sees the same value; a plain conversion may be fused
        // with the product and rounded differently at different uses); lo:
        // the residual of the exact product (fma), rounded to f16.
        const h2 hp = __builtin_bit_cast(
            h2, __builtin_amdgcn_cvt_pkrtz(xs[e] * a.qscale,
                                           xs[e + 1] * a.qscale));
        qf[kc][e] = hp[0];
        qf[kc][e + 1] = hp[1];
        ql[kc][e] = (_Float16)__builtin_fmaf(xs[e], a.qscale, -(float)hp[0]);
        ql[kc][e + 1] =
            (_Float16)__builtin_fmaf(xs[e + 1], a.qscale, -(float)hp[1]);
      }
    }
  }

  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[t][j] = 0.f;
  float m = kNegBig, l = 0.f;

  // K row this lane feeds to the S product: sigma(ln), see the header.
  const int sig = 16 * (ln >> 4) + 8 * ((ln >> 2) & 1) + 4 * ((ln >> 3) & 1) +
                  (ln & 3);
  // ds_read_b64_tr_b16 over a 16-lane group: lane 4a + c of the group gets
  // element c of the 8-byte rows addressed by lanes a, a + 4, a + 8, a + 12.
  // For lane l to receive V[k0 + 8hl + e][d0 + l % 32], e = 0..3, group
  // lane s addresses key 8hl + s / 4 and dims 16 * (l / 16 % 2) + 4 (s % 4).
  const int tr_key = 8 * hl + ((lane & 15) >> 2);
  const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  const char *kbase = reinterpret_cast<const char *>(a.kc) +
                      (size_t)kvh * a.head_stride * 2;
  const char *vbase = reinterpret_cast<const char *>(a.vc) +
                      (size_t)kvh * a.head_stride * 2;
  // Tile loads. K goes to LDS row-major, so its 16-byte chunks are taken in
  // row order (chunk c: key c / CPR, column chunk c % CPR: whole rows per
  // lane group, coalesced). Row-major V (TRV) is taken the same way (a chunk
  // of K and the same chunk of V share key, block id and offset) and read
  // transposed with ds_read_b64_tr_b16. Transposed V is taken in key-pair
  // order (pair c % (BN/2), column chunk c / (BN/2)): a lane loads keys 2p
  // and 2p+1 of one column chunk and writes 8 dwords Vt[d][2p..2p+1];
  // consecutive lanes write consecutive dwords of one Vt row (with BN 64, a
  // half-wave covers the 32 banks once). Block ids are fetched one tile
  // ahead so a tile's loads issue back to back; loads are unconditional
  // (invalid ones read block 0) and invalid V is zeroed at the LDS store,
  // because masked keys get probability 0 and 0 * (stale V) must stay 0.
  constexpr int NPR = BN / 2;                     // key pairs per tile
  constexpr int VP = NPR * CPR;                   // V chunk pairs per tile
  constexpr int CHV = TRV ? 1 : (VP >= NTH ? VP / NTH : 1);  // per thread
  const bool v_lane = VP >= NTH || tid < VP;

  // Are all the blocks holding keys below k_end valid? One scan of its
  // table range (after the first tiles' loads are out, below; until then
  // all_ok is false, so those loads take the path that checks every block
  // id); then the masks need no per-key flags (key < row_hi already
  // implies key < k_end). Loads still check every block id themselves.
  bool all_ok = false;

  // Per-lane constants: tiles start at multiples of the tile width BN, so
  // a chunk's byte offset inside its (block, head) tile and its block index
  // relative to the tile's first block are the same for every tile (for
  // block_size > BN the tile's own offset inside the block is added per
  // tile).
  uint32_t k_key[CHK], k_off[CHK], k_db[CHK];
#pragma unroll
  for (int i = 0; i < CHK; ++i) {
    const int c = tid + NTH * i;
    k_key[i] = (uint32_t)(c / CPR);
    // (under DMA the chunk is read from the slot this lane writes)
    const uint32_t dc =
        DMA ? (uint32_t)(c % CPR) ^ swz<HD>(k_key[i]) : (uint32_t)(c % CPR);
    k_off[i] = ((k_key[i] & bs_mask) * HD + dc * 8) * 2;
    k_db[i] = k_key[i] >> a.bs_log2;
  }
  // (one block of all heads is far below 4 GiB; checked on the host)
  const uint32_t blk_bytes = (uint32_t)(a.block_stride * 2);
  // Tiles in flight: one ahead, or two for one-wave (decode) workgroups,
  // whose single wave's compute per tile is shorter than a load's latency.
  // (Two in multi-wave workgroups gained at most 1 %; not used.)
  // Register sets are selected by a compile-time index (a runtime index
  // would put the arrays in scratch).
  constexpr int DEPTH = WAVES == 1 ? 2 : 1;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, DEPTH - 1>;
  uint32_t v_key[CHV], v_off[CHV], v_db[CHV];
  if constexpr (!TRV) {
#pragma unroll
    for (int j = 0; j < CHV; ++j) {
      const int c = tid + NTH * j;
      v_key[j] = 2u * (uint32_t)(c % NPR);
      v_off[j] = ((v_key[j] & bs_mask) * HD + (c / NPR) * 8) * 2;
      v_db[j] = v_key[j] >> a.bs_log2;
    }
  }
  uint32_t kid[CHK], vid[CHV];
  // Row-major V: vr holds the K chunks' V; transposed: vr0 / vr1 the pairs.
  u32x4 kr[DEPTH][CHK], vr[DEPTH][TRV ? CHK : 1];
  u32x4 vr0[DEPTH][CHV], vr1[DEPTH][CHV];
  uint32_t kbits[DEPTH], vbits[DEPTH];

  // From head_dim 64 up, one wave-wide load covers 512 / head_dim <= 8
  // keys, all in one block (blocks hold >= 8): a chunk's block id is
  // wave-uniform and comes by a scalar load through the constant address
  // space. A vector load would count in the same in-order queue as the K/V
  // loads in flight, so waiting for the ids would wait for those too.
  constexpr bool SCALAR_IDS = HD >= 64;
  typedef const __attribute__((address_space(4))) uint32_t cu32;
  cu32 *ctable = (cu32 *)(uintptr_t)table;
  auto fetch_ids = [&](uint32_t kt) {
    const uint32_t b0 = kt >> a.bs_log2, last = a.max_blocks - 1u;
    if constexpr (SCALAR_IDS) {
#pragma unroll
      for (int i = 0; i < CHK; ++i) {
        // the chunk's first key (lane 0's): lanes add lane / CPR < 512 / HD
        const uint32_t key0 = (64u * wave + (uint32_t)(NTH * i)) / CPR;
        kid[i] = ctable[min(b0 + (key0 >> a.bs_log2), last)];
      }
    } else {
#pragma unroll
      for (int i = 0; i < CHK; ++i) kid[i] = table[min(b0 + k_db[i], last)];
    }
    if constexpr (!TRV) {
#pragma unroll
      for (int j = 0; j < CHV; ++j) vid[j] = table[min(b0 + v_db[j], last)];
    }
  };
  // Fused append (decode mode only: the one-wave instantiation): the item
  // holding the appended key loads the new K/V row into registers (after
  // its first tiles' loads are out), writes it into LDS over whatever the
  // cache held in the tile holding that key, and stores it to its slot at
  // the end (lanes < CPR, one 16-byte chunk each).
  static_assert(WAVES != 1 || (CPR <= NTH && (TRV || HD <= NTH)),
                "one lane per 16-byte chunk of the row (and per V element)");
  u32x4 new_kc{}, new_vc{};
  uint16_t new_ve = 0;  // transposed V: element tid of the new row (f16)
  const size_t new_src = ((size_t)b * a.n_kv + kvh) * HD;
  // B: the LDS buffer of tile kt (tile i uses buffer i % NBUF), a
  // compile-time index so LDS addresses fold into instruction offsets.
  auto load = [&](auto S, auto B, uint32_t kt) {
    constexpr int si = decltype(S)::value;
    const uint32_t t_off = (kt & bs_mask) * HD * 2;  // 0 unless bs > 64
    if constexpr (DMA) {
      // Instruction i of wave w fills chunks 64w + NTH*i .. + 63 of the
      // tile's buffer (tile j uses buffer j % 2, as in step): 1 KiB, whole
      // rows (four at head_dim 128, eight at 64), one block id. Keys not
      // read load zeros.
      typedef __attribute__((address_space(3))) void lds_t;
      unsigned char *lb = smem + decltype(B)::value * LD::buf;
      if (all_ok && kt + BN <= k_end) {  // uniform: every key read
#pragma unroll
        for (int i = 0; i < CHK; ++i) {
          const uint32_t dst = (64u * wave + (uint32_t)(NTH * i)) * 16u;
          // Buffer loads: the block's address (uniform) goes into a
          // resource descriptor built by scalar instructions, the lane adds
          // its 32-bit offset; no vector address arithmetic.
          const uint64_t tb = (uint64_t)kid[i] * blk_bytes + t_off;
          dma16(kbase + tb, k_off[i], lb + dst);
          dma16(vbase + tb, k_off[i], lb + LD::k_bytes + dst);
        }
        return;
      }
      const uint64_t zero = reinterpret_cast<uint64_t>(g_pf_zero) + lane * 16;
#pragma unroll
      for (int i = 0; i < CHK; ++i) {
        const uint32_t dst = (64u * wave + (uint32_t)(NTH * i)) * 16u;
        const bool use = kid[i] < a.num_blocks && kt + k_key[i] < k_end;
        const uint64_t off =
            (uint64_t)kid[i] * blk_bytes + (t_off + k_off[i]);
        // (one address each, selected as integers: no divergent loads)
        const uint64_t kp = use ? reinterpret_cast<uint64_t>(kbase) + off : zero;
        const uint64_t vp = use ? reinterpret_cast<uint64_t>(vbase) + off : zero;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(kp),
                                         (lds_t *)(lb + dst), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(vp),
                                         (lds_t *)(lb + LD::k_bytes + dst),
                                         16, 0, 0);
        // (the key flags are read only while all_ok is false)
        if (!all_ok && (lane & (CPR - 1)) == 0)  // (a row's first lane)
          lb[LD::k_bytes + LD::v_bytes + k_key[i]] = (uint8_t)use;
      }
      return;
    }
    if (all_ok && kt + BN <= k_end) {
      // Every key of the tile is below k_end and every block valid: no
      // flags, no id checks (the common case, uniform).
      kbits[si] = ~0u;
      vbits[si] = ~0u;
#pragma unroll
      for (int i = 0; i < CHK; ++i) {
        const uint64_t off = (uint64_t)kid[i] * blk_bytes + (t_off + k_off[i]);
        kr[si][i] = ld16<WAVES == 1>(kbase + off);
        if constexpr (TRV)
          vr[si][i] = ld16<WAVES == 1>(vbase + off);
      }
      if constexpr (!TRV) {
        if (v_lane) {
#pragma unroll
          for (int j = 0; j < CHV; ++j) {
            const char *vp =
                vbase + (uint64_t)vid[j] * blk_bytes + (t_off + v_off[j]);
            vr0[si][j] = ld16<WAVES == 1>(vp);
            vr1[si][j] = ld16<WAVES == 1>(vp + HD * 2);
          }
        }
      }
      return;
    }
    kbits[si] = 0;
    vbits[si] = 0;
    // A chunk whose key is not read (past k_end, or an unreadable block)
    // loads the lane's chunk-0 address again instead: that line is fetched
    // anyway (or is block 0's), so the masked keys of a sequence's last
    // block cost no HBM bytes. Its value is masked out at the LDS store.
    const uint64_t off0 = (uint64_t)(kid[0] < a.num_blocks ? kid[0] : 0u) *
                              blk_bytes + (t_off + k_off[0]);
#pragma unroll
    for (int i = 0; i < CHK; ++i) {
      // The address checks its own block id: all_ok covers only the blocks
      // of keys below k_end, and the last tile may reach past them.
      const bool use = kid[i] < a.num_blocks && kt + k_key[i] < k_end;
      kbits[si] |= (uint32_t)use << i;
      const uint64_t off =
          use ? (uint64_t)kid[i] * blk_bytes + (t_off + k_off[i]) : off0;
      kr[si][i] = ld16<WAVES == 1>(kbase + off);
      if constexpr (TRV)
        vr[si][i] = ld16<WAVES == 1>(vbase + off);
    }
    if constexpr (!TRV) {
#pragma unroll
      for (int j = 0; j < CHV; ++j) {
        const bool okb = vid[j] < a.num_blocks;
        const uint32_t tok = kt + v_key[j];
        vbits[si] |= (uint32_t)(okb && tok < k_end) << (2 * j);
        vbits[si] |= (uint32_t)(okb && tok + 1 < k_end) << (2 * j + 1);
        // (a pair wholly unread loads the lane's chunk-0 pair again)
        const bool use = okb && tok < k_end;
        const char *vp =
            vbase + (use ? (uint64_t)vid[j] * blk_bytes + (t_off + v_off[j])
                         : (uint64_t)(vid[0] < a.num_blocks ? vid[0] : 0u) *
                                   blk_bytes + (t_off + v_off[0]));
        if (v_lane) {
          vr0[si][j] = ld16<WAVES == 1>(vp);
          vr1[si][j] = ld16<WAVES == 1>(vp + HD * 2);
        }
      }
    }
  };

  // One tile: stage register set S into LDS, refill S with the tile DEPTH
  // ahead, compute.
  auto step = [&](auto S, auto B, uint32_t kt) {
    constexpr int si = decltype(S)::value;
    constexpr int bi = LD::NBUF == 2 ? decltype(B)::value : 0;
    // the buffer of the tile DEPTH ahead
    using BN_ = std::integral_constant<int, LD::NBUF == 2 ? 1 - bi : 0>;
    // Every key of the tile readable: all blocks valid, tile inside k_end.
    const bool tile_ok = all_ok && kt + BN <= k_end;
    // Tile i uses buffer i % NBUF; with two, every wave has passed the
    // previous tile's barrier, so none still reads tile i - 2's buffer.
    unsigned char *lb = smem + bi * LD::buf;
    uint16_t *ks = reinterpret_cast<uint16_t *>(lb);
    // V: row-major (vs, stride KS) or transposed (Vt[d][key], stride VS).
    uint16_t *vs = reinterpret_cast<uint16_t *>(lb + LD::k_bytes);
    uint8_t *kok = lb + LD::k_bytes + LD::v_bytes;
    if constexpr (LD::NBUF == 1)
      region_sync();  // the previous tile is no longer read
#pragma unroll
    for (int i = 0; i < (DMA ? 0 : CHK); ++i) {
      const int c = tid + NTH * i;
      const int key = c / CPR, dc = c % CPR;
      *reinterpret_cast<u32x4 *>(ks + key * KS + dc * 8) = kr[si][i];
      if constexpr (TRV) {
        const bool vok = tile_ok || ((kbits[si] >> i) & 1u);
        *reinterpret_cast<u32x4 *>(vs + key * VRS + dc * 8) =
            vok ? vr[si][i] : u32x4{0u, 0u, 0u, 0u};
      }
      // Every loader of a key writes the same flag.
      if (!all_ok) kok[key] = (uint8_t)((kbits[si] >> i) & 1u);
    }
    if constexpr (!TRV) {
      if (v_lane) {
#pragma unroll
        for (int j = 0; j < CHV; ++j) {
          const int c = tid + NTH * j;
          const int pr = c % NPR, dc = c / NPR;
          uint32_t *row = reinterpret_cast<uint32_t *>(vs + dc * 8 * VS) + pr;
          // Low halves of both keys go to row d = 8dc + 2e, high halves to
          // d + 1; keys past the readable range are zeroed.
          if (tile_ok) {  // uniform: every key of the tile is readable
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              row[(2 * e) * (VS / 2)] = __builtin_amdgcn_perm(
                  vr1[si][j][e], vr0[si][j][e], 0x05040100u);
              row[(2 * e + 1) * (VS / 2)] = __builtin_amdgcn_perm(
                  vr1[si][j][e], vr0[si][j][e], 0x07060302u);
            }
          } else {
            const uint32_t mask =
                ((vbits[si] >> (2 * j)) & 1u ? 0xffffu : 0u) |
                ((vbits[si] >> (2 * j + 1)) & 1u ? 0xffff0000u : 0u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              row[(2 * e) * (VS / 2)] =
                  __builtin_amdgcn_perm(vr1[si][j][e], vr0[si][j][e],
                                        0x05040100u) & mask;
              row[(2 * e + 1) * (VS / 2)] =
                  __builtin_amdgcn_perm(vr1[si][j][e], vr0[si][j][e],
                                        0x07060302u) & mask;
            }
          }
        }
      }
    }
    if constexpr (WAVES == 1) {
      if (newtok - kt < (uint32_t)BN) {  // this tile holds the new key
        const uint32_t r = newtok - kt;
        if (tid < CPR) {
          *reinterpret_cast<u32x4 *>(ks + r * KS + tid * 8) = new_kc;
          if constexpr (TRV)
            *reinterpret_cast<u32x4 *>(vs + r * VRS + tid * 8) = new_vc;
        }
        if constexpr (!TRV) {
          if (tid < HD) vs[tid * VS + r] = new_ve;
        }
        if (!all_ok && tid == 0) kok[r] = 1;
      }
    }
    // (DMA: this wave's copies into the tile must have landed before the
    // barrier publishes it: s_waitcnt with vmcnt 0, expcnt and lgkmcnt at
    // their maxima, 0x0f70 in this architecture's encoding)
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0x0f70);
    region_sync();
    if (kt + DEPTH * BN < k_end) {
      load(S, BN_{}, kt + DEPTH * BN);
      fetch_ids(kt + (DEPTH + 1) * BN);
    }
    // Does any row of the wave see a key of the tile? (Wave-uniform, and
    // the same for both waves of a pair.)
    const bool active = kt < w_end && kt + BN > w_begin;
    if (!SPLIT && !active) return;

    f32x16 s[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) s[t][j] = 0.f;
    // The two sub-tiles' accumulation chains alternate, so each MFMA's
    // dependency on the previous one of its chain is hidden.
    if (active) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        half8 kf[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if constexpr (DMA)
            kf[t] = *reinterpret_cast<const half8 *>(
                ks + (32 * t + sig) * KS +
                (((uint32_t)(2 * kc + hl) ^ swz<HD>((uint32_t)sig)) * 8));
          else
            kf[t] = *reinterpret_cast<const half8 *>(
                ks + (32 * t + sig) * KS + dh * (KC * 16) + kc * 16 + hl * 8);
          s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t], qf[kc], s[t], 0,
                                                        0, 0);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t)
          s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[t], ql[kc], s[t], 0,
                                                        0, 0);
      }
    }
    if constexpr (SPLIT) {
      // Add the partner's half of S^T. Each wave writes its own slot after
      // this tile's first barrier; the partner read it before reaching the
      // next tile's. Both waves add the same two values, so their S, and
      // with it their softmax state, are identical.
      float4 *xs = reinterpret_cast<float4 *>(smem + LD::NBUF * LD::buf);
      if (active) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            xs[(wave * NT * 4 + t * 4 + q4) * 64 + lane] =
                make_float4(s[t][4 * q4], s[t][4 * q4 + 1], s[t][4 * q4 + 2],
                            s[t][4 * q4 + 3]);
      }
      __syncthreads();
      if (!active) return;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float4 x = xs[((wave ^ 1u) * NT * 4 + t * 4 + q4) * 64 + lane];
          s[t][4 * q4] += x.x;
          s[t][4 * q4 + 1] += x.y;
          s[t][4 * q4 + 2] += x.z;
          s[t][4 * q4 + 3] += x.w;
        }
    }

    // Mask (only where some row of the wave does not see the whole tile),
    // then the online softmax; register j of sub-tile t is key
    // kt + 32t + 16(j/8) + 8hl + j%8.
    float mx = kNegBig;
    if (tile_ok && kt >= w_lo_max && kt + BN <= w_hi_min) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 16; j += 2) mx = vmax3(mx, s[t][j], s[t][j + 1]);
    } else {
      // Register j of sub-tile t holds key kt + 8hl + c, c = 32t + 16(j/8)
      // + j%8 (a constant): valid for lo <= c < hi and a readable block.
      // Each run of 8 registers gets a bit mask of its valid keys first
      // (range bits, and with unreadable blocks the key flags' bits), then
      // one select per register: no branches per key.
      const int32_t lo = (int32_t)(row_lo - kt) - 8 * hl;
      const int32_t hi = (int32_t)(row_hi - kt) - 8 * hl;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int g8 = 0; g8 < 2; ++g8) {
          const int32_t c0 = 32 * t + 16 * g8;
          const uint32_t a0 = (uint32_t)min(max(lo - c0, 0), 8);
          const uint32_t a1 = (uint32_t)min(max(hi - c0, 0), 8);
          // keys e in [a0, a1)
          uint32_t vm = a1 > a0 ? ((1u << (a1 - a0)) - 1u) << a0 : 0u;
          if (!all_ok) {  // (uniform) flags: one byte (0 or 1) per key
            const uint32_t k0 = 32 * t + 16 * g8 + 8 * hl;
            const uint2 fw = *reinterpret_cast<const uint2 *>(kok + k0);
            // Bytes b0..b3 of a word (each 0 or 1) to bits 0..3: the product
            // puts byte i's bit at 24 + i, with no carries into those bits.
            const uint32_t f4l = ((fw.x & 0x01010101u) * 0x01020408u) >> 24;
            const uint32_t f4h = ((fw.y & 0x01010101u) * 0x01020408u) >> 24;
            vm &= f4l | (f4h << 4);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool valid = (vm >> e) & 1u;
            const float x = valid ? s[t][8 * g8 + e] : -__builtin_inff();
            s[t][8 * g8 + e] = x;
            mx = fmaxf(mx, x);
          }
        }
    }
    mx = max_halves(mx);
    // Lazy rescale: the reference max m moves only when the tile's max
    // exceeds it by more than 2^8, so probabilities stay <= 256 (exact
    // in f16's range) and O and l are rescaled on few tiles; the final
    // division by l cancels whichever m was used.
    const bool grow = mx > m + 8.0f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? mx : m;
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[dt][j] *= alpha;
    }
    half8 pb[NT][2];
    float psum = 0.f;
    const h2 ones = h2{(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pb[t][c][e] = (_Float16)__builtin_amdgcn_exp2f(s[t][8 * c + e] - m);
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          psum = __builtin_amdgcn_fdot2(h2{pb[t][c][e], pb[t][c][e + 1]},
                                        ones, psum, false);
      }
    l += psum;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          // V^T fragment: dims dt*32 + ln, keys 32t + 16c + 8hl .. +8.
          half8 vf;
          if constexpr (TRV) {
            // Two transposing reads of 4 keys each; the lane's address is
            // the (key, dim) its 16-lane group hands out.
            v4h lo, hi;
            if constexpr (DMA) {
              // rows tr_key and tr_key + 4 (< 16) of the sub-tile, each at
              // its own swizzled slot (chunks 4dt .. 4dt + 3)
              const uint32_t ch = (uint32_t)(4 * dt) + ((uint32_t)tr_dim >> 3);
              const uint16_t *vr = vs + (32 * t + 16 * c + tr_key) * VRS +
                                   (tr_dim & 7);
              lo = tr_read(vr + ((ch ^ swz<HD>((uint32_t)tr_key)) * 8));
              hi = tr_read(vr + 4 * VRS +
                           ((ch ^ swz<HD>((uint32_t)tr_key + 4u)) * 8));
            } else {
              const uint16_t *vp = vs + (32 * t + 16 * c + tr_key) * VRS +
                                   (dh * DT + dt) * 32 + tr_dim;
              lo = tr_read(vp);
              hi = tr_read(vp + 4 * VRS);
            }
            vf = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          } else {
            vf = *reinterpret_cast<const half8 *>(
                vs + ((dh * DT + dt) * 32 + ln) * VS + 32 * t + 16 * c + 8 * hl);
          }
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pb[t][c], o[dt],
                                                         0, 0, 0);
        }
  };

  if (k_begin < k_end) {
    fetch_ids(k_begin);
    load(I0{}, I0{}, k_begin);
    fetch_ids(k_begin + BN);
    if constexpr (DEPTH == 2) {
      if (k_begin + BN < k_end) load(I1{}, I0{}, k_begin + BN);  // (NBUF 1)
      fetch_ids(k_begin + 2 * BN);
    }
    // The table scan, with the first tiles' loads in flight.
    int bad = 0;
    for (uint32_t i = (k_begin >> a.bs_log2) + tid;
         i <= ((k_end - 1u) >> a.bs_log2); i += NTH)
      bad |= table[i] >= a.num_blocks;
    all_ok = !region_or(bad);
  }
  if constexpr (WAVES == 1) {
    if (newtok != 0xFFFFFFFFu) {
      if (tid < CPR) {
        new_kc = new_row_chunk(a.new_k, a.new_f32, new_src + tid * 8);
        new_vc = new_row_chunk(a.new_v, a.new_f32, new_src + tid * 8);
      }
      if constexpr (!TRV) {
        if (tid < HD) {
          const _Float16 v =
              a.new_f32
                  ? (_Float16) static_cast<const float *>(a.new_v)[new_src + tid]
                  : __builtin_bit_cast(_Float16, static_cast<const uint16_t *>(
                                                     a.new_v)[new_src + tid]);
          new_ve = __builtin_bit_cast(uint16_t, v);
        }
      }
    }
  }
  // Two tiles per iteration: register sets (DEPTH 2) or LDS buffers
  // (NBUF 2) alternate with compile-time indices.
  using Bx1 = std::integral_constant<int, 1>;
  for (uint32_t kt = k_begin; kt < k_end;) {
    step(I0{}, I0{}, kt);
    kt += BN;
    if (kt >= k_end) break;
    if constexpr (DEPTH == 1)
      step(I0{}, Bx1{}, kt);
    else
      step(I1{}, I0{}, kt);
    kt += BN;
  }

  if constexpr (WAVES == 1) {
    if (newtok != 0xFFFFFFFFu && tid < CPR) {
      const uint32_t nb = a.new_blk[b], no = a.new_off[b];
      if (nb < a.num_blocks && no < (1u << a.bs_log2)) {
        const size_t dst =
            ((size_t)nb * a.n_kv + kvh) * a.head_stride + (size_t)no * HD;
        *reinterpret_cast<u32x4 *>(const_cast<uint16_t *>(a.kc) + dst +
                                   tid * 8) = new_kc;
        *reinterpret_cast<u32x4 *>(const_cast<uint16_t *>(a.vc) + dst +
                                   tid * 8) = new_vc;
      }
    }
  }
  if constexpr (KSPLIT > 1) {
    // Merge the waves' states into wave 0: lane-wise (every wave holds the
    // same rows in the same layout), weights 2^(m_w - M).
    constexpr int NV = 2 + DT * 16;  // floats a lane stores
    static_assert((KSPLIT - 1) * NV * 64 * 4 <= KSPLIT * LD::bytes,
                  "merge area within the workgroup's LDS");
    float *xs = reinterpret_cast<float *>(smem_all);
    __syncthreads();  // every wave is done with its tiles
    if (kwave > 0) {
      float *dst = xs + (size_t)(kwave - 1) * NV * 64 + lane;
      dst[0] = m;
      dst[64] = l;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) dst[(2 + dt * 16 + j) * 64] = o[dt][j];
    }
    __syncthreads();
    if (kwave > 0) return;
#pragma unroll
    for (int w = 1; w < KSPLIT; ++w) {
      const float *src = xs + (size_t)(w - 1) * NV * 64 + lane;
      const float mw = src[0], lw = src[64];
      const float M = fmaxf(m, mw);
      const float aw = __builtin_amdgcn_exp2f(m - M);
      const float bw = __builtin_amdgcn_exp2f(mw - M);
      l = l * aw + lw * bw;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          o[dt][j] = o[dt][j] * aw + src[(2 + dt * 16 + j) * 64] * bw;
      m = M;
    }
  }
  const float lt = sum_halves(l);
  if (gl || slot != kNoSlot) {  // split decode sequences: partials
    if (row_ok) {
      const size_t idx = (size_t)my_slot * a.n_heads + head;
      float *op = a.ws_acc + idx * HD;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<float4 *>(op + (dh * DT + dt) * 32 + 8 * q4 +
                                      4 * hl) =
              make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2],
                          o[dt][4 * q4 + 3]);
      if (hl == 0 && dh == 0) {
        a.ws_ml[idx * 2] = m;
        a.ws_ml[idx * 2 + 1] = lt;
      }
    }
    return;
  }
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (row_ok) {
    float *op = a.out + qrow * HD;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4 *>(op + (dh * DT + dt) * 32 + 8 * q4 +
                                    4 * hl) =
            make_float4(o[dt][4 * q4] * inv, o[dt][4 * q4 + 1] * inv,
                        o[dt][4 * q4 + 2] * inv, o[dt][4 * q4 + 3] * inv);
  }
}

template <int HD, int WAVES>
void launch_prefill(const PrefillArgs &a, dim3 grid, hipStream_t st) {
  // Past 64 KiB (head_dim 128 and 256 double-buffered) the dynamic LDS size
  // is declared to the runtime, once per instantiation and device.
  if constexpr (Lds<HD, WAVES>::bytes > 65536) {
    static std::atomic<uint64_t> done{0};
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev < 64 &&
        !(done.load(std::memory_order_relaxed) >> dev & 1u)) {
      // (a refusal shows as the launch's own error)
      if (hipFuncSetAttribute(
              reinterpret_cast<const void *>(&prefill_kernel<HD, WAVES>),
              hipFuncAttributeMaxDynamicSharedMemorySize,
              (int)Lds<HD, WAVES>::bytes) == hipSuccess)
        done.fetch_or(1ull << dev, std::memory_order_relaxed);
    }
  }
  hipLaunchKernelGGL((prefill_kernel<HD, WAVES>), grid, dim3(64 * WAVES),
                     (Lds<HD, WAVES>::bytes), st, a);
}

// Waves per workgroup: 4 at head_dim 128 with the tiles staged by LDS DMA,
// two workgroups per CU (1.5-2 % faster than one 8-wave workgroup with
// register staging, which is what fits without DMA); 8 at 256 (four
// pairs); 4 at 64, where 8-wave workgroups would cost the third resident
// wave per SIMD (measured ~7 % slower), and at 32. RVKV_PREFILL_WAVES=4|8
// overrides at 64 and 128.
uint32_t prefill_waves(uint32_t hd) {
  static const char *env = getenv("RVKV_PREFILL_WAVES");
  static const uint32_t forced = env ? (uint32_t)atoi(env) : 0u;
  if (hd == 128) return forced == 8 ? 8u : 4u;
  if (split_dims((int)hd)) return 8u;  // (four pairs)
  if (hd == 64 && (forced == 4 || forced == 8)) return forced;
  return 4u;
}

}  // namespace

extern "C" {

int rvkv_paged_prefill(rvkv_pool *pool, uint32_t layer, const float *q,
                       const uint32_t *block_tables,
                       const uint32_t *pos_offset,
                       const uint32_t *read_num_tokens, uint32_t batch,
                       uint32_t q_len, uint32_t max_blocks, uint32_t n_heads,
                       float scale, int32_t window, float *out) {
  const char *op = "paged_prefill";
  if (!pool) return fail(RVKV_EINVAL, op, "pool is NULL");
  if (layer >= pool->n_layers)
    return fail(RVKV_EINVAL, op, "layer out of range");
  if (batch == 0 || q_len == 0) return RVKV_OK;
  if (!q || !block_tables || !pos_offset || !read_num_tokens || !out)
    return fail(RVKV_EINVAL, op,
                "NULL q/block_tables/pos_offset/read_num_tokens/out");
  if (max_blocks == 0) return fail(RVKV_EINVAL, op, "max_blocks is 0");
  if (n_heads == 0 || n_heads % pool->n_kv != 0)
    return fail(RVKV_EINVAL, op,
                "n_heads must be a positive multiple of n_kv_heads");
  const uint32_t hd = pool->head_dim, bs = pool->block_size;
  if ((uintptr_t)q % 16 || (uintptr_t)out % 16)
    return fail(RVKV_EINVAL, op, "q and out must be 16-byte aligned");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(RVKV_EINVAL, op, "scale must be positive and finite");
  // The matrix-core kernel takes f16 cells, head_dim 32/64/128/256 and
  // power-of-two blocks of >= 8 tokens; every other shape (and an f32
  // cache) runs the generic kernel.
  if (pool->f32() || (hd != 32 && hd != 64 && hd != 128 && hd != 256) ||
      bs < 8 || (bs & (bs - 1)) != 0 ||
      (uint64_t)max_blocks * bs > 0x80000000ull ||
      pool->block_elems * 2 >= 0x100000000ull)
    return rvkv_detail::generic_attention(
        op, pool, layer, q, block_tables, max_blocks, pos_offset,
        read_num_tokens, batch, q_len, n_heads, 0xFFFFFFFFu, scale, window,
        out);
  const uint64_t rows = (uint64_t)(n_heads / pool->n_kv) * q_len;
  if (rows > 0x7fffffffull)
    return fail(RVKV_EUNSUPPORTED, op, "q_len too large for one launch");

  PrefillArgs a{};
  a.q = q;
  a.out = out;
  a.kc = pool->tensor(layer, 0);
  a.vc = pool->tensor(layer, 1);
  a.tables = block_tables;
  a.pos_offset = pos_offset;
  a.read_num = read_num_tokens;
  a.block_stride = pool->block_elems;
  a.head_stride = bs * hd;
  a.q_len = q_len;
  a.max_blocks = max_blocks;
  a.num_blocks = pool->num_blocks;
  a.n_heads = n_heads;
  a.group = n_heads / pool->n_kv;
  uint32_t lg = 0;
  while ((1u << lg) < bs) ++lg;
  a.bs_log2 = lg;
  a.rows = (uint32_t)rows;
  const uint32_t waves = prefill_waves(hd);
  const uint32_t bm = kWaveRows * (split_dims((int)hd) ? waves / 2 : waves);
  a.n_tiles = (uint32_t)((rows + bm - 1) / bm);
  a.qscale = scale * 1.4426950408889634f;
  a.window = window;
  a.batch = batch;
  a.n_kv = pool->n_kv;
  const uint64_t n_wg = (uint64_t)a.n_tiles * pool->n_kv * batch;
  if (n_wg > 0x7fffffffull)
    return fail(RVKV_EUNSUPPORTED, op, "too many query tiles for one launch");
  const dim3 grid((uint32_t)n_wg);
  switch (hd) {
    case 32: launch_prefill<32, 4>(a, grid, pool->stream); break;
    case 64:
      if (waves == 8) launch_prefill<64, 8>(a, grid, pool->stream);
      else launch_prefill<64, 4>(a, grid, pool->stream);
      break;
    case 128:
      if (waves == 4) launch_prefill<128, 4>(a, grid, pool->stream);
      else launch_prefill<128, 8>(a, grid, pool->stream);
      break;
    default: launch_prefill<256, 8>(a, grid, pool->stream); break;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

}  // extern "C"

namespace rvkv_detail {

bool mfma_decode_wanted(const rvkv_pool *pool, uint32_t n_heads) {
  static const char *env = getenv("RVKV_DECODE_MFMA");
  const uint32_t group = pool->n_kv ? n_heads / pool->n_kv : 0;
  const bool shape_ok = !pool->f32() && pool->head_dim == 64 && group >= 1 &&
                        group <= 32 &&
                        pool->block_elems * 2 < 0x100000000ull &&
                        pool->block_size >= 8 &&
                        (pool->block_size & (pool->block_size - 1)) == 0 &&
                        pool->block_size <= 256;
  if (env && env[0] == '0') return false;
  if (env && env[0] == '1') return shape_ok;
  // From four query heads per KV head the matrix cores beat the VALU
  // decode: Llama-3.2-1B's shape (G = 4) at 64 x 2048 49.9 vs 52.7 us a
  // layer, at 256 x 4096 326 vs 343 us (with items of about half a
  // sequence); below four the VALU decode's work per key is small enough.
  return shape_ok && group >= 4;
}

int mfma_decode(const rvkv_pool *pool, uint32_t layer, const float *q,
                const uint32_t *tables, const uint32_t *ctx_lens,
                uint32_t max_blocks, uint32_t n_heads, float scale,
                int32_t window, const uint4 *items, uint32_t n_items,
                float *ws_acc, float *ws_ml, float *out, const void *new_k,
                const void *new_v, const uint32_t *new_blk,
                const uint32_t *new_off, bool new_f32,
                const uint32_t *groups, uint32_t dec_parts,
                uint32_t dec_part_tokens, uint32_t dec_ctx_cap,
                uint32_t ksplit) {
  const char *op = "paged_decode";
  if (n_items == 0) return RVKV_OK;
  PrefillArgs a{};
  a.q = q;
  a.out = out;
  a.kc = pool->tensor(layer, 0);
  a.vc = pool->tensor(layer, 1);
  a.tables = tables;
  a.pos_offset = ctx_lens;  // unused in decode mode
  a.read_num = ctx_lens;
  a.block_stride = pool->block_elems;
  a.head_stride = pool->block_size * pool->head_dim;
  a.q_len = 1;
  a.max_blocks = max_blocks;
  a.num_blocks = pool->num_blocks;
  a.n_heads = n_heads;
  a.group = n_heads / pool->n_kv;
  uint32_t lg = 0;
  while ((1u << lg) < pool->block_size) ++lg;
  a.bs_log2 = lg;
  a.rows = a.group;
  a.n_tiles = 1;
  a.qscale = scale * 1.4426950408889634f;
  a.window = window;
  a.batch = 0;
  a.n_kv = pool->n_kv;
  a.items = items;
  a.groups = groups;
  a.dec_parts = items ? 0u : dec_parts;
  a.dec_part_tokens = dec_part_tokens;
  a.dec_ctx_cap = dec_ctx_cap;
  a.ws_acc = ws_acc;
  a.ws_ml = ws_ml;
  a.new_k = new_k;
  a.new_v = new_v;
  a.new_blk = new_blk;
  a.new_off = new_off;
  a.new_f32 = new_f32;
  if (ksplit == 4)
    hipLaunchKernelGGL((prefill_kernel<64, 1, 4>), dim3(n_items, pool->n_kv),
                       dim3(256), (4 * Lds<64, 1>::bytes), pool->stream, a);
  else if (ksplit == 2)
    hipLaunchKernelGGL((prefill_kernel<64, 1, 2>), dim3(n_items, pool->n_kv),
                       dim3(128), (2 * Lds<64, 1>::bytes), pool->stream, a);
  else
    hipLaunchKernelGGL((prefill_kernel<64, 1>), dim3(n_items, pool->n_kv),
                       dim3(64), (Lds<64, 1>::bytes), pool->stream, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

}  // namespace rvkv_detail
