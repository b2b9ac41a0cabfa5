// pool.h - internals shared by the librvkv sources: the pool object and the
// thread-local last-error helpers behind rvkv_last_error().
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/rvkv.h"

// Physical cache layout, per layer and per K/V tensor, f16:
//   [num_blocks][n_kv_heads][block_size][head_dim]
// Cells are f16 (elem_bytes 2) or f32 (elem_bytes 4, rvllm's own cache
// dtype). The byte-moving kernels (append of same-typed rows, gather, copy,
// inspection) see an f32 cell as two 16-bit words: the *16 sizes below count
// 16-bit words, the *_elems ones cells.
struct rvkv_pool {
  uint32_t n_layers, num_blocks, block_size, n_kv, head_dim;
  uint32_t elem_bytes;   // 2 or 4
  uint32_t hd16;         // head_dim * elem_bytes / 2
  hipStream_t stream;
  int device;
  uint16_t *base;        // 2 * n_layers tensors
  size_t tensor_elems;   // num_blocks * n_kv * block_size * head_dim
  size_t block_elems;    // n_kv * block_size * head_dim
  size_t tensor16, block16;

  uint16_t *tensor(uint32_t layer, uint32_t which) const {
    return base + ((size_t)layer * 2 + which) * tensor16;
  }
  bool f32() const { return elem_bytes == 4; }
};

namespace rvkv_detail {
// Records "<op>: <reason>" as the last error and returns code.
int fail(int code, const char *op, const char *reason);
// Records "<op>: <HIP error string>" and returns RVKV_EHIP.
int hip_fail(const char *op, hipError_t e);
// Matrix-core decode over a decode plan's work items (prefill.hip): used
// for large GQA groups, where the VALU decode is instruction-bound. groups:
// the plan's shared-prefix member lists (items flagged 0x80000000 in their
// seq field index them). items NULL: decode without a plan, n_items =
// batch * dec_parts uniform partitions of dec_part_tokens keys, read counts
// capped at dec_ctx_cap (partials to ws_acc / ws_ml slot sequence *
// dec_parts + partition, merged by the uniform reduction pass). ksplit 2:
// each item's keys split over the two waves of its workgroup, merged in
// the workgroup.
bool mfma_decode_wanted(const rvkv_pool *pool, uint32_t n_heads);
int mfma_decode(const rvkv_pool *pool, uint32_t layer, const float *q,
                const uint32_t *tables, const uint32_t *ctx_lens,
                uint32_t max_blocks, uint32_t n_heads, float scale,
                int32_t window, const uint4 *items, uint32_t n_items,
                float *ws_acc, float *ws_ml, float *out,
                const void *new_k = nullptr, const void *new_v = nullptr,
                const uint32_t *new_blk = nullptr,
                const uint32_t *new_off = nullptr, bool new_f32 = false,
                const uint32_t *groups = nullptr, uint32_t dec_parts = 0,
                uint32_t dec_part_tokens = 0,
                uint32_t dec_ctx_cap = 0xFFFFFFFFu, uint32_t ksplit = 1);
// Paged attention for shapes the tuned kernels do not take (generic.hip):
// any head_dim <= 1024, any block size, f16 or f32 cells, f32 arithmetic.
// pos_offset NULL: decode (one row per sequence at read_num - 1). Keys
// per sequence are capped at min(ctx_cap, max_blocks * block_size).
bool generic_head_dim_ok(uint32_t hd);
int generic_attention(const char *op, const rvkv_pool *pool, uint32_t layer,
                      const float *q, const uint32_t *tables,
                      uint32_t max_blocks, const uint32_t *pos_offset,
                      const uint32_t *read_num, uint32_t batch,
                      uint32_t q_len, uint32_t n_heads, uint32_t ctx_cap,
                      float scale, int32_t window, float *out);
}  // namespace rvkv_detail
