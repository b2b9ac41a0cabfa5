// pool.h - internals shared by the librvkv sources: the pool object and the
// thread-local last-error helpers behind rvkv_last_error().
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/rvkv.h"

// Physical cache layout, per layer and per K/V tensor, f16:
//   [num_blocks][n_kv_heads][block_size][head_dim]
struct rvkv_pool {
  uint32_t n_layers, num_blocks, block_size, n_kv, head_dim;
  hipStream_t stream;
  int device;
  uint16_t *base;        // 2 * n_layers tensors
  size_t tensor_elems;   // num_blocks * n_kv * block_size * head_dim
  size_t block_elems;    // n_kv * block_size * head_dim

  uint16_t *tensor(uint32_t layer, uint32_t which) const {
    return base + ((size_t)layer * 2 + which) * tensor_elems;
  }
};

namespace rvkv_detail {
// Records "<op>: <reason>" as the last error and returns code.
int fail(int code, const char *op, const char *reason);
// Records "<op>: <HIP error string>" and returns RVKV_EHIP.
int hip_fail(const char *op, hipError_t e);
}  // namespace rvkv_detail
