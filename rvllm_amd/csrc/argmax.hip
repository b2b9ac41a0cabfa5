// argmax.hip - per-row greedy token pick over a logits matrix, the step
// after the paged-attention path (rvllm: src/cuda/kernels/argmax.cu via
// argmax_wrapper, src/cuda/ops.rs:516-550, queued behind the forward at
// src/cuda/engine.rs:118-125).
//
// Semantics are those of the greedy scan in Sampler::sample_slice
// (src/sampler.rs:64-75): the first maximum wins (lowest index on ties),
// NaN is never a maximum, and a row with nothing above -inf gives 0.
//
// One 256-thread workgroup per row. The row streams through 16-byte loads
// when it is 16-byte aligned and a multiple of 4 long (scalar otherwise);
// each lane keeps its best (value, index), with strictly-greater updates so
// its own first maximum wins; the wave reduces by xor shuffles and the four
// waves through LDS, preferring the larger value and, on equal values, the
// smaller index. HBM-bound: rows * row_len * 4 bytes read once.
#include "pool.h"

using rvkv_detail::fail;
using rvkv_detail::hip_fail;

namespace {

__device__ __forceinline__ void take(float &bv, uint32_t &bi, float v,
                                     uint32_t i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

template <bool VEC>
__global__ void __launch_bounds__(256)
    argmax_kernel(const float *__restrict__ x, uint32_t row_len,
                  uint32_t *__restrict__ out) {
  const float *row = x + (size_t)blockIdx.x * row_len;
  float bv = -__builtin_inff();
  uint32_t bi = 0xffffffffu;
  if constexpr (VEC) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    const uint32_t n4 = row_len / 4;
    for (uint32_t c = threadIdx.x; c < n4; c += 256) {
      const float4 v = r4[c];
      const uint32_t i = 4 * c;
      if (v.x > bv) { bv = v.x; bi = i; }
      if (v.y > bv) { bv = v.y; bi = i + 1; }
      if (v.z > bv) { bv = v.z; bi = i + 2; }
      if (v.w > bv) { bv = v.w; bi = i + 3; }
    }
  } else {
    for (uint32_t i = threadIdx.x; i < row_len; i += 256) {
      const float v = row[i];
      if (v > bv) { bv = v; bi = i; }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    take(bv, bi, ov, oi);
  }
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) take(bv, bi, sv[w], si[w]);
    out[blockIdx.x] = bi == 0xffffffffu ? 0u : bi;
  }
}

}  // namespace

extern "C" {

int rvkv_argmax(const float *logits, uint32_t rows, uint32_t row_len,
                uint32_t *out, rvkv_stream stream) {
  const char *op = "argmax";
  if (rows == 0) return RVKV_OK;
  if (!logits || !out) return fail(RVKV_EINVAL, op, "NULL logits or out");
  if (row_len == 0) return fail(RVKV_EINVAL, op, "row_len must be positive");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool vec = row_len % 4 == 0 && (uintptr_t)logits % 16 == 0;
  if (vec)
    hipLaunchKernelGGL(argmax_kernel<true>, dim3(rows), dim3(256), 0, st,
                       logits, row_len, out);
  else
    hipLaunchKernelGGL(argmax_kernel<false>, dim3(rows), dim3(256), 0, st,
                       logits, row_len, out);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? RVKV_OK : hip_fail(op, e);
}

}  // extern "C"
