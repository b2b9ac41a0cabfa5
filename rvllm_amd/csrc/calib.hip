// calib.hip - the streaming-read calibration the roofline figures are read
// against: how fast this device reads a buffer of a given size once, with
// nothing else in the launch (no tables, no arithmetic worth the name).
// It has no counterpart in rvllm; it exists so a paged-KV launch of B bytes
// can be compared with the best plain read of B bytes on the same device
// (and a byte mover with the best plain copy of its read and write bytes,
// and a paged decode with a plain read of the same tiles in table order).
// Built into its own librvkv_calib.so for the benchmark: it is not part of
// the product ABI (include/rvkv.h).
//
// Each workgroup streams one contiguous slice with 16-byte non-temporal
// loads, four in flight per lane, and folds them into a sum that is stored
// only if it equals an impossible sentinel (so the loads are not optimised
// away and nothing is written). The non-temporal hint is worth ~10 % over
// plain loads; the best workgroup count depends on the size (over 4.3 GB:
// 7.0 TB/s at 2048, 6.5 at 8192, 6.6 at 16384, 7.2 at 65536), so callers
// take the best of several.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace {

thread_local std::string g_calib_error;

int calib_fail(const char *reason) {
  g_calib_error = std::string("read_probe: ") + reason;
  return -1;
}

constexpr int kReadThreads = 256;
constexpr int kReadUnroll = 4;

__global__ void __launch_bounds__(kReadThreads)
    read_probe_kernel(const uint4 *__restrict__ buf, uint64_t n16,
                      uint64_t per_wg, uint32_t *__restrict__ sink) {
  const uint64_t lo = (uint64_t)blockIdx.x * per_wg;
  const uint64_t hi = lo + per_wg < n16 ? lo + per_wg : n16;
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v *b4 = reinterpret_cast<const u32x4v *>(buf);
  uint32_t acc = 0;
  for (uint64_t i = lo + threadIdx.x; i < hi;
       i += (uint64_t)kReadThreads * kReadUnroll) {
    u32x4v v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint64_t j = i + (uint64_t)u * kReadThreads;
      v[u] = j < hi ? __builtin_nontemporal_load(b4 + j) : u32x4v{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u && sink) sink[0] = acc;  // practically never
}

// The mixed read/write counterpart: each unit reads RA and writes WA
// 16-byte words (a doubled side is two contiguous halves, so every load and
// store instruction covers one contiguous run), non-temporal loads and
// stores, four units in flight per lane. RA:WA = 2:1, 1:1 and 1:2 match the
// byte movers (f32 rows appended as f16, f16 copies, f16 gathered to f32).
template <int RA, int WA>
__global__ void __launch_bounds__(kReadThreads)
    copy_probe_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                      uint64_t n_units, uint64_t per_wg) {
  const uint64_t lo = (uint64_t)blockIdx.x * per_wg;
  const uint64_t hi = lo + per_wg < n_units ? lo + per_wg : n_units;
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v *s4 = reinterpret_cast<const u32x4v *>(src);
  u32x4v *d4 = reinterpret_cast<u32x4v *>(dst);
  for (uint64_t i = lo + threadIdx.x; i < hi;
       i += (uint64_t)kReadThreads * kReadUnroll) {
    u32x4v v[kReadUnroll][RA];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint64_t j = i + (uint64_t)u * kReadThreads;
#pragma unroll
      for (int r = 0; r < RA; ++r)
        v[u][r] = j < hi ? __builtin_nontemporal_load(s4 + r * n_units + j)
                         : u32x4v{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const uint64_t j = i + (uint64_t)u * kReadThreads;
      if (j >= hi) continue;
      u32x4v w = v[u][0];
      if constexpr (RA == 2) w ^= v[u][1];
#pragma unroll
      for (int r = 0; r < WA; ++r)
        __builtin_nontemporal_store(r ? ~w : w, d4 + r * n_units + j);
    }
  }
}

// Paged read: one wave per workgroup streams its share of `tiles` (ids
// into a buffer of tile_bytes tiles) with eight wave-wide 1 KB loads in
// flight, non-temporal, nothing computed: the access pattern of a paged
// decode (every (block, head) tile of a layer read once, in table order)
// without its arithmetic.
constexpr int kPagedUnroll = 8;
__global__ void __launch_bounds__(64)
    paged_probe_kernel(const char *__restrict__ base,
                       const uint32_t *__restrict__ ids, uint32_t n_ids,
                       uint32_t tiles_per_wg, uint32_t loads_per_tile,
                       uint32_t tile_bytes, uint32_t *__restrict__ sink) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  typedef const __attribute__((address_space(4))) uint32_t cu32;
  const uint32_t t0 = blockIdx.x * tiles_per_wg;
  const uint32_t t1 = t0 + tiles_per_wg < n_ids ? t0 + tiles_per_wg : n_ids;
  cu32 *t = (cu32 *)(uintptr_t)ids;
  uint32_t acc = 0;
  const uint32_t l_end = (t1 > t0 ? t1 - t0 : 0) * loads_per_tile;
  for (uint32_t l0 = 0; l0 < l_end; l0 += kPagedUnroll) {
    u32x4v v[kPagedUnroll];
#pragma unroll
    for (int u = 0; u < kPagedUnroll; ++u) {
      const uint32_t l = l0 + u < l_end ? l0 + u : l_end - 1;
      const uint32_t id = t[t0 + l / loads_per_tile];
      const u32x4v *p = reinterpret_cast<const u32x4v *>(
                            base + (size_t)id * tile_bytes +
                            (size_t)(l % loads_per_tile) * 1024) +
                        threadIdx.x;
      v[u] = __builtin_nontemporal_load(p);
    }
#pragma unroll
    for (int u = 0; u < kPagedUnroll; ++u) acc ^= v[u][0] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u && sink) sink[0] = acc;
}

}  // namespace

extern "C" {

const char *rvkv_calib_last_error(void) { return g_calib_error.c_str(); }

// Returns 0, or -1 with the reason in rvkv_calib_last_error().
int rvkv_calib_read_probe(const void *buf, size_t bytes, uint32_t workgroups,
                          uint32_t *sink, void *stream) {
  if (bytes == 0) return 0;
  if (!buf) return calib_fail("buf is NULL");
  if ((uintptr_t)buf % 16 || bytes % 16)
    return calib_fail("buf and bytes must be 16-byte aligned");
  if (workgroups == 0) workgroups = 16384;
  const uint64_t n16 = bytes / 16;
  const uint64_t per_wg = (n16 + workgroups - 1) / workgroups;
  hipLaunchKernelGGL(read_probe_kernel, dim3(workgroups), dim3(kReadThreads),
                     0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint4 *>(buf), n16, per_wg, sink);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : calib_fail(hipGetErrorString(e));
}

// Reads n_ids tiles of tile_bytes (a multiple of 1024) at base + id *
// tile_bytes, ids from a device table, in `workgroups` one-wave workgroups
// (0: n_ids / 256). Returns 0, or -1 with the reason.
int rvkv_calib_paged_probe(const void *base, uint32_t tile_bytes,
                           const uint32_t *ids, uint32_t n_ids,
                           uint32_t workgroups, void *stream) {
  if (n_ids == 0) return 0;
  if (!base || !ids) return calib_fail("base/ids is NULL");
  if (tile_bytes == 0 || tile_bytes % 1024 || (uintptr_t)base % 16)
    return calib_fail("tiles must be whole KiB, base 16-byte aligned");
  if (workgroups == 0) workgroups = n_ids / 256 ? n_ids / 256 : 1;
  const uint32_t per = (n_ids + workgroups - 1) / workgroups;
  workgroups = (n_ids + per - 1) / per;
  hipLaunchKernelGGL(paged_probe_kernel, dim3(workgroups), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream),
                     static_cast<const char *>(base), ids, n_ids, per,
                     tile_bytes / 1024, tile_bytes, nullptr);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : calib_fail(hipGetErrorString(e));
}

// Reads read_bytes from src and writes write_bytes to dst in one launch;
// read_bytes:write_bytes must be 2:1, 1:1 or 1:2, both multiples of 16 (of
// 32 for the doubled side). Returns 0, or -1 with the reason.
int rvkv_calib_copy_probe(const void *src, void *dst, size_t read_bytes,
                          size_t write_bytes, uint32_t workgroups,
                          void *stream) {
  if (read_bytes == 0 || write_bytes == 0) return 0;
  if (!src || !dst) return calib_fail("src/dst is NULL");
  if ((uintptr_t)src % 16 || (uintptr_t)dst % 16)
    return calib_fail("src and dst must be 16-byte aligned");
  int ra, wa;
  if (read_bytes == 2 * write_bytes) {
    ra = 2; wa = 1;
  } else if (read_bytes == write_bytes) {
    ra = 1; wa = 1;
  } else if (2 * read_bytes == write_bytes) {
    ra = 1; wa = 2;
  } else {
    return calib_fail("read:write must be 2:1, 1:1 or 1:2");
  }
  if (read_bytes % (16 * ra) || write_bytes % (16 * wa))
    return calib_fail("sizes must be whole 16-byte units");
  if (workgroups == 0) workgroups = 16384;
  const uint64_t n_units = read_bytes / (16 * ra);
  const uint64_t per_wg = (n_units + workgroups - 1) / workgroups;
  const uint4 *s = static_cast<const uint4 *>(src);
  uint4 *d = static_cast<uint4 *>(dst);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (ra == 2)
    hipLaunchKernelGGL((copy_probe_kernel<2, 1>), dim3(workgroups),
                       dim3(kReadThreads), 0, st, s, d, n_units, per_wg);
  else if (wa == 2)
    hipLaunchKernelGGL((copy_probe_kernel<1, 2>), dim3(workgroups),
                       dim3(kReadThreads), 0, st, s, d, n_units, per_wg);
  else
    hipLaunchKernelGGL((copy_probe_kernel<1, 1>), dim3(workgroups),
                       dim3(kReadThreads), 0, st, s, d, n_units, per_wg);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : calib_fail(hipGetErrorString(e));
}

}  // extern "C"
