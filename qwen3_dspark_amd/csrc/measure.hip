// Measurement utilities: the HBM streaming-read ceiling of the part (the
// yardstick the attention kernels' bandwidth is compared with) and the read
// bandwidth each XCD gets from a given region (the calibration of
// XCD-balanced work plans).
//
// stream_read_kernel<NT>: workgroup w reads its own contiguous slice of a
// linear buffer (bytes / workgroups) with 16-byte loads, eight loads in
// flight per thread, default (NT = false) or non-temporal (NT = true) cache
// policy, and writes one XOR checksum per workgroup so that no load can be
// dropped.  No reference counterpart: it measures the machine, not the path.
#include "common.h"

namespace dspark {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int SR_THREADS = 256;
constexpr int SR_UNROLL = 8;

template <bool NT>
__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const u32x4_t* __restrict__ src, int64_t n16,
                                                                 uint32_t* __restrict__ out) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b = (int64_t)blockIdx.x * per;
  const int64_t e = min(n16, b + per);
  uint32_t acc = 0;
  for (int64_t i = b + threadIdx.x; i < e; i += (int64_t)SR_THREADS * SR_UNROLL) {
    u32x4_t v[SR_UNROLL];
    #pragma unroll
    for (int u = 0; u < SR_UNROLL; ++u) {
      const int64_t j = min(i + (int64_t)u * SR_THREADS, e - 1);   // in range; duplicates do not change the rate
      v[u] = NT ? __builtin_nontemporal_load(src + j) : src[j];
    }
    #pragma unroll
    for (int u = 0; u < SR_UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  #pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off);
  __shared__ uint32_t wave_acc[SR_THREADS / WAVE];
  if ((threadIdx.x & (WAVE - 1)) == 0) wave_acc[threadIdx.x / WAVE] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    #pragma unroll
    for (int w = 0; w < SR_THREADS / WAVE; ++w) x ^= wave_acc[w];
    out[blockIdx.x] = x;
  }
}

// xcd_stamp_kernel: the same per-workgroup slices, non-temporal loads, and
// three words per workgroup: its start and end (s_memrealtime, a 100 MHz
// constant clock) and the XCD it ran on (low 32 bits) with the slice's XOR
// checksum (high 32 bits), so that no load can be dropped.  Workgroups are
// dealt round-robin over the 8 XCDs, so workgroup w runs on XCD w mod 8.
__global__ __launch_bounds__(SR_THREADS) void xcd_stamp_kernel(const u32x4_t* __restrict__ src, int64_t n16,
                                                               uint64_t* __restrict__ stamps) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b = (int64_t)blockIdx.x * per;
  const int64_t e = min(n16, b + per);
  uint32_t acc = 0;
  for (int64_t i = b + threadIdx.x; i < e; i += (int64_t)SR_THREADS * SR_UNROLL) {
    u32x4_t v[SR_UNROLL];
    #pragma unroll
    for (int u = 0; u < SR_UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + min(i + (int64_t)u * SR_THREADS, e - 1));
    #pragma unroll
    for (int u = 0; u < SR_UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  #pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off);
  __shared__ uint32_t wave_acc[SR_THREADS / WAVE];
  if ((threadIdx.x & (WAVE - 1)) == 0) wave_acc[threadIdx.x / WAVE] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0, xcc;
    #pragma unroll
    for (int w = 0; w < SR_THREADS / WAVE; ++w) x ^= wave_acc[w];
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    stamps[3 * (int64_t)blockIdx.x] = t0;
    stamps[3 * (int64_t)blockIdx.x + 1] = t1;
    stamps[3 * (int64_t)blockIdx.x + 2] = (uint64_t)(xcc & 15) | ((uint64_t)x << 32);
  }
}

}  // namespace dspark

using namespace dspark;

extern "C" int dspark_stream_read(const void* src, int64_t bytes, int nontemporal, int workgroups, void* out,
                                  void* stream) {
  clear_error();
  DSPARK_REQUIRE(src && out, "null pointer argument");
  DSPARK_REQUIRE(bytes >= 16 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
  DSPARK_REQUIRE(workgroups >= 1 && workgroups <= (1 << 20), "workgroups must be in [1, 2^20]");
  DSPARK_REQUIRE(((uintptr_t)src & 15) == 0, "src must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nontemporal)
    hipLaunchKernelGGL(stream_read_kernel<true>, dim3((unsigned)workgroups), dim3(SR_THREADS), 0, s,
                       static_cast<const u32x4_t*>(src), n16, static_cast<uint32_t*>(out));
  else
    hipLaunchKernelGGL(stream_read_kernel<false>, dim3((unsigned)workgroups), dim3(SR_THREADS), 0, s,
                       static_cast<const u32x4_t*>(src), n16, static_cast<uint32_t*>(out));
  return launch_status("stream_read_kernel");
}

extern "C" int dspark_xcd_read_stamps(const void* src, int64_t bytes, int workgroups, void* stamps, void* stream) {
  clear_error();
  DSPARK_REQUIRE(src && stamps, "null pointer argument");
  DSPARK_REQUIRE(bytes >= 16 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
  DSPARK_REQUIRE(workgroups >= 8 && workgroups <= (1 << 20) && workgroups % 8 == 0,
                 "workgroups must be a multiple of 8 in [8, 2^20]");
  DSPARK_REQUIRE(((uintptr_t)src & 15) == 0 && ((uintptr_t)stamps & 7) == 0,
                 "src must be 16-byte and stamps 8-byte aligned");
  hipLaunchKernelGGL(xcd_stamp_kernel, dim3((unsigned)workgroups), dim3(SR_THREADS), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4_t*>(src), bytes / 16,
                     static_cast<uint64_t*>(stamps));
  return launch_status("xcd_stamp_kernel");
}
