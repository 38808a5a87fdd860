// Shared device helpers for the DSpark attention hot path on gfx950 (CDNA4).
//
// Shapes are fixed to the Qwen3-0.6B attention geometry used by the DSpark
// target and draft: 16 query heads, 8 KV heads, head dim 128 (GQA group 2).
// Every K/V tensor is addressed as rows of [8 KV heads][128] bf16, i.e. one
// 2 KiB "token row" per position, which is the layout of the persistent
// resident store [layers, slots, capacity, 8, 128], its scratch
// [layers, max_q, 8, 128] and of packed THD tensors [tokens, 8, 128].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dspark {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int HQ = 16;              // query heads
constexpr int HKV = 8;              // KV heads
constexpr int HD = 128;             // head dim
constexpr int KV_ROW = HKV * HD;    // elements per K or V token row
constexpr int Q_ROW = HQ * HD;      // elements per Q/O token row
constexpr int WAVE = 64;

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
  #pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
  return z;
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

// Eight FP32 values rounded to bf16 (round to nearest even, as torch's
// Tensor.to(torch.bfloat16)).
__device__ __forceinline__ bf16x8 to_bf16x8(const f32x4& lo, const f32x4& hi) {
  bf16x8 r;
  #pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = (bf16)lo[i];
    r[4 + i] = (bf16)hi[i];
  }
  return r;
}

__device__ __forceinline__ bf16x8 ld8(const float* p) {
  return to_bf16x8(*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4));
}

__device__ __forceinline__ float wave_max_across_groups(float x) {
  // The 4 lanes {n, n+16, n+32, n+48} hold the same MFMA column (query row).
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float wave_sum_across_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Number of key chunks a request of `len` keys is split into (at least one,
// so that requests with no keys still own a work item).
__device__ __forceinline__ int chunks_for(int len, int chunk) {
  return len <= 0 ? 1 : (len + chunk - 1) / chunk;
}

// Locate the request that owns linear chunk index `cl`.  Per-request key
// counts come from a cumulative array `cu` (len = cu[r+1]-cu[r]) or a plain
// length array `lens`.  Executed redundantly by every wave of a workgroup;
// all lanes return the same (request, first-chunk) pair, or request -1 when
// `cl` lies beyond the last request's chunks.
__device__ __forceinline__ void locate_chunk(const int32_t* __restrict__ cu,
                                             const int32_t* __restrict__ lens,
                                             int n_req, int chunk, int cl,
                                             int& req, int& first) {
  const int lane = threadIdx.x & (WAVE - 1);
  int running = 0;
  for (int r0 = 0; r0 < n_req; r0 += WAVE) {
    const int r = r0 + lane;
    int n = 0;
    if (r < n_req) n = chunks_for(cu ? (cu[r + 1] - cu[r]) : lens[r], chunk);
    int incl = n;
    #pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    const int total = __shfl(incl, WAVE - 1);
    if (cl < running + total) {
      const unsigned long long hit = __ballot(r < n_req && running + incl > cl);
      const int L = __ffsll((long long)hit) - 1;
      const int excl = incl - n;
      req = r0 + L;
      first = running + __shfl(excl, L);
      return;
    }
    running += total;
  }
  req = -1;
  first = running;
}

// Direct global->LDS load of 16 bytes per lane: lane L's data lands at LDS
// byte address `lds` + 16*L (`lds` must be wave-uniform).  Issued as inline
// assembly so that the compiler neither waits on it nor reorders LDS reads
// around it; kernels order it with explicit vmcnt waits and barriers, and
// must then issue no compiler-visible global loads while such loads are in
// flight (the compiler's own vmcnt waits would drain them).  The LDS address
// is an M0 input operand ("{m0}"): the compiler writes M0 itself and knows
// its value, so no M0 use of its own can be corrupted by this statement.
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gptr), "{m0}"(lds) : "memory");
}

// The same load with the non-temporal hint, for data read once per launch
// (streamed context rows): it reads HBM at a markedly higher rate than the
// default cache policy.
__device__ __forceinline__ void lds_dma16_nt(const void* gptr, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(gptr), "{m0}"(lds) : "memory");
}

// Direct global->LDS load of 4 bytes per lane: lane L's word lands at LDS
// byte address `lds` + 4*L; ordered like lds_dma16.
__device__ __forceinline__ void lds_dma4(const void* gptr, uint32_t lds) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(gptr), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace dspark

// ---------------------------------------------------------------------------
// Host-side error reporting shared by the C-ABI entry points.
// ---------------------------------------------------------------------------
namespace dspark {
enum Status : int { OK = 0, INVALID_ARGUMENT = -1, HIP_FAILURE = -2 };
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
// Returns OK if the last launch succeeded, else records `what` and the HIP error.
int launch_status(const char* what);
}  // namespace dspark

#define DSPARK_REQUIRE(cond, ...)                 \
  do {                                            \
    if (!(cond)) {                                \
      ::dspark::set_error(__VA_ARGS__);           \
      return ::dspark::INVALID_ARGUMENT;          \
    }                                             \
  } while (0)
