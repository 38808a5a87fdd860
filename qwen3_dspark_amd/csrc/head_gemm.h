// One 128-output-column "head" of a linear layer for 64 tokens, on gfx950:
//   C^T[dim][token] = W[dim][:] . x[token][:]      (dim < 128, token < 64)
// shared by the projection kernels (the target's verify-layer prologue and
// the draft context K/V projection).
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16): A = 16 weight rows, B = 16
// tokens.  The workgroup has 8 waves, two per SIMD so that one wave's LDS
// reads and MFMA chain overlap the other's: wave w owns token group
// tg = w mod 4 (tokens t0 + 16 tg .. +15) and column half kh = w / 4 of
// every ring stage (split K); the two halves are summed through LDS at the
// end.  Every lane of waves 0-3 then holds
// acc[mt][e] = C^T[16*mt + 4*grp + e][token t0 + 16w + col], i.e. the 128
// dims of one token spread over its 4 lane groups, so a per-head reduction
// (RMSNorm) needs two cross-lane shuffles and the RoPE partner of dim d
// (d + 64 = tile mt + 4) sits in the same lane.
//
// The head's weight slice [128, hidden] and the workgroup's token rows
// stream through a 3-stage LDS ring fed by direct-to-LDS loads.  A stage is
// two 64-column sub-stages (128 hidden columns, one barrier): every thread
// issues exactly 3 loads per sub-stage (2 weight pieces, 1 token piece), so
// the weights are read once per workgroup and shared by the 8 waves, with 2
// stages in flight.  (Six single sub-stage stages, 5 in flight, took ≈0.5 us
// more per 448-token prologue: twice the barriers.)
#pragma once
#include "common.h"

namespace dspark {

constexpr int HG_TOKENS = 64;                    // tokens per workgroup, 16 per token group
constexpr int HG_WAVES = 8;                      // 4 token groups x 2 column halves
constexpr int HG_KB = 64;                        // hidden columns per sub-stage
constexpr int HG_SUB = 2;                        // sub-stages per ring stage (one barrier each)
constexpr int HG_STAGES = 3;                     // ring depth (2 stages in flight)
constexpr int HG_W_BYTES = HD * HG_KB * 2;       // 128 weight rows x 128 B = 16 KiB
constexpr int HG_X_BYTES = 16 * HG_KB * 2;       // 16 token rows x 128 B per token group
constexpr int HG_SUB_BYTES = HG_W_BYTES + 4 * HG_X_BYTES;     // 24 KiB
constexpr int HG_STAGE_BYTES = HG_SUB * HG_SUB_BYTES;         // 48 KiB
constexpr int HG_SMEM = HG_STAGES * HG_STAGE_BYTES;            // 144 KiB
constexpr int HG_COLS = HG_KB * HG_SUB;          // hidden columns per ring stage (hidden must be a multiple)

// 16-byte chunk swizzle of a 128-byte LDS row: the 16 rows 16*mt + col that
// one fragment read touches land on 16 distinct bank groups.
__device__ __forceinline__ int hg_swz(int row) { return (row >> 1) & 7; }

// w: first of the head's 128 weight rows (row stride `hidden`); x: token
// rows (row stride `hidden`), `tokens` of them; t0: the workgroup's first
// token.  Rows past `tokens` re-read the last token (their results are
// discarded by the caller).  With SUMSQ, ss receives this lane's share of
// sum(x^2) over its token's row (the 4 lane groups of a column together
// cover the row once).  acc and ss are complete in waves 0-3 only; the
// caller returns waves 4-7 before using them.  Ends with a workgroup
// barrier and no direct loads in flight.
template <bool SUMSQ>
__device__ __forceinline__ void head_tile_gemm(const bf16* __restrict__ w, const bf16* __restrict__ x, int tokens,
                                               int hidden, int t0, unsigned char* smem, f32x4 (&acc)[8], float& ss) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int tg = wave & 3;
  const int kh = wave >> 2;
  const int steps = hidden / HG_COLS;

  // Direct loads: lane L of a 1 KiB piece (8 rows x 128 B) fetches row
  // 8*piece + L/8, global chunk (L%8) ^ swz(row), landing at LDS chunk L%8.
  // Wave w loads weight pieces 2w, 2w+1 and token rows 8w .. 8w+7.
  const uint32_t smem_lds = lds_address(smem);
  const int prow = lane >> 3;
  auto issue = [&](int step) {
    const int st = min(step, steps - 1);   // past the end: re-read the last stage (never used)
    #pragma unroll
    for (int sub = 0; sub < HG_SUB; ++sub) {
      const uint32_t base = smem_lds + (uint32_t)((step % HG_STAGES) * HG_STAGE_BYTES + sub * HG_SUB_BYTES);
      const int k0 = (st * HG_SUB + sub) * HG_KB;
      #pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int piece = 2 * wave + i;
        const int row = 8 * piece + prow;
        const bf16* src = w + (size_t)row * hidden + k0 + 8 * ((lane & 7) ^ hg_swz(row));
        lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)(piece * 1024)));
      }
      const int row = 8 * wave + prow;      // token row of the tile; row % 16 within its group
      const int tok = min(t0 + row, tokens - 1);
      const bf16* src = x + (size_t)tok * hidden + k0 + 8 * ((lane & 7) ^ hg_swz(row & 15));
      lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)(HG_W_BYTES + wave * 1024)));
    }
  };

  #pragma unroll
  for (int mt = 0; mt < 8; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  ss = 0.f;
  #pragma unroll
  for (int p = 0; p < HG_STAGES - 1; ++p) issue(p);
  for (int s = 0; s < steps; ++s) {
    // this thread's stage-s loads landed: the 3 loads per sub-stage of each
    // of the HG_STAGES - 2 later stages may still be in flight
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * HG_SUB * (HG_STAGES - 2)) : "memory");
    asm volatile("s_barrier" ::: "memory");            // ... and everyone else's
    issue(s + HG_STAGES - 1);
    #pragma unroll
    for (int sub = 0; sub < HG_SUB; ++sub) {
      const unsigned char* wst = smem + (s % HG_STAGES) * HG_STAGE_BYTES + sub * HG_SUB_BYTES;
      const unsigned char* xst = wst + HG_W_BYTES + tg * HG_X_BYTES;
      const int c = 4 * kh + grp;
      const bf16x8 xb = *reinterpret_cast<const bf16x8*>(xst + col * 128 + ((c ^ hg_swz(col)) << 4));
      if (SUMSQ) {
        #pragma unroll
        for (int i = 0; i < 8; ++i) ss += (float)xb[i] * (float)xb[i];
      }
      #pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        const int row = 16 * mt + col;
        const bf16x8 wa = *reinterpret_cast<const bf16x8*>(wst + row * 128 + ((c ^ hg_swz(row)) << 4));
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xb, acc[mt], 0, 0, 0);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();   // every wave is done with the ring: reuse it for the sum
  float* part = reinterpret_cast<float*>(smem) + ((size_t)tg * 64 + lane) * 36;
  if (kh == 1) {
    #pragma unroll
    for (int mt = 0; mt < 8; ++mt) *reinterpret_cast<f32x4*>(part + 4 * mt) = acc[mt];
    part[32] = ss;
  }
  __syncthreads();
  if (kh == 0) {
    #pragma unroll
    for (int mt = 0; mt < 8; ++mt) acc[mt] += *reinterpret_cast<const f32x4*>(part + 4 * mt);
    ss += part[32];
  }
}

// RMSNorm over the 128 dims of each lane's token (weights nw[128]) in place.
__device__ __forceinline__ void head_rms_norm(f32x4 (&acc)[8], const bf16* __restrict__ nw, float eps, int grp) {
  float ss = 0.f;
  #pragma unroll
  for (int mt = 0; mt < 8; ++mt)
    #pragma unroll
    for (int e = 0; e < 4; ++e) ss += acc[mt][e] * acc[mt][e];
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  const float r = rsqrtf(ss * (1.0f / HD) + eps);
  #pragma unroll
  for (int mt = 0; mt < 8; ++mt)
    #pragma unroll
    for (int e = 0; e < 4; ++e) acc[mt][e] = acc[mt][e] * r * (float)nw[16 * mt + 4 * grp + e];
}

// Rotate-half RoPE at absolute position pos with the model's float32
// inverse frequencies inv_freq[64]: angle pos * inv_freq[d] formed in FP32.
__device__ __forceinline__ void head_rope(f32x4 (&acc)[8], const float* __restrict__ inv_freq, float pos, int grp) {
  #pragma unroll
  for (int mt = 0; mt < 4; ++mt)
    #pragma unroll
    for (int e = 0; e < 4; ++e) {
      float s, c;
      sincosf(pos * inv_freq[16 * mt + 4 * grp + e], &s, &c);
      const float lo = acc[mt][e], hi = acc[mt + 4][e];
      acc[mt][e] = lo * c - hi * s;
      acc[mt + 4][e] = hi * c + lo * s;
    }
}

// Store the lane's 128 dims as bf16 (4 consecutive dims per tile).
__device__ __forceinline__ void head_store(const f32x4 (&acc)[8], bf16* out, int grp) {
  out += 4 * grp;
  #pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    bf16x4 o;
    #pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (bf16)acc[mt][e];
    *reinterpret_cast<bf16x4*>(out + 16 * mt) = o;
  }
}

}  // namespace dspark
