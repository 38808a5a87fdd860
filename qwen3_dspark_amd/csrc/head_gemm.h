// One 128-output-column "head" of a linear layer for 64 tokens, on gfx950:
//   C^T[dim][token] = W[dim][:] . x[token][:]      (dim < 128, token < 64)
// shared by the projection kernels (the target's verify-layer prologue and
// the draft context K/V projection).
//
// MFMA mapping (v_mfma_f32_32x32x16_bf16): A = 32 weight rows, B = 32
// tokens.  A lane l of the A (B) operand supplies row (column) l%32 at
// k = 8(l/32) + i; accumulator register r of lane l is row
// 8(r/4) + 4(l/32) + r%4, column l%32.  The workgroup has 8 waves, two per
// SIMD, wave w taking
//   tg = w & 1         tokens t0 + 32 tg .. + 31,
//   dh = (w >> 1) & 1  dim tiles dh and dh + 2 (dims 32 dh .. + 31 and
//                      their rotate-half partners + 64),
//   kq = w >> 2        sub-stage kq of every ring stage (split K),
// so that each wave reads 2 A and 1 B fragment per two MFMAs.  The two K
// halves are then combined by a reduce-scatter through LDS: wave kq keeps
// accumulator registers 8 kq .. 8 kq + 7 and takes the partner wave's
// share of them.  Every lane of every wave ends with 16 dims of one token,
//   v[a][4 jj + i] = C^T[32 (dh + 2a) + 8 (2 kq + jj) + 4 (l/32) + i][t0 + 32 tg + l%32],
// so the RoPE partner of v[0][e] (dim d < 64) is v[1][e] (dim d + 64), a
// per-token reduction over the 128 dims spans one lane pair (l, l ^ 32)
// and the 4 waves of the token group, and the lane pair together holds 8
// consecutive dims per (a, jj) for 16-byte stores.
//
// The head's weight slice [128, hidden] and the workgroup's token rows
// stream through a 3-stage LDS ring fed by direct-to-LDS loads.  A stage is
// two 64-column sub-stages (128 hidden columns, one barrier): every thread
// issues exactly 3 loads per sub-stage (2 weight pieces, 1 token piece), so
// the weights are read once per workgroup and shared by the 8 waves, with 2
// stages in flight.  The last two stages issue nothing (the waits count
// down to zero instead), so no load outlives the tile.
#pragma once
#include "common.h"

namespace dspark {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int HG_TOKENS = 64;                    // tokens per workgroup
constexpr int HG_WAVES = 8;                      // 2 token groups x 2 dim-tile pairs x 2 column halves
constexpr int HG_KB = 64;                        // hidden columns per sub-stage
constexpr int HG_SUB = 2;                        // sub-stages per ring stage (one barrier each)
constexpr int HG_STAGES = 3;                     // ring depth (2 stages in flight)
constexpr int HG_W_BYTES = HD * HG_KB * 2;       // 128 weight rows x 128 B = 16 KiB
constexpr int HG_X_BYTES = 16 * HG_KB * 2;       // 16 token rows x 128 B
constexpr int HG_SUB_BYTES = HG_W_BYTES + 4 * HG_X_BYTES;     // 24 KiB
constexpr int HG_STAGE_BYTES = HG_SUB * HG_SUB_BYTES;         // 48 KiB
constexpr int HG_SMEM = HG_STAGES * HG_STAGE_BYTES;            // 144 KiB
constexpr int HG_COLS = HG_KB * HG_SUB;          // hidden columns per ring stage (hidden must be a multiple)
static_assert(HG_STAGES == 3, "the ring's wait counts assume one stage in flight behind the current one");

// LDS reused once the ring is drained: the K-half exchange (32 KiB), the
// row sums of squares of the token rows (2 KiB) and the per-token partial
// sums of a head_row_sumsq (1 KiB).
constexpr int HG_XCH_OFF = 0;
constexpr int HG_SSX_OFF = 32768;
constexpr int HG_ROW_OFF = HG_SSX_OFF + HG_WAVES * WAVE * 4;
static_assert(HG_ROW_OFF + 2 * 4 * 32 * 4 <= HG_SMEM, "epilogue scratch exceeds the ring");

// 16-byte chunk swizzle of a 128-byte LDS row: the 16 rows that one
// 16-lane phase of a fragment read touches land on 16 distinct bank groups.
__device__ __forceinline__ int hg_swz(int row) { return (row >> 1) & 7; }

// Where this lane's values live (see the layout above).
struct HeadLane {
  int n, hl, tg, dh, kq;
  __device__ __forceinline__ HeadLane() {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    n = lane & 31;
    hl = lane >> 5;
    tg = wave & 1;
    dh = (wave >> 1) & 1;
    kq = wave >> 2;
  }
  // first of the 4 consecutive dims of v[a][4 jj .. 4 jj + 3]
  __device__ __forceinline__ int dim(int a, int jj) const { return 32 * (dh + 2 * a) + 8 * (2 * kq + jj) + 4 * hl; }
  // the lane's token within the workgroup's tile
  __device__ __forceinline__ int token() const { return 32 * tg + n; }
};

// w: first of the head's 128 weight rows (row stride `hidden`); x: token
// rows (row stride `hidden`), `tokens` of them; t0: the workgroup's first
// token.  Rows past `tokens` re-read the last token (their results are
// discarded by the caller).  pre_combine() runs once the ring has drained
// and before the exchange (a place to issue the epilogue's global loads).
// With SUMSQ, ss receives sum(x^2) over the lane's token row (the same
// value in all lanes of that token).  The exchange is read after the
// function's last barrier: afterwards the caller may use only the
// HG_ROW_OFF region (head_row_sumsq) of the ring's LDS.
template <bool SUMSQ, typename PreCombine>
__device__ __forceinline__ void head_tile_gemm(const bf16* __restrict__ w, const bf16* __restrict__ x, int tokens,
                                               int hidden, int t0, unsigned char* smem, float (&v)[2][8], float& ss,
                                               PreCombine&& pre_combine) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const HeadLane L;
  const int steps = hidden / HG_COLS;

  // Direct loads: lane L of a 1 KiB piece (8 rows x 128 B) fetches row
  // 8*piece + L/8, global chunk (L%8) ^ swz(row), landing at LDS chunk L%8.
  // Wave w loads weight pieces 2w, 2w+1 and token rows 8w .. 8w+7.
  const uint32_t smem_lds = lds_address(smem);
  const int prow = lane >> 3;
  auto issue = [&](int step) {
    #pragma unroll
    for (int sub = 0; sub < HG_SUB; ++sub) {
      const uint32_t base = smem_lds + (uint32_t)((step % HG_STAGES) * HG_STAGE_BYTES + sub * HG_SUB_BYTES);
      const int k0 = (step * HG_SUB + sub) * HG_KB;
      #pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int piece = 2 * wave + i;
        const int row = 8 * piece + prow;
        const bf16* src = w + (size_t)row * hidden + k0 + 8 * ((lane & 7) ^ hg_swz(row));
        lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)(piece * 1024)));
      }
      const int row = 8 * wave + prow;      // token row of the tile
      const int tok = min(t0 + row, tokens - 1);
      const bf16* src = x + (size_t)tok * hidden + k0 + 8 * ((lane & 7) ^ hg_swz(row));
      lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)(HG_W_BYTES + wave * 1024)));
    }
  };

  f32x16 acc[2];
  #pragma unroll
  for (int a = 0; a < 2; ++a)
    #pragma unroll
    for (int r = 0; r < 16; ++r) acc[a][r] = 0.f;
  ss = 0.f;
  issue(0);
  if (steps > 1) issue(1);
  const int R = L.token();
  for (int s = 0; s < steps; ++s) {
    // this thread's stage-s loads landed (stage s + 1, when there is one,
    // may still be in flight: its 3 loads per sub-stage) ...
    if (s + 1 < steps) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * HG_SUB) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");            // ... and everyone else's
    if (s + 2 < steps) issue(s + 2);
    const unsigned char* wst = smem + (s % HG_STAGES) * HG_STAGE_BYTES + L.kq * HG_SUB_BYTES;
    const unsigned char* xst = wst + HG_W_BYTES;
    #pragma unroll
    for (int ks = 0; ks < HG_KB / 16; ++ks) {
      const int c = 2 * ks + L.hl;
      const bf16x8 xb = *reinterpret_cast<const bf16x8*>(xst + R * 128 + ((c ^ hg_swz(R)) << 4));
      if (SUMSQ) {
        #pragma unroll
        for (int i = 0; i < 8; ++i) ss += (float)xb[i] * (float)xb[i];
      }
      #pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int row = 32 * (L.dh + 2 * a) + L.n;
        const bf16x8 wa = *reinterpret_cast<const bf16x8*>(wst + row * 128 + ((c ^ hg_swz(row)) << 4));
        acc[a] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa, xb, acc[a], 0, 0, 0);
      }
    }
  }
  pre_combine();
  __syncthreads();   // every wave is done with the ring: reuse it for the exchange

  // Reduce-scatter of the K halves: wave kq hands over registers
  // 8 (1 - kq) .. + 7 and keeps 8 kq .. + 7.  Slots are [pair][kq][quad][lane]
  // f32x4, so each 16-byte LDS access of a wave is contiguous.
  const int pair = wave & 3;
  f32x4* xch = reinterpret_cast<f32x4*>(smem + HG_XCH_OFF);
  #pragma unroll
  for (int a = 0; a < 2; ++a)
    #pragma unroll
    for (int q = 0; q < 2; ++q) {
      f32x4 g;
      #pragma unroll
      for (int i = 0; i < 4; ++i) g[i] = L.kq == 0 ? acc[a][8 + 4 * q + i] : acc[a][4 * q + i];
      xch[((pair * 2 + L.kq) * 4 + 2 * a + q) * 64 + lane] = g;
    }
  float* ssx = reinterpret_cast<float*>(smem + HG_SSX_OFF);
  if (SUMSQ) {
    ss += __shfl_xor(ss, 32);                   // the two k-chunks of each kstep
    ssx[wave * 64 + lane] = ss;
  }
  __syncthreads();
  #pragma unroll
  for (int a = 0; a < 2; ++a)
    #pragma unroll
    for (int q = 0; q < 2; ++q) {
      const f32x4 o = xch[((pair * 2 + (L.kq ^ 1)) * 4 + 2 * a + q) * 64 + lane];
      #pragma unroll
      for (int i = 0; i < 4; ++i) v[a][4 * q + i] = (L.kq == 0 ? acc[a][4 * q + i] : acc[a][8 + 4 * q + i]) + o[i];
    }
  if (SUMSQ) ss += ssx[(wave ^ 4) * 64 + lane];  // the other column half of the row
}

// sum over the 128 dims of v^2 for the lane's token.  Every wave of the
// workgroup must call it (it holds a barrier); all lanes of a token get the
// same value.
__device__ __forceinline__ float head_row_sumsq(const float (&v)[2][8], unsigned char* smem) {
  const HeadLane L;
  float s = 0.f;
  #pragma unroll
  for (int a = 0; a < 2; ++a)
    #pragma unroll
    for (int e = 0; e < 8; ++e) s += v[a][e] * v[a][e];
  s += __shfl_xor(s, 32);
  float* b = reinterpret_cast<float*>(smem + HG_ROW_OFF) + L.tg * 4 * 32;
  if (L.hl == 0) b[(L.dh * 2 + L.kq) * 32 + L.n] = s;
  __syncthreads();
  return b[L.n] + b[32 + L.n] + b[64 + L.n] + b[96 + L.n];
}

// The lane's 16 norm weights of a [128] RMSNorm weight vector.
struct HeadNormW {
  bf16x4 w[2][2];
  __device__ __forceinline__ void load(const bf16* __restrict__ nw) {
    const HeadLane L;
    #pragma unroll
    for (int a = 0; a < 2; ++a)
      #pragma unroll
      for (int jj = 0; jj < 2; ++jj) w[a][jj] = *reinterpret_cast<const bf16x4*>(nw + L.dim(a, jj));
  }
};

// RMSNorm y = w x / sqrt(mean(x^2) + eps) with the row's sum of squares.
__device__ __forceinline__ void head_rms_norm(float (&v)[2][8], const HeadNormW& nw, float eps, float sumsq) {
  const float r = rsqrtf(sumsq * (1.0f / HD) + eps);
  #pragma unroll
  for (int a = 0; a < 2; ++a)
    #pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      #pragma unroll
      for (int i = 0; i < 4; ++i) v[a][4 * jj + i] = v[a][4 * jj + i] * r * (float)nw.w[a][jj][i];
}

// cos / sin of the lane's 8 rotary angles (dims L.dim(0, jj) + i < 64).
struct HeadRope {
  f32x4 c[2], s[2];
  // from a precomputed row: cos of the 64 angles, then their sin (float32)
  __device__ __forceinline__ void load(const float* __restrict__ row) {
    const HeadLane L;
    #pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      c[jj] = *reinterpret_cast<const f32x4*>(row + L.dim(0, jj));
      s[jj] = *reinterpret_cast<const f32x4*>(row + 64 + L.dim(0, jj));
    }
  }
  // angle pos * inv_freq[d] formed in FP32, the model's float32 table
  __device__ __forceinline__ void compute(const float* __restrict__ inv_freq, float pos) {
    const HeadLane L;
    #pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const f32x4 f = *reinterpret_cast<const f32x4*>(inv_freq + L.dim(0, jj));
      #pragma unroll
      for (int i = 0; i < 4; ++i) {
        float sn, cs;
        sincosf(pos * f[i], &sn, &cs);
        c[jj][i] = cs;
        s[jj][i] = sn;
      }
    }
  }
};

// Rotate-half RoPE: (x_d, x_{d+64}) -> (x_d cos - x_{d+64} sin, x_{d+64} cos + x_d sin).
__device__ __forceinline__ void head_rope(float (&v)[2][8], const HeadRope& r) {
  #pragma unroll
  for (int jj = 0; jj < 2; ++jj)
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = v[0][4 * jj + i], hi = v[1][4 * jj + i];
      v[0][4 * jj + i] = lo * r.c[jj][i] - hi * r.s[jj][i];
      v[1][4 * jj + i] = hi * r.c[jj][i] + lo * r.s[jj][i];
    }
}

// Store the lane pair's 32 dims of its token as bf16 (row = the token's
// 128-dim head): lane hl of the pair writes dims
// 32 (dh + 2a) + 16 kq + 8 hl .. + 7 for a = 0, 1, after swapping one
// 8-byte half with its partner.  Both lanes of the pair must execute it;
// `valid` gates the store only.
__device__ __forceinline__ void head_store(const float (&v)[2][8], bf16* row, bool valid) {
  const HeadLane L;
  #pragma unroll
  for (int a = 0; a < 2; ++a) {
    uint32_t pk[2][2];
    #pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      bf16x4 b;
      #pragma unroll
      for (int i = 0; i < 4; ++i) b[i] = (bf16)v[a][4 * jj + i];
      __builtin_memcpy(pk[jj], &b, 8);
    }
    // lane hl keeps its jj = hl half and receives the partner's jj = hl half
    const uint32_t g0 = L.hl ? pk[0][0] : pk[1][0];
    const uint32_t g1 = L.hl ? pk[0][1] : pk[1][1];
    const uint32_t r0 = (uint32_t)__shfl_xor((int)g0, 32);
    const uint32_t r1 = (uint32_t)__shfl_xor((int)g1, 32);
    uint32_t o[4];
    if (L.hl == 0) {
      o[0] = pk[0][0]; o[1] = pk[0][1]; o[2] = r0; o[3] = r1;
    } else {
      o[0] = r0; o[1] = r1; o[2] = pk[1][0]; o[3] = pk[1][1];
    }
    if (valid) {
      bf16x8 ov;
      __builtin_memcpy(&ov, o, 16);
      *reinterpret_cast<bf16x8*>(row + 32 * (L.dh + 2 * a) + 16 * L.kq + 8 * L.hl) = ov;
    }
  }
}

}  // namespace dspark
