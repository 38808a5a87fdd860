// Verify-layer prologue for gfx950: the Qwen3 attention steps that produce
// the kernel's inputs, in one launch per layer.
//
//   q = RoPE(RMSNorm_q(x Wq^T)),  k = RoPE(RMSNorm_k(x Wk^T)),  v = x Wv^T
//
// per 128-dim head (16 query heads, 8 KV heads), RMSNorm y = w x /
// sqrt(mean(x^2) + eps), RoPE in the rotate-half form with angles
// pos * inv_freq[d] (float32, the model's table).  This is what transformers'
// Qwen3Attention computes before the cache update / attention call used by
// dspark_qwen/persistent_qwen_target.py:45-95; the K/V rows can be written
// straight into the transaction scratch, replacing stage_layer's copy
// (dspark_qwen/persistent_target_kv.py:427-438).
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16): C^T[dim][token] = W[dim][:] .
// x[token][:], A = 16 weight rows, B = 16 tokens.  Every lane ends with 4
// consecutive dims (16*mt + 4*grp + e) of one token for each of the 8 dim
// tiles of a head, so the RMSNorm sum needs two cross-lane shuffles and the
// RoPE partner (d + 64 = tile mt + 4) sits in the same lane.  Accumulation
// and the epilogue are FP32; outputs are rounded to bf16 once.
#include "common.h"

namespace dspark {

constexpr int PRO_TOKENS = 64;                 // tokens per workgroup, 16 per wave
constexpr int PRO_KB = 64;                     // hidden columns per ring stage
constexpr int PRO_STAGES = 6;                  // ring depth (5 stages in flight)
constexpr int PRO_W_BYTES = HD * PRO_KB * 2;   // 128 weight rows x 128 B = 16 KiB
constexpr int PRO_X_BYTES = 16 * PRO_KB * 2;   // 16 token rows x 128 B per wave
constexpr int PRO_STAGE_BYTES = PRO_W_BYTES + 4 * PRO_X_BYTES;   // 24 KiB
constexpr int PRO_SMEM = PRO_STAGES * PRO_STAGE_BYTES;            // 144 KiB

struct PrologueArgs {
  const bf16* x;             // [T, hidden]
  const bf16* wq;            // [16*128, hidden]  (nn.Linear weight layout)
  const bf16* wk;            // [8*128, hidden]
  const bf16* wv;            // [8*128, hidden]
  const bf16* q_norm;        // [128]
  const bf16* k_norm;        // [128]
  const float* inv_freq;     // [64]
  const int64_t* positions;  // [T] absolute positions
  bf16* q_out;               // [T, 16, 128]
  bf16* k_out;               // token rows of 8*128, kv_row_stride apart
  bf16* v_out;
  int64_t kv_row_stride;     // elements
  int tokens;
  int hidden;
  float eps;
};

// 16-byte chunk swizzle of a 128-byte LDS row: the 16 rows 16*mt + col that
// one fragment read touches land on 16 distinct bank groups.
__device__ __forceinline__ int pro_swz(int row) { return (row >> 1) & 7; }

// grid: 32 heads (0-15 q, 16-23 k, 24-31 v) x ceil(T / 64) token tiles, one
// dimension (see the XCD mapping below); 4 waves of 16
// tokens.  The head's weight slice [128, hidden] and the workgroup's token
// rows stream through a 6-stage LDS ring fed by direct-to-LDS loads (every
// thread issues exactly 6 per stage: 4 weight pieces, 2 of its wave's token
// pieces), so the weights are read once per workgroup and shared by the 4
// waves, with 5 stages in flight.
__global__ __launch_bounds__(256) void qkv_prologue_kernel(PrologueArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[PRO_SMEM];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  // XCD-aware placement: workgroups are dealt round-robin over the 8 XCDs
  // (each with its own L2), so the token tiles of one head are given ids
  // that share id % 8 - the head's weight slice is then fetched from HBM by
  // one L2 and served to all of its tiles from there.
  const int tiles = (a.tokens + PRO_TOKENS - 1) / PRO_TOKENS;
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int head = xcd + 8 * (slot / tiles);
  const int t0 = (slot % tiles) * PRO_TOKENS + wave * 16;
  const int kind = head < HQ ? 0 : (head < HQ + HKV ? 1 : 2);
  const int hh = kind == 0 ? head : (kind == 1 ? head - HQ : head - HQ - HKV);
  const bf16* w = (kind == 0 ? a.wq : (kind == 1 ? a.wk : a.wv)) + (size_t)hh * HD * a.hidden;
  const int steps = a.hidden / PRO_KB;

  // Direct loads: lane L of a 1 KiB piece (8 rows x 128 B) fetches row
  // 8*piece + L/8, global chunk (L%8) ^ swz(row), landing at LDS chunk L%8.
  const uint32_t smem_lds = lds_address(smem);
  const int prow = lane >> 3;
  auto issue = [&](int step) {
    const int st = min(step, steps - 1);   // past the end: re-read the last stage (never used)
    const uint32_t base = smem_lds + (uint32_t)((step % PRO_STAGES) * PRO_STAGE_BYTES);
    const int k0 = st * PRO_KB;
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = 4 * wave + i;
      const int row = 8 * piece + prow;
      const bf16* src = w + (size_t)row * a.hidden + k0 + 8 * ((lane & 7) ^ pro_swz(row));
      lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)(piece * 1024)));
    }
    #pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = 8 * i + prow;
      const int tok = min(t0 + row, a.tokens - 1);
      const bf16* src = a.x + (size_t)tok * a.hidden + k0 + 8 * ((lane & 7) ^ pro_swz(row));
      lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (uint32_t)(PRO_W_BYTES + wave * PRO_X_BYTES + i * 1024)));
    }
  };

  f32x4 acc[8];
  #pragma unroll
  for (int mt = 0; mt < 8; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  #pragma unroll
  for (int p = 0; p < PRO_STAGES - 1; ++p) issue(p);
  for (int s = 0; s < steps; ++s) {
    // this thread's stage-s loads landed: the 6 loads of each of the
    // PRO_STAGES - 2 later stages may still be in flight
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * (PRO_STAGES - 2)) : "memory");
    asm volatile("s_barrier" ::: "memory");            // ... and everyone else's
    issue(s + PRO_STAGES - 1);
    const unsigned char* wst = smem + (s % PRO_STAGES) * PRO_STAGE_BYTES;
    const unsigned char* xst = wst + PRO_W_BYTES + wave * PRO_X_BYTES;
    #pragma unroll
    for (int u = 0; u < PRO_KB / 32; ++u) {
      const int c = 4 * u + grp;
      const bf16x8 xb = *reinterpret_cast<const bf16x8*>(xst + col * 128 + ((c ^ pro_swz(col)) << 4));
      #pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        const int row = 16 * mt + col;
        const bf16x8 wa = *reinterpret_cast<const bf16x8*>(wst + row * 128 + ((c ^ pro_swz(row)) << 4));
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, xb, acc[mt], 0, 0, 0);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (t0 >= a.tokens) return;   // wave-uniform; no barrier follows
  const int tok = min(t0 + col, a.tokens - 1);

  if (kind < 2) {
    float ss = 0.f;
    #pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      #pragma unroll
      for (int e = 0; e < 4; ++e) ss += acc[mt][e] * acc[mt][e];
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    const float r = rsqrtf(ss * (1.0f / HD) + a.eps);
    const bf16* nw = kind == 0 ? a.q_norm : a.k_norm;
    #pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      #pragma unroll
      for (int e = 0; e < 4; ++e) acc[mt][e] = acc[mt][e] * r * (float)nw[16 * mt + 4 * grp + e];
    const float pos = (float)a.positions[tok];
    #pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      #pragma unroll
      for (int e = 0; e < 4; ++e) {
        float s, c;
        sincosf(pos * a.inv_freq[16 * mt + 4 * grp + e], &s, &c);
        const float lo = acc[mt][e], hi = acc[mt + 4][e];
        acc[mt][e] = lo * c - hi * s;
        acc[mt + 4][e] = hi * c + lo * s;
      }
  }

  if (t0 + col < a.tokens) {
    bf16* out = kind == 0 ? a.q_out + (size_t)(t0 + col) * Q_ROW
                          : (kind == 1 ? a.k_out : a.v_out) + (size_t)(t0 + col) * a.kv_row_stride;
    out += (size_t)hh * HD + 4 * grp;
    #pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      bf16x4 o;
      #pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (bf16)acc[mt][e];
      *reinterpret_cast<bf16x4*>(out + 16 * mt) = o;
    }
  }
}

}  // namespace dspark

using namespace dspark;

extern "C" int dspark_qkv_prologue(const void* x, const void* wq, const void* wk, const void* wv,
                                   const void* q_norm, const void* k_norm, const float* inv_freq,
                                   const int64_t* positions, int tokens, int hidden, float eps,
                                   void* q_out, void* k_out, void* v_out, int64_t kv_row_stride, void* stream) {
  clear_error();
  DSPARK_REQUIRE(x && wq && wk && wv && q_norm && k_norm && inv_freq && positions && q_out && k_out && v_out,
                 "null pointer argument");
  DSPARK_REQUIRE(tokens >= 1 && hidden >= PRO_KB && hidden % PRO_KB == 0, "need tokens >= 1 and hidden a multiple of %d",
                 PRO_KB);
  DSPARK_REQUIRE(kv_row_stride >= KV_ROW && kv_row_stride % 8 == 0, "kv_row_stride must be >= 1024 and a multiple of 8");
  DSPARK_REQUIRE(eps > 0.f, "eps must be positive");
  const uintptr_t any = (uintptr_t)x | (uintptr_t)wq | (uintptr_t)wk | (uintptr_t)wv | (uintptr_t)q_out |
                        (uintptr_t)k_out | (uintptr_t)v_out;
  DSPARK_REQUIRE(any % 16 == 0, "tensors must be 16-byte aligned");
  PrologueArgs a{static_cast<const bf16*>(x), static_cast<const bf16*>(wq), static_cast<const bf16*>(wk),
                 static_cast<const bf16*>(wv), static_cast<const bf16*>(q_norm), static_cast<const bf16*>(k_norm),
                 inv_freq, positions, static_cast<bf16*>(q_out), static_cast<bf16*>(k_out),
                 static_cast<bf16*>(v_out), kv_row_stride, tokens, hidden, eps};
  hipLaunchKernelGGL(qkv_prologue_kernel, dim3((HQ + 2 * HKV) * ((tokens + PRO_TOKENS - 1) / PRO_TOKENS)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("qkv_prologue_kernel");
}
