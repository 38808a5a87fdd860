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
#include "head_gemm.h"

namespace dspark {

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

// grid: 32 heads (0-15 q, 16-23 k, 24-31 v) x ceil(T / 64) token tiles, one
// dimension (see the XCD mapping below); 8 waves, of which waves 0-3 (16
// tokens each) run the epilogue.
__global__ __launch_bounds__(HG_WAVES * WAVE) void qkv_prologue_kernel(PrologueArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[HG_SMEM];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  // XCD-aware placement: workgroups are dealt round-robin over the 8 XCDs
  // (each with its own L2), so the token tiles of one head are given ids
  // that share id % 8 - the head's weight slice is then fetched from HBM by
  // one L2 and served to all of its tiles from there.
  const int tiles = (a.tokens + HG_TOKENS - 1) / HG_TOKENS;
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int head = xcd + 8 * (slot / tiles);
  const int t0 = (slot % tiles) * HG_TOKENS;
  const int kind = head < HQ ? 0 : (head < HQ + HKV ? 1 : 2);
  const int hh = kind == 0 ? head : (kind == 1 ? head - HQ : head - HQ - HKV);
  const bf16* w = (kind == 0 ? a.wq : (kind == 1 ? a.wk : a.wv)) + (size_t)hh * HD * a.hidden;

  f32x4 acc[8];
  float ss;
  head_tile_gemm<false>(w, a.x, a.tokens, a.hidden, t0, smem, acc, ss);
  if (wave >= 4) return;        // the second column half; no barrier follows
  const int tw = t0 + 16 * wave;
  if (tw >= a.tokens) return;   // wave-uniform; no barrier follows
  const int tok = min(tw + col, a.tokens - 1);
  if (kind < 2) {
    head_rms_norm(acc, kind == 0 ? a.q_norm : a.k_norm, a.eps, grp);
    head_rope(acc, a.inv_freq, (float)a.positions[tok], grp);
  }
  if (tw + col < a.tokens) {
    bf16* out = kind == 0 ? a.q_out + (size_t)(tw + col) * Q_ROW
                          : (kind == 1 ? a.k_out : a.v_out) + (size_t)(tw + col) * a.kv_row_stride;
    head_store(acc, out + (size_t)hh * HD, grp);
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
  DSPARK_REQUIRE(tokens >= 1 && hidden >= HG_COLS && hidden % HG_COLS == 0, "need tokens >= 1 and hidden a multiple of %d",
                 HG_COLS);
  DSPARK_REQUIRE(kv_row_stride >= KV_ROW && kv_row_stride % 8 == 0, "kv_row_stride must be >= 1024 and a multiple of 8");
  DSPARK_REQUIRE(eps > 0.f, "eps must be positive");
  const uintptr_t any = (uintptr_t)x | (uintptr_t)wq | (uintptr_t)wk | (uintptr_t)wv | (uintptr_t)q_out |
                        (uintptr_t)k_out | (uintptr_t)v_out;
  DSPARK_REQUIRE(any % 16 == 0, "tensors must be 16-byte aligned");
  PrologueArgs a{static_cast<const bf16*>(x), static_cast<const bf16*>(wq), static_cast<const bf16*>(wk),
                 static_cast<const bf16*>(wv), static_cast<const bf16*>(q_norm), static_cast<const bf16*>(k_norm),
                 inv_freq, positions, static_cast<bf16*>(q_out), static_cast<bf16*>(k_out),
                 static_cast<bf16*>(v_out), kv_row_stride, tokens, hidden, eps};
  hipLaunchKernelGGL(qkv_prologue_kernel, dim3((HQ + 2 * HKV) * ((tokens + HG_TOKENS - 1) / HG_TOKENS)), dim3(HG_WAVES * WAVE), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("qkv_prologue_kernel");
}
