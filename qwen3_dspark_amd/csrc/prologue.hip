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
// The rotary cos/sin either come from a table of the transaction's rows
// (dspark_rope_table: computed once and shared by every layer, as the
// model computes its position embeddings once per forward) or are formed
// in the epilogue from the positions; both give the same bits.
//
// Work: one workgroup per (head, 64-token tile) on the shared 32x32x16
// MFMA tile (head_gemm.h); all 8 waves run the epilogue on 16 dims of one
// token per lane.  Accumulation and the epilogue are FP32; outputs are
// rounded to bf16 once.
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
  const float* rope;         // optional [T][128]: cos of the 64 angles, then their sin
  bf16* q_out;               // [T, 16, 128]
  bf16* k_out;               // token rows of 8*128, kv_row_stride apart
  bf16* v_out;
  int64_t kv_row_stride;     // elements
  int tokens;
  int hidden;
  float eps;
};

// grid: 32 heads (0-15 q, 16-23 k, 24-31 v) x ceil(T / 64) token tiles, one
// dimension (see the XCD mapping below); 8 waves.
__global__ __launch_bounds__(HG_WAVES * WAVE) void qkv_prologue_kernel(PrologueArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[HG_SMEM];
  // XCD-aware placement: workgroups are dealt round-robin over the 8 XCDs
  // (each with its own L2), so the token tiles of one head are given ids
  // that share id % 8 - the head's weight slice is then fetched from HBM by
  // one L2 and served to all of its tiles from there.
  const int tiles = (a.tokens + HG_TOKENS - 1) / HG_TOKENS;
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int head = xcd + 8 * (slot / tiles);
  const int t0 = (slot % tiles) * HG_TOKENS;
  const int kind = head < HQ ? 0 : (head < HQ + HKV ? 1 : 2);       // workgroup-uniform
  const int hh = kind == 0 ? head : (kind == 1 ? head - HQ : head - HQ - HKV);
  const bf16* w = (kind == 0 ? a.wq : (kind == 1 ? a.wk : a.wv)) + (size_t)hh * HD * a.hidden;

  const HeadLane L;
  const int row = t0 + L.token();
  const int tok = min(row, a.tokens - 1);
  HeadNormW nw;
  HeadRope rope;
  float pos = 0.f;
  float v[2][8];
  float ss;
  // the epilogue's operands are fetched while the K halves are exchanged
  head_tile_gemm<false>(w, a.x, a.tokens, a.hidden, t0, smem, v, ss, [&]() {
    if (kind < 2) {
      nw.load(kind == 0 ? a.q_norm : a.k_norm);
      if (a.rope) rope.load(a.rope + (size_t)tok * 128);
      else pos = (float)a.positions[tok];
    }
  });
  if (kind < 2) {
    head_rms_norm(v, nw, a.eps, head_row_sumsq(v, smem));
    if (!a.rope) rope.compute(a.inv_freq, pos);
    head_rope(v, rope);
  }
  bf16* out = kind == 0 ? a.q_out + (size_t)tok * Q_ROW : (kind == 1 ? a.k_out : a.v_out) + (size_t)tok * a.kv_row_stride;
  head_store(v, out + (size_t)hh * HD, row < a.tokens);
}

// cos and sin of pos[t] * inv_freq[d] (FP32 angle, d < 64) for every row:
// table[t][d] = cos, table[t][64 + d] = sin.
__global__ __launch_bounds__(256) void rope_table_kernel(const float* __restrict__ inv_freq,
                                                         const int64_t* __restrict__ positions, int tokens,
                                                         float* __restrict__ table) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= tokens * 64) return;
  const int t = i >> 6, d = i & 63;
  float s, c;
  sincosf((float)positions[t] * inv_freq[d], &s, &c);
  table[(size_t)t * 128 + d] = c;
  table[(size_t)t * 128 + 64 + d] = s;
}

}  // namespace dspark

using namespace dspark;

extern "C" int dspark_qkv_prologue(const void* x, const void* wq, const void* wk, const void* wv,
                                   const void* q_norm, const void* k_norm, const float* inv_freq,
                                   const int64_t* positions, const float* rope, int tokens, int hidden, float eps,
                                   void* q_out, void* k_out, void* v_out, int64_t kv_row_stride, void* stream) {
  clear_error();
  DSPARK_REQUIRE(x && wq && wk && wv && q_norm && k_norm && inv_freq && positions && q_out && k_out && v_out,
                 "null pointer argument");
  DSPARK_REQUIRE(tokens >= 1 && hidden >= HG_COLS && hidden % HG_COLS == 0, "need tokens >= 1 and hidden a multiple of %d",
                 HG_COLS);
  DSPARK_REQUIRE(kv_row_stride >= KV_ROW && kv_row_stride % 8 == 0, "kv_row_stride must be >= 1024 and a multiple of 8");
  DSPARK_REQUIRE(eps > 0.f, "eps must be positive");
  const uintptr_t any = (uintptr_t)x | (uintptr_t)wq | (uintptr_t)wk | (uintptr_t)wv | (uintptr_t)q_out |
                        (uintptr_t)k_out | (uintptr_t)v_out | (uintptr_t)inv_freq | (uintptr_t)rope;
  DSPARK_REQUIRE(any % 16 == 0, "tensors must be 16-byte aligned");
  DSPARK_REQUIRE(((uintptr_t)q_norm | (uintptr_t)k_norm) % 8 == 0, "norm weights must be 8-byte aligned");
  PrologueArgs a{static_cast<const bf16*>(x), static_cast<const bf16*>(wq), static_cast<const bf16*>(wk),
                 static_cast<const bf16*>(wv), static_cast<const bf16*>(q_norm), static_cast<const bf16*>(k_norm),
                 inv_freq, positions, rope, static_cast<bf16*>(q_out), static_cast<bf16*>(k_out),
                 static_cast<bf16*>(v_out), kv_row_stride, tokens, hidden, eps};
  hipLaunchKernelGGL(qkv_prologue_kernel, dim3((HQ + 2 * HKV) * ((tokens + HG_TOKENS - 1) / HG_TOKENS)), dim3(HG_WAVES * WAVE), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("qkv_prologue_kernel");
}

extern "C" int dspark_rope_table(const float* inv_freq, const int64_t* positions, int tokens, float* table,
                                 void* stream) {
  clear_error();
  DSPARK_REQUIRE(inv_freq && positions && table, "null pointer argument");
  DSPARK_REQUIRE(tokens >= 1 && tokens <= (1 << 24), "tokens must be in [1, 2^24]");
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((tokens * 64 + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), inv_freq, positions, tokens, table);
  return launch_status("rope_table_kernel");
}
