// Draft context K/V projection for gfx950: everything DSpark's draft does to
// newly committed target features after its `fc` layer, for all draft
// layers in one launch, written straight into the slotted draft pool.
//
//   ctx = RMSNorm_ctx(f)                       f = fc(features), [T, hidden]
//   k_l = RoPE(RMSNorm_k,l(ctx Wk_l^T)),  v_l = ctx Wv_l^T      per 128-dim head
//
// (dspark_qwen/model.py:141-146 project_context_kv, :41-45 project_kv and
// :22-24 rotate, as used by dspark_qwen/packed_draft.py:147-158
// append_committed).  RMSNorm y = w x / sqrt(mean(x^2) + eps); RoPE in the
// rotate-half form at each token's absolute position.
//
// The context norm is applied without materialising ctx: its weight w_c is
// folded into the projection weights once by the host (Wk_l diag(w_c),
// Wv_l diag(w_c)), and its per-token factor 1/sqrt(mean(f^2) + eps) commutes
// with the projection, so each workgroup accumulates sum(f^2) of its tokens
// while the rows stream through LDS for the MFMAs and scales the FP32
// result in the epilogue.  Accumulation and epilogue are FP32; every output
// is rounded to bf16 once.
//
// Work: one workgroup per (layer, K or V, KV head) x 64-token tile (the
// shared 32x32x16 MFMA tile of head_gemm.h), XCD-aware so that the token tiles of one weight
// slice share an L2.  Token t belongs to the request whose record
// (slot, first position, first token, count) covers it; its row goes to
// (slot, position) of every layer's pool.  A non-finite output sets *flag
// (the caller publishes the rows only when it is clear).
#include "head_gemm.h"

namespace dspark {

struct DraftProjArgs {
  const bf16* x;             // [T, hidden] fc output (before the context norm)
  const bf16* w;             // [layers][2][8*128][hidden]: folded k_proj then v_proj
  const bf16* k_norm;        // [layers][128]
  const float* inv_freq;     // [64]
  const int32_t* req;        // [n_req][4]: slot, first position, first token, token count
  bf16* k_pool;              // layer 0 of the pool; element (slot, head, pos, d) at
  bf16* v_pool;              //   slot*slot_stride + head*head_stride + pos*128 + d
  int64_t layer_stride;      // elements
  int64_t slot_stride;
  int64_t head_stride;
  int32_t* flag;             // optional: set to 1 on a non-finite output
  int tokens;
  int hidden;
  int layers;
  int n_req;
  float eps_ctx;
  float eps_k;
};

__global__ __launch_bounds__(HG_WAVES * WAVE) void draft_kv_project_kernel(DraftProjArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[HG_SMEM];
  const int lane = threadIdx.x & 63;
  const int tiles = (a.tokens + HG_TOKENS - 1) / HG_TOKENS;
  const int xcd = blockIdx.x & 7;
  const int slot_id = blockIdx.x >> 3;
  const int job = xcd + 8 * (slot_id / tiles);        // layer * 16 + (V ? 8 : 0) + head
  const int t0 = (slot_id % tiles) * HG_TOKENS;
  const int layer = job >> 4;
  const bool is_v = (job & 8) != 0;                   // workgroup-uniform
  const int head = job & 7;
  const bf16* w = a.w + ((size_t)(2 * layer + (is_v ? 1 : 0)) * KV_ROW + (size_t)head * HD) * a.hidden;

  const HeadLane L;
  const int row = t0 + L.token();
  const int tok = min(row, a.tokens - 1);
  HeadNormW nw;
  float v[2][8];
  float ss;
  head_tile_gemm<true>(w, a.x, a.tokens, a.hidden, t0, smem, v, ss, [&]() {
    if (!is_v) nw.load(a.k_norm + (size_t)layer * HD);
  });

  // Context norm: the token row's sum of squares, applied as one scale of
  // the FP32 result.
  const float r = rsqrtf(ss / (float)a.hidden + a.eps_ctx);
  #pragma unroll
  for (int i = 0; i < 2; ++i)
    #pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] *= r;

  // The request holding this token: the last record whose first token <= tok.
  int lo = 0, hi = a.n_req - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.req[4 * mid + 2] <= tok) lo = mid;
    else hi = mid - 1;
  }
  const int32_t* rq = a.req + 4 * lo;
  const int pos = rq[1] + (tok - rq[2]);
  if (!is_v) {
    head_rms_norm(v, nw, a.eps_k, head_row_sumsq(v, smem));
    HeadRope rope;
    rope.compute(a.inv_freq, (float)pos);
    head_rope(v, rope);
  }
  const bool valid = row < a.tokens;
  if (a.flag) {
    bool bad = false;
    #pragma unroll
    for (int i = 0; i < 2; ++i)
      #pragma unroll
      for (int e = 0; e < 8; ++e) bad |= !__builtin_isfinite(v[i][e]);
    if (__builtin_amdgcn_ballot_w64(bad && valid) && lane == 0) *a.flag = 1;   // idempotent vector store
  }
  bf16* out = (is_v ? a.v_pool : a.k_pool) + (size_t)layer * a.layer_stride + (size_t)rq[0] * a.slot_stride +
              (size_t)head * a.head_stride + (size_t)pos * HD;
  head_store(v, out, valid);
}

}  // namespace dspark

using namespace dspark;

extern "C" int dspark_draft_kv_project(const void* x, int tokens, int hidden, const void* w, const void* k_norm,
                                       int layers, const float* inv_freq, const int32_t* req, int n_req,
                                       float eps_ctx, float eps_k, void* k_pool, void* v_pool, int64_t layer_stride,
                                       int64_t slot_stride, int64_t head_stride, int32_t* flag, void* stream) {
  clear_error();
  DSPARK_REQUIRE(x && w && k_norm && inv_freq && req && k_pool && v_pool, "null pointer argument");
  DSPARK_REQUIRE(tokens >= 1 && hidden >= HG_COLS && hidden % HG_COLS == 0, "need tokens >= 1 and hidden a multiple of %d",
                 HG_COLS);
  DSPARK_REQUIRE(layers >= 1 && layers <= 64, "layers must be in [1, 64] (got %d)", layers);
  DSPARK_REQUIRE(n_req >= 1 && n_req <= tokens, "n_req must be in [1, tokens]");
  DSPARK_REQUIRE(eps_ctx > 0.f && eps_k > 0.f, "eps must be positive");
  DSPARK_REQUIRE(layer_stride >= 0 && slot_stride >= 0 && head_stride >= HD && head_stride % 8 == 0 &&
                     slot_stride % 8 == 0 && layer_stride % 8 == 0,
                 "pool strides must be multiples of 8 elements (head stride >= 128)");
  const uintptr_t any = (uintptr_t)x | (uintptr_t)w | (uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)inv_freq;
  DSPARK_REQUIRE(any % 16 == 0, "tensors must be 16-byte aligned");
  DSPARK_REQUIRE((uintptr_t)k_norm % 8 == 0, "k_norm must be 8-byte aligned");
  const int64_t tiles = (tokens + HG_TOKENS - 1) / HG_TOKENS;
  DSPARK_REQUIRE(tiles * layers * 2 * HKV <= 0x7fffffffLL, "too many tokens");
  DraftProjArgs a{static_cast<const bf16*>(x), static_cast<const bf16*>(w), static_cast<const bf16*>(k_norm), inv_freq,
                  req, static_cast<bf16*>(k_pool), static_cast<bf16*>(v_pool), layer_stride, slot_stride, head_stride,
                  flag, tokens, hidden, layers, n_req, eps_ctx, eps_k};
  hipLaunchKernelGGL(draft_kv_project_kernel, dim3((unsigned)(tiles * layers * 2 * HKV)), dim3(HG_WAVES * WAVE), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("draft_kv_project_kernel");
}

// ---------------------------------------------------------------------------
// The same projection for large appends, after a library GEMM.
//
// From a few thousand tokens on, the projection is a plain GEMM-bound
// problem (T x hidden by hidden x layers*2*1024) that hipBLASLt runs at a
// much higher MFMA rate than the fused 64-token tiles above.  The host then
// computes y = f Wfold^T (the folded weights as one [layers*2*1024, hidden]
// matrix) and this kernel applies everything else: the context-norm factor
// 1/sqrt(mean(f^2) + eps) of each token, k_norm and RoPE on the K heads, and
// the store into each request's pool slot, with the same finiteness flag.
// y may be FP32 (the GEMM's accumulator, as the fused kernel keeps it: the
// outputs are then rounded to bf16 once, at the same point) or bf16 (the
// reference's autocast rounding of k_proj / v_proj).
//
// Work: 16 tokens per workgroup, one per 16-lane group; lane c of a group
// holds dims 8c .. 8c+7 of a head, so each (token, head) is one coalesced
// 256-byte load and one 256-byte store.  A group walks all layers x (K, V)
// x heads of its token with the token's norm factor and RoPE angles
// computed once.
// ---------------------------------------------------------------------------
namespace dspark {

struct DraftEpiArgs {
  const void* y;             // [T, y_stride] bf16 or FP32: columns [layer][K or V][head][128]
  const bf16* x;             // [T, hidden] fc output (for the context-norm factor)
  const bf16* k_norm;        // [layers][128]
  const float* inv_freq;     // [64]
  const int32_t* req;        // [n_req][4]: slot, first position, first token, token count
  bf16* k_pool;
  bf16* v_pool;
  int64_t y_stride;          // elements
  int64_t layer_stride;
  int64_t slot_stride;
  int64_t head_stride;
  int32_t* flag;
  int tokens;                // rows of y and x in this call
  int token0;                // index of row 0 among the records' tokens
  int hidden;
  int layers;
  int n_req;
  float eps_ctx;
  float eps_k;
};

// Eight consecutive values of a y row as FP32.
__device__ __forceinline__ void load_y8(const bf16* p, float (&v)[8]) {
  const bf16x8 b = ld8(p);
  #pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)b[e];
}
__device__ __forceinline__ void load_y8(const float* p, float (&v)[8]) {
  const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
  #pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = lo[e];
    v[4 + e] = hi[e];
  }
}

template <typename YT>
__global__ __launch_bounds__(256) void draft_kv_epilogue_kernel(DraftEpiArgs a) {
  const int lane = threadIdx.x & 63;
  const int c = threadIdx.x & 15;                      // 8-dim chunk of a head
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool valid = row < a.tokens;
  const int t = min(row, a.tokens - 1);

  // context-norm factor: the group's 16 lanes split the row
  float ss = 0.f;
  const bf16* xr = a.x + (size_t)t * a.hidden;
  for (int d = 8 * c; d < a.hidden; d += 128) {
    const bf16x8 v = ld8(xr + d);
    #pragma unroll
    for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
  }
  #pragma unroll
  for (int off = 8; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss / (float)a.hidden + a.eps_ctx);

  // the request holding this token
  const int tok = a.token0 + t;
  int lo = 0, hi = a.n_req - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.req[4 * mid + 2] <= tok) lo = mid;
    else hi = mid - 1;
  }
  const int32_t* rq = a.req + 4 * lo;
  const int pos = rq[1] + (tok - rq[2]);

  // RoPE angles of this lane's dims: dim 8c+e pairs with dim 8c+e +- 64,
  // which lane c ^ 8 holds; both use inv_freq[(8c+e) mod 64].
  float cs[8], sn[8];
  #pragma unroll
  for (int e = 0; e < 8; ++e) sincosf((float)pos * a.inv_freq[(8 * c + e) & 63], &sn[e], &cs[e]);
  const bool upper = c >= 8;

  bool bad = false;
  for (int layer = 0; layer < a.layers; ++layer) {
    float kw[8];
    #pragma unroll
    for (int e = 0; e < 8; ++e) kw[e] = (float)a.k_norm[(size_t)layer * HD + 8 * c + e];
    const YT* yl = static_cast<const YT*>(a.y) + (size_t)t * a.y_stride + (size_t)layer * 2 * KV_ROW;
    bf16* kout = a.k_pool + (size_t)layer * a.layer_stride + (size_t)rq[0] * a.slot_stride + (size_t)pos * HD + 8 * c;
    bf16* vout = a.v_pool + (size_t)layer * a.layer_stride + (size_t)rq[0] * a.slot_stride + (size_t)pos * HD + 8 * c;
    #pragma unroll 2
    for (int h = 0; h < HKV; ++h) {
      // K head h: norm factor, k_norm, RoPE
      float k[8];
      load_y8(yl + (size_t)h * HD + 8 * c, k);
      float kss = 0.f;
      #pragma unroll
      for (int e = 0; e < 8; ++e) {
        k[e] *= r;
        kss += k[e] * k[e];
      }
      #pragma unroll
      for (int off = 8; off >= 1; off >>= 1) kss += __shfl_xor(kss, off);
      const float kr = rsqrtf(kss * (1.0f / HD) + a.eps_k);
      #pragma unroll
      for (int e = 0; e < 8; ++e) k[e] = k[e] * kr * kw[e];
      bf16x8 ko;
      #pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float other = __shfl_xor(k[e], 8);
        // lower half: lo*cos - hi*sin; upper half: hi*cos + lo*sin
        const float o = upper ? k[e] * cs[e] + other * sn[e] : k[e] * cs[e] - other * sn[e];
        bad |= !__builtin_isfinite(o);
        ko[e] = (bf16)o;
      }
      // V head h: the norm factor only
      float vv[8];
      load_y8(yl + KV_ROW + (size_t)h * HD + 8 * c, vv);
      bf16x8 vo;
      #pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float o = vv[e] * r;
        bad |= !__builtin_isfinite(o);
        vo[e] = (bf16)o;
      }
      if (valid) {
        *reinterpret_cast<bf16x8*>(kout + (size_t)h * a.head_stride) = ko;
        *reinterpret_cast<bf16x8*>(vout + (size_t)h * a.head_stride) = vo;
      }
    }
  }
  if (a.flag && __builtin_amdgcn_ballot_w64(bad && valid) && lane == 0) *a.flag = 1;   // idempotent vector store
}

}  // namespace dspark

extern "C" int dspark_draft_kv_epilogue(const void* y, int y_dtype, int64_t y_stride, const void* x, int tokens, int token0,
                                        int hidden, const void* k_norm, int layers, const float* inv_freq,
                                        const int32_t* req, int n_req, float eps_ctx, float eps_k, void* k_pool,
                                        void* v_pool, int64_t layer_stride, int64_t slot_stride, int64_t head_stride,
                                        int32_t* flag, void* stream) {
  clear_error();
  DSPARK_REQUIRE(y && x && k_norm && inv_freq && req && k_pool && v_pool, "null pointer argument");
  DSPARK_REQUIRE(y_dtype == 0 || y_dtype == 1, "y_dtype must be 0 (bf16) or 1 (fp32)");
  DSPARK_REQUIRE(tokens >= 1 && token0 >= 0 && hidden >= 128 && hidden % 128 == 0,
                 "need tokens >= 1, token0 >= 0 and hidden a multiple of 128");
  DSPARK_REQUIRE(layers >= 1 && layers <= 64, "layers must be in [1, 64] (got %d)", layers);
  DSPARK_REQUIRE(y_stride >= (int64_t)layers * 2 * KV_ROW && y_stride % 8 == 0,
                 "y rows must hold layers*2*1024 columns, stride a multiple of 8");
  DSPARK_REQUIRE(n_req >= 1, "n_req must be >= 1");
  DSPARK_REQUIRE(eps_ctx > 0.f && eps_k > 0.f, "eps must be positive");
  DSPARK_REQUIRE(layer_stride >= 0 && slot_stride >= 0 && head_stride >= HD && head_stride % 8 == 0 &&
                     slot_stride % 8 == 0 && layer_stride % 8 == 0,
                 "pool strides must be multiples of 8 elements (head stride >= 128)");
  const uintptr_t any = (uintptr_t)y | (uintptr_t)x | (uintptr_t)k_pool | (uintptr_t)v_pool;
  DSPARK_REQUIRE(any % 16 == 0, "tensors must be 16-byte aligned");
  DraftEpiArgs a{y, static_cast<const bf16*>(x), static_cast<const bf16*>(k_norm), inv_freq,
                 req, static_cast<bf16*>(k_pool), static_cast<bf16*>(v_pool), y_stride, layer_stride, slot_stride,
                 head_stride, flag, tokens, token0, hidden, layers, n_req, eps_ctx, eps_k};
  if (y_dtype)
    hipLaunchKernelGGL(draft_kv_epilogue_kernel<float>, dim3((unsigned)((tokens + 15) / 16)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(draft_kv_epilogue_kernel<bf16>, dim3((unsigned)((tokens + 15) / 16)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
  return launch_status("draft_kv_epilogue_kernel");
}
