/*
 * CPU restatement of the DSpark attention hot path (TEST INFRASTRUCTURE ONLY:
 * used by tests/ to check results and by bench.py as the CPU baseline).
 *
 * Semantics restated from
 *   dspark_qwen/varlen_target.py:98-112        (bottom-right causal oracle)
 *   dspark_qwen/packed_draft.py:35-47          (noncausal oracle)
 *   dspark_qwen/persistent_qwen_target.py:30-42 (capacity-tail causal oracle)
 *   dspark_qwen/persistent_target_kv.py:392-460 (verify keys = committed ++ staged)
 *   dspark_qwen/model.py:12-19                 (draft block mask)
 * Inputs are bf16 bit patterns; arithmetic is FP32 with FP32 exp (expf),
 * an exact softmax per row (max, exp, sum, weighted V sum).
 * Shapes: 16 query heads, 8 KV heads, head dim 128 (GQA group 2).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define HQ 16
#define HKV 8
#define HD 128
#define KV_ROW (HKV * HD)
#define Q_ROW (HQ * HD)

static inline float bf(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* One (request, KV head) group: nrows query rows (pointers to 128 bf16),
 * nk keys (row pointers), per-row visible set [0,hi1[r]) U [lo2[r],hi2[r]). */
static void attend_group(int nrows, const uint16_t* const* qrow, float* const* orow,
                         int nk, const uint16_t* const* krow, const uint16_t* const* vrow,
                         const int* hi1, const int* lo2, const int* hi2, float scale,
                         float* scores /* nrows*nk */, float* qf /* nrows*HD */, float* tmp /* HD */) {
  for (int r = 0; r < nrows; ++r)
    for (int d = 0; d < HD; ++d) qf[r * HD + d] = bf(qrow[r][d]);
  for (int j = 0; j < nk; ++j) {
    for (int d = 0; d < HD; ++d) tmp[d] = bf(krow[j][d]);
    for (int r = 0; r < nrows; ++r) {
      float s = 0.f;
      const float* qq = qf + r * HD;
      for (int d = 0; d < HD; ++d) s += qq[d] * tmp[d];
      const int vis = (j < hi1[r]) || (j >= lo2[r] && j < hi2[r]);
      scores[r * nk + j] = vis ? s * scale : -INFINITY;
    }
  }
  for (int r = 0; r < nrows; ++r) {
    float m = -INFINITY;
    for (int j = 0; j < nk; ++j) m = fmaxf(m, scores[r * nk + j]);
    float sum = 0.f;
    for (int j = 0; j < nk; ++j) {
      const float p = (scores[r * nk + j] == -INFINITY) ? 0.f : expf(scores[r * nk + j] - m);
      scores[r * nk + j] = p;
      sum += p;
    }
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    for (int j = 0; j < nk; ++j) scores[r * nk + j] *= inv;
    for (int d = 0; d < HD; ++d) orow[r][d] = 0.f;
  }
  for (int j = 0; j < nk; ++j) {
    for (int d = 0; d < HD; ++d) tmp[d] = bf(vrow[j][d]);
    for (int r = 0; r < nrows; ++r) {
      const float p = scores[r * nk + j];
      if (p == 0.f) continue;
      float* o = orow[r];
      for (int d = 0; d < HD; ++d) o[d] += p * tmp[d];
    }
  }
}

typedef struct {
  int nk;
  int nrows;
} GroupShape;

static void run_groups(int n_groups, int threads,
                       void (*one)(int group, float* work, size_t work_elems, const void* ctx),
                       size_t work_elems, const void* ctx) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
  {
    float* work = (float*)malloc(work_elems * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (int gi = 0; gi < n_groups; ++gi) one(gi, work, work_elems, ctx);
    free(work);
  }
#else
  (void)threads;
  float* work = (float*)malloc(work_elems * sizeof(float));
  for (int gi = 0; gi < n_groups; ++gi) one(gi, work, work_elems, ctx);
  free(work);
#endif
}

/* ---------------- varlen (packed, exact-K or capacity tail) ---------------- */
typedef struct {
  const uint16_t *q, *k, *v;
  const int32_t *cu_q, *cu_k;
  int causal;
  float scale;
  float* out;
  int max_k, max_q;
} VarlenCtx;

static void varlen_one(int gi, float* work, size_t work_elems, const void* vctx) {
  const VarlenCtx* c = (const VarlenCtx*)vctx;
  (void)work_elems;
  const int r = gi / HKV, g = gi % HKV;
  const int q0 = c->cu_q[r], nq = c->cu_q[r + 1] - q0;
  const int k0 = c->cu_k[r], nk = c->cu_k[r + 1] - k0;
  const int nrows = 2 * nq;
  const uint16_t** qrow = (const uint16_t**)malloc(sizeof(void*) * nrows);
  float** orow = (float**)malloc(sizeof(void*) * nrows);
  const uint16_t** krow = (const uint16_t**)malloc(sizeof(void*) * (nk > 0 ? nk : 1));
  const uint16_t** vrow = (const uint16_t**)malloc(sizeof(void*) * (nk > 0 ? nk : 1));
  int* lim = (int*)malloc(sizeof(int) * 3 * nrows);
  for (int i = 0; i < nq; ++i)
    for (int h = 0; h < 2; ++h) {
      const int row = 2 * i + h;
      qrow[row] = c->q + (size_t)(q0 + i) * Q_ROW + (size_t)(2 * g + h) * HD;
      orow[row] = c->out + (size_t)(q0 + i) * Q_ROW + (size_t)(2 * g + h) * HD;
      lim[row] = c->causal ? nk - nq + i + 1 : nk;
      lim[nrows + row] = 0;
      lim[2 * nrows + row] = 0;
    }
  for (int j = 0; j < nk; ++j) {
    krow[j] = c->k + (size_t)(k0 + j) * KV_ROW + (size_t)g * HD;
    vrow[j] = c->v + (size_t)(k0 + j) * KV_ROW + (size_t)g * HD;
  }
  attend_group(nrows, qrow, orow, nk, krow, vrow, lim, lim + nrows, lim + 2 * nrows, c->scale,
               work, work + (size_t)nrows * nk, work + (size_t)nrows * nk + (size_t)nrows * HD);
  free(qrow); free(orow); free(krow); free(vrow); free(lim);
}

void oracle_varlen_attn(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const int32_t* cu_q, const int32_t* cu_k, int n_req, int causal,
                        float scale, float* out, int threads) {
  VarlenCtx c = {q, k, v, cu_q, cu_k, causal, scale, out, 0, 0};
  for (int r = 0; r < n_req; ++r) {
    const int nk = cu_k[r + 1] - cu_k[r], nq = cu_q[r + 1] - cu_q[r];
    if (nk > c.max_k) c.max_k = nk;
    if (nq > c.max_q) c.max_q = nq;
  }
  const size_t work = (size_t)2 * c.max_q * c.max_k + (size_t)2 * c.max_q * HD + HD;
  run_groups(n_req * HKV, threads, varlen_one, work, &c);
}

/* ---------------- verify (resident ++ scratch) ---------------- */
typedef struct {
  const uint16_t *q, *k_res, *v_res, *k_scr, *v_scr;
  const int32_t *slots, *ctx, *cu_q;
  int64_t cap;
  float scale;
  float* out;
} VerifyCtx;

static void verify_one(int gi, float* work, size_t work_elems, const void* vctx) {
  const VerifyCtx* c = (const VerifyCtx*)vctx;
  (void)work_elems;
  const int r = gi / HKV, g = gi % HKV;
  const int q0 = c->cu_q[r], nq = c->cu_q[r + 1] - q0;
  const int cc = c->ctx[r], nk = cc + nq;
  const int nrows = 2 * nq;
  const uint16_t** qrow = (const uint16_t**)malloc(sizeof(void*) * nrows);
  float** orow = (float**)malloc(sizeof(void*) * nrows);
  const uint16_t** krow = (const uint16_t**)malloc(sizeof(void*) * nk);
  const uint16_t** vrow = (const uint16_t**)malloc(sizeof(void*) * nk);
  int* lim = (int*)malloc(sizeof(int) * 3 * nrows);
  for (int i = 0; i < nq; ++i)
    for (int h = 0; h < 2; ++h) {
      const int row = 2 * i + h;
      qrow[row] = c->q + (size_t)(q0 + i) * Q_ROW + (size_t)(2 * g + h) * HD;
      orow[row] = c->out + (size_t)(q0 + i) * Q_ROW + (size_t)(2 * g + h) * HD;
      lim[row] = cc + i + 1;
      lim[nrows + row] = 0;
      lim[2 * nrows + row] = 0;
    }
  const size_t base = (size_t)c->slots[r] * (size_t)c->cap;
  for (int j = 0; j < cc; ++j) {
    krow[j] = c->k_res + (base + j) * KV_ROW + (size_t)g * HD;
    vrow[j] = c->v_res + (base + j) * KV_ROW + (size_t)g * HD;
  }
  for (int t = 0; t < nq; ++t) {
    krow[cc + t] = c->k_scr + (size_t)(q0 + t) * KV_ROW + (size_t)g * HD;
    vrow[cc + t] = c->v_scr + (size_t)(q0 + t) * KV_ROW + (size_t)g * HD;
  }
  attend_group(nrows, qrow, orow, nk, krow, vrow, lim, lim + nrows, lim + 2 * nrows, c->scale,
               work, work + (size_t)nrows * nk, work + (size_t)nrows * nk + (size_t)nrows * HD);
  free(qrow); free(orow); free(krow); free(vrow); free(lim);
}

void oracle_verify_attn(const uint16_t* q, const uint16_t* k_res, const uint16_t* v_res,
                        const uint16_t* k_scr, const uint16_t* v_scr,
                        const int32_t* slots, const int32_t* ctx, const int32_t* cu_q,
                        int n_req, int64_t ctx_capacity, float scale, float* out, int threads) {
  VerifyCtx c = {q, k_res, v_res, k_scr, v_scr, slots, ctx, cu_q, ctx_capacity, scale, out};
  int max_k = 0, max_q = 0;
  for (int r = 0; r < n_req; ++r) {
    const int nq = cu_q[r + 1] - cu_q[r];
    if (ctx[r] + nq > max_k) max_k = ctx[r] + nq;
    if (nq > max_q) max_q = nq;
  }
  const size_t work = (size_t)2 * max_q * max_k + (size_t)2 * max_q * HD + HD;
  run_groups(n_req * HKV, threads, verify_one, work, &c);
}

/* ---------------- draft (multi-block) ---------------- */
typedef struct {
  const uint16_t *q, *k_ctx, *v_ctx, *k_blk, *v_blk;
  const int64_t* ctx_off;
  const int32_t *ctx_len, *cu_b, *anchors;
  float scale;
  float* out;
} DraftCtx;

#define BLK 7

static void draft_one(int gi, float* work, size_t work_elems, const void* vctx) {
  const DraftCtx* c = (const DraftCtx*)vctx;
  (void)work_elems;
  const int r = gi / HKV, g = gi % HKV;
  const int b0 = c->cu_b[r], nb = c->cu_b[r + 1] - b0;
  const int cc = c->ctx_len[r], nk = cc + BLK * nb;
  const int nrows = 2 * BLK * nb;
  const uint16_t** qrow = (const uint16_t**)malloc(sizeof(void*) * nrows);
  float** orow = (float**)malloc(sizeof(void*) * nrows);
  const uint16_t** krow = (const uint16_t**)malloc(sizeof(void*) * nk);
  const uint16_t** vrow = (const uint16_t**)malloc(sizeof(void*) * nk);
  int* lim = (int*)malloc(sizeof(int) * 3 * nrows);
  for (int b = 0; b < nb; ++b)
    for (int i = 0; i < BLK; ++i)
      for (int h = 0; h < 2; ++h) {
        const int row = 2 * (BLK * b + i) + h;
        const size_t tok = (size_t)BLK * (b0 + b) + i;
        qrow[row] = c->q + tok * Q_ROW + (size_t)(2 * g + h) * HD;
        orow[row] = c->out + tok * Q_ROW + (size_t)(2 * g + h) * HD;
        lim[row] = c->anchors[b0 + b];
        lim[nrows + row] = cc + BLK * b;
        lim[2 * nrows + row] = cc + BLK * (b + 1);
      }
  const size_t base = (size_t)c->ctx_off[r];
  for (int j = 0; j < cc; ++j) {
    krow[j] = c->k_ctx + (base + j) * KV_ROW + (size_t)g * HD;
    vrow[j] = c->v_ctx + (base + j) * KV_ROW + (size_t)g * HD;
  }
  for (int t = 0; t < BLK * nb; ++t) {
    krow[cc + t] = c->k_blk + ((size_t)BLK * b0 + t) * KV_ROW + (size_t)g * HD;
    vrow[cc + t] = c->v_blk + ((size_t)BLK * b0 + t) * KV_ROW + (size_t)g * HD;
  }
  attend_group(nrows, qrow, orow, nk, krow, vrow, lim, lim + nrows, lim + 2 * nrows, c->scale,
               work, work + (size_t)nrows * nk, work + (size_t)nrows * nk + (size_t)nrows * HD);
  free(qrow); free(orow); free(krow); free(vrow); free(lim);
}

void oracle_draft_attn(const uint16_t* q, const uint16_t* k_ctx, const uint16_t* v_ctx,
                       const int64_t* ctx_off, const int32_t* ctx_len,
                       const uint16_t* k_blk, const uint16_t* v_blk,
                       const int32_t* cu_b, const int32_t* anchors, int n_req,
                       float scale, float* out, int threads) {
  DraftCtx c = {q, k_ctx, v_ctx, k_blk, v_blk, ctx_off, ctx_len, cu_b, anchors, scale, out};
  int max_k = 0, max_rows = 0;
  for (int r = 0; r < n_req; ++r) {
    const int nb = cu_b[r + 1] - cu_b[r];
    if (ctx_len[r] + BLK * nb > max_k) max_k = ctx_len[r] + BLK * nb;
    if (2 * BLK * nb > max_rows) max_rows = 2 * BLK * nb;
  }
  const size_t work = (size_t)max_rows * max_k + (size_t)max_rows * HD + HD;
  run_groups(n_req * HKV, threads, draft_one, work, &c);
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
