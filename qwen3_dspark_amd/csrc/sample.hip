// Float64 sampling law and speculative verification on gfx950: the consumer
// of the target's verification output, after the LM head.
//
//   p_j = softmax(logits_j / T) in float64           (tensor_sampling.py:
//                                                     logits_to_probabilities)
//   draft token t_j with law q_j is accepted iff u_j < min(1, p_j[t_j] / q_j[t_j]);
//   the first rejection emits a draw from (p_j - q_j)+ normalised, a fully
//   accepted block a bonus draw from p_n; EOS and the output budget stop early
//                                                    (tensor_sampling.py:
//                                                     verify_proposal)
//   a draw from a law r is the first index whose running sum of r exceeds u
//   (searchsorted(cumsum(r), u, right=True)), else the last index of
//   positive mass                                    (sample_categorical)
//
// The p rows are never materialised for verification: one pass over the
// logits gives each row's max and sum of exp (split over many workgroups),
// and every p value needed later is formed from them on the fly.  The
// uniforms are inputs, consumed in the reference's draw order, so a given
// tape of draws fixes every integer outcome.  All probability arithmetic is
// float64 (the model's logits are bf16 or fp32).
#include <cfloat>

#include "common.h"

namespace dspark {

constexpr int ST_CHUNK = 8192;            // logits per row-statistics workgroup

__device__ __forceinline__ double load_logit(const void* logits, int dtype, int64_t idx) {
  if (dtype == 0) return (double)(float)static_cast<const bf16*>(logits)[idx];
  return (double)static_cast<const float*>(logits)[idx];
}

// ---------------------------------------------------------------------------
// Float64 law arithmetic, shared by every kernel below, so that the row
// statistics and every p value come from the same operations.
//
// LawScale, x / T: for T in [2^-100, 2^100] the quotient q = x * (1/T) gets
// one correction, q + fma(-q, T, x) * (1/T) with fused operations
// (Markstein's correction step), which yields the correctly rounded x / T:
// for finite float or bf16 x (|x| < 2^128) no step overflows or underflows.
// The oracle's tests compare it with true division over every finite bf16
// value at 17 temperatures and over 2e7 random fp32 values and temperatures
// in [2^-50, 2^50].  Other T divide.
//
// law_exp, exp(z) for z <= 0, by Tang's table-driven method: z = k ln2/32 + r
// with k = rint(32 z / ln2), |r| <= ln2/64 (Cody-Waite reduction; ln2/32 =
// L1 + L2 with L1 on 37 bits, so that k L1 is exact for |k| < 2^16);
// exp(r) - 1 by its degree-6 Taylor polynomial (truncation < 4e-18
// relative); exp(z) = 2^(k >> 5) (t_j + (t_j p + l_j)), j = k & 31, where
// 2^(j/32) = t_j + l_j to twice double precision.  Measured error <= 0.56
// ulp over 2e7 arguments in [-746, 0].  z below -746, -inf and NaN give 0
// (a row holding a non-finite logit is flagged by the row statistics).
// ---------------------------------------------------------------------------
__constant__ __attribute__((aligned(16))) double LAW_EXP_TAB[64] = {
    0x1.0000000000000p+0, 0x0.0p+0,
    0x1.059b0d3158574p+0, 0x1.d73e2a475b465p-55,
    0x1.0b5586cf9890fp+0, 0x1.8a62e4adc610bp-54,
    0x1.11301d0125b51p+0, -0x1.6c51039449b3ap-54,
    0x1.172b83c7d517bp+0, -0x1.19041b9d78a76p-55,
    0x1.1d4873168b9aap+0, 0x1.e016e00a2643cp-54,
    0x1.2387a6e756238p+0, 0x1.9b07eb6c70573p-54,
    0x1.29e9df51fdee1p+0, 0x1.612e8afad1255p-55,
    0x1.306fe0a31b715p+0, 0x1.6f46ad23182e4p-55,
    0x1.371a7373aa9cbp+0, -0x1.63aeabf42eae2p-54,
    0x1.3dea64c123422p+0, 0x1.ada0911f09ebcp-55,
    0x1.44e086061892dp+0, 0x1.89b7a04ef80d0p-59,
    0x1.4bfdad5362a27p+0, 0x1.d4397afec42e2p-56,
    0x1.5342b569d4f82p+0, -0x1.07abe1db13cadp-55,
    0x1.5ab07dd485429p+0, 0x1.6324c054647adp-54,
    0x1.6247eb03a5585p+0, -0x1.383c17e40b497p-54,
    0x1.6a09e667f3bcdp+0, -0x1.bdd3413b26456p-54,
    0x1.71f75e8ec5f74p+0, -0x1.16e4786887a99p-55,
    0x1.7a11473eb0187p+0, -0x1.41577ee04992fp-55,
    0x1.82589994cce13p+0, -0x1.d4c1dd41532d8p-54,
    0x1.8ace5422aa0dbp+0, 0x1.6e9f156864b27p-54,
    0x1.93737b0cdc5e5p+0, -0x1.75fc781b57ebcp-57,
    0x1.9c49182a3f090p+0, 0x1.c7c46b071f2bep-56,
    0x1.a5503b23e255dp+0, -0x1.d2f6edb8d41e1p-54,
    0x1.ae89f995ad3adp+0, 0x1.7a1cd345dcc81p-54,
    0x1.b7f76f2fb5e47p+0, -0x1.5584f7e54ac3bp-56,
    0x1.c199bdd85529cp+0, 0x1.11065895048ddp-55,
    0x1.cb720dcef9069p+0, 0x1.503cbd1e949dbp-56,
    0x1.d5818dcfba487p+0, 0x1.2ed02d75b3707p-55,
    0x1.dfc97337b9b5fp+0, -0x1.1a5cd4f184b5cp-54,
    0x1.ea4afa2a490dap+0, -0x1.e9c23179c2893p-54,
    0x1.f50765b6e4540p+0, 0x1.9d3e12dd8a18bp-54};
constexpr double EXP_INV_L = 0x1.71547652b82fep+5;   // 32 / ln2
constexpr double EXP_L1 = 0x1.62e42fefa0000p-6;      // ln2/32, high 37 bits
constexpr double EXP_L2 = 0x1.cf79abc9e3b3ap-45;      // ln2/32 - L1

struct LawScale {
  double T, rT;
  bool fast;
  __device__ __forceinline__ double operator()(double x) const {
    if (!fast) return x / T;
    const double q = __dmul_rn(x, rT);
    return __fma_rn(__fma_rn(-q, T, x), rT, q);
  }
};

inline LawScale law_scale(double T) {
  return LawScale{T, 1.0 / T, T >= 0x1p-100 && T <= 0x1p100};
}

// tab: LAW_EXP_TAB, or a copy of it in LDS (stage_exp_table).
__device__ __forceinline__ double law_exp(double z, const double* tab) {
  z = fmax(z, -746.0);
  const double k = rint(__dmul_rn(z, EXP_INV_L));
  const int n = (int)k;
  const double r = __fma_rn(-k, EXP_L2, __fma_rn(-k, EXP_L1, z));
  double c = __fma_rn(r, 1.0 / 720, 1.0 / 120);
  c = __fma_rn(r, c, 1.0 / 24);
  c = __fma_rn(r, c, 1.0 / 6);
  c = __fma_rn(r, c, 0.5);
  const double p = __fma_rn(__dmul_rn(r, r), c, r);
  const double2 t = *reinterpret_cast<const double2*>(tab + 2 * (n & 31));
  return ldexp(__dadd_rn(t.x, __fma_rn(t.x, p, t.y)), n >> 5);
}

// Copies the table into LDS; the caller's next barrier publishes it.
__device__ __forceinline__ void stage_exp_table(double* lds) {
  if (threadIdx.x < 64) lds[threadIdx.x] = LAW_EXP_TAB[threadIdx.x];
}

// p(v) = exp(x_v / T - M) / S.
__device__ __forceinline__ double law_p(double x, const LawScale& sc, double M, double S, const double* tab) {
  return law_exp(sc(x) - M, tab) / S;
}

// Block-wide sum for 256 threads (4 waves); `buf` holds 4 doubles.
__device__ __forceinline__ double block_sum(double x, double* buf) {
  #pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) buf[wave] = x;
  __syncthreads();
  return buf[0] + buf[1] + buf[2] + buf[3];
}

// ---------------------------------------------------------------------------
// Row statistics: per (row, chunk of ST_CHUNK logits) the max of x/T and the
// sum of exp(x/T - max); a non-finite x or x/T marks the row in `bad`.
// Division by T > 0 is monotone, so the max is taken over the raw logits and
// divided once: max(x/T) == max(x)/T exactly; T == 1 divides nothing
// (x/1 == x).  One pass over the logits: each thread keeps its ST_PER
// values in registers (bf16 and fp32 logits are exact in float) between the
// max and the sum.  A full chunk of a 16-byte aligned row is read with
// 16-byte loads (a wave reads 1 KiB contiguous per load); other chunks with
// element loads.
// ---------------------------------------------------------------------------
constexpr int ST_THREADS = 256;
constexpr int ST_PER = ST_CHUNK / ST_THREADS;   // logits per thread

template <int DT>   // 0: bf16 logits, 1: fp32
__global__ __launch_bounds__(ST_THREADS) void row_stats_kernel(const void* logits, int64_t row_stride, int vocab,
                                                               LawScale sc, int chunks, double* stats,
                                                               int32_t* bad) {
  constexpr int VEC = DT == 0 ? 8 : 4;                 // logits per 16-byte load
  __shared__ double buf[4];
  __shared__ __attribute__((aligned(16))) double tab[64];
  const int row = blockIdx.x / chunks;
  const int c = blockIdx.x - row * chunks;
  const int v0 = c * ST_CHUNK;
  const int v1 = min(v0 + ST_CHUNK, vocab);
  const int64_t base = (int64_t)row * row_stride + v0;
  const int tid = threadIdx.x;
  const bool vec = v1 - v0 == ST_CHUNK && ((base * (DT == 0 ? 2 : 4)) & 15) == 0 &&
                   ((uintptr_t)logits & 15) == 0;        // uniform over the workgroup
  stage_exp_table(tab);
  // Values this thread does not hold are -inf: they leave the max alone and
  // add exp(-inf) = 0 to the sum.
  float xs[ST_PER];
  bool nonfinite = false;
  if (vec) {
    // value i of this thread: element VEC * (tid + ST_THREADS * (i / VEC)) + i % VEC
    #pragma unroll
    for (int j = 0; j < ST_PER / VEC; ++j) {
      const int64_t e = base + (int64_t)VEC * (tid + ST_THREADS * j);
      if (DT == 0) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(logits) + e);
        #pragma unroll
        for (int u = 0; u < VEC; ++u) xs[VEC * j + u] = (float)v[u];
      } else {
        const f32x4 v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(logits) + e);
        #pragma unroll
        for (int u = 0; u < VEC; ++u) xs[VEC * j + u] = v[u];
      }
    }
    #pragma unroll
    for (int i = 0; i < ST_PER; ++i) nonfinite |= !isfinite(xs[i]);
  } else {
    // value i of this thread: element tid + ST_THREADS * i (when below v1)
    #pragma unroll
    for (int i = 0; i < ST_PER; ++i) {
      const int v = v0 + tid + ST_THREADS * i;
      const bool held = v < v1;
      xs[i] = held ? (float)load_logit(logits, DT, (int64_t)row * row_stride + v) : -INFINITY;
      nonfinite |= held && !isfinite(xs[i]);
    }
  }
  float xmax = -INFINITY;
  #pragma unroll
  for (int i = 0; i < ST_PER; ++i) xmax = fmaxf(xmax, xs[i]);
  #pragma unroll
  for (int off = 32; off >= 1; off >>= 1) xmax = fmaxf(xmax, __shfl_xor(xmax, off));
  const int wave = tid >> 6;
  if ((tid & 63) == 0) buf[wave] = xmax;
  __syncthreads();   // also publishes the exp table
  const double m = sc((double)fmaxf(fmaxf(buf[0], buf[1]), fmaxf(buf[2], buf[3])));
  double sum = 0.0;
  if (sc.fast) {
    // finite x / T stays finite: only the logits need the check
    #pragma unroll
    for (int i = 0; i < ST_PER; ++i) sum += law_exp(sc((double)xs[i]) - m, tab);
  } else {
    #pragma unroll
    for (int i = 0; i < ST_PER; ++i) {
      const double y = (double)xs[i] / sc.T;
      nonfinite |= (vec || v0 + tid + ST_THREADS * i < v1) && !isfinite(y);
      sum += law_exp(y - m, tab);
    }
  }
  sum = block_sum(sum, buf);
  if (tid == 0) {
    stats[2 * ((int64_t)row * chunks + c)] = m;
    stats[2 * ((int64_t)row * chunks + c) + 1] = sum;
  }
  if (__builtin_amdgcn_ballot_w64(nonfinite) && (tid & 63) == 0 && bad) bad[row] = 1;   // vector store
}

// Combined (max, sum) of one row from its chunk statistics.
__device__ __forceinline__ void row_law(const double* stats, int row, int chunks, double& M, double& S) {
  const double* st = stats + 2 * (int64_t)row * chunks;
  M = -INFINITY;
  for (int c = 0; c < chunks; ++c) M = fmax(M, st[2 * c]);
  S = 0.0;
  for (int c = 0; c < chunks; ++c) S += st[2 * c + 1] * law_exp(st[2 * c] - M, LAW_EXP_TAB);
}

// ---------------------------------------------------------------------------
// Categorical draws.  A draw job names one law over the vocabulary:
//   LAW      p(v) = exp(x_v / T - M) / S of one logit row,
//   RESIDUAL (p(v) - q(v))+ of one logit row and one draft law row,
//            normalised by its sum,
//   PROBS    a materialised float64 law row,
// and a uniform u.  The draw is the first index whose running sum exceeds u,
// else the last index of positive mass.  The vocabulary is cut into 256
// consecutive segments: a wide launch sums every segment of every job with
// coalesced loads (SEG_SLICES workgroups per job), then one workgroup per
// job scans its segment sums in order and one wave walks the segment where
// the running sum passes u with a wave-level inclusive scan.  The sums are
// float64 in another association than a sequential cumulative sum: only a u
// within about an ulp of a boundary can land on the neighbouring index.
// ---------------------------------------------------------------------------
constexpr int NSEG = 256;                 // segments per job
constexpr int SEG_SLICES = 32;            // segment-sum workgroups per job
constexpr int SEG_PER_SLICE = NSEG / SEG_SLICES;
static_assert(SEG_PER_SLICE % 4 == 0, "each wave sums the same number of segments");

enum DrawKind { DK_NONE = 0, DK_LAW = 1, DK_RESIDUAL = 2, DK_PROBS = 3 };

struct DrawJob {
  int64_t src;        // element offset of the logit or probability row
  int64_t qrow;       // element offset of the draft law row (RESIDUAL)
  int64_t out;        // where the drawn token goes
  double M, S, u;     // row max / sum of the logit row, the uniform
  int32_t kind;
  int32_t req;        // verification request (-1: a plain row draw)
  int64_t pad;
};
static_assert(sizeof(DrawJob) == 64, "draw job layout");

struct DrawSrc {
  const void* logits;
  int dtype;
  LawScale sc;
  const double* q;
  const double* probs;
  int vocab;
};

__device__ __forceinline__ double draw_value(const DrawSrc& s, const DrawJob& j, int v, const double* tab) {
  if (j.kind == DK_PROBS) return s.probs[j.src + v];
  const double p = law_p(load_logit(s.logits, s.dtype, j.src + v), s.sc, j.M, j.S, tab);
  return j.kind == DK_RESIDUAL ? fmax(p - s.q[j.qrow + v], 0.0) : p;
}

__device__ __forceinline__ void segment_bounds(int seg, int vocab, int& s0, int& s1) {
  const int per = (vocab + NSEG - 1) / NSEG;
  s0 = min(seg * per, vocab);
  s1 = min(s0 + per, vocab);
}

// This lane's share of one segment's sum and last index of positive mass:
// values v = s0 + lane + 64 i in increasing order (the order of a plain
// strided loop), their loads issued SEG_BATCH strips at a time (indices
// clamped into the segment, values past it dropped) so that a wave waits
// for one round trip per batch instead of one per strip.
constexpr int SEG_BATCH = 8;

template <int KIND, int DT>
__device__ __forceinline__ void segment_part(const DrawSrc& src, const DrawJob& j, int s0, int s1, int lane,
                                             const double* tab, double& part, int& last) {
  for (int v0 = s0 + lane; v0 < s1; v0 += WAVE * SEG_BATCH) {
    double x[SEG_BATCH], qv[SEG_BATCH];
    #pragma unroll
    for (int u = 0; u < SEG_BATCH; ++u) {
      const int v = min(v0 + WAVE * u, s1 - 1);
      if (KIND == DK_PROBS) x[u] = src.probs[j.src + v];
      else x[u] = DT == 0 ? (double)(float)static_cast<const bf16*>(src.logits)[j.src + v]
                          : (double)static_cast<const float*>(src.logits)[j.src + v];
      if (KIND == DK_RESIDUAL) qv[u] = src.q[j.qrow + v];
    }
    #pragma unroll
    for (int u = 0; u < SEG_BATCH; ++u) {
      const int v = v0 + WAVE * u;
      double r = KIND == DK_PROBS ? x[u] : law_p(x[u], src.sc, j.M, j.S, tab);
      if (KIND == DK_RESIDUAL) r = fmax(r - qv[u], 0.0);
      if (v < s1) {
        part += r;
        if (r > 0.0) last = v;
      }
    }
  }
}

// grid: jobs x SEG_SLICES; each wave sums SEG_PER_SLICE / 4 segments.
__global__ __launch_bounds__(256) void segment_sums_kernel(DrawSrc src, const DrawJob* jobs, double* segsum,
                                                           int32_t* seglast) {
  __shared__ __attribute__((aligned(16))) double tab[64];
  const int job = blockIdx.x / SEG_SLICES;
  const int slice = blockIdx.x - job * SEG_SLICES;
  const DrawJob j = jobs[job];
  if (j.kind == DK_NONE) return;                    // uniform across the workgroup
  stage_exp_table(tab);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int i = 0; i < SEG_PER_SLICE / 4; ++i) {
    const int seg = slice * SEG_PER_SLICE + wave * (SEG_PER_SLICE / 4) + i;
    int s0, s1;
    segment_bounds(seg, src.vocab, s0, s1);
    double part = 0.0;
    int last = -1;
    if (j.kind == DK_PROBS)
      segment_part<DK_PROBS, 0>(src, j, s0, s1, lane, tab, part, last);
    else if (src.dtype == 0)
      j.kind == DK_LAW ? segment_part<DK_LAW, 0>(src, j, s0, s1, lane, tab, part, last)
                       : segment_part<DK_RESIDUAL, 0>(src, j, s0, s1, lane, tab, part, last);
    else
      j.kind == DK_LAW ? segment_part<DK_LAW, 1>(src, j, s0, s1, lane, tab, part, last)
                       : segment_part<DK_RESIDUAL, 1>(src, j, s0, s1, lane, tab, part, last);
    #pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      part += __shfl_xor(part, off);
      last = max(last, __shfl_xor(last, off));
    }
    if (lane == 0) {
      segsum[(int64_t)job * NSEG + seg] = part;
      seglast[(int64_t)job * NSEG + seg] = last;
    }
  }
}

__device__ __forceinline__ double wave_inclusive_scan(double x, int lane) {
  #pragma unroll
  for (int off = 1; off < WAVE; off <<= 1) {
    const double y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  return x;
}

struct DrawOut {
  int64_t* tokens;          // drawn token of job j goes to tokens[jobs[j].out]
  int32_t* meta;            // verification requests: [n_req][8] (see the C ABI)
  const int32_t* budget;
  const int32_t* stops;
  int n_stops;
};

enum VerifyError { VE_OK = 0, VE_TOKEN = 1, VE_ZERO_Q = 2, VE_LOGITS = 3, VE_RESIDUAL = 4, VE_UNIFORM = 5, VE_SHAPE = 6 };
enum Extra { EX_NONE = 0, EX_RESIDUAL = 1, EX_BONUS = 2 };
enum Stop { ST_ROUND = 0, ST_EOS = 1, ST_BUDGET = 2 };

__device__ __forceinline__ bool is_stop(const int32_t* stops, int n_stops, int64_t tok) {
  for (int i = 0; i < n_stops; ++i)
    if (stops[i] == tok) return true;
  return false;
}

// grid: jobs; 256 threads (thread t owns segment t).
__global__ __launch_bounds__(256) void draw_kernel(DrawSrc src, const DrawJob* jobs, const double* segsum,
                                                   const int32_t* seglast, DrawOut o) {
  __shared__ double scan[NSEG];
  __shared__ double buf[4];
  __shared__ int found[2];
  const DrawJob j = jobs[blockIdx.x];
  if (j.kind == DK_NONE) return;                    // uniform across the workgroup
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const double part = segsum[(int64_t)blockIdx.x * NSEG + t];
  int last = seglast[(int64_t)blockIdx.x * NSEG + t];
  #pragma unroll
  for (int off = 32; off >= 1; off >>= 1) last = max(last, __shfl_xor(last, off));
  double norm = 1.0;
  if (j.kind == DK_RESIDUAL) {
    norm = block_sum(part, buf);
    if (!(norm > 0.0)) {
      if (t == 0 && j.req >= 0) o.meta[8 * j.req + 6] = VE_RESIDUAL;
      return;
    }
  }
  if (t == 0) {
    found[0] = INT32_MAX;
    found[1] = -1;
  }
  scan[t] = part / norm;
  __syncthreads();
  if (lane == 0) atomicMax(&found[1], last);
  for (int off = 1; off < NSEG; off <<= 1) {         // inclusive scan in segment order
    const double add = t >= off ? scan[t - off] : 0.0;
    __syncthreads();
    scan[t] += add;
    __syncthreads();
  }
  const double before = t ? scan[t - 1] : 0.0;
  if (before <= j.u && j.u < scan[t]) found[0] = -2 - t;   // at most one segment: the scan never falls
  __syncthreads();
  const int mark = found[0];
  __syncthreads();
  if (mark <= -2) {
    if (wave == 0) {
      const int seg = -2 - mark;
      int s0, s1;
      segment_bounds(seg, src.vocab, s0, s1);
      double run = seg ? scan[seg - 1] : 0.0;
      int hit = INT32_MAX, pos = -1;
      for (int v0 = s0; v0 < s1 && hit == INT32_MAX; v0 += WAVE) {
        const int v = v0 + lane;
        const double r = v < s1 ? draw_value(src, j, v, LAW_EXP_TAB) / norm : 0.0;
        if (r > 0.0) pos = v;
        const double incl = run + wave_inclusive_scan(r, lane);
        const unsigned long long over = __builtin_amdgcn_ballot_w64(v < s1 && incl > j.u);
        if (over) hit = v0 + __builtin_ctzll(over);
        run = __shfl(incl, WAVE - 1);
      }
      // no crossing reproduced: the segment's last index of positive mass
      #pragma unroll
      for (int off = 32; off >= 1; off >>= 1) pos = max(pos, __shfl_xor(pos, off));
      if (lane == 0) found[0] = hit != INT32_MAX ? hit : pos;
    }
  } else if (t == 0) {
    found[0] = found[1];                             // u at or beyond the total mass
  }
  __syncthreads();
  if (t == 0) {
    const int tok = found[0];
    if (j.req < 0) {
      o.tokens[j.out] = tok;
    } else {
      int32_t* meta = o.meta + 8 * j.req;
      const int emitted = meta[0];
      o.tokens[j.out + emitted] = tok;
      meta[0] = emitted + 1;
      meta[4] = is_stop(o.stops, o.n_stops, tok) ? ST_EOS : (emitted + 1 == o.budget[j.req] ? ST_BUDGET : ST_ROUND);
    }
  }
}

// ---------------------------------------------------------------------------
// Speculative verification decisions: one wave per request (verify_proposal's
// loop); the final draw, if any, becomes a draw job for the two launches
// above.
// ---------------------------------------------------------------------------
struct VerifyArgs {
  const void* logits;        // [rows, >= vocab], row_stride apart; request r owns rows cu_rows[r] .. cu_rows[r+1]
  int dtype;                 // 0 bf16, 1 fp32
  int64_t row_stride;
  int vocab;
  LawScale sc;               // division by the temperature
  const double* stats;       // row statistics, `chunks` (max, sum) pairs per row
  int chunks;
  const int32_t* bad;        // [rows] non-finite flags
  const int32_t* cu_rows;    // [n_req + 1]
  const int64_t* tokens;     // [rows - n_req] draft tokens; request r's at cu_rows[r] - r
  const double* q;           // [rows - n_req, vocab] draft laws, same order
  const double* uniforms;    // [rows]: request r draws from uniforms[cu_rows[r] ..]
  const int32_t* budget;     // [n_req] remaining output budget
  const int32_t* stops;      // [n_stops] EOS ids
  int n_stops;
  int n_req;
  int64_t* out_tokens;       // [rows]: request r writes up to n_r + 1 tokens at cu_rows[r]
  int32_t* out_meta;         // [n_req][8]: emitted, accepted, rejected index, extra, stop, draws, error, 0
  DrawJob* jobs;             // [n_req]
};

constexpr int MAX_PROPOSAL = 255;          // draft tokens per request in one verification

// One wave per request: the lanes form every row's (max, sum) and every
// proposed token's acceptance ratio min(1, p/q) in parallel, then lane 0
// walks the proposal in order.
__global__ __launch_bounds__(64) void verify_plan_kernel(VerifyArgs a) {
  __shared__ double alpha[MAX_PROPOSAL];
  __shared__ double law[2 * (MAX_PROPOSAL + 1)];
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  const int row0 = a.cu_rows[r];
  const int n = a.cu_rows[r + 1] - row0 - 1;
  const int d0 = row0 - r;
  const int V = a.vocab;
  if (n < 0 || n > MAX_PROPOSAL) {                       // wave-uniform; nothing else is read
    if (lane == 0) {
      DrawJob job{};
      job.kind = DK_NONE;
      job.req = r;
      a.jobs[r] = job;
      int32_t* meta = a.out_meta + 8 * r;
      for (int i = 0; i < 8; ++i) meta[i] = 0;
      meta[6] = VE_SHAPE;
    }
    return;
  }
  int err = VE_OK;
  for (int j = lane; j <= n; j += WAVE) {
    if (a.bad[row0 + j]) err = max(err, 3 * 16);            // ordered: logits, then token range, then zero q
    if (j < n) {
      const int64_t tok = a.tokens[d0 + j];
      if (tok < 0 || tok >= V) err = max(err, 2 * 16);
    }
  }
  #pragma unroll
  for (int off = 32; off >= 1; off >>= 1) err = max(err, __shfl_xor(err, off));
  if (err == 0) {
    for (int j = lane; j < n; j += WAVE)
      if (!(a.q[(int64_t)(d0 + j) * V + a.tokens[d0 + j]] > 0.0)) err = 1 * 16;
    #pragma unroll
    for (int off = 32; off >= 1; off >>= 1) err = max(err, __shfl_xor(err, off));
  }
  err = err == 3 * 16 ? VE_LOGITS : (err == 2 * 16 ? VE_TOKEN : (err == 1 * 16 ? VE_ZERO_Q : VE_OK));
  if (err == VE_OK) {
    for (int j = lane; j <= n; j += WAVE) {
      double M, S;
      row_law(a.stats, row0 + j, a.chunks, M, S);
      law[2 * j] = M;
      law[2 * j + 1] = S;
      if (j < n) {
        const int64_t tok = a.tokens[d0 + j];
        const double p = law_p(load_logit(a.logits, a.dtype, (int64_t)(row0 + j) * a.row_stride + tok), a.sc, M, S,
                               LAW_EXP_TAB);
        alpha[j] = fmin(p / a.q[(int64_t)(d0 + j) * V + tok], 1.0);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (lane != 0) return;
  int emitted = 0, accepted = 0, rejected = -1, extra = EX_NONE, stop = ST_ROUND, draws = 0, final_row = -1;
  if (err == VE_OK && a.budget[r] == 0) {
    stop = ST_BUDGET;
  } else if (err == VE_OK) {
    bool done = false;
    for (int j = 0; j < n && !done; ++j) {
      const double u = a.uniforms[row0 + draws++];
      if (!(u >= 0.0 && u < 1.0)) {
        err = VE_UNIFORM;
        break;
      }
      if (u >= alpha[j]) {
        rejected = j;
        accepted = j;
        extra = EX_RESIDUAL;
        final_row = j;
        done = true;
        break;
      }
      const int64_t tok = a.tokens[d0 + j];
      a.out_tokens[row0 + emitted++] = tok;
      accepted = j + 1;
      if (is_stop(a.stops, a.n_stops, tok)) {
        stop = ST_EOS;
        done = true;
      } else if (emitted == a.budget[r]) {
        stop = ST_BUDGET;
        done = true;
      }
    }
    if (!done && err == VE_OK) {
      extra = EX_BONUS;
      final_row = n;
      accepted = n;
    }
  }
  DrawJob job{};
  job.kind = DK_NONE;
  job.req = r;
  job.out = row0;
  if (err == VE_OK && final_row >= 0) {
    const double u = a.uniforms[row0 + draws++];
    if (!(u >= 0.0 && u < 1.0)) {
      err = VE_UNIFORM;
    } else {
      job.M = law[2 * final_row];
      job.S = law[2 * final_row + 1];
      job.u = u;
      job.src = (int64_t)(row0 + final_row) * a.row_stride;
      job.qrow = (int64_t)(d0 + final_row) * V;
      job.kind = extra == EX_BONUS ? DK_LAW : DK_RESIDUAL;
    }
  }
  a.jobs[r] = job;
  int32_t* meta = a.out_meta + 8 * r;
  meta[0] = emitted;
  meta[1] = accepted;
  meta[2] = rejected;
  meta[3] = extra;
  meta[4] = stop;
  meta[5] = draws;
  meta[6] = err;
  meta[7] = 0;
}

// ---------------------------------------------------------------------------
// Materialised laws and plain categorical draws (the draft's proposal side).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void probs_kernel(const void* logits, int dtype, int64_t row_stride, int vocab,
                                                    LawScale sc, const double* stats, int chunks, double* probs) {
  __shared__ __attribute__((aligned(16))) double tab[64];
  stage_exp_table(tab);
  __syncthreads();
  const int row = blockIdx.y;
  double M, S;
  row_law(stats, row, chunks, M, S);
  const int64_t base = (int64_t)row * row_stride;
  for (int v = blockIdx.x * blockDim.x + threadIdx.x; v < vocab; v += gridDim.x * blockDim.x)
    probs[(int64_t)row * vocab + v] = law_p(load_logit(logits, dtype, base + v), sc, M, S, tab);
}

__global__ __launch_bounds__(256) void row_jobs_kernel(int rows, int vocab, const double* uniforms, DrawJob* jobs) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  DrawJob j{};
  j.src = (int64_t)row * vocab;
  j.out = row;
  j.u = uniforms[row];
  j.kind = DK_PROBS;
  j.req = -1;
  jobs[row] = j;
}

}  // namespace dspark

using namespace dspark;

namespace {
int stat_chunks(int vocab) { return (vocab + ST_CHUNK - 1) / ST_CHUNK; }
}

extern "C" int64_t dspark_row_stats_bytes(int rows, int vocab) {
  if (rows < 1 || vocab < 1) return -1;
  return (int64_t)rows * stat_chunks(vocab) * 2 * (int64_t)sizeof(double);
}

extern "C" int dspark_logit_row_stats(const void* logits, int dtype, int rows, int vocab, int64_t row_stride,
                                      double temperature, double* stats, int32_t* bad, void* stream) {
  clear_error();
  DSPARK_REQUIRE(logits && stats && bad, "null pointer argument");
  DSPARK_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (bf16) or 1 (fp32)");
  DSPARK_REQUIRE(rows >= 1 && vocab >= 1 && row_stride >= vocab, "need rows, vocab >= 1 and row_stride >= vocab");
  DSPARK_REQUIRE(temperature > 0.0 && temperature < DBL_MAX, "temperature must be finite and positive");
  const int64_t grid = (int64_t)rows * stat_chunks(vocab);
  DSPARK_REQUIRE(grid <= 0x7fffffffLL, "too many rows");
  if (dtype == 0)
    hipLaunchKernelGGL(row_stats_kernel<0>, dim3((unsigned)grid), dim3(ST_THREADS), 0, static_cast<hipStream_t>(stream),
                       logits, row_stride, vocab, law_scale(temperature), stat_chunks(vocab), stats, bad);
  else
    hipLaunchKernelGGL(row_stats_kernel<1>, dim3((unsigned)grid), dim3(ST_THREADS), 0, static_cast<hipStream_t>(stream),
                       logits, row_stride, vocab, law_scale(temperature), stat_chunks(vocab), stats, bad);
  return launch_status("row_stats_kernel");
}

namespace {
// [jobs: DrawJob][segment sums: double x 256][segment last indices: int32 x 256] per job
int64_t draw_workspace(int jobs) { return (int64_t)jobs * ((int64_t)sizeof(DrawJob) + NSEG * 12); }

int launch_draws(const DrawSrc& src, DrawJob* jobs, int n_jobs, const DrawOut& o, hipStream_t s) {
  double* segsum = reinterpret_cast<double*>(jobs + n_jobs);
  int32_t* seglast = reinterpret_cast<int32_t*>(segsum + (int64_t)n_jobs * NSEG);
  hipLaunchKernelGGL(segment_sums_kernel, dim3((unsigned)((int64_t)n_jobs * SEG_SLICES)), dim3(256), 0, s, src, jobs,
                     segsum, seglast);
  int rc = launch_status("segment_sums_kernel");
  if (rc != OK) return rc;
  hipLaunchKernelGGL(draw_kernel, dim3(n_jobs), dim3(256), 0, s, src, jobs, segsum, seglast, o);
  return launch_status("draw_kernel");
}
}  // namespace

extern "C" int64_t dspark_draw_workspace_bytes(int jobs) {
  if (jobs < 1) return -1;
  return draw_workspace(jobs);
}

extern "C" int dspark_spec_verify(const void* logits, int dtype, int64_t row_stride, int vocab, double temperature,
                                  const double* stats, const int32_t* bad, const int32_t* cu_rows, int n_req,
                                  const int64_t* tokens, const double* q, const double* uniforms,
                                  const int32_t* budget, const int32_t* stops, int n_stops, int64_t* out_tokens,
                                  int32_t* out_meta, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  DSPARK_REQUIRE(logits && stats && bad && cu_rows && tokens && q && uniforms && budget && out_tokens && out_meta &&
                     workspace,
                 "null pointer argument");
  DSPARK_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (bf16) or 1 (fp32)");
  DSPARK_REQUIRE(vocab >= 1 && row_stride >= vocab && n_req >= 1 && n_req <= (1 << 24),
                 "need vocab >= 1, row_stride >= vocab, n_req in [1, 2^24]");
  DSPARK_REQUIRE(temperature > 0.0 && temperature < DBL_MAX, "temperature must be finite and positive");
  DSPARK_REQUIRE(n_stops >= 0 && (n_stops == 0 || stops), "stops must be given when n_stops > 0");
  DSPARK_REQUIRE(workspace_bytes >= draw_workspace(n_req) && (reinterpret_cast<uintptr_t>(workspace) & 63) == 0,
                 "workspace must be 64-byte aligned and hold dspark_draw_workspace_bytes(n_req) bytes");
  DrawJob* jobs = static_cast<DrawJob*>(workspace);
  VerifyArgs a{logits, dtype, row_stride, vocab, law_scale(temperature), stats, stat_chunks(vocab), bad, cu_rows, tokens, q,
               uniforms, budget, stops, n_stops, n_req, out_tokens, out_meta, jobs};
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(verify_plan_kernel, dim3(n_req), dim3(64), 0, s, a);
  int rc = launch_status("verify_plan_kernel");
  if (rc != OK) return rc;
  const DrawSrc src{logits, dtype, law_scale(temperature), q, nullptr, vocab};
  const DrawOut o{out_tokens, out_meta, budget, stops, n_stops};
  return launch_draws(src, jobs, n_req, o, s);
}

extern "C" int dspark_logits_to_probs(const void* logits, int dtype, int rows, int vocab, int64_t row_stride,
                                      double temperature, const double* stats, double* probs, void* stream) {
  clear_error();
  DSPARK_REQUIRE(logits && stats && probs, "null pointer argument");
  DSPARK_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (bf16) or 1 (fp32)");
  DSPARK_REQUIRE(rows >= 1 && rows <= 65535 && vocab >= 1 && row_stride >= vocab,
                 "need rows in [1, 65535], vocab >= 1 and row_stride >= vocab");
  DSPARK_REQUIRE(temperature > 0.0 && temperature < DBL_MAX, "temperature must be finite and positive");
  const unsigned gx = (unsigned)std::min<int64_t>((vocab + 255) / 256, 64);
  hipLaunchKernelGGL(probs_kernel, dim3(gx, rows), dim3(256), 0, static_cast<hipStream_t>(stream), logits, dtype,
                     row_stride, vocab, law_scale(temperature), stats, stat_chunks(vocab), probs);
  return launch_status("probs_kernel");
}

extern "C" int dspark_sample_rows(const double* probs, int rows, int vocab, const double* uniforms, int64_t* out,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  DSPARK_REQUIRE(probs && uniforms && out && workspace, "null pointer argument");
  DSPARK_REQUIRE(rows >= 1 && rows <= (1 << 24) && vocab >= 1, "need rows in [1, 2^24] and vocab >= 1");
  DSPARK_REQUIRE(workspace_bytes >= draw_workspace(rows) && (reinterpret_cast<uintptr_t>(workspace) & 63) == 0,
                 "workspace must be 64-byte aligned and hold dspark_draw_workspace_bytes(rows) bytes");
  DrawJob* jobs = static_cast<DrawJob*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(row_jobs_kernel, dim3((rows + 255) / 256), dim3(256), 0, s, rows, vocab, uniforms, jobs);
  int rc = launch_status("row_jobs_kernel");
  if (rc != OK) return rc;
  const DrawSrc src{nullptr, 0, law_scale(1.0), nullptr, probs, vocab};
  const DrawOut o{out, nullptr, nullptr, nullptr, 0};
  return launch_draws(src, jobs, rows, o, s);
}
