// DSpark attention kernels for gfx950 (MI355X).
//
// Three entry points (varlen and verify share one MFMA inner loop; draft has
// its own 32-row core, described with its section):
//   * varlen    - packed THD attention over cu_seqlens (exact-K or
//                 capacity-tail K/V), bottom-right causal or noncausal.
//                 Replaces aten::_flash_attention_forward as called by
//                 dspark_qwen/rocm_varlen.py:111-114 (causal),
//                 dspark_qwen/packed_draft.py:26-29 (noncausal) and
//                 dspark_qwen/persistent_qwen_target.py:231-234 (capacity).
//   * verify    - the same causal attention, but K/V are read straight from
//                 the persistent resident store (committed context) and the
//                 per-layer scratch (new rows), i.e. the gather of
//                 dspark_qwen/persistent_target_kv.py:441-460 is fused into
//                 the load path and never materialised.
//   * draft     - multi-block DSpark draft attention: each 7-row block sees
//                 context positions j < anchor plus its own 7 rows
//                 (dspark_qwen/model.py:12-19); context is streamed once per
//                 request for all of its blocks.
//
// varlen / verify MFMA mapping (v_mfma_f32_16x16x32_bf16, wave64):
//   S^T[key][row] = K[key][:] . Q[row][:]   A = K (16 keys, via LDS), B = Q^T
//   O^T[d][row]  += V^T[d][key] P^T[key][row]  A = V^T (via LDS), B = P^T
// A 16-row tile holds 8 query tokens x the 2 query heads of one KV head
// (row = 2*token + head_in_group).  The S^T accumulator leaves every lane
// with the 8 scores of ONE query row (keys 8*grp .. 8*grp+7 of a 32-key
// tile), which is exactly the B operand layout the PV MFMA needs, and the
// O^T accumulator again leaves every lane with values of its own row, so
// the online softmax (FlashAttention-2, Dao 2023) needs only two cross-lane
// shuffles per tile for the row maximum.  The reduction order inside an MFMA
// is irrelevant as long as A and B use the same (lane group, slot) -> k
// assignment, which both operands here do by construction.
//
// Long contexts are split into key segments (flash-decoding, Dao et al.
// 2023).  With a host-built segment list every workgroup (run, KV head)
// streams the segments of its run: a balanced list gives every run the same
// number of keys, cutting requests where runs meet (stream-K style), so the
// grid drains evenly whatever the mix of context lengths.  A request held by
// more than one segment writes FP32 partial (max, sum, unnormalised O)
// triples that merge_kernel combines; the kernel boundary makes them visible
// without any per-workgroup cache flush.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace dspark {

constexpr int KT = 32;                 // keys per wave iteration
constexpr int WORK_INTS = 8;           // int32 per work record
constexpr int REQ_INTS = 4;            // int32 per request record (merge)
constexpr int ROWB = HD * 2;           // bytes per LDS K/V row (256)
constexpr int OPITCH = HD + 4;         // floats per row in the merge buffer

// XOR swizzle of the 16-byte chunk index of LDS row k (rows are 256 B,
// i.e. 16 chunks spanning all banks).  Conflict-free for the access
// patterns on a K/V tile:
//  - row writes (registers or direct loads): 16 lanes write the 16 chunks
//    of one row, any per-row XOR keeps them distinct;
//  - transpose reads (V^T): a 16-lane group reads 4 rows r (r<4) with the
//    same k>>3, chunks 2c and 2c+1; swz = 4r + ((k>>3)&3) moves the 4 rows
//    to distinct chunk pairs;
//  - K fragment reads (draft, from LDS): 16 lanes read rows 8q+4j+e (q<4,
//    e<4), one chunk; (k&3, (k>>3)&3) takes all 16 values.
__device__ __forceinline__ int swz(int k) {
  return ((k & 3) << 2) | ((k >> 3) & 3);
}

__device__ __forceinline__ int lds_chunk_off(int k, int chunk16) {
  return k * ROWB + ((chunk16 ^ swz(k)) << 4);
}

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// V^T A-operand for dims 16*nb .. 16*nb+15 from an LDS tile whose row k holds
// key k: lane (j, grp) receives V[8*grp + s][16*nb + j] for s = 0..7, via two
// transpose reads (ds_read_b64_tr_b16: within each 16-lane group, lane
// 4*r+c supplies row r, dims 4c..4c+3 of a 4x16 tile; lane j receives
// column j of the 4 rows).
__device__ __forceinline__ bf16x8 lds_vt(const unsigned char* tile, int nb, int lane) {
  const int grp = lane >> 4;
  const int r = (lane >> 2) & 3;
  const int c4 = lane & 3;
  const int chunk = 2 * nb + (c4 >> 1);
  const int k0 = 8 * grp + r;
  const int k1 = k0 + 4;
  const unsigned char* p0 = tile + k0 * ROWB + ((chunk ^ swz(k0)) << 4) + ((c4 & 1) << 3);
  const unsigned char* p1 = tile + k1 * ROWB + ((chunk ^ swz(k1)) << 4) + ((c4 & 1) << 3);
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p0);
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p1);
  bf16x8 v;
  #pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = lo[i];
    v[4 + i] = hi[i];
  }
  return v;
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One online-softmax + PV update for a 32-key tile.
//   s0/s1  : S^T accumulators (keys kbase+4j+e for j=0/1, e=0..3)
//   vis    : keys < vis are visible for this lane's row
//   vt     : V^T A-operands for the 8 dim blocks
struct RowState {
  float m;       // running max (log2 domain, already scaled)
  float l;       // per-lane partial denominator
  f32x4 o[8];    // O^T accumulators: o[nb][e] = O[row][16nb+4grp+e]
};

__device__ __forceinline__ void row_init(RowState& st) {
  st.m = -INFINITY;
  st.l = 0.f;
  #pragma unroll
  for (int nb = 0; nb < 8; ++nb) st.o[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// The running maximum only moves up when a tile's maximum exceeds it by more
// than RESCALE_SLACK (log2 units), so O and l are rescaled rarely (once per
// row for typical score distributions) instead of every tile.  Exact for
// any reference value: O and l always share the same reference max, which
// the split-K merges carry along; probabilities stay <= 2^RESCALE_SLACK,
// far from FP32/bf16 overflow.  The rescale branch is wave-uniform.
constexpr float RESCALE_SLACK = 8.0f;

template <bool MASKED>
__device__ __forceinline__ bf16x8 softmax_update(RowState& st, const f32x4& s0, const f32x4& s1,
                                                 int kbase, int vis, float scale_log2) {
  float x[8];
  #pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = s0[e] * scale_log2;
    x[4 + e] = s1[e] * scale_log2;
    if (MASKED) {
      if (kbase + e >= vis) x[e] = -INFINITY;
      if (kbase + 4 + e >= vis) x[4 + e] = -INFINITY;
    }
  }
  float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
  mx = wave_max_across_groups(mx);
  const bool raise = mx > st.m + RESCALE_SLACK;
  if (__builtin_amdgcn_ballot_w64(raise)) {
    // Rows that do not raise keep factor 1 (their max may still be -inf,
    // and -inf - -inf must not reach exp2).
    const float alpha = raise ? fast_exp2(st.m - mx) : 1.0f;
    st.l *= alpha;
    #pragma unroll
    for (int nb = 0; nb < 8; ++nb) st.o[nb] *= alpha;
    if (raise) st.m = mx;
  }
  const float m_use = (st.m == -INFINITY) ? 0.f : st.m;
  bf16x8 pb;
  float ps = 0.f;
  #pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float p = fast_exp2(x[i] - m_use);
    ps += p;
    pb[i] = (bf16)p;
  }
  st.l += ps;
  return pb;
}

__device__ __forceinline__ void pv_update(RowState& st, const bf16x8& pb, const bf16x8* vt) {
  #pragma unroll
  for (int nb = 0; nb < 8; ++nb)
    st.o[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[nb], pb, st.o[nb], 0, 0, 0);
}

__device__ __forceinline__ void qk_tile(const bf16x8 (&kf)[2][4], const bf16x8 (&qf)[4], f32x4& s0, f32x4& s1) {
  s0 = f32x4{0.f, 0.f, 0.f, 0.f};
  s1 = f32x4{0.f, 0.f, 0.f, 0.f};
  #pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[0][ks], qf[ks], s0, 0, 0, 0);
    s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[1][ks], qf[ks], s1, 0, 0, 0);
  }
}


// ---------------------------------------------------------------------------
// split-K partials
// ---------------------------------------------------------------------------
// Work item p owns part_o[p][16][128] (unnormalised O) and part_ml[p][16][2]
// (running max in the log2 domain, running sum).  The partials of one
// (request, KV head, tile) are p0 + c*pstride for its chunks c = 0..nch-1.
template <int ND>
__device__ __forceinline__ void merge_partials(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                               size_t p0, size_t pstride, int nch, int row, int d0,
                                               float (&acc)[ND], float& L) {
  // One pass in groups of four chunks: every load of a group is issued
  // before any use, then the (max, sum, O) triples are folded in with the
  // online-softmax rule.  Chunks with no visible key (max = -inf) add
  // nothing.
  float M = -INFINITY;
  L = 0.f;
  #pragma unroll
  for (int i = 0; i < ND; ++i) acc[i] = 0.f;
  for (int c0 = 0; c0 < nch; c0 += 4) {
    float mc[4], lc[4];
    f32x4 x[4][ND / 4];
    #pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t p = p0 + (size_t)min(c0 + u, nch - 1) * pstride;
      mc[u] = part_ml[(p * 16 + row) * 2];
      lc[u] = part_ml[(p * 16 + row) * 2 + 1];
      const float* po = part_o + (p * 16 + row) * HD + d0;
      #pragma unroll
      for (int i = 0; i < ND / 4; ++i) x[u][i] = *reinterpret_cast<const f32x4*>(po + 4 * i);
    }
    #pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (c0 + u >= nch || mc[u] == -INFINITY) continue;
      if (mc[u] > M) {
        const float sc = fast_exp2(M - mc[u]);
        L *= sc;
        #pragma unroll
        for (int i = 0; i < ND; ++i) acc[i] *= sc;
        M = mc[u];
      }
      const float w = fast_exp2(mc[u] - M);
      L += w * lc[u];
      #pragma unroll
      for (int i = 0; i < ND / 4; ++i) {
        acc[4 * i] += w * x[u][i][0];
        acc[4 * i + 1] += w * x[u][i][1];
        acc[4 * i + 2] += w * x[u][i][2];
        acc[4 * i + 3] += w * x[u][i][3];
      }
    }
  }
}


// Sum of chunks_for() over requests [0, r), executed by each wave.
__device__ __forceinline__ int chunk_base(const int32_t* cu, const int32_t* lens, int r, int chunk) {
  const int lane = threadIdx.x & 63;
  int acc = 0;
  for (int r0 = 0; r0 < r; r0 += WAVE) {
    const int rr = r0 + lane;
    int n = 0;
    if (rr < r) n = chunks_for(cu ? (cu[rr + 1] - cu[rr]) : lens[rr], chunk);
    #pragma unroll
    for (int off = 32; off >= 1; off >>= 1) n += __shfl_xor(n, off);
    acc += n;
  }
  return acc;
}

// ---------------------------------------------------------------------------
// varlen / verify
// ---------------------------------------------------------------------------
struct VarlenArgs {
  const bf16* q;          // [nq, 16, 128]
  const bf16* k_a;        // segment A: [rows, 8, 128]
  const bf16* v_a;
  const bf16* k_b;        // segment B (verify: scratch layer [max_q, 8, 128])
  const bf16* v_b;
  const int32_t* cu_q;    // [B+1]
  const int32_t* cu_k;    // [B+1]
  const int32_t* slots;   // verify: resident slot per request
  int64_t slot_stride;    // verify: elements between resident slots
  int64_t a_tok_stride;   // segment A elements between token rows
  int64_t a_head_stride;  // segment A elements between KV heads
  const int32_t* work;    // optional segment list (see the C ABI)
  bf16* stage_k;          // verify with staging: scratch written from segment B (k_b/v_b = new rows)
  bf16* stage_v;
  bf16* out;              // [nq, 16, 128]
  float* part_o;          // [n_cl*8*tmax][16][128]
  float* part_ml;         // [n_cl*8*tmax][16][2]
  int n_req;
  int n_work;             // segment records in the work list
  int n_slots;            // no list: (chunk, KV head) slots, 8 * chunks
  int causal;
  int chunk;
  int tmax;
  float scale_log2;
};

// Per wave a 32-key K tile and a 32-key V tile (8 KiB each); the 4-wave
// merge buffer (34,304 B) reuses the start once the tiles are done.
constexpr int VARLEN_SMEM = 2 * 4 * KT * ROWB;                      // 65536 B
static_assert(VARLEN_SMEM >= 4 * 16 * OPITCH * 4 + 4 * 16 * 2 * 4, "the tiles must cover the merge buffer");

// One key segment of one request: keys [k0, k1) of request r, whose
// queries start at row q0 (ql of them) and whose keys number kl; start is
// the first key row (varlen) or the resident slot (verify).  A request cut
// into several segments writes FP32 partials to slot pslot (>= 0) for the
// merge kernel; a request held by one segment (pslot < 0) writes its output.
struct Segment {
  int r, k0, k1, pslot, q0, ql, kl, start;
};

// Fixed chunking without a work list: linear chunk index cl of the grid
// (requests in order, ceil(kl / chunk) chunks each, at least one).
__device__ __forceinline__ bool chunk_segment(const VarlenArgs& a, bool verify, int cl, Segment& s) {
  int r, first;
  locate_chunk(a.cu_k, nullptr, a.n_req, a.chunk, cl, r, first);
  if (r < 0) return false;
  const int c = cl - first;
  s.r = r;
  s.q0 = a.cu_q[r];
  s.ql = a.cu_q[r + 1] - s.q0;
  s.kl = a.cu_k[r + 1] - a.cu_k[r];
  s.start = verify ? a.slots[r] : a.cu_k[r];
  s.k0 = c * a.chunk;
  s.k1 = min(s.k0 + a.chunk, s.kl);
  s.pslot = chunks_for(s.kl, a.chunk) > 1 ? first + c : -1;
  return true;
}

// The addressing of one segment for one (KV head, row tile); every field is
// wave-uniform.  Key j of the request lives in part A (committed rows) for
// j < a_len, else in part B (rows new to this call).
struct SegView {
  const bf16* kA;
  const bf16* vA;
  const bf16* kB;
  const bf16* vB;
  size_t bbase;   // part B offset of the request's first new row, KV head g
  int a_len;
  int k0;
  int kend;       // keys [k0, kend) are visible to some row of the tile
  int kfast;      // tiles below kfast need no clamping, source choice or mask
  int q0, ql, kl, pslot;
  bool live;      // the tile has query rows (8t < ql)
  bool ends;      // the segment holds the request's last key
};

template <bool VERIFY>
__device__ __forceinline__ SegView seg_view(const VarlenArgs& a, const Segment& sg, int g, int t) {
  SegView v;
  // The segment is wave-uniform; say so, so that its fields and everything
  // derived from them stay in scalar registers.
  v.q0 = __builtin_amdgcn_readfirstlane(sg.q0);
  v.ql = __builtin_amdgcn_readfirstlane(sg.ql);
  v.kl = __builtin_amdgcn_readfirstlane(sg.kl);
  const int start = __builtin_amdgcn_readfirstlane(sg.start);
  v.k0 = __builtin_amdgcn_readfirstlane(sg.k0);
  const int k1 = __builtin_amdgcn_readfirstlane(sg.k1);
  v.pslot = __builtin_amdgcn_readfirstlane(sg.pslot);
  v.live = 8 * t < v.ql;
  v.ends = k1 == v.kl;
  if (VERIFY) {
    v.a_len = v.kl - v.ql;
    const size_t abase = (size_t)start * (size_t)a.slot_stride + (size_t)g * a.a_head_stride;
    v.kA = a.k_a + abase;
    v.vA = a.v_a + abase;
    v.bbase = (size_t)v.q0 * KV_ROW + (size_t)g * HD;
    v.kB = a.k_b + v.bbase;
    v.vB = a.v_b + v.bbase;
  } else {
    v.a_len = v.kl;
    const size_t abase = (size_t)start * KV_ROW + (size_t)g * HD;
    v.kA = a.k_a + abase;
    v.vA = a.v_a + abase;
    v.kB = v.kA;
    v.vB = v.vA;
    v.bbase = 0;
  }
  const int last_tok = min(8 * t + 7, v.ql - 1);
  const int tile_lim = a.causal ? v.kl - v.ql + last_tok + 1 : v.kl;
  v.kend = v.live ? min(k1, tile_lim) : v.k0;
  // Keys below kfast come from part A and are visible to every row of this
  // tile (bottom-right causal: row tok sees keys <= kl - ql + tok).
  v.kfast = min(min(v.kend, v.a_len), a.causal ? v.kl - v.ql + 8 * t + 1 : v.kl);
  return v;
}

// One 32-key tile in registers as loaded: K and V alike as 4 full rows per
// load (lane (col, grp) of load i holds key 4*i+grp, dims 8col..+8), so
// every load instruction reads 4 whole 256-byte rows.  Both go through LDS:
// K comes back as the S^T A-operand, V as V^T.
struct Tile {
  bf16x8 k[8];
  bf16x8 v[8];
};

// Per-lane byte offsets of the fast (unclamped, part A) tile loads; they
// depend only on the token stride, so they hold for every segment and for
// K and V alike.
struct FastOffsets {
  uint32_t r[8];
};

// K/V rows are read once per call: non-temporal loads.
__device__ __forceinline__ bf16x8 ld8_nt(const void* p) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}

// A tile below kfast: part A rows at wave-uniform base + per-lane offsets.
__device__ __forceinline__ void load_fast(const VarlenArgs& a, const SegView& s, const FastOffsets& fo, int kt,
                                          Tile& T) {
  const char* kb = reinterpret_cast<const char*>(s.kA + (size_t)kt * a.a_tok_stride);
  const char* vb = reinterpret_cast<const char*>(s.vA + (size_t)kt * a.a_tok_stride);
  #pragma unroll
  for (int i = 0; i < 8; ++i) {
    T.k[i] = ld8_nt(kb + fo.r[i]);
    T.v[i] = ld8_nt(vb + fo.r[i]);
  }
}

// Any tile: rows clamped, each from part A or B.
__device__ __forceinline__ void load_slow(const VarlenArgs& a, const SegView& s, int kt, Tile& T) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  // Row kk of this request, clamped to kend-1 so that every load is in
  // range; rows past kend are masked out of the softmax and zeroed in V.
  auto row = [&](const bf16* pa, const bf16* pb, int kk) -> const bf16* {
    kk = min(kk, s.kend - 1);
    return kk < s.a_len ? pa + (size_t)kk * a.a_tok_stride : pb + (size_t)(kk - s.a_len) * KV_ROW;
  };
  #pragma unroll
  for (int i = 0; i < 8; ++i) {
    T.k[i] = ld8_nt(row(s.kA, s.kB, kt + 4 * i + grp) + 8 * col);
    T.v[i] = ld8_nt(row(s.vA, s.vB, kt + 4 * i + grp) + 8 * col);
  }
}

// Q of this lane's row of segment s.
__device__ __forceinline__ void load_q(const VarlenArgs& a, const SegView& s, int g, int t, bf16x8 (&qf)[4]) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int tok = 8 * t + (col >> 1);
  const bool row_ok = tok < s.ql;
  const bf16* qp = a.q + (size_t)(s.q0 + (row_ok ? tok : 0)) * Q_ROW + (size_t)(2 * g + (col & 1)) * HD + 8 * grp;
  #pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = row_ok ? ld8(qp + 32 * ks) : zero8();
}

// One run of segments for one (KV head, row tile): wave w computes tiles
// k0 + 32w, k0 + 32(w+4), ... of each segment.
// fetch(n, sg) yields the run's n-th segment (false past the end); every
// branch on it is uniform across the workgroup.
template <bool VERIFY, typename Fetch>
__device__ __forceinline__ void varlen_run(const VarlenArgs& a, unsigned char* smem, int g, int t, Fetch fetch) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  FastOffsets fo;
  {
    const int64_t ts = a.a_tok_stride;
    #pragma unroll
    for (int i = 0; i < 8; ++i) fo.r[i] = (uint32_t)(((4 * i + grp) * ts + 8 * col) * 2);
  }
  unsigned char* vs = smem + wave * KT * ROWB;
  unsigned char* kst = smem + (4 + wave) * KT * ROWB;
  const int tok = 8 * t + (col >> 1);

  Segment sg;
  if (!fetch(0, sg)) return;
  SegView cur = seg_view<VERIFY>(a, sg, g, t);
  bf16x8 qf[4];
  for (int n = 0;; ++n) {
    load_q(a, cur, g, t, qf);
    Segment nsg;
    const bool more = fetch(n + 1, nsg);

    const bool row_ok = tok < cur.ql;
    const int lim = row_ok ? (a.causal ? cur.kl - cur.ql + tok + 1 : cur.kl) : 0;
    const int vis = min(lim, cur.kend);
    RowState st;
    row_init(st);
    auto compute = [&](Tile& T, int kt, auto masked) {
      constexpr bool MASKED = decltype(masked)::value;
      if (MASKED && kt + KT > cur.kend) {
        #pragma unroll
        for (int i2 = 0; i2 < 8; ++i2)
          if (kt + 4 * i2 + grp >= cur.kend) T.v[i2] = zero8();
      }
      #pragma unroll
      for (int i = 0; i < 8; ++i) {
        *reinterpret_cast<bf16x8*>(kst + lds_chunk_off(4 * i + grp, col)) = T.k[i];
        *reinterpret_cast<bf16x8*>(vs + lds_chunk_off(4 * i + grp, col)) = T.v[i];
      }
      wave_lds_sync();
      // S^T A-operand of sub-tile j, k-step ks: lane (col, grp) takes key
      // 8*(col/4) + 4j + col%4, dims 32ks + 8grp .. +8, so that each lane's
      // 8 scores are 8 consecutive keys (the P^T operand of the PV step).
      // The 16 lanes of a group read 16 rows whose swizzles differ.
      bf16x8 kf[2][4];
      #pragma unroll
      for (int j = 0; j < 2; ++j)
        #pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          kf[j][ks] = *reinterpret_cast<const bf16x8*>(
              kst + lds_chunk_off(8 * (col >> 2) + 4 * j + (col & 3), 4 * ks + grp));
      f32x4 s0, s1;
      qk_tile(kf, qf, s0, s1);
      const bf16x8 pb = softmax_update<MASKED>(st, s0, s1, kt + 8 * grp, vis, a.scale_log2);
      bf16x8 vt[8];
      #pragma unroll
      for (int nb = 0; nb < 8; ++nb) vt[nb] = lds_vt(vs, nb, lane);
      pv_update(st, pb, vt);
      wave_lds_sync();
    };
    int kt = cur.k0 + KT * wave_u;
    for (; kt + KT <= cur.kfast; kt += KT * 4) {
      Tile T;
      load_fast(a, cur, fo, kt, T);
      compute(T, kt, std::false_type{});
    }
    for (; kt < cur.kend; kt += KT * 4) {
      Tile T;
      load_slow(a, cur, kt, T);
      compute(T, kt, std::true_type{});
    }
    // Fused stage: the workgroup holding the request's last segment (row
    // tile 0) is the only reader of its new rows for KV head g, so it also
    // copies them into the scratch layer.  The first 256 16-byte pieces are
    // loaded here and stored after the merge, which hides their latency.
    const bool stage = VERIFY && a.stage_k && cur.ends && t == 0;
    const int n_stage = 2 * cur.ql * 16;
    auto stage_off = [&](int i, bool& v_half) -> size_t {
      v_half = i >= cur.ql * 16;
      const int rem = v_half ? i - cur.ql * 16 : i;
      return cur.bbase + (size_t)(rem >> 4) * KV_ROW + (size_t)(rem & 15) * 8;
    };
    bf16x8 staged = zero8();
    if (stage && (int)threadIdx.x < n_stage) {
      bool vh;
      const size_t off = stage_off(threadIdx.x, vh);
      staged = *reinterpret_cast<const bf16x8*>((vh ? a.v_b : a.k_b) + off);
    }

    if (cur.live) {
      st.l = wave_sum_across_groups(st.l);
      __syncthreads();
      float* ob = reinterpret_cast<float*>(smem);
      float* mlb = reinterpret_cast<float*>(smem + 4 * 16 * OPITCH * 4);
      #pragma unroll
      for (int nb = 0; nb < 8; ++nb)
        *reinterpret_cast<f32x4*>(ob + (wave * 16 + col) * OPITCH + 16 * nb + 4 * grp) = st.o[nb];
      if (grp == 0) {
        mlb[(wave * 16 + col) * 2 + 0] = st.m;
        mlb[(wave * 16 + col) * 2 + 1] = st.l;
      }
      __syncthreads();

      const int tid = threadIdx.x;
      const int row = tid >> 4;
      const int d0 = (tid & 15) * 8;
      float M = -INFINITY;
      #pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, mlb[(w * 16 + row) * 2]);
      float L = 0.f;
      float acc[8];
      #pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.f;
      #pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float mw = mlb[(w * 16 + row) * 2];
        const float sc = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
        L += sc * mlb[(w * 16 + row) * 2 + 1];
        const float* src = ob + (w * 16 + row) * OPITCH + d0;
        #pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += sc * src[i];
      }
      const int tok_r = 8 * t + (row >> 1);
      const int head_r = 2 * g + (row & 1);
      if (cur.pslot >= 0) {
        const size_t p = (size_t)(cur.pslot * 8 + g) * a.tmax + t;
        float* po = a.part_o + (p * 16 + row) * HD + d0;
        *reinterpret_cast<f32x4*>(po) = f32x4{acc[0], acc[1], acc[2], acc[3]};
        *reinterpret_cast<f32x4*>(po + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
        if ((tid & 15) == 0) {
          a.part_ml[(p * 16 + row) * 2 + 0] = M;
          a.part_ml[(p * 16 + row) * 2 + 1] = L;
        }
      } else if (tok_r < cur.ql) {
        bf16x8 ov;
        #pragma unroll
        for (int i = 0; i < 8; ++i) ov[i] = (bf16)(acc[i] / L);
        *reinterpret_cast<bf16x8*>(a.out + (size_t)(cur.q0 + tok_r) * Q_ROW + (size_t)head_r * HD + d0) = ov;
      }
    }
    if (stage) {
      for (int i = threadIdx.x; i < n_stage; i += 256) {
        bool vh;
        const size_t off = stage_off(i, vh);
        const bf16x8 x = i < 256 ? staged : *reinterpret_cast<const bf16x8*>((vh ? a.v_b : a.k_b) + off);
        *reinterpret_cast<bf16x8*>((vh ? a.stage_v : a.stage_k) + off) = x;
      }
    }
    __syncthreads();   // the next segment reuses the V tiles and the merge buffer
    if (!more) break;
    cur = seg_view<VERIFY>(a, nsg, g, t);
  }
}

// Timeline build (compiled with DSPARK_TIMELINE into a separate profiling
// library; the product library has none of this): lane 0 of wave 0 of every
// draft workgroup records, per segment it runs, the 100 MHz constant clock
// at the segment's start, once its first ring loads are issued, once the
// first context stage (or the own rows) has landed, at the end of the key
// stream and after the half merge and output write, plus where it ran.  The
// stamps are held in scalar registers and stored after the segment's write,
// so the ring's load accounting sees no extra memory operation.  Every
// verification workgroup of a work-list launch records its start and end.
#ifdef DSPARK_TIMELINE
constexpr int TL_WGS = 8192;                         // workgroups recorded
constexpr int TL_ITEMS = 16;                         // segments recorded per workgroup
constexpr int TL_WORDS = 8;
__device__ uint64_t tl_stamps[TL_WGS * TL_ITEMS * TL_WORDS];
// Persistent mode, per workgroup: entry, first ticket known, loop left, exit.
__device__ uint64_t tl_wg[TL_WGS * 4];
// Verification with a work list, per workgroup: start, end, where (HW_ID,
// XCC_ID << 32, bit 63 set), keys streamed | segments << 32.
__device__ uint64_t tl_vwg[TL_WGS * 4];
__device__ __forceinline__ uint64_t tl_now() { return __builtin_amdgcn_s_memrealtime(); }
#define TL_DECL uint64_t tl_t[5] = {0, 0, 0, 0, 0};
#define TL_MARK(i) (tl_t[i] = tl_now())
#else
#define TL_DECL
#define TL_MARK(i) ((void)0)
#endif

// With a work list, the 8 workgroups of run w (one per KV head g) all run
// on XCD w mod 8: workgroups are dealt round-robin over the 8 XCDs, so
// blockIdx.x = 8 (8 (w / 8) + g) + w mod 8 (the run count is a multiple of
// 8).  A plan can then size the runs of each XCD to its measured speed.
// Without a list, a persistent grid walks the fixed chunks (item, KV head)
// with a stride of the grid size, so per-workgroup start-up is paid once
// per CU slot.
template <bool VERIFY>
__global__ __launch_bounds__(256, 2) void varlen_attn_kernel(VarlenArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[VARLEN_SMEM];
  const int slot = blockIdx.x >> 3;
  const int g = a.work ? (slot & 7) : (blockIdx.x & 7);
  if (a.work) {
    const int run = ((slot >> 3) << 3) | (blockIdx.x & 7);
    const int32_t* range = a.work + WORK_INTS * a.n_work + run;
    const int b = min(max(range[0], 0), a.n_work);      // clamped: never past the records
    const int e = min(max(range[1], b), a.n_work);
#ifdef DSPARK_TIMELINE
    const uint64_t tl_start = tl_now();
    int tl_keys = 0;
#endif
    varlen_run<VERIFY>(a, smem, g, blockIdx.y, [&](int n, Segment& sg) {
      if (b + n >= e) return false;
      const int32_t* w = a.work + WORK_INTS * (b + n);
      sg = Segment{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
#ifdef DSPARK_TIMELINE
      tl_keys += sg.k1 - sg.k0;
#endif
      return true;
    });
#ifdef DSPARK_TIMELINE
    const uint64_t tl_end = tl_now();
    const int wid = blockIdx.x + gridDim.x * blockIdx.y;
    if (threadIdx.x == 0 && wid < TL_WGS) {
      uint32_t hw, xcc;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
      uint64_t* t = tl_vwg + 4 * (size_t)wid;
      t[0] = tl_start;
      t[1] = tl_end;
      t[2] = (uint64_t)hw | ((uint64_t)(xcc & 15) << 32) | ((uint64_t)1 << 63);
      t[3] = (uint64_t)(uint32_t)tl_keys | ((uint64_t)(uint32_t)(e - b) << 32);
    }
#endif
    return;
  }
  varlen_run<VERIFY>(a, smem, g, blockIdx.y, [&](int n, Segment& sg) {
    const int idx = blockIdx.x + n * gridDim.x;
    return idx < a.n_slots && chunk_segment(a, VERIFY, idx >> 3, sg);
  });
}

// ---------------------------------------------------------------------------
// draft (multi-block, context streamed once per request)
// ---------------------------------------------------------------------------
struct DraftArgs {
  const void* q;            // [7*n_blocks, 16, 128] bf16 or fp32 (q_f32), request-major, block-major
  const void* k_ctx;        // context pool (bf16, or fp32 in the KF32 instance), element (row, head, d) at
  const bf16* v_ctx;        //   row*tok_stride + head*head_stride + d
  const int64_t* ctx_idx;   // optional physical row per (request, position)
  const int64_t* ctx_off;   // [B] first row (or first ctx_idx entry) of request r
  const int32_t* ctx_len;   // [B] committed context rows of request r
  const void* k_blk;        // [7*n_blocks, 8, 128] projected block K (same type as k_ctx)
  const bf16* v_blk;        //   and V (bf16)
  const int32_t* cu_b;      // [B+1] block offsets
  const int32_t* anchors;   // [n_blocks] context rows visible to each block
  bf16* out;                // [7*n_blocks, 16, 128]
  float* part_o;
  float* part_ml;
  int64_t tok_stride;
  int64_t head_stride;
  const int32_t* work;      // optional segment list (see the C ABI)
  int* queue;               // persistent mode: ticket counters (self-resetting; see draft_persistent)
  const int32_t* seg_anc;   // persistent mode: 8 anchors per segment record (its blocks', padded)
  int n_work;               // segment records in the work list
  int n_runs;               // runs of the work list (persistent mode: items = 8 * n_runs)
  int queues;               // persistent mode: 1 (one queue) or 8 (one per XCD, head g on XCD g)
  int n_req;
  int chunk;
  int tmax;                 // max blocks per request (<= 8)
  int q_f32;                // Q is fp32 (rounded to bf16 at load)
  float scale_log2;
};

constexpr int BLOCK_ROWS = 7;
constexpr int MAX_BLOCKS = 8;                        // draft blocks per request
constexpr int CHUNK_ALIGN = 64;                      // fixed chunks are multiples of this many keys

// One context segment of one request: keys [k0, k1) of request r (whose
// blocks are b0 .. b0+nb, largest anchor amax).  The segment ending the
// request (`last`) also attends the blocks' own rows.  A request held by
// more than one segment writes FP32 partials per block to slot pslot (>= 0);
// a request held by one segment writes its output.
struct DraftSeg {
  int r, k0, k1, pslot, b0, nb, amax;
  bool last;
  int off1;   // 1 + ctx_off[r] when the plan carries it, else 0
};

// A pair of draft blocks is attended as one 32-row tile: row n is block
// 2p + n/16 of pair p, token (n%16)/2, query head 2g + n%2 (rows with token
// 7 and rows of a block the request does not have carry zero Q and are never
// written).  Wave w of the workgroup takes pair p = w/2 and key half
// h = w%2: rows 32h .. 32h+31 of every 64-key ring stage (the two halves
// are merged at the end), so that each wave reads half of each stage from
// LDS and a request with few blocks still keeps two waves busy.
//
// v_mfma_f32_32x32x16_bf16 (wave64): A lane l supplies row l%32 at
// k = 8(l/32) + i, B lane l supplies column l%32 at the same k, and
// accumulator register r of lane l is row 8(r/4) + 4(l/32) + r%4, column
// l%32.  With A = K (rows = key slots) and B = Q^T, lane l holds 16 scores
// of query row l%32; registers 8t .. 8t+7 are the B operand (P^T) of PV
// k-step t when the A operand (V^T) of lane l takes slots
// 8(2t + i/4) + 4(l/32) + i%4, i = 0..7.
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) int lds_i32;

constexpr int DWAVES = 8;                            // waves per workgroup: 4 pairs x 2 key halves
constexpr int DSTEP = 64;                            // context keys per ring stage
static_assert(DWAVES == MAX_BLOCKS, "the pairs cover the most blocks a request may hold");
static_assert(CHUNK_ALIGN % DSTEP == 0, "fixed chunks hold whole stages");

// The context ring: each stage holds DSTEP K rows then DSTEP V rows, filled
// by direct global->LDS loads of 1 KiB pieces (PER_WAVE per wave).  Rows are
// XOR-swizzled by 16-byte chunk: a bf16 row (256 B) holds chunk c at
// c ^ swz(row); an fp32 K row (the reference's AMP pool,
// packed_draft.py:222-235; 512 B) holds the low four floats of bf16 chunk c
// at 16-byte position c ^ swz(row) and the high four at 16 + (c ^ swz(row)).
// The segment ending a request first stages the blocks' own rows in the last
// slot (pair p's 16 K rows at rows 16p .. 16p+15, then 64 V rows likewise,
// swizzled by row % 16), attends them, and only then lets the context stream
// reuse that slot.  After the stream, the key halves merge through the
// drained ring.
template <bool KF32>
struct PairRing {
  static constexpr int KROW = KF32 ? 2 * ROWB : ROWB;   // bytes per staged K row
  // Three stages (two in flight): measured faster than four for the bf16
  // ring (≈121 against ≈124 us per draft call; two stages: ≈135 us).
  static constexpr int STAGES = 3;                         // ring: 144 KiB (fp32 K) or 96 KiB
  static constexpr int K_BYTES = DSTEP * KROW;
  static constexpr int STAGE_BYTES = K_BYTES + DSTEP * ROWB;
  static constexpr int K_PIECES = K_BYTES / 1024;
  static constexpr int PER_WAVE = STAGE_BYTES / 1024 / DWAVES;
  // bf16 instance: the segment's bf16 Q rows are loaded into LDS with the
  // ring (pair p's 32 tile rows at rows 32p .. 32p+31, 256 B each, swizzled
  // by row), so no ordinary load precedes the ring's loads.
  static constexpr int Q_OFF = STAGES * STAGE_BYTES;
  static constexpr int Q_BYTES = KF32 ? 0 : 4 * 32 * ROWB;
  static constexpr int SMEM = Q_OFF + Q_BYTES;
  // Indexed context only: per ring slot, each wave's copy of the stage's
  // DSTEP physical row indices (32-bit), after the ring and Q.
  static constexpr int IDX_OFF = SMEM;
  static constexpr int IDX_BYTES = STAGES * DWAVES * DSTEP * 4;
  static constexpr int OWN_SLOT = (STAGES - 1) * STAGE_BYTES;
  static constexpr int MERGE_FLOATS = 64 + 2;              // per lane: O^T, max, sum
  static constexpr int MERGE_BYTES = MERGE_FLOATS * WAVE * 4;
  static_assert(PER_WAVE * DWAVES * 1024 == STAGE_BYTES, "stage pieces must divide evenly over the waves");
  static_assert(SMEM + IDX_BYTES <= 158 * 1024, "ring exceeds the LDS of a CU");
  static_assert(DSTEP == WAVE, "a stage's indices are one word per lane");
  static_assert(Q_BYTES == 0 || Q_BYTES == PER_WAVE * DWAVES * 1024, "a Q load is one piece round");
  // The half merge may reach into the own-row slot: a barrier separates
  // the own-block reads from the merge writes also when no context stage runs.
  static_assert(4 * MERGE_BYTES <= SMEM, "the half merge fits the ring");
};

// Staged row of key slot m (0..31).  Rows are permuted so that the 16 lanes
// of a K-fragment read (slots 16u .. 16u+15) see 16 distinct swizzles.
__device__ __forceinline__ int slot_row(int m) {
  return 8 * ((m >> 2) & 3) + (m & 3) + 4 * (m >> 4);
}

// Staged row of the key behind accumulator register r of a lane in half hh
// (= l/32): slot_row(8(r/4) + 4hh + r%4).
__device__ __forceinline__ int acc_row(int r, int hh) {
  return 16 * ((r >> 2) & 1) + 8 * hh + 4 * (r >> 3) + (r & 3);
}

struct PairState {
  float m;         // running reference max of the lane's row (log2 domain)
  float l;         // per-lane partial sum (16 of the row's 32 slots per tile)
  f32x16 o[4];     // O^T accumulators for dims 32D .. 32D+31
};

// Per-lane LDS byte offsets of a 32-key tile, written so that every read of
// the tile is the base XOR a constant (plus an immediate):
//  * K fragment of k-step ks (dims 16ks .. 16ks+15; the lane reads bf16
//    chunk (2ks + l/32) ^ swz(kr) of staged row kr):  k ^ 32ks (fp32 rows:
//    the low half there, the high half 256 bytes above);
//  * V^T of PV k-step t, dims 32D .. 32D+31: two transpose reads (each
//    16-lane group reads 4 rows x 16 dims; lane 4*row + c supplies dims
//    4c .. 4c+3 of its row) of the rows behind slots 16t + 4(l/32) + i and
//    16t + 8 + 4(l/32) + i (i < 4):  (v ^ 64D) + 1024t and
//    (v ^ 64D ^ V1_XOR) + V1_ADD + 1024t.
// Swizzles and chunk numbers occupy address bits 4..7 and rows start at
// multiples of 256 bytes, so the XORs never carry into a row.
struct TileOffsets {
  uint32_t k;
  uint32_t v;
};

// Context stage: slot m's key is staged row slot_row(m).  The rows behind
// the V^T reads are 8(l/32) + 4t + i (swizzle 4i + l/32) and 16 more
// (swizzle ^ 2).
constexpr uint32_t CTX_V1_XOR = 32;
constexpr uint32_t CTX_V1_ADD = 16 * ROWB;
template <int KROW>
__device__ __forceinline__ TileOffsets ctx_tile_offsets(int lane) {
  const int hh = lane >> 5;
  const int rr = (lane >> 2) & 3;
  const int c4 = lane & 3;
  const int kr = slot_row(lane & 31);
  const int vr = 8 * hh + rr;
  return TileOffsets{(uint32_t)(kr * KROW + ((16 * hh) ^ (16 * swz(kr)))),
                     (uint32_t)(vr * ROWB + ((32 * ((lane >> 4) & 1) + 16 * (c4 >> 1)) ^ (16 * swz(vr))) + 8 * (c4 & 1))};
}

// Own rows of a pair: staged row v (0..31) of the tile is row
// 8(v/16) + v%8 (block v/16 of the pair, token v%8) of the 16 staged K and
// 16 staged V rows; half 1's slots (v%16 >= 8) repeat half 0's rows.  The
// rows behind the V^T reads are 4t + i (swizzle 4i) and 8 more (swizzle ^ 1).
constexpr uint32_t OWN_V1_XOR = 16;
constexpr uint32_t OWN_V1_ADD = 8 * ROWB;
template <int KROW>
__device__ __forceinline__ TileOffsets own_tile_offsets(int lane) {
  const int hh = lane >> 5;
  const int rr = (lane >> 2) & 3;
  const int c4 = lane & 3;
  const int sr = slot_row(lane & 31);
  const int kr = 8 * (sr >> 4) + (sr & 7);
  return TileOffsets{(uint32_t)(kr * KROW + ((16 * hh) ^ (16 * swz(kr)))),
                     (uint32_t)(rr * ROWB + ((32 * ((lane >> 4) & 1) + 16 * (c4 >> 1)) ^ (16 * swz(rr))) + 8 * (c4 & 1))};
}

// The K fragment at LDS address `addr`: bf16 as staged, or fp32 rounded to
// bf16 (round to nearest even, the bits of attending a bf16 copy).
template <bool KF32>
__device__ __forceinline__ bf16x8 lds_k_frag(uint32_t addr) {
  if constexpr (KF32) {
    const f32x4 lo = *(const lds_f32x4*)(uintptr_t)addr;
    const f32x4 hi = *(const lds_f32x4*)(uintptr_t)(addr + 256);
    return to_bf16x8(lo, hi);
  } else {
    return *(const lds_bf16x8*)(uintptr_t)addr;
  }
}

__device__ __forceinline__ bf16x4 lds_tr4(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(uintptr_t)addr);
}

// One 32-key tile of a pair: S^T = K Q^T, online softmax, O^T += V^T P^T.
// ka/va: LDS addresses of the lane's K and V bases (TileOffsets plus the K
// and V base of the tile).  In a masked tile `visible(r)` says whether the
// key of accumulator register r is visible to the lane's query row.
//
// The running maximum only moves up when a tile's maximum exceeds it by more
// than RESCALE_SLACK (log2 units), so O and l are rescaled rarely instead of
// every tile.  Exact for any reference value: O and l always share the same
// reference max, which the split-K merge carries along; probabilities stay
// <= 2^RESCALE_SLACK, far from FP32/bf16 overflow.  The rescale branch is
// wave-uniform.
template <bool KF32, uint32_t V1_XOR, uint32_t V1_ADD, class Vis>
__device__ __forceinline__ void pair_tile(PairState& st, const bf16x8 (&qf)[8], uint32_t ka, uint32_t va, bool masked,
                                          Vis visible, float scale_log2) {
  // Every LDS read of the tile is issued up front: the K fragments, then
  // the V^T halves, whose latency the QK chain and the softmax then hide.
  bf16x8 kf[8];
  #pragma unroll
  for (int ks = 0; ks < 8; ++ks) kf[ks] = lds_k_frag<KF32>(ka ^ (32u * ks));
  __builtin_amdgcn_sched_barrier(0);
  bf16x4 vlo[2][4], vhi[2][4];
  #pragma unroll
  for (int t = 0; t < 2; ++t)
    #pragma unroll
    for (int D = 0; D < 4; ++D) {
      vlo[t][D] = lds_tr4((va ^ (64u * D)) + 1024u * t);
      vhi[t][D] = lds_tr4((va ^ (64u * D) ^ V1_XOR) + V1_ADD + 1024u * t);
    }
  f32x16 s = {};
  #pragma unroll
  for (int ks = 0; ks < 8; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
  #pragma unroll
  for (int r = 0; r < 16; ++r) s[r] *= scale_log2;
  if (masked) {
    #pragma unroll
    for (int r = 0; r < 16; ++r)
      if (!visible(r)) s[r] = -INFINITY;
  }
  float mx = s[0];
  #pragma unroll
  for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));    // lanes l and l^32 hold the same row
  const bool raise = mx > st.m + RESCALE_SLACK;
  if (__builtin_amdgcn_ballot_w64(raise)) {
    // Rows that do not raise keep factor 1 (their max may still be -inf,
    // and -inf - -inf must not reach exp2).
    const float alpha = raise ? fast_exp2(st.m - mx) : 1.0f;
    st.l *= alpha;
    #pragma unroll
    for (int D = 0; D < 4; ++D) st.o[D] *= alpha;
    if (raise) st.m = mx;
  }
  const float m_use = (st.m == -INFINITY) ? 0.f : st.m;
  bf16x8 pb[2];
  float ps = 0.f;
  #pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float p = fast_exp2(s[r] - m_use);
    ps += p;
    pb[r >> 3][r & 7] = (bf16)p;
  }
  st.l += ps;
  #pragma unroll
  for (int t = 0; t < 2; ++t)
    #pragma unroll
    for (int D = 0; D < 4; ++D) {
      bf16x8 vt;
      #pragma unroll
      for (int i = 0; i < 4; ++i) {
        vt[i] = vlo[t][D][i];
        vt[4 + i] = vhi[t][D][i];
      }
      st.o[D] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt, pb[t], st.o[D], 0, 0, 0);
    }
}

// A wave-uniform read-only kernel input through the constant address space,
// i.e. a scalar load: it waits on lgkmcnt, never on the vmcnt that orders
// the ring.
template <class T>
__device__ __forceinline__ T ld_const(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

// ld_const of element i (wave-uniform; stated, so that the address stays in
// scalar registers).
template <class T>
__device__ __forceinline__ T ld_const(const T* p, int i) {
  return ld_const(p + __builtin_amdgcn_readfirstlane(i));
}

// The register operands must hold their loaded values here: the compiler
// places its wait for them before this point, while no direct-to-LDS load
// is in flight yet (a wait placed later would drain the ring).
template <class T>
__device__ __forceinline__ void settle_one(const T& x) {
  asm volatile("" ::"v"(x));
}

template <class... T>
__device__ __forceinline__ void settle(const T&... x) {
  (settle_one(x), ...);
}

// The persistent loop's next item, staged in LDS: ticket, segment record,
// 8 anchors.
constexpr int NXT_REC = 1;
constexpr int NXT_ANC = 1 + WORK_INTS;
constexpr int NXT_INTS = 1 + WORK_INTS + 8;

__device__ __forceinline__ int persistent_items(const DraftArgs& a) {
  return a.queues == 8 ? a.n_work : 8 * a.n_work;
}

__device__ __forceinline__ int persistent_run(const DraftArgs& a, int t) { return a.queues == 8 ? t : t >> 3; }

// Workgroups serving one queue (the grid is a multiple of 8).  Member i of
// a queue takes ticket i first without drawing; drawn tickets start after
// the members'.
__device__ __forceinline__ int persistent_members(const DraftArgs& a) {
  return a.queues == 8 ? (int)(gridDim.x >> 3) : (int)gridDim.x;
}

// Called by one lane: stage ticket t and, if it names an item, that item's
// record and anchors (plain vector loads; the lane waits for them).
__device__ __forceinline__ void stage_next(const DraftArgs& a, int* nxt, int t) {
  nxt[0] = t;
  if (t < persistent_items(a)) {
    const int run = persistent_run(a, t);
    const int4* rec = reinterpret_cast<const int4*>(a.work + WORK_INTS * run);
    const int4* anc = reinterpret_cast<const int4*>(a.seg_anc + 8 * run);
    const int4 r0 = rec[0], r1 = rec[1], a0 = anc[0], a1 = anc[1];
    const int v[16] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w, a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    #pragma unroll
    for (int j = 0; j < 16; ++j) nxt[NXT_REC + j] = v[j];
  }
}

// atomicAdd whose result is read much later: the address carries an
// opaque zero offset, so the compiler issues one plain atomic for the
// calling lanes instead of a wave-aggregated one, whose result it would wait
// for right away.
__device__ __forceinline__ int atomic_add_deferred(int* p, int v) {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return atomicAdd(p + z, v);
}

// Wave w of the workgroup attends blocks 2(w/2) and 2(w/2)+1 of the
// segment's request over key half w%2 of every stage.  INDEXED: context
// rows come through a per-request physical index vector (the append-order
// pool), else they are consecutive rows; the non-indexed instance has no
// ordinary global loads inside the stage loop, so nothing forces a full
// vmcnt drain between ring stages.  KF32: context and block K are fp32.
// No early return: every wave reaches the end, so that the caller may place
// workgroup barriers between items.
template <bool INDEXED, bool KF32>
__device__ __forceinline__ void draft_pair_item(const DraftArgs& a, unsigned char* smem, const DraftSeg& sg, int g,
                                                int item, int* ticket_ctr = nullptr, int* nxt = nullptr,
                                                int tid = -1) {
  using R = PairRing<KF32>;
  TL_DECL
  TL_MARK(0);
  constexpr int KEL = KF32 ? 4 : 2;                 // bytes per K element
  // The thread index: threadIdx.x, or a copy the persistent loop makes
  // opaque per item, so that nothing derived from it is kept live across items.
  if (tid < 0) tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pw = wave >> 1;                         // block pair
  const int kh = wave & 1;                          // key half of each stage
  const int hh = lane >> 5;
  const int n = lane & 31;
  const int r = __builtin_amdgcn_readfirstlane(sg.r);
  const int k0 = __builtin_amdgcn_readfirstlane(sg.k0);
  const int k1 = __builtin_amdgcn_readfirstlane(sg.k1);
  const int pslot = __builtin_amdgcn_readfirstlane(sg.pslot);
  const int b0 = __builtin_amdgcn_readfirstlane(sg.b0);
  const int nb = __builtin_amdgcn_readfirstlane(sg.nb);
  const int amax = __builtin_amdgcn_readfirstlane(sg.amax);
  const bool last = sg.last;
  const int kend = min(k1, amax);
  const bool active = 2 * pw < nb;
  const int bi = n >> 4;
  const int blk = 2 * pw + bi;
  const int tok = (n & 15) >> 1;
  const bool row_ok = blk < nb && tok < BLOCK_ROWS;
  // Context rows visible to each block of the pair (a missing second block
  // copies the first's, so that the pair's limits are the first block's).
  // Persistent mode: the segment's anchors were staged in LDS with its record.
  auto anchor = [&](int j) {
    return nxt ? __builtin_amdgcn_readfirstlane(nxt[NXT_ANC + j]) : ld_const(a.anchors + b0 + j);
  };
  const int anc0 = active ? min(anchor(2 * pw), k1) : 0;
  const int anc1 = 2 * pw + 1 < nb ? min(anchor(2 * pw + 1), k1) : anc0;
  const int vis = row_ok ? (bi ? anc1 : anc0) : 0;
  const int pair_hi = max(anc0, anc1);              // keys at or past this are seen by neither block
  const int full_lim = min(min(anc0, anc1), kend);  // keys below this need no mask
  // Q rows of the tile (rows outside the blocks read row 0 and are zeroed);
  // every load is issued before any is used.
  // Q of the tile: bf16 Q through LDS (q_lds), else loaded here.
  const bool q_lds = R::Q_BYTES > 0 && !a.q_f32;
  bf16x8 qf[8];
  if (!q_lds) {
    const size_t qe = (size_t)(BLOCK_ROWS * (b0 + (row_ok ? blk : 0)) + (row_ok ? tok : 0)) * Q_ROW +
                      (size_t)(2 * g + (n & 1)) * HD + 8 * hh;
    if (a.q_f32) {
      const float* qp = static_cast<const float*>(a.q) + qe;
      f32x4 lo[8], hi[8];
      #pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        lo[ks] = *reinterpret_cast<const f32x4*>(qp + 16 * ks);
        hi[ks] = *reinterpret_cast<const f32x4*>(qp + 16 * ks + 4);
      }
      #pragma unroll
      for (int ks = 0; ks < 8; ++ks) qf[ks] = to_bf16x8(lo[ks], hi[ks]);
    } else {
      #pragma unroll
      for (int ks = 0; ks < 8; ++ks) qf[ks] = ld8(static_cast<const bf16*>(a.q) + qe + 16 * ks);
    }
    // Both forms complete here, before the row select: a select on a branch
    // that skipped the loads would leave registers with loads possibly in
    // flight, and the compiler would wait for them among the ring's loads.
    settle(qf[0], qf[1], qf[2], qf[3], qf[4], qf[5], qf[6], qf[7]);
    #pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = row_ok ? qf[ks] : zero8();
    settle(qf[0], qf[1], qf[2], qf[3], qf[4], qf[5], qf[6], qf[7]);
  }
  const int off1 = __builtin_amdgcn_readfirstlane(sg.off1);
  const int64_t coff = off1 > 0 ? (int64_t)(off1 - 1) : ld_const(a.ctx_off + r);

  const char* kbase = static_cast<const char*>(a.k_ctx) + (size_t)g * a.head_stride * KEL;
  const char* vbase = reinterpret_cast<const char*>(a.v_ctx) + (size_t)g * a.head_stride * 2;
  // Consecutive context: row kk of this request (clamped into range) as a
  // byte address.
  auto ctx_row = [&](const char* base, int el, int kk) -> const char* {
    kk = min(kk, kend - 1);
    return base + (size_t)(coff + kk) * (size_t)a.tok_stride * el;
  };
  // Own row `row` (0..63: pair row/16, block 2(row/16) + (row%16)/8, token
  // min(row%8, 6), clamped to the request's blocks) as an element index.
  auto own_row = [&](int row) {
    const int b = min(2 * (row >> 4) + ((row >> 3) & 1), nb - 1);
    return (size_t)(BLOCK_ROWS * (b0 + b) + min(row & 7, BLOCK_ROWS - 1)) * KV_ROW + (size_t)g * HD;
  };
  const uint32_t smem_lds = lds_address(smem);
  // Indexed context: the physical rows of stage s come through LDS.  Each
  // wave loads its own copy of the stage's DSTEP indices (their low words;
  // the indices lie below 2^31), clamped into range like ctx_row, together
  // with the ring stage s - 2, so that they have landed when stage s issues
  // and no compiler-visible load falls among the ring's loads.
  const uint32_t idx_base = smem_lds + (uint32_t)(R::IDX_OFF + wave * DSTEP * 4);
  auto idx_slot = [&](int step) { return idx_base + (uint32_t)((step % R::STAGES) * DWAVES * DSTEP * 4); };
  auto issue_idx = [&](int step) {
    const int kk = min(k0 + step * DSTEP + lane, kend - 1);
    lds_dma4(a.ctx_idx + coff + kk, __builtin_amdgcn_readfirstlane(idx_slot(step)));
  };
  // One slot of pieces of 1 KiB; wave w issues pieces PER_WAVE*w ..
  // +PER_WAVE-1 (the K/V choice is uniform per piece).
  //  * bf16 K / V piece: rows 4*pr .. +3; lane L fetches row 4*pr + L/16,
  //    16-byte chunk (L%16) ^ swz(row).
  //  * fp32 K piece: rows 2*pr, 2*pr+1; lane L fetches row 2*pr + L/32 at
  //    position p = L%32: floats 4*(2*((p%16) ^ swz(row)) + p/16) .. +3.
  // Context stages swizzle by the stage row, the own rows by row % 16.
  auto fill = [&](uint32_t slot, auto k_src, auto v_src, int sw_mask) {
    #pragma unroll
    for (int i = 0; i < R::PER_WAVE; ++i) {
      const int piece = wave * R::PER_WAVE + i;
      const char* src;
      if (piece < R::K_PIECES) {
        if constexpr (KF32) {
          const int k = 2 * piece + (lane >> 5);
          const int p = lane & 31;
          src = k_src(k) + 16 * (2 * ((p & 15) ^ swz(k & sw_mask)) + (p >> 4));
        } else {
          const int k = 4 * piece + (lane >> 4);
          src = k_src(k) + 16 * ((lane & 15) ^ swz(k & sw_mask));
        }
      } else {
        const int k = 4 * (piece - R::K_PIECES) + (lane >> 4);
        src = v_src(k) + 16 * ((lane & 15) ^ swz(k & sw_mask));
      }
      lds_dma16_nt(src, __builtin_amdgcn_readfirstlane(slot + (uint32_t)(piece * 1024)));
    }
  };
  // Stage `step` of the context: with indices, the indices of stage
  // step + STAGES - 1 load first (into the slot that stage step - 1 has
  // finished with), then the stage's rows at the addresses read from LDS.
  auto issue = [&](int step) {
    const uint32_t slot = smem_lds + (uint32_t)((step % R::STAGES) * R::STAGE_BYTES);
    if constexpr (INDEXED) {
      issue_idx(step + R::STAGES - 1);
      const uint32_t ix = idx_slot(step);
      auto phys = [&](int k) { return (size_t)(uint32_t)*(const lds_i32*)(uintptr_t)(ix + 4 * k); };
      fill(slot, [&](int k) { return kbase + phys(k) * (size_t)a.tok_stride * KEL; },
           [&](int k) { return vbase + phys(k) * (size_t)a.tok_stride * 2; }, 63);
    } else {
      const int ks = k0 + step * DSTEP;
      fill(slot, [&](int k) { return ctx_row(kbase, KEL, ks + k); }, [&](int k) { return ctx_row(vbase, 2, ks + k); },
           63);
    }
  };

  PairState st;
  st.m = -INFINITY;
  st.l = 0.f;
  #pragma unroll
  for (int D = 0; D < 4; ++D) st.o[D] = f32x16{};
  const int n_steps = kend > k0 ? (kend - k0 + DSTEP - 1) / DSTEP : 0;

  // No drain here: a previous item's output stores may still be in flight
  // when this item's ring loads issue.  The ring's counted waits stay exact
  // with them: loads complete in order among themselves, so an older store
  // still pending only lengthens a vmcnt(N) wait, and the compiler's own Q
  // loads above have completed before the first ring load.
  // Persistent mode: lane 0 of wave 1 (a key-half-1 wave, idle once it has
  // handed its state to the merge) draws the workgroup's next ticket when
  // this segment's stream ends (a ticket drawn at the start would reserve
  // the next item for a busy workgroup and undo the longest-first order),
  // then, during the merge, stages that item's record and anchors in LDS.
  const bool fetcher = ticket_ctr && tid == WAVE;
  int next_ticket = 0;
  auto draw = [&]() {
    if (fetcher) next_ticket = atomic_add_deferred(ticket_ctr, 1) + persistent_members(a);
  };
  // Indexed: the first two stages' indices load first of all.
  if constexpr (INDEXED) {
    if (n_steps > 0) {
      issue_idx(0);
      issue_idx(1);
    }
  }
  // bf16 Q rows, issued first: slot row R = 32p + n holds tile row n of
  // pair p (rows with no query read block 0, token 0 and are zeroed later).
  const uint32_t q_lds_row = smem_lds + (uint32_t)(R::Q_OFF + (32 * pw + n) * ROWB);
  if (q_lds) {
    #pragma unroll
    for (int i = 0; i < R::PER_WAVE; ++i) {
      const int piece = wave * R::PER_WAVE + i;
      const int row = 4 * piece + (lane >> 4);
      const int bq = 2 * (row >> 5) + ((row >> 4) & 1);
      const int tq = (row & 15) >> 1;
      const bool ok = bq < nb && tq < BLOCK_ROWS;
      const bf16* src = static_cast<const bf16*>(a.q) + (size_t)(BLOCK_ROWS * (b0 + (ok ? bq : 0)) + (ok ? tq : 0)) * Q_ROW +
                        (size_t)(2 * g + (row & 1)) * HD + 8 * ((lane & 15) ^ swz(row));
      lds_dma16(src, __builtin_amdgcn_readfirstlane(smem_lds + (uint32_t)(R::Q_OFF + piece * 1024)));
    }
  }
  // After a barrier that follows the Q loads' landing.
  auto read_q = [&]() {
    const int sw = swz(32 * pw + n);
    #pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const bf16x8 x = *(const lds_bf16x8*)(uintptr_t)(q_lds_row + (((2 * ks + hh) ^ sw) << 4));
      qf[ks] = row_ok ? x : zero8();
    }
  };

  // Own-block keys (bidirectional within each block), once per request,
  // ahead of the context (their loads share the ring's latency).  The
  // kh = 0 wave of each pair attends them.
  if (last) {
    fill(smem_lds + (uint32_t)R::OWN_SLOT,
         [&](int k) {
           return reinterpret_cast<const char*>(a.k_blk) + own_row(k) * KEL;
         },
         [&](int k) { return reinterpret_cast<const char*>(a.v_blk + own_row(k)); }, 15);
  }
  // Only stages that hold context are loaded, so the number of ring loads
  // still in flight behind a given one is known: all but the newest
  // `behind` stages of LPS loads each (PER_WAVE pieces, and with indices
  // one index load) have landed after wait_stages.
  constexpr int LPS = R::PER_WAVE + (INDEXED ? 1 : 0);
  auto wait_stages = [](int behind) {
    if (behind <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (behind == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPS) : "memory");
    else if (behind == 2 || R::STAGES < 4) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LPS) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * LPS) : "memory");
  };
  static_assert(R::STAGES <= 4, "wait_stages covers at most three stages in flight");
  static_assert(R::STAGES == 3 || !INDEXED, "the index prologue loads two stages");
  const int prologue = min(R::STAGES - 1, n_steps);
  if constexpr (INDEXED) {
    // The first two stages' indices have landed once at most the Q and own
    // row loads issued after them are in flight.
    if (n_steps > 0) {
      const int after = (q_lds ? R::PER_WAVE : 0) + (last ? R::PER_WAVE : 0);
      if (after == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      else if (after == R::PER_WAVE) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(R::PER_WAVE) : "memory");
      else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * R::PER_WAVE) : "memory");
    }
  }
  #pragma unroll
  for (int p = 0; p < R::STAGES - 1; ++p)
    if (p < prologue) issue(p);
  TL_MARK(1);
  if (last) {
    wait_stages(prologue);   // the Q and own rows, issued first, have landed
    asm volatile("s_barrier" ::: "memory");
    TL_MARK(2);
    if (q_lds) read_q();
    if (active && kh == 0) {
      // Register r of a lane in half hh holds block (r/4)%2 of the pair,
      // token 4(r/8) + r%4 (token 7: r = 11, 15); half 1 repeats half 0.
      const TileOffsets oo = own_tile_offsets<R::KROW>(lane);
      const uint32_t own = smem_lds + (uint32_t)R::OWN_SLOT;
      pair_tile<KF32, OWN_V1_XOR, OWN_V1_ADD>(
          st, qf, own + (uint32_t)(16 * pw * R::KROW) + oo.k, own + (uint32_t)(R::K_BYTES + 16 * pw * ROWB) + oo.v,
          true, [&](int rg) { return row_ok && hh == 0 && ((rg >> 2) & 1) == bi && rg != 11 && rg != 15; },
          a.scale_log2);
    }
  }

  const TileOffsets co = ctx_tile_offsets<R::KROW>(lane);
  auto compute = [&](int step) {
    const int kt = k0 + step * DSTEP + 32 * kh;
    if (kt >= pair_hi) return;
    const uint32_t stage = smem_lds + (uint32_t)((step % R::STAGES) * R::STAGE_BYTES);
    // The key of register r is visible iff kt + acc_row(r, hh) < vis.
    const int lim = vis - kt - 8 * hh;
    pair_tile<KF32, CTX_V1_XOR, CTX_V1_ADD>(
        st, qf, stage + (uint32_t)(32 * kh * R::KROW) + co.k, stage + (uint32_t)(R::K_BYTES + 32 * kh * ROWB) + co.v,
        kt + 32 > full_lim, [&](int rg) { return acc_row(rg, 0) < lim; }, a.scale_log2);
  };
  if (n_steps > 0) {
    // Every thread issues exactly PER_WAVE loads per context stage, so at
    // the top of step s the stages issued after stage s number
    // min(n_steps - 1 - s, STAGES - 2).
    auto step = [&](int s) {
      wait_stages(min(n_steps - 1 - s, R::STAGES - 2));
      asm volatile("s_barrier" ::: "memory");
#ifdef DSPARK_TIMELINE
      if (s == 0 && !last) TL_MARK(2);
#endif
      if (s == 0 && q_lds && !last) read_q();
      if (s + R::STAGES - 1 < n_steps) issue(s + R::STAGES - 1);
      if (active) compute(s);
    };
    for (int s = 0; s < n_steps; ++s) step(s);
  }
  // The next ticket is drawn when the stream ends, so that its round trip
  // overlaps the merge below (a draw inside the stream loop, right after the
  // ring's last stage load, made the compiler spill the loop's registers).
  draw();
  asm volatile("s_barrier" ::: "memory");   // every wave is done with the ring and the own rows
  TL_MARK(3);

  // The key halves merge: the kh = 1 wave of each pair leaves its state in
  // the drained ring (register-major, lane-minor), the kh = 0 wave folds it
  // in with the online-softmax rule and writes the result.
  float* mb = reinterpret_cast<float*>(smem + pw * R::MERGE_BYTES);
  if (active && kh == 1) {
    #pragma unroll
    for (int D = 0; D < 4; ++D)
      #pragma unroll
      for (int e = 0; e < 16; ++e) mb[(16 * D + e) * WAVE + lane] = st.o[D][e];
    mb[64 * WAVE + lane] = st.m;
    mb[65 * WAVE + lane] = st.l;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __syncthreads();
  if (fetcher) stage_next(a, nxt, next_ticket);
  if (active && kh == 0) {
    const float m1 = mb[64 * WAVE + lane];
    const float l1 = mb[65 * WAVE + lane];
    const float mt = fmaxf(st.m, m1);
    // Scale factors of the two halves; a half with no visible key
    // (max -inf) contributes nothing.
    const float a0 = st.m == -INFINITY ? 0.f : fast_exp2(st.m - mt);
    const float a1 = m1 == -INFINITY ? 0.f : fast_exp2(m1 - mt);
    st.m = mt;
    st.l = st.l * a0 + l1 * a1;
    #pragma unroll
    for (int D = 0; D < 4; ++D)
      #pragma unroll
      for (int e = 0; e < 16; ++e) st.o[D][e] = st.o[D][e] * a0 + mb[(16 * D + e) * WAVE + lane] * a1;

    const float l = st.l + __shfl_xor(st.l, 32);
    if (blk < nb) {
      if (pslot < 0) {
        if (tok < BLOCK_ROWS) {
          bf16* op = a.out + (size_t)(BLOCK_ROWS * (b0 + blk) + tok) * Q_ROW + (size_t)(2 * g + (n & 1)) * HD + 4 * hh;
          const float inv = 1.0f / l;
          #pragma unroll
          for (int D = 0; D < 4; ++D)
            #pragma unroll
            for (int q = 0; q < 4; ++q) {
              bf16x4 ov;
              #pragma unroll
              for (int e = 0; e < 4; ++e) ov[e] = (bf16)(st.o[D][4 * q + e] * inv);
              *reinterpret_cast<bf16x4*>(op + 32 * D + 8 * q) = ov;
            }
        }
      } else {
        const size_t p = (size_t)(pslot * 8 + g) * a.tmax + blk;
        float* po = a.part_o + (p * 16 + (n & 15)) * HD + 4 * hh;
        #pragma unroll
        for (int D = 0; D < 4; ++D)
          #pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4*>(po + 32 * D + 8 * q) =
                f32x4{st.o[D][4 * q], st.o[D][4 * q + 1], st.o[D][4 * q + 2], st.o[D][4 * q + 3]};
        if (hh == 0) {
          a.part_ml[(p * 16 + (n & 15)) * 2 + 0] = st.m;
          a.part_ml[(p * 16 + (n & 15)) * 2 + 1] = l;
        }
      }
    }
  }
#ifdef DSPARK_TIMELINE
  TL_MARK(4);
  if (threadIdx.x == 0 && blockIdx.x < TL_WGS && item < TL_ITEMS) {
    uint32_t hw, xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    uint64_t* t = tl_stamps + ((size_t)blockIdx.x * TL_ITEMS + item) * TL_WORDS;
    #pragma unroll
    for (int i = 0; i < 5; ++i) t[i] = tl_t[i];
    t[5] = (uint64_t)hw | ((uint64_t)(xcc & 15) << 32) | ((uint64_t)1 << 63);
    t[6] = (uint64_t)(uint32_t)r | ((uint64_t)(uint32_t)(k1 - k0) << 32);
    t[7] = (uint64_t)(uint32_t)nb | ((uint64_t)(uint32_t)n_steps << 16) | ((uint64_t)(last ? 1 : 0) << 32) |
           ((uint64_t)(uint32_t)(pslot >= 0) << 33);
  }
#else
  (void)item;
#endif
}

// With a work list, workgroup (run w, KV head g) runs the segments of run w
// (blockIdx.x = 8w + g).  Without one, workgroup (chunk, KV head) runs one
// fixed chunk of `chunk` context rows, chunks in request order.  Every
// branch is uniform across the workgroup.

// Persistent mode (a.queue): the grid is a fixed set of workgroups (one per
// CU) that take items - (run, KV head) pairs of a plan with one segment per
// run, runs in list order - from device ticket counters, so a CU starts its
// next item as soon as it is done instead of waiting for the hardware
// dispatcher.  Member i of a queue starts with ticket i without drawing;
// later tickets are drawn (counter + members) when the current segment's
// stream ends, and the next item's record and anchors are staged in LDS
// while the current one merges (draft_pair_item), so an item starts without
// a memory round trip.  With one queue, ticket t is run t / 8, head t % 8;
// with a queue per XCD, workgroup b serves head b % 8 (its XCD when
// workgroups are dealt round-robin) and ticket t of that queue is run t.
// Counter layout per queue: {tickets drawn, workgroups done}.  The last
// workgroup of a queue to finish sets both back to zero, so every launch
// finds them zero (the caller zeroes them once, at allocation).  Between
// items the workgroup keeps no state in registers (the item runs at the
// register limit of two waves per SIMD), and each item gets an opaque copy
// of the thread index so that nothing derived from it stays live across
// items.
template <bool INDEXED, bool KF32>
__device__ __forceinline__ void draft_persistent(const DraftArgs& a, unsigned char* smem) {
  static_assert(WORK_INTS == 8, "the staged record is 8 words");
  __shared__ int nxt[NXT_INTS];
  const bool per_head = a.queues == 8;
  int* ctr = a.queue + (per_head ? 2 * (int)(blockIdx.x & 7) : 0);
#ifdef DSPARK_TIMELINE
  const uint64_t tl_entry = tl_now();
#endif
  if (threadIdx.x == WAVE) stage_next(a, nxt, per_head ? (int)(blockIdx.x >> 3) : (int)blockIdx.x);
  __syncthreads();
#ifdef DSPARK_TIMELINE
  const uint64_t tl_first = tl_now();
  int item = 0;
#else
  constexpr int item = 0;
#endif
  for (;;) {
    const int t = __builtin_amdgcn_readfirstlane(nxt[0]);
    if (t >= persistent_items(a)) break;
    int w[WORK_INTS];
    #pragma unroll
    for (int j = 0; j < WORK_INTS; ++j) w[j] = __builtin_amdgcn_readfirstlane(nxt[NXT_REC + j]);
    const DraftSeg sg{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[2] >= w[6], w[7]};
    const int g = per_head ? (int)(blockIdx.x & 7) : (t & 7);
    int tid;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
    draft_pair_item<INDEXED, KF32>(a, smem, sg, g, item, ctr, nxt, tid);
#ifdef DSPARK_TIMELINE
    ++item;
#endif
    __syncthreads();   // the next segment refills the ring the last one read; publishes nxt
  }
#ifdef DSPARK_TIMELINE
  const uint64_t tl_left = tl_now();
#endif
  if (threadIdx.x == 0) {
    const int members = persistent_members(a);
    const int finished = atomicAdd(ctr + 1, 1);
    if (finished == members - 1) {   // every member has drawn its last ticket: reset for the next launch
      atomicExch(ctr, 0);
      atomicExch(ctr + 1, 0);
    }
#ifdef DSPARK_TIMELINE
    if (blockIdx.x < TL_WGS) {
      uint64_t* wg = tl_wg + 4 * (size_t)blockIdx.x;
      wg[0] = tl_entry;
      wg[1] = tl_first;
      wg[2] = tl_left;
      wg[3] = tl_now() | ((uint64_t)1 << 63);
    }
#endif
  }
}

template <bool INDEXED, bool KF32>
__global__ __launch_bounds__(DWAVES * WAVE) void draft_attn_persistent_kernel(DraftArgs a) {
  // 1 KiB alignment: tile offsets are XORed into LDS addresses.
  __shared__ __attribute__((aligned(1024))) unsigned char smem[PairRing<KF32>::SMEM + (INDEXED ? PairRing<KF32>::IDX_BYTES : 0)];
  draft_persistent<INDEXED, KF32>(a, smem);
}

template <bool INDEXED, bool KF32>
__global__ __launch_bounds__(DWAVES * WAVE) void draft_attn_kernel(DraftArgs a) {
  // 1 KiB alignment: tile offsets are XORed into LDS addresses.
  __shared__ __attribute__((aligned(1024))) unsigned char smem[PairRing<KF32>::SMEM + (INDEXED ? PairRing<KF32>::IDX_BYTES : 0)];
  const int g = blockIdx.x & 7;
  if (a.work) {
    // The run's range and (speculatively) record number `run`, which is the
    // run's only record in a plan of one segment per run, load together.
    const int run = blockIdx.x >> 3;
    const int32_t* range = a.work + WORK_INTS * a.n_work + run;
    const int32_t* spec = a.work + WORK_INTS * min(run, a.n_work - 1);
    int w[WORK_INTS];
    #pragma unroll
    for (int j = 0; j < WORK_INTS; ++j) w[j] = ld_const(spec + j);
    const int lo = min(max(ld_const(range), 0), a.n_work);     // clamped: never past the records
    const int hi = min(max(ld_const(range + 1), lo), a.n_work);
    for (int i = lo; i < hi; ++i) {
      if (i != run) {
        #pragma unroll
        for (int j = 0; j < WORK_INTS; ++j) w[j] = ld_const(a.work + WORK_INTS * i + j);
      }
      const DraftSeg sg{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[2] >= w[6], w[7]};
      draft_pair_item<INDEXED, KF32>(a, smem, sg, g, i - lo);
      __syncthreads();   // the next segment refills the ring the last one read
    }
    return;
  }
  int r, first;
  locate_chunk(nullptr, a.ctx_len, a.n_req, a.chunk, blockIdx.x >> 3, r, first);
  if (r < 0) return;
  const int c = (blockIdx.x >> 3) - first;
  const int ctx = a.ctx_len[r];
  const int nch = chunks_for(ctx, a.chunk);
  const int b0 = a.cu_b[r];
  const int nb = a.cu_b[r + 1] - b0;
  int amax = 0;
  for (int b = 0; b < nb; ++b) amax = max(amax, a.anchors[b0 + b]);
  const DraftSeg sg{r, c * a.chunk, min(c * a.chunk + a.chunk, ctx), nch > 1 ? first + c : -1, b0, nb, amax,
                    c == nch - 1, 0};
  draft_pair_item<INDEXED, KF32>(a, smem, sg, g, 0);
}

// ---------------------------------------------------------------------------
// split-K merge: one workgroup per (request, KV head, tile) with >1 chunk
// ---------------------------------------------------------------------------
struct MergeArgs {
  const int32_t* req;      // optional [B][4]: chunk base, chunk count, first output row / block, rows / blocks
  const int32_t* cu_q;     // varlen/verify
  const int32_t* cu_k;     // varlen/verify chunk counts
  const int32_t* ctx_len;  // draft chunk counts
  const int32_t* cu_b;     // draft block offsets
  const float* part_o;
  const float* part_ml;
  bf16* out;
  int n_req;
  int chunk;
  int tmax;
  int draft;
};

// Workgroup (8r + g, t) merges request r, KV head g, row tile t (draft: block
// t) of a request held by more than one chunk: its id is
// g mod 8, so it runs on the XCD whose L2 holds the partials that the chunk
// kernel's head-g workgroups (ids = g mod 8 as well) just wrote.
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  const int r = blockIdx.x >> 3;
  const int g = blockIdx.x & 7;
  const int t = blockIdx.y;
  int len, out_row0, rows_valid;
  if (a.req) {
    const int32_t* m = a.req + REQ_INTS * r;
    const int nch = m[1];
    if (nch == 1) return;
    int row0, valid;
    if (a.draft) {
      if (t >= m[3]) return;
      row0 = BLOCK_ROWS * (m[2] + t);
      valid = BLOCK_ROWS;
    } else {
      if (8 * t >= m[3]) return;
      row0 = m[2] + 8 * t;
      valid = min(8, m[3] - 8 * t);
    }
    const int tid = threadIdx.x;
    const int row = tid >> 4;
    const int d0 = (tid & 15) * 8;
    if ((row >> 1) >= valid) return;
    float acc[8];
    float L;
    merge_partials<8>(a.part_o, a.part_ml, (size_t)(m[0] * 8 + g) * a.tmax + t, (size_t)8 * a.tmax, nch, row, d0,
                      acc, L);
    bf16x8 ov;
    #pragma unroll
    for (int i = 0; i < 8; ++i) ov[i] = (bf16)(acc[i] / L);
    *reinterpret_cast<bf16x8*>(a.out + (size_t)(row0 + (row >> 1)) * Q_ROW + (size_t)(2 * g + (row & 1)) * HD + d0) = ov;
    return;
  }
  if (a.draft) {
    const int b0 = a.cu_b[r];
    if (t >= a.cu_b[r + 1] - b0) return;
    len = a.ctx_len[r];
    out_row0 = BLOCK_ROWS * (b0 + t);
    rows_valid = BLOCK_ROWS;
  } else {
    const int q0 = a.cu_q[r];
    const int ql = a.cu_q[r + 1] - q0;
    if (8 * t >= ql) return;
    len = a.cu_k[r + 1] - a.cu_k[r];
    out_row0 = q0 + 8 * t;
    rows_valid = min(8, ql - 8 * t);
  }
  const int nch = chunks_for(len, a.chunk);
  if (nch == 1) return;
  const int first = chunk_base(a.draft ? nullptr : a.cu_k, a.draft ? a.ctx_len : nullptr, r, a.chunk);
  const int tid = threadIdx.x;
  const int row = tid >> 4;
  const int d0 = (tid & 15) * 8;
  if ((row >> 1) >= rows_valid) return;
  float acc[8];
  float L;
  merge_partials<8>(a.part_o, a.part_ml, (size_t)(first * 8 + g) * a.tmax + t, (size_t)8 * a.tmax, nch, row, d0, acc, L);
  bf16x8 ov;
  #pragma unroll
  for (int i = 0; i < 8; ++i) ov[i] = (bf16)(acc[i] / L);
  *reinterpret_cast<bf16x8*>(a.out + (size_t)(out_row0 + (row >> 1)) * Q_ROW + (size_t)(2 * g + (row & 1)) * HD + d0) = ov;
}

}  // namespace dspark

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {

using namespace dspark;

constexpr float LOG2E = 1.4426950408889634f;

// Workgroups resident at once for the varlen/verify kernel (2 per CU at its
// register budget), times the number of row tiles sharing the machine.
unsigned persistent_grid(int n_slots, int tiles) {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  const int64_t resident = std::max<int64_t>(8, (int64_t)cus * 2 / std::max(tiles, 1) / 8 * 8);
  return (unsigned)std::min<int64_t>(n_slots, resident);
}

int64_t n_chunk_items(int n_req, int64_t rows_bound, int chunk) {
  return (rows_bound + chunk - 1) / chunk + n_req;
}

// [part_o: items x 16 x 128 f32][part_ml: items x 16 x 2 f32]
int64_t workspace_bytes(int n_req, int64_t rows_bound, int tiles, int chunk) {
  const int64_t items = n_chunk_items(n_req, rows_bound, chunk) * HKV * tiles;
  return items * 16 * (HD + 2) * (int64_t)sizeof(float);
}

int launch_merge(const MergeArgs& m, int n_req, int tiles, hipStream_t s) {
  DSPARK_REQUIRE((int64_t)n_req * HKV <= 0x7fffffffLL, "too many requests for the merge grid (%d)", n_req);
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)n_req * HKV, tiles), dim3(256), 0, s, m);
  return launch_status("merge_kernel");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_shape(int n_req, int64_t rows_bound, int tiles, int chunk, float scale) {
  DSPARK_REQUIRE(n_req >= 1, "n_req must be >= 1 (got %d)", n_req);
  DSPARK_REQUIRE(rows_bound >= 0, "key row bound must be >= 0");
  DSPARK_REQUIRE(tiles >= 1 && tiles <= 65535, "row tiles out of range (%d)", tiles);
  DSPARK_REQUIRE(chunk >= 32 && chunk % 32 == 0 && chunk <= (1 << 20), "chunk must be a multiple of 32 in [32, 2^20] (got %d)", chunk);
  DSPARK_REQUIRE(scale > 0.f && scale < 1e30f, "scale must be positive and finite");
  const int64_t items = n_chunk_items(n_req, rows_bound, chunk) * HKV;
  DSPARK_REQUIRE(items <= 0x7fffffffLL, "too many chunk work items (%lld)", (long long)items);
  return OK;
}

int check_common(int n_req, int64_t rows_bound, int tiles, int chunk, float scale,
                 int64_t ws_bytes, const void* ws) {
  const int rc = check_shape(n_req, rows_bound, tiles, chunk, scale);
  if (rc != OK) return rc;
  const int64_t need = workspace_bytes(n_req, rows_bound, tiles, chunk);
  DSPARK_REQUIRE(ws_bytes >= need, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)need);
  DSPARK_REQUIRE(need == 0 || (ws != nullptr && aligned16(ws)), "workspace must be a 16-byte aligned device pointer");
  return OK;
}

}  // namespace

extern "C" int64_t dspark_attn_workspace_bytes(int n_req, int64_t key_rows_bound, int row_tiles, int chunk) {
  if (n_req < 1 || key_rows_bound < 0 || row_tiles < 1 || chunk < 32) return -1;
  return workspace_bytes(n_req, key_rows_bound, row_tiles, chunk);
}

namespace {

// Shared by the varlen and verification entry points: argument checks that
// depend on the dispatch form, the split-K workspace layout and both launches.
// With a work list the partial slots are bounded by its record count, else by
// the fixed-chunk bound of key_rows_bound.
template <bool VERIFY>
int varlen_launch(VarlenArgs& a, int64_t key_rows_bound, int max_q, float scale, int chunk, const int32_t* work,
                  int n_work, int n_groups, void* workspace, int64_t workspace_bytes_, void* stream, const char* what) {
  DSPARK_REQUIRE(max_q >= 1, "max_q must be >= 1");
  DSPARK_REQUIRE(!work || (n_work >= 1 && n_groups >= 8 && n_groups <= (1 << 24) && n_groups % 8 == 0),
                 "a work list needs n_work >= 1 and n_groups a multiple of 8 in [8, 2^24]");
  const int tiles = (max_q + 7) / 8;
  int rc = check_shape(work ? n_work : a.n_req, work ? 0 : key_rows_bound, tiles, chunk, scale);
  if (rc != OK) return rc;
  const int64_t n_cl = work ? (int64_t)n_work : n_chunk_items(a.n_req, key_rows_bound, chunk);
  const int64_t need = workspace_bytes(work ? n_work : a.n_req, work ? 0 : key_rows_bound, tiles, chunk);
  DSPARK_REQUIRE(workspace_bytes_ >= need, "workspace too small: %lld < %lld bytes", (long long)workspace_bytes_,
                 (long long)need);
  DSPARK_REQUIRE(need == 0 || (workspace != nullptr && aligned16(workspace)),
                 "workspace must be a 16-byte aligned device pointer");
  a.work = work;
  a.n_work = n_work;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = a.part_o + n_cl * HKV * tiles * 16 * HD;
  a.chunk = chunk;
  a.tmax = tiles;
  a.scale_log2 = scale * LOG2E;
  a.n_slots = (int)(n_cl * HKV);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = work ? (unsigned)n_groups * HKV : persistent_grid(a.n_slots, tiles);
  hipLaunchKernelGGL(varlen_attn_kernel<VERIFY>, dim3(grid, tiles), dim3(256), 0, s, a);
  rc = launch_status(what);
  if (rc != OK) return rc;
  MergeArgs m{work ? work + WORK_INTS * n_work + n_groups + 1 : nullptr, a.cu_q, a.cu_k, nullptr, nullptr, a.part_o,
              a.part_ml, a.out, a.n_req, chunk, tiles, 0};
  return launch_merge(m, a.n_req, tiles, s);
}

}  // namespace

extern "C" int dspark_varlen_attn_fwd(const void* q, const void* k, const void* v,
                                      const int32_t* cu_q, const int32_t* cu_k, int n_req,
                                      int64_t q_rows, int64_t k_rows, int max_q, int causal,
                                      float scale, int chunk, const int32_t* work, int n_work, int n_groups,
                                      void* out, void* workspace,
                                      int64_t workspace_bytes_, void* stream) {
  clear_error();
  DSPARK_REQUIRE(q && k && v && cu_q && cu_k && out, "null pointer argument");
  DSPARK_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), "Q/K/V/out must be 16-byte aligned");
  DSPARK_REQUIRE(q_rows >= 1 && k_rows >= 1, "Q and K must be nonempty");
  DSPARK_REQUIRE(max_q >= 1 && max_q <= q_rows, "max_q must be in [1, q_rows]");
  DSPARK_REQUIRE(n_req >= 1, "n_req must be >= 1 (got %d)", n_req);
  VarlenArgs a{};
  a.q = static_cast<const bf16*>(q);
  a.k_a = static_cast<const bf16*>(k);
  a.v_a = static_cast<const bf16*>(v);
  a.k_b = a.k_a;
  a.v_b = a.v_a;
  a.cu_q = cu_q;
  a.cu_k = cu_k;
  a.slots = nullptr;
  a.slot_stride = 0;
  a.a_tok_stride = KV_ROW;
  a.a_head_stride = HD;
  a.out = static_cast<bf16*>(out);
  a.n_req = n_req;
  a.causal = causal ? 1 : 0;
  return varlen_launch<false>(a, k_rows, max_q, scale, chunk, work, n_work, n_groups, workspace, workspace_bytes_,
                              stream, "varlen_attn_kernel");
}

namespace {
int verify_launch(const void* q, const void* k_res, const void* v_res, const void* k_b, const void* v_b,
                  void* stage_k, void* stage_v, const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                  int n_req, int64_t slot_stride, int64_t tok_stride, int64_t head_stride,
                  int64_t key_rows_bound, int max_q, float scale, int chunk,
                  const int32_t* work, int n_work, int n_groups, void* out, void* workspace,
                  int64_t workspace_bytes_, void* stream) {
  DSPARK_REQUIRE(q && k_res && v_res && k_b && v_b && cu_q && cu_k && slots && out, "null pointer argument");
  DSPARK_REQUIRE(aligned16(q) && aligned16(k_res) && aligned16(v_res) && aligned16(k_b) && aligned16(v_b) && aligned16(out) &&
                 aligned16(stage_k) && aligned16(stage_v),
                 "Q/K/V/out must be 16-byte aligned");
  DSPARK_REQUIRE(slot_stride >= 0 && tok_stride >= HD && tok_stride % 8 == 0 && head_stride >= HD && head_stride % 8 == 0,
                 "resident strides must be multiples of 8 elements (token/head strides >= 128)");
  DSPARK_REQUIRE(n_req >= 1, "n_req must be >= 1 (got %d)", n_req);
  DSPARK_REQUIRE(key_rows_bound >= 0, "key row bound must be >= 0");
  VarlenArgs a{};
  a.q = static_cast<const bf16*>(q);
  a.k_a = static_cast<const bf16*>(k_res);
  a.v_a = static_cast<const bf16*>(v_res);
  a.k_b = static_cast<const bf16*>(k_b);
  a.v_b = static_cast<const bf16*>(v_b);
  a.stage_k = static_cast<bf16*>(stage_k);
  a.stage_v = static_cast<bf16*>(stage_v);
  a.cu_q = cu_q;
  a.cu_k = cu_k;
  a.slots = slots;
  a.slot_stride = slot_stride;
  a.a_tok_stride = tok_stride;
  a.a_head_stride = head_stride;
  a.out = static_cast<bf16*>(out);
  a.n_req = n_req;
  a.causal = 1;
  return varlen_launch<true>(a, key_rows_bound, max_q, scale, chunk, work, n_work, n_groups, workspace,
                             workspace_bytes_, stream, "verify_attn_kernel");
}
}  // namespace

extern "C" int dspark_verify_attn_fwd(const void* q, const void* k_res, const void* v_res,
                                      const void* k_scr, const void* v_scr,
                                      const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                                      int n_req, int64_t slot_stride, int64_t tok_stride, int64_t head_stride,
                                      int64_t key_rows_bound, int max_q, float scale, int chunk,
                                      const int32_t* work, int n_work, int n_groups, void* out, void* workspace,
                                      int64_t workspace_bytes_, void* stream) {
  clear_error();
  return verify_launch(q, k_res, v_res, k_scr, v_scr, nullptr, nullptr, cu_q, cu_k, slots, n_req, slot_stride,
                       tok_stride, head_stride, key_rows_bound, max_q, scale, chunk, work, n_work, n_groups, out,
                       workspace, workspace_bytes_, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free verification attention: the split-K partials live in a
// file-scope device array instead of a caller workspace.  Each GPU the
// library runs on holds its own copy of the array (NOALLOC_SCRATCH_BYTES)
// until the process ends; every call on that GPU shares it.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t NOALLOC_SCRATCH_BYTES = 32ll << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
std::atomic<void*> g_scratch_ptr[NOALLOC_MAX_DEVICES];
std::mutex g_scratch_lock;

// Device address of `scratch` on the current device, resolved once per
// device with that device current.  The array's name is only a host-side
// handle: kernels get this address, never the symbol.
int scratch_address(void** out) {
  int dev = -1;
  DSPARK_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < NOALLOC_MAX_DEVICES,
                 "no usable current HIP device (need an index below %d)", NOALLOC_MAX_DEVICES);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
        return HIP_FAILURE;
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return OK;
}
}  // namespace

extern "C" int64_t dspark_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int dspark_verify_attn_fwd_noalloc(const void* q, const void* k_res, const void* v_res,
                                              const void* k_scr, const void* v_scr,
                                              const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                                              int n_req, int64_t slot_stride, int64_t tok_stride,
                                              int64_t head_stride, int64_t key_rows_bound, int max_q, float scale,
                                              int chunk, const int32_t* work, int n_work, int n_groups, void* out,
                                              void* stream) {
  clear_error();
  DSPARK_REQUIRE(q && k_res && v_res && k_scr && v_scr && cu_q && cu_k && slots && out, "null pointer argument");
  DSPARK_REQUIRE(max_q >= 1, "max_q must be >= 1");
  const int tiles = (max_q + 7) / 8;
  const int64_t need = work ? dspark_attn_workspace_bytes(n_work, 0, tiles, chunk)
                            : dspark_attn_workspace_bytes(n_req, key_rows_bound, tiles, chunk);
  DSPARK_REQUIRE(need >= 0, "invalid request, key bound, row tile or chunk sizes");
  DSPARK_REQUIRE(need <= NOALLOC_SCRATCH_BYTES,
                 "split-K partials need %lld bytes, more than the %lld-byte static scratch of the allocation-free "
                 "entry point (use dspark_verify_attn_fwd with a workspace)",
                 (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != OK) return rc;
  return verify_launch(q, k_res, v_res, k_scr, v_scr, nullptr, nullptr, cu_q, cu_k, slots, n_req, slot_stride,
                       tok_stride, head_stride, key_rows_bound, max_q, scale, chunk, work, n_work, n_groups, out,
                       ws, NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int dspark_verify_attn_staged_fwd(const void* q, const void* k_res, const void* v_res,
                                             const void* k_new, const void* v_new, void* k_scr, void* v_scr,
                                             const int32_t* cu_q, const int32_t* cu_k, const int32_t* slots,
                                             int n_req, int64_t slot_stride, int64_t tok_stride, int64_t head_stride,
                                             int64_t key_rows_bound, int max_q, float scale, int chunk,
                                             const int32_t* work, int n_work, int n_groups, void* out, void* workspace,
                                             int64_t workspace_bytes_, void* stream) {
  clear_error();
  DSPARK_REQUIRE(k_scr && v_scr, "null pointer argument");
  DSPARK_REQUIRE(k_new != k_scr && v_new != v_scr, "new rows and scratch must be distinct buffers");
  return verify_launch(q, k_res, v_res, k_new, v_new, k_scr, v_scr, cu_q, cu_k, slots, n_req, slot_stride,
                       tok_stride, head_stride, key_rows_bound, max_q, scale, chunk, work, n_work, n_groups, out,
                       workspace, workspace_bytes_, stream);
}

extern "C" int dspark_draft_attn_fwd(const void* q, int q_dtype, const void* k_ctx, const void* v_ctx,
                                     int k_dtype, const int64_t* ctx_idx, const int64_t* ctx_off,
                                     const int32_t* ctx_len, int64_t tok_stride, int64_t head_stride,
                                     const void* k_blk, const void* v_blk,
                                     const int32_t* cu_blocks, const int32_t* anchors,
                                     int n_req, int64_t ctx_rows_bound, int max_blocks, float scale, int chunk,
                                     const int32_t* work, int n_work, int n_groups,
                                     int workgroups, int queues, int32_t* queue, const int32_t* seg_anchors,
                                     void* out, void* workspace, int64_t workspace_bytes_, void* stream) {
  clear_error();
  DSPARK_REQUIRE(q && k_ctx && v_ctx && ctx_off && ctx_len && k_blk && v_blk && cu_blocks && anchors && out,
                 "null pointer argument");
  DSPARK_REQUIRE(workgroups == 0 || (work && aligned16(work) && queue && aligned16(queue) && seg_anchors &&
                                     aligned16(seg_anchors) && (queues == 1 || queues == 8) && workgroups >= 8 &&
                                     workgroups % 8 == 0 && workgroups <= (1 << 16) && n_work == n_groups),
                 "persistent mode needs a 16-byte aligned work list of one segment per run with its segment "
                 "anchors, a 16-byte aligned queue buffer, queues 1 or 8 and workgroups a multiple of 8 in "
                 "[8, 65536]");
  DSPARK_REQUIRE(aligned16(q) && aligned16(k_ctx) && aligned16(v_ctx) && aligned16(k_blk) && aligned16(v_blk) && aligned16(out),
                 "Q/K/V/out must be 16-byte aligned");
  DSPARK_REQUIRE(tok_stride >= HD && tok_stride % 8 == 0 && head_stride >= HD && head_stride % 8 == 0,
                 "context strides must be multiples of 8 elements and >= 128");
  DSPARK_REQUIRE((q_dtype == 0 || q_dtype == 1) && (k_dtype == 0 || k_dtype == 1),
                 "q_dtype and k_dtype must be 0 (bf16) or 1 (fp32)");
  DSPARK_REQUIRE(max_blocks >= 1 && max_blocks <= MAX_BLOCKS,
                 "max_blocks must be in [1, %d] (got %d)", MAX_BLOCKS, max_blocks);
  DSPARK_REQUIRE(chunk % CHUNK_ALIGN == 0, "draft chunk must be a multiple of %d", CHUNK_ALIGN);
  DSPARK_REQUIRE(n_req >= 1, "n_req must be >= 1 (got %d)", n_req);
  DSPARK_REQUIRE(!work || (n_work >= 1 && n_groups >= 1 && n_groups <= (1 << 24)),
                 "a work list needs n_work >= 1 and n_groups in [1, 2^24]");
  int rc = check_shape(work ? n_work : n_req, work ? 0 : ctx_rows_bound, max_blocks, chunk, scale);
  if (rc != OK) return rc;
  const int64_t n_cl = work ? (int64_t)n_work : n_chunk_items(n_req, ctx_rows_bound, chunk);
  const int64_t need = workspace_bytes(work ? n_work : n_req, work ? 0 : ctx_rows_bound, max_blocks, chunk);
  DSPARK_REQUIRE(workspace_bytes_ >= need, "workspace too small: %lld < %lld bytes", (long long)workspace_bytes_,
                 (long long)need);
  DSPARK_REQUIRE(need == 0 || (workspace != nullptr && aligned16(workspace)),
                 "workspace must be a 16-byte aligned device pointer");
  DraftArgs a{};
  a.q = q;
  a.q_f32 = q_dtype;
  a.k_ctx = k_ctx;
  a.v_ctx = static_cast<const bf16*>(v_ctx);
  a.ctx_idx = ctx_idx;
  a.ctx_off = ctx_off;
  a.ctx_len = ctx_len;
  a.k_blk = k_blk;
  a.v_blk = static_cast<const bf16*>(v_blk);
  a.cu_b = cu_blocks;
  a.anchors = anchors;
  a.out = static_cast<bf16*>(out);
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = a.part_o + n_cl * HKV * max_blocks * 16 * HD;
  a.tok_stride = tok_stride;
  a.head_stride = head_stride;
  a.work = work;
  a.queue = workgroups ? queue : nullptr;
  a.seg_anc = seg_anchors;
  a.n_work = n_work;
  a.n_runs = n_groups;
  a.queues = queues;
  a.n_req = n_req;
  a.chunk = chunk;
  a.tmax = max_blocks;
  a.scale_log2 = scale * LOG2E;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t grid = workgroups ? (int64_t)workgroups : work ? (int64_t)n_groups * HKV : n_cl * HKV;
  DSPARK_REQUIRE(grid <= 0x7fffffffLL, "grid too large");
  const dim3 blocks((unsigned)grid), threads(DWAVES * WAVE);
  if (workgroups) {
    if (ctx_idx && k_dtype)
      hipLaunchKernelGGL((draft_attn_persistent_kernel<true, true>), blocks, threads, 0, s, a);
    else if (ctx_idx)
      hipLaunchKernelGGL((draft_attn_persistent_kernel<true, false>), blocks, threads, 0, s, a);
    else if (k_dtype)
      hipLaunchKernelGGL((draft_attn_persistent_kernel<false, true>), blocks, threads, 0, s, a);
    else
      hipLaunchKernelGGL((draft_attn_persistent_kernel<false, false>), blocks, threads, 0, s, a);
  } else if (ctx_idx && k_dtype)
    hipLaunchKernelGGL((draft_attn_kernel<true, true>), blocks, threads, 0, s, a);
  else if (ctx_idx)
    hipLaunchKernelGGL((draft_attn_kernel<true, false>), blocks, threads, 0, s, a);
  else if (k_dtype)
    hipLaunchKernelGGL((draft_attn_kernel<false, true>), blocks, threads, 0, s, a);
  else
    hipLaunchKernelGGL((draft_attn_kernel<false, false>), blocks, threads, 0, s, a);
  rc = launch_status("draft_attn_kernel");
  if (rc != OK) return rc;
  MergeArgs m{work ? work + WORK_INTS * n_work + n_groups + 1 : nullptr, nullptr, nullptr, ctx_len, cu_blocks,
              a.part_o, a.part_ml, a.out, n_req, chunk, max_blocks, 1};
  return launch_merge(m, n_req, max_blocks, s);
}

#ifdef DSPARK_TIMELINE
// Timeline build only: copy the per-workgroup draft stamps (TL_WGS x
// TL_ITEMS records of TL_WORDS words) to host memory, then clear them.
// Synchronous (waits for the device).  Not part of the product ABI.
extern "C" int dspark_timeline_fetch(void* host, int64_t bytes) {
  clear_error();
  const int64_t have = (int64_t)sizeof(uint64_t) * TL_WGS * TL_ITEMS * TL_WORDS;
  DSPARK_REQUIRE(host && bytes == have, "need a host buffer of exactly %lld bytes", (long long)have);
  DSPARK_REQUIRE(hipDeviceSynchronize() == hipSuccess, "device synchronisation failed");
  DSPARK_REQUIRE(hipMemcpyFromSymbol(host, HIP_SYMBOL(tl_stamps), (size_t)have, 0, hipMemcpyDeviceToHost) == hipSuccess,
                 "timeline copy failed");
  void* dev = nullptr;
  DSPARK_REQUIRE(hipGetSymbolAddress(&dev, HIP_SYMBOL(tl_stamps)) == hipSuccess && dev, "timeline symbol lookup failed");
  DSPARK_REQUIRE(hipMemset(dev, 0, (size_t)have) == hipSuccess, "timeline clear failed");
  return OK;
}

extern "C" int64_t dspark_timeline_bytes(void) {
  return (int64_t)sizeof(uint64_t) * TL_WGS * TL_ITEMS * TL_WORDS;
}

// The verification workgroup stamps (TL_WGS x 4 words), then cleared.
extern "C" int dspark_timeline_fetch_verify(void* host, int64_t bytes) {
  clear_error();
  const int64_t have = (int64_t)sizeof(uint64_t) * TL_WGS * 4;
  DSPARK_REQUIRE(host && bytes == have, "need a host buffer of exactly %lld bytes", (long long)have);
  DSPARK_REQUIRE(hipDeviceSynchronize() == hipSuccess, "device synchronisation failed");
  DSPARK_REQUIRE(hipMemcpyFromSymbol(host, HIP_SYMBOL(tl_vwg), (size_t)have, 0, hipMemcpyDeviceToHost) == hipSuccess,
                 "timeline copy failed");
  void* dev = nullptr;
  DSPARK_REQUIRE(hipGetSymbolAddress(&dev, HIP_SYMBOL(tl_vwg)) == hipSuccess && dev, "timeline symbol lookup failed");
  DSPARK_REQUIRE(hipMemset(dev, 0, (size_t)have) == hipSuccess, "timeline clear failed");
  return OK;
}

// The persistent-mode workgroup stamps (TL_WGS x 4 words), then cleared.
extern "C" int dspark_timeline_fetch_wg(void* host, int64_t bytes) {
  clear_error();
  const int64_t have = (int64_t)sizeof(uint64_t) * TL_WGS * 4;
  DSPARK_REQUIRE(host && bytes == have, "need a host buffer of exactly %lld bytes", (long long)have);
  DSPARK_REQUIRE(hipDeviceSynchronize() == hipSuccess, "device synchronisation failed");
  DSPARK_REQUIRE(hipMemcpyFromSymbol(host, HIP_SYMBOL(tl_wg), (size_t)have, 0, hipMemcpyDeviceToHost) == hipSuccess,
                 "timeline copy failed");
  void* dev = nullptr;
  DSPARK_REQUIRE(hipGetSymbolAddress(&dev, HIP_SYMBOL(tl_wg)) == hipSuccess && dev, "timeline symbol lookup failed");
  DSPARK_REQUIRE(hipMemset(dev, 0, (size_t)have) == hipSuccess, "timeline clear failed");
  return OK;
}
#endif
