// Persistent target KV transaction kernels for gfx950.
//
//   txn_metadata : device restatement of PersistentTargetKV.begin's host
//                  list building (dspark_qwen/persistent_target_kv.py:392-411)
//                  from per-request (slot, context, query) triples.  Produces
//                  the seven workspace arrays bit-exactly, tail included.
//   kv_stage     : copy a layer's new K/V rows into scratch
//                  (persistent_target_kv.py:436-437).
//   kv_commit    : copy every layer's accepted prefix scratch rows into the
//                  resident slots in one launch (persistent_target_kv.py:479-483);
//                  rows beyond the accepted prefix are never copied (rollback).
//   kv_gather    : the capacity-length K/V of prepare_attention
//                  (persistent_target_kv.py:452-459) in one pass: committed
//                  rows from resident, new rows from scratch, tail zeroed.
//
// The copy kernels move 16-byte vectors.  The resident store is addressed
// through byte strides, so both its head-major layout [slots, H, cap, D]
// (PersistentTargetKV's: one contiguous stream per (slot, KV head)) and a
// token-major layout work; scratch and outputs are token-major rows.
#include "common.h"

namespace dspark {

constexpr int MAX_SCAN = 4096;   // requests per transaction handled by the block scan

// Exclusive block scan of a[0..n) (n <= MAX_SCAN) into out[0..n] (out[n] = total),
// executed by all 256 threads of the workgroup.
__device__ void block_exclusive_scan(const int32_t* vals, int n, int32_t* out, int32_t* tmp) {
  // 256 threads: each sums a run of `per` values, the runs are scanned with
  // wave shuffles plus the 4 wave totals, then each thread writes its run.
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int per = (n + 255) / 256;
  const int beg = min(n, tid * per);
  const int end = min(n, beg + per);
  int s = 0;
  for (int i = beg; i < end; ++i) s += vals[i];
  int incl = s;
  #pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) incl += t;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int run = incl - s;
  for (int w = 0; w < wave; ++w) run += tmp[w];
  for (int i = beg; i < end; ++i) {
    out[i] = run;
    run += vals[i];
  }
  if (tid == 0) out[n] = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  __syncthreads();
}

struct TxnArgs {
  const int32_t* req;        // [3][B]: slot, context, query per request
  int64_t* committed_idx;    // [kcap]
  int64_t* scratch_idx;      // [kcap]
  uint8_t* from_scratch;     // [kcap]
  uint8_t* valid;            // [kcap]
  int64_t* positions;        // [nq]
  int32_t* cu_q;             // [B+1]
  int32_t* cu_k;             // [B+1]
  int64_t ctx_capacity;
  int64_t kcap;
  int64_t nq;
  int n_req;
};

__global__ __launch_bounds__(256) void txn_metadata_kernel(TxnArgs a) {
  __shared__ int32_t s_len[MAX_SCAN];
  __shared__ int32_t s_cuk[MAX_SCAN + 1];
  __shared__ int32_t s_cuq[MAX_SCAN + 1];
  __shared__ int32_t s_tmp[256];
  const int B = a.n_req;
  const int32_t* slot = a.req;
  const int32_t* ctx = a.req + B;
  const int32_t* ql = a.req + 2 * B;
  for (int i = threadIdx.x; i < B; i += 256) s_len[i] = ctx[i] + ql[i];
  __syncthreads();
  block_exclusive_scan(s_len, B, s_cuk, s_tmp);
  for (int i = threadIdx.x; i < B; i += 256) s_len[i] = ql[i];
  __syncthreads();
  block_exclusive_scan(s_len, B, s_cuq, s_tmp);

  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i <= B; i += 256) {
      a.cu_q[i] = s_cuq[i];
      a.cu_k[i] = s_cuk[i];
    }
  }
  if (gid < a.kcap) {
    const int64_t j = gid;
    const int32_t logical = s_cuk[B];
    int64_t old = 0, nw = 0;
    uint8_t choose = 0, ok = 0;
    if (j < logical) {
      // request r with s_cuk[r] <= j < s_cuk[r+1]
      int lo = 0, hi = B - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_cuk[mid] <= j) lo = mid; else hi = mid - 1;
      }
      const int r = lo;
      const int64_t off = j - s_cuk[r];
      const int c = ctx[r];
      ok = 1;
      if (off < c) {
        old = (int64_t)slot[r] * a.ctx_capacity + off;
      } else {
        nw = (int64_t)s_cuq[r] + (off - c);
        choose = 1;
      }
    }
    a.committed_idx[j] = old;
    a.scratch_idx[j] = nw;
    a.from_scratch[j] = choose;
    a.valid[j] = ok;
  }
  if (gid < a.nq) {
    const int64_t i = gid;
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cuq[mid] <= i) lo = mid; else hi = mid - 1;
    }
    a.positions[i] = (int64_t)ctx[lo] + (i - s_cuq[lo]);
  }
}

// Row copy kernels.  A row is `row_vecs` 16-byte vectors (2 KiB for the
// Qwen3 [8][128] bf16 token row); every thread moves one vector.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct StageArgs {
  const u32x4* k_new;   // [rows][row_vecs]
  const u32x4* v_new;
  u32x4* k_scr;         // scratch layer base
  u32x4* v_scr;
  int64_t n_vec;        // rows * row_vecs
};

__global__ __launch_bounds__(256) void kv_stage_kernel(StageArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < a.n_vec) {
    a.k_scr[i] = a.k_new[i];
    a.v_scr[i] = a.v_new[i];
  }
}

// Resident addressing (bytes): piece (slot, head, pos) of `piece_vecs`
// 16-byte vectors starts at slot*slot_stride + head*head_stride +
// pos*tok_stride within a layer.  Token-major [slots, cap, H, D] and
// head-major [slots, H, cap, D] stores are both expressed this way.
// Scratch and materialised outputs are token-major rows of H pieces.
struct ResidentGeometry {
  int64_t layer_stride;   // bytes per resident layer
  int64_t slot_stride;
  int64_t head_stride;
  int64_t tok_stride;
  int64_t ctx_capacity;   // positions per slot
  int heads;
  int piece_vecs;         // 16-byte vectors per (token, head) piece
};

__device__ __forceinline__ u32x4* resident_vec(char* base, const ResidentGeometry& g, int64_t layer, int64_t slot,
                                              int64_t head, int64_t pos, int64_t v) {
  return reinterpret_cast<u32x4*>(base + layer * g.layer_stride + slot * g.slot_stride + head * g.head_stride +
                                  pos * g.tok_stride) + v;
}

struct CommitArgs {
  char* k_res;
  char* v_res;
  const u32x4* k_scr;     // [L, max_q, H*piece_vecs]
  const u32x4* v_scr;
  const int32_t* req;     // [3][B]: slot, context, query (pre-commit)
  const int32_t* cu_q;    // [B+1] scratch row offset of each request
  const int32_t* n_acc;   // [B] accepted prefix
  ResidentGeometry geo;
  int64_t layer_scr;      // vectors per scratch layer
  int64_t total;          // n_req * max_q * heads * piece_vecs
  int n_req;
  int max_q;
};

// grid: (ceil(total / 256), layers); one 16-byte vector per thread.  The
// host keeps total below 2^31, so the index splits in 32-bit arithmetic, and
// the request's four values are loaded together before the accepted test.
__global__ __launch_bounds__(256) void kv_commit_kernel(CommitArgs a) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int row_vecs = a.geo.heads * a.geo.piece_vecs;
  const int rowi = i / row_vecs;
  const int within = i - rowi * row_vecs;
  const int h = within / a.geo.piece_vecs;
  const int v = within - h * a.geo.piece_vecs;
  const int r = rowi / a.max_q;
  const int t = rowi - r * a.max_q;
  const int layer = blockIdx.y;
  const int n_acc = a.n_acc[r];
  const int32_t slot = a.req[r];
  const int32_t c = a.req[a.n_req + r];
  const int32_t q0 = a.cu_q[r];
  if (t >= n_acc) return;
  const int64_t src = layer * a.layer_scr + ((int64_t)q0 + t) * row_vecs + within;
  *resident_vec(a.k_res, a.geo, layer, slot, h, c + t, v) = a.k_scr[src];
  *resident_vec(a.v_res, a.geo, layer, slot, h, c + t, v) = a.v_scr[src];
}

struct GatherArgs {
  const char* k_res;            // resident layer base
  const char* v_res;
  const u32x4* k_scr;           // scratch layer base, rows [max_q]
  const u32x4* v_scr;
  const int64_t* committed_idx; // [kcap]: slot * capacity + position
  const int64_t* scratch_idx;
  const uint8_t* from_scratch;
  const uint8_t* valid;
  u32x4* k_out;                 // [kcap][H*piece_vecs]
  u32x4* v_out;
  ResidentGeometry geo;
  int64_t total;                // kcap * heads * piece_vecs
  int64_t res_rows;             // slots * capacity (bound for committed_idx)
  int64_t scr_rows;             // bound for scratch_idx
};

__global__ __launch_bounds__(256) void kv_gather_kernel(GatherArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int64_t row_vecs = (int64_t)a.geo.heads * a.geo.piece_vecs;
  const int64_t j = i / row_vecs;
  const int64_t within = i - j * row_vecs;
  u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
  if (a.valid[j]) {
    if (a.from_scratch[j]) {
      const int64_t s = a.scratch_idx[j];
      if (s >= 0 && s < a.scr_rows) {
        kx = a.k_scr[s * row_vecs + within];
        vx = a.v_scr[s * row_vecs + within];
      }
    } else {
      const int64_t s = a.committed_idx[j];
      if (s >= 0 && s < a.res_rows) {
        const int64_t slot = s / a.geo.ctx_capacity;
        const int64_t pos = s - slot * a.geo.ctx_capacity;
        const int64_t h = within / a.geo.piece_vecs;
        const int64_t v = within - h * a.geo.piece_vecs;
        kx = *resident_vec(const_cast<char*>(a.k_res), a.geo, 0, slot, h, pos, v);
        vx = *resident_vec(const_cast<char*>(a.v_res), a.geo, 0, slot, h, pos, v);
      }
    }
  }
  a.k_out[i] = kx;
  a.v_out[i] = vx;
}

// Draft context pool append: new projected K/V rows of several requests
// (source rows in chunk order, [heads, rows, piece] or [rows, heads, piece]
// per layer through byte strides) into each request's slot at positions
// start..start+count-1 of every layer, in one launch.  Rows land beyond the
// pool's committed lengths, so nothing becomes visible until the host
// advances the lengths; an optional flag reports any nonfinite element so
// that the host can refuse the append without publishing it
// (dspark_qwen/packed_draft.py:130-168 checks finiteness before the cat).
constexpr int APPEND_MAX_LAYERS = 16;

struct AppendArgs {
  char* k_pool;
  char* v_pool;
  const char* k_src[APPEND_MAX_LAYERS];
  const char* v_src[APPEND_MAX_LAYERS];
  const int32_t* req;       // [4][B]: slot, start position, source row offset (ascending), count
  int32_t* nonfinite;       // optional flag, set to 1 on any Inf/NaN
  ResidentGeometry geo;
  int64_t src_head_stride;  // bytes
  int64_t src_row_stride;   // bytes
  int64_t total;            // source rows * heads * piece_vecs
  int n_req;
  int elem_bytes;           // 2 (bf16) or 4 (fp32): finiteness test granularity
};

__device__ __forceinline__ bool vec_nonfinite(u32x4 x, int elem_bytes) {
  bool bad = false;
  #pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned w = x[i];
    if (elem_bytes == 2) bad |= ((w & 0x7F80u) == 0x7F80u) || ((w & 0x7F800000u) == 0x7F800000u);
    else bad |= (w & 0x7F800000u) == 0x7F800000u;
  }
  return bad;
}

// grid: (ceil(total / 256), layers)
__global__ __launch_bounds__(256) void pool_append_kernel(AppendArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int layer = blockIdx.y;
  const int64_t row_vecs = (int64_t)a.geo.heads * a.geo.piece_vecs;
  const int64_t row = i / row_vecs;
  const int64_t within = i - row * row_vecs;
  const int64_t h = within / a.geo.piece_vecs;
  const int64_t v = within - h * a.geo.piece_vecs;
  const int32_t* offs = a.req + 2 * a.n_req;
  int lo = 0, hi = a.n_req - 1;   // last request whose source offset <= row
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offs[mid] <= row) lo = mid; else hi = mid - 1;
  }
  const int64_t t = row - offs[lo];
  if (t < 0 || t >= a.req[3 * a.n_req + lo]) return;
  const int64_t slot = a.req[lo], pos = a.req[a.n_req + lo] + t;
  const int64_t src = h * a.src_head_stride + row * a.src_row_stride + v * 16;
  bool bad = false;
  if (a.k_pool) {
    const u32x4 kx = *reinterpret_cast<const u32x4*>(a.k_src[layer] + src);
    *resident_vec(a.k_pool, a.geo, layer, slot, h, pos, v) = kx;
    bad = vec_nonfinite(kx, a.elem_bytes);
  }
  if (a.v_pool) {
    const u32x4 vx = *reinterpret_cast<const u32x4*>(a.v_src[layer] + src);
    *resident_vec(a.v_pool, a.geo, layer, slot, h, pos, v) = vx;
    bad = bad || vec_nonfinite(vx, a.elem_bytes);
  }
  if (a.nonfinite && bad) atomicOr(a.nonfinite, 1);
}

}  // namespace dspark

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {
using namespace dspark;
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

extern "C" int dspark_txn_metadata(const int32_t* req, int n_req, int64_t ctx_capacity,
                                   int64_t key_capacity, int64_t query_tokens,
                                   int64_t* committed_idx, int64_t* scratch_idx,
                                   uint8_t* from_scratch, uint8_t* valid, int64_t* positions,
                                   int32_t* cu_q, int32_t* cu_k, void* stream) {
  clear_error();
  DSPARK_REQUIRE(req && committed_idx && scratch_idx && from_scratch && valid && positions && cu_q && cu_k,
                 "null pointer argument");
  DSPARK_REQUIRE(n_req >= 1 && n_req <= MAX_SCAN, "n_req must be in [1, %d]", MAX_SCAN);
  DSPARK_REQUIRE(ctx_capacity >= 1 && key_capacity >= 1 && query_tokens >= 1, "capacities must be positive");
  const int64_t work = key_capacity > query_tokens ? key_capacity : query_tokens;
  const int64_t blocks = (work + 255) / 256;
  DSPARK_REQUIRE(blocks <= 0x7fffffffLL, "key capacity too large");
  TxnArgs a{req, committed_idx, scratch_idx, from_scratch, valid, positions, cu_q, cu_k,
            ctx_capacity, key_capacity, query_tokens, n_req};
  hipLaunchKernelGGL(txn_metadata_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return launch_status("txn_metadata_kernel");
}

extern "C" int dspark_kv_stage(const void* k_new, const void* v_new, void* k_scr_layer, void* v_scr_layer,
                               int64_t rows, int64_t row_bytes, void* stream) {
  clear_error();
  DSPARK_REQUIRE(k_new && v_new && k_scr_layer && v_scr_layer, "null pointer argument");
  DSPARK_REQUIRE(aligned16(k_new) && aligned16(v_new) && aligned16(k_scr_layer) && aligned16(v_scr_layer),
                 "buffers must be 16-byte aligned");
  DSPARK_REQUIRE(rows >= 1, "rows must be >= 1");
  DSPARK_REQUIRE(row_bytes >= 16 && row_bytes % 16 == 0, "row bytes must be a positive multiple of 16");
  StageArgs a{static_cast<const u32x4*>(k_new), static_cast<const u32x4*>(v_new),
              static_cast<u32x4*>(k_scr_layer), static_cast<u32x4*>(v_scr_layer), rows * (row_bytes / 16)};
  const int64_t blocks = (a.n_vec + 255) / 256;
  DSPARK_REQUIRE(blocks <= 0x7fffffffLL, "stage too large");
  hipLaunchKernelGGL(kv_stage_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return launch_status("kv_stage_kernel");
}

namespace {
int check_geometry(const ResidentGeometry& g) {
  DSPARK_REQUIRE(g.heads >= 1 && g.piece_vecs >= 1 && g.ctx_capacity >= 1, "resident geometry sizes must be positive");
  DSPARK_REQUIRE(g.layer_stride % 16 == 0 && g.slot_stride % 16 == 0 && g.head_stride % 16 == 0 && g.tok_stride % 16 == 0,
                 "resident strides must be multiples of 16 bytes");
  return OK;
}
}  // namespace

extern "C" int dspark_kv_commit(void* k_res, void* v_res, const void* k_scr, const void* v_scr,
                                const int32_t* req, const int32_t* cu_q, const int32_t* n_accepted,
                                int n_req, int max_q, int layers, int64_t layer_stride, int64_t slot_stride,
                                int64_t head_stride, int64_t tok_stride, int64_t ctx_capacity, int heads,
                                int64_t piece_bytes, int64_t scratch_rows, void* stream) {
  clear_error();
  DSPARK_REQUIRE(k_res && v_res && k_scr && v_scr && req && cu_q && n_accepted, "null pointer argument");
  DSPARK_REQUIRE(aligned16(k_res) && aligned16(v_res) && aligned16(k_scr) && aligned16(v_scr),
                 "buffers must be 16-byte aligned");
  DSPARK_REQUIRE(n_req >= 1 && max_q >= 1 && layers >= 1 && scratch_rows >= 1, "sizes must be positive");
  DSPARK_REQUIRE(piece_bytes >= 16 && piece_bytes % 16 == 0, "piece bytes must be a positive multiple of 16");
  DSPARK_REQUIRE(layers <= 65535, "too many layers");
  ResidentGeometry geo{layer_stride, slot_stride, head_stride, tok_stride, ctx_capacity, heads, (int)(piece_bytes / 16)};
  int rc = check_geometry(geo);
  if (rc != OK) return rc;
  const int64_t row_vecs = (int64_t)heads * geo.piece_vecs;
  const int64_t total = (int64_t)n_req * max_q * row_vecs;
  const int64_t blocks = (total + 255) / 256;
  DSPARK_REQUIRE(total <= 0x7fffffffLL, "commit grid too large");
  CommitArgs a{static_cast<char*>(k_res), static_cast<char*>(v_res),
               static_cast<const u32x4*>(k_scr), static_cast<const u32x4*>(v_scr),
               req, cu_q, n_accepted, geo, scratch_rows * row_vecs, total, n_req, max_q};
  hipLaunchKernelGGL(kv_commit_kernel, dim3((unsigned)blocks, layers), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("kv_commit_kernel");
}

extern "C" int dspark_kv_gather(const void* k_res_layer, const void* v_res_layer,
                                const void* k_scr_layer, const void* v_scr_layer,
                                const int64_t* committed_idx, const int64_t* scratch_idx,
                                const uint8_t* from_scratch, const uint8_t* valid,
                                int64_t key_capacity, int64_t slots, int64_t slot_stride, int64_t head_stride,
                                int64_t tok_stride, int64_t ctx_capacity, int heads, int64_t piece_bytes,
                                int64_t scr_rows, void* k_out, void* v_out, void* stream) {
  clear_error();
  DSPARK_REQUIRE(k_res_layer && v_res_layer && k_scr_layer && v_scr_layer && committed_idx && scratch_idx &&
                 from_scratch && valid && k_out && v_out, "null pointer argument");
  DSPARK_REQUIRE(aligned16(k_res_layer) && aligned16(v_res_layer) && aligned16(k_scr_layer) && aligned16(v_scr_layer) &&
                 aligned16(k_out) && aligned16(v_out), "buffers must be 16-byte aligned");
  DSPARK_REQUIRE(key_capacity >= 1 && slots >= 1 && scr_rows >= 1, "sizes must be positive");
  DSPARK_REQUIRE(piece_bytes >= 16 && piece_bytes % 16 == 0, "piece bytes must be a positive multiple of 16");
  ResidentGeometry geo{0, slot_stride, head_stride, tok_stride, ctx_capacity, heads, (int)(piece_bytes / 16)};
  int rc = check_geometry(geo);
  if (rc != OK) return rc;
  const int64_t row_vecs = (int64_t)heads * geo.piece_vecs;
  GatherArgs a{static_cast<const char*>(k_res_layer), static_cast<const char*>(v_res_layer),
               static_cast<const u32x4*>(k_scr_layer), static_cast<const u32x4*>(v_scr_layer),
               committed_idx, scratch_idx, from_scratch, valid,
               static_cast<u32x4*>(k_out), static_cast<u32x4*>(v_out), geo, key_capacity * row_vecs,
               slots * ctx_capacity, scr_rows};
  const int64_t blocks = (a.total + 255) / 256;
  DSPARK_REQUIRE(blocks <= 0x7fffffffLL, "key capacity too large");
  hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return launch_status("kv_gather_kernel");
}

extern "C" int dspark_pool_append(void* k_pool, void* v_pool, int64_t layer_stride, int64_t slot_stride,
                                  int64_t head_stride, int64_t tok_stride, int64_t capacity, int heads,
                                  int64_t piece_bytes, int elem_bytes, int layers,
                                  const void* const* k_src, const void* const* v_src,
                                  int64_t src_head_stride, int64_t src_row_stride, int64_t src_rows,
                                  const int32_t* req, int n_req, int32_t* nonfinite, void* stream) {
  clear_error();
  DSPARK_REQUIRE((k_pool || v_pool) && !k_pool == !k_src && !v_pool == !v_src && req, "null pointer argument");
  DSPARK_REQUIRE(layers >= 1 && layers <= APPEND_MAX_LAYERS, "layers must be in [1, %d]", APPEND_MAX_LAYERS);
  DSPARK_REQUIRE(n_req >= 1 && src_rows >= 1, "sizes must be positive");
  DSPARK_REQUIRE(elem_bytes == 2 || elem_bytes == 4, "element size must be 2 or 4 bytes");
  DSPARK_REQUIRE(piece_bytes >= 16 && piece_bytes % 16 == 0, "piece bytes must be a positive multiple of 16");
  DSPARK_REQUIRE(src_head_stride % 16 == 0 && src_row_stride % 16 == 0, "source strides must be multiples of 16 bytes");
  DSPARK_REQUIRE(aligned16(k_pool) && aligned16(v_pool), "buffers must be 16-byte aligned");
  AppendArgs a{};
  for (int l = 0; l < layers; ++l) {
    DSPARK_REQUIRE((!k_pool || k_src[l]) && (!v_pool || v_src[l]), "null pointer argument");
    a.k_src[l] = k_pool ? static_cast<const char*>(k_src[l]) : nullptr;
    a.v_src[l] = v_pool ? static_cast<const char*>(v_src[l]) : nullptr;
    DSPARK_REQUIRE(aligned16(a.k_src[l]) && aligned16(a.v_src[l]), "buffers must be 16-byte aligned");
  }
  ResidentGeometry geo{layer_stride, slot_stride, head_stride, tok_stride, capacity, heads, (int)(piece_bytes / 16)};
  int rc = check_geometry(geo);
  if (rc != OK) return rc;
  a.k_pool = static_cast<char*>(k_pool);
  a.v_pool = static_cast<char*>(v_pool);
  a.req = req;
  a.nonfinite = nonfinite;
  a.geo = geo;
  a.src_head_stride = src_head_stride;
  a.src_row_stride = src_row_stride;
  a.total = src_rows * heads * geo.piece_vecs;
  a.n_req = n_req;
  a.elem_bytes = elem_bytes;
  const int64_t blocks = (a.total + 255) / 256;
  DSPARK_REQUIRE(blocks <= 0x7fffffffLL, "append grid too large");
  hipLaunchKernelGGL(pool_append_kernel, dim3((unsigned)blocks, layers), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("pool_append_kernel");
}
