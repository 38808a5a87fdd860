// Packed varlen layout construction and KV row gather for gfx950.
//
//   layout_build : PackedLayout.from_metadata (dspark_qwen/varlen_target.py:28-60)
//                  on the device.  From flat int64 request markers and
//                  request-local positions of queries and keys it derives the
//                  requests (runs of equal query markers), their query/key
//                  lengths, int32 cumulative lengths and the int64 gather list
//                  (each request's keys in physical order, requests in query
//                  order), and validates the three layout rules.  The host
//                  reads one small summary (error code, first failing request,
//                  request count, markers, lengths) to raise the reference's
//                  ValueError messages in the reference's precedence.
//   pool_gather  : PackedLayout.gather_kv (varlen_target.py:74-82): rows of a
//                  head-major [H, N, piece] pool selected by the gather list
//                  into token-major [n, H, piece], K and V in one launch.
//
// Validation without a per-request search: a request's keys are valid iff
// every key position p lies in [0, k), scattering key j to slot cu_k + p
// fills all k slots (no duplicate positions) and the physical indices in the
// slots increase with p (physical order == position order).  That is exactly
// "positions of the request's keys, in physical order, equal 0..k-1".
#include "common.h"

namespace dspark {

constexpr int LAYOUT_MAX_REQ = 8192;   // requests per layout (LDS-resident sort)
constexpr int LAYOUT_THREADS = 1024;

enum LayoutError : int64_t {
  LAYOUT_OK = 0,
  LAYOUT_NOT_CONTIGUOUS = 1,   // a request's queries are split into several runs
  LAYOUT_BAD_PREFIX = 2,       // keys are not the complete prefix 0..k-1 (or k < q)
  LAYOUT_BAD_SUFFIX = 3,       // query positions are not k-q..k-1
  LAYOUT_TOO_MANY = 4,         // more requests than the build supports
};

// summary: [0] error, [1] first failing request, [2] requests B, [3] sum K,
//          [4 + r] marker, [4 + M + r] query length, [4 + 2M + r] key length.
struct LayoutArgs {
  const int64_t* qr;
  const int64_t* qp;
  const int64_t* kr;
  const int64_t* kp;
  int64_t nq;
  int64_t nk;
  int32_t* cu_q;      // [M + 1]
  int32_t* cu_k;      // [M + 1]
  int64_t* gather;    // [nk]
  int64_t* summary;   // [4 + 3M]
  int32_t* seg_q;     // [nq] request of each query
  int64_t* sorted_m;  // [M]  markers, ascending
  int32_t* sorted_r;  // [M]  request of each sorted marker
  int32_t* seg_k;     // [nk] request of each key, -1 if its marker has no queries
  int32_t* k_cnt;     // [M]
  int32_t* flags;     // [M]  bit 0: bad prefix, bit 1: bad suffix
  int max_req;        // M
};

__device__ __forceinline__ int block_inclusive_scan_1024(int x, int* tmp) {
  // Wave scan, then a scan of the 16 wave totals.
  const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
  #pragma unroll
  for (int off = 1; off < WAVE; off <<= 1) {
    const int t = __shfl_up(x, off);
    if (lane >= off) x += t;
  }
  if (lane == WAVE - 1) tmp[wave] = x;
  __syncthreads();
  if (threadIdx.x < 16) {
    int w = tmp[threadIdx.x];
    #pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const int t = __shfl_up(w, off, 16);
      if ((int)threadIdx.x >= off) w += t;
    }
    tmp[16 + threadIdx.x] = w;
  }
  __syncthreads();
  const int before = wave ? tmp[16 + wave - 1] : 0;
  const int total = tmp[31];
  __syncthreads();
  tmp[32] = total;
  return x + before;
}

// One workgroup: query runs -> requests, query cumulative lengths, sorted
// markers and the duplicate-marker (non-contiguous queries) check.
__global__ __launch_bounds__(LAYOUT_THREADS) void layout_queries_kernel(LayoutArgs a) {
  __shared__ int64_t s_m[LAYOUT_MAX_REQ];
  __shared__ int32_t s_r[LAYOUT_MAX_REQ];
  __shared__ int s_tmp[40];
  const int tid = threadIdx.x;
  const int M = a.max_req;
  int running = 0;
  for (int64_t base = 0; base < a.nq; base += LAYOUT_THREADS) {
    const int64_t i = base + tid;
    int flag = 0;
    int64_t m = 0;
    if (i < a.nq) {
      m = a.qr[i];
      flag = (i == 0 || a.qr[i - 1] != m) ? 1 : 0;
    }
    const int incl = block_inclusive_scan_1024(flag, s_tmp);
    const int total = s_tmp[32];
    const int seg = running + incl - 1;
    if (i < a.nq) {
      a.seg_q[i] = seg < M ? seg : M - 1;
      if (flag && seg < M) {
        s_m[seg] = m;
        a.cu_q[seg] = (int32_t)i;
      }
    }
    running += total;
    __syncthreads();
  }
  const int B = running;
  if (B > M) {
    if (tid == 0) {
      a.summary[0] = LAYOUT_TOO_MANY;
      a.summary[1] = 0;
      a.summary[2] = B;
      a.summary[3] = 0;
    }
    return;
  }
  if (tid == 0) a.cu_q[B] = (int32_t)a.nq;
  __syncthreads();
  for (int r = tid; r < B; r += LAYOUT_THREADS) {
    a.summary[4 + r] = s_m[r];
    a.summary[4 + M + r] = a.cu_q[r + 1] - a.cu_q[r];
    a.k_cnt[r] = 0;
    a.flags[r] = 0;
  }
  // Bitonic sort of (marker, request) over the next power of two >= B.
  int P = 1;
  while (P < B) P <<= 1;
  for (int r = B + tid; r < P; r += LAYOUT_THREADS) {
    s_m[r] = INT64_MAX;
    s_r[r] = INT32_MAX;
  }
  for (int r = tid; r < B; r += LAYOUT_THREADS) s_r[r] = r;
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P; i += LAYOUT_THREADS) {
        const int l = i ^ j;
        if (l > i) {
          const bool up = (i & k) == 0;
          const bool gt = s_m[i] > s_m[l] || (s_m[i] == s_m[l] && s_r[i] > s_r[l]);
          if (gt == up) {
            const int64_t tm = s_m[i];
            s_m[i] = s_m[l];
            s_m[l] = tm;
            const int32_t tr = s_r[i];
            s_r[i] = s_r[l];
            s_r[l] = tr;
          }
        }
      }
      __syncthreads();
    }
  }
  int dup = 0;
  for (int r = tid; r < B; r += LAYOUT_THREADS) {
    a.sorted_m[r] = s_m[r];
    a.sorted_r[r] = s_r[r];
    if (r + 1 < B && s_m[r] == s_m[r + 1]) dup = 1;
  }
  dup = __syncthreads_or(dup);
  if (tid == 0) {
    a.summary[0] = dup ? LAYOUT_NOT_CONTIGUOUS : LAYOUT_OK;
    a.summary[1] = 0;
    a.summary[2] = B;
    a.summary[3] = 0;
  }
}

__device__ __forceinline__ bool layout_stopped(const LayoutArgs& a) {
  const int64_t e = a.summary[0];
  return e == LAYOUT_TOO_MANY || e == LAYOUT_NOT_CONTIGUOUS;
}

// Keys -> owning request (binary search over the sorted markers), key counts
// per request (wave-aggregated atomics) and the -1 fill of the gather list.
__global__ __launch_bounds__(256) void layout_keys_kernel(LayoutArgs a) {
  if (layout_stopped(a)) return;
  const int B = (int)a.summary[2];
  const int lane = threadIdx.x & (WAVE - 1);
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j - lane < a.nk; j += (int64_t)gridDim.x * 256) {
    int r = -1;
    if (j < a.nk) {
      a.gather[j] = -1;
      const int64_t m = a.kr[j];
      int lo = 0, hi = B;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (a.sorted_m[mid] < m) lo = mid + 1; else hi = mid;
      }
      if (lo < B && a.sorted_m[lo] == m) r = a.sorted_r[lo];
      a.seg_k[j] = r;
    }
    // Wave aggregation: one atomic per distinct request in the wave.
    unsigned long long todo = __ballot(r >= 0);
    while (todo) {
      const int leader = __ffsll((long long)todo) - 1;
      const int lr = __shfl(r, leader);
      const unsigned long long same = __ballot(r == lr);
      if (lane == leader) atomicAdd(&a.k_cnt[lr], (int)__popcll(same));
      todo &= ~same;
    }
  }
}

// One workgroup: key lengths, k >= q check, key cumulative lengths.
__global__ __launch_bounds__(LAYOUT_THREADS) void layout_offsets_kernel(LayoutArgs a) {
  __shared__ int s_tmp[40];
  if (layout_stopped(a)) return;
  const int B = (int)a.summary[2];
  const int M = a.max_req;
  const int tid = threadIdx.x;
  int running = 0;
  for (int base = 0; base < B; base += LAYOUT_THREADS) {
    const int r = base + tid;
    const int k = r < B ? a.k_cnt[r] : 0;
    const int incl = block_inclusive_scan_1024(k, s_tmp);
    const int total = s_tmp[32];
    if (r < B) {
      a.cu_k[r] = running + incl - k;
      a.summary[4 + 2 * M + r] = k;
      if (k < a.summary[4 + M + r]) a.flags[r] |= 1;
    }
    running += total;
    __syncthreads();
  }
  if (tid == 0) {
    a.cu_k[B] = running;
    a.summary[3] = running;
  }
}

// Scatter each key to slot cu_k[r] + position; out-of-range positions mark
// the request's prefix invalid.
__global__ __launch_bounds__(256) void layout_scatter_kernel(LayoutArgs a) {
  if (layout_stopped(a)) return;
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < a.nk; j += (int64_t)gridDim.x * 256) {
    const int r = a.seg_k[j];
    if (r < 0) continue;
    const int64_t p = a.kp[j];
    const int32_t beg = a.cu_k[r], len = a.cu_k[r + 1] - beg;
    if (p < 0 || p >= len) atomicOr(&a.flags[r], 1);
    else a.gather[beg + p] = j;
  }
}

// Slots: every slot filled and physical indices increasing inside a request.
// Queries: position of the t-th query of request r is k - q + t.
__global__ __launch_bounds__(256) void layout_check_kernel(LayoutArgs a) {
  if (layout_stopped(a)) return;
  const int B = (int)a.summary[2];
  const int M = a.max_req;
  const int64_t total_k = a.summary[3];
  const int64_t n = total_k > a.nq ? total_k : a.nq;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    if (i < total_k) {
      int lo = 0, hi = B - 1;   // last r with cu_k[r] <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.cu_k[mid] <= i) lo = mid; else hi = mid - 1;
      }
      const int64_t g = a.gather[i];
      bool bad = g < 0;
      if (!bad && i + 1 < a.cu_k[lo + 1]) {
        const int64_t g2 = a.gather[i + 1];
        bad = g2 >= 0 && g2 <= g;
      }
      if (bad) atomicOr(&a.flags[lo], 1);
    }
    if (i < a.nq) {
      const int r = a.seg_q[i];
      const int64_t q = a.summary[4 + M + r], k = a.summary[4 + 2 * M + r];
      if (k >= q && a.qp[i] != k - q + (i - a.cu_q[r])) atomicOr(&a.flags[r], 2);
    }
  }
}

// First failing request in query order decides the error (prefix before
// suffix for the same request), as the reference's per-request loop does.
__global__ __launch_bounds__(LAYOUT_THREADS) void layout_summary_kernel(LayoutArgs a) {
  __shared__ int s_first;
  if (layout_stopped(a)) return;
  const int B = (int)a.summary[2];
  if (threadIdx.x == 0) s_first = INT32_MAX;
  __syncthreads();
  for (int r = threadIdx.x; r < B; r += LAYOUT_THREADS)
    if (a.flags[r]) atomicMin(&s_first, r);
  __syncthreads();
  if (threadIdx.x == 0 && s_first != INT32_MAX) {
    a.summary[0] = (a.flags[s_first] & 1) ? LAYOUT_BAD_PREFIX : LAYOUT_BAD_SUFFIX;
    a.summary[1] = s_first;
  }
}

struct GatherArgs {
  const unsigned char* src[2];
  unsigned char* dst[2];
  const int64_t* idx;
  int64_t n_rows;
  int64_t src_rows;
  int64_t head_stride;   // bytes between heads of the source
  int64_t row_stride;    // bytes between rows of the source
  int64_t piece_vecs;    // 16-byte vectors per (row, head)
  int heads;
};

__global__ __launch_bounds__(256) void pool_gather_kernel(GatherArgs g) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const unsigned char* src = g.src[blockIdx.y];
  unsigned char* dst = g.dst[blockIdx.y];
  const int64_t per_row = (int64_t)g.heads * g.piece_vecs;
  const int64_t total = g.n_rows * per_row;
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < total; v += (int64_t)gridDim.x * 256) {
    const int64_t s = v / per_row;
    const int64_t rem = v - s * per_row;
    const int64_t h = rem / g.piece_vecs;
    const int64_t e = rem - h * g.piece_vecs;
    const int64_t row = g.idx[s];
    u32x4 x = {0u, 0u, 0u, 0u};
    if (row >= 0 && row < g.src_rows)
      x = *reinterpret_cast<const u32x4*>(src + h * g.head_stride + row * g.row_stride + e * 16);
    *reinterpret_cast<u32x4*>(dst + v * 16) = x;
  }
}

int64_t layout_workspace(int64_t nq, int64_t nk, int max_req) {
  auto up = [](int64_t b) { return (b + 255) & ~int64_t(255); };
  return up(4 * nq) + up(8 * (int64_t)max_req) + 3 * up(4 * (int64_t)max_req) + up(4 * nk);
}

}  // namespace dspark

using namespace dspark;

extern "C" int64_t dspark_layout_workspace_bytes(int64_t nq, int64_t nk, int max_req) {
  if (nq < 1 || nk < 0 || max_req < 1 || max_req > LAYOUT_MAX_REQ) return -1;
  return layout_workspace(nq, nk, max_req);
}

extern "C" int dspark_layout_build(const int64_t* query_requests, const int64_t* query_positions, int64_t nq,
                                   const int64_t* key_requests, const int64_t* key_positions, int64_t nk,
                                   int max_req, int32_t* cu_q, int32_t* cu_k, int64_t* gather,
                                   int64_t* summary, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  DSPARK_REQUIRE(query_requests && query_positions && cu_q && cu_k && summary && workspace,
                 "dspark_layout_build: null pointer");
  DSPARK_REQUIRE(nk == 0 || (key_requests && key_positions && gather), "dspark_layout_build: null key pointer");
  DSPARK_REQUIRE(nq >= 1 && nq < (int64_t(1) << 31) && nk >= 0 && nk < (int64_t(1) << 31),
                 "dspark_layout_build: need 1 <= queries < 2^31 and 0 <= keys < 2^31");
  DSPARK_REQUIRE(max_req >= 1 && max_req <= LAYOUT_MAX_REQ, "dspark_layout_build: max_req must be in [1, %d]",
                 LAYOUT_MAX_REQ);
  DSPARK_REQUIRE(workspace_bytes >= layout_workspace(nq, nk, max_req), "dspark_layout_build: workspace too small");
  LayoutArgs a{};
  a.qr = query_requests;
  a.qp = query_positions;
  a.kr = key_requests;
  a.kp = key_positions;
  a.nq = nq;
  a.nk = nk;
  a.cu_q = cu_q;
  a.cu_k = cu_k;
  a.gather = gather;
  a.summary = summary;
  a.max_req = max_req;
  auto up = [](int64_t b) { return (b + 255) & ~int64_t(255); };
  unsigned char* w = static_cast<unsigned char*>(workspace);
  a.seg_q = reinterpret_cast<int32_t*>(w);
  w += up(4 * nq);
  a.sorted_m = reinterpret_cast<int64_t*>(w);
  w += up(8 * (int64_t)max_req);
  a.sorted_r = reinterpret_cast<int32_t*>(w);
  w += up(4 * (int64_t)max_req);
  a.k_cnt = reinterpret_cast<int32_t*>(w);
  w += up(4 * (int64_t)max_req);
  a.flags = reinterpret_cast<int32_t*>(w);
  w += up(4 * (int64_t)max_req);
  a.seg_k = reinterpret_cast<int32_t*>(w);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_items = nk > nq ? nk : nq;
  const unsigned grid = (unsigned)std::min<int64_t>(std::max<int64_t>((n_items + 255) / 256, 1), 2048);
  hipLaunchKernelGGL(layout_queries_kernel, dim3(1), dim3(LAYOUT_THREADS), 0, s, a);
  if (nk > 0) hipLaunchKernelGGL(layout_keys_kernel, dim3(grid), dim3(256), 0, s, a);
  hipLaunchKernelGGL(layout_offsets_kernel, dim3(1), dim3(LAYOUT_THREADS), 0, s, a);
  if (nk > 0) hipLaunchKernelGGL(layout_scatter_kernel, dim3(grid), dim3(256), 0, s, a);
  hipLaunchKernelGGL(layout_check_kernel, dim3(grid), dim3(256), 0, s, a);
  hipLaunchKernelGGL(layout_summary_kernel, dim3(1), dim3(LAYOUT_THREADS), 0, s, a);
  return launch_status("dspark_layout_build");
}

extern "C" int dspark_pool_gather(const void* k_src, const void* v_src, int64_t src_rows, int64_t head_stride,
                                  int64_t row_stride, int heads, int64_t piece_bytes, const int64_t* indices,
                                  int64_t n_rows, void* k_dst, void* v_dst, void* stream) {
  clear_error();
  DSPARK_REQUIRE(n_rows >= 0 && src_rows >= 0 && heads >= 1, "dspark_pool_gather: invalid sizes");
  if (n_rows == 0) return OK;
  DSPARK_REQUIRE(k_src && v_src && k_dst && v_dst && indices, "dspark_pool_gather: null pointer");
  DSPARK_REQUIRE(piece_bytes > 0 && piece_bytes % 16 == 0 && head_stride % 16 == 0 && row_stride % 16 == 0,
                 "dspark_pool_gather: piece and strides must be multiples of 16 bytes");
  DSPARK_REQUIRE(((uintptr_t)k_src | (uintptr_t)v_src | (uintptr_t)k_dst | (uintptr_t)v_dst) % 16 == 0,
                 "dspark_pool_gather: pointers must be 16-byte aligned");
  GatherArgs g{};
  g.src[0] = static_cast<const unsigned char*>(k_src);
  g.src[1] = static_cast<const unsigned char*>(v_src);
  g.dst[0] = static_cast<unsigned char*>(k_dst);
  g.dst[1] = static_cast<unsigned char*>(v_dst);
  g.idx = indices;
  g.n_rows = n_rows;
  g.src_rows = src_rows;
  g.head_stride = head_stride;
  g.row_stride = row_stride;
  g.piece_vecs = piece_bytes / 16;
  g.heads = heads;
  const int64_t vecs = n_rows * heads * g.piece_vecs;
  const unsigned grid = (unsigned)std::min<int64_t>((vecs + 255) / 256, 4096);
  hipLaunchKernelGGL(pool_gather_kernel, dim3(grid, 2), dim3(256), 0, static_cast<hipStream_t>(stream), g);
  return launch_status("dspark_pool_gather");
}

// ---------------------------------------------------------------------------
// Append-order KV cache of PackedTarget / VarlenPackedTarget
// (dspark_qwen/packed_target.py:30-113): per layer K and V [1, H, N, piece]
// with physical rows in append order (requests interleaved) and int64
// key_requests / key_positions [N].
//
//   crop_plan    : keep = (request != marker) | (position < length)
//                  (packed_target.py:99-108) as a stable compaction: the
//                  source row of every kept output row, and the compacted
//                  markers/positions.  Tile counts, a one-workgroup scan of
//                  the tile totals, then a per-tile scan that scatters.
//   rows_rebuild : every layer's K and V rebuilt in one launch, output row j
//                  taken from plan[j] (crop) or, without a plan, from the old
//                  rows then the appended rows (append: the reference's cat).
// ---------------------------------------------------------------------------
namespace dspark {

constexpr int PLAN_TILE = 4096;            // rows per tile (256 threads x 16)
constexpr int REBUILD_MAX_LAYERS = 64;

struct CropPlanArgs {
  const int64_t* kr;
  const int64_t* kp;
  int64_t n;
  int64_t marker;
  int64_t length;
  int32_t* tile_kept;     // [tiles] kept rows per tile, then exclusive offsets
  int64_t* plan;          // [n_kept] source row of each kept row
  int64_t* out_kr;        // [n_kept]
  int64_t* out_kp;        // [n_kept]
  int64_t tiles;
};

__device__ __forceinline__ bool crop_keeps(const CropPlanArgs& a, int64_t i) {
  return a.kr[i] != a.marker || a.kp[i] < a.length;
}

__global__ __launch_bounds__(256) void crop_count_kernel(CropPlanArgs a) {
  __shared__ int s_sum;
  if (threadIdx.x == 0) s_sum = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * PLAN_TILE;
  int kept = 0;
  for (int k = threadIdx.x; k < PLAN_TILE; k += 256) {
    const int64_t i = base + k;
    if (i < a.n && crop_keeps(a, i)) ++kept;
  }
  atomicAdd(&s_sum, kept);
  __syncthreads();
  if (threadIdx.x == 0) a.tile_kept[blockIdx.x] = s_sum;
}

// One workgroup: exclusive scan of the tile totals in place.
__global__ __launch_bounds__(LAYOUT_THREADS) void crop_scan_kernel(CropPlanArgs a) {
  __shared__ int s_tmp[40];
  int running = 0;
  for (int64_t base = 0; base < a.tiles; base += LAYOUT_THREADS) {
    const int64_t t = base + threadIdx.x;
    const int v = t < a.tiles ? a.tile_kept[t] : 0;
    const int incl = block_inclusive_scan_1024(v, s_tmp);
    const int total = s_tmp[32];
    if (t < a.tiles) a.tile_kept[t] = running + incl - v;
    running += total;
    __syncthreads();
  }
}

// Per tile: rows in order, 16 consecutive rows per thread, block scan of the
// per-thread counts; kept rows scatter to their output slot.
__global__ __launch_bounds__(256) void crop_scatter_kernel(CropPlanArgs a) {
  __shared__ int s_tmp[256];
  const int64_t base = (int64_t)blockIdx.x * PLAN_TILE + (int64_t)threadIdx.x * 16;
  int kept = 0;
  for (int k = 0; k < 16; ++k) {
    const int64_t i = base + k;
    if (i < a.n && crop_keeps(a, i)) ++kept;
  }
  s_tmp[threadIdx.x] = kept;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {   // Hillis-Steele inclusive scan
    const int v = threadIdx.x >= off ? s_tmp[threadIdx.x - off] : 0;
    __syncthreads();
    s_tmp[threadIdx.x] += v;
    __syncthreads();
  }
  int64_t out = a.tile_kept[blockIdx.x] + s_tmp[threadIdx.x] - kept;
  for (int k = 0; k < 16; ++k) {
    const int64_t i = base + k;
    if (i < a.n && crop_keeps(a, i)) {
      a.plan[out] = i;
      a.out_kr[out] = a.kr[i];
      a.out_kp[out] = a.kp[i];
      ++out;
    }
  }
}

struct RebuildArgs {
  const char* src[REBUILD_MAX_LAYERS];     // per (layer, K|V): old rows [H, n_old, piece]
  const char* add[REBUILD_MAX_LAYERS];     // appended rows [H, n_add, piece] (append only)
  char* dst[REBUILD_MAX_LAYERS];           // new rows [H, n_out, piece]
  const int64_t* plan;                     // crop: source row per output row; null for append
  int64_t n_old;
  int64_t n_add;
  int64_t n_out;
  int64_t piece_vecs;
  int heads;
};

// grid: (ceil(n_out * heads * piece_vecs / 256), tensors)
__global__ __launch_bounds__(256) void rows_rebuild_kernel(RebuildArgs a) {
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_head = a.n_out * a.piece_vecs;
  if (i >= per_head * a.heads) return;
  const int t = blockIdx.y;
  const int64_t h = i / per_head;
  const int64_t rem = i - h * per_head;
  const int64_t row = rem / a.piece_vecs;
  const int64_t e = rem - row * a.piece_vecs;
  const u32x4_t* from;
  if (a.plan) {
    from = reinterpret_cast<const u32x4_t*>(a.src[t]) + (h * a.n_old + a.plan[row]) * a.piece_vecs + e;
  } else if (row < a.n_old) {
    from = reinterpret_cast<const u32x4_t*>(a.src[t]) + (h * a.n_old + row) * a.piece_vecs + e;
  } else {
    from = reinterpret_cast<const u32x4_t*>(a.add[t]) + (h * a.n_add + row - a.n_old) * a.piece_vecs + e;
  }
  reinterpret_cast<u32x4_t*>(a.dst[t])[i] = *from;
}

}  // namespace dspark

extern "C" int64_t dspark_crop_plan_workspace_bytes(int64_t n) {
  if (n < 0) return -1;
  return 4 * std::max<int64_t>((n + PLAN_TILE - 1) / PLAN_TILE, 1);
}

extern "C" int dspark_crop_plan(const int64_t* key_requests, const int64_t* key_positions, int64_t n,
                                int64_t marker, int64_t length, int64_t* plan, int64_t* out_requests,
                                int64_t* out_positions, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  DSPARK_REQUIRE(n >= 0 && n < (int64_t(1) << 40), "dspark_crop_plan: invalid row count");
  if (n == 0) return OK;
  DSPARK_REQUIRE(key_requests && key_positions && plan && out_requests && out_positions && workspace,
                 "dspark_crop_plan: null pointer");
  DSPARK_REQUIRE(workspace_bytes >= dspark_crop_plan_workspace_bytes(n), "dspark_crop_plan: workspace too small");
  CropPlanArgs a{key_requests, key_positions, n, marker, length, static_cast<int32_t*>(workspace),
                 plan, out_requests, out_positions, (n + PLAN_TILE - 1) / PLAN_TILE};
  DSPARK_REQUIRE(a.tiles <= 0x7fffffffLL, "dspark_crop_plan: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(crop_count_kernel, dim3((unsigned)a.tiles), dim3(256), 0, s, a);
  hipLaunchKernelGGL(crop_scan_kernel, dim3(1), dim3(LAYOUT_THREADS), 0, s, a);
  hipLaunchKernelGGL(crop_scatter_kernel, dim3((unsigned)a.tiles), dim3(256), 0, s, a);
  return launch_status("dspark_crop_plan");
}

extern "C" int dspark_rows_rebuild(const void* const* src, const void* const* add, void* const* dst, int tensors,
                                   int heads, int64_t piece_bytes, int64_t n_old, int64_t n_add,
                                   const int64_t* plan, int64_t n_out, void* stream) {
  clear_error();
  DSPARK_REQUIRE(src && dst, "dspark_rows_rebuild: null pointer");
  DSPARK_REQUIRE(tensors >= 1 && tensors <= REBUILD_MAX_LAYERS, "dspark_rows_rebuild: tensors must be in [1, %d]",
                 REBUILD_MAX_LAYERS);
  DSPARK_REQUIRE(heads >= 1 && n_old >= 0 && n_add >= 0 && n_out >= 0, "dspark_rows_rebuild: invalid sizes");
  DSPARK_REQUIRE(piece_bytes >= 16 && piece_bytes % 16 == 0, "dspark_rows_rebuild: piece bytes must be a multiple of 16");
  DSPARK_REQUIRE(plan ? n_out <= n_old : n_out == n_old + n_add,
                 "dspark_rows_rebuild: output rows must be n_old + n_add (append) or <= n_old (crop)");
  if (n_out == 0) return OK;
  DSPARK_REQUIRE(plan || n_add == 0 || add, "dspark_rows_rebuild: null pointer");
  RebuildArgs a{};
  for (int t = 0; t < tensors; ++t) {
    DSPARK_REQUIRE(dst[t] && (n_old == 0 || src[t]) && (plan || n_add == 0 || add[t]),
                   "dspark_rows_rebuild: null pointer");
    DSPARK_REQUIRE(((uintptr_t)dst[t] | (uintptr_t)(src[t]) | (uintptr_t)(add ? add[t] : nullptr)) % 16 == 0,
                   "dspark_rows_rebuild: pointers must be 16-byte aligned");
    a.src[t] = static_cast<const char*>(src[t]);
    a.add[t] = add ? static_cast<const char*>(add[t]) : nullptr;
    a.dst[t] = static_cast<char*>(dst[t]);
  }
  a.plan = plan;
  a.n_old = n_old;
  a.n_add = n_add;
  a.n_out = n_out;
  a.piece_vecs = piece_bytes / 16;
  a.heads = heads;
  const int64_t blocks = (n_out * heads * a.piece_vecs + 255) / 256;
  DSPARK_REQUIRE(blocks <= 0x7fffffffLL, "dspark_rows_rebuild: grid too large");
  hipLaunchKernelGGL(rows_rebuild_kernel, dim3((unsigned)blocks, tensors), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("dspark_rows_rebuild");
}
