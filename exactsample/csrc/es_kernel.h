// exactsample device code: sampling and speculative-draft verification on gfx950.
//
// Two kernels per call (es_launch), on the caller's stream:
//
//  es_main, rows x slices blocks of 256 threads, each one register tile of up
//  to 16 x 4 logits per thread (es_wide replaces it, with slices of several
//  tiles read group by group, when a row needs more than MAX_SLICES tiles;
//  such calls store no list candidates): one pass over a slice of a
//  row: validation (NaN/+inf anywhere), the valid count, the largest valid
//  logit and, for rows a list can finish, every valid logit at or above a
//  threshold chosen so that the slice's top L are stored, or exactly its first
//  L after a radix cut (reference: fused.cuh:409-519 row_stats, :686-798
//  row_hist/row_gather); stream rows also draw their slice's certified
//  Gumbel-max (reference: fused.cuh:532-681 row_scan); binned top-p rows bin
//  their slice's kept weights on an absolute grid (slice_bins). Each slice
//  writes a SlicePart with plain stores; the row's first slice also records
//  the row's resolved request parameters and checks its per-row metadata.
//
//  es_finish, one block per row, then Plan::helpers blocks per row that share
//  a binned top-p row's boundary pass (and leave at once on other rows), then
//  ceil(R / 256) request blocks that validate each request's metadata and
//  write the outputs of every request that fails it (reference:
//  csrc/verify/verify.cu:6-56, initialize). A row block (the kernel boundary makes
//  every slice's stores visible) merges the slices in slice order and
//  finishes the row:
//    - failed and greedy rows directly;
//    - top-k rows from the union of the slices' candidates in one wave, in FP64
//      with the oracle's formulas (reference: fused.cuh:1250-1412);
//    - other list rows (small top-p nuclei) with the whole block;
//    - binned top-p rows from the merged bins and one pass shared by the row's
//      blocks, the last to arrive finishing (FullRow::topp_binned);
//    - every other row on the full-row path, re-reading the row: exact radix
//      cuts, exact top-p boundary, certified FP32 draws with FP64 rescoring
//      (reference: fused.cuh:1446-1810).
//  The block that completes a request's last row commits the request
//  (reference: verify.cu:169-217, finalize).
//
// Results never depend on the slice count, the slot or the arrival order:
// merges run in slice order, candidate sets are exact up to a recorded
// frontier and are sorted before use, and every decision is either exact or
// certified with a bound and otherwise recomputed in FP64.
#include "es_device.h"
#include "es_layout.h"
#include "es_superacc.h"
#include "es_plan.h"
#include <limits.h>
#include <type_traits>
#include <stdio.h>

namespace es {

constexpr float SCORE_ERR = 1.9073486e-06f;  // |s32 - s| <= SCORE_ERR * (1 + |x| + |G|)
constexpr float PRUNE_MARGIN = 1e-3f;
constexpr float SUM_PRUNE = -40.f;        // weights below e^-40 are bounded, not summed
constexpr double SUM_PRUNE_W = 4.25e-18;  // e^-40 rounded up
constexpr int TOPP_SLICE_NEED = 64;       // candidates per slice for a top-p list
constexpr int LIST_LIMIT = 1024;          // largest candidate union the merge takes
constexpr int HEAD_BINS = 256;            // quarter-logit bins below the maximum for the union's head
constexpr int TOPP_HEAD = 96;             // entries a top-p list sorts first
// Binned top-p rows: each slice bins its kept tokens on the grid y = l * 4 / T
// (bin b holds y in [b, b + 1), a quarter of a unit of x = (l - max) / T), in
// the TP_COARSE bins below its reference maximum: per bin the count and the
// sum of e^((y - b - 1/2) / 4), i.e. the weights relative to the bin's centre.
// The grid is absolute, so the slices' bins merge by addition.
constexpr double TP_Y_PER_X = 4.0;

// ---------------------------------------------------------------------------
// Element types.
template <int DT> struct Ty;
template <> struct Ty<ES_F32> { using T = float; using W = float; using Key = uint32_t; };
template <> struct Ty<ES_F64> { using T = double; using W = double; using Key = uint64_t; };
template <> struct Ty<ES_BF16> { using T = uint16_t; using W = float; using Key = uint32_t; };
template <> struct Ty<ES_F16> { using T = uint16_t; using W = float; using Key = uint32_t; };

template <int DT> __device__ __forceinline__ typename Ty<DT>::W widen(typename Ty<DT>::T x);
template <> __device__ __forceinline__ float widen<ES_F32>(float x) { return x; }
template <> __device__ __forceinline__ double widen<ES_F64>(double x) { return x; }
template <> __device__ __forceinline__ float widen<ES_BF16>(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }
template <> __device__ __forceinline__ float widen<ES_F16>(uint16_t x) {
  _Float16 h;
  __builtin_memcpy(&h, &x, 2);
  return float(h);
}

template <class W> __device__ __forceinline__ W neg_inf() { return W(-INFINITY); }

// One row of logits; tokens are read in groups of four (one Philox block).
template <int DT, bool VEC> struct RowView {
  using T = typename Ty<DT>::T;
  using W = typename Ty<DT>::W;
  const T* base;
  int64_t stride;
  int vocab;
  __device__ __forceinline__ RowView(const es_matrix& m, int64_t row, int vocab_)
      : base(static_cast<const T*>(m.data) + row * m.s0), stride(m.s1), vocab(vocab_) {}
  __device__ __forceinline__ void load(int g, W v[4]) const {
    const int t = 4 * g;
    if constexpr (VEC) {
      if constexpr (DT == ES_F32) {
        const float4 x = *reinterpret_cast<const float4*>(base + t);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      } else if constexpr (DT == ES_F64) {
        const double2 x = reinterpret_cast<const double2*>(base + t)[0];
        const double2 y = reinterpret_cast<const double2*>(base + t)[1];
        v[0] = x.x; v[1] = x.y; v[2] = y.x; v[3] = y.y;
      } else {
        const uint2 x = *reinterpret_cast<const uint2*>(base + t);
        v[0] = widen<DT>(uint16_t(x.x)); v[1] = widen<DT>(uint16_t(x.x >> 16));
        v[2] = widen<DT>(uint16_t(x.y)); v[3] = widen<DT>(uint16_t(x.y >> 16));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = t + j < vocab ? widen<DT>(base[int64_t(t + j) * stride]) : neg_inf<W>();
    }
  }
  __device__ __forceinline__ W value(int t) const { return widen<DT>(base[int64_t(t) * stride]); }
};

// ---------------------------------------------------------------------------
// Argument access.
__device__ __forceinline__ int64_t at(const es_vec_i64& v, int64_t i) { return v.data[i * v.stride]; }
__device__ __forceinline__ double at(const es_vec_f64& v, int64_t i) { return v.data[i * v.stride]; }
__device__ __forceinline__ int64_t draft_at(const es_arguments& a, int64_t req, int64_t i) {
  return a.draft_ids[req * a.draft_s0 + i * a.draft_s1];
}
// Bits j of group g: is token 4g + j allowed by the mask?
__device__ __forceinline__ uint32_t group_bits(const es_arguments& a, int64_t row, int g) {
  if (!a.mask) return 0xfu;
  const int t = 4 * g;
  if (t >= a.vocab) return 0u;
  return (uint32_t(a.mask[row * a.mask_s0 + int64_t(t >> 5) * a.mask_s1]) >> (t & 31)) & 0xfu;
}
__device__ __forceinline__ bool allowed(const es_arguments& a, int64_t row, int t) {
  return !a.mask || ((uint32_t(a.mask[row * a.mask_s0 + int64_t(t >> 5) * a.mask_s1]) >> (t & 31)) & 1u);
}

__device__ __forceinline__ uint8_t* row_region(const es_arguments& a, int64_t row) {
  return a.workspace + HEADER_BYTES + row * ROW_BYTES;
}
__device__ __forceinline__ RowResult* row_result(const es_arguments& a, int64_t row) {
  return reinterpret_cast<RowResult*>(row_region(a, row) + OFF_RESULT);
}
__device__ __forceinline__ RowState* row_state(const es_arguments& a, int64_t row) {
  return reinterpret_cast<RowState*>(row_region(a, row) + OFF_STATE);
}
__device__ __forceinline__ Counters* counters(const es_arguments& a, int64_t row) {
  return reinterpret_cast<Counters*>(row_region(a, row) + OFF_COUNTERS);
}
__device__ __forceinline__ SlicePart* slice_parts(const es_arguments& a, int64_t row) {
  return reinterpret_cast<SlicePart*>(row_region(a, row) + OFF_PARTS);
}
template <class W> __device__ __forceinline__ Cand<W>* candidates(const es_arguments& a, int64_t row) {
  return reinterpret_cast<Cand<W>*>(row_region(a, row) + OFF_CAND);
}
// A stream row's slice keeps its pick where a list row keeps candidates.
struct Pick;
template <class W> __device__ __forceinline__ Pick* slice_pick(const es_arguments& a, int64_t row, int slice, int cap) {
  return reinterpret_cast<Pick*>(candidates<W>(a, row) + int64_t(slice) * cap);
}
// A binned top-p row's slice keeps its bins at the end of the row region:
// TP_COARSE FP64 masses, then TP_COARSE 16-bit counts.
__device__ __forceinline__ double* slice_bin_mass(const es_arguments& a, int64_t row, int slice) {
  return reinterpret_cast<double*>(row_region(a, row) + ROW_BYTES - size_t(slice + 1) * TP_SLICE_BIN_BYTES);
}
// The boundary area of a binned top-p row of `slices` slices: the gathered
// count, the finishing blocks' picks and the gathered IDs (or the bitmap).
__device__ __forceinline__ uint32_t* bound_count(const es_arguments& a, int64_t row, int slices) {
  return reinterpret_cast<uint32_t*>(row_region(a, row) + bound_area_offset(slices));
}
__device__ __forceinline__ uint32_t* bound_picks(const es_arguments& a, int64_t row, int slices) {
  return bound_count(a, row, slices) + 2;
}
__device__ __forceinline__ uint32_t* bound_ids(const es_arguments& a, int64_t row, int slices) {
  return bound_picks(a, row, slices) + slices * int(TP_PICK_BYTES / 4);
}
// The shared fine bins after the bitmap: masses, then counts.
__device__ __forceinline__ double* bound_fine_mass(const es_arguments& a, int64_t row, int slices) {
  return reinterpret_cast<double*>(bound_ids(a, row, slices) + bound_fine_offset(a.vocab));
}
__device__ __forceinline__ uint32_t* bound_fine_count(const es_arguments& a, int64_t row, int slices) {
  return reinterpret_cast<uint32_t*>(bound_fine_mass(a, row, slices) + TP_FINE_SHARED);
}
__device__ __forceinline__ uint16_t* slice_bin_count(const es_arguments& a, int64_t row, int slice) {
  return reinterpret_cast<uint16_t*>(slice_bin_mass(a, row, slice) + TP_COARSE);
}

// ---------------------------------------------------------------------------
// Metadata (reference verify.cu:6-40; oracle reference.py:177-196).
__device__ __forceinline__ bool offsets_malformed(const es_arguments& a) {
  int bad = 0;
  if (threadIdx.x == 0) bad = at(a.cu_rows, 0) != 0 || at(a.cu_rows, a.requests) != a.rows;
  for (int64_t i = threadIdx.x; i < a.requests; i += BLOCK) {
    const int64_t x = at(a.cu_rows, i), y = at(a.cu_rows, i + 1);
    bad |= x < 0 || y > a.rows || x > y;
  }
  return __syncthreads_or(bad) != 0;
}

__device__ __forceinline__ int32_t metadata_status(const es_arguments& a, int64_t req, bool malformed) {
  if (malformed) return ES_INVALID_INPUT;
  const int64_t begin = at(a.cu_rows, req), end = at(a.cu_rows, req + 1);
  if (begin < 0 || end > a.rows || end <= begin || end - begin > a.max_draft + 1) return ES_INVALID_INPUT;
  const double t = at(a.temperature, req), p = at(a.top_p, req), m = at(a.min_p, req);
  const int64_t k = at(a.top_k, req), kind = at(a.draft_kind, req), stream = at(a.stream, req);
  if (!isfinite(t) || t < 0 || !isfinite(p) || p <= 0 || p > 1 || !isfinite(m) || m < 0 || m > 1 ||
      k < 0 || k > a.vocab || kind < 0 || kind > 1)
    return ES_INVALID_INPUT;
  if ((a.mode == 1 && kind == 1) || (kind == 1 && end - begin > 1 && !a.draft.data) || stream < 0 ||
      uint64_t(stream) > 0xffffffffull)
    return ES_INVALID_INPUT;
  for (int64_t row = begin; row < end; ++row) {
    const int64_t pos = at(a.position, row);
    if (pos < 0 || uint64_t(pos) > 0xffffffffull) return ES_INVALID_INPUT;
    if (row + 1 < end) {
      const int64_t id = draft_at(a, req, row - begin);
      if (id < 0 || id >= a.vocab) return ES_INVALID_INPUT;
    }
  }
  return ES_OK;
}

// The request owning a row of a well-formed batch: the last one starting at or before it.
__device__ __forceinline__ int64_t request_of(const es_arguments& a, int64_t row) {
  int64_t lo = 0, hi = a.requests - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (at(a.cu_rows, mid) <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The path_used value of every request of the call: dispatch 1 ("reference")
// finishes every row on the exact full-row path (reference: verify.cu:5,51).
__device__ __forceinline__ int32_t path_of(const es_arguments& a) {
  return a.dispatch == 1 ? ES_PATH_REFERENCE : ES_PATH_FUSED;
}
__device__ __forceinline__ void write_failed_request(const es_arguments& a, int64_t req, int32_t status, int32_t path) {
  int64_t* tokens = a.tokens + req * a.token_s0;
  for (int64_t i = 0; i <= a.max_draft; ++i) tokens[i * a.token_s1] = -1;
  a.accepted[req * a.accepted_s] = 0;
  a.status[req * a.status_s] = status;
  a.path[req * a.path_s] = path;
}

// Cross-block data. Blocks of one row or request run on different XCDs, whose
// L2 caches are not coherent with each other. Everything one block writes for
// another is stored with device-scope (write-through, sc1) atomic stores and
// read with device-scope atomic loads, so no agent-scope fence (an L2
// write-back and invalidate per block) is needed. Ordering comes from waiting
// for the stores to be acknowledged (vmcnt(0)) before the arrival atomic.
__device__ __forceinline__ void st_dev(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev32(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_dev32(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T> __device__ __forceinline__ void publish(T* dst, const T& v) {
  static_assert(sizeof(T) % 8 == 0, "published in 8-byte words");
  uint64_t w[sizeof(T) / 8];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 8; ++i) st_dev(reinterpret_cast<uint64_t*>(dst) + i, w[i]);
}
template <class T> __device__ __forceinline__ T fetch(const T* src) {
  static_assert(sizeof(T) % 8 == 0, "fetched in 8-byte words");
  uint64_t w[sizeof(T) / 8];
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 8; ++i) w[i] = ld_dev(reinterpret_cast<const uint64_t*>(src) + i);
  T v;
  __builtin_memcpy(&v, w, sizeof(T));
  return v;
}
// Every thread's outstanding stores acknowledged (s_waitcnt vmcnt(0)).
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Arrival on a counter (zeroed earlier in the call); true in every thread of
// the block that arrives last, which may then fetch what the others
// published. The arrival is an agent-scope acquire-release operation: every
// block's stores (acknowledged by every wave, then the barrier) happen before
// its arrival, and the last block's later loads happen after all arrivals.
__device__ __forceinline__ bool arrive(uint32_t* counter, uint32_t expected, int* s_flag) {
  stores_done();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = old + 1 == expected;
  }
  __syncthreads();
  return *s_flag != 0;
}

// The largest slice maximum of a row published in this call: the word holds
// (generation << 32) | key; one of another generation (an earlier call, a
// fresh workspace) counts as nothing published. Keys only grow within a call,
// and each row has at most MAX_SLICES publishers, so the loop ends.
__device__ __forceinline__ void publish_max(unsigned long long* word, uint32_t gen, uint32_t key) {
  const unsigned long long mine = (static_cast<unsigned long long>(gen) << 32) | key;
  unsigned long long old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (uint32_t(old >> 32) != gen || uint32_t(old) < key) {
    const unsigned long long seen = atomicCAS(word, old, mine);
    if (seen == old) break;
    old = seen;
  }
}
// The published maximum (a lower bound on the row maximum), -inf if none.
__device__ __forceinline__ double published_max(unsigned long long* word, uint32_t gen) {
  const unsigned long long v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return uint32_t(v >> 32) == gen ? double(key_value(uint32_t(v))) : -INFINITY;
}
// The largest float at or below v.
__device__ __forceinline__ float float_at_or_below(double v) {
  const float f = float(v);
  return double(f) > v ? nextafterf(f, -INFINITY) : f;
}

// ---------------------------------------------------------------------------
// Shared memory of a block (one union; each phase uses one member).
// A certified FP32 Gumbel-max: the best score mid (higher, then lower ID),
// an interval [lo, hi] holding its exact score, and a bound on every other
// candidate's score.
struct Pick { float mid, lo, hi, others; int id; };
__device__ __forceinline__ Pick pick_none() { return Pick{-INFINITY, -INFINITY, -INFINITY, -INFINITY, INT_MAX}; }
__device__ __forceinline__ Pick pick_join(Pick x, Pick y) {
  const bool yw = y.mid > x.mid || (y.mid == x.mid && y.id < x.id);
  Pick w = yw ? y : x;
  const Pick l = yw ? x : y;
  w.others = fmaxf(fmaxf(x.others, y.others), l.hi);
  return w;
}

template <class W> struct Shared {
  union {
    struct {
      W red_w[WAVES];
      W red_w2[WAVES];
      int red_i[WAVES];
      int red_i2[WAVES];
      double red_d[WAVES];
    } r;
    struct {
      W v[LIST_LIMIT];
      int id[LIST_LIMIT];
      W sv[LIST_LIMIT];
      int sid[LIST_LIMIT];
      double w[LIST_LIMIT];
    } list;
    struct {
      unsigned cnt[2048];
      double mass[2048];
    } hist;
  } u;
  double dred[WAVES];
  DD ddred[WAVES];
  int ired[WAVES];
  float fred[WAVES];
  unsigned long long limbs[SACC_LIMBS];
  int flag;
  int n;
  // Merged row statistics and parameters, broadcast to the block.
  double maximum, runner_up, frontier, sum, err;
  int greedy, runner_up_id, valid, bad, n_cand_total, pruned, frontier_id;
  int n_cand[MAX_SLICES];
  int req_found;
  int64_t req;
  int32_t status;
  int pick;
  unsigned __int128 ck;
  // Slice-block lookup and statistics, one entry per wave (never reused).
  int lk_bad[WAVES], lk_found[WAVES];
  int64_t lk_begin[WAVES], lk_end[WAVES];
  W st_max[WAVES], st_thr[WAVES];
  int st_id[WAVES], st_valid[WAVES], st_bad[WAVES];
  int appended;
  // Stream rows: block merges of picks, the merged pick and the slices to scan again.
  Pick picks[WAVES];
  double sp_mid, sp_lo, sp_hi, sp_others;
  int sp_id;
  unsigned long long sp_rescan;
  // The merge wave's decision, broadcast to the block.
  RowResult wres;
  int wroute, wfallbacks, wdone;
};

// The request's parameters, read once per block.
struct Params {
  int64_t req, begin, end;
  double temperature, top_p, min_p;
  int64_t top_k;
  int32_t status;    // ES_INVALID_INPUT for malformed offsets or invalid request scalars
  int32_t meta_bad;  // a position or draft ID of the request out of range
  int draft_row, verify, coupled, full_q, draft_id;
  RngAddr rng;
};

// A stream row samples from every kept token in one streaming pass: a
// positive temperature, no top-k cut, top-p 1 and no full proposal; min-p
// rows qualify unless the ratio test needs their kept mass.
__device__ __forceinline__ bool stream_row(const Params& p, int64_t vocab) {
  return p.temperature > 0 && !p.full_q && !(p.top_p < 1) && (p.top_k == 0 || p.top_k >= vocab) &&
         !(p.verify && !p.coupled && p.min_p > 0);
}
// The draw a stream row needs: the residual (substream 2, draft excluded) for
// a draft row in ratio mode, the sample (substream 0) otherwise.
__device__ __forceinline__ uint32_t stream_sub(const Params& p) { return p.verify && !p.coupled ? 2u : 0u; }
static_assert(sizeof(Params) <= ROW_META_BYTES, "Params fits the row's meta area");
__device__ __forceinline__ Params* row_meta(const es_arguments& a, int64_t row) {
  return reinterpret_cast<Params*>(row_region(a, row) + OFF_META);
}

// The row's request and its parameters, checked by the whole block: the
// offsets are scanned once (malformed check and owner lookup together) and the
// per-row checks of the request run one row per thread, so the prologue is a
// few independent load rounds rather than a dependent chain.
template <class SH>
__device__ __forceinline__ void block_params(const es_arguments& a, int64_t row, Params* p, SH& sh) {
  const int tid = threadIdx.x;
  if (tid == 0) sh.req_found = -1;
  __syncthreads();
  int bad = 0;
  if (tid == 0) bad = at(a.cu_rows, 0) != 0 || at(a.cu_rows, a.requests) != a.rows;
  for (int64_t i = tid; i < a.requests; i += BLOCK) {
    const int64_t x = at(a.cu_rows, i), y = at(a.cu_rows, i + 1);
    bad |= x < 0 || y > a.rows || x > y;
    if (x <= row && row < y) sh.req_found = int(i);
  }
  const bool malformed = __syncthreads_or(bad) != 0;
  if (malformed || sh.req_found < 0) {
    if (tid == 0) p->status = ES_INVALID_INPUT;
    __syncthreads();
    return;
  }
  const int64_t req = sh.req_found;
  const int64_t begin = at(a.cu_rows, req), end = at(a.cu_rows, req + 1);
  int mbad = end - begin > a.max_draft + 1;
  if (!mbad) {
    if (tid == 0) {
      const double t = at(a.temperature, req), pp = at(a.top_p, req), m = at(a.min_p, req);
      const int64_t k = at(a.top_k, req), kind = at(a.draft_kind, req), stream = at(a.stream, req);
      mbad |= !isfinite(t) || t < 0 || !isfinite(pp) || pp <= 0 || pp > 1 || !isfinite(m) || m < 0 || m > 1 ||
              k < 0 || k > a.vocab || kind < 0 || kind > 1;
      mbad |= (a.mode == 1 && kind == 1) || (kind == 1 && end - begin > 1 && !a.draft.data) || stream < 0 ||
              uint64_t(stream) > 0xffffffffull;
    }
    for (int64_t r = begin + tid; r < end; r += BLOCK) {
      const int64_t pos = at(a.position, r);
      mbad |= pos < 0 || uint64_t(pos) > 0xffffffffull;
      if (r + 1 < end) {
        const int64_t id = draft_at(a, req, r - begin);
        mbad |= id < 0 || id >= a.vocab;
      }
    }
  }
  mbad = __syncthreads_or(mbad);
  if (tid == 0) {
    p->req = req;
    p->status = mbad ? ES_INVALID_INPUT : ES_OK;
    if (!mbad) {
      p->begin = begin;
      p->end = end;
      p->temperature = at(a.temperature, req);
      p->top_p = at(a.top_p, req);
      p->min_p = at(a.min_p, req);
      p->top_k = at(a.top_k, req);
      p->draft_row = row + 1 < end;
      p->coupled = a.mode == 1;
      p->verify = p->draft_row && !p->coupled;
      p->full_q = p->draft_row && at(a.draft_kind, req) == 1;
      p->draft_id = p->draft_row ? int(draft_at(a, req, row - begin)) : -1;
      p->rng.seed = uint64_t(at(a.seed, req));
      p->rng.stream = uint32_t(at(a.stream, req));
      p->rng.position = uint32_t(at(a.position, row));
    }
  }
  __syncthreads();
}

// The owner lookup and scalar parameters of a slice block. x0 and x1 are
// cu_rows[tid] and cu_rows[tid + 1] (valid for tid < requests), loaded before
// the logit tile: waits for them then leave the tile loads in flight. Longer
// offset vectors are scanned in further chunks here. The request's scalar
// parameters are checked (reference verify.cu:6-40); the per-row positions and
// draft IDs are checked by the block that merges the row (request_rows_ok).
template <class SH>
__device__ __forceinline__ void slice_lookup(const es_arguments& a, int64_t row, int64_t x0, int64_t x1, Params* p,
                                             SH& sh) {
  const int tid = threadIdx.x;
  const int64_t R = a.requests;
  int bad = 0, found = -1;
  int64_t fb = 0, fe = 0;
  auto visit = [&](int64_t i, int64_t x, int64_t y) {
    bad |= x < 0 || y > a.rows || x > y || (i == 0 && x != 0) || (i == R - 1 && y != a.rows);
    if (x <= row && row < y) { found = int(i); fb = x; fe = y; }
  };
  if (tid < R) visit(tid, x0, x1);
  for (int64_t i = tid + BLOCK; i < R; i += BLOCK) visit(i, at(a.cu_rows, i), at(a.cu_rows, i + 1));
  const uint64_t any_found = __ballot(found >= 0);
  const int src = any_found ? __ffsll((unsigned long long)any_found) - 1 : 0;
  const int wfound = any_found ? lane_read(found, src) : -1;
  const int64_t wb = lane_read(fb, src), we = lane_read(fe, src);
  const int wbad = __ballot(bad) != 0;
  if (lane_id() == 0) {
    sh.lk_bad[wave_id()] = wbad;
    sh.lk_found[wave_id()] = wfound;
    sh.lk_begin[wave_id()] = wb;
    sh.lk_end[wave_id()] = we;
  }
  __syncthreads();
  int malformed = 0, req = -1;
  int64_t begin = 0, end = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    malformed |= sh.lk_bad[w];
    if (req < 0 && sh.lk_found[w] >= 0) { req = sh.lk_found[w]; begin = sh.lk_begin[w]; end = sh.lk_end[w]; }
  }
  req = __builtin_amdgcn_readfirstlane(req);
  p->status = ES_OK;
  p->meta_bad = 0;
  if (malformed || req < 0 || end - begin > a.max_draft + 1) {
    p->status = ES_INVALID_INPUT;
    return;
  }
  const double t = at(a.temperature, req), pp = at(a.top_p, req), m = at(a.min_p, req);
  const int64_t k = at(a.top_k, req), kind = at(a.draft_kind, req), stream = at(a.stream, req);
  const bool scalar_bad = !isfinite(t) || t < 0 || !isfinite(pp) || pp <= 0 || pp > 1 || !isfinite(m) || m < 0 ||
                          m > 1 || k < 0 || k > a.vocab || kind < 0 || kind > 1 || (a.mode == 1 && kind == 1) ||
                          (kind == 1 && end - begin > 1 && !a.draft.data) || stream < 0 ||
                          uint64_t(stream) > 0xffffffffull;
  if (scalar_bad) {
    p->status = ES_INVALID_INPUT;
    return;
  }
  p->req = req;
  p->begin = begin;
  p->end = end;
  p->temperature = t;
  p->top_p = pp;
  p->min_p = m;
  p->top_k = k;
  p->draft_row = row + 1 < end;
  p->coupled = a.mode == 1;
  p->verify = p->draft_row && !p->coupled;
  p->full_q = p->draft_row && kind == 1;
  p->draft_id = -1;
  p->rng.stream = uint32_t(stream);
}

// What the candidate pass takes for a row, decided by the request's scalars
// (the slice blocks and the finishing block compute it alike): need = 0 no
// candidates, > 0 the slice's top `need`, -1 every valid token if they fit.
struct ListPlan {
  int need, L;
  bool sorted_list;  // a top-k row (k <= 64, within the slice capacity) finished by one wave
  bool need_topp;    // a top-p list: the slices also sum their kept weights
  bool binned;       // a top-p row without a top-k cut or min-p: the slices bin their kept weights
};
__device__ __forceinline__ ListPlan list_plan(const Params& p, int list_max, int cap, int64_t vocab, int slices) {
  ListPlan lp{0, 0, false, false, false};
  if (p.temperature > 0 && list_max > 0 && !p.full_q && !stream_row(p, vocab)) {
    if (p.top_k >= 1 && p.top_k <= list_max) lp.need = int(p.top_k);
    else if (p.top_p < 1 && p.min_p == 0 && (p.top_k == 0 || p.top_k >= vocab) && slices <= TP_SLICES_MAX)
      lp.binned = true;
    else if (p.top_p < 1 && p.min_p == 0) lp.need = TOPP_SLICE_NEED;
    else lp.need = -1;
  }
  lp.L = lp.need > 0 ? min(lp.need, cap) : 0;
  lp.sorted_list = lp.need > 0 && lp.L == lp.need && lp.need <= WAVE && p.top_k >= 1 && p.top_k <= list_max;
  lp.need_topp = lp.need == TOPP_SLICE_NEED && p.top_p < 1 && !(p.top_k >= 1 && p.top_k <= list_max);
  return lp;
}

// The per-row metadata of a request (positions and draft IDs in range),
// checked by one wave.
__device__ __forceinline__ bool request_rows_ok(const es_arguments& a, const Params& p) {
  int bad = 0;
  for (int64_t r = p.begin + lane_id(); r < p.end; r += WAVE) {
    const int64_t pos = at(a.position, r);
    bad |= pos < 0 || uint64_t(pos) > 0xffffffffull;
    if (r + 1 < p.end) {
      const int64_t id = draft_at(a, p.req, r - p.begin);
      bad |= id < 0 || id >= a.vocab;
    }
  }
  return __ballot(bad) == 0;
}

// The row's RNG address and draft ID (range-checked by request_rows_ok
// before any use that depends on the range).
__device__ __forceinline__ void load_row_rng(const es_arguments& a, int64_t row, Params* p) {
  p->rng.seed = uint64_t(at(a.seed, p->req));
  p->rng.position = uint32_t(at(a.position, row));
  p->draft_id = p->draft_row ? int(draft_at(a, p->req, row - p->begin)) : -1;
}

// ---------------------------------------------------------------------------
// The commit of one request from its rows' results (reference verify.cu:169-217),
// run by one wave. Lane l takes rows begin + l, begin + l + 64, ...
__device__ __forceinline__ void finalize_request(const es_arguments& a, int64_t req) {
  const int lane = lane_id();
  const int64_t begin = at(a.cu_rows, req), end = at(a.cu_rows, req + 1);
  int64_t* tokens = a.tokens + req * a.token_s0;
  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t base = begin; base < end; base += WAVE) {
      const int64_t row = base + lane;
      int s = ES_OK;
      if (row < end) {
        const RowResult rr = fetch(row_result(a, row));
        s = pass == 0 ? rr.target_status : rr.status;
      }
      const uint64_t bad = __ballot(s != ES_OK);
      if (bad) {
        const int first = lane_read(s, __ffsll((unsigned long long)bad) - 1);
        for (int64_t i = lane; i <= a.max_draft; i += WAVE) tokens[i * a.token_s1] = -1;
        if (lane == 0) {
          a.accepted[req * a.accepted_s] = 0;
          a.status[req * a.status_s] = first;
          a.path[req * a.path_s] = path_of(a);
        }
        return;
      }
    }
  }
  const uint64_t seed = uint64_t(at(a.seed, req));
  const uint32_t stream = uint32_t(at(a.stream, req));
  int64_t stop = end - 1;
  for (int64_t base = begin; base < end - 1; base += WAVE) {
    const int64_t row = base + lane;
    bool reject = false;
    if (row < end - 1) {
      const RowResult r = fetch(row_result(a, row));
      const int64_t draft = draft_at(a, req, row - begin);
      if (a.mode == 1) {
        reject = r.sample != draft;
      } else {
        const Words w = philox(seed, stream, uint32_t(at(a.position, row)), 1u, 0u);
        reject = !(uniform64(w.w[0]) < fmin(1.0, r.p / r.q));
      }
    }
    const uint64_t rejected = __ballot(reject);
    if (rejected) { stop = base + __ffsll((unsigned long long)rejected) - 1; break; }
  }
  const RowResult r = fetch(row_result(a, stop));
  const int token = stop == end - 1 || a.mode == 1 ? r.sample : r.residual;
  const int64_t accepted = stop - begin;
  const bool empty = stop < end - 1 && token < 0;  // an impossible rejection: invalid, never a token
  for (int64_t i = lane; i <= a.max_draft; i += WAVE) {
    int64_t t = -1;
    if (!empty) t = i < accepted ? draft_at(a, req, i) : i == accepted ? int64_t(token) : -1;
    tokens[i * a.token_s1] = t;
  }
  if (lane == 0) {
    a.accepted[req * a.accepted_s] = empty ? 0 : int32_t(accepted);
    a.status[req * a.status_s] = empty ? ES_INVALID_INPUT : ES_OK;
    a.path[req * a.path_s] = path_of(a);
  }
}

// The call's FP64 recomputation count, workspace word 1: cleared by es_main's
// first block (or by the first request block of a call without rows), then
// added to by each es_finish block that needed one (the kernel boundary
// orders the two).
__device__ __forceinline__ void add_fallbacks(const es_arguments& a, unsigned n) {
  if (n) atomicAdd(reinterpret_cast<unsigned*>(a.workspace) + 1, n);
}

// Publishes a finished row and runs the request commit when this row
// completes its request. Every thread calls it.
template <class W>
__device__ __forceinline__ void complete_row(const es_arguments& a, int64_t row, const Params& p,
                                             const RowResult& result, int fallbacks, int route, Shared<W>& sh) {
  if (threadIdx.x == 0) {
    if (p.end - p.begin > 1) publish(row_result(a, row), result);  // read by the request's finalize
    RowState* st = row_state(a, row);
    st->part = PART_DONE;
    st->route = route;
    st_dev32(&st->fallbacks, fallbacks);
  }
  const int64_t nrows = p.end - p.begin;
  if (nrows == 1) {
    // A request of one row (no drafts) is committed from the result in hand.
    if (threadIdx.x <= a.max_draft) {
      const bool ok = result.status == ES_OK;
      a.tokens[p.req * a.token_s0 + threadIdx.x * a.token_s1] = threadIdx.x == 0 && ok ? result.sample : -1;
    }
    for (int64_t i = int64_t(threadIdx.x) + BLOCK; i <= a.max_draft; i += BLOCK) a.tokens[p.req * a.token_s0 + i * a.token_s1] = -1;
    if (threadIdx.x == 0) {
      a.accepted[p.req * a.accepted_s] = 0;
      a.status[p.req * a.status_s] = result.status;
      a.path[p.req * a.path_s] = path_of(a);
    }
  } else if (arrive(&counters(a, p.begin)->request, uint32_t(nrows), &sh.flag)) {
    if (wave_id() == 0) finalize_request(a, p.req);
  }
}

__device__ __forceinline__ void skip_row(const es_arguments& a, int64_t row) {
  if (threadIdx.x == 0) {
    RowState* st = row_state(a, row);
    st->part = PART_SKIP;
    st->fallbacks = 0;
  }
}

// ---------------------------------------------------------------------------
// Composite order keys: larger means earlier in (logit desc, ID asc) order.
typedef unsigned __int128 u128;
template <class W> struct CK;
template <> struct CK<float> {
  static constexpr int BITS = 64;
  __device__ static __forceinline__ u128 make(float v, int id) {
    return u128((uint64_t(order_key(v)) << 32) | uint64_t(~uint32_t(id)));
  }
  __device__ static __forceinline__ float value(u128 ck) { return key_value(uint32_t(uint64_t(ck) >> 32)); }
};
template <> struct CK<double> {
  static constexpr int BITS = 96;
  __device__ static __forceinline__ u128 make(double v, int id) { return (u128(order_key(v)) << 32) | u128(~uint32_t(id)); }
  __device__ static __forceinline__ double value(u128 ck) { return key_value(uint64_t(ck >> 32)); }
};
__device__ __forceinline__ int ck_id(u128 ck) { return int(~uint32_t(uint64_t(ck))); }

// ---------------------------------------------------------------------------
// Bin of an entry d logits below the row maximum: quarter-logit bins, the last
// one for everything 63.75 or more below. Monotone in d, so a prefix of bins
// holds a prefix of the (value desc) order.
__device__ __forceinline__ int head_bin(double d) {
  return d < double(HEAD_BINS - 1) / 4 ? int(d * 4) : HEAD_BINS - 1;
}

// FP64 draws over a sorted list in LDS: argmax of log(p_i) + G_i with the
// oracle's formula (reference.py:94-104), lowest ID on ties; -1 when empty.
template <class W>
__device__ __forceinline__ int list_draw(const Params& p, Shared<W>& sh, int n, int sub, int excluded) {
  double best = -INFINITY;
  int best_id = INT_MAX;
  for (int i = threadIdx.x; i < n; i += BLOCK) {
    const int id = sh.u.list.sid[i];
    const double pi = sh.u.list.w[i];
    if (id == excluded || !(pi > 0)) continue;
    const double s = log(pi) + gumbel64(word_of(p.rng, uint32_t(sub), uint32_t(id)));
    if (s > best || (s == best && id < best_id)) { best = s; best_id = id; }
  }
  // Reduce (score, id) across the block.
  struct SI { double s; int id; };
  SI v{best, best_id};
  auto op = [](SI x, SI y) { return (y.s > x.s || (y.s == x.s && y.id < x.id)) ? y : x; };
  v = wave_all(v, op, SI{-INFINITY, INT_MAX});
  __syncthreads();
  if (lane_id() == 0) { sh.dred[wave_id()] = v.s; sh.ired[wave_id()] = v.id; }
  __syncthreads();
  SI r{sh.dred[0], sh.ired[0]};
  for (int w = 1; w < WAVES; ++w) r = op(r, SI{sh.dred[w], sh.ired[w]});
  __syncthreads();
  return r.id == INT_MAX ? -1 : r.id;
}

// DD sum over the block in thread order (deterministic for a fixed block shape).
template <class W> __device__ __forceinline__ DD block_dd(DD v, Shared<W>& sh) {
  return block_all(v, [](DD x, DD y) { return dd_add(x, y); }, sh.ddred, DD{0, 0});
}

// The correctly rounded sum of sh.u.list.w[0, n): certified DD, else exact
// (an exact sum on a rounding tie is part of the FP64 path, not a fallback).
template <class W> __device__ __forceinline__ double list_fsum(Shared<W>& sh, int n) {
  DD acc{0, 0};
  for (int i = threadIdx.x; i < n; i += BLOCK) acc = dd_add(acc, DD{sh.u.list.w[i], 0});
  acc = block_dd(acc, sh);
  double r;
  if (dd_round_certain(acc, dd_sum_error(acc, n), &r)) return r;
  sacc_clear(sh.limbs);
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += BLOCK) sacc_add(sh.limbs, sh.u.list.w[i]);
  __syncthreads();
  if (wave_id() == 0) {  // rounded across wave 0, read by the block
    const double sum = sacc_round_wave(sh.limbs);
    if (lane_id() == 0) sh.dred[0] = sum;
  }
  __syncthreads();
  r = sh.dred[0];
  __syncthreads();
  return r;
}

// Does round(P) reach t, for P known as a DD within err? 1 yes, 0 no, -1 not certain.
__device__ __forceinline__ int dd_reaches(DD P, double err, double t) {
  const double below = nextafter(t, 0.0);
  const DD lo = dd_add(P, DD{-t, 0});       // P - t
  if (lo.hi - err >= 0) return 1;           // P >= t
  const DD lo2 = dd_add(P, DD{-below, 0});  // P - pred(t)
  if (lo2.hi + err < 0) return 0;           // P < pred(t)
  return -1;
}

// Finishes a list row from the candidates of its slices. Returns false when the
// candidates cannot settle the row; the full-row path then takes it.
// The kept set is a prefix of (logit desc, ID asc) order: min-p and positivity
// remove a suffix, top-k keeps a prefix and top-p keeps a prefix.
template <class W>
__device__ __forceinline__ bool list_finish(const es_arguments& a, int64_t row, const Params& p, Shared<W>& sh, int slices,
                            int cap_slice, bool topk_mode, int n_keep, RowResult* result, int* fallbacks,
                                              int* why) {
  // Every valid token at or before (F, F_id) in (value desc, ID asc) order
  // is among the candidates; sorted, they are the exact head of the order.
  const double F = sh.frontier;
  const int F_id = sh.frontier_id;
  if (!(F < INFINITY)) { *why = 1; return false; }
  if (threadIdx.x == 0) sh.n = 0;
  __syncthreads();
  const Cand<W>* cands = candidates<W>(a, row);
  const int total_slots = slices * cap_slice;
  for (int idx = threadIdx.x; idx < total_slots; idx += BLOCK) {
    const int s = idx / cap_slice, i = idx - s * cap_slice;
    if (i >= sh.n_cand[s]) continue;
    const Cand<W> c = fetch(cands + idx);
    if (!(double(c.v) > F || (double(c.v) == F && c.id <= F_id))) continue;
    const int slot = atomicAdd(&sh.n, 1);
    if (slot < LIST_LIMIT) { sh.u.list.v[slot] = c.v; sh.u.list.id[slot] = c.id; }
  }
  __syncthreads();
  const int n_u = sh.n;
  __syncthreads();
  if (n_u > LIST_LIMIT || n_u == 0) { *why = 2; return false; }
  if (topk_mode && n_u < n_keep) { *why = 3; return false; }
  // Only the head of the union is needed: bin the entries by distance below
  // the row maximum (quarter-logit bins) and keep the bins up to the one that
  // completes the first `want` entries; rank-sort just those.
  const int want = topk_mode ? n_keep : min(n_u, TOPP_HEAD);
  const double M0 = sh.maximum;
  unsigned* bins = reinterpret_cast<unsigned*>(sh.u.list.sid);  // HEAD_BINS counters
  for (int i = threadIdx.x; i < HEAD_BINS; i += BLOCK) bins[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n_u; i += BLOCK)
    atomicAdd(&bins[head_bin(M0 - double(sh.u.list.v[i]))], 1u);
  __syncthreads();
  int cut_bin = HEAD_BINS - 1;
  {
    const int c = threadIdx.x < HEAD_BINS ? int(bins[threadIdx.x]) : 0;
    int tot;
    const int incl = block_scan_add(c, sh.ired, &tot);
    if (threadIdx.x < HEAD_BINS && incl >= want && incl - c < want) sh.pick = int(threadIdx.x);
    __syncthreads();
    cut_bin = sh.pick;
    __syncthreads();
  }
  // Compact the head entries into (sv, sid), rank-sort them into (v, id),
  // and copy the sorted head back to (sv, sid).
  if (threadIdx.x == 0) sh.n = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n_u; i += BLOCK) {
    const W x = sh.u.list.v[i];
    if (head_bin(M0 - double(x)) <= cut_bin) {
      const int slot = atomicAdd(&sh.n, 1);
      sh.u.list.sv[slot] = x;
      sh.u.list.sid[slot] = sh.u.list.id[i];
    }
  }
  __syncthreads();
  const int n_h = sh.n;  // every entry outside the head comes after all of these
  const bool whole_union = n_h == n_u;
  const int n_out = topk_mode ? n_keep : n_h;
  // Rank sort: each thread ranks its entries against all n_h, four loads in flight.
  for (int i = threadIdx.x; i < n_h; i += BLOCK) {
    const W vi = sh.u.list.sv[i];
    const int ii = sh.u.list.sid[i];
    int rank = 0, j = 0;
    for (; j + 4 <= n_h; j += 4) {
      const W v0 = sh.u.list.sv[j], v1 = sh.u.list.sv[j + 1], v2 = sh.u.list.sv[j + 2], v3 = sh.u.list.sv[j + 3];
      const int d0 = sh.u.list.sid[j], d1 = sh.u.list.sid[j + 1], d2 = sh.u.list.sid[j + 2], d3 = sh.u.list.sid[j + 3];
      rank += before(v0, d0, vi, ii) + before(v1, d1, vi, ii) + before(v2, d2, vi, ii) + before(v3, d3, vi, ii);
    }
    for (; j < n_h; ++j) rank += before(sh.u.list.sv[j], sh.u.list.sid[j], vi, ii);
    if (rank < n_out) { sh.u.list.v[rank] = vi; sh.u.list.id[rank] = ii; }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n_out; i += BLOCK) {
    sh.u.list.sv[i] = sh.u.list.v[i];
    sh.u.list.sid[i] = sh.u.list.id[i];
  }
  __syncthreads();
  // FP64 weights with the oracle's formula, and the min-p/positivity cut.
  const double M = sh.maximum, T = p.temperature;
  int first_out = INT_MAX;
  for (int i = threadIdx.x; i < n_out; i += BLOCK) {
    const double w = exp((double(sh.u.list.sv[i]) - M) / T);
    sh.u.list.w[i] = w;
    if (!(w >= p.min_p && w > 0.0)) first_out = min(first_out, i);
  }
  first_out = block_all(first_out, [](int x, int y) { return x < y ? x : y; }, sh.ired, INT_MAX);
  const int n1 = min(n_out, first_out);
  int n2 = n1;
  if (p.top_p < 1) {
    double lo_t, hi_t;
    const bool whole = topk_mode || (whole_union && n_u == sh.valid);  // the list is the whole kept set
    if (whole) {
      const double total = list_fsum(sh, n1);
      lo_t = hi_t = p.top_p * total;
    } else {
      if (!(sh.err >= 0) || !(sh.sum - sh.err > 0)) { *why = 4; return false; }
      lo_t = p.top_p * (sh.sum - sh.err) * (1 - 1e-15);
      hi_t = p.top_p * (sh.sum + sh.err) * (1 + 1e-15);
    }
    // Inclusive DD prefix sums: thread t owns entries [4t, 4t + 4).
    constexpr int PER = LIST_LIMIT / BLOCK;
    DD local{0, 0};
    for (int u = 0; u < PER; ++u) {
      const int i = PER * threadIdx.x + u;
      if (i < n1) local = dd_add(local, DD{sh.u.list.w[i], 0});
    }
    // Exclusive scan of the per-thread sums in thread order.
    const DD incl = wave_scan(local, [](DD x, DD y) { return dd_add(x, y); }, DD{0, 0});
    const int lane = lane_id();
    __syncthreads();
    if (lane == WAVE - 1) sh.ddred[wave_id()] = incl;
    __syncthreads();
    DD before_w{0, 0};
    for (int w = 0; w < wave_id(); ++w) before_w = dd_add(before_w, sh.ddred[w]);
    const DD excl_t = dd_add(before_w, dd_add(incl, DD{-local.hi, -local.lo}));
    int first_lo = INT_MAX, first_hi = INT_MAX, unsure = INT_MAX;
    DD run = excl_t;
    for (int u = 0; u < PER; ++u) {
      const int i = PER * threadIdx.x + u;
      if (i >= n1) break;
      run = dd_add(run, DD{sh.u.list.w[i], 0});
      const double err = dd_sum_error(run, i + 1) + 4 * 0x1p-104 * run.hi;
      const int rl = dd_reaches(run, err, lo_t), rh = dd_reaches(run, err, hi_t);
      if (rl != 0) first_lo = min(first_lo, i);
      if (rh != 0) first_hi = min(first_hi, i);
      if (rl < 0 || rh < 0) unsure = min(unsure, i);
    }
    auto mn = [](int x, int y) { return x < y ? x : y; };
    first_lo = block_all(first_lo, mn, sh.ired, INT_MAX);
    first_hi = block_all(first_hi, mn, sh.ired, INT_MAX);
    unsure = block_all(unsure, mn, sh.ired, INT_MAX);
    if (first_lo == INT_MAX && first_hi == INT_MAX && unsure == INT_MAX) {
      // No prefix of the list reaches the target.
      if (!whole) { *why = 6; return false; }  // the nucleus extends past the list
      n2 = n1;
    } else {
      if (unsure <= first_hi || first_lo != first_hi) { *why = 5; return false; }
      n2 = first_hi + 1;
    }
  }
  const double den = list_fsum(sh, n2);
  for (int i = threadIdx.x; i < n2; i += BLOCK) sh.u.list.w[i] = sh.u.list.w[i] / den;
  __syncthreads();
  RowResult r{0, 1, -1, -1, ES_OK, ES_OK};
  if (p.verify) {
    int at_draft = INT_MAX;
    for (int i = threadIdx.x; i < n2; i += BLOCK)
      if (sh.u.list.sid[i] == p.draft_id) at_draft = i;
    at_draft = block_all(at_draft, [](int x, int y) { return x < y ? x : y; }, sh.ired, INT_MAX);
    const double px = at_draft == INT_MAX ? 0.0 : sh.u.list.w[at_draft];
    const double u = uniform64(word_of(p.rng, 1u, 0u));
    const bool accept = u < fmin(1.0, px);
    r.p = accept ? 1.0 : 0.0;
    if (!accept) r.residual = list_draw(p, sh, n2, 2, p.draft_id);
  } else {
    r.sample = list_draw(p, sh, n2, 0, -1);
  }
  *result = r;
  return true;
}

// ---------------------------------------------------------------------------
// Top-k rows (k <= 64) finished by one wave from the slices' sorted lists.
//
// Every slice stored its first min(k, valid) tokens in (value desc, ID asc)
// order; the last of them is its frontier (none when it stored every valid
// token). The union is complete down to the earliest frontier F, and the
// slice owning F stored k tokens up to it, so the row's first k tokens are in
// the union at or before F. Among those entries a bitwise search on ballots
// finds the k-th largest value T; the pool (the entries >= T: the first k
// plus any ties at T) is rank-sorted and the FP64 finish follows the oracle
// (reference.py:60-104): weights exp((l - max) / T), the min-p/positivity
// cut, the top-k prefix, the shortest top-p prefix by certified double-double
// prefix sums, the correctly rounded denominator and the Gumbel-argmax draw.
//
// Returns 1 with *out set, 0 when the union or the pool does not fit (the
// block list takes the row) and -1 when a rounding could not be certified
// (the full-row path recomputes it exactly).
constexpr int WAVE_BATCH = 8;      // candidate slots per lane fetched together
constexpr int UNION_PER_LANE = 8;  // union entries per lane the wave selects from

// The position of each lane's (v, id) among the first n lanes' entries in
// (value desc, ID asc) order; entries are distinct. Lane values are read with
// readlane (no LDS round trips).
template <class W> __device__ __forceinline__ int wave_rank(W v, int id, int n) {
  int rank = 0;
  if constexpr (sizeof(W) == 4) {
    // One 64-bit key per entry, larger = earlier: the value's order key, then
    // the inverted ID. Read four lanes at a time, so the reads of a batch do
    // not wait on one another.
    const uint64_t key = (uint64_t(order_key(v)) << 32) | uint64_t(~uint32_t(id));
    int j = 0;
    for (; j + 4 <= n; j += 4) {
      uint64_t k[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) k[u] = lane_read(key, j + u);
#pragma unroll
      for (int u = 0; u < 4; ++u) rank += k[u] > key;
    }
    for (; j < n; ++j) rank += lane_read(key, j) > key;
  } else {
    for (int j = 0; j < n; ++j) rank += before(lane_read(v, j), lane_read(id, j), v, id);
  }
  return rank;
}

// The slot layout of the merge wave's prefetch: slice s's first `pref`
// candidates at slots s * pref + i; idx / pref by a 20-bit reciprocal, exact
// for idx < 2^12 and pref < 256.
struct SlotMap {
  int pref;
  uint32_t inv;
  __device__ __forceinline__ explicit SlotMap(int pref_) : pref(pref_), inv(((1u << 20) + uint32_t(pref_) - 1) / uint32_t(pref_)) {}
  __device__ __forceinline__ int slice(int idx) const { return int((uint64_t(uint32_t(idx)) * inv) >> 20); }
};

template <class W>
__device__ __forceinline__ int wave_topk(const es_arguments& a, int64_t row, const Params& p, Shared<W>& sh,
                                         const Cand<W> (&pre)[WAVE_BATCH], const SlotMap& map, int slices, int cap,
                                         int lane_n_cand, double M, double F, int F_id, int valid_all,
                                         RowResult* out) {
  using K = typename std::conditional<sizeof(W) == 8, uint64_t, uint32_t>::type;
  const int lane = lane_id();
  const int pref = map.pref;
  // The union at or before F, compacted into LDS. The row's greedy token (the
  // lowest ID holding the maximum M) is among it: every slice stored its
  // tokens at its own maximum.
  int n_u = 0, greedy = INT_MAX;
  auto add = [&](bool take, const Cand<W>& c) {
    const uint64_t mk = __ballot(take);
    const int pos = n_u + __popcll(mk & ((1ull << lane) - 1ull));
    if (take && pos < WAVE * UNION_PER_LANE) { sh.u.list.v[pos] = c.v; sh.u.list.id[pos] = c.id; }
    if (take && double(c.v) == M && c.id < greedy) greedy = c.id;
    n_u += __popcll(mk);
  };
  auto at_or_before_F = [&](const Cand<W>& c) {
    const double d = double(c.v);
    return d > F || (d == F && c.id <= F_id);
  };
  // The slot's slice count is read for every slot first (independent LDS
  // reads, one wait), then the slots are appended.
  bool take_r[WAVE_BATCH];
#pragma unroll
  for (int r = 0; r < WAVE_BATCH; ++r) {
    const int idx = lane + WAVE * r;
    const int sl = map.slice(idx);
    const int n_sl = sh.n_cand[min(sl, MAX_SLICES - 1)];
    take_r[r] = (idx < slices * pref) & (idx - sl * pref < n_sl);
  }
#pragma unroll
  for (int r = 0; r < WAVE_BATCH; ++r) add(take_r[r] && at_or_before_F(pre[r]), pre[r]);
  // Candidates beyond the prefetch (a slice that stored more than `pref`).
  const Cand<W>* cands = candidates<W>(a, row);
  const bool overflow = __ballot(lane < slices && lane_n_cand > pref) != 0;
  for (int sl = 0; overflow && sl < slices; ++sl) {
    const int n_s = sh.n_cand[sl];
    for (int base = pref; base < n_s; base += WAVE) {
      const int i = base + lane;
      Cand<W> c{};
      if (i < n_s) c = fetch(cands + sl * cap + i);
      add(i < n_s && at_or_before_F(c), c);
    }
  }
  greedy = wave_all(greedy, [](int x, int y) { return x < y ? x : y; }, INT_MAX);
  if (lane == 0) sh.greedy = greedy;
  const int n_keep = p.top_k > 0 && p.top_k < valid_all ? int(p.top_k) : valid_all;
  if (n_u > WAVE * UNION_PER_LANE) return 0;
  if (n_u < n_keep || n_keep < 1) return -1;  // cannot happen for a complete union
  W v = neg_inf<W>();
  int id = INT_MAX;
  int n_pool;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (n_u <= WAVE) {
    // The whole union fits one entry per lane: it is the pool.
    n_pool = n_u;
    if (lane < n_pool) { v = sh.u.list.v[lane]; id = sh.u.list.id[lane]; }
  } else {
    // Bins of the union by distance below the row maximum (quarter logits, the
    // last bin for 63.75 and more): monotone in the order, so the bins up to the
    // one holding the n_keep-th entry hold a prefix of the order (the pool).
    unsigned* bins = reinterpret_cast<unsigned*>(sh.u.list.sid);  // HEAD_BINS counters
#pragma unroll
    for (int r = 0; r < HEAD_BINS / WAVE; ++r) bins[lane + WAVE * r] = 0;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int per = (n_u + WAVE - 1) / WAVE;
    int bin_of[UNION_PER_LANE];
#pragma unroll
    for (int r = 0; r < UNION_PER_LANE; ++r) {
      const int idx = lane + WAVE * r;
      bin_of[r] = HEAD_BINS;
      if (r < per && idx < n_u) {
        bin_of[r] = head_bin(M - double(sh.u.list.v[idx]));
        atomicAdd(&bins[bin_of[r]], 1u);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // Lane l owns bins [4l, 4l + 4): the first bin whose running total reaches n_keep.
    constexpr int BPL = HEAD_BINS / WAVE;
    unsigned bc[BPL], local = 0;
#pragma unroll
    for (int q = 0; q < BPL; ++q) { bc[q] = bins[BPL * lane + q]; local += bc[q]; }
    const unsigned incl_b = wave_scan_add(local);
    int mine_cut = INT_MAX;
    unsigned run = incl_b - local;
#pragma unroll
    for (int q = 0; q < BPL; ++q) {
      run += bc[q];
      if (mine_cut == INT_MAX && run >= unsigned(n_keep)) mine_cut = BPL * lane + q;
    }
    const int cut_bin = wave_all(mine_cut, [](int x, int y) { return x < y ? x : y; }, INT_MAX);
    // The pool: union entries in bins up to cut_bin, one per lane.
    n_pool = 0;
#pragma unroll
    for (int r = 0; r < UNION_PER_LANE; ++r) {
      if (r >= per) break;
      const int idx = lane + WAVE * r;
      const bool take = idx < n_u && bin_of[r] <= cut_bin;
      const uint64_t mk = __ballot(take);
      const int pos = n_pool + __popcll(mk & ((1ull << lane) - 1ull));
      if (take && pos < WAVE) { sh.u.list.sv[pos] = sh.u.list.v[idx]; sh.u.list.w[pos] = double(sh.u.list.id[idx]); }
      n_pool += __popcll(mk);
    }
    if (n_pool > WAVE) return 0;  // a wide tie at the k-th value
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // Rank sort of the pool, one entry per lane.
    if (lane < n_pool) { v = sh.u.list.sv[lane]; id = int(sh.u.list.w[lane]); }
  }
  const int rank = wave_rank(v, id, n_pool);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (lane < n_pool) { sh.u.list.v[rank] = v; sh.u.list.id[rank] = id; }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  if (lane < n_pool) { v = sh.u.list.v[lane]; id = sh.u.list.id[lane]; }
  // Weights and the min-p/positivity cut (a suffix of the order).
  const double T = p.temperature;
  const bool in_k = lane < n_keep;
  const double w = in_k ? exp((double(v) - M) / T) : 0.0;
  const uint64_t out_mask = __ballot(in_k && !(w >= p.min_p && w > 0.0));
  const int n1 = out_mask ? min(n_keep, __ffsll((unsigned long long)out_mask) - 1) : n_keep;
  const double wk = lane < n1 ? w : 0.0;
  // Inclusive double-double prefix sums in lane order, each with its bound.
  const DD incl = wave_scan(DD{wk, 0}, [](DD x, DD y) { return dd_add(x, y); }, DD{0, 0});
  const double err = dd_sum_error(incl, lane + 1) + 4 * 0x1p-104 * incl.hi;
  // The correctly rounded sum of the first n weights (math.fsum): certified
  // from the double-double prefix, or, when the exact sum may sit on a
  // rounding tie (sums of two or three bf16-derived weights often do),
  // computed exactly with the LDS superaccumulator.
  auto rounded_prefix = [&](int n) {
    const DD s = lane_read(incl, n - 1);
    double r;
    if (dd_round_certain(s, dd_sum_error(s, n) + 4 * 0x1p-104 * s.hi, &r)) return r;
    if (lane < SACC_LIMBS) sh.limbs[lane] = 0;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane < n) sacc_add(sh.limbs, wk);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    return sacc_round_wave(sh.limbs);
  };
  if (n1 == 0) return -1;  // the maximum always survives; defensive
  double den = rounded_prefix(n1);
  int count = n1;
  if (p.top_p < 1) {
    // The shortest prefix whose rounded sum reaches top_p * den
    // (reference.py:76-83): certain lanes from the double-double bounds, the
    // uncertain ones before the first certain hit decided exactly, in order.
    const double target = p.top_p * den;
    const int reach = lane < n1 ? dd_reaches(incl, err, target) : 0;
    const uint64_t yes = __ballot(reach == 1);
    const int first_yes = yes ? __ffsll((unsigned long long)yes) - 1 : n1;
    uint64_t unsure = __ballot(reach < 0) & (first_yes < WAVE ? (1ull << first_yes) - 1ull : ~0ull);
    count = yes ? first_yes + 1 : n1;
    while (unsure) {
      const int j = __ffsll((unsigned long long)unsure) - 1;
      unsure &= unsure - 1;
      if (rounded_prefix(j + 1) >= target) { count = j + 1; break; }
    }
    if (count != n1) den = rounded_prefix(count);
  }
  const bool kept = lane < count;
  const double pr = kept ? wk / den : 0.0;
  // Gumbel-argmax over kept tokens with positive probability, lowest ID on
  // ties. The scores log(p) + G differ from x + G by the common -log(den), so
  // an FP32 x + G with its certified bound decides unless two scores are
  // within FP32 error; then the FP64 scores decide.
  auto draw = [&](uint32_t sub, int excluded) {
    const bool in = kept && pr > 0 && id != excluded;
    const uint32_t word = word_of(p.rng, sub, uint32_t(in ? id : 0));
    Pick pk = pick_none();
    if (in) {
      const float x = float((double(v) - M) / T), g = gumbel32(word), sc = x + g;
      const float e = SCORE_ERR * (1.f + fabsf(x) + fabsf(g));
      pk = Pick{sc, sc - e, sc + e, -INFINITY, id};
    }
    pk = wave_all(pk, pick_join, pick_none());
    if (pk.id == INT_MAX) return -1;
    if (pk.lo > pk.others) return pk.id;
    double s = -INFINITY;
    int sid = INT_MAX;
    if (in) {
      s = log(pr) + gumbel64(word);
      sid = id;
    }
    struct SI { double s; int id; };
    const SI best = wave_all(SI{s, sid}, [](SI x, SI y) { return (y.s > x.s || (y.s == x.s && y.id < x.id)) ? y : x; },
                             SI{-INFINITY, INT_MAX});
    return best.id == INT_MAX ? -1 : best.id;
  };
  RowResult r{0, 1, -1, -1, ES_OK, ES_OK};
  if (p.verify) {
    const uint64_t at = __ballot(kept && id == p.draft_id);
    const double px = at ? lane_read(pr, __ffsll((unsigned long long)at) - 1) : 0.0;
    const double u = uniform64(word_of(p.rng, 1u, 0u));
    const bool accept = u < fmin(1.0, px);
    r.p = accept ? 1.0 : 0.0;
    if (!accept) r.residual = draw(2u, p.draft_id);
  } else {
    r.sample = draw(0u, -1);
  }
  *out = r;
  return 1;
}

// ---------------------------------------------------------------------------
// The streaming draw of stream rows (reference: fused.cuh:532-681 row_scan and
// its Pick merge :301-314).
template <class SH> __device__ __forceinline__ Pick block_pick(Pick pk, SH& sh) {
  pk = wave_all(pk, pick_join, pick_none());
  __syncthreads();
  if (lane_id() == 0) sh.picks[wave_id()] = pk;
  __syncthreads();
  Pick r = sh.picks[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) r = pick_join(r, sh.picks[w]);
  __syncthreads();
  return r;
}

// A thread's Kahan sum of exp(x) over kept tokens with x >= SUM_PRUNE, its
// error bound term, and the count of kept tokens below SUM_PRUNE.
struct KahanSum {
  float s = 0.f, c = 0.f, e = 0.f;
  int pruned = 0;
  float pruned_max = -INFINITY;  // the largest x left out
  __device__ __forceinline__ void add(float x) {
    if (!(x >= SUM_PRUNE)) {
      ++pruned;
      pruned_max = fmaxf(pruned_max, x);
      return;
    }
    const float w = weight32(x), d = w - c, t = s + d;
    c = (t - s) - d;
    s = t;
    e += w * (X_ERR * (1.f + fabsf(x)));
  }
};

// One group of four tokens into a thread's certified pick: tokens whose bit
// is set in `bits`, above -inf, not `excluded` and passing keep(v, x), scored
// x + G(word(sub, t)) with x = tp.x32(v). A token whose score bound stays
// under `bar` (the floor, then the thread's best lower bound) needs no Philox
// word; one Philox call serves the group's four tokens. With SUM, every such
// token (the excluded one too) also goes into `sum`.
template <bool SUM, bool SLOW, class W, class Keep>
__device__ __forceinline__ void pick_group(int g, const W (&x)[4], uint32_t bits, const Temp<W>& tp,
                                           const RngAddr& rng, uint32_t sub, int excluded, Keep&& keep, Pick& best,
                                           float& bar, KahanSum* sum) {
  // Score bounds from xe = x + SE |x| (SE = SCORE_ERR): a token scores at
  // most x + G + SE (1 + |x| + |G|) <= xe + UB0 before its noise is known
  // (G < GUMBEL_MAX), and <= xe + gb + UB1 with the noise bound gb (|gb| <
  // GUMBEL_UPPER_MAX). A token whose bound is below the bar cannot win: only
  // its bound joins `others`. The screens use the bar as the group starts.
  constexpr float UB0 = GUMBEL_MAX + SCORE_ERR * (1.f + GUMBEL_MAX);
  constexpr float UB1 = SCORE_ERR * (1.f + GUMBEL_UPPER_MAX);
  float xs[4], xe[4];
  uint32_t live = 0;
  const float bar0 = bar - UB0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const W v = x[j];
    xs[j] = tp.template x32_as<SLOW>(v);
    xe[j] = fmaf(fabsf(xs[j]), SCORE_ERR, xs[j]);
    const bool ok = ((bits >> j) & 1u) && v > neg_inf<W>() && keep(v, xs[j]);
    if constexpr (SUM) {
      if (ok) sum->add(xs[j]);
    }
    const bool cand = ok && 4 * g + j != excluded;
    const bool low = xe[j] < bar0;
    best.others = fmaxf(best.others, cand && low ? xe[j] + UB0 : -INFINITY);
    live |= cand && !low ? 1u << j : 0u;
  }
  if (!live) return;
  const Words w4 = philox(rng.seed, rng.stream, rng.position, sub, uint32_t(g));
  const float bar1 = bar - UB1;
  uint32_t close = 0;  // tokens whose bound reaches the bar: scored with the accurate noise
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float ub = xe[j] + gumbel_upper(w4.w[j]);
    const bool on = (live >> j) & 1u;
    const bool low = ub < bar1;
    best.others = fmaxf(best.others, on && low ? ub + UB1 : -INFINITY);
    close |= on && !low ? 1u << j : 0u;
  }
  while (close) {
    const int j = __ffs(close) - 1;
    close &= close - 1;
    const uint32_t w = j == 0 ? w4.w[0] : j == 1 ? w4.w[1] : j == 2 ? w4.w[2] : w4.w[3];
    const float xj = j == 0 ? xs[0] : j == 1 ? xs[1] : j == 2 ? xs[2] : xs[3];
    const float G = gumbel32(w), sc = xj + G, e = SCORE_ERR * (1.f + fabsf(xj) + fabsf(G));
    const int t = 4 * g + j;
    if (sc > best.mid || (sc == best.mid && t < best.id)) {
      best.others = fmaxf(best.others, best.hi);
      best = Pick{sc, sc - e, sc + e, best.others, t};
    } else {
      best.others = fmaxf(best.others, sc + e);
    }
    bar = fmaxf(bar, best.lo - PRUNE_MARGIN);
  }
}

// The thread's certified pick over the allowed tokens of groups [g_begin,
// g_end) read from memory, B groups in flight per thread (thread k takes
// g_begin + k, + BLOCK, ...).
template <int B, bool SUM, bool SLOW, int DT, bool VEC, class Keep>
__device__ __forceinline__ Pick range_pick_as(const es_arguments& a, int64_t row, const RowView<DT, VEC>& view,
                                              int g_begin, int g_end, const Temp<typename Ty<DT>::W>& tp,
                                              const RngAddr& rng, uint32_t sub, int excluded, float floor,
                                              Keep&& keep, KahanSum* sum) {
  using W = typename Ty<DT>::W;
  Pick best = pick_none();
  float bar = floor - PRUNE_MARGIN;
  // Every lane runs the same number of rounds (groups past the range carry no
  // tokens), so after each round the wave can share its best lower bound: a
  // token whose upper bound stays below it cannot win, and is kept only as a
  // loser's bound, as with the thread's own best.
  for (int base0 = g_begin; base0 < g_end; base0 += B * BLOCK) {
    const int base = base0 + int(threadIdx.x);
    W x[B][4];
    uint32_t mb[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int g = base + u * BLOCK;
      view.load(min(g, g_end - 1), x[u]);
      mb[u] = g < g_end ? group_bits(a, row, g) : 0u;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      pick_group<SUM, SLOW>(base + u * BLOCK, x[u], mb[u], tp, rng, sub, excluded, keep, best, bar, sum);
    const float wave_lo = wave_all(best.lo, [](float p, float q) { return p > q ? p : q; }, -INFINITY);
    bar = fmaxf(bar, wave_lo - PRUNE_MARGIN);
  }
  return best;
}
template <int B, bool SUM, int DT, bool VEC, class Keep>
__device__ __forceinline__ Pick range_pick(const es_arguments& a, int64_t row, const RowView<DT, VEC>& view,
                                           int g_begin, int g_end, const Temp<typename Ty<DT>::W>& tp,
                                           const RngAddr& rng, uint32_t sub, int excluded, float floor, Keep&& keep,
                                           KahanSum* sum) {
  if (tp.slow)
    return range_pick_as<B, SUM, true>(a, row, view, g_begin, g_end, tp, rng, sub, excluded, floor, keep, sum);
  return range_pick_as<B, SUM, false>(a, row, view, g_begin, g_end, tp, rng, sub, excluded, floor, keep, sum);
}

// ---------------------------------------------------------------------------
// The full-row path's binned top-p boundary works on bins of the absolute
// grid y = l * 4 / T (see slice_bins): bin b = floor(y) holds a run of
// consecutive tokens of the (logit desc, ID asc) order, since floor(l * 4 / T)
// is monotone in l. A dense boundary bin is split 64 ways on the finer grid
// floor(64 y), which nests in it.
constexpr int TP_BINS = 1024;  // fine bins of the boundary's coarse range, at most
constexpr int TP_GATHER_MAX = 2048;  // gathered tokens of the boundary's bins, at most (4-byte logits)
template <class W> constexpr int tp_gather_cap() { return sizeof(W) == 4 ? TP_GATHER_MAX : TP_GATHER_MAX / 2; }
constexpr int TP_FINE = 64;  // fine bins per coarse bin (y * 64 on the same grid)
constexpr int TP_SCALARS = 16;

// e^d for |d| <= 1/8: the Taylor polynomial through d^9 (truncation below
// 3e-16 relative, inside the 1e-14 the bin masses' bound allows), in FP64
// with explicit fused multiply-adds.
__device__ __forceinline__ double exp_center(double d) {
  double r = 1.0 / 362880.0;
  r = fma(r, d, 1.0 / 40320.0);
  r = fma(r, d, 1.0 / 5040.0);
  r = fma(r, d, 1.0 / 720.0);
  r = fma(r, d, 1.0 / 120.0);
  r = fma(r, d, 1.0 / 24.0);
  r = fma(r, d, 1.0 / 6.0);
  r = fma(r, d, 0.5);
  r = fma(r, d, 1.0);
  return fma(r, d, 1.0);
}

// e^d for |d| <= 1/64 + tiny: the Taylor polynomial through d^7 (truncation
// below 2e-17), in FP64 with explicit fused multiply-adds.
__device__ __forceinline__ double exp_near_zero(double d) {
  double r = 1.0 / 5040.0;
  r = fma(r, d, 1.0 / 720.0);
  r = fma(r, d, 1.0 / 120.0);
  r = fma(r, d, 1.0 / 24.0);
  r = fma(r, d, 1.0 / 6.0);
  r = fma(r, d, 0.5);
  r = fma(r, d, 1.0);
  return fma(r, d, 1.0);
}

// The row's bins (es_finish only; the gathered tokens of the boundary bins
// live in the block's list union).
// A wave's queue of groups whose tokens may win a Gumbel-max draw, drained
// 64 at a time with one group per lane (see DensePick): room for a round of
// PQ_ROUND offers per lane on top of 63 left from the last drain.
constexpr int PQ_ROUND = 8;
constexpr int PQ_CAP = WAVE * (PQ_ROUND + 1);
struct PickQueue {
  int g[WAVES][PQ_CAP];          // group
  uint32_t live[WAVES][PQ_CAP];  // its candidates (bit j: token 4 g + j)
};

struct TopPBins {
  double mass[TP_GATHER_MAX];  // fine bins: sum over the bin's kept tokens of their weights relative to
                              // the bin's centre; later the gathered tokens' FP64 weights
  unsigned cnt[TP_BINS];  // kept tokens in the bin
  double scal[TP_SCALARS];
  int n;                  // tokens gathered
  PickQueue pq;
};

// A certified FP32 Gumbel-max over groups of four tokens whose Philox block
// is computed densely: lanes queue the groups that hold candidates (a group
// index and a 4-bit mask), and once 64 groups are queued the wave draws them
// one group per lane: it reads the group's four values again (cache hits),
// computes one Philox call for them, screens each candidate with the cheap
// bound and, if that reaches the bar, computes the accurate noise; then it
// shares its best lower bound as the new bar. Scattered candidates thus cost
// a Philox call per group instead of one per wave step, and the streaming
// loop that finds them stays free of the draw's code. Every lane calls every
// member.
struct DensePick {
  Pick best;
  float bar;
  int n;  // queued (wave-uniform)
  __device__ __forceinline__ void init(float floor) {
    best = pick_none();
    bar = floor - PRUNE_MARGIN;
    n = 0;
  }
  // Queues group g if `cand` (bit j: token 4 g + j) is not empty.
  __device__ __forceinline__ void offer(PickQueue& q, int g, uint32_t cand) {
    const uint64_t has = __ballot(cand != 0);
    if (!has) return;
    const int w = wave_id();
    const int pos = n + __popcll(has & ((1ull << lane_id()) - 1ull));
    if (cand) {
      q.g[w][pos] = g;
      q.live[w][pos] = cand;
    }
    n += __popcll(has);
  }
  // Draws queued groups once 64 are waiting (or all of them with `all`):
  // prep(g, queued, xs) gives the FP32 x of group g's four tokens and returns
  // the tokens to draw, a subset of those queued (it may act on the others).
  template <class Prep>
  __device__ __forceinline__ void drain(PickQueue& q, const RngAddr& rng, uint32_t sub, bool all, Prep&& prep) {
    const int w = wave_id(), lane = lane_id();
    while (n >= WAVE || (all && n > 0)) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      // The last `take` entries, one per lane (the order of draws does not
      // change the pick).
      const int take = min(n, WAVE), from = n - take;
      float xs[4];
      uint32_t live = 0;
      int g = 0;
      if (lane < take) {
        g = q.g[w][from + lane];
        live = prep(g, q.live[w][from + lane], xs);
      }
      if (live) {
        const Words w4 = philox(rng.seed, rng.stream, rng.position, sub, uint32_t(g));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!((live >> j) & 1u)) continue;
          const uint32_t word = w4.w[j];
          const float gb = gumbel_upper(word);
          const float ub2 = xs[j] + gb + SCORE_ERR * (1.f + fabsf(xs[j]) + fabsf(gb));
          if (ub2 < bar) {
            best.others = fmaxf(best.others, ub2);
            continue;
          }
          const float G = gumbel32(word), sc = xs[j] + G, e = SCORE_ERR * (1.f + fabsf(xs[j]) + fabsf(G));
          const int t = 4 * g + j;
          if (sc > best.mid || (sc == best.mid && t < best.id)) {
            best.others = fmaxf(best.others, best.hi);
            best = Pick{sc, sc - e, sc + e, best.others, t};
          } else {
            best.others = fmaxf(best.others, sc + e);
          }
          bar = fmaxf(bar, best.lo - PRUNE_MARGIN);
        }
      }
      // Share the bar; later offers reuse the entries drawn.
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      n = from;
      bar = fmaxf(bar, wave_all(best.lo, [](float u, float v) { return u > v ? u : v; }, -INFINITY) - PRUNE_MARGIN);
    }
  }
};

// Sorts keys[0, n) descending in the block (bitonic, n a power of two >= 64;
// every thread calls it).
template <class K> __device__ __forceinline__ void block_sort_desc(K* keys, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int i = threadIdx.x; i < (n >> 1); i += BLOCK) {
        const int lo = 2 * i - (i & (stride - 1));  // the pair (lo, lo + stride)
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;          // this run sorts descending
        const K x = keys[lo], y = keys[hi];
        if ((x < y) == desc) {
          keys[lo] = y;
          keys[hi] = x;
        }
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Full-row path: one block re-reads the row (and the proposal row) as often as
// it needs. Exact integer cuts, exact (certified or superaccumulated) FP64
// sums, certified FP32 draws with FP64 rescoring.
template <int DT, bool VEC> struct FullRow {
  using W = typename Ty<DT>::W;
  static constexpr int TG = 8;  // groups of four per thread in flight
  const es_arguments& a;
  int64_t row;
  const Params& p;
  Shared<W>& sh;
  RowView<DT, VEC> view, qview;
  int groups;
  Temp<W> tp;
  int fallbacks;

  TopPBins* tb;  // the binned top-p boundary's storage, or null

  __device__ __forceinline__ FullRow(const es_arguments& a_, int64_t row_, const Params& p_, Shared<W>& sh_, int groups_,
                                     TopPBins* tb_ = nullptr)
      : a(a_), row(row_), p(p_), sh(sh_), view(a_.target, row_, int(a_.vocab)), qview(a_.draft, row_, int(a_.vocab)),
        groups(groups_), fallbacks(0), tb(tb_) {}

  // Calls f(t, v, allowed) for every token of the row (or of the proposal row).
  template <bool Q, class F> __device__ __forceinline__ void each(F&& f) const {
    const RowView<DT, VEC>& vw = Q ? qview : view;
    for (int base = threadIdx.x; base < groups; base += BLOCK * TG) {
      W v[TG][4];
      uint32_t bits[TG];
#pragma unroll
      for (int u = 0; u < TG; ++u) {
        const int g = base + u * BLOCK;
        if (g < groups) {
          vw.load(g, v[u]);
          bits[u] = Q ? 0xfu : group_bits(a, row, g);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) v[u][j] = neg_inf<W>();
          bits[u] = 0;
        }
      }
#pragma unroll
      for (int u = 0; u < TG; ++u) {
        const int g = base + u * BLOCK;
        if (g >= groups) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) f(4 * g + j, v[u][j], ((bits[u] >> j) & 1u) != 0);
      }
    }
  }

  __device__ __forceinline__ bool valid_tok(W v, bool ok) const { return ok && v > neg_inf<W>(); }

  // The correctly rounded sum of f(t, v) over tokens (f returns a weight >= 0,
  // or 0 to skip); certified DD first, exact superaccumulator otherwise.
  template <bool Q, class F> __device__ __forceinline__ double exact_sum(F&& f, bool count_fallback) {
    if (count_fallback) ++fallbacks;
    DD acc{0, 0};
    int n = 0;
    each<Q>([&](int t, W v, bool ok) {
      const double w = f(t, v, ok);
      if (w > 0) { acc = dd_add(acc, DD{w, 0}); ++n; }
    });
    acc = block_dd(acc, sh);
    n = block_all(n, [](int x, int y) { return x + y; }, sh.ired, 0);
    double r;
    if (dd_round_certain(acc, dd_sum_error(acc, n), &r)) return r;
    sacc_clear(sh.limbs);
    __syncthreads();
    each<Q>([&](int t, W v, bool ok) {
      const double w = f(t, v, ok);
      if (w > 0) sacc_add(sh.limbs, w);
    });
    __syncthreads();
    if (wave_id() == 0) {  // rounded across wave 0, read by the block
      const double sum = sacc_round_wave(sh.limbs);
      if (lane_id() == 0) sh.dred[0] = sum;
    }
    __syncthreads();
    r = sh.dred[0];
    __syncthreads();
    return r;
  }

  // The n-th (1-based) composite key, in descending order, among tokens where
  // pred(t, v, ok) holds: radix selection over 11-bit digits of the composite.
  template <class Pred> __device__ __forceinline__ u128 select_nth(int n, Pred&& pred) {
    constexpr int NB = CK<W>::BITS;
    constexpr int D = 11;
    u128 prefix = 0;
    int known = 0, need = n;
    while (known < NB) {
      const int width = min(D, NB - known), shift = NB - known - width;
      const int buckets = 1 << width;
      for (int i = threadIdx.x; i < buckets; i += BLOCK) sh.u.hist.cnt[i] = 0;
      __syncthreads();
      each<false>([&](int t, W v, bool ok) {
        if (!pred(t, v, ok)) return;
        const u128 ck = CK<W>::make(v, t);
        if (known && (ck >> (NB - known)) != prefix) return;
        atomicAdd(&sh.u.hist.cnt[int(ck >> shift) & (buckets - 1)], 1u);
      });
      __syncthreads();
      // Descending digits: thread t owns buckets [buckets - 1 - PER t - u].
      const int per = (buckets + BLOCK - 1) / BLOCK;
      int local = 0;
      for (int u = 0; u < per; ++u) {
        const int d = buckets - 1 - (per * threadIdx.x + u);
        if (d >= 0) local += int(sh.u.hist.cnt[d]);
      }
      int total;
      const int incl = block_scan_add(local, sh.ired, &total);
      int run = incl - local;
      for (int u = 0; u < per; ++u) {
        const int d = buckets - 1 - (per * threadIdx.x + u);
        if (d < 0) break;
        const int c = int(sh.u.hist.cnt[d]);
        if (run < need && run + c >= need) { sh.pick = d; sh.n = run; sh.flag = c; }
        run += c;
      }
      __syncthreads();
      const int d = sh.pick, count = sh.flag;
      need -= sh.n;
      __syncthreads();
      prefix = (prefix << width) | u128(d);
      known += width;
      if (count == 1 && known < NB) {  // a unique token: read its whole key
        each<false>([&](int t, W v, bool ok) {
          if (!pred(t, v, ok)) return;
          const u128 ck = CK<W>::make(v, t);
          if ((ck >> (NB - known)) == prefix) sh.ck = ck;
        });
        __syncthreads();
        const u128 r = sh.ck;
        __syncthreads();
        return r;
      }
    }
    return prefix;
  }

  // The first composite key (descending order) among tokens where pred holds at
  // which the correctly rounded running sum of weight(t, v) reaches top_p
  // times the correctly rounded sum of all of them (reference.py:73-83). The
  // first histogram pass, which reads every weight, also sums them: a
  // certified double-double sum, or the exact sum when its rounding is not
  // certain.
  template <class Pred, class Wt>
  __device__ __forceinline__ u128 mass_boundary(double top_p, Pred&& pred, Wt&& weight) {
    constexpr int NB = CK<W>::BITS;
    constexpr int D = 11;
    u128 prefix = 0;
    int known = 0;
    double base_lo = 0, base_hi = 0;  // exact mass before the current region
    double target = 0, below_t = 0;
    while (known < NB) {
      const int width = min(D, NB - known), shift = NB - known - width;
      const int buckets = 1 << width;
      for (int i = threadIdx.x; i < buckets; i += BLOCK) { sh.u.hist.cnt[i] = 0; sh.u.hist.mass[i] = 0; }
      __syncthreads();
      DD acc{0, 0};
      int n_all = 0;
      each<false>([&](int t, W v, bool ok) {
        if (!pred(t, v, ok)) return;
        const u128 ck = CK<W>::make(v, t);
        if (known && (ck >> (NB - known)) != prefix) return;
        const int d = int(ck >> shift) & (buckets - 1);
        const double w = weight(t, v);
        atomicAdd(&sh.u.hist.cnt[d], 1u);
        atomicAdd(&sh.u.hist.mass[d], w);
        if (!known && w > 0) { acc = dd_add(acc, DD{w, 0}); ++n_all; }
      });
      __syncthreads();
      if (!known) {
        acc = block_dd(acc, sh);
        n_all = block_all(n_all, [](int x, int y) { return x + y; }, sh.ired, 0);
        double total;
        if (!dd_round_certain(acc, dd_sum_error(acc, n_all), &total))
          total = exact_sum<false>([&](int t, W v, bool ok) -> double { return pred(t, v, ok) ? weight(t, v) : 0.0; },
                                   false);
        target = top_p * total;
        below_t = nextafter(target, 0.0);
      }
      const int per = (buckets + BLOCK - 1) / BLOCK;
      // Walk buckets in descending order with interval bounds.
      double local = 0, local_err = 0;
      for (int u = 0; u < per; ++u) {
        const int d = buckets - 1 - (per * threadIdx.x + u);
        if (d < 0) break;
        const double m = sh.u.hist.mass[d];
        local += m;
        local_err += double(sh.u.hist.cnt[d]) * 0x1p-52 * m;
      }
      // Exclusive prefix over threads (FP64, fixed order) with a generous bound.
      struct ME { double m, e; };
      const ME sc = wave_scan(ME{local, local_err}, [](ME x, ME y) { return ME{x.m + y.m, x.e + y.e}; }, ME{0, 0});
      const double incl = sc.m, incl_e = sc.e;
      const int lane = lane_id();
      __syncthreads();
      if (lane == WAVE - 1) { sh.dred[wave_id()] = incl; reinterpret_cast<double*>(sh.ddred)[wave_id()] = incl_e; }
      __syncthreads();
      double before_m = 0, before_e = 0;
      for (int w = 0; w < wave_id(); ++w) { before_m += sh.dred[w]; before_e += reinterpret_cast<double*>(sh.ddred)[w]; }
      double run = before_m + incl - local, run_e = before_e + incl_e - local_err;
      int first = INT_MAX, first_sure = INT_MAX;
      for (int u = 0; u < per; ++u) {
        const int d = buckets - 1 - (per * threadIdx.x + u);
        if (d < 0) break;
        const int c = int(sh.u.hist.cnt[d]);
        const double m = sh.u.hist.mass[d];
        run += m;
        run_e += double(c) * 0x1p-52 * m;
        if (c == 0) continue;
        const double slack = run_e + 1e-15 * run + 1e-300;
        const double hi = base_hi + run + slack, lo = base_lo + run - slack;
        const int rank = per * threadIdx.x + u;  // position in descending order
        if (!(hi < below_t)) first = min(first, rank);
        if (lo >= target) first_sure = min(first_sure, rank);
      }
      auto mn = [](int x, int y) { return x < y ? x : y; };
      first = block_all(first, mn, sh.ired, INT_MAX);
      first_sure = block_all(first_sure, mn, sh.ired, INT_MAX);
      if (first == INT_MAX) {
        // Rounding never reaches the target inside this region: take its last token.
        first = first_sure = INT_MAX - 1;
      }
      int chosen = -1;
      int rank = first;
      while (chosen < 0) {
        if (rank == INT_MAX - 1) {  // last nonempty bucket of the region
          int last = -1;
          for (int d = threadIdx.x; d < buckets; d += BLOCK)
            if (sh.u.hist.cnt[d]) last = max(last, buckets - 1 - d);
          last = block_all(last, [](int x, int y) { return x > y ? x : y; }, sh.ired, INT_MIN);
          chosen = last;
          break;
        }
        if (rank == first_sure) { chosen = rank; break; }
        // Not certain: the exact rounded mass through the end of this bucket.
        const int d = buckets - 1 - rank;
        const u128 end_ck = ((prefix << width) | u128(d)) << shift;  // lowest key of bucket d
        const double through = exact_sum<false>([&](int t, W v, bool ok) -> double {
          if (!pred(t, v, ok)) return 0.0;
          return CK<W>::make(v, t) >= end_ck ? weight(t, v) : 0.0;
        }, true);
        if (through >= target) { chosen = rank; break; }
        // Move to the next nonempty bucket.
        int next = INT_MAX;
        for (int dd = threadIdx.x; dd < buckets; dd += BLOCK) {
          const int r = buckets - 1 - dd;
          if (r > rank && sh.u.hist.cnt[dd]) next = min(next, r);
        }
        next = block_all(next, mn, sh.ired, INT_MAX);
        if (next == INT_MAX) { chosen = rank; break; }  // cannot happen: the region reaches the target
        rank = next;
      }
      const int d = buckets - 1 - chosen;
      const int count = int(sh.u.hist.cnt[d]);
      // Mass before bucket d inside the region, with its bound.
      double mb = 0, mbe = 0;
      for (int dd = threadIdx.x; dd < buckets; dd += BLOCK)
        if (dd > d) { mb += sh.u.hist.mass[dd]; mbe += double(sh.u.hist.cnt[dd]) * 0x1p-52 * sh.u.hist.mass[dd]; }
      mb = block_all(mb, [](double x, double y) { return x + y; }, sh.dred, 0.0);
      mbe = block_all(mbe, [](double x, double y) { return x + y; }, sh.dred, 0.0);
      const double slack = mbe + 1e-15 * mb + 1e-300;
      base_lo = base_lo + mb - slack;
      base_hi = base_hi + mb + slack;
      __syncthreads();
      prefix = (prefix << width) | u128(d);
      known += width;
      if (count == 1 && known < NB) {
        each<false>([&](int t, W v, bool ok) {
          if (!pred(t, v, ok)) return;
          const u128 ck = CK<W>::make(v, t);
          if ((ck >> (NB - known)) == prefix) sh.ck = ck;
        });
        __syncthreads();
        const u128 r = sh.ck;
        __syncthreads();
        return r;
      }
    }
    return prefix;
  }

  // ---- The binned top-p boundary ----
  // The top-p cut of a row whose slices binned its kept weights (TP_COARSE
  // bins of a quarter unit of x on the absolute grid y = l * 4 / T, see
  // slice_bins), in one pass over the row shared by the row's `parts`
  // finishing blocks, plus the finisher's own passes when the boundary's bins
  // are dense:
  //  1. each block merges the slices' bins into the row's 64 bins below the
  //     maximum (the same bits in every block); from certified prefix bounds
  //     against top_p times the total they give the bins [b_lo, b_hi] that
  //     may hold the boundary (reference.py:73-83);
  //  2. each block's part of the row: the tokens of [b_lo, b_hi] are gathered
  //     (their IDs into the row's boundary area; a lone block gathers keys)
  //     or, past the area's capacity, the runs holding them are marked; the
  //     certified FP32 Gumbel-max of draw `sub` (draft `excluded` left out)
  //     over the tokens before them, which are certainly kept, is the block's
  //     pick. The last block to arrive finishes: for a dense range it bins the
  //     marked runs 64 times finer and gathers the fine bins that may hold the
  //     boundary, drawing the range's tokens before them;
  //  3. the gathered tokens are sorted (logit desc, ID asc) with their FP64
  //     weights (the oracle's formula); the boundary is the first whose
  //     double-double prefix sum plus the mass before them certainly reaches
  //     the target. The total is refined with the gathered weights' exact
  //     sum; an uncertain boundary with nothing before the gathered tokens is
  //     settled with exact prefix sums.
  // The draw's pick over the gathered part of the nucleus joins the pick of
  // the tokens before it. Returns false, changing nothing the caller relies
  // on, when the bins cannot settle the row (the boundary below the binned
  // range, too many tokens in its bins, an uncertain boundary after the first
  // bin, a grid out of range); the caller then takes mass_boundary.
  struct BinnedCut {
    u128 cut;               // keep composite keys >= cut
    double den_lo, den_hi;  // the nucleus mass (the rounded prefix through the cut) lies in [den_lo, den_hi]
    bool den_exact;         // den_lo == den_hi is the correctly rounded value
    Pick pick;              // certified pick of draw `sub` over the nucleus
  };
  using GKey = typename std::conditional<sizeof(W) == 4, uint64_t, u128>::type;
  static constexpr int GATHER_CAP = tp_gather_cap<W>();
  static constexpr int FINE_PER_COARSE = TP_FINE;
  static_assert(GATHER_CAP * sizeof(GKey) <= sizeof(Shared<W>::u), "gathered keys fit the union");

  __device__ __forceinline__ GKey gkey(W v, int t) const { return GKey(CK<W>::make(v, t)); }
  __device__ __forceinline__ W gvalue(GKey k) const { return CK<W>::value(u128(k)); }
  __device__ __forceinline__ int gid(GKey k) const { return ck_id(u128(k)); }

  // One pass over the row, TG groups of four in flight per thread and one
  // group processed at a time (the loaded groups rotate through a fixed
  // register slot, keeping the loop body to one copy): f(g, x, bits) per
  // group. The dense boundary's passes when no bitmap lists their runs.
  template <class F> __device__ __forceinline__ void each_group(F&& f) const {
    constexpr int TG = 16;
    for (int base0 = 0; base0 < groups; base0 += BLOCK * TG) {
      const int base = base0 + int(threadIdx.x);
      W x[TG][4];
      uint32_t bits[TG];
#pragma unroll
      for (int u = 0; u < TG; ++u) {
        const int g = base + u * BLOCK;
        if (g < groups) {
          view.load(g, x[u]);
          bits[u] = group_bits(a, row, g);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) x[u][j] = neg_inf<W>();
          bits[u] = 0;
        }
      }
#pragma unroll 1
      for (int u = 0; u < TG; ++u) {
        f(base + u * BLOCK, x[0], bits[0]);
#pragma unroll
        for (int q = 0; q + 1 < TG; ++q) {
#pragma unroll
          for (int j = 0; j < 4; ++j) x[q][j] = x[q + 1][j];
          bits[q] = bits[q + 1];
        }
      }
    }
  }

  // One pass over the groups group_at(i), i in [i_begin, i_end), PQ_ROUND
  // groups in flight per thread: a group holding a valid token with lowest
  // <= x32 <= highest is queued on dp (those tokens' bits), and
  // classify(g, queued, xs) settles the queued tokens as dp draws them (see
  // DensePick::drain). Every thread calls it.
  struct SameGroup {
    __device__ __forceinline__ int operator()(int i) const { return i; }
  };
  template <class C, class At = SameGroup>
  __device__ __forceinline__ void queue_pass(int i_begin, int i_end, float lowest, DensePick& dp, uint32_t sub,
                                             C&& classify, float highest = INFINITY, At group_at = At{}) {
    PickQueue& q = tb->pq;
    for (int base0 = i_begin; base0 < i_end; base0 += BLOCK * PQ_ROUND) {  // a uniform trip count: dp's queue is per wave
      const int base = base0 + int(threadIdx.x);
      W x[PQ_ROUND][4];
      uint32_t bits[PQ_ROUND];
      int gs[PQ_ROUND];
#pragma unroll
      for (int u = 0; u < PQ_ROUND; ++u) {
        const int i = base + u * BLOCK;
        const int g = group_at(min(i, i_end - 1));
        gs[u] = g;
        view.load(min(g, groups - 1), x[u]);
        bits[u] = i < i_end && g < groups ? group_bits(a, row, g) : 0u;
      }
#pragma unroll
      for (int u = 0; u < PQ_ROUND; ++u) {
        uint32_t queued = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const W v = x[u][j];
          const float xv = tp.x32(v);
          if (((bits[u] >> j) & 1u) && v > neg_inf<W>() && xv >= lowest && xv <= highest) queued |= 1u << j;
        }
        dp.offer(q, gs[u], queued);
      }
      dp.drain(q, p.rng, sub, false, classify);
    }
    dp.drain(q, p.rng, sub, true, classify);
  }

  // The runs of TP_RUN tokens marked in `bitmap` (words [0, nwords)), listed
  // in LDS (the upper part of the bins' mass array, free in the dense
  // passes): returns their number, or -1 when more than TP_RUN_LIST are
  // marked (nothing listed). Every thread calls it.
  static constexpr int TP_RUN_LIST = TP_GATHER_MAX * 2 - TP_BINS * 2;  // 32-bit entries past the fine bins
  __device__ __forceinline__ uint32_t* run_list() const { return reinterpret_cast<uint32_t*>(tb->mass + TP_BINS); }
  __device__ __forceinline__ int list_runs(const uint32_t* bitmap, int nwords) {
    const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
    const int per = (nwords + BLOCK - 1) / BLOCK;  // words per thread, consecutive
    const int w_begin = min(nwords, tid * per), w_end = min(nwords, w_begin + per);
    int cnt = 0;
    for (int w = w_begin; w < w_end; ++w) cnt += int(__popc(bitmap[w]));
    const int incl = wave_scan(cnt, [](int x, int y) { return x + y; }, 0);
    __syncthreads();
    if (lane == WAVE - 1) sh.ired[wid] = incl;
    __syncthreads();
    int idx = incl - cnt, total = 0;
    for (int w = 0; w < WAVES; ++w) {
      if (w < wid) idx += sh.ired[w];
      total += sh.ired[w];
    }
    __syncthreads();
    if (total > TP_RUN_LIST) return -1;
    uint32_t* list = run_list();
    for (int w = w_begin; w < w_end; ++w) {
      for (uint32_t wd = bitmap[w]; wd; wd &= wd - 1) list[idx++] = uint32_t(32 * w + __ffs(wd) - 1);
    }
    __syncthreads();
    return total;
  }
  // f(g, x, bits) on every group of the n listed runs, as loaded, four runs
  // in flight per thread. No barrier inside.
  template <class F> __device__ __forceinline__ void listed_pass(int n, F&& f) {
    const uint32_t* list = run_list();
    constexpr int GPR = TP_RUN / 4;  // groups per run
    constexpr int RPT = 4;           // runs per thread per round
    for (int r0 = int(threadIdx.x); r0 < n; r0 += BLOCK * RPT) {
      W x[RPT * GPR][4];
      uint32_t bits[RPT * GPR];
      int gs[RPT * GPR];
#pragma unroll
      for (int u = 0; u < RPT; ++u) {
        const int li = r0 + u * BLOCK;
        const int run = li < n ? int(list[li]) : -1;
#pragma unroll
        for (int h = 0; h < GPR; ++h) {
          const int g = run * GPR + h, i = u * GPR + h;
          gs[i] = run >= 0 && g < groups ? g : -1;
          view.load(gs[i] >= 0 ? g : 0, x[i]);
          bits[i] = gs[i] >= 0 ? group_bits(a, row, g) : 0u;
        }
      }
#pragma unroll 1
      for (int i = 0; i < RPT * GPR; ++i) {
        if (gs[i] >= 0) f(gs[i], x[i], bits[i]);
      }
    }
  }

  int bin_slices = 0;  // > 0: the row's slices binned its kept weights
  // This block's share of a binned top-p row's boundary pass: groups
  // [part gps, (part + 1) gps) of the row's `parts` finishing blocks
  // (parts > 1), or the whole row (parts 1).
  int part = 0, parts = 1, gps = 0;
  // Whether this block finishes the row: after a shared pass the last block
  // to arrive; when the pass is not shared, the row's first block alone.
  bool finisher = true;

  __device__ __forceinline__ bool topp_binned(uint32_t sub, int excluded, int floor_id, BinnedCut* out) {
    // Before the arrival every finishing block of the row takes the same
    // decisions from the same data: when the pass is not shared (or cannot
    // settle the row) the first block goes on alone and the others leave.
    auto bail = [&]() {
      finisher = part == 0;
      return false;
    };
    if (!bin_slices || !tb || tp.slow) return bail();
    TopPBins& b = *tb;
    const int tid = threadIdx.x, lane = lane_id(), wid = wave_id();
    const double inv_t = 1.0 / p.temperature, inv4 = TP_Y_PER_X / p.temperature;
    const double M = tp.M, yM = M * inv4;
    if (!(fabs(yM) < 0x1p50)) return bail();
    const double top = floor(yM), dM = top - yM;  // dM in (-1, 0]
    // A mass's relative error besides its adds: the polynomial, y's formation
    // (|y| 2^-53 per token and for dM) and the FP64 exp of the bin factor.
    const double rel = 1e-14 + fabs(yM) * 0x1p-50;
    auto coarse_of = [&](W v) -> double { return top - floor(double(v) * inv4); };
    // The x of the lower edge of row bin k (bin top - k holds y in [top - k, top - k + 1)).
    auto coarse_edge = [&](double k) -> float { return float((dM - k) * (1.0 / TP_Y_PER_X)); };
    // ---- 1. The row's bins: one wave merges the slices' bins in slice order
    // after loading them all, so every finishing block gets the same bits;
    // lane k holds row bin k. The bins past the row's TP_COARSE and the
    // slices' FP32 far parts make the far mass. From certified prefix bounds
    // against top_p times the total: the bins [b_lo, b_hi] that may hold the
    // boundary (reference.py:73-83) and the mass before and outside them. ----
    if (tid == 0) b.n = 0;
    if (wid == 0) {
      double fr = -INFINITY, tau = 0, psum = 0, perr = 0;
      if (lane < bin_slices) {
        const SlicePart q = slice_parts(a, row)[lane];
        fr = q.frontier; tau = q.tau; psum = q.sum; perr = q.err;
      }
      double ms[TP_SLICES_MAX];
      unsigned cs[TP_SLICES_MAX];
#pragma unroll
      for (int sl = 0; sl < TP_SLICES_MAX; ++sl) {
        ms[sl] = 0;
        cs[sl] = 0;
        if (sl < bin_slices) {
          ms[sl] = slice_bin_mass(a, row, sl)[lane];
          cs[sl] = slice_bin_count(a, row, sl)[lane];
        }
      }
      double m = 0, fp = 0, fpe = 0;  // row bin `lane`; mass past the row's bins and its bound
      unsigned c = 0;
      bool off_grid = false;
#pragma unroll
      for (int sl = 0; sl < TP_SLICES_MAX; ++sl) {
        const double d = sl < bin_slices ? top - lane_read(fr, sl) : double(TP_COARSE);  // slice bin j is row bin j + d
        off_grid |= !(d >= 0);
        const double k = double(lane) + d;
        if (sl < bin_slices && !(k < double(TP_COARSE)) && cs[sl]) {
          const double f = exp((dM + 0.5 - k) * (1.0 / TP_Y_PER_X)) * ms[sl];
          fp += f;
          fpe += f * (rel + double(cs[sl]) * 0x1p-52);
        }
        const int src = d < double(TP_COARSE) && d >= 0 ? lane - int(d) : -1;
        const double mv = __shfl(ms[sl], src < 0 ? 0 : src);
        const unsigned cv = __shfl(cs[sl], src < 0 ? 0 : src);
        if (src >= 0) {
          m += mv;
          c += cv;
        }
      }
      if (lane < bin_slices) {  // the slices' FP32 far parts, from their reference maximum to the row's
        const double sh_x = (tau - M) * inv_t;
        const double sc = exp(sh_x);
        fp += psum * sc;
        fpe += (perr + 1e-15 * psum) * sc * (1 + 1e-13) + psum * sc * (fabs(sh_x) * 0x1p-50 + 1e-15);
      }
      const double fp_all = wave_all(fp, [](double x, double y) { return x + y; }, 0.0);
      const double fpe_all = wave_all(fpe, [](double x, double y) { return x + y; }, 0.0) + 0x1p-44 * fp_all;
      const double mm = exp((dM + 0.5 - double(lane)) * (1.0 / TP_Y_PER_X)) * m;
      const double e = mm * (rel + double(c) * 0x1p-52);
      struct ME { double m, e; };
      auto add = [](ME x, ME y) { return ME{x.m + y.m, x.e + y.e}; };
      const ME inc = wave_scan(ME{mm, e}, add, ME{0, 0});
      const ME tot = lane_read(inc, WAVE - 1);
      const double slack = inc.e + 0x1p-44 * inc.m, tslack = tot.e + 0x1p-44 * tot.m;
      const double s_lo = tot.m - tslack + fp_all - fpe_all, s_hi = tot.m + tslack + fp_all + fpe_all;
      const double lo_t = p.top_p * s_lo * (1 - 0x1p-50), hi_t = p.top_p * s_hi * (1 + 0x1p-50);
      const uint64_t may = __ballot(inc.m + slack >= lo_t * (1 - 0x1p-50));
      const uint64_t sure = __ballot(inc.m - slack >= hi_t);
      const int b_lo = may ? __ffsll((unsigned long long)may) - 1 : TP_COARSE;
      const int b_hi = sure ? __ffsll((unsigned long long)sure) - 1 : TP_COARSE;
      const int count = wave_all(lane >= b_lo && lane <= b_hi ? int(c) : 0, [](int x, int y) { return x + y; }, 0);
      const ME before = wave_all(lane < b_lo ? ME{mm, e} : ME{0, 0}, add, ME{0, 0});
      const ME after = wave_all(lane > b_hi ? ME{mm, e} : ME{0, 0}, add, ME{0, 0});
      const bool bad_grid = __ballot(off_grid) != 0;
      if (lane == 0) {
        b.scal[0] = b_lo; b.scal[1] = b_hi; b.scal[2] = count;
        b.scal[3] = lo_t; b.scal[4] = hi_t;
        const double be = before.e + 0x1p-44 * before.m, ae = after.e + 0x1p-44 * after.m;
        b.scal[5] = fmax(before.m - be, 0.0); b.scal[6] = before.m + be;
        // Everything outside [b_lo, b_hi]: the bins before and after, and the far tail.
        b.scal[7] = fmax(before.m - be + after.m - ae + fp_all - fpe_all, 0.0);
        b.scal[8] = before.m + be + after.m + ae + fp_all + fpe_all;
        b.scal[9] = bad_grid;
      }
    }
    __syncthreads();
    const int b_lo = int(b.scal[0]), b_hi = int(b.scal[1]), count = int(b.scal[2]);
    double lo_t = b.scal[3], hi_t = b.scal[4];
    double eb_lo = b.scal[5], eb_hi = b.scal[6];
    const double rest_lo = b.scal[7], rest_hi = b.scal[8];
    const bool bad_grid = b.scal[9] != 0;
    __syncthreads();
    // The boundary may lie in the far tail (or a slice's grid is off the row's).
    if (bad_grid || b_hi >= TP_COARSE || b_lo > b_hi || count == 0) return bail();
    // ---- 2. This block's share of the pass: the tokens of [b_lo, b_hi]
    // gathered (unless more than the list holds: dense), and the pick over
    // the tokens before them. A shared pass gathers token IDs into the row's
    // boundary area; a lone block gathers keys into its list. ----
    GKey* keys = reinterpret_cast<GKey*>(&sh.u);
    double* wts = b.mass;  // the gathered weights, once the fine bins are done with
    const bool shared_pass = parts > 1;
    const int gcap = shared_pass ? min(GATHER_CAP, bound_capacity(bin_slices)) : GATHER_CAP;
    const bool dense = count > gcap;
    const float edge_before = coarse_edge(double(b_lo) - 1.0);  // x at or above it: coarse bin < b_lo
    const float edge_range = coarse_edge(double(b_hi));          // x below it: coarse bin > b_hi
    constexpr float SCREEN = 1e-5f;  // above x32's error for |x| <= 17
    float floor_score = -INFINITY;
    if (floor_id >= 0 && floor_id != excluded && b_lo > 0) {
      const W v = view.value(floor_id);
      const float x = tp.x32(v);
      if (tp.kept(v, x) && coarse_of(v) < double(b_lo)) {
        const float g = gumbel32(word_of(p.rng, sub, uint32_t(floor_id)));
        floor_score = x + g - SCORE_ERR * (1.f + fabs(x) + fabsf(g));
      }
    }
    DensePick dp;
    dp.init(floor_score);
    uint32_t* const gcount = bound_count(a, row, bin_slices);  // the area's layout follows the slices
    uint32_t* const gids = bound_ids(a, row, bin_slices);
    // A dense range is binned 64 times finer (y * 64 on the same grid: fine
    // bin f of coarse bin k is 64 k + (63 - (floor(64 y) - 64 floor(y)))):
    // by a lone block in the same pass; by a shared pass's blocks, when the
    // range is at most TP_FINE_SHARED fine bins; else after a shared pass by
    // the finisher, which visits only the runs of TP_RUN tokens the pass
    // marked in the boundary area's bitmap (when it fits), else the whole row.
    const double fine_top = (top + 1) * FINE_PER_COARSE - 1;  // fine index of a token: fine_top - floor(y * 64)
    const double fine_base = double(b_lo) * FINE_PER_COARSE;
    const int nfine = (b_hi - b_lo + 1) * FINE_PER_COARSE;
    if (dense && nfine > TP_BINS) return bail();
    const int bitmap_words = int(min<int64_t>(bound_bitmap_words(a.vocab), INT_MAX));
    const bool marks = dense && shared_pass && bitmap_words <= bound_capacity(bin_slices);
    const bool fine_local = dense && !shared_pass;
    // A shared pass over a narrow dense range also bins it finer: each block
    // its share in LDS, added to the row's fine bins before the arrival.
    const bool fine_shared = marks && nfine <= TP_FINE_SHARED && bound_fine_fits(bin_slices, a.vocab);
    if (fine_local || fine_shared) {
      for (int i = tid; i < nfine; i += BLOCK) { b.mass[i] = 0; b.cnt[i] = 0; }
      __syncthreads();
    }
    auto fine_of = [&](W v) { return fine_top - floor(double(v) * inv4 * FINE_PER_COARSE); };
    auto add_fine = [&](W v) {
      const double fy = double(v) * inv4 * FINE_PER_COARSE, fb = floor(fy);
      const int i = int(fine_top - fb - fine_base);  // in [0, nfine): the fine grid nests in the coarse one
      if (i < 0 || i >= nfine) return;
      atomicAdd(&b.mass[i], exp_near_zero((fy - fb - 0.5) * (1.0 / (TP_Y_PER_X * FINE_PER_COARSE))));
      atomicAdd(&b.cnt[i], 1u);
    };
    // A queued group's tokens: the ones before the range drawn (the draft
    // left out); the ones in it gathered, or for a dense range marked or
    // binned finer.
    auto classify = [&](int g, uint32_t queued, float (&xs)[4]) -> uint32_t {
      W v[4];
      view.load(g, v);
      uint32_t draw = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xs[j] = tp.x32(v[j]);
        if (!((queued >> j) & 1u) || !tp.kept(v[j], xs[j])) continue;
        const int t = 4 * g + j;
        bool before = xs[j] > edge_before + SCREEN;
        if (!before) {
          const double k = coarse_of(v[j]);
          before = k < double(b_lo);
          if (!before && k <= double(b_hi)) {
            if (!dense) {
              if (shared_pass) {
                const uint32_t slot = atomicAdd(gcount, 1u);
                if (slot < uint32_t(gcap)) gids[slot] = uint32_t(t);
              } else {
                const int slot = atomicAdd(&b.n, 1);
                if (slot < GATHER_CAP) keys[slot] = gkey(v[j], t);
              }
            } else {
              if (marks) {
                const int run = t / TP_RUN;
                atomicOr(&gids[run >> 5], 1u << (run & 31));
              }
              if (fine_local || fine_shared) add_fine(v[j]);
            }
          }
        }
        if (before && t != excluded) draw |= 1u << j;
      }
      return draw;
    };
    {
      const int g_begin = shared_pass ? part * gps : 0;
      const int g_end = shared_pass ? min(g_begin + gps, groups) : groups;
      // Tokens below `lowest` are neither before the range nor to be gathered, marked or binned.
      const float lowest = (dense && !marks && !fine_local ? edge_before : edge_range) - SCREEN;
      queue_pass(g_begin, g_end, lowest, dp, sub, classify);
    }
    Pick best = dp.best;
    if (fine_shared) {
      __syncthreads();
      double* const fm = bound_fine_mass(a, row, bin_slices);
      uint32_t* const fc = bound_fine_count(a, row, bin_slices);
      for (int i = tid; i < nfine; i += BLOCK) {
        if (b.cnt[i]) {
          atomicAdd(&fm[i], b.mass[i]);
          atomicAdd(&fc[i], b.cnt[i]);
        }
      }
    }
    if (shared_pass) {
      const Pick mine = block_pick(best, sh);
      if (tid == 0) {
        uint32_t* rec = bound_picks(a, row, bin_slices) + part * int(TP_PICK_BYTES / 4);
        rec[0] = __float_as_uint(mine.mid); rec[1] = __float_as_uint(mine.lo); rec[2] = __float_as_uint(mine.hi);
        rec[3] = __float_as_uint(mine.others); rec[4] = uint32_t(mine.id);
      }
      if (!arrive(&counters(a, row)->bound, uint32_t(parts), &sh.flag)) {
        finisher = false;
        return false;
      }
      finisher = true;
      // The last block: every block's pick, joined; one thread carries it on.
      Pick theirs = pick_none();
      if (tid < parts) {
        const uint32_t* rec = bound_picks(a, row, bin_slices) + tid * int(TP_PICK_BYTES / 4);
        theirs = Pick{__uint_as_float(rec[0]), __uint_as_float(rec[1]), __uint_as_float(rec[2]),
                      __uint_as_float(rec[3]), int(rec[4])};
      }
      const Pick all = block_pick(theirs, sh);
      best = tid == 0 ? all : pick_none();
      dp.best = best;
      dp.bar = fmaxf(dp.bar, all.lo - PRUNE_MARGIN);
      if (!dense) {
        const int n = int(__hip_atomic_load(gcount, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (n != count || n > gcap) return false;
        for (int i = tid; i < n; i += BLOCK) {
          const int t = int(gids[i]);
          keys[i] = gkey(view.value(t), t);
        }
        if (tid == 0) b.n = n;
      }
    }
    __syncthreads();
    if (dense) {
      // Only the coarse range's tokens matter from here on.
      auto in_coarse = [&](W v, float x, double* k) {
        if (x > edge_before + SCREEN || !tp.kept(v, x)) return false;
        *k = coarse_of(v);
        return *k >= double(b_lo) && *k <= double(b_hi);
      };
      // The tokens of a group that may lie in the coarse range, by an FP32
      // screen (most of a marked run does not): the FP64 tests then run only
      // for these, one at a time per lane.
      auto screened = [&](const W (&x)[4], uint32_t bits) {
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xs = tp.x32(x[j]);
          if (((bits >> j) & 1u) && x[j] > neg_inf<W>() && xs >= edge_range - SCREEN && xs <= edge_before + SCREEN)
            m |= 1u << j;
        }
        return m;
      };
      auto pick_of = [](const W (&x)[4], int j) { return j == 0 ? x[0] : j == 1 ? x[1] : j == 2 ? x[2] : x[3]; };
      // The marked runs, listed once for both passes (-1: the whole row).
      const int listed = marks ? list_runs(gids, bitmap_words) : -1;
      if (fine_shared) {
        // Every block's share, summed before the arrival.
        const double* const fm = bound_fine_mass(a, row, bin_slices);
        const uint32_t* const fc = bound_fine_count(a, row, bin_slices);
        for (int i = tid; i < nfine; i += BLOCK) { b.mass[i] = fm[i]; b.cnt[i] = fc[i]; }
        __syncthreads();
      } else if (!fine_local) {
        // The finisher bins the coarse range finer: only the marked runs, or
        // the whole row when the bitmap did not fit or marks too many.
        for (int i = tid; i < nfine; i += BLOCK) { b.mass[i] = 0; b.cnt[i] = 0; }
        __syncthreads();
        auto bin_group = [&](int, const W (&x)[4], uint32_t bits) {
          for (uint32_t m = screened(x, bits); m; m &= m - 1) {
            const W v = pick_of(x, __ffs(m) - 1);
            double k;
            if (in_coarse(v, tp.x32(v), &k)) add_fine(v);
          }
        };
        if (listed >= 0) listed_pass(listed, bin_group);
        else each_group(bin_group);
        __syncthreads();
      }
      // The fine prefix, after the mass before the coarse range, in thread order.
      const double base = fine_base;
      int f_lo, f_hi;
      const double fdM = (dM + 1.0) * (1.0 / TP_Y_PER_X);
      double fm = 0, fe = 0;
      constexpr int PF = TP_BINS / BLOCK;
      double mm[PF], ee[PF];
#pragma unroll
      for (int q = 0; q < PF; ++q) {
        const int i = PF * tid + q;
        mm[q] = 0; ee[q] = 0;
        if (i < nfine) {
          const double fidx = base + double(i);
          mm[q] = exp(fdM - (fidx + 0.5) * (1.0 / (TP_Y_PER_X * FINE_PER_COARSE))) * b.mass[i];
          ee[q] = mm[q] * (rel + double(b.cnt[i]) * 0x1p-52);
        }
        fm += mm[q]; fe += ee[q];
      }
      struct ME { double m, e; };
      const ME inc = wave_scan(ME{fm, fe}, [](ME x, ME y) { return ME{x.m + y.m, x.e + y.e}; }, ME{0, 0});
      __syncthreads();
      if (lane == WAVE - 1) { b.scal[8 + wid] = inc.m; b.scal[12 + wid] = inc.e; }
      __syncthreads();
      double rm = (eb_lo + eb_hi) * 0.5, re = (eb_hi - eb_lo) * 0.5;
      for (int w = 0; w < wid; ++w) { rm += b.scal[8 + w]; re += b.scal[12 + w]; }
      rm += inc.m - fm;
      re += inc.e - fe;
      int flo = INT_MAX, fhi = INT_MAX, fcount = 0;
      double feb_lo = 0, feb_hi = 0;
      bool have_before = false;
#pragma unroll
      for (int q = 0; q < PF; ++q) {
        const int i = PF * tid + q;
        rm += mm[q]; re += ee[q];
        if (i >= nfine) continue;
        const double sl = re + 0x1p-44 * rm;
        if (rm + sl >= lo_t * (1 - 0x1p-50)) flo = min(flo, i);
        if (rm - sl >= hi_t) fhi = min(fhi, i);
      }
      auto mn = [](int x, int y) { return x < y ? x : y; };
      f_lo = block_all(flo, mn, sh.ired, INT_MAX);
      f_hi = block_all(fhi, mn, sh.ired, INT_MAX);
      if (f_hi == INT_MAX || f_lo > f_hi) return false;
      // The mass before fine bin f_lo and the count of [f_lo, f_hi].
      rm = (eb_lo + eb_hi) * 0.5; re = (eb_hi - eb_lo) * 0.5;
      for (int w = 0; w < wid; ++w) { rm += b.scal[8 + w]; re += b.scal[12 + w]; }
      rm += inc.m - fm;
      re += inc.e - fe;
#pragma unroll
      for (int q = 0; q < PF; ++q) {
        const int i = PF * tid + q;
        if (i == f_lo) { const double sl = re + 0x1p-44 * rm; feb_lo = rm - sl; feb_hi = rm + sl; have_before = true; }
        rm += mm[q]; re += ee[q];
        if (i >= f_lo && i <= f_hi && i < nfine) fcount += int(b.cnt[i]);
      }
      __syncthreads();
      if (have_before) { b.scal[5] = fmax(feb_lo, 0.0); b.scal[6] = feb_hi; }
      fcount = block_all(fcount, [](int x, int y) { return x + y; }, sh.ired, 0);
      eb_lo = b.scal[5];
      eb_hi = b.scal[6];
      __syncthreads();
      if (fcount == 0 || fcount > GATHER_CAP) return false;
      f_lo += int(base);  // absolute fine indices from here on
      f_hi += int(base);
      // The second dense pass, by this block alone, over the listed runs'
      // groups or the whole row: the tokens of fine bins [f_lo, f_hi]
      // gathered, the coarse range's tokens before f_lo drawn (the tokens
      // before the coarse range were drawn in the first pass), queued and
      // drawn densely as in the shared pass.
      {
        auto settle_queued = [&](int g, uint32_t queued, float (&xs)[4]) -> uint32_t {
          W v[4];
          view.load(g, v);
          uint32_t draw = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            xs[j] = tp.x32(v[j]);
            double k;
            if (!((queued >> j) & 1u) || !in_coarse(v[j], xs[j], &k)) continue;
            const double f = fine_of(v[j]);
            const int t = 4 * g + j;
            if (f < double(f_lo)) {
              if (t != excluded) draw |= 1u << j;
            } else if (f <= double(f_hi)) {
              const int slot = atomicAdd(&b.n, 1);
              if (slot < GATHER_CAP) keys[slot] = gkey(v[j], t);
            }
          }
          return draw;
        };
        if (listed >= 0) {
          const uint32_t* list = run_list();
          constexpr int GPR = TP_RUN / 4;  // groups per run
          auto listed_group = [list](int i) { return int(list[i / GPR]) * GPR + i % GPR; };
          queue_pass(0, listed * GPR, edge_range - SCREEN, dp, sub, settle_queued, edge_before + SCREEN, listed_group);
        } else {
          queue_pass(0, groups, edge_range - SCREEN, dp, sub, settle_queued, edge_before + SCREEN);
        }
      }
      best = dp.best;
    }
    __syncthreads();
    const int n = b.n;
    if (n == 0 || n > GATHER_CAP) return false;
    // ---- 3. The boundary among the gathered tokens. ----
    int n_pad = 64;
    while (n_pad < n) n_pad <<= 1;
    for (int i = n + tid; i < n_pad; i += BLOCK) keys[i] = GKey(0);
    block_sort_desc(keys, n_pad);
    for (int i = tid; i < n; i += BLOCK) wts[i] = exp(tp.x64(gvalue(keys[i])));
    __syncthreads();
    // Thread t owns sorted entries [per t, per t + per): inclusive
    // double-double prefix sums of the FP64 weights, in order. A pass finds
    // the first entry whose prefix (plus the mass before, in [elo, ehi])
    // certainly reaches the target interval [tlo, thi] and the first that
    // may, and records entry `want`'s prefix bounds in sh.sp_lo / sh.sp_hi;
    // the whole sum and its bound go to sh.sp_mid / sh.sp_others.
    const int per = (n_pad + BLOCK - 1) / BLOCK;
    auto mn = [](int x, int y) { return x < y ? x : y; };
    auto prefix_pass = [&](double tlo, double thi, double elo, double ehi, int want, int* first_yes,
                           int* first_unsure) {
      DD local{0, 0};
      for (int u = 0; u < per; ++u) {
        const int i = per * tid + u;
        if (i < n) local = dd_add(local, DD{wts[i], 0});
      }
      const DD inc = wave_scan(local, [](DD x, DD y) { return dd_add(x, y); }, DD{0, 0});
      __syncthreads();
      if (lane == WAVE - 1) sh.ddred[wid] = inc;
      __syncthreads();
      DD run{0, 0};
      for (int w = 0; w < wid; ++w) run = dd_add(run, sh.ddred[w]);
      run = dd_add(run, dd_add(inc, DD{-local.hi, -local.lo}));
      int fy = INT_MAX, fu = INT_MAX;
      for (int u = 0; u < per; ++u) {
        const int i = per * tid + u;
        if (i >= n) break;
        run = dd_add(run, DD{wts[i], 0});
        const double err = dd_sum_error(run, i + 1) + 4 * 0x1p-104 * run.hi;
        const int yes = dd_reaches(dd_add(run, DD{elo, 0}), err, thi);
        const int no = dd_reaches(dd_add(run, DD{ehi, 0}), err, tlo);
        if (yes == 1) fy = min(fy, i);
        else if (no != 0) fu = min(fu, i);
        if (i == want) {
          sh.sp_lo = (run.hi + elo + run.lo - err) * (1 - 0x1p-50);
          sh.sp_hi = (run.hi + ehi + run.lo + err) * (1 + 0x1p-50);
        }
        if (i == n - 1) {
          sh.sp_mid = run.hi + run.lo;
          sh.sp_others = err + 0x1p-100 * run.hi;
        }
      }
      *first_yes = block_all(fy, mn, sh.ired, INT_MAX);
      *first_unsure = block_all(fu, mn, sh.ired, INT_MAX);
    };
    int first_yes, first_unsure;
    prefix_pass(lo_t, hi_t, eb_lo, eb_hi, -1, &first_yes, &first_unsure);
    // The total refined: the gathered weights' sum (near exact) and the
    // bounded mass outside the coarse range. When the total's rounding is then
    // certain (both bounds strictly inside one double's rounding interval,
    // tested with exact differences) the target is exact: the oracle's
    // top_p * fsum(kept).
    if (!dense) {
      const double lo = (sh.sp_mid - sh.sp_others + rest_lo) * (1 - 0x1p-51);
      const double hi = (sh.sp_mid + sh.sp_others + rest_hi) * (1 + 0x1p-51);
      __syncthreads();
      if (lo > 0 && lo <= hi) {
        const double d = 0.5 * lo + 0.5 * hi;
        const double down = d - nextafter(d, 0.0), up = nextafter(d, INFINITY) - d;
        if (lo - d > -0.5 * down && hi - d < 0.5 * up) {
          lo_t = hi_t = p.top_p * d;
        } else {
          lo_t = fmax(lo_t, p.top_p * lo * (1 - 0x1p-50));
          hi_t = fmin(hi_t, p.top_p * hi * (1 + 0x1p-50));
        }
      }
    }
    prefix_pass(lo_t, hi_t, eb_lo, eb_hi, -1, &first_yes, &first_unsure);
    // The correctly rounded sum of the first m gathered weights (LDS superaccumulator).
    auto rounded_prefix = [&](int m) {
      sacc_clear(sh.limbs);
      __syncthreads();
      for (int i = tid; i < m; i += BLOCK) sacc_add(sh.limbs, wts[i]);
      __syncthreads();
      if (wid == 0) {
        const double r = sacc_round_wave(sh.limbs);
        if (lane == 0) sh.dred[0] = r;
      }
      __syncthreads();
      const double r = sh.dred[0];
      __syncthreads();
      return r;
    };
    int cut_i;
    bool den_exact = false;
    double den = 0;
    if (first_unsure < first_yes) {
      // Settled exactly only when nothing precedes the gathered tokens: the
      // correctly rounded total gives the target, and exact prefix sums of
      // the gathered weights decide the uncertain entries in order.
      if (b_lo != 0 || dense) return false;
      double target;
      if (lo_t == hi_t) {
        target = lo_t;
      } else {
        ++fallbacks;
        const double total = exact_sum<false>([&](int, W v, bool ok) -> double {
          return valid_tok(v, ok) && tp.kept(v, tp.x32(v)) ? exp(tp.x64(v)) : 0.0;
        }, false);
        target = p.top_p * total;
        prefix_pass(target, target, 0.0, 0.0, -1, &first_yes, &first_unsure);
      }
      cut_i = first_yes;
      for (int i = first_unsure; i < first_yes; ++i) {
        const double r = rounded_prefix(i + 1);
        if (r >= target) { cut_i = i; den = r; den_exact = true; break; }
      }
      if (cut_i == INT_MAX) return false;
      if (!den_exact) { den = rounded_prefix(cut_i + 1); den_exact = true; }
    } else {
      if (first_yes == INT_MAX) return false;
      cut_i = first_yes;
    }
    // The nucleus mass: the prefix through the cut, with its bounds.
    if (!den_exact) prefix_pass(lo_t, hi_t, eb_lo, eb_hi, cut_i, &first_yes, &first_unsure);
    __syncthreads();
    out->cut = u128(keys[cut_i]);
    out->den_exact = den_exact;
    out->den_lo = den_exact ? den : sh.sp_lo;
    out->den_hi = den_exact ? den : sh.sp_hi;
    // The pick over the gathered part of the nucleus, joined with the pick before it.
    for (int i = tid; i <= cut_i; i += BLOCK) {
      const W v = gvalue(keys[i]);
      const int t = gid(keys[i]);
      if (t == excluded) continue;
      const float x = tp.x32(v), g = gumbel32(word_of(p.rng, sub, uint32_t(t))), sc = x + g;
      const float e = SCORE_ERR * (1.f + fabsf(x) + fabsf(g));
      best = pick_join(best, Pick{sc, sc - e, sc + e, -INFINITY, t});
    }
    out->pick = block_pick(best, sh);
    return true;
  }

  // Certified FP32 draw over tokens where in(t, v, ok) holds (excluded
  // removed), FP64 rescoring when the certificate fails. floor_id is a token
  // certainly in the set (or -1).
  template <class In> __device__ __forceinline__ int draw(int sub, int excluded, int floor_id, In&& in) {
    if (threadIdx.x == 0) {
      float floor = -INFINITY;
      if (floor_id >= 0) {
        const W v = view.value(floor_id);
        const float x = tp.x32(v);
        const float g = gumbel32(word_of(p.rng, uint32_t(sub), uint32_t(floor_id)));
        floor = x + g - SCORE_ERR * (1.f + fabsf(x) + fabsf(g));
      }
      sh.fred[0] = floor;
    }
    __syncthreads();
    const float floor = sh.fred[0];
    __syncthreads();
    float best_mid = -INFINITY, best_lo = -INFINITY, best_hi = -INFINITY, others = -INFINITY;
    int best_id = INT_MAX;
    float bar = floor - PRUNE_MARGIN;
    each<false>([&](int t, W v, bool ok) {
      if (t == excluded || !in(t, v, ok)) return;
      const float x = tp.x32(v);
      const float ub = x + GUMBEL_MAX + SCORE_ERR * (1.f + fabsf(x) + GUMBEL_MAX);
      if (ub < bar) { others = fmaxf(others, ub); return; }
      const uint32_t w = word_of(p.rng, uint32_t(sub), uint32_t(t));
      const float gb = gumbel_upper(w);
      const float ub2 = x + gb + SCORE_ERR * (1.f + fabsf(x) + fabsf(gb));
      if (ub2 < bar) { others = fmaxf(others, ub2); return; }
      const float G = gumbel32(w), s = x + G, e = SCORE_ERR * (1.f + fabsf(x) + fabsf(G));
      if (s > best_mid || (s == best_mid && t < best_id)) {
        others = fmaxf(others, best_hi);
        best_mid = s; best_lo = s - e; best_hi = s + e; best_id = t;
      } else {
        others = fmaxf(others, s + e);
      }
      bar = fmaxf(bar, best_lo - PRUNE_MARGIN);
    });
    // Block merge of the certified picks.
    struct Pk { float mid, lo, hi, others; int id; };
    Pk pk{best_mid, best_lo, best_hi, others, best_id};
    auto op = [](Pk x, Pk y) {
      const bool yw = y.mid > x.mid || (y.mid == x.mid && y.id < x.id);
      Pk w = yw ? y : x, l = yw ? x : y;
      w.others = fmaxf(fmaxf(x.others, y.others), l.hi);
      return w;
    };
    pk = wave_all(pk, op, Pk{-INFINITY, -INFINITY, -INFINITY, -INFINITY, INT_MAX});
    __shared__ Pk s_pk[WAVES];
    __syncthreads();
    if (lane_id() == 0) s_pk[wave_id()] = pk;
    __syncthreads();
    Pk r = s_pk[0];
    for (int w = 1; w < WAVES; ++w) r = op(r, s_pk[w]);
    __syncthreads();
    if (r.id == INT_MAX) return -1;
    if (r.lo > r.others) return r.id;
    // FP64 rescoring of every token whose upper bound reaches the winner's lower bound.
    ++fallbacks;
    const float threshold = r.lo;
    double best = -INFINITY;
    int bid = INT_MAX;
    each<false>([&](int t, W v, bool ok) {
      if (t == excluded || !in(t, v, ok)) return;
      const float x = tp.x32(v);
      const float ub = x + GUMBEL_MAX + SCORE_ERR * (1.f + fabsf(x) + GUMBEL_MAX);
      if (ub < threshold) return;
      const uint32_t w = word_of(p.rng, uint32_t(sub), uint32_t(t));
      const float gb = gumbel_upper(w);
      if (x + gb + SCORE_ERR * (1.f + fabsf(x) + fabsf(gb)) < threshold) return;
      const double s = tp.x64(v) + gumbel64(w);
      if (s > best || (s == best && t < bid)) { best = s; bid = t; }
    });
    struct SI { double s; int id; };
    SI si{best, bid};
    auto op2 = [](SI x, SI y) { return (y.s > x.s || (y.s == x.s && y.id < x.id)) ? y : x; };
    si = wave_all(si, op2, SI{-INFINITY, INT_MAX});
    __syncthreads();
    if (lane_id() == 0) { sh.dred[wave_id()] = si.s; sh.ired[wave_id()] = si.id; }
    __syncthreads();
    SI res{sh.dred[0], sh.ired[0]};
    for (int w = 1; w < WAVES; ++w) res = op2(res, SI{sh.dred[w], sh.ired[w]});
    __syncthreads();
    return res.id == INT_MAX ? -1 : res.id;
  }

  // Finishes the row. Greedy rows without a full proposal and failed rows
  // never come here.
  __device__ __forceinline__ RowResult run(double maximum, int greedy, int runner_up_id, int valid) {
    RowResult r{0, 1, -1, -1, ES_OK, ES_OK};
    const bool full_q = p.full_q != 0;
    // ---- The actual proposal q of a full-q draft row (reference.py:206-216). ----
    double qmax = -INFINITY, sq = 0, wq_draft = 0;
    if (full_q) {
      int qbad = 0, qvalid = 0;
      W qm = neg_inf<W>();
      each<true>([&](int, W y, bool) {
        qbad |= isnan(y) || y == W(INFINITY);
        qvalid += y > neg_inf<W>();
        qm = y > qm ? y : qm;
      });
      qbad = block_all(qbad, [](int x, int y) { return x | y; }, sh.ired, 0);
      qvalid = block_all(qvalid, [](int x, int y) { return x + y; }, sh.ired, 0);
      qm = block_all(qm, [](W x, W y) { return x > y ? x : y; }, sh.u.r.red_w, neg_inf<W>());
      int qstatus = qbad ? ES_INVALID_INPUT : qvalid == 0 ? ES_NO_VALID_TOKEN : ES_OK;
      qmax = double(qm);
      if (qstatus == ES_OK) {
        // sq = fsum over q's support of exp(y - qmax) (no filters, T = 1).
        sq = exact_sum<true>([&](int, W y, bool) -> double {
          return y > neg_inf<W>() ? exp(double(y) - qmax) : 0.0;
        }, false);
        const W yd = qview.value(p.draft_id);
        wq_draft = yd > neg_inf<W>() ? exp(double(yd) - qmax) : 0.0;
        if (!(wq_draft / sq > 0)) qstatus = ES_DRAFT_ZERO_PROB;
      }
      if (qstatus != ES_OK) { r.status = qstatus; return r; }
    }
    auto qprob = [&](int t) -> double {
      const W y = qview.value(t);
      return y > neg_inf<W>() ? exp(double(y) - qmax) / sq : 0.0;
    };
    // ---- Greedy full-q rows: p is a point mass at the greedy token. ----
    if (p.temperature == 0) {
      r.sample = greedy;
      if (p.verify) {
        const double qx = wq_draft / sq;
        const double px = p.draft_id == greedy ? 1.0 : 0.0;
        const double u = uniform64(word_of(p.rng, 1u, 0u));
        const bool accept = u < fmin(1.0, px / qx);
        r.p = accept ? 1.0 : 0.0;
        if (!accept) r.residual = fmax(1.0 - qprob(greedy), 0.0) > 0 ? greedy : -1;
      }
      return r;
    }
    tp.init(maximum, p.temperature, p.min_p);
    // ---- Kept set: valid, min-p and positivity (a prefix of the order). ----
    auto kept = [&](int, W v, bool ok) { return valid_tok(v, ok) && tp.kept(v, tp.x32(v)); };
    // ---- Top-k: an exact cut at the k-th token (reference.py:67-71). ----
    // The kept count is needed only when k may cut: k < valid tokens.
    u128 cut = 0;  // keep ck >= cut
    bool topk_cut = false;
    if (p.top_k > 0 && p.top_k < valid) {
      int nk = 0;
      each<false>([&](int t, W v, bool ok) { nk += kept(t, v, ok); });
      nk = block_all(nk, [](int x, int y) { return x + y; }, sh.ired, 0);
      if (p.top_k < nk) {
        cut = select_nth(int(p.top_k), kept);
        topk_cut = true;
      }
    }
    auto in_k = [&](int t, W v, bool ok) { return kept(t, v, ok) && CK<W>::make(v, t) >= cut; };
    auto w64 = [&](int, W v) -> double { return exp(tp.x64(v)); };
    double den = 0;
    bool den_exact = false;
    // The floor of a draw: the first token of the order that the draw may take.
    const int floor_token = greedy >= 0 && greedy < int(a.vocab) ? greedy : -1;
    // The residual's floor: the greedy token, or the runner-up when the draft is greedy.
    const int residual_floor = p.draft_id == greedy ? (runner_up_id != INT_MAX ? runner_up_id : -1) : floor_token;
    // ---- Top-p: the shortest prefix whose fsum reaches top_p * fsum(all) (reference.py:73-85). ----
    bool binned = false;  // the cut, its mass bounds and the draw's pick come from the bins
    BinnedCut bc;
    if (p.top_p < 1 && !topk_cut && !full_q && tb) {
      binned = topp_binned(p.verify ? 2u : 0u, p.verify ? p.draft_id : -1, p.verify ? residual_floor : floor_token,
                           &bc);
      if (!finisher) return r;  // another finishing block of the row takes it from here
      if (binned) {
        cut = bc.cut;
        den = bc.den_lo;
        den_exact = bc.den_exact;
      }
    }
    // A pick that settles the draw: certified, or certainly empty.
    auto settled = [](const Pick& pk) { return pk.id == INT_MAX ? !(pk.others > -INFINITY) : pk.lo > pk.others; };
    if (p.top_p < 1 && !binned) {
      cut = mass_boundary(p.top_p, in_k, w64);
      // The kept mass is needed by the ratio test and the residual only: a
      // draw compares x + G, the same for every token up to log(den).
      if (p.verify) {
        den = exact_sum<false>([&](int t, W v, bool ok) -> double {
          return in_k(t, v, ok) && CK<W>::make(v, t) >= cut ? w64(t, v) : 0.0;
        }, false);
        den_exact = true;
      }
    }
    auto in_final = [&](int t, W v, bool ok) { return in_k(t, v, ok) && CK<W>::make(v, t) >= cut; };
    // ---- Ratio test (reference.py:229-230). ----
    if (p.verify) {
      const W vx = view.value(p.draft_id);
      const bool x_in = in_final(p.draft_id, vx, allowed(a, row, p.draft_id));
      const double u = uniform64(word_of(p.rng, 1u, 0u));
      bool accept = false;
      if (x_in) {
        if (binned && !den_exact) {
          // The nucleus mass bounds from the bins first.
          const double wx = exp(tp.x64(vx));
          const double rlo = fmin(1.0, wx / bc.den_hi) * (1 - 1e-12), rhi = fmin(1.0, wx / bc.den_lo) * (1 + 1e-12);
          const bool bounded = bc.den_lo > 0 && bc.den_hi >= bc.den_lo;
          if (bounded && u < rlo) accept = true;
          else if (bounded && u >= rhi) accept = false;
          else {
            den = exact_sum<false>([&](int t, W v, bool ok) -> double { return in_final(t, v, ok) ? w64(t, v) : 0.0; }, false);
            den_exact = true;
            ++fallbacks;
            accept = u < fmin(1.0, wx / den);
          }
        } else if (!den_exact) {
          // FP32 sum of kept weights with its bound first.
          float s = 0, c = 0, e = 0;
          int pruned = 0;
          each<false>([&](int t, W v, bool ok) {
            if (!in_final(t, v, ok)) return;
            const float x = tp.x32(v);
            if (x < SUM_PRUNE) { ++pruned; return; }
            const float w = weight32(x), d = w - c, tt = s + d;
            c = (tt - s) - d; s = tt;
            e += w * (X_ERR * (1.f + fabsf(x)));
          });
          const double sum = block_all(double(s) - double(c), [](double x, double y) { return x + y; }, sh.dred, 0.0);
          const double et = block_all(double(e), [](double x, double y) { return x + y; }, sh.dred, 0.0);
          pruned = block_all(pruned, [](int x, int y) { return x + y; }, sh.ired, 0);
          const double esp = 1.01 * et + 4.8e-7 * sum + pruned * SUM_PRUNE_W;
          const double wx = exp(tp.x64(vx));
          const double qx_lo = full_q ? wq_draft / sq * (1 - 1e-15) : 1.0, qx_hi = full_q ? wq_draft / sq * (1 + 1e-15) : 1.0;
          const double rlo = fmin(1.0, wx / (sum + esp) / qx_hi) * (1 - 1e-12);
          const double rhi = fmin(1.0, wx / (sum - esp) / qx_lo) * (1 + 1e-12);
          const bool bounded = esp >= 0 && sum - esp > 0;
          if (bounded && u < rlo) accept = true;
          else if (bounded && u >= rhi) accept = false;
          else {
            den = exact_sum<false>([&](int t, W v, bool ok) -> double { return in_final(t, v, ok) ? w64(t, v) : 0.0; }, false);
            den_exact = true;
            ++fallbacks;
            accept = u < fmin(1.0, (wx / den) / (full_q ? wq_draft / sq : 1.0));
          }
        } else {
          const double px = exp(tp.x64(vx)) / den;
          accept = u < fmin(1.0, px / (full_q ? wq_draft / sq : 1.0));
        }
      }
      r.p = accept ? 1.0 : 0.0;
      if (accept) return r;
      if (!full_q) {
        if (binned && settled(bc.pick)) {
          r.residual = bc.pick.id == INT_MAX ? -1 : bc.pick.id;
          return r;
        }
        const int floor_id = residual_floor;
        int fl = floor_id >= 0 && floor_id < int(a.vocab) ? floor_id : -1;
        if (fl >= 0 && fl != greedy) {
          const W vf = view.value(fl);
          if (!in_final(fl, vf, allowed(a, row, fl))) fl = -1;
        }
        r.residual = draw(2, p.draft_id, fl, in_final);
        return r;
      }
      // Full-q residual max(p - q, 0) in FP64 over the kept set (reference.py:236).
      if (!den_exact) {
        den = exact_sum<false>([&](int t, W v, bool ok) -> double { return in_final(t, v, ok) ? w64(t, v) : 0.0; }, false);
        den_exact = true;
      }
      double best = -INFINITY;
      int bid = INT_MAX;
      each<false>([&](int t, W v, bool ok) {
        if (!in_final(t, v, ok)) return;
        const double pr = exp(tp.x64(v)) / den;
        const double rr = fmax(pr - qprob(t), 0.0);
        if (!(rr > 0)) return;
        const double s = log(rr) + gumbel64(word_of(p.rng, 2u, uint32_t(t)));
        if (s > best || (s == best && t < bid)) { best = s; bid = t; }
      });
      struct SI { double s; int id; };
      SI si{best, bid};
      auto op2 = [](SI x, SI y) { return (y.s > x.s || (y.s == x.s && y.id < x.id)) ? y : x; };
      si = wave_all(si, op2, SI{-INFINITY, INT_MAX});
      __syncthreads();
      if (lane_id() == 0) { sh.dred[wave_id()] = si.s; sh.ired[wave_id()] = si.id; }
      __syncthreads();
      SI res{sh.dred[0], sh.ired[0]};
      for (int w = 1; w < WAVES; ++w) res = op2(res, SI{sh.dred[w], sh.ired[w]});
      __syncthreads();
      r.residual = res.id == INT_MAX ? -1 : res.id;
      return r;
    }
    if (binned && settled(bc.pick)) {
      r.sample = bc.pick.id == INT_MAX ? -1 : bc.pick.id;
      return r;
    }
    r.sample = draw(0, -1, floor_token, in_final);
    return r;
  }
};

// A stream row's slice: its certified draw over the slice's tokens that may
// be kept, read again from memory (cache hits), stored where a list row keeps
// candidates (reference: fused.cuh:532-681 row_scan). Scores are relative to
// a reference maximum: the slice's, or for a min-p row the largest slice
// maximum of the row published so far, a lower bound on the row maximum, so
// the tokens that may be kept against it (valid, not certainly below min-p or
// underflowing) are a superset of the kept ones. A min-p slice whose pick
// falls under the threshold of a larger maximum published meanwhile draws
// again against that one. The merge settles which pick is kept, exactly, and
// scans again any slice whose pick is not. Ratio rows also sum their kept
// weights (relative to the slice maximum).
struct SliceDraw { double sum, err, mref; int pruned; };
template <int DT, bool VEC, class W>
__device__ __forceinline__ SliceDraw slice_draw(const es_arguments& a, int64_t row, int slice, Params p,
                                             const RowView<DT, VEC>& view, int g0, int g1, double smax, int first_id,
                                             int cap_slice, uint32_t gen, Shared<W>& sh) {
  constexpr int B = 4;  // groups in flight per thread
  const int tid = threadIdx.x;
  load_row_rng(a, row, &p);
  const uint32_t sub = stream_sub(p);
  const int excluded = sub == 2u ? p.draft_id : -1;
  unsigned long long* key = &counters(a, row)->max_key;
  auto published = [&]() {
    if (tid == 0) sh.dred[0] = published_max(key, gen);
    __syncthreads();
    const double m = sh.dred[0];
    __syncthreads();
    return m;
  };
  double mref = smax;
  if (p.min_p > 0) {
    if (tid == 0) publish_max(key, gen, order_key(float_at_or_below(smax)));
    mref = fmax(smax, published());
  }
  Temp<W> ts;
  ts.init(mref, p.temperature, p.min_p);
  // x may be kept: x + X_ERR |x| >= ln(min_p) - tol (x32 is within X_ERR |x| of x), and no underflow.
  const float keep_lo = ts.ln_min_p - ts.min_p_tol;
  auto maybe_kept = [&](W, float x) { return x > -746.5f && fmaf(fabsf(x), X_ERR, x) >= keep_lo; };
  // The floor: the slice maximum's own score, when it may be drawn.
  auto floor_of = [&]() {
    if (tid == 0) {
      float f = -INFINITY;
      const float x = ts.x32(W(smax));
      if (first_id != excluded && maybe_kept(W(smax), x)) {
        const float g = gumbel32(word_of(p.rng, sub, uint32_t(first_id)));
        f = x + g - SCORE_ERR * (1.f + fabsf(x) + fabsf(g));
      }
      sh.fred[0] = f;
    }
    __syncthreads();
    const float f = sh.fred[0];
    __syncthreads();
    return f;
  };
  SliceDraw out{0.0, 0.0, mref, 0};
  Pick pk;
  if (sub == 2u) {
    // Ratio rows (never min-p ones) also sum their kept weights for the acceptance test.
    KahanSum ks;
    pk = range_pick<B, true>(a, row, view, g0, g1, ts, p.rng, sub, excluded, floor_of(), maybe_kept, &ks);
    out.sum = block_all(double(ks.s) - double(ks.c), [](double x, double y) { return x + y; }, sh.dred, 0.0);
    // The FP32 terms' bound, the Kahan sums' and the block's FP64 tree.
    out.err = 1.01 * block_all(double(ks.e), [](double x, double y) { return x + y; }, sh.dred, 0.0) +
              4.8e-7 * out.sum;
    out.pruned = block_all(ks.pruned, [](int x, int y) { return x + y; }, sh.ired, 0);
    pk = block_pick(pk, sh);
  } else {
    if (p.min_p > 0) {
      pk = range_pick<B, false>(a, row, view, g0, g1, ts, p.rng, sub, excluded, floor_of(), maybe_kept, nullptr);
    } else {
      // Without min-p a token may be kept unless its weight underflows.
      pk = range_pick<B, false>(a, row, view, g0, g1, ts, p.rng, sub, excluded, floor_of(),
                                [](W, float x) { return x > -746.5f; }, nullptr);
    }
    pk = block_pick(pk, sh);
    if (p.min_p > 0 && pk.id != INT_MAX) {
      const double m2 = published();
      if (m2 > mref) {
        ts.init(m2, p.temperature, p.min_p);
        const W vp = view.value(pk.id);
        if (!ts.kept(vp, ts.x32(vp))) {
          out.mref = m2;
          pk = range_pick<B, false>(a, row, view, g0, g1, ts, p.rng, sub, excluded, floor_of(), maybe_kept, nullptr);
          pk = block_pick(pk, sh);
        }
      }
    }
  }
  if (tid == 0) *slice_pick<W>(a, row, slice, cap_slice) = pk;
  return out;
}

// ---------------------------------------------------------------------------
// The slice's tokens in the register tile's order. Token (i, j) of a thread
// is 4 * (gb + BLOCK * i) + j, so IDs rise with (i, thread, j); tokens that
// are masked or outside the slice have the value -inf. The tile itself dies
// after the statistics pass: MemVisit reads every token again from memory,
// CandVisit only the groups that can hold a candidate.
template <int DT, bool VEC, int G> struct MemVisit {
  using W = typename Ty<DT>::W;
  RowView<DT, VEC> view;
  const int32_t* mask;  // the row's mask words, or null
  int64_t mask_s1;
  int gb, g1, groups;
  __device__ __forceinline__ MemVisit(const es_arguments& a, int64_t row, const RowView<DT, VEC>& v, int gb_, int g1_,
                                      int groups_)
      : view(v), mask(a.mask ? a.mask + row * a.mask_s0 : nullptr), mask_s1(a.mask_s1), gb(gb_), g1(g1_),
        groups(groups_) {}
  template <class F> __device__ __forceinline__ void operator()(F&& f) const {
#pragma unroll 1
    for (int i = 0; i < G; ++i) {
      const int g = gb + BLOCK * i, gc = min(g, groups - 1);
      W x[4];
      view.load(gc, x);
      uint32_t mb = g < g1 ? 0xfu : 0u;
      if (mask && 4 * gc < view.vocab) mb &= uint32_t(mask[int64_t((4 * gc) >> 5) * mask_s1]) >> ((4 * gc) & 31);
#pragma unroll
      for (int j = 0; j < 4; ++j) f(i, j, ((mb >> j) & 1u) ? x[j] : neg_inf<W>(), 4 * g + j);
    }
  }
};

// The slice's tokens in the groups marked in `cmask` (bit i: group row i of
// the tile may hold a candidate), read again from memory four groups at a
// time, in the tile's order; masked tokens have the value -inf. groups(f)
// calls f(i, x[4]) per marked group with the raw values.
template <int DT, bool VEC, int G> struct CandVisit {
  using W = typename Ty<DT>::W;
  RowView<DT, VEC> view;
  uint32_t cmask;
  int gb;
  uint64_t allow;
  template <class F> __device__ __forceinline__ void groups(F&& f) const {
    uint32_t m = cmask;
    while (__ballot(m != 0)) {
      int idx[4];
      bool has[4];
      W x[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        has[q] = m != 0;
        idx[q] = has[q] ? __ffs(m) - 1 : 0;
        m = has[q] ? m & (m - 1) : m;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (has[q]) view.load(gb + BLOCK * idx[q], x[q]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (has[q]) f(idx[q], x[q]);
      }
    }
  }
  template <class F> __device__ __forceinline__ void operator()(F&& f) const {
    groups([&](int i, const W (&x)[4]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) f(i, j, ((allow >> (4 * i + j)) & 1ull) ? x[j] : neg_inf<W>(), 4 * (gb + BLOCK * i) + j);
    });
  }
};

// The groups of the tile whose maximum reaches `floor`, as a bit mask.
template <class W, int G> __device__ __forceinline__ uint32_t groups_reaching(const W (&gm)[G], W floor) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < G; ++i) m |= uint32_t(gm[i] >= floor) << i;
  return m;
}

// One bit per token where pred(value, id) holds (valid tokens only).
template <class W, class Visit, class Pred>
__device__ __forceinline__ uint64_t collect_bits(const Visit& visit, Pred&& pred) {
  uint64_t bits = 0;
  visit([&](int i, int j, W x, int t) {
    if (pred(x, t) && x > neg_inf<W>()) bits |= 1ull << (4 * i + j);
  });
  return bits;
}

// Appends the tokens whose bits are set to the block's list in LDS (in any
// order: the list is sorted afterwards) and returns the block's total.
template <class W, class Visit>
__device__ __forceinline__ int append_taken(const Visit& visit, uint64_t bits, Shared<W>& sh) {
  const int mine = __popcll(bits);
  int slot = mine ? atomicAdd(&sh.appended, mine) : 0;
  if (mine) {
    visit([&](int i, int j, W x, int t) {
      if ((bits >> (4 * i + j)) & 1ull) {
        if (slot < LIST_LIMIT) {
          sh.u.list.v[slot] = x;
          sh.u.list.id[slot] = t;
        }
        ++slot;
      }
    });
  }
  __syncthreads();
  return sh.appended;
}

// Stores the tokens whose bits are set, in visit order, at out[0, popcount).
template <class W, class Visit>
__device__ __forceinline__ void publish_taken(const Visit& visit, uint64_t bits, Cand<W>* out) {
  int o = 0;
  visit([&](int i, int j, W x, int t) {
    if ((bits >> (4 * i + j)) & 1ull) {
      Cand<W> c{};
      c.v = x;
      c.id = t;
      publish(out + o, c);
      ++o;
    }
  });
}

// The slice's L-th valid token in (value desc, ID asc) order, given that at
// least L valid tokens are >= floor: radix selection over the value's order
// key among those tokens (8-bit digits), then the tie broken by ID, which is
// the (i, thread, j) order of the visit.
template <class W, int G, class Visit>
__device__ __forceinline__ void slice_cut(const Visit& visit, int L, W floor, Shared<W>& sh, W* out_v, int* out_id) {
  using K = typename std::conditional<sizeof(W) == 8, uint64_t, uint32_t>::type;
  constexpr int KB = int(sizeof(K) * 8);
  // Scratch in the block's union: 256 counters, then G x BLOCK tie counts.
  unsigned* hist = reinterpret_cast<unsigned*>(&sh.u);
  static_assert(sizeof(sh.u) >= (256 + G * BLOCK + WAVES * G) * sizeof(int), "slice_cut scratch");
  K prefix = 0, known = 0;
  int need = L;
  for (int shift = KB - 8; shift >= 0; shift -= 8) {
    __syncthreads();
    hist[threadIdx.x] = 0;
    __syncthreads();
    visit([&](int, int, W x, int) {
      if (x >= floor && x > neg_inf<W>()) {
        const K k = order_key(x);
        if ((k & known) == prefix) atomicAdd(&hist[int(k >> shift) & 255], 1u);
      }
    });
    __syncthreads();
    const int c = int(hist[255 - threadIdx.x]);  // descending digits, one per thread
    int tot;
    const int incl = block_scan_add(c, sh.ired, &tot);
    if (incl >= need && incl - c < need) { sh.pick = 255 - int(threadIdx.x); sh.n = incl - c; }
    __syncthreads();
    need -= sh.n;
    prefix |= K(sh.pick) << shift;
    known |= K(255) << shift;
  }
  const W cut_v = key_value(prefix);
  // `need` tokens with value cut_v are taken, the lowest IDs first. IDs rise
  // with (i, thread, j): the per-(i, thread) tie counts locate the group row
  // i holding the need-th tie (totals over threads per i), then the thread
  // (a scan over threads at that i), then the tie inside the thread's group.
  int* ties = reinterpret_cast<int*>(&sh.u) + 256;  // [G][BLOCK]
  for (int i = 0; i < G; ++i) ties[i * BLOCK + threadIdx.x] = 0;
  visit([&](int i, int, W x, int) { ties[i * BLOCK + threadIdx.x] += x == cut_v; });
  int* row_tot = reinterpret_cast<int*>(&sh.u) + 256 + G * BLOCK;  // [WAVES][G]
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int t = wave_all(ties[i * BLOCK + threadIdx.x], [](int x, int y) { return x + y; }, 0);
    if (lane_id() == 0) row_tot[wave_id() * G + i] = t;
  }
  if (threadIdx.x == 0) sh.ck = INT_MAX;
  __syncthreads();
  int gi = 0, before = 0;
  for (; gi < G; ++gi) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) t += row_tot[w * G + gi];
    if (before + t >= need) break;
    before += t;
  }
  gi = min(gi, G - 1);
  const int c = ties[gi * BLOCK + threadIdx.x];
  int all;
  const int incl = block_scan_add(c, sh.ired, &all) + before;
  if (c > 0 && incl >= need && incl - c < need) {
    const int rank = need - (incl - c);  // the rank of the last taken tie inside this thread's group
    int seen = 0, id = INT_MAX;
    visit([&](int i, int, W x, int t) {
      if (i == gi && x == cut_v && ++seen == rank) id = t;
    });
    sh.ck = id;
  }
  __syncthreads();
  *out_v = cut_v;
  *out_id = int(sh.ck);
  __syncthreads();
}

// ---------------------------------------------------------------------------
// The kernel.
// The kernels' arguments read in place, in the kernel argument segment. A
// by-value kernel parameter whose address is taken (every helper takes the
// arguments by reference) is first copied whole into registers at kernel
// entry: 98 dwords that do not fit in SGPRs, so the copy runs as a chain of
// load, wait and spill rounds before any of the kernel's own loads. Read in
// place, each field is a scalar load where it is used. The explicit
// arguments sit at the segment's start in declaration order, each at its
// natural alignment, which is also KernelArgs' layout.
struct KernelArgs {
  es_arguments a;
  Plan pl;
};
static_assert(offsetof(KernelArgs, pl) == sizeof(es_arguments), "Plan follows es_arguments");
__device__ __forceinline__ const KernelArgs& kernel_args() {
  typedef const __attribute__((address_space(4))) KernelArgs* ArgPtr;
  return *(const KernelArgs*)(ArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
}

// A request block (reference: verify.cu:6-56 initialize), run by es_finish:
// the offsets check, header word 0, and the outputs of requests whose
// metadata is invalid. Header word 1 (the FP64 recompute count) is cleared by
// es_main's first block, or here when there are no rows.
__device__ __forceinline__ void request_block(const es_arguments& a, int rb) {
  const int tid = threadIdx.x;
  const bool malformed = offsets_malformed(a);
  if (rb == 0 && tid == 0) {
    reinterpret_cast<int32_t*>(a.workspace)[0] = malformed;
    if (a.rows == 0) reinterpret_cast<uint32_t*>(a.workspace)[1] = 0;
  }
  const int64_t req = int64_t(rb) * BLOCK + tid;
  if (req < a.requests) {
    const int32_t st = metadata_status(a, req, malformed);
    if (st != ES_OK) write_failed_request(a, req, st, path_of(a));
  }
}

// A slice block's request lookup and, in the row's first slice, the record
// the finishing block reads: the request's parameters, its per-row metadata
// check and the RNG address. The request's first row also zeroes the
// request's arrival counter, which the finishing kernel counts on after the
// kernel boundary.
template <class W>
__device__ __forceinline__ void slice_params(const es_arguments& a, int64_t row, int slice, int64_t x0, int64_t x1,
                                             Params* p, Shared<W>& sh) {
  slice_lookup(a, row, x0, x1, p, sh);
  if (slice == 0 && wave_id() == 0) {
    if (p->status == ES_OK) {
      load_row_rng(a, row, p);
      p->meta_bad = !request_rows_ok(a, *p);
    }
    if (lane_id() == 0) {
      *row_meta(a, row) = *p;
      if (p->status == ES_OK && row == p->begin) counters(a, row)->request = 0;
    }
  }
}

// The slice's summary, written by one thread with plain stores (the kernel
// boundary makes it visible to the finishing kernel).
__device__ __forceinline__ void write_part(const es_arguments& a, int64_t row, int slice, double smax, int first_id,
                                           double frontier, int frontier_id, double tau, double sum, double err,
                                           int valid, int n_cand, int pruned, int bad) {
  SlicePart part;
  part.max_v = smax;
  part.second_v = -INFINITY;
  part.frontier = frontier;
  part.tau = tau;  // a stream row's reference maximum for its pick
  part.sum = sum;
  part.err = err;
  part.max_id = first_id;
  part.second_id = frontier_id;
  part.valid = valid;
  part.n_cand = n_cand;
  part.pruned = pruned;
  part.flags = bad;
  slice_parts(a, row)[slice] = part;
}

// A binned top-p row's slice (reference: fused.cuh:686-750, row_hist, whose
// distance histogram and kept-mass sum this replaces): every valid token of
// the slice is binned on the absolute grid y = l * 4 / T against a reference
// maximum m_ref (the slice's, or the largest slice maximum of the row
// published so far, a lower bound on the row maximum): bin b = floor(y) at
// local index floor(m_ref * 4 / T) - b. The 64 bins below m_ref get the count
// and the sum of e^((y - b - 1/2) / 4) in FP64 (the weights relative to the
// bin's centre, a degree-11 polynomial); tokens further down go to an FP32
// Kahan sum of their weights relative to m_ref with the certified bound
// (tokens below e^-40 are bounded by the largest of them). Returns false (the
// row then takes the full-row path's radix boundary) when m_ref * 4 / T is
// out of range for the grid.
struct SliceBins { double mref, top, far_sum, far_err; };
template <int DT, bool VEC, class W>
__device__ __forceinline__ bool slice_bins(const es_arguments& a, int64_t row, int slice, const Params& p,
                                           const RowView<DT, VEC>& view, int g0, int g1, W smax, uint32_t gen,
                                           Shared<W>& sh, SliceBins* out) {
  const int tid = threadIdx.x;
  unsigned long long* key = &counters(a, row)->max_key;
  double* lmass = reinterpret_cast<double*>(&sh.u);
  unsigned* lcnt = reinterpret_cast<unsigned*>(lmass + TP_COARSE);
  if (tid == 0) {
    publish_max(key, gen, order_key(float_at_or_below(double(smax))));
    sh.dred[0] = published_max(key, gen);
  }
  if (tid < TP_COARSE) {
    lmass[tid] = 0;
    lcnt[tid] = 0;
  }
  __syncthreads();
  const double mref = fmax(double(smax), sh.dred[0]);
  const double inv4 = TP_Y_PER_X / p.temperature;
  const double yref = mref * inv4;
  if (!(fabs(yref) < 0x1p50)) return false;
  const double top = floor(yref);
  Temp<W> ts;
  ts.init(mref, p.temperature, 0.0);
  KahanSum ks;
  for (int base = g0 + tid; base < g1; base += 4 * BLOCK) {
    W x[4][4];
    uint32_t mb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = base + u * BLOCK;
      view.load(min(g, g1 - 1), x[u]);
      mb[u] = g < g1 ? group_bits(a, row, g) : 0u;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const W v = x[u][j];
        if (!(((mb[u] >> j) & 1u) && v > neg_inf<W>())) continue;
        const double y = double(v) * inv4, b = floor(y), k = top - b;
        if (k < double(TP_COARSE)) {
          atomicAdd(&lmass[int(k)], exp_center((y - b - 0.5) * (1.0 / TP_Y_PER_X)));
          atomicAdd(&lcnt[int(k)], 1u);
        } else {
          ks.add(ts.x32(v));
        }
      }
    }
  }
  __syncthreads();
  if (tid < TP_COARSE) {
    slice_bin_mass(a, row, slice)[tid] = lmass[tid];
    slice_bin_count(a, row, slice)[tid] = uint16_t(lcnt[tid]);
  }
  const double sum = block_all(double(ks.s) - double(ks.c), [](double x, double y) { return x + y; }, sh.dred, 0.0);
  const double e = block_all(double(ks.e), [](double x, double y) { return x + y; }, sh.dred, 0.0);
  const int pruned = block_all(ks.pruned, [](int x, int y) { return x + y; }, sh.ired, 0);
  const float pmax = block_all(ks.pruned_max, [](float x, float y) { return x > y ? x : y; }, sh.fred, -INFINITY);
  out->mref = mref;
  out->top = top;
  out->far_sum = sum;
  // The FP32 terms' bound, the Kahan sums' and the block's FP64 tree; the
  // tokens left out are each below e^(x32 (1 - 1e-6)).
  out->far_err = 1.01 * e + 4.8e-7 * sum + (pruned ? double(pruned) * exp(double(pmax) * (1 - 1e-6)) : 0.0);
  return true;
}

// es_wide, the slice pass of a call whose rows need more than MAX_SLICES
// register tiles (launched in place of es_main): each slice of several tiles
// is read group by group for the statistics (NaN/+inf anywhere, the valid
// count, the maximum with its lowest ID) and the streaming draw. Such calls
// store no list candidates (the host runs them with list_max 0), so filtered
// rows take the full-row path.
template <int DT, bool VEC>
__global__ void __launch_bounds__(BLOCK) es_wide(es_arguments, Plan) {
  using W = typename Ty<DT>::W;
  __shared__ Shared<W> sh;
  const es_arguments& a = kernel_args().a;
  const Plan pl = kernel_args().pl;
  const int tid = threadIdx.x, lane = lane_id();
  if (blockIdx.x == 0 && tid == 0) reinterpret_cast<uint32_t*>(a.workspace)[1] = 0;  // the FP64 recompute count
  const int64_t row = int(blockIdx.x) / pl.slices;
  const int slice = int(blockIdx.x) - int(row) * pl.slices;
  int64_t x0 = 0, x1 = 0;
  if (tid < a.requests) {
    x0 = at(a.cu_rows, tid);
    x1 = at(a.cu_rows, tid + 1);
  }
  Params p;
  slice_params(a, row, slice, x0, x1, &p, sh);
  if (p.status != ES_OK) return;
  const RowView<DT, VEC> view(a.target, row, int(a.vocab));
  const int g0 = slice * pl.gps, g1 = min(g0 + pl.gps, pl.groups);
  int bad_l = 0, valid_l = 0, fid_l = INT_MAX;
  W m_l = neg_inf<W>();
  for (int base = g0 + tid; base < g1; base += 4 * BLOCK) {
    W x[4][4];
    uint32_t mb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = base + u * BLOCK;
      view.load(min(g, g1 - 1), x[u]);
      mb[u] = g < g1 ? group_bits(a, row, g) : 0u;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = base + u * BLOCK;
      if (g >= g1) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const W y = x[u][j];
        bad_l |= y != y || y == W(INFINITY);
        const bool ok = ((mb[u] >> j) & 1u) && y > neg_inf<W>();
        valid_l += ok;
        if (ok && y > m_l) { m_l = y; fid_l = 4 * g + j; }
      }
    }
  }
  struct MI { W v; int id; };
  const MI wm = wave_all(MI{m_l, fid_l}, [](MI x, MI y) { return (y.v > x.v || (y.v == x.v && y.id < x.id)) ? y : x; },
                         MI{neg_inf<W>(), INT_MAX});
  const int valid_w = wave_all(valid_l, [](int x, int y) { return x + y; }, 0);
  const int bad_w = __ballot(bad_l) != 0;
  if (lane == 0) {
    sh.st_max[wave_id()] = wm.v;
    sh.st_id[wave_id()] = wm.id;
    sh.st_valid[wave_id()] = valid_w;
    sh.st_bad[wave_id()] = bad_w;
  }
  __syncthreads();
  W smax = neg_inf<W>();
  int first_id = INT_MAX, valid = 0, bad = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    if (sh.st_max[w] > smax || (sh.st_max[w] == smax && sh.st_id[w] < first_id)) {
      smax = sh.st_max[w];
      first_id = sh.st_id[w];
    }
    valid += sh.st_valid[w];
    bad |= sh.st_bad[w];
  }
  double psum = 0, perr = 0, tau = -INFINITY;
  int pruned = 0;
  if (a.dispatch != 1 && stream_row(p, a.vocab) && !bad && valid > 0) {
    const SliceDraw sd = slice_draw<DT, VEC>(a, row, slice, p, view, g0, g1, double(smax), first_id, pl.cap_slice,
                                             pl.generation, sh);
    psum = sd.sum;
    perr = sd.err;
    pruned = sd.pruned;
    tau = sd.mref;
  }
  if (tid == 0) write_part(a, row, slice, double(smax), first_id, -INFINITY, INT_MAX, tau, psum, perr, valid, 0, pruned, bad);
}

template <int DT, bool VEC, int G>
__global__ void __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(5))) es_main(es_arguments, Plan) {
  using W = typename Ty<DT>::W;
  __shared__ Shared<W> sh;
  const es_arguments& a = kernel_args().a;
  const Plan pl = kernel_args().pl;
  const int tid = threadIdx.x;
  const int lane = lane_id();

  // Every block is a slice block: the request checks run in the finishing
  // kernel, so that none of this kernel's resident slots is held by them.
  if (blockIdx.x == 0 && tid == 0) reinterpret_cast<uint32_t*>(a.workspace)[1] = 0;  // the FP64 recompute count

  // ---- Slice blocks. ----
  const int b = int(blockIdx.x);
  const int64_t row = b / pl.slices;
  const int slice = b - int(row) * pl.slices;
  const int vocab = int(a.vocab);
  const RowView<DT, VEC> view(a.target, row, vocab);
  const int g0 = slice * pl.gps, g1 = min(g0 + pl.gps, pl.groups);

  // The first chunk of the offsets, then the tile: waiting for the offsets
  // (vmcnt counts loads in issue order) leaves the tile loads in flight. Every
  // lane loads the whole tile (indexes clamped into the slice), so there is no
  // branch per load.
  int64_t x0 = 0, x1 = 0;
  if (tid < a.requests) {
    x0 = at(a.cu_rows, tid);
    x1 = at(a.cu_rows, tid + 1);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Tile loads. Groups past the slice's end are loaded as copies of its last
  // group: they never change the maximum or the checks below, and `allow`
  // keeps them out of counts and candidates.
  W v[G][4];
  const int gb = g0 + tid;
#pragma unroll
  for (int i = 0; i < G; ++i) view.load(min(gb + BLOCK * i, g1 - 1), v[i]);
  const int n_in = g1 > gb ? min(G, (g1 - gb + BLOCK - 1) / BLOCK) : 0;  // groups of the tile in the slice
  uint64_t allow = 4 * n_in >= 64 ? ~0ull : (1ull << (4 * n_in)) - 1ull;
  if (a.mask) {
    // Group gb + BLOCK * i has its bits in mask word (gb >> 3) + 32 i, at the
    // same shift for every i.
    uint64_t mbits = 0;
    const int32_t* mp = a.mask + row * a.mask_s0 + int64_t(gb >> 3) * a.mask_s1;
    const int64_t step = 32 * a.mask_s1;
    const int shift = (4 * gb) & 31;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      if (i < n_in) mbits |= uint64_t((uint32_t(mp[i * step]) >> shift) & 0xfu) << (4 * i);
    }
    allow &= mbits;
  }
  Params p;
  slice_params(a, row, slice, x0, x1, &p, sh);
  if (p.status != ES_OK) return;
  const ListPlan lp = list_plan(p, a.list_max, pl.cap_slice, a.vocab, pl.slices);
  int need = lp.need;
  const int L = lp.L;
  const bool sorted_list = lp.sorted_list, need_topp = lp.need_topp;
  const int j_thr = (L + WAVES - 1) / WAVES;  // thread maxima per wave behind the candidate threshold

  // ---- Statistics (reference: fused.cuh:409-519 row_stats). ----
  // One pass over the tile, which dies here: per-group maxima (all that later
  // steps keep), the slice's maximum and, when it is needed, its lowest ID
  // (IDs rise with (i, thread, j)), and a non-finite detector over the tile
  // (fma(x, 0, acc) turns NaN for a NaN or infinite x and stays so). Groups
  // past the slice's end are copies: their maxima are -inf.
  const bool track_first = !sorted_list;  // greedy rows, lists a wave cannot take, the full-row path
  W gm[G];
  W mx = neg_inf<W>(), nf = W(0);
  int fid_l = INT_MAX;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const W m01 = v[i][1] > v[i][0] ? v[i][1] : v[i][0], m23 = v[i][3] > v[i][2] ? v[i][3] : v[i][2];
    const int jm = m23 > m01 ? (v[i][3] > v[i][2] ? 3 : 2) : (v[i][1] > v[i][0] ? 1 : 0);
    const W gmi = m23 > m01 ? m23 : m01;
#pragma unroll
    for (int j = 0; j < 4; ++j) nf = fma(v[i][j], W(0), nf);
    gm[i] = i < n_in ? gmi : neg_inf<W>();
    if (track_first) {
      const bool up = gm[i] > mx;
      fid_l = up ? 4 * (gb + BLOCK * i) + jm : fid_l;
      mx = up ? gm[i] : mx;
    } else {
      mx = gm[i] > mx ? gm[i] : mx;
    }
  }
  {
    const W wmax = wave_all(mx, [](W x, W y) { return x > y ? x : y; }, neg_inf<W>());
    const int wid = track_first ? wave_all(mx == wmax && wmax > neg_inf<W>() ? fid_l : INT_MAX,
                                           [](int x, int y) { return x < y ? x : y; }, INT_MAX)
                                : INT_MAX;
    const W tw = L > 0 ? key_value(wave_kth_largest(order_key(mx), j_thr)) : neg_inf<W>();
    const int nonfinite_w = __ballot(!(nf == W(0))) != 0;
    if (lane == 0) {
      sh.st_max[wave_id()] = wmax;
      sh.st_id[wave_id()] = wid;
      sh.st_bad[wave_id()] = nonfinite_w;
      sh.st_thr[wave_id()] = tw;
    }
  }
  if (tid == 0) sh.appended = 0;
  __syncthreads();
  int valid = 4 * (g1 - g0), bad = 0, first_id = INT_MAX, special = 0;
  W smax = neg_inf<W>(), thr_all = W(INFINITY);
  auto combine = [&]() {
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      if (sh.st_max[w] > smax || (sh.st_max[w] == smax && sh.st_id[w] < first_id)) {
        smax = sh.st_max[w];
        first_id = sh.st_id[w];
      }
      thr_all = sh.st_thr[w] < thr_all ? sh.st_thr[w] : thr_all;
    }
  };
  combine();
#pragma unroll
  for (int w = 0; w < WAVES; ++w) special |= sh.st_bad[w];
  if (special || a.mask || !VEC) {
    // Exact pass over the slice read again: a non-finite value, a mask or
    // element loads. NaN/+inf anywhere (even masked) makes the row invalid;
    // valid tokens are the allowed ones above -inf, and the group maxima are
    // taken over them.
    int bad_l = 0, valid_l = 0;
    W m2 = neg_inf<W>();
    fid_l = INT_MAX;
    // A fresh copy of gb: the tile's load addresses are then not reused here,
    // so the compiler need not keep all of them alive across the stats pass.
    int gbx = gb;
    asm volatile("" : "+v"(gbx));
    // Four groups in flight at a time (the scheduling barrier keeps the
    // compiler from hoisting every load, which would hold a second tile).
#pragma unroll
    for (int i0 = 0; i0 < G; i0 += 4) {
      W x[4][4];
#pragma unroll
      for (int q = 0; q < 4 && i0 + q < G; ++q) view.load(min(gbx + BLOCK * (i0 + q), g1 - 1), x[q]);
#pragma unroll
      for (int q = 0; q < 4 && i0 + q < G; ++q) {
        const int i = i0 + q;
        W g2 = neg_inf<W>();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const W y = x[q][j];
          bad_l |= y != y || y == W(INFINITY);
          const bool ok = ((allow >> (4 * i + j)) & 1ull) && y > neg_inf<W>();
          valid_l += ok;
          const bool up = ok && y > m2;
          fid_l = up ? 4 * (gb + BLOCK * i) + j : fid_l;
          m2 = up ? y : m2;
          g2 = ok && y > g2 ? y : g2;
        }
        gm[i] = g2;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    struct MI { W v; int id; };
    const MI wm = wave_all(MI{m2, fid_l}, [](MI x, MI y) { return (y.v > x.v || (y.v == x.v && y.id < x.id)) ? y : x; },
                           MI{neg_inf<W>(), INT_MAX});
    const W tw = L > 0 ? key_value(wave_kth_largest(order_key(m2), j_thr)) : neg_inf<W>();
    const int valid_w = wave_all(valid_l, [](int x, int y) { return x + y; }, 0);
    const int bad_w = __ballot(bad_l) != 0;
    __syncthreads();
    if (lane == 0) {
      sh.st_max[wave_id()] = wm.v;
      sh.st_id[wave_id()] = wm.id;
      sh.st_valid[wave_id()] = valid_w;
      sh.st_bad[wave_id()] = bad_w;
      sh.st_thr[wave_id()] = tw;
    }
    __syncthreads();
    valid = 0;
    first_id = INT_MAX;
    smax = neg_inf<W>();
    thr_all = W(INFINITY);
    combine();
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      valid += sh.st_valid[w];
      bad |= sh.st_bad[w];
    }
  }
  if (bad) need = 0;

  // ---- Candidates for a list row. ----
  // Only groups whose maximum reaches the threshold are read again (they are
  // few: the slice's top tokens); the rest of the slice is never revisited.
  const MemVisit<DT, VEC, G> mem(a, row, view, gb, g1, pl.groups);
  double frontier = -INFINITY, psum = 0, perr = 0, tau = -INFINITY;
  int n_cand = 0, pruned = 0, fid = INT_MAX;
  if (sorted_list && need > 0) {
    // Top-k rows: every valid token >= the threshold (at least L of them),
    // stored in any order; the merge wave selects. Complete down to (thr,
    // every ID), or entirely when thr is -inf.
    const W thr = need < valid ? thr_all : neg_inf<W>();
    const W take_from = thr > W(-3.4028234663852886e38) ? thr : W(-3.4028234663852886e38);
    const CandVisit<DT, VEC, G> cand{view, groups_reaching<W, G>(gm, take_from), gb, allow};
    Cand<W>* out = candidates<W>(a, row) + slice * pl.cap_slice;
    // Each candidate group takes slots from an LDS counter and stores its
    // tokens at once; slots past the capacity are not written (the exact cut
    // below then rewrites the list).
    const int limit = pl.cap_slice;
    cand.groups([&](int i, const W (&x)[4]) {
      int cnt = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) cnt += ((allow >> (4 * i + j)) & 1ull) && x[j] >= take_from;
      if (cnt) {
        int o = atomicAdd(&sh.appended, cnt);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (((allow >> (4 * i + j)) & 1ull) && x[j] >= take_from) {
            if (o < limit) {
              Cand<W> c{};
              c.v = x[j];
              c.id = 4 * (gb + BLOCK * i) + j;
              out[o] = c;
            }
            ++o;
          }
        }
      }
    });
    __syncthreads();
    const int total = sh.appended;
    if (total <= limit) {
      n_cand = total;
      frontier = double(thr);
    } else {
      // Too many (ties, or a low threshold): exactly the first L instead.
      W cut_v;
      int cut_id;
      slice_cut<W, G>(cand, L, take_from, sh, &cut_v, &cut_id);
      if (tid == 0) sh.appended = 0;
      __syncthreads();
      const uint64_t cb = collect_bits<W>(cand, [&](W x, int t) { return x > cut_v || (x == cut_v && t <= cut_id); });
      const int cm = __popcll(cb);
      const int cs = cm ? atomicAdd(&sh.appended, cm) : 0;
      if (cm) publish_taken<W>(cand, cb, out + cs);
      n_cand = L;
      frontier = double(cut_v);
      fid = cut_id;
    }
  } else if (need != 0) {
    const int cap = pl.cap_slice;
    W thr = need > 0 && need < valid ? thr_all : neg_inf<W>();
    // Tokens at or above the threshold: one bit per token of this thread.
    // -inf is never taken: the threshold is raised to the lowest finite value.
    const W take_from = thr > W(-3.4028234663852886e38) ? thr : W(-3.4028234663852886e38);
    const CandVisit<DT, VEC, G> cand{view, groups_reaching<W, G>(gm, take_from), gb, allow};
    uint64_t take_bits = collect_bits<W>(cand, [&](W x, int) { return x >= take_from; });
    int mine = __popcll(take_bits);
    int total;
    int offset = block_scan_add(mine, sh.ired, &total) - mine;
    fid = INT_MAX;  // complete down to (thr, any ID)
    if (total > cap && need > 0) {
      // Too many (ties, or a low threshold): take exactly the slice's first L
      // tokens in (value desc, ID asc) order instead.
      const int L = min(need, cap);
      W cut_v;
      int cut_id;
      slice_cut<W, G>(cand, L, take_from, sh, &cut_v, &cut_id);
      take_bits = collect_bits<W>(cand, [&](W x, int t) { return x > cut_v || (x == cut_v && t <= cut_id); });
      mine = __popcll(take_bits);
      offset = block_scan_add(mine, sh.ired, &total) - mine;
      thr = cut_v;
      fid = cut_id;
    }
    if (total <= cap) {
      // Few tokens per thread qualify: re-read their values (cache hits)
      // rather than index the register tile.
      Cand<W>* out = candidates<W>(a, row) + slice * cap + offset;
      int o = 0;
      while (take_bits) {
        const int k = __ffsll((unsigned long long)take_bits) - 1;
        take_bits &= take_bits - 1;
        const int t = 4 * (gb + BLOCK * (k >> 2)) + (k & 3);
        Cand<W> c{};
        c.v = view.value(t);
        c.id = t;
        publish(out + o, c);
        ++o;
      }
      n_cand = total;
      // Every valid token of the slice at or before (thr, fid) in (value desc,
      // ID asc) order is stored.
      frontier = double(thr);
    } else {
      n_cand = 0;
      frontier = INFINITY;  // nothing certain
      fid = -1;
    }
    // Top-p lists also need the kept weights' sum, relative to the slice
    // maximum: FP32 weights and Kahan sums per thread with the certified
    // bound (as the streaming draw's ratio rows), an FP64 block tree. Weights
    // below e^-40 are counted, not summed.
    if (need_topp) {
      Temp<W> ts;
      ts.init(double(smax), p.temperature, 0.0);
      KahanSum ks;
      for (int base = g0 + tid; base < g1; base += 4 * BLOCK) {
        W x[4][4];
        uint32_t mb[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int g = base + u * BLOCK;
          view.load(min(g, g1 - 1), x[u]);
          mb[u] = g < g1 ? group_bits(a, row, g) : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (((mb[u] >> j) & 1u) && x[u][j] > neg_inf<W>()) ks.add(ts.x32(x[u][j]));
          }
        }
      }
      psum = block_all(double(ks.s) - double(ks.c), [](double x, double y) { return x + y; }, sh.dred, 0.0);
      // The FP32 terms' bound, the Kahan sums' and the block's FP64 tree.
      perr = 1.01 * block_all(double(ks.e), [](double x, double y) { return x + y; }, sh.dred, 0.0) + 4.8e-7 * psum;
      pruned = block_all(ks.pruned, [](int x, int y) { return x + y; }, sh.ired, 0);
    }
  } else if (lp.binned && !bad && valid > 0) {
    // A binned top-p row: the slice's bins (n_cand TP_COARSE marks them
    // usable), its top bin in `frontier`, its reference maximum in `tau`.
    // The first slice readies the finishing blocks' arrival counter, gathered
    // count and, when they fit the boundary area, the bitmap and fine bins.
    if (slice == 0) {
      if (tid == 0) {
        counters(a, row)->bound = 0;
        *bound_count(a, row, pl.slices) = 0;
      }
      const int64_t words = bound_bitmap_words(a.vocab);
      if (words <= bound_capacity(pl.slices)) {
        uint32_t* bitmap = bound_ids(a, row, pl.slices);
        for (int i = tid; i < int(words); i += BLOCK) bitmap[i] = 0;
      }
      if (bound_fine_fits(pl.slices, a.vocab)) {
        double* fm = bound_fine_mass(a, row, pl.slices);
        uint32_t* fc = bound_fine_count(a, row, pl.slices);
        for (int i = tid; i < TP_FINE_SHARED; i += BLOCK) { fm[i] = 0; fc[i] = 0; }
      }
    }
    SliceBins sb;
    if (slice_bins<DT, VEC>(a, row, slice, p, view, g0, g1, smax, pl.generation, sh, &sb)) {
      tau = sb.mref;
      frontier = sb.top;
      psum = sb.far_sum;
      perr = sb.far_err;
      n_cand = TP_COARSE;
    } else {
      n_cand = -1;
    }
  } else if (a.dispatch != 1 && stream_row(p, a.vocab) && !bad && valid > 0) {
    const SliceDraw sd = slice_draw<DT, VEC>(a, row, slice, p, view, g0, g1, double(smax), first_id, pl.cap_slice,
                                             pl.generation, sh);
    psum = sd.sum;
    perr = sd.err;
    pruned = sd.pruned;
    tau = sd.mref;
  }
  if (tid == 0) write_part(a, row, slice, double(smax), first_id, frontier, fid, tau, psum, perr, valid, n_cand, pruned, bad);
}

// ---------------------------------------------------------------------------
// A pick with FP64 scores relative to the row maximum (slices' picks after
// their shift).
struct DPick { double mid, lo, hi, others; int id; };
__device__ __forceinline__ DPick dpick_none() { return DPick{-INFINITY, -INFINITY, -INFINITY, -INFINITY, INT_MAX}; }
__device__ __forceinline__ DPick dpick_join(DPick x, DPick y) {
  const bool yw = y.mid > x.mid || (y.mid == x.mid && y.id < x.id);
  DPick w = yw ? y : x;
  const DPick l = yw ? x : y;
  w.others = fmax(fmax(x.others, y.others), l.hi);
  return w;
}

// Finishes a stream row from its slices' picks (merged into sh.sp_* by the
// merge wave): scans again, exactly against the row maximum, the slices whose
// pick is not kept, then takes the winner when its interval clears every
// other score, and for a draft row in ratio mode settles u < min(1, p_x)
// with the slices' kept mass (reference: fused.cuh:532-681, the last slice's
// commit; reference.py:229-230). False when a certificate fails: the
// full-row path then decides.
template <int DT, bool VEC, class W>
__device__ __forceinline__ bool stream_finish(const es_arguments& a, int64_t row, const Params& p, const Plan& pl,
                                              Shared<W>& sh, RowResult* out, int* why) {
  const RowView<DT, VEC> view(a.target, row, int(a.vocab));
  Temp<W> tm;
  tm.init(sh.maximum, p.temperature, p.min_p);
  const uint32_t sub = stream_sub(p);
  const int excluded = sub == 2u ? p.draft_id : -1;
  DPick best{sh.sp_mid, sh.sp_lo, sh.sp_hi, sh.sp_others, sh.sp_id};
  unsigned long long again = sh.sp_rescan;
  __syncthreads();
  while (again) {
    const int s = __ffsll(again) - 1;
    again &= again - 1;
    const int gs = s * pl.gps, ge = min(gs + pl.gps, pl.groups);
    const float floor = best.id != INT_MAX ? float(best.lo) : -INFINITY;
    Pick r = range_pick<4, false>(a, row, view, gs, ge, tm, p.rng, sub, excluded, floor,
                                  [&](W v, float x) { return tm.kept(v, x); }, nullptr);
    r = block_pick(r, sh);
    best = dpick_join(best, DPick{double(r.mid), double(r.lo), double(r.hi), double(r.others), r.id});
  }
  if (best.id != INT_MAX && !(best.lo > best.others)) {
    *why = 8;  // scores too close for FP32: the full-row path rescores them in FP64
    return false;
  }
  const int token = best.id == INT_MAX ? -1 : best.id;
  if (sub != 2u) {
    out->sample = token;
    return true;
  }
  // Ratio test of the draft (one-hot q: p_x / q_x = p_x).
  bool accept = false;
  const int x = p.draft_id;
  const W vx = view.value(x);
  if (allowed(a, row, x) && vx > neg_inf<W>() && tm.kept(vx, tm.x32(vx))) {
    const double u = uniform64(word_of(p.rng, 1u, 0u));
    const double S = sh.sum, E = sh.err, wx = exp(tm.x64(vx));
    const bool bounded = E >= 0 && S - E > 0;
    const double rlo = fmin(1.0, wx / (S + E)) * (1 - 1e-12), rhi = fmin(1.0, wx / (S - E)) * (1 + 1e-12);
    if (bounded && u < rlo) {
      accept = true;
    } else if (!(bounded && u >= rhi)) {
      *why = 9;  // the acceptance needs the exact mass
      return false;
    }
  }
  out->p = accept ? 1.0 : 0.0;
  if (!accept) out->residual = token;
  return true;
}

// ---------------------------------------------------------------------------
// The finishing kernel: one block per row, after the slice pass (the kernel
// boundary makes the slices' summaries and candidates visible). Wave 0 merges
// the slices in slice order and, for a top-k row, finishes it (the row's
// first slice block already checked the per-row metadata); then the block
// routes the row: failed,
// greedy, finished by the wave, the FP64 block list, or the full-row path
// (reference: fused.cuh:803-933 prologue, :1250-1412 list, :1446-1810 full
// row). The row is then committed (verify.cu:169-217 for drafted requests).
template <int DT, bool VEC>
__global__ void __launch_bounds__(BLOCK) es_finish(es_arguments, Plan) {
  using W = typename Ty<DT>::W;
  __shared__ Shared<W> sh;
  __shared__ TopPBins tbins;  // the full-row path's binned top-p boundary
  const es_arguments& a = kernel_args().a;
  const Plan pl = kernel_args().pl;
  // Blocks: one per row (part 0), then pl.helpers per row (parts 1 ...
  // pl.helpers), which take part only in the boundary pass of a binned top-p
  // row and otherwise leave at once, then the request blocks. The request
  // blocks wait on nothing, so the rows' blocks take the device's first slots.
  const int64_t n_helpers = a.rows * pl.helpers;
  if (int64_t(blockIdx.x) >= a.rows + n_helpers) {
    request_block(a, int(int64_t(blockIdx.x) - a.rows - n_helpers));
    return;
  }
  const int64_t hb = int64_t(blockIdx.x) - a.rows;  // >= 0: a helper block
  const int64_t row = hb >= 0 ? hb / pl.helpers : int64_t(blockIdx.x);
  const int part = hb >= 0 ? 1 + int(hb - row * pl.helpers) : 0;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  // One round of loads: the slices' summaries and every candidate slot wave 0
  // may need, then the row's parameters (recorded by its first slice block).
  // The summaries and slots are issued first: they depend on nothing loaded,
  // and issued after the parameters they would wait for them.
  const SlotMap map(min(pl.cap_slice, WAVE * WAVE_BATCH / pl.slices));
  Cand<W> pre[WAVE_BATCH];
  SlicePart q;
  q.max_v = -INFINITY; q.second_v = -INFINITY; q.frontier = -INFINITY; q.tau = -INFINITY;
  q.sum = 0; q.err = 0; q.max_id = INT_MAX; q.second_id = INT_MAX; q.valid = 0; q.n_cand = 0; q.pruned = 0; q.flags = 0;
  if (wave_id() == 0) {
    if (lane < pl.slices) q = slice_parts(a, row)[lane];
    const Cand<W>* cands = candidates<W>(a, row);
#pragma unroll
    for (int r = 0; r < WAVE_BATCH; ++r) {
      const int idx = lane + WAVE * r;
      const int sl = map.slice(idx);
      pre[r] = Cand<W>{};
      if (part == 0 && idx < pl.slices * map.pref) pre[r] = cands[sl * pl.cap_slice + (idx - sl * map.pref)];
    }
  }
  const Params p = *row_meta(a, row);
  if (tid == 0 && part == 0) counters(a, row)->max_key = 0;  // the slices published their maxima; ready for the next call
  if (p.status != ES_OK || p.meta_bad) {
    // Malformed offsets or invalid request metadata: the request block reports it.
    if (part == 0) skip_row(a, row);
    return;
  }
  const int list_max = a.list_max;
  const ListPlan lp = list_plan(p, list_max, pl.cap_slice, a.vocab, pl.slices);
  if (part > 0 && !lp.binned) return;
  const bool sorted_list = lp.sorted_list, need_topp = lp.need_topp;
  const bool stream = a.dispatch != 1 && stream_row(p, a.vocab);  // dispatch 1: the full-row path
  const bool stream_sum = stream && stream_sub(p) == 2u;  // the ratio test needs the kept mass
  if (wave_id() == 0) {
    if (lane < pl.slices) sh.n_cand[lane] = q.n_cand;
    struct T2d { double v1; int i1; double v2; int i2; };
    auto top2d = [](T2d x, T2d y) {
      const bool yw = before(y.v1, y.i1, x.v1, x.i1);
      const T2d w = yw ? y : x, l = yw ? x : y;
      const bool second_l = before(l.v1, l.i1, w.v2, w.i2);
      return T2d{w.v1, w.i1, second_l ? l.v1 : w.v2, second_l ? l.i1 : w.i2};
    };
    // Slices report their maximum only: the runner-up is the best other slice maximum.
    T2d t2{q.max_v, q.max_id, -INFINITY, INT_MAX};
    t2 = wave_all(t2, top2d, T2d{-INFINITY, INT_MAX, -INFINITY, INT_MAX});
    const int vsum = wave_all(q.valid, [](int x, int y) { return x + y; }, 0);
    const int bsum = wave_all(q.flags, [](int x, int y) { return x | y; }, 0);
    // The earliest frontier in (value desc, ID asc) order: every slice is
    // complete down to it.
    struct Fr { double v; int id; };
    Fr fr{lane < pl.slices ? q.frontier : -INFINITY, lane < pl.slices ? q.second_id : INT_MAX};
    fr = wave_all(fr, [](Fr x, Fr o) { return (o.v > x.v || (o.v == x.v && o.id < x.id)) ? o : x; },
                  Fr{-INFINITY, INT_MAX});
    const int nct = wave_all(q.n_cand, [](int x, int y) { return x + y; }, 0);
    // Top-p sums rescaled from slice maxima to the row maximum (FP64).
    // (only top-p lists carry them: need == TOPP_SLICE_NEED in the slices).
    double s_sum = 0, s_err = 0;
    int s_pr = 0;
    if (need_topp || stream_sum) {
      s_pr = q.pruned;
      if (lane < pl.slices && q.valid > 0) {
        const double shift = (t2.v1 - q.max_v) / p.temperature;
        const double scale = exp(-shift);
        if (shift > 700) { s_err = (q.sum + q.err) * scale + q.pruned * SUM_PRUNE_W; s_pr = 0; }
        else { s_sum = q.sum * scale; s_err = (q.err + 4e-16 * q.sum) * scale * (1 + 1e-14); }
      }
      s_sum = wave_all(s_sum, [](double x, double y) { return x + y; }, 0.0);
      s_err = wave_all(s_err, [](double x, double y) { return x + y; }, 0.0);
      s_pr = wave_all(s_pr, [](int x, int y) { return x + y; }, 0);
    }
    if (lane == 0) {
      sh.maximum = t2.v1; sh.greedy = t2.i1; sh.runner_up = t2.v2; sh.runner_up_id = t2.i2;
      sh.valid = vsum; sh.bad = bsum; sh.frontier = fr.v; sh.frontier_id = fr.id; sh.n_cand_total = nct;
      sh.sum = s_sum;
      sh.err = s_err + s_pr * SUM_PRUNE_W + 1e-15 * s_sum;
    }
    if (stream && bsum == 0 && vsum > 0) {
      // The slices' picks, shifted from slice maxima to the row maximum. A
      // slice holds kept tokens when its maximum is kept; its pick counts
      // when the pick itself is kept (exactly, against the row maximum), and
      // otherwise the slice is scanned again below.
      const RowView<DT, VEC> view(a.target, row, int(a.vocab));
      Temp<W> tm;
      tm.init(t2.v1, p.temperature, p.min_p);
      DPick mine = dpick_none();
      bool rescan = false;
      if (lane < pl.slices && q.valid > 0) {
        const W ms = W(q.max_v);
        if (tm.kept(ms, tm.x32(ms))) {
          const Pick sp = *slice_pick<W>(a, row, lane, pl.cap_slice);
          const double shift = (t2.v1 - q.tau) / p.temperature;
          const double eps = 1e-12 * (1.0 + shift + fabs(double(sp.mid)));
          bool take = sp.id != INT_MAX;
          if (take) {
            const W vx = view.value(sp.id);
            take = tm.kept(vx, tm.x32(vx));
            rescan = !take;
          }
          if (take) mine = DPick{double(sp.mid) - shift, double(sp.lo) - shift - eps, double(sp.hi) - shift + eps,
                                 -INFINITY, sp.id};
          if (!rescan) mine.others = double(sp.others) - shift + eps;
        }
      }
      mine = wave_all(mine, dpick_join, dpick_none());
      const unsigned long long again = __ballot(rescan);
      if (lane == 0) {
        sh.sp_mid = mine.mid; sh.sp_lo = mine.lo; sh.sp_hi = mine.hi; sh.sp_others = mine.others;
        sh.sp_id = mine.id; sh.sp_rescan = again;
      }
    }
    // A top-k row is finished here by this wave.
    int wdone = 0;
    RowResult wr{0, 1, -1, -1, ES_OK, ES_OK};
    if (sorted_list && bsum == 0 && vsum > 0) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      wdone = wave_topk(a, row, p, sh, pre, map, pl.slices, pl.cap_slice, q.n_cand, t2.v1, fr.v, fr.id, vsum,
                        &wr);
    }
    if (lane == 0) {
      sh.wdone = wdone;
      sh.wres = wr;
    }
  }
  __syncthreads();
  const int status = sh.bad ? ES_INVALID_INPUT : sh.valid == 0 ? ES_NO_VALID_TOKEN : ES_OK;
  if (part > 0 && status != ES_OK) return;
  if (tid == 0 && part == 0) {
    RowState* st = row_state(a, row);
    st->maximum = sh.maximum; st->runner_up = sh.runner_up; st->greedy = sh.greedy;
    st->runner_up_id = sh.runner_up_id; st->valid = sh.valid; st->status = status;
  }
  RowResult result{0, 1, -1, -1, status, status};
  int fallbacks = 0, route = 0, why = 0;
  if (status != ES_OK) {
    route = 1;
  } else if (p.temperature == 0 && !p.full_q) {
    // Greedy: a point mass at the lowest-ID maximum (reference.py:56-58).
    route = 2;
    result.sample = sh.greedy;
    if (p.verify) {
      const bool accept = p.draft_id == sh.greedy;
      result.p = accept ? 1.0 : 0.0;
      if (!accept) result.residual = sh.greedy;
    }
  } else if (sorted_list && sh.wdone == 1) {
    route = 3;
    result = sh.wres;
  } else {
    bool done = false;
    if (stream) {
      route = 5;
      done = stream_finish<DT, VEC>(a, row, p, pl, sh, &result, &why);
    } else if (sorted_list && sh.wdone < 0) {
      why = 7;  // a rounding the wave could not certify: the full-row path decides
    } else if (lp.binned) {
      why = 10;  // a binned top-p row: the full-row path from the slices' bins
    } else if (p.temperature > 0 && !p.full_q && list_max > 0) {
      const int valid_all = sh.valid;
      const int n_keep = p.top_k > 0 && p.top_k < valid_all ? int(p.top_k) : valid_all;
      const bool topk_list = n_keep <= list_max;
      const bool topp_list = !topk_list && p.top_p < 1 && n_keep == valid_all && p.min_p == 0;
      if (topk_list || topp_list) {
        route = topk_list ? 3 : 4;
        done = list_finish(a, row, p, sh, pl.slices, pl.cap_slice, topk_list, topk_list ? n_keep : 0, &result,
                           &fallbacks, &why);
      }
    }
    if (!done) {
      // The full-row path: the row (and proposal row) read again as needed.
      const double maximum = sh.maximum;
      const int greedy = sh.greedy, runner_up_id = sh.runner_up_id, valid = sh.valid;
      __syncthreads();
      FullRow<DT, VEC> full(a, row, p, sh, pl.groups, &tbins);
      if (lp.binned) {
        int usable = 1;
        for (int sl = 0; sl < pl.slices; ++sl) usable &= sh.n_cand[sl] == TP_COARSE;
        full.bin_slices = usable ? pl.slices : 0;
        full.parts = usable && pl.helpers > 0 ? pl.helpers + 1 : 1;
        full.part = part;
        full.gps = ((pl.groups + pl.helpers) / (pl.helpers + 1) + 1) & ~1;  // an even share: runs stay whole
      }
      if (part > 0 && full.parts == 1) return;  // only a shared boundary pass has helpers
      result = full.run(maximum, greedy, runner_up_id, valid);
      if (!full.finisher) return;  // another of the row's blocks finishes it
      result.target_status = ES_OK;
      fallbacks += full.fallbacks;
      route = 100 + why;  // why the list could not finish it (0: not a list row)
    }
  }
  complete_row(a, row, p, result, fallbacks, route, sh);
  if (tid == 0) add_fallbacks(a, unsigned(fallbacks));
}


}  // namespace es


// ---------------------------------------------------------------------------
// Per-dtype launchers, instantiated in one translation unit per dtype.
namespace es {
template <int DT, bool VEC, int G>
hipError_t launch_main(const es_arguments& a, const Plan& pl, hipStream_t stream, hipEvent_t split) {
  // hipLaunchKernel reports this launch's own error (a stale error of the
  // caller's thread is neither returned nor cleared).
  es_arguments args = a;
  Plan plan = pl;
  void* params[] = {&args, &plan};
  // es_main: the slice blocks; es_finish: one block per row, the request
  // blocks, then `helpers` blocks per row.
  hipError_t err = hipSuccess;
  const void* slice_kernel = pl.tiles > 1 ? reinterpret_cast<const void*>(&es_wide<DT, VEC>)
                                          : reinterpret_cast<const void*>(&es_main<DT, VEC, G>);
  if (a.rows > 0)
    err = hipLaunchKernel(slice_kernel, dim3(unsigned(pl.slice_blocks)), dim3(BLOCK), params, 0, stream);
  if (err == hipSuccess && split) err = hipEventRecord(split, stream);
  if (err != hipSuccess) return err;
  return hipLaunchKernel(reinterpret_cast<const void*>(&es_finish<DT, VEC>),
                         dim3(unsigned(a.rows + pl.req_blocks + a.rows * pl.helpers)), dim3(BLOCK), params, 0,
                         stream);
}

// Contiguous rows aligned to a group of four use vector loads and, for f32
// and bf16, the 16-group tile; any other layout or dtype uses the 4-group tile.
template <int DT>
hipError_t launch_dtype(const es_arguments& a, const Plan& pl, int g, bool vec, hipStream_t stream, hipEvent_t split) {
  if (!vec) return launch_main<DT, false, 4>(a, pl, stream, split);
  if constexpr (DT == ES_F32 || DT == ES_BF16) {
    if (g == 16) return launch_main<DT, true, 16>(a, pl, stream, split);
  }
  return launch_main<DT, true, 4>(a, pl, stream, split);
}
}  // namespace es
