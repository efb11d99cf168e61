// Workspace layout of one call. Host and device agree on it; nothing outside
// the library reads it except the FP64 recomputation counter (header word 1).
//
//   [0, 8)            header: int32 malformed-offsets flag, uint32 fallback count
//   8 + r * ROW_BYTES row r's region (ROW_BYTES = 12320, the reference's
//                     32 B RowResult + 12288 B scratch per row, api.h:37-43):
//                     result, state, counters, meta, slice parts, candidates
//
// No byte of the workspace has to hold a particular value when a call starts
// (a fresh, poisoned or half-used workspace all work): every word a call
// reads is written earlier in the same call, the arrival counters are reset
// by the slice pass before the finishing kernel counts on them, and the
// published row maxima carry the call's generation.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace es {

constexpr size_t HEADER_BYTES = 8;
constexpr size_t ROW_SCRATCH = 12288;
constexpr size_t ROW_RESULT_BYTES = 32;
constexpr size_t ROW_BYTES = ROW_RESULT_BYTES + ROW_SCRATCH;
constexpr int MAX_SLICES = 64;

// The outcome of one row, consumed by the request's finalize step.
// p and q encode the ratio decision (p = 1 accepted, 0 rejected; q = 1), so
// finalize's test u < min(1, p / q) reproduces it; sample is the substream-0
// draw (bonus rows, coupled rows), residual the substream-2 draw after a rejection.
struct RowResult {
  double p, q;
  int32_t sample, residual, status, target_status;
};
static_assert(sizeof(RowResult) == ROW_RESULT_BYTES, "RowResult is 32 bytes");

// Which step finished a row in this call.
enum Part : int32_t { PART_SKIP = 0, PART_DONE = 1, PART_FULL = 2 };

// The merged statistics of a row (written by the block that merges it).
struct RowState {
  double maximum;       // largest valid logit
  double runner_up;     // second valid logit in (value desc, id asc) order, -inf if none
  int32_t greedy;       // lowest ID with the largest valid logit
  int32_t runner_up_id; // INT_MAX if none
  int32_t valid;        // allowed tokens with a logit above -inf
  int32_t status;
  int32_t part;
  int32_t fallbacks;    // FP64 recomputations this row needed in this call
  int32_t route;        // how the row was finished (diagnostics)
  int32_t pad;
};
static_assert(sizeof(RowState) == 48, "RowState layout");

// request: rows of the request completed (an arrival counter, kept in the
// request's first row; set to 0 by the slice pass of that row's first slice).
// bound: a binned top-p row's finishing blocks done with their share of the
// boundary pass (set to 0 by the row's first slice).
// max_key: the largest slice maximum published so far in this call, as
// (generation << 32) | FP32 order key of the maximum rounded down; min-p
// slices read it as a lower bound on the row maximum, and a word of another
// generation counts as nothing published.
struct Counters {
  uint32_t request, bound;
  unsigned long long max_key;
};
static_assert(sizeof(Counters) == 16, "Counters layout");

// One slice's summary of its part of the row.
struct SlicePart {
  double max_v;      // largest valid logit in the slice, -inf if none
  double second_v;   // second in (value desc, id asc) order, -inf
  double frontier;   // largest valid logit not stored as a candidate; -inf if none, +inf if unusable
  double tau;        // a stream row's reference maximum: its pick's scores are relative to it
  double sum;        // sum of exp((l - max_v) / T) over kept tokens: FP64 for top-p lists, FP32 for ratio stream rows
  double err;        // a bound on its error (tokens below e^-40 excluded: they are `pruned`)
  int32_t max_id, second_id, valid, n_cand, pruned, flags;
};
static_assert(sizeof(SlicePart) == 72, "SlicePart layout");

// The row's request parameters as the slice pass resolved them (written by
// the row's first slice block, read by the finishing block).
constexpr size_t ROW_META_BYTES = 128;

constexpr size_t OFF_RESULT = 0;
constexpr size_t OFF_STATE = OFF_RESULT + ROW_RESULT_BYTES;
constexpr size_t OFF_COUNTERS = OFF_STATE + sizeof(RowState);
constexpr size_t OFF_META = OFF_COUNTERS + sizeof(Counters);
constexpr size_t OFF_PARTS = OFF_META + ROW_META_BYTES;
constexpr size_t OFF_CAND = OFF_PARTS + MAX_SLICES * sizeof(SlicePart);
constexpr size_t CAND_BYTES = ROW_BYTES - OFF_CAND;
static_assert(OFF_CAND % 16 == 0, "candidate area alignment");

// A stored candidate: value and token ID.
template <class W> struct Cand { W v; int32_t id; };
template <> struct Cand<double> { double v; int32_t id, pad; };
template <class W> constexpr int cand_capacity() { return int(CAND_BYTES / sizeof(Cand<W>)); }

// Binned top-p rows (at most TP_SLICES_MAX slices): slice s keeps TP_COARSE
// FP64 bin masses and TP_COARSE 16-bit counts at the row region's end (its
// bins end TP_SLICE_BIN_BYTES * s bytes before it). Between the used slice
// parts and the bins lies the boundary area of the row's finishing blocks: a
// 32-bit count of gathered tokens, a 32-bit pad, one 24-byte pick per
// finishing block, then either the gathered token IDs (32-bit) or, for a
// boundary range too dense to gather, a bitmap of the runs of TP_RUN tokens
// that hold its tokens (bit r of word w: tokens [TP_RUN (32 w + r), + TP_RUN)).
constexpr int TP_COARSE = 64;
constexpr int TP_RUN = 8;
constexpr size_t TP_SLICE_BIN_BYTES = TP_COARSE * (sizeof(double) + sizeof(uint16_t));
constexpr int TP_SLICES_MAX = int(CAND_BYTES / TP_SLICE_BIN_BYTES);
constexpr size_t TP_PICK_BYTES = 24;
constexpr size_t bound_area_offset(int slices) { return OFF_PARTS + size_t(slices) * sizeof(SlicePart); }
// 32-bit words (token IDs or bitmap words) the boundary area of a row of `slices` slices holds.
constexpr int bound_capacity(int slices) {
  return int((ROW_BYTES - size_t(slices) * TP_SLICE_BIN_BYTES - bound_area_offset(slices) - 8 -
              size_t(slices) * TP_PICK_BYTES) / 4);
}
// Bitmap words of a vocabulary.
constexpr int64_t bound_bitmap_words(int64_t vocab) { return (vocab + 32 * TP_RUN - 1) / (32 * TP_RUN); }
// After the bitmap (at an even word, so 8-byte aligned) and when it fits,
// the fine bins of a dense range that the finishing blocks sum during their
// pass: TP_FINE_SHARED FP64 masses, then as many 32-bit counts.
constexpr int TP_FINE_SHARED = 128;
constexpr int64_t bound_fine_offset(int64_t vocab) { return (bound_bitmap_words(vocab) + 1) & ~int64_t(1); }
constexpr bool bound_fine_fits(int slices, int64_t vocab) {
  return bound_fine_offset(vocab) + 3 * TP_FINE_SHARED <= bound_capacity(slices);
}
static_assert(bound_fine_fits(TP_SLICES_MAX, 151936), "the shared fine bins fit a 151,936-token row at the most slices");
static_assert(bound_capacity(TP_SLICES_MAX) >= 960, "the boundary area holds 960 IDs at the most slices");
static_assert(bound_bitmap_words(int64_t(TP_SLICES_MAX) * 16 * 4 * 256) <= bound_capacity(TP_SLICES_MAX),
              "the bitmap of the largest binned row fits the boundary area");
}  // namespace es
