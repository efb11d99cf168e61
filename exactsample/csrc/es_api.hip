// Host side of exactsample_amd: launch geometry, dtype dispatch and the C ABI
// (include/exactsample_amd.h).
#include <limits.h>
#include <algorithm>
#include <atomic>
#include <mutex>
#include <stdio.h>
#include "es_layout.h"
#include "es_plan.h"

namespace {
constexpr int kBlock = 256;  // threads per block of the kernel
constexpr int64_t kFinishSlots = 512;  // es_finish blocks resident at once on MI355X: 256 CUs x 2
thread_local char g_last_hip_error[256] = "";
thread_local hipEvent_t g_split_event = nullptr;
std::atomic<uint32_t> g_generation{0};

// A tag for the row maxima a call publishes in its workspace: consecutive
// calls get different tags, and 0 (a zeroed word) is never one.
uint32_t next_generation() {
  uint32_t g = g_generation.fetch_add(1, std::memory_order_relaxed) + 1;
  if (g == 0) g = g_generation.fetch_add(1, std::memory_order_relaxed) + 1;
  return g;
}

constexpr int64_t elem_size(int dt) { return dt == ES_F64 ? 8 : dt == ES_F32 ? 4 : 2; }

// Rows contiguous and aligned to a group of four elements (target and draft).
bool vectorizable_matrix(const es_arguments& a, const es_matrix& m) {
  const int64_t es = elem_size(m.dtype);
  return !m.data || (m.s1 == 1 && a.vocab % 4 == 0 && (m.s0 * es) % (4 * es) == 0 &&
                     reinterpret_cast<uintptr_t>(m.data) % uintptr_t(4 * es) == 0);
}
template <int DT> bool vectorizable(const es_arguments& a) {
  return vectorizable_matrix(a, a.target) && vectorizable_matrix(a, a.draft);
}

// Per-thread register tile (groups of four) and slices per row. For lists
// (top-k, top-p) the largest tile wins at every batch size measured (1 to 320
// rows of V = 151,936): more, smaller slices cost more in the finishing
// kernel's merge than they gain in parallelism. A call whose caller promises
// no list rows (list_max 0) and that would not fill the device's CUs with
// 16-group slices takes the 4-group tile: streaming draws then spread their
// Philox work over four times the blocks. Strided rows, f16 and f64 always
// use the 4-group tile.
struct Geometry { int g, slices; };
Geometry choose_geometry(int64_t rows, int64_t groups, bool large_tiles, int32_t list_max) {
  auto slices_of = [&](int g) { return int((groups + int64_t(g) * kBlock - 1) / (int64_t(g) * kBlock)); };
  const int s16 = slices_of(16);
  const int g = large_tiles && (list_max > 0 || rows * s16 >= 256) ? 16 : 4;
  return Geometry{g, slices_of(g)};
}

}  // namespace

void es::note_hip_error(hipError_t err) {
  snprintf(g_last_hip_error, sizeof(g_last_hip_error), "%s", hipGetErrorString(err));
}

extern "C" {

size_t es_workspace_size(int64_t rows, int64_t vocab, int32_t reference) {
  if (rows < 0 || vocab < 0) return 0;
  const unsigned __int128 scratch = reference ? (unsigned __int128)vocab * 20u : 0u;
  const unsigned __int128 per = es::ROW_RESULT_BYTES + (scratch > es::ROW_SCRATCH ? scratch : es::ROW_SCRATCH);
  const unsigned __int128 total = es::HEADER_BYTES + (unsigned __int128)rows * per;
  if (total > (unsigned __int128)SIZE_MAX) return 0;
  return size_t(total);
}

size_t es_fallback_counter_offset(void) { return 4; }

const char* es_error_string(int32_t code) {
  switch (code) {
    case ES_SUCCESS: return "success";
    case ES_ERR_NULL_ARGUMENT: return "a required pointer argument is null";
    case ES_ERR_BAD_DIMENSION: return "rows, requests, vocab or max_draft out of the supported range";
    case ES_ERR_BAD_OPTION: return "mode, dispatch or list_max out of range";
    case ES_ERR_WORKSPACE_SIZE: return "workspace capacity exceeded";
    case ES_ERR_WORKSPACE_ALIGN: return "workspace alignment must be 8 bytes";
    case ES_ERR_BAD_DTYPE: return "unsupported logits dtype (draft logits must match the target dtype)";
    case ES_ERR_LAUNCH: return "exactsample kernel launch failed";
    case ES_ERR_STATIC_CAPACITY:
      return "the call needs more than the library's static workspace (ES_STATIC_WORKSPACE_BYTES: 8 + rows x 12320 bytes)";
    default: return "unknown exactsample_amd error";
  }
}

const char* es_last_hip_error(void) { return g_last_hip_error; }

void es_set_split_event(void* event) { g_split_event = static_cast<hipEvent_t>(event); }

}  // extern "C"

namespace {

// es_launch's checks and launches. With `own_workspace` the workspace is the
// library's static array (set by the caller), so the caller's workspace
// fields are neither required nor checked.
int32_t launch_call(const es_arguments& a, void* stream_ptr, bool own_workspace) {
  g_last_hip_error[0] = 0;
  if (a.requests < 0 || a.rows < 0 || a.vocab <= 0 || a.vocab > INT32_MAX || a.rows > 65535 ||
      a.requests > INT32_MAX || a.max_draft < 0 || a.max_draft >= INT32_MAX)
    return ES_ERR_BAD_DIMENSION;
  if (a.requests == 0 && a.rows != 0) return ES_ERR_BAD_DIMENSION;
  if (a.mode < 0 || a.mode > 1 || a.dispatch < 0 || a.dispatch > 2 || a.list_max < 0 || a.list_max > 256)
    return ES_ERR_BAD_OPTION;
  if (a.requests == 0) return ES_SUCCESS;
  if (!a.target.data && a.rows > 0) return ES_ERR_NULL_ARGUMENT;
  if (!a.cu_rows.data || !a.top_k.data || !a.draft_kind.data || !a.seed.data || !a.stream.data ||
      !a.temperature.data || !a.top_p.data || !a.min_p.data || (!a.draft_ids && a.max_draft > 0) ||
      !a.tokens || !a.accepted ||
      !a.status || !a.path || !a.workspace || (!a.position.data && a.rows > 0))
    return ES_ERR_NULL_ARGUMENT;
  if (a.target.dtype < ES_F32 || a.target.dtype > ES_BF16) return ES_ERR_BAD_DTYPE;
  if (a.draft.data && a.draft.dtype != a.target.dtype) return ES_ERR_BAD_DTYPE;
  if (!own_workspace) {
    const size_t need = es_workspace_size(a.rows, a.vocab, a.dispatch == 1);
    if (need == 0 || a.workspace_bytes < need) return ES_ERR_WORKSPACE_SIZE;
    if (reinterpret_cast<uintptr_t>(a.workspace) % 8 != 0) return ES_ERR_WORKSPACE_ALIGN;
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  // dispatch 1 ("reference"): every row is finished on the exact full-row
  // path, so the slices gather no list candidates.
  es_arguments run = a;
  if (a.dispatch == 1) run.list_max = 0;
  const int64_t groups = (a.vocab + 3) / 4;
  const bool large_tiles = (a.target.dtype == ES_F32 || a.target.dtype == ES_BF16) &&
                           vectorizable_matrix(a, a.target) && vectorizable_matrix(a, a.draft);
  const Geometry geo = choose_geometry(a.rows, groups, large_tiles, run.list_max);
  es::Plan pl{};
  pl.groups = int(groups);
  pl.req_blocks = int((a.requests + kBlock - 1) / kBlock);
  // A vocabulary needing more than MAX_SLICES tiles gives each slice several
  // tiles (read group by group) and stores no list candidates.
  int64_t tiles = 1, slices = geo.slices;
  if (slices > es::MAX_SLICES) {
    tiles = (slices + es::MAX_SLICES - 1) / es::MAX_SLICES;
    const int64_t span = tiles * geo.g * kBlock;
    slices = (groups + span - 1) / span;
    run.list_max = 0;
  }
  if (a.rows == 0) {
    pl.slices = 1;
    pl.gps = int(groups);
    pl.tiles = 1;
  } else {
    pl.slices = int(slices);
    pl.gps = int(tiles * geo.g * kBlock);  // every slice but the last is exactly `tiles` tiles
    pl.tiles = int(tiles);
  }
  const int cap_total = a.target.dtype == ES_F64 ? es::cand_capacity<double>() : es::cand_capacity<float>();
  pl.cap_slice = cap_total / pl.slices;
  pl.slice_blocks = int(a.rows * pl.slices);
  // A binned top-p row (list rows only) has its boundary pass shared by
  // `parts` finishing blocks, each taking an equal share of its groups; the blocks of other
  // rows exit at once. About one round of the device's resident finishing
  // blocks (two per CU) for the call, at least two per row.
  pl.helpers = 0;
  if (run.list_max > 0 && pl.tiles == 1 && pl.slices > 1 && pl.slices <= es::TP_SLICES_MAX) {
    const int64_t parts = std::min<int64_t>(pl.slices, std::max<int64_t>(2, (kFinishSlots + a.rows - 1) / a.rows));
    pl.helpers = int(parts - 1);
  }
  pl.generation = next_generation();
  hipError_t err = hipSuccess;
  switch (a.target.dtype) {
    case ES_F32: err = es::launch_dtype<ES_F32>(run, pl, geo.g, vectorizable<ES_F32>(a), stream, g_split_event); break;
    case ES_F64: err = es::launch_dtype<ES_F64>(run, pl, geo.g, vectorizable<ES_F64>(a), stream, g_split_event); break;
    case ES_F16: err = es::launch_dtype<ES_F16>(run, pl, geo.g, vectorizable<ES_F16>(a), stream, g_split_event); break;
    default: err = es::launch_dtype<ES_BF16>(run, pl, geo.g, vectorizable<ES_BF16>(a), stream, g_split_event); break;
  }
  if (err != hipSuccess) {
    es::note_hip_error(err);
    return ES_ERR_LAUNCH;
  }
  return ES_SUCCESS;
}

// The workspace of es_launch_static: one copy per GPU, held until the process
// ends. Host code never uses this name as an address (on the host it is a
// stand-in); the device address of each GPU's copy comes from
// hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) uint8_t scratch[ES_STATIC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (looked up on the device's first call).
int32_t scratch_of_current_device(uint8_t** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) {
    es::note_hip_error(err);
    return ES_ERR_LAUNCH;
  }
  if (device < 0 || device >= kMaxDevices) return ES_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      es::note_hip_error(err);
      return ES_ERR_LAUNCH;
    }
    g_scratch_ptr[device] = static_cast<uint8_t*>(ptr);
  }
  *out = g_scratch_ptr[device];
  return ES_SUCCESS;
}

}  // namespace

extern "C" {

int32_t es_launch(const es_arguments* args, void* stream_ptr) {
  if (!args) return ES_ERR_NULL_ARGUMENT;
  return launch_call(*args, stream_ptr, false);
}

int32_t es_launch_static(const es_arguments* args, void* stream_ptr) {
  if (!args) return ES_ERR_NULL_ARGUMENT;
  // The rows' regions, whatever the dispatch: the kernels use 8 + rows * 12,320 bytes.
  const size_t need = es_workspace_size(args->rows, args->vocab, 0);
  if (args->rows < 0 || args->vocab <= 0 || need == 0) return ES_ERR_BAD_DIMENSION;
  if (need > ES_STATIC_WORKSPACE_BYTES) return ES_ERR_STATIC_CAPACITY;
  es_arguments run = *args;
  const int32_t found = scratch_of_current_device(&run.workspace);
  if (found != ES_SUCCESS) return found;
  run.workspace_bytes = ES_STATIC_WORKSPACE_BYTES;
  return launch_call(run, stream_ptr, true);
}

}  // extern "C"
