// What the host decides per call and the per-dtype launchers it calls.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exactsample_amd.h"

namespace es {

// Records a HIP error's text for es_last_hip_error (this thread).
void note_hip_error(hipError_t err);

// Launch geometry chosen by the host for a call.
struct Plan {
  int32_t slices;        // blocks per row
  int32_t groups;        // groups of 4 tokens per row
  int32_t gps;           // groups per slice
  int32_t req_blocks;    // request blocks, last in es_finish's grid
  int32_t cap_slice;     // candidates one slice may store
  int32_t slice_blocks;  // rows x slices: es_main's grid
  int32_t tiles;         // register tiles per slice (> 1 only for vocabularies past MAX_SLICES tiles)
  int32_t helpers;       // es_finish blocks per row beyond the first: a binned top-p row's boundary pass,
                         // each of the helpers + 1 blocks taking ceil(slices / (helpers + 1)) slices
  uint32_t generation;   // this call's tag for the published row maxima (never repeats on consecutive calls)
};

// Launches the two kernels of a call for logits of dtype DT with a register
// tile of g groups of four per thread; vec selects vector loads (contiguous,
// aligned rows). A non-null split event is recorded between the kernels.
template <int DT> hipError_t launch_dtype(const es_arguments& a, const Plan& pl, int g, bool vec, hipStream_t stream,
                                          hipEvent_t split);
extern template hipError_t launch_dtype<ES_F32>(const es_arguments&, const Plan&, int, bool, hipStream_t, hipEvent_t);
extern template hipError_t launch_dtype<ES_BF16>(const es_arguments&, const Plan&, int, bool, hipStream_t, hipEvent_t);
extern template hipError_t launch_dtype<ES_F16>(const es_arguments&, const Plan&, int, bool, hipStream_t, hipEvent_t);
extern template hipError_t launch_dtype<ES_F64>(const es_arguments&, const Plan&, int, bool, hipStream_t, hipEvent_t);

}  // namespace es
