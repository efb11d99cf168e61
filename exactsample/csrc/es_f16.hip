// The f16 instantiation of the kernel (one translation unit per dtype builds in parallel).
#include "es_kernel.h"

namespace es {
template hipError_t launch_dtype<ES_F16>(const es_arguments&, const Plan&, int, bool, hipStream_t, hipEvent_t);
}
