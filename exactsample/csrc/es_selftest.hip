// Device self-test of the FP32 Gumbel noise that the certified draws use
// (gumbel32 and gumbel_upper in es_device.h), over any range of 32-bit Philox
// words, against the FP64 noise G(w) = -log(-log u), u = (w + 0.5) / 2^32.
//
// The draws assume, for every word, |gumbel32(w) - G(w)| <= GUMBEL_ERR (1 + |G|),
// gumbel_upper(w) >= G(w) and G(w) < GUMBEL_MAX. Those depend on this device's
// logf / log1pf / __logf, so they are checked here, on the device, with the
// library's own build flags (reference: tests/exhaustive/gumbel_bound.cu:1-78
// makes the same three checks of its CUDA noise).
#include "es_device.h"
#include "es_plan.h"

namespace {
using namespace es;

// G(w) in FP64; -log u comes from log1p(-(1 - u)) for u >= 1/2, where 1 - u
// is exact from the word's complement, so the tail keeps its precision.
__device__ double noise64(uint32_t w) {
  const double e = w < 0x80000000u ? -log((double(w) + 0.5) * (1.0 / 4294967296.0))
                                   : -log1p(-(double(~w) + 0.5) * (1.0 / 4294967296.0));
  return -log(e);
}

// Report words: 0 words checked, 1 error-bound violations, 2 upper-bound
// violations, 3 range violations, 4 largest error / bound (FP64 bits, >= 0),
// 5 smallest gumbel_upper - G, 6 largest G, 7 smallest G (5-7 as order keys).
constexpr int REPORT_WORDS = 8;

__global__ void reset_report(uint64_t* report) {
  const int i = int(threadIdx.x);
  if (i < REPORT_WORDS) report[i] = (i == 5 || i == 7) ? ~uint64_t(0) : uint64_t(0);
}

__global__ void __launch_bounds__(BLOCK) check_noise(uint64_t first, uint64_t count, uint64_t* report) {
  double worst = 0.0, slack = INFINITY, hi = -INFINITY, lo = INFINITY;
  uint64_t n = 0, bad_err = 0, bad_upper = 0, bad_range = 0;
  const uint64_t step = uint64_t(gridDim.x) * BLOCK;
  for (uint64_t i = uint64_t(blockIdx.x) * BLOCK + threadIdx.x; i < count; i += step) {
    const uint32_t w = uint32_t(first + i);
    const double g = noise64(w);
    const double ratio = fabs(double(gumbel32(w)) - g) / (double(GUMBEL_ERR) * (1.0 + fabs(g)));
    const double margin = double(gumbel_upper(w)) - g;
    worst = fmax(worst, ratio);
    slack = fmin(slack, margin);
    hi = fmax(hi, g);
    lo = fmin(lo, g);
    bad_err += ratio > 1.0;
    bad_upper += margin < 0.0;
    bad_range += !(g < double(GUMBEL_MAX));
    ++n;
  }
  const auto add = [](uint64_t x, uint64_t y) { return x + y; };
  const auto big = [](double x, double y) { return fmax(x, y); };
  const auto small = [](double x, double y) { return fmin(x, y); };
  n = wave_all(n, add, uint64_t(0));
  bad_err = wave_all(bad_err, add, uint64_t(0));
  bad_upper = wave_all(bad_upper, add, uint64_t(0));
  bad_range = wave_all(bad_range, add, uint64_t(0));
  worst = wave_all(worst, big, 0.0);
  slack = wave_all(slack, small, double(INFINITY));
  hi = wave_all(hi, big, -double(INFINITY));
  lo = wave_all(lo, small, double(INFINITY));
  if (lane_id() == 0 && n != 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(report + 0), (unsigned long long)n);
    atomicAdd(reinterpret_cast<unsigned long long*>(report + 1), (unsigned long long)bad_err);
    atomicAdd(reinterpret_cast<unsigned long long*>(report + 2), (unsigned long long)bad_upper);
    atomicAdd(reinterpret_cast<unsigned long long*>(report + 3), (unsigned long long)bad_range);
    atomicMax(reinterpret_cast<unsigned long long*>(report + 4), (unsigned long long)__double_as_longlong(worst));
    atomicMin(reinterpret_cast<unsigned long long*>(report + 5), (unsigned long long)order_key(slack));
    atomicMax(reinterpret_cast<unsigned long long*>(report + 6), (unsigned long long)order_key(hi));
    atomicMin(reinterpret_cast<unsigned long long*>(report + 7), (unsigned long long)order_key(lo));
  }
}
}  // namespace

extern "C" int32_t es_check_gumbel(uint64_t first_word, uint64_t count, uint64_t* report, void* stream) {
  if (!report) return ES_ERR_NULL_ARGUMENT;
  if (first_word > (uint64_t(1) << 32) || count > (uint64_t(1) << 32) - first_word) return ES_ERR_BAD_DIMENSION;
  if (reinterpret_cast<uintptr_t>(report) % 8 != 0) return ES_ERR_WORKSPACE_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* reset_args[] = {&report};
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(&reset_report), dim3(1), dim3(64), reset_args, 0, s);
  if (err == hipSuccess && count != 0) {
    const uint64_t blocks = (count + BLOCK - 1) / BLOCK;
    void* check_args[] = {&first_word, &count, &report};
    err = hipLaunchKernel(reinterpret_cast<const void*>(&check_noise), dim3(unsigned(blocks < 4096 ? blocks : 4096)),
                          dim3(BLOCK), check_args, 0, s);
  }
  if (err != hipSuccess) {
    es::note_hip_error(err);
    return ES_ERR_LAUNCH;
  }
  return ES_SUCCESS;
}
