// Device self-tests of the FP32 arithmetic the certified decisions rely on,
// made on the device with the library's own build flags, since they depend
// on this device's logf / log1pf / __logf / expf:
//
// es_check_gumbel: the FP32 Gumbel noise (gumbel32 and gumbel_upper in
// es_device.h) over any range of 32-bit Philox words, against the FP64 noise
// G(w) = -log(-log u), u = (w + 0.5) / 2^32. The draws assume, for every word,
// |gumbel32(w) - G(w)| <= GUMBEL_ERR (1 + |G|), gumbel_upper(w) >= G(w) and
// G(w) < GUMBEL_MAX (reference: tests/exhaustive/gumbel_bound.cu:1-78 makes
// the same three checks of its CUDA noise), and gumbel_upper(w) <
// GUMBEL_UPPER_MAX (counted with the range violations).
//
// es_check_weights: the FP32 weights of the certified sums (weight32 and
// Temp::x32 in es_device.h): every FP32 x in [-40, 0] against FP64 exp, and
// the formation of x32 = (v - M) * (1 / T) and the combined weight bound on
// pseudo-random (v, M, T) triples (reference: csrc/verify/fused.cuh:62-67,
// whose X_ERR states the same bound for its CUDA expf).
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
    bad_range += !(g < double(GUMBEL_MAX)) || !(gumbel_upper(w) < GUMBEL_UPPER_MAX);
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

// Report words of es_check_weights: 0 indices checked, 1 weight violations
// (|weight32(x) / exp(x) - 1| > X_ERR_EXP over the FP32 x in [-40, 0]),
// 2 formation violations (|x32 - x| > X_ERR_FORM |x| + 2^-126), 3 combined
// violations (|weight32(x32) / exp(x) - 1| > X_ERR (1 + |x|), x in [-40, 0]),
// 4 largest |weight32(x) / exp(x) - 1|, 5 largest |x32 - x| / |x| (|x| >=
// 2^-100), 6 largest combined error / bound (4-6 as FP64 bits, >= 0), 7 FP32
// x values of [-40, 0] checked.
constexpr uint32_t LAST_X_BITS = 0x42200000u;  // 40.0f: indices 0..LAST_X_BITS give -0 .. -40

// A pseudo-random (v, M, T) of index i: M = +-2^[-6, 10), v = fl(M - d) with
// d = 2^[-36, 12), T log-uniform in [2^-10, 2^6] or one of the common values.
__device__ void triple_of(uint64_t i, float* v, float* M, double* T) {
  const Words r = philox(0x5EEDF00DCAFEull, uint32_t(i), uint32_t(i >> 32), 7u, 0u);
  const float fm = 1.f + float(r.w[0] & 0xFFFFFFu) * 0x1p-24f;
  float m = ldexpf(fm, int((r.w[0] >> 24) & 15u) - 6);
  if ((r.w[0] >> 28) & 1u) m = -m;
  if ((r.w[3] & 255u) == 0) m = 0.f;
  const double d = ldexp(1.0 + double(r.w[1] & 0xFFFFFFu) * 0x1p-24, int((r.w[1] >> 24) % 48u) - 36);
  *M = m;
  *v = float(double(m) - d);
  const double common[8] = {1.0, 0.6, 0.7, 0.5, 2.0, 0.9, 1.3, 0.3};
  *T = (r.w[2] & 255u) < 32u ? common[r.w[2] & 7u] : exp2(double(r.w[2] >> 8) * 0x1p-24 * 16.0 - 10.0);
}

__global__ void __launch_bounds__(BLOCK) check_weights(uint64_t first, uint64_t count, uint64_t* report) {
  double worst_exp = 0.0, worst_form = 0.0, worst_comb = 0.0;
  uint64_t n = 0, bad_exp = 0, bad_form = 0, bad_comb = 0, n_exp = 0;
  const uint64_t step = uint64_t(gridDim.x) * BLOCK;
  for (uint64_t k = uint64_t(blockIdx.x) * BLOCK + threadIdx.x; k < count; k += step) {
    const uint64_t i = first + k;
    if (i <= LAST_X_BITS) {
      const float x = __uint_as_float(0x80000000u | uint32_t(i));
      const double e = fabs(double(weight32(x)) / exp(double(x)) - 1.0);
      worst_exp = fmax(worst_exp, e);
      bad_exp += !(e <= X_ERR_EXP);
      ++n_exp;
    }
    float v, M;
    double T;
    triple_of(i, &v, &M, &T);
    Temp<float> tp;
    tp.init(double(M), T, 0.0);
    const float x32 = tp.x32(v);
    const double x = tp.x64(v);
    const double form = fabs(double(x32) - x);
    bad_form += !(form <= X_ERR_FORM * fabs(x) + 0x1p-126);
    if (fabs(x) >= 0x1p-100) worst_form = fmax(worst_form, form / fabs(x));
    if (x >= -40.0) {
      const double r = fabs(double(weight32(x32)) / exp(x) - 1.0) / (double(X_ERR) * (1.0 + fabs(x)));
      worst_comb = fmax(worst_comb, r);
      bad_comb += !(r <= 1.0);
    }
    ++n;
  }
  const auto add = [](uint64_t a, uint64_t b) { return a + b; };
  const auto big = [](double a, double b) { return fmax(a, b); };
  n = wave_all(n, add, uint64_t(0));
  bad_exp = wave_all(bad_exp, add, uint64_t(0));
  bad_form = wave_all(bad_form, add, uint64_t(0));
  bad_comb = wave_all(bad_comb, add, uint64_t(0));
  n_exp = wave_all(n_exp, add, uint64_t(0));
  worst_exp = wave_all(worst_exp, big, 0.0);
  worst_form = wave_all(worst_form, big, 0.0);
  worst_comb = wave_all(worst_comb, big, 0.0);
  if (lane_id() == 0 && n != 0) {
    unsigned long long* rep = reinterpret_cast<unsigned long long*>(report);
    atomicAdd(rep + 0, (unsigned long long)n);
    atomicAdd(rep + 1, (unsigned long long)bad_exp);
    atomicAdd(rep + 2, (unsigned long long)bad_form);
    atomicAdd(rep + 3, (unsigned long long)bad_comb);
    atomicMax(rep + 4, (unsigned long long)__double_as_longlong(worst_exp));
    atomicMax(rep + 5, (unsigned long long)__double_as_longlong(worst_form));
    atomicMax(rep + 6, (unsigned long long)__double_as_longlong(worst_comb));
    atomicAdd(rep + 7, (unsigned long long)n_exp);
  }
}

__global__ void zero_report(uint64_t* report) {
  if (threadIdx.x < REPORT_WORDS) report[threadIdx.x] = 0;
}
}  // namespace

extern "C" int32_t es_check_weights(uint64_t first_index, uint64_t count, uint64_t* report, void* stream) {
  if (!report) return ES_ERR_NULL_ARGUMENT;
  if (first_index > (uint64_t(1) << 32) || count > (uint64_t(1) << 32) - first_index) return ES_ERR_BAD_DIMENSION;
  if (reinterpret_cast<uintptr_t>(report) % 8 != 0) return ES_ERR_WORKSPACE_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* zero_args[] = {&report};
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(&zero_report), dim3(1), dim3(64), zero_args, 0, s);
  if (err == hipSuccess && count != 0) {
    const uint64_t blocks = (count + BLOCK - 1) / BLOCK;
    void* check_args[] = {&first_index, &count, &report};
    err = hipLaunchKernel(reinterpret_cast<const void*>(&check_weights), dim3(unsigned(blocks < 8192 ? blocks : 8192)),
                          dim3(BLOCK), check_args, 0, s);
  }
  if (err != hipSuccess) {
    es::note_hip_error(err);
    return ES_ERR_LAUNCH;
  }
  return ES_SUCCESS;
}

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
