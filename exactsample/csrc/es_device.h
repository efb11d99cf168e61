// Device primitives for the gfx950 sampling path: 64-lane wave reductions,
// block reductions in a fixed order, Philox4x32-10, order-preserving keys,
// double-double sums and the FP32 Gumbel noise with its certified bound.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include "exactsample_amd.h"

namespace es {

constexpr int WAVE = 64;
constexpr int BLOCK = 256;            // every kernel runs 4 waves of 64 lanes
constexpr int WAVES = BLOCK / WAVE;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / WAVE; }

// ---------------------------------------------------------------------------
// Cross-lane exchange. __shfl_xor over the full 64-lane wave.
__device__ __forceinline__ float xshfl(float v, int m) { return __shfl_xor(v, m, WAVE); }
__device__ __forceinline__ double xshfl(double v, int m) { return __shfl_xor(v, m, WAVE); }
__device__ __forceinline__ int xshfl(int v, int m) { return __shfl_xor(v, m, WAVE); }
__device__ __forceinline__ unsigned xshfl(unsigned v, int m) { return __shfl_xor(v, m, WAVE); }
__device__ __forceinline__ uint64_t xshfl(uint64_t v, int m) {
  return (uint64_t(__shfl_xor(unsigned(v >> 32), m, WAVE)) << 32) | __shfl_xor(unsigned(v), m, WAVE);
}

// ---------------------------------------------------------------------------
// Wave scans and reductions on DPP lane moves. A __shfl lowers to
// ds_bpermute, an LDS round trip per step; the DPP row shifts and row
// broadcasts below cost a few cycles each. They need every lane of the wave
// active (all callers run them in wave-uniform control flow).
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143;

// Lane i receives x from its DPP source lane; lanes whose source lies outside
// their row, or whose row is not in ROWS, receive `fill`.
template <int CTRL, int ROWS, class T> __device__ __forceinline__ T dpp_move(T x, T fill) {
  static_assert(sizeof(T) % 4 == 0, "32-bit words");
  constexpr int N = int(sizeof(T) / 4);
  int a[N], f[N];
  __builtin_memcpy(a, &x, sizeof(T));
  __builtin_memcpy(f, &fill, sizeof(T));
#pragma unroll
  for (int k = 0; k < N; ++k) a[k] = __builtin_amdgcn_update_dpp(f[k], a[k], CTRL, ROWS, 0xF, false);
  T r;
  __builtin_memcpy(&r, a, sizeof(T));
  return r;
}

// The value of lane `src` (wave-uniform) in every lane.
template <class T> __device__ __forceinline__ T lane_read(T x, int src) {
  static_assert(sizeof(T) % 4 == 0, "32-bit words");
  constexpr int N = int(sizeof(T) / 4);
  int a[N];
  __builtin_memcpy(a, &x, sizeof(T));
#pragma unroll
  for (int k = 0; k < N; ++k) a[k] = __builtin_amdgcn_readlane(a[k], src);
  T r;
  __builtin_memcpy(&r, a, sizeof(T));
  return r;
}

// Inclusive scan in lane order: lane i gets op(... op(op(x0, x1), x2) ..., xi)
// up to the grouping of the steps. `identity` must satisfy op(identity, x) == x.
template <class T, class Op> __device__ __forceinline__ T wave_scan(T x, Op op, T identity) {
  x = op(dpp_move<DPP_ROW_SHR1, 0xF>(x, identity), x);
  x = op(dpp_move<DPP_ROW_SHR2, 0xF>(x, identity), x);
  x = op(dpp_move<DPP_ROW_SHR4, 0xF>(x, identity), x);
  x = op(dpp_move<DPP_ROW_SHR8, 0xF>(x, identity), x);
  x = op(dpp_move<DPP_ROW_BCAST15, 0xA>(x, identity), x);  // rows 1 and 3 take the row before's last lane
  x = op(dpp_move<DPP_ROW_BCAST31, 0xC>(x, identity), x);  // rows 2 and 3 take lane 31
  return x;
}

// op over all 64 lanes, the same value in every lane (lane 63's scan).
template <class T, class Op> __device__ __forceinline__ T wave_all(T v, Op op, T identity) {
  return lane_read(wave_scan(v, op, identity), WAVE - 1);
}

// op over the block, combined across waves in wave order; every thread gets it.
// `scratch` holds WAVES entries and may be reused right after the call.
template <class T, class Op> __device__ __forceinline__ T block_all(T v, Op op, T* scratch, T identity) {
  v = wave_all(v, op, identity);
  __syncthreads();
  if (lane_id() == 0) scratch[wave_id()] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) r = op(r, scratch[w]);
  return r;
}

// Inclusive prefix sum over the wave in lane order.
template <class T> __device__ __forceinline__ T wave_scan_add(T v) {
  return wave_scan(v, [](T x, T y) { return x + y; }, T(0));
}

// The j-th largest (1-based) of the wave's 64 unsigned keys, by a bitwise
// search on ballots (no cross-lane data movement).
template <class K> __device__ __forceinline__ K wave_kth_largest(K key, int j) {
  K prefix = 0;
#pragma unroll
  for (int b = int(sizeof(K) * 8) - 1; b >= 0; --b) {
    const K cand = prefix | (K(1) << b);
    if (__popcll(__ballot(key >= cand)) >= j) prefix = cand;
  }
  return prefix;
}

// Inclusive prefix sum over the block in thread order; *total receives the sum.
__device__ __forceinline__ int block_scan_add(int v, int* scratch, int* total) {
  int incl = wave_scan_add(v);
  __syncthreads();
  if (lane_id() == WAVE - 1) scratch[wave_id()] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    const int s = scratch[w];
    before += w < wave_id() ? s : 0;
    all += s;
  }
  *total = all;
  return incl + before;
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Random123), counter = (stream, position, substream, token/4),
// key = (seed lo, seed hi). Contract: docs/rng.md:1-28 of the reference.
struct Words { uint32_t w[4]; };

__host__ __device__ __forceinline__ Words philox(uint64_t seed, uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3) {
  uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = uint64_t(0xD2511F53u) * c0;
    const uint64_t p1 = uint64_t(0xCD9E8D57u) * c2;
    const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
    c1 = uint32_t(p1);
    c3 = uint32_t(p0);
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return Words{{c0, c1, c2, c3}};
}

struct RngAddr { uint64_t seed; uint32_t stream, position; };

__device__ __forceinline__ uint32_t word_of(const RngAddr& r, uint32_t sub, uint32_t token) {
  const Words w = philox(r.seed, r.stream, r.position, sub, token >> 2);
  const uint32_t lane = token & 3u;
  return lane == 0 ? w.w[0] : lane == 1 ? w.w[1] : lane == 2 ? w.w[2] : w.w[3];
}

// u = (w + 0.5) / 2^32, exact in FP64 (docs/rng.md:17-19).
__host__ __device__ __forceinline__ double uniform64(uint32_t w) { return (double(w) + 0.5) * (1.0 / 4294967296.0); }

// The oracle's noise: -log(-log(u)) in FP64.
__device__ __forceinline__ double gumbel64(uint32_t w) { return -log(-log(uniform64(w))); }

// FP32 noise. -log(u) comes from log(u) for u < 1/2 and from log1p(-(1-u)) for
// u >= 1/2, with 1-u formed from the complement of the word, so the large-noise
// tail keeps the word's full resolution. Its distance from the FP64 value is at
// most GUMBEL_ERR * (1 + |G|) for every 32-bit word (checked exhaustively on the
// device by tests/test_gumbel_bound.py).
constexpr float GUMBEL_ERR = 1.9073486e-06f;  // 2^-19
constexpr float GUMBEL_MAX = 22.875f;          // above the largest noise, 22.87386
__device__ __forceinline__ float gumbel32(uint32_t w) {
  const float e = w < 0x80000000u ? -logf((float(w) + 0.5f) * 2.3283064365386963e-10f)
                                  : -log1pf(-(float(~w) + 0.5f) * 2.3283064365386963e-10f);
  return -logf(e);
}
// A cheap upper bound on the same noise, one native log: for w < 2^31, u <
// 1/2, so -log(u) > log 2 and G < -log(log 2) = 0.366513 < 0.3666; otherwise
// -log(u) >= 1 - u, with the native base-2 log and a relative margin. Checked
// to bound G, and to stay below 23, for every word.
__device__ __forceinline__ float gumbel_upper(uint32_t w) {
  const float e = (float(~w) + 0.5f) * 2.3283064365386963e-10f;
  const float g = -__logf(e * (1.f - 4e-6f));
  return w < 0x80000000u ? 0.3666f : g + 4e-6f * (1.f + fabsf(g));
}
constexpr float GUMBEL_UPPER_MAX = 23.f;  // gumbel_upper(w) < GUMBEL_UPPER_MAX for every word

// ---------------------------------------------------------------------------
// Temperature arithmetic and FP32 weights, with the bounds the certified
// decisions use (checked on the device by es_check_weights):
//  - formation: |x32 - x| <= X_ERR_FORM |x| + 2^-126 for x32 = Temp::x32(v)
//    and the oracle's x = (l - max) / T in FP64 (three FP32 roundings: the
//    difference, 1 / T and the product, each within 2^-24);
//  - weights: |weight32(x) / exp(x) - 1| <= X_ERR_EXP for every FP32 x in
//    [-40, 0] (all 1.1e9 of them);
//  - together: |weight32(x32) / exp(x) - 1| <= X_ERR (1 + |x|), since
//    X_ERR_EXP + 1.0001 X_ERR_FORM |x| <= X_ERR (1 + |x|).
constexpr float X_ERR = 4.8e-7f;        // |x32 - x| <= X_ERR * |x|; |w32/w - 1| <= X_ERR * (1 + |x|)
constexpr double X_ERR_FORM = 1.8e-7;   // 3 * 2^-24, rounded up
constexpr double X_ERR_EXP = 2.9e-7;    // X_ERR - X_ERR_FORM, rounded down

// The FP32 weight of an FP32 x (the library's expf, as every FP32 sum uses it).
__device__ __forceinline__ float weight32(float x) { return expf(x); }

// ---------------------------------------------------------------------------
// Unsigned keys in value order; -0 and +0 get the same key (the oracle compares
// values, and -0 == +0).
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ uint64_t order_key(double v) {
  const uint64_t b = uint64_t(__double_as_longlong(v == 0.0 ? 0.0 : v));
  return (b >> 63) ? ~b : (b | (uint64_t(1) << 63));
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
__device__ __forceinline__ double key_value(uint64_t k) {
  return __longlong_as_double((long long)((k >> 63) ? (k & ~(uint64_t(1) << 63)) : ~k));
}

// (value desc, id asc): does a come before b?
template <class W> __device__ __forceinline__ bool before(W av, int ai, W bv, int bi) {
  return av > bv || (av == bv && ai < bi);
}

// ---------------------------------------------------------------------------
// Double-double arithmetic for exact-looking FP64 sums.
struct DD { double hi, lo; };
__device__ __forceinline__ DD dd_add(DD a, DD b) {
  const double s = a.hi + b.hi;
  const double v = s - a.hi;
  const double e = (a.hi - (s - v)) + (b.hi - v);
  const double lo = (a.lo + b.lo) + e;
  const double hi = s + lo;
  return DD{hi, lo - (hi - s)};
}
__device__ __forceinline__ DD xshfl(DD d, int m) { return DD{xshfl(d.hi, m), xshfl(d.lo, m)}; }

// The correctly rounded value of a non-negative DD sum whose exact value lies
// within `err` of hi + lo, if that is certain. Returns false when the exact sum
// may round to a neighbour (then the caller computes it exactly).
__device__ __forceinline__ bool dd_round_certain(DD s, double err, double* out) {
  const double hi = s.hi;
  if (!(hi > 0) || !isfinite(hi)) { *out = hi; return hi == 0 && err == 0; }
  const double up = nextafter(hi, INFINITY) - hi;
  const double down = hi - nextafter(hi, 0.0);
  const bool ok = s.lo + err < 0.5 * up && s.lo - err > -0.5 * down;
  *out = hi;
  return ok;
}

// Relative error bound of a DD sum of n non-negative terms formed by dd_add in any
// order, plus an absolute allowance for terms near the subnormal range.
__device__ __forceinline__ double dd_sum_error(DD s, double n) {
  return n * 0x1p-100 * s.hi + n * 0x1p-1060;
}

// Temperature arithmetic shared by the slice pass, the list and the full-row
// parts.
template <class W> struct Temp {
  double M, T, min_p;
  float inv_t, ln_min_p, min_p_tol;
  bool slow;
  __device__ __forceinline__ void init(double maximum, double temperature, double min_p_) {
    M = maximum; T = temperature; min_p = min_p_;
    inv_t = float(1.0 / temperature);
    slow = !(inv_t < 1e30f);
    ln_min_p = min_p > 0 ? float(log(min_p)) : -INFINITY;
    min_p_tol = min_p > 0 ? 1e-6f * (1.f + fabsf(ln_min_p)) : 0.f;
  }
  // The oracle's x = (l - max) / T in FP64 (reference.py:63).
  __device__ __forceinline__ double x64(W v) const { return (double(v) - M) / T; }
  // FP32 x with |x32 - x| <= X_ERR_FORM * |x| + 2^-126; SLOW: 1 / T is out
  // of FP32 range (`slow`), so the difference is divided in FP64. Loops that
  // run per token choose the form once (x32_as), so no token pays for the
  // FP64 divide.
  template <bool SLOW> __device__ __forceinline__ float x32_as(W v) const {
    if constexpr (sizeof(W) == 8) {
      return float(x64(v));
    } else {
      const float d = v - float(M);
      if constexpr (SLOW) return float(double(d) / T);
      else return d * inv_t;
    }
  }
  __device__ __forceinline__ float x32(W v) const { return slow ? x32_as<true>(v) : x32_as<false>(v); }
  // exp(x) >= min_p and exp(x) > 0 for the FP64 x, settled in FP32 when x is
  // clear of both thresholds and in FP64 otherwise. The margin X_ERR |x| +
  // min_p_tol covers x32's formation error and ln_min_p's rounding.
  __device__ __forceinline__ bool kept(W v, float x) const {
    if (x > -744.f && fabsf(x - ln_min_p) > X_ERR * fabsf(x) + min_p_tol) return x > ln_min_p;
    if (x < -745.2f) return false;
    const double w = exp(x64(v));
    return w > 0 && w >= min_p;
  }
};

}  // namespace es
