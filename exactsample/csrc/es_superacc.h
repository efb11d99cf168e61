// Exact sums of non-negative doubles in LDS: every term is split into 32-bit
// chunks of its exact value in units of 2^-1074 and added to 64-bit limbs with
// LDS atomics; one wave then propagates carries and rounds to nearest, ties
// to even. The result equals Python's math.fsum (the correctly rounded exact
// sum) of the same terms, in any order. Used only when a double-double sum
// cannot certify its own rounding.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace es {

constexpr int SACC_LIMBS = 40;  // 1280 bits: terms up to 2^80 with 2^31 of them

__device__ __forceinline__ void sacc_clear(unsigned long long* limbs) {
  for (int i = threadIdx.x; i < SACC_LIMBS; i += blockDim.x) limbs[i] = 0;
}

// Adds a finite w >= 0.
__device__ __forceinline__ void sacc_add(unsigned long long* limbs, double w) {
  const uint64_t bits = uint64_t(__double_as_longlong(w));
  const int e = int((bits >> 52) & 0x7ff);
  uint64_t m = bits & ((uint64_t(1) << 52) - 1);
  if (m == 0 && e == 0) return;
  int pos = 0;  // w = m * 2^pos units
  if (e != 0) { m |= uint64_t(1) << 52; pos = e - 1; }
  const int s = pos & 31;
  // Terms are weights <= 1, so pos <= 1022 and limb + 2 < SACC_LIMBS; the clamp
  // only keeps an out-of-contract term inside the array.
  const int limb = min(pos >> 5, SACC_LIMBS - 3);
  const uint32_t c0 = uint32_t(m << s);
  const uint32_t c1 = s ? uint32_t(m >> (32 - s)) : uint32_t(m >> 32);
  const uint32_t c2 = s ? uint32_t(m >> (64 - s)) : 0u;
  if (c0) atomicAdd(&limbs[limb], (unsigned long long)c0);
  if (c1) atomicAdd(&limbs[limb + 1], (unsigned long long)c1);
  if (c2) atomicAdd(&limbs[limb + 2], (unsigned long long)c2);
}

// The correctly rounded sum, computed by one whole wave once the adds are
// visible (every lane calls it and gets the result), without touching the
// limbs: lane i holds limb i,
// carries move up one lane per step until none is left (at most one per limb
// after the first step), and the leading limb, the significand bits and the
// sticky flag are read across lanes.
__device__ __forceinline__ double sacc_round_wave(const unsigned long long* limbs) {
  const int lane = int(__lane_id());
  unsigned long long v = lane < SACC_LIMBS ? limbs[lane] : 0ull;
  while (__ballot((v >> 32) != 0)) {
    const unsigned long long up = __shfl_up(v >> 32, 1u);
    v = (v & 0xffffffffull) + (lane > 0 ? up : 0ull);
    if (lane >= SACC_LIMBS) v = 0;  // beyond the top limb: out of contract, dropped
  }
  const unsigned long long nz = __ballot(v != 0);
  if (!nz) return 0.0;
  auto limb = [&](int i) -> uint64_t { return i < SACC_LIMBS ? uint64_t(__shfl(v, i)) : 0; };
  const int top = 63 - __clzll((long long)nz);
  const int lead = 31 - __clz(uint32_t(limb(top)));
  const int nbits = top * 32 + lead + 1;
  if (nbits <= 53) {
    const uint64_t x = (limb(1) << 32) | limb(0);
    return ldexp(double(x), -1074);
  }
  const int lowbit = nbits - 64 > 0 ? nbits - 64 : 0;
  const int li = lowbit >> 5, sh = lowbit & 31;
  const uint64_t w0 = limb(li), w1 = limb(li + 1), w2 = limb(li + 2);
  const uint64_t lo64 = w0 | (w1 << 32);
  const uint64_t w = sh ? (lo64 >> sh) | (w2 << (64 - sh)) : lo64;
  bool sticky = __ballot(lane < li && v != 0) != 0;  // any set bit below lowbit
  if (sh && (w0 & ((1ull << sh) - 1))) sticky = true;
  const int width = nbits - lowbit;
  const int drop = width - 53;
  uint64_t mant = w >> drop;
  const uint64_t rest = w & ((uint64_t(1) << drop) - 1), half = uint64_t(1) << (drop - 1);
  if (rest > half || (rest == half && (sticky || (mant & 1)))) {
    ++mant;
    if (mant == (uint64_t(1) << 53)) return ldexp(double(mant >> 1), lowbit + drop + 1 - 1074);
  }
  return ldexp(double(mant), lowbit + drop - 1074);
}

}  // namespace es
