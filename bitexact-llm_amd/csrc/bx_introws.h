// Integer rules shared by the row kernels and the element-wise helpers (exact-mode RMSNorm, division, SiLU) and the
// block reductions they use. Every rule restates the reference function it cites.
#pragma once

#include "bx_common.h"

namespace bx {

constexpr int64_t kEps60 = 11529215046068LL;   // round(1e-5 2^60) (src/bitexact/exact/ops.py:21)
constexpr int64_t kNegBig = -(1LL << 20);      // ops.NEG_BIG
constexpr int kQB = 22;                        // |q| <= 2^22

// Block reductions (every thread of the block calls them, sbuf holds 16 entries): wave reductions in DPP and
// LDS-only barriers (a __syncthreads would also wait for every outstanding global load and store); the leading
// barrier keeps a reduction's sbuf writes behind the previous reduction's reads.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ int64_t block_max64(int64_t v, int64_t* sbuf) {
  v = wave_reduce64_dpp<true>(v);
  const int lane = threadIdx.x & 63;
  lds_sync();
  if (lane == 0) sbuf[threadIdx.x >> 6] = v;
  lds_sync();
  return wave_reduce64_dpp<true>(lane < (int)(blockDim.x >> 6) ? sbuf[lane] : INT64_MIN);
}

__device__ __forceinline__ int64_t block_sum64(int64_t v, int64_t* sbuf) {
  v = wave_reduce64_dpp<false>(v);
  const int lane = threadIdx.x & 63;
  lds_sync();
  if (lane == 0) sbuf[threadIdx.x >> 6] = v;
  lds_sync();
  return wave_reduce64_dpp<false>(lane < (int)(blockDim.x >> 6) ? sbuf[lane] : 0);
}

// floor(sqrt(x)) for 0 <= x < 2^62, exact (float estimate, then integer corrections; intops.isqrt's value)
__device__ __forceinline__ int64_t isqrt64(int64_t x) {
  uint64_t s = (uint64_t)sqrt((double)x);
  while (s * s > (uint64_t)x) --s;
  while ((s + 1) * (s + 1) <= (uint64_t)x) ++s;
  return (int64_t)s;
}

// ops.div_round (src/bitexact/exact/ops.py:37-57): round(a 2^p / r) by 28-bit long division, r > 0, rinv =
// 1 / (double) r (every quotient digit is estimated by a multiplication and corrected to the exact floor; a
// caller dividing many values by one r forms rinv once). Digit steps with nothing left to shift (c = 0) add
// floor(R / r) = 0 and are skipped.
//
// Short form: for 0 <= p <= 62, r < 2^34 and |a 2^p / r| < 2^51 the long division never wraps, so its value is
// round-half-up of the exact quotient. The float64 estimate qd (three roundings of relative size 2^-53) is then
// within 1 of floor(a 2^p / r); the remainder a 2^p - q r of that estimate is below 2 r < 2^63 in magnitude, so
// it is exact in wrapping 64-bit arithmetic, and one correction step brings q to the floor.
__device__ __forceinline__ int64_t div_round64(int64_t a, int64_t p, int64_t r, double rinv) {
  if (p >= 0 && p <= 62 && r < (1LL << 34)) {
    const double qd = (double)a * ldexp(1.0, (int)p) * rinv;
    if (qd < 2251799813685248.0 && qd > -2251799813685248.0) {
      int64_t q = (int64_t)floor(qd);
      int64_t rem = (int64_t)(((uint64_t)a << p) - (uint64_t)q * (uint64_t)r);
      if (rem < 0) { --q; rem += r; }
      if (rem >= r) { ++q; rem -= r; }
      return q + (2 * rem >= r ? 1 : 0);
    }
  }
  int64_t Q = fdiv_rcp(a, r, rinv);
  int64_t R = a - Q * r;
  int64_t left = imax(p, 0);
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const int64_t c = imin(left, 28);
    if (c > 0) {
      const int64_t X = shl(R, c);
      const int64_t q1 = fdiv_rcp(X, r, rinv);
      Q = add_wrap(shl(Q, c), q1);
      R = X - q1 * r;
      left -= c;
    }
  }
  const int64_t up = Q + (2 * R >= r ? 1 : 0);
  const int64_t k = imin(imax(-p, 1), 62);
  const int64_t down = add_wrap(Q, 1LL << (k - 1)) >> k;
  return p >= 0 ? up : down;
}

constexpr int64_t kL2E30 = 1549082005LL;   // round(log2(e) 2^30) (ops.L2E30)

// ops.exp2neg_lut(t, lut, 30) given the two table entries a = lut[idx], b = lut[idx + 1] at idx = (t mod 2^26) >> 12
__device__ __forceinline__ int64_t exp2neg30_from(int64_t t, int64_t a, int64_t b) {
  const int64_t n = t >> 26, f = t & ((1LL << 26) - 1);
  const int64_t rr = f & 4095;
  const int64_t v = add_wrap(a, rshc(mul_wrap(b - a, rr), 12));
  return rshc(v, 30 + n);
}

// silu(g) u at 2 FR for one element (ops.silu_mul, src/bitexact/exact/ops.py:119-130), given the two table entries
// la = lut[idx], lb = lut[idx + 1] at silu_index(g); bad |= silu_mul's `not ok`.
__device__ __forceinline__ int silu_index(int64_t g, int FR) {
  const int64_t ga = g < 0 ? (int64_t)(0 - (uint64_t)g) : g;
  const int64_t t = rshc(imin(ga, 64LL << FR) * kL2E30, FR + 4);   // FR + 30 - FT2
  return (int)((t & ((1LL << 26) - 1)) >> 12);
}

__device__ __forceinline__ int64_t silu_elem(int64_t g, int64_t u, int64_t la, int64_t lb, int FR, int& bad) {
  const int64_t ga = g < 0 ? (int64_t)(0 - (uint64_t)g) : g;
  const int64_t E = exp2neg30_from(rshc(imin(ga, 64LL << FR) * kL2E30, FR + 4), la, lb);
  const int64_t den = (1LL << 30) + E;
  const int64_t sig = g >= 0 ? fdiv_fast((1LL << 61) + den, 2 * den) : fdiv_fast(2 * (E << 30) + den, 2 * den);
  const int64_t gc = imin(imax(g, -(1LL << 32)), 1LL << 32);
  const int64_t sv = rshc(mul_wrap(gc, sig), 30);
  const int64_t ua = u < 0 ? (int64_t)(0 - (uint64_t)u) : u;
  const int64_t sa = sv < 0 ? -sv : sv;
  bad |= (bitlen(sa) + bitlen(ua) > 62) | (ga > (1LL << 32));
  return mul_wrap(sv, u);
}

// ops.softmax_w's weight of one visible key (src/bitexact/exact/ops.py:133-143 over exp2neg_lut, 108-116): z =
// max - raw >= 0, zshift = kbits + 3 - sh - FZ, weight at fp bits.
__device__ __forceinline__ int64_t weight64(int64_t z, int64_t zshift, const int64_t* lut, int64_t l2e, int fp) {
  int64_t zf = imin(rshc(z, zshift), 48LL << 26);
  const int64_t t = rshc(mul_wrap(zf, l2e), 28);
  const int64_t n = t >> 26, f = t & ((1LL << 26) - 1);
  const int64_t idx = f >> 12, rr = f & 4095;
  const int64_t a = lut[idx];
  const int64_t v = add_wrap(a, rshc(mul_wrap(lut[idx + 1] - a, rr), 12));
  return rshc(v, 60 - fp + n);
}

}  // namespace bx
