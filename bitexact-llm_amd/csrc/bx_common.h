// Shared device code for the bitexact HIP library (gfx950 / MI355X).
//
// Integer rules follow the reference's torch int64 semantics exactly: two's complement wrap (the library is
// built with -fwrapv and wrapping sums are done in uint64), `<<` by >= 64 gives 0, `>>` by >= 64 gives the
// sign. Every helper cites the reference rule it restates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bitexact_hip.h"

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

namespace bx {

constexpr int64_t kLim3 = 8355711;     // 3 signed base-256 digits (src/bitexact/intops.py:11)
constexpr int64_t kNeg = -(1LL << 62);  // masked score (src/bitexact/exact/ops.py:138)

// ---- host-side error plumbing ----
void set_error(const char* fmt, ...);
int check_launch(const char* what);
int device_cus();   // compute units of the current device (cached per device)

// ---- shifts with torch's CPU semantics ----
__device__ __forceinline__ int64_t shl(int64_t x, int64_t s) {   // s >= 0
  return s >= 64 ? 0 : (int64_t)((uint64_t)x << s);
}
__device__ __forceinline__ int64_t sar(int64_t x, int64_t s) {   // s >= 0
  return x >> (s > 63 ? 63 : s);
}
__device__ __forceinline__ int64_t add_wrap(int64_t a, int64_t b) {
  return (int64_t)((uint64_t)a + (uint64_t)b);
}
__device__ __forceinline__ int64_t mul_wrap(int64_t a, int64_t b) {
  return (int64_t)((uint64_t)a * (uint64_t)b);
}
__device__ __forceinline__ int64_t imin(int64_t a, int64_t b) { return a < b ? a : b; }
__device__ __forceinline__ int64_t imax(int64_t a, int64_t b) { return a > b ? a : b; }

// ops.rshc (src/bitexact/exact/ops.py:25-34): round(x / 2^s), s clamped to [-62, 62].
__device__ __forceinline__ int64_t rshc(int64_t x, int64_t s) {
  s = imin(imax(s, -62), 62);
  if (s > 0) return add_wrap(x, 1LL << (s - 1)) >> s;
  return shl(x, -s);
}

// intops.rsh (src/bitexact/intops.py:24-33): round(x / 2^s) ties up for s > 0, x 2^-s for s <= 0, shifts by
// 64 or more as torch's int64 shifts give them.
__device__ __forceinline__ int64_t rsh64(int64_t x, int64_t s) {
  if (s > 0) return sar(add_wrap(x, shl(1, s - 1)), s);
  return shl(x, -s);
}

// intops.bitlen (src/bitexact/intops.py:14-21) for x >= 0: 64 - clz.
__device__ __forceinline__ int64_t bitlen(int64_t x) {
  return x > 0 ? 64 - __clzll((unsigned long long)x) : 0;
}

// floor(a / b) for b > 0 (intops.fdiv, src/bitexact/intops.py:36-38).
__device__ __forceinline__ int64_t fdiv(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a - q * b < 0) ? q - 1 : q;
}

// floor(a / b) for b > 0 from a float64 estimate and exact integer corrections (the same value as fdiv). The
// estimate is used when |a / b| <= 2^52: its error is then at most a few units, so a - q b cannot overflow for
// |a| < 2^62 and b < 2^60, and the loops bring q to the floor quotient. Larger quotients take fdiv.
__device__ __forceinline__ int64_t fdiv_fast(int64_t a, int64_t b) {
  const double qd = (double)a / (double)b;
  if (!(qd < 4503599627370496.0 && qd > -4503599627370496.0)) return fdiv(a, b);
  int64_t q = (int64_t)qd;
  int64_t r = a - q * b;
  while (r < 0) { --q; r += b; }
  while (r >= b) { ++q; r -= b; }
  return q;
}

// floor(a / b) for b > 0 given binv = 1 / (double) b: fdiv_fast with the float64 estimate formed by a
// multiplication. Its relative error is a few 2^-53, so for |a / b| <= 2^52 the estimate is within a few units and
// the same integer corrections bring it to the floor quotient (fdiv_fast's overflow bounds hold unchanged).
__device__ __forceinline__ int64_t fdiv_rcp(int64_t a, int64_t b, double binv) {
  const double qd = (double)a * binv;
  if (!(qd < 4503599627370496.0 && qd > -4503599627370496.0)) return fdiv(a, b);
  int64_t q = (int64_t)qd;
  int64_t r = a - q * b;
  while (r < 0) { --q; r += b; }
  while (r >= b) { ++q; r -= b; }
  return q;
}

// s0 + 2^8 s1 + 2^16 s2 + 2^24 s3 + 2^32 s4 (wrapping) for five int32 partial sums, formed in 32-bit halves: term
// s_i 2^(8 i) is (s_i >> (32 - 8 i)) 2^32 + ((uint32) s_i << 8 i) with an arithmetic shift, so the low words add with
// carries and the high words take the shifted-out parts; no 64-bit shift or add is needed.
__device__ __forceinline__ int64_t join5(int32_t s0, int32_t s1, int32_t s2, int32_t s3, int32_t s4) {
  unsigned c0, c1, c2;
  uint32_t lo = __builtin_addc((uint32_t)s0, (uint32_t)s1 << 8, 0u, &c0);
  lo = __builtin_addc(lo, (uint32_t)s2 << 16, 0u, &c1);
  lo = __builtin_addc(lo, (uint32_t)s3 << 24, 0u, &c2);
  const uint32_t hi = (uint32_t)(s0 >> 31) + (uint32_t)(s1 >> 24) + (uint32_t)(s2 >> 16) + (uint32_t)(s3 >> 8) +
                      (uint32_t)s4 + c0 + c1 + c2;
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Signed base-256 digit and remainder (intops.split_limbs, src/bitexact/intops.py:62-70).
__device__ __forceinline__ int32_t limb_lo(int32_t r) { return ((r + 128) & 255) - 128; }
__device__ __forceinline__ int64_t limb_lo64(int64_t r) { return ((r + 128) & 255) - 128; }

// wmm.epilogue (src/bitexact/exact/wmm.py:132-150) over ops.combine + ops.shift_round_hl
// (src/bitexact/exact/ops.py:60-79): y = round((T 2^d + B) 2^p), and the `checked` loss / range test.
__device__ __forceinline__ int64_t exact_round(int64_t T, int64_t B, int64_t d, int64_t p, bool& bad) {
  const int64_t s = 32 - d;
  int64_t H = T >> s;
  int64_t L = (int64_t)((uint64_t)(T & ((1LL << s) - 1)) << d);
  L = add_wrap(L, B);
  H = add_wrap(H, L >> 32);
  L = L & 0xFFFFFFFFLL;
  const int64_t k = p < 0 ? -p : 0;
  int64_t y;
  if (p >= 0) {
    const int64_t pp = p > 30 ? 30 : p;
    y = (int64_t)(((uint64_t)H << (32 + pp)) + ((uint64_t)L << pp));
  } else if (k < 32) {
    y = add_wrap((int64_t)((uint64_t)H << (32 - k)), (L + (1LL << (k - 1))) >> k);
  } else {
    const int64_t k2 = k > 94 ? 94 : k;
    const int64_t carry = (k2 == 32) ? ((L + (1LL << 31)) >> 32) : (1LL << (k2 - 33));
    y = add_wrap(H, carry) >> imin(k2 - 32, 62);
  }
  const int64_t up_limit = 1LL << (31 - imin(imax(p, 0), 30));
  const int64_t small_limit = 1LL << (31 + imin(imax(-p, 1), 31));
  const bool up_lost = (H >= up_limit) | (H < -up_limit) | ((p > 30) & ((H != 0) | (L != 0)));
  const bool small_lost = (H >= small_limit) | (H < -small_limit);
  const bool lost = (p >= 0) ? up_lost : ((p > -32) & small_lost);
  bad = lost | (y <= -(1LL << 62)) | (y >= (1LL << 62));
  return y;
}

// exact_round with a short path for the common case. With k = -p >= d, k <= 62, |T| < 2^59 and |B| < 2^60:
// floor((T 2^d + B + 2^(k-1)) / 2^k) = floor((T + floor((B + 2^(k-1)) / 2^d)) / 2^(k-d)) (nested floors of
// power-of-two divisions), every intermediate fits int64, |y| < 2^59, and wmm.epilogue's checked conditions
// are all false there, so the value and the flag equal the full rule's. Anything else takes the full rule.
__device__ __forceinline__ int64_t exact_round_fast(int64_t T, int64_t B, int64_t d, int64_t p, bool& bad) {
  const int64_t k = -p;
  const bool fast = (k >= d) & (k >= 1) & (k <= 62) & (T < (1LL << 59)) & (T > -(1LL << 59)) & (B < (1LL << 60)) &
                    (B > -(1LL << 60));
  if (fast) {
    bad = false;
    return (T + ((B + (1LL << (k - 1))) >> d)) >> (k - d);
  }
  return exact_round(T, B, d, p, bad);
}

__device__ __forceinline__ uint32_t pack4(int32_t a, int32_t b, int32_t c, int32_t d) {
  return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) | ((uint32_t)(d & 255) << 24);
}

// Three int8 limb words (4 values each) of 4 int32 values (intops.split_limbs, src/bitexact/intops.py:62-70).
__device__ __forceinline__ void split3(v4i v, uint32_t& l0, uint32_t& l1, uint32_t& l2) {
  int32_t a0[4], a1[4], a2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    int32_t r = v[e];
    a0[e] = limb_lo(r);
    r = (r - a0[e]) >> 8;
    a1[e] = limb_lo(r);
    r = (r - a1[e]) >> 8;
    a2[e] = limb_lo(r);
  }
  l0 = pack4(a0[0], a0[1], a0[2], a0[3]);
  l1 = pack4(a1[0], a1[1], a1[2], a1[3]);
  l2 = pack4(a2[0], a2[1], a2[2], a2[3]);
}

// Raw buffer loads (stride 0, byte range [0, kBufRange)): an offset at or past the range returns zero without
// a memory access but still counts as an outstanding load, so a skipped step costs no traffic and the
// compiler's wait counts stay the same on every path.
constexpr int kBufRange = 0x7fffffff;
constexpr int kBufSkip = 0x7fffffff;   // offset of a skipped load

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, kBufRange, 0x00020000);
}

__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Asynchronous 16-byte load per lane straight into LDS (buffer_load_dwordx4 ... lds): the wave's 64 lanes fill
// 1 KiB at `lds` (M0 base), lane l at byte 16 l, from buffer offset voff + soff.
__device__ __forceinline__ void buf_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// Ring-stage barrier: wait until at most n of this wave's vector memory operations (the asynchronous LDS
// loads of later stages) are outstanding and all its LDS reads are done (gfx9 s_waitcnt encoding: vmcnt <= n,
// lgkmcnt = 0), then a bare s_barrier. __syncthreads() would add a release fence, i.e. vmcnt(0), and drain
// the whole ring every iteration; the memory clobber keeps the compiler from moving LDS accesses across.
template <int n>
__device__ __forceinline__ void ring_barrier() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));
  asm volatile("s_barrier" ::: "memory");
}

// Workspace slots are written by one block and read by another, possibly on another XCD (whose L2 is its own):
// agent-scope relaxed atomic stores and loads keep them coherent without a cache-wide fence.
__device__ __forceinline__ void ws_store(int64_t* a, int64_t v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int64_t ws_load(int64_t* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- wavefront reductions (wave64) ----
__device__ __forceinline__ int64_t wave_max64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = imax(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// DPP forms: a row rotation (row_ror:n, dpp_ctrl 0x120 + n) of both 32-bit halves; rotations by 1, 2, 4 and 8
// leave every lane of a 16-lane row with the row's reduction, and the four rows meet through readlane, so the
// result is wave-uniform without any LDS traffic (the shuffles above go through the LDS crossbar). Every lane of
// the wave must be active.
template <int CTRL>
__device__ __forceinline__ int64_t dpp64(int64_t v) {
  const int lo = __builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp((int)(v >> 32), (int)(v >> 32), CTRL, 0xF, 0xF, false);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const int lo = __builtin_amdgcn_readlane((int)v, l), hi = __builtin_amdgcn_readlane((int)(v >> 32), l);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
template <bool MAX>
__device__ __forceinline__ int64_t op64(int64_t a, int64_t b) { return MAX ? imax(a, b) : add_wrap(a, b); }
template <bool MAX>
__device__ __forceinline__ int64_t wave_reduce64_dpp(int64_t v) {
  v = op64<MAX>(v, dpp64<0x121>(v));
  v = op64<MAX>(v, dpp64<0x122>(v));
  v = op64<MAX>(v, dpp64<0x124>(v));
  v = op64<MAX>(v, dpp64<0x128>(v));
  return op64<MAX>(op64<MAX>(readlane64(v, 0), readlane64(v, 16)), op64<MAX>(readlane64(v, 32), readlane64(v, 48)));
}
// Block reduction over NW waves with an LDS-only barrier (no wait for outstanding global loads or stores);
// `slot` (NW entries) must not be reused by another reduction before every wave has passed this one.
template <bool MAX, int NW>
__device__ __forceinline__ int64_t block_reduce64_dpp(int64_t v, int64_t* slot, int64_t identity) {
  v = wave_reduce64_dpp<MAX>(v);
  const int lane = threadIdx.x & 63;
  if (lane == 0) slot[threadIdx.x >> 6] = v;
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
  return wave_reduce64_dpp<MAX>(lane < NW ? slot[lane] : identity);
}
__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  return v;
}

}  // namespace bx

// Phase timers (measurement builds only: compiled with -DBX_PHASES, a separate library): BX_PHASE(kid, k) records
// the 100 MHz real-time counter for phase boundary k (0..7) of kernel slot kid (0..3) in block b (< 1024) of the
// launch, thread 0 only. BX_PHASE_DEFINE(name) gives a source file its table and the exported reader
// bx_phases_<name>(host): the table as uint64 [4][1024][8]; without -DBX_PHASES the reader returns BX_EINVAL and
// the marks compile to nothing.
#ifdef BX_PHASES
#define BX_PHASE(kid, k)                                                                   \
  do {                                                                                     \
    if (threadIdx.x == 0) {                                                                \
      const unsigned bx_b_ = blockIdx.x + blockIdx.y * gridDim.x;                          \
      if (bx_b_ < 1024) g_bx_phase[kid][bx_b_][k] = __builtin_amdgcn_s_memrealtime();      \
    }                                                                                      \
  } while (0)
#define BX_PHASE_TABLE static __device__ uint64_t g_bx_phase[4][1024][8];
#define BX_PHASE_DEFINE(name)                                                                              \
  extern "C" int bx_phases_##name(uint64_t* host) {                                                        \
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_bx_phase), sizeof(g_bx_phase)) == hipSuccess ? BX_OK : BX_EINVAL; \
  }
#else
#define BX_PHASE(kid, k) \
  do {                   \
  } while (0)
#define BX_PHASE_TABLE
#define BX_PHASE_DEFINE(name) \
  extern "C" int bx_phases_##name(uint64_t*) { return BX_EINVAL; }
#endif

#define BX_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      bx::set_error(__VA_ARGS__);      \
      return BX_EINVAL;                \
    }                                  \
  } while (0)
