// The reference's Python helper rules as device kernels: the element-wise integer rules of src/bitexact/intops.py,
// src/bitexact/exact/ops.py, src/bitexact/int8/ops.py and the RoPE / division steps of the two segs modules
// (bx_int_elementwise), and their per-row reductions (bx_int_rowop: exact quant, rms, masked softmax weights; int8
// rms, quant_rows, pre_norm, softmax; row amax). They back the bitexact.intops / exact.ops / int8.ops functions
// and the module-level segs stages, so a caller of the reference's helpers gets the same integers from the GPU.
//
// Operands are strided views: operand j of an element-wise call reads element (r, c) of the [rows, inner] output
// grid at p + r srow + c scol (bytes 1, 2, 4 or 8, signed), or is the constant `imm` when p is null, so
// broadcasting (a row vector, a column vector, a scalar) costs no copy. Integer arithmetic is torch's int64:
// two's complement wrap, shifts by 64 or more as the reference's CPU tensors give them.
#include "bx_common.h"
#include "bx_introws.h"

#include <algorithm>

namespace bx {

constexpr int kMaxIn = 5;
struct Operand {
  const void* p;
  int64_t srow, scol, imm;
  int32_t bytes;
};

struct ElemArgs {
  Operand in[kMaxIn];
  void* out0;
  void* out1;
  int32_t ob0, ob1;   // output element bytes (8 int64, 4 int32, 1 int8)
  int64_t rows, inner;
  const int64_t* lut;
  int64_t lut_len;
  int64_t iarg, iarg2;
  int32_t* flag;
  int32_t op;
};

__device__ __forceinline__ int64_t ld(const Operand& o, int64_t r, int64_t c) {
  if (o.p == nullptr) return o.imm;
  const int64_t off = r * o.srow + c * o.scol;
  switch (o.bytes) {
    case 8: return ((const int64_t*)o.p)[off];
    case 4: return ((const int32_t*)o.p)[off];
    case 2: return ((const int16_t*)o.p)[off];
    default: return ((const int8_t*)o.p)[off];
  }
}

__device__ __forceinline__ void st(void* p, int32_t bytes, int64_t i, int64_t v) {
  if (bytes == 8) ((int64_t*)p)[i] = v;
  else if (bytes == 4) ((int32_t*)p)[i] = (int32_t)v;
  else ((int8_t*)p)[i] = (int8_t)v;
}

// torch's floor division of int64 (b != 0)
__device__ __forceinline__ int64_t floordiv(int64_t a, int64_t b) {
  if (b == -1) return (int64_t)(0 - (uint64_t)a);
  const int64_t q = a / b;
  return (q * b != a && ((a < 0) != (b < 0))) ? q - 1 : q;
}

// x << s for s >= 0 and x >> -s otherwise (torch: shifts by >= 64 give 0, or the sign)
__device__ __forceinline__ int64_t shift_lr(int64_t x, int64_t s) { return s >= 0 ? shl(x, s) : sar(x, -s); }

// ops.combine (src/bitexact/exact/ops.py:60-66): (H, L) with H 2^32 + L = T 2^d + B, 0 <= L < 2^32
__device__ __forceinline__ void combine_hl(int64_t T, int64_t d, int64_t B, int64_t& H, int64_t& L) {
  const int64_t s = 32 - d;
  H = sar(T, s);
  L = shl(T & add_wrap(shl(1, s), -1), d);
  L = add_wrap(L, B);
  H = add_wrap(H, L >> 32);
  L = L & 0xFFFFFFFFLL;
}

// ops.shift_round_hl (src/bitexact/exact/ops.py:69-79): round((H 2^32 + L) 2^p)
__device__ __forceinline__ int64_t shift_round_hl(int64_t H, int64_t L, int64_t p) {
  const int64_t k = p < 0 ? -p : 0;
  if (p >= 0) {
    const int64_t pp = imin(p, 30);
    return add_wrap(shl(H, 32 + pp), shl(L, pp));
  }
  if (k < 32) {
    const int64_t k1 = imax(k, 1);
    return add_wrap(shl(H, 32 - k1), add_wrap(L, 1LL << (k1 - 1)) >> k1);
  }
  const int64_t k2 = imin(k, 94);
  const int64_t carry = k2 == 32 ? (add_wrap(L, 1LL << 31) >> 32) : shl(1, imax(k2 - 33, 0));
  return sar(add_wrap(H, carry), imin(k2 - 32, 62));
}

// ops.exp2neg_lut (src/bitexact/exact/ops.py:108-116): 2^-t at out_bits, t >= 0 at FT2 = 26 bits
__device__ __forceinline__ int64_t exp2neg_lut(int64_t t, const int64_t* lut, int64_t out_bits) {
  const int64_t n = t >> 26, f = t & ((1LL << 26) - 1);
  const int64_t idx = f >> 12, rr = f & 4095;
  const int64_t a = lut[idx];
  const int64_t v = add_wrap(a, rshc(mul_wrap(lut[idx + 1] - a, rr), 12));
  return rshc(v, 60 - out_bits + n);
}

enum ElemOp {
  E_BITLEN = 1,     // intops.bitlen(a)
  E_RSH = 2,        // intops.rsh(a, b)
  E_RSHC = 3,       // exact ops.rshc(a, b)
  E_FDIV = 4,       // intops.fdiv(a, b)
  E_RDIV = 5,       // intops.rdiv(a, b)
  E_ISQRT = 6,      // intops.isqrt(a)
  E_DIVROUND = 7,   // ops.div_round(a, b = p, c = r)
  E_COMBINE = 8,    // ops.combine(T = a, d = b, B = c) -> (H, L)
  E_SHRHL = 9,      // ops.shift_round_hl(H = a, L = b, p = c)
  E_EXP2NEG = 10,   // ops.exp2neg_lut(a, lut, iarg)
  E_SILU_MUL = 11,  // ops.silu_mul(g = a, u = b, lut) at FR = iarg: P; flag where not ok
  E_EXP_OF = 12,    // int8 ops.exp_of(a, lut), iarg = EXP_MIN << FA
  E_SILU8 = 13,     // int8 ops.silu(a, lut), iarg = FR - FA, iarg2 = SILU_LIM << FA
  E_NORM24 = 14,    // int8 ops.norm24(mant = a, e = b) -> (mant, e)
  E_MULSUB = 15,    // rsh(a b - c d, iarg)
  E_MULADD = 16,    // rsh(a b + c d, iarg)
  E_ABSFLAG = 17,   // flag where |a| > iarg (and out0 = a when given)
  E_LIMBS = 18,     // intops.split_limbs(a, iarg): out0 = iarg planes [iarg][rows inner], out1 = remainder;
                    // iarg2 > 0: out0 holds iarg2 elements, the ones past the planes are zeroed (stack_limbs padding)
  E_JOIN = 19,      // intops.join_limbs: a + (b << 8) + (c << 16) over the first iarg of them
  E_ADD = 20,       // a + b
  E_SUB = 21,       // a - b
  E_MUL = 22,       // a b
  E_SHIFT = 23,     // a << b (b >= 0) or a >> -b
  E_NDIV = 24,      // segs.ndiv: div_round(a x b, d - e + iarg, c) for (x, gm, r, ge, er)
  E_PRODGE = 25,    // flag where a b (wrapping int64 product) >= 2^iarg
  E_MUL_RSH = 26,   // rsh(a b, iarg)
  E_RDIVSH = 27,    // rdiv(a << iarg, b)
  E_GTFLAG = 28,    // flag where a > iarg
};

__global__ __launch_bounds__(256) void elem_kernel(ElemArgs p) {
  const int64_t n = p.rows * p.inner;
  const int64_t step = (int64_t)gridDim.x * 256;
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < max(n, p.iarg2 > 0 ? p.iarg2 : 0); i += step) {
    if (i >= n) {   // padding rows of a stacked limb matrix: past the iarg planes
      if (p.op == E_LIMBS && i >= p.iarg * n) st(p.out0, p.ob0, i, 0);
      continue;
    }
    const int64_t r = i / p.inner, c = i - r * p.inner;
    const int64_t a = ld(p.in[0], r, c);
    int64_t v = 0, v1 = 0;
    switch (p.op) {
      case E_BITLEN: v = bitlen(a); break;
      case E_RSH: v = rsh64(a, ld(p.in[1], r, c)); break;
      case E_RSHC: v = rshc(a, ld(p.in[1], r, c)); break;
      case E_FDIV: {
        const int64_t b = ld(p.in[1], r, c);
        bad |= b == 0;
        v = b == 0 ? 0 : floordiv(a, b);
        break;
      }
      case E_RDIV: {
        const int64_t b = ld(p.in[1], r, c), d = 2 * b;
        bad |= d == 0;
        v = d == 0 ? 0 : floordiv(add_wrap(2 * a, b), d);
        break;
      }
      case E_ISQRT: bad |= a < 0; v = a < 0 ? 0 : isqrt64(a); break;
      case E_DIVROUND: {
        const int64_t pp = ld(p.in[1], r, c), rr = ld(p.in[2], r, c);
        bad |= rr <= 0;
        v = rr <= 0 ? 0 : div_round64(a, pp, rr, 1.0 / (double)rr);
        break;
      }
      case E_COMBINE: combine_hl(a, ld(p.in[1], r, c), ld(p.in[2], r, c), v, v1); break;
      case E_SHRHL: v = shift_round_hl(a, ld(p.in[1], r, c), ld(p.in[2], r, c)); break;
      case E_EXP2NEG: v = exp2neg_lut(a, p.lut, p.iarg); break;
      case E_SILU_MUL: {
        const int idx = silu_index(a, (int)p.iarg);
        v = silu_elem(a, ld(p.in[1], r, c), p.lut[idx], p.lut[idx + 1], (int)p.iarg, bad);
        break;
      }
      case E_EXP_OF: {
        const int64_t idx = a - p.iarg;
        const bool past = idx >= p.lut_len;
        bad |= past;
        v = idx < 0 ? 0 : p.lut[past ? p.lut_len - 1 : idx];
        break;
      }
      case E_SILU8: {
        const int64_t sh = p.iarg, lo = -p.iarg2, hi = p.iarg2;
        const int64_t gi = a >> sh;
        const int64_t rr = a - shl(gi, sh);
        const int64_t ix = imin(imax(gi, lo), hi - 1) - lo;
        const int64_t la = p.lut[ix];
        const int64_t val = add_wrap(la, rsh64(mul_wrap(p.lut[ix + 1] - la, rr), sh));
        v = gi >= hi ? a : gi < lo ? 0 : val;
        break;
      }
      case E_NORM24: {
        const int64_t b = bitlen(a) - 24;
        v = rsh64(a, b);
        v1 = ld(p.in[1], r, c) + b;
        break;
      }
      case E_MULSUB:
        v = rsh64(mul_wrap(a, ld(p.in[1], r, c)) - mul_wrap(ld(p.in[2], r, c), ld(p.in[3], r, c)), p.iarg);
        break;
      case E_MULADD:
        v = rsh64(add_wrap(mul_wrap(a, ld(p.in[1], r, c)), mul_wrap(ld(p.in[2], r, c), ld(p.in[3], r, c))), p.iarg);
        break;
      case E_ABSFLAG: bad |= (a < 0 ? (int64_t)(0 - (uint64_t)a) : a) > p.iarg; v = a; break;
      case E_LIMBS: {
        int64_t rem = a;
        for (int l = 0; l < p.iarg; ++l) {
          const int64_t lo = limb_lo64(rem);
          st(p.out0, p.ob0, (int64_t)l * n + i, lo);
          rem = (rem - lo) >> 8;
        }
        if (p.out1 != nullptr) st(p.out1, p.ob1, i, rem);
        continue;
      }
      case E_JOIN: {
        v = a;
        for (int l = 1; l < p.iarg; ++l) v = add_wrap(v, shl(ld(p.in[l], r, c), 8 * l));
        break;
      }
      case E_ADD: v = add_wrap(a, ld(p.in[1], r, c)); break;
      case E_SUB: v = add_wrap(a, (int64_t)(0 - (uint64_t)ld(p.in[1], r, c))); break;
      case E_MUL: v = mul_wrap(a, ld(p.in[1], r, c)); break;
      case E_SHIFT: v = shift_lr(a, ld(p.in[1], r, c)); break;
      case E_NDIV: {
        const int64_t rr = ld(p.in[2], r, c);
        const int64_t pp = ld(p.in[3], r, c) - ld(p.in[4], r, c) + p.iarg;
        bad |= rr <= 0;
        v = rr <= 0 ? 0 : div_round64(mul_wrap(a, ld(p.in[1], r, c)), pp, rr, 1.0 / (double)rr);
        break;
      }
      case E_PRODGE: bad |= mul_wrap(a, ld(p.in[1], r, c)) >= shl(1, p.iarg); v = 0; break;
      case E_MUL_RSH: v = rsh64(mul_wrap(a, ld(p.in[1], r, c)), p.iarg); break;
      case E_RDIVSH: {
        const int64_t b = ld(p.in[1], r, c), d = 2 * b;
        bad |= d == 0;
        v = d == 0 ? 0 : floordiv(add_wrap(2 * shl(a, p.iarg), b), d);
        break;
      }
      case E_GTFLAG: bad |= a > p.iarg; v = a; break;
      default: bad = 1; break;
    }
    if (p.out0 != nullptr) st(p.out0, p.ob0, i, v);
    if (p.out1 != nullptr) st(p.out1, p.ob1, i, v1);
  }
  if (bad && p.flag != nullptr) p.flag[0] = 1;
}

// ---- row reductions, one 256-thread block per row ----
enum RowOp {
  R_QUANT = 1,      // exact ops.quant(P, eps = in[0]): out0 q int64 [rows, D], out1 sh [rows]
  R_RMS = 2,        // exact ops.rms(x): out0 r, out1 er; iargs[0] = FR
  R_RMS8 = 3,       // int8 ops.rms(x): out0 r, out1 shx; iargs[0] = FR
  R_SOFTMAX_W = 4,  // exact ops.softmax_w(raw, ok = in[0], sh = in[1], kbits, lut, fp, l2e): out0 p, out1 den
  R_SOFTMAX8 = 5,   // int8 segs.softmax(raw, qpos = in[0], expt, hd): out0 p, out1 den
  R_QROWS8 = 6,     // int8 ops.quant_rows(z, nl): out0 q int64, out1 as_, out2 sh; out3 stacked limbs (optional)
  R_PRENORM8 = 7,   // int8 segs.pre_norm(x, gamma = in[0], nl): out0 q int64 (optional), out1 mant, out2 e, out3 limbs
  R_AMAX = 8,       // max |x| of the row: out0 [rows]
};

struct RowArgs {
  Operand in[3];
  const int64_t* x;
  int64_t ldx;
  void* out[4];
  int64_t rows, D;
  const int64_t* lut;
  int64_t lut_len;
  int64_t ia[6];
  int32_t* flag;
  int32_t op;
};

constexpr int kRT = 256;
constexpr int64_t kEps40 = 10995116;   // round(1e-5 2^40) (src/bitexact/int8/ops.py:18)

__device__ __forceinline__ int64_t iabs(int64_t v) { return v < 0 ? (int64_t)(0 - (uint64_t)v) : v; }

// int8 ops.quant_rows (src/bitexact/int8/ops.py:24-35) of one element given the row's sh and as_
__device__ __forceinline__ int64_t quant8(int64_t z, int64_t sh, int64_t as_, int64_t qm) {
  return floordiv(add_wrap(2 * mul_wrap(rsh64(z, sh), qm), as_), 2 * as_);
}

__global__ __launch_bounds__(kRT) void row_kernel(RowArgs p) {
  __shared__ int64_t sbuf[16];
  const int64_t r = blockIdx.x;
  const int64_t* xr = p.x + r * p.ldx;
  const int64_t D = p.D;
  int bad = 0;
  switch (p.op) {
    case R_AMAX: {
      int64_t m = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) m = imax(m, iabs(xr[c]));
      m = block_max64(m, sbuf);
      if (threadIdx.x == 0) ((int64_t*)p.out[0])[r] = m;
      break;
    }
    case R_QUANT: {   // e = bitlen|P| + eps (P != 0), sh = max e - QB (>= NEG_BIG), q = rshc(P, sh - eps)
      int64_t e = kNegBig;
      for (int64_t c = threadIdx.x; c < D; c += kRT) {
        const int64_t P = xr[c];
        if (P != 0) e = imax(e, bitlen(iabs(P)) + ld(p.in[0], r, c));
      }
      e = block_max64(e, sbuf);
      const int64_t sh = imax(e - kQB, kNegBig);
      for (int64_t c = threadIdx.x; c < D; c += kRT)
        ((int64_t*)p.out[0])[r * D + c] = rshc(xr[c], sh - ld(p.in[0], r, c));
      if (threadIdx.x == 0) ((int64_t*)p.out[1])[r] = sh;
      break;
    }
    case R_RMS: {   // ops.rms (src/bitexact/exact/ops.py:92-105); D = 2^lg
      const int64_t FR = p.ia[0];
      const int lg = 63 - __clzll((unsigned long long)D);
      int64_t amax = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) amax = imax(amax, iabs(xr[c]));
      amax = imax(block_max64(amax, sbuf), 1);
      const int64_t shx = imax(bitlen(amax) - 25, -6);
      int64_t S = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) {
        const int64_t xs = rshc(xr[c], shx);
        S = add_wrap(S, mul_wrap(xs, xs));
      }
      S = block_sum64(S, sbuf);
      const int64_t T = add_wrap(S, rshc(kEps60 * D, 60 - 2 * (FR - shx)));
      const int64_t m = floordiv(62 + lg - bitlen(T), 2);
      const int64_t s = 2 * m - lg;
      const int64_t V = s >= 0 ? shl(T, s) : sar(T, -s);
      if (threadIdx.x == 0) {
        ((int64_t*)p.out[0])[r] = isqrt64(V);
        ((int64_t*)p.out[1])[r] = shx - FR - m;
      }
      break;
    }
    case R_RMS8: {   // int8 ops.rms (src/bitexact/int8/ops.py:76-84)
      const int64_t FR = p.ia[0];
      int64_t amax = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) amax = imax(amax, iabs(xr[c]));
      amax = imax(block_max64(amax, sbuf), 1);
      const int64_t shx = bitlen(amax) - 24;
      int64_t S = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) {
        const int64_t xs = rsh64(xr[c], shx);
        S = add_wrap(S, mul_wrap(xs, xs));
      }
      S = block_sum64(S, sbuf);
      const int64_t ms = floordiv(S, D);
      const int64_t eps = rsh64(kEps40, 40 - 2 * (FR - shx));
      if (threadIdx.x == 0) {
        const int64_t v = add_wrap(ms, eps);
        bad |= v < 0;
        ((int64_t*)p.out[0])[r] = v < 0 ? 0 : isqrt64(v);
        ((int64_t*)p.out[1])[r] = shx;
      }
      break;
    }
    case R_SOFTMAX_W: {   // ops.softmax_w (src/bitexact/exact/ops.py:133-143)
      const int64_t kbits = p.ia[0], fp = p.ia[1], l2e = p.ia[2];
      int64_t mx = kNeg;
      for (int64_t c = threadIdx.x; c < D; c += kRT) mx = imax(mx, ld(p.in[0], r, c) ? xr[c] : kNeg);
      mx = block_max64(mx, sbuf);
      const int64_t zshift = kbits + 3 - ld(p.in[1], r, 0) - 26;
      int64_t sum = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) {
        const int64_t w = ld(p.in[0], r, c) ? weight64(add_wrap(mx, -xr[c]), zshift, p.lut, l2e, (int)fp) : 0;
        ((int64_t*)p.out[0])[r * D + c] = w;
        sum = add_wrap(sum, w);
      }
      sum = block_sum64(sum, sbuf);
      if (threadIdx.x == 0) ((int64_t*)p.out[1])[r] = sum;
      break;
    }
    case R_SOFTMAX8: {   // int8 segs.softmax (src/bitexact/int8/segs.py:90-99) with score_rule (36-44), exp_of
      const int64_t qpos = ld(p.in[0], r, 0);
      const int64_t mul = p.ia[0], zsh = p.ia[1], fefp = p.ia[2], emin = p.ia[3];   // mul 0: head_dim 64
      int64_t mx = kNeg;
      for (int64_t c = threadIdx.x; c < D; c += kRT) mx = imax(mx, c <= qpos ? xr[c] : kNeg);
      mx = block_max64(mx, sbuf);
      int64_t sum = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT) {
        int64_t w = 0;
        if (c <= qpos) {
          const int64_t d = add_wrap(xr[c], -mx);
          int64_t z = mul == 0 ? rsh64(d, zsh) : rsh64(mul_wrap(imax(d, -(1LL << 38)), mul), zsh);
          z = imax(z, -(1LL << 40));
          const int64_t idx = z - emin;
          const bool past = idx >= p.lut_len;
          bad |= past;
          const int64_t e = idx < 0 ? 0 : p.lut[past ? p.lut_len - 1 : idx];
          w = rsh64(e, fefp);
        }
        ((int64_t*)p.out[0])[r * D + c] = w;
        sum = add_wrap(sum, w);
      }
      sum = block_sum64(sum, sbuf);
      if (threadIdx.x == 0) ((int64_t*)p.out[1])[r] = sum;
      break;
    }
    case R_QROWS8:
    case R_PRENORM8: {
      const bool pre = p.op == R_PRENORM8;
      const int64_t nl = p.ia[0], qm = 127LL << (8 * (nl - 1));
      // pre_norm: r, shx = rms(x) and z = x gamma (src/bitexact/int8/segs.py:47-52); else z = x
      int64_t rr = 0, shx = 0;
      if (pre) {
        const int64_t FR = p.ia[1];
        int64_t amax = 0;
        for (int64_t c = threadIdx.x; c < D; c += kRT) amax = imax(amax, iabs(xr[c]));
        amax = imax(block_max64(amax, sbuf), 1);
        shx = bitlen(amax) - 24;
        int64_t S = 0;
        for (int64_t c = threadIdx.x; c < D; c += kRT) {
          const int64_t xs = rsh64(xr[c], shx);
          S = add_wrap(S, mul_wrap(xs, xs));
        }
        S = block_sum64(S, sbuf);
        const int64_t v = add_wrap(floordiv(S, D), rsh64(kEps40, 40 - 2 * (FR - shx)));
        bad |= v < 0;
        rr = v < 0 ? 0 : isqrt64(v);
      }
      int64_t amax = 0;
      for (int64_t c = threadIdx.x; c < D; c += kRT)
        amax = imax(amax, iabs(pre ? mul_wrap(xr[c], ld(p.in[0], r, c)) : xr[c]));
      amax = imax(block_max64(amax, sbuf), 1);
      const int64_t sh = bitlen(amax) - 30;
      const int64_t as_ = rsh64(amax, sh);
      for (int64_t c = threadIdx.x; c < D; c += kRT) {
        const int64_t z = pre ? mul_wrap(xr[c], ld(p.in[0], r, c)) : xr[c];
        const int64_t q = quant8(z, sh, as_, qm);
        if (p.out[0] != nullptr) ((int64_t*)p.out[0])[r * D + c] = q;
        if (p.out[3] != nullptr) {   // limb l of row r at stacked row l rows + r
          int64_t rem = q;
          for (int l = 0; l < nl; ++l) {
            const int64_t lo = limb_lo64(rem);
            ((int8_t*)p.out[3])[((int64_t)l * p.rows + r) * D + c] = (int8_t)lo;
            rem = (rem - lo) >> 8;
          }
        }
      }
      if (threadIdx.x == 0) {
        if (pre) {   // mant, e = norm24(rdiv(as_ << 30, r), sh - FG - shx - 30)
          const int64_t FG = p.ia[2];
          bad |= rr <= 0;
          const int64_t m0 = rr <= 0 ? 0 : floordiv(add_wrap(2 * shl(as_, 30), rr), 2 * rr);
          const int64_t b = bitlen(m0) - 24;
          ((int64_t*)p.out[1])[r] = rsh64(m0, b);
          ((int64_t*)p.out[2])[r] = sh - FG - shx - 30 + b;
        } else {
          ((int64_t*)p.out[1])[r] = as_;
          ((int64_t*)p.out[2])[r] = sh;
        }
      }
      break;
    }
    default: bad = 1; break;
  }
  if (bad && p.flag != nullptr) p.flag[0] = 1;
}

// A streaming read of `bytes` (16-byte nontemporal loads, grid-stride, a few in flight per thread): the practical
// HBM read ceiling of one launch at a given size, for the decode GEMMs' roofline.
__global__ void stream_read_kernel(const v4i* __restrict__ src, int64_t n16, int32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int acc = 0;
  constexpr int U = 4;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    v4i v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const v4i v = src[i];
    acc ^= v.x ^ v.w;
  }
  if (acc == 0x5eed5eed) sink[0] = acc;   // keeps the loads; practically never taken
}

// Back-to-back int8 MFMAs from registers (CH independent accumulator chains per wave, no memory traffic in the
// loop): the dense int8 rate the matrix cores sustain, for the prefill kernels' roofline. SHAPE 0:
// v_mfma_i32_32x32x32_i8 (65536 ops), 1: v_mfma_i32_16x16x64_i8 (32768 ops). RND: the operands take fresh
// pseudo-random bytes every iteration (a 32-bit LCG per dword, 16 VALU per 4 MFMAs), as a GEMM's limbs do; the
// matrix cores' clock under load depends on how many operand bits switch, so constant operands overstate the rate
// (mul = 1, inc = 0 runs the same instructions on constant operands: the control).
template <int SHAPE, bool RND>
__global__ void mfma_rate_kernel(int iters, int32_t mul, int32_t inc, int32_t* sink) {
  constexpr int CH = 4;
  const int lane = threadIdx.x & 63;
  v4i a = {lane, lane * 3, lane ^ 5, 7}, b = {lane * 5, 1, lane + 2, lane ^ 9};
  int32_t x = 0;
  if constexpr (SHAPE == 0) {
    v16i acc[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[c][e] = c;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int c = 0; c < CH; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
      if (RND) {
        a = a * mul + inc;
        b = b * mul + (inc ^ 0x55555555);
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) x ^= acc[c][e];
  } else {
    v4i acc[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[c] = v4i{c, c, c, c};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int c = 0; c < CH; ++c) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
      if (RND) {
        a = a * mul + inc;
        b = b * mul + (inc ^ 0x55555555);
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) x ^= acc[c][0] ^ acc[c][1] ^ acc[c][2] ^ acc[c][3];
  }
  if (x == 0x5eed5eed) sink[0] = x;   // keeps the MFMAs; practically never taken
}

static int fill_operands(Operand* o, int nin, const void* const* ptrs, const int64_t* desc) {
  BX_REQUIRE(nin >= 0 && nin <= kMaxIn, "at most %d operands", kMaxIn);
  for (int j = 0; j < kMaxIn; ++j) o[j] = Operand{nullptr, 0, 0, 0, 8};
  for (int j = 0; j < nin; ++j) {
    o[j].p = ptrs ? ptrs[j] : nullptr;
    o[j].srow = desc[4 * j];
    o[j].scol = desc[4 * j + 1];
    o[j].imm = desc[4 * j + 2];
    o[j].bytes = (int32_t)desc[4 * j + 3];
    BX_REQUIRE(o[j].bytes == 1 || o[j].bytes == 2 || o[j].bytes == 4 || o[j].bytes == 8, "operand %d: bad width", j);
  }
  return BX_OK;
}

}  // namespace bx

using namespace bx;

extern "C" int bx_int_elementwise(int32_t op, int32_t nin, const void* const* ptrs, const int64_t* desc, void* out0,
                                  int32_t ob0, void* out1, int32_t ob1, int64_t rows, int64_t inner,
                                  const int64_t* lut, int64_t lut_len, int64_t iarg, int64_t iarg2, int32_t* flag,
                                  bx_stream_t stream) {
  BX_REQUIRE(op >= E_BITLEN && op <= E_GTFLAG, "unknown element-wise rule %d", op);
  BX_REQUIRE(rows >= 0 && inner >= 0, "negative size");
  BX_REQUIRE(desc != nullptr || nin == 0, "null operand descriptors");
  ElemArgs p = {};
  if (int rc = fill_operands(p.in, nin, ptrs, desc)) return rc;
  p.out0 = out0; p.out1 = out1; p.ob0 = ob0; p.ob1 = ob1;
  p.rows = rows; p.inner = inner; p.lut = lut; p.lut_len = lut_len; p.iarg = iarg; p.iarg2 = iarg2;
  p.flag = flag; p.op = op;
  const bool needs_lut = op == E_EXP2NEG || op == E_SILU_MUL || op == E_EXP_OF || op == E_SILU8;
  BX_REQUIRE(!needs_lut || (lut != nullptr && lut_len > 1), "this rule needs its table");
  BX_REQUIRE(op != E_LIMBS || (iarg >= 1 && iarg <= 8), "split_limbs: 1..8 limbs");
  BX_REQUIRE(op != E_JOIN || (iarg >= 1 && iarg <= nin), "join_limbs: one operand per limb");
  const int64_t n = std::max(rows * inner, iarg2 > 0 && op == E_LIMBS ? iarg2 : 0);
  if (n == 0) return BX_OK;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 8192);
  elem_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(p);
  return check_launch("elem_kernel");
}

extern "C" int bx_int_rowop(int32_t op, int32_t nin, const void* const* ptrs, const int64_t* desc, const int64_t* x,
                            int64_t ldx, int64_t rows, int64_t D, void* out0, void* out1, void* out2, void* out3,
                            const int64_t* lut, int64_t lut_len, const int64_t* iargs, int32_t* flag,
                            bx_stream_t stream) {
  BX_REQUIRE(op >= R_QUANT && op <= R_AMAX, "unknown row rule %d", op);
  BX_REQUIRE(rows >= 0 && D >= 0 && ldx >= D, "bad sizes");
  BX_REQUIRE(nin <= 3, "at most 3 operands");
  RowArgs p = {};
  Operand o[kMaxIn];
  if (int rc = fill_operands(o, nin, ptrs, desc)) return rc;
  for (int j = 0; j < 3; ++j) p.in[j] = o[j];
  p.x = x; p.ldx = ldx; p.rows = rows; p.D = D;
  p.out[0] = out0; p.out[1] = out1; p.out[2] = out2; p.out[3] = out3;
  p.lut = lut; p.lut_len = lut_len; p.flag = flag; p.op = op;
  for (int j = 0; j < 6; ++j) p.ia[j] = iargs ? iargs[j] : 0;
  if (op == R_RMS) BX_REQUIRE(D > 0 && (D & (D - 1)) == 0 && D <= 4096, "row length a power of two <= 4096");
  if (op == R_SOFTMAX_W || op == R_SOFTMAX8) BX_REQUIRE(lut != nullptr && lut_len > 1, "this rule needs its table");
  if (op == R_QROWS8 || op == R_PRENORM8) BX_REQUIRE(p.ia[0] >= 1 && p.ia[0] <= 3, "nl must be 1, 2 or 3");
  if (rows == 0) return BX_OK;
  BX_REQUIRE(x != nullptr && D > 0, "null rows");
  row_kernel<<<(unsigned)rows, kRT, 0, (hipStream_t)stream>>>(p);
  return check_launch("row_kernel");
}

extern "C" int bx_stream_read(const void* src, int64_t bytes, int32_t blocks, int32_t threads, int32_t* sink,
                              bx_stream_t stream) {
  BX_REQUIRE(src && sink && bytes > 0 && bytes % 16 == 0 && ((uintptr_t)src & 15) == 0, "bad stream-read buffer");
  BX_REQUIRE(blocks > 0 && threads > 0 && threads <= 1024 && threads % 64 == 0, "bad launch shape");
  stream_read_kernel<<<blocks, threads, 0, (hipStream_t)stream>>>((const v4i*)src, bytes / 16, sink);
  return check_launch("stream_read_kernel");
}

extern "C" int bx_mfma_rate(int32_t shape, int32_t iters, int32_t blocks, int32_t threads, int32_t* sink,
                            bx_stream_t stream) {
  BX_REQUIRE(sink && shape >= 0 && shape <= 5 && iters > 0, "bad mfma-rate arguments");
  BX_REQUIRE(blocks > 0 && threads > 0 && threads <= 1024 && threads % 64 == 0, "bad launch shape");
  const hipStream_t st = (hipStream_t)stream;
  const int32_t mul = shape >= 4 ? 1 : 1664525, inc = shape >= 4 ? 0 : 1013904223;
  if (shape == 0) mfma_rate_kernel<0, false><<<blocks, threads, 0, st>>>(iters, mul, inc, sink);
  else if (shape == 1) mfma_rate_kernel<1, false><<<blocks, threads, 0, st>>>(iters, mul, inc, sink);
  else if (shape % 2 == 0) mfma_rate_kernel<0, true><<<blocks, threads, 0, st>>>(iters, mul, inc, sink);
  else mfma_rate_kernel<1, true><<<blocks, threads, 0, st>>>(iters, mul, inc, sink);
  return check_launch("mfma_rate_kernel");
}
