// Row-wise integer stages around the GEMMs and the attention, one 256-thread block per row with wavefront
// int64 reductions: RMSNorm + per-row quantization (segs.norm_quant), the masked softmax weights
// (segs.softmax), and the attention output rule (segs.attn_out = div_round + regroup + quant).
#include "bx_common.h"

namespace bx {

constexpr int64_t kEps60 = 11529215046068LL;   // round(1e-5 2^60) (src/bitexact/exact/ops.py:21)
constexpr int64_t kNegBig = -(1LL << 20);      // ops.NEG_BIG
constexpr int kQB = 22;                        // |q| <= 2^22

__device__ __forceinline__ int64_t block_max64(int64_t v, int64_t* sbuf) {
  v = wave_max64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sbuf[wave] = v;
  __syncthreads();
  int64_t r = sbuf[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = imax(r, sbuf[i]);
  return r;
}

__device__ __forceinline__ int64_t block_sum64(int64_t v, int64_t* sbuf) {
  v = wave_sum64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sbuf[wave] = v;
  __syncthreads();
  int64_t r = 0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r += sbuf[i];
  return r;
}

// floor(sqrt(x)) for 0 <= x < 2^62, exact (float estimate, then integer corrections; intops.isqrt's value)
__device__ __forceinline__ int64_t isqrt64(int64_t x) {
  uint64_t s = (uint64_t)sqrt((double)x);
  while (s * s > (uint64_t)x) --s;
  while ((s + 1) * (s + 1) <= (uint64_t)x) ++s;
  return (int64_t)s;
}

// ops.div_round (src/bitexact/exact/ops.py:37-57): round(a 2^p / r) by 28-bit long division, r > 0
__device__ __forceinline__ int64_t div_round64(int64_t a, int64_t p, int64_t r) {
  int64_t Q = fdiv(a, r);
  int64_t R = a - Q * r;
  int64_t left = imax(p, 0);
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const int64_t c = imin(left, 28);
    const int64_t X = shl(R, c);
    const int64_t q1 = fdiv(X, r);
    Q = add_wrap(shl(Q, c), q1);
    R = X - q1 * r;
    left -= c;
  }
  const int64_t up = Q + (2 * R >= r ? 1 : 0);
  const int64_t k = imin(imax(-p, 1), 62);
  const int64_t down = add_wrap(Q, 1LL << (k - 1)) >> k;
  return p >= 0 ? up : down;
}

// ---- segs.norm_quant (src/bitexact/exact/segs.py:59-63) over ops.rms (src/bitexact/exact/ops.py:92-105) and
// ops.quant (src/bitexact/exact/ops.py:82-89). P rows are kept in LDS between the two passes. ----
__global__ __launch_bounds__(256) void norm_quant_kernel(const int64_t* x, int64_t ldx, const int64_t* gm,
                                                         const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh, int D,
                                                         int lg, int FR, int FN, int32_t* err) {
  extern __shared__ __align__(16) char smem[];
  int64_t* Ps = (int64_t*)smem;
  __shared__ int64_t sbuf[8];
  const int64_t* xr = x + (int64_t)blockIdx.x * ldx;
  int64_t amax = 0;
  for (int i = threadIdx.x; i < D; i += 256) {
    const int64_t v = xr[i];
    amax = imax(amax, v < 0 ? -v : v);
  }
  amax = block_max64(amax, sbuf);
  if (threadIdx.x == 0 && amax >= (1LL << 40)) err[0] = 1;
  const int64_t shx = imax(bitlen(imax(amax, 1)) - 25, -6);
  int64_t S = 0;
  for (int i = threadIdx.x; i < D; i += 256) {
    const int64_t xs = rshc(xr[i], shx);
    S = add_wrap(S, mul_wrap(xs, xs));
  }
  S = block_sum64(S, sbuf);
  const int64_t T = add_wrap(S, rshc(kEps60 * (int64_t)D, 60 - 2 * (FR - shx)));
  const int64_t m = fdiv(62 + lg - bitlen(T), 2);
  const int64_t s = 2 * m - lg;
  const int64_t V = s >= 0 ? shl(T, s) : sar(T, -s);
  const int64_t r = isqrt64(V), er = shx - FR - m;
  int64_t emax = kNegBig;
  for (int i = threadIdx.x; i < D; i += 256) {
    const int64_t P = div_round64(mul_wrap(xr[i], gm[i]), ge[i] - FR - er + FN, r);
    Ps[i] = P;
    if (P != 0) emax = imax(emax, bitlen(P < 0 ? -P : P) - FN);
  }
  emax = block_max64(emax, sbuf);
  const int64_t shr = imax(emax - kQB, kNegBig);
  for (int i = threadIdx.x; i < D; i += 256) q[(int64_t)blockIdx.x * ldq + i] = (int32_t)rshc(Ps[i], shr + FN);
  if (threadIdx.x == 0) sh[blockIdx.x] = shr;
}

// ---- segs.softmax (src/bitexact/exact/segs.py:102-105) over ops.softmax_w: key s visible iff s <= qpos ----
__device__ __forceinline__ int64_t weight64(int64_t z, int64_t zshift, const int64_t* lut, int64_t l2e, int fp) {
  int64_t zf = imin(rshc(z, zshift), 48LL << 26);
  const int64_t t = rshc(mul_wrap(zf, l2e), 28);
  const int64_t n = t >> 26, f = t & ((1LL << 26) - 1);
  const int64_t idx = f >> 12, rr = f & 4095;
  const int64_t a = lut[idx];
  const int64_t v = add_wrap(a, rshc(mul_wrap(lut[idx + 1] - a, rr), 12));
  return rshc(v, 60 - fp + n);
}

__global__ __launch_bounds__(256) void softmax_kernel(const int64_t* raw, int64_t ldr, const int64_t* qpos,
                                                      const int64_t* sh, int S, int kbits, const int64_t* lut,
                                                      int64_t l2e, int fp, int32_t* p, int64_t ldp, int64_t* den) {
  __shared__ int64_t sbuf[8];
  const int64_t row = blockIdx.x;
  const int64_t* rr = raw + row * ldr;
  const int64_t qp = qpos[row];
  int64_t mx = kNeg;
  for (int i = threadIdx.x; i < S; i += 256)
    if (i <= qp) mx = imax(mx, rr[i]);
  mx = block_max64(mx, sbuf);
  const int64_t zshift = kbits + 3 - sh[row] - 26;
  int64_t sum = 0;
  for (int i = threadIdx.x; i < S; i += 256) {
    const int64_t w = i <= qp ? weight64(mx - rr[i], zshift, lut, l2e, fp) : 0;
    p[row * ldp + i] = (int32_t)w;
    sum += w;
  }
  sum = block_sum64(sum, sbuf);
  if (threadIdx.x == 0) den[row] = sum;
}

// ---- segs.attn_out (src/bitexact/exact/segs.py:108-113, 187-188): o = div_round(num, FR - FV, den), regrouped to
// one row of H HD values per token, then quantized per row with eps = -FR. Output row o, head hh:
// group = (o / T) HKV + hh / g, query = (hh % g) T + o % T, with g = H / HKV. ----
__global__ __launch_bounds__(256) void attn_out_kernel(const int64_t* num, int64_t sn_group, int64_t sn_query,
                                                       const int64_t* den, int64_t sd_group, int T, int HKV, int g,
                                                       int HD, int FR, int FV, int32_t* q, int64_t ldq, int64_t* sh) {
  extern __shared__ __align__(16) char smem[];
  int64_t* Os = (int64_t*)smem;
  __shared__ int64_t sbuf[8];
  const int o = blockIdx.x;
  const int W = HKV * g * HD;
  int64_t emax = kNegBig;
  for (int c = threadIdx.x; c < W; c += 256) {
    const int hh = c / HD, d = c % HD;
    const int64_t group = (int64_t)(o / T) * HKV + hh / g, query = (int64_t)(hh % g) * T + o % T;
    const int64_t dn = den[group * sd_group + query];   // >= 1 whenever the query sees a key (itself)
    const int64_t v = dn > 0 ? div_round64(num[group * sn_group + query * sn_query + d], FR - FV, dn) : 0;
    Os[c] = v;
    if (v != 0) emax = imax(emax, bitlen(v < 0 ? -v : v) - FR);
  }
  emax = block_max64(emax, sbuf);
  const int64_t shr = imax(emax - kQB, kNegBig);
  for (int c = threadIdx.x; c < W; c += 256) q[(int64_t)o * ldq + c] = (int32_t)rshc(Os[c], shr + FR);
  if (threadIdx.x == 0) sh[o] = shr;
}

}  // namespace bx

using namespace bx;

static void allow_lds_rows(const void* k, size_t lds) {
  if (lds > 64 * 1024) hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

extern "C" int bx_rmsnorm_quant(const int64_t* x, int64_t ldx, const int64_t* gm, const int64_t* ge, int32_t* q,
                                int64_t ldq, int64_t* sh, int32_t M, int32_t D, int32_t FR, int32_t FN, int32_t* err,
                                bx_stream_t stream) {
  int lg = 0;
  while ((1 << lg) < D) ++lg;
  BX_REQUIRE(D > 0 && (1 << lg) == D && lg <= 12, "row length a power of two <= 4096");
  BX_REQUIRE(M >= 0 && ldx >= D && ldq >= D, "bad sizes");
  BX_REQUIRE(x && gm && ge && q && sh && err, "null pointer");
  if (M == 0) return BX_OK;
  const size_t lds = (size_t)D * 8;
  allow_lds_rows((const void*)norm_quant_kernel, lds);
  norm_quant_kernel<<<M, 256, lds, (hipStream_t)stream>>>(x, ldx, gm, ge, q, ldq, sh, D, lg, FR, FN, err);
  return check_launch("norm_quant_kernel");
}

extern "C" int bx_softmax_w(const int64_t* raw, int64_t ldr, const int64_t* qpos, const int64_t* sh, int32_t rows,
                            int32_t S, int32_t kbits, const int64_t* lut, int64_t l2e, int32_t fp, int32_t* p,
                            int64_t ldp, int64_t* den, bx_stream_t stream) {
  BX_REQUIRE(rows >= 0 && S >= 0 && ldr >= S && ldp >= S, "bad sizes");
  BX_REQUIRE(raw && qpos && sh && lut && p && den, "null pointer");
  if (rows == 0) return BX_OK;
  softmax_kernel<<<rows, 256, 0, (hipStream_t)stream>>>(raw, ldr, qpos, sh, S, kbits, lut, l2e, fp, p, ldp, den);
  return check_launch("softmax_kernel");
}

extern "C" int bx_attn_out(const int64_t* num, int64_t sn_group, int64_t sn_query, const int64_t* den,
                           int64_t sd_group, int32_t rows, int32_t T, int32_t HKV, int32_t g, int32_t HD, int32_t FR,
                           int32_t FV, int32_t* q, int64_t ldq, int64_t* sh, bx_stream_t stream) {
  BX_REQUIRE(rows >= 0 && T > 0 && HKV > 0 && g > 0 && HD > 0 && rows % T == 0, "bad sizes");
  BX_REQUIRE(ldq >= (int64_t)HKV * g * HD, "ldq too small");
  BX_REQUIRE(num && den && q && sh, "null pointer");
  if (rows == 0) return BX_OK;
  const size_t lds = (size_t)HKV * g * HD * 8;
  allow_lds_rows((const void*)attn_out_kernel, lds);
  attn_out_kernel<<<rows, 256, lds, (hipStream_t)stream>>>(num, sn_group, sn_query, den, sd_group, T, HKV, g, HD, FR,
                                                          FV, q, ldq, sh);
  return check_launch("attn_out_kernel");
}
