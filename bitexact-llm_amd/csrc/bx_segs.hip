// Element-wise segments between the matrix products:
//  * exact mode: RoPE of the qkv linear output, per-(token, head) quantization of q and the regroup by KV head,
//    fused in one pass (segs.rope_y + segs.q_group, src/bitexact/exact/segs.py:66-99);
//  * int8 mode: per-row quantization of the GEMM input with the limbs written as the stacked int8 rows the
//    GEMM reads (int8.ops.quant_rows + intops.stack_limbs, src/bitexact/int8/ops.py:24-35,
//    src/bitexact/intops.py:73-79), and the linear post-segment (int8.segs.post, src/bitexact/int8/segs.py:62-67).
// All arithmetic is int64 with the reference's wrapping and shift rules; every reduction is a maximum.
#include "bx_common.h"
#include "bx_rope.h"

namespace bx {


// intops.rdiv (src/bitexact/intops.py:41-43): floor((2a + b) / (2b)), b > 0.
__device__ __forceinline__ int64_t rdiv64(int64_t a, int64_t b) { return fdiv(add_wrap(2 * a, b), 2 * b); }

__device__ __forceinline__ int64_t seg_block_max(int64_t v, int64_t* sbuf) {
  v = wave_max64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) sbuf[wave] = v;
  __syncthreads();
  int64_t r = sbuf[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = imax(r, sbuf[i]);
  return r;
}

// Grid (token, head-row group of 4): wave w of block (token, j) takes head row 4 j + w (one row per wave, so the
// rows' loads are in flight together instead of one row after another); lane l holds dims l + 64 e.
template <int HD>
__global__ __launch_bounds__(256) void rope_qgroup_kernel(RopeArgs p) {
  constexpr int E = HD / 64;
  const int token = blockIdx.x, b = token / p.T, t = token - b * p.T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t pos_raw = p.pos[(int64_t)b * p.spb + (int64_t)t * p.spt];
  bool bad = pos_raw < 0 || pos_raw >= p.npos;          // the reference's table index would fail: flagged
  const int64_t pos = imin(imax(pos_raw, 0), p.npos - 1);
  const int g = p.H / p.HKV, rows = p.H + 2 * p.HKV;
  const int64_t eps = -(int64_t)(p.FR + p.FT);
  for (int hr = blockIdx.y * 4 + wave; hr < rows && hr < (int)blockIdx.y * 4 + 4; hr += 4) {
    int64_t out[E];
    rope_row<HD>(p, token, hr, pos, lane, out, bad);
    if (hr < p.H) {
      // q head: quantized, stored at its grouped row
      const int64_t shq = rope_q_shift<HD>(p, out, bad);
      const int kvh = hr / g, gi = hr - kvh * g;
      const int64_t row = ((int64_t)b * p.HKV + kvh) * ((int64_t)g * p.T) + (int64_t)gi * p.T + t;
#pragma unroll
      for (int e = 0; e < E; ++e) p.qg[row * HD + lane + 64 * e] = (int32_t)rshc(out[e], shq - eps);
      if (lane == 0) p.shg[row] = shq;
    } else {
      rope_kv_store<HD>(p, token, hr, lane, out, bad);
    }
  }
  if (wave_or(bad ? 1 : 0) && lane == 0) p.err[0] = 1;
}

// int8 quant_rows + stack_limbs: one block per row. amax is brought to 30 bits (sh), as_ = rsh(amax, sh),
// q = rdiv(rsh(z, sh) qmax, as_); limb i of q[m] goes to stacked row i M + m. With mant / e given, also the
// row scale of segs.pre_plain: (mant, e) = norm24(as_, sh - FR) (src/bitexact/int8/segs.py:56-59,
// src/bitexact/int8/ops.py:73-76).
__global__ __launch_bounds__(256) void int8_quant_rows_kernel(const int64_t* z, int64_t ldz, int M, int K, int nl,
                                                              int FR, int8_t* a, int64_t* as_out, int64_t* sh_out,
                                                              int64_t* mant, int64_t* e) {
  __shared__ int64_t sbuf[4];
  const int m = blockIdx.x;
  const int64_t* zr = z + (int64_t)m * ldz;
  int64_t amax = 0;
  for (int k = threadIdx.x; k < K; k += 256) {
    const int64_t x = zr[k];
    amax = imax(amax, x < 0 ? -x : x);
  }
  amax = imax(seg_block_max(amax, sbuf), 1);
  const int64_t sh = bitlen(amax) - 30;
  const int64_t as = rsh64(amax, sh);
  const int64_t qmax = 127LL << (8 * (nl - 1));
  for (int k = threadIdx.x; k < K; k += 256) {
    int64_t r = rdiv64(mul_wrap(rsh64(zr[k], sh), qmax), as);
    for (int i = 0; i < nl; ++i) {
      const int64_t lo = limb_lo64(r);
      a[((int64_t)i * M + m) * K + k] = (int8_t)lo;
      r = (r - lo) >> 8;
    }
  }
  if (threadIdx.x == 0) {
    as_out[m] = as;
    sh_out[m] = sh;
    if (mant) {
      const int64_t b = bitlen(as) - 24;
      mant[m] = rsh64(as, b);
      e[m] = sh - FR + b;
    }
  }
}

// int8.segs.post: t = rsh(acc m_c, fmsh) (flag when |t| >= 2^38), y = rsh(t mant_r, 24 - FR - e_r).
__global__ __launch_bounds__(256) void int8_post_kernel(const int64_t* acc, int64_t ldacc, const int64_t* mc, int fmsh,
                                                        const int64_t* mant, const int64_t* e, int FR, int64_t* y,
                                                        int64_t ldy, int M, int N, int32_t* flag) {
  const int64_t total = (int64_t)M * N;
  bool big = false;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
    const int64_t t = rsh64(mul_wrap(acc[(int64_t)m * ldacc + n], mc[n]), fmsh);
    big |= t >= (1LL << 38) || t <= -(1LL << 38);
    y[(int64_t)m * ldy + n] = rsh64(mul_wrap(t, mant[m]), 24 - FR - e[m]);
  }
  if (wave_or(big ? 1 : 0) && (threadIdx.x & 63) == 0) flag[0] = 1;
}

// wmm.epilogue over segs.lin_y's inputs (src/bitexact/exact/wmm.py:132-150, src/bitexact/exact/segs.py:25-32):
// T = sum of the split partials, B = dense residual or the ELL gather sum_j q[m, ec[n, j]] ev[n, j], then the
// one rounding at p = sh[m] + g[n] - d[n] + FR; flag[0] = 1 where the checked rule fails.
__global__ __launch_bounds__(256) void exact_epilogue_kernel(const int64_t* T, int64_t ldt, int64_t sts, int nsplit,
                                                             const int64_t* B, int64_t ldb, const int32_t* q,
                                                             int64_t ldq, int K, const int32_t* ec, const int64_t* ev,
                                                             int R, const int64_t* d, const int64_t* g,
                                                             const int64_t* sh, int FR, int checked, int64_t* y,
                                                             int64_t ldy, int M, int N, int32_t* flag) {
  const int64_t total = (int64_t)M * N;
  bool bad_any = false, corrupt = false;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
    int64_t t = 0;
    for (int s = 0; s < nsplit; ++s) t = add_wrap(t, T[s * sts + (int64_t)m * ldt + n]);
    int64_t b = 0;
    if (B) {
      b = B[(int64_t)m * ldb + n];
    } else {
      for (int j = 0; j < R; ++j) {
        // valid ELL columns are in [0, K); a corrupt one reads column 0 and raises the flag
        const uint32_t c0 = (uint32_t)ec[(int64_t)n * R + j];
        const bool out = c0 >= (uint32_t)K;
        corrupt |= out;
        const int c = out ? 0 : (int)c0;
        b = add_wrap(b, mul_wrap((int64_t)q[(int64_t)m * ldq + c], ev[(int64_t)n * R + j]));
      }
    }
    const int64_t dn = d[n];
    bool bad;
    y[(int64_t)m * ldy + n] = exact_round(t, b, dn, sh[m] + g[n] - dn + FR, bad);
    bad_any |= bad;
  }
  if (wave_or(((checked && bad_any) || corrupt) ? 1 : 0) && flag != nullptr && (threadIdx.x & 63) == 0) flag[0] = 1;
}

}  // namespace bx

using namespace bx;

static int rope_common(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spb, int64_t spt,
                       const int64_t* cos, const int64_t* sin, int32_t npos, int32_t B, int32_t T, int32_t H,
                       int32_t HKV, int32_t HD, int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ,
                       int32_t* qg, int64_t* shg, int64_t* k, int64_t* v, int32_t* err, int8_t* cache, int64_t sc_nb,
                       int64_t sc_h, int64_t sc_bs, const int64_t* slot, int32_t bs, hipStream_t stream);

extern "C" int bx_rope_qgroup(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spb, int64_t spt,
                              const int64_t* cos, const int64_t* sin, int32_t npos, int32_t B, int32_t T, int32_t H,
                              int32_t HKV, int32_t HD, int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ,
                              int32_t* qg, int64_t* shg, int64_t* k, int64_t* v, int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(k && v, "null pointer");
  return rope_common(y, ldy, pos, spb, spt, cos, sin, npos, B, T, H, HKV, HD, FR, FT, FK, FV, FZ, qg, shg, k, v, err,
                     nullptr, 0, 0, 0, nullptr, 1, (hipStream_t)stream);
}

extern "C" int bx_rope_qgroup_store(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spb, int64_t spt,
                                    const int64_t* cos, const int64_t* sin, int32_t npos, int32_t B, int32_t T,
                                    int32_t H, int32_t HKV, int32_t HD, int32_t FR, int32_t FT, int32_t FK, int32_t FV,
                                    int32_t FZ, int32_t* qg, int64_t* shg, int64_t* k, int64_t* v, int8_t* cache,
                                    int64_t sc_nb, int64_t sc_h, int64_t sc_bs, const int64_t* slot, int32_t bs,
                                    int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(cache && slot && bs > 0, "null cache / slot");
  BX_REQUIRE(sc_bs >= 8LL * HD && sc_h >= (int64_t)bs * sc_bs && sc_nb >= (int64_t)HKV * sc_h, "cache strides");
  return rope_common(y, ldy, pos, spb, spt, cos, sin, npos, B, T, H, HKV, HD, FR, FT, FK, FV, FZ, qg, shg, k, v, err,
                     cache, sc_nb, sc_h, sc_bs, slot, bs, (hipStream_t)stream);
}

static int rope_common(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spb, int64_t spt,
                       const int64_t* cos, const int64_t* sin, int32_t npos, int32_t B, int32_t T, int32_t H,
                       int32_t HKV, int32_t HD, int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ,
                       int32_t* qg, int64_t* shg, int64_t* k, int64_t* v, int32_t* err, int8_t* cache, int64_t sc_nb,
                       int64_t sc_h, int64_t sc_bs, const int64_t* slot, int32_t bs, hipStream_t stream) {
  BX_REQUIRE(B >= 0 && T >= 0 && H > 0 && HKV > 0 && H % HKV == 0, "bad head counts");
  BX_REQUIRE(HD == 64 || HD == 128, "head_dim 64 or 128");
  BX_REQUIRE(ldy >= (int64_t)(H + 2 * HKV) * HD, "ldy too small");
  BX_REQUIRE(npos > 0, "empty rope tables");
  if (B == 0 || T == 0) return BX_OK;
  BX_REQUIRE(y && pos && cos && sin && qg && shg && err, "null pointer");
  RopeArgs p = {y, ldy, pos, spb, spt, cos, sin, npos, B, T, H, HKV, HD, FR, FT, FK, FV, FZ, qg, shg, k, v, err,
                cache, sc_nb, sc_h, sc_bs, slot, bs};
  const dim3 blocks(B * T, (H + 2 * HKV + 3) / 4);
  if (HD == 64)
    rope_qgroup_kernel<64><<<blocks, 256, 0, (hipStream_t)stream>>>(p);
  else
    rope_qgroup_kernel<128><<<blocks, 256, 0, (hipStream_t)stream>>>(p);
  return check_launch("rope_qgroup_kernel");
}

extern "C" int bx_int8_quant_rows(const int64_t* z, int64_t ldz, int32_t M, int32_t K, int32_t nl, int32_t FR,
                                  int8_t* a, int64_t* as_, int64_t* sh, int64_t* mant, int64_t* e,
                                  bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && K >= 0 && ldz >= K, "bad sizes");
  BX_REQUIRE(nl >= 1 && nl <= 3, "nl must be 1, 2 or 3");
  if (M == 0) return BX_OK;
  BX_REQUIRE(z && a && as_ && sh, "null pointer");
  BX_REQUIRE((mant == nullptr) == (e == nullptr), "mant and e come together");
  int8_quant_rows_kernel<<<M, 256, 0, (hipStream_t)stream>>>(z, ldz, M, K, nl, FR, a, as_, sh, mant, e);
  return check_launch("int8_quant_rows_kernel");
}

extern "C" int bx_int8_post(const int64_t* acc, int64_t ldacc, const int64_t* m, int32_t fmsh, const int64_t* mant,
                            const int64_t* e, int32_t FR, int64_t* y, int64_t ldy, int32_t M, int32_t N, int32_t* flag,
                            bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && N >= 0 && ldacc >= N && ldy >= N, "bad sizes");
  if (M == 0 || N == 0) return BX_OK;
  BX_REQUIRE(acc && m && mant && e && y && flag, "null pointer");
  const int64_t total = (int64_t)M * N;
  const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  int8_post_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(acc, ldacc, m, fmsh, mant, e, FR, y, ldy, M, N, flag);
  return check_launch("int8_post_kernel");
}

extern "C" int bx_exact_epilogue(const int64_t* T, int64_t ldt, int64_t sts, int32_t nsplit, const int64_t* B,
                                 int64_t ldb, const int32_t* q, int64_t ldq, int32_t K, const int32_t* ell_col,
                                 const int64_t* ell_val, int32_t R, const int64_t* d, const int64_t* g,
                                 const int64_t* sh, int32_t FR, int32_t checked, int64_t* y, int64_t ldy, int32_t M,
                                 int32_t N, int32_t* flag, bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && N >= 0 && nsplit >= 1 && ldt >= N && ldy >= N, "bad sizes");
  BX_REQUIRE(B == nullptr || ldb >= N, "ldb too small");
  BX_REQUIRE(B != nullptr || R == 0 || (q && ell_col && ell_val && K > 0 && ldq >= K), "residual missing");
  BX_REQUIRE(!checked || flag, "checked needs a flag pointer");
  if (M == 0 || N == 0) return BX_OK;
  BX_REQUIRE(T && d && g && sh && y, "null pointer");
  const int64_t total = (int64_t)M * N;
  const int blocks = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  exact_epilogue_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(T, ldt, sts, nsplit, B, ldb, q, ldq, K, ell_col,
                                                                ell_val, B ? 0 : R, d, g, sh, FR, checked, y, ldy, M,
                                                                N, flag);
  return check_launch("exact_epilogue_kernel");
}
