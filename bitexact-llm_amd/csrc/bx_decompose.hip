// bf16 weight -> exact 3-limb dense part + sparse residual, on the device.
//
// consts.decompose (src/bitexact/exact/consts.py:67-107) per output row n: w = sm 2^ex (bf16_parts), row grid
// g = smallest exponent with max |W| <= LIM3 where W = sign trunc(|sm| 2^(ex - g)); the bits dropped by the
// truncation form the residual R on the finer grid gf = min(g, lowest residual bit), d = g - gf <= 30.
// W 2^g + R 2^gf == w exactly. One 256-thread block per row; pass 1 writes limbs / g / d / counts, pass 2
// (after the host has sized R = max count) writes the residual in ELL order (k ascending).
#include "bx_common.h"

namespace bx {

struct Bf16 {
  int64_t mag, ex;
  bool neg, bad;
};

// consts.bf16_parts (src/bitexact/exact/consts.py:33-42)
__device__ __forceinline__ Bf16 bf16_parts(uint16_t b) {
  Bf16 r;
  const int e = (b >> 7) & 0xFF, m = b & 0x7F;
  r.bad = e == 255;
  r.mag = e > 0 ? (m | 0x80) : m;
  r.ex = (int64_t)(e > 0 ? e : 1) - 134;
  r.neg = (b >> 15) == 1;
  return r;
}

__device__ __forceinline__ int64_t lowbit9(int64_t x) { return x ? __ffsll((unsigned long long)x) - 1 : 99; }

template <typename T, typename F>
__device__ T block_reduce(T v, F op, T* sbuf) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if (lane == 0) sbuf[wave] = v;
  __syncthreads();
  T r = sbuf[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = op(r, sbuf[i]);
  __syncthreads();
  return r;
}

struct RowGrid {
  int64_t g, gf;
};

// The row's grid g and residual grid gf (shared by both passes).
__device__ RowGrid row_grid(const uint16_t* wr, int K, int* errp, int64_t* sbuf) {
  int64_t top = -1000000;
  int badw = 0;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const Bf16 v = bf16_parts(wr[k]);
    badw |= v.bad;
    if (v.mag > 0) top = imax(top, v.ex + bitlen(v.mag));
  }
  top = block_reduce<int64_t>(top, [](int64_t a, int64_t b) { return imax(a, b); }, sbuf);
  int64_t g = top - 23;
  // one increment at most: every |W| < 2^(top - g) = 2^23, and after g + 1 every |W| < 2^22 <= LIM3
  int64_t big = 0;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const Bf16 v = bf16_parts(wr[k]);
    const int64_t s = imin(v.ex - g, 40);
    if (v.mag > 0 && s >= 0 && shl(v.mag, s) > kLim3) big = 1;
  }
  big = block_reduce<int64_t>(big, [](int64_t a, int64_t b) { return a | b; }, sbuf);
  g += big;
  if (top < -100000) g = 0;
  int64_t low = 1000000;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const Bf16 v = bf16_parts(wr[k]);
    const int64_t s = v.ex - g;
    if (s < 0) {
      const int64_t sc = imin(-s, 40);
      const int64_t rmag = v.mag - ((v.mag >> sc) << sc);
      if (rmag > 0) low = imin(low, v.ex + lowbit9(rmag));
    }
  }
  low = block_reduce<int64_t>(low, [](int64_t a, int64_t b) { return imin(a, b); }, sbuf);
  const int64_t bw = block_reduce<int64_t>((int64_t)badw, [](int64_t a, int64_t b) { return a | b; }, sbuf);
  if (bw && threadIdx.x == 0) errp[0] = 1;
  RowGrid r;
  r.g = g;
  r.gf = imin(low, g);
  return r;
}

__global__ __launch_bounds__(256) void decompose_rows_kernel(const uint16_t* w, int N, int K, int8_t* limbs,
                                                             int64_t* g_out, int64_t* d_out, int32_t* cnt,
                                                             int32_t* err) {
  __shared__ int64_t sbuf[8];
  const int n = blockIdx.x;
  const uint16_t* wr = w + (int64_t)n * K;
  const RowGrid rg = row_grid(wr, K, err, sbuf);
  int64_t c = 0;
  const int64_t plane = (int64_t)N * K;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const Bf16 v = bf16_parts(wr[k]);
    const int64_t s = v.ex - rg.g;
    int64_t dmag, rmag = 0;
    if (s >= 0) {
      dmag = shl(v.mag, imin(s, 40));
    } else {
      const int64_t sc = imin(-s, 40);
      dmag = v.mag >> sc;
      rmag = v.mag - (dmag << sc);
    }
    c += rmag > 0;
    int64_t W = v.neg ? -dmag : dmag;
    int8_t* o = limbs + (int64_t)n * K + k;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int64_t lo = limb_lo64(W);
      o[i * plane] = (int8_t)lo;
      W = (W - lo) >> 8;
    }
  }
  c = block_reduce<int64_t>(c, [](int64_t a, int64_t b) { return a + b; }, sbuf);
  if (threadIdx.x == 0) {
    const int64_t d = rg.g - rg.gf;
    g_out[n] = rg.g;
    d_out[n] = d;
    cnt[n] = (int32_t)c;
    if (d > 30 || d < 0) err[0] = 1;
  }
}

__global__ __launch_bounds__(256) void decompose_residual_kernel(const uint16_t* w, int N, int K, const int64_t* g,
                                                                 const int64_t* d, int32_t* ecol, int64_t* evalv,
                                                                 int R) {
  __shared__ int32_t scan[256];
  const int n = blockIdx.x, t = threadIdx.x;
  const uint16_t* wr = w + (int64_t)n * K;
  const int64_t gn = g[n], gf = gn - d[n];
  const int chunk = (K + 255) / 256;
  const int kb = t * chunk, ke = min(K, kb + chunk);
  int mine = 0;
  for (int k = kb; k < ke; ++k) {
    const Bf16 v = bf16_parts(wr[k]);
    const int64_t s = v.ex - gn;
    if (s < 0) {
      const int64_t sc = imin(-s, 40);
      mine += (v.mag - ((v.mag >> sc) << sc)) > 0;
    }
  }
  scan[t] = mine;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {   // inclusive Hillis-Steele scan
    const int add = t >= o ? scan[t - o] : 0;
    __syncthreads();
    scan[t] += add;
    __syncthreads();
  }
  int j = scan[t] - mine;
  const int total = scan[255];
  for (int k = kb; k < ke; ++k) {
    const Bf16 v = bf16_parts(wr[k]);
    const int64_t s = v.ex - gn;
    if (s < 0) {
      const int64_t sc = imin(-s, 40);
      const int64_t rmag = v.mag - ((v.mag >> sc) << sc);
      if (rmag > 0) {
        const int64_t rs = v.ex - gf;
        int64_t rv = rs >= 0 ? shl(rmag, rs) : (rmag >> imin(-rs, 63));
        if (v.neg) rv = -rv;
        if (j < R) {
          ecol[(int64_t)n * R + j] = k;
          evalv[(int64_t)n * R + j] = rv;
        }
        ++j;
      }
    }
  }
  for (int jj = total + t; jj < R; jj += 256) {
    ecol[(int64_t)n * R + jj] = 0;
    evalv[(int64_t)n * R + jj] = 0;
  }
}

}  // namespace bx

using namespace bx;

extern "C" int bx_decompose_rows(const uint16_t* w, int32_t N, int32_t K, int8_t* limbs, int64_t* g, int64_t* d,
                                 int32_t* cnt, int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(N >= 0 && K >= 0, "negative size");
  BX_REQUIRE(w && limbs && g && d && cnt && err, "null pointer");
  if (N == 0) return BX_OK;
  decompose_rows_kernel<<<N, 256, 0, (hipStream_t)stream>>>(w, N, K, limbs, g, d, cnt, err);
  return check_launch("decompose_rows_kernel");
}

extern "C" int bx_decompose_residual(const uint16_t* w, int32_t N, int32_t K, const int64_t* g, const int64_t* d,
                                     int32_t* ell_col, int64_t* ell_val, int32_t R, bx_stream_t stream) {
  BX_REQUIRE(N >= 0 && K >= 0 && R >= 0, "negative size");
  if (N == 0 || R == 0) return BX_OK;
  BX_REQUIRE(w && g && d && ell_col && ell_val, "null pointer");
  decompose_residual_kernel<<<N, 256, 0, (hipStream_t)stream>>>(w, N, K, g, d, ell_col, ell_val, R);
  return check_launch("decompose_residual_kernel");
}
