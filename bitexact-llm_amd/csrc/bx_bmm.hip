// Exact batched integer matrix product (bitexact.bmm.bmm, src/bitexact/bmm.py:27-102):
// c int64 [Z, M, N] = a [Z, M, K] @ b [Z, K, N] for int32 or int64 operands with arbitrary strides, each operand
// taken as its first na / nb signed base-256 digits (what the reference's limb split keeps; identical for
// values within the limbs). 64 x 64 output tiles per 256-thread block, 32-deep K tiles in LDS, exact int64
// multiply-adds (every product of two 3-limb values is below 2^47, K < 43690 keeps the sums below 2^63).
#include "bx_common.h"

namespace bx {

__device__ __forceinline__ int64_t keep_limbs(int64_t x, int n) {
  int64_t r = x, v = 0;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (i < n) {
      const int64_t lo = limb_lo64(r);
      v += lo << (8 * i);
      r = (r - lo) >> 8;
    }
  }
  return v;
}

template <typename TA, typename TB>
__global__ __launch_bounds__(256) void bmm_kernel(const TA* a, int64_t saz, int64_t sam, int64_t sak, const TB* b,
                                                  int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz,
                                                  int64_t scm, int64_t scn, int M, int N, int K, int na, int nb) {
  __shared__ int32_t As[32][65];   // [k][m]
  __shared__ int32_t Bs[32][65];   // [k][n]
  const int64_t z = blockIdx.z;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tid = threadIdx.x, tm = tid / 16, tn = tid % 16;   // 4 x 4 outputs per thread
  int64_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0;
  for (int k0 = 0; k0 < K; k0 += 32) {
    __syncthreads();
    for (int u = tid; u < 32 * 64; u += 256) {
      const int kk = u / 64, mm = u % 64;
      const int m = m0 + mm, k = k0 + kk;
      As[kk][mm] = (m < M && k < K) ? (int32_t)keep_limbs((int64_t)a[z * saz + (int64_t)m * sam + (int64_t)k * sak], na) : 0;
      const int n = n0 + mm;
      Bs[kk][mm] = (n < N && k < K) ? (int32_t)keep_limbs((int64_t)b[z * sbz + (int64_t)k * sbk + (int64_t)n * sbn], nb) : 0;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < 32; ++kk) {
      int64_t av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][tm + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tn + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + tm + 16 * i, n = n0 + tn + 16 * j;
      if (m < M && n < N) c[z * scz + (int64_t)m * scm + (int64_t)n * scn] = acc[i][j];
    }
}

}  // namespace bx

using namespace bx;

extern "C" int bx_limb_bmm(const void* a, int32_t a_bytes, int64_t saz, int64_t sam, int64_t sak, const void* b,
                           int32_t b_bytes, int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz, int64_t scm,
                           int64_t scn, int32_t Z, int32_t M, int32_t N, int32_t K, int32_t na, int32_t nb,
                           bx_stream_t stream) {
  BX_REQUIRE(Z >= 0 && M >= 0 && N >= 0 && K >= 0, "negative size");
  BX_REQUIRE(K < 43690, "K must stay below 43690");
  BX_REQUIRE(na >= 1 && na <= 3 && nb >= 1 && nb <= 3, "limbs per operand in [1, 3]");
  BX_REQUIRE((a_bytes == 4 || a_bytes == 8) && (b_bytes == 4 || b_bytes == 8), "operands must be int32 or int64");
  BX_REQUIRE(Z <= 65535, "Z <= 65535");
  if (Z == 0 || M == 0 || N == 0) return BX_OK;
  BX_REQUIRE(a && b && c, "null pointer");
  dim3 grid((N + 63) / 64, (M + 63) / 64, Z);
  hipStream_t st = (hipStream_t)stream;
  if (a_bytes == 4 && b_bytes == 4)
    bmm_kernel<int32_t, int32_t><<<grid, 256, 0, st>>>((const int32_t*)a, saz, sam, sak, (const int32_t*)b, sbz, sbk,
                                                      sbn, c, scz, scm, scn, M, N, K, na, nb);
  else if (a_bytes == 4)
    bmm_kernel<int32_t, int64_t><<<grid, 256, 0, st>>>((const int32_t*)a, saz, sam, sak, (const int64_t*)b, sbz, sbk,
                                                      sbn, c, scz, scm, scn, M, N, K, na, nb);
  else if (b_bytes == 4)
    bmm_kernel<int64_t, int32_t><<<grid, 256, 0, st>>>((const int64_t*)a, saz, sam, sak, (const int32_t*)b, sbz, sbk,
                                                      sbn, c, scz, scm, scn, M, N, K, na, nb);
  else
    bmm_kernel<int64_t, int64_t><<<grid, 256, 0, st>>>((const int64_t*)a, saz, sam, sak, (const int64_t*)b, sbz, sbk,
                                                      sbn, c, scz, scm, scn, M, N, K, na, nb);
  return check_launch("bmm_kernel");
}
