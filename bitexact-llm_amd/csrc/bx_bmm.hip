// Exact batched integer matrix product (bitexact.bmm.bmm, src/bitexact/bmm.py:27-102) on int8 MFMA:
// c int64 [Z, M, N] = a [Z, M, K] @ b [Z, K, N] for int32 or int64 operands with arbitrary strides, each operand taken
// as its first na / nb signed base-256 digits (what the reference's limb split keeps; identical for values within
// the limbs).
//
// A 256-thread block owns 64 rows (512 threads: 128 rows) x up to 16 consecutive 64-column tiles and walks each tile's K in 64-deep steps
// (one flattened sequence, so the next tile's loads overlap this tile's stores; with one k step the A tile is split
// once and kept). Each step's operand tiles are
// loaded four k values per thread (the thread-to-element map follows whichever of the operand's strides is 1, so the loads
// coalesce for q.k with K^T and for p.v alike), split into signed int8 limbs and written to LDS as limb planes
// [limb][row][64 k] (16-byte k chunks XOR-swizzled by row so the MFMA operand reads are conflict-free); the next
// step's values are loaded into registers while the current step's MFMAs run. Wave w computes rows 16 w .. 16 w + 15
// against all 64 columns with v_mfma_i32_16x16x64_i8: limb pair (i, j) accumulates into the int32 set of weight
// s = i + j (|sum| <= 3 K 2^14 < 2^31 for K < 43690, the reference's bound), and the int64 result sum_s c_s 2^(8 s)
// is formed once, in registers, before the store.
#include "bx_common.h"

#include <algorithm>
#include <cstdlib>

namespace bx {

constexpr int kBT = 64;                 // output tile edge, k step
constexpr int kPlane = kBT * kBT;       // bytes of one limb plane of a tile (64 rows x 64 k)

__device__ __forceinline__ int swz(int row, int chunk) { return row * kBT + ((chunk ^ ((row >> 2) & 3)) << 4); }

template <typename T>
__device__ __forceinline__ uint32_t ldv(const T* p, int64_t off, bool ok) { return ok ? (uint32_t)p[off] : 0u; }

// The low 32 bits of the four values (row r, k = k0 + 4 q .. + 3) of one operand (the limb split below reads only
// the low 24); rows past R or k past K read as 0.
template <typename T>
__device__ __forceinline__ void load4(const T* base, int64_t sr, int64_t sk, int r, int R, int k, int K, uint32_t v[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = ldv(base, (int64_t)r * sr + (int64_t)(k + e) * sk, r < R && k + e < K);
}

// Signed limbs of four values, packed by k into one 32-bit word per limb, written to the n limb planes. The first
// n signed base-256 digits of any v are the bytes of v + 0x808080 (mod 2^(8 n)) less 128 each (adding 128 at every
// digit position turns the signed split's floor steps into plain byte extraction), so each plane word is one byte
// gather of the four biased values and an xor.
__device__ __forceinline__ void store4(int8_t* planes, int n, int pstride, int row, int q, const uint32_t v[4]) {
  const uint32_t u0 = v[0] + 0x808080u, u1 = v[1] + 0x808080u, u2 = v[2] + 0x808080u, u3 = v[3] + 0x808080u;
  int8_t* dst = planes + swz(row, q >> 2) + (q & 3) * 4;
  for (int l = 0; l < n; ++l) {
    const uint32_t sel = (uint32_t)l | ((uint32_t)(4 + l) << 8) | 0x0c0c0000u;   // [x.b_l, y.b_l, 0, 0]
    const uint32_t lo = __builtin_amdgcn_perm(u1, u0, sel), hi = __builtin_amdgcn_perm(u3, u2, sel);
    *(uint32_t*)(dst + l * pstride) = __builtin_amdgcn_perm(hi, lo, 0x05040100u) ^ 0x80808080u;
  }
}

// default column tiles per block, walked in sequence (the next tile's loads overlap this one's stores); with two row
// tiles, q.k at config 4: 4 / 8 / 16 / 32 tiles 1.21 / 1.22 / 1.11-1.14 / 1.12 ms, p.v flat
constexpr int kNTI = 16;

// RT row tiles of 64 per block (256 RT threads; wave w computes rows 16 w .. 16 w + 15 of the 64 RT): with RT = 2
// each B tile is loaded and split once for 128 rows.
// PF: operand steps fetched ahead into registers (2: each step's loads have two steps of MFMAs to land behind). The
// step loop runs as PF unrolled substeps with the register set chosen at compile time; at PF = 1 this form took p.v
// at config 4 from 1.24 to 0.90 ms over a plain step loop (same registers, same integers); PF = 2 measured 0.88-0.89.
template <typename TA, typename TB, int NA, int NB, bool A1, int RT, int PF>
__global__ __launch_bounds__(256 * RT) void bmm_mfma_kernel(const TA* a, int64_t saz, int64_t sam, int64_t sak,
                                                            const TB* b, int64_t sbz, int64_t sbk, int64_t sbn,
                                                            int64_t* c, int64_t scz, int64_t scm, int64_t scn, int M,
                                                            int N, int K, int nti) {
  constexpr int NS = NA + NB - 1, NT = 256 * RT, AP = kPlane * RT, GB = 4 / RT;   // B load groups per thread
  __shared__ __align__(16) int8_t As[NA * AP];
  __shared__ __align__(16) int8_t Bs[NB * kPlane];
  const int64_t z = blockIdx.z;
  const int m0 = blockIdx.y * kBT * RT, nb0 = blockIdx.x * kBT * nti;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const TA* ab = a + z * saz;
  const TB* bb = b + z * sbz;
  // thread -> (row, k quad) of the load groups (A: 64 RT rows, 4 groups; B: 64 rows, GB groups); k-major when k is
  // the contiguous stride
  const bool a_k = sak == 1, b_k = sbk == 1;
  int ar[4], aq[4], br[GB], bq[GB];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int idx = tid + NT * g;
    ar[g] = a_k ? idx / 16 : idx % (64 * RT);
    aq[g] = a_k ? idx % 16 : idx / (64 * RT);
  }
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const int idx = tid + NT * g;
    br[g] = b_k ? idx / 16 : idx % 64;
    bq[g] = b_k ? idx % 16 : idx / 64;
  }
  // steps: (column tile j, k step) flattened, j outer
  const int ksteps = max(1, (K + kBT - 1) / kBT);
  const int ntile = min(nti, (N - nb0 + kBT - 1) / kBT);
  const int nsteps = ntile * ksteps;
  uint32_t va[PF][4][4], vb[PF][GB][4];
  // A1 (one k step, K <= 64, e.g. q.k over a head dimension): the A tile is the same for every column tile, so its
  // limb planes are loaded and split once and stay in LDS
  constexpr bool a_once = A1;
  auto fetch = [&](int st, uint32_t (&fa4)[4][4], uint32_t (&fb4)[GB][4]) {
    const int j = st / ksteps, k0 = (st % ksteps) * kBT;
    const bool fa = !a_once || st == 0;   // block-uniform
#pragma unroll
    for (int g = 0; g < 4; ++g)
      if (fa) load4(ab, sam, sak, m0 + ar[g], M, k0 + 4 * aq[g], K, fa4[g]);
#pragma unroll
    for (int g = 0; g < GB; ++g) load4(bb, sbn, sbk, nb0 + j * kBT + br[g], N, k0 + 4 * bq[g], K, fb4[g]);
  };
  v4i acc[NS][4];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[s][cb] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int h = 0; h < PF; ++h)
    if (h < nsteps) fetch(h, va[h], vb[h]);
  const int r16 = lane & 15, ch = lane >> 4;
  for (int st0 = 0; st0 < nsteps; st0 += PF)
#pragma unroll
  for (int h = 0; h < PF; ++h) {
    const int st = st0 + h;
    if (st >= nsteps) break;              // block-uniform
    const bool sa = !a_once || st == 0;   // block-uniform
#pragma unroll
    for (int g = 0; g < 4; ++g)
      if (sa) store4(As, NA, AP, ar[g], aq[g], va[h][g]);
#pragma unroll
    for (int g = 0; g < GB; ++g) store4(Bs, NB, kPlane, br[g], bq[g], vb[h][g]);
    __syncthreads();
    if (st + PF < nsteps) fetch(st + PF, va[h], vb[h]);   // later steps' values travel while this step's MFMAs run
    v4i af[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) af[i] = *(const v4i*)(As + i * AP + swz(16 * wave + r16, ch));
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const v4i bf = *(const v4i*)(Bs + j * kPlane + swz(16 * cb + r16, ch));
#pragma unroll
        for (int i = 0; i < NA; ++i)
          acc[i + j][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf, acc[i + j][cb], 0, 0, 0);
      }
    __syncthreads();
    if (st % ksteps != ksteps - 1) continue;
    // the column tile is complete: lane l holds column 16 cb + l % 16, rows 4 (l / 16) + e of the wave's 16 rows
    const int n0 = nb0 + (st / ksteps) * kBT;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const int n = n0 + 16 * cb + r16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * wave + 4 * ch + e;
        int64_t v = 0;
#pragma unroll
        for (int s = 0; s < NS; ++s) v += (int64_t)acc[s][cb][e] << (8 * s);
        if (m < M && n < N) {
          c[z * scz + (int64_t)m * scm + (int64_t)n * scn] = v;
        }
      }
#pragma unroll
      for (int s = 0; s < NS; ++s) acc[s][cb] = v4i{0, 0, 0, 0};
    }
  }
}

template <typename TA, typename TB, int NA, bool A1, int RT, int PF>
static void launch_nb(int nb, dim3 grid, hipStream_t st, const TA* a, int64_t saz, int64_t sam, int64_t sak,
                      const TB* b, int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz, int64_t scm,
                      int64_t scn, int M, int N, int K, int nti) {
  if (nb == 1)
    bmm_mfma_kernel<TA, TB, NA, 1, A1, RT, PF><<<grid, 256 * RT, 0, st>>>(a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else if (nb == 2)
    bmm_mfma_kernel<TA, TB, NA, 2, A1, RT, PF><<<grid, 256 * RT, 0, st>>>(a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else
    bmm_mfma_kernel<TA, TB, NA, 3, A1, RT, PF><<<grid, 256 * RT, 0, st>>>(a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
}

template <typename TA, typename TB, bool A1, int RT, int PF>
static void launch_na(int na, int nb, dim3 grid, hipStream_t st, const void* a, int64_t saz, int64_t sam, int64_t sak,
                      const void* b, int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz, int64_t scm,
                      int64_t scn, int M, int N, int K, int nti) {
  const TA* A = (const TA*)a;
  const TB* B = (const TB*)b;
  if (na == 1) launch_nb<TA, TB, 1, A1, RT, PF>(nb, grid, st, A, saz, sam, sak, B, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else if (na == 2) launch_nb<TA, TB, 2, A1, RT, PF>(nb, grid, st, A, saz, sam, sak, B, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else launch_nb<TA, TB, 3, A1, RT, PF>(nb, grid, st, A, saz, sam, sak, B, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
}

// one k step (K <= 64): the A tile's limb planes are formed once per block; from 128 rows, blocks of two row tiles
// (config-4 shapes: q.k 1.17-1.24 vs 1.80-1.84 ms, p.v 1.25 vs 1.41; four row tiles: 1.25 / 1.39). BX_BMM_RT=1
// keeps one row tile (experiments; the same integers either way).
template <typename TA, typename TB, bool A1>
static void launch_rt(int na, int nb, dim3 grid, hipStream_t st, const void* a, int64_t saz, int64_t sam, int64_t sak,
                      const void* b, int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz, int64_t scm,
                      int64_t scn, int M, int N, int K, int nti) {
  static const int rt_env = getenv("BX_BMM_RT") ? atoi(getenv("BX_BMM_RT")) : 2;
  static const int pf_env = getenv("BX_BMM_PF") ? atoi(getenv("BX_BMM_PF")) : 1;   // 2: experiments
  if (rt_env == 2 && M >= 2 * kBT) {
    grid.y = (M + 2 * kBT - 1) / (2 * kBT);
    if (!A1 && pf_env == 2)
      launch_na<TA, TB, A1, 2, 2>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
    else
      launch_na<TA, TB, A1, 2, 1>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  } else {
    launch_na<TA, TB, A1, 1, 1>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  }
}

template <typename TA, typename TB>
static void launch_k(int na, int nb, dim3 grid, hipStream_t st, const void* a, int64_t saz, int64_t sam, int64_t sak,
                     const void* b, int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz, int64_t scm,
                     int64_t scn, int M, int N, int K, int nti) {
  if (K <= kBT)
    launch_rt<TA, TB, true>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else
    launch_rt<TA, TB, false>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
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
  // BX_BMM_NTI: column tiles per block (experiments; the same integers for any value)
  static const int nti_env = getenv("BX_BMM_NTI") ? atoi(getenv("BX_BMM_NTI")) : kNTI;
  const int nti = std::max(1, std::min(nti_env, 64));
  const dim3 grid((N + kBT * nti - 1) / (kBT * nti), (M + kBT - 1) / kBT, Z);
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) {   // an empty sum: zeros (one step per column tile over a zero-length K reads nothing)
    bmm_mfma_kernel<int32_t, int32_t, 1, 1, false, 1, 1><<<grid, 256, 0, st>>>((const int32_t*)a, saz, sam, sak, (const int32_t*)b,
                                                                  sbz, sbk, sbn, c, scz, scm, scn, M, N, 0, nti);
    return check_launch("bmm_mfma_kernel");
  }
  if (a_bytes == 4 && b_bytes == 4)
    launch_k<int32_t, int32_t>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else if (a_bytes == 4)
    launch_k<int32_t, int64_t>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else if (b_bytes == 4)
    launch_k<int64_t, int32_t>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  else
    launch_k<int64_t, int64_t>(na, nb, grid, st, a, saz, sam, sak, b, sbz, sbk, sbn, c, scz, scm, scn, M, N, K, nti);
  return check_launch("bmm_mfma_kernel");
}
