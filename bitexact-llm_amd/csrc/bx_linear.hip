// Exact-mode limb GEMM and int8-mode GEMM for gfx950.
//
// Two kernel families share one epilogue:
//  * skinny_kernel (decode, <= 64 stacked activation rows): the limb rows of the activations (exact mode:
//    limb i of q[m] is row i*M+m; int8 mode: the caller's stacked rows) sit in LDS for the block's K slice;
//    every wave streams 16 weight rows straight from HBM into MFMA B operands (16-byte loads, no LDS), one
//    v_mfma_i32_16x16x64_i8 per (16-row block, weight plane). Int32 products go through LDS once and are
//    joined in int64 (sum C_j[i M + m] 2^(8(i+j))). Split-K partials meet in an int64 workspace with atomics;
//    the last block of a column tile (a device-scope counter) applies the epilogue and re-zeroes workspace
//    and counter, so one launch does everything.
//  * wide_kernel (prefill): 32x64 wave tiles of v_mfma_i32_32x32x32_i8 over LDS-staged, double-buffered
//    64-deep K tiles. Exact mode splits int32 q into 3 int8 limb planes on the way into LDS and runs the
//    9 limb products into 5 int32 accumulators by limb weight i + j (|acc| <= 3 K 2^14 < 2^31 for
//    K < 43690), joined in int64 in registers and rounded in the fused epilogue with the sparse residual.
// Integer sums are exact in any order, so tiles, splits and schedules never change a bit.
#include "bx_common.h"

namespace bx {

enum Mode { RAW32 = 0, JOIN = 1, WMM_T = 2, EXACT = 3 };

struct LinArgs {
  const int32_t* q;      // exact: q int32 [M, ldq]
  int64_t ldq;
  const int8_t* a;       // int8 mode: stacked limb rows [rows_a, K]
  const int8_t* w;       // weight planes
  int64_t ld_plane, ld_row;
  const int64_t* sh;
  const int64_t* d;
  const int64_t* g;
  const int32_t* cnt;
  const int32_t* ecol;
  const int64_t* eval;
  int R;
  void* out;
  int32_t* flag;
  int checked, FR;
  int M, N, K;           // output rows, columns, depth
  int rows_a;            // stacked activation rows (exact: 3M, JOIN: nl M, RAW32: M)
  int nl;                // JOIN limbs
  int64_t* ws;           // split-K int64 [M, N]
  int32_t* sem;          // split-K counters, one per column tile
  int ks;                // K per split (multiple of 64)
};

// ---- epilogue shared by both kernels: one output element from its exact int64 dense value ----
template <int MODE>
__device__ __forceinline__ void finalize(const LinArgs& p, int m, int n, int64_t v, bool& bad) {
  const int64_t o = (int64_t)m * p.N + n;
  if (MODE == RAW32) {
    ((int32_t*)p.out)[o] = (int32_t)v;
  } else if (MODE == JOIN || MODE == WMM_T) {
    ((int64_t*)p.out)[o] = v;
  } else {
    // segs.lin_y (src/bitexact/exact/segs.py:25-32): B from the ELL residual, then wmm.epilogue.
    int64_t B = 0;
    if (p.R > 0) {
      const int c = p.cnt[n];
      const int32_t* qr = p.q + (int64_t)m * p.ldq;
      const int32_t* ec = p.ecol + (int64_t)n * p.R;
      const int64_t* ev = p.eval + (int64_t)n * p.R;
      for (int j = 0; j < c; ++j) B = add_wrap(B, mul_wrap((int64_t)qr[ec[j]], ev[j]));
    }
    const int64_t dn = p.d[n];
    const int64_t pe = p.sh[m] + p.g[n] - dn + p.FR;
    bool b;
    ((int64_t*)p.out)[o] = exact_round(v, B, dn, pe, b);
    bad |= b;
  }
}

__device__ __forceinline__ uint32_t pack4(int32_t a, int32_t b, int32_t c, int32_t d) {
  return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) | ((uint32_t)(d & 255) << 24);
}

// Three int8 limb words (4 values each) of 4 int32 values.
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

// =====================================================================================================
// skinny kernel: 256 threads, 4 waves x 16 weight rows = 64 output columns per block, grid (N/64, splits)
// =====================================================================================================
constexpr int kSkU = 4;   // k steps of 64 in flight per wave

template <int NB, int RB, int MODE>
__global__ __launch_bounds__(256) void skinny_kernel(LinArgs p) {
  extern __shared__ __align__(16) char smem[];
  __shared__ int s_last;
  constexpr int RA = 16 * RB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * 64;
  const int k0 = blockIdx.y * p.ks;
  const int kend = min(p.K, k0 + p.ks);
  const int kpad = ((kend - k0) + 63) & ~63;
  const int LDA = kpad + 16;
  int8_t* As = (int8_t*)smem;

  // ---- stage the activation limb rows of this K slice in LDS ----
  if (MODE == EXACT || MODE == WMM_T) {
    const int nq = kpad >> 2;
    for (int c = tid; c < p.M * nq; c += 256) {
      const int m = c / nq, kq = c - m * nq, k = k0 + kq * 4;
      v4i v = {0, 0, 0, 0};
      if (k < kend) v = *(const v4i*)(p.q + (int64_t)m * p.ldq + k);
      uint32_t l0, l1, l2;
      split3(v, l0, l1, l2);
      *(uint32_t*)(As + (0 * p.M + m) * LDA + kq * 4) = l0;
      *(uint32_t*)(As + (1 * p.M + m) * LDA + kq * 4) = l1;
      *(uint32_t*)(As + (2 * p.M + m) * LDA + kq * 4) = l2;
    }
    const int nc = kpad >> 4;
    for (int c = tid; c < (RA - 3 * p.M) * nc; c += 256) {
      const int r = 3 * p.M + c / nc, kc = c % nc;
      *(v4i*)(As + r * LDA + kc * 16) = v4i{0, 0, 0, 0};
    }
  } else {
    const int nc = kpad >> 4;
    for (int c = tid; c < RA * nc; c += 256) {
      const int r = c / nc, kc = c - r * nc, k = k0 + kc * 16;
      v4i v = {0, 0, 0, 0};
      if (r < p.rows_a && k < kend) v = *(const v4i*)(p.a + (int64_t)r * p.K + k);
      *(v4i*)(As + r * LDA + kc * 16) = v;
    }
  }
  __syncthreads();

  // ---- stream weights: lane -> weight row n (= MFMA B column), 16 bytes at k = 16 (lane / 16) ----
  const int nrow = n0 + wave * 16 + (lane & 15);
  const bool nok = nrow < p.N;
  const int kl = (lane >> 4) * 16;
  const int8_t* wrow = p.w + (int64_t)(nok ? nrow : 0) * p.ld_row;
  const int8_t* arow = As + (lane & 15) * LDA + kl;
  v4i acc[RB][NB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = v4i{0, 0, 0, 0};

  for (int kk = 0; kk < kpad; kk += 64 * kSkU) {
    v4i b[kSkU][NB];
#pragma unroll
    for (int u = 0; u < kSkU; ++u) {
      const int k = k0 + kk + u * 64 + kl;
#pragma unroll
      for (int j = 0; j < NB; ++j)
        b[u][j] = (nok && k < kend) ? *(const v4i*)(wrow + j * p.ld_plane + k) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kSkU; ++u) {
      if (kk + u * 64 < kpad) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const v4i av = *(const v4i*)(arow + r * 16 * LDA + kk + u * 64);
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[r][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[u][j], acc[r][j], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();

  // ---- int32 products to LDS: Cs[j][row][col], row = MFMA row (stacked limb row), col in [0, 64) ----
  int32_t* Cs = (int32_t*)smem;
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r * 16 + (lane >> 4) * 4 + e, col = wave * 16 + (lane & 15);
        Cs[(j * RA + row) * 64 + col] = acc[r][j][e];
      }
  __syncthreads();

  bool bad = false;
  const bool split = gridDim.y > 1;
  for (int e = tid; e < p.M * 64; e += 256) {
    const int m = e >> 6, c = e & 63, n = n0 + c;
    if (n >= p.N) continue;
    int64_t v;
    if (MODE == RAW32) {
      v = Cs[m * 64 + c];
    } else if (MODE == JOIN) {
      v = 0;
      for (int i = 0; i < p.nl; ++i) v += (int64_t)Cs[(i * p.M + m) * 64 + c] << (8 * i);
    } else {
      v = 0;
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) v += (int64_t)Cs[(j * RA + i * p.M + m) * 64 + c] << (8 * (i + j));
    }
    if (split)
      atomicAdd((unsigned long long*)&p.ws[(int64_t)m * p.N + n], (unsigned long long)v);
    else
      finalize<MODE>(p, m, n, v, bad);
  }
  if (split) {
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&p.sem[blockIdx.x], 1) == (int)gridDim.y - 1;
    __syncthreads();
    if (s_last) {
      __threadfence();
      for (int e = tid; e < p.M * 64; e += 256) {
        const int m = e >> 6, n = n0 + (e & 63);
        if (n >= p.N) continue;
        const int64_t v = (int64_t)atomicExch((unsigned long long*)&p.ws[(int64_t)m * p.N + n], 0ull);
        finalize<MODE>(p, m, n, v, bad);
      }
      if (tid == 0) atomicExch(&p.sem[blockIdx.x], 0);
    }
  }
  if (MODE == EXACT && p.checked && bad) p.flag[0] = 1;
}

// =====================================================================================================
// wide kernel: WM x WN waves, wave tile 32 x 64 (two 32x32 MFMA column blocks), BK = 64, 2 LDS stages
// =====================================================================================================
constexpr int kRow = 80;   // LDS bytes per 64-byte operand row (16 bytes of padding: conflict-free b128 reads)

template <int NA, int NB, int MODE, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void wide_kernel(LinArgs p) {
  constexpr int NT = WM * WN * 64;
  constexpr int BM = 32 * WM, BN = 64 * WN;
  constexpr int NS = NA + NB - 1;
  constexpr bool AQ = (MODE == EXACT || MODE == WMM_T);
  constexpr int A_BYTES = NA * BM * kRow, STAGE = (NA * BM + NB * BN) * kRow;
  constexpr int CA = AQ ? (BM * 16) / NT : (NA * BM * 4) / NT;   // 16-byte A source chunks per thread
  constexpr int CB = (NB * BN * 4) / NT;                          // 16-byte B chunks per thread
  static_assert(CA * NT == (AQ ? BM * 16 : NA * BM * 4) && CB * NT == NB * BN * 4, "tile/thread mismatch");
  extern __shared__ __align__(16) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int nk = (p.K + 63) >> 6;

  v4i ra[CA], rb[CB];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * NT;
      if (AQ) {
        const int row = c >> 4, kq = c & 15, m = m0 + row, k = kt * 64 + kq * 4;
        ra[i] = (m < p.M && k < p.K) ? *(const v4i*)(p.q + (int64_t)m * p.ldq + k) : v4i{0, 0, 0, 0};
      } else {
        const int pl = c / (BM * 4), rem = c - pl * (BM * 4), row = rem >> 2, kc = rem & 3;
        const int m = m0 + row, k = kt * 64 + kc * 16;
        ra[i] = (m < p.M && k < p.K) ? *(const v4i*)(p.a + ((int64_t)pl * p.M + m) * p.K + k) : v4i{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int c = tid + i * NT;
      const int pl = c / (BN * 4), rem = c - pl * (BN * 4), row = rem >> 2, kc = rem & 3;
      const int n = n0 + row, k = kt * 64 + kc * 16;
      rb[i] = (n < p.N && k < p.K) ? *(const v4i*)(p.w + pl * p.ld_plane + (int64_t)n * p.ld_row + k)
                                   : v4i{0, 0, 0, 0};
    }
  };
  auto store = [&](int s) {
    char* base = smem + s * STAGE;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * NT;
      if (AQ) {
        const int row = c >> 4, kq = c & 15;
        uint32_t l0, l1, l2;
        split3(ra[i], l0, l1, l2);
        *(uint32_t*)(base + 0 * BM * kRow + row * kRow + kq * 4) = l0;
        *(uint32_t*)(base + 1 * BM * kRow + row * kRow + kq * 4) = l1;
        *(uint32_t*)(base + 2 * BM * kRow + row * kRow + kq * 4) = l2;
      } else {
        const int pl = c / (BM * 4), rem = c - pl * (BM * 4), row = rem >> 2, kc = rem & 3;
        *(v4i*)(base + pl * BM * kRow + row * kRow + kc * 16) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int c = tid + i * NT;
      const int pl = c / (BN * 4), rem = c - pl * (BN * 4), row = rem >> 2, kc = rem & 3;
      *(v4i*)(base + A_BYTES + pl * BN * kRow + row * kRow + kc * 16) = rb[i];
    }
  };

  v16i acc[NS][2];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[s][t][e] = 0;

  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load(kt + 1);
    const char* base = smem + (kt & 1) * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int koff = h * 32 + (lane >> 5) * 16;
      v4i av[NA], bv[NB][2];
#pragma unroll
      for (int i = 0; i < NA; ++i) av[i] = *(const v4i*)(base + i * BM * kRow + (wm * 32 + (lane & 31)) * kRow + koff);
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          bv[j][t] = *(const v4i*)(base + A_BYTES + j * BN * kRow + (wn * 64 + t * 32 + (lane & 31)) * kRow + koff);
#pragma unroll
      for (int i = 0; i < NA; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int t = 0; t < 2; ++t)
            acc[i + j][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[j][t], acc[i + j][t], 0, 0, 0);
    }
    if (kt + 1 < nk) store((kt + 1) & 1);
    __syncthreads();
  }

  bool bad = false;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      const int n = n0 + wn * 64 + t * 32 + (lane & 31);
      if (m < p.M && n < p.N) {
        int64_t v = 0;
#pragma unroll
        for (int s = 0; s < NS; ++s) v += (int64_t)acc[s][t][e] << (8 * s);
        finalize<MODE>(p, m, n, v, bad);
      }
    }
  if (MODE == EXACT && p.checked && bad) p.flag[0] = 1;
}

// =====================================================================================================
// host dispatch
// =====================================================================================================
struct SkinnyPlan {
  int rb, split, ks, tiles;
  size_t lds;
  int64_t ws_bytes;
};

static SkinnyPlan plan_skinny(int rows_a, int M_out, int N, int K, int nb) {
  SkinnyPlan s;
  s.rb = rows_a <= 16 ? 1 : rows_a <= 32 ? 2 : 4;
  const int RA = 16 * s.rb;
  s.tiles = (N + 63) / 64;
  const int nk = (K + 63) / 64;
  const int target = 2 * device_cus();
  int split = (target + s.tiles - 1) / s.tiles;
  split = split < 1 ? 1 : split > nk ? nk : split;
  int kstep = (nk + split - 1) / split;
  const int kmax = ((65536 / RA) - 16) / 64;   // A slice in LDS <= 64 KiB
  if (kstep > kmax) kstep = kmax;
  s.ks = kstep * 64;
  s.split = (K + s.ks - 1) / s.ks;
  const size_t a_lds = (size_t)RA * (s.ks + 16), c_lds = (size_t)nb * RA * 64 * 4;
  s.lds = a_lds > c_lds ? a_lds : c_lds;
  s.ws_bytes = s.split > 1 ? (int64_t)M_out * N * 8 + 256 + (int64_t)s.tiles * 4 : 0;
  return s;
}

template <int NB, int MODE>
static int launch_skinny(LinArgs& p, const SkinnyPlan& s, hipStream_t st) {
  p.ks = s.ks;
  if (s.split > 1) {
    p.ws = (int64_t*)p.ws;
    p.sem = (int32_t*)((char*)p.ws + (((int64_t)p.M * p.N * 8 + 255) & ~255LL));
  }
  dim3 grid(s.tiles, s.split);
  if (s.rb == 1)
    skinny_kernel<NB, 1, MODE><<<grid, 256, s.lds, st>>>(p);
  else if (s.rb == 2)
    skinny_kernel<NB, 2, MODE><<<grid, 256, s.lds, st>>>(p);
  else
    skinny_kernel<NB, 4, MODE><<<grid, 256, s.lds, st>>>(p);
  return check_launch("skinny_kernel");
}

template <int NA, int NB, int MODE, int WM, int WN>
static int launch_wide_cfg(LinArgs& p, hipStream_t st) {
  constexpr int BM = 32 * WM, BN = 64 * WN;
  const size_t lds = 2 * (size_t)(NA * BM + NB * BN) * kRow;
  static bool attr_set[64] = {false};
  int dev = 0;
  hipGetDevice(&dev);
  if (dev >= 0 && dev < 64 && !attr_set[dev]) {
    hipFuncSetAttribute((const void*)wide_kernel<NA, NB, MODE, WM, WN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)lds);
    attr_set[dev] = true;
  }
  dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM);
  wide_kernel<NA, NB, MODE, WM, WN><<<grid, WM * WN * 64, lds, st>>>(p);
  return check_launch("wide_kernel");
}

template <int NA, int NB, int MODE>
static int launch_wide(LinArgs& p, hipStream_t st) {
  const int64_t big = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (big >= device_cus()) return launch_wide_cfg<NA, NB, MODE, 4, 2>(p, st);
  return launch_wide_cfg<NA, NB, MODE, 2, 2>(p, st);
}

static bool aligned16(const void* x) { return ((uintptr_t)x & 15) == 0; }

}  // namespace bx

using namespace bx;

static int exact_common(LinArgs& p, int mode, int64_t ws_bytes, hipStream_t st) {
  BX_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, "negative size");
  BX_REQUIRE(p.K % 16 == 0, "K %% 16 != 0 (K=%d)", p.K);
  BX_REQUIRE(p.K < 43690, "K >= 43690: int32 limb sums could overflow");
  BX_REQUIRE(p.ldq % 4 == 0 && p.ldq >= p.K, "ldq must be >= K and a multiple of 4");
  BX_REQUIRE(p.ld_row % 16 == 0 && p.ld_plane % 16 == 0, "limb strides must be multiples of 16");
  BX_REQUIRE(aligned16(p.q) && aligned16(p.w), "q and limbs must be 16-byte aligned");
  if (p.M == 0 || p.N == 0) return BX_OK;
  p.rows_a = 3 * p.M;
  if (p.rows_a <= 64) {
    SkinnyPlan s = plan_skinny(p.rows_a, p.M, p.N, p.K, 3);
    if (s.split > 1) BX_REQUIRE(p.ws != nullptr && ws_bytes >= s.ws_bytes, "workspace too small (%lld < %lld)",
                                (long long)ws_bytes, (long long)s.ws_bytes);
    return mode == EXACT ? launch_skinny<3, EXACT>(p, s, st) : launch_skinny<3, WMM_T>(p, s, st);
  }
  return mode == EXACT ? launch_wide<3, 3, EXACT>(p, st) : launch_wide<3, 3, WMM_T>(p, st);
}

extern "C" int bx_exact_linear(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs,
                               int64_t ld_plane, int64_t ld_row, const int64_t* d, const int64_t* g,
                               const int32_t* ell_cnt, const int32_t* ell_col, const int64_t* ell_val, int32_t R,
                               int64_t* y, int32_t M, int32_t N, int32_t K, int32_t FR, int32_t checked,
                               int32_t* flag, void* ws, int64_t ws_bytes, bx_stream_t stream) {
  LinArgs p = {};
  p.q = q; p.ldq = ldq; p.w = limbs; p.ld_plane = ld_plane; p.ld_row = ld_row;
  p.sh = sh; p.d = d; p.g = g; p.cnt = ell_cnt; p.ecol = ell_col; p.eval = ell_val; p.R = R;
  p.out = y; p.flag = flag; p.checked = checked; p.FR = FR; p.M = M; p.N = N; p.K = K;
  p.ws = (int64_t*)ws;
  BX_REQUIRE(R >= 0 && (R == 0 || (ell_cnt && ell_col && ell_val)), "ELL residual arrays missing");
  BX_REQUIRE(!checked || flag, "checked needs a flag pointer");
  BX_REQUIRE(sh && d && g && y, "null pointer");
  return exact_common(p, EXACT, ws_bytes, (hipStream_t)stream);
}

extern "C" int bx_exact_wmm(const int32_t* q, int64_t ldq, const int8_t* limbs, int64_t ld_plane, int64_t ld_row,
                            int64_t* T, int32_t M, int32_t N, int32_t K, void* ws, int64_t ws_bytes,
                            bx_stream_t stream) {
  LinArgs p = {};
  p.q = q; p.ldq = ldq; p.w = limbs; p.ld_plane = ld_plane; p.ld_row = ld_row;
  p.out = T; p.M = M; p.N = N; p.K = K; p.ws = (int64_t*)ws;
  return exact_common(p, WMM_T, ws_bytes, (hipStream_t)stream);
}

extern "C" int64_t bx_exact_linear_workspace(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || 3 * M > 64) return 0;
  return plan_skinny(3 * M, M, N, K, 3).ws_bytes;
}

static int int8_common(LinArgs& p, int mode, int64_t ws_bytes, hipStream_t st) {
  BX_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, "negative size");
  BX_REQUIRE(p.K % 16 == 0, "K %% 16 != 0 (K=%d)", p.K);
  BX_REQUIRE((int64_t)p.K * 127 * 128 < (1LL << 31), "K too large for exact int32 sums");
  BX_REQUIRE(aligned16(p.a) && aligned16(p.w), "a and w must be 16-byte aligned");
  if (p.M == 0 || p.N == 0) return BX_OK;
  if (p.rows_a <= 64) {
    SkinnyPlan s = plan_skinny(p.rows_a, p.M, p.N, p.K, 1);
    if (s.split > 1) BX_REQUIRE(p.ws != nullptr && ws_bytes >= s.ws_bytes, "workspace too small (%lld < %lld)",
                                (long long)ws_bytes, (long long)s.ws_bytes);
    return mode == JOIN ? launch_skinny<1, JOIN>(p, s, st) : launch_skinny<1, RAW32>(p, s, st);
  }
  if (mode == RAW32) return launch_wide<1, 1, RAW32>(p, st);
  if (p.nl == 1) return launch_wide<1, 1, JOIN>(p, st);
  if (p.nl == 2) return launch_wide<2, 1, JOIN>(p, st);
  return launch_wide<3, 1, JOIN>(p, st);
}

extern "C" int bx_int8_gemm(const int8_t* a, const int8_t* w, int32_t* c, int32_t R, int32_t N, int32_t K, void* ws,
                            int64_t ws_bytes, bx_stream_t stream) {
  LinArgs p = {};
  p.a = a; p.w = w; p.ld_row = K; p.ld_plane = 0; p.out = c; p.M = R; p.N = N; p.K = K;
  p.rows_a = R; p.nl = 1; p.ws = (int64_t*)ws;
  return int8_common(p, RAW32, ws_bytes, (hipStream_t)stream);
}

extern "C" int bx_int8_gemm_join(const int8_t* a, const int8_t* w, int64_t* y, int32_t M, int32_t N, int32_t K,
                                 int32_t nl, void* ws, int64_t ws_bytes, bx_stream_t stream) {
  BX_REQUIRE(nl >= 1 && nl <= 3, "nl must be 1, 2 or 3");
  LinArgs p = {};
  p.a = a; p.w = w; p.ld_row = K; p.ld_plane = 0; p.out = y; p.M = M; p.N = N; p.K = K;
  p.rows_a = nl * M; p.nl = nl; p.ws = (int64_t*)ws;
  return int8_common(p, JOIN, ws_bytes, (hipStream_t)stream);
}

extern "C" int64_t bx_int8_gemm_workspace(int32_t rows, int32_t N, int32_t K) {
  if (rows <= 0 || N <= 0 || K <= 0 || rows > 64) return 0;
  // the join output has fewer rows than the stacked input; size for the larger (raw) case
  return plan_skinny(rows, rows, N, K, 1).ws_bytes;
}
