// Exact integer attention for gfx950: paged limb-plane KV store, paged decode attention, and fused prefill
// attention over a contiguous integer cache.
//
// What is computed (src/bitexact/exact/ops.py:133-143, src/bitexact/vllm_plugin/tri_exact_attn.py:1-15):
//   raw[i, s] = sum_d q[i, d] K[s, d]                 exact int64 (|q|, |K| within 3 signed base-256 limbs)
//   mx[i]     = max over visible keys s <= qpos[i] of raw[i, s]
//   zf        = min(rshc(mx - raw, FK + 3 - sh[i] - FZ), 48 << FZ); t = rshc(zf l2e, 28)
//   p         = exp2neg_lut(t, lut, FP)   (2^-f table at 2^60 + linear interpolation; 0 for hidden keys)
//   den[i]    = sum_s p,   num[i, d] = sum_s p V[s, d]                  exact int64
// Two sweeps over the keys are required (the quantized exp table does not allow online rescaling,
// src/bitexact/vllm_plugin/tri_paged.py:16-19). Maxima and sums are exact in any order, so the key split and
// the tiling never change a bit.
//
// Kernel shape: one block of 256 threads per (query tile, key range). 64-key tiles are staged in LDS as
// int32 K / V rows (paged caches hold int8 limb planes that are joined on the way in). Thread t = (wave w,
// lane l) owns key l of the tile for the scores of queries w, w + 4, ... and output dims l, l + 64 of the
// same queries for p V, so query-indexed LDS reads are wave-uniform broadcasts and key/dim-indexed reads
// hit distinct banks (rows padded by one word).
#include "bx_common.h"
#include "bx_rope.h"
#include "bx_introws.h"

#include <algorithm>
#include <type_traits>

namespace bx {

BX_PHASE_TABLE

constexpr int kFK = 17, kFZ = 26, kFP = 22, kFT2 = 26, kExp2Bits = 14, kExp2One = 60;

// A weight is exactly 0 once n >= FP + 2: the interpolated table value v lies in [0, 2^60] (the table falls
// from 2^60), and rshc(v, 60 - FP + n) with a shift of at least 62 rounds it to 0 whatever entry was read. Such
// scores (most of them: softmax weights are mostly negligible) read entry 0, so their loads share one cache
// line instead of scattering over the 128 KiB table.
constexpr int64_t kZeroN = kFP + 2;

// attn_weight in two halves, so that a caller can issue the table loads of many scores before using any:
// WeightAt holds the table position of one score (always inside the table: 0 <= idx < 2^14, whatever z is,
// so loads for hidden keys are safe and their weight is discarded).
struct WeightAt {
  int64_t n, rr;
  int idx;
};

__device__ __forceinline__ WeightAt weight_at(int64_t z, int64_t zshift, int64_t l2e) {
  int64_t zf = rshc(z, zshift);
  zf = imin(zf, 48LL << kFZ);
  const int64_t t = rshc(mul_wrap(zf, l2e), kFZ + 28 - kFT2);
  const int64_t f = t & ((1LL << kFT2) - 1);
  WeightAt w;
  w.n = t >> kFT2;
  w.idx = w.n < kZeroN ? (int)(f >> (kFT2 - kExp2Bits)) : 0;
  w.rr = f & ((1LL << (kFT2 - kExp2Bits)) - 1);
  return w;
}

// weight_at for zshift >= 0, 0 <= l2e < 2^31 and 0 <= z < 2^62 (z = mx - raw of a visible key): zf = rshc(z, zshift)
// is then >= 0 and at most 48 2^26 after the clamp, so zf l2e is one 32 x 32 -> 64-bit product below 3 2^61
// and t, n, f come from 64-bit shifts of it; the same position as weight_at. Negative z (hidden keys, whose
// weight is discarded) is clamped to 0, which keeps the position inside the table.
__device__ __forceinline__ WeightAt weight_at_nn(int64_t z, int64_t zshift, int64_t l2e) {
  int64_t zf = rshc(z, zshift);
  zf = zf < 0 ? 0 : zf > (48LL << kFZ) ? (48LL << kFZ) : zf;
  const uint64_t prod = (uint64_t)(uint32_t)zf * (uint64_t)(uint32_t)l2e;
  const uint64_t t = (prod + (1ULL << (kFZ + 28 - kFT2 - 1))) >> (kFZ + 28 - kFT2);
  const uint32_t f = (uint32_t)t & ((1u << kFT2) - 1);
  WeightAt w;
  w.n = (int64_t)(t >> kFT2);
  w.idx = w.n < kZeroN ? (int)(f >> (kFT2 - kExp2Bits)) : 0;
  w.rr = f & ((1u << (kFT2 - kExp2Bits)) - 1);
  return w;
}

__device__ __forceinline__ int64_t weight_of(const WeightAt& w, int64_t a, int64_t b) {
  const int64_t v = add_wrap(a, rshc(mul_wrap(b - a, w.rr), kFT2 - kExp2Bits));
  return rshc(v, kExp2One - kFP + w.n);
}

// softmax_w's weight of one visible key (src/bitexact/exact/ops.py:133-143 over exp2neg_lut, 108-116).
__device__ __forceinline__ int64_t attn_weight(int64_t z, int64_t zshift, const int64_t* lut, int64_t l2e) {
  int64_t zf = rshc(z, zshift);
  zf = imin(zf, 48LL << kFZ);
  const int64_t t = rshc(mul_wrap(zf, l2e), kFZ + 28 - kFT2);
  const int64_t n = t >> kFT2;
  const int64_t f = t & ((1LL << kFT2) - 1);
  const int64_t idx = n < kZeroN ? f >> (kFT2 - kExp2Bits) : 0;
  const int64_t rr = f & ((1LL << (kFT2 - kExp2Bits)) - 1);
  const int64_t a = lut[idx];
  const int64_t v = add_wrap(a, rshc(mul_wrap(lut[idx + 1] - a, rr), kFT2 - kExp2Bits));
  return rshc(v, kExp2One - kFP + n);
}

// int8-mode weight of a visible key (int8.segs.softmax, src/bitexact/int8/segs.py:90-99; tri_paged._zscale,
// src/bitexact/vllm_plugin/tri_paged.py:93-99): d = raw - mx <= 0 at 2 FQ bits, z = rsh(d, zsh) (head_dim 64)
// or rsh(max(d, -2^38) zmul, zsh) (head_dim 128, zmul = round(2^24 / sqrt 2)); the weight is the table entry
// rsh(e^z 2^FE, FE - FP) of z at step 2^-FA over [EXP_MIN, 0], 0 below it.
constexpr int64_t kI8ZClamp = -(1LL << 38);
constexpr int64_t kI8ZLo = -32LL * 4096;         // EXP_MIN << FA: table index 0
// The table index of int8_weight (negative: weight 0).
__device__ __forceinline__ int64_t int8_index(int64_t d, int zsh, int64_t zmul) {
  const int64_t z = zmul == 0 ? rsh64(d, zsh) : rsh64(mul_wrap(imax(d, kI8ZClamp), zmul), zsh);
  return imax(z, kI8ZLo - 1) - kI8ZLo;
}

__device__ __forceinline__ int64_t int8_weight(int64_t d, int zsh, int64_t zmul, const int32_t* ptab) {
  const int64_t idx = int8_index(d, zsh, zmul);
  return idx >= 0 ? (int64_t)ptab[idx] : 0;
}

// int32 value -> the value of its first three signed base-256 digits (what a 3-limb split keeps).
__device__ __forceinline__ int32_t keep3(int32_t x) {
  const int32_t a0 = limb_lo(x);
  int32_t r = (x - a0) >> 8;
  const int32_t a1 = limb_lo(r);
  r = (r - a1) >> 8;
  const int32_t a2 = limb_lo(r);
  return a0 + a1 * 256 + a2 * 65536;
}

struct AttnArgs {
  // queries
  const int32_t* q;
  int64_t sq_tile, sq_row;        // element strides: between query groups (z or (r,h)) and between queries
  const int64_t* sh;              // per query exponent, index = group * sh_tile + query
  int64_t sh_tile;
  const int64_t* qpos;            // per query position: qpos[(group / qpos_div) * qpos_tile + query * qpos_row]
  int64_t qpos_tile, qpos_row;
  int qpos_div;
  int nq;                         // queries per group (decode M <= 4, prefill gT)
  // keys: paged limb planes or contiguous int32
  const int8_t* cache;            // [nb, HKV, bs, 8 HD]
  int64_t sc_nb, sc_h, sc_bs;
  const int32_t* bt;
  int64_t sbt;
  const int64_t* rmap;
  int bs, hkv;
  int nblk;                       // paged: block-table entries per row
  const int32_t* K;               // contiguous: [Z, S, HD] with strides
  const int32_t* V;
  int64_t sk_z, sk_s, sv_z, sv_s;
  int S;                          // contiguous: keys available
  // table, scale (exact mode)
  const int64_t* lut;
  int64_t l2e;
  // int8 mode: int64 queries and the weight table (wrule 1)
  const int64_t* q64;
  const int32_t* ptab;
  int wrule, zsh;
  int64_t zmul;
  // outputs
  int64_t* num;
  int64_t* den;
  int64_t snum_tile, snum_row;
  int64_t sden_tile;
  // split-KV state
  int nsplit;
  int64_t* mx_ws;                 // [groups, nq] running maxima stored as mx - NEG (0 = none yet)
  int64_t* num_ws;                // [groups, nq, HD]
  int64_t* den_ws;                // [groups, nq]
  int32_t* sem;                   // [groups]
  uint64_t exch_ticks;            // attn_dec_exch_kernel: longest wait for the other splits' maxima (100 MHz ticks)
};

template <int QT, int HD>
struct AttnSmem {
  int32_t Qs[QT][HD];
  int32_t Ks[64][HD + 1];
  int32_t Vs[64][HD + 1];
  int32_t Ps[QT][65];
  int64_t qpos[QT];
  int64_t shift[QT];              // per query: FK + 3 - FZ - sh
  int64_t mx[QT];
  int s_last;
};

template <int QT, int HD, bool PAGED>
__device__ __forceinline__ void load_kv_tile(const AttnArgs& p, AttnSmem<QT, HD>& sm, int group, int h, int key0, int nkeys,
                                             bool want_v) {
  constexpr int UNITS = 64 * (HD / 16);          // (key, 16-dim chunk) units per tile
  for (int u = threadIdx.x; u < UNITS; u += 256) {
    const int kk = u / (HD / 16), c = u % (HD / 16);
    const int s = key0 + kk;
    int32_t kv[16], vv[16];
    if (kk < nkeys) {
      if (PAGED) {
        const int64_t brow = p.rmap ? p.rmap[group / p.hkv] : group / p.hkv;
        const int blk = p.bt[brow * p.sbt + s / p.bs];
        const int8_t* row = p.cache + (int64_t)blk * p.sc_nb + (int64_t)h * p.sc_h + (int64_t)(s % p.bs) * p.sc_bs;
        const v4i k0 = *(const v4i*)(row + c * 16), k1 = *(const v4i*)(row + HD + c * 16),
                  k2 = *(const v4i*)(row + 2 * HD + c * 16);
        v4i v0 = {0, 0, 0, 0}, v1 = v0, v2 = v0;
        if (want_v) {
          v0 = *(const v4i*)(row + 3 * HD + c * 16);
          v1 = *(const v4i*)(row + 4 * HD + c * 16);
          v2 = *(const v4i*)(row + 5 * HD + c * 16);
        }
        const int8_t* pk0 = (const int8_t*)&k0;
        const int8_t* pk1 = (const int8_t*)&k1;
        const int8_t* pk2 = (const int8_t*)&k2;
        const int8_t* pv0 = (const int8_t*)&v0;
        const int8_t* pv1 = (const int8_t*)&v1;
        const int8_t* pv2 = (const int8_t*)&v2;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          kv[e] = (int32_t)pk0[e] + (int32_t)pk1[e] * 256 + (int32_t)pk2[e] * 65536;
          vv[e] = (int32_t)pv0[e] + (int32_t)pv1[e] * 256 + (int32_t)pv2[e] * 65536;
        }
      } else {
        const int32_t* kr = p.K + (int64_t)group * p.sk_z + (int64_t)s * p.sk_s + c * 16;
        const int32_t* vr = p.V + (int64_t)group * p.sv_z + (int64_t)s * p.sv_s + c * 16;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          kv[e] = keep3(kr[e]);
          vv[e] = want_v ? keep3(vr[e]) : 0;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) kv[e] = vv[e] = 0;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sm.Ks[kk][c * 16 + e] = kv[e];
      if (want_v) sm.Vs[kk][c * 16 + e] = vv[e];
    }
  }
}

// raw scores of this thread's queries (w + 4 j) against key lane l of the staged tile
template <int QT, int HD>
__device__ __forceinline__ void tile_scores(const AttnSmem<QT, HD>& sm, int64_t (&raw)[QT / 4]) {
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < QT / 4; ++j) raw[j] = 0;
#pragma unroll 8
  for (int d = 0; d < HD; ++d) {
    const int64_t kd = sm.Ks[l][d];
#pragma unroll
    for (int j = 0; j < QT / 4; ++j) raw[j] += (int64_t)sm.Qs[w + 4 * j][d] * kd;
  }
}

// Stage queries of the tile (3-limb values), their exponents / positions; returns the visible key count.
template <int QT, int HD>
__device__ __forceinline__ int64_t stage_queries(const AttnArgs& p, AttnSmem<QT, HD>& sm, int group, int q0, int nvalid) {
  for (int u = threadIdx.x; u < QT * HD; u += 256) {
    const int i = u / HD, d = u % HD;
    const int64_t qi = group * p.sq_tile + (int64_t)(q0 + i) * p.sq_row + d;
    sm.Qs[i][d] = i < nvalid ? keep3(p.q64 ? (int32_t)p.q64[qi] : p.q[qi]) : 0;
  }
  if (threadIdx.x < QT) {
    const int i = threadIdx.x;
    const bool ok = i < nvalid;
    sm.qpos[i] = ok ? p.qpos[(group / p.qpos_div) * p.qpos_tile + (int64_t)(q0 + i) * p.qpos_row] : -1;
    sm.shift[i] = ok && p.sh ? (int64_t)(kFK + 3 - kFZ) - p.sh[group * p.sh_tile + q0 + i] : 0;
    sm.mx[i] = kNeg;
  }
  __syncthreads();
  int64_t kend = 0;
  for (int i = 0; i < QT; ++i) kend = imax(kend, sm.qpos[i] + 1);
  return kend;
}

// Sweep 1: per-query maxima over visible keys in [lo, hi) into sm.mx (LDS atomic max).
template <int QT, int HD, bool PAGED>
__device__ void sweep_max(const AttnArgs& p, AttnSmem<QT, HD>& sm, int group, int h, int64_t lo, int64_t hi) {
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t best[QT / 4];
#pragma unroll
  for (int j = 0; j < QT / 4; ++j) best[j] = kNeg;
  for (int64_t k0 = lo; k0 < hi; k0 += 64) {
    const int nk = (int)imin(64, hi - k0);
    __syncthreads();
    load_kv_tile<QT, HD, PAGED>(p, sm, group, h, (int)k0, nk, false);
    __syncthreads();
    int64_t raw[QT / 4];
    tile_scores<QT, HD>(sm, raw);
#pragma unroll
    for (int j = 0; j < QT / 4; ++j) {
      const bool vis = l < nk && k0 + l <= sm.qpos[w + 4 * j];
      if (vis) best[j] = imax(best[j], raw[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < QT / 4; ++j) {
    const int64_t m = wave_max64(best[j]);
    if (l == 0) atomicMax((long long*)&sm.mx[w + 4 * j], (long long)m);
  }
  __syncthreads();
}

// Sweep 2: weights from the maxima in sm.mx; accumulates den / num for the thread's queries.
template <int QT, int HD, bool PAGED>
__device__ void sweep_acc(const AttnArgs& p, AttnSmem<QT, HD>& sm, int group, int h, int64_t lo, int64_t hi,
                          int64_t (&den)[QT / 4], int64_t (&num)[QT / 4][HD / 64]) {
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < QT / 4; ++j) {
    den[j] = 0;
#pragma unroll
    for (int c = 0; c < HD / 64; ++c) num[j][c] = 0;
  }
  for (int64_t k0 = lo; k0 < hi; k0 += 64) {
    const int nk = (int)imin(64, hi - k0);
    __syncthreads();
    load_kv_tile<QT, HD, PAGED>(p, sm, group, h, (int)k0, nk, true);
    __syncthreads();
    int64_t raw[QT / 4];
    tile_scores<QT, HD>(sm, raw);
#pragma unroll
    for (int j = 0; j < QT / 4; ++j) {
      const int i = w + 4 * j;
      const bool vis = l < nk && k0 + l <= sm.qpos[i];
      int64_t pw = 0;
      if (vis)
        pw = p.wrule == 0 ? attn_weight(sm.mx[i] - raw[j], sm.shift[i], p.lut, p.l2e)
                          : int8_weight(raw[j] - sm.mx[i], p.zsh, p.zmul, p.ptab);
      den[j] += pw;
      sm.Ps[i][l] = (int32_t)pw;
    }
    __syncthreads();
#pragma unroll 4
    for (int s = 0; s < nk; ++s) {
#pragma unroll
      for (int c = 0; c < HD / 64; ++c) {
        const int64_t vd = sm.Vs[s][l + 64 * c];
#pragma unroll
        for (int j = 0; j < QT / 4; ++j) num[j][c] += (int64_t)sm.Ps[w + 4 * j][s] * vd;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < QT / 4; ++j) den[j] = wave_sum64(den[j]);
}

// Key range [lo, hi) of split `sp` of [0, kend) in 64-key multiples.
__device__ __forceinline__ void split_range(int64_t kend, int nsplit, int sp, int64_t& lo, int64_t& hi) {
  const int64_t chunk = ((kend + nsplit - 1) / nsplit + 63) / 64 * 64;
  lo = imin(kend, sp * chunk);
  hi = imin(kend, lo + chunk);
}

// grid (groups * query tiles, nsplit). nsplit == 1: both sweeps, outputs written directly.
// nsplit > 1 and PHASE 0: maxima only (atomic max into mx_ws). PHASE 1: sums into the workspace; the last
// block of a group writes the outputs and restores the workspace (maxima, sums and counter back to 0).
template <int QT, int HD, bool PAGED, int PHASE>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs p) {
  extern __shared__ __align__(16) char smem_raw[];
  AttnSmem<QT, HD>& sm = *(AttnSmem<QT, HD>*)smem_raw;
  const int tiles = (p.nq + QT - 1) / QT;
  const int group = blockIdx.x / tiles, q0 = (blockIdx.x % tiles) * QT;
  const int nvalid = min(QT, p.nq - q0);
  const int h = PAGED ? group % p.hkv : 0;
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t kend = stage_queries<QT, HD>(p, sm, group, q0, nvalid);
  int64_t lo, hi;
  split_range(kend, gridDim.y, blockIdx.y, lo, hi);

  if (gridDim.y == 1) {
    sweep_max<QT, HD, PAGED>(p, sm, group, h, lo, hi);
    int64_t den[QT / 4], num[QT / 4][HD / 64];
    sweep_acc<QT, HD, PAGED>(p, sm, group, h, lo, hi, den, num);
#pragma unroll
    for (int j = 0; j < QT / 4; ++j) {
      const int i = w + 4 * j;
      if (i < nvalid) {
#pragma unroll
        for (int c = 0; c < HD / 64; ++c)
          p.num[group * p.snum_tile + (int64_t)(q0 + i) * p.snum_row + l + 64 * c] = num[j][c];
        if (l == 0) p.den[group * p.sden_tile + q0 + i] = den[j];
      }
    }
    return;
  }
  const int64_t gq = (int64_t)group * p.nq + q0;   // workspace row of the tile's first query
  if (PHASE == 0) {
    sweep_max<QT, HD, PAGED>(p, sm, group, h, lo, hi);
    if (threadIdx.x < nvalid && hi > lo)
      atomicMax((long long*)&p.mx_ws[gq + threadIdx.x], (long long)(sm.mx[threadIdx.x] - kNeg));
    return;
  }
  if (threadIdx.x < QT) sm.mx[threadIdx.x] = threadIdx.x < nvalid ? p.mx_ws[gq + threadIdx.x] + kNeg : kNeg;
  __syncthreads();
  int64_t den[QT / 4], num[QT / 4][HD / 64];
  sweep_acc<QT, HD, PAGED>(p, sm, group, h, lo, hi, den, num);
  if (hi > lo) {
#pragma unroll
    for (int j = 0; j < QT / 4; ++j) {
      const int i = w + 4 * j;
      if (i < nvalid) {
#pragma unroll
        for (int c = 0; c < HD / 64; ++c)
          atomicAdd((unsigned long long*)&p.num_ws[(gq + i) * HD + l + 64 * c], (unsigned long long)num[j][c]);
        if (l == 0) atomicAdd((unsigned long long*)&p.den_ws[gq + i], (unsigned long long)den[j]);
      }
    }
  }
  // every split arrives (empty ones too), the last one publishes and restores the workspace
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int tile_id = blockIdx.x;
    const bool last = atomicAdd(&p.sem[tile_id], 1) == (int)gridDim.y - 1;
    if (last) atomicExch(&p.sem[tile_id], 0);
    sm.s_last = last;
  }
  __syncthreads();
  if (!sm.s_last) return;
  for (int u = threadIdx.x; u < nvalid * HD; u += 256) {
    const int i = u / HD, d = u % HD;
    p.num[group * p.snum_tile + (int64_t)(q0 + i) * p.snum_row + d] =
        (int64_t)atomicExch((unsigned long long*)&p.num_ws[(gq + i) * HD + d], 0ull);
  }
  if (threadIdx.x < nvalid) {
    p.den[group * p.sden_tile + q0 + threadIdx.x] =
        (int64_t)atomicExch((unsigned long long*)&p.den_ws[gq + threadIdx.x], 0ull);
    atomicExch((unsigned long long*)&p.mx_ws[gq + threadIdx.x], 0ull);
  }
}

// ---- paged decode attention on MFMA ----
// Grid (query tiles of <= 4 queries, key splits); a block is 8 independent waves, wave w taking the 16-key blocks
// w, w + 8, ... of the block's key range, with the next block's limb loads in flight while one is used.
// Scores: v_mfma_i32_16x16x64_i8 with the queries' limbs as A (row m = 4 query + limb; the fourth row of each
// query is zero) and one K limb plane as B straight from the cache (lane: key lane & 15, dims of chunk
// lane >> 4 -- the key row is contiguous along the MFMA depth). Lane l receives query l >> 4's limb rows for key
// l & 15 and joins them in int64: raw = sum_j sum_i acc_j[i] 2^(8 (i + j)) (|acc| <= HD 2^14, exact in int32).
// Sweep 1 keeps per-lane maxima. Sweep 2 turns scores into weights, puts the block's weights and joined V rows
// in the wave's own LDS slice and accumulates p V in int64 with one lane per dimension. Waves, then splits,
// are summed in a fixed order: partial maxima and sums go to per-split workspace slots with plain stores and the
// last block of a tile (counter) combines them, so no value is accumulated with atomics.
constexpr int kDecWaves = 8;
constexpr int kDecMaxSplit = 64;
constexpr int64_t kDecWsSplitBudget = 4096;
constexpr uint64_t kDecExchTicks = 20000;     // the exchange kernel's longest wait: 200 us at 100 MHz
constexpr int kDecExchBlocks = 256;           // the exchange kernel: at most one block per compute unit   // the workspace query sizes for min(64, 4096 / tiles) splits

template <int HD>
struct DecSmem {
  union {
    int32_t Vs[kDecWaves][16][HD + 1];   // sweep 2: each wave's joined V rows
    int64_t red[kDecWaves][4][HD];        // after it: each wave's p V sums
  };
  alignas(16) int32_t Ps[kDecWaves][16][4];   // sweep 2: [wave][key][query], one 16-byte read per key
  int64_t qpos[4];
  int64_t shift[4];
  int64_t mx[4];
  int64_t den[kDecWaves][4];
  int s_last;
};

template <int HD>
struct KvRegs {
  v4i k[3][HD / 64];
  v4i v[3][HD / 64];
};

// The cache block of key s (the block table entry: one load, issued an iteration ahead of the rows it locates).
__device__ __forceinline__ int dec_page(const AttnArgs& p, int64_t brow, int s) { return p.bt[brow * p.sbt + s / p.bs]; }

template <int HD, bool WANT_K, bool WANT_V>
__device__ __forceinline__ void dec_rows(const AttnArgs& p, int blk, int h, int s, KvRegs<HD>& r) {
  const int c = (threadIdx.x & 63) >> 4;
  const int8_t* row = p.cache + (int64_t)blk * p.sc_nb + (int64_t)h * p.sc_h + (int64_t)(s % p.bs) * p.sc_bs + c * 16;
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int kk = 0; kk < HD / 64; ++kk) {
      if (WANT_K) r.k[j][kk] = *(const v4i*)(row + j * HD + kk * 64);
      if (WANT_V) r.v[j][kk] = *(const v4i*)(row + (3 + j) * HD + kk * 64);
    }
}

template <int HD>
__device__ __forceinline__ int64_t dec_score(const v4i (&qa)[HD / 64], const KvRegs<HD>& r) {
  int64_t raw = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int kk = 0; kk < HD / 64; ++kk) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[kk], r.k[j][kk], acc, 0, 0, 0);
    const int64_t t = (int64_t)acc[0] + ((int64_t)acc[1] << 8) + ((int64_t)acc[2] << 16);
    raw += t << (8 * j);
  }
  return raw;
}

// workspace slots of tile t (per split sp): maxima (stored as mx - kNeg), p V sums, weight sums; then counters
struct DecWs {
  int64_t* mx;    // [T][NS][4]
  int64_t* num;   // [T][NS][4][HD]
  int64_t* den;   // [T][NS][4]
  int32_t* sem;   // [T]
};
__host__ __device__ __forceinline__ int64_t dec_ws_bytes(int64_t T, int64_t NS, int HD) {
  return T * NS * 4 * 8 * (2 + HD) + T * 4 + 256;
}

__device__ __forceinline__ DecWs dec_ws(const AttnArgs& p, int T, int NS, int HD) {
  const int64_t slots = (int64_t)T * NS * 4;
  char* b = (char*)p.mx_ws;
  DecWs w;
  w.mx = (int64_t*)b;
  w.num = (int64_t*)(b + slots * 8);
  w.den = (int64_t*)(b + slots * 8 * (1 + HD));
  w.sem = (int32_t*)(b + slots * 8 * (2 + HD));
  return w;
}

// The MFMA A operand of a tile's queries: limb (m & 3) of query (m >> 2), m = lane & 15, dims kk 64 +
// (lane >> 4) 16 + [0, 16); the fourth row of each query and queries past nvalid are 0. In two steps, so that a
// caller can issue the query loads first and use them after its other requests: dec_q_load reads the lane's 16
// values per 64 dims (16-byte loads when q is 16-byte aligned), dec_q_limbs packs the lane's limb.
template <int HD>
struct DecQ {
  int32_t x[HD / 64][16];
};

template <int HD>
__device__ __forceinline__ void dec_q_load(const AttnArgs& p, int group, int q0, int nvalid, int lane, DecQ<HD>& q) {
  const int m = lane & 15, qi = m >> 2, li = m & 3, c = lane >> 4;
  const bool live = qi < nvalid && li < 3;
  const int64_t base = group * p.sq_tile + (int64_t)(q0 + qi) * p.sq_row + c * 16;
  const bool vec = !p.q64 && ((reinterpret_cast<uintptr_t>(p.q + base)) & 15) == 0;
#pragma unroll
  for (int kk = 0; kk < HD / 64; ++kk) {
    if (vec) {
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const v4i v = live ? *(const v4i*)(p.q + base + kk * 64 + e4 * 4) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) q.x[kk][e4 * 4 + e] = v[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t qidx = base + kk * 64 + e;
        q.x[kk][e] = live ? (p.q64 ? (int32_t)p.q64[qidx] : p.q[qidx]) : 0;
      }
    }
  }
}

template <int HD>
__device__ __forceinline__ void dec_q_limbs(const DecQ<HD>& q, int lane, v4i (&qa)[HD / 64]) {
  const int li = lane & 3;
#pragma unroll
  for (int kk = 0; kk < HD / 64; ++kk) {
    int32_t word[4];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      uint32_t wv = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int32_t x = q.x[kk][e4 * 4 + e];
        const int32_t a0 = limb_lo(x);
        x = (x - a0) >> 8;
        const int32_t a1 = limb_lo(x);
        x = (x - a1) >> 8;
        const int32_t a2 = limb_lo(x);
        const int32_t v = li == 0 ? a0 : li == 1 ? a1 : li == 2 ? a2 : 0;
        wv |= (uint32_t)(v & 255) << (8 * e);
      }
      word[e4] = (int32_t)wv;
    }
    qa[kk] = v4i{word[0], word[1], word[2], word[3]};
  }
}

template <int HD>
__device__ __forceinline__ void dec_qa(const AttnArgs& p, int group, int q0, int nvalid, int lane, v4i (&qa)[HD / 64]) {
  DecQ<HD> q;
  dec_q_load<HD>(p, group, q0, nvalid, lane, q);
  dec_q_limbs<HD>(q, lane, qa);
}

// The block's p V and weight sums (waves added in order) to the outputs (one split) or to the split's workspace
// slots; the last block of a tile (counter) adds the slots in split order, writes the outputs and puts the
// workspace back to zero (maxima slots included).
template <int HD>
__device__ __forceinline__ void dec_finish(const AttnArgs& p, DecSmem<HD>& sm, const DecWs& ws, int64_t den,
                                           int64_t (&num)[4][HD / 64], int tile, int sp, int NS, int group, int q0,
                                           int nvalid) {
  constexpr int KK = HD / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, kl = lane & 15, qo = lane >> 4;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) den += __shfl_xor(den, o, 64);
  if (kl == 0) sm.den[w][qo] = den;
  __syncthreads();                                 // red overlays the waves' V rows
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) sm.red[w][i][lane + 64 * kk] = num[i][kk];
  __syncthreads();
  // the block's sums, waves in order: thread u -> (query u / HD, dim u % HD)
  for (int u = threadIdx.x; u < 4 * HD + 4; u += kDecWaves * 64) {
    int64_t t = 0;
    if (u < 4 * HD) {
      for (int ww = 0; ww < kDecWaves; ++ww) t += sm.red[ww][u / HD][u % HD];
    } else {
      for (int ww = 0; ww < kDecWaves; ++ww) t += sm.den[ww][u - 4 * HD];
    }
    const int i = u < 4 * HD ? u / HD : u - 4 * HD;
    if (i >= nvalid) continue;
    if (NS == 1) {
      if (u < 4 * HD) p.num[group * p.snum_tile + (int64_t)(q0 + i) * p.snum_row + u % HD] = t;
      else p.den[group * p.sden_tile + q0 + i] = t;
    } else {
      const int64_t slot = (int64_t)tile * NS + sp;
      if (u < 4 * HD) ws_store(&ws.num[(slot * 4 + i) * HD + u % HD], t);
      else ws_store(&ws.den[slot * 4 + i], t);
    }
  }
  if (NS == 1) return;
  // every split arrives (its slot stores complete first); the last one adds the slots in split order
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = atomicAdd(&ws.sem[tile], 1) == NS - 1;
    if (last) atomicExch(&ws.sem[tile], 0);
    sm.s_last = last;
  }
  __syncthreads();
  if (!sm.s_last) return;
  // every (split, entry) slot is read at once and added into LDS (exact in any order); the slots go back to
  // zero, so the workspace is left as it was found
  int64_t* fin = &sm.red[0][0][0];                 // 4 HD + 4 sums
  for (int u = threadIdx.x; u < 4 * HD + 4; u += kDecWaves * 64) fin[u] = 0;
  __syncthreads();
  constexpr int NT = kDecWaves * 64, UB = 8;      // UB slot loads in flight per thread
  const int nslot = NS * (4 * HD + 4);
  for (int u0 = threadIdx.x; u0 < nslot; u0 += NT * UB) {
    int64_t v[UB];
    int64_t* src[UB];
#pragma unroll
    for (int b = 0; b < UB; ++b) {
      const int u = u0 + b * NT;
      const int k = u / (4 * HD + 4), e = u % (4 * HD + 4);
      const int64_t slot = (int64_t)tile * NS + k;
      src[b] = e < 4 * HD ? &ws.num[slot * 4 * HD + e] : &ws.den[slot * 4 + (e - 4 * HD)];
      v[b] = u < nslot ? ws_load(src[b]) : 0;
    }
#pragma unroll
    for (int b = 0; b < UB; ++b) {
      const int u = u0 + b * NT;
      if (u < nslot) {
        atomicAdd((unsigned long long*)&fin[u % (4 * HD + 4)], (unsigned long long)v[b]);
        ws_store(src[b], 0);
      }
    }
  }
  for (int u = threadIdx.x; u < NS * 4; u += kDecWaves * 64) ws_store(&ws.mx[(int64_t)tile * NS * 4 + u], 0);
  __syncthreads();
  for (int u = threadIdx.x; u < nvalid * HD; u += kDecWaves * 64)
    p.num[group * p.snum_tile + (int64_t)(q0 + u / HD) * p.snum_row + u % HD] = fin[u];
  if (threadIdx.x < nvalid) p.den[group * p.sden_tile + q0 + threadIdx.x] = fin[4 * HD + threadIdx.x];
}

// The decode step's attention output stage (segs.attn_out: div_round + regroup + quant, src/bitexact/exact/segs.py
// and ops.py; the standalone form is attn_out_kernel in csrc/bx_rows.hip) fused into the one-block decode
// attention: ws_p int64 [R, H HD] (scratch) and ws_e int64 [R] / cnt int32 [R] (zero-filled workspace, left zero)
// are the exchange, q int32 [R, ldq] and sh int64 [R] the outputs.
struct AoArgs {
  int64_t* ws_p;
  int64_t* ws_e;
  int32_t* cnt;
  int32_t* q;
  int64_t ldq;
  int64_t* sh;
  int8_t* planes;   // optional: q's signed int8 limb planes [3][R][H HD] (limb i of q[n][c] at i plane + n H HD + c)
  int64_t plane;    // R H HD
  int FR, FV;
};

// The block's sums as dec_finish forms them (waves in order), then its queries' quotients P = div_round(num, FR -
// FV, den) (0 where den = 0), their exponent maximum into the token's slot (atomicMax of emax - kNegBig + 1) and the
// quotients into the token's row of ws_p (agent-scope stores, complete before the count); the token's last block
// quantizes the whole row against the row maximum (rshc(P, shr + FR), shr = max(emax - kQB, NEG_BIG)) and resets
// the slot and the count. No block waits for another.
template <int HD>
__device__ __forceinline__ void dec_finish_ao(const AttnArgs& p, const AoArgs& ao, DecSmem<HD>& sm, int64_t den,
                                              int64_t (&num)[4][HD / 64], int group, int nvalid) {
  constexpr int KK = HD / 64, NT = kDecWaves * 64;
  __shared__ int64_t s_den[4];
  __shared__ int64_t s_red[NT / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, kl = lane & 15, qo = lane >> 4;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) den += __shfl_xor(den, o, 64);
  if (kl == 0) sm.den[w][qo] = den;
  __syncthreads();                                 // red overlays the waves' V rows
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) sm.red[w][i][lane + 64 * kk] = num[i][kk];
  if (threadIdx.x < 4) {
    int64_t t = 0;
    for (int ww = 0; ww < kDecWaves; ++ww) t += sm.den[ww][threadIdx.x];
    s_den[threadIdx.x] = t;
  }
  __syncthreads();
  const int n = group / p.hkv, h = group % p.hkv, G = p.nq;
  const int64_t W = (int64_t)p.hkv * G * HD;
  int64_t emax = kNegBig;
  for (int u = threadIdx.x; u < nvalid * HD; u += NT) {
    const int i = u / HD, d = u % HD;
    int64_t t = 0;
    for (int ww = 0; ww < kDecWaves; ++ww) t += sm.red[ww][i][d];
    const int64_t dn = s_den[i];                   // >= 1 whenever the query sees a key (itself)
    const int64_t v = dn > 0 ? div_round64(t, ao.FR - ao.FV, dn, 1.0 / (double)dn) : 0;
    ws_store(&ao.ws_p[n * W + (int64_t)(h * G + i) * HD + d], v);
    if (v != 0) emax = imax(emax, bitlen(v < 0 ? -v : v) - ao.FR);
  }
  emax = block_max64(emax, s_red);
  if (threadIdx.x == 0) atomicMax((unsigned long long*)&ao.ws_e[n], (unsigned long long)(emax - kNegBig + 1));
  __builtin_amdgcn_s_waitcnt(0);                   // this thread's stores and atomic are complete before the count
  __syncthreads();
  if (threadIdx.x == 0) sm.s_last = atomicAdd(&ao.cnt[n], 1) == p.hkv - 1;
  __syncthreads();
  if (!sm.s_last) return;
  const int64_t em = (int64_t)ws_load(&ao.ws_e[n]) + kNegBig - 1;
  const int64_t shr = imax(em - kQB, kNegBig);
  for (int64_t c = threadIdx.x; c < W; c += NT) {
    const int32_t qv = (int32_t)rshc(ws_load(&ao.ws_p[n * W + c]), shr + ao.FR);
    ao.q[n * ao.ldq + c] = qv;
    if (ao.planes != nullptr) {   // the exact linear's activation planes (split_q_kernel's limbs)
      int32_t r = qv;
#pragma unroll
      for (int l = 0; l < 3; ++l) {
        const int32_t lo = limb_lo(r);
        ao.planes[l * ao.plane + n * W + c] = (int8_t)lo;
        r = (r - lo) >> 8;
      }
    }
  }
  if (threadIdx.x == 0) {
    ao.sh[n] = shr;
    ws_store(&ao.ws_e[n], 0);
    atomicExch(&ao.cnt[n], 0);
  }
}

// RAW (single launch only): sweep 1 keeps every score of the block's key range (p.S >= hi - lo of them per
// query) in dynamic LDS and sweep 2 reads them back, so K is read once.
template <int HD, int PHASE, bool RAW>
__global__ __launch_bounds__(kDecWaves * 64) void attn_dec_kernel(AttnArgs p) {
  __shared__ DecSmem<HD> sm;
  extern __shared__ __align__(16) int64_t raw_cache[];
  constexpr int KK = HD / 64;
  const int tiles = (p.nq + 3) / 4;
  const int tile = blockIdx.x, T = gridDim.x, sp = blockIdx.y, NS = gridDim.y;
  const int group = tile / tiles, q0 = (tile % tiles) * 4;
  const int nvalid = min(4, p.nq - q0);
  const int h = group % p.hkv;
  const int64_t brow = p.rmap ? p.rmap[group / p.hkv] : group / p.hkv;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kl = lane & 15, qo = lane >> 4;
  const DecWs ws = dec_ws(p, T, NS, HD);

  if (threadIdx.x < 4) {
    const int i = threadIdx.x;
    const bool ok = i < nvalid;
    sm.qpos[i] = ok ? p.qpos[(group / p.qpos_div) * p.qpos_tile + (int64_t)(q0 + i) * p.qpos_row] : -1;
    sm.shift[i] = ok && p.sh ? (int64_t)(kFK + 3 - kFZ) - p.sh[group * p.sh_tile + q0 + i] : 0;
    sm.mx[i] = kNeg;
  }
  v4i qa[KK];
  dec_qa<HD>(p, group, q0, nvalid, lane, qa);
  __syncthreads();
  int64_t kend = 0;
  for (int i = 0; i < 4; ++i) kend = imax(kend, sm.qpos[i] + 1);
  int64_t lo64, hi64;
  split_range(kend, NS, sp, lo64, hi64);
  const int lo = (int)lo64, hi = (int)hi64;
  const int64_t my_qpos = sm.qpos[qo];
  const int nb16 = (hi - lo + 15) / 16;

  // ---- sweep 1: maxima over visible keys ----
  if (PHASE == 0 || NS == 1) {
    int64_t best = kNeg;
    KvRegs<HD> cur, nxt;
    // pipeline per wave: rows of block b + 8 and the page of block b + 16 are requested while block b is used
    int pg = 0;
    if (w < nb16) dec_rows<HD, true, false>(p, dec_page(p, brow, min(lo + w * 16 + kl, hi - 1)), h,
                                            min(lo + w * 16 + kl, hi - 1), cur);
    if (w + kDecWaves < nb16) pg = dec_page(p, brow, min(lo + (w + kDecWaves) * 16 + kl, hi - 1));
    for (int b = w; b < nb16; b += kDecWaves) {
      const int s = lo + b * 16 + kl;
      if (b + kDecWaves < nb16) dec_rows<HD, true, false>(p, pg, h, min(s + 16 * kDecWaves, hi - 1), nxt);
      if (b + 2 * kDecWaves < nb16) pg = dec_page(p, brow, min(s + 32 * kDecWaves, hi - 1));
      const int64_t raw = dec_score<HD>(qa, cur);
      if (RAW && s < hi && s - lo < p.S) raw_cache[qo * p.S + (s - lo)] = raw;
      if (s < hi && s <= my_qpos) best = imax(best, raw);
      cur = nxt;
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) best = imax(best, __shfl_xor(best, o, 64));
    if (kl == 0) atomicMax((long long*)&sm.mx[qo], (long long)best);
    __syncthreads();
    if (NS > 1) {                       // PHASE 0: this split's maxima (kNeg: none) into its slot
      if (threadIdx.x < 4) ws_store(&ws.mx[((int64_t)tile * NS + sp) * 4 + threadIdx.x], sm.mx[threadIdx.x] - kNeg);
      return;
    }
  } else {                              // PHASE 1 of a split launch: the maxima over every split
    __syncthreads();                    // sm.mx holds kNeg
    for (int u = threadIdx.x; u < NS * 4; u += kDecWaves * 64)      // every split's slot at once
      atomicMax((long long*)&sm.mx[u & 3], (long long)(ws_load(&ws.mx[(int64_t)tile * NS * 4 + u]) + kNeg));
    __syncthreads();
  }

  // ---- sweep 2: weights, den, num ----
  const int64_t mx = sm.mx[qo];
  const int64_t shift = sm.shift[qo];
  int64_t den = 0;
  int64_t num[4][KK];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) num[i][kk] = 0;
  KvRegs<HD> cur, nxt;
  int pg = 0;
  if (w < nb16) dec_rows<HD, !RAW, true>(p, dec_page(p, brow, min(lo + w * 16 + kl, hi - 1)), h,
                                        min(lo + w * 16 + kl, hi - 1), cur);
  if (w + kDecWaves < nb16) pg = dec_page(p, brow, min(lo + (w + kDecWaves) * 16 + kl, hi - 1));
  for (int b = w; b < nb16; b += kDecWaves) {
    const int s = lo + b * 16 + kl;
    const int64_t raw = RAW ? (s < hi && s - lo < p.S ? raw_cache[qo * p.S + (s - lo)] : 0) : dec_score<HD>(qa, cur);
    // the weight's table loads go out before the next block's requests (loads complete in order: waiting for
    // them then does not wait for the prefetch) and unconditionally (a hidden key's weight is discarded)
    WeightAt wat;
    int64_t ta = 0, tb = 0, i8 = 0;
    if (p.wrule == 0) {
      wat = weight_at(mx - raw, shift, p.l2e);
      ta = p.lut[wat.idx];
      tb = p.lut[wat.idx + 1];
    } else {
      i8 = int8_index(raw - mx, p.zsh, p.zmul);
      ta = p.ptab[imin(imax(i8, 0), -kI8ZLo)];   // a visible key has d <= 0, so idx <= -kI8ZLo (z = 0)
    }
    if (b + kDecWaves < nb16) dec_rows<HD, !RAW, true>(p, pg, h, min(s + 16 * kDecWaves, hi - 1), nxt);
    if (b + 2 * kDecWaves < nb16) pg = dec_page(p, brow, min(s + 32 * kDecWaves, hi - 1));
    int64_t pw = p.wrule == 0 ? weight_of(wat, ta, tb) : (i8 >= 0 ? ta : 0);
    if (!(qo < nvalid && s < hi && s <= my_qpos)) pw = 0;
    den += pw;
    sm.Ps[w][kl][qo] = (int32_t)pw;
    const int c = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int32_t w0 = cur.v[0][kk][e4], w1 = cur.v[1][kk][e4], w2 = cur.v[2][kk][e4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t b0 = (w0 << (24 - 8 * e)) >> 24, b1 = (w1 << (24 - 8 * e)) >> 24, b2 = (w2 << (24 - 8 * e)) >> 24;
          sm.Vs[w][kl][kk * 64 + c * 16 + e4 * 4 + e] = b0 + b1 * 256 + b2 * 65536;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);           // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      int64_t vd[KK];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) vd[kk] = sm.Vs[w][k][lane + 64 * kk];
      const v4i pk = *(const v4i*)&sm.Ps[w][k][0];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t pv = pk[i];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) num[i][kk] += pv * vd[kk];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    cur = nxt;
  }
  dec_finish<HD>(p, sm, ws, den, num, tile, sp, NS, group, q0, nvalid);
}

// A key's weight in two halves: dec_w_issue sends the table loads of one score (always inside the table,
// whatever the score: a hidden key's weight is discarded), dec_w_value forms the weight once they are in.
struct DecW {
  WeightAt wat;
  int64_t ta, tb, i8;
};

__device__ __forceinline__ DecW dec_w_issue(const AttnArgs& p, int64_t raw, int64_t mx, int64_t shift) {
  DecW d;
  d.tb = 0;
  d.i8 = 0;
  if (p.wrule == 0) {
    d.wat = weight_at(mx - raw, shift, p.l2e);
    d.ta = p.lut[d.wat.idx];
    d.tb = p.lut[d.wat.idx + 1];
  } else {
    d.i8 = int8_index(raw - mx, p.zsh, p.zmul);
    d.ta = p.ptab[imin(imax(d.i8, 0), -kI8ZLo)];   // a visible key has d <= 0, so idx <= -kI8ZLo (z = 0)
  }
  return d;
}

__device__ __forceinline__ int64_t dec_w_value(const AttnArgs& p, const DecW& d) {
  return p.wrule == 0 ? weight_of(d.wat, d.ta, d.tb) : (d.i8 >= 0 ? d.ta : 0);
}

// p V of one 16-key block of a wave: the weights (lane: key kl, query qo) and the joined V rows (from the three
// limb planes the lane holds: key kl, dims of chunk lane >> 4) meet in the wave's LDS slice; lane l then adds
// sum_k p[k][i] V[k][l + 64 kk] for the four queries i.
template <int HD>
__device__ __forceinline__ void dec_pv(DecSmem<HD>& sm, int w, int lane, int64_t pw, const v4i (&v)[3][HD / 64],
                                       int64_t (&num)[4][HD / 64]) {
  constexpr int KK = HD / 64;
  const int kl = lane & 15, qo = lane >> 4, c = lane >> 4;
  sm.Ps[w][kl][qo] = (int32_t)pw;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int32_t w0 = v[0][kk][e4], w1 = v[1][kk][e4], w2 = v[2][kk][e4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t b0 = (w0 << (24 - 8 * e)) >> 24, b1 = (w1 << (24 - 8 * e)) >> 24, b2 = (w2 << (24 - 8 * e)) >> 24;
        sm.Vs[w][kl][kk * 64 + c * 16 + e4 * 4 + e] = b0 + b1 * 256 + b2 * 65536;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);           // lgkmcnt(0): this wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    int64_t vd[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) vd[kk] = sm.Vs[w][k][lane + 64 * kk];
    const v4i pk = *(const v4i*)&sm.Ps[w][k][0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t pv = pk[i];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) num[i][kk] += pv * vd[kk];
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
}

// One key row's three limb planes (K: planes 0-2, V: planes 3-5 of the cache row) for the lane: key s of cache
// block pg, dims of chunk lane >> 4.
template <int HD>
__device__ __forceinline__ void dec_planes(const AttnArgs& p, int pg, int h, int s, int first, v4i (&r)[3][HD / 64]) {
  const int c = (threadIdx.x & 63) >> 4;
  const int8_t* row = p.cache + (int64_t)pg * p.sc_nb + (int64_t)h * p.sc_h + (int64_t)(s % p.bs) * p.sc_bs + c * 16;
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int kk = 0; kk < HD / 64; ++kk) r[j][kk] = *(const v4i*)(row + (first + j) * HD + kk * 64);
}

template <int HD>
__device__ __forceinline__ int64_t dec_score_k(const v4i (&qa)[HD / 64], const v4i (&k)[3][HD / 64]) {
  int64_t raw = 0;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int kk = 0; kk < HD / 64; ++kk) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[kk], k[j][kk], acc, 0, 0, 0);
    const int64_t t = (int64_t)acc[0] + ((int64_t)acc[1] << 8) + ((int64_t)acc[2] << 16);
    raw += t << (8 * j);
  }
  return raw;
}

// ---- paged decode attention, one block per query tile, up to kDecRawKeys keys ----
// The tile's block-table entries are copied to LDS first, so locating a key row costs an LDS read rather than a
// memory round trip. Each wave keeps the limb rows of its next DR 16-key blocks in flight (a register ring, the
// loop unrolled by DR). Sweep 1 streams K, keeps every score in LDS and the per-query maxima; sweep 2 streams V
// and forms weights and p V from the kept scores, so K and V are each read once.
// RP (decode steps with one token per sequence): the block first runs the rope kernel's work for its (token, KV
// head): waves 0 .. nq - 1 RoPE and quantize the group's q heads into LDS, waves 4 and 5 RoPE the k head and
// store the k and v limbs at the token's cache slot (each waits for its stores before the barrier, so the
// sweeps read them back). The launch then replaces the standalone rope kernel.
constexpr int kDecDepth = 3;
template <int HD, bool RP = false, bool AO = false>
__global__ __launch_bounds__(kDecWaves * 64) void attn_dec_raw_kernel(AttnArgs p, RopeArgs r, AoArgs ao) {
  static_assert(!RP || kDecWaves >= 6, "the rope prologue uses waves 0-3 (q heads), 4 (k) and 5 (v)");
  BX_PHASE(1, 0);
  __shared__ DecSmem<HD> sm;
  extern __shared__ __align__(16) int64_t raw_cache[];     // [4][p.S] scores, then the block-table entries
  constexpr int KK = HD / 64, DR = kDecDepth;
  const int tiles = (p.nq + 3) / 4;
  const int tile = blockIdx.x;
  const int group = tile / tiles, q0 = (tile % tiles) * 4;
  const int nvalid = min(4, p.nq - q0);
  const int h = group % p.hkv;
  const int64_t brow = p.rmap ? p.rmap[group / p.hkv] : group / p.hkv;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kl = lane & 15, qo = lane >> 4;
  int32_t* spg = (int32_t*)(raw_cache + 4 * (int64_t)p.S);
  __shared__ int32_t s_q[RP ? 4 : 1][RP ? HD : 1];
  __shared__ int64_t s_shq[4];

  DecQ<HD> qv;
  if constexpr (!RP) dec_q_load<HD>(p, group, q0, nvalid, lane, qv);
  // the block-table row (every entry the launch may reach: p.S / bs + 1), independent of the positions
  const int npg = p.S / p.bs + 1 < p.nblk ? p.S / p.bs + 1 : p.nblk;
  for (int i = threadIdx.x; i < npg; i += kDecWaves * 64) spg[i] = p.bt[brow * p.sbt + i];
  // RP: the wave's first DR key blocks that lie wholly below the token's position (no prologue store touches
  // them) are requested before the prologue, straight from the block table; the sweep loads the rest
  v4i kr[DR][3][KK];
  int npre = 0;                                             // wave-uniform: kr[0 .. npre) already requested
  if constexpr (RP) {
    const int64_t pos0 = r.pos[(int64_t)(group / p.hkv) * r.spb];
    const int64_t pe = pos0 < p.S ? pos0 : p.S - 1;        // the last visible key
#pragma unroll
    for (int d = 0; d < DR; ++d) {
      const int i = w + d * kDecWaves;
      if (npre == d && pos0 >= 0 && (int64_t)(i + 1) * 16 <= pe) {   // wave-uniform
        const int s = i * 16 + kl;
        dec_planes<HD>(p, p.bt[brow * p.sbt + s / p.bs], h, s, 0, kr[d]);
        npre = d + 1;
      }
    }
  }
  int64_t qp[4];
  if constexpr (RP) {
    // token group / hkv, KV head h, its nq q heads h nq ..; one position for the group (the token's)
    const int n = group / p.hkv;
    const int64_t pos_raw = r.pos[(int64_t)n * r.spb];
    bool bad = pos_raw < 0 || pos_raw >= r.npos;        // the reference's table index would fail: flagged
    const int64_t pos = imin(imax(pos_raw, 0), r.npos - 1);
    int64_t out[KK];
    if (w < nvalid) {
      rope_row<HD>(r, n, h * p.nq + w, pos, lane, out, bad);
      const int64_t shq = rope_q_shift<HD>(r, out, bad);
#pragma unroll
      for (int e = 0; e < KK; ++e) s_q[w][lane + 64 * e] = (int32_t)rshc(out[e], shq + r.FR + r.FT);
      if (lane == 0) s_shq[w] = shq;
    } else if (w == 4 || w == 5) {
      const int hr = r.H + (w - 4) * r.HKV + h;
      rope_row<HD>(r, n, hr, pos, lane, out, bad);
      rope_kv_store<HD>(r, n, hr, lane, out, bad);
      __builtin_amdgcn_s_waitcnt(0);                     // the cache stores are complete before the barrier
    }
    if (wave_or(bad ? 1 : 0) && lane == 0) r.err[0] = 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) qp[i] = i < nvalid ? pos_raw : -1;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      qp[i] = i < nvalid ? p.qpos[(group / p.qpos_div) * p.qpos_tile + (int64_t)(q0 + i) * p.qpos_row] : -1;
  }
  const int kend = (int)imin(imax(imax(qp[0], qp[1]), imax(qp[2], qp[3])) + 1, p.S);   // qpos < nblk bs <= p.S
  const int64_t my_qpos = qo == 0 ? qp[0] : qo == 1 ? qp[1] : qo == 2 ? qp[2] : qp[3];
  if (threadIdx.x < 4) sm.mx[threadIdx.x] = kNeg;
  int64_t shift = 0;
  if constexpr (!RP) shift = qo < nvalid && p.sh ? (int64_t)(kFK + 3 - kFZ) - p.sh[group * p.sh_tile + q0 + qo] : 0;
  __syncthreads();
  if constexpr (RP) {
    // the queries from LDS in dec_q_load's lane layout: query (lane & 15) >> 2, dims 16 (lane >> 4) + e
    const int m = lane & 15, qi = m >> 2, c = lane >> 4;
    const bool live = qi < nvalid && (m & 3) < 3;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int e = 0; e < 16; ++e) qv.x[kk][e] = live ? s_q[qi][kk * 64 + c * 16 + e] : 0;
    shift = qo < nvalid ? (int64_t)(kFK + 3 - kFZ) - s_shq[qo] : 0;
  }
  v4i qa[KK];
  dec_q_limbs<HD>(qv, lane, qa);
  const int nb16 = (kend + 15) / 16;
  BX_PHASE(1, 1);
  auto rows = [&](int i, int first, v4i (&r)[3][KK]) {
    const int s = min(i * 16 + kl, kend - 1);
    dec_planes<HD>(p, spg[s / p.bs], h, s, first, r);
  };

  // ---- sweep 1: K, scores into LDS, maxima ----
  {
#pragma unroll
    for (int d = 0; d < DR; ++d)
      if (d >= npre && w + d * kDecWaves < nb16) rows(w + d * kDecWaves, 0, kr[d]);
    int64_t best = kNeg;
    for (int b0 = w; b0 < nb16; b0 += DR * kDecWaves) {
#pragma unroll
      for (int d = 0; d < DR; ++d) {
        const int i = b0 + d * kDecWaves;
        if (i < nb16) {                              // wave-uniform
          const int64_t raw = dec_score_k<HD>(qa, kr[d]);
          if (i + DR * kDecWaves < nb16) rows(i + DR * kDecWaves, 0, kr[d]);
          const int s = i * 16 + kl;
          if (s < kend) raw_cache[qo * p.S + s] = raw;
          if (s < kend && s <= my_qpos) best = imax(best, raw);
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) best = imax(best, __shfl_xor(best, o, 64));
    if (kl == 0) atomicMax((long long*)&sm.mx[qo], (long long)best);
  }
  BX_PHASE(1, 2);
  // the first V rows go out before the maxima are complete
  v4i vr[DR][3][KK];
#pragma unroll
  for (int d = 0; d < DR; ++d)
    if (w + d * kDecWaves < nb16) rows(w + d * kDecWaves, 3, vr[d]);
  __builtin_amdgcn_s_waitcnt(0xc07f);             // LDS only (lgkmcnt(0)): the V loads stay in flight
  asm volatile("s_barrier" ::: "memory");

  BX_PHASE(1, 3);
  // ---- sweep 2: V, weights from the kept scores, den, p V ----
  const int64_t mx = sm.mx[qo];
  int64_t den = 0;
  int64_t num[4][KK];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) num[i][kk] = 0;
  for (int b0 = w; b0 < nb16; b0 += DR * kDecWaves) {
#pragma unroll
    for (int d = 0; d < DR; ++d) {
      const int i = b0 + d * kDecWaves;
      if (i < nb16) {                                // wave-uniform
        const int s = i * 16 + kl;
        const int64_t raw = s < kend ? raw_cache[qo * p.S + s] : 0;
        const DecW wt = dec_w_issue(p, raw, mx, shift);
        int64_t pw = dec_w_value(p, wt);
        if (!(qo < nvalid && s < kend && s <= my_qpos)) pw = 0;
        den += pw;
        dec_pv<HD>(sm, w, lane, pw, vr[d], num);
        if (i + DR * kDecWaves < nb16) rows(i + DR * kDecWaves, 3, vr[d]);
      }
    }
  }
  BX_PHASE(1, 4);
  if constexpr (AO)
    dec_finish_ao<HD>(p, ao, sm, den, num, group, nvalid);
  else
    dec_finish<HD>(p, sm, DecWs{}, den, num, tile, 0, 1, group, q0, nvalid);
  BX_PHASE(1, 5);
}

// ---- paged decode attention, key splits in one launch ----
// Grid (query tiles, key splits), every block normally resident at once (the host takes this kernel for at most
// one block per compute unit). A block's key range is at most 16 NBW kDecWaves keys, so wave w holds the K and V
// limb rows of its NBW 16-key blocks in registers: the block-table entries, then every K and V row, are requested
// at once, before the queries are read. Scores stay in registers. The splits of a tile exchange their maxima
// through the workspace: each publishes its own (as mx - kNeg + 1; 0 = not yet published) and waits for the
// others' for at most p.exch_ticks of the 100 MHz real-time counter; a block that has not seen them all by then
// computes the maxima over the tile's keys itself, so the wait always ends and the integers never depend on which
// blocks ran together. Weights, p V and the split sums then follow attn_dec_kernel's sweep 2 and dec_finish,
// so K and V are each read once.
template <int HD, int NBW>
__global__ __launch_bounds__(kDecWaves * 64) void attn_dec_exch_kernel(AttnArgs p) {
  BX_PHASE(0, 0);
  __shared__ DecSmem<HD> sm;
  __shared__ int64_t s_best[kDecWaves][4];
  constexpr int KK = HD / 64;
  const int tiles = (p.nq + 3) / 4;
  const int tile = blockIdx.x, T = gridDim.x, sp = blockIdx.y, NS = gridDim.y;
  const int group = tile / tiles, q0 = (tile % tiles) * 4;
  const int nvalid = min(4, p.nq - q0);
  const int h = group % p.hkv;
  const int64_t brow = p.rmap ? p.rmap[group / p.hkv] : group / p.hkv;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kl = lane & 15, qo = lane >> 4;
  const DecWs ws = dec_ws(p, T, NS, HD);

  DecQ<HD> qv;                                     // the queries first: used after every other request
  dec_q_load<HD>(p, group, q0, nvalid, lane, qv);
  // the tile's query positions, read by every lane (the key range needs their maximum)
  int64_t qp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    qp[i] = i < nvalid ? p.qpos[(group / p.qpos_div) * p.qpos_tile + (int64_t)(q0 + i) * p.qpos_row] : -1;
  const int64_t kend = imax(imax(qp[0], qp[1]), imax(qp[2], qp[3])) + 1;
  const int64_t my_qpos = qo == 0 ? qp[0] : qo == 1 ? qp[1] : qo == 2 ? qp[2] : qp[3];
  int64_t lo64, hi64;
  split_range(kend, NS, sp, lo64, hi64);
  const int lo = (int)lo64, hi = (int)hi64;
  const int nb16 = (hi - lo + 15) / 16;            // <= NBW kDecWaves (the host's bound on the split size)
  int pg[NBW];
#pragma unroll
  for (int t = 0; t < NBW; ++t)
    pg[t] = w + t * kDecWaves < nb16 ? dec_page(p, brow, min(lo + (w + t * kDecWaves) * 16 + kl, hi - 1)) : 0;
  KvRegs<HD> kv[NBW];
#pragma unroll
  for (int t = 0; t < NBW; ++t)
    if (w + t * kDecWaves < nb16)
      dec_rows<HD, true, true>(p, pg[t], h, min(lo + (w + t * kDecWaves) * 16 + kl, hi - 1), kv[t]);
  if (threadIdx.x < 4) sm.mx[threadIdx.x] = kNeg;
  const int64_t shift = qo < nvalid && p.sh ? (int64_t)(kFK + 3 - kFZ) - p.sh[group * p.sh_tile + q0 + qo] : 0;
  v4i qa[KK];
  dec_q_limbs<HD>(qv, lane, qa);

  // scores and this split's maxima
  int64_t raw[NBW];
  int64_t best = kNeg;
#pragma unroll
  for (int t = 0; t < NBW; ++t) {
    raw[t] = 0;
    if (w + t * kDecWaves < nb16) {                // wave-uniform
      const int s = lo + (w + t * kDecWaves) * 16 + kl;
      raw[t] = dec_score<HD>(qa, kv[t]);
      if (s < hi && s <= my_qpos) best = imax(best, raw[t]);
    }
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) best = imax(best, __shfl_xor(best, o, 64));
  if (kl == 0) s_best[w][qo] = best;
  __syncthreads();
  BX_PHASE(0, 1);
  if (threadIdx.x < 4) {
    int64_t m = kNeg;
    for (int ww = 0; ww < kDecWaves; ++ww) m = imax(m, s_best[ww][threadIdx.x]);
    ws_store(&ws.mx[((int64_t)tile * NS + sp) * 4 + threadIdx.x], m - kNeg + 1);
  }
  bool seen = true;
  if (threadIdx.x < NS * 4) {
    int64_t* a = &ws.mx[(int64_t)tile * NS * 4 + threadIdx.x];
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    int64_t v = ws_load(a);
    while (v == 0 && __builtin_amdgcn_s_memrealtime() - t0 < p.exch_ticks) {
      __builtin_amdgcn_s_sleep(1);
      v = ws_load(a);
    }
    seen = v != 0;
    if (seen) atomicMax((long long*)&sm.mx[threadIdx.x & 3], (long long)(v - 1 + kNeg));
  }
  if (!__syncthreads_and(seen)) {
    // maxima over every key of the tile, from the cache (rows of 16 keys, the waves in turn)
    const int nall = (int)((kend + 15) / 16);
    int64_t b2 = kNeg;
    for (int i = w; i < nall; i += kDecWaves) {
      const int s = min(i * 16 + kl, (int)kend - 1);
      KvRegs<HD> r;
      dec_rows<HD, true, false>(p, dec_page(p, brow, s), h, s, r);
      const int64_t sc = dec_score<HD>(qa, r);
      if (i * 16 + kl < kend && s <= my_qpos) b2 = imax(b2, sc);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) b2 = imax(b2, __shfl_xor(b2, o, 64));
    if (kl == 0) atomicMax((long long*)&sm.mx[qo], (long long)b2);
    __syncthreads();
  }

  BX_PHASE(0, 2);
  // weights (every table load first), den, p V
  const int64_t mx = sm.mx[qo];
  int64_t pw[NBW];
  {
    WeightAt wat[NBW];
    int64_t ta[NBW], tb[NBW], i8[NBW];
#pragma unroll
    for (int t = 0; t < NBW; ++t) {
      if (p.wrule == 0) {
        wat[t] = weight_at(mx - raw[t], shift, p.l2e);
        ta[t] = p.lut[wat[t].idx];
        tb[t] = p.lut[wat[t].idx + 1];
      } else {
        i8[t] = int8_index(raw[t] - mx, p.zsh, p.zmul);
        ta[t] = p.ptab[imin(imax(i8[t], 0), -kI8ZLo)];   // a visible key has d <= 0, so idx <= -kI8ZLo (z = 0)
      }
    }
#pragma unroll
    for (int t = 0; t < NBW; ++t) {
      const int s = lo + (w + t * kDecWaves) * 16 + kl;
      pw[t] = p.wrule == 0 ? weight_of(wat[t], ta[t], tb[t]) : (i8[t] >= 0 ? ta[t] : 0);
      if (!(w + t * kDecWaves < nb16 && qo < nvalid && s < hi && s <= my_qpos)) pw[t] = 0;
    }
  }
  int64_t den = 0;
  int64_t num[4][KK];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) num[i][kk] = 0;
  const int c = lane >> 4;
#pragma unroll
  for (int t = 0; t < NBW; ++t) {
    if (w + t * kDecWaves >= nb16) break;          // wave-uniform
    den += pw[t];
    sm.Ps[w][kl][qo] = (int32_t)pw[t];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int32_t w0 = kv[t].v[0][kk][e4], w1 = kv[t].v[1][kk][e4], w2 = kv[t].v[2][kk][e4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t b0 = (w0 << (24 - 8 * e)) >> 24, b1 = (w1 << (24 - 8 * e)) >> 24, b2 = (w2 << (24 - 8 * e)) >> 24;
          sm.Vs[w][kl][kk * 64 + c * 16 + e4 * 4 + e] = b0 + b1 * 256 + b2 * 65536;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);           // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      int64_t vd[KK];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) vd[kk] = sm.Vs[w][k][lane + 64 * kk];
      const v4i pk = *(const v4i*)&sm.Ps[w][k][0];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t pv = pk[i];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) num[i][kk] += pv * vd[kk];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  }
  BX_PHASE(0, 3);
  dec_finish<HD>(p, sm, ws, den, num, tile, sp, NS, group, q0, nvalid);
  BX_PHASE(0, 4);
}

// ---- fused prefill attention on MFMA (contiguous int32 K / V) ----
// A block (4 waves) owns 64 consecutive query rows of one group z; wave w owns rows 16 w .. 16 w + 15. Keys go
// in 64-key tiles staged in LDS as int8 limb planes: K row-major (Ks[j][key][dim], the QK B operand: a lane's
// 16 bytes are 16 dims of one key) and V transposed (Vt[j][dim][key], the PV B operand: 16 keys of one dim).
// QK: for each 16-key block, A = limb i of the wave's 16 queries (registers), B = K limb plane j; the nine limb
// products accumulate by weight i + j in five int32 sets, joined in int64 per score (lane: query rows
// 4 (lane >> 4) + e, key lane & 15). Sweep 1 keeps per-row maxima; sweep 2 turns scores into weights p, writes
// p's three limbs to the wave's LDS slice (Pl[i][query][key]) and runs PV on MFMA: A = limb i of p (16
// queries x 64 keys), B = V limb plane j (64 keys x 16 dims), five int32 sets per 16-dim block, exact while
// S 3 2^14 < 2^31 (S < 43690), joined in int64 at the end.
template <int HD>
struct PreSmem {
  int8_t Ks[3][64][HD + 16];
  int8_t Vt[3][HD][64 + 16];
  int8_t Pl[4][3][16][64 + 16];
};

// A tile's K / V rows in registers (thread -> K: (key, 16-dim chunk) units; V: (4 keys, 4 dims) units), loaded
// while the previous tile is computed, then split into limb planes in LDS.
template <int HD>
struct PreRegs {
  v4i k[HD / 64][4];
  v4i v[HD / 64][4];
};

template <int HD>
__device__ __forceinline__ void pre_load(const AttnArgs& p, PreRegs<HD>& r, int z, int key0, int kend, bool want_v) {
#pragma unroll
  for (int t = 0; t < HD / 64; ++t) {
    const int u = threadIdx.x + t * 256;
    const int kk = u / (HD / 16), c = u % (HD / 16);
    const int s = min(key0 + kk, kend - 1);
    const int32_t* kr = p.K + (int64_t)z * p.sk_z + (int64_t)s * p.sk_s + c * 16;
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) r.k[t][e4] = *(const v4i*)(kr + e4 * 4);
    if (want_v) {
      const int kq = u % 16, dq = u / 16;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int sv = min(key0 + 4 * kq + m, kend - 1);
        r.v[t][m] = *(const v4i*)(p.V + (int64_t)z * p.sv_z + (int64_t)sv * p.sv_s + dq * 4);
      }
    }
  }
}

template <int HD>
__device__ __forceinline__ void pre_store(PreSmem<HD>& sm, const PreRegs<HD>& r, bool want_v) {
#pragma unroll
  for (int t = 0; t < HD / 64; ++t) {
    const int u = threadIdx.x + t * 256;
    const int kk = u / (HD / 16), c = u % (HD / 16);
    uint32_t w0[4], w1[4], w2[4];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) split3(r.k[t][e4], w0[e4], w1[e4], w2[e4]);
    *(v4i*)&sm.Ks[0][kk][c * 16] = v4i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3]};
    *(v4i*)&sm.Ks[1][kk][c * 16] = v4i{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
    *(v4i*)&sm.Ks[2][kk][c * 16] = v4i{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
    if (want_v) {
      const int kq = u % 16, dq = u / 16;
      uint32_t l[4][3];
#pragma unroll
      for (int m = 0; m < 4; ++m) split3(r.v[t][m], l[m][0], l[m][1], l[m][2]);
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t word = ((l[0][j] >> (8 * d)) & 255) | (((l[1][j] >> (8 * d)) & 255) << 8) |
                                (((l[2][j] >> (8 * d)) & 255) << 16) | (((l[3][j] >> (8 * d)) & 255) << 24);
          *(uint32_t*)&sm.Vt[j][dq * 4 + d][kq * 4] = word;
        }
    }
  }
}

template <int HD>
__device__ __forceinline__ void pre_scores(const PreSmem<HD>& sm, const v4i (&qa)[3][HD / 64], int kb, int64_t (&raw)[4]) {
  const int lane = threadIdx.x & 63;
  v4i acc[5];
#pragma unroll
  for (int w = 0; w < 5; ++w) acc[w] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int kk = 0; kk < HD / 64; ++kk)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const v4i b = *(const v4i*)&sm.Ks[j][kb * 16 + (lane & 15)][kk * 64 + (lane >> 4) * 16];
#pragma unroll
      for (int i = 0; i < 3; ++i) acc[i + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[i][kk], b, acc[i + j], 0, 0, 0);
    }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    int64_t r = 0;
#pragma unroll
    for (int w = 0; w < 5; ++w) r += (int64_t)acc[w][e] << (8 * w);
    raw[e] = r;
  }
}

template <int HD>
__global__ __launch_bounds__(256, HD == 64 ? 2 : 1) void attn_pre_kernel(AttnArgs p) {
  extern __shared__ __align__(16) char smem_raw[];
  PreSmem<HD>& sm = *(PreSmem<HD>*)smem_raw;
  constexpr int KK = HD / 64, DB = HD / 16;
  const int tiles = (p.nq + 63) / 64;
  const int z = blockIdx.x / tiles, q0 = (blockIdx.x % tiles) * 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // A operands: limb i of query q0 + 16 w + (lane & 15), dims kk 64 + (lane >> 4) 16 + [0, 16)
  v4i qa[3][KK];
  {
    const int qr = min(q0 + 16 * w + (lane & 15), p.nq - 1);
    const int32_t* qp = p.q + (int64_t)z * p.sq_tile + (int64_t)qr * p.sq_row;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint32_t l[3][4];
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        split3(*(const v4i*)(qp + kk * 64 + (lane >> 4) * 16 + e4 * 4), l[0][e4], l[1][e4], l[2][e4]);
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) qa[i][kk] = v4i{(int)l[i][0], (int)l[i][1], (int)l[i][2], (int)l[i][3]};
    }
  }
  // this lane's output rows: 16 w + 4 (lane >> 4) + e
  int64_t qpos[4], shift[4], mx[4];
  int64_t kend = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = q0 + 16 * w + 4 * (lane >> 4) + e;
    const bool ok = r < p.nq;
    qpos[e] = ok ? p.qpos[(z / p.qpos_div) * p.qpos_tile + (int64_t)r * p.qpos_row] : -1;
    shift[e] = ok ? (int64_t)(kFK + 3 - kFZ) - p.sh[z * p.sh_tile + r] : 0;
    mx[e] = kNeg;
    kend = imax(kend, qpos[e] + 1);
  }
  // the block's key range: the largest visible key of its rows (bounded by the cache)
  __shared__ int64_t s_kend;
  if (threadIdx.x == 0) s_kend = 0;
  __syncthreads();
  atomicMax((long long*)&s_kend, (long long)kend);
  __syncthreads();
  const int kb_end = (int)imin(s_kend, (int64_t)p.S);
  const int ntile = (kb_end + 63) / 64;

  // ---- sweep 1: row maxima ----
  PreRegs<HD> kv;
  if (ntile > 0) pre_load<HD>(p, kv, z, 0, kb_end, false);
  for (int t = 0; t < ntile; ++t) {
    __syncthreads();
    pre_store<HD>(sm, kv, false);
    __syncthreads();
    if (t + 1 < ntile) pre_load<HD>(p, kv, z, (t + 1) * 64, kb_end, false);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      int64_t raw[4];
      pre_scores<HD>(sm, qa, kb, raw);
      const int s = t * 64 + kb * 16 + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (s < kb_end && s <= qpos[e]) mx[e] = imax(mx[e], raw[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mx[e] = imax(mx[e], __shfl_xor(mx[e], o, 64));

  // ---- sweep 2: weights, den, PV ----
  int64_t den[4] = {0, 0, 0, 0};
  v4i pacc[DB][5];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int ww = 0; ww < 5; ++ww) pacc[d][ww] = v4i{0, 0, 0, 0};
  if (ntile > 0) pre_load<HD>(p, kv, z, 0, kb_end, true);
  for (int t = 0; t < ntile; ++t) {
    __syncthreads();
    pre_store<HD>(sm, kv, true);
    __syncthreads();
    if (t + 1 < ntile) pre_load<HD>(p, kv, z, (t + 1) * 64, kb_end, true);
    // per 16-key block, its 8 table loads are issued before any weight is formed (a load under a per-score
    // branch would wait alone); NKB blocks at a time
    constexpr int NKB = 1;
#pragma unroll
    for (int kb2 = 0; kb2 < 4; kb2 += NKB) {
      WeightAt wa[NKB][4];
      int64_t ta[NKB][4], tb[NKB][4];
#pragma unroll
      for (int h = 0; h < NKB; ++h) {
        int64_t raw[4];
        pre_scores<HD>(sm, qa, kb2 + h, raw);
#pragma unroll
        for (int e = 0; e < 4; ++e) wa[h][e] = weight_at(mx[e] - raw[e], shift[e], p.l2e);
      }
#pragma unroll
      for (int h = 0; h < NKB; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ta[h][e] = p.lut[wa[h][e].idx];
          tb[h][e] = p.lut[wa[h][e].idx + 1];
        }
#pragma unroll
      for (int h = 0; h < NKB; ++h) {
      const int kb = kb2 + h;
      const int s = t * 64 + kb * 16 + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t w8 = weight_of(wa[h][e], ta[h][e], tb[h][e]);
        const int64_t pw = (s < kb_end && s <= qpos[e]) ? w8 : 0;
        den[e] += pw;
        int32_t x = (int32_t)pw;                         // 0 <= p <= 2^22: three limbs
        const int32_t a0 = limb_lo(x);
        x = (x - a0) >> 8;
        const int32_t a1 = limb_lo(x);
        x = (x - a1) >> 8;
        const int row = 4 * (lane >> 4) + e, col = kb * 16 + (lane & 15);
        sm.Pl[w][0][row][col] = (int8_t)a0;
        sm.Pl[w][1][row][col] = (int8_t)a1;
        sm.Pl[w][2][row][col] = (int8_t)limb_lo(x);
      }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);                  // this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    v4i pa[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) pa[i] = *(const v4i*)&sm.Pl[w][i][lane & 15][(lane >> 4) * 16];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const v4i b = *(const v4i*)&sm.Vt[j][d * 16 + (lane & 15)][(lane >> 4) * 16];
#pragma unroll
        for (int i = 0; i < 3; ++i) pacc[d][i + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa[i], b, pacc[d][i + j], 0, 0, 0);
      }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) den[e] += __shfl_xor(den[e], o, 64);
  // outputs: lane holds rows 4 (lane >> 4) + e of the wave, dims d 16 + (lane & 15)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = q0 + 16 * w + 4 * (lane >> 4) + e;
    if (r >= p.nq) continue;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      int64_t v = 0;
#pragma unroll
      for (int ww = 0; ww < 5; ++ww) v += (int64_t)pacc[d][ww][e] << (8 * ww);
      p.num[z * p.snum_tile + (int64_t)r * p.snum_row + d * 16 + (lane & 15)] = v;
    }
    if ((lane & 15) == 0) p.den[z * p.sden_tile + r] = den[e];
  }
}

// ---- fused prefill attention, limb-plane form (contiguous int32 K / V, with a scratch buffer) ----
// pre_split_kernel writes K and V once as int8 limb planes, padded with zeros to Sp (a multiple of 64 keys):
// Kp [Z][3][Sp][HD] (key rows: the QK A operand) and Vp [Z][3][HD][Sp] (dim rows: the PV B operand), the keys of
// every 64-key tile of Vp in MFMA k order: position 16 c + 4 kb + e holds key 16 kb + 4 c + e. That is the order in
// which the transposed QK product leaves the weights in the lanes (below), so the weights go from registers
// straight into the PV A operand.
__device__ __forceinline__ int pre_vpos(int key) {   // tile key -> its Vp position
  return ((key >> 2) & 3) * 16 + ((key >> 4) & 3) * 4 + (key & 3);
}

__global__ __launch_bounds__(256) void pre_split_kernel(AttnArgs p, int8_t* kp, int8_t* vp, int64_t* tab2, int Z, int Sp,
                                                        int HD) {
  const int CR = HD / 16;
  const int64_t nk = (int64_t)Z * Sp * CR;          // K units: (z, key, 16-dim chunk)
  const int64_t nv = (int64_t)Z * (Sp / 4) * (HD / 4);   // V units: (z, 4 keys, 4 dims)
  const int64_t nt = 1 << kExp2Bits;                 // table pairs: (lut[i], lut[i + 1] - lut[i])
  for (int64_t u = blockIdx.x * 256LL + threadIdx.x; u < nk + nv + nt; u += (int64_t)gridDim.x * 256) {
    if (u >= nk + nv) {
      const int64_t i = u - nk - nv;
      const int64_t a = p.lut[i];
      tab2[2 * i] = a;
      tab2[2 * i + 1] = p.lut[i + 1] - a;
    } else if (u < nk) {
      const int c = (int)(u % CR), s = (int)((u / CR) % Sp), z = (int)(u / ((int64_t)CR * Sp));
      uint32_t l[3][4];
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const v4i v = s < p.S ? *(const v4i*)(p.K + (int64_t)z * p.sk_z + (int64_t)s * p.sk_s + c * 16 + e4 * 4)
                              : v4i{0, 0, 0, 0};
        split3(v, l[0][e4], l[1][e4], l[2][e4]);
      }
#pragma unroll
      for (int j = 0; j < 3; ++j)
        *(v4i*)(kp + (((int64_t)z * 3 + j) * Sp + s) * HD + c * 16) =
            v4i{(int)l[j][0], (int)l[j][1], (int)l[j][2], (int)l[j][3]};
    } else {
      const int64_t w = u - nk;
      const int d4 = (int)(w % (HD / 4)), s4 = (int)((w / (HD / 4)) % (Sp / 4)), z = (int)(w / ((int64_t)(HD / 4) * (Sp / 4)));
      uint32_t l[4][3];   // [key m][plane j]: the 4 dims' limbs
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int s = s4 * 4 + m;
        const v4i v = s < p.S ? *(const v4i*)(p.V + (int64_t)z * p.sv_z + (int64_t)s * p.sv_s + d4 * 4) : v4i{0, 0, 0, 0};
        split3(v, l[m][0], l[m][1], l[m][2]);
      }
      const int key0 = (s4 * 4) & 63, tile0 = (s4 * 4) & ~63;
      const int pos = tile0 + pre_vpos(key0);      // the 4 keys stay consecutive
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t word = ((l[0][j] >> (8 * d)) & 255) | (((l[1][j] >> (8 * d)) & 255) << 8) |
                                (((l[2][j] >> (8 * d)) & 255) << 16) | (((l[3][j] >> (8 * d)) & 255) << 24);
          *(uint32_t*)(vp + (((int64_t)z * 3 + j) * HD + d4 * 4 + d) * Sp + pos) = word;
        }
    }
  }
}

// attn_pre2_kernel: a block (8 waves at head_dim 64, 4 at 128) owns 16 rows per wave of consecutive query rows of
// one group z, wave w rows 16 w .. 16 w + 15.
// The 64-key tiles of the limb planes stream through an NS-stage LDS ring filled by buffer_load ... lds (1 KiB
// per wave instruction; 16-byte chunks XOR-swizzled by row so the 16 rows an MFMA operand read touches fall in
// distinct bank groups). QK is computed transposed: A = K limb plane j (16 keys x 64 dims), B = limb i of the
// wave's 16 queries (registers), so lane l receives query l & 15's scores for keys 16 kb + 4 (l >> 4) + e; the
// nine limb products accumulate by weight i + j in five int32 sets, joined in int64. Sweep 1 keeps the per-query
// maxima. Sweep 2 forms the weights in the same lanes; their three limbs, packed in key order 4 kb + e, are the
// PV A operand as they stand (16 queries x 64 keys in Vp's order), and B = V limb plane j (64 keys x 16 dims):
// five int32 sets per 16-dim block (exact while S 3 2^14 < 2^31), joined in int64 at the end. The table loads of
// a tile's 16 weights go out together, before the tile's next ring stage is requested.
// Byte k of each of four words, in order, as one word (two v_perm_b32 and an or).
template <int k>
__device__ __forceinline__ uint32_t gather_bytes(const uint32_t (&a)[4]) {
  const uint32_t lo = __builtin_amdgcn_perm(a[1], a[0], 0x0c0c0400u + k * 0x101u);        // a0.k, a1.k, 0, 0
  const uint32_t hi = __builtin_amdgcn_perm(a[3], a[2], 0x04000c0cu + k * 0x01010000u);    // 0, 0, a2.k, a3.k
  return lo | hi;
}

template <int HD>
struct Pre2 {
  static constexpr int KK = HD / 64, CR = HD / 16, DB = HD / 16;
  static constexpr int NS = HD == 64 ? 3 : 2;        // ring stages
  static constexpr int PB = 3 * 64 * HD;             // one operand's three planes of a tile (bytes)
  static constexpr int STAGE = 2 * PB;               // K then V
  static constexpr int KI = PB / 1024;               // 1 KiB instructions per operand
  static constexpr int NW = HD == 64 ? 8 : 4;        // waves (16 query rows each): 2 per SIMD at HD 64, 1 at 128
  static constexpr int LPK = (KI + NW - 1) / NW;     // sweep 1 (K only): instructions per issuing wave
  static constexpr int LPT = 2 * KI / NW;            // sweep 2: instructions per wave
  static constexpr size_t LDS = (size_t)NS * STAGE;
};

__device__ __forceinline__ int pre_swzk(int k, int HD) { return HD == 64 ? (k >> 2) & 3 : (k >> 1) & 7; }
__device__ __forceinline__ int pre_swzv(int d) { return (d >> 2) & 3; }

template <int HD>
__global__ __launch_bounds__(64 * Pre2<HD>::NW, 1) void attn_pre2_kernel(AttnArgs p, const int8_t* planes, int Z,
                                                                         int Sp, const char* tab2) {
  using C = Pre2<HD>;
  constexpr int QR = 16 * C::NW;                     // query rows per block
  constexpr int KK = C::KK, DB = C::DB, NS = C::NS;
  extern __shared__ __align__(16) char smem[];
  __shared__ int s_kend;
  const int tiles = (p.nq + QR - 1) / QR;
  const int z = blockIdx.x % Z, q0 = (tiles - 1 - blockIdx.x / Z) * QR;    // late (long) row tiles first
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kl = lane & 15, c = lane >> 4;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(planes), (short)0, kBufRange, 0x00020000);
  const int64_t vbase = (int64_t)Z * 3 * Sp * HD;

  // the lane's query (B operand rows) and its position / exponent
  const int qr = q0 + 16 * w + kl;
  v4i qb[3][KK];
  {
    const int32_t* qp = p.q + (int64_t)z * p.sq_tile + (int64_t)min(qr, p.nq - 1) * p.sq_row;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint32_t l[3][4];
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) split3(*(const v4i*)(qp + kk * 64 + c * 16 + e4 * 4), l[0][e4], l[1][e4], l[2][e4]);
#pragma unroll
      for (int i = 0; i < 3; ++i) qb[i][kk] = v4i{(int)l[i][0], (int)l[i][1], (int)l[i][2], (int)l[i][3]};
    }
  }
  const bool live = qr < p.nq;
  // (positions past S - 1 see every key: the caller's contract keeps qpos < S, so the clamp changes nothing)
  const int my_qpos =
      live ? (int)imin(p.qpos[(z / p.qpos_div) * p.qpos_tile + (int64_t)qr * p.qpos_row], (int64_t)p.S) : -1;
  const int64_t shift = live ? (int64_t)(kFK + 3 - kFZ) - p.sh[z * p.sh_tile + qr] : 0;
  if (threadIdx.x == 0) s_kend = 0;
  __syncthreads();
  {
    int64_t ke = wave_max64(my_qpos + 1);
    if (lane == 0) atomicMax(&s_kend, (int)ke);
  }
  __syncthreads();
  const int kend = min(s_kend, p.S);                 // keys [0, kend) are visible to some row of the block
  const int ntile = (kend + 63) / 64;

  // DMA offsets of the wave's instructions (tile 0) and their per-tile step
  auto dma_off = [&](int n, int& off, int& step) {
    if (n < C::KI) {
      const int j = n / (C::KI / 3), o = (n % (C::KI / 3)) * 1024 + lane * 16;
      const int k = o / HD, cc = ((o % HD) / 16) ^ pre_swzk(k, HD);
      off = (int)((((int64_t)z * 3 + j) * Sp + k) * HD + cc * 16);
      step = 64 * HD;
    } else {
      const int m = n - C::KI;
      const int j = m / (C::KI / 3), o = (m % (C::KI / 3)) * 1024 + lane * 16;
      const int d = o / 64, cc = ((o % 64) / 16) ^ pre_swzv(d);
      off = (int)(vbase + (((int64_t)z * 3 + j) * HD + d) * Sp + cc * 16);
      step = 64;
    }
  };
  int off1[C::LPK], stp1[C::LPK], off2[C::LPT], stp2[C::LPT];
#pragma unroll
  for (int i = 0; i < C::LPK; ++i) dma_off(min(w * C::LPK + i, C::KI - 1), off1[i], stp1[i]);
#pragma unroll
  for (int i = 0; i < C::LPT; ++i) dma_off(w * C::LPT + i, off2[i], stp2[i]);
  const bool k_issuer = w * C::LPK < C::KI;          // sweep 1: the waves that load K
  auto issue1 = [&](int t) {
    char* base = smem + (t % NS) * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::LPK; ++i)
      if (w * C::LPK + i < C::KI) buf_lds16(rs, base + (w * C::LPK + i) * 1024, off1[i] + t * stp1[i], 0);
  };
  auto issue2 = [&](int t) {
    char* base = smem + (t % NS) * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::LPT; ++i) buf_lds16(rs, base + (w * C::LPT + i) * 1024, off2[i] + t * stp2[i], 0);
  };
  // scores of 16-key block kb of the staged tile for the lane's query: keys 16 kb + 4 c + e
  auto qk = [&](const int8_t* kbase, int kb, int64_t (&raw)[4]) {
    v4i acc[5];
#pragma unroll
    for (int u = 0; u < 5; ++u) acc[u] = v4i{0, 0, 0, 0};
    const int k = kb * 16 + kl;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const v4i a = *(const v4i*)(kbase + j * 64 * HD + k * HD + (((kk * 4 + c) ^ pre_swzk(k, HD)) * 16));
#pragma unroll
        for (int i = 0; i < 3; ++i) acc[i + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qb[i][kk], acc[i + j], 0, 0, 0);
      }
    // |acc| <= 64 KK 2^14 = 2^(20 + KK - 1): the pairs acc0 + 2^8 acc1 and acc2 + 2^8 acc3 are exact in int32
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int32_t lo = acc[0][e] + (acc[1][e] << 8), mid = acc[2][e] + (acc[3][e] << 8);
      raw[e] = (int64_t)lo + ((int64_t)mid << 16) + ((int64_t)acc[4][e] << 32);
    }
  };

  // ---- sweep 1: the lane's query maximum over its keys ----
  int64_t mx = kNeg;
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    if (t < ntile) issue1(t);
  for (int t = 0; t < ntile; ++t) {
    if (k_issuer && t + NS - 2 < ntile)
      ring_barrier<C::LPK * (NS - 2)>();
    else
      ring_barrier<0>();
    if (t + NS - 1 < ntile) issue1(t + NS - 1);
    const int8_t* kbase = (const int8_t*)smem + (t % NS) * C::STAGE;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      int64_t raw[4];
      qk(kbase, kb, raw);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (t * 64 + kb * 16 + 4 * c + e <= my_qpos) mx = imax(mx, raw[e]);
    }
  }
  mx = imax(mx, __shfl_xor(mx, 16, 64));
  mx = imax(mx, __shfl_xor(mx, 32, 64));
  ring_barrier<0>();                                 // every wave is done with the ring

  // ---- sweep 2: weights, den, p V ----
  // (fast: no query of the wave has a negative exponent shift and l2e < 2^31, so no visible key's zf or zf l2e
  // can wrap: weight_at_nn)
  const bool fast = tab2 != nullptr && __builtin_amdgcn_ballot_w64(shift < 0) == 0 && p.l2e >= 0 &&
                    p.l2e < (1LL << 31);
  const auto rtab = buf_rsrc(tab2 != nullptr ? (const void*)tab2 : (const void*)p.lut);   // (entry, next - entry)
  int64_t den = 0;
  v4i pacc[DB][5];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int u = 0; u < 5; ++u) pacc[d][u] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    if (t < ntile) issue2(t);
  // fast: zf = rshc(mx - raw, s) = (cz - raw) >> s with cz = mx + 2^(s - 1) (wrapping, as rshc's add), s clamped
  // to 62 as rshc clamps it; the weight's interpolation reads the (entry, next - entry) pair table in one load
  const int s62 = (int)imin(imax(shift, 0), 62);
  const int64_t cz = add_wrap(mx, s62 > 0 ? (1LL << (s62 - 1)) : 0);
  const int wmin_qpos = (int)-wave_max64(-(int64_t)my_qpos);      // the wave's smallest position
  auto tile2 = [&](int t, auto fast_t, auto full_t) {
    constexpr bool kFast = decltype(fast_t)::value, kFull = decltype(full_t)::value;   // kFull: every key visible
    const int8_t* kbase = (const int8_t*)smem + (t % NS) * C::STAGE;
    const int8_t* vbs = kbase + C::PB;
    int64_t raw[4][4];
    int32_t x[4][4];
    if constexpr (kFast) {
      // two halves of the tile: the first half's scores, table positions and table loads, then the second half's,
      // so the second half's MFMAs and integer work run while the first half's table rows are in flight; then the
      // next stage's request
      int idx[4][4], n[4][4], rr[4][4];
      v4i tv[4][4];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int kb = 2 * hf; kb < 2 * hf + 2; ++kb) qk(kbase, kb, raw[kb]);
#pragma unroll
      for (int kb = 2 * hf; kb < 2 * hf + 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint64_t zf = (uint64_t)((cz - raw[kb][e]) >> s62);
          zf = zf < (48ULL << kFZ) ? zf : (48ULL << kFZ);     // hidden keys (negative) clamp too: inside the table
          const uint64_t prod = (uint64_t)(uint32_t)zf * (uint64_t)(uint32_t)p.l2e + (1ULL << 27);
          // n = prod >> 54 and f = (prod >> 28) mod 2^26 from the product's two words
          const uint32_t ph = (uint32_t)(prod >> 32), pl = (uint32_t)prod;
          n[kb][e] = (int)(ph >> (28 + kFT2 - 32));
          const uint32_t f = __builtin_amdgcn_alignbit(ph, pl, 28) & ((1u << kFT2) - 1);
          idx[kb][e] = n[kb][e] < kZeroN ? (int)(f >> (kFT2 - kExp2Bits)) : 0;
          rr[kb][e] = (int)(f & ((1u << (kFT2 - kExp2Bits)) - 1));
        }
#pragma unroll
      for (int kb = 2 * hf; kb < 2 * hf + 2; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) tv[kb][e] = buf_load16(rtab, idx[kb][e] * 16);
      __builtin_amdgcn_sched_barrier(0);
      }
      if (t + NS - 1 < ntile) issue2(t + NS - 1);    // after the table loads: waiting for them leaves it in flight
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t av = (int64_t)(((uint64_t)(uint32_t)tv[kb][e][1] << 32) | (uint32_t)tv[kb][e][0]);
          const int64_t dv = (int64_t)(((uint64_t)(uint32_t)tv[kb][e][3] << 32) | (uint32_t)tv[kb][e][2]);
          const int64_t v = av + ((dv * rr[kb][e] + (1LL << (kFT2 - kExp2Bits - 1))) >> (kFT2 - kExp2Bits));
          // rshc(v, 38 + n) for 0 <= v < 2^61: ((v >> (s - 1)) + 1) >> 1 with s = min(38 + n, 62)
          const int sh2 = min(kExp2One - kFP + n[kb][e], 62) - 1;
          int32_t w = ((int32_t)(v >> sh2) + 1) >> 1;
          if (!kFull && t * 64 + kb * 16 + 4 * c + e > my_qpos) w = 0;
          x[kb][e] = w;
        }
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) qk(kbase, kb, raw[kb]);
      WeightAt wa[4][4];
      int64_t ta[4][4], tb[4][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) wa[kb][e] = weight_at(mx - raw[kb][e], shift, p.l2e);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ta[kb][e] = p.lut[wa[kb][e].idx];
          tb[kb][e] = p.lut[wa[kb][e].idx + 1];
        }
      if (t + NS - 1 < ntile) issue2(t + NS - 1);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          x[kb][e] = t * 64 + kb * 16 + 4 * c + e <= my_qpos ? (int32_t)weight_of(wa[kb][e], ta[kb][e], tb[kb][e]) : 0;
    }
    v4i pa[3] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
    int32_t dt = 0;                                   // the tile's weight sum: <= 64 2^22, exact in int32
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      // 0 <= x <= 2^22: signed base-256 limbs; limb_lo(x) as a byte is x & 255, the next digit is
      // (x + 128) >> 8 and the one after it (x + 128 + 2^15) >> 16 (nested floors), so limb i's byte is byte i of
      // x, x + 128 and x + 32896; four keys' bytes go into one word with two byte permutes and an or
      uint32_t v0[4], v1[4], v2[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dt += x[kb][e];
        v0[e] = (uint32_t)x[kb][e];
        v1[e] = v0[e] + 128u;
        v2[e] = v0[e] + 32896u;
      }
      pa[0][kb] = (int)gather_bytes<0>(v0);
      pa[1][kb] = (int)gather_bytes<1>(v1);
      pa[2][kb] = (int)gather_bytes<2>(v2);
    }
    den += dt;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const int row = d * 16 + kl;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const v4i b = *(const v4i*)(vbs + j * HD * 64 + row * 64 + ((c ^ pre_swzv(row)) * 16));
#pragma unroll
        for (int i = 0; i < 3; ++i) pacc[d][i + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa[i], b, pacc[d][i + j], 0, 0, 0);
      }
    }
  };
  auto sweep2 = [&](auto fast_t) {
    for (int t = 0; t < ntile; ++t) {
      if (t + NS - 2 < ntile)
        ring_barrier<C::LPT * (NS - 2)>();
      else
        ring_barrier<0>();
      if (t * 64 + 63 <= wmin_qpos)               // wave-uniform: every key of the tile is visible to every query
        tile2(t, fast_t, std::true_type{});
      else
        tile2(t, fast_t, std::false_type{});
    }
  };
  if (fast)
    sweep2(std::true_type{});
  else
    sweep2(std::false_type{});
  den += __shfl_xor(den, 16, 64);
  den += __shfl_xor(den, 32, 64);
  // outputs: lane holds queries 4 c + e of the wave, dims 16 d + kl
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int qw = 4 * c + e, r = q0 + 16 * w + qw;
    const int64_t dq = __shfl(den, qw, 64);
    if (r >= p.nq) continue;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      int64_t v = 0;
#pragma unroll
      for (int u = 0; u < 5; ++u) v += (int64_t)pacc[d][u][e] << (8 * u);
      p.num[z * p.snum_tile + (int64_t)r * p.snum_row + d * 16 + kl] = v;
    }
    if (kl == 0) p.den[z * p.sden_tile + r] = dq;
  }
}

// ---- KV store into the limb-plane cache (tri_paged.store, src/bitexact/vllm_plugin/tri_paged.py:311-335) ----
template <typename T>
__global__ __launch_bounds__(128) void kv_store_kernel(int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs,
                                                       const int64_t* slot, const T* k, int64_t skn, int64_t skh,
                                                       const T* v, int64_t svn, int64_t svh, int HD, int bs) {
  const int64_t n = blockIdx.x, h = blockIdx.y;
  const int64_t sl = slot[n];
  if (sl < 0) return;                                  // dummy / padded tokens carry slot -1
  int8_t* base = cache + (sl / bs) * sc_nb + h * sc_h + (sl % bs) * sc_bs;
  for (int d = threadIdx.x; d < HD; d += blockDim.x) {
    int32_t kr = (int32_t)k[n * skn + h * skh + d], vr = (int32_t)v[n * svn + h * svh + d];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int32_t k0 = limb_lo(kr), v0 = limb_lo(vr);
      base[i * HD + d] = (int8_t)k0;
      base[(3 + i) * HD + d] = (int8_t)v0;
      kr = (kr - k0) >> 8;
      vr = (vr - v0) >> 8;
    }
  }
}

}  // namespace bx

using namespace bx;

// ======================================== C ABI ========================================

static void allow_lds_attn(const void* k, size_t lds) {
  if (lds > 64 * 1024) hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

template <int QT, int HD, bool PAGED>
static int launch_attn(AttnArgs& p, int groups, hipStream_t st) {
  const int tiles = (p.nq + QT - 1) / QT;
  const size_t lds = sizeof(AttnSmem<QT, HD>);
  dim3 grid(groups * tiles, p.nsplit);
  if (lds > 64 * 1024) {
    hipFuncSetAttribute((const void*)attn_kernel<QT, HD, PAGED, 0>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipFuncSetAttribute((const void*)attn_kernel<QT, HD, PAGED, 1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  }
  if (p.nsplit > 1) {
    attn_kernel<QT, HD, PAGED, 0><<<grid, 256, lds, st>>>(p);
    if (int rc = check_launch("attn_kernel(max)")) return rc;
  }
  attn_kernel<QT, HD, PAGED, 1><<<grid, 256, lds, st>>>(p);
  return check_launch("attn_kernel");
}

constexpr int kDecRawKeys = 2048;               // single-launch score cache: 4 x 2048 x 8 B of LDS

template <int HD>
static int launch_dec(AttnArgs& p, int groups, int64_t max_keys, hipStream_t st) {
  const int tiles = (p.nq + 3) / 4;
  dim3 grid(groups * tiles, p.nsplit);
  const int64_t chunk = ((max_keys + p.nsplit - 1) / p.nsplit + 63) / 64 * 64;   // keys per split, at most
  if (p.nsplit > 1 && chunk <= 64 * kDecWaves && (int64_t)grid.x * grid.y <= kDecExchBlocks) {
    // BX_ATTN_EXCH_TICKS (tests): a shorter wait, down to 0, where blocks compute the maxima they have not seen
    const char* et = getenv("BX_ATTN_EXCH_TICKS");
    p.exch_ticks = et ? (uint64_t)strtoull(et, nullptr, 10) : kDecExchTicks;
    if (chunk <= 32 * kDecWaves) attn_dec_exch_kernel<HD, 2><<<grid, kDecWaves * 64, 0, st>>>(p);
    else attn_dec_exch_kernel<HD, 4><<<grid, kDecWaves * 64, 0, st>>>(p);
    return check_launch("attn_dec_exch_kernel");
  }
  if (p.nsplit > 1) {
    attn_dec_kernel<HD, 0, false><<<grid, kDecWaves * 64, 0, st>>>(p);
    if (int rc = check_launch("attn_dec_kernel(max)")) return rc;
    attn_dec_kernel<HD, 1, false><<<grid, kDecWaves * 64, 0, st>>>(p);
    return check_launch("attn_dec_kernel");
  }
  if (max_keys <= kDecRawKeys) {
    p.S = (int)((max_keys + 15) / 16 * 16);
    const size_t lds = (size_t)4 * p.S * 8 + ((size_t)p.S / p.bs + 2) * 4;   // scores + block-table entries
    hipFuncSetAttribute((const void*)attn_dec_raw_kernel<HD>, hipFuncAttributeMaxDynamicSharedMemorySize,
                        (int)(4 * kDecRawKeys * 8 + (kDecRawKeys + 2) * 4));
    attn_dec_raw_kernel<HD><<<grid, kDecWaves * 64, lds, st>>>(p, RopeArgs{}, AoArgs{});
    return check_launch("attn_dec_raw_kernel");
  }
  attn_dec_kernel<HD, 1, false><<<grid, kDecWaves * 64, 0, st>>>(p);
  return check_launch("attn_dec_kernel");
}

// split-KV workspace: mx [Gq] + num [Gq, HD] + den [Gq] + counters [tiles]; zero-filled = idle
static int64_t attn_ws_bytes(int64_t gq, int64_t tiles, int HD) { return gq * 8 * (2 + HD) + tiles * 4 + 256; }

static void bind_attn_ws(AttnArgs& p, void* ws, int64_t gq, int HD) {
  char* b = (char*)ws;
  p.mx_ws = (int64_t*)b;
  p.num_ws = (int64_t*)(b + gq * 8);
  p.den_ws = (int64_t*)(b + gq * 8 * (1 + HD));
  p.sem = (int32_t*)(b + gq * 8 * (2 + HD));
}

static int64_t dec_split_cap(int64_t T) { return std::max<int64_t>(1, std::min<int64_t>(kDecMaxSplit, kDecWsSplitBudget / std::max<int64_t>(T, 1))); }

extern "C" int64_t bx_attn_paged_workspace(int32_t R, int32_t HKV, int32_t M, int32_t HD) {
  const int64_t T = (int64_t)R * HKV * ((M + 3) / 4);                                  // query tiles
  return dec_ws_bytes(T, dec_split_cap(T), HD);
}

extern "C" int bx_exact_attn_paged(const int32_t* q, const int64_t* sh, const int64_t* qpos, int64_t sqpos_r,
                                   const int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs,
                                   const int32_t* bt, int64_t sbt, int32_t nblk, const int64_t* rmap, const int64_t* lut,
                                   int64_t l2e, int64_t* num, int64_t* den, int32_t R, int32_t HKV, int32_t M,
                                   int32_t HD, int32_t nsplit, void* ws, int64_t ws_bytes, bx_stream_t stream) {
  BX_REQUIRE(R >= 0 && HKV > 0 && M >= 1 && M <= 4, "need 1 <= M <= 4 queries per (row, KV head)");
  BX_REQUIRE(HD == 64 || HD == 128, "head_dim must be 64 or 128");
  BX_REQUIRE((int64_t)nblk * bs < 43690, "keys per row must stay below 43690");
  BX_REQUIRE(nsplit >= 1 && nsplit <= 64, "nsplit in [1, 64]");
  BX_REQUIRE(sc_bs >= 6 * HD && sc_nb % 16 == 0 && sc_h % 16 == 0 && sc_bs % 16 == 0 && ((uintptr_t)cache & 15) == 0,
             "cache rows must hold the 6 HD limb bytes, 16-byte aligned");
  BX_REQUIRE(q && sh && qpos && bt && rmap && lut && num && den, "null pointer");
  if (R == 0) return BX_OK;
  AttnArgs p = {};
  p.q = q; p.sq_tile = (int64_t)M * HD; p.sq_row = HD;
  p.sh = sh; p.sh_tile = M;
  p.qpos = qpos; p.qpos_tile = sqpos_r; p.qpos_row = 1; p.qpos_div = HKV; p.nq = M;
  p.cache = cache; p.sc_nb = sc_nb; p.sc_h = sc_h; p.sc_bs = sc_bs; p.bt = bt; p.sbt = sbt; p.rmap = rmap;
  p.bs = bs; p.hkv = HKV; p.nblk = nblk;
  p.lut = lut; p.l2e = l2e;
  p.num = num; p.den = den; p.snum_tile = (int64_t)M * HD; p.snum_row = HD; p.sden_tile = M;
  p.nsplit = nsplit;
  if (nsplit > 1) {
    const int64_t T = (int64_t)R * HKV * ((M + 3) / 4);
    const int64_t need = dec_ws_bytes(T, nsplit, HD);
    BX_REQUIRE(ws != nullptr && ws_bytes >= need, "workspace too small for %d splits (%lld < %lld)", nsplit,
               (long long)ws_bytes, (long long)need);
    BX_REQUIRE(((uintptr_t)ws & 7) == 0, "workspace must be 8-byte aligned");
    p.mx_ws = (int64_t*)ws;
  }
  const int64_t max_keys = (int64_t)nblk * bs;     // qpos < nblk bs: the block table's reach
  return HD == 64 ? launch_dec<64>(p, R * HKV, max_keys, (hipStream_t)stream)
                  : launch_dec<128>(p, R * HKV, max_keys, (hipStream_t)stream);
}

static int attn_rope_common(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos, const int64_t* cos,
                            const int64_t* sin, int32_t npos, int32_t H, int32_t FR, int32_t FT, int32_t FK, int32_t FV,
                            int32_t FZ, const int64_t* slot, int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs,
                            int32_t bs, const int32_t* bt, int64_t sbt, int32_t nblk, const int64_t* rmap,
                            const int64_t* lut, int64_t l2e, int64_t* num, int64_t* den, int32_t R, int32_t HKV,
                            int32_t HD, int32_t* err, const AoArgs* ao, hipStream_t st) {
  BX_REQUIRE(R >= 0 && HKV > 0 && H % HKV == 0 && H / HKV >= 1 && H / HKV <= 4, "need 1 <= H / HKV <= 4");
  BX_REQUIRE(HD == 64 || HD == 128, "head_dim must be 64 or 128");
  BX_REQUIRE(FK == kFK && FZ == kFZ, "the attention's fixed-point formats (FK, FZ) are compiled in");
  BX_REQUIRE((int64_t)nblk * bs <= kDecRawKeys, "the fused form takes at most %d keys per row", kDecRawKeys);
  BX_REQUIRE(ldy >= (int64_t)(H + 2 * HKV) * HD && npos > 0, "bad qkv rows or rope tables");
  BX_REQUIRE(sc_bs >= 6 * HD && sc_nb % 16 == 0 && sc_h % 16 == 0 && sc_bs % 16 == 0 && ((uintptr_t)cache & 15) == 0,
             "cache rows must hold the 6 HD limb bytes, 16-byte aligned");
  BX_REQUIRE(sc_h >= (int64_t)bs * sc_bs && sc_nb >= (int64_t)HKV * sc_h, "cache strides");
  BX_REQUIRE(y && pos && cos && sin && slot && bt && rmap && lut && err, "null pointer");
  BX_REQUIRE(ao != nullptr || (num && den), "null pointer");
  if (R == 0) return BX_OK;
  const int M = H / HKV;
  AttnArgs p = {};
  p.nq = M;
  p.cache = cache; p.sc_nb = sc_nb; p.sc_h = sc_h; p.sc_bs = sc_bs; p.bt = bt; p.sbt = sbt; p.rmap = rmap;
  p.bs = bs; p.hkv = HKV; p.nblk = nblk;
  p.lut = lut; p.l2e = l2e;
  p.num = num; p.den = den; p.snum_tile = (int64_t)M * HD; p.snum_row = HD; p.sden_tile = M;
  p.nsplit = 1;
  RopeArgs r = {y, ldy, pos, spos, 0, cos, sin, npos, R, 1, H, HKV, HD, FR, FT, FK, FV, FZ, nullptr, nullptr, nullptr,
                nullptr, err, cache, sc_nb, sc_h, sc_bs, slot, bs};
  const int64_t max_keys = (int64_t)nblk * bs;
  p.S = (int)((max_keys + 15) / 16 * 16);
  const size_t lds = (size_t)4 * p.S * 8 + ((size_t)p.S / p.bs + 2) * 4;   // scores + block-table entries
  const dim3 grid(R * HKV, 1);
  const int maxlds = (int)(4 * kDecRawKeys * 8 + (kDecRawKeys + 2) * 4);
#define BX_RAW_ROPE(HDV, AOV)                                                                                       \
  do {                                                                                                           \
    hipFuncSetAttribute((const void*)attn_dec_raw_kernel<HDV, true, AOV>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                        maxlds);                                                                                 \
    attn_dec_raw_kernel<HDV, true, AOV><<<grid, kDecWaves * 64, lds, st>>>(p, r, ao ? *ao : AoArgs{});              \
  } while (0)
  if (HD == 64 && ao) BX_RAW_ROPE(64, true);
  else if (HD == 64) BX_RAW_ROPE(64, false);
  else if (ao) BX_RAW_ROPE(128, true);
  else BX_RAW_ROPE(128, false);
#undef BX_RAW_ROPE
  return check_launch("attn_dec_raw_kernel(rope)");
}

extern "C" int bx_exact_attn_paged_rope(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos,
                                        const int64_t* cos, const int64_t* sin, int32_t npos, int32_t H, int32_t FR,
                                        int32_t FT, int32_t FK, int32_t FV, int32_t FZ, const int64_t* slot,
                                        int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs,
                                        const int32_t* bt, int64_t sbt, int32_t nblk, const int64_t* rmap,
                                        const int64_t* lut, int64_t l2e, int64_t* num, int64_t* den, int32_t R,
                                        int32_t HKV, int32_t HD, int32_t* err, bx_stream_t stream) {
  return attn_rope_common(y, ldy, pos, spos, cos, sin, npos, H, FR, FT, FK, FV, FZ, slot, cache, sc_nb, sc_h, sc_bs, bs,
                          bt, sbt, nblk, rmap, lut, l2e, num, den, R, HKV, HD, err, nullptr, (hipStream_t)stream);
}

extern "C" int64_t bx_attn_rope_out_workspace(int32_t R) {
  if (R <= 0) return 0;
  return (int64_t)R * 12 + 256;
}

extern "C" int64_t bx_attn_rope_out_scratch(int32_t R, int32_t H, int32_t HD) {
  if (R <= 0 || H <= 0 || HD <= 0) return 0;
  return (int64_t)R * H * HD * 8;
}

static int attn_rope_out(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos, const int64_t* cos,
                         const int64_t* sin, int32_t npos, int32_t H, int32_t FR, int32_t FT, int32_t FK, int32_t FV,
                         int32_t FZ, const int64_t* slot, int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs,
                         int32_t bs, const int32_t* bt, int64_t sbt, int32_t nblk, const int64_t* rmap,
                         const int64_t* lut, int64_t l2e, int32_t* q, int64_t ldq, int64_t* sh, int8_t* planes,
                         int32_t R, int32_t HKV, int32_t HD, int32_t* err, void* ws, int64_t ws_bytes, void* tmp,
                         int64_t tmp_bytes, hipStream_t stream) {
  BX_REQUIRE(q && sh && ldq >= (int64_t)H * HD, "null q / sh or ldq too small");
  BX_REQUIRE(ws && ws_bytes >= bx_attn_rope_out_workspace(R) && ((uintptr_t)ws & 7) == 0,
             "workspace too small (%lld < %lld)", (long long)ws_bytes, (long long)bx_attn_rope_out_workspace(R));
  BX_REQUIRE(tmp && tmp_bytes >= bx_attn_rope_out_scratch(R, H, HD) && ((uintptr_t)tmp & 7) == 0,
             "scratch too small (%lld < %lld)", (long long)tmp_bytes, (long long)bx_attn_rope_out_scratch(R, H, HD));
  BX_REQUIRE(FR - FV >= 0 && FR - FV <= 62, "FR - FV outside [0, 62]");
  AoArgs ao;
  ao.ws_p = (int64_t*)tmp;
  ao.ws_e = (int64_t*)ws;
  ao.cnt = (int32_t*)(ao.ws_e + R);
  ao.q = q; ao.ldq = ldq; ao.sh = sh; ao.FR = FR; ao.FV = FV;
  ao.planes = planes; ao.plane = (int64_t)R * H * HD;
  return attn_rope_common(y, ldy, pos, spos, cos, sin, npos, H, FR, FT, FK, FV, FZ, slot, cache, sc_nb, sc_h, sc_bs, bs,
                          bt, sbt, nblk, rmap, lut, l2e, nullptr, nullptr, R, HKV, HD, err, &ao, stream);
}

extern "C" int bx_exact_attn_paged_rope_out(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos,
                                            const int64_t* cos, const int64_t* sin, int32_t npos, int32_t H,
                                            int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ,
                                            const int64_t* slot, int8_t* cache, int64_t sc_nb, int64_t sc_h,
                                            int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt, int32_t nblk,
                                            const int64_t* rmap, const int64_t* lut, int64_t l2e, int32_t* q,
                                            int64_t ldq, int64_t* sh, int32_t R, int32_t HKV, int32_t HD, int32_t* err,
                                            void* ws, int64_t ws_bytes, void* tmp, int64_t tmp_bytes,
                                            bx_stream_t stream) {
  return attn_rope_out(y, ldy, pos, spos, cos, sin, npos, H, FR, FT, FK, FV, FZ, slot, cache, sc_nb, sc_h, sc_bs, bs, bt,
                       sbt, nblk, rmap, lut, l2e, q, ldq, sh, nullptr, R, HKV, HD, err, ws, ws_bytes, tmp, tmp_bytes,
                       (hipStream_t)stream);
}

extern "C" int bx_exact_attn_paged_rope_out_planes(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos,
                                                   const int64_t* cos, const int64_t* sin, int32_t npos, int32_t H,
                                                   int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ,
                                                   const int64_t* slot, int8_t* cache, int64_t sc_nb, int64_t sc_h,
                                                   int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt,
                                                   int32_t nblk, const int64_t* rmap, const int64_t* lut, int64_t l2e,
                                                   int32_t* q, int64_t ldq, int64_t* sh, int8_t* planes, int32_t R,
                                                   int32_t HKV, int32_t HD, int32_t* err, void* ws, int64_t ws_bytes,
                                                   void* tmp, int64_t tmp_bytes, bx_stream_t stream) {
  BX_REQUIRE(planes, "null planes");
  return attn_rope_out(y, ldy, pos, spos, cos, sin, npos, H, FR, FT, FK, FV, FZ, slot, cache, sc_nb, sc_h, sc_bs, bs, bt,
                       sbt, nblk, rmap, lut, l2e, q, ldq, sh, planes, R, HKV, HD, err, ws, ws_bytes, tmp, tmp_bytes,
                       (hipStream_t)stream);
}

extern "C" int bx_int8_attn_paged(const int64_t* q, const int64_t* qpos, int64_t sqpos_r, const int8_t* cache,
                                  int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt,
                                  int32_t nblk, const int32_t* ptab, int32_t ptab_len, int64_t* num, int64_t* den,
                                  int32_t R, int32_t HKV, int32_t M, int32_t HD, int32_t nsplit, void* ws,
                                  int64_t ws_bytes, bx_stream_t stream) {
  BX_REQUIRE(R >= 0 && HKV > 0 && M >= 1, "need M >= 1 queries per (row, KV head)");
  BX_REQUIRE(HD == 64 || HD == 128, "head_dim must be 64 or 128");
  BX_REQUIRE((int64_t)nblk * bs < 43690, "keys per row must stay below 43690");
  BX_REQUIRE(nsplit >= 1 && nsplit <= 64, "nsplit in [1, 64]");
  BX_REQUIRE(ptab_len >= (int32_t)(-kI8ZLo) + 1, "weight table needs 2^17 + 1 entries");
  BX_REQUIRE(sc_bs >= 6 * HD && sc_nb % 16 == 0 && sc_h % 16 == 0 && sc_bs % 16 == 0 && ((uintptr_t)cache & 15) == 0,
             "cache rows must hold the 6 HD limb bytes, 16-byte aligned");
  BX_REQUIRE(q && qpos && bt && ptab && num && den, "null pointer");
  if (R == 0) return BX_OK;
  AttnArgs p = {};
  p.q64 = q; p.sq_tile = (int64_t)M * HD; p.sq_row = HD;
  p.qpos = qpos; p.qpos_tile = sqpos_r; p.qpos_row = 1; p.qpos_div = HKV; p.nq = M;
  p.cache = cache; p.sc_nb = sc_nb; p.sc_h = sc_h; p.sc_bs = sc_bs; p.bt = bt; p.sbt = sbt; p.rmap = nullptr;
  p.bs = bs; p.hkv = HKV; p.nblk = nblk;
  // int8.segs.score_rule (src/bitexact/int8/segs.py:29-37): FQ = 14, FA = 12; head_dim 128 scales by 2^-1/2
  p.wrule = 1; p.ptab = ptab;
  p.zsh = 2 * 14 + 3 - 12 + (HD == 128 ? 24 : 0);
  p.zmul = HD == 128 ? 11863283 : 0;
  p.num = num; p.den = den; p.snum_tile = (int64_t)M * HD; p.snum_row = HD; p.sden_tile = M;
  p.nsplit = nsplit;
  if (nsplit > 1) {
    const int64_t T = (int64_t)R * HKV * ((M + 3) / 4);
    const int64_t need = dec_ws_bytes(T, nsplit, HD);
    BX_REQUIRE(ws != nullptr && ws_bytes >= need, "workspace too small for %d splits (%lld < %lld)", nsplit,
               (long long)ws_bytes, (long long)need);
    BX_REQUIRE(((uintptr_t)ws & 7) == 0, "workspace must be 8-byte aligned");
    p.mx_ws = (int64_t*)ws;
  }
  const int64_t max_keys = (int64_t)nblk * bs;     // qpos < nblk bs: the block table's reach
  return HD == 64 ? launch_dec<64>(p, R * HKV, max_keys, (hipStream_t)stream)
                  : launch_dec<128>(p, R * HKV, max_keys, (hipStream_t)stream);
}

// the limb-plane form's scratch: K and V planes, 3 Z Sp HD bytes each (Sp = S rounded up to 64 keys)
static int64_t pre2_planes(int64_t Z, int64_t S, int64_t HD) { return 2 * 3 * Z * ((S + 63) / 64 * 64) * HD; }
static int64_t pre2_scratch(int64_t Z, int64_t S, int64_t HD) { return pre2_planes(Z, S, HD) + (16LL << kExp2Bits); }

extern "C" int64_t bx_attn_prefill_scratch(int32_t Z, int32_t S, int32_t HD) {
  if (Z <= 0 || S <= 0 || (HD != 64 && HD != 128)) return 0;
  const int64_t b = pre2_scratch(Z, S, HD);
  return b < kBufRange - 16 ? b : 0;                 // larger: the register-staged form (no scratch)
}

extern "C" int bx_exact_attn_prefill(const int32_t* qg, int64_t sq_z, int64_t sq_row, const int64_t* shg,
                                     int64_t ssh_z, const int64_t* qpos, int64_t sqpos_z, int64_t sqpos_row,
                                     const int32_t* K, int64_t sk_z, int64_t sk_s, const int32_t* V, int64_t sv_z,
                                     int64_t sv_s, int32_t S, const int64_t* lut, int64_t l2e, int64_t* num,
                                     int64_t* den, int32_t Z, int32_t gT, int32_t HD, void* tmp, int64_t tmp_bytes,
                                     bx_stream_t stream) {
  BX_REQUIRE(Z >= 0 && gT >= 0 && S >= 0, "negative size");
  BX_REQUIRE(HD == 64 || HD == 128, "head_dim must be 64 or 128");
  BX_REQUIRE(S < 43690, "keys must stay below 43690");
  BX_REQUIRE(qg && shg && qpos && K && V && lut && num && den, "null pointer");
  BX_REQUIRE(ssh_z == gT, "shg must be [Z, gT, 1] contiguous");
  BX_REQUIRE(((uintptr_t)qg & 15) == 0 && ((uintptr_t)K & 15) == 0 && ((uintptr_t)V & 15) == 0 && sq_z % 4 == 0 &&
                 sq_row % 4 == 0 && sk_z % 4 == 0 && sk_s % 4 == 0 && sv_z % 4 == 0 && sv_s % 4 == 0,
             "qg, K, V: 16-byte aligned rows (base and strides multiples of 4 elements)");
  if (Z == 0 || gT == 0) return BX_OK;
  AttnArgs p = {};
  p.q = qg; p.sq_tile = sq_z; p.sq_row = sq_row;
  p.sh = shg; p.sh_tile = ssh_z;
  p.qpos = qpos; p.qpos_tile = sqpos_z; p.qpos_row = sqpos_row; p.qpos_div = 1; p.nq = gT;
  p.K = K; p.V = V; p.sk_z = sk_z; p.sk_s = sk_s; p.sv_z = sv_z; p.sv_s = sv_s; p.S = S;
  p.lut = lut; p.l2e = l2e;
  p.num = num; p.den = den; p.snum_tile = (int64_t)gT * HD; p.snum_row = HD; p.sden_tile = gT;
  p.nsplit = 1;
  // keys visible to a query never exceed the cache length S: qpos beyond S - 1 is the caller's contract
  hipStream_t st = (hipStream_t)stream;
  if (tmp != nullptr && S > 0) {
    const int64_t need = pre2_scratch(Z, S, HD);
    BX_REQUIRE(need < kBufRange - 16, "limb planes above 2 GiB: call without scratch");
    BX_REQUIRE(tmp_bytes >= need && ((uintptr_t)tmp & 15) == 0, "scratch too small (%lld < %lld) or not 16-byte aligned",
               (long long)tmp_bytes, (long long)need);
    const int Sp = (S + 63) / 64 * 64;
    int8_t* pl = (int8_t*)tmp;
    const int64_t units = (int64_t)Z * Sp * (HD / 16) + (int64_t)Z * (Sp / 4) * (HD / 4) + (1LL << kExp2Bits);
    int64_t* tab2 = (int64_t*)(pl + pre2_planes(Z, S, HD));
    pre_split_kernel<<<(int)std::min<int64_t>((units + 255) / 256, 8192), 256, 0, st>>>(
        p, pl, pl + (int64_t)Z * 3 * Sp * HD, tab2, Z, Sp, HD);
    if (int rc = check_launch("pre_split_kernel")) return rc;
    if (HD == 64) {
      allow_lds_attn((const void*)attn_pre2_kernel<64>, Pre2<64>::LDS);
      attn_pre2_kernel<64><<<Z * ((gT + 127) / 128), 512, Pre2<64>::LDS, st>>>(p, pl, Z, Sp, (const char*)tab2);
    } else {
      allow_lds_attn((const void*)attn_pre2_kernel<128>, Pre2<128>::LDS);
      attn_pre2_kernel<128><<<Z * ((gT + 63) / 64), 256, Pre2<128>::LDS, st>>>(p, pl, Z, Sp, (const char*)tab2);
    }
    return check_launch("attn_pre2_kernel");
  }
  const int tiles = (gT + 63) / 64;
  if (HD == 64) {
    allow_lds_attn((const void*)attn_pre_kernel<64>, sizeof(PreSmem<64>));
    attn_pre_kernel<64><<<Z * tiles, 256, sizeof(PreSmem<64>), st>>>(p);
  } else {
    allow_lds_attn((const void*)attn_pre_kernel<128>, sizeof(PreSmem<128>));
    attn_pre_kernel<128><<<Z * tiles, 256, sizeof(PreSmem<128>), st>>>(p);
  }
  return check_launch("attn_pre_kernel");
}

extern "C" int bx_kv_store(int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs, const int64_t* slot,
                           const void* k, int64_t skn, int64_t skh, const void* v, int64_t svn, int64_t svh,
                           int32_t elem_bytes, int32_t N, int32_t HKV, int32_t HD, bx_stream_t stream) {
  BX_REQUIRE(N >= 0 && HKV > 0 && HD > 0 && bs > 0, "bad sizes");
  BX_REQUIRE(elem_bytes == 4 || elem_bytes == 8, "k / v must be int32 or int64");
  BX_REQUIRE(sc_bs >= 6 * HD, "cache rows must hold the 6 HD limb bytes");
  if (N == 0) return BX_OK;
  BX_REQUIRE(cache && slot && k && v, "null pointer");
  dim3 grid(N, HKV);
  if (elem_bytes == 8)
    kv_store_kernel<int64_t><<<grid, 128, 0, (hipStream_t)stream>>>(cache, sc_nb, sc_h, sc_bs, slot, (const int64_t*)k,
                                                                   skn, skh, (const int64_t*)v, svn, svh, HD, bs);
  else
    kv_store_kernel<int32_t><<<grid, 128, 0, (hipStream_t)stream>>>(cache, sc_nb, sc_h, sc_bs, slot, (const int32_t*)k,
                                                                   skn, skh, (const int32_t*)v, svn, svh, HD, bs);
  return check_launch("kv_store_kernel");
}

BX_PHASE_DEFINE(attn)
