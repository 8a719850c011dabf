// Row-wise integer stages around the GEMMs and the attention, one block per row (1024 threads, 512 for the norm:
// a decode step has few rows, so each row spreads over a whole CU; softmax rows use 256; the SiLU stage of few rows
// goes over column chunks) with DPP wavefront int64 reductions: RMSNorm + per-row quantization (segs.norm_quant,
// optionally after the residual add or the
// embedding gather), SiLU gating + quantization (segs.silu_y + quant_silu), the masked softmax weights
// (segs.softmax), and the attention output rule (segs.attn_out = div_round + regroup + quant).
#include "bx_common.h"
#include "bx_introws.h"

#include <algorithm>

namespace bx {

BX_PHASE_TABLE


constexpr int kRowThreads = 1024;
constexpr int kRowU = 4;   // elements per thread whose loads are issued together

// ---- segs.norm_quant (src/bitexact/exact/segs.py:59-63) over ops.rms (src/bitexact/exact/ops.py:92-105) and
// ops.quant (src/bitexact/exact/ops.py:82-89), on the residual row the block first forms:
//   SRC_X    the row of x as it is;
//   SRC_ADD  x + y (segs.add_y, src/bitexact/exact/segs.py:40-41), written back to x;
//   SRC_EMB  emb[ids[row]] widened to int64 (the model's `emb[ids].long()`, exact/model.py:130), written to x.
// With gm null only the residual row is formed and bound-checked (the last layer's add). The row and P stay in LDS between the
// passes. ----
enum RowSrc { SRC_X = 0, SRC_ADD = 1, SRC_EMB = 2 };

struct NormArgs {
  int64_t* x;
  int64_t ldx;
  const int64_t* y;
  int64_t ldy;
  const int32_t* emb;
  const int64_t* ids;
  const int64_t* gm;
  const int64_t* ge;
  int32_t* q;
  int64_t ldq;
  int64_t* sh;
  int D, lg, FR, FN;
  int32_t* err;
  int8_t* planes;   // optional: q's signed int8 limb planes [3][M][D] (limb i of q[m][k] at i M D + m D + k)
  int64_t plane;    // M D
};

// One block of kNormThreads per row (a decode row of 2048 is 2 elements a thread, all loads in flight at once):
// the block reductions stay cheap (wave reductions in DPP, one LDS-only barrier each), and the gamma loads go out
// with the row's loads rather than after the reductions. 1024 threads measured +0.4 % on the engine step over 512
// (256: 17.2 vs 12.5 us per launch in an earlier form).
constexpr int kNormThreads = 1024, kNormU = 2;
template <int SRC>
__global__ __launch_bounds__(kNormThreads) void norm_quant_kernel(NormArgs p) {
  BX_PHASE(0, 0);
  constexpr int NT = kNormThreads, U = kNormU, NW = NT / 64;
  extern __shared__ __align__(16) char smem[];
  int64_t* Xs = (int64_t*)smem;
  int64_t* Ps = Xs + p.D;
  __shared__ int64_t sbuf[3][NW];
  const int D = p.D;
  int64_t* xr = p.x + (int64_t)blockIdx.x * p.ldx;
  const int32_t* er_row = nullptr;
  if (SRC == SRC_EMB) er_row = p.emb + p.ids[blockIdx.x] * (int64_t)D;
  const int64_t* yr = SRC == SRC_ADD ? p.y + (int64_t)blockIdx.x * p.ldy : nullptr;
  int64_t amax = 0;
  int64_t gmv0[U], gev0[U];   // the first group's gamma pairs, requested with the row
  // U elements per thread at a time, every load issued before the first store (the write-back to x could
  // alias later loads, which would otherwise wait for it one element at a time)
  for (int i0 = threadIdx.x; i0 < D; i0 += U * NT) {
    int64_t v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = min(i0 + k * NT, D - 1);
      if (SRC == SRC_EMB) v[k] = er_row[i];
      else if (SRC == SRC_ADD) v[k] = add_wrap(xr[i], yr[i]);
      else v[k] = xr[i];
    }
    if (i0 == (int)threadIdx.x && p.gm != nullptr) {
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int i = min(i0 + k * NT, D - 1);
        gmv0[k] = p.gm[i];
        gev0[k] = p.ge[i];
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = i0 + k * NT;
      if (i < D) {
        if (SRC != SRC_X) xr[i] = v[k];
        Xs[i] = v[k];
        amax = imax(amax, v[k] < 0 ? -v[k] : v[k]);
      }
    }
  }
  BX_PHASE(0, 1);
  amax = block_reduce64_dpp<true, NW>(amax, sbuf[0], 0);
  if (threadIdx.x == 0 && amax >= (1LL << 40)) p.err[0] = 1;
  if (p.gm == nullptr) return;
  const int64_t shx = imax(bitlen(imax(amax, 1)) - 25, -6);
  int64_t S = 0;
  for (int i = threadIdx.x; i < D; i += NT) {
    const int64_t xs = rshc(Xs[i], shx);
    S = add_wrap(S, mul_wrap(xs, xs));
  }
  S = block_reduce64_dpp<false, NW>(S, sbuf[1], 0);
  const int64_t T = add_wrap(S, rshc(kEps60 * (int64_t)D, 60 - 2 * (p.FR - shx)));
  const int64_t m = fdiv(62 + p.lg - bitlen(T), 2);
  const int64_t s = 2 * m - p.lg;
  const int64_t V = s >= 0 ? shl(T, s) : sar(T, -s);
  const int64_t r = isqrt64(V), er = shx - p.FR - m;
  const double rinv = 1.0 / (double)r;
  BX_PHASE(0, 2);
  int64_t emax = kNegBig;
  for (int i0 = threadIdx.x; i0 < D; i0 += U * NT) {
    int64_t gmv[U], gev[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = min(i0 + k * NT, D - 1);
      gmv[k] = i0 == (int)threadIdx.x ? gmv0[k] : p.gm[i];
      gev[k] = i0 == (int)threadIdx.x ? gev0[k] : p.ge[i];
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = i0 + k * NT;
      if (i < D) {
        const int64_t P = div_round64(mul_wrap(Xs[i], gmv[k]), gev[k] - p.FR - er + p.FN, r, rinv);
        Ps[i] = P;
        if (P != 0) emax = imax(emax, bitlen(P < 0 ? -P : P) - p.FN);
      }
    }
  }
  BX_PHASE(0, 3);
  emax = block_reduce64_dpp<true, NW>(emax, sbuf[2], kNegBig);
  const int64_t shr = imax(emax - kQB, kNegBig);
  for (int i = threadIdx.x; i < D; i += NT) {
    const int32_t qv = (int32_t)rshc(Ps[i], shr + p.FN);
    p.q[(int64_t)blockIdx.x * p.ldq + i] = qv;
    if (p.planes != nullptr) {   // the limb split of the exact GEMM's activation planes (split_q_kernel's)
      int8_t* dst = p.planes + (int64_t)blockIdx.x * D + i;
      int32_t r = qv;
#pragma unroll
      for (int l = 0; l < 3; ++l) {
        const int32_t lo = limb_lo(r);
        dst[l * p.plane] = (int8_t)lo;
        r = (r - lo) >> 8;
      }
    }
  }
  if (threadIdx.x == 0) p.sh[blockIdx.x] = shr;
  BX_PHASE(0, 4);
}

// ---- segs.silu_y + segs.quant_silu (src/bitexact/exact/segs.py:120-128) over ops.silu_mul
// (src/bitexact/exact/ops.py:119-130): per row of gu = [gate | up] at FR, P = silu(gate) up at 2 FR exactly,
// then the row quantization at eps = -2 FR. err[0] = 1 where silu_mul's ok is false (|g| > 2^32, or an element
// with bitlen(|s|) + bitlen(|u|) > 62). ----
__global__ __launch_bounds__(kRowThreads) void silu_quant_kernel(const int64_t* gu, int64_t ldgu, int ff, const int64_t* lut,
                                                         int FR, int32_t* q, int64_t ldq, int64_t* sh, int32_t* err) {
  extern __shared__ __align__(16) char smem[];
  int64_t* Ps = (int64_t*)smem;
  __shared__ int64_t sbuf[16];
  const int64_t* row = gu + (int64_t)blockIdx.x * ldgu;
  const int eps = -2 * FR;
  int64_t emax = kNegBig;
  int bad = 0;
  // kSiluU elements per thread at a time: their row loads, then their table loads, are issued together (one
  // element after another, each waited for its own two dependent loads)
  constexpr int kSiluU = 4;
  for (int i0 = threadIdx.x; i0 < ff; i0 += kSiluU * kRowThreads) {
  int64_t gv[kSiluU], uv[kSiluU], la[kSiluU], lb[kSiluU];
#pragma unroll
  for (int k = 0; k < kSiluU; ++k) {
    const int i = min(i0 + k * kRowThreads, ff - 1);
    gv[k] = row[i];
    uv[k] = row[ff + i];
  }
#pragma unroll
  for (int k = 0; k < kSiluU; ++k) {
    const int idx = silu_index(gv[k], FR);
    la[k] = lut[idx];
    lb[k] = lut[idx + 1];
  }
#pragma unroll
  for (int k = 0; k < kSiluU; ++k) {
    const int i = i0 + k * kRowThreads;
    if (i >= ff) continue;
    const int64_t P = silu_elem(gv[k], uv[k], la[k], lb[k], FR, bad);
    Ps[i] = P;
    if (P != 0) emax = imax(emax, bitlen(P < 0 ? (int64_t)(0 - (uint64_t)P) : P) + eps);
  }
  }
  if (bad) err[0] = 1;
  emax = block_max64(emax, sbuf);
  const int64_t shr = imax(emax - kQB, kNegBig);
  for (int i = threadIdx.x; i < ff; i += kRowThreads) q[(int64_t)blockIdx.x * ldq + i] = (int32_t)rshc(Ps[i], shr - eps);
  if (threadIdx.x == 0) sh[blockIdx.x] = shr;
}

// ---- intops.first_argmax (src/bitexact/intops.py:55-59): index of the first maximum of each int64 row. A lane
// keeps its first maximum (columns rise along its loop, only a strictly larger value replaces it); the block
// then takes the row maximum and the smallest index holding it. Integer max / min: no order dependence. ----
__global__ __launch_bounds__(1024) void first_argmax_kernel(const int64_t* v, int64_t ldv, int N, int64_t* out) {
  __shared__ int64_t smax[16], sidx[16];
  const int64_t* row = v + (int64_t)blockIdx.x * ldv;
  int64_t best = INT64_MIN, idx = N;
  constexpr int U = 8;                             // loads in flight per thread
  int i0 = threadIdx.x;
  for (; i0 + (U - 1) * 1024 < N; i0 += U * 1024) {
    int64_t x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = __builtin_nontemporal_load(row + i0 + u * 1024);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (x[u] > best || idx == N) { best = x[u]; idx = i0 + u * 1024; }
  }
  for (int i = i0; i < N; i += 1024) {
    const int64_t x = row[i];
    if (x > best || idx == N) { best = x; idx = i; }
  }
  int64_t m = best;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = imax(m, __shfl_xor(m, o, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) smax[wave] = m;
  __syncthreads();
  int64_t rm = smax[0];
  for (int w = 1; w < 16; ++w) rm = imax(rm, smax[w]);
  int64_t cand = (best == rm) ? idx : N;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cand = imin(cand, __shfl_xor(cand, o, 64));
  if (lane == 0) sidx[wave] = cand;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t r = sidx[0];
    for (int w = 1; w < 16; ++w) r = imin(r, sidx[w]);
    out[blockIdx.x] = r;
  }
}

// ---- segs.softmax (src/bitexact/exact/segs.py:102-105) over ops.softmax_w: key s visible iff s <= qpos ----
__global__ __launch_bounds__(256) void softmax_kernel(const int64_t* raw, int64_t ldr, const int64_t* qpos,
                                                      const int64_t* sh, int S, int kbits, const int64_t* lut,
                                                      int64_t l2e, int fp, int32_t* p, int64_t ldp, int64_t* den) {
  __shared__ int64_t sbuf[16];
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
__global__ __launch_bounds__(kRowThreads) void attn_out_kernel(const int64_t* num, int64_t sn_group, int64_t sn_query,
                                                       const int64_t* den, int64_t sd_group, int T, int HKV, int g,
                                                       int HD, int FR, int FV, int32_t* q, int64_t ldq, int64_t* sh) {
  extern __shared__ __align__(16) char smem[];
  int64_t* Os = (int64_t*)smem;
  __shared__ int64_t sbuf[16];
  const int o = blockIdx.x;
  const int W = HKV * g * HD;
  int64_t emax = kNegBig;
  for (int c = threadIdx.x; c < W; c += kRowThreads) {
    const int hh = c / HD, d = c % HD;
    const int64_t group = (int64_t)(o / T) * HKV + hh / g, query = (int64_t)(hh % g) * T + o % T;
    const int64_t dn = den[group * sd_group + query];   // >= 1 whenever the query sees a key (itself)
    const int64_t v = dn > 0 ? div_round64(num[group * sn_group + query * sn_query + d], FR - FV, dn, 1.0 / (double)dn) : 0;
    Os[c] = v;
    if (v != 0) emax = imax(emax, bitlen(v < 0 ? -v : v) - FR);
  }
  emax = block_max64(emax, sbuf);
  const int64_t shr = imax(emax - kQB, kNegBig);
  for (int c = threadIdx.x; c < W; c += kRowThreads) q[(int64_t)o * ldq + c] = (int32_t)rshc(Os[c], shr + FR);
  if (threadIdx.x == 0) sh[o] = shr;
}

// The same stage split over column chunks for few rows (one block per row would leave most CUs idle while each
// streams its 16 ff bytes of gate | up): grid (C, M), chunk index fastest, chunks of about 1024 columns.
constexpr int kSiluPartThreads = 256;
// Block (m, c) keeps its chunk's P in LDS, publishes the chunk's exponent maximum
// (as emax - kNegBig + 1; 0 = not yet published) and waits for the other chunks of its row for at most `ticks` of
// the 100 MHz real-time counter. A block that has not seen them all by then forms the row's maximum itself from
// gu (the same integers, slower), so the wait always ends. The row's last block to finish reading resets its
// slots and counter: the zero-filled workspace is left as it was found.
constexpr uint64_t kSiluTicks = 20000;   // 200 us
__global__ __launch_bounds__(kSiluPartThreads) void silu_fused_kernel(const int64_t* gu, int64_t ldgu, int ff,
                                                                      int chunk, const int64_t* lut, int FR,
                                                                      int64_t* slots, int32_t* cnt, uint64_t ticks,
                                                                      int32_t* q, int64_t ldq, int64_t* sh,
                                                                      int8_t* planes, int32_t* err) {
  extern __shared__ __align__(16) int64_t Ps[];   // [chunk]
  __shared__ int64_t sbuf[16];
  __shared__ int64_t s_row;
  const int m = blockIdx.y, c = blockIdx.x, C = gridDim.x;   // chunk index fastest: a row's chunks run together
  const int64_t* row = gu + (int64_t)m * ldgu;
  const int i_lo = c * chunk, i_hi = min(ff, i_lo + chunk);
  const int eps = -2 * (int)FR;
  int64_t emax = kNegBig;
  int bad = 0;
  constexpr int U = 4;
  for (int i0 = i_lo + threadIdx.x; i0 < i_hi; i0 += U * kSiluPartThreads) {
    int64_t gv[U], uv[U], la[U], lb[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = min(i0 + k * kSiluPartThreads, i_hi - 1);
      gv[k] = row[i];
      uv[k] = row[ff + i];
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int idx = silu_index(gv[k], FR);
      la[k] = lut[idx];
      lb[k] = lut[idx + 1];
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = i0 + k * kSiluPartThreads;
      if (i >= i_hi) continue;
      const int64_t v = silu_elem(gv[k], uv[k], la[k], lb[k], FR, bad);
      Ps[i - i_lo] = v;
      if (v != 0) emax = imax(emax, bitlen(v < 0 ? (int64_t)(0 - (uint64_t)v) : v) + eps);
    }
  }
  if (bad) err[0] = 1;
  emax = block_max64(emax, sbuf);
  if (threadIdx.x == 0) {
    s_row = emax;
    ws_store(&slots[(int64_t)m * C + c], emax - kNegBig + 1);
  }
  lds_sync();
  bool seen = true;
  if ((int)threadIdx.x < C && (int)threadIdx.x != c) {
    int64_t* a = &slots[(int64_t)m * C + threadIdx.x];
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    int64_t v = ws_load(a);
    while (v == 0 && __builtin_amdgcn_s_memrealtime() - t0 < ticks) {
      __builtin_amdgcn_s_sleep(1);
      v = ws_load(a);
    }
    seen = v != 0;
    if (seen) atomicMax((long long*)&s_row, (long long)(v - 1 + kNegBig));
  }
  const bool all = __syncthreads_and(seen);
  // Thread 0's own publish (an agent-scope store) is complete before its count (s_waitcnt), so no publish can
  // arrive after the row's last block has reset the slots. (An agent-scope release / acquire fence would write back
  // and invalidate the whole L2 on this chip; the waits on the coherent stores are all that is needed.)
  if (threadIdx.x == 0) __builtin_amdgcn_s_waitcnt(0);
  if (threadIdx.x == 0 && atomicAdd(&cnt[m], 1) == C - 1) {
    for (int j = 0; j < C; ++j) ws_store(&slots[(int64_t)m * C + j], 0);
    atomicExch(&cnt[m], 0);
  }
  int64_t rmax = s_row;
  if (!all) {   // the row's maximum from gu (blocks of the row that did not run alongside this one)
    int64_t e2 = kNegBig;
    int bad2 = 0;
    for (int i = threadIdx.x; i < ff; i += kSiluPartThreads) {
      const int64_t g = row[i];
      const int idx = silu_index(g, FR);
      const int64_t v = silu_elem(g, row[ff + i], lut[idx], lut[idx + 1], FR, bad2);
      if (v != 0) e2 = imax(e2, bitlen(v < 0 ? (int64_t)(0 - (uint64_t)v) : v) + eps);
    }
    rmax = block_max64(e2, sbuf);
  }
  const int64_t shr = imax(rmax - kQB, kNegBig);
  const int64_t plane = (int64_t)gridDim.y * ff;
  for (int i = i_lo + threadIdx.x; i < i_hi; i += kSiluPartThreads) {
    const int32_t qv = (int32_t)rshc(Ps[i - i_lo], shr - eps);
    q[(int64_t)m * ldq + i] = qv;
    if (planes != nullptr) {
      int32_t r = qv;
#pragma unroll
      for (int l = 0; l < 3; ++l) {
        const int32_t lo = limb_lo(r);
        planes[l * plane + (int64_t)m * ff + i] = (int8_t)lo;
        r = (r - lo) >> 8;
      }
    }
  }
  if (c == 0 && threadIdx.x == 0) sh[m] = shr;
}


// first_argmax split over column chunks for few rows (one block per row streams the whole row on one CU):
// argmax_part_kernel, grid (M, C), writes each chunk's (maximum, its first index) to scratch slots; argmax_fin_kernel
// takes, per row, the first chunk holding the row maximum (chunks in column order, so ties keep the smallest index).
constexpr int kArgThreads = 256;
__global__ __launch_bounds__(kArgThreads) void argmax_part_kernel(const int64_t* v, int64_t ldv, int N, int chunk,
                                                                  int64_t* slots) {
  __shared__ int64_t smax[kArgThreads / 64], sidx[kArgThreads / 64];
  const int m = blockIdx.x, c = blockIdx.y, C = gridDim.y;
  const int64_t* row = v + (int64_t)m * ldv;
  const int i_lo = c * chunk, i_hi = min(N, i_lo + chunk);
  int64_t best = INT64_MIN, idx = N;
  constexpr int U = 8;
  int i0 = i_lo + threadIdx.x;
  for (; i0 + (U - 1) * kArgThreads < i_hi; i0 += U * kArgThreads) {
    int64_t x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = __builtin_nontemporal_load(row + i0 + u * kArgThreads);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (x[u] > best || idx == N) { best = x[u]; idx = i0 + u * kArgThreads; }
  }
  for (int i = i0; i < i_hi; i += kArgThreads) {
    const int64_t x = row[i];
    if (x > best || idx == N) { best = x; idx = i; }
  }
  int64_t mx = best;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = imax(mx, __shfl_xor(mx, o, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) smax[wave] = mx;
  __syncthreads();
  int64_t rm = smax[0];
  for (int w = 1; w < kArgThreads / 64; ++w) rm = imax(rm, smax[w]);
  int64_t cand = (best == rm) ? idx : N;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cand = imin(cand, __shfl_xor(cand, o, 64));
  if (lane == 0) sidx[wave] = cand;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t ri = sidx[0];
    for (int w = 1; w < kArgThreads / 64; ++w) ri = imin(ri, sidx[w]);
    slots[((int64_t)m * C + c) * 2] = rm;
    slots[((int64_t)m * C + c) * 2 + 1] = ri;
  }
}

__global__ __launch_bounds__(64) void argmax_fin_kernel(const int64_t* slots, int M, int N, int C, int64_t* out) {
  const int m = blockIdx.x * 64 + threadIdx.x;
  if (m >= M) return;
  int64_t best = INT64_MIN, idx = N;
  for (int c = 0; c < C; ++c) {
    const int64_t sv = slots[((int64_t)m * C + c) * 2], si = slots[((int64_t)m * C + c) * 2 + 1];
    if (sv > best || idx == N) { best = sv; idx = si; }
  }
  out[m] = idx;
}

// A greedy decode step's next inputs, one thread per sequence: ids = the step's first-max tokens, pos + 1, and the
// cache slot of the new position through the block table (slot = bt[rmap, pos / bs] bs + pos % bs).
__global__ void decode_advance_kernel(const int64_t* next, int64_t* ids, int64_t* pos, int64_t* slot, const int32_t* bt,
                                      int64_t sbt, const int64_t* rmap, int bs, int N) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t p = pos[n] + 1;
  ids[n] = next[n];
  pos[n] = p;
  slot[n] = (int64_t)bt[rmap[n] * sbt + p / bs] * bs + p % bs;
}

}  // namespace bx

using namespace bx;

static void allow_lds_rows(const void* k, size_t lds) {
  if (lds > 64 * 1024) hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

static int launch_norm(NormArgs& p, int src, int32_t M, bx_stream_t stream) {
  int lg = 0;
  while ((1 << lg) < p.D) ++lg;
  BX_REQUIRE(p.D > 0 && (1 << lg) == p.D && lg <= 12, "row length a power of two <= 4096");
  BX_REQUIRE(M >= 0 && p.ldx >= p.D, "bad sizes");
  BX_REQUIRE(p.x && p.err, "null pointer");
  BX_REQUIRE(!p.gm || (p.ge && p.q && p.sh && p.ldq >= p.D), "gamma given without the quantized outputs");
  if (M == 0) return BX_OK;
  p.lg = lg;
  const size_t lds = (size_t)p.D * 16;
  const void* k = src == SRC_ADD ? (const void*)norm_quant_kernel<SRC_ADD>
                  : src == SRC_EMB ? (const void*)norm_quant_kernel<SRC_EMB> : (const void*)norm_quant_kernel<SRC_X>;
  allow_lds_rows(k, lds);
  hipStream_t st = (hipStream_t)stream;
  if (src == SRC_ADD) norm_quant_kernel<SRC_ADD><<<M, kNormThreads, lds, st>>>(p);
  else if (src == SRC_EMB) norm_quant_kernel<SRC_EMB><<<M, kNormThreads, lds, st>>>(p);
  else norm_quant_kernel<SRC_X><<<M, kNormThreads, lds, st>>>(p);
  return check_launch("norm_quant_kernel");
}

extern "C" int bx_rmsnorm_quant(const int64_t* x, int64_t ldx, const int64_t* gm, const int64_t* ge, int32_t* q,
                                int64_t ldq, int64_t* sh, int32_t M, int32_t D, int32_t FR, int32_t FN, int32_t* err,
                                bx_stream_t stream) {
  BX_REQUIRE(gm && ge && q && sh, "null pointer");
  NormArgs p = {const_cast<int64_t*>(x), ldx, nullptr, 0, nullptr, nullptr, gm, ge, q, ldq, sh, D, 0, FR, FN, err, nullptr, 0};
  return launch_norm(p, SRC_X, M, stream);
}

extern "C" int bx_add_rmsnorm_quant(int64_t* x, int64_t ldx, const int64_t* y, int64_t ldy, const int64_t* gm,
                                    const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh, int32_t M, int32_t D,
                                    int32_t FR, int32_t FN, int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(y && ldy >= D, "y: null or ldy too small");
  NormArgs p = {x, ldx, y, ldy, nullptr, nullptr, gm, ge, q, ldq, sh, D, 0, FR, FN, err, nullptr, 0};
  return launch_norm(p, SRC_ADD, M, stream);
}

extern "C" int bx_add_rmsnorm_quant_planes(int64_t* x, int64_t ldx, const int64_t* y, int64_t ldy, const int64_t* gm,
                                           const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh, int8_t* planes,
                                           int32_t M, int32_t D, int32_t FR, int32_t FN, int32_t* err,
                                           bx_stream_t stream) {
  BX_REQUIRE(!y || ldy >= D, "ldy too small");
  BX_REQUIRE(gm && ge && q && sh && planes, "null pointer");
  BX_REQUIRE(D % 16 == 0, "D %% 16 != 0 (the limb planes are the exact GEMM's K-major operand)");
  NormArgs p = {x, ldx, y, ldy, nullptr, nullptr, gm, ge, q, ldq, sh, D, 0, FR, FN, err, planes, (int64_t)M * D};
  return launch_norm(p, y ? SRC_ADD : SRC_X, M, stream);   // y null: the norm of x as it is (x not written)
}

extern "C" int bx_embed_rmsnorm_quant(const int32_t* emb, const int64_t* ids, int64_t* x, int64_t ldx,
                                      const int64_t* gm, const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh,
                                      int32_t M, int32_t D, int32_t FR, int32_t FN, int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(emb && ids, "null pointer");
  NormArgs p = {x, ldx, nullptr, 0, emb, ids, gm, ge, q, ldq, sh, D, 0, FR, FN, err, nullptr, 0};
  return launch_norm(p, SRC_EMB, M, stream);
}

extern "C" int bx_embed_rmsnorm_quant_planes(const int32_t* emb, const int64_t* ids, int64_t* x, int64_t ldx,
                                             const int64_t* gm, const int64_t* ge, int32_t* q, int64_t ldq,
                                             int64_t* sh, int8_t* planes, int32_t M, int32_t D, int32_t FR,
                                             int32_t FN, int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(emb && ids && gm && ge && q && sh && planes, "null pointer");
  BX_REQUIRE(D % 16 == 0, "D %% 16 != 0 (the limb planes are the exact GEMM's K-major operand)");
  NormArgs p = {x, ldx, nullptr, 0, emb, ids, gm, ge, q, ldq, sh, D, 0, FR, FN, err, planes, (int64_t)M * D};
  return launch_norm(p, SRC_EMB, M, stream);
}

extern "C" int bx_silu_quant(const int64_t* gu, int64_t ldgu, int32_t ff, const int64_t* lut, int32_t FR, int32_t* q,
                             int64_t ldq, int64_t* sh, int32_t M, int32_t* err, bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && ff > 0 && ldgu >= 2 * (int64_t)ff && ldq >= ff, "bad sizes");
  BX_REQUIRE(ff <= 16384, "ff > 16384 (row kept in LDS)");
  BX_REQUIRE(FR >= 0 && FR <= 24, "FR outside [0, 24]");
  BX_REQUIRE(gu && lut && q && sh && err, "null pointer");
  if (M == 0) return BX_OK;
  const size_t lds = (size_t)ff * 8;
  allow_lds_rows((const void*)silu_quant_kernel, lds);
  silu_quant_kernel<<<M, kRowThreads, lds, (hipStream_t)stream>>>(gu, ldgu, ff, lut, FR, q, ldq, sh, err);
  return check_launch("silu_quant_kernel");
}

// silu chunks: about 1024 elements each, at most 64 per row
static int silu_chunks(int ff) { return std::min(64, std::max(1, (ff + 1023) / 1024)); }

extern "C" int64_t bx_silu_quant_scratch(int32_t M, int32_t ff) {
  if (M <= 0 || ff <= 0) return 0;
  return (int64_t)M * silu_chunks(ff) * 8 + (int64_t)M * 4;
}

extern "C" int bx_silu_quant_ws(const int64_t* gu, int64_t ldgu, int32_t ff, const int64_t* lut, int32_t FR, int32_t* q,
                                int64_t ldq, int64_t* sh, int8_t* planes, int32_t M, int32_t* err, void* tmp,
                                int64_t tmp_bytes, bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && ff > 0 && ldgu >= 2 * (int64_t)ff && ldq >= ff, "bad sizes");
  BX_REQUIRE(FR >= 0 && FR <= 24, "FR outside [0, 24]");
  BX_REQUIRE(gu && lut && q && sh && err, "null pointer");
  if (M == 0) return BX_OK;
  BX_REQUIRE(tmp && tmp_bytes >= bx_silu_quant_scratch(M, ff) && ((uintptr_t)tmp & 7) == 0,
             "scratch too small (%lld < %lld)", (long long)tmp_bytes, (long long)bx_silu_quant_scratch(M, ff));
  BX_REQUIRE(!planes || ff % 16 == 0, "limb planes need ff %% 16 == 0");
  const int C = silu_chunks(ff), chunk = (ff + C - 1) / C;
  // dynamic LDS (the chunk's products) plus the kernel's static LDS must stay within the default 64 KiB
  BX_REQUIRE((int64_t)chunk * 8 <= 63 * 1024, "ff too large for the one-launch form");
  int64_t* slots = (int64_t*)tmp;
  int32_t* cnt = (int32_t*)(slots + (int64_t)M * C);
  // BX_SILU_TICKS (tests): a shorter wait, down to 0, where blocks form the row maximum they have not seen
  const char* et = getenv("BX_SILU_TICKS");
  const uint64_t ticks = et ? (uint64_t)strtoull(et, nullptr, 10) : kSiluTicks;
  silu_fused_kernel<<<dim3(C, M), kSiluPartThreads, (size_t)chunk * 8, (hipStream_t)stream>>>(
      gu, ldgu, ff, chunk, lut, FR, slots, cnt, ticks, q, ldq, sh, planes, err);
  return check_launch("silu_fused_kernel");
}

extern "C" int bx_first_argmax(const int64_t* v, int64_t ldv, int32_t M, int32_t N, int64_t* out, bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && N > 0 && ldv >= N, "bad sizes");
  BX_REQUIRE(v && out, "null pointer");
  if (M == 0) return BX_OK;
  first_argmax_kernel<<<M, 1024, 0, (hipStream_t)stream>>>(v, ldv, N, out);
  return check_launch("first_argmax_kernel");
}

static int argmax_chunks(int N) { return std::min(64, std::max(1, (N + 8191) / 8192)); }

extern "C" int64_t bx_first_argmax_scratch(int32_t M, int32_t N) {
  if (M <= 0 || N <= 0) return 0;
  return (int64_t)M * argmax_chunks(N) * 16;
}

extern "C" int bx_first_argmax_ws(const int64_t* v, int64_t ldv, int32_t M, int32_t N, int64_t* out, void* tmp,
                                  int64_t tmp_bytes, bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && N > 0 && ldv >= N, "bad sizes");
  BX_REQUIRE(v && out, "null pointer");
  if (M == 0) return BX_OK;
  BX_REQUIRE(tmp && tmp_bytes >= bx_first_argmax_scratch(M, N) && ((uintptr_t)tmp & 7) == 0,
             "scratch too small (%lld < %lld)", (long long)tmp_bytes, (long long)bx_first_argmax_scratch(M, N));
  const int C = argmax_chunks(N), chunk = (N + C - 1) / C;
  int64_t* slots = (int64_t*)tmp;
  argmax_part_kernel<<<dim3(M, C), kArgThreads, 0, (hipStream_t)stream>>>(v, ldv, N, chunk, slots);
  if (int rc = check_launch("argmax_part_kernel")) return rc;
  argmax_fin_kernel<<<(M + 63) / 64, 64, 0, (hipStream_t)stream>>>(slots, M, N, C, out);
  return check_launch("argmax_fin_kernel");
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
  attn_out_kernel<<<rows, kRowThreads, lds, (hipStream_t)stream>>>(num, sn_group, sn_query, den, sd_group, T, HKV, g, HD, FR,
                                                          FV, q, ldq, sh);
  return check_launch("attn_out_kernel");
}

BX_PHASE_DEFINE(rows)

extern "C" int bx_decode_advance(const int64_t* next, int64_t* ids, int64_t* pos, int64_t* slot, const int32_t* bt,
                                 int64_t sbt, int32_t nblk, const int64_t* rmap, int32_t bs, int32_t N,
                                 bx_stream_t stream) {
  BX_REQUIRE(N >= 0 && bs > 0 && nblk > 0 && sbt >= nblk, "bad sizes");
  if (N == 0) return BX_OK;
  BX_REQUIRE(next && ids && pos && slot && bt && rmap, "null pointer");
  decode_advance_kernel<<<(N + 255) / 256, 256, 0, (hipStream_t)stream>>>(next, ids, pos, slot, bt, sbt, rmap, bs, N);
  return check_launch("decode_advance_kernel");
}
