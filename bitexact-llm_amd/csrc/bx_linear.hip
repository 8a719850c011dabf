// Exact-mode limb GEMM and int8-mode GEMM for gfx950.
//
// Two kernel families share one epilogue:
//  * gemv_kernel (decode, <= 64 stacked activation rows). The limb rows of the activations (exact mode: limb i
//    of q[m] is row i*M+m, split from int32 q while staging; int8 mode: the caller's stacked rows) sit in LDS
//    for the block's K range. A block is CG column groups x KS k-slices of waves; every wave streams its 16
//    weight rows straight from HBM into MFMA B operands (unconditional 16-byte loads, U k-steps per group,
//    two groups in flight), one v_mfma_i32_16x16x64_i8 per (16-row block, weight plane). The first group is
//    requested before the activations are staged. The k-slices meet in LDS with ds_add (int32 sums are exact:
//    |sum| <= K 2^14 < 2^31), then the int32 limb products are joined in int64 (sum C_j[i M+m] 2^(8(i+j))).
//  * tile_kernel (prefill and the 128-row int8 case). An LDS ring (2 or 3 stages) is filled by asynchronous
//    global_load_lds_dwordx4 (1 KiB per wave instruction, XOR-swizzled 16-byte chunks so the MFMA operand
//    reads are bank-conflict free); 32x64 wave tiles of v_mfma_i32_32x32x32_i8 run the NA x NB limb products
//    into NA + NB - 1 int32 accumulators by limb weight i + j (|acc| <= 3 K 2^14 < 2^31 for K < 43690), joined
//    in int64 in registers. Exact mode reads int8 limb planes of q written by split_q_kernel.
//  * staged_kernel (int8 decode, <= 8 stacked rows): weight k-slices copied into LDS as contiguous 1 KiB pieces,
//    MFMA from LDS, no split-K. wide_kernel (exact decode, 65..96 limb rows) is described at its definition.
// The gemv and tile kernels split K over blocks when the tile grid is small: partials meet in an int64 workspace with atomics and
// the last block of a tile (device-scope counter) applies the epilogue and re-zeroes workspace and counter,
// so one launch does everything. Integer sums are exact in any order, so tiles, splits and schedules never
// change a bit.
#include "bx_common.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

namespace bx {

BX_PHASE_TABLE

enum Mode { RAW32 = 0, JOIN = 1, WMM_T = 2, EXACT = 3 };

struct LinArgs {
  const int32_t* q;      // exact: q int32 [M, ldq]
  int64_t ldq;
  const int8_t* a;       // int8 limb rows: stacked [rows_a, K] (gemv) or planes [NA][M][K] (tile)
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
  int32_t* sem;          // split-K counters, one per output tile
  int ks;                // K bytes per block (multiple of 64)
  int spw;               // gemv: k steps per wave
  int nla;               // gemv: stacked activation groups (exact 3, JOIN nl, RAW32 1); rows_a = nla M
  int tiles, parts_lg, mp;   // gemv: column tiles, log2 of the row parts per tile, output rows per part
  int xcd_remap;             // xtile: XCD-grouped tile order, row tiles per group (0: off; tile count a multiple of 8)
  int xt_pre;                // xtile: ring stages requested before the epilogue context is written (1..3)
};

// Residual column index. Valid ELL data is always in [0, K) with counts in [0, R]; a corrupt index or count
// (a damaged weight file) marks the output as untrustworthy: `corrupt` is raised (it sets flag[0] = 1 whenever
// the caller passed a flag, checked or not) and the entry reads column 0 instead of memory outside q.
__device__ __forceinline__ int kcol(const LinArgs& p, int32_t c, bool& corrupt) {
  const bool out = (uint32_t)c >= (uint32_t)p.K;
  corrupt |= out;
  return out ? 0 : c;
}

__device__ __forceinline__ int kcnt(const LinArgs& p, int32_t c, bool& corrupt) {
  const bool out = (uint32_t)c > (uint32_t)p.R;
  corrupt |= out;
  return out ? 0 : c;
}

// The kernels' flag write: numeric bound violations when `checked`, corrupt residual indices always.
__device__ __forceinline__ void write_flag(const LinArgs& p, bool bad, bool corrupt) {
  if (p.flag != nullptr && ((p.checked && bad) || corrupt)) p.flag[0] = 1;
}

// ---- epilogue shared by both kernels: one output element from its exact int64 dense value ----
template <int MODE>
__device__ __forceinline__ void finalize(const LinArgs& p, int m, int n, int64_t v, bool& bad, bool& corrupt) {
  const int64_t o = (int64_t)m * p.N + n;
  if (MODE == RAW32) {
    ((int32_t*)p.out)[o] = (int32_t)v;
  } else if (MODE == JOIN || MODE == WMM_T) {
    ((int64_t*)p.out)[o] = v;
  } else {
    // segs.lin_y (src/bitexact/exact/segs.py:25-32): B from the ELL residual, then wmm.epilogue.
    int64_t B = 0;
    if (p.R > 0) {
      const int c = kcnt(p, p.cnt[n], corrupt);
      const int32_t* qr = p.q + (int64_t)m * p.ldq;
      const int32_t* ec = p.ecol + (int64_t)n * p.R;
      const int64_t* ev = p.eval + (int64_t)n * p.R;
      for (int j = 0; j < c; ++j) B = add_wrap(B, mul_wrap((int64_t)qr[kcol(p, ec[j], corrupt)], ev[j]));
    }
    const int64_t dn = p.d[n];
    const int64_t pe = p.sh[m] + p.g[n] - dn + p.FR;
    bool b;
    ((int64_t*)p.out)[o] = exact_round_fast(v, B, dn, pe, b);
    bad |= b;
  }
}

// finalize<EXACT> with the row shift and the column's d, g and residual count already read (shm, dn, g, cnt_raw).
__device__ __forceinline__ void finalize_pre(const LinArgs& p, int m, int n, int64_t v, int64_t shm, int64_t dn,
                                             int64_t g, int32_t cnt_raw, bool& bad, bool& corrupt) {
  int64_t B = 0;
  if (p.R > 0) {
    const int c = kcnt(p, cnt_raw, corrupt);
    const int32_t* qr = p.q + (int64_t)m * p.ldq;
    const int32_t* ec = p.ecol + (int64_t)n * p.R;
    const int64_t* ev = p.eval + (int64_t)n * p.R;
    for (int j = 0; j < c; ++j) B = add_wrap(B, mul_wrap((int64_t)qr[kcol(p, ec[j], corrupt)], ev[j]));
  }
  bool b;
  ((int64_t*)p.out)[(int64_t)m * p.N + n] = exact_round_fast(v, B, dn, shm + g - dn + p.FR, b);
  bad |= b;
}

// Per-column epilogue context, loaded once per thread when a thread keeps one output column: d, g, and the
// first kRes residual entries of the column in registers (more entries, rare, are read from memory).
constexpr int kRes = 4;
struct ColCtx {
  int64_t d, gdr;        // d[n] and g[n] - d[n] + FR
  int cnt;
  bool corrupt;          // an index or count of the column's list is out of range
  int wmax;              // largest count over the wave's columns (wave-uniform loop bound)
  int32_t ec[kRes];
  int64_t ev[kRes];
  const int32_t* ecp;
  const int64_t* evp;
};

// The column's raw context, loaded with no value-dependent step (a kernel requests it before its main loop and
// forms the ColCtx after it, so the loads' latency hides behind the loop): the first min(kRes, R) list slots
// are read whatever the count, and col_ctx_from masks them.
struct ColPre {
  int64_t d, g;
  int32_t cnt;
  int32_t ec[kRes];
  int64_t ev[kRes];
};

__device__ __forceinline__ ColPre col_pre(const LinArgs& p, int n) {
  ColPre c;
  const int nn = min(n, p.N - 1);
  c.d = p.d[nn];
  c.g = p.g[nn];
  c.cnt = p.R > 0 ? p.cnt[nn] : 0;
#pragma unroll
  for (int j = 0; j < kRes; ++j) {
    const bool slot = j < p.R;   // uniform
    c.ec[j] = slot ? p.ecol[(int64_t)nn * p.R + j] : 0;
    c.ev[j] = slot ? p.eval[(int64_t)nn * p.R + j] : 0;
  }
  return c;
}

__device__ __forceinline__ ColCtx col_ctx_from(const LinArgs& p, int n, const ColPre& r) {
  ColCtx c;
  const int nn = min(n, p.N - 1);
  c.d = r.d;
  c.gdr = r.g - r.d + p.FR;
  c.corrupt = false;
  c.cnt = p.R > 0 ? kcnt(p, r.cnt, c.corrupt) : 0;   // entries stay inside the row's R slots
  c.wmax = (int)wave_max64(c.cnt);
  c.ecp = p.ecol + (int64_t)nn * p.R;
  c.evp = p.eval + (int64_t)nn * p.R;
#pragma unroll
  for (int j = 0; j < kRes; ++j) {
    const bool has = j < c.cnt;
    c.ec[j] = has ? kcol(p, r.ec[j], c.corrupt) : 0;
    c.ev[j] = has ? r.ev[j] : 0;
  }
  return c;
}

__device__ __forceinline__ ColCtx col_ctx(const LinArgs& p, int n) { return col_ctx_from(p, n, col_pre(p, n)); }

// The residuals of NR rows of the lane's column, gathered together: one wave-uniform branch per residual entry
// with NR independent loads under it, so a column costs about wmax load latencies instead of NR wmax (per-row
// calls put each row's loads behind its own branch). Integer sums wrap modulo 2^64, so the order of the terms
// does not matter.
template <int NR>
__device__ __forceinline__ void residual_rows(const LinArgs& p, const ColCtx& cc, const int (&mrow)[NR],
                                              int64_t (&B)[NR], bool& corrupt) {
#pragma unroll
  for (int e = 0; e < NR; ++e) B[e] = 0;
  if (cc.wmax <= 0) return;   // wave-uniform
#pragma unroll
  for (int j = 0; j < kRes; ++j) {
    if (j < cc.wmax) {        // wave-uniform; padded entries have ev = 0
      const int col = cc.ec[j];   // checked in col_ctx
      int32_t qv[NR];
#pragma unroll
      for (int e = 0; e < NR; ++e) qv[e] = p.q[(int64_t)mrow[e] * p.ldq + col];
#pragma unroll
      for (int e = 0; e < NR; ++e) B[e] = add_wrap(B[e], mul_wrap((int64_t)qv[e], cc.ev[j]));
    }
  }
  for (int j = kRes; j < cc.cnt; ++j) {
    const int col = kcol(p, cc.ecp[j], corrupt);
    const int64_t ev = cc.evp[j];
#pragma unroll
    for (int e = 0; e < NR; ++e) B[e] = add_wrap(B[e], mul_wrap((int64_t)p.q[(int64_t)mrow[e] * p.ldq + col], ev));
  }
}

__device__ __forceinline__ void finalize_col(const LinArgs& p, const ColCtx& cc, int m, int n, int64_t shm, int64_t v,
                                             int64_t B, bool& bad, bool& corrupt) {
  bool b;
  corrupt |= cc.corrupt;
  ((int64_t*)p.out)[(int64_t)m * p.N + n] = exact_round_fast(v, B, cc.d, shm + cc.gdr, b);
  bad |= b;
}

// Split-K handshake: after every thread has added its partials to the workspace, returns true in the last
// block of tile `tile` (all threads), which then owns the sums; that block also resets the tile counter.
// The workspace and the counters are only ever accessed with agent-scope read-modify-write atomics, which are
// performed at the device's coherence point, so no cache flush is needed (an agent-scope fence here would
// write back and invalidate the XCD's whole L2 in every block): each wave waits until its atomics are
// acknowledged (s_waitcnt) before the barrier, so every partial is in memory before the counter moves, and the
// last block reads the sums back with atomic exchanges.
__device__ __forceinline__ bool splitk_last(const LinArgs& p, int tile, int nsplit, int* s_last) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = atomicAdd(&p.sem[tile], 1) == nsplit - 1;
    if (last) atomicExch(&p.sem[tile], 0);
    *s_last = last;
  }
  __syncthreads();
  return *s_last;
}

__device__ __forceinline__ int64_t ws_take(const LinArgs& p, int m, int n) {
  return (int64_t)atomicExch((unsigned long long*)&p.ws[(int64_t)m * p.N + n], 0ull);
}

__device__ __forceinline__ void ws_add(const LinArgs& p, int m, int n, int64_t v) {
  atomicAdd((unsigned long long*)&p.ws[(int64_t)m * p.N + n], (unsigned long long)v);
}


// =====================================================================================================
// gemv kernel (decode)
// =====================================================================================================
// Activation staging, in two phases so that the activation loads are issued before the weight loads: vector
// memory operations complete in order, so activations requested after the weights could only be written to
// LDS once every weight had arrived. Chunk c of the block's slice is 4 int32 of q (exact: row c / nq, split
// into 3 limb rows while stored) or 16 int8 of a stacked row (JOIN / RAW32: local row c / nq, which is group
// i = row / Ml, output row m0 + row % Ml). Local row layout: group i at rows [i Ml, (i + 1) Ml), zero rows up
// to RA, zero columns past kend.
constexpr int kAB = 8;   // chunks per thread requested ahead of the weights


// floor(x / d) for 0 <= x < 2^21 from rcp ~ 1 / d (v_rcp_f32, relative error <= 2^-23): the quotient of
// x + 1/2 is at least 1 / (2 d) away from an integer and its float error is below (x + 1/2) 2^-22 / d.
__device__ __forceinline__ int qdiv(int x, float rcp) { return (int)(((float)x + 0.5f) * rcp); }

struct ASlice {
  int m0, Ml, k0, kend, nq, rows, total, LDA;
  float ml_rcp, nq_rcp;
};

template <int MODE>
__device__ __forceinline__ ASlice a_slice(const LinArgs& p, int m0, int Ml, int k0, int kend, int kpad, int LDA) {
  ASlice a;
  a.m0 = m0; a.Ml = Ml; a.k0 = k0; a.kend = kend; a.LDA = LDA;
  a.nq = (MODE == EXACT || MODE == WMM_T) ? kpad >> 2 : kpad >> 4;
  a.rows = (MODE == EXACT || MODE == WMM_T) ? Ml : p.nla * Ml;
  a.total = a.rows * a.nq;
  a.ml_rcp = __builtin_amdgcn_rcpf((float)Ml);
  a.nq_rcp = __builtin_amdgcn_rcpf((float)a.nq);
  return a;
}

// chunk (r, kq) of the slice: row r, 4-int32 (exact) or 16-byte column kq
// Chunks past the slice read the slice's first chunk (unconditional loads, no branches; a wave past the end
// issues one request per instruction).
// ares: buffer resource at the activations (exact: q, else the stacked rows); chunks past the slice are
// skipped loads.
template <int MODE>
__device__ __forceinline__ v4i a_load(const LinArgs& p, __amdgpu_buffer_rsrc_t ares, const ASlice& a, int r, int kq) {
  int off;
  if (MODE == EXACT || MODE == WMM_T) {
    off = ((a.m0 + r) * (int)p.ldq + min(a.k0 + kq * 4, p.K - 4)) * 4;
  } else {
    const int grp = qdiv(r, a.ml_rcp), grow = grp * p.M + a.m0 + (r - grp * a.Ml);
    off = grow * p.K + min(a.k0 + kq * 16, p.K - 16);
  }
  return buf_load16(ares, r < a.rows ? off : kBufSkip);
}

// Stores one chunk; chunks past the slice go to a 64-byte dummy slot of LDS (unconditional stores: a store
// under a branch lets the compiler sink its load into the branch, where it waits for every earlier load).
template <int MODE>
__device__ __forceinline__ void a_store(int8_t* As, int8_t* dummy, const ASlice& a, int r, int kq, v4i v) {
  const bool in = r < a.rows;
  if (MODE == EXACT || MODE == WMM_T) {
    uint32_t l0, l1, l2;
    split3(v, l0, l1, l2);
    const bool z = a.k0 + kq * 4 >= a.kend;
    int8_t* d = in ? As + r * a.LDA + kq * 4 : dummy;
    const int pl = in ? a.Ml * a.LDA : 16;
    *(uint32_t*)d = z ? 0u : l0;
    *(uint32_t*)(d + pl) = z ? 0u : l1;
    *(uint32_t*)(d + 2 * pl) = z ? 0u : l2;
  } else {
    *(v4i*)(in ? As + r * a.LDA + kq * 16 : dummy) = a.k0 + kq * 16 < a.kend ? v : v4i{0, 0, 0, 0};
  }
}

// Chunk walk of one thread: chunks tid, tid + NT, tid + 2 NT, ... as (row, column) pairs, stepped without
// divisions.
struct AWalk {
  int r, kq, dr, dq;
  __device__ __forceinline__ void init(const ASlice& a, int c, int NT) {   // c, NT < 2^21
    r = qdiv(c, a.nq_rcp);
    kq = c - r * a.nq;
    dr = qdiv(NT, a.nq_rcp);
    dq = NT - dr * a.nq;
  }
  __device__ __forceinline__ void step(const ASlice& a) {
    r += dr;
    kq += dq;
    if (kq >= a.nq) {
      kq -= a.nq;
      ++r;
    }
  }
};

// phase 1: the first kAB chunks of this thread. Batches wholly past the slice are not issued (a block-uniform
// branch: every vector memory instruction costs address-unit time, even one that reads nothing); these
// loads precede the weight loads, so skipping them does not change any wait on a weight.
template <int MODE, int NT>
__device__ __forceinline__ void a_issue(const LinArgs& p, __amdgpu_buffer_rsrc_t ares, const ASlice& a,
                                        v4i (&v)[kAB]) {
  AWalk w;
  w.init(a, threadIdx.x, NT);
#pragma unroll
  for (int i = 0; i < kAB; ++i) {
    if (i * NT < a.total) v[i] = a_load<MODE>(p, ares, a, w.r, w.kq);
    w.step(a);
  }
}

// phase 2: store them, load + store the rest (slices beyond kAB NT chunks), zero the padding rows
template <int RA, int MODE, int NT>
__device__ __forceinline__ void a_finish(const LinArgs& p, __amdgpu_buffer_rsrc_t ares, const ASlice& a,
                                         const v4i (&v)[kAB], int8_t* As, int8_t* dummy, int kpad) {
  const int tid = threadIdx.x;
  AWalk w;
  w.init(a, tid, NT);
#pragma unroll
  for (int i = 0; i < kAB; ++i) {
    if (i * NT < a.total) a_store<MODE>(As, dummy, a, w.r, w.kq, v[i]);
    w.step(a);
  }
  for (int b = kAB * NT; b < a.total; b += 4 * NT) {
    AWalk w2 = w;
    v4i x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a_load<MODE>(p, ares, a, w2.r, w2.kq);
      w2.step(a);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a_store<MODE>(As, dummy, a, w.r, w.kq, x[i]);
      w.step(a);
    }
  }
  const int used = (MODE == EXACT || MODE == WMM_T ? 3 : p.nla) * a.Ml, nc = kpad >> 4;
  for (int c = tid; c < (RA - used) * nc; c += NT) {
    const int r = used + c / nc, kc = c % nc;
    *(v4i*)(As + r * a.LDA + kc * 16) = v4i{0, 0, 0, 0};
  }
}

// Block barrier for LDS only: waits for this wave's LDS operations (lgkmcnt 0) but not for its outstanding
// global loads (vmcnt left at its maximum), unlike __syncthreads(), whose fence waits for every load.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
  asm volatile("s_barrier" ::: "memory");
}

// gemv block -> (column tile, row part). With several parts the parts of one column tile are consecutive
// blocks of one XCD (blocks are dispatched to the 8 XCDs round-robin), so the later parts' weight reads hit
// that XCD's L2 instead of HBM. Any mapping gives the same integers.
__device__ __forceinline__ void gemv_block(const LinArgs& p, int& tile, int& part) {
  const int L = blockIdx.x, lg = p.parts_lg;   // parts = 2^lg
  if (lg > 0 && (p.tiles & 7) == 0) {
    const int xcd = L & 7, slot = L >> 3;
    part = slot & ((1 << lg) - 1);
    tile = (slot >> lg) * 8 + xcd;
  } else {
    tile = L >> lg;
    part = L & ((1 << lg) - 1);
  }
}

template <int NB, int RB, int CG, int KS, int U, int MODE>
__global__ __launch_bounds__(64 * CG * KS) void gemv_kernel(LinArgs p) {
  constexpr int NT = 64 * CG * KS, RA = 16 * RB, BNC = 16 * CG;
  extern __shared__ __align__(16) char smem[];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = wave % CG, kslice = wave / CG;
  int tile, part;
  BX_PHASE(2, 0);
  gemv_block(p, tile, part);
  const int n0 = tile * BNC;
  const int m0 = part * p.mp, Ml = min(p.mp, p.M - m0);
  const int k0 = blockIdx.y * p.ks;
  const int kend = min(p.K, k0 + p.ks);
  const int nst = (kend - k0 + 63) >> 6;           // k steps of 64 in this block
  const int kpad = nst * 64;
  const int LDA = kpad + 16;
  int8_t* As = (int8_t*)smem;
  int32_t* Cs = (int32_t*)(smem + ((RA * LDA + 15) & ~15));   // [NB][RA][BNC]

  // this wave's weight row and k steps [s0, s1)
  const int kl = (lane >> 4) * 16;
  const __amdgpu_buffer_rsrc_t wres = buf_rsrc(p.w + (int64_t)n0 * p.ld_row);
  const int wrow = (min(n0 + cg * 16 + (lane & 15), p.N - 1) - n0) * (int)p.ld_row;
  const int s0 = kslice * p.spw, s1 = min(nst, s0 + p.spw);
  const int ngroups = s1 > s0 ? (s1 - s0 + U - 1) / U : 0;
  const int kmax = p.K - 16;
  // Steps past this wave's range are range-checked buffer loads that read nothing (the first group is issued
  // unconditionally so that the waits for the activation stores never include it).
  auto issue = [&](v4i(&b)[U][NB], int s) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int off = wrow + j * (int)p.ld_plane + min(k0 + (s + u) * 64 + kl, kmax);
        b[u][j] = buf_load16(wres, s + u < s1 ? off : kBufSkip);
      }
  };
  v4i acc[RB][NB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = v4i{0, 0, 0, 0};
  const int8_t* arow = As + (lane & 15) * LDA + kl;
  auto compute = [&](v4i(&b)[U][NB], int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s + u < s1) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const v4i av = *(const v4i*)(arow + r * 16 * LDA + (s + u) * 64);
#pragma unroll
          for (int j = 0; j < NB; ++j) acc[r][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[u][j], acc[r][j], 0, 0, 0);
        }
      }
    }
  };

  // activations first, then the weights (the first group, and the second when there is one); the activation
  // rows are written to LDS while the weights are in flight
  // exact: the epilogue context, requested before everything else and kept in LDS (threads < BNC: column d, g and
  // residual count; the next Ml threads, when the block has them: the row shifts)
  __shared__ int64_t s_cd[MODE == EXACT ? BNC : 1], s_cg[MODE == EXACT ? BNC : 1], s_csh[MODE == EXACT ? 64 : 1];
  __shared__ int32_t s_cc[MODE == EXACT ? BNC : 1];
  int64_t gx0 = 0, gx1 = 0;
  int32_t gcnt = 0;
  if constexpr (MODE == EXACT) {
    if (tid < BNC) {
      const int nn = min(n0 + tid, p.N - 1);
      gx0 = p.d[nn];
      gx1 = p.g[nn];
      gcnt = p.R > 0 ? p.cnt[nn] : 0;
    } else if (BNC + Ml <= NT && tid < BNC + Ml) {
      gx0 = p.sh[m0 + tid - BNC];
    }
  }
  const ASlice asl = a_slice<MODE>(p, m0, Ml, k0, kend, kpad, LDA);
  const __amdgpu_buffer_rsrc_t ares = buf_rsrc(MODE == EXACT || MODE == WMM_T ? (const void*)p.q : (const void*)p.a);
  v4i av[kAB];
  a_issue<MODE, NT>(p, ares, asl, av);
  v4i b0[U][NB], b1[U][NB];
  issue(b0, s0);
  // keep every weight request ahead of the first wait for an activation: the memory clobber orders the
  // loads, the register operands stop uses of the activation values (and their waits) from moving up
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < kAB; ++i) asm volatile("" : "+v"(av[i]));
  a_finish<RA, MODE, NT>(p, ares, asl, av, As, (int8_t*)(Cs + NB * RA * BNC), kpad);
  for (int i = tid; i < NB * RA * BNC; i += NT) Cs[i] = 0;
  if constexpr (MODE == EXACT) {
    if (tid < BNC) {
      s_cd[tid] = gx0;
      s_cg[tid] = gx1;
      s_cc[tid] = gcnt;
    } else if (BNC + Ml <= NT && tid < BNC + Ml) {
      s_csh[tid - BNC] = gx0;
    }
    if (BNC + Ml > NT)                                      // block-uniform: too few threads to hold them all
      for (int r = tid; r < Ml; r += NT) s_csh[r] = p.sh[m0 + r];
  }
  lds_barrier();
  BX_PHASE(2, 1);

  // later groups: one more in flight while a group is consumed (block-uniform conditions: no load is issued
  // that reads nothing)
  for (int gi = 0; gi < ngroups; gi += 2) {
    const int sa = s0 + gi * U, sb = sa + U;
    if (gi + 1 < ngroups) issue(b1, sb);
    compute(b0, sa);
    if (gi + 2 < ngroups) issue(b0, sb + U);
    if (gi + 1 < ngroups) compute(b1, sb);
  }

  BX_PHASE(2, 2);
  // ---- reduce the k-slices in LDS: Cs[j][row][col] += acc (row = stacked limb row, col in [0, BNC)) ----
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r * 16 + (lane >> 4) * 4 + e, col = cg * 16 + (lane & 15);
        if (KS == 1)
          Cs[(j * RA + row) * BNC + col] = acc[r][j][e];
        else
          atomicAdd(&Cs[(j * RA + row) * BNC + col], acc[r][j][e]);
      }
  __syncthreads();
  BX_PHASE(2, 3);

  bool bad = false, corrupt = false;
  const int nsplit = gridDim.y;
  for (int e = tid; e < Ml * BNC; e += NT) {
    const int m = e / BNC, c = e - m * BNC, n = n0 + c;
    if (n >= p.N) continue;
    int64_t v;
    if (MODE == RAW32) {
      v = Cs[m * BNC + c];
    } else if (MODE == JOIN) {
      v = 0;
      for (int i = 0; i < p.nl; ++i) v += (int64_t)Cs[(i * Ml + m) * BNC + c] << (8 * i);
    } else {
      v = 0;
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) v += (int64_t)Cs[(j * RA + i * Ml + m) * BNC + c] << (8 * (i + j));
    }
    if (nsplit > 1)
      ws_add(p, m0 + m, n, v);
    else if constexpr (MODE == EXACT)
      finalize_pre(p, m0 + m, n, v, s_csh[m], s_cd[c], s_cg[c], s_cc[c], bad, corrupt);
    else
      finalize<MODE>(p, m0 + m, n, v, bad, corrupt);
  }
  BX_PHASE(2, 4);
  if (nsplit > 1 && splitk_last(p, blockIdx.x, nsplit, &s_last)) {
    for (int e = tid; e < Ml * BNC; e += NT) {
      const int m = e / BNC, c = e - m * BNC, n = n0 + c;
      if (n >= p.N) continue;
      if constexpr (MODE == EXACT)
        finalize_pre(p, m0 + m, n, ws_take(p, m0 + m, n), s_csh[m], s_cd[c], s_cg[c], s_cc[c], bad, corrupt);
      else
        finalize<MODE>(p, m0 + m, n, ws_take(p, m0 + m, n), bad, corrupt);
    }
  }
  if (MODE == EXACT) write_flag(p, bad, corrupt);
  BX_PHASE(2, 5);
}

// =====================================================================================================
// split q into int8 limb planes (tile-kernel input): planes [3][M][K]
// =====================================================================================================
__global__ __launch_bounds__(256) void split_q_kernel(const int32_t* q, int64_t ldq, int M, int K, int8_t* planes) {
  const int nk = K >> 4;
  const int64_t total = (int64_t)M * nk, plane = (int64_t)M * K;
  for (int64_t c = blockIdx.x * 256LL + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int m = (int)(c / nk), k = (int)(c - (int64_t)m * nk) * 16;
    const int32_t* src = q + (int64_t)m * ldq + k;
    v4i o0, o1, o2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t l0, l1, l2;
      split3(*(const v4i*)(src + 4 * i), l0, l1, l2);
      o0[i] = (int32_t)l0;
      o1[i] = (int32_t)l1;
      o2[i] = (int32_t)l2;
    }
    int8_t* dst = planes + (int64_t)m * K + k;
    *(v4i*)dst = o0;
    *(v4i*)(dst + plane) = o1;
    *(v4i*)(dst + 2 * plane) = o2;
  }
}

// =====================================================================================================
// tile kernel (prefill): WM x WN waves, wave tile (32 TM) x (32 TN), BK = 64, S-stage async LDS ring,
// grid (N / BN, M / BM, splits)
// =====================================================================================================
// 16-byte chunk swizzle of a BK-byte LDS row (CH = BK / 16 chunks): rows that share LDS banks get different
// chunk slots, so the 16 lanes of each MFMA operand read phase hit 16 distinct bank groups.
template <int BK>
__device__ __forceinline__ int swz(int row) {
  return BK == 128 ? row & 7 : BK == 64 ? (row >> 2) & 3 : (row >> 3) & 1;
}

__device__ __forceinline__ void async16(const void* g, void* lds_base) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)g,
                                   (void __attribute__((address_space(3)))*)lds_base, 16, 0, 0);
}

// ---- epilogue of the tile kernels, straight from the accumulators: lane (l % 32) owns column (wn TN + t) 32 +
// l % 32 of each 32-column block t, so the column contexts (d, g, residual list) stay in registers; the row
// exponents are read from LDS. Stores of 32 lanes cover 256 contiguous bytes of a row. With K split over blocks
// (gridDim.z > 1) the partials go to the workspace and the last block of the tile applies the epilogue. ----
template <int NS, int MODE, int WM, int WN, int TM, int TN>
__device__ __forceinline__ void tile_epilogue(const LinArgs& p, v16i (&acc)[NS][TM][TN], int m0, int n0, int wm,
                                              int wn) {
  constexpr int NW = WM * WN, BM = 32 * TM * WM;
  const int tid = threadIdx.x, lane = tid & 63;
  __shared__ int s_last;
  __shared__ int64_t s_sh[MODE == EXACT ? BM : 1];
  if (MODE == EXACT)
    for (int r = tid; r < BM; r += NW * 64) s_sh[r] = p.sh[min(m0 + r, p.M - 1)];
  __syncthreads();
  bool bad = false, corrupt = false;
  const int nsplit = gridDim.z;
  ColCtx cc[TN];
  if (MODE == EXACT)
#pragma unroll
    for (int t = 0; t < TN; ++t) cc[t] = col_ctx(p, n0 + (wn * TN + t) * 32 + (lane & 31));
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int n = n0 + (wn * TN + t) * 32 + (lane & 31);
#pragma unroll
      for (int e0 = 0; e0 < 16; e0 += 8) {   // 8 rows at a time: 16 would spill registers
        int64_t B[8];
        if (MODE == EXACT && nsplit == 1) {
          int mrow[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int e = e0 + u;
            mrow[u] = min(m0 + (wm * TM + a) * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3), p.M - 1);
          }
          residual_rows<8>(p, cc[t], mrow, B, corrupt);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
        const int e = e0 + u;
        const int r = (wm * TM + a) * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3), m = m0 + r;
        int64_t v = 0;
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) v += (int64_t)acc[s2][a][t][e] << (8 * s2);
        if (m < p.M && n < p.N) {
          if (nsplit > 1)
            ws_add(p, m, n, v);
          else if (MODE == EXACT)
            finalize_col(p, cc[t], m, n, s_sh[r], v, B[u], bad, corrupt);
          else
            finalize<MODE>(p, m, n, v, bad, corrupt);
        }
        }
      }
    }
  if (nsplit > 1 && splitk_last(p, blockIdx.y * gridDim.x + blockIdx.x, nsplit, &s_last)) {
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int n = n0 + (wn * TN + t) * 32 + (lane & 31);
#pragma unroll
        for (int e0 = 0; e0 < 16; e0 += 8) {
          int64_t v[8], B[8];
          int mrow[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int e = e0 + u, m = m0 + (wm * TM + a) * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
            mrow[u] = min(m, p.M - 1);
            v[u] = (m < p.M && n < p.N) ? ws_take(p, m, n) : 0;
          }
          if (MODE == EXACT) residual_rows<8>(p, cc[t], mrow, B, corrupt);
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int e = e0 + u, r = (wm * TM + a) * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3), m = m0 + r;
            if (m < p.M && n < p.N) {
              if (MODE == EXACT)
                finalize_col(p, cc[t], m, n, s_sh[r], v[u], B[u], bad, corrupt);
              else
                finalize<MODE>(p, m, n, v[u], bad, corrupt);
            }
          }
        }
      }
  }
  if (MODE == EXACT) write_flag(p, bad, corrupt);
}

template <int NA, int NB, int MODE, int WM, int WN, int TM, int TN, int BK, int S>
__global__ __launch_bounds__(WM * WN * 64) void tile_kernel(LinArgs p) {
  static_assert(BK == 32 || BK == 64 || BK == 128, "k tile");
  constexpr int NW = WM * WN;
  constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
  constexpr int NS = NA + NB - 1;
  constexpr int CH = BK / 16, RPI = 1024 / BK;                 // chunks per row, rows per 1 KiB instruction
  constexpr int SA = NA * BM * BK, STAGE = SA + NB * BN * BK;
  constexpr int LA = NA * BM / RPI, LT = LA + NB * BN / RPI;   // 1 KiB load instructions per stage
  constexpr int LWL = LT / NW, LWX = LT % NW;                 // per wave: LWL + 1 for the first LWX waves
  static_assert((LWL + (LWX > 0)) * (S - 2) < 64, "vmcnt range");
  extern __shared__ __align__(16) char smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int kt0 = blockIdx.z * (p.ks / BK);
  const int nk = min((p.K + BK - 1) / BK, kt0 + p.ks / BK) - kt0;
  const int ktail = p.K / BK;                 // first k tile that reaches past K (only when K % BK != 0)

  // Each 1 KiB load instruction covers RPI rows x BK bytes: lane L -> row L / CH of the group, LDS slot L % CH,
  // global chunk (L % CH) ^ swz(row); swz only sees row bits that are the same for every instruction, so the
  // lane's chunk is fixed. Rows past M / N are clamped (discarded in the epilogue); k chunks past K are clamped
  // and zeroed in the A operand so they contribute nothing. Addresses are recomputed per issue (few VALU ops)
  // rather than held in registers next to the accumulators.
  const int lrow = lane / CH;
  const int lch = ((lane % CH) ^ swz<BK>(lrow)) << 4;
  const int64_t aplane = (int64_t)p.M * p.K;
  const bool xwave = wave < LWX;
  const int inst0 = xwave ? wave * (LWL + 1) : LWX * (LWL + 1) + (wave - LWX) * LWL;
  auto issue = [&](int kt, int stage) {
    char* sbase = smem + stage * STAGE + inst0 * 1024;
    const int kk = min(kt * BK + lch, p.K - 16);
#pragma unroll
    for (int i = 0; i < LWL + (LWX > 0); ++i) {
      if (i == LWL && !xwave) break;
      const int inst = inst0 + i;
      const int8_t* src;
      if (inst < LA) {
        const int pl = inst / (BM / RPI), row = (inst % (BM / RPI)) * RPI + lrow;
        src = p.a + pl * aplane + (int64_t)min(m0 + row, p.M - 1) * p.K + kk;
      } else {
        const int ib = inst - LA, pl = ib / (BN / RPI), row = (ib % (BN / RPI)) * RPI + lrow;
        src = p.w + pl * p.ld_plane + (int64_t)min(n0 + row, p.N - 1) * p.ld_row + kk;
      }
      async16(src, sbase + i * 1024);
    }
  };

  v16i acc[NS][TM][TN];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[s][a][t][e] = 0;

#pragma unroll
  for (int t = 0; t < S - 1; ++t)
    if (t < nk) issue(kt0 + t, t);

  for (int it = 0; it < nk; ++it) {
    if (it + S - 2 >= nk) {
      ring_barrier<0>();
    } else if constexpr (LWX == 0) {
      ring_barrier<LWL * (S - 2)>();
    } else {
      if (xwave)
        ring_barrier<(LWL + 1) * (S - 2)>();
      else
        ring_barrier<LWL * (S - 2)>();
    }
    if (it + S - 1 < nk) issue(kt0 + it + S - 1, (it + S - 1) % S);
    const char* base = smem + (it % S) * STAGE;
    const int kt = kt0 + it;
#pragma unroll
    for (int h = 0; h < BK / 32; ++h) {
      const int c = 2 * h + (lane >> 5);
      const bool kok = kt < ktail || kt * BK + c * 16 < p.K;
      v4i av[NA][TM], bv[NB][TN];
#pragma unroll
      for (int i = 0; i < NA; ++i)
#pragma unroll
        for (int a = 0; a < TM; ++a) {
          const int arow = (wm * TM + a) * 32 + (lane & 31);
          av[i][a] = *(const v4i*)(base + i * BM * BK + arow * BK + ((c ^ swz<BK>(arow)) << 4));
          if (!kok) av[i][a] = v4i{0, 0, 0, 0};
        }
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const int brow = (wn * TN + t) * 32 + (lane & 31);
          bv[j][t] = *(const v4i*)(base + SA + j * BN * BK + brow * BK + ((c ^ swz<BK>(brow)) << 4));
        }
#pragma unroll
      for (int i = 0; i < NA; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int t = 0; t < TN; ++t)
              acc[i + j][a][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i][a], bv[j][t], acc[i + j][a][t], 0, 0, 0);
    }
  }

  tile_epilogue<NS, MODE, WM, WN, TM, TN>(p, acc, m0, n0, wm, wn);
}

// =====================================================================================================
// xtile kernel: the exact prefill GEMM (3 x 3 limb planes, K % 64 == 0) on 128 x 128 block tiles, software
// pipelined.
//  * Main loop: 8 waves (4 x 2) of 32 x 64 wave tiles, five int32 accumulator sets by limb weight i + j. The
//    3-stage LDS ring (64-deep k tiles, 48 KiB each) is filled by buffer_load_dwordx4 ... lds (the k advance is
//    the scalar offset, so a lane keeps one 32-bit offset per load instruction) with the tile kernel's XOR
//    swizzle. A wave works in half-steps of 32 k: while the 18 MFMAs of one half-step run, the 9 LDS operand
//    reads of the next are in flight (two operand sets in registers). The ring barrier sits between the two
//    half-steps of a k tile; the stage it frees is refilled 3 k tiles ahead.
//  * Epilogue context in LDS: before the loop, the block's row exponents, each column's d and g - d + FR, and a
//    compact list of the columns' residual entries (k, v; at most kXtEmax per block) are staged in LDS. When the
//    ring stops refilling (3 k tiles before the end), the freed stage receives, by LDS DMA gathers, q[m][k] of
//    every listed entry for the block's 128 rows, so the epilogue's residual terms are LDS reads instead of
//    dependent global round trips. Blocks with more entries read the residual from global memory.
// =====================================================================================================
constexpr int kXtBM = 128, kXtBN = 128, kXtBK = 64, kXtS = 3, kXtEmax = 96;
constexpr int kXtStage = 6 * kXtBM * kXtBK;                               // 48 KiB
constexpr int kXtCtx = 3 * kXtBM * 8 + kXtEmax * 12 + 132 * 4 + 32;       // epilogue context after the ring
constexpr size_t kXtLds = (size_t)kXtS * kXtStage + kXtCtx;

template <int TM, int TN>
struct XtOps {
  v4i a[3][TM], b[3][TN];
};


__device__ __forceinline__ void buf_lds4(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff, 0, 0, 0);
}

// WM x WN waves of (32 TM) x (32 TN) wave tiles; launched as 4 x 2 waves of 32 x 64 (2 waves per SIMD: the five
// accumulator sets take 160 registers). 2 x 2 waves of 64 x 64 at one wave per SIMD would halve the operand reads
// per MFMA, but the compiler then moves the 320 accumulators between AGPRs and VGPRs inside the loop.
template <int MODE, int WM, int WN, int TM, int TN>
__global__ __launch_bounds__(WM * WN * 64) void xtile_kernel(LinArgs p) {
  BX_PHASE(0, 0);
  constexpr int NW = WM * WN, BM = kXtBM, BN = kXtBN, BK = kXtBK, S = kXtS, STAGE = kXtStage;
  static_assert(32 * WM * TM == BM && 32 * WN * TN == BN, "wave layout");
  constexpr int SA = 3 * BM * BK, LPW = 48 / NW;            // 1 KiB load instructions per wave per stage
  constexpr bool EX = MODE == EXACT;
  extern __shared__ __align__(16) char smem[];
  int64_t* s_sh = (int64_t*)(smem + S * STAGE);             // [BM] row exponents
  int64_t* s_d = s_sh + BM;                                 // [BN] d
  int64_t* s_gdr = s_d + BN;                                // [BN] g - d + FR
  int64_t* s_ev = s_gdr + BN;                               // [kXtEmax] residual values of the compact list
  int32_t* s_ek = (int32_t*)(s_ev + kXtEmax);               // [kXtEmax] residual columns (k) of the list
  int32_t* s_cs = s_ek + kXtEmax;                           // [BN + 1] list start of each column
  int64_t* s_mm = (int64_t*)(s_cs + 132);                   // [4] min / max of the row exponents, per half

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar) from here on
  const int wm = wave % WM, wn = wave / WM;
  // XCD-aware tile order: blocks are dispatched round-robin over the 8 XCDs (block b on XCD b % 8); the tiles an
  // XCD runs together form 4-row x 8-column patches, so they share A and B rows in that XCD's L2
  int tx = blockIdx.x, ty = blockIdx.y;
  if (p.xcd_remap) {
    const int T = gridDim.x * gridDim.y, b = blockIdx.y * gridDim.x + blockIdx.x;
    const int v = (b & 7) * (T >> 3) + (b >> 3);
    const int R = p.xcd_remap;
    const int grp = v / (R * gridDim.x), in = v - grp * R * gridDim.x;
    ty = grp * R + in % R;
    tx = in / R;
  }
  const int m0 = ty * BM, n0 = tx * BN;
  const int nk = p.K / BK;                                  // K % 64 == 0 and no K split (planner)

  // ---- epilogue context, requested first (threads 0 - 255: a column's d, g, count and first kRes list slots,
  // or a row's exponent, into registers), then the ring fill goes out behind it, then the context is written to
  // LDS from registers while the ring lands: the start costs one round trip, not three in a row ----
  int E = 0;
  bool ctx_corrupt = false;             // a residual index or count of the block's columns is out of range
  int64_t cx_a = 0, cx_b = 0;           // d and g of the column, or the row exponent
  int32_t cx_cnt = 0;
  int32_t cx_ec[kRes];
  int64_t cx_ev[kRes];
  if (EX && tid < 256) {
    const int c = tid & 127;
    if (tid < 128) {
      const int n = min(n0 + c, p.N - 1);
      cx_a = p.d[n];
      cx_b = p.g[n];
      cx_cnt = p.R > 0 ? p.cnt[n] : 0;
#pragma unroll
      for (int j = 0; j < kRes; ++j) {
        const bool slot = j < p.R;   // uniform
        cx_ec[j] = slot ? p.ecol[(int64_t)n * p.R + j] : 0;
        cx_ev[j] = slot ? p.eval[(int64_t)n * p.R + j] : 0;
      }
    } else {
      cx_a = p.sh[min(m0 + c, p.M - 1)];
    }
  }

  // ---- ring loads: the first half of the waves load the A planes, the second half the B planes; instruction i of
  // a wave covers 16 rows x 64 bytes (lane: row lane / 4, 16-byte chunk lane % 4, swizzled) ----
  const int lrow = lane >> 2, lch = ((lane & 3) ^ swz<BK>(lrow)) << 4;
  const bool isA = wave < NW / 2;
  const __amdgpu_buffer_rsrc_t rsrc = isA ? __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.a), (short)0,
                                                                               kBufRange, 0x00020000)
                                          : __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.w), (short)0,
                                                                               kBufRange, 0x00020000);
  int voff[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int inst = (wave % (NW / 2)) * LPW + i, pl = inst >> 3, row = (inst & 7) * 16 + lrow;
    voff[i] = isA ? pl * p.M * p.K + min(m0 + row, p.M - 1) * p.K + lch
                  : pl * (int)p.ld_plane + min(n0 + row, p.N - 1) * (int)p.ld_row + lch;
  }
  auto issue = [&](int kt, int stage) {
    char* sbase = smem + stage * STAGE + wave * LPW * 1024;
#pragma unroll
    for (int i = 0; i < LPW; ++i) buf_lds16(rsrc, sbase + i * 1024, voff[i], kt * BK);
  };

  // The first LDS write waits for every LDS DMA in flight (the compiler cannot tell the context area from the
  // ring), so p.xt_pre stages go out before the context is written and the rest after it.
  for (int t = 0; t < p.xt_pre; ++t)
    if (t < nk) issue(t, t);

  if (EX && tid < 256) {
    const int c = tid & 127;
    if (tid < 128) {
      const int cnt = p.R > 0 ? kcnt(p, cx_cnt, ctx_corrupt) : 0;
      s_d[c] = cx_a;
      s_gdr[c] = cx_b - cx_a + p.FR;
      s_cs[c] = n0 + c < p.N ? cnt : 0;
    } else {
      const int64_t v = cx_a;
      s_sh[c] = v;
      int64_t lo = v, hi = v;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        lo = imin(lo, __shfl_xor(lo, o, 64));
        hi = imax(hi, __shfl_xor(hi, o, 64));
      }
      if (lane == 0) {
        s_mm[2 * (c >> 6)] = lo;
        s_mm[2 * (c >> 6) + 1] = hi;
      }
    }
  }
  if (EX) ring_barrier<63>();                               // LDS only: the counts are visible
  if (EX && wave == 0) {                                    // exclusive prefix of the 128 counts, 2 per lane
    const int c0 = s_cs[2 * lane], c1 = s_cs[2 * lane + 1];
    int x = c0 + c1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    const int excl = x - c0 - c1;
    s_cs[2 * lane] = excl;
    s_cs[2 * lane + 1] = excl + c0;
    if (lane == 63) s_cs[BN] = x;
  }
  if (EX) ring_barrier<63>();
  if (EX) E = s_cs[BN];
  if (EX && tid < 128 && E <= kXtEmax) {                    // the compact list: (k, v) of every entry
    const int c = tid, n = min(n0 + c, p.N - 1);
    const int e0 = s_cs[c], e1 = s_cs[c + 1];
#pragma unroll
    for (int j = 0; j < kRes; ++j)
      if (e0 + j < e1) {
        s_ek[e0 + j] = kcol(p, cx_ec[j], ctx_corrupt);
        s_ev[e0 + j] = cx_ev[j];
      }
    for (int e = e0 + kRes; e < e1; ++e) {                  // rare: more entries than the registers hold
      s_ek[e] = kcol(p, p.ecol[(int64_t)n * p.R + (e - e0)], ctx_corrupt);
      s_ev[e] = p.eval[(int64_t)n * p.R + (e - e0)];
    }
  }

  auto load_ops = [&](XtOps<TM, TN>& o, int stage, int h) {
    const char* base = smem + stage * STAGE;
    const int c = 2 * h + (lane >> 5);
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int a2 = 0; a2 < TM; ++a2) {
        const int arow = (wm * TM + a2) * 32 + (lane & 31);
        o.a[i][a2] = *(const v4i*)(base + i * BM * BK + arow * BK + ((c ^ swz<BK>(arow)) << 4));
      }
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int brow = (wn * TN + t) * 32 + (lane & 31);
        o.b[j][t] = *(const v4i*)(base + SA + j * BN * BK + brow * BK + ((c ^ swz<BK>(brow)) << 4));
      }
  };

  // q gathers for the compact residual list into the freed stage: entry e, rows 0..127 at gbase + 512 e
  const __amdgpu_buffer_rsrc_t qrsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(p.q), (short)0, kBufRange, 0x00020000);
  auto gather = [&](char* gbase) {
    for (int x = wave; x < 2 * E; x += NW) {
      const int e = x >> 1, r = (x & 1) * 64 + lane;
      buf_lds4(qrsrc, gbase + e * 512 + (x & 1) * 256, (min(m0 + r, p.M - 1) * (int)p.ldq + s_ek[e]) * 4);
    }
  };
  const bool gat = EX && E > 0 && E <= kXtEmax;
  char* gbase = nullptr;

  v16i acc[5][TM][TN];
#pragma unroll
  for (int s2 = 0; s2 < 5; ++s2)
#pragma unroll
    for (int a2 = 0; a2 < TM; ++a2)
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[s2][a2][t][e] = 0;

  // the nine limb products, A-limb major: an A operand stays on the matrix core's inputs for 3 TN MFMAs in a row
  // (fewer operand bits switch, which the clock under load rewards: +1 % on the M = 2048 prefill shapes); products
  // into one accumulator are still at least four MFMAs apart
  auto mfmas = [&](const XtOps<TM, TN>& o) {
#pragma unroll
    for (int u = 0; u < 9; ++u) {
      constexpr int I[9] = {0, 0, 0, 1, 1, 1, 2, 2, 2}, J[9] = {0, 1, 2, 0, 1, 2, 0, 1, 2};
      const int i = I[u], j = J[u];
#pragma unroll
      for (int a2 = 0; a2 < TM; ++a2)
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[i + j][a2][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a[i][a2], o.b[j][t], acc[i + j][a2][t], 0, 0, 0);
    }
  };

  BX_PHASE(0, 1);
  for (int t = p.xt_pre; t < S; ++t)
    if (t < nk) issue(t, t);
  // first k tile landed (later stages may still be in flight) and visible to every wave
  if (S - 1 < nk)
    ring_barrier<LPW * (S - 1)>();
  else
    ring_barrier<0>();

  BX_PHASE(0, 2);
  XtOps<TM, TN> cur, nxt;
  if (nk > 0) load_ops(cur, 0, 0);
  // One k tile: the second half-step's operands are read during the first half-step's MFMAs, the ring barrier,
  // then (REFILL) the freed stage's refill and the next tile's first operands during the second half-step's MFMAs.
  // Iterations with and without the refill are separate loops, so no branch splits a scheduling region.
  constexpr int NR = 3 * (TM + TN), MR = 9 * TM * TN / NR;   // LDS reads and MFMAs per read in a half-step
  static_assert(NR * MR == 9 * TM * TN && LPW <= NR, "interleave");
  auto step = [&](int it, auto refill) {
    constexpr bool REFILL = decltype(refill)::value;
    const int st = it % S;
    load_ops(nxt, st, 1);
    mfmas(cur);
    // interleave: NR x (MR MFMAs, 1 LDS read)
#pragma unroll
    for (int g2 = 0; g2 < NR; ++g2) {
      __builtin_amdgcn_sched_group_barrier(0x008, MR, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // k tile it + 1 landed (the tiles after it may be in flight), and no wave reads stage st any more
    if (REFILL)
      ring_barrier<LPW * (S - 2)>();
    else
      ring_barrier<0>();
    __builtin_amdgcn_sched_barrier(0);
    if (REFILL) issue(it + S, st);
    load_ops(cur, (it + 1) % S, 0);
    mfmas(nxt);
    if (REFILL) {
      // LPW x (MR MFMAs, 1 buffer load, 1 LDS read), then the remaining LDS reads with MR MFMAs each
#pragma unroll
      for (int g2 = 0; g2 < LPW; ++g2) {
        __builtin_amdgcn_sched_group_barrier(0x008, MR, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
#pragma unroll
      for (int g2 = LPW; g2 < NR; ++g2) {
        __builtin_amdgcn_sched_group_barrier(0x008, MR, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    } else {
#pragma unroll
      for (int g2 = 0; g2 < NR; ++g2) {
        __builtin_amdgcn_sched_group_barrier(0x008, MR, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int it = 0;
  for (; it + S < nk; ++it) step(it, std::true_type{});
  for (; it + 1 < nk; ++it) {
    step(it, std::false_type{});
    if (gat && gbase == nullptr) {      // the ring stopped refilling: stage it % S, free since this step's barrier,
                                        // takes the residual gathers
      gbase = smem + (it % S) * STAGE;
      gather(gbase);
    }
  }
  if (nk > 0) {
    load_ops(nxt, (nk - 1) % S, 1);
    mfmas(cur);
    mfmas(nxt);
  }
  BX_PHASE(0, 3);
  if (gat && gbase == nullptr) {        // short K: the ring was never retired, gather into stage 0 now
    ring_barrier<0>();
    gbase = smem;
    gather(gbase);
  }
  ring_barrier<0>();                    // gathers landed; context visible
  BX_PHASE(0, 4);

  // ---- epilogue: lane (l % 32) owns column (wn TN + t) 32 + l % 32 of each 32-column block t and rows
  // wm 32 + (e / 4) 8 + (l / 32) 4 + e % 4 of the 32 x 32 MFMA block ----
  bool bad = false, corrupt = ctx_corrupt;
  const int32_t* gq = (const int32_t*)gbase;
  // Rounding: exact_round_fast's quick form applies where k = -(sh + g - d + FR) satisfies d <= k, 1 <= k <= 62 and
  // |T| < 2^59, |B| < 2^60. The k conditions hold for every row of a column when they hold for the block's smallest
  // and largest row exponent; |T| < 2^59 holds for K <= 8192 (3-limb q and W: |q W| < 2^46). So a lane checks its
  // column once and each element only checks |B|; an element outside takes the full rule.
  int64_t shlo = 0, shhi = 0;
  if (EX) {
    shlo = imin(s_mm[0], s_mm[2]);
    shhi = imax(s_mm[1], s_mm[3]);
  }
  // full tiles (every row < M and column < N: all of lm_head's) skip the per-output bounds tests
  const bool full = m0 + BM <= p.M && n0 + BN <= p.N;   // block-uniform
  auto epi = [&](auto full_t) {
    constexpr bool FULL = decltype(full_t)::value;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int nl = (wn * TN + t) * 32 + (lane & 31), n = n0 + nl;
      int64_t dn = 0, gdr = 0;
      int cs0 = 0, cs1 = 0;
      bool colok = false;
      if (EX) {
        dn = s_d[nl];
        gdr = s_gdr[nl];
        if (E > 0 && E <= kXtEmax) {
          cs0 = s_cs[nl];
          cs1 = s_cs[nl + 1];
        }
        colok = p.K <= 8192 && shhi + gdr + dn <= 0 && shhi + gdr <= -1 && shlo + gdr >= -62;
      }
#pragma unroll
      for (int a2 = 0; a2 < TM; ++a2)
#pragma unroll
      for (int e0 = 0; e0 < 16; e0 += 4) {
        int64_t B[4] = {0, 0, 0, 0};
        int rl[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = e0 + u;
          rl[u] = (wm * TM + a2) * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        }
        if (EX && E > kXtEmax && n < p.N) {   // long residual lists: read from global memory
          const int c = kcnt(p, p.cnt[n], corrupt);
          for (int j = 0; j < c; ++j) {
            const int col = kcol(p, p.ecol[(int64_t)n * p.R + j], corrupt);
            const int64_t v = p.eval[(int64_t)n * p.R + j];
#pragma unroll
            for (int u = 0; u < 4; ++u)
              B[u] = add_wrap(B[u], mul_wrap((int64_t)p.q[(int64_t)min(m0 + rl[u], p.M - 1) * p.ldq + col], v));
          }
        } else if (EX) {
          for (int x = cs0; x < cs1; ++x) {
            const int64_t v = s_ev[x];
#pragma unroll
            for (int u = 0; u < 4; ++u) B[u] = add_wrap(B[u], mul_wrap((int64_t)gq[x * 128 + rl[u]], v));
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = e0 + u, m = m0 + rl[u];
          const int64_t v = join5(acc[0][a2][t][e], acc[1][a2][t][e], acc[2][a2][t][e], acc[3][a2][t][e],
                                  acc[4][a2][t][e]);
          const bool inb = FULL || (m < p.M && n < p.N);
          int64_t y = v;
          if (EX) {
            const int64_t k = -(s_sh[rl[u]] + gdr);
            const bool fast = colok && (uint64_t)(B[u] + (1LL << 60)) < (uint64_t)(1LL << 61);
            y = (v + ((B[u] + (1LL << (k - 1))) >> dn)) >> (k - dn);
            if (__builtin_amdgcn_ballot_w64(!fast)) {   // rare: some lane needs the full rule
              if (!fast) {
                bool b;
                y = exact_round(v, B[u], dn, -k, b);
                bad |= b && inb;
              }
            }
          }
          if (inb) __builtin_nontemporal_store(y, (int64_t*)p.out + (int64_t)m * p.N + n);
        }
      }
    }
  };
  if (full)
    epi(std::true_type{});
  else
    epi(std::false_type{});
  if (EX) write_flag(p, bad, corrupt);
  BX_PHASE(0, 5);
}

// =====================================================================================================
// stream kernel: decode GEMMs (at most 128 stacked activation rows) as a weight stream through an LDS ring.
// A block owns 64 output columns and a K range (the grid splits K when the column tiles alone do not fill the
// chip). Its weight rows (NB planes x 64 x 128-byte k chunks) and all its activation rows (padded to RP, a
// multiple of 32) go through an S-stage ring filled by buffer_load_dwordx4 ... lds (1 KiB = 8 rows x 128 bytes per
// instruction; 16-byte chunks XOR-swizzled by (row / 2) % 8 so the 16 rows an MFMA operand read touches fall in 16
// distinct bank groups), S - 1 stages ahead of the MFMAs. Each of the 4 waves owns 16 columns:
// v_mfma_i32_16x16x64_i8 over the valid 16-row activation blocks and the NB weight planes (exact mode may run 8
// waves as 4 column groups x 2 row groups, WR = 2; int8 at 128 rows splits the rows instead, RS). The int32 limb
// products meet in LDS (or, for the join of whole 16-row limb blocks, in registers) and are joined per output in
// int64. A block walks its K range (the whole K unless the plan splits it over the zeroed workspace).
// =====================================================================================================
constexpr int kStBK = 128, kStC = 64;

// The largest wave count <= nw that divides the ring's load instructions per stage.
constexpr int st_issuers(int lt, int nw) { return lt % nw == 0 ? nw : st_issuers(lt, nw - 1); }

// WR = 2 (exact mode): 8 waves as 4 column groups x 2 row groups (wave w: columns 16 (w % 4) .., row blocks
// (w / 4) RBM / 2 ..), two waves per SIMD over the same ring; the ring's load instructions go to the first IW waves.
template <int RBM, int NB, int S, int MODE, int NWV = 4, int WR = 1>
__global__ __launch_bounds__(64 * NWV) void stream_kernel(LinArgs p) {
  BX_PHASE(1, 0);
  constexpr int CG = NWV / WR, RH = RBM / WR;                     // column groups, row blocks per wave
  constexpr int RP = RBM < 2 ? 32 : 16 * RBM, BK = kStBK, C = 16 * CG, NT = 64 * NWV;   // loaded rows: x 32
  constexpr int SA = RP * BK, STAGE = SA + NB * C * BK;
  constexpr int LA = RP / 8, LT = LA + NB * C / 8;                // 1 KiB load instructions per stage
  constexpr int IW = st_issuers(LT, NWV), LPW = LT / IW;          // issuing waves, instructions per issuing wave
  static_assert(WR == 1 || (WR == 2 && RBM % 2 == 0 && NB == 3), "row groups: exact mode, even row blocks");
  // RS: at 128 rows and one weight plane a wave owns two 16-row blocks x every column of the tile, not 16 columns x
  // every row: a k chunk's LDS operand reads per block drop from 4 x (128 + 16) rows to 4 x (32 + 64)
  constexpr bool RS = RBM == 2 * NWV && NB == 1 && MODE != EXACT && MODE != WMM_T && WR == 1;
  constexpr int CB = C / 16;
  static_assert(!RS || RBM == 2 * CB, "RS layout: as many accumulators as the row-block layout");
  static_assert(IW * LPW == LT, "load instructions per stage must split over the issuing waves");
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cgw = wave % CG, rgw = wave / CG;                 // the wave's column group and row group
  const bool issuer = wave < IW;
  const int n0 = blockIdx.x * C, kb = blockIdx.y * p.ks;
  const int nks = min(p.ks, p.K - kb) / BK;
  const int rows = p.rows_a;                                  // <= 16 RBM (rows past it repeat the last row)

  const auto ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.a), (short)0, kBufRange, 0x00020000);
  const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.w), (short)0, kBufRange, 0x00020000);
  // exact: the epilogue context of the thread's column (tid % C), requested before the ring
  ColPre cpre;
  if constexpr (MODE == EXACT) cpre = col_pre(p, n0 + tid % C);
  // exact: the row shifts too (thread m holds sh[m] until the epilogue puts them in LDS)
  static_assert(MODE != EXACT || RP <= NT, "one row shift per thread");
  int64_t shpre = 0;
  if constexpr (MODE == EXACT) shpre = p.sh[min(tid, p.M - 1)];
  int voff[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int inst = min(wave * LPW + i, LT - 1);
    const int r8 = inst < LA ? inst : (inst - LA) % (C / 8);      // 8-row group within the A or W plane tile
    const int row = r8 * 8 + (lane >> 3);
    const int lch = ((lane & 7) ^ ((row >> 1) & 7)) << 4;
    if (inst < LA) {
      voff[i] = min(row, rows - 1) * p.K + kb + lch;
    } else {
      const int pl = (inst - LA) / (C / 8);
      voff[i] = pl * (int)p.ld_plane + min(n0 + row, p.N - 1) * (int)p.ld_row + kb + lch;
    }
  }
  auto issue = [&](int it, int stage) {
    if (!issuer) return;                                      // wave-uniform
    char* sbase = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int inst = wave * LPW + i;
      buf_lds16(inst < LA ? ra : rw, sbase + inst * 1024, voff[i], it * BK);
    }
  };

  v4i acc[RH][NB];
#pragma unroll
  for (int r = 0; r < RH; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = v4i{0, 0, 0, 0};

#pragma unroll
  for (int t = 0; t < S - 1; ++t)
    if (t < nks) issue(t, t);
  const int r16 = lane & 15, wrow = cgw * 16 + r16;
  for (int it = 0; it < nks; ++it) {
    // stage it landed (later ones may be in flight) and every wave is done with stage it - 1
    if (it + S - 2 < nks)
      ring_barrier<LPW * (S - 2)>();
    else
      ring_barrier<0>();
    if (it == 1) BX_PHASE(1, 1);
    if (it + S - 1 < nks) issue(it + S - 1, (it + S - 1) % S);
    const char* base = smem + (it % S) * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 4 * h + (lane >> 4);
      if constexpr (RS) {
        // wave w: row blocks w and w + NWV, every column block of the tile (acc[q CB + cb])
        v4i b[CB], a[2];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const int brow = cb * 16 + r16;
          b[cb] = *(const v4i*)(base + SA + brow * BK + ((c ^ ((brow >> 1) & 7)) << 4));
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int arow = (wave + NWV * q) * 16 + r16;
          a[q] = *(const v4i*)(base + arow * BK + ((c ^ ((arow >> 1) & 7)) << 4));
        }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
            acc[q * CB + cb][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[q], b[cb], acc[q * CB + cb][0], 0, 0, 0);
        continue;
      }
      v4i b[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j)
        b[j] = *(const v4i*)(base + SA + (j * C + wrow) * BK + ((c ^ ((wrow >> 1) & 7)) << 4));
      v4i a[RH];
#pragma unroll
      for (int r = 0; r < RH; ++r) {
        const int arow = (rgw * RH + r) * 16 + r16;
        a[r] = *(const v4i*)(base + arow * BK + ((c ^ ((arow >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int r = 0; r < RH; ++r)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[r][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[r], b[j], acc[r][j], 0, 0, 0);
    }
  }

  ring_barrier<0>();
  BX_PHASE(1, 2);
  bool bad = false, corrupt = false;
  const int Mo = MODE == RAW32 ? rows : p.M;                   // output rows
  if constexpr (RS) {
    // JOIN at M = 64 with two limbs: limb rows m and 64 + m sit in the lane's row blocks w and w + 4
    if (MODE == JOIN && p.M == 64 && p.nl == 2) {   // block-uniform
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int n = n0 + cb * 16 + (lane & 15);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t v = (int64_t)acc[cb][0][e] + ((int64_t)acc[CB + cb][0][e] << 8);
          const int m = wave * 16 + (lane >> 4) * 4 + e;
          if (n < p.N) ((int64_t*)p.out)[(int64_t)m * p.N + n] = v;
        }
      }
      return;
    }
  }
  // ---- JOIN with whole 16-row limb blocks (M % 16 == 0): limb row i M + m sits in block m / 16 + i M / 16 of the
  // same lane and element, so the join is done in registers ----
  if constexpr (MODE == JOIN && NB == 1 && !RS) {
    if (p.M % 16 == 0 && p.nl * p.M <= RP) {   // block-uniform
      const int n = n0 + wave * 16 + (lane & 15), bm = p.M >> 4;
#pragma unroll
      for (int r = 0; r < RBM; ++r) {
        if (r < bm) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            int64_t v = 0;
#pragma unroll
            for (int i = 0; i < 3; ++i) {
              const int ri = r + i * bm;
              if (i < p.nl && ri < RBM) v += (int64_t)acc[ri < RBM ? ri : 0][0][e] << (8 * i);
            }
            const int m = r * 16 + (lane >> 4) * 4 + e;
            if (n < p.N) ((int64_t*)p.out)[(int64_t)m * p.N + n] = v;
          }
        }
      }
      return;
    }
  }
  // ---- products to LDS: Cs[j][row][col] (row: stacked activation row, col: block column; pitch C + 1 so the
  // four row groups of a store land in different banks) ----
  constexpr int CP = C + 1;
  int32_t* Cs = (int32_t*)smem;
  if constexpr (RS) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          Cs[((wave + NWV * q) * 16 + (lane >> 4) * 4 + e) * CP + cb * 16 + (lane & 15)] = acc[q * CB + cb][0][e];
  } else {
#pragma unroll
    for (int r = 0; r < RH; ++r)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          Cs[(j * RP + (rgw * RH + r) * 16 + (lane >> 4) * 4 + e) * CP + cgw * 16 + (lane & 15)] = acc[r][j][e];
  }
  __shared__ int64_t s_shm[MODE == EXACT ? RP : 1];
  if constexpr (MODE == EXACT)
    if (tid < RP) s_shm[tid] = shpre;
  __syncthreads();
  const int nla = MODE == JOIN ? p.nl : MODE == RAW32 ? 1 : 3;
  if constexpr (MODE == EXACT || MODE == WMM_T) {
    // a wave per row group, a lane per column: the column's epilogue context is read once and the residual
    // gathers of 8 rows go out together
    // (K split: the partial sums go to the zeroed int64 workspace and the tile's last block finishes them)
    constexpr int RG = NT / C;
    __shared__ int s_last;
    const int c = tid % C, rg = tid / C, n = n0 + c;
    const bool split = gridDim.y > 1;
    ColCtx cc;
    if constexpr (MODE == EXACT) cc = col_ctx_from(p, n, cpre);
    auto finish8 = [&](int m0, const int (&mrow)[8], const int64_t (&v)[8]) {
      int64_t B[8];
      if constexpr (MODE == EXACT) residual_rows<8>(p, cc, mrow, B, corrupt);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int m = m0 + e * RG;
        if (m < Mo && n < p.N) {
          if constexpr (MODE == EXACT) finalize_col(p, cc, m, n, s_shm[m], v[e], B[e], bad, corrupt);
          else ((int64_t*)p.out)[(int64_t)m * p.N + n] = v[e];
        }
      }
    };
    for (int m0 = rg; m0 < Mo; m0 += 8 * RG) {     // wave-uniform
      int mrow[8];
      int64_t v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mrow[e] = min(m0 + e * RG, Mo - 1);
        v[e] = 0;
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j) v[e] += (int64_t)Cs[(j * RP + i * p.M + mrow[e]) * CP + c] << (8 * (i + j));
      }
      if (split) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (m0 + e * RG < Mo && n < p.N) ws_add(p, m0 + e * RG, n, v[e]);
      } else {
        finish8(m0, mrow, v);
      }
    }
    if (split && splitk_last(p, blockIdx.x, gridDim.y, &s_last)) {
      for (int m0 = rg; m0 < Mo; m0 += 8 * RG) {
        int mrow[8];
        int64_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int m = m0 + e * RG;
          mrow[e] = min(m, Mo - 1);
          v[e] = (m < Mo && n < p.N) ? ws_take(p, m, n) : 0;
        }
        finish8(m0, mrow, v);
      }
    }
    if (MODE == EXACT) write_flag(p, bad, corrupt);
    BX_PHASE(1, 3);
    return;
  }
  for (int o = tid; o < Mo * C; o += NT) {
    const int m = o / C, c = o - m * C, n = n0 + c;
    if (n >= p.N) continue;
    int64_t v = 0;
    if (MODE == RAW32) {
      v = Cs[m * CP + c];
    } else {
      for (int i = 0; i < nla; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) v += (int64_t)Cs[(j * RP + i * p.M + m) * CP + c] << (8 * (i + j));
    }
    finalize<MODE>(p, m, n, v, bad, corrupt);
  }
  if (MODE == EXACT) write_flag(p, bad, corrupt);
}

// =====================================================================================================
// wide kernel (exact-mode decode with 65..96 limb rows, wide N)
// =====================================================================================================
// A block owns BNC = 16 CG output columns and every limb row of q (RA = 16 RBW WR >= 3 M), so each weight byte
// is read once and no row part re-reads it (the gemv splits 96 limb rows into two parts, and the second part
// re-reads the weights). The K range is walked in CK-byte chunks. The limb rows of a chunk (the planes of q
// written by split_q_kernel) go through an S = 3 stage LDS ring filled by asynchronous global_load_lds_dwordx4
// (1 KiB per wave instruction = 1024 / CK rows; chunk slots XOR-swizzled by row so the MFMA operand reads hit
// distinct banks); rows past the activations repeat the last row and only feed output rows that are never
// read. Waves are CG column groups x WR row groups; each streams its 16 weight rows from HBM straight into
// v_mfma_i32_16x16x64_i8 B operands. A chunk's weight and limb-row loads form one group, issued two chunks
// ahead. Limb products accumulate in int32 (exact: |sum| <= K 2^14 < 2^31), meet in LDS and are joined in
// int64 per output (sum C_j[i M + m] 2^(8 (i + j))).
constexpr int kWideCK = 256;   // K granularity of the wide plan (chunks are 128 bytes)

template <int NB, int RBW, int WR, int CG, int S, int CK, int MODE>
__global__ __launch_bounds__(64 * WR * CG) void wide_kernel(LinArgs p) {
  constexpr int NW = WR * CG, NT = 64 * NW, RA = 16 * RBW * WR, BNC = 16 * CG, NSTEP = CK / 64;
  constexpr int RPI = 1024 / CK, CHN = CK / 16;                    // rows per 1 KiB load instruction, chunks per row
  constexpr int STAGE = RA * CK, NI = RA / RPI;                    // bytes and load instructions per stage
  constexpr int IPW = (NI + NW - 1) / NW;                          // load instructions per wave per stage (bound)
  static_assert(RA % RPI == 0 && (CK == 128 || CK == 256), "chunk shape");
  extern __shared__ __align__(16) char smem[];
  int32_t* Cs = (int32_t*)smem;                                    // after the K loop: [NB][RA][BNC]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = wave % CG, wr = wave / CG;
  const int n0 = blockIdx.x * BNC;
  const int M = p.M, rows = p.rows_a;
  const int nchunk = p.K / CK;

  // asynchronous activation loads: instruction i of a stage covers rows RPI i .. RPI i + RPI - 1; lane L -> row
  // RPI i + L / CHN, LDS slot L % CHN, global chunk slot ^ (row % CHN)
  const int8_t* abase = p.a;
  auto a_issue = [&](int ch) {
    char* stage = smem + (ch % S) * STAGE;
#pragma unroll
    for (int t = 0; t < IPW; ++t) {
      const int i = wave + t * NW;
      if (i < NI) {
        const int row = RPI * i + lane / CHN;
        const int gc = (lane % CHN) ^ (row % CHN);
        const int8_t* src = abase + (int64_t)min(row, rows - 1) * p.K + ch * CK + gc * 16;
        async16(src, stage + i * 1024);
      }
    }
  };
  // weights: this wave's 16 columns, NB planes, NSTEP k steps of a chunk
  const __amdgpu_buffer_rsrc_t wres = buf_rsrc(p.w + (int64_t)n0 * p.ld_row);
  const int wrow = (min(n0 + cg * 16 + (lane & 15), p.N - 1) - n0) * (int)p.ld_row;
  const int kl = (lane >> 4) * 16;
  auto w_issue = [&](v4i(&b)[NSTEP][NB], int ch) {
#pragma unroll
    for (int u = 0; u < NSTEP; ++u)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        b[u][j] = buf_load16(wres, wrow + j * (int)p.ld_plane + ch * CK + u * 64 + kl);
  };
  v4i acc[RBW][NB];
#pragma unroll
  for (int r = 0; r < RBW; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[r][j] = v4i{0, 0, 0, 0};
  auto compute = [&](const v4i(&b)[NSTEP][NB], int ch) {
    const char* stage = smem + (ch % S) * STAGE;
#pragma unroll
    for (int u = 0; u < NSTEP; ++u)
#pragma unroll
      for (int r = 0; r < RBW; ++r) {
        const int row = (wr * RBW + r) * 16 + (lane & 15);
        const int slot = (u * 4 + (lane >> 4)) ^ (row % CHN);
        const v4i a = *(const v4i*)(stage + row * CK + slot * 16);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[r][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[u][j], acc[r][j], 0, 0, 0);
      }
  };

  // Group g = chunk g's weight loads, then its activation loads; groups are issued S - 1 = 2 chunks ahead and
  // vector memory operations complete in order, so before chunk c is read this wave waits until at most the
  // group issued after it (c + 1) is outstanding, and for everything on the last chunk. LDS reads of the
  // previous chunk are drained too (lgkmcnt 0) before the barrier lets any wave refill that stage.
  static_assert(S == 3, "three register sets and three ring stages");
  // vector memory operations per group: the weights, then IPW activation loads (IPW - 1 for the waves past
  // NI % NW when the instructions do not divide evenly)
  constexpr int NG_HI = NSTEP * NB + IPW, NG_LO = NI % NW == 0 ? NG_HI : NG_HI - 1;
  const bool hi_wave = NI % NW == 0 || wave < NI % NW;
  v4i ws0[NSTEP][NB], ws1[NSTEP][NB], ws2[NSTEP][NB];
  if (0 < nchunk) { w_issue(ws0, 0); a_issue(0); }
  if (1 < nchunk) { w_issue(ws1, 1); a_issue(1); }
  auto step = [&](int c, v4i(&cur)[NSTEP][NB], v4i(&nxt)[NSTEP][NB]) {
    if (c + 1 >= nchunk)
      ring_barrier<0>();
    else if (hi_wave)
      ring_barrier<NG_HI>();
    else
      ring_barrier<NG_LO>();
    if (c + 2 < nchunk) { w_issue(nxt, c + 2); a_issue(c + 2); }
    compute(cur, c);
  };
  for (int ch = 0; ch < nchunk; ch += 3) {
    step(ch, ws0, ws2);
    if (ch + 1 >= nchunk) break;
    step(ch + 1, ws1, ws0);
    if (ch + 2 >= nchunk) break;
    step(ch + 2, ws2, ws1);
  }
  __syncthreads();                              // Cs overlays the activation ring
#pragma unroll
  for (int r = 0; r < RBW; ++r)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = (wr * RBW + r) * 16 + (lane >> 4) * 4 + e, col = cg * 16 + (lane & 15);
        Cs[(j * RA + row) * BNC + col] = acc[r][j][e];
      }
  __syncthreads();
  bool bad = false, corrupt = false;
  for (int e = tid; e < M * BNC; e += NT) {
    const int m = e / BNC, c = e - m * BNC, n = n0 + c;
    if (n >= p.N) continue;
    int64_t v = 0;
    if (MODE == RAW32) {
      v = Cs[m * BNC + c];
    } else if (MODE == JOIN) {
      for (int i = 0; i < p.nl; ++i) v += (int64_t)Cs[(i * M + m) * BNC + c] << (8 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) v += (int64_t)Cs[(j * RA + i * M + m) * BNC + c] << (8 * (i + j));
    }
    finalize<MODE>(p, m, n, v, bad, corrupt);
  }
  if (MODE == EXACT) write_flag(p, bad, corrupt);
}

// =====================================================================================================
// staged kernel (int8 decode with <= 8 stacked activation rows)
// =====================================================================================================
// A block owns BNC output columns and the whole K range; its waves are CGW column groups x KSW k-slices. Wave
// (cg, ks) copies its CR weight rows' KW-byte slices into a private LDS region with asynchronous
// global_load_lds_dwordx4, one contiguous 1 KiB piece (1024 / KW rows) per instruction, all requested at once,
// and its activation fragments straight into registers; then it runs v_mfma_i32_16x16x64_i8 from LDS. The
// k-slices meet in LDS and the limb rows are joined in int64 per output. Contiguous 1 KiB pieces matter: a CU's
// load pipeline moves contiguous kilobytes markedly faster than the 64-byte row segments of a direct MFMA-operand
// load (measured: 5.7 vs 7.3-7.9 us for config 2's down GEMM at M = 1, whose 16.8 MB stream in 4.0 us at best).
// C8: blocks of 8 columns (CR = 8; lanes 8-15 of the MFMA B operand repeat rows 0-7), so that N = 2048 still
// gives 256 blocks without splitting K.
template <int CW, int CGW, int KSW, int KW, int C8, int MODE>
__global__ __launch_bounds__(64 * CGW * KSW) void staged_kernel(LinArgs p) {
  constexpr int NW = CGW * KSW, NT = 64 * NW, CWE = C8 ? 1 : CW;
  constexpr int CR = C8 ? 8 : 16 * CW, BNC = CR * CGW, RPI = 1024 / KW, NI = CR / RPI, STEPS = KW / 64;
  constexpr int PITCH = 1024 + 16;   // LDS bytes per 1 KiB piece (the pad spreads rows over the banks)
  static_assert(KW == 512 || KW == 1024, "k slice");
  extern __shared__ __align__(16) char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cg = wave % CGW, ks = wave / CGW;
  const int n0 = blockIdx.x * BNC + cg * CR, k0 = ks * KW;
  char* wl = smem + wave * NI * PITCH;
  {
    const int lr = lane / (64 / RPI), lb = (lane % (64 / RPI)) * 16;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = min(n0 + i * RPI + lr, p.N - 1);   // rows past N repeat the last row (never stored)
      async16(p.w + (int64_t)row * p.ld_row + k0 + lb, wl + i * PITCH);
    }
  }
  const auto ar = buf_rsrc(p.a);
  const int r16 = lane & 15, kc = (lane >> 4) * 16;
  v4i av[STEPS];
  {
    const int off = min(r16, p.rows_a - 1) * p.K + k0 + kc;   // rows past rows_a repeat the last row
#pragma unroll
    for (int s = 0; s < STEPS; ++s) av[s] = buf_load16(ar, off + s * 64);
  }
  __builtin_amdgcn_s_waitcnt(0);   // the wave's own copies and loads (its LDS region is private)
  v4i acc[CWE];
#pragma unroll
  for (int c = 0; c < CWE; ++c) acc[c] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
#pragma unroll
    for (int c = 0; c < CWE; ++c) {
      const int row = C8 ? (r16 & 7) : c * 16 + r16;
      const v4i b = *(const v4i*)(wl + (row / RPI) * PITCH + (row % RPI) * KW + s * 64 + kc);
      acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[s], b, acc[c], 0, 0, 0);
    }
  __syncthreads();
  v4i* red = (v4i*)smem;   // [ks][cg][c][lane]
#pragma unroll
  for (int c = 0; c < CWE; ++c) red[((ks * CGW + cg) * CWE + c) * 64 + lane] = acc[c];
  __syncthreads();
  // output (m, n): limb row i M + m (< 16) of column cl sits at lane (row / 4) * 16 + cl % 16, element row % 4
  const uint32_t* ri = (const uint32_t*)smem;
  const int col = threadIdx.x % BNC, cgo = col / CR, cl = col % CR, cc = cl >> 4, j = cl & 15;
  const int n = blockIdx.x * BNC + col;
  const int nla = MODE == JOIN ? p.nl : 1;
  bool bad = false, corrupt = false;
  for (int m = threadIdx.x / BNC; m < p.M; m += NT / BNC) {
    int64_t v = 0;
    for (int i = 0; i < nla; ++i) {
      const int r = i * p.M + m, e = ((r >> 2) * 16 + j) * 4 + (r & 3);
      uint32_t sum = 0;   // int32 sums wrap exactly; the total fits (|sum| <= K 2^14 < 2^31)
#pragma unroll
      for (int k2 = 0; k2 < KSW; ++k2) sum += ri[((k2 * CGW + cgo) * CWE + cc) * 256 + e];
      v += (int64_t)(int32_t)sum << (8 * i);
    }
    if (n < p.N) finalize<MODE>(p, m, n, v, bad, corrupt);
  }
}

// =====================================================================================================
// host planning and dispatch
// =====================================================================================================
// tile configurations: (WM, WN, TM, TN, S)
enum TileCfg { T_BIG = 0, T_MID = 1, T_NARROW = 2, T_DEC = 3, T_SMALL = 4 };
struct TileShape {
  int wm, wn, tm, tn, bk, stages;
};
static const TileShape kTiles[5] = {{2, 2, 2, 2, 64, 3},    // 128 x 128, 64x64 wave tiles (prefill)
                                    {2, 2, 1, 2, 64, 3},    // 64 x 128 (few tiles)
                                    {2, 1, 1, 1, 64, 8},    // 64 x 32, deep ring (<= 64 output rows, decode)
                                    {2, 2, 1, 1, 128, 4},   // 64 x 64 (int8 decode, 65..128 limb rows): 128-byte
                                                            // k tiles, so a load instruction covers 8 rows x a
                                                            // whole 128-byte line (15.6 vs 17.4 us at BK = 64)
                                    {2, 2, 1, 1, 128, 2}};  // 64 x 64 (exact, when 64 x 128 tiles fill half the chip)
// 5 accumulator sets: 32x64 wave tiles. Two stages: the next stage's loads are issued right after the barrier
// that frees its buffer. A third stage was measured slower (config-3 down 1730-1810 vs 1900-1960 TOPS, gate / up
// 1700-1830 vs 1890-1930). A CU streams at most ~35 GB/s even from L2 (measured), so a second stage in flight adds
// no bandwidth, only more queued requests ahead of the waves' LDS reads.
static const TileShape kTileExact = {4, 2, 1, 2, 64, 2};

struct Plan {
  int stream;                     // stream kernel: activation row blocks RBM (0: none)
  int nwv;                        // stream kernel: waves per block (16 columns each)
  int wide;                       // wide kernel configuration (0: none)
  int staged;                     // staged kernel configuration (0: none)
  bool gemv;
  int rb, cg, ks_waves, u, spw;   // gemv
  int parts, mp;                  // gemv row parts, output rows per part
  int tile;                       // tile config
  int tiles_x, tiles_y, split, kbytes;
  size_t lds;
  int64_t ws_bytes;               // zero-invariant split-K region
  int64_t tmp_bytes;              // scratch (exact tile path: q limb planes)
};

static int64_t ws_size(int M_out, int N, int tiles) {
  return (((int64_t)M_out * N * 8 + 255) & ~255LL) + (int64_t)tiles * 4;
}

constexpr size_t kGemvLds = 150 * 1024;   // of the 160 KiB per CU

// Decode-kernel shape: column group count cg (16 cg columns per block), row parts (output rows per block
// mp = ceil(M / parts), na mp stacked rows <= 64) and k splits, chosen by a cost in HBM-byte equivalents:
// the weight bytes once, the extra L2-to-CU traffic (weights re-read by the other parts, activations re-read
// by every column tile) at 1/5 of that, the split-K atomics (three 8-byte operations per output per split),
// a chip that is not full and a second round of blocks. Returns false when no shape fits.
static bool gemv_shape(int na, int M, int N, int K, int nb, bool exact, int cus, Plan& best) {
  const int nst = (K + 63) / 64;
  const double W = (double)N * K * nb;
  const double A = exact ? 4.0 * M * K : (double)na * M * K;
  double best_cost = 1e300;
  bool found = false;
  for (int cg = 1; cg <= 4; cg *= 2) {
    const int BNC = 16 * cg, NT = 64 * 16;
    const int c = (N + BNC - 1) / BNC;
    for (int parts = 1; parts <= 8 && parts <= M; parts *= 2) {
      const int mp = (M + parts - 1) / parts;
      if ((M + mp - 1) / mp != parts) continue;        // no empty part
      const int rows = na * mp;
      if (rows > 64) continue;
      const int RA = rows <= 16 ? 16 : rows <= 32 ? 32 : 64;
      const size_t c_lds = (size_t)nb * RA * BNC * 4;
      int split = 0;
      size_t lds = 0;
      for (int k = 1; k <= nst; ++k) {
        const int steps = (nst + k - 1) / k;
        lds = (((size_t)RA * (steps * 64 + 16) + 15) & ~(size_t)15) + c_lds + 64;
        if (lds > kGemvLds) continue;
        split = (nst + steps - 1) / steps;
        if ((int64_t)c * parts * split >= cus) break;
      }
      if (split == 0) continue;
      const int64_t blocks = (int64_t)c * parts * split;
      const int per_cu = (int)std::min<size_t>(160 * 1024 / lds, 2048 / NT);
      const int64_t rounds = (blocks + (int64_t)cus * per_cu - 1) / ((int64_t)cus * per_cu);
      double cost = W + 0.2 * (W * (parts - 1) + A * c);
      if (split > 1) cost += 24.0 * M * N * split;
      if (blocks < cus) cost += W * ((double)cus / blocks - 1.0);
      cost += W * 0.5 * (rounds - 1);
      if (cost < best_cost) {
        best_cost = cost;
        found = true;
        best.cg = cg;
        best.parts = parts;
        best.mp = mp;
        best.rb = RA / 16;
        best.split = split;
      }
    }
  }
  return found;
}

// rows_a: stacked activation rows; nb: weight planes (exact 3, int8 1); na: activation planes on the tile path
static bool gemv_shape(int na, int M, int N, int K, int nb, bool exact, int cus, Plan& best);

// wide configuration (exact mode: 65..96 limb rows, N / 64 >= 128 column tiles, K a multiple of 256)
enum WideCfg { W_NONE = 0, W_E96 = 1 };

static int wide_cfg(int rows_a, int N, int K, bool exact) {
  // int8 (one weight plane) stays on the gemv: its row parts measured as fast or faster (11.5 vs 22 us at
  // M = 64, N = 8192); with three weight planes the wide kernel wins (37 vs 53 us at M = 32, N = 16384)
  if (!exact || rows_a <= 64 || rows_a > 96 || K % kWideCK != 0 || (N + 63) / 64 < 128) return W_NONE;
  return W_E96;
}

// staged configuration (int8, <= 8 stacked rows: one 16-row MFMA block, activations are a small share of a
// CU's bytes): S_C8 = 8-column blocks of K / 1024 waves when that makes 1..2 blocks per CU (down: N = 2048,
// K = 8192); S_C64 = 64-column blocks of 2 x 4 waves over K = 2048 when there is a block per CU (gate / up)
enum StagedCfg { S_NONE = 0, S_C8 = 1, S_C64 = 2 };

static int staged_cfg(int rows_a, int N, int K, bool exact, int cus) {
  if (exact || rows_a > 8) return S_NONE;
  const int b8 = (N + 7) / 8;
  if (K % 1024 == 0 && (K / 1024 == 2 || K / 1024 == 4 || K / 1024 == 8 || K / 1024 == 16) && b8 >= cus &&
      b8 <= 2 * cus)
    return S_C8;
  if (K == 2048 && (N + 63) / 64 >= cus) return S_C64;
  return S_NONE;
}

// Stream plan: <= 128 stacked activation rows (int8 decode; exact decode from 49 limb rows, 17 <= M <= 42),
// K % 128 == 0, 64-column tiles. Int8 takes it when the tiles alone cover the chip (no K split). Measured per launch
// (graph replay, 1x MI355X) against the gemv / staged kernels: M = 64, N = 16384: 14.3 vs 15.7 us; M = 8: 8.6 vs
// 8.9 us; M = 1: 8.2 vs 8.4 us. With N = 2048 or 8192 the K split it would need lost to them (7.2 - 21 vs 6.0 -
// 16 us), so those shapes keep them. Exact mode at M = 32: N = 16384: 26.5 vs 39.1 us (wide kernel), N = 128256:
// 203 vs 289 us; narrow N splits K over the zeroed workspace when every block keeps >= 1024 k (N = 2048, K = 8192:
// 24.3 vs 30.4 us on the 64 x 64 tile); at K = 2048 (8 splits of 256 k: 16.4 vs 11.7 us) the gemv stays.
static bool stream_plan(int rows_a, int M_out, int N, int K, bool exact, bool planes, int cus, Plan& s) {
  static const int on = getenv("BX_STREAM") ? atoi(getenv("BX_STREAM")) : 1;
  if (!on || rows_a > 128 || rows_a < (exact ? 49 : 1) || K % kStBK != 0) return false;
  s.tiles_x = (N + kStC - 1) / kStC;
  s.tiles_y = 1;
  s.split = 1;
  s.nwv = 4;
  // int8 at 65..128 stacked rows with N too narrow for 64-column tiles to cover the chip but wide enough for
  // 32-column ones: 2-wave blocks, one per CU, no K split (M = 64, N = 8192, K = 2048: 11.6 vs 12.0 us on the gemv;
  // at M = 1 / 8 the gemv and staged kernels stay: 6.0-6.3 vs 6.6-6.9 us)
  static const int st32 = getenv("BX_ST32") ? atoi(getenv("BX_ST32")) : 1;
  if (!exact && st32 && rows_a > 64 && s.tiles_x < cus && (N + 31) / 32 >= cus) {
    s.nwv = 2;
    s.tiles_x = (N + 31) / 32;
  }
  if (s.tiles_x < cus) {   // exact only: K split until the tiles cover the chip
    if (!exact) return false;
    const int nch = K / kStBK;
    const int want = std::min(nch, (cus + s.tiles_x - 1) / s.tiles_x);
    const int per = (nch + want - 1) / want;
    if (per < 8 || (planes && rows_a > 64 && rows_a <= 96)) {
      // with q's limb planes from the caller (no split launch) and 65..96 limb rows: 32-column blocks, >= 1024 k
      // each, in one round of blocks that covers most of the chip (M = 32, N = 3072, K = 2048: 14.1 vs
      // 18.8 us for the gemv; N = 2048, K = 8192: 4 splits of 2048 k, 21.3 vs 22.1 us for 64-column blocks in 8
      // splits). Otherwise, under 1024 k per block the split's fixed costs lose to the gemv.
      if (!planes || rows_a <= 64 || rows_a > 96) return false;
      s.nwv = 2;
      s.tiles_x = (N + 31) / 32;
      s.split = std::max(1, std::min(cus / s.tiles_x, nch / 8));
      const int per_split = (nch + s.split - 1) / s.split;   // k chunks per block; no block left without k
      s.split = (nch + per_split - 1) / per_split;
      // one round of blocks, covering at least 3/4 of the chip, or half of it with >= 1024 k a block (N = 2048,
      // K = 2048: 128 blocks, 11.2 vs 11.8 us on the gemv)
      const int nbk = s.tiles_x * s.split;
      if (nbk > cus || (4 * nbk < 3 * cus && (2 * nbk < cus || per_split < 8))) return false;
    } else {
      s.split = (nch + per - 1) / per;
    }
  }
  // long exact grids with the caller's planes at 65..96 rows (lm_head: 2004 tiles of 64): 32-column blocks, two per
  // CU (M = 32, N = 128256: 185.7 vs 196.5 us; at N = 16384, one round of 64-column tiles, 26.4 vs 25.7, so one-round
  // grids keep those)
  if (exact && planes && rows_a > 64 && rows_a <= 96 && s.split == 1 && s.tiles_x > 2 * cus) {
    s.nwv = 2;
    s.tiles_x = (N + 31) / 32;
  }
  s.stream = rows_a <= 16 ? 1 : rows_a <= 32 ? 2 : rows_a <= 64 ? 4 : (exact && rows_a <= 96) ? 6 : 8;
  s.kbytes = (K / kStBK + s.split - 1) / s.split * kStBK;
  s.ws_bytes = s.split > 1 ? ws_size(M_out, N, s.tiles_x) : 0;
  s.tmp_bytes = exact ? 3LL * M_out * K : 0;   // exact: q limb planes (unless the caller brings them)
  return true;
}

// planes: the caller supplies q's limb planes (exact mode), so a plane-reading kernel costs no split launch
static Plan make_plan(int rows_a, int M_out, int N, int K, int nb, int na, bool exact, bool planes = false) {
  Plan s = {};
  const int cus = device_cus();
  const int nst = (K + 63) / 64;
  if (stream_plan(rows_a, M_out, N, K, exact, planes, cus, s)) return s;
  s.wide = wide_cfg(rows_a, N, K, exact);
  s.staged = staged_cfg(rows_a, N, K, exact, cus);
  if (s.staged != S_NONE) {
    s.split = 1;
    return s;
  }
  // int8 decode with 65..128 stacked rows over a wide N (>= one 64-column tile per CU): 64 x 64 tiles with an
  // 8-stage ring read each weight once (17.2 vs 22.3 us for the gemv's two row parts at M = 64, N = 16384); at
  // N = 8192 the tiles would fill half the chip and the gemv stays faster
  const bool dec_tile = !exact && rows_a > 64 && M_out <= 64 && (N + 63) / 64 >= cus;
  if (s.wide != W_NONE) {
    s.tiles_x = (N + 63) / 64;
    s.tiles_y = 1;
    s.split = 1;
    s.tmp_bytes = exact ? 3LL * M_out * K : 0;   // exact: q limb planes
    return s;
  }
  // exact GEMMs of 22..32 rows (66..96 limb rows) with a long K (the engine's down projection, K = 8192) go to the
  // MFMA tiles with K split: 25.6 vs 29.5 us at M = 32, N = 2048 (plus a limb split, unless the caller brings q's
  // limb planes); at K = 2048 the gemv stays (11.0 vs 16.7 us at N = 2048). Wider N (where the plan would pick the
  // 64 x 32 deep-ring tile) was not measured and stays on the gemv.
  const bool long_k_tile = exact && M_out > 21 && M_out <= 32 && K >= 8192 && N <= 3072;   // measured at N = 2048
  if (!long_k_tile && !dec_tile && rows_a <= 128 && gemv_shape(na, M_out, N, K, nb, exact, cus, s)) {
    s.gemv = true;
    const int RA = 16 * s.rb, BNC = 16 * s.cg;
    const int steps = (nst + s.split - 1) / s.split;
    // k steps per wave: at least 2 (fewer k-slices when the block range is short); one load group when
    // every step of the wave fits 8 loads, so all of a wave's weights are requested at once
    s.ks_waves = 16 / s.cg;
    while (s.ks_waves > 1 && (steps + s.ks_waves - 1) / s.ks_waves < 2) s.ks_waves /= 2;
    if (s.ks_waves < 16 / s.cg / 4) s.ks_waves = 1;   // instantiated k-slice counts: 16/cg, 8/cg, 4/cg, 1
    s.spw = (steps + s.ks_waves - 1) / s.ks_waves;
    // three weight planes: two k steps per group (four would need more than the 128 registers a lane of a
    // 1024-thread block has, and spill)
    const int maxu = nb == 3 ? 2 : 8;
    s.u = s.spw <= 2 ? 2 : s.spw <= 4 ? 4 : maxu;
    if (s.u > maxu) s.u = maxu;
    s.kbytes = steps * 64;
    s.split = (nst + steps - 1) / steps;
    s.tiles_x = (N + BNC - 1) / BNC;
    s.tiles_y = s.parts;
    s.lds = (((size_t)RA * (s.kbytes + 16) + 15) & ~(size_t)15) + (size_t)nb * RA * BNC * 4 + 64;
  } else {
    s.gemv = false;
    const int64_t big = (int64_t)((M_out + 127) / 128) * ((N + 127) / 128);
    if (dec_tile)
      s.tile = T_DEC;
    else if (M_out <= 64 && 2 * ((N + 31) / 32) >= cus)
      s.tile = T_NARROW;
    else
      s.tile = big >= cus ? T_BIG : T_MID;
    // exact prefill with few tiles (k / v projections, N = 512): 64 x 64 tiles keep every CU busy (a CU streams
    // at most ~35 GB/s, so idle CUs cost more than the smaller tiles' lower reuse)
    if (exact && s.tile == T_MID && 2 * (int64_t)((M_out + 63) / 64) * ((N + 127) / 128) <= cus) s.tile = T_SMALL;
    const TileShape ts = (s.tile == T_BIG && na * nb == 9) ? kTileExact : kTiles[s.tile];
    const int BM = 32 * ts.tm * ts.wm, BN = 32 * ts.tn * ts.wn;
    s.tiles_x = (N + BN - 1) / BN;
    s.tiles_y = (M_out + BM - 1) / BM;
    const int tiles = s.tiles_x * s.tiles_y;
    const int nkt = (K + ts.bk - 1) / ts.bk;             // k tiles of this configuration
    int split = 1;
    if (2 * tiles < cus) {
      split = (cus + tiles - 1) / tiles;
      const int max_split = nkt / 4 > 1 ? nkt / 4 : 1;   // keep >= 4 k tiles per split
      split = split > max_split ? max_split : split;
    }
    const int kper = (nkt + split - 1) / split;
    s.kbytes = kper * ts.bk;                             // a split's K range: whole k tiles
    s.split = (nkt + kper - 1) / kper;
    s.lds = (size_t)ts.stages * (na * BM + nb * BN) * ts.bk;
    if (exact) s.tmp_bytes = 3LL * M_out * K;
  }
  s.ws_bytes = s.split > 1 ? ws_size(M_out, N, s.tiles_x * s.tiles_y) : 0;
  return s;
}

template <typename KernelT>
static void allow_lds(KernelT kernel, size_t lds) {
  if (lds > 64 * 1024) hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

static void bind_ws(LinArgs& p, const Plan& s) {
  if (s.split > 1) p.sem = (int32_t*)((char*)p.ws + (((int64_t)p.M * p.N * 8 + 255) & ~255LL));
}

template <int NB, int RB, int CG, int KS, int U, int MODE>
static int launch_gemv_cfg(LinArgs& p, const Plan& s, hipStream_t st) {
  allow_lds(gemv_kernel<NB, RB, CG, KS, U, MODE>, s.lds);
  gemv_kernel<NB, RB, CG, KS, U, MODE><<<dim3(s.tiles_x * s.parts, s.split), 64 * CG * KS, s.lds, st>>>(p);
  return check_launch("gemv_kernel");
}

template <int NB, int RB, int CG, int KS, int MODE>
static int launch_gemv_u(LinArgs& p, const Plan& s, hipStream_t st) {
  if constexpr (NB == 3) {
    return launch_gemv_cfg<NB, RB, CG, KS, 2, MODE>(p, s, st);
  } else {
    if (s.u == 2) return launch_gemv_cfg<NB, RB, CG, KS, 2, MODE>(p, s, st);
    if (s.u == 4) return launch_gemv_cfg<NB, RB, CG, KS, 4, MODE>(p, s, st);
    return launch_gemv_cfg<NB, RB, CG, KS, 8, MODE>(p, s, st);
  }
}

template <int NB, int RB, int CG, int MODE>
static int launch_gemv_ks(LinArgs& p, const Plan& s, hipStream_t st) {
  constexpr int KSMAX = 16 / CG;
  if (s.ks_waves == KSMAX) return launch_gemv_u<NB, RB, CG, KSMAX, MODE>(p, s, st);
  if (s.ks_waves == KSMAX / 2) return launch_gemv_u<NB, RB, CG, KSMAX / 2, MODE>(p, s, st);
  if constexpr (KSMAX / 4 > 1)
    if (s.ks_waves == KSMAX / 4) return launch_gemv_u<NB, RB, CG, KSMAX / 4, MODE>(p, s, st);
  if (s.ks_waves == 1) return launch_gemv_u<NB, RB, CG, 1, MODE>(p, s, st);
  set_error("gemv: no kernel for %d k-slices", s.ks_waves);
  return BX_EINVAL;
}

template <int NB, int CG, int MODE>
static int launch_gemv_rb(LinArgs& p, const Plan& s, hipStream_t st) {
  if (s.rb == 1) return launch_gemv_ks<NB, 1, CG, MODE>(p, s, st);
  if (s.rb == 2) return launch_gemv_ks<NB, 2, CG, MODE>(p, s, st);
  return launch_gemv_ks<NB, 4, CG, MODE>(p, s, st);
}

template <int NB, int MODE>
static int launch_gemv(LinArgs& p, const Plan& s, hipStream_t st) {
  // 32-bit buffer offsets: a block's weight rows in every plane, and the whole activation array
  const int64_t wspan = (int64_t)(NB - 1) * p.ld_plane + (int64_t)64 * p.ld_row + p.K;
  const int64_t aspan = MODE == EXACT || MODE == WMM_T ? (int64_t)p.M * p.ldq * 4 : (int64_t)p.rows_a * p.K;
  BX_REQUIRE(wspan < kBufRange - 16 && aspan < kBufRange - 16 && p.ld_plane >= 0,
             "decode path: limb planes and activations must span less than 2 GiB");
  p.ks = s.kbytes;
  p.spw = s.spw;
  p.tiles = s.tiles_x;
  p.parts_lg = s.parts == 1 ? 0 : s.parts == 2 ? 1 : s.parts == 4 ? 2 : 3;
  p.mp = s.mp;
  p.nla = MODE == EXACT || MODE == WMM_T ? 3 : MODE == JOIN ? p.nl : 1;
  bind_ws(p, s);
  if (s.cg == 4) return launch_gemv_rb<NB, 4, MODE>(p, s, st);
  if (s.cg == 2) return launch_gemv_rb<NB, 2, MODE>(p, s, st);
  return launch_gemv_rb<NB, 1, MODE>(p, s, st);
}

template <int NA, int NB, int MODE, int WM, int WN, int TM, int TN, int BK, int S>
static int launch_tile_cfg(LinArgs& p, const Plan& s, hipStream_t st) {
  allow_lds(tile_kernel<NA, NB, MODE, WM, WN, TM, TN, BK, S>, s.lds);
  tile_kernel<NA, NB, MODE, WM, WN, TM, TN, BK, S><<<dim3(s.tiles_x, s.tiles_y, s.split), WM * WN * 64, s.lds, st>>>(p);
  return check_launch("tile_kernel");
}

// The xtile kernel's conditions: whole 64-deep k tiles, no K split, 32-bit buffer offsets for q, its limb planes
// and the weight planes.
static bool xtile_fits(const LinArgs& p, const Plan& s) {
  return s.split == 1 && p.K % kXtBK == 0 && 3LL * p.M * p.K < kBufRange - 16 &&
         2 * p.ld_plane + (int64_t)p.N * p.ld_row < kBufRange - 16 && (int64_t)p.M * p.ldq * 4 < kBufRange - 16;
}

template <int NA, int NB, int MODE>
static int launch_tile(LinArgs& p, const Plan& s, hipStream_t st) {
  p.ks = s.kbytes;
  bind_ws(p, s);
  if (s.tile == T_BIG) {
    if constexpr (NA * NB == 9 && (MODE == EXACT || MODE == WMM_T)) {
      // BX_XTILE=0 / BX_XCD=0 switch the pipelined tile / its XCD-grouped order off (the same integers either way)
      static const int xt = getenv("BX_XTILE") ? atoi(getenv("BX_XTILE")) : 1;
      static const int xcd = getenv("BX_XCD") ? atoi(getenv("BX_XCD")) : 4;   // row tiles per XCD group
      if (xt && xtile_fits(p, s)) {
        p.xcd_remap = (xcd > 0 && (s.tiles_x * s.tiles_y) % 8 == 0 && s.tiles_y % xcd == 0) ? xcd : 0;
        static const int pre = getenv("BX_XT_PRE") ? atoi(getenv("BX_XT_PRE")) : 1;
        p.xt_pre = std::max(0, std::min(pre, kXtS));
        allow_lds(xtile_kernel<MODE, 4, 2, 1, 2>, kXtLds);
        xtile_kernel<MODE, 4, 2, 1, 2><<<dim3(s.tiles_x, s.tiles_y, 1), 512, kXtLds, st>>>(p);
        return check_launch("xtile_kernel");
      }
      return launch_tile_cfg<NA, NB, MODE, 4, 2, 1, 2, 64, 2>(p, s, st);   // kTileExact
    } else if constexpr (NA * NB == 9) {
      return launch_tile_cfg<NA, NB, MODE, 4, 2, 1, 2, 64, 2>(p, s, st);   // kTileExact
    }
    else
      return launch_tile_cfg<NA, NB, MODE, 2, 2, 2, 2, 64, 3>(p, s, st);
  }
  if (s.tile == T_MID) return launch_tile_cfg<NA, NB, MODE, 2, 2, 1, 2, 64, 3>(p, s, st);
  if constexpr (NA * NB == 9)
    if (s.tile == T_SMALL) return launch_tile_cfg<NA, NB, MODE, 2, 2, 1, 1, 128, 2>(p, s, st);
  if constexpr (NB == 1) {
    if (s.tile == T_DEC) return launch_tile_cfg<NA, NB, MODE, 2, 2, 1, 1, 128, 4>(p, s, st);
  }
  return launch_tile_cfg<NA, NB, MODE, 2, 1, 1, 1, 64, 8>(p, s, st);
}

template <int NB, int RBW, int WR, int CG, int CK, int MODE>
static int launch_wide_cfg(LinArgs& p, const Plan& s, hipStream_t st) {
  constexpr int S = 3, RA = 16 * RBW * WR, BNC = 16 * CG;
  const size_t lds = std::max<size_t>((size_t)S * RA * CK, (size_t)NB * RA * BNC * 4);
  BX_REQUIRE(p.rows_a <= RA && p.K % CK == 0, "wide plan shape");
  allow_lds(wide_kernel<NB, RBW, WR, CG, S, CK, MODE>, lds);
  wide_kernel<NB, RBW, WR, CG, S, CK, MODE><<<s.tiles_x, 64 * WR * CG, lds, st>>>(p);
  return check_launch("wide_kernel");
}

template <int MODE>
static int launch_wide(LinArgs& p, const Plan& s, hipStream_t st) {
  // weight offsets of a block are 32-bit buffer offsets
  BX_REQUIRE((int64_t)p.ld_plane * 2 + (int64_t)64 * p.ld_row + p.K < (1LL << 31), "weight span exceeds 2^31 bytes");
  return launch_wide_cfg<3, 3, 2, 4, 128, MODE>(p, s, st);        // 96 limb rows: q of up to 32 tokens
}

template <int CW, int CGW, int KSW, int KW, int C8, int MODE>
static int launch_staged_cfg(LinArgs& p, hipStream_t st) {
  constexpr int CR = C8 ? 8 : 16 * CW, BNC = CR * CGW, NW = CGW * KSW;
  const size_t lds = std::max((size_t)NW * (CR * KW / 1024) * 1040, (size_t)NW * (C8 ? 1 : CW) * 1024);
  BX_REQUIRE(p.rows_a <= 16 && p.K == KSW * KW, "staged plan shape");
  allow_lds(staged_kernel<CW, CGW, KSW, KW, C8, MODE>, lds);
  staged_kernel<CW, CGW, KSW, KW, C8, MODE><<<(p.N + BNC - 1) / BNC, 64 * NW, lds, st>>>(p);
  return check_launch("staged_kernel");
}

template <int MODE>
static int launch_staged(LinArgs& p, const Plan& s, hipStream_t st) {
  // activation offsets are 32-bit buffer offsets
  BX_REQUIRE((int64_t)p.rows_a * p.K < kBufRange - 16, "activations span more than 2 GiB");
  if (s.staged == S_C64) return launch_staged_cfg<2, 2, 4, 512, 0, MODE>(p, st);
  switch (p.K / 1024) {
    case 2: return launch_staged_cfg<1, 1, 2, 1024, 1, MODE>(p, st);
    case 4: return launch_staged_cfg<1, 1, 4, 1024, 1, MODE>(p, st);
    case 8: return launch_staged_cfg<1, 1, 8, 1024, 1, MODE>(p, st);
    default: return launch_staged_cfg<1, 1, 16, 1024, 1, MODE>(p, st);
  }
}

template <int RBM, int NB, int S, int MODE, int NWV = 4, int WR = 1>
static int launch_stream_cfg(LinArgs& p, const Plan& s, hipStream_t st) {
  constexpr int RP = RBM < 2 ? 32 : 16 * RBM, C = 16 * NWV / WR;
  const size_t lds = std::max((size_t)S * kStBK * (RP + NB * C), (size_t)NB * RP * (C + 1) * 4);
  allow_lds(stream_kernel<RBM, NB, S, MODE, NWV, WR>, lds);
  stream_kernel<RBM, NB, S, MODE, NWV, WR><<<dim3(s.tiles_x, s.split), 64 * NWV, lds, st>>>(p);
  return check_launch("stream_kernel");
}

template <int MODE>
static int launch_stream(LinArgs& p, const Plan& s, hipStream_t st) {
  constexpr bool EX = MODE == EXACT || MODE == WMM_T;
  BX_REQUIRE((int64_t)p.rows_a * p.K < kBufRange - 16 &&
                 (EX ? 2 * p.ld_plane : 0) + (int64_t)p.N * p.ld_row < kBufRange - 16,
             "stream path: activations and weights must span less than 2 GiB");
  p.ks = s.kbytes;
  bind_ws(p, s);
  if constexpr (EX) {   // three weight planes: 4-stage rings (3 at 128 rows) within the 160 KiB of LDS
    if (s.stream == 1) return launch_stream_cfg<1, 3, 4, MODE>(p, s, st);
    if (s.stream == 2) return launch_stream_cfg<2, 3, 4, MODE>(p, s, st);
    // from 49 rows, grids of at most two rounds of blocks: 8 waves in two row groups (two waves per SIMD; measured
    // per launch at N = 16384, K = 2048: M = 20 24.5 vs 25.4 us, M = 40 26.7 vs 29.0, M = 32 equal; lm_head's 2004
    // blocks were 1.5 % slower, so long grids keep 4 waves over every row; BX_ST_WR=1 turns the form off)
    static const int wr = getenv("BX_ST_WR") ? atoi(getenv("BX_ST_WR")) : 2;
    const bool two = wr == 2 && (int64_t)s.tiles_x * s.split <= 2 * device_cus();
    if (s.stream == 4) return two ? launch_stream_cfg<4, 3, 4, MODE, 8, 2>(p, s, st)
                                  : launch_stream_cfg<4, 3, 4, MODE>(p, s, st);
    // 32-column blocks at 65..96 rows (planner): 4 waves as 2 column groups x 2 row groups, so every SIMD has one
    // (wqkv N = 3072: 12.2 vs 14.0 us with 2 waves over every row; down N = 2048, K = 8192: 19.4 vs 21.1)
    // (a 3-stage ring, 72 KiB: two blocks fit a CU; lm_head 185.7 vs 196.5 us, engine +0.45 % on wqkv / wo / wd)
    if (s.nwv == 2) return wr == 2 ? launch_stream_cfg<6, 3, 3, MODE, 4, 2>(p, s, st)
                                   : launch_stream_cfg<6, 3, 4, MODE, 2>(p, s, st);
    if (s.stream == 6) return two ? launch_stream_cfg<6, 3, 4, MODE, 8, 2>(p, s, st)
                                  : launch_stream_cfg<6, 3, 4, MODE>(p, s, st);
    return two ? launch_stream_cfg<8, 3, 3, MODE, 8, 2>(p, s, st) : launch_stream_cfg<8, 3, 3, MODE>(p, s, st);
  }
  // ring depth: 4 stages at 16 rows (8 measured ~0.5 us slower per launch at M = 1), 8 at 32 / 64, 6 at 128
  if (s.nwv == 2) {   // 32-column blocks (planner: int8 N with 32-column tiles covering the chip)
    if (s.stream == 1) return launch_stream_cfg<1, 1, 4, MODE, 2>(p, s, st);
    if (s.stream == 2) return launch_stream_cfg<2, 1, 8, MODE, 2>(p, s, st);
    if (s.stream == 4) return launch_stream_cfg<4, 1, 8, MODE, 2>(p, s, st);
    return launch_stream_cfg<8, 1, 6, MODE, 2>(p, s, st);
  }
  if (s.stream == 1) return launch_stream_cfg<1, 1, 4, MODE>(p, s, st);
  if (s.stream == 2) return launch_stream_cfg<2, 1, 8, MODE>(p, s, st);
  if (s.stream == 4) return launch_stream_cfg<4, 1, 8, MODE>(p, s, st);
  return launch_stream_cfg<8, 1, 6, MODE>(p, s, st);
}

static bool aligned16(const void* x) { return ((uintptr_t)x & 15) == 0; }

static int need_ws(const LinArgs& p, const Plan& s, int64_t ws_bytes, const void* tmp, int64_t tmp_bytes) {
  if (s.ws_bytes > 0)
    BX_REQUIRE(p.ws != nullptr && ws_bytes >= s.ws_bytes, "workspace too small (%lld < %lld)", (long long)ws_bytes,
               (long long)s.ws_bytes);
  if (s.tmp_bytes > 0)
    BX_REQUIRE(tmp != nullptr && tmp_bytes >= s.tmp_bytes && aligned16(tmp), "scratch too small (%lld < %lld)",
               (long long)tmp_bytes, (long long)s.tmp_bytes);
  return BX_OK;
}

}  // namespace bx

using namespace bx;

static int exact_common(LinArgs& p, int mode, int64_t ws_bytes, void* tmp, int64_t tmp_bytes, hipStream_t st,
                        const int8_t* planes = nullptr) {
  BX_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, "negative size");
  BX_REQUIRE(p.K % 16 == 0, "K %% 16 != 0 (K=%d)", p.K);
  BX_REQUIRE(p.K < 43690, "K >= 43690: int32 limb sums could overflow");
  BX_REQUIRE(p.ldq % 4 == 0 && p.ldq >= p.K, "ldq must be >= K and a multiple of 4");
  BX_REQUIRE(p.ld_row % 16 == 0 && p.ld_plane % 16 == 0, "limb strides must be multiples of 16");
  BX_REQUIRE(aligned16(p.q) && aligned16(p.w), "q and limbs must be 16-byte aligned");
  if (p.M == 0 || p.N == 0) return BX_OK;
  BX_REQUIRE(p.K > 0, "K == 0");
  p.rows_a = 3 * p.M;
  Plan s = make_plan(p.rows_a, p.M, p.N, p.K, 3, 3, true, planes != nullptr);
  if (planes != nullptr) s.tmp_bytes = 0;   // the caller's limb planes replace the scratch
  if (int rc = need_ws(p, s, ws_bytes, tmp, tmp_bytes)) return rc;
  if (s.gemv) return mode == EXACT ? launch_gemv<3, EXACT>(p, s, st) : launch_gemv<3, WMM_T>(p, s, st);
  if (planes != nullptr) {
    p.a = planes;
  } else {
    int8_t* tp = (int8_t*)tmp;
    const int64_t chunks = (int64_t)p.M * (p.K / 16);
    const int blocks = (int)((chunks + 255) / 256 < 4096 ? (chunks + 255) / 256 : 4096);
    split_q_kernel<<<blocks, 256, 0, st>>>(p.q, p.ldq, p.M, p.K, tp);
    if (int rc = check_launch("split_q_kernel")) return rc;
    p.a = tp;
  }
  if (s.stream) return mode == EXACT ? launch_stream<EXACT>(p, s, st) : launch_stream<WMM_T>(p, s, st);
  if (s.wide) return mode == EXACT ? launch_wide<EXACT>(p, s, st) : launch_wide<WMM_T>(p, s, st);
  return mode == EXACT ? launch_tile<3, 3, EXACT>(p, s, st) : launch_tile<3, 3, WMM_T>(p, s, st);
}

extern "C" int bx_exact_linear(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs,
                               int64_t ld_plane, int64_t ld_row, const int64_t* d, const int64_t* g,
                               const int32_t* ell_cnt, const int32_t* ell_col, const int64_t* ell_val, int32_t R,
                               int64_t* y, int32_t M, int32_t N, int32_t K, int32_t FR, int32_t checked,
                               int32_t* flag, void* ws, int64_t ws_bytes, void* tmp, int64_t tmp_bytes,
                               bx_stream_t stream) {
  LinArgs p = {};
  p.q = q; p.ldq = ldq; p.w = limbs; p.ld_plane = ld_plane; p.ld_row = ld_row;
  p.sh = sh; p.d = d; p.g = g; p.cnt = ell_cnt; p.ecol = ell_col; p.eval = ell_val; p.R = R;
  p.out = y; p.flag = flag; p.checked = checked; p.FR = FR; p.M = M; p.N = N; p.K = K;
  p.ws = (int64_t*)ws;
  BX_REQUIRE(R >= 0 && (R == 0 || (ell_cnt && ell_col && ell_val)), "ELL residual arrays missing");
  BX_REQUIRE(!checked || flag, "checked needs a flag pointer");
  BX_REQUIRE(sh && d && g && y, "null pointer");
  return exact_common(p, EXACT, ws_bytes, tmp, tmp_bytes, (hipStream_t)stream);
}

extern "C" int bx_exact_linear_planes(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs,
                                      int64_t ld_plane, int64_t ld_row, const int64_t* d, const int64_t* g,
                                      const int32_t* ell_cnt, const int32_t* ell_col, const int64_t* ell_val,
                                      int32_t R, int64_t* y, int32_t M, int32_t N, int32_t K, int32_t FR,
                                      int32_t checked, int32_t* flag, void* ws, int64_t ws_bytes,
                                      const int8_t* q_planes, bx_stream_t stream) {
  BX_REQUIRE(q_planes && aligned16(q_planes), "q_planes: null or not 16-byte aligned");
  LinArgs p = {};
  p.q = q; p.ldq = ldq; p.w = limbs; p.ld_plane = ld_plane; p.ld_row = ld_row;
  p.sh = sh; p.d = d; p.g = g; p.cnt = ell_cnt; p.ecol = ell_col; p.eval = ell_val; p.R = R;
  p.out = y; p.flag = flag; p.checked = checked; p.FR = FR; p.M = M; p.N = N; p.K = K;
  p.ws = (int64_t*)ws;
  BX_REQUIRE(R >= 0 && (R == 0 || (ell_cnt && ell_col && ell_val)), "ELL residual arrays missing");
  BX_REQUIRE(!checked || flag, "checked needs a flag pointer");
  BX_REQUIRE(sh && d && g && y, "null pointer");
  return exact_common(p, EXACT, ws_bytes, nullptr, 0, (hipStream_t)stream, q_planes);
}

extern "C" int bx_exact_wmm(const int32_t* q, int64_t ldq, const int8_t* limbs, int64_t ld_plane, int64_t ld_row,
                            int64_t* T, int32_t M, int32_t N, int32_t K, void* ws, int64_t ws_bytes, void* tmp,
                            int64_t tmp_bytes, bx_stream_t stream) {
  LinArgs p = {};
  p.q = q; p.ldq = ldq; p.w = limbs; p.ld_plane = ld_plane; p.ld_row = ld_row;
  p.out = T; p.M = M; p.N = N; p.K = K; p.ws = (int64_t*)ws;
  BX_REQUIRE(T, "null pointer");
  return exact_common(p, WMM_T, ws_bytes, tmp, tmp_bytes, (hipStream_t)stream);
}

extern "C" int64_t bx_exact_linear_workspace(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return make_plan(3 * M, M, N, K, 3, 3, true).ws_bytes;
}

extern "C" int64_t bx_exact_linear_scratch(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return make_plan(3 * M, M, N, K, 3, 3, true).tmp_bytes;
}

extern "C" int64_t bx_exact_linear_planes_workspace(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return make_plan(3 * M, M, N, K, 3, 3, true, true).ws_bytes;
}

extern "C" int32_t bx_exact_linear_reads_planes(int32_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return make_plan(3 * M, M, N, K, 3, 3, true, true).gemv ? 0 : 1;
}

static int int8_common(LinArgs& p, int mode, int64_t ws_bytes, hipStream_t st) {
  BX_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, "negative size");
  BX_REQUIRE(p.K % 16 == 0, "K %% 16 != 0 (K=%d)", p.K);
  BX_REQUIRE((int64_t)p.K * 127 * 128 < (1LL << 31), "K too large for exact int32 sums");
  BX_REQUIRE(aligned16(p.a) && aligned16(p.w), "a and w must be 16-byte aligned");
  if (p.M == 0 || p.N == 0) return BX_OK;
  BX_REQUIRE(p.K > 0, "K == 0");
  const int na = mode == RAW32 ? 1 : p.nl;
  const Plan s = make_plan(p.rows_a, p.M, p.N, p.K, 1, na, false);
  if (int rc = need_ws(p, s, ws_bytes, nullptr, 0)) return rc;
  if (s.stream) return mode == JOIN ? launch_stream<JOIN>(p, s, st) : launch_stream<RAW32>(p, s, st);
  if (s.staged) return mode == JOIN ? launch_staged<JOIN>(p, s, st) : launch_staged<RAW32>(p, s, st);
  if (s.gemv) return mode == JOIN ? launch_gemv<1, JOIN>(p, s, st) : launch_gemv<1, RAW32>(p, s, st);
  if (mode == RAW32) return launch_tile<1, 1, RAW32>(p, s, st);
  if (p.nl == 1) return launch_tile<1, 1, JOIN>(p, s, st);
  if (p.nl == 2) return launch_tile<2, 1, JOIN>(p, s, st);
  return launch_tile<3, 1, JOIN>(p, s, st);
}

extern "C" int bx_int8_gemm(const int8_t* a, const int8_t* w, int32_t* c, int32_t R, int32_t N, int32_t K, void* ws,
                            int64_t ws_bytes, bx_stream_t stream) {
  LinArgs p = {};
  p.a = a; p.w = w; p.ld_row = K; p.ld_plane = 0; p.out = c; p.M = R; p.N = N; p.K = K;
  p.rows_a = R; p.nl = 1; p.ws = (int64_t*)ws;
  BX_REQUIRE(c, "null pointer");
  return int8_common(p, RAW32, ws_bytes, (hipStream_t)stream);
}

extern "C" int bx_int8_gemm_join(const int8_t* a, const int8_t* w, int64_t* y, int32_t M, int32_t N, int32_t K,
                                 int32_t nl, void* ws, int64_t ws_bytes, bx_stream_t stream) {
  BX_REQUIRE(nl >= 1 && nl <= 3, "nl must be 1, 2 or 3");
  LinArgs p = {};
  p.a = a; p.w = w; p.ld_row = K; p.ld_plane = 0; p.out = y; p.M = M; p.N = N; p.K = K;
  p.rows_a = nl * M; p.nl = nl; p.ws = (int64_t*)ws;
  BX_REQUIRE(y, "null pointer");
  return int8_common(p, JOIN, ws_bytes, (hipStream_t)stream);
}

extern "C" int64_t bx_int8_gemm_workspace(int32_t M, int32_t N, int32_t K, int32_t nl) {
  if (M <= 0 || N <= 0 || K <= 0 || nl < 1 || nl > 3) return 0;
  return make_plan(nl * M, M, N, K, 1, nl, false).ws_bytes;
}

// Which kernel bx_exact_linear launches for (M, N, K) (tests use it to prove they reach every configuration):
// out[0] = 1 gemv, 2 wide, 3 tile, 5 stream; out[1] = tile configuration (0 T_BIG, 1 T_MID, 2 T_NARROW, 3 T_DEC,
// 4 T_SMALL; -1 otherwise); out[2] = K splits; out[3] = blocks per split.
static int exact_plan_out(const Plan& s, int32_t* out) {
  out[0] = s.stream ? 5 : s.gemv ? 1 : s.wide ? 2 : 3;
  out[1] = (s.gemv || s.wide || s.stream) ? -1 : s.tile;
  out[2] = s.split;
  out[3] = s.gemv ? s.tiles_x * s.parts : s.tiles_x * s.tiles_y;
  return BX_OK;
}

extern "C" int bx_exact_linear_plan(int32_t M, int32_t N, int32_t K, int32_t* out) {
  BX_REQUIRE(out && M > 0 && N > 0 && K > 0, "bad plan query");
  return exact_plan_out(make_plan(3 * M, M, N, K, 3, 3, true), out);
}

extern "C" int bx_exact_linear_planes_plan(int32_t M, int32_t N, int32_t K, int32_t* out) {
  BX_REQUIRE(out && M > 0 && N > 0 && K > 0, "bad plan query");
  return exact_plan_out(make_plan(3 * M, M, N, K, 3, 3, true, true), out);
}

// The int8 GEMM's plan for M output rows of nl stacked limbs (nl = 0: the raw int32 GEMM of M stacked rows):
// out[0] = 1 gemv, 3 tile, 4 staged, 5 stream; out[1] = tile configuration (-1 otherwise); out[2] = K splits; out[3] =
// blocks per split; out[4] = gemv column groups (16 columns each); out[5] = gemv row parts.
extern "C" int bx_int8_gemm_plan(int32_t M, int32_t N, int32_t K, int32_t nl, int32_t* out) {
  BX_REQUIRE(out && M > 0 && N > 0 && K > 0 && nl >= 0 && nl <= 3, "bad plan query");
  const Plan s = nl == 0 ? make_plan(M, M, N, K, 1, 1, false) : make_plan(nl * M, M, N, K, 1, nl, false);
  out[0] = s.stream ? 5 : s.staged ? 4 : s.gemv ? 1 : 3;
  out[1] = (s.gemv || s.staged || s.stream) ? -1 : s.tile;
  out[2] = s.split;
  out[3] = s.gemv ? s.tiles_x * s.parts : s.tiles_x * s.tiles_y;
  out[4] = s.gemv ? s.cg : 0;
  out[5] = s.gemv ? s.parts : 0;
  return BX_OK;
}

// ---- the exact linear without caller buffers ----
// `scratch` is a file-scope device array: each GPU the library runs on holds its own copy until the process ends.
// Its first kNoAllocWs bytes are the split-K workspace (int64 partial sums and tile counters), the rest the q limb
// planes. Host code never passes `scratch` itself to a kernel (in host code the name is only a stand-in): the
// device address comes from hipGetSymbolAddress, once per device, with that device current.
constexpr int64_t kNoAllocWs = 8LL << 20;
constexpr int64_t kNoAllocTmp = 24LL << 20;
static __device__ __align__(256) int8_t scratch[kNoAllocWs + kNoAllocTmp];

namespace bx {

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64] = {};

static int scratch_ptr(void** out) {
  int dev = -1;
  BX_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64, "no current HIP device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      return BX_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BX_OK;
}

__global__ __launch_bounds__(256) void zero_kernel(int4* p, int64_t n16) {
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256) p[i] = int4{0, 0, 0, 0};
}

}  // namespace bx

extern "C" int64_t bx_exact_linear_noalloc_limit(void) { return kNoAllocWs + kNoAllocTmp; }

extern "C" int bx_exact_linear_noalloc(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs,
                                       int64_t ld_plane, int64_t ld_row, const int64_t* d, const int64_t* g,
                                       const int32_t* ell_cnt, const int32_t* ell_col, const int64_t* ell_val,
                                       int32_t R, int64_t* y, int32_t M, int32_t N, int32_t K, int32_t FR,
                                       int32_t checked, int32_t* flag, bx_stream_t stream) {
  BX_REQUIRE(M >= 0 && N >= 0 && K >= 0, "negative size");
  if (M == 0 || N == 0) return BX_OK;
  BX_REQUIRE(K > 0, "K == 0");
  const Plan s = make_plan(3 * M, M, N, K, 3, 3, true);
  BX_REQUIRE(s.ws_bytes <= kNoAllocWs, "no-alloc linear: split-K workspace of %lld bytes exceeds the static %lld",
             (long long)s.ws_bytes, (long long)kNoAllocWs);
  BX_REQUIRE(s.tmp_bytes <= kNoAllocTmp, "no-alloc linear: limb-plane scratch of %lld bytes exceeds the static %lld",
             (long long)s.tmp_bytes, (long long)kNoAllocTmp);
  void* base = nullptr;
  if (int rc = scratch_ptr(&base)) return rc;
  // the workspace contract wants zeros on entry; the array keeps whatever the last call left, so clear the part
  // this call uses (a fill kernel, so the call stays capturable)
  if (s.ws_bytes > 0) {
    const int64_t n16 = (s.ws_bytes + 15) / 16;
    const int blocks = (int)std::min<int64_t>((n16 + 255) / 256, 1024);
    zero_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>((int4*)base, n16);
    if (int rc = check_launch("zero_kernel")) return rc;
  }
  return bx_exact_linear(q, ldq, sh, limbs, ld_plane, ld_row, d, g, ell_cnt, ell_col, ell_val, R, y, M, N, K, FR,
                         checked, flag, base, kNoAllocWs, (int8_t*)base + kNoAllocWs, kNoAllocTmp, stream);
}

BX_PHASE_DEFINE(linear)
