// RoPE + q grouping + K / V store of one (token, head row) (segs.rope_y + segs.q_group, src/bitexact/exact/segs.py:
// 66-99; the fused store of src/bitexact/vllm_plugin/exact_fuse.py:372-386), shared by the standalone rope kernel
// (csrc/bx_segs.hip) and the decode attention that runs it as its prologue (csrc/bx_attn.hip).
#pragma once
#include "bx_common.h"

namespace bx {

constexpr int64_t kSegNegBig = -(1LL << 20);   // ops.NEG_BIG
constexpr int kSegQB = 22;                     // |q| <= 2^22

struct RopeArgs {
  const int64_t* y;        // [B T, ldy] at FR: q heads, k heads, v heads (H + 2 HKV) HD columns
  int64_t ldy;
  const int64_t* pos;      // [B, T] (strides spb, spt)
  int64_t spb, spt;
  const int64_t* cos;      // [n_pos, HD / 2] at FT
  const int64_t* sin;
  int npos;
  int B, T, H, HKV, HD;
  int FR, FT, FK, FV, FZ;
  int32_t* qg;             // [B HKV, g T, HD]
  int64_t* shg;            // [B HKV, g T]
  int64_t* k;              // [B, T, HKV, HD] (null: not written)
  int64_t* v;
  int32_t* err;
  int8_t* cache;           // paged limb-plane cache [nb][HKV][bs][8 HD] (null: no store)
  int64_t sc_nb, sc_h, sc_bs;
  const int64_t* slot;     // [B T] cache slot of each token (< 0: not stored)
  int bs;
};

// The three int8 limbs of a K (plane 0) or V (plane 3) value into the paged cache at the token's slot, as the
// reference's fused qkv kernel stores them (src/bitexact/vllm_plugin/exact_fuse.py:223-236; tri_paged.store's
// layout, src/bitexact/vllm_plugin/tri_paged.py:311-335): limb i at byte (plane + i) HD + d of the slot's row.
__device__ __forceinline__ void store_limbs(const RopeArgs& p, int token, int h, int plane, int d, int64_t x) {
  if (!p.cache) return;
  const int64_t sl = p.slot[token];
  if (sl < 0) return;                                  // dummy / padded tokens carry slot -1
  int8_t* base = p.cache + (sl / p.bs) * p.sc_nb + h * p.sc_h + (sl % p.bs) * p.sc_bs + (int64_t)plane * p.HD + d;
  int32_t r = (int32_t)x;                              // |x| <= 8355711: three signed base-256 limbs
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int32_t l = limb_lo(r);
    base[i * p.HD] = (int8_t)l;
    r = (r - l) >> 8;
  }
}

// One head row hr (q heads [0, H), k heads [H, H + HKV), v heads after) of token `token` at position pos (clamped;
// an out-of-range position flags), one wave, lane l holding dims l + 64 e: the RoPE'd value (k / q) or the value
// itself (v). Flags |x| >= 2^31.
template <int HD>
__device__ __forceinline__ void rope_row(const RopeArgs& p, int token, int hr, int64_t pos, int lane,
                                         int64_t (&out)[HD / 64], bool& bad) {
  constexpr int E = HD / 64, HALF = HD / 2;
  const int64_t* x = p.y + (int64_t)token * p.ldy + (int64_t)hr * HD;
  const int64_t* cr = p.cos + pos * HALF;
  const int64_t* sr = p.sin + pos * HALF;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    const int64_t xv = x[d];
    bad |= (xv >= (1LL << 31)) || (xv <= -(1LL << 31));
    if (hr < p.H + p.HKV) {
      // _rope_full (src/bitexact/exact/segs.py:66-69): (x1 c - x2 s, x2 c + x1 s)
      const int dd = d < HALF ? d : d - HALF;
      const int64_t xp = x[d < HALF ? d + HALF : d - HALF];
      const int64_t c = cr[dd], s = sr[dd];
      out[e] = d < HALF ? add_wrap(mul_wrap(xv, c), -mul_wrap(xp, s)) : add_wrap(mul_wrap(xv, c), mul_wrap(xp, s));
    } else {
      out[e] = xv;
    }
  }
}

// A q head row's quantization (ops.quant(Pq, -(FR + FT)) over its HD values): the exponent shq (flags one above
// FK + 3 - FZ); q = rshc(out, shq + FR + FT).
template <int HD>
__device__ __forceinline__ int64_t rope_q_shift(const RopeArgs& p, const int64_t (&out)[HD / 64], bool& bad) {
  const int64_t eps = -(int64_t)(p.FR + p.FT);
  int64_t emax = kSegNegBig;
#pragma unroll
  for (int e = 0; e < HD / 64; ++e)
    if (out[e] != 0) emax = imax(emax, bitlen(out[e] < 0 ? -out[e] : out[e]) + eps);
  emax = wave_max64(emax);
  const int64_t shq = imax(emax - kSegQB, kSegNegBig);
  bad |= shq > p.FK + 3 - p.FZ;
  return shq;
}

// A k (plane 0) or v (plane 3) head row's cache values (|x| <= kLim3, else flagged), stored as limbs at the token's
// slot; also into p.k / p.v when given.
template <int HD>
__device__ __forceinline__ void rope_kv_store(const RopeArgs& p, int token, int hr, int lane, const int64_t (&out)[HD / 64],
                                              bool& bad) {
  const bool isk = hr < p.H + p.HKV;
  const int h = isk ? hr - p.H : hr - p.H - p.HKV;
#pragma unroll
  for (int e = 0; e < HD / 64; ++e) {
    const int64_t kv = rshc(out[e], isk ? p.FR + p.FT - p.FK : p.FR - p.FV);
    bad |= kv > kLim3 || kv < -kLim3;
    int64_t* dst = isk ? p.k : p.v;
    if (dst) dst[((int64_t)token * p.HKV + h) * HD + lane + 64 * e] = kv;
    store_limbs(p, token, h, isk ? 0 : 3, lane + 64 * e, kv);
  }
}

}  // namespace bx
