/* bitexact_hip.h -- C ABI of the MI355X (gfx950) integer linear and attention kernels.
 *
 * Every entry point takes plain device pointers, element strides and sizes, launches on `stream` (0 = the
 * null stream) and returns BX_OK or a negative code; bx_last_error() then names the violated contract.
 * BX_EINVAL is an argument/shape contract violation (the Python layer re-raises it as AssertionError, as the
 * reference's `assert`s do). Numeric bound violations never fail a call: they set the caller's int32 flag
 * (flag[0] = 1, never cleared), the reference's sticky device flag (src/bitexact/vllm_plugin/exact_gemm.py:110-118).
 * No call synchronizes the host with the device and no call allocates device memory. Temporary buffers are
 * the caller's: `ws` (split-K partial sums; size from the matching *_workspace function; zero-filled once by
 * the caller before its first use and left zero-filled by every call) and, for the exact linear, `tmp`
 * (scratch for the int8 limb planes of q; size from bx_exact_linear_scratch; no initial contents needed).
 * Calls that share one workspace or scratch buffer must not overlap in time (use one pair per stream).
 *
 * Layouts (row-major, k contiguous unless a stride says otherwise):
 *   q       int32 [M, ldq]            exact-mode activations, |q| <= 2^22
 *   limbs   int8  [3][N][ld_row]      plane stride ld_plane: the 3 signed base-256 digits of the dense weight
 *   d, g    int64 [N]                 residual grid offset and row grid exponent of each output row
 *   ELL     cnt int32 [N], col int32 [N, R], val int64 [N, R]   sparse residual, R entries per row max
 */
#ifndef BITEXACT_HIP_H
#define BITEXACT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* bx_stream_t; /* hipStream_t */

#define BX_OK 0
#define BX_EINVAL (-1)
#define BX_EHIP (-2)

const char* bx_last_error(void);
int bx_version(void);

/* ---- exact mode linear ---- */

/* Replaces FusedLin.__call__ (src/bitexact/vllm_plugin/exact_gemm.py:284-316) and
 * segs.lin_y(*Lin(q), sh, checked) (src/bitexact/exact/segs.py:25-32, src/bitexact/exact/model.py:61-70):
 * y int64 [M, N] = round((q W^T 2^d + B) 2^(sh + g - d + FR)) with B = sum_j q[m, col[n,j]] val[n,j];
 * when `checked`, sets flag[0] = 1 where wmm.epilogue(checked=True) would (src/bitexact/exact/wmm.py:132-150).
 * A corrupt residual list (a column outside [0, K) or a count outside [0, R]) also sets flag[0] = 1, checked or
 * not, whenever `flag` is given; a bad column reads q[m][0] and a bad count drops the row's list instead of
 * reading outside q. The Python layer validates the ELL arrays once when weights are loaded
 * (bitexact.exact.model.validate_ell).
 * Requires K % 16 == 0, ldq % 4 == 0, ld_row % 16 == 0, 16-byte aligned q and limbs. */
int bx_exact_linear(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs, int64_t ld_plane,
                    int64_t ld_row, const int64_t* d, const int64_t* g, const int32_t* ell_cnt,
                    const int32_t* ell_col, const int64_t* ell_val, int32_t R, int64_t* y, int32_t M, int32_t N,
                    int32_t K, int32_t FR, int32_t checked, int32_t* flag, void* ws, int64_t ws_bytes, void* tmp,
                    int64_t tmp_bytes, bx_stream_t stream);
/* bx_exact_linear with q's int8 limb planes supplied by the caller (q_planes int8 [3][M][K], limb i of q[m][k] at
 * i M K + m K + k, as bx_add_rmsnorm_quant_planes writes them), so no limb-split launch and no scratch. q is still
 * read (residual terms and the row-vector decode path). Same rule and arguments otherwise. Replaces the same
 * reference calls as bx_exact_linear; the reference splits q into limb planes inside its GEMM kernels
 * (src/bitexact/exact/wmm.py:79-121), so this entry has no separate reference counterpart. */
int bx_exact_linear_planes(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs, int64_t ld_plane,
                           int64_t ld_row, const int64_t* d, const int64_t* g, const int32_t* ell_cnt,
                           const int32_t* ell_col, const int64_t* ell_val, int32_t R, int64_t* y, int32_t M,
                           int32_t N, int32_t K, int32_t FR, int32_t checked, int32_t* flag, void* ws,
                           int64_t ws_bytes, const int8_t* q_planes, bx_stream_t stream);
int64_t bx_exact_linear_workspace(int32_t M, int32_t N, int32_t K);
int64_t bx_exact_linear_scratch(int32_t M, int32_t N, int32_t K);
/* Planner queries for bx_exact_linear_planes, which may take another kernel than bx_exact_linear at the same shape
 * (q's limb planes at hand make a plane-reading kernel cheaper): its workspace size, and whether it reads the
 * planes at all (1) or streams q itself (0), so a caller knows when producing the planes pays. No reference
 * counterpart (see bx_exact_linear_planes). */
int64_t bx_exact_linear_planes_workspace(int32_t M, int32_t N, int32_t K);
int32_t bx_exact_linear_reads_planes(int32_t M, int32_t N, int32_t K);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): bx_exact_linear with its split-K workspace and limb-plane
 * scratch taken from a static device array of bx_exact_linear_noalloc_limit() bytes (32 MiB: 8 MiB workspace,
 * 24 MiB scratch) that each GPU holds until the process ends. Shapes whose plan needs more fail with BX_EINVAL.
 * Allocates nothing. Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU (two
 * streams, two threads) race and give wrong results. Same rule, arguments and flag as bx_exact_linear. */
int bx_exact_linear_noalloc(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs, int64_t ld_plane,
                            int64_t ld_row, const int64_t* d, const int64_t* g, const int32_t* ell_cnt,
                            const int32_t* ell_col, const int64_t* ell_val, int32_t R, int64_t* y, int32_t M,
                            int32_t N, int32_t K, int32_t FR, int32_t checked, int32_t* flag, bx_stream_t stream);
int64_t bx_exact_linear_noalloc_limit(void);
/* Introspection, no reference counterpart (the reference picks Triton configs per shape from static tables,
 * src/bitexact/vllm_plugin/exact_gemm.py:205-226): which kernel bx_exact_linear runs for (M, N, K).
 * out int32 [4] = {kernel: 1 gemv, 2 wide, 3 tile, 5 stream; tile config: 0 128x128, 1 64x128, 2 64x32, 3 64x64 int8 decode,
 * 4 64x64 exact, -1 none; K splits; blocks per split}. Tests use it to show every configuration is reached. */
int bx_exact_linear_plan(int32_t M, int32_t N, int32_t K, int32_t* out);
/* The same for bx_exact_linear_planes. */
int bx_exact_linear_planes_plan(int32_t M, int32_t N, int32_t K, int32_t* out);

/* Replaces wmm_triton / wmm_cublas / wmm_cpu (src/bitexact/exact/wmm.py:79-121): the exact dense product
 * T int64 [M, N] = q W^T (one slice of the reference's [split, M, N] partials). */
int bx_exact_wmm(const int32_t* q, int64_t ldq, const int8_t* limbs, int64_t ld_plane, int64_t ld_row,
                 int64_t* T, int32_t M, int32_t N, int32_t K, void* ws, int64_t ws_bytes, void* tmp,
                 int64_t tmp_bytes, bx_stream_t stream);

/* Replaces consts.decompose (src/bitexact/exact/consts.py:67-107) on the device, pass 1 of 2: bf16 raw bits
 * w [N, K] -> limbs int8 [3, N, K], g, d int64 [N], cnt int32 [N] (residual entries per row). Sets err[0] = 1
 * for inf/nan weights or a residual grid finer than 30 bits (the reference's asserts). */
int bx_decompose_rows(const uint16_t* w, int32_t N, int32_t K, int8_t* limbs, int64_t* g, int64_t* d,
                      int32_t* cnt, int32_t* err, bx_stream_t stream);
/* Pass 2: the residual entries in ELL form, col int32 [N, R] / val int64 [N, R] (k ascending per row,
 * zero padded), with R >= max(cnt). */
int bx_decompose_residual(const uint16_t* w, int32_t N, int32_t K, const int64_t* g, const int64_t* d,
                          int32_t* ell_col, int64_t* ell_val, int32_t R, bx_stream_t stream);

/* ---- int8 mode GEMM ---- */

/* Replaces gemm_skinny.int_mm (src/bitexact/int8/gemm_skinny.py:80-97) and torch._int_mm:
 * c int32 [R, N] = a int8 [R, K] @ w int8 [N, K]^T (exact while K * 127 * 128 < 2^31).
 * Requires K % 16 == 0 and 16-byte aligned a, w. */
int bx_int8_gemm(const int8_t* a, const int8_t* w, int32_t* c, int32_t R, int32_t N, int32_t K, void* ws,
                 int64_t ws_bytes, bx_stream_t stream);
/* int_mm followed by intops.join_limbs (src/bitexact/intops.py:82-87, src/bitexact/int8/segs.py:126):
 * y int64 [M, N] = sum_{i < nl} (a[i M:(i+1) M] @ w^T) 2^(8 i); a holds nl limb row blocks of M rows. */
int bx_int8_gemm_join(const int8_t* a, const int8_t* w, int64_t* y, int32_t M, int32_t N, int32_t K, int32_t nl,
                      void* ws, int64_t ws_bytes, bx_stream_t stream);
/* Introspection, no reference counterpart: the int8 GEMM's kernel for M rows of nl limbs (nl = 0: raw int32 GEMM of M
 * stacked rows). out int32 [6] = {kernel: 1 gemv, 3 tile, 4 staged, 5 stream; tile config or -1; K splits; blocks per split;
 * gemv column groups; gemv row parts}. */
int bx_int8_gemm_plan(int32_t M, int32_t N, int32_t K, int32_t nl, int32_t* out);
int64_t bx_int8_gemm_workspace(int32_t M, int32_t N, int32_t K, int32_t nl); /* raw int_mm: M = R, nl = 1 */

/* ---- integer attention ---- */

/* Replaces tri_exact_attn.attend (src/bitexact/vllm_plugin/tri_exact_attn.py:138-165): paged exact attention for
 * M <= 4 queries per (row, KV head). q int32 [R, HKV, M, HD] contiguous, sh int64 [R, HKV, M], qpos int64
 * [R, M] (row stride sqpos_r; key s visible to query i iff s <= qpos[r, i]), cache int8 limb planes
 * [nb, HKV, bs, >= 6 HD] (element strides sc_nb, sc_h, sc_bs; K limbs at bytes [0, 3 HD), V at [3 HD, 6 HD)),
 * bt int32 block table (row stride sbt, nblk columns), rmap int64 [R] (block-table row of each q row),
 * lut int64 [2^14 + 1] (2^-f at 2^60), l2e = round(log2(e) / sqrt(HD / 64) 2^28). Outputs num int64
 * [R, HKV, M, HD], den int64 [R, HKV, M]. nsplit > 1 splits the keys over blocks (two launches) and needs ws. */
int bx_exact_attn_paged(const int32_t* q, const int64_t* sh, const int64_t* qpos, int64_t sqpos_r, const int8_t* cache,
                        int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt,
                        int32_t nblk, const int64_t* rmap, const int64_t* lut, int64_t l2e, int64_t* num, int64_t* den,
                        int32_t R, int32_t HKV, int32_t M, int32_t HD, int32_t nsplit, void* ws, int64_t ws_bytes,
                        bx_stream_t stream);

/* Replaces the decode step's exact_fuse.qkv + tri_exact_attn.attend pair (src/bitexact/vllm_plugin/exact_fuse.py:
 * 372-386, tri_exact_attn.py:138-165) when every token of the step belongs to its own sequence (decode): one launch
 * does the rope kernel's work (bx_rope_qgroup_store: RoPE of the q and k heads of y int64 [R, >= (H + 2 HKV) HD]
 * (row stride ldy) at pos int64 [R] (stride spos) with the cos / sin tables [npos, HD / 2], the per-head
 * quantization of q, the k / v limbs stored at slot int64 [R] of the cache, bound violations to err[0]) and then
 * the attention of bx_exact_attn_paged with M = H / HKV <= 4 queries per (token, KV head) at qpos = pos, over at
 * most 2048 keys per row, no key split. Outputs num int64 [R, HKV, M, HD], den int64 [R, HKV, M]; the grouped
 * queries are not written. FK and FZ must be the compiled formats (17, 26). */
int bx_exact_attn_paged_rope(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos, const int64_t* cos,
                             const int64_t* sin, int32_t npos, int32_t H, int32_t FR, int32_t FT, int32_t FK,
                             int32_t FV, int32_t FZ, const int64_t* slot, int8_t* cache, int64_t sc_nb, int64_t sc_h,
                             int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt, int32_t nblk,
                             const int64_t* rmap, const int64_t* lut, int64_t l2e, int64_t* num, int64_t* den,
                             int32_t R, int32_t HKV, int32_t HD, int32_t* err, bx_stream_t stream);

/* bx_exact_attn_paged_rope with the attention output stage fused as well (segs.attn_out, the reference's div_round +
 * regroup + quant after the attention: src/bitexact/exact/segs.py, exact/ops.py): instead of num / den it writes
 * q int32 [R, ldq >= H HD] and sh int64 [R], the quantized rows the wo linear reads, equal to bx_attn_out over the
 * num / den it replaces. ws: bx_attn_rope_out_workspace(R) bytes, zero-filled (left zero); tmp:
 * bx_attn_rope_out_scratch(R, H, HD) bytes of scratch. Each token's last block quantizes the row. */
int64_t bx_attn_rope_out_workspace(int32_t R);
int64_t bx_attn_rope_out_scratch(int32_t R, int32_t H, int32_t HD);
int bx_exact_attn_paged_rope_out(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos, const int64_t* cos,
                                 const int64_t* sin, int32_t npos, int32_t H, int32_t FR, int32_t FT, int32_t FK,
                                 int32_t FV, int32_t FZ, const int64_t* slot, int8_t* cache, int64_t sc_nb,
                                 int64_t sc_h, int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt, int32_t nblk,
                                 const int64_t* rmap, const int64_t* lut, int64_t l2e, int32_t* q, int64_t ldq,
                                 int64_t* sh, int32_t R, int32_t HKV, int32_t HD, int32_t* err, void* ws,
                                 int64_t ws_bytes, void* tmp, int64_t tmp_bytes, bx_stream_t stream);
/* bx_exact_attn_paged_rope_out that also writes q's signed int8 limb planes, planes int8 [3][R][H HD] (limb i of
 * q[n][c] at i R H HD + n H HD + c, the split the exact linear's activation planes use), so the wo linear that reads
 * q needs no split launch (the reference has no counterpart; it serves the same segs.attn_out call as the entry
 * above). */
int bx_exact_attn_paged_rope_out_planes(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spos,
                                        const int64_t* cos, const int64_t* sin, int32_t npos, int32_t H, int32_t FR,
                                        int32_t FT, int32_t FK, int32_t FV, int32_t FZ, const int64_t* slot,
                                        int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs,
                                        const int32_t* bt, int64_t sbt, int32_t nblk, const int64_t* rmap,
                                        const int64_t* lut, int64_t l2e, int32_t* q, int64_t ldq, int64_t* sh,
                                        int8_t* planes, int32_t R, int32_t HKV, int32_t HD, int32_t* err, void* ws,
                                        int64_t ws_bytes, void* tmp, int64_t tmp_bytes, bx_stream_t stream);
/* Workspace bytes of the paged attentions (exact and int8) for up to min(64, 4096 / T) key splits, T = R HKV
 * ceil(M / 4) query tiles; a call with more splits than the workspace holds is rejected. */
int64_t bx_attn_paged_workspace(int32_t R, int32_t HKV, int32_t M, int32_t HD);

/* Replaces tri_paged.attend (src/bitexact/vllm_plugin/tri_paged.py:363-430), the int8-mode paged attention: q int64
 * [R, HKV, M, HD] (within 3 limbs; any M, tiles of 4 queries), qpos [R, M] (row stride sqpos_r), the same limb-plane
 * cache and block table rows bt [R, *] as bx_exact_attn_paged, weight table ptab int32 (tri_paged.weight_table,
 * 2^17 + 1 entries): raw = q.K, mx = max over visible keys, z by int8.segs.score_rule, p = ptab[z - EXP_MIN 2^FA]
 * (0 below the table) -> num int64 [R, HKV, M, HD], den int64 [R, HKV, M, 1]. Workspace as bx_exact_attn_paged. */
int bx_int8_attn_paged(const int64_t* q, const int64_t* qpos, int64_t sqpos_r, const int8_t* cache, int64_t sc_nb,
                       int64_t sc_h, int64_t sc_bs, int32_t bs, const int32_t* bt, int64_t sbt, int32_t nblk,
                       const int32_t* ptab, int32_t ptab_len, int64_t* num, int64_t* den, int32_t R, int32_t HKV,
                       int32_t M, int32_t HD, int32_t nsplit, void* ws, int64_t ws_bytes, bx_stream_t stream);

/* Fused form of exact/model.py's attention (src/bitexact/exact/model.py:113-119: bmm(qg, K^T), segs.softmax,
 * bmm(p, V)): qg int32 [Z, gT, HD] (strides sq_z, sq_row), shg int64 [Z, gT] (ssh_z = gT), qpos int64 [Z, gT]
 * (strides), K / V int32 [Z, S, HD] (strides; the integer Cache layout), outputs num int64 [Z, gT, HD],
 * den int64 [Z, gT]. The score matrix is never materialized. qg, K and V rows must be 16-byte aligned (base and
 * strides multiples of 4 elements); K / V values are taken as their three signed base-256 limbs. tmp (16-byte
 * aligned, at least bx_attn_prefill_scratch(Z, S, HD) bytes, no contents kept; null: the register-staged form, no
 * scratch) receives K and V as int8 limb planes once per call, which the main kernel streams into LDS. */
int bx_exact_attn_prefill(const int32_t* qg, int64_t sq_z, int64_t sq_row, const int64_t* shg, int64_t ssh_z,
                          const int64_t* qpos, int64_t sqpos_z, int64_t sqpos_row, const int32_t* K, int64_t sk_z,
                          int64_t sk_s, const int32_t* V, int64_t sv_z, int64_t sv_s, int32_t S, const int64_t* lut,
                          int64_t l2e, int64_t* num, int64_t* den, int32_t Z, int32_t gT, int32_t HD, void* tmp,
                          int64_t tmp_bytes, bx_stream_t stream);
/* Scratch bytes of bx_exact_attn_prefill's limb-plane form (0: not available for these sizes; pass null). No
 * reference counterpart. */
int64_t bx_attn_prefill_scratch(int32_t Z, int32_t S, int32_t HD);

/* Replaces tri_paged.store (src/bitexact/vllm_plugin/tri_paged.py:311-335): K / V (int32 or int64 [N, HKV, HD] with
 * token / head strides) written as 3 int8 limb planes each at cache slots slot int64 [N]; slot < 0 is skipped.
 * Slots are not range-checked on the device: slot < nb bs is the caller's contract, as for the reference's
 * slot mapping. */
int bx_kv_store(int8_t* cache, int64_t sc_nb, int64_t sc_h, int64_t sc_bs, int32_t bs, const int64_t* slot,
                const void* k, int64_t skn, int64_t skh, const void* v, int64_t svn, int64_t svh, int32_t elem_bytes,
                int32_t N, int32_t HKV, int32_t HD, bx_stream_t stream);

/* Replaces bitexact.bmm.bmm (src/bitexact/bmm.py:78-102): exact int64 c [Z, M, N] = a [Z, M, K] @ b [Z, K, N] for
 * int32 / int64 operands (element sizes a_bytes / b_bytes) with arbitrary strides, each within na / nb limbs. */
int bx_limb_bmm(const void* a, int32_t a_bytes, int64_t saz, int64_t sam, int64_t sak, const void* b, int32_t b_bytes,
                int64_t sbz, int64_t sbk, int64_t sbn, int64_t* c, int64_t scz, int64_t scm, int64_t scn, int32_t Z,
                int32_t M, int32_t N, int32_t K, int32_t na, int32_t nb, bx_stream_t stream);

/* ---- row stages ---- */

/* Replaces segs.norm_quant (src/bitexact/exact/segs.py:59-63): RMSNorm of x int64 [M, D] at FR with gamma
 * (gm 2^ge per column), then per-row quantization at -FN: q int32 [M, D], sh int64 [M]; err[0] = 1 when
 * max |x| >= 2^40. D a power of two <= 4096. */
int bx_rmsnorm_quant(const int64_t* x, int64_t ldx, const int64_t* gm, const int64_t* ge, int32_t* q, int64_t ldq,
                     int64_t* sh, int32_t M, int32_t D, int32_t FR, int32_t FN, int32_t* err, bx_stream_t stream);

/* Replaces Segs.add_norm_y = segs.add_y + norm_q (src/bitexact/exact/segs.py:40-41, 175-178; exact_fuse.add_norm,
 * src/bitexact/vllm_plugin/exact_fuse.py:361-364): x += y in place (x, y int64 [M, D] at FR), then with gm non-null
 * bx_rmsnorm_quant's rule on the new x. gm null: the add and its bound check alone (the engine's last layer). */
int bx_add_rmsnorm_quant(int64_t* x, int64_t ldx, const int64_t* y, int64_t ldy, const int64_t* gm, const int64_t* ge,
                         int32_t* q, int64_t ldq, int64_t* sh, int32_t M, int32_t D, int32_t FR, int32_t FN, int32_t* err,
                         bx_stream_t stream);

/* bx_add_rmsnorm_quant (gm required) that also writes the new q's signed int8 limb planes (planes int8
 * [3][M][D], limb i of q[m][k] at i M D + m D + k) for bx_exact_linear_planes. D % 16 == 0. Replaces the same
 * reference stage (exact_fuse.add_norm, src/bitexact/vllm_plugin/exact_fuse.py:361-364). y null: no add, the
 * norm of x as it is (bx_rmsnorm_quant with the planes; x is not written), e.g. the final norm before lm_head
 * (segs.norm_quant, src/bitexact/exact/segs.py:59-63). */
int bx_add_rmsnorm_quant_planes(int64_t* x, int64_t ldx, const int64_t* y, int64_t ldy, const int64_t* gm,
                                const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh, int8_t* planes, int32_t M,
                                int32_t D, int32_t FR, int32_t FN, int32_t* err, bx_stream_t stream);

/* Replaces the model's `emb[ids].long()` + pre_norm (src/bitexact/exact/model.py:130-132; exact_fuse.embed_norm,
 * src/bitexact/vllm_plugin/exact_fuse.py:356-358): x[m] = emb[ids[m]] (emb int32 [V, D] at FR, widened to int64),
 * then bx_rmsnorm_quant's rule (skipped when gm is null). ids are not range-checked. */
int bx_embed_rmsnorm_quant(const int32_t* emb, const int64_t* ids, int64_t* x, int64_t ldx, const int64_t* gm,
                           const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh, int32_t M, int32_t D, int32_t FR,
                           int32_t FN, int32_t* err, bx_stream_t stream);
/* bx_embed_rmsnorm_quant (gm required) that also writes q's signed int8 limb planes (as
 * bx_add_rmsnorm_quant_planes, D % 16 == 0) for the first layer's bx_exact_linear_planes. Same reference stage. */
int bx_embed_rmsnorm_quant_planes(const int32_t* emb, const int64_t* ids, int64_t* x, int64_t ldx, const int64_t* gm,
                                  const int64_t* ge, int32_t* q, int64_t ldq, int64_t* sh, int8_t* planes, int32_t M,
                                  int32_t D, int32_t FR, int32_t FN, int32_t* err, bx_stream_t stream);

/* Replaces Segs.gu_silu_y = segs.silu_y + quant_silu (src/bitexact/exact/segs.py:120-128, 180-182) over
 * ops.silu_mul (src/bitexact/exact/ops.py:119-130): gu int64 [M, 2 ff] = [gate | up] at FR; q int32 [M, ff],
 * sh int64 [M] the row quantization of silu(gate) up at eps = -2 FR; err[0] = 1 where silu_mul's ok is false.
 * lut: the 2^-f table (exp2, 16385 entries at 2^60). ff <= 16384. */
int bx_silu_quant(const int64_t* gu, int64_t ldgu, int32_t ff, const int64_t* lut, int32_t FR, int32_t* q, int64_t ldq,
                  int64_t* sh, int32_t M, int32_t* err, bx_stream_t stream);

/* bx_silu_quant split over column chunks of about 1024 elements, for few rows (one block per row leaves most CUs
 * idle): one launch on `stream`; the chunks of a row exchange their maxima through the caller's workspace (tmp,
 * 8-byte aligned, at least bx_silu_quant_scratch(M, ff) bytes, zero-filled before its first use and left
 * zero-filled by every call; ff <= 524288). Same rule, outputs and flag as bx_silu_quant, the
 * reference stage it replaces (src/bitexact/exact/segs.py:120-128, 180-182). planes (optional, ff % 16 == 0): q's
 * signed int8 limb planes [3][M][ff] for bx_exact_linear_planes. */
int bx_silu_quant_ws(const int64_t* gu, int64_t ldgu, int32_t ff, const int64_t* lut, int32_t FR, int32_t* q,
                     int64_t ldq, int64_t* sh, int8_t* planes, int32_t M, int32_t* err, void* tmp, int64_t tmp_bytes,
                     bx_stream_t stream);
int64_t bx_silu_quant_scratch(int32_t M, int32_t ff);

/* Replaces intops.first_argmax (src/bitexact/intops.py:55-59), the greedy token of tri_logits
 * (src/bitexact/vllm_plugin/tri_logits.py:1-20): out[m] = the first index of the maximum of row m of v int64 [M, N]. */
int bx_first_argmax(const int64_t* v, int64_t ldv, int32_t M, int32_t N, int64_t* out, bx_stream_t stream);

/* bx_first_argmax split over column chunks of about 8192 for few rows: two launches on `stream`, with each chunk's
 * (maximum, first index) in the caller's scratch (tmp, 8-byte aligned, at least bx_first_argmax_scratch(M, N)
 * bytes; no contents kept). Same result as bx_first_argmax, the reference rule it replaces
 * (src/bitexact/intops.py:55-59). */
int bx_first_argmax_ws(const int64_t* v, int64_t ldv, int32_t M, int32_t N, int64_t* out, void* tmp, int64_t tmp_bytes,
                       bx_stream_t stream);
int64_t bx_first_argmax_scratch(int32_t M, int32_t N);

/* Replaces segs.softmax (src/bitexact/exact/segs.py:102-105, ops.softmax_w): weights p int32 [rows, S] at fp bits of
 * the scores raw int64 [rows, S] (key s visible iff s <= qpos[row]; hidden keys weigh 0) and den int64 [rows]. */
int bx_softmax_w(const int64_t* raw, int64_t ldr, const int64_t* qpos, const int64_t* sh, int32_t rows, int32_t S,
                 int32_t kbits, const int64_t* lut, int64_t l2e, int32_t fp, int32_t* p, int64_t ldp, int64_t* den,
                 bx_stream_t stream);

/* Replaces Segs.attn_out (src/bitexact/exact/segs.py:108-113, 187-188): o = div_round(num, FR - FV, den) regrouped to
 * rows of H HD values (row o, head hh reads group (o / T) HKV + hh / g, query (hh % g) T + o % T), then
 * quantized per row at -FR: q int32 [rows, H HD], sh int64 [rows]. */
int bx_attn_out(const int64_t* num, int64_t sn_group, int64_t sn_query, const int64_t* den, int64_t sd_group,
                int32_t rows, int32_t T, int32_t HKV, int32_t g, int32_t HD, int32_t FR, int32_t FV, int32_t* q,
                int64_t ldq, int64_t* sh, bx_stream_t stream);

/* ---- element-wise segments ---- */

/* Replaces Segs.qkv_y = segs.rope_y + segs.q_group (src/bitexact/exact/segs.py:78-99, 170-173): y int64 [B T, ldy]
 * (q heads, k heads, v heads at FR), positions pos [B, T] (element strides spb, spt), integer cos / sin tables
 * [npos, HD / 2] at FT -> qg int32 [B HKV, g T, HD] (q quantized per (token, head) at -(FR + FT), grouped by KV
 * head), shg int64 [B HKV, g T], k int64 [B, T, HKV, HD] at FK, v at FV. err[0] = 1 where q_group's check fails
 * (|y| >= 2^31, |k| or |v| > 8355711, q exponent > FK + 3 - FZ) or a position lies outside the tables. */
int bx_rope_qgroup(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spb, int64_t spt, const int64_t* cos,
                   const int64_t* sin, int32_t npos, int32_t B, int32_t T, int32_t H, int32_t HKV, int32_t HD,
                   int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ, int32_t* qg, int64_t* shg, int64_t* k,
                   int64_t* v, int32_t* err, bx_stream_t stream);

/* Replaces exact_fuse._qkv_kernel with STORE (src/bitexact/vllm_plugin/exact_fuse.py:179-236, called by
 * exact_fuse.qkv, 372-386): bx_rope_qgroup, and the K / V values stored as three int8 limb planes into the paged
 * cache (tri_paged.store's layout, src/bitexact/vllm_plugin/tri_paged.py:311-335) at slot[token] (cache int8
 * [nb][HKV][bs][8 HD] with byte strides sc_nb, sc_h, sc_bs; tokens with slot < 0 are not stored). k / v may be
 * null (then only the cache receives them). Slots are not range-checked (slot < nb bs is the caller's contract). */
int bx_rope_qgroup_store(const int64_t* y, int64_t ldy, const int64_t* pos, int64_t spb, int64_t spt,
                         const int64_t* cos, const int64_t* sin, int32_t npos, int32_t B, int32_t T, int32_t H,
                         int32_t HKV, int32_t HD, int32_t FR, int32_t FT, int32_t FK, int32_t FV, int32_t FZ,
                         int32_t* qg, int64_t* shg, int64_t* k, int64_t* v, int8_t* cache, int64_t sc_nb,
                         int64_t sc_h, int64_t sc_bs, const int64_t* slot, int32_t bs, int32_t* err,
                         bx_stream_t stream);

/* Replaces wmm.epilogue and segs.lin_y (src/bitexact/exact/wmm.py:132-150, src/bitexact/exact/segs.py:25-32): T int64
 * [nsplit, M, N] split partials (slice stride sts, row stride ldt) summed, residual B int64 [M, ldb] or (B null)
 * the ELL gather sum_j q[m, ell_col[n, j]] ell_val[n, j] (R entries per column), then y = round((T 2^d + B)
 * 2^(sh + g - d + FR)) once; with `checked`, flag[0] = 1 where wmm.epilogue(checked=True) flags. */
int bx_exact_epilogue(const int64_t* T, int64_t ldt, int64_t sts, int32_t nsplit, const int64_t* B, int64_t ldb,
                      const int32_t* q, int64_t ldq, int32_t K, const int32_t* ell_col, const int64_t* ell_val,
                      int32_t R, const int64_t* d, const int64_t* g, const int64_t* sh, int32_t FR, int32_t checked,
                      int64_t* y, int64_t ldy, int32_t M, int32_t N, int32_t* flag, bx_stream_t stream);

/* Replaces int8 ops.quant_rows + intops.stack_limbs (src/bitexact/int8/ops.py:24-35, src/bitexact/intops.py:73-79)
 * and, with mant / e given, segs.pre_plain's row scale norm24(as_, sh - FR) (src/bitexact/int8/segs.py:56-59):
 * z int64 [M, ldz] -> a int8 [nl M, K] (limb i of row m at row i M + m, no padding rows), as_, sh [M]. */
int bx_int8_quant_rows(const int64_t* z, int64_t ldz, int32_t M, int32_t K, int32_t nl, int32_t FR, int8_t* a,
                       int64_t* as_, int64_t* sh, int64_t* mant, int64_t* e, bx_stream_t stream);

/* Replaces int8 segs.post (src/bitexact/int8/segs.py:62-67) on the joined products acc int64 [M, ldacc]:
 * y = rsh(rsh(acc m_c, fmsh) mant_r, 24 - FR - e_r); flag[0] = 1 when some |rsh(acc m_c, fmsh)| >= 2^38. */
int bx_int8_post(const int64_t* acc, int64_t ldacc, const int64_t* m, int32_t fmsh, const int64_t* mant,
                 const int64_t* e, int32_t FR, int64_t* y, int64_t ldy, int32_t M, int32_t N, int32_t* flag,
                 bx_stream_t stream);

/* ---- the reference's Python helper rules, element-wise and per row ---- */

/* Replaces the element-wise rules of intops (src/bitexact/intops.py:14-87: bitlen, rsh, fdiv, rdiv, isqrt,
 * split_limbs, stack_limbs, join_limbs), exact ops (src/bitexact/exact/ops.py:25-130: rshc, div_round, combine,
 * shift_round_hl, exp2neg_lut, silu_mul), int8 ops (src/bitexact/int8/ops.py:38-108: bitlen32, rdiv32, norm24,
 * exp_of, silu) and the RoPE / division / bound steps of exact segs (src/bitexact/exact/segs.py:49-113) and int8
 * segs (src/bitexact/int8/segs.py:70-118). `op` selects the rule (csrc/bx_elem.hip ElemOp, 1..28); operand j
 * (j < nin <= 5) is element (r, c) of the [rows, inner] output grid at ptrs[j] + r desc[4j] + c desc[4j+1] with
 * desc[4j+3] bytes per element (1, 2, 4, 8; signed), or the constant desc[4j+2] when ptrs[j] is null. Outputs are
 * contiguous [rows, inner] with ob0 / ob1 bytes per element; lut is the rule's table (lut_len entries); iarg /
 * iarg2 its integer parameters; rule violations (a zero divisor, a table index past the end, a failed bound) set
 * flag[0] = 1 when flag is given. */
int bx_int_elementwise(int32_t op, int32_t nin, const void* const* ptrs, const int64_t* desc, void* out0, int32_t ob0,
                       void* out1, int32_t ob1, int64_t rows, int64_t inner, const int64_t* lut, int64_t lut_len,
                       int64_t iarg, int64_t iarg2, int32_t* flag, bx_stream_t stream);

/* Replaces the per-row rules exact ops.quant / ops.rms / ops.softmax_w (src/bitexact/exact/ops.py:82-143) and int8
 * ops.rms / ops.quant_rows (src/bitexact/int8/ops.py:24-35, 76-84), int8 segs.pre_norm / segs.softmax
 * (src/bitexact/int8/segs.py:47-52, 90-99) and a row max |x|, one block per row of x int64 [rows, ldx] (D
 * columns). Operands as for bx_int_elementwise over the [rows, D] grid (nin <= 3); iargs[6] the rule's integer
 * parameters; outputs out0..out3 per rule (csrc/bx_elem.hip RowOp). */
int bx_int_rowop(int32_t op, int32_t nin, const void* const* ptrs, const int64_t* desc, const int64_t* x, int64_t ldx,
                 int64_t rows, int64_t D, void* out0, void* out1, void* out2, void* out3, const int64_t* lut,
                 int64_t lut_len, const int64_t* iargs, int32_t* flag, bx_stream_t stream);

/* A greedy decode step's input update (the caller's loop in the reference: src/bitexact/vllm_plugin/exact_run.py
 * decode loop / vLLM's scheduler), in one launch: ids[n] = next[n], pos[n] += 1, slot[n] = bt[rmap[n], pos[n] / bs]
 * bs + pos[n] % bs, for N sequences (int64 next / ids / pos / slot / rmap [N], int32 bt row stride sbt, nblk
 * columns; the new position must stay inside the table). */
int bx_decode_advance(const int64_t* next, int64_t* ids, int64_t* pos, int64_t* slot, const int32_t* bt, int64_t sbt,
                      int32_t nblk, const int64_t* rmap, int32_t bs, int32_t N, bx_stream_t stream);

/* No counterpart in the reference: a measurement probe for the decode GEMMs' roofline. Streams `bytes` from src
 * (16-byte nontemporal loads, grid-stride over blocks x threads) and discards them: the practical read ceiling of
 * one launch at that size. sink: an int32 [1] device word (practically never written). */
int bx_stream_read(const void* src, int64_t bytes, int32_t blocks, int32_t threads, int32_t* sink, bx_stream_t stream);

/* No counterpart in the reference: a measurement probe for the prefill kernels' roofline. Each of blocks x threads
 * lanes' waves issues iters x 4 independent int8 MFMAs from registers (shape 0: v_mfma_i32_32x32x32_i8, 65536 ops;
 * 1: v_mfma_i32_16x16x64_i8, 32768 ops; 2 and 3: the same with fresh pseudo-random operand bytes every iteration;
 * 4 and 5: the instructions of 2 and 3 with the operands held constant)
 * with no memory traffic: the dense int8 rate the matrix cores sustain.
 * sink: an int32 [1] device word (practically never written). */
int bx_mfma_rate(int32_t shape, int32_t iters, int32_t blocks, int32_t threads, int32_t* sink, bx_stream_t stream);

/* No counterpart in the reference: phase timers of the measurement build (libbitexact_hip_phases.so, compiled
 * with -DBX_PHASES). Each copies its source file's table, uint64 [4 kernel slots][1024 blocks][8 marks] of the
 * 100 MHz real-time counter as the kernels last wrote them, into host memory: linear (slot 0 the exact prefill
 * tile: start, context built, first stage landed, loop end, gathers landed, end; slot 1 the stream kernel:
 * start, chunk 1, loop end, end), attn (slot 0 the split decode attention: start, scores, maxima exchanged,
 * weights and p V, end; slot 1 the one-block decode attention: start, prologue, K sweep, V requested, V sweep,
 * end), rows (slot 0 the norm: start, row loaded, divisor, quotients, end). The product library returns
 * BX_EINVAL. */
int bx_phases_linear(uint64_t* host);
int bx_phases_attn(uint64_t* host);
int bx_phases_rows(uint64_t* host);

#ifdef __cplusplus
}
#endif

#endif /* BITEXACT_HIP_H */
