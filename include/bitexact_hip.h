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

/* Replaces FusedLin.__call__ (src/bitexact/vllm_plugin/exact_gemm.py:509-541) and
 * segs.lin_y(*Lin(q), sh, checked) (src/bitexact/exact/segs.py:25-32, src/bitexact/exact/model.py:253-262):
 * y int64 [M, N] = round((q W^T 2^d + B) 2^(sh + g - d + FR)) with B = sum_j q[m, col[n,j]] val[n,j];
 * when `checked`, sets flag[0] = 1 where wmm.epilogue(checked=True) would (src/bitexact/exact/wmm.py:132-150).
 * Requires K % 16 == 0, ldq % 4 == 0, ld_row % 16 == 0, 16-byte aligned q and limbs. */
int bx_exact_linear(const int32_t* q, int64_t ldq, const int64_t* sh, const int8_t* limbs, int64_t ld_plane,
                    int64_t ld_row, const int64_t* d, const int64_t* g, const int32_t* ell_cnt,
                    const int32_t* ell_col, const int64_t* ell_val, int32_t R, int64_t* y, int32_t M, int32_t N,
                    int32_t K, int32_t FR, int32_t checked, int32_t* flag, void* ws, int64_t ws_bytes, void* tmp,
                    int64_t tmp_bytes, bx_stream_t stream);
int64_t bx_exact_linear_workspace(int32_t M, int32_t N, int32_t K);
int64_t bx_exact_linear_scratch(int32_t M, int32_t N, int32_t K);

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

/* Replaces gemm_skinny.int_mm (src/bitexact/int8/gemm_skinny.py:188-205) and torch._int_mm:
 * c int32 [R, N] = a int8 [R, K] @ w int8 [N, K]^T (exact while K * 127 * 128 < 2^31).
 * Requires K % 16 == 0 and 16-byte aligned a, w. */
int bx_int8_gemm(const int8_t* a, const int8_t* w, int32_t* c, int32_t R, int32_t N, int32_t K, void* ws,
                 int64_t ws_bytes, bx_stream_t stream);
/* int_mm followed by intops.join_limbs (src/bitexact/intops.py:82-87, src/bitexact/int8/segs.py:338):
 * y int64 [M, N] = sum_{i < nl} (a[i M:(i+1) M] @ w^T) 2^(8 i); a holds nl limb row blocks of M rows. */
int bx_int8_gemm_join(const int8_t* a, const int8_t* w, int64_t* y, int32_t M, int32_t N, int32_t K, int32_t nl,
                      void* ws, int64_t ws_bytes, bx_stream_t stream);
int64_t bx_int8_gemm_workspace(int32_t M, int32_t N, int32_t K, int32_t nl); /* raw int_mm: M = R, nl = 1 */

#ifdef __cplusplus
}
#endif

#endif /* BITEXACT_HIP_H */
