"""bitexact (MI355X): the reference's integer linear / attention operator surface, backed by hand-written
HIP kernels for gfx950 through the C ABI in include/bitexact_hip.h.

Modules mirror the reference's (src/bitexact/...):
  bitexact.exact.consts       decompose (bf16 -> 3 int8 limbs + sparse residual, on the device), tables
  bitexact.exact.wmm          wmm_hip: the exact dense product T = q W^T
  bitexact.exact.model        Lin (gemm="hip"): constants-dict linear with the fused exact epilogue
  bitexact.vllm_plugin.exact_gemm  FusedLin: the plugin's exact linear call
  bitexact.int8.gemm_skinny   int_mm / int_mm_join: int8-mode GEMM
"""

__version__ = "0.1.0"
