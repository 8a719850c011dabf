"""ctypes binding of libbitexact_hip.so (the C ABI declared in include/bitexact_hip.h).

Every kernel call goes through `call`: launches happen on torch's current stream of the tensors' device, a
BX_EINVAL return is re-raised as AssertionError (the reference's shape/contract asserts) and BX_EHIP as
RuntimeError. There is no fallback: without the built library or a GPU the import of a kernel module fails.
"""

import ctypes
import os
import threading

import torch

# BX_PHASES=1 loads the measurement build (the same kernels with phase timestamps; bench.py --phases)
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib",
                         "libbitexact_hip_phases.so" if os.environ.get("BX_PHASES") == "1" else "libbitexact_hip.so")
_lib = None
_lock = threading.Lock()

P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64

# name -> (restype, argtypes); the order and meaning follow include/bitexact_hip.h
SIGNATURES = {
    "bx_version": (ctypes.c_int, []),
    "bx_last_error": (ctypes.c_char_p, []),
    "bx_exact_linear": (ctypes.c_int, [P, I64, P, P, I64, I64, P, P, P, P, P, I32, P, I32, I32, I32, I32, I32, P,
                                       P, I64, P, I64, P]),
    "bx_exact_linear_planes": (ctypes.c_int, [P, I64, P, P, I64, I64, P, P, P, P, P, I32, P, I32, I32, I32, I32,
                                              I32, P, P, I64, P, P]),
    "bx_exact_linear_workspace": (I64, [I32, I32, I32]),
    "bx_exact_linear_scratch": (I64, [I32, I32, I32]),
    "bx_exact_linear_plan": (ctypes.c_int, [I32, I32, I32, P]),
    "bx_exact_linear_planes_plan": (ctypes.c_int, [I32, I32, I32, P]),
    "bx_exact_linear_planes_workspace": (I64, [I32, I32, I32]),
    "bx_exact_linear_reads_planes": (I32, [I32, I32, I32]),
    "bx_int8_gemm_plan": (ctypes.c_int, [I32, I32, I32, I32, P]),
    "bx_exact_linear_noalloc": (ctypes.c_int, [P, I64, P, P, I64, I64, P, P, P, P, P, I32, P, I32, I32, I32, I32,
                                               I32, P, P]),
    "bx_exact_linear_noalloc_limit": (I64, []),
    "bx_exact_wmm": (ctypes.c_int, [P, I64, P, I64, I64, P, I32, I32, I32, P, I64, P, I64, P]),
    "bx_decompose_rows": (ctypes.c_int, [P, I32, I32, P, P, P, P, P, P]),
    "bx_decompose_residual": (ctypes.c_int, [P, I32, I32, P, P, P, P, I32, P]),
    "bx_int8_gemm": (ctypes.c_int, [P, P, P, I32, I32, I32, P, I64, P]),
    "bx_int8_gemm_join": (ctypes.c_int, [P, P, P, I32, I32, I32, I32, P, I64, P]),
    "bx_int8_gemm_workspace": (I64, [I32, I32, I32, I32]),
    "bx_exact_attn_paged": (ctypes.c_int, [P, P, P, I64, P, I64, I64, I64, I32, P, I64, I32, P, P, I64, P, P, I32, I32,
                                           I32, I32, I32, P, I64, P]),
    "bx_exact_attn_paged_rope": (ctypes.c_int, [P, I64, P, I64, P, P, I32, I32, I32, I32, I32, I32, I32, P, P, I64, I64,
                                                I64, I32, P, I64, I32, P, P, I64, P, P, I32, I32, I32, P, P]),
    "bx_attn_rope_out_workspace": (I64, [I32]),
    "bx_attn_rope_out_scratch": (I64, [I32, I32, I32]),
    "bx_exact_attn_paged_rope_out": (ctypes.c_int, [P, I64, P, I64, P, P, I32, I32, I32, I32, I32, I32, I32, P, P, I64,
                                                    I64, I64, I32, P, I64, I32, P, P, I64, P, I64, P, I32, I32, I32,
                                                    P, P, I64, P, I64, P]),
    "bx_exact_attn_paged_rope_out_planes": (ctypes.c_int, [P, I64, P, I64, P, P, I32, I32, I32, I32, I32, I32, I32, P,
                                                           P, I64, I64, I64, I32, P, I64, I32, P, P, I64, P, I64, P,
                                                           P, I32, I32, I32, P, P, I64, P, I64, P]),
    "bx_attn_paged_workspace": (I64, [I32, I32, I32, I32]),
    "bx_exact_attn_prefill": (ctypes.c_int, [P, I64, I64, P, I64, P, I64, I64, P, I64, I64, P, I64, I64, I32, P, I64,
                                             P, P, I32, I32, I32, P, I64, P]),
    "bx_attn_prefill_scratch": (I64, [I32, I32, I32]),
    "bx_kv_store": (ctypes.c_int, [P, I64, I64, I64, I32, P, P, I64, I64, P, I64, I64, I32, I32, I32, I32, P]),
    "bx_limb_bmm": (ctypes.c_int, [P, I32, I64, I64, I64, P, I32, I64, I64, I64, P, I64, I64, I64, I32, I32, I32, I32,
                                   I32, I32, P]),
    "bx_rmsnorm_quant": (ctypes.c_int, [P, I64, P, P, P, I64, P, I32, I32, I32, I32, P, P]),
    "bx_add_rmsnorm_quant": (ctypes.c_int, [P, I64, P, I64, P, P, P, I64, P, I32, I32, I32, I32, P, P]),
    "bx_add_rmsnorm_quant_planes": (ctypes.c_int, [P, I64, P, I64, P, P, P, I64, P, P, I32, I32, I32, I32, P, P]),
    "bx_embed_rmsnorm_quant": (ctypes.c_int, [P, P, P, I64, P, P, P, I64, P, I32, I32, I32, I32, P, P]),
    "bx_embed_rmsnorm_quant_planes": (ctypes.c_int, [P, P, P, I64, P, P, P, I64, P, P, I32, I32, I32, I32, P, P]),
    "bx_silu_quant": (ctypes.c_int, [P, I64, I32, P, I32, P, I64, P, I32, P, P]),
    "bx_silu_quant_ws": (ctypes.c_int, [P, I64, I32, P, I32, P, I64, P, P, I32, P, P, I64, P]),
    "bx_silu_quant_scratch": (I64, [I32, I32]),
    "bx_first_argmax_ws": (ctypes.c_int, [P, I64, I32, I32, P, P, I64, P]),
    "bx_first_argmax_scratch": (I64, [I32, I32]),
    "bx_first_argmax": (ctypes.c_int, [P, I64, I32, I32, P, P]),
    "bx_softmax_w": (ctypes.c_int, [P, I64, P, P, I32, I32, I32, P, I64, I32, P, I64, P, P]),
    "bx_attn_out": (ctypes.c_int, [P, I64, I64, P, I64, I32, I32, I32, I32, I32, I32, I32, P, I64, P, P]),
    "bx_int8_attn_paged": (ctypes.c_int, [P, P, I64, P, I64, I64, I64, I32, P, I64, I32, P, I32, P, P, I32, I32, I32,
                                          I32, I32, P, I64, P]),
    "bx_exact_epilogue": (ctypes.c_int, [P, I64, I64, I32, P, I64, P, I64, I32, P, P, I32, P, P, P, I32, I32, P, I64,
                                         I32, I32, P, P]),
    "bx_rope_qgroup": (ctypes.c_int, [P, I64, P, I64, I64, P, P, I32, I32, I32, I32, I32, I32, I32, I32, I32, I32,
                                      I32, P, P, P, P, P, P]),
    "bx_rope_qgroup_store": (ctypes.c_int, [P, I64, P, I64, I64, P, P, I32, I32, I32, I32, I32, I32, I32, I32, I32,
                                            I32, I32, P, P, P, P, P, I64, I64, I64, P, I32, P, P]),
    "bx_int8_quant_rows": (ctypes.c_int, [P, I64, I32, I32, I32, I32, P, P, P, P, P, P]),
    "bx_int8_post": (ctypes.c_int, [P, I64, P, I32, P, P, I32, P, I64, I32, I32, P, P]),
    "bx_int_elementwise": (ctypes.c_int, [I32, I32, P, P, P, I32, P, I32, I64, I64, P, I64, I64, I64, P, P]),
    "bx_int_rowop": (ctypes.c_int, [I32, I32, P, P, P, I64, I64, I64, P, P, P, P, P, I64, P, P, P]),
    "bx_stream_read": (ctypes.c_int, [P, I64, I32, I32, P, P]),
    "bx_mfma_rate": (ctypes.c_int, [I32, I32, I32, I32, P, P]),
    "bx_decode_advance": (ctypes.c_int, [P, P, P, P, P, I64, I32, P, I32, I32, P]),
    "bx_phases_linear": (ctypes.c_int, [P]),
    "bx_phases_attn": (ctypes.c_int, [P]),
    "bx_phases_rows": (ctypes.c_int, [P]),
}


def lib():
    """The loaded library; raises if it was not built (python bitexact-llm_amd/build.py)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(_LIB_PATH):
                    raise ImportError(f"{_LIB_PATH} is missing: build it with `python bitexact-llm_amd/build.py`")
                L = ctypes.CDLL(_LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    f = getattr(L, name)
                    f.restype = res
                    f.argtypes = args
                _lib = L
    return _lib


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc == 0:
        return
    msg = lib().bx_last_error().decode(errors="replace")
    if rc == -1:
        raise AssertionError(f"{name}: {msg}")
    raise RuntimeError(f"{name} failed ({rc}): {msg}")


def require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise AssertionError("bitexact HIP kernels take device tensors only (no CPU path)")


# ---- per (device, stream) buffers: the split-K workspace (zero-filled; every call leaves it zeroed) and a
# scratch buffer (no contents kept between calls) ----
_ws = {}


def _buffer(kind, dev, nbytes):
    if nbytes <= 0:
        return None, 0
    key = (kind, dev.index, torch.cuda.current_stream(dev).cuda_stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = (torch.zeros if kind == "ws" else torch.empty)(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _ws[key] = buf
    return buf, buf.numel()


def workspace(dev, nbytes):
    return _buffer("ws", dev, nbytes)


def scratch(dev, nbytes):
    return _buffer("tmp", dev, nbytes)
