"""PyTorch operator registration of the HIP kernels: torch.ops.bitexact_hip.*.

Every kernel-calling function of the package is defined here as a `bitexact_hip::<name>` operator with a
schema (mutated arguments marked `(a!)`), a CUDA implementation (the ctypes call into libbitexact_hip.so) and a
fake implementation (output shapes and dtypes only), so torch.compile traces through the package without a graph
break and FakeTensor / meta propagation works. The package's Python functions route through the operator while
torch.compile is tracing and call the implementation directly otherwise (no dispatcher cost per launch in eager
code and in captured HIP graphs).
"""

import torch

NS = "bitexact_hip"
_LIB = torch.library.Library(NS, "DEF")


def op(schema, fake):
    """Decorator: registers `impl` as bitexact_hip::<name> (CUDA) with `fake` as its fake / meta kernel and
    returns a function that calls the operator under torch.compile and `impl` directly otherwise."""
    name = schema.split("(", 1)[0]

    def deco(impl):
        _LIB.define(schema)
        _LIB.impl(name, impl, "CUDA")
        torch.library.register_fake(f"{NS}::{name}", fake, lib=_LIB)
        packet = getattr(torch.ops.bitexact_hip, name)

        def route(*args, **kwargs):
            if torch.compiler.is_compiling():
                return packet(*args, **kwargs)
            return impl(*args, **kwargs)

        route.__name__ = name
        route.__doc__ = impl.__doc__
        route.op = packet
        route.impl = impl
        return route

    return deco


def empty(shape, dtype, like):
    return torch.empty(shape, dtype=dtype, device=like.device)
