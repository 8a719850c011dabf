"""bench.py -- the hot path on one MI355X: int8-mode decode GEMMs (HBM GB/s) and exact-mode prefill limb GEMMs
(effective limb-op TOPS against the dense int8 MFMA peak).

One step = one pass over BASELINE config 2's decode GEMMs as the reference's int8 MLP issues them: batch M in
{1, 8, 64} x {gate|up fused (wgu = cat(gate, up): K=2048, N=2 x 8192), down K=8192 N=2048}, int8 weights uniform
in [-127, 127], activations N(0,1) quantized per row into 2 int8 limbs, int64 joined output
(bitexact.int8.gemm_skinny.int_mm_join). Separate gate / up GEMMs are timed too (per_gemm). Weights rotate over
>= 1 GiB of copies per shape (4x the 256 MB MALL) so every launch reads them from HBM. The steps are captured
in a HIP graph and timed with HIP events on the launch stream.
value = sum of algorithmic bytes (N K + 2 M K + 8 M N per GEMM) / time, in GB/s.

Also measured (config 3): exact-mode prefill, M = 2048 over every Llama-3.2-1B linear, reported as effective
TOPS = 9 x 2 M N K / time and as a fraction of the 5.0 POP/s dense int8 peak. And a CPU baseline: the oracle's
float64 restatement of the same GEMMs (oracle/bxref.py imm, the reference's CPU path) on a bounded sample.

Config 4 (integer attention, B=4, H=32, HKV=8, HD=64, causal, S=2048) is measured too: the paged decode step
(HBM bytes B HKV S 6 HD of limb planes per call, caches rotated over >= 1 GiB) and the fused prefill attention
(effective limb-op TOPS, 2 x 9 x 2 HD B H T(T+1)/2 per call).

Config 5 (random-init Llama-3.2-1B in exact mode, greedy decode at batch 32, context 1024, paged KV block 16) is
measured end to end through the decode engine: tokens/s over graph-replayed steps, and the check that a
sequence's logits hash does not depend on the batch size (1, 8, 32).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-prefill] [--no-attn] [--no-engine] [--no-cpu]
       python bench.py --eager ...        launches without graphs (for counter collection)
       python bench.py --copy-calibrate   only a 1 GiB device copy, 20 times (HBM counter scale)
"""

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "bitexact-llm_amd"))

HBM_PEAK_GBS = 8000.0
# HBM bytes per decode launch (average over the step's 6 GEMMs) from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# runs of `bench.py --eager --no-prefill --no-attn --no-cpu --no-engine`, each scaled by what the same counter reads
# for a plain 1 GiB device copy (profiles/decode_gemm_config2_hbm_traffic.txt).
DECODE_TRAFFIC_PER_LAUNCH = 30033462
INT8_PEAK_TOPS = 5000.0
# The reference's int8 MLP issues gate and up as one GEMM over wgu = cat(gate, up) [2 x 8192, 2048]
# (src/bitexact/int8/consts.py:68, src/bitexact/int8/model.py:106), then down; the step follows that call pattern.
DECODE_SHAPES = [("gate_up", 16384, 2048), ("down", 2048, 8192)]
SEPARATE_SHAPES = [("gate", 8192, 2048), ("up", 8192, 2048), ("down", 2048, 8192)]
DECODE_M = (1, 8, 64)
PREFILL_SHAPES = [("q_o", 2048, 2048), ("k_v", 512, 2048), ("gate_up_each", 8192, 2048), ("down", 2048, 8192),
                  ("qkv_fused", 3072, 2048), ("gate_up_fused", 16384, 2048), ("lm_head", 128256, 2048)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def quant_rows2(z):
    """int8.ops.quant_rows(z, 2) on the device with torch int64 ops (input preparation, not timed):
    sh = bitlen(amax) - 30, as_ = rsh(amax, sh), q = rdiv(rsh(z, sh) * 32512, as_)."""
    import torch
    amax = z.abs().amax(-1).clamp(min=1)
    b = torch.frexp(amax.double()).exponent.long()
    b = b - ((torch.ones_like(b) << (b - 1).clamp(min=0)) > amax).long()
    sh = b - 30

    def rsh(x, s):
        pos, neg = s.clamp(min=0), (-s).clamp(min=0)
        half = torch.where(pos > 0, torch.ones_like(pos) << (pos - 1).clamp(min=0), torch.zeros_like(pos))
        return ((x + half) >> pos) << neg
    as_ = rsh(amax, sh)
    zs = rsh(z, sh[:, None])
    n = 2 * zs * 32512 + as_[:, None]
    return torch.div(n, 2 * as_[:, None], rounding_mode="floor")


def stack2(q):
    import torch
    lo = ((q + 128) & 255) - 128
    hi = (q - lo) >> 8
    return torch.cat([lo, hi]).to(torch.int8).contiguous()


def quant40(x):
    """exact.ops.quant(P, -40) of P = round(x 2^40) on the device (input preparation, not timed)."""
    import torch
    P = torch.floor(x * 2.0 ** 40 + 0.5).long()
    amax = P.abs().amax(-1).clamp(min=1)
    b = torch.frexp(amax.double()).exponent.long()
    b = b - ((torch.ones_like(b) << (b - 1).clamp(min=0)) > amax).long()
    sh = b - 40 - 22
    s = (sh + 40).clamp(-62, 62)[:, None]
    pos = s.clamp(min=0)
    half = torch.where(pos > 0, torch.ones_like(pos) << (pos - 1).clamp(min=0), torch.zeros_like(pos))
    q = ((P + half) >> pos) << (-s).clamp(min=0)
    return q.to(torch.int32).contiguous(), sh


EAGER = False


def time_graph(fn_steps, warmup, steps, stream):
    """Capture `steps` calls of fn_steps(i) in one graph (and `warmup` in another); return seconds for the
    timed replay, measured with HIP events recorded on the capture/launch stream."""
    import torch
    # inputs (weights, decompositions, index arrays such as the ELL residual columns and block tables) were
    # written on the default stream; the launch stream is a separate non-blocking stream, so wait for them
    # before the first launch
    torch.cuda.synchronize()
    if EAGER:
        with torch.cuda.stream(stream):
            for i in range(warmup):
                fn_steps(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(steps):
                fn_steps(warmup + i)
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3
    gw, gt = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn_steps(0)                      # allocations (outputs, workspaces) before capture
        torch.cuda.synchronize()
        if warmup:
            with torch.cuda.graph(gw, stream=stream):
                for i in range(warmup):
                    fn_steps(i)
        with torch.cuda.graph(gt, stream=stream):
            for i in range(steps):
                fn_steps(warmup + i)
        torch.cuda.synchronize()
        if warmup:
            gw.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        gt.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


def bench_decode(dev, steps, warmup):
    import torch
    from bitexact.int8.gemm_skinny import int_mm_join
    g = torch.Generator(device=dev).manual_seed(1234)
    copies = {}
    for name, N, K in DECODE_SHAPES:
        if (N, K) not in copies:
            n = max(4, -(-(1 << 30) // (N * K)))
            copies[(N, K)] = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
                              for _ in range(n)]
    gc = torch.Generator().manual_seed(99)
    acts = {}
    for M in DECODE_M:
        for K in (2048, 8192):
            x = torch.randn(M, K, generator=gc, dtype=torch.float64).to(dev)
            acts[(M, K)] = stack2(quant_rows2(torch.floor(x * 2.0 ** 16 + 0.5).long()))
    outs = {}
    plan = [(M, name, N, K) for M in DECODE_M for name, N, K in DECODE_SHAPES]
    step_bytes = sum(N * K + 2 * M * K + 8 * M * N for M, _, N, K in plan)

    def step(i):
        for j, (M, name, N, K) in enumerate(plan):
            cs = copies[(N, K)]
            outs[j] = int_mm_join(acts[(M, K)], cs[(i * 3 + j) % len(cs)], M, 2)

    stream = torch.cuda.Stream(dev)
    sec = time_graph(step, warmup, steps, stream)
    per = []
    for M, name, N, K in plan + [(M, nm, N, K) for M in DECODE_M for nm, N, K in SEPARATE_SHAPES if nm != "down"]:
        if (N, K) not in copies:        # per-GEMM figures, each on its own graph (rotation as above)
            n = max(4, -(-(1 << 30) // (N * K)))
            copies[(N, K)] = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
                              for _ in range(n)]
        cs = copies[(N, K)]
        reps = 64
        s = time_graph(lambda i: int_mm_join(acts[(M, K)], cs[i % len(cs)], M, 2), 8, reps, stream)
        b = N * K + 2 * M * K + 8 * M * N
        per.append({"M": M, "gemm": name, "N": N, "K": K, "us": round(s / reps * 1e6, 3),
                    "GBps": round(b / (s / reps) / 1e9, 1)})
    del copies
    torch.cuda.empty_cache()
    return sec, step_bytes, len(plan), per


def bench_read_ceiling(dev, reps=64):
    """The practical read ceiling at the decode GEMMs' sizes: a bare streaming-read kernel (bx_stream_read: 16-byte
    nontemporal loads, grid-stride, nothing computed) over 16.8 MB (a down GEMM's weights) and 33.6 MB (gate|up),
    and 268 MB for the large-read asymptote, rotating over >= 1 GiB of buffers so every launch reads HBM,
    graph-replayed and timed with HIP events on the launch stream like the GEMMs. Best of a few launch shapes."""
    import ctypes
    import torch
    from bitexact import _hip
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream(dev)
    out = {}
    for name, nbytes in (("16.8MB", 2048 * 8192), ("33.6MB", 16384 * 2048), ("268MB", 1 << 28)):
        n = max(4, -(-(1 << 30) // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n)]
        for b in bufs:
            b.fill_(1)
        best = None
        for blocks, threads in ((256, 512), (512, 256), (1024, 256)):
            def run(i, blocks=blocks, threads=threads):
                _hip.call("bx_stream_read", ctypes.c_void_p(bufs[i % n].data_ptr()), nbytes, blocks, threads,
                          _hip.ptr(sink), _hip.stream_of(sink))
            sec = time_graph(run, 8, reps, stream) / reps
            if best is None or sec < best[0]:
                best = (sec, blocks, threads)
        out[name] = {"bytes": nbytes, "us": round(best[0] * 1e6, 3), "GBps": round(nbytes / best[0] / 1e9, 1),
                     "frac_hbm": round(nbytes / best[0] / 1e9 / HBM_PEAK_GBS, 4), "blocks": best[1],
                     "threads": best[2]}
        del bufs
        torch.cuda.empty_cache()
    return out


def bench_mfma_rate(dev, reps=8, iters=4096):
    """The dense int8 rate the matrix cores sustain: bx_mfma_rate (back-to-back MFMAs from registers, 4 independent
    chains per wave, no memory traffic; constant operands, and fresh pseudo-random operand bytes every iteration as a
    GEMM's limbs have, and the random form's instructions on constant operands as its control) at 1 and 2 waves
    per SIMD over 1024 blocks, graph-replayed and timed with
    HIP events on the launch stream. Against this, a prefill kernel's MFMA fraction separates the matrix cores'
    practical rate (clock under load) from the kernel's own scheduling losses."""
    import ctypes
    import torch
    from bitexact import _hip
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream(dev)
    out = {}
    for name, shape, ops in (("32x32x32_i8_const", 0, 65536), ("16x16x64_i8_const", 1, 32768),
                             ("32x32x32_i8_random", 2, 65536), ("16x16x64_i8_random", 3, 32768),
                             ("32x32x32_i8_control", 4, 65536), ("16x16x64_i8_control", 5, 32768)):
        best = None
        for blocks, threads in ((1024, 256), (1024, 512)):
            def run(i, shape=shape, blocks=blocks, threads=threads):
                _hip.call("bx_mfma_rate", shape, iters, blocks, threads, _hip.ptr(sink), _hip.stream_of(sink))
            sec = time_graph(run, 2, reps, stream) / reps
            tops = blocks * (threads // 64) * iters * 4 * ops / sec / 1e12
            if best is None or tops > best[0]:
                best = (tops, threads // 256, sec)
        out[name] = {"TOPS": round(best[0], 1), "frac_int8_peak": round(best[0] / INT8_PEAK_TOPS, 4),
                     "waves_per_simd": best[1], "us": round(best[2] * 1e6, 1)}
    return out


def _phase_table(name):
    """The measurement build's phase table of one source file (bx_phases_<name>): int64 [4, 1024, 8] ticks."""
    import ctypes
    import numpy as np
    from bitexact import _hip
    buf = np.zeros(4 * 1024 * 8, dtype=np.uint64)
    if _hip.lib()["bx_phases_" + name](ctypes.c_void_p(buf.ctypes.data)) != 0:
        raise RuntimeError("the phase timers need the measurement build: BX_PHASES=1 (libbitexact_hip_phases.so)")
    return buf.reshape(4, 1024, 8).astype(np.int64)


def _phase_summary(t, nblocks, names):
    """Mean / min / max (us) of each phase between consecutive marks over the first nblocks blocks (100 MHz ticks),
    and the span from the first block's start to the last block's last mark."""
    t = t[:nblocks]
    out = {}
    for k, nm in enumerate(names):
        d = (t[:, k + 1] - t[:, k]) / 100.0
        out[nm] = {"mean": round(float(d.mean()), 2), "min": round(float(d.min()), 2), "max": round(float(d.max()), 2)}
    out["block_total_mean"] = round(float(((t[:, len(names)] - t[:, 0]) / 100.0).mean()), 2)
    out["launch_span"] = round(float((t[:, len(names)].max() - t[:, 0].min()) / 100.0), 2)
    out["blocks"] = int(nblocks)
    return out


def bench_phases(dev):
    """Phase timestamps of the main kernels (the measurement build, BX_PHASES=1): the exact prefill tile at
    lm_head / q-o / down shapes (M = 2048), the exact decode stream kernel at the engine's gate|up shape (M = 32
    with q's limb planes), the split decode attention at config 4, the one-block decode attention at the engine's
    shape (batch 32, context 1024) alone and as the decode step's fused launch, the add + norm at the engine's shape
    (32 rows of 2048), and the int8 decode down GEMM at M = 64 and 8 (config 2, gemv kernel). Each is launched a
    few times over rotating copies of its weights / cache (>= 400 MB, beyond the 256 MB last-level cache, so the
    timed launch reads HBM); the table holds the last launch's first 1024 blocks."""
    import torch
    from bitexact.exact import ops
    from bitexact.exact.consts import decompose, exp2_table
    from bitexact.vllm_plugin import tri_exact_attn
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    res = {}
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    for name, M, N, K in (("xtile lm_head 2048x128256x2048", 2048, 128256, 2048),
                          ("xtile q_o 2048x2048x2048", 2048, 2048, 2048),
                          ("xtile down 2048x2048x8192", 2048, 2048, 8192),
                          ("stream gate|up 32x16384x2048 (engine)", 32, 16384, 2048)):
        ncop = max(1, min(4, -(-(400 << 20) // (3 * N * K))))   # weight copies: each launch reads HBM
        decs = []
        for c in range(ncop):
            w = (torch.randn(N, K, generator=torch.Generator(device=dev).manual_seed(N + K + c), device=dev) *
                 0.02).to(torch.bfloat16)
            decs.append(decompose(w))
            del w
        q, sh = quant40(torch.randn(M, K, generator=torch.Generator().manual_seed(5), dtype=torch.float64).to(dev))
        pl = None
        if M == 32:
            pl = torch.empty(3, M, K, dtype=torch.int8, device=dev)
            v = q.to(torch.int64)
            for i in range(3):
                lo = ((v + 128) & 255) - 128
                pl[i] = lo.to(torch.int8)
                v = (v - lo) >> 8
        for i in range(max(3, ncop)):
            dec = decs[i % ncop]
            exact_linear(q, sh, dec["limbs"], dec["d"], dec["g"], dec["ell_cnt"], dec["ell_col"], dec["ell_val"],
                         dec["R"], flag, False, q_planes=pl)
        torch.cuda.synchronize()
        t = _phase_table("linear")
        if M == 32:
            res[name] = _phase_summary(t[1], (N + 63) // 64, ["fill+chunk0", "chunks 1..", "epilogue"])
        else:
            res[name] = _phase_summary(t[0], min(1024, ((N + 127) // 128) * ((M + 127) // 128)),
                                       ["context", "first stage", "loop", "gathers", "epilogue"])
        del decs, dec, q, sh
        torch.cuda.empty_cache()
    lut = exp2_table(dev)
    g = torch.Generator(device=dev).manual_seed(77)
    for name, B, S, nsplit, slot, names in (
            ("decode attention split (config 4: B=4, ctx 2048)", 4, 2048, None, 0,
             ["K/V + scores", "maxima exchange", "weights + pV", "finish"]),
            ("decode attention one block (engine: B=32, ctx 1024)", 32, 1024, 1, 1,
             ["prologue", "K sweep", "V request", "V sweep", "finish"])):
        HKV, grp, HD, bs = 8, 4, 64, 16
        nblk = S // bs
        nb = B * nblk
        ncop = -(-(400 << 20) // (nb * HKV * bs * 8 * HD))           # cache copies: each launch reads HBM
        caches = [torch.randint(-128, 128, (nb, HKV, bs, 8 * HD), dtype=torch.int8, device=dev, generator=g)
                  for _ in range(ncop)]
        bt = torch.randperm(nb, device=dev, generator=g).to(torch.int32).reshape(B, nblk)
        rmap = torch.arange(B, device=dev)
        qa = torch.randint(-(1 << 22), (1 << 22) + 1, (B, HKV, grp, HD), device=dev, generator=g).to(torch.int32)
        sha = torch.randint(-40, -25, (B, HKV, grp), device=dev, generator=g)
        qpos = torch.full((B, grp), S - 1, dtype=torch.long, device=dev)
        for i in range(max(3, ncop)):
            tri_exact_attn.attend(qa, sha, qpos, caches[i % ncop], bt, rmap, lut, 387270501, nsplit=nsplit)
        torch.cuda.synchronize()
        t = _phase_table("attn")
        nblocks = B * HKV * (8 if nsplit is None else 1)
        res[name] = _phase_summary(t[slot], min(1024, nblocks), names)
        del caches
        torch.cuda.empty_cache()
    x = torch.randint(-(1 << 36), 1 << 36, (32, 2048), device=dev, generator=g)
    y = torch.randint(-(1 << 36), 1 << 36, (32, 2048), device=dev, generator=g)
    gm = torch.randint(1 << 7, 1 << 8, (2048,), device=dev, generator=g)
    ge = torch.full((2048,), -7, dtype=torch.long, device=dev)
    for _ in range(3):
        ops.add_norm_y(y, x.clone(), gm, ge, flag=flag, planes=True)
    torch.cuda.synchronize()
    # the decode step's fused launch at the engine's shape (rope prologue, attention, output stage with limb planes):
    # 32 tokens at position 1023, 8 KV heads of 4 q heads, rotating caches
    from bitexact.exact.consts import FT, llama3_inv_freq, rope_tables
    N, H, HKV, HD, bs, nblk = 32, 32, 8, 64, 16, 65
    cos, sin = rope_tables(2048, FT, llama3_inv_freq(HD))
    cos, sin = cos.to(dev), sin.to(dev)
    gy = torch.Generator(device=dev).manual_seed(3)
    y = torch.randint(-(1 << 30), 1 << 30, (N, (H + 2 * HKV) * HD), device=dev, generator=gy)
    pos = torch.full((N,), 1023, dtype=torch.long, device=dev)
    bt = torch.randperm(N * nblk, device=dev, generator=gy).to(torch.int32).view(N, nblk)
    rmap = torch.arange(N, device=dev)
    slot = bt[rmap, pos // bs].long() * bs + pos % bs
    ncop = -(-(400 << 20) // (N * nblk * HKV * bs * 8 * HD))
    caches = [torch.randint(-128, 128, (N * nblk, HKV, bs, 8 * HD), dtype=torch.int8, device=dev, generator=gy)
              for _ in range(ncop)]
    for i in range(max(3, ncop)):
        tri_exact_attn.rope_attend_out(y, pos, cos, sin, (H, HKV, HD), caches[i % ncop], slot, bt, rmap, lut,
                                       387270501, flag, planes=True)
    torch.cuda.synchronize()
    res["decode step attention (engine: rope + attention + output stage, 32 tokens, ctx 1024)"] = _phase_summary(
        _phase_table("attn")[1], N * HKV, ["rope prologue", "K sweep", "V request", "V sweep", "finish + output"])
    del caches
    torch.cuda.empty_cache()
    # int8 decode down GEMMs (config 2: K = 8192, N = 2048) on the gemv kernel: 256 blocks (4 K splits)
    from bitexact.int8.gemm_skinny import int_mm_join
    gw = torch.Generator(device=dev).manual_seed(1)
    wc = [torch.randint(-127, 128, (2048, 8192), dtype=torch.int8, device=dev, generator=gw) for _ in range(24)]
    for M in (64, 8):
        xm = torch.randn(M, 8192, generator=torch.Generator().manual_seed(M), dtype=torch.float64).to(dev)
        am = stack2(quant_rows2(torch.floor(xm * 2.0 ** 16 + 0.5).long()))
        for i in range(len(wc)):
            int_mm_join(am, wc[i], M, 2)
        torch.cuda.synchronize()
        res[f"gemv int8 down {M}x2048x8192 (config 2)"] = _phase_summary(
            _phase_table("linear")[2], 256, ["activations to LDS", "k loop", "k-slice reduce", "split-K adds",
                                             "last split: sums + outputs"])
    del wc
    torch.cuda.empty_cache()
    res["add + norm (engine: 32 rows of 2048)"] = _phase_summary(_phase_table("rows")[0], 32,
                                                                ["row loaded", "divisor", "quotients", "quantize"])
    return res


def bench_prefill(dev, reps=10):
    import torch
    from bitexact.exact.consts import decompose
    from bitexact.vllm_plugin.exact_gemm import exact_linear
    M = 2048
    gc = torch.Generator().manual_seed(5)
    stream = torch.cuda.Stream(dev)
    res, tot_ops, tot_s = [], 0, 0.0
    for name, N, K in PREFILL_SHAPES:
        gw = torch.Generator(device=dev).manual_seed(N + K)
        w = (torch.randn(N, K, generator=gw, device=dev) * 0.02).to(torch.bfloat16)
        dec = decompose(w)
        q, sh = quant40(torch.randn(M, K, generator=gc, dtype=torch.float64).to(dev))
        flag = torch.zeros(1, dtype=torch.int32, device=dev)
        outs = {}

        def run(i):
            outs[0] = exact_linear(q, sh, dec["limbs"], dec["d"], dec["g"], dec["ell_cnt"], dec["ell_col"],
                                   dec["ell_val"], dec["R"], flag, True)
        s = time_graph(run, 2, reps, stream) / reps
        check_prefill_sample(name, w, q, sh, outs[0], flag)
        del w
        ops = 9 * 2 * M * N * K
        tops = ops / s / 1e12
        res.append({"gemm": name, "M": M, "N": N, "K": K, "us": round(s * 1e6, 1), "TOPS": round(tops, 1),
                    "frac": round(tops / INT8_PEAK_TOPS, 4)})
        if name not in ("qkv_fused", "gate_up_fused"):
            mult = {"q_o": 2, "k_v": 2, "gate_up_each": 2}.get(name, 1)
            tot_ops += mult * ops
            tot_s += mult * s
        del dec, q
        torch.cuda.empty_cache()
    return res, tot_ops / tot_s / 1e12


def check_prefill_sample(name, w, q, sh, y, flag, nrows=4, ncols=64):
    """The timed output against oracle/bxref.py's exact linear on a sample: nrows rows (first, last, two seeded)
    x ncols columns (first, last, seeded). The decomposition is row-local, so the oracle decomposes only the
    sampled weight rows. Raises if any sampled output or the flag differs."""
    import numpy as np
    import torch
    sys.path.insert(0, HERE)
    from oracle import bxref as R
    M, N = y.shape
    rng = np.random.default_rng(M + N)
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, nrows - 2)]))
    cols = np.unique(np.concatenate([[0, N - 1], rng.integers(0, N, ncols - 2)]))
    dec = R.decompose(w[torch.from_numpy(cols).to(w.device)].cpu().view(torch.int16).numpy())
    ref, rflag = R.exact_linear(q[torch.from_numpy(rows).to(q.device)].cpu().long().numpy(),
                                dec, sh[torch.from_numpy(rows).to(sh.device)].cpu().numpy())
    got = y.cpu().numpy()[np.ix_(rows, cols)]
    if not np.array_equal(got, ref) or (rflag and not bool(flag.item())):
        raise AssertionError(f"exact prefill {name}: sampled outputs differ from the oracle")


def bench_attention(dev, reps=20):
    """Config 4: paged exact decode attention (one query per head, group 4 -> M = 4 per KV head) over a
    2048-token context per sequence, and the fused exact prefill attention over the whole causal T = 2048."""
    import torch
    from bitexact.exact.attention import prefill
    from bitexact.exact.consts import exp2_table
    from bitexact.vllm_plugin import tri_exact_attn
    B, H, HKV, HD, S, bs = 4, 32, 8, 64, 2048, 16
    grp = H // HKV
    lim = 8355711
    l2e = 387270501
    lut = exp2_table(dev)
    g = torch.Generator(device=dev).manual_seed(77)
    nblk = S // bs
    nb = B * nblk
    cache_bytes = nb * HKV * bs * 8 * HD
    ncop = max(4, -(-(1 << 30) // cache_bytes))
    caches = [torch.randint(-128, 128, (nb, HKV, bs, 8 * HD), dtype=torch.int8, device=dev, generator=g)
              for _ in range(ncop)]
    bt = torch.randperm(nb, device=dev, generator=g).to(torch.int32).reshape(B, nblk)
    rmap = torch.arange(B, device=dev)
    q = torch.randint(-(1 << 22), (1 << 22) + 1, (B, HKV, grp, HD), device=dev, generator=g).to(torch.int32)
    sh = torch.randint(-40, -25, (B, HKV, grp), device=dev, generator=g)
    qpos = torch.full((B, grp), S - 1, dtype=torch.long, device=dev)
    stream = torch.cuda.Stream(dev)
    outs = {}

    def dstep(i):
        outs[0] = tri_exact_attn.attend(q, sh, qpos, caches[i % ncop], bt, rmap, lut, l2e)
    s_dec = time_graph(dstep, 4, reps * 4, stream) / (reps * 4)
    dbytes = B * HKV * S * 6 * HD
    del caches
    torch.cuda.empty_cache()
    # prefill: qg [B HKV, grp T, HD] grouped queries, K / V [B HKV, S, HD], causal positions
    T = S
    Z = B * HKV
    qg = torch.randint(-(1 << 22), (1 << 22) + 1, (Z, grp * T, HD), device=dev, generator=g).to(torch.int32)
    shg = torch.randint(-40, -25, (Z, grp * T, 1), device=dev, generator=g)
    K = torch.randint(-lim, lim + 1, (Z, S, HD), device=dev, generator=g).to(torch.int32)
    V = torch.randint(-lim, lim + 1, (Z, S, HD), device=dev, generator=g).to(torch.int32)
    qp = torch.arange(T, device=dev).repeat(grp).reshape(1, grp * T, 1).expand(Z, grp * T, 1).contiguous()

    def pstep(i):
        outs[1] = prefill(qg, shg, K, V, qp, lut, l2e)
    s_pre = time_graph(pstep, 1, 3, stream) / 3
    ops = 2 * 9 * 2 * HD * B * H * T * (T + 1) // 2
    return {"workload": "config 4: B=4, H=32, HKV=8, HD=64, causal, context 2048, paged block 16",
            "decode_us": round(s_dec * 1e6, 2), "decode_bytes": dbytes,
            "decode_GBps": round(dbytes / s_dec / 1e9, 1), "decode_frac_hbm": round(dbytes / s_dec / 1e9 / HBM_PEAK_GBS, 4),
            "prefill_ms": round(s_pre * 1e3, 3), "prefill_limb_ops": ops,
            "prefill_TOPS": round(ops / s_pre / 1e12, 2),
            "prefill_frac_int8_peak": round(ops / s_pre / 1e12 / INT8_PEAK_TOPS, 4)}


def bench_bmm(dev, reps=5):
    """bitexact.bmm.bmm (the reference model's unfused attention products) at config 4's shapes: q.k
    [32, 8192, 64] x [32, 64, 2048] (int64 scores, 4.3 GB written: HBM-write bound) and p.v [32, 8192, 2048] x
    [32, 2048, 64] (3-limb weights and values: MFMA bound). Limb-op TOPS = 9 x 2 Z M N K per call."""
    import torch
    from bitexact.bmm import bmm
    g = torch.Generator(device=dev).manual_seed(21)
    Z, gT, S, HD = 32, 8192, 2048, 64
    lim = 8355711
    qg = torch.randint(-(1 << 22), (1 << 22) + 1, (Z, gT, HD), device=dev, generator=g).to(torch.int32)
    Kc = torch.randint(-lim, lim + 1, (Z, S, HD), device=dev, generator=g).to(torch.int32)
    stream = torch.cuda.Stream(dev)
    outs = {}
    s_qk = time_graph(lambda i: outs.__setitem__(0, bmm(qg, Kc.transpose(1, 2))), 1, reps, stream) / reps
    # a row sample of q.k against the oracle's exact product
    sys.path.insert(0, HERE)
    from oracle import bxref as R
    import numpy as np
    zs, rows = [0, Z - 1], [0, 4097, gT - 1]
    for z in zs:
        ref = R.bmm(qg[z, rows].cpu().numpy()[None], Kc[z].cpu().numpy().T[None])[0]
        if not np.array_equal(outs[0][z, rows].cpu().numpy(), ref):
            raise AssertionError("bmm q.k differs from the oracle")
    del outs[0]
    torch.cuda.empty_cache()
    p = torch.randint(0, 1 << 22, (Z, gT, S), device=dev, generator=g).to(torch.int32)
    V = torch.randint(-lim, lim + 1, (Z, S, HD), device=dev, generator=g).to(torch.int32)
    s_pv = time_graph(lambda i: outs.__setitem__(1, bmm(p, V)), 1, reps, stream) / reps
    ops_qk = 9 * 2 * Z * gT * S * HD
    return {"workload": "config 4 shapes: q.k [32, 8192, 64] x [32, 64, 2048], p.v [32, 8192, 2048] x [32, 2048, 64]",
            "qk_us": round(s_qk * 1e6, 1), "qk_TOPS": round(ops_qk / s_qk / 1e12, 1),
            "qk_write_GBps": round(8 * Z * gT * S / s_qk / 1e9, 1),
            "qk_frac_hbm": round(8 * Z * gT * S / s_qk / 1e9 / HBM_PEAK_GBS, 4),
            "pv_us": round(s_pv * 1e6, 1), "pv_TOPS": round(ops_qk / s_pv / 1e12, 1),
            "pv_frac_int8_peak": round(ops_qk / s_pv / 1e12 / INT8_PEAK_TOPS, 4)}


def bench_engine(dev, steps, warmup, B=32, ctx=1024, bs=16):
    """Config 5: a random-init Llama-3.2-1B (16 layers, bf16 N(0,0.02) weights decomposed on the device) in exact
    mode. Prefill B sequences of ctx seeded random token ids into the paged block-16 KV cache, then time greedy
    decode steps at batch B (forward + logits + first-max + next-step inputs, one HIP graph per step replayed
    `steps` times). Also checks that sequence 0's first decode logits hash is the same at batch 1, 8 and B."""
    import torch
    from bitexact.exact.consts import random_constants
    from bitexact.generate import logits_sha
    from bitexact.vllm_plugin.exact_run import ExactEngine
    t0 = time.time()
    eng = ExactEngine(random_constants(None, seed=0, device=dev), dev)
    torch.cuda.synchronize()
    t_build = time.time() - t0
    nblk = -(-(ctx + warmup + steps + 2) // bs)
    bt = (1 + torch.arange(B * nblk, device=dev, dtype=torch.int32)).view(B, nblk)
    kvs = eng.new_cache(1 + B * nblk, bs)
    g = torch.Generator().manual_seed(5)
    prompts = torch.randint(0, eng.V, (B, ctx), generator=g).to(dev)
    # prefill in chunks of whole sequences
    t0 = time.time()
    first = torch.empty(B, dtype=torch.long, device=dev)
    chunk = max(1, 4096 // ctx)
    for s0 in range(0, B, chunk):
        seqs = torch.arange(s0, min(B, s0 + chunk), device=dev)
        n = seqs.numel()
        pos = torch.arange(ctx, device=dev).repeat(n)
        rmap = seqs.repeat_interleave(ctx)
        slot = bt[rmap, pos // bs].long() * bs + pos % bs
        x = eng.forward(kvs, prompts[s0:s0 + n].reshape(-1), pos, slot, bt, rmap)
        first[s0:s0 + n] = eng.greedy(eng.logits(x.view(n, ctx, -1)[:, -1].contiguous()))
    torch.cuda.synchronize()
    t_prefill = time.time() - t0
    # batch invariance: sequence 0's first decode step at batch 1, 8 and B (row-local rules: same bits)
    shas = {}
    for b in (1, 8, B):
        pos = torch.full((b,), ctx, device=dev, dtype=torch.long)
        rmap = torch.arange(b, device=dev)
        slot = bt[rmap, pos // bs].long() * bs + pos % bs
        x = eng.forward(kvs, first[:b], pos, slot, bt, rmap, one_per_seq=True)
        shas[b] = logits_sha(eng.logits(x)[0])
    # timed decode: static inputs updated on the device by each step
    ids = first.clone()
    pos = torch.full((B,), ctx, device=dev, dtype=torch.long)
    rmap = torch.arange(B, device=dev)
    slot = bt[rmap, pos // bs].long() * bs + pos % bs

    def step(i):
        x = eng.forward(kvs, ids, pos, slot, bt, rmap, one_per_seq=True)
        eng.advance(eng.logits(x), ids, pos, slot, bt, rmap, bs)      # ids, pos, slot for the next step

    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        step(0)                                          # allocations and workspaces before capture
    torch.cuda.synchronize()
    pos.fill_(ctx)
    slot.copy_(bt[rmap, pos // bs].long() * bs + pos % bs)
    ids.copy_(first)
    sec = time_graph(step, warmup, steps, stream)
    overflow = bool(eng.err)
    tok_s = B * steps / sec
    return {"workload": "config 5: random-init Llama-3.2-1B exact mode (16 layers, D 2048, FF 8192, V 128256, "
                        "bf16 N(0,0.02) weights), greedy decode at batch %d, context %d, paged KV block %d" % (B, ctx, bs),
            "tokens_per_s": round(tok_s, 1), "ms_per_step": round(sec / steps * 1e3, 4), "batch": B, "context": ctx,
            "steps": steps, "warmup": warmup, "weight_bytes_per_step": eng_weight_bytes(eng),
            "weight_GBps": round(eng_weight_bytes(eng) * steps / sec / 1e9, 1),
            "logits_sha_batch_1_8_%d_equal" % B: len(set(shas.values())) == 1, "logits_sha_seq0": shas[1][:16],
            "overflow_flag": overflow, "build_s": round(t_build, 1), "prefill_s": round(t_prefill, 2)}


def eng_weight_bytes(eng):
    """Limb-plane bytes one decode step streams: every linear's 3 int8 planes."""
    return sum(int(f.limbs.numel()) for f in eng.fused.values())


def copy_calibrate(dev):
    """A plain 1 GiB device copy, 20 times: the HBM counters read for it scale the bench's counters."""
    import torch
    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each_way": 1 << 30, "copies": 20}), flush=True)


def _blas_threads():
    from threadpoolctl import threadpool_info
    return max([i.get("num_threads", 1) for i in threadpool_info()] or [1])


def cpu_baseline(budget_s=6.0):
    """oracle/bxref.py's float64 restatement of the int8 GEMM (the reference's CPU path imm,
    src/bitexact/int8/ops.py:87-90) on the config-2 shapes at M = 8, on the host cores; GB/s of the same
    algorithmic bytes as the GPU figure."""
    import numpy as np
    sys.path.insert(0, HERE)
    from oracle import bxref as R
    rng = np.random.default_rng(0)
    M, t_tot, b_tot, runs = 8, 0.0, 0, 0
    t_start = time.perf_counter()
    ws = {(N, K): rng.integers(-127, 128, (N, K)).astype(np.int8) for _, N, K in DECODE_SHAPES}
    while time.perf_counter() - t_start < budget_s:
        for name, N, K in DECODE_SHAPES:
            q = rng.integers(-32512, 32513, (M, K))
            t0 = time.perf_counter()
            R.imm(q, ws[(N, K)])
            t_tot += time.perf_counter() - t0
            b_tot += N * K + 2 * M * K + 8 * M * N
        runs += 1
    return {"value": round(b_tot / t_tot / 1e9, 3), "unit": "GB/s", "cores": _blas_threads(),
            "host_cores": os.cpu_count(), "kind": "port",
            "sample": f"oracle float64 imm (numpy BLAS) on config-2 gate/up/down at M={M}, {runs} passes, "
                      f"{t_tot:.1f} s of GEMM time"}


def cpu_baseline_exact(budget_s=6.0):
    """The exact linear on the host cores as the reference's CPU path computes it: oracle/bxref.py's float64
    wmm_f64 + residual + epilogue (src/bitexact/exact/wmm.py:117-150) on config 1 (M = 8, K = N = 2048) and on
    config 3's q/o shape (M = 2048, K = N = 2048); effective limb-op TOPS (9 x 2 M N K per call), as the GPU's."""
    import numpy as np
    import torch
    sys.path.insert(0, HERE)
    from oracle import bxref as R
    out = {}
    for tag, M in (("config1_M8", 8), ("config3_q_o_M2048", 2048)):
        N = K = 2048
        g = torch.Generator().manual_seed(M)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
        dec = R.decompose(w.view(torch.int16).numpy())
        rng = np.random.default_rng(M)
        q = rng.integers(-(1 << 22), (1 << 22) + 1, (M, K))
        sh = rng.integers(-30, -20, M)
        t_tot, runs = 0.0, 0
        while t_tot < budget_s / 2 and runs < 1000:
            t0 = time.perf_counter()
            T = R.wmm_f64(q, dec["W"])
            B = R.residual(q, dec["rr"], dec["rc"], dec["rv"], N)
            R.epilogue(T, B, dec["d"], dec["g"], sh, R.FR, True)
            t_tot += time.perf_counter() - t0
            runs += 1
        ops = 9 * 2 * M * N * K
        out[tag] = {"us_per_call": round(t_tot / runs * 1e6, 1), "TOPS": round(ops * runs / t_tot / 1e12, 4),
                    "calls": runs}
    out.update({"unit": "limb-op TOPS", "cores": _blas_threads(), "host_cores": os.cpu_count(), "kind": "port",
                "sample": "oracle float64 wmm_f64 + residual + epilogue (the reference's wmm_cpu chain), "
                          "bf16 N(0,0.02) weights, |q| <= 2^22"})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--warmup", type=int, default=6)
    ap.add_argument("--no-decode", action="store_true", help="profiling runs: skip the decode step (no value)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-attn", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-engine", action="store_true")
    ap.add_argument("--engine-steps", type=int, default=20)
    ap.add_argument("--eager", action="store_true")
    ap.add_argument("--copy-calibrate", action="store_true")
    ap.add_argument("--phases", action="store_true",
                    help="phase timestamps of the main kernels (loads the measurement build, BX_PHASES=1)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.phases:
        os.environ["BX_PHASES"] = "1"          # before the library loads: the measurement build
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the hot path has no collectives); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_calibrate:
        copy_calibrate(dev)
        return
    if args.phases:
        print(json.dumps({"phases": bench_phases(dev), "unit": "us (100 MHz real-time counter)"}), flush=True)
        return
    if args.no_decode:
        sec, step_bytes, launches, per, value = 1.0, 0, 1, [], None
    else:
        log("decode GEMMs ...")
        sec, step_bytes, launches, per = bench_decode(dev, args.steps, args.warmup)
        value = step_bytes * args.steps / sec / 1e9

    def r(x, n):
        return None if x is None else round(x, n)
    # roofline of the decode launches (each one kernel); algorithmic bytes per launch
    # over its average duration (graph replay timed with HIP events on the launch stream)
    per_launch_s = sec / args.steps / launches
    achieved = None if value is None else step_bytes / launches / per_launch_s / 1e9
    out = {"metric": "int8 decode GEMM HBM GB/s (config 2); exact prefill limb-GEMM TOPS and % int8 MFMA peak "
                     "(config 3); 1 GPU",
           "value": r(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(sec / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8 (int32 accumulate, int64 join)", "data": "synthetic",
           "config": {"workload": "config 2: int8-mode decode GEMMs, M in {1,8,64} x gate|up as the reference's fused "
                                  "wgu (K=2048, N=2x8192), down (K=8192, N=2048), 2 activation limbs, int64 joined "
                                  "output",
                      "gemms_per_step": launches, "bytes_per_step": step_bytes, "weight_rotation": ">=1 GiB/shape"},
           "roofline": {"bound": "hbm",
                        "kernel": "decode GEMM launches (stream_kernel gate|up at M=1/8/64, staged_kernel M=1 down, "
                                  "gemv_kernel M=8/64 down)",
                        "achieved": r(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": r(None if achieved is None else achieved / HBM_PEAK_GBS, 4),
                        "traffic": DECODE_TRAFFIC_PER_LAUNCH, "algorithmic_bytes_per_launch": step_bytes // launches,
                        "launch_us": round(per_launch_s * 1e6, 3)},
           "per_gemm": per}
    if value is not None:
        log("read ceiling ...")
        ceil = bench_read_ceiling(dev)
        # the step at the measured ceiling rates: each GEMM's algorithmic bytes at its size's bare-read rate
        rate = {2048: ceil["16.8MB"]["GBps"], 16384: ceil["33.6MB"]["GBps"]}
        step_at_ceiling = sum((N * K + 2 * M * K + 8 * M * N) / (rate[N] * 1e9)
                              for M in DECODE_M for _, N, K in DECODE_SHAPES)
        ceil["step_us_at_ceiling"] = round(step_at_ceiling * 1e6, 2)
        ceil["step_GBps_at_ceiling"] = round(step_bytes / step_at_ceiling / 1e9, 1)
        ceil["frac_of_ceiling"] = round(step_at_ceiling / (sec / args.steps), 4)
        out["read_ceiling"] = ceil
    if not args.no_prefill:
        log("exact prefill GEMMs ...")
        res, tops = bench_prefill(dev)
        out["exact_prefill"] = {"workload": "config 3: exact limb GEMM, M=2048, Llama-3.2-1B linears (bf16 N(0,0.02) "
                                            "weights, 3-limb N(0,1) activations), fused epilogue",
                                "TOPS": round(tops, 1), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                "peak_TOPS": INT8_PEAK_TOPS, "per_gemm": res}
    log("mfma rate ...")
    out["mfma_rate"] = bench_mfma_rate(dev)
    if not args.no_attn:
        log("attention ...")
        out["exact_attention"] = bench_attention(dev)
    if not args.no_attn:
        log("bmm ...")
        out["bmm"] = bench_bmm(dev)
    if not args.no_engine:
        log("exact decode engine (config 5) ...")
        out["exact_engine"] = bench_engine(dev, args.engine_steps, 3)
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline()
        out["cpu_baseline_exact"] = cpu_baseline_exact()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
