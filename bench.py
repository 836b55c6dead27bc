#!/usr/bin/env python3
"""gdn2 token-mixer benchmark on one MI355X.

Headline workload: chunkwise prefill of B=8 sequences of
T=4096 tokens, H=16 heads, d_k = d_v = 128, bf16 inputs, fp32 log-decay and
state, chunk 64, in-kernel q/k L2 norm, final state written.  A "step" is one
full forward of that batch with the inputs already resident in HBM.

Also measured: the single-token decode step, N=64
sequences x 16 heads, fp32 state [64,16,128,128] updated in place, 1024
consecutive steps captured in one HIP graph.

Also measured: a 0.68 B-parameter hybrid decoder (18 gdn2
+ 6 attention layers) prefilling 4 x 2048 tokens and decoding 256 greedily, with
the decode step replayed as one HIP graph.

Prints one JSON line: value = prefill tokens/s, with the roofline of the
prefill kernels (HBM-bound), the decode figures, and the CPU baseline (the C
restatement of the reference recurrence, oracle/gdn2_cpu.c, timed on this
host's cores on the same prefill inputs).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

METRIC = "gdn2 prefill tokens/s + decode µs/step; % of MFMA / HBM roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

PREFILL = dict(B=8, T=4096, H=16, K=128, V=128, C=64)
DECODE = dict(N=64, H=16, K=128, V=128, steps=1024)
DECODE_BEYOND_MALL = dict(N=256, steps=256)  # 268 MB of state, more than the 256 MB MALL
TRAIN = dict(B=4, T=8192, H=16, K=128, V=128, C=64)
# Mixer prologue / epilogue at config 3's module shape (hidden 1024, 16 heads x 64).
PROLOGUE = dict(B=4, T=2048, H=16, Dh=64, W=4)


def prefill_flops(B, T, H, K, V, C):
    """Dense chunkwise WY work per token-head: 6KV + 2C(3K+2V) + C^2/3."""
    return B * T * H * (6 * K * V + 2 * C * (3 * K + 2 * V) + C * C / 3.0)


def prefill_bytes(B, T, H, K, V):
    """Algorithmic HBM bytes: q,k,b,v,w bf16 + g fp32 in, o bf16 out, fp32 final state."""
    per_th = 2 * (3 * K + 2 * V) + 4 * K + 2 * V
    return B * T * H * per_th + B * H * K * V * 4


def decode_bytes(N, H, K, V):
    """Per step: fp32 state read + write, q,k,b,v,w bf16 + g fp32 in, o bf16 out."""
    return 2 * N * H * K * V * 4 + N * H * (2 * (3 * K + 2 * V) + 4 * K + 2 * V)


def train_bytes(B, T, H, K, V):
    """Algorithmic HBM bytes of fwd+bwd: q,k,v,b,w bf16 + g fp32 read twice, dO read,
    o written, dq,dk,dv,db,dw bf16 + dg fp32 written."""
    fwd = 2 * (3 * K + 2 * V) + 4 * K + 2 * V
    bwd = 2 * (3 * K + 2 * V) + 4 * K + 2 * V + 2 * (3 * K + 2 * V) + 4 * K
    return B * T * H * (fwd + bwd)


def train_flops(B, T, H, K, V, C):
    """Dense chunkwise work per token-head: forward 6KV + 2C(3K+2V) + C^2/3, backward
    16KV + 14CK + 10CV + 4C^2."""
    return B * T * H * (6 * K * V + 2 * C * (3 * K + 2 * V) + C * C / 3.0
                        + 16 * K * V + 14 * C * K + 10 * C * V + 4 * C * C)


def make_prefill_inputs(torch, dev, B, T, H, K, V, seed=1):
    """Config-1 recipe: q,k ~ N(0,1) L2-normalised; v ~ N(0,1); beta = sigmoid(N);
    g = -softplus(N + 2); beta and g per (b,t,h), broadcast to the channel-wise API."""
    F = torch.nn.functional
    gen = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    q = F.normalize(torch.randn(B, T, H, K, generator=gen, device=dev), dim=-1).to(bf)
    k = F.normalize(torch.randn(B, T, H, K, generator=gen, device=dev), dim=-1).to(bf)
    v = torch.randn(B, T, H, V, generator=gen, device=dev).to(bf)
    beta = torch.sigmoid(torch.randn(B, T, H, 1, generator=gen, device=dev))
    g = -F.softplus(torch.randn(B, T, H, 1, generator=gen, device=dev) + 2.0)
    g = g.expand(B, T, H, K).contiguous()
    b = beta.expand(B, T, H, K).to(bf).contiguous()
    w = beta.expand(B, T, H, V).to(bf).contiguous()
    return q, k, v, g, b, w


def bench_prefill(torch, nat, dev, steps, warmup):
    B, T, H, K, V, C = (PREFILL[x] for x in ("B", "T", "H", "K", "V", "C"))
    q, k, v, g, b, w = make_prefill_inputs(torch, dev, B, T, H, K, V)
    lib = nat.load()
    io, gd = nat.DTYPE_BF16, nat.DTYPE_F32
    ws_bytes = lib.gdn2_chunk_fwd_workspace_size(B, T, H, K, V, io, None, B)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    scale = K**-0.5
    flags = nat.FLAG_L2NORM_QK
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def prep():
        st = lib.gdn2_chunk_fwd_prep(q.data_ptr(), k.data_ptr(), g.data_ptr(), b.data_ptr(), io, gd,
                                     None, None, 0.0, None, None, B, B, T, H, K, V, scale, flags,
                                     ws.data_ptr(), ws_bytes, sh)
        nat.check(st, "gdn2_chunk_fwd_prep")

    def scan():
        st = lib.gdn2_chunk_fwd_scan(v.data_ptr(), w.data_ptr(), io, o.data_ptr(), None,
                                     ht.data_ptr(), None, None, B, B, T, H, K, V, ws.data_ptr(),
                                     ws_bytes, sh)
        nat.check(st, "gdn2_chunk_fwd_scan")

    for _ in range(warmup):
        prep()
        scan()
    torch.cuda.synchronize(dev)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for e in evs:
        e[0].record(stream)
        prep()
        e[1].record(stream)
        scan()
        e[2].record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    t_prep = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    t_scan = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)
    if not torch.isfinite(o.float()).all() or not torch.isfinite(ht).all():
        raise RuntimeError("non-finite prefill output")
    ms_step = wall * 1e3 / steps
    return dict(ms_step=ms_step, t_prep_ms=t_prep, t_scan_ms=t_scan,
                inputs=(q, k, v, g, b, w))


def bench_train(torch, nat, dev, steps, warmup):
    """C4: training forward (saving the backward's workspace) then backward, bf16."""
    B, T, H, K, V = (TRAIN[x] for x in ("B", "T", "H", "K", "V"))
    q, k, v, g, b, w = make_prefill_inputs(torch, dev, B, T, H, K, V, seed=4)
    gen = torch.Generator(device=dev).manual_seed(40)
    do = torch.randn(B, T, H, V, generator=gen, device=dev).to(torch.bfloat16)
    lib = nat.load()
    io, gd = nat.DTYPE_BF16, nat.DTYPE_F32
    sv_bytes = lib.gdn2_chunk_train_workspace_size(B, T, H, K, V, io, None, B)
    bw_bytes = lib.gdn2_chunk_bwd_workspace_size(B, T, H, K, V, io, None, B)
    sv = torch.empty(sv_bytes, dtype=torch.uint8, device=dev)
    bw = torch.empty(bw_bytes, dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    dq, dk, db = torch.empty_like(q), torch.empty_like(k), torch.empty_like(b)
    dv, dw, dg = torch.empty_like(v), torch.empty_like(w), torch.empty_like(g)
    scale = K**-0.5
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def fwd():
        st = lib.gdn2_chunk_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), b.data_ptr(),
                                w.data_ptr(), io, gd, o.data_ptr(), None, None, None, None, 0.0, None,
                                None, B, B, T, H, K, V, scale,
                                nat.FLAG_L2NORM_QK | nat.FLAG_SAVE_FOR_BWD, sv.data_ptr(), sv_bytes, sh)
        nat.check(st, "gdn2_chunk_fwd (training)")

    def bwd():
        st = lib.gdn2_chunk_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), b.data_ptr(),
                                w.data_ptr(), io, gd, do.data_ptr(), None, dq.data_ptr(),
                                dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), db.data_ptr(),
                                dw.data_ptr(), None, None, None, B, B, T, H, K, V, scale,
                                nat.FLAG_L2NORM_QK, sv.data_ptr(), sv_bytes, bw.data_ptr(), bw_bytes,
                                sh)
        nat.check(st, "gdn2_chunk_bwd")

    for _ in range(warmup):
        fwd()
        bwd()
    torch.cuda.synchronize(dev)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for e in evs:
        e[0].record(stream)
        fwd()
        e[1].record(stream)
        bwd()
        e[2].record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    t_f = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    t_b = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)
    for x in (o, dq, dk, dv, db, dw, dg):
        if not torch.isfinite(x.float()).all():
            raise RuntimeError("non-finite training output")
    ms = wall * 1e3 / steps
    nbytes = train_bytes(B, T, H, K, V)
    flops = train_flops(B, T, H, K, V, TRAIN["C"])
    t_op = (t_f + t_b) * 1e-3
    return {"tokens_per_s": round(B * T / (ms * 1e-3), 1), "ms_per_step": round(ms, 4),
            "fwd_ms": round(t_f, 4), "bwd_ms": round(t_b, 4),
            "algorithmic_bytes": nbytes, "achieved_GBps": round(nbytes / t_op / 1e9, 1),
            "frac_hbm_peak": round(nbytes / t_op / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_flop": flops, "achieved_TFLOPs": round(flops / t_op / 1e12, 2),
            "frac_mfma_peak": round(flops / t_op / 1e12 / BF16_PEAK_TFLOPS, 4),
            "config": {"workload": "C4 gdn2 chunkwise forward (training, workspace kept) + backward",
                       "B": B, "T": T, "H": H, "d_k": K, "d_v": V, "chunk": TRAIN["C"],
                       "dtype": "bf16 q,k,v,b,w,dO; fp32 g; fp32 accumulation",
                       "grads": "dq, dk, dv, dg, db, dw"}}


def bench_decode(torch, nat, dev, reps=3, eager_steps=0, variant="plain", N=None, steps=None):
    """Config-2 decode steps in one HIP graph.  ``variant``: "plain" (state [N,H,K,V] in place),
    "pooled" (the states live in a pool of 2N slots addressed through int32
    ssm_state_indices, updated in place) or "transposed" ([N,H,V,K] states).  ``N`` and
    ``steps`` override config 2's 64 sequences and 1024 steps (the line whose state does
    not fit the 256 MB MALL uses N = 256)."""
    H, K, V = (DECODE[x] for x in ("H", "K", "V"))
    N = DECODE["N"] if N is None else N
    S = DECODE["steps"] if steps is None else steps
    F = torch.nn.functional
    gen = torch.Generator(device=dev).manual_seed(2)
    bf = torch.bfloat16
    state = torch.randn(N, H, K, V, generator=gen, device=dev) * 0.02
    rows, slots = N, None
    if variant == "pooled":
        rows = 2 * N
        state = torch.randn(rows, H, K, V, generator=gen, device=dev) * 0.02
        slots = torch.randperm(rows, generator=gen, device=dev)[:N].to(torch.int32)
    elif variant == "transposed":
        state = state.transpose(-1, -2).contiguous()
    q = F.normalize(torch.randn(S, N, 1, H, K, generator=gen, device=dev), dim=-1).to(bf)
    k = F.normalize(torch.randn(S, N, 1, H, K, generator=gen, device=dev), dim=-1).to(bf)
    v = torch.randn(S, N, 1, H, V, generator=gen, device=dev).to(bf)
    beta = torch.sigmoid(torch.randn(S, N, 1, H, 1, generator=gen, device=dev))
    g = (-F.softplus(torch.randn(S, N, 1, H, 1, generator=gen, device=dev) + 2.0)).expand(
        S, N, 1, H, K).contiguous()
    b = beta.expand(S, N, 1, H, K).to(bf).contiguous()
    w = beta.expand(S, N, 1, H, V).to(bf).contiguous()
    o = torch.empty(S, N, 1, H, V, dtype=bf, device=dev)
    lib = nat.load()
    scale = K**-0.5
    sz_k, sz_v, sz_g = N * H * K * 2, N * H * V * 2, N * H * K * 4

    flags = nat.FLAG_L2NORM_QK
    if variant == "pooled":
        flags |= nat.FLAG_INPLACE_FINAL_STATE
    if variant == "transposed":
        flags |= nat.FLAG_TRANSPOSE_STATE
    slab = H * K * V

    def step(i, sh):
        if variant == "plain":
            st = lib.gdn2_recurrent_fwd(
                q.data_ptr() + i * sz_k, k.data_ptr() + i * sz_k, v.data_ptr() + i * sz_v,
                g.data_ptr() + i * sz_g, b.data_ptr() + i * sz_k, w.data_ptr() + i * sz_v,
                nat.DTYPE_BF16, nat.DTYPE_F32, o.data_ptr() + i * sz_v,
                state.data_ptr(), state.data_ptr(), None, None, 0.0, None, N,
                N, 1, H, H, K, V, scale, flags, sh)
        else:
            st = lib.gdn2_recurrent_fwd_ex(
                q.data_ptr() + i * sz_k, k.data_ptr() + i * sz_k, v.data_ptr() + i * sz_v,
                g.data_ptr() + i * sz_g, b.data_ptr() + i * sz_k, w.data_ptr() + i * sz_v,
                nat.DTYPE_BF16, nat.DTYPE_F32, o.data_ptr() + i * sz_v,
                state.data_ptr(), rows, slab, state.data_ptr(), rows, slab, None, None, 0.0,
                None, N, nat.ptr(slots), nat.DTYPE_I32, 0 if slots is None else N, 1, None,
                nat.DTYPE_I32, N, 1, H, H, K, V, scale, flags, sh)
        nat.check(st, "gdn2_recurrent_fwd")

    if eager_steps:
        sh = torch.cuda.current_stream(dev).cuda_stream
        for i in range(eager_steps):
            step(i, sh)
        torch.cuda.synchronize(dev)
        return None
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for i in range(4):
            step(i, side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sh = torch.cuda.current_stream(dev).cuda_stream
        for i in range(S):
            step(i, sh)
    graph.replay()
    torch.cuda.synchronize(dev)
    times = []
    cur = torch.cuda.current_stream(dev)
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        graph.replay()
        e1.record(cur)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    if not torch.isfinite(state).all() or not torch.isfinite(o.float()).all():
        raise RuntimeError("non-finite decode output")
    us_step = statistics.median(times) * 1e3 / S
    nbytes = decode_bytes(N, H, K, V)
    gbs = nbytes / (us_step * 1e-6) / 1e9
    return dict(us_per_step=round(us_step, 3), steps=S, reps=reps,
                bytes_per_step=nbytes, achieved_GBps=round(gbs, 1),
                frac_hbm_peak=round(gbs / HBM_PEAK_GBS, 4),
                config={"workload": f"C2 decode N{N} H{H} K{K} V{V}, fp32 state in place, {S} steps "
                                    "in one HIP graph", "dtype": "bf16 in / fp32 state",
                        "state": variant, "state_bytes": N * H * K * V * 4})


def copy_ceiling(torch, dev, reps=3, copies=256, N=None):
    """Device-to-device copy of a tensor the size of the C2 state (67.1 MB read + 67.1 MB
    written; N sequences' states with ``N``), `copies` back to back in one HIP graph: the
    practical read+write bandwidth the decode step is compared with."""
    H, K, V = (DECODE[x] for x in ("H", "K", "V"))
    N = DECODE["N"] if N is None else N
    src = torch.randn(N, H, K, V, device=dev)
    dst = torch.empty_like(src)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(3):
            dst.copy_(src)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(copies):
            dst.copy_(src)
    graph.replay()
    torch.cuda.synchronize(dev)
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    us = statistics.median(times) * 1e3 / copies
    nbytes = 2 * src.numel() * 4
    return {"bytes": nbytes, "us_per_copy": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}


def bench_prologue(torch, dev, reps=20):
    """The mixer's prologue and epilogue kernels at config 3's module shape.

    * Prologue: the q/k/v short convolution + SiLU in one launch.
    * Epilogue: the gated RMS norm.
    * Decode step: the fused kernel (conv, gates, recurrence and gated norm in one
      launch) against the separate HIP passes, one token per sequence.
    * Prefill: the chunk op with the gated norm in its scan's output stage against the
      chunk op followed by the norm pass.

    Both are set against the torch ops of the reference module that they replace
    (gdn2.py:395-452). Each is timed as a HIP-graph replay of `reps` calls. The HBM
    bytes are algorithmic: each input read once, each output written once.
    """
    import torch.nn.functional as F

    from qwendopamine_amd import ops

    B, T, H, Dh, W = (PROLOGUE[x] for x in ("B", "T", "H", "Dh", "W"))
    D = H * Dh
    bf = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(5)
    xs = [torch.randn(B, T, D, generator=gen, device=dev).to(bf) for _ in range(3)]
    ws = [(torch.randn(D, 1, W, generator=gen, device=dev) * 0.5).to(bf) for _ in range(3)]
    o = torch.randn(B, T, H, Dh, generator=gen, device=dev).to(bf)
    z = torch.randn(B, T, H, Dh, generator=gen, device=dev).to(bf)
    nw = torch.randn(Dh, generator=gen, device=dev).to(bf)

    def conv_hip():
        ops.short_convolution(xs, ws, None, None, output_final_state=True)

    def conv_torch():
        for x, w in zip(xs, ws):
            xt = x.transpose(1, 2)
            F.silu(F.conv1d(xt, w, None, padding=W - 1, groups=D)[..., :T]).transpose(1, 2)
            xt[:, :, -(W - 1):]

    def norm_hip():
        ops.gated_rmsnorm(o, z, nw, 1e-5)

    def norm_torch():
        (o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + 1e-5) * nw) * F.silu(z)

    def timed(fn):
        # `reps` calls captured in one HIP graph: the replay times the kernels,
        # not the Python launch path of each call.
        with torch.no_grad():
            side = torch.cuda.Stream(dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                for _ in range(3):
                    fn()
            torch.cuda.current_stream(dev).wait_stream(side)
            torch.cuda.synchronize(dev)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(reps):
                    fn()
            graph.replay()
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) * 1e3 / reps

    # Decode step at the same module shape (one token for each of the B sequences): the
    # fused kernel (conv + gates + recurrence + gated norm, caches and state updated in
    # place) against the three separate HIP passes it replaces.
    yd = torch.randn(B, 7 * D, generator=gen, device=dev).to(bf)
    qr, kr, vr, bl, wl, gr, zd = yd.split(D, dim=-1)
    caches = [torch.randn(B, D, W - 1, generator=gen, device=dev).to(bf) for _ in range(3)]
    state = torch.randn(B, H, Dh, Dh, generator=gen, device=dev) * 0.05
    A_log = torch.log(torch.rand(H, generator=gen, device=dev) * 15 + 1)
    dt_bias = torch.randn(H * Dh, generator=gen, device=dev) * 0.5
    sp = lambda t: t.view(B, 1, H, Dh)  # noqa: E731

    def dec_fused():
        ops.decode_step_fused([qr, kr, vr], ws, None, caches, gr, bl, wl, state, zd, nw, 1e-5, num_heads=H,
                              head_dim=Dh, A_log=A_log, dt_bias=dt_bias, update_cache_in_place=True)

    def dec_separate():
        (q, k, v), _ = ops.short_convolution([qr.unsqueeze(1), kr.unsqueeze(1), vr.unsqueeze(1)], ws, None,
                                             caches, True, out_caches=caches)
        od, _ = ops.fused_recurrent_gdn2_fwd(sp(q), sp(k), sp(v), sp(gr), sp(bl), sp(wl), A_log=A_log,
                                             dt_bias=dt_bias, initial_state=state, inplace_final_state=True,
                                             use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                                             bw_logits=True)
        ops.gated_rmsnorm(od, sp(zd), nw, 1e-5)

    # Prefill at the same shape: the chunk op (in-kernel gate, b / w logits) followed by the
    # gated norm, against the chunk op with the norm in its scan's output stage.
    pq, pk, pv, pf, pb, pw = (torch.randn(B, T, H, Dh, generator=gen, device=dev).to(bf) for _ in range(6))
    pkw = dict(use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, A_log=A_log, dt_bias=dt_bias,
               bw_logits=True)

    def pre_separate():
        op_, _ = ops.chunk_gdn2(pq, pk, pv, pf, pb, pw, output_final_state=True, **pkw)
        ops.gated_rmsnorm(op_, z, nw, 1e-5)

    def pre_fused():
        ops.chunk_gdn2_gated_norm(pq, pk, pv, pf, pb, pw, z, nw, 1e-5, output_final_state=True, **pkw)

    # Prefill from the raw projections (q / k / v as column ranges of one projection output,
    # as the module holds them): the convolution pass then the chunk op, against the chunk op
    # that convolves q / k / v itself.  Both follow with the gated norm pass (B4 x 16 heads is
    # below the sequence-head count where the module fuses the norm).
    yr = torch.randn(B, T, 3 * D, generator=gen, device=dev).to(bf)
    rq, rk, rv = yr[..., :D], yr[..., D:2 * D], yr[..., 2 * D:]

    def pconv_separate():
        (q, k, v), _ = ops.short_convolution([rq, rk, rv], ws, None, None, True)
        op_, _ = ops.chunk_gdn2(q.view(B, T, H, Dh), k.view(B, T, H, Dh), v.view(B, T, H, Dh), pf, pb, pw,
                                output_final_state=True, **pkw)
        ops.gated_rmsnorm(op_, z, nw, 1e-5)

    def pconv_fused():
        op_, _ = ops.chunk_gdn2_conv(rq, rk, rv, ws, pf, pb, pw, num_heads=H, output_final_state=True, **pkw)
        ops.gated_rmsnorm(op_, z, nw, 1e-5)

    # The same call with the decay gate's inputs as a GatedDeltaNet2 of this shape makes them
    # (its f_proj of random hidden states, its A_log / dt_bias init).  The random logits above
    # with decay rates up to 16 put most 16-token decay spans beyond 2^115, where the diagonal
    # blocks take the slower quarter-referred and exact pair paths; the module's init puts none
    # there.  Both are reported.
    from qwendopamine_amd import GatedDeltaNet2

    torch.manual_seed(3)
    gmod = GatedDeltaNet2(hidden_size=D, num_heads=H, head_dim=Dh).to(dev, bf).eval()
    with torch.no_grad():
        mf = gmod.f_proj(torch.randn(B, T, D, generator=gen, device=dev).to(bf)).view(B, T, H, Dh)
    mkw = dict(pkw, A_log=gmod.A_log.detach().float(), dt_bias=gmod.dt_bias.detach().float())
    del gmod

    def pconv_fused_module():
        op_, _ = ops.chunk_gdn2_conv(rq, rk, rv, ws, mf, pb, pw, num_heads=H, output_final_state=True, **mkw)
        ops.gated_rmsnorm(op_, z, nw, 1e-5)

    def wide_fraction(f, kw):
        with torch.no_grad():
            gl = ops.gate_activation(f.float(), kw["A_log"], kw["dt_bias"], None)
            span = -(gl.view(B, T // 16, 16, H, Dh).sum(2)) / math.log(2.0)
        return round(float((span > 115).float().mean()), 4)

    # Training: forward + backward of the q / k / v convolutions and of the gated norm, on the
    # HIP kernels (autograd functions) against torch's autograd through the reference's ops.
    xg = [x.detach().clone().requires_grad_(True) for x in xs]
    wg = [w.detach().clone().requires_grad_(True) for w in ws]
    dyc = torch.randn(B, T, D, generator=gen, device=dev).to(bf)
    og, zg = o.detach().clone().requires_grad_(True), z.detach().clone().requires_grad_(True)
    nwg = nw.detach().clone().requires_grad_(True)
    dyn = torch.randn(B, T, H, Dh, generator=gen, device=dev).to(bf)

    def conv_train_hip():
        for x, w in zip(xg, wg):
            ops.short_conv_autograd(x, w, None, "silu").backward(dyc)

    def conv_train_torch():
        for x, w in zip(xg, wg):
            F.silu(F.conv1d(x.transpose(1, 2), w, None, padding=W - 1, groups=D)[..., :T]).transpose(1, 2) \
                .backward(dyc)

    def norm_train_hip():
        ops.gated_rmsnorm_autograd(og, zg, nwg, 1e-5).backward(dyn)

    def norm_train_torch():
        (og * torch.rsqrt(og.pow(2).mean(-1, keepdim=True) + 1e-5) * nwg * F.silu(zg)).backward(dyn)

    def eager(fn, reps_=10):
        for _ in range(3):
            fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps_):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) * 1e3 / reps_

    train_t = {k: eager(f) for k, f in (("conv_hip", conv_train_hip), ("conv_torch", conv_train_torch),
                                         ("norm_hip", norm_train_hip), ("norm_torch", norm_train_torch))}

    conv_bytes = 6 * B * T * D * 2
    norm_bytes = 3 * B * T * H * Dh * 2
    # fused decode: state read + write, raw q/k/v/g/b/w/z rows, conv caches read + write,
    # conv weights, normalised output
    dec_bytes = 2 * B * H * Dh * Dh * 4 + 7 * B * D * 2 + 2 * 3 * B * D * (W - 1) * 2 + 3 * D * W * 2 + B * D * 2
    # Floors of a one-launch decode step in the same graph replay: a launch that does
    # (almost) nothing, and one elementwise pass that reads and writes the decode's
    # state once (1 MB at this shape), torch's kernels.
    tiny = torch.zeros(64, device=dev)
    state_copy = state.clone()

    def floor_launch():
        tiny.add_(1.0)

    def floor_state():
        state_copy.mul_(1.0)

    t = {k: timed(f) for k, f in (("conv", conv_hip), ("conv_torch", conv_torch),
                                  ("norm", norm_hip), ("norm_torch", norm_torch),
                                  ("floor_launch", floor_launch), ("floor_state", floor_state),
                                  ("dec_fused", dec_fused), ("dec_separate", dec_separate),
                                  ("pre_fused", pre_fused), ("pre_separate", pre_separate),
                                  ("pconv_fused", pconv_fused), ("pconv_separate", pconv_separate),
                                  ("pconv_fused_module", pconv_fused_module))}
    return {
        "config": {"workload": "C3 module shape: B4 T2048, q/k/v 1024 channels, conv width 4; "
                               "norm over 16 heads x 64", "dtype": "bf16"},
        "short_conv_qkv": {"us": round(t["conv"], 2), "torch_us": round(t["conv_torch"], 2),
                           "algorithmic_bytes": conv_bytes,
                           "achieved_GBps": round(conv_bytes / (t["conv"] * 1e-6) / 1e9, 1),
                           "frac_hbm_peak": round(conv_bytes / (t["conv"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "gated_rmsnorm": {"us": round(t["norm"], 2), "torch_us": round(t["norm_torch"], 2),
                          "algorithmic_bytes": norm_bytes,
                          "achieved_GBps": round(norm_bytes / (t["norm"] * 1e-6) / 1e9, 1),
                          "frac_hbm_peak": round(norm_bytes / (t["norm"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "decode_step": {"workload": f"B{B} one token, {H} heads x {Dh}, conv caches and state in place",
                        "fused_us": round(t["dec_fused"], 2), "separate_hip_us": round(t["dec_separate"], 2),
                        "algorithmic_bytes": dec_bytes,
                        "achieved_GBps": round(dec_bytes / (t["dec_fused"] * 1e-6) / 1e9, 1),
                        "floor_launch_us": round(t["floor_launch"], 2),
                        "floor_state_rw_us": round(t["floor_state"], 2)},
        "training_fwd_bwd": {"workload": "forward + backward, eager (autograd), same shapes",
                             "short_conv_qkv_us": round(train_t["conv_hip"], 1),
                             "short_conv_qkv_torch_us": round(train_t["conv_torch"], 1),
                             "gated_rmsnorm_us": round(train_t["norm_hip"], 1),
                             "gated_rmsnorm_torch_us": round(train_t["norm_torch"], 1)},
        "prefill_norm": {"workload": f"B{B} T{T}, {H} heads x {Dh}: chunk op + gated norm",
                         "fused_us": round(t["pre_fused"], 2), "separate_hip_us": round(t["pre_separate"], 2)},
        "prefill_conv": {"workload": f"B{B} T{T}, {H} heads x {Dh}: q/k/v convolutions + chunk op + gated norm, "
                                     "from the raw projections",
                         "fused_us": round(t["pconv_fused"], 2), "separate_hip_us": round(t["pconv_separate"], 2),
                         "hbm_bytes_removed": conv_bytes,
                         "gate_inputs": "random logits, decay rates exp(A_log) in [1, 16]",
                         "wide_span_fraction": wide_fraction(pf, pkw),
                         "fused_module_gates_us": round(t["pconv_fused_module"], 2),
                         "module_gates_wide_span_fraction": wide_fraction(mf, mkw)},
    }


def bench_e2e(torch, dev, n_prompt=2048, n_new=256, batch=4):
    """Config 3 end to end: the hybrid decoder host (qwendopamine_amd.hybrid, 24 layers,
    18 gdn2 + 6 attention, about 0.68 B parameters, random init, bf16) prefills
    `batch` random prompts of `n_prompt` tokens, then decodes `n_new` tokens greedily.

    * Prefill: eager (the gdn2 layers run the chunk kernels).
    * Decode: the step is captured once as a HIP graph and replayed (the gdn2 layers run
      the decode kernel).
    * The first decode step (eager, before capture) is timed separately.
    * The reported rates count prompt tokens for prefill and generated tokens for decode;
      e2e counts both over the total time.
    """
    from qwendopamine_amd.hybrid import GreedyDecoder, HybridConfig, HybridDecoder

    torch.manual_seed(3)
    cfg = HybridConfig.c3()
    model = HybridDecoder(cfg).to(dev, torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(3)
    prompt = torch.randint(0, cfg.vocab_size, (batch, n_prompt), generator=gen, device=dev)
    dec = GreedyDecoder(model, use_graph=True)

    def ev():
        return torch.cuda.Event(enable_timing=True)

    # Warm-up run at the full prompt length (library handles, kernel selection, graph
    # capture, and the allocator's blocks for every prefill buffer, which a shorter
    # warm-up leaves to the timed prefill), then the timed run.
    dec.generate(prompt, 4)
    torch.cuda.synchronize(dev)
    e = [ev() for _ in range(4)]
    t0 = time.perf_counter()
    e[0].record()
    dec.prefill(prompt, n_new)
    e[1].record()
    dec.step()  # eager first step + capture
    e[2].record()
    for _ in range(n_new - 2):
        dec.step()
    e[3].record()
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    t_pre, t_first, t_dec = (e[i].elapsed_time(e[i + 1]) for i in range(3))
    n_rep = n_new - 2
    total_ms = t_pre + t_first + t_dec
    last_tok = dec.tok.clone()
    check = e2e_check(torch, dec, prompt, n_new, cfg.vocab_size)
    check["timed_run_last_tokens_in_range"] = bool(((last_tok >= 0) & (last_tok < cfg.vocab_size)).all())
    if not (check["timed_run_last_tokens_in_range"] and check["logits_finite"] and check["tokens_in_range"]
            and check["graph_equals_eager"]):
        raise RuntimeError(f"config-3 decode check failed: {check}")
    # HBM bytes one decode step must read (and write): every weight but the embedding
    # table (of which the batch's rows are read), the attention layers' KV caches up to
    # the current position (mean over the timed steps), and the gdn2 layers' recurrent
    # states and conv caches (read and written in place).
    io = next(model.parameters()).element_size()
    n_gdn2 = sum(cfg.is_gdn2(i) for i in range(cfg.n_layer))
    n_attn = cfg.n_layer - n_gdn2
    hv = int(cfg.head_size * cfg.expand_v)
    weights = sum(p.numel() * p.element_size() for n, p in model.named_parameters()
                  if not n.startswith("wte.")) + batch * cfg.n_embd * io
    pos_mean = n_prompt + 1 + (n_new - 2) / 2.0
    kv = int(n_attn * 2 * batch * cfg.n_query_groups * pos_mean * cfg.head_size * io)
    states = n_gdn2 * batch * cfg.n_head * cfg.head_size * hv * 4 * 2
    convs = n_gdn2 * batch * cfg.n_head * (2 * cfg.head_size + hv) * (cfg.conv_size - 1) * io * 2
    step_bytes = weights + kv + states + convs
    step_s = t_dec / n_rep * 1e-3
    return {
        "config": {"workload": "C3 hybrid decoder, prefill B4 x 2048 then greedy decode 256",
                   "layers": "24 (18 gdn2 + 6 attention)", "hidden": cfg.n_embd,
                   "heads": f"{cfg.n_head} x {cfg.head_size}", "ffn": cfg.intermediate_size,
                   "vocab": cfg.vocab_size, "params": sum(p.numel() for p in model.parameters()),
                   "dtype": "bf16", "data": "random init, random token ids"},
        "prefill_ms": round(t_pre, 3),
        "prefill_tokens_per_s": round(batch * n_prompt / (t_pre * 1e-3), 1),
        "decode_first_step_ms": round(t_first, 3),
        "decode_ms_per_step": round(t_dec / n_rep, 4),
        "decode_tokens_per_s": round(batch * n_rep / (t_dec * 1e-3), 1),
        "e2e_tokens_per_s": round(batch * (n_prompt + n_new) / (total_ms * 1e-3), 1),
        "wall_s": round(wall, 3),
        "decode_step_bytes": {"weights": weights, "kv_cache": kv, "gdn2_states": states,
                              "gdn2_conv_caches": convs, "total": step_bytes},
        "decode_achieved_GBps": round(step_bytes / step_s / 1e9, 1),
        "decode_frac_hbm_peak": round(step_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
        "check": check,
    }


def e2e_check(torch, dec, prompt, n_new, vocab, n_eager=32):
    """Untimed checks of the config-3 decode: a graph run over all ``n_new`` steps with
    the logits kept (every step's logits finite, every token in range), and an eager run
    of the first ``n_eager`` steps that must give the graph run's tokens."""
    from qwendopamine_amd.hybrid import GreedyDecoder

    runs = {}
    for use_graph, n in ((True, n_new), (False, n_eager)):
        d = GreedyDecoder(dec.model, use_graph=use_graph, keep_logits=True)
        toks = [d.prefill(prompt, n_new).clone()]
        finite = [torch.isfinite(d.logits).all()]
        for _ in range(n - 1):
            toks.append(d.step().clone())
            finite.append(torch.isfinite(d.logits).all())
        torch.cuda.synchronize()
        runs[use_graph] = (torch.cat(toks, 1), bool(torch.stack(finite).all()))
    tg, fg = runs[True]
    te, fe = runs[False]
    return {"steps_checked": n_new, "logits_finite": fg and fe,
            "tokens_in_range": bool(((tg >= 0) & (tg < vocab)).all()),
            "eager_steps_compared": n_eager, "graph_equals_eager": bool(torch.equal(tg[:, :n_eager], te))}


def traffic_probe(torch, nat, dev):
    """Short run for the rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE): first three
    kernels whose bytes are known, which calibrate the counters -- a 256 MiB
    device-to-device copy (256 MiB read + written), a 1 GiB fill (written only) and a
    sum over the same 1 GiB (read only) -- then two prefill ops, eight eager decode
    steps, eight eager decode steps with the state beyond the MALL (N = 256) and two
    training forward + backward steps."""
    a = torch.empty(64 << 20, dtype=torch.float32, device=dev).uniform_()
    c = torch.empty_like(a)
    c.copy_(a)
    torch.cuda.synchronize(dev)
    del a, c
    big = torch.empty(256 << 20, dtype=torch.float32, device=dev)
    big.fill_(1.0)
    total = big.sum()
    torch.cuda.synchronize(dev)
    del big, total
    bench_prefill(torch, nat, dev, steps=2, warmup=0)
    bench_decode(torch, nat, dev, eager_steps=8)
    bench_decode(torch, nat, dev, eager_steps=8, N=DECODE_BEYOND_MALL["N"], steps=8)
    bench_train(torch, nat, dev, steps=2, warmup=0)
    print("traffic probe done", flush=True)


def _profile_value(name, key):
    """Integer ``key: value`` line of a committed counter summary under profiles/ (None if absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith(key + ":"):
                    return int(ln.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def measured_traffic():
    """HBM bytes per prefill op from the committed FETCH_SIZE / WRITE_SIZE summary."""
    return _profile_value("chunk_fwd_C1_traffic.md", "traffic_bytes_per_op")


def measured_mfma_flop():
    """bf16 MFMA FLOP executed per prefill op from the committed SQ counter summary."""
    return _profile_value("chunk_kernels_mfma_counters.md", "executed_bf16_mfma_flop_per_prefill_op")


def _cpu_model():
    """``lscpu`` model name of this host (``/proc/cpuinfo`` as a fallback)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            if ln.strip().startswith("Model name:"):
                return ln.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, runs=5):
    """One warm-up call, then the median of ``runs`` timed calls (seconds)."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(torch, inputs):
    """The CPU baselines of BASELINE's plan, on this host's cores (a reported baseline only).

    * Config 0 (fp32 B1 T512 H4 K=V=64, seed 0), the whole workload: the PyTorch CPU
      restatement of the reference recurrence (``oracle/gdn2_torch.recurrent_fwd``), its
      safe chunkwise form (``chunk_fwd``) and the C port (``oracle/gdn2_cpu.c``), each on
      every core of the affinity mask and on one thread; median of 5 runs after a warm-up.
    * Config 1 (the GPU workload, fp32 recurrence on the same bf16-rounded inputs): the C
      port on every core over the full batch, and on one thread over a sample (sequence 0,
      all 16 heads, its first 1024 tokens); median of 5 runs after a warm-up.
    ``value`` is the config-1 figure on every core, in tokens (all heads) per second.
    """
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cpu_lib
    from oracle import gdn2_oracle as orc
    from oracle import gdn2_torch

    cores = len(os.sched_getaffinity(0))
    prev_threads = torch.get_num_threads()
    names = ("q", "k", "v", "g", "b", "w")

    # ---- config 0
    c0 = orc.make_inputs(0, 1, 512, 4, 64, 64)
    c0_np = [c0[n].astype("float32") for n in names]
    c0_t = [torch.from_numpy(a) for a in c0_np]
    B0, T0, H0 = 1, 512, 4
    c0_res = {}
    for label, nth in (("all_cores", cores), ("one_thread", 1)):
        torch.set_num_threads(nth)
        r = {}
        r["torch_recurrent"] = B0 * T0 / _median_time(lambda: gdn2_torch.recurrent_fwd(*c0_t))
        r["torch_chunk"] = B0 * T0 / _median_time(lambda: gdn2_torch.chunk_fwd(*c0_t))
        r["c_port"] = B0 * T0 / _median_time(lambda: cpu_lib.recurrent_fwd_f32(*c0_np, nthreads=nth))
        c0_res[label] = {k: round(v, 1) for k, v in r.items()}
    torch.set_num_threads(prev_threads)

    # ---- config 1
    q, k, v, g, b, w = (x.float().cpu().numpy() for x in inputs)
    B, T, H, K = q.shape
    full = (q, k, v, g, b, w)
    t_all = _median_time(lambda: cpu_lib.recurrent_fwd_f32(*full, nthreads=cores))
    Ts = min(T, 1024)
    sample = tuple(x[:1, :Ts] for x in full)
    t_one = _median_time(lambda: cpu_lib.recurrent_fwd_f32(*sample, nthreads=1))
    model = _cpu_model()
    used = min(cores, B * H)
    return {
        "value": round(B * T / t_all, 1), "unit": "tokens/s", "cores": used, "kind": "port",
        "sample": (f"config 1 full batch (B{B} T{T} H{H} K{K}), fp32 token recurrence of the C port "
                   f"(oracle/gdn2_cpu.c, OpenMP over the {B * H} sequence-heads, {cores} threads "
                   f"requested), median of 5 runs of {t_all:.3f} s after a warm-up; cpu: {model}"),
        "cpu_model": model,
        "affinity_cores": cores,
        "one_thread": {"value": round(Ts / t_one, 1), "unit": "tokens/s",
                       "sample": f"sequence 0, all {H} heads, first {Ts} tokens; median of 5 "
                                 f"runs of {t_one:.3f} s"},
        "config0": {"unit": "tokens/s", "workload": "fp32 B1 T512 H4 K=V=64, seed 0 (whole workload)",
                    "all_cores_threads": cores, **c0_res,
                    "note": "config 0 has 4 sequence-heads, so the C port keeps at most 4 threads busy"},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train", action="store_true")
    ap.add_argument("--no-prologue", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-3 end-to-end decoder run")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="short run for rocprofv3 counter passes; prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (--gpus 1); multi-GPU sharding of the "
              "gdn2 path is a design note, not a measured configuration.", file=sys.stderr)
        return 2

    import torch

    from qwendopamine_amd import _native as nat

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    if args.traffic_probe:
        traffic_probe(torch, nat, dev)
        return 0
    P = PREFILL
    res = bench_prefill(torch, nat, dev, args.steps, args.warmup)
    B, T, H, K, V, C = P["B"], P["T"], P["H"], P["K"], P["V"], P["C"]
    tokens = B * T
    ms = res["ms_step"]
    nbytes = prefill_bytes(B, T, H, K, V)
    flops = prefill_flops(B, T, H, K, V, C)
    t_op_ms = res["t_prep_ms"] + res["t_scan_ms"]
    achieved = nbytes / (t_op_ms * 1e-3) / 1e9
    mfma_exec = measured_mfma_flop()
    out = {
        "metric": METRIC,
        "value": round(tokens / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (BASELINE config-1 recipe, seeded)",
        "config": {"workload": "C1 gdn2 chunkwise prefill", "B": B, "T": T, "H": H, "d_k": K,
                   "d_v": V, "chunk": C, "inputs": "bf16 q,k,v,b,w; fp32 g; fp32 state",
                   "l2norm_in_kernel": True, "final_state": True, "parallelism": "single GPU"},
        "roofline": {
            "bound": "hbm",
            "kernel": "gdn2 chunk forward = chunk_prep_kernel + chunk_scan_kernel (one op)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "algorithmic_bytes": nbytes,
            "op_ms": round(t_op_ms, 4),
            "kernels_ms": {"chunk_prep_kernel": round(res["t_prep_ms"], 4),
                           "chunk_scan_kernel": round(res["t_scan_ms"], 4)},
            "mfma": {"algorithmic_flop": flops,
                     "achieved_TFLOPs": round(flops / (t_op_ms * 1e-3) / 1e12, 2),
                     "peak_TFLOPs": BF16_PEAK_TFLOPS,
                     "frac": round(flops / (t_op_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                     "counter_flop": mfma_exec,
                     "counter_frac": (None if mfma_exec is None else
                                      round(mfma_exec / (t_op_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))},
        },
    }
    if not args.no_decode:
        out["decode"] = bench_decode(torch, nat, dev)
        for variant in ("pooled", "transposed"):
            r = bench_decode(torch, nat, dev, variant=variant)
            out["decode"][variant] = {x: r[x] for x in ("us_per_step", "achieved_GBps",
                                                        "frac_hbm_peak")}
        cc = copy_ceiling(torch, dev)
        out["decode"]["copy_ceiling"] = cc
        out["decode"]["frac_copy_ceiling"] = round(out["decode"]["achieved_GBps"] / cc["GBps"], 4)
        # The config-2 state (67 MB) stays in the 256 MB MALL across graph steps; this
        # line's state (268 MB) does not, so its rate is a DRAM rate.
        big = bench_decode(torch, nat, dev, N=DECODE_BEYOND_MALL["N"], steps=DECODE_BEYOND_MALL["steps"])
        cc_big = copy_ceiling(torch, dev, copies=64, N=DECODE_BEYOND_MALL["N"])
        big["copy_ceiling"] = cc_big
        big["frac_copy_ceiling"] = round(big["achieved_GBps"] / cc_big["GBps"], 4)
        out["decode"]["beyond_mall"] = big
    if not args.no_train:
        out["train"] = bench_train(torch, nat, dev, max(2, args.steps // 2), 1)
    if not args.no_prologue:
        out["prologue_epilogue"] = bench_prologue(torch, dev)
    if not args.no_e2e:
        out["e2e_c3"] = bench_e2e(torch, dev)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, res["inputs"])
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
