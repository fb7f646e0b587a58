#!/usr/bin/env python3
"""Benchmark of the MI355X KDA backend on one GPU.

Metric: "KDA prefill tokens/s (T=8192,H=16,d=128 bf16) + decode-step HBM GB/s".

* value      : chunkwise prefill throughput (tokens/s) on the long-context
               workload B=1, T=8192, H=16, K=V=128, bf16 inputs, f32 state
               N(0, 0.02), chunk 64 — output and final state are produced.
               One step = one prefill over the whole batch, inputs resident
               in HBM; timed with HIP events over exactly `--steps` steps.
* decode     : the memory-bound decode step at B=256, H=32, K=V=128 with the
               512 MiB f32 state updated in place for 64 consecutive steps,
               reported as algorithmic HBM GB/s.
* roofline   : the prefill's compulsory HBM bytes (q, k, g, v, beta read,
               output written, f32 initial and final state: 170.13 MB at
               this shape) over the dominant kernel's time (per-kernel HIP
               events on the launch stream), against the MI355X HBM peak
               (8 TB/s); `roofline_operator` gives the same bytes over the
               whole operator's time, and the chunk GEMM flops against the
               dense bf16 MFMA peak (2.5 PFLOP/s).
* dropin     : the same prefill and decode through the Python drop-in API
               (kda.chunkwise_kda / kda.recurrent_kda with its validation,
               casts and per-call allocations), not only the C ABI.
* cpu_baseline: the oracle's PyTorch-CPU restatement of the reference path
               (oracle/kda_oracle.py) on a bounded sample of the same
               workload, on the host cores (thread count reported).
* fused_stages: the kernels around the operator (kda.fused) on the same
               shape, as HBM GB/s (not part of `value`).
* prefill_k64: the prefill at the gpu_48gb head shape (K = V = 64).
* prefill_f32: f32 inputs at the prefill shape (the split-bf16 chunk path),
               next to the exact recurrence kernel on the same sequence.
* prefill_configs: the other prefill workloads, B=8 T=1024 H=8 and 4 packed
               documents (65536 tokens) at H=64, tokens/s and roofline.
* decay_fusion: the decay feeding the prefill: gates kernel then chunk
               kernel, against the chunk kernel forming g from the logits.
* backward   : the chunkwise backward (all input gradients) on the prefill
               workload, ms and tokens/s (not part of `value`), with the
               oracle's backward on a T=1024 sample as its CPU baseline.
* cache_reorder: the beam-search reorder of a whole decode cache (8 KDA
               layers at the decode shape) through kda_cache_gather, as HBM
               GB/s, next to the per-tensor index_select it replaces (not part
               of `value`).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (REPO / "kimi-k3-pytorch_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "KDA prefill tokens/s (T=8192,H=16,d=128 bf16) + decode-step HBM GB/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

# long-context prefill workload
P_B, P_T, P_H, P_K, P_V = 1, 8192, 16, 128, 128
# decode workload
D_B, D_H, D_K, D_V, D_STEPS = 256, 32, 128, 128, 64
# Untimed prefill launches before the headline's warm-up steps: the GPU's
# clock ramps up over the first ~10 ms of sustained work (per-step times
# fall from ~131 to ~123 us over the first ~100 prefills and climb back
# after ~1 s idle), so a few warm-up steps leave every timed step on the ramp.
SETTLE_MS = 50.0


PREFILL_KERNELS = ("chunk_map_kernel", "chunk_segment_kernel<summary>", "segment_combine_kernel",
                   "chunk_segment_kernel<output>")
BWD_KERNELS = ("bwd::prep_kernel", "bwd::seg_maps_kernel", "bwd::seg_combine_kernel", "bwd::seg_kernel<run>",
               "bwd::grad_pair_kernel")


def prefill_bytes(B, T, H, K, V, n_state_io=2):
    """Compulsory HBM bytes: q,k,g,v (bf16) + beta + output (bf16) + f32 states in/out."""
    return 2 * B * T * H * (3 * K + V) + 2 * B * T * H + 2 * B * T * H * V + 4 * B * H * K * V * n_state_io


def prefill_flops(B, T, H, K, V, C=64):
    """Causal-counted chunk GEMM flops: 6KV + (3C+1)K + 2(C+1)V per token per head."""
    return B * T * H * (6 * K * V + (3 * C + 1) * K + 2 * (C + 1) * V)


def decode_bytes(B, H, K, V):
    """State read + write (f32) plus the token's q,k,g,v,beta (bf16) and output (bf16)."""
    return 2 * 4 * B * H * K * V + 2 * B * H * (3 * K + V) + 2 * B * H + 2 * B * H * V


def _inputs(B, T, H, K, V, state_std, seed, device):
    import torch

    from tests._inputs import workload

    q, k, v, g, beta, state = workload(B, T, H, K, V, state_std=state_std, seed=seed)
    dev = lambda t: None if t is None else t.to(device).contiguous()  # noqa: E731
    return dev(q), dev(k), dev(v), dev(g), dev(beta), dev(state)


def _settle(fn, ms=SETTLE_MS):
    """Untimed calls of `fn` for `ms` milliseconds of sustained GPU work, so
    that a leg's timed calls run at the settled clock.  Returns the count."""
    import torch

    n = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        n += 10
    return n


def bench_prefill(steps, warmup, shape=(P_B, P_T, P_H, P_K, P_V), settle_ms=0.0):
    import torch

    from kda import _lib

    lib = _lib.load()
    device = torch.device("cuda", 0)
    B, T, H, K, V = shape
    q, k, v, g, beta, s0 = _inputs(B, T, H, K, V, 0.02, 0, device)
    total = B * T
    out = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=device)
    s_out = torch.empty(B, H, K, V, dtype=torch.float32, device=device)
    code = _lib.dtype_code(torch.bfloat16)
    ws_bytes = lib.kda_chunk_fwd_workspace_bytes(B, total, 0, H, K, V, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code,
            s0.data_ptr(), s_out.data_ptr(), 0, out.data_ptr(), None, T, None,
            B, total, H, K, V, ws.data_ptr(), ws_bytes, stream)

    def step():
        _lib.check(lib.kda_chunk_fwd(*args))

    settle = {"ms": settle_ms, "launches": _settle(step, settle_ms) if settle_ms > 0 else 0}
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps

    # per-kernel HIP-event timing on the launch stream
    kms = (ctypes.c_float * 4)()
    nk = ctypes.c_int(0)
    sums = [0.0] * 4
    reps = max(5, min(steps, 20))
    for _ in range(reps):
        _lib.check(lib.kda_chunk_fwd_profiled(*args, kms, ctypes.byref(nk)))
        for i in range(4):
            sums[i] += kms[i]
    per_kernel = {name: sums[i] / reps for i, name in enumerate(PREFILL_KERNELS)}
    if settle_ms > 0:
        return ms, per_kernel, ws_bytes, settle
    return ms, per_kernel, ws_bytes


def bench_decode(warmup):
    import torch

    from kda import _lib

    lib = _lib.load()
    device = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(1)
    state = (torch.randn(D_B, D_H, D_K, D_V, generator=gen) * 0.02).to(device)
    q, k, v, g, beta, _ = _inputs(D_B, D_STEPS, D_H, D_K, D_V, None, 2, device)
    out = torch.empty(D_B, 1, D_H, D_V, dtype=torch.bfloat16, device=device)
    code = _lib.dtype_code(torch.bfloat16)
    stream = torch.cuda.current_stream(device).cuda_stream
    # one token per sequence per step: slice step t out of the [B, 64, H, *] inputs
    steps_in = [tuple(x[:, t:t + 1].contiguous() for x in (q, k, v, g, beta)) for t in range(D_STEPS)]

    def step(t):
        qq, kk, vv, gg, bb = steps_in[t]
        _lib.check(lib.kda_decode_step(qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), gg.data_ptr(), bb.data_ptr(),
                                       code, state.data_ptr(), state.data_ptr(), 0, out.data_ptr(),
                                       D_B, D_H, D_K, D_V, stream))

    _settle(lambda: step(0))
    for t in range(warmup):
        step(t % D_STEPS)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(D_STEPS):
        step(t)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / D_STEPS


def bench_fused(reps=50):
    """The fused stages around the operator on the prefill shape (B=1, T=8192,
    H=16, D=128, bf16): ShortConv + SiLU + L2 norm of one projection, the
    decay and beta gates in one launch, and RMSNorm with the output gate.
    Each is launched `reps` times back to back through the C ABI into
    preallocated outputs, between two HIP events on the launch stream;
    algorithmic bytes = every input read once and every output written once
    (the conv weight and gate parameters, a few KiB, are not counted)."""
    import torch

    from kda import _lib, _prep

    lib = _lib.load()
    device = torch.device("cuda", 0)
    gen = torch.Generator(device=device).manual_seed(7)
    B, T, H, D = P_B, P_T, P_H, P_K
    C = H * D
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=device).to(torch.bfloat16)  # noqa: E731
    x, w, y = rnd(B, T, C), rnd(C, 4), rnd(B, T, C)
    z, zb, a_log, bl = rnd(B, T, H, D), rnd(H, D), torch.zeros(H, device=device), rnd(B, T, H)
    g, alpha, beta = torch.empty_like(z), torch.empty_like(z), torch.empty_like(bl)
    o, nw, gl, out = rnd(B, T, H, D), rnd(H, D), rnd(B, T, C), rnd(B, T, H, D)
    bf, el = _lib.dtype_code(torch.bfloat16), 2
    stream = _prep.stream(device)
    cases = {
        "conv_silu_l2norm": (
            lambda: lib.kda_conv_silu_fwd(x.data_ptr(), w.data_ptr(), None, None, y.data_ptr(), None, None,
                                          B, T, C, 4, D, 1, 1e-6, bf, stream),
            2 * B * T * C * el),
        "decay_and_beta_gates": (
            lambda: lib.kda_gates_fwd(z.data_ptr(), zb.data_ptr(), a_log.data_ptr(), -5.0, g.data_ptr(),
                                      alpha.data_ptr(), bl.data_ptr(), beta.data_ptr(), B * T, H, D, bf, stream),
            3 * B * T * H * D * el + 2 * B * T * H * el),
        "rmsnorm_output_gate": (
            lambda: lib.kda_rmsnorm_gate_fwd(o.data_ptr(), nw.data_ptr(), 1, gl.data_ptr(), out.data_ptr(),
                                             B * T, H, D, 1e-6, bf, stream),
            3 * B * T * H * D * el),
    }
    res = {}
    for name, (fn, nbytes) in cases.items():
        _settle(lambda: _lib.check(fn()))
        for _ in range(3):
            _lib.check(fn())
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        kernel = {"conv_silu_l2norm": "conv_silu_kernel", "decay_and_beta_gates": "gates_kernel",
                  "rmsnorm_output_gate": "rmsnorm_gate_kernel"}[name]
        res[name] = {"ms": round(ms, 5), "algorithmic_bytes": nbytes, "achieved_gbs": round(gbs, 1),
                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel)}
    return res


def bench_fused_backward(reps=20):
    """The backward of the fused stages on the prefill shape (B=1, T=8192,
    H=16, D=128, bf16), each through the C ABI `reps` times between two HIP
    events: the ShortConv + SiLU + L2 norm backward of one projection (kernel
    size 4, bias, weight and bias gradients), the decay and beta gates'
    backward (decay bias and A_log gradients), and the RMSNorm x output gate
    backward (per-head weight gradient).  Algorithmic bytes = the activations
    and incoming gradients read once and the input gradients written once
    (parameters and their f32 gradient accumulators, a few KiB, not counted)."""
    import torch

    from kda import _lib, _prep

    lib = _lib.load()
    device = torch.device("cuda", 0)
    gen = torch.Generator(device=device).manual_seed(11)
    B, T, H, D = P_B, P_T, P_H, P_K
    C, rows = H * D, P_B * P_T
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=device).to(torch.bfloat16)  # noqa: E731
    f32 = lambda *shape: torch.zeros(*shape, device=device)  # noqa: E731
    x, w, cb, dy, dx = rnd(B, T, C), 0.3 * rnd(C, 4), 0.1 * rnd(C), rnd(B, T, C), rnd(B, T, C)
    cdw, cdb = f32(C, 4), f32(C)
    z, zb, a_log, dg, dz = rnd(rows, H, D), rnd(H, D), torch.zeros(H, device=device), rnd(rows, H, D), rnd(rows, H, D)
    bl, dbt, dbl = rnd(rows, H), rnd(rows, H), rnd(rows, H)
    gdzb, gdal = f32(H, D), f32(H)
    o, nw, gl, do, dox, dgl = rnd(rows, H, D), rnd(H, D), rnd(rows, H, D), rnd(rows, H, D), rnd(rows, H, D), \
        rnd(rows, H, D)
    ndw = f32(H, D)
    bf, el = _lib.dtype_code(torch.bfloat16), 2
    stream = _prep.stream(device)
    cases = {
        "conv_silu_l2norm_bwd": (
            "conv_silu_bwd_kernel",
            lambda: lib.kda_conv_silu_bwd(x.data_ptr(), w.data_ptr(), cb.data_ptr(), None, None, dy.data_ptr(), None,
                                          dx.data_ptr(), None, cdw.data_ptr(), cdb.data_ptr(), B, T, C, 4, D, 1,
                                          1e-6, bf, stream),
            3 * B * T * C * el),
        "decay_and_beta_gates_bwd": (
            "gates_bwd_kernel",
            lambda: lib.kda_gates_bwd(z.data_ptr(), zb.data_ptr(), a_log.data_ptr(), -5.0, dg.data_ptr(), None,
                                      dz.data_ptr(), gdzb.data_ptr(), gdal.data_ptr(), bl.data_ptr(),
                                      dbt.data_ptr(), dbl.data_ptr(), rows, H, D, bf, stream),
            3 * rows * H * D * el + 3 * rows * H * el),
        "rmsnorm_output_gate_bwd": (
            "rmsnorm_gate_bwd_kernel",
            lambda: lib.kda_rmsnorm_gate_bwd(o.data_ptr(), nw.data_ptr(), 1, gl.data_ptr(), do.data_ptr(),
                                             dox.data_ptr(), dgl.data_ptr(), ndw.data_ptr(), rows, H, D, 1e-6, bf,
                                             stream),
            5 * rows * H * D * el),
    }
    res = {}
    for name, (kernel, fn, nbytes) in cases.items():
        _settle(lambda: _lib.check(fn()))
        for _ in range(3):
            _lib.check(fn())
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": round(ms, 5), "algorithmic_bytes": nbytes, "achieved_gbs": round(gbs, 1),
                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel)}
    return res


def bench_layer_train(reps=5):
    """One KDA layer (d_model 2048 = 16 heads x 128, ShortConv kernel 4, decay
    rank 128, random bf16 weights in the reference's layouts) on B=1, T=8192
    bf16 synthetic hidden states through kda.layer.kda_attention_forward in
    chunkwise mode: the forward alone, and forward + backward of the sum of
    the outputs (every weight and the input requiring gradients), `reps`
    timed calls each after 2 untimed ones, between two HIP events."""
    import math

    import torch

    from kda.layer import KDALayerWeights, kda_attention_forward

    device = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(41)
    H, D, R, B, T = P_H, P_K, 128, P_B, P_T
    dm = H * D
    rnd = lambda *shape, s=0.02: (torch.randn(*shape, generator=gen) * s).to(device, torch.bfloat16)  # noqa: E731
    dt = torch.exp(torch.rand(H, D, generator=gen) * (math.log(0.1) - math.log(0.001)) + math.log(0.001))
    w = dict(num_heads=H, key_head_dim=D, value_head_dim=D,
             q_proj=rnd(dm, dm), k_proj=rnd(dm, dm), v_proj=rnd(dm, dm),
             q_conv=rnd(dm, 4, s=0.3), k_conv=rnd(dm, 4, s=0.3), v_conv=rnd(dm, 4, s=0.3),
             beta_proj=rnd(H, dm), alpha_down=rnd(R, dm), alpha_up=rnd(dm, R),
             b_alpha=(dt + torch.log(-torch.expm1(-dt))).to(device, torch.bfloat16),
             a_log=(0.1 * torch.randn(H, generator=gen)).to(device),
             norm_weight=(1 + 0.1 * torch.randn(H, D, generator=gen)).to(device, torch.bfloat16),
             gate_proj=rnd(dm, dm), output_proj=rnd(dm, dm))
    for k, v in w.items():
        if isinstance(v, torch.Tensor):
            v.requires_grad_()
    weights = KDALayerWeights(**w)
    x = (torch.randn(B, T, dm, generator=gen)).to(device, torch.bfloat16).requires_grad_()

    def fwd():
        with torch.no_grad():
            kda_attention_forward(weights, x, mode="chunkwise")

    def train():
        out = kda_attention_forward(weights, x, mode="chunkwise")
        out.hidden_states.float().sum().backward()

    res = {"workload": f"KDA layer d_model {dm} ({H} heads x {D}), ShortConv 4, decay rank {R}, B={B} T={T} "
                       "bf16, random weights, synthetic hidden states, chunkwise mode"}
    for name, fn in (("forward", fwd), ("forward_backward", train)):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        res[name] = {"ms": round(ms, 4), "tokens_per_s": round(B * T / (ms * 1e-3), 1)}
    return res


def bench_decay_fusion(reps=20):
    """The decay feeding the prefill at the long-context shape, two ways:
    kda_gates_fwd writing g (bf16) followed by kda_chunk_fwd reading it, and
    kda_chunk_fwd_decay forming g from the logits inside the chunk kernel (g
    never written or read: 2 x 33.5 MB less traffic).  `reps` back-to-back
    calls of each through the C ABI, HIP events on the launch stream."""
    import torch

    from kda import _lib, _prep

    lib = _lib.load()
    device = torch.device("cuda", 0)
    q, k, v, _, beta, s0 = _inputs(P_B, P_T, P_H, P_K, P_V, 0.02, 0, device)
    gen = torch.Generator(device=device).manual_seed(11)
    z = torch.randn(P_B, P_T, P_H, P_K, generator=gen, device=device).to(torch.bfloat16)
    zb = (0.5 * torch.randn(P_H, P_K, generator=gen, device=device)).to(torch.bfloat16)
    a_log = torch.zeros(P_H, device=device)
    g = torch.empty_like(z)
    out = torch.empty(P_B, P_T, P_H, P_V, dtype=torch.bfloat16, device=device)
    s1 = torch.empty(P_B, P_H, P_K, P_V, device=device)
    code = _lib.dtype_code(torch.bfloat16)
    total = P_B * P_T
    ws_bytes = lib.kda_chunk_fwd_workspace_bytes(P_B, total, 0, P_H, P_K, P_V, code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    stream = _prep.stream(device)
    tail = (s0.data_ptr(), s1.data_ptr(), 0, out.data_ptr(), None, P_T, None, P_B, total, P_H, P_K, P_V,
            ws.data_ptr(), ws_bytes, stream)

    def two_step():
        _lib.check(lib.kda_gates_fwd(z.data_ptr(), zb.data_ptr(), a_log.data_ptr(), -5.0, g.data_ptr(), None, None,
                                     None, total, P_H, P_K, code, stream))
        _lib.check(lib.kda_chunk_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code,
                                     *tail))

    def fused():
        _lib.check(lib.kda_chunk_fwd_decay(q.data_ptr(), k.data_ptr(), v.data_ptr(), z.data_ptr(), zb.data_ptr(),
                                           a_log.data_ptr(), -5.0, beta.data_ptr(), code, *tail))

    res = {"workload": f"decay logits -> prefill B={P_B} T={P_T} H={P_H} K=V={P_K} bf16, f32 state"}
    for name, fn in (("gates_then_chunk_fwd", two_step), ("chunk_fwd_decay", fused)):
        _settle(fn)
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        res[name] = {"ms": round(ms, 5), "tokens_per_s": round(total / (ms * 1e-3), 1)}
    return res


def bench_backward(reps=10, shape=None, dtype_name="bf16"):
    """The chunkwise backward (kda_chunk_bwd) on the prefill workload (or
    `shape` = (B, T, H, K, V), inputs of `dtype_name`): all input gradients
    and dS0 from upstream gradients of the output and the final state.
    `reps` back-to-back calls through the C ABI into preallocated outputs,
    HIP events on the launch stream."""
    import torch

    from kda import _lib, _prep

    lib = _lib.load()
    device = torch.device("cuda", 0)
    headline = shape is None and dtype_name == "bf16"
    B, T, H, K, V = (P_B, P_T, P_H, P_K, P_V) if shape is None else shape
    dt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype_name]
    q, k, v, g, beta, s0 = _inputs(B, T, H, K, V, 0.02, 0, device)  # bf16 values, f32 state
    q, k, v, g, beta = (t.to(dt) for t in (q, k, v, g, beta))
    gen = torch.Generator(device=device).manual_seed(9)
    d_out = torch.randn(B, T, H, V, generator=gen, device=device).to(dt)
    d_final = torch.randn(B, H, K, V, generator=gen, device=device)
    grads = [torch.empty_like(t) for t in (q, k, v, g, beta)]
    ds0 = torch.empty_like(s0)
    code = _lib.dtype_code(dt)
    nbytes = lib.kda_chunk_bwd_workspace_bytes(B, T, H, K, V, code)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    stream = _prep.stream(device)

    def call():
        _lib.check(lib.kda_chunk_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                                     d_out.data_ptr(), code, s0.data_ptr(), d_final.data_ptr(),
                                     *[t.data_ptr() for t in grads], ds0.data_ptr(), B, T, H, K, V,
                                     ws.data_ptr(), nbytes, stream))

    _settle(call)
    for _ in range(2):
        call()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        call()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    out = {
        "workload": f"chunkwise backward B={B} T={T} H={H} K={K} V={V}, {dtype_name} inputs, f32 accumulation "
                    "(dq, dk, dv, dg, dbeta, dS0)",
        "ms": round(ms, 4),
        "tokens_per_s": round(B * T / (ms * 1e-3), 1),
        "workspace_bytes": nbytes,
    }
    if headline:  # the counter record is of this shape
        per_kernel = [measured_traffic(k) for k in BWD_KERNELS]
        traffic = None if None in per_kernel else sum(per_kernel)
        out["traffic"] = traffic
        out["traffic_gbs"] = None if traffic is None else round(traffic / (ms * 1e-3) / 1e9, 1)
    return out


def bench_cache(layers=8, reps=10):
    """Reorder of a whole decode cache by a random permutation of the batch:
    `layers` KDA layers at the decode shape (f32 state [256, 32, 128, 128],
    three bf16 ShortConv histories [256, 3, 4096], int64 offsets [256]), 40
    tensors in one kda_cache_gather launch into preallocated outputs.
    Algorithmic bytes = every row read once and written once.  The same
    reorder as one torch index_select per tensor (what KDAState.reorder does
    per layer) is timed beside it."""
    import torch

    from kda import _lib, _prep

    lib = _lib.load()
    device = torch.device("cuda", 0)
    B, W = D_B, D_H * D_K
    tensors = []
    for _ in range(layers):
        tensors.append(torch.empty(B, D_H, D_K, D_V, device=device).uniform_())
        tensors += [torch.empty(B, 3, W, device=device, dtype=torch.bfloat16).uniform_() for _ in range(3)]
        tensors.append(torch.arange(B, device=device, dtype=torch.long))
    outs = [torch.empty_like(t) for t in tensors]
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(3)).to(device)
    n = len(tensors)
    src = (ctypes.c_void_p * n)(*[t.data_ptr() for t in tensors])
    dst = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    rows = (ctypes.c_int64 * n)(*[t[0].numel() * t.element_size() for t in tensors])
    status = torch.zeros(1, dtype=torch.int32, device=device)
    stream = _prep.stream(device)
    nbytes = 2 * sum(t.numel() * t.element_size() for t in tensors)

    def native():
        _lib.check(lib.kda_cache_gather(src, dst, rows, n, perm.data_ptr(), B, B, status.data_ptr(), stream))

    def per_tensor():
        for t, o in zip(tensors, outs):
            torch.index_select(t, 0, perm, out=o)

    res = {}
    for name, fn in (("kda_cache_gather", native), ("torch_index_select_per_tensor", per_tensor)):
        _settle(fn)
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": round(ms, 4), "achieved_gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    native()
    torch.cuda.synchronize()
    if int(status.item()) != 0 or not torch.equal(outs[0], tensors[0][perm]):
        raise RuntimeError("cache reorder check failed")
    return {
        "workload": f"reorder of {layers} KDA layers' decode caches, B={B} H={D_H} K=V={D_K} f32 states + "
                    f"3 bf16 ShortConv histories [B,3,{W}] + offsets ({n} tensors), random permutation",
        "algorithmic_bytes": nbytes,
        "traffic": measured_traffic("cache_gather_kernel"),
        **res,
    }


def cpu_threads():
    """Threads for the CPU baseline: the cores this process may run on, capped by
    OMP_NUM_THREADS when the environment sets it (the share of the host that a
    one-GPU job is given).  The host's total count is reported beside it."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        avail = min(avail, int(env))
    return max(1, avail)


def cpu_baseline(prefill_sample_t=2048, decode_sample_b=32, repeats=3):
    """The oracle's CPU restatement, timed like benchmarks/benchmark_kda.py:30-40
    (one warm-up, then min over repeats of time.perf_counter, inference_mode)."""
    import torch

    from oracle import kda_oracle as ora
    from tests._inputs import workload

    threads = cpu_threads()
    torch.set_num_threads(threads)

    def timed(fn):
        with torch.inference_mode():
            fn()
            best = float("inf")
            for _ in range(repeats):
                t0 = time.perf_counter()
                fn()
                best = min(best, time.perf_counter() - t0)
        return best

    q, k, v, g, beta, s0 = workload(1, prefill_sample_t, P_H, P_K, P_V, state_std=0.02, seed=0)
    t_pre = timed(lambda: ora.chunkwise(q, k, v, g, beta, s0, chunk_size=64, secondary_tile_size=16))
    qd, kd, vd, gd, bd, _ = workload(decode_sample_b, 1, D_H, D_K, D_V, seed=2)
    sd = torch.randn(decode_sample_b, D_H, D_K, D_V) * 0.02
    t_dec = timed(lambda: ora.recurrent(qd, kd, vd, gd, bd, sd))
    bwd_t = prefill_sample_t // 2
    qb, kb, vb, gb, bb, sb = (t.float() for t in workload(1, bwd_t, P_H, P_K, P_V, state_std=0.02, seed=0))
    gen = torch.Generator().manual_seed(9)
    d_out, d_final = torch.randn(1, bwd_t, P_H, P_V, generator=gen), torch.randn(1, P_H, P_K, P_V, generator=gen)
    t_bwd = timed(lambda: ora.chunkwise_backward(qb, kb, vb, gb, bb, sb, d_out, d_final))
    return {
        "prefill": {
            "value": prefill_sample_t / t_pre, "unit": "tokens/s", "cores": threads, "kind": "port",
            "host_cpu_count": os.cpu_count(),
            "sample": f"oracle chunkwise (torch CPU, f32 work) B=1 T={prefill_sample_t} H={P_H} K=V=128 bf16, "
                      f"min of {repeats} after 1 warm-up",
        },
        "decode": {
            "value": decode_bytes(decode_sample_b, D_H, D_K, D_V) / t_dec / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle recurrent one step (torch CPU) B={decode_sample_b} H={D_H} K=V=128, "
                      f"min of {repeats} after 1 warm-up",
        },
        "backward": {
            "value": bwd_t / t_bwd, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle chunkwise_backward (torch CPU, f32) B=1 T={bwd_t} H={P_H} K=V=128, "
                      f"min of {repeats} after 1 warm-up",
        },
    }


COUNTERS_FILE = REPO / "profiles" / "kernel_counters.json"
CSRC = REPO / "kimi-k3-pytorch_amd" / "csrc"


def _sha16(data):
    import hashlib

    return hashlib.sha256(data).hexdigest()[:16]


def source_hashes():
    """Hash of every HIP/C++ source and header the kernels are built from."""
    files = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")) + list(CSRC.glob("*.h")))
    return {f.name: _sha16(f.read_bytes()) for f in files}


def kernel_source(key):
    """The source file that defines the kernel behind a counter key (None for
    kernels that are not this library's)."""
    import re

    base = key.split("::")[-1].split("<")[0]
    for f in sorted(CSRC.glob("*.hip")):
        if re.search(r"__global__[^;{]*\b" + re.escape(base) + r"\s*\(", f.read_text()):
            return f.name
    return None


def kernel_key(name):
    """Short, stable key of a rocprofv3 kernel name (mangled or demangled):
    the kernel's identifier, the phase of chunk_segment_kernel, and a
    `bwd::` prefix for the backward's kernels."""
    import re

    if name.startswith("_Z"):
        # length-prefixed identifiers of the mangled name: the first *_kernel one
        ids, i = [], 2
        while i < len(name):
            m = re.match(r"(\d+)", name[i:])
            if m is None:
                i += 1
                continue
            n = int(m.group(1))
            start = i + len(m.group(1))
            ids.append(name[start:start + n])
            i = start + n
        base = next((x for x in ids if x.endswith("_kernel")), name)
        mode = re.search(r"Li(\d)E", name)
    else:
        found = re.search(r"([A-Za-z_][A-Za-z0-9_]*_kernel)\b", name) or re.search(r"([A-Za-z_]\w*kernel\w*)", name)
        base = found.group(1) if found else name
        mode = re.search(r",\s*(\d)\s*>", name)
    key = base
    if key == "chunk_segment_kernel":
        key += {"0": "<summary>", "1": "<output, prepared>", "2": "<output>"}.get(mode.group(1) if mode else "", "")
    if key == "seg_kernel":  # the segmented state scans: value-column maps, transition maps, rerun
        key += {"0": "<maps Q>", "1": "<maps P>", "2": "<run>"}.get(mode.group(1) if mode else "", "")
    if "bwd" in name and not key.startswith("bwd"):
        key = "bwd::" + key
    return key


def load_counters():
    """The committed counter record with only the kernels whose defining source
    file (and the shared headers) are unchanged since the counters were taken;
    None when there is no record."""
    try:
        data = json.loads(COUNTERS_FILE.read_text())
    except (OSError, ValueError):
        return None
    now, then = source_hashes(), data.get("source_hashes", {})
    shared = [n for n in now if n.endswith(".h")]
    current = {}
    for key, entry in data.get("kernels", {}).items():
        src = entry.get("source")
        if src is None:
            continue
        if all(now.get(n) == then.get(n) for n in [src, *shared]):
            current[key] = entry
    data["kernels"] = current
    return data


def measured_traffic(kernel, counters=None):
    """HBM bytes per launch of `kernel` from the committed TCC counter record
    (read + written), or None if there is no current record for it."""
    data = counters if counters is not None else load_counters()
    try:
        entry = data["kernels"][kernel]
        return int(entry["read_bytes"] + entry["write_bytes"])
    except (KeyError, TypeError):
        return None


def counters_summary(dirs, out=None, tag=None):
    """Summarise rocprofv3 --pmc runs over `--profile-pass` (one directory per
    pass, each with run_counter_collection.csv) into profiles/kernel_counters.json
    and a markdown table on stdout.  HBM bytes come from the TCC/EA request
    counts: reads = 128 B x (TCC_EA0_RDREQ - TCC_EA0_RDREQ_32B) + 32 B x
    TCC_EA0_RDREQ_32B (gfx950 issues 128-byte read requests: the profile
    pass's 256 MiB device copy shows exactly 2^21 of them), writes = 64 B x
    TCC_EA0_WRREQ_64B + 32 B x (TCC_EA0_WRREQ - TCC_EA0_WRREQ_64B).  MFMA
    busy % = SQ_VALU_MFMA_BUSY_CYCLES (summed over the SIMDs) / (GRBM_GUI_ACTIVE
    per XCC x SIMDs); rocprofv3 sums GRBM_GUI_ACTIVE over the XCCs."""
    import csv
    from collections import defaultdict

    per = defaultdict(lambda: defaultdict(list))  # key -> counter -> [value per dispatch]
    dur = defaultdict(list)
    n_xcc, n_simd = 8, 1024
    for d in dirs:
        for f in Path(d).rglob("*agent_info.csv"):
            for row in csv.DictReader(open(f)):
                if row.get("Name", "").startswith("gfx"):
                    n_xcc, n_simd = int(row["Num_Xcc"]), int(row["Simd_Count"])
        for f in Path(d).rglob("*counter_collection.csv"):
            seen = set()
            for row in csv.DictReader(open(f)):
                key = kernel_key(row["Kernel_Name"])
                per[key][row["Counter_Name"]].append(float(row["Counter_Value"]))
                if row["Dispatch_Id"] not in seen:
                    seen.add(row["Dispatch_Id"])
                    dur[key].append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) * 1e-3)
    mean = lambda xs: sum(xs) / len(xs) if xs else None  # noqa: E731

    def read_bytes(c):
        r32 = c.get("TCC_EA0_RDREQ_32B_sum", 0.0)
        return int(128 * (c["TCC_EA0_RDREQ_sum"] - r32) + 32 * r32)

    def write_bytes(c):
        w64 = c.get("TCC_EA0_WRREQ_64B_sum", 0.0)
        return int(64 * w64 + 32 * (c["TCC_EA0_WRREQ_sum"] - w64))

    kernels = {}
    for key, cs in per.items():
        c = {n: mean(v) for n, v in cs.items()}
        e = {"dispatches": max(len(v) for v in cs.values())}
        if "TCC_EA0_RDREQ_sum" in c:
            e["read_bytes"] = read_bytes(c)
        if "TCC_EA0_WRREQ_sum" in c:
            e["write_bytes"] = write_bytes(c)
        if c.get("SQ_VALU_MFMA_BUSY_CYCLES") is not None and c.get("GRBM_GUI_ACTIVE"):
            e["mfma_busy_pct"] = round(100 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (c["GRBM_GUI_ACTIVE"] / n_xcc * n_simd), 2)
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in c:
            e["mfma_bf16_flop"] = int(512 * c["SQ_INSTS_VALU_MFMA_MOPS_BF16"])
        if "SQ_INSTS_VALU_MFMA_MOPS_F32" in c:
            e["mfma_f32_flop"] = int(512 * c["SQ_INSTS_VALU_MFMA_MOPS_F32"])
        if dur[key]:
            e["counter_run_us"] = round(mean(dur[key]), 2)
            if e.get("mfma_bf16_flop"):
                e["mfma_bf16_frac_of_peak"] = round(e["mfma_bf16_flop"] / (e["counter_run_us"] * 1e-6)
                                                    / (BF16_PEAK_TFLOPS * 1e12), 4)
        e["counters"] = {n: round(v, 1) for n, v in c.items()}
        e["source"] = kernel_source(key)
        kernels[key] = e
    data = {
        "source": "rocprofv3 --pmc <counters> --kernel-trace -- python3 bench.py --profile-pass (one MI355X)",
        "source_hashes": source_hashes(),
        "rules": " ".join(counters_summary.__doc__.split("HBM bytes come from")[1].split()),
        "kernels": kernels,
    }
    if tag is not None:
        # one prefill configuration: this library's kernels under "<tag>::",
        # merged into the record of the same sources (a record of other
        # sources is dropped)
        kernels = {f"{tag}::{k}": e for k, e in kernels.items() if e["source"] is not None}
        try:
            old = json.loads(Path(out or COUNTERS_FILE).read_text())
        except (OSError, ValueError):
            old = {}
        merged = dict(old.get("kernels", {})) if old.get("source_hashes") == data["source_hashes"] else {}
        merged.update(kernels)
        data = dict(old or data, source_hashes=data["source_hashes"], kernels=merged)
        Path(out or COUNTERS_FILE).write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
        print("| kernel | dispatches | read MB | written MB | MFMA busy % | bf16 MFMA GFLOP | of bf16 peak | "
              "us (counter run) |")
        print("|---|---|---|---|---|---|---|---|")
        for key in sorted(kernels):
            e = kernels[key]
            fmt = lambda x, sc=1e6: "—" if x is None else f"{x / sc:.1f}"  # noqa: E731
            print(f"| `{key}` | {e['dispatches']} | {fmt(e.get('read_bytes'))} | {fmt(e.get('write_bytes'))} | "
                  f"{e.get('mfma_busy_pct', '—')} | {fmt(e.get('mfma_bf16_flop'), 1e9)} | "
                  f"{e.get('mfma_bf16_frac_of_peak', '—')} | {e.get('counter_run_us', '—')} |")
        return
    # the 256 MiB device copy of the profile pass (the runtime's copy kernel also
    # serves torch's small copies; the largest dispatch is this one)
    copies = [(r, w) for key, cs in per.items() if "copyBuffer" in key
              for r, w in zip(cs.get("TCC_EA0_RDREQ_sum", []), cs.get("TCC_EA0_WRREQ_sum", []) or [None] * 999)]
    rd = max((v for key, cs in per.items() if "copyBuffer" in key for v in cs.get("TCC_EA0_RDREQ_sum", [])),
             default=None)
    wr = max((v for key, cs in per.items() if "copyBuffer" in key for v in cs.get("TCC_EA0_WRREQ_sum", [])),
             default=None)
    w64 = max((v for key, cs in per.items() if "copyBuffer" in key for v in cs.get("TCC_EA0_WRREQ_64B_sum", [])),
              default=0.0)
    del copies
    if rd is not None:
        data["copy_check"] = {
            "bytes_each_way": 256 * 2**20,
            "read_requests": int(rd),
            "read_bytes": int(128 * rd),
            "write_bytes": None if wr is None else int(64 * w64 + 32 * (wr - w64)),
        }
    Path(out or COUNTERS_FILE).write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    print("| kernel | dispatches | read MB | written MB | MFMA busy % | bf16 MFMA GFLOP | of bf16 peak | us (counter run) |")
    print("|---|---|---|---|---|---|---|---|")
    for key in sorted(kernels):
        e = kernels[key]
        fmt = lambda x, sc=1e6: "—" if x is None else f"{x / sc:.1f}"  # noqa: E731
        print(f"| `{key}` | {e['dispatches']} | {fmt(e.get('read_bytes'))} | {fmt(e.get('write_bytes'))} | "
              f"{e.get('mfma_busy_pct', '—')} | {fmt(e.get('mfma_bf16_flop'), 1e9)} | "
              f"{e.get('mfma_bf16_frac_of_peak', '—')} | {e.get('counter_run_us', '—')} |")
    if "copy_check" in data:
        print(f"copy check: {data['copy_check']}")


def profile_pass(which="all"):
    """The workload of the counter runs: after one warm-up round, one prefill at
    the benchmark shape, one in-place decode step at the benchmark shape, and a
    256 MiB device-to-device copy whose byte counts check the counters; then
    the fused stages and their backward, the backward and the cache reorder legs once each (their
    warm-up calls included).  With a configuration name: that prefill only,
    a warm-up call and a measured one."""
    import torch

    import kda

    if which != "all":
        call, _ = config_call(which)
        call()
        call()
        torch.cuda.synchronize()
        print(f"profile pass {which} done", flush=True)
        return

    device = torch.device("cuda", 0)
    q, k, v, g, beta, s0 = _inputs(P_B, P_T, P_H, P_K, P_V, 0.02, 0, device)
    qd, kd, vd, gd, bd, _ = _inputs(D_B, 1, D_H, D_K, D_V, None, 2, device)
    state = torch.randn(D_B, D_H, D_K, D_V, generator=torch.Generator().manual_seed(1)).mul_(0.02).to(device)
    src = torch.rand(256 * 2**20 // 4, generator=torch.Generator().manual_seed(3)).to(device)
    dst = torch.empty_like(src)
    with torch.no_grad():
        for _ in range(2):
            kda.chunkwise_kda(q, k, v, g, beta, s0, True)
            kda.recurrent_kda(qd, kd, vd, gd, bd, state, True, update_state_in_place=True)
            dst.copy_(src)
    torch.cuda.synchronize()
    bench_fused(reps=1)
    bench_fused_backward(reps=1)
    bench_backward(reps=1)
    bench_cache(reps=1)
    print("profile pass done", flush=True)


def bench_dropin(steps, warmup):
    """The prefill and the decode step through the Python drop-in API, as the
    reference's callers use them (src/kda/kda.py:133-151): validation, input
    preparation and per-call output and workspace allocation included."""
    import torch

    import kda

    device = torch.device("cuda", 0)
    q, k, v, g, beta, s0 = _inputs(P_B, P_T, P_H, P_K, P_V, 0.02, 0, device)
    gen = torch.Generator().manual_seed(1)
    state = (torch.randn(D_B, D_H, D_K, D_V, generator=gen) * 0.02).to(device)
    dq, dk, dv, dg, db, _ = _inputs(D_B, D_STEPS, D_H, D_K, D_V, None, 2, device)
    steps_in = [tuple(x[:, t:t + 1].contiguous() for x in (dq, dk, dv, dg, db)) for t in range(D_STEPS)]

    def timed(fn, n):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    with torch.no_grad():
        _settle(lambda: kda.chunkwise_kda(q, k, v, g, beta, s0, True))
        pre_ms = timed(lambda i: kda.chunkwise_kda(q, k, v, g, beta, s0, True), steps)
        dec_ms = timed(lambda i: kda.recurrent_kda(*steps_in[i % D_STEPS], state, True, update_state_in_place=True),
                       D_STEPS)
    return {
        "prefill": {"api": "kda.chunkwise_kda(q, k, v, g, beta, initial_state, output_final_state=True)",
                    "ms": round(pre_ms, 5), "tokens_per_s": round(P_B * P_T / (pre_ms * 1e-3), 1)},
        "decode": {"api": "kda.recurrent_kda(q, k, v, g, beta, state, True, update_state_in_place=True)",
                   "ms_per_step": round(dec_ms, 5),
                   "gbs": round(decode_bytes(D_B, D_H, D_K, D_V) / (dec_ms * 1e-3) / 1e9, 1)},
    }


# The other prefill configurations, by the key their counter records carry.
PREFILL_CONFIGS = {
    "b8_t1024_h8": (8, 1024, 8, 128, None),
    "packed_4docs_t65536_h64": (1, 65536, 64, 128, [0, 32768, 49152, 61440, 65536]),
    "k64_t8192_h16": (1, 8192, 16, 64, None),
}


def config_call(name):
    """The C-ABI prefill of one configuration with its inputs on the GPU (drawn
    with the distributions of the prefill workload), its workspace
    preallocated: (call, metadata).  The K=V=64 shape starts from an
    N(0, 0.02) state, as the long-context workload does."""
    import torch

    from kda import _lib

    lib = _lib.load()
    device = torch.device("cuda", 0)
    code = _lib.dtype_code(torch.bfloat16)
    stream = torch.cuda.current_stream(device).cuda_stream
    B, T, H, K, offsets = PREFILL_CONFIGS[name]
    V = K
    gen = torch.Generator(device=device).manual_seed(5)
    shape_k = (B, T, H, K)
    q = torch.nn.functional.normalize(torch.randn(shape_k, generator=gen, device=device), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(shape_k, generator=gen, device=device), dim=-1).bfloat16()
    v = torch.randn(B, T, H, V, generator=gen, device=device).bfloat16()
    g = (-torch.nn.functional.softplus(torch.randn(shape_k, generator=gen, device=device) + 2)).bfloat16()
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen, device=device)).bfloat16()
    n_seq = B if offsets is None else len(offsets) - 1
    s_in = None
    if name.startswith("k64"):
        s_in = torch.randn(n_seq, H, K, V, generator=gen, device=device).mul_(0.02)
    o = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=device)
    s_out = torch.empty(n_seq, H, K, V, dtype=torch.float32, device=device)
    cu = None if offsets is None else torch.tensor(offsets, dtype=torch.int32, device=device)
    # dense: tokens per sequence; packed documents: the longest document,
    # which a caller that packs them knows (the schedule's hint)
    span = T if offsets is None else max(b - a for a, b in zip(offsets[:-1], offsets[1:]))
    longest = 0 if offsets is None else span
    ws_bytes = lib.kda_chunk_fwd_workspace_bytes(n_seq, B * T, longest, H, K, V, code)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    keep = (q, k, v, g, beta, s_in, o, s_out, cu, ws)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code, _lib.ptr(s_in),
            s_out.data_ptr(), 0, o.data_ptr(), _lib.ptr(cu), span, None, n_seq, B * T, H, K, V, ws.data_ptr(),
            ws_bytes, stream)

    def call(_keep=keep):
        _lib.check(lib.kda_chunk_fwd(*args))

    L, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(lib.kda_chunk_fwd_plan(n_seq, B * T, longest, H, K, V, code, ctypes.byref(L), ctypes.byref(segs)))
    n_state_io = 1 if s_in is None else 2
    meta = {
        "workload": f"kda chunkwise prefill B={B} T={T} H={H} K=V={K} bf16, "
                    + ("N(0,0.02) initial state, " if s_in is not None else "zero initial state, ")
                    + ("final state out" if offsets is None else f"cu_seqlens={offsets}, per-document final states"),
        "tokens": B * T,
        "algorithmic_bytes": 2 * B * T * H * (3 * K + V) + 2 * B * T * H + 2 * B * T * H * V
                             + 4 * n_state_io * n_seq * H * K * V,
        "algorithmic_flops": prefill_flops(B, T, H, K, V),
        "chunks_per_segment": L.value,
    }
    return call, meta


def bench_configs(steps, warmup, counters=None):
    """The other prefill configurations the metric reports as tokens/s and
    roofline: B=8, T=1024, H=8 (zero initial state, final state out), the
    packed documents cu_seqlens = [0, 32768, 49152, 61440, 65536] at H=64
    (per-document final states), both K=V=128, and the reference's shipped
    head shape K=V=64 at B=1, T=8192, H=16; bf16, through the C ABI with the
    workspace preallocated.  Each carries the HBM bytes and MFMA busy of its
    kernels from the committed counter record under its own key."""
    import torch

    out = {}
    for name in PREFILL_CONFIGS:
        call, meta = config_call(name)
        _settle(call)
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        nbytes, flops = meta["algorithmic_bytes"], meta["algorithmic_flops"]
        rec = {k: v for k, v in (counters or {}).get("kernels", {}).items() if k.startswith(name + "::")}
        out[name] = {
            "workload": meta["workload"],
            "ms": round(ms, 5),
            "tokens_per_s": round(meta["tokens"] / (ms * 1e-3), 1),
            "algorithmic_bytes": nbytes,
            "achieved_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "frac_bf16_mfma": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "chunks_per_segment": meta["chunks_per_segment"],
            "traffic": (sum(int(e["read_bytes"] + e["write_bytes"]) for e in rec.values())
                        if rec and all("read_bytes" in e and "write_bytes" in e for e in rec.values()) else None),
            "kernels_mfma_busy_pct": {k.split("::", 1)[1]: e.get("mfma_busy_pct") for k, e in rec.items()} or None,
        }
        del call
    return out


def bench_prefill_f32(steps, warmup):
    """f32 inputs at the long-context shape through kda.chunkwise_kda: the
    split-bf16 chunk path of a dense call, the same sequence as one packed
    document (gathered into a padded batch for the same path), and the exact
    recurrence kernel (the packed call through the C ABI without the longest
    document's length, which that path needs)."""
    import torch

    import kda
    from kda import _lib

    device = torch.device("cuda", 0)
    q, k, v, g, beta, s0 = (t.float() for t in _inputs(P_B, P_T, P_H, P_K, P_V, 0.02, 0, device))

    def timed(fn, n, w):
        for _ in range(w):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    lib = _lib.load()
    code = _lib.dtype_code(torch.float32)
    L, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(lib.kda_chunk_fwd_plan(P_B, P_B * P_T, 0, P_H, P_K, P_V, code, ctypes.byref(L), ctypes.byref(segs)))
    out = torch.empty(P_B, P_T, P_H, P_V, device=device)
    s_out = torch.empty(P_B, P_H, P_K, P_V, device=device)
    cu = torch.tensor([0, P_T], dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream

    def recurrence():
        _lib.check(lib.kda_chunk_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code,
                                     s0.data_ptr(), s_out.data_ptr(), code, out.data_ptr(), cu.data_ptr(), 0, None, 1,
                                     P_T, P_H, P_K, P_V, None, 0, stream))

    with torch.no_grad():
        _settle(lambda: kda.chunkwise_kda(q, k, v, g, beta, s0, True))
        split_ms = timed(lambda: kda.chunkwise_kda(q, k, v, g, beta, s0, True), steps, warmup)
        packed_ms = timed(lambda: kda.chunkwise_kda(q, k, v, g, beta, s0, True, cu_seqlens=[0, P_T]), steps, warmup)
        rec_ms = timed(recurrence, 2, 1)
    nbytes = 2 * prefill_bytes(P_B, P_T, P_H, P_K, P_V, n_state_io=1)  # every tensor f32
    return {
        "workload": f"kda.chunkwise_kda B={P_B} T={P_T} H={P_H} K=V={P_K} f32 inputs, f32 state N(0,0.02) in, "
                    "final state out",
        "plan": L.value,
        "ms": round(split_ms, 5),
        "tokens_per_s": round(P_B * P_T / (split_ms * 1e-3), 1),
        "achieved_gbs": round(nbytes / (split_ms * 1e-3) / 1e9, 1),
        "algorithmic_bytes": nbytes,
        "packed_one_document_ms": round(packed_ms, 5),
        "packed_over_dense": round(packed_ms / split_ms, 3),
        "recurrence_kernel_ms": round(rec_ms, 5),
        "speedup_vs_recurrence": round(rec_ms / split_ms, 2),
    }


def prefill_plan():
    from kda import _lib

    lib = _lib.load()
    import torch

    L, segs = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(lib.kda_chunk_fwd_plan(P_B, P_B * P_T, 0, P_H, P_K, P_V, _lib.dtype_code(torch.bfloat16),
                                      ctypes.byref(L), ctypes.byref(segs)))
    return {"chunks_per_segment": L.value, "segments": segs.value}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-pass", nargs="?", const="all", default=None,
                    choices=["all", *PREFILL_CONFIGS],
                    help="run the counter-collection workload only (for rocprofv3 --pmc): all legs, or one "
                         "prefill configuration")
    ap.add_argument("--counters-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc output directories into profiles/kernel_counters.json")
    ap.add_argument("--counters-out", default=None, help="where --counters-summary writes its JSON")
    ap.add_argument("--counters-tag", default=None, choices=list(PREFILL_CONFIGS),
                    help="file the summarised kernels under this prefill configuration's key, merged into "
                         "the existing record")
    args = ap.parse_args()
    if args.counters_summary:
        counters_summary(args.counters_summary, args.counters_out, args.counters_tag)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the KDA operator has no collective; --gpus {args.gpus} "
              "is not supported: run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    if args.profile_pass:
        profile_pass(args.profile_pass)
        return 0

    ms, per_kernel, ws_bytes, settle = bench_prefill(args.steps, args.warmup, settle_ms=SETTLE_MS)
    dec_ms = bench_decode(args.warmup)
    counters = load_counters()

    tokens_per_s = P_B * P_T / (ms * 1e-3)
    pbytes = prefill_bytes(P_B, P_T, P_H, P_K, P_V)
    pflops = prefill_flops(P_B, P_T, P_H, P_K, P_V)
    ran = {n: t for n, t in per_kernel.items() if t > 0}
    dom = max(ran, key=ran.get)
    dom_ms = ran[dom]
    dbytes = decode_bytes(D_B, D_H, D_K, D_V)
    dec_gbs = dbytes / (dec_ms * 1e-3) / 1e9
    traffic = {n: measured_traffic(n, counters) for n in ran}
    op_traffic = None if None in traffic.values() else sum(traffic.values())
    mfma = {n: (counters or {}).get("kernels", {}).get(n, {}).get("mfma_busy_pct") for n in ran}

    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "clock_settle": dict(settle, note="untimed prefill launches before the warm-up steps, so that the "
                             "timed steps run at the GPU's settled clock (from a cold start the first ~100 "
                             "prefills run up to 7% slower while the clock ramps)"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded q,k L2-normalised, g=-softplus(N(0,1)+2), beta=sigmoid(N(0,1)))",
        "config": {
            "workload": "kda chunkwise prefill, long context",
            "batch": P_B, "tokens": P_T, "heads": P_H, "key_dim": P_K, "value_dim": P_V, "chunk": 64,
            "inputs": "bf16", "state": "f32 N(0,0.02) initial, final state returned",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(pbytes / (dom_ms * 1e-3) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(pbytes / (dom_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": op_traffic,
            "algorithmic_bytes": pbytes,
            "kernel_ms": round(dom_ms, 5),
            "note": "achieved = the operator's compulsory bytes (q, k, g, v, beta, output, f32 initial and "
                    "final state) / the dominant kernel's time; traffic = HBM bytes per prefill, all kernels, "
                    "from the committed TCC counter record of these sources (null if it is stale)",
        },
        "roofline_operator": {
            "bound": "hbm",
            "plan": prefill_plan(),
            "kernels_ms": {k: round(v, 5) for k, v in per_kernel.items()},
            "kernels_traffic": traffic,
            "kernels_mfma_busy_pct": mfma,
            "achieved_gbs": round(pbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(pbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "achieved_tflops": round(pflops / (ms * 1e-3) / 1e12, 2),
            "frac_bf16_mfma": round(pflops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "algorithmic_flops": pflops,
            "workspace_bytes": ws_bytes,
        },
        "decode": {
            "workload": f"decode step B={D_B} H={D_H} K=V=128, f32 state updated in place, {D_STEPS} steps",
            "value": round(dec_gbs, 1),
            "unit": "GB/s",
            "ms_per_step": round(dec_ms, 5),
            "roofline": {
                "bound": "hbm", "kernel": "recurrent_kernel", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic("recurrent_kernel", counters), "algorithmic_bytes": dbytes,
            },
        },
    }
    result["dropin"] = bench_dropin(args.steps, args.warmup)
    result["fused_stages"] = {
        "workload": f"B={P_B} T={P_T} H={P_H} D={P_K} bf16, 50 back-to-back C-ABI launches each",
        "kernels": bench_fused(),
    }
    result["fused_stages_backward"] = {
        "workload": f"B={P_B} T={P_T} H={P_H} D={P_K} bf16, 20 back-to-back C-ABI launches each",
        "kernels": bench_fused_backward(),
    }
    result["layer_train"] = bench_layer_train()
    k64_ms, k64_kernels, _, _ = bench_prefill(args.steps, args.warmup, shape=(1, 8192, 16, 64, 64),
                                              settle_ms=SETTLE_MS)
    k64_bytes = prefill_bytes(1, 8192, 16, 64, 64)
    result["prefill_k64"] = {
        "workload": "kda chunkwise prefill B=1 T=8192 H=16 K=V=64 bf16 (the gpu_48gb head shape), f32 state "
                    "N(0,0.02) in, final state out",
        "ms": round(k64_ms, 5),
        "tokens_per_s": round(8192 / (k64_ms * 1e-3), 1),
        "kernels_ms": {n: round(t, 5) for n, t in k64_kernels.items()},
        "achieved_gbs": round(k64_bytes / (k64_ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(k64_bytes / (k64_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "algorithmic_bytes": k64_bytes,
    }
    result["prefill_f32"] = bench_prefill_f32(args.steps, args.warmup)
    result["prefill_configs"] = bench_configs(args.steps, args.warmup, counters)
    result["decay_fusion"] = bench_decay_fusion()
    result["backward"] = bench_backward()
    # the reference's shipped head shape, and f32 inputs (split-bf16 operands)
    result["backward"]["k64_t8192_h16"] = bench_backward(shape=(P_B, P_T, P_H, 64, 64))
    result["backward"]["f32_inputs"] = bench_backward(dtype_name="f32")
    result["cache_reorder"] = bench_cache()
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
        result["cpu_baseline"] = cpu["prefill"]
        result["decode"]["cpu_baseline"] = cpu["decode"]
        result["backward"]["cpu_baseline"] = cpu["backward"]
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
