"""kda_chunk_fwd_noalloc (the prefill on the library's static device scratch)
against kda_chunk_fwd (the same kernels on a caller workspace), through the C
ABI: bit-identical outputs and final states on two calls in a row, the second
one smaller, and a clear refusal of a prefill whose workspace exceeds the
scratch.  A caller under HIP graph capture makes one eager call first (it
looks up the device's scratch address and raises the kernels' LDS limit),
then captures the call; the graph's replays match kda_chunk_fwd bit for bit."""

from __future__ import annotations

import re

import pytest
import torch

from kda import _lib
from tests._inputs import workload

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _noalloc():
    lib = _lib.load()
    return lib, lib.kda_chunk_fwd_noalloc


def _run(lib, noalloc, shape, seed, cu=None):
    B, T, H, K, V = shape
    q, k, v, g, beta, s0 = (None if t is None else t.to(DEV).contiguous()
                            for t in workload(*shape, state_std=0.02, seed=seed))
    if cu is not None:
        s0 = torch.randn(len(cu) - 1, H, K, V, generator=torch.Generator().manual_seed(seed)).mul_(0.02).to(DEV)
    n_seq = B if cu is None else len(cu) - 1
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV)
    # dense: tokens per sequence; packed documents: the longest document (the schedule's hint)
    span = T if cu is None else max(b - a for a, b in zip(cu[:-1], cu[1:]))
    code = _lib.dtype_code(torch.bfloat16)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    outs = []
    for use_noalloc in (False, True):
        out = torch.full((B, T, H, V), float("nan"), dtype=torch.bfloat16, device=DEV)
        s1 = torch.full((n_seq, H, K, V), float("nan"), dtype=torch.float32, device=DEV)
        common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code, s0.data_ptr(),
                  s1.data_ptr(), 0, out.data_ptr(), _lib.ptr(cu_t), span, None, n_seq, B * T, H, K, V)
        if use_noalloc:
            _lib.check(noalloc(*common, stream))
        else:
            ws_bytes = lib.kda_chunk_fwd_workspace_bytes(n_seq, B * T, 0 if cu is None else span, H, K, V, code)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
            _lib.check(lib.kda_chunk_fwd(*common, ws.data_ptr(), ws_bytes, stream))
        torch.cuda.synchronize()
        outs.append((out, s1))
    (o_ref, s_ref), (o_got, s_got) = outs
    assert torch.isfinite(o_got.float()).all() and torch.isfinite(s_got).all()
    # the same kernels on the same inputs: identical bits
    assert torch.equal(o_got.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(s_got.view(torch.int32), s_ref.view(torch.int32))


def test_noalloc_prefill_matches_workspace_prefill_twice():
    lib, noalloc = _noalloc()
    # the long-context workload (segmented schedule, ~72 MB of workspace) ...
    _run(lib, noalloc, (1, 8192, 16, 128, 128), seed=0)
    # ... then a smaller one right after, on the same scratch
    _run(lib, noalloc, (1, 4096, 8, 128, 128), seed=1)
    _run(lib, noalloc, (2, 1000, 4, 128, 128), seed=4)
    # packed documents (chunk and segment maps in the scratch)
    _run(lib, noalloc, (1, 700, 2, 128, 64), seed=2, cu=[0, 300, 301, 700])


def test_noalloc_refuses_a_prefill_beyond_the_scratch():
    lib, noalloc = _noalloc()
    code = _lib.dtype_code(torch.bfloat16)
    # one 262144-token sequence at H=16 needs far more than the 128 MiB scratch;
    # the size check rejects it before any pointer is touched or kernel launched
    need = lib.kda_chunk_fwd_workspace_bytes(1, 262144, 0, 16, 128, 128, code)
    status = noalloc(1, 1, 1, 1, 1, code, None, None, 0, 1, None, 262144, None, 1, 262144, 16, 128, 128,
                     torch.cuda.current_stream(DEV).cuda_stream)
    assert status == _lib.KDA_ERR_WORKSPACE
    text = lib.kda_status_string(status).decode()
    assert "static scratch" in text and str(need) in text
    # the size the library was built with, as it reports it
    held = int(re.search(r"static scratch holds (\d+)", text).group(1))
    assert need > held and held == _lib.NOALLOC_SCRATCH_BYTES
    # the library still works afterwards
    _run(lib, noalloc, (1, 130, 2, 128, 128), seed=3)


def test_noalloc_prefill_replays_in_a_hip_graph():
    lib, noalloc = _noalloc()
    shape = (1, 8192, 16, 128, 128)  # the segmented schedule: three kernels per call
    B, T, H, K, V = shape
    q, k, v, g, beta, s0 = (t.to(DEV).contiguous() for t in workload(*shape, state_std=0.02, seed=5))
    code = _lib.dtype_code(torch.bfloat16)
    out = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=DEV)
    s1 = torch.empty(B, H, K, V, dtype=torch.float32, device=DEV)
    common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), code, s0.data_ptr(),
              s1.data_ptr(), 0, out.data_ptr(), None, T, None, B, B * T, H, K, V)
    # the workspace prefill, eager
    ws_bytes = lib.kda_chunk_fwd_workspace_bytes(B, B * T, 0, H, K, V, code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    _lib.check(lib.kda_chunk_fwd(*common, ws.data_ptr(), ws_bytes, torch.cuda.current_stream(DEV).cuda_stream))
    torch.cuda.synchronize()
    o_ref, s_ref = out.clone(), s1.clone()
    # one eager call of the entry point (set-up per device), then the capture
    _lib.check(noalloc(*common, torch.cuda.current_stream(DEV).cuda_stream))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = noalloc(*common, torch.cuda.current_stream(DEV).cuda_stream)
    assert status == _lib.KDA_OK
    for replay in range(3):
        # eager work between the replays: clear the results
        out.fill_(float("nan"))
        s1.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), o_ref.view(torch.int16)), f"replay {replay}"
        assert torch.equal(s1.view(torch.int32), s_ref.view(torch.int32)), f"replay {replay}"
