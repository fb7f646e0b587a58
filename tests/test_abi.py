"""The C-ABI library loads and exports every entry point include/kda_mi355x.h
declares (no compute calls: this suite runs without a GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from kda import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "kda_mi355x.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kda_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = declared_functions()
    for required in ("kda_recurrent_fwd", "kda_decode_step", "kda_chunk_fwd", "kda_chunk_fwd_workspace_bytes",
                     "kda_ut_transform", "kda_abi_version", "kda_status_string"):
        assert required in names


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run kimi-k3-pytorch_amd/build_lib.py)")
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [name for name in declared_functions() if not hasattr(raw, name)]
    assert missing == []


def test_python_binding_types_every_declared_symbol():
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_abi_version_and_status_strings():
    lib = _lib.load()
    assert lib.kda_abi_version() == _lib.ABI_VERSION
    assert lib.kda_status_string(0).decode() == "ok"
    assert "invalid argument" in lib.kda_status_string(1).decode()


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _lib.load()
    # null input pointers: rejected by the argument checks, nothing is launched
    status = lib.kda_recurrent_fwd(None, None, None, None, None, 2, None, None, 0, None, None, None, 4, None,
                                   1, 4, 1, 128, 128, None)
    assert status == _lib.KDA_ERR_INVALID_ARGUMENT
    assert "non-null" in lib.kda_status_string(status).decode()
    # mismatched state dtype for bf16 inputs
    status = lib.kda_decode_step(1, 1, 1, 1, 1, 2, None, 1, 3, 1, 1, 1, 128, 128, None)
    assert status == _lib.KDA_ERR_INVALID_ARGUMENT
    # dense layout whose sizes do not add up
    status = lib.kda_chunk_fwd(1, 1, 1, 1, 1, 2, None, None, 0, 1, None, 3, None, 2, 7, 1, 128, 128, None, 0, None)
    assert status == _lib.KDA_ERR_INVALID_ARGUMENT


def test_plan_cuts_a_dominant_packed_document():
    """Packed documents that fill the GPU with one chain per (document, head)
    keep one segment each, unless the longest document (the caller's hint)
    would run well past a balanced pass: then every document is cut into
    segments of the balanced pass's chunk-steps per CU.  Without a GPU the
    planner assumes 256 CUs (the MI355X count)."""
    lib = _lib.load()
    code = _lib.dtype_code(__import__("torch").bfloat16)

    def plan(n, total, longest, heads):
        cps, segs = ctypes.c_int64(0), ctypes.c_int64(0)
        _lib.check(lib.kda_chunk_fwd_plan(n, total, longest, heads, 128, 128, code, ctypes.byref(cps),
                                          ctypes.byref(segs)))
        return cps.value

    # cu_seqlens = [0, 32768, 49152, 61440, 65536] at H=64: 256 chains of which
    # 64 run 512 chunks, against 256 chunk-steps per CU for a balanced pass
    assert plan(4, 65536, 32768, 64) == 256
    assert plan(4, 65536, 0, 64) == 0  # no hint: one segment per document
    assert plan(4, 65536, 16384, 64) == 0  # four equal documents are already balanced
    assert plan(4, 65536, 20000, 64) == 0  # within a quarter of balanced
    # dense sequences ignore the hint argument's absence (0) and keep their plan
    assert plan(1, 8192, 0, 16) == 8
    more = lib.kda_chunk_fwd_workspace_bytes(4, 65536, 32768, 64, 128, 128, code)
    assert more > lib.kda_chunk_fwd_workspace_bytes(4, 65536, 0, 64, 128, 128, code)
    assert lib.kda_chunk_fwd_workspace_bytes(4, 65536, 65537, 64, 128, 128, code) == 0
    # a hint past the packed tokens is an invalid argument, rejected before any launch
    status = lib.kda_chunk_fwd(1, 1, 1, 1, 1, code, None, None, 0, 1, 1, 70000, None, 4, 65536, 64, 128, 128, None,
                               0, None)
    assert status == _lib.KDA_ERR_INVALID_ARGUMENT
    assert "longest document" in lib.kda_status_string(status).decode()


def test_plan_takes_a_chunk_path_for_every_float_input_up_to_key_dim_128():
    """bf16, f16 and f32 inputs with K <= 128 never run the token recurrence:
    the MFMA path (bf16/f16 on its grid) or the split-bf16 chunk path (>= 0 or
    -2), dense or packed, any value width; K past 128 and f64 inputs run the
    exact recurrence (-1)."""
    torch = __import__("torch")
    lib = _lib.load()

    def plan(n, total, longest, heads, K, V, dtype):
        cps, segs = ctypes.c_int64(0), ctypes.c_int64(0)
        _lib.check(lib.kda_chunk_fwd_plan(n, total, longest, heads, K, V, _lib.dtype_code(dtype), ctypes.byref(cps),
                                          ctypes.byref(segs)))
        return cps.value

    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        for K in (1, 3, 40, 64, 100, 128):
            for V in (1, 5, 48, 128, 129, 200, 256, 300, 512):
                for n, total, longest in ((1, 8192, 0), (4, 4096, 0), (3, 1000, 700)):
                    assert plan(n, total, longest, 4, K, V, dtype) != -1, (dtype, K, V, n, longest)
        assert plan(1, 8192, 0, 4, 129, 128, dtype) == -1
        assert plan(3, 1000, 700, 4, 256, 64, dtype) == -1
    assert plan(1, 8192, 0, 4, 128, 128, torch.float64) == -1
    # the packed split path's workspace is a padded batch of the longest document
    code = _lib.dtype_code(torch.float32)
    packed = lib.kda_chunk_fwd_workspace_bytes(3, 1000, 700, 4, 128, 128, code)
    assert packed > lib.kda_chunk_fwd_workspace_bytes(1, 3 * 700, 0, 4, 128, 128, code)


def declared_arities() -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(kda_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_arity_matches_header():
    arities = declared_arities()
    assert sorted(arities) == declared_functions()
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        assert len(argtypes) == arities[name], name


def test_fused_entry_points_reject_unsupported_layouts():
    # every case fails a host-side check before anything is launched
    lib = _lib.load()
    bf16 = _lib.dtype_code(__import__("torch").bfloat16)
    a, b = 4096, 8192  # 16-byte aligned stand-in addresses (never dereferenced)
    conv = lambda **kw: lib.kda_conv_silu_fwd(  # noqa: E731
        kw.get("x", a), a, None, None, b, None, None, 1, 8, kw.get("c", 256), kw.get("k", 4), kw.get("d", 128),
        kw.get("norm", 1), 1e-6, bf16, None)
    assert conv(k=9) == _lib.KDA_ERR_UNSUPPORTED
    assert conv(c=288, d=96) == _lib.KDA_ERR_UNSUPPORTED  # normalised heads are powers of two
    assert conv(c=260, norm=0) == _lib.KDA_ERR_UNSUPPORTED  # rows are whole 16-byte vectors
    assert conv(x=a + 2) == _lib.KDA_ERR_INVALID_ARGUMENT  # misaligned
    assert conv(c=250) == _lib.KDA_ERR_INVALID_ARGUMENT  # channels not a multiple of head_dim
    gates = lambda z, k: lib.kda_gates_fwd(z, None, a, -5.0, b, None, None, None, 4, 2, k, bf16, None)  # noqa: E731
    assert gates(a, 12) == _lib.KDA_ERR_UNSUPPORTED  # key_dim not a multiple of 8 bf16 elements
    assert gates(a + 8, 16) == _lib.KDA_ERR_INVALID_ARGUMENT
    norm = lambda x, d: lib.kda_rmsnorm_gate_fwd(x, None, 0, None, b, 4, 2, d, 1e-6, bf16, None)  # noqa: E731
    assert norm(a, 96) == _lib.KDA_ERR_UNSUPPORTED
    assert norm(a, 1024) == _lib.KDA_ERR_UNSUPPORTED
    assert norm(a + 4, 128) == _lib.KDA_ERR_INVALID_ARGUMENT


def test_backward_entry_point_rejects_bad_arguments():
    # host-side checks only: nothing is launched
    lib = _lib.load()
    import torch

    bf16, f64 = _lib.dtype_code(torch.bfloat16), _lib.dtype_code(torch.float64)
    a = 4096
    ptrs = [a] * 6

    def call(dtype=bf16, K=128, V=128, ws=None, ws_bytes=0, dq=a):
        return lib.kda_chunk_bwd(*ptrs, dtype, None, None, dq, a, a, a, a, None, 1, 64, 1, K, V, ws, ws_bytes, None)

    assert call(dtype=f64) == _lib.KDA_ERR_WORKSPACE  # f64 is computed in f64; no workspace given
    assert call(dtype=7) == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(K=256) == _lib.KDA_ERR_UNSUPPORTED
    assert call(dq=None) == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call() == _lib.KDA_ERR_WORKSPACE  # no workspace
    need = lib.kda_chunk_bwd_workspace_bytes(1, 64, 1, 128, 128, bf16)
    assert need > 0 and call(ws=a, ws_bytes=need - 1) == _lib.KDA_ERR_WORKSPACE
    assert call(ws=a + 4, ws_bytes=need) == _lib.KDA_ERR_INVALID_ARGUMENT  # misaligned workspace
    assert lib.kda_chunk_bwd_workspace_bytes(0, 64, 1, 128, 128, bf16) == 0
    assert lib.kda_chunk_bwd_workspace_bytes(1, 64, 1, 128, 128, 7) == 0  # unknown dtype


@pytest.mark.parametrize("B,T,H,K,V", [(1, 8192, 16, 128, 128), (2, 1000, 3, 64, 48), (4, 130, 2, 100, 5)])
def test_backward_workspace_per_dtype(B, T, H, K, V):
    # one record per (sequence, head, chunk) plus the segment records of both
    # scans; f32 inputs keep split-bf16 operand records (hi and lo planes) and
    # f32 states, bf16/f16 inputs single-operand records and bf16 S, dS, Vt
    import torch

    lib = _lib.load()
    kp, vp = (64 if K <= 64 else 128), (V + 31) // 32 * 32
    nc = (T + 63) // 64
    cc, ck, cv, kv = 64 * 64, 64 * kp, 64 * vp, kp * vp

    def record(split):
        s = 1 if split else 2
        rec = 2 * cc + cc // s + 5 * ck // s + ck + cv + kp + 2 * (kv // s) + cv // s + cv + 3 * ck + 2 * cc + kp
        return (rec + 63) // 64 * 64

    want_segs = min(max(-(-256 // (2 * B * H)), 1), nc)
    seg_len = -(-nc // want_segs)
    segs = -(-nc // seg_len)
    seg = 2 * B * H * segs * (kp * kp + 2 * kp * vp)
    for dtype, split in ((torch.float32, True), (torch.bfloat16, False), (torch.float16, False)):
        got = lib.kda_chunk_bwd_workspace_bytes(B, T, H, K, V, _lib.dtype_code(dtype))
        assert got == 4 * (B * H * nc * record(split) + seg), dtype
    f64 = lib.kda_chunk_bwd_workspace_bytes(B, T, H, K, V, _lib.dtype_code(torch.float64))
    assert f64 > 0
    if (B, T, H, K, V) == (1, 8192, 16, 128, 128):
        assert record(True) == 151808 and record(False) == 108800  # 593 and 425 KiB


def test_recurrent_backward_entry_point_rejects_bad_arguments():
    # host-side checks only: nothing is launched
    lib = _lib.load()
    import torch

    f32, bf16 = _lib.dtype_code(torch.float32), _lib.dtype_code(torch.bfloat16)
    a = 4096

    def call(dtype=f32, states=a, ws=None, ws_bytes=0, tokens=4):
        return lib.kda_recurrent_bwd(a, a, a, a, a, a, None, states, None, None, a, a, a, a, a, None,
                                     1, tokens, 2, 16, 16, dtype, ws, ws_bytes, None)

    assert call(dtype=bf16) == _lib.KDA_ERR_INVALID_ARGUMENT  # the work type only: f32 or f64
    assert call(states=None) == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(tokens=0) == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call() == _lib.KDA_ERR_WORKSPACE
    need = lib.kda_recurrent_bwd_workspace_bytes(1, 2, 16, 16, f32)
    assert need > 0 and call(ws=a, ws_bytes=need - 1) == _lib.KDA_ERR_WORKSPACE
    assert lib.kda_recurrent_bwd_workspace_bytes(1, 2, 16, 16, _lib.dtype_code(torch.float64)) == 2 * need


def test_noalloc_scratch_size_matches_the_header():
    text = HEADER.read_text()
    m = re.search(r"#define KDA_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    assert m is not None
    assert int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES


@pytest.mark.parametrize("B,T,H,K,V", [(1, 8192, 16, 128, 128), (2, 1000, 3, 64, 48), (4, 130, 2, 100, 5)])
def test_split_path_forward_workspace_is_its_own_records(B, T, H, K, V):
    # f32 inputs take the split-bf16 chunk path: one record of the forward's
    # operands per (sequence, head, chunk) plus the forward scan's segment
    # records, smaller than the backward's workspace at every shape
    lib = _lib.load()
    kp, vp = (64 if K <= 64 else 128), (V + 31) // 32 * 32
    nc = (T + 63) // 64
    record = 64 * 64 + 3 * 64 * kp + 2 * 64 * vp + kp + kp * vp
    record = (record + 63) // 64 * 64
    want_segs = min(max(-(-256 // (B * H)), 1), nc)
    seg_len = -(-nc // want_segs)
    segs = -(-nc // seg_len)
    expect = 4 * (B * H * nc * record + B * H * segs * (kp * kp + 2 * kp * vp))
    got = lib.kda_chunk_fwd_workspace_bytes(B, B * T, 0, H, K, V, _lib.dtype_code(torch.float32))
    assert got == expect
    assert got < lib.kda_chunk_bwd_workspace_bytes(B, T, H, K, V, _lib.dtype_code(torch.float32))
    if (B, T, H, K, V) == (1, 8192, 16, 128, 128):
        assert record == 61568 and got == 554696704
