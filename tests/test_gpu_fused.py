"""GPU parity of the fused stages around the operator (kda.fused) against the
CPU oracle.

Tolerances (max|x - ref| / max|ref| per tensor): f64 1e-12, f32 1e-5 (same
arithmetic, different summation order), bf16/f16 1e-2 against the oracle's
f32 run on the same values (the kernels round once at the end; the reference
rounds after each step, which the tolerance covers).
"""

from __future__ import annotations

import pytest
import torch

import kda
from kda import fused
from oracle import kda_oracle as ora
from tests._inputs import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float64: 1e-12, torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def _rand(*shape, dtype, seed, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=gen, dtype=torch.float64) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("normalize,heads,head_dim", [(True, 2, 128), (True, 3, 64), (False, 2, 96)])
def test_conv_silu_matches_oracle(dtype, normalize, heads, head_dim):
    B, T, K = 2, 70, 4  # T crosses a 64-token tile
    C = heads * head_dim
    x = _rand(B, T, C, dtype=dtype, seed=1)
    w = _rand(C, K, dtype=dtype, seed=2, scale=0.5)
    b = _rand(C, dtype=dtype, seed=3, scale=0.1)
    hist = _rand(B, K - 1, C, dtype=dtype, seed=4)
    mask = torch.arange(T)[None, :] < torch.tensor([T, 41])[:, None]
    ref_y, ref_h = ora.conv_silu(x, w, b, hist, mask, num_heads=heads, normalize=normalize, eps=1e-6)
    y, st = fused.conv_silu(x.to(DEV), w.to(DEV), b.to(DEV), kda.ShortConvState(hist.to(DEV)), mask.to(DEV),
                            num_heads=heads, normalize=normalize, eps=1e-6, output_final_state=True)
    assert y.shape == (B, T, heads, head_dim) and y.dtype == dtype
    assert rel_err(y.reshape(B, T, C), ref_y) < TOL[dtype]
    assert torch.equal(st.buffer.cpu(), ref_h)  # the history is copied, not computed
    assert torch.count_nonzero(y[1, 41:]) == 0


def test_conv_silu_decode_steps_equal_prefill():
    # one prefill call, then token-by-token decode through the returned state
    B, T, C, K = 3, 12, 256, 4
    x = _rand(B, T, C, dtype=torch.bfloat16, seed=5).to(DEV)
    w = _rand(C, K, dtype=torch.bfloat16, seed=6, scale=0.5).to(DEV)
    full, st_full = fused.conv_silu(x, w, None, None, None, num_heads=2, normalize=True, output_final_state=True)
    pre, st = fused.conv_silu(x[:, :5], w, None, None, None, num_heads=2, normalize=True, output_final_state=True)
    outs = [pre]
    for t in range(5, T):
        y, st = fused.conv_silu(x[:, t:t + 1], w, None, st, None, num_heads=2, normalize=True,
                                output_final_state=True)
        outs.append(y)
    assert torch.equal(torch.cat(outs, dim=1), full)
    assert torch.equal(st.buffer, st_full.buffer)


@pytest.mark.parametrize("taps", [1, 2, 8])
def test_conv_silu_kernel_sizes(taps):
    B, T, C = 1, 33, 128
    x = _rand(B, T, C, dtype=torch.float32, seed=7)
    w = _rand(C, taps, dtype=torch.float32, seed=8)
    hist = _rand(B, taps - 1, C, dtype=torch.float32, seed=9)
    ref_y, ref_h = ora.conv_silu(x, w, None, hist)
    y, st = fused.conv_silu(x.to(DEV), w.to(DEV), None, kda.ShortConvState(hist.to(DEV)),
                            output_final_state=True)
    assert rel_err(y, ref_y) < 1e-5
    if taps > 1:
        assert torch.equal(st.buffer.cpu(), ref_h)


def test_conv_silu_long_context_shape():
    # the q projection of the B=1 T=8192 H=16 d=128 prefill
    B, T, H, D = 1, 8192, 16, 128
    x = _rand(B, T, H * D, dtype=torch.bfloat16, seed=10)
    w = _rand(H * D, 4, dtype=torch.bfloat16, seed=11, scale=0.5)
    ref_y, _ = ora.conv_silu(x, w, None, None, None, num_heads=H, normalize=True)
    y, _ = fused.conv_silu(x.to(DEV), w.to(DEV), num_heads=H, normalize=True)
    assert rel_err(y.reshape(B, T, H * D), ref_y) < 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_gates_match_oracle(dtype):
    B, T, H, K = 2, 37, 3, 128
    z = _rand(B, T, H, K, dtype=dtype, seed=12, scale=3.0)
    zb = _rand(H, K, dtype=dtype, seed=13)
    a_log = _rand(H, dtype=torch.float32, seed=14, scale=0.5)
    bl = _rand(B, T, H, dtype=dtype, seed=15, scale=4.0)
    ref_g, ref_a = ora.lower_bounded_decay(z, a_log, -5.0, zb)
    g, alpha = fused.lower_bounded_decay(z.to(DEV), a_log.to(DEV), -5.0, bias=zb.to(DEV))
    assert g.dtype == dtype and alpha.dtype == dtype
    assert rel_err(g, ref_g) < TOL[dtype] and rel_err(alpha, ref_a) < TOL[dtype]
    beta = fused.beta_gate(bl.to(DEV))
    assert rel_err(beta, ora.beta_gate(bl)) < TOL[dtype]
    eps = torch.finfo(dtype).eps
    assert float(beta.min()) >= eps and float(beta.max()) <= 1 - eps
    assert float(g.max()) <= -5.0 * eps * (1 - 1e-3) and float(g.min()) >= -5.0


def test_gates_unaligned_logits_are_copied():
    z = _rand(1, 5, 2, 128, dtype=torch.bfloat16, seed=16).to(DEV)
    flat = torch.cat((torch.zeros(1, dtype=torch.bfloat16, device=DEV), z.flatten()))
    shifted = flat[1:].view(1, 5, 2, 128)  # 2-byte offset: not 16-byte aligned
    a_log = torch.zeros(2, device=DEV)
    g1, _ = fused.lower_bounded_decay(shifted, a_log)
    g2, _ = fused.lower_bounded_decay(z, a_log)
    assert torch.equal(g1, g2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("head_dim,per_head,gate", [(128, True, True), (64, False, False), (256, True, False)])
def test_rmsnorm_gate_matches_oracle(dtype, head_dim, per_head, gate):
    B, T, H = 2, 19, 3
    x = _rand(B, T, H, head_dim, dtype=dtype, seed=17, scale=2.0)
    w = _rand(*((H, head_dim) if per_head else (head_dim,)), dtype=dtype, seed=18)
    gl = _rand(B, T, H * head_dim, dtype=dtype, seed=19) if gate else None
    ref = ora.rmsnorm_gate(x, w, 1e-6, gl)
    y = fused.rmsnorm_gate(x.to(DEV), w.to(DEV), 1e-6, gate_logits=None if gl is None else gl.to(DEV))
    assert y.dtype == dtype and y.shape == x.shape
    assert rel_err(y, ref) < TOL[dtype]


def test_rmsnorm_gate_long_context_shape():
    B, T, H, D = 1, 8192, 16, 128
    x = _rand(B, T, H, D, dtype=torch.bfloat16, seed=20)
    w = _rand(H, D, dtype=torch.bfloat16, seed=21)
    gl = _rand(B, T, H * D, dtype=torch.bfloat16, seed=22)
    y = fused.rmsnorm_gate(x.to(DEV), w.to(DEV), 1e-6, gate_logits=gl.to(DEV))
    assert rel_err(y, ora.rmsnorm_gate(x, w, 1e-6, gl)) < 1e-2


@pytest.mark.parametrize("dtype,head_dim", [(torch.bfloat16, 16), (torch.float32, 32), (torch.float32, 512),
                                            (torch.float64, 256), (torch.float64, 512)])
def test_conv_silu_head_layouts(dtype, head_dim):
    # narrow heads (2-8 lanes) and heads wider than 64 16-byte vectors; K=6 takes the 8-tap kernel
    B, T, H, K = 2, 37, 2, 6
    C = H * head_dim
    x = _rand(B, T, C, dtype=dtype, seed=23)
    w = _rand(C, K, dtype=dtype, seed=24, scale=0.5)
    hist = _rand(B, K - 1, C, dtype=dtype, seed=25)
    mask = torch.arange(T)[None, :] < torch.tensor([T, 3])[:, None]
    ref_y, ref_h = ora.conv_silu(x, w, None, hist, mask, num_heads=H, normalize=True, eps=1e-6)
    y, st = fused.conv_silu(x.to(DEV), w.to(DEV), None, kda.ShortConvState(hist.to(DEV)), mask.to(DEV),
                            num_heads=H, normalize=True, eps=1e-6, output_final_state=True)
    assert rel_err(y.reshape(B, T, C), ref_y) < TOL[dtype]
    assert torch.equal(st.buffer.cpu(), ref_h)


def test_conv_silu_unaligned_input_is_copied():
    x = _rand(2, 20, 256, dtype=torch.bfloat16, seed=26).to(DEV)
    w = _rand(256, 4, dtype=torch.bfloat16, seed=27).to(DEV)
    flat = torch.cat((torch.zeros(1, dtype=torch.bfloat16, device=DEV), x.flatten()))
    shifted = flat[1:].view(2, 20, 256)  # 2-byte offset: not 16-byte aligned
    y1, _ = fused.conv_silu(shifted, w, num_heads=2, normalize=True)
    y2, _ = fused.conv_silu(x, w, num_heads=2, normalize=True)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("dtype,head_dim", [(torch.bfloat16, 16), (torch.float64, 32), (torch.float32, 512),
                                            (torch.float64, 512)])
def test_rmsnorm_gate_head_layouts(dtype, head_dim):
    B, T, H = 1, 11, 4
    x = _rand(B, T, H, head_dim, dtype=dtype, seed=28, scale=2.0)
    w = _rand(H, head_dim, dtype=dtype, seed=29)
    gl = _rand(B, T, H * head_dim, dtype=dtype, seed=30)
    y = fused.rmsnorm_gate(x.to(DEV), w.to(DEV), 1e-6, gate_logits=gl.to(DEV))
    assert rel_err(y, ora.rmsnorm_gate(x, w, 1e-6, gl)) < TOL[dtype]


def test_gates_beta_only_large():
    # more beta rows than one grid-stride pass covers
    bl = _rand(3, 8192, 40, dtype=torch.float32, seed=31, scale=4.0)
    beta = fused.beta_gate(bl.to(DEV))
    assert rel_err(beta, ora.beta_gate(bl)) < 1e-5
