"""Gradients of the fused stages (kda_conv_silu_bwd, kda_gates_bwd,
kda_rmsnorm_gate_bwd) against torch.autograd through the oracle's stages on
the CPU (the reference takes these gradients from autograd through
src/kda/projections.py:164-218, src/kda/decay.py:36-43,
src/kimi_primitives/short_conv.py:69-98, headwise_rmsnorm.py:39-64 and
output_gate.py:62-75), and torch.autograd.gradcheck of the GPU stages in
f64 (finite differences of the GPU forward).

Tolerances (max|x - ref| / max|ref| per gradient): f64 1e-10, f32 1e-5,
bf16 2e-2 against the oracle's autograd in f64 on the same values; the layer
under autograd in f64 1e-8.
"""

from __future__ import annotations

import pytest
import torch

from kda import ShortConvState, fused
from kda.layer import KDALayerWeights, kda_attention_forward
from oracle import kda_oracle as ora
from tests._inputs import layer_weights, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float64: 1e-10, torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _rand(*shape, seed=0, scale=1.0, dtype=torch.float64):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64) * scale).to(dtype)


def _leaves(*ts):
    """(GPU leaf, CPU f64 leaf) pairs of the same values."""
    out = []
    for t in ts:
        if t is None:
            out.append((None, None))
            continue
        out.append((t.to(DEV).requires_grad_(), t.detach().double().requires_grad_()))
    return out


def _cmp(label, pairs, dtype):
    for name, (g, r) in pairs.items():
        if r is None:
            continue
        # a gradient is rounded to its parameter's type (A_log is always f32)
        tol = max(TOL[dtype], 1e-6 if g.dtype == torch.float32 else 0.0)
        e = rel_err(g, r)
        print(f"{label} d{name}: {e:.2e}")
        assert e < tol, (label, name, e)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("taps", [4, 3])
@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("tokens", [37, 300, 2048])
def test_conv_silu_gradients(dtype, taps, normalize, tokens):
    # runs of 16 positions, 16 of them per block at K = 4 (8 for other K):
    # T = 37 is three runs of one block; T = 300 spans two blocks per channel
    # block, the waves' LDS reduction of dw and dbias in a full block and in
    # one with idle waves; T = 2048 sums dw and dbias over 8 (16) blocks
    B, T, H, D = 2, tokens, 4, 64
    C = H * D
    x = _rand(B, T, C, seed=1, dtype=dtype)
    w = _rand(C, taps, seed=2, scale=0.3, dtype=dtype)
    b = _rand(C, seed=3, scale=0.1, dtype=dtype)
    hist = _rand(B, taps - 1, C, seed=4, dtype=dtype)
    mask = torch.ones(B, T, dtype=torch.bool)
    mask[1, T - 8:] = False
    (xg, xr), (wg, wr), (bg, br), (hg, hr) = _leaves(x, w, b, hist)
    dy = _rand(B, T, C, seed=5, dtype=torch.float64)
    dh = _rand(B, taps - 1, C, seed=6, dtype=torch.float64)
    y, nxt = fused.conv_silu(xg, wg, bg, ShortConvState(hg), mask.to(DEV), num_heads=H, normalize=normalize,
                             output_final_state=True)
    ((y.double().reshape(B, T, C) * dy.to(DEV)).sum() + (nxt.buffer.double() * dh.to(DEV)).sum()).backward()
    ry, rn = ora.conv_silu(xr, wr, br, hr, mask, num_heads=H, normalize=normalize)
    ((ry * dy).sum() + (rn * dh).sum()).backward()
    _cmp(f"conv {dtype} T={T} K={taps} norm={normalize}", {"x": (xg.grad, xr.grad), "w": (wg.grad, wr.grad),
                                                      "b": (bg.grad, br.grad), "hist": (hg.grad, hr.grad)}, dtype)


def test_conv_silu_decode_step_gradients():
    # T = 1 through the history (the decode path), kernel size 4, bf16-free f64
    B, C, K = 3, 128, 4
    x = _rand(B, 1, C, seed=7)
    w = _rand(C, K, seed=8, scale=0.3)
    hist = _rand(B, K - 1, C, seed=9)
    (xg, xr), (wg, wr), (hg, hr) = _leaves(x, w, hist)
    y, nxt = fused.conv_silu(xg, wg, None, ShortConvState(hg), num_heads=2, normalize=True, output_final_state=True)
    (y.sum() + 0.5 * nxt.buffer.square().sum()).backward()
    ry, rn = ora.conv_silu(xr, wr, None, hr, num_heads=2, normalize=True)
    (ry.sum() + 0.5 * rn.square().sum()).backward()
    _cmp("conv decode", {"x": (xg.grad, xr.grad), "w": (wg.grad, wr.grad), "hist": (hg.grad, hr.grad)},
         torch.float64)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,H,K", [(33, 4, 64), (700, 64, 48)])
def test_decay_and_beta_gradients(dtype, T, H, K):
    # (700, 64, 48): blocks of several rows per row group, and heads whose
    # 16-byte positions straddle a block's 256 (48 channels are 6 of them in
    # bf16, 12 in f32, 24 in f64)
    B = 2
    z = _rand(B, T, H, K, seed=11, scale=2.0, dtype=dtype)
    z[0, :3] = 1000.0  # saturated for every head's exp(A_log) >= 0.2, in f64 too: clamped to 1 - eps, no gradient
    bias = _rand(H, K, seed=12, scale=0.5, dtype=dtype)
    a_log = _rand(H, seed=13, scale=0.3, dtype=torch.float32)
    bl = _rand(B, T, H, seed=14, dtype=dtype)
    (zg, zr), (bg, br), (ag, ar), (lg, lr) = _leaves(z, bias, a_log, bl)
    dgw, daw, dbw = _rand(B, T, H, K, seed=15), _rand(B, T, H, K, seed=16), _rand(B, T, H, seed=17)
    g, alpha = fused.lower_bounded_decay(zg, ag, -5.0, bias=bg)
    beta = fused.beta_gate(lg)
    ((g.double() * dgw.to(DEV)).sum() + (alpha.double() * daw.to(DEV)).sum()
     + (beta.double() * dbw.to(DEV)).sum()).backward()
    # the oracle's formulas (oracle.lower_bounded_decay / beta_gate) in f64, with
    # the clamp bounds of the tensors' dtype (src/kda/decay.py:40, projections.py:208)
    eps = torch.finfo(dtype).eps
    rg = -5.0 * torch.sigmoid(ar.exp()[None, None, :, None] * (zr + br)).clamp(eps, 1 - eps)
    ralpha = rg.exp()
    rbeta = torch.sigmoid(lr).clamp(eps, 1 - eps)
    if dtype == torch.float64:
        og, oalpha = ora.lower_bounded_decay(zr.detach(), ar.detach(), -5.0, bias=br.detach())
        assert torch.equal(og, rg.detach()) and torch.equal(ora.beta_gate(lr.detach()), rbeta.detach())
    ((rg * dgw).sum() + (ralpha * daw).sum() + (rbeta * dbw).sum()).backward()
    assert torch.count_nonzero(zg.grad[0, :3]) == 0
    _cmp(f"gates {dtype}", {"z": (zg.grad, zr.grad), "bias": (bg.grad, br.grad), "a_log": (ag.grad, ar.grad),
                            "beta_logits": (lg.grad, lr.grad)}, dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("weight", ["per_head", "shared", None])
@pytest.mark.parametrize("gate", [True, False])
@pytest.mark.parametrize("T", [21, 2100])
def test_rmsnorm_gate_gradients(dtype, weight, gate, T):
    # T = 2100 (4200 rows): a head's blocks stride over its rows more than once
    B, H, D = 2, 4, 128
    x = _rand(B, T, H, D, seed=21, dtype=dtype)
    w = None if weight is None else _rand(*((H, D) if weight == "per_head" else (D,)), seed=22, scale=0.5,
                                          dtype=dtype) + 1
    gl = _rand(B, T, H * D, seed=23, dtype=dtype) if gate else None
    (xg, xr), (wg, wr), (gg, gr) = _leaves(x, w, gl)
    dy = _rand(B, T, H, D, seed=24)
    (fused.rmsnorm_gate(xg, wg, 1e-6, gate_logits=gg).double() * dy.to(DEV)).sum().backward()
    (ora.rmsnorm_gate(xr, wr, 1e-6, gate_logits=gr) * dy).sum().backward()
    _cmp(f"norm {dtype} w={weight} gate={gate}", {"x": (xg.grad, xr.grad),
                                                  "w": (None if wg is None else wg.grad, None if wr is None else wr.grad),
                                                  "gate": (None if gg is None else gg.grad,
                                                           None if gr is None else gr.grad)}, dtype)


def test_gradcheck_of_the_gpu_stages():
    # finite differences of the GPU forward itself, in f64
    gen = lambda *s: torch.randn(*s, dtype=torch.float64, device=DEV).requires_grad_()  # noqa: E731
    torch.manual_seed(0)
    x, w, b, h = gen(1, 9, 32), (0.3 * torch.randn(32, 4, dtype=torch.float64, device=DEV)).requires_grad_(), \
        gen(32), gen(1, 3, 32)
    assert torch.autograd.gradcheck(
        lambda x, w, b, h: fused.conv_silu(x, w, b, ShortConvState(h), num_heads=2, normalize=True,
                                           output_final_state=True)[0], (x, w, b, h))
    z, bias, a_log = gen(1, 5, 2, 16), gen(2, 16), (0.2 * torch.randn(2, dtype=torch.float64, device=DEV))
    a32 = a_log.float().requires_grad_()
    assert torch.autograd.gradcheck(lambda z, b: fused.lower_bounded_decay(z, a32.detach(), -5.0, bias=b), (z, bias))
    xn, wn, gl = gen(1, 3, 2, 16), gen(2, 16), gen(1, 3, 32)
    assert torch.autograd.gradcheck(lambda x, w, g: fused.rmsnorm_gate(x, w, 1e-6, gate_logits=g), (xn, wn, gl))
    assert torch.autograd.gradcheck(fused.beta_gate, (gen(2, 7, 3),))


def test_layer_trains_through_the_backend_f64():
    # the whole layer under autograd (src/kda/kda.py:98-183; training in
    # attention_layer.py:114): every weight and the input get the gradients of
    # the oracle layer's autograd
    cfg = dict(d_model=32, heads=2, key_dim=16, value_dim=16, conv=4, rank=8)
    w = layer_weights(cfg["d_model"], cfg["heads"], cfg["key_dim"], cfg["value_dim"], conv=cfg["conv"],
                      rank=cfg["rank"], dtype=torch.float64, seed=31, biases=True)
    w["a_log"] = w["a_log"].double()
    names = [k for k, v in w.items() if isinstance(v, torch.Tensor)]
    gw = {k: (w[k].to(DEV).requires_grad_() if k in names else w[k]) for k in w}
    rw = {k: (w[k].clone().requires_grad_() if k in names else w[k]) for k in w}
    x = _rand(2, 70, cfg["d_model"], seed=32)
    mask = torch.ones(2, 70, dtype=torch.bool)
    mask[1, 60:] = False
    xg, xr = x.to(DEV).requires_grad_(), x.clone().requires_grad_()
    dy = _rand(2, 70, cfg["d_model"], seed=33)
    out = kda_attention_forward(KDALayerWeights(**gw), xg, mask.to(DEV), mode="chunkwise", output_final_state=True)
    ((out.hidden_states * dy.to(DEV)).sum() + out.state.recurrent_state.square().sum()).backward()
    ro, rst = ora.kda_layer(rw, xr, mask, mode="chunkwise", output_final_state=True)
    ((ro * dy).sum() + rst[0].square().sum()).backward()
    worst = 0.0
    for k in names + ["x"]:
        gt, rt = (xg, xr) if k == "x" else (gw[k], rw[k])
        e = rel_err(gt.grad, rt.grad)
        worst = max(worst, e)
        print(f"layer d{k}: {e:.2e}")
    assert worst < 1e-8


def test_parameter_gradients_under_deterministic_mode():
    # the parameter gradients are summed with float atomics: deterministic
    # mode raises for them (as torch's nondeterministic ops do), warns with
    # warn_only, and leaves input-only gradients alone
    x = _rand(1, 40, 128, seed=21, dtype=torch.float32).to(DEV).requires_grad_()
    w = _rand(128, 4, seed=22, scale=0.3, dtype=torch.float32).to(DEV)
    try:
        torch.use_deterministic_algorithms(True)
        y, _ = fused.conv_silu(x, w, num_heads=2, normalize=True)
        y.sum().backward()  # input gradient only: allowed
        assert x.grad is not None
        wg = w.clone().requires_grad_()
        y, _ = fused.conv_silu(x, wg, num_heads=2, normalize=True)
        with pytest.raises(RuntimeError, match="deterministic"):
            y.sum().backward()
        torch.use_deterministic_algorithms(True, warn_only=True)
        y, _ = fused.conv_silu(x, wg, num_heads=2, normalize=True)
        with pytest.warns(UserWarning, match="deterministic"):
            y.sum().backward()
        assert wg.grad is not None
    finally:
        torch.use_deterministic_algorithms(False)
