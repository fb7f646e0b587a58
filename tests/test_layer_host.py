"""Host-side checks of the caller harness (kda/layer.py): KDALayerWeights takes
a module with the reference's attribute names (src/kda/kda.py:45-62,
src/kda/projections.py:35-73, src/kda/decay.py:24-26,
src/kimi_primitives/output_gate.py:34-39) and hands over either detached
views (inference) or the parameters themselves (training).  No GPU."""

from __future__ import annotations

from types import SimpleNamespace

import torch

from kda.layer import KDALayerWeights

H, K, V, D, CONV, RANK = 2, 8, 8, 16, 4, 4


def _linear(out_f, in_f, bias):
    return SimpleNamespace(weight=torch.nn.Parameter(torch.randn(out_f, in_f)),
                           bias=torch.nn.Parameter(torch.randn(out_f)) if bias else None)


def _conv(width, bias):
    return SimpleNamespace(weight=torch.nn.Parameter(torch.randn(width, CONV)),
                           bias=torch.nn.Parameter(torch.randn(width)) if bias else None)


def _module(bias):
    torch.manual_seed(0)
    proj = SimpleNamespace(
        q_proj=_linear(H * K, D, bias), k_proj=_linear(H * K, D, bias), v_proj=_linear(H * V, D, bias),
        q_conv=_conv(H * K, bias), k_conv=_conv(H * K, bias), v_conv=_conv(H * V, bias),
        beta_proj=_linear(H, D, bias), alpha_down=_linear(RANK, D, False), alpha_up=_linear(H * K, RANK, False),
        b_alpha=torch.nn.Parameter(torch.randn(H * K)),
    )
    cfg = SimpleNamespace(num_heads=H, key_head_dim=K, value_head_dim=V, g_min=-5.0, eps=1e-6,
                          accumulate_state_in_fp32=True)
    return SimpleNamespace(
        config=cfg, projections=proj, decay=SimpleNamespace(A_log=torch.nn.Parameter(torch.randn(H))),
        output_norm=SimpleNamespace(weight=torch.nn.Parameter(torch.randn(H, V))),
        output_gate=SimpleNamespace(gate_proj=_linear(D, D, bias), output_proj=_linear(D, D, bias)),
    )


def test_from_module_maps_every_parameter():
    m = _module(bias=True)
    w = KDALayerWeights.from_module(m)
    p = m.projections
    pairs = {
        "q_proj": p.q_proj.weight, "k_proj": p.k_proj.weight, "v_proj": p.v_proj.weight,
        "q_conv": p.q_conv.weight, "k_conv": p.k_conv.weight, "v_conv": p.v_conv.weight,
        "beta_proj": p.beta_proj.weight, "alpha_down": p.alpha_down.weight, "alpha_up": p.alpha_up.weight,
        "b_alpha": p.b_alpha, "a_log": m.decay.A_log, "norm_weight": m.output_norm.weight,
        "gate_proj": m.output_gate.gate_proj.weight, "output_proj": m.output_gate.output_proj.weight,
        "q_proj_bias": p.q_proj.bias, "k_proj_bias": p.k_proj.bias, "v_proj_bias": p.v_proj.bias,
        "q_conv_bias": p.q_conv.bias, "k_conv_bias": p.k_conv.bias, "v_conv_bias": p.v_conv.bias,
        "beta_bias": p.beta_proj.bias, "gate_bias": m.output_gate.gate_proj.bias,
        "output_bias": m.output_gate.output_proj.bias,
    }
    for name, ref in pairs.items():
        got = getattr(w, name)
        assert torch.equal(got, ref), name
        assert not got.requires_grad, name  # detached views for inference
        assert got.data_ptr() == ref.data_ptr(), name  # no copy
    assert (w.d_model, w.key_width, w.value_width, w.conv_kernel_size) == (D, H * K, H * V, CONV)
    assert (w.num_heads, w.key_head_dim, w.value_head_dim, w.g_min, w.eps) == (H, K, V, -5.0, 1e-6)


def test_from_module_for_training_keeps_the_parameters():
    m = _module(bias=False)
    w = KDALayerWeights.from_module(m, detach=False)
    assert w.q_proj is m.projections.q_proj.weight and w.q_proj.requires_grad
    assert w.a_log is m.decay.A_log and w.output_proj is m.output_gate.output_proj.weight
    assert w.q_proj_bias is None and w.gate_bias is None and w.q_conv_bias is None
