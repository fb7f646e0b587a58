"""Fused stages around the KDA operator, one HIP kernel each.

* ``conv_silu``: the ShortConv + SiLU (+ per-head L2 normalisation for q and
  k) that KDAProjections applies to each projection
  (src/kda/projections.py:100-140,164-206 over CausalShortConv1D,
  src/kimi_primitives/short_conv.py:69-98), with its incremental history and
  right-padding semantics; decode is the T=1 case.
* ``lower_bounded_decay`` / ``beta_gate``: LowerBoundedDecay
  (src/kda/decay.py:30-43, with the decay-logit bias of
  projections.py:211-218) and the beta gate (projections.py:207-209).
* ``chunkwise_kda_with_decay``: the decay and the chunkwise operator in one
  pass, g formed from the logits inside the chunk kernel (no HBM round trip
  of g).
* ``rmsnorm_gate``: HeadwiseRMSNorm (src/kimi_primitives/headwise_rmsnorm.py:39-64)
  times the sigmoid output gate (src/kimi_primitives/output_gate.py:62-75),
  i.e. the input of the output projection.

Every function runs on the tensors' GPU stream through libkda_mi355x.so and
returns new tensors; there is no CPU fallback.  Arithmetic is f32 (f64 for
f64 tensors) with one rounding to the tensors' dtype, where the reference
rounds after each step in the model dtype.
"""

from __future__ import annotations

import warnings

import torch

from . import _lib, _prep
from .state import ShortConvState
from .utils import validate_attention_mask

_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float64)


def _alert_nondeterministic(what: str) -> None:
    """The parameter gradients of the fused-stage backwards are summed over
    workgroups with float atomics, so their rounding can change from run to
    run.  Under ``torch.use_deterministic_algorithms(True)`` this raises, as
    torch's own nondeterministic operations do (a warning with
    ``warn_only=True``); the input gradients are deterministic and unaffected."""
    if not torch.are_deterministic_algorithms_enabled():
        return
    msg = (f"{what} sums its parameter gradients with float atomics and has no deterministic "
           "implementation; turn off torch.use_deterministic_algorithms or keep the parameters frozen")
    if torch.is_deterministic_algorithms_warn_only_enabled():
        warnings.warn(msg)
    else:
        raise RuntimeError(msg)


def _check_dtype(name: str, tensor: torch.Tensor, dtype: torch.dtype) -> None:
    if tensor.dtype != dtype:
        raise TypeError(f"{name} must have dtype {dtype}, got {tensor.dtype}")


def _check_device(name: str, tensor: torch.Tensor, device: torch.device) -> None:
    if tensor.device != device:
        raise ValueError(f"{name} must be on {device}, got {tensor.device}")


def _aligned(tensor: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the kernels move 16-byte vectors)."""
    tensor = tensor.contiguous()
    return tensor if tensor.data_ptr() % 16 == 0 else tensor.clone()


def conv_silu(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    state: ShortConvState | None = None,
    attention_mask: torch.Tensor | None = None,
    *,
    num_heads: int | None = None,
    normalize: bool = False,
    eps: float = 1e-6,
    output_final_state: bool = False,
) -> tuple[torch.Tensor, ShortConvState | None]:
    """Depthwise causal ShortConv over ``x [B,T,C]``, SiLU, and optionally
    L2 normalisation over each of ``num_heads`` heads.

    ``weight [C,K]`` is in lag order (``weight[c, j]`` multiplies ``x[t-j]``,
    short_conv.py:12-18); ``state`` carries the last ``K-1`` inputs.  Right
    padding (``attention_mask``) gives zero outputs and never enters the
    returned history (projections.py:119-140).  Returns ``y`` as ``[B,T,H,C/H]``
    when ``num_heads`` is given (``[B,T,C]`` otherwise) and the next state when
    ``output_final_state``.
    """
    if x.ndim != 3:
        raise ValueError(f"x must have shape [B,T,C], got {tuple(x.shape)}")
    batch, tokens, channels = x.shape
    if tokens == 0:
        raise ValueError("conv_silu does not support empty sequences")
    if x.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {x.dtype}")
    if weight.ndim != 2 or weight.shape[0] != channels or weight.shape[1] < 1:
        raise ValueError(f"weight must have shape [{channels},K], got {tuple(weight.shape)}")
    kernel_size = weight.shape[1]
    _check_dtype("weight", weight, x.dtype)
    _check_device("weight", weight, x.device)
    if bias is not None:
        if bias.shape != (channels,):
            raise ValueError(f"bias must have shape [{channels}], got {tuple(bias.shape)}")
        _check_dtype("bias", bias, x.dtype)
        _check_device("bias", bias, x.device)
    if state is not None:
        expected = (batch, kernel_size - 1, channels)
        if state.buffer.shape != expected:
            raise ValueError(f"state buffer must have shape {expected}, got {tuple(state.buffer.shape)}")
        _check_dtype("state buffer", state.buffer, x.dtype)
        _check_device("state buffer", state.buffer, x.device)
    if num_heads is not None and (num_heads <= 0 or channels % num_heads != 0):
        raise ValueError(f"channels {channels} must split into num_heads={num_heads} heads")
    if normalize and num_heads is None:
        raise ValueError("normalize needs num_heads")
    if eps <= 0:
        raise ValueError("eps must be > 0")
    validate_attention_mask(attention_mask, batch, tokens)
    _lib.require_gpu(x)
    head_dim = channels // num_heads if num_heads is not None else channels
    hist = None if state is None else state.buffer
    valid = _prep.valid_lengths(attention_mask, x.device)
    cfg = (head_dim, bool(normalize), float(eps), bool(output_final_state))
    if _needs_grad(x, weight, bias, hist):
        y, hist_out = _ConvSilu.apply(x, weight, bias, hist, valid, cfg)
        if not output_final_state:
            hist_out = None
    else:
        y, hist_out = _conv_forward(x, weight, bias, hist, valid, *cfg)
    if num_heads is not None:
        y = y.view(batch, tokens, num_heads, head_dim)
    return y, (ShortConvState(hist_out) if hist_out is not None else None)


def _needs_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def _conv_forward(x, weight, bias, hist, valid, head_dim, normalize, eps, want_hist):
    lib = _lib.load()
    batch, tokens, channels = x.shape
    kernel_size = weight.shape[1]
    xc = _aligned(x)
    wc = weight.contiguous()
    bc = None if bias is None else bias.contiguous()
    hc = None if hist is None or kernel_size == 1 else _aligned(hist)
    y = torch.empty_like(xc)
    hist_out = None
    if want_hist:
        hist_out = torch.empty(batch, kernel_size - 1, channels, dtype=x.dtype, device=x.device)
    status = lib.kda_conv_silu_fwd(
        xc.data_ptr(), wc.data_ptr(), _lib.ptr(bc), _lib.ptr(hc), y.data_ptr(),
        _lib.ptr(hist_out) if hist_out is not None and kernel_size > 1 else None, _lib.ptr(valid),
        batch, tokens, channels, kernel_size, head_dim, 1 if normalize else 0, float(eps),
        _lib.dtype_code(x.dtype), _prep.stream(x.device),
    )
    _lib.check(status)
    return y, hist_out


def _acc_dtype(dtype: torch.dtype) -> torch.dtype:
    """Type of the kernels' parameter-gradient accumulators."""
    return torch.float64 if dtype == torch.float64 else torch.float32


class _ConvSilu(torch.autograd.Function):
    """conv_silu under autograd: the native forward and ``kda_conv_silu_bwd``
    (input, weight, bias and history gradients; the returned history's own
    gradient flows back to the inputs it was copied from)."""

    @staticmethod
    def forward(ctx, x, weight, bias, hist, valid, cfg):
        y, hist_out = _conv_forward(x, weight, bias, hist, valid, *cfg)
        ctx.save_for_backward(x, weight, bias, hist, valid)
        ctx.cfg = cfg
        if hist_out is None:
            hist_out = torch.empty(0, dtype=x.dtype, device=x.device)
            ctx.mark_non_differentiable(hist_out)
        return y, hist_out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dy, dhist):
        x, weight, bias, hist, valid = ctx.saved_tensors
        head_dim, normalize, eps, want_hist = ctx.cfg
        lib = _lib.load()
        batch, tokens, channels = x.shape
        kernel_size = weight.shape[1]
        if dy is None:
            dy = torch.zeros_like(x)
        dyc = _aligned(dy.to(x.dtype))
        dh = None
        if want_hist and dhist is not None and dhist.numel() > 0 and kernel_size > 1:
            dh = _aligned(dhist.to(x.dtype))
        xc = _aligned(x)
        hc = None if hist is None or kernel_size == 1 else _aligned(hist)
        dx = torch.empty_like(xc)
        need_w, need_b, need_h = ctx.needs_input_grad[1], ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        if need_w or (need_b and bias is not None):
            _alert_nondeterministic("the ShortConv+SiLU backward (kda_conv_silu_bwd)")
        acc = _acc_dtype(x.dtype)
        dw = torch.zeros(channels, kernel_size, dtype=acc, device=x.device) if need_w else None
        db = torch.zeros(channels, dtype=acc, device=x.device) if need_b and bias is not None else None
        dhi = torch.empty_like(hc) if need_h and hc is not None else None
        _lib.check(lib.kda_conv_silu_bwd(
            xc.data_ptr(), weight.contiguous().data_ptr(), _lib.ptr(None if bias is None else bias.contiguous()),
            _lib.ptr(hc), _lib.ptr(valid), dyc.data_ptr(), _lib.ptr(dh), dx.data_ptr(), _lib.ptr(dhi),
            _lib.ptr(dw), _lib.ptr(db), batch, tokens, channels, kernel_size, head_dim, 1 if normalize else 0,
            float(eps), _lib.dtype_code(x.dtype), _prep.stream(x.device),
        ))
        if need_h and hist is not None and dhi is None:
            dhi = torch.zeros_like(hist)  # kernel size 1: the history is never read
        return (dx if ctx.needs_input_grad[0] else None,
                None if dw is None else dw.to(weight.dtype),
                None if db is None else db.to(bias.dtype),
                dhi, None, None)


def _gates(decay_logits, a_log, g_min, bias, beta_logits, want_alpha):
    ref = decay_logits if decay_logits is not None else beta_logits
    if ref.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {ref.dtype}")
    g = alpha = beta = None
    rows = heads = key_dim = 0
    z = zb = al = None
    if decay_logits is not None:
        if decay_logits.ndim != 4:
            raise ValueError(f"logits must have shape [B,T,H,K], got {tuple(decay_logits.shape)}")
        batch, tokens, heads, key_dim = decay_logits.shape
        rows = batch * tokens
        _lib.require_gpu(decay_logits)
        if a_log.shape != (heads,):
            raise ValueError(f"A_log must have shape [{heads}], got {tuple(a_log.shape)}")
        _check_device("A_log", a_log, decay_logits.device)
        if g_min >= 0:
            raise ValueError("g_min must be negative")
        if bias is not None:
            if bias.shape != (heads, key_dim):
                raise ValueError(f"bias must have shape [{heads},{key_dim}], got {tuple(bias.shape)}")
            _check_device("bias", bias, decay_logits.device)
            zb = _aligned(bias.to(decay_logits.dtype))
        z = _aligned(decay_logits)
        al = a_log.to(torch.float32).contiguous()
        g = torch.empty_like(z)
        alpha = torch.empty_like(z) if want_alpha else None
    if beta_logits is not None:
        if beta_logits.ndim < 1:
            raise ValueError("beta logits must have at least one dimension")
        _lib.require_gpu(beta_logits)
        bl = beta_logits.contiguous()
        beta = torch.empty_like(bl)
        if decay_logits is None:
            rows, heads, key_dim = 1, bl.numel(), 1
        elif bl.numel() != rows * heads:
            raise ValueError("beta logits must have shape [B,T,H] matching the decay logits")
    else:
        bl = None
    lib = _lib.load()
    status = lib.kda_gates_fwd(
        _lib.ptr(z), _lib.ptr(zb), _lib.ptr(al), float(g_min), _lib.ptr(g), _lib.ptr(alpha),
        _lib.ptr(bl), _lib.ptr(beta), rows, heads, key_dim, _lib.dtype_code(ref.dtype), _prep.stream(ref.device),
    )
    _lib.check(status)
    return g, alpha, beta


def lower_bounded_decay(
    logits: torch.Tensor,
    a_log: torch.Tensor,
    g_min: float = -5.0,
    *,
    bias: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(g, exp(g))`` with ``g = g_min * clamp(sigmoid(exp(A_log) * (logits + bias)), eps, 1-eps)``
    for ``logits [B,T,H,K]``, ``A_log [H]`` and an optional bias ``[H,K]``
    (decay.py:30-43; eps is the dtype's machine epsilon).  Differentiable in
    the logits, A_log and the bias (``kda_gates_bwd``)."""
    if _needs_grad(logits, a_log, bias):
        return _Decay.apply(logits, a_log, bias, float(g_min))
    g, alpha, _ = _gates(logits, a_log, g_min, bias, None, True)
    return g, alpha


def beta_gate(logits: torch.Tensor) -> torch.Tensor:
    """``clamp(sigmoid(logits), eps, 1-eps)`` elementwise (projections.py:207-209);
    differentiable (``kda_gates_bwd``)."""
    if _needs_grad(logits):
        return _Beta.apply(logits)
    _, _, beta = _gates(None, None, -1.0, None, logits, False)
    return beta


class _Decay(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, a_log, bias, g_min):
        g, alpha, _ = _gates(logits, a_log, g_min, bias, None, True)
        ctx.save_for_backward(logits, a_log, bias)
        ctx.g_min = g_min
        return g, alpha

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dg, dalpha):
        logits, a_log, bias = ctx.saved_tensors
        lib = _lib.load()
        batch, tokens, heads, key_dim = logits.shape
        z = _aligned(logits)
        zb = None if bias is None else _aligned(bias.to(logits.dtype))
        al = a_log.to(torch.float32).contiguous()
        if dg is None:
            dg = torch.zeros_like(z)
        dgc = _aligned(dg.to(z.dtype))
        dac = None if dalpha is None else _aligned(dalpha.to(z.dtype))
        dz = torch.empty_like(z)
        acc = _acc_dtype(z.dtype)
        dzb = torch.zeros(heads, key_dim, dtype=acc, device=z.device) if bias is not None and ctx.needs_input_grad[2] \
            else None
        dal = torch.zeros(heads, dtype=acc, device=z.device) if ctx.needs_input_grad[1] else None
        if dzb is not None or dal is not None:
            _alert_nondeterministic("the decay gate backward (kda_gates_bwd)")
        _lib.check(lib.kda_gates_bwd(
            z.data_ptr(), _lib.ptr(zb), al.data_ptr(), ctx.g_min, dgc.data_ptr(), _lib.ptr(dac), dz.data_ptr(),
            _lib.ptr(dzb), _lib.ptr(dal), None, None, None, batch * tokens, heads, key_dim,
            _lib.dtype_code(z.dtype), _prep.stream(z.device),
        ))
        return (dz if ctx.needs_input_grad[0] else None, None if dal is None else dal.to(a_log.dtype),
                None if dzb is None else dzb.to(bias.dtype), None)


class _Beta(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits):
        _, _, beta = _gates(None, None, -1.0, None, logits, False)
        ctx.save_for_backward(logits)
        return beta

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dbeta):
        (logits,) = ctx.saved_tensors
        lib = _lib.load()
        bl = logits.contiguous()
        db = dbeta.to(bl.dtype).contiguous()
        dl = torch.empty_like(bl)
        _lib.check(lib.kda_gates_bwd(
            None, None, None, -1.0, None, None, None, None, None, bl.data_ptr(), db.data_ptr(), dl.data_ptr(),
            1, bl.numel(), 1, _lib.dtype_code(bl.dtype), _prep.stream(bl.device),
        ))
        return dl


def chunkwise_kda_with_decay(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    decay_logits: torch.Tensor,
    a_log: torch.Tensor,
    beta: torch.Tensor,
    *,
    decay_bias: torch.Tensor | None = None,
    g_min: float = -5.0,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    attention_mask: torch.Tensor | None = None,
    accumulate_state_in_fp32: bool = True,
    cu_seqlens: torch.Tensor | list[int] | None = None,
):
    """``chunkwise_kda(q, k, v, g, beta, ...)`` with ``g = lower_bounded_decay(
    decay_logits, a_log, g_min, bias=decay_bias)[0]`` (src/kda/decay.py:36-43,
    src/kda/kda.py:131-151), the decay formed inside the chunk kernel so that g
    never makes a round trip through HBM.  The result equals the two-step
    composition bit for bit.  Shapes off the MFMA path (K above 128 or not a
    multiple of 16, V not a multiple of 16 in 16..256, f32/f64 inputs) and calls under autograd run the
    two steps (both in HIP kernels); so does f16/bf16 work without an f32 state."""
    from .chunkwise import chunkwise_kda, needs_grad
    from .recurrent import KDAOperatorOutput
    from .utils import accumulation_dtype, validate_core_inputs, validate_cu_seqlens

    offsets = None
    if cu_seqlens is not None:
        offsets = validate_cu_seqlens(cu_seqlens, q.shape[0] if q.ndim == 4 else -1,
                                      q.shape[1] if q.ndim == 4 else -1, attention_mask)
    num_states = None if offsets is None else len(offsets) - 1
    batch, tokens, heads, key_dim, value_dim = validate_core_inputs(
        q, k, v, decay_logits, beta, initial_state, attention_mask, num_states=num_states)
    _lib.require_gpu(q)
    if a_log.shape != (heads,):
        raise ValueError(f"A_log must have shape [{heads}], got {tuple(a_log.shape)}")
    if decay_bias is not None and decay_bias.shape != (heads, key_dim):
        raise ValueError(f"bias must have shape [{heads},{key_dim}], got {tuple(decay_bias.shape)}")
    if g_min >= 0:
        raise ValueError("g_min must be negative")
    work_dtype = accumulation_dtype(v.dtype, accumulate_state_in_fp32)
    dtypes = {t.dtype for t in (q, k, v, decay_logits, beta)}
    fused_ok = (len(dtypes) == 1 and q.dtype in (torch.bfloat16, torch.float16) and work_dtype == torch.float32
                and key_dim <= 128 and key_dim % 16 == 0 and value_dim % 16 == 0 and 16 <= value_dim <= 256
                and not needs_grad(q, k, v, decay_logits, beta, initial_state, a_log, decay_bias))
    if not fused_ok:
        g, _ = lower_bounded_decay(decay_logits, a_log, g_min, bias=decay_bias)
        return chunkwise_kda(q, k, v, g, beta, initial_state, output_final_state, attention_mask,
                             accumulate_state_in_fp32=accumulate_state_in_fp32, cu_seqlens=cu_seqlens)
    lib = _lib.load()
    device = q.device
    qc, kc, vc, zc, bc = (t.contiguous() for t in (q, k, v, decay_logits, beta))
    zb = None if decay_bias is None else decay_bias.to(device=device, dtype=q.dtype).contiguous()
    al = a_log.to(device=device, dtype=torch.float32).contiguous()
    n_seq = batch if offsets is None else len(offsets) - 1
    total = batch * tokens
    s_in = _prep.state_arg(initial_state, torch.float32)
    s_out = (torch.empty(n_seq, heads, key_dim, value_dim, dtype=torch.float32, device=device)
             if output_final_state else None)
    out = torch.empty(batch, tokens, heads, value_dim, dtype=q.dtype, device=device)
    cu = None if offsets is None else _prep.cu_tensor(offsets, device)
    valid = _prep.valid_lengths(attention_mask, device)
    code = _lib.dtype_code(q.dtype)
    longest = _prep.longest_document(offsets)
    ws_bytes = lib.kda_chunk_fwd_workspace_bytes(n_seq, total, longest, heads, key_dim, value_dim, code)
    workspace = _prep.workspace(ws_bytes, device, "chunkwise_kda_with_decay")
    _lib.check(lib.kda_chunk_fwd_decay(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), zc.data_ptr(), _lib.ptr(zb), al.data_ptr(), float(g_min),
        bc.data_ptr(), code, _lib.ptr(s_in), _lib.ptr(s_out), _lib.dtype_code(torch.float32), out.data_ptr(),
        _lib.ptr(cu), tokens if offsets is None else longest, _lib.ptr(valid), n_seq, total, heads, key_dim,
        value_dim, _lib.ptr(workspace), ws_bytes, _prep.stream(device)))
    hidden = out if out.dtype == v.dtype else out.to(v.dtype)
    return KDAOperatorOutput(hidden_states=hidden, final_state=s_out)


def rmsnorm_gate(
    x: torch.Tensor,
    weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    *,
    gate_logits: torch.Tensor | None = None,
) -> torch.Tensor:
    """Head-wise RMSNorm of ``x [B,T,H,D]`` (weight ``[H,D]`` per head, ``[D]``
    shared, or None), times ``sigmoid(gate_logits)`` (``[B,T,H*D]``) when given.
    headwise_rmsnorm.py:39-64 and output_gate.py:62-75."""
    if x.ndim != 4:
        raise ValueError(f"x must have shape [B,T,H,Dh], got {tuple(x.shape)}")
    if x.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {x.dtype}")
    batch, tokens, heads, head_dim = x.shape
    per_head = 0
    if weight is not None:
        if weight.shape == (heads, head_dim):
            per_head = 1
        elif weight.shape != (head_dim,):
            raise ValueError(f"weight must have shape [{heads},{head_dim}] or [{head_dim}], got {tuple(weight.shape)}")
        _check_device("weight", weight, x.device)
    if gate_logits is not None:
        if gate_logits.shape != (batch, tokens, heads * head_dim):
            raise ValueError(
                f"gate_logits must have shape {(batch, tokens, heads * head_dim)}, got {tuple(gate_logits.shape)}"
            )
        _check_dtype("gate_logits", gate_logits, x.dtype)
        _check_device("gate_logits", gate_logits, x.device)
    if eps <= 0:
        raise ValueError("eps must be > 0")
    _lib.require_gpu(x)
    if _needs_grad(x, weight, gate_logits):
        return _RMSNormGate.apply(x, weight, gate_logits, float(eps), per_head)
    return _norm_forward(x, weight, gate_logits, eps, per_head)


def _norm_forward(x, weight, gate_logits, eps, per_head):
    lib = _lib.load()
    batch, tokens, heads, head_dim = x.shape
    xc = _aligned(x)
    wc = None if weight is None else _aligned(weight.to(x.dtype))
    gc = None if gate_logits is None else _aligned(gate_logits)
    y = torch.empty_like(xc)
    status = lib.kda_rmsnorm_gate_fwd(
        xc.data_ptr(), _lib.ptr(wc), per_head, _lib.ptr(gc), y.data_ptr(), batch * tokens, heads, head_dim,
        float(eps), _lib.dtype_code(x.dtype), _prep.stream(x.device),
    )
    _lib.check(status)
    return y


class _RMSNormGate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, gate_logits, eps, per_head):
        y = _norm_forward(x, weight, gate_logits, eps, per_head)
        ctx.save_for_backward(x, weight, gate_logits)
        ctx.cfg = (eps, per_head)
        return y

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dy):
        x, weight, gate_logits = ctx.saved_tensors
        eps, per_head = ctx.cfg
        lib = _lib.load()
        batch, tokens, heads, head_dim = x.shape
        xc = _aligned(x)
        wc = None if weight is None else _aligned(weight.to(x.dtype))
        gc = None if gate_logits is None else _aligned(gate_logits)
        dyc = _aligned(dy.to(x.dtype))
        dx = torch.empty_like(xc)
        dgl = None if gc is None else torch.empty_like(gc)
        dw = None
        if weight is not None and ctx.needs_input_grad[1]:
            dw = torch.zeros(weight.shape, dtype=_acc_dtype(x.dtype), device=x.device)
            _alert_nondeterministic("the RMSNorm x gate backward (kda_rmsnorm_gate_bwd)")
        _lib.check(lib.kda_rmsnorm_gate_bwd(
            xc.data_ptr(), _lib.ptr(wc), per_head, _lib.ptr(gc), dyc.data_ptr(), dx.data_ptr(), _lib.ptr(dgl),
            _lib.ptr(dw), batch * tokens, heads, head_dim, float(eps), _lib.dtype_code(x.dtype),
            _prep.stream(x.device),
        ))
        return (dx if ctx.needs_input_grad[0] else None, None if dw is None else dw.to(weight.dtype),
                dgl if gate_logits is not None and ctx.needs_input_grad[2] else None, None, None)


__all__ = ["beta_gate", "chunkwise_kda_with_decay", "conv_silu", "lower_bounded_decay", "rmsnorm_gate"]
