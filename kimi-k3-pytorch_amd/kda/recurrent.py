"""Exact token recurrence (decode and ``mode="recurrent"``) on the gfx950 backend.

Drop-in for ``recurrent_kda`` (src/kda/recurrent.py:25-80): same signature,
defaults, validation errors and dtype rules; the arithmetic runs in the HIP
kernel behind ``kda_recurrent_fwd`` / ``kda_decode_step``.

Additive keyword-only extensions (every existing call is unchanged):
* ``cu_seqlens``: packed documents ``[1, sum T, H, *]``; each document is an
  independent recurrence, ``initial_state``/``final_state`` are ``[N,H,K,V]``.
* ``update_state_in_place``: write the new state into ``initial_state``
  (which must already be contiguous and in the work dtype) and return it as
  ``final_state``; the default keeps the reference's functional update
  (src/kda/recurrent.py:50-59).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, _prep
from .utils import accumulation_dtype, validate_core_inputs, validate_cu_seqlens


@dataclass
class KDAOperatorOutput:
    """Output and updated recurrent matrix from a KDA operator backend
    (src/kda/recurrent.py:16-22)."""

    hidden_states: torch.Tensor
    final_state: torch.Tensor | None = None
    states_per_token: tuple[torch.Tensor, ...] | None = None


def recurrent_kda(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    attention_mask: torch.Tensor | None = None,
    *,
    accumulate_state_in_fp32: bool = True,
    return_states_per_token: bool = False,
    cu_seqlens: torch.Tensor | list[int] | None = None,
    update_state_in_place: bool = False,
) -> KDAOperatorOutput:
    """Exact KDA recurrence with decay, delta update, then read-after-write."""
    offsets = None
    if cu_seqlens is not None:
        offsets = validate_cu_seqlens(cu_seqlens, q.shape[0] if q.ndim == 4 else -1,
                                      q.shape[1] if q.ndim == 4 else -1, attention_mask)
    num_states = None if offsets is None else len(offsets) - 1
    batch, tokens, heads, key_dim, value_dim = validate_core_inputs(
        q, k, v, g, beta, initial_state, attention_mask, num_states=num_states
    )
    if return_states_per_token and offsets is not None:
        raise ValueError("return_states_per_token is not supported with cu_seqlens")
    _lib.require_gpu(q)
    work_dtype = accumulation_dtype(v.dtype, accumulate_state_in_fp32)
    from .chunkwise import differentiable, needs_grad

    if needs_grad(q, k, v, g, beta, initial_state):
        if update_state_in_place:
            raise RuntimeError("the MI355X KDA backward does not support update_state_in_place")
        if return_states_per_token:
            from .chunkwise import _mask_differentiable

            qm, gm, bm = _mask_differentiable(q, g, beta, attention_mask)
            hidden, final, hist = _RecurrentStatesFunction.apply(qm, k, v, gm, bm, initial_state, output_final_state,
                                                                 work_dtype)
            return KDAOperatorOutput(hidden_states=hidden, final_state=final if output_final_state else None,
                                     states_per_token=tuple(hist.unbind(0)))
        return differentiable(q, k, v, g, beta, initial_state, output_final_state, attention_mask, work_dtype,
                              recurrent=True, offsets=offsets)
    lib = _lib.load()

    (qc, kc, vc, gc, bc), kernel_dtype, arith = _prep.kernel_inputs(q, k, v, g, beta, work_dtype)
    device = q.device
    n_seq = batch if offsets is None else len(offsets) - 1
    total = batch * tokens

    if update_state_in_place:
        if initial_state is None:
            raise ValueError("update_state_in_place needs an initial_state")
        if initial_state.dtype != arith or not initial_state.is_contiguous():
            raise ValueError(
                f"update_state_in_place needs a contiguous {arith} initial_state, "
                f"got {initial_state.dtype} (contiguous={initial_state.is_contiguous()})"
            )
        s_in = initial_state
        s_out = initial_state
    else:
        s_in = _prep.state_arg(initial_state, arith, work_dtype)
        need_state = output_final_state or return_states_per_token
        s_out = torch.empty(n_seq, heads, key_dim, value_dim, dtype=arith, device=device) if need_state else None

    out = torch.empty(batch, tokens, heads, value_dim, dtype=kernel_dtype, device=device)
    hist = None
    if return_states_per_token:
        hist = torch.empty(tokens, n_seq, heads, key_dim, value_dim, dtype=arith, device=device)

    stream = _prep.stream(device)
    code = _lib.dtype_code(kernel_dtype)
    scode = _lib.dtype_code(arith)
    if offsets is None and tokens == 1 and hist is None and s_out is not None:
        # one decode step: the state streams through once (mask rows are all valid at T=1)
        status = lib.kda_decode_step(
            qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr(), bc.data_ptr(), code,
            _lib.ptr(s_in), s_out.data_ptr(), scode, out.data_ptr(),
            batch, heads, key_dim, value_dim, stream,
        )
    else:
        cu = None if offsets is None else _prep.cu_tensor(offsets, device)
        valid = _prep.valid_lengths(attention_mask, device)
        status = lib.kda_recurrent_fwd(
            qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr(), bc.data_ptr(), code,
            _lib.ptr(s_in), _lib.ptr(s_out), scode, out.data_ptr(), _lib.ptr(hist),
            _lib.ptr(cu), tokens, _lib.ptr(valid), n_seq, total, heads, key_dim, value_dim, stream,
        )
    _lib.check(status)

    hidden = out if out.dtype == v.dtype else out.to(v.dtype)
    final = None
    if output_final_state:
        final = s_out if s_out.dtype == work_dtype else s_out.to(work_dtype)
    states = None
    if hist is not None:
        states = tuple(x if x.dtype == work_dtype else x.to(work_dtype) for x in hist.unbind(0))
    return KDAOperatorOutput(hidden_states=hidden, final_state=final, states_per_token=states)


class _RecurrentStatesFunction(torch.autograd.Function):
    """``recurrent_kda`` with its per-token states under autograd: the recurrent
    kernel forward, and ``kda_recurrent_bwd`` (a token-by-token backward in the
    work dtype that takes a gradient for every returned state)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, output_final_state, work_dtype):
        out = recurrent_kda(q, k, v, g, beta, initial_state, output_final_state, return_states_per_token=True,
                            accumulate_state_in_fp32=work_dtype != v.dtype)
        hist = torch.stack(out.states_per_token)
        ctx.save_for_backward(q, k, v, g, beta, initial_state, hist)
        return out.hidden_states, out.final_state, hist

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, d_hidden, d_final, d_hist):
        q, k, v, g, beta, initial_state, hist = ctx.saved_tensors
        lib = _lib.load()
        batch, tokens, heads, key_dim = q.shape
        value_dim = v.shape[-1]
        device = q.device
        arith = torch.float64 if hist.dtype == torch.float64 else torch.float32
        cast = lambda t: None if t is None else t.detach().to(arith).contiguous()  # noqa: E731
        qa, ka, va, ga, ba, s0, ha, dha, dfa = (cast(t) for t in (q, k, v, g, beta, initial_state, hist, d_hist,
                                                                  d_final))
        if d_hidden is None:
            d_hidden = torch.zeros(batch, tokens, heads, value_dim, dtype=arith, device=device)
        do = cast(d_hidden)
        dq, dk, dg = (torch.empty_like(qa) for _ in range(3))
        dv, dbeta = torch.empty_like(va), torch.empty_like(ba)
        ds0 = torch.empty_like(s0) if s0 is not None and ctx.needs_input_grad[5] else None
        code = _lib.dtype_code(arith)
        ws_bytes = lib.kda_recurrent_bwd_workspace_bytes(batch, heads, key_dim, value_dim, code)
        workspace = _prep.workspace(ws_bytes, device, "the recurrent_kda backward")
        _lib.check(lib.kda_recurrent_bwd(
            qa.data_ptr(), ka.data_ptr(), va.data_ptr(), ga.data_ptr(), ba.data_ptr(), do.data_ptr(), _lib.ptr(s0),
            ha.data_ptr(), _lib.ptr(dha), _lib.ptr(dfa), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(),
            dbeta.data_ptr(), _lib.ptr(ds0), batch, tokens, heads, key_dim, value_dim, code, _lib.ptr(workspace),
            ws_bytes, _prep.stream(device),
        ))
        grads = [dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
                 None if ds0 is None else ds0.to(initial_state.dtype)]
        return (*[gr if need else None for gr, need in zip(grads, ctx.needs_input_grad[:6])], None, None)
