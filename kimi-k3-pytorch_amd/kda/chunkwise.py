"""Chunkwise-parallel KDA prefill on the gfx950 backend.

Drop-in for ``chunkwise_kda`` (src/kda/chunkwise.py:17-107): same signature,
defaults, validation errors and dtype rules.  The kernels use a fixed
64-token chunk with 16-row sub-tiles internally; the exact chunkwise
algorithm's result does not depend on ``chunk_size`` or
``secondary_tile_size`` (the reference pins that invariance in
tests/kda/test_kda_chunkwise_equivalence.py:42-57 and
tests/kda/test_kda_ut_transform.py:94-103), so both are validated exactly as
the reference does and otherwise only select nothing.

Additive keyword-only extension: ``cu_seqlens`` (packed documents
``[1, sum T, H, *]``, state reset at every document start, per-document
``initial_state``/``final_state`` of shape ``[N,H,K,V]``).

Gradients: with autograd enabled and an input that requires grad, the call
goes through ``_ChunkwiseFunction``, whose backward is the HIP chunk backward
(``kda_chunk_bwd``: f32 arithmetic for bf16/f16/f32 inputs, f64 for f64
inputs) with key_dim <= 128; the attention mask is applied with
differentiable tensor ops first (src/kda/utils.py:82-94), so padded positions
get zero gradients.  With ``create_graph=True`` the gradients are themselves
differentiable (dense inputs): the double backward is
``kda_chunk_grad_tangent``, in f64 arithmetic.  Packed
documents (``cu_seqlens``) are differentiated in buckets of similar length:
documents within a fifth of the bucket's longest are stacked into one
zero-padded dense batch (zero rows are identity steps of the recurrence), a
lone document runs on its slice of the packed tensors in place, and each
bucket's workspace stays within max(the longest document's, 1 GiB).  A
backward call, or a prefill, whose workspace would pass
``WORKSPACE_LIMIT`` (4 GiB) runs its heads in groups, on contiguous copies of
the head slices.  Value dims past 128 differentiate in column slices.  Key
dims past 128, second derivatives of packed documents and third derivatives
raise instead of dropping gradients.
"""

from __future__ import annotations

import warnings

import numpy as np
import torch

from . import _lib, _prep
from .recurrent import KDAOperatorOutput
from .utils import accumulation_dtype, validate_core_inputs, validate_cu_seqlens


def chunkwise_kda(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    attention_mask: torch.Tensor | None = None,
    *,
    chunk_size: int = 64,
    secondary_tile_size: int = 16,
    accumulate_state_in_fp32: bool = True,
    cu_seqlens: torch.Tensor | list[int] | None = None,
) -> KDAOperatorOutput:
    """Exact chunkwise KDA using UT/WY parallel computation within each chunk."""
    if chunk_size <= 0 or secondary_tile_size <= 0:
        raise ValueError("chunk_size and secondary_tile_size must be > 0")
    if secondary_tile_size > chunk_size:
        raise ValueError("secondary_tile_size must be <= chunk_size")
    offsets = None
    if cu_seqlens is not None:
        offsets = validate_cu_seqlens(cu_seqlens, q.shape[0] if q.ndim == 4 else -1,
                                      q.shape[1] if q.ndim == 4 else -1, attention_mask)
    num_states = None if offsets is None else len(offsets) - 1
    batch, tokens, heads, key_dim, value_dim = validate_core_inputs(
        q, k, v, g, beta, initial_state, attention_mask, num_states=num_states
    )
    _lib.require_gpu(q)
    work_dtype = accumulation_dtype(v.dtype, accumulate_state_in_fp32)
    if needs_grad(q, k, v, g, beta, initial_state):
        return differentiable(q, k, v, g, beta, initial_state, output_final_state, attention_mask, work_dtype,
                              recurrent=False, offsets=offsets)
    return _forward(q, k, v, g, beta, initial_state, output_final_state, attention_mask, work_dtype, offsets,
                    batch, tokens, heads, key_dim, value_dim)


# Most bytes one kernel call may take as workspace before its heads run in
# groups: the chunk backward's (and the split-bf16 prefill's) is linear in
# the heads, about 115 KB per token and head at K=V=128 for bf16/f16 inputs
# and 160 KB for f32 inputs.
WORKSPACE_LIMIT = 4 << 30


def _forward(q, k, v, g, beta, initial_state, output_final_state, attention_mask, work_dtype, offsets,
             batch, tokens, heads, key_dim, value_dim) -> KDAOperatorOutput:
    lib = _lib.load()
    (qc, kc, vc, gc, bc), kernel_dtype, arith = _prep.kernel_inputs(q, k, v, g, beta, work_dtype)
    if key_dim > 128 and kernel_dtype != torch.float64:
        # the chunk kernels hold at most 128 key channels per state: the exact
        # token recurrence runs instead (f64 inputs take it by design)
        warnings.warn(f"chunkwise_kda: key_dim {key_dim} > 128 runs the token-by-token recurrence kernel, "
                      "not the chunk-parallel path (much slower on long sequences)", RuntimeWarning, stacklevel=3)
    device = q.device
    n_seq = batch if offsets is None else len(offsets) - 1
    total = batch * tokens
    s_in = _prep.state_arg(initial_state, arith, work_dtype)
    s_out = (
        torch.empty(n_seq, heads, key_dim, value_dim, dtype=arith, device=device)
        if output_final_state
        else None
    )
    out = torch.empty(batch, tokens, heads, value_dim, dtype=kernel_dtype, device=device)
    cu = None if offsets is None else _prep.cu_tensor(offsets, device)
    valid = _prep.valid_lengths(attention_mask, device)
    code = _lib.dtype_code(kernel_dtype)
    # packed documents: the longest document's length is the schedule's hint
    longest = _prep.longest_document(offsets)

    def need(n_h):
        return lib.kda_chunk_fwd_workspace_bytes(n_seq, total, longest, n_h, key_dim, value_dim, code)

    # a prefill whose workspace passes WORKSPACE_LIMIT (f32 inputs and shapes
    # off the MFMA path take the split-bf16 chunk path, whose per-chunk records
    # are 240 KiB per head at K = V = 128; packed documents there are a
    # zero-padded batch) runs its heads in groups
    n_h = _head_group(need, heads)
    ws_bytes = need(n_h)
    workspace = _prep.workspace(ws_bytes, device, "chunkwise_kda")

    def call(ins, s_i, s_o, o, n):
        status = lib.kda_chunk_fwd(
            *(t.data_ptr() for t in ins), code,
            _lib.ptr(s_i), _lib.ptr(s_o), _lib.dtype_code(arith), o.data_ptr(),
            _lib.ptr(cu), tokens if offsets is None else longest, _lib.ptr(valid), n_seq, total, n, key_dim,
            value_dim,
            _lib.ptr(workspace), ws_bytes, _prep.stream(device),
        )
        _lib.check(status)

    if n_h == heads:
        call((qc, kc, vc, gc, bc), s_in, s_out, out, heads)
    else:
        for h0 in range(0, heads, n_h):
            n = min(n_h, heads - h0)
            o = torch.empty(batch, tokens, n, value_dim, dtype=kernel_dtype, device=device)
            s_o = None if s_out is None else torch.empty(n_seq, n, key_dim, value_dim, dtype=arith, device=device)
            call([t.narrow(2, h0, n).contiguous() for t in (qc, kc, vc, gc, bc)],
                 None if s_in is None else s_in.narrow(1, h0, n).contiguous(), s_o, o, n)
            out.narrow(2, h0, n).copy_(o)
            if s_out is not None:
                s_out.narrow(1, h0, n).copy_(s_o)
    hidden = out if out.dtype == v.dtype else out.to(v.dtype)
    final = None
    if s_out is not None:
        final = s_out if s_out.dtype == work_dtype else s_out.to(work_dtype)
    return KDAOperatorOutput(hidden_states=hidden, final_state=final)


def needs_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors)


def differentiable(q, k, v, g, beta, initial_state, output_final_state, attention_mask, work_dtype, *,
                   recurrent: bool, offsets: list[int] | None = None) -> KDAOperatorOutput:
    """The operator under autograd: masked inputs, the forward of
    ``recurrent_kda`` (recurrent=True) or ``chunkwise_kda``, and the HIP chunk
    backward, whose gradients are those of the exact recurrence either way.
    ``offsets`` are validated packed-document boundaries (or None)."""
    if q.shape[-1] > 128:
        raise RuntimeError("the MI355X KDA backward supports key_dim up to 128")
    qm, gm, bm = _mask_differentiable(q, g, beta, attention_mask)
    hidden, final = _ChunkwiseFunction.apply(qm, k, v, gm, bm, initial_state, output_final_state, work_dtype,
                                             recurrent, offsets)
    return KDAOperatorOutput(hidden_states=hidden, final_state=final)


def _mask_differentiable(q, g, beta, attention_mask):
    """Zero q, g and beta at padded positions with tensor ops that autograd
    differentiates (src/kda/utils.py:82-94)."""
    if attention_mask is None:
        return q, g, beta
    keep = attention_mask.to(device=q.device, dtype=torch.bool)
    return (torch.where(keep[:, :, None, None], q, torch.zeros((), dtype=q.dtype, device=q.device)),
            torch.where(keep[:, :, None, None], g, torch.zeros((), dtype=g.dtype, device=g.device)),
            torch.where(keep[:, :, None], beta, torch.zeros((), dtype=beta.dtype, device=beta.device)))


def _document_buckets(lengths: list[int], fits) -> list[list[int]]:
    """Documents (indices) grouped for the backward: sorted by length, each
    bucket takes the longest remaining document and every next one at least
    0.8 of its length (at most a fifth of the bucket's rows are padding), as
    long as fits(count, longest) holds for the workspace."""
    order = sorted(range(len(lengths)), key=lambda i: -lengths[i])
    buckets: list[list[int]] = []
    for i in order:
        if buckets:
            head = lengths[buckets[-1][0]]
            if 5 * lengths[i] >= 4 * head and fits(len(buckets[-1]) + 1, head):
                buckets[-1].append(i)
                continue
        buckets.append([i])
    return buckets


def _head_group(need, heads) -> int:
    """Heads per kernel call: all of them when the call's workspace,
    need(heads) bytes, fits WORKSPACE_LIMIT, else the most that fit (at least
    one)."""
    # the size grows with the heads: the largest count that fits, by bisection
    lo, hi = 1, heads
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if need(mid) <= WORKSPACE_LIMIT:
            lo = mid
        else:
            hi = mid - 1
    return lo


class _Workspace:
    """One workspace for the calls of a backward, grown to the largest
    request (the torch caching allocator keeps the bytes for reuse)."""

    def __init__(self, device):
        self.device, self.tensor, self.nbytes = device, None, 0

    def get(self, nbytes):
        if nbytes > self.nbytes:
            self.tensor = None
            self.tensor = _prep.workspace(nbytes, self.device, "the chunkwise_kda backward")
            self.nbytes = nbytes
        return self.tensor


def _by_head_groups(lib, call, tensors, grads_out, s_init, ds_fin, ds_init, n_b, n_tok, heads, key_dim,
                    value_dim, workspace, code):
    """One chunk-backward over [n_b, n_tok, heads, *] tensors, split into
    head groups when the whole call's workspace would pass WORKSPACE_LIMIT.
    Heads are independent in KDA (every state, decay and gradient is per
    head), so a group is the same computation on contiguous copies of its
    head slices, its gradients copied back."""
    def need(n):
        return lib.kda_chunk_bwd_workspace_bytes(n_b, n_tok, n, key_dim, value_dim, code)

    n_h = _head_group(need, heads)
    ws_bytes = need(n_h)
    ws = workspace.get(ws_bytes)
    if n_h == heads:
        call(tensors, grads_out, s_init, ds_fin, ds_init, n_b, n_tok, heads, ws, ws_bytes)
        return

    def part(t, h0, h1, axis):
        return None if t is None else t.narrow(axis, h0, h1 - h0).contiguous()

    for h0 in range(0, heads, n_h):
        h1 = min(heads, h0 + n_h)
        ins = [part(t, h0, h1, 2) for t in tensors]
        outs = [torch.empty_like(t) for t in ins[:5]]
        ds_g = None if ds_init is None else ds_init.new_empty((n_b, h1 - h0) + tuple(ds_init.shape[2:]))
        call(ins, outs, part(s_init, h0, h1, 1), part(ds_fin, h0, h1, 1), ds_g, n_b, n_tok, h1 - h0, ws,
             ws_bytes)
        for dst, src in zip(grads_out, outs):
            dst.narrow(2, h0, h1 - h0).copy_(src)
        if ds_init is not None:
            ds_init.narrow(1, h0, h1 - h0).copy_(ds_g)


def _packed_backward(lib, offsets, inputs, grads, s0, ds_t, ds0, heads, key_dim, value_dim, device, run, code):
    """The chunk backward of packed documents in few calls: documents of
    similar length are stacked into one zero-padded dense batch [n, T_b, H, *]
    per bucket.  A zero row (q = k = v = g = beta = 0, dO = 0) neither decays,
    writes nor reads the state, which is how the kernels treat the rows past a
    sequence's end, so every document's gradients are those of its own call.
    A bucket of one document runs on the packed tensors in place."""
    lengths = [b - a for a, b in zip(offsets[:-1], offsets[1:])]
    longest = max(lengths)
    # the workspace a call per document needs anyway (sized for the longest),
    # or 1 GiB, bounds each bucket's, within WORKSPACE_LIMIT (past it a
    # bucket's heads go in groups)
    budget = min(max(lib.kda_chunk_bwd_workspace_bytes(1, longest, heads, key_dim, value_dim, code), 1 << 30),
                 WORKSPACE_LIMIT)

    def fits(n, n_tok):
        return lib.kda_chunk_bwd_workspace_bytes(n, n_tok, heads, key_dim, value_dim, code) <= budget

    buckets = _document_buckets(lengths, fits)
    for bk in buckets:
        if len(bk) == 1:
            i = bk[0]
            a = offsets[i]
            views = [t[:, a:a + lengths[i]] for t in inputs]
            gviews = [t[:, a:a + lengths[i]] for t in grads]
            if all(t.is_contiguous() for t in views + gviews):
                run(views, gviews, None if s0 is None else s0[i:i + 1], None if ds_t is None else ds_t[i:i + 1],
                    None if ds0 is None else ds0[i:i + 1], 1, lengths[i])
                continue
        n_tok = lengths[bk[0]]
        # packed row of each real row of the bucket, and its row in the padded batch
        lens_b = np.array([lengths[i] for i in bk], dtype=np.int64)
        starts_b = np.array([offsets[i] for i in bk], dtype=np.int64)
        doc = np.repeat(np.arange(len(bk)), lens_b)
        pos = np.arange(int(lens_b.sum())) - np.repeat(np.cumsum(lens_b) - lens_b, lens_b)
        src_rows = torch.from_numpy(starts_b[doc] + pos).to(device)
        dst_rows = torch.from_numpy(doc * n_tok + pos).to(device)
        padded = []
        for t in inputs:
            flat = t.new_zeros((len(bk) * n_tok,) + tuple(t.shape[2:]))
            flat[dst_rows] = t[0].index_select(0, src_rows)
            padded.append(flat.view((len(bk), n_tok) + tuple(t.shape[2:])))
        pgrads = [torch.empty_like(p) for p in padded[:5]]
        idx = torch.tensor(bk, device=device)
        s_b = None if s0 is None else s0.index_select(0, idx).contiguous()
        dst_b = None if ds_t is None else ds_t.index_select(0, idx).contiguous()
        ds0_b = None if ds0 is None else torch.empty_like(s_b)
        run(padded, pgrads, s_b, dst_b, ds0_b, len(bk), n_tok)
        for dst, src in zip(grads, pgrads):
            dst[0].index_copy_(0, src_rows, src.view((-1,) + tuple(src.shape[2:])).index_select(0, dst_rows))
        if ds0 is not None:
            ds0.index_copy_(0, idx, ds0_b)


class _ChunkwiseFunction(torch.autograd.Function):
    """The operator on masked, dense inputs with the HIP chunk backward."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, output_final_state, work_dtype, recurrent, offsets):
        batch, tokens, heads, key_dim = q.shape
        value_dim = v.shape[-1]
        if recurrent:
            from .recurrent import recurrent_kda

            out = recurrent_kda(q, k, v, g, beta, initial_state, output_final_state,
                                accumulate_state_in_fp32=work_dtype != v.dtype, cu_seqlens=offsets)
        else:
            out = _forward(q, k, v, g, beta, initial_state, output_final_state, None, work_dtype, offsets,
                           batch, tokens, heads, key_dim, value_dim)
        ctx.save_for_backward(q, k, v, g, beta, initial_state)
        ctx.work_dtype = work_dtype
        ctx.offsets = offsets
        if out.final_state is None:
            return out.hidden_states, None
        return out.hidden_states, out.final_state

    @staticmethod
    def backward(ctx, d_hidden, d_final):
        q, k, v, g, beta, initial_state = ctx.saved_tensors
        needs = ctx.needs_input_grad[:6]
        if torch.is_grad_enabled():
            # create_graph: the gradients themselves are differentiable (second
            # derivatives through kda_chunk_grad_tangent)
            if ctx.offsets is not None:
                raise RuntimeError("second derivatives of the MI355X KDA operator need dense inputs (no cu_seqlens)")
            if d_hidden is None:
                d_hidden = torch.zeros(v.shape[:3] + v.shape[3:], dtype=v.dtype, device=v.device)
            grads = _ChunkwiseGrad.apply(q, k, v, g, beta, initial_state, d_hidden, d_final, ctx.work_dtype, needs)
        else:
            grads = _chunk_gradients(q, k, v, g, beta, initial_state, d_hidden, d_final, ctx.work_dtype,
                                     ctx.offsets, needs)
        return (*[gr if need else None for gr, need in zip(grads, needs)], None, None, None, None)


class _ChunkwiseGrad(torch.autograd.Function):
    """The chunk backward as a differentiable function of the operator's
    inputs and of its output and final-state cotangents (second derivatives,
    dense inputs).  Forward: the HIP backward (``_chunk_gradients``).
    Backward: ``kda_chunk_grad_tangent``, the f64 backward kernel run on
    value-and-derivative pairs along the incoming cotangents of the
    gradients.  Second derivatives are symmetric, so that directional
    derivative is the cotangent of the inputs, and the directional
    derivatives of the output and of the final state are the cotangents of
    their own cotangents: the double backward, in f64 arithmetic for every
    input dtype.  (A third derivative raises.)"""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, d_hidden, d_final, work_dtype, needs):
        grads = _chunk_gradients(q, k, v, g, beta, initial_state, d_hidden, d_final, work_dtype, None, needs)
        ctx.save_for_backward(q, k, v, g, beta, initial_state, d_hidden, d_final)
        ctx.work_dtype = work_dtype
        return tuple(grads)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, wq, wk, wv, wg, wb, ws0):
        q, k, v, g, beta, s0, d_hidden, d_final = ctx.saved_tensors
        lib = _lib.load()
        f64 = torch.float64
        device = q.device
        batch, tokens, heads, key_dim = q.shape
        value_dim = v.shape[-1]
        # the values the forward and the first backward computed on (rounded
        # to the work dtype as they were), in f64
        ins, _, _ = _prep.kernel_inputs(q, k, v, g, beta, ctx.work_dtype)
        x = [t.to(f64).contiguous() for t in ins]
        s0d = _prep.state_arg(None if s0 is None else s0.detach(), f64, ctx.work_dtype)
        d_out = d_hidden.to(f64).contiguous()
        ds_t = None if d_final is None else d_final.to(f64).contiguous()
        tan = [None if w is None else w.to(f64).contiguous() for w in (wq, wk, wv, wg, wb)]
        t_s0 = None if ws0 is None or s0 is None else ws0.to(f64).contiguous()
        need = ctx.needs_input_grad
        outs = [torch.empty_like(t) if need[i] else None for i, t in enumerate(x)]
        g_s0 = torch.empty_like(s0d) if s0 is not None and need[5] else None
        t_out = torch.empty(batch, tokens, heads, value_dim, dtype=f64, device=device) if need[6] else None
        t_fin = (torch.empty(batch, heads, key_dim, value_dim, dtype=f64, device=device)
                 if d_final is not None and need[7] else None)
        ws_bytes = lib.kda_chunk_grad_tangent_workspace_bytes(batch, tokens, heads, key_dim, value_dim)
        ws = _prep.workspace(ws_bytes, device, "the chunkwise_kda second derivative")
        _lib.check(lib.kda_chunk_grad_tangent(
            *(t.data_ptr() for t in x), _lib.ptr(s0d), d_out.data_ptr(), _lib.ptr(ds_t),
            *(_lib.ptr(t) for t in tan), _lib.ptr(t_s0), *(_lib.ptr(o) for o in outs), _lib.ptr(g_s0),
            _lib.ptr(t_out), _lib.ptr(t_fin), batch, tokens, heads, key_dim, value_dim, _lib.ptr(ws), ws_bytes,
            _prep.stream(device),
        ))
        grads = [None if o is None else o.to(t.dtype) for o, t in zip(outs, (q, k, v, g, beta))]
        return (*grads, None if g_s0 is None else g_s0.to(s0.dtype),
                None if t_out is None else t_out.to(d_hidden.dtype),
                None if t_fin is None else t_fin.to(d_final.dtype), None, None)


def _chunk_gradients(q, k, v, g, beta, initial_state, d_hidden, d_final, work_dtype, offsets, needs):
    """The HIP chunk backward: gradients of the output and final state's
    loss with respect to q, k, v, g, beta and the initial state."""
    lib = _lib.load()
    (qc, kc, vc, gc, bc), kernel_dtype, _ = _prep.kernel_inputs(q, k, v, g, beta, work_dtype)
    batch, tokens, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    device = q.device
    if d_hidden is None:
        d_hidden = torch.zeros(batch, tokens, heads, value_dim, dtype=kernel_dtype, device=device)
    d_out = d_hidden.to(kernel_dtype).contiguous()
    state_dtype = torch.float64 if kernel_dtype == torch.float64 else torch.float32
    s0 = _prep.state_arg(None if initial_state is None else initial_state.detach(), state_dtype, work_dtype)
    ds_t = None if d_final is None else d_final.to(state_dtype).contiguous()
    dq, dk, dv, dg = (torch.empty_like(t) for t in (qc, kc, vc, gc))
    dbeta = torch.empty_like(bc)
    n_state = batch if offsets is None else len(offsets) - 1
    ds0 = None
    if initial_state is not None and needs[5]:
        ds0 = torch.empty(n_state, heads, key_dim, value_dim, dtype=state_dtype, device=device)
    code = _lib.dtype_code(kernel_dtype)
    stream = _prep.stream(device)

    def call(tensors, grads_out, s_init, ds_fin, ds_init, n_b, n_tok, n_h, ws, ws_bytes, vdim):
        status = lib.kda_chunk_bwd(
            *(t.data_ptr() for t in tensors), code, _lib.ptr(s_init), _lib.ptr(ds_fin),
            *(t.data_ptr() for t in grads_out), _lib.ptr(ds_init), n_b, n_tok, n_h, key_dim, vdim,
            _lib.ptr(ws), ws_bytes, stream,
        )
        _lib.check(status)

    workspace = _Workspace(device)

    def backward_of(vc, d_out, s0, ds_t, grads, ds0):
        """The kernels' backward over one value slice (at most 128 columns)."""
        vdim = vc.shape[-1]

        def run(tensors, grads_out, s_init, ds_fin, ds_init, n_b, n_tok):
            _by_head_groups(lib, lambda *a: call(*a, vdim), tensors, grads_out, s_init, ds_fin, ds_init, n_b,
                            n_tok, heads, key_dim, vdim, workspace, code)

        if offsets is None:
            run((qc, kc, vc, gc, bc, d_out), grads, s0, ds_t, ds0, batch, tokens)
        else:
            _packed_backward(lib, offsets, (qc, kc, vc, gc, bc, d_out), grads, s0, ds_t, ds0, heads,
                             key_dim, vdim, device, run, code)

    if value_dim <= 128:
        backward_of(vc, d_out, s0, ds_t, (dq, dk, dv, dg, dbeta), ds0)
    else:
        # value columns never interact: the operator over V columns is the
        # operators over column slices sharing q, k, g and beta, whose
        # gradients add up over the slices; v and the state get theirs per slice
        acc = [torch.zeros(t.shape, dtype=torch.float64 if kernel_dtype == torch.float64 else torch.float32,
                           device=device) for t in (dq, dk, dg, dbeta)]
        for c0 in range(0, value_dim, 128):
            c1 = min(c0 + 128, value_dim)
            part = (lambda t: None if t is None else t[..., c0:c1].contiguous())  # noqa: E731
            g_s = [torch.empty_like(t) for t in (dq, dk)] + [torch.empty_like(part(vc))] + \
                [torch.empty_like(t) for t in (dg, dbeta)]
            ds0_s = None if ds0 is None else torch.empty_like(part(ds0))
            backward_of(part(vc), part(d_out), part(s0), part(ds_t), g_s, ds0_s)
            for a, gs in zip(acc, (g_s[0], g_s[1], g_s[3], g_s[4])):
                a += gs
            dv[..., c0:c1] = g_s[2]
            if ds0 is not None:
                ds0[..., c0:c1] = ds0_s
        for dst, a in zip((dq, dk, dg, dbeta), acc):
            dst.copy_(a)
    grads = [dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
             None if ds0 is None else ds0.to(initial_state.dtype)]
    return grads

