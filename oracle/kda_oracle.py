"""CPU oracle for the Kimi Delta Attention (KDA) operator path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the reference the GPU results are
compared with, or as the timed CPU baseline.

This is a PyTorch-on-CPU restatement of the reference operator
(pablo-reyes8/kimi-k3-pytorch, ``src/kda``).  It keeps the reference's
algorithmic steps so that it doubles as "the reference's own CPU path" for the
CPU baseline, but the code is written independently:

* ``recurrent``            follows ``src/kda/recurrent.py:38-80``
* ``tiled_causal_decay_dot`` follows ``src/kda/utils.py:97-143``
* ``ut_transform_internal`` follows ``src/kda/ut_transform.py:23-58``
* ``chunkwise``            follows ``src/kda/chunkwise.py:34-107``
* ``work_dtype``           follows ``src/kda/utils.py:74-79``
* ``mask_inputs``          follows ``src/kda/utils.py:82-94``
* ``chunkwise_backward``   differentiates ``chunkwise`` (the reference gets
  these gradients from autograd through src/kda/chunkwise.py:34-107)
* ``varlen_chunkwise`` / ``varlen_recurrent`` have no reference counterpart
  (the reference has no ``cu_seqlens``); they are defined as independent runs
  of the functions above on each document, which is the semantics the GPU
  path implements.
* ``short_conv``           follows ``src/kimi_primitives/short_conv.py:69-98``
* ``conv_silu``            follows ``src/kda/projections.py:100-140,164-206``
* ``lower_bounded_decay``  follows ``src/kda/decay.py:30-43`` (+ projections.py:211-218)
* ``beta_gate``            follows ``src/kda/projections.py:207-209``
* ``rmsnorm_gate``         follows ``src/kimi_primitives/headwise_rmsnorm.py:39-64``
  and the gate product of ``src/kimi_primitives/output_gate.py:62-75``
* ``kda_layer``            follows ``KimiDeltaAttention.forward`` (``src/kda/kda.py:98-183``)
  over ``src/kda/projections.py:144-225``: the stages above composed with
  the operator, in the reference's dtype flow (each stage's result in the
  activation dtype)
* ``gather_rows``          follows ``KDAState.reorder`` / ``clone``
  (``src/kda/state.py:41-67``) taken over every layer by
  ``src/hybrid_backbone/cache.py:56-61,112-126``

How each function is pinned (tests/test_oracle_*.py):

* ``recurrent``: the reference's literal known-answer tests
  (tests/kda/test_kda_recurrent.py:70-139), the matrix/error-correction
  identity (:48-67), an independent scalar C implementation
  (``oracle/kda_recurrent_ref.c``) and the beta=0 closed form.
* ``tiled_causal_decay_dot``: brute-force pairwise sums on tiny inputs and
  tile-size invariance.
* ``ut_transform_internal``: an explicit inverse (``torch.linalg.inv``) and a
  row-by-row forward substitution.
* ``chunkwise``: equality with ``recurrent`` in float64 at 2e-11 over the
  reference's shape/chunk grid, prefix causality and mask==truncation.
* varlen: per-document equality (by construction) plus state reset checks.
* ``chunkwise_backward``: torch.autograd through ``chunkwise`` and through
  ``recurrent`` in f64 (the reference's own gradient tests,
  tests/kda/test_kda_chunkwise_equivalence.py:92-134), gradcheck of
  ``chunkwise``, chunk-size invariance, and extreme decays.
* ``short_conv``: ``torch.nn.functional.conv1d`` on the history-padded input,
  streaming (two calls chained through the history equal one call).
* ``conv_silu``: masked rows equal the truncated run, unit head norms.
* ``lower_bounded_decay`` / ``beta_gate``: the sigmoid midpoint, the clamp
  bounds, monotonicity.
* ``rmsnorm_gate``: unit mean square, scale invariance, the gate midpoint.
* ``gather_rows``: the reference's reorder test (indices [2, 0, 2] pick those
  batch rows of every layer, tests/hybrid_backbone/test_hybrid_cache.py:82-101),
  a permutation followed by its inverse is the identity, and a clone is a
  byte-equal copy that shares no memory.

Rounding: the reference's bit-level float32/bfloat16 rounding order (einsum /
BLAS / LAPACK) is not reproduced; parity is judged with tolerances.
"""

from __future__ import annotations

import torch

__all__ = [
    "work_dtype",
    "mask_inputs",
    "recurrent",
    "tiled_causal_decay_dot",
    "ut_transform_internal",
    "chunkwise",
    "varlen_recurrent",
    "varlen_chunkwise",
    "chunkwise_backward",
    "short_conv",
    "conv_silu",
    "gather_rows",
    "lower_bounded_decay",
    "beta_gate",
    "rmsnorm_gate",
]


def work_dtype(activation_dtype: torch.dtype, accumulate_state_in_fp32: bool = True) -> torch.dtype:
    """Arithmetic dtype of the operator (src/kda/utils.py:74-79)."""
    if accumulate_state_in_fp32 and activation_dtype in (torch.float16, torch.bfloat16):
        return torch.float32
    return activation_dtype


def mask_inputs(q, g, beta, attention_mask):
    """Zero q, g and beta at padded positions (src/kda/utils.py:82-94).

    A padded token then neither decays, writes nor reads the state."""
    if attention_mask is None:
        return q, g, beta
    keep = attention_mask.to(torch.bool)
    q = torch.where(keep[:, :, None, None], q, torch.zeros((), dtype=q.dtype))
    g = torch.where(keep[:, :, None, None], g, torch.zeros((), dtype=g.dtype))
    beta = torch.where(keep[:, :, None], beta, torch.zeros((), dtype=beta.dtype))
    return q, g, beta


def _prepare(q, k, v, g, beta, initial_state, attention_mask, accumulate_state_in_fp32):
    dtype = work_dtype(v.dtype, accumulate_state_in_fp32)
    qw, kw, vw, gw, bw = (t.to(dtype) for t in (q, k, v, g, beta))
    qw, gw, bw = mask_inputs(qw, gw, bw, attention_mask)
    batch, _, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    state = torch.zeros(batch, heads, key_dim, value_dim, dtype=dtype)
    if initial_state is not None:
        state = state + initial_state.to(dtype)
    return dtype, qw, kw, vw, gw, bw, state


def recurrent(
    q, k, v, g, beta, initial_state=None, attention_mask=None, *,
    accumulate_state_in_fp32: bool = True, return_states: bool = False,
):
    """Token-by-token KDA (src/kda/recurrent.py:38-80).

    Per token t (recurrent.py:66-72):
      S <- diag(exp g_t) S ;  e = v_t - S^T k_t ;  S <- S + beta_t k_t e^T ;  o_t = S^T q_t
    Returns (output in v.dtype, final state in the work dtype, [states]).
    """
    dtype, qw, kw, vw, gw, bw, state = _prepare(
        q, k, v, g, beta, initial_state, attention_mask, accumulate_state_in_fp32)
    tokens = q.shape[1]
    outputs = []
    history = []
    for t in range(tokens):
        state = state * gw[:, t].exp().unsqueeze(-1)
        recalled = (state * kw[:, t].unsqueeze(-1)).sum(dim=-2)
        error = vw[:, t] - recalled
        write = (bw[:, t].unsqueeze(-1) * kw[:, t]).unsqueeze(-1) * error.unsqueeze(-2)
        state = state + write
        outputs.append((state * qw[:, t].unsqueeze(-1)).sum(dim=-2))
        if return_states:
            history.append(state)
    out = torch.stack(outputs, dim=1).to(v.dtype)
    return out, state, (tuple(history) if return_states else None)


def tiled_causal_decay_dot(left, right, log_left, log_right, tile: int, *, include_diagonal: bool):
    """out[b,h,i,j] = sum_c left[i,c] exp(log_left[i,c] - log_right[j,c]) right[j,c]
    for j <= i (or j < i), computed tile by tile with an explicit pairwise
    exponent (src/kda/utils.py:97-143).  Inputs are ``[B,H,C,K]``."""
    if tile <= 0:
        raise ValueError("tile_size must be > 0")
    batch, heads, count, _ = left.shape
    out = torch.zeros(batch, heads, count, count, dtype=left.dtype)
    rows = torch.arange(count)
    for r0 in range(0, count, tile):
        r1 = min(r0 + tile, count)
        for c0 in range(0, r1, tile):
            c1 = min(c0 + tile, count)
            pair_log = log_left[:, :, r0:r1, None, :] - log_right[:, :, None, c0:c1, :]
            weighted = left[:, :, r0:r1, None, :] * pair_log.exp()
            block = (weighted * right[:, :, None, c0:c1, :]).sum(dim=-1)
            ri = rows[r0:r1, None]
            ci = rows[None, c0:c1]
            keep = (ri >= ci) if include_diagonal else (ri > ci)
            out[:, :, r0:r1, c0:c1] = block * keep.to(block.dtype)
    return out


def ut_transform_internal(k, v, g, beta, tile: int):
    """UT/WY transform of one chunk, internal ``[B,H,C,*]`` layout
    (src/kda/ut_transform.py:23-58).

    log_gamma = cumsum(g);  A = strict-lower decayed k k^T;  L = I + diag(beta) A;
    M = L^{-1} diag(beta);  W = M (exp(log_gamma) * k);  U = M v.
    """
    count = k.shape[2]
    log_gamma = g.cumsum(dim=2)
    strict = tiled_causal_decay_dot(k, k, log_gamma, log_gamma, tile, include_diagonal=False)
    lower = torch.eye(count, dtype=k.dtype) + beta.unsqueeze(-1) * strict
    rhs = torch.diag_embed(beta)
    M = torch.linalg.solve_triangular(lower, rhs, upper=False, unitriangular=True)
    k_gamma = log_gamma.exp() * k
    return {
        "M": M,
        "W": M @ k_gamma,
        "U": M @ v,
        "log_gamma": log_gamma,
        "k_gamma": k_gamma,
    }


def chunkwise(
    q, k, v, g, beta, initial_state=None, attention_mask=None, *,
    chunk_size: int = 64, secondary_tile_size: int = 16, accumulate_state_in_fp32: bool = True,
):
    """Chunkwise KDA with the UT transform inside each chunk
    (src/kda/chunkwise.py:34-107).  Returns (output, final state)."""
    dtype, qw, kw, vw, gw, bw, state = _prepare(
        q, k, v, g, beta, initial_state, attention_mask, accumulate_state_in_fp32)
    tokens = q.shape[1]
    pieces = []
    for start in range(0, tokens, chunk_size):
        stop = min(start + chunk_size, tokens)
        qc, kc, vc, gc = (x[:, start:stop].transpose(1, 2) for x in (qw, kw, vw, gw))
        bc = bw[:, start:stop].transpose(1, 2)
        ut = ut_transform_internal(kc, vc, gc, bc, secondary_tile_size)
        lg = ut["log_gamma"]
        pseudo = ut["U"] - ut["W"] @ state                                   # chunkwise.py:76
        causal_qk = tiled_causal_decay_dot(qc, kc, lg, lg, secondary_tile_size,
                                           include_diagonal=True)         # chunkwise.py:77-84
        out_c = (lg.exp() * qc) @ state + causal_qk @ pseudo                # chunkwise.py:85-88
        pieces.append(out_c.transpose(1, 2))
        last = lg[:, :, -1]                                                  # chunkwise.py:91
        to_end = (last.unsqueeze(2) - lg).exp() * kc                         # chunkwise.py:93-99
        state = state * last.exp().unsqueeze(-1) + to_end.transpose(-2, -1) @ pseudo  # :92,100-102
    out = torch.cat(pieces, dim=1).to(v.dtype)
    return out, state


def _split_docs(cu_seqlens):
    bounds = [int(x) for x in torch.as_tensor(cu_seqlens).tolist()]
    return list(zip(bounds[:-1], bounds[1:]))


def varlen_recurrent(q, k, v, g, beta, cu_seqlens, initial_states=None, *,
                     accumulate_state_in_fp32: bool = True):
    """Packed documents ``[1, sum T, H, *]``: each document is an independent
    ``recurrent`` run starting from its own initial state (or zero)."""
    outs, finals = [], []
    for index, (s0, s1) in enumerate(_split_docs(cu_seqlens)):
        init = None if initial_states is None else initial_states[index:index + 1]
        o, s, _ = recurrent(q[:, s0:s1], k[:, s0:s1], v[:, s0:s1], g[:, s0:s1], beta[:, s0:s1],
                            init, accumulate_state_in_fp32=accumulate_state_in_fp32)
        outs.append(o)
        finals.append(s)
    return torch.cat(outs, dim=1), torch.cat(finals, dim=0)


def varlen_chunkwise(q, k, v, g, beta, cu_seqlens, initial_states=None, *,
                     chunk_size: int = 64, secondary_tile_size: int = 16,
                     accumulate_state_in_fp32: bool = True):
    """Packed documents: each document is an independent ``chunkwise`` run."""
    outs, finals = [], []
    for index, (s0, s1) in enumerate(_split_docs(cu_seqlens)):
        init = None if initial_states is None else initial_states[index:index + 1]
        o, s = chunkwise(q[:, s0:s1], k[:, s0:s1], v[:, s0:s1], g[:, s0:s1], beta[:, s0:s1],
                         init, chunk_size=chunk_size, secondary_tile_size=secondary_tile_size,
                         accumulate_state_in_fp32=accumulate_state_in_fp32)
        outs.append(o)
        finals.append(s)
    return torch.cat(outs, dim=1), torch.cat(finals, dim=0)



# ---- backward of the chunkwise operator ---------------------------------------

def _pair_exp(lg):
    """exp(lg_i - lg_j) for the position pairs j <= i of a chunk, zero above
    the diagonal (where the exponent is positive and may overflow): [B,H,C,C,K]."""
    n = lg.shape[2]
    upper = torch.ones(n, n, dtype=torch.bool).triu(1)
    diff = (lg.unsqueeze(3) - lg.unsqueeze(2)).masked_fill(upper[:, :, None], float("-inf"))
    return diff.exp()


def chunkwise_backward(q, k, v, g, beta, initial_state, d_out, d_final_state=None, *, chunk_size: int = 64):
    """Gradients of ``chunkwise`` (src/kda/chunkwise.py:34-107, with the UT
    transform of src/kda/ut_transform.py:23-58) written out chunk by chunk.

    Inputs are the (already masked) operator inputs; ``d_out [B,T,H,V]`` and
    ``d_final_state [B,H,K,V]`` (None: zero) are the upstream gradients.
    Computes in f64 for f64 inputs and f32 otherwise and returns
    ``(dq, dk, dv, dg, dbeta, d_initial_state)`` in that dtype.

    Per chunk, with lg = cumsum(g), E_ij = exp(lg_i - lg_j), A = strict-lower
    sum_k k_i k_j E_ij, Aqk = lower sum_k q_i k_j E_ij, N = (I + diag(b) A)^-1,
    M = N diag(b), Kg = e^lg k, Qg = e^lg q, D = e^lg_last,
    Kt = e^(lg_last - lg) k, W = M Kg, U = M v, Vt = U - W S:
      forward   O = Qg S + Aqk Vt,   S' = D S + Kt^T Vt
      backward  dVt = Kt dS' + Aqk^T dO
                dS  = D dS' + Qg^T dO - W^T dVt
                dQg = dO S^T, dAqk = tril(dO Vt^T), dKt = Vt dS'^T,
                dD = rowsum(dS' * S), dW = -dVt S^T, dv = M^T dVt,
                dM = dVt v^T + dW Kg^T, dKg = M^T dW,
                db_j = sum_i N_ij dM_ij,  dL = -strict(N^T (dM diag b) N^T),
                dA = diag(b) dL,  db_i += sum_j dL_ij A_ij,
      then the pair sums of dA and dAqk, the exp factors, and
      dg = reverse cumulative sum of d lg within the chunk.
    """
    cd = torch.float64 if q.dtype == torch.float64 else torch.float32
    qw, kw, vw, gw, dO = (t.to(cd).transpose(1, 2) for t in (q, k, v, g, d_out))  # [B,H,T,*]
    bw = beta.to(cd).transpose(1, 2)  # [B,H,T]
    batch, heads, tokens, key_dim = qw.shape
    value_dim = vw.shape[-1]
    state = torch.zeros(batch, heads, key_dim, value_dim, dtype=cd)
    if initial_state is not None:
        state = state + initial_state.to(cd)
    spans = [(s0, min(s0 + chunk_size, tokens)) for s0 in range(0, tokens, chunk_size)]

    def chunk_terms(s0, s1):
        qc, kc, vc, gc, bc = qw[:, :, s0:s1], kw[:, :, s0:s1], vw[:, :, s0:s1], gw[:, :, s0:s1], bw[:, :, s0:s1]
        n = s1 - s0
        lg = gc.cumsum(dim=2)
        E = _pair_exp(lg)
        strict = torch.ones(n, n, dtype=torch.bool).tril(-1)
        lower = torch.ones(n, n, dtype=torch.bool).tril()
        A = ((kc.unsqueeze(3) * kc.unsqueeze(2)) * E).sum(-1) * strict
        Aqk = ((qc.unsqueeze(3) * kc.unsqueeze(2)) * E).sum(-1) * lower
        L = torch.eye(n, dtype=cd) + bc.unsqueeze(-1) * A
        N = torch.linalg.solve_triangular(L, torch.eye(n, dtype=cd).expand_as(L), upper=False, unitriangular=True)
        M = N * bc.unsqueeze(-2)
        last = lg[:, :, -1]
        t = dict(q=qc, k=kc, v=vc, b=bc, lg=lg, E=E, A=A, Aqk=Aqk, N=N, M=M, strict=strict, lower=lower,
                 Kg=lg.exp() * kc, Qg=lg.exp() * qc, D=last.exp(), Kt=(last.unsqueeze(2) - lg).exp() * kc)
        t["W"] = M @ t["Kg"]
        t["U"] = M @ vc
        return t

    starts = []
    for s0, s1 in spans:  # forward: the state at each chunk start
        c = chunk_terms(s0, s1)
        starts.append(state)
        vt = c["U"] - c["W"] @ state
        state = c["D"].unsqueeze(-1) * state + c["Kt"].transpose(-2, -1) @ vt

    dq, dk, dv, dg = (torch.zeros_like(x) for x in (qw, kw, vw, gw))
    dbeta = torch.zeros_like(bw)
    dS = torch.zeros(batch, heads, key_dim, value_dim, dtype=cd)
    if d_final_state is not None:
        dS = dS + d_final_state.to(cd)
    for (s0, s1), S in zip(reversed(spans), reversed(starts)):
        c = chunk_terms(s0, s1)
        dOc = dO[:, :, s0:s1]
        vt = c["U"] - c["W"] @ S
        dvt = c["Kt"] @ dS + c["Aqk"].transpose(-2, -1) @ dOc
        dQg = dOc @ S.transpose(-2, -1)
        dAqk = (dOc @ vt.transpose(-2, -1)) * c["lower"]
        dKt = vt @ dS.transpose(-2, -1)
        dD = (dS * S).sum(-1)
        dW = -dvt @ S.transpose(-2, -1)
        dv[:, :, s0:s1] = c["M"].transpose(-2, -1) @ dvt
        dM = dvt @ c["v"].transpose(-2, -1) + dW @ c["Kg"].transpose(-2, -1)
        dKg = c["M"].transpose(-2, -1) @ dW
        N, b = c["N"], c["b"]
        db = (N * dM).sum(-2)
        Nt = N.transpose(-2, -1)
        dL = -(Nt @ (dM * b.unsqueeze(-2)) @ Nt) * c["strict"]
        dA = b.unsqueeze(-1) * dL
        db = db + (dL * c["A"]).sum(-1)
        # pair sums: A_ij = sum_k k_i k_j E_ij (strict), Aqk_ij = sum_k q_i k_j E_ij (lower)
        E, qc, kc = c["E"], c["q"], c["k"]
        PA = dA.unsqueeze(-1) * E            # [B,H,i,j,K]
        PQ = dAqk.unsqueeze(-1) * E
        dk_c = (PA * kc.unsqueeze(2)).sum(3) + (PA * kc.unsqueeze(3)).sum(2) + (PQ * qc.unsqueeze(3)).sum(2)
        dq_c = (PQ * kc.unsqueeze(2)).sum(3)
        pa = PA * kc.unsqueeze(3) * kc.unsqueeze(2)
        pq = PQ * qc.unsqueeze(3) * kc.unsqueeze(2)
        dlg = pa.sum(3) - pa.sum(2) + pq.sum(3) - pq.sum(2)
        # exp factors
        elg = c["lg"].exp()
        dk_c = dk_c + elg * dKg
        dlg = dlg + c["Kg"] * dKg
        dq_c = dq_c + elg * dQg
        dlg = dlg + c["Qg"] * dQg
        to_end = (c["lg"][:, :, -1:] - c["lg"]).exp()
        dk_c = dk_c + to_end * dKt
        dlg = dlg - c["Kt"] * dKt
        dlast = (c["Kt"] * dKt).sum(2) + c["D"] * dD
        dlg[:, :, -1] = dlg[:, :, -1] + dlast
        dq[:, :, s0:s1] = dq_c
        dk[:, :, s0:s1] = dk_c
        dg[:, :, s0:s1] = dlg.flip(2).cumsum(2).flip(2)
        dbeta[:, :, s0:s1] = db
        dS = c["D"].unsqueeze(-1) * dS + c["Qg"].transpose(-2, -1) @ dOc - c["W"].transpose(-2, -1) @ dvt
    back = lambda x: x.transpose(1, 2).contiguous()  # noqa: E731
    return back(dq), back(dk), back(dv), back(dg), back(dbeta), dS


# ---- the fused stages around the operator ------------------------------------

def _compute_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def short_conv(x, weight, bias=None, history=None):
    """Depthwise causal convolution over ``x [B,T,C]`` with lag-ordered
    ``weight [C,K]`` (``weight[c, j]`` multiplies ``x[t - j]``) and the last
    ``K-1`` inputs ``history [B,K-1,C]`` (zeros when None), as
    CausalShortConv1D.forward (src/kimi_primitives/short_conv.py:69-98).
    Computes in f32 (f64 for f64); returns (y, next history)."""
    cd = _compute_dtype(x.dtype)
    batch, tokens, channels = x.shape
    taps = weight.shape[1]
    hist = (torch.zeros(batch, taps - 1, channels, dtype=x.dtype) if history is None else history)
    combined = torch.cat((hist, x), dim=1).to(cd)
    w = weight.to(cd)
    y = torch.zeros(batch, tokens, channels, dtype=cd)
    for j in range(taps):
        # input at t - j sits at combined row (taps - 1) + t - j
        y = y + w[:, j] * combined[:, taps - 1 - j:taps - 1 - j + tokens]
    if bias is not None:
        y = y + bias.to(cd)
    nxt = combined[:, combined.shape[1] - (taps - 1):].to(x.dtype)
    return y, nxt


def conv_silu(x, weight, bias=None, history=None, attention_mask=None, *, num_heads=None,
              normalize=False, eps=1e-6):
    """ShortConv, SiLU and (``normalize``) L2 normalisation per head, with a
    right-padded row run on its valid prefix only (padded outputs zero,
    padding never in the history), as KDAProjections._run_conv and forward
    (src/kda/projections.py:100-140,185-204).  Returns (y [B,T,C] in the
    compute dtype, next history)."""
    batch, tokens, channels = x.shape
    outs, hists = [], []
    for b in range(batch):
        length = tokens if attention_mask is None else int(attention_mask[b].sum())
        hb = None if history is None else history[b:b + 1]
        y, nxt = short_conv(x[b:b + 1, :length], weight, bias, hb)
        y = y * torch.sigmoid(y)
        if normalize:
            heads = y.reshape(1, length, num_heads, channels // num_heads)
            norm = heads.square().sum(dim=-1, keepdim=True).sqrt()
            y = (heads / torch.clamp(norm, min=eps)).reshape(1, length, channels)
        outs.append(torch.cat((y, torch.zeros(1, tokens - length, channels, dtype=y.dtype)), dim=1))
        hists.append(nxt)
    return torch.cat(outs, dim=0), torch.cat(hists, dim=0)


def _clamp_eps(p, dtype):
    eps = torch.finfo(dtype).eps
    return p.clamp(eps, 1.0 - eps)


def lower_bounded_decay(logits, a_log, g_min=-5.0, bias=None):
    """``g = g_min * clamp(sigmoid(exp(A_log[h]) * z), eps, 1-eps)``, ``alpha = exp(g)``
    with ``z = logits (+ bias [H,K])`` and eps the logits dtype's machine
    epsilon (src/kda/decay.py:30-43, projections.py:211-218).  Compute dtype
    f32 (f64 for f64)."""
    cd = _compute_dtype(logits.dtype)
    z = logits.to(cd)
    if bias is not None:
        z = z + bias.to(cd)
    scale = a_log.to(cd).exp()[None, None, :, None]
    p = _clamp_eps(torch.sigmoid(scale * z), logits.dtype)
    g = g_min * p
    return g, g.exp()


def beta_gate(logits):
    """``clamp(sigmoid(logits), eps, 1-eps)`` (src/kda/projections.py:207-209)."""
    return _clamp_eps(torch.sigmoid(logits.to(_compute_dtype(logits.dtype))), logits.dtype)


def rmsnorm_gate(x, weight=None, eps=1e-6, gate_logits=None):
    """``x * rsqrt(mean(x^2) + eps) * weight`` over each head of ``x [B,T,H,D]``
    (src/kimi_primitives/headwise_rmsnorm.py:39-64), times
    ``sigmoid(gate_logits)`` (``[B,T,H*D]``) when given
    (src/kimi_primitives/output_gate.py:62-75)."""
    cd = _compute_dtype(x.dtype)
    xf = x.to(cd)
    y = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    if weight is not None:
        y = y * (weight.to(cd) if weight.ndim == 2 else weight.to(cd)[None, :])
    if gate_logits is not None:
        y = y * torch.sigmoid(gate_logits.to(cd)).reshape(x.shape)
    return y


def gather_rows(arrays, index=None):
    """Batch-row gather of every cache tensor: ``out[i] = a[index[i]]``.

    ``arrays`` are numpy arrays (or CPU tensors) sharing dimension 0; the rows
    are copied one at a time as bytes, so any dtype is exact.  ``index=None``
    is the clone (every row in order).  Raises ``IndexError`` for an index
    outside ``[0, batch)``, like ``index_select``.
    """
    import numpy as np

    out = []
    for a in arrays:
        a = np.ascontiguousarray(a.numpy() if isinstance(a, torch.Tensor) else a)
        n = a.shape[0]
        rows = range(n) if index is None else [int(i) for i in index]
        src = a.reshape(n, -1).view(np.uint8)
        dst = np.empty((len(rows), src.shape[1]), dtype=np.uint8)
        for r, i in enumerate(rows):
            if not 0 <= i < n:
                raise IndexError(f"index {i} out of range for a batch of {n}")
            dst[r] = src[i]
        out.append(dst.view(a.dtype).reshape((len(rows),) + a.shape[1:]))
    return out


# ---- the layer around the operator -------------------------------------------

def kda_layer(w, x, attention_mask=None, state=None, mode="chunkwise", output_final_state=False):
    """KimiDeltaAttention.forward (src/kda/kda.py:98-183, diagnostics left out)
    with the projections of KDAProjections.forward (src/kda/projections.py:144-225).

    ``w`` is a dict with the fields of ``kda.layer.KDALayerWeights`` (linear
    weights ``[out, in]``, ShortConv weights ``[C, K_conv]`` in lag order, ...);
    ``state`` is ``(recurrent [B,H,K,V], q_hist, k_hist, v_hist, offset [B])`` or
    None.  Each stage's result is rounded to the activation dtype as the
    reference's modules return it; arithmetic inside a stage is f32 (f64 for
    f64).  Returns (output [B,T,d_model], next state tuple or None)."""
    dt = x.dtype
    cd = _compute_dtype(dt)

    def lin(inp, weight, bias=None):
        out = torch.nn.functional.linear(inp.to(cd), weight.to(cd), None if bias is None else bias.to(cd))
        return out.to(dt)

    batch, tokens, _ = x.shape
    heads, kd, vd = w["num_heads"], w["key_head_dim"], w["value_head_dim"]
    return_state = output_final_state or mode == "decode"
    hists = (None, None, None) if state is None else state[1:4]
    convs = []
    for name, hist, norm in (("q", hists[0], True), ("k", hists[1], True), ("v", hists[2], False)):
        y, nxt = conv_silu(lin(x, w[f"{name}_proj"], w.get(f"{name}_proj_bias")), w[f"{name}_conv"].to(dt),
                           w.get(f"{name}_conv_bias"), hist, attention_mask, num_heads=heads, normalize=norm,
                           eps=w["eps"])
        convs.append((y.to(dt).reshape(batch, tokens, heads, -1), nxt))
    (q, qn), (k, kn), (v, vn) = convs
    beta = beta_gate(lin(x, w["beta_proj"], w.get("beta_bias"))).to(dt)
    z = lin(lin(x, w["alpha_down"]), w["alpha_up"]).reshape(batch, tokens, heads, kd)
    g, _ = lower_bounded_decay(z, w["a_log"], w["g_min"], bias=w["b_alpha"].to(dt))
    g = g.to(dt)
    initial = None if state is None else state[0]
    acc32 = w.get("accumulate_state_in_fp32", True)
    if mode == "chunkwise":
        core, final = chunkwise(q, k, v, g, beta, initial, attention_mask, chunk_size=w.get("chunk_size", 64),
                                secondary_tile_size=w.get("secondary_tile_size", 16), accumulate_state_in_fp32=acc32)
    else:
        core, final, _ = recurrent(q, k, v, g, beta, initial, attention_mask, accumulate_state_in_fp32=acc32)
    norm_w = w.get("norm_weight")
    gated = rmsnorm_gate(core.to(dt), None if norm_w is None else norm_w.to(dt), w["eps"],
                         gate_logits=lin(x, w["gate_proj"], w.get("gate_bias"))).to(dt)
    out = lin(gated.reshape(batch, tokens, heads * vd), w["output_proj"], w.get("output_bias"))
    if attention_mask is not None:
        out = out * attention_mask[..., None].to(dt)
    nxt = None
    if return_state:
        lengths = (torch.full((batch,), tokens, dtype=torch.long) if attention_mask is None
                   else attention_mask.sum(dim=1).to(torch.long))
        offset = lengths if state is None else state[4] + lengths
        nxt = (final, qn, kn, vn, offset)
    return out, nxt
