"""GPU parity of the chunkwise backward (kda_chunk_bwd through
chunkwise_kda's autograd) against the oracle's explicit backward, which is
itself pinned against autograd through the oracle's forward.

Tolerances (max|x - ref| / max|ref| per gradient): f32 inputs 2e-4 (f32
arithmetic against the f64 oracle on the same values), bf16 inputs 2e-2
(gradients computed in f32 and rounded once to bf16), f64 inputs 1e-10 (f64
arithmetic in another order).  Value widths past 128 differentiate in column
slices of at most 128 (q, k, g and beta gradients summed over the slices).
"""

from __future__ import annotations

import pytest
import torch

import kda
from oracle import kda_oracle as ora
from tests._inputs import random_core, record_margin, rel_err, workload

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 2e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}
NAMES = ("dq", "dk", "dv", "dg", "dbeta", "ds0")


def _case(B, T, H, K, V, dtype, seed):
    q, k, v, g, beta, s0 = workload(B, T, H, K, V, state_std=0.5, seed=seed, dtype=dtype)
    gen = torch.Generator().manual_seed(seed + 1)
    d_out = torch.randn(B, T, H, V, generator=gen).to(dtype)
    d_final = torch.randn(B, H, K, V, generator=gen)
    return (q, k, v, g, beta, s0), d_out, d_final


def _gpu_grads(inputs, d_out, d_final, mask=None, final=True):
    leaves = [t.to(DEV).requires_grad_() for t in inputs]
    res = kda.chunkwise_kda(*leaves, final, None if mask is None else mask.to(DEV))
    loss = (res.hidden_states.double() * d_out.to(DEV).double()).sum()
    if final:
        loss = loss + (res.final_state.double() * d_final.to(DEV).double()).sum()
    loss.backward()
    return [t.grad for t in leaves]


def _oracle_grads(inputs, d_out, d_final, final=True):
    q, k, v, g, beta, s0 = (t.double() for t in inputs)
    return ora.chunkwise_backward(q, k, v, g, beta, s0, d_out.double(), d_final.double() if final else None,
                                  chunk_size=64)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,K,V", [(2, 150, 2, 128, 128), (1, 64, 1, 64, 32), (2, 37, 3, 16, 48),
                                       (1, 200, 2, 128, 96), (1, 70, 1, 100, 40), (1, 90, 2, 64, 200),
                                       (8, 130, 16, 64, 64)])  # B x H = 128: one segment per sequence
def test_backward_matches_oracle(dtype, B, T, H, K, V):
    inputs, d_out, d_final = _case(B, T, H, K, V, dtype, seed=T + K)
    got = _gpu_grads(inputs, d_out, d_final)
    ref = _oracle_grads(inputs, d_out, d_final)
    for name, a, b, x in zip(NAMES, got, ref, inputs):
        assert a.dtype == x.dtype and a.shape == x.shape, name
        assert torch.isfinite(a).all(), name
        assert rel_err(a, b) < TOL[dtype], (name, rel_err(a, b))


def test_backward_without_initial_state_or_final_state():
    (q, k, v, g, beta, _), d_out, _ = _case(1, 100, 2, 128, 128, torch.float32, seed=3)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v, g, beta)]
    res = kda.chunkwise_kda(*leaves)
    (res.hidden_states * d_out.to(DEV)).sum().backward()
    ref = ora.chunkwise_backward(*(t.double() for t in (q, k, v, g, beta)), None, d_out.double(), None)
    for name, a, b in zip(NAMES, [t.grad for t in leaves], ref):
        assert rel_err(a, b) < TOL[torch.float32], name


def test_backward_with_right_padding_mask():
    B, T, H, K, V = 2, 90, 2, 128, 64
    inputs, d_out, d_final = _case(B, T, H, K, V, torch.float32, seed=4)
    mask = torch.arange(T)[None, :] < torch.tensor([T, 53])[:, None]
    got = _gpu_grads(inputs, d_out, d_final, mask=mask)
    q, k, v, g, beta, s0 = inputs
    qm, gm, bm = ora.mask_inputs(q, g, beta, mask)
    ref = list(_oracle_grads((qm, k, v, gm, bm, s0), d_out, d_final))
    keep = mask.double()
    ref[0] = ref[0] * keep[:, :, None, None]
    ref[3] = ref[3] * keep[:, :, None, None]
    ref[4] = ref[4] * keep[:, :, None]
    for name, a, b in zip(NAMES, got, ref):
        assert rel_err(a, b) < TOL[torch.float32], name
    assert torch.count_nonzero(got[0][1, 53:]) == 0 and torch.count_nonzero(got[4][1, 53:]) == 0


def test_backward_long_context_heads_subset():
    # B=1 T=8192 H=16 bf16 (the prefill workload); heads are independent, so the
    # oracle checks heads 0 and 15 of the full-size GPU gradients
    B, T, H, K, V = 1, 8192, 16, 128, 128
    inputs, d_out, d_final = _case(B, T, H, K, V, torch.bfloat16, seed=5)
    got = _gpu_grads(inputs, d_out, d_final)
    for h in (0, 15):
        sub = [t[:, :, h:h + 1] for t in inputs[:5]] + [inputs[5][:, h:h + 1]]
        ref = _oracle_grads(sub, d_out[:, :, h:h + 1], d_final[:, h:h + 1])
        errs = {}
        for name, a, b in zip(NAMES, got, ref):
            a_h = a[:, h:h + 1] if name == "ds0" else a[:, :, h:h + 1]
            errs[name] = rel_err(a_h, b)
        print(f"backward T=8192 head {h}: " + " ".join(f"{n} {e:.2e}" for n, e in errs.items()))
        record_margin(f"backward B=1 T=8192 H=16 K=V=128 bf16, head {h}", TOL[torch.bfloat16], **errs)
        for name, e in errs.items():
            assert e < TOL[torch.bfloat16], (name, h, e)


def test_backward_gpu_48gb_shape_full_length():
    # B=1 T=8192 H=16 K=V=64 bf16, the head shape of the reference's shipped
    # GPU profiles (config/kimi_full_pipeline/gpu_48gb/model.yaml:19); two heads
    # against the oracle at full length
    B, T, H, K, V = 1, 8192, 16, 64, 64
    inputs, d_out, d_final = _case(B, T, H, K, V, torch.bfloat16, seed=55)
    got = _gpu_grads(inputs, d_out, d_final)
    for h in (2, 13):
        sub = [t[:, :, h:h + 1] for t in inputs[:5]] + [inputs[5][:, h:h + 1]]
        ref = _oracle_grads(sub, d_out[:, :, h:h + 1], d_final[:, h:h + 1])
        errs = {}
        for name, a, b in zip(NAMES, got, ref):
            a_h = a[:, h:h + 1] if name == "ds0" else a[:, :, h:h + 1]
            errs[name] = rel_err(a_h, b)
        print(f"backward K=V=64 T=8192 head {h}: " + " ".join(f"{n} {e:.2e}" for n, e in errs.items()))
        record_margin(f"backward B=1 T=8192 H=16 K=V=64 bf16, head {h}", TOL[torch.bfloat16], **errs)
        for name, e in errs.items():
            assert e < TOL[torch.bfloat16], (name, h, e)


@pytest.mark.parametrize("B,T,H,K,V", [(1, 5, 2, 2, 3), (2, 130, 2, 128, 128), (1, 70, 1, 100, 40)])
def test_f64_backward_matches_oracle(B, T, H, K, V):
    # f64 inputs differentiate in f64 arithmetic (kda_chunk_bwd_f64.hip)
    inputs, d_out, d_final = _case(B, T, H, K, V, torch.float64, seed=T + 1)
    inputs = tuple(t.double() for t in inputs)  # the initial state too
    got = _gpu_grads(inputs, d_out, d_final.double())
    ref = _oracle_grads(inputs, d_out, d_final)
    for name, a, b in zip(NAMES, got, ref):
        assert a.dtype == torch.float64, name
        assert rel_err(a, b) < 1e-10, (name, rel_err(a, b))


@pytest.mark.parametrize("op", ["chunkwise", "recurrent"])
def test_f64_gradcheck_like_the_reference(op):
    # tests/kda/test_kda_chunkwise_equivalence.py:115-134 and
    # tests/kda/test_kda_recurrent.py:184-193 (gradcheck; the second derivative
    # of gradgradcheck is not provided by this backend)
    inputs, _, _ = _case(1, 3, 1, 2, 2, torch.float64, seed=21)
    leaves = tuple(t.double().to(DEV).requires_grad_() for t in inputs)
    fn = kda.chunkwise_kda if op == "chunkwise" else kda.recurrent_kda

    def function(*xs):
        res = fn(*xs, True)
        return res.hidden_states, res.final_state

    assert torch.autograd.gradcheck(function, leaves, fast_mode=True)


def test_recurrent_and_chunkwise_f64_gradients_agree():
    # tests/kda/test_kda_chunkwise_equivalence.py:92-112: rtol 2e-10, atol 2e-11
    inputs, _, _ = _case(1, 5, 2, 2, 3, torch.float64, seed=22)
    rec = [t.double().to(DEV).requires_grad_() for t in inputs]
    chk = [t.double().to(DEV).requires_grad_() for t in inputs]
    r = kda.recurrent_kda(*rec, output_final_state=True)
    c = kda.chunkwise_kda(*chk, output_final_state=True, chunk_size=3, secondary_tile_size=2)
    (r.hidden_states.square().sum() + r.final_state.square().sum()).backward()
    (c.hidden_states.square().sum() + c.final_state.square().sum()).backward()
    for a, b in zip(rec, chk):
        torch.testing.assert_close(a.grad, b.grad, rtol=2e-10, atol=2e-11)


@pytest.mark.parametrize("op", ["chunkwise", "recurrent"])
def test_gradgradcheck_like_the_reference(op):
    # the reference's test_recurrent_gradcheck_and_gradgradcheck
    # (tests/kda/test_kda_recurrent.py:184-198): f64, B=1, T=2, H=1, K=V=2,
    # gradcheck of output and final state, gradgradcheck of the output; the
    # second derivatives come from kda_chunk_grad_tangent
    fn_op = kda.chunkwise_kda if op == "chunkwise" else kda.recurrent_kda
    inputs = tuple(t.to(DEV).requires_grad_() for t in random_core(batch=1, tokens=2, heads=1, key_dim=2,
                                                                    value_dim=2))
    both = lambda *xs: (fn_op(*xs, output_final_state=True).hidden_states,  # noqa: E731
                        fn_op(*xs, output_final_state=True).final_state)
    assert torch.autograd.gradcheck(both, inputs, fast_mode=True)
    assert torch.autograd.gradgradcheck(lambda *xs: fn_op(*xs).hidden_states, inputs, fast_mode=True)


@pytest.mark.parametrize("B,T,H,K,V", [(2, 70, 2, 5, 3), (1, 130, 1, 16, 8)])
def test_gradgradcheck_across_chunks_with_mask(B, T, H, K, V):
    # several chunks, right padding, the final state in the loss, every input
    # (initial state included) and both cotangents differentiated twice
    q, k, v, g, beta, state = random_core(batch=B, tokens=T, heads=H, key_dim=K, value_dim=V, seed=T)
    g = g * 0.1  # a slow decay keeps every chunk's terms in play
    mask = torch.ones(B, T, dtype=torch.bool)
    mask[-1, T - 11:] = False
    inputs = tuple(t.to(DEV).requires_grad_() for t in (q, k, v, g, beta, state))

    def fn(*xs):
        r = kda.chunkwise_kda(*xs, True, mask.to(DEV))
        return r.hidden_states, r.final_state

    assert torch.autograd.gradgradcheck(fn, inputs, fast_mode=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_second_derivative_in_lower_precision_inputs(dtype):
    # the double backward of f32/bf16 inputs runs in f64 on the same (rounded)
    # values: a Hessian-vector product through the f32 first backward agrees
    # with the f64 one to the first backward's precision
    q, k, v, g, beta, state = workload(1, 90, 2, 32, 16, state_std=0.3, seed=8, dtype=dtype)
    gen = torch.Generator().manual_seed(9)
    u = [torch.randn(t.shape, generator=gen, dtype=torch.float64) for t in (q, k, v, g, beta)]

    def hvp(tensors, st):
        leaves = [t.to(DEV).requires_grad_() for t in tensors]
        s0 = st.to(DEV).requires_grad_()
        r = kda.chunkwise_kda(*leaves, s0, True)
        loss = r.hidden_states.double().square().sum() + r.final_state.double().square().sum()
        grads = torch.autograd.grad(loss, leaves + [s0], create_graph=True)
        dot = sum((gr.double() * w.to(DEV)).sum() for gr, w in zip(grads[:5], u))
        return torch.autograd.grad(dot, leaves + [s0])

    got = hvp((q, k, v, g, beta), state)
    ref = hvp([t.double() for t in (q, k, v, g, beta)], state.double())
    for name, a, b in zip(NAMES, got, ref):
        e = rel_err(a, b)
        print(f"{dtype} Hessian-vector product {name}: {e:.2e}")
        assert e < TOL[dtype], (name, e)


def test_third_derivative_and_packed_second_derivative_raise():
    q, k, v, g, beta, state = (t.to(DEV).double() for t in workload(1, 6, 1, 16, 16, state_std=0.1, seed=3))
    q.requires_grad_()
    out = kda.chunkwise_kda(q, k, v, g, beta, state, True).hidden_states
    (gq,) = torch.autograd.grad(out.square().sum(), q, create_graph=True)
    (hq,) = torch.autograd.grad(gq.square().sum(), q, create_graph=True)
    with pytest.raises(RuntimeError, match="once_differentiable|twice"):
        hq.sum().backward()
    out = kda.chunkwise_kda(q, k, v, g, beta, None, True, cu_seqlens=[0, 2, 6]).hidden_states
    with pytest.raises(RuntimeError, match="dense inputs"):
        torch.autograd.grad(out.square().sum(), q, create_graph=True)


def test_backward_refuses_unsupported_cases():
    q2, k2, v2, g2, b2, _ = (t.to(DEV) for t in workload(1, 8, 1, 16, 16, state_std=0.1))
    with pytest.raises(RuntimeError, match="up to 128"):
        kda.chunkwise_kda(*(t.repeat(1, 1, 1, 9) for t in (q2.requires_grad_(), k2)), v2, g2.repeat(1, 1, 1, 9), b2)


@pytest.mark.parametrize("op", ["chunkwise", "recurrent"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_packed_documents_gradients_match_per_document_oracle(op, dtype):
    # cu_seqlens under autograd: every document's slice of the gradients (and
    # its initial-state gradient) equals the oracle's backward of that document
    lens = [70, 1, 130, 64]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    H, K, V = 2, 128, 64
    q, k, v, g, beta, _ = workload(1, cu[-1], H, K, V, state_std=0.5, seed=12, dtype=dtype)
    gen = torch.Generator().manual_seed(13)
    s0 = torch.randn(len(lens), H, K, V, generator=gen) * 0.5
    d_out = torch.randn(1, cu[-1], H, V, generator=gen).to(dtype)
    d_final = torch.randn(len(lens), H, K, V, generator=gen)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v, g, beta, s0)]
    fn = kda.chunkwise_kda if op == "chunkwise" else kda.recurrent_kda
    res = fn(*leaves, True, cu_seqlens=torch.tensor(cu, dtype=torch.int32))
    ((res.hidden_states.float() * d_out.to(DEV).float()).sum() + (res.final_state * d_final.to(DEV)).sum()).backward()
    for i, (a0, a1) in enumerate(zip(cu[:-1], cu[1:])):
        doc = [t[:, a0:a1] for t in (q, k, v, g, beta)] + [s0[i:i + 1]]
        ref = _oracle_grads(doc, d_out[:, a0:a1], d_final[i:i + 1])
        for name, leaf, b in zip(NAMES, leaves, ref):
            a = leaf.grad[i:i + 1] if name == "ds0" else leaf.grad[:, a0:a1]
            assert torch.isfinite(a).all(), (name, i)
            assert rel_err(a, b) < TOL[dtype], (name, i, rel_err(a, b))


def test_many_packed_documents_backward_in_length_buckets():
    # 24 documents of 40..200 tokens: the backward stacks documents within a
    # fifth of each other's length into zero-padded batches (a few calls instead
    # of one per document); every document's gradients equal those of its own
    # call, and two of them the oracle's
    from kda.chunkwise import _document_buckets

    gen = torch.Generator().manual_seed(70)
    lens = [int(x) for x in torch.randint(40, 201, (24,), generator=gen)]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    buckets = _document_buckets(lens, lambda n, t: True)
    assert len(buckets) < len(lens) and max(len(b) for b in buckets) > 2
    H, K, V = 2, 128, 64
    q, k, v, g, beta, _ = workload(1, cu[-1], H, K, V, state_std=0.5, seed=71, dtype=torch.float32)
    s0 = torch.randn(len(lens), H, K, V, generator=gen) * 0.5
    d_out = torch.randn(1, cu[-1], H, V, generator=gen)
    d_final = torch.randn(len(lens), H, K, V, generator=gen)
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v, g, beta, s0)]
    res = kda.chunkwise_kda(*leaves, True, cu_seqlens=cu)
    ((res.hidden_states * d_out.to(DEV)).sum() + (res.final_state * d_final.to(DEV)).sum()).backward()
    for i, (a0, a1) in enumerate(zip(cu[:-1], cu[1:])):
        doc = [t[:, a0:a1] for t in (q, k, v, g, beta)] + [s0[i:i + 1]]
        alone = _gpu_grads(doc, d_out[:, a0:a1], d_final[i:i + 1])
        for name, leaf, b in zip(NAMES, leaves, alone):
            a = leaf.grad[i:i + 1] if name == "ds0" else leaf.grad[:, a0:a1]
            assert rel_err(a, b) < 1e-5, (name, i, rel_err(a, b))
    for i in (0, 17):
        a0, a1 = cu[i], cu[i + 1]
        ref = _oracle_grads([t[:, a0:a1] for t in (q, k, v, g, beta)] + [s0[i:i + 1]], d_out[:, a0:a1],
                            d_final[i:i + 1])
        for name, leaf, b in zip(NAMES, leaves, ref):
            a = leaf.grad[i:i + 1] if name == "ds0" else leaf.grad[:, a0:a1]
            assert rel_err(a, b) < TOL[torch.float32], (name, i)


@pytest.mark.parametrize("key_dim", [128, 64])
@pytest.mark.parametrize("regime", ["steep", "rising"])
def test_backward_exact_path_regimes(regime, key_dim):
    # chunks whose decay falls by more than 80 within 16 tokens, or whose g is
    # positive somewhere, take the exact pairwise path instead of the MFMA
    # factorisation (a second pass over the key channels, four quarters at
    # key_dim 128 and two at 64); both must match the oracle
    B, T, H, K, V = 1, 128, 2, key_dim, 64
    inputs, d_out, d_final = _case(B, T, H, K, V, torch.float32, seed=6)
    q, k, v, g, beta, s0 = inputs
    gen = torch.Generator().manual_seed(7)
    if regime == "steep":
        g = -6.0 - 6.0 * torch.rand(B, T, H, K, generator=gen)
    else:
        g = 0.02 * torch.randn(B, T, H, K, generator=gen)
    inputs = (q, k, v, g, beta, s0)
    got = _gpu_grads(inputs, d_out, d_final)
    ref = _oracle_grads(inputs, d_out, d_final)
    # dg is a reverse cumulative sum of terms that cancel when the decay is
    # steep: the oracle itself evaluated in f32 misses the f64 dg by 2e-5
    # (key_dim 128) and 8e-5 (64) while the other gradients stay near 2e-7,
    # so each gradient is held to 2e-4 or five times plain f32's own error
    ref32 = ora.chunkwise_backward(q.float(), k.float(), v.float(), g.float(), beta.float(), s0.float(),
                                   d_out.float(), d_final.float(), chunk_size=64)
    for name, a, b, c in zip(NAMES, got, ref, ref32):
        assert torch.isfinite(a).all(), name
        tol = max(TOL[torch.float32], 5.0 * rel_err(c, b))
        assert rel_err(a, b) < tol, (name, rel_err(a, b), tol)


def test_recurrent_kda_gradients_match_oracle():
    # recurrent_kda under autograd: the recurrent forward, the chunk backward
    # (the same gradients as the exact recurrence, test_kda_recurrent.py:184-198)
    inputs, d_out, d_final = _case(2, 40, 2, 64, 32, torch.float32, seed=8)
    leaves = [t.to(DEV).requires_grad_() for t in inputs]
    res = kda.recurrent_kda(*leaves, True)
    ((res.hidden_states * d_out.to(DEV)).sum() + (res.final_state * d_final.to(DEV)).sum()).backward()
    ref = _oracle_grads(inputs, d_out, d_final)
    for name, a, b in zip(NAMES, [t.grad for t in leaves], ref):
        assert rel_err(a, b) < TOL[torch.float32], name
    with pytest.raises(RuntimeError, match="update_state_in_place"):
        kda.recurrent_kda(*leaves, True, update_state_in_place=True)


def test_decode_step_gradients():
    # a single decode step (T=1) under autograd
    inputs, d_out, d_final = _case(3, 1, 2, 128, 128, torch.bfloat16, seed=9)
    got = []
    leaves = [t.to(DEV).requires_grad_() for t in inputs]
    res = kda.recurrent_kda(*leaves, True)
    ((res.hidden_states.float() * d_out.to(DEV).float()).sum() + (res.final_state * d_final.to(DEV)).sum()).backward()
    got = [t.grad for t in leaves]
    ref = _oracle_grads(inputs, d_out, d_final)
    for name, a, b in zip(NAMES, got, ref):
        assert rel_err(a, b) < TOL[torch.bfloat16], name


def test_backward_f16_inputs():
    inputs, d_out, d_final = _case(1, 130, 2, 128, 128, torch.float16, seed=10)
    got = _gpu_grads(inputs, d_out, d_final)
    ref = _oracle_grads(inputs, d_out, d_final)
    for name, a, b, x in zip(NAMES, got, ref, inputs):
        assert a.dtype == x.dtype, name
        assert rel_err(a, b) < TOL[torch.float16], (name, rel_err(a, b))


def test_workspace_beyond_free_memory_raises_a_clear_error():
    # the wrappers check a kernel workspace against the device's free memory
    # before allocating it (a 32,768-token document at H=64 needs ~20 GB)
    from kda import _prep

    with pytest.raises(RuntimeError, match="needs a workspace of .* GiB"):
        _prep.workspace(1 << 50, torch.device(DEV), "the chunkwise_kda backward")
    assert _prep.workspace(0, torch.device(DEV), "nothing") is None
    assert _prep.workspace(4096, torch.device(DEV), "a small call").numel() == 4096


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float64])
def test_backward_in_head_groups_matches_one_call(monkeypatch, dtype):
    # a call whose workspace passes WORKSPACE_LIMIT runs its heads in
    # groups (here 5 heads in groups of 2, 2 and 1): the gradients are those of
    # the single call (the groups' segment plans differ, so to rounding) and
    # the oracle's
    from kda import chunkwise, _lib

    B, T, H, K, V = 2, 200, 5, 128, 96
    inputs, d_out, d_final = _case(B, T, H, K, V, dtype, seed=81)
    if dtype == torch.float64:
        inputs, d_final = tuple(t.double() for t in inputs), d_final.double()
    whole = _gpu_grads(inputs, d_out, d_final)
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    limit = lib.kda_chunk_bwd_workspace_bytes(B, T, 2, K, V, code)
    assert lib.kda_chunk_bwd_workspace_bytes(B, T, 3, K, V, code) > limit
    monkeypatch.setattr(chunkwise, "WORKSPACE_LIMIT", limit)
    assert chunkwise._head_group(lambda n: lib.kda_chunk_bwd_workspace_bytes(B, T, n, K, V, code), H) == 2
    grouped = _gpu_grads(inputs, d_out, d_final)
    ref = _oracle_grads(inputs, d_out, d_final)
    same = 1e-12 if dtype == torch.float64 else 1e-5
    for name, a, b, r in zip(NAMES, grouped, whole, ref):
        assert rel_err(a, b) < same, (name, rel_err(a, b))
        assert rel_err(a, r) < TOL.get(dtype, 1e-10), (name, rel_err(a, r))


def test_packed_backward_in_head_groups(monkeypatch):
    # packed documents with the head split: each bucket's call goes in head
    # groups; every document's gradients still equal those of its own call
    from kda import chunkwise, _lib

    lens = [150, 140, 60]
    cu = [0, 150, 290, 350]
    H, K, V = 3, 64, 64
    q, k, v, g, beta, _ = workload(1, cu[-1], H, K, V, state_std=0.5, seed=91, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(92)
    s0 = torch.randn(len(lens), H, K, V, generator=gen) * 0.5
    d_out = torch.randn(1, cu[-1], H, V, generator=gen).bfloat16()
    d_final = torch.randn(len(lens), H, K, V, generator=gen)
    lib = _lib.load()
    monkeypatch.setattr(chunkwise, "WORKSPACE_LIMIT",
                        lib.kda_chunk_bwd_workspace_bytes(1, 150, 1, K, V, _lib.dtype_code(torch.bfloat16)))
    leaves = [t.to(DEV).requires_grad_() for t in (q, k, v, g, beta, s0)]
    res = kda.chunkwise_kda(*leaves, True, cu_seqlens=cu)
    ((res.hidden_states.float() * d_out.to(DEV).float()).sum()
     + (res.final_state * d_final.to(DEV)).sum()).backward()
    monkeypatch.undo()
    for i, (a0, a1) in enumerate(zip(cu[:-1], cu[1:])):
        doc = [t[:, a0:a1] for t in (q, k, v, g, beta)] + [s0[i:i + 1]]
        alone = _gpu_grads(doc, d_out[:, a0:a1], d_final[i:i + 1])
        for name, leaf, b in zip(NAMES, leaves, alone):
            a = leaf.grad[i:i + 1] if name == "ds0" else leaf.grad[:, a0:a1]
            assert torch.isfinite(a).all(), (name, i)
            assert rel_err(a, b) < 1e-2, (name, i, rel_err(a, b))
