"""``AXSMultiheadAttentionUnified`` (modules_unified.py:192-264 in the
reference) checked stage by stage on the GPU, forward and backward, against
an fp64 restatement of the reference's forward fed with the GPU's own
intermediate tensors at each stage boundary:

  q, k, v, out projections  FQ(in) FQ(W)^T + b           rel-L2 <= 1e-3
  scores, mask, softmax     (q k^T) * d^-1/2 + mask       rel-L2 <= 1e-5
  probability FQ            stochastic NF5 FQ with the    bit-exact
                            library's dither stream (seed drawn from
                            torch's CPU generator), restated by the oracle
  probs_q . v               fp64                          rel-L2 <= 1e-5
  backward                  the reference's autograd graph in fp64 through
                            the same quantized probabilities (STE through
                            both FQs), dY taken as given  rel-L2 <= 1e-3

Feeding each stage the GPU's inputs keeps a LUT-cell flip of one FQ (an
input within 1e-4 of a code boundary) from standing in for an error
elsewhere; the stochastic formula itself is pinned to the reference by
tests/golden/stochastic.npz through the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _fq64(t: torch.Tensor) -> torch.Tensor:
    """Nearest NF5 FQ (C oracle) of a float tensor, as float64 on the CPU."""
    a = t.detach().float().cpu().numpy()
    return torch.from_numpy(oracle.fake_quantize(a, 32)).double()


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return oracle.rel_l2(a.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())


@pytest.mark.parametrize("B,T,E,H", [(2, 64, 128, 4), (3, 48, 256, 4)])
def test_attention_stagewise_parity(B, T, E, H):
    import axs.unified as u
    from axs.unified import modules_unified as mu

    print(f"[attention B={B} T={T} E={E} H={H}]", flush=True)
    torch.manual_seed(3)
    mha = u.AXSMultiheadAttentionUnified(E, H).to(DEV)
    projs = {"q": mha.q_proj, "k": mha.k_proj, "v": mha.v_proj, "o": mha.out_proj}
    for p in projs.values():
        p.quantize_grad = False          # dY as given: a deterministic backward to restate
    g = torch.Generator().manual_seed(B * T)
    x = torch.randn(B, T, E, generator=g).to(DEV).requires_grad_(True)
    mask = torch.triu(torch.full((T, T), float("-inf"), device=DEV), diagonal=1)

    cap = {}
    handles = [m.register_forward_hook(lambda mod, inp, out, n=n: cap.__setitem__(n, (inp[0].detach(), out.detach())))
               for n, m in projs.items()]
    real_fq = mu.fake_quantize_unified

    def fq_spy(t, bs, rounding):
        out = real_fq(t, bs, rounding)
        cap["p"] = (t.detach().clone(), out.detach().clone(), rounding)
        return out

    mu.fake_quantize_unified = fq_spy
    try:
        torch.manual_seed(1234)
        y = mha(x, x, x, attn_mask=mask)
    finally:
        mu.fake_quantize_unified = real_fq
        for h in handles:
            h.remove()
    torch.manual_seed(1234)
    seed = int(torch.randint(0, 2**62, (1,)).item())

    D = E // H
    # projections
    W = {n: (m.weight.detach().cpu().double(), m.bias.detach().cpu().double()) for n, m in projs.items()}
    for n in projs:
        inp, out = cap[n]
        want = _fq64(inp).reshape(-1, E) @ _fq64(W[n][0]).T + W[n][1]
        e = _rel(out.reshape(-1, E), want)
        print(f"  {n}_proj rel-L2 {e:.2e}", flush=True)
        assert e <= 1e-3, n
    q = cap["q"][1].cpu().double().reshape(B, T, H, D).transpose(1, 2)
    k = cap["k"][1].cpu().double().reshape(B, T, H, D).transpose(1, 2)
    v = cap["v"][1].cpu().double().reshape(B, T, H, D).transpose(1, 2)
    scores = (q @ k.transpose(-2, -1)) * mha.scale + mask.cpu().double()
    probs = torch.softmax(scores, dim=-1)
    p_in, p_q, rounding = cap["p"]
    assert rounding == "stochastic"
    e = _rel(p_in, probs)
    print(f"  softmax rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-5
    # the probability FQ: bit-exact given the library's draws
    pin = p_in.cpu().numpy().reshape(-1, T)
    want_pq = oracle.fake_quantize(pin, 32, oracle.uniform(seed, 0, pin.size)).reshape(p_q.shape)
    got_pq = p_q.cpu().numpy()
    assert np.array_equal(got_pq.view(np.uint32), want_pq.view(np.uint32)), "probability FQ differs from the oracle"
    pq = p_q.cpu().double()
    attn = (pq @ v).transpose(1, 2).reshape(B, T, E)
    e = _rel(cap["o"][0], attn)
    print(f"  probs.v rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-5
    assert torch.equal(y.detach(), cap["o"][1])

    # backward: the reference's graph in fp64 from the GPU's intermediates
    dy = torch.randn(B, T, E, generator=g)
    y.backward(dy.to(DEV))
    d = dy.double().reshape(-1, E)
    a_in = cap["o"][0].cpu()
    d_attn = (d @ _fq64(W["o"][0])).reshape(B, T, H, D).transpose(1, 2)
    g_o = (d.T @ _fq64(a_in).reshape(-1, E), d.sum(0))
    d_pq = d_attn @ v.transpose(-2, -1)                      # STE: dprobs = dprobs_q
    dv = pq.transpose(-2, -1) @ d_attn
    pr = p_in.cpu().double()
    d_scores = pr * (d_pq - (d_pq * pr).sum(-1, keepdim=True))
    dq = (d_scores @ k) * mha.scale
    dk = (d_scores.transpose(-2, -1) @ q) * mha.scale
    xq = _fq64(cap["q"][0]).reshape(-1, E)
    dx = torch.zeros(B * T, E, dtype=torch.float64)
    grads = {"o": g_o}
    dsum = {"o": d.abs().sum(0)}
    for n, dd in (("q", dq), ("k", dk), ("v", dv)):
        dflat = dd.transpose(1, 2).reshape(-1, E)
        dx += dflat @ _fq64(W[n][0])
        grads[n] = (dflat.T @ xq, dflat.sum(0))
        dsum[n] = dflat.abs().sum(0)
    e = _rel(x.grad.reshape(-1, E), dx)
    print(f"  dX rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-3
    for n, m in projs.items():
        ew = _rel(m.weight.grad, grads[n][0])
        # bias gradients against the scale of the column sums they add up: the
        # key bias's exact gradient is 0 (a shift of every key moves a query's
        # scores together, which the softmax ignores), so both sides are
        # rounding residue there and a relative error would be meaningless
        want_b = grads[n][1]
        scale = max(want_b.norm().item(), dsum[n].norm().item())
        eb = (m.bias.grad.detach().double().cpu() - want_b).norm().item() / scale
        print(f"  d{n}_proj W {ew:.2e} b {eb:.2e}", flush=True)
        assert ew <= 1e-3 and eb <= 1e-3, n


@pytest.mark.parametrize("bias", [True, False, "some"])
def test_linear_group_matches_separate(bias):
    """axs_linear_group_unified (weights stacked, input packed once): each
    forward output equals its own axs_linear_unified bit for bit; the
    backward (nearest dY) gives dX = sum_i dY_i FQ(W_i), dW_i = dY_i^T FQ(X)
    and db_i = sum dY_i within the linear's rel-L2 1e-3 (db 1e-5) of fp64."""
    from axs.unified import axs_linear_group_unified, axs_linear_unified

    g = torch.Generator().manual_seed(11)
    M, K, sizes = 300, 256, (256, 128, 96)
    x = torch.randn(M, K, generator=g)
    ws = [torch.randn(n, K, generator=g) * K ** -0.5 for n in sizes]
    bs = [torch.randn(n, generator=g) for n in sizes]
    if bias is False:
        bs = [None] * 3
    elif bias == "some":
        bs[1] = None
    xd = x.to(DEV).requires_grad_(True)
    wd = [w.to(DEV).requires_grad_(True) for w in ws]
    bd = [None if b is None else b.to(DEV).requires_grad_(True) for b in bs]
    ys = axs_linear_group_unified(xd, wd, bd, 32, True, False)
    assert [tuple(y.shape) for y in ys] == [(M, n) for n in sizes]
    for y, w, b in zip(ys, wd, bd):
        sep = axs_linear_unified(xd.detach(), w.detach(), None if b is None else b.detach(), 32, True, False)
        assert torch.equal(y.detach(), sep), "grouped forward differs from the separate one"
    dys = [torch.randn(M, n, generator=g) for n in sizes]
    torch.autograd.backward(ys, [d.to(DEV) for d in dys])
    xq = _fq64(x)
    dx = sum(d.double() @ _fq64(w) for d, w in zip(dys, ws))
    assert _rel(xd.grad, dx) <= 1e-3
    for d, w, b in zip(dys, wd, bd):
        assert _rel(w.grad, d.double().T @ xq) <= 1e-3
        if b is not None:
            assert _rel(b.grad, d.double().sum(0)) <= 1e-5


@pytest.mark.parametrize("shape", [(300, 256, (256, 128, 96)), (8192, 256, (256, 256, 256))])
def test_linear_group_backward_is_a_reordering(shape):
    """The grouped backward against the three separate backwards on the GPU
    (nearest dY, same operands): the stacked statistics only move each
    fp16 operand row by a power of two, so the products are the same; what
    differs is the order of fp32 additions (dX: one accumulator over all
    stacked outputs instead of three results added afterwards; dW: the
    split-K plan of the stacked shape).  So the gradients agree to fp32
    rounding, far inside the linear's 1e-3 against fp64: a change in what
    is computed (a dropped group, a wrong row scale) fails here."""
    from axs.unified import axs_linear_group_unified, axs_linear_unified

    M, K, sizes = shape
    g = torch.Generator().manual_seed(12)
    x = torch.randn(M, K, generator=g).to(DEV)
    ws = [(torch.randn(n, K, generator=g) * K ** -0.5).to(DEV) for n in sizes]
    bs = [torch.randn(n, generator=g).to(DEV) for n in sizes]
    # dY rows of very different scale per group, as q/k/v gradients have
    dys = [(torch.randn(M, n, generator=g) * 10.0 ** (2 - 2 * i)).to(DEV) for i, n in enumerate(sizes)]

    def grads(grouped):
        xd = x.clone().requires_grad_(True)
        wd = [w.clone().requires_grad_(True) for w in ws]
        bd = [b.clone().requires_grad_(True) for b in bs]
        if grouped:
            ys = axs_linear_group_unified(xd, wd, bd, 32, True, False)
        else:
            ys = [axs_linear_unified(xd, w, b, 32, True, False) for w, b in zip(wd, bd)]
        torch.autograd.backward(ys, dys)
        return xd.grad, [w.grad for w in wd], [b.grad for b in bd]

    gx, gw, gb = grads(True)
    sx, sw, sb = grads(False)
    assert _rel(gx, sx.double()) <= 1e-6
    for a, b in zip(gw, sw):
        assert _rel(a, b.double()) <= 1e-6
    for a, b in zip(gb, sb):
        assert _rel(a, b.double()) <= 1e-6


def test_self_attention_groups_projections():
    """Self-attention runs q/k/v as one grouped linear: the output equals the
    one-by-one projections' (forced by a hook on q_proj) bit for bit."""
    import axs.unified as u

    torch.manual_seed(5)
    mha = u.AXSMultiheadAttentionUnified(128, 4).to(DEV)
    x = torch.randn(2, 32, 128, generator=torch.Generator().manual_seed(6)).to(DEV)
    calls = []
    orig = u.functional_unified.axs_linear_unified
    torch.manual_seed(7)
    y_grouped = mha(x, x, x)
    h = mha.q_proj.register_forward_hook(lambda m, i, o: calls.append(1))
    torch.manual_seed(7)
    y_sep = mha(x, x, x)
    h.remove()
    assert calls == [1] and orig is u.functional_unified.axs_linear_unified
    assert torch.equal(y_grouped, y_sep)
