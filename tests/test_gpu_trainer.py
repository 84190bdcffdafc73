"""GPU parity of the trainer-support kernels (soft-capped cross entropy) against the oracle."""

from __future__ import annotations

import math
import numpy as np
import pytest
import torch

from oracle import kda_oracle as O
from tests.kda_testutil import rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import ops
    from experiment_swa_kda_amd.model import softcap_cross_entropy


def _case(rows, vocab, stride, scale, seed, ignore_every=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, stride, generator=g) * scale).bfloat16()
    t = torch.randint(0, vocab, (rows,), generator=g)
    if ignore_every:
        t[::ignore_every] = -1
    return x, t


@pytest.mark.parametrize("rows,vocab,stride,scale,ignore_every", [
    (300, 1000, 1024, 3.0, 7),      # padded vocabulary, ignored rows
    (64, 32768, 32768, 1.0, 0),     # the trainer's vocabulary
    (33, 4101, 4104, 60.0, 3),      # saturated tanh, ragged vocab tail
    (5, 8, 8, 1.0, 0),              # one vector per row
])
def test_softcap_ce_matches_oracle(rows, vocab, stride, scale, ignore_every):
    x, t = _case(rows, vocab, stride, scale, seed=rows + vocab, ignore_every=ignore_every)
    loss_o, rows_o, lse_o, d_o = O.softcap_cross_entropy(x.double().numpy(), t.numpy(), vocab, 15.0, -1)
    xd, td = x.cuda().requires_grad_(), t.cuda()
    loss = softcap_cross_entropy(xd, td, vocab, 15.0, -1)
    loss.backward()
    # f32 arithmetic with ~1 ulp exp/rcp: the loss to ~1e-6, the bf16 gradient to bf16 rounding
    assert abs(loss.item() - loss_o) <= 1e-5 * max(1.0, abs(loss_o))
    lr, lse = ops.softcap_cross_entropy_forward(xd.detach(), td, vocab, 15.0, -1)
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse_o, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(lr.cpu().double().numpy(), rows_o, rtol=2e-5, atol=2e-5)
    d = xd.grad.float().cpu()
    assert rel_err(d, d_o) < 5e-3
    assert torch.all(d[:, vocab:] == 0)
    if ignore_every:
        assert torch.all(d[::ignore_every] == 0)


@pytest.mark.parametrize("cap", [15.0, 60.0])
def test_softcap_ce_extreme_logits_match_oracle(cap):
    """The kernels look z up per bf16 bit pattern and clamp |x| outside [2^-24, 2^9): zeros,
    bf16 denormals, tiny, huge and infinite logits (targets on them too) still match the
    fp64 oracle, which evaluates tanh exactly."""
    rows, vocab = 24, 8192  # two full 4096-column chunks per row: the kernels' fast path
    x, t = _case(rows, vocab, vocab, 4.0, seed=11)
    specials = torch.tensor([0.0, -0.0, 1e-40, -1e-39, 3e-8, -6e-8, 1e-30, 600.0, -600.0,
                             1e4, -3e38, float("inf"), float("-inf"), 300.0, -511.0, 2.0 ** -24])
    g = torch.Generator().manual_seed(3)
    for r in range(rows):
        cols = torch.randperm(vocab, generator=g)[:64]
        x[r, cols] = specials[torch.arange(64) % len(specials)].bfloat16()
        if r % 3 == 0:
            x[r, t[r]] = specials[r % len(specials)].bfloat16()
    loss_o, rows_o, lse_o, d_o = O.softcap_cross_entropy(x.double().numpy(), t.numpy(), vocab, cap, -1)
    xd, td = x.cuda().requires_grad_(), t.cuda()
    loss = softcap_cross_entropy(xd, td, vocab, cap, -1)
    loss.backward()
    assert abs(loss.item() - loss_o) <= 1e-5 * max(1.0, abs(loss_o))
    lr, lse = ops.softcap_cross_entropy_forward(xd.detach(), td, vocab, cap, -1)
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse_o, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(lr.cpu().double().numpy(), rows_o, rtol=2e-5, atol=2e-5)
    assert rel_err(xd.grad.float().cpu(), d_o) < 5e-3


@pytest.mark.parametrize("vocab", [8192, 8200])
def test_softcap_ce_nan_logit_poisons_row(vocab):
    """A NaN logit anywhere in a row (fast full-chunk path at vocab 8192, masked tail at 8200)
    makes that row's loss and lse NaN and its gradient row NaN, as tanh followed by the library
    cross entropy does; the other rows stay finite and match the oracle."""
    rows = 8
    x, t = _case(rows, vocab, vocab + (-vocab % 8), 4.0, seed=13)
    x[2, 17] = float("nan")
    x[5, vocab - 1] = float("nan")  # in the tail chunk when vocab = 8200
    xd, td = x.cuda(), t.cuda()
    lr, lse = ops.softcap_cross_entropy_forward(xd, td, vocab, 15.0, -1)
    lr, lse = lr.cpu(), lse.cpu()
    bad = torch.zeros(rows, dtype=torch.bool)
    bad[[2, 5]] = True
    assert torch.isnan(lr[bad]).all() and torch.isnan(lse[bad]).all()
    assert torch.isfinite(lr[~bad]).all() and torch.isfinite(lse[~bad]).all()
    good = (~bad).nonzero().flatten()
    _, rows_o, lse_o, _ = O.softcap_cross_entropy(x[good].double().numpy(), t[good].numpy(), vocab, 15.0, -1)
    np.testing.assert_allclose(lse[good].double().numpy(), lse_o, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(lr[good].double().numpy(), rows_o, rtol=2e-5, atol=2e-5)
    g = ops.softcap_cross_entropy_backward(xd, td, lse.cuda(), torch.tensor(1.0, device="cuda"), vocab, 15.0)
    g = g.float().cpu()[:, :vocab]
    assert torch.isnan(g[bad]).all()
    assert torch.isfinite(g[~bad]).all()
    assert math.isnan(softcap_cross_entropy(xd, td, vocab, 15.0, -1).item())


def test_softcap_ce_deterministic_and_scaled_gradient():
    x, t = _case(128, 2048, 2048, 2.0, seed=5)
    xd, td = x.cuda(), t.cuda()
    _, lse1 = ops.softcap_cross_entropy_forward(xd, td, 2048, 15.0)
    _, lse2 = ops.softcap_cross_entropy_forward(xd, td, 2048, 15.0)
    assert torch.equal(lse1, lse2)
    # the upstream gradient scales the logit gradient linearly
    g1 = ops.softcap_cross_entropy_backward(xd, td, lse1, torch.tensor(1.0, device="cuda"), 2048, 15.0)
    g2 = ops.softcap_cross_entropy_backward(xd, td, lse1, torch.tensor(0.25, device="cuda"), 2048, 15.0)
    assert torch.equal((g1.float() * 0.25).bfloat16(), g2)


@pytest.mark.parametrize("rows,vocab,ignore_every,expected,actual", [
    (64, 32768, 0, 1.0, 1.0),     # the trainer's vocabulary, gradient as assumed
    (37, 32768, 5, 0.25, 0.25),   # ignored rows, the graphed update's 1/4 scale
    (300, 4096, 7, 1.0, 0.3),     # one vector per thread; actual gradient differs: rescaled
    (16, 12288, 3, 0.5, -2.0),    # three vectors per thread; negative upstream gradient
])
def test_softcap_ce_fused_matches_oracle(rows, vocab, ignore_every, expected, actual):
    """The one-pass forward + backward: loss, row losses and lse against the fp64 oracle,
    and the logit gradient for the actual upstream gradient, whether or not it is the one
    the forward assumed."""
    x, t = _case(rows, vocab, vocab, 2.0, seed=rows + 3, ignore_every=ignore_every)
    loss_o, rows_o, lse_o, d_o = O.softcap_cross_entropy(x.double().numpy(), t.numpy(), vocab, 15.0, -1)
    xd, td = x.cuda().requires_grad_(), t.cuda()
    loss = softcap_cross_entropy(xd, td, vocab, 15.0, -1, expected_grad=expected)
    assert loss.grad_fn is not None and "Fused" in type(loss.grad_fn).__name__
    loss.backward(torch.tensor(actual, device="cuda"))
    assert abs(loss.item() - loss_o) <= 1e-5 * max(1.0, abs(loss_o))
    lr, lse, g, count = ops.softcap_cross_entropy_fused(xd.detach(), td, vocab, 15.0, -1, expected)
    np.testing.assert_allclose(lse.cpu().double().numpy(), lse_o, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(lr.cpu().double().numpy(), rows_o, rtol=2e-5, atol=2e-5)
    assert count.item() == float((t != -1).sum())
    assert rel_err(g.float().cpu(), expected * d_o) < 5e-3
    d = xd.grad.float().cpu()
    assert rel_err(d, actual * d_o) < 5e-3
    if ignore_every:
        assert torch.all(d[::ignore_every] == 0)
    # the two-kernel path gives the same values to rounding
    lr2, lse2 = ops.softcap_cross_entropy_forward(xd.detach(), td, vocab, 15.0, -1)
    assert torch.allclose(lse, lse2, rtol=1e-6, atol=1e-6)
    g2 = ops.softcap_cross_entropy_backward(xd.detach(), td, lse2, torch.tensor(expected, device="cuda") / count,
                                            vocab, 15.0)
    assert rel_err(g.float().cpu(), g2.float().cpu().double().numpy()) < 1e-2


def test_softcap_ce_fused_nan_row_and_fallbacks():
    """A NaN logit poisons its row's loss, lse and gradient in the one-pass kernel too; a
    second backward raises (the gradient buffer is handed out in place); shapes the kernel
    does not take (vocabulary padding, rows over 32768 columns) and forward-only calls use the
    two-kernel path."""
    rows, vocab = 8, 8192
    x, t = _case(rows, vocab, vocab, 4.0, seed=21)
    x[2, 17] = float("nan")
    xd, td = x.cuda(), t.cuda()
    lr, lse, g, _ = ops.softcap_cross_entropy_fused(xd, td, vocab, 15.0, -1, 1.0)
    lr, lse, g = lr.cpu(), lse.cpu(), g.float().cpu()
    assert math.isnan(lr[2]) and math.isnan(lse[2]) and torch.isnan(g[2]).all()
    good = torch.tensor([r for r in range(rows) if r != 2])
    assert torch.isfinite(lr[good]).all() and torch.isfinite(g[good]).all()
    _, rows_o, lse_o, _ = O.softcap_cross_entropy(x[good].double().numpy(), t[good].numpy(), vocab, 15.0, -1)
    np.testing.assert_allclose(lse[good].double().numpy(), lse_o, rtol=2e-6, atol=2e-6)
    x2, t2 = _case(4, 4096, 4096, 1.0, seed=22)
    xg = x2.cuda().requires_grad_()
    loss = softcap_cross_entropy(xg, t2.cuda(), 4096, 15.0, -1, expected_grad=1.0)
    loss.backward(retain_graph=True)
    with pytest.raises(RuntimeError):
        loss.backward()
    assert not ops.softcap_cross_entropy_fused_supported(8000, 8192)
    assert not ops.softcap_cross_entropy_fused_supported(4100, 4104)
    assert not ops.softcap_cross_entropy_fused_supported(65536, 65536)
    assert ops.softcap_cross_entropy_fused_supported(32768, 32768)
    x3, t3 = _case(4, 1000, 1024, 1.0, seed=23)
    x3d = x3.cuda().requires_grad_()
    loss = softcap_cross_entropy(x3d, t3.cuda(), 1000, 15.0, -1, expected_grad=1.0)
    assert "Fused" not in type(loss.grad_fn).__name__
    with torch.no_grad():
        loss = softcap_cross_entropy(xg, t2.cuda(), 4096, 15.0, -1, expected_grad=1.0)
    assert loss.grad_fn is None


def test_softcap_ce_rejects_bad_arguments():
    x = torch.zeros(4, 12, dtype=torch.bfloat16, device="cuda")
    t = torch.zeros(4, dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError):
        ops.softcap_cross_entropy_forward(x, t, 10, 15.0)  # stride not a multiple of 8
    with pytest.raises(RuntimeError):
        ops.softcap_cross_entropy_forward(x[:, :8], t, 10, 15.0)  # vocab > stride


@pytest.mark.parametrize("M,N,K", [
    (8192, 384, 384),   # the trainer's projections
    (8192, 1536, 384),  # MLP
    (8192, 2312, 384),  # the six fused input projections: 4 ranges of 4 blocks each
    (9000, 1536, 384),  # several blocks per range, the last range ragged
    (4097, 128, 384),   # ragged contraction
    (1000, 3, 384),     # unaligned output rows (element path)
    (777, 130, 24),     # ragged tile edges
    (64, 16, 8),        # one step, one split
])
def test_weight_grad_matches_matmul(M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    dy = torch.randn(M, N, generator=g).bfloat16()
    x = torch.randn(M, K, generator=g).bfloat16()
    exp = dy.double().T @ x.double()
    dw = ops.weight_grad(dy.cuda(), x.cuda())
    assert dw.dtype == torch.float32 and dw.shape == (N, K)
    assert rel_err(dw.cpu(), exp) < 1e-5
    assert torch.equal(dw, ops.weight_grad(dy.cuda(), x.cuda()))  # fixed-order reduction


def test_weight_grad_strided_views_and_empty():
    g = torch.Generator().manual_seed(9)
    big = torch.randn(2048, 1024, generator=g).bfloat16().cuda()
    dy, x = big[:, 8:392], big[:, 512:896]  # leading dimension 1024
    exp = dy.double().T @ x.double()
    assert rel_err(ops.weight_grad(dy, x), exp) < 1e-5
    z = ops.weight_grad(big[:0, :64], big[:0, :32])
    assert z.shape == (64, 32) and torch.all(z == 0)


def test_linear_autograd_uses_f32_weight_gradient():
    from experiment_swa_kda_amd.kda import Linear
    torch.manual_seed(0)
    lin = Linear(384, 256, bias=False).cuda()
    x = torch.randn(4, 300, 384, device="cuda").bfloat16().requires_grad_()
    y = lin(x)
    gy = torch.randn_like(y)
    y.backward(gy)
    w16 = lin.weight.detach().bfloat16().double()
    assert rel_err(lin.weight.grad, gy.double().reshape(-1, 256).T @ x.detach().double().reshape(-1, 384)) < 1e-5
    assert rel_err(x.grad, (gy.double() @ w16)) < 1e-2


def test_relu2_and_resid_mix_match_torch():
    from experiment_swa_kda_amd.model import relu2, resid_mix
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 100, 64, generator=g).bfloat16().cuda().requires_grad_()
    y = relu2(x)
    gy = torch.randn(y.shape, generator=g).bfloat16().cuda()
    y.backward(gy)
    xr = x.detach().double().requires_grad_()
    yr = torch.relu(xr).square()
    yr.backward(gy.double())
    assert rel_err(y, yr) < 4e-3 and rel_err(x.grad, xr.grad) < 4e-3

    lam_r = torch.tensor([1.1, 0.9, 1.05], device="cuda", requires_grad=True)
    lam_0 = torch.tensor([0.2, 0.1, 0.05], device="cuda", requires_grad=True)
    a = torch.randn(2, 300, 128, generator=g).bfloat16().cuda().requires_grad_()
    a0 = torch.randn(2, 300, 128, generator=g).bfloat16().cuda().requires_grad_()
    z = resid_mix(a, a0, lam_r, lam_0, 1)
    gz = torch.randn(z.shape, generator=g).bfloat16().cuda()
    z.backward(gz)
    ad, a0d = a.detach().double(), a0.detach().double()
    zr = 0.9 * ad + 0.1 * a0d
    assert rel_err(z, zr) < 4e-3
    assert rel_err(a.grad, 0.9 * gz.double()) < 4e-3 and rel_err(a0.grad, 0.1 * gz.double()) < 4e-3
    ga = float((gz.double() * ad).sum()); gb = float((gz.double() * a0d).sum())
    assert lam_r.grad[0] == 0 and lam_r.grad[2] == 0 and lam_0.grad[0] == 0
    assert abs(float(lam_r.grad[1]) - ga) < 1e-4 * max(1.0, abs(ga))
    assert abs(float(lam_0.grad[1]) - gb) < 1e-4 * max(1.0, abs(gb))


@pytest.mark.parametrize("D", [128, 384, 768])
def test_rms_norm_matches_torch(D):
    from experiment_swa_kda_amd.model import norm
    g = torch.Generator().manual_seed(D)
    x = (torch.randn(5, 77, D, generator=g) * 3).bfloat16().cuda().requires_grad_()
    y = norm(x)
    gy = torch.randn(y.shape, generator=g).bfloat16().cuda()
    y.backward(gy)
    xr = x.detach().clone().requires_grad_()
    yr = torch.nn.functional.rms_norm(xr, (D,))   # the reference's norm() on the same device
    yr.backward(gy)
    assert rel_err(y, yr) < 4e-3 and rel_err(x.grad, xr.grad) < 1e-2
    x64 = x.detach().double().requires_grad_()
    y64 = x64 * torch.rsqrt((x64 * x64).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
    y64.backward(gy.double())
    assert rel_err(y, y64) < 4e-3 and rel_err(x.grad, x64.grad) < 4e-3


@pytest.mark.parametrize("D", [384, 128])
def test_fused_mix_and_add_norms_match_separate_ops(D):
    """The residual mix fused into the following norm, and the residual add fused into its
    norm, give the values of the separate resid_mix / add / norm ops bit for bit; their
    gradients (the residual branch added inside the norm VJP, one rounding) agree with the
    separate ops' and with an f64 chain."""
    from experiment_swa_kda_amd import model as M
    g = torch.Generator().manual_seed(D + 1)
    B, T, i = 2, 65, 2
    mk = lambda s=1.0: (torch.randn(B, T, D, generator=g) * s).bfloat16().cuda().requires_grad_()
    x, x0, mixed = mk(2.0), mk(), mk(0.5)
    lam_r = (1 + 0.1 * torch.randn(4, generator=g)).cuda().requires_grad_()
    lam_0 = (0.2 * torch.randn(4, generator=g)).cuda().requires_grad_()
    gh, gh2, gy = (torch.randn(B, T, D, generator=g).bfloat16().cuda() for _ in range(3))

    def run(fused):
        leaves = [t.detach().clone().requires_grad_() for t in (x, x0, mixed, lam_r, lam_0)]
        a, a0, m, lr, l0 = leaves
        if fused:
            s, h = M._ResidMixNorm.apply(a, a0, lr, l0, i, M._RMS_EPS)
            y, h2 = M._AddNorm.apply(s, m, M._RMS_EPS)
        else:
            s = M.resid_mix(a, a0, lr, l0, i)
            h = M.norm(s)
            y = s + m
            h2 = M.norm(y)
        ((h.float() * gh.float()).sum() + (h2.float() * gh2.float()).sum() + (y.float() * gy.float()).sum()).backward()
        return (s, h, y, h2), [t.grad for t in leaves]

    (vf, gf), (vs, gs) = run(True), run(False)
    for a, b in zip(vf, vs):
        assert torch.equal(a, b)
    # f64 chain of the same function
    xd, x0d, md = (t.detach().double().requires_grad_() for t in (x, x0, mixed))
    lrd, l0d = lam_r.detach().double().requires_grad_(), lam_0.detach().double().requires_grad_()
    eps = torch.finfo(torch.float32).eps
    nrm = lambda v: v * torch.rsqrt((v * v).mean(-1, keepdim=True) + eps)
    sd = lrd[i] * xd + l0d[i] * x0d
    sd.retain_grad()
    yd = sd + md
    ((nrm(sd) * gh.double()).sum() + (nrm(yd) * gh2.double()).sum() + (yd * gy.double()).sum()).backward()
    for a, b, e in zip(gf[:3], gs[:3], (xd.grad, x0d.grad, md.grad)):
        assert rel_err(a, e) < 1e-2 and rel_err(b, e) < 1e-2
    # the lambda gradients are sums of many cancelling terms: bf16 rounding of the gradient of s
    # (2^-9 relative per term) is bounded by 2^-8 of the sum of the terms' magnitudes
    for k, (a, b, e, v) in enumerate(zip(gf[3:], gs[3:], (lrd.grad, l0d.grad), (xd, x0d))):
        scale = float((sd.grad.abs() * v.detach().abs()).sum())
        for got in (a, b):
            assert float((got.double().cpu() - e.cpu()).abs().max()) < 2 ** -8 * scale, (k, got, e, scale)


@pytest.mark.parametrize("n_tok,vocab,dim", [
    (8192, 32768, 384),   # the trainer's lookup: B2 x T4096, vocab 32768, d384
    (3000, 100, 256),     # many repeats per row, ragged last workgroup
    (5, 40, 8),           # fewer tokens than one window
    (0, 64, 16),          # no tokens: all-zero gradient
])
def test_embedding_backward_matches_index_add(n_tok, vocab, dim):
    g = torch.Generator().manual_seed(n_tok + vocab)
    idx = torch.randint(0, vocab, (n_tok,), generator=g)
    if n_tok > 10:
        idx[: n_tok // 3] = 7  # a frequent token
    dy = torch.randn(n_tok, dim, generator=g).bfloat16()
    exp = torch.zeros(vocab, dim, dtype=torch.float64).index_add_(0, idx, dy.double())
    dw = ops.embedding_backward(idx.cuda(), dy.cuda(), vocab)
    assert dw.dtype == torch.bfloat16 and dw.shape == (vocab, dim)
    # f32 sums, one bf16 rounding per element
    torch.testing.assert_close(dw.cpu().double(), exp, atol=1e-2, rtol=8e-3)
    assert torch.equal(dw, ops.embedding_backward(idx.cuda(), dy.cuda(), vocab))
    # as the gradient of the model's lookup, through autograd
    from experiment_swa_kda_amd.model import embed
    table = torch.nn.Embedding(vocab, dim).cuda().to(torch.bfloat16)
    if n_tok:
        embed(table, idx.cuda().view(1, -1)).backward(dy.cuda().view(1, n_tok, dim))
        assert torch.equal(table.weight.grad, dw)


def test_embedding_backward_ignores_out_of_range_ids():
    idx = torch.tensor([0, 5, 99, -3, 64, 5], device="cuda")
    dy = torch.ones(6, 16, dtype=torch.bfloat16, device="cuda")
    dw = ops.embedding_backward(idx, dy, 64)
    assert dw[5].float().eq(2).all() and dw[0].float().eq(1).all() and dw.float().sum() == 3 * 16


def test_softcap_ce_mean_and_count():
    rows = torch.randn(5000, device="cuda").abs()
    t = torch.randint(0, 10, (5000,), device="cuda")
    t[::4] = -1
    loss, count = ops.softcap_cross_entropy_mean(rows * (t != -1), t, -1)
    assert count.item() == float((t != -1).sum())
    exp = (rows.double() * (t != -1)).sum() / (t != -1).sum()
    assert abs(loss.item() - exp.item()) < 1e-5 * exp.item()
    loss2, _ = ops.softcap_cross_entropy_mean(rows, t, -1)
    assert torch.equal(loss2, ops.softcap_cross_entropy_mean(rows, t, -1)[0])
    allign, n0 = ops.softcap_cross_entropy_mean(rows[:10], torch.full((10,), -1, device="cuda"), -1)
    assert n0.item() == 0 and torch.isnan(allign)


def test_scalar_scale_gradient():
    from experiment_swa_kda_amd.model import scalar_scale
    g = torch.Generator().manual_seed(11)
    lam = torch.tensor([0.37], device="cuda", requires_grad=True)
    t = torch.randn(2, 4095, 1, generator=g).bfloat16().cuda().requires_grad_()
    y = scalar_scale(lam, t)
    gy = torch.randn(y.shape, generator=g).bfloat16().cuda()
    y.backward(gy)
    assert torch.equal(y, lam.detach().bfloat16() * t.detach())
    exp = (gy.double() * t.detach().double()).sum()
    assert abs(lam.grad.item() - exp.item()) < 1e-4 * max(1.0, abs(exp.item()))
    assert torch.equal(t.grad, gy * lam.detach().bfloat16())


def test_tuned_gemm_selection_loads_and_computes_the_product():
    """The committed TunableOp selection file matches this stack's validators, and a GEMM
    routed through a recorded solution (the lm_head shape) still computes x @ W^T."""
    from experiment_swa_kda_amd.model import use_tuned_gemms
    try:
        assert use_tuned_gemms()
        g = torch.Generator(device="cuda").manual_seed(0)
        x = torch.randn(8192, 384, device="cuda", generator=g).bfloat16()
        w = torch.randn(32768, 384, device="cuda", generator=g).bfloat16()
        y = torch.nn.functional.linear(x, w)
        ref = x[::97].float() @ w.float().t()
        assert rel_err(y[::97].float().cpu(), ref.cpu().double().numpy()) < 1e-2
    finally:
        torch.cuda.tunable.enable(False)
