"""Pins the numpy float64 oracle against closed forms, torch library routines,
autograd and finite differences (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kda_oracle as O


def make_inputs(B=2, T=7, H=2, K=4, V=3, seed=1729, state=True):
    r = np.random.default_rng(seed)
    d = dict(
        q=r.standard_normal((B, T, H, K)),
        k=r.standard_normal((B, T, H, K)),
        v=r.standard_normal((B, T, H, V)),
        g=r.standard_normal((B, T, H, K)),
        beta=r.standard_normal((B, T, H)),
        A_log=r.standard_normal(H) * 0.2,
        dt_bias=r.standard_normal(H * K) * 0.3,
        s0=r.standard_normal((B, H, V, K)) * 0.1 if state else None,
    )
    return d


def run_fwd(d, **kw):
    return O.kda_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                         initial_state=d["s0"], **kw)


# --- gate ------------------------------------------------------------------

def test_gate_bounded_monotone_endpoints():
    # tests/test_kda_operator.py:62-74
    raw = np.array([-100.0, -2.0, 0.0, 2.0, 100.0]).reshape(1, 1, 1, 5)
    g = O.k3_decay_gate(raw, np.array([0.3]), np.zeros(5))
    expected = -5.0 * torch.sigmoid(torch.tensor(np.exp(0.3) * raw)).numpy()
    np.testing.assert_allclose(g, expected, rtol=1e-14, atol=1e-300)
    assert np.all(g >= -5) and np.all(g <= 0)
    assert np.all(g[..., 1:] < g[..., :-1])
    assert abs(g[..., 0].item()) < 1e-12 and abs(g[..., -1].item() + 5) < 1e-12


def test_gate_backward_matches_autograd():
    r = np.random.default_rng(3)
    raw = torch.tensor(r.standard_normal((2, 3, 2, 4)), requires_grad=True)
    A = torch.tensor(r.standard_normal(2), requires_grad=True)
    b = torch.tensor(r.standard_normal(8), requires_grad=True)
    g = -5.0 * torch.sigmoid(A.exp().view(2, 1) * (raw + b.view(2, 4)))
    cot = torch.tensor(r.standard_normal(g.shape))
    ga = torch.autograd.grad(g, (raw, A, b), cot)
    gn = O.k3_decay_gate_backward(raw.detach().numpy(), A.detach().numpy(), b.detach().numpy(), -5.0, cot.numpy())
    for a, n in zip(ga, gn):
        np.testing.assert_allclose(n, a.numpy(), rtol=1e-12, atol=1e-12)


# --- recurrence closed forms (tests/test_kda_operator.py:77-137) ------------

def test_one_token_zero_state_closed_form():
    d = make_inputs(B=1, T=1, H=2, K=4, V=3, state=False)
    o, s = run_fwd(d)
    key = d["k"][:, 0] / np.linalg.norm(d["k"][:, 0], axis=-1, keepdims=True)
    beta = 1 / (1 + np.exp(-d["beta"][:, 0]))
    exp_state = np.einsum("bhk,bhv->bhvk", beta[..., None] * key, d["v"][:, 0])
    query = d["q"][:, 0] / np.linalg.norm(d["q"][:, 0], axis=-1, keepdims=True) * 0.5
    np.testing.assert_allclose(s, exp_state, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(o[:, 0], np.einsum("bhk,bhvk->bhv", query, exp_state), rtol=1e-12, atol=1e-12)


def test_exact_key_overwrites_orthogonal_survives():
    state = np.zeros((1, 1, 2, 2))
    state[0, 0, :, 0] = [3.0, -1.0]
    q = np.array([[[[1.0, 0.0]], [[0.0, 1.0]]]])
    v = np.array([[[[5.0, 7.0]], [[11.0, 13.0]]]])
    o, s = O.kda_forward(q, q.copy(), v, np.full_like(q, -100.0), np.full((1, 2, 1), 100.0),
                         np.zeros(1), np.zeros(2), initial_state=state)
    np.testing.assert_allclose(s[0, 0, :, 0], v[0, 0, 0], atol=1e-8)
    np.testing.assert_allclose(s[0, 0, :, 1], v[0, 1, 0], atol=1e-8)


def test_decay_before_delta_scalar():
    one = np.ones((1, 1, 1, 1))
    o, s = O.kda_forward(one, one, one * 10, one * 0, np.zeros((1, 1, 1)), np.zeros(1), np.zeros(1),
                         initial_state=one * 2)
    dec = 2 * np.exp(-2.5)
    exp = dec + 0.5 * (10 - dec)
    assert s.item() == pytest.approx(exp, abs=1e-14)
    assert o.item() == pytest.approx(exp, abs=1e-14)


def test_causal_prefix_and_batch_independence():
    d = make_inputs(state=False)
    full, _ = run_fwd(d)
    p = {n: (a[:, :4] if n in ("q", "k", "v", "g", "beta") else a) for n, a in d.items()}
    short, _ = run_fwd(p)
    np.testing.assert_allclose(full[:, :4], short, rtol=1e-13, atol=1e-13)
    for b in range(2):
        single = {n: (a[b:b + 1] if n in ("q", "k", "v", "g", "beta") else a) for n, a in d.items()}
        o, _ = run_fwd(single)
        np.testing.assert_allclose(full[b:b + 1], o, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("gate_mode", ["k3", "logdecay"])
@pytest.mark.parametrize("T,chunk", [(1, 4), (7, 4), (33, 16), (64, 64), (130, 64)])
def test_chunked_wy_equals_token_loop(T, chunk, gate_mode):
    d = make_inputs(B=2, T=T, H=2, K=8, V=5, seed=T)
    if gate_mode == "logdecay":
        d["g"] = -np.log1p(np.exp(d["g"] * 2))  # -softplus, unbounded below
    a = run_fwd(d, gate_mode=gate_mode)
    b = O.kda_forward_chunked(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                              initial_state=d["s0"], gate_mode=gate_mode, chunk=chunk)
    np.testing.assert_allclose(b[0], a[0], rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(b[1], a[1], rtol=1e-10, atol=1e-11)


# --- backward: torch.autograd and finite differences -----------------------

def torch_loop(q, k, v, g, beta, A_log, dt_bias, s0, gate_mode, scale=None):
    K = q.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    qn = F.normalize(q, dim=-1) * scale
    kn = F.normalize(k, dim=-1)
    H = q.shape[2]
    if gate_mode == "k3":
        dec = -5.0 * torch.sigmoid(A_log.exp().view(H, 1) * (g + dt_bias.view(H, K)))
    else:
        dec = g
    b = beta.sigmoid()
    S = s0.transpose(-1, -2)
    outs = []
    for t in range(q.shape[1]):
        S = S * dec[:, t].exp().unsqueeze(-1)
        r = v[:, t] - torch.einsum("bhk,bhkv->bhv", kn[:, t], S)
        S = S + torch.einsum("bhk,bhv->bhkv", b[:, t].unsqueeze(-1) * kn[:, t], r)
        outs.append(torch.einsum("bhk,bhkv->bhv", qn[:, t], S))
    return torch.stack(outs, 1), S.transpose(-1, -2)


@pytest.mark.parametrize("gate_mode", ["k3", "logdecay"])
@pytest.mark.parametrize("ckpt", [3, 64])
def test_backward_matches_autograd(gate_mode, ckpt):
    d = make_inputs(B=2, T=9, H=2, K=4, V=3, seed=11)
    names = ["q", "k", "v", "g", "beta", "A_log", "dt_bias", "s0"]
    tt = {n: torch.tensor(d[n], requires_grad=True) for n in names}
    o, s = torch_loop(*(tt[n] for n in names), gate_mode)
    r = np.random.default_rng(5)
    do = r.standard_normal(o.shape)
    ds = r.standard_normal(s.shape)
    grads = torch.autograd.grad((o, s), [tt[n] for n in names], (torch.tensor(do), torch.tensor(ds)), allow_unused=True)
    mine = O.kda_backward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                          initial_state=d["s0"], grad_output=do, grad_final_state=ds,
                          gate_mode=gate_mode, checkpoint=ckpt)
    order = [0, 1, 2, 3, 4, 5, 6, 7]
    for n, i, gt in zip(names, order, grads):
        if mine[i] is None:
            assert gate_mode == "logdecay" and n in ("A_log", "dt_bias")
            continue
        np.testing.assert_allclose(np.asarray(mine[i]).reshape(gt.shape), gt.numpy(), rtol=1e-10, atol=1e-11,
                                   err_msg=n)


def test_backward_matches_finite_differences():
    d = make_inputs(B=1, T=5, H=1, K=3, V=2, seed=2)
    r = np.random.default_rng(8)
    do = r.standard_normal((1, 5, 1, 2))
    ds = r.standard_normal((1, 1, 2, 3))

    def loss(dd):
        o, s = run_fwd(dd)
        return (o * do).sum() + (s * ds).sum()

    g = O.kda_backward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                       initial_state=d["s0"], grad_output=do, grad_final_state=ds)
    for idx, n in enumerate(["q", "k", "v", "g", "beta", "A_log", "dt_bias", "s0"]):
        arr = d[n]
        flat = arr.reshape(-1)
        for j in range(0, flat.size, max(1, flat.size // 5)):
            e = 1e-6
            dp = {m: (a.copy() if a is not None else None) for m, a in d.items()}
            dm = {m: (a.copy() if a is not None else None) for m, a in d.items()}
            dp[n].reshape(-1)[j] += e
            dm[n].reshape(-1)[j] -= e
            fd = (loss(dp) - loss(dm)) / (2 * e)
            assert np.asarray(g[idx]).reshape(-1)[j] == pytest.approx(fd, rel=1e-5, abs=1e-7), n


def test_varlen_equals_separate_sequences():
    d = make_inputs(B=1, T=20, H=2, K=4, V=3, state=False)
    cu = [0, 5, 6, 20]
    o, s = O.kda_varlen_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], cu)
    for i in range(3):
        a, b = cu[i], cu[i + 1]
        oo, ss = O.kda_forward(d["q"][:, a:b], d["k"][:, a:b], d["v"][:, a:b], d["g"][:, a:b],
                               d["beta"][:, a:b], d["A_log"], d["dt_bias"])
        np.testing.assert_array_equal(o[:, a:b], oo)
        np.testing.assert_array_equal(s[i:i + 1], ss)
    # state reset: sequence 2 differs from the continuation of sequence 1
    cont, _ = O.kda_forward(d["q"][:, :20], d["k"][:, :20], d["v"][:, :20], d["g"][:, :20],
                            d["beta"][:, :20], d["A_log"], d["dt_bias"])
    assert not np.allclose(cont[:, 6:], o[:, 6:])


# --- conv -------------------------------------------------------------------

def test_conv_matches_torch_conv1d_and_autograd():
    r = np.random.default_rng(99)
    x = torch.tensor(r.standard_normal((2, 9, 6)), requires_grad=True)
    w = torch.tensor(r.standard_normal((6, 4)), requires_grad=True)
    st = torch.tensor(r.standard_normal((2, 6, 4)), requires_grad=True)
    inp = torch.cat((st[..., 1:], x.transpose(1, 2)), dim=-1)
    y = F.silu(F.conv1d(inp, w.unsqueeze(1), groups=6)).transpose(1, 2)
    fin = inp[..., -4:]
    mine_y, mine_fin = O.causal_conv_forward(x.detach().numpy(), w.detach().numpy(), st.detach().numpy())
    np.testing.assert_allclose(mine_y, y.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mine_fin, fin.detach().numpy(), rtol=0, atol=0)
    dy = r.standard_normal(y.shape)
    dfin = r.standard_normal(fin.shape)
    ga = torch.autograd.grad((y, fin), (x, w, st), (torch.tensor(dy), torch.tensor(dfin)))
    gm = O.causal_conv_backward(x.detach().numpy(), w.detach().numpy(), dy, st.detach().numpy(), dfin)
    for a, m in zip(ga, gm):
        np.testing.assert_allclose(m, a.numpy(), rtol=1e-11, atol=1e-11)


def test_conv_full_sequence_matches_decode():
    r = np.random.default_rng(4)
    x = r.standard_normal((2, 9, 6))
    w = r.standard_normal((6, 4))
    full, fs = O.causal_conv_forward(x, w)
    st = None
    pieces = []
    for t in range(9):
        p, st = O.causal_conv_forward(x[:, t:t + 1], w, st)
        pieces.append(p)
    np.testing.assert_allclose(np.concatenate(pieces, 1), full, rtol=1e-13, atol=1e-13)
    np.testing.assert_array_equal(st, fs)


# --- rmsnorm gate -----------------------------------------------------------

def test_rmsnorm_gate_matches_torch():
    r = np.random.default_rng(6)
    x = torch.tensor(r.standard_normal((3, 5, 16)), requires_grad=True)
    gt = torch.tensor(r.standard_normal((3, 5, 16)), requires_grad=True)
    w = torch.tensor(r.standard_normal(16), requires_grad=True)
    y = F.rms_norm(x, (16,), weight=w, eps=1e-5) * gt.sigmoid()
    my, inv = O.rmsnorm_gate_forward(x.detach().numpy(), gt.detach().numpy(), w.detach().numpy(), 1e-5)
    np.testing.assert_allclose(my, y.detach().numpy(), rtol=1e-12, atol=1e-12)
    dy = r.standard_normal(y.shape)
    ga = torch.autograd.grad(y, (x, gt, w), torch.tensor(dy))
    gm = O.rmsnorm_gate_backward(x.detach().numpy(), gt.detach().numpy(), w.detach().numpy(), 1e-5, dy)
    for a, m in zip(ga, gm):
        np.testing.assert_allclose(m, a.numpy(), rtol=1e-11, atol=1e-11)


# --- soft-capped cross entropy ------------------------------------------------

def test_softcap_cross_entropy_matches_torch():
    g = torch.Generator().manual_seed(11)
    rows, vocab, stride = 37, 50, 56
    x = (torch.randn(rows, stride, generator=g, dtype=torch.float64) * 20).requires_grad_()
    t = torch.randint(0, vocab, (rows,), generator=g)
    t[::5] = -1
    z = 15.0 * torch.tanh(x[:, :vocab] / 15.0)
    ref = F.cross_entropy(z, t, ignore_index=-1)
    ref.backward()
    loss, loss_rows, lse, d = O.softcap_cross_entropy(x.detach().numpy(), t.numpy(), vocab, 15.0, -1)
    assert abs(loss - ref.item()) < 1e-12
    np.testing.assert_allclose(d, x.grad.numpy(), rtol=0, atol=1e-14)
    assert np.all(d[:, vocab:] == 0) and np.all(d[::5] == 0)
    np.testing.assert_allclose(lse, torch.logsumexp(z, -1).detach().numpy(), rtol=1e-13)
    assert np.all(loss_rows[::5] == 0)


def test_softcap_cross_entropy_uniform_closed_form():
    # equal logits: every row's loss is log(vocab), the gradient (1/vocab - onehot) / rows
    rows, vocab = 4, 10
    x = np.full((rows, vocab), 3.0)
    t = np.array([0, 3, 9, 2])
    loss, _, _, d = O.softcap_cross_entropy(x, t, vocab, 15.0)
    assert abs(loss - np.log(vocab)) < 1e-13
    sech2 = 1.0 - np.tanh(3.0 / 15.0) ** 2
    exp = np.full((rows, vocab), 1.0 / vocab)
    exp[np.arange(rows), t] -= 1.0
    np.testing.assert_allclose(d, exp / rows * sech2, atol=1e-15)


def test_varlen_empty_sequence_passes_state_and_gradient_through():
    """An empty packed sequence leaves the others unchanged; its final state is its initial
    state and its state gradient is the final-state gradient (closed form)."""
    r = np.random.default_rng(11)
    T, H, K, V = 12, 1, 8, 8
    q, k, g = (r.standard_normal((1, T, H, K)) for _ in range(3))
    v = r.standard_normal((1, T, H, V))
    b = r.standard_normal((1, T, H))
    A, dt = np.zeros(H), np.zeros(H * K)
    s0, gS = r.standard_normal((3, H, V, K)), r.standard_normal((3, H, V, K))
    do = r.standard_normal((1, T, H, V))
    o3, f3 = O.kda_varlen_forward(q, k, v, g, b, A, dt, [0, 5, 5, 12], initial_state=s0)
    o2, f2 = O.kda_varlen_forward(q, k, v, g, b, A, dt, [0, 5, 12], initial_state=s0[[0, 2]])
    np.testing.assert_array_equal(o3, o2)
    np.testing.assert_array_equal(f3[1], s0[1])
    np.testing.assert_array_equal(f3[[0, 2]], f2)
    g3 = O.kda_varlen_backward(q, k, v, g, b, A, dt, [0, 5, 5, 12], grad_output=do, grad_final_state=gS,
                               initial_state=s0)
    g2 = O.kda_varlen_backward(q, k, v, g, b, A, dt, [0, 5, 12], grad_output=do, grad_final_state=gS[[0, 2]],
                               initial_state=s0[[0, 2]])
    for a3, a2 in zip(g3[:7], g2[:7]):
        np.testing.assert_allclose(a3, a2, rtol=0, atol=1e-12)
    np.testing.assert_array_equal(g3[7][1], gS[1])
    np.testing.assert_allclose(g3[7][[0, 2]], g2[7], rtol=0, atol=1e-12)


def _layer_weights(layer):
    w = lambda m: m.weight.detach().double().numpy()  # noqa: E731
    return dict(q_weight=w(layer.q_proj), k_weight=w(layer.k_proj), v_weight=w(layer.v_proj),
                q_conv_weight=layer.q_conv1d.weight[:, 0].detach().double().numpy(),
                k_conv_weight=layer.k_conv1d.weight[:, 0].detach().double().numpy(),
                v_conv_weight=layer.v_conv1d.weight[:, 0].detach().double().numpy(),
                forget_a_weight=w(layer.f_a_proj), forget_b_weight=w(layer.f_b_proj),
                beta_weight=w(layer.b_proj), A_log=layer.A_log.detach().double().numpy(),
                dt_bias=layer.dt_bias.detach().double().numpy(),
                output_gate_weight=w(layer.g_proj), norm_weight=w(layer.o_norm),
                output_weight=w(layer.o_proj), num_heads=layer.num_heads, norm_eps=layer.o_norm.eps)


def test_full_layer_backward_matches_autograd_and_finite_differences():
    """The oracle's mixer-block VJP against (1) torch autograd through the package's eager
    reference mode, an independent statement of the block, and (2) central finite
    differences of ``full_layer`` for single entries of several parameters."""
    from experiment_swa_kda_amd.kda import KimiDeltaAttention

    torch.manual_seed(0)
    layer = KimiDeltaAttention(16, 2, 8, mode="reference")
    gen = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.3)
        layer.A_log.copy_(torch.tensor([-0.3, 0.2]))
    x = torch.randn(2, 11, 16, generator=gen, dtype=torch.float64)
    gy = torch.randn(2, 11, 16, generator=gen, dtype=torch.float64)
    wts = _layer_weights(layer)
    got = O.full_layer_backward(x.numpy(), gy.numpy(), **wts)

    xr = x.clone().requires_grad_()
    y, _ = layer(xr, mode="reference")
    (y * gy).sum().backward()
    ref = {"x": xr.grad}
    for name, mod in (("q_proj", layer.q_proj), ("k_proj", layer.k_proj), ("v_proj", layer.v_proj),
                      ("g_proj", layer.g_proj), ("f_a_proj", layer.f_a_proj), ("f_b_proj", layer.f_b_proj),
                      ("b_proj", layer.b_proj), ("o_proj", layer.o_proj), ("o_norm", layer.o_norm)):
        ref[name] = mod.weight.grad
    for name in ("q_conv1d", "k_conv1d", "v_conv1d"):
        ref[name] = getattr(layer, name).weight.grad[:, 0]
    ref["A_log"], ref["dt_bias"] = layer.A_log.grad, layer.dt_bias.grad
    assert set(ref) == set(got)
    for name, r in ref.items():
        r = r.double().numpy()
        assert got[name].shape == r.shape, name
        # the reference mode runs the recurrence in f32
        assert np.linalg.norm(got[name] - r) <= 1e-4 * np.linalg.norm(r), name

    def loss(w):
        out, _ = O.full_layer(x.numpy(), **w)
        return float((out * gy.numpy()).sum())

    for key, grad_key, idx in (("q_conv_weight", "q_conv1d", (3, 1)), ("A_log", "A_log", (1,)),
                               ("forget_b_weight", "f_b_proj", (5, 2)), ("norm_weight", "o_norm", (4,)),
                               ("v_weight", "v_proj", (7, 9))):
        h = 1e-6
        wp, wm = dict(wts), dict(wts)
        wp[key] = wts[key].copy()
        wm[key] = wts[key].copy()
        wp[key][idx] += h
        wm[key][idx] -= h
        fd = (loss(wp) - loss(wm)) / (2 * h)
        assert abs(fd - got[grad_key][idx]) <= 1e-6 * max(1.0, abs(fd)), key


def test_cpu_baseline_path_matches_oracle():
    """The timed CPU baseline computes the same operator as the oracle."""
    from oracle.reference_path import reference_kda_cpu

    g = torch.Generator().manual_seed(3)
    q, k, z = (torch.randn(2, 9, 2, 8, generator=g) for _ in range(3))
    v = torch.randn(2, 9, 2, 6, generator=g)
    bl = torch.randn(2, 9, 2, generator=g)
    A, dt = torch.randn(2, generator=g) * 0.2, torch.randn(16, generator=g) * 0.3
    s0 = torch.randn(2, 2, 6, 8, generator=g) * 0.1
    o, s = reference_kda_cpu(q, k, v, z, bl, A, dt, initial_state=s0)
    eo, es = O.kda_forward(*(t.double().numpy() for t in (q, k, v, z, bl, A, dt)), initial_state=s0.double().numpy())
    np.testing.assert_allclose(o.double().numpy(), eo, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(s.double().numpy(), es, atol=1e-5, rtol=1e-5)
