"""Pins of the decoder oracle (oracle/gpt_oracle.py, nanochat/gpt.py:548-608) on the CPU:
closed forms and properties a wrong index, sign or term would break, and the same
composition written with torch.nn.functional ops."""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import gpt_oracle as G
from oracle import kda_oracle as O

D, H, VOCAB, VP = 32, 2, 40, 64


def _params(rng, n_layer, zero_blocks=False):
    K = D // H
    layers = []
    for _ in range(n_layer):
        w = lambda *s: rng.standard_normal(s) * 0.2  # noqa: E731
        layers.append(dict(
            q_weight=w(D, D), k_weight=w(D, D), v_weight=w(D, D),
            q_conv_weight=w(D, 4), k_conv_weight=w(D, 4), v_conv_weight=w(D, 4),
            forget_a_weight=w(K, D), forget_b_weight=w(D, K), beta_weight=w(H, D),
            A_log=rng.standard_normal(H) * 0.3, dt_bias=rng.standard_normal(D) * 0.3,
            output_gate_weight=w(D, D), norm_weight=1 + 0.1 * rng.standard_normal(K),
            output_weight=np.zeros((D, D)) if zero_blocks else w(D, D), num_heads=H, norm_eps=1e-5,
            c_fc=w(4 * D, D), c_proj=np.zeros((D, 4 * D)) if zero_blocks else w(D, 4 * D)))
    return dict(wte=rng.standard_normal((VP, D)), lm_head=rng.standard_normal((VP, D)) * 0.3,
                resid_lambdas=1 + 0.2 * rng.standard_normal(n_layer), x0_lambdas=0.3 * rng.standard_normal(n_layer),
                smear_gate=rng.standard_normal((1, 24)), smear_lambda=0.7, backout_lambda=0.3, layers=layers)


def test_causal_prefix():
    rng = np.random.default_rng(0)
    p = _params(rng, 3)
    idx = rng.integers(0, VOCAB, (2, 9))
    full = G.gpt_forward(idx, p, vocab=VOCAB)
    for t in (2, 5):
        np.testing.assert_allclose(G.gpt_forward(idx[:, :t], p, vocab=VOCAB), full[:, :t], rtol=1e-10, atol=1e-12)


def test_backout_of_the_middle_layer_cancels_the_residual():
    # n_layer 2: the cached residual is the last layer's output (index n_layer // 2 = 1);
    # with zero blocks and backout_lambda 1 the head sees norm(0) = 0: logits 0, loss ln V
    rng = np.random.default_rng(1)
    p = _params(rng, 2, zero_blocks=True)
    p["backout_lambda"] = 1.0
    idx = rng.integers(0, VOCAB, (2, 6))
    assert np.abs(G.gpt_forward(idx, p, vocab=VOCAB)).max() < 1e-12
    loss = G.gpt_forward(idx, p, vocab=VOCAB, targets=rng.integers(0, VOCAB, (2, 6)))
    assert abs(loss - math.log(VOCAB)) < 1e-12
    # cached one layer earlier or later it would not cancel
    p3 = _params(rng, 3, zero_blocks=True)
    p3["backout_lambda"] = 1.0
    assert np.abs(G.gpt_forward(idx, p3, vocab=VOCAB)).max() > 1e-3


def test_zero_block_trunk_closed_form():
    # zero blocks: x_{i+1} = r_i x_i + a_i x0, so x_n = alpha_n x0 and the head sees
    # norm((alpha_n - b alpha_{mid+1}) x0) (the epsilon makes the norm depend on the scale)
    rng = np.random.default_rng(2)
    p = _params(rng, 4, zero_blocks=True)
    idx = rng.integers(0, VOCAB, (2, 7))
    x0 = G.smear(G.rms_norm(p["wte"][idx]), p["smear_gate"], p["smear_lambda"])
    for b in (0.3, 5.0):
        p["backout_lambda"] = b
        alpha, a_mid = 1.0, None
        for i in range(4):
            alpha = p["resid_lambdas"][i] * alpha + p["x0_lambdas"][i]
            a_mid = alpha if i == 2 else a_mid
        c = alpha - b * a_mid
        want = 15 * np.tanh(G.rms_norm(c * x0) @ p["lm_head"].T[:, :VOCAB] / 15)
        np.testing.assert_allclose(G.gpt_forward(idx, p, vocab=VOCAB), want, rtol=1e-12, atol=1e-12)


def test_smear_reaches_only_the_next_position():
    rng = np.random.default_rng(3)
    p = _params(rng, 1, zero_blocks=True)
    p["x0_lambdas"][:] = 0.0
    idx = rng.integers(0, VOCAB, (1, 8))
    idx2 = idx.copy()
    idx2[0, 3] = (idx[0, 3] + 1) % VOCAB
    a, b = G.gpt_forward(idx, p, vocab=VOCAB), G.gpt_forward(idx2, p, vocab=VOCAB)
    changed = np.abs(a - b).max(-1)[0]
    assert changed[3] > 1e-6 and changed[4] > 1e-6
    assert changed[:3].max() == 0 and changed[5:].max() < 1e-12
    p["smear_lambda"] = 0.0
    a, b = G.gpt_forward(idx, p, vocab=VOCAB), G.gpt_forward(idx2, p, vocab=VOCAB)
    assert np.abs(a - b).max(-1)[0][4] < 1e-12


def _torch_forward(idx, p, targets=None):
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))  # noqa: E731
    nrm = lambda x: F.rms_norm(x, (x.shape[-1],), eps=torch.finfo(torch.float32).eps)  # noqa: E731
    x = nrm(t(p["wte"])[torch.as_tensor(idx)])
    gate = p["smear_lambda"] * torch.sigmoid(x[:, 1:, :24] @ t(p["smear_gate"]).T)
    x = torch.cat([x[:, :1], x[:, 1:] + gate * x[:, :-1]], dim=1)
    x0, mid, xm = x, len(p["layers"]) // 2, None
    for i, layer in enumerate(p["layers"]):
        x = float(p["resid_lambdas"][i]) * x + float(p["x0_lambdas"][i]) * x0
        args = {k: v for k, v in layer.items() if k not in ("c_fc", "c_proj")}
        x = x + t(O.full_layer(nrm(x).numpy(), **args)[0])
        x = x + F.relu(nrm(x) @ t(layer["c_fc"]).T).square() @ t(layer["c_proj"]).T
        xm = x if i == mid else xm
    x = nrm(x - p["backout_lambda"] * xm)
    logits = 15 * torch.tanh((x @ t(p["lm_head"]).T)[..., :VOCAB] / 15)
    if targets is None:
        return logits.numpy()
    return F.cross_entropy(logits.reshape(-1, VOCAB), torch.as_tensor(targets).reshape(-1), ignore_index=-1).item()


def test_matches_torch_functional_composition():
    rng = np.random.default_rng(4)
    p = _params(rng, 3)
    idx = rng.integers(0, VOCAB, (2, 9))
    tg = rng.integers(0, VOCAB, (2, 9))
    tg[0, 2] = -1
    np.testing.assert_allclose(G.gpt_forward(idx, p, vocab=VOCAB), _torch_forward(idx, p), rtol=1e-9, atol=1e-9)
    assert abs(G.gpt_forward(idx, p, vocab=VOCAB, targets=tg) - _torch_forward(idx, p, tg)) < 1e-9
