"""BASELINE config 4 on the GPU: the KDA mixer block at model width 384 against the float64
oracle (forward and every gradient), and the 6-layer all-KDA decoder at its benchmark
workload (vocab 32768, B2 T4096, 4 accumulation micro-steps, seed 42) trained eagerly and
as a replayed HIP graph (nanochat/gpt.py:543-608, scripts/base_train.py:467-633)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import kda_oracle as O
from tests.kda_testutil import cosine, mixer_oracle_weights, np64, rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import KimiDeltaAttention
    from experiment_swa_kda_amd.model import GPT, GPTConfig, GraphedUpdate, make_optimizer


def test_mixer_block_d384_forward_and_gradients_match_oracle():
    torch.manual_seed(0)
    layer = KimiDeltaAttention(384, 3, 128, mode="project_chunk").cuda()
    g = torch.Generator().manual_seed(42)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.05).to(p.device))
        layer.A_log.copy_(torch.tensor([-0.5, 0.0, 0.4]))
        layer.o_norm.weight.copy_(1 + 0.1 * torch.randn(128, generator=g))
    x = torch.randn(1, 512, 384, generator=g).bfloat16().cuda().requires_grad_()
    gy = torch.randn(1, 512, 384, generator=g).bfloat16().cuda()
    y, _ = layer(x)
    y.backward(gy)
    wts = mixer_oracle_weights(layer)
    ey, _ = O.full_layer(np64(x), **wts)
    assert rel_err(y, ey) < 2e-2, rel_err(y, ey)
    eg = O.full_layer_backward(np64(x), np64(gy), **wts)
    got = {"x": x.grad}
    for name in ("q_proj", "k_proj", "v_proj", "g_proj", "f_a_proj", "f_b_proj", "b_proj", "o_proj", "o_norm"):
        got[name] = getattr(layer, name).weight.grad
    for name in ("q_conv1d", "k_conv1d", "v_conv1d"):
        got[name] = getattr(layer, name).weight.grad[:, 0]
    got["A_log"], got["dt_bias"] = layer.A_log.grad, layer.dt_bias.grad
    assert set(got) == set(eg)
    bad = {n: cosine(got[n], eg[n]) for n in got if not cosine(got[n], eg[n]) >= 0.9999}
    assert not bad, bad


def _model():
    torch.manual_seed(42)
    cfg = GPTConfig(sequence_len=4096, vocab_size=32768, n_layer=6, n_head=3, n_embd=384)
    m = GPT(cfg).cuda()
    m.init_weights()
    return m


def test_config4_six_layer_update_eager_and_graphed():
    B, T, accum, V = 2, 4096, 4, 32768
    g = torch.Generator(device="cuda").manual_seed(42)
    data = [torch.randint(0, V, (B, T + 1), device="cuda", generator=g) for _ in range(accum)]

    eager = _model()
    opt = make_optimizer(eager, capturable=True)
    eager_losses, eager_params = [], []
    for upd in range(2):  # the same four micro-batches twice: the second loss must be lower
        total = 0.0
        for mb in data:
            loss = eager(mb[:, :-1], mb[:, 1:]) / accum
            loss.backward()
            total += loss.item()
        if upd == 0:
            assert abs(total - math.log(V)) < 0.05, total  # near-uniform logits at init
            for n, p in eager.named_parameters():
                assert p.grad is not None and torch.isfinite(p.grad).all(), n
            assert eager.lm_head.weight.grad.abs().sum() > 0
        opt.step()
        opt.zero_grad(set_to_none=True)
        eager_losses.append(total)
        eager_params.append([p.detach().clone() for p in eager.parameters()])
    assert eager_losses[1] < eager_losses[0], eager_losses

    graphed = _model()
    opt_g = make_optimizer(graphed, capturable=True)
    static = [d.clone() for d in data]
    update = GraphedUpdate(graphed, opt_g, static, warmup=2)
    for upd in range(2):
        loss = update().item()
        assert abs(loss - eager_losses[upd]) <= 1e-4 * eager_losses[upd], (upd, loss, eager_losses[upd])
        for (n, pg), pe in zip(graphed.named_parameters(), eager_params[upd]):
            assert torch.isfinite(pg).all(), n
            assert rel_err(pg, pe) < 1e-4, (upd, n)
