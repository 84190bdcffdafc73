"""GPU tests of the mixer block and the all-KDA decoder on the HIP kernels."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gpt_oracle as G
from oracle import kda_oracle as O
from tests.kda_testutil import cosine, mixer_oracle_weights, np64, rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import KimiDeltaAttention, project_runtime_events, reset_project_runtime_events
    from experiment_swa_kda_amd.model import GPT, GPTConfig


def test_mixer_block_project_matches_oracle_full_layer():
    torch.manual_seed(0)
    layer = KimiDeltaAttention(256, 2, 128, mode="project_chunk").cuda()
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_((torch.randn(p.shape, generator=g) * 0.06).to(p.device))
        layer.A_log.zero_()
        layer.o_norm.weight.fill_(1.0)
    x = (torch.randn(2, 150, 256, generator=g)).cuda().bfloat16()
    reset_project_runtime_events()
    y, _ = layer(x)
    comps = {e["component"] for e in project_runtime_events()}
    assert "chunk_forward_conv_norm_gate" in comps
    w = lambda m: np64(m.weight.bfloat16())  # noqa: E731  (the block computes with bf16 weights)
    ey, _ = O.full_layer(
        np64(x), q_weight=w(layer.q_proj), k_weight=w(layer.k_proj), v_weight=w(layer.v_proj),
        q_conv_weight=np64(layer.q_conv1d.weight[:, 0].bfloat16()), k_conv_weight=np64(layer.k_conv1d.weight[:, 0].bfloat16()),
        v_conv_weight=np64(layer.v_conv1d.weight[:, 0].bfloat16()), forget_a_weight=w(layer.f_a_proj),
        forget_b_weight=w(layer.f_b_proj), beta_weight=w(layer.b_proj), A_log=np64(layer.A_log),
        dt_bias=np64(layer.dt_bias), output_gate_weight=w(layer.g_proj), norm_weight=np64(layer.o_norm.weight),
        output_weight=w(layer.o_proj), num_heads=2, norm_eps=1e-5)
    # bf16 activations between the block's GEMMs: compare at the bf16 block level
    assert rel_err(y, ey) < 3e-2, rel_err(y, ey)


def test_mixer_block_backward_matches_reference_mode():
    torch.manual_seed(1)
    layer = KimiDeltaAttention(256, 2, 128, mode="project_chunk").cuda()
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0, 0.06)
        layer.o_norm.weight.fill_(1.0)
    x = torch.randn(1, 100, 256, device="cuda").bfloat16().requires_grad_()
    y, _ = layer(x)
    y.float().square().mean().backward()
    g_proj = {n: p.grad.clone() for n, p in layer.named_parameters()}
    gx = x.grad.clone()
    layer.zero_grad()
    x.grad = None
    y2, _ = layer(x.float().detach().requires_grad_(), mode="reference")
    # the reference mode runs f32 end to end; gradients agree to bf16 precision
    y2.square().mean().backward()
    for n, p in layer.named_parameters():
        assert cosine(g_proj[n], p.grad) > 0.995, n
    assert rel_err(y, y2) < 3e-2


def test_tiny_gpt_trains_and_matches_reference_mode_logits():
    cfg = GPTConfig(sequence_len=128, vocab_size=512, n_layer=2, n_head=2, n_embd=256)
    torch.manual_seed(0)
    model = GPT(cfg).cuda()
    model.init_weights()
    with torch.no_grad():
        for b in model.transformer.h:
            b.attn.o_proj.weight.normal_(0, 0.02)
            b.mlp.c_proj.weight.normal_(0, 0.02)
    idx = torch.randint(0, 512, (2, 129), device="cuda")
    loss = model(idx[:, :-1], idx[:, 1:])
    loss.backward()
    assert torch.isfinite(loss)
    for n, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n
    with torch.no_grad():
        logits = model(idx[:, :-1])
        for b in model.transformer.h:
            b.attn.mode = "reference"
        ref = model(idx[:, :-1])
    assert rel_err(logits, ref) < 2e-2


@pytest.mark.parametrize("n_embd,n_head", [(256, 2), (384, 3)])
def test_gpt_logits_and_loss_match_oracle(n_embd, n_head):
    """The decoder's forward (smear, residual and x0 lambdas, KDA blocks, MLPs, backout,
    soft-capped head and loss) against the float64 oracle of nanochat/gpt.py:548-608, at a
    small width and at config 4's d384 / 3 heads of 128."""
    cfg = GPTConfig(sequence_len=128, vocab_size=500, n_layer=3, n_head=n_head, n_embd=n_embd)
    torch.manual_seed(1)
    model = GPT(cfg).cuda()
    model.init_weights()
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for b in model.transformer.h:
            b.attn.o_proj.weight.copy_(torch.randn(b.attn.o_proj.weight.shape, generator=g) * 0.03)
            b.mlp.c_proj.weight.copy_(torch.randn(b.mlp.c_proj.weight.shape, generator=g) * 0.03)
            b.attn.A_log.copy_(torch.randn(n_head, generator=g) * 0.3)
        model.lm_head.weight.copy_(torch.randn(model.lm_head.weight.shape, generator=g) * 0.05)
        model.resid_lambdas.copy_(1 + 0.1 * torch.randn(3, generator=g))
        model.x0_lambdas.copy_(0.2 * torch.randn(3, generator=g))
        model.smear_lambda.fill_(0.6)
        model.smear_gate.weight.copy_(torch.randn(1, 24, generator=g) * 0.3)
        model.backout_lambda.fill_(0.35)
    idx = torch.randint(0, 500, (2, 97), generator=g).cuda()  # T = 96: one full and one partial chunk
    idx[1, 40] = 499
    tg = idx[:, 1:].clone()
    tg[0, 7] = -1
    bf = lambda w: np64(w.bfloat16())  # noqa: E731
    params = dict(wte=np64(model.transformer.wte.weight), lm_head=bf(model.lm_head.weight),
                  resid_lambdas=np64(model.resid_lambdas), x0_lambdas=np64(model.x0_lambdas),
                  smear_gate=bf(model.smear_gate.weight), smear_lambda=model.smear_lambda.item(),
                  backout_lambda=model.backout_lambda.item(),
                  layers=[dict(mixer_oracle_weights(b.attn), c_fc=bf(b.mlp.c_fc.weight), c_proj=bf(b.mlp.c_proj.weight))
                          for b in model.transformer.h])
    x = idx[:, :-1].cpu().numpy()
    with torch.no_grad():
        logits = model(idx[:, :-1])
        loss = model(idx[:, :-1], tg)
    want = G.gpt_forward(x, params, vocab=500)
    assert logits.shape == want.shape
    assert rel_err(logits, want) < 3e-2, rel_err(logits, want)
    want_loss = G.gpt_forward(x, params, vocab=500, targets=tg.cpu().numpy())
    assert abs(float(loss) - want_loss) < 2e-2 * want_loss, (float(loss), want_loss)


def test_gpt_scalar_gradients_match_oracle_finite_differences():
    """d loss / d (resid_lambdas, x0_lambdas, smear_lambda, backout_lambda) of the decoder
    (autograd through the HIP residual-mix, norm, smear and backout kernels) against central
    differences of the float64 decoder oracle's loss."""
    cfg = GPTConfig(sequence_len=128, vocab_size=300, n_layer=3, n_head=2, n_embd=256)
    torch.manual_seed(3)
    model = GPT(cfg).cuda()
    model.init_weights()
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        for b in model.transformer.h:
            b.attn.o_proj.weight.copy_(torch.randn(b.attn.o_proj.weight.shape, generator=g) * 0.03)
            b.mlp.c_proj.weight.copy_(torch.randn(b.mlp.c_proj.weight.shape, generator=g) * 0.03)
        model.lm_head.weight.copy_(torch.randn(model.lm_head.weight.shape, generator=g) * 0.1)
        model.resid_lambdas.copy_(1 + 0.1 * torch.randn(3, generator=g))
        model.x0_lambdas.copy_(0.2 * torch.randn(3, generator=g))
        model.smear_lambda.fill_(0.6)
        model.smear_gate.weight.copy_(torch.randn(1, 24, generator=g) * 0.3)
        model.backout_lambda.fill_(0.35)
    idx = torch.randint(0, 300, (2, 65), generator=g).cuda()
    loss = model(idx[:, :-1], idx[:, 1:])
    loss.backward()
    got = torch.cat([model.resid_lambdas.grad, model.x0_lambdas.grad, model.smear_lambda.grad,
                     model.backout_lambda.grad]).double().cpu().numpy()
    bf = lambda w: np64(w.bfloat16())  # noqa: E731
    base = dict(wte=np64(model.transformer.wte.weight), lm_head=bf(model.lm_head.weight),
                resid_lambdas=np64(model.resid_lambdas), x0_lambdas=np64(model.x0_lambdas),
                smear_gate=bf(model.smear_gate.weight), smear_lambda=model.smear_lambda.item(),
                backout_lambda=model.backout_lambda.item(),
                layers=[dict(mixer_oracle_weights(b.attn), c_fc=bf(b.mlp.c_fc.weight), c_proj=bf(b.mlp.c_proj.weight))
                        for b in model.transformer.h])
    x, tg = idx[:, :-1].cpu().numpy(), idx[:, 1:].cpu().numpy()

    def loss_at(which, i, d):
        p = dict(base, resid_lambdas=base["resid_lambdas"].copy(), x0_lambdas=base["x0_lambdas"].copy())
        if which in ("resid_lambdas", "x0_lambdas"):
            p[which][i] += d
        else:
            p[which] += d
        return G.gpt_forward(x, p, vocab=300, targets=tg)

    h = 1e-4
    want = np.array([(loss_at(w, i, h) - loss_at(w, i, -h)) / (2 * h)
                     for w, i in [("resid_lambdas", j) for j in range(3)] + [("x0_lambdas", j) for j in range(3)]
                     + [("smear_lambda", 0), ("backout_lambda", 0)]])
    # d/d resid_lambdas[2] and d/d backout_lambda are small differences of larger inner
    # products with the middle layer's output, so the bf16 activations move them most: the
    # mixers' eager reference mode lands 7-8 % from the float64 values for these two, this
    # path 13-18 %; the rest agree to 1-3 %.  Measured: largest error 0.0027
    # against a largest gradient of 0.041 (cosine 0.9993).
    assert cosine(got, want) >= 0.995, (got, want)
    assert np.abs(got - want).max() <= 0.1 * np.abs(want).max(), (got, want)


def test_graphed_update_matches_eager_updates():
    """The captured update replays the eager update: same losses and parameters over
    several replays with fresh data copied in between (eager work between replays)."""
    from experiment_swa_kda_amd.model import GraphedUpdate, make_optimizer
    cfg = GPTConfig(sequence_len=128, vocab_size=512, n_layer=2, n_head=2, n_embd=256)
    g = torch.Generator(device="cuda").manual_seed(1)
    data = [[torch.randint(0, 512, (2, 129), device="cuda", generator=g) for _ in range(2)] for _ in range(5)]

    def fresh():
        torch.manual_seed(0)
        m = GPT(cfg).cuda()
        m.init_weights()
        with torch.no_grad():
            for b in m.transformer.h:
                b.attn.o_proj.weight.normal_(0, 0.02)
                b.mlp.c_proj.weight.normal_(0, 0.02)
        return m

    eager = fresh()
    opt_e = make_optimizer(eager, capturable=True)
    eager_losses, eager_params = [], []
    for step in range(5):
        total = 0.0
        for mb in data[step]:
            loss = eager(mb[:, :-1], mb[:, 1:]) / 2
            loss.backward()
            total += loss.item()
        opt_e.step()
        opt_e.zero_grad(set_to_none=True)
        eager_losses.append(total)
        eager_params.append([p.detach().clone() for p in eager.parameters()])

    graphed = fresh()
    opt_g = make_optimizer(graphed, capturable=True)
    static = [d.clone() for d in data[0]]
    update = GraphedUpdate(graphed, opt_g, static, warmup=2)
    # construction (warm-up updates included) leaves the model as it found it
    for p, q in zip(graphed.parameters(), fresh().parameters()):
        assert torch.equal(p, q)
    for upd in range(5):
        for i in range(2):
            static[i].copy_(data[upd][i])
        loss = update().item()
        assert abs(loss - eager_losses[upd]) < 1e-4 * abs(eager_losses[upd]), (upd, loss, eager_losses[upd])
        # every replay, not only the last, reproduces the eager parameters
        for (n, pg), pe in zip(graphed.named_parameters(), eager_params[upd]):
            assert rel_err(pg, pe) < 1e-4, (upd, n)


@pytest.mark.parametrize("inplace", [False, True])
def test_kv_cache_decode_matches_full_forward(inplace):
    """Prefill through the chunk kernels, then one-token decode steps through the recurrent
    kernel: every step's logits equal the full-sequence forward at that position."""
    from experiment_swa_kda_amd.model import KVCache
    cfg = GPTConfig(sequence_len=128, vocab_size=512, n_layer=2, n_head=2, n_embd=256)
    torch.manual_seed(0)
    model = GPT(cfg).cuda()
    model.init_weights()
    with torch.no_grad():
        for b in model.transformer.h:
            b.attn.o_proj.weight.normal_(0, 0.02)
            b.mlp.c_proj.weight.normal_(0, 0.02)
    g = torch.Generator(device="cuda").manual_seed(2)
    B, T, P = 2, 48, 37
    idx = torch.randint(0, 512, (B, T), device="cuda", generator=g)
    with torch.no_grad():
        full = model(idx)
        cache = KVCache(B, 2, T, 128, 2, "cuda", torch.bfloat16, inplace_state=inplace)
        pre = model(idx[:, :P], kv_cache=cache)
        assert cache.get_pos() == P
        assert rel_err(pre, full[:, :P]) < 2e-2
        mem = [cache.get_kda_state(i).memory for i in range(2)]
        for t in range(P, T):
            step = model(idx[:, t:t + 1], kv_cache=cache)
            assert rel_err(step[:, 0], full[:, t]) < 2e-2, t
        assert cache.get_pos() == T
        same = [cache.get_kda_state(i).memory.data_ptr() == mem[i].data_ptr() for i in range(2)]
        assert all(same) == inplace
        assert cache.state_nbytes() > 2 * B * 2 * 128 * 128 * 4


def test_kv_cache_prefill_expands_batch_one():
    from experiment_swa_kda_amd.model import KVCache
    cfg = GPTConfig(sequence_len=64, vocab_size=512, n_layer=2, n_head=2, n_embd=256)
    torch.manual_seed(0)
    model = GPT(cfg).cuda()
    model.init_weights()
    idx = torch.randint(0, 512, (1, 20), device="cuda")
    with torch.no_grad():
        one = KVCache(1, 2, 64, 128, 2, "cuda", torch.bfloat16)
        model(idx, kv_cache=one)
        many = KVCache(3, 2, 64, 128, 2, "cuda", torch.bfloat16)
        many.prefill(one)
        assert many.get_pos() == 20
        nxt = torch.randint(0, 512, (1, 1), device="cuda")
        a = model(nxt, kv_cache=one)
        b = model(nxt.expand(3, 1).contiguous(), kv_cache=many)
    for r in range(3):
        assert torch.equal(b[r], a[0])
    with pytest.raises(ValueError):
        KVCache(1, 2, 64, 128, 2, "cuda", torch.bfloat16, mixer_types="KL")
