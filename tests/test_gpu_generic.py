"""GPU parity of the head dims other than 64 / 128 against the float64 oracle: the
zero-padded chunked route (K, V <= 128) and the token-serial kernels (larger K or V):
forward, backward, packed sequences, decode, the norm-gate kernels and the mixer paths that
route to them.  The reference takes any head dim through its generic lane
(nanochat/mixers/cuda_kda/chunk.cu:135-213, :578-870)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as O
from tests.kda_testutil import cosine, make_kda_inputs, np64, rel_err
from tests.test_gpu_backward import check, cotangents, gpu_grads, oracle_grads

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import kda, ops

# K, V <= 128 take the zero-padded chunked route: (16, 16), (32, 48), (96, 96), (128, 96), (7, 5).
# The rest take the token-serial kernels, one pair per keys-per-lane instance (K <= 16, 32,
# 64, 128, 256), with V not a multiple of 16 (partial column groups): (16, 136), (32, 144),
# (64, 200), (100, 130), (200, 40), (256, 64).
SHAPES = [(16, 16), (32, 48), (96, 96), (128, 96), (7, 5),
          (16, 136), (32, 144), (64, 200), (100, 130), (200, 40), (256, 64)]


def oracle_fwd(d, gate):
    return O.kda_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                         np64(d["A_log"]), np64(d["dt_bias"]), initial_state=np64(d["s0"]),
                         gate_mode="k3" if gate == "k3" else "logdecay")


def run_fwd(d, gate, cu=None):
    K = d["q"].shape[-1]
    out, fin, _ = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                    d["s0"], True, -5.0, K ** -0.5, cu_seqlens=cu, gate=gate)
    return out, fin


@pytest.mark.parametrize("KV", SHAPES)
@pytest.mark.parametrize("T", [1, 15, 16, 17, 50])
def test_generic_forward(KV, T):
    K, V = KV
    print(f"generic forward K={K} V={V} T={T}", flush=True)
    d = make_kda_inputs(2, T, 2, K, V, seed=K * 1000 + V + T, state=True)
    out, fin = run_fwd(d, "k3")
    eo, ef = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 2e-2, rel_err(out, eo)
    assert rel_err(fin, ef) < 2e-2, rel_err(fin, ef)
    torch.testing.assert_close(out.double().cpu(), torch.tensor(eo), atol=5e-3, rtol=5e-3)


@pytest.mark.parametrize("KV", [(32, 48), (96, 96), (256, 64)])
def test_generic_forward_precomputed_gate_no_state(KV):
    K, V = KV
    d = make_kda_inputs(1, 70, 3, K, V, seed=K + V, gate="precomputed", dist="baseline")
    out, fin = run_fwd(d, "precomputed")
    eo, ef = oracle_fwd(d, "precomputed")
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2


def test_generic_forward_deterministic():
    d = make_kda_inputs(2, 90, 2, 96, 80, seed=5, state=True)
    a, fa = run_fwd(d, "k3")
    b, fb = run_fwd(d, "k3")
    assert torch.equal(a, b) and torch.equal(fa, fb)


@pytest.mark.parametrize("KV", SHAPES)
@pytest.mark.parametrize("T", [1, 16, 33])
def test_generic_backward(KV, T):
    K, V = KV
    print(f"generic backward K={K} V={V} T={T}", flush=True)
    d = make_kda_inputs(2, T, 2, K, V, seed=7 * K + V + T, state=True)
    do, dsT = cotangents(d, 50 + T)
    check(gpu_grads(d, "k3", do, dsT), oracle_grads(d, "k3", do, dsT))


@pytest.mark.parametrize("KV", [(32, 48), (96, 96), (200, 40)])
def test_generic_backward_precomputed_gate(KV):
    K, V = KV
    d = make_kda_inputs(1, 70, 3, K, V, seed=K * 3 + V, gate="precomputed", state=True, dist="baseline")
    do, dsT = cotangents(d, 9)
    check(gpu_grads(d, "precomputed", do, dsT), oracle_grads(d, "precomputed", do, dsT))


def test_generic_backward_long_sequence():
    # many 16-token blocks and sub-blocks (K = 256 recomputes 4-token sub-blocks)
    d = make_kda_inputs(1, 300, 2, 256, 48, seed=77, state=True)
    do, dsT = cotangents(d, 78)
    check(gpu_grads(d, "k3", do, dsT), oracle_grads(d, "k3", do, dsT))


def test_generic_backward_deterministic():
    d = make_kda_inputs(2, 40, 2, 96, 96, seed=8, state=True)
    do, dsT = cotangents(d, 9)
    a = gpu_grads(d, "k3", do, dsT)
    b = gpu_grads(d, "k3", do, dsT)
    for x, y in zip(a, b):
        assert x is None or torch.equal(x, y)


@pytest.mark.parametrize("KV", [(48, 80), (160, 24)])
@pytest.mark.parametrize("gate", ["k3", "precomputed"])
def test_generic_varlen(gate, KV):
    # packed sequences of ragged lengths, one of them empty
    K, V = KV
    cu = torch.tensor([0, 5, 5, 40, 57, 100], dtype=torch.int32, device="cuda")
    d = make_kda_inputs(1, 100, 2, K, V, seed=11, gate=gate)
    g = torch.Generator().manual_seed(12)
    d["s0"] = (torch.randn(5, 2, V, K, generator=g) * 0.05).cuda()
    out, fin = run_fwd(d, gate, cu)
    gm = "k3" if gate == "k3" else "logdecay"
    eo, ef = O.kda_varlen_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                                  np64(d["A_log"]), np64(d["dt_bias"]), cu.cpu().numpy(),
                                  initial_state=np64(d["s0"]), gate_mode=gm)
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2
    do, dsT = cotangents(d, 13, n_states=5)
    check(gpu_grads(d, gate, do, dsT, cu), oracle_grads(d, gate, do, dsT, cu))


@pytest.mark.parametrize("K", [32, 96, 200])
def test_generic_decode_matches_oracle_and_in_place(K):
    V = 72
    d = make_kda_inputs(3, 1, 2, K, V, seed=K, state=True)
    out, fin = ops.recurrent_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                    d["s0"], True, -5.0, K ** -0.5)
    eo, ef = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2
    st = d["s0"].clone()
    out2, fin2 = ops.recurrent_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                      st, True, -5.0, K ** -0.5, out_state=st)
    assert fin2.data_ptr() == st.data_ptr()
    assert torch.equal(out2, out) and torch.equal(st, fin)


@pytest.mark.parametrize("D", [16, 96, 200, 1024])
def test_generic_norm_gate(D):
    g = torch.Generator().manual_seed(D)
    x = torch.randn(2, 33, 3, D, generator=g).bfloat16().cuda()
    gt = torch.randn(2, 33, 3, D, generator=g).bfloat16().cuda()
    w = (1 + 0.1 * torch.randn(D, generator=g)).float().cuda()
    dy = torch.randn(2, 33, 3, D, generator=g).bfloat16().cuda()
    y, inv = ops.rmsnorm_gate_forward(x, gt, w, 1e-5)
    ey, _ = O.rmsnorm_gate_forward(np64(x), np64(gt), np64(w), 1e-5)
    assert rel_err(y, ey) < 1e-2
    dx, dg, dw = ops.rmsnorm_gate_backward(x, gt, w, inv, dy, 1e-5)
    edx, edg, edw = O.rmsnorm_gate_backward(np64(x), np64(gt), np64(w), 1e-5, np64(dy))
    assert cosine(dx, edx) > 0.9999 and cosine(dg, edg) > 0.9999 and cosine(dw, edw) > 0.9999
    assert rel_err(dw, edw) < 1e-2


def test_generic_project_chunk_autograd_and_norm_gate():
    # the operator API routes K = V = 96 to the token-serial kernels, forward and backward
    d = make_kda_inputs(2, 40, 2, 96, 96, seed=21)
    leaves = {n: d[n].detach().clone().requires_grad_() for n in ("q", "k", "v", "g", "beta")}
    out, _ = kda(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], d["A_log"], d["dt_bias"],
                 mode="project_chunk", allow_fallback=False)
    eo, _ = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 2e-2
    g = torch.Generator().manual_seed(22)
    do = torch.randn(out.shape, generator=g).bfloat16().cuda()
    out.backward(do)
    exp = O.kda_backward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                         np64(d["A_log"]), np64(d["dt_bias"]), grad_output=np64(do), gate_mode="k3")
    for name, e in zip(("q", "k", "v", "g", "beta"), exp[:5]):
        assert cosine(leaves[name].grad, e) > 0.9999, name
    og = torch.randn(out.shape, generator=g).bfloat16().cuda()
    w = torch.ones(96, device="cuda")
    from experiment_swa_kda_amd.kda import kda_norm_gate
    y = kda_norm_gate(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], og, w)
    ey, _ = O.rmsnorm_gate_forward(eo, np64(og), np64(w), 1e-5)
    assert rel_err(y, ey) < 2e-2


def test_generic_mixer_block_matches_reference_mode():
    # head_dim 96: the stateless mixer runs the stacked projections, the 864-channel
    # convolution, the token-serial KDA kernels and the generic norm-gate kernels
    from experiment_swa_kda_amd import KimiDeltaAttention, project_runtime_events, reset_project_runtime_events
    torch.manual_seed(3)
    layer = KimiDeltaAttention(288, 3, 96, mode="project_chunk").cuda()
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0, 0.06)
        layer.o_norm.weight.fill_(1.0)
    x = torch.randn(2, 70, 288, device="cuda").bfloat16().requires_grad_()
    reset_project_runtime_events()
    y, _ = layer(x)
    comps = {e["component"] for e in project_runtime_events()}
    assert {"chunk_forward", "rmsnorm_gate_forward"} <= comps, comps
    y.float().square().mean().backward()
    grads = {n: p.grad.clone() for n, p in layer.named_parameters()}
    gx = x.grad.clone()
    layer.zero_grad()
    x2 = x.float().detach().requires_grad_()
    y2, _ = layer(x2, mode="reference")
    y2.square().mean().backward()
    assert rel_err(y, y2) < 3e-2
    assert cosine(gx, x2.grad) > 0.995
    for n, p in layer.named_parameters():
        assert cosine(grads[n], p.grad) > 0.995, n


def test_generic_kv_cache_decode_matches_full_forward():
    """head_dim 96: prefill through the token-serial chunk path, then one-token decode
    steps through the recurrent entry point (token-serial kernel at T = 1)."""
    from experiment_swa_kda_amd.model import GPT, GPTConfig, KVCache
    cfg = GPTConfig(sequence_len=64, vocab_size=512, n_layer=2, n_head=3, n_embd=288)
    torch.manual_seed(0)
    model = GPT(cfg).cuda()
    model.init_weights()
    with torch.no_grad():
        for b in model.transformer.h:
            b.attn.o_proj.weight.normal_(0, 0.02)
            b.mlp.c_proj.weight.normal_(0, 0.02)
    g = torch.Generator(device="cuda").manual_seed(2)
    B, T, P = 2, 30, 21
    idx = torch.randint(0, 512, (B, T), device="cuda", generator=g)
    with torch.no_grad():
        full = model(idx)
        cache = KVCache(B, 3, T, 96, 2, "cuda", torch.bfloat16, inplace_state=True)
        pre = model(idx[:, :P], kv_cache=cache)
        assert rel_err(pre, full[:, :P]) < 2e-2
        for t in range(P, T):
            step = model(idx[:, t:t + 1], kv_cache=cache)
            assert rel_err(step[:, 0], full[:, t]) < 2e-2, t
