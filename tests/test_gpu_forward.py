"""GPU parity of the HIP forward kernels against the float64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as O
from tests.kda_testutil import make_kda_inputs, np64, rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import ops


def run_chunk(d, gate, final=True, cu=None):
    out, fin, _ = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                    d["s0"], final, -5.0, d["q"].shape[-1] ** -0.5, cu_seqlens=cu, gate=gate)
    return out, fin


def oracle_fwd(d, gate):
    return O.kda_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                         np64(d["A_log"]), np64(d["dt_bias"]), initial_state=np64(d["s0"]),
                         gate_mode="k3" if gate == "k3" else "logdecay")


@pytest.mark.parametrize("T", [1, 2, 3, 4, 31, 32, 33, 63, 64, 65, 127, 128, 129, 257])
def test_chunk_forward_boundary_lengths_d64(T):
    d = make_kda_inputs(1, T, 2, 64, 64, seed=100 + T, state=True)
    out, fin = run_chunk(d, "k3")
    eo, ef = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2
    torch.testing.assert_close(out.double().cpu(), torch.tensor(eo), atol=5e-3, rtol=5e-3)
    torch.testing.assert_close(fin.double().cpu(), torch.tensor(ef), atol=5e-3, rtol=5e-3)


# the reference's frozen boundary lengths at its production head dim
# (configs/research/kda_cuda_ownership.toml:42-43)
@pytest.mark.parametrize("T", [1, 2, 3, 4, 63, 64, 65, 127, 128, 129, 257])
def test_chunk_forward_boundary_lengths_d128(T):
    d = make_kda_inputs(1, T, 3, 128, 128, seed=400 + T, state=True)
    out, fin = run_chunk(d, "k3")
    eo, ef = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2
    torch.testing.assert_close(out.double().cpu(), torch.tensor(eo), atol=5e-3, rtol=5e-3)
    torch.testing.assert_close(fin.double().cpu(), torch.tensor(ef), atol=5e-3, rtol=5e-3)


@pytest.mark.parametrize("gate", ["k3", "precomputed"])
@pytest.mark.parametrize("KV", [(128, 128), (64, 128), (128, 64)])
def test_chunk_forward_d128(gate, KV):
    K, V = KV
    d = make_kda_inputs(2, 200, 3, K, V, seed=7, gate=gate, state=True, dist="baseline")
    out, fin = run_chunk(d, gate)
    eo, ef = oracle_fwd(d, gate)
    assert rel_err(out, eo) < 2e-2, rel_err(out, eo)
    assert rel_err(fin, ef) < 2e-2, rel_err(fin, ef)


def test_chunk_forward_deterministic():
    d = make_kda_inputs(2, 300, 3, 128, 128, seed=3)
    a = run_chunk(d, "k3")
    b = run_chunk(d, "k3")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_chunk_forward_varlen():
    d = make_kda_inputs(1, 400, 2, 64, 64, seed=9, state=False)
    cu = torch.tensor([0, 1, 70, 128, 129, 400], dtype=torch.int32, device="cuda")
    out, fin = run_chunk(d, "k3", cu=cu)
    eo, ef = O.kda_varlen_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                                  np64(d["A_log"]), np64(d["dt_bias"]), cu.cpu().numpy())
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2


def test_extreme_gates_finite():
    d = make_kda_inputs(1, 256, 2, 64, 64, seed=5)
    g = d["g"].clone()
    g[..., ::2] = -100.0
    g[..., 1::2] = 100.0
    d["g"] = g
    out, fin = run_chunk(d, "k3")
    assert torch.isfinite(out).all() and torch.isfinite(fin).all()
    eo, ef = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 2e-2


def test_steep_precomputed_decay_uses_exact_path():
    # per-token log decay ~ -8 exceeds the 80-nat span guard inside 16-token blocks
    d = make_kda_inputs(1, 130, 2, 64, 64, seed=6, gate="precomputed", state=True)
    d["g"] = d["g"] * 8.0
    out, fin = run_chunk(d, "precomputed")
    eo, ef = oracle_fwd(d, "precomputed")
    assert torch.isfinite(out).all()
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2


@pytest.mark.parametrize("K", [64, 128])
def test_decode_matches_oracle_and_chunk(K):
    d = make_kda_inputs(4, 17, 3, K, K, seed=11, state=True)
    state = d["s0"]
    outs = []
    for t in range(17):
        o, state = ops.recurrent_decode(d["q"][:, t:t + 1], d["k"][:, t:t + 1], d["v"][:, t:t + 1],
                                        d["g"][:, t:t + 1], d["beta"][:, t:t + 1], d["A_log"], d["dt_bias"],
                                        state, True, -5.0, K ** -0.5)
        outs.append(o)
    out = torch.cat(outs, 1)
    eo, ef = oracle_fwd(d, "k3")
    assert rel_err(out, eo) < 1e-2 and rel_err(state, ef) < 1e-3
    co, cf = run_chunk(d, "k3")
    torch.testing.assert_close(out.float(), co.float(), atol=5e-3, rtol=5e-3)


def test_decode_in_place_and_input_preserved():
    d = make_kda_inputs(2, 1, 3, 128, 128, seed=12, state=True)
    s = d["s0"].clone()
    o1, f1 = ops.recurrent_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                  s, True, -5.0, 128 ** -0.5)
    assert torch.equal(s, d["s0"])
    o2, f2 = ops.recurrent_decode(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
                                  s, True, -5.0, 128 ** -0.5, out_state=s)
    assert torch.equal(o1, o2) and torch.equal(f1, s)


@pytest.mark.parametrize("T,state,W,C", [(1, True, 4, 384), (3, True, 4, 384), (50, False, 4, 384),
                                         (257, True, 4, 384), (33, True, 3, 384), (128, True, 4, 136),
                                         (129, False, 2, 8), (255, True, 8, 264), (7, True, 1, 128)])
def test_conv_forward_backward(T, state, W, C):
    g = torch.Generator().manual_seed(T)
    B = 2
    x = torch.randn(B, T, C, generator=g).bfloat16()
    w = (torch.randn(C, W, generator=g) * 0.5).bfloat16()
    st = torch.randn(B, C, W, generator=g).bfloat16() if state else None
    dy = torch.randn(B, T, C, generator=g).bfloat16()
    dfin = torch.randn(B, C, W, generator=g).bfloat16()
    y, fin = ops.causal_conv_forward(x.cuda(), w.cuda(), None if st is None else st.cuda(), True)
    ey, ef = O.causal_conv_forward(np64(x), np64(w), np64(st))
    assert rel_err(y, ey) < 5e-3
    np.testing.assert_array_equal(np64(fin), ef)
    dx, dw, dst = ops.causal_conv_backward(x.cuda(), w.cuda(), None if st is None else st.cuda(), dy.cuda(), dfin.cuda())
    edx, edw, edst = O.causal_conv_backward(np64(x), np64(w), np64(dy), np64(st), np64(dfin))
    assert rel_err(dx, edx) < 5e-3 and rel_err(dw, edw) < 5e-3
    if state:
        assert rel_err(dst, edst) < 5e-3


@pytest.mark.parametrize("T,D", [(100, 128), (37, 64), (1, 128)])
def test_rmsnorm_gate_forward_backward(T, D):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, T, 3, D, generator=g).bfloat16()
    gt = torch.randn(2, T, 3, D, generator=g).bfloat16()
    w = torch.randn(D, generator=g).float()
    dy = torch.randn(2, T, 3, D, generator=g).bfloat16()
    y, inv = ops.rmsnorm_gate_forward(x.cuda(), gt.cuda(), w.cuda(), 1e-5)
    ey, einv = O.rmsnorm_gate_forward(np64(x), np64(gt), np64(w), 1e-5)
    assert rel_err(y, ey) < 5e-3 and rel_err(inv, einv.reshape(-1)) < 1e-5
    dx, dg, dw = ops.rmsnorm_gate_backward(x.cuda(), gt.cuda(), w.cuda(), inv, dy.cuda(), 1e-5)
    edx, edg, edw = O.rmsnorm_gate_backward(np64(x), np64(gt), np64(w), 1e-5, np64(dy))
    assert rel_err(dx, edx) < 5e-3 and rel_err(dg, edg) < 5e-3 and rel_err(dw, edw) < 1e-4


def test_unaligned_views_are_copied_before_the_kernels():
    """A contiguous view at an odd element offset is not 16-byte aligned; the host layer
    copies it, so results equal those of the aligned tensor."""
    g = torch.Generator().manual_seed(5)
    base = torch.randn(2 * 64 * 128 + 1, generator=g).bfloat16().cuda()
    x = base[1:].view(2, 64, 128)
    assert x.data_ptr() % 16 != 0
    w = (torch.randn(128, 4, generator=g) * 0.5).bfloat16().cuda()
    y, _ = ops.causal_conv_forward(x, w, None, False)
    y2, _ = ops.causal_conv_forward(x.clone(), w, None, False)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("gate,K,V,T", [("k3", 128, 128, 200), ("precomputed", 64, 64, 130),
                                         ("k3", 128, 64, 65), ("k3", 64, 128, 1)])
def test_chunk_forward_norm_gate_fused_matches_separate(gate, K, V, T):
    """The fused epilogue equals the separate norm kernel on the same o (up to the order of
    the f32 row sum), o is unchanged, and the norm output matches the oracle chain."""
    d = make_kda_inputs(2, T, 3, K, V, seed=T + K, gate=gate, state=False)
    g = torch.Generator().manual_seed(T)
    og = torch.randn(2, T, 3, V, generator=g).bfloat16().cuda()
    w = (1 + 0.3 * torch.randn(V, generator=g)).float().cuda()
    scale = K ** -0.5
    o, normed, inv, fin, _ = ops.chunk_forward_norm_gate(
        d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], None, True, -5.0,
        scale, og, w, 1e-5, gate=gate)
    o_ref, fin_ref, _ = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"],
                                          d["dt_bias"], None, True, -5.0, scale, gate=gate)
    assert torch.equal(o, o_ref) and torch.equal(fin, fin_ref)
    y_ref, inv_ref = ops.rmsnorm_gate_forward(o_ref, og, w, 1e-5)
    torch.testing.assert_close(inv, inv_ref, rtol=1e-6, atol=0)
    # one bf16 ulp where the f32 row sums round differently
    torch.testing.assert_close(normed.float(), y_ref.float(), rtol=8e-3, atol=1e-6)
    eo, _ = oracle_fwd(d, gate)
    ey, _ = O.rmsnorm_gate_forward(eo, np64(og), np64(w), 1e-5)
    assert rel_err(normed, ey) < 2e-2


def test_chunk_forward_norm_gate_autograd_matches_unfused():
    from experiment_swa_kda_amd.kda import _ProjectRMSNormGateAutograd, kda, kda_norm_gate
    d = make_kda_inputs(1, 150, 2, 128, 128, seed=5, state=False)
    g = torch.Generator().manual_seed(5)
    og = torch.randn(1, 150, 2, 128, generator=g).bfloat16().cuda()
    dy = torch.randn(1, 150, 2, 128, generator=g).bfloat16().cuda()
    names = ["q", "k", "v", "g", "beta"]

    def run(fused):
        leaves = {n: d[n].detach().clone().requires_grad_() for n in names}
        A = d["A_log"].detach().clone().requires_grad_()
        dt = d["dt_bias"].detach().clone().requires_grad_()
        gt = og.clone().requires_grad_()
        w = (1 + 0.3 * torch.randn(128, generator=torch.Generator().manual_seed(6))).cuda().requires_grad_()
        if fused:
            y = kda_norm_gate(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], A, dt,
                              gt, w, eps=1e-5)
        else:
            o, _ = kda(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"], A, dt,
                       mode="project_chunk")
            y = _ProjectRMSNormGateAutograd.apply(o, gt, w, 1e-5)
        y.backward(dy)
        return [y] + [leaves[n].grad for n in names] + [A.grad, dt.grad, gt.grad, w.grad]

    a, b = run(True), run(False)
    for x, e in zip(a, b):
        assert x is not None and e is not None
        cos = torch.nn.functional.cosine_similarity(x.double().flatten(), e.double().flatten(), dim=0)
        assert cos > 0.9999, float(cos)


@pytest.mark.parametrize("B,T,H,D,W", [(2, 150, 3, 128, 4), (1, 200, 2, 64, 4), (2, 17, 1, 128, 3),
                                       (1, 5, 2, 64, 4), (1, 1, 1, 128, 2), (1, 64, 2, 128, 1),
                                       (3, 1, 2, 64, 4)])
def test_chunk_forward_conv_matches_separate_conv(B, T, H, D, W):
    """The short convolution + SiLU computed in the chunk forward's first kernel: q, k, v
    equal kda_causal_conv_forward's bit for bit (halo rows across waves and chunks, rows
    before the sequence start, a partial last chunk), o and the normed output equal the
    unfused chunk forward on them, and the q activations match the oracle convolution."""
    g = torch.Generator().manual_seed(T * 7 + D + W)
    C = H * D
    wide = torch.randn(B, T, 3 * C + 24, generator=g).bfloat16().cuda()   # a column slice of a wider row
    x = wide[..., :3 * C]
    cw = (torch.randn(3 * C, W, generator=g) * 0.5).bfloat16().cuda()
    raw = torch.randn(B, T, H, D, generator=g).bfloat16().cuda()
    beta = torch.randn(B, T, H, generator=g).bfloat16().cuda()
    A_log = (torch.rand(H, generator=g) - 0.5).float().cuda()
    dt = (0.1 * torch.randn(H * D, generator=g)).float().cuda()
    og = torch.randn(B, T, H, D, generator=g).bfloat16().cuda()
    nw = (1 + 0.3 * torch.randn(D, generator=g)).float().cuda()
    q, k, v, o, normed, inv, _ = ops.chunk_forward_conv_norm_gate(x, cw, raw, beta, A_log, dt, -5.0, D ** -0.5,
                                                                   og, nw, 1e-5, H)
    y, _ = ops.causal_conv_forward(x.contiguous(), cw, None, False)
    qs, ks, vs = (t.reshape(B, T, H, D) for t in y.split(C, dim=-1))
    assert torch.equal(q, qs) and torch.equal(k, ks) and torch.equal(v, vs)
    o2, n2, inv2, _, _ = ops.chunk_forward_norm_gate(qs.contiguous(), ks.contiguous(), vs.contiguous(), raw, beta,
                                                     A_log, dt, None, False, -5.0, D ** -0.5, og, nw, 1e-5)
    assert torch.equal(o, o2) and torch.equal(normed, n2) and torch.equal(inv, inv2)
    # the output gate and beta logits read as column slices of the same packed rows as x
    packed = torch.zeros(B, T, 4 * C + 24, dtype=torch.bfloat16, device="cuda")
    packed[..., :3 * C] = x
    packed[..., 3 * C:4 * C] = og.reshape(B, T, C)
    packed[..., 4 * C + 8:4 * C + 8 + H] = beta
    r = ops.chunk_forward_conv_norm_gate(packed[..., :3 * C], cw, raw, packed[..., 4 * C + 8:4 * C + 8 + H], A_log,
                                         dt, -5.0, D ** -0.5, packed[..., 3 * C:4 * C].view(B, T, H, D), nw, 1e-5, H)
    assert torch.equal(r[3], o) and torch.equal(r[4], normed) and torch.equal(r[5], inv)
    ey, _ = O.causal_conv_forward(np64(x[..., :C]), np64(cw[:C]), None)
    assert rel_err(q.reshape(B, T, C), ey) < 1e-2


@pytest.mark.parametrize("B,T,C,W", [(2, 300, 384, 4), (3, 1, 128, 4), (1, 70, 64, 3)])
def test_conv_backward_strided_rows_equal_dense(B, T, C, W):
    """x read as a column slice of wider rows and dx written into a slice of wider rows give
    the dense convolution backward's dx and dweight bit for bit, and leave the rest of the
    wider rows untouched."""
    g = torch.Generator().manual_seed(B * 1000 + T + C + W)
    wide = torch.randn(B, T, C + 40, generator=g).bfloat16().cuda()
    x = wide[..., 8:8 + C]
    w = (torch.randn(C, W, generator=g) * 0.5).bfloat16().cuda()
    dy = torch.randn(B, T, C, generator=g).bfloat16().cuda()
    dx_ref, dw_ref, _ = ops.causal_conv_backward(x.contiguous(), w, None, dy, None)
    out = torch.full((B, T, C + 24), 7.0, dtype=torch.bfloat16, device="cuda")
    dx, dw, _ = ops.causal_conv_backward(x, w, None, dy, None, dx_out=out[..., 16:16 + C])
    assert torch.equal(dx, dx_ref) and torch.equal(dw, dw_ref)
    assert torch.equal(out[..., 16:16 + C], dx_ref)
    assert bool((out[..., :16] == 7.0).all()) and bool((out[..., 16 + C:] == 7.0).all())


def test_mixer_fused_conv_equals_separate_conv():
    """KimiDeltaAttention's stateless path with the convolutions fused into the chunk forward
    gives the same output and the same gradient for every parameter and the input, bit for
    bit, as the path with the separate convolution launch."""
    from experiment_swa_kda_amd import KimiDeltaAttention
    torch.manual_seed(0)
    layer = KimiDeltaAttention(256, 2, 128, mode="project_chunk").cuda()
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0, 0.06)
        layer.o_norm.weight.fill_(1.0)
    x0 = torch.randn(2, 200, 256, device="cuda").bfloat16()
    dy = torch.randn(2, 200, 256, device="cuda").bfloat16()
    res = []
    for fuse in (True, False):
        layer.fuse_conv = fuse
        layer.zero_grad()
        x = x0.clone().requires_grad_()
        y, _ = layer(x)
        y.backward(dy)
        res.append([y, x.grad] + [p.grad.clone() for p in layer.parameters()])
    for a, b in zip(*res):
        assert torch.equal(a, b)
