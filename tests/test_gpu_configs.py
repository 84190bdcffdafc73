"""Parity of the HIP path at the BASELINE configurations' full sizes.

Gates (north star): bf16 outputs and final state within norm-relative error 2e-2 of the
float64 oracle; every gradient cosine >= 0.9999; forward bitwise deterministic.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as O
from tests.kda_testutil import cosine, np64, rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import kda, ops

GRAD_NAMES = ("dq", "dk", "dv", "dgate", "dbeta", "dA_log", "ddt_bias", "dS0")


def baseline_inputs(B, T, H, K, V, seed, gate):
    """BASELINE config 1/2/5 distributions: q,k L2-normalised from N(0,1), v ~ N(0,1),
    beta logits ~ N(0,1); precomputed gate g = -exp(A_log) softplus(N(0,1) + dt_bias),
    A_log ~ U(-1,1), dt_bias = 0 (config 1 uses g = -softplus(N(0,1)), i.e. A_log = 0)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    v = torch.randn(B, T, H, V, generator=g)
    z = torch.randn(B, T, H, K, generator=g)
    bl = torch.randn(B, T, H, generator=g)
    A_log = torch.rand(H, generator=g) * 2 - 1 if gate == "precomputed-alog" else torch.zeros(H)
    gv = (-A_log.exp().view(1, 1, H, 1) * torch.nn.functional.softplus(z)).float()
    do = torch.randn(B, T, H, V, generator=g)
    return dict(q=q.bfloat16().cuda(), k=k.bfloat16().cuda(), v=v.bfloat16().cuda(), g=gv.cuda(),
                beta=bl.bfloat16().cuda(), do=do.bfloat16().cuda())


def run_fwd_bwd(d, cu=None, dsT=None, s0=None):
    K = d["q"].shape[-1]
    out, fin, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], None, None, s0, True, -5.0,
                                     K ** -0.5, cu_seqlens=cu, gate="precomputed")
    grads = ops.chunk_backward(d["q"], d["k"], d["v"], d["g"], d["beta"], None, None, s0, ws, d["do"], dsT,
                               -5.0, K ** -0.5, cu_seqlens=cu, gate="precomputed")
    return out, fin, grads


def check_grads(actual, expected, tag):
    report = {}
    for name, a, e in zip(GRAD_NAMES, actual, expected):
        if e is None or a is None:
            continue
        report[name] = round(cosine(a, e), 7)
    print(tag, report)
    bad = {n: c for n, c in report.items() if not c >= 0.9999}
    assert not bad, f"{tag}: gradient cosine below 0.9999: {bad}"


def test_config1_fwd_bwd_vs_fp64():
    # B1 T256 H2 D64, seed 0, g = -softplus(N(0,1)), zero initial state
    d = baseline_inputs(1, 256, 2, 64, 64, seed=0, gate="precomputed")
    out, fin, grads = run_fwd_bwd(d)
    args = (np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]))
    eo, ef = O.kda_forward(*args, gate_mode="logdecay")
    assert rel_err(out, eo) <= 2e-2 and rel_err(fin, ef) <= 2e-2
    eg = O.kda_backward(*args, grad_output=np64(d["do"]), gate_mode="logdecay")
    check_grads(grads, eg, "config1")


def test_config2_full_size_fwd_bwd_vs_fp64_and_deterministic():
    # B2 T4096 H3 D128, seed 42, the BASELINE config-2 gate with A_log ~ U(-1,1)
    d = baseline_inputs(2, 4096, 3, 128, 128, seed=42, gate="precomputed-alog")
    out, fin, grads = run_fwd_bwd(d)
    out2, fin2, _ = run_fwd_bwd(d)
    assert torch.equal(out, out2) and torch.equal(fin, fin2), "forward is not bitwise deterministic"
    args = (np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]))
    eo, ef = O.kda_forward(*args, gate_mode="logdecay")
    r_o, r_s = rel_err(out, eo), rel_err(fin, ef)
    print("config2 forward rel err: output", r_o, "state", r_s)
    assert r_o <= 2e-2 and r_s <= 2e-2
    eg = O.kda_backward(*args, grad_output=np64(d["do"]), gate_mode="logdecay")
    check_grads(grads, eg, "config2")


def test_config2_k3_gate_forward_full_size():
    # the reference's own Level-1 inputs: K3 gate, raw ~ N(0,1), A_log = dt_bias = 0
    g = torch.Generator().manual_seed(4100 + 4096)
    B, T, H, K = 2, 4096, 3, 128
    q, k, v, z = (torch.randn(B, T, H, K, generator=g).bfloat16().cuda() for _ in range(4))
    bl = torch.randn(B, T, H, generator=g).bfloat16().cuda()
    A_log, dt = torch.zeros(H, device="cuda"), torch.zeros(H * K, device="cuda")
    out, fin = kda(q, k, v, z, bl, A_log, dt, output_final_state=True, mode="project_chunk", allow_fallback=False)
    eo, ef = O.kda_forward(np64(q), np64(k), np64(v), np64(z), np64(bl), np64(A_log), np64(dt))
    assert rel_err(out, eo) <= 2e-2 and rel_err(fin, ef) <= 2e-2


def test_config2_k3_gate_backward_full_size():
    # the reference's gradient-lane inputs: K3 gate, every activation ~ N(0,1) (seed
    # 4100 + T + 1 there), A_log = dt_bias = 0, upstream gradient ~ N(0,1); all eight
    # gradients against the fp64 oracle
    g = torch.Generator().manual_seed(4100 + 4096 + 1)
    B, T, H, K = 2, 4096, 3, 128
    q, k, v, z = (torch.randn(B, T, H, K, generator=g).bfloat16().cuda() for _ in range(4))
    bl = torch.randn(B, T, H, generator=g).bfloat16().cuda()
    do = torch.randn(B, T, H, K, generator=g).bfloat16().cuda()
    A_log, dt = torch.zeros(H, device="cuda"), torch.zeros(H * K, device="cuda")
    out, fin, ws = ops.chunk_forward(q, k, v, z, bl, A_log, dt, None, True, -5.0, K ** -0.5, gate="k3")
    grads = ops.chunk_backward(q, k, v, z, bl, A_log, dt, None, ws, do, None, -5.0, K ** -0.5, gate="k3")
    args = (np64(q), np64(k), np64(v), np64(z), np64(bl), np64(A_log), np64(dt))
    eo, ef = O.kda_forward(*args)
    assert rel_err(out, eo) <= 2e-2 and rel_err(fin, ef) <= 2e-2
    eg = O.kda_backward(*args, grad_output=np64(do))
    check_grads(grads, eg, "config2-k3")


def test_config3_decode_continues_chunked_prefill():
    # B64 H3 D128: chunked prefill of T=1024 -> state, then 256 single-token steps; the
    # decode outputs must match the chunked forward over T+256 (and the fp64 oracle)
    g = torch.Generator().manual_seed(42)
    B, T0, N, H, K = 64, 1024, 256, 3, 128
    q = torch.nn.functional.normalize(torch.randn(B, T0 + N, H, K, generator=g), dim=-1).bfloat16().cuda()
    k = torch.nn.functional.normalize(torch.randn(B, T0 + N, H, K, generator=g), dim=-1).bfloat16().cuda()
    v = torch.randn(B, T0 + N, H, K, generator=g).bfloat16().cuda()
    A_log = (torch.rand(H, generator=g) * 2 - 1)
    gv = (-A_log.exp().view(1, 1, H, 1) * torch.nn.functional.softplus(torch.randn(B, T0 + N, H, K, generator=g)))
    gv = gv.float().cuda()
    bl = torch.randn(B, T0 + N, H, generator=g).bfloat16().cuda()
    sc = K ** -0.5
    _, state, _ = ops.chunk_forward(q[:, :T0], k[:, :T0], v[:, :T0], gv[:, :T0], bl[:, :T0], None, None, None,
                                    True, -5.0, sc, gate="precomputed")
    outs = []
    for t in range(T0, T0 + N):
        o, _ = ops.recurrent_decode(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], gv[:, t:t + 1], bl[:, t:t + 1],
                                    None, None, state, True, -5.0, sc, gate="precomputed", out_state=state)
        outs.append(o)
    dec = torch.cat(outs, 1)
    full, fin, _ = ops.chunk_forward(q, k, v, gv, bl, None, None, None, True, -5.0, sc, gate="precomputed")
    assert rel_err(dec, full[:, T0:]) <= 1e-2
    assert rel_err(state, fin) <= 1e-2
    # fp64 oracle on a slice of the batch
    sl = slice(0, 4)
    eo, ef = O.kda_forward(np64(q[sl]), np64(k[sl]), np64(v[sl]), np64(gv[sl]), np64(bl[sl]), gate_mode="logdecay")
    assert rel_err(dec[sl], eo[:, T0:]) <= 2e-2 and rel_err(state[sl], ef) <= 2e-2


def test_config5_varlen_fwd_bwd_vs_per_sequence_fp64():
    # H8 D128, 16384 packed tokens, lengths ~ U(128, 8192) at seed 7 (last truncated)
    rng = np.random.default_rng(7)
    lens, total = [], 16384
    while sum(lens) < total:
        lens.append(int(min(rng.integers(128, 8193), total - sum(lens))))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device="cuda")
    d = baseline_inputs(1, total, 8, 128, 128, seed=7, gate="precomputed-alog")
    out, fin, grads = run_fwd_bwd(d, cu=cu)
    args = (np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]), None, None, cu.cpu().numpy())
    eo, ef = O.kda_varlen_forward(*args, gate_mode="logdecay")
    print("config5 lengths", lens, "rel err out", rel_err(out, eo), "state", rel_err(fin, ef))
    assert rel_err(out, eo) <= 2e-2 and rel_err(fin, ef) <= 2e-2
    eg = O.kda_varlen_backward(*args, grad_output=np64(d["do"]), gate_mode="logdecay")
    check_grads(grads, eg, "config5")
