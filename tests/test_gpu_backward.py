"""GPU parity of the HIP chunked backward against the float64 oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda_oracle as O
from tests.kda_testutil import cosine, make_kda_inputs, np64, rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import ops

NAMES = ("dq", "dk", "dv", "dgate", "dbeta", "dA_log", "ddt_bias", "dS0")


def gpu_grads(d, gate, do, dsT, cu=None):
    K = d["q"].shape[-1]
    _, _, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"],
                                 True, -5.0, K ** -0.5, cu_seqlens=cu, gate=gate)
    return ops.chunk_backward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"], ws,
                              do, dsT, -5.0, K ** -0.5, cu_seqlens=cu, gate=gate)


def oracle_grads(d, gate, do, dsT, cu=None):
    gm = "k3" if gate == "k3" else "logdecay"
    args = (np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]), np64(d["A_log"]),
            np64(d["dt_bias"]))
    if cu is None:
        return O.kda_backward(*args, initial_state=np64(d["s0"]), grad_output=np64(do),
                              grad_final_state=np64(dsT), gate_mode=gm)
    return O.kda_varlen_backward(*args, cu.cpu().numpy(), grad_output=np64(do), grad_final_state=np64(dsT),
                                 initial_state=np64(d["s0"]), gate_mode=gm)


def cotangents(d, seed, n_states=None):
    g = torch.Generator().manual_seed(seed)
    do = torch.randn(d["v"].shape, generator=g).bfloat16().cuda()
    B, T, H, V = d["v"].shape
    K = d["q"].shape[-1]
    n = B if n_states is None else n_states
    dsT = torch.randn(n, H, V, K, generator=g).cuda()
    return do, dsT


def check(actual, expected, *, cos_min=0.9999, skip=()):
    report = {}
    for name, a, e in zip(NAMES, actual, expected):
        if e is None or name in skip:
            continue
        if a is None:
            raise AssertionError(f"{name} missing")
        c = cosine(a, e)
        report[name] = (c, rel_err(a, e))
    print({n: (round(c, 7), round(r, 5)) for n, (c, r) in report.items()})
    bad = {n: v for n, v in report.items() if not v[0] >= cos_min}
    assert not bad, f"cosine below {cos_min}: {bad} (all: {report})"
    return report


@pytest.mark.parametrize("T", [1, 2, 31, 33, 64, 65, 129])
def test_backward_d64_boundaries(T):
    d = make_kda_inputs(1, T, 2, 64, 64, seed=200 + T, state=True)
    do, dsT = cotangents(d, T)
    check(gpu_grads(d, "k3", do, dsT), oracle_grads(d, "k3", do, dsT))


# the reference's frozen boundary lengths at its production head dim
# (configs/research/kda_cuda_ownership.toml:42-43)
@pytest.mark.parametrize("T", [1, 2, 3, 4, 63, 64, 65, 127, 128, 129, 257])
def test_backward_d128_boundaries(T):
    d = make_kda_inputs(1, T, 3, 128, 128, seed=300 + T, state=True)
    do, dsT = cotangents(d, 1000 + T)
    check(gpu_grads(d, "k3", do, dsT), oracle_grads(d, "k3", do, dsT))


def test_backward_wait_timeout_is_reported():
    """With the fused backward's wait bound set to 0 from the host, every tile whose chunk
    the reverse scan has not yet finished gives up at once (every kernel still exits
    normally): the status call must report it, the given-up tiles' gradients must be NaN,
    ops.chunk_backward must raise, and a later call with the default bound must be correct."""
    from experiment_swa_kda_amd import _lib

    lib = _lib.load()
    d = make_kda_inputs(2, 1024, 3, 128, 128, seed=77, state=True)
    do, dsT = cotangents(d, 77)
    K = 128
    _, _, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"],
                                 True, -5.0, K ** -0.5, gate="k3")
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"], ws, do, dsT, -5.0,
            K ** -0.5)
    print("wait-timeout test: B2 T1024 H3 D128, wait limit 0", flush=True)
    assert lib.kda_debug_set_wait_limit(0) == 0
    try:
        grads, p, scratch = ops.chunk_backward_launch(*args, gate="k3")
        with pytest.raises(RuntimeError, match="timed out"):
            ops.chunk_backward_status(p, scratch)
        dq, dk, dv, dg, db, dA, ddt, _ = grads
        # the first tiles (the sequences' last chunks) start before the scan's first step
        assert torch.isnan(dq.float()).any() and torch.isnan(dv.float()).any()
        assert torch.isnan(dg.float()).any() and torch.isnan(db.float()).any()
        assert torch.isnan(dA).all() and torch.isnan(ddt).any()
        # every token row is either fully NaN or fully finite (whole tiles are poisoned)
        rows = torch.isnan(dq.float()).any(-1)
        assert torch.equal(rows, torch.isnan(dq.float()).all(-1))
        with pytest.raises(RuntimeError, match="timed out"):
            ops.chunk_backward(*args, gate="k3")
    finally:
        lib.kda_debug_set_wait_limit(-1)
    grads = ops.chunk_backward(*args, gate="k3")  # default bound: no failure, flag cleared
    check(grads, oracle_grads(d, "k3", do, dsT))


@pytest.mark.parametrize("gate", ["k3", "precomputed"])
@pytest.mark.parametrize("KV", [(128, 128), (64, 128), (128, 64)])
def test_backward_d128(gate, KV):
    K, V = KV
    d = make_kda_inputs(2, 160, 3, K, V, seed=21, gate=gate, state=True, dist="baseline")
    do, dsT = cotangents(d, 3)
    check(gpu_grads(d, gate, do, dsT), oracle_grads(d, gate, do, dsT))


def test_backward_reference_tolerances_t33():
    # tests/test_kda_cuda.py:120-147: 8e-3 for q/k/v/S0 and 2e-2 for gate/beta/A_log/dt_bias
    d = make_kda_inputs(1, 33, 2, 64, 64, seed=20260805 + 33 + 64, state=True)
    do, dsT = cotangents(d, 1)
    act = gpu_grads(d, "k3", do, dsT)
    exp = oracle_grads(d, "k3", do, dsT)
    for name, a, e in zip(NAMES, act, exp):
        tol = 2e-2 if name in ("dgate", "dbeta", "dA_log", "ddt_bias") else 8e-3
        torch.testing.assert_close(a.double().cpu().reshape(np.shape(e)), torch.tensor(e), atol=tol, rtol=tol,
                                   msg=lambda m, n=name: f"{n}: {m}")


def test_backward_varlen():
    d = make_kda_inputs(1, 300, 2, 64, 64, seed=31, state=True)
    cu = torch.tensor([0, 5, 64, 65, 200, 300], dtype=torch.int32, device="cuda")
    d["s0"] = torch.randn(5, 2, 64, 64, generator=torch.Generator().manual_seed(2)).cuda() * 0.05
    do, dsT = cotangents(d, 4, n_states=5)
    check(gpu_grads(d, "k3", do, dsT, cu), oracle_grads(d, "k3", do, dsT, cu))


def test_backward_steep_decay_exact_path():
    d = make_kda_inputs(1, 130, 2, 64, 64, seed=8, gate="precomputed", state=True)
    d["g"] = d["g"] * 8.0
    do, dsT = cotangents(d, 5)
    act = gpu_grads(d, "precomputed", do, dsT)
    for a in act:
        if a is not None:
            assert torch.isfinite(a).all()
    check(act, oracle_grads(d, "precomputed", do, dsT))


def test_backward_extreme_gates_finite():
    d = make_kda_inputs(1, 256, 2, 64, 64, seed=5, state=True)
    g = d["g"].clone()
    g[..., ::2] = -100.0
    g[..., 1::2] = 100.0
    d["g"] = g
    do, dsT = cotangents(d, 6)
    for a in gpu_grads(d, "k3", do, dsT):
        assert torch.isfinite(a).all()


@pytest.mark.parametrize("T,KV", [(1100, (64, 64)), (600, (128, 128))])
def test_long_sequences_states_and_gradients(T, KV):
    """Multi-chunk sequences with a ragged last chunk: initial state in, final state out and
    every gradient including dS0, against the float64 oracle."""
    K, V = KV
    d = make_kda_inputs(2, T, 2, K, V, seed=T, gate="precomputed", state=True, dist="baseline")
    o, fin, _ = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"],
                                  True, -5.0, K ** -0.5, gate="precomputed")
    eo, ef = O.kda_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                           np64(d["A_log"]), np64(d["dt_bias"]), initial_state=np64(d["s0"]), gate_mode="logdecay")
    assert rel_err(o, eo) < 2e-2 and rel_err(fin, ef) < 2e-2
    do, dsT = cotangents(d, 9)
    check(gpu_grads(d, "precomputed", do, dsT), oracle_grads(d, "precomputed", do, dsT))


@pytest.mark.parametrize("B,T,H,KV,gate", [(1, 8192, 2, (128, 128), "precomputed"),
                                            (1, 6500, 1, (64, 64), "k3")])
def test_segmented_scan_long_sequence(B, T, H, KV, gate):
    """Sequences of >= 96 chunks with few recurrences take the segmented forward scan
    (segment maps, combine, replay; 11-12 chunks per segment, ragged last segment and
    chunk): output, final state and every gradient against the float64 oracle."""
    K, V = KV
    d = make_kda_inputs(B, T, H, K, V, seed=T + 1, gate=gate, state=True, dist="baseline")
    o, fin, _ = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"],
                                  True, -5.0, K ** -0.5, gate=gate)
    gm = "k3" if gate == "k3" else "logdecay"
    eo, ef = O.kda_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                           np64(d["A_log"]), np64(d["dt_bias"]), initial_state=np64(d["s0"]), gate_mode=gm)
    assert rel_err(o, eo) < 2e-2 and rel_err(fin, ef) < 2e-2, (rel_err(o, eo), rel_err(fin, ef))
    do, dsT = cotangents(d, 5)
    check(gpu_grads(d, gate, do, dsT), oracle_grads(d, gate, do, dsT))


def test_varlen_mixed_lengths():
    """Packed sequences of 1, 3, 58 and 2 chunks, each with its own initial state."""
    lens = [40, 150, 3700, 100]
    T = sum(lens)
    d = make_kda_inputs(1, T, 2, 64, 64, seed=77, state=True)
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32, device="cuda")
    d["s0"] = torch.randn(len(lens), 2, 64, 64, generator=torch.Generator().manual_seed(3)).cuda() * 0.05
    do, dsT = cotangents(d, 11, n_states=len(lens))
    check(gpu_grads(d, "k3", do, dsT, cu), oracle_grads(d, "k3", do, dsT, cu))


def test_dense_decay_rounds_equal_separate_stages():
    """With at least one tile per CU the backward runs the dense and decay tiles as full
    rounds of one kernel (the launch that finishes the dense tiles starts the first decay
    tiles).  Its gradients must equal, bit for bit, the stage-by-stage run (scan, all dense
    tiles, all decay tiles, parameter reduction) on the same workspace."""
    import ctypes
    from experiment_swa_kda_amd import _lib
    from experiment_swa_kda_amd._lib import ptr
    d = make_kda_inputs(2, 4096, 3, 128, 128, seed=21, dist="baseline")  # 384 tiles
    do, _ = cotangents(d, 22)
    K = 128
    full = gpu_grads(d, "k3", do, None)
    _, _, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], None,
                                 False, -5.0, K ** -0.5, gate="k3")
    p = ops._problem(d["q"], d["v"], None, ops.GATE_MODES["k3"], -5.0, K ** -0.5)
    lib = _lib.load()
    scratch = torch.empty(lib.kda_chunk_backward_scratch_bytes(ctypes.byref(p)), dtype=torch.uint8, device="cuda")
    outs = [torch.empty_like(d[n]) for n in ("q", "k", "v", "g", "beta")]
    dA, ddt = torch.empty_like(d["A_log"]), torch.empty_like(d["dt_bias"])
    args = (ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(d["g"]), ptr(d["beta"]), ptr(d["A_log"]), ptr(d["dt_bias"]),
            None, ptr(ws), ptr(do), None, *[ptr(x) for x in outs], ptr(dA), ptr(ddt), None, ptr(scratch),
            torch.cuda.current_stream().cuda_stream)
    for stage in (10, 11, 12, 13):
        _lib.check(lib.kda_chunk_backward_stage(stage, ctypes.byref(p), *args), f"stage {stage}")
    torch.cuda.synchronize()
    staged = outs + [dA, ddt.reshape(full[6].shape)]
    for a, b in zip(full[:7], staged):
        assert torch.equal(a, b)


def test_varlen_with_empty_sequences():
    """Zero-length sequences in cu_seqlens (non-decreasing offsets, as the reference allows):
    their final state is the initial state and their state gradient passes straight through."""
    d = make_kda_inputs(1, 300, 2, 64, 64, seed=41, state=True)
    cu = torch.tensor([0, 70, 70, 200, 200, 300], dtype=torch.int32, device="cuda")
    d["s0"] = torch.randn(5, 2, 64, 64, generator=torch.Generator().manual_seed(5)).cuda() * 0.05
    do, dsT = cotangents(d, 6, n_states=5)
    K = d["q"].shape[-1]
    out, fin, _ = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"],
                                    True, -5.0, K ** -0.5, cu_seqlens=cu, gate="k3")
    assert torch.equal(fin[1], d["s0"][1]) and torch.equal(fin[3], d["s0"][3])
    eo, ef = O.kda_varlen_forward(np64(d["q"]), np64(d["k"]), np64(d["v"]), np64(d["g"]), np64(d["beta"]),
                                  np64(d["A_log"]), np64(d["dt_bias"]), cu.cpu().numpy(),
                                  initial_state=np64(d["s0"]), gate_mode="k3")
    assert rel_err(out, eo) < 2e-2 and rel_err(fin, ef) < 2e-2
    grads = gpu_grads(d, "k3", do, dsT, cu)
    assert torch.equal(grads[7][1], dsT[1]) and torch.equal(grads[7][3], dsT[3])
    check(grads, oracle_grads(d, "k3", do, dsT, cu))


@pytest.mark.parametrize("gate", ["precomputed", "k3"])
def test_graphed_forward_backward_replays_match_eager(gate):
    """One forward+backward through the autograd API captured as a HIP graph (the step the
    benchmark times): every replay, with new inputs copied in and eager work in between,
    gives the eager outputs and gradients bit for bit."""
    from experiment_swa_kda_amd import kda
    names = ("q", "k", "v", "g", "beta", "A_log", "dt_bias")
    static = {n: x.clone().requires_grad_() for n, x in
              make_kda_inputs(1, 192, 2, 128, 128, seed=40, gate=gate, dist="baseline").items() if n in names}
    do = torch.randn(1, 192, 2, 128, device="cuda").bfloat16()

    def step(t):
        for x in t.values():
            x.grad = None
        out, _ = kda(*[t[n] for n in names], mode="project_chunk", gate=gate, allow_fallback=False)
        out.backward(do)
        return out

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = step(static)
    for seed in (41, 42, 43):
        fresh = make_kda_inputs(1, 192, 2, 128, 128, seed=seed, gate=gate, dist="baseline")
        with torch.no_grad():
            for n in names:
                static[n].copy_(fresh[n])
        graph.replay()
        eager = {n: fresh[n].clone().requires_grad_() for n in names}
        out = step(eager)
        torch.cuda.synchronize()
        assert torch.equal(out_static, out), seed
        for n in names:
            if eager[n].grad is None:  # A_log, dt_bias with a precomputed gate
                assert static[n].grad is None, (seed, n)
            else:
                assert torch.equal(static[n].grad, eager[n].grad), (seed, n)


@pytest.mark.parametrize("K", [64, 128])
def test_packed_qkv_gradients_equal_separate(K):
    """dq, dk, dv written side by side into one [B, T, 3 H K] tensor (grad_row_stride) are
    the separately written gradients, bit for bit; the other gradients are unchanged."""
    d = make_kda_inputs(2, 130, 3, K, K, seed=37, gate="k3", state=False, dist="baseline")
    do, _ = cotangents(d, 5)
    _, _, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], None,
                                 False, -5.0, K ** -0.5, gate="k3")
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], None, ws, do, None, -5.0, K ** -0.5)
    sep = ops.chunk_backward(*args, gate="k3")
    packed = ops.chunk_backward(*args, gate="k3", packed_qkv_grad=True)
    B, T, H = 2, 130, 3
    dqkv = packed[0].view(B, T, 3, H, K)
    for j in range(3):
        assert torch.equal(dqkv[:, :, j], sep[j])
    for a, b in zip(sep[3:7], packed[3:7]):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_dbeta_into_packed_rows_equals_dense():
    """dbeta_logits written as a column slice of wider per-token rows (beta_row_stride), with
    the padding columns after it zeroed, is the dense dbeta bit for bit; the other columns of
    the rows are left alone."""
    B, T, H, K = 2, 130, 3, 64
    d = make_kda_inputs(B, T, H, K, K, seed=41, gate="k3", state=False, dist="baseline")
    do, _ = cotangents(d, 6)
    N, off, pad = 32, 8, 5
    rows = torch.randn(B, T, N, device="cuda").to(torch.bfloat16)
    rows[..., off:off + H] = d["beta"]
    beta_view = rows[..., off:off + H]
    _, _, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], None,
                                 False, -5.0, K ** -0.5, gate="k3")
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], None, ws, do, None, -5.0, K ** -0.5)
    dense = ops.chunk_backward(*args, gate="k3")
    out = torch.full((B, T, N), 7.0, device="cuda", dtype=torch.bfloat16)
    sargs = (d["q"], d["k"], d["v"], d["g"], beta_view) + args[5:]
    strided = ops.chunk_backward(*sargs, gate="k3", dbeta_out=out[..., off:off + H], dbeta_pad=pad)
    assert torch.equal(out[..., off:off + H], dense[4])
    assert torch.equal(out[..., off + H:off + H + pad], torch.zeros_like(out[..., :pad]))
    assert torch.equal(out[..., :off], torch.full_like(out[..., :off], 7.0))
    assert torch.equal(out[..., off + H + pad:], torch.full_like(out[..., off + H + pad:], 7.0))
    for j in (0, 1, 2, 3, 5, 6):
        assert torch.equal(strided[j], dense[j])


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128])
def test_norm_gate_backward_strided_gate_equals_dense(D):
    """The norm-gate VJP reading its gate from, and writing dgate into, column slices of
    wider per-token rows gives the dense results bit for bit."""
    B, T, H = 2, 77, 3
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(B, T, H, D, device="cuda", generator=g).to(torch.bfloat16)
    N = H * D + 24
    rows = torch.randn(B, T, N, device="cuda", generator=g).to(torch.bfloat16)
    gate = rows[..., 8:8 + H * D].view(B, T, H, D)
    w = torch.randn(D, device="cuda", generator=g)
    dy = torch.randn(B, T, H, D, device="cuda", generator=g).to(torch.bfloat16)
    _, inv = ops.rmsnorm_gate_forward(x, gate.contiguous(), w, 1e-5)
    ref = ops.rmsnorm_gate_backward(x, gate.contiguous(), w, inv, dy, 1e-5)
    out = torch.full((B, T, N), 3.0, device="cuda", dtype=torch.bfloat16)
    got = ops.rmsnorm_gate_backward(x, gate, w, inv, dy, 1e-5, dgate_out=out[..., 16:16 + H * D].view(B, T, H, D))
    assert torch.equal(got[0], ref[0]) and torch.equal(got[2], ref[2])
    assert torch.equal(out[..., 16:16 + H * D].view(B, T, H, D), ref[1])
    assert torch.equal(out[..., :16], torch.full_like(out[..., :16], 3.0))
    assert torch.equal(out[..., 16 + H * D:], torch.full_like(out[..., 16 + H * D:], 3.0))
