"""The allocation-free chunked backward (kda_chunk_backward_noalloc) called through the
C ABI: its gradients equal, bit for bit, kda_chunk_backward's with a caller scratch buffer,
on two calls in a row (the second on a smaller problem, so stale contents of the shared
static scratch from the first call must not leak into it), plus the size limit."""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests.kda_testutil import make_kda_inputs

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from experiment_swa_kda_amd import _lib, ops
    from experiment_swa_kda_amd._lib import ptr


def _backward_both(B, T, H, K, V, seed, state):
    d = make_kda_inputs(B, T, H, K, V, seed=seed, state=state, dist="baseline")
    g = torch.Generator().manual_seed(seed + 1)
    do = torch.randn(B, T, H, V, generator=g).bfloat16().cuda()
    dfin = (torch.randn(B, H, V, K, generator=g) * 0.1).cuda() if state else None
    scale = K ** -0.5
    _, _, ws = ops.chunk_forward(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], d["s0"],
                                 state, -5.0, scale, gate="k3")
    p = ops._problem(d["q"], d["v"], None, ops.GATE_MODES["k3"], -5.0, scale)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream

    def outs():
        o = [torch.empty_like(d[n]) for n in ("q", "k", "v", "g", "beta")]
        o += [torch.empty_like(d["A_log"]), torch.empty_like(d["dt_bias"])]
        o.append(torch.empty_like(d["s0"]) if state else None)
        return o

    head = (ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(d["g"]), ptr(d["beta"]), ptr(d["A_log"]),
            ptr(d["dt_bias"]), ptr(d["s0"]), ptr(ws), ptr(do), ptr(dfin))
    ref = outs()
    scratch = torch.empty(lib.kda_chunk_backward_scratch_bytes(ctypes.byref(p)), dtype=torch.uint8, device="cuda")
    _lib.check(lib.kda_chunk_backward(ctypes.byref(p), *head, *[ptr(x) for x in ref], ptr(scratch), stream),
               "kda_chunk_backward")
    got = outs()
    _lib.check(lib.kda_chunk_backward_noalloc(ctypes.byref(p), *head, *[ptr(x) for x in got], stream),
               "kda_chunk_backward_noalloc")
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_backward_equals_caller_scratch_twice():
    # config 2 at full size, then a smaller ragged problem with an initial state
    for B, T, H, K, V, seed, state in ((2, 4096, 3, 128, 128, 42, False), (1, 300, 2, 64, 128, 7, True)):
        print(f"noalloc case B{B} T{T} H{H} K{K} V{V}", flush=True)
        ref, got = _backward_both(B, T, H, K, V, seed, state)
        for a, b in zip(ref, got):
            assert (a is None and b is None) or torch.equal(a, b)


def test_noalloc_backward_rejects_problems_beyond_the_static_scratch():
    lib = _lib.load()
    limit = lib.kda_chunk_backward_noalloc_max_scratch_bytes()
    assert limit == 128 << 20
    p = _lib.ChunkProblem(batch=8, seq_len=8192, heads=8, key_dim=128, value_dim=128, num_seqs=8,
                          cu_seqlens=None, gate_mode=0, lower_bound=-5.0, scale=0.1)
    assert lib.kda_chunk_backward_scratch_bytes(ctypes.byref(p)) > limit
    rc = lib.kda_chunk_backward_noalloc(ctypes.byref(p), *([None] * 19), None)
    assert rc != 0 and "static array" in lib.kda_last_error().decode()
