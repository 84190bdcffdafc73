"""CPU tests of the host side: C-ABI exports, API contracts, error behaviour, and the
explicit eager reference mode against the oracle (no GPU compute)."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import experiment_swa_kda_amd as kmod
from experiment_swa_kda_amd import _lib
from experiment_swa_kda_amd.kda import KDAState, KimiDeltaAttention, k3_decay_gate, kda
from oracle import kda_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "kda_mi355x.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kda_\w+)\s*\(", text)))


@pytest.mark.skipif(not _lib.is_built(), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    syms = header_symbols()
    assert len(syms) >= 14
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in include/kda_mi355x.h but not exported"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


@pytest.mark.skipif(not _lib.is_built(), reason="library not built")
def test_c_abi_rejects_bad_problems_without_gpu():
    lib = _lib.load()
    p = _lib.ChunkProblem(batch=1, seq_len=8, heads=1, key_dim=257, value_dim=64, num_seqs=1,
                          cu_seqlens=None, gate_mode=0, lower_bound=-5.0, scale=0.1)
    assert lib.kda_chunk_workspace_bytes(ctypes.byref(p)) == 0
    assert "key_dim" in lib.kda_last_error().decode()
    # head dims other than 64 / 128 take the token-serial kernels: state checkpoints every
    # 16 tokens as the workspace, per-wave gradient partials as the backward scratch
    p.key_dim = 96
    assert lib.kda_chunk_workspace_bytes(ctypes.byref(p)) >= 1 * 1 * 64 * 96 * 4
    assert lib.kda_chunk_backward_scratch_bytes(ctypes.byref(p)) >= 16 * 8 * (3 * 96 + 1) * 4
    p.value_dim = 0
    assert lib.kda_chunk_workspace_bytes(ctypes.byref(p)) == 0
    assert "value_dim" in lib.kda_last_error().decode()
    p.value_dim = 64
    p.key_dim = 64
    assert lib.kda_chunk_workspace_bytes(ctypes.byref(p)) > 0
    rc = lib.kda_chunk_forward(ctypes.byref(p), *([None] * 11), None)
    assert rc != 0 and "null" in lib.kda_last_error().decode()
    p.num_seqs = 2
    rc = lib.kda_chunk_forward(ctypes.byref(p), *([None] * 11), None)
    assert rc != 0 and "num_seqs" in lib.kda_last_error().decode()
    assert lib.kda_causal_conv_forward(1, 4, 12, 4, None, None, None, None, None, None) != 0
    assert "multiple of 8" in lib.kda_last_error().decode()
    assert lib.kda_rmsnorm_gate_forward(4, 96, None, None, None, 1e-5, None, None, None) != 0
    assert "null" in lib.kda_last_error().decode()
    assert lib.kda_rmsnorm_gate_forward(4, 1025, None, None, None, 1e-5, None, None, None) != 0
    assert "dim" in lib.kda_last_error().decode()
    assert lib.kda_recurrent_decode(1, 1, 32, 64, 0, -5.0, 0.1, *([None] * 10), None) != 0
    assert lib.kda_recurrent_decode(1, 1, 257, 64, 0, -5.0, 0.1, *([None] * 10), None) != 0
    assert "key_dim" in lib.kda_last_error().decode()
    # a gradient row stride shorter than a token's H * max(K, V) values is refused before any
    # launch (the pointers are never dereferenced)
    p = _lib.ChunkProblem(batch=1, seq_len=8, heads=2, key_dim=64, value_dim=64, num_seqs=1, cu_seqlens=None,
                          gate_mode=1, lower_bound=-5.0, scale=0.125, grad_row_stride=64)
    fake = ctypes.c_void_p(1 << 20)
    rc = lib.kda_chunk_backward(ctypes.byref(p), *([fake] * 20), None)
    assert rc != 0 and "grad_row_stride" in lib.kda_last_error().decode()
    # the beta / norm-gate row strides are checked the same way
    for field, value, words in (("beta_row_stride", 1, "beta_row_stride"), ("beta_grad_pad", 3, "beta_grad_pad"),
                                ("norm_gate_row_stride", 100, "norm_gate_row_stride")):
        p = _lib.ChunkProblem(batch=1, seq_len=8, heads=2, key_dim=64, value_dim=64, num_seqs=1, cu_seqlens=None,
                              gate_mode=1, lower_bound=-5.0, scale=0.125, **{field: value})
        rc = lib.kda_chunk_backward(ctypes.byref(p), *([fake] * 20), None)
        assert rc != 0 and words in lib.kda_last_error().decode()
    rc = lib.kda_rmsnorm_gate_backward_strided(9, 64, 3, *([fake] * 2), 64, *([fake] * 3), 1e-5, fake, fake, 192,
                                               fake, fake, None)
    assert rc != 0 and "strides" in lib.kda_last_error().decode()


def make(B=2, T=7, H=2, K=4, V=3, seed=1729, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return dict(
        q=torch.randn(B, T, H, K, generator=g, dtype=dtype),
        k=torch.randn(B, T, H, K, generator=g, dtype=dtype),
        v=torch.randn(B, T, H, V, generator=g, dtype=dtype),
        g=torch.randn(B, T, H, K, generator=g, dtype=dtype),
        beta=torch.randn(B, T, H, generator=g, dtype=dtype),
        A_log=torch.randn(H, generator=g, dtype=dtype) * 0.2,
        dt_bias=torch.randn(H, K, generator=g, dtype=dtype) * 0.3,
        s0=torch.randn(B, H, V, K, generator=g, dtype=dtype) * 0.1,
    )


def call(d, **kw):
    return kda(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"],
               initial_state=d["s0"], output_final_state=True, mode="reference", **kw)


def n64(t):
    return t.detach().double().numpy()


@pytest.mark.parametrize("shape", [(1, 1, 1, 4, 3), (2, 7, 2, 4, 3), (1, 64, 2, 16, 11)])
def test_reference_mode_matches_oracle(shape):
    # tests/test_kda_operator.py:199-218
    d = make(*shape)
    o, s = call(d)
    eo, es = O.kda_forward(n64(d["q"]), n64(d["k"]), n64(d["v"]), n64(d["g"]), n64(d["beta"]),
                           n64(d["A_log"]), n64(d["dt_bias"]), initial_state=n64(d["s0"]))
    assert o.shape == shape[:3] + (shape[4],) and s.shape == (shape[0], shape[2], shape[4], shape[3])
    assert s.dtype == torch.float32
    np.testing.assert_allclose(n64(o), eo, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(n64(s), es, atol=1e-5, rtol=1e-5)


def test_reference_mode_gradients_match_oracle():
    # tests/test_kda_operator.py:221-248
    d = {k_: v_.clone().requires_grad_(True) for k_, v_ in make(1, 5, 2, 4, 3).items()}
    o, s = call(d)
    r = np.random.default_rng(0)
    do, ds = r.standard_normal(o.shape), r.standard_normal(s.shape)
    names = ["q", "k", "v", "g", "beta", "A_log", "dt_bias", "s0"]
    got = torch.autograd.grad((o, s), [d[x] for x in names], (torch.tensor(do).float(), torch.tensor(ds).float()))
    exp = O.kda_backward(*(n64(d[x]) for x in names[:7]), initial_state=n64(d["s0"]), grad_output=do,
                         grad_final_state=ds)
    for name, a, e in zip(names, got, exp):
        np.testing.assert_allclose(n64(a), np.asarray(e).reshape(a.shape), atol=2e-4, rtol=2e-4, err_msg=name)


def test_k3_gate_matches_oracle_and_bounds():
    raw = torch.randn(2, 3, 2, 4, dtype=torch.float64)
    A = torch.randn(2, dtype=torch.float64)
    b = torch.randn(2, 4, dtype=torch.float64)
    np.testing.assert_allclose(k3_decay_gate(raw, A, b).numpy(), O.k3_decay_gate(raw.numpy(), A.numpy(), b.numpy()),
                               rtol=1e-12, atol=1e-14)
    with pytest.raises(ValueError, match="negative"):
        k3_decay_gate(raw, A, b, lower_bound=0.0)


def test_contract_errors():
    d = make(1, 2, 2, 4, 3)
    d["s0"] = torch.zeros(1, 2, 4, 3)
    with pytest.raises(ValueError, match=r"V-first|\[B, H, V, K\]"):
        call(d)
    d = make(1, 2, 2, 4, 3)
    with pytest.raises(ValueError, match="unknown KDA mode"):
        kda(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"], mode="flash")
    with pytest.raises(ValueError, match="A_log"):
        kda(d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"][:1], d["dt_bias"])
    with pytest.raises(ValueError, match="beta logits"):
        kda(d["q"], d["k"], d["v"], d["g"], d["beta"][..., :1], d["A_log"], d["dt_bias"])


@pytest.mark.parametrize("mode", ["project_chunk", "project_recurrent"])
def test_project_modes_fail_closed_on_cpu(mode, monkeypatch):
    # project_* modes never fall back to the eager loop, whatever allow_fallback says
    # (reference kda.py:588-598)
    import importlib

    impl = importlib.import_module("experiment_swa_kda_amd.kda")

    def forbidden(*args, **kwargs):
        raise AssertionError("project call reached the eager loop")

    monkeypatch.setattr(impl, "_reference_kda", forbidden)
    d = make(1, 3, 2, 64, 64)
    with pytest.raises(RuntimeError, match="project CUDA KDA backend unavailable"):
        kda(d["q"].bfloat16(), d["k"].bfloat16(), d["v"].bfloat16(), d["g"].bfloat16(), d["beta"].bfloat16(),
            d["A_log"], d["dt_bias"], mode=mode, allow_fallback=True)


@pytest.mark.parametrize("mode", ["chunk", "recurrent"])
def test_optimized_modes_fallback_contract_on_cpu(mode):
    # reference kda.py:633-673: an unsupported chunk/recurrent call raises with
    # allow_fallback=False and runs the eager loop with allow_fallback=True
    d = make(1, 5, 2, 8, 8)
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], d["A_log"], d["dt_bias"])
    with pytest.raises(RuntimeError, match=f"optimized {mode} KDA backend unavailable"):
        kda(*args, initial_state=d["s0"], output_final_state=True, mode=mode, allow_fallback=False)
    got, got_state = kda(*args, initial_state=d["s0"], output_final_state=True, mode=mode)
    want, want_state = kda(*args, initial_state=d["s0"], output_final_state=True, mode="reference")
    assert torch.equal(got, want) and torch.equal(got_state, want_state)
    out, none_state = kda(*args, mode=mode)
    assert none_state is None and out.shape == d["v"].shape


def test_layer_recurrent_mode_token_decode_matches_full_sequence():
    # restates tests/test_kda_layer.py:148-169: mode="recurrent" on CPU falls back to the
    # eager loop; decoding one token at a time equals the full-sequence reference forward
    layer = KimiDeltaAttention(16, 2, 8, conv_size=4, layer_idx=0, mode="reference")
    gen = torch.Generator().manual_seed(314159)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.08)
        layer.A_log.copy_(torch.tensor([-0.2, 0.15]))
        layer.dt_bias.copy_(torch.linspace(-0.4, 0.3, 16))
    layer.eval()
    x = torch.randn(2, 11, 16, generator=torch.Generator().manual_seed(19))
    full, full_state = layer(x, state=None, output_final_state=True, mode="reference")
    state, pieces = None, []
    for t in range(x.shape[1]):
        piece, state = layer(x[:, t:t + 1], state=state, output_final_state=True, mode="recurrent")
        pieces.append(piece)
    torch.testing.assert_close(torch.cat(pieces, 1), full, atol=3e-5, rtol=3e-5)
    for a, b in ((state.memory, full_state.memory), (state.q_conv, full_state.q_conv),
                 (state.k_conv, full_state.k_conv), (state.v_conv, full_state.v_conv)):
        torch.testing.assert_close(a, b, atol=3e-5, rtol=3e-5)


def test_layer_structure_and_reference_forward_matches_oracle():
    # tests/test_kda_layer.py:85-145
    layer = KimiDeltaAttention(16, 2, 8, conv_size=4, layer_idx=0, mode="reference")
    gen = torch.Generator().manual_seed(314159)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.08)
        layer.A_log.copy_(torch.tensor([-0.2, 0.15]))
        layer.dt_bias.copy_(torch.linspace(-0.4, 0.3, 16))
    assert layer.g_proj.weight.shape == (16, 16) and layer.f_a_proj.weight.shape == (8, 16)
    assert layer.q_conv1d.groups == 16 and layer.q_conv1d.kernel_size == (4,)
    x = torch.randn(2, 9, 16, generator=torch.Generator().manual_seed(7))
    y, st = layer(x, state=None, output_final_state=True, mode="reference")
    w = lambda m: n64(m.weight)  # noqa: E731
    ey, (mem, qf, kf, vf) = O.full_layer(
        n64(x), q_weight=w(layer.q_proj), k_weight=w(layer.k_proj), v_weight=w(layer.v_proj),
        q_conv_weight=n64(layer.q_conv1d.weight[:, 0]), k_conv_weight=n64(layer.k_conv1d.weight[:, 0]),
        v_conv_weight=n64(layer.v_conv1d.weight[:, 0]), forget_a_weight=w(layer.f_a_proj),
        forget_b_weight=w(layer.f_b_proj), beta_weight=w(layer.b_proj), A_log=n64(layer.A_log),
        dt_bias=n64(layer.dt_bias), output_gate_weight=w(layer.g_proj), norm_weight=n64(layer.o_norm.weight),
        output_weight=w(layer.o_proj), num_heads=2, norm_eps=1e-5)
    assert isinstance(st, KDAState) and st.memory.shape == (2, 2, 8, 8) and st.q_conv.shape == (2, 16, 4)
    np.testing.assert_allclose(n64(y), ey, atol=2e-5, rtol=2e-5)
    for a, e in ((st.memory, mem), (st.q_conv, qf), (st.k_conv, kf), (st.v_conv, vf)):
        np.testing.assert_allclose(n64(a), e, atol=2e-5, rtol=2e-5)


def test_layer_nonzero_state_not_mutated_and_causal():
    layer = KimiDeltaAttention(16, 2, 8, mode="reference")
    g = torch.Generator().manual_seed(23)
    st = KDAState(torch.randn(2, 2, 8, 8, generator=g), torch.randn(2, 16, 4, generator=g),
                  torch.randn(2, 16, 4, generator=g), torch.randn(2, 16, 4, generator=g))
    orig = [t.clone() for t in (st.memory, st.q_conv, st.k_conv, st.v_conv)]
    x = torch.randn(2, 5, 16, generator=g)
    layer(x, state=st, output_final_state=True)
    for a, b in zip((st.memory, st.q_conv, st.k_conv, st.v_conv), orig):
        assert torch.equal(a, b)
    x2 = x.clone()
    x2[:, 3:] = torch.randn(2, 2, 16, generator=g)
    a, _ = layer(x)
    b, _ = layer(x2)
    assert torch.equal(a[:, :3], b[:, :3])


def test_provenance_names_native_symbols():
    prov = kmod.kda_backend_provenance()
    syms = set(header_symbols())
    for comp, entry in prov["components"].items():
        assert entry["owner"] == "project"
        assert entry["symbol"] in syms, comp


def test_kv_cache_contract_on_cpu():
    """The decode cache keeps the reference KVCache's KDA-layer contract
    (nanochat/engine.py:92-221): per-layer KDAState slots, type checks, position, reset."""
    from experiment_swa_kda_amd.model import KVCache
    from experiment_swa_kda_amd.kda import KDAState
    c = KVCache(2, 3, 64, 128, 4, "cpu", torch.bfloat16)
    assert c.allocated_kda_layers == (0, 1, 2, 3) and c.get_pos() == 0
    with pytest.raises(TypeError):
        c.set_kda_state(1, "not a state")
    with pytest.raises(ValueError):
        c.get_kda_state(7)
    with pytest.raises(ValueError):
        c.get_layer_cache(0)
    st = KDAState(torch.zeros(2, 3, 128, 128), torch.zeros(2, 384, 4), torch.zeros(2, 384, 4), torch.zeros(2, 384, 4))
    c.set_kda_state(2, st)
    c.advance(5)
    assert c.get_pos() == 5 and c.get_kda_state(2) is st
    assert c.state_nbytes() == (2 * 3 * 128 * 128 + 3 * 2 * 384 * 4) * 4
    c.reset()
    assert c.get_pos() == 0 and c.get_kda_state(2) is None
    with pytest.raises(ValueError):
        KVCache(1, 3, 64, 128, 2, "cpu", torch.bfloat16, mixer_types="KS")


def test_build_refuses_vgpr_spills():
    """The build's spill check reads hipcc's kernel-resource-usage remarks per kernel."""
    from experiment_swa_kda_amd.build import vgpr_spills

    remarks = "\n".join([
        "x.hip:1:1: remark: Function Name: _Z1av [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: _Z1bv [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     SGPRs Spill: 16 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     VGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert vgpr_spills(remarks) == {"_Z1bv": 3}
    assert vgpr_spills("") == {}


def test_gemm_selection_file_is_pinned_to_gfx950():
    """The committed TunableOp table names the stack it was tuned on and holds the
    trainer's lm_head shape (8192 tokens x 384 -> 32768)."""
    import os
    from experiment_swa_kda_amd import model
    lines = open(model.GEMM_SELECTION_FILE).read().splitlines()
    val = {l.split(",")[1]: l.split(",", 2)[2] for l in lines if l.startswith("Validator,")}
    assert val["GCN_ARCH_NAME"].startswith("gfx950")
    assert {"PT_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION"} <= set(val)
    assert any(",tn_32768_8192_384_" in l for l in lines)
    assert os.path.basename(model.GEMM_SELECTION_FILE) == "gemm_selection_gfx950.csv"
