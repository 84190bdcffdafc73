"""Shared helpers for the KDA parity tests: seeded inputs and error metrics."""

from __future__ import annotations

import numpy as np
import torch


def rel_err(actual, expected) -> float:
    """Norm-relative error ||a - e||_2 / ||e||_2 (float64)."""
    a = np.asarray(actual.detach().double().cpu() if torch.is_tensor(actual) else actual, np.float64)
    e = np.asarray(expected.detach().double().cpu() if torch.is_tensor(expected) else expected, np.float64)
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))


def cosine(actual, expected) -> float:
    a = np.asarray(actual.detach().double().cpu() if torch.is_tensor(actual) else actual, np.float64).ravel()
    e = np.asarray(expected.detach().double().cpu() if torch.is_tensor(expected) else expected, np.float64).ravel()
    na, ne = np.linalg.norm(a), np.linalg.norm(e)
    if na == 0 and ne == 0:
        return 1.0
    return float(a @ e / (na * ne))


def np64(t):
    return None if t is None else t.detach().double().cpu().numpy()


def mixer_oracle_weights(layer):
    """kda_oracle.full_layer keyword arguments of a KimiDeltaAttention layer (the layer
    multiplies with bf16 copies of its f32 weights)."""
    w = lambda m: np64(m.weight.bfloat16())  # noqa: E731
    c = lambda m: np64(m.weight[:, 0].bfloat16())  # noqa: E731
    return dict(q_weight=w(layer.q_proj), k_weight=w(layer.k_proj), v_weight=w(layer.v_proj),
                q_conv_weight=c(layer.q_conv1d), k_conv_weight=c(layer.k_conv1d), v_conv_weight=c(layer.v_conv1d),
                forget_a_weight=w(layer.f_a_proj), forget_b_weight=w(layer.f_b_proj), beta_weight=w(layer.b_proj),
                A_log=np64(layer.A_log), dt_bias=np64(layer.dt_bias), output_gate_weight=w(layer.g_proj),
                norm_weight=np64(layer.o_norm.weight), output_weight=w(layer.o_proj), num_heads=layer.num_heads,
                norm_eps=layer.o_norm.eps)


def make_kda_inputs(B, T, H, K, V, *, seed, gate="k3", state=False, dist="reference", device="cuda"):
    """Seeded bf16 activations, f32 params (built on the CPU, then moved).

    dist="reference": every activation ~N(0,1) (tests/test_kda_cuda.py:30-47).
    dist="baseline":  q,k L2-normalised, v ~N(0,1), beta logits ~N(0,1), and for
                      gate="precomputed" g = -exp(A_log) softplus(N(0,1)) with
                      A_log ~ U(-1,1).
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    v = torch.randn(B, T, H, V, generator=g)
    z = torch.randn(B, T, H, K, generator=g)
    beta = torch.randn(B, T, H, generator=g)
    if dist == "baseline":
        q = torch.nn.functional.normalize(q, dim=-1)
        k = torch.nn.functional.normalize(k, dim=-1)
        A_log = torch.rand(H, generator=g) * 2 - 1
        dt_bias = torch.zeros(H * K)
    else:
        A_log = torch.randn(H, generator=g) * 0.2
        dt_bias = torch.randn(H * K, generator=g) * 0.3
    if gate == "precomputed":
        gv = -A_log.exp().view(1, 1, H, 1) * torch.nn.functional.softplus(z + dt_bias.view(1, 1, H, K))
        gv = gv.float()
    else:
        gv = z.bfloat16()
    s0 = torch.randn(B, H, V, K, generator=g) * 0.05 if state else None
    out = dict(q=q.bfloat16(), k=k.bfloat16(), v=v.bfloat16(), g=gv, beta=beta.bfloat16(),
               A_log=A_log.float(), dt_bias=dt_bias.float(), s0=s0)
    return {n: (t.to(device) if t is not None else None) for n, t in out.items()}
