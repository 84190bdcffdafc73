"""CPU baseline: the reference's eager CPU path for the KDA operator, restated in torch.

TEST/BENCH INFRASTRUCTURE ONLY (imported by bench.py's cpu_baseline leg and tests).

Restates nanochat/mixers/kda.py:269-327 (``_reference_kda``): an f32 token loop of
einsums whose backward is PyTorch autograd through the loop — the path the reference
runs with ``mode="reference"`` and falls back to on CPU.  Timed on the host cores as a
reported baseline, never as the product.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def reference_kda_cpu(q, k, v, gate, beta_logits, A_log, dt_bias, *, initial_state=None,
                      lower_bound=-5.0, scale=None, gate_mode="k3"):
    """f32 token loop (nanochat/mixers/kda.py:286-327); returns (o, final state V-first)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    qf = F.normalize(q.float(), p=2, dim=-1) * scale
    kf = F.normalize(k.float(), p=2, dim=-1)
    vf = v.float()
    if gate_mode == "k3":
        decay = lower_bound * torch.sigmoid(A_log.float().exp().reshape(H, 1)
                                            * (gate.float() + dt_bias.float().reshape(H, K)))
    else:
        decay = gate.float()
    beta = beta_logits.float().sigmoid()
    if initial_state is None:
        state = torch.zeros(B, H, K, V, dtype=torch.float32)
    else:
        state = initial_state.float().transpose(-1, -2)
    outs = []
    for t in range(T):
        ki = kf[:, t]
        state = state * decay[:, t].exp().unsqueeze(-1)
        resid = vf[:, t] - torch.einsum("bhk,bhkv->bhv", ki, state)
        state = state + torch.einsum("bhk,bhv->bhkv", beta[:, t].unsqueeze(-1) * ki, resid)
        outs.append(torch.einsum("bhk,bhkv->bhv", qf[:, t], state))
    return torch.stack(outs, dim=1), state.transpose(-1, -2)


def time_fwd_bwd(B, T, H, K, V, *, repeats=3, seed=42, threads=None):
    """Median seconds of one f32 forward+backward at [B,T,H,K/V] on the CPU."""
    import statistics
    import time

    if threads:
        torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g).requires_grad_()
    k = torch.randn(B, T, H, K, generator=g).requires_grad_()
    v = torch.randn(B, T, H, V, generator=g).requires_grad_()
    z = torch.randn(B, T, H, K, generator=g).requires_grad_()
    bl = torch.randn(B, T, H, generator=g).requires_grad_()
    A_log = torch.zeros(H).requires_grad_()
    dt = torch.zeros(H * K).requires_grad_()
    do = torch.randn(B, T, H, V, generator=g)
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        o, _ = reference_kda_cpu(q, k, v, z, bl, A_log, dt)
        o.backward(do)
        times.append(time.perf_counter() - t0)
        for x in (q, k, v, z, bl, A_log, dt):
            x.grad = None
    return statistics.median(times)
