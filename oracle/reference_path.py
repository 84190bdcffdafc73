"""CPU baseline: the reference's eager CPU path for the KDA operator, restated in torch.

TEST/BENCH INFRASTRUCTURE ONLY (imported by bench.py's cpu_baseline leg and tests).

Restates nanochat/mixers/kda.py:269-327 (``_reference_kda``): an f32 loop over tokens
whose backward is PyTorch autograd through the loop -- the path the reference runs with
``mode="reference"`` and falls back to on CPU.  Timed on the host cores as a reported
baseline, never as the product.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def reference_kda_cpu(q, k, v, gate, beta_logits, A_log, dt_bias, *, initial_state=None,
                      lower_bound=-5.0, scale=None, gate_mode="k3"):
    """f32 token loop with a value-major state S [B,H,V,K]; returns (o, final state)."""
    n_b, n_t, n_h, n_k = q.shape
    n_v = v.shape[-1]
    qn = F.normalize(q.float(), dim=-1) * (n_k ** -0.5 if scale is None else scale)
    kn = F.normalize(k.float(), dim=-1)
    if gate_mode == "k3":
        bias = dt_bias.float().view(n_h, n_k)
        log_decay = lower_bound * torch.sigmoid(A_log.float().exp()[:, None] * (gate.float() + bias))
    else:
        log_decay = gate.float()
    decay = log_decay.exp()
    beta = torch.sigmoid(beta_logits.float())
    S = torch.zeros(n_b, n_h, n_v, n_k) if initial_state is None else initial_state.float()
    rows = []
    for t in range(n_t):
        S = S * decay[:, t, :, None, :]
        err = v[:, t].float() - torch.einsum("bhvk,bhk->bhv", S, kn[:, t])
        S = S + torch.einsum("bhv,bhk->bhvk", beta[:, t, :, None] * err, kn[:, t])
        rows.append(torch.einsum("bhvk,bhk->bhv", S, qn[:, t]))
    return torch.stack(rows, dim=1), S


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
