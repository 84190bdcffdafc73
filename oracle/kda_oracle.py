"""CPU oracle for the KDA operator path (numpy, float64).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product package (``experiment_swa_kda_amd``) never imports it and
never falls back to it.

Every function restates the reference algorithm of vpareek2/experiment_swa_kda
in plain numpy at float64:

* ``k3_decay_gate``            tests/kda_oracle.py:31-47, nanochat/mixers/kda.py:230-243
* ``l2_normalize``             torch.nn.functional.normalize semantics used at
                               tests/kda_oracle.py:83-84 (x / max(||x||, 1e-12))
* ``kda_forward``              tests/kda_oracle.py:50-127 (token loop, V-first state)
* ``kda_backward``             hand-derived reverse mode of the same loop; the
                               reference states it analytically in the token-serial
                               CUDA backward nanochat/mixers/cuda_kda/chunk.cu:578-870
* ``kda_forward_chunked``      chunked WY form of the same recurrence, following the
                               algebra of nanochat/mixers/cuda_kda/chunk_wy_forward.cu
                               (A/M build :125-405, U/W :761-863, state scan
                               :940-1276, output :1498-1588)
* ``kda_varlen_forward/backward``  per-sequence loop (the reference has no varlen;
                               sequences are independent with a state reset)
* ``causal_conv_forward/backward`` tests/kda_oracle.py:130-161 (state includes the
                               current token), nanochat/mixers/kda.py:136-212
* ``rmsnorm_gate_forward/backward`` tests/kda_oracle.py:164-173,
                               nanochat/mixers/kda.py:46-59
* ``softcap_cross_entropy``    the trainer's loss, nanochat/gpt.py:600-608
                               (softcap * tanh(logits / softcap), mean cross entropy
                               with ignore_index=-1)

Pinning (each function is checked by tests/test_oracle.py against something
other than its own formula):

* k3_decay_gate: bounds/monotonicity/endpoints (tests/test_kda_operator.py:62-74)
  and torch.sigmoid at float64.
* kda_forward: the one-token closed form, exact-key overwrite, decay-before-delta
  scalar closed form (tests/test_kda_operator.py:77-137), causal prefix and
  batch independence, and equality with the independent chunked WY algorithm.
* kda_backward: torch.autograd through a float64 torch statement of the loop and
  central finite differences of ``kda_forward``.
* causal_conv_*: torch.nn.functional.conv1d (grouped) and autograd; decode equals
  full sequence (tests/test_kda_operator.py:167-180).
* rmsnorm_gate_*: torch.nn.functional.rms_norm and autograd.
* softcap_cross_entropy: torch.nn.functional.cross_entropy (ignore_index, mean) at
  float64 and autograd through it; a uniform-logit closed form.
* full_layer: composed only of the functions above and matrix products; checked
  against the mixer's eager reference mode in tests/test_cpu_api.py.
"""

from __future__ import annotations

import numpy as np

NORM_EPS = 1e-12


# ----------------------------------------------------------------------------
# gate / normalisation primitives
# ----------------------------------------------------------------------------

def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-x[pos]))
    ex = np.exp(x[~pos])
    out[~pos] = ex / (1.0 + ex)
    return out


def k3_decay_gate(raw_gate, A_log, dt_bias, lower_bound=-5.0):
    """lb * sigmoid(exp(A_log[h]) * (raw + dt_bias[h, k]))  (tests/kda_oracle.py:31-47)."""
    raw_gate = np.asarray(raw_gate, np.float64)
    heads, key_dim = raw_gate.shape[-2:]
    A_log = np.asarray(A_log, np.float64).reshape(heads)
    bias = np.asarray(dt_bias, np.float64).reshape(heads, key_dim)
    if lower_bound >= 0:
        raise ValueError("lower_bound must be negative")
    return lower_bound * sigmoid(np.exp(A_log)[:, None] * (raw_gate + bias))


def k3_decay_gate_backward(raw_gate, A_log, dt_bias, lower_bound, dg):
    """VJP of k3_decay_gate -> (draw_gate, dA_log, ddt_bias) (chunk_wy_backward.cu:3802-3990)."""
    raw_gate = np.asarray(raw_gate, np.float64)
    heads, key_dim = raw_gate.shape[-2:]
    A = np.asarray(A_log, np.float64).reshape(heads)
    bias = np.asarray(dt_bias, np.float64).reshape(heads, key_dim)
    pre = raw_gate + bias
    s = sigmoid(np.exp(A)[:, None] * pre)
    dz = dg * lower_bound * s * (1.0 - s) * np.exp(A)[:, None]
    red = tuple(range(dz.ndim - 2))
    ddt = dz.sum(axis=red).reshape(-1)
    dA = (dz * pre).sum(axis=red).sum(axis=-1)
    return dz, dA, ddt


def l2_normalize(x):
    """x / max(||x||_2, 1e-12) over the last axis (F.normalize)."""
    x = np.asarray(x, np.float64)
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    return x / np.maximum(n, NORM_EPS)


def l2_normalize_backward(x, dy):
    x = np.asarray(x, np.float64)
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    clamped = n <= NORM_EPS
    nn_ = np.maximum(n, NORM_EPS)
    y = x / nn_
    dx = (dy - y * (y * dy).sum(-1, keepdims=True)) / nn_
    return np.where(clamped, dy / NORM_EPS, dx)


def _activate(q, k, v, gate, beta_logits, A_log, dt_bias, lower_bound, scale, gate_mode):
    key_dim = q.shape[-1]
    scale = key_dim ** -0.5 if scale is None else scale
    qn = l2_normalize(q) * scale
    kn = l2_normalize(k)
    if gate_mode == "k3":
        g = k3_decay_gate(gate, A_log, dt_bias, lower_bound)
    elif gate_mode == "logdecay":
        g = np.asarray(gate, np.float64)
    else:
        raise ValueError(f"unknown gate mode {gate_mode}")
    beta = sigmoid(beta_logits)
    return qn, kn, np.asarray(v, np.float64), g, beta, scale


# ----------------------------------------------------------------------------
# recurrence (token loop)
# ----------------------------------------------------------------------------

def kda_forward(q, k, v, gate, beta_logits, A_log=None, dt_bias=None, *, initial_state=None,
                lower_bound=-5.0, scale=None, gate_mode="k3"):
    """Token-loop KDA (tests/kda_oracle.py:50-127).

    q, k, gate: [B,T,H,K]; v: [B,T,H,V]; beta_logits: [B,T,H];
    initial_state: V-first [B,H,V,K].  Returns (o [B,T,H,V], final state [B,H,V,K]).
    ``gate_mode="logdecay"`` takes ``gate`` as the already-activated log decay g.
    """
    q = np.asarray(q, np.float64)
    B, T, H, K = q.shape
    V = np.asarray(v).shape[-1]
    qn, kn, v, g, beta, _ = _activate(q, k, v, gate, beta_logits, A_log, dt_bias,
                                      lower_bound, scale, gate_mode)
    if initial_state is None:
        S = np.zeros((B, H, K, V))
    else:
        S = np.asarray(initial_state, np.float64).transpose(0, 1, 3, 2).copy()
    out = np.zeros((B, T, H, V))
    for t in range(T):
        S = S * np.exp(g[:, t])[..., None]
        pred = np.einsum("bhk,bhkv->bhv", kn[:, t], S)
        resid = v[:, t] - pred
        S = S + np.einsum("bhk,bhv->bhkv", beta[:, t][..., None] * kn[:, t], resid)
        out[:, t] = np.einsum("bhk,bhkv->bhv", qn[:, t], S)
    return out, S.transpose(0, 1, 3, 2).copy()


def kda_backward(q, k, v, gate, beta_logits, A_log=None, dt_bias=None, *, initial_state=None,
                 grad_output=None, grad_final_state=None, lower_bound=-5.0, scale=None,
                 gate_mode="k3", checkpoint=64):
    """Reverse mode of ``kda_forward``.

    Returns (dq, dk, dv, dgate, dbeta_logits, dA_log, ddt_bias, dinitial_state).  For
    ``gate_mode="logdecay"`` dgate is dL/dg and dA_log/ddt_bias are None.  The
    per-token algebra mirrors the analytic token-serial backward of the reference
    (chunk.cu:578-870): dv = dr, dS1 = dS2 - k (x) dr, dg = e^g * sum_v S*dS1.
    States are recomputed from checkpoints every ``checkpoint`` tokens.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    B, T, H, K = q.shape
    V = np.asarray(v).shape[-1]
    qn, kn, vv, g, beta, scale = _activate(q, k, v, gate, beta_logits, A_log, dt_bias,
                                           lower_bound, scale, gate_mode)
    do = np.zeros((B, T, H, V)) if grad_output is None else np.asarray(grad_output, np.float64)
    if initial_state is None:
        S0 = np.zeros((B, H, K, V))
    else:
        S0 = np.asarray(initial_state, np.float64).transpose(0, 1, 3, 2).copy()

    def step(S, t):
        S1 = S * np.exp(g[:, t])[..., None]
        pred = np.einsum("bhk,bhkv->bhv", kn[:, t], S1)
        r = vv[:, t] - pred
        S2 = S1 + np.einsum("bhk,bhv->bhkv", beta[:, t][..., None] * kn[:, t], r)
        return S1, r, S2

    # forward pass storing checkpoints at multiples of `checkpoint`
    ckpts = {}
    S = S0
    for t in range(T):
        if t % checkpoint == 0:
            ckpts[t] = S
        S = step(S, t)[2]
    if grad_final_state is None:
        dS = np.zeros((B, H, K, V))
    else:
        dS = np.asarray(grad_final_state, np.float64).transpose(0, 1, 3, 2).copy()

    dqn = np.zeros_like(qn)
    dkn = np.zeros_like(kn)
    dv = np.zeros_like(vv)
    dg = np.zeros_like(g)
    dbeta = np.zeros_like(beta)
    for c0 in range(((T - 1) // checkpoint) * checkpoint if T else 0, -1, -checkpoint):
        c1 = min(c0 + checkpoint, T)
        states = [ckpts[c0]]
        for t in range(c0, c1 - 1):
            states.append(step(states[-1], t)[2])
        for t in range(c1 - 1, c0 - 1, -1):
            S_prev = states[t - c0]
            S1, r, S2 = step(S_prev, t)
            dS2 = dS + np.einsum("bhk,bhv->bhkv", qn[:, t], do[:, t])
            dqn[:, t] = np.einsum("bhkv,bhv->bhk", S2, do[:, t])
            dS2r = np.einsum("bhkv,bhv->bhk", dS2, r)
            dbeta[:, t] = (kn[:, t] * dS2r).sum(-1)
            dkn_t = beta[:, t][..., None] * dS2r
            dr = beta[:, t][..., None] * np.einsum("bhk,bhkv->bhv", kn[:, t], dS2)
            dv[:, t] = dr
            dkn_t -= np.einsum("bhkv,bhv->bhk", S1, dr)
            dkn[:, t] = dkn_t
            dS1 = dS2 - np.einsum("bhk,bhv->bhkv", kn[:, t], dr)
            eg = np.exp(g[:, t])
            dg[:, t] = eg * (S_prev * dS1).sum(-1)
            dS = dS1 * eg[..., None]

    dq = l2_normalize_backward(q, dqn * scale)
    dk = l2_normalize_backward(k, dkn)
    bl = np.asarray(beta_logits, np.float64)
    dbl = dbeta * beta * (1.0 - beta)
    if gate_mode == "k3":
        dgate, dA, ddt = k3_decay_gate_backward(gate, A_log, dt_bias, lower_bound, dg)
    else:
        dgate, dA, ddt = dg, None, None
    dS0 = dS.transpose(0, 1, 3, 2).copy()
    del bl
    return dq, dk, dv, dgate, dbl, dA, ddt, dS0


# ----------------------------------------------------------------------------
# chunked WY form (an independent algorithm for the same recurrence)
# ----------------------------------------------------------------------------

def kda_forward_chunked(q, k, v, gate, beta_logits, A_log=None, dt_bias=None, *,
                        initial_state=None, lower_bound=-5.0, scale=None, gate_mode="k3",
                        chunk=64):
    """Chunked WY forward (chunk_wy_forward.cu:125-405, 761-863, 940-1276, 1498-1588).

    Per chunk, with G = inclusive cumulative log decay inside the chunk:
      A[i,j] = sum_c qn[i,c] kn[j,c] exp(G[i,c]-G[j,c])        (j <= i)
      M[i,j] = beta[i] sum_c kn[i,c] kn[j,c] exp(G[i,c]-G[j,c])  (j <  i)
      T = (I + M)^-1,  U = T (beta v),  W = T (beta kn exp(G))
      delta = U - W S,  o = (qn exp(G)) S + A delta
      S <- diag(exp(G_last)) S + (kn exp(G_last - G))^T delta
    Pairwise exponents are formed as differences, never as exp(G) * exp(-G).
    """
    q = np.asarray(q, np.float64)
    B, T, H, K = q.shape
    V = np.asarray(v).shape[-1]
    qn, kn, vv, g, beta, _ = _activate(q, k, v, gate, beta_logits, A_log, dt_bias,
                                       lower_bound, scale, gate_mode)
    if initial_state is None:
        S = np.zeros((B, H, K, V))
    else:
        S = np.asarray(initial_state, np.float64).transpose(0, 1, 3, 2).copy()
    out = np.zeros((B, T, H, V))
    for c0 in range(0, T, chunk):
        c1 = min(c0 + chunk, T)
        n = c1 - c0
        # [B,H,n,K] views
        Q = qn[:, c0:c1].transpose(0, 2, 1, 3)
        Kc = kn[:, c0:c1].transpose(0, 2, 1, 3)
        Vc = vv[:, c0:c1].transpose(0, 2, 1, 3)
        bt = beta[:, c0:c1].transpose(0, 2, 1)
        G = np.cumsum(g[:, c0:c1].transpose(0, 2, 1, 3), axis=2)
        diff = G[:, :, :, None, :] - G[:, :, None, :, :]  # [B,H,i,j,K]
        lower = np.tril(np.ones((n, n)), 0)
        strict = np.tril(np.ones((n, n)), -1)
        E = np.exp(np.where(lower[None, None, :, :, None] > 0, diff, -np.inf))
        Amat = np.einsum("bhic,bhjc,bhijc->bhij", Q, Kc, E)
        Mmat = bt[..., None] * np.einsum("bhic,bhjc,bhijc->bhij", Kc, Kc, E) * strict
        Tm = np.linalg.inv(np.eye(n) + Mmat)
        U = Tm @ (bt[..., None] * Vc)
        W = Tm @ (bt[..., None] * Kc * np.exp(G))
        delta = U - W @ S
        O = (Q * np.exp(G)) @ S + Amat @ delta
        out[:, c0:c1] = O.transpose(0, 2, 1, 3)
        Glast = G[:, :, -1:, :]
        Kd = Kc * np.exp(Glast - G)
        S = np.exp(Glast[:, :, 0, :])[..., None] * S + Kd.transpose(0, 1, 3, 2) @ delta
    return out, S.transpose(0, 1, 3, 2).copy()


# ----------------------------------------------------------------------------
# packed variable-length sequences
# ----------------------------------------------------------------------------

def kda_varlen_forward(q, k, v, gate, beta_logits, A_log, dt_bias, cu_seqlens, *,
                       initial_state=None, lower_bound=-5.0, scale=None, gate_mode="k3"):
    """Packed [1,N,H,*] inputs; the state resets at each boundary of ``cu_seqlens``.

    Returns (o [1,N,H,V], final states [S,H,V,K]).  No reference counterpart exists;
    each sequence runs the token loop of tests/kda_oracle.py:50-127 independently.
    """
    cu = [int(x) for x in cu_seqlens]
    outs, finals = [], []
    for i in range(len(cu) - 1):
        a, b = cu[i], cu[i + 1]
        s0 = None if initial_state is None else np.asarray(initial_state)[i:i + 1]
        o, s = kda_forward(q[:, a:b], k[:, a:b], v[:, a:b], gate[:, a:b], beta_logits[:, a:b],
                           A_log, dt_bias, initial_state=s0, lower_bound=lower_bound,
                           scale=scale, gate_mode=gate_mode)
        outs.append(o)
        finals.append(s)
    return np.concatenate(outs, axis=1), np.concatenate(finals, axis=0)


def kda_varlen_backward(q, k, v, gate, beta_logits, A_log, dt_bias, cu_seqlens, *,
                        grad_output, grad_final_state=None, initial_state=None,
                        lower_bound=-5.0, scale=None, gate_mode="k3"):
    """Per-sequence backward of ``kda_varlen_forward``; parameter grads are summed."""
    cu = [int(x) for x in cu_seqlens]
    parts = []
    for i in range(len(cu) - 1):
        a, b = cu[i], cu[i + 1]
        s0 = None if initial_state is None else np.asarray(initial_state)[i:i + 1]
        gS = None if grad_final_state is None else np.asarray(grad_final_state)[i:i + 1]
        if b == a:
            # an empty sequence: final state = initial state, so its gradient passes through
            H, K, V = q.shape[2], q.shape[3], v.shape[3]
            z = lambda x: np.zeros((1, 0) + x.shape[2:])  # noqa: E731
            dS0 = np.zeros((1, H, V, K)) if gS is None else np.array(gS, dtype=np.float64)
            parts.append((z(q), z(k), z(v), z(gate), z(beta_logits), np.zeros_like(np.asarray(A_log, dtype=np.float64)),
                          np.zeros_like(np.asarray(dt_bias, dtype=np.float64)), dS0))
            continue
        parts.append(kda_backward(q[:, a:b], k[:, a:b], v[:, a:b], gate[:, a:b],
                                  beta_logits[:, a:b], A_log, dt_bias, initial_state=s0,
                                  grad_output=grad_output[:, a:b], grad_final_state=gS,
                                  lower_bound=lower_bound, scale=scale, gate_mode=gate_mode))
    cat = lambda idx: np.concatenate([p[idx] for p in parts], axis=1)  # noqa: E731
    dA = None if gate_mode != "k3" else sum(p[5] for p in parts)
    ddt = None if gate_mode != "k3" else sum(p[6] for p in parts)
    dS0 = np.concatenate([p[7] for p in parts], axis=0)
    return cat(0), cat(1), cat(2), cat(3), cat(4), dA, ddt, dS0


# ----------------------------------------------------------------------------
# depthwise causal short convolution + SiLU
# ----------------------------------------------------------------------------

def _silu(x):
    return x * sigmoid(x)


def causal_conv_forward(x, weight, initial_state=None, activation=True):
    """x [B,T,D], weight [D,W], state [B,D,W] incl. current token (tests/kda_oracle.py:130-161).

    Returns (y [B,T,D], final_state [B,D,W]).
    """
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    B, T, D = x.shape
    W = w.shape[-1]
    st = np.zeros((B, D, W)) if initial_state is None else np.asarray(initial_state, np.float64)
    # padded sequence: the W-1 most recent cached inputs, then x
    xp = np.concatenate([st[:, :, 1:].transpose(0, 2, 1), x], axis=1)  # [B, W-1+T, D]
    pre = np.zeros((B, T, D))
    for j in range(W):
        pre += xp[:, j:j + T] * w[None, None, :, j]
    y = _silu(pre) if activation else pre
    final = xp[:, -W:].transpose(0, 2, 1).copy() if T + W - 1 >= W else None
    return y, final


def causal_conv_backward(x, weight, grad_output, initial_state=None, grad_final_state=None,
                         activation=True):
    """Returns (dx, dweight, dinitial_state)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    B, T, D = x.shape
    W = w.shape[-1]
    st = np.zeros((B, D, W)) if initial_state is None else np.asarray(initial_state, np.float64)
    xp = np.concatenate([st[:, :, 1:].transpose(0, 2, 1), x], axis=1)
    pre = np.zeros((B, T, D))
    for j in range(W):
        pre += xp[:, j:j + T] * w[None, None, :, j]
    dy = np.asarray(grad_output, np.float64)
    if activation:
        s = sigmoid(pre)
        dpre = dy * (s * (1.0 + pre * (1.0 - s)))
    else:
        dpre = dy
    dxp = np.zeros_like(xp)
    dw = np.zeros_like(w)
    for j in range(W):
        dxp[:, j:j + T] += dpre * w[None, None, :, j]
        dw[:, j] = (dpre * xp[:, j:j + T]).sum(axis=(0, 1))
    if grad_final_state is not None:
        dxp[:, -W:] += np.asarray(grad_final_state, np.float64).transpose(0, 2, 1)
    dx = dxp[:, W - 1:]
    dst = np.zeros((B, D, W))
    dst[:, :, 1:] = dxp[:, :W - 1].transpose(0, 2, 1)
    return dx, dw, dst


# ----------------------------------------------------------------------------
# output RMSNorm * sigmoid(gate)
# ----------------------------------------------------------------------------

def rmsnorm_gate_forward(x, gate, weight, eps):
    """y = x * rsqrt(mean(x^2) + eps) * w * sigmoid(gate) (tests/kda_oracle.py:164-173)."""
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return x * inv * np.asarray(weight, np.float64) * sigmoid(gate), inv[..., 0]


def rmsnorm_gate_backward(x, gate, weight, eps, grad_output):
    """Returns (dx, dgate, dweight)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    D = x.shape[-1]
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    s = sigmoid(gate)
    n = x * inv
    dy = np.asarray(grad_output, np.float64)
    dn_w = dy * s  # grad wrt (n * w)
    dgate = dy * n * w * s * (1.0 - s)
    dw = (dn_w * n).reshape(-1, D).sum(0)
    dn = dn_w * w
    dx = inv * (dn - n * (dn * n).sum(-1, keepdims=True) / D)
    return dx, dgate, dw


def softcap_cross_entropy(logits, targets, vocab, softcap=15.0, ignore_index=-1):
    """Mean soft-capped cross entropy and its logit gradient (nanochat/gpt.py:600-608).

    logits [rows, stride] (columns >= vocab are padding), targets [rows].  Returns
    (loss, loss_rows, lse_rows, dlogits) with dlogits = d loss / d logits (zero in padding
    columns and ignored rows)."""
    x = np.asarray(logits, np.float64)
    t = np.asarray(targets, np.int64)
    th = np.tanh(x[:, :vocab] / softcap)
    z = softcap * th
    m = z.max(-1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(-1, keepdims=True)))[:, 0]
    valid = t != ignore_index
    rows = np.arange(x.shape[0])
    tz = np.where(valid, z[rows, np.where(valid, t, 0)], 0.0)
    loss_rows = np.where(valid, lse - tz, 0.0)
    count = valid.sum()
    loss = loss_rows.sum() / count if count else np.nan
    p = np.exp(z - lse[:, None])
    p[rows[valid], t[valid]] -= 1.0
    dz = np.where(valid[:, None], p, 0.0) / max(count, 1)
    d = np.zeros_like(x)
    d[:, :vocab] = dz * (1.0 - th * th)
    return loss, loss_rows, lse, d


# ----------------------------------------------------------------------------
# full mixer block
# ----------------------------------------------------------------------------

def full_layer(x, *, q_weight, k_weight, v_weight, q_conv_weight, k_conv_weight, v_conv_weight,
               forget_a_weight, forget_b_weight, beta_weight, A_log, dt_bias, output_gate_weight,
               norm_weight, output_weight, num_heads, norm_eps, initial_state=None,
               lower_bound=-5.0):
    """Independent composition of the K3 mixer (tests/kda_oracle.py:176-236).

    ``initial_state`` is None or a tuple (memory, q_conv, k_conv, v_conv).  Returns
    (output [B,T,D], (memory, q_conv, k_conv, v_conv)).
    """
    f = lambda a: np.asarray(a, np.float64)  # noqa: E731
    x = f(x)
    B, T, _ = x.shape
    st = (None, None, None, None) if initial_state is None else initial_state
    qp, kp, vp = x @ f(q_weight).T, x @ f(k_weight).T, x @ f(v_weight).T
    q, qf = causal_conv_forward(qp, q_conv_weight, st[1])
    k, kf = causal_conv_forward(kp, k_conv_weight, st[2])
    v, vf = causal_conv_forward(vp, v_conv_weight, st[3])
    K = q.shape[-1] // num_heads
    Vd = v.shape[-1] // num_heads
    q = q.reshape(B, T, num_heads, K)
    k = k.reshape(B, T, num_heads, K)
    v = v.reshape(B, T, num_heads, Vd)
    raw = ((x @ f(forget_a_weight).T) @ f(forget_b_weight).T).reshape(B, T, num_heads, K)
    bl = x @ f(beta_weight).T
    o, mem = kda_forward(q, k, v, raw, bl, A_log, dt_bias, initial_state=st[0], lower_bound=lower_bound)
    gate = (x @ f(output_gate_weight).T).reshape(B, T, num_heads, Vd)
    y, _ = rmsnorm_gate_forward(o, gate, norm_weight, norm_eps)
    return y.reshape(B, T, -1) @ f(output_weight).T, (mem, qf, kf, vf)


def full_layer_backward(x, grad_output, *, q_weight, k_weight, v_weight, q_conv_weight,
                        k_conv_weight, v_conv_weight, forget_a_weight, forget_b_weight,
                        beta_weight, A_log, dt_bias, output_gate_weight, norm_weight,
                        output_weight, num_heads, norm_eps, lower_bound=-5.0):
    """Reverse mode of ``full_layer`` (no initial state) by the chain rule through the
    pinned backward functions above and the projections' transposes
    (nanochat/mixers/kda.py:729-798 is the forward being differentiated).

    Returns a dict of gradients keyed like the mixer's parameters (``q_proj``,
    ``q_conv1d``, ``f_a_proj``, ``A_log``, ``o_norm``, ...) plus ``x``; weight gradients
    have the parameters' shapes ([out, in] for projections, [D, W] for convolutions).
    """
    f = lambda a: np.asarray(a, np.float64)  # noqa: E731
    x = f(x)
    B, T, C = x.shape
    x2 = x.reshape(-1, C)
    # forward, keeping what the backward needs
    qp, kp, vp = x @ f(q_weight).T, x @ f(k_weight).T, x @ f(v_weight).T
    q, _ = causal_conv_forward(qp, q_conv_weight)
    k, _ = causal_conv_forward(kp, k_conv_weight)
    v, _ = causal_conv_forward(vp, v_conv_weight)
    K = q.shape[-1] // num_heads
    Vd = v.shape[-1] // num_heads
    q4, k4, v4 = q.reshape(B, T, num_heads, K), k.reshape(B, T, num_heads, K), v.reshape(B, T, num_heads, Vd)
    fa = x @ f(forget_a_weight).T
    raw = (fa @ f(forget_b_weight).T).reshape(B, T, num_heads, K)
    bl = x @ f(beta_weight).T
    o, _ = kda_forward(q4, k4, v4, raw, bl, A_log, dt_bias, lower_bound=lower_bound)
    gate = (x @ f(output_gate_weight).T).reshape(B, T, num_heads, Vd)
    y, _ = rmsnorm_gate_forward(o, gate, norm_weight, norm_eps)
    y2 = y.reshape(-1, num_heads * Vd)
    # backward
    dout = f(grad_output).reshape(-1, f(output_weight).shape[0])
    g = {"o_proj": dout.T @ y2}
    dy = (dout @ f(output_weight)).reshape(B, T, num_heads, Vd)
    do, dgate, g["o_norm"] = rmsnorm_gate_backward(o, gate, norm_weight, norm_eps, dy)
    dgate2 = dgate.reshape(-1, num_heads * Vd)
    g["g_proj"] = dgate2.T @ x2
    dx = dgate2 @ f(output_gate_weight)
    dq, dk, dv, draw, dbl, g["A_log"], ddt, _ = kda_backward(
        q4, k4, v4, raw, bl, A_log, dt_bias, grad_output=do, lower_bound=lower_bound)
    g["dt_bias"] = np.asarray(ddt).reshape(np.shape(dt_bias))
    dbl2 = dbl.reshape(-1, num_heads)
    g["b_proj"] = dbl2.T @ x2
    dx = dx + dbl2 @ f(beta_weight)
    draw2 = draw.reshape(-1, num_heads * K)
    g["f_b_proj"] = draw2.T @ fa.reshape(-1, fa.shape[-1])
    dfa = draw2 @ f(forget_b_weight)
    g["f_a_proj"] = dfa.T @ x2
    dx = dx + dfa @ f(forget_a_weight)
    for name, pre, w_proj, w_conv, d in (("q", qp, q_weight, q_conv_weight, dq),
                                         ("k", kp, k_weight, k_conv_weight, dk),
                                         ("v", vp, v_weight, v_conv_weight, dv)):
        dpre, g[f"{name}_conv1d"], _ = causal_conv_backward(pre, w_conv, d.reshape(B, T, -1))
        dpre2 = dpre.reshape(-1, dpre.shape[-1])
        g[f"{name}_proj"] = dpre2.T @ x2
        dx = dx + dpre2 @ f(w_proj)
    g["x"] = dx.reshape(B, T, C)
    return g
