"""Torch-facing wrappers of the MI355X KDA kernels and the ``nanochat_kda`` operator set.

PyTorch is only plumbing here: it allocates device memory and provides the current HIP
stream.  Every compute call goes through the C ABI of libkda_mi355x.so (``_lib``); there
is no eager or CPU fallback, and a missing library raises RuntimeError.

The ``torch.ops.nanochat_kda`` registrations reproduce the reference schemas
(nanochat/mixers/cuda_kda/chunk.cu:2117-2134, recurrent_decode.cu:185-194,
causal_convolution_forward.cu:241-244, causal_convolution_backward.cu:455-460,
rmsnorm_gate.cu:277-284).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import ChunkProblem, KDA_GATE_K3, KDA_GATE_LOGDECAY, check, ptr

GATE_MODES = {"k3": KDA_GATE_K3, "precomputed": KDA_GATE_LOGDECAY}


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(what: str, *tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{what}: tensors must be on a ROCm device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: all tensors must be on the same device")
    if dev is None:
        raise RuntimeError(f"{what}: no device tensor given")
    return dev


def _c(t):
    """Contiguous and 16-byte aligned (the kernels move 16-byte vectors): a view with an
    unaligned storage offset is copied."""
    if t is None:
        return None
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _check_dtype(what, t, dtype, name):
    if t is not None and t.dtype != dtype:
        raise RuntimeError(f"{what}: {name} must be {dtype}, got {t.dtype}")


# ---------------------------------------------------------------------------
# chunked forward / backward
# ---------------------------------------------------------------------------

def _problem(q, v, cu_seqlens, gate_mode, lower_bound, scale) -> ChunkProblem:
    B, T, H, K = q.shape
    V = v.shape[-1]
    p = ChunkProblem()
    p.batch, p.seq_len, p.heads, p.key_dim, p.value_dim = B, T, H, K, V
    if cu_seqlens is None:
        p.num_seqs = B
        p.cu_seqlens = None
    else:
        p.num_seqs = cu_seqlens.numel() - 1
        p.cu_seqlens = cu_seqlens.data_ptr()
    p.gate_mode = gate_mode
    p.lower_bound = float(lower_bound)
    p.scale = float(scale)
    return p


def _check_chunk_inputs(what, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state,
                        cu_seqlens, gate_mode):
    dev = _require_cuda(what, q, k, v, gate, beta_logits, A_log, dt_bias, initial_state, cu_seqlens)
    for name, t in (("q", q), ("k", k), ("v", v), ("beta_logits", beta_logits)):
        _check_dtype(what, t, torch.bfloat16, name)
    _check_dtype(what, gate, torch.bfloat16 if gate_mode == KDA_GATE_K3 else torch.float32, "gate")
    if gate_mode == KDA_GATE_K3:
        if A_log is None or dt_bias is None:
            raise RuntimeError(f"{what}: the K3 gate needs A_log and dt_bias")
        _check_dtype(what, A_log, torch.float32, "A_log")
        _check_dtype(what, dt_bias, torch.float32, "dt_bias")
    _check_dtype(what, initial_state, torch.float32, "initial_state")
    if q.ndim != 4 or k.shape != q.shape or gate.shape != q.shape:
        raise RuntimeError(f"{what}: q, k and gate must share shape [B, T, H, K]")
    B, T, H, K = q.shape
    if v.ndim != 4 or v.shape[:3] != q.shape[:3]:
        raise RuntimeError(f"{what}: v must have shape [B, T, H, V]")
    if beta_logits.shape != q.shape[:3]:
        raise RuntimeError(f"{what}: beta_logits must have shape [B, T, H]")
    if not (1 <= K <= 256 and 1 <= v.shape[-1] <= 4096):
        raise RuntimeError(f"{what}: head dimensions must be K in [1, 256] and V in [1, 4096] "
                           f"(got K={K}, V={v.shape[-1]})")
    n = B if cu_seqlens is None else cu_seqlens.numel() - 1
    if cu_seqlens is not None:
        if B != 1:
            raise RuntimeError(f"{what}: cu_seqlens requires batch size 1")
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
            raise RuntimeError(f"{what}: cu_seqlens must be a 1-D int32 tensor with >= 2 entries")
    if initial_state is not None and initial_state.shape != (n, H, v.shape[-1], K):
        raise RuntimeError(f"{what}: initial_state must be V-first [N, H, V, K] = {(n, H, v.shape[-1], K)}")
    return dev


def _output_bytes(B, T, H, V):
    """Byte offset of the residual workspace when it lives behind the output tensor."""
    return (B * T * H * V * 2 + 255) // 256 * 256


def chunk_forward(q, k, v, gate_values, beta_logits, A_log, dt_bias, initial_state,
                  output_final_state, lower_bound, scale, *, cu_seqlens=None, gate="k3",
                  residuals_behind_output=False):
    """Chunked forward.  Returns (output, final_state or None, workspace).

    ``gate_values`` is the bf16 raw gate (``gate="k3"``) or the f32 log decay
    (``gate="precomputed"``).  The workspace holds the residuals that
    :func:`chunk_backward` consumes.  With ``residuals_behind_output`` the output and
    the workspace share one allocation (output first, the workspace at the next 256-byte
    boundary), so a caller that keeps only the output keeps the residuals too: the
    ``torch.ops.nanochat_kda`` schemas pass no workspace between forward and backward.
    """
    gm = GATE_MODES[gate]
    dev = _check_chunk_inputs("chunk_forward", q, k, v, gate_values, beta_logits, A_log, dt_bias,
                              initial_state, cu_seqlens, gm)
    q, k, v, gate_values, beta_logits = (_c(t) for t in (q, k, v, gate_values, beta_logits))
    A_log, dt_bias, initial_state = _c(A_log), _c(dt_bias), _c(initial_state)
    B, T, H, K = q.shape
    V = v.shape[-1]
    n = B if cu_seqlens is None else cu_seqlens.numel() - 1
    p = _problem(q, v, cu_seqlens, gm, lower_bound, scale)
    lib = _lib.load()
    ws_bytes = lib.kda_chunk_workspace_bytes(ctypes.byref(p))
    if ws_bytes == 0 and (B * T > 0 or n > 0):
        check(1, "chunk_workspace_bytes")
    if residuals_behind_output:
        off = _output_bytes(B, T, H, V)
        buf = torch.empty(off + max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        output = buf[:B * T * H * V * 2].view(torch.bfloat16).view(B, T, H, V)
        workspace = buf[off:]
    else:
        workspace = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        output = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    final_state = torch.empty(n, H, V, K, dtype=torch.float32, device=dev) if output_final_state else None
    with torch.cuda.device(dev):
        rc = lib.kda_chunk_forward(
            ctypes.byref(p), ptr(q), ptr(k), ptr(v), ptr(gate_values), ptr(beta_logits),
            ptr(A_log), ptr(dt_bias), ptr(initial_state), ptr(output), ptr(final_state),
            ptr(workspace), _stream(dev))
    check(rc, "kda_chunk_forward")
    return output, final_state, workspace


def chunk_forward_norm_gate(q, k, v, gate_values, beta_logits, A_log, dt_bias, initial_state,
                            output_final_state, lower_bound, scale, norm_gate, norm_weight, eps, *,
                            cu_seqlens=None, gate="k3"):
    """Chunked forward with the output RMSNorm * weight * sigmoid(norm_gate) fused into its
    last kernel.  Returns (output o, normed output, inverse_rms, final_state or None,
    workspace): o and inverse_rms are what :func:`rmsnorm_gate_backward` needs."""
    gm = GATE_MODES[gate]
    dev = _check_chunk_inputs("chunk_forward_norm_gate", q, k, v, gate_values, beta_logits, A_log,
                              dt_bias, initial_state, cu_seqlens, gm)
    _check_dtype("chunk_forward_norm_gate", norm_gate, torch.bfloat16, "norm_gate")
    _check_dtype("chunk_forward_norm_gate", norm_weight, torch.float32, "norm_weight")
    if norm_gate.shape != v.shape or norm_weight.shape != (v.shape[-1],):
        raise RuntimeError("chunk_forward_norm_gate: norm_gate must be shaped like v and norm_weight [V]")
    q, k, v, gate_values, beta_logits = (_c(t) for t in (q, k, v, gate_values, beta_logits))
    A_log, dt_bias, initial_state = _c(A_log), _c(dt_bias), _c(initial_state)
    norm_gate, norm_weight = _c(norm_gate), _c(norm_weight)
    B, T, H, K = q.shape
    V = v.shape[-1]
    n = B if cu_seqlens is None else cu_seqlens.numel() - 1
    p = _problem(q, v, cu_seqlens, gm, lower_bound, scale)
    lib = _lib.load()
    ws_bytes = lib.kda_chunk_workspace_bytes(ctypes.byref(p))
    if ws_bytes == 0 and (B * T > 0 or n > 0):
        check(1, "chunk_workspace_bytes")
    workspace = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    output = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    normed = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    inv = torch.empty(B * T * H, dtype=torch.float32, device=dev)
    final_state = torch.empty(n, H, V, K, dtype=torch.float32, device=dev) if output_final_state else None
    with torch.cuda.device(dev):
        rc = lib.kda_chunk_forward_norm_gate(
            ctypes.byref(p), ptr(q), ptr(k), ptr(v), ptr(gate_values), ptr(beta_logits),
            ptr(A_log), ptr(dt_bias), ptr(initial_state), ptr(output), ptr(final_state),
            ptr(workspace), ptr(norm_gate), ptr(norm_weight), float(eps), ptr(normed), ptr(inv),
            _stream(dev))
    check(rc, "kda_chunk_forward_norm_gate")
    return output, normed, inv, final_state, workspace


def chunk_forward_conv_norm_gate(qkv_in, conv_weight, gate_values, beta_logits, A_log, dt_bias,
                                 lower_bound, scale, norm_gate, norm_weight, eps, heads, *, gate="k3"):
    """:func:`chunk_forward_norm_gate` with the short convolution + SiLU of q, k, v computed
    by the chunk forward's first kernel (stateless path: no convolution or recurrent state).
    ``qkv_in`` [B,T,3HK] bf16 holds the pre-convolution q, k, v projections side by side; it
    may be a column slice of a wider row (unit channel stride, row stride a multiple of 8).
    ``conv_weight`` [3HK, W] bf16, W <= 4.  Returns (q, k, v, o, normed, inverse_rms,
    workspace) with q, k, v the post-SiLU activations [B,T,H,K], bit-identical to
    :func:`causal_conv_forward`'s."""
    gm = GATE_MODES[gate]
    what = "chunk_forward_conv_norm_gate"
    dev = _require_cuda(what, qkv_in, conv_weight, gate_values, beta_logits, A_log, dt_bias, norm_gate,
                        norm_weight)
    _check_dtype(what, qkv_in, torch.bfloat16, "qkv_in")
    _check_dtype(what, conv_weight, torch.bfloat16, "conv_weight")
    B, T, C3 = qkv_in.shape
    H = int(heads)
    if C3 % (3 * H):
        raise RuntimeError(f"{what}: qkv_in width {C3} is not 3 * heads * head_dim")
    D = C3 // (3 * H)
    if conv_weight.ndim != 2 or conv_weight.shape[0] != C3 or not 1 <= conv_weight.shape[1] <= 4:
        raise RuntimeError(f"{what}: conv_weight must be [3HK, W] with W in [1, 4]")
    if _row_stride(qkv_in) is None:
        qkv_in = qkv_in.contiguous()
    ld = _row_stride(qkv_in)
    q = torch.empty(B, T, H, D, dtype=torch.bfloat16, device=dev)
    k, v = torch.empty_like(q), torch.empty_like(q)
    _check_chunk_inputs(what, q, k, v, gate_values, beta_logits, A_log, dt_bias, None, None, gm)
    _check_dtype(what, norm_gate, torch.bfloat16, "norm_gate")
    _check_dtype(what, norm_weight, torch.float32, "norm_weight")
    if norm_gate.shape != v.shape or norm_weight.shape != (D,):
        raise RuntimeError(f"{what}: norm_gate must be shaped like v and norm_weight [V]")
    gate_values = _c(gate_values)
    A_log, dt_bias, norm_weight = _c(A_log), _c(dt_bias), _c(norm_weight)
    conv_weight = _c(conv_weight)
    # beta_logits and norm_gate may be column slices of wider per-token rows
    beta_ld = _token_stride(beta_logits, H)
    if beta_ld is None:
        beta_logits, beta_ld = beta_logits.contiguous(), H
    gate_ld = _token_stride(norm_gate, H * D)
    if gate_ld is None:
        norm_gate, gate_ld = norm_gate.contiguous(), H * D
    p = _problem(q, v, None, gm, lower_bound, scale)
    p.beta_row_stride = beta_ld
    p.norm_gate_row_stride = gate_ld
    lib = _lib.load()
    ws_bytes = lib.kda_chunk_workspace_bytes(ctypes.byref(p))
    if ws_bytes == 0 and B * T > 0:
        check(1, "chunk_workspace_bytes")
    workspace = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    output = torch.empty(B, T, H, D, dtype=torch.bfloat16, device=dev)
    normed = torch.empty_like(output)
    inv = torch.empty(B * T * H, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.kda_chunk_forward_conv_norm_gate(
            ctypes.byref(p), ptr(qkv_in), int(ld), ptr(conv_weight), int(conv_weight.shape[1]),
            ptr(q), ptr(k), ptr(v), ptr(gate_values), ptr(beta_logits), ptr(A_log), ptr(dt_bias),
            ptr(output), ptr(workspace), ptr(norm_gate), ptr(norm_weight), float(eps), ptr(normed),
            ptr(inv), _stream(dev))
    check(rc, "kda_chunk_forward_conv_norm_gate")
    return q, k, v, output, normed, inv, workspace


def chunk_backward(q, k, v, gate_values, beta_logits, A_log, dt_bias, initial_state, workspace,
                   grad_output, grad_final_state, lower_bound, scale, *, cu_seqlens=None,
                   gate="k3", packed_qkv_grad=False, dbeta_out=None, dbeta_pad=0):
    """Exact chunked backward.  Returns the eight gradients
    (dq, dk, dv, dgate, dbeta_logits, dA_log, ddt_bias, dinitial_state).  With
    ``packed_qkv_grad`` (K == V) dq, dk and dv are written side by side into one
    [B, T, 3 H K] tensor, which is returned in place of dq (dk and dv are then None).
    ``dbeta_out`` [B, T, H] (a column slice of wider per-token rows) receives dbeta_logits,
    and the ``dbeta_pad`` elements after each token's H values are set to zero.

    Outside graph capture the call then reads the launch's failure flag (a synchronisation
    of the stream) and raises RuntimeError if an in-kernel wait gave up; under capture the
    NaN that such a failure writes into the gradients is the report."""
    grads, p, scratch = chunk_backward_launch(
        q, k, v, gate_values, beta_logits, A_log, dt_bias, initial_state, workspace, grad_output,
        grad_final_state, lower_bound, scale, cu_seqlens=cu_seqlens, gate=gate,
        packed_qkv_grad=packed_qkv_grad, dbeta_out=dbeta_out, dbeta_pad=dbeta_pad)
    if not torch.cuda.is_current_stream_capturing():
        chunk_backward_status(p, scratch)
    return grads


def chunk_backward_status(p, scratch):
    """Raise RuntimeError if the last backward on ``scratch`` (problem ``p``) reported a
    wait that gave up (kda_chunk_backward_status; synchronises the stream)."""
    lib = _lib.load()
    with torch.cuda.device(scratch.device):
        check(lib.kda_chunk_backward_status(ctypes.byref(p), ptr(scratch), _stream(scratch.device)),
              "kda_chunk_backward")


def chunk_backward_launch(q, k, v, gate_values, beta_logits, A_log, dt_bias, initial_state, workspace,
                          grad_output, grad_final_state, lower_bound, scale, *, cu_seqlens=None,
                          gate="k3", packed_qkv_grad=False, dbeta_out=None, dbeta_pad=0):
    """The launch half of :func:`chunk_backward`: returns (gradients, problem, scratch)
    without reading the failure flag."""
    gm = GATE_MODES[gate]
    dev = _check_chunk_inputs("chunk_backward", q, k, v, gate_values, beta_logits, A_log, dt_bias,
                              initial_state, cu_seqlens, gm)
    q, k, v, gate_values = (_c(t) for t in (q, k, v, gate_values))
    if dbeta_out is None:
        beta_logits = _c(beta_logits)
    A_log, dt_bias, initial_state = _c(A_log), _c(dt_bias), _c(initial_state)
    B, T, H, K = q.shape
    V = v.shape[-1]
    n = B if cu_seqlens is None else cu_seqlens.numel() - 1
    if grad_output is None:
        grad_output = torch.zeros(B, T, H, V, dtype=torch.bfloat16, device=dev)
    grad_output = grad_output.to(torch.bfloat16).contiguous()
    if grad_final_state is not None:
        grad_final_state = grad_final_state.to(torch.float32).contiguous()
    p = _problem(q, v, cu_seqlens, gm, lower_bound, scale)
    lib = _lib.load()
    sc_bytes = lib.kda_chunk_backward_scratch_bytes(ctypes.byref(p))
    scratch = torch.empty(max(sc_bytes, 256), dtype=torch.uint8, device=dev)
    if packed_qkv_grad:
        if V != K:
            raise ValueError("chunk_backward: packed_qkv_grad needs key_dim == value_dim")
        dqkv = torch.empty(B, T, 3 * H * K, dtype=q.dtype, device=dev)
        p.grad_row_stride = 3 * H * K
        dq, dk, dv = dqkv[..., :H * K], dqkv[..., H * K:2 * H * K], dqkv[..., 2 * H * K:]
    else:
        dq = torch.empty_like(q)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
    dgate = torch.empty_like(gate_values)
    if dbeta_out is not None:
        ld = _token_stride(dbeta_out, H)
        if ld is None or dbeta_out.shape != beta_logits.shape or dbeta_out.dtype != torch.bfloat16 \
                or ld < H + dbeta_pad or _token_stride(beta_logits, H) != ld:
            raise RuntimeError("chunk_backward: dbeta_out must be a bf16 [B, T, H] slice of per-token rows "
                               "with room for the padding, with the row stride of beta_logits")
        dbeta = dbeta_out
        p.beta_row_stride = ld
        p.beta_grad_pad = int(dbeta_pad)
    else:
        if dbeta_pad:
            raise RuntimeError("chunk_backward: dbeta_pad needs dbeta_out")
        dbeta = torch.empty_like(beta_logits)
    if gm == KDA_GATE_K3:
        dA = torch.empty_like(A_log)
        ddt = torch.empty_like(dt_bias)
    else:
        dA = ddt = None
    dinit = torch.empty_like(initial_state) if initial_state is not None else None
    with torch.cuda.device(dev):
        rc = lib.kda_chunk_backward(
            ctypes.byref(p), ptr(q), ptr(k), ptr(v), ptr(gate_values), ptr(beta_logits),
            ptr(A_log), ptr(dt_bias), ptr(initial_state), ptr(workspace), ptr(grad_output),
            ptr(grad_final_state), ptr(dq), ptr(dk), ptr(dv), ptr(dgate), ptr(dbeta), ptr(dA),
            ptr(ddt), ptr(dinit), ptr(scratch), _stream(dev))
    check(rc, "kda_chunk_backward")
    if packed_qkv_grad:
        return (dqkv, None, None, dgate, dbeta, dA, ddt, dinit), p, scratch
    return (dq, dk, dv, dgate, dbeta, dA, ddt, dinit), p, scratch


# ---------------------------------------------------------------------------
# decode, convolution, norm-gate
# ---------------------------------------------------------------------------

def recurrent_decode(q, k, v, gate_values, beta_logits, A_log, dt_bias, initial_state,
                     output_final_state, lower_bound, scale, *, gate="k3", out_state=None):
    """One recurrent step (T == 1).  Returns (output [B,1,H,V], final_state or None).

    ``out_state`` may be given to receive the new state (it may alias ``initial_state``).
    """
    gm = GATE_MODES[gate]
    dev = _check_chunk_inputs("recurrent_decode", q, k, v, gate_values, beta_logits, A_log,
                              dt_bias, initial_state, None, gm)
    if q.shape[1] != 1:
        raise RuntimeError("recurrent_decode: expects exactly one token (T == 1)")
    q, k, v, gate_values, beta_logits = (_c(t) for t in (q, k, v, gate_values, beta_logits))
    A_log, dt_bias = _c(A_log), _c(dt_bias)
    if initial_state is not None and not initial_state.is_contiguous():
        initial_state = initial_state.contiguous()
    B, _, H, K = q.shape
    V = v.shape[-1]
    output = torch.empty(B, 1, H, V, dtype=torch.bfloat16, device=dev)
    final_state = None
    if out_state is not None:
        final_state = out_state
    elif output_final_state:
        final_state = torch.empty(B, H, V, K, dtype=torch.float32, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.kda_recurrent_decode(B, H, K, V, gm, float(lower_bound), float(scale), ptr(q),
                                      ptr(k), ptr(v), ptr(gate_values), ptr(beta_logits),
                                      ptr(A_log), ptr(dt_bias), ptr(initial_state), ptr(output),
                                      ptr(final_state), _stream(dev))
    check(rc, "kda_recurrent_decode")
    return output, final_state


def causal_conv_forward(x, weight, initial_state, output_final_state):
    """x [B,T,C] bf16, weight [C,W] bf16, state [B,C,W] bf16 -> (y, final_state or None)."""
    dev = _require_cuda("causal_convolution_forward", x, weight, initial_state)
    for name, t in (("x", x), ("weight", weight), ("initial_state", initial_state)):
        _check_dtype("causal_convolution_forward", t, torch.bfloat16, name)
    x, weight, initial_state = _c(x), _c(weight), _c(initial_state)
    B, T, C = x.shape
    W = weight.shape[-1]
    if weight.shape != (C, W):
        raise RuntimeError("causal_convolution_forward: weight must have shape [C, W]")
    if initial_state is not None and initial_state.shape != (B, C, W):
        raise RuntimeError("causal_convolution_forward: initial_state must have shape [B, C, W]")
    y = torch.empty_like(x)
    fin = torch.empty(B, C, W, dtype=x.dtype, device=dev) if output_final_state else None
    with torch.cuda.device(dev):
        rc = _lib.load().kda_causal_conv_forward(B, T, C, W, ptr(x), ptr(weight), ptr(initial_state),
                                                 ptr(y), ptr(fin), _stream(dev))
    check(rc, "kda_causal_conv_forward")
    return y, fin


def _row_stride(t):
    """Row stride (elements per token) with which the kernels can step through the B*T rows
    of a [B, T, C] tensor, or None: unit channel stride, 16-byte aligned, a stride that is a
    multiple of 8 of at least C, and batches that follow each other (a column slice of a
    wider [B, T, N] row qualifies)."""
    B, T, C = t.shape
    if t.stride(2) != 1 or t.data_ptr() % 16:
        return None
    ld = t.stride(1) if T > 1 else (t.stride(0) if B > 1 else C)
    if ld % 8 or ld < C or (B > 1 and t.stride(0) != T * ld):
        return None
    return ld


def _token_stride(t, inner):
    """Elements between consecutive tokens of a [B, T, *rest] tensor whose per-token block
    of ``inner`` elements is dense (a column slice of a wider per-token row), or None when
    the kernels cannot step through it that way."""
    B, T = t.shape[:2]
    if t.numel() == 0:
        return None
    expect = 1
    for d in range(t.ndim - 1, 1, -1):
        if t.stride(d) != expect:
            return None
        expect *= t.shape[d]
    if expect != inner:
        return None
    ld = t.stride(1) if T > 1 else (t.stride(0) if B > 1 else inner)
    if ld < inner or (B > 1 and t.stride(0) != T * ld):
        return None
    return ld


def causal_conv_backward(x, weight, initial_state, grad_output, grad_final_state, *, dx_out=None):
    """Returns (dx, dweight, dinitial_state or None).  ``x`` may be a column slice of wider
    rows (read in place); ``dx_out`` may be given to receive dx, also possibly such a slice."""
    dev = _require_cuda("causal_convolution_backward", x, weight, initial_state, grad_output,
                        grad_final_state)
    if _row_stride(x) is None:
        x = x.contiguous()
    weight, initial_state = _c(weight), _c(initial_state)
    B, T, C = x.shape
    W = weight.shape[-1]
    if grad_output is None:
        grad_output = torch.zeros_like(x)
    grad_output = grad_output.to(torch.bfloat16).contiguous()
    if grad_final_state is not None:
        grad_final_state = grad_final_state.to(torch.bfloat16).contiguous()
    lib = _lib.load()
    scratch = torch.empty(lib.kda_causal_conv_backward_scratch_bytes(B, T, C, W), dtype=torch.uint8,
                          device=dev)
    if dx_out is not None:
        if dx_out.shape != x.shape or dx_out.dtype != torch.bfloat16 or _row_stride(dx_out) is None:
            raise ValueError("causal_conv_backward: dx_out must be a row-strided bf16 [B, T, C] tensor")
        dx = dx_out
    else:
        dx = torch.empty(B, T, C, dtype=torch.bfloat16, device=dev)
    dw = torch.empty_like(weight)
    dst = torch.empty_like(initial_state) if initial_state is not None else None
    ldx, ldd = _row_stride(x), _row_stride(dx)
    with torch.cuda.device(dev):
        rc = lib.kda_causal_conv_backward_strided(B, T, C, W, ptr(x), ldx, ptr(weight), ptr(initial_state),
                                                  ptr(grad_output), ptr(grad_final_state), ptr(dx), ldd,
                                                  ptr(dw), ptr(dst), ptr(scratch), _stream(dev))
    check(rc, "kda_causal_conv_backward")
    return dx, dw, dst


def rmsnorm_gate_forward(x, gate, weight, eps):
    """x, gate [..., D] bf16; weight [D] f32 -> (y bf16, inv_rms f32 [rows])."""
    dev = _require_cuda("rmsnorm_gate_forward", x, gate, weight)
    _check_dtype("rmsnorm_gate_forward", x, torch.bfloat16, "x")
    _check_dtype("rmsnorm_gate_forward", gate, torch.bfloat16, "gate")
    _check_dtype("rmsnorm_gate_forward", weight, torch.float32, "weight")
    if x.shape != gate.shape:
        raise RuntimeError("rmsnorm_gate_forward: x and gate must share a shape")
    x, gate, weight = _c(x), _c(gate), _c(weight)
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    y = torch.empty_like(x)
    inv = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_rmsnorm_gate_forward(rows, D, ptr(x), ptr(gate), ptr(weight),
                                                  float(eps), ptr(y), ptr(inv), _stream(dev))
    check(rc, "kda_rmsnorm_gate_forward")
    return y, inv


def rmsnorm_gate_backward(x, gate, weight, inv_rms, grad_output, eps, *, dgate_out=None):
    """Returns (dx bf16, dgate bf16, dweight f32).  For [B, T, H, D] operands the gate may
    be a column slice of wider per-token rows, and ``dgate_out`` (same shape, also such a
    slice) receives dgate."""
    dev = _require_cuda("rmsnorm_gate_backward", x, gate, weight, inv_rms, grad_output)
    x, weight, inv_rms = _c(x), _c(weight), _c(inv_rms)
    grad_output = grad_output.to(torch.bfloat16).contiguous()
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    heads, gld, dgld = 1, D, D
    if x.ndim == 4 and gate.shape == x.shape:
        heads = x.shape[2]
        gld = _token_stride(gate, heads * D)
        if gld is None or gld % 8 or gate.data_ptr() % 16:
            gate, gld = gate.contiguous(), heads * D
        dgld = heads * D
    else:
        gate = _c(gate)
    if dgate_out is not None:
        dgld = _token_stride(dgate_out, heads * D) if dgate_out.ndim == 4 else None
        if dgate_out.shape != gate.shape or dgate_out.dtype != torch.bfloat16 or dgld is None \
                or dgld % 8 or dgate_out.data_ptr() % 16:
            raise RuntimeError("rmsnorm_gate_backward: dgate_out must be a bf16 [B, T, H, D] slice of "
                               "per-token rows (16-byte aligned, row stride a multiple of 8)")
        dg = dgate_out
    else:
        dg = torch.empty(gate.shape, dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    scratch = torch.empty(lib.kda_rmsnorm_gate_backward_scratch_bytes(rows, D), dtype=torch.uint8,
                          device=dev)
    dx = torch.empty_like(x)
    dw = torch.empty_like(weight)
    with torch.cuda.device(dev):
        rc = lib.kda_rmsnorm_gate_backward_strided(rows, D, heads, ptr(x), ptr(gate), int(gld), ptr(weight),
                                                   ptr(inv_rms), ptr(grad_output), float(eps), ptr(dx),
                                                   ptr(dg), int(dgld), ptr(dw), ptr(scratch), _stream(dev))
    check(rc, "kda_rmsnorm_gate_backward")
    return dx, dg, dw


# ---------------------------------------------------------------------------
# torch.ops.nanochat_kda registrations (reference schemas)
# ---------------------------------------------------------------------------

_LIBRARY = None


def softcap_cross_entropy_forward(logits, targets, vocab, softcap, ignore_index=-1):
    """logits [rows, stride] bf16 (stride >= vocab), targets [rows] int64 ->
    (loss_rows f32 [rows], lse_rows f32 [rows])."""
    dev = _require_cuda("softcap_cross_entropy_forward", logits, targets)
    _check_dtype("softcap_cross_entropy_forward", logits, torch.bfloat16, "logits")
    _check_dtype("softcap_cross_entropy_forward", targets, torch.int64, "targets")
    if logits.ndim != 2 or targets.shape != logits.shape[:1]:
        raise RuntimeError("softcap_cross_entropy_forward: logits [rows, stride] and targets [rows]")
    logits, targets = _c(logits), _c(targets)
    rows, stride = logits.shape
    loss = torch.empty(rows, dtype=torch.float32, device=dev)
    lse = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_softcap_cross_entropy_forward(rows, int(vocab), stride, float(softcap),
                                                           ptr(logits), ptr(targets), int(ignore_index),
                                                           ptr(loss), ptr(lse), _stream(dev))
    check(rc, "kda_softcap_cross_entropy_forward")
    return loss, lse


def softcap_cross_entropy_mean(loss_rows, targets, ignore_index=-1):
    """(mean loss over non-ignored rows, that row count): two f32 device scalars."""
    dev = _require_cuda("softcap_cross_entropy_mean", loss_rows, targets)
    _check_dtype("softcap_cross_entropy_mean", loss_rows, torch.float32, "loss_rows")
    _check_dtype("softcap_cross_entropy_mean", targets, torch.int64, "targets")
    loss_rows, targets = _c(loss_rows), _c(targets)
    out = torch.empty(2, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_softcap_cross_entropy_mean(loss_rows.numel(), ptr(loss_rows), ptr(targets),
                                                        int(ignore_index), ptr(out), out.data_ptr() + 4,
                                                        _stream(dev))
    check(rc, "kda_softcap_cross_entropy_mean")
    return out[0], out[1]


def softcap_cross_entropy_fused_supported(vocab, stride):
    """True where the one-pass forward + backward kernel takes rows of this shape (every
    column is vocabulary, a multiple of 4096 columns, at most 32768)."""
    return bool(_lib.load().kda_softcap_cross_entropy_fused_supported(int(vocab), int(stride)))


def softcap_cross_entropy_fused(logits, targets, vocab, softcap, ignore_index=-1, expected_grad=1.0):
    """Forward and backward in one read of the logits: -> (loss_rows, lse_rows, grad_logits,
    count).  grad_logits is the gradient for an upstream dL/dmean of ``expected_grad``
    (rescale it with rescale_bf16_if_changed when the actual one differs); count is the
    non-ignored row count (f32 device scalar)."""
    dev = _require_cuda("softcap_cross_entropy_fused", logits, targets)
    _check_dtype("softcap_cross_entropy_fused", logits, torch.bfloat16, "logits")
    _check_dtype("softcap_cross_entropy_fused", targets, torch.int64, "targets")
    if logits.ndim != 2 or targets.shape != logits.shape[:1]:
        raise RuntimeError("softcap_cross_entropy_fused: logits [rows, stride] and targets [rows]")
    logits, targets = _c(logits), _c(targets)
    rows, stride = logits.shape
    loss = torch.empty(rows, dtype=torch.float32, device=dev)
    lse = torch.empty(rows, dtype=torch.float32, device=dev)
    grad = torch.empty_like(logits)
    sc = torch.empty(2, dtype=torch.float32, device=dev)  # count, grad scale
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.kda_softcap_cross_entropy_count(rows, ptr(targets), int(ignore_index), float(expected_grad),
                                                 ptr(sc), sc.data_ptr() + 4, _stream(dev))
        check(rc, "kda_softcap_cross_entropy_count")
        rc = lib.kda_softcap_cross_entropy_fused(rows, int(vocab), stride, float(softcap), ptr(logits),
                                                 ptr(targets), int(ignore_index), sc.data_ptr() + 4, ptr(loss),
                                                 ptr(lse), ptr(grad), _stream(dev))
    check(rc, "kda_softcap_cross_entropy_fused")
    return loss, lse, grad, sc[0]


def rescale_bf16_if_changed(data, actual, expected):
    """data (bf16, contiguous, numel % 8 == 0) *= actual / expected in place unless the
    device scalar ``actual`` equals ``expected`` (decided on the device, no host sync)."""
    dev = _require_cuda("rescale_bf16_if_changed", data, actual)
    _check_dtype("rescale_bf16_if_changed", data, torch.bfloat16, "data")
    if not data.is_contiguous():
        raise RuntimeError("rescale_bf16_if_changed: data must be contiguous")
    actual = actual.to(torch.float32).reshape(1).contiguous()
    with torch.cuda.device(dev):
        rc = _lib.load().kda_bf16_rescale_if_changed(data.numel(), ptr(data), ptr(actual), float(expected),
                                                     _stream(dev))
    check(rc, "kda_bf16_rescale_if_changed")
    return data


def embedding_backward(idx, grad_output, vocab):
    """Gradient of an embedding lookup: idx int64 [...], grad_output bf16 [..., dim] ->
    grad_weight bf16 [vocab, dim] (token-order f32 sums, deterministic)."""
    dev = _require_cuda("embedding_backward", idx, grad_output)
    _check_dtype("embedding_backward", idx, torch.int64, "idx")
    _check_dtype("embedding_backward", grad_output, torch.bfloat16, "grad_output")
    dim = grad_output.shape[-1]
    if grad_output.shape[:-1] != idx.shape:
        raise RuntimeError("embedding_backward: grad_output must be idx.shape + [dim]")
    idx, grad_output = _c(idx), _c(grad_output)
    dw = torch.empty(vocab, dim, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_embedding_backward(idx.numel(), int(vocab), int(dim), ptr(idx), ptr(grad_output),
                                                ptr(dw), _stream(dev))
    check(rc, "kda_embedding_backward")
    return dw


def softcap_cross_entropy_backward(logits, targets, lse, grad_scale, vocab, softcap, ignore_index=-1):
    """grad_scale: f32 device scalar (dL/dmean / non-ignored count) -> grad [rows, stride] bf16."""
    dev = _require_cuda("softcap_cross_entropy_backward", logits, targets, lse, grad_scale)
    logits, targets, lse = _c(logits), _c(targets), _c(lse)
    grad_scale = grad_scale.to(torch.float32).reshape(1).contiguous()
    rows, stride = logits.shape
    grad = torch.empty_like(logits)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_softcap_cross_entropy_backward(rows, int(vocab), stride, float(softcap),
                                                            ptr(logits), ptr(targets), int(ignore_index),
                                                            ptr(lse), ptr(grad_scale), ptr(grad),
                                                            _stream(dev))
    check(rc, "kda_softcap_cross_entropy_backward")
    return grad

def weight_grad(grad_output, x):
    """dW [N, K] f32 = grad_output[M, N]^T x[M, K] (bf16, 2-D, unit column stride)."""
    dev = _require_cuda("weight_grad", grad_output, x)
    _check_dtype("weight_grad", grad_output, torch.bfloat16, "grad_output")
    _check_dtype("weight_grad", x, torch.bfloat16, "x")
    if grad_output.ndim != 2 or x.ndim != 2 or grad_output.shape[0] != x.shape[0]:
        raise RuntimeError("weight_grad: grad_output [M, N] and x [M, K] expected")
    if grad_output.stride(1) != 1 or (grad_output.shape[0] > 1 and grad_output.stride(0) < grad_output.shape[1]):
        grad_output = grad_output.contiguous()
    if x.stride(1) != 1 or (x.shape[0] > 1 and x.stride(0) < x.shape[1]):
        x = x.contiguous()
    M, N = grad_output.shape
    K = x.shape[1]
    lib = _lib.load()
    scratch = torch.empty(lib.kda_weight_grad_scratch_bytes(M, N, K), dtype=torch.uint8, device=dev)
    dw = torch.empty(N, K, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.kda_weight_grad(M, N, K, ptr(grad_output), max(grad_output.stride(0), N), ptr(x),
                                 max(x.stride(0), K), ptr(dw), ptr(scratch), _stream(dev))
    check(rc, "kda_weight_grad")
    return dw

def _glue_check(what, *tensors):
    dev = _require_cuda(what, *tensors)
    for t in tensors:
        _check_dtype(what, t, torch.bfloat16, "tensor")
        if t.shape != tensors[0].shape:
            raise RuntimeError(f"{what}: tensors must share a shape")
        if t.numel() % 8:
            raise RuntimeError(f"{what}: element count must be a multiple of 8")
    return dev


def resid_mix_forward(x, x0, a, b):
    """y = a x + b x0 (bf16); a, b are f32 device scalars (one-element views)."""
    dev = _glue_check("resid_mix_forward", x, x0)
    x, x0, a, b = _c(x), _c(x0), _c(a), _c(b)
    y = torch.empty_like(x)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_resid_mix_forward(x.numel(), ptr(a), ptr(b), ptr(x), ptr(x0), ptr(y),
                                               _stream(dev))
    check(rc, "kda_resid_mix_forward")
    return y


def resid_mix_backward(x, x0, lam_a, lam_b, slot, grad):
    """Backward of y = lam_a[slot] x + lam_b[slot] x0 for f32 lambda vectors: returns
    (dx, dx0, dlam_a, dlam_b), the lambda gradients full-length and zero except at slot."""
    dev = _glue_check("resid_mix_backward", x, x0, grad)
    x, x0, grad, lam_a, lam_b = _c(x), _c(x0), _c(grad), _c(lam_a), _c(lam_b)
    n = lam_a.numel()
    if lam_a.dtype != torch.float32 or lam_b.dtype != torch.float32 or lam_b.numel() != n or not 0 <= slot < n:
        raise ValueError("resid_mix_backward: f32 lambda vectors of one length and a slot inside them")
    lib = _lib.load()
    scratch = torch.empty(lib.kda_resid_mix_backward_scratch_bytes(x.numel()), dtype=torch.uint8, device=dev)
    dx, dx0 = torch.empty_like(x), torch.empty_like(x0)
    da = torch.empty(n, dtype=torch.float32, device=dev)
    db = torch.empty(n, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.kda_resid_mix_backward(x.numel(), ptr(lam_a) + 4 * slot, ptr(lam_b) + 4 * slot, ptr(x), ptr(x0),
                                        ptr(grad), ptr(dx), ptr(dx0), ptr(da), ptr(db), slot, n, ptr(scratch),
                                        _stream(dev))
    check(rc, "kda_resid_mix_backward")
    return dx, dx0, da, db


def relu2_forward(x):
    dev = _glue_check("relu2_forward", x)
    x = _c(x)
    y = torch.empty_like(x)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_relu2_forward(x.numel(), ptr(x), ptr(y), _stream(dev))
    check(rc, "kda_relu2_forward")
    return y


def relu2_backward(x, grad):
    dev = _glue_check("relu2_backward", x, grad)
    x, grad = _c(x), _c(grad)
    dx = torch.empty_like(x)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_relu2_backward(x.numel(), ptr(x), ptr(grad), ptr(dx), _stream(dev))
    check(rc, "kda_relu2_backward")
    return dx

def rms_norm_forward(x, eps):
    """y = x / sqrt(mean(x^2) + eps) over the last dim (bf16) -> (y, rinv f32 [rows])."""
    dev = _require_cuda("rms_norm_forward", x)
    _check_dtype("rms_norm_forward", x, torch.bfloat16, "x")
    x = _c(x)
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    y = torch.empty_like(x)
    rinv = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_rms_norm_forward(rows, D, float(eps), ptr(x), ptr(y), ptr(rinv), _stream(dev))
    check(rc, "kda_rms_norm_forward")
    return y, rinv


def rms_norm_backward(x, rinv, grad, grad_add=None):
    """dx of rms_norm, plus ``grad_add`` (the gradient reaching x by another path) when given."""
    dev = _require_cuda("rms_norm_backward", x, rinv, grad)
    x, rinv, grad = _c(x), _c(rinv), _c(grad.to(torch.bfloat16))
    if grad_add is not None:
        grad_add = _c(grad_add.to(torch.bfloat16))
        if grad_add.shape != x.shape:
            raise ValueError("rms_norm_backward: grad_add must be shaped like x")
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    dx = torch.empty_like(x)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_rms_norm_backward_add(rows, D, ptr(x), ptr(rinv), ptr(grad), ptr(grad_add), ptr(dx),
                                                   _stream(dev))
    check(rc, "kda_rms_norm_backward")
    return dx


def mix_rms_norm_forward(x, x2, eps, a=None, b=None):
    """s = a x + b x2 (one-element f32 tensors a, b; None means 1) rounded to bf16, and its
    rms_norm: returns (s, y, rinv)."""
    dev = _require_cuda("mix_rms_norm_forward", x, x2)
    _check_dtype("mix_rms_norm_forward", x, torch.bfloat16, "x")
    _check_dtype("mix_rms_norm_forward", x2, torch.bfloat16, "x2")
    if x2.shape != x.shape:
        raise ValueError("mix_rms_norm_forward: x and x2 must have the same shape")
    for w in (a, b):
        if w is not None and (w.dtype != torch.float32 or w.numel() != 1 or w.device != x.device):
            raise ValueError("mix_rms_norm_forward: a and b must be one-element f32 tensors on x's device")
    x, x2 = _c(x), _c(x2)
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    s, y = torch.empty_like(x), torch.empty_like(x)
    rinv = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().kda_mix_rms_norm_forward(rows, D, float(eps), ptr(a), ptr(b), ptr(x), ptr(x2), ptr(s),
                                                  ptr(y), ptr(rinv), _stream(dev))
    check(rc, "kda_mix_rms_norm_forward")
    return s, y, rinv

def _op_chunk_forward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                      output_final_state, lower_bound, scale):
    # the schema has no workspace output: the residuals ride in the output's allocation
    out, fin, _ = chunk_forward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                                output_final_state, lower_bound, scale, residuals_behind_output=True)
    return out, fin


def _residuals_of(output, q, v, gate_mode, lower_bound, scale):
    """The workspace stored behind ``output`` by the schema forward, or None when ``output``
    was not made by it (wrong allocation size or a view into another tensor)."""
    B, T, H, _ = q.shape
    V = v.shape[-1]
    p = _problem(q, v, None, gate_mode, lower_bound, scale)
    ws_bytes = max(_lib.load().kda_chunk_workspace_bytes(ctypes.byref(p)), 256)
    off = _output_bytes(B, T, H, V)
    storage = output.untyped_storage()
    if (output.storage_offset() != 0 or not output.is_contiguous() or output.dtype != torch.bfloat16
            or tuple(output.shape) != (B, T, H, V) or storage.nbytes() != off + ws_bytes):
        return None
    return torch.empty(0, dtype=torch.uint8, device=output.device).set_(storage, off, (ws_bytes,))


def _op_chunk_backward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state, output,
                       final_state, grad_output, grad_final_state, lower_bound, scale):
    # Residuals come from behind `output` (as the reference stores them); an output that
    # does not carry them (made elsewhere) costs one recomputation of the forward.
    del final_state
    ws = _residuals_of(output, q, v, KDA_GATE_K3, lower_bound, scale)
    if ws is None:
        _, _, ws = chunk_forward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                                 False, lower_bound, scale)
    return chunk_backward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state, ws,
                          grad_output, grad_final_state, lower_bound, scale)


def _op_recurrent_decode(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                         output_final_state, lower_bound, scale):
    return recurrent_decode(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                            output_final_state, lower_bound, scale)


def _op_conv_backward(x, weight, initial_state, output, final_state, grad_output, grad_final_state):
    del output, final_state
    return causal_conv_backward(x, weight, initial_state, grad_output, grad_final_state)


def _op_norm_backward(x, gate, weight, inverse_rms, grad_output, epsilon):
    return rmsnorm_gate_backward(x, gate, weight, inverse_rms, grad_output, epsilon)


SCHEMAS = {
    "chunk_forward": (
        "chunk_forward(Tensor q, Tensor k, Tensor v, Tensor raw_gate, Tensor beta_logits, "
        "Tensor A_log, Tensor dt_bias, Tensor? initial_state, bool output_final_state, "
        "float lower_bound, float scale) -> (Tensor output, Tensor? final_state)",
        _op_chunk_forward),
    "chunk_backward": (
        "chunk_backward(Tensor q, Tensor k, Tensor v, Tensor raw_gate, Tensor beta_logits, "
        "Tensor A_log, Tensor dt_bias, Tensor? initial_state, Tensor output, Tensor? final_state, "
        "Tensor grad_output, Tensor? grad_final_state, float lower_bound, float scale) -> "
        "(Tensor dq, Tensor dk, Tensor dv, Tensor draw_gate, Tensor dbeta_logits, Tensor dA_log, "
        "Tensor ddt_bias, Tensor? dinitial_state)",
        _op_chunk_backward),
    "recurrent_decode": (
        "recurrent_decode(Tensor q, Tensor k, Tensor v, Tensor raw_gate, Tensor beta_logits, "
        "Tensor A_log, Tensor dt_bias, Tensor? initial_state, bool output_final_state, "
        "float lower_bound, float scale) -> (Tensor output, Tensor? final_state)",
        _op_recurrent_decode),
    "causal_convolution_forward": (
        "causal_convolution_forward(Tensor x, Tensor weight, Tensor? initial_state, "
        "bool output_final_state) -> (Tensor output, Tensor? final_state)",
        causal_conv_forward),
    "causal_convolution_backward": (
        "causal_convolution_backward(Tensor x, Tensor weight, Tensor? initial_state, "
        "Tensor output, Tensor? final_state, Tensor grad_output, Tensor? grad_final_state) -> "
        "(Tensor dx, Tensor dweight, Tensor? dinitial_state)",
        _op_conv_backward),
    "rmsnorm_gate_forward": (
        "rmsnorm_gate_forward(Tensor x, Tensor gate, Tensor weight, float epsilon) -> "
        "(Tensor output, Tensor inverse_rms)",
        rmsnorm_gate_forward),
    "rmsnorm_gate_backward": (
        "rmsnorm_gate_backward(Tensor x, Tensor gate, Tensor weight, Tensor inverse_rms, "
        "Tensor grad_output, float epsilon) -> (Tensor dx, Tensor dgate, Tensor dweight)",
        _op_norm_backward),
}


def register_operators() -> None:
    """Define ``torch.ops.nanochat_kda.*`` once, implemented for the ROCm device."""
    global _LIBRARY
    if _LIBRARY is not None:
        return
    lib = torch.library.Library("nanochat_kda", "DEF")
    for name, (schema, fn) in SCHEMAS.items():
        lib.define(schema)
        lib.impl(name, fn, "CUDA")
    _LIBRARY = lib
