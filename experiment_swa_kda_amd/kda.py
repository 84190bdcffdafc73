"""Kimi Delta Attention mixer API backed by the MI355X (gfx950) HIP kernels.

Drop-in for the public surface of the reference module nanochat/mixers/kda.py
(``KDAState`` :23-35, ``Linear`` :38-43, ``RMSNormGated`` :46-59, ``ShortConvolution``
:123-212, ``k3_decay_gate`` :230-243, ``kda`` :561-673, ``KimiDeltaAttention`` :676-798,
``prepare_kda_backend`` :478-488) with the same names, defaults, shapes and exceptions.

Modes:
  * ``"reference"``  — the eager PyTorch token loop of the reference (:269-327), run only
    when explicitly requested (CPU or GPU tensors, autograd backward).
  * ``"project_chunk"`` / ``"chunk"`` — the chunked WY HIP kernels with the exact HIP
    backward (``chunk`` names the reference's FLA comparator slot; here it is served by
    the same kernels).
  * ``"project_recurrent"`` / ``"recurrent"`` — inference-only; one token runs the HIP
    decode step, longer inputs run the chunked HIP forward without autograd.
The ``project_*`` modes fail closed: an unsupported call raises RuntimeError whatever
``allow_fallback`` says.  ``chunk`` / ``recurrent`` follow the reference contract: an
unsupported call (CPU tensors, f32 activations, an unsupported head size, gradients
through ``recurrent``) runs the eager loop when ``allow_fallback=True`` and raises
RuntimeError otherwise; a supported call always runs the HIP kernels.

Two keyword extensions serve the benchmark configurations: ``gate="precomputed"``
feeds an already-activated f32 log decay g in place of ``raw_gate`` (A_log and dt_bias
are then unused), and ``cu_seqlens`` packs variable-length sequences with a state reset
at each boundary.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

MODES = {"reference", "chunk", "recurrent", "project_chunk", "project_recurrent"}


@dataclass
class KDAState:
    """Everything a KDA layer carries from one decode step to the next.

    ``memory`` is the f32 recurrent matrix of every (batch, head), stored value-major as
    ``[B, H, V, K]``: row v is the key-space vector that produces output channel v.
    ``q_conv``, ``k_conv`` and ``v_conv`` are the short-convolution windows ``[B, D, W]``;
    each holds the W latest pre-convolution projections, the newest (the token just
    processed) in the last slot.
    """

    memory: torch.Tensor
    q_conv: torch.Tensor
    k_conv: torch.Tensor
    v_conv: torch.Tensor


_SPLIT_WGRAD_MAX = 1 << 21  # weights up to 2M entries take the split-contraction kernel


def _mm_f32(a, b):
    """a @ b of bf16 matrices with the f32 accumulator stored as the f32 result (no bf16
    rounding and no separate conversion pass), where torch offers it."""
    try:
        return torch.mm(a, b, out_dtype=torch.float32)
    except (TypeError, RuntimeError):
        return (a @ b).float()


class _LinearBF16(torch.autograd.Function):
    """y = x W^T with an f32 master weight cast to bf16; the weight gradient comes from the
    split-contraction HIP kernel straight in f32 (nanochat/gpt.py:52-57)."""

    @staticmethod
    def forward(ctx, x, weight, bias, w16=None):
        # w16: the weight already cast (a copy made once per training update), else cast here
        w = w16 if w16 is not None else weight.to(torch.bfloat16)
        ctx.save_for_backward(x, w)
        ctx.has_bias = bias is not None
        return F.linear(x, w, None if bias is None else bias.to(torch.bfloat16))

    @staticmethod
    def backward(ctx, grad):
        x, w = ctx.saved_tensors
        g2 = grad.reshape(-1, grad.shape[-1])
        dx = (g2 @ w).reshape(x.shape) if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            x2 = x.reshape(-1, x.shape[-1])
            if w.numel() <= _SPLIT_WGRAD_MAX:
                dw = ops.weight_grad(g2, x2)
            else:  # a large output (the lm_head) already fills the GPU as one library GEMM,
                # which writes the f32 gradient itself
                dw = _mm_f32(g2.t(), x2)
        db = g2.float().sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dx, dw, db, None


class _StackedLinearBF16(torch.autograd.Function):
    """y = x [W_1; ...; W_n; 0]^T for several f32 weights that read the same input, with the
    stacked bf16 weight (zero rows padding the width) given or built here; the one f32 weight
    gradient is handed back to each W_i as its row block."""

    @staticmethod
    def forward(ctx, x, w16, pad, *weights):
        if w16 is None:
            w16 = torch.cat(list(weights) + [weights[0].new_zeros(pad, weights[0].shape[1])]).to(torch.bfloat16)
        ctx.save_for_backward(x, w16)
        ctx.rows = [w.shape[0] for w in weights]
        return F.linear(x, w16)

    @staticmethod
    def backward(ctx, grad):
        x, w = ctx.saved_tensors
        g2 = grad.reshape(-1, grad.shape[-1])
        dx = (g2 @ w).reshape(x.shape) if ctx.needs_input_grad[0] else None
        dws = [None] * len(ctx.rows)
        if any(ctx.needs_input_grad[3:]):
            dw = ops.weight_grad(g2, x.reshape(-1, x.shape[-1]))
            dws = list(torch.split(dw[: sum(ctx.rows)], ctx.rows, dim=0))
        return (dx, None, None, *dws)


class _SplitColumns(torch.autograd.Function):
    """Splits the last dimension into contiguous column blocks; the backward writes the
    blocks' gradients back side by side with one concatenation (slicing views instead would
    make autograd zero-fill and copy a full-width gradient per block)."""

    @staticmethod
    def forward(ctx, y, sizes):
        ctx.sizes = sizes
        return tuple(t.contiguous() for t in torch.split(y, sizes, dim=-1))

    @staticmethod
    def backward(ctx, *grads):
        ref = next(g for g in grads if g is not None)
        full = [g if g is not None else ref.new_zeros(*ref.shape[:-1], n) for g, n in zip(grads, ctx.sizes)]
        return torch.cat(full, dim=-1), None


class Linear(nn.Linear):
    """nn.Linear whose parameters stay f32 while the product runs in the input's dtype
    (bf16 on the GPU: the weight is cast per call and its gradient comes back in f32)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda and x.dtype == torch.bfloat16 and self.weight.dtype == torch.float32:
            return _LinearBF16.apply(x, self.weight, self.bias, getattr(self, "_w16", None))
        bias = None if self.bias is None else self.bias.to(dtype=x.dtype)
        return F.linear(x, self.weight.to(dtype=x.dtype), bias)


def _norm_gate_eager(x, gate, weight, eps):
    """Per-row RMS normalisation of the last axis with a learned scale, computed in the
    input's dtype, then multiplied by the logistic of ``gate``."""
    scaled = F.rms_norm(x, x.shape[-1:], weight.to(x.dtype), eps)
    return scaled * torch.sigmoid(gate)


class RMSNormGated(nn.Module):
    """Output normalisation of the mixer: ``rms_norm(x) * weight * sigmoid(gate)`` over the
    head dimension (parameter ``weight``, initialised to ones)."""

    def __init__(self, hidden_size: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        return _norm_gate_eager(x, gate, self.weight, self.eps)


# ---------------------------------------------------------------------------
# runtime provenance (reference kda.py:62-90, 469-488)
# ---------------------------------------------------------------------------

_RUNTIME_EVENTS: list[dict[str, str]] = []


def reset_project_runtime_events() -> None:
    _RUNTIME_EVENTS.clear()


def project_runtime_events() -> list[dict[str, str]]:
    return list(_RUNTIME_EVENTS)


def _record(component: str) -> None:
    _RUNTIME_EVENTS.append({"component": component, "backend": "project"})


def _record_backward(output: torch.Tensor, component: str) -> torch.Tensor:
    if output.requires_grad:
        output.register_hook(lambda grad: (_record(component), grad)[1])
    return output


_COMPONENTS = {
    "chunk_forward": ("kda_chunk_forward", "chunk_fwd.hip"),
    "chunk_backward": ("kda_chunk_backward", "chunk_bwd.hip"),
    "chunk_forward_norm_gate": ("kda_chunk_forward_norm_gate", "chunk_fwd.hip"),
    "chunk_forward_conv_norm_gate": ("kda_chunk_forward_conv_norm_gate", "chunk_fwd.hip"),
    "recurrent_decode": ("kda_recurrent_decode", "decode.hip"),
    "causal_convolution_forward": ("kda_causal_conv_forward", "conv.hip"),
    "causal_convolution_backward": ("kda_causal_conv_backward", "conv.hip"),
    "rmsnorm_gate_forward": ("kda_rmsnorm_gate_forward", "norm_gate.hip"),
    "rmsnorm_gate_backward": ("kda_rmsnorm_gate_backward", "norm_gate.hip"),
}


def kda_backend_provenance() -> dict:
    """Which native symbol and source own each component of the project backend."""
    from . import _lib

    return {
        "library": _lib.LIB_PATH,
        "components": {
            name: {"owner": "project", "symbol": sym, "source": f"csrc/{src}",
                   "torch_operator": f"nanochat_kda::{name}"}
            for name, (sym, src) in _COMPONENTS.items()
        },
    }


def prepare_kda_backend(backend: str = "fla_triton") -> None:
    """Load the native library and register ``torch.ops.nanochat_kda`` (fails closed).

    ``"project_cuda"`` and ``"fla_triton"`` (the reference's comparator slot) both name
    the HIP kernels here.
    """
    if backend not in {"project_cuda", "fla_triton"}:
        raise ValueError(f"unknown optimized KDA backend: {backend}")
    from . import _lib

    _lib.load()
    ops.register_operators()


# ---------------------------------------------------------------------------
# gate and validation
# ---------------------------------------------------------------------------

def _gate_shapes(raw_gate, A_log, dt_bias):
    if raw_gate.ndim != 4:
        raise ValueError("raw_gate must have shape [B, T, H, K]")
    heads, key_dim = raw_gate.shape[-2:]
    if A_log.shape != (heads,):
        raise ValueError(f"A_log must have shape {(heads,)}")
    if dt_bias.numel() != heads * key_dim:
        raise ValueError(f"dt_bias must contain {heads * key_dim} values")
    return heads, key_dim


def k3_decay_gate(raw_gate, A_log, dt_bias, lower_bound: float = -5.0):
    """K3 lower-bounded log decay: ``lb * sigmoid(exp(A) * (z+b))``."""
    heads, key_dim = _gate_shapes(raw_gate, A_log, dt_bias)
    if lower_bound >= 0:
        raise ValueError("lower_bound must be negative")
    return lower_bound * torch.sigmoid(A_log.exp().reshape(heads, 1) * (raw_gate + dt_bias.reshape(heads, key_dim)))


def _validate_operator_inputs(q, k, v, raw_gate, beta_logits, initial_state, num_states=None):
    if q.shape != k.shape or q.shape != raw_gate.shape or q.ndim != 4:
        raise ValueError("q, k, and raw_gate must share shape [B, T, H, K]")
    if v.ndim != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError("v must have shape [B, T, H, V]")
    if beta_logits.shape != q.shape[:3]:
        raise ValueError("beta logits must have shape [B, T, H]")
    batch, length, heads, key_dim = q.shape
    value_dim = v.shape[-1]
    if initial_state is not None:
        n = batch if num_states is None else num_states
        expected = (n, heads, value_dim, key_dim)
        if initial_state.shape != expected:
            raise ValueError(f"initial_state must be V-first [B, H, V, K] with shape {expected}")
    return batch, length, heads, key_dim, value_dim


def _reference_kda(q, k, v, raw_gate, beta_logits, A_log, dt_bias, *, initial_state, lower_bound,
                   scale, gate="k3"):
    """Eager f32 token-by-token recurrence with the semantics of reference kda.py:269-327.

    The state is kept value-major, ``S[b, h] : [V, K]``, the same layout as ``KDAState``,
    so no transposes are needed.  Per token t (all heads at once):
      S <- S * exp(g_t)             (per key channel, broadcast over V)
      S <- S + beta_t (v_t - S k_t) k_t^T
      o_t = S q_t
    with q, k unit-normalised per head (q additionally multiplied by ``scale``, default
    K^-1/2) and beta = sigmoid(beta_logits).  Differentiable by autograd; runs on any device.
    """
    n_b, n_t, n_h, n_k, n_v = _validate_operator_inputs(q, k, v, raw_gate, beta_logits, initial_state)
    q_scale = n_k ** -0.5 if scale is None else scale
    qs = F.normalize(q.float(), dim=-1) * q_scale
    ks = F.normalize(k.float(), dim=-1)
    vs = v.float()
    if gate == "k3":
        _gate_shapes(raw_gate, A_log, dt_bias)
        log_decay = k3_decay_gate(raw_gate.float(), A_log.float(), dt_bias.float(), lower_bound=lower_bound)
    else:
        log_decay = raw_gate.float()
    decay = log_decay.exp()
    beta = torch.sigmoid(beta_logits.float())
    S = (q.new_zeros(n_b, n_h, n_v, n_k, dtype=torch.float32) if initial_state is None
         else initial_state.float())
    rows = []
    for t in range(n_t):
        S = S * decay[:, t, :, None, :]
        k_t = ks[:, t]
        err = vs[:, t] - (S @ k_t[..., None])[..., 0]
        S = S + (beta[:, t, :, None] * err)[..., None] * k_t[:, :, None, :]
        rows.append((S @ qs[:, t, :, :, None])[..., 0])
    out = torch.stack(rows, 1) if rows else vs.new_zeros(n_b, 0, n_h, n_v)
    return out.to(v.dtype), S.contiguous()


def _backend_reason(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state, *, lower_bound,
                    gate):
    if not q.is_cuda:
        return "MI355X KDA requires a ROCm device"
    activations = (q, k, v, beta_logits) + ((raw_gate,) if gate == "k3" else ())
    params = (A_log, dt_bias) if gate == "k3" else ()
    if any(t.device != q.device for t in (*activations, raw_gate, *params)):
        return "all KDA tensors must be on the same device"
    if any(t.dtype != torch.bfloat16 for t in activations):
        return "MI355X KDA requires bfloat16 activations"
    if gate == "k3":
        if A_log.dtype != torch.float32 or dt_bias.dtype != torch.float32:
            return "A_log and dt_bias must be float32"
        if not (-5.0 <= lower_bound < 0.0):
            return "safe-gate lower_bound must be in [-5, 0)"
    elif raw_gate.dtype != torch.float32:
        return "a precomputed log decay must be float32"
    # 64 / 128 run the chunked kernels, other sizes the token-serial ones
    if not (1 <= q.shape[-1] <= 256 and 1 <= v.shape[-1] <= 4096):
        return "head dimensions must be K in [1, 256] and V in [1, 4096]"
    if initial_state is not None:
        if initial_state.device != q.device:
            return "initial_state must be on the same device as q"
        if initial_state.dtype != torch.float32:
            return "initial_state must be float32"
    return None


# ---------------------------------------------------------------------------
# autograd boundaries (reference kda.py:383-466)
# ---------------------------------------------------------------------------

class _ProjectKDAAutograd(torch.autograd.Function):
    """Chunked KDA: forward saves the residual workspace, backward runs the HIP VJP."""

    @staticmethod
    def forward(ctx, forward_component, backward_component, q, k, v, raw_gate, beta_logits, A_log,
                dt_bias, initial_state, output_final_state, lower_bound, scale, cu_seqlens=None,
                gate="k3"):
        output, final_state, workspace = ops.chunk_forward(
            q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state, output_final_state,
            lower_bound, scale, cu_seqlens=cu_seqlens, gate=gate)
        ctx.backward_component = backward_component
        ctx.has_initial = initial_state is not None
        ctx.lower_bound = lower_bound
        ctx.scale = scale
        ctx.gate = gate
        ctx.save_for_backward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                              workspace, cu_seqlens)
        return output, final_state

    @staticmethod
    def backward(ctx, grad_output, grad_final_state):
        q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state, workspace, cu_seqlens = ctx.saved_tensors
        grads = ops.chunk_backward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                                   workspace, grad_output, grad_final_state, ctx.lower_bound,
                                   ctx.scale, cu_seqlens=cu_seqlens, gate=ctx.gate)
        if len(grads) != 8:
            raise RuntimeError("project chunk backward must return eight gradients")
        dq, dk, dv, draw_gate, dbeta, dA, ddt, dinitial = grads
        if ddt is not None:
            ddt = ddt.reshape(dt_bias.shape)
        if not ctx.has_initial:
            dinitial = None
        return (None, None, dq, dk, dv, draw_gate, dbeta, dA, ddt, dinitial, None, None, None,
                None, None)


class _ProjectRMSNormGateAutograd(torch.autograd.Function):
    """Fused RMSNorm * sigmoid(gate) on the HIP kernels (reference kda.py:418-436)."""

    @staticmethod
    def forward(ctx, x, gate, weight, epsilon):
        output, inverse_rms = ops.rmsnorm_gate_forward(x, gate, weight, epsilon)
        ctx.epsilon = epsilon
        ctx.save_for_backward(x, gate, weight, inverse_rms)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        x, gate, weight, inverse_rms = ctx.saved_tensors
        dx, dgate, dweight = ops.rmsnorm_gate_backward(x, gate, weight, inverse_rms,
                                                       grad_output, ctx.epsilon)
        return dx, dgate, dweight, None


class _ProjectKDANormGateAutograd(torch.autograd.Function):
    """Chunked KDA with the output RMSNorm * sigmoid(gate) fused into its last kernel
    (producer/consumer fusion of reference kda.py:761-770).  The forward keeps o and the
    inverse RMS; the backward runs the norm VJP and then the chunk VJP on its dx."""

    @staticmethod
    def forward(ctx, q, k, v, raw_gate, beta_logits, A_log, dt_bias, output_gate, norm_weight,
                epsilon, lower_bound, scale, gate="k3"):
        o, normed, inverse_rms, _, workspace = ops.chunk_forward_norm_gate(
            q, k, v, raw_gate, beta_logits, A_log, dt_bias, None, False, lower_bound, scale,
            output_gate, norm_weight, epsilon, gate=gate)
        ctx.epsilon, ctx.lower_bound, ctx.scale, ctx.gate = epsilon, lower_bound, scale, gate
        ctx.save_for_backward(q, k, v, raw_gate, beta_logits, A_log, dt_bias, output_gate,
                              norm_weight, o, inverse_rms, workspace)
        return normed

    @staticmethod
    def backward(ctx, grad_normed):
        (q, k, v, raw_gate, beta_logits, A_log, dt_bias, output_gate, norm_weight, o,
         inverse_rms, workspace) = ctx.saved_tensors
        do, dgate_out, dweight = ops.rmsnorm_gate_backward(o, output_gate, norm_weight, inverse_rms,
                                                           grad_normed, ctx.epsilon)
        dq, dk, dv, draw_gate, dbeta, dA, ddt, _ = ops.chunk_backward(
            q, k, v, raw_gate, beta_logits, A_log, dt_bias, None, workspace, do, None,
            ctx.lower_bound, ctx.scale, gate=ctx.gate)
        if ddt is not None:
            ddt = ddt.reshape(dt_bias.shape)
        return (dq, dk, dv, draw_gate, dbeta, dA, ddt, dgate_out, dweight, None, None, None, None)


class _ProjectMixerCore(torch.autograd.Function):
    """The stateless mixer between the stacked input projection and o_proj, on the projection
    output y = [qkv_in | output gate | f_a | beta logits | pad] itself: f_b_proj of the f_a
    columns, then one chunk forward with the short convolution + SiLU of q, k, v in its first
    kernel (reading qkv_in in place) and the output RMSNorm * sigmoid(gate) in its last (the
    producer/consumer fusions of reference kda.py:744-770).  The backward runs the norm VJP,
    the chunk VJP (dq, dk, dv side by side) and the convolution VJP of the three projections
    in one launch, and writes every column block of dL/dy into one tensor (the convolution VJP
    and the f_b_proj input gradient straight into their column slices): no copies of the
    blocks on the way in, no concatenation on the way back."""

    @staticmethod
    def forward(ctx, y, conv_w16, fb_weight, fb_w16, A_log, dt_bias, norm_weight, epsilon, lower_bound,
                scale, heads, conv_q, conv_k, conv_v):
        # conv_q/k/v: the three f32 [C, 1, W] convolution weights; conv_w16 their stacked bf16
        # [3C, W] copy (made once per training update), else stacked here
        B, T, N = y.shape
        H = int(heads)
        C, D = fb_weight.shape  # f_b_proj: D -> C
        w16 = fb_w16 if fb_w16 is not None else fb_weight.to(torch.bfloat16)
        conv_weight = conv_w16 if conv_w16 is not None else \
            torch.cat([conv_q, conv_k, conv_v]).squeeze(1).to(torch.bfloat16)
        qkv_in = y[..., :3 * C]
        fa = y[..., 4 * C:4 * C + D]
        output_gate = y[..., 3 * C:4 * C].view(B, T, H, D)  # column slices, read in place
        beta_logits = y[..., 4 * C + D:4 * C + D + H]
        raw_gate = F.linear(fa, w16).view(B, T, H, D)
        q, k, v, o, normed, inverse_rms, workspace = ops.chunk_forward_conv_norm_gate(
            qkv_in, conv_weight, raw_gate, beta_logits, A_log, dt_bias, lower_bound, scale,
            output_gate, norm_weight, epsilon, H)
        ctx.epsilon, ctx.lower_bound, ctx.scale, ctx.dims = epsilon, lower_bound, scale, (C, D, H)
        ctx.save_for_backward(y, conv_weight, w16, q, k, v, raw_gate, beta_logits, A_log, dt_bias,
                              output_gate, norm_weight, o, inverse_rms, workspace)
        return normed

    @staticmethod
    def backward(ctx, grad_normed):
        (y, conv_weight, w16, q, k, v, raw_gate, beta_logits, A_log, dt_bias, output_gate, norm_weight, o,
         inverse_rms, workspace) = ctx.saved_tensors
        C, D, H = ctx.dims
        B, T, N = y.shape
        dy = torch.empty(B, T, N, dtype=torch.bfloat16, device=y.device)
        # every column block of dy is written by the kernel that produces it: the output-gate
        # gradient by the norm VJP, dbeta (and zeros in the pad columns) by the chunk VJP
        do, _, dweight = ops.rmsnorm_gate_backward(o, output_gate, norm_weight, inverse_rms, grad_normed,
                                                   ctx.epsilon, dgate_out=dy[..., 3 * C:4 * C].view(B, T, H, D))
        dqkv, _, _, draw_gate, _, dA, ddt, _ = ops.chunk_backward(
            q, k, v, raw_gate, beta_logits, A_log, dt_bias, None, workspace, do, None,
            ctx.lower_bound, ctx.scale, gate="k3", packed_qkv_grad=True,
            dbeta_out=dy[..., 4 * C + D:4 * C + D + H], dbeta_pad=N - (4 * C + D + H))
        _, dconv, _ = ops.causal_conv_backward(y[..., :3 * C], conv_weight, None, dqkv, None,
                                               dx_out=dy[..., :3 * C])
        g2 = draw_gate.reshape(B * T, C)
        dy2 = dy.view(B * T, N)
        torch.mm(g2, w16, out=dy2[:, 4 * C:4 * C + D])
        dfb = ops.weight_grad(g2, y.view(B * T, N)[:, 4 * C:4 * C + D])
        dcq, dck, dcv = dconv.float().view(3, C, 1, -1).unbind(0)
        return (dy, None, dfb, None, dA, ddt.reshape(dt_bias.shape), dweight, None, None, None, None,
                dcq, dck, dcv)


def kda_norm_gate(q, k, v, raw_gate, beta_logits, A_log, dt_bias, output_gate, norm_weight, *,
                  eps=1e-5, lower_bound=-5.0, scale=None, gate="k3"):
    """``rms_norm(kda(...), norm_weight, eps) * sigmoid(output_gate)`` for the chunked HIP
    path with the norm fused into the chunk forward's output kernel (no initial or final
    state, as in training).  Same validation and result as ``kda(mode="project_chunk")``
    followed by ``RMSNormGated``."""
    if gate not in ("k3", "precomputed"):
        raise ValueError(f"unknown gate parameterisation: {gate}")
    _validate_operator_inputs(q, k, v, raw_gate, beta_logits, None, None)
    if gate == "k3":
        _gate_shapes(raw_gate, A_log, dt_bias)
    reason = _backend_reason(q, k, v, raw_gate, beta_logits, A_log, dt_bias, None,
                             lower_bound=lower_bound, gate=gate)
    if reason is not None:
        raise RuntimeError(f"project CUDA KDA backend unavailable: {reason}")
    if q.shape[-1] not in (64, 128) or v.shape[-1] not in (64, 128):
        # the token-serial kernels have no fused epilogue: the norm runs as its own kernel
        out, _ = kda(q, k, v, raw_gate, beta_logits, A_log, dt_bias, mode="project_chunk",
                     lower_bound=lower_bound, scale=scale, gate=gate)
        out = _ProjectRMSNormGateAutograd.apply(out, output_gate, norm_weight, float(eps))
        _record("rmsnorm_gate_forward")
        return _record_backward(out, "rmsnorm_gate_backward")
    resolved_scale = float(scale if scale is not None else q.shape[-1] ** -0.5)
    out = _ProjectKDANormGateAutograd.apply(q, k, v, raw_gate, beta_logits, A_log, dt_bias,
                                            output_gate, norm_weight, float(eps),
                                            float(lower_bound), resolved_scale, gate)
    _record("chunk_forward_norm_gate")
    return _record_backward(out, "chunk_backward")


class _ProjectConvolutionAutograd(torch.autograd.Function):
    """Causal conv + SiLU on the HIP kernels (reference kda.py:439-466)."""

    @staticmethod
    def forward(ctx, forward_component, backward_component, x, weight, initial_state,
                output_final_state):
        output, final_state = ops.causal_conv_forward(x, weight, initial_state, output_final_state)
        ctx.backward_component = backward_component
        ctx.has_initial = initial_state is not None
        ctx.save_for_backward(x, weight, initial_state)
        return output, final_state

    @staticmethod
    def backward(ctx, grad_output, grad_final_state):
        x, weight, initial_state = ctx.saved_tensors
        dx, dweight, dinitial = ops.causal_conv_backward(x, weight, initial_state, grad_output,
                                                         grad_final_state)
        if not ctx.has_initial:
            dinitial = None
        return None, None, dx, dweight, dinitial, None


# ---------------------------------------------------------------------------
# operator entry point
# ---------------------------------------------------------------------------

def kda(q, k, v, raw_gate, beta_logits, A_log, dt_bias, *, initial_state=None,
        output_final_state=False, mode="reference", lower_bound=-5.0, scale=None,
        allow_fallback=True, cu_seqlens=None, gate="k3", state_in_place=False):
    """Run KDA through the requested backend (reference kda.py:561-673).

    Returns ``(output [B,T,H,V], final_state [N,H,V,K] or None)``.  ``project_*`` modes
    never fall back to the eager loop; ``chunk`` / ``recurrent`` run it for calls the HIP
    kernels cannot take when ``allow_fallback`` is true (reference kda.py:633-673).
    ``state_in_place`` (an extension for decode caches): a
    single-token recurrent step writes the new state into ``initial_state`` and returns
    that tensor, instead of allocating a new one; by default the initial state is never
    written, as in the reference.
    """
    if mode not in MODES:
        raise ValueError(f"unknown KDA mode: {mode}")
    if gate not in ("k3", "precomputed"):
        raise ValueError(f"unknown gate parameterisation: {gate}")
    num_states = None if cu_seqlens is None else int(cu_seqlens.numel()) - 1
    _validate_operator_inputs(q, k, v, raw_gate, beta_logits, initial_state, num_states)
    if gate == "k3":
        _gate_shapes(raw_gate, A_log, dt_bias)
    if mode == "reference":
        if cu_seqlens is not None:
            raise ValueError("mode='reference' does not take cu_seqlens")
        output, final_state = _reference_kda(q, k, v, raw_gate, beta_logits, A_log, dt_bias,
                                             initial_state=initial_state, lower_bound=lower_bound,
                                             scale=scale, gate=gate)
        return output, final_state if output_final_state else None

    prefix = "project CUDA KDA backend unavailable" if mode.startswith("project_") else \
        f"optimized {mode} KDA backend unavailable"
    reason = _backend_reason(q, k, v, raw_gate, beta_logits, A_log, dt_bias, initial_state,
                             lower_bound=lower_bound, gate=gate)
    requested = mode.removeprefix("project_")
    if requested == "recurrent" and torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q, k, v, raw_gate, beta_logits, A_log, dt_bias)):
        reason = f"{'project ' if mode.startswith('project_') else ''}recurrent KDA is inference-only"
    if reason is None and mode == "project_recurrent" and q.shape[1] != 1:
        reason = "project recurrent KDA decodes exactly one token per call"
    if reason is not None:
        if mode.startswith("project_") or not allow_fallback or cu_seqlens is not None:
            raise RuntimeError(f"{prefix}: {reason}")
        output, final_state = _reference_kda(q, k, v, raw_gate, beta_logits, A_log, dt_bias,
                                             initial_state=initial_state, lower_bound=lower_bound,
                                             scale=scale, gate=gate)
        return output, final_state if output_final_state else None
    if cu_seqlens is not None:
        cu_seqlens = cu_seqlens.to(device=q.device, dtype=torch.int32)
        host = cu_seqlens.cpu()
        if q.shape[0] != 1 or int(host[0]) != 0 or int(host[-1]) != q.shape[1] or bool((host[1:] < host[:-1]).any()):
            raise ValueError("cu_seqlens must start at 0, be non-decreasing and end at T (batch 1)")
    resolved_scale = float(scale if scale is not None else q.shape[-1] ** -0.5)
    if requested == "chunk":
        output, final_state = _ProjectKDAAutograd.apply(
            "chunk_forward", "chunk_backward", q, k, v, raw_gate, beta_logits, A_log, dt_bias,
            initial_state, output_final_state, float(lower_bound), resolved_scale, cu_seqlens, gate)
        _record("chunk_forward")
        return _record_backward(output, "chunk_backward"), final_state
    if q.shape[1] == 1 and cu_seqlens is None:
        in_place = state_in_place and initial_state is not None and initial_state.is_contiguous()
        output, final_state = ops.recurrent_decode(q, k, v, raw_gate, beta_logits, A_log, dt_bias,
                                                   initial_state, output_final_state,
                                                   float(lower_bound), resolved_scale, gate=gate,
                                                   out_state=initial_state if in_place else None)
        _record("recurrent_decode")
        return output, final_state
    output, final_state, _ = ops.chunk_forward(q, k, v, raw_gate, beta_logits, A_log, dt_bias,
                                               initial_state, output_final_state, float(lower_bound),
                                               resolved_scale, cu_seqlens=cu_seqlens, gate=gate)
    _record("chunk_forward")
    return output, final_state


# ---------------------------------------------------------------------------
# short convolution and the mixer block
# ---------------------------------------------------------------------------

def _short_conv_eager(x, weight, history):
    """Causal depthwise convolution + SiLU in the input's dtype.

    ``x`` [B, T, C]; ``weight`` [C, W]; ``history`` [B, C, W-1], the inputs that precede
    x[:, 0] (zeros for a fresh sequence).  y[b, t, c] = silu(sum_j weight[c, j] *
    z[b, c, t + j]) with z = history ++ x along time.  Returns (y, z)."""
    z = torch.cat((history, x.transpose(1, 2)), dim=2)          # [B, C, W-1+T]
    windows = z.unfold(2, weight.shape[1], 1)                    # [B, C, T, W]
    y = (windows * weight[None, :, None, :]).sum(-1)
    return F.silu(y).transpose(1, 2), z


class ShortConvolution(nn.Conv1d):
    """Per-channel causal convolution of width ``kernel_size`` followed by SiLU, with a
    cache that is passed in and returned, never written in place.

    The cache (``state``) is ``[B, C, W]``: the W most recent inputs, newest last, so a
    one-token call with the returned cache continues the sequence exactly.  The module is
    an ``nn.Conv1d`` only for its parameter (``weight`` [C, 1, W]); the forward never calls
    the library convolution.
    """

    def __init__(self, hidden_size: int, kernel_size: int = 4):
        super().__init__(hidden_size, hidden_size, kernel_size, groups=hidden_size, bias=False,
                         padding=kernel_size - 1)

    def forward(self, x, state=None, *, output_final_state=False, backend="fla_triton"):
        """``backend``: "project_cuda" / "fla_triton" run the HIP kernels on device tensors
        (the latter names the reference's comparator slot); "reference" runs the eager
        form on any device (reference kda.py:136-212)."""
        if x.ndim != 3 or x.shape[-1] != self.in_channels:
            raise ValueError(f"x must have shape [B,T,{self.in_channels}]")
        n_b, n_t, n_c = x.shape
        width = self.kernel_size[0]
        if state is not None and state.shape != (n_b, n_c, width):
            raise ValueError(f"convolution state must have shape {(n_b, n_c, width)}")
        cache = (x.new_zeros(n_b, n_c, width) if state is None
                 else state.to(device=x.device, dtype=x.dtype).clone())
        if n_t == 0:
            return x.new_empty(n_b, 0, n_c), (cache if output_final_state else None)
        taps = self.weight[:, 0, :].to(dtype=x.dtype)
        if x.is_cuda and backend != "reference":
            if backend not in {"fla_triton", "project_cuda"}:
                raise ValueError(f"unknown CUDA short-convolution backend: {backend}")
            y, last = _ProjectConvolutionAutograd.apply(
                "causal_convolution_forward", "causal_convolution_backward", x, taps,
                cache if state is not None else None, output_final_state)
            _record("causal_convolution_forward")
            return _record_backward(y, "causal_convolution_backward"), last
        if backend == "project_cuda":
            raise RuntimeError("project CUDA causal convolution cannot fall back on CPU")
        y, z = _short_conv_eager(x, taps, cache[..., 1:])
        # a copy, so the returned cache does not keep the whole sequence alive
        return y, (z[..., z.shape[-1] - width:].clone() if output_final_state else None)


class KimiDeltaAttention(nn.Module):
    """The KDA token mixer of one decoder layer (reference kda.py:676-798).

    x -> q, k, v projections, each through its short convolution + SiLU; a low-rank
    (f_a, f_b) projection gives the per-channel K3 gate input and ``b_proj`` the beta
    logits; the KDA recurrence; a per-head RMS norm gated by sigmoid(g_proj(x)); the
    output projection.  Parameter names, shapes and initial values follow the reference
    so state dicts are interchangeable.
    """

    def __init__(self, hidden_size: int, num_heads: int, head_dim: int, conv_size: int = 4,
                 layer_idx: int | None = None, mode: str = "reference", norm_eps: float = 1e-5,
                 lower_bound: float = -5.0, allow_fallback: bool = True):
        super().__init__()
        if hidden_size != num_heads * head_dim:
            raise ValueError("initial KDA implementation requires hidden_size = num_heads * head_dim")
        if conv_size <= 0:
            raise ValueError("conv_size must be positive")
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.conv_size = conv_size
        self.layer_idx = layer_idx
        self.mode = mode
        self.lower_bound = lower_bound
        self.allow_fallback = allow_fallback
        # stateless training path: run the three short convolutions inside the chunk
        # forward's first kernel (False: the separate convolution launch; same results)
        self.fuse_conv = True

        self.q_proj = Linear(hidden_size, hidden_size, bias=False)
        self.k_proj = Linear(hidden_size, hidden_size, bias=False)
        self.v_proj = Linear(hidden_size, hidden_size, bias=False)
        self.q_conv1d = ShortConvolution(hidden_size, conv_size)
        self.k_conv1d = ShortConvolution(hidden_size, conv_size)
        self.v_conv1d = ShortConvolution(hidden_size, conv_size)

        self.A_log = nn.Parameter(torch.zeros(num_heads, dtype=torch.float32))
        self.f_a_proj = Linear(hidden_size, head_dim, bias=False)
        self.f_b_proj = Linear(head_dim, hidden_size, bias=False)
        self.dt_bias = nn.Parameter(torch.zeros(hidden_size, dtype=torch.float32))
        self.b_proj = Linear(hidden_size, num_heads, bias=False)

        self.g_proj = Linear(hidden_size, hidden_size, bias=False)
        self.o_norm = RMSNormGated(head_dim, eps=norm_eps)
        self.o_proj = Linear(hidden_size, hidden_size, bias=False)

    def forward(self, hidden_states, state: KDAState | None = None, output_final_state: bool = False,
                mode: str | None = None, allow_fallback: bool | None = None,
                state_in_place: bool = False):
        """``state_in_place`` (extension): a one-token recurrent step updates
        ``state.memory`` in place (see ``kda``); the returned state holds that tensor."""
        if hidden_states.ndim != 3 or hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"hidden_states must have shape [B,T,{self.hidden_size}]")
        mode = self.mode if mode is None else mode
        fallback = self.allow_fallback if allow_fallback is None else allow_fallback
        if state is None and not output_final_state and self._batched_ok(hidden_states, mode):
            return self._forward_batched(hidden_states, mode, fallback), None
        return self._forward_stepwise(hidden_states, state, output_final_state, mode, fallback,
                                      state_in_place)

    def _batched_ok(self, x, mode):
        # the stacked-projection path needs no carried state and the HIP kernels' dtypes
        return (mode in ("project_chunk", "chunk") and x.is_cuda and x.dtype == torch.bfloat16
                and x.shape[1] > 0 and self.q_proj.weight.dtype == torch.float32)

    def _forward_stepwise(self, x, state, keep_state, mode, fallback, state_in_place):
        """General path (carried state, decode, CPU, reference mode): each of q, k, v is its
        own projection followed by its short convolution, whose window is read from and
        returned in the ``KDAState``."""
        heads = (x.shape[0], x.shape[1], self.num_heads, self.head_dim)
        backend = {"reference": "reference"}.get(mode, "project_cuda" if mode.startswith("project_")
                                                 else "fla_triton")
        branches = {}
        for name in ("q", "k", "v"):
            carry = getattr(state, f"{name}_conv") if state is not None else None
            conv = getattr(self, f"{name}_conv1d")
            seq, window = conv(getattr(self, f"{name}_proj")(x), carry, output_final_state=keep_state,
                               backend=backend)
            branches[name] = (seq.reshape(heads), window)
        gate_in = self.f_b_proj(self.f_a_proj(x)).reshape(heads)
        out, memory = kda(branches["q"][0], branches["k"][0], branches["v"][0], gate_in, self.b_proj(x),
                          self.A_log, self.dt_bias,
                          initial_state=state.memory if state is not None else None,
                          output_final_state=keep_state, mode=mode, lower_bound=self.lower_bound,
                          allow_fallback=fallback, state_in_place=state_in_place)
        out = self._gated_norm(out, self.g_proj(x).reshape(heads), mode)
        y = self.o_proj(out.reshape(x.shape[0], x.shape[1], self.hidden_size))
        if not keep_state:
            return y, None
        return y, KDAState(memory, branches["q"][1], branches["k"][1], branches["v"][1])

    def _gated_norm(self, o, gate, mode):
        """RMSNorm(o)·sigmoid(gate): the HIP kernel pair whenever its dtypes and head size fit,
        else the module's own (eager or per-op) path."""
        kernel_fits = (mode != "reference" and o.is_cuda and o.dtype == torch.bfloat16
                       and gate.dtype == torch.bfloat16 and self.head_dim <= 1024
                       and self.o_norm.weight.dtype == torch.float32)
        if not kernel_fits:
            return self.o_norm(o, gate)
        o = _ProjectRMSNormGateAutograd.apply(o, gate, self.o_norm.weight, self.o_norm.eps)
        _record("rmsnorm_gate_forward")
        return _record_backward(o, "rmsnorm_gate_backward")

    def _in_pad(self):
        return -(4 * self.hidden_size + self.head_dim + self.num_heads) % 8

    def stacked_input_weight_bf16(self):
        """The stacked bf16 input projection [W_q; W_k; W_v; W_g; W_fa; W_b; 0] that the
        stateless path multiplies by (built from the current f32 weights)."""
        w = self._in_weights()
        return torch.cat(list(w) + [w[0].new_zeros(self._in_pad(), w[0].shape[1])]).to(torch.bfloat16)

    def _in_weights(self):
        return (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.g_proj.weight,
                self.f_a_proj.weight, self.b_proj.weight)

    def _forward_batched(self, hidden_states, mode, allow_fallback):
        """Stateless training / prefill path: the same computation as ``forward`` with the six
        projections that read ``hidden_states`` (q, k, v, g, f_a, b) as one GEMM and the three
        short convolutions as one launch over the concatenated channels.  One weight-gradient
        and one input-gradient GEMM replace six of each, and the input gradient needs no
        accumulation of six partial gradients."""
        batch, length, C = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        # zero rows pad the output width to a multiple of 8 (16-byte rows for the kernels)
        pad = self._in_pad()
        y = _StackedLinearBF16.apply(hidden_states, getattr(self, "_w16_in", None), pad, *self._in_weights())
        convs = (self.q_conv1d.weight, self.k_conv1d.weight, self.v_conv1d.weight)
        if D in (64, 128) and convs[0].shape[-1] <= 4 and self.o_norm.weight.dtype == torch.float32 \
                and self.fuse_conv and self.f_b_proj.weight.dtype == torch.float32 \
                and all(w.dtype == torch.float32 for w in convs):
            # the column blocks of y read in place; convolution in the chunk forward's first
            # kernel, output norm in its last
            mixed = _ProjectMixerCore.apply(
                y, getattr(self, "_conv_w16", None), self.f_b_proj.weight, getattr(self.f_b_proj, "_w16", None),
                self.A_log, self.dt_bias, self.o_norm.weight, float(self.o_norm.eps), float(self.lower_bound),
                float(D ** -0.5), H, *convs)
            _record("chunk_forward_conv_norm_gate")
            mixed = _record_backward(mixed, "chunk_backward")
            return self.o_proj(mixed.reshape(batch, length, C))
        conv_w = torch.cat(convs, dim=0).squeeze(1).to(torch.bfloat16)
        qkv_in, gate_lin, fa, beta_logits, _ = _SplitColumns.apply(y, (3 * C, C, D, H, pad))
        raw_gate = self.f_b_proj(fa).view(batch, length, H, D)
        output_gate = gate_lin.view(batch, length, H, D)
        qkv, _ = _ProjectConvolutionAutograd.apply("causal_convolution_forward", "causal_convolution_backward",
                                                   qkv_in, conv_w, None, False)
        _record("causal_convolution_forward")
        qkv = _record_backward(qkv, "causal_convolution_backward")
        q, k, v = (t.view(batch, length, H, D) for t in _SplitColumns.apply(qkv, (C, C, C)))
        if D in (64, 128) and self.o_norm.weight.dtype == torch.float32:
            # the output norm fused into the chunk forward's last kernel
            mixed = kda_norm_gate(q, k, v, raw_gate, beta_logits, self.A_log, self.dt_bias, output_gate,
                                  self.o_norm.weight, eps=self.o_norm.eps, lower_bound=self.lower_bound)
            return self.o_proj(mixed.reshape(batch, length, C))
        mixed, _ = kda(q, k, v, raw_gate, beta_logits, self.A_log, self.dt_bias, initial_state=None,
                       output_final_state=False, mode=mode, lower_bound=self.lower_bound,
                       allow_fallback=allow_fallback)
        return self.o_proj(self._gated_norm(mixed, output_gate, mode).reshape(batch, length, C))


__all__ = ["KDAState", "KimiDeltaAttention", "k3_decay_gate", "kda", "kda_norm_gate", "prepare_kda_backend",
           "ShortConvolution", "RMSNormGated", "Linear", "kda_backend_provenance",
           "project_runtime_events", "reset_project_runtime_events"]
