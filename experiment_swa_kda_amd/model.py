"""All-KDA nanochat-style decoder used to measure training throughput.

Restates the structure of the reference model for the ``window_pattern="K"`` case
(nanochat/gpt.py: ``Block`` :159-205, ``GPT.__init__`` :208-260, ``init_weights``
:262-330, ``forward`` :543-600): bf16 token embedding, RMS norms, smear gate,
per-layer residual / x0 scalars, KDA mixer + ReLU^2 MLP blocks, mid-depth backout,
soft-capped logits and cross entropy.  Master weights stay f32 and are cast to the
activation dtype inside ``Linear`` (nanochat/gpt.py:52-57).  The KDA mixer is the HIP
``KimiDeltaAttention`` of this package in ``project_chunk`` mode (conv, KDA core and
output norm-gate on the gfx950 kernels; projections are PyTorch GEMMs).  With a
``KVCache`` (nanochat/engine.py:92-221) the model prefills through the chunk kernels and
decodes one token at a time through the recurrent decode kernel.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .kda import KDAState, KimiDeltaAttention, Linear


@dataclass
class GPTConfig:
    sequence_len: int = 4096
    vocab_size: int = 32768
    n_layer: int = 6
    n_head: int = 3
    n_embd: int = 384
    mode: str = "project_chunk"


class KVCache:
    """Inference cache for a decoder whose layers are all KDA mixers.

    Interface of nanochat/engine.py:92-221 (constructor arguments, ``reset``, ``get_pos``,
    ``get_kda_state`` / ``set_kda_state``, ``advance``, ``prefill``, ``state_nbytes`` and
    their exceptions) restricted to KDA layers: a KDA layer's whole history is its
    fixed-size ``KDAState`` (f32 memory [B,H,V,K] and three conv windows), so nothing
    grows with the sequence.  ``mixer_types`` entries other than "K" are rejected, since
    attention layers are not part of this build.  ``prev_embedding`` holds the last
    token's normalised embedding for the model's smear.  ``inplace_state`` (extension):
    one-token steps overwrite each layer's memory tensor instead of allocating a new one.
    """

    def __init__(self, batch_size, num_heads, seq_len, head_dim, num_layers, device, dtype,
                 mixer_types=None, conv_size=4, inplace_state=False):
        kinds = tuple(mixer_types) if mixer_types else ("K",) * num_layers
        if len(kinds) != num_layers or not set(kinds) <= set("LSK"):
            raise ValueError("mixer_types must contain one L/S/K entry per layer")
        if set(kinds) != {"K"}:
            raise ValueError("this cache holds KDA layers only; attention layers are not part of this build")
        self.mixer_types = kinds
        self.batch_size, self.max_seq_len = batch_size, seq_len
        self.n_layers, self.n_heads, self.head_dim = num_layers, num_heads, head_dim
        self.conv_size, self.inplace_state = conv_size, inplace_state
        self.allocated_kv_layers = ()
        self.allocated_kda_layers = tuple(range(num_layers))
        self._states: list[KDAState | None] = [None] * num_layers
        self.cache_seqlens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        self.prev_embedding = None

    def _kda_slot(self, layer_idx):
        if layer_idx not in self.allocated_kda_layers:
            raise ValueError(f"layer {layer_idx} is attention and has no KDA state")
        return layer_idx

    def reset(self):
        self._states = [None] * self.n_layers
        self.prev_embedding = None
        self.cache_seqlens.zero_()

    def get_pos(self):
        return int(self.cache_seqlens[0].item())

    def get_layer_cache(self, layer_idx):
        raise ValueError(f"layer {layer_idx} is KDA and has no KV cache")

    def get_kda_state(self, layer_idx):
        return self._states[self._kda_slot(layer_idx)]

    def set_kda_state(self, layer_idx, state):
        slot = self._kda_slot(layer_idx)
        if not (state is None or isinstance(state, KDAState)):
            raise TypeError("KDA state must be a KDAState instance")
        self._states[slot] = state

    def advance(self, num_tokens):
        self.cache_seqlens.add_(num_tokens)

    def _to_batch(self, t):
        """A private copy of ``t`` with batch ``self.batch_size`` (a batch of one is
        repeated)."""
        if t.shape[0] != 1 and t.shape[0] != self.batch_size:
            raise ValueError("source KDA state batch cannot be expanded to destination")
        return t.expand(self.batch_size, *t.shape[1:]).clone()

    def prefill(self, other):
        """Start this cache from ``other`` (typically a batch-1 prompt prefill that is then
        sampled several times): copies every layer state and the smear embedding."""
        if self.get_pos() != 0:
            raise ValueError("Cannot prefill a non-empty KV cache")
        if (other.n_layers, other.n_heads, other.head_dim) != (self.n_layers, self.n_heads, self.head_dim):
            raise ValueError("cache geometry mismatch")
        if other.mixer_types != self.mixer_types or other.max_seq_len > self.max_seq_len:
            raise ValueError("cache layout mismatch")
        self._states = [
            None if st is None else KDAState(*(self._to_batch(t) for t in (st.memory, st.q_conv, st.k_conv, st.v_conv)))
            for st in (other.get_kda_state(i) for i in self.allocated_kda_layers)
        ]
        self.cache_seqlens.fill_(other.get_pos())
        if other.prev_embedding is not None:
            self.prev_embedding = self._to_batch(other.prev_embedding)

    def state_nbytes(self):
        total = 0
        for st in self._states:
            if st is not None:
                total += sum(t.numel() * t.element_size() for t in (st.memory, st.q_conv, st.k_conv, st.v_conv))
        if self.prev_embedding is not None:
            total += self.prev_embedding.numel() * self.prev_embedding.element_size()
        return total


class _SoftcapCrossEntropy(torch.autograd.Function):
    """Mean soft-capped cross entropy on the HIP kernels: forward reads the bf16 logits once,
    backward reads them again and writes the bf16 logit gradient (nanochat/gpt.py:600-608)."""

    @staticmethod
    def forward(ctx, logits, targets, vocab, softcap, ignore_index):
        loss_rows, lse = ops.softcap_cross_entropy_forward(logits, targets, vocab, softcap, ignore_index)
        loss, count = ops.softcap_cross_entropy_mean(loss_rows, targets, ignore_index)
        ctx.save_for_backward(logits, targets, lse, count)
        ctx.args = (vocab, softcap, ignore_index)
        return loss

    @staticmethod
    def backward(ctx, grad):
        logits, targets, lse, count = ctx.saved_tensors
        vocab, softcap, ignore_index = ctx.args
        scale = grad.float() / count
        dlogits = ops.softcap_cross_entropy_backward(logits, targets, lse, scale, vocab, softcap,
                                                     ignore_index)
        return dlogits, None, None, None, None


class _SoftcapCrossEntropyFused(torch.autograd.Function):
    """The same loss with its gradient formed in the forward pass: one read of the logits
    writes the row losses and the logit gradient for an assumed upstream gradient
    ``expected_grad``.  The backward returns that buffer, rescaled on the device only if the
    actual upstream gradient differs (no host synchronisation either way)."""

    @staticmethod
    def forward(ctx, logits, targets, vocab, softcap, ignore_index, expected_grad):
        loss_rows, _, dlogits, _ = ops.softcap_cross_entropy_fused(logits, targets, vocab, softcap,
                                                                   ignore_index, expected_grad)
        loss, _ = ops.softcap_cross_entropy_mean(loss_rows, targets, ignore_index)
        ctx.save_for_backward(dlogits)
        ctx.expected = expected_grad
        ctx.used = False
        return loss

    @staticmethod
    def backward(ctx, grad):
        if ctx.used:  # the gradient buffer is handed out (and rescaled) in place
            raise RuntimeError("softcap_cross_entropy: the fused form's backward can run only once")
        ctx.used = True
        (dlogits,) = ctx.saved_tensors
        ops.rescale_bf16_if_changed(dlogits, grad, ctx.expected)
        return dlogits, None, None, None, None, None


def softcap_cross_entropy(logits, targets, vocab, softcap=15.0, ignore_index=-1, expected_grad=None):
    """mean cross_entropy(softcap * tanh(logits[:, :vocab] / softcap), targets) over rows whose
    target is not ignore_index; logits [rows, padded vocab].  bf16 CUDA logits run the fused
    HIP kernels, anything else the eager f32 form.  With ``expected_grad`` (the dL/dloss the
    caller will back-propagate) and a gradient to form, rows whose columns are all vocabulary
    take the one-pass forward + backward kernel."""
    if logits.is_cuda and logits.dtype == torch.bfloat16:
        if (expected_grad is not None and expected_grad != 0 and torch.is_grad_enabled() and logits.requires_grad
                and logits.ndim == 2 and ops.softcap_cross_entropy_fused_supported(vocab, logits.shape[1])):
            return _SoftcapCrossEntropyFused.apply(logits, targets, vocab, float(softcap), ignore_index,
                                                   float(expected_grad))
        return _SoftcapCrossEntropy.apply(logits, targets, vocab, float(softcap), ignore_index)
    z = softcap * torch.tanh(logits[:, :vocab].float() / softcap)
    return F.cross_entropy(z, targets, ignore_index=ignore_index)


class _Relu2(torch.autograd.Function):
    """relu(x)^2 as one HIP pass forward and one backward (nanochat/gpt.py:151-156)."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return ops.relu2_forward(x)

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        return ops.relu2_backward(x, grad)


class _EmbeddingLookup(torch.autograd.Function):
    """Token-embedding lookup whose backward is the library's sort-free embedding gradient:
    the library sort + unique path of the default backward records memory-set nodes, which
    must stay out of a captured HIP graph."""

    @staticmethod
    def forward(ctx, idx, weight):
        ctx.save_for_backward(idx)
        ctx.vocab = weight.shape[0]
        return F.embedding(idx, weight)

    @staticmethod
    def backward(ctx, grad):
        (idx,) = ctx.saved_tensors
        return None, ops.embedding_backward(idx, grad, ctx.vocab)


def embed(table: nn.Embedding, idx):
    w = table.weight
    if w.is_cuda and w.dtype == torch.bfloat16 and w.shape[1] % 8 == 0 and w.shape[1] <= 512:
        return _EmbeddingLookup.apply(idx, w)
    return table(idx)


class _ScalarScale(torch.autograd.Function):
    """lam.to(t.dtype) * t for a one-element f32 parameter ``lam`` and a bf16 tensor ``t``;
    the gradient of ``lam`` (a sum over every element of t) comes from the library's
    fixed-order reduction (the weight-gradient kernel with N = K = 1)."""

    @staticmethod
    def forward(ctx, lam, t):
        ctx.save_for_backward(lam, t)
        return lam.to(t.dtype) * t

    @staticmethod
    def backward(ctx, grad):
        lam, t = ctx.saved_tensors
        dlam = ops.weight_grad(grad.reshape(-1, 1), t.reshape(-1, 1)).reshape(lam.shape)
        return dlam, grad * lam.to(grad.dtype)


def scalar_scale(lam, t):
    if t.is_cuda and t.dtype == torch.bfloat16 and lam.numel() == 1:
        return _ScalarScale.apply(lam, t)
    return lam.to(t.dtype) * t


def relu2(x):
    if x.is_cuda and x.dtype == torch.bfloat16 and x.numel() % 8 == 0:
        return _Relu2.apply(x)
    return F.relu(x).square()


class _ResidMix(torch.autograd.Function):
    """x = resid_lambdas[i] x + x0_lambdas[i] x0 (nanochat/gpt.py:585-587) as one HIP pass;
    the backward forms dx, dx0 and both scalar gradients in one pass plus a fixed-order
    reduction."""

    @staticmethod
    def forward(ctx, x, x0, lam_r, lam_0, i):
        ctx.save_for_backward(x, x0, lam_r, lam_0)
        ctx.i = i
        return ops.resid_mix_forward(x, x0, lam_r[i:i + 1], lam_0[i:i + 1])

    @staticmethod
    def backward(ctx, grad):
        x, x0, lam_r, lam_0 = ctx.saved_tensors
        dx, dx0, da, db = ops.resid_mix_backward(x, x0, lam_r, lam_0, ctx.i, grad)
        return dx, dx0, da, db, None


def resid_mix(x, x0, lam_r, lam_0, i):
    if (x.is_cuda and x.dtype == torch.bfloat16 and x0.dtype == torch.bfloat16
            and x.shape == x0.shape and x.numel() % 8 == 0):
        return _ResidMix.apply(x, x0, lam_r, lam_0, i)
    return lam_r[i] * x + lam_0[i] * x0


class _RMSNorm(torch.autograd.Function):
    """F.rms_norm(x, (D,)) without weight on the HIP row kernels (nanochat/gpt.py:46-48)."""

    @staticmethod
    def forward(ctx, x, eps):
        y, rinv = ops.rms_norm_forward(x, eps)
        ctx.save_for_backward(x, rinv)
        return y

    @staticmethod
    def backward(ctx, grad):
        x, rinv = ctx.saved_tensors
        return ops.rms_norm_backward(x, rinv, grad), None


# F.rms_norm's default eps for a bf16 input (its f32 computation type)
_RMS_EPS = torch.finfo(torch.float32).eps


def norm(x):
    D = x.size(-1)
    if x.is_cuda and x.dtype == torch.bfloat16 and D % 128 == 0 and D // 128 in (1, 2, 3, 4, 6, 8):
        return _RMSNorm.apply(x, _RMS_EPS)
    return F.rms_norm(x, (D,))


def _norm_fusable(x):
    D = x.size(-1)
    return x.is_cuda and x.dtype == torch.bfloat16 and D % 128 == 0 and D // 128 in (1, 2, 3, 4, 6, 8)


class _ResidMixNorm(torch.autograd.Function):
    """(s, norm(s)) for s = resid_lambdas[i] x + x0_lambdas[i] x0 in one pass (the residual
    mix of nanochat/gpt.py:585-587 and the pre-norm of the block it feeds, gpt.py:200).  The
    backward adds the gradient that reaches s through the residual branch to the norm VJP in
    the same pass (no separate accumulation), then runs the residual-mix VJP."""

    @staticmethod
    def forward(ctx, x, x0, lam_r, lam_0, i, eps):
        s, y, rinv = ops.mix_rms_norm_forward(x, x0, eps, lam_r[i:i + 1], lam_0[i:i + 1])
        ctx.save_for_backward(x, x0, lam_r, lam_0, s, rinv)
        ctx.i = i
        return s, y

    @staticmethod
    def backward(ctx, grad_s, grad_y):
        x, x0, lam_r, lam_0, s, rinv = ctx.saved_tensors
        t = grad_s if grad_y is None else ops.rms_norm_backward(s, rinv, grad_y, grad_s)
        if t is None:
            return None, None, None, None, None, None
        dx, dx0, da, db = ops.resid_mix_backward(x, x0, lam_r, lam_0, ctx.i, t)
        return dx, dx0, da, db, None, None


class _AddNorm(torch.autograd.Function):
    """(s, norm(s)) for the residual add s = a + b (gpt.py:202-205) in one pass; the backward
    forms the gradient of s (residual branch + norm VJP) in one pass and hands it to both."""

    @staticmethod
    def forward(ctx, a, b, eps):
        s, y, rinv = ops.mix_rms_norm_forward(a, b, eps)
        ctx.save_for_backward(s, rinv)
        return s, y

    @staticmethod
    def backward(ctx, grad_s, grad_y):
        s, rinv = ctx.saved_tensors
        t = grad_s if grad_y is None else ops.rms_norm_backward(s, rinv, grad_y, grad_s)
        return t, t, None


class MLP(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.c_fc = Linear(d, 4 * d, bias=False)
        self.c_proj = Linear(4 * d, d, bias=False)

    def forward(self, x):
        return self.c_proj(relu2(self.c_fc(x)))


class Block(nn.Module):
    def __init__(self, cfg: GPTConfig, layer_idx: int):
        super().__init__()
        self.attn = KimiDeltaAttention(cfg.n_embd, cfg.n_head, cfg.n_embd // cfg.n_head, conv_size=4,
                                       layer_idx=layer_idx, mode=cfg.mode, allow_fallback=False)
        self.mlp = MLP(cfg.n_embd)

    def forward(self, x, kv_cache=None):
        """nanochat/gpt.py:180-205 for a KDA layer: with a cache, the layer's state is read
        from and written back to it, and a one-token step runs the recurrent decode kernel."""
        state = None if kv_cache is None else kv_cache.get_kda_state(self.attn.layer_idx)
        mode = None
        if x.is_cuda and self.attn.mode.startswith("project_"):
            mode = "project_recurrent" if kv_cache is not None and x.shape[1] == 1 else "project_chunk"
        mixed, state = self.attn(norm(x), state=state, output_final_state=kv_cache is not None, mode=mode,
                                 state_in_place=kv_cache is not None and kv_cache.inplace_state)
        if kv_cache is not None:
            kv_cache.set_kda_state(self.attn.layer_idx, state)
        x = x + mixed
        return x + self.mlp(norm(x))

    def forward_mixed(self, x, x0, lam_r, lam_0, i):
        """The training path of ``block(resid_mix(x, x0, lam_r, lam_0, i))`` (no cache) with
        the residual mix fused into the first norm and the residual add into the second;
        the same values."""
        xin, h = _ResidMixNorm.apply(x, x0, lam_r, lam_0, i, _RMS_EPS)
        mode = "project_chunk" if self.attn.mode.startswith("project_") else None
        mixed, _ = self.attn(h, state=None, output_final_state=False, mode=mode)
        y, h2 = _AddNorm.apply(xin, mixed, _RMS_EPS)
        return y + self.mlp(h2)


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig, pad_vocab_size_to: int = 64):
        super().__init__()
        self.config = cfg
        padded = ((cfg.vocab_size + pad_vocab_size_to - 1) // pad_vocab_size_to) * pad_vocab_size_to
        self.padded_vocab = padded
        self.transformer = nn.ModuleDict({
            "wte": nn.Embedding(padded, cfg.n_embd),
            "h": nn.ModuleList([Block(cfg, i) for i in range(cfg.n_layer)]),
        })
        self.lm_head = Linear(cfg.n_embd, padded, bias=False)
        self.resid_lambdas = nn.Parameter(torch.ones(cfg.n_layer))
        self.x0_lambdas = nn.Parameter(torch.zeros(cfg.n_layer))
        self.smear_gate = Linear(24, 1, bias=False)
        self.smear_lambda = nn.Parameter(torch.zeros(1))
        self.backout_lambda = nn.Parameter(0.2 * torch.ones(1))
        # the constant weight of x in the backout mix x - backout_lambda * mid
        self.register_buffer("_one", torch.ones(1), persistent=False)
        # the dL/dloss the caller will back-propagate (1 for loss.backward()); the soft-capped
        # cross entropy forms its logit gradient for it in the forward pass and rescales in
        # the backward only if the actual one differs.  None: gradient formed in the backward.
        self.loss_grad_hint = 1.0

    def cache_bf16_weights(self) -> list:
        """Casts the f32 projection weights to bf16 once: every Linear the forward calls and
        each mixer's stacked input projection and stacked convolution weights keep the copy and use it until
        drop_bf16_weights() (one training update's microsteps all see the same weights).
        Returns the copies."""
        out = []
        with torch.no_grad():
            stacked = set()
            for m in self.modules():
                if isinstance(m, KimiDeltaAttention):
                    m._w16_in = m.stacked_input_weight_bf16()
                    m._conv_w16 = torch.cat([m.q_conv1d.weight, m.k_conv1d.weight, m.v_conv1d.weight]
                                            ).squeeze(1).to(torch.bfloat16)
                    out += [m._w16_in, m._conv_w16]
                    stacked.update(id(w) for w in m._in_weights())
            for m in self.modules():
                if isinstance(m, Linear) and m.weight.dtype == torch.float32 and id(m.weight) not in stacked:
                    m._w16 = m.weight.to(torch.bfloat16)
                    out.append(m._w16)
        return out

    def drop_bf16_weights(self) -> None:
        for m in self.modules():
            if isinstance(m, KimiDeltaAttention):
                m._w16_in = None
                m._conv_w16 = None
            if isinstance(m, Linear):
                m._w16 = None

    @torch.no_grad()
    def init_weights(self, generator=None):
        """Initialisation of nanochat/gpt.py:262-330 for KDA blocks."""
        d = self.config.n_embd
        s = 3 ** 0.5 * d ** -0.5
        nn.init.normal_(self.transformer.wte.weight, 0.0, 0.8, generator=generator)
        nn.init.normal_(self.lm_head.weight, 0.0, 0.001, generator=generator)
        for block in self.transformer.h:
            m = block.attn
            for proj in (m.q_proj, m.k_proj, m.v_proj, m.f_a_proj, m.f_b_proj, m.b_proj, m.g_proj):
                nn.init.uniform_(proj.weight, -s, s, generator=generator)
            for conv in (m.q_conv1d, m.k_conv1d, m.v_conv1d):
                nn.init.uniform_(conv.weight, -s, s, generator=generator)
            nn.init.zeros_(m.A_log)
            dt = torch.exp(torch.rand(m.dt_bias.shape, generator=generator, device=m.dt_bias.device)
                           * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp(min=1e-4)
            m.dt_bias.copy_(dt + torch.log(-torch.expm1(-dt)))
            nn.init.ones_(m.o_norm.weight)
            nn.init.zeros_(m.o_proj.weight)
            nn.init.uniform_(block.mlp.c_fc.weight, -s * 0.4, s * 0.4, generator=generator)
            nn.init.zeros_(block.mlp.c_proj.weight)
        n = self.config.n_layer
        for i in range(n):
            self.resid_lambdas[i] = 1.15 - 0.10 * i / max(n - 1, 1)
            self.x0_lambdas[i] = 0.20 - 0.15 * i / max(n - 1, 1)
        nn.init.zeros_(self.smear_lambda)
        nn.init.constant_(self.backout_lambda, 0.2)
        nn.init.uniform_(self.smear_gate.weight, 0.0, 0.02, generator=generator)
        self.transformer.wte.to(dtype=torch.bfloat16)

    def _smear(self, x, before):
        """Adds a gated copy of each token's predecessor embedding (a cheap bigram feature,
        nanochat/gpt.py:564-581).  ``before`` is the embedding preceding x[:, 0], or None
        when position 0 has no predecessor (it is then left unchanged)."""
        if before is None:
            if x.shape[1] < 2:
                return x
            head, tail, prev = x[:, :1], x[:, 1:], x[:, :-1]
        else:
            head, tail, prev = x[:, :0], x, torch.cat([before, x[:, :-1]], dim=1)
        weight = scalar_scale(self.smear_lambda, torch.sigmoid(self.smear_gate(tail[..., :24])))
        return torch.cat([head, tail + weight * prev], dim=1)

    def forward(self, idx, targets=None, kv_cache=None):
        """Logits ``15 tanh(lm_head(x)/15)`` [B, T, vocab] in f32, or with ``targets`` the
        mean cross entropy of those logits (the forward of nanochat/gpt.py:543-608 for an
        all-KDA model: no rotary tables or value embeddings).  With a cache, a prompt
        prefill (T > 1) smears within the prompt only, and a one-token step smears with the
        cached previous embedding."""
        n_tok = idx.shape[1]
        x = norm(embed(self.transformer.wte, idx).to(torch.bfloat16))
        before = None
        if kv_cache is not None:
            before = kv_cache.prev_embedding if n_tok == 1 else None
            kv_cache.prev_embedding = x[:, -1:]
        x = x0 = self._smear(x, before)
        mid = self.config.n_layer // 2
        mid_out = None
        fused = kv_cache is None and _norm_fusable(x) and x0.shape == x.shape
        for i, block in enumerate(self.transformer.h):
            if fused:
                x = block.forward_mixed(x, x0, self.resid_lambdas, self.x0_lambdas, i)
            else:
                x = block(resid_mix(x, x0, self.resid_lambdas, self.x0_lambdas, i).to(torch.bfloat16), kv_cache)
            mid_out = x if i == mid else mid_out
        if kv_cache is not None:
            kv_cache.advance(n_tok)
        if mid_out is not None and fused:  # remove the mid-depth features before the head
            _, h = _ResidMixNorm.apply(x, mid_out, self._one, -self.backout_lambda, 0, _RMS_EPS)
        else:
            if mid_out is not None:
                x = resid_mix(x, mid_out, self._one, -self.backout_lambda, 0)
            h = norm(x)
        logits = self.lm_head(h)
        if targets is not None:
            return softcap_cross_entropy(logits.flatten(0, 1), targets.flatten(), self.config.vocab_size,
                                         15.0, -1, expected_grad=self.loss_grad_hint)
        return 15 * torch.tanh(logits[..., : self.config.vocab_size].float() / 15)


GEMM_SELECTION_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_selection_gfx950.csv")


def use_tuned_gemms(path: str = GEMM_SELECTION_FILE) -> bool:
    """Routes the trainer's library GEMMs (the projections and the lm_head, through
    torch.mm / F.linear) to the hipBLASLt / rocBLAS solutions recorded in `path` for their
    exact shapes, using torch's TunableOp in lookup-only mode: nothing is tuned at run time,
    and shapes not in the file keep the library's default choice.  The file's validator
    lines pin the torch, HIP, hipBLASLt and rocBLAS versions and the GPU; if they do not
    match the running stack, TunableOp is switched off again and False is returned (the
    default solutions are then used).  The file is written by
    experiment_swa_kda_amd/tune_gemms.py.  Process-wide: it affects every GEMM in the process."""
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(False)
    ok = os.path.exists(path) and bool(tun.read_file(path))
    # TunableOp writes its result table to its file name when the process exits; keep
    # that away from the package's file and the working directory
    tun.set_filename(os.devnull)
    if not ok:
        tun.enable(False)
    return ok


def make_optimizer(model: GPT, lr: float = 3e-3, capturable: bool = False):
    """AdamW over all parameters (the reference uses MuonAdamW, nanochat/optim.py; the
    optimizer is outside the KDA path and only has to run every update).  ``capturable``
    keeps the step count on the device so that the update can be replayed from a graph."""
    return torch.optim.AdamW(model.parameters(), lr=lr, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.0,
                             fused=True, capturable=capturable)


class GraphedUpdate:
    """One training update (``len(batches)`` gradient-accumulation microsteps of forward +
    backward, then the optimizer step) captured once as a HIP graph and replayed.

    The reference compiles the model with torch.compile (scripts/base_train.py:267) to cut
    per-op overhead; here the same kernels are recorded once and replayed, so one update is
    one graph launch instead of a few thousand host-side dispatches.  Every kernel of the
    update runs on each replay.  ``batches`` are static [B, T + 1] token buffers: copy the
    next data into them before calling.  The optimizer must be capturable
    (make_optimizer(..., capturable=True)); every launch in the KDA library is
    stream-ordered and host-synchronisation free, as capture requires.
    """

    def __init__(self, model: GPT, opt, batches, warmup: int = 2):
        """Runs ``warmup`` eager updates on ``batches`` (they create the optimizer state and
        the allocator pools that the capture reuses), then restores the parameters and
        resets the optimizer state, so construction leaves the model as it found it: the
        first replay is the first update."""
        self.model, self.opt, self.batches = model, opt, batches
        saved = [p.detach().clone() for p in model.parameters()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._update()
            with torch.no_grad():
                for p, s in zip(model.parameters(), saved):
                    p.copy_(s)
                for state in opt.state.values():
                    for t in state.values():
                        if torch.is_tensor(t):
                            t.zero_()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        del saved
        self.graph = torch.cuda.CUDAGraph()
        opt.zero_grad(set_to_none=True)
        with torch.cuda.graph(self.graph):
            self.loss = self._update(zero=False)
        torch.cuda.synchronize()

    def _update(self, zero: bool = True):
        """The microsteps' parameter gradients are summed with one multi-tensor add per
        microstep (autograd.grad, then _foreach_add_) instead of one accumulation kernel per
        parameter: the same f32 sums in the same order as ``loss.backward()`` would leave in
        ``.grad``, which is where they end up before the optimizer step.  The projection
        weights are cast to bf16 once per update rather than once per microstep."""
        n = len(self.batches)
        params = [p for p in self.model.parameters() if p.requires_grad]
        acc, total = None, None
        self._w16 = self.model.cache_bf16_weights()  # kept alive with the captured graph
        try:
            for mb in self.batches:
                self.model.loss_grad_hint = 1.0 / n  # the loss below is scaled by 1/n
                loss = self.model(mb[:, :-1], mb[:, 1:]) / n
                grads = torch.autograd.grad(loss, params, allow_unused=True)
                if acc is None:
                    # owned copies where autograd hands out an expanded or strided view
                    acc = [g if g is None or g.is_contiguous() else g.contiguous() for g in grads]
                else:
                    groups = {}  # the multi-tensor kernels take one dtype per call
                    for a, g in zip(acc, grads):
                        if a is not None and g is not None:
                            d, s_ = groups.setdefault((a.dtype, g.dtype), ([], []))
                            d.append(a)
                            s_.append(g if g.is_contiguous() else g.contiguous())
                    for d, s_ in groups.values():
                        torch._foreach_add_(d, s_)
                    acc = [g.contiguous() if a is None and g is not None else a for a, g in zip(acc, grads)]
                total = loss.detach() if total is None else total + loss.detach()
        finally:
            self.model.drop_bf16_weights()
            self.model.loss_grad_hint = 1.0
        for p, g in zip(params, acc):
            p.grad = g
        self.opt.step()
        if zero:
            self.opt.zero_grad(set_to_none=True)
        return total

    def __call__(self):
        """Runs one update; returns the (static) mean loss tensor of the update."""
        self.graph.replay()
        return self.loss
