"""CPU oracle for the all-KDA decoder around the operator (numpy, float64).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, and only as the
checker; the product package never imports it.

``gpt_forward`` restates the forward of nanochat/gpt.py:548-608 for a model whose every
layer is a KDA mixer (window_pattern "K", so no rotary tables and no value embeddings,
nanochat/gpt.py:240-245 builds those only for attention layers):

* token embedding, then ``norm`` (F.rms_norm over the last dim, float32 epsilon)
  nanochat/gpt.py:49-50, 562-564;
* smear: position t >= 1 adds ``smear_lambda * sigmoid(x_t[:24] . smear_gate) * x_{t-1}``
  nanochat/gpt.py:567-571;
* trunk: before layer i the residual is ``resid_lambdas[i] * x + x0_lambdas[i] * x0``
  (x0 = the smeared embedding), nanochat/gpt.py:585-590; the block adds
  ``mixer(norm(x))`` then ``mlp(norm(x))`` with mlp = c_proj(relu(c_fc(x))^2),
  nanochat/gpt.py:146-157, 180-205; the mixer is ``kda_oracle.full_layer`` (the K3 block,
  tests/kda_oracle.py:176-236);
* backout: the residual after layer n_layer // 2 is cached and
  ``backout_lambda * x_mid`` is subtracted before the final norm, nanochat/gpt.py:586-597;
* head: logits = lm_head(norm(x)) cut to the vocabulary, soft-capped
  ``15 tanh(logits / 15)``, mean cross entropy with ignore_index -1 when targets are
  given (``kda_oracle.softcap_cross_entropy``), nanochat/gpt.py:599-616.

Pinning (tests/test_gpt_oracle.py): causal prefix property; a backout of 1 at the middle
layer of a 2-layer model with zero blocks cancels the residual exactly (logits 0, loss
ln V); the zero-block trunk's closed-form scale; a smear that only reaches
the next position; and equality with ``torch.nn.functional`` ops (rms_norm, sigmoid,
relu, tanh, cross_entropy) composed over the same parameters.
"""

from __future__ import annotations

import numpy as np

from oracle import kda_oracle as O

F32_EPS = float(np.finfo(np.float32).eps)


def rms_norm(x):
    """F.rms_norm(x, (D,)) with the float32 epsilon (torch's default for bf16/f32 inputs)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + F32_EPS)


def mlp(x, c_fc, c_proj):
    """nanochat/gpt.py:146-157: c_proj(relu(c_fc(x))^2)."""
    h = np.maximum(x @ np.asarray(c_fc, np.float64).T, 0.0)
    return (h * h) @ np.asarray(c_proj, np.float64).T


def smear(x, smear_gate, smear_lambda):
    """nanochat/gpt.py:567-571 (training form: the whole sequence is present)."""
    if x.shape[1] < 2:
        return x
    g = smear_lambda * O.sigmoid(x[:, 1:, :24] @ np.asarray(smear_gate, np.float64).reshape(-1))
    out = x.copy()
    out[:, 1:] = x[:, 1:] + g[..., None] * x[:, :-1]
    return out


def gpt_forward(idx, params, *, vocab, targets=None, softcap=15.0):
    """Logits [B, T, vocab] (soft-capped), or the mean loss when ``targets`` is given.

    ``params``: dict with ``wte`` [Vp, D], ``lm_head`` [Vp, D], ``resid_lambdas`` [L],
    ``x0_lambdas`` [L], ``smear_gate`` [1, 24], ``smear_lambda``, ``backout_lambda`` and
    ``layers``: a list of dicts, each the keyword arguments of ``kda_oracle.full_layer``
    for its mixer plus ``c_fc`` and ``c_proj`` for its MLP."""
    idx = np.asarray(idx, np.int64)
    f = lambda a: np.asarray(a, np.float64)  # noqa: E731
    x = rms_norm(f(params["wte"])[idx])
    x = smear(x, params["smear_gate"], float(params["smear_lambda"]))
    x0 = x
    n_layer = len(params["layers"])
    mid = n_layer // 2
    x_mid = None
    for i, layer in enumerate(params["layers"]):
        x = float(params["resid_lambdas"][i]) * x + float(params["x0_lambdas"][i]) * x0
        mixer_args = {k: v for k, v in layer.items() if k not in ("c_fc", "c_proj")}
        mixed, _ = O.full_layer(rms_norm(x), **mixer_args)
        x = x + mixed
        x = x + mlp(rms_norm(x), layer["c_fc"], layer["c_proj"])
        if i == mid:
            x_mid = x
    if x_mid is not None:
        x = x - float(params["backout_lambda"]) * x_mid
    logits = rms_norm(x) @ f(params["lm_head"]).T
    if targets is None:
        return softcap * np.tanh(logits[..., :vocab] / softcap)
    B, T, Vp = logits.shape
    loss, _, _, _ = O.softcap_cross_entropy(logits.reshape(B * T, Vp), np.asarray(targets).reshape(-1), vocab,
                                            softcap, -1)
    return loss
