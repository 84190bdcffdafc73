"""MI355X-native Kimi Delta Attention operator (hand-written HIP kernels for gfx950).

Public API mirrors the reference mixer module nanochat/mixers/kda.py.
"""

from .kda import (  # noqa: F401
    KDAState,
    KimiDeltaAttention,
    Linear,
    RMSNormGated,
    ShortConvolution,
    k3_decay_gate,
    kda,
    kda_backend_provenance,
    prepare_kda_backend,
    project_runtime_events,
    reset_project_runtime_events,
)

__all__ = ["KDAState", "KimiDeltaAttention", "k3_decay_gate", "kda", "prepare_kda_backend"]
