"""ctypes binding of libkda_mi355x.so (the C ABI declared in include/kda_mi355x.h).

The library is loaded from this package directory only.  There is no fallback: if it
is missing or fails to load, every native entry point raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkda_mi355x.so")

KDA_OK = 0
KDA_GATE_K3 = 0
KDA_GATE_LOGDECAY = 1

# exported symbol -> (restype, argtypes); mirrors include/kda_mi355x.h
_P = ctypes.c_void_p
_I = ctypes.c_int32
_F = ctypes.c_float
_L = ctypes.c_int64


class ChunkProblem(ctypes.Structure):
    """struct kda_chunk_problem."""

    _fields_ = [
        ("batch", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("key_dim", ctypes.c_int32),
        ("value_dim", ctypes.c_int32),
        ("num_seqs", ctypes.c_int32),
        ("cu_seqlens", ctypes.c_void_p),
        ("gate_mode", ctypes.c_int32),
        ("lower_bound", ctypes.c_float),
        ("scale", ctypes.c_float),
        ("grad_row_stride", ctypes.c_int32),
        ("beta_row_stride", ctypes.c_int32),
        ("beta_grad_pad", ctypes.c_int32),
        ("norm_gate_row_stride", ctypes.c_int32),
    ]


_PP = ctypes.POINTER(ChunkProblem)

SIGNATURES = {
    "kda_last_error": (ctypes.c_char_p, []),
    "kda_version": (ctypes.c_char_p, []),
    "kda_chunk_workspace_bytes": (ctypes.c_size_t, [_PP]),
    "kda_chunk_backward_scratch_bytes": (ctypes.c_size_t, [_PP]),
    "kda_chunk_forward": (ctypes.c_int, [_PP] + [_P] * 11 + [_P]),
    "kda_chunk_forward_norm_gate": (ctypes.c_int, [_PP] + [_P] * 13 + [_F, _P, _P, _P]),
    "kda_chunk_forward_conv_norm_gate": (ctypes.c_int, [_PP, _P, _L, _P, _I] + [_P] * 11 + [_F, _P, _P, _P]),
    "kda_chunk_backward": (ctypes.c_int, [_PP] + [_P] * 20 + [_P]),
    "kda_chunk_backward_noalloc": (ctypes.c_int, [_PP] + [_P] * 19 + [_P]),
    "kda_chunk_backward_noalloc_max_scratch_bytes": (ctypes.c_size_t, []),
    "kda_chunk_backward_status": (ctypes.c_int, [_PP, _P, _P]),
    "kda_debug_set_wait_limit": (ctypes.c_int, [_L]),
    "kda_chunk_forward_stage": (ctypes.c_int, [_I, _PP] + [_P] * 11 + [_P]),
    "kda_chunk_backward_stage": (ctypes.c_int, [_I, _PP] + [_P] * 20 + [_P]),
    "kda_recurrent_decode": (ctypes.c_int, [_I, _I, _I, _I, _I, _F, _F] + [_P] * 10 + [_P]),
    "kda_causal_conv_forward": (ctypes.c_int, [_I, _I, _I, _I] + [_P] * 5 + [_P]),
    "kda_causal_conv_backward_scratch_bytes": (ctypes.c_size_t, [_I, _I, _I, _I]),
    "kda_causal_conv_backward": (ctypes.c_int, [_I, _I, _I, _I] + [_P] * 9 + [_P]),
    "kda_causal_conv_backward_strided": (ctypes.c_int, [_I, _I, _I, _I, _P, _L] + [_P] * 5 + [_L] + [_P] * 4),
    "kda_rmsnorm_gate_forward": (ctypes.c_int, [_L, _I, _P, _P, _P, _F, _P, _P, _P]),
    "kda_rmsnorm_gate_backward_scratch_bytes": (ctypes.c_size_t, [_L, _I]),
    "kda_rmsnorm_gate_backward": (ctypes.c_int, [_L, _I, _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P]),
    "kda_rmsnorm_gate_backward_strided": (ctypes.c_int, [_L, _I, _I, _P, _P, _L, _P, _P, _P, _F, _P, _P, _L, _P,
                                                         _P, _P]),
    "kda_softcap_cross_entropy_forward": (ctypes.c_int, [_L, _I, _L, _F, _P, _P, _L, _P, _P, _P]),
    "kda_softcap_cross_entropy_backward": (ctypes.c_int, [_L, _I, _L, _F, _P, _P, _L, _P, _P, _P, _P]),
    "kda_softcap_cross_entropy_fused_supported": (ctypes.c_int, [_I, _L]),
    "kda_softcap_cross_entropy_fused": (ctypes.c_int, [_L, _I, _L, _F, _P, _P, _L, _P, _P, _P, _P, _P]),
    "kda_softcap_cross_entropy_count": (ctypes.c_int, [_L, _P, _L, _F, _P, _P, _P]),
    "kda_bf16_rescale_if_changed": (ctypes.c_int, [_L, _P, _P, _F, _P]),
    "kda_weight_grad_scratch_bytes": (ctypes.c_size_t, [_L, _I, _I]),
    "kda_weight_grad": (ctypes.c_int, [_L, _I, _I, _P, _L, _P, _L, _P, _P, _P]),
    "kda_resid_mix_backward_scratch_bytes": (ctypes.c_size_t, [_L]),
    "kda_resid_mix_forward": (ctypes.c_int, [_L, _P, _P, _P, _P, _P, _P]),
    "kda_resid_mix_backward": (ctypes.c_int, [_L] + [_P] * 9 + [_I, _I, _P, _P]),
    "kda_relu2_forward": (ctypes.c_int, [_L, _P, _P, _P]),
    "kda_rms_norm_forward": (ctypes.c_int, [_L, _I, _F, _P, _P, _P, _P]),
    "kda_rms_norm_backward": (ctypes.c_int, [_L, _I, _P, _P, _P, _P, _P]),
    "kda_mix_rms_norm_forward": (ctypes.c_int, [_L, _I, _F, _P, _P, _P, _P, _P, _P, _P, _P]),
    "kda_rms_norm_backward_add": (ctypes.c_int, [_L, _I, _P, _P, _P, _P, _P, _P]),
    "kda_relu2_backward": (ctypes.c_int, [_L, _P, _P, _P, _P]),
    "kda_softcap_cross_entropy_mean": (ctypes.c_int, [_L, _P, _P, _L, _P, _P, _P]),
    "kda_mfma_probe": (ctypes.c_int, [_I, _I, _I, _P, ctypes.POINTER(ctypes.c_double), _P]),
    "kda_embedding_backward": (ctypes.c_int, [_L, _I, _I, _P, _P, _P, _P]),
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load the shared library once; raise RuntimeError when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"MI355X KDA library not built: {LIB_PATH} is missing "
                "(run `python -m experiment_swa_kda_amd.build`)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def is_built() -> bool:
    return os.path.exists(LIB_PATH)


def check(rc: int, what: str) -> None:
    if rc != KDA_OK:
        msg = load().kda_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor or None."""
    return None if t is None else t.data_ptr()
