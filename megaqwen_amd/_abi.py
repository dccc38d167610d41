"""ctypes binding of the C ABI declared in include/megaqwen_amd.h.

The shared library is built in-tree by `megaqwen_amd/build.py`. There is no
fallback: if the library is missing or fails to load, every entry point
raises.
"""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmegaqwen_amd.so")

MQ_OK = 0
MQ_ERR_ARG = -1
MQ_ERR_HIP = -2
MQ_ERR_DEVICE = -3
MQ_ERR_ALLOC = -4

LAYER_FIELDS = (
    "input_layernorm_weight",
    "q_proj_weight",
    "k_proj_weight",
    "v_proj_weight",
    "q_norm_weight",
    "k_norm_weight",
    "o_proj_weight",
    "post_attn_layernorm_weight",
    "gate_proj_weight",
    "up_proj_weight",
    "down_proj_weight",
)


class LDGLayerWeights(ctypes.Structure):
    """Mirror of the C struct (reference: csrc/megakernel/fused_decode_ldg.cu:24-36)."""

    _fields_ = [(name, ctypes.c_void_p) for name in LAYER_FIELDS]


_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

# name -> argtypes; every entry returns int (MQ_OK or MQ_ERR_*) except mq_strerror.
_DECODE_ARGS = [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                _vp, _i, _i, _i, _i, _f, _vp]
SIGNATURES = {
    "launch_ldg_decode": _DECODE_ARGS,
    "launch_ldg_decode_with_logits": _DECODE_ARGS[:2] + [_vp] + _DECODE_ARGS[2:],
    "mq_decode_layer": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _f, _vp],
    # ids, out, seq_len, embed, layers (host array), final norm, lm head, cos, sin, k, v, 17 scratch,
    # num_layers, max_seq_len, scale, stream
    "launch_prefill_float": [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_vp] * 17 + [_i, _i, _f, _vp],
    "mq_reset_workspace": [_i],
    "mq_strerror": [_i],
}

_lib = None


class MegakernelError(RuntimeError):
    pass


def lib():
    """Load the in-tree library once; raises if it is missing (no CPU fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise MegakernelError(
            f"{LIB_PATH} not found: build it with `python -m megaqwen_amd.build` (hipcc, gfx950)")
    h = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(h, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "mq_strerror" else ctypes.c_int
    _lib = h
    return h


def check(status: int, what: str) -> None:
    if status != MQ_OK:
        msg = lib().mq_strerror(status).decode()
        raise MegakernelError(f"{what} failed: {msg} ({status})")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
