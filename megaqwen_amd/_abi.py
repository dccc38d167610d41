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
# decode-kernel variants of mq_decode_variant (include/megaqwen_amd.h)
MQ_VARIANT_BASELINE = 0
MQ_VARIANT_UNSPLIT = 1
MQ_VARIANT_SPLIT = 2
# Longest context of the decode kernel (positions 0 .. MAX_CONTEXT - 1; mq_decode_plan
# rejects the rest)
MAX_CONTEXT = 16384

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


class MqDecodeStep(ctypes.Structure):
    """Mirror of the device-resident step descriptor (include/megaqwen_amd.h)."""

    _fields_ = [("token", ctypes.c_int), ("position", ctypes.c_int), ("epoch", ctypes.c_uint),
                ("count", ctypes.c_int)]


_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

# name -> argtypes; every entry returns int (MQ_OK or MQ_ERR_*) except mq_strerror.
_DECODE_ARGS = [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                _vp, _i, _i, _i, _i, _f, _vp]
SIGNATURES = {
    "launch_ldg_decode": _DECODE_ARGS,
    "launch_ldg_decode_with_logits": _DECODE_ARGS[:2] + [_vp] + _DECODE_ARGS[2:],
    "launch_ldg_decode_noalloc": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp],
    # variant, token, out, logits, embed, layers, final norm, lm head, cos, sin, k, v, hidden, normed,
    # num_layers, position, cache_len, max_seq_len, scale, stream
    "mq_decode_variant": [_i, _i, _vp, _vp] + [_vp] * 10 + [_i, _i, _i, _i, _f, _vp],
    "mq_decode_layer": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _f, _vp],
    # ids, out, seq_len, embed, layers (host array), final norm, lm head, cos, sin, k, v, 17 scratch,
    # num_layers, max_seq_len, scale, stream
    "launch_prefill_float": [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_vp] * 17 + [_i, _i, _f, _vp],
    "launch_prefill_megakernel": [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_vp] * 12 + [_i, _i, _f, _vp],
    "mq_decode_step_init": [_vp, _i, _i, _i, _vp],
    # step, out_ids, capacity, split_instance, embed, layers, final norm, lm head, cos, sin, k, v,
    # hidden_buffer, g_normalized, num_layers, max_seq_len, scale, stream
    "mq_decode_step_device": [_vp, _vp, _i, _i] + [_vp] * 10 + [_i, _i, _f, _vp],
    "mq_decode_plan": [_i, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "mq_set_launch_mode": [_i],
    "mq_debug_set_error": [_i, ctypes.c_uint],
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


def decode_plan(position: int) -> dict:
    """The decode kernel's work split for the query at `position` (C ABI `mq_decode_plan`,
    host only): kernel instance (0: contexts <= 256 positions; 1: any; 2: any, a chunk's
    LDS passes pipelined, chosen where a chunk takes more than one pass), number of
    attention chunks, positions per chunk, LDS passes per chunk."""
    inst, ns, ch, npass = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(lib().mq_decode_plan(int(position), ctypes.byref(inst), ctypes.byref(ns), ctypes.byref(ch),
                               ctypes.byref(npass)), "mq_decode_plan")
    return {"instance": inst.value, "nsplit": ns.value, "chunk": ch.value, "npass": npass.value}
