"""Drop-in for the reference chat module's kernel binding (`chat.py:17-29, 48-56, 59-344`).

The reference JIT-compiles `fused_decode_ldg.cu` with a pybind module exposing
`init_ldg_layer_weights`, `init_ldg_embed_weight`, `decode_ldg` and
`decode_ldg_with_logits` (`chat.py:147-323`), chosen by a decode-kernel variant
policy (`select_optimal_kernel_variant`, `chat.py:22-29`). Here the same functions,
with the same argument lists, call the gfx950 library (`launch_ldg_decode` /
`launch_ldg_decode_with_logits` of `include/megaqwen_amd.h`) through ctypes on
torch's current stream. The reference's scratch tensors (g_activations ..
block_max_idxs) are accepted and ignored, except `hidden_buffer` and
`g_normalized`, which receive the final hidden state and the final-norm output
as in the reference.

Variants. The reference's variants are NVIDIA source rewrites (fast-math,
128-block grids), one compiled module each (`chat.py:36-46, 59-64`). The MI355X knob
is the decode kernel instance (`mq_decode_plan`), and a kernel object's variant
fixes it for every `decode_ldg` launch (C ABI `mq_decode_variant`): "unsplit"
attends with one workgroup per XCD and serves contexts of at most
SHORT_CONTEXT_POSITIONS positions (a step past that raises ValueError); "split"
splits the attention over up to 16 workgroups per XCD and serves every length
(past 4096 positions the instance that pipelines a chunk's LDS passes);
"baseline" picks per step (the launcher's own choice, the faster valid instance).
All three give the same tokens, logits and caches.
"""

from __future__ import annotations

import math

import torch

from . import _abi
from . import config as C
from .rope import precompute_rope_freqs  # noqa: F401  (chat.py:48-56)

NUM_LAYERS = C.NUM_LAYERS
HIDDEN_SIZE = C.HIDDEN_SIZE
NUM_KV_HEADS = C.NUM_KV_HEADS
HEAD_DIM = C.HEAD_DIM
INTERMEDIATE_SIZE = C.INTERMEDIATE_SIZE
MAX_SEQ_LEN = 512  # chat.py:15

SUPPORTED_DECODE_KERNEL_VARIANTS = ("baseline", "unsplit", "split")
# variant -> mq_decode_variant's variant code
_VARIANT_CODE = {"baseline": _abi.MQ_VARIANT_BASELINE, "unsplit": _abi.MQ_VARIANT_UNSPLIT,
                 "split": _abi.MQ_VARIANT_SPLIT}
AUTO_KERNEL_VARIANT = "auto"
# Longest context the "unsplit" instance serves (the kernel's one-pass LDS capacity).
SHORT_CONTEXT_POSITIONS = 256


def select_optimal_kernel_variant(max_new_tokens: int, prompt_len: int = 0) -> str:
    """Best decode-kernel instance for a whole generation (reference policy: chat.py:22-29,
    which picks by generation length). A generation whose last position stays within the
    unsplit instance's capacity runs unsplit (one attention workgroup per XCD, no chunk
    merge); a longer one needs the split instance."""
    if max_new_tokens <= 0:
        raise ValueError("max_new_tokens must be positive")
    if prompt_len < 0:
        raise ValueError("prompt_len must be non-negative")
    last_position = prompt_len + max_new_tokens - 1
    return "unsplit" if last_position < SHORT_CONTEXT_POSITIONS else "split"


def _ptr(t):
    return None if t is None else t.data_ptr()


class LDGKernel:
    """The reference's per-variant compiled module (chat.py:59-344): holds the device array of
    layer-weight structs and the embedding set by the init functions (the reference keeps
    them in static globals, chat.py:147-149)."""

    def __init__(self, variant: str = "baseline"):
        if variant not in SUPPORTED_DECODE_KERNEL_VARIANTS:
            supported = ", ".join(SUPPORTED_DECODE_KERNEL_VARIANTS)
            raise ValueError(f"unsupported kernel variant '{variant}', expected one of: {supported}")
        self.variant = variant
        self._layer_tensors = None
        self._d_layer_weights = None
        self._num_layers = 0
        self._embed = None
        _abi.lib()

    # chat.py:151-186
    def init_ldg_layer_weights(self, input_layernorm_weights, q_proj_weights, k_proj_weights, v_proj_weights,
                               q_norm_weights, k_norm_weights, o_proj_weights, post_attn_layernorm_weights,
                               gate_proj_weights, up_proj_weights, down_proj_weights) -> None:
        from .megakernel_decode import _check_layer_list, make_layer_struct_array

        lists = (input_layernorm_weights, q_proj_weights, k_proj_weights, v_proj_weights, q_norm_weights,
                 k_norm_weights, o_proj_weights, post_attn_layernorm_weights, gate_proj_weights, up_proj_weights,
                 down_proj_weights)
        n = len(input_layernorm_weights)
        if any(len(x) != n for x in lists):
            raise ValueError("every weight list needs one tensor per layer")
        flat = [t for i in range(n) for t in (x[i] for x in lists)]
        _check_layer_list(flat, n)
        self._layer_tensors = flat  # keeps the tensors alive (chat.py:376-400)
        self._d_layer_weights = make_layer_struct_array(flat, n)
        self._num_layers = n

    # chat.py:188-190
    def init_ldg_embed_weight(self, embed_weight) -> None:
        self._embed = embed_weight

    def _launch(self, logits, input_token_id, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache,
                v_cache, hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate,
                g_normalized, block_max_vals, block_max_idxs, num_layers, position, cache_len, max_seq_len) -> int:
        if self._d_layer_weights is None or self._embed is None:
            raise RuntimeError("call init_ldg_layer_weights and init_ldg_embed_weight first")
        if num_layers > self._num_layers:
            raise ValueError(f"num_layers {num_layers} exceeds the {self._num_layers} initialised layers")
        if self.variant == "unsplit" and position >= SHORT_CONTEXT_POSITIONS:
            raise ValueError(f"the 'unsplit' kernel variant serves positions below {SHORT_CONTEXT_POSITIONS}, "
                             f"got {position}; use 'split' or 'baseline'")
        # the reference's other scratch tensors (g_activations .. block_max_idxs) are accepted and unused
        del g_activations, g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate, block_max_vals, block_max_idxs
        out = torch.empty(1, dtype=torch.int32, device=k_cache.device)
        args = [_VARIANT_CODE[self.variant], int(input_token_id), _ptr(out), _ptr(logits), _ptr(self._embed),
                _ptr(self._d_layer_weights), _ptr(final_norm_weight), _ptr(lm_head_weight), _ptr(cos_table),
                _ptr(sin_table), _ptr(k_cache), _ptr(v_cache), _ptr(hidden_buffer), _ptr(g_normalized),
                int(num_layers), int(position), int(cache_len), int(max_seq_len), 1.0 / math.sqrt(HEAD_DIM),
                torch.cuda.current_stream().cuda_stream]
        lib = _abi.lib()
        _abi.check(lib.mq_decode_variant(*args), f"decode_ldg ({self.variant} variant)")
        tok = int(out.item())  # the reference synchronises the stream and reads the token (chat.py:250-251)
        if tok < 0:
            lib.mq_reset_workspace(k_cache.device.index or 0)
            raise _abi.MegakernelError(f"decode kernel reported error flags {-tok - 1}; workspace reset")
        return tok

    # chat.py:192-252
    def decode_ldg(self, input_token_id, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
                   hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate,
                   g_normalized, block_max_vals, block_max_idxs, num_layers, position, cache_len,
                   max_seq_len) -> int:
        return self._launch(None, input_token_id, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache,
                            v_cache, hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out,
                            g_mlp_intermediate, g_normalized, block_max_vals, block_max_idxs, num_layers, position,
                            cache_len, max_seq_len)

    # chat.py:254-316
    def decode_ldg_with_logits(self, input_token_id, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache,
                               v_cache, hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out,
                               g_mlp_intermediate, g_normalized, block_max_vals, block_max_idxs, num_layers,
                               position, cache_len, max_seq_len):
        logits = torch.empty(C.VOCAB_SIZE, dtype=torch.float32, device=k_cache.device)
        tok = self._launch(logits, input_token_id, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache,
                           v_cache, hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out,
                           g_mlp_intermediate, g_normalized, block_max_vals, block_max_idxs, num_layers, position,
                           cache_len, max_seq_len)
        return tok, logits


def compile_kernel(variant: str = "baseline") -> LDGKernel:
    """The reference's `compile_kernel` (chat.py:59-344) returns a JIT-built module; the
    gfx950 library is built ahead of time, so this returns a binding object with the
    module's four functions. Unknown variants raise ValueError (chat.py:60-62)."""
    return LDGKernel(variant)


_default = None


def _kernel() -> LDGKernel:
    global _default
    if _default is None:
        _default = LDGKernel()
    return _default


# Module-level functions, for callers that use this module itself as the compiled module.
def init_ldg_layer_weights(*lists):
    return _kernel().init_ldg_layer_weights(*lists)


def init_ldg_embed_weight(embed_weight):
    return _kernel().init_ldg_embed_weight(embed_weight)


def decode_ldg(*args):
    return _kernel().decode_ldg(*args)


def decode_ldg_with_logits(*args):
    return _kernel().decode_ldg_with_logits(*args)
