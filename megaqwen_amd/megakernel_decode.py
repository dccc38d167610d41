"""Python surface of the megakernel, mirroring the reference's
`csrc/megakernel/megakernel_decode.py` (classes `MegakernelDecoder` :90-242,
`MegakernelPrefillDecoder` :375-660, `MegakernelGenerator` :1136-1211,
`MegakernelPrefillGenerator` :1214-1307, `load_qwen3_weights` :1077-1133).

Same constructor arguments, methods and error behaviour; the kernels behind
them are the gfx950 HIP kernels of `libmegaqwen_amd.so`, called through the C
ABI (`include/megaqwen_amd.h`) on torch's current HIP stream. PyTorch is only
used for device memory and streams.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _abi
from . import config as C
from . import rope, weights
from .config import HEAD_DIM, HIDDEN_SIZE, INTERMEDIATE_SIZE, KV_SIZE, NUM_KV_HEADS, NUM_LAYERS, Q_SIZE, VOCAB_SIZE

ATTN_SCALE = 1.0 / math.sqrt(HEAD_DIM)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_layer_list(layer_weights_flat, num_layers):
    if len(layer_weights_flat) != 11 * num_layers:
        raise ValueError(f"expected {11 * num_layers} layer tensors, got {len(layer_weights_flat)}")
    for i, t in enumerate(layer_weights_flat):
        name = C.LAYER_WEIGHT_NAMES[i % 11]
        shape = C.LAYER_WEIGHT_SHAPES[name]
        if tuple(t.shape) != shape or t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"layer {i // 11} {name}: expected contiguous cuda bf16 {shape}, got "
                             f"{t.dtype} {tuple(t.shape)} on {t.device}")


def make_layer_struct_array(layer_weights_flat, num_layers) -> torch.Tensor:
    """Pack the 11-per-layer pointers into a DEVICE array of LDGLayerWeights
    (reference: megakernel_decode.py:113-132 cudaMemcpy of the struct vector)."""
    arr = (_abi.LDGLayerWeights * num_layers)()
    for i in range(num_layers):
        for f, name in enumerate(_abi.LAYER_FIELDS):
            setattr(arr[i], name, layer_weights_flat[i * 11 + f].data_ptr())
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.to("cuda")


class MegakernelDecoder:
    """One-token-at-a-time greedy decoder (reference `MegakernelDecoder`, megakernel_decode.py:90-242).

    `decode_step(token)` writes the KV slot at `position()`, returns the greedy
    next token and advances the position; `reset()` zeroes the KV cache and the
    position.
    """

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table, sin_table,
                 num_layers: int, max_seq_len: int):
        _check_layer_list(layer_weights_flat, num_layers)
        for name, t, shape in (("embed_weight", embed_weight, (VOCAB_SIZE, HIDDEN_SIZE)),
                               ("lm_head_weight", lm_head_weight, (VOCAB_SIZE, HIDDEN_SIZE)),
                               ("final_norm_weight", final_norm_weight, (HIDDEN_SIZE,))):
            if tuple(t.shape) != shape or t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name}: expected contiguous cuda bf16 {shape}")
        for name, t in (("cos_table", cos_table), ("sin_table", sin_table)):
            if t.dim() != 2 or t.shape[1] != HEAD_DIM or t.shape[0] < max_seq_len or t.dtype != torch.bfloat16:
                raise ValueError(f"{name}: expected bf16 [>= max_seq_len, {HEAD_DIM}]")
        self.num_layers_ = num_layers
        self.max_seq_len_ = max_seq_len
        self.embed_weight_ = embed_weight
        self.final_norm_weight_ = final_norm_weight
        self.lm_head_weight_ = lm_head_weight
        self.cos_table_ = cos_table.contiguous()
        self.sin_table_ = sin_table.contiguous()
        self.layer_weights_tensors_ = list(layer_weights_flat)
        self.d_layer_weights_ = make_layer_struct_array(self.layer_weights_tensors_, num_layers)
        dev = embed_weight.device
        bf, f32 = dict(dtype=torch.bfloat16, device=dev), dict(dtype=torch.float32, device=dev)
        self.k_cache_ = torch.zeros(num_layers, NUM_KV_HEADS, max_seq_len, HEAD_DIM, **bf)
        self.v_cache_ = torch.zeros(num_layers, NUM_KV_HEADS, max_seq_len, HEAD_DIM, **bf)
        # Reference scratch buffers (megakernel_decode.py:148-159); kept for ABI parity.
        self.hidden_buffer_ = torch.empty(HIDDEN_SIZE, **bf)
        self.g_activations_ = torch.empty(HIDDEN_SIZE, **f32)
        self.g_residual_ = torch.empty(HIDDEN_SIZE, **f32)
        self.g_q_ = torch.empty(Q_SIZE, **f32)
        self.g_k_ = torch.empty(KV_SIZE, **f32)
        self.g_v_ = torch.empty(KV_SIZE, **f32)
        self.g_attn_out_ = torch.empty(Q_SIZE, **f32)
        self.g_mlp_intermediate_ = torch.empty(INTERMEDIATE_SIZE, **f32)
        self.g_normalized_ = torch.empty(HIDDEN_SIZE, **f32)
        self.block_max_vals_ = torch.empty(1184, **f32)
        self.block_max_idxs_ = torch.empty(1184, dtype=torch.int32, device=dev)
        self.output_token_ = torch.empty(1, dtype=torch.int32, device=dev)
        self.position_ = 0
        self.attn_scale_ = ATTN_SCALE
        _abi.lib()

    # -- launch helpers --------------------------------------------------------
    def _launch(self, token: int, logits: torch.Tensor | None = None) -> None:
        if not 0 <= token < VOCAB_SIZE:
            raise ValueError(f"token id {token} out of range")
        if self.position_ >= self.max_seq_len_:
            raise RuntimeError("KV cache full: position >= max_seq_len")
        args = [token, _ptr(self.output_token_)]
        if logits is not None:
            args.append(_ptr(logits))
        args += [
            _ptr(self.embed_weight_), _ptr(self.d_layer_weights_), _ptr(self.final_norm_weight_),
            _ptr(self.lm_head_weight_), _ptr(self.cos_table_), _ptr(self.sin_table_), _ptr(self.k_cache_),
            _ptr(self.v_cache_), _ptr(self.hidden_buffer_), _ptr(self.g_activations_), _ptr(self.g_residual_),
            _ptr(self.g_q_), _ptr(self.g_k_), _ptr(self.g_v_), _ptr(self.g_attn_out_),
            _ptr(self.g_mlp_intermediate_), _ptr(self.g_normalized_), _ptr(self.block_max_vals_),
            _ptr(self.block_max_idxs_), self.num_layers_, self.position_, self.position_ + 1, self.max_seq_len_,
            self.attn_scale_, _stream(),
        ]
        fn = _abi.lib().launch_ldg_decode_with_logits if logits is not None else _abi.lib().launch_ldg_decode
        _abi.check(fn(*args), "launch_ldg_decode")

    def _read_token(self) -> int:
        tok = int(self.output_token_.item())
        if tok < 0:
            _abi.lib().mq_reset_workspace(self.embed_weight_.device.index or 0)
            raise _abi.MegakernelError(f"kernel reported error flags {-tok - 1} (decode watchdog, or a prompt id "
                                       f"out of range in prefill); workspace reset")
        return tok

    # -- reference API ---------------------------------------------------------
    def decode_step(self, input_token_id: int) -> int:
        self._launch(int(input_token_id))
        self.position_ += 1
        return self._read_token()

    def decode_step_async(self, input_token_id: int) -> torch.Tensor:
        """Launch one step without the device->host read; returns the device token tensor."""
        self._launch(int(input_token_id))
        self.position_ += 1
        return self.output_token_

    def decode_step_with_logits(self, input_token_id: int):
        """Greedy step that also returns the bf16-rounded logits as fp32 [151936]."""
        logits = torch.empty(VOCAB_SIZE, dtype=torch.float32, device=self.embed_weight_.device)
        self._launch(int(input_token_id), logits)
        self.position_ += 1
        return self._read_token(), logits

    def reset(self) -> None:
        self.position_ = 0
        self.k_cache_.zero_()
        self.v_cache_.zero_()

    def position(self) -> int:
        return self.position_

    def set_position(self, pos: int) -> None:
        if not 0 <= pos <= self.max_seq_len_:
            raise ValueError("position out of range")
        self.position_ = pos

    def get_k_cache(self) -> torch.Tensor:
        return self.k_cache_

    def get_v_cache(self) -> torch.Tensor:
        return self.v_cache_

    def hidden_state(self) -> torch.Tensor:
        """Final hidden state (bf16 [1024]) of the last step."""
        return self.hidden_buffer_

    def normalized_state(self) -> torch.Tensor:
        """Final-norm output (fp32 [1024]) of the last step."""
        return self.g_normalized_


def make_layer_struct_host(layer_weights_flat, num_layers):
    """HOST array of PrefillLayerWeights, as the reference passes to the prefill
    launcher (megakernel_decode.py:516); the caller keeps it alive."""
    arr = (_abi.LDGLayerWeights * num_layers)()
    for i in range(num_layers):
        for f, name in enumerate(_abi.LAYER_FIELDS):
            setattr(arr[i], name, layer_weights_flat[i * 11 + f].data_ptr())
    return arr


class MegakernelPrefillDecoder(MegakernelDecoder):
    """Prompt prefill + greedy decode (reference `MegakernelPrefillDecoder`,
    megakernel_decode.py:375-660).

    `prefill_step(ids)` runs the whole prompt through the MFMA prefill kernels,
    writes KV slots 0..S-1, sets the position to S and returns the greedy next
    token; `decode_step` then continues one token at a time. Raises for an empty
    prompt or one longer than `max_prefill_len` (the reference's checks, :499-504).
    """

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table, sin_table,
                 num_layers: int, max_seq_len: int, max_prefill_len: int = 512):
        super().__init__(embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table, sin_table,
                         num_layers, max_seq_len)
        if not 1 <= max_prefill_len <= max_seq_len:
            raise ValueError("max_prefill_len must be in [1, max_seq_len]")
        self.max_prefill_len_ = max_prefill_len
        self.h_layer_weights_ = make_layer_struct_host(self.layer_weights_tensors_, num_layers)
        dev = embed_weight.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        P = max_prefill_len
        # Prefill scratch in the reference's shapes (megakernel_decode.py:453-466); the ones
        # this build fuses away are not allocated and are passed as NULL.
        self.hidden_float_ = torch.empty(P, HIDDEN_SIZE, **bf)
        self.normalized_ = torch.empty(P, HIDDEN_SIZE, **bf)
        self.q_proj_ = torch.empty(P, Q_SIZE, **bf)
        self.k_proj_ = torch.empty(P, KV_SIZE, **bf)
        self.v_proj_ = torch.empty(P, KV_SIZE, **bf)
        self.attn_out_ = torch.empty(P, Q_SIZE, **bf)
        self.mlp_norm_ = torch.empty(P, HIDDEN_SIZE, **bf)
        # gate_out / up_out hold the kernel's fp32 k-split partial sums (4 KB a row)
        self.gate_out_ = torch.empty(P, INTERMEDIATE_SIZE, **bf)
        self.up_out_ = torch.empty(P, INTERMEDIATE_SIZE, **bf)
        self.mlp_intermediate_ = torch.empty(P, INTERMEDIATE_SIZE, **bf)
        self.final_hidden_ = torch.empty(HIDDEN_SIZE, **bf)
        self.input_tokens_ = torch.empty(P, dtype=torch.int32, device=dev)

    def prefill_step_async(self, input_token_ids) -> torch.Tensor:
        """Launch the prefill without the device->host read; returns the device token tensor."""
        ids = torch.as_tensor(input_token_ids, dtype=torch.int32).reshape(-1)
        n = int(ids.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if n > self.max_prefill_len_:
            raise RuntimeError("Prefill sequence length exceeds maximum")
        self.input_tokens_[:n].copy_(ids.to(self.input_tokens_.device), non_blocking=False)
        st = _abi.lib().launch_prefill_float(
            _ptr(self.input_tokens_), _ptr(self.output_token_), n, _ptr(self.embed_weight_),
            ctypes.addressof(self.h_layer_weights_), _ptr(self.final_norm_weight_), _ptr(self.lm_head_weight_),
            _ptr(self.cos_table_), _ptr(self.sin_table_), _ptr(self.k_cache_), _ptr(self.v_cache_),
            _ptr(self.hidden_float_), None, _ptr(self.normalized_), _ptr(self.q_proj_), _ptr(self.k_proj_),
            _ptr(self.v_proj_), _ptr(self.attn_out_), None, _ptr(self.mlp_norm_), _ptr(self.gate_out_), _ptr(self.up_out_),
            _ptr(self.mlp_intermediate_), None, _ptr(self.final_hidden_), _ptr(self.block_max_vals_),
            _ptr(self.block_max_idxs_), _ptr(self.hidden_buffer_), self.num_layers_, self.max_seq_len_,
            self.attn_scale_, _stream())
        _abi.check(st, "launch_prefill_float")
        self.position_ = n
        return self.output_token_

    def prefill_step(self, input_token_ids) -> int:
        self.prefill_step_async(input_token_ids)
        return self._read_token()


def decode_layer(hidden_in: torch.Tensor, layer_weights: list, cos_table, sin_table, k_cache, v_cache,
                 position: int, attn_scale: float = ATTN_SCALE) -> torch.Tensor:
    """Run one decoder block on a bf16 hidden vector at `position` (C ABI `mq_decode_layer`).

    k_cache / v_cache: bf16 [8, max_seq, 128] (or [1, 8, max_seq, 128]); slot
    `position` is written. Returns the block output (bf16 [1024]).
    """
    _check_layer_list(layer_weights, 1)
    max_seq = k_cache.shape[-2]
    out = torch.empty_like(hidden_in)
    d_lw = make_layer_struct_array(layer_weights, 1)
    st = _abi.lib().mq_decode_layer(_ptr(hidden_in), _ptr(out), _ptr(d_lw), _ptr(cos_table), _ptr(sin_table),
                                    _ptr(k_cache), _ptr(v_cache), position, max_seq, attn_scale, _stream())
    _abi.check(st, "mq_decode_layer")
    torch.cuda.current_stream().synchronize()
    return out


def load_qwen3_weights(model_name: str | None = None, seed: int = 0, max_seq_len: int = 2048, device="cuda",
                       num_layers: int = NUM_LAYERS):
    """Seeded synthetic Qwen3-0.6B weights in the reference's return format
    (megakernel_decode.py:1077-1133). The reference downloads `model_name` from
    the HF hub; this build has no network, so `model_name` must be None or a
    local directory (not supported yet) and weights come from `seed`. RoPE
    tables use theta 1e6 (the reference's 1e4 at :1098 is a bug).
    """
    if model_name is not None:
        raise NotImplementedError("loading a checkpoint is not supported offline; pass model_name=None")
    sd = weights.make_state_dict(seed=seed, num_layers=num_layers)
    embed = sd["model.embed_tokens.weight"].to(device)
    flat = [t.to(device) for t in weights.layer_weights_flat(sd, num_layers)]
    cos, sin = rope.rope_tables(max_seq_len)
    return {
        "embed_weight": embed,
        "layer_weights": flat,
        "final_norm_weight": sd["model.norm.weight"].to(device),
        "lm_head_weight": embed,  # tied
        "cos_table": cos.to(device),
        "sin_table": sin.to(device),
        "tokenizer": None,
        "state_dict": sd,
    }


class MegakernelGenerator:
    """High-level greedy generator (reference megakernel_decode.py:1136-1211).

    Prompts are token-id lists (no tokenizer is available offline).
    """

    def __init__(self, model_name=None, max_seq_len: int = 2048, seed: int = 0, weights_dict=None):
        w = weights_dict or load_qwen3_weights(model_name, seed=seed, max_seq_len=max_seq_len)
        self.weights = w
        self.decoder = MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                         w["lm_head_weight"], w["cos_table"], w["sin_table"],
                                         len(w["layer_weights"]) // 11, max_seq_len)
        self.tokenizer = w.get("tokenizer")
        self.max_seq_len = max_seq_len

    def _ids(self, prompt):
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("string prompts need a tokenizer; pass a list of token ids")
            return self.tokenizer.encode(prompt, add_special_tokens=True)
        return [int(t) for t in prompt]

    def generate_ids(self, prompt, max_new_tokens: int = 100, stop_tokens=None):
        self.decoder.reset()
        ids = self._ids(prompt)
        if not ids:
            raise ValueError("empty prompt")
        for t in ids[:-1]:
            self.decoder.decode_step(t)
        cur = ids[-1]
        out = []
        stop = set(stop_tokens or [])
        for _ in range(max_new_tokens):
            nxt = self.decoder.decode_step(cur)
            if nxt in stop:
                break
            out.append(nxt)
            cur = nxt
            if self.decoder.position() >= self.max_seq_len - 1:
                break
        return out

    def generate(self, prompt, max_new_tokens: int = 100, temperature: float = 1.0, stop_tokens=None):
        ids = self.generate_ids(prompt, max_new_tokens, stop_tokens)
        return self.tokenizer.decode(ids, skip_special_tokens=True) if self.tokenizer else ids

    def generate_stream(self, prompt, max_new_tokens: int = 100, stop_tokens=None):
        self.decoder.reset()
        ids = self._ids(prompt)
        for t in ids[:-1]:
            self.decoder.decode_step(t)
        cur = ids[-1]
        stop = set(stop_tokens or [])
        for _ in range(max_new_tokens):
            nxt = self.decoder.decode_step(cur)
            if nxt in stop:
                break
            yield self.tokenizer.decode([nxt]) if self.tokenizer else nxt
            cur = nxt
            if self.decoder.position() >= self.max_seq_len - 1:
                break


class MegakernelPrefillGenerator:
    """Generator using the prefill kernels for the prompt and the decode kernel after
    it (reference megakernel_decode.py:1214-1307). Prompts are token-id lists."""

    def __init__(self, model_name=None, max_seq_len: int = 2048, max_prefill_len: int = 512, seed: int = 0,
                 weights_dict=None):
        w = weights_dict or load_qwen3_weights(model_name, seed=seed, max_seq_len=max_seq_len)
        self.weights = w
        self.decoder = MegakernelPrefillDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                                w["lm_head_weight"], w["cos_table"], w["sin_table"],
                                                len(w["layer_weights"]) // 11, max_seq_len, max_prefill_len)
        self.tokenizer = w.get("tokenizer")
        self.max_seq_len = max_seq_len
        self.max_prefill_len = max_prefill_len

    def _ids(self, prompt):
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("string prompts need a tokenizer; pass a list of token ids")
            prompt = self.tokenizer.encode(prompt, add_special_tokens=True)
        ids = [int(t) for t in prompt]
        if len(ids) > self.max_prefill_len:
            raise ValueError(f"Prompt length {len(ids)} exceeds max prefill length {self.max_prefill_len}")
        return ids

    def generate_ids(self, prompt, max_new_tokens: int = 100, stop_tokens=None):
        self.decoder.reset()
        nxt = self.decoder.prefill_step(torch.tensor(self._ids(prompt), dtype=torch.int32))
        out, stop = [], set(stop_tokens or [])
        for _ in range(max_new_tokens):
            if nxt in stop:
                break
            out.append(nxt)
            if self.decoder.position() >= self.max_seq_len - 1:
                break
            nxt = self.decoder.decode_step(nxt)
        return out

    def generate(self, prompt, max_new_tokens: int = 100, stop_tokens=None):
        ids = self.generate_ids(prompt, max_new_tokens, stop_tokens)
        return self.tokenizer.decode(ids, skip_special_tokens=True) if self.tokenizer else ids

    def generate_stream(self, prompt, max_new_tokens: int = 100, stop_tokens=None):
        self.decoder.reset()
        nxt = self.decoder.prefill_step(torch.tensor(self._ids(prompt), dtype=torch.int32))
        stop = set(stop_tokens or [])
        for _ in range(max_new_tokens):
            if nxt in stop:
                break
            yield self.tokenizer.decode([nxt]) if self.tokenizer else nxt
            if self.decoder.position() >= self.max_seq_len - 1:
                break
            nxt = self.decoder.decode_step(nxt)

    def prefill_only(self, prompt):
        self.decoder.reset()
        nxt = self.decoder.prefill_step(torch.tensor(self._ids(prompt), dtype=torch.int32))
        return nxt, self.decoder.position()
