"""Python surface of the megakernel, mirroring the reference's
`csrc/megakernel/megakernel_decode.py` (classes `MegakernelDecoder` :90-242,
`MegakernelPrefillDecoder` :375-660, `MegakernelFusedPrefillDecoder` :788-943,
`MegakernelGenerator` :1136-1211, `MegakernelPrefillGenerator` :1214-1307,
`MegakernelFusedPrefillGenerator` :1310-1407, `load_qwen3_weights` :1077-1133).

Same constructor arguments, methods and error behaviour; the kernels behind
them are the gfx950 HIP kernels of `libmegaqwen_amd.so`, called through the C
ABI (`include/megaqwen_amd.h`) on torch's current HIP stream. PyTorch is only
used for device memory and streams.
"""

from __future__ import annotations

import ctypes
import json
import math
import os

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

    def _device(self) -> int:
        return self.embed_weight_.device.index or 0

    def _read_token(self, position_before: int) -> int:
        tok = int(self.output_token_.item())
        if tok < 0:
            # The failed step's KV slots hold whatever the abandoned waits left: the position
            # goes back to before the step, so the next step rewrites them.
            self.position_ = position_before
            _abi.lib().mq_reset_workspace(self._device())
            raise _abi.MegakernelError(f"kernel reported error flags {-tok - 1} (decode watchdog, or a prompt id "
                                       f"out of range in prefill); workspace reset, position restored to "
                                       f"{position_before}")
        return tok

    # -- reference API ---------------------------------------------------------
    def decode_step(self, input_token_id: int) -> int:
        p = self.position_
        self._launch(int(input_token_id))
        self.position_ += 1
        return self._read_token(p)

    def decode_step_async(self, input_token_id: int) -> torch.Tensor:
        """Launch one step without the device->host read; returns the device token tensor."""
        self._launch(int(input_token_id))
        self.position_ += 1
        return self.output_token_

    def decode_step_with_logits(self, input_token_id: int):
        """Greedy step that also returns the bf16-rounded logits as fp32 [151936]."""
        p = self.position_
        logits = torch.empty(VOCAB_SIZE, dtype=torch.float32, device=self.embed_weight_.device)
        self._launch(int(input_token_id), logits)
        self.position_ += 1
        return self._read_token(p), logits

    # -- device-resident generation ---------------------------------------------
    def _step_buffers(self, capacity: int):
        if getattr(self, "step_", None) is None or self.out_ids_.numel() < capacity:
            dev = self.embed_weight_.device
            self.step_ = torch.zeros(4, dtype=torch.int32, device=dev)  # MqDecodeStep
            self.out_ids_ = torch.empty(max(capacity, 64), dtype=torch.int32, device=dev)
            self.graphs_ = {}
        return self.step_, self.out_ids_

    def _launch_device_step(self, capacity: int, split_instance: int) -> None:
        st = _abi.lib().mq_decode_step_device(
            _ptr(self.step_), _ptr(self.out_ids_), capacity, split_instance, _ptr(self.embed_weight_),
            _ptr(self.d_layer_weights_), _ptr(self.final_norm_weight_), _ptr(self.lm_head_weight_),
            _ptr(self.cos_table_), _ptr(self.sin_table_), _ptr(self.k_cache_), _ptr(self.v_cache_),
            _ptr(self.hidden_buffer_), _ptr(self.g_normalized_), self.num_layers_, self.max_seq_len_,
            self.attn_scale_, _stream())
        _abi.check(st, "mq_decode_step_device")

    def generate_device(self, input_token_id: int, n_steps: int, use_graph: bool = True, chunk: int = 64,
                        stop_tokens=None) -> list[int]:
        """Greedy-decode `n_steps` tokens from `input_token_id` at `position()` without a
        host read per token (reference idea: experimental/qwen_persistent_kernel.cu:1028-1033).

        Each launch takes its input token, position and epoch from a device-resident step
        that the previous launch advanced. Steps run in chunks of `chunk` launches, as
        one replay of a captured HIP graph per chunk (`use_graph`) or as direct launches;
        the host reads the chunk's tokens once at its end, to stop at a stop token. A
        chunk runs the kernel instance that `_abi.decode_plan` names for its last position
        (short contexts below 256, LDS passes pipelined from 4096). Returns the generated ids (up to and
        excluding a stop token, like `generate`).
        """
        if n_steps < 1:
            raise ValueError("n_steps must be positive")
        if not 0 <= input_token_id < VOCAB_SIZE:
            raise ValueError(f"token id {input_token_id} out of range")
        if self.position_ + n_steps > self.max_seq_len_:
            raise RuntimeError("KV cache full: position + n_steps > max_seq_len")
        stop = set(stop_tokens or [])
        chunk = max(1, min(chunk, n_steps))
        step, out_ids = self._step_buffers(chunk)
        cap = out_ids.numel()
        lib = _abi.lib()
        out: list[int] = []
        token = int(input_token_id)
        while len(out) < n_steps:
            k = min(chunk, n_steps - len(out))
            p0 = self.position_
            # the instance of the chunk's last position serves every earlier one too (past the
            # 16384-position limit the kernel itself reports the error)
            split = _abi.decode_plan(min(p0 + k - 1, _abi.MAX_CONTEXT - 1))["instance"]
            _abi.check(lib.mq_decode_step_init(_ptr(step), token, p0, k, _stream()), "mq_decode_step_init")
            if use_graph:
                key = (k, split)
                g = self.graphs_.get(key)
                if g is None:
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        for _ in range(k):
                            self._launch_device_step(cap, split)
                    self.graphs_[key] = g
                    # capture records the launches without running them: the step is intact
                g.replay()
            else:
                for _ in range(k):
                    self._launch_device_step(cap, split)
            ids = out_ids[:k].tolist()  # one host read per chunk
            done = 0
            for t in ids:
                if t < 0:
                    self.position_ = p0 + done
                    lib.mq_reset_workspace(self._device())
                    raise _abi.MegakernelError(f"device-resident step at position {self.position_} failed "
                                               f"(flags {-t - 1}); workspace reset")
                done += 1
                if t in stop:
                    self.position_ = p0 + done
                    return out
                out.append(t)
            self.position_ = p0 + k
            token = ids[-1]
        return out

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
        # a failed prefill leaves the cache undefined: the position goes back to 0
        return self._read_token(0)

    def final_normed_state(self) -> torch.Tensor:
        """Final-norm output (bf16 [1024]) of the prompt's last row after prefill_step."""
        return self.final_hidden_


class MegakernelFusedPrefillDecoder(MegakernelPrefillDecoder):
    """The reference's fused-prefill decoder (megakernel_decode.py:788-943: a cooperative
    batched-GEMV prefill megakernel for prompts of at most 64 tokens). Same constructor,
    methods and errors, and the same launcher: `launch_prefill_megakernel` with the
    reference's fp32 scratch ([max_prefill_len, n] float32, :859-868). On MI355X that
    launcher runs the MFMA prefill kernels, which serve short prompts as well (default
    max_prefill_len 64, as in the reference); tokens and caches equal launch_prefill_float's.
    After prefill_step, `final_hidden_` holds the last row's final-norm output as fp32 and
    `hidden_buffer_` the last row before the final norm (bf16), as the reference writes them."""

    def __init__(self, embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table, sin_table,
                 num_layers: int, max_seq_len: int, max_prefill_len: int = 64):
        super().__init__(embed_weight, layer_weights_flat, final_norm_weight, lm_head_weight, cos_table, sin_table,
                         num_layers, max_seq_len, max_prefill_len)
        # the reference's fused-prefill scratch: all float32 (megakernel_decode.py:859-868)
        P, dev = self.max_prefill_len_, embed_weight.device
        f32 = dict(dtype=torch.float32, device=dev)
        self.hidden_ = torch.empty(P, HIDDEN_SIZE, **f32)
        self.residual_ = torch.empty(P, HIDDEN_SIZE, **f32)
        self.normalized_ = torch.empty(P, HIDDEN_SIZE, **f32)
        self.q_proj_ = torch.empty(P, Q_SIZE, **f32)
        self.k_proj_ = torch.empty(P, KV_SIZE, **f32)
        self.v_proj_ = torch.empty(P, KV_SIZE, **f32)
        self.attn_out_ = torch.empty(P, Q_SIZE, **f32)
        self.mlp_intermediate_ = torch.empty(P, INTERMEDIATE_SIZE, **f32)
        self.final_hidden_ = torch.empty(HIDDEN_SIZE, **f32)
        # the bf16 buffers of launch_prefill_float are not used by this launcher
        del self.hidden_float_, self.mlp_norm_, self.gate_out_, self.up_out_

    def prefill_step_async(self, input_token_ids) -> torch.Tensor:
        ids = torch.as_tensor(input_token_ids, dtype=torch.int32).reshape(-1)
        n = int(ids.numel())
        if n == 0:
            raise RuntimeError("Empty input sequence")
        if n > self.max_prefill_len_:
            raise RuntimeError("Prefill sequence length exceeds maximum")
        self.input_tokens_[:n].copy_(ids.to(self.input_tokens_.device), non_blocking=False)
        st = _abi.lib().launch_prefill_megakernel(
            _ptr(self.input_tokens_), _ptr(self.output_token_), n, _ptr(self.embed_weight_),
            ctypes.addressof(self.h_layer_weights_), _ptr(self.final_norm_weight_), _ptr(self.lm_head_weight_),
            _ptr(self.cos_table_), _ptr(self.sin_table_), _ptr(self.k_cache_), _ptr(self.v_cache_),
            _ptr(self.hidden_), _ptr(self.residual_), _ptr(self.normalized_), _ptr(self.q_proj_), _ptr(self.k_proj_),
            _ptr(self.v_proj_), _ptr(self.attn_out_), _ptr(self.mlp_intermediate_), _ptr(self.final_hidden_),
            _ptr(self.hidden_buffer_), _ptr(self.block_max_vals_), _ptr(self.block_max_idxs_), self.num_layers_,
            self.max_seq_len_, self.attn_scale_, _stream())
        _abi.check(st, "launch_prefill_megakernel")
        self.position_ = n
        return self.output_token_

    def final_normed_state(self) -> torch.Tensor:
        """Final-norm output of the prompt's last row after prefill_step, as bf16 [1024] (the
        launcher writes it as fp32 holding bf16 values)."""
        return self.final_hidden_.to(torch.bfloat16)


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


def sample_next_token(logits: torch.Tensor, temperature: float, generator: torch.Generator | None = None) -> int:
    """Temperature sampling of one token from fp32 logits [vocab] (the reference's sampling
    step, generate.py:325-329: softmax(logits / T), then one multinomial draw)."""
    if not temperature > 0:
        raise ValueError("temperature must be positive for sampling")
    probs = torch.softmax(logits.float() / temperature, dim=-1)
    return int(torch.multinomial(probs, num_samples=1, generator=generator).item())


# ---------------------------------------------------------------- checkpoints

def _check_qwen3_config(cfg: dict) -> None:
    want = {"hidden_size": HIDDEN_SIZE, "intermediate_size": INTERMEDIATE_SIZE,
            "num_attention_heads": C.NUM_Q_HEADS, "num_key_value_heads": NUM_KV_HEADS, "head_dim": HEAD_DIM,
            "vocab_size": VOCAB_SIZE}
    bad = {k: (cfg.get(k), v) for k, v in want.items() if cfg.get(k, v) != v}
    if bad:
        raise ValueError(f"checkpoint is not Qwen3-0.6B shaped: {bad} (found, expected)")
    if not 1 <= int(cfg.get("num_hidden_layers", NUM_LAYERS)) <= 32:
        raise ValueError("num_hidden_layers must be in [1, 32]")


def rope_theta_of(cfg: dict) -> float:
    """RoPE theta from an HF config dict (v5 `rope_parameters`, or the older `rope_theta`)."""
    rp = cfg.get("rope_parameters") or {}
    return float(rp.get("rope_theta", cfg.get("rope_theta", C.ROPE_THETA)))


def find_local_checkpoint(model_name: str) -> str | None:
    """A local directory holding `model_name`: the path itself if it is a directory, else
    the snapshot of that repo id in the offline HF hub cache
    ($HF_HUB_CACHE, $HF_HOME/hub or ~/.cache/huggingface/hub). No download is attempted."""
    if os.path.isdir(model_name):
        return model_name
    roots = [os.environ.get("HF_HUB_CACHE"),
             os.path.join(os.environ["HF_HOME"], "hub") if os.environ.get("HF_HOME") else None,
             os.path.expanduser("~/.cache/huggingface/hub")]
    for root in roots:
        snaps = os.path.join(root, "models--" + model_name.replace("/", "--"), "snapshots") if root else None
        if snaps and os.path.isdir(snaps):
            for rev in sorted(os.listdir(snaps)):
                d = os.path.join(snaps, rev)
                if os.path.exists(os.path.join(d, "config.json")):
                    return d
    return None


def load_state_dict_dir(path: str):
    """HF-format safetensors checkpoint directory -> (state_dict of CPU bf16 tensors, config dict).
    Reads `model.safetensors`, or the shards listed in `model.safetensors.index.json`."""
    from safetensors.torch import load_file

    cfg = json.load(open(os.path.join(path, "config.json")))
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        files = sorted(set(json.load(open(index))["weight_map"].values()))
    else:
        files = ["model.safetensors"]
    sd = {}
    for f in files:
        for k, v in load_file(os.path.join(path, f)).items():
            sd[k] = v.to(torch.bfloat16).contiguous()
    return sd, cfg


def save_qwen3_checkpoint(state_dict: dict, path: str, num_layers: int = NUM_LAYERS) -> None:
    """Write a state dict as an HF-format checkpoint directory (model.safetensors +
    config.json, tied embeddings, no lm_head tensor): the format load_qwen3_weights reads."""
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    save_file({k: v.contiguous() for k, v in state_dict.items() if k != "lm_head.weight"},
              os.path.join(path, "model.safetensors"), metadata={"format": "pt"})
    cfg = {"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "hidden_size": HIDDEN_SIZE,
           "intermediate_size": INTERMEDIATE_SIZE, "num_hidden_layers": num_layers,
           "num_attention_heads": C.NUM_Q_HEADS, "num_key_value_heads": NUM_KV_HEADS, "head_dim": HEAD_DIM,
           "vocab_size": VOCAB_SIZE, "rms_norm_eps": C.RMS_EPS, "rope_theta": C.ROPE_THETA,
           "tie_word_embeddings": True, "max_position_embeddings": C.MAX_POSITION_EMBEDDINGS,
           "hidden_act": "silu", "attention_bias": False, "torch_dtype": "bfloat16"}
    json.dump(cfg, open(os.path.join(path, "config.json"), "w"), indent=1)


def _local_tokenizer(path: str):
    if not any(os.path.exists(os.path.join(path, f)) for f in ("tokenizer.json", "tokenizer_config.json")):
        return None
    from transformers import AutoTokenizer

    return AutoTokenizer.from_pretrained(path, local_files_only=True)


def load_qwen3_weights(model_name: str | None = None, seed: int = 0, max_seq_len: int = 2048, device="cuda",
                       num_layers: int = NUM_LAYERS, norms: str = "ones"):
    """Qwen3-0.6B weights in the reference's return format (megakernel_decode.py:1077-1133:
    embed, flat 28 x 11 layer list, final norm, tied LM head, RoPE tables, tokenizer).

    model_name=None: the seeded synthetic weights of `megaqwen_amd.weights` (`seed`,
    `norms`). Otherwise a local HF-format checkpoint: a directory, or a repo id found in
    the offline HF hub cache (the reference downloads it; there is no network here).
    safetensors are read with HF key names; `lm_head.weight` is used when present and
    untied, else the LM head is the embedding. The RoPE tables use the checkpoint's theta
    (Qwen3: 1e6; the reference's own table builder hard-codes 1e4 at :1098, a bug).
    """
    cfg = None
    tokenizer = None
    if model_name is None:
        sd = weights.make_state_dict(seed=seed, num_layers=num_layers, norms=norms)
        theta = C.ROPE_THETA
    else:
        path = find_local_checkpoint(model_name)
        if path is None:
            raise FileNotFoundError(f"no local checkpoint for {model_name!r}: pass a directory with config.json and "
                                    f"*.safetensors, or place the repo in the offline HF hub cache")
        sd, cfg = load_state_dict_dir(path)
        _check_qwen3_config(cfg)
        num_layers = int(cfg.get("num_hidden_layers", NUM_LAYERS))
        theta = rope_theta_of(cfg)
        tokenizer = _local_tokenizer(path)
    embed = sd["model.embed_tokens.weight"].to(device)
    tied = cfg is None or cfg.get("tie_word_embeddings", True) or "lm_head.weight" not in sd
    lm_head = embed if tied else sd["lm_head.weight"].to(device)
    flat = [t.to(device) for t in weights.layer_weights_flat(sd, num_layers)]
    cos, sin = rope.rope_tables(max_seq_len, theta=theta)
    return {
        "embed_weight": embed,
        "layer_weights": flat,
        "final_norm_weight": sd["model.norm.weight"].to(device),
        "lm_head_weight": lm_head,
        "cos_table": cos.to(device),
        "sin_table": sin.to(device),
        "tokenizer": tokenizer,
        "state_dict": sd,
        "config": cfg,
    }


# ---------------------------------------------------------------- generators

class _GeneratorBase:
    """Prompt handling, stop tokens and the decode loop shared by the generators. Prompts
    are strings (with a tokenizer from a local checkpoint) or lists of token ids."""

    decoder: MegakernelDecoder
    tokenizer = None
    max_seq_len: int

    def _encode(self, prompt) -> list[int]:
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("string prompts need a tokenizer; pass a list of token ids")
            return self.tokenizer.encode(prompt, add_special_tokens=True)
        return [int(t) for t in prompt]

    def _stop(self, stop_tokens):
        if stop_tokens is not None:
            return set(stop_tokens)
        eos = getattr(self.tokenizer, "eos_token_id", None)
        return {eos} if eos is not None else set()

    def _detok(self, ids):
        return self.tokenizer.decode(ids, skip_special_tokens=True) if self.tokenizer else ids

    def _continue(self, first: int, max_new_tokens: int, stop: set, do_sample: bool, temperature: float,
                  generator, first_is_output: bool):
        """Yield generated ids. first_is_output: `first` is already a generated token (after
        a prefill) rather than the last prompt token."""
        dec = self.decoder
        cur = first
        if first_is_output:
            if cur in stop or max_new_tokens < 1:
                return
            yield cur
            max_new_tokens -= 1
        for _ in range(max_new_tokens):
            if dec.position() >= self.max_seq_len - 1:
                return
            if do_sample:
                _, lg = dec.decode_step_with_logits(cur)
                nxt = sample_next_token(lg, temperature, generator)
            else:
                nxt = dec.decode_step(cur)
            if nxt in stop:
                return
            yield nxt
            cur = nxt

    @staticmethod
    def _sampling(do_sample, temperature, seed):
        if do_sample and not temperature > 0:
            raise ValueError("temperature must be positive when do_sample is set")
        if not do_sample:
            return None
        g = torch.Generator(device="cuda")
        if seed is not None:
            g.manual_seed(int(seed))
        return g


class MegakernelGenerator(_GeneratorBase):
    """High-level generator (reference megakernel_decode.py:1136-1211): prompt tokens run
    through the decode kernel one at a time, then greedy (or, with do_sample, temperature)
    decoding. Greedy is the kernel's fused argmax; a positive temperature does not change
    an argmax, so it only matters with do_sample (generate.py:325-329)."""

    def __init__(self, model_name=None, max_seq_len: int = 2048, seed: int = 0, weights_dict=None):
        w = weights_dict or load_qwen3_weights(model_name, seed=seed, max_seq_len=max_seq_len)
        self.weights = w
        self.decoder = MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                         w["lm_head_weight"], w["cos_table"], w["sin_table"],
                                         len(w["layer_weights"]) // 11, max_seq_len)
        self.tokenizer = w.get("tokenizer")
        self.max_seq_len = max_seq_len

    def _prompt(self, prompt) -> int:
        self.decoder.reset()
        ids = self._encode(prompt)
        if not ids:
            raise ValueError("empty prompt")
        if len(ids) >= self.max_seq_len:
            raise ValueError(f"prompt of {len(ids)} tokens does not fit max_seq_len {self.max_seq_len}")
        for t in ids[:-1]:
            self.decoder.decode_step_async(t)
        return ids[-1]

    def generate_ids(self, prompt, max_new_tokens: int = 100, stop_tokens=None, temperature: float = 1.0,
                     do_sample: bool = False, seed=None, device_loop: bool = False):
        """Generated ids. device_loop (greedy only): the device-resident loop of
        MegakernelDecoder.generate_device (no host read per token)."""
        g = self._sampling(do_sample, temperature, seed)
        last = self._prompt(prompt)
        stop = self._stop(stop_tokens)
        if device_loop and not do_sample:
            n = min(max_new_tokens, self.max_seq_len - 1 - self.decoder.position())
            return self.decoder.generate_device(last, n, stop_tokens=stop) if n > 0 else []
        return list(self._continue(last, max_new_tokens, stop, do_sample, temperature, g, False))

    def generate(self, prompt, max_new_tokens: int = 100, temperature: float = 1.0, stop_tokens=None,
                 do_sample: bool = False, seed=None):
        return self._detok(self.generate_ids(prompt, max_new_tokens, stop_tokens, temperature, do_sample, seed))

    def generate_stream(self, prompt, max_new_tokens: int = 100, stop_tokens=None, temperature: float = 1.0,
                        do_sample: bool = False, seed=None):
        g = self._sampling(do_sample, temperature, seed)
        last = self._prompt(prompt)
        for t in self._continue(last, max_new_tokens, self._stop(stop_tokens), do_sample, temperature, g, False):
            yield self.tokenizer.decode([t]) if self.tokenizer else t


class MegakernelPrefillGenerator(_GeneratorBase):
    """Generator using the prefill kernels for the prompt and the decode kernel after it
    (reference megakernel_decode.py:1214-1307)."""

    decoder_class = MegakernelPrefillDecoder
    default_max_prefill_len = 512

    def __init__(self, model_name=None, max_seq_len: int = 2048, max_prefill_len: int | None = None, seed: int = 0,
                 weights_dict=None):
        max_prefill_len = self.default_max_prefill_len if max_prefill_len is None else max_prefill_len
        w = weights_dict or load_qwen3_weights(model_name, seed=seed, max_seq_len=max_seq_len)
        self.weights = w
        self.decoder = self.decoder_class(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                          w["lm_head_weight"], w["cos_table"], w["sin_table"],
                                          len(w["layer_weights"]) // 11, max_seq_len, max_prefill_len)
        self.tokenizer = w.get("tokenizer")
        self.max_seq_len = max_seq_len
        self.max_prefill_len = max_prefill_len

    def _ids(self, prompt):
        ids = self._encode(prompt)
        if len(ids) > self.max_prefill_len:
            raise ValueError(f"Prompt length {len(ids)} exceeds max prefill length {self.max_prefill_len}")
        return ids

    def _prefill(self, prompt) -> int:
        self.decoder.reset()
        return self.decoder.prefill_step(torch.tensor(self._ids(prompt), dtype=torch.int32))

    def generate_ids(self, prompt, max_new_tokens: int = 100, stop_tokens=None, temperature: float = 1.0,
                     do_sample: bool = False, seed=None):
        g = self._sampling(do_sample, temperature, seed)
        nxt = self._prefill(prompt)
        return list(self._continue(nxt, max_new_tokens, self._stop(stop_tokens), do_sample, temperature, g, True))

    def generate(self, prompt, max_new_tokens: int = 100, stop_tokens=None, temperature: float = 1.0,
                 do_sample: bool = False, seed=None):
        return self._detok(self.generate_ids(prompt, max_new_tokens, stop_tokens, temperature, do_sample, seed))

    def generate_stream(self, prompt, max_new_tokens: int = 100, stop_tokens=None, temperature: float = 1.0,
                        do_sample: bool = False, seed=None):
        g = self._sampling(do_sample, temperature, seed)
        nxt = self._prefill(prompt)
        for t in self._continue(nxt, max_new_tokens, self._stop(stop_tokens), do_sample, temperature, g, True):
            yield self.tokenizer.decode([t]) if self.tokenizer else t

    def prefill_only(self, prompt):
        nxt = self._prefill(prompt)
        return nxt, self.decoder.position()


class MegakernelFusedPrefillGenerator(MegakernelPrefillGenerator):
    """The reference's fused-prefill generator (megakernel_decode.py:1310-1407; prompts of at
    most 64 tokens by default), on MegakernelFusedPrefillDecoder."""

    decoder_class = MegakernelFusedPrefillDecoder
    default_max_prefill_len = 64
