"""Seeded random-init Qwen3-0.6B weights in HF `state_dict` order.

The reference loads real weights from the HF hub (`csrc/megakernel/megakernel_decode.py:1077-1133`,
`load_qwen3_weights`); no checkpoint is reachable offline, so every test and
benchmark uses synthetic weights generated here:

* `g = torch.Generator("cpu").manual_seed(seed)`;
* the HF `Qwen3ForCausalLM` state_dict keys are walked in their canonical
  order (embed, then per layer q/k/v/o, q_norm/k_norm, gate/up/down,
  input/post norms, then the final norm; `lm_head` is tied to the embedding);
* each matrix is `randn(shape, generator=g) * 0.02` in fp32, cast to bf16
  (round-to-nearest-even);
* every norm weight is 1, or, with `norms="random"`,
  `bf16(1 + 0.1 * randn)` drawn per norm tensor from a second generator
  (`manual_seed(seed + 1000)`), so the matrices are unchanged and every gamma
  (input, post-attention, q/k and final norms of every layer) is distinct: that
  variant exists to show that each gamma is applied, and to the right place.

`layer_weights_flat` follows the reference's 11-per-layer order
(`megakernel_decode.py:1106-1120`).
"""

from __future__ import annotations

import hashlib

import torch

from . import config as C


def hf_state_dict_keys(num_layers: int = C.NUM_LAYERS) -> list[str]:
    """HF `Qwen3ForCausalLM.state_dict()` key order (transformers 5.15.0), lm_head excluded (tied)."""
    keys = ["model.embed_tokens.weight"]
    for i in range(num_layers):
        p = f"model.layers.{i}."
        keys += [
            p + "self_attn.q_proj.weight",
            p + "self_attn.k_proj.weight",
            p + "self_attn.v_proj.weight",
            p + "self_attn.o_proj.weight",
            p + "self_attn.q_norm.weight",
            p + "self_attn.k_norm.weight",
            p + "mlp.gate_proj.weight",
            p + "mlp.up_proj.weight",
            p + "mlp.down_proj.weight",
            p + "input_layernorm.weight",
            p + "post_attention_layernorm.weight",
        ]
    keys.append("model.norm.weight")
    return keys


def _shape_of(key: str) -> tuple[int, ...]:
    if key == "model.embed_tokens.weight":
        return (C.VOCAB_SIZE, C.HIDDEN_SIZE)
    if key == "model.norm.weight":
        return (C.HIDDEN_SIZE,)
    name = key.split(".")[-2]
    return C.LAYER_WEIGHT_SHAPES[name]


def _is_norm(key: str) -> bool:
    return key.endswith("norm.weight")


NORM_STD = 0.1


def make_state_dict(seed: int = 0, num_layers: int = C.NUM_LAYERS, std: float = 0.02,
                    norms: str = "ones") -> dict[str, torch.Tensor]:
    """Return the seeded bf16 state dict (CPU tensors), HF key names, lm_head tied.

    norms: "ones" (every norm weight 1) or "random" (bf16(1 + NORM_STD * randn) from
    `manual_seed(seed + 1000)`, walked in the same key order).
    """
    if norms not in ("ones", "random"):
        raise ValueError(f"norms must be 'ones' or 'random', got {norms!r}")
    g = torch.Generator("cpu").manual_seed(seed)
    gn = torch.Generator("cpu").manual_seed(seed + 1000)
    sd: dict[str, torch.Tensor] = {}
    for key in hf_state_dict_keys(num_layers):
        shape = _shape_of(key)
        if _is_norm(key):
            if norms == "ones":
                sd[key] = torch.ones(shape, dtype=torch.bfloat16)
            else:
                sd[key] = (1.0 + NORM_STD * torch.randn(shape, generator=gn, dtype=torch.float32)).to(torch.bfloat16)
        else:
            sd[key] = (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(torch.bfloat16)
    return sd


def layer_weights_flat(sd: dict[str, torch.Tensor], num_layers: int = C.NUM_LAYERS) -> list[torch.Tensor]:
    """Flatten into the reference's 28 x 11 order (megakernel_decode.py:1106-1120)."""
    out = []
    for i in range(num_layers):
        p = f"model.layers.{i}."
        out += [
            sd[p + "input_layernorm.weight"],
            sd[p + "self_attn.q_proj.weight"],
            sd[p + "self_attn.k_proj.weight"],
            sd[p + "self_attn.v_proj.weight"],
            sd[p + "self_attn.q_norm.weight"],
            sd[p + "self_attn.k_norm.weight"],
            sd[p + "self_attn.o_proj.weight"],
            sd[p + "post_attention_layernorm.weight"],
            sd[p + "mlp.gate_proj.weight"],
            sd[p + "mlp.up_proj.weight"],
            sd[p + "mlp.down_proj.weight"],
        ]
    return [t.contiguous() for t in out]


def tensor_sha256(t: torch.Tensor) -> str:
    """sha256 of a tensor's raw bytes (detects RNG drift across torch versions)."""
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def random_prompt(n: int, seed: int = 1, vocab: int = C.VOCAB_SIZE) -> list[int]:
    """Uniform random token ids from `manual_seed(seed)`."""
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()


def bf16_to_u16(t: torch.Tensor):
    """bf16 CPU tensor -> numpy uint16 array of the raw bits (for the numpy oracle)."""
    return t.contiguous().view(torch.int16).numpy().view("uint16")
