"""RoPE cos/sin tables identical to HF Qwen3's rotary embedding.

HF (`transformers/models/qwen3/modeling_qwen3.py:121,126-137`) computes
`inv_freq = 1 / theta ** (arange(0, 128, 2) / 128)` in fp32, `freqs = pos * inv_freq`
(fp32), `emb = cat(freqs, freqs)`, and casts `cos(emb)`, `sin(emb)` to bf16.
The reference's table builder (`chat.py:48-56`) has the same shape
`[max_seq, 128]` with duplicated halves; `load_qwen3_weights`
(`csrc/megakernel/megakernel_decode.py:1096-1102`) uses theta = 1e4, which is
wrong for Qwen3 — this module always uses the configured theta (1e6).

The tables are computed on the CPU with torch so they match HF bit for bit;
the kernels only consume them.
"""

from __future__ import annotations

import torch

from . import config as C


def inv_freq(theta: float = C.ROPE_THETA, head_dim: int = C.HEAD_DIM) -> torch.Tensor:
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rope_tables(max_seq_len: int, theta: float = C.ROPE_THETA, head_dim: int = C.HEAD_DIM):
    """Return (cos, sin) bf16 CPU tensors of shape [max_seq_len, head_dim]."""
    if max_seq_len <= 0:
        raise ValueError("max_seq_len must be positive")
    inv = inv_freq(theta, head_dim)
    pos = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(pos, inv)
    emb = torch.cat((freqs, freqs), dim=-1).contiguous()
    return emb.cos().to(torch.bfloat16).contiguous(), emb.sin().to(torch.bfloat16).contiguous()


def precompute_rope_freqs(head_dim: int, max_seq_len: int, theta: float = C.ROPE_THETA, device="cpu"):
    """Reference-named helper (`chat.py:48-56`): returns (cos, sin) bf16 on `device`."""
    cos, sin = rope_tables(max_seq_len, theta, head_dim)
    return cos.to(device), sin.to(device)
