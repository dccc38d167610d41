"""numpy restatement of HF Qwen3 bf16 numerics — TEST INFRASTRUCTURE ONLY.

This module is the parity checker for the MI355X kernels. Only `tests/`,
`__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import it;
the product path never does.

What it restates. The north star names "the reference's PyTorch/HF
implementation" as the oracle: third-party HF `transformers` 5.15.0
(`Qwen3ForCausalLM`, not vendored in the reference; the reference pins
`transformers>=4.40.0`, `requirements.txt:2`). The reference calls it at
`csrc/megakernel/megakernel_decode.py:1082-1094` and `verify_correctness.py:10-33`.
Each function below cites the HF lines it follows (paths relative to
`transformers/`). Every bf16 rounding point of HF is reproduced explicitly:
values are carried as float32 arrays holding bf16-representable numbers and
`bf16r` rounds to nearest-even at exactly the places HF casts to bf16.

Accumulation order of the fp32 dot products is numpy/BLAS's, not oneDNN's,
so results can differ from HF by single bf16 ulps where a value sits on a
rounding boundary; the parity tests quantify that against HF fixtures.

Pinning (see tests/test_oracle.py): RoPE tables bitwise vs HF's rotary module;
`rmsnorm`, `apply_rope`, `silu_mul`, `linear` against closed forms and fp64 brute
force; `attention_rows` against invariants (cache_len 1 -> V[0]; equal keys ->
mean of V; GQA h -> h//2), fp64 softmax, and past 512 keys (the blocked online
softmax, `flash_block_update`) against fp64 and a one-block run at 513..8448 keys,
with planted rescale mistakes shown to fail; the single decoder block against the
HF fixture for config 2, with unit and with random norm gammas (misplaced gammas
shown to fail); end-to-end greedy ids and logits against HF's prefill path
(config 1) and HF's decode path (config 1, unit and random gammas).
"""

from __future__ import annotations

import numpy as np

HIDDEN = 1024
INTER = 3072
NQ = 16
NKV = 8
HD = 128
EPS = 1e-6
SCALE = np.float32(HD ** -0.5)  # HF Qwen3Attention.scaling (modeling_qwen3.py:221)


# ---------------------------------------------------------------- bf16 helpers

def bf16r(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out).astype(np.float32)


def u16_to_f32(u) -> np.ndarray:
    """Raw bf16 bits (uint16) -> float32."""
    u = np.ascontiguousarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << 16).view(np.float32)


def f32_to_u16(x) -> np.ndarray:
    """float32 holding bf16 values -> raw bf16 bits (rounds first)."""
    return (bf16r(x).view(np.uint32) >> 16).astype(np.uint16)


# ---------------------------------------------------------------- layer pieces

def rmsnorm(x, w, eps: float = EPS) -> np.ndarray:
    """Qwen3RMSNorm (modeling_qwen3.py:59-64) on bf16 input `x` (last axis).

    fp32: var = mean(x^2); y = bf16(x * rsqrt(var + eps)); out = bf16(w * y).
    rsqrt is taken as 1/sqrt (two correctly rounded fp32 ops).
    """
    x = np.asarray(x, dtype=np.float32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    rstd = np.float32(1.0) / np.sqrt(var + np.float32(eps), dtype=np.float32)
    y = bf16r(x * rstd)
    return bf16r(np.asarray(w, dtype=np.float32) * y)


def linear(w, x) -> np.ndarray:
    """nn.Linear without bias on bf16 tensors: bf16(x @ w.T), fp32 accumulation."""
    return bf16r(np.asarray(x, dtype=np.float32) @ np.asarray(w, dtype=np.float32).T)


def rotate_half(x) -> np.ndarray:
    """modeling_qwen3.py:140-144: cat(-x2, x1) over the last axis (exact in bf16)."""
    h = x.shape[-1] // 2
    return np.concatenate((-x[..., h:], x[..., :h]), axis=-1)


def apply_rope(x, cos, sin) -> np.ndarray:
    """apply_rotary_pos_emb (modeling_qwen3.py:147-170) in bf16: three rounded ops."""
    a = bf16r(x * cos)
    b = bf16r(rotate_half(x) * sin)
    return bf16r(a + b)


def silu_mul(g, u) -> np.ndarray:
    """Qwen3MLP act (modeling_qwen3.py:81-83): bf16(bf16(silu(g)) * u), silu in fp32."""
    g = np.asarray(g, dtype=np.float32)
    s = bf16r(g / (np.float32(1.0) + np.exp(-g, dtype=np.float32)))
    return bf16r(s * np.asarray(u, dtype=np.float32))


def attention_rows(q, K, V, q_pos, scale=SCALE, kv_split: int | None = None) -> np.ndarray:
    """Causal attention for query rows following torch's CPU flash kernel.

    HF's default attention is sdpa (`modeling_utils.py:1928`), which on the CPU
    for bf16 runs aten's flash-attention kernel: scores s = (q.k) * scale in
    fp32; kv processed in blocks of `kv_split` (512 if kv_len >= 512 else kv_len)
    with a running max; p = exp(s - max) in fp32, summed unrounded, but cast to
    bf16 before the P.V product; out = bf16(acc * (1 / sum)).

    q: [R, 128] (bf16 values), K, V: [L, 128]; q_pos[r] is the last key index row
    r may attend (causal). Returns [R, 128] bf16 values.
    """
    q = np.asarray(q, dtype=np.float32)
    K = np.asarray(K, dtype=np.float32)
    V = np.asarray(V, dtype=np.float32)
    q_pos = np.asarray(q_pos)
    R = q.shape[0]
    L = K.shape[0]
    if kv_split is None:
        kv_split = 512 if L >= 512 else L
    m = np.full((R, 1), -np.inf, dtype=np.float32)
    lsum = np.zeros((R, 1), dtype=np.float32)
    acc = np.zeros((R, q.shape[1]), dtype=np.float32)
    col = np.arange(L)
    for s0 in range(0, L, kv_split):
        s1 = min(L, s0 + kv_split)
        s = (q @ K[s0:s1].T).astype(np.float32) * np.float32(scale)
        mask = col[None, s0:s1] > q_pos[:, None]
        s = np.where(mask, np.float32(-np.inf), s)
        m, lsum, acc = flash_block_update(m, lsum, acc, s, V[s0:s1])
    return bf16r(acc * (np.float32(1.0) / lsum))


def flash_block_update(m, lsum, acc, s, Vb):
    """One kv block of the online softmax (torch's CPU flash kernel, see attention_rows):
    the running max m, sum lsum and accumulator acc are rescaled by exp(m_old - m_new)
    before the block's exp(s - m_new) (summed in fp32, cast to bf16 for P.V) is added."""
    bm = np.maximum(m, s.max(axis=1, keepdims=True))
    bm_safe = np.where(np.isinf(bm), np.float32(0), bm)
    p = np.exp(s - bm_safe, dtype=np.float32)
    alpha = np.where(np.isinf(m), np.float32(0), np.exp(m - bm_safe, dtype=np.float32))
    lsum = p.sum(axis=1, keepdims=True, dtype=np.float32) + alpha * lsum
    acc = acc * alpha + bf16r(p) @ Vb
    return bm, lsum, acc


def attention_decode_fp64(q, K, V, scale=float(SCALE)) -> np.ndarray:
    """Exact softmax attention in float64 (no rounding) for pinning tests."""
    q = np.asarray(q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    s = (K @ q) * scale
    p = np.exp(s - s.max())
    return (p / p.sum()) @ V


# ---------------------------------------------------------------- model

class LayerWeights:
    """One decoder layer's weights as float32 arrays (bf16-valued)."""

    __slots__ = ("input_ln", "q", "k", "v", "q_norm", "k_norm", "o", "post_ln", "gate", "up", "down")

    def __init__(self, arrays):
        for name, a in zip(self.__slots__, arrays):
            setattr(self, name, a)


def qkv_project(lw: LayerWeights, y, cos, sin):
    """q/k/v projections, per-head QK-norm, RoPE (modeling_qwen3.py:247-257).

    y: [S, 1024] normalized input; cos, sin: [S, 128]. Returns q [S,16,128],
    k [S,8,128] (post-RoPE, what the KV cache stores), v [S,8,128].
    """
    S = y.shape[0]
    q = linear(lw.q, y).reshape(S, NQ, HD)
    k = linear(lw.k, y).reshape(S, NKV, HD)
    v = linear(lw.v, y).reshape(S, NKV, HD)
    q = rmsnorm(q, lw.q_norm)
    k = rmsnorm(k, lw.k_norm)
    q = apply_rope(q, cos[:, None, :], sin[:, None, :])
    k = apply_rope(k, cos[:, None, :], sin[:, None, :])
    return q, k, v


def decoder_layer(lw: LayerWeights, h, positions, cos_tab, sin_tab, k_cache, v_cache, trace=None):
    """Qwen3DecoderLayer.forward (modeling_qwen3.py:304-323) for S new tokens.

    h: [S, 1024] bf16 hidden; positions: [S] absolute positions (consecutive);
    k_cache, v_cache: [8, max_seq, 128] arrays updated in place at `positions`.
    Returns the new hidden [S, 1024].
    """
    positions = np.asarray(positions)
    y = rmsnorm(h, lw.input_ln)
    q, k, v = qkv_project(lw, y, cos_tab[positions], sin_tab[positions])
    k_cache[:, positions, :] = k.transpose(1, 0, 2)
    v_cache[:, positions, :] = v.transpose(1, 0, 2)
    L = int(positions[-1]) + 1
    attn = np.empty((h.shape[0], NQ, HD), dtype=np.float32)
    for hq in range(NQ):
        g = kv_head_of(hq)
        attn[:, hq, :] = attention_rows(q[:, hq, :], k_cache[g, :L], v_cache[g, :L], positions)
    attn = attn.reshape(h.shape[0], NQ * HD)
    o = linear(lw.o, attn)
    h1 = residual_add(h, o)
    y2 = rmsnorm(h1, lw.post_ln)
    m = silu_mul(linear(lw.gate, y2), linear(lw.up, y2))
    d = linear(lw.down, m)
    out = residual_add(h1, d)
    if trace is not None:
        trace.update(y=y, q=q, k=k, v=v, attn=attn, o=o, h1=h1, y2=y2, m=m, d=d, out=out)
    return out


class Qwen3Oracle:
    """Batch-1 Qwen3 forward with explicit KV cache, HF rounding points.

    Weights come in as bf16 raw bits (uint16 numpy arrays) in the reference's
    flat order (28 x 11, `megakernel_decode.py:1106-1120`) plus embed / final
    norm. lm_head is tied to the embedding.
    """

    def __init__(self, embed_u16, layers_u16, final_norm_u16, cos_u16, sin_u16, max_seq_len: int):
        self.embed = u16_to_f32(embed_u16)
        self.layers = [LayerWeights([u16_to_f32(a) for a in layers_u16[i * 11:(i + 1) * 11]])
                       for i in range(len(layers_u16) // 11)]
        self.final_norm = u16_to_f32(final_norm_u16)
        self.cos = u16_to_f32(cos_u16)
        self.sin = u16_to_f32(sin_u16)
        self.max_seq_len = max_seq_len
        n = len(self.layers)
        self.k_cache = np.zeros((n, NKV, max_seq_len, HD), dtype=np.float32)
        self.v_cache = np.zeros((n, NKV, max_seq_len, HD), dtype=np.float32)
        self.position = 0

    def reset(self):
        self.k_cache[:] = 0
        self.v_cache[:] = 0
        self.position = 0

    def forward(self, ids, start: int):
        """Run tokens `ids` at positions start.. ; returns (final hidden [S,1024], normed [S,1024])."""
        ids = np.asarray(ids)
        positions = np.arange(start, start + len(ids))
        if positions[-1] >= self.max_seq_len:
            raise ValueError("position exceeds max_seq_len")
        h = self.embed[ids]
        for li, lw in enumerate(self.layers):
            h = decoder_layer(lw, h, positions, self.cos, self.sin, self.k_cache[li], self.v_cache[li])
        return h, rmsnorm(h, self.final_norm)

    def logits(self, normed) -> np.ndarray:
        """Tied LM head, bf16 logits (modeling_qwen3.py:493-495)."""
        return linear(self.embed, normed)

    def decode_step(self, token: int):
        """One decode step at self.position; returns (greedy next id, bf16 logits)."""
        _, y = self.forward([token], self.position)
        self.position += 1
        lg = self.logits(y[-1:])[0]
        return int(argmax_first(lg)), lg

    def prefill(self, ids):
        """Process a prompt at positions 0..S-1; returns (next id, last-position bf16 logits)."""
        self.reset()
        _, y = self.forward(ids, 0)
        self.position = len(ids)
        lg = self.logits(y[-1:])[0]
        return int(argmax_first(lg)), lg

    def greedy(self, prompt, n_new: int, topk: int = 8, full_steps=()):
        """HF-style greedy generation: prefill prompt, then n_new decode steps.

        Returns (ids, per-step top-k ids, per-step top-k bf16 logit values,
        {step: full logits} for the steps in `full_steps`).
        """
        nxt, lg = self.prefill(prompt)
        ids, tk_ids, tk_vals, full = [], [], [], {}
        for step in range(n_new):
            ids.append(nxt)
            ti = topk_first(lg, topk)
            tk_ids.append(ti)
            tk_vals.append(lg[ti])
            if step in full_steps:
                full[step] = lg
            if step + 1 < n_new:
                nxt, lg = self.decode_step(nxt)
        return ids, np.array(tk_ids), np.array(tk_vals), full


def kv_head_of(hq: int) -> int:
    """repeat_kv (modeling_qwen3.py:173-182): q head hq reads kv head hq // (16 // 8)."""
    return hq // (NQ // NKV)


def residual_add(a, b) -> np.ndarray:
    """Residual add in bf16 (modeling_qwen3.py:316,322)."""
    return bf16r(a + b)


def argmax_first(x) -> int:
    """torch.argmax semantics: index of the first maximum (generation/utils.py:2925)."""
    return int(np.argmax(np.asarray(x, dtype=np.float32)))


def topk_first(x, k: int) -> np.ndarray:
    """Top-k indices by value descending, ties broken by lower index."""
    x = np.asarray(x, dtype=np.float32)
    idx = np.lexsort((np.arange(x.size), -x))
    return idx[:k]
