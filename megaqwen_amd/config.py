"""Qwen3-0.6B shape constants shared by the host code and the HIP kernels.

Mirrors `csrc/megakernel/megakernel_decode.py:17-25` and `csrc/megakernel/config.cuh:33-40`
of the reference (hidden 1024, 16 q / 8 kv heads of 128, MLP 3072, 28 layers,
vocab 151936).  RMSNorm eps and RoPE theta follow the HF Qwen3 config
(`transformers/models/qwen3/configuration_qwen3.py`), theta = 1e6.
"""

HIDDEN_SIZE = 1024
INTERMEDIATE_SIZE = 3072
NUM_Q_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
Q_SIZE = NUM_Q_HEADS * HEAD_DIM
KV_SIZE = NUM_KV_HEADS * HEAD_DIM
NUM_LAYERS = 28
VOCAB_SIZE = 151936
RMS_EPS = 1e-6
ROPE_THETA = 1e6
MAX_POSITION_EMBEDDINGS = 40960

# Index of each tensor inside one layer's 11-entry slice of `layer_weights_flat`
# (reference order: megakernel_decode.py:1106-1120, LDGLayerWeights fused_decode_ldg.cu:24-36).
LAYER_WEIGHT_NAMES = (
    "input_layernorm",
    "q_proj",
    "k_proj",
    "v_proj",
    "q_norm",
    "k_norm",
    "o_proj",
    "post_attention_layernorm",
    "gate_proj",
    "up_proj",
    "down_proj",
)

LAYER_WEIGHT_SHAPES = {
    "input_layernorm": (HIDDEN_SIZE,),
    "q_proj": (Q_SIZE, HIDDEN_SIZE),
    "k_proj": (KV_SIZE, HIDDEN_SIZE),
    "v_proj": (KV_SIZE, HIDDEN_SIZE),
    "q_norm": (HEAD_DIM,),
    "k_norm": (HEAD_DIM,),
    "o_proj": (HIDDEN_SIZE, Q_SIZE),
    "post_attention_layernorm": (HIDDEN_SIZE,),
    "gate_proj": (INTERMEDIATE_SIZE, HIDDEN_SIZE),
    "up_proj": (INTERMEDIATE_SIZE, HIDDEN_SIZE),
    "down_proj": (HIDDEN_SIZE, INTERMEDIATE_SIZE),
}

# Algorithmic HBM bytes of one decode step (bf16 weights, batch 1).
def _numel(shape):
    n = 1
    for d in shape:
        n *= d
    return n


LAYER_PARAMS = sum(_numel(s) for s in LAYER_WEIGHT_SHAPES.values())
WEIGHT_BYTES_PER_TOKEN = 2 * (NUM_LAYERS * LAYER_PARAMS + VOCAB_SIZE * HIDDEN_SIZE + 2 * HIDDEN_SIZE)
KV_BYTES_PER_POSITION = NUM_LAYERS * 2 * NUM_KV_HEADS * HEAD_DIM * 2


def decode_bytes(position: int) -> int:
    """Algorithmic bytes moved by one decode step whose query sits at `position`.

    Weights (layers + tied LM head + embedding row + final norm) + KV read of
    positions 0..position + KV write of slot `position`.
    """
    return WEIGHT_BYTES_PER_TOKEN + KV_BYTES_PER_POSITION * (position + 1) + KV_BYTES_PER_POSITION


# Matrix-product flops of one prefill of S tokens (the MFMA work).
LINEAR_PARAMS = NUM_LAYERS * sum(_numel(s) for n, s in LAYER_WEIGHT_SHAPES.items() if len(s) == 2)


def prefill_flops(seq_len: int) -> int:
    """2 flops per multiply-add: the 7 linear layers of every layer for all S rows,
    causal attention (QK^T and PV over keys 0..s for row s, 16 query heads of 128),
    and the tied LM head for the last row."""
    S = seq_len
    linear = 2 * S * LINEAR_PARAMS
    attention = NUM_LAYERS * NUM_Q_HEADS * 2 * 2 * HEAD_DIM * S * (S + 1) // 2
    lm_head = 2 * VOCAB_SIZE * HIDDEN_SIZE
    return linear + attention + lm_head
