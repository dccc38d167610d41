import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def golden(name):
    return os.path.join(GOLDEN, name)


@pytest.fixture(scope="session")
def state_dict():
    from megaqwen_amd import weights

    return weights.make_state_dict(seed=0)


@pytest.fixture(scope="session")
def oracle_model(state_dict):
    """The numpy oracle on the seeded weights (max_seq 2048)."""
    from megaqwen_amd import rope, weights
    from oracle import qwen3_oracle as O

    flat = weights.layer_weights_flat(state_dict)
    u = weights.bf16_to_u16
    cos, sin = rope.rope_tables(2048)
    return O.Qwen3Oracle(u(state_dict["model.embed_tokens.weight"]), [u(t) for t in flat],
                         u(state_dict["model.norm.weight"]), u(cos), u(sin), 2048)


@pytest.fixture(scope="session")
def gpu_weights(state_dict):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from megaqwen_amd import rope, weights

    dev = "cuda"
    flat = [t.to(dev) for t in weights.layer_weights_flat(state_dict)]
    embed = state_dict["model.embed_tokens.weight"].to(dev)
    cos, sin = rope.rope_tables(16384)
    return {
        "embed_weight": embed,
        "layer_weights": flat,
        "final_norm_weight": state_dict["model.norm.weight"].to(dev),
        "lm_head_weight": embed,
        "cos_table": cos.to(dev),
        "sin_table": sin.to(dev),
    }


@pytest.fixture(scope="session")
def gpu_weights_gamma():
    """The seeded weights with random norm gains (every norm weight bf16(1 + 0.1 randn),
    distinct per layer and norm) on the GPU, RoPE tables for 1024 positions."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from megaqwen_amd import rope, weights

    sd = weights.make_state_dict(seed=0, norms="random")
    dev = "cuda"
    embed = sd["model.embed_tokens.weight"].to(dev)
    cos, sin = rope.rope_tables(1024)
    return {"state_dict": sd, "embed_weight": embed,
            "layer_weights": [t.to(dev) for t in weights.layer_weights_flat(sd)],
            "final_norm_weight": sd["model.norm.weight"].to(dev), "lm_head_weight": embed,
            "cos_table": cos.to(dev), "sin_table": sin.to(dev)}


def load_npz(name):
    return np.load(golden(name), allow_pickle=False)
