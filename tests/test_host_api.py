"""CPU tests of the Python surface's host logic: error recovery of the decoder state
machine, temperature sampling, the local checkpoint loader and the generators' loops
(with the C ABI replaced by a stand-in that records calls; no kernel runs here)."""

import json
import os

import pytest
import torch

from megaqwen_amd import _abi
from megaqwen_amd import config as C
from megaqwen_amd import megakernel_decode as MK
from megaqwen_amd import weights


class _FakeLib:
    """Stands in for the C ABI: records each launch's position and writes a scripted
    token where the kernel would (the output tensor is a CPU tensor here)."""

    def __init__(self, tokens):
        self.tokens = list(tokens)
        self.launches = []
        self.resets = 0

    def launch_ldg_decode(self, *args):
        import ctypes
        self.launches.append(args[-5])  # position
        ctypes.c_int.from_address(args[1]).value = self.tokens.pop(0)
        return 0

    def mq_reset_workspace(self, dev):
        self.resets += 1
        return 0

    def mq_strerror(self, st):
        return b"x"


def _cpu_decoder(fake, monkeypatch, max_seq=16):
    dec = object.__new__(MK.MegakernelDecoder)
    dec.max_seq_len_ = max_seq
    dec.num_layers_ = 28
    dec.position_ = 0
    dec.attn_scale_ = MK.ATTN_SCALE
    dec.output_token_ = torch.zeros(1, dtype=torch.int32)
    for name in ("embed_weight_", "d_layer_weights_", "final_norm_weight_", "lm_head_weight_", "cos_table_",
                 "sin_table_", "k_cache_", "v_cache_", "hidden_buffer_", "g_activations_", "g_residual_", "g_q_",
                 "g_k_", "g_v_", "g_attn_out_", "g_mlp_intermediate_", "g_normalized_", "block_max_vals_",
                 "block_max_idxs_"):
        setattr(dec, name, torch.zeros(1))
    monkeypatch.setattr(MK, "_stream", lambda: 0)
    monkeypatch.setattr(MK._abi, "lib", lambda: fake)
    return dec


def test_failed_step_restores_position_and_resets_workspace(monkeypatch):
    """A negative token (kernel error) raises MegakernelError, resets the workspace and
    moves the position back, so the next step rewrites the failed step's KV slots."""
    fake = _FakeLib([5, 6, -2, 7])
    dec = _cpu_decoder(fake, monkeypatch)
    assert dec.decode_step(1) == 5
    assert dec.decode_step(5) == 6
    assert dec.position() == 2
    with pytest.raises(_abi.MegakernelError):
        dec.decode_step(6)
    assert dec.position() == 2 and fake.resets == 1
    assert dec.decode_step(6) == 7
    assert fake.launches == [0, 1, 2, 2]
    assert dec.position() == 3


def test_position_cap_and_token_range(monkeypatch):
    fake = _FakeLib([1] * 4)
    dec = _cpu_decoder(fake, monkeypatch, max_seq=2)
    with pytest.raises(ValueError):
        dec.decode_step(C.VOCAB_SIZE)
    with pytest.raises(ValueError):
        dec.decode_step(-1)
    dec.decode_step(3)
    dec.decode_step(3)
    with pytest.raises(RuntimeError, match="KV cache full"):
        dec.decode_step(3)
    assert fake.launches == [0, 1]


def test_sampling_follows_the_softmax():
    """sample_next_token draws from softmax(logits / T) (generate.py:325-329)."""
    logits = torch.tensor([0.0, 1.0, 2.0, -30.0])
    g = torch.Generator().manual_seed(0)
    n = 4000
    draws = torch.tensor([MK.sample_next_token(logits, 0.7, g) for _ in range(n)])
    p = torch.softmax(logits / 0.7, dim=0)
    freq = torch.bincount(draws, minlength=4).float() / n
    assert torch.all((freq - p).abs() <= 4 * torch.sqrt(p * (1 - p) / n) + 1e-3)
    assert freq[3] == 0
    # low temperature concentrates on the argmax
    g.manual_seed(1)
    assert all(MK.sample_next_token(logits, 0.01, g) == 2 for _ in range(50))
    with pytest.raises(ValueError):
        MK.sample_next_token(logits, 0.0, g)


def test_checkpoint_round_trip(tmp_path):
    """save_qwen3_checkpoint -> load_qwen3_weights(dir): HF key names, tied LM head, the
    reference's flat 11-per-layer order, RoPE theta from the config."""
    sd = weights.make_state_dict(seed=3, num_layers=2, norms="random")
    MK.save_qwen3_checkpoint(sd, str(tmp_path), num_layers=2)
    w = MK.load_qwen3_weights(str(tmp_path), max_seq_len=32, device="cpu")
    assert torch.equal(w["embed_weight"], sd["model.embed_tokens.weight"])
    assert w["lm_head_weight"].data_ptr() == w["embed_weight"].data_ptr()
    flat = weights.layer_weights_flat(sd, 2)
    assert len(w["layer_weights"]) == 22
    for a, b in zip(w["layer_weights"], flat):
        assert torch.equal(a, b)
    assert torch.equal(w["final_norm_weight"], sd["model.norm.weight"])
    from megaqwen_amd import rope
    cos, sin = rope.rope_tables(32)
    assert torch.equal(w["cos_table"], cos) and torch.equal(w["sin_table"], sin)
    assert w["config"]["num_hidden_layers"] == 2
    assert w["tokenizer"] is None


def test_checkpoint_untied_head_and_theta(tmp_path):
    sd = weights.make_state_dict(seed=3, num_layers=1)
    MK.save_qwen3_checkpoint(sd, str(tmp_path), num_layers=1)
    cfg = json.load(open(tmp_path / "config.json"))
    cfg["tie_word_embeddings"] = False
    del cfg["rope_theta"]
    cfg["rope_parameters"] = {"rope_type": "default", "rope_theta": 10000.0}
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    from safetensors.torch import load_file, save_file
    t = load_file(str(tmp_path / "model.safetensors"))
    t["lm_head.weight"] = (t["model.embed_tokens.weight"].float() * 2).to(torch.bfloat16)
    save_file(t, str(tmp_path / "model.safetensors"))
    w = MK.load_qwen3_weights(str(tmp_path), max_seq_len=8, device="cpu")
    assert torch.equal(w["lm_head_weight"], t["lm_head.weight"])
    from megaqwen_amd import rope
    assert torch.equal(w["cos_table"], rope.rope_tables(8, theta=1e4)[0])


def test_checkpoint_errors(tmp_path, monkeypatch):
    monkeypatch.setenv("HF_HUB_CACHE", str(tmp_path / "hub"))
    monkeypatch.setenv("HOME", str(tmp_path))
    with pytest.raises(FileNotFoundError):
        MK.load_qwen3_weights("Qwen/Qwen3-0.6B", device="cpu")
    sd = weights.make_state_dict(seed=0, num_layers=1)
    snap = tmp_path / "hub" / "models--Qwen--Qwen3-0.6B" / "snapshots" / "abc"
    MK.save_qwen3_checkpoint(sd, str(snap), num_layers=1)
    assert MK.find_local_checkpoint("Qwen/Qwen3-0.6B") == str(snap)
    cfg = json.load(open(snap / "config.json"))
    cfg["hidden_size"] = 2048
    json.dump(cfg, open(snap / "config.json", "w"))
    with pytest.raises(ValueError, match="Qwen3-0.6B shaped"):
        MK.load_qwen3_weights("Qwen/Qwen3-0.6B", device="cpu")


class _ScriptedDecoder:
    """Decoder stand-in for the generator loops: step k returns script[k]."""

    def __init__(self, script, logits=None):
        self.script = list(script)
        self.pos = 0
        self.fed = []
        self.logits = logits

    def reset(self):
        self.pos = 0

    def position(self):
        return self.pos

    def decode_step_async(self, t):
        self.fed.append(t)
        self.pos += 1

    def decode_step(self, t):
        self.fed.append(t)
        self.pos += 1
        return self.script.pop(0)

    def decode_step_with_logits(self, t):
        return self.decode_step(t), self.logits

    def prefill_step(self, ids):
        self.fed.extend(ids.tolist())
        self.pos = len(ids)
        return self.script.pop(0)


def _gen(cls, script, max_seq=64, **kw):
    g = object.__new__(cls)
    g.decoder = _ScriptedDecoder(script, **kw)
    g.tokenizer = None
    g.max_seq_len = max_seq
    g.max_prefill_len = 8
    return g


def test_generator_loop_semantics():
    """Prompt tokens through decode, stop tokens excluded, position cap (reference
    megakernel_decode.py:1158-1185)."""
    g = _gen(MK.MegakernelGenerator, [10, 11, 12, 13, 14])
    assert g.generate_ids([1, 2, 3], max_new_tokens=5, stop_tokens=[13]) == [10, 11, 12]
    assert g.decoder.fed == [1, 2, 3, 10, 11, 12]
    g = _gen(MK.MegakernelGenerator, list(range(100, 200)), max_seq=6)
    assert len(g.generate_ids([1, 2], max_new_tokens=50)) == 4  # positions up to max_seq - 1
    with pytest.raises(ValueError):
        _gen(MK.MegakernelGenerator, []).generate_ids("text")


def test_prefill_generator_loop_semantics():
    g = _gen(MK.MegakernelPrefillGenerator, [7, 8, 9, 10])
    assert g.generate_ids([1, 2, 3], max_new_tokens=3) == [7, 8, 9]
    g = _gen(MK.MegakernelFusedPrefillGenerator, [7, 8])
    with pytest.raises(ValueError, match="exceeds max prefill length"):
        g.generate_ids(list(range(9)))
    assert MK.MegakernelFusedPrefillGenerator.default_max_prefill_len == 64


def test_sampling_path_uses_logits():
    logits = torch.full((C.VOCAB_SIZE,), -1e4)
    logits[4242] = 0.0
    g = _gen(MK.MegakernelGenerator, [1, 1, 1], logits=logits)
    g._sampling = staticmethod(lambda d, t, s: torch.Generator().manual_seed(0) if d else None)
    assert g.generate_ids([5], max_new_tokens=3, do_sample=True, temperature=0.8) == [4242, 4242, 4242]
    with pytest.raises(ValueError):
        MK._GeneratorBase._sampling(True, 0.0, None)
