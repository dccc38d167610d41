"""Write the HF golden fixtures used by the parity tests.

Runs third-party HF `transformers` (5.15.0 in the build container; the
reference's oracle per its `requirements.txt:2` and call sites
`csrc/megakernel/megakernel_decode.py:1082-1094`, `verify_correctness.py:10-33`)
on the seeded synthetic weights of `megaqwen_amd.weights`. Nothing from the
reference repository is imported or executed. The fixtures are small `.npz` /
`.json` files committed next to this script; GPU boxes never run it.

Usage: python tests/golden/make_golden.py [rope] [block] [c1] [c4] [c3] [c5] [c1d] [blockg] [c1g] [c4g]

* c1d: config 1 on HF's decode path (the prompt fed one token at a time through the
  KV cache, as the megakernel decoder does), full logits at steps 0, 15 and 31;
* blockg / c1g / c4g: the block, config-1 (decode path) and a 64-token prefill case
  on the `norms="random"` weights, whose norm gammas all differ from 1 and from
  each other.
"""

from __future__ import annotations

import json
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))

from megaqwen_amd import config as C  # noqa: E402
from megaqwen_amd import rope, weights  # noqa: E402

TOPK = 8


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def hf_config():
    from transformers import Qwen3Config

    return Qwen3Config(
        vocab_size=C.VOCAB_SIZE, hidden_size=C.HIDDEN_SIZE, intermediate_size=C.INTERMEDIATE_SIZE,
        num_hidden_layers=C.NUM_LAYERS, num_attention_heads=C.NUM_Q_HEADS, num_key_value_heads=C.NUM_KV_HEADS,
        head_dim=C.HEAD_DIM, rms_norm_eps=C.RMS_EPS,
        rope_parameters={"rope_type": "default", "rope_theta": C.ROPE_THETA},
        tie_word_embeddings=True, max_position_embeddings=C.MAX_POSITION_EMBEDDINGS,
        attention_bias=False, hidden_act="silu", attn_implementation="sdpa",
    )


def hf_model(sd):
    from transformers import Qwen3ForCausalLM

    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        model = Qwen3ForCausalLM(hf_config())
    finally:
        torch.set_default_dtype(prev)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert set(missing) <= {"lm_head.weight"}, missing
    model.tie_weights()
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    assert model.model.rotary_emb.inv_freq.dtype == torch.float32
    assert model.config._attn_implementation == "sdpa"
    return model.eval()


def write_rope():
    """HF rotary cos/sin vs our tables, bitwise, for positions 0..8447."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    n = 8448
    rot = Qwen3RotaryEmbedding(hf_config())
    x = torch.zeros(1, dtype=torch.bfloat16)
    cos_hf, sin_hf = rot(x, torch.arange(n)[None, :])
    cos, sin = rope.rope_tables(n)
    same = bool(torch.equal(cos_hf[0], cos) and torch.equal(sin_hf[0], sin))
    sample = [0, 1, 2, 200, 511, 2047, 8191, 8447]
    np.savez_compressed(os.path.join(HERE, "rope_hf.npz"), positions=np.array(sample),
                        cos=u16(cos_hf[0][sample]), sin=u16(sin_hf[0][sample]))
    meta = {"n": n, "bitwise_equal_to_rope_tables": same,
            "cos_sha256": weights.tensor_sha256(cos_hf[0].contiguous()),
            "sin_sha256": weights.tensor_sha256(sin_hf[0].contiguous())}
    json.dump(meta, open(os.path.join(HERE, "rope_hf.json"), "w"), indent=1)
    print("rope", meta)


def block_inputs():
    """Config 2 inputs: hidden N(0,1) and KV[0..199] N(0,1), bf16, from manual_seed(2)."""
    g = torch.Generator("cpu").manual_seed(2)
    hidden = torch.randn(C.HIDDEN_SIZE, generator=g).to(torch.bfloat16)
    k = torch.randn(C.NUM_KV_HEADS, 200, C.HEAD_DIM, generator=g).to(torch.bfloat16)
    v = torch.randn(C.NUM_KV_HEADS, 200, C.HEAD_DIM, generator=g).to(torch.bfloat16)
    return hidden, k, v


def write_block(sd, name="block_pos200"):
    """Config 2: one decoder block (layer 0 weights) decoding at position 200."""
    from transformers import DynamicCache
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding

    cfg = hf_config()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        layer = Qwen3DecoderLayer(cfg, 0)
    finally:
        torch.set_default_dtype(prev)
    lsd = {k[len("model.layers.0."):]: v for k, v in sd.items() if k.startswith("model.layers.0.")}
    layer.load_state_dict(lsd, strict=True)
    layer.eval()
    rot = Qwen3RotaryEmbedding(cfg)
    hidden, k0, v0 = block_inputs()
    cache = DynamicCache(config=cfg)
    cache.update(k0[None], v0[None], 0)
    traces = {}

    def hook(name):
        def f(mod, inp, out):
            traces[name] = (out[0] if isinstance(out, tuple) else out).detach().clone()
        return f

    layer.self_attn.register_forward_hook(hook("attn_o"))
    layer.self_attn.o_proj.register_forward_pre_hook(lambda m, a: traces.__setitem__("attn", a[0].detach().clone()))
    layer.mlp.down_proj.register_forward_pre_hook(lambda m, a: traces.__setitem__("m", a[0].detach().clone()))
    pos = torch.tensor([[200]])
    with torch.no_grad():
        cos, sin = rot(hidden[None, None], pos)
        out = layer(hidden[None, None], attention_mask=None, position_ids=pos, past_key_values=cache,
                    use_cache=True, position_embeddings=(cos, sin))
    out = out[0] if isinstance(out, tuple) else out
    kc, vc = cache.layers[0].keys, cache.layers[0].values
    assert kc.shape == (1, 8, 201, 128)
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        out=u16(out.reshape(-1)), k_slot=u16(kc[0, :, 200]), v_slot=u16(vc[0, :, 200]),
        attn=u16(traces["attn"].reshape(-1)), o=u16(traces["attn_o"].reshape(-1)), m=u16(traces["m"].reshape(-1)),
        hidden_sha=np.frombuffer(weights.tensor_sha256(hidden).encode(), dtype=np.uint8),
    )
    print("block written", out.reshape(-1)[:4])


def hf_greedy(model, prompt, n_new, topk=TOPK, full_logit_steps=(), decode_path=False):
    """Greedy decode with HF forward + DynamicCache (== generate(do_sample=False)).

    decode_path: feed the prompt one token at a time (HF's decode path for every
    position) instead of one prefill forward."""
    from transformers import DynamicCache

    ids = torch.tensor([prompt])
    cache = DynamicCache(config=model.config)
    out_ids, tk_ids, tk_vals, full = [], [], [], {}
    t0 = time.perf_counter()
    with torch.no_grad():
        if decode_path:
            for t in prompt:
                res = model(input_ids=torch.tensor([[t]]), past_key_values=cache, use_cache=True)
        else:
            res = model(input_ids=ids, past_key_values=cache, use_cache=True)
        t_prefill = time.perf_counter() - t0
        t1 = time.perf_counter()
        for step in range(n_new):
            lg = res.logits[0, -1].to(torch.float32)  # bf16 logits upcast (generation/utils.py:2894)
            nxt = int(torch.argmax(lg))                 # first max (generation/utils.py:2925)
            vals, idx = torch.sort(lg, descending=True, stable=True)
            tk_ids.append(idx[:topk].numpy().astype(np.int32))
            tk_vals.append(vals[:topk].numpy())
            if step in full_logit_steps:
                full[step] = u16(res.logits[0, -1])
            out_ids.append(nxt)
            if step + 1 < n_new:
                res = model(input_ids=torch.tensor([[nxt]]), past_key_values=cache, use_cache=True)
        t_decode = time.perf_counter() - t1
    return out_ids, np.stack(tk_ids), np.stack(tk_vals), full, t_prefill, t_decode


def write_greedy(model, name, prompt_len, n_new, full_steps=(), decode_path=False, norms="ones"):
    prompt = weights.random_prompt(prompt_len, seed=1)
    ids, tki, tkv, full, tp, td = hf_greedy(model, prompt, n_new, full_logit_steps=full_steps, decode_path=decode_path)
    margins = tkv[:, 0] - tkv[:, 1]
    arrays = dict(prompt=np.array(prompt, dtype=np.int32), ids=np.array(ids, dtype=np.int32),
                  topk_ids=tki, topk_vals=tkv.astype(np.float32), margins=margins.astype(np.float32))
    for s, v in full.items():
        arrays[f"logits_step{s}"] = v
    np.savez_compressed(os.path.join(HERE, f"greedy_{name}.npz"), **arrays)
    meta = {"prompt_len": prompt_len, "n_new": n_new, "hf_prefill_s": tp, "hf_decode_s": td,
            "prompt_path": "decode (one token at a time)" if decode_path else "prefill", "norms": norms,
            "min_margin": float(margins.min()), "n_zero_margin": int((margins == 0).sum()),
            "transformers": __import__("transformers").__version__, "torch": torch.__version__,
            "threads": torch.get_num_threads()}
    json.dump(meta, open(os.path.join(HERE, f"greedy_{name}.json"), "w"), indent=1)
    print(name, meta, ids[:16])


def main(argv):
    what = set(argv) or {"rope", "block", "c1"}
    torch.set_num_threads(os.cpu_count())
    if "rope" in what:
        write_rope()
    if what & {"blockg", "c1g", "c4g"}:
        sdg = weights.make_state_dict(seed=0, norms="random")
        gh = {k: weights.tensor_sha256(sdg[k]) for k in
              ["model.layers.0.input_layernorm.weight", "model.layers.13.self_attn.k_norm.weight",
               "model.layers.27.post_attention_layernorm.weight", "model.norm.weight"]}
        json.dump(gh, open(os.path.join(HERE, "weights_gamma_sha256.json"), "w"), indent=1)
        if "blockg" in what:
            write_block(sdg, "block_pos200_gamma")
        if what & {"c1g", "c4g"}:
            model = hf_model(sdg)
            if "c1g" in what:
                write_greedy(model, "c1g", 8, 32, full_steps=(0, 31), decode_path=True, norms="random")
            if "c4g" in what:
                write_greedy(model, "c4g", 64, 16, full_steps=(0,), norms="random")
            del model
    need_sd = what & {"block", "c1", "c3", "c4", "c5", "c1d"}
    if not need_sd:
        return
    t0 = time.perf_counter()
    sd = weights.make_state_dict(seed=0)
    print(f"weights generated in {time.perf_counter() - t0:.1f}s")
    hashes = {k: weights.tensor_sha256(sd[k]) for k in
              ["model.embed_tokens.weight", "model.layers.0.self_attn.q_proj.weight",
               "model.layers.27.mlp.down_proj.weight"]}
    json.dump(hashes, open(os.path.join(HERE, "weights_sha256.json"), "w"), indent=1)
    if "block" in what:
        write_block(sd)
    if what & {"c1", "c3", "c4", "c5", "c1d"}:
        model = hf_model(sd)
        if "c1" in what:
            write_greedy(model, "c1", 8, 32, full_steps=(0, 31))
        if "c1d" in what:
            write_greedy(model, "c1d", 8, 32, full_steps=(0, 15, 31), decode_path=True)
        if "c4" in what:
            write_greedy(model, "c4", 512, 128, full_steps=(0,))
        if "c3" in what:
            write_greedy(model, "c3", 16, 2048)
        if "c5" in what:
            write_greedy(model, "c5", 8192, 256)


if __name__ == "__main__":
    main(sys.argv[1:])
