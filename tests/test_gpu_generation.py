"""GPU tests of the generation rows around the decode kernel, each against HF's fixtures:

* device-resident generation (token and position in device memory, HIP graph replays; the
  reference's idea at experimental/qwen_persistent_kernel.cu:1028-1033): config 1 and the
  random-gamma decode-path run free-running from their prompts, against HF's ids;
* a checkpoint written to disk (HF key names, safetensors, tied LM head) and read back by
  `load_qwen3_weights(dir)` (the reference's loader, csrc/megakernel/megakernel_decode.py:
  1077-1133, reads a downloaded one), driven through the kernels by the generator;
* the chat module's decode-kernel variants (chat.py:17-29, 59-64): each fixes the kernel
  instance of its decode_ldg launches, and all give the same tokens, logits and caches.
"""

import math

import pytest
import torch

from conftest import load_npz
from megaqwen_amd import _abi
from megaqwen_amd import chat_abi
from megaqwen_amd import megakernel_decode as MK
from parity_helpers import DECODE_PATH_FLOORS, EXACT_FLOORS, TIE_TOL

pytestmark = pytest.mark.gpu


def _decoder(w, max_seq=1024):
    return MK.MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["lm_head_weight"],
                                w["cos_table"], w["sin_table"], 28, max_seq)


def _same_prefix(a, b):
    return next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), min(len(a), len(b)))


def _device_run(dec, prompt, n, use_graph, chunk):
    dec.reset()
    for t in prompt[:-1]:
        dec.decode_step_async(t)
    return dec.generate_device(prompt[-1], n, use_graph=use_graph, chunk=chunk)


@pytest.mark.parametrize("use_graph,chunk", [(True, 8), (True, 32), (False, 32)])
def test_device_resident_config1_vs_hf(gpu_weights, use_graph, chunk):
    """Config 1 (8-token prompt, 32 greedy tokens) through the device-resident loop: with
    chunks of 8 the same captured graph replays four times (a host read between replays).
    The ids equal HF's for all 32 steps (the free-running floor), as the host loop's do."""
    fx = load_npz("greedy_c1.npz")
    prompt, hf = fx["prompt"].tolist(), fx["ids"].tolist()
    dec = _decoder(gpu_weights)
    got = _device_run(dec, prompt, len(hf), use_graph, chunk)
    n = _same_prefix(got, hf)
    first_tie = next((i for i, m in enumerate(fx["margins"]) if m <= TIE_TOL), len(hf))
    print(f"device-resident config 1 (graph={use_graph}, chunk {chunk}): identical to HF for {n}/{len(hf)}",
          flush=True)
    assert got[:first_tie] == hf[:first_tie]
    assert n >= EXACT_FLOORS["c1_free_running"]
    assert dec.position() == len(prompt) - 1 + len(hf)


def test_device_resident_random_gammas_vs_hf(gpu_weights_gamma):
    """HF's decode-path run with random norm gains (c1g) through the device-resident loop as
    graph replays: identical to HF for at least the free-running floor of the host loop."""
    fx = load_npz("greedy_c1g.npz")
    prompt, hf = fx["prompt"].tolist(), fx["ids"].tolist()
    dec = _decoder(gpu_weights_gamma)
    got = _device_run(dec, prompt, len(hf), True, 16)
    n = _same_prefix(got, hf)
    print(f"device-resident c1g: identical to HF for {n}/{len(hf)}", flush=True)
    assert n >= DECODE_PATH_FLOORS["c1g"]["free_running"]


def test_checkpoint_on_disk_through_the_kernels(state_dict, tmp_path):
    """The seeded weights written as an HF-format checkpoint directory (model.safetensors +
    config.json, no lm_head tensor), read back by load_qwen3_weights(dir) and run by the
    generator: config 1's 32 ids equal HF's, through the host loop and the device-resident
    loop."""
    fx = load_npz("greedy_c1.npz")
    prompt, hf = fx["prompt"].tolist(), fx["ids"].tolist()
    path = str(tmp_path / "qwen3-seeded")
    MK.save_qwen3_checkpoint(state_dict, path)
    print("checkpoint written", flush=True)
    gen = MK.MegakernelGenerator(model_name=path, max_seq_len=256)
    w = gen.weights
    assert w["config"]["tie_word_embeddings"] and w["lm_head_weight"] is w["embed_weight"]
    assert torch.equal(w["layer_weights"][6].cpu(), state_dict["model.layers.0.self_attn.o_proj.weight"])
    host = gen.generate_ids(prompt, max_new_tokens=len(hf), stop_tokens=[])
    dev = gen.generate_ids(prompt, max_new_tokens=len(hf), stop_tokens=[], device_loop=True)
    print(f"loaded checkpoint: host loop {_same_prefix(host, hf)}/{len(hf)}, device loop "
          f"{_same_prefix(dev, hf)}/{len(hf)} identical to HF", flush=True)
    assert _same_prefix(host, hf) >= EXACT_FLOORS["c1_free_running"]
    assert dev == host


def _chat_kernel(w, variant):
    k = chat_abi.compile_kernel(variant)
    lw = w["layer_weights"]
    k.init_ldg_layer_weights(*[[lw[11 * i + f] for i in range(28)] for f in range(11)])
    k.init_ldg_embed_weight(w["embed_weight"])
    return k


def _chat_run(kernel, w, tokens, p0, caches):
    """decode_ldg_with_logits over `tokens` from position p0 on the given caches (modified)."""
    k_cache, v_cache = caches
    S = k_cache.shape[2]
    dev = "cuda"
    f32 = dict(dtype=torch.float32, device=dev)
    scratch = [torch.zeros(1024, dtype=torch.bfloat16, device=dev), torch.zeros(1024, **f32),
               torch.zeros(1024, **f32), torch.zeros(2048, **f32), torch.zeros(1024, **f32), torch.zeros(1024, **f32),
               torch.zeros(2048, **f32), torch.zeros(3072, **f32), torch.zeros(1024, **f32), torch.zeros(1184, **f32),
               torch.zeros(1184, dtype=torch.int32, device=dev)]
    out, logits = [], []
    for i, t in enumerate(tokens):
        pos = p0 + i
        tok, lg = kernel.decode_ldg_with_logits(t, w["final_norm_weight"], w["lm_head_weight"], w["cos_table"],
                                                w["sin_table"], k_cache, v_cache, *scratch, 28, pos, pos + 1, S)
        out.append(tok)
        logits.append(lg)
    return out, torch.stack(logits), scratch[0].clone(), scratch[8].clone()


def _caches(S, fill, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.zeros(28, 8, S, 128, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    if fill:
        k[:, :, :fill] = torch.randn(28, 8, fill, 128, generator=g, device="cuda").to(torch.bfloat16)
        v[:, :, :fill] = torch.randn(28, 8, fill, 128, generator=g, device="cuda").to(torch.bfloat16)
    return k, v


@pytest.mark.parametrize("p0", [0, 120, 300])
def test_kernel_variants_select_the_instance_and_agree(gpu_weights, p0):
    """Each variant fixes the kernel instance of its launches: "split" runs instance 1 even at
    short contexts (one attention chunk, handed out to the XCD's other workgroups) and
    "unsplit" instance 0 (every group-A workgroup attends itself); "baseline" picks per step.
    From a pre-filled context at p0, 12 steps give bitwise-identical tokens, logits, final
    states and caches under every variant that serves p0; "unsplit" raises past 256."""
    w = gpu_weights
    toks = [(1000 + 37 * i) % 151936 for i in range(12)]
    S = 512
    runs = {}
    for variant in ("baseline", "split", "unsplit"):
        caches = _caches(S, p0, 5)
        kern = _chat_kernel(w, variant)
        if variant == "unsplit" and p0 + len(toks) - 1 >= chat_abi.SHORT_CONTEXT_POSITIONS:
            with pytest.raises(ValueError, match="unsplit"):
                _chat_run(kern, w, toks, p0, caches)
            continue
        ids, lg, hid, nrm = _chat_run(kern, w, toks, p0, caches)
        runs[variant] = (ids, lg, hid, nrm, caches[0][:, :, :p0 + len(toks)], caches[1][:, :, :p0 + len(toks)])
        print(f"p0 {p0} {variant}: {ids[:6]}...", flush=True)
    base = runs["baseline"]
    assert min(base[0]) >= 0
    for variant, r in runs.items():
        assert r[0] == base[0], variant
        for a, b in zip(r[1:], base[1:]):
            assert torch.equal(a, b), variant


def test_split_variant_runs_the_split_instance_at_short_contexts(gpu_weights):
    """The variant reaches the kernel: the C ABI call with MQ_VARIANT_SPLIT at position 10 is
    accepted, and MQ_VARIANT_UNSPLIT at position 256 is refused before any launch."""
    w = gpu_weights
    L = _abi.lib()
    d_layers = MK.make_layer_struct_array(w["layer_weights"], 28)
    k, v = _caches(512, 0, 1)
    out = torch.full((1,), -5, dtype=torch.int32, device="cuda")
    hidden = torch.zeros(1024, dtype=torch.bfloat16, device="cuda")
    common = [w["embed_weight"].data_ptr(), d_layers.data_ptr(), w["final_norm_weight"].data_ptr(),
              w["lm_head_weight"].data_ptr(), w["cos_table"].data_ptr(), w["sin_table"].data_ptr(), k.data_ptr(),
              v.data_ptr(), hidden.data_ptr(), None, 28]
    stream = torch.cuda.current_stream().cuda_stream
    scale = 1.0 / math.sqrt(128)
    assert L.mq_decode_variant(_abi.MQ_VARIANT_SPLIT, 42, out.data_ptr(), None, *common, 10, 11, 512, scale,
                               stream) == _abi.MQ_OK
    torch.cuda.synchronize()
    assert 0 <= int(out.item()) < 151936
    assert L.mq_decode_variant(_abi.MQ_VARIANT_UNSPLIT, 42, out.data_ptr(), None, *common, 256, 257, 512, scale,
                               stream) == _abi.MQ_ERR_ARG
