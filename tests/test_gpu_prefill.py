"""GPU parity tests of the prefill kernels (`launch_prefill_float`), called through
the C ABI via MegakernelPrefillDecoder.

Against the numpy oracle on small seeded models (ragged prompt lengths, a prompt
longer than one 512-key attention block) and against HF's config-4 fixture
(512-token prompt, 128 greedy steps) on the full model. Tolerances are those of
parity_helpers (bf16 ulps, logit max-abs, HF near-ties).
"""

import numpy as np
import pytest
import torch

from conftest import load_npz
from megaqwen_amd import _abi
from megaqwen_amd import megakernel_decode as MK
from megaqwen_amd import rope, weights
from oracle import qwen3_oracle as O
from parity_helpers import EXACT_FLOORS, LOGIT_MAX_ABS, TIE_TOL, f32, hf_tie_set, ulp_close

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def embed_gpu(state_dict):
    return state_dict["model.embed_tokens.weight"].cuda()


def small_pair(state_dict, embed_gpu, n_layers, max_seq):
    """(GPU prefill decoder, oracle) over the first n_layers seeded layers."""
    flat = weights.layer_weights_flat(state_dict, n_layers)
    cos, sin = rope.rope_tables(max_seq)
    norm = state_dict["model.norm.weight"]
    dec = MK.MegakernelPrefillDecoder(embed_gpu, [t.cuda() for t in flat], norm.cuda(), embed_gpu, cos.cuda(),
                                      sin.cuda(), n_layers, max_seq, max_prefill_len=max_seq)
    u = weights.bf16_to_u16
    orc = O.Qwen3Oracle(u(state_dict["model.embed_tokens.weight"]), [u(t) for t in flat], u(norm), u(cos), u(sin),
                        max_seq)
    return dec, orc


def prompt_ids(n, seed):
    return weights.random_prompt(n, seed=seed)


@pytest.mark.parametrize("S", [1, 37, 100, 130, 256, 300])
def test_prefill_vs_oracle_ragged(state_dict, embed_gpu, S):
    """2-layer model, prompt lengths that are not multiples of any tile: K/V slots,
    the residual stream, the final-norm row and the greedy token against the oracle.
    The lengths cover each short-prompt tile shape (up to 64, 128 and 256 tokens) and
    the S = 512 shapes with gate/up's warm-up row (257 to 384 tokens)."""
    print(f"prefill S={S}", flush=True)
    dec, orc = small_pair(state_dict, embed_gpu, 2, 320)
    ids = prompt_ids(S, seed=10 + S)
    tok = dec.prefill_step(ids)
    otok, olg = orc.prefill(ids)
    assert dec.position() == S
    kg, vg = f32(dec.get_k_cache()), f32(dec.get_v_cache())
    # layer 0: the inputs are identical, so only 1-ulp flips from fp32 accumulation order.
    # RoPE's difference of two products of magnitude up to ~4 can cancel towards 0, and
    # a 1-ulp flip of either product then moves the result by the products' ulp (2^-5).
    ok, dmax, frac = ulp_close(kg[0, :, :S], orc.k_cache[0, :, :S], max_ulps=1, max_frac=0.3, floor=2.0 ** -5)
    print(f"k layer 0: max {dmax:.3g} frac {frac:.3f}")
    assert ok
    ok, dmax, frac = ulp_close(vg[0, :, :S], orc.v_cache[0, :, :S], max_ulps=1, max_frac=0.05)
    print(f"v layer 0: max {dmax:.3g} frac {frac:.3f}")
    assert ok
    # layer 1 inherits layer 0's ulp flips: compare as vectors
    assert rel_l2(kg[1, :, :S], orc.k_cache[1, :, :S]) < 1e-2
    assert rel_l2(vg[1, :, :S], orc.v_cache[1, :, :S]) < 1e-2
    h, y = orc.forward(ids, 0)  # re-run to get the hidden states (same caches)
    hg = f32(dec.hidden_float_[:S])
    print(f"hidden rel L2 {rel_l2(hg, h):.3g}")
    assert rel_l2(hg, h) < 1e-2
    assert np.max(np.abs(f32(dec.final_hidden_) - y[-1])) <= 0.1
    # hidden_bf16_out receives a copy of final_hidden (the final-norm row), as in the reference
    # (csrc/megakernel/fused_prefill.cu:843-849)
    assert torch.equal(dec.hidden_buffer_, dec.final_hidden_)
    top2 = np.sort(olg)[-2:]
    if top2[1] - top2[0] > 2 * LOGIT_MAX_ABS:
        assert tok == otok
    # slots past the prompt stay untouched (zero after construction)
    assert not dec.get_k_cache()[:, :, S:].any() and not dec.get_v_cache()[:, :, S:].any()


def test_prefill_two_attention_blocks(state_dict, embed_gpu):
    """S = 600 > 512: rows past 512 take two key blocks (running-max rescale).
    The attention output itself is compared element-wise with the oracle's, the
    block output as a vector (its elements inherit flips through the MLP)."""
    S = 600
    print(f"prefill S={S}", flush=True)
    dec, orc = small_pair(state_dict, embed_gpu, 1, 640)
    ids = prompt_ids(S, seed=99)
    dec.prefill_step(ids)
    trace = {}
    kc, vc = np.zeros_like(orc.k_cache[0]), np.zeros_like(orc.v_cache[0])
    h = O.decoder_layer(orc.layers[0], orc.embed[ids], np.arange(S), orc.cos, orc.sin, kc, vc, trace=trace)
    att, oatt = f32(dec.attn_out_[:S]), trace["attn"]
    for lo, hi in ((0, 512), (512, S)):
        ok, dmax, frac = ulp_close(att[lo:hi], oatt[lo:hi], max_ulps=2, max_frac=0.1)
        print(f"attention rows {lo}..{hi - 1}: max {dmax:.3g} frac {frac:.3f} rel L2 {rel_l2(att[lo:hi], oatt[lo:hi]):.3g}")
        assert ok
    hg = f32(dec.hidden_float_[:S])
    print(f"1-layer output rel L2 {rel_l2(hg, h):.3g}")
    assert rel_l2(hg, h) < 5e-3


@pytest.mark.parametrize("S", [1100, 2100, 4200, 5400, 7200])
def test_prefill_long_tile_shapes_vs_oracle(state_dict, embed_gpu, S):
    """Prompts that take the larger GEMM tiles (q/k/v 128- and 256-row tiles, gate/up
    128 x 256 and 256 x 256, o_proj/down_proj 128 x 256 and 256 x 256) and the flash-form
    attention: the layer's K/V slots and attention output element-wise against the oracle,
    the layer output as a vector."""
    print(f"prefill S={S}", flush=True)
    dec, orc = small_pair(state_dict, embed_gpu, 1, S + 16)
    ids = prompt_ids(S, seed=7 + S)
    dec.prefill_step(ids)
    trace = {}
    kc, vc = np.zeros_like(orc.k_cache[0]), np.zeros_like(orc.v_cache[0])
    h = O.decoder_layer(orc.layers[0], orc.embed[ids], np.arange(S), orc.cos, orc.sin, kc, vc, trace=trace)
    kg, vg = f32(dec.get_k_cache()), f32(dec.get_v_cache())
    ok, dmax, frac = ulp_close(kg[0, :, :S], kc[:, :S], max_ulps=1, max_frac=0.3, floor=2.0 ** -5)
    print(f"k: max {dmax:.3g} frac {frac:.3f}")
    assert ok
    ok, dmax, frac = ulp_close(vg[0, :, :S], vc[:, :S], max_ulps=1, max_frac=0.05)
    print(f"v: max {dmax:.3g} frac {frac:.3f}")
    assert ok
    att, oatt = f32(dec.attn_out_[:S]), trace["attn"]
    ok, dmax, frac = ulp_close(att, oatt, max_ulps=2, max_frac=0.1)
    print(f"attention: max {dmax:.3g} frac {frac:.3f} rel L2 {rel_l2(att, oatt):.3g}")
    assert ok
    hg = f32(dec.hidden_float_[:S])
    print(f"1-layer output rel L2 {rel_l2(hg, h):.3g}")
    assert rel_l2(hg, h) < 5e-3


def test_prefill_matches_token_by_token_decode(state_dict, embed_gpu):
    """Prefill's K/V cache and next token agree with feeding the same prompt to the
    decode kernel one token at a time (two independent kernels, one model)."""
    fx = load_npz("greedy_c1.npz")
    prompt = fx["prompt"].tolist()
    dec, _ = small_pair(state_dict, embed_gpu, 4, 64)
    tok_p = dec.prefill_step(prompt)
    kp, vp = dec.get_k_cache().clone(), dec.get_v_cache().clone()
    dec.reset()
    for t in prompt[:-1]:
        dec.decode_step(t)
    tok_d, lg = dec.decode_step_with_logits(prompt[-1])
    n = len(prompt)
    assert rel_l2(f32(dec.get_k_cache()[:, :, :n]), f32(kp[:, :, :n])) < 1e-2
    assert rel_l2(f32(dec.get_v_cache()[:, :, :n]), f32(vp[:, :, :n])) < 1e-2
    top2 = np.sort(lg.cpu().numpy())[-2:]
    if top2[1] - top2[0] > 2 * LOGIT_MAX_ABS:
        assert tok_p == tok_d


def test_prefill_repeatable_and_rejects_bad_ids(state_dict, embed_gpu):
    """Identical prompts give bitwise-identical caches and tokens; an id outside the
    vocabulary is reported as an error, and the next prefill is unaffected."""
    dec, _ = small_pair(state_dict, embed_gpu, 2, 128)
    ids = prompt_ids(50, seed=5)
    outs = []
    for _ in range(2):
        dec.reset()
        outs.append((dec.prefill_step(ids), dec.get_k_cache().clone(), dec.get_v_cache().clone()))
    assert outs[0][0] == outs[1][0]
    assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][2], outs[1][2])
    with pytest.raises(_abi.MegakernelError):
        dec.prefill_step(ids[:10] + [151936] + ids[11:])
    dec.reset()
    assert dec.prefill_step(ids) == outs[0][0]
    with pytest.raises(RuntimeError):
        dec.prefill_step([])
    with pytest.raises(RuntimeError):
        dec.prefill_step(list(range(129)))


@pytest.fixture(scope="module")
def prefill_decoder(gpu_weights):
    w = gpu_weights
    return MK.MegakernelPrefillDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                       w["lm_head_weight"], w["cos_table"], w["sin_table"], 28, 1024, 512)


def test_config4_prefill_then_decode_vs_hf(prefill_decoder):
    """Config 4: 512-token prompt through the MFMA prefill, then 127 greedy decode
    steps on HF's own token stream; every id equals HF's where HF's top-2 margin
    exceeds TIE_TOL and lies in HF's tie set otherwise."""
    fx = load_npz("greedy_c4.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    dec = prefill_decoder
    dec.reset()
    print("config 4 prefill", flush=True)
    nxt = dec.prefill_step(torch.tensor(prompt, dtype=torch.int32))
    got = [nxt]
    for step in range(1, len(hf_ids)):
        got.append(dec.decode_step(hf_ids[step - 1]))
    exact = 0
    for step, (g, r) in enumerate(zip(got, hf_ids)):
        if fx["margins"][step] > TIE_TOL:
            assert g == r, (step, g, r)
        else:
            assert g in hf_tie_set(fx, step), (step, g)
        exact += g == r
    print(f"config 4 teacher-forced: {exact}/{len(hf_ids)} ids identical to HF")
    assert exact >= EXACT_FLOORS["c4_teacher_forced"]


def test_config4_free_running(prefill_decoder):
    """Free-running greedy after the 512-token prefill: identical to HF up to HF's
    first near-tie step."""
    fx = load_npz("greedy_c4.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    dec = prefill_decoder
    dec.reset()
    cur = dec.prefill_step(prompt)
    ids = [cur]
    for _ in range(len(hf_ids) - 1):
        cur = dec.decode_step(cur)
        ids.append(cur)
    first_tie = next((i for i, m in enumerate(fx["margins"]) if m <= TIE_TOL), len(hf_ids))
    match = next((i for i, (a, b) in enumerate(zip(ids, hf_ids)) if a != b), len(hf_ids))
    print(f"config 4 free-running: identical for {match}/{len(hf_ids)}; first HF near-tie at {first_tie}")
    assert ids[:first_tie] == hf_ids[:first_tie]
    assert match >= EXACT_FLOORS["c4_free_running"]


def test_config5_long_context_vs_hf(gpu_weights):
    """Config 5: an 8192-token prompt through the prefill kernels, then 256 greedy
    decode steps at positions 8192..8447 (every attention workgroup takes two LDS
    passes) on HF's own token stream; ids equal HF's where HF's top-2 margin exceeds
    TIE_TOL and lie in HF's tie set otherwise."""
    fx = load_npz("greedy_c5.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    w = gpu_weights
    dec = MK.MegakernelPrefillDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                      w["lm_head_weight"], w["cos_table"], w["sin_table"], 28, 8448, 8192)
    print("config 5 prefill", flush=True)
    got = [dec.prefill_step(prompt)]
    print("config 5 decode", flush=True)
    for step in range(1, len(hf_ids)):
        got.append(dec.decode_step(hf_ids[step - 1]))
    exact = 0
    for step, (g, r) in enumerate(zip(got, hf_ids)):
        if fx["margins"][step] > TIE_TOL:
            assert g == r, (step, g, r)
        else:
            assert g in hf_tie_set(fx, step), (step, g)
        exact += g == r
    print(f"config 5 teacher-forced: {exact}/{len(hf_ids)} ids identical to HF")
    assert exact >= EXACT_FLOORS["c5_teacher_forced"]
