"""GPU parity tests of the decode megakernel, called through the C ABI.

Checks against the HF fixtures (tests/golden) and the numpy oracle on the
same seeded inputs. Tolerances: bf16 values within the stated ulps; logits
max-abs <= LOGIT_MAX_ABS and mean-abs <= LOGIT_MEAN_ABS (HF's own decode-path
vs prefill-path logits differ by max-abs 0.041); greedy ids exact.
"""

import numpy as np
import pytest
import torch

from conftest import load_npz
from megaqwen_amd import megakernel_decode as MK
from megaqwen_amd import rope, weights
from oracle import qwen3_oracle as O
from parity_helpers import EXACT_FLOORS, LOGIT_MAX_ABS, LOGIT_MEAN_ABS, TIE_TOL, f32, hf_tie_set, ulp_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer0(gpu_weights):
    return gpu_weights["layer_weights"][:11]


def run_block_gpu(layer0, gpu_weights, hidden_u16, kc, vc, pos):
    """kc, vc: float32 [8, max_seq, 128] (bf16 values) -> (out, k slot, v slot, caches after)."""
    dev = "cuda"
    h = torch.from_numpy(hidden_u16.view(np.int16)).view(torch.bfloat16).to(dev)
    k = torch.from_numpy(O.f32_to_u16(kc).view(np.int16)).view(torch.bfloat16).to(dev).unsqueeze(0).contiguous()
    v = torch.from_numpy(O.f32_to_u16(vc).view(np.int16)).view(torch.bfloat16).to(dev).unsqueeze(0).contiguous()
    out = MK.decode_layer(h, layer0, gpu_weights["cos_table"], gpu_weights["sin_table"], k, v, pos)
    return f32(out), f32(k[0]), f32(v[0])


def oracle_block(state_dict, hidden_u16, kc, vc, pos):
    flat = weights.layer_weights_flat(state_dict, 1)
    lw = O.LayerWeights([O.u16_to_f32(weights.bf16_to_u16(t)) for t in flat])
    cos, sin = rope.rope_tables(kc.shape[1])
    kc2, vc2 = kc.copy(), vc.copy()
    out = O.decoder_layer(lw, O.u16_to_f32(hidden_u16)[None], np.array([pos]),
                          O.u16_to_f32(weights.bf16_to_u16(cos)), O.u16_to_f32(weights.bf16_to_u16(sin)), kc2, vc2)
    return out[0], kc2, vc2


def test_block_config2_matches_hf(gpu_weights, layer0, state_dict):
    """Config 2: one decoder block at position 200 on N(0,1) hidden and KV[0..199]."""
    from make_golden import block_inputs

    hidden, k0, v0 = block_inputs()
    fx = load_npz("block_pos200.npz")
    kc = np.zeros((8, 256, 128), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :200] = O.u16_to_f32(weights.bf16_to_u16(k0))
    vc[:, :200] = O.u16_to_f32(weights.bf16_to_u16(v0))
    out, kg, vg = run_block_gpu(layer0, gpu_weights, weights.bf16_to_u16(hidden), kc, vc, 200)
    # 1-ulp flips from fp32 accumulation order compound through the block: the
    # oracle itself differs from HF in 21% of the outputs (all within 1 ulp).
    # Outputs h1 + d that cancel towards 0 keep the operands' ulp (~2^-6 for
    # residual-stream values in [2, 4)), hence the floor.
    ok, dmax, frac = ulp_close(out, O.u16_to_f32(fx["out"]), max_ulps=2, max_frac=0.4, floor=2.0 ** -6)
    ref, _, _ = oracle_block(state_dict, weights.bf16_to_u16(hidden), kc, vc, 200)
    _, omax, ofrac = ulp_close(out, ref, max_ulps=2, max_frac=0.4)
    print(f"block out vs HF: max {dmax:.4g} frac {frac:.3f}; vs oracle: max {omax:.4g} frac {ofrac:.3f}")
    assert ok and dmax <= 2e-2
    okk, _, fk = ulp_close(kg[:, 200], O.u16_to_f32(fx["k_slot"]).reshape(8, 128), max_ulps=1, max_frac=0.05)
    okv, _, fv = ulp_close(vg[:, 200], O.u16_to_f32(fx["v_slot"]).reshape(8, 128), max_ulps=1, max_frac=0.05)
    print(f"k slot mismatch frac {fk:.4f}, v slot {fv:.4f}")
    assert okk and okv
    # only slot 200 changed
    assert np.array_equal(kg[:, :200], kc[:, :200]) and np.array_equal(kg[:, 201:], kc[:, 201:])
    assert np.array_equal(vg[:, :200], vc[:, :200]) and np.array_equal(vg[:, 201:], vc[:, 201:])


@pytest.mark.parametrize("pos", [0, 1, 31, 32, 33, 200, 255, 256, 257, 511, 512, 1023, 1024, 2047, 4097, 8191, 8192, 8447,
                                 12000, 16383])
def test_block_attention_splits_vs_oracle(gpu_weights, layer0, state_dict, pos):
    """Split-K attention over every split count, and past 8192 positions the two LDS
    passes per workgroup: random N(0,1) cache, query at `pos`. Positions up to 255 run the
    kernel instance without split code (255: one full 256-row LDS pass), 256 on the other."""
    print(f"block pos {pos}", flush=True)
    g = torch.Generator().manual_seed(100 + pos)
    max_seq = 16384
    hidden = torch.randn(1024, generator=g).to(torch.bfloat16)
    kc = np.zeros((8, max_seq, 128), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :pos] = torch.randn(8, pos, 128, generator=g).to(torch.bfloat16).float().numpy()
    vc[:, :pos] = torch.randn(8, pos, 128, generator=g).to(torch.bfloat16).float().numpy()
    hu = weights.bf16_to_u16(hidden)
    out, kg, vg = run_block_gpu(layer0, gpu_weights, hu, kc, vc, pos)
    ref, kr, vr = oracle_block(state_dict, hu, kc, vc, pos)
    ok, dmax, frac = ulp_close(out, ref, max_ulps=2, max_frac=0.4, floor=2.0 ** -6)
    print(f"pos {pos}: out max {dmax:.4g} frac {frac:.3f}")
    assert ok
    # k goes through a 1024-term dot, QK-norm and RoPE: 1-ulp flips only
    okk, kmax, kfrac = ulp_close(kg[:, pos], kr[:, pos], 1, 0.3)
    okv, vmax, vfrac = ulp_close(vg[:, pos], vr[:, pos], 1, 0.3)
    print(f"pos {pos}: k slot frac {kfrac:.3f}, v slot frac {vfrac:.3f}")
    assert okk and okv


@pytest.fixture(scope="module")
def decoder(gpu_weights):
    w = gpu_weights
    return MK.MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["lm_head_weight"],
                                w["cos_table"], w["sin_table"], 28, 2048)


def test_greedy_config1_teacher_forced_vs_hf(decoder):
    """Config 1 on HF's own token stream: the GPU argmax equals HF's id at every
    step whose HF top-2 margin exceeds TIE_TOL, lies in HF's tie set otherwise,
    and full logits at the first and last step are within tolerance."""
    fx = load_npz("greedy_c1.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    n = len(hf_ids)
    decoder.reset()
    for t in prompt[:-1]:
        decoder.decode_step(t)
    stream = [prompt[-1]] + hf_ids[:-1]
    exact = 0
    for step in range(n):
        nxt, lg = decoder.decode_step_with_logits(stream[step])
        lg = lg.cpu().numpy()
        assert nxt == int(np.argmax(lg))
        if step in (0, n - 1):
            d = np.abs(lg - O.u16_to_f32(fx[f"logits_step{step}"]))
            print(f"step {step}: logits max-abs {d.max():.4g} mean {d.mean():.4g}")
            assert d.max() <= LOGIT_MAX_ABS and d.mean() <= LOGIT_MEAN_ABS
        if fx["margins"][step] > TIE_TOL:
            assert nxt == hf_ids[step], (step, nxt, hf_ids[step])
        else:
            assert nxt in hf_tie_set(fx, step), (step, nxt)
        exact += nxt == hf_ids[step]
    print(f"teacher-forced: {exact}/{n} ids identical to HF")
    assert exact >= EXACT_FLOORS["c1_teacher_forced"]


def test_greedy_config1_free_running(decoder):
    """Free-running greedy from the 8-token prompt against HF's config-1 run: identical
    for the measured floor of tokens (all 32), and in any case up to HF's first near-tie."""
    fx = load_npz("greedy_c1.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    decoder.reset()
    for t in prompt[:-1]:
        decoder.decode_step(t)
    cur, ids = prompt[-1], []
    for _ in range(len(hf_ids)):
        cur = decoder.decode_step(cur)
        ids.append(cur)
    print("gpu", ids)
    print("hf ", hf_ids)
    first_tie = next((i for i, m in enumerate(fx["margins"]) if m <= TIE_TOL), len(hf_ids))
    match = next((i for i, (a, b) in enumerate(zip(ids, hf_ids)) if a != b), len(hf_ids))
    print(f"free-running: identical for {match}/{len(hf_ids)} tokens; first HF near-tie at step {first_tie}")
    assert ids[:first_tie] == hf_ids[:first_tie]
    assert match >= EXACT_FLOORS["c1_free_running"]


def test_decode_is_bitwise_repeatable(decoder):
    """Same inputs -> identical tokens, logits and KV cache (exchange protocol determinism)."""
    fx = load_npz("greedy_c1.npz")
    prompt = fx["prompt"].tolist()
    outs = []
    for _ in range(2):
        decoder.reset()
        for t in prompt[:-1]:
            decoder.decode_step(t)
        tok, lg = decoder.decode_step_with_logits(prompt[-1])
        outs.append((tok, lg.clone(), decoder.get_k_cache()[:, :, :8].clone(), decoder.get_v_cache()[:, :, :8].clone()))
    assert outs[0][0] == outs[1][0]
    for a, b in zip(outs[0][1:], outs[1][1:]):
        assert torch.equal(a, b)


def test_decode_vs_oracle_teacher_forced(decoder, oracle_model):
    """Per-step logits of the GPU decoder vs the oracle on the same token stream."""
    fx = load_npz("greedy_c1.npz")
    stream = fx["prompt"].tolist() + fx["ids"].tolist()[:8]
    decoder.reset()
    oracle_model.reset()
    for i, t in enumerate(stream):
        tok, lg = decoder.decode_step_with_logits(t)
        otok, olg = oracle_model.decode_step(t)
        d = np.abs(lg.cpu().numpy() - olg)
        assert d.max() <= LOGIT_MAX_ABS and d.mean() <= LOGIT_MEAN_ABS, (i, d.max(), d.mean())
        top2 = np.sort(olg)[-2:]
        if top2[1] - top2[0] > 2 * LOGIT_MAX_ABS:
            assert tok == otok, i


def test_hidden_and_normalized_outputs(decoder, oracle_model):
    """hidden_buffer / g_normalized keep the reference's output contract (fused_decode_ldg.cu:688-722)."""
    decoder.reset()
    oracle_model.reset()
    tok = decoder.decode_step(1234)
    h, y = oracle_model.forward([1234], 0)
    gh = f32(decoder.hidden_state())
    # after 28 layers of independent bf16 rounding the states drift element-wise;
    # compare as vectors
    rel = np.linalg.norm(gh - h[0]) / np.linalg.norm(h[0])
    print(f"final hidden vs oracle: relative L2 {rel:.4g}")
    assert rel <= 2e-2
    assert np.max(np.abs(decoder.normalized_state().cpu().numpy() - y[0])) <= 0.1
    assert 0 <= tok < 151936


def test_watchdog_never_fires_and_position_cap(decoder):
    decoder.reset()
    decoder.set_position(2047)
    tok = decoder.decode_step(5)
    assert tok >= 0
    with pytest.raises(RuntimeError):
        decoder.decode_step(tok)
    decoder.reset()


def test_config3_2048_steps_teacher_forced_vs_hf(gpu_weights):
    """Config 3: 16-token prompt, then 2048 greedy decode steps on HF's own token
    stream (positions up to 2062); ids equal HF's where HF's top-2 margin exceeds
    TIE_TOL and lie in HF's tie set otherwise."""
    fx = load_npz("greedy_c3.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    w = gpu_weights
    dec = MK.MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["lm_head_weight"],
                               w["cos_table"], w["sin_table"], 28, 2048 + 16)
    for t in prompt[:-1]:
        dec.decode_step(t)
    stream = [prompt[-1]] + hf_ids[:-1]
    exact = 0
    for step, t in enumerate(stream):
        g = dec.decode_step(t)
        if fx["margins"][step] > TIE_TOL:
            assert g == hf_ids[step], (step, g, hf_ids[step])
        else:
            assert g in hf_tie_set(fx, step), (step, g)
        exact += g == hf_ids[step]
    print(f"config 3 teacher-forced: {exact}/{len(hf_ids)} ids identical to HF")
    assert exact >= EXACT_FLOORS["c3_teacher_forced"]
