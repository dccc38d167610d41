"""GPU parity against HF on the same path and with non-unit norm gammas.

* Decode path: HF's config-1 run with the prompt fed one token at a time through its KV
  cache (`greedy_c1d`), the path the megakernel decoder takes, compared per position:
  logits at steps 0, 15 and 31, teacher-forced ids at every step, free-running ids.
* Random gammas (`norms="random"`: every norm weight bf16(1 + 0.1 randn), distinct per
  layer and norm): the config-2 block, the decode-path greedy run and a 64-token prefill
  against HF fixtures made with those weights, so that a gamma that is dropped, swapped
  or taken from the wrong layer shows.
* Prefill logits: the 512-token prompt's last-row logits (from the prefill's final-norm
  output) against HF's config-4 fixture.

Logit bounds (measured, stated in parity_helpers): the north star's max-abs 2e-2 per
position is not reachable by any implementation whose fp32 dot products accumulate in a
different order from HF's oneDNN kernels; the numpy oracle itself lands at 0.047 max-abs
with 2-3% of logits past 2e-2 (tests/test_oracle.py), and HF's own prefill and decode
paths differ by 0.039 at the same position. The GPU bounds below are the oracle's.
"""

import numpy as np
import pytest
import torch

from conftest import load_npz
from megaqwen_amd import megakernel_decode as MK
from oracle import qwen3_oracle as O
from parity_helpers import (DECODE_PATH_FLOORS, LOGIT_FRAC_OVER_2E2, LOGIT_MAX_ABS, LOGIT_MEAN_ABS, TIE_TOL, f32,
                            hf_tie_set, logit_stats, ulp_close)

pytestmark = pytest.mark.gpu


def _decoder(w, max_seq=1024):
    return MK.MegakernelPrefillDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"],
                                       w["lm_head_weight"], w["cos_table"], w["sin_table"], 28, max_seq, 512)


def _decode_path(dec, fx, steps):
    """Prompt token by token, then HF's own ids (teacher-forced); returns ids and {step: logits}."""
    prompt, ids = fx["prompt"].tolist(), fx["ids"].tolist()
    dec.reset()
    for t in prompt[:-1]:
        dec.decode_step(t)
    got, full = [], {}
    for s, t in enumerate([prompt[-1]] + ids[:-1]):
        tok, lg = dec.decode_step_with_logits(t)
        got.append(tok)
        if s in steps:
            full[s] = lg.cpu().numpy()
    return got, full


def _free_running(dec, prompt, n):
    dec.reset()
    for t in prompt[:-1]:
        dec.decode_step(t)
    cur, out = prompt[-1], []
    for _ in range(n):
        cur = dec.decode_step(cur)
        out.append(cur)
    return out


def _check_ids(name, got, fx):
    hf = fx["ids"].tolist()
    exact = sum(a == b for a, b in zip(got, hf))
    for s, (g, r) in enumerate(zip(got, hf)):
        assert g == r or (fx["margins"][s] <= TIE_TOL and g in hf_tie_set(fx, s)), (name, s, g, r)
    return exact


@pytest.mark.parametrize("name,weights_kind,steps", [("c1d", "ones", (0, 15, 31)), ("c1g", "random", (0, 31))])
def test_decode_path_vs_hf_decode_path(gpu_weights, gpu_weights_gamma, name, weights_kind, steps):
    fx = load_npz(f"greedy_{name}.npz")
    w = gpu_weights if weights_kind == "ones" else gpu_weights_gamma
    dec = _decoder(w)
    got, full = _decode_path(dec, fx, steps)
    exact = _check_ids(name, got, fx)
    print(f"{name} decode path teacher-forced: {exact}/{len(got)} ids identical to HF")
    for s in steps:
        mx, mean, frac = logit_stats(full[s], O.u16_to_f32(fx[f"logits_step{s}"]))
        print(f"{name} step {s}: logits max-abs {mx:.4f} mean-abs {mean:.5f} frac > 2e-2 {frac:.4f}")
        assert mx <= LOGIT_MAX_ABS and mean <= LOGIT_MEAN_ABS and frac <= LOGIT_FRAC_OVER_2E2
    free = _free_running(dec, fx["prompt"].tolist(), len(got))
    hf = fx["ids"].tolist()
    same_prefix = next((i for i, (a, b) in enumerate(zip(free, hf)) if a != b), len(hf))
    print(f"{name} decode path free-running: identical for {same_prefix}/{len(hf)} tokens")
    floor = DECODE_PATH_FLOORS[name]
    assert exact >= floor["teacher_forced"] and same_prefix >= floor["free_running"]


def test_gamma_block_vs_hf(gpu_weights_gamma):
    """Config 2's block with random gammas (input, q/k and post-attention norms) against
    HF: the same bar as the unit-gamma block test."""
    from make_golden import block_inputs

    hidden, k0, v0 = block_inputs()
    fx = load_npz("block_pos200_gamma.npz")
    layer0 = gpu_weights_gamma["layer_weights"][:11]
    k = torch.zeros(1, 8, 256, 128, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    k[0, :, :200] = k0.cuda()
    v[0, :, :200] = v0.cuda()
    out = MK.decode_layer(hidden.cuda(), layer0, gpu_weights_gamma["cos_table"], gpu_weights_gamma["sin_table"], k, v,
                          200)
    ok, dmax, frac = ulp_close(f32(out), O.u16_to_f32(fx["out"]), max_ulps=2, max_frac=0.4, floor=2.0 ** -6)
    print(f"gamma block out vs HF: max {dmax:.4g} frac {frac:.3f}")
    assert ok and dmax <= 2e-2
    okk, _, fk = ulp_close(f32(k[0, :, 200]), O.u16_to_f32(fx["k_slot"]).reshape(8, 128), max_ulps=1, max_frac=0.05)
    okv, _, fv = ulp_close(f32(v[0, :, 200]), O.u16_to_f32(fx["v_slot"]).reshape(8, 128), max_ulps=1, max_frac=0.05)
    print(f"gamma k slot mismatch frac {fk:.4f}, v slot {fv:.4f}")
    assert okk and okv


def _prefill_logits(dec, w):
    """Tied-LM-head logits of the prefill's final-norm output (bf16 row), fp32 accumulate,
    rounded to bf16 like HF's logits."""
    y = dec.final_normed_state().float()
    return O.bf16r((w["lm_head_weight"].float() @ y).cpu().numpy())


@pytest.mark.parametrize("name,weights_kind", [("c4", "ones"), ("c4g", "random")])
def test_prefill_last_row_logits_vs_hf(gpu_weights, gpu_weights_gamma, name, weights_kind):
    """The prompt through the MFMA prefill: first token and last-row logits against HF's
    prefill path, then teacher-forced decode steps."""
    fx = load_npz(f"greedy_{name}.npz")
    w = gpu_weights if weights_kind == "ones" else gpu_weights_gamma
    dec = _decoder(w)
    prompt, hf = fx["prompt"].tolist(), fx["ids"].tolist()
    first = dec.prefill_step(torch.tensor(prompt, dtype=torch.int32))
    lg = _prefill_logits(dec, w)
    mx, mean, frac = logit_stats(lg, O.u16_to_f32(fx["logits_step0"]))
    print(f"{name} prefill logits: max-abs {mx:.4f} mean-abs {mean:.5f} frac > 2e-2 {frac:.4f}")
    assert mx <= LOGIT_MAX_ABS and mean <= LOGIT_MEAN_ABS and frac <= LOGIT_FRAC_OVER_2E2
    got = [first]
    n = min(len(hf), 16)
    for s in range(1, n):
        got.append(dec.decode_step(hf[s - 1]))
    exact = _check_ids(name, got, {k: fx[k] for k in fx.files} | {"ids": fx["ids"][:n]})
    print(f"{name} prefill + decode teacher-forced: {exact}/{n} identical to HF")
