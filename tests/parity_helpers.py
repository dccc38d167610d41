"""Shared tolerances and comparison helpers of the GPU parity tests.

Tolerances: bf16 values within the stated ulps; logits max-abs <= LOGIT_MAX_ABS (4 bf16
ulps at |logit| in [2, 4)), mean-abs <= LOGIT_MEAN_ABS and at most LOGIT_FRAC_OVER_2E2 of
them further than 2e-2 from HF's; greedy ids exact outside HF's own near-ties, with the
measured exact-match counts as floors. The north star's 2e-2 max-abs is not reachable by
an implementation whose fp32 dot products accumulate in another order than HF's oneDNN
kernels: single-ulp flips compound through 28 layers of bf16 rounding. The numpy oracle
lands at max-abs 0.047 and 2-3% past 2e-2 against HF's decode path (tests/test_oracle.py);
HF's own prefill and decode paths differ by 0.039 at the same position; the GPU measures
0.039-0.051 and 1.6-2.9%.
"""

import numpy as np
import torch

from oracle import qwen3_oracle as O

LOGIT_MAX_ABS = 0.0625
LOGIT_MEAN_ABS = 0.01
# Share of logits further than the north star's 2e-2 from HF's (the oracle: 2-3%).
LOGIT_FRAC_OVER_2E2 = 0.05

# Exact-match regression floors: the counts this build measures against HF's fixtures
# (every id that differs is one of HF's near-ties within TIE_TOL; c1d's step 1 is an exact
# tie, margin 0). A one-token regression fails them. They depend on the fp32 accumulation
# order of the kernels: a change of that order re-measures them, with the reason stated.
DECODE_PATH_FLOORS = {
    "c1d": {"teacher_forced": 31, "free_running": 1},
    "c1g": {"teacher_forced": 31, "free_running": 26},
}
# Re-measured when the decode kernel's residual-norm sums of squares moved from 32
# per-workgroup sums to two per-wave half sums (the matvec sums kept their order): c3
# 1986 -> 1988, c4 117 -> 118, c5 242 -> 247; c1 unchanged. c5 247 -> 249 when prompts
# longer than 1024 tokens moved to the flash-form prefill attention (its softmax sums and
# P.V accumulate in another order).
EXACT_FLOORS = {
    "c1_teacher_forced": 32, "c1_free_running": 32,
    "c3_teacher_forced": 1988,
    "c4_teacher_forced": 118, "c4_free_running": 7,
    "c5_teacher_forced": 249,
}


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t):
    return O.u16_to_f32(u16(t))


def logit_stats(a, b):
    """(max-abs, mean-abs, share of |a - b| > 2e-2) of two logit vectors."""
    d = np.abs(np.asarray(a, np.float32) - np.asarray(b, np.float32))
    return float(d.max()), float(d.mean()), float((d > 2e-2).mean())


def ulp_close(a, b, max_ulps=1, max_frac=0.05, floor=2.0 ** -8):
    """bf16 arrays a, b (fp32-held) differ by <= max_ulps bf16 ulps of max(|b|, floor-scale),
    in <= max_frac of the elements. The floor covers values that cancel to near
    zero (e.g. h + o), whose absolute error is set by the operands' ulps."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    ulp = np.maximum(np.abs(b), 1e-30).view(np.uint32) & 0x7F800000
    ulp = np.maximum((ulp.view(np.float32) * 2.0 ** -7).astype(np.float32), floor)
    d = np.abs(a - b)
    return bool(np.all(d <= max_ulps * ulp) and (d > 0).mean() <= max_frac), float(d.max()), float((d > 0).mean())


# Near-tie tolerance for argmax comparisons: two candidates whose bf16 logits
# differ by less than this are a tie under the logit tolerance.
TIE_TOL = LOGIT_MAX_ABS


def hf_tie_set(fx, step):
    vals, ids = fx["topk_vals"][step], fx["topk_ids"][step]
    return set(ids[vals >= vals[0] - TIE_TOL].tolist())
