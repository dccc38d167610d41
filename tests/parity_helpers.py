"""Shared tolerances and comparison helpers of the GPU parity tests.

Tolerances: bf16 values within the stated ulps; logits max-abs <= LOGIT_MAX_ABS
and mean-abs <= LOGIT_MEAN_ABS (HF's own decode-path vs prefill-path logits
differ by max-abs 0.041); greedy ids exact outside HF's own near-ties.
"""

import numpy as np
import torch

from oracle import qwen3_oracle as O

LOGIT_MAX_ABS = 0.0625
LOGIT_MEAN_ABS = 0.01


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t):
    return O.u16_to_f32(u16(t))


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
