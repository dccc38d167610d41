"""GPU test of launch_ldg_decode_noalloc (the decode entry point that allocates nothing)
against launch_ldg_decode, both called through the C ABI on identical inputs: two calls in
a row, the second smaller (fewer layers, shorter context), each bit-identical to the
allocating entry point in token, final hidden state, final-norm output and K/V cache."""

import ctypes
import math

import numpy as np
import pytest
import torch

from megaqwen_amd import _abi
from megaqwen_amd import megakernel_decode as MK

pytestmark = pytest.mark.gpu


def _run(entry, w, d_layers, n_layers, kc, vc, token, pos, max_seq):
    dev = "cuda"
    out = torch.full((1,), -7, dtype=torch.int32, device=dev)
    hidden = torch.zeros(1024, dtype=torch.bfloat16, device=dev)
    normed = torch.zeros(1024, dtype=torch.float32, device=dev)
    k, v = kc.clone(), vc.clone()
    L = _abi.lib()
    stream = torch.cuda.current_stream().cuda_stream
    common = (w["embed_weight"].data_ptr(), d_layers.data_ptr(), w["final_norm_weight"].data_ptr(),
              w["lm_head_weight"].data_ptr(), w["cos_table"].data_ptr(), w["sin_table"].data_ptr(), k.data_ptr(),
              v.data_ptr(), hidden.data_ptr())
    scale = 1.0 / math.sqrt(128)
    if entry == "noalloc":
        st = L.launch_ldg_decode_noalloc(token, out.data_ptr(), *common, normed.data_ptr(), n_layers, pos, pos + 1,
                                         max_seq, scale, stream)
    else:
        st = L.launch_ldg_decode(token, out.data_ptr(), *common, *([None] * 7), normed.data_ptr(), None, None,
                                 n_layers, pos, pos + 1, max_seq, scale, stream)
    assert st == _abi.MQ_OK
    torch.cuda.synchronize()
    return int(out.item()), hidden, normed, k, v


@pytest.mark.parametrize("order", ["first", "repeat"])
def test_noalloc_matches_allocating_entry(gpu_weights, order):
    w = gpu_weights
    max_seq = 512
    g = torch.Generator().manual_seed(77)
    kc = torch.randn(28, 8, max_seq, 128, generator=g).to(torch.bfloat16).cuda()
    vc = torch.randn(28, 8, max_seq, 128, generator=g).to(torch.bfloat16).cuda()
    # second call smaller: 2 layers and a 41-position context after 28 layers and 301
    for n_layers, pos, token in ((28, 300, 4321), (2, 40, 987)):
        d_layers = MK.make_layer_struct_array(w["layer_weights"][:11 * n_layers], n_layers)
        ref = _run("alloc", w, d_layers, n_layers, kc[:n_layers].contiguous(), vc[:n_layers].contiguous(), token,
                   pos, max_seq)
        got = _run("noalloc", w, d_layers, n_layers, kc[:n_layers].contiguous(), vc[:n_layers].contiguous(), token,
                   pos, max_seq)
        print(f"{order}: layers {n_layers} pos {pos}: token {got[0]} (allocating entry {ref[0]})", flush=True)
        assert got[0] == ref[0] and got[0] >= 0
        for a, b in zip(got[1:], ref[1:]):
            assert torch.equal(a, b)


def test_noalloc_rejects_sizes_past_its_limit():
    L = _abi.lib()
    args = [1, 1] + [1] * 9 + [1, 28, 16384, 16385, 20000, 0.088, None]
    assert L.launch_ldg_decode_noalloc(*args) == _abi.MQ_ERR_ARG
    args = [1, 1] + [1] * 9 + [1, 33, 0, 1, 16, 0.088, None]
    assert L.launch_ldg_decode_noalloc(*args) == _abi.MQ_ERR_ARG
