"""GPU tests of the boundary's further entry points, called through the C ABI:

* the chat module's binding (`decode_ldg` / `decode_ldg_with_logits` with the reference's
  chat.py:192-316 argument lists) on config 1 against the HF fixture;
* device-resident generation (`mq_decode_step_device`), direct and as replayed HIP
  graphs, against the host-driven loop, across the 256-position instance boundary;
* the cooperative launch against the ordinary one (identical bits);
* recovery after a kernel-reported error: negative token -> MegakernelError ->
  workspace reset -> the next step matches an error-free run, at the same position;
* the fused-prefill decoder names routed to the MFMA prefill.
"""

import numpy as np
import pytest
import torch

from conftest import load_npz
from megaqwen_amd import _abi
from megaqwen_amd import chat_abi
from megaqwen_amd import megakernel_decode as MK
from parity_helpers import TIE_TOL, hf_tie_set

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def decoder(gpu_weights):
    w = gpu_weights
    return MK.MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["lm_head_weight"],
                                w["cos_table"], w["sin_table"], 28, 2048)


def test_chat_binding_config1_vs_hf(gpu_weights):
    """A caller written against chat.py (MegakernelChat.generate, chat.py:466-574): weights
    as 11 per-layer lists, the prompt fed through decode_ldg one position at a time with
    the reference's scratch tensors, then greedy decoding; ids against HF's config-1
    fixture (ties within TIE_TOL accepted), logits of the last step via
    decode_ldg_with_logits."""
    w = gpu_weights
    fx = load_npz("greedy_c1.npz")
    prompt, hf_ids = fx["prompt"].tolist(), fx["ids"].tolist()
    kernel = chat_abi.compile_kernel(chat_abi.select_optimal_kernel_variant(len(hf_ids), len(prompt)))
    lw = w["layer_weights"]
    kernel.init_ldg_layer_weights(*[[lw[11 * i + f] for i in range(28)] for f in range(11)])
    kernel.init_ldg_embed_weight(w["embed_weight"])
    dev, S = "cuda", chat_abi.MAX_SEQ_LEN
    k_cache = torch.zeros(28, 8, S, 128, dtype=torch.bfloat16, device=dev)
    v_cache = torch.zeros_like(k_cache)
    f32 = dict(dtype=torch.float32, device=dev)
    scratch = [torch.zeros(1024, dtype=torch.bfloat16, device=dev), torch.zeros(1024, **f32),
               torch.zeros(1024, **f32), torch.zeros(2048, **f32), torch.zeros(1024, **f32), torch.zeros(1024, **f32),
               torch.zeros(2048, **f32), torch.zeros(3072, **f32), torch.zeros(1024, **f32), torch.zeros(1184, **f32),
               torch.zeros(1184, dtype=torch.int32, device=dev)]
    cos, sin = chat_abi.precompute_rope_freqs(128, S, 1e6, dev)

    def step(tok, pos, logits=False):
        fn = kernel.decode_ldg_with_logits if logits else kernel.decode_ldg
        return fn(tok, w["final_norm_weight"], w["embed_weight"], cos, sin, k_cache, v_cache, *scratch, 28, pos,
                  pos + 1, S)

    for pos, t in enumerate(prompt[:-1]):
        step(t, pos)
    stream = [prompt[-1]] + hf_ids[:-1]
    got = []
    for i, t in enumerate(stream):
        pos = len(prompt) - 1 + i
        if i == len(stream) - 1:
            tok, lg = step(t, pos, logits=True)
            assert tok == int(torch.argmax(lg))
        else:
            tok = step(t, pos)
        got.append(tok)
    exact = sum(a == b for a, b in zip(got, hf_ids))
    print(f"chat binding teacher-forced: {exact}/{len(hf_ids)} identical to HF")
    for s, (g, r) in enumerate(zip(got, hf_ids)):
        assert g == r or (fx["margins"][s] <= TIE_TOL and g in hf_tie_set(fx, s)), (s, g, r)
    # the binding writes the final hidden state and final-norm output like the reference
    assert torch.count_nonzero(scratch[0]) > 0 and torch.count_nonzero(scratch[8]) > 0


def _host_loop(dec, prompt, n):
    dec.reset()
    for t in prompt[:-1]:
        dec.decode_step_async(t)
    cur, out = prompt[-1], []
    for _ in range(n):
        cur = dec.decode_step(cur)
        out.append(cur)
    return out


@pytest.mark.parametrize("use_graph", [False, True])
def test_device_resident_generation_matches_host_loop(decoder, use_graph):
    """Tokens fed back on the device (each launch reads token, position and epoch from the
    step the previous launch advanced) equal the host loop's, over chunks that cross the
    256-position instance boundary; with HIP graphs every chunk is a replay, the same
    graph replays several times with host reads and eager launches in between, and every
    replay is checked against the eager result."""
    prompt = [11, 22, 33, 44, 55, 66, 77, 88]
    n = 300
    want = _host_loop(decoder, prompt, n)
    for rep in range(2):
        decoder.reset()
        for t in prompt[:-1]:
            decoder.decode_step_async(t)
        got = decoder.generate_device(prompt[-1], n, use_graph=use_graph, chunk=48)
        print(f"graph={use_graph} rep {rep}: {sum(a == b for a, b in zip(got, want))}/{n} equal", flush=True)
        assert got == want
        assert decoder.position() == len(prompt) - 1 + n
        # eager work between replays, then the host loop again
        assert _host_loop(decoder, prompt, 8) == want[:8]


def test_device_resident_stop_token(decoder):
    prompt = [5, 6, 7]
    want = _host_loop(decoder, prompt, 40)
    stop = want[20]
    first = want.index(stop)
    decoder.reset()
    for t in prompt[:-1]:
        decoder.decode_step_async(t)
    got = decoder.generate_device(prompt[-1], 40, chunk=16, stop_tokens=[stop])
    assert got == want[:first]
    assert decoder.position() == len(prompt) - 1 + first + 1


def test_cooperative_launch_is_bitwise_identical(decoder):
    L = _abi.lib()
    outs = []
    for mode in (0, 1, 0):
        prev = L.mq_set_launch_mode(mode)
        try:
            decoder.reset()
            for t in (1, 2, 3, 4):
                decoder.decode_step(t)
            tok, lg = decoder.decode_step_with_logits(5)
        finally:
            L.mq_set_launch_mode(prev)
        outs.append((tok, lg.clone(), decoder.get_k_cache()[:, :, :5].clone()))
    for o in outs[1:]:
        assert o[0] == outs[0][0] and torch.equal(o[1], outs[0][1]) and torch.equal(o[2], outs[0][2])


def test_recovery_after_reported_error(decoder):
    """The error word is preset from the host (as a failed wait would set it): the launch
    completes, reports a negative token, decode_step raises MegakernelError, resets the
    workspace and restores the position; the next step then equals an error-free run."""
    L = _abi.lib()
    prompt = [101, 202, 303, 404]
    decoder.reset()
    for t in prompt:
        decoder.decode_step(t)
    ref_tok, ref_lg = decoder.decode_step_with_logits(505)
    decoder.reset()
    for t in prompt:
        decoder.decode_step(t)
    assert L.mq_debug_set_error(torch.cuda.current_device(), 1) == _abi.MQ_OK
    with pytest.raises(_abi.MegakernelError):
        decoder.decode_step(505)
    assert decoder.position() == len(prompt)
    tok, lg = decoder.decode_step_with_logits(505)
    assert tok == ref_tok and torch.equal(lg, ref_lg)


def test_fused_prefill_names(gpu_weights):
    w = gpu_weights
    args = (w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["lm_head_weight"], w["cos_table"],
            w["sin_table"], 28, 256)
    fused = MK.MegakernelFusedPrefillDecoder(*args)
    plain = MK.MegakernelPrefillDecoder(*args, 64)
    assert fused.max_prefill_len_ == 64
    ids = list(range(1000, 1040))
    a = fused.prefill_step(ids)
    b = plain.prefill_step(ids)
    # launch_prefill_megakernel (fp32 scratch) against launch_prefill_float: the same token
    # and caches, bit for bit
    assert a == b and torch.equal(fused.get_k_cache()[:, :, :40], plain.get_k_cache()[:, :, :40])
    assert torch.equal(fused.get_v_cache()[:, :, :40], plain.get_v_cache()[:, :, :40])
    # its outputs as the reference's fused launcher writes them: final_hidden the final-norm
    # row as fp32, hidden_bf16_out the last row before the final norm
    assert fused.final_hidden_.dtype == torch.float32
    assert torch.equal(fused.final_hidden_, plain.final_hidden_.float())
    assert torch.equal(fused.final_normed_state(), plain.final_normed_state())
    assert torch.equal(fused.hidden_buffer_, plain.hidden_float_[39])
    with pytest.raises(RuntimeError):
        fused.prefill_step(list(range(65)))
    gen = MK.MegakernelFusedPrefillGenerator(weights_dict=w, max_seq_len=256)
    ids_out = gen.generate_ids(ids, max_new_tokens=4)
    assert ids_out[0] == a and len(ids_out) == 4


# ---------------------------------------------------------------- contexts past 4096 positions
LONG_P0 = 4088  # 16 steps from here cross 4096, where chunks take two LDS passes


@pytest.fixture(scope="module")
def long_decoder(gpu_weights):
    w = gpu_weights
    return MK.MegakernelDecoder(w["embed_weight"], w["layer_weights"], w["final_norm_weight"], w["lm_head_weight"],
                                w["cos_table"], w["sin_table"], 28, 4160)


def _fill_caches(dec, upto, seed):
    """Positions < upto of both caches hold N(0, 1) bf16 values (a pre-filled context)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    for c in (dec.get_k_cache(), dec.get_v_cache()):
        c.zero_()
        c[:, :, :upto] = torch.randn(c[:, :, :upto].shape, generator=g, device="cuda").to(torch.bfloat16)
    torch.cuda.synchronize()


def test_device_resident_generation_across_the_pipelined_instance(long_decoder):
    """Chunks of the device-resident loop before position 4096 run instance 1, later ones
    instance 2 (a chunk's LDS passes pipelined); tokens and both caches equal the host
    loop's (which picks the instance per step), directly and as graph replays."""
    dec = long_decoder
    assert _abi.decode_plan(4095)["instance"] == 1 and _abi.decode_plan(4096)["instance"] == 2
    n, tok = 16, 1234
    _fill_caches(dec, LONG_P0, 0)
    k0, v0 = dec.get_k_cache().clone(), dec.get_v_cache().clone()
    dec.set_position(LONG_P0)
    want, cur = [], tok
    for _ in range(n):
        cur = dec.decode_step(cur)
        want.append(cur)
    kw, vw = dec.get_k_cache().clone(), dec.get_v_cache().clone()
    for use_graph in (False, True, True):
        dec.get_k_cache().copy_(k0)
        dec.get_v_cache().copy_(v0)
        dec.set_position(LONG_P0)
        got = dec.generate_device(tok, n, use_graph=use_graph, chunk=4)
        print(f"graph={use_graph}: {sum(a == b for a, b in zip(got, want))}/{n} equal", flush=True)
        assert got == want
        assert torch.equal(dec.get_k_cache(), kw) and torch.equal(dec.get_v_cache(), vw)


def test_pipelined_instance_is_bitwise_identical(long_decoder):
    """Past 4096 positions instances 1 and 2 differ only in when a chunk's later LDS passes
    are copied: forced through mq_decode_step_device, both give the same tokens and caches."""
    dec = long_decoder
    n, tok, p0 = 8, 777, LONG_P0 + 12
    L = _abi.lib()
    outs = []
    for inst in (1, 2, 1):
        _fill_caches(dec, p0, 1)
        step, out_ids = dec._step_buffers(n)
        _abi.check(L.mq_decode_step_init(MK._ptr(step), tok, p0, n, MK._stream()), "mq_decode_step_init")
        for _ in range(n):
            dec._launch_device_step(out_ids.numel(), inst)
        ids = out_ids[:n].tolist()
        print(f"instance {inst}: {ids}", flush=True)
        assert min(ids) >= 0
        outs.append((ids, dec.get_k_cache().clone(), dec.get_v_cache().clone()))
    for ids, kc, vc in outs[1:]:
        assert ids == outs[0][0]
        assert torch.equal(kc, outs[0][1]) and torch.equal(vc, outs[0][2])
