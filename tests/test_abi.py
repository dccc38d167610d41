"""CPU tests of the C ABI boundary: the library loads, exports every entry
point include/*.h declares, and rejects invalid arguments on the host before
touching the GPU (no compute calls here)."""

import ctypes
import glob
import os
import re
import subprocess

import pytest

from megaqwen_amd import _abi

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("launch_ldg_decode", "launch_ldg_decode_with_logits", "mq_decode_layer", "launch_prefill_float",
              "launch_prefill_megakernel", "mq_reset_workspace", "mq_strerror"):
        assert n in names, n


def test_library_exports_every_declared_symbol():
    assert os.path.exists(_abi.LIB_PATH), "build the library first (python -m megaqwen_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s+(\w+)$", out, flags=re.M))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_python_binding_covers_header():
    assert set(_abi.SIGNATURES) == set(declared_functions())


def test_layer_struct_layout():
    assert ctypes.sizeof(_abi.LDGLayerWeights) == 11 * 8
    assert _abi.LDGLayerWeights.down_proj_weight.offset == 80


def _decode_args(**over):
    a = dict(token=1, out=1, embed=1, layers=1, norm=1, lm=1, cos=1, sin=1, k=1, v=1, hidden=1,
             num_layers=28, position=0, cache_len=1, max_seq_len=16, scale=0.088)
    a.update(over)
    return [a["token"], a["out"], a["embed"], a["layers"], a["norm"], a["lm"], a["cos"], a["sin"], a["k"], a["v"],
            a["hidden"]] + [None] * 10 + [a["num_layers"], a["position"], a["cache_len"], a["max_seq_len"],
                                           a["scale"], None]


@pytest.mark.parametrize("bad", [
    dict(out=None), dict(embed=None), dict(layers=None), dict(k=None),
    dict(num_layers=0), dict(num_layers=33), dict(position=-1), dict(position=16), dict(cache_len=5),
    dict(token=-1), dict(token=151936), dict(scale=0.0), dict(scale=float("nan")), dict(max_seq_len=0),
])
def test_decode_rejects_invalid_arguments(bad):
    st = _abi.lib().launch_ldg_decode(*_decode_args(**bad))
    assert st == _abi.MQ_ERR_ARG


def test_decode_layer_rejects_invalid_arguments():
    L = _abi.lib()
    assert L.mq_decode_layer(None, 1, 1, 1, 1, 1, 1, 0, 16, 0.088, None) == _abi.MQ_ERR_ARG
    assert L.mq_decode_layer(1, 1, 1, 1, 1, 1, 1, 16, 16, 0.088, None) == _abi.MQ_ERR_ARG
    assert L.mq_decode_layer(1, 1, 1, 1, 1, 1, 1, 0, 16, -1.0, None) == _abi.MQ_ERR_ARG


def _prefill_args(**over):
    layers = (_abi.LDGLayerWeights * 2)()
    for i in range(2):
        for name in _abi.LAYER_FIELDS:
            setattr(layers[i], name, 1)
    if over.pop("null_layer_field", False):
        layers[1].down_proj_weight = None
    a = dict(ids=1, out=1, seq_len=8, embed=1, layers=ctypes.addressof(layers), norm=1, lm=1, cos=1, sin=1, k=1,
             v=1, num_layers=2, max_seq_len=16, scale=0.088)
    a.update(over)
    scratch = [1] * 17
    scratch[1] = scratch[7] = scratch[12] = None  # unused by this build
    if a.pop("null_scratch", False):
        scratch[3] = None  # q_proj
    if a.pop("null_partials", False):
        scratch[10] = None  # up_out: holds partial sums in this build
    return layers, [a["ids"], a["out"], a["seq_len"], a["embed"], a["layers"], a["norm"], a["lm"], a["cos"],
                    a["sin"], a["k"], a["v"]] + scratch + [a["num_layers"], a["max_seq_len"], a["scale"], None]


@pytest.mark.parametrize("bad", [
    dict(ids=None), dict(out=None), dict(layers=None), dict(k=None), dict(null_scratch=True), dict(null_partials=True),
    dict(null_layer_field=True), dict(seq_len=0), dict(seq_len=17), dict(num_layers=0), dict(num_layers=33),
    dict(max_seq_len=0), dict(scale=0.0), dict(scale=float("inf")),
])
def test_prefill_rejects_invalid_arguments(bad):
    keep, args = _prefill_args(**bad)
    assert _abi.lib().launch_prefill_float(*args) == _abi.MQ_ERR_ARG
    del keep


@pytest.mark.parametrize("bad", [
    dict(ids=None), dict(out=None), dict(layers=None), dict(k=None), dict(null_scratch=True),
    dict(null_layer_field=True), dict(seq_len=0), dict(seq_len=17), dict(num_layers=0), dict(num_layers=33),
    dict(max_seq_len=0), dict(scale=0.0), dict(scale=float("nan")),
])
def test_prefill_megakernel_rejects_invalid_arguments(bad):
    """launch_prefill_megakernel (the reference's fused-prefill launcher,
    csrc/megakernel/fused_prefill_megakernel.cu:938-1016): every scratch argument is required
    (the activations and partial sums are carved from them); bad sizes and pointers are refused
    on the host before any HIP call."""
    keep, args = _prefill_args(**{k: v for k, v in bad.items() if k != "null_scratch"})
    scratch = [1] * 12  # hidden .. block_max_idxs
    if bad.get("null_scratch"):
        scratch[7] = None  # mlp_intermediate
    margs = args[:11] + scratch + args[28:]
    assert _abi.lib().launch_prefill_megakernel(*margs) == _abi.MQ_ERR_ARG
    del keep


def test_strerror():
    L = _abi.lib()
    assert L.mq_strerror(0) == b"ok"
    assert b"argument" in L.mq_strerror(-1)
    with pytest.raises(_abi.MegakernelError):
        _abi.check(-1, "x")


def test_decode_plan_bounds_every_position():
    """The kernel's attention split, queried through the C ABI for every accepted position:
    at most 16 chunks (one per group-A workgroup of an XCD), each within four LDS passes of
    256 rows, none empty, together covering the context (the kernel also proves this at
    compile time with a static_assert)."""
    L = _abi.lib()
    inst, ns, ch, npass = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    refs = [ctypes.byref(x) for x in (inst, ns, ch, npass)]
    for p in range(16384):
        assert L.mq_decode_plan(p, *refs) == _abi.MQ_OK
        n = p + 1
        assert inst.value == (0 if p < 256 else 2 if npass.value > 1 else 1)
        assert 1 <= ns.value <= 16 and ch.value <= 1024 and npass.value == (ch.value + 255) // 256 <= 4
        assert ch.value * ns.value >= n and (ns.value - 1) * ch.value < n
        if p < 256:
            assert ns.value == 1 and ch.value == n
    for p in (-1, 16384):
        assert L.mq_decode_plan(p, *refs) == _abi.MQ_ERR_ARG
    assert _abi.decode_plan(8447) == {"instance": 2, "nsplit": 16, "chunk": 528, "npass": 3}
    assert _abi.decode_plan(16383) == {"instance": 2, "nsplit": 16, "chunk": 1024, "npass": 4}
    assert _abi.decode_plan(4095) == {"instance": 1, "nsplit": 16, "chunk": 256, "npass": 1}
    assert _abi.decode_plan(4096) == {"instance": 2, "nsplit": 16, "chunk": 257, "npass": 2}
    assert _abi.decode_plan(1023) == {"instance": 1, "nsplit": 4, "chunk": 256, "npass": 1}


def test_device_step_entries_reject_invalid_arguments():
    L = _abi.lib()
    assert L.mq_decode_step_init(None, 1, 0, 4, None) == _abi.MQ_ERR_ARG
    assert L.mq_decode_step_init(1, -1, 0, 4, None) == _abi.MQ_ERR_ARG
    assert L.mq_decode_step_init(1, 151936, 0, 4, None) == _abi.MQ_ERR_ARG
    assert L.mq_decode_step_init(1, 1, 16384, 4, None) == _abi.MQ_ERR_ARG
    assert L.mq_decode_step_init(1, 1, 0, 0, None) == _abi.MQ_ERR_ARG
    good = dict(step=1, out=1, cap=4, split=0)

    def args(**o):
        a = dict(good, **o)
        return [a["step"], a["out"], a["cap"], a["split"]] + [1] * 10 + [28, 16, 0.088, None]
    for bad in (dict(step=None), dict(out=None), dict(cap=0), dict(split=3), dict(split=-1)):
        assert L.mq_decode_step_device(*args(**bad)) == _abi.MQ_ERR_ARG
    a = args()
    a[14] = 0  # num_layers
    assert L.mq_decode_step_device(*a) == _abi.MQ_ERR_ARG
    assert ctypes.sizeof(_abi.MqDecodeStep) == 16


def test_launch_mode_switch():
    L = _abi.lib()
    prev = L.mq_set_launch_mode(1)
    assert L.mq_set_launch_mode(prev) == 1
    assert L.mq_set_launch_mode(prev) == prev


def test_noalloc_entry_rejects_sizes_past_its_limit():
    L = _abi.lib()
    base = [1, 1] + [1] * 9 + [1]
    assert L.launch_ldg_decode_noalloc(*(base + [28, 16384, 16385, 20000, 0.088, None])) == _abi.MQ_ERR_ARG
    assert L.launch_ldg_decode_noalloc(*(base + [33, 0, 1, 16, 0.088, None])) == _abi.MQ_ERR_ARG
    assert L.launch_ldg_decode_noalloc(*([1, None] + [1] * 9 + [1, 28, 0, 1, 16, 0.088, None])) == _abi.MQ_ERR_ARG


def test_decode_variant_rejects_invalid_arguments():
    """mq_decode_variant: an unknown variant, the unsplit variant from position 256 on, and the
    decode entry's own argument checks give MQ_ERR_ARG before any HIP call."""
    L = _abi.lib()
    good = [1, 1, None] + [1] * 10 + [28, 300, 301, 512, 0.088, None]  # token .. stream, position 300

    def call(variant, **kw):
        a = list(good)
        if "position" in kw:
            a[14], a[15] = kw["position"], kw["position"] + 1
        if "out" in kw:
            a[1] = kw["out"]
        return L.mq_decode_variant(variant, *a)

    assert call(3) == _abi.MQ_ERR_ARG and call(-1) == _abi.MQ_ERR_ARG
    assert call(_abi.MQ_VARIANT_UNSPLIT, position=256) == _abi.MQ_ERR_ARG
    assert call(_abi.MQ_VARIANT_UNSPLIT, position=300) == _abi.MQ_ERR_ARG
    assert call(_abi.MQ_VARIANT_SPLIT, position=16384) == _abi.MQ_ERR_ARG
    for v in (_abi.MQ_VARIANT_BASELINE, _abi.MQ_VARIANT_UNSPLIT, _abi.MQ_VARIANT_SPLIT):
        assert call(v, position=10, out=None) == _abi.MQ_ERR_ARG
