"""CPU tests of the chat module's decode-kernel selection policy (the reference's
tests/test_chat_kernel_selection.py:15-37, with MI355X's kernel instances in place of
its NVIDIA source variants) and of its binding's host-side checks."""

import pytest

from megaqwen_amd import _abi
from megaqwen_amd.chat_abi import (
    AUTO_KERNEL_VARIANT,
    SHORT_CONTEXT_POSITIONS,
    SUPPORTED_DECODE_KERNEL_VARIANTS,
    compile_kernel,
    select_optimal_kernel_variant,
)


def test_short_generation_prefers_unsplit():
    assert select_optimal_kernel_variant(1) == "unsplit"
    assert select_optimal_kernel_variant(SHORT_CONTEXT_POSITIONS) == "unsplit"
    assert select_optimal_kernel_variant(SHORT_CONTEXT_POSITIONS - 16, prompt_len=16) == "unsplit"


def test_long_generation_prefers_split():
    assert select_optimal_kernel_variant(SHORT_CONTEXT_POSITIONS + 1) == "split"
    assert select_optimal_kernel_variant(SHORT_CONTEXT_POSITIONS - 15, prompt_len=16) == "split"
    assert select_optimal_kernel_variant(500) == "split"


def test_kernel_selection_rejects_non_positive_decode_length():
    with pytest.raises(ValueError, match="max_new_tokens must be positive"):
        select_optimal_kernel_variant(0)
    with pytest.raises(ValueError, match="max_new_tokens must be positive"):
        select_optimal_kernel_variant(-1)


def test_supported_kernel_variants_include_auto_and_instances():
    assert AUTO_KERNEL_VARIANT == "auto"
    assert "baseline" in SUPPORTED_DECODE_KERNEL_VARIANTS
    assert "unsplit" in SUPPORTED_DECODE_KERNEL_VARIANTS
    assert "split" in SUPPORTED_DECODE_KERNEL_VARIANTS


def test_policy_agrees_with_the_kernels_own_plan():
    """The policy's threshold is the kernel's: the last position of an "unsplit"
    generation runs the instance 0 plan with one attention chunk."""
    for n_new in range(1, 600, 7):
        last = n_new - 1
        plan = _abi.decode_plan(last)
        assert (select_optimal_kernel_variant(n_new) == "unsplit") == (plan["instance"] == 0)


def test_unknown_variant_rejected():
    with pytest.raises(ValueError, match="unsupported kernel variant"):
        compile_kernel("fastmath")


def test_decode_ldg_needs_init():
    import torch

    k = compile_kernel("baseline")
    t = torch.zeros(1)
    with pytest.raises(RuntimeError, match="init_ldg_layer_weights"):
        k.decode_ldg(1, t, t, t, t, t, t, t, t, t, t, t, t, t, t, t, t, t, 28, 0, 1, 512)


def test_unsplit_variant_refuses_long_contexts_before_launching():
    """The variant fixes the kernel instance of every decode_ldg launch: "unsplit" (instance 0,
    contexts of at most 256 positions) raises for a step at position 256 or later, on the
    host, before any launch."""
    import torch

    k = compile_kernel("unsplit")
    k._d_layer_weights, k._embed, k._num_layers = torch.zeros(1), torch.zeros(1), 28
    t = torch.zeros(1)
    with pytest.raises(ValueError, match="'unsplit' kernel variant serves positions below 256"):
        k.decode_ldg(1, t, t, t, t, t, t, t, t, t, t, t, t, t, t, t, t, t, 28, SHORT_CONTEXT_POSITIONS,
                     SHORT_CONTEXT_POSITIONS + 1, 512)
