"""CPU contract tests of the public API.

The first group restates every assertion of the reference's own contract
suite (tests/test_api.py:13-109): fallback parity, dispatch reasons,
validation messages, custom scale, cross-attention. The second group covers
the dispatch rules that need a GPU tensor, through the pure rule function with
the facts a gfx950 device would report.
"""

from __future__ import annotations

import pytest
import torch

from triton_flash_attention import (
    DispatchDecision,
    TritonAttention,
    explain_dispatch,
    scaled_dot_product_attention,
)
from triton_flash_attention import attention as attn


# --- reference contract (tests/test_api.py) --------------------------------
@pytest.mark.parametrize("causal", [False, True])
def test_auto_dispatch_fallback_matches_reference(causal: bool) -> None:
    torch.manual_seed(0)
    query = torch.randn(2, 4, 7, 32, requires_grad=True)
    key = torch.randn(2, 4, 7, 32, requires_grad=True)
    value = torch.randn(2, 4, 7, 32, requires_grad=True)
    grad = torch.randn_like(query)
    actual = scaled_dot_product_attention(query, key, value, is_causal=causal)
    expected = torch.nn.functional.scaled_dot_product_attention(query, key, value, is_causal=causal)
    torch.testing.assert_close(actual, expected)
    actual_grads = torch.autograd.grad(actual, (query, key, value), grad)
    expected_grads = torch.autograd.grad(expected, (query, key, value), grad)
    for a, e in zip(actual_grads, expected_grads):
        torch.testing.assert_close(a, e)


def test_gqa_fallback_matches_reference() -> None:
    torch.manual_seed(1)
    query = torch.randn(1, 4, 11, 32)
    key = torch.randn(1, 2, 11, 32)
    value = torch.randn(1, 2, 11, 32)
    actual = scaled_dot_product_attention(query, key, value, is_causal=True, enable_gqa=True)
    expected = torch.nn.functional.scaled_dot_product_attention(
        query, key, value, is_causal=True, enable_gqa=True)
    torch.testing.assert_close(actual, expected)


def test_dispatch_explains_ineligible_device() -> None:
    tensor = torch.randn(1, 1, 3, 32)
    assert explain_dispatch(tensor, tensor, tensor) == DispatchDecision(
        backend="torch", reason="the Triton kernel requires a CUDA tensor")


def test_strict_triton_backend_rejects_ineligible_device() -> None:
    tensor = torch.randn(1, 1, 3, 32)
    with pytest.raises(RuntimeError, match="requires a CUDA tensor"):
        scaled_dot_product_attention(tensor, tensor, tensor, backend="triton")


@pytest.mark.parametrize(
    ("mutator", "message"),
    [
        (lambda q, k, v: (q.squeeze(0), k, v), "query must have shape"),
        (lambda q, k, v: (q[..., :-1], k, v), "query and key head dimensions"),
        (lambda q, k, v: (q, k[:, :1], v[:, :1]), "pass enable_gqa=True"),
    ],
)
def test_validation_errors(mutator, message: str) -> None:
    query = torch.randn(1, 2, 5, 32)
    key = torch.randn_like(query)
    value = torch.randn_like(query)
    query, key, value = mutator(query, key, value)
    with pytest.raises(ValueError, match=message):
        scaled_dot_product_attention(query, key, value)


def test_explicit_torch_backend_honors_custom_scale() -> None:
    query = torch.randn(1, 2, 5, 32)
    key = torch.randn_like(query)
    value = torch.randn_like(query)
    actual = scaled_dot_product_attention(query, key, value, scale=0.25, backend="torch")
    expected = torch.nn.functional.scaled_dot_product_attention(query, key, value, scale=0.25)
    torch.testing.assert_close(actual, expected)


def test_cross_attention_fallback_matches_reference() -> None:
    # The reference's cross-attention test inputs (N_q 3, N_kv 5, value head
    # size 16 != 32): on the CPU the device rule sends them to SDPA; neither the
    # lengths nor the head sizes decide any more.
    query = torch.randn(1, 2, 3, 32)
    key = torch.randn(1, 2, 5, 32)
    value = torch.randn(1, 2, 5, 16)
    decision = explain_dispatch(query, key, value)
    assert decision.backend == "torch"
    assert "CUDA tensor" in decision.reason
    actual = scaled_dot_product_attention(query, key, value)
    expected = torch.nn.functional.scaled_dot_product_attention(query, key, value)
    torch.testing.assert_close(actual, expected)
    # a value head size the kernels cannot hold is rejected before the device rule
    value = torch.randn(1, 2, 5, 160)
    decision = explain_dispatch(query, key, value)
    assert decision.backend == "torch" and "equal query/key and value head sizes" in decision.reason


# --- remaining validation and argument checks (ref attention.py:584-626, 806-815)
def test_argument_type_checks() -> None:
    t = torch.randn(1, 1, 4, 32)
    with pytest.raises(ValueError, match="backend must be one of"):
        scaled_dot_product_attention(t, t, t, backend="cuda")
    with pytest.raises(TypeError, match="is_causal must be a bool"):
        scaled_dot_product_attention(t, t, t, is_causal=1)
    with pytest.raises(TypeError, match="enable_gqa must be a bool"):
        scaled_dot_product_attention(t, t, t, enable_gqa=None)
    for bad in (float("nan"), float("inf"), "0.5"):
        with pytest.raises(ValueError, match="scale must be a finite real number"):
            scaled_dot_product_attention(t, t, t, scale=bad)
    with pytest.raises(TypeError, match="query must be a torch.Tensor"):
        scaled_dot_product_attention([1.0], t, t)


def test_validation_order_and_messages() -> None:
    q = torch.randn(1, 4, 6, 32)
    with pytest.raises(ValueError, match="dimensions must all be greater than zero"):
        explain_dispatch(q[:, :, :0], q, q)
    with pytest.raises(ValueError, match="same dtype"):
        explain_dispatch(q, q.double(), q)
    with pytest.raises(ValueError, match="batch dimensions must match"):
        explain_dispatch(q, torch.randn(2, 4, 6, 32), torch.randn(2, 4, 6, 32))
    with pytest.raises(ValueError, match="key and value batch, head, and sequence"):
        explain_dispatch(q, q, torch.randn(1, 4, 7, 32))
    with pytest.raises(ValueError, match="must be divisible"):
        explain_dispatch(q, torch.randn(1, 3, 6, 32), torch.randn(1, 3, 6, 32), enable_gqa=True)


def test_exports_match_reference_surface() -> None:
    import triton_flash_attention as pkg

    assert set(pkg.__all__) == {"DispatchDecision", "TritonAttention", "explain_dispatch",
                                "scaled_dot_product_attention"}
    assert issubclass(TritonAttention, torch.autograd.Function)
    with pytest.raises(Exception):
        DispatchDecision("torch", "x").backend = "triton"  # frozen dataclass


# --- dispatch rules that need a GPU tensor, via the pure rule function --------
def _facts(**overrides):
    base = dict(q_len=128, kv_len=128, head_dim=64, value_head_dim=64, device_type="cuda",
                dtype=torch.float16, arch="gfx950:sramecc+:xnack-", library_error=None)
    base.update(overrides)
    return attn._DispatchFacts(**base)


def test_rule_eligible_gfx950_selects_custom_kernel() -> None:
    d = attn._decide(_facts())
    assert d.backend == "triton"
    for D in (32, 64, 128):
        assert attn._decide(_facts(head_dim=D, value_head_dim=D)).backend == "triton"
    # bfloat16 is served too (the reference sends it to SDPA, attention.py:653-656)
    d = attn._decide(_facts(dtype=torch.bfloat16))
    assert d.backend == "triton" and "bfloat16" in d.reason
    # A value head size other than D is served when both are supported sizes
    # (the reference sends D_v != D to SDPA, attention.py:643-646).
    for D, Dv in ((64, 32), (32, 128), (128, 64)):
        d = attn._decide(_facts(head_dim=D, value_head_dim=Dv))
        assert d.backend == "triton" and f"zero-padded to {max(D, Dv)}" in d.reason
    # Other head sizes up to 128 run zero-padded to the next kernel size (the
    # reference sends every size but 32, 64, 128 to SDPA, attention.py:657-661).
    for D, Dv, width in ((16, 16, 32), (40, 40, 64), (96, 96, 128), (80, 48, 128), (1, 33, 64)):
        d = attn._decide(_facts(head_dim=D, value_head_dim=Dv))
        assert d.backend == "triton" and f"zero-padded to {width}" in d.reason, (D, Dv)
    assert "zero-padded" not in attn._decide(_facts()).reason
    # Cross-attention is served too (the reference sends it to SDPA, attention.py:639-642).
    for q_len, kv_len in ((128, 64), (3, 5000)):
        d = attn._decide(_facts(q_len=q_len, kv_len=kv_len))
        assert d.backend == "triton" and "cross-attention" in d.reason
    assert "self-attention" in attn._decide(_facts()).reason


@pytest.mark.parametrize(
    ("overrides", "reason"),
    [
        (dict(value_head_dim=160), "equal query/key and value head sizes"),
        (dict(value_head_dim=16, head_dim=256), "two different ones of at most 128"),
        (dict(device_type="cpu"), "requires a CUDA tensor"),
        (dict(dtype=torch.float32), "supports float16 and bfloat16"),
        (dict(dtype=torch.float64), "supports float16 and bfloat16"),
        (dict(head_dim=160, value_head_dim=160), "head_dim must be one of (32, 64, 128)"),
        (dict(head_dim=256, value_head_dim=256), "zero-padded to one of them"),
        (dict(q_len=1 << 24, kv_len=1 << 24), "too long"),
        (dict(q_len=1 << 24), "too long"),
        (dict(kv_len=1 << 24), "too long"),
        (dict(arch="gfx942:sramecc+:xnack-"), "gfx950"),
        (dict(arch=""), "gfx950"),
        (dict(library_error="missing"), "kernel library is not available"),
    ],
)
def test_rule_fallback_reasons(overrides, reason) -> None:
    d = attn._decide(_facts(**overrides))
    assert d.backend == "torch"
    assert reason in d.reason


def test_rule_order_is_first_match() -> None:
    # value head size wins over everything, dtype wins over head_dim and arch
    d = attn._decide(_facts(kv_len=3, value_head_dim=200, dtype=torch.float32, arch="gfx90a"))
    assert "value head sizes" in d.reason
    d = attn._decide(_facts(dtype=torch.float32, head_dim=192, value_head_dim=192, arch="gfx90a"))
    assert "float16" in d.reason


def test_missing_library_raises_in_auto_mode(monkeypatch) -> None:
    """A gfx950 device without its kernel library is a broken install: auto
    mode raises instead of silently running PyTorch."""
    calls = {}

    def fake_dispatch(q, k, v):
        calls["n"] = calls.get("n", 0) + 1
        return DispatchDecision("torch", f"{attn._REASON_LIBRARY}: not built")

    monkeypatch.setattr(attn, "_dispatch", fake_dispatch)
    t = torch.randn(1, 1, 4, 32)
    with pytest.raises(RuntimeError, match="kernel library is not available"):
        attn.scaled_dot_product_attention(t, t, t)
    # backend="torch" never consults the library
    out = attn.scaled_dot_product_attention(t, t, t, backend="torch")
    torch.testing.assert_close(out, torch.nn.functional.scaled_dot_product_attention(t, t, t))
    assert calls["n"] == 1
