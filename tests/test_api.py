"""CPU contract tests of the public API.

The first group restates every assertion of the reference's own contract
suite (tests/test_api.py:13-109): fallback parity, dispatch reasons,
validation messages, custom scale, cross-attention. The second group covers
the dispatch rules that need a GPU tensor, through the pure rule function with
the facts a gfx950 device would report.
"""

from __future__ import annotations

import warnings

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
    # The reference's test, verbatim (tests/test_api.py:100-109): on the CPU
    # cross-attention inputs fall back with the reference's first-rule reason.
    query = torch.randn(1, 2, 3, 32)
    key = torch.randn(1, 2, 5, 32)
    value = torch.randn(1, 2, 5, 16)
    decision = explain_dispatch(query, key, value)
    assert decision.backend == "torch"
    assert "self-attention" in decision.reason
    actual = scaled_dot_product_attention(query, key, value)
    expected = torch.nn.functional.scaled_dot_product_attention(query, key, value)
    torch.testing.assert_close(actual, expected)


def test_cross_attention_fallback_reason_names_the_deciding_rule() -> None:
    query = torch.randn(1, 2, 3, 32)
    key = torch.randn(1, 2, 5, 32)
    d = explain_dispatch(query, key, torch.randn(1, 2, 5, 16))
    assert d.reason.startswith("the custom kernel currently specializes in self-attention")
    assert "requires a CUDA tensor" in d.reason
    # a value head size the kernels cannot hold is rejected before the device rule
    d = explain_dispatch(query, key, torch.randn(1, 2, 5, 160))
    assert d.backend == "torch" and "self-attention" in d.reason
    assert "equal query/key and value head sizes" in d.reason
    with pytest.raises(RuntimeError, match="self-attention"):
        scaled_dot_product_attention(query, key, key, backend="triton")


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
    # ... and where it falls back, the reason starts with the reference's first rule
    for overrides in (dict(device_type="cpu"), dict(dtype=torch.float32), dict(arch="gfx942"),
                      dict(library_error="missing"), dict(value_head_dim=160)):
        d = attn._decide(_facts(q_len=3, kv_len=5, **overrides))
        assert d.backend == "torch"
        assert d.reason.startswith("the custom kernel currently specializes in self-attention")


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


def test_missing_library_falls_back_in_auto_mode(monkeypatch) -> None:
    """As in the reference (attention.py:829-839), auto mode never raises for
    an unavailable backend: a gfx950 device without its kernel library runs
    SDPA, with one RuntimeWarning per process; strict mode raises."""
    calls = {}

    def fake_dispatch(q, k, v):
        calls["n"] = calls.get("n", 0) + 1
        return DispatchDecision("torch", f"{attn._REASON_LIBRARY}: not built")

    monkeypatch.setattr(attn, "_dispatch", fake_dispatch)
    monkeypatch.setattr(attn, "_library_warned", False)
    t = torch.randn(1, 1, 4, 32)
    with pytest.warns(RuntimeWarning, match="kernel library is not available"):
        out = attn.scaled_dot_product_attention(t, t, t)
    torch.testing.assert_close(out, torch.nn.functional.scaled_dot_product_attention(t, t, t))
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # once per process
        attn.scaled_dot_product_attention(t, t, t)
    with pytest.raises(RuntimeError, match="kernel library is not available"):
        attn.scaled_dot_product_attention(t, t, t, backend="triton")
    # backend="torch" never consults the library
    out = attn.scaled_dot_product_attention(t, t, t, backend="torch")
    torch.testing.assert_close(out, torch.nn.functional.scaled_dot_product_attention(t, t, t))
    assert calls["n"] == 3


# --- every finite scale is served (ref attention.py:812-815, 844-845) ----------
def test_kernel_scale_modes() -> None:
    assert attn._kernel_scale(0.125) == (0.125, "plain")
    assert attn._kernel_scale(-0.5) == (0.5, "negate")
    for tiny in (0.0, -0.0, 1e-40, -1e-40, 1e-50):  # zero or subnormal in float32
        assert attn._kernel_scale(tiny) == (1.0, "zero"), tiny
    assert attn._kernel_scale(2.0 ** -126) == (2.0 ** -126, "plain")
    assert attn._kernel_scale(1e39) is None  # float32 overflow
    assert attn._kernel_scale(3e38) is None  # scale * log2(e) overflows float32


def test_kernel_scale_served_scales_pass_the_library_check() -> None:
    """Every kernel scale the Python layer sends passes the C ABI's scale check,
    and the library rejects what _kernel_scale maps away. A call that passes
    every check reaches the launch, which fails on a host without a GPU (the
    fake pointers are never touched); on a GPU host only the rejections run."""
    from triton_flash_attention import _lib

    ok, why = _lib.available()
    assert ok, why
    lib = _lib.load()
    P = 0x10000

    def rc(scale):
        return lib.fa_fwd(P, P, P, P, P, 1, 1, 1, 16, 32, scale, 0, None)

    for s in (0.0, -1.0, 1e-40, -1e-40, float("inf"), float("nan")):
        assert rc(s) == _lib.FA_ERR_BAD_SCALE, s
    if torch.cuda.is_available():
        return
    for s in (0.125, -0.5, 0.0, 1e-40, 2.0 ** -126, 1e30, -7.0):
        served = attn._kernel_scale(s)
        assert served is not None and served[0] > 0
        assert rc(served[0]) > 0, s  # reached the launch: a HIP error, not FA_ERR_BAD_SCALE


def test_scale_transforms_are_exact_in_fp64() -> None:
    """The score identity the negate and zero modes rest on, with the
    reference's rounding of the backward's scaled operands (attention.py:435,
    515: fp16(k * c), c = float32(scale / ln 2)), on fp16 inputs."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(3, 40, 64, generator=g).half()
    k = torch.randn(3, 50, 64, generator=g).half()
    for scale in (-0.125, -1.7, -3e-5):
        c = torch.tensor(scale * attn._LOG2E, dtype=torch.float32)
        cn = torch.tensor(-scale * attn._LOG2E, dtype=torch.float32)
        assert float(cn) == -float(c)
        s_ref = (q.double() @ k.double().transpose(1, 2)) * float(c)
        s_neg = ((-q).double() @ k.double().transpose(1, 2)) * float(cn)
        assert torch.equal(s_ref, s_neg)
        k_ref = (k.float() * c).half()
        k_neg = (k.float() * cn).half()
        assert torch.equal(k_ref, -k_neg)
    # with a subnormal scale every exp2 argument s * c - m rounds to -m in float32
    s = (q.float() @ k.float().transpose(1, 2))
    c = torch.tensor(1e-40 * attn._LOG2E, dtype=torch.float32)
    m = (s * c).amax(-1, keepdim=True)
    assert torch.equal(torch.exp2(s * c - m), torch.ones_like(s))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [-0.3, 0.0])
def test_cpu_fallback_honors_nonpositive_scales(scale, causal) -> None:
    # The CPU path is SDPA itself, as in the reference; this torch build's CPU
    # SDPA returns NaN for causal inputs with a scale <= 0 (it scales after
    # masking), and the fallback reproduces that bit for bit. The gfx950
    # kernels mask after scaling, like the reference's kernel (attention.py:61-66).
    q = torch.randn(1, 2, 9, 32)
    out = scaled_dot_product_attention(q, q, q, scale=scale, is_causal=causal)
    ref = torch.nn.functional.scaled_dot_product_attention(q, q, q, scale=scale, is_causal=causal)
    torch.testing.assert_close(out, ref, equal_nan=True, rtol=0, atol=0)


# --- the Python eligibility bounds are the library's own ----------------------
@pytest.mark.parametrize("width", [32, 64, 128])
def test_length_bound_matches_library_workspace_query(width) -> None:
    """_decide sends exactly the lengths the C ABI accepts (fa_capi.hip
    check_common / check_kv_length) to the kernel, at the boundary for each
    kernel width; the workspace queries check before any HIP call."""
    from triton_flash_attention import _lib

    lib = _lib.load()
    n_max = attn._max_sequence(width)
    for n in (n_max - 1, n_max, n_max + 1):
        fits = attn._sequence_fits(n, width)
        assert fits == (n <= n_max)
        d_q = attn._decide(_facts(q_len=n, kv_len=64, head_dim=width, value_head_dim=width))
        d_kv = attn._decide(_facts(q_len=64, kv_len=n, head_dim=width, value_head_dim=width))
        rc_q = lib.fa_fwd_workspace_bytes(1, 1, 1, n, 64, width, 0)
        rc_kv = lib.fa_fwd_workspace_bytes(1, 1, 1, 64, n, width, 0)
        rc_dkdv = lib.fa_bwd_dkdv_workspace_bytes_kv(1, 1, 1, 64, n, width, 0)
        assert (rc_q >= 0) == fits == (d_q.backend == "triton"), (n, rc_q, d_q)
        assert (rc_kv >= 0) == fits == (d_kv.backend == "triton"), (n, rc_kv, d_kv)
        assert (rc_dkdv >= 0) == fits
        if not fits:
            assert rc_q == rc_kv == _lib.FA_ERR_TOO_LARGE
    # a smaller head size is checked at the kernel width it is padded to
    d = attn._decide(_facts(q_len=attn._max_sequence(128), kv_len=64, head_dim=96,
                            value_head_dim=96))
    assert d.backend == "triton"
    d = attn._decide(_facts(q_len=attn._max_sequence(128) + 1, kv_len=64, head_dim=96,
                            value_head_dim=96))
    assert d.backend == "torch" and "too long" in d.reason


def test_batch_heads_bound_matches_library() -> None:
    from triton_flash_attention import _lib

    lib = _lib.load()
    limit = attn._MAX_BATCH_HEADS
    assert lib.fa_fwd_workspace_bytes(1, limit - 1, 1, 16, 16, 64, 0) >= 0
    assert lib.fa_fwd_workspace_bytes(1, limit, 1, 16, 16, 64, 0) == _lib.FA_ERR_TOO_LARGE
    assert attn._decide(_facts(batch_heads=limit - 1)).backend == "triton"
    d = attn._decide(_facts(batch_heads=limit))
    assert d.backend == "torch" and "batch * heads" in d.reason


# --- BASELINE configuration 1 through the package on the CPU -----------------
def test_config1_runs_the_reference_cpu_path_through_the_package() -> None:
    """configs[0] (B1 H4 N257 D64 bidirectional, fp16 on the CPU) through the
    public API: the CPU input takes the reference's SDPA fallback
    (attention.py:647-648 -> 774-786), so the output is bit for bit a direct
    F.scaled_dot_product_attention call on this host, and within fp16 accuracy
    of the committed fp64 golden O (tests/golden/make_golden.py)."""
    from pathlib import Path

    import numpy as np

    data = np.load(Path(__file__).resolve().parent / "golden" / "attention_fp64.npz")
    name = "config1_b1_h4_n257_d64_bidir"
    q, k, v = (torch.from_numpy(data[f"{name}/{t}"]) for t in ("q", "k", "v"))
    assert q.dtype == torch.float16 and tuple(q.shape) == (1, 4, 257, 64)
    decision = explain_dispatch(q, k, v)
    assert decision == DispatchDecision("torch", "the Triton kernel requires a CUDA tensor")
    out = scaled_dot_product_attention(q, k, v)
    direct = torch.nn.functional.scaled_dot_product_attention(q, k, v)
    assert out.dtype == torch.float16 and torch.equal(out, direct)
    golden = torch.from_numpy(data[f"{name}/o"]).double()
    assert float((out.double() - golden).abs().max()) <= 2e-3
    rel = float(torch.linalg.vector_norm(out.double() - golden) / torch.linalg.vector_norm(golden))
    assert rel <= 5e-3
    with pytest.raises(RuntimeError, match="requires a CUDA tensor"):
        scaled_dot_product_attention(q, k, v, backend="triton")
