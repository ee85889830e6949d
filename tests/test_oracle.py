"""Pins the CPU oracle (oracle/fa_oracle.c) before it is trusted as the checker.

Every oracle function is checked against something independent of it:
  * PyTorch fp64 SDPA + autograd + logsumexp (the library routine the
    reference falls back to, attention.py:786), live and through the committed
    golden fixtures (tests/golden/attention_fp64.npz, made by
    tests/golden/make_golden.py with torch only);
  * closed forms the mathematics fixes (causal row 0, Q = 0, constant V, N = 1,
    the GQA group-sum identity, integer dot products);
  * numpy's float16 conversion for the fp16 rounding helper;
and planted mistakes (a doubled scale, a flipped mask, a dropped GQA sum, a
missing Delta term) are shown to fail those checks, so the checks have teeth.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_fp64.npz"


def _inputs(B, Hq, Hkv, N, D, seed, mult=1.0, n_kv=None, d_v=None):
    g = torch.Generator("cpu").manual_seed(seed)
    n_kv = N if n_kv is None else n_kv
    d_v = D if d_v is None else d_v
    q = (torch.randn((B, Hq, N, D), generator=g) * mult).half()
    k = (torch.randn((B, Hkv, n_kv, D), generator=g) * mult).half()
    v = (torch.randn((B, Hkv, n_kv, d_v), generator=g) * mult).half()
    do = (torch.randn((B, Hq, N, d_v), generator=g) * mult).half()
    return q, k, v, do


def _torch_fp64(q, k, v, do, causal, scale=None):
    Hq, Hkv, N, D = q.shape[1], k.shape[1], q.shape[2], q.shape[3]
    Nkv = k.shape[2]
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(
        q64, k64, v64, is_causal=causal, scale=scale, enable_gqa=Hq != Hkv)
    dq, dk, dv = torch.autograd.grad(o, (q64, k64, v64), do.double())
    sc = D ** -0.5 if scale is None else scale
    with torch.no_grad():
        s = q64 @ k64.repeat_interleave(Hq // Hkv, 1).transpose(-1, -2) * sc
        if causal:
            # top-left: query i sees keys j <= i (SDPA's mask for N != Nkv too)
            s = s.masked_fill(torch.ones(N, Nkv, dtype=torch.bool).triu(1), -math.inf)
        lse2 = torch.logsumexp(s, -1) / math.log(2.0)
    exact_delta = (o.detach() * do.double()).sum(-1)
    return {"o": o.detach().numpy(), "lse": lse2.numpy(), "dq": dq.numpy(),
            "dk": dk.numpy(), "dv": dv.numpy(), "delta": exact_delta.numpy()}


def _maxdiff(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


# ---------------------------------------------------------------------------
# fp16 rounding
# ---------------------------------------------------------------------------
def test_round_half_matches_numpy_float16():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100_000) * np.logspace(-9, 5.2, 100_000)
    # exact ties between neighbouring fp16 values, subnormals and the overflow edge
    halves = np.arange(0, 0x7C00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = (np.arange(0, 0x7C00, 7, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    ties = (halves + nxt) / 2
    edge = np.array([65504.0, 65519.999, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0])
    for arr in (x, -x, ties, -ties, edge, -edge):
        with np.errstate(over="ignore"):
            expected = arr.astype(np.float16).astype(np.float64)
        np.testing.assert_array_equal(oracle.round_half(arr), expected)


# ---------------------------------------------------------------------------
# Forward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 2, 17, 32), (2, 4, 2, 65, 64), (1, 3, 1, 50, 128),
                                   (1, 1, 1, 1, 64), (2, 2, 2, 130, 32)])
def test_forward_matches_torch_fp64(shape, causal):
    B, Hq, Hkv, N, D = shape
    q, k, v, do = _inputs(B, Hq, Hkv, N, D, seed=N + D)
    ref = _torch_fp64(q, k, v, do, causal)
    o, lse = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    assert _maxdiff(o, ref["o"]) < 1e-12
    assert _maxdiff(lse, ref["lse"]) < 1e-12


def test_forward_custom_scale_matches_torch_fp64():
    q, k, v, do = _inputs(1, 2, 2, 33, 64, seed=3)
    for scale in (0.01, 0.3, 2.0):
        ref = _torch_fp64(q, k, v, do, True, scale)
        o, lse = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), True, scale)
        assert _maxdiff(o, ref["o"]) < 1e-12
        assert _maxdiff(lse, ref["lse"]) < 1e-12


@pytest.mark.parametrize("causal", [False, True])
def test_online_recurrence_equals_closed_form(causal):
    """The reference's tiled online softmax is tiling-independent in exact
    arithmetic: in fp64 it must equal the two-pass closed form for any tiles."""
    q, k, v, _ = _inputs(2, 2, 2, 301, 64, seed=5)
    o, lse = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    for bm, bn in ((64, 32), (128, 32), (128, 64), (16, 16)):
        oo, ll = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal, online=True,
                            block_m=bm, block_n=bn, round_p=False)
        assert _maxdiff(oo, o) < 1e-12 and _maxdiff(ll, lse) < 1e-12


def test_online_fp16_p_rounding_stays_within_half_ulp_bound():
    """With P rounded to fp16 for P.V (attention.py:73) each term moves by at
    most 2^-11 relative, so |O_fp16P - O| <= 2^-11 * max|v| (weights sum to 1)."""
    q, k, v, _ = _inputs(1, 2, 2, 200, 64, seed=6)
    o, _ = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), True)
    oo, _ = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), True, online=True, round_p=True)
    bound = 2.0 ** -11 * float(np.abs(v.numpy()).max())
    diff = _maxdiff(oo, o)
    assert 0 < diff <= bound


def test_forward_closed_forms():
    q, k, v, _ = _inputs(1, 2, 2, 120, 64, seed=7)
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
    # causal row 0 sees only key 0: O[0] = V[0], LSE2 = s00 / ln 2
    o, lse = oracle.fwd(qn, kn, vn, True)
    np.testing.assert_allclose(o[:, :, 0], vn[:, :, 0].astype(np.float64), atol=1e-14)
    s00 = (qn[:, :, 0].astype(np.float64) * kn[:, :, 0]).sum(-1) / 8.0
    np.testing.assert_allclose(lse[:, :, 0], s00 / math.log(2.0), atol=1e-12)
    # Q = 0: uniform weights over the visible keys
    z = np.zeros_like(qn)
    o, lse = oracle.fwd(z, kn, vn, True)
    counts = np.arange(1, 121, dtype=np.float64)
    np.testing.assert_allclose(o, np.cumsum(vn.astype(np.float64), 2) / counts[:, None], atol=1e-13)
    np.testing.assert_allclose(lse, np.broadcast_to(np.log2(counts), lse.shape), atol=1e-13)
    o, lse = oracle.fwd(z, kn, vn, False)
    np.testing.assert_allclose(lse, np.log2(120.0), atol=1e-13)
    # N = 1: O = V
    o, _ = oracle.fwd(qn[:, :, :1], kn[:, :, :1], vn[:, :, :1], False)
    np.testing.assert_allclose(o, vn[:, :, :1].astype(np.float64), atol=1e-15)


# ---------------------------------------------------------------------------
# Delta and backward
# ---------------------------------------------------------------------------
def test_preprocess_exact_on_integers():
    rng = np.random.default_rng(1)
    o = rng.integers(-8, 8, size=(2, 3, 5, 32)).astype(np.float64)
    do = rng.integers(-8, 8, size=(2, 3, 5, 32)).astype(np.float64)
    np.testing.assert_array_equal(oracle.bwd_preprocess(o, do), (o * do).sum(-1))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 2, 17, 32), (2, 4, 2, 65, 64), (1, 4, 1, 40, 128),
                                   (1, 6, 3, 33, 64)])
def test_backward_matches_torch_autograd_fp64(shape, causal):
    B, Hq, Hkv, N, D = shape
    q, k, v, do = _inputs(B, Hq, Hkv, N, D, seed=2 * N + D)
    ref = _torch_fp64(q, k, v, do, causal)
    _, lse = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    dq, dk, dv = oracle.bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), lse, ref["delta"], causal)
    assert _maxdiff(dq, ref["dq"]) < 1e-12
    assert _maxdiff(dk, ref["dk"]) < 1e-12
    assert _maxdiff(dv, ref["dv"]) < 1e-12


def test_backward_closed_forms():
    q, k, v, do = _inputs(1, 2, 2, 90, 64, seed=8)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    # constant V rows: dP_ij = dO_i . v0 = Delta_i so dS = 0 -> dQ = dK = 0
    vc = np.broadcast_to(vn[:, :, :1], vn.shape).copy()
    r = oracle.attention(qn, kn, vc, don, True, o16=np.broadcast_to(vc, qn.shape))
    assert np.max(np.abs(r["dq"])) < 1e-12 and np.max(np.abs(r["dk"])) < 1e-12
    # dV = P^T dO: with Q = 0 and causal, dV_j = sum_{i>=j} dO_i / (i+1)
    z = np.zeros_like(qn)
    r = oracle.attention(z, kn, vn, don, True)
    w = 1.0 / np.arange(1, 91, dtype=np.float64)
    expected = np.flip(np.cumsum(np.flip(don.astype(np.float64) * w[:, None], 2), 2), 2)
    np.testing.assert_allclose(r["dv"], expected, atol=1e-12)
    # N = 1: P = 1, dS = dO.v - Delta = 0 when Delta uses the exact O (= V)
    r = oracle.attention(qn[:, :, :1], kn[:, :, :1], vn[:, :, :1], don[:, :, :1], False,
                         o16=vn[:, :, :1])
    assert np.max(np.abs(r["dq"])) < 1e-15 and np.max(np.abs(r["dk"])) < 1e-15
    np.testing.assert_allclose(r["dv"], don[:, :, :1].astype(np.float64), atol=1e-15)


# ---------------------------------------------------------------------------
# Cross-attention (Nkv != N): the reference's SDPA fallback, attention.py:639-642
# ---------------------------------------------------------------------------
CROSS_SHAPES = [(1, 2, 2, 17, 40, 32), (2, 4, 2, 65, 23, 64), (1, 3, 1, 1, 50, 128),
                (1, 2, 1, 50, 1, 64), (1, 4, 4, 33, 97, 32)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", CROSS_SHAPES)
def test_cross_attention_matches_torch_fp64(shape, causal):
    B, Hq, Hkv, N, Nkv, D = shape
    q, k, v, do = _inputs(B, Hq, Hkv, N, D, seed=N + 3 * Nkv + D, n_kv=Nkv)
    ref = _torch_fp64(q, k, v, do, causal)
    o, lse = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    assert o.shape == (B, Hq, N, D) and lse.shape == (B, Hq, N)
    assert _maxdiff(o, ref["o"]) < 1e-12
    assert _maxdiff(lse, ref["lse"]) < 1e-12
    dq, dk, dv = oracle.bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), lse, ref["delta"], causal)
    assert dk.shape == (B, Hkv, Nkv, D)
    assert _maxdiff(dq, ref["dq"]) < 1e-12
    assert _maxdiff(dk, ref["dk"]) < 1e-12
    assert _maxdiff(dv, ref["dv"]) < 1e-12


def test_cross_attention_causal_closed_forms():
    """Top-left causal with unequal lengths reduces to self-attention pieces:
    N < Nkv never looks past key N-1 (keys beyond get zero gradients);
    N > Nkv gives rows i >= Nkv the bidirectional result over all keys. A
    bottom-right mask (the other convention for unequal lengths) fails both."""
    q, k, v, do = _inputs(1, 2, 2, 40, 64, seed=12, n_kv=100)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    cross = oracle.attention(qn, kn, vn, don, True)
    self_ = oracle.attention(qn, kn[:, :, :40], vn[:, :, :40], don, True)
    for name in ("o", "lse", "dq"):
        assert _maxdiff(cross[name], self_[name]) < 1e-12
    assert _maxdiff(cross["dk"][:, :, :40], self_["dk"]) < 1e-12
    assert np.all(cross["dk"][:, :, 40:] == 0) and np.all(cross["dv"][:, :, 40:] == 0)
    # bottom-right alignment would let query 0 see keys 0..60: a different O
    shifted = oracle.fwd(qn[:, :, :1], kn[:, :, :61], vn[:, :, :61], False)[0]
    assert _maxdiff(cross["o"][:, :, :1], shifted) > 1e-3

    q, k, v, do = _inputs(1, 2, 1, 90, 32, seed=13, n_kv=30)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    o, lse = oracle.fwd(qn, kn, vn, True)
    o_top, lse_top = oracle.fwd(qn[:, :, :30], kn, vn, True)
    o_all, lse_all = oracle.fwd(qn[:, :, 30:], kn, vn, False)
    assert _maxdiff(o[:, :, :30], o_top) < 1e-12 and _maxdiff(lse[:, :, :30], lse_top) < 1e-12
    assert _maxdiff(o[:, :, 30:], o_all) < 1e-12 and _maxdiff(lse[:, :, 30:], lse_all) < 1e-12


# ---------------------------------------------------------------------------
# Value head size != query/key head size (the fallback's other case, attention.py:643-646)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 2, 33, 33, 64, 32), (2, 4, 2, 40, 70, 32, 128),
                                   (1, 3, 1, 65, 17, 128, 64)])
def test_value_head_size_matches_torch_fp64(shape, causal):
    B, Hq, Hkv, N, Nkv, D, Dv = shape
    q, k, v, do = _inputs(B, Hq, Hkv, N, D, seed=N + Nkv + D + 7 * Dv, n_kv=Nkv, d_v=Dv)
    ref = _torch_fp64(q, k, v, do, causal)
    o, lse = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    assert o.shape == (B, Hq, N, Dv)
    assert _maxdiff(o, ref["o"]) < 1e-12
    assert _maxdiff(lse, ref["lse"]) < 1e-12
    for fold in (False, True):
        dq, dk, dv = oracle.bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), lse, ref["delta"],
                                causal, fold=fold)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
        tol = 1e-12 if not fold else 5e-2  # fold rounds the score operands to fp16
        assert _maxdiff(dq, ref["dq"]) < tol
        assert _maxdiff(dk, ref["dk"]) < tol
        assert _maxdiff(dv, ref["dv"]) < tol


def test_zero_padding_a_head_size_is_exact():
    """Zero columns appended to the narrower of (q, k) and v leave O, LSE and
    the gradients of the real columns unchanged and give zero gradients in the
    padded ones: the identity the library's D_v != D path relies on."""
    q, k, v, do = _inputs(1, 4, 2, 50, 32, seed=21, n_kv=61, d_v=128)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    r = oracle.attention(qn, kn, vn, don, True, fold_bwd=True)
    pad = lambda a, w: np.concatenate([a, np.zeros(a.shape[:-1] + (w - a.shape[-1],))], -1)
    p = oracle.attention(pad(qn, 128), pad(kn, 128), vn, don, True, 32 ** -0.5, fold_bwd=True)
    for name in ("o", "lse", "delta", "dv"):
        assert _maxdiff(r[name], p[name]) == 0.0
    for name in ("dq", "dk"):
        assert _maxdiff(r[name], p[name][..., :32]) == 0.0
        assert not p[name][..., 32:].any()
    q, k, v, do = _inputs(1, 2, 2, 40, 128, seed=22, d_v=64)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    r = oracle.attention(qn, kn, vn, don, False, fold_bwd=True)
    p = oracle.attention(qn, kn, pad(vn, 128), pad(don, 128), False, fold_bwd=True)
    for name in ("lse", "delta", "dq", "dk"):
        assert _maxdiff(r[name], p[name]) == 0.0
    for name in ("o", "dv"):
        assert _maxdiff(r[name], p[name][..., :64]) == 0.0
        assert not p[name][..., 64:].any()


def test_gqa_group_sum_identity():
    """dK/dV of a shared K/V head equal the sum over its query heads of the
    MHA gradients computed with K/V repeated per query head."""
    q, k, v, do = _inputs(1, 6, 2, 70, 32, seed=9)
    r = oracle.attention(q.numpy(), k.numpy(), v.numpy(), do.numpy(), True)
    kr, vr = k.repeat_interleave(3, 1), v.repeat_interleave(3, 1)
    m = oracle.attention(q.numpy(), kr.numpy(), vr.numpy(), do.numpy(), True)
    for name in ("o", "lse", "dq"):
        assert _maxdiff(r[name], m[name]) < 1e-12
    assert _maxdiff(r["dk"], m["dk"].reshape(1, 2, 3, 70, 32).sum(2)) < 1e-12
    assert _maxdiff(r["dv"], m["dv"].reshape(1, 2, 3, 70, 32).sum(2)) < 1e-12


# ---------------------------------------------------------------------------
# Golden fixtures (torch fp64, committed)
# ---------------------------------------------------------------------------
def _golden_cases():
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files if "/" in k})
    return data, names


def test_golden_fixtures_match_oracle():
    data, names = _golden_cases()
    assert len(names) >= 14
    for name in names:
        g = {k.split("/")[1]: data[k] for k in data.files if k.startswith(name + "/")}
        B, Hq, Hkv, N, D, causal = (int(x) for x in g["meta"])
        assert g["q"].dtype == np.float16
        o, lse = oracle.fwd(g["q"], g["k"], g["v"], bool(causal))
        assert _maxdiff(o, g["o"]) < 1e-6, name
        assert _maxdiff(lse, g["lse2"]) < 1e-12, name
        if "do" not in g:
            continue
        np.testing.assert_array_equal(oracle.round_half(g["o16"]), g["o16"].astype(np.float64))
        delta16 = oracle.bwd_preprocess(g["o16"], g["do"])
        assert _maxdiff(delta16, g["delta"]) < 1e-12, name
        exact_delta = oracle.bwd_preprocess(o, g["do"])
        dq, dk, dv = oracle.bwd(g["q"], g["k"], g["v"], g["do"], lse, exact_delta, bool(causal))
        for key, val in (("dq", dq), ("dk", dk), ("dv", dv)):
            scale = max(1.0, float(np.abs(g[key]).max()))
            assert _maxdiff(val, g[key]) < 1e-6 * scale, f"{name} {key}"


def test_golden_config1_cpu_fallback_is_close_to_fp64():
    """Configuration 1 runs the reference's CPU fallback (fp16 torch SDPA); its
    fp16 output agrees with the fp64 oracle to fp16 accuracy."""
    data = np.load(GOLDEN)
    name = "config1_b1_h4_n257_d64_bidir"
    o, _ = oracle.fwd(data[name + "/q"], data[name + "/k"], data[name + "/v"], False)
    assert _maxdiff(o, data[name + "/o_cpu_fp16_sdpa"]) < 2e-3


# ---------------------------------------------------------------------------
# Backward with the reference's fp16-rounded score operands (fold=True):
# k_scaled = fp16(k * (sm_scale * log2 e)) for dK/dV, q_scaled likewise for dQ
# (attention.py:435, 515), the product taken in fp32.
# ---------------------------------------------------------------------------
INV_LN2 = 1.4426950408889634


def _scale_with_c32(target: float) -> float:
    """A scale whose fp32 product with fp32(1/ln 2) is exactly ``target``."""
    s = np.float32(target / INV_LN2)
    for _ in range(64):
        c = np.float32(s) * np.float32(INV_LN2)
        if c == np.float32(target):
            return float(s)
        s = np.nextafter(s, np.float32(np.inf) if c < target else np.float32(-np.inf))
    raise AssertionError("no fp32 scale found")


def _numpy_folded_bwd(q, k, v, do, lse2, delta, causal, scale, fold=True):
    """Tiny-input restatement in numpy (float16 casts via numpy, bfloat16 casts
    via torch; not the oracle's rounding code)."""
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    c32 = np.float32(scale) * np.float32(INV_LN2)
    if fold == "bfloat16":
        f16 = lambda x: torch.from_numpy(c32 * x.astype(np.float32)).to(torch.bfloat16) \
            .double().numpy()
    else:
        f16 = lambda x: (c32 * x.astype(np.float32)).astype(np.float16).astype(np.float64)
    dq = np.zeros(q.shape)
    dk = np.zeros(k.shape)
    dv = np.zeros(v.shape)
    vis = np.tril(np.ones((N, N), bool)) if causal else np.ones((N, N), bool)
    for b in range(B):
        for h in range(Hq):
            hk = h // G
            Q, K, V, dO = q[b, h], k[b, hk], v[b, hk], do[b, h]
            lse = lse2[b, h][:, None]
            p_k = np.where(vis, np.exp2(Q @ f16(K).T - lse), 0.0)
            p_q = np.where(vis, np.exp2(f16(Q) @ K.T - lse), 0.0)
            dp = dO @ V.T
            dv[b, hk] += p_k.T @ dO
            dk[b, hk] += scale * (p_k * (dp - delta[b, h][:, None])).T @ Q
            dq[b, h] = scale * (p_q * (dp - delta[b, h][:, None])) @ K
    return dq, dk, dv


def test_folded_backward_is_exact_when_c_is_a_power_of_two():
    # operands n/8 and c32 = 2^-3: fp16(c32 x) = x/8 exactly
    rng = np.random.default_rng(12)
    q, k, v, do = (rng.integers(-12, 13, size=s).astype(np.float64) / 8.0
                   for s in ((1, 4, 24, 32), (1, 2, 24, 32), (1, 2, 24, 32), (1, 4, 24, 32)))
    scale = _scale_with_c32(0.125)
    for causal in (False, True):
        _, lse = oracle.fwd(q, k, v, causal, scale)
        delta = oracle.bwd_preprocess(oracle.round_half(oracle.fwd(q, k, v, causal, scale)[0]), do)
        exact = oracle.bwd(q, k, v, do, lse, delta, causal, scale)
        for fold in (True, "bfloat16"):  # x/8 has <= 4 significant bits: exact in both
            folded = oracle.bwd(q, k, v, do, lse, delta, causal, scale, fold=fold)
            for a, b in zip(folded, exact):
                # only the double vs fp32 value of c separates them (~1e-8 relative)
                assert _maxdiff(a, b) <= 1e-6 * max(1.0, float(np.abs(b).max()))


@pytest.mark.parametrize("fold", [True, "bfloat16"])
@pytest.mark.parametrize("causal", [False, True])
def test_folded_backward_matches_numpy_restatement(causal, fold):
    q, k, v, do = _inputs(1, 4, 2, 9, 16, seed=31)
    qn, kn, vn, don = (t.numpy().astype(np.float64) for t in (q, k, v, do))
    scale = 0.37
    o, lse = oracle.fwd(qn, kn, vn, causal, scale)
    delta = oracle.bwd_preprocess(oracle.round_half(o), don)
    got = oracle.bwd(qn, kn, vn, don, lse, delta, causal, scale, fold=fold)
    want = _numpy_folded_bwd(qn, kn, vn, don, lse, delta, causal, scale, fold)
    for a, b in zip(got, want):
        assert _maxdiff(a, b) < 1e-12


@pytest.mark.parametrize("fold,bound", [(True, 2e-3), ("bfloat16", 8e-3)])
def test_folded_backward_differs_within_the_operand_rounding(fold, bound):
    q, k, v, do = _inputs(1, 2, 2, 40, 64, seed=32)
    qn, kn, vn, don = (t.numpy().astype(np.float64) for t in (q, k, v, do))
    o, lse = oracle.fwd(qn, kn, vn, True)
    delta = oracle.bwd_preprocess(oracle.round_half(o), don)
    exact = oracle.bwd(qn, kn, vn, don, lse, delta, True)
    folded = oracle.bwd(qn, kn, vn, don, lse, delta, True, fold=fold)
    for a, b in zip(folded, exact):
        rel = float(np.linalg.norm(a - b) / np.linalg.norm(b))
        # the rounding is applied (dV too: its P uses the rounded K) ...
        assert rel > 1e-7
        # ... and is no larger than a half-ulp operand perturbation (2^-11 for
        # fp16, 2^-8 for bf16) allows
        assert rel < bound


# ---------------------------------------------------------------------------
# Planted mistakes: each variant of the oracle must fail the checks above.
# ---------------------------------------------------------------------------
def test_planted_mistakes_are_caught():
    q, k, v, do = _inputs(1, 4, 2, 48, 64, seed=10)
    ref = _torch_fp64(q, k, v, do, True)
    qn, kn, vn, don = q.numpy(), k.numpy(), v.numpy(), do.numpy()
    # doubled softmax scale
    o, _ = oracle.fwd(qn, kn, vn, True, scale=2 * 64 ** -0.5)
    assert _maxdiff(o, ref["o"]) > 1e-3
    # mask flipped to bidirectional
    o, _ = oracle.fwd(qn, kn, vn, False)
    assert _maxdiff(o, ref["o"]) > 1e-3
    # wrong GQA map (query head h reads K/V head h % Hkv instead of h // group)
    perm = np.array([0, 2, 1, 3])
    o, _ = oracle.fwd(qn[:, perm], kn, vn, True)
    assert _maxdiff(o[:, np.argsort(perm)], ref["o"]) > 1e-3
    # Delta term dropped from dS
    _, lse = oracle.fwd(qn, kn, vn, True)
    dq, dk, _ = oracle.bwd(qn, kn, vn, don, lse, np.zeros_like(ref["delta"]), True)
    assert _maxdiff(dq, ref["dq"]) > 1e-3 and _maxdiff(dk, ref["dk"]) > 1e-3
    # natural-log LSE fed where the base-2 LSE is expected
    dq, _, dv = oracle.bwd(qn, kn, vn, don, lse * math.log(2.0), ref["delta"], True)
    assert _maxdiff(dv, ref["dv"]) > 1e-3
