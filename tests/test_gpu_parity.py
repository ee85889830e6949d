"""GPU parity of the gfx950 kernels against the CPU oracle and the reference path.

Everything here goes through the product path (libfa_gfx950.so via the public
API with ``backend="triton"``, which raises instead of falling back) and is
compared with:
  * the fp64 CPU oracle (oracle/fa_oracle.c) at sizes it finishes in seconds,
    and on head slices of the full BASELINE configurations;
  * a plain PyTorch fp32 reference on the GPU at the full configurations;
  * PyTorch SDPA (the reference's own path on ROCm, attention.py:774-786) at
    the reference test shapes and tolerances (tests/test_cuda_correctness.py).
Tolerances: O, dQ, dK, dV max-abs <= 2e-2 and
relative L2 <= 5e-3; base-2 LSE max-abs <= 1e-4.
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

from fa_testutil import (
    CONFIGS,
    LSE_TOL,
    MAX_ABS_TOL,
    REL_L2_TOL,
    assert_close,
    errors,
    make_inputs,
    torch_reference_fp32,
)
from oracle import oracle
from triton_flash_attention import _lib, _ops, explain_dispatch, scaled_dot_product_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _library_loaded():
    torch.backends.cuda.matmul.allow_tf32 = False
    ok, why = _lib.available()
    assert ok, f"libfa_gfx950.so must load on the GPU box: {why}"
    props = torch.cuda.get_device_properties(0)
    _note(f"device: {props.name} {getattr(props, 'gcnArchName', '?')} CUs={props.multi_processor_count}")


def run_kernel(q, k, v, do, causal, scale=None):
    """Forward + backward through the public API on the GPU; LSE from the same
    forward kernel via the op layer. Returns CPU float64 numpy arrays."""
    enable_gqa = q.shape[1] != k.shape[1]
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    dod = do.to(DEV)
    out = scaled_dot_product_attention(
        qd, kd, vd, is_causal=causal, enable_gqa=enable_gqa, scale=scale, backend="triton"
    )
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), dod)
    s = q.shape[-1] ** -0.5 if scale is None else scale
    o2, lse = _ops.flash_fwd(qd.detach().contiguous(), kd.detach().contiguous(),
                             vd.detach().contiguous(), causal, s)
    torch.cuda.synchronize()
    assert torch.equal(o2, out.detach()), "public API and op layer disagree"
    return {
        "o16": out.detach().cpu(),
        "o": out.detach().double().cpu().numpy(),
        "lse": lse.double().cpu().numpy(),
        "dq": dq.double().cpu().numpy(),
        "dk": dk.double().cpu().numpy(),
        "dv": dv.double().cpu().numpy(),
    }


def check_against_oracle(got, q, k, v, do, causal, scale=None, tag=""):
    # The backward is checked against the reference's own algorithm: scores
    # from its fp16-rounded scaled operands (attention.py:435, 515).
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal, scale,
                           o16=got["o16"].numpy(), fold_bwd=True)
    report = {}
    for name in ("o", "dq", "dk", "dv"):
        report[name] = assert_close(f"{tag} {name}", got[name], ref[name])
    lse_err = float(np.max(np.abs(got["lse"] - ref["lse"])))
    assert lse_err <= LSE_TOL, f"{tag} lse: max-abs {lse_err:.3e} (tol {LSE_TOL:.0e})"
    report["lse"] = lse_err
    _note(f"{tag}: " + ", ".join(
        f"{k}={v[0]:.2e}/{v[1]:.2e}" if isinstance(v, tuple) else f"{k}={v:.2e}"
        for k, v in report.items()))
    return report


# ---------------------------------------------------------------------------
# Reference test shapes (tests/test_cuda_correctness.py:87-101) plus D=128.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sequence", [17, 129])
@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_reference_shapes_match_oracle(sequence, head_dim, causal):
    q, k, v, do = make_inputs(1, 2, 2, sequence, head_dim, seed=123, mult=0.5, do_mult=0.1)
    got = run_kernel(q, k, v, do, causal)
    check_against_oracle(got, q, k, v, do, causal, tag=f"N={sequence} D={head_dim} causal={causal}")


def test_reference_gqa_shape_matches_oracle():
    q, k, v, do = make_inputs(1, 4, 2, 65, 64, seed=123, mult=0.5, do_mult=0.1)
    got = run_kernel(q, k, v, do, True)
    check_against_oracle(got, q, k, v, do, True, tag="GQA 4->2 N=65 D=64 causal")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sequence", [17, 129])
@pytest.mark.parametrize("head_dim", [32, 64])
def test_matches_torch_sdpa_like_reference_suite(sequence, head_dim, causal):
    """The reference's own differential test, against PyTorch SDPA evaluated
    in fp32 on the GPU (atol 2e-2 for O, 3e-2 for grads, rtol 0)."""
    torch.manual_seed(123)
    q = (torch.randn(1, 2, sequence, head_dim, device=DEV, dtype=torch.float16) * 0.5)
    k = (torch.randn(1, 2, sequence, head_dim, device=DEV, dtype=torch.float16) * 0.5)
    v = (torch.randn(1, 2, sequence, head_dim, device=DEV, dtype=torch.float16) * 0.5)
    do = torch.randn_like(q) * 0.1
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    actual = scaled_dot_product_attention(qa, ka, va, is_causal=causal, backend="triton")
    qe, ke, ve = (t.float().requires_grad_() for t in (q, k, v))
    expected = torch.nn.functional.scaled_dot_product_attention(qe, ke, ve, is_causal=causal)
    torch.testing.assert_close(actual.float(), expected, atol=2e-2, rtol=0)
    ga = torch.autograd.grad(actual, (qa, ka, va), do)
    ge = torch.autograd.grad(expected, (qe, ke, ve), do.float())
    for a, e in zip(ga, ge):
        torch.testing.assert_close(a.float(), e, atol=3e-2, rtol=0)


# ---------------------------------------------------------------------------
# Tails and tile boundaries, GQA groups, custom scale.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("sequence", [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 255, 256, 257, 300])
def test_tails_match_oracle(sequence):
    for causal in (False, True):
        q, k, v, do = make_inputs(2, 2, 2, sequence, 64, seed=7 + sequence)
        got = run_kernel(q, k, v, do, causal)
        check_against_oracle(got, q, k, v, do, causal, tag=f"tail N={sequence} causal={causal}")


@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("heads", [(4, 1), (8, 2), (6, 3), (3, 3)])
def test_gqa_groups_match_oracle(head_dim, heads):
    hq, hkv = heads
    for causal in (False, True):
        q, k, v, do = make_inputs(2, hq, hkv, 150, head_dim, seed=11 * hq + hkv)
        got = run_kernel(q, k, v, do, causal)
        check_against_oracle(got, q, k, v, do, causal,
                             tag=f"GQA {hq}->{hkv} D={head_dim} causal={causal}")


def test_custom_scale_matches_oracle():
    q, k, v, do = make_inputs(1, 2, 2, 200, 64, seed=5)
    for scale in (0.05, 0.25, 1.0):
        got = run_kernel(q, k, v, do, True, scale=scale)
        check_against_oracle(got, q, k, v, do, True, scale=scale, tag=f"scale={scale}")


# (B, Hq, Hkv, N_q, N_kv, D, causal, dtype): the C++ binding's envelope, including
# the library's split plans (split-KV forward and split dQ, split dK/dV with the
# combined launch) and cross-attention.
NATIVE_CASES = [
    (2, 4, 4, 300, 300, 64, True, torch.float16),
    (1, 8, 2, 777, 777, 32, False, torch.float16),
    (1, 4, 4, 260, 260, 128, True, torch.bfloat16),
    (2, 16, 4, 2049, 2049, 64, True, torch.float16),
    (1, 8, 2, 3, 6000, 128, False, torch.float16),
    (1, 4, 2, 300, 900, 64, True, torch.float16),
    (1, 4, 1, 900, 300, 32, False, torch.bfloat16),
]


def _api_fwd_bwd(q, k, v, do, causal, grad_of=(0, 1, 2)):
    ts = [t.to(DEV) for t in (q, k, v)]
    for i in grad_of:
        ts[i].requires_grad_()
    out = scaled_dot_product_attention(*ts, is_causal=causal, enable_gqa=q.shape[1] != k.shape[1],
                                       backend="triton")
    grads = torch.autograd.grad(out, [ts[i] for i in grad_of], do.to(DEV))
    torch.cuda.synchronize()
    return out.detach(), grads, type(out.grad_fn).__name__


@pytest.mark.parametrize("case", NATIVE_CASES, ids=lambda c: "B{}Hq{}Hkv{}Nq{}Nkv{}D{}".format(
    *c[:6]) + ("causal" if c[6] else "bidir") + str(c[7])[6:])
def test_native_binding_matches_the_python_function_bitwise(case, monkeypatch):
    """The public API's training path through the C++ autograd binding makes the
    Python TritonAttention Function's library calls, so O, dQ, dK and dV are
    equal bit for bit; also with a subset of inputs requiring grad and on a
    side stream."""
    from triton_flash_attention import _native
    from triton_flash_attention import attention as api

    B, Hq, Hkv, N, Nkv, D, causal, dtype = case
    _note(f"native B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} causal={causal} {dtype}")
    assert _native.available(), _native.status()
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + Nkv + D, n_kv=Nkv, dtype=dtype)
    o_n, g_n, node_n = _api_fwd_bwd(q, k, v, do, causal)
    with monkeypatch.context() as m:
        m.setattr(api, "_native_serves", lambda *a: False)
        o_p, g_p, node_p = _api_fwd_bwd(q, k, v, do, causal)
        o_p2, g_p2, _ = _api_fwd_bwd(q, k, v, do, causal, grad_of=(1, 2))
    assert node_p == "TritonAttentionBackward" and node_n != node_p, (node_n, node_p)
    assert torch.equal(o_n, o_p)
    for name, a, b in zip(("dq", "dk", "dv"), g_n, g_p):
        assert torch.equal(a, b), name
    o_n2, g_n2, _ = _api_fwd_bwd(q, k, v, do, causal, grad_of=(1, 2))
    assert torch.equal(o_n2, o_p2) and all(torch.equal(a, b) for a, b in zip(g_n2, g_p2))
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        o_s, g_s, _ = _api_fwd_bwd(q, k, v, do, causal)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o_p) and all(torch.equal(a, b) for a, b in zip(g_s, g_p))
    # No gradient: the binding's forward-only entry, the same launch.
    with torch.no_grad():
        o_i = scaled_dot_product_attention(q.to(DEV), k.to(DEV), v.to(DEV), is_causal=causal,
                                           enable_gqa=Hq != Hkv, backend="triton")
    torch.cuda.synchronize()
    assert o_i.grad_fn is None and torch.equal(o_i, o_p)


# (B, Hq, Hkv, N, D): one MHA shape at a kernel head size, one padded head size
# (40 runs at 64), one GQA group of 4 with a ragged length.
NON_POSITIVE_SCALE_CASES = [(1, 2, 2, 150, 64), (1, 2, 2, 129, 40), (2, 8, 2, 97, 32)]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [-0.3, 0.0, 1e-40])
@pytest.mark.parametrize("case", NON_POSITIVE_SCALE_CASES,
                         ids=lambda c: "B{}Hq{}Hkv{}N{}D{}".format(*c))
def test_non_positive_scales_run_forward_and_backward_on_the_kernels(case, scale, causal):
    """Scales that are negative, zero or subnormal in float32 run on the gfx950
    kernels through the query transforms of attention._kernel_scale ("negate":
    -q at |scale|, dQ negated back; "zero": a zero q at scale 1, dQ = 0), with
    head padding and GQA on top. O, dQ, dK, dV and the base-2 LSE are checked
    against the fp64 oracle evaluated at the scale as given."""
    from triton_flash_attention import attention as api

    B, Hq, Hkv, N, D = case
    tag = f"scale={scale} B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal}"
    _note(tag)
    assert api._kernel_scale(scale)[1] == ("negate" if scale < 0 else "zero")
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + int(causal), mult=0.8)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    assert explain_dispatch(qd, kd, vd, enable_gqa=Hq != Hkv).backend == "triton"
    out = scaled_dot_product_attention(qd, kd, vd, is_causal=causal, scale=scale,
                                       enable_gqa=Hq != Hkv, backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    with torch.no_grad():
        lse = api._padded_forward(qd.detach(), kd.detach(), vd.detach(), causal, scale)[4]
    torch.cuda.synchronize()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal, scale,
                           o16=out.detach().cpu().numpy(), fold_bwd=True)
    report = {}
    for name, t in (("o", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        a = t.detach().double().cpu().numpy()
        if name in ("dq", "dk") and scale >= 0:
            # The exact dQ = scale dS K and dK = scale dS^T Q are below 1e-40 * |dS| |K|
            # (0 at scale 0), which fp16 holds as 0; the kernels return exact zeros
            # (dQ set to zero, dK from the zero query).
            assert not t.any(), f"{tag}: {name} of a zero or subnormal scale is exactly zero"
            assert np.max(np.abs(ref[name])) < 1e-30
            continue
        report[name] = assert_close(f"{tag} {name}", a, ref[name])
    lse_err = float(np.max(np.abs(lse.double().cpu().numpy() - ref["lse"])))
    assert lse_err <= LSE_TOL, f"{tag} lse: max-abs {lse_err:.3e} (tol {LSE_TOL:.0e})"
    _note(f"{tag}: " + ", ".join(f"{k}={v[0]:.2e}/{v[1]:.2e}" for k, v in report.items())
          + f", lse={lse_err:.2e}")


# ---------------------------------------------------------------------------
# Closed-form special cases (values fixed by the mathematics).
# ---------------------------------------------------------------------------
def test_causal_row_zero_sees_only_key_zero():
    q, k, v, do = make_inputs(1, 2, 2, 300, 64, seed=3)
    got = run_kernel(q, k, v, do, True)
    np.testing.assert_allclose(got["o"][:, :, 0, :], v.double().numpy()[:, :, 0, :],
                               rtol=1e-3, atol=1e-6)
    s00 = (q.double()[:, :, 0, :] * k.double()[:, :, 0, :]).sum(-1) * 64 ** -0.5 / np.log(2.0)
    assert np.max(np.abs(got["lse"][:, :, 0] - s00.numpy())) < LSE_TOL


def test_zero_query_gives_uniform_attention():
    q, k, v, do = make_inputs(1, 2, 2, 190, 32, seed=4)
    q = torch.zeros_like(q)
    for causal in (False, True):
        got = run_kernel(q, k, v, do, causal)
        vd = v.double().numpy()
        if causal:
            expected = np.cumsum(vd, axis=2) / np.arange(1, 191)[None, None, :, None]
            lse = np.log2(np.arange(1, 191, dtype=np.float64))
        else:
            expected = np.broadcast_to(vd.mean(axis=2, keepdims=True), vd.shape)
            lse = np.full(190, np.log2(190.0))
        assert_close(f"uniform causal={causal}", got["o"], expected)
        assert np.max(np.abs(got["lse"] - lse[None, None, :])) < LSE_TOL


def test_constant_value_rows_give_zero_qk_gradients():
    q, k, v, do = make_inputs(1, 2, 2, 160, 64, seed=8)
    v = v[:, :, :1, :].expand_as(v).contiguous()
    got = run_kernel(q, k, v, do, True)
    np.testing.assert_allclose(got["o"], v.double().numpy(), atol=1e-3)
    assert np.max(np.abs(got["dq"])) < 2e-3 and np.max(np.abs(got["dk"])) < 2e-3


def test_split_dkdv_matches_single_pass():
    """The split-and-reduce dK/dV (few key tiles per KV head) agrees with the
    single-pass kernel up to fp32 summation order."""
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, 8, 2, 1500, 64, seed=12))
    for causal in (False, True):
        o, lse = _ops.flash_fwd(q, k, v, causal, 0.125)
        delta = _ops.flash_bwd_preprocess(o, do)
        lib = _lib.load()
        assert lib.fa_bwd_dkdv_workspace_bytes(1, 8, 2, 1500, 64, int(causal)) > 0
        dk1, dv1 = _ops.flash_bwd_dkdv(q, k, v, do, lse, delta, causal, 0.125)  # split
        dk2, dv2 = torch.empty_like(k), torch.empty_like(v)
        rc = lib.fa_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
                             lse.data_ptr(), delta.data_ptr(), dk2.data_ptr(), dv2.data_ptr(),
                             1, 8, 2, 1500, 64, 0.125, int(causal),
                             torch.cuda.current_stream().cuda_stream)
        _lib.check(rc)
        torch.cuda.synchronize()
        assert_close("split dk", dk1.float(), dk2.float(), max_abs=2e-3, rel_l2=1e-3)
        assert_close("split dv", dv1.float(), dv2.float(), max_abs=2e-3, rel_l2=1e-3)


# (B, Hq, Hkv, N_q, N_kv, D, causal): the dK/dV launch splits and dQ does not,
# so fa_bwd runs the Delta pass and the combined dK/dV + dQ launch.
PAIR_CASES = [
    (1, 8, 2, 1500, 1500, 64, True),
    (1, 8, 2, 1500, 1500, 64, False),
    (2, 16, 4, 2049, 2049, 64, True),
    (2, 16, 4, 2049, 2049, 32, True),
    (1, 8, 2, 1000, 1300, 64, True),
    (1, 4, 1, 900, 700, 32, False),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("case", PAIR_CASES, ids=lambda c: "B{}Hq{}Hkv{}Nq{}Nkv{}D{}".format(
    *c[:6]) + ("causal" if c[6] else "bidir"))
def test_combined_backward_launch_matches_separate_launches_and_reference(case, dtype):
    """The combined launch runs the very dK/dV and dQ work-groups of the
    separate launches: with the same Delta its dQ is bitwise that of fa_bwd_dq
    (self-attention), and its dK, dV those of the split fa_bwd_dkdv_ws when
    both split the key tiles into as many chunks (else equal to fp32
    summation order); two calls are
    bitwise identical; and all three match the fp32 reference (the oracle for
    cross-attention, through the public API)."""
    B, Hq, Hkv, N, Nkv, D, causal = case
    tag = f"combined backward {case} {str(dtype)[6:]}"
    _note(tag)
    lib = _lib.load()
    c = int(causal)
    assert lib.fa_bwd_dkdv_workspace_bytes_kv(B, Hq, Hkv, N, Nkv, D, c) > 0  # dK/dV splits
    assert lib.fa_bwd_dq_workspace_bytes(B, Hq, Hkv, N, Nkv, D, c) == 0  # dQ does not
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + Nkv + D,
                                                    n_kv=Nkv, dtype=dtype))
    scale = D ** -0.5
    o, lse = _ops.flash_fwd(q, k, v, causal, scale)
    dq, dk, dv = _ops.flash_bwd(q, k, v, o, lse, do, causal, scale)
    again = _ops.flash_bwd(q, k, v, o, lse, do, causal, scale)
    delta = _ops.flash_bwd_preprocess(o, do)
    dk_s, dv_s = _ops.flash_bwd_dkdv(q, k, v, do, lse, delta, causal, scale)
    if N == Nkv:
        dq_s = _ops.flash_bwd_dq(q, k, v, do, lse, delta, causal, scale)
    else:  # no Delta-reading dQ entry for cross-attention: the fused one, to fp32 rounding
        dq_s = _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, causal, scale)[1]
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), again):
        assert torch.equal(a, b), f"{tag}: {name} differs between two calls"
    if lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, Nkv, D, c) == \
            lib.fa_bwd_dkdv_workspace_bytes_kv(B, Hq, Hkv, N, Nkv, D, c):  # same chunking
        assert torch.equal(dk, dk_s) and torch.equal(dv, dv_s), f"{tag}: dK/dV differ"
    else:  # fewer chunks beside dQ: the same sums in another fp32 order
        assert_close(f"{tag} dk vs split launch", dk.float(), dk_s.float(), max_abs=2e-3,
                     rel_l2=1e-3)
        assert_close(f"{tag} dv vs split launch", dv.float(), dv_s.float(), max_abs=2e-3,
                     rel_l2=1e-3)
    if N == Nkv:
        assert torch.equal(dq, dq_s), f"{tag}: dQ differs from fa_bwd_dq"
    else:
        assert_close(f"{tag} dq vs fused-Delta dQ", dq.float(), dq_s.float(),
                     max_abs=2e-3, rel_l2=1e-3)
    if N != Nkv:  # the public API on the same inputs against the oracle's cross-attention
        cpu = tuple(t.cpu() for t in (q, k, v, do))
        check = check_bf16_against_oracle if dtype == torch.bfloat16 else check_against_oracle
        check(run_kernel(*cpu, causal), *cpu, causal, tag=tag)
        return
    ref = torch_reference_fp32(q, k, v, do, causal, o16=o)
    tols = (dict(max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL)
            if dtype == torch.bfloat16 else {})
    for name, a in (("dq", dq), ("dk", dk), ("dv", dv)):
        ma, rl = assert_close(f"{tag} {name}", a.float(), ref[name], **tols)
        _note(f"  {name}: max-abs {ma:.2e} rel-L2 {rl:.2e}")


def test_two_key_group_forward_rule_matches_oracle():
    """D = 32 causal launches over few heads run the two-key-group forward
    (each work-group's keys split over two 4-wave groups, merged through LDS):
    results match the oracle and, to fp32 rounding, the table's forward."""
    for (B, Hq, Hkv, N) in [(1, 4, 2, 1500), (1, 2, 1, 333)]:
        tag = f"key-group forward B={B} Hq={Hq} Hkv={Hkv} N={N} D=32"
        _note(tag)
        q, k, v, do = make_inputs(B, Hq, Hkv, N, 32, seed=N)
        got = run_kernel(q, k, v, do, True)
        check_against_oracle(got, q, k, v, do, True, tag=tag)
        qd, kd, vd = (t.to(DEV) for t in (q, k, v))
        o_rule, lse_rule = _ops.flash_fwd(qd, kd, vd, True, 32 ** -0.5)
        _lib.set_tiling(_lib.KERNEL_FWD, 32, True, 6)
        try:
            o_tab, lse_tab = _ops.flash_fwd(qd, kd, vd, True, 32 ** -0.5)
        finally:
            _lib.set_tiling(_lib.KERNEL_FWD, 32, True, -1)
        torch.cuda.synchronize()
        assert_close(tag + " o vs table forward", o_rule.float(), o_tab.float(),
                     max_abs=2e-3, rel_l2=1e-3)
        assert float((lse_rule - lse_tab).abs().max()) <= 1e-5, tag


FWD_GRID_VARIANT = 6  # the pipelined forward, one work-group per (query tile, head)
FWD_PLAN_VARIANT = 9  # the same tiling as a persistent grid of bin-packed jobs


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, N_q, N_kv, D, dtype)
    (4, 16, 16, 4096, 4096, 64, torch.float16),  # c2: 2048 jobs of 4..128 units on 768 slots
    (4, 16, 16, 4096, 4096, 32, torch.float16),
    (1, 32, 8, 8192, 8192, 64, torch.float16),   # GQA: heads permuted so a group shares an XCD
    (2, 16, 16, 8192, 8192, 64, torch.bfloat16),
    (4, 16, 16, 4000, 4096, 64, torch.float16),  # ragged last query tile, more keys
    (8, 8, 2, 4096, 6000, 64, torch.float16),    # cross-attention, GQA
], ids=lambda c: "x".join(str(x) for x in c[:6]) + f"-{str(c[6])[6:]}")
def test_persistent_forward_plan_matches_grid_bitwise(case):
    """Under the causal mask the plan variant runs each (query tile, head) job
    with the grid form's code, in another order on a persistent grid: O and LSE
    equal the grid form's bit for bit (so every job ran once). On a 256-CU
    MI355X these shapes get a plan; the grid form itself is checked against
    the oracle elsewhere, and here against the fp32 reference on a few heads."""
    B, Hq, Hkv, N, Nkv, D, dt = case
    tag = f"plan forward B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} {dt}"
    _note(tag)
    q, k, v, _ = make_inputs(B, Hq, Hkv, N, D, seed=N + D, n_kv=Nkv)
    qd, kd, vd = (t.to(DEV).to(dt) for t in (q, k, v))
    scale = D ** -0.5
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    outs = {}
    for var in (FWD_GRID_VARIANT, FWD_PLAN_VARIANT):
        _lib.set_tiling(_lib.KERNEL_FWD, D, True, var)
        try:
            info = _lib.fwd_plan_info(B, Hq, Hkv, N, Nkv, D, True)
            outs[var] = _ops.flash_fwd(qd, kd, vd, True, scale)
        finally:
            _lib.set_tiling(_lib.KERNEL_FWD, D, True, -1)
        if var == FWD_PLAN_VARIANT:
            _note(f"  plan: {info}")
            if cus == 256:
                assert info["plan_workgroups"] == 768, info
                assert 0 < info["plan_makespan"] < info["grid_makespan"], info
        else:
            assert info["plan_workgroups"] == 0, info
    torch.cuda.synchronize()
    (o_g, lse_g), (o_p, lse_p) = outs[FWD_GRID_VARIANT], outs[FWD_PLAN_VARIANT]
    assert torch.equal(o_p, o_g), tag + ": O differs from the grid form"
    assert torch.equal(lse_p, lse_g), tag + ": LSE differs from the grid form"
    # a few heads against plain fp32 attention (top-left causal mask: query i
    # sees keys 0..i, as SDPA's is_causal for any N_q, N_kv)
    mask = torch.ones((N, Nkv), device=DEV, dtype=torch.bool).triu_(1)
    for h in (0, Hq // 2, Hq - 1):
        kvh = h // (Hq // Hkv)
        s = torch.matmul(qd[0, h].float(), kd[0, kvh].float().t().contiguous()) * scale
        s = s.masked_fill(mask, float("-inf"))
        lse_ref = torch.logsumexp(s, dim=-1) * (1.0 / math.log(2.0))
        o_ref = torch.matmul(torch.softmax(s, dim=-1), vd[0, kvh].float())
        assert_close(f"{tag} head {h} o vs fp32", o_p[0, h].double().cpu().numpy(),
                     o_ref.double().cpu().numpy())
        lse_err = float((lse_p[0, h] - lse_ref).abs().max())
        assert lse_err <= LSE_TOL, f"{tag} head {h} lse vs fp32: {lse_err:.3e}"


def test_whole_backward_without_a_workspace_runs_one_pass():
    """fa_bwd with no workspace on a shape that would take the combined plan
    runs every launch in one pass (fused-Delta dQ, unsplit dK/dV): the same
    results as those launches, within tolerance of the combined plan."""
    B, Hq, Hkv, N, D = 1, 8, 2, 1500, 64
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=77))
    lib = _lib.load()
    o, lse = _ops.flash_fwd(q, k, v, True, 0.125)
    delta, dq, dk, dv = (torch.empty((B, Hq, N), device=DEV), torch.empty_like(q),
                         torch.empty_like(k), torch.empty_like(v))
    rc = lib.fa_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                    lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                    B, Hq, Hkv, N, N, D, 0.125, 1, None, 0, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    delta1, dq1 = _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, True, 0.125)
    dk1, dv1 = torch.empty_like(k), torch.empty_like(v)
    _lib.check(lib.fa_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
                               lse.data_ptr(), delta1.data_ptr(), dk1.data_ptr(), dv1.data_ptr(),
                               B, Hq, Hkv, N, D, 0.125, 1, torch.cuda.current_stream().cuda_stream))
    dq2, dk2, dv2 = _ops.flash_bwd(q, k, v, o, lse, do, True, 0.125)  # combined plan
    torch.cuda.synchronize()
    assert torch.equal(delta, delta1) and torch.equal(dq, dq1)
    assert torch.equal(dk, dk1) and torch.equal(dv, dv1)
    for name, a, b in (("dq", dq, dq2), ("dk", dk, dk2), ("dv", dv, dv2)):
        assert_close(f"one pass vs combined {name}", a.float(), b.float(), max_abs=2e-3,
                     rel_l2=1e-3)


def test_short_query_dq_rule_matches_oracle_and_the_pipelined_tiling():
    """dQ at D = 128 without the mask runs the classic tiling for fewer than
    128 queries (a shape rule over the table): results agree with the oracle
    and, to fp32 summation order, with the table's pipelined tiling forced by
    fa_set_tiling, in one pass and with the split dQ."""
    for (B, Hq, Hkv, N, Nkv) in [(2, 8, 2, 16, 700), (1, 32, 8, 40, 6000)]:
        tag = f"short-query dq B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D=128"
        print(tag, flush=True)
        q, k, v, do = make_inputs(B, Hq, Hkv, N, 128, seed=N + Nkv, mult=0.5, n_kv=Nkv)
        got = run_kernel(q, k, v, do, False)
        check_against_oracle(got, q, k, v, do, False, tag=tag)
        qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
        o, lse = _ops.flash_fwd(qd, kd, vd, False, 128 ** -0.5)
        delta_rule, dq_rule = _ops.flash_bwd_dq_delta(qd, kd, vd, o, dod, lse, False, 128 ** -0.5)
        _lib.set_tiling(_lib.KERNEL_DQ, 128, False, 4)
        try:
            delta_pipe, dq_pipe = _ops.flash_bwd_dq_delta(qd, kd, vd, o, dod, lse, False,
                                                          128 ** -0.5)
        finally:
            _lib.set_tiling(_lib.KERNEL_DQ, 128, False, -1)
        torch.cuda.synchronize()
        assert_close(tag + " dq rule vs pipelined", dq_rule.float(), dq_pipe.float(),
                     max_abs=2e-3, rel_l2=1e-3)
        torch.testing.assert_close(delta_rule, delta_pipe, rtol=1e-5, atol=1e-5, msg=tag)


def test_short_query_dkdv_rule_at_d128_runs_the_classic_tiling():
    """dK/dV at D = 128 without the mask runs the classic 4 x 32 tiling (at two
    waves per SIMD) for at most 128 queries: the public API's dK, dV agree with
    the oracle, the op layer's are bit-identical to that tiling forced by
    fa_set_tiling (the table's pipelined tiling 4 past 128 queries and under
    the mask) and agree with the other to fp32 summation order, and the
    whole backward (fa_bwd) gives the same. One pass and split launches, fp16
    and bf16."""
    cases = [(8, 32, 8, 16, 2048, False, torch.float16, True),  # 1024 key tiles: one pass
             (2, 8, 2, 100, 700, False, torch.float16, True),
             (1, 32, 1, 128, 600, False, torch.float16, True),  # 5 key tiles: 4 chunks
             (1, 8, 8, 128, 1500, False, torch.float16, True),
             (1, 8, 2, 129, 1000, False, torch.float16, False),
             (2, 8, 2, 64, 900, True, torch.float16, False),
             (2, 8, 2, 64, 900, False, torch.bfloat16, True)]
    for (B, Hq, Hkv, N, Nkv, causal, dtype, takes) in cases:
        D = 128
        tag = f"short-query dkdv rule B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} causal={causal} {dtype}"
        _note(tag)
        q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + Nkv, mult=0.5, n_kv=Nkv, dtype=dtype)
        if dtype == torch.float16:
            check_against_oracle(run_kernel(q, k, v, do, causal), q, k, v, do, causal, tag=tag)
        qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
        scale = D ** -0.5
        o, lse = _ops.flash_fwd(qd, kd, vd, causal, scale)
        delta = _ops.flash_bwd_preprocess(o, dod)
        rule = _ops.flash_bwd_dkdv(qd, kd, vd, dod, lse, delta, causal, scale)
        whole = _ops.flash_bwd(qd, kd, vd, o, lse, dod, causal, scale)
        forced = {}
        for variant in (1, 4):
            _lib.set_tiling(_lib.KERNEL_DKDV, D, causal, variant)
            try:
                forced[variant] = _ops.flash_bwd_dkdv(qd, kd, vd, dod, lse, delta, causal, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_DKDV, D, causal, -1)
        torch.cuda.synchronize()
        same = forced[1] if takes else forced[4]
        assert torch.equal(rule[0], same[0]) and torch.equal(rule[1], same[1]), tag
        tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
            dict(max_abs=1e-2, rel_l2=4e-3)
        for i, name in ((0, "dk"), (1, "dv")):
            assert_close(f"{tag} {name} classic vs pipelined", forced[1][i].float(),
                         forced[4][i].float(), **tol)
            assert_close(f"{tag} {name} whole backward", whole[i + 1].float(), rule[i].float(),
                         **tol)


@pytest.mark.parametrize("head_dim", [32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_pipelined_dq_waves_without_queries_match_oracle(head_dim, causal):
    """The pipelined dQ tilings (4, and its 16x16x32 form 5) with waves that own
    no query row: 16, 40 and 96 queries leave 3, 2 and 1 of a 128-row
    work-group's four 32-row waves empty. Those waves only feed the shared K/V
    ring. dQ and Delta against the oracle, in split mode (16 and 96 queries
    against 4096 and 2500 keys) and in one pass (40 against 300), and the two
    tilings against each other."""
    scale = head_dim ** -0.5
    for B, Hq, Hkv, N, Nkv in ((1, 4, 1, 16, 4096), (2, 4, 2, 40, 300), (1, 2, 1, 96, 2500)):
        q, k, v, do = make_inputs(B, Hq, Hkv, N, head_dim, seed=3 * N + Nkv, mult=0.5, n_kv=Nkv)
        qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
        o, lse = _ops.flash_fwd(qd, kd, vd, causal, scale)
        torch.cuda.synchronize()
        ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal, scale,
                               o16=o.cpu().numpy(), fold_bwd=True)
        got = {}
        for var in (4, 5):
            tag = f"dq variant {var} B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={head_dim} " \
                  f"causal={causal}"
            _note(tag)
            _lib.set_tiling(_lib.KERNEL_DQ, head_dim, causal, var)
            try:
                delta, dq = _ops.flash_bwd_dq_delta(qd, kd, vd, o, dod, lse, causal, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_DQ, head_dim, causal, -1)
            torch.cuda.synchronize()
            assert_close(tag, dq.double().cpu().numpy(), ref["dq"])
            d_err = float(np.max(np.abs(delta.double().cpu().numpy() - ref["delta"])))
            assert d_err <= 1e-4, f"{tag} delta {d_err:.3e}"
            got[var] = dq
        assert_close(f"D={head_dim} N_q={N} dq variant 4 vs 5", got[4].float(), got[5].float(),
                     max_abs=2e-3, rel_l2=1e-3)


def test_causal_dq_rule_at_d128_matches_oracle_and_the_classic_tiling():
    """dQ at D = 128 under the mask runs the pipelined tiling for launches of at
    most 768 work-groups of 128 queries (a shape rule over the table's classic
    4 x 32 tiling): results agree with the oracle and, to fp32 summation order,
    with the classic tiling forced by fa_set_tiling, self- and cross-attention,
    fp16 and bf16, one pass and with the split dQ."""
    for (B, Hq, Hkv, N, Nkv, dtype) in [(1, 4, 1, 300, 300, torch.float16),
                                        (2, 8, 2, 129, 700, torch.float16),
                                        (1, 2, 2, 777, 777, torch.bfloat16),
                                        (1, 4, 2, 128, 9000, torch.float16)]:
        tag = f"causal dq rule B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D=128 {dtype}"
        print(tag, flush=True)
        q, k, v, do = make_inputs(B, Hq, Hkv, N, 128, seed=N + Nkv + 1, mult=0.5, n_kv=Nkv,
                                  dtype=dtype)
        if dtype == torch.float16:
            got = run_kernel(q, k, v, do, True)
            check_against_oracle(got, q, k, v, do, True, tag=tag)
        qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
        o, lse = _ops.flash_fwd(qd, kd, vd, True, 128 ** -0.5)
        delta_rule, dq_rule = _ops.flash_bwd_dq_delta(qd, kd, vd, o, dod, lse, True, 128 ** -0.5)
        _lib.set_tiling(_lib.KERNEL_DQ, 128, True, 1)
        try:
            delta_cl, dq_cl = _ops.flash_bwd_dq_delta(qd, kd, vd, o, dod, lse, True, 128 ** -0.5)
        finally:
            _lib.set_tiling(_lib.KERNEL_DQ, 128, True, -1)
        torch.cuda.synchronize()
        tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
            dict(max_abs=1e-2, rel_l2=4e-3)
        assert_close(tag + " dq rule vs classic", dq_rule.float(), dq_cl.float(), **tol)
        torch.testing.assert_close(delta_rule, delta_cl, rtol=1e-5, atol=1e-5, msg=tag)


def test_dq_rule_runs_the_16x16_tiling():
    """dQ launches of at least 769 work-groups of 128 queries run the pipelined
    tiling on 16x16x32 MFMAs (tiling 5) at D = 64, and at D = 32 without the
    mask: the rule's result is bit-identical to the tiling it should take
    forced by fa_set_tiling (5 there, the table's 4 for D = 32 under the mask)
    and agrees with the other to fp32 summation order. Then, through the public
    API at a small launch with tiling 5 set, against the oracle. fp16 and bf16,
    MHA and GQA, ragged N."""
    for (B, Hq, Hkv, N, D, causal, dtype, takes) in [
            (4, 16, 16, 4096, 64, False, torch.float16, True),
            (4, 16, 16, 4000, 64, True, torch.float16, True),
            (2, 32, 8, 1600, 64, False, torch.bfloat16, True),
            (4, 16, 16, 4096, 32, False, torch.float16, True),
            (4, 16, 16, 4096, 32, True, torch.float16, False)]:
        assert (N + 127) // 128 * B * Hq >= 769
        tag = f"dq rule B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} {dtype}"
        print(tag, flush=True)
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + Hq, mult=0.5,
                                                       dtype=dtype))
        scale = D ** -0.5
        o, lse = _ops.flash_fwd(q, k, v, causal, scale)
        delta_rule, dq_rule = _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, causal, scale)
        forced = {}
        for variant in (5, 4):
            _lib.set_tiling(_lib.KERNEL_DQ, D, causal, variant)
            try:
                forced[variant] = _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, causal, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_DQ, D, causal, -1)
        torch.cuda.synchronize()
        same = forced[5] if takes else forced[4]
        assert torch.equal(dq_rule, same[1]) and torch.equal(delta_rule, same[0]), tag
        tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
            dict(max_abs=1e-2, rel_l2=4e-3)
        assert_close(tag + " dq 16x16 vs 32x32", forced[5][1].float(), forced[4][1].float(), **tol)
        torch.testing.assert_close(forced[5][0], forced[4][0], rtol=1e-5, atol=1e-5, msg=tag)
    # The 16x16 tiling through the public API against the oracle (GQA, ragged).
    for D, causal in ((64, False), (64, True), (32, False)):
        q, k, v, do = make_inputs(1, 6, 2, 333, D, seed=3033 + D, mult=0.5)
        _lib.set_tiling(_lib.KERNEL_DQ, D, causal, 5)
        try:
            got = run_kernel(q, k, v, do, causal)
        finally:
            _lib.set_tiling(_lib.KERNEL_DQ, D, causal, -1)
        check_against_oracle(got, q, k, v, do, causal,
                             tag=f"dq tiling 5 B1 Hq6 Hkv2 N333 D{D} causal={causal}")


def test_dkdv_rule_runs_the_16x16_tiling():
    """dK/dV launches that do not split run the pipelined tiling on 16x16x32
    MFMAs (tiling 5) at D = 64, and at D = 32 without the mask: the rule's dK,
    dV are bit-identical to the tiling it should take forced by fa_set_tiling
    (5 there; the table's 4 for a split launch and for D = 32 under the mask)
    and agree with the other to fp32 summation order; through the whole
    backward (fa_bwd) as well. fp16 and bf16, both masks, MHA and GQA."""
    cases = [(4, 16, 16, 4096, 64, True, torch.float16, True),
             (8, 32, 8, 2048, 64, False, torch.bfloat16, True),  # 1024 key tiles
             (2, 16, 4, 2049, 64, True, torch.float16, False),  # 136 key tiles: splits
             (4, 16, 16, 4096, 32, False, torch.float16, True),
             (4, 16, 16, 4096, 32, True, torch.float16, False)]
    for (B, Hq, Hkv, N, D, causal, dtype, takes) in cases:
        splits = (N + 127) // 128 * B * Hkv < 768
        assert takes == (not splits and (D == 64 or not causal))
        tag = f"dkdv rule B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} {dtype}"
        print(tag, flush=True)
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + B, mult=0.5,
                                                       dtype=dtype))
        scale = D ** -0.5
        o, lse = _ops.flash_fwd(q, k, v, causal, scale)
        delta = _ops.flash_bwd_preprocess(o, do)
        rule = _ops.flash_bwd_dkdv(q, k, v, do, lse, delta, causal, scale)
        whole = _ops.flash_bwd(q, k, v, o, lse, do, causal, scale)
        forced = {}
        for variant in (5, 4):
            _lib.set_tiling(_lib.KERNEL_DKDV, D, causal, variant)
            try:
                forced[variant] = _ops.flash_bwd_dkdv(q, k, v, do, lse, delta, causal, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_DKDV, D, causal, -1)
        torch.cuda.synchronize()
        same = forced[5] if takes else forced[4]
        assert torch.equal(rule[0], same[0]) and torch.equal(rule[1], same[1]), tag
        tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
            dict(max_abs=1e-2, rel_l2=4e-3)
        for i, name in ((0, "dk"), (1, "dv")):
            assert_close(f"{tag} {name} 16x16 vs 32x32", forced[5][i].float(), forced[4][i].float(),
                         **tol)
            assert_close(f"{tag} {name} whole backward", whole[i + 1].float(), rule[i].float(),
                         **tol)


def test_d32_causal_forward_rule_runs_the_16x16_tiling():
    """Causal forward launches at D = 32 from 512 queries that do not take the
    two-key-group tiling run tiling 6 on 16x16x32 MFMAs (tiling 10): O and LSE
    are bit-identical to the tiling the rule should take forced by
    fa_set_tiling (10, 8 for few heads, the table's 6 otherwise), and tiling 10
    agrees with 6 to fp32 summation order. Then tiling 10 through the public
    API against the oracle (GQA, ragged N, both masks, D = 32 and 64)."""
    for (B, Hq, Hkv, N, D, causal, dtype, expect) in [
            (4, 16, 16, 4096, 32, True, torch.float16, 10),
            (4, 16, 16, 4000, 32, True, torch.float16, 10),
            (32, 16, 4, 512, 32, True, torch.bfloat16, 10),
            (1, 16, 16, 8192, 32, True, torch.float16, 8),   # few heads: two key groups
            (64, 16, 16, 256, 32, True, torch.float16, 6),   # short queries
            (4, 16, 16, 4096, 32, False, torch.float16, 6),
            (4, 16, 16, 4096, 64, True, torch.float16, 6)]:
        tag = f"fwd rule B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} {dtype}"
        print(tag, flush=True)
        q, k, v, _ = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + B, dtype=dtype))
        scale = D ** -0.5
        rule = _ops.flash_fwd(q, k, v, causal, scale)
        forced = {}
        for variant in {expect, 10, 6}:
            _lib.set_tiling(_lib.KERNEL_FWD, D, causal, variant)
            try:
                forced[variant] = _ops.flash_fwd(q, k, v, causal, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_FWD, D, causal, -1)
        torch.cuda.synchronize()
        assert torch.equal(rule[0], forced[expect][0]) and \
            torch.equal(rule[1], forced[expect][1]), tag
        tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
            dict(max_abs=1e-2, rel_l2=4e-3)
        assert_close(tag + " o 16x16 vs 32x32", forced[10][0].float(), forced[6][0].float(), **tol)
        assert float((forced[10][1] - forced[6][1]).abs().max()) <= 1e-5, tag
    for D, causal in ((32, True), (32, False), (64, True)):
        q, k, v, do = make_inputs(1, 6, 2, 333, D, seed=4044 + D)
        _lib.set_tiling(_lib.KERNEL_FWD, D, causal, 10)
        try:
            got = run_kernel(q, k, v, do, causal)
        finally:
            _lib.set_tiling(_lib.KERNEL_FWD, D, causal, -1)
        check_against_oracle(got, q, k, v, do, causal,
                             tag=f"fwd tiling 10 B1 Hq6 Hkv2 N333 D{D} causal={causal}")


def test_small_causal_forward_rule_runs_the_64_query_tiling():
    """Causal launches at D <= 64 of at least 2048 queries whose 128-query
    work-groups W number 384-512, or 256-512 with at most 4096 queries, run
    the 16x16x32 forward with 64-query work-groups (tiling 11): O and LSE are
    bit-identical to the tiling the rule should take forced by fa_set_tiling
    (11 there; the other rules' 6 or 8 at the boundaries), and tiling 11
    agrees with 6 to fp32 summation order. Then tiling 11 through the public
    API against the oracle (GQA, ragged N, both masks, D = 32 and 64)."""
    for (B, Hq, Hkv, N, D, dtype, expect) in [
            (1, 16, 16, 2048, 64, torch.float16, 11),   # W = 256, N <= 4096
            (1, 8, 8, 4096, 64, torch.bfloat16, 11),    # W = 256
            (1, 24, 12, 2048, 64, torch.float16, 11),   # W = 384, GQA
            (1, 16, 16, 4096, 32, torch.float16, 11),   # W = 512 (not two key groups)
            (1, 4, 4, 8192, 64, torch.float16, 6),      # W = 256 with N > 4096: split-KV
            (1, 4, 4, 8192, 32, torch.float16, 8),      # the same at D = 32: two key groups
            (2, 16, 4, 2049, 64, torch.float16, 6),     # c3: W = 544
            (1, 32, 8, 1024, 64, torch.float16, 6)]:    # N < 2048
        tag = f"fwd rule B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal {dtype}"
        print(tag, flush=True)
        q, k, v, _ = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + Hq, dtype=dtype))
        scale = D ** -0.5
        rule = _ops.flash_fwd(q, k, v, True, scale)
        forced = {}
        for variant in {expect, 11, 6}:
            _lib.set_tiling(_lib.KERNEL_FWD, D, True, variant)
            try:
                forced[variant] = _ops.flash_fwd(q, k, v, True, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_FWD, D, True, -1)
        torch.cuda.synchronize()
        assert torch.equal(rule[0], forced[expect][0]) and \
            torch.equal(rule[1], forced[expect][1]), tag
        tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
            dict(max_abs=1e-2, rel_l2=4e-3)
        assert_close(tag + " o 64- vs 128-query", forced[11][0].float(), forced[6][0].float(), **tol)
        assert float((forced[11][1] - forced[6][1]).abs().max()) <= 1e-5, tag
    for D, causal in ((32, True), (32, False), (64, True), (64, False)):
        q, k, v, do = make_inputs(1, 6, 2, 333, D, seed=5055 + D)
        _lib.set_tiling(_lib.KERNEL_FWD, D, causal, 11)
        try:
            got = run_kernel(q, k, v, do, causal)
        finally:
            _lib.set_tiling(_lib.KERNEL_FWD, D, causal, -1)
        check_against_oracle(got, q, k, v, do, causal,
                             tag=f"fwd tiling 11 B1 Hq6 Hkv2 N333 D{D} causal={causal}")


def test_decoding_forward_rule_runs_the_64_query_tiling():
    """Launches of at most 32 queries (decoding, any head size) whose queries fit
    one 64-query work-group of packed heads (N_q <= 64 / P, P = gcd(Hq / Hkv,
    4) heads per work-group) run tiling 11: O and LSE are bit-identical to
    tiling 11 forced (past that bound to tiling 6, and at D = 128 to the
    4-wave tiling 2 that short queries take),
    tiling 11 agrees with 6 to fp32 summation order and, at a small shape,
    matches the oracle. Split-KV (long keys) and packed GQA included. Without
    the mask 33-64 queries (one 64-query work-group per head, no packing) take
    it too; under the mask they keep the previous choice."""
    for (B, Hq, Hkv, Nq, Nkv, D, dtype, expect) in [
            (8, 32, 8, 1, 8192, 64, torch.float16, 11),     # P = 4: up to 16 queries
            (8, 32, 8, 16, 8192, 64, torch.bfloat16, 11),
            (8, 32, 8, 17, 8192, 64, torch.float16, 6),     # two query tiles per head
            (4, 16, 8, 32, 4096, 32, torch.float16, 11),    # P = 2: up to 32 queries
            (2, 16, 16, 32, 16384, 64, torch.float16, 11),  # MHA, split keys
            (8, 32, 8, 1, 8192, 128, torch.float16, 11),    # D = 128: 96 KiB ring
            (4, 16, 16, 32, 4096, 128, torch.bfloat16, 11),
            (8, 32, 8, 17, 8192, 128, torch.float16, 2),    # past the bound: short-query rule
            (8, 32, 8, 48, 8192, 64, torch.float16, 11),    # 33-64 queries: one work-group
            (1, 32, 8, 64, 32768, 128, torch.bfloat16, 11),  # per head, split keys
            (4, 16, 16, 40, 16384, 32, torch.float16, 11),
            (8, 32, 8, 65, 8192, 64, torch.float16, 6),     # two query tiles per head
            (4, 32, 8, 96, 8192, 128, torch.float16, 2)]:
        tag = f"decode rule B={B} Hq={Hq} Hkv={Hkv} N_q={Nq} N_kv={Nkv} D={D} {dtype}"
        print(tag, flush=True)
        q, k, v, _ = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, Nq, D, seed=Nq + Nkv + D,
                                                       n_kv=Nkv, dtype=dtype))
        scale = D ** -0.5
        rule = _ops.flash_fwd(q, k, v, False, scale)
        forced = {}
        base = 6 if D <= 64 else 2  # the 128-query tiling decoding took before
        for variant in ({expect, base} if expect == 11 else {expect}):
            _lib.set_tiling(_lib.KERNEL_FWD, D, False, variant)
            try:
                forced[variant] = _ops.flash_fwd(q, k, v, False, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_FWD, D, False, -1)
        torch.cuda.synchronize()
        same = forced[expect]
        assert torch.equal(rule[0], same[0]) and torch.equal(rule[1], same[1]), tag
        if expect == 11:
            tol = dict(max_abs=2e-3, rel_l2=1e-3) if dtype == torch.float16 else \
                dict(max_abs=1e-2, rel_l2=4e-3)
            assert_close(tag + " o 64- vs 128-query", rule[0].float(), forced[base][0].float(),
                         **tol)
            assert float((rule[1] - forced[base][1]).abs().max()) <= 1e-5, tag
    for D in (64, 128):
        q, k, v, do = make_inputs(2, 8, 2, 5, D, seed=6066 + D, n_kv=777)
        got = run_kernel(q, k, v, do, False)
        check_against_oracle(got, q, k, v, do, False, tag=f"decode B2 Hq8 Hkv2 N_q5 N_kv777 D{D}")
    q, k, v, do = make_inputs(2, 8, 2, 50, 128, seed=6166, n_kv=900)
    got = run_kernel(q, k, v, do, False)
    check_against_oracle(got, q, k, v, do, False, tag="short queries B2 Hq8 Hkv2 N_q50 N_kv900 D128")
    # under the mask 33-64 queries keep the 128-query tiling
    q, k, v, _ = (t.to(DEV) for t in make_inputs(4, 16, 4, 48, 64, seed=48, n_kv=4096))
    rule = _ops.flash_fwd(q, k, v, True, 0.125)
    _lib.set_tiling(_lib.KERNEL_FWD, 64, True, 6)
    try:
        forced6 = _ops.flash_fwd(q, k, v, True, 0.125)
    finally:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, -1)
    torch.cuda.synchronize()
    assert torch.equal(rule[0], forced6[0]) and torch.equal(rule[1], forced6[1])


def test_forward_without_grad_matches_the_autograd_path():
    """Inputs that need no gradient (or calls under torch.no_grad()) take the
    forward launch without the autograd Function: bit-identical output, no
    graph, for native and zero-padded head sizes, fp16 and bf16, GQA."""
    for (B, Hq, Hkv, N, Nkv, D, Dv, dtype) in [(2, 8, 2, 300, 300, 64, 64, torch.float16),
                                               (1, 4, 4, 77, 500, 40, 40, torch.bfloat16),
                                               (1, 6, 3, 129, 129, 64, 32, torch.float16)]:
        q, k, v, _ = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N + D, n_kv=Nkv,
                                                      d_v=Dv, dtype=dtype))
        gqa = Hq != Hkv
        with_grad = scaled_dot_product_attention(
            q.clone().requires_grad_(), k.clone().requires_grad_(), v.clone().requires_grad_(),
            is_causal=True, enable_gqa=gqa, backend="triton")
        plain = scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=gqa,
                                             backend="triton")
        with torch.no_grad():
            no_grad = scaled_dot_product_attention(q.clone().requires_grad_(), k, v,
                                                   is_causal=True, enable_gqa=gqa,
                                                   backend="triton")
        assert with_grad.grad_fn is not None
        assert plain.grad_fn is None and no_grad.grad_fn is None
        assert plain.shape == no_grad.shape == with_grad.shape == (B, Hq, N, Dv)
        assert torch.equal(plain, with_grad.detach()) and torch.equal(no_grad, plain)


def test_forward_mode_ad_is_not_silently_dropped():
    """Dual tensors carry tangents without requires_grad: the call goes through
    the autograd Function, which defines no jvp (as the reference's), so it
    raises rather than returning an output without a tangent."""
    import torch.autograd.forward_ad as fwAD

    q, k, v, _ = (t.to(DEV) for t in make_inputs(1, 2, 2, 64, 64, seed=5))
    with fwAD.dual_level():
        qd = fwAD.make_dual(q, torch.randn_like(q))
        with pytest.raises(RuntimeError):
            scaled_dot_product_attention(qd, k, v, is_causal=True, backend="triton")


def test_two_threads_on_their_own_streams_match_sequential_results():
    """The op layer launches on the calling thread's current stream and the
    library keeps no per-call global state: two threads, each on its own
    stream (default priority), running fwd + bwd concurrently on different
    inputs (one taking the split paths) reproduce the sequential results
    bit for bit."""
    import threading

    shapes = [(2, 8, 2, 333, 333, 64, True), (1, 32, 8, 16, 5000, 128, False)]
    inputs = []
    for i, (B, Hq, Hkv, N, Nkv, D, causal) in enumerate(shapes):
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=80 + i, n_kv=Nkv))
        inputs.append((q, k, v, do, causal, D ** -0.5))

    def step(q, k, v, do, causal, scale):
        o, lse = _ops.flash_fwd(q, k, v, causal, scale)
        return (o, lse) + tuple(_ops.flash_bwd(q, k, v, o, lse, do, causal, scale))

    want = [step(*args) for args in inputs]
    torch.cuda.synchronize()
    got = [None, None]
    errors = []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for _ in range(5):
                    out = step(*inputs[i])
                stream.synchronize()
            got[i] = out
        except Exception as exc:  # reported on the main thread
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not errors, errors
    assert all(not th.is_alive() for th in threads)
    for i in range(2):
        for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), got[i], want[i]):
            assert torch.equal(a, b), f"thread {i} {name} differs from the sequential result"


def test_tiling_sweep_times_every_variant_and_restores_the_table():
    """benchmarks.tiling_sweep times each compiled tiling of each kernel once,
    marks the table's choice, and leaves the table selected afterwards."""
    from benchmarks.tiling_sweep import sweep

    before = {k: _lib.get_tiling(k, 64, True)["variant"]
              for k in (_lib.KERNEL_FWD, _lib.KERNEL_DKDV, _lib.KERNEL_DQ)}
    rows = sweep(batch=1, query_heads=4, kv_heads=2, seq_len=300, head_dim=64, causal=True,
                 kernels=["fwd", "dkdv", "dq"], reps=2)
    for name, kind in (("fwd", _lib.KERNEL_FWD), ("dkdv", _lib.KERNEL_DKDV), ("dq", _lib.KERNEL_DQ)):
        mine = [r for r in rows if r["kernel"] == name]
        assert [r["variant"] for r in mine] == [t["variant"] for t in _lib.tiling_variants(kind, 64, True)]
        assert sum(r["table"] for r in mine) == 1
        assert all(r["us"] > 0 and r["tflops_executed"] > 0 for r in mine)
        assert _lib.get_tiling(kind, 64, True)["variant"] == before[kind]
    # bf16, restricted to named tilings (both have bf16 builds)
    rows = sweep(batch=1, query_heads=4, kv_heads=2, seq_len=300, head_dim=64, causal=True,
                 kernels=["fwd"], reps=2, dtype=torch.bfloat16, variants=[6, 10])
    assert [r["variant"] for r in rows] == [6, 10] and all(r["us"] > 0 for r in rows)
    assert _lib.get_tiling(_lib.KERNEL_FWD, 64, True)["variant"] == before[_lib.KERNEL_FWD]


def test_tiling_ab_alternates_tilings_and_restores_the_table():
    """benchmarks.tiling_ab times the named tilings in interleaved rounds and
    reports medians and ratios to the first; the table is selected afterwards."""
    from benchmarks.tiling_ab import ab, parse_shape

    for kernel, kind, variants in (("fwd", _lib.KERNEL_FWD, [6, 10]), ("dq", _lib.KERNEL_DQ, [4, 5])):
        before = _lib.get_tiling(kind, 32, True)["variant"]
        r = ab(kernel, variants, parse_shape("1,4,2,300,32,causal,bfloat16"), rounds=2, reps=2)
        assert sorted(r["us"]) == sorted(str(v) for v in variants)
        assert r["ratio"][str(variants[0])] == 1.0 and all(x > 0 for x in r["us"].values())
        assert _lib.get_tiling(kind, 32, True)["variant"] == before


@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_every_tiling_variant_matches_oracle(head_dim, causal):
    """Each compiled tiling of each kernel (fwd, dK/dV single-pass and split,
    dQ) against the oracle on a ragged GQA shape, not only the defaults."""
    B, Hq, Hkv, N, D = 1, 8, 1, 520, head_dim
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=77, mult=0.5)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    scale = D ** -0.5
    lib = _lib.load()
    # the op layer's dK/dV (dk1, dv1 below) takes the split path on this shape
    assert lib.fa_bwd_dkdv_workspace_bytes(B, Hq, Hkv, N, D, int(causal)) > 0
    stream = torch.cuda.current_stream().cuda_stream
    o, lse = _ops.flash_fwd(qd, kd, vd, causal, scale)
    delta = _ops.flash_bwd_preprocess(o, dod)
    torch.cuda.synchronize()
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal, scale,
                           o16=o.cpu().numpy(), fold_bwd=True)

    def close(tag, got, name):
        assert_close(tag, torch.as_tensor(got).double().cpu().numpy(), ref[name])

    kinds = ((_lib.KERNEL_FWD, "fwd"), (_lib.KERNEL_DKDV, "dkdv"), (_lib.KERNEL_DQ, "dq"))
    for kind, kname in kinds:
        for var in _lib.tiling_variants(kind, D, causal):
            tag = f"D={D} causal={causal} {kname} variant {var['variant']} " \
                  f"({var['waves']} waves, tile {var['tile']})"
            _note(tag)
            _lib.set_tiling(kind, D, causal, var["variant"])
            try:
                if kind == _lib.KERNEL_FWD:
                    o2, lse2 = _ops.flash_fwd(qd, kd, vd, causal, scale)
                    torch.cuda.synchronize()
                    close(tag + " o", o2, "o")
                    lse_err = float(np.max(np.abs(lse2.double().cpu().numpy() - ref["lse"])))
                    assert lse_err <= LSE_TOL, f"{tag} lse {lse_err:.3e}"
                elif kind == _lib.KERNEL_DKDV:
                    dk1, dv1 = _ops.flash_bwd_dkdv(qd, kd, vd, dod, lse, delta, causal, scale)
                    dk2, dv2 = torch.empty_like(kd), torch.empty_like(vd)
                    _lib.check(lib.fa_bwd_dkdv(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                               dod.data_ptr(), lse.data_ptr(), delta.data_ptr(),
                                               dk2.data_ptr(), dv2.data_ptr(), B, Hq, Hkv, N, D,
                                               scale, int(causal), stream))
                    torch.cuda.synchronize()
                    close(tag + " dk (split)", dk1, "dk")
                    close(tag + " dv (split)", dv1, "dv")
                    close(tag + " dk", dk2, "dk")
                    close(tag + " dv", dv2, "dv")
                else:
                    dq = _ops.flash_bwd_dq(qd, kd, vd, dod, lse, delta, causal, scale)
                    torch.cuda.synchronize()
                    close(tag + " dq", dq, "dq")
            finally:
                _lib.set_tiling(kind, D, causal, -1)


@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_fused_delta_matches_separate_launches(head_dim):
    """fa_bwd_dq_delta (Delta inside the dQ launch where the tiling supports
    it, else preprocess + dQ) agrees with fa_bwd_preprocess followed by
    fa_bwd_dq, for the default tiling and for another compiled tiling."""
    B, Hq, Hkv, N, D = 2, 4, 2, 333, head_dim
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=31, mult=0.5))
    scale = D ** -0.5
    for causal in (False, True):
        o, lse = _ops.flash_fwd(q, k, v, causal, scale)
        delta_ref = _ops.flash_bwd_preprocess(o, do)
        dq_ref = _ops.flash_bwd_dq(q, k, v, do, lse, delta_ref, causal, scale)
        default = _lib.get_tiling(_lib.KERNEL_DQ, D, causal)["variant"]
        other = [t["variant"] for t in _lib.tiling_variants(_lib.KERNEL_DQ, D, causal)
                 if t["variant"] != default][0]  # a classic tiling: preprocess + dQ
        for variant in (-1, other):
            _lib.set_tiling(_lib.KERNEL_DQ, D, causal, variant)
            try:
                delta, dq = _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, causal, scale)
            finally:
                _lib.set_tiling(_lib.KERNEL_DQ, D, causal, -1)
            torch.cuda.synchronize()
            tag = f"D={D} causal={causal} dq variant {variant}"
            torch.testing.assert_close(delta, delta_ref, rtol=1e-5, atol=1e-5, msg=tag)
            assert_close(f"{tag} dq", dq.float(), dq_ref.float(), max_abs=2e-3, rel_l2=1e-3)


def test_deterministic_backward():
    q, k, v, do = make_inputs(2, 8, 2, 333, 64, seed=9)
    a = run_kernel(q, k, v, do, True)
    b = run_kernel(q, k, v, do, True)
    for name in ("o", "lse", "dq", "dk", "dv"):
        assert np.array_equal(a[name], b[name]), f"{name} differs between identical runs"


def test_strided_inputs_are_made_contiguous():
    q, k, v, do = make_inputs(1, 2, 2, 96, 64, seed=10)
    qs = q.transpose(1, 2).contiguous().transpose(1, 2)  # same values, non-contiguous
    assert not qs.is_contiguous()
    got = run_kernel(qs, k, v, do, False)
    check_against_oracle(got, q, k, v, do, False, tag="strided q")


def test_dispatch_selects_custom_kernel_on_gfx950():
    q = torch.randn(1, 2, 64, 64, device=DEV, dtype=torch.float16)
    decision = explain_dispatch(q, q, q)
    assert decision.backend == "triton", decision.reason
    q32 = q.float()
    assert explain_dispatch(q32, q32, q32).backend == "torch"
    q160 = torch.randn(1, 2, 64, 160, device=DEV, dtype=torch.float16)
    assert explain_dispatch(q160, q160, q160).backend == "torch"
    q48 = torch.randn(1, 2, 64, 48, device=DEV, dtype=torch.float16)
    assert "zero-padded to 64" in explain_dispatch(q48, q48, q48).reason
    out = scaled_dot_product_attention(q32, q32, q32)  # auto falls back to SDPA
    ref = torch.nn.functional.scaled_dot_product_attention(q32, q32, q32)
    torch.testing.assert_close(out, ref)
    with pytest.raises(RuntimeError, match="float16"):
        scaled_dot_product_attention(q32, q32, q32, backend="triton")


# ---------------------------------------------------------------------------
# BASELINE configurations at full size.
# ---------------------------------------------------------------------------
def _config_cases():
    for name in ("c2", "c3", "c4", "c5"):
        for causal in CONFIGS[name]["causal"]:
            yield pytest.param(name, causal, id=f"{name}-{'causal' if causal else 'bidir'}")


@pytest.mark.parametrize("name,causal", list(_config_cases()))
def test_full_config_matches_fp32_reference(name, causal):
    cfg = CONFIGS[name]
    B, Hq, Hkv, N, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["N"], cfg["D"]
    _note(f"{name} causal={causal}: B={B} Hq={Hq} Hkv={Hkv} N={N} D={D}")
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, cfg["seed"], cfg["mult"])
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    qa, ka, va = (t.clone().requires_grad_() for t in (qd, kd, vd))
    out = scaled_dot_product_attention(qa, ka, va, is_causal=causal, enable_gqa=Hq != Hkv,
                                       backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qa, ka, va), dod)
    _, lse = _ops.flash_fwd(qd, kd, vd, causal, D ** -0.5)
    torch.cuda.synchronize()
    ref = torch_reference_fp32(qd, kd, vd, dod, causal, o16=out.detach())
    torch.cuda.synchronize()
    for tname, t in (("o", out.detach()), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.isfinite(t).all(), f"{name} {tname} has non-finite values"
        ma, rl = assert_close(f"{name} {tname}", t.float(), ref[tname])
        _note(f"  {tname}: max-abs {ma:.3e} rel-L2 {rl:.3e}")
    lse_err = float((lse - ref["lse"]).abs().max())
    _note(f"  lse: max-abs {lse_err:.3e}")
    assert lse_err <= LSE_TOL

    _check_oracle_slices(name, q, k, v, do, out.detach(), lse, dq, dk, dv, causal, ref["lse"])
    # The whole key/value head 0 group of batch 0 where the oracle finishes in
    # seconds (c2, c3): every row and key, full N.
    G = Hq // Hkv
    if N * N * D * G <= 2 ** 32:
        sl = slice(0, G)
        got = {
            "o16": out.detach()[:1, sl].cpu(),
            "o": out.detach()[:1, sl].double().cpu().numpy(),
            "lse": lse[:1, sl].double().cpu().numpy(),
            "dq": dq[:1, sl].double().cpu().numpy(),
            "dk": dk[:1, :1].double().cpu().numpy(),
            "dv": dv[:1, :1].double().cpu().numpy(),
        }
        check_against_oracle(got, q[:1, sl], k[:1, :1], v[:1, :1], do[:1, sl], causal,
                             tag=f"{name} oracle head group")


# Rows and keys of the fp64-oracle slices of the full configurations.
SLICE_FIRST_ROWS = 16
SLICE_LAST_ROWS = 64
SLICE_KEYS = 64


def _check_oracle_slices(name, q, k, v, do, out, lse, dq, dk, dv, causal, lse_fp32):
    """fp64-oracle checks on slices of a full configuration, for every GQA
    query head of batch 0's key/value head 0:
      * O, LSE and dQ of the first 16 and the last 64 query rows (the tail
        tile included). Under the causal mask row r sees keys 0..r, so each
        row is its own oracle call on those keys (unmasked); bidirectional
        rows take one call against every key.
      * dK and dV of the last 64 keys. Under the causal mask only the last 64
        queries see them, so the oracle's backward on the last 64 queries and
        keys (the top-left mask at equal offsets) is exact; bidirectional keys
        take every query. P comes from the independent fp32 PyTorch LSE and
        Delta from the kernel's stored O, as in the reference backward
        (attention.py:252-254).
    The backward uses the reference's fp16-rounded score operands (fold)."""
    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]
    hs = slice(0, G)
    f64 = lambda t: t.double().cpu().numpy()
    qh, kh, vh, doh = q[:1, hs], k[:1, :1], v[:1, :1], do[:1, hs]
    o16 = out[:1, hs].cpu()
    rows = sorted(set(range(min(SLICE_FIRST_ROWS, N))) | set(range(max(0, N - SLICE_LAST_ROWS), N)))
    got_o, got_lse, got_dq = f64(out[:1, hs, rows]), f64(lse[:1, hs, rows]), f64(dq[:1, hs, rows])
    if causal:
        parts = [oracle.attention(qh[:, :, r:r + 1].numpy(), kh[:, :, :r + 1].numpy(),
                                  vh[:, :, :r + 1].numpy(), doh[:, :, r:r + 1].numpy(), False,
                                  o16=o16[:, :, r:r + 1].numpy(), fold_bwd=True) for r in rows]
        ref = {t: np.concatenate([p[t] for p in parts], axis=2) for t in ("o", "lse", "dq")}
    else:
        ref = oracle.attention(qh[:, :, rows].numpy(), kh.numpy(), vh.numpy(),
                               doh[:, :, rows].numpy(), False, o16=o16[:, :, rows].numpy(),
                               fold_bwd=True)
    report = {}
    for t, got in (("o", got_o), ("dq", got_dq)):
        report[t] = assert_close(f"{name} oracle rows {t}", got, ref[t])
    lse_err = float(np.max(np.abs(got_lse - ref["lse"])))
    assert lse_err <= LSE_TOL, f"{name} oracle rows lse: {lse_err:.3e}"
    # dK, dV of the last SLICE_KEYS keys
    k0 = max(0, N - SLICE_KEYS)
    qrows = slice(k0, N) if causal else slice(0, N)
    delta = oracle.bwd_preprocess(o16[:, :, qrows].numpy(), doh[:, :, qrows].numpy())
    _, rdk, rdv = oracle.bwd(qh[:, :, qrows].numpy(), kh[:, :, k0:].numpy(), vh[:, :, k0:].numpy(),
                             doh[:, :, qrows].numpy(), f64(lse_fp32[:1, hs, qrows]), delta,
                             causal, fold=True)
    report["dk"] = assert_close(f"{name} oracle keys dk", f64(dk[:1, :1, k0:]), rdk)
    report["dv"] = assert_close(f"{name} oracle keys dv", f64(dv[:1, :1, k0:]), rdv)
    _note(f"  {name} fp64 oracle slices ({len(rows)} rows x {G} heads, {N - k0} keys): "
          + ", ".join(f"{t}={e[0]:.2e}/{e[1]:.2e}" for t, e in report.items())
          + f", lse={lse_err:.2e}")


# ---------------------------------------------------------------------------
# Committed golden vectors (tests/golden/attention_fp64.npz: torch fp64 SDPA,
# autograd and logsumexp, made without the oracle) against the HIP path.
# ---------------------------------------------------------------------------
def _golden():
    from pathlib import Path

    data = np.load(Path(__file__).resolve().parent / "golden" / "attention_fp64.npz")
    names = sorted({key.split("/")[0] for key in data.files if "/" in key})
    return data, names


def _golden_case(data, name):
    return {key.split("/")[1]: data[key] for key in data.files if key.startswith(name + "/")}


def test_config1_hip_path_matches_golden():
    """BASELINE configs[0] (B1 H4 N257 D64 bidirectional, seeded fp16 inputs)
    on the HIP path: the committed golden inputs, O against the golden fp64
    O and LSE against the golden base-2 LSE at the north-star tolerances."""
    data, _ = _golden()
    g = _golden_case(data, "config1_b1_h4_n257_d64_bidir")
    q, k, v = (torch.from_numpy(g[t]).to(DEV) for t in ("q", "k", "v"))
    assert tuple(q.shape) == (1, 4, 257, 64) and q.dtype == torch.float16
    assert explain_dispatch(q, k, v).backend == "triton"
    out = scaled_dot_product_attention(q, k, v, backend="triton")
    o2, lse = _ops.flash_fwd(q, k, v, False, 64 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, o2)
    ma, rl = assert_close("c1 o", out.double().cpu().numpy(), g["o"])
    lse_err = float(np.max(np.abs(lse.double().cpu().numpy() - g["lse2"])))
    assert lse_err <= LSE_TOL, f"c1 lse {lse_err:.3e}"
    # and the reference's own CPU path (fp16 SDPA on the CPU) on the same inputs
    cpu = torch.nn.functional.scaled_dot_product_attention(*(t.cpu() for t in (q, k, v)))
    assert_close("c1 o vs CPU SDPA", out.double().cpu(), cpu.double())
    _note(f"c1 HIP vs golden: o {ma:.2e}/{rl:.2e}, lse {lse_err:.2e}")


def test_every_golden_case_matches_on_the_hip_path():
    """Every committed golden case through the public API on the GPU: O, LSE,
    and (where the case has dO) dQ, dK, dV against the fp64 golden values."""
    data, names = _golden()
    assert len(names) >= 15
    for name in names:
        g = _golden_case(data, name)
        B, Hq, Hkv, N, D, causal = (int(x) for x in g["meta"])
        q, k, v = (torch.from_numpy(g[t]) for t in ("q", "k", "v"))
        qd, kd, vd = (t.to(DEV) for t in (q, k, v))
        o2, lse = _ops.flash_fwd(qd, kd, vd, bool(causal), D ** -0.5)
        report = {}
        if "do" in g:
            got = run_kernel(q, k, v, torch.from_numpy(g["do"]), bool(causal))
            for t in ("o", "dq", "dk", "dv"):
                report[t] = assert_close(f"golden {name} {t}", got[t], g[t])
        else:
            out = scaled_dot_product_attention(qd, kd, vd, is_causal=bool(causal),
                                               enable_gqa=Hq != Hkv, backend="triton")
            report["o"] = assert_close(f"golden {name} o", out.double().cpu().numpy(), g["o"])
        torch.cuda.synchronize()
        lse_err = float(np.max(np.abs(lse.double().cpu().numpy() - g["lse2"])))
        assert lse_err <= LSE_TOL, f"golden {name} lse: {lse_err:.3e}"
        _note(f"golden {name}: " + ", ".join(f"{t}={e[0]:.1e}/{e[1]:.1e}" for t, e in report.items())
              + f", lse={lse_err:.1e}")


# ---------------------------------------------------------------------------
# bfloat16, an element type this build adds (the reference sends bf16 to torch
# SDPA, attention.py:653-656). bf16's unit roundoff (2^-9) is 4x fp16's
# (2^-11), so O, dQ, dK, dV get 4x the fp16 tolerances; LSE is an fp32
# quantity of inputs that are exact in the oracle and keeps its tolerance.
# The backward is compared with the oracle's bf16-rounded score operands.
# ---------------------------------------------------------------------------
BF16_MAX_ABS_TOL = 4 * MAX_ABS_TOL
BF16_REL_L2_TOL = 4 * REL_L2_TOL


def check_bf16_against_oracle(got, q, k, v, do, causal, scale=None, tag=""):
    f = lambda t: t.float().numpy()
    ref = oracle.attention(f(q), f(k), f(v), f(do), causal, scale,
                           o16=got["o16"].float().numpy(), fold_bwd="bfloat16")
    report = {}
    for name in ("o", "dq", "dk", "dv"):
        report[name] = assert_close(f"{tag} {name}", got[name], ref[name],
                                    max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL)
    lse_err = float(np.max(np.abs(got["lse"] - ref["lse"])))
    assert lse_err <= LSE_TOL, f"{tag} lse: max-abs {lse_err:.3e} (tol {LSE_TOL:.0e})"
    _note(f"{tag}: " + ", ".join(f"{k}={v[0]:.2e}/{v[1]:.2e}" for k, v in report.items())
          + f", lse={lse_err:.2e}")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sequence", [17, 129])
@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_bf16_reference_shapes_match_oracle(sequence, head_dim, causal):
    q, k, v, do = make_inputs(1, 2, 2, sequence, head_dim, seed=123, mult=0.5, do_mult=0.1,
                              dtype=torch.bfloat16)
    got = run_kernel(q, k, v, do, causal)
    assert got["o16"].dtype == torch.bfloat16
    check_bf16_against_oracle(got, q, k, v, do, causal,
                              tag=f"bf16 N={sequence} D={head_dim} causal={causal}")


@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_bf16_gqa_tail_matches_oracle(head_dim):
    q, k, v, do = make_inputs(2, 6, 3, 300, head_dim, seed=55, dtype=torch.bfloat16)
    for causal in (False, True):
        got = run_kernel(q, k, v, do, causal)
        check_bf16_against_oracle(got, q, k, v, do, causal,
                                  tag=f"bf16 GQA 6->3 N=300 D={head_dim} causal={causal}")


def test_bf16_dispatch_selects_the_custom_kernel():
    q = torch.randn(1, 2, 64, 64, device=DEV, dtype=torch.bfloat16)
    d = explain_dispatch(q, q, q)
    assert d.backend == "triton" and "bfloat16" in d.reason


def test_bf16_full_c2_matches_fp32_reference():
    cfg = CONFIGS["c2"]
    B, Hq, Hkv, N, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["N"], cfg["D"]
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, cfg["seed"], cfg["mult"], dtype=torch.bfloat16)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    qa, ka, va = (t.clone().requires_grad_() for t in (qd, kd, vd))
    out = scaled_dot_product_attention(qa, ka, va, is_causal=True, backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qa, ka, va), dod)
    _, lse = _ops.flash_fwd(qd, kd, vd, True, D ** -0.5)
    torch.cuda.synchronize()
    ref = torch_reference_fp32(qd, kd, vd, dod, True, o16=out.detach())
    torch.cuda.synchronize()
    for tname, t in (("o", out.detach()), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert t.dtype == torch.bfloat16 and torch.isfinite(t).all()
        ma, rl = assert_close(f"bf16 c2 {tname}", t.float(), ref[tname],
                              max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL)
        _note(f"  bf16 c2 {tname}: max-abs {ma:.3e} rel-L2 {rl:.3e}")
    assert float((lse - ref["lse"]).abs().max()) <= LSE_TOL


# ---------------------------------------------------------------------------
# Cross-attention (N_q != N_kv): the reference sends it to torch SDPA
# (attention.py:639-642); the kernels compute that fallback's result, with
# SDPA's top-left causal mask, checked against the oracle's closed form (pinned
# to torch fp64 SDPA for unequal lengths on the CPU).
# ---------------------------------------------------------------------------
CROSS_CASES = [
    # (B, Hq, Hkv, N_q, N_kv): fewer queries than keys (GQA, split dK/dV),
    # more queries than keys, one query, one key
    (1, 8, 1, 600, 700),
    (2, 4, 4, 777, 129),
    (1, 2, 1, 1, 513),
    (1, 2, 2, 1000, 1),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("case", CROSS_CASES, ids=lambda c: f"B{c[0]}H{c[1]}-{c[2]}Nq{c[3]}Nkv{c[4]}")
def test_cross_attention_matches_oracle(case, head_dim, causal):
    B, Hq, Hkv, N, Nkv = case
    tag = f"cross B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={head_dim} causal={causal}"
    _note(tag)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, head_dim, seed=N + Nkv + head_dim, mult=0.5,
                              n_kv=Nkv)
    assert explain_dispatch(q.to(DEV), k.to(DEV), v.to(DEV),
                            enable_gqa=Hq != Hkv).backend == "triton"
    got = run_kernel(q, k, v, do, causal)
    assert got["dk"].shape == (B, Hkv, Nkv, head_dim)
    check_against_oracle(got, q, k, v, do, causal, tag=tag)
    if causal and N < Nkv:
        # keys past the last query are never seen: exactly zero gradients
        assert not got["dk"][:, :, N:].any() and not got["dv"][:, :, N:].any()


@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_cross_attention_every_tiling_variant(head_dim, causal):
    """Each compiled tiling of each kernel with N_q != N_kv in both directions:
    forward, dK/dV split and single pass, dQ with Delta."""
    scale = head_dim ** -0.5
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for B, Hq, Hkv, N, Nkv in ((1, 4, 2, 200, 450), (1, 4, 2, 450, 200)):
        q, k, v, do = make_inputs(B, Hq, Hkv, N, head_dim, seed=5 * N + Nkv, mult=0.5, n_kv=Nkv)
        qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
        o, lse = _ops.flash_fwd(qd, kd, vd, causal, scale)
        delta = _ops.flash_bwd_preprocess(o, dod)
        torch.cuda.synchronize()
        ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal, scale,
                               o16=o.cpu().numpy(), fold_bwd=True)

        def close(tag, got, name):
            assert_close(tag, torch.as_tensor(got).double().cpu().numpy(), ref[name])

        kinds = ((_lib.KERNEL_FWD, "fwd"), (_lib.KERNEL_DKDV, "dkdv"), (_lib.KERNEL_DQ, "dq"))
        for kind, kname in kinds:
            for var in _lib.tiling_variants(kind, head_dim, causal):
                tag = f"cross N_q={N} N_kv={Nkv} D={head_dim} causal={causal} {kname} " \
                      f"variant {var['variant']} ({var['waves']} waves, tile {var['tile']})"
                _note(tag)
                _lib.set_tiling(kind, head_dim, causal, var["variant"])
                try:
                    if kind == _lib.KERNEL_FWD:
                        o2, lse2 = _ops.flash_fwd(qd, kd, vd, causal, scale)
                        torch.cuda.synchronize()
                        close(tag + " o", o2, "o")
                        lse_err = float(np.max(np.abs(lse2.double().cpu().numpy() - ref["lse"])))
                        assert lse_err <= LSE_TOL, f"{tag} lse {lse_err:.3e}"
                    elif kind == _lib.KERNEL_DKDV:
                        dk1, dv1 = _ops.flash_bwd_dkdv(qd, kd, vd, dod, lse, delta, causal, scale)
                        dk2, dv2 = torch.empty_like(kd), torch.empty_like(vd)
                        _lib.check(lib.fa_bwd_dkdv_ws_kv(
                            qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), dod.data_ptr(),
                            lse.data_ptr(), delta.data_ptr(), dk2.data_ptr(), dv2.data_ptr(),
                            B, Hq, Hkv, N, Nkv, head_dim, scale, int(causal), None, 0, stream))
                        torch.cuda.synchronize()
                        close(tag + " dk (split)", dk1, "dk")
                        close(tag + " dv (split)", dv1, "dv")
                        close(tag + " dk", dk2, "dk")
                        close(tag + " dv", dv2, "dv")
                    else:
                        delta2, dq = _ops.flash_bwd_dq_delta(qd, kd, vd, o, dod, lse, causal, scale)
                        torch.cuda.synchronize()
                        torch.testing.assert_close(delta2, delta, rtol=1e-5, atol=1e-5, msg=tag)
                        close(tag + " dq", dq, "dq")
                finally:
                    _lib.set_tiling(kind, head_dim, causal, -1)


@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_bf16_cross_attention_matches_oracle(head_dim):
    for B, Hq, Hkv, N, Nkv in ((1, 6, 3, 300, 611), (2, 4, 2, 333, 97)):
        q, k, v, do = make_inputs(B, Hq, Hkv, N, head_dim, seed=N * Nkv, dtype=torch.bfloat16,
                                  n_kv=Nkv)
        for causal in (False, True):
            got = run_kernel(q, k, v, do, causal)
            assert got["o16"].dtype == torch.bfloat16
            check_bf16_against_oracle(
                got, q, k, v, do, causal,
                tag=f"bf16 cross N_q={N} N_kv={Nkv} D={head_dim} causal={causal}")


# ---------------------------------------------------------------------------
# Head sizes other than the kernels' (the reference sends them to SDPA,
# attention.py:643-646, 657-661): served by zero-padding to a kernel size.
# ---------------------------------------------------------------------------
VALUE_HEAD_CASES = [
    # (B, Hq, Hkv, N_q, N_kv, D, D_v, dtype): value head size != query/key head size
    (1, 4, 2, 300, 300, 64, 32, torch.float16),
    (2, 4, 4, 129, 257, 32, 128, torch.float16),
    (1, 2, 1, 333, 97, 128, 64, torch.float16),
    # head sizes between the kernel sizes, equal or not
    (1, 4, 2, 200, 200, 16, 16, torch.float16),
    (1, 2, 2, 150, 150, 40, 40, torch.float16),
    (2, 4, 2, 129, 300, 80, 80, torch.float16),
    (1, 4, 4, 257, 257, 96, 96, torch.float16),
    (1, 2, 1, 100, 333, 112, 48, torch.float16),
    (1, 2, 2, 64, 64, 8, 24, torch.float16),
    (1, 4, 2, 190, 190, 96, 96, torch.bfloat16),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", VALUE_HEAD_CASES,
                         ids=lambda c: f"Nq{c[3]}Nkv{c[4]}-D{c[5]}Dv{c[6]}-{str(c[7])[6:]}")
def test_value_head_size_matches_oracle(case, causal):
    B, Hq, Hkv, N, Nkv, D, Dv, dtype = case
    tag = (f"D_v B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} D_v={Dv} {dtype} "
           f"causal={causal}")
    _note(tag)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + Nkv + D + Dv, mult=0.5, n_kv=Nkv, d_v=Dv,
                              dtype=dtype)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    gqa = Hq != Hkv
    decision = explain_dispatch(qd, kd, vd, enable_gqa=gqa)
    assert decision.backend == "triton" and "zero-padded" in decision.reason, decision.reason
    out = scaled_dot_product_attention(qd, kd, vd, is_causal=causal, enable_gqa=gqa,
                                       backend="triton")
    assert out.shape == (B, Hq, N, Dv) and out.is_contiguous()
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    width = next(w for w in (32, 64, 128) if w >= max(D, Dv))
    pad = lambda t: torch.nn.functional.pad(t, (0, width - t.shape[-1])).to(DEV)
    _, lse = _ops.flash_fwd(pad(q), pad(k), pad(v), causal, D ** -0.5)
    torch.cuda.synchronize()
    f = lambda t: t.float().numpy()
    bf16 = dtype == torch.bfloat16
    ref = oracle.attention(f(q), f(k), f(v), f(do), causal,
                           o16=out.detach().float().cpu().numpy(),
                           fold_bwd="bfloat16" if bf16 else True)
    tols = dict(max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL) if bf16 else {}
    report = {}
    for name, t in (("o", out.detach()), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert t.dtype == dtype
        report[name] = assert_close(f"{tag} {name}", t.double().cpu().numpy(), ref[name], **tols)
    lse_err = float(np.max(np.abs(lse.double().cpu().numpy() - ref["lse"])))
    assert lse_err <= LSE_TOL, f"{tag} lse: max-abs {lse_err:.3e}"
    _note(f"{tag}: " + ", ".join(f"{k}={v[0]:.2e}/{v[1]:.2e}" for k, v in report.items())
          + f", lse={lse_err:.2e}")


# ---------------------------------------------------------------------------
# HIP graph capture (torch.cuda.CUDAGraph over the op layer)
# ---------------------------------------------------------------------------
def test_hip_graph_capture_replays_match_eager():
    """Forward + backward captured in one HIP graph and replayed several times,
    with eager work and synchronizations between replays, and once after new
    values were copied into the captured inputs: every replay is bit-identical
    to the eager result (the kernels are deterministic). The shape takes the
    split dK/dV path, so its workspace is allocated inside the capture; the
    launches record no memset."""
    B, Hq, Hkv, N, D = 1, 8, 2, 1500, 64
    causal, scale = True, D ** -0.5
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=41))
    assert _lib.load().fa_bwd_dkdv_workspace_bytes(B, Hq, Hkv, N, D, 1) > 0

    def step():
        o, lse = _ops.flash_fwd(q, k, v, causal, scale)
        dq, dk, dv = _ops.flash_bwd(q, k, v, o, lse, do, causal, scale)
        return o, lse, dq, dk, dv

    names = ("o", "lse", "dq", "dk", "dv")
    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    torch.cuda.synchronize()
    for replay in range(3):
        filler = torch.randn(1 << 20, device=DEV) * 2.0  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        _note(f"graph replay {replay}: filler {float(filler.abs().max()):.2f}")
        for name, got, want in zip(names, captured, eager):
            assert torch.equal(got, want), f"replay {replay}: {name} differs from eager"
    # new values in the captured input buffers: the replay reads them
    q2, k2, v2, do2 = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=42))
    for dst, src in ((q, q2), (k, k2), (v, v2), (do, do2)):
        dst.copy_(src)
    eager2 = [t.clone() for t in step()]
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for name, got, want, old in zip(names, captured, eager2, eager):
        assert torch.equal(got, want), f"replay on new inputs: {name} differs from eager"
        assert not torch.equal(got, old), f"replay on new inputs: {name} unchanged"


# ---------------------------------------------------------------------------
# Seeded random sweep over the envelope the GPU path serves
# ---------------------------------------------------------------------------
def _random_cases(count=24, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        Hkv = int(rng.choice([1, 2, 4]))
        Hq = Hkv * int(rng.choice([1, 2, 3, 4]))
        N = int(rng.integers(1, 400))
        Nkv = N if rng.random() < 0.5 else int(rng.integers(1, 400))
        D = int(rng.choice([16, 32, 48, 64, 96, 128]))
        Dv = D if rng.random() < 0.7 else int(rng.choice([32, 64, 80, 128]))
        cases.append(dict(
            B=int(rng.choice([1, 2, 3])), Hq=Hq, Hkv=Hkv, N=N, Nkv=Nkv, D=D, Dv=Dv,
            causal=bool(rng.random() < 0.5),
            dtype=torch.bfloat16 if rng.random() < 0.25 else torch.float16,
            scale=None if rng.random() < 0.6 else float(rng.uniform(0.05, 0.5)),
            seed=seed + i))
    return cases


def _wide_random_cases(count=96, seed=97):
    """A wider envelope than _random_cases: GQA groups up to 8, head sizes that
    pad (8 to 112), query lengths up to 2000 and key lengths up to 6000 (so the
    split forward, split dQ and split dK/dV paths run), bounded so the CPU
    oracle stays at about a second per case."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        Hkv = int(rng.choice([1, 2, 4, 8]))
        Hq = Hkv * int(rng.choice([1, 2, 3, 4, 8]))
        B = int(rng.choice([1, 2, 3]))
        N = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(1, 700)),
                            int(rng.integers(700, 2000))]))
        Nkv = N if rng.random() < 0.4 else int(rng.choice([int(rng.integers(1, 700)),
                                                           int(rng.integers(700, 6000))]))
        D = int(rng.choice([8, 16, 24, 32, 40, 64, 72, 96, 112, 128]))
        Dv = D if rng.random() < 0.7 else int(rng.choice([16, 32, 64, 100, 128]))
        if B * Hq * N * Nkv * max(D, Dv) > 6e8:
            continue
        cases.append(dict(
            B=B, Hq=Hq, Hkv=Hkv, N=N, Nkv=Nkv, D=D, Dv=Dv, causal=bool(rng.random() < 0.5),
            dtype=torch.bfloat16 if rng.random() < 0.3 else torch.float16,
            scale=None if rng.random() < 0.6 else float(rng.uniform(0.03, 0.6)),
            seed=seed * 1000 + len(cases)))
    return cases


@pytest.mark.parametrize("case", _random_cases() + _wide_random_cases(),
                         ids=lambda c: f"seed{c['seed']}")
def test_random_envelope_matches_oracle(case):
    c = case
    tag = (f"random seed={c['seed']} B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} N_q={c['N']} "
           f"N_kv={c['Nkv']} D={c['D']} D_v={c['Dv']} causal={c['causal']} "
           f"{str(c['dtype'])[6:]} scale={c['scale']}")
    _note(tag)
    q, k, v, do = make_inputs(c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], seed=c["seed"], mult=0.5,
                              dtype=c["dtype"], n_kv=c["Nkv"], d_v=c["Dv"])
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    gqa = c["Hq"] != c["Hkv"]
    assert explain_dispatch(qd, kd, vd, enable_gqa=gqa).backend == "triton"
    out = scaled_dot_product_attention(qd, kd, vd, is_causal=c["causal"], scale=c["scale"],
                                       enable_gqa=gqa, backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    torch.cuda.synchronize()
    f = lambda t: t.float().numpy()
    bf16 = c["dtype"] == torch.bfloat16
    ref = oracle.attention(f(q), f(k), f(v), f(do), c["causal"], c["scale"],
                           o16=out.detach().float().cpu().numpy(),
                           fold_bwd="bfloat16" if bf16 else True)
    tols = dict(max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL) if bf16 else {}
    for name, t in (("o", out.detach()), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert t.dtype == c["dtype"] and t.shape == {"o": (c["B"], c["Hq"], c["N"], c["Dv"]),
                                                    "dq": q.shape, "dk": k.shape,
                                                    "dv": v.shape}[name]
        assert_close(f"{tag} {name}", t.double().cpu().numpy(), ref[name], **tols)


def _large_random_cases(count=8, seed=11):
    """Seeded large shapes (N_q, N_kv 1000-16384, GQA groups 1-8, padded head
    sizes, both masks and dtypes), bounded so the fp32 reference of one key/
    value head group fits in a few GiB."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 2, 4, 8]))
        B = int(rng.choice([1, 2]))
        N = int(rng.integers(1000, 16385))
        Nkv = N if rng.random() < 0.7 else int(rng.integers(1000, 16385))
        D = int(rng.choice([32, 64, 128, 128, 64, 96, 48]))
        if G * N * Nkv > 2 ** 29 or B * Hkv * G * N * Nkv * D > 1e12:
            continue
        cases.append(dict(B=B, Hq=Hkv * G, Hkv=Hkv, N=N, Nkv=Nkv, D=D,
                          causal=bool(rng.random() < 0.5),
                          dtype=torch.bfloat16 if rng.random() < 0.25 else torch.float16,
                          scale=None if rng.random() < 0.7 else float(rng.uniform(0.05, 0.4)),
                          seed=seed * 1000 + len(cases)))
    return cases


def _fp32_group_reference(q, k, v, do, causal, scale):
    """Plain fp32 attention of one key/value head on the GPU: q, do [G, N_q, D],
    k, v [N_kv, D] (top-left causal mask). O, base-2 LSE, dQ, dK, dV."""
    q, k, v = (t.float().clone().requires_grad_() for t in (q, k, v))
    s = torch.matmul(q, k.t().contiguous().unsqueeze(0).expand(q.shape[0], -1, -1)) * scale
    if causal:
        mask = torch.ones((q.shape[1], k.shape[0]), device=q.device, dtype=torch.bool).triu_(1)
        s = s.masked_fill(mask, float("-inf"))
    lse2 = torch.logsumexp(s, dim=-1) * (1.0 / math.log(2.0))
    o = torch.matmul(torch.softmax(s, dim=-1), v.unsqueeze(0).expand(q.shape[0], -1, -1))
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do.float())
    return o.detach(), lse2.detach(), dq, dk, dv


@pytest.mark.parametrize("case", _large_random_cases(), ids=lambda c: f"seed{c['seed']}")
def test_random_large_shapes_match_fp32_reference(case):
    """Seeded random large shapes through the public API against plain fp32
    attention on the GPU, one key/value head group at a time: O, dQ, dK, dV at
    the north-star tolerances (bf16: 4x) and LSE at 1e-4 for the native head
    sizes. (One-off runs of the same generator passed 400 shapes.)"""
    c = case
    tag = (f"large seed={c['seed']} B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} N_q={c['N']} "
           f"N_kv={c['Nkv']} D={c['D']} causal={c['causal']} {str(c['dtype'])[6:]} "
           f"scale={c['scale']}")
    _note(tag)
    B, Hq, Hkv, D = c["B"], c["Hq"], c["Hkv"], c["D"]
    G = Hq // Hkv
    q, k, v, do = make_inputs(B, Hq, Hkv, c["N"], D, seed=c["seed"], mult=0.5, dtype=c["dtype"],
                              n_kv=c["Nkv"])
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    qg, kg, vg = (t.clone().requires_grad_() for t in (qd, kd, vd))
    out = scaled_dot_product_attention(qg, kg, vg, is_causal=c["causal"], scale=c["scale"],
                                       enable_gqa=G > 1, backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qg, kg, vg), dod)
    scale = D ** -0.5 if c["scale"] is None else c["scale"]
    lse = _ops.flash_fwd(qd, kd, vd, c["causal"], scale)[1] if D in (32, 64, 128) else None
    torch.cuda.synchronize()
    bf16 = c["dtype"] == torch.bfloat16
    tols = dict(max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL) if bf16 else {}
    for b in range(B):
        for h in range(Hkv):
            hs = slice(h * G, (h + 1) * G)
            o_r, l_r, dq_r, dk_r, dv_r = _fp32_group_reference(
                qd[b, hs], kd[b, h], vd[b, h], dod[b, hs], c["causal"], scale)
            for name, got, exp in (("o", out[b, hs], o_r), ("dq", dq[b, hs], dq_r),
                                   ("dk", dk[b, h], dk_r), ("dv", dv[b, h], dv_r)):
                assert_close(f"{tag} b{b} h{h} {name}", got.detach().double().cpu().numpy(),
                             exp.double().cpu().numpy(), **tols)
            if lse is not None:
                err = float((lse[b, hs] - l_r).abs().max())
                assert err <= LSE_TOL, f"{tag} b{b} h{h} lse {err:.2e}"


@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, N_q, N_kv, D, causal, dtype)
    (1, 2, 1, 100, 77, 64, False, torch.float16),    # keys past the last 32-key unit
    (2, 4, 2, 142, 7, 64, True, torch.float16),      # causal cross-attention, N_q > N_kv
    (1, 4, 4, 16, 3000, 64, False, torch.float16),   # split dQ: a range's padding unit
    (1, 2, 1, 90, 45, 128, False, torch.bfloat16),
    (1, 2, 1, 70, 33, 32, False, torch.float16),
], ids=lambda c: "x".join(str(x) for x in c[:7]) + f"-{str(c[7])[6:]}")
def test_dq_with_very_negative_scores_and_a_key_tail(case):
    """Every score of every row far below zero (base-2 LSE below -128), with
    keys past the last 32-key unit or past a split range. Those keys load as
    zero rows; their P must be 0, as the reference's valid-key mask makes it
    (attention.py:339-340). A zero score against an LSE below -128 would
    otherwise overflow exp2 to inf, and inf times the zero key row is NaN in
    dQ. A random sweep with inputs x4 and scales up to 8 found this in causal
    cross-attention; bidirectional launches with N_kv % 32 != 0 and split dQ
    ranges had the same exposure."""
    B, Hq, Hkv, N, Nkv, D, causal, dt = case
    tag = f"negative scores B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} causal={causal} {dt}"
    _note(tag)
    g = torch.Generator("cpu").manual_seed(N * 1000 + Nkv)
    a = 4.6  # q ~ +a, k ~ -a per element: scores ~ -a^2 D, times scale log2(e) < -128
    q = (a + 0.3 * torch.randn((B, Hq, N, D), generator=g)).to(dt)
    k = (-a + 0.3 * torch.randn((B, Hkv, Nkv, D), generator=g)).to(dt)
    v = torch.randn((B, Hkv, Nkv, D), generator=g).to(dt)
    do = torch.randn((B, Hq, N, D), generator=g).to(dt)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    gqa = Hq != Hkv
    out = scaled_dot_product_attention(qd, kd, vd, is_causal=causal, enable_gqa=gqa,
                                       backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    _, lse = _ops.flash_fwd(qd.detach(), kd.detach(), vd.detach(), causal, D ** -0.5)
    torch.cuda.synchronize()
    assert float(lse.max()) < -128, f"{tag}: the case must put every LSE below -128"
    for name, t in (("o", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert bool(torch.isfinite(t).all()), f"{tag}: {name} is not finite"
    f = lambda t: t.float().numpy()
    bf16 = dt == torch.bfloat16
    ref = oracle.attention(f(q), f(k), f(v), f(do), causal, None,
                           o16=out.detach().float().cpu().numpy(),
                           fold_bwd="bfloat16" if bf16 else True)
    max_abs, rel_l2 = (BF16_MAX_ABS_TOL, BF16_REL_L2_TOL) if bf16 else (MAX_ABS_TOL, REL_L2_TOL)
    for name, t in (("o", out.detach()), ("dq", dq), ("dk", dk), ("dv", dv)):
        # dQ sums scale dS K over keys whose common -4.6 part cancels (each row of
        # dS sums to zero), leaving a result ~15x smaller than its terms: the
        # operands' rounding weighs that much more in its relative error
        rel = 4 * rel_l2 if name == "dq" else rel_l2
        assert_close(f"{tag} {name}", t.double().cpu().numpy(), ref[name], max_abs=max_abs,
                     rel_l2=rel)


def test_gradients_beyond_the_fp16_grid_of_the_tolerance():
    """One key and 1845 queries under the causal mask: every query attends to
    key 0 with P = 1, so dV of that key sums 1845 dO rows and reaches |dV| of
    about 80. An fp16 output cannot hold such values to the north-star max-abs
    2e-2: half an fp16 ulp is 0.031 on [64, 128). A 4000-shape random sweep
    found this: the fp64 value 67.2196 lies 0.0009 above the rounding midpoint
    67.21875, and the kernel's fp32 sum landed on the other neighbour, 67.1875
    (error 0.032). The bound here is the tolerance or, where fp16 cannot meet
    it, half an ulp of the fp64 value plus 1e-3 of fp32 summation; rel-L2 stays
    at the north-star 5e-3."""
    B, Hq, Hkv, N, Nkv, D = 2, 8, 8, 1845, 1, 64
    tag = f"single key B={B} H={Hq} N_q={N} N_kv={Nkv} D={D} causal"
    _note(tag)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=20000710, mult=0.5, n_kv=Nkv)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = scaled_dot_product_attention(qd, kd, vd, is_causal=True, backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), do.to(DEV))
    torch.cuda.synchronize()
    f = lambda t: t.float().numpy()
    ref = oracle.attention(f(q), f(k), f(v), f(do), True, None,
                           o16=out.detach().float().cpu().numpy(), fold_bwd=True)
    assert np.abs(ref["dv"]).max() > 64  # the case reaches past the tolerance's fp16 grid
    # O = V[0], and dQ = dK = 0 in exact arithmetic (one key: dS = P (dP - Delta) = 0):
    # the north-star tolerances as they stand
    for name, t in (("o", out.detach()), ("dq", dq), ("dk", dk)):
        assert_close(f"{tag} {name}", t.double().cpu().numpy(), ref[name])
    got, exp = dv.double().cpu().numpy(), ref["dv"]
    half_ulp = np.spacing(np.abs(exp).astype(np.float16)).astype(np.float64) / 2
    bound = np.maximum(MAX_ABS_TOL, half_ulp + 1e-3)
    err = np.abs(got - exp)
    assert (err <= bound).all(), f"{tag} dv: {int((err > bound).sum())} beyond the bound"
    rel = float(np.linalg.norm(got - exp) / np.linalg.norm(exp))
    assert rel <= REL_L2_TOL, f"{tag} dv: rel-L2 {rel:.2e}"
    _note(f"  dv: max-abs {err.max():.3e} at |ref| {np.abs(exp).flat[err.argmax()]:.2f}, "
          f"rel-L2 {rel:.2e}")


# ---------------------------------------------------------------------------
# Split-KV forward (few work-groups: decoding, few heads)
# ---------------------------------------------------------------------------
SPLIT_FWD_CASES = [
    # (B, Hq, Hkv, N_q, N_kv, D, causal, dtype)
    (1, 32, 8, 1, 4000, 128, False, torch.float16),   # decoding, GQA
    (2, 4, 2, 16, 3000, 64, False, torch.float16),
    (1, 2, 2, 2100, 5000, 64, True, torch.float16),   # top-left causal: the ranges cover the
                                                      # 2100 visible keys; early tiles see one
    (1, 2, 2, 2048, 2048, 32, True, torch.float16),   # self-attention with few heads
    (1, 3, 1, 77, 5000, 64, False, torch.bfloat16),
    (1, 4, 4, 2100, 2600, 128, True, torch.bfloat16),
]


@pytest.mark.parametrize("case", SPLIT_FWD_CASES,
                         ids=lambda c: f"Nq{c[3]}Nkv{c[4]}D{c[5]}{'c' if c[6] else 'b'}-{str(c[7])[6:]}")
def test_split_forward_matches_unsplit_and_oracle(case):
    """The split-KV forward (fa_fwd_ws, chosen by the op layer when the
    workspace query asks for it) agrees with the one-pass forward (fa_fwd_kv,
    no workspace) up to fp32 summation order, and with the oracle."""
    B, Hq, Hkv, N, Nkv, D, causal, dtype = case
    tag = f"split fwd B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} causal={causal} {dtype}"
    _note(tag)
    lib = _lib.load()
    ws = lib.fa_fwd_workspace_bytes(B, Hq, Hkv, N, Nkv, D, int(causal))
    assert ws > 0, "the case must take the split path"
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + Nkv + D, n_kv=Nkv, dtype=dtype)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    scale = D ** -0.5
    o_split, lse_split = _ops.flash_fwd(qd, kd, vd, causal, scale)  # takes the split path
    o_one, lse_one = torch.empty_like(qd), torch.empty_like(lse_split)
    bf16 = dtype == torch.bfloat16
    fn = lib.fa_fwd_kv_bf16 if bf16 else lib.fa_fwd_kv
    _lib.check(fn(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o_one.data_ptr(), lse_one.data_ptr(),
                  B, Hq, Hkv, N, Nkv, D, scale, int(causal), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.isfinite(o_split.float()).all() and torch.isfinite(lse_split).all()
    assert_close(f"{tag} o split vs one pass", o_split.float(), o_one.float(),
                 max_abs=4e-3 if not bf16 else 3e-2, rel_l2=1e-3 if not bf16 else 8e-3)
    assert float((lse_split - lse_one).abs().max()) <= 1e-5, tag
    f = lambda t: t.float().numpy()
    o_ref, lse_ref = oracle.fwd(f(q), f(k), f(v), causal, scale)
    tols = dict(max_abs=BF16_MAX_ABS_TOL, rel_l2=BF16_REL_L2_TOL) if bf16 else {}
    assert_close(f"{tag} o", o_split.double().cpu().numpy(), o_ref, **tols)
    lse_err = float(np.max(np.abs(lse_split.double().cpu().numpy() - lse_ref)))
    assert lse_err <= LSE_TOL, f"{tag} lse {lse_err:.3e}"
    _note(f"{tag}: lse err {lse_err:.2e}, workspace {ws} bytes")


def test_split_forward_under_hip_graph_capture():
    """The split-KV forward (two launches: partials, then the merge) captured
    in a HIP graph with its workspace allocated inside the capture: replays
    are bit-identical to eager, also after new values enter the inputs."""
    B, Hq, Hkv, N, Nkv, D = 2, 8, 2, 3, 6000, 128
    assert _lib.load().fa_fwd_workspace_bytes(B, Hq, Hkv, N, Nkv, D, 0) > 0
    q, k, v, _ = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=51, n_kv=Nkv))
    step = lambda: _ops.flash_fwd(q, k, v, False, D ** -0.5)
    eager = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for replay in range(3):
        torch.randn(1 << 18, device=DEV).sum()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(captured, eager):
            assert torch.equal(got, want), f"replay {replay} differs from eager"
    q2 = make_inputs(B, Hq, Hkv, N, D, seed=52, n_kv=Nkv)[0].to(DEV)
    q.copy_(q2)
    eager2 = [t.clone() for t in step()]
    graph.replay()
    torch.cuda.synchronize()
    for got, want in zip(captured, eager2):
        assert torch.equal(got, want), "replay on new inputs differs from eager"


# ---------------------------------------------------------------------------
# Long sequences (32-bit slab offsets, many key splits)
# ---------------------------------------------------------------------------
def test_long_sequences():
    # causal self-attention at N = 32768, D = 128: fwd + bwd against the fp32 reference
    B, H, N, D = 1, 2, 32768, 128
    _note(f"long self-attention B={B} H={H} N={N} D={D} causal")
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, H, H, N, D, seed=61, mult=0.5))
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    out = scaled_dot_product_attention(qa, ka, va, is_causal=True, backend="triton")
    dq, dk, dv = torch.autograd.grad(out, (qa, ka, va), do)
    _, lse = _ops.flash_fwd(q, k, v, True, D ** -0.5)
    ref = torch_reference_fp32(q, k, v, do, True, o16=out.detach())
    torch.cuda.synchronize()
    for name, t in (("o", out.detach()), ("dq", dq), ("dk", dk), ("dv", dv)):
        ma, rl = assert_close(f"long N={N} {name}", t.float(), ref[name])
        _note(f"  {name}: max-abs {ma:.2e} rel-L2 {rl:.2e}")
    assert float((lse - ref["lse"]).abs().max()) <= LSE_TOL
    del ref, qa, ka, va, out, dq, dk, dv
    torch.cuda.empty_cache()
    # decoding against 262144 keys (GQA 8 -> 1): the split forward against the oracle
    B, Hq, Hkv, Nq, Nkv, D = 1, 8, 1, 4, 262144, 128
    _note(f"long decode B={B} Hq={Hq} Hkv={Hkv} N_q={Nq} N_kv={Nkv} D={D}")
    assert _lib.load().fa_fwd_workspace_bytes(B, Hq, Hkv, Nq, Nkv, D, 0) > 0
    q, k, v, _ = make_inputs(B, Hq, Hkv, Nq, D, seed=62, n_kv=Nkv)
    o, lse = _ops.flash_fwd(q.to(DEV), k.to(DEV), v.to(DEV), False, D ** -0.5)
    torch.cuda.synchronize()
    o_ref, lse_ref = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), False)
    assert_close("long decode o", o.double().cpu().numpy(), o_ref)
    assert float(np.max(np.abs(lse.double().cpu().numpy() - lse_ref))) <= LSE_TOL


def _chunked_reference(q, k, v, do, o16, scale, chunk=1 << 21):
    """fp64 forward and backward of one key/value head on the GPU, keys in
    chunks: q, do [G, n, D] (the group's query heads), k, v [N_kv, D], o16 the
    kernel's stored O. The backward's scores use the fp16-rounded scaled
    operands the kernels use, fp16(c k) for dK/dV and fp16(c q) for dQ with
    c = scale / ln 2, as the oracle's fold mode does. Returns O, LSE2, dQ and
    a generator of (key slice, dK, dV) chunks, computed as it is consumed."""
    G, n, D = q.shape
    c = scale / math.log(2.0)
    qf = q.double().reshape(G * n, D)
    dof = do.double().reshape(G * n, D)
    m = torch.full((G * n,), -math.inf, dtype=torch.float64, device=q.device)
    l = torch.zeros_like(m)
    acc = torch.zeros_like(qf)
    for c0 in range(0, k.shape[0], chunk):
        s2 = (qf @ k[c0:c0 + chunk].double().t().contiguous()) * c
        m_new = torch.maximum(m, s2.max(dim=1).values)
        alpha = torch.exp2(m - m_new)
        p = torch.exp2(s2 - m_new[:, None])
        l = l * alpha + p.sum(dim=1)
        acc = acc * alpha[:, None] + p @ v[c0:c0 + chunk].double()
        m = m_new
    o = acc / l[:, None]
    lse2 = m + torch.log2(l)
    delta = (o16.double().reshape(G * n, D) * dof).sum(dim=1)
    q16 = (q.double() * c).half().double().reshape(G * n, D)
    dq = torch.zeros_like(qf)
    for c0 in range(0, k.shape[0], chunk):
        kc, vc = k[c0:c0 + chunk].double(), v[c0:c0 + chunk].double()
        p_q = torch.exp2(q16 @ kc.t().contiguous() - lse2[:, None])
        dq += (p_q * (dof @ vc.t().contiguous() - delta[:, None])) @ kc * scale

    def kv_chunks():
        for c0 in range(0, k.shape[0], chunk):
            kc, vc = k[c0:c0 + chunk].double(), v[c0:c0 + chunk].double()
            p_kv = torch.exp2(qf @ (kc * c).half().double().t().contiguous() - lse2[:, None])
            ds_kv = p_kv * (dof @ vc.t().contiguous() - delta[:, None])
            yield (slice(c0, c0 + chunk), (ds_kv.t().contiguous() @ qf) * scale,
                   p_kv.t().contiguous() @ dof)

    return o.reshape(G, n, D), lse2.reshape(G, n), dq.reshape(G, n, D), kv_chunks()


def test_longest_key_sequence_the_library_accepts():
    """The largest N_kv the C ABI accepts at D = 32 (2 GiB key and value slabs:
    N_kv D 2 + 4096 D 2 < 2^31): forward (split-KV, packed GQA) and backward
    (dK/dV over 262 k key tiles, split dQ) through the op layer against an fp64
    reference. Each query row has its own dominant key among the last six
    (the last key is row 0's), so a lost or misaddressed final row shows in
    O, LSE and dK/dV. Also checks that the API's own limit stays within the
    library's."""
    D, G, n = 32, 2, 3
    Nkv = (1 << 31) // (2 * D) - 4096 - 1
    lib = _lib.load()
    assert lib.fa_fwd_workspace_bytes(1, G, 1, n, Nkv, D, 0) > 0
    assert lib.fa_fwd_workspace_bytes(1, G, 1, n, Nkv + 1, D, 0) == _lib.FA_ERR_TOO_LARGE
    from triton_flash_attention import attention as attn
    assert attn._max_sequence(D) == Nkv
    _note(f"longest key sequence B=1 Hq={G} Hkv=1 N_q={n} N_kv={Nkv} D={D}")
    gen = torch.Generator(device=DEV).manual_seed(71)
    q = (torch.randn((1, G, n, D), generator=gen, device=DEV) * 0.5).half()
    k = (torch.randn((1, 1, Nkv, D), generator=gen, device=DEV) * 0.5).half()
    v = (torch.randn((1, 1, Nkv, D), generator=gen, device=DEV) * 0.5).half()
    do = (torch.randn((1, G, n, D), generator=gen, device=DEV) * 0.5).half()
    scale = D ** -0.5
    # Key N_kv-1-r is query row r's own: score 24 with it (e^24 >> N_kv), value 3 - r.
    for r in range(G * n):
        qr = q[0, r // n, r % n].float()
        k[0, 0, Nkv - 1 - r] = (qr * (24.0 / scale / float(qr @ qr))).half()
        v[0, 0, Nkv - 1 - r] = 3.0 - r
    o, lse = _ops.flash_fwd(q, k, v, False, scale)
    dq, dk, dv = _ops.flash_bwd(q, k, v, o, lse, do, False, scale)
    torch.cuda.synchronize()
    o_ref, lse_ref, dq_ref, grads = _chunked_reference(q[0], k[0, 0], v[0, 0], do[0], o[0], scale)
    for r in range(G * n):  # each row's planted key, the last row among them, dominates
        assert abs(float(o[0, r // n, r % n].float().mean()) - (3.0 - r)) < 0.05, r
    assert_close("longest o", o[0].double(), o_ref)
    assert float((lse[0].double() - lse_ref).abs().max()) <= LSE_TOL
    assert_close("longest dq", dq[0].double(), dq_ref)
    num = {"dk": 0.0, "dv": 0.0}
    den = {"dk": 0.0, "dv": 0.0}
    worst = {"dk": 0.0, "dv": 0.0}
    for sl, dk_ref, dv_ref in grads:
        for name, got, ref in (("dk", dk[0, 0, sl], dk_ref), ("dv", dv[0, 0, sl], dv_ref)):
            diff = got.double() - ref
            num[name] += float((diff * diff).sum())
            den[name] += float((ref * ref).sum())
            worst[name] = max(worst[name], float(diff.abs().max()))
    for name in ("dk", "dv"):
        rel = math.sqrt(num[name]) / math.sqrt(den[name])
        _note(f"  {name}: max-abs {worst[name]:.2e} rel-L2 {rel:.2e}")
        assert worst[name] <= MAX_ABS_TOL and rel <= REL_L2_TOL, (name, worst[name], rel)


# ---------------------------------------------------------------------------
# Packed GQA forward (N_q <= 32: a work-group serves several query heads)
# ---------------------------------------------------------------------------
PACKED_CASES = [
    # (B, Hq, Hkv, N_q, N_kv, D, causal)
    (2, 8, 4, 1, 700, 64, False),     # group 2 -> 2 heads per work-group
    (1, 12, 4, 7, 3000, 32, True),    # group 3 -> no packing
    (2, 16, 4, 32, 1500, 128, True),  # group 4 -> 4 heads, causal
    (1, 12, 2, 5, 2500, 64, False),   # group 6 -> 2 heads
    (1, 16, 2, 1, 9000, 128, False),  # group 8 -> 4 heads, split
    (3, 8, 2, 17, 333, 32, True),     # group 4, short keys (no split)
]


@pytest.mark.parametrize("case", PACKED_CASES,
                         ids=lambda c: f"H{c[1]}-{c[2]}Nq{c[3]}Nkv{c[4]}D{c[5]}{'c' if c[6] else 'b'}")
def test_packed_gqa_forward_matches_oracle(case):
    B, Hq, Hkv, N, Nkv, D, causal = case
    tag = f"packed B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} causal={causal}"
    _note(tag)
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=3 * N + Nkv + D, mult=0.5, n_kv=Nkv)
    got = run_kernel(q, k, v, do, causal)
    check_against_oracle(got, q, k, v, do, causal, tag=tag)


@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_packed_gqa_every_forward_tiling(head_dim):
    """Every compiled forward tiling (2, 4 and 8 waves pack 2, 4 and 8 heads
    of a group of 8) on decoding shapes, one pass and split."""
    scale = head_dim ** -0.5
    for B, Hq, Hkv, N, Nkv, causal in ((1, 16, 2, 3, 600, True), (1, 16, 2, 1, 5000, False)):
        q, k, v, _ = make_inputs(B, Hq, Hkv, N, head_dim, seed=N + Nkv, mult=0.5, n_kv=Nkv)
        o_ref, lse_ref = oracle.fwd(q.numpy(), k.numpy(), v.numpy(), causal, scale)
        qd, kd, vd = (t.to(DEV) for t in (q, k, v))
        for var in _lib.tiling_variants(_lib.KERNEL_FWD, head_dim, causal):
            tag = (f"packed N_q={N} N_kv={Nkv} D={head_dim} causal={causal} fwd variant "
                   f"{var['variant']} ({var['waves']} waves, tile {var['tile']})")
            _note(tag)
            _lib.set_tiling(_lib.KERNEL_FWD, head_dim, causal, var["variant"])
            try:
                o, lse = _ops.flash_fwd(qd, kd, vd, causal, scale)
                torch.cuda.synchronize()
            finally:
                _lib.set_tiling(_lib.KERNEL_FWD, head_dim, causal, -1)
            assert_close(tag + " o", o.double().cpu().numpy(), o_ref)
            lse_err = float(np.max(np.abs(lse.double().cpu().numpy() - lse_ref)))
            assert lse_err <= LSE_TOL, f"{tag} lse {lse_err:.3e}"


# ---------------------------------------------------------------------------
# Split dQ (few work-groups: short queries against many keys, few heads)
# ---------------------------------------------------------------------------
SPLIT_DQ_CASES = [
    # (B, Hq, Hkv, N_q, N_kv, D, causal, dtype)
    (1, 32, 8, 128, 5000, 128, False, torch.float16),
    (1, 2, 2, 2100, 4000, 64, True, torch.float16),    # top-left causal: ranges over the
                                                       # visible keys; later ones empty
    (1, 2, 2, 2048, 2048, 32, True, torch.float16),    # self-attention with few heads
    (1, 6, 3, 40, 4100, 64, False, torch.bfloat16),
]


@pytest.mark.parametrize("case", SPLIT_DQ_CASES,
                         ids=lambda c: f"Nq{c[3]}Nkv{c[4]}D{c[5]}{'c' if c[6] else 'b'}-{str(c[7])[6:]}")
def test_split_dq_matches_unsplit_and_oracle(case):
    """fa_bwd_dq_delta_ws (taken by the op layer when the workspace query
    asks for a split) agrees with the one-pass fa_bwd_dq_delta_kv up to fp32
    summation order, writes the same Delta, and the whole backward matches
    the oracle."""
    B, Hq, Hkv, N, Nkv, D, causal, dtype = case
    tag = f"split dq B={B} Hq={Hq} Hkv={Hkv} N_q={N} N_kv={Nkv} D={D} causal={causal} {dtype}"
    _note(tag)
    lib = _lib.load()
    assert lib.fa_bwd_dq_workspace_bytes(B, Hq, Hkv, N, Nkv, D, int(causal)) > 0
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + 2 * Nkv + D, mult=0.5, n_kv=Nkv,
                              dtype=dtype)
    bf16 = dtype == torch.bfloat16
    got = run_kernel(q, k, v, do, causal)  # the op layer's backward takes the split dQ
    if bf16:
        check_bf16_against_oracle(got, q, k, v, do, causal, tag=tag)
    else:
        check_against_oracle(got, q, k, v, do, causal, tag=tag)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    scale = D ** -0.5
    o, lse = _ops.flash_fwd(qd, kd, vd, causal, scale)
    delta_s, dq_s = torch.empty_like(lse), torch.empty_like(qd)
    delta_1, dq_1 = torch.empty_like(lse), torch.empty_like(qd)
    ws_bytes = lib.fa_bwd_dq_workspace_bytes(B, Hq, Hkv, N, Nkv, D, int(causal))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    args = (qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr(), dod.data_ptr(),
            lse.data_ptr())
    split_fn = lib.fa_bwd_dq_delta_ws_bf16 if bf16 else lib.fa_bwd_dq_delta_ws
    one_fn = lib.fa_bwd_dq_delta_kv_bf16 if bf16 else lib.fa_bwd_dq_delta_kv
    _lib.check(split_fn(*args, delta_s.data_ptr(), dq_s.data_ptr(), B, Hq, Hkv, N, Nkv, D, scale,
                        int(causal), ws.data_ptr(), ws_bytes, stream))
    _lib.check(one_fn(*args, delta_1.data_ptr(), dq_1.data_ptr(), B, Hq, Hkv, N, Nkv, D, scale,
                      int(causal), stream))
    torch.cuda.synchronize()
    torch.testing.assert_close(delta_s, delta_1, rtol=0, atol=0)
    assert_close(f"{tag} dq split vs one pass", dq_s.float(), dq_1.float(),
                 max_abs=4e-3 if not bf16 else 3e-2, rel_l2=1e-3 if not bf16 else 8e-3)


def _random_decode_cases(count=16, seed=4096):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        Hkv = int(rng.choice([1, 2, 4]))
        Hq = Hkv * int(rng.choice([1, 2, 3, 4, 6, 8]))
        D = int(rng.choice([16, 32, 64, 96, 128]))
        cases.append(dict(
            B=int(rng.choice([1, 2])), Hq=Hq, Hkv=Hkv, N=int(rng.integers(1, 41)),
            Nkv=int(rng.integers(1024, 6000)), D=D,
            Dv=D if rng.random() < 0.8 else int(rng.choice([32, 64, 128])),
            causal=bool(rng.random() < 0.3),
            dtype=torch.bfloat16 if rng.random() < 0.25 else torch.float16,
            scale=None if rng.random() < 0.7 else float(rng.uniform(0.05, 0.5)),
            seed=seed + i))
    return cases


@pytest.mark.parametrize("case", _random_decode_cases(), ids=lambda c: f"seed{c['seed']}")
def test_random_decode_envelope_matches_oracle(case):
    """Seeded random decoding shapes (few queries, long keys): packed GQA,
    split-KV forward and split dQ in combination with padded head sizes,
    bf16 and custom scales, through the public API against the oracle."""
    test_random_envelope_matches_oracle(case)
