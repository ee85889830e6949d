"""C-ABI checks that need no GPU: the built library loads, exports every
function include/fa_gfx950.h declares, and rejects bad arguments with the
documented FA_ERR_* codes and messages before making any HIP call."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from triton_flash_attention import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "fa_gfx950.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def header_constants() -> dict[str, int]:
    text = HEADER.read_text()
    return {m.group(1): int(m.group(2)) for m in
            re.finditer(r"#define\s+(FA_[A-Z0-9_]+)\s+\(?(-?\d+)\)?", text)}


@pytest.fixture(scope="module")
def lib():
    ok, why = _lib.available()
    assert ok, why
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert {"fa_fwd", "fa_bwd_preprocess", "fa_bwd_dkdv", "fa_bwd_dq", "fa_last_error",
            "fa_abi_version"} <= set(names)
    raw = ctypes.CDLL(str(_lib.library_path()))
    for name in names:
        assert hasattr(raw, name), f"{name} declared in {HEADER.name} but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature in _lib.py"


def test_error_codes_match_header(lib):
    consts = header_constants()
    assert consts["FA_ABI_VERSION"] == _lib.ABI_VERSION == lib.fa_abi_version()
    for name in ("FA_OK", "FA_ERR_NULL_POINTER", "FA_ERR_BAD_SHAPE", "FA_ERR_HEAD_DIM",
                 "FA_ERR_TOO_LARGE", "FA_ERR_BAD_SCALE", "FA_ERR_BAD_TILING",
                 "FA_ERR_MISALIGNED"):
        assert consts[name] == getattr(_lib, name), name


# Fake device addresses: never dereferenced, because every call below is
# rejected by argument checks that run before any HIP call.
P = 0x10000


def _fwd(lib, q=P, k=P, v=P, o=P, lse=P, B=1, Hq=2, Hkv=2, N=64, D=64, scale=0.125, causal=1):
    return lib.fa_fwd(q, k, v, o, lse, B, Hq, Hkv, N, D, scale, causal, None)


@pytest.mark.parametrize(
    ("kwargs", "code", "message"),
    [
        (dict(q=None), "FA_ERR_NULL_POINTER", "null pointer"),
        (dict(B=0), "FA_ERR_BAD_SHAPE", "must be positive"),
        (dict(N=-3), "FA_ERR_BAD_SHAPE", "must be positive"),
        (dict(Hq=3, Hkv=2), "FA_ERR_BAD_SHAPE", "divisible"),
        (dict(D=48), "FA_ERR_HEAD_DIM", "head_dim must be one of (32, 64, 128)"),
        (dict(D=256), "FA_ERR_HEAD_DIM", "head_dim"),
        (dict(N=1 << 24, D=128), "FA_ERR_TOO_LARGE", "too large"),
        (dict(q=P + 2), "FA_ERR_MISALIGNED", "16-byte aligned"),
        (dict(lse=P + 4), "FA_ERR_MISALIGNED", "16-byte aligned"),
        (dict(scale=0.0), "FA_ERR_BAD_SCALE", "scale"),
        (dict(scale=-1.0), "FA_ERR_BAD_SCALE", "scale"),
        (dict(scale=float("nan")), "FA_ERR_BAD_SCALE", "scale"),
    ],
)
def test_fwd_rejects_bad_arguments(lib, kwargs, code, message):
    rc = _fwd(lib, **kwargs)
    assert rc == getattr(_lib, code)
    assert message in _lib.last_error()
    with pytest.raises(_lib.FlashAttentionError, match=re.escape(message)):
        _lib.check(rc)


def test_backward_entry_points_reject_bad_arguments(lib):
    args = [P] * 7
    rc = lib.fa_bwd_dkdv(*args, None, 1, 4, 2, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_NULL_POINTER
    rc = lib.fa_bwd_dkdv(*args, P, 1, 4, 3, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE
    rc = lib.fa_bwd_dq(*args, 1, 4, 2, 64, 96, 0.125, 1, None)
    assert rc == _lib.FA_ERR_HEAD_DIM
    rc = lib.fa_bwd_dq(P, P, P, P, P, P + 8, P, 1, 4, 2, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_MISALIGNED
    rc = lib.fa_bwd_dq_delta(P, P, P, P, P, P, None, P, 1, 4, 2, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_NULL_POINTER
    rc = lib.fa_bwd_dq_delta(P, P, P, P, P, P, P, P, 1, 4, 3, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE
    rc = lib.fa_bwd_dq_delta(P, P, P, P + 8, P, P, P, P, 1, 4, 2, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_MISALIGNED
    assert "fa_bwd_dq_delta" in _lib.last_error()
    rc = lib.fa_bwd_dq_delta(P, P, P, P, P, P, P, P, 1, 4, 2, 64, 64, -1.0, 1, None)
    assert rc == _lib.FA_ERR_BAD_SCALE
    rc = lib.fa_bwd_preprocess(P, P, None, 1, 1, 8, 64, None)
    assert rc == _lib.FA_ERR_NULL_POINTER
    rc = lib.fa_bwd_preprocess(P, P, P, 1, 1, 8, 40, None)
    assert rc == _lib.FA_ERR_HEAD_DIM


def test_tiling_table_is_complete(lib):
    for kernel in (_lib.KERNEL_FWD, _lib.KERNEL_DKDV, _lib.KERNEL_DQ):
        for D in (32, 64, 128):
            for causal in (False, True):
                t = _lib.get_tiling(kernel, D, causal)
                variants = {v["variant"]: v for v in _lib.tiling_variants(kernel, D, causal)}
                assert variants[t["variant"]] == t
                assert t["rows"] == 32 * t["waves"] and t["tile"] % 32 == 0
    with pytest.raises(_lib.FlashAttentionError):
        _lib.get_tiling(7, 64, True)
    with pytest.raises(_lib.FlashAttentionError):
        _lib.get_tiling(0, 48, True)


def test_tiling_override_round_trip(lib):
    default = _lib.get_tiling(_lib.KERNEL_FWD, 64, True)
    n = lib.fa_num_tiling_variants(_lib.KERNEL_FWD, 64, 1)
    last = _lib.tiling_variants(_lib.KERNEL_FWD, 64, True)[-1]["variant"]
    try:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, last)
        assert _lib.get_tiling(_lib.KERNEL_FWD, 64, True)["variant"] == last
        with pytest.raises(_lib.FlashAttentionError):
            _lib.set_tiling(_lib.KERNEL_FWD, 64, True, n)
    finally:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, -1)
    assert _lib.get_tiling(_lib.KERNEL_FWD, 64, True) == default


def test_tiling_override_is_safe_while_another_thread_reads_it(lib):
    """fa_set_tiling toggles one entry on one thread while a second thread
    resolves that entry (the read every launch makes) and a third sets another
    entry: every read is the default or the override, and the entries do not
    disturb each other. ctypes releases the GIL around each call, so the
    threads run the library concurrently."""
    import threading

    default = _lib.get_tiling(_lib.KERNEL_FWD, 64, True)["variant"]
    other = next(v["variant"] for v in _lib.tiling_variants(_lib.KERNEL_FWD, 64, True)
                 if v["variant"] != default)
    dq_default = _lib.get_tiling(_lib.KERNEL_DQ, 32, False)["variant"]
    stop = threading.Event()
    seen, bad = set(), []

    def writer():
        for i in range(20000):
            assert lib.fa_set_tiling(_lib.KERNEL_FWD, 64, 1, other if i % 2 == 0 else -1) == 0
        stop.set()

    def other_writer():
        while not stop.is_set():
            assert lib.fa_set_tiling(_lib.KERNEL_DQ, 32, 1, -1) == 0

    def reader():
        out = (ctypes.c_int * 4)()
        while not stop.is_set():
            assert lib.fa_get_tiling(_lib.KERNEL_FWD, 64, 1, out) == 0
            seen.add(out[3])
            if out[3] not in (default, other):
                bad.append(out[3])
            assert lib.fa_get_tiling(_lib.KERNEL_DQ, 32, 0, out) == 0
            if out[3] != dq_default:
                bad.append(("dq", out[3]))

    threads = [threading.Thread(target=f) for f in (writer, other_writer, reader)]
    try:
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=60)
    finally:
        stop.set()
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, -1)
    assert not bad, bad[:5]
    assert seen <= {default, other} and seen
    assert _lib.get_tiling(_lib.KERNEL_FWD, 64, True)["variant"] == default


def _list_schedule_makespan(costs, slots):
    """Jobs in the given order, each to the first slot to free up."""
    import heapq

    ends = [0] * slots
    for c in costs:
        heapq.heapreplace(ends, ends[0] + c)
    return max(ends)


def test_forward_job_plan_on_a_256_cu_device(lib):
    """The persistent causal forward's job plan is host logic (no GPU needed
    with an explicit CU count). At c2 (2048 causal jobs on 256 CUs x 3
    work-groups) the grid form's heaviest-first list schedule ends in a tail;
    the plan runs one work-group per slot with a bin of jobs whose modelled
    length is below the grid's and not below the slots' mean (a lower bound
    every schedule obeys). Job cost: the 32-key units it streams plus a fixed
    2-unit part, as the library models it."""
    plan_variant = 9
    try:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, plan_variant)
        info = _lib.fwd_plan_info(4, 16, 16, 4096, 4096, 64, True, 256)
        costs = [4 * (t + 1) + 2 for t in reversed(range(32)) for _ in range(64)]
        mean = -(-sum(costs) // 768)
        assert info["grid_workgroups"] == 2048
        assert info["grid_makespan"] == _list_schedule_makespan(costs, 768)
        assert info["plan_workgroups"] == 768
        assert mean <= info["plan_makespan"] <= 0.97 * info["grid_makespan"]
        # the grid form where a plan cannot help: bidirectional (equal jobs),
        # one slot round or less (c3), a longest job above the slots' mean
        for args in [(4, 16, 16, 4096, 4096, 64, False), (2, 16, 4, 2049, 2049, 64, True),
                     (2, 16, 16, 4096, 4096, 64, True)]:
            assert _lib.fwd_plan_info(*args, 256)["plan_workgroups"] == 0, args
        # a different CU count plans for its own slots
        assert _lib.fwd_plan_info(4, 16, 16, 4096, 4096, 64, True, 128)["grid_makespan"] > \
            info["grid_makespan"]
    finally:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, -1)
    # D = 128 has no plan variant
    assert _lib.fwd_plan_info(2, 32, 32, 8192, 8192, 128, True, 256)["plan_workgroups"] == 0
    with pytest.raises(_lib.FlashAttentionError):
        _lib.fwd_plan_info(4, 16, 16, 4096, 4096, 48, True, 256)


def test_launch_without_a_device_reports_the_hip_error(lib):
    """On a host with no GPU, a well-formed call reaches the launch and the HIP
    runtime's error comes back as a positive code with its message (the fake
    pointers are never touched: no kernel can run without a device)."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("only meaningful on a host without a GPU")
    rc = _fwd(lib)
    assert rc > 0
    assert "fa_fwd launch" in _lib.last_error()


def test_bf16_twins_check_like_fp16_and_fall_back_to_the_default_tiling(lib):
    """The _bf16 entry points share the fp16 argument checks (named after the
    bf16 symbol), and a bf16 call whose kernel has an fp16-only tiling
    override runs the default tiling instead of failing."""
    import torch

    rc = lib.fa_fwd_bf16(None, P, P, P, P, 1, 2, 2, 64, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_NULL_POINTER and "fa_fwd_bf16" in _lib.last_error()
    rc = lib.fa_bwd_dq_bf16(P, P, P, P, P, P, P, 1, 2, 2, 64, 48, 0.125, 1, None)
    assert rc == _lib.FA_ERR_HEAD_DIM
    if torch.cuda.is_available():
        # The call below passes every argument check and reaches a launch; with a
        # device present that launch would read the fake address P.
        pytest.skip("the override fallback launch is checked only on a host without a GPU")
    fp16_only = [v["variant"] for v in _lib.tiling_variants(_lib.KERNEL_FWD, 64, True)
                 if v["variant"] != _lib.get_tiling(_lib.KERNEL_FWD, 64, True)["variant"]][0]
    try:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, fp16_only)
        rc = lib.fa_fwd_bf16(P, P, P, P, P, 1, 2, 2, 64, 64, 0.125, 1, None)
        assert rc != _lib.FA_ERR_BAD_TILING
        assert rc > 0 and "fa_fwd_bf16 launch" in _lib.last_error()
    finally:
        _lib.set_tiling(_lib.KERNEL_FWD, 64, True, -1)


def test_dkdv_workspace_sizing_and_rejection(lib):
    # MHA with many key tiles: single pass, no workspace
    assert lib.fa_bwd_dkdv_workspace_bytes(4, 16, 16, 4096, 64, 1) == 0
    # GQA with 2 KV heads: split into partials; size = nsplit * 2 planes * B*Hkv*N*D * 4 bytes
    plane = 1 * 2 * 16381 * 32
    ws = lib.fa_bwd_dkdv_workspace_bytes(1, 8, 2, 16381, 32, 1)
    assert ws > 0 and ws % (2 * plane * 4) == 0 and ws // (2 * plane * 4) <= 16
    # causal launches this poorly filled split further than bidirectional ones
    ws_bidir = lib.fa_bwd_dkdv_workspace_bytes(1, 8, 2, 16381, 32, 0)
    assert 0 < ws_bidir < ws and ws_bidir % (2 * plane * 4) == 0
    assert lib.fa_bwd_dkdv_workspace_bytes(1, 8, 2, 16381, 48, 1) == _lib.FA_ERR_HEAD_DIM
    # a workspace smaller than required is rejected before any launch
    rc = lib.fa_bwd_dkdv_ws(P, P, P, P, P, P, P, P, 1, 8, 2, 16381, 32, 0.17, 1, P, ws - 16, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE
    assert "smaller than" in _lib.last_error()


def test_cross_attention_entries_check_both_lengths(lib):
    # fa_fwd_kv(q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale, causal, stream)
    rc = lib.fa_fwd_kv(None, P, P, P, P, 1, 2, 2, 64, 80, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_NULL_POINTER and "fa_fwd_kv: null pointer" in _lib.last_error()
    rc = lib.fa_fwd_kv_bf16(P, P, P, P, P, 1, 2, 2, 64, 0, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE and "N_kv must be positive" in _lib.last_error()
    rc = lib.fa_fwd_kv(P, P, P, P, P, 1, 2, 2, 0, 80, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE
    rc = lib.fa_fwd_kv(P, P, P, P, P, 1, 2, 2, 64, 1 << 24, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_TOO_LARGE and "key/value sequence length" in _lib.last_error()
    rc = lib.fa_bwd_dq_delta_kv(P, P, P, P, P, P, P, P, 1, 4, 2, 64, 80, 96, 0.125, 1, None)
    assert rc == _lib.FA_ERR_HEAD_DIM
    rc = lib.fa_bwd_dq_delta_kv_bf16(P, P, P, P, P, P, P, P, 1, 4, 2, 64, -3, 64, 0.125, 1, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE
    rc = lib.fa_bwd_dkdv_ws_kv(P, P, P, P, P, P, P, P + 8, 1, 4, 2, 64, 80, 64, 0.125, 1,
                               None, 0, None)
    assert rc == _lib.FA_ERR_MISALIGNED
    rc = lib.fa_bwd_dkdv_ws_kv_bf16(P, P, P, P, P, P, P, P, 1, 4, 2, 64, 80, 64, -1.0, 1,
                                    None, 0, None)
    assert rc == _lib.FA_ERR_BAD_SCALE


def test_cross_attention_workspace_follows_the_key_length(lib):
    for args in ((4, 16, 16, 4096, 64, 1), (1, 8, 2, 16381, 32, 1), (1, 8, 2, 700, 64, 0)):
        B, Hq, Hkv, N, D, causal = args
        assert lib.fa_bwd_dkdv_workspace_bytes_kv(B, Hq, Hkv, N, N, D, causal) == \
            lib.fa_bwd_dkdv_workspace_bytes(*args)
    # the split partials are [nsplit, 2, B, Hkv, N_kv, D] fp32; N_q only sets how
    # much work each key tile has, and too little (300 queries) is not split
    ws = lib.fa_bwd_dkdv_workspace_bytes_kv(1, 8, 2, 5000, 300, 64, 1)
    plane = 1 * 2 * 300 * 64 * 4
    assert ws > 0 and ws % (2 * plane) == 0 and ws // (2 * plane) <= 16
    assert lib.fa_bwd_dkdv_workspace_bytes_kv(1, 8, 2, 300, 300, 64, 1) == 0
    rc = lib.fa_bwd_dkdv_ws_kv(P, P, P, P, P, P, P, P, 1, 8, 2, 5000, 300, 64, 0.125, 1,
                               P, ws - 16, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE and "smaller than" in _lib.last_error()


def test_split_forward_workspace_sizing_and_rejection(lib):
    # enough work-groups (the headline shape, or a long prompt): no split
    assert lib.fa_fwd_workspace_bytes(4, 16, 16, 4096, 4096, 64, 1) == 0
    assert lib.fa_fwd_workspace_bytes(1, 32, 8, 4096, 4096, 128, 1) == 0
    # too few keys to split
    assert lib.fa_fwd_workspace_bytes(1, 32, 8, 1, 700, 128, 0) == 0
    # decoding: one query against 32768 keys, 32 heads -> split, [nsplit, B, Hq, N_q, D + 1] fp32
    ws = lib.fa_fwd_workspace_bytes(1, 32, 8, 1, 32768, 128, 0)
    per_split = 1 * 32 * 1 * (128 + 1) * 4
    assert ws > 0 and ws % per_split == 0 and 2 <= ws // per_split <= 64
    # under the (top-left) mask only the first min(N_q, N_kv) keys are seen by
    # any query, and the key ranges cover those: 128 queries against 32768
    # keys have too few to split (the forward and dQ split without the mask);
    # 4096 against 32768 split the first 4096 keys into ranges of >= 1024
    assert lib.fa_fwd_workspace_bytes(1, 32, 8, 128, 32768, 128, 0) > 0
    assert lib.fa_fwd_workspace_bytes(1, 32, 8, 128, 32768, 128, 1) == 0
    assert lib.fa_bwd_dq_workspace_bytes(1, 32, 8, 128, 32768, 128, 0) > 0
    assert lib.fa_bwd_dq_workspace_bytes(1, 32, 8, 128, 32768, 128, 1) == 0
    per_split = 1 * 2 * 4096 * (128 + 1) * 4
    causal_ws = lib.fa_fwd_workspace_bytes(1, 2, 2, 4096, 32768, 128, 1)
    assert causal_ws % per_split == 0 and 2 <= causal_ws // per_split <= 4
    assert lib.fa_fwd_workspace_bytes(1, 2, 2, 4096, 32768, 128, 0) // per_split > 4
    assert lib.fa_fwd_workspace_bytes(1, 32, 8, 1, 32768, 96, 0) == _lib.FA_ERR_HEAD_DIM
    assert lib.fa_fwd_workspace_bytes(1, 32, 8, 1, 0, 128, 0) == _lib.FA_ERR_BAD_SHAPE
    # a workspace smaller than required is rejected before any launch
    rc = lib.fa_fwd_ws(P, P, P, P, P, 1, 32, 8, 1, 32768, 128, 0.09, 0, P, ws - 16, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE and "smaller than" in _lib.last_error()
    rc = lib.fa_fwd_ws_bf16(P, P, P, P, P, 1, 32, 8, 1, 32768, 128, 0.09, 0, P + 8, ws, None)
    assert rc == _lib.FA_ERR_MISALIGNED


def test_whole_backward_workspace_is_both_splits_and_rejects_bad_arguments(lib):
    """fa_bwd's workspace holds the dQ partials, then (at a 256-byte boundary)
    the dK/dV partials: the sum of what the per-kernel queries report, except
    that in the combined plan (dK/dV splits, dQ does not and has at most 768
    work-groups of 128 queries) the dK/dV chunks aim at 3072 work-groups
    counting the dQ ones, between 2 and 16 of them."""
    for args in [(4, 16, 16, 4096, 4096, 64, 1), (2, 16, 4, 2049, 2049, 64, 1),
                 (1, 8, 2, 16381, 16381, 32, 1), (1, 32, 8, 128, 32768, 128, 0),
                 (1, 8, 2, 5000, 300, 64, 1), (1, 4, 1, 700, 900, 64, 0),
                 (1, 8, 2, 16381, 16381, 128, 1), (1, 4, 1, 16381, 16381, 32, 1),
                 (1, 6, 2, 16384, 16384, 64, 0)]:
        dq = lib.fa_bwd_dq_workspace_bytes(*args)
        dkdv = lib.fa_bwd_dkdv_workspace_bytes_kv(*args)
        assert dq >= 0 and dkdv >= 0
        got = lib.fa_bwd_workspace_bytes(*args)
        B, Hq, Hkv, N, Nkv, D, causal = args
        dq_wgs = -(-N // 128) * B * Hq
        if dkdv == 0 or dq > 0 or D == 128 or dq_wgs > 768:
            # the per-kernel launches, one after the other
            assert got == (((dq + 255) // 256 * 256 + dkdv) if dkdv else dq), args
        else:  # combined launch
            plane = 2 * B * Hkv * Nkv * D * 4
            assert got % plane == 0 and 2 <= got // plane <= 16, args
            if (B, Hq, Hkv, N, D, causal) == (2, 16, 4, 2049, 64, 1):
                assert got == 4 * plane  # c3: capped by 32 query units per chunk
            if (B, Hq, Hkv, N, D, causal) == (1, 6, 2, 16384, 64, 0):
                assert got == 9 * plane  # (3072 - 768) / 256 rounded up
    assert lib.fa_bwd_workspace_bytes(4, 16, 16, 4096, 4096, 64, 1) == 0
    assert lib.fa_bwd_workspace_bytes(1, 8, 2, 16381, 16381, 48, 1) == _lib.FA_ERR_HEAD_DIM
    assert lib.fa_bwd_workspace_bytes(1, 8, 2, 16381, 0, 32, 1) == _lib.FA_ERR_BAD_SHAPE
    # fa_bwd(q, k, v, o, dO, lse, delta, dq, dk, dv, B, Hq, Hkv, N_q, N_kv, D, scale,
    #        causal, workspace, workspace_bytes, stream)
    ptrs = [P] * 10
    shape = (2, 16, 4, 2049, 2049, 64)
    ws = lib.fa_bwd_workspace_bytes(*shape, 1)
    assert ws > 0
    rc = lib.fa_bwd(*ptrs[:9], None, *shape, 0.125, 1, P, ws, None)
    assert rc == _lib.FA_ERR_NULL_POINTER and "fa_bwd: null pointer" in _lib.last_error()
    rc = lib.fa_bwd(*ptrs, 2, 16, 3, 2049, 2049, 64, 0.125, 1, P, ws, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE
    rc = lib.fa_bwd_bf16(*ptrs, 2, 16, 4, 2049, 2049, 96, 0.125, 1, P, ws, None)
    assert rc == _lib.FA_ERR_HEAD_DIM
    rc = lib.fa_bwd(P, P, P, P, P, P + 8, P, P, P, P, *shape, 0.125, 1, P, ws, None)
    assert rc == _lib.FA_ERR_MISALIGNED
    rc = lib.fa_bwd(*ptrs, *shape, 0.0, 1, P, ws, None)
    assert rc == _lib.FA_ERR_BAD_SCALE
    rc = lib.fa_bwd(*ptrs, *shape, 0.125, 1, P, ws - 16, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE and "smaller than" in _lib.last_error()
    rc = lib.fa_bwd_bf16(*ptrs, *shape, 0.125, 1, P + 4, ws, None)
    assert rc == _lib.FA_ERR_MISALIGNED


def test_split_dq_workspace_sizing_and_rejection(lib):
    assert lib.fa_bwd_dq_workspace_bytes(4, 16, 16, 4096, 4096, 64, 1) == 0
    assert lib.fa_bwd_dq_workspace_bytes(1, 32, 8, 128, 700, 128, 0) == 0  # too few keys
    ws = lib.fa_bwd_dq_workspace_bytes(1, 32, 8, 128, 32768, 128, 0)
    per_split = 1 * 32 * 128 * 128 * 4  # [nsplit, B, Hq, N_q, D] fp32
    assert ws > 0 and ws % per_split == 0 and 2 <= ws // per_split <= 32
    assert lib.fa_bwd_dq_workspace_bytes(1, 32, 8, 128, 32768, 80, 0) == _lib.FA_ERR_HEAD_DIM
    rc = lib.fa_bwd_dq_delta_ws(P, P, P, P, P, P, P, P, 1, 32, 8, 128, 32768, 128, 0.09, 0,
                                P, ws - 16, None)
    assert rc == _lib.FA_ERR_BAD_SHAPE and "smaller than" in _lib.last_error()
    rc = lib.fa_bwd_dq_delta_ws_bf16(P, P, P, P, P, P, P, P, 1, 32, 8, 128, 32768, 128, 0.09, 0,
                                     P + 4, ws, None)
    assert rc == _lib.FA_ERR_MISALIGNED


def test_native_binding_loads_and_takes_the_library_entry_points(lib):
    """The C++ autograd binding is built next to the library and initialised
    with the library's own entry points (no GPU needed); the public API hands
    it the plain training calls only."""
    import torch

    from triton_flash_attention import _native
    from triton_flash_attention import attention as api

    ok, why = _native.status()
    assert ok, why
    assert _native._module.ready()
    for name in _native.ENTRY_POINTS:
        assert name in declared_functions(), name
    q = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    assert api._native_serves(q, q, 0.125)
    assert not api._native_serves(q, q, -0.125)          # negated query: Python Function
    assert not api._native_serves(q, q, 0.0)             # zero query: Python Function
    assert not api._native_serves(q, q[..., :32], 0.125)  # D_v != D: padded
    q40 = torch.zeros(1, 2, 8, 40, dtype=torch.float16)
    assert not api._native_serves(q40, q40, 0.125)        # padded head size
    # Arguments the binding cannot serve are rejected before any HIP call.
    with pytest.raises(RuntimeError, match="one GPU"):
        _native._module.attention(q, q, q, True, 0.125)
    with pytest.raises(RuntimeError, match="must be 4-D"):
        _native._module.attention(q[0], q[0], q[0], True, 0.125)
