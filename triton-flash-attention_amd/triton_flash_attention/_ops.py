"""Tensor-level calls into libfa_gfx950.so.

PyTorch only provides device memory and the current HIP stream here: each
function checks layout on the host (the C ABI sees raw pointers), allocates
its outputs with the caching allocator, and launches one C-ABI entry point on
``torch.cuda.current_stream(device)``. There is no fallback: if the library
is missing these functions raise.

Reference launches replaced (triton_flash_attention/attention.py):
    flash_fwd            -> _attn_fwd[grid]              690-718
    flash_bwd_preprocess -> _attn_bwd_preprocess[grid]   736-744
    flash_bwd_dkdv       -> _attn_bwd[grid], phase 1     754-770 (428-505)
    flash_bwd_dq         -> _attn_bwd[grid], phase 2     754-770 (507-573)
    flash_bwd_dq_delta   -> preprocess + phase 2         736-744, 754-770
    flash_bwd            -> preprocess + both phases     720-770 (TritonAttention.backward)

The forward and the backward also serve cross-attention (key/value length
N_kv != query length N), which the reference sends to torch SDPA
(attention.py:639-642): those calls go to the library's ``*_kv`` entry points.
"""

from __future__ import annotations

import contextlib
import ctypes

import torch

from . import _lib


# torch's current raw stream handle of a device, without building a Python
# Stream object (about 9 us per call on the public path); the public call where
# this torch build lacks it.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    if _raw_stream is not None:
        index = t.device.index
        return ctypes.c_void_p(_raw_stream(torch.cuda.current_device() if index is None else index))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _device_guard(device: torch.device):
    """Make ``device`` current for the launches (a no-op when it already is)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


class LaunchTimer:
    """Brackets every kernel launch made through this module with HIP events
    recorded on the launch stream (torch's current stream), so per-kernel
    average durations can be read after a timed region:

        with LaunchTimer() as timer:
            ...                      # any fwd/bwd calls
        torch.cuda.synchronize()
        timer.mean_ms("dkdv")
    """

    _active: "LaunchTimer | None" = None

    def __init__(self) -> None:
        self.events: dict[str, list[tuple[torch.cuda.Event, torch.cuda.Event]]] = {}

    def __enter__(self) -> "LaunchTimer":
        LaunchTimer._active = self
        return self

    def __exit__(self, *exc) -> None:
        LaunchTimer._active = None

    def _begin(self) -> torch.cuda.Event:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def _end(self, name: str, start: torch.cuda.Event) -> None:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self.events.setdefault(name, []).append((start, ev))

    def durations_ms(self, name: str) -> list[float]:
        return [a.elapsed_time(b) for a, b in self.events.get(name, [])]

    def mean_ms(self, name: str) -> float:
        d = self.durations_ms(name)
        return sum(d) / len(d) if d else float("nan")


def _launch(name: str, fn, *args) -> int:
    timer = LaunchTimer._active
    if timer is None:
        return fn(*args)
    start = timer._begin()
    rc = fn(*args)
    timer._end(name, start)
    return rc


def _require(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor")


# Element types of the 16-bit tensors and the suffix of their library entry points.
_ELEM_SUFFIX = {torch.float16: "", torch.bfloat16: "_bf16"}


def _elem_dtype(t: torch.Tensor, name: str) -> torch.dtype:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype not in _ELEM_SUFFIX:
        raise ValueError(f"{name} must be torch.float16 or torch.bfloat16, got {t.dtype}")
    return t.dtype


def _entry(lib, base: str, dtype: torch.dtype):
    """The library entry point of ``base`` for tensors of ``dtype``."""
    return getattr(lib, base + _ELEM_SUFFIX[dtype])


def _entry_lengths(lib, base: str, dtype: torch.dtype, n: int, n_kv: int):
    """(entry point, length arguments): the self-attention entry with (N,),
    or its cross-attention twin ``base_kv`` with (N_q, N_kv)."""
    if n == n_kv:
        return _entry(lib, base, dtype), (n,)
    return _entry(lib, base + "_kv", dtype), (n, n_kv)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """The kernels move 128-bit vectors: a view whose data pointer is not
    16-byte aligned is copied into a fresh (aligned) allocation."""
    return t if t.data_ptr() % 16 == 0 else t.clone(memory_format=torch.contiguous_format)


def _qkv_dims(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple[int, ...]:
    """(B, Hq, Hkv, N, N_kv, D) of q [B,Hq,N,D] and k, v [B,Hkv,N_kv,D]."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must be 4-D [batch, heads, sequence, head_dim]")
    B, Hq, N, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError(
            f"k and v must have shape [{B}, Hkv, N_kv, {D}]; got {tuple(k.shape)}, {tuple(v.shape)}"
        )
    return B, Hq, k.shape[1], N, k.shape[2], D


def flash_fwd(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """O [B,Hq,N,D] (the inputs' fp16 or bf16) and base-2 LSE [B,Hq,N] fp32.

    Launches with few work-groups (decoding, few heads) get a workspace from
    the caching allocator for the library's split-KV mode."""
    dt = _elem_dtype(q, "q")
    for name, t in (("q", q), ("k", k), ("v", v)):
        _require(t, name, dt, q.device)
    B, Hq, Hkv, N, Nkv, D = _qkv_dims(q, k, v)
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    lib = _lib.load()
    c = int(bool(causal))
    ws_bytes = lib.fa_fwd_workspace_bytes(B, Hq, Hkv, N, Nkv, D, c)
    if ws_bytes < 0:
        _lib.check(ws_bytes)
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, N), device=q.device, dtype=torch.float32)
    with _device_guard(q.device):
        if ws_bytes > 0:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
            rc = _launch(
                "fwd", _entry(lib, "fa_fwd_ws", dt),
                q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                B, Hq, Hkv, N, Nkv, D, float(scale), c, ws.data_ptr(), ws_bytes, _stream(q),
            )
        else:
            fn, lengths = _entry_lengths(lib, "fa_fwd", dt, N, Nkv)
            rc = _launch(
                "fwd", fn,
                q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                B, Hq, Hkv, *lengths, D, float(scale), c, _stream(q),
            )
    _lib.check(rc)
    return o, lse


def flash_bwd_preprocess(o: torch.Tensor, do: torch.Tensor) -> torch.Tensor:
    """Delta [B,H,N] fp32 = rowsum(O * dO)."""
    dt = _elem_dtype(o, "o")
    _require(o, "o", dt, o.device)
    _require(do, "dO", dt, o.device)
    if do.shape != o.shape or o.ndim != 4:
        raise ValueError("o and dO must have the same 4-D shape")
    B, H, N, D = o.shape
    o, do = _aligned(o), _aligned(do)
    lib = _lib.load()
    delta = torch.empty((B, H, N), device=o.device, dtype=torch.float32)
    with _device_guard(o.device):
        rc = _launch("preprocess", _entry(lib, "fa_bwd_preprocess", dt),
                     o.data_ptr(), do.data_ptr(), delta.data_ptr(), B, H, N, D, _stream(o))
    _lib.check(rc)
    return delta


def _check_bwd_inputs(q, k, v, do, lse, delta):
    dt = _elem_dtype(q, "q")
    for name, t in (("q", q), ("k", k), ("v", v), ("dO", do)):
        _require(t, name, dt, q.device)
    for name, t in (("lse", lse), ("delta", delta)):
        _require(t, name, torch.float32, q.device)
    dims = _qkv_dims(q, k, v)
    B, Hq, _, N, _, _ = dims
    if do.shape != q.shape:
        raise ValueError("dO must have the shape of q")
    if lse.shape != (B, Hq, N) or delta.shape != (B, Hq, N):
        raise ValueError("lse and delta must have shape [B, Hq, N]")
    return dims


def _aligned_all(*tensors):
    return tuple(_aligned(t) for t in tensors)


def flash_bwd_dkdv(
    q, k, v, do, lse, delta, causal: bool, scale: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """dK, dV [B,Hkv,N_kv,D] in q's dtype (GQA groups reduced in fp32, deterministic).

    Shapes with too few key tiles to fill the GPU get a workspace (from the
    caching allocator) for the library's split-and-reduce mode."""
    B, Hq, Hkv, N, Nkv, D = _check_bwd_inputs(q, k, v, do, lse, delta)
    q, k, v, do, lse, delta = _aligned_all(q, k, v, do, lse, delta)
    lib = _lib.load()
    fn, lengths = _entry_lengths(lib, "fa_bwd_dkdv_ws", q.dtype, N, Nkv)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if N == Nkv:
        ws_bytes = lib.fa_bwd_dkdv_workspace_bytes(B, Hq, Hkv, N, D, int(bool(causal)))
    else:
        ws_bytes = lib.fa_bwd_dkdv_workspace_bytes_kv(B, Hq, Hkv, N, Nkv, D, int(bool(causal)))
    if ws_bytes < 0:
        _lib.check(ws_bytes)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None
    with _device_guard(q.device):
        rc = _launch(
            "dkdv", fn,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), lse.data_ptr(),
            delta.data_ptr(), dk.data_ptr(), dv.data_ptr(),
            B, Hq, Hkv, *lengths, D, float(scale), int(bool(causal)),
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q),
        )
    _lib.check(rc)
    return dk, dv


def flash_bwd_dq(q, k, v, do, lse, delta, causal: bool, scale: float) -> torch.Tensor:
    """dQ [B,Hq,N,D] in q's dtype (self-attention; cross-attention takes
    :func:`flash_bwd_dq_delta`)."""
    B, Hq, Hkv, N, Nkv, D = _check_bwd_inputs(q, k, v, do, lse, delta)
    if N != Nkv:
        raise ValueError("flash_bwd_dq serves N_kv == N; use flash_bwd_dq_delta for cross-attention")
    q, k, v, do, lse, delta = _aligned_all(q, k, v, do, lse, delta)
    lib = _lib.load()
    dq = torch.empty_like(q)
    with _device_guard(q.device):
        rc = _launch(
            "dq", _entry(lib, "fa_bwd_dq", q.dtype),
            q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), lse.data_ptr(),
            delta.data_ptr(), dq.data_ptr(),
            B, Hq, Hkv, N, D, float(scale), int(bool(causal)), _stream(q),
        )
    _lib.check(rc)
    return dq


def flash_bwd_dq_delta(q, k, v, o, do, lse, causal: bool, scale: float):
    """Delta [B,H,N] fp32 = rowsum(O * dO) and dQ [B,Hq,N,D] (q's dtype) in one
    call (one launch when the dQ tiling computes Delta itself). Launches with
    few work-groups get a workspace for the library's split-KV dQ."""
    B, Hq, Hkv, N, Nkv, D = _qkv_dims(q, k, v)
    _require(o, "o", _elem_dtype(q, "q"), q.device)
    if o.shape != q.shape:
        raise ValueError("o must have the shape of q")
    delta = torch.empty((B, Hq, N), device=q.device, dtype=torch.float32)
    _check_bwd_inputs(q, k, v, do, lse, delta)
    q, k, v, o, do, lse = _aligned_all(q, k, v, o, do, lse)
    lib = _lib.load()
    c = int(bool(causal))
    ws_bytes = lib.fa_bwd_dq_workspace_bytes(B, Hq, Hkv, N, Nkv, D, c)
    if ws_bytes < 0:
        _lib.check(ws_bytes)
    extra = ()
    if ws_bytes > 0:  # few work-groups: dQ splits its keys over a workspace
        fn, lengths = _entry(lib, "fa_bwd_dq_delta_ws", q.dtype), (N, Nkv)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        extra = (ws.data_ptr(), ws_bytes)
    else:
        fn, lengths = _entry_lengths(lib, "fa_bwd_dq_delta", q.dtype, N, Nkv)
    dq = torch.empty_like(q)
    with _device_guard(q.device):
        rc = _launch(
            "dq", fn,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
            lse.data_ptr(), delta.data_ptr(), dq.data_ptr(),
            B, Hq, Hkv, *lengths, D, float(scale), c, *extra, _stream(q),
        )
    _lib.check(rc)
    return delta, dq


def flash_bwd(
    q, k, v, o, lse, do, causal: bool, scale: float
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """dQ, dK, dV of one backward through the library's whole-backward entry
    point ``fa_bwd`` (all of TritonAttention.backward's launches,
    attention.py:720-770), with one pass of checks, allocations and stream
    lookup (the host cost matters at small shapes). The split workspace, when
    the shape needs one, comes from the caching allocator. The library picks
    the launch plan: dQ with Delta fused, then dK/dV reading that Delta; or,
    when the dK/dV launch has too few key tiles to fill the GPU and splits
    while dQ does not and is short too, a Delta pass and one combined
    dK/dV + dQ launch."""
    dt = _elem_dtype(q, "q")
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o), ("dO", do)):
        _require(t, name, dt, q.device)
    _require(lse, "lse", torch.float32, q.device)
    B, Hq, Hkv, N, Nkv, D = _qkv_dims(q, k, v)
    if o.shape != q.shape or do.shape != q.shape:
        raise ValueError("o and dO must have the shape of q")
    if lse.shape != (B, Hq, N):
        raise ValueError("lse must have shape [B, Hq, N]")
    q, k, v, o, do, lse = _aligned_all(q, k, v, o, do, lse)
    lib = _lib.load()
    c = int(bool(causal))
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, Nkv, D, c)
    if ws_bytes < 0:
        _lib.check(ws_bytes)
    delta = torch.empty((B, Hq, N), device=q.device, dtype=torch.float32)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None
    with _device_guard(q.device):
        _lib.check(_launch(
            "bwd", _entry(lib, "fa_bwd", dt),
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
            lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
            B, Hq, Hkv, N, Nkv, D, float(scale), c,
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q),
        ))
    return dq, dk, dv
