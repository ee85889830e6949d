"""Public attention API: validation, backend dispatch and the autograd bridge.

This mirrors the host side of the reference (triton_flash_attention/attention.py):
the same public names, keyword-only signatures, defaults, validation order and
messages, and the same PyTorch SDPA fallback. What changes is the device side:
eligible inputs run the hand-written gfx950 HIP kernels of libfa_gfx950.so
through :mod:`._ops` instead of Triton kernels.

Dispatch rules (first match wins; reference rules at attention.py:629-670):
  1. value head size != query head size     -> torch   (ref 643-646), unless both are
     and either is above 128                           at most 128 (added)
  2. not a GPU ("cuda") tensor              -> torch   (ref 647-648)
  3. dtype is not float16 or bfloat16       -> torch   (ref 653-656 accepts float16
                                                        only; bfloat16 is an added
                                                        dtype of the gfx950 kernels)
  4. head_dim above 128                     -> torch   (ref 657-661 also rejects every
                                                        size other than 32, 64, 128)
  5. sequence or batch*heads too large for  -> torch   (no reference counterpart; the
     the library's 32-bit addressing                    exact bounds of fa_capi.hip)
  6. device is not gfx950                   -> torch   (replaces ref 662-666, SM >= 8)
  7. libfa_gfx950.so not loadable           -> torch   (replaces ref 649-652, the ROCm
                                                        reject)
  8. otherwise                              -> "triton" (the custom kernel backend)

Cross-attention (N_q != N_kv) is served by the gfx950 kernels, which take
separate query and key/value lengths and compute what the reference's SDPA
fallback computes, top-left causal mask included (query i sees keys j <= i).
Where rules 1-7 send cross-attention inputs to torch, the reason starts with
the reference's first-rule reason (ref 639-642, "the custom kernel currently
specializes in self-attention") so that callers matching on it keep working,
followed by the rule that decided here. Head sizes other than the kernels'
32, 64 and 128, and a value head size other than the query/key one, are served
up to 128: :class:`TritonAttention` zero-pads the operands to the smallest
kernel width that holds both sizes (zero columns add exact zeros to every dot
product) and slices the results back.

The backend keeps the reference's name "triton" so existing call sites
(``backend="triton"``) run unchanged; it now means "the custom fused kernel".
As in the reference, ``backend="auto"`` never raises for an unavailable
backend: a missing or unloadable kernel library on a gfx950 device falls back
to SDPA with the library's error as the reason (and one RuntimeWarning per
process, since that is a broken install), while ``backend="triton"`` raises.

Every finite scale is served, as the reference's kernel serves it
(ref 812-815, 844-845): the kernels take a positive scale, so a negative one
runs on the negated query (q.k scale = (-q).k |scale| exactly, dQ negated
back) and a zero one (also a scale that rounds to zero in float32) runs on a
zero query at scale 1 (every score is exactly 0, as with scale 0; dQ = 0).
"""

from __future__ import annotations

import ctypes
import math
import warnings
from dataclasses import dataclass
from numbers import Real
from typing import Literal

import torch

from . import _lib, _native, _ops

_SUPPORTED_HEAD_DIMS = (32, 64, 128)  # the kernels' widths; smaller sizes are zero-padded
_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)
_SUPPORTED_ARCH = "gfx950"
Backend = Literal["auto", "triton", "torch"]

_REASON_LIBRARY = "the gfx950 kernel library is not available"
# The reference's first rule (attention.py:639-642), kept as the start of the
# reason whenever cross-attention inputs fall back.
_REASON_CROSS = "the custom kernel currently specializes in self-attention"


def _sequence_fits(length: int, width: int) -> bool:
    """The library's per-head slab bound for a sequence of ``length`` rows at
    kernel width ``width`` (fa_capi.hip check_common / check_kv_length:
    rows are addressed with 32-bit byte offsets, a 4096-row margin included)."""
    return length * width * 2 + 4096 * width * 2 < (1 << 31)


def _max_sequence(width: int) -> int:
    """The longest sequence :func:`_sequence_fits` accepts at ``width``."""
    return ((1 << 31) - 1 - 4096 * width * 2) // (width * 2)


# fa_capi.hip check_common: batch * query heads < 2^30.
_MAX_BATCH_HEADS = 1 << 30


@dataclass(frozen=True)
class DispatchDecision:
    """The selected backend and the concrete reason for the decision."""

    backend: Literal["triton", "torch"]
    reason: str


def _validate_inputs(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    enable_gqa: bool,
) -> None:
    """Shape/device/dtype contract of the public API (ref attention.py:584-626)."""
    for name, tensor in (("query", query), ("key", key), ("value", value)):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if tensor.ndim != 4:
            raise ValueError(
                f"{name} must have shape (batch, heads, sequence, head_dim); "
                f"got {tuple(tensor.shape)}"
            )
        if 0 in tensor.shape:
            raise ValueError(f"{name} dimensions must all be greater than zero")

    if not (query.device == key.device == value.device):
        raise ValueError("query, key, and value must be on the same device")
    if not (query.dtype == key.dtype == value.dtype):
        raise ValueError("query, key, and value must have the same dtype")
    if not (query.shape[0] == key.shape[0] == value.shape[0]):
        raise ValueError("query, key, and value batch dimensions must match")
    if key.shape[:3] != value.shape[:3]:
        raise ValueError(
            "key and value batch, head, and sequence dimensions must match"
        )
    if query.shape[3] != key.shape[3]:
        raise ValueError("query and key head dimensions must match")

    q_heads, kv_heads = query.shape[1], key.shape[1]
    if q_heads != kv_heads and not enable_gqa:
        raise ValueError(
            "query has a different number of heads from key/value; pass "
            "enable_gqa=True to use grouped-query attention"
        )
    if q_heads % kv_heads:
        raise ValueError(
            "the number of query heads must be divisible by the number of "
            "key/value heads"
        )


_arch_cache: dict[int, str] = {}


def _device_arch(device: torch.device) -> str:
    index = device.index if device.index is not None else torch.cuda.current_device()
    arch = _arch_cache.get(index)
    if arch is None:
        props = torch.cuda.get_device_properties(index)
        arch = getattr(props, "gcnArchName", "") or ""
        _arch_cache[index] = arch
    return arch


@dataclass(frozen=True)
class _DispatchFacts:
    """What the dispatch rules look at, gathered from already-validated inputs."""

    q_len: int
    kv_len: int
    head_dim: int
    value_head_dim: int
    device_type: str
    dtype: torch.dtype
    batch_heads: int = 1             # batch * query heads
    arch: str | None = None          # filled in only for GPU tensors
    library_error: str | None = None  # None when libfa_gfx950.so loaded


def _kernel_width(head_dim: int, value_head_dim: int) -> int | None:
    """The smallest kernel head size that holds both sizes, or None above 128."""
    need = max(head_dim, value_head_dim)
    return next((w for w in _SUPPORTED_HEAD_DIMS if w >= need), None)


def _decide(facts: _DispatchFacts) -> DispatchDecision:
    """First-match dispatch rules (ref attention.py:639-670, module docstring).

    Cross-attention inputs that fall back keep the reference's first-rule
    reason in front (ref 639-642), then the rule that decided here."""
    decision = _decide_rules(facts)
    if decision.backend == "torch" and facts.q_len != facts.kv_len:
        return DispatchDecision(
            "torch", f"{_REASON_CROSS} (cross-attention runs on gfx950 only; here {decision.reason})"
        )
    return decision


def _decide_rules(facts: _DispatchFacts) -> DispatchDecision:
    if facts.value_head_dim != facts.head_dim and (
        _kernel_width(facts.head_dim, facts.value_head_dim) is None
    ):
        return DispatchDecision(
            "torch",
            "the custom kernel requires equal query/key and value head sizes, or two "
            f"different ones of at most {_SUPPORTED_HEAD_DIMS[-1]}",
        )
    if facts.device_type != "cuda":
        return DispatchDecision("torch", "the Triton kernel requires a CUDA tensor")
    if facts.dtype not in _SUPPORTED_DTYPES:
        return DispatchDecision(
            "torch", "the custom mixed-precision path currently supports float16 and bfloat16"
        )
    width = _kernel_width(facts.head_dim, facts.value_head_dim)
    if width is None:
        supported = ", ".join(str(dim) for dim in _SUPPORTED_HEAD_DIMS)
        return DispatchDecision(
            "torch",
            f"head_dim must be one of ({supported}) for the Triton path, or a smaller size "
            "that is zero-padded to one of them",
        )
    if not (_sequence_fits(facts.q_len, width) and _sequence_fits(facts.kv_len, width)):
        return DispatchDecision(
            "torch", "the sequence is too long for the 32-bit addressed gfx950 kernel"
        )
    if facts.batch_heads >= _MAX_BATCH_HEADS:
        return DispatchDecision(
            "torch", "batch * heads is too large for the 32-bit addressed gfx950 kernel"
        )
    arch = facts.arch or ""
    if not arch.startswith(_SUPPORTED_ARCH):
        return DispatchDecision(
            "torch",
            "the tuned kernel requires an AMD Instinct MI355X (gfx950) GPU; "
            f"found {arch or 'an unknown device'}",
        )
    if facts.library_error is not None:
        return DispatchDecision("torch", f"{_REASON_LIBRARY}: {facts.library_error}")
    kind = "self-attention" if facts.q_len == facts.kv_len else "cross-attention"
    padded = ""
    if (facts.head_dim, facts.value_head_dim) != (width, width):
        sizes = (str(facts.head_dim) if facts.value_head_dim == facts.head_dim
                 else f"{facts.head_dim} / value {facts.value_head_dim}")
        padded = f" (head_dim {sizes}: zero-padded to {width})"
    return DispatchDecision(
        "triton",
        f"gfx950 {str(facts.dtype).removeprefix('torch.')} {kind} with a supported "
        "head dimension" + padded,
    )


def explain_dispatch(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    enable_gqa: bool = False,
) -> DispatchDecision:
    """Explain whether the custom gfx950 kernel can serve these inputs."""
    _validate_inputs(query, key, value, enable_gqa=enable_gqa)
    return _dispatch(query, key, value)


def _dispatch(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> DispatchDecision:
    """The dispatch decision for inputs that already passed ``_validate_inputs``
    (the public API validates once, then decides)."""
    arch = library_error = None
    if query.device.type == "cuda":
        ok, why = _lib.available()
        arch, library_error = _device_arch(query.device), None if ok else why
    return _decide(_DispatchFacts(
        q_len=query.shape[2],
        kv_len=key.shape[2],
        head_dim=query.shape[3],
        value_head_dim=value.shape[3],
        device_type=query.device.type,
        dtype=query.dtype,
        batch_heads=query.shape[0] * query.shape[1],
        arch=arch,
        library_error=library_error,
    ))


class TritonAttention(torch.autograd.Function):
    """Low-level autograd bridge for the custom forward and backward kernels.

    Same contract as the reference class (attention.py:673-771):
    ``apply(query, key, value, causal, softmax_scale) -> output`` on contiguous
    fp16 or bf16 query [B, Hq, N, D], key [B, Hkv, N_kv, D] and value
    [B, Hkv, N_kv, D_v] tensors; backward returns ``(dQ, dK, dV, None, None)``.
    Unless D and D_v are the same kernel size (32, 64 or 128), the kernels run
    at the smallest kernel size that holds both, on zero-padded copies of the
    operands (and of dO), and the outputs are sliced back: zero columns change
    no dot product, and their gradients are exactly zero. A scale that is not
    positive in float32 runs as :func:`_kernel_scale` describes.
    """

    @staticmethod
    def forward(ctx, query, key, value, causal, softmax_scale):
        head_dim, value_head_dim = query.shape[-1], value.shape[-1]
        query, key, value, output, lse, kscale, mode = _padded_forward(
            query, key, value, causal, softmax_scale)
        ctx.save_for_backward(query, key, value, output, lse)
        ctx.head_dims = (head_dim, value_head_dim)
        ctx.softmax_scale = kscale
        ctx.scale_mode = mode
        ctx.causal = bool(causal)
        return _unpad_output(output, value_head_dim)

    @staticmethod
    def backward(ctx, grad_output):
        query, key, value, output, lse = ctx.saved_tensors
        head_dim, value_head_dim = ctx.head_dims
        grad_output = _pad_head(grad_output.contiguous(), query.shape[-1])
        grad_query, grad_key, grad_value = _ops.flash_bwd(
            query, key, value, output, lse, grad_output, ctx.causal, ctx.softmax_scale
        )
        if ctx.scale_mode == "negate":
            grad_query = -grad_query  # d/dq of (-q).k |scale|
        elif ctx.scale_mode == "zero":
            grad_query = torch.zeros_like(grad_query)  # the scores do not depend on q
        if head_dim != query.shape[-1]:
            grad_query, grad_key = grad_query[..., :head_dim], grad_key[..., :head_dim]
        if value_head_dim != query.shape[-1]:
            grad_value = grad_value[..., :value_head_dim]
        return grad_query, grad_key, grad_value, None, None


def _native_serves(query: torch.Tensor, value: torch.Tensor, softmax_scale: float) -> bool:
    """Whether the C++ binding (``_native``) runs this call: it makes
    TritonAttention's launches (or, without autograd, the forward's) for a
    positive scale and one kernel head size for q, k and v; padded head sizes,
    negative or zero scales and forward-mode AD stay in Python."""
    head_dim = query.shape[-1]
    return (head_dim in _SUPPORTED_HEAD_DIMS and value.shape[-1] == head_dim
            and not _forward_ad_active() and _kernel_scale(softmax_scale)[1] == "plain"
            and _native.available())


def _forward_ad_active() -> bool:
    """Inside a forward-mode AD level, dual tensors carry tangents without
    requires_grad; such calls go through the autograd Function, which (like
    the reference's) defines no jvp and raises instead of dropping them."""
    return getattr(torch.autograd.forward_ad, "_current_level", -1) >= 0


_LOG2E = 1.4426950408889634  # the kernels' fp32 constant scale * log2(e) (fa_kernels.hpp)


def _float32(x: float) -> float:
    return ctypes.c_float(x).value


def _kernel_scale(softmax_scale: float) -> tuple[float, str] | None:
    """(positive kernel scale, query transform) serving ``softmax_scale``, or
    None when float32 cannot hold it.

    The library takes a scale whose float32 value c = scale * log2(e) is
    positive and normal (fa_capi.hip check_scale). The reference's kernel takes
    any finite scale (attention.py:812-815, 844-845), so:
      * "plain":  scale as given;
      * "negate": scale < 0 runs on -q at |scale|; every score (-q).k |scale|
        equals q.k scale exactly (fp16 negation and round-to-nearest are
        sign-symmetric, also for the backward's fp16(c q) and fp16(c k)
        operands), and dQ is negated back;
      * "zero":   |scale| below the float32 normal range (0 included) runs on
        a zero query at scale 1: every score is exactly 0 either way (with a
        subnormal scale every exp2 argument rounds to 0 in float32), so P, O,
        LSE, dV and dK (= scale dS^T Q, which is 0) agree, and dQ (= scale dS K)
        is 0.
    """
    s32 = _float32(softmax_scale)
    if not math.isfinite(s32) or not math.isfinite(_float32(abs(s32) * _LOG2E)):
        return None
    if abs(s32) < 2.0 ** -126:
        return 1.0, "zero"
    if s32 < 0.0:
        return -float(softmax_scale), "negate"
    return float(softmax_scale), "plain"


def _padded_forward(query, key, value, causal, softmax_scale):
    """The forward launch at the kernel width: (padded q, k, v, O, LSE, kernel
    scale, scale mode), q as the kernels saw it (see :func:`_kernel_scale`)."""
    width = _kernel_width(query.shape[-1], value.shape[-1])
    if width is None:
        raise ValueError(
            f"head sizes {query.shape[-1]} / {value.shape[-1]}: the gfx950 kernels serve at "
            f"most {_SUPPORTED_HEAD_DIMS[-1]}"
        )
    served = _kernel_scale(float(softmax_scale))
    if served is None:
        raise ValueError(f"scale {softmax_scale!r} overflows the kernels' float32 arithmetic")
    kscale, mode = served
    if mode == "negate":
        query = -query
    elif mode == "zero":
        query = torch.zeros_like(query)
    query, key, value = (_pad_head(t, width) for t in (query, key, value))
    output, lse = _ops.flash_fwd(query, key, value, bool(causal), kscale)
    return query, key, value, output, lse, kscale, mode


def _unpad_output(output: torch.Tensor, value_head_dim: int) -> torch.Tensor:
    return (output if output.shape[-1] == value_head_dim
            else output[..., :value_head_dim].contiguous())


def _pad_head(t: torch.Tensor, width: int) -> torch.Tensor:
    """``t``, or a contiguous copy with its last dimension zero-padded to ``width``."""
    return t if t.shape[-1] == width else torch.nn.functional.pad(t, (0, width - t.shape[-1]))


def _torch_sdpa(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    is_causal: bool,
    scale: float | None,
    enable_gqa: bool,
) -> torch.Tensor:
    """The reference's fallback (attention.py:774-786), unchanged in meaning."""
    kwargs = {"is_causal": is_causal, "scale": scale}
    if enable_gqa:
        kwargs["enable_gqa"] = True
    return torch.nn.functional.scaled_dot_product_attention(query, key, value, **kwargs)


def scaled_dot_product_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    is_causal: bool = False,
    scale: float | None = None,
    enable_gqa: bool = False,
    backend: Backend = "auto",
) -> torch.Tensor:
    """Compute scaled dot-product attention with safe backend selection.

    The custom gfx950 path supports forward/backward, causal and bidirectional
    attention, arbitrary positive sequence lengths, GQA and any finite scale,
    for float16 or bfloat16 self- or cross-attention with head_dim and value
    head_dim up to 128 (32, 64 and 128 natively, other sizes zero-padded).
    Other inputs fall back to PyTorch when ``backend="auto"``;
    ``backend="triton"`` requires the custom kernel and raises RuntimeError
    otherwise; ``backend="torch"`` always uses PyTorch SDPA.
    """
    if backend not in ("auto", "triton", "torch"):
        raise ValueError("backend must be one of: 'auto', 'triton', 'torch'")
    if not isinstance(is_causal, bool):
        raise TypeError("is_causal must be a bool")
    if not isinstance(enable_gqa, bool):
        raise TypeError("enable_gqa must be a bool")
    if scale is not None and (
        not isinstance(scale, Real) or not math.isfinite(float(scale))
    ):
        raise ValueError("scale must be a finite real number or None")
    _validate_inputs(query, key, value, enable_gqa=enable_gqa)

    if backend == "torch":
        return _torch_sdpa(
            query, key, value, is_causal=is_causal, scale=scale, enable_gqa=enable_gqa
        )

    decision = _dispatch(query, key, value)
    softmax_scale = float(scale) if scale is not None else query.shape[-1] ** -0.5
    if decision.backend == "triton" and _kernel_scale(softmax_scale) is None:
        decision = DispatchDecision(
            "torch", f"scale {softmax_scale!r} overflows the gfx950 kernel's float32 arithmetic")
    if decision.backend == "torch":
        if backend == "triton":
            raise RuntimeError(f"Triton backend is unavailable: {decision.reason}")
        if _REASON_LIBRARY in decision.reason:
            _warn_library_once(decision.reason)
        return _torch_sdpa(
            query, key, value, is_causal=is_causal, scale=scale, enable_gqa=enable_gqa
        )

    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if (torch.is_grad_enabled() and (query.requires_grad or key.requires_grad
                                     or value.requires_grad)) or _forward_ad_active():
        if _native_serves(query, value, softmax_scale):
            # The same library calls as TritonAttention, from C++ (less host time).
            return _native.attention(query, key, value, is_causal, softmax_scale)
        return TritonAttention.apply(query, key, value, is_causal, softmax_scale)
    # No gradient can flow (inference, or under torch.no_grad()): the same
    # forward launch without the autograd Function's bookkeeping.
    if _native_serves(query, value, softmax_scale):
        return _native.forward(query, key, value, is_causal, softmax_scale)
    output = _padded_forward(query, key, value, is_causal, softmax_scale)[3]
    return _unpad_output(output, value.shape[-1])


_library_warned = False


def _warn_library_once(reason: str) -> None:
    """One RuntimeWarning per process when an eligible gfx950 input falls back
    because the kernel library did not load (a broken install)."""
    global _library_warned
    if not _library_warned:
        _library_warned = True
        warnings.warn(f"falling back to torch SDPA: {reason}", RuntimeWarning, stacklevel=3)
