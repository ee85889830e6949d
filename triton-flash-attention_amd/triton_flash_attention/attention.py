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
  5. sequence too long for 32-bit offsets   -> torch   (no reference counterpart)
  6. device is not gfx950                   -> torch   (replaces ref 662-666, SM >= 8)
  7. libfa_gfx950.so not loadable           -> torch   (replaces ref 649-652, the ROCm
                                                        reject); see below
  8. otherwise                              -> "triton" (the custom kernel backend)

The reference's first rule, cross-attention (N_q != N_kv) -> torch (ref 639-642),
is gone: the gfx950 kernels take separate query and key/value lengths and
compute what that SDPA fallback does, top-left causal mask included (query i
sees keys j <= i). Head sizes other than the kernels' 32, 64 and 128, and a
value head size other than the query/key one, are served up to 128:
:class:`TritonAttention` zero-pads the operands to the smallest kernel width
that holds both sizes (zero columns add exact zeros to every dot product) and
slices the results back.

The backend keeps the reference's name "triton" so existing call sites
(``backend="triton"``) run unchanged; it now means "the custom fused kernel".
On a gfx950 device an eligible input whose kernel library is missing is a
broken install, not an unsupported input: ``scaled_dot_product_attention``
raises instead of silently falling back (rule 8), unless ``backend="torch"``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from numbers import Real
from typing import Literal

import torch

from . import _lib, _ops

_SUPPORTED_HEAD_DIMS = (32, 64, 128)  # the kernels' widths; smaller sizes are zero-padded
_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)
_SUPPORTED_ARCH = "gfx950"
# Per-head slabs are addressed with 32-bit byte offsets (include/fa_gfx950.h).
_MAX_SLAB_BYTES = (1 << 31) - 4096 * 128 * 2
Backend = Literal["auto", "triton", "torch"]

_REASON_LIBRARY = "the gfx950 kernel library is not available"


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
    arch: str | None = None          # filled in only for GPU tensors
    library_error: str | None = None  # None when libfa_gfx950.so loaded


def _kernel_width(head_dim: int, value_head_dim: int) -> int | None:
    """The smallest kernel head size that holds both sizes, or None above 128."""
    need = max(head_dim, value_head_dim)
    return next((w for w in _SUPPORTED_HEAD_DIMS if w >= need), None)


def _decide(facts: _DispatchFacts) -> DispatchDecision:
    """First-match dispatch rules (ref attention.py:639-670, module docstring)."""
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
    if max(facts.q_len, facts.kv_len) * width * 2 > _MAX_SLAB_BYTES:
        return DispatchDecision(
            "torch", "the sequence is too long for the 32-bit addressed gfx950 kernel"
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
    no dot product, and their gradients are exactly zero.
    """

    @staticmethod
    def forward(ctx, query, key, value, causal, softmax_scale):
        head_dim, value_head_dim = query.shape[-1], value.shape[-1]
        query, key, value, output, lse = _padded_forward(query, key, value, causal, softmax_scale)
        ctx.save_for_backward(query, key, value, output, lse)
        ctx.head_dims = (head_dim, value_head_dim)
        ctx.softmax_scale = float(softmax_scale)
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
        if head_dim != query.shape[-1]:
            grad_query, grad_key = grad_query[..., :head_dim], grad_key[..., :head_dim]
        if value_head_dim != query.shape[-1]:
            grad_value = grad_value[..., :value_head_dim]
        return grad_query, grad_key, grad_value, None, None


def _forward_ad_active() -> bool:
    """Inside a forward-mode AD level, dual tensors carry tangents without
    requires_grad; such calls go through the autograd Function, which (like
    the reference's) defines no jvp and raises instead of dropping them."""
    return getattr(torch.autograd.forward_ad, "_current_level", -1) >= 0


def _padded_forward(query, key, value, causal, softmax_scale):
    """The forward launch at the kernel width: (padded q, k, v, O, LSE)."""
    width = _kernel_width(query.shape[-1], value.shape[-1])
    if width is None:
        raise ValueError(
            f"head sizes {query.shape[-1]} / {value.shape[-1]}: the gfx950 kernels serve at "
            f"most {_SUPPORTED_HEAD_DIMS[-1]}"
        )
    query, key, value = (_pad_head(t, width) for t in (query, key, value))
    output, lse = _ops.flash_fwd(query, key, value, bool(causal), float(softmax_scale))
    return query, key, value, output, lse


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
    attention, arbitrary positive sequence lengths, and GQA, for float16 or
    bfloat16 self- or cross-attention with head_dim and value head_dim up to 128
    (32, 64 and 128 natively, other sizes zero-padded). Other inputs
    fall back to PyTorch when ``backend="auto"``; ``backend="triton"`` requires
    the custom kernel and raises RuntimeError otherwise; ``backend="torch"``
    always uses PyTorch SDPA.
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
    if decision.backend == "torch":
        if backend == "triton" or decision.reason.startswith(_REASON_LIBRARY):
            raise RuntimeError(f"Triton backend is unavailable: {decision.reason}")
        return _torch_sdpa(
            query, key, value, is_causal=is_causal, scale=scale, enable_gqa=enable_gqa
        )

    softmax_scale = float(scale) if scale is not None else query.shape[-1] ** -0.5
    if not softmax_scale > 0.0:
        # The kernels fold the scale into a base-2 exponent and require scale > 0.
        if backend == "triton":
            raise RuntimeError(
                "Triton backend is unavailable: the gfx950 kernel requires scale > 0"
            )
        return _torch_sdpa(
            query, key, value, is_causal=is_causal, scale=scale, enable_gqa=enable_gqa
        )
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if (torch.is_grad_enabled() and (query.requires_grad or key.requires_grad
                                     or value.requires_grad)) or _forward_ad_active():
        return TritonAttention.apply(query, key, value, is_causal, softmax_scale)
    # No gradient can flow (inference, or under torch.no_grad()): the same
    # forward launch without the autograd Function's bookkeeping.
    output = _padded_forward(query, key, value, is_causal, softmax_scale)[3]
    return _unpad_output(output, value.shape[-1])
