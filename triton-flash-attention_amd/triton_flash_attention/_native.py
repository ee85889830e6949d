"""Loader of the C++ autograd binding (``_fa_native.so``, csrc/fa_native.cpp).

The binding runs the public API's training path (forward + backward through
the autograd engine) in C++ with the same library calls as the Python
``TritonAttention`` Function, so its results are identical bit for bit; it
only saves host time. It is built in-tree next to libfa_gfx950.so
(``_build.build_native``) and takes the entry points of the copy of the
library that ``_lib`` has loaded. If it is missing or fails to load, the
public API uses the Python Function (the same kernels); ``status()`` says why.
"""

from __future__ import annotations

import ctypes
import importlib.machinery
import importlib.util
from pathlib import Path

from . import _lib

NAME = "_fa_native"
PATH = Path(__file__).resolve().parent / f"{NAME}.so"

# Entry points handed to init(), in its argument order.
ENTRY_POINTS = ("fa_fwd_kv", "fa_fwd_kv_bf16", "fa_fwd_ws", "fa_fwd_ws_bf16", "fa_bwd",
                "fa_bwd_bf16", "fa_fwd_workspace_bytes", "fa_bwd_workspace_bytes",
                "fa_last_error")

_module = None
_error: str | None = None
_tried = False


def _load():
    global _module, _error, _tried
    _tried = True
    if not PATH.exists():
        _error = f"{PATH.name} is not built"
        return
    ok, why = _lib.available()
    if not ok:
        _error = why
        return
    try:
        import torch  # noqa: F401  (the binding links against torch's libraries)

        loader = importlib.machinery.ExtensionFileLoader(NAME, str(PATH))
        spec = importlib.util.spec_from_file_location(NAME, str(PATH), loader=loader)
        module = importlib.util.module_from_spec(spec)
        loader.exec_module(module)
        lib = _lib.load()
        module.init(*(ctypes.cast(getattr(lib, n), ctypes.c_void_p).value for n in ENTRY_POINTS))
    except Exception as exc:  # noqa: BLE001 - reported by status()
        _error = f"{PATH.name} failed to load: {exc}"
        return
    _module = module


def available() -> bool:
    if not _tried:
        _load()
    return _module is not None


def status() -> tuple[bool, str]:
    """(loaded, reason it is not)."""
    return available(), _error or ""


def forward(query, key, value, causal: bool, scale: float):
    """O = attention(query, key, value) without autograd, through the binding
    (same served case as :func:`attention`)."""
    return _module.forward(query, key, value, bool(causal), float(scale))


def attention(query, key, value, causal: bool, scale: float):
    """O = attention(query, key, value), differentiable, through the binding.
    The caller guarantees the served case: contiguous fp16/bf16 GPU tensors,
    one head size for q, k, v among 32, 64, 128, and a positive scale."""
    return _module.attention(query, key, value, bool(causal), float(scale))
