"""ctypes binding of libfa_gfx950.so, the C ABI declared in include/fa_gfx950.h.

Only this module touches the shared library. Every entry point returns 0 on
success, a negative ``FA_ERR_*`` code for a rejected argument, or a positive
``hipError_t``; :func:`check` turns a non-zero code into :class:`FlashAttentionError`
carrying the library's thread-local message (``fa_last_error``).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from ._build import LIB_PATH

ABI_VERSION = 7

FA_OK = 0
FA_ERR_NULL_POINTER = -1
FA_ERR_BAD_SHAPE = -2
FA_ERR_HEAD_DIM = -3
FA_ERR_TOO_LARGE = -4
FA_ERR_BAD_SCALE = -5
FA_ERR_BAD_TILING = -6
FA_ERR_MISALIGNED = -7

KERNEL_FWD = 0
KERNEL_DKDV = 1
KERNEL_DQ = 2

# Every symbol include/fa_gfx950.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F32 = ctypes.c_float
_INT_P = ctypes.POINTER(ctypes.c_int)

SIGNATURES: dict[str, tuple[object, tuple[object, ...]]] = {
    "fa_fwd": (_INT, (_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _INT, _P)),
    "fa_bwd_preprocess": (_INT, (_P, _P, _P, _I64, _I64, _I64, _I64, _P)),
    "fa_bwd_dkdv": (
        _INT,
        (_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _INT, _P),
    ),
    "fa_bwd_dkdv_workspace_bytes": (_I64, (_I64, _I64, _I64, _I64, _I64, _INT)),
    "fa_bwd_dkdv_ws": (
        _INT,
        (_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _INT, _P, _I64, _P),
    ),
    "fa_bwd_dq": (
        _INT,
        (_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _INT, _P),
    ),
    "fa_bwd_dq_delta": (
        _INT,
        (_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F32, _INT, _P),
    ),
    "fa_fwd_plan_info": (_INT, (_I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, ctypes.POINTER(ctypes.c_int64))),
    "fa_last_error": (ctypes.c_char_p, ()),
    "fa_abi_version": (_INT, ()),
    "fa_get_tiling": (_INT, (_INT, _I64, _INT, _INT_P)),
    "fa_num_tiling_variants": (_INT, (_INT, _I64, _INT)),
    "fa_describe_tiling_variant": (_INT, (_INT, _I64, _INT, _INT, _INT_P)),
    "fa_set_tiling": (_INT, (_INT, _I64, _INT, _INT)),
}
# bfloat16 twins of the launches: the same arguments.
for _name in ("fa_fwd", "fa_bwd_preprocess", "fa_bwd_dkdv", "fa_bwd_dkdv_ws", "fa_bwd_dq",
              "fa_bwd_dq_delta"):
    SIGNATURES[_name + "_bf16"] = SIGNATURES[_name]
# Cross-attention launches: one more length (N_kv) after N, fp16 and bf16.
SIGNATURES["fa_bwd_dkdv_workspace_bytes_kv"] = (_I64, (_I64, _I64, _I64, _I64, _I64, _I64, _INT))
for _name, _n_ptr in (("fa_fwd", 5), ("fa_bwd_dkdv_ws", 8), ("fa_bwd_dq_delta", 8)):
    _res, _args = SIGNATURES[_name]
    _kv = (_res, _args[:_n_ptr + 4] + (_I64,) + _args[_n_ptr + 4:])  # ..., N_q, N_kv, D, ...
    SIGNATURES[_name + "_kv"] = _kv
    SIGNATURES[_name + "_kv_bf16"] = _kv
del _name, _n_ptr, _res, _args, _kv
# Forward with a split-KV workspace: fa_fwd_kv's arguments, then workspace, its size, stream.
SIGNATURES["fa_fwd_workspace_bytes"] = (_I64, (_I64, _I64, _I64, _I64, _I64, _I64, _INT))
SIGNATURES["fa_fwd_ws"] = (_INT, SIGNATURES["fa_fwd_kv"][1][:-1] + (_P, _I64, _P))
SIGNATURES["fa_fwd_ws_bf16"] = SIGNATURES["fa_fwd_ws"]
# dQ with Delta and a split-KV workspace: fa_bwd_dq_delta_kv's arguments, then workspace, size, stream.
SIGNATURES["fa_bwd_dq_workspace_bytes"] = SIGNATURES["fa_fwd_workspace_bytes"]
SIGNATURES["fa_bwd_dq_delta_ws"] = (_INT, SIGNATURES["fa_bwd_dq_delta_kv"][1][:-1] + (_P, _I64, _P))
SIGNATURES["fa_bwd_dq_delta_ws_bf16"] = SIGNATURES["fa_bwd_dq_delta_ws"]
# Whole backward: q, k, v, o, dO, lse, delta, dq, dk, dv, B, Hq, Hkv, N_q, N_kv, D, scale,
# causal, workspace, its size, stream.
SIGNATURES["fa_bwd_workspace_bytes"] = SIGNATURES["fa_fwd_workspace_bytes"]
SIGNATURES["fa_bwd"] = (
    _INT,
    (_P,) * 10 + (_I64, _I64, _I64, _I64, _I64, _I64, _F32, _INT, _P, _I64, _P),
)
SIGNATURES["fa_bwd_bf16"] = SIGNATURES["fa_bwd"]
# Forward without allocation (device-resident scratch): fa_fwd_kv's arguments.
SIGNATURES["fa_fwd_noalloc"] = SIGNATURES["fa_fwd_kv"]
SIGNATURES["fa_fwd_noalloc_max_workspace_bytes"] = (_I64, ())


class FlashAttentionError(RuntimeError):
    """A libfa_gfx950 call failed (argument rejected or HIP error)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"libfa_gfx950 error {code}: {message}")
        self.code = code


class LibraryUnavailable(RuntimeError):
    """libfa_gfx950.so is missing or could not be loaded."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def library_path() -> Path:
    return LIB_PATH


def _bind(lib: ctypes.CDLL) -> None:
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = list(argtypes)


def load() -> ctypes.CDLL:
    """Load and bind the library once per process; raise LibraryUnavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            _load_error = (
                f"{path.name} is not built (expected at {path}); run "
                "`python -m triton_flash_attention._build`"
            )
            raise LibraryUnavailable(_load_error)
        # torch must be imported first so the library binds to the HIP runtime
        # torch already loaded (same soname) and shares its streams.
        import torch  # noqa: F401

        try:
            lib = ctypes.CDLL(str(path))
            _bind(lib)
        except (OSError, AttributeError) as exc:
            _load_error = f"could not load {path}: {exc}"
            raise LibraryUnavailable(_load_error) from exc
        version = lib.fa_abi_version()
        if version != ABI_VERSION:
            _load_error = f"{path.name} has ABI version {version}, expected {ABI_VERSION}"
            raise LibraryUnavailable(_load_error)
        _lib = lib
        _load_error = None
        return lib


def available() -> tuple[bool, str]:
    """(True, "") if the library loads, else (False, reason)."""
    try:
        load()
    except LibraryUnavailable as exc:
        return False, str(exc)
    return True, ""


def last_error() -> str:
    raw = load().fa_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def check(code: int) -> None:
    if code != FA_OK:
        raise FlashAttentionError(code, last_error())


def get_tiling(kernel: int, head_dim: int, causal: bool) -> dict[str, int]:
    out = (ctypes.c_int * 4)()
    check(load().fa_get_tiling(kernel, head_dim, int(causal), out))
    return {"waves": out[0], "rows": out[1], "tile": out[2], "variant": out[3]}


def tiling_variants(kernel: int, head_dim: int, causal: bool) -> list[dict[str, int]]:
    lib = load()
    count = lib.fa_num_tiling_variants(kernel, head_dim, int(causal))
    if count < 0:
        check(count)
    result = []
    for index in range(count):
        out = (ctypes.c_int * 4)()
        rc = lib.fa_describe_tiling_variant(kernel, head_dim, int(causal), index, out)
        if rc == FA_ERR_BAD_TILING:
            continue  # not compiled for this head_dim
        check(rc)
        result.append({"waves": out[0], "rows": out[1], "tile": out[2], "variant": out[3]})
    return result


def fwd_plan_info(B: int, Hq: int, Hkv: int, N_q: int, N_kv: int, D: int, causal: bool,
                  compute_units: int = 0) -> dict[str, int]:
    """The forward's launch plan for these sizes (fa_fwd_plan_info): work-groups
    of the persistent job-plan grid (0: the grid form runs), of the grid form,
    and the modelled makespans (32-key units per slot) of both."""
    out = (ctypes.c_int64 * 4)()
    check(load().fa_fwd_plan_info(B, Hq, Hkv, N_q, N_kv, D, int(causal), compute_units, out))
    return {"plan_workgroups": out[0], "grid_workgroups": out[1],
            "plan_makespan": out[2], "grid_makespan": out[3]}


def set_tiling(kernel: int, head_dim: int, causal: bool, variant: int) -> None:
    """Select a compiled tiling for this process (variant < 0 restores the table)."""
    check(load().fa_set_tiling(kernel, head_dim, int(causal), variant))
