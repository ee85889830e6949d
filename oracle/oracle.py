"""numpy front end of the CPU oracle (fa_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's parity and baseline legs, never by the triton_flash_attention
package. All results are float64.

Functions and the reference lines they restate
(/root/reference/triton_flash_attention/attention.py):
    fwd(..., online=False)  closed-form softmax attention, LSE base 2 (61-79, 230-231)
    fwd(..., online=True)   the tiled online-softmax recurrence with fp16 P (25-79, 170-234)
    bwd_preprocess          Delta = rowsum(O * dO) (237-255)
    bwd(..., fold=False)    dQ, dK, dV from LSE (258-350, 403-573), GQA group sums (503-505),
                            scores c q.k in exact arithmetic
    fwd / bwd with k, v of length Nkv != N: cross-attention as the reference's SDPA
                            fallback computes it (639-642, 830-838; top-left causal mask)
    fwd / bwd with v of head size Dv != D: the same fallback's other case (643-646)
    bwd(..., fold=True)     the same with the reference's fp16-rounded score operands,
                            fp16(c k) for dK/dV and fp16(c q) for dQ (435, 515);
                            fold="bfloat16" rounds them to bf16 (the added bf16 path)
    round_half              fp16 round-to-nearest-even (the .to(tl.float16) casts)
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"
SOURCE = ORACLE_DIR / "fa_oracle.c"

_lib = None


def build() -> Path:
    """Compile fa_oracle.c with the committed Makefile (always recompiles)."""
    subprocess.run(["make", "-B", "-s", "-C", str(ORACLE_DIR), "liboracle.so"], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    F64 = ctypes.c_double
    INT = ctypes.c_int
    lib.oracle_round_half.restype = F64
    lib.oracle_round_half.argtypes = [F64]
    lib.oracle_round_half_array.restype = None
    lib.oracle_round_half_array.argtypes = [P, P, I64]
    lib.oracle_fwd_direct.restype = None
    lib.oracle_fwd_direct.argtypes = [P, P, P, I64, I64, I64, I64, I64, I64, I64, F64, INT, P, P]
    lib.oracle_fwd_online.restype = None
    lib.oracle_fwd_online.argtypes = [P, P, P, I64, I64, I64, I64, I64, F64, INT, I64, I64, INT, P, P]
    lib.oracle_bwd_preprocess.restype = None
    lib.oracle_bwd_preprocess.argtypes = [P, P, I64, I64, P]
    lib.oracle_bwd.restype = None
    lib.oracle_bwd.argtypes = [P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, F64, INT, INT,
                               P, P, P]
    _lib = lib
    return lib


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.float64)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _dims(q, k, v):
    """(B, Hq, Hkv, N, Nkv, D, Dv) of q [B,Hq,N,D], k [B,Hkv,Nkv,D], v [B,Hkv,Nkv,Dv]."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must be 4-D [B, H, N, D]")
    B, Hq, N, D = q.shape
    if k.shape[:3] != v.shape[:3] or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("k/v shape mismatch")
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    return B, Hq, Hkv, N, k.shape[2], D, v.shape[3]


def round_half(x) -> np.ndarray:
    x = _f64(x)
    y = np.empty_like(x)
    _load().oracle_round_half_array(_ptr(x), _ptr(y), x.size)
    return y


def fwd(q, k, v, causal: bool, scale: float | None = None, *, online: bool = False,
        block_m: int = 128, block_n: int = 32, round_p: bool = True):
    """(O, LSE2): O [B,Hq,N,Dv] and base-2 LSE [B,Hq,N], float64. The closed
    form also takes k, v of another length Nkv (SDPA's top-left causal mask)
    and v of another head size Dv; the online form restates the reference's
    self-attention tiling only."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, Hq, Hkv, N, Nkv, D, Dv = _dims(q, k, v)
    if online and (Nkv != N or Dv != D):
        raise ValueError("the online form is self-attention with one head size only")
    scale = D ** -0.5 if scale is None else float(scale)
    o = np.empty((B, Hq, N, Dv), dtype=np.float64)
    lse = np.empty((B, Hq, N), dtype=np.float64)
    lib = _load()
    if online:
        lib.oracle_fwd_online(_ptr(q), _ptr(k), _ptr(v), B, Hq, Hkv, N, D, scale, int(causal),
                              block_m, block_n, int(round_p), _ptr(o), _ptr(lse))
    else:
        lib.oracle_fwd_direct(_ptr(q), _ptr(k), _ptr(v), B, Hq, Hkv, N, Nkv, D, Dv, scale,
                              int(causal), _ptr(o), _ptr(lse))
    return o, lse


def bwd_preprocess(o, do) -> np.ndarray:
    o, do = _f64(o), _f64(do)
    if o.shape != do.shape:
        raise ValueError("o and dO shapes differ")
    D = o.shape[-1]
    rows = o.size // D
    delta = np.empty(o.shape[:-1], dtype=np.float64)
    _load().oracle_bwd_preprocess(_ptr(o), _ptr(do), rows, D, _ptr(delta))
    return delta


_FOLD_MODES = {False: 0, True: 1, "float16": 1, "bfloat16": 2}


def bwd(q, k, v, do, lse2, delta, causal: bool, scale: float | None = None, *,
        fold: bool | str = False):
    """(dQ, dK, dV) float64 from the saved base-2 LSE and Delta. ``fold``: score
    operands rounded as the reference backward rounds them (attention.py:435,
    515), to fp16 (True or "float16") or to bf16 ("bfloat16")."""
    if fold not in _FOLD_MODES:
        raise ValueError(f"fold must be one of {list(_FOLD_MODES)}")
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    lse2, delta = _f64(lse2), _f64(delta)
    B, Hq, Hkv, N, Nkv, D, Dv = _dims(q, k, v)
    scale = D ** -0.5 if scale is None else float(scale)
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    _load().oracle_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(lse2), _ptr(delta),
                       B, Hq, Hkv, N, Nkv, D, Dv, scale, int(causal), _FOLD_MODES[fold],
                       _ptr(dq), _ptr(dk), _ptr(dv))
    return dq, dk, dv


def attention(q, k, v, do, causal: bool, scale: float | None = None, *, o16=None,
              fold_bwd: bool | str = False):
    """Full reference computation: O, LSE2, Delta, dQ, dK, dV (float64).

    Delta uses the fp16-rounded O the kernel stores, like the reference
    (attention.py:252-254); pass the kernel's own fp16 O as ``o16`` to use it
    exactly, otherwise the oracle's O is rounded to fp16.
    """
    o, lse = fwd(q, k, v, causal, scale)
    o_stored = round_half(o) if o16 is None else _f64(o16)
    delta = bwd_preprocess(o_stored, do)
    dq, dk, dv = bwd(q, k, v, do, lse, delta, causal, scale, fold=fold_bwd)
    return {"o": o, "lse": lse, "delta": delta, "dq": dq, "dk": dk, "dv": dv}
