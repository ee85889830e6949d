"""Shared helpers for the test suite: seeded inputs, error metrics, and a plain
PyTorch fp32 attention reference for full-size GPU checks."""

from __future__ import annotations

import math

import numpy as np
import torch

# The five BASELINE.json configurations (B, Hq, Hkv, N, D, causal modes, input scale).
CONFIGS = {
    "c1": dict(B=1, Hq=4, Hkv=4, N=257, D=64, causal=(False,), mult=1.0, seed=1001),
    "c2": dict(B=4, Hq=16, Hkv=16, N=4096, D=64, causal=(True,), mult=1.0, seed=1002),
    "c3": dict(B=2, Hq=16, Hkv=4, N=2049, D=64, causal=(True,), mult=1.0, seed=1003),
    "c4": dict(B=2, Hq=32, Hkv=32, N=8192, D=128, causal=(False, True), mult=0.5, seed=1004),
    "c5": dict(B=1, Hq=8, Hkv=2, N=16381, D=32, causal=(True,), mult=1.0, seed=1005),
}

# Tolerances stated by BASELINE.json's north_star.
MAX_ABS_TOL = 2e-2
REL_L2_TOL = 5e-3
LSE_TOL = 1e-4


def make_inputs(B, Hq, Hkv, N, D, seed, mult=1.0, do_mult=None, dtype=torch.float16, n_kv=None,
                d_v=None):
    """q, k, v, dO as CPU tensors of ``dtype`` (fp16 by default): fp32 N(0,1)
    from a seeded CPU generator drawn in the order q, k, v, dO, times ``mult``
    (dO times ``do_mult``, default ``mult``), then cast. k and v have ``n_kv``
    rows (default N); v and dO have head size ``d_v`` (default D)."""
    g = torch.Generator("cpu").manual_seed(seed)
    do_mult = mult if do_mult is None else do_mult
    n_kv = N if n_kv is None else n_kv
    d_v = D if d_v is None else d_v
    q = torch.randn((B, Hq, N, D), generator=g, dtype=torch.float32) * mult
    k = torch.randn((B, Hkv, n_kv, D), generator=g, dtype=torch.float32) * mult
    v = torch.randn((B, Hkv, n_kv, d_v), generator=g, dtype=torch.float32) * mult
    do = torch.randn((B, Hq, N, d_v), generator=g, dtype=torch.float32) * do_mult
    return q.to(dtype), k.to(dtype), v.to(dtype), do.to(dtype)


def errors(actual, expected) -> tuple[float, float]:
    """(max-abs error, relative L2 error ||a-e|| / ||e||) in float64."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    diff = a - e
    max_abs = float(np.max(np.abs(diff))) if diff.size else 0.0
    denom = float(np.linalg.norm(e))
    rel = float(np.linalg.norm(diff)) / denom if denom > 0 else float(np.linalg.norm(diff))
    return max_abs, rel


def errors_torch(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float]:
    a = actual.double()
    e = expected.double()
    diff = a - e
    max_abs = float(diff.abs().max()) if diff.numel() else 0.0
    denom = float(torch.linalg.vector_norm(e))
    num = float(torch.linalg.vector_norm(diff))
    return max_abs, (num / denom if denom > 0 else num)


def assert_close(name, actual, expected, max_abs=MAX_ABS_TOL, rel_l2=REL_L2_TOL):
    if isinstance(actual, torch.Tensor):
        ma, rl = errors_torch(actual, expected)
    else:
        ma, rl = errors(actual, expected)
    assert ma <= max_abs and rl <= rel_l2, (
        f"{name}: max-abs {ma:.3e} (tol {max_abs:.1e}), rel-L2 {rl:.3e} (tol {rel_l2:.1e})"
    )
    return ma, rl


@torch.no_grad()
def torch_reference_fp32(q, k, v, do, causal, scale=None, o16=None):
    """Plain PyTorch fp32 attention forward + backward on q's device.

    Processes one key/value head (and its GQA group of query heads) at a time
    with explicit contiguous matmuls. Returns fp32 tensors O, LSE2 (base 2),
    dQ, dK, dV. Delta uses ``o16`` (the fp16 output the kernel stored) when
    given, otherwise the reference O rounded to fp16 — the Delta definition of
    the reference backward (attention.py:252-254).
    """
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    scale = D ** -0.5 if scale is None else float(scale)
    dev = q.device
    o = torch.empty((B, Hq, N, D), device=dev, dtype=torch.float32)
    lse2 = torch.empty((B, Hq, N), device=dev, dtype=torch.float32)
    dq = torch.empty_like(o)
    dk = torch.empty((B, Hkv, N, D), device=dev, dtype=torch.float32)
    dv = torch.empty_like(dk)
    mask = None
    if causal:
        mask = torch.ones((N, N), device=dev, dtype=torch.bool).triu_(1)
    for b in range(B):
        for h in range(Hkv):
            hs = slice(h * G, (h + 1) * G)
            qh = q[b, hs].float()
            kh = k[b, h].float()
            vh = v[b, h].float()
            doh = do[b, hs].float()
            s = torch.matmul(qh, kh.t().contiguous()) * scale  # [G, N, N]
            if mask is not None:
                s.masked_fill_(mask, -math.inf)
            lse = torch.logsumexp(s, dim=-1)
            p = torch.exp(s - lse[..., None])
            del s
            oh = torch.matmul(p, vh)
            o[b, hs] = oh
            lse2[b, hs] = lse * (1.0 / math.log(2.0))
            ostored = o16[b, hs].float() if o16 is not None else oh.half().float()
            delta = (ostored * doh).sum(-1)
            dp = torch.matmul(doh, vh.t().contiguous())
            ds = p * (dp - delta[..., None])
            del dp
            dq[b, hs] = torch.matmul(ds, kh) * scale
            dk[b, h] = torch.matmul(ds.transpose(1, 2).contiguous(), qh).sum(0) * scale
            dv[b, h] = torch.matmul(p.transpose(1, 2).contiguous(), doh).sum(0)
            del p, ds
    return {"o": o, "lse": lse2, "dq": dq, "dk": dk, "dv": dv}
