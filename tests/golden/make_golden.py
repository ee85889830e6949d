"""Writes tests/golden/attention_fp64.npz: small golden vectors for the oracle.

The reference ships no golden vectors (its tests compare live against
torch.nn.functional.scaled_dot_product_attention). These fixtures are made
with PyTorch alone, in float64 on the CPU, independently of the oracle:
  o      = F.scaled_dot_product_attention(q, k, v, is_causal, enable_gqa) (fp64)
  lse2   = logsumexp of the scaled, masked scores / ln 2 (base-2 LSE, the
           quantity the reference stores at attention.py:230)
  o16    = o rounded to fp16 (the stored output)
  delta  = rowsum(o16 * dO)  (attention.py:252-254, O as stored in fp16)
  dq, dk, dv = the exact fp64 autograd of SDPA (its Delta is the unrounded
           rowsum(o * dO), so tests compare the oracle's backward fed with that
           exact Delta).
Inputs are drawn from seeded CPU generators in fp32 and cast to fp16 (the
values the kernels see). Shapes: the reference test shapes
(tests/test_cuda_correctness.py:87-101) plus head_dim 128, and the
CPU-fallback configuration of BASELINE.json.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "attention_fp64.npz"

# name: (B, Hq, Hkv, N, D, causal, input scale, dO scale, seed)
CASES = {}
for D, N, H in ((32, 17, 2), (32, 129, 2), (64, 17, 2), (64, 129, 1), (128, 17, 1), (128, 65, 1)):
    for causal in (False, True):
        CASES[f"mha_n{N}_d{D}_{'causal' if causal else 'bidir'}"] = (
            1, H, H, N, D, causal, 0.5, 0.1, 100 + D + N + int(causal))
CASES["gqa4to2_n65_d64_causal"] = (1, 4, 2, 65, 64, True, 0.5, 0.1, 123)
CASES["gqa4to1_n40_d32_bidir"] = (2, 4, 1, 40, 32, False, 1.0, 1.0, 77)
CASES["config1_b1_h4_n257_d64_bidir"] = (1, 4, 4, 257, 64, False, 1.0, 1.0, 1001)


def make_case(B, Hq, Hkv, N, D, causal, mult, do_mult, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    q = (torch.randn((B, Hq, N, D), generator=g) * mult).half()
    k = (torch.randn((B, Hkv, N, D), generator=g) * mult).half()
    v = (torch.randn((B, Hkv, N, D), generator=g) * mult).half()
    do = (torch.randn((B, Hq, N, D), generator=g) * do_mult).half()
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    gqa = Hq != Hkv
    o = torch.nn.functional.scaled_dot_product_attention(
        q64, k64, v64, is_causal=causal, enable_gqa=gqa)
    dq, dk, dv = torch.autograd.grad(o, (q64, k64, v64), do.double())
    with torch.no_grad():
        kr = k64.repeat_interleave(Hq // Hkv, dim=1)
        s = torch.matmul(q64, kr.transpose(-1, -2)) / math.sqrt(D)
        if causal:
            s = s.masked_fill(torch.ones(N, N, dtype=torch.bool).triu(1), -math.inf)
        lse2 = torch.logsumexp(s, dim=-1) / math.log(2.0)
        o16 = o.detach().half()
        delta = (o16.double() * do.double()).sum(-1)
    f32 = np.float32  # outputs stored in fp32: ~1e-7 relative, far below any plausible bug
    out = {
        "q": q.numpy(), "k": k.numpy(), "v": v.numpy(), "do": do.numpy(),
        "o": o.detach().numpy().astype(f32), "o16": o16.numpy(),
        "lse2": lse2.numpy(), "delta": delta.numpy(),
        "dq": dq.numpy().astype(f32), "dk": dk.numpy().astype(f32),
        "dv": dv.numpy().astype(f32),
        "meta": np.array([B, Hq, Hkv, N, D, int(causal)], dtype=np.int64),
    }
    return out


def main() -> None:
    arrays = {}
    for name, spec in CASES.items():
        for key, value in make_case(*spec).items():
            if name.startswith("config1") and key in ("do", "delta", "dq", "dk", "dv", "o16"):
                continue  # configuration 1 is forward-only
            arrays[f"{name}/{key}"] = value
    # Config-1 is the reference's CPU fallback itself: also record the fp16
    # CPU SDPA output of this torch build (torch-version dependent).
    B, Hq, Hkv, N, D, causal, mult, _, seed = CASES["config1_b1_h4_n257_d64_bidir"]
    q = torch.from_numpy(arrays["config1_b1_h4_n257_d64_bidir/q"])
    k = torch.from_numpy(arrays["config1_b1_h4_n257_d64_bidir/k"])
    v = torch.from_numpy(arrays["config1_b1_h4_n257_d64_bidir/v"])
    arrays["config1_b1_h4_n257_d64_bidir/o_cpu_fp16_sdpa"] = (
        torch.nn.functional.scaled_dot_product_attention(q, k, v).numpy())
    arrays["_torch_version"] = np.array(torch.__version__)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size / 1024:.0f} KiB, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
