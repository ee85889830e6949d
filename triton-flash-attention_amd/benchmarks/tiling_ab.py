"""Interleaved A/B of two or more tilings of one kernel at a list of shapes.

Differences of a few percent between tilings are smaller than the spread
between boxes and between runs on one box (the clock follows the chip's power
limit), so the sweep's one-after-the-other timings (``tiling_sweep``) cannot
rank them. This runs the named tilings in alternation: each round times every
tiling once (``reps`` back-to-back launches between HIP events, after three
untimed ones), and each tiling's result is the median over ``rounds`` rounds.
Output: one JSON line per shape with the medians (µs) and each tiling's ratio
to the first one named; with ``--markdown`` also a table.

    python -m benchmarks.tiling_ab --kernel fwd --variants 6,10 \\
        --shape 4,16,16,4096,32,causal --shape 8,16,16,2048,32,causal,bfloat16

A shape is ``B,Hq,Hkv,N,D,mask[,dtype[,N_kv]]`` with mask ``causal`` or
``noncausal``, dtype ``float16`` (default) or ``bfloat16``, and N_kv keys
(default N; decoding shapes have few queries against many keys). A tiling with no
build for the shape's head size or dtype runs the table's tiling
(``fa_set_tiling``), so name compiled ones (``tiling_sweep`` lists them). ``auto``
names the library's own choice (the table and its shape rules, as with no tiling
set). The table is restored afterwards, also after an error.
"""

from __future__ import annotations

import argparse
import json
import statistics
from typing import Any

import torch

from triton_flash_attention import _lib, _ops

KERNELS = {"fwd": _lib.KERNEL_FWD, "dkdv": _lib.KERNEL_DKDV, "dq": _lib.KERNEL_DQ}


def parse_shape(text: str) -> dict[str, Any]:
    parts = [p.strip() for p in text.split(",")]
    if len(parts) not in (6, 7, 8):
        raise ValueError(f"shape {text!r}: expected B,Hq,Hkv,N,D,mask[,dtype[,N_kv]]")
    B, Hq, Hkv, N, D = (int(p) for p in parts[:5])
    mask = parts[5]
    dtype = parts[6] if len(parts) >= 7 else "float16"
    Nkv = int(parts[7]) if len(parts) == 8 else N
    if mask not in ("causal", "noncausal"):
        raise ValueError(f"shape {text!r}: mask must be causal or noncausal")
    if dtype not in ("float16", "bfloat16"):
        raise ValueError(f"shape {text!r}: dtype must be float16 or bfloat16")
    if min(B, Hq, Hkv, N, Nkv) <= 0 or Hq % Hkv or D not in (32, 64, 128):
        raise ValueError(f"shape {text!r}: positive sizes, Hq a multiple of Hkv, D in 32/64/128")
    return {"B": B, "Hq": Hq, "Hkv": Hkv, "N": N, "Nkv": Nkv, "D": D, "causal": mask == "causal",
            "dtype": dtype}


def label(variant: int) -> str:
    return "auto" if variant < 0 else str(variant)


def parse_variants(text: str) -> list[int]:
    """Comma-separated tiling indices; ``auto`` (-1) is the library's own choice."""
    out = []
    for x in (t.strip() for t in text.split(",")):
        if not x:
            continue
        v = -1 if x == "auto" else int(x)
        if v < -1:
            raise ValueError(f"tiling {x!r}: an index >= 0 or auto")
        out.append(v)
    return out


def ab(kernel: str, variants: list[int], shape: dict[str, Any], rounds: int = 7,
       reps: int = 20, seed: int = 1) -> dict[str, Any]:
    """Medians (µs) of each tiling over interleaved rounds, and ratios to the first.

    A variant of -1 runs with no tiling set: the library's table and shape rules."""
    B, Hq, Hkv, N, D, causal = (shape[k] for k in ("B", "Hq", "Hkv", "N", "D", "causal"))
    Nkv = shape.get("Nkv", N)
    dtype = getattr(torch, shape["dtype"])
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)
    q, do = (torch.randn(B, Hq, N, D, device=dev, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, Hkv, Nkv, D, device=dev, generator=g).to(dtype) for _ in range(2))
    scale = D ** -0.5
    o, lse = _ops.flash_fwd(q, k, v, causal, scale)
    delta = _ops.flash_bwd_preprocess(o, do)
    run = {
        "fwd": lambda: _ops.flash_fwd(q, k, v, causal, scale),
        "dkdv": lambda: _ops.flash_bwd_dkdv(q, k, v, do, lse, delta, causal, scale),
        "dq": lambda: _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, causal, scale),
    }[kernel]
    kind = KERNELS[kernel]
    times: dict[int, list[float]] = {var: [] for var in variants}
    try:
        for _ in range(rounds):
            for var in variants:
                _lib.set_tiling(kind, D, causal, var)
                for _ in range(3):
                    run()
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(reps):
                    run()
                end.record()
                torch.cuda.synchronize()
                times[var].append(start.elapsed_time(end) * 1e3 / reps)
    finally:
        _lib.set_tiling(kind, D, causal, -1)
    med = {var: statistics.median(t) for var, t in times.items()}
    first = variants[0]
    return {"kernel": kernel, **shape,
            "us": {label(var): round(m, 1) for var, m in med.items()},
            "ratio": {label(var): round(m / med[first], 3) for var, m in med.items()}}


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--kernel", choices=tuple(KERNELS), required=True)
    parser.add_argument("--variants", required=True,
                        help="comma-separated tiling indices (two or more); auto = the "
                             "library's own choice")
    parser.add_argument("--shape", action="append", required=True,
                        help="B,Hq,Hkv,N,D,mask[,dtype[,N_kv]]; repeat for more shapes")
    parser.add_argument("--rounds", type=int, default=7)
    parser.add_argument("--reps", type=int, default=20, help="launches per timing")
    parser.add_argument("--markdown", action="store_true", help="also print a table")
    args = parser.parse_args(argv)
    try:
        variants = parse_variants(args.variants)
        shapes = [parse_shape(s) for s in args.shape]
    except ValueError as e:
        raise SystemExit(str(e))
    if len(variants) < 2 or len(set(variants)) != len(variants):
        raise SystemExit("--variants needs two or more distinct tiling indices")
    if args.rounds <= 0 or args.reps <= 0:
        raise SystemExit("--rounds and --reps must be positive")
    if not torch.cuda.is_available():
        raise SystemExit("the tiling A/B needs a GPU")
    rows = []
    for shape in shapes:
        rows.append(ab(args.kernel, variants, shape, args.rounds, args.reps))
        print(json.dumps(rows[-1]), flush=True)
    if args.markdown:
        cols = " | ".join(f"tiling {label(v)} µs" for v in variants)
        print(f"| shape | {cols} | "
              + " | ".join(f"{label(v)} / {label(variants[0])}" for v in variants[1:]) + " |")
        print("|---|" + "---:|" * (2 * len(variants) - 1))
        for r in rows:
            kv = f" N_kv{r['Nkv']}" if r["Nkv"] != r["N"] else ""
            name = (f"B{r['B']} Hq{r['Hq']} Hkv{r['Hkv']} N{r['N']}{kv} D{r['D']} "
                    f"{'causal' if r['causal'] else 'bidirectional'} {r['dtype']}")
            us = " | ".join(str(r["us"][label(v)]) for v in variants)
            ratios = " | ".join(f"{r['ratio'][label(v)]:.3f}" for v in variants[1:])
            print(f"| {name} | {us} | {ratios} |")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
