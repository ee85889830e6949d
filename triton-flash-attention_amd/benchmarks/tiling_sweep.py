"""Time every compiled tiling of the forward, dK/dV and dQ kernels at one shape.

The library's static tiling table (``kDefault`` in ``csrc/fa_capi.hip``) takes
the place of the reference's Triton autotuning, which searches tile sizes per
(N, D, causal) on first use (attention.py:82-90, 353-381). This sweep is the
search, run offline: for each kernel it selects each compiled tiling with
``fa_set_tiling``, times that kernel alone through the op layer with HIP events
on the current stream, and reports the fastest next to the table's choice. The
table is restored when it returns, also after an error. Inputs are fp16 unless
``--dtype bfloat16``; bfloat16 is compiled for some tilings only, and a bf16
launch whose set tiling has no bf16 build runs the table's tiling
(fa_set_tiling), so a bf16 sweep should name compiled ones with ``--variants``.

    python -m benchmarks.tiling_sweep --batch 4 --query-heads 16 --seq-len 4096 \\
        --head-dim 64 --mask causal
"""

from __future__ import annotations

import argparse
import csv
from pathlib import Path
from typing import Any

import torch

from triton_flash_attention import _lib, _ops

KERNELS = {"fwd": _lib.KERNEL_FWD, "dkdv": _lib.KERNEL_DKDV, "dq": _lib.KERNEL_DQ}

# Matmul-equivalents of 2*B*Hq*pairs*D FLOP each kernel executes: the forward
# computes S and P.V; dK/dV recomputes S and dP and forms dV and dK; dQ
# recomputes S and dP and forms dQ.
MATMULS = {"fwd": 2, "dkdv": 4, "dq": 3}


def executed_flops(kernel: str, *, batch: int, query_heads: int, seq_len: int, head_dim: int,
                   causal: bool) -> int:
    """FLOP the kernel executes (not the 3.5 x forward convention of the
    benchmark harness): causal launches count the N(N+1)/2 visible pairs."""
    pairs = seq_len * (seq_len + 1) // 2 if causal else seq_len * seq_len
    return MATMULS[kernel] * 2 * batch * query_heads * pairs * head_dim


def _time_us(fn, reps: int) -> float:
    """Median over three trials of the mean duration of ``reps`` back-to-back calls."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    trials = []
    for _ in range(3):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        trials.append(start.elapsed_time(end) * 1e3 / reps)
    return sorted(trials)[1]


def sweep(*, batch: int, query_heads: int, kv_heads: int, seq_len: int, head_dim: int,
          causal: bool, kernels: list[str], reps: int = 10, seed: int = 0,
          with_choice: bool = False, dtype: torch.dtype = torch.float16,
          variants: list[int] | None = None) -> list[dict[str, Any]]:
    """One row per (kernel, compiled tiling): waves, rows per work-group, tile,
    whether the table picks it, mean µs per launch and executed TFLOP/s. With
    ``with_choice`` each kernel also gets a row with variant ``"auto"``: no
    tiling set, so the library runs what it picks for this shape (the table
    refined by its shape rules). ``variants`` restricts the sweep to those
    tiling indices (all compiled ones by default)."""
    g = torch.Generator("cpu").manual_seed(seed)
    shapes = ((batch, query_heads, seq_len, head_dim), (batch, kv_heads, seq_len, head_dim),
              (batch, kv_heads, seq_len, head_dim), (batch, query_heads, seq_len, head_dim))
    q, k, v, do = (torch.randn(s, generator=g).to(dtype).cuda() for s in shapes)
    scale = head_dim ** -0.5
    o, lse = _ops.flash_fwd(q, k, v, causal, scale)
    delta = _ops.flash_bwd_preprocess(o, do)
    runners = {
        "fwd": lambda: _ops.flash_fwd(q, k, v, causal, scale),
        "dkdv": lambda: _ops.flash_bwd_dkdv(q, k, v, do, lse, delta, causal, scale),
        "dq": lambda: _ops.flash_bwd_dq_delta(q, k, v, o, do, lse, causal, scale),
    }
    rows = []
    for name in kernels:
        kind = KERNELS[name]
        table = _lib.get_tiling(kind, head_dim, causal)["variant"]
        flop = executed_flops(name, batch=batch, query_heads=query_heads, seq_len=seq_len,
                              head_dim=head_dim, causal=causal)
        try:
            for var in _lib.tiling_variants(kind, head_dim, causal):
                if variants is not None and var["variant"] not in variants:
                    continue
                _lib.set_tiling(kind, head_dim, causal, var["variant"])
                us = _time_us(runners[name], reps)
                rows.append({"kernel": name, "variant": var["variant"], "waves": var["waves"],
                             "rows": var["rows"], "tile": var["tile"],
                             "table": var["variant"] == table, "us": round(us, 1),
                             "tflops_executed": round(flop / us / 1e6, 1)})
        finally:
            _lib.set_tiling(kind, head_dim, causal, -1)
        if with_choice:
            us = _time_us(runners[name], reps)
            rows.append({"kernel": name, "variant": "auto", "waves": "", "rows": "", "tile": "",
                         "table": False, "us": round(us, 1),
                         "tflops_executed": round(flop / us / 1e6, 1)})
    return rows


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--batch", type=int, default=4)
    parser.add_argument("--query-heads", type=int, default=16)
    parser.add_argument("--kv-heads", type=int, default=None,
                        help="key/value heads (GQA); defaults to --query-heads")
    parser.add_argument("--seq-len", type=int, default=4096)
    parser.add_argument("--head-dim", type=int, choices=(32, 64, 128), default=64)
    parser.add_argument("--mask", choices=("causal", "noncausal"), default="causal")
    parser.add_argument("--kernels", default="fwd,dkdv,dq",
                        help="comma-separated subset of fwd,dkdv,dq")
    parser.add_argument("--reps", type=int, default=10, help="launches per timing trial")
    parser.add_argument("--dtype", choices=("float16", "bfloat16"), default="float16")
    parser.add_argument("--variants", default=None,
                        help="comma-separated tiling indices to time (default: every compiled one)")
    parser.add_argument("--output", type=Path, default=None, help="optional CSV file")
    return parser


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    kernels = [s.strip() for s in args.kernels.split(",") if s.strip()]
    unknown = [s for s in kernels if s not in KERNELS]
    if unknown or not kernels:
        raise SystemExit(f"unknown kernels {unknown}; choose from {list(KERNELS)}")
    kv_heads = args.kv_heads or args.query_heads
    if min(args.batch, args.query_heads, kv_heads, args.seq_len, args.reps) <= 0:
        raise SystemExit("sizes and --reps must be positive")
    if args.query_heads % kv_heads:
        raise SystemExit("--query-heads must be a multiple of --kv-heads")
    try:
        variants = ([int(x) for x in args.variants.split(",") if x.strip()]
                    if args.variants else None)
    except ValueError:
        raise SystemExit(f"--variants must be comma-separated integers, got {args.variants!r}")
    if not torch.cuda.is_available():
        raise SystemExit("the tiling sweep needs a GPU")
    rows = sweep(batch=args.batch, query_heads=args.query_heads, kv_heads=kv_heads,
                 seq_len=args.seq_len, head_dim=args.head_dim, causal=args.mask == "causal",
                 kernels=kernels, reps=args.reps, with_choice=True,
                 dtype=getattr(torch, args.dtype), variants=variants)
    print(f"B={args.batch} Hq={args.query_heads} Hkv={kv_heads} N={args.seq_len} "
          f"D={args.head_dim} {args.mask}" + (f" {args.dtype}" if args.dtype != "float16" else ""))
    print("| kernel | variant | waves | rows | tile | table | µs | TFLOP/s executed |")
    print("|---|---:|---:|---:|---:|:---:|---:|---:|")
    for r in rows:
        print(f"| {r['kernel']} | {r['variant']} | {r['waves']} | {r['rows']} | {r['tile']} | "
              f"{'*' if r['table'] else ''} | {r['us']:.1f} | {r['tflops_executed']:.1f} |")
    for name in kernels:
        mine = [r for r in rows if r["kernel"] == name and r["variant"] != "auto"]
        best = min(mine, key=lambda r: r["us"])
        table = next(r for r in mine if r["table"])
        auto = next(r for r in rows if r["kernel"] == name and r["variant"] == "auto")
        print(f"{name}: fastest variant {best['variant']} ({best['us']:.1f} µs), "
              f"table variant {table['variant']} ({table['us']:.1f} µs), "
              f"library's choice for this shape {auto['us']:.1f} µs")
    if args.output is not None:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        with args.output.open("w", newline="") as f:
            writer = csv.DictWriter(f, fieldnames=list(rows[0]))
            writer.writeheader()
            writer.writerows(rows)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
