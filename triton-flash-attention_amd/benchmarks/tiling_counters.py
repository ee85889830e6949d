"""Hardware counters for every compiled tiling: the counter side of the tiling table.

The static tiling table (``kDefault`` in ``csrc/fa_capi.hip``) replaces the
reference's Triton autotuner (attention.py:82-90, 353-381). ``tiling_sweep``
times every compiled tiling of each kernel; this module reads the counters of
the same sweep, recorded by rocprofv3, and reports per tiling the MFMA pipe's
busy fraction, VALU and LDS instructions per MFMA and LDS bank conflicts, so
each table entry can be read against its runners-up.

Record (from ``triton-flash-attention_amd/``; one rocprofv3 pass per shape,
8 SQ counters and one GRBM counter, the most one pass can hold):

    rocprofv3 --pmc SQ_WAVES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS \\
        SQ_VALU_MFMA_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_LDS \\
        SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE --output-format csv -d OUT -o c2 -- \\
        python3 -m benchmarks.tiling_sweep --batch 4 --query-heads 16 \\
        --seq-len 4096 --head-dim 64 --mask causal --reps 1

Summarise (no GPU needed):

    python -m benchmarks.tiling_counters OUT/c2_counter_collection.csv \\
        --head-dim 64 --mask causal --title "c2: ..."

Derived quantities, per dispatch and then averaged over the dispatches of one
kernel symbol:
  cycles     = GRBM_GUI_ACTIVE / XCDs (the counter sums the XCDs' GRBMs)
  MFMA busy  = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs * cycles)
  clock      = cycles / (End_Timestamp - Start_Timestamp)
  VALU/MFMA  = SQ_INSTS_VALU / SQ_INSTS_MFMA (SQ_INSTS_VALU counts the MFMAs too)
  LDS/MFMA   = SQ_INSTS_LDS / SQ_INSTS_MFMA
  conflicts  = SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS (cycles stalled on bank
               conflicts per cycle of LDS instruction activity)
  wait       = SQ_WAIT_INST_ANY / SQ_WAVES (cycles each wave waited on any
               dependency, per wave)
Durations under counter collection are serialised dispatches with the counters
armed; they rank tilings but are a few percent above the sweep's own timings.
"""

from __future__ import annotations

import argparse
import csv
import re
import sys
from collections import defaultdict
from pathlib import Path

# MI355X: 8 XCDs x 32 CUs x 4 SIMDs.
XCDS = 8
SIMDS = 1024

KIND_OF = {
    "fwd_kernel": "fwd", "fwd_pipe_kernel": "fwd", "fwd_pipe_jobs_kernel": "fwd",
    "fwd_pipe16_kernel": "fwd",
    "dkdv_kernel": "dkdv", "dkdv_pipe_kernel": "dkdv", "dkdv_pipe16_kernel": "dkdv",
    "dq_kernel": "dq", "dq_pipe_kernel": "dq", "dq_pipe16_kernel": "dq",
}
# Classic tilings (waves, streamed tile) -> variant index, as registered in
# fa_fwd.hip (kFwdVariants) and fa_bwd.hip (kDkdvVariants, kDqVariants).
CLASSIC = {
    "fwd": {(4, 64): 0, (8, 64): 1, (4, 32): 2, (2, 64): 3, (4, 128): 4},
    "dkdv": {(4, 64): 0, (4, 32): 1, (2, 64): 2, (8, 64): 3},
    "dq": {(4, 64): 0, (4, 32): 1, (2, 64): 2, (8, 64): 3},
}


def parse_symbol(name: str):
    """(kernel kind, variant index, template arguments) of a demangled kernel
    name, or (None, None, args) for a helper kernel (Delta pass, split sums,
    split-KV combine)."""
    m = re.search(r"fa::(\w+)<([^>]*)>", name)
    if not m:
        return None, None, ()
    base, args = m.group(1), tuple(a.strip() for a in m.group(2).split(","))
    kind = KIND_OF.get(base)
    if kind is None:
        return None, None, (base,) + args
    ints = [int(a) for a in args if re.fullmatch(r"-?\d+", a)]
    if base == "fwd_pipe_jobs_kernel":
        return kind, 9, args
    if base == "fwd_pipe16_kernel":  # 16x16x32 MFMA form of tiling 6: <D, causal, E, QB>
        return kind, (11 if ints and ints[-1] == 1 else 10), args
    if base == "fwd_pipe_kernel":
        # <D, causal, NW, UPS, E, KG>
        nw, ups, kg = ints[1], ints[2], ints[3] if len(ints) > 3 else 1
        if kg == 2:
            return kind, 8, args
        if ups == 2:
            return kind, 5, args
        return kind, (7 if nw == 8 else 6), args
    if base in ("dkdv_pipe_kernel", "dq_pipe_kernel"):
        return kind, 4, args
    if base in ("dkdv_pipe16_kernel", "dq_pipe16_kernel"):  # 16x16x32 MFMA form
        return kind, 5, args
    # classic: <D, causal, NW, TILE, E>
    return kind, CLASSIC[kind].get((ints[1], ints[2])), args


def read_dispatches(paths):
    """Dispatch id -> {'name', 'dur_ns', counter: value} over rocprofv3
    counter_collection.csv files (one row per counter per dispatch)."""
    out = {}
    for fi, path in enumerate(paths):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                key = (fi, int(row["Dispatch_Id"]))
                d = out.setdefault(key, {"name": row["Kernel_Name"],
                                         "dur_ns": int(row["End_Timestamp"]) -
                                         int(row["Start_Timestamp"])})
                d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(
                    row["Counter_Value"])
    return out


def summarise(dispatches):
    """Kernel symbol -> averaged derived quantities."""
    groups = defaultdict(list)
    for d in dispatches.values():
        groups[d["name"]].append(d)
    rows = []
    for name, ds in groups.items():
        def mean(f):
            vals = [f(d) for d in ds]
            vals = [v for v in vals if v is not None]
            return sum(vals) / len(vals) if vals else None

        def ratio(a, b):
            return lambda d: d[a] / d[b] if d.get(a) is not None and d.get(b) else None

        def cycles(d):
            return d["GRBM_GUI_ACTIVE"] / XCDS if d.get("GRBM_GUI_ACTIVE") else None

        kind, variant, args = parse_symbol(name)
        rows.append({
            "name": name, "kind": kind, "variant": variant, "args": args,
            "dispatches": len(ds),
            "us": mean(lambda d: d["dur_ns"] / 1e3),
            "mfma_busy": mean(lambda d: d["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMDS * cycles(d))
                              if cycles(d) and "SQ_VALU_MFMA_BUSY_CYCLES" in d else None),
            "clock_ghz": mean(lambda d: cycles(d) / d["dur_ns"] if cycles(d) and d["dur_ns"]
                              else None),
            "valu_per_mfma": mean(ratio("SQ_INSTS_VALU", "SQ_INSTS_MFMA")),
            "lds_per_mfma": mean(ratio("SQ_INSTS_LDS", "SQ_INSTS_MFMA")),
            "conflict": mean(ratio("SQ_LDS_BANK_CONFLICT", "SQ_ACTIVE_INST_LDS")),
            "wait_per_wave": mean(ratio("SQ_WAIT_INST_ANY", "SQ_WAVES")),
        })
    order = {"fwd": 0, "dkdv": 1, "dq": 2, None: 3}
    rows.sort(key=lambda r: (order[r["kind"]], -1 if r["variant"] is None else r["variant"],
                             r["name"]))
    return rows


def table_variants(head_dim: int, causal: bool):
    """The table's variant per kernel kind for (head_dim, causal), from the
    library (fa_get_tiling; no GPU involved), or {} if it does not load."""
    try:
        from triton_flash_attention import _lib

        if not _lib.available()[0]:
            return {}
        return {kind: _lib.get_tiling(k, head_dim, causal)["variant"]
                for kind, k in (("fwd", _lib.KERNEL_FWD), ("dkdv", _lib.KERNEL_DKDV),
                                ("dq", _lib.KERNEL_DQ))}
    except Exception:  # noqa: BLE001 - the marker column is optional
        return {}


def fmt(v, spec, scale=1.0, suffix=""):
    return "—" if v is None else format(v * scale, spec) + suffix


def render(rows, title: str, defaults) -> str:
    lines = [f"## {title}", "",
             "| kernel | variant | table | symbol | dispatches | µs | MFMA busy | clock GHz | "
             "VALU/MFMA | LDS/MFMA | bank-conflict cycles / LDS cycles | wait cycles / wave |",
             "|---|---:|:---:|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        sym = re.sub(r"^void fa::", "", r["name"]).split("(")[0]
        m = re.match(r"_ZN2fa(\d+)", sym)  # helpers arrive mangled: keep the bare name
        if m:
            sym = sym[m.end():m.end() + int(m.group(1))]
        mark = "*" if r["kind"] and defaults.get(r["kind"]) == r["variant"] else ""
        lines.append(
            f"| {r['kind'] or 'helper'} | {'' if r['variant'] is None else r['variant']} | "
            f"{mark} | `{sym}` | {r['dispatches']} | {fmt(r['us'], '.1f')} | "
            f"{fmt(r['mfma_busy'], '.1f', 100, '%')} | {fmt(r['clock_ghz'], '.2f')} | "
            f"{fmt(r['valu_per_mfma'], '.2f')} | {fmt(r['lds_per_mfma'], '.2f')} | "
            f"{fmt(r['conflict'], '.4f')} | {fmt(r['wait_per_wave'], '.0f')} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("csv", nargs="+", type=Path, help="rocprofv3 counter_collection.csv files")
    ap.add_argument("--head-dim", type=int, choices=(32, 64, 128), required=True)
    ap.add_argument("--mask", choices=("causal", "noncausal"), required=True)
    ap.add_argument("--title", default=None)
    args = ap.parse_args(argv)
    rows = summarise(read_dispatches(args.csv))
    title = args.title or f"D={args.head_dim} {args.mask}"
    sys.stdout.write(render(rows, title, table_variants(args.head_dim, args.mask == "causal")))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
