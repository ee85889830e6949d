"""HBM bytes per launch from rocprofv3's FETCH_SIZE / WRITE_SIZE counters.

bench.py's ``roofline.traffic`` reads ``profiles/traffic.json``; this module
writes it from two counter passes per workload, each of the same bench.py
command with a calibration copy of known size in the same process:

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o c2 -- \\
        python3 bench.py --workload c2 --steps 3 --warmup 1 --cpu-seconds 0 \\
        --calibrate-copy-mib 256 --no-parity --no-reference-protocol
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o c2 -- (same)
    python -m benchmarks.traffic_summary OUT c2 c3 ... --json ../profiles/traffic.json

(run from ``triton-flash-attention_amd/``). The counters report KiB per
dispatch; each is scaled by what it reads for the copy
(``__amd_rocclr_copyBuffer``, which reads and writes the copy's size once),
and averaged over the dispatches of each kernel. The algorithmic bytes are
the tensors a launch must read and write once (fp16 [B, H, N, D] operands,
fp32 [B, Hq, N] LSE and Delta).
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

COPY_KERNEL = "__amd_rocclr_copyBuffer"
# The kernel of each bench.py kernel-pass entry (the launches of fa_bwd's
# default plan: forward, dQ with Delta, dK/dV; split plans add helper kernels;
# "pipe16" are the 16x16x32 MFMA forms).
KINDS = {"fwd": "fwd(_pipe)?_kernel", "dkdv": "dkdv(_pipe(16)?)?_kernel",
         "dq": "dq(_pipe(16)?)?_kernel"}


def per_kernel_kib(path: Path, counter: str) -> dict[str, list[float]]:
    out = defaultdict(list)
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] == counter:
                out[row["Kernel_Name"]].append(float(row["Counter_Value"]))
    return out


def algorithmic_bytes(kind: str, B: int, Hq: int, Hkv: int, N: int, D: int) -> int:
    q = B * Hq * N * D * 2
    kv = B * Hkv * N * D * 2
    vec = B * Hq * N * 4
    if kind == "fwd":  # Q, K, V -> O, LSE
        return q + 2 * kv + q + vec
    if kind == "dkdv":  # Q, K, V, dO, LSE, Delta -> dK, dV
        return q + 2 * kv + q + 2 * vec + 2 * kv
    return q + 2 * kv + 2 * q + vec + q + vec  # dQ: Q, K, V, O, dO, LSE -> dQ, Delta


def summarise(out_dir: Path, workload: str) -> dict:
    from bench import WORKLOADS

    B, Hq, Hkv, N, D = WORKLOADS[workload][:5]
    fetch = per_kernel_kib(out_dir / "fetch" / f"{workload}_counter_collection.csv", "FETCH_SIZE")
    write = per_kernel_kib(out_dir / "write" / f"{workload}_counter_collection.csv", "WRITE_SIZE")
    copy = 256 << 20
    f_copy = next(v for k, v in fetch.items() if COPY_KERNEL in k)
    w_copy = next(v for k, v in write.items() if COPY_KERNEL in k)
    f_factor = copy / (sum(f_copy) / len(f_copy) * 1024)
    w_factor = copy / (sum(w_copy) / len(w_copy) * 1024)
    result = {"_calibration": {"copy_bytes": copy, "fetch_factor": round(f_factor, 4),
                               "write_factor": round(w_factor, 4)}}
    for kind, stem in KINDS.items():
        names = [k for k in fetch if re.search(rf"fa::{stem}<", k)]
        if not names:
            continue
        name = max(names, key=lambda k: len(fetch[k]))
        fb = sum(fetch[name]) / len(fetch[name]) * 1024 * f_factor
        wb = sum(write[name]) / len(write[name]) * 1024 * w_factor
        result[kind] = {
            "hbm_bytes_per_launch": int(fb + wb), "fetch_bytes": int(fb), "write_bytes": int(wb),
            "algorithmic_bytes": algorithmic_bytes(kind, B, Hq, Hkv, N, D),
            "kernel": re.sub(r"^void fa::", "", name).split("(")[0],
        }
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("out_dir", type=Path)
    ap.add_argument("workloads", nargs="+")
    ap.add_argument("--json", type=Path, default=None, help="write the summary here")
    args = ap.parse_args(argv)
    data = {w: summarise(args.out_dir, w) for w in args.workloads}
    MiB = 1 << 20
    print("| workload | kernel | instance | fetch MiB | write MiB | HBM MiB / launch | "
          "algorithmic MiB | ratio |")
    print("|---|---|---|---:|---:|---:|---:|---:|")
    for w, d in data.items():
        for kind in KINDS:
            if kind in d:
                e = d[kind]
                print(f"| {w} | {kind} | `{e['kernel']}` | {e['fetch_bytes'] / MiB:.1f} | "
                      f"{e['write_bytes'] / MiB:.1f} | {e['hbm_bytes_per_launch'] / MiB:.1f} | "
                      f"{e['algorithmic_bytes'] / MiB:.1f} | "
                      f"{e['hbm_bytes_per_launch'] / e['algorithmic_bytes']:.2f} |")
    if args.json:
        args.json.write_text(json.dumps(data, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
