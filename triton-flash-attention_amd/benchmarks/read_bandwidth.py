"""Decoding forward against a plain streaming read of the same K/V bytes.

The decoding forward (a few queries against a long key sequence) is bound by
reading K and V. This measures, on one GPU and in one process, the library's
forward (the op layer's ``flash_fwd``: split-KV launch plus merge) and
``read_kernel`` (read_bandwidth.hip: 16-byte loads in a grid-stride loop, the
fastest of a sweep of grid sizes and loads in flight) over the same K/V
buffer, in three cache states before each repetition:

* ``warm``: nothing in between; K/V stay in L2 / the 256 MB MALL where they fit.
* ``cold-dirty``: 512 MiB written first (the benchmark harness's protocol,
  benchmark_attention.py ``bench_gpu``). K/V come from HBM, and the dirty
  lines the write left in the MALL are written back while the kernel runs.
* ``cold-clean``: 512 MiB read first (``read_kernel``): K/V come from HBM and
  nothing is left to write back.

Every repetition starts behind a ``spin_kernel`` of ~200 µs, so the host has
queued the HIP events and the launches before the GPU reaches them: the event
pair times GPU work only. Median of ``--reps``.

Run from ``triton-flash-attention_amd/`` on a GPU box:

    python -m benchmarks.read_bandwidth            # the five decoding shapes
    python -m benchmarks.read_bandwidth --shapes f1 --reps 30
"""

from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import subprocess
import sys
import tempfile
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

# The forward shapes of the decoding harness runs: B, Hq, Hkv, N_q, N_kv, D.
SHAPES = {
    "f1": (1, 32, 8, 1, 32768, 128),
    "f2": (8, 32, 8, 1, 8192, 128),
    "f3": (32, 32, 8, 1, 2048, 128),
    "f4": (8, 32, 8, 16, 8192, 128),
    "f5": (4, 16, 16, 1, 16384, 64),
}
READ_CONFIGS = [(blocks, unr) for blocks in (1024, 2048, 4096, 8192) for unr in (1, 4, 8)]
FLUSH_BYTES = 512 << 20
SPIN_US = 200
WALL_CLOCK_MHZ = 100  # MI300-series constant wall clock (hipDeviceAttributeWallClockRate)


def build(out_dir: Path) -> ctypes.CDLL:
    so = out_dir / "libread_bandwidth.so"
    subprocess.run(["hipcc", "--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", "-shared", "-fPIC", "-o", str(so),
                    str(HERE / "read_bandwidth.hip")], check=True, capture_output=True)
    lib = ctypes.CDLL(str(so))
    lib.launch_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                ctypes.c_int, ctypes.c_void_p]
    lib.launch_spin.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    return lib


class Bench:
    def __init__(self, lib: ctypes.CDLL, device: torch.device):
        self.lib = lib
        self.flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=device)
        self.flush_out = torch.empty(8192 * 256, dtype=torch.int32, device=device)
        self.spin_out = torch.empty(1, dtype=torch.int32, device=device)

    @staticmethod
    def stream() -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def read(self, buf: torch.Tensor, nbytes: int, out: torch.Tensor, blocks: int, unr: int):
        rc = self.lib.launch_read(buf.data_ptr(), nbytes, out.data_ptr(), blocks, unr, self.stream())
        if rc != 0:
            raise RuntimeError(f"read_kernel launch failed: hipError {rc}")

    def before(self, mode: str, rep: int):
        self.lib.launch_spin(SPIN_US * WALL_CLOCK_MHZ, self.spin_out.data_ptr(), self.stream())
        if mode == "cold-dirty":
            self.flush.fill_(rep & 0xFF)
        elif mode == "cold-clean":
            self.read(self.flush, FLUSH_BYTES, self.flush_out, 4096, 4)

    def time(self, fn, mode: str, reps: int) -> float:
        """Median µs of fn over reps (after two untimed ones), GPU time only."""
        pairs = []
        for r in range(reps + 2):
            self.before(mode, r)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            pairs.append((a, b))
        torch.cuda.synchronize()
        return statistics.median(a.elapsed_time(b) * 1e3 for a, b in pairs[2:])


def run_shape(bench: Bench, name: str, reps: int) -> dict:
    from triton_flash_attention import _ops

    B, Hq, Hkv, Nq, Nkv, D = SHAPES[name]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    # K and V in one buffer, so one read_kernel launch covers exactly their bytes.
    kv = torch.randn(2, B, Hkv, Nkv, D, device=dev, dtype=torch.float16, generator=g)
    k, v = kv[0], kv[1]
    q = torch.randn(B, Hq, Nq, D, device=dev, dtype=torch.float16, generator=g)
    kv_bytes = kv.numel() * 2
    scale = D ** -0.5
    row = {"shape": name, "B": B, "Hq": Hq, "Hkv": Hkv, "N_q": Nq, "N_kv": Nkv, "D": D,
           "kv_MB": round(kv_bytes / 1e6, 1)}
    for mode in ("warm", "cold-dirty", "cold-clean"):
        t_fwd = bench.time(lambda: _ops.flash_fwd(q, k, v, False, scale), mode, reps)
        best = None
        for blocks, unr in READ_CONFIGS:
            out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
            t = bench.time(lambda: bench.read(kv, kv_bytes, out, blocks, unr), mode, reps)
            if best is None or t < best[0]:
                best = (t, blocks, unr)
        row[mode] = {"fwd_us": round(t_fwd, 1), "fwd_TBs": round(kv_bytes / t_fwd / 1e6, 2),
                     "read_us": round(best[0], 1), "read_TBs": round(kv_bytes / best[0] / 1e6, 2),
                     "read_blocks_unr": list(best[1:]),
                     "fwd_of_read": round(best[0] / t_fwd, 3)}
    return row


def render(rows: list[dict]) -> str:
    out = ["| shape | B | Hq | Hkv | N_q | N_kv | D | K/V MB | cache state | read µs (TB/s) | "
           "forward µs (TB/s) | forward / read rate |",
           "|---|---:|---:|---:|---:|---:|---:|---:|---|---:|---:|---:|"]
    for r in rows:
        for mode in ("warm", "cold-dirty", "cold-clean"):
            m = r[mode]
            out.append(f"| {r['shape']} | {r['B']} | {r['Hq']} | {r['Hkv']} | {r['N_q']} | "
                       f"{r['N_kv']} | {r['D']} | {r['kv_MB']} | {mode} | "
                       f"{m['read_us']} ({m['read_TBs']}) | {m['fwd_us']} ({m['fwd_TBs']}) | "
                       f"{m['fwd_of_read']:.2f} |")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shapes", nargs="+", default=list(SHAPES), choices=list(SHAPES))
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--json", type=Path, default=None, help="also write the rows here")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("read_bandwidth needs a GPU")
    with tempfile.TemporaryDirectory() as tmp:
        bench = Bench(build(Path(tmp)), torch.device("cuda:0"))
        rows = []
        for name in args.shapes:
            rows.append(run_shape(bench, name, args.reps))
            print(json.dumps(rows[-1]), flush=True)
    print(render(rows))
    if args.json:
        args.json.write_text(json.dumps(rows, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
