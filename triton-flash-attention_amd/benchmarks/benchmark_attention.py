"""Benchmark the custom gfx950 kernels against PyTorch SDPA over a shape sweep.

Same FLOP model, memory model, runner semantics, CLI flags and CSV/metadata
columns as the reference harness (benchmarks/benchmark_attention.py); timing
uses HIP events on the current stream with an L2/MALL flush between
repetitions instead of ``triton.testing.do_bench``.

    python -m benchmarks.benchmark_attention --sequence-lengths 512,1024,2048,4096 \\
        --head-dims 64,128 --batch 4 --query-heads 16 --mode forward-backward --mask causal
"""

from __future__ import annotations

import argparse
import csv
import json
import platform
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import torch

from triton_flash_attention import scaled_dot_product_attention

# MI355X fp16 dense MFMA peak: 256 CUs x 2.4 GHz x 4096 FLOP/clk/CU.
MI355X_FP16_PEAK_TFLOPS = 2516.6


def _positive_int(value: str) -> int:
    parsed = int(value)
    if parsed <= 0:
        raise argparse.ArgumentTypeError("value must be greater than zero")
    return parsed


def _int_list(value: str) -> list[int]:
    try:
        values = [_positive_int(item.strip()) for item in value.split(",")]
    except ValueError as exc:
        raise argparse.ArgumentTypeError("expected comma-separated integers") from exc
    if not values:
        raise argparse.ArgumentTypeError("list cannot be empty")
    return values


def attention_flops(
    *,
    batch: int,
    query_heads: int,
    sequence: int,
    head_dim: int,
    causal: bool,
    mode: str,
    kv_sequence: int | None = None,
) -> int:
    """Algorithmic FLOPs (reference convention, benchmark_attention.py:36-54):
    forward = 4 * B * Hq * pairs * D with pairs = N(N+1)/2 causal, N^2
    otherwise; backward = 2.5x forward; forward-backward = 3.5x forward.
    With ``kv_sequence`` (cross-attention, an extension) pairs = N_q * N_kv,
    or under the causal mask the top-left visible pairs sum_i min(i+1, N_kv)."""
    pairs = _visible_pairs(sequence, sequence if kv_sequence is None else kv_sequence, causal)
    forward = 4 * batch * query_heads * pairs * head_dim
    if mode == "forward":
        return forward
    if mode == "backward":
        return int(2.5 * forward)
    if mode == "forward-backward":
        return int(3.5 * forward)
    raise ValueError(f"unknown mode: {mode}")


def _visible_pairs(n_q: int, n_kv: int, causal: bool) -> int:
    """(query, key) pairs a query sequence of n_q attends over n_kv keys;
    causal: query i sees keys j <= i (SDPA's top-left mask)."""
    if not causal:
        return n_q * n_kv
    full = min(n_q, n_kv)
    return full * (full + 1) // 2 + (n_q - full) * n_kv


def memory_model(
    *,
    batch: int,
    query_heads: int,
    sequence: int,
    element_size: int = 2,
    kv_sequence: int | None = None,
) -> dict[str, float]:
    """One materialized score matrix versus the saved fp32 LSE vector, MiB
    (``kv_sequence``: the key length of cross-attention, an extension)."""
    mib = float(1 << 20)
    n_kv = sequence if kv_sequence is None else kv_sequence
    return {
        "naive_score_mib": batch * query_heads * sequence * n_kv * element_size / mib,
        "saved_lse_mib": batch * query_heads * sequence * 4 / mib,
    }


def make_runner(
    *,
    provider: str,
    mode: str,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    grad_output: torch.Tensor,
    causal: bool,
    enable_gqa: bool,
):
    """A closure running one forward, backward or forward+backward of the
    public API (reference _make_runner, benchmark_attention.py:74-113)."""
    backend = "triton" if provider == "triton" else "torch"

    def attention():
        return scaled_dot_product_attention(
            query, key, value, is_causal=causal, enable_gqa=enable_gqa, backend=backend
        )

    if mode == "forward":
        return attention

    if mode == "backward":
        output = attention()

        def backward():
            query.grad = key.grad = value.grad = None
            output.backward(grad_output, retain_graph=True)

        return backward

    def forward_backward():
        query.grad = key.grad = value.grad = None
        attention().backward(grad_output)

    return forward_backward


def bench_gpu(fn, *, warmup_ms: float = 100.0, rep_ms: float = 300.0,
              quantiles=(0.5, 0.2, 0.8), flush_bytes: int = 512 << 20) -> list[float]:
    """Quantiles (ms) of ``fn``'s duration. Each repetition is bracketed by HIP
    events on the current stream and preceded by a write of ``flush_bytes``
    (larger than the 256 MiB MALL) so no repetition starts with a warm cache."""
    flush = torch.empty(flush_bytes // 4, dtype=torch.int32, device="cuda")
    fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(5):
        flush.zero_()
        fn()
    end.record()
    torch.cuda.synchronize()
    estimate = max(start.elapsed_time(end) / 5, 1e-3)
    n_warmup = max(1, int(warmup_ms / estimate))
    n_rep = max(5, int(rep_ms / estimate))
    for _ in range(n_warmup):
        fn()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    for i in range(n_rep):
        flush.zero_()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    times = torch.tensor([s.elapsed_time(e) for s, e in zip(starts, ends)], dtype=torch.float64)
    return [float(torch.quantile(times, q)) for q in quantiles]


def benchmark_case(
    *,
    provider: str,
    mode: str,
    batch: int,
    query_heads: int,
    kv_heads: int,
    sequence: int,
    head_dim: int,
    causal: bool,
    warmup_ms: int,
    rep_ms: int,
    kv_sequence: int | None = None,
) -> dict[str, Any]:
    requires_grad = mode != "forward"
    shape_q = (batch, query_heads, sequence, head_dim)
    shape_kv = (batch, kv_heads, sequence if kv_sequence is None else kv_sequence, head_dim)
    kw = dict(device="cuda", dtype=torch.float16, requires_grad=requires_grad)
    query = torch.randn(shape_q, **kw)
    key = torch.randn(shape_kv, **kw)
    value = torch.randn(shape_kv, **kw)
    grad_output = torch.randn_like(query)
    runner = make_runner(
        provider=provider, mode=mode, query=query, key=key, value=value,
        grad_output=grad_output, causal=causal, enable_gqa=query_heads != kv_heads,
    )
    median, low, high = bench_gpu(runner, warmup_ms=warmup_ms, rep_ms=rep_ms)
    flops = attention_flops(batch=batch, query_heads=query_heads, sequence=sequence,
                            head_dim=head_dim, causal=causal, mode=mode, kv_sequence=kv_sequence)
    memory = memory_model(batch=batch, query_heads=query_heads, sequence=sequence,
                          kv_sequence=kv_sequence)
    tflops = flops / (median * 1e-3) / 1e12
    cross = {} if kv_sequence is None else {"kv_sequence": kv_sequence}
    return {
        "provider": provider,
        "mode": mode,
        "causal": causal,
        "batch": batch,
        "query_heads": query_heads,
        "kv_heads": kv_heads,
        "sequence": sequence,
        **cross,
        "head_dim": head_dim,
        "median_ms": round(median, 5),
        "p20_ms": round(low, 5),
        "p80_ms": round(high, 5),
        "tflops": round(tflops, 3),
        "pct_of_peak": round(100.0 * tflops / MI355X_FP16_PEAK_TFLOPS, 2),
        **{name: round(value, 3) for name, value in memory.items()},
    }


def metadata() -> dict[str, Any]:
    props = torch.cuda.get_device_properties(0)
    return {
        "timestamp_utc": datetime.now(timezone.utc).isoformat(),
        "gpu": torch.cuda.get_device_name(),
        "arch": getattr(props, "gcnArchName", ""),
        "compute_units": props.multi_processor_count,
        "torch": torch.__version__,
        "hip_runtime": torch.version.hip,
        "python": platform.python_version(),
    }


def write_results(rows: list[dict[str, Any]], meta: dict[str, Any], output: Path) -> None:
    output.parent.mkdir(parents=True, exist_ok=True)
    with output.open("w", newline="", encoding="utf-8") as handle:
        writer = csv.DictWriter(handle, fieldnames=list(rows[0]), lineterminator="\n")
        writer.writeheader()
        writer.writerows(rows)
    output.with_suffix(".metadata.json").write_text(
        json.dumps(meta, indent=2) + "\n", encoding="utf-8"
    )


def print_rows(rows: list[dict[str, Any]]) -> None:
    columns = ("provider", "mode", "causal", "sequence", "head_dim", "median_ms", "tflops",
               "pct_of_peak")
    print("  ".join(f"{column:>12}" for column in columns))
    for row in rows:
        print("  ".join(f"{str(row[column]):>12}" for column in columns))


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--sequence-lengths", type=_int_list, default=[512, 1024, 2048, 4096],
                        help="comma-separated sequence lengths")
    parser.add_argument("--head-dims", type=_int_list, default=[64, 128],
                        help="comma-separated head dimensions")
    parser.add_argument("--batch", type=_positive_int, default=4)
    parser.add_argument("--query-heads", type=_positive_int, default=16)
    parser.add_argument("--kv-heads", type=_positive_int, default=None,
                        help="set below query-heads to benchmark GQA")
    parser.add_argument("--kv-sequence-length", type=_positive_int, default=None,
                        help="key/value length for cross-attention (an extension; the "
                             "default is each query sequence length)")
    parser.add_argument("--mode", choices=("forward", "backward", "forward-backward"),
                        default="forward-backward")
    parser.add_argument("--mask", choices=("causal", "noncausal", "both"), default="causal")
    parser.add_argument("--providers", default="torch,triton",
                        help="comma-separated subset of torch,triton")
    parser.add_argument("--warmup-ms", type=_positive_int, default=100)
    parser.add_argument("--rep-ms", type=_positive_int, default=300)
    parser.add_argument("--output", type=Path, default=Path("benchmarks/results/latest.csv"))
    return parser


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("a GPU is required to run the benchmark")
    kv_heads = args.kv_heads or args.query_heads
    if args.query_heads % kv_heads:
        raise SystemExit("--query-heads must be divisible by --kv-heads")
    unsupported = set(args.head_dims) - {32, 64, 128}
    if unsupported:
        raise SystemExit("the custom gfx950 path supports head dimensions 32, 64, and 128")
    providers = [p.strip() for p in args.providers.split(",") if p.strip()]
    if not providers or set(providers) - {"torch", "triton"}:
        raise SystemExit("--providers must be a subset of torch,triton")
    causal_values = {"causal": [True], "noncausal": [False], "both": [False, True]}[args.mask]
    rows = []
    for causal in causal_values:
        for head_dim in args.head_dims:
            for sequence in args.sequence_lengths:
                for provider in providers:
                    print(f"benchmarking {provider}: N={sequence}, D={head_dim}, causal={causal}",
                          flush=True)
                    rows.append(benchmark_case(
                        provider=provider, mode=args.mode, batch=args.batch,
                        query_heads=args.query_heads, kv_heads=kv_heads, sequence=sequence,
                        head_dim=head_dim, causal=causal, warmup_ms=args.warmup_ms,
                        rep_ms=args.rep_ms, kv_sequence=args.kv_sequence_length,
                    ))
    meta = metadata()
    write_results(rows, meta, args.output)
    print(json.dumps(meta, indent=2))
    print_rows(rows)
    print(f"wrote {args.output} and {args.output.with_suffix('.metadata.json')}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
