"""Known answers for the FLOP and memory model (reference
tests/test_benchmark_model.py:4-42) and the BASELINE configuration counts."""

from __future__ import annotations

import importlib.util
from pathlib import Path

from benchmarks.benchmark_attention import attention_flops, memory_model

ROOT = Path(__file__).resolve().parent.parent


def test_causal_forward_counts_only_visible_pairs() -> None:
    assert attention_flops(batch=1, query_heads=1, sequence=4, head_dim=8, causal=True,
                           mode="forward") == 4 * 10 * 8


def test_backward_is_two_and_a_half_forward_passes() -> None:
    kw = dict(batch=2, query_heads=4, sequence=16, head_dim=32, causal=False)
    assert attention_flops(mode="backward", **kw) == int(2.5 * attention_flops(mode="forward", **kw))


def test_memory_model_is_linear_for_saved_lse() -> None:
    small = memory_model(batch=1, query_heads=1, sequence=128)
    large = memory_model(batch=1, query_heads=1, sequence=256)
    assert large["saved_lse_mib"] == 2 * small["saved_lse_mib"]
    assert large["naive_score_mib"] == 4 * small["naive_score_mib"]


def test_baseline_configuration_flop_counts() -> None:
    """fwd+bwd algorithmic FLOPs quoted for the BASELINE configurations."""
    fb = "forward-backward"
    assert attention_flops(batch=4, query_heads=16, sequence=4096, head_dim=64, causal=True,
                           mode=fb) == 481_153_777_664
    assert attention_flops(batch=4, query_heads=16, sequence=4096, head_dim=64, causal=True,
                           mode="forward") == 137_472_507_904
    assert attention_flops(batch=2, query_heads=16, sequence=2049, head_dim=64, causal=True,
                           mode=fb) == 60_217_651_200
    assert attention_flops(batch=2, query_heads=32, sequence=8192, head_dim=128, causal=False,
                           mode=fb) == 7_696_581_394_432
    assert attention_flops(batch=2, query_heads=32, sequence=8192, head_dim=128, causal=True,
                           mode=fb) == 3_848_760_459_264
    assert attention_flops(batch=1, query_heads=8, sequence=16381, head_dim=32, causal=True,
                           mode=fb) == 480_889_547_264
    # the published RTX 5050 figure: 4.8115e11 FLOP / 36.22221 ms = 13.283 TFLOP/s
    assert round(481_153_777_664 / 36.22221e-3 / 1e12, 3) == 13.283
    # the reference memory model at that shape: 2048 MiB of scores vs 1 MiB of LSE
    m = memory_model(batch=4, query_heads=16, sequence=4096)
    assert m == {"naive_score_mib": 2048.0, "saved_lse_mib": 1.0}


def test_per_kernel_flops_sum_to_the_fwd_bwd_convention() -> None:
    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for causal in (False, True):
        total = sum(bench.kernel_flops(k, 4, 16, 4096, 64, causal) for k in ("fwd", "dkdv", "dq"))
        assert total == attention_flops(batch=4, query_heads=16, sequence=4096, head_dim=64,
                                        causal=causal, mode="forward-backward")


def test_bench_refuses_more_than_one_gpu(capsys) -> None:
    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    assert bench.main(["--gpus", "8"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_bench_device_label_without_a_marketing_name(monkeypatch) -> None:
    """Where the device name table is missing the name comes back empty; the
    bench line then names the architecture and compute units."""
    import types

    import torch

    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    props = types.SimpleNamespace(name="", gcnArchName="gfx950:sramecc+:xnack-",
                                  multi_processor_count=256)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda i: props)
    assert bench.device_label() == "gfx950:sramecc+:xnack-, 256 CUs"
    props.name = "AMD Instinct MI355X"
    assert bench.device_label() == "AMD Instinct MI355X (gfx950:sramecc+:xnack-, 256 CUs)"


def test_tiling_sweep_counts_executed_matmuls() -> None:
    """The sweep's executed FLOP: the forward equals the harness's forward count;
    dK/dV and dQ recompute S and dP, so the three kernels execute 9 matmuls
    where the harness's 3.5 x forward convention counts 7."""
    from benchmarks.tiling_sweep import executed_flops

    kw = dict(batch=2, query_heads=3, seq_len=17, head_dim=32)
    for causal in (False, True):
        fwd = executed_flops("fwd", causal=causal, **kw)
        assert fwd == attention_flops(batch=2, query_heads=3, sequence=17, head_dim=32,
                                      causal=causal, mode="forward")
        assert executed_flops("dkdv", causal=causal, **kw) == 2 * fwd
        assert 2 * executed_flops("dq", causal=causal, **kw) == 3 * fwd
    assert executed_flops("fwd", batch=1, query_heads=1, seq_len=4, head_dim=8,
                          causal=True) == 2 * 2 * 10 * 8


def test_tiling_sweep_rejects_bad_arguments() -> None:
    import pytest

    from benchmarks.tiling_sweep import main

    with pytest.raises(SystemExit):
        main(["--kernels", "fwd,bogus"])
    with pytest.raises(SystemExit):
        main(["--query-heads", "6", "--kv-heads", "4"])
    with pytest.raises(SystemExit, match="comma-separated integers"):
        main(["--variants", "6,x"])
    with pytest.raises(SystemExit):
        main(["--dtype", "float32"])


def test_cross_attention_flops_count_top_left_visible_pairs() -> None:
    """kv_sequence (the cross-attention extension): N_q * N_kv pairs without the
    mask; under SDPA's top-left causal mask query i sees min(i+1, N_kv) keys
    (brute-force count). kv_sequence = sequence is the reference's count."""
    kw = dict(batch=1, query_heads=1, head_dim=1, mode="forward")
    for n_q, n_kv in ((3, 7), (7, 3), (1, 32768), (5, 5)):
        brute = sum(min(i + 1, n_kv) for i in range(n_q))
        assert attention_flops(sequence=n_q, kv_sequence=n_kv, causal=True, **kw) == 4 * brute
        assert attention_flops(sequence=n_q, kv_sequence=n_kv, causal=False, **kw) == 4 * n_q * n_kv
    for causal in (False, True):
        assert attention_flops(sequence=9, kv_sequence=9, causal=causal, **kw) == \
            attention_flops(sequence=9, causal=causal, **kw)
    cross = memory_model(batch=1, query_heads=1, sequence=4, kv_sequence=1024)
    assert cross["naive_score_mib"] == memory_model(batch=1, query_heads=1, sequence=64)["naive_score_mib"]


def test_tiling_ab_parses_shapes_and_rejects_bad_arguments() -> None:
    import pytest

    from benchmarks.tiling_ab import label, main, parse_shape, parse_variants

    assert parse_shape("4,16,16,4096,64,causal") == {
        "B": 4, "Hq": 16, "Hkv": 16, "N": 4096, "Nkv": 4096, "D": 64, "causal": True,
        "dtype": "float16"}
    assert parse_shape("2,16,4,2049,32,noncausal,bfloat16")["dtype"] == "bfloat16"
    assert parse_shape("8,32,8,1,64,noncausal,float16,8192")["Nkv"] == 8192
    for bad in ("4,16,16,4096,64", "4,16,16,4096,64,sliding", "4,16,16,4096,48,causal",
                "4,6,4,4096,64,causal", "4,16,16,4096,64,causal,float32",
                "4,16,16,1,64,noncausal,float16,0"):
        with pytest.raises(ValueError):
            parse_shape(bad)
    with pytest.raises(SystemExit):
        main(["--kernel", "fwd", "--variants", "6", "--shape", "1,1,1,64,64,causal"])
    with pytest.raises(SystemExit):
        main(["--kernel", "fwd", "--variants", "6,6", "--shape", "1,1,1,64,64,causal"])
    with pytest.raises(SystemExit):
        main(["--kernel", "fwd", "--variants", "6,10", "--shape", "1,1,1,64,65,causal"])
    # auto is the library's own choice (no tiling set: -1); it counts as one tiling
    assert parse_variants("auto, 4,1") == [-1, 4, 1]
    assert [label(v) for v in (-1, 0, 5)] == ["auto", "0", "5"]
    for bad in ("-2,4", "four,4"):
        with pytest.raises(ValueError):
            parse_variants(bad)
    with pytest.raises(SystemExit):
        main(["--kernel", "dq", "--variants", "auto,auto", "--shape", "1,1,1,64,64,causal"])
