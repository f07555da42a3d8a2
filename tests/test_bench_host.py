"""Host-side pieces of bench.py's contract (no GPU): the one-GPU refusal, the buffer rotation that
keeps every timed launch out of the 256 MB Infinity Cache, and the seeded synthetic inputs."""

from __future__ import annotations

import torch

import bench


def test_more_than_one_gpu_exits_with_a_message(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    err = capsys.readouterr().err
    assert "one GPU" in err and "--gpus 2" in err


def test_rotation_covers_more_than_the_infinity_cache():
    # C1: 67,108,864 bytes per buffer set (two planes in, two out)
    sets = bench._n_sets(67_108_864)
    assert sets * 67_108_864 >= bench.ROTATE_BYTES > 4 * 256 * 2**20
    assert bench._n_sets(10 * 2**30) == 1  # a set larger than the rotation target is used alone


def test_synthetic_inputs_are_seeded_and_shaped():
    a_re, a_im = bench.make_c2c_input(8, 1024)
    b_re, b_im = bench.make_c2c_input(8, 1024)
    assert a_re.shape == (8, 1024) and a_re.dtype == torch.float32
    assert torch.equal(a_re, b_re) and torch.equal(a_im, b_im) and not torch.equal(a_re, a_im)
    x = bench.make_stft_input(3, 16000)
    assert x.shape == (3, 16000) and x.dtype == torch.float32
    assert torch.equal(x, bench.make_stft_input(3, 16000))
    # three sinusoids of amplitude < 1 plus N(0, 0.1) noise
    assert 0.05 < float(x.std()) < 2.0


def test_copy_ceiling_library_exports_its_entry_points():
    # the bench's measured copy ceilings come from libtfa_copy.so (built with the library): it
    # loads without a GPU and exports the split-plane and one-stream copies bench.py binds
    import os
    import pytest

    path = os.path.join(bench.ROOT, "trnfft_amd", "libtfa_copy.so")
    if not os.path.exists(path):
        pytest.skip("libtfa_copy.so not built")
    lib = bench._copy_lib()
    for name in ("tfa_bench_copy2", "tfa_bench_copy2_variants", "tfa_bench_copy1"):
        assert hasattr(lib, name)
    assert lib.tfa_bench_copy2_variants() == 4


def test_trace_summary_splits_the_headline_dispatches_by_region(tmp_path):
    # a synthetic kernel trace in rocprofv3's CSV form: the headline kernel's dispatches in
    # bench_headline's launch order, each region with its own duration, other kernels between
    import csv

    warmup, steps = 2, 3
    R = 2 * bench.ROOFLINE_STEPS
    regions = [("graph_warmup", 3 * R, 14000), ("graph_timed", 3 * R, 12800), ("eager_fixed", 3 * R, 12700),
               ("warmup_steps", 2 * warmup, 13000), ("timed_steps", 3 * 2 * steps, 12900), ("isolated_pairs", 200, 15000)]
    path = tmp_path / "run_kernel_trace.csv"
    t = 1_000_000
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for _, cnt, dur in regions:
            for k in range(cnt):
                name = "void tfa::c2c_lds_kernel<1024, %d, false, false, 8, 512>(float const*)" % (-1 if k % 2 == 0 else 1)
                w.writerow({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + dur})
                t += dur + 100
            w.writerow({"Kernel_Name": "void copy2_kernel<1, true, true>(...)", "Start_Timestamp": t,
                        "End_Timestamp": t + 5000})
            t += 50_000
    out = bench.trace_summary(str(path), warmup, steps)
    assert out["dispatches"] == sum(cnt for _, cnt, _ in regions)
    for name, cnt, dur in regions:
        assert out[name]["dispatches"] == cnt
        assert abs(out[name]["avg_us"] - dur / 1000) < 1e-9
    # back-to-back dispatches 100 ns apart: the span per dispatch of a replay is duration + gap,
    # less the one gap after the last dispatch
    span = out["graph_timed"]["span_per_dispatch_us"]
    assert len(span) == 3
    assert all(abs(s - (12.8 + 0.1 * (R - 1) / R)) <= 5e-4 for s in span)  # reported to 0.001 us
