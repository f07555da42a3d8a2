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
