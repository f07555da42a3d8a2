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
