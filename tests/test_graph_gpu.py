"""HIP-graph capture of the HIP path: every replay must equal the eager result bit for bit.

The library records no memset nodes (all kernels write every output element), so captured
transforms replay correctly; each case replays three times with unrelated eager work between.
"""

from __future__ import annotations

import pytest
import torch

import trnfft_amd
from conftest import seeded_complex
from trnfft_amd import ComplexTensor

pytestmark = pytest.mark.gpu


def _capture(fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up outside capture (plans and tables are created here)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            out = fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return g, out


@pytest.mark.parametrize("n,batch", [(1024, 512), (1000, 64), (1 << 16, 4), (4099, 8)])
@pytest.mark.parametrize("inverse", [False, True])
def test_graph_replay_matches_eager(n, batch, inverse):
    re, im = seeded_complex(batch, n, seed=5)
    x = ComplexTensor(re.cuda(), im.cuda())
    op = trnfft_amd.ifft if inverse else trnfft_amd.fft
    eager = op(x)
    g, out = _capture(lambda: op(x))
    other = ComplexTensor(torch.randn(batch, n, device="cuda"), torch.randn(batch, n, device="cuda"))
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.real, eager.real) and torch.equal(out.imag, eager.imag)
        op(other)  # unrelated eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_stft_and_fft2():
    g0 = torch.Generator().manual_seed(9)
    wave = torch.randn(4, 20000, generator=g0).cuda()
    img = torch.rand(2, 256, 512, generator=g0).cuda()
    e1 = trnfft_amd.stft(wave, n_fft=512, hop_length=256)
    e2 = trnfft_amd.fft2(img)
    g, (o1, o2) = _capture(lambda: (trnfft_amd.stft(wave, n_fft=512, hop_length=256), trnfft_amd.fft2(img)))
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o1.real, e1.real) and torch.equal(o1.imag, e1.imag)
        assert torch.equal(o2.real, e2.real) and torch.equal(o2.imag, e2.imag)
        trnfft_amd.fft(torch.randn(16, 64, device="cuda"))
        torch.cuda.synchronize()


def test_graph_replay_real_istft_and_split_bluestein():
    # r2c / c2r kernels, the fused inverse STFT, and the split Bluestein path (its workspace is a
    # tensor allocated inside the captured region, so it comes from the graph's memory pool)
    g0 = torch.Generator().manual_seed(10)
    rows = torch.randn(64, 1024, generator=g0).cuda()
    bins = ComplexTensor(torch.randn(64, 513, generator=g0).cuda(), torch.randn(64, 513, generator=g0).cuda())
    spec = trnfft_amd.stft(torch.randn(3, 12000, generator=g0).cuda(), n_fft=512, hop_length=128)
    few = ComplexTensor(torch.randn(3, 8201, generator=g0).cuda(), torch.randn(3, 8201, generator=g0).cuda())

    def ops():
        return (trnfft_amd.rfft(rows), trnfft_amd.irfft(bins), trnfft_amd.istft(spec, n_fft=512, hop_length=128),
                trnfft_amd.fft(few))

    e = ops()
    g, o = _capture(ops)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o[0].real, e[0].real) and torch.equal(o[0].imag, e[0].imag)
        assert torch.equal(o[1], e[1])
        assert torch.equal(o[2], e[2])
        assert torch.equal(o[3].real, e[3].real) and torch.equal(o[3].imag, e[3].imag)
        trnfft_amd.fft(torch.randn(16, 64, device="cuda"))
        torch.cuda.synchronize()


def test_graph_replay_short_rows_small_images_and_strided_axes():
    # the staged kernels: short c2c rows (N = 16, 32, 64), short real rows, single-pass small
    # images, strided axes with few trailing columns and Bluestein down a strided axis
    g0 = torch.Generator().manual_seed(21)
    a = ComplexTensor(torch.randn(300, 32, generator=g0).cuda(), torch.randn(300, 32, generator=g0).cuda())
    b = ComplexTensor(torch.randn(700, 16, generator=g0).cuda(), torch.randn(700, 16, generator=g0).cuda())
    c = ComplexTensor(torch.randn(130, 64, generator=g0).cuda(), torch.randn(130, 64, generator=g0).cuda())
    r = torch.randn(513, 16, generator=g0).cuda()
    img = ComplexTensor(torch.randn(19, 16, 16, generator=g0).cuda(), torch.randn(19, 16, 16, generator=g0).cuda())
    few = ComplexTensor(torch.randn(9, 128, 3, generator=g0).cuda(), torch.randn(9, 128, 3, generator=g0).cuda())
    blue = ComplexTensor(torch.randn(3, 100, 40, generator=g0).cuda(), torch.randn(3, 100, 40, generator=g0).cuda())

    def run():
        return (trnfft_amd.fft(a), trnfft_amd.ifft(b), trnfft_amd.fft(c), trnfft_amd.rfft(r), trnfft_amd.fft2(img),
                trnfft_amd.fftn(few, dim=(1,)), trnfft_amd.ifftn(blue, dim=(1,)))

    eager = run()
    g, outs = _capture(run)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.real, e.real) and torch.equal(o.imag, e.imag)
        trnfft_amd.fft(a)  # unrelated eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_multipass_paths():
    # the strided multi-pass path (a 2^17 axis down a strided dimension, workspace from the
    # caching allocator inside the capture) and the 2^24 contiguous three-pass path
    g0 = torch.Generator().manual_seed(21)
    vol = ComplexTensor(torch.randn(2, 1 << 17, 8, generator=g0).cuda(), torch.randn(2, 1 << 17, 8, generator=g0).cuda())
    row = ComplexTensor(torch.randn(1, 1 << 24, generator=g0).cuda(), torch.randn(1, 1 << 24, generator=g0).cuda())
    e1 = trnfft_amd.fftn(vol, dim=(1,))
    e2 = trnfft_amd.fft(row)
    g, (o1, o2) = _capture(lambda: (trnfft_amd.fftn(vol, dim=(1,)), trnfft_amd.fft(row)))
    other = ComplexTensor(torch.randn(2, 1 << 17, 8, device="cuda"), torch.randn(2, 1 << 17, 8, device="cuda"))
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o1.real, e1.real) and torch.equal(o1.imag, e1.imag)
        assert torch.equal(o2.real, e2.real) and torch.equal(o2.imag, e2.imag)
        trnfft_amd.ifftn(other, dim=(1,))  # unrelated eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("n,batch", [(1024, 256), (1 << 18, 2), (4099, 4)])
def test_graph_replay_after_plan_cache_clear(n, batch):
    # a captured graph holds the plan's device tables: clearing the cache (and collecting the
    # Python plan objects) must not free them while the graph can still be replayed
    import gc

    from trnfft_amd.plan import clear_plan_cache

    clear_plan_cache()
    re, im = seeded_complex(batch, n, seed=6)
    x = ComplexTensor(re.cuda(), im.cuda())
    eager = trnfft_amd.fft(x)
    g, out = _capture(lambda: trnfft_amd.fft(x))
    clear_plan_cache()
    gc.collect()
    # new plans of other lengths allocate device tables after the clear
    for m in (2048, 999, 1 << 17):
        trnfft_amd.fft(ComplexTensor(torch.randn(2, m, device="cuda"), torch.randn(2, m, device="cuda")))
    torch.cuda.synchronize()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.real, eager.real) and torch.equal(out.imag, eager.imag)
