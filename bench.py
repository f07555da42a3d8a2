#!/usr/bin/env python3
"""Benchmark of the trnfft_amd HIP FFT path on one MI355X.

Headline (the BASELINE metric): batched fp32 c2c FFT, 4096 signals x N=1024,
one step = one forward FFT of one batch plus one inverse FFT of another batch, with inputs
resident in HBM and the buffer sets rotated over > 1 GiB so no launch reads data left in the
256 MB Infinity Cache by the previous one.  Reported:
  value      GFLOP/s (5 N log2 N per transform) of the whole timed region
  roofline   the c2c kernel's algorithmic bytes per launch / its average launch duration
             (HIP events on the launch stream) against 8 TB/s
  cpu_baseline  the reference's pytorch path (its literal per-k radix-2 loop, restated in
             oracle/) timed on this host's cores on the same workload
  secondary  the other BASELINE configs (STFT, Bluestein, fft2, four-step N=2^20, GEMMs):
             kernel time, GFLOP/s, algorithmic GB/s and fraction of 8 TB/s

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
FP32_PEAK = 157.3e12  # MI355X dense fp32 (matrix), flop/s


def make_c2c_input(batch: int, n: int, seed: int = 42):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, n, generator=g), torch.randn(batch, n, generator=g)


def make_stft_input(batch: int, length: int, seed: int = 42, sr: int = 16000) -> torch.Tensor:
    """Sum of 3 random-frequency sinusoids + N(0, 0.1) noise per waveform."""
    g = torch.Generator().manual_seed(seed)
    t = torch.arange(length, dtype=torch.float64) / sr
    f = 50.0 + (7950.0 - 50.0) * torch.rand(batch, 3, 1, generator=g, dtype=torch.float64)
    a = 0.1 + 0.9 * torch.rand(batch, 3, 1, generator=g, dtype=torch.float64)
    ph = 2 * math.pi * torch.rand(batch, 3, 1, generator=g, dtype=torch.float64)
    x = (a * torch.sin(2 * math.pi * f * t + ph)).sum(dim=1)
    x = x + 0.1 * torch.randn(batch, length, generator=g, dtype=torch.float64)
    return x.float()


def flops_fft(n: int, batch: int) -> float:
    return 5.0 * n * math.log2(n) * batch


class EventTimer:
    """Per-launch HIP event pairs on the launch stream; returns mean/median launch duration."""

    def __init__(self):
        self.pairs = []

    def record(self, fn):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        self.pairs.append((s, e))

    def durations_s(self):
        torch.cuda.synchronize()
        return [s.elapsed_time(e) * 1e-3 for s, e in self.pairs]


def _median(v):
    v = sorted(v)
    return v[len(v) // 2]


def _copy_lib():
    """libtfa_copy.so (built with the library): plain split-plane copy kernels, the measured
    ceiling for a transform's traffic."""
    lib = ctypes.CDLL(os.path.join(ROOT, "trnfft_amd", "libtfa_copy.so"))
    lib.tfa_bench_copy2.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_void_p]
    lib.tfa_bench_copy2.restype = ctypes.c_int
    lib.tfa_bench_copy2_variants.restype = ctypes.c_int
    lib.tfa_bench_copy1.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    lib.tfa_bench_copy1.restype = ctypes.c_int
    return lib


def bench_copy_ceiling(plane_floats: int, warm_s: float = 0.03):
    """Best time of the native split-plane copy variants (two planes of plane_floats fp32 read,
    two written: a transform's algorithmic traffic) over buffer sets rotated past the Infinity
    Cache, each variant timed like the secondary configs; returns (seconds, per-variant seconds)."""
    lib = _copy_lib()
    dev = torch.device("cuda", torch.cuda.current_device())
    S = _n_sets(4 * plane_floats * 4)
    srcs = [(torch.randn(plane_floats, device=dev), torch.randn(plane_floats, device=dev)) for _ in range(S)]
    dsts = [(torch.empty(plane_floats, device=dev), torch.empty(plane_floats, device=dev)) for _ in range(S)]
    times = []
    for v in range(lib.tfa_bench_copy2_variants()):
        def fn(k, st, v=v):
            a, b = srcs[k]
            c, d = dsts[(k + 1) % S]
            rc = lib.tfa_bench_copy2(a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), plane_floats, v, st)
            if rc:
                raise RuntimeError(f"tfa_bench_copy2 variant {v}: hip error {rc}")
        times.append(_time_rot(fn, S, warm_s=warm_s))
    for a, b in zip(srcs, dsts[1:] + dsts[:1]):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    del srcs, dsts
    return min(times), times


def bench_copy_1stream(floats: int, warm_s: float = 0.03):
    """The same bytes as one contiguous stream (floats fp32 read from one buffer, written to
    another; non-temporal float4), buffer sets rotated like bench_copy_ceiling: the fastest plain
    copy of a transform's traffic on this part.  Returns seconds per copy."""
    lib = _copy_lib()
    dev = torch.device("cuda", torch.cuda.current_device())
    S = _n_sets(2 * floats * 4)
    srcs = [torch.randn(floats, device=dev) for _ in range(S)]
    dsts = [torch.empty(floats, device=dev) for _ in range(S)]

    def fn(k, st):
        rc = lib.tfa_bench_copy1(srcs[k].data_ptr(), dsts[(k + 1) % S].data_ptr(), floats, st)
        if rc:
            raise RuntimeError(f"tfa_bench_copy1: hip error {rc}")

    t = _time_rot(fn, S, warm_s=warm_s)
    for a, b in zip(srcs, dsts[1:] + dsts[:1]):
        assert torch.equal(a, b)
    del srcs, dsts
    return t


def _traffic_from_profiles(kernel_tag: str):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE (profiles/*.md), or None."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_pmc.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", open(path).read())
    return float(m.group(1)) if m else None


# ---------------------------------------------------------------------------------------------
# headline: batched c2c N=1024
# ---------------------------------------------------------------------------------------------


ROOFLINE_STEPS = 200  # fixed back-to-back region for roofline.t_launch: 200 steps = 400 launches


def bench_headline(steps: int, warmup: int):
    import trnfft_amd
    from trnfft_amd import _lib
    from trnfft_amd.plan import native_plan

    batch, n = 4096, 1024
    dev = torch.device("cuda", torch.cuda.current_device())
    plane = batch * n * 4
    sets = max(4, math.ceil((1.25 * 2**30) / (4 * plane)))  # in+out (2 planes each) per set > 1.25 GiB total
    re, im = make_c2c_input(batch, n)
    ins = []
    for s in range(sets):
        # distinct data per set (rolled copies of the seeded batch)
        r = torch.roll(re, shifts=s, dims=0).to(dev)
        i = torch.roll(im, shifts=s, dims=0).to(dev)
        ins.append((r, i))
    outs = [(torch.empty_like(ins[0][0]), torch.empty_like(ins[0][0])) for _ in range(sets)]
    pf = native_plan(_lib.KIND_C2C, n, False, dev.index)
    pi = native_plan(_lib.KIND_C2C, n, True, dev.index)
    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    args_f = [
        (pf.handle, batch, ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
         ctypes.c_void_p(c.data_ptr()), ctypes.c_void_p(d.data_ptr()), None, stream)
        for (a, b), (c, d) in zip(ins, outs)
    ]
    # inverse of another set's input (same work, and its data is not the just-written output)
    args_i = [
        (pi.handle, batch, ctypes.c_void_p(ins[(k + sets // 2) % sets][0].data_ptr()),
         ctypes.c_void_p(ins[(k + sets // 2) % sets][1].data_ptr()),
         ctypes.c_void_p(outs[(k + sets // 2) % sets][0].data_ptr()),
         ctypes.c_void_p(outs[(k + sets // 2) % sets][1].data_ptr()), None, stream)
        for k in range(sets)
    ]
    execute = lib.tfa_execute

    def step(k, strm=None):
        af, ai = args_f[k % sets], args_i[k % sets]
        if strm is not None:
            af, ai = af[:-1] + (strm,), ai[:-1] + (strm,)
        rc = execute(*af)
        rc |= execute(*ai)
        if rc:
            _lib.check(rc, "tfa_execute")

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)

    def eager_region(k_steps):
        """Events around k_steps eager steps (one C-ABI call per launch from Python), bracketed by
        synchronize on both sides; returns (GPU seconds, wall seconds)."""
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record()
        for k in range(k_steps):
            step(k)
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) * 1e-3, time.perf_counter() - t0

    # roofline.t_launch: a fixed region of ROOFLINE_STEPS steps (2 x ROOFLINE_STEPS back-to-back
    # launches, alternating directions over the rotated sets), independent of --steps, captured
    # once into a HIP graph (no host work between launches); 3 warm-up replays, then 3 timed
    # replays, median
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            strm = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for k in range(ROOFLINE_STEPS):
                step(k, strm)
    torch.cuda.current_stream().wait_stream(cap)
    for _ in range(3):  # the first replays after capture run measurably slower
        graph.replay()
    graph_regions = []
    for _ in range(3):
        torch.cuda.synchronize()
        ev0.record()
        graph.replay()
        ev1.record()
        torch.cuda.synchronize()
        graph_regions.append(ev0.elapsed_time(ev1) * 1e-3)
    t_launch = _median(graph_regions) / (2 * ROOFLINE_STEPS)
    # the same fixed region launched eagerly, for comparison
    t_launch_eager = _median([eager_region(ROOFLINE_STEPS)[0] for _ in range(3)]) / (2 * ROOFLINE_STEPS)

    # the timed region reported as `value`: W warm-up steps, then exactly K steps, three times,
    # median.  It follows the fixed regions above without a pause, so the GPU has been running
    # this kernel for some 45 ms when it starts: back-to-back regions of 400 launches read 14.8,
    # 13.9, 13.2, 12.9 and then 12.7 us per launch from the process's first launches on, and the
    # same after a stretch of isolated launches.
    for k in range(warmup):
        step(k)
    torch.cuda.synchronize()
    regions = sorted(eager_region(steps) for _ in range(3))
    t_region, wall = regions[1]

    # per-launch kernel durations (separate pass, event pairs around each launch)
    timer = EventTimer()
    for k in range(100):
        timer.record(lambda k=k: execute(*args_f[k % sets]))
        timer.record(lambda k=k: execute(*args_i[k % sets]))
    d = timer.durations_s()

    # correctness of what was timed: the last graph step's two outputs (written after every
    # other access to those buffers in the graph) equal fresh eager transforms, bit for bit
    kf, ki = (ROOFLINE_STEPS - 1) % sets, (ROOFLINE_STEPS - 1 + sets // 2) % sets
    chk = trnfft_amd.fft(trnfft_amd.ComplexTensor(ins[kf][0], ins[kf][1]))
    chk_i = trnfft_amd.ifft(trnfft_amd.ComplexTensor(ins[ki][0], ins[ki][1]))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(chk.real, outs[kf][0]) and torch.equal(chk.imag, outs[kf][1])
    assert torch.equal(chk_i.real, outs[ki][0]) and torch.equal(chk_i.imag, outs[ki][1])
    del graph


    # the achievable rate for these bytes: native split-plane copies (two 16 MiB planes read, two
    # written per launch, rotated like the transform), best of four access styles
    del ins, outs, args_f, args_i
    torch.cuda.empty_cache()
    t_copy, copy_times = bench_copy_ceiling(batch * n)
    # and the same bytes as one contiguous stream (the fastest plain copy of them)
    t_copy1 = bench_copy_1stream(2 * batch * n)

    flops_step = 2 * flops_fft(n, batch)
    bytes_launch = 2 * 2 * plane  # read re+im, write re+im
    return {
        "t_copy_s": t_copy,
        "t_copy1_s": t_copy1,
        "copy_variants_us": [round(t * 1e6, 3) for t in copy_times],
        "t_region_s": t_region,
        "wall_s": wall,
        "ms_per_step": t_region / steps * 1e3,
        "value": flops_step * steps / t_region / 1e9,
        "regions_ms": [round(r[0] * 1e3, 4) for r in regions],
        "graph_regions_ms": [round(r * 1e3, 4) for r in graph_regions],
        "t_launch_s": t_launch,
        "t_launch_eager_s": t_launch_eager,
        "t_launch_median_s": _median(d),
        "bytes_launch": bytes_launch,
        "buffer_sets": sets,
    }


# ---------------------------------------------------------------------------------------------
# secondary configs (each: kernel time with events, median over launches)
# ---------------------------------------------------------------------------------------------


ROTATE_BYTES = 1.25 * 2**30  # > 4x the 256 MB Infinity Cache


def _n_sets(set_bytes: int) -> int:
    """Buffer sets to rotate so that consecutive launches never find their data in the MALL."""
    return max(1, math.ceil(ROTATE_BYTES / set_bytes))


def _time_rot(fn, n_sets: int, reps: int = 100, warm: int = 3, warm_s: float = 0.03) -> float:
    """Average launch duration of fn(k, stream) over `reps` back-to-back launches (k = buffer set
    k % n_sets) on the current stream, HIP events around the region, synchronize on both sides;
    median of three regions.  Eager launches: the host enqueues faster than these kernels run,
    so the region is the kernels' own time (a captured graph adds ~100 us per replay).  The
    untimed warm-up runs the same launches for at least `warm_s` seconds first: the GPU runs the
    first ~20 ms of work after a pause measurably slower."""
    cur = torch.cuda.current_stream()
    h = ctypes.c_void_p(cur.cuda_stream)
    t0 = time.perf_counter()
    k = 0
    while k < warm or time.perf_counter() - t0 < warm_s:
        for _ in range(8):
            fn(k % n_sets, h)
            k += 1
        torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    regions = []
    for _ in range(3):
        torch.cuda.synchronize()
        ev0.record()
        for k in range(reps):
            fn(k % n_sets, h)
        ev1.record()
        torch.cuda.synchronize()
        regions.append(ev0.elapsed_time(ev1) * 1e-3 / reps)
    return _median(regions)


def bench_secondary():
    from trnfft_amd import _lib
    from trnfft_amd.plan import native_plan

    dev = torch.device("cuda", torch.cuda.current_device())
    L = _lib.lib()

    def P(t):
        return ctypes.c_void_p(t.data_ptr() if t is not None else 0)

    def chk(rc):
        if rc:
            _lib.check(rc, "secondary")

    def rolled(t, n):
        """n distinct device copies of t (rows rolled), each a buffer set's input."""
        return [torch.roll(t, shifts=k, dims=0).to(dev) for k in range(n)]

    out = {}

    def rec(name, t, flops, nbytes, kind="hbm", note="", sets=None):
        r = {"ms": round(t * 1e3, 4), "gflops": round(flops / t / 1e9, 1), "gbps": round(nbytes / t / 1e9, 1)}
        if kind == "hbm":
            r["frac_hbm"] = round(nbytes / t / HBM_PEAK, 4)
        else:
            r["frac_fp32_mfma"] = round(flops / t / FP32_PEAK, 4)
        if sets is not None:
            r["buffer_sets"] = sets
        if note:
            r["note"] = note
        out[name] = r

    # C2: STFT 64 x 160000, n_fft 512, hop 256 (center, reflect, periodic Hann, onesided).  The
    # reference's result layout: contiguous (64, 257, 626) planes (its ComplexTensor makes the
    # transposed spectra contiguous, trnfft/complex.py:29-33); frames-major spectra (torch.stft's
    # memory order, an opt-in here) as a separate line
    bm = _lib.STFT_CENTER | _lib.STFT_ONESIDED
    fm = bm | _lib.STFT_FRAMES_MAJOR
    nbytes = 64 * 160000 * 4 + 2 * 64 * 257 * 626 * 4
    S = _n_sets(nbytes)
    xs = rolled(make_stft_input(64, 160000), S)
    win = torch.hann_window(512).to(dev)
    specs = {}
    for tag, flags, shape in [("", bm, (64, 257, 626)), ("_frames_major", fm, (64, 626, 257))]:
        pl = native_plan(_lib.KIND_STFT, 512, False, dev.index, hop=256, flags=flags)
        os_ = [(torch.empty(*shape, device=dev), torch.empty(*shape, device=dev)) for _ in range(S)]
        t = _time_rot(lambda k, st: chk(L.tfa_stft_execute(pl.handle, 64, 160000, P(xs[k]), P(win), P(os_[k][0]),
                                                           P(os_[k][1]), st)), S)
        rec("c2_stft_64x160000_nfft512" + tag, t, 40064 * 5 * 512 * 9, nbytes, sets=S,
            note="spectra (64, 257, 626) contiguous: the reference's layout" if not tag else
            "spectra (64, 626, 257): torch.stft's memory order (opt-in)")
        specs[tag] = (flags, os_)
    # inverse of C2 (fused istft: completion, inverse transform, window, overlap-add, envelope, trim)
    # from each layout
    ys = [torch.empty(64, 160000, device=dev) for _ in range(S)]
    for tag, (flags, os_) in specs.items():
        ipl = native_plan(_lib.KIND_STFT, 512, True, dev.index, hop=256, flags=flags)
        t = _time_rot(lambda k, st: chk(L.tfa_istft_execute(ipl.handle, 64, 626, P(os_[k][0]), P(os_[k][1]), P(win),
                                                            P(ys[k]), 160000, st)), S)
        rec("c2_istft_64x257x626_nfft512" + tag, t, 40064 * 5 * 512 * 9, nbytes, sets=S,
            note="inverse of c2: spectra " + ("(64, 257, 626), the reference's layout" if not tag else
                                              "(64, 626, 257)") + " in, 64 x 160000 samples out")
    del specs, ys
    # C2's signals at n_fft 400 (25 ms at 16 kHz), hop 160: one Bluestein chain per frame (the
    # reference's layout)
    w400 = torch.hann_window(400).to(dev)
    p400 = native_plan(_lib.KIND_STFT, 400, False, dev.index, hop=160, flags=bm)
    frames = 1 + 160000 // 160
    nbytes = 64 * 160000 * 4 + 2 * 64 * 201 * frames * 4
    os_ = [(torch.empty(64, 201, frames, device=dev), torch.empty(64, 201, frames, device=dev)) for _ in range(S)]
    t = _time_rot(lambda k, st: chk(L.tfa_stft_execute(p400.handle, 64, 160000, P(xs[k]), P(w400), P(os_[k][0]),
                                                   P(os_[k][1]), st)), S)
    rec("stft_64x160000_nfft400", t, 64 * frames * 2 * 5 * 768 * math.log2(768), nbytes, sets=S,
        note="non-power-of-two n_fft: two 768-point transforms per frame (gflops counts those), VALU-bound")
    # its inverse: one inverse Bluestein chain per frame (1024 points: every sample is kept)
    ip400 = native_plan(_lib.KIND_STFT, 400, True, dev.index, hop=160, flags=bm)
    ys = [torch.empty(64, 160000, device=dev) for _ in range(S)]
    t = _time_rot(lambda k, st: chk(L.tfa_istft_execute(ip400.handle, 64, frames, P(os_[k][0]), P(os_[k][1]),
                                                        P(w400), P(ys[k]), 160000, st)), S)
    rec("istft_64x201x1001_nfft400", t, 64 * frames * 2 * 5 * 1024 * 10, nbytes, sets=S,
        note="inverse of the n_fft 400 line: two 1024-point transforms per frame (gflops counts those), VALU-bound")
    del xs, os_, ys
    # C3: Bluestein (fused, one launch)
    for n, b in [(1000, 1024), (4099, 256)]:
        nbytes = 4 * b * n * 4
        S = _n_sets(nbytes)
        re, im = make_c2c_input(b, n)
        ins = list(zip(rolled(re, S), rolled(im, S)))
        outs = [(torch.empty(b, n, device=dev), torch.empty(b, n, device=dev)) for _ in range(S)]
        pl = native_plan(_lib.KIND_BLUESTEIN, n, False, dev.index)
        wsb = pl.workspace_bytes(b)  # the split three-pass path (few rows) uses a workspace
        ws = torch.empty(max(1, wsb // 4), device=dev) if wsb else None
        t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, b, P(ins[k][0]), P(ins[k][1]), P(outs[k][0]),
                                                  P(outs[k][1]), P(ws), st)), S)
        rec(f"c3_bluestein_{b}x{n}", t, flops_fft(n, b), nbytes, sets=S,
            note="split three-pass path (workspace in the Infinity Cache)" if wsb else "fused one-launch kernel")
        del ins, outs, ws
    # C4b: four-step N = 2^20, batch 16 (the workspace is written and read within one call)
    nbytes = 4 * 16 * (1 << 20) * 4
    S = _n_sets(nbytes)
    re, im = make_c2c_input(16, 1 << 20)
    ins = list(zip(rolled(re, S), rolled(im, S)))
    outs = [(torch.empty(16, 1 << 20, device=dev), torch.empty(16, 1 << 20, device=dev)) for _ in range(S)]
    pl = native_plan(_lib.KIND_C2C, 1 << 20, False, dev.index)
    ws = torch.empty(pl.workspace_bytes(16) // 4, device=dev)
    t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, 16, P(ins[k][0]), P(ins[k][1]), P(outs[k][0]),
                                              P(outs[k][1]), P(ws), st)), S)
    rec("c4b_fourstep_16x2^20", t, flops_fft(1 << 20, 16), nbytes, sets=S,
        note="two HBM passes; algorithmic bytes = one read + one write")
    del ins, outs, ws
    # C4a: fft2 32 x 2048 x 2048 real, U[0, 1) (1.5 GiB per set: no rotation needed)
    g = torch.Generator().manual_seed(42)
    img = torch.rand(32, 2048, 2048, generator=g).to(dev)
    yr = torch.empty_like(img)
    yi = torch.empty_like(img)
    pl = native_plan(_lib.KIND_FFT2, 2048, False, dev.index, n2=2048)
    t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, 32, P(img), None, P(yr), P(yi), None, st)), 1, reps=30, warm=1)
    rec("c4a_fft2_32x2048x2048", t, 32 * 5 * 2048 * 2048 * 22, 32 * 2048 * 2048 * (4 + 8), sets=1,
        note="two HBM passes; algorithmic bytes = real read + complex write")
    del img, yr, yi
    # C5a: ComplexLinear 8192 x 1024 -> 1024 (Kaiming-uniform U(+-1/32) weights, zero bias); MFMA-bound.
    # Buffer sets (x, W, y: 142.6 MB each) rotated past the Infinity Cache like the other configs
    nbytes = 142614528
    S = _n_sets(nbytes)
    g = torch.Generator().manual_seed(42)
    xr0, xi0 = torch.randn(8192, 1024, generator=g), torch.randn(8192, 1024, generator=g)
    wr0 = (torch.rand(1024, 1024, generator=g) * 2 - 1).div_(32)
    wi0 = (torch.rand(1024, 1024, generator=g) * 2 - 1).div_(32)
    xs = list(zip(rolled(xr0, S), rolled(xi0, S)))
    ws = list(zip(rolled(wr0, S), rolled(wi0, S)))
    br = torch.zeros(1024, device=dev)
    bi = torch.zeros(1024, device=dev)
    ys = [(torch.empty(8192, 1024, device=dev), torch.empty(8192, 1024, device=dev)) for _ in range(S)]
    t = _time_rot(lambda k, st: chk(L.tfa_complex_gemm(8192, 1024, 1024, P(xs[k][0]), P(xs[k][1]), 1024, P(ws[k][0]),
                                                   P(ws[k][1]), 1024, 1, P(br), P(bi), P(ys[k][0]), P(ys[k][1]),
                                                   1024, st)), S)
    rec("c5a_complex_linear_8192x1024x1024", t, 8.0 * 8192 * 1024 * 1024, nbytes, kind="mfma", sets=S)
    del xs, ws, ys
    # C5b: DFT-as-GEMM, 65536 x N=256 forward, and the same shape on the Stockham kernel
    nbytes = 4 * 65536 * 256 * 4
    S = _n_sets(nbytes)
    re, im = make_c2c_input(65536, 256)
    ins = list(zip(rolled(re, S), rolled(im, S)))
    outs = [(torch.empty(65536, 256, device=dev), torch.empty(65536, 256, device=dev)) for _ in range(S)]
    pl = native_plan(_lib.KIND_DFT_GEMM, 256, False, dev.index)
    t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, 65536, P(ins[k][0]), P(ins[k][1]), P(outs[k][0]),
                                              P(outs[k][1]), None, st)), S)
    rec("c5b_dft_gemm_65536x256", t, 8.0 * 65536 * 256 * 256, 268959744, kind="mfma", sets=S,
        note="flops = 8*M*N*N of the complex GEMM (the FFT-equivalent is 671 MFLOP)")
    pl = native_plan(_lib.KIND_C2C, 256, False, dev.index)
    t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, 65536, P(ins[k][0]), P(ins[k][1]), P(outs[k][0]),
                                              P(outs[k][1]), None, st)), S)
    rec("c5b_stockham_65536x256", t, flops_fft(256, 65536), nbytes, sets=S)
    del ins, outs
    # rfft / irfft as r2c / c2r kernels, 4096 rows x N=1024 (the headline shape, real signals)
    b, n = 4096, 1024
    nbytes = b * n * 4 + 2 * b * (n // 2 + 1) * 4
    S = _n_sets(nbytes)
    re, im = make_c2c_input(b, n)
    xs = rolled(re, S)
    bins = [(torch.empty(b, n // 2 + 1, device=dev), torch.empty(b, n // 2 + 1, device=dev)) for _ in range(S)]
    pl = native_plan(_lib.KIND_REAL, n, False, dev.index)
    t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, b, P(xs[k]), None, P(bins[k][0]), P(bins[k][1]), None,
                                              st)), S)
    rec("rfft_r2c_4096x1024", t, flops_fft(n, b) / 2, nbytes, sets=S, note="flops = 2.5 N log2 N per row")
    pl = native_plan(_lib.KIND_REAL, n, True, dev.index)
    t = _time_rot(lambda k, st: chk(L.tfa_execute(pl.handle, b, P(bins[k][0]), P(bins[k][1]), P(xs[(k + 1) % S]),
                                              None, None, st)), S)
    rec("irfft_c2r_4096x1024", t, flops_fft(n, b) / 2, nbytes, sets=S, note="flops = 2.5 N log2 N per row")
    del xs, bins
    # achievable-rate references: native split-plane copies of the headline's and C3b's traffic
    # (best of four access styles, same rotation and timing)
    for name, planef, what in [("copy_2x16MiB_planes", 4096 * 1024, "the headline's bytes (C1)"),
                               ("copy_2x4MiB_planes", 256 * 4099, "C3b's bytes (256 x 4099)")]:
        t, _ = bench_copy_ceiling(planef)
        rec(name, t, 0, 4 * planef * 4, sets=_n_sets(4 * planef * 4),
            note=f"native split-plane copy of {what}: the achievable rate for that traffic")
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------------------------
# CPU baseline: the reference's pytorch path (literal per-k radix-2 loop) on host cores
# ---------------------------------------------------------------------------------------------


CPU_K_LIMIT = 256  # literal-loop positions timed per stage in the capped samples (the rest extrapolated)


def bench_cpu_baseline():
    """The reference's pytorch CPU path (restated in oracle/, every power-of-two transform through
    the literal per-k loop of trnfft/fft_core.py:67-117) on this host's cores, for every BASELINE
    config.  Configs whose full run would take minutes are timed on a stated sample: stages with
    more than CPU_K_LIMIT butterfly positions run only the first CPU_K_LIMIT (each position of a
    stage does identical work, so the stage time scales by positions / run), and C4a runs one of
    its 32 images (scaled x 32)."""
    sys.path.insert(0, ROOT)
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    try:
        lscpu = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        model = next((l.split(":", 1)[1].strip() for l in lscpu.splitlines() if l.startswith("Model name")), "")
    except Exception:
        model = ""

    def timed(fn, k_limit=None, reps=1):
        """Median over reps of the (extrapolated) seconds of fn() under the literal loop, the
        wall seconds actually run for it, and the fraction of butterfly positions run."""
        secs, frac = [], 1.0
        for _ in range(reps):
            with oracle.LiteralLoopTiming(k_limit) as t:
                fn()
            secs.append((t.seconds, t.seconds - t.skipped_s))
            frac = t.positions_run / max(1, t.positions_total)
        sec, ran = sorted(secs)[len(secs) // 2]
        return sec, ran, frac

    configs = {}

    def rec(name, fn, flops, sample, k_limit=None, reps=1, scale=1.0):
        sec, ran, frac = timed(fn, k_limit, reps)
        sec *= scale
        configs[name] = {
            "seconds": round(sec, 4),
            "gflops": round(flops / sec / 1e9, 4),
            "reps": reps,
            # wall seconds actually measured for the sample (before extrapolation / scaling)
            "measured_seconds": round(ran, 4),
            "extrapolated": bool(k_limit) or scale != 1.0,
            "sample": sample + (f"; literal loop capped at {k_limit} positions per stage "
                                f"({100 * frac:.1f} % of positions run, rest extrapolated)" if k_limit else ""),
        }

    # C1: 4096 x 1024 fft + ifft (the headline workload), full, median of 3
    re, im = make_c2c_input(4096, 1024)
    oracle.cooley_tukey_loop(re[:64], im[:64], False)  # warm-up

    def c1():
        fr, fi = oracle.fft_core(re, im, False)
        oracle.fft_core(fr, fi, True)

    rec("c1_c2c_4096x1024_fwd_inv", c1, 2 * flops_fft(1024, 4096), "full workload (fft then ifft)", reps=3)
    # C2: STFT 64 x 160000, n_fft 512, hop 256, periodic Hann, reflect centre, onesided (api.py:291-365)
    x = make_stft_input(64, 160000)
    win = torch.hann_window(512)
    rec("c2_stft_64x160000_nfft512", lambda: oracle.stft(x, 512, 256, window=win), 40064 * 5 * 512 * 9,
        "full workload")
    # C3: Bluestein (fft_core.py:1285-1376): three m-point transforms per call
    for n, b, lim in [(1000, 1024, None), (4099, 256, CPU_K_LIMIT)]:
        re, im = make_c2c_input(b, n)
        rec(f"c3_bluestein_{b}x{n}", lambda: oracle.fft_core(re, im, False), flops_fft(n, b), "full batch", k_limit=lim)
    # C4a: fft2 of 32 real 2048 x 2048 images (api.py:105-139, transposes + two axis passes): one image
    g = torch.Generator().manual_seed(42)
    img = torch.rand(1, 2048, 2048, generator=g)
    rec("c4a_fft2_32x2048x2048", lambda: oracle.fft2(img), 32 * 5 * 2048 * 2048 * 22,
        "1 of the 32 images, time x 32", k_limit=CPU_K_LIMIT, scale=32.0)
    # C4b: 16 x 2^20 c2c (the reference's CPU path runs the radix-2 loop at any length)
    re, im = make_c2c_input(16, 1 << 20)
    rec("c4b_c2c_16x2^20", lambda: oracle.fft_core(re, im, False), flops_fft(1 << 20, 16), "full batch",
        k_limit=CPU_K_LIMIT)
    # C5a: ComplexLinear 8192 x 1024 -> 1024, four F.linear (nn.py:43-48), median of 3
    g = torch.Generator().manual_seed(42)
    xr, xi = torch.randn(8192, 1024, generator=g), torch.randn(8192, 1024, generator=g)
    wr = (torch.rand(1024, 1024, generator=g) * 2 - 1).div_(32)
    wi = (torch.rand(1024, 1024, generator=g) * 2 - 1).div_(32)
    rec("c5a_complex_linear_8192x1024x1024", lambda: oracle.complex_linear((xr, xi), wr, wi),
        8.0 * 8192 * 1024 * 1024, "full workload, 4 sgemm (torch CPU)", reps=3)
    # C5b: 65536 x 256 forward; the reference's CPU path runs the radix-2 loop (DFT-GEMM is NKI-only)
    re, im = make_c2c_input(65536, 256)
    rec("c5b_c2c_65536x256", lambda: oracle.fft_core(re, im, False), flops_fft(256, 65536),
        "full workload (radix-2 loop: the pytorch backend never takes the DFT-GEMM route)")
    del re, im, x, img, xr, xi

    head = configs["c1_c2c_4096x1024_fwd_inv"]
    return {
        "value": head["gflops"],
        "unit": "GFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"C1 full workload 4096x1024 fft+ifft, reference radix-2 per-k loop "
        f"(oracle.cooley_tukey_loop, trnfft/fft_core.py:53-117), torch CPU fp32, median of 3, "
        f"{head['seconds']:.2f} s/step; host: {model}",
        "host": model,
        "configs": configs,
    }


HEADLINE_KERNEL = "c2c_lds_kernel<1024, "


def trace_summary(csv_path: str, warmup: int, steps: int) -> dict:
    """Per-region average duration of the headline kernel's dispatches in a rocprofv3 kernel trace
    of `bench.py --steps K --warmup W` (the *_kernel_trace.csv of --kernel-trace), from the
    order bench_headline launches them in (both directions counted together):
      graph warm-up replays   3 x 2*ROOFLINE_STEPS
      graph timed replays     3 x 2*ROOFLINE_STEPS   <- roofline.t_launch
      eager fixed region      3 x 2*ROOFLINE_STEPS   <- roofline.t_launch_eager
      warm-up steps           2*W
      timed K-step regions    3 x 2*K                 <- value
      isolated event pairs    200                     <- roofline.t_launch_isolated_median
    For the graph regions it also reports the span from the first dispatch's start to the last's
    end divided by the dispatch count (what the events around a replay measure)."""
    import csv

    rows = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if HEADLINE_KERNEL in r.get("Kernel_Name", ""):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort()
    R = 2 * ROOFLINE_STEPS
    bounds = [("graph_warmup", 3 * R), ("graph_timed", 3 * R), ("eager_fixed", 3 * R), ("warmup_steps", 2 * warmup),
              ("timed_steps", 3 * 2 * steps), ("isolated_pairs", 200)]
    out, i = {"dispatches": len(rows)}, 0
    for name, cnt in bounds:
        seg = rows[i:i + cnt]
        i += cnt
        if len(seg) < cnt:
            break
        durs = [(e - b) * 1e-3 for b, e in seg]
        reg = {"dispatches": cnt, "avg_us": round(sum(durs) / cnt, 3), "median_us": round(_median(durs), 3)}
        if name.startswith("graph") or name == "eager_fixed":
            spans = [(seg[j + R - 1][1] - seg[j][0]) * 1e-3 / R for j in range(0, cnt, R)]
            reg["span_per_dispatch_us"] = [round(x, 3) for x in spans]
        out[name] = reg
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise a rocprofv3 kernel trace of a bench run made with the same --steps/--warmup "
                    "by region (no GPU needed) and exit")
    args = ap.parse_args(argv)
    if args.trace_summary:
        print(json.dumps(trace_summary(args.trace_summary, args.warmup, args.steps), indent=1))
        return 0
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only (requested --gpus {args.gpus}): every config here is a batch "
            "of independent transforms, which would shard by batch rows with no communication",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    head = bench_headline(args.steps, args.warmup)
    achieved = head["bytes_launch"] / head["t_launch_s"]
    result = {
        "metric": "batched c2c FFT GFLOP/s (5N·log2N) + % peak HBM GB/s, fp32, N=1024..2^20",
        "value": round(head["value"], 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0,1) re/im, seed 42, 4096x1024 (BASELINE config 1)",
        "timed_regions_ms": head["regions_ms"],
        "ms_per_step_wall": round(head["wall_s"] / args.steps * 1e3, 5),
        "config": {
            "workload": "batched c2c FFT, 4096 x N=1024 fp32 split re/im; step = forward fft of one batch + "
            "inverse fft of another, buffers rotated over >1 GiB; the K-step region (eager launches, events "
            "around it, synchronize on both sides) timed 3 times, median reported",
            "n": 1024,
            "batch": 4096,
            "buffer_sets": head["buffer_sets"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "c2c_lds_kernel<1024>",
            "achieved": round(achieved / 1e9, 1),
            "peak": 8000.0,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK, 4),
            "traffic": _traffic_from_profiles("c2c_lds_n1024"),
            "t_launch_us": round(head["t_launch_s"] * 1e6, 3),
            "t_launch_from": f"median of 3 replays of one HIP graph of {2 * ROOFLINE_STEPS} back-to-back launches "
            "(fixed, independent of --steps)",
            "graph_regions_ms": head["graph_regions_ms"],
            "t_launch_eager_us": round(head["t_launch_eager_s"] * 1e6, 3),
            "t_launch_isolated_median_us": round(head["t_launch_median_s"] * 1e6, 3),
            "bytes_per_launch": head["bytes_launch"],
            "copy_gbps": round(head["bytes_launch"] / head["t_copy_s"] / 1e9, 1),
            "copy_from": "native split-plane copy of the same bytes (libtfa_copy.so), best of 4 access styles, "
            "same buffer rotation",
            "copy_variants_us": head["copy_variants_us"],
            "frac_of_copy": round(head["t_copy_s"] / head["t_launch_s"], 4),
            "copy_1stream_gbps": round(head["bytes_launch"] / head["t_copy1_s"] / 1e9, 1),
            "copy_1stream_from": "the same bytes as one contiguous 32 MiB stream (libtfa_copy.so, non-temporal "
            "float4), same rotation: the fastest plain copy of them",
            "frac_of_1stream_copy": round(head["t_copy1_s"] / head["t_launch_s"], 4),
        },
    }
    if not args.no_secondary:
        result["secondary"] = bench_secondary()
    if not args.no_cpu:
        result["cpu_baseline"] = bench_cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
