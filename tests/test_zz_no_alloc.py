"""The allocation-free entry point (tfa_execute_noalloc) against tfa_execute with a caller
workspace, through the C ABI: same kernels, so the outputs must be bit-identical.  Two calls in
a row, the second with a smaller input, for each plan family that uses scratch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import seeded_complex
from trnfft_amd import _lib
from trnfft_amd.plan import native_plan

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _P(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _run_both(plan, batch, n_in, n_out, seed):
    lib = _lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    re, im = seeded_complex(batch, n_in, seed=seed)
    re, im = re.cuda(), im.cuda()
    ws_bytes = plan.workspace_bytes(batch)
    ws = torch.empty(max(1, ws_bytes // 4), device="cuda") if ws_bytes else None
    ref = (torch.empty(batch, n_out, device="cuda"), torch.empty(batch, n_out, device="cuda"))
    got = (torch.full((batch, n_out), float("nan"), device="cuda"), torch.full((batch, n_out), float("nan"), device="cuda"))
    rc = lib.tfa_execute(plan.handle, batch, _P(re), _P(im), _P(ref[0]), _P(ref[1]), _P(ws), stream)
    _lib.check(rc, "tfa_execute")
    rc = lib.tfa_execute_noalloc(plan.handle, batch, _P(re), _P(im), _P(got[0]), _P(got[1]), stream)
    _lib.check(rc, "tfa_execute_noalloc")
    torch.cuda.synchronize()
    return ws_bytes, ref, got


@pytest.mark.parametrize("kind,n,batches", [
    (_lib.KIND_C2C, 1 << 20, (6, 2)),     # four-step: 48 MiB then 16 MiB of scratch
    (_lib.KIND_C2C, 1 << 24, (1, 1)),     # 2^24 three-pass path: 128 MiB -> rejected (checked below)
    (_lib.KIND_BLUESTEIN, 6000, (40, 3)),  # split Bluestein below 64 rows (m = 16384)
    (_lib.KIND_BLUESTEIN, 20000, (4, 1)),  # split Bluestein, m = 65536
    (_lib.KIND_C2C, 1024, (64, 8)),       # no scratch: plain tfa_execute
])
def test_noalloc_matches_execute(kind, n, batches):
    plan = native_plan(kind, n, False, torch.cuda.current_device())
    for i, batch in enumerate(batches):
        need = plan.workspace_bytes(batch)
        if need > SCRATCH_BYTES:
            lib = _lib.lib()
            x = torch.zeros(batch, n, device="cuda")
            rc = lib.tfa_execute_noalloc(plan.handle, batch, _P(x), _P(x), _P(x), _P(x),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == _lib.TFA_ERR_INVALID
            assert b"scratch" in lib.tfa_last_error()
            continue
        ws_bytes, ref, got = _run_both(plan, batch, n, n, seed=31 + i)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), (kind, n, batch, ws_bytes)


def test_noalloc_rejects_oversized_scratch_with_a_clear_error():
    plan = native_plan(_lib.KIND_C2C, 1 << 20, True, torch.cuda.current_device())
    batch = 9  # 72 MiB of four-step scratch
    assert plan.workspace_bytes(batch) > SCRATCH_BYTES
    lib = _lib.lib()
    x = torch.zeros(1, device="cuda")
    rc = lib.tfa_execute_noalloc(plan.handle, batch, _P(x), _P(x), _P(x), _P(x), None)
    assert rc == _lib.TFA_ERR_INVALID
    assert b"64" in lib.tfa_last_error() or b"67108864" in lib.tfa_last_error()


def test_noalloc_calls_on_two_streams_are_ordered():
    # eager calls on two streams share the GPU's scratch; the library orders them on the device
    # (each waits for the previous call's event), so every output equals tfa_execute's with a
    # workspace of its own, bit for bit, though the host enqueues the calls back to back
    lib = _lib.lib()
    dev = torch.cuda.current_device()
    plan = native_plan(_lib.KIND_C2C, 1 << 20, False, dev)
    blue = native_plan(_lib.KIND_BLUESTEIN, 20000, True, dev)  # split Bluestein, m = 65536
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    cases = []
    for i in range(6):
        p, n, batch = (plan, 1 << 20, 4) if i % 2 == 0 else (blue, 20000, 3)
        re, im = seeded_complex(batch, n, seed=70 + i)
        re, im = re.cuda(), im.cuda()
        ws = torch.empty(p.workspace_bytes(batch) // 4, device="cuda")
        ref = (torch.empty(batch, n, device="cuda"), torch.empty(batch, n, device="cuda"))
        _lib.check(lib.tfa_execute(p.handle, batch, _P(re), _P(im), _P(ref[0]), _P(ref[1]), _P(ws),
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "tfa_execute")
        got = (torch.full((batch, n), float("nan"), device="cuda"), torch.full((batch, n), float("nan"), device="cuda"))
        cases.append((p, batch, re, im, ref, got))
    torch.cuda.synchronize()
    for i, (p, batch, re, im, ref, got) in enumerate(cases):
        s = streams[i % 2]
        rc = lib.tfa_execute_noalloc(p.handle, batch, _P(re), _P(im), _P(got[0]), _P(got[1]),
                                     ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "tfa_execute_noalloc")
    torch.cuda.synchronize()
    for i, (p, batch, re, im, ref, got) in enumerate(cases):
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), i
