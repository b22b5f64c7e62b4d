"""drt_op_q4_linear_noalloc (no workspace argument, no device allocation) against
drt_op_q4_linear with a caller workspace, through the C-ABI: three calls in a
row, each with a smaller input than the one before (the shared scratch keeps
the previous call's contents), each bit-exact with the workspace entry point (same kernels, same
workspace layout), on the weight-streaming, large-M and decode-sized paths; a
shape beyond the scratch is refused before any launch."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def test_q4_linear_noalloc_matches_the_workspace_entry_point():
    from diffusorrt_amd import _lib, kernels
    from diffusorrt_amd import synthetic as syn

    lib = _lib.load()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the weight-streaming path (m <= 32, n * k >= 8M weights: fp32 K slices in the
    # scratch, summed with the bias by the slice pass), then large-M (split-K
    # partials in the scratch), then a smaller decode-sized call
    for m, n, k, seed in [(32, 3584, 18944, 40), (128, 3072, 1024, 41), (8, 1024, 2048, 42)]:
        _say("q4_linear_noalloc", m, n, k)
        gen = torch.Generator().manual_seed(seed)
        q = syn.random_q4(gen, n, k, scale_lo=0.005, scale_hi=0.02, centred=False)
        w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
        x = torch.randn((m, k), generator=gen).cuda()
        bias = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16).cuda()
        y_ws = torch.full((m, n), float("nan"), device="cuda")
        y_na = torch.full((m, n), float("nan"), device="cuda")
        ws_bytes = lib.drt_op_q4_linear_workspace_bytes(m, n, k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        _lib.check(lib.drt_op_q4_linear(_ptr(w.qw), _ptr(w.sb), _ptr(x), _lib.F32, m, n, k,
                                        _ptr(bias), _ptr(y_ws), _ptr(ws), ws_bytes, stream))
        _lib.check(lib.drt_op_q4_linear_noalloc(_ptr(w.qw), _ptr(w.sb), _ptr(x), _lib.F32, m, n,
                                                k, _ptr(bias), _ptr(y_na), stream))
        torch.cuda.synchronize()
        a, b = y_ws.cpu().numpy(), y_na.cpu().numpy()
        assert np.isfinite(b).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # 18944 x 18944 at 1024 rows needs far more than the 64 MiB scratch: refused
    # by the host check, nothing is launched (the pointers are never touched)
    assert lib.drt_op_q4_linear_workspace_bytes(1024, 18944, 18944) > (64 << 20)
    st = lib.drt_op_q4_linear_noalloc(_ptr(w.qw), _ptr(w.sb), _ptr(x), _lib.F32, 1024, 18944,
                                      18944, None, _ptr(y_na), stream)
    assert st == _lib.INVALID_ARGUMENT and "scratch" in _lib.last_error()
