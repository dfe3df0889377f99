"""GPU check of the allocation-free GEMV entry point (sgq_gemv_q4_0_noalloc,
called through the C ABI): its output equals sgq_gemv_q4_0's bit for bit (the
same kernels; only where the x limb table lives differs) and the f64 oracle
at the GEMV bar, on two calls in a row, the second with a smaller input (the
device scratch array keeps the first call's contents), and sizes beyond the
array are refused."""
import ctypes as C

import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host, rel_err

pytestmark = pytest.mark.gpu


def _noalloc(sgq, w, x, y, n, k):
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return sgq.lib().sgq_gemv_q4_0_noalloc(stream, C.c_void_p(w.data_ptr()),
                                            C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr()),
                                            n, k)


@pytest.mark.parametrize("shapes", [[(21504, 5376), (5376, 1000)], [(5376, 4096), (320, 77)]])
def test_gemv_noalloc_matches_gemv_and_oracle(ctx, oracle, shapes):
    import sgq

    for i, (k, n) in enumerate(shapes):
        print(f"gemv noalloc call {i}: k={k} n={n}", flush=True)
        rng = oracle.Rng(0x0A11 + 7 * k + n)
        w = rng.random_q4_0(n * k // 32)
        x = rng.f32_vec(k)
        tw, tx = dev(w), dev(x)
        y_na = torch.full((n,), float("nan"), device="cuda")
        y_ref = empty(n, torch.float32)
        assert _noalloc(sgq, tw, tx, y_na, n, k) == 0, sgq.lib().sgq_last_error()
        torch.cuda.synchronize()
        ctx.gemv_q4_0(tw, tx, y_ref, n, k)
        ctx.synchronize()
        torch.cuda.synchronize()
        got = host(y_na)
        assert np.array_equal(got.view(np.uint32), host(y_ref).view(np.uint32)), (k, n)
        want = oracle.gemv_rows(w, x, k, np.arange(n))
        rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
        assert_close(got, want, 1e-3, 3e-4 * rms, f"noalloc k={k} n={n}")
        assert rel_err(got, want) <= 1e-4


def test_gemv_noalloc_rejects_oversize_and_null(ctx):
    import sgq

    w = empty(18 * 4, torch.uint8)
    x = empty(65600, torch.float32)
    y = empty(4, torch.float32)
    assert _noalloc(sgq, w, x, y, 1, 65600) == 6
    assert b"65536" in sgq.lib().sgq_last_error()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert sgq.lib().sgq_gemv_q4_0_noalloc(stream, None, C.c_void_p(x.data_ptr()),
                                            C.c_void_p(y.data_ptr()), 1, 64) == 6


def test_gemv_noalloc_refuses_a_second_stream_while_busy(ctx, oracle):
    """A call on stream B while the previous call, on stream A, is still
    queued behind a long kernel is refused (the two would share the scratch
    array); once A has drained, B is accepted and the result is right."""
    import sgq

    k, n = 5376, 512
    rng = oracle.Rng(0x0A12)
    w, x = rng.random_q4_0(n * k // 32), rng.f32_vec(k)
    tw, tx = dev(w), dev(x)
    ya, yb = empty(n, torch.float32), empty(n, torch.float32)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    L = sgq.lib()

    def call(s, y):
        return L.sgq_gemv_q4_0_noalloc(C.c_void_p(s.cuda_stream), C.c_void_p(tw.data_ptr()),
                                       C.c_void_p(tx.data_ptr()), C.c_void_p(y.data_ptr()), n, k)

    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        torch.cuda._sleep(200_000_000)  # ~0.1 s of spinning ahead of the call on A
    assert call(sa, ya) == 0, L.sgq_last_error()
    assert call(sb, yb) == 6
    assert b"another stream" in L.sgq_last_error()
    assert call(sa, ya) == 0  # the same stream is ordered: accepted
    sa.synchronize()
    assert call(sb, yb) == 0, L.sgq_last_error()
    sb.synchronize()
    assert torch.equal(ya, yb)
    want = oracle.gemv_rows(w, x, k, np.arange(n))
    assert rel_err(host(yb), want) <= 1e-4
