"""GPU parity: the Q6_K logits GEMV (libsgq) vs the f64 CPU oracle.

Template: crates/sg-gpu/tests/parity_logits.rs (seeded random_q6k_rows in
the padded 4416-byte row layout, x through f16, f64 reference over the
q6_k.rs dequantization, 30·tanh(v/30) softcap, bit-determinism).  The
reference asserts 2e-2; the kernel computes exact (q-32) f16 values against
the f16 x with f32 sums, so it is held to |err| <= 1e-4·|want| + 2e-5.
"""
import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host

pytestmark = pytest.mark.gpu

K, STRIDE = 5376, 4416  # 21 super-blocks of 210 B, padded to a 16-byte multiple


def _inputs(oracle, seed, n, k=K, stride=STRIDE):
    rng = oracle.Rng(seed)
    w = rng.random_q6_k_rows(n, k, stride)
    x = oracle.through_f16(rng.f32_vec(k))
    return w, x


def test_q6k_logits_match_oracle(ctx, oracle):
    """parity_logits.rs:53-101: 96 vocabulary rows, softcap 30."""
    n = 96
    w, x = _inputs(oracle, 0xC6, n)
    y = empty(n, torch.float32)
    ctx.gemv_q6_k(dev(w), STRIDE, dev(x), y, n, K, 30.0)
    torch.cuda.synchronize()
    want = oracle.gemv_q6_k_logits(w, STRIDE, x, n, K, 30.0)
    assert_close(host(y), want, 1e-4, 2e-5, "gemv_q6_k_logits")


@pytest.mark.parametrize("n,k,stride", [(4099, 5376, 4416), (1000, 256, 224), (777, 6144, 5040)])
def test_q6k_raw_dot_and_shapes(ctx, oracle, n, k, stride):
    """Ragged row counts, the smallest and largest k, an fp32 x (the kernel
    rounds it to f16, the reference's activation type), no softcap."""
    rng = oracle.Rng(0xC8 + k)
    w = rng.random_q6_k_rows(n, k, stride)
    x = rng.f32_vec(k) * 3.0
    y = empty(n, torch.float32)
    ctx.gemv_q6_k(dev(w), stride, dev(x), y, n, k, 0.0)
    torch.cuda.synchronize()
    want = oracle.gemv_q6_k_logits(w, stride, oracle.through_f16(x), n, k, 0.0)
    scale = float(np.abs(want).max())
    assert_close(host(y), want, 1e-4, 1e-5 * scale, f"gemv_q6_k n={n} k={k}")


def test_q6k_logits_bit_deterministic(ctx, oracle):
    """parity_logits.rs:103-146: bit-identical across runs."""
    n = 512
    w, x = _inputs(oracle, 0xC7, n)
    tw, tx = dev(w), dev(x)
    a, b = empty(n, torch.float32), empty(n, torch.float32)
    ctx.gemv_q6_k(tw, STRIDE, tx, a, n, K, 30.0)
    ctx.gemv_q6_k(tw, STRIDE, tx, b, n, K, 30.0)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_q6k_name_dispatch_matches_typed(ctx, oracle):
    """load_kernel("gemv_q6_k_logits") + dispatch(bindings 0..2, groups
    [N,1,1]) as registered by the reference (build.rs:322-327: K 5376, rows
    padded to 4416 B, softcap 30) gives the typed entry point's bits."""
    import sgq

    n = 300
    w, x = _inputs(oracle, 0xC9, n)
    tw, tx = dev(w), dev(x)
    ref = empty(n, torch.float32)
    ctx.gemv_q6_k(tw, STRIDE, tx, ref, n, K, 30.0)
    kern = ctx.load_kernel("gemv_q6_k_logits_f32")
    assert kern.bindings == 3 and kern.push_bytes == 0
    y = empty(n, torch.float32)
    ctx.dispatch_blocking(kern, [sgq.BufferBinding.buffer(0, tw), sgq.BufferBinding.buffer(1, tx),
                                 sgq.BufferBinding.buffer(2, y)], None, [n, 1, 1])
    torch.cuda.synchronize()
    assert torch.equal(ref, y)
    with pytest.raises(sgq.ValidationError):  # weights binding too small for 2N rows
        ctx.dispatch(kern, [sgq.BufferBinding.buffer(0, tw), sgq.BufferBinding.buffer(1, tx),
                            sgq.BufferBinding.buffer(2, y)], None, [2 * n, 1, 1])


def test_q6k_rejects_bad_shapes(ctx):
    import sgq

    w = empty(4416 * 4, torch.uint8)
    x = empty(K, torch.float32)
    y = empty(4, torch.float32)
    with pytest.raises(sgq.ValidationError):  # unpadded stride: not a multiple of 16
        ctx.gemv_q6_k(w, 4410, x, y, 4, K)
    with pytest.raises(sgq.ValidationError):  # k not a multiple of 256
        ctx.gemv_q6_k(w, 4416, x, y, 4, K - 128)
    with pytest.raises(sgq.ValidationError):  # stride too short for k/256 blocks
        ctx.gemv_q6_k(w, 4400, x, y, 4, K)
