"""GPU parity: rmsnorm / rope / geglu / add_scaled (libsgq) vs the oracle.

Template: crates/sg-gpu/tests/parity_elementwise.rs (rmsnorm rows :26-70,
rope :72-137, geglu, add_scaled :176-214, determinism :216).  The oracle is
f64 (rmsnorm, rope, geglu) or the same f32 expression (add_scaled), so the
bars are: add_scaled bit-exact; the others |err| <= 2e-6*|want| + 2e-6*rms
(f32 rounding of a handful of operations; the reference's bar was 1e-3 with
f16 storage).  Each operator is run both as a typed entry point and through
load_kernel/dispatch under the reference's variant names.
"""
import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host

pytestmark = pytest.mark.gpu


def _close(got, want, what):
    rms = float(np.sqrt(np.mean(np.asarray(want, np.float64) ** 2))) or 1.0
    assert_close(got, want, 2e-6, 2e-6 * rms, what)


@pytest.mark.parametrize("row_len,rows,plus_one", [(5376, 7, False), (5376, 3, True),
                                                   (512, 33, False), (256, 65, True),
                                                   (128, 300, False), (100, 5, False)])
def test_rmsnorm_matches_oracle(ctx, oracle, row_len, rows, plus_one):
    rng = oracle.Rng(0xE1 + row_len + rows)
    x = rng.f32_vec(rows * row_len) * np.float32(3.0)
    w = rng.f32_vec(row_len)
    want = oracle.rmsnorm(x, w, row_len, 1e-6, plus_one)
    y = empty(rows * row_len, torch.float32)
    ctx.rmsnorm(dev(x), dev(w), y, rows, row_len, plus_one)
    torch.cuda.synchronize()
    _close(host(y), want, f"rmsnorm {row_len}x{rows}")


def test_rmsnorm_weightless_and_name_dispatch(ctx, oracle):
    import sgq

    rows, row_len = 9, 5376
    rng = oracle.Rng(0xE2)
    x = rng.f32_vec(rows * row_len)
    w = rng.f32_vec(row_len)
    y = empty(rows * row_len, torch.float32)
    ctx.rmsnorm(dev(x), None, y, rows, row_len)
    torch.cuda.synchronize()
    _close(host(y), oracle.rmsnorm(x, None, row_len), "weightless")
    for name, p1 in (("rmsnorm_5376_f32", False), ("rmsnorm_5376_plus1_f32", True)):
        k = ctx.load_kernel(name)
        y2 = empty(rows * row_len, torch.float32)
        ctx.dispatch_blocking(k, [sgq.BufferBinding.buffer(0, dev(x)), sgq.BufferBinding.buffer(1, dev(w)),
                                  sgq.BufferBinding.buffer(2, y2)], None, [rows, 1, 1])
        _close(host(y2), oracle.rmsnorm(x, w, row_len, 1e-6, p1), name)


@pytest.mark.parametrize("name,head_dim,rot,n_heads", [
    ("rope_sliding_q", 256, 256, 32), ("rope_sliding_k", 256, 256, 16),
    ("rope_global_q", 512, 128, 32), ("rope_global_k", 512, 128, 4),
    ("rope_hd128_sliding_q", 128, 128, 32), ("rope_hd128_global_k", 128, 32, 16)])
def test_rope_variants_match_oracle(ctx, oracle, name, head_dim, rot, n_heads):
    """Partial rotation pairs (i, i+head_dim/2) over the whole head and leaves
    pairs past rot/2 alone (rope.wgsl:1-25, rope.rs:13-16)."""
    import sgq

    n_tok = 5
    rng = oracle.Rng(0xE3 + head_dim + n_heads)
    x = rng.f32_vec(n_tok * n_heads * head_dim)
    pos = np.array([0, 1, 7, 1000, 123456], np.uint32)
    theta = 1e6 if "global" in name else 1e4
    # the live pairs' table [token × rot/2 × 2]; angles use head_dim in the
    # exponent (rope.rs:27-48)
    cs = oracle.cos_sin_table(pos, head_dim, theta)[:, :rot // 2, :].copy()
    want = oracle.rope(x, head_dim, rot, n_heads, cs)
    tx = dev(x)
    ctx.rope(tx, dev(cs), n_tok, n_heads, head_dim, rot)
    torch.cuda.synchronize()
    _close(host(tx), want, name)
    tx2 = dev(x)
    k = ctx.load_kernel(name if "hd128" in name else name + "_f32")
    ctx.dispatch_blocking(k, [sgq.BufferBinding.buffer(0, tx2), sgq.BufferBinding.buffer(1, dev(cs))],
                          None, [(n_tok * n_heads * rot // 2 + 255) // 256, 1, 1])
    _close(host(tx2), want, name + " dispatch")
    # pairs past the live ones are untouched
    xr = x.reshape(n_tok * n_heads, head_dim)
    gr = host(tx2).reshape(n_tok * n_heads, head_dim)
    half = head_dim // 2
    assert np.array_equal(gr[:, rot // 2:half], xr[:, rot // 2:half])
    assert np.array_equal(gr[:, half + rot // 2:], xr[:, half + rot // 2:])


def test_geglu_and_add_scaled(ctx, oracle):
    import sgq

    n = 21504 * 3 + 17
    rng = oracle.Rng(0xE4)
    g = rng.f32_vec(n) * np.float32(2.0)
    u = rng.f32_vec(n)
    y = empty(n, torch.float32)
    ctx.geglu(dev(g), dev(u), y)
    torch.cuda.synchronize()
    _close(host(y), oracle.geglu(g, u), "geglu")
    k = ctx.load_kernel("geglu_f32")
    y2 = empty(n, torch.float32)
    ctx.dispatch_blocking(k, [sgq.BufferBinding.buffer(0, dev(g)), sgq.BufferBinding.buffer(1, dev(u)),
                              sgq.BufferBinding.buffer(2, y2)], None, [(n + 255) // 256, 1, 1])
    assert torch.equal(y, y2)
    # gelu KATs (reference.rs:561-570) through the kernel
    kg = np.array([1.0, -2.0], np.float32)
    ky = empty(2, torch.float32)
    ctx.geglu(dev(kg), dev(np.ones(2, np.float32)), ky)
    torch.cuda.synchronize()
    assert np.allclose(host(ky), [0.841192, -0.0454023], atol=1e-6)

    a, b = rng.f32_vec(n), rng.f32_vec(n)
    ya = empty(n, torch.float32)
    ctx.add_scaled(dev(a), dev(b), ya, 0.75)
    torch.cuda.synchronize()
    assert np.array_equal(host(ya).view(np.uint32), oracle.add_scaled(a, b, 0.75).view(np.uint32))
    import struct
    k = ctx.load_kernel("add_scaled_f32")
    yb = empty(n, torch.float32)
    ctx.dispatch_blocking(k, [sgq.BufferBinding.buffer(0, dev(a)), sgq.BufferBinding.buffer(1, dev(b)),
                              sgq.BufferBinding.buffer(2, yb)], struct.pack("<f", 0.75),
                          [(n + 255) // 256, 1, 1])
    assert torch.equal(ya, yb)


def test_elementwise_bit_deterministic(ctx, oracle):
    rows, row_len = 64, 5376
    x = dev(oracle.Rng(0xE5).f32_vec(rows * row_len))
    w = dev(oracle.Rng(0xE6).f32_vec(row_len))
    a, b = empty(rows * row_len, torch.float32), empty(rows * row_len, torch.float32)
    ctx.rmsnorm(x, w, a, rows, row_len)
    ctx.rmsnorm(x, w, b, rows, row_len)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
