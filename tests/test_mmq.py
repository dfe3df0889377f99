"""GPU parity: Q4_0×Q8 int8-MFMA GEMM (libsgq) vs the f64 MMQ oracle.

Template: crates/sg-gpu/tests/parity_mmq.rs:190-294 (seeded inputs,
mmq_q4_0_q8 f64 oracle) and :296-448 (variant-vs-variant cross-checks).
Bars: every per-block i32 dot is exact by construction of the check below
(an integer-scaled tile must come out as exact integers); fp32 outputs within
1e-3 relative (|err| <= 1e-3*|want| + 1e-4*rms) and normwise <= 2e-6; split-K
equals split 1 within fp32 reassociation (normwise <= 4e-6).
"""
import struct

import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host, rel_err

pytestmark = pytest.mark.gpu


def _quant_on_gpu(ctx, x_t, m, k):
    xs = empty(m * k // 32, torch.int16)
    xq = empty(m * k, torch.int8)
    ctx.quant_q8_0(x_t, xs, xq)
    return xq, xs


def _check_pairs(oracle, w, xq, xs, y, k, ms, ns, what):
    want = oracle.mmq_pairs(w, xq, xs, k, ms, ns)
    got = y[ms, ns]
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, what)
    assert rel_err(got, want) <= 2e-6, (what, rel_err(got, want))


@pytest.mark.parametrize("m,k,n", [(16, 512, 64), (64, 512, 128), (130, 1024, 200),
                                   (1, 256, 33), (257, 2048, 129)])
def test_mmq_small_full_check(ctx, oracle, m, k, n):
    """Every output element vs the oracle on small and ragged shapes
    (parity_mmq.rs seeds 0x4D/0x5E style inputs)."""
    print(f"mmq small m={m} k={k} n={n}", flush=True)
    rng = oracle.Rng(0x4D + m + n)
    w = rng.random_q4_0(n * k // 32)
    x = oracle.through_f16(rng.f32_vec(m * k))
    xq_t, xs_t = _quant_on_gpu(ctx, dev(x), m, k)
    y = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(dev(w), xq_t, xs_t, y, m, n, k)
    torch.cuda.synchronize()
    xs, xq = oracle.quant_q8_0(x)
    assert np.array_equal(host(xs_t, np.uint16), xs.reshape(-1))
    assert np.array_equal(host(xq_t), xq.reshape(-1))
    want = oracle.mmq_q4_0_q8(w, x, m, k, n)
    got = host(y).reshape(m, n)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, f"mmq {m}x{k}x{n}")
    assert rel_err(got, want) <= 2e-6


def test_mmq_integer_tile_is_exact(ctx, oracle):
    """coop_i8_smoke (crates/sg-gpu/tests/coop_i8_smoke.rs) inputs
    a[i][k] = (i+k)%7-3, b[k][j] = (k*j)%11-5 on a 16×16×16 tile, padded to
    K=64 with zeros, all scales 1.0: the GEMM must return the exact integer
    product — this pins the MFMA operand layout and the i32 block dots."""
    M = N = 16
    K = 64
    a = np.zeros((M, K), np.int64)
    b = np.zeros((K, N), np.int64)
    for i in range(16):
        for kk in range(16):
            a[i, kk] = (i + kk) % 7 - 3
            b[kk, i] = (kk * i) % 11 - 5
    want = a @ b
    # weights: row j of W is column j of b, as Q4_0 nibbles (q = b + 8), d = 1
    w = np.zeros((N, K // 32, 18), np.uint8)
    one = np.array([1.0], np.float16).view(np.uint8)
    for j in range(N):
        for blk in range(K // 32):
            w[j, blk, 0:2] = one
            q = [int(b[blk * 32 + t, j]) + 8 for t in range(32)]
            w[j, blk, 2:] = [q[t] | (q[t + 16] << 4) for t in range(16)]
    xs = np.full(M * K // 32, np.array([1.0], np.float16).view(np.uint16)[0], np.uint16)
    y = empty(M * N, torch.float32)
    ctx.gemm_q4_0_q8(dev(w.reshape(-1)), dev(a.astype(np.int8).reshape(-1)), dev(xs), y, M, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(host(y).reshape(M, N), want.astype(np.float32))


def test_mmq_config2_sampled(ctx, oracle):
    """BASELINE config 2 (M=512, K=5376, N=21504), its distribution generated on
    the device, Q8 activations from the device quantizer (checked bit-exact),
    ~2000 sampled outputs vs the f64 oracle."""
    m, k, n = 512, 5376, 21504
    tw = empty(n * k // 32 * 18, torch.uint8)
    ctx.fill_q4_0_random(tw, n * k // 32, seed=21, sigma=0.02)
    tx = empty(m * k, torch.float32)
    ctx.fill_normal(tx, seed=22)
    xq_t, xs_t = _quant_on_gpu(ctx, tx, m, k)
    y = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, y, m, n, k)
    torch.cuda.synchronize()
    w, xq, xs = host(tw), host(xq_t), host(xs_t, np.uint16)
    s2, q2 = oracle.quant_q8_0(host(tx))
    assert np.array_equal(xs, s2.reshape(-1)) and np.array_equal(xq, q2.reshape(-1))
    g = np.random.default_rng(5)
    ms = np.concatenate([g.integers(0, m, 2000), [0, m - 1, 511, 0]])
    ns = np.concatenate([g.integers(0, n, 2000), [0, n - 1, 0, n - 1]])
    _check_pairs(oracle, w, xq, xs, host(y).reshape(m, n), k, ms, ns, "config 2")


@pytest.mark.parametrize("split", [1, 2, 4, 8])
def test_mmq_splitk_down_proj(ctx, oracle, split):
    """BASELINE config 3 shape family (K=21504, N=5376; M=256 to bound test
    time), X = gelu(N(0,1))*N(0,1) → Q8: split-K 1/2/4/8 vs split 1
    (normwise <= 4e-6) and sampled outputs vs the oracle."""
    print(f"mmq split-K {split}", flush=True)
    m, k, n = 256, 21504, 5376
    tw = empty(n * k // 32 * 18, torch.uint8)
    ctx.fill_q4_0_random(tw, n * k // 32, seed=31, sigma=0.02)
    g = empty(m * k, torch.float32)
    u = empty(m * k, torch.float32)
    ctx.fill_normal(g, seed=32)
    ctx.fill_normal(u, seed=33)
    x = (torch.nn.functional.gelu(g, approximate="tanh") * u).contiguous()
    xq_t, xs_t = _quant_on_gpu(ctx, x, m, k)
    y1 = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, y1, m, n, k)
    ys = empty(m * n, torch.float32)
    part = empty(split * m * n, torch.float32) if split > 1 else None
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, ys, m, n, k, split, part)
    ys2 = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, ys2, m, n, k, split, part)
    torch.cuda.synchronize()
    assert torch.equal(ys, ys2), "split-K result not bit-deterministic"
    assert rel_err(host(ys), host(y1)) <= 4e-6  # fp32 reassociation over 672 blocks
    gen = np.random.default_rng(split)
    ms = gen.integers(0, m, 300)
    ns = gen.integers(0, n, 300)
    _check_pairs(oracle, host(tw), host(xq_t), host(xs_t, np.uint16), host(ys).reshape(m, n), k,
                 ms, ns, f"split {split}")


def test_mmq_name_dispatch_variants(ctx, oracle):
    """gemm_q4_0_i8_swz_m4n1_k{K}_n{N}: bindings (w, x, x_scales, y), groups
    [M/64, N/16]; gemm_q4_0_i8_bb_pfd4: K=21504/N=5376 baked, groups
    [m_pad/64, 336]; both equal the typed entry point bit for bit."""
    import sgq

    m, k, n = 128, 5376, 2048
    rng = oracle.Rng(0x319)
    w = dev(rng.random_q4_0(n * k // 32))
    x = dev(oracle.through_f16(rng.f32_vec(m * k)))
    xq, xs = _quant_on_gpu(ctx, x, m, k)
    ref = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(w, xq, xs, ref, m, n, k)
    kern = ctx.load_kernel("gemm_q4_0_i8_swz_m4n1_k5376_n2048_f32")
    y = empty(m * n, torch.float32)
    B = sgq.BufferBinding.buffer
    ctx.dispatch_blocking(kern, [B(0, w), B(1, xq), B(2, xs), B(3, y)], None, [m // 64, n // 16, 1])
    assert torch.equal(ref, y)

    m, k, n = 64, 21504, 5376
    w = empty(n * k // 32 * 18, torch.uint8)
    ctx.fill_q4_0_random(w, n * k // 32, seed=5, sigma=0.02)
    x = empty(m * k, torch.float32)
    ctx.fill_normal(x, seed=6)
    xq, xs = _quant_on_gpu(ctx, x, m, k)
    ref = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(w, xq, xs, ref, m, n, k)
    down = ctx.load_kernel("gemm_q4_0_i8_bb_pfd4_f32")
    y = empty(m * n, torch.float32)
    ctx.dispatch_blocking(down, [B(0, w), B(1, xq), B(2, xs), B(3, y)], None, [m // 64, 336, 1])
    assert torch.equal(ref, y)
    with pytest.raises(sgq.ValidationError):
        ctx.dispatch(down, [B(0, w), B(1, xq), B(2, xs), B(3, y)], None, [m // 64, 300, 1])


def test_mmq_rejects_bad_split(ctx):
    import sgq

    w = empty(18 * 64, torch.uint8)
    xq = empty(64 * 64, torch.int8)
    xs = empty(64 * 2, torch.int16)
    y = empty(64 * 32, torch.float32)
    with pytest.raises(sgq.ValidationError):
        ctx.gemm_q4_0_q8(w, xq, xs, y, 64, 32, 64, 3, empty(3 * 64 * 32, torch.float32))


@pytest.mark.parametrize("split", [1, 2, 4, 8])
def test_mmq_config3_m2048(ctx, oracle, split):
    """BASELINE config 3 at its stated M=2048 (K=21504, N=5376, X =
    gelu(N(0,1))*N(0,1) -> Q8): split-K 1/2/4/8 against split 1 (normwise
    <= 4e-6, fp32 reassociation) and 400 sampled outputs against the oracle,
    including the four corners."""
    print(f"mmq config 3 M=2048 split {split}", flush=True)
    m, k, n = 2048, 21504, 5376
    tw = empty(n * k // 32 * 18, torch.uint8)
    ctx.fill_q4_0_random(tw, n * k // 32, seed=41, sigma=0.02)
    g = empty(m * k, torch.float32)
    u = empty(m * k, torch.float32)
    ctx.fill_normal(g, seed=42)
    ctx.fill_normal(u, seed=43)
    x = (torch.nn.functional.gelu(g, approximate="tanh") * u).contiguous()
    del g, u
    xq_t, xs_t = _quant_on_gpu(ctx, x, m, k)
    del x
    y1 = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, y1, m, n, k)
    ys = empty(m * n, torch.float32)
    part = empty(split * m * n, torch.float32) if split > 1 else None
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, ys, m, n, k, split, part)
    torch.cuda.synchronize()
    assert rel_err(host(ys), host(y1)) <= 4e-6
    gen = np.random.default_rng(100 + split)
    ms = np.concatenate([gen.integers(0, m, 396), [0, 0, m - 1, m - 1]])
    ns = np.concatenate([gen.integers(0, n, 396), [0, n - 1, 0, n - 1]])
    _check_pairs(oracle, host(tw), host(xq_t), host(xs_t, np.uint16), host(ys).reshape(m, n), k,
                 ms, ns, f"config 3 split {split}")


@pytest.mark.parametrize("m,k,n", [(512, 5376, 21504), (2048, 21504, 5376), (768, 5376, 21504)])
def test_mmq_tail_split_matches_plain(ctx, m, k, n):
    """split_k = 1 with a partials buffer: the tiles past the last whole round
    of resident workgroups are split over K and summed in part order (config
    2 and config 3 at split 1 have such a part-filled round; M=768 has none
    to split).  Every output written (the buffer starts as NaN), equal to the
    unsplit call up to the K reassociation of the tail tiles."""
    print(f"mmq tail split m={m} k={k} n={n}", flush=True)
    tw = empty(n * k // 32 * 18, torch.uint8)
    ctx.fill_q4_0_random(tw, n * k // 32, seed=31, sigma=0.02)
    tx = empty(m * k, torch.float32)
    ctx.fill_normal(tx, seed=32)
    xq_t, xs_t = _quant_on_gpu(ctx, tx, m, k)
    y0 = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, y0, m, n, k)
    y1 = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
    part = empty(m * n, torch.float32)
    ctx.gemm_q4_0_q8(tw, xq_t, xs_t, y1, m, n, k, 1, part)
    torch.cuda.synchronize()
    a, b = host(y0), host(y1)
    assert np.isfinite(b).all(), "tail split left outputs unwritten"
    top = float(np.abs(a).max())
    assert np.abs(a - b).max() <= 2e-6 * top, f"max diff {np.abs(a - b).max()} vs {top}"
    # whole tiles are bit-identical; only the tail tiles (< 1 round) may differ
    assert np.count_nonzero(a != b) <= 512 * 128 * 128
