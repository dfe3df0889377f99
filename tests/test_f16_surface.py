"""GPU parity of the reference's variant names with the reference's own
activation type: f16 in, f16 out (crates/sg-gpu/shaders/gemv_q4_0.wgsl:18-19,
rmsnorm.wgsl:14-16, rope.wgsl:26, geglu.wgsl:7-9, add_scaled.wgsl:12-14,
gemm_q4_0_i8.wgsl:63, kv_quant_q8.wgsl:24-26, kv_dequant_q8.wgsl:9-11,
kv_append_global_q8.wgsl:19-24, kv_append_global_v_q8.wgsl:20-25,
gemv_q6_k_logits.wgsl:18-20).  Every shader widens its f16 inputs, computes
in f32 and rounds the result to f16 once, so the bars are:

- rmsnorm / rope / geglu: within one f16 ulp of the oracle's value on the
  widened inputs (a rounding to nearest of a value the f32 kernel and the
  f64-or-f32 oracle agree on to far below half an ulp, except where the
  exact value sits next to a rounding midpoint), geglu plus the fp32 form's
  absolute 2e-6 of the rms (gelu's 1 + tanh cancels in f32 for negative
  gates);
- add_scaled: bit-exact (the same f32 expression, then RTNE);
- gemv: one f16 ulp plus the limb form's 2e-5 of max |y| (x enters as
  15-bit fixed point per 32-block, as in the fp32 form);
- the int8 GEMMs: bit-exact against the fp32 form's output rounded to f16
  (the same accumulators, rounded in the store);
- Q8_0 quant / append / dequant and the Q6_K logits: bit-exact.
"""
import struct

import numpy as np
import pytest
import torch

from _util import dev, empty, host, sample_rows, zeros_synced

pytestmark = pytest.mark.gpu


def _h(oracle, x):
    """fp32 host values -> (f16 device tensor, the widened fp32 values)."""
    bits = oracle.f32_to_f16_bits(np.asarray(x, np.float32))
    return dev(bits), oracle.f16_bits_to_f32(bits)


def _got(oracle, t):
    return oracle.f16_bits_to_f32(host(t, np.uint16)).astype(np.float64)


def _ulp16(v):
    """Spacing of f16 at |v| (2^-24 below the normal range)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _within_ulps(got, want, what, ulps=1.0, atol=0.0):
    want = np.asarray(want, np.float64)
    err = np.abs(got - want) - ulps * _ulp16(want)
    i = int(np.argmax(err))
    assert err.flat[i] <= atol, (f"{what}: element {i}: got {got.flat[i]!r} "
                                 f"want {want.flat[i]!r}")


def _B(i, t):
    import sgq

    return sgq.BufferBinding.buffer(i, t)


@pytest.mark.parametrize("name,row_len,rows,plus_one", [
    ("rmsnorm_5376", 5376, 3, False), ("rmsnorm_5376_plus1", 5376, 2, True),
    ("rmsnorm_512", 512, 32, False), ("rmsnorm_256", 256, 33, False),
    ("rmsnorm_256_plus1", 256, 16, True)])
def test_rmsnorm_f16(ctx, oracle, name, row_len, rows, plus_one):
    rng = oracle.Rng(0xF1 + row_len + rows)
    tx, x = _h(oracle, rng.f32_vec(rows * row_len) * np.float32(3.0))
    w = rng.f32_vec(row_len)
    y = empty(rows * row_len, torch.int16)
    ctx.dispatch_blocking(ctx.load_kernel(name), [_B(0, tx), _B(1, dev(w)), _B(2, y)], None,
                          [rows, 1, 1])
    _within_ulps(_got(oracle, y), oracle.rmsnorm(x, w, row_len, 1e-6, plus_one), name)


@pytest.mark.parametrize("name,head_dim,rot,n_heads", [
    ("rope_sliding_q", 256, 256, 32), ("rope_sliding_k", 256, 256, 16),
    ("rope_global_q", 512, 128, 32), ("rope_global_k", 512, 128, 4)])
def test_rope_f16_in_place(ctx, oracle, name, head_dim, rot, n_heads):
    n_tok = 3
    rng = oracle.Rng(0xF2 + head_dim + n_heads)
    tx, x = _h(oracle, rng.f32_vec(n_tok * n_heads * head_dim))
    pos = np.array([0, 9, 4097], np.uint32)
    theta = 1e6 if "global" in name else 1e4
    cs = oracle.cos_sin_table(pos, head_dim, theta)[:, :rot // 2, :].copy()
    ctx.dispatch_blocking(ctx.load_kernel(name), [_B(0, tx), _B(1, dev(cs))], None,
                          [(n_tok * n_heads * rot // 2 + 255) // 256, 1, 1])
    got = _got(oracle, tx)
    _within_ulps(got, oracle.rope(x, head_dim, rot, n_heads, cs), name)
    # pairs past the live ones keep their f16 bits
    g = got.reshape(-1, head_dim)
    xr = x.reshape(-1, head_dim)
    half = head_dim // 2
    assert np.array_equal(g[:, rot // 2:half], xr[:, rot // 2:half])


def test_geglu_and_add_scaled_f16(ctx, oracle):
    n = 21504 + 77
    rng = oracle.Rng(0xF3)
    tg, g = _h(oracle, rng.f32_vec(n) * np.float32(2.0))
    tu, u = _h(oracle, rng.f32_vec(n))
    y = empty(n, torch.int16)
    ctx.dispatch_blocking(ctx.load_kernel("geglu"), [_B(0, tg), _B(1, tu), _B(2, y)], None,
                          [(n + 255) // 256, 1, 1])
    want = oracle.geglu(g, u)
    # the f32 tanh of gelu's 1 + tanh(...) cancels for negative gate values:
    # an absolute 2e-6 of the rms, as the fp32 form's bar
    rms = float(np.sqrt(np.mean(np.asarray(want, np.float64) ** 2)))
    _within_ulps(_got(oracle, y), want, "geglu f16", atol=2e-6 * rms)
    ya = empty(n, torch.int16)
    ctx.dispatch_blocking(ctx.load_kernel("add_scaled"), [_B(0, tg), _B(1, tu), _B(2, ya)],
                          struct.pack("<f", 0.8125), [(n + 255) // 256, 1, 1])
    want = oracle.f32_to_f16_bits(oracle.add_scaled(g, u, 0.8125))
    assert np.array_equal(host(ya, np.uint16), want)


@pytest.mark.parametrize("k,n,generic", [(5376, 4096, False), (8192, 1024, False),
                                         (16384, 640, False), (21504, 512, False),
                                         (5376, 700, True), (320, 333, True)])
def test_gemv_q4_0_f16(ctx, oracle, k, n, generic):
    """gemv_q4_0_k{K} and gemv_q4_0_generic (push k) with f16 x and y:
    K = 320 takes the register path (K % 256 != 0), the others the
    streamed one; f16 y equals the fp32 form's y rounded to f16 up to the
    limb form's noise."""
    rng = oracle.Rng(0xF4 + k + n)
    w = rng.random_q4_0(n * k // 32)
    tx, x = _h(oracle, rng.f32_vec(k))
    tw = dev(w)
    y = empty(n, torch.int16)
    if generic:
        kern, push = ctx.load_kernel("gemv_q4_0_generic"), struct.pack("<I", k)
    else:
        kern, push = ctx.load_kernel(f"gemv_q4_0_k{k}"), None
    ctx.dispatch_blocking(kern, [_B(0, tw), _B(1, tx), _B(2, y)], push, [n, 1, 1])
    rows = sample_rows(n)
    want = oracle.gemv_rows(w, x, k, rows)
    got = _got(oracle, y)[rows]
    _within_ulps(got, want, f"gemv f16 k={k}", atol=2e-5 * float(np.abs(want).max()))


def test_gemv_q6_k_logits_f16_x(ctx, oracle):
    """f16 x: the fp32 form rounds x to f16 first, so the two forms agree
    bit for bit on an f16-representable x."""
    n, K, stride = 300, 5376, 4416
    rng = oracle.Rng(0xF5)
    w = dev(rng.random_q6_k_rows(n, K, stride))
    tx, x = _h(oracle, rng.f32_vec(K))
    a, b = empty(n, torch.float32), empty(n, torch.float32)
    ctx.dispatch_blocking(ctx.load_kernel("gemv_q6_k_logits"), [_B(0, w), _B(1, tx), _B(2, a)],
                          None, [n, 1, 1])
    ctx.dispatch_blocking(ctx.load_kernel("gemv_q6_k_logits_f32"),
                          [_B(0, w), _B(1, dev(x)), _B(2, b)], None, [n, 1, 1])
    assert torch.equal(a, b)


def test_gemm_i8_f16_output(ctx, oracle):
    """gemm_q4_0_i8_swz_m4n1_* and gemm_q4_0_i8_bb_pfd4 write f16 y: the
    fp32 form's sums, each rounded to nearest even."""
    B = _B
    m, k, n = 128, 5376, 2048
    rng = oracle.Rng(0xF6)
    w = dev(rng.random_q4_0(n * k // 32))
    x = dev(oracle.through_f16(rng.f32_vec(m * k)))
    xs, xq = empty(m * k // 32, torch.int16), empty(m * k, torch.int8)
    ctx.quant_q8_0(x, xs, xq)
    y32, y16 = empty(m * n, torch.float32), empty(m * n, torch.int16)
    ctx.dispatch_blocking(ctx.load_kernel("gemm_q4_0_i8_swz_m4n1_k5376_n2048_f32"),
                          [B(0, w), B(1, xq), B(2, xs), B(3, y32)], None, [m // 64, n // 16, 1])
    ctx.dispatch_blocking(ctx.load_kernel("gemm_q4_0_i8_swz_m4n1_k5376_n2048"),
                          [B(0, w), B(1, xq), B(2, xs), B(3, y16)], None, [m // 64, n // 16, 1])
    assert np.array_equal(host(y16, np.uint16), oracle.f32_to_f16_bits(host(y32)))

    m, k, n = 64, 21504, 5376
    w = empty(n * k // 32 * 18, torch.uint8)
    ctx.fill_q4_0_random(w, n * k // 32, seed=7, sigma=0.02)
    x = empty(m * k, torch.float32)
    ctx.fill_normal(x, seed=8)
    xs, xq = empty(m * k // 32, torch.int16), empty(m * k, torch.int8)
    ctx.quant_q8_0(x, xs, xq)
    y32, y16 = empty(m * n, torch.float32), empty(m * n, torch.int16)
    ctx.dispatch_blocking(ctx.load_kernel("gemm_q4_0_i8_bb_pfd4_f32"),
                          [B(0, w), B(1, xq), B(2, xs), B(3, y32)], None, [m // 64, 336, 1])
    ctx.dispatch_blocking(ctx.load_kernel("gemm_q4_0_i8_bb_pfd4"),
                          [B(0, w), B(1, xq), B(2, xs), B(3, y16)], None, [m // 64, 336, 1])
    assert np.array_equal(host(y16, np.uint16), oracle.f32_to_f16_bits(host(y32)))


def test_kv_quant_dequant_append_f16(ctx, oracle):
    import sgq

    B = _B
    n = 2048 * 3
    rng = oracle.Rng(0xF7)
    tx, x = _h(oracle, rng.f32_vec(n) * np.float32(4.0))
    s_want, q_want = oracle.quant_q8_0(x)
    ts, tq = empty(n // 32, torch.int16), empty(n, torch.int8)
    kq = ctx.load_kernel("kv_quant_q8")
    ctx.dispatch_blocking(kq, [B(0, tx), B(1, ts), B(2, tq)], None, kq.groups_for(n // 32))
    assert np.array_equal(host(ts, np.uint16), s_want)
    assert np.array_equal(host(tq), q_want)
    # kv_dequant_q8: f16(d·q)
    out = empty(n, torch.int16)
    ctx.dispatch_blocking(ctx.load_kernel("kv_dequant_q8"), [B(0, ts), B(1, tq), B(2, out)], None,
                          [(n // 32 + 63) // 64, 1, 1])
    want = oracle.f32_to_f16_bits(oracle.dequant_q8_0(s_want, q_want))
    assert np.array_equal(host(out, np.uint16), want)
    # kv_append_global_q8: 3 rows of 2048 at slot pos + t
    row, pos, slots = 2048, 4, 9
    scales = torch.full((slots * row // 32,), 7, dtype=torch.int16, device="cuda")
    quants = torch.full((slots * row,), 3, dtype=torch.int8, device="cuda")
    step = zeros_synced(4, torch.int32)
    ctx.step_write(step, sgq.StepState(pos, 0, pos + 3, 0))
    ka = ctx.load_kernel("kv_append_global_q8")
    ctx.dispatch_blocking(ka, [B(0, tx), B(1, scales), B(2, quants), B(3, step)], None,
                          ka.groups_for(3 * row // 32))
    hs = host(scales, np.uint16).reshape(slots, row // 32)
    hq = host(quants).reshape(slots, row)
    assert np.array_equal(hs[pos:pos + 3].reshape(-1), s_want)
    assert np.array_equal(hq[pos:pos + 3].reshape(-1), q_want)
    assert (hs[:pos] == 7).all() and (hq[pos + 3:] == 3).all()
    with pytest.raises(sgq.ValidationError):  # a partial row
        ctx.dispatch(ka, [sgq.BufferBinding(0, tx, 0, row * 2 + 64), B(1, scales), B(2, quants),
                          B(3, step)], None, ka.groups_for(row // 32))


def test_kv_append_global_v_q8_f16(ctx, oracle):
    """Key-blocked V append from f16 rows (kv_append_global_v_q8.wgsl:
    20-75): quants and scales equal the oracle's on the widened rows; a
    source that is not whole rows, or quants too short, is refused."""
    import sgq

    B = _B
    row, n_tok, pos = 2048, 45, 32
    rng = oracle.Rng(0xF8)
    tsrc, src = _h(oracle, rng.f32_vec(n_tok * row))
    slots = pos + 64
    wq = np.zeros(slots * row, np.int8)
    ws = np.zeros(slots // 32 * row, np.uint16)
    oracle.kv_append_v_q8(src, n_tok, row, pos, wq, ws)
    tq, ts = dev(np.zeros_like(wq)), dev(np.zeros_like(ws))
    step = zeros_synced(4, torch.int32)
    ctx.step_write(step, sgq.StepState(pos, 0, 0, 0))
    k = ctx.load_kernel("kv_append_global_v_q8")
    ctx.dispatch_blocking(k, [B(0, tsrc), B(1, ts), B(2, tq), B(3, step)], None,
                          [(n_tok + 31) // 32 * row // 256, 1, 1])
    assert np.array_equal(host(ts, np.uint16), ws)
    assert np.array_equal(host(tq), wq)
    with pytest.raises(sgq.ValidationError):
        ctx.dispatch(k, [sgq.BufferBinding(0, tsrc, 0, row * 2 * 3 + 2), B(1, ts), B(2, tq),
                         B(3, step)], None, [1, 1, 1])
    with pytest.raises(sgq.ValidationError):
        ctx.dispatch(k, [B(0, tsrc), B(1, ts), sgq.BufferBinding(2, tq, 0, row * 10), B(3, step)],
                     None, [1, 1, 1])
