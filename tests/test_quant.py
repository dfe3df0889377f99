"""GPU parity: Q8_0 quantization, dequantization and KV append vs the oracle.

Template: crates/sg-gpu/tests/parity_kv.rs:131-212.  The reference allows
quants to differ by ±1 (its GPU reciprocal is 2.5 ulp); libsgq uses an
IEEE-correct reciprocal, so scales AND quants are required bit-exact.
"""
import numpy as np
import pytest
import torch

from _util import dev, empty, host, zeros_synced

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [32, 4096 + 256, 512 * 5376])
def test_quant_q8_0_bit_exact(ctx, oracle, n):
    print(f"quant n={n}", flush=True)
    x = oracle.through_f16(oracle.Rng(0xB2).f32_vec(n))
    if n > 96:
        x[64:96] = 0.0  # an all-zero block: d = 0, id = 0 path
    s_want, q_want = oracle.quant_q8_0(x)
    ts, tq = empty(n // 32, torch.int16), empty(n, torch.int8)
    ctx.quant_q8_0(dev(x), ts, tq)
    torch.cuda.synchronize()
    assert np.array_equal(host(ts, np.uint16), s_want), "f16 scales differ"
    assert np.array_equal(host(tq), q_want), "quants differ"


def test_quant_q8_0_geglu_distribution_full_size(ctx, oracle):
    """BASELINE config 3 activations (gelu(N(0,1))*N(0,1), 2048×21504): bit-exact."""
    m, k = 2048, 21504
    g = empty(m * k, torch.float32)
    u = empty(m * k, torch.float32)
    ctx.fill_normal(g, seed=7)
    ctx.fill_normal(u, seed=8)
    x = (torch.nn.functional.gelu(g, approximate="tanh") * u).contiguous()
    ts, tq = empty(m * k // 32, torch.int16), empty(m * k, torch.int8)
    ctx.quant_q8_0(x, ts, tq)
    torch.cuda.synchronize()
    s_want, q_want = oracle.quant_q8_0(host(x))
    assert np.array_equal(host(ts, np.uint16), s_want)
    assert np.array_equal(host(tq), q_want)


def test_dequant_q8_0_exact(ctx, oracle):
    n = 8192
    x = oracle.Rng(0xB3).f32_vec(n)
    s, q = oracle.quant_q8_0(x)
    out = empty(n, torch.float32)
    ctx.dequant_q8_0(dev(s), dev(q), out)
    torch.cuda.synchronize()
    assert np.array_equal(host(out), oracle.dequant_q8_0(s, q))


def test_quant_is_bit_deterministic(ctx, oracle):
    x = dev(oracle.Rng(0xB4).f32_vec(1 << 16))
    a = (empty(1 << 11, torch.int16), empty(1 << 16, torch.int8))
    b = (empty(1 << 11, torch.int16), empty(1 << 16, torch.int8))
    ctx.quant_q8_0(x, *a)
    ctx.quant_q8_0(x, *b)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_kv_quant_q8_name_dispatch(ctx, oracle):
    """kv_quant_q8 through load_kernel/dispatch: bindings (src, scales,
    quants), blocks = arrayLength(src)/32 (kv_quant_q8.wgsl:30-35)."""
    import sgq

    n = 2048 + 64
    x = oracle.Rng(0xB5).f32_vec(n)
    s_want, q_want = oracle.quant_q8_0(x)
    kern = ctx.load_kernel("kv_quant_q8_f32")
    ts, tq = empty(n // 32, torch.int16), empty(n, torch.int8)
    ctx.dispatch_blocking(kern, [sgq.BufferBinding.buffer(0, dev(x)), sgq.BufferBinding.buffer(1, ts),
                                 sgq.BufferBinding.buffer(2, tq)], None, kern.groups_for(n // 32))
    assert np.array_equal(host(ts, np.uint16), s_want)
    assert np.array_equal(host(tq), q_want)


def test_kv_append_global_q8_places_rows_at_pos(ctx, oracle):
    """kv_append_global_q8 (kv_append_global_q8.wgsl:29-60): rows land at
    slot pos+t, untouched slots keep their contents."""
    import sgq

    row, n_tok, pos, slots = 2048, 3, 5, 12
    x = oracle.Rng(0xB6).f32_vec(n_tok * row)
    s_want, q_want = oracle.quant_q8_0(x)
    scales = torch.full((slots * row // 32,), 7, dtype=torch.int16, device="cuda")
    quants = torch.full((slots * row,), 3, dtype=torch.int8, device="cuda")
    step = zeros_synced(4, torch.int32)
    ctx.step_write(step, sgq.StepState(pos=pos, kv_len_sliding=0, kv_len_global=pos + n_tok, q0=pos))
    kern = ctx.load_kernel("kv_append_global_q8_f32")
    ctx.dispatch_blocking(kern, [sgq.BufferBinding.buffer(0, dev(x)), sgq.BufferBinding.buffer(1, scales),
                                 sgq.BufferBinding.buffer(2, quants), sgq.BufferBinding.buffer(3, step)],
                          None, [n_tok * row // 32 // 64 + 1, row // 32, 1])
    hs = host(scales, np.uint16).reshape(slots, row // 32)
    hq = host(quants).reshape(slots, row)
    assert list(host(step)) == [pos, 0, pos + n_tok, pos]
    assert np.array_equal(hs[pos:pos + n_tok].reshape(-1), s_want)
    assert np.array_equal(hq[pos:pos + n_tok].reshape(-1), q_want)
    assert (hs[:pos] == 7).all() and (hs[pos + n_tok:] == 7).all()
    assert (hq[:pos] == 3).all() and (hq[pos + n_tok:] == 3).all()
