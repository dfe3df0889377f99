"""GPU parity: Q8_0-KV attention (libsgq) vs the f64 oracle.

Template: crates/sg-gpu/tests/parity_attn.rs — decode split-K cases
(kv_len, n_splits) = (17,1), (17,4), (1024,8), (3,8), (333,5), (4096,4)
(parity_attn.rs:67-70, :1008), the oracle attention_head on the DEQUANTIZED
cache (parity_attn.rs:1001-1100), bit-determinism for a fixed split count.
Tolerance: fp32 within 1e-3 relative — |err| <= 1e-3*|want| + 1e-4*rms(want)
per element — against the f64 softmax of the same dequantized K/V.
"""
import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host

pytestmark = pytest.mark.gpu

HD = 128


def _cache(oracle, rng, slots, n_kv):
    """A Q8_0 K/V cache from N(0,1)-ish values: (kq, ks, vq, vs, k_deq, v_deq)."""
    k = rng.f32_vec(slots * n_kv * HD)
    v = rng.f32_vec(slots * n_kv * HD)
    ks, kq = oracle.quant_q8_0(k)
    vs, vq = oracle.quant_q8_0(v)
    return kq, ks, vq, vs, oracle.dequant_q8_0(ks, kq), oracle.dequant_q8_0(vs, vq)


def _want(oracle, q, kd, vd, kv_len, n_q, n_kv, scale):
    out = np.empty((n_q, HD), np.float32)
    for h in range(n_q):
        out[h] = oracle.attention_head(q, kd, vd, 0, h, n_q, n_kv, HD, scale, 0, kv_len - 1)
    return out


def _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, splits, scale):
    out = empty(n_q * HD, torch.float32)
    ctx.attn_decode_q8(dev(q), dev(kq), dev(ks), dev(vq), dev(vs), kv_len, n_q, n_kv, out,
                       n_splits=splits, scale=scale)
    torch.cuda.synchronize()
    return host(out).reshape(n_q, HD)


@pytest.mark.parametrize("kv_len,splits", [(17, 1), (17, 4), (1024, 8), (3, 8), (333, 5),
                                           (333, 1), (4096, 4), (1024, 16), (1, 1), (300, 256)])
def test_attn_decode_matches_oracle(ctx, oracle, kv_len, splits):
    print(f"attn decode kv_len={kv_len} splits={splits}", flush=True)
    n_q, n_kv = 32, 16
    rng = oracle.Rng(0xA77 + kv_len + splits)
    kq, ks, vq, vs, kd, vd = _cache(oracle, rng, kv_len, n_kv)
    q = rng.f32_vec(n_q * HD)
    scale = 1.0 / np.sqrt(HD)
    got = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, splits, scale)
    want = _want(oracle, q, kd, vd, kv_len, n_q, n_kv, scale)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, f"decode kv_len={kv_len} splits={splits}")


@pytest.mark.parametrize("kv_len,splits", [(4096, 16), (32768, 32)])
def test_attn_decode_baseline_contexts(ctx, oracle, kv_len, splits):
    """BASELINE config 4 decode contexts (4K, 32K; 32 q / 16 kv heads, hd 128),
    scale 1.0 as the reference pins with QK-norm, checked on all heads."""
    n_q, n_kv = 32, 16
    rng = oracle.Rng(0xA79 + kv_len)
    kq, ks, vq, vs, kd, vd = _cache(oracle, rng, kv_len, n_kv)
    q = rng.f32_vec(n_q * HD) * np.float32(0.1)
    got = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, splits, 1.0)
    want = _want(oracle, q, kd, vd, kv_len, n_q, n_kv, 1.0)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, f"decode ctx {kv_len}")


def test_attn_decode_ring_prefix_and_gqa_1(ctx, oracle):
    """A partially filled ring (kv_len < slots: only the first kv_len slots
    count, attn_decode_sliding.wgsl:15-20) and n_q == n_kv."""
    n_q = n_kv = 8
    slots, kv_len = 1024, 700
    rng = oracle.Rng(0xA7B)
    kq, ks, vq, vs, kd, vd = _cache(oracle, rng, slots, n_kv)
    q = rng.f32_vec(n_q * HD)
    got = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, 16, 0.125)
    want = _want(oracle, q, kd, vd, kv_len, n_q, n_kv, 0.125)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, "ring prefix")


def test_attn_decode_uniform_keys_kat(ctx, oracle):
    """reference.rs:572-586 in spirit: identical keys -> output is the mean of
    the values (exact for values that are multiples of the Q8 step)."""
    n_q, n_kv, kv_len = 4, 2, 64
    k = np.ones(kv_len * n_kv * HD, np.float32)
    v = np.tile(np.arange(kv_len, dtype=np.float32)[:, None], (1, n_kv * HD)).reshape(-1)
    ks, kq = oracle.quant_q8_0(k)
    vs, vq = oracle.quant_q8_0(v)
    q = np.ones(n_q * HD, np.float32)
    got = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, 4, 0.01)
    vd = oracle.dequant_q8_0(vs, vq).reshape(kv_len, n_kv, HD)
    want = vd.astype(np.float64).mean(axis=0)[0, 0]
    assert np.allclose(got, want, rtol=1e-5)


def test_attn_decode_bit_deterministic(ctx, oracle):
    """Same split count twice -> identical bits (parity_attn.rs:1102-1206);
    another split count agrees to rounding."""
    n_q, n_kv, kv_len = 32, 16, 2000
    rng = oracle.Rng(0xA7C)
    kq, ks, vq, vs, kd, vd = _cache(oracle, rng, kv_len, n_kv)
    q = rng.f32_vec(n_q * HD)
    a = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, 32, 0.1)
    b = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, 32, 0.1)
    c = _run(ctx, q, kq, ks, vq, vs, kv_len, n_q, n_kv, 7, 0.1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.allclose(a, c, rtol=1e-5, atol=1e-6)


def test_attn_decode_128k_sampled_heads(ctx, oracle):
    """BASELINE config 4 at its longest context, 131072 slots (570 MB of Q8_0
    K/V, generated and quantized on the device: the quantizer is bit-exact
    against the oracle), 256 splits, scale 1.0; every head computed, six
    heads (spanning both q heads of a kv head and the first/last kv head)
    checked against the f64 oracle over the dequantized cache."""
    n_q, n_kv, kv_len, splits = 32, 16, 131072, 256
    print(f"attn decode 128K kv_len={kv_len} splits={splits}", flush=True)
    n = kv_len * n_kv * HD
    kv = []
    for seed in (0x128A, 0x128B):
        x = empty(n, torch.float32)
        ctx.fill_normal(x, seed=seed)
        s = empty(n // 32, torch.int16)
        qn = empty(n, torch.int8)
        ctx.quant_q8_0(x, s, qn)
        del x
        kv += [qn, s]
    kq, ks, vq, vs = kv
    rng = oracle.Rng(0x128C)
    q = rng.f32_vec(n_q * HD) * np.float32(0.1)
    out = empty(n_q * HD, torch.float32)
    ctx.attn_decode_q8(dev(q), kq, ks, vq, vs, kv_len, n_q, n_kv, out, n_splits=splits, scale=1.0)
    torch.cuda.synchronize()
    got = host(out).reshape(n_q, HD)
    assert np.isfinite(got).all()
    kd = oracle.dequant_q8_0(host(ks, np.uint16), host(kq))
    vd = oracle.dequant_q8_0(host(vs, np.uint16), host(vq))
    heads = [0, 1, 14, 15, 30, 31]
    want = np.stack([oracle.attention_head(q, kd, vd, 0, h, n_q, n_kv, HD, 1.0, 0, kv_len - 1)
                     for h in heads])
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got[heads], want, 1e-3, 1e-4 * rms, "decode 128K")
