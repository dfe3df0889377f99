"""GPU parity: prefill flash attention over a Q8_0 cache vs the f64 oracle.

Template: crates/sg-gpu/tests/parity_attn.rs (prefill cases, q0 in {0, 200},
causal and sliding, oracle attention_head with t0 = 0 or the window start,
parity_attn.rs:688-784) and BASELINE config 4 (4096 queries, 32 q / 16 kv
heads, hd 128, causal and sliding-1024).  The oracle attends the exactly
dequantized K/V in f64; the kernel rounds K, V, q and P to f16 (as the
reference's f16 PV path does: 2^-12 relative each), which leaves up to ~1e-3
absolute on queries that see only a few keys of magnitude ~2.  The bar is
1e-3 relative to the output scale: normwise max|err|/max|want| <= 1e-3, and
elementwise |err| <= 2e-3*|want| + 1e-3*max|want| (the reference's own
prefill tolerance was 1e-2).
"""
import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host, rel_err

pytestmark = pytest.mark.gpu

HD = 128


def _case(oracle, seed, n_slots, n_kv, n_tok, n_q, qscale=1.0):
    rng = oracle.Rng(seed)
    k = rng.f32_vec(n_slots * n_kv * HD)
    v = rng.f32_vec(n_slots * n_kv * HD)
    ks, kq = oracle.quant_q8_0(k)
    vs, vq = oracle.quant_q8_0(v)
    q = rng.f32_vec(n_tok * n_q * HD) * np.float32(qscale)
    return q, kq, ks, vq, vs, oracle.dequant_q8_0(ks, kq), oracle.dequant_q8_0(vs, vq)


def _run(ctx, q, kq, ks, vq, vs, n_tok, q0, n_q, n_kv, window, scale):
    out = empty(n_tok * n_q * HD, torch.float32)
    ctx.attn_prefill_q8(dev(q), dev(kq), dev(ks), dev(vq), dev(vs), n_tok, q0, n_q, n_kv, out,
                        window=window, scale=scale)
    torch.cuda.synchronize()
    return host(out).reshape(n_tok, n_q, HD)


def _want_rows(oracle, q, kd, vd, rows, q0, n_q, n_kv, window, scale):
    out = np.empty((len(rows), n_q, HD), np.float32)
    for r, i in enumerate(rows):
        p = q0 + i
        t0 = max(0, p + 1 - window) if window else 0
        for h in range(n_q):
            out[r, h] = oracle.attention_head(q, kd, vd, i, h, n_q, n_kv, HD, scale, t0, p)
    return out


def _check(got, want, what):
    top = float(np.abs(want).max())
    assert_close(got, want, 2e-3, 1e-3 * top, what)
    assert rel_err(got, want) <= 1e-3, (what, rel_err(got, want))


@pytest.mark.parametrize("n_tok,q0,window,n_q,n_kv", [
    (1, 0, 0, 32, 16), (37, 0, 0, 32, 16), (128, 0, 0, 32, 16), (300, 0, 0, 32, 16),
    (130, 200, 0, 32, 16), (200, 0, 64, 32, 16), (150, 100, 64, 8, 8), (257, 31, 100, 4, 2)])
def test_attn_prefill_matches_oracle(ctx, oracle, n_tok, q0, window, n_q, n_kv):
    print(f"prefill attn n_tok={n_tok} q0={q0} window={window} heads={n_q}/{n_kv}", flush=True)
    scale = 1.0 / np.sqrt(HD)
    q, kq, ks, vq, vs, kd, vd = _case(oracle, 0xF1A5 + n_tok + q0 + window, q0 + n_tok, n_kv,
                                      n_tok, n_q)
    got = _run(ctx, q, kq, ks, vq, vs, n_tok, q0, n_q, n_kv, window, scale)
    rows = list(range(n_tok))
    want = _want_rows(oracle, q, kd, vd, rows, q0, n_q, n_kv, window, scale)
    _check(got, want, f"prefill n_tok={n_tok} q0={q0} w={window}")


@pytest.mark.parametrize("window", [0, 1024])
def test_attn_prefill_config4_sampled(ctx, oracle, window):
    """BASELINE config 4 prefill: 4096 queries, 32 q / 16 kv, causal and
    sliding-1024; sampled query rows (all heads) against the oracle."""
    n_tok, n_q, n_kv = 4096, 32, 16
    print(f"prefill attn config 4 window={window}", flush=True)
    scale = 1.0 / np.sqrt(HD)
    q, kq, ks, vq, vs, kd, vd = _case(oracle, 0xC0F4 + window, n_tok, n_kv, n_tok, n_q)
    got = _run(ctx, q, kq, ks, vq, vs, n_tok, 0, n_q, n_kv, window, scale)
    rows = [0, 1, 63, 127, 128, 1023, 1024, 1025, 2047, 3000, 4094, 4095]
    want = _want_rows(oracle, q, kd, vd, rows, 0, n_q, n_kv, window, scale)
    _check(got[rows], want, f"config 4 w={window}")
    assert np.isfinite(got).all()


def test_attn_prefill_kats(ctx, oracle):
    """reference.rs:572-596: identical keys -> each query's output is the
    mean of the values it sees; window 2 -> mean of the last two values."""
    n_tok, n_q, n_kv = 40, 2, 1
    k = np.zeros(n_tok * HD, np.float32)
    v = np.tile(np.arange(n_tok, dtype=np.float32)[:, None] * 0.25, (1, HD)).reshape(-1)
    ks, kq = oracle.quant_q8_0(k)
    vs, vq = oracle.quant_q8_0(v)
    q = np.ones(n_tok * n_q * HD, np.float32)
    vd = oracle.dequant_q8_0(vs, vq).reshape(n_tok, HD)[:, 0].astype(np.float64)
    for window in (0, 2):
        got = _run(ctx, q, kq, ks, vq, vs, n_tok, 0, n_q, n_kv, window, 0.1)
        for i in range(n_tok):
            lo = max(0, i + 1 - window) if window else 0
            want = vd[lo:i + 1].mean()
            assert np.allclose(got[i], want, rtol=2e-3, atol=1e-3), (window, i)


def test_attn_prefill_is_bit_deterministic(ctx, oracle):
    n_tok, n_q, n_kv = 300, 8, 4
    q, kq, ks, vq, vs, _, _ = _case(oracle, 0xDE7, n_tok, n_kv, n_tok, n_q)
    a = _run(ctx, q, kq, ks, vq, vs, n_tok, 0, n_q, n_kv, 0, 0.1)
    b = _run(ctx, q, kq, ks, vq, vs, n_tok, 0, n_q, n_kv, 0, 0.1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("hd,n_tok,q0,window,n_q,n_kv", [
    (256, 1, 0, 0, 32, 16), (256, 300, 0, 0, 32, 16), (256, 150, 77, 64, 32, 16),
    (256, 200, 0, 100, 4, 2), (512, 1, 0, 0, 32, 4), (512, 130, 0, 0, 32, 4),
    (512, 100, 41, 0, 32, 4), (512, 70, 5, 33, 8, 1)])
def test_attn_prefill_wide_head_dims_match_oracle(ctx, oracle, hd, n_tok, q0, window, n_q, n_kv):
    """head_dim 256 / 512 (the released checkpoint's sliding and global
    layers: 32 q heads over 16 kv heads of 256, or over 4 kv heads of 512),
    every row and head against the f64 oracle at the same bar."""
    print(f"prefill attn hd={hd} n_tok={n_tok} q0={q0} window={window} heads={n_q}/{n_kv}",
          flush=True)
    rng = oracle.Rng(0xD1DE + hd + n_tok + q0 + window)
    n_slots = q0 + n_tok
    k = rng.f32_vec(n_slots * n_kv * hd)
    v = rng.f32_vec(n_slots * n_kv * hd)
    ks, kq = oracle.quant_q8_0(k)
    vs, vq = oracle.quant_q8_0(v)
    q = rng.f32_vec(n_tok * n_q * hd)
    kd, vd = oracle.dequant_q8_0(ks, kq), oracle.dequant_q8_0(vs, vq)
    scale = 1.0 / np.sqrt(hd)
    out = empty(n_tok * n_q * hd, torch.float32)
    ctx.attn_prefill_q8(dev(q), dev(kq), dev(ks), dev(vq), dev(vs), n_tok, q0, n_q, n_kv, out,
                        window=window, scale=scale, head_dim=hd)
    torch.cuda.synchronize()
    got = host(out).reshape(n_tok, n_q, hd)
    want = np.empty_like(got)
    for i in range(n_tok):
        p = q0 + i
        t0 = max(0, p + 1 - window) if window else 0
        for h in range(n_q):
            want[i, h] = oracle.attention_head(q, kd, vd, i, h, n_q, n_kv, hd, scale, t0, p)
    _check(got, want, f"prefill hd={hd} n_tok={n_tok} q0={q0} w={window}")
