"""GPU parity: int8 PV with key-blocked V (scope row f4) against the oracle.

Template: crates/sg-gpu/tests/parity_attn.rs:786-887 (attn_prefill_global_
flash_sp_ipv: q0 in {0, 200}, Q8 K, key-blocked V from q8_quant_v) and
:964-999 (the V quant layout).
- kv_append_v_q8: bit-exact against the oracle's restatement of
  kv_append_global_v_q8.wgsl (scales and quants), typed and by name.
- attn_prefill_ipv: against oracle.attention_head_ipv, which models the
  kernel's P quantization (per query and 32-key block, denominator over the
  dequantized P) on the dequantized K and key-blocked V.  The kernel rounds q
  and K to f16 for QK (as the f16-PV prefill) and quantizes P against the
  running max (the oracle: the final max), so a block's f16 P scale may round
  differently (2^-11): bar |err| <= 2e-3*|want| + 2e-3*max|want| and
  normwise 2e-3, with the oracle's q (times scale·log2(e), the kernel's
  score units) and K rounded to f16 as the kernel's QK operands are (P's
  quantization turns score noise into whole steps).  Against the full-precision softmax the P quantization
  itself costs up to ~1/127 of max|v| (the reference bounds its own kernel
  at 4e-2 absolute); that error is printed, not asserted.
"""
import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host, rel_err, zeros_synced

pytestmark = pytest.mark.gpu

HD = 128


def _cache(oracle, seed, slots, n_kv):
    rng = oracle.Rng(seed)
    k = rng.f32_vec(slots * n_kv * HD)
    v = rng.f32_vec(slots * n_kv * HD)
    ks, kq = oracle.quant_q8_0(k)
    row = n_kv * HD
    vq = np.zeros(slots * row, np.int8)
    vs = np.zeros(((slots + 31) // 32) * row, np.uint16)
    oracle.kv_append_v_q8(v, slots, row, 0, vq, vs)
    kd = oracle.dequant_q8_0(ks, kq)
    vd = oracle.dequant_v_keyblocked(vq, vs, slots, row)
    return rng, kq, ks, vq, vs, kd, vd


def test_kv_append_v_q8_bit_exact(ctx, oracle):
    import sgq

    row, n_tok, pos, slots = 2048, 45, 64, 160
    src = oracle.Rng(0xA75).f32_vec(n_tok * row)
    wq = np.zeros(slots * row, np.int8)
    ws = np.zeros((slots // 32) * row, np.uint16)
    oracle.kv_append_v_q8(src, n_tok, row, pos, wq, ws)
    tq = zeros_synced(slots * row, torch.int8)
    ts = zeros_synced((slots // 32) * row, torch.int16)
    ctx.kv_append_v_q8(dev(src), n_tok, row, pos, tq, ts)
    torch.cuda.synchronize()
    assert np.array_equal(host(ts, np.uint16), ws)
    assert np.array_equal(host(tq), wq)
    # by name, pos from the step buffer
    tq.zero_()
    ts.zero_()
    step = zeros_synced(8, torch.int32)
    ctx.step_write(step, sgq.StepState(pos, 0, 0, 0))
    k = ctx.load_kernel("kv_append_global_v_q8_f32")
    B = sgq.BufferBinding.buffer
    ctx.dispatch_blocking(k, [B(0, dev(src)), B(1, ts), B(2, tq), B(3, step)], None,
                          [(n_tok + 31) // 32 * row // 256, 1, 1])
    assert np.array_equal(host(ts, np.uint16), ws)
    assert np.array_equal(host(tq), wq)
    with pytest.raises(sgq.ValidationError):
        ctx.kv_append_v_q8(dev(src), n_tok, row, 17, tq, ts)  # pos not a multiple of 32


def _want(oracle, q, kd, vd, rows, q0, n_q, n_kv, scale, ipv=True):
    """The int8-PV oracle on the operands of the kernel's QK: q and the
    dequantized K rounded to f16 (the kernel's f16 MFMA inputs).  P's
    quantization turns score noise into whole quantization steps, so the
    oracle must see the same scores, not just close ones."""
    f = oracle.attention_head_ipv if ipv else oracle.attention_head
    if ipv:
        # the kernel rounds q·scale·log2(e) to f16 (its scores are in log2
        # units); the same rounding, undone in f32, gives the oracle its q
        c = np.float32(scale) * np.float32(1.44269504088896341)
        q = (oracle.through_f16(np.asarray(q, np.float32) * c) / c).astype(np.float32)
        kd = oracle.through_f16(kd)
    out = np.empty((len(rows), n_q, HD), np.float32)
    for r, i in enumerate(rows):
        for h in range(n_q):
            out[r, h] = f(q, kd, vd, i, h, n_q, n_kv, HD, scale, 0, q0 + i)
    return out


def _run(ctx, q, kq, ks, vq, vs, n_tok, q0, n_q, n_kv, scale):
    out = empty(n_tok * n_q * HD, torch.float32)
    ctx.attn_prefill_ipv(dev(q), dev(kq), dev(ks), dev(vq), dev(vs), n_tok, q0, n_q, n_kv, out,
                         scale=scale)
    torch.cuda.synchronize()
    return host(out).reshape(n_tok, n_q, HD)


def _check(got, want, what):
    top = float(np.abs(want).max())
    assert_close(got, want, 2e-3, 2e-3 * top, what)
    assert rel_err(got, want) <= 2e-3, (what, rel_err(got, want))


@pytest.mark.parametrize("n_tok,q0,n_q,n_kv", [(1, 0, 32, 16), (37, 0, 32, 16), (300, 0, 32, 16),
                                               (64, 200, 32, 16), (130, 200, 8, 8),
                                               (257, 31, 4, 2)])
def test_attn_prefill_ipv_matches_oracle(ctx, oracle, n_tok, q0, n_q, n_kv):
    print(f"prefill ipv n_tok={n_tok} q0={q0} heads={n_q}/{n_kv}", flush=True)
    scale = 1.0 / np.sqrt(HD)
    rng, kq, ks, vq, vs, kd, vd = _cache(oracle, 0x1B7 + n_tok + q0, q0 + n_tok, n_kv)
    q = rng.f32_vec(n_tok * n_q * HD)
    got = _run(ctx, q, kq, ks, vq, vs, n_tok, q0, n_q, n_kv, scale)
    rows = list(range(n_tok))
    want = _want(oracle, q, kd, vd, rows, q0, n_q, n_kv, scale)
    _check(got, want, f"ipv n_tok={n_tok} q0={q0}")
    exact = _want(oracle, q, kd, vd, rows[:8], q0, n_q, n_kv, scale, ipv=False)
    print(f"  vs full-precision P: max abs {np.abs(got[:8] - exact).max():.2e} "
          f"(max|v| {np.abs(vd).max():.2f})", flush=True)


def test_attn_prefill_ipv_config4_sampled_and_by_name(ctx, oracle):
    """BASELINE config 4 causal prefill (4096 queries, 32 q / 16 kv) with int8
    PV, sampled rows against the oracle; the registry name with q0 from the
    step buffer equals the typed entry point bit for bit."""
    import struct

    import sgq

    n_tok, n_q, n_kv = 4096, 32, 16
    print("prefill ipv config 4", flush=True)
    scale = 1.0 / np.sqrt(HD)
    rng, kq, ks, vq, vs, kd, vd = _cache(oracle, 0xC0F5, n_tok, n_kv)
    q = rng.f32_vec(n_tok * n_q * HD)
    got = _run(ctx, q, kq, ks, vq, vs, n_tok, 0, n_q, n_kv, scale)
    rows = [0, 1, 31, 32, 63, 127, 128, 1023, 2047, 3000, 4095]
    _check(got[rows], _want(oracle, q, kd, vd, rows, 0, n_q, n_kv, scale), "ipv config 4")
    k = ctx.load_kernel("attn_prefill_global_flash_ipv_hd128")
    out = empty(n_tok * n_q * HD, torch.float32)
    step = zeros_synced(8, torch.int32)
    ctx.step_write(step, sgq.StepState(0, 0, 0, 0))
    B = sgq.BufferBinding.buffer
    ctx.dispatch_blocking(k, [B(0, dev(q)), B(1, dev(kq)), B(2, dev(ks)), B(3, dev(vq)),
                              B(4, dev(vs)), B(5, out), B(6, step)],
                          struct.pack("<f", scale), [n_q, n_tok // 16, 1])
    assert np.array_equal(host(out).reshape(n_tok, n_q, HD).view(np.uint32), got.view(np.uint32))
