"""GPU parity: the attention / KV-append variants through the name-based
dispatch surface (load_kernel + dispatch with bindings, push constants and the
step buffer), as the reference's record_layer records them
(crates/sg-model/src/graph.rs:560-656), against the typed entry points (bit
for bit) and the f64 oracle.

Geometry baked into the hd128 names: 32 query / 16 kv heads of 128, Q8_0 K
and V pages, window and ring 1024.  Tolerances as the typed tests: decode
|err| <= 1e-3*|want| + 1e-4*rms (tests/test_attn.py), prefill normwise 1e-3
of the output scale (tests/test_prefill_attn.py).
"""
import ctypes as C
import struct

import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host, rel_err, zeros_synced

pytestmark = pytest.mark.gpu

HD, NQ, NKV, RING = 128, 32, 16, 1024


def _bind(sgq, *tensors):
    return [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(tensors)]


def _cache(oracle, seed, slots):
    rng = oracle.Rng(seed)
    k = rng.f32_vec(slots * NKV * HD)
    v = rng.f32_vec(slots * NKV * HD)
    ks, kq = oracle.quant_q8_0(k)
    vs, vq = oracle.quant_q8_0(v)
    return rng, kq, ks, vq, vs, oracle.dequant_q8_0(ks, kq), oracle.dequant_q8_0(vs, vq)


def _step(ctx, pos, kv_sl, kv_gl, q0):
    import sgq

    step = zeros_synced(8, torch.int32)
    ctx.step_write(step, sgq.StepState(pos, kv_sl, kv_gl, q0))
    return step


def _decode_by_name(ctx, kind, q, kq, ks, vq, vs, step, splits, scale):
    import sgq

    attn = ctx.load_kernel(f"attn_decode_{kind}_q8_hd128")
    red = ctx.load_kernel("attn_reduce_d128")
    part = empty(NQ * splits * (HD + 2), torch.float32)
    out = empty(NQ * HD, torch.float32)
    ctx.dispatch(attn, _bind(sgq, q, kq, ks, vq, vs, part, step),
                 struct.pack("<If", splits, scale), [NKV, splits, 1])
    ctx.dispatch_blocking(red, _bind(sgq, part, out), struct.pack("<I", splits), [NQ, 1, 1])
    return out


@pytest.mark.parametrize("kv_len,splits", [(4096, 16), (333, 5), (1, 1), (17, 1), (3000, 64)])
def test_decode_global_by_name_equals_typed_and_oracle(ctx, oracle, kv_len, splits):
    print(f"dispatch attn_decode_global kv_len={kv_len} splits={splits}", flush=True)
    rng, kq, ks, vq, vs, kd, vd = _cache(oracle, 0xD15 + kv_len, kv_len)
    q = rng.f32_vec(NQ * HD)
    scale = 1.0 / np.sqrt(HD)
    tq, tkq, tks, tvq, tvs = dev(q), dev(kq), dev(ks), dev(vq), dev(vs)
    got = host(_decode_by_name(ctx, "global", tq, tkq, tks, tvq, tvs,
                               _step(ctx, kv_len - 1, 0, kv_len, 0), splits, scale))
    typed = empty(NQ * HD, torch.float32)
    ctx.attn_decode_q8(tq, tkq, tks, tvq, tvs, kv_len, NQ, NKV, typed, n_splits=splits,
                       scale=scale)
    torch.cuda.synchronize()
    typed = host(typed)
    if splits > 1:  # same split kernel, same merge
        assert np.array_equal(got.view(np.uint32), typed.view(np.uint32))
    want = np.stack([oracle.attention_head(q, kd, vd, 0, h, NQ, NKV, HD, scale, 0, kv_len - 1)
                     for h in range(NQ)]).reshape(-1)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, "decode by name")


def test_decode_sliding_ring_by_name_and_graph_replay(ctx, oracle):
    """A full 1024-slot ring (kv_len_sliding = step[1] = 1024 at pos 1500):
    softmax over every slot; then the same two dispatches recorded once as a
    graph and replayed with the step buffer rewritten (kv_len 1024 -> 700 ->
    1024), each replay equal to an eager dispatch."""
    import sgq

    rng, kq, ks, vq, vs, kd, vd = _cache(oracle, 0x51D, RING)
    q = rng.f32_vec(NQ * HD)
    tq, tkq, tks, tvq, tvs = dev(q), dev(kq), dev(ks), dev(vq), dev(vs)
    scale = 1.0
    print("dispatch attn_decode_sliding ring", flush=True)
    eager = host(_decode_by_name(ctx, "sliding", tq, tkq, tks, tvq, tvs,
                                 _step(ctx, 1500, RING, 0, 0), 16, scale))
    want = np.stack([oracle.attention_head(q, kd, vd, 0, h, NQ, NKV, HD, scale, 0, RING - 1)
                     for h in range(NQ)]).reshape(-1)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(eager, want, 1e-3, 1e-4 * rms, "sliding ring by name")

    attn = ctx.load_kernel("attn_decode_sliding_q8_hd128")
    red = ctx.load_kernel("attn_reduce_d128")
    step = zeros_synced(8, torch.int32)
    part = empty(NQ * 16 * (HD + 2), torch.float32)
    out = empty(NQ * HD, torch.float32)
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        with sgq.GraphRecorder(ctx) as rec:
            ctx.dispatch(attn, _bind(sgq, tq, tkq, tks, tvq, tvs, part, step),
                         struct.pack("<If", 16, scale), [NKV, 16, 1])
            ctx.dispatch(red, _bind(sgq, part, out), struct.pack("<I", 16), [NQ, 1, 1])
        for kv_sl in (RING, 700, RING):
            ctx.step_write(step, sgq.StepState(1500, kv_sl, 0, 0))
            rec.graph.submit()
            ctx.synchronize()
            got = host(out).copy()
            ref = host(_decode_by_name(ctx, "sliding", tq, tkq, tks, tvq, tvs,
                                       _step(ctx, 1500, kv_sl, 0, 0), 16, scale))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), kv_sl
            torch.randn(1024, device="cuda").sum().item()  # unrelated eager work
    finally:
        ctx.set_stream(None)


def test_fill_zero_refused_while_capturing(ctx):
    import sgq

    buf = torch.ones(64, device="cuda")
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        with pytest.raises(sgq.ValidationError):
            with sgq.GraphRecorder(ctx):
                sgq._check(sgq.lib().sgq_buf_fill_zero(ctx.handle, C.c_void_p(buf.data_ptr()),
                                                      buf.numel() * 4))
        sgq._check(sgq.lib().sgq_buf_fill_zero(ctx.handle, C.c_void_p(buf.data_ptr()),
                                              buf.numel() * 4))
        ctx.synchronize()
    finally:
        ctx.set_stream(None)
    assert float(buf.abs().sum()) == 0.0


@pytest.mark.parametrize("n_tok,q0", [(300, 0), (130, 200)])
def test_prefill_global_flash_by_name_equals_typed(ctx, oracle, n_tok, q0):
    """q0 comes from step[3] on the device; the linear cache holds the chunk."""
    import sgq

    print(f"dispatch attn_prefill_global_flash n_tok={n_tok} q0={q0}", flush=True)
    rng, kq, ks, vq, vs, kd, vd = _cache(oracle, 0xF1 + q0, q0 + n_tok)
    q = rng.f32_vec(n_tok * NQ * HD)
    tq, tkq, tks, tvq, tvs = dev(q), dev(kq), dev(ks), dev(vq), dev(vs)
    scale = 1.0 / np.sqrt(HD)
    k = ctx.load_kernel("attn_prefill_global_flash_q8_hd128")
    out = empty(n_tok * NQ * HD, torch.float32)
    ctx.dispatch_blocking(k, _bind(sgq, tq, tkq, tks, tvq, tvs, out, _step(ctx, 0, 0, 0, q0)),
                          struct.pack("<f", scale), [NQ, (n_tok + 15) // 16, 1])
    typed = empty(n_tok * NQ * HD, torch.float32)
    ctx.attn_prefill_q8(tq, tkq, tks, tvq, tvs, n_tok, q0, NQ, NKV, typed, window=0, scale=scale)
    torch.cuda.synchronize()
    assert np.array_equal(host(out).view(np.uint32), host(typed).view(np.uint32))


def test_prefill_sliding_ring_by_name_matches_oracle(ctx, oracle):
    """Two key ranges: positions before q0 from a full 1024-slot ring (slot =
    pos % 1024, q0 = 1531 > ring), positions from q0 on from the chunk's own
    pages; a 600-token chunk spans several 256-key tiles.  Every row and head
    against the oracle over the position-ordered keys with the window start
    t0 = max(0, p - 1023)."""
    import sgq

    q0, n_tok = 1531, 600
    print(f"dispatch attn_prefill_sliding_ring q0={q0} n_tok={n_tok}", flush=True)
    rng, rkq, rks, rvq, rvs, rkd, rvd = _cache(oracle, 0x7171, RING)
    _, ckq, cks, cvq, cvs, ckd, cvd = _cache(oracle, 0x7272, n_tok)
    q = rng.f32_vec(n_tok * NQ * HD)
    scale = 1.0 / np.sqrt(HD)
    row = NKV * HD
    kd = np.zeros((q0 + n_tok, row), np.float32)
    vd = np.zeros((q0 + n_tok, row), np.float32)
    for p in range(q0 - RING, q0):
        kd[p] = rkd.reshape(RING, row)[p % RING]
        vd[p] = rvd.reshape(RING, row)[p % RING]
    kd[q0:] = ckd.reshape(n_tok, row)
    vd[q0:] = cvd.reshape(n_tok, row)
    k = ctx.load_kernel("attn_prefill_sliding_ring_q8_hd128")
    out = empty(n_tok * NQ * HD, torch.float32)
    ctx.dispatch_blocking(
        k, _bind(sgq, dev(q), dev(rkq), dev(rks), dev(rvq), dev(rvs), dev(ckq), dev(cks),
                 dev(cvq), dev(cvs), out, _step(ctx, q0, 0, 0, q0)),
        struct.pack("<f", scale), [NKV, n_tok, 1])
    got = host(out).reshape(n_tok, NQ, HD)
    kf, vf = kd.reshape(-1), vd.reshape(-1)
    want = np.empty_like(got)
    for i in range(n_tok):
        p = q0 + i
        for h in range(NQ):
            want[i, h] = oracle.attention_head(q, kf, vf, i, h, NQ, NKV, HD, scale,
                                               max(0, p + 1 - RING), p)
    top = float(np.abs(want).max())
    assert_close(got, want, 2e-3, 1e-3 * top, "sliding ring prefill")
    assert rel_err(got, want) <= 1e-3


def test_kv_append_sliding_by_name_wraps_the_ring(ctx, oracle):
    """kv_append_sliding_q8: 5 tokens at step[0] = 1022 land in slots 1022,
    1023, 0, 1, 2 with kv_quant_q8 scales and quants, bit for bit."""
    import sgq

    n_tok = 5
    rng = oracle.Rng(0xA99)
    src = rng.f32_vec(n_tok * NKV * HD)
    s_want, q_want = oracle.quant_q8_0(src)
    scales = zeros_synced(RING * NKV * HD // 32, torch.int16)
    quants = zeros_synced(RING * NKV * HD, torch.int8)
    k = ctx.load_kernel("kv_append_sliding_q8")
    ctx.dispatch_blocking(k, _bind(sgq, dev(src), scales, quants, _step(ctx, 1022, 0, 0, 0)),
                          None, [n_tok, NKV * HD // 32, 1])
    hs = host(scales).view(np.uint16).reshape(RING, -1)
    hq = host(quants).reshape(RING, -1)
    for t in range(n_tok):
        slot = (1022 + t) % RING
        assert np.array_equal(hs[slot], s_want.reshape(n_tok, -1)[t]), t
        assert np.array_equal(hq[slot], q_want.reshape(n_tok, -1)[t]), t
    assert not hs[3:1022].any() and not hq[3:1022].any()
