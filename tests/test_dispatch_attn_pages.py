"""GPU parity: the real checkpoint's decode-side names over f16 pages
(attn_decode_sliding / _global / _global_q8k, attn_reduce_d256 / _d512,
kv_append_sliding / _global) through the name-based dispatch surface, bound
as the reference's record_layer binds them (crates/sg-model/src/graph.rs:
572-650), against the f64 oracle.

Geometry baked into the names (crates/sg-gpu/build.rs:255-394): 32 query
heads; sliding head_dim 256 over 16 kv heads, ring 1024; global head_dim 512
over 4 kv heads.  q, K and V are f16 (the oracle sees the same f16 values);
attn_decode_global_q8k reads K from Q8_0 pages (f16 scale per 32 dims).
Tolerance |err| <= 1e-3*|want| + 1e-4*rms: the f16 rounding of the output
(<= 2^-11 relative) plus the split-softmax's f32 error.  The partials are
checked against each split's own chunk: m = max score, l = sum exp(s - m),
and an empty split holds m = -3e38, l = 0 (attn_decode_sliding.wgsl:60-121).
The appends are placement copies: bit-exact.
"""
import struct

import numpy as np
import pytest
import torch

from _util import assert_close, dev, empty, host, zeros_synced

pytestmark = pytest.mark.gpu

NQ, RING = 32, 1024
GEOM = {"sliding": (256, 16, 1), "global": (512, 4, 2), "global_q8k": (512, 4, 2)}


def _bind(sgq, *tensors):
    return [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(tensors)]


def _step(ctx, pos, kv_sl, kv_gl, q0=0):
    import sgq

    step = zeros_synced(8, torch.int32)
    ctx.step_write(step, sgq.StepState(pos, kv_sl, kv_gl, q0))
    return step


def _pages(oracle, seed, kind, slots):
    """f16 q / K / V (and Q8_0 K for q8k) with their f32 values as read."""
    hd, nkv, _ = GEOM[kind]
    rng = oracle.Rng(seed)
    q = oracle.f32_to_f16_bits(rng.f32_vec(NQ * hd))
    k = rng.f32_vec(slots * nkv * hd)
    v = oracle.f32_to_f16_bits(rng.f32_vec(slots * nkv * hd))
    if kind == "global_q8k":
        ks, kq = oracle.quant_q8_0(k)
        kf = oracle.dequant_q8_0(ks, kq)
        kbind = (dev(kq), dev(ks))
    else:
        kb = oracle.f32_to_f16_bits(k)
        kf = oracle.f16_bits_to_f32(kb)
        kbind = (dev(kb),)
    return (q, oracle.f16_bits_to_f32(q), kbind, kf, dev(v), oracle.f16_bits_to_f32(v))


def _decode(ctx, kind, tq, kbind, tv, step, splits, scale):
    import sgq

    hd, nkv, _ = GEOM[kind]
    attn = ctx.load_kernel(f"attn_decode_{kind}")
    red = ctx.load_kernel(f"attn_reduce_d{hd}")
    part = empty(NQ * splits * (hd + 2), torch.float32)
    out = empty(NQ * hd, torch.int16)
    ctx.dispatch(attn, _bind(sgq, tq, *kbind, tv, part, step),
                 struct.pack("<If", splits, scale), [nkv, splits, 1])
    ctx.dispatch_blocking(red, _bind(sgq, part, out), struct.pack("<I", splits), [NQ, 1, 1])
    return part, out


@pytest.mark.parametrize("kind,kv_len,splits", [
    ("sliding", 1024, 16), ("sliding", 333, 5), ("sliding", 1, 1), ("sliding", 7, 16),
    ("global", 4096, 32), ("global", 100, 32), ("global", 65, 3),
    ("global_q8k", 4096, 32), ("global_q8k", 2000, 32), ("global_q8k", 1, 1),
    # more splits than the merge reads per pass (64): chunks rescaled to a
    # running max, a ragged last chunk, empty splits at the end
    ("sliding", 1024, 130), ("global", 4096, 200),
])
def test_decode_pages_by_name_matches_oracle(ctx, oracle, kind, kv_len, splits):
    hd, nkv, word = GEOM[kind]
    qpk = NQ // nkv
    print(f"dispatch attn_decode_{kind} kv_len={kv_len} splits={splits}", flush=True)
    q16, qf, kbind, kf, tv, vf = _pages(oracle, 0xF16 + kv_len + hd, kind, kv_len)
    scale = 1.0 / np.sqrt(hd) if kind == "sliding" else 1.0
    kvs = [0, kv_len, 0] if word == 1 else [0, 0, kv_len]
    step = _step(ctx, kv_len - 1, kvs[1], kvs[2])
    part, out = _decode(ctx, kind, dev(q16), kbind, tv, step, splits, scale)
    got = oracle.f16_bits_to_f32(host(out, np.uint16))
    want = np.stack([oracle.attention_head(qf, kf, vf, 0, h, NQ, nkv, hd, scale, 0, kv_len - 1)
                     for h in range(NQ)]).reshape(-1)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got, want, 1e-3, 1e-4 * rms, f"attn_decode_{kind}")

    # each split's (m, l) over its own chunk, in the reference's layout
    part = host(part).reshape(NQ, splits, hd + 2)
    chunk = -(-kv_len // splits)
    kk = kf.reshape(kv_len, nkv, hd).astype(np.float64)
    for h in (0, NQ // 2 + 1, NQ - 1):
        s_all = kk[:, h // qpk, :] @ qf.reshape(NQ, hd)[h].astype(np.float64) * scale
        for s in range(splits):
            t0, t1 = min(s * chunk, kv_len), min(s * chunk + chunk, kv_len)
            m, l = part[h, s, hd], part[h, s, hd + 1]
            if t0 == t1:
                assert m == np.float32(-3.0e38) and l == 0.0, (h, s, m, l)
                assert not part[h, s, :hd].any(), (h, s)
                continue
            mw = s_all[t0:t1].max()
            assert abs(m - mw) <= 1e-5 * max(1.0, abs(mw)), (h, s, m, mw)
            lw = np.exp(s_all[t0:t1] - mw).sum()
            assert abs(l - lw) <= 1e-4 * lw, (h, s, l, lw)


def test_decode_pages_long_context_many_tiles(ctx, oracle):
    """attn_decode_global_q8k at 32768 slots over the reference's 32 splits:
    16 tiles of 64 slots per split, so the running max and the rescale of
    the accumulator are exercised across many tiles; keys drift upward along
    the context (k·(1 + t/8192)) so that later tiles keep raising the max.
    Sampled heads against the oracle at the decode bar."""
    kind, kv_len, splits = "global_q8k", 32768, 32
    hd, nkv, _ = GEOM[kind]
    print(f"dispatch attn_decode_{kind} kv_len={kv_len} splits={splits}", flush=True)
    rng = oracle.Rng(0x32C)
    q16 = oracle.f32_to_f16_bits(rng.f32_vec(NQ * hd))
    qf = oracle.f16_bits_to_f32(q16)
    k = rng.f32_vec(kv_len * nkv * hd).reshape(kv_len, -1)
    k *= (1.0 + np.arange(kv_len, dtype=np.float32) / 8192.0)[:, None]
    ks, kq = oracle.quant_q8_0(k.reshape(-1))
    kf = oracle.dequant_q8_0(ks, kq)
    vb = oracle.f32_to_f16_bits(rng.f32_vec(kv_len * nkv * hd))
    vf = oracle.f16_bits_to_f32(vb)
    scale = 1.0 / np.sqrt(hd)
    part, out = _decode(ctx, kind, dev(q16), (dev(kq), dev(ks)), dev(vb),
                        _step(ctx, kv_len - 1, 0, kv_len), splits, scale)
    got = oracle.f16_bits_to_f32(host(out, np.uint16)).reshape(NQ, hd)
    heads = [0, 7, 8, 19, 31]
    want = np.stack([oracle.attention_head(qf, kf, vf, 0, h, NQ, nkv, hd, scale, 0, kv_len - 1)
                     for h in heads])
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert_close(got[heads], want, 1e-3, 1e-4 * rms, "attn_decode_global_q8k 32K")


def test_decode_pages_head_mapping_isolates_kv_heads(ctx, oracle):
    """V constant per kv head (value = kv head index + 1): every query head's
    output is exactly its own kv head's value whatever the softmax weights,
    which pins query head h -> kv head h / (32 / n_kv) on both geometries."""
    for kind in ("sliding", "global"):
        hd, nkv, word = GEOM[kind]
        kv_len = 300
        q16, _, kbind, _, _, _ = _pages(oracle, 0xA11 + hd, kind, kv_len)
        v = np.repeat(np.arange(1, nkv + 1, dtype=np.float32), hd)
        v = np.tile(v, kv_len)
        tv = dev(oracle.f32_to_f16_bits(v))
        kvs = [0, kv_len, 0] if word == 1 else [0, 0, kv_len]
        _, out = _decode(ctx, kind, dev(q16), kbind, tv, _step(ctx, 0, kvs[1], kvs[2]), 7, 1.0)
        got = oracle.f16_bits_to_f32(host(out, np.uint16)).reshape(NQ, hd)
        want = (np.arange(NQ) // (NQ // nkv) + 1).astype(np.float32)
        assert np.allclose(got, want[:, None], rtol=1e-3, atol=0), kind


@pytest.mark.parametrize("kind,pos,n_tok", [("sliding", 1000, 50), ("sliding", 5, 1),
                                            ("global", 37, 5), ("global", 0, 64)])
def test_kv_append_f16_by_name_places_rows(ctx, oracle, kind, pos, n_tok):
    import sgq

    row = 16 * 256 if kind == "sliding" else 4 * 512
    slots = RING if kind == "sliding" else pos + n_tok + 3
    rng = oracle.Rng(0xA99 + pos)
    src = oracle.f32_to_f16_bits(rng.f32_vec(n_tok * row))
    dst0 = oracle.f32_to_f16_bits(rng.f32_vec(slots * row))
    tdst = dev(dst0)
    k = ctx.load_kernel(f"kv_append_{kind}")
    groups = [-(-n_tok * row // 256), 1, 1]
    ctx.dispatch_blocking(k, _bind(sgq, dev(src), tdst, _step(ctx, pos, 0, 0)), b"", groups)
    want = dst0.reshape(slots, row).copy()
    for t in range(n_tok):
        want[(pos + t) % RING if kind == "sliding" else pos + t] = src.reshape(n_tok, row)[t]
    assert np.array_equal(host(tdst, np.uint16).reshape(slots, row), want)


def test_real_decode_layer_graph_replay(ctx, oracle):
    """The global layer's V append, attention over Q8_0 K and f16 V, and
    reduce, recorded once as a graph and replayed with the step buffer
    rewritten (graph.rs:633-650): each replay equals the eager dispatches of
    the same step."""
    import sgq

    kind, splits = "global_q8k", 32
    hd, nkv, _ = GEOM[kind]
    cap = 600
    q16, _, kbind, _, tv, _ = _pages(oracle, 0x9A9, kind, cap)
    tq = dev(q16)
    rng = oracle.Rng(0x9AA)
    new_v = dev(oracle.f32_to_f16_bits(rng.f32_vec(nkv * hd)))
    app = ctx.load_kernel("kv_append_global")
    attn = ctx.load_kernel("attn_decode_global_q8k")
    red = ctx.load_kernel("attn_reduce_d512")
    step = zeros_synced(8, torch.int32)
    part = empty(NQ * splits * (hd + 2), torch.float32)
    out = empty(NQ * hd, torch.int16)
    v_eager = tv.clone()
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        with sgq.GraphRecorder(ctx) as rec:
            ctx.dispatch(app, _bind(sgq, new_v, tv, step), b"", [nkv * hd // 256, 1, 1])
            ctx.dispatch(attn, _bind(sgq, tq, *kbind, tv, part, step),
                         struct.pack("<If", splits, 1.0), [nkv, splits, 1])
            ctx.dispatch(red, _bind(sgq, part, out), struct.pack("<I", splits), [NQ, 1, 1])
        for pos in (100, 101, 599, 7):
            ctx.step_write(step, sgq.StepState(pos, 0, pos + 1, 0))
            rec.graph.submit()
            ctx.synchronize()
            got = host(out).copy()
            st = _step(ctx, pos, 0, pos + 1)
            ctx.dispatch_blocking(app, _bind(sgq, new_v, v_eager, st), b"",
                                  [nkv * hd // 256, 1, 1])
            _, ref = _decode(ctx, kind, tq, kbind, v_eager, st, splits, 1.0)
            assert np.array_equal(got, host(ref)), pos
            torch.randn(1024, device="cuda").sum().item()  # unrelated eager work
    finally:
        ctx.set_stream(None)


def test_pages_names_validate_groups_and_ranges(ctx):
    import sgq

    hd, nkv = 512, 4
    attn = ctx.load_kernel("attn_decode_global")
    tq = empty(NQ * hd, torch.int16)
    kv = empty(64 * nkv * hd, torch.int16)
    part = empty(NQ * 4 * (hd + 2), torch.float32)
    step = _step(ctx, 0, 0, 64)
    with pytest.raises(sgq.ValidationError):  # groups.x is the kv head count
        ctx.dispatch(attn, _bind(sgq, tq, kv, kv, part, step), struct.pack("<If", 4, 1.0),
                     [16, 4, 1])
    with pytest.raises(sgq.ValidationError):  # part too small for 8 splits
        ctx.dispatch(attn, _bind(sgq, tq, kv, kv, part, step), struct.pack("<If", 8, 1.0),
                     [nkv, 8, 1])
    red = ctx.load_kernel("attn_reduce_d256")
    with pytest.raises(sgq.ValidationError):  # out too small for hd256 rows
        ctx.dispatch(red, _bind(sgq, part, empty(NQ * 128, torch.int16)),
                     struct.pack("<I", 4), [NQ, 1, 1])
    for bad in (0, 70000):  # split counts past the decode grid's limit
        with pytest.raises(sgq.ValidationError):
            ctx.dispatch(red, _bind(sgq, part, empty(NQ * 256, torch.int16)),
                         struct.pack("<I", bad), [NQ, 1, 1])
    app = ctx.load_kernel("kv_append_sliding")
    with pytest.raises(sgq.ValidationError):  # a partial row
        ctx.dispatch(app, _bind(sgq, empty(100, torch.int16), kv, step), b"", [1, 1, 1])
    with pytest.raises(sgq.ValidationError):  # groups short of the rows
        ctx.dispatch(app, _bind(sgq, empty(2 * 4096, torch.int16), empty(RING * 4096, torch.int16),
                                step), b"", [16, 1, 1])
    ctx.synchronize()


# --- prefill over the reference's page formats ------------------------------
# attn_prefill_sliding[_ring] (hd256, 16 kv heads, window 1024, ring 1024),
# attn_prefill_global[_flash[_sp]] (hd512, 4 kv heads, causal, f16 pages),
# _sp_q8 (f16 q, Q8_0 K and V dequantized to f16, as that shader does) and
# _sp_iq (int8 q and Q8_0 K: score = sum over blocks of q_scale·k_scale·
# integer dot; f16 V), _sp_ipv[_bcast] (the same with int8 V under key-blocked
# scales and P quantized per query and 32-key block; oracle attention_head_ipv).
# q0 = step[3].  Bar: the typed prefill tests' (|err| <=
# 2e-3·|want| + 1e-3·max|want|, normwise 1e-3) plus the f16 rounding of the
# output (2^-11 of max|want|): normwise 1.5e-3.  Cache slots the kernel must
# not read hold f16 NaN.
F16_NAN = np.uint16(0x7E00)
PREFILL = {  # name: (head_dim, n_kv, window, per-token grid)
    "attn_prefill_sliding": (256, 16, 1024, True),
    "attn_prefill_sliding_ring": (256, 16, 1024, True),
    "attn_prefill_global": (512, 4, 0, True),
    "attn_prefill_global_flash": (512, 4, 0, False),
    "attn_prefill_global_flash_sp": (512, 4, 0, False),
    "attn_prefill_global_flash_sp_q8": (512, 4, 0, False),
    "attn_prefill_global_flash_sp_iq": (512, 4, 0, False),
    "attn_prefill_global_flash_sp_ipv": (512, 4, 0, False),
    "attn_prefill_global_flash_sp_ipv_bcast": (512, 4, 0, False),
}


def _prefill_check(got, want, what):
    top = float(np.abs(want).max())
    assert_close(got, want, 2e-3, 1.5e-3 * top, what)
    err = float(np.abs(got.astype(np.float64) - want).max()) / top
    assert err <= 1.5e-3, (what, err)


def _prefill_by_name(ctx, name, binds, m, scale):
    import sgq

    hd, nkv, _, per_token = PREFILL[name]
    k = ctx.load_kernel(name)
    groups = [nkv, m, 1] if per_token else [NQ, m // 16, 1]
    ctx.dispatch_blocking(k, [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(binds)],
                          struct.pack("<f", scale), groups)


@pytest.mark.parametrize("name,q0,m", [
    ("attn_prefill_sliding", 1200, 100), ("attn_prefill_sliding", 0, 37),
    ("attn_prefill_sliding_ring", 1500, 160), ("attn_prefill_sliding_ring", 0, 64),
    ("attn_prefill_sliding_ring", 700, 1), ("attn_prefill_sliding_ring", 1000, 90),
    ("attn_prefill_global", 300, 50), ("attn_prefill_global_flash", 0, 128),
    ("attn_prefill_global_flash_sp", 77, 48), ("attn_prefill_global_flash_sp_q8", 200, 64),
    ("attn_prefill_global_flash_sp_iq", 0, 256), ("attn_prefill_global_flash_sp_iq", 333, 32),
])
def test_prefill_pages_by_name_matches_oracle(ctx, oracle, name, q0, m):
    hd, nkv, window, _ = PREFILL[name]
    print(f"dispatch {name} q0={q0} M={m}", flush=True)
    rng = oracle.Rng(0x9F + q0 + 7 * m + hd)
    n = q0 + m
    qf = rng.f32_vec(m * NQ * hd)
    kf = rng.f32_vec(n * nkv * hd)
    vf = rng.f32_vec(n * nkv * hd)
    scale = 1.0 if name.endswith("_iq") else 1.0 / np.sqrt(hd)
    row = nkv * hd
    step = _step(ctx, q0, 0, 0, q0)
    out = torch.full((m * NQ * hd,), 0x7E00, dtype=torch.int16, device="cuda")

    def nan_padded(bits, rows):  # cache rows past position n - 1 hold NaN
        full = np.full(rows * row, F16_NAN, np.uint16)
        full[:bits.size] = bits
        return full

    if name.endswith("_iq") or name.endswith("_q8"):
        ks, kq = oracle.quant_q8_0(kf)
        if name.endswith("_iq"):
            qs, qq = oracle.quant_q8_0(qf)
            qd = oracle.dequant_q8_0(qs, qq)
            kd = oracle.dequant_q8_0(ks, kq)
            vb = oracle.f32_to_f16_bits(vf)
            vd = oracle.f16_bits_to_f32(vb)
            binds = [dev(qq), dev(qs), dev(kq), dev(ks), dev(nan_padded(vb, n + 40)), out, step]
        else:
            q16 = oracle.f32_to_f16_bits(qf)
            qd = oracle.f16_bits_to_f32(q16)
            vs, vq = oracle.quant_q8_0(vf)
            kd, vd = oracle.dequant_q8_0_f16(ks, kq), oracle.dequant_q8_0_f16(vs, vq)
            binds = [dev(q16), dev(kq), dev(ks), dev(vq), dev(vs), out, step]
    else:
        q16, kb, vb = (oracle.f32_to_f16_bits(x) for x in (qf, kf, vf))
        qd, kd, vd = (oracle.f16_bits_to_f32(x) for x in (q16, kb, vb))
        if name.endswith("_ring"):
            kr = np.full(RING * row, F16_NAN, np.uint16)
            vr = kr.copy()
            for p in range(max(0, q0 - RING), q0):  # the ring before this chunk's append
                sl = (p % RING) * row
                kr[sl:sl + row], vr[sl:sl + row] = kb[p * row:(p + 1) * row], vb[p * row:(p + 1) * row]
            binds = [dev(q16), dev(kr), dev(vr), dev(kb[q0 * row:]), dev(vb[q0 * row:]), out, step]
        else:
            binds = [dev(q16), dev(nan_padded(kb, n + 40)), dev(nan_padded(vb, n + 40)), out, step]
    _prefill_by_name(ctx, name, binds, m, scale)
    got = oracle.f16_bits_to_f32(host(out, np.uint16)).reshape(m, NQ, hd)
    want = oracle.attention(qd, kd, vd, m, q0, NQ, nkv, hd, window, scale)
    _prefill_check(got, want, f"{name} q0={q0} M={m}")


@pytest.mark.parametrize("name,q0,m", [
    ("attn_prefill_global_flash_sp_ipv", 0, 128), ("attn_prefill_global_flash_sp_ipv", 200, 64),
    ("attn_prefill_global_flash_sp_ipv_bcast", 37, 32),
])
def test_prefill_ipv_by_name_matches_oracle(ctx, oracle, name, q0, m):
    """int8 PV at head_dim 512 against oracle.attention_head_ipv on the same
    dequantized q, K and key-blocked V (the scores are exact here, as the
    int8 QK is).  P is quantized against the running max in the kernel and the
    final max in the oracle, so a block's f16 P scale may round differently
    (2^-11): the int8-PV bar of the head_dim-128 test (2e-3) plus the f16
    output rounding.  V-scale rows past the last key hold f16 NaN."""
    hd, nkv = 512, 4
    print(f"dispatch {name} q0={q0} M={m}", flush=True)
    rng = oracle.Rng(0x1F5 + q0 + m)
    n, row = q0 + m, nkv * hd
    qs, qq = oracle.quant_q8_0(rng.f32_vec(m * NQ * hd))
    ks, kq = oracle.quant_q8_0(rng.f32_vec(n * row))
    vq = np.zeros(n * row, np.int8)
    vs = np.zeros(((n + 31) // 32) * row, np.uint16)
    oracle.kv_append_v_q8(rng.f32_vec(n * row), n, row, 0, vq, vs)
    qd, kd = oracle.dequant_q8_0(qs, qq), oracle.dequant_q8_0(ks, kq)
    vd = oracle.dequant_v_keyblocked(vq, vs, n, row)
    vs_pad = np.concatenate([vs, np.full(2 * row, F16_NAN, np.uint16)])
    out = torch.full((m * NQ * hd,), 0x7E00, dtype=torch.int16, device="cuda")
    scale = 1.0 / np.sqrt(hd)
    _prefill_by_name(ctx, name, [dev(qq), dev(qs), dev(kq), dev(ks), dev(vq), dev(vs_pad), out,
                                 _step(ctx, q0, 0, 0, q0)], m, scale)
    got = oracle.f16_bits_to_f32(host(out, np.uint16)).reshape(m, NQ, hd)
    want = np.empty_like(got)
    for i in range(m):
        for h in range(NQ):
            want[i, h] = oracle.attention_head_ipv(qd, kd, vd, i, h, NQ, nkv, hd, scale, 0, q0 + i)
    top = float(np.abs(want).max())
    assert_close(got, want, 2e-3, 2.5e-3 * top, f"{name} q0={q0} M={m}")
    err = float(np.abs(got.astype(np.float64) - want).max()) / top
    assert err <= 2.5e-3, (name, err)


def test_prefill_sliding_ring_equals_linear_view(ctx, oracle):
    """The two-range form (history from the pre-append ring, the chunk from
    its own pages) and the linear form over the same positions attend the
    same keys in the same order: bit-identical outputs."""
    hd, nkv, q0, m = 256, 16, 2100, 200
    row = nkv * hd
    rng = oracle.Rng(0x2A9)
    q16 = oracle.f32_to_f16_bits(rng.f32_vec(m * NQ * hd))
    kb = oracle.f32_to_f16_bits(rng.f32_vec((q0 + m) * row))
    vb = oracle.f32_to_f16_bits(rng.f32_vec((q0 + m) * row))
    kr = np.empty(RING * row, np.uint16)
    vr = np.empty(RING * row, np.uint16)
    for p in range(q0 - RING, q0):
        sl = (p % RING) * row
        kr[sl:sl + row], vr[sl:sl + row] = kb[p * row:(p + 1) * row], vb[p * row:(p + 1) * row]
    step = _step(ctx, q0, 0, 0, q0)
    a = empty(m * NQ * hd, torch.int16)
    b = empty(m * NQ * hd, torch.int16)
    _prefill_by_name(ctx, "attn_prefill_sliding_ring",
                     [dev(q16), dev(kr), dev(vr), dev(kb[q0 * row:]), dev(vb[q0 * row:]), a, step],
                     m, 0.0625)
    _prefill_by_name(ctx, "attn_prefill_sliding", [dev(q16), dev(kb), dev(vb), b, step], m, 0.0625)
    assert np.array_equal(host(a), host(b))


def test_prefill_pages_names_validate(ctx):
    import sgq

    k = ctx.load_kernel("attn_prefill_global_flash_sp_iq")
    q = empty(64 * NQ * 512 // 2, torch.int16)
    bad = [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(
        [q, q, q, q, q, empty(64 * NQ * 512, torch.int16), _step(ctx, 0, 0, 0, 0)])]
    with pytest.raises(sgq.ValidationError):  # groups.x is the query head count
        ctx.dispatch(k, bad, struct.pack("<f", 1.0), [4, 4, 1])
    with pytest.raises(sgq.ValidationError):  # out holds 64 rows, groups ask for 80
        ctx.dispatch(k, bad, struct.pack("<f", 1.0), [NQ, 5, 1])
    ring = ctx.load_kernel("attn_prefill_sliding_ring")
    small = empty(100 * 16 * 256, torch.int16)
    with pytest.raises(sgq.ValidationError):  # a ring of 100 slots
        ctx.dispatch(ring, [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(
            [empty(8 * NQ * 256, torch.int16), small, small, small, small,
             empty(8 * NQ * 256, torch.int16), _step(ctx, 0, 0, 0, 0)])],
                     struct.pack("<f", 1.0), [16, 8, 1])
    ctx.synchronize()


def test_prefill_ring_graph_replay_with_step_q0(ctx, oracle):
    """record_prefill_layer's use (graph.rs:1176-1190): attn_prefill_sliding_ring
    recorded once into a graph and replayed for two chunks, the step buffer
    rewritten with each chunk's q0 and the pages refilled between replays;
    every replay equals an eager dispatch of the same chunk bit for bit and
    the oracle at the prefill bar."""
    import sgq

    hd, nkv, m = 256, 16, 48
    row = nkv * hd
    name = "attn_prefill_sliding_ring"
    k = ctx.load_kernel(name)
    tq = empty(m * NQ * hd, torch.int16)
    tkr = empty(RING * row, torch.int16)
    tvr = empty(RING * row, torch.int16)
    tkc = empty(m * row, torch.int16)
    tvc = empty(m * row, torch.int16)
    out = empty(m * NQ * hd, torch.int16)
    step = zeros_synced(8, torch.int32)
    binds = [tq, tkr, tvr, tkc, tvc, out, step]
    B = [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(binds)]
    push = struct.pack("<f", 0.0625)
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        with sgq.GraphRecorder(ctx) as rec:
            ctx.dispatch(k, B, push, [nkv, m, 1])
        for q0 in (1200, 37):
            print(f"graph replay {name} q0={q0}", flush=True)
            rng = oracle.Rng(0x6A + q0)
            q16 = oracle.f32_to_f16_bits(rng.f32_vec(m * NQ * hd))
            kb = oracle.f32_to_f16_bits(rng.f32_vec((q0 + m) * row))
            vb = oracle.f32_to_f16_bits(rng.f32_vec((q0 + m) * row))
            kr = np.zeros(RING * row, np.uint16)
            vr = np.zeros(RING * row, np.uint16)
            for p in range(max(0, q0 - RING), q0):
                sl = (p % RING) * row
                kr[sl:sl + row], vr[sl:sl + row] = kb[p * row:(p + 1) * row], vb[p * row:(p + 1) * row]
            for t, a in ((tq, q16), (tkr, kr), (tvr, vr), (tkc, kb[q0 * row:]), (tvc, vb[q0 * row:])):
                t.copy_(torch.from_numpy(a.view(np.int16)).to("cuda"))
            ctx.step_write(step, sgq.StepState(q0, 0, 0, q0))
            ctx.synchronize()
            rec.graph.submit()
            ctx.synchronize()
            got = host(out).copy()
            ctx.dispatch_blocking(k, B, push, [nkv, m, 1])
            assert np.array_equal(got, host(out)), q0
            want = oracle.attention(*(oracle.f16_bits_to_f32(x) for x in (q16, kb, vb)), m, q0, NQ,
                                    nkv, hd, 1024, 0.0625)
            _prefill_check(oracle.f16_bits_to_f32(got.view(np.uint16)).reshape(m, NQ, hd), want,
                           f"graph replay q0={q0}")
            torch.randn(1024, device="cuda").sum().item()  # unrelated eager work
    finally:
        ctx.set_stream(None)


def test_chunked_sliding_prefill_attend_then_append(ctx, oracle):
    """The sliding layer's prefill order in record_prefill_layer
    (graph.rs:1176-1190): per chunk, attn_prefill_sliding_ring over the ring
    as it stands before the chunk's append plus the chunk's own pages, then
    kv_append_sliding of the chunk's K and V.  Three chunks of 400 tokens
    (the ring wraps during the third); every chunk's rows, on sampled query
    heads, against the oracle over the linear positions at the prefill bar."""
    import sgq

    hd, nkv, m, chunks = 256, 16, 400, 3
    row = nkv * hd
    rng = oracle.Rng(0xC4C)
    total = m * chunks
    kb = oracle.f32_to_f16_bits(rng.f32_vec(total * row))
    vb = oracle.f32_to_f16_bits(rng.f32_vec(total * row))
    kf, vf = oracle.f16_bits_to_f32(kb), oracle.f16_bits_to_f32(vb)
    attn = ctx.load_kernel("attn_prefill_sliding_ring")
    app = ctx.load_kernel("kv_append_sliding")
    ring_k = zeros_synced(RING * row, torch.int16)
    ring_v = zeros_synced(RING * row, torch.int16)
    out = empty(m * NQ * hd, torch.int16)
    B = sgq.BufferBinding.buffer
    for c in range(chunks):
        q0 = c * m
        print(f"chunked sliding prefill chunk {c} q0={q0}", flush=True)
        q16 = oracle.f32_to_f16_bits(rng.f32_vec(m * NQ * hd))
        ck, cv = dev(kb[q0 * row:(q0 + m) * row]), dev(vb[q0 * row:(q0 + m) * row])
        step = _step(ctx, q0, 0, 0, q0)
        ctx.dispatch(attn, [B(0, dev(q16)), B(1, ring_k), B(2, ring_v), B(3, ck), B(4, cv), B(5, out),
                            B(6, step)], struct.pack("<f", 0.0625), [nkv, m, 1])
        groups = [m * row // 256, 1, 1]
        ctx.dispatch(app, [B(0, ck), B(1, ring_k), B(2, step)], b"", groups)
        ctx.dispatch_blocking(app, [B(0, cv), B(1, ring_v), B(2, step)], b"", groups)
        got = oracle.f16_bits_to_f32(host(out, np.uint16)).reshape(m, NQ, hd)
        qf = oracle.f16_bits_to_f32(q16)
        heads = [0, 9, 22, 23]  # sampled query heads (23: the second of kv head 11)
        want = np.stack([np.stack([oracle.attention_head(qf, kf, vf, i, h, NQ, nkv, hd, 0.0625,
                                                         max(0, q0 + i + 1 - 1024), q0 + i)
                                   for h in heads]) for i in range(m)])
        _prefill_check(got[:, heads], want, f"chunk {c}")


@pytest.mark.parametrize("kind", ["sliding", "global_q8k"])
def test_empty_context_merges_to_zero(ctx, oracle, kind):
    """kv_len 0: every split is empty (m = -3e38, l = 0, acc = 0) and the
    merged row is 0 (attn_reduce.wgsl's acc/l would be 0/0 here; the
    reference's graph never runs a step with an empty cache)."""
    hd, nkv, word = GEOM[kind]
    q16, _, kbind, _, tv, _ = _pages(oracle, 0xE0E + hd, kind, 64)
    step = _step(ctx, 0, 0, 0)
    part, out = _decode(ctx, kind, dev(q16), kbind, tv, step, 4, 1.0)
    p = host(part).reshape(NQ, 4, hd + 2)
    assert (p[:, :, hd] == np.float32(-3e38)).all() and (p[:, :, hd + 1] == 0).all()
    assert (host(out, np.uint16) == 0).all()
