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

from _util import assert_close, dev, empty, host

pytestmark = pytest.mark.gpu

NQ, RING = 32, 1024
GEOM = {"sliding": (256, 16, 1), "global": (512, 4, 2), "global_q8k": (512, 4, 2)}


def _bind(sgq, *tensors):
    return [sgq.BufferBinding.buffer(i, t) for i, t in enumerate(tensors)]


def _step(ctx, pos, kv_sl, kv_gl, q0=0):
    import sgq

    step = torch.zeros(8, dtype=torch.int32, device="cuda")
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
    step = torch.zeros(8, dtype=torch.int32, device="cuda")
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
    app = ctx.load_kernel("kv_append_sliding")
    with pytest.raises(sgq.ValidationError):  # a partial row
        ctx.dispatch(app, _bind(sgq, empty(100, torch.int16), kv, step), b"", [1, 1, 1])
    with pytest.raises(sgq.ValidationError):  # groups short of the rows
        ctx.dispatch(app, _bind(sgq, empty(2 * 4096, torch.int16), empty(RING * 4096, torch.int16),
                                step), b"", [16, 1, 1])
    ctx.synchronize()
