"""CPU pinning of the oracle (oracle/sgo.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own
formula: the reference's known-answer vectors (tests/golden/
reference_kats.json), an independent implementation (numpy's IEEE float16,
a pure-Python xorshift64*, numpy float64 linear algebra), or a mathematical
invariant (brute force on tiny inputs, closed forms, error bounds).
"""
import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


# --- RNG (mod.rs:7-32) vs an independent pure-Python xorshift64* -------------
def _py_xorshift(seed, n):
    M = (1 << 64) - 1
    x = max(seed, 1)
    out = []
    for _ in range(n):
        x ^= x >> 12
        x ^= (x << 25) & M
        x ^= x >> 27
        out.append((x * 0x2545F4914F6CDD1D) & M)
    return out


@pytest.mark.parametrize("seed", [0, 1, 0x6E44, 0xAB, 0x4D, 0xB2, 0xA77])
def test_rng_matches_python_xorshift(oracle, seed):
    r = oracle.Rng(seed)
    assert [int(v) for v in r.u64_vec(64)] == _py_xorshift(seed, 64)


def test_rng_f32_is_uniform_pm2(oracle):
    raw = _py_xorshift(0xD0, 1000)
    want = np.array([(np.float32(v >> 40) / np.float32(1 << 24)) * np.float32(4) - np.float32(2)
                     for v in raw], np.float32)
    got = oracle.Rng(0xD0).f32_vec(1000)
    assert np.array_equal(got, want)
    assert got.min() >= -2.0 and got.max() < 2.0


# --- f16 codec vs numpy's IEEE binary16 (round-to-nearest-even) ---------------
def test_f16_codec_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),   # subnormal range
        (rng.standard_normal(20000) * 7e4).astype(np.float32),    # overflow range
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 2 ** -25, 2 ** -24, 3 * 2 ** -26,
                  np.inf, -np.inf, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32),
    ])
    # every f16 value and the midpoints between neighbours (tie cases)
    allh = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((allh[:-1].astype(np.float64) + allh[1:].astype(np.float64)) / 2).astype(np.float32)
    x = np.concatenate([x, allh, -allh, mids, -mids])
    got = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = oracle.f16_bits_to_f32(np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16))
    want_back = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    same = (back == want_back) | (np.isnan(back) & np.isnan(want_back))
    assert same.all()


# --- Q4_0 dequant (q4_0.rs:31-42) ---------------------------------------------
def _block(d, qs):
    h = np.array([d], np.float16).view(np.uint16)[0]
    return np.array([h & 0xFF, h >> 8] + list(qs), np.uint8)


def test_q4_0_known_block(oracle):
    k = KATS["q4_0_known_block"]
    out = oracle.q4_0_dequant(_block(k["d"], k["qs"]), 1, 32)[0]
    assert out[0] == k["expect"]["0"] and out[16] == k["expect"]["16"]
    assert all(out[i] == 0.0 for i in range(32) if i not in (0, 16))


def test_q4_0_extremes(oracle):
    k = KATS["q4_0_extremes"]
    out = oracle.q4_0_dequant(_block(k["d"], k["qs"]), 1, 32)[0]
    assert out[0] == k["expect"]["0"] and out[16] == k["expect"]["16"]


def test_q4_0_random_blocks_nibble_layout(oracle):
    """Every weight equals d*(nibble-8) with the low/high nibble layout; the
    f32 product is exact, so compare bit-for-bit with float64 math."""
    w = oracle.Rng(0x6E44).random_q4_0(500)
    out = oracle.q4_0_dequant(w, 500, 32)
    blocks = w.reshape(500, 18)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    qs = blocks[:, 2:]
    lo = (qs & 15).astype(np.float64) - 8
    hi = (qs >> 4).astype(np.float64) - 8
    want = np.concatenate([lo, hi], axis=1) * d[:, None]
    assert np.array_equal(out.astype(np.float64), want)


def test_random_q4_0_matches_reference_generator(oracle):
    """random_q4_0 (parity_gemv.rs:23-33): d = f16(f32()*0.05) then 16 bytes."""
    raw = _py_xorshift(0xAB, 17 * 3)
    w = oracle.Rng(0xAB).random_q4_0(3).reshape(3, 18)
    for b in range(3):
        r = raw[17 * b:17 * b + 17]
        u = (np.float32(r[0] >> 40) / np.float32(1 << 24)) * np.float32(4) - np.float32(2)
        d = np.float16(u * np.float32(0.05)).view(np.uint16)
        assert int(w[b, 0]) | (int(w[b, 1]) << 8) == int(d)
        assert list(w[b, 2:]) == [v & 0xFF for v in r[1:]]


# --- GEMV oracle and the CPU baseline matmul (reference.rs:402-444) -------------
def test_gemv_rows_and_matmul_match_float64(oracle):
    rng = oracle.Rng(0xD0)
    n, k = 37, 512
    w = rng.random_q4_0(n * k // 32)
    x = oracle.through_f16(rng.f32_vec(k))
    deq = oracle.q4_0_dequant(w, n, k).astype(np.float64)
    want = deq @ x.astype(np.float64)
    got = oracle.gemv_rows(w, x, k, np.arange(n))
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    mm1 = oracle.matmul_q4_0(w, x, 1, n, k, threads=1)[0]
    mm4 = oracle.matmul_q4_0(w, x, 1, n, k, threads=4)[0]
    assert np.array_equal(mm1, mm4)  # row-parallel: deterministic
    assert np.allclose(mm1, want, rtol=1e-6, atol=1e-6)


def test_dot_f64_lane_order(oracle):
    """dot_f64: 8 f64 lanes summed in order, then the sequential tail."""
    a = np.arange(1, 20, dtype=np.float32) * np.float32(0.1)
    b = np.ones(19, np.float32)
    lanes = [sum(float(a[i]) for i in range(j, 16, 8)) for j in range(8)]
    want = 0.0
    for v in lanes:
        want += v
    for i in range(16, 19):
        want += float(a[i])
    assert oracle.dot_f64(a, b) == want


# --- Q8_0 (mod.rs:272-286, kv_quant_q8.wgsl) ------------------------------------
def test_quant_q8_0_scales_closed_form_and_bounds(oracle):
    x = oracle.through_f16(oracle.Rng(0xB2).f32_vec(4096 + 256))
    x[64:96] = 0.0
    s, q = oracle.quant_q8_0(x)
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1).astype(np.float32)
    d = amax * np.float32(1.0 / 127.0)
    assert np.array_equal(s, d.astype(np.float16).view(np.uint16))
    assert s[2] == 0 and (q[64:96] == 0).all()  # all-zero block: d = 0, q = 0
    qb = q.reshape(-1, 32).astype(np.float64)
    err = np.abs(qb * d[:, None] - blocks)
    assert (err <= d[:, None].astype(np.float64) * (0.5 + 1e-5)).all()
    assert np.abs(q).max() <= 127
    # the element at amax quantizes to +-127 exactly
    idx = np.abs(blocks).argmax(axis=1)
    assert (np.abs(qb[np.arange(len(idx)), idx])[amax > 0] == 127).all()


def test_q8_quant_div_and_v_layout(oracle):
    """q8_quant (division form) and q8_quant_v agree with quant_q8_0 on blocks
    where the two scale rules give the same f16, and q8_quant_v's key blocks
    equal q8_quant_div over the gathered column (mod.rs:98-134)."""
    rng = oracle.Rng(0xA79)
    keys, nkv, hd = 45, 2, 32  # a short final key block
    v = oracle.through_f16(rng.f32_vec(keys * nkv * hd))
    q, s, deq = oracle.q8_quant_v(v, keys, nkv, hd)
    vv = v.reshape(keys, nkv, hd)
    qq = q.reshape(keys, nkv, hd)
    for h in range(nkv):
        for c in (0, 7, 31):
            col = vv[:, h, c]
            for kb in range(2):
                seg = col[kb * 32:(kb + 1) * 32]
                pad = np.zeros(32, np.float32)
                pad[:len(seg)] = seg
                s2, q2, _ = oracle.q8_quant_div(pad)
                assert s[(kb * nkv + h) * hd + c] == s2[0]
                assert np.array_equal(qq[kb * 32:kb * 32 + len(seg), h, c], q2[:len(seg)])
    assert np.allclose(deq.reshape(keys, nkv, hd), vv, atol=np.abs(v).max() / 127)


def test_dequant_q8_0(oracle):
    x = oracle.Rng(0xB3).f32_vec(256)
    s, q = oracle.quant_q8_0(x)
    d = s.view(np.float16).astype(np.float32)
    assert np.array_equal(oracle.dequant_q8_0(s, q), (q.reshape(-1, 32) * d[:, None]).reshape(-1))


# --- MMQ (mod.rs:311-340) ---------------------------------------------------------
def test_block_dot_brute_force(oracle):
    rng = oracle.Rng(0x4D)
    for _ in range(50):
        wblk = rng.random_q4_0(1)
        xq = (rng.u64_vec(32) % 256).astype(np.int64) - 128
        xq = xq.astype(np.int8)
        qs = wblk[2:]
        wq = [(int(qs[j]) & 15) - 8 for j in range(16)] + [(int(qs[j]) >> 4) - 8 for j in range(16)]
        assert oracle.block_dot(wblk, xq) == sum(int(a) * b for a, b in zip(xq, wq))


def test_mmq_oracle_tiny_brute_force_and_nrmse(oracle):
    """16×512×64 as parity_mmq.rs:68-91: exact-arithmetic brute force and
    nrmse < 0.02 against the full-precision matmul."""
    rng = oracle.Rng(0x5E)
    m, k, n = 16, 512, 64
    w = rng.random_q4_0(n * k // 32)
    x = oracle.through_f16(rng.f32_vec(m * k)).reshape(m, k)
    got = oracle.mmq_q4_0_q8(w, x, m, k, n)
    s, q = oracle.quant_q8_0(x)
    da = s.view(np.float16).astype(np.float64).reshape(m, k // 32)
    deq_w = oracle.q4_0_dequant(w, n, k).astype(np.float64)
    xd = q.reshape(m, k // 32, 32).astype(np.float64) * da[:, :, None]
    want = xd.reshape(m, k) @ deq_w.T
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    full = x.astype(np.float64) @ deq_w.T
    nrmse = np.sqrt(np.mean((got - full) ** 2)) / np.sqrt(np.mean(full ** 2))
    assert nrmse < 0.02
    pairs = oracle.mmq_pairs(w, q, s, k, np.array([0, 3, 15]), np.array([0, 10, 63]))
    assert np.array_equal(pairs, got[[0, 3, 15], [0, 10, 63]])
    dots = oracle.mmq_block_dots(w, q, k, 3, 10)
    assert dots.shape == (k // 32,)
    assert dots[5] == oracle.block_dot(w[(10 * (k // 32) + 5) * 18:][:18], q.reshape(m, k)[3, 160:192])


# --- elementwise ---------------------------------------------------------------
def test_gelu_tanh_kats(oracle):
    g = KATS["gelu_tanh"]
    for x, y in g["points"]:
        assert abs(oracle.gelu_tanh(x) - y) < g["abs_tol"]
    for x, y in g["exact"]:
        assert oracle.gelu_tanh(x) == y
    gv = np.array([1.0, -2.0, 0.5], np.float32)
    uv = np.array([2.0, 1.0, -1.0], np.float32)
    out = oracle.geglu(gv, uv)
    assert abs(out[0] - 2 * 0.841192) < 2e-6 and abs(out[1] + 0.0454023) < 1e-6


def test_rmsnorm_matches_numpy(oracle):
    x = oracle.Rng(1).f32_vec(3 * 128).reshape(3, 128)
    w = oracle.Rng(2).f32_vec(128)
    got = oracle.rmsnorm(x, w, 128)
    xd = x.astype(np.float64)
    inv = 1 / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert np.allclose(got, xd * inv * w, rtol=1e-6, atol=1e-7)
    assert np.allclose(oracle.rmsnorm(x, None, 128), xd * inv, rtol=1e-6, atol=1e-7)


def test_rope_kats(oracle):
    t = oracle.cos_sin_table([0], 256, 10000.0).reshape(-1)
    assert (t[0::2] == 1.0).all() and (t[1::2] == 0.0).all()
    k = KATS["rope_first_pair"]
    t = oracle.cos_sin_table([k["pos"]], k["head_dim"], k["theta"]).reshape(-1)
    assert t[0] == np.float32(k["expect_cos0"]) and t[1] == np.float32(k["expect_sin0"])
    k = KATS["rope_proportional"]
    f = np.array([1.0] * 64 + [1e30] * 192, np.float32)
    t = oracle.cos_sin_table([k["pos"]], 512, k["theta"], f).reshape(-1, 2)
    assert (t[64:, 0] == 1.0).all() and (np.abs(t[64:, 1]) < 1e-15).all()
    assert t[0, 0] == np.float32(k["expect_cos0"])
    assert t[63, 0] == np.float32(math.cos(k["pair63_angle"]))
    k = KATS["rope_neox_pairing"]
    assert list(oracle.apply_rope_f32(k["row"], k["cs"])) == k["expect"]
    # f64 rope (mod.rs:198-216) agrees with apply_rope on a live-everywhere table
    row = oracle.Rng(9).f32_vec(2 * 4 * 64)
    cs = oracle.cos_sin_table([5, 6], 64, 10000.0)
    r64 = oracle.rope(row, 64, 64, 4, cs)
    r32 = np.concatenate([oracle.apply_rope_f32(row[i * 64:(i + 1) * 64], cs[i // 4].reshape(-1))
                          for i in range(8)])
    assert np.allclose(r64, r32, atol=1e-6)


def test_attention_kats(oracle):
    k = KATS["attention_uniform"]
    out = oracle.attention(k["q"], k["ck"], k["cv"], 1, k["q0"], k["n_q_heads"], k["n_kv"],
                           k["hd"], None, 1.0).reshape(-1)
    for idx, v in k["expect"]:
        assert abs(out[idx] - v) < k["abs_tol"]
    k = KATS["attention_window"]
    out = oracle.attention(k["q"], k["ck"], k["cv"], 1, k["q0"], 1, 1, 1, k["window"], 1.0)
    assert abs(out.reshape(-1)[0] - 25.0) < 1e-6


def test_attention_head_matches_numpy_softmax(oracle):
    rng = oracle.Rng(0xA77)
    L, nq, nkv, hd = 40, 4, 2, 32
    q = rng.f32_vec(nq * hd)
    k = rng.f32_vec(L * nkv * hd)
    v = rng.f32_vec(L * nkv * hd)
    for qh in range(nq):
        out = oracle.attention_head(q, k, v, 0, qh, nq, nkv, hd, 0.17, 3, 31)
        kvh = qh // 2
        kk = k.reshape(L, nkv, hd)[3:32, kvh].astype(np.float64)
        vv = v.reshape(L, nkv, hd)[3:32, kvh].astype(np.float64)
        s = kk @ q.reshape(nq, hd)[qh].astype(np.float64) * 0.17
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out, p @ vv, rtol=1e-6, atol=1e-7)


def test_add_scaled(oracle):
    a = np.array([1.0, 2.0], np.float32)
    b = np.array([3.0, -1.0], np.float32)
    assert list(oracle.add_scaled(a, b, 0.5)) == [2.0, 0.5]


# --- Q6_K dequant (q6_k.rs:41-62) ---------------------------------------------
def _q6_block(d, scales, ql=0, qh=0):
    blk = np.zeros(210, np.uint8)
    blk[:128] = ql
    blk[128:192] = qh
    blk[192:208] = np.array(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_q6_k_known_block(oracle):
    """q6_k.rs:92-124: all-zero quants give -16; single-byte edits move
    weights 0 and 96 and leave weight 64."""
    k = KATS["q6_k_known_block"]
    blk = _q6_block(k["d"], k["scales"])
    assert (oracle.q6_k_dequant(blk, 1, 256)[0] == k["all_zero_expect"]).all()
    for step in k["steps"]:
        for i, v in step["set"].get("ql", []):
            blk[i] = v
        for i, v in step["set"].get("qh", []):
            blk[128 + i] = v
        for i, v in step["set"].get("qh_or", []):
            blk[128 + i] |= v
        for i, v in step["set"].get("scales", []):
            blk[192 + i] = np.array([v], np.int8).view(np.uint8)[0]
        out = oracle.q6_k_dequant(blk, 1, 256)[0]
        for i, v in step["expect"]:
            assert out[i] == v, (i, out[i], v)


def test_q6_k_negative_scales(oracle):
    """q6_k.rs:126-138: q = 63 everywhere, scale -128, d = 1 -> -3968."""
    k = KATS["q6_k_negative_scales"]
    blk = _q6_block(k["d"], [k["scale"]] * 16, ql=k["ql"], qh=k["qh"])
    assert (oracle.q6_k_dequant(blk, 1, 256)[0] == k["expect_all"]).all()
    assert KATS["q6_k_block_bytes"]["block_bytes"] == 210


def _q6_encode(q, scales, d):
    """Inverse of the Q6_K layout, written from the other side: weight w of
    the block sits in half h = w // 128, group g = (w % 128) // 32, lane
    l = w % 32; its low nibble in ql[64h + l + 32(g & 1)] (high nibble when
    g >= 2), its top two bits in qh[32h + l] at bit 2g; its scale is
    scales[8h + l // 16 + 2g]."""
    blk = np.zeros(210, np.uint8)
    for w in range(256):
        h, g, l = w // 128, (w % 128) // 32, w % 32
        lo, hi = q[w] & 15, q[w] >> 4
        qi = 64 * h + l + 32 * (g & 1)
        blk[qi] |= lo << (4 if g >= 2 else 0)
        blk[128 + 32 * h + l] |= hi << (2 * g)
    blk[192:208] = np.array(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([d], np.float16).view(np.uint8)
    return blk


def test_q6_k_layout_round_trip(oracle):
    """Random 6-bit quants and sub-scales placed by the inverse layout come
    back as d*scale*(q-32) with the sub-block of 16 weights each scale covers
    (exact: small integers times an f16)."""
    rs = np.random.default_rng(7)
    for _ in range(20):
        q = rs.integers(0, 64, 256)
        sc = rs.integers(-128, 128, 16)
        d = np.float16(rs.uniform(-2, 2))
        out = oracle.q6_k_dequant(_q6_encode(q, sc, d), 1, 256)[0]
        w = np.arange(256)
        h, g, l = w // 128, (w % 128) // 32, w % 32
        scale = sc[8 * h + l // 16 + 2 * g]
        want = (np.float32(d) * scale.astype(np.float32)) * (q - 32).astype(np.float32)
        assert np.array_equal(out, want.astype(np.float32))


def test_q6_k_logits_oracle_matches_numpy(oracle):
    """gemv_q6_k_logits oracle: f64 dot over the dequantized rows and the
    30*tanh(v/30) softcap, against numpy on the same rows."""
    rng = oracle.Rng(0xC6)
    n, k, stride = 12, 5376, 4416
    w = rng.random_q6_k_rows(n, k, stride)
    x = oracle.through_f16(rng.f32_vec(k))
    got = oracle.gemv_q6_k_logits(w, stride, x, n, k, 30.0)
    deq = oracle.q6_k_dequant(w, n, k, stride).astype(np.float64)
    want = 30.0 * np.tanh((deq @ x.astype(np.float64)) / 30.0)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)
    assert (w.reshape(n, stride)[:, 4410:] == 0).all()


# --- int8 PV: key-blocked V append and block-quantized P ----------------------
def test_kv_append_v_q8_is_quant_q8_0_per_key_block_column(oracle):
    """kv_append_global_v_q8.wgsl:32-75: every (32-key block, column) is the
    kv_quant_q8 rule (quant_q8_0, pinned above) over that column's live keys,
    placed at key-block pos/32 + t/32; the quants keep the [key x row]
    layout; a short final block covers its live keys (q8_quant_v layout,
    mod.rs:98-134)."""
    rng = oracle.Rng(0xA7E)
    n_tok, row, pos = 45, 64, 64
    src = oracle.through_f16(rng.f32_vec(n_tok * row))
    slots = pos + n_tok + 19
    quants = np.zeros(slots * row, np.int8)
    scales = np.zeros(((slots + 31) // 32) * row, np.uint16)
    oracle.kv_append_v_q8(src, n_tok, row, pos, quants, scales)
    x = src.reshape(n_tok, row)
    qq = quants.reshape(slots, row)
    ss = scales.reshape(-1, row)
    for c in (0, 5, 63):
        for tb in range(2):
            seg = x[tb * 32:(tb + 1) * 32, c]
            pad = np.zeros(32, np.float32)
            pad[:len(seg)] = seg
            s2, q2 = oracle.quant_q8_0(pad)
            assert ss[pos // 32 + tb, c] == s2.reshape(-1)[0]
            assert np.array_equal(qq[pos + tb * 32:pos + tb * 32 + len(seg), c], q2.reshape(-1)[:len(seg)])
    assert not qq[:pos].any() and not qq[pos + n_tok:].any()
    assert not ss[:pos // 32].any()
    # same layout as q8_quant_v wherever the division and multiply scale rules agree
    qv, sv, _ = oracle.q8_quant_v(src, n_tok, 1, row)
    agree = sv.reshape(-1, row) == ss[pos // 32:pos // 32 + 2]
    assert agree.mean() > 0.9
    deq = oracle.dequant_v_keyblocked(quants[pos * row:], scales[(pos // 32) * row:], n_tok, row)
    assert np.allclose(deq.reshape(n_tok, row), x, atol=np.abs(x).max() / 127)


def test_attention_ipv_kats_and_bound(oracle):
    """Block-quantized P (attn_prefill_global_flash_sp_ipv.wgsl:134-181):
    identical keys -> every p is 1 -> q = 127 everywhere -> the mean of V, as
    the exact softmax (reference.rs:572-586); one dominant key per block and
    the others at p ~ 1e-3 -> those round to q = 0 and vanish from numerator
    AND denominator (the reference sums the dequantized P), so the output is
    the dominant key's V exactly; random inputs stay within the quantization
    bound of the exact softmax."""
    hd, n = 32, 64
    k = np.zeros(n * hd, np.float32)
    v = np.tile(np.arange(n, dtype=np.float32)[:, None] * 0.25, (1, hd)).reshape(-1)
    q = np.ones(hd, np.float32)
    out = oracle.attention_head_ipv(q, k, v, 0, 0, 1, 1, hd, 0.1, 0, n - 1)
    assert np.allclose(out, v.reshape(n, hd)[:, 0].mean(), rtol=1e-6)
    # window of 40 keys across two blocks (8..47): blocks restricted to the window
    out = oracle.attention_head_ipv(q, k, v, 0, 0, 1, 1, hd, 0.1, 8, 47)
    assert np.allclose(out, v.reshape(n, hd)[8:48, 0].mean(), rtol=1e-6)
    # dominant key: scores 0 for key 5, log(1e-3) for the rest of its block
    k2 = np.zeros((32, hd), np.float32)
    q2 = np.zeros(hd, np.float32)
    q2[0] = 1.0
    k2[:, 0] = np.float32(np.log(1e-3))
    k2[5, 0] = 0.0
    v2 = (np.arange(32 * hd, dtype=np.float32) % 7).reshape(32, hd)
    out = oracle.attention_head_ipv(q2, k2.reshape(-1), v2.reshape(-1), 0, 0, 1, 1, hd, 1.0, 0, 31)
    assert np.array_equal(out, v2[5])
    exact = oracle.attention_head(q2, k2.reshape(-1), v2.reshape(-1), 0, 0, 1, 1, hd, 1.0, 0, 31)
    assert np.abs(exact - v2[5]).max() > 1e-3
    # random: within ~1/127 of max|v| of the exact softmax
    rng = oracle.Rng(0x1B7)
    L, nq, nkv, hd = 200, 4, 2, 64
    qr, kr, vr = rng.f32_vec(nq * hd), rng.f32_vec(L * nkv * hd), rng.f32_vec(L * nkv * hd)
    for h in range(nq):
        a = oracle.attention_head_ipv(qr, kr, vr, 0, h, nq, nkv, hd, 0.125, 0, L - 1)
        b = oracle.attention_head(qr, kr, vr, 0, h, nq, nkv, hd, 0.125, 0, L - 1)
        assert 0 < np.abs(a - b).max() <= np.abs(vr).max() / 127
