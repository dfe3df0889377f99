"""CPU pins of the decoder-forward oracle (oracle/model.py), independent of the
GPU and of the oracle's own composition.

The reference's model-level checks (crates/sg-model/tests/cpu_reference.rs:
25-93) need the real GGUF; they are applied here to random weights:
  - a multi-token forward equals prefill-then-decode and token-by-token
    decode, bit for bit (cpu_reference.rs:84-92);
  - global-layer K differs from V under the shared projection (:66-82);
  - logits are finite, within the softcap and not flat (:53-64).
Beyond those, special weights that reduce the forward to a closed form, and
invariances the architecture fixes (reference.rs:157-316), so that a plausible
structural mistake fails one of them:
  - post norms zero -> every branch vanishes and the logits are
    cap*tanh(E . rmsnorm(x0 * prod(s)) / cap) with x0 = E[token]*sqrt(H)
    (pins the embed scale, layer_output_scale, output norm, softcap, and that
    the post norms act on the branch, not on the residual stream);
  - at position 0 softmax over one key is the identity, so the attention
    output is the (Q8_0 round-tripped) value row of the head's kv group;
  - one layer: logits do not depend on layer_output_scale (the final norm
    absorbs a scale of the whole residual stream; a scale applied before the
    FFN would not be absorbed);
  - scaling attn_q / attn_k / attn_v / attn_output / ffn_down by 2 leaves the
    logits unchanged (q/k/v norms and the post norms), scaling ffn_gate does
    not (GELU is not homogeneous);
  - a sliding layer ignores tokens older than the window and sees the oldest
    one inside it (keys > pos - window); a global layer sees all.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from oracle.model import LAYER_TENSORS, OracleDecoder, OraclePrefill


def _cfg(**kw):
    c = dict(n_layers=2, hidden=256, ffn=512, n_q_heads=4, n_kv_heads=2, head_dim=128,
             vocab=512, sliding_window=1024, global_every=2, max_ctx=64,
             rope_theta_sliding=10000.0, rope_theta_global=1e6, global_rope_frac=0.25,
             eps=1e-6, attn_scale=1.0, final_softcap=30.0, global_k_eq_v=1)
    c.update(kw)
    return c


def _weights(c, seed=0x51DE, sigma_scale=1.0):
    """Q4_0 matrices from the reference generator (d = |N(0,0.02)|), norm
    weights around 1, layer_output_scale 1; per-kind geometry and a Q6_K
    embedding (padded rows) when the config asks for them."""
    rng = O.Rng(seed)
    H, F = c["hidden"], c["ffn"]
    if c.get("embed_q6k"):
        stride = ((H // 256) * 210 + 15) // 16 * 16
        emb = rng.random_q6_k_rows(c["vocab"], H, stride)
    else:
        emb = rng.random_q4_0(c["vocab"] * H // 32)
    w = {("token_embd", -1): emb,
         ("output_norm", -1): (1.0 + 0.1 * rng.f32_vec(H)).astype(np.float32)}
    for l in range(c["n_layers"]):
        ge = c["global_every"]
        glob = l % ge == ge - 1
        hd = (c.get("head_dim_global") or c["head_dim"]) if glob else c["head_dim"]
        nkv = (c.get("n_kv_heads_global") or c["n_kv_heads"]) if glob else c["n_kv_heads"]
        qd, kd = c["n_q_heads"] * hd, nkv * hd
        shapes = {"attn_q": (qd, H), "attn_k": (kd, H), "attn_v": (kd, H), "attn_output": (H, qd),
                  "ffn_gate": (F, H), "ffn_up": (F, H), "ffn_down": (H, F)}
        norms = {"attn_norm": H, "attn_q_norm": hd, "attn_k_norm": hd,
                 "post_attention_norm": H, "ffn_norm": H, "post_ffw_norm": H}
        for name in LAYER_TENSORS:
            if name in shapes:
                n, k = shapes[name]
                w[(name, l)] = rng.random_q4_0(n * k // 32)
            elif name in norms:
                w[(name, l)] = (1.0 + 0.1 * rng.f32_vec(norms[name])).astype(np.float32)
            else:
                w[(name, l)] = np.ones(1, np.float32)
    return w


def _scale_q4_0(wbytes, factor):
    """Multiply every block scale d of a Q4_0 tensor by ``factor`` (a power of
    two: exact in f16 for these magnitudes)."""
    b = wbytes.copy().reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float32) * factor
    b[:, :2] = d.astype(np.float16).reshape(-1, 1).view(np.uint8)
    return b.reshape(-1)


def _prefill(c, w, tokens, q8=False):
    p = OraclePrefill(c, w)
    p.q8_activations = q8
    return p, p.prefill(tokens)


TOKENS = [2, 509, 100, 476, 211]


def test_forward_equals_prefill_then_decode_bitexact():
    """cpu_reference.rs:84-92, plus token-by-token decode of the whole prompt."""
    c = _cfg(n_layers=4, sliding_window=3)
    w = _weights(c)
    _, a = _prefill(c, w, TOKENS)
    p, _ = _prefill(c, w, TOKENS[:-1])
    b = p.decode(TOKENS[-1])
    d = OracleDecoder(c, w)
    for t in TOKENS:
        e = d.decode(t)
    assert a.view(np.uint32).tolist() == b.view(np.uint32).tolist()
    assert a.view(np.uint32).tolist() == e.view(np.uint32).tolist()


def test_logits_finite_capped_not_flat_and_global_k_ne_v():
    """cpu_reference.rs:53-82 on random weights."""
    c = _cfg(n_layers=2, global_every=2)
    w = _weights(c)
    p = OraclePrefill(c, w)
    p.q8_activations = False
    p.taps = {}
    logits = p.prefill(TOKENS)
    cap = c["final_softcap"]
    assert logits.shape == (c["vocab"],)
    assert np.isfinite(logits).all()
    assert (np.abs(logits) <= cap).all()
    assert logits.max() - logits.min() > 1.0, "logits suspiciously flat"
    assert p.is_global(1) and not p.is_global(0)
    k, v = p.taps[("k_rope", 1)], p.taps[("v_norm", 1)]
    assert k.shape == v.shape
    assert (np.abs(k - v) > 1e-3).sum() > k.size // 2, "global K and V near-identical"
    # with K=V off the global layer's V comes from attn_v, so the shared
    # projection is what makes V a function of Wk: scaling Wv then is a no-op
    # only when K=V is on
    w2 = dict(w)
    w2[("attn_v", 1)] = _scale_q4_0(w[("attn_v", 1)], 0.0)
    _, l_on = _prefill(c, w2, TOKENS)
    assert np.array_equal(l_on, logits)


def _closed_form_no_branches(c, w, token):
    """Zero post norms: x_L = x0 * prod(s), logits = cap*tanh(E.rmsnorm(x_L)/cap).
    numpy float64 throughout; the embedding row dequantized from its bytes."""
    H = c["hidden"]
    blk = w[("token_embd", -1)].reshape(-1, 18).astype(np.uint8)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    qs = blk[:, 2:].astype(np.int64)
    vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=1) * d[:, None]
    E = vals.reshape(c["vocab"], H)
    x = E[token] * math.sqrt(H)
    for l in range(c["n_layers"]):
        x = x * float(w[("layer_output_scale", l)][0])
    xn = x / np.sqrt(np.mean(x * x) + c["eps"]) * w[("output_norm", -1)].astype(np.float64)
    cap = c["final_softcap"]
    return cap * np.tanh(E @ xn / cap)


@pytest.mark.parametrize("big", [False, True])
def test_zero_post_norms_reduce_to_closed_form(big):
    """Every branch is rmsnorm(.)*0 = 0, so only embed -> scales -> final norm
    -> tied head -> softcap remain.  eps = 1 makes sqrt(H) and the layer
    scales visible through the final norm; ``big`` scales the embedding so the
    softcap saturates."""
    c = _cfg(n_layers=3, eps=1.0)
    w = _weights(c)
    if big:
        w[("token_embd", -1)] = _scale_q4_0(w[("token_embd", -1)], 64.0)
    scales = [0.5, 2.0, 0.25]
    for l in range(c["n_layers"]):
        w[("post_attention_norm", l)] = np.zeros(c["hidden"], np.float32)
        w[("post_ffw_norm", l)] = np.zeros(c["hidden"], np.float32)
        w[("layer_output_scale", l)] = np.array([scales[l]], np.float32)
    d = OracleDecoder(c, w)
    for i, t in enumerate(TOKENS[:3]):
        got = d.decode(t).astype(np.float64)
        want = _closed_form_no_branches(c, w, t)
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6 * c["final_softcap"],
                                   err_msg=f"step {i}")
    if big:
        assert np.abs(want).max() > 0.9 * c["final_softcap"]


def test_position_zero_attention_is_the_value_row():
    """One layer at position 0 with the FFN branch zeroed: softmax over the only
    key is 1, so a = V (per kv group, Q8_0 round-tripped), and
    x1 = (x0 + rmsnorm(Wo a) * w_post) * s.  K=V off: V from attn_v."""
    c = _cfg(n_layers=1, global_every=1, global_k_eq_v=0)
    w = _weights(c)
    w[("post_ffw_norm", 0)] = np.zeros(c["hidden"], np.float32)
    w[("layer_output_scale", 0)] = np.array([0.5], np.float32)
    H, hd, nq, nkv, eps = c["hidden"], c["head_dim"], c["n_q_heads"], c["n_kv_heads"], c["eps"]
    tok = 77
    emb = O.q4_0_dequant(w[("token_embd", -1)], c["vocab"], H)
    x0 = (emb[tok] * np.float32(math.sqrt(H))).astype(np.float32)
    xn = O.rmsnorm(x0, w[("attn_norm", 0)], H, eps)
    v = O.gemv_rows(w[("attn_v", 0)], xn, H, np.arange(nkv * hd))
    v = O.rmsnorm(v, None, hd, eps)
    s, q = O.quant_q8_0(v)
    v = O.dequant_q8_0(s, q).reshape(nkv, hd)
    a = np.concatenate([v[h // (nq // nkv)] for h in range(nq)])
    o = O.gemv_rows(w[("attn_output", 0)], a, nq * hd, np.arange(H))
    x1 = ((x0 + O.rmsnorm(o, w[("post_attention_norm", 0)], H, eps)) * np.float32(0.5))
    xf = O.rmsnorm(x1.astype(np.float32), w[("output_norm", -1)], H, eps)
    want = 30.0 * np.tanh(emb.astype(np.float64) @ xf.astype(np.float64) / 30.0)
    got = OracleDecoder(c, w).decode(tok)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_layer_output_scale_absorbed_by_final_norm_on_one_layer():
    c = _cfg(n_layers=1, global_every=1)
    w = _weights(c)
    _, base = _prefill(c, w, TOKENS)
    w4 = dict(w)
    w4[("layer_output_scale", 0)] = np.array([4.0], np.float32)
    _, scaled = _prefill(c, w4, TOKENS)
    np.testing.assert_allclose(scaled, base, rtol=1e-5, atol=1e-5)
    # two layers: the second layer's branches are O(1) against a stream scaled
    # by 4, so the answer must move
    c2 = _cfg(n_layers=2)
    w = _weights(c2)
    _, base2 = _prefill(c2, w, TOKENS)
    w4 = dict(w)
    w4[("layer_output_scale", 0)] = np.array([4.0], np.float32)
    _, scaled2 = _prefill(c2, w4, TOKENS)
    assert np.abs(scaled2 - base2).max() > 1e-2


@pytest.mark.parametrize("name,invariant", [
    ("attn_q", True), ("attn_k", True), ("attn_v", True), ("attn_output", True),
    ("ffn_down", True), ("ffn_gate", False)])
def test_weight_scale_invariance_pins_the_norms(name, invariant):
    """q/k norms, the weightless v norm and the two post norms make the
    forward homogeneous of degree 0 in those matrices; GELU makes it not so
    in ffn_gate.  Layer 0 is sliding with its own attn_v; layer 1 global
    with K=V."""
    c = _cfg(n_layers=2)
    w = _weights(c)
    _, base = _prefill(c, w, TOKENS)
    w2 = dict(w)
    w2[(name, 0)] = _scale_q4_0(w[(name, 0)], 2.0)
    _, moved = _prefill(c, w2, TOKENS)
    diff = np.abs(moved - base).max()
    if invariant:
        assert diff <= 2e-5 * np.abs(base).max(), f"{name}: {diff}"
    else:
        assert diff > 1e-3, f"{name}: {diff}"


def test_sliding_window_boundary_and_global_reach():
    """One sliding layer, window 3: the last query (pos 5) attends keys 3,4,5.
    Changing the token at pos 2 leaves the logits bit-identical; at pos 3 it
    moves them.  A global layer sees pos 0."""
    c = _cfg(n_layers=1, global_every=2, sliding_window=3)
    w = _weights(c)
    toks = [5, 6, 7, 8, 9, 10]
    _, base = _prefill(c, w, toks)
    outside = list(toks)
    outside[2] = 300
    _, o = _prefill(c, w, outside)
    assert np.array_equal(o, base)
    inside = list(toks)
    inside[3] = 300
    _, i = _prefill(c, w, inside)
    assert np.abs(i - base).max() > 1e-4
    cg = _cfg(n_layers=1, global_every=1, sliding_window=3)
    _, gb = _prefill(cg, w, toks)
    far = list(toks)
    far[0] = 300
    _, gf = _prefill(cg, w, far)
    assert np.abs(gf - gb).max() > 1e-4


def _real_cfg(**kw):
    """The real checkpoint's geometry (crates/sg-gguf/src/desc.rs:66-93) at a
    small width: 32 q heads, sliding 16 kv x 256, global 4 kv x 512, K=V on
    global layers, Q6_K embedding / tied head."""
    c = _cfg(n_layers=3, hidden=512, ffn=512, n_q_heads=32, n_kv_heads=16, head_dim=256,
             head_dim_global=512, n_kv_heads_global=4, embed_q6k=1, vocab=256,
             global_every=3, sliding_window=3)
    c.update(kw)
    return c


def test_real_geometry_forward_invariants():
    """cpu_reference.rs:25-93 at the real per-kind geometry: decode ==
    prefill bit for bit, K != V on the global layer, logits sane; and the
    embedding scale, output norm and softcap closed form through the Q6_K
    tied head with zero post norms."""
    c = _real_cfg()
    w = _weights(c)
    _, a = _prefill(c, w, TOKENS)
    d = OracleDecoder(c, w)
    for t in TOKENS:
        e = d.decode(t)
    assert a.view(np.uint32).tolist() == e.view(np.uint32).tolist()
    p = OraclePrefill(c, w)
    p.q8_activations = False
    p.taps = {}
    logits = p.prefill(TOKENS)
    assert np.isfinite(logits).all() and (np.abs(logits) <= 30.0).all()
    assert logits.max() - logits.min() > 1.0
    k, v = p.taps[("k_rope", 2)], p.taps[("v_norm", 2)]
    assert k.shape == (len(TOKENS), 4 * 512)
    assert (np.abs(k - v) > 1e-3).sum() > k.size // 2
    # zero post norms: logits = cap*tanh(E . rmsnorm(x0 * prod(s)) / cap), E the
    # dequantized Q6_K rows (independent numpy dequant of the block layout)
    c0 = _real_cfg(eps=1.0)
    w0 = _weights(c0, seed=0x66)
    for l in range(c0["n_layers"]):
        w0[("post_attention_norm", l)] = np.zeros(c0["hidden"], np.float32)
        w0[("post_ffw_norm", l)] = np.zeros(c0["hidden"], np.float32)
        w0[("layer_output_scale", l)] = np.array([0.5], np.float32)
    H = c0["hidden"]
    stride = ((H // 256) * 210 + 15) // 16 * 16
    raw = w0[("token_embd", -1)].reshape(c0["vocab"], stride)[:, :(H // 256) * 210]
    blk = raw.reshape(c0["vocab"], H // 256, 210).astype(np.int64)
    ql, qh, sc = blk[..., :128], blk[..., 128:192], blk[..., 192:208].astype(np.int8)
    dd = raw.reshape(c0["vocab"], H // 256, 210)[..., 208:210].copy().view(np.float16)[..., 0]
    E = np.zeros((c0["vocab"], H // 256, 256))
    for h in range(2):
        for l in range(32):
            qs = [(ql[..., 64 * h + l] & 15) | ((qh[..., 32 * h + l] & 3) << 4),
                  (ql[..., 64 * h + l + 32] & 15) | (((qh[..., 32 * h + l] >> 2) & 3) << 4),
                  (ql[..., 64 * h + l] >> 4) | (((qh[..., 32 * h + l] >> 4) & 3) << 4),
                  (ql[..., 64 * h + l + 32] >> 4) | (((qh[..., 32 * h + l] >> 6) & 3) << 4)]
            for j in range(4):
                E[..., 128 * h + 32 * j + l] = (dd.astype(np.float64) *
                                                sc[..., 8 * h + l // 16 + 2 * j] * (qs[j] - 32))
    E = E.reshape(c0["vocab"], H)
    tok = 17
    x = E[tok] * np.sqrt(H) * 0.5 ** c0["n_layers"]
    xn = x / np.sqrt(np.mean(x * x) + 1.0) * w0[("output_norm", -1)].astype(np.float64)
    want = 30.0 * np.tanh(E @ xn / 30.0)
    got = OracleDecoder(c0, w0).decode(tok)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-5)


def test_q8_activation_noise_spread():
    """How far the Q8_0-activation prefill moves under float noise: the
    oracle against itself with 1e-6 relative noise on every activation
    before its Q8_0 round trip.  Flipped quants move the logits by ~1e-3 ..
    1e-2 at 4 layers and hidden 512, the scale of the GPU prefill's
    deviations from the oracle (its f32 MMQ sums differ from the oracle's
    f64 dots by that much); the GPU prefill bar at the real geometry is set
    above it.  Pinned here: the spread is non-zero for some seed (quants do
    flip) and stays below 2e-2."""
    c = _cfg(n_layers=4, hidden=512, ffn=1024, global_every=2, sliding_window=4, embed_q6k=1,
             vocab=512)
    w = _weights(c, seed=0x31C)
    toks = [3, 14, 159, 200]
    _, base = _prefill(c, w, toks, q8=True)
    spreads = []
    for trial in range(3):
        rng = np.random.default_rng(trial)
        op = OraclePrefill(c, w)
        clean = op._q8rt

        def noisy(x2d, clean=clean, rng=rng):
            return clean((x2d * (1 + 1e-6 * rng.standard_normal(x2d.shape))).astype(np.float32))

        op._q8rt = noisy
        out = op.prefill(toks)
        spreads.append(float(np.abs(out - base).max() / np.abs(base).max()))
    assert max(spreads) > 0.0, spreads
    assert max(spreads) < 2e-2, spreads


def test_f16_graph_rounds_every_buffer_and_keeps_page_formats():
    """F16Graph (the reference GPU graph's storage, graph.rs:282-313,
    :581-611): every layer output is f16-representable, sliding caches hold
    the f16 K/V rows themselves, global caches Q8_0 K and f16 V; and it stays
    within f16 noise of the fp32 forward on the same weights."""
    from oracle.model import F16Graph

    c = _cfg(n_layers=2, global_every=2)
    w = _weights(c)
    ref16, ref32 = F16Graph(c, w), OracleDecoder(c, w)
    ref16.taps = {}
    for t in (5, 77, 3):
        got, want = ref16.decode(t), ref32.decode(t)
        top = float(np.abs(want).max())
        assert np.abs(got - want).max() <= 2e-2 * top
        assert not np.array_equal(got, want)  # the roundings are really there
        for l in range(2):
            x = ref16.taps[("x_layer", l)]
            assert np.array_equal(O.through_f16(x), x)
        k, v = ref16.taps[("k_rope", 1)], ref16.taps[("v_norm", 1)]
        s, q = O.quant_q8_0(k)
        assert np.array_equal(ref16.k_cache[1][-1], O.dequant_q8_0(s, q))
        assert np.array_equal(ref16.v_cache[1][-1], v)
        assert np.array_equal(ref16.k_cache[0][-1], ref16.taps[("k_rope", 0)])
        assert np.array_equal(O.through_f16(v), v)
