"""GPU parity: the decoder at the real checkpoint's geometry (scope row f3)
against the CPU oracle decoder, and GGUF files with its tensor table.

Geometry of crates/sg-gguf/src/desc.rs:66-93 at a small width: 32 query
heads; sliding layers 16 kv heads of 256; global layers 4 kv heads of 512
with K=V (no attn_v tensor); the tied embedding / LM head in Q6_K
(q6_k.rs:25-62, rows padded to 16 bytes on the device as the reference
uploads them); rope_freqs of 256 factors for the global layers' partial
rotation.  These models decode in mode 2 (the fused GEMVs of the
benchmark's step around the any-geometry attention: post-projection, VALU
split attention at head_dim 256/512 with 2 or 8 query heads per kv head, a
merge into the O projection's limbs; the Q6_K head after a norm from the
down GEMV's partial sums) or mode 3 (one kernel per operator), and prefill
in chunks through the int8 MMQs and the head_dim 256/512 prefill attention.
Bar: the logits bar of tests/test_model.py (prefill: _check_prefill_logits);
the head rounds x to f16 (gemv_q6_k_logits semantics), the oracle uses the
fp32 x in an f64 dot.  The oracle attends the device's K/V pages after
checking them against its own Q8_0 rows (_device_kv).
"""
import struct

import numpy as np
import pytest
import torch

from _util import empty, host
from test_model import _check_logits, _weights

pytestmark = pytest.mark.gpu


def _device_kv(model, oracle, flips, loose=False):
    """OracleDecoder.kv_source: the device's dequantized K/V rows of (layer,
    position), after checking them against the oracle's own Q8_0 rows.  Per
    32-element block: the f16 scales agree within one ulp (amax/127 sits
    near a rounding boundary when the GPU's and the oracle's inputs differ
    by float noise; such a block then differs everywhere, by at most a step
    and 127 scale ulps); in blocks whose scales agree, every element within
    one step (a quant flips where the inputs straddle a rounding boundary).
    The counts (flipped quants, blocks with another scale) are a loose
    sanity bound only: the noise grows with depth and position (up to ~27%
    of a row's blocks and ~1.5% of its quants at 520 positions).  At this
    geometry one flip moves a score by a whole step, and the 4-kv-head,
    head_dim-512 attention amplifies it past the logits bar (the oracle
    against itself with 2e-5 relative noise on every linear output: up to
    1.8e-2 with its own Q8 pages, 4e-4 with shared ones), so the oracle
    attends the device's pages.  ``loose``: after a prefill with Q8_0
    activations the rows only have to agree within 10% of their largest
    element (activation flips upstream move them by more than a step)."""
    def src(layer, pos, k_row, v_row):
        L = model.cfg
        glob = layer % L.global_every == L.global_every - 1
        hd = L.head_dim_global if glob else L.head_dim
        nkv = L.n_kv_heads_global if glob else L.n_kv_heads
        slots = L.max_ctx if glob else min(L.sliding_window, L.max_ctx)
        slot = pos if glob else pos % slots
        row = nkv * hd
        out = []
        for kind, mine in (("k", k_row), ("v", v_row)):
            q = model.read_tensor(f"{kind}_quants", layer, np.int8).reshape(slots, row)[slot]
            sc = model.read_tensor(f"{kind}_scales", layer, np.uint16).reshape(slots, row // 32)[slot]
            dev = oracle.dequant_q8_0(sc, q)
            if loose:
                # after a prefill with Q8_0 activations (see _check_prefill_logits)
                err = float(np.abs(dev - mine).max() / max(np.abs(mine).max(), 1e-30))
                assert err <= 0.1, (kind, layer, pos, err)
                out.append(dev)
                continue
            # the oracle's block scale: its largest |q| is 127
            mine_sc = np.abs(mine.reshape(-1, 32)).max(axis=1) / np.float32(127)
            mine_bits = mine_sc.astype(np.float16).view(np.uint16)
            ulps = np.abs(mine_bits.astype(np.int32) - sc.astype(np.int32))
            assert (ulps <= 1).all(), (kind, layer, pos, ulps.max())
            same = np.repeat(ulps == 0, 32)
            step = np.repeat(oracle.f16_bits_to_f32(sc), 32)
            diff = np.abs(dev - mine)
            # one step, plus 127 scale ulps (2^-10 relative) where the scales differ
            tol = step * np.where(same, 1.0001, 1.0001 + 127.0 / 1024)
            assert (diff <= tol + 1e-30).all(), (kind, layer, pos, (diff / step).max())
            flips.append(int((diff[same] > 0).sum()))
            assert flips[-1] <= row // 10, (kind, layer, pos, flips[-1])
            assert (~same).sum() <= row // 2, (kind, layer, pos, int((~same).sum()) // 32)
            out.append(dev)
        return out[0], out[1]
    return src


def _check_prefill_logits(got, want):
    """The prefill bar at this geometry.  Every linear layer of the prefill
    sees Q8_0 activations, and the GPU's and the oracle's inputs to each
    quantization differ by float noise (f32 MMQ sums against f64 dots): a
    quant near a rounding boundary then flips, and one flip moves the logits
    by up to ~1e-2 here.  The oracle against itself with 1e-6 relative noise
    before each Q8_0 round trip spreads its logits by up to ~6e-3
    (tests/test_oracle_model.py::test_q8_activation_noise_spread).  So: max
    error within 2e-2 of the largest logit, and the GPU's top token within
    that of the oracle's best."""
    top = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    assert err <= 2e-2 * top, ("prefill logits", err / top)
    g, w_ = int(np.argmax(got)), int(np.argmax(want))
    assert want[g] >= want[w_] - 2e-2 * top, f"prefill top-1 differs: {g} vs {w_}"


def _real_cfg(sgq, **kw):
    base = dict(n_layers=6, hidden=512, ffn=1024, n_q_heads=32, n_kv_heads=16, head_dim=256,
                head_dim_global=512, n_kv_heads_global=4, embed_q6k=1, vocab=1024,
                sliding_window=4, global_every=3, max_ctx=24, seed=0x31B)
    base.update(kw)
    return sgq.default_model_config(**base)


@pytest.mark.parametrize("mode", [2, 3])
def test_real_geometry_decode_matches_oracle(ctx, oracle, mode):
    """6 layers (4 sliding with a 4-slot ring, 2 global), 10 steps: the ring
    wraps twice and the global layers grow."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"real geometry decode, mode {mode}", flush=True)
    cfg = _real_cfg(sgq)
    model = sgq.Model(ctx, cfg)
    assert model.decode_mode == 2
    model.decode_mode = mode
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    flips = []
    ref.kv_source = _device_kv(model, oracle, flips)
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([1, 1023, 5, 5, 100, 0, 999, 42, 7, 3]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    for bad in (0, 1):  # the head_dim-128 kernels only
        with pytest.raises(sgq.ValidationError):
            model.decode_mode = bad
    model.close()


@pytest.mark.parametrize("mode", [2, 3])
def test_real_geometry_long_context_matches_oracle(ctx, oracle, mode):
    """A full 256-slot sliding ring that wraps (4 splits of 64 slots) and
    global layers over ~520 positions (9 splits, the last one partial):
    synthetic K/V pages (sgq_model_fill_cache) read back into the oracle."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"real geometry long context, mode {mode}", flush=True)
    cfg = _real_cfg(sgq, sliding_window=256, max_ctx=600, seed=0x31E)
    model = sgq.Model(ctx, cfg)
    model.decode_mode = mode
    model.fill_cache(517)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    pages = {}
    for l in range(cfg.n_layers):
        for kind in ("k", "v"):
            pages[(l, kind)] = (model.read_tensor(f"{kind}_scales", l, np.uint16),
                                model.read_tensor(f"{kind}_quants", l, np.int8))
    ref.preload_cache(pages, 517)
    ref.kv_source = _device_kv(model, oracle, [])
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([11, 900, 2, 77]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


@pytest.mark.parametrize("mode", [2, 3])
def test_real_geometry_8k_context_matches_oracle(ctx, oracle, mode):
    """The benchmark's context at this geometry: an 8192-position cache
    (sgq_model_fill_cache) under a full 1024-slot sliding ring (16 splits)
    and a global layer at head_dim 512 with 8 query heads per kv head over
    8193+ positions (129 live splits of 64 slots, the merge over all of
    them), then decode steps against the oracle reading the device's
    pages."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"real geometry 8K context, mode {mode}", flush=True)
    cfg = _real_cfg(sgq, n_layers=3, sliding_window=1024, max_ctx=8200, seed=0x31F)
    model = sgq.Model(ctx, cfg)
    model.decode_mode = mode
    model.fill_cache(8192)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    pages = {}
    for l in range(cfg.n_layers):
        for kind in ("k", "v"):
            pages[(l, kind)] = (model.read_tensor(f"{kind}_scales", l, np.uint16),
                                model.read_tensor(f"{kind}_quants", l, np.int8))
    ref.preload_cache(pages, 8192)
    ref.kv_source = _device_kv(model, oracle, [])
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([5, 600]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_real_geometry_long_prompt_decode_continues_prefill(ctx, oracle):
    """A 1099-token prompt in chunks of 512 (the third chunk starts past the
    1024-slot sliding window, so the ring has wrapped) followed by one
    decode step, against the same 1100 tokens prefilled on a model with the
    same weights: the decode step reads the prefill's ring and global
    pages and must give the last position's logits to the prefill bar
    (decode runs its GEMVs on 15-bit activations where the prefill's MMQs
    take Q8_0 ones, hence that bar) with the same top-1."""
    import sgq

    print("real geometry long prompt: decode continues prefill", flush=True)
    rng = np.random.default_rng(0x5107)
    cfg = _real_cfg(sgq, n_layers=3, sliding_window=1024, max_ctx=1200, prefill_chunk=512,
                    seed=0x320)
    toks = [int(t) for t in rng.integers(0, cfg.vocab, 1100)]
    a = sgq.Model(ctx, cfg)
    la = empty(cfg.vocab, torch.float32)
    a.prefill(toks[:-1])
    a.decode(toks[-1], la)
    b = sgq.Model(ctx, cfg)
    lb = empty(cfg.vocab, torch.float32)
    b.prefill(toks, lb)
    torch.cuda.synchronize()
    assert a.position == b.position == 1100
    _check_prefill_logits(host(la), host(lb))
    a.close()
    b.close()


def test_real_geometry_prefill_graph_and_decode(ctx, oracle):
    """Chunked prefill (two chunks: 16 + 5 tokens, the second attending the
    first's cached keys and its own pages; int8 MMQs on Q8_0 activations,
    head_dim 256/512 prefill attention) against the oracle's prefill with
    the same Q8_0 activation round trips, then graph decode steps; the
    recorded graph replays the step bit for bit."""
    import sgq
    from oracle.model import OraclePrefill

    print("real geometry prefill + graph", flush=True)
    # no ring wrap inside the prompt: the oracle reads the device's pages of
    # every prompt position after the whole prefill
    cfg = _real_cfg(sgq, seed=0x31C, sliding_window=24, max_ctx=32, prefill_chunk=16)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OraclePrefill(d, _weights(model, d))
    ref.kv_source = _device_kv(model, oracle, [], loose=True)
    toks = [3, 14, 159, 265, 358, 979, 323, 846, 264, 338, 327, 950, 288, 419, 716, 939, 937,
            510, 582, 97, 494]
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    _check_prefill_logits(host(logits), ref.prefill(toks))
    eager = sgq.Model(ctx, cfg)
    eager.prefill(toks)
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        a = empty(cfg.vocab, torch.float32)
        for i, t in enumerate([7, 77, 777]):
            model.decode(t, logits, graph=True)
            eager.decode(t, a)
            ctx.synchronize()
            g, e = host(logits), host(a)
            assert np.array_equal(g.view(np.uint32), e.view(np.uint32)), f"replay {i}"
            _check_logits(g, ref.decode(t), f"graph {i}")
    finally:
        ctx.set_stream(None)
    model.close()
    eager.close()


def test_real_geometry_prefill_ring_wrap_matches_one_chunk(ctx, oracle):
    """A 21-token prompt through an 8-slot sliding ring in chunks of 8 and of
    4: the later chunks read the ring (wrapped: early positions leave it as
    later ones arrive) together with their own chunk pages, at head_dim 256
    (ring) and 512 (linear cache).  Against the same prompt in one chunk
    (every key from the chunk's pages) on a model with the same weights:
    the same Q8_0 rows, and with at most 21 keys per query every query's
    keys sit in one 32-key attention tile in all three runs, so the logits
    agree bit for bit (a wrong slot moves them by O(1): swapping two prompt
    tokens moves them by 1.7× the largest logit); then two decode steps
    from each cache, also bit for bit."""
    import sgq

    print("real geometry prefill ring wrap", flush=True)
    toks = [3, 14, 159, 265, 358, 979, 323, 846, 264, 338, 327, 950, 288, 419, 716, 939, 937,
            510, 582, 97, 494]
    models, outs = [], []
    for chunk in (32, 8, 4):
        cfg = _real_cfg(sgq, seed=0x31D, sliding_window=8, max_ctx=40, prefill_chunk=chunk)
        m = sgq.Model(ctx, cfg)
        lg = empty(cfg.vocab, torch.float32)
        m.prefill(toks, lg)
        torch.cuda.synchronize()
        models.append(m)
        outs.append(host(lg))
    for c, o in zip((8, 4), outs[1:]):
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), f"chunk {c}"
    for i, t in enumerate([7, 77]):
        got = []
        for m in models:
            lg = empty(m.cfg.vocab, torch.float32)
            m.decode(t, lg)
            torch.cuda.synchronize()
            got.append(host(lg))
        for c, g in zip((8, 4), got[1:]):
            assert np.array_equal(g.view(np.uint32), got[0].view(np.uint32)), f"decode {i}, chunk {c}"
    for m in models:
        m.close()


@pytest.mark.parametrize("mode", [2, 3])
def test_other_kv_groupings_decode_matches_oracle(ctx, oracle, mode):
    """The any-geometry attention's other PV forms: head_dim 256 with 8
    query heads per kv head (one dim per lane over all slots) and head_dim
    512 with 4 (two dims per lane), 8 steps with a wrapping 4-slot ring."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"kv groupings 8 / 4, mode {mode}", flush=True)
    cfg = _real_cfg(sgq, n_kv_heads=4, n_kv_heads_global=8, seed=0x31F)
    model = sgq.Model(ctx, cfg)
    model.decode_mode = mode
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    ref.kv_source = _device_kv(model, oracle, [])
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([1, 1023, 5, 5, 100, 0, 999, 42]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_benchmark_geometry_mode3_matches_oracle(ctx, oracle):
    """Mode 3 at the benchmark's geometry (head_dim 128, Q4_0 head) is the same
    model as modes 0 and 2: checked against the oracle."""
    import sgq
    from oracle.model import OracleDecoder
    from test_model import _small_cfg

    print("benchmark geometry in mode 3", flush=True)
    cfg = _small_cfg(sgq, seed=0x3E)
    model = sgq.Model(ctx, cfg)
    model.decode_mode = 3
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([1, 2047, 5, 100, 0, 1999]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def _write_real_gguf(path, cfg, oracle, seed):
    """The reference's tensor table (desc.rs:150-193) at cfg's geometry: Q6_K
    token_embd (unpadded rows), rope_freqs [head_dim_global/2], no attn_v on
    global layers."""
    from _gguf import write_gguf

    rng = oracle.Rng(seed)
    H, F = cfg.hidden, cfg.ffn
    row = (H // 256) * 210
    emb = rng.random_q6_k_rows(cfg.vocab, H, row).tobytes()

    def q4(k, n):
        return rng.random_q4_0(n * k // 32).tobytes()

    def f32(n):
        return (np.float32(1.0) + np.float32(0.1) * rng.f32_vec(n)).astype(np.float32).tobytes()

    half = cfg.head_dim_global // 2
    live = int(round(cfg.global_rope_frac * half))
    t = [("token_embd.weight", [H, cfg.vocab], "Q6_K", emb),
         ("output_norm.weight", [H], "F32", f32(H)),
         ("rope_freqs.weight", [half], "F32",
          np.array([1.0] * live + [1e30] * (half - live), np.float32).tobytes())]
    for l in range(cfg.n_layers):
        glob = l % cfg.global_every == cfg.global_every - 1
        hd = cfg.head_dim_global if glob else cfg.head_dim
        nkv = cfg.n_kv_heads_global if glob else cfg.n_kv_heads
        QD, KD = cfg.n_q_heads * hd, nkv * hd
        b = f"blk.{l}."
        t += [(b + "attn_q.weight", [H, QD], "Q4_0", q4(H, QD)),
              (b + "attn_k.weight", [H, KD], "Q4_0", q4(H, KD))]
        if not glob:
            t.append((b + "attn_v.weight", [H, KD], "Q4_0", q4(H, KD)))
        t += [(b + "attn_output.weight", [QD, H], "Q4_0", q4(QD, H)),
              (b + "attn_q_norm.weight", [hd], "F32", f32(hd)),
              (b + "attn_k_norm.weight", [hd], "F32", f32(hd)),
              (b + "attn_norm.weight", [H], "F32", f32(H)),
              (b + "post_attention_norm.weight", [H], "F32", f32(H)),
              (b + "ffn_norm.weight", [H], "F32", f32(H)),
              (b + "post_ffw_norm.weight", [H], "F32", f32(H)),
              (b + "ffn_gate.weight", [H, F], "Q4_0", q4(H, F)),
              (b + "ffn_up.weight", [H, F], "Q4_0", q4(H, F)),
              (b + "ffn_down.weight", [F, H], "Q4_0", q4(F, H)),
              (b + "layer_output_scale.weight", [1], "F32", struct.pack("<f", 0.9))]
    write_gguf(path, [("general.architecture", "str", "gemma4")], t)
    return {name: blob for name, _, _, blob in t}


def test_real_geometry_gguf_loads_and_decodes(ctx, oracle, tmp_path):
    """A GGUF with the real checkpoint's tensor table loads (Q6_K rows land at
    the padded device stride, every other tensor byte for byte) and the model
    then decodes the file's weights as the oracle does; a file of the
    benchmark geometry is refused by this model."""
    import sgq
    from oracle.model import OracleDecoder

    print("real geometry gguf", flush=True)
    cfg = _real_cfg(sgq, seed=0x31D)
    path = tmp_path / "real.gguf"
    blobs = _write_real_gguf(path, cfg, oracle, 0x99)
    model = sgq.Model(ctx, cfg)
    g = sgq.Gguf(str(path))
    model.load_gguf(g)
    H = cfg.hidden
    row, stride = (H // 256) * 210, ((H // 256) * 210 + 15) // 16 * 16
    dev_emb = model.read_tensor("token_embd").reshape(cfg.vocab, stride)
    assert dev_emb[:, :row].tobytes() == blobs["token_embd.weight"]
    assert not dev_emb[:, row:].any()
    assert model.read_tensor("attn_q", 2).tobytes() == blobs["blk.2.attn_q.weight"]
    assert model.read_tensor("attn_k_norm", 5).tobytes() == blobs["blk.5.attn_k_norm.weight"]
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    ref.kv_source = _device_kv(model, oracle, [])
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([3, 1000, 17, 4]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), f"gguf {i}")
    g.close()
    # a benchmark-geometry file (head_dim 128 everywhere, Q4_0 embedding)
    from test_model import _small_cfg, _write_model_gguf

    small = tmp_path / "small.gguf"
    _write_model_gguf(small, _small_cfg(sgq, hidden=512), oracle, 0x66)
    with pytest.raises(sgq.ValidationError):
        model.load_gguf(sgq.Gguf(str(small)))
    model.close()
