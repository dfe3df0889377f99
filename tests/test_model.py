"""GPU parity: the decode-step driver (sgq_model_*) vs the CPU oracle decoder.

Template: the reference's GPU-vs-CPU model checks (crates/sg-model/tests/
gpu_forward.rs: logits of the GPU graph vs ReferenceModel::forward with a
max-abs / top-1 agreement).  The oracle reads the very weights the library
generated (sgq_model_tensor) and runs reference.rs:157-316 in f64/f32 with
Q8_0 K/V pages.

Tolerance on logits, per step: |err| <= 2e-3*|want| + 2e-3*max|want|
elementwise, and top-1 agreement up to ties within that tolerance (the GPU's
argmax scores within 2e-3*max|want| of the oracle's best).  The GPU differs from
the oracle by the GEMV's x limbs (|err| <= 1.7e-5*amax per block), f32 vs f64
accumulation, and an occasional Q8_0 rounding flip of a K/V element or, in
prefill, of an activation.
"""
import numpy as np
import pytest
import torch

from _util import assert_close, empty, host

pytestmark = pytest.mark.gpu


def _weights(model, cfg):
    from oracle.model import LAYER_TENSORS

    w = {("token_embd", -1): model.read_tensor("token_embd"),
         ("output_norm", -1): model.read_tensor("output_norm")}
    for l in range(cfg["n_layers"]):
        for name in LAYER_TENSORS:
            try:
                w[(name, l)] = model.read_tensor(name, l)
            except Exception:
                if name != "attn_v":
                    raise
    return w


def _check_logits(got, want, step):
    top = float(np.abs(want).max())
    assert_close(got, want, 2e-3, 2e-3 * top, f"logits step {step}")
    # top-1 agreement up to ties within the tolerance: the GPU's choice scores
    # within 2e-3·max|want| of the oracle's best in the oracle's own logits
    g, w_ = int(np.argmax(got)), int(np.argmax(want))
    assert want[g] >= want[w_] - 2e-3 * top, f"top-1 differs at step {step}: {g} vs {w_}"


def _small_cfg(sgq, **kw):
    base = dict(n_layers=4, hidden=512, ffn=1024, n_q_heads=4, n_kv_heads=2, vocab=2048,
                sliding_window=4, global_every=2, max_ctx=16, seed=0x1234)
    base.update(kw)
    return sgq.default_model_config(**base)


@pytest.mark.parametrize("k_eq_v", [1, 0])
def test_model_small_decode_matches_oracle(ctx, oracle, k_eq_v):
    """4 layers (2 sliding with a 4-slot ring, 2 global), 10 steps: the ring
    wraps twice, global layers grow linearly."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"model small k_eq_v={k_eq_v}", flush=True)
    cfg = _small_cfg(sgq, global_k_eq_v=k_eq_v)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    tokens = [1, 2047, 5, 5, 100, 0, 1999, 42, 7, 3]
    for i, t in enumerate(tokens):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    assert model.position == len(tokens)
    model.close()


def test_model_graph_replays_match_eager(ctx):
    """hipGraph decode == eager decode, bit for bit, on every replay, with the
    program's own eager work and synchronizations between replays."""
    import sgq

    print("model graph vs eager", flush=True)
    cfg = _small_cfg(sgq, seed=0x777)
    eager = sgq.Model(ctx, cfg)
    graphed = sgq.Model(ctx, cfg)
    s = torch.cuda.Stream()
    a = empty(cfg.vocab, torch.float32)
    b = empty(cfg.vocab, torch.float32)
    ctx.set_stream(s)
    try:
        for i, t in enumerate([3, 9, 27, 81, 243, 729, 11, 13]):
            eager.decode(t, a)
            graphed.decode(t, b, graph=True)
            ctx.synchronize()
            scratch = torch.randn(4096, device="cuda").sum()  # unrelated eager work
            torch.cuda.synchronize()
            ga, gb = host(a), host(b)
            assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), f"replay {i}"
            assert np.isfinite(ga).all() and float(scratch) == float(scratch)
    finally:
        ctx.set_stream(None)
    eager.close()
    graphed.close()


def test_model_reset_reproduces(ctx):
    import sgq

    cfg = _small_cfg(sgq, seed=0x99)
    m = sgq.Model(ctx, cfg)
    out = empty(cfg.vocab, torch.float32)
    first = []
    for t in (4, 8, 15):
        m.decode(t, out)
        torch.cuda.synchronize()
        first.append(host(out).copy())
    m.reset()
    assert m.position == 0
    for i, t in enumerate((4, 8, 15)):
        m.decode(t, out)
        torch.cuda.synchronize()
        assert np.array_equal(first[i].view(np.uint32), host(out).view(np.uint32))
    m.close()


def test_model_full_width_two_layers_matches_oracle(ctx, oracle):
    """The benchmark widths (hidden 5376, ffn 21504, 32 q / 16 kv heads,
    vocab 262144) at 2 layers (one sliding, one global): 3 steps."""
    import sgq
    from oracle.model import OracleDecoder

    print("model full width 2 layers", flush=True)
    cfg = sgq.default_model_config(n_layers=2, global_every=2, max_ctx=64, seed=0xF00D)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([2, 262143, 31337]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_model_long_context_matches_oracle(ctx, oracle):
    """A 1024-slot sliding ring that is full and wraps (positions 1030..1033,
    one 1024-slot attention pass per kv head) and global layers over ~1030
    positions: synthetic K/V pages (sgq_model_fill_cache) read back into the
    oracle's cache."""
    import sgq
    from oracle.model import OracleDecoder

    print("model long context", flush=True)
    cfg = _small_cfg(sgq, sliding_window=1024, max_ctx=1100, seed=0x10C)
    model = sgq.Model(ctx, cfg)
    model.fill_cache(1030)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    pages = {}
    for l in range(cfg.n_layers):
        for kind in ("k", "v"):
            pages[(l, kind)] = (model.read_tensor(f"{kind}_scales", l, np.uint16),
                                model.read_tensor(f"{kind}_quants", l, np.int8))
    ref.preload_cache(pages, 1030)
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([11, 1500, 2, 77]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


@pytest.mark.parametrize("chunk,n_tok", [(64, 37), (16, 37), (4, 10)])
def test_model_prefill_matches_oracle_then_decodes(ctx, oracle, chunk, n_tok):
    """Prefill in chunks (keys before a chunk come from the 4-slot sliding
    ring or the linear global cache, the chunk's own from its pages), last-
    token logits vs the oracle's prefill (Q8_0 activations into every linear
    layer, as the reference's MMQ path), then 3 decode steps from the caches
    the prefill filled."""
    import sgq
    from oracle.model import OraclePrefill

    print(f"model prefill chunk={chunk} n_tok={n_tok}", flush=True)
    cfg = _small_cfg(sgq, max_ctx=64, prefill_chunk=chunk, seed=0x9F + chunk)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OraclePrefill(d, _weights(model, d))
    rng = np.random.default_rng(chunk + n_tok)
    toks = rng.integers(0, cfg.vocab, n_tok)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    assert model.position == n_tok
    # prefill chunks in the oracle mirror the driver's chunking
    want = None
    for c0 in range(0, n_tok, chunk):
        want = ref.prefill(toks[c0:c0 + chunk])
    _check_logits(host(logits), want, "prefill")
    for i, t in enumerate([5, 900, 33]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), f"after prefill {i}")
    model.close()


def test_model_prefill_past_window_matches_oracle(ctx, oracle):
    """A 1100-token prompt in chunks of 512 at the benchmark's 1024-slot
    sliding window: the third chunk (positions 1024..1099) reads keys from
    the wrapped ring (slots = position mod 1024) over several 128-key LDS
    tiles together with its own pages, and the global layers from the
    linear cache; last-token logits vs the oracle's chunked prefill, then
    2 decode steps from the caches the prefill filled."""
    import sgq
    from oracle.model import OraclePrefill

    print("model prefill past the window", flush=True)
    cfg = _small_cfg(sgq, sliding_window=1024, max_ctx=1200, prefill_chunk=512, seed=0x1100)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OraclePrefill(d, _weights(model, d))
    toks = np.random.default_rng(0x1100).integers(0, cfg.vocab, 1100)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    want = None
    for c0 in range(0, len(toks), 512):
        want = ref.prefill(toks[c0:c0 + 512])
    _check_logits(host(logits), want, "prefill")
    for i, t in enumerate([5, 900]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), f"after prefill {i}")
    model.close()


def test_model_prefill_full_width(ctx, oracle):
    """The benchmark widths at 2 layers, a 300-token prompt in one chunk."""
    import sgq
    from oracle.model import OraclePrefill

    print("model prefill full width", flush=True)
    cfg = sgq.default_model_config(n_layers=2, global_every=2, max_ctx=512, prefill_chunk=512,
                                   seed=0xBEE)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OraclePrefill(d, _weights(model, d))
    toks = np.random.default_rng(7).integers(0, cfg.vocab, 300)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    _check_logits(host(logits), ref.prefill(toks), "prefill full width")
    model.close()


def _write_model_gguf(path, cfg, oracle, seed, rope_ok=True):
    """A GGUF holding every tensor of `cfg` (random Q4_0 matrices, N(1, .1)
    norms) as the reference's exporter names them (desc.rs:150-193)."""
    import struct

    from _gguf import write_gguf

    rng = oracle.Rng(seed)
    H, F, hd = cfg.hidden, cfg.ffn, 128
    QD, KD = cfg.n_q_heads * hd, cfg.n_kv_heads * hd

    def q4(k, n):
        return rng.random_q4_0(n * k // 32).tobytes()

    def f32(n, mean=1.0):
        return (np.float32(mean) + np.float32(0.1) * rng.f32_vec(n)).astype(np.float32).tobytes()

    t = [("token_embd.weight", [H, cfg.vocab], "Q4_0", q4(H, cfg.vocab)),
         ("output_norm.weight", [H], "F32", f32(H))]
    live = int(round(cfg.global_rope_frac * hd / 2))
    rf = [1.0] * live + [1e30] * (hd // 2 - live)
    if not rope_ok:
        rf[0] = 2.0
    t.append(("rope_freqs.weight", [hd // 2], "F32", np.array(rf, np.float32).tobytes()))
    for l in range(cfg.n_layers):
        glob = l % cfg.global_every == cfg.global_every - 1
        b = f"blk.{l}."
        t += [(b + "attn_q.weight", [H, QD], "Q4_0", q4(H, QD)),
              (b + "attn_k.weight", [H, KD], "Q4_0", q4(H, KD))]
        if not (glob and cfg.global_k_eq_v):
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


def test_model_loads_gguf_weights(ctx, oracle, tmp_path):
    """sgq_model_load_gguf puts every tensor in place byte for byte, and the
    model then decodes the file's weights (vs the oracle on the same bytes);
    a shape mismatch or a wrong rope_freqs is refused before any write."""
    import sgq
    from oracle.model import OracleDecoder

    print("model gguf load", flush=True)
    cfg = _small_cfg(sgq, seed=0x6A)
    path = tmp_path / "small.gguf"
    blobs = _write_model_gguf(path, cfg, oracle, 0x66)
    model = sgq.Model(ctx, cfg)
    g = sgq.Gguf(str(path))
    model.load_gguf(g)
    assert model.read_tensor("token_embd").tobytes() == blobs["token_embd.weight"]
    assert model.read_tensor("ffn_down", 3).tobytes() == blobs["blk.3.ffn_down.weight"]
    assert model.read_tensor("attn_q_norm", 1).tobytes() == blobs["blk.1.attn_q_norm.weight"]
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([3, 1000, 17]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), f"gguf {i}")
    # a file for another shape, or with the wrong rope factors, is refused
    other = _small_cfg(sgq, hidden=768, seed=0x6A)
    with pytest.raises(sgq.ValidationError):
        sgq.Model(ctx, other).load_gguf(g)
    bad = tmp_path / "bad_rope.gguf"
    _write_model_gguf(bad, cfg, oracle, 0x66, rope_ok=False)
    with pytest.raises(sgq.ValidationError):
        model.load_gguf(sgq.Gguf(str(bad)))
    g.close()
    model.close()


def test_model_rejects_bad_inputs(ctx):
    import sgq

    cfg = _small_cfg(sgq, max_ctx=2)
    m = sgq.Model(ctx, cfg)
    out = empty(cfg.vocab, torch.float32)
    with pytest.raises(sgq.GpuError):
        m.decode(cfg.vocab, out)  # token out of range
    m.decode(1, out)
    m.decode(1, out)
    with pytest.raises(sgq.GpuError):
        m.decode(1, out)  # context full
    m.close()
    with pytest.raises(sgq.GpuError):
        sgq.Model(ctx, sgq.default_model_config(head_dim=64))
    with pytest.raises(sgq.GpuError):
        sgq.Model(ctx, sgq.default_model_config(n_q_heads=48))  # 3 q heads per kv head
    m = sgq.Model(ctx, _small_cfg(sgq, max_ctx=8))
    with pytest.raises(sgq.GpuError):
        m.prefill(np.arange(9))  # longer than max_ctx
    with pytest.raises(sgq.GpuError):
        m.prefill([cfg.vocab])  # token out of range
    m.close()
