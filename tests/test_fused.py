"""Fused decode (sgq_model_set_decode_mode(model, 2)): six launches per
layer, with the norms, residual updates and GeGLU moved into the GEMV
prologues/epilogues and the q/k/v post-projection into the attention launch.  Checked against
the oracle decoder (crates/sg-model/src/reference.rs:157-316 restated in
oracle/model.py) on the same weights, at the tolerance of the
kernel-per-operator path, plus graph replays, determinism and mode switches
mid-context."""
import numpy as np
import pytest
import torch

from _util import empty, host
from test_model import _check_logits, _small_cfg, _weights

pytestmark = pytest.mark.gpu


def _fused(model):
    model.decode_mode = 2
    assert model.decode_mode == 2
    return model


class _side_stream:
    """Graph capture needs a non-null stream: run the block on a side one."""

    def __init__(self, ctx):
        self.ctx, self.s = ctx, torch.cuda.Stream()

    def __enter__(self):
        self.ctx.set_stream(self.s)

    def __exit__(self, *exc):
        self.ctx.synchronize()
        self.ctx.set_stream(None)


@pytest.mark.parametrize("k_eq_v", [1, 0])
def test_fused_small_matches_oracle(ctx, oracle, k_eq_v):
    """4 layers (4-slot sliding ring, 2 global), 10 steps: the ring wraps."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"fused small k_eq_v={k_eq_v}", flush=True)
    cfg = _small_cfg(sgq, global_k_eq_v=k_eq_v)
    model = _fused(sgq.Model(ctx, cfg))
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([1, 2047, 5, 5, 100, 0, 1999, 42, 7, 3]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_fused_graph_replays_match_eager(ctx):
    """The captured step (one graph, replayed with new step words) gives
    the bits of eager fused steps, with unrelated eager work between
    replays; a second run from reset repeats them (determinism)."""
    import sgq

    print("fused graph vs eager", flush=True)
    cfg = _small_cfg(sgq, seed=0x31)
    m = _fused(sgq.Model(ctx, cfg))
    out = empty(cfg.vocab, torch.float32)
    toks = (4, 8, 15, 16, 23, 42)
    eager = []
    for t in toks:
        m.decode(t, out)
        eager.append(host(out).copy())
    with _side_stream(ctx):
        for run in range(2):
            m.reset()
            for i, t in enumerate(toks):
                m.decode(t, out, graph=True)
                ctx.synchronize()
                scratch = torch.randn(4096, device="cuda").sum()  # eager work between replays
                torch.cuda.synchronize()
                del scratch
                assert np.array_equal(eager[i].view(np.uint32), host(out).view(np.uint32)), \
                    f"run {run} step {i}"
    m.close()


def test_fused_mode_switch_mid_context(ctx, oracle):
    """Kernel-per-operator and fused steps on one context: every step matches
    the oracle; decode mode 1 (the removed persistent step) is refused."""
    import sgq
    from oracle.model import OracleDecoder

    print("fused mode switch", flush=True)
    cfg = _small_cfg(sgq, seed=0x5A)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    with _side_stream(ctx):
        with pytest.raises(sgq.ValidationError):
            model.decode_mode = 1
        for i, (t, mode) in enumerate([(9, 0), (8, 2), (7, 2), (6, 0), (5, 2), (4, 0), (3, 2)]):
            model.decode_mode = mode
            model.decode(t, logits, graph=bool(i & 1))
            model.status()
            _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_fused_full_width_matches_oracle(ctx, oracle):
    """The benchmark widths (hidden 5376, ffn 21504, 32 q / 16 kv heads,
    vocab 262144) at 2 layers (one sliding, one global): 3 steps."""
    import sgq
    from oracle.model import OracleDecoder

    print("fused full width", flush=True)
    cfg = sgq.default_model_config(n_layers=2, global_every=2, max_ctx=64, seed=0xF00D)
    model = _fused(sgq.Model(ctx, cfg))
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([2, 262143, 31337]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_fused_long_context_matches_oracle(ctx, oracle):
    """A full, wrapping 1024-slot ring and ~1030-position global layers
    (synthetic pages read back into the oracle's cache); 16 splits per
    sliding kv head meet in the merge."""
    import sgq
    from oracle.model import OracleDecoder

    print("fused long context", flush=True)
    cfg = _small_cfg(sgq, sliding_window=1024, max_ctx=1100, seed=0x10C)
    model = _fused(sgq.Model(ctx, cfg))
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
    with _side_stream(ctx):
        for i, t in enumerate([11, 1500, 2, 77]):
            model.decode(t, logits, graph=True)
            ctx.synchronize()
            _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_fused_after_prefill(ctx, oracle):
    """Prefill (MMQ path, 2 chunks) fills the caches; fused decode
    continues from them."""
    import sgq
    from oracle.model import OraclePrefill

    print("fused after prefill", flush=True)
    cfg = _small_cfg(sgq, max_ctx=64, prefill_chunk=16, seed=0xB0B)
    model = _fused(sgq.Model(ctx, cfg))
    d = cfg.as_dict()
    ref = OraclePrefill(d, _weights(model, d))
    toks = np.random.default_rng(21).integers(0, cfg.vocab, 21)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    want = None
    for c0 in range(0, len(toks), 16):
        want = ref.prefill(toks[c0:c0 + 16])
    _check_logits(host(logits), want, "prefill")
    for i, t in enumerate([3, 4, 5]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), f"after prefill {i}")
    model.close()


@pytest.mark.parametrize("ffn", [8192, 21504])
@pytest.mark.parametrize("mode", [0, 2])
def test_k_sliced_down_projection_matches_oracle(ctx, oracle, ffn, mode):
    """FFN widths whose down projection runs in 2 (8192) or 4 (21504)
    K-slices: the kernel-per-operator mode writes the slice partials with
    one K-slice per workgroup (its part of the limb table in LDS), the fused
    mode keeps the whole table in LDS and sums the slices in the residual
    epilogue; both against the oracle decoder."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"k-sliced down ffn={ffn} mode={mode}", flush=True)
    cfg = _small_cfg(sgq, n_layers=2, ffn=ffn, seed=0x51CE + ffn)
    model = sgq.Model(ctx, cfg)
    model.decode_mode = mode
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([7, 1000, 3, 2047, 64]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()
