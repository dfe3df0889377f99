"""GPU parity of the benchmark decoder itself (62 layers,
hidden 5376, ffn 21504, 32 q / 16 kv heads of 128, 5:1 sliding(1024):global,
vocab 262144, Q4_0 weights) against the CPU oracle decoder on the very
weights the library generated, plus heavy-tailed activations through the
fused decode.

- decode at an 8K context: sgq_model_fill_cache(8192) K/V pages read back
  into the oracle's cache, then two decode steps, logits checked at full
  width (2e-3 bar and top-1, as tests/test_model.py);
- prefill of a short prompt through all 62 layers vs OraclePrefill, then a
  decode step from the caches it filled;
- a 4096-token prefill (BASELINE's prefill workload): finite logits within
  the softcap, not flat, and the next decode step equally so (the oracle
  cannot run 4096 tokens through 62 layers in a test's time).
"""
import numpy as np
import pytest
import torch

from _util import empty, host
from test_model import _check_logits, _small_cfg, _weights

pytestmark = pytest.mark.gpu


def _cfg5(sgq, **kw):
    return sgq.default_model_config(seed=0xC5, **kw)


def _pages(model, n_layers):
    return {(l, kind): (model.read_tensor(f"{kind}_scales", l, np.uint16),
                        model.read_tensor(f"{kind}_quants", l, np.int8))
            for l in range(n_layers) for kind in ("k", "v")}


def _oracle(cls, model, cfg):
    d = cfg.as_dict()
    ref = cls(d, _weights(model, d))
    ref.threads = 16
    return ref


@pytest.mark.timeout(600)
def test_config5_decode_8k_matches_oracle(ctx, oracle):
    import sgq
    from oracle.model import OracleDecoder

    print("config 5: 62 layers, decode at 8K vs oracle", flush=True)
    cfg = _cfg5(sgq, max_ctx=8200)
    model = sgq.Model(ctx, cfg)
    model.fill_cache(8192)
    ref = _oracle(OracleDecoder, model, cfg)
    ref.preload_cache(_pages(model, cfg.n_layers), 8192)
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([262143, 4242]):
        model.decode(t, logits, graph=False)
        torch.cuda.synchronize()
        print(f"  step {i}: oracle", flush=True)
        _check_logits(host(logits), ref.decode(t), f"config 5 step {i}")
    model.close()


class _side_stream:
    """Graph capture needs a non-null stream: run the block on a side one."""

    def __init__(self, ctx):
        self.ctx, self.s = ctx, torch.cuda.Stream()

    def __enter__(self):
        self.ctx.set_stream(self.s)
        return self.s

    def __exit__(self, *exc):
        self.ctx.synchronize()
        self.ctx.set_stream(None)


@pytest.mark.timeout(600)
def test_config5_fused_graph_decode_8k_matches_oracle(ctx, oracle):
    """The benchmarked path itself: decode mode 2 (fused GEMV prologues and
    epilogues, 16-split attention with its merges), replayed as one hipGraph
    per step on a side stream, 62 layers over an 8192-slot context; three
    steps at full logits width against the oracle."""
    import sgq
    from oracle.model import OracleDecoder

    print("config 5: 62 layers, fused hipGraph decode at 8K vs oracle", flush=True)
    cfg = _cfg5(sgq, max_ctx=8200)
    with _side_stream(ctx):
        model = sgq.Model(ctx, cfg)
        model.decode_mode = 2
        model.fill_cache(8192)
        ctx.synchronize()
        ref = _oracle(OracleDecoder, model, cfg)
        ref.preload_cache(_pages(model, cfg.n_layers), 8192)
        logits = empty(cfg.vocab, torch.float32)
        for i, t in enumerate([262143, 4242, 17]):
            model.decode(t, logits, graph=True)
            ctx.synchronize()
            print(f"  step {i}: oracle", flush=True)
            _check_logits(host(logits), ref.decode(t), f"config 5 fused graph step {i}")
        model.close()


@pytest.mark.timeout(600)
def test_config5_fused_graph_after_prefill_matches_oracle(ctx, oracle):
    """A 12-token prefill through all 62 layers, then decode mode 2 as hipGraph
    replays from the caches the prefill filled, against the oracle."""
    import sgq
    from oracle.model import OraclePrefill

    print("config 5: 62 layers, prefill then fused hipGraph decode vs oracle", flush=True)
    cfg = _cfg5(sgq, max_ctx=64)
    with _side_stream(ctx):
        model = sgq.Model(ctx, cfg)
        ref = _oracle(OraclePrefill, model, cfg)
        toks = np.random.default_rng(56).integers(0, cfg.vocab, 12)
        logits = empty(cfg.vocab, torch.float32)
        model.prefill(toks, logits)
        ctx.synchronize()
        _check_logits(host(logits), ref.prefill(toks), "config 5 prefill (fused run)")
        model.decode_mode = 2
        for i, t in enumerate([99, 262000]):
            model.decode(t, logits, graph=True)
            ctx.synchronize()
            _check_logits(host(logits), ref.decode(t), f"config 5 fused graph after prefill {i}")
        model.close()


@pytest.mark.timeout(600)
def test_config5_prefill_matches_oracle_then_decodes(ctx, oracle):
    import sgq
    from oracle.model import OraclePrefill

    print("config 5: 62 layers, 12-token prefill vs oracle", flush=True)
    cfg = _cfg5(sgq, max_ctx=64)
    model = sgq.Model(ctx, cfg)
    ref = _oracle(OraclePrefill, model, cfg)
    toks = np.random.default_rng(55).integers(0, cfg.vocab, 12)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    _check_logits(host(logits), ref.prefill(toks), "config 5 prefill")
    model.decode(99, logits)
    torch.cuda.synchronize()
    _check_logits(host(logits), ref.decode(99), "config 5 decode after prefill")
    model.close()


def _sane(logits, cap, what):
    assert np.isfinite(logits).all(), what
    assert (np.abs(logits) <= cap).all(), what
    assert logits.max() - logits.min() > 1.0, f"{what}: logits flat"


@pytest.mark.timeout(300)
def test_config5_prefill_4096_properties(ctx):
    import sgq

    print("config 5: 4096-token prefill properties", flush=True)
    cfg = _cfg5(sgq, max_ctx=4100)
    model = sgq.Model(ctx, cfg)
    toks = np.random.default_rng(4096).integers(0, cfg.vocab, 4096)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    torch.cuda.synchronize()
    assert model.position == 4096
    _sane(host(logits), cfg.final_softcap, "prefill 4096")
    first = host(logits).copy()
    model.decode(7, logits)
    torch.cuda.synchronize()
    _sane(host(logits), cfg.final_softcap, "decode after 4096")
    assert not np.array_equal(first, host(logits))
    model.close()


def test_model_heavy_tailed_activations_match_oracle(ctx, oracle):
    """Norm weights with one channel in 32 scaled by 10..100 make every GEMV
    input (attn-norm -> QKV, ffn-norm -> gate/up, and through GeGLU the down
    projection's) a block with a large outlier: the limb form's hard case.
    Fused decode vs the oracle on the same weights, 6 steps, at the logits
    bar; the error an f16 rounding of every linear input (the reference's
    activation type) gives on the same model is printed beside it (larger
    here: up to 2.5e-3 of the top logit, and f16 overflows at step 4 of
    this case on the CPU emulation)."""
    import sgq
    from oracle.model import OracleDecoder

    class F16Inputs(OracleDecoder):
        def _lin(self, name, layer, x, n_out):
            return super()._lin(name, layer, oracle.through_f16(x), n_out)

    print("model heavy-tailed activations", flush=True)
    cfg = _small_cfg(sgq, hidden=1024, ffn=2048, seed=0x0B7)
    model = sgq.Model(ctx, cfg)
    g = np.random.default_rng(0x0B7)
    H = cfg.hidden
    for l in range(cfg.n_layers):
        for name in ("attn_norm", "ffn_norm"):
            w = model.read_tensor(name, l).copy()
            pos = np.arange(0, H, 32) + g.integers(0, 32, H // 32)
            w[pos] *= (10.0 ** g.uniform(1, 2, pos.size)).astype(np.float32)
            model.write_tensor(name, w, l)
    d = cfg.as_dict()
    wts = _weights(model, d)
    ref = OracleDecoder(d, wts)
    f16 = F16Inputs(d, wts)
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([1, 2047, 5, 100, 0, 1999]):
        model.decode(t, logits)
        torch.cuda.synchronize()
        want, alt = ref.decode(t), f16.decode(t)
        top = float(np.abs(want).max())
        print(f"  step {i}: gpu {np.abs(host(logits) - want).max() / top:.2e}, "
              f"f16 inputs {np.abs(alt - want).max() / top:.2e} of max|logit|", flush=True)
        _check_logits(host(logits), want, f"outliers step {i}")
    model.close()
