"""Persistent decode (sgq_model_set_decode_mode(model, 1)): one cooperative
launch per step, stages separated by grid barriers.  Checked against the
oracle decoder (crates/sg-model/src/reference.rs:157-316 restated in
oracle/model.py) on the same weights, at the tolerance of the multi-kernel
path, plus determinism and mode switches mid-context."""
import numpy as np
import pytest
import torch

from _util import empty, host
from test_model import _check_logits, _small_cfg, _weights

pytestmark = pytest.mark.gpu


def _persistent(model):
    model.decode_mode = 1
    assert model.decode_mode == 1
    return model


@pytest.mark.parametrize("k_eq_v", [1, 0])
def test_persist_small_matches_oracle(ctx, oracle, k_eq_v):
    """4 layers (4-slot sliding ring, 2 global), 10 steps: the ring wraps."""
    import sgq
    from oracle.model import OracleDecoder

    print(f"persist small k_eq_v={k_eq_v}", flush=True)
    cfg = _small_cfg(sgq, global_k_eq_v=k_eq_v)
    model = _persistent(sgq.Model(ctx, cfg))
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([1, 2047, 5, 5, 100, 0, 1999, 42, 7, 3]):
        model.decode(t, logits)
        model.status()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_persist_deterministic_and_graph_form(ctx):
    """Two runs of the same tokens give identical bits; the _graph entry
    point runs the same launch."""
    import sgq

    print("persist determinism", flush=True)
    cfg = _small_cfg(sgq, seed=0x31)
    m = _persistent(sgq.Model(ctx, cfg))
    out = empty(cfg.vocab, torch.float32)
    first = []
    for t in (4, 8, 15, 16, 23, 42):
        m.decode(t, out)
        m.status()
        first.append(host(out).copy())
    m.reset()
    for i, t in enumerate((4, 8, 15, 16, 23, 42)):
        m.decode(t, out, graph=bool(i & 1))
        m.status()
        assert np.array_equal(first[i].view(np.uint32), host(out).view(np.uint32)), f"step {i}"
    m.close()


def test_persist_mode_switch_mid_context(ctx, oracle):
    """Kernel-per-operator steps, then persistent steps, then back, on one
    context: every step matches the oracle."""
    import sgq
    from oracle.model import OracleDecoder

    print("persist mode switch", flush=True)
    cfg = _small_cfg(sgq, seed=0x5A)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, (t, mode) in enumerate([(9, 0), (8, 0), (7, 1), (6, 1), (5, 1), (4, 0), (3, 1)]):
        model.decode_mode = mode
        model.decode(t, logits)
        model.status()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_persist_full_width_matches_oracle(ctx, oracle):
    """The benchmark widths (hidden 5376, ffn 21504, 32 q / 16 kv heads,
    vocab 262144) at 2 layers (one sliding, one global): 3 steps."""
    import sgq
    from oracle.model import OracleDecoder

    print("persist full width", flush=True)
    cfg = sgq.default_model_config(n_layers=2, global_every=2, max_ctx=64, seed=0xF00D)
    model = _persistent(sgq.Model(ctx, cfg))
    d = cfg.as_dict()
    ref = OracleDecoder(d, _weights(model, d))
    logits = empty(cfg.vocab, torch.float32)
    for i, t in enumerate([2, 262143, 31337]):
        model.decode(t, logits)
        model.status()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_persist_long_context_matches_oracle(ctx, oracle):
    """A full, wrapping 1024-slot ring and ~1030-position global layers
    (synthetic pages read back into the oracle's cache)."""
    import sgq
    from oracle.model import OracleDecoder

    print("persist long context", flush=True)
    cfg = _small_cfg(sgq, sliding_window=1024, max_ctx=1100, seed=0x10C)
    model = _persistent(sgq.Model(ctx, cfg))
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
        model.status()
        _check_logits(host(logits), ref.decode(t), i)
    model.close()


def test_persist_after_prefill(ctx, oracle):
    """Prefill (MMQ path, 2 chunks) fills the caches; persistent decode
    continues from them."""
    import sgq
    from oracle.model import OraclePrefill

    print("persist after prefill", flush=True)
    cfg = _small_cfg(sgq, max_ctx=64, prefill_chunk=16, seed=0xB0B)
    model = _persistent(sgq.Model(ctx, cfg))
    d = cfg.as_dict()
    ref = OraclePrefill(d, _weights(model, d))
    toks = np.random.default_rng(21).integers(0, cfg.vocab, 21)
    logits = empty(cfg.vocab, torch.float32)
    model.prefill(toks, logits)
    model.status()
    want = None
    for c0 in range(0, len(toks), 16):
        want = ref.prefill(toks[c0:c0 + 16])
    _check_logits(host(logits), want, "prefill")
    for i, t in enumerate([3, 4, 5]):
        model.decode(t, logits)
        model.status()
        _check_logits(host(logits), ref.decode(t), f"after prefill {i}")
    model.close()
