"""A whole decoder layer recorded purely through the reference's dispatch
surface, in record_layer's order (crates/sg-model/src/graph.rs:478-656), at
the released checkpoint's geometry, replayed as a graph for three positions
and compared with the oracle decoder on the same weights and caches.

Nothing here goes through sgq_model_*: every operator is looked up by its
reference variant name (rmsnorm_5376, gemv_q4_0_k5376, rmsnorm_256/_512,
rope_{sliding,global}_{q,k}, kv_append_sliding, kv_append_global_q8,
kv_append_global, attn_decode_sliding, attn_decode_global_q8k,
attn_reduce_d256/_d512, gemv_q4_0_k8192/_k16384/_k21504, add_scaled, geglu)
and bound to f16 activation buffers, f16 sliding K/V rings and a Q8_0-K /
f16-V global cache, exactly as graph.rs:282-313 and :360-385 allocate them;
the per-step inputs arrive as stage_token writes them (graph.rs:1487-1529):
the residual row, the step buffer and the cos/sin tables.

Oracles (oracle/model.py):
- F16Graph: the forward with every buffer between two operators rounded to
  f16 and the caches in the graph's page formats, i.e. what the reference's
  graph stores.  Bar: max |error| per layer output 4e-3 of max |x| (the
  two sides round about twenty intermediate buffers to f16 each, and a
  value near a rounding midpoint can go either way: half an f16 ulp is
  2.4e-4 of a value, and such flips add up over a layer; measured 0.7e-3 to
  2.4e-3).
- The fp32 decoder (reference.rs:157-316) on the same caches: bar 1e-2, the
  size of the f16 storage itself, so the f16 restatement cannot share a
  mistake with the kernels unnoticed.
"""
import math
import struct

import numpy as np
import pytest
import torch

from _util import dev, empty, host, rel_err, zeros_synced
from test_model import _weights

pytestmark = pytest.mark.gpu

H, F, NQ = 5376, 21504, 32
RING = 1024
SPLITS_SL, SPLITS_GL = 16, 32  # graph.rs:36-37
P0 = 1100                     # positions already cached (the ring has wrapped)


def _cfg(sgq):
    return sgq.default_model_config(n_layers=2, global_every=2, head_dim=256,
                                    head_dim_global=512, n_kv_heads=16, n_kv_heads_global=4,
                                    vocab=256, max_ctx=64, seed=0x1A7)


class _Graph:
    """The buffers of graph.rs:282-313 for one sliding and one global layer."""

    def __init__(self, ctx, sgq, wts, cfg):
        self.ctx, self.sgq = ctx, sgq
        h16 = lambda n: zeros_synced(n, torch.int16)  # noqa: E731
        self.qd = {"s": NQ * 256, "g": NQ * 512}
        self.kvd = {"s": 16 * 256, "g": 4 * 512}
        self.x, self.xn, self.o, self.on, self.x2, self.fin, self.f, self.fn2 = \
            (h16(H) for _ in range(8))
        self.g, self.u, self.gu = h16(F), h16(F), h16(F)
        self.q_raw = {k: h16(v) for k, v in self.qd.items()}
        self.q = {k: h16(v) for k, v in self.qd.items()}
        self.attn = {k: h16(v) for k, v in self.qd.items()}
        self.kp = {k: h16(v) for k, v in self.kvd.items()}
        self.k = {k: h16(v) for k, v in self.kvd.items()}
        self.vp_sl = h16(self.kvd["s"])
        self.v = {k: h16(v) for k, v in self.kvd.items()}
        self.part = {"s": empty(NQ * SPLITS_SL * 258, torch.float32),
                     "g": empty(NQ * SPLITS_GL * 514, torch.float32)}
        self.step = zeros_synced(4, torch.int32)
        self.cs = {"s": empty(128 * 2, torch.float32), "g": empty(64 * 2, torch.float32)}
        self.ones = torch.ones(512, dtype=torch.float32, device="cuda")
        self.w = {key: dev(a) for key, a in wts.items()}
        self.scale = {l: float(wts[("layer_output_scale", l)][0]) for l in range(2)}
        self.kern = {}

    def k_(self, name):
        if name not in self.kern:
            self.kern[name] = self.ctx.load_kernel(name)
        return self.kern[name]

    def dispatch(self, name, bufs, push, groups):
        B = self.sgq.BufferBinding.buffer
        self.ctx.dispatch(self.k_(name), [B(i, t) for i, t in enumerate(bufs)], push, groups)

    def rms(self, name, x, w, y, rows):  # graph.rs:1602-1621
        self.dispatch(name, [x, w, y], None, [rows, 1, 1])

    def gemv(self, name, w, x, y, rows):
        self.dispatch(name, [w, x, y], None, [rows, 1, 1])

    def record_layer(self, l, kv):
        """graph.rs:478-656, dispatch by dispatch."""
        kind = "g" if l % 2 == 1 else "s"
        sliding = kind == "s"
        hd, n_kv = (256, 16) if sliding else (512, 4)
        W = lambda n: self.w[(n, l)]  # noqa: E731
        q_raw, q, kp, k, v = self.q_raw[kind], self.q[kind], self.kp[kind], self.k[kind], self.v[kind]
        rms_hd = "rmsnorm_256" if sliding else "rmsnorm_512"
        rope_q, rope_k = ("rope_sliding_q", "rope_sliding_k") if sliding else \
            ("rope_global_q", "rope_global_k")
        cs = self.cs[kind]
        wo = "gemv_q4_0_k8192" if sliding else "gemv_q4_0_k16384"
        # attention block
        self.rms("rmsnorm_5376", self.x, W("attn_norm"), self.xn, 1)
        self.gemv("gemv_q4_0_k5376", W("attn_q"), self.xn, q_raw, self.qd[kind])
        self.gemv("gemv_q4_0_k5376", W("attn_k"), self.xn, kp, self.kvd[kind])
        if sliding:
            self.gemv("gemv_q4_0_k5376", W("attn_v"), self.xn, self.vp_sl, self.kvd[kind])
            vp = self.vp_sl
        else:
            vp = kp
        self.rms(rms_hd, q_raw, W("attn_q_norm"), q, 32)
        self.rms(rms_hd, kp, W("attn_k_norm"), k, n_kv)
        self.rms(rms_hd, vp, self.ones, v, n_kv)  # V-norm: weightless
        live = hd // 2 if sliding else hd // 8
        self.dispatch(rope_q, [q, cs], None, [(32 * live + 255) // 256, 1, 1])
        self.dispatch(rope_k, [k, cs], None, [(n_kv * live + 255) // 256, 1, 1])
        kvd = self.kvd[kind]
        if sliding:
            for src, dst in ((k, kv["k"]), (v, kv["v"])):
                self.dispatch("kv_append_sliding", [src, dst, self.step], None,
                              [(kvd + 255) // 256, 1, 1])
        else:
            self.dispatch("kv_append_global_q8", [k, kv["k_scales"], kv["k_quants"], self.step],
                          None, [(kvd // 32 + 63) // 64, 1, 1])
            self.dispatch("kv_append_global", [v, kv["v"], self.step], None,
                          [(kvd + 255) // 256, 1, 1])
        splits = SPLITS_SL if sliding else SPLITS_GL
        push = struct.pack("<If", splits, 1.0)
        if sliding:
            self.dispatch("attn_decode_sliding", [q, kv["k"], kv["v"], self.part[kind], self.step],
                          push, [n_kv, splits, 1])
        else:
            self.dispatch("attn_decode_global_q8k", [q, kv["k_quants"], kv["k_scales"], kv["v"],
                                                     self.part[kind], self.step],
                          push, [n_kv, splits, 1])
        self.dispatch("attn_reduce_d256" if sliding else "attn_reduce_d512",
                      [self.part[kind], self.attn[kind]], struct.pack("<I", splits), [32, 1, 1])
        self.gemv(wo, W("attn_output"), self.attn[kind], self.o, H)
        self.rms("rmsnorm_5376", self.o, W("post_attention_norm"), self.on, 1)
        self.dispatch("add_scaled", [self.x, self.on, self.x2], struct.pack("<f", 1.0),
                      [(H + 255) // 256, 1, 1])
        # FFN block
        self.rms("rmsnorm_5376", self.x2, W("ffn_norm"), self.fin, 1)
        for wn, dst in (("ffn_gate", self.g), ("ffn_up", self.u)):
            self.gemv("gemv_q4_0_k5376", W(wn), self.fin, dst, F)
        self.dispatch("geglu", [self.g, self.u, self.gu], None, [(F + 255) // 256, 1, 1])
        self.gemv("gemv_q4_0_k21504", W("ffn_down"), self.gu, self.f, H)
        self.rms("rmsnorm_5376", self.f, W("post_ffw_norm"), self.fn2, 1)
        self.dispatch("add_scaled", [self.x2, self.fn2, self.x], struct.pack("<f", self.scale[l]),
                      [(H + 255) // 256, 1, 1])


def _caches(oracle, rng):
    """Device pages for P0 cached positions and the rows the oracle sees."""
    kvd_s, kvd_g = 16 * 256, 4 * 512
    ring_k = oracle.f32_to_f16_bits(rng.f32_vec(RING * kvd_s) * np.float32(0.5))
    ring_v = oracle.f32_to_f16_bits(rng.f32_vec(RING * kvd_s))
    cap = P0 + 8
    gk = rng.f32_vec(cap * kvd_g) * np.float32(0.5)
    gks, gkq = oracle.quant_q8_0(gk)
    gv = oracle.f32_to_f16_bits(rng.f32_vec(cap * kvd_g))
    dev_kv = [{"k": dev(ring_k), "v": dev(ring_v)},
              {"k_quants": dev(gkq), "k_scales": dev(gks), "v": dev(gv)}]
    rk = oracle.f16_bits_to_f32(ring_k).reshape(RING, kvd_s)
    rv = oracle.f16_bits_to_f32(ring_v).reshape(RING, kvd_s)
    zero = np.zeros(kvd_s, np.float32)
    # positions older than the window are never attended: zero rows stand in
    k0 = [rk[p % RING].copy() if p >= P0 - RING else zero for p in range(P0)]
    v0 = [rv[p % RING].copy() if p >= P0 - RING else zero for p in range(P0)]
    gkd = oracle.dequant_q8_0(gks, gkq).reshape(cap, kvd_g)
    gvd = oracle.f16_bits_to_f32(gv).reshape(cap, kvd_g)
    k1 = [gkd[p].copy() for p in range(P0)]
    v1 = [gvd[p].copy() for p in range(P0)]
    return dev_kv, ([k0, k1], [v0, v1])


@pytest.mark.timeout(600)
def test_record_layer_by_name_matches_oracle(ctx, oracle):
    import sgq
    from oracle.model import F16Graph, OracleDecoder

    print("record_layer by name: one sliding + one global layer, released geometry", flush=True)
    cfg = _cfg(sgq)
    model = sgq.Model(ctx, cfg)
    d = cfg.as_dict()
    wts = _weights(model, d)
    model.close()
    rng = oracle.Rng(0x1A8)
    dev_kv, (kc, vc) = _caches(oracle, rng)

    x0s = [oracle.f32_to_f16_bits(rng.f32_vec(H) * np.float32(2.0)) for _ in range(3)]

    class Staged:
        step_x = None

        def _embed(self, token):
            return oracle.f16_bits_to_f32(self.step_x)

    class Ref16(Staged, F16Graph):
        pass

    class Ref32(Staged, OracleDecoder):
        _cache_rows = F16Graph._cache_rows

    refs = [Ref16(d, wts), Ref32(d, wts)]
    for r in refs:
        r.threads = 16
        r.taps = {}
        r.k_cache = [list(c) for c in kc]
        r.v_cache = [list(c) for c in vc]
        r.pos = P0

    gr = _Graph(ctx, sgq, wts, cfg)
    s = torch.cuda.Stream()
    ctx.set_stream(s)
    try:
        # one eager pass over throwaway pages first: every kernel's one-time
        # launch set-up happens outside the capture
        scratch = [{"k": torch.zeros_like(dev_kv[0]["k"]), "v": torch.zeros_like(dev_kv[0]["v"])},
                   {n: torch.zeros_like(t) for n, t in dev_kv[1].items()}]
        ctx.step_write(gr.step, sgq.StepState(0, 1, 1, 0))
        for l in range(2):
            gr.record_layer(l, scratch[l])
        ctx.synchronize()
        del scratch
        graphs = []
        for l in range(2):
            with sgq.GraphRecorder(ctx) as rec:
                gr.record_layer(l, dev_kv[l])
            graphs.append(rec.graph)
        ctx.synchronize()
        gl = refs[0].global_factors
        for i, x0 in enumerate(x0s):
            pos = P0 + i
            # stage_token (graph.rs:1487-1529): residual row, step, rope tables
            gr.x.copy_(torch.from_numpy(x0.view(np.int16)))
            cs_s = oracle.cos_sin_table([pos], 256, d["rope_theta_sliding"])
            cs_g = oracle.cos_sin_table([pos], 512, d["rope_theta_global"], gl)[:, :64, :]
            gr.cs["s"].copy_(torch.from_numpy(np.ascontiguousarray(cs_s).reshape(-1)))
            gr.cs["g"].copy_(torch.from_numpy(np.ascontiguousarray(cs_g).reshape(-1)))
            torch.cuda.synchronize()
            ctx.step_write(gr.step, sgq.StepState(pos, min(pos + 1, RING), pos + 1, 0))
            got = []
            for g in graphs:
                g.submit()
                ctx.synchronize()
                got.append(oracle.f16_bits_to_f32(host(gr.x, np.uint16)))
            for r in refs:
                r.step_x = x0
                r.decode(0)
            for l in range(2):
                e16 = rel_err(got[l], refs[0].taps[("x_layer", l)])
                e32 = rel_err(got[l], refs[1].taps[("x_layer", l)])
                print(f"  pos {pos} layer {l}: vs f16 graph {e16:.2e}, vs fp32 {e32:.2e}",
                      flush=True)
                assert e16 <= 4e-3, (pos, l, e16)
                assert e32 <= 1e-2, (pos, l, e32)
            # the appended K/V rows are the oracle's, in the graph's page formats
            kr = host(dev_kv[0]["k"], np.uint16).reshape(RING, 4096)[pos % RING]
            want = refs[0].k_cache[0][pos]
            assert rel_err(oracle.f16_bits_to_f32(kr), want) <= 2e-3, pos
    finally:
        ctx.set_stream(None)
