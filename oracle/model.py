"""CPU decoder forward pass of the reference model family, over the oracle's
C primitives.

TEST INFRASTRUCTURE ONLY: the checker for libsgq's decode-step driver
(sgq_model_*), imported by tests/ and ``__graft_entry__.smoke()``.  Never part
of the product path.

Follows crates/sg-model/src/reference.rs:157-316 (ReferenceModel::forward):
  x = dequant(E[token]) * embed_scale            (reference.rs:163-172)
  per layer (reference.rs:184-303):
    xn = rmsnorm(x, attn_norm)
    q = rope(rmsnorm_h(Wq xn, q_norm)); k = rope(rmsnorm_h(Wk xn, k_norm))
    v = rmsnorm_h(Wv xn) weightless; global layers take v from Wk xn
        (attention_k_eq_v, reference.rs:214-222)
    a = attention over the window (sliding) or all keys (global),
        scale attn_scale                         (reference.rs:483-531)
    x += rmsnorm(Wo a, post_attention_norm)
    x += rmsnorm(Wd (gelu_tanh(Wg fn) * Wu fn), post_ffw_norm),
        fn = rmsnorm(x, ffn_norm)
    x *= layer_output_scale
  logits = cap * tanh((E rmsnorm(x, output_norm)) / cap)  (reference.rs:307-316)
One deviation, on purpose, to match the GPU graph instead of the f32 CPU
cache: K and V are stored as Q8_0 pages (kv_quant_q8, crates/sg-gpu/shaders/
kv_quant_q8.wgsl:30-57, recorded by crates/sg-model/src/graph.rs:560-600), so
the oracle round-trips each K/V row through Q8_0 before caching it.
RoPE: NEOX, angles in f64 via cos_sin_table (crates/sg-model/src/rope.rs:
27-48); global layers use divisor factors [1]*live + [1e30]*rest, which is
how partial_rotary_factor materializes (rope.rs:13-16).
Linear layers use CpuModel::matmul's dequant_row + 8-lane f64 dot
(matmul_q4_0); everything is fp32 between ops, as in the reference.
"""
from __future__ import annotations

import math

import numpy as np

from . import oracle as O


class OracleDecoder:
    """``weights``: dict of host arrays keyed like sgq_model_tensor
    ((name, layer) -> array; Q4_0 tensors as uint8 bytes, the rest float32).
    ``cfg``: dict with the sgq_model_config fields."""

    def __init__(self, cfg: dict, weights: dict):
        self.c = cfg
        self.w = weights
        L = cfg["n_layers"]
        self.k_cache = [[] for _ in range(L)]
        self.v_cache = [[] for _ in range(L)]
        self.pos = 0
        # taps[(name, layer)] = the row(s) of the last forward, when a dict:
        # "k_rope" and "v_norm" (reference.rs:153-155 tap names); prefill also
        # leaves ("x_out", -1), the residual rows after the last layer
        self.taps = None
        # kv_source(layer, pos, k_row, v_row) -> (k_row, v_row): the Q8_0
        # round-tripped rows decode() caches, replaceable by the caller (a
        # test hands in the device's own pages, so that a rounding flip of a
        # quant near a rounding boundary does not make the two caches differ)
        self.kv_source = None
        hd_g = cfg.get("head_dim_global") or cfg["head_dim"]
        live = int(round(cfg["global_rope_frac"] * hd_g / 2))
        self.global_factors = np.array([1.0] * live + [1e30] * (hd_g // 2 - live), np.float32)

    def preload_cache(self, pages: dict, n_tokens: int):
        """Start from a filled context: ``pages[(layer, "k"|"v")]`` = (scales,
        quants) of the device cache pages.  Global layers hold position p at
        slot p; ring layers at slot p % slots (positions older than the ring
        are never attended)."""
        c = self.c
        for l in range(c["n_layers"]):
            hd, nkv = self.geometry(l)
            for kind, cache in (("k", self.k_cache), ("v", self.v_cache)):
                sc, q = pages[(l, kind)]
                rows = O.dequant_q8_0(sc, q).reshape(-1, nkv * hd)
                slots = rows.shape[0]
                cache[l] = [rows[p % slots].copy() for p in range(n_tokens)]
        self.pos = n_tokens

    def is_global(self, layer: int) -> bool:
        ge = self.c["global_every"]
        return layer % ge == ge - 1

    def geometry(self, layer: int):
        """(head_dim, n_kv_heads) of the layer's kind: the global kind may
        differ (the real checkpoint: sliding 256 x 16, global 512 x 4;
        crates/sg-gguf/src/desc.rs:66-93)."""
        c = self.c
        if self.is_global(layer):
            return (c.get("head_dim_global") or c["head_dim"],
                    c.get("n_kv_heads_global") or c["n_kv_heads"])
        return c["head_dim"], c["n_kv_heads"]

    def _embed_rows(self, tokens):
        """Dequantized embedding rows: Q4_0, or Q6_K rows at the device's
        padded stride (q6_k.rs:41-62)."""
        c, H = self.c, self.c["hidden"]
        emb = self.w[("token_embd", -1)]
        if c.get("embed_q6k"):
            stride = ((H // 256) * 210 + 15) // 16 * 16
            return np.stack([O.q6_k_dequant(emb[t * stride:(t + 1) * stride], 1, H, stride)[0]
                             for t in tokens])
        rb = (H // 32) * 18
        return np.stack([O.q4_0_dequant(emb[t * rb:(t + 1) * rb], 1, H)[0] for t in tokens])

    def _head(self, xf):
        """Tied LM head with the softcap (reference.rs:307-316)."""
        c, H = self.c, self.c["hidden"]
        emb = self.w[("token_embd", -1)]
        if c.get("embed_q6k"):
            stride = ((H // 256) * 210 + 15) // 16 * 16
            logits = O.gemv_q6_k_logits(emb, stride, xf, c["vocab"], H, softcap=0.0)
        else:
            logits = O.matmul_q4_0(emb, xf, 1, c["vocab"], H, threads=self.threads)[0]
        cap = np.float64(c["final_softcap"])
        return (cap * np.tanh(logits.astype(np.float64) / cap)).astype(np.float32)

    def _embed(self, token: int) -> np.ndarray:
        """The residual row a decode step starts from (reference.rs:163-172)."""
        row = self._embed_rows([token])[0]
        return (row * np.float32(math.sqrt(self.c["hidden"]))).astype(np.float32)

    # host threads of the row-parallel matmul (results do not depend on it)
    threads = 8

    def _lin(self, name, layer, x, n_out):
        """CpuModel::matmul over one token (reference.rs:402-444): the same
        dequant_row + 8-lane dot_f64 as the prefill's multi-token matmul, so a
        token-by-token decode reproduces a multi-token forward bit for bit."""
        k = x.size
        return O.matmul_q4_0(self.w[(name, layer)], x, 1, n_out, k, threads=self.threads)[0]

    def _q8_round_trip(self, row):
        s, q = O.quant_q8_0(row)
        return O.dequant_q8_0(s, q)

    def _act(self, x):
        """Storage of an activation buffer between two operators: fp32 here
        (reference.rs); F16Graph rounds to f16 as the GPU graph's buffers do."""
        return x

    def _cache_rows(self, layer, k, v):
        """The K/V rows a layer's cache holds for the new position: Q8_0 round
        trips of both (the page format the oracle's caches model)."""
        return self._q8_round_trip(k), self._q8_round_trip(v)

    def decode(self, token: int) -> np.ndarray:
        c, w = self.c, self.w
        H, F = c["hidden"], c["ffn"]
        nq = c["n_q_heads"]
        eps = c["eps"]
        x = self._embed(token)
        pos = self.pos
        A = self._act
        for l in range(c["n_layers"]):
            glob = self.is_global(l)
            hd, nkv = self.geometry(l)
            xn = A(O.rmsnorm(x, w[("attn_norm", l)], H, eps))
            q = A(self._lin("attn_q", l, xn, nq * hd))
            k_proj = A(self._lin("attn_k", l, xn, nkv * hd))
            if glob and c["global_k_eq_v"]:
                v = k_proj.copy()
            else:
                v = A(self._lin("attn_v", l, xn, nkv * hd))
            if glob:
                cs = O.cos_sin_table([pos], hd, c["rope_theta_global"], self.global_factors)
            else:
                cs = O.cos_sin_table([pos], hd, c["rope_theta_sliding"])
            q = A(O.rmsnorm(q, w[("attn_q_norm", l)], hd, eps))
            q = A(O.rope(q, hd, hd, nq, cs))
            k = A(O.rmsnorm(k_proj, w[("attn_k_norm", l)], hd, eps))
            k = A(O.rope(k, hd, hd, nkv, cs))
            v = A(O.rmsnorm(v, None, hd, eps))
            if self.taps is not None:
                self.taps[("k_rope", l)], self.taps[("v_norm", l)] = k, v
            kr, vr = self._cache_rows(l, k, v)
            if self.kv_source is not None:
                kr, vr = self.kv_source(l, pos, kr, vr)
            self.k_cache[l].append(kr)
            self.v_cache[l].append(vr)
            ck = np.concatenate(self.k_cache[l])
            cv = np.concatenate(self.v_cache[l])
            window = None if glob else c["sliding_window"]
            a = A(O.attention(q, ck, cv, 1, pos, nq, nkv, hd, window, c["attn_scale"]).reshape(-1))
            o = A(self._lin("attn_output", l, a, H))
            o = A(O.rmsnorm(o, w[("post_attention_norm", l)], H, eps))
            x = A((x + o).astype(np.float32))
            fn = A(O.rmsnorm(x, w[("ffn_norm", l)], H, eps))
            g = A(self._lin("ffn_gate", l, fn, F))
            u = A(self._lin("ffn_up", l, fn, F))
            h = A(O.geglu(g, u))
            f = A(self._lin("ffn_down", l, h, H))
            f = A(O.rmsnorm(f, w[("post_ffw_norm", l)], H, eps))
            x = (x + f).astype(np.float32)
            x = A((x * w[("layer_output_scale", l)][0]).astype(np.float32))
            if self.taps is not None:
                self.taps[("x_layer", l)] = x
        self.pos += 1
        xf = O.rmsnorm(x, w[("output_norm", -1)], H, eps)
        return self._head(xf)


class F16Graph(OracleDecoder):
    """The decode forward as the reference's GPU graph stores it
    (crates/sg-model/src/graph.rs:478-729): every activation buffer between
    two operators is f16 (graph.rs:282-313), so each operator's fp32 result
    is rounded to f16 before the next reads it; the caches hold K and V as
    record_layer appends them: f16 rows on sliding layers, Q8_0 K and f16 V
    on global layers (graph.rs:581-611).  Operators themselves are the
    oracle's (f32/f64, reference.rs)."""

    def _act(self, x):
        return O.through_f16(x)

    def _cache_rows(self, layer, k, v):
        if self.is_global(layer):
            return self._q8_round_trip(k), v.copy()
        return k.copy(), v.copy()


class OraclePrefill(OracleDecoder):
    """Prefill of a token chunk (crates/sg-model/src/graph.rs:1451-1482 with
    the MMQ record_prefill_layer path): every linear layer sees its input
    round-tripped through Q8_0 (kv_quant_q8 semantics, per row, 32-blocks),
    as the reference quantizes activations before its int8 MMQs; attention
    is causal (window on sliding layers) over the cached positions plus the
    chunk.  Decoding after it continues with the inherited decode().

    ``q8_activations = False`` skips those activation round trips: the
    forward is then ReferenceModel::forward over several tokens (f32
    activations, reference.rs:157-316), which a token-by-token decode must
    reproduce bit for bit (crates/sg-model/tests/cpu_reference.rs:84-92)."""

    q8_activations = True

    def _q8rt(self, x2d):
        if not self.q8_activations:
            return np.ascontiguousarray(x2d, np.float32)
        s, q = O.quant_q8_0(np.ascontiguousarray(x2d, np.float32).reshape(-1))
        return O.dequant_q8_0(s, q).reshape(x2d.shape)

    def _mm(self, name, layer, x2d, n_out):
        M, K = x2d.shape
        return O.matmul_q4_0(self.w[(name, layer)], x2d, M, n_out, K, threads=self.threads)

    def prefill(self, tokens) -> np.ndarray:
        c, w = self.c, self.w
        H, F = c["hidden"], c["ffn"]
        nq = c["n_q_heads"]
        eps = c["eps"]
        M = len(tokens)
        q0 = self.pos
        x = self._embed_rows(tokens)
        x = (x * np.float32(math.sqrt(H))).astype(np.float32)
        pos = np.arange(q0, q0 + M, dtype=np.uint32)
        hd_g = c.get("head_dim_global") or c["head_dim"]
        cs_sl = O.cos_sin_table(pos, c["head_dim"], c["rope_theta_sliding"])
        cs_gl = O.cos_sin_table(pos, hd_g, c["rope_theta_global"], self.global_factors)
        for l in range(c["n_layers"]):
            glob = self.is_global(l)
            hd, nkv = self.geometry(l)
            xn = self._q8rt(O.rmsnorm(x, w[("attn_norm", l)], H, eps))
            q = self._mm("attn_q", l, xn, nq * hd)
            k_proj = self._mm("attn_k", l, xn, nkv * hd)
            v = k_proj.copy() if glob and c["global_k_eq_v"] else self._mm("attn_v", l, xn, nkv * hd)
            cs = cs_gl if glob else cs_sl
            q = O.rope(O.rmsnorm(q, w[("attn_q_norm", l)], hd, eps), hd, hd, nq, cs)
            k = O.rope(O.rmsnorm(k_proj, w[("attn_k_norm", l)], hd, eps), hd, hd, nkv, cs)
            v = O.rmsnorm(v, None, hd, eps)
            if self.taps is not None:
                self.taps[("k_rope", l)], self.taps[("v_norm", l)] = k, v
            for i in range(M):
                kr, vr = self._q8_round_trip(k[i]), self._q8_round_trip(v[i])
                if self.kv_source is not None:
                    kr, vr = self.kv_source(l, q0 + i, kr, vr)
                self.k_cache[l].append(kr)
                self.v_cache[l].append(vr)
            ck = np.concatenate(self.k_cache[l])
            cv = np.concatenate(self.v_cache[l])
            window = None if glob else c["sliding_window"]
            a = O.attention(q, ck, cv, M, q0, nq, nkv, hd, window, c["attn_scale"])
            o = self._mm("attn_output", l, self._q8rt(a.reshape(M, nq * hd)), H)
            x = (x + O.rmsnorm(o, w[("post_attention_norm", l)], H, eps)).astype(np.float32)
            fn = self._q8rt(O.rmsnorm(x, w[("ffn_norm", l)], H, eps))
            g = self._mm("ffn_gate", l, fn, F)
            u = self._mm("ffn_up", l, fn, F)
            f = self._mm("ffn_down", l, self._q8rt(O.geglu(g, u)), H)
            x = (x + O.rmsnorm(f, w[("post_ffw_norm", l)], H, eps)).astype(np.float32)
            x = (x * w[("layer_output_scale", l)][0]).astype(np.float32)
        self.pos += M
        if self.taps is not None:
            self.taps[("x_out", -1)] = x
        xf = O.rmsnorm(x[-1], w[("output_norm", -1)], H, eps)
        return self._head(xf)


LAYER_TENSORS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
                 "attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm",
                 "post_ffw_norm", "layer_output_scale")
