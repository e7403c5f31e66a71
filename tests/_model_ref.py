"""CPU reference of one greedy decode step, assembled from oracle functions
in the reference's op order and kernel selection (cuda/layer.rs:99-709,
1210-1456, 2125-2259; matmul.rs:96-104 gemv_n_split for the single-pass vs
split-K choice)."""
import numpy as np

import oracle
from taraference_amd import synth


def n_split(k):
    return 1 if (k < 4096 and 4 * k <= 24 * 1024) else 4


class RefModel:
    def __init__(self, cfg, layers, embedding, max_seq):
        self.c = cfg
        self.L = layers
        self.E, self.ecb = embedding
        self.Ec, self.eccb = synth.q6k_compact(self.E, cfg["n_embd"])
        stride = cfg["n_kv"] * cfg["head_dim"]
        self.K = [np.zeros((max_seq, stride), np.uint16) for _ in layers]
        self.V = [np.zeros((max_seq, stride), np.uint16) for _ in layers]
        self.comp = {}

    def _q8(self, x):
        return oracle.quantize_q8(x)

    def _global_q8(self, wm, n_rows, x, q6k, out=None):
        """try_gemv_global_q8 with the reference's kernel choice."""
        w, cb = wm
        n_cols = w.shape[0]
        q8, d8 = self._q8(x)
        ns = n_split(n_rows)
        use_res = 0 if out is None else 2
        if q6k:
            key = id(w)
            if key not in self.comp:
                self.comp[key] = synth.q6k_compact(w, n_rows)
            comp, ccb = self.comp[key]
            if ns >= 4:
                return oracle.gemv_q6k_compact_q8_kway(comp, q8, d8, n_rows, n_cols, ccb,
                                                       8 if n_rows >= 4096 else 4,
                                                       use_res=use_res, out=out)
            return oracle.gemv_q6k_compact_q8(comp, q8, d8, n_rows, n_cols, ccb,
                                              use_res=use_res, out=out)
        if ns > 1:
            part = oracle.gemv_q4k_q8_splitk(w, q8, d8, n_rows, n_cols, cb, ns)
            return oracle.gemv_splitk_reduce(part, n_cols, ns, use_res=use_res, out=out)
        return oracle.gemv_q4k_q8(w, q8, d8, n_rows, n_cols, cb, use_res=use_res, out=out)

    def step(self, token, pos):
        c = self.c
        e, hd = c["n_embd"], c["head_dim"]
        nq, nkv = c["n_head"] * hd, c["n_kv"] * hd
        x = oracle.embed_row(self.E, 210, token, e, self.ecb)
        scale = float(np.float32(1.0 / np.sqrt(hd)))
        for li, L in enumerate(self.L):
            xb = oracle.rms_norm(x, L["attn_norm"], c["rms_eps"])
            q8, d8 = self._q8(xb)
            wq, cb = L["wq"]
            q, k = oracle.gemv_q4k_pair(wq, L["wk"][0], q8, d8, e, nq, nkv, cb, L["bq"], L["bk"])
            v = oracle.gemv_q6k_f32(L["wv"][0], xb, e, nkv, L["wv"][1], bias=L["bv"])
            q = oracle.rope_neox(q, c["n_head"], hd, pos, c["rope_theta"])
            k = oracle.rope_neox(k, c["n_kv"], hd, pos, c["rope_theta"])
            self.K[li][pos] = oracle.f32_to_f16(k)
            self.V[li][pos] = oracle.f32_to_f16(v)
            part = oracle.flash_partial(q, self.K[li], self.V[li], c["n_head"], c["n_kv"], hd,
                                        pos, 8, scale)
            att = oracle.flash_reduce(part, c["n_head"], hd, 8)
            x = self._global_q8(L["wo"], nq, att, False, out=x)
            xb = oracle.rms_norm(x, L["ffn_norm"], c["rms_eps"])
            q8, d8 = self._q8(xb)
            g, gcb = L["gate"]
            h = oracle.gemv_q4k_ffn(g, L["up"][0], q8, d8, e, c["n_ff"], gcb, 1)
            x = self._global_q8(L["down"], c["n_ff"], h, L["down_q6k"], out=x)
        xb = oracle.rms_norm(x, np.ones(e, np.float32), c["rms_eps"])
        logits = self._global_q8((self.E, self.ecb), e, xb, True)
        return logits, oracle.argmax(logits)

    def prefill(self, tokens, pos0=0):
        """The n_tok-row prompt forward (forward.rs:42-71, layer.rs with
        n_tok > 1): f32 GEMMs (kernels/gemm.cu), add_bias, rope, copy_kv,
        prefill attention (attn/fast_v2.cu), GEMM + add for wo and down,
        silu_mul; then the decode head on the last row.  Fills the K/V rows
        pos0 .. pos0+n-1; returns (logits, argmax) of the last token."""
        c = self.c
        e, hd, F = c["n_embd"], c["head_dim"], c["n_ff"]
        nq, nkv = c["n_head"] * hd, c["n_kv"] * hd
        T = len(tokens)
        scale = float(np.float32(1.0 / np.sqrt(hd)))
        x = np.stack([oracle.embed_row(self.E, 210, int(t), e, self.ecb) for t in tokens])

        def rows_norm(a, w):
            return np.stack([oracle.rms_norm(r, w, c["rms_eps"]) for r in a])

        def gemm(wm, a, n_rows, q6k):
            w, cb = wm
            fn = oracle.gemm_q6k if q6k else oracle.gemm_q4k
            return fn(w, np.ascontiguousarray(a, np.float32), n_rows, w.shape[0], cb, a.shape[0])

        for li, L in enumerate(self.L):
            xb = rows_norm(x, L["attn_norm"])
            q = gemm(L["wq"], xb, e, False)
            k = gemm(L["wk"], xb, e, False)
            v = gemm(L["wv"], xb, e, True)
            if L.get("bq") is not None:
                q = q + L["bq"]
                k = k + L["bk"]
                v = v + L["bv"]
            for t in range(T):
                q[t] = oracle.rope_neox(q[t], c["n_head"], hd, pos0 + t, c["rope_theta"])
                k[t] = oracle.rope_neox(k[t], c["n_kv"], hd, pos0 + t, c["rope_theta"])
                self.K[li][pos0 + t] = oracle.f32_to_f16(k[t])
                self.V[li][pos0 + t] = oracle.f32_to_f16(v[t])
            att = oracle.attn_prefill(q, self.K[li], self.V[li], c["n_head"], c["n_kv"], hd,
                                      pos0, T, scale)
            x = (x + gemm(L["wo"], att, nq, False)).astype(np.float32)
            xb = rows_norm(x, L["ffn_norm"])
            g = gemm(L["gate"], xb, e, False)
            u = gemm(L["up"], xb, e, False)
            with np.errstate(over="ignore"):  # exp(-g) = inf -> silu 0, as __expf
                h = ((g / (np.float32(1) + np.exp(-g))) * u).astype(np.float32)
            x = (x + gemm(L["down"], h, F, L["down_q6k"])).astype(np.float32)
        xb = oracle.rms_norm(x[-1], np.ones(e, np.float32), c["rms_eps"])
        logits = self._global_q8((self.E, self.ecb), e, xb, True)
        return logits, oracle.argmax(logits)


class RefModelMixed:
    """CPU reference decode step for any mix of Q4_K / Q6_K / Q5_0 / Q8_0
    matrices ((bytes, col_bytes, ggml type) tuples), assembled in the
    reference's operator order with its kernel choices as the runtime's path
    0 makes them (matmul.rs try_gemv_qkv -> try_gemv_pair / Q5_0 dual ->
    gemv; try_gemv_global_q8 for Q4_K / Q6_K / Q8_0, the f32 GEMV for
    Q5_0; gate/up fused for Q4_K, else two GEMVs and silu_mul)."""

    def __init__(self, cfg, layers, embedding, max_seq, output_norm=None):
        self.c = cfg
        self.L = layers
        self.E = embedding
        self.onorm = (np.ones(cfg["n_embd"], np.float32) if output_norm is None
                      else np.asarray(output_norm, np.float32))
        stride = cfg["n_kv"] * cfg["head_dim"]
        self.K = [np.zeros((max_seq, stride), np.uint16) for _ in layers]
        self.V = [np.zeros((max_seq, stride), np.uint16) for _ in layers]
        self.comp = {}

    def _embed(self, token):
        from _util import q5_0_dequant, q8_0_dequant
        w, cb, ty = self.E
        e = self.c["n_embd"]
        row = np.ascontiguousarray(w[token])
        if ty in (12, 14):
            return oracle.embed_row(w, 144 if ty == 12 else 210, token, e, cb)
        bb = 34 if ty == 8 else 22
        deq = q8_0_dequant if ty == 8 else q5_0_dequant
        return deq(row[: (e // 32) * bb].reshape(-1, bb)).reshape(-1).astype(np.float32)

    def _q8(self, wm, n_rows, x, bias=None, out=None):
        """try_gemv_global_q8 (quantize x once, the Q8 GEMV)."""
        w, cb, ty = wm
        n_cols = w.shape[0]
        q8, d8 = oracle.quantize_q8(x)
        use_res = 0 if out is None else 2
        if ty == 8:
            return oracle.gemv_q8_0_q8(w, q8, d8, n_rows, n_cols, cb, bias=bias, use_res=use_res,
                                       out=out)
        if ty == 14:
            key = id(w)
            if key not in self.comp:
                self.comp[key] = synth.q6k_compact(w, n_rows)
            comp, ccb = self.comp[key]
            if n_split(n_rows) >= 4:
                return oracle.gemv_q6k_compact_q8_kway(comp, q8, d8, n_rows, n_cols, ccb,
                                                       8 if n_rows >= 4096 else 4, bias=bias,
                                                       use_res=use_res, out=out)
            return oracle.gemv_q6k_compact_q8(comp, q8, d8, n_rows, n_cols, ccb, bias=bias,
                                              use_res=use_res, out=out)
        ns = n_split(n_rows)
        if ns > 1:
            part = oracle.gemv_q4k_q8_splitk(w, q8, d8, n_rows, n_cols, cb, ns)
            return oracle.gemv_splitk_reduce(part, n_cols, ns, bias=bias, use_res=use_res, out=out)
        return oracle.gemv_q4k_q8(w, q8, d8, n_rows, n_cols, cb, bias=bias, use_res=use_res,
                                  out=out)

    def _gemv(self, wm, n_rows, x, bias=None, out=None):
        """try_gemv_global_q8, else the f32-activation GEMV (matmul.rs:118)."""
        w, cb, ty = wm
        if ty in (12, 8) or ty == 14:
            return self._q8(wm, n_rows, x, bias, out)
        use_res = 0 if out is None else 2
        return oracle.gemv_q5_0_f32(w, x, n_rows, w.shape[0], cb, bias=bias, use_res=use_res,
                                    out=out)

    def _f32_gemv(self, wm, n_rows, x, bias=None):
        """gemv(): the f32-activation kernels (Q8_0 quantizes x inside)."""
        w, cb, ty = wm
        if ty == 14:
            return oracle.gemv_q6k_f32(w, x, n_rows, w.shape[0], cb, bias=bias)
        if ty == 6:
            return oracle.gemv_q5_0_f32(w, x, n_rows, w.shape[0], cb, bias=bias)
        return self._q8(wm, n_rows, x, bias)

    def step(self, token, pos):
        c = self.c
        e, hd, F = c["n_embd"], c["head_dim"], c["n_ff"]
        nq = c["n_head"] * hd
        scale = float(np.float32(1.0 / np.sqrt(hd)))
        x = self._embed(token)
        for li, L in enumerate(self.L):
            xb = oracle.rms_norm(x, L["attn_norm"], c["rms_eps"])
            tq, tk, tv = L["wq"][2], L["wk"][2], L["wv"][2]
            if tq == tk == tv and tq in (6, 8):
                q = self._gemv(L["wq"], e, xb, L["bq"]) if tq == 6 else self._q8(L["wq"], e, xb, L["bq"])
                k = self._gemv(L["wk"], e, xb, L["bk"]) if tq == 6 else self._q8(L["wk"], e, xb, L["bk"])
                v = self._gemv(L["wv"], e, xb, L["bv"]) if tq == 6 else self._q8(L["wv"], e, xb, L["bv"])
            else:
                q = self._gemv(L["wq"], e, xb, L["bq"])
                k = self._gemv(L["wk"], e, xb, L["bk"])
                v = self._f32_gemv(L["wv"], e, xb, L["bv"])
            q = oracle.rope_neox(q, c["n_head"], hd, pos, c["rope_theta"])
            k = oracle.rope_neox(k, c["n_kv"], hd, pos, c["rope_theta"])
            self.K[li][pos] = oracle.f32_to_f16(k)
            self.V[li][pos] = oracle.f32_to_f16(v)
            part = oracle.flash_partial(q, self.K[li], self.V[li], c["n_head"], c["n_kv"], hd,
                                        pos, 8, scale)
            att = oracle.flash_reduce(part, c["n_head"], hd, 8)
            x = self._gemv(L["wo"], nq, att, out=x)
            xb = oracle.rms_norm(x, L["ffn_norm"], c["rms_eps"])
            if L["gate"][2] == 12 and L["up"][2] == 12:
                q8, d8 = oracle.quantize_q8(xb)
                h = oracle.gemv_q4k_ffn(L["gate"][0], L["up"][0], q8, d8, e, F, L["gate"][1], 1)
            else:
                g = self._f32_gemv(L["gate"], e, xb)
                u = self._f32_gemv(L["up"], e, xb)
                with np.errstate(over="ignore"):
                    h = ((g / (np.float32(1) + np.exp(-g))) * u).astype(np.float32)
            x = self._gemv(L["down"], F, h, out=x)
        xb = oracle.rms_norm(x, self.onorm, c["rms_eps"])
        self.head_x = xb  # the lm_head input (for flip-aware tolerances)
        logits = self._gemv(self.E, e, xb)
        return logits, oracle.argmax(logits)
