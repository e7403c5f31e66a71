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
