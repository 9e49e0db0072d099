"""Independent numpy (float64) implementation of the pieces the C oracle
restates, written from the GGUF block specs and the textbook formulas rather
than from the oracle's code, so that a mistake in either one shows up as a
disagreement. Used only by tests.
"""
from __future__ import annotations

import struct

import numpy as np

Q8_0, Q4_K, F32 = 8, 12, 0


def f16_to_f64(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float64)


def dequant_q8_0(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    blk = np.asarray(raw, dtype=np.uint8).reshape(rows, k // 32, 34)
    d = f16_to_f64(blk[:, :, 0:2].copy().view(np.uint16)[..., 0])
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)
    return (d[..., None] * q).reshape(rows, k)


def q4k_scales(sc12: np.ndarray):
    """sc12: [..., 12] uint8 -> (sc[..., 8], m[..., 8]) per the GGUF K-quant packing."""
    s = sc12.astype(np.int64)
    sc = np.empty(s.shape[:-1] + (8,), dtype=np.int64)
    m = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def dequant_q4_k(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    blk = np.asarray(raw, dtype=np.uint8).reshape(rows, k // 256, 144)
    hdr = blk[:, :, 0:4].copy().view(np.uint16)
    d = f16_to_f64(hdr[..., 0])
    dmin = f16_to_f64(hdr[..., 1])
    sc, m = q4k_scales(blk[:, :, 4:16])
    qs = blk[:, :, 16:].reshape(rows, k // 256, 4, 32)
    lo = qs & 0xF
    hi = qs >> 4
    q = np.stack([lo, hi], axis=3).reshape(rows, k // 256, 8, 32).astype(np.float64)  # sub-block 2g, 2g+1
    y = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * m[..., None]
    return y.reshape(rows, k)


def dequant_q5_k(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """GGUF Q5_K: [d f16, dmin f16, scales 12, qh 32, qs 128]; the value of element
    32 s + l is d sc_s (nibble + 16 * (bit s of qh[l])) - dmin m_s."""
    blk = np.asarray(raw, dtype=np.uint8).reshape(rows, k // 256, 176)
    hdr = blk[:, :, 0:4].copy().view(np.uint16)
    d, dmin = f16_to_f64(hdr[..., 0]), f16_to_f64(hdr[..., 1])
    sc, m = q4k_scales(blk[:, :, 4:16])
    qh = blk[:, :, 16:48].astype(np.int64)                         # [.., l]
    qs = blk[:, :, 48:].reshape(rows, k // 256, 4, 32)
    nib = np.stack([qs & 0xF, qs >> 4], axis=3).reshape(rows, k // 256, 8, 32).astype(np.int64)
    hi = (qh[:, :, None, :] >> np.arange(8)[None, None, :, None]) & 1  # [.., s, l]
    q = (nib + 16 * hi).astype(np.float64)
    y = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * m[..., None]
    return y.reshape(rows, k)


def dequant_q6_k(raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """GGUF Q6_K: [ql 128, qh 64, scales int8 16, d f16]; element 128 n + 32 g + l
    has the nibble (g // 2) of ql[64 n + 32 (g % 2) + l] and bits 2g..2g+1 of
    qh[32 n + l] on top, value d * scales[e // 16] * (q - 32)."""
    blk = np.asarray(raw, dtype=np.uint8).reshape(rows, k // 256, 210)
    ql = blk[:, :, :128].reshape(rows, k // 256, 2, 2, 32).astype(np.int64)   # [n, g%2, l]
    qh = blk[:, :, 128:192].reshape(rows, k // 256, 2, 32).astype(np.int64)   # [n, l]
    sc = blk[:, :, 192:208].view(np.int8).astype(np.float64)                 # [16]
    d = f16_to_f64(blk[:, :, 208:210].copy().view(np.uint16)[..., 0])
    q = np.empty((rows, k // 256, 2, 4, 32), dtype=np.int64)
    for g in range(4):
        nib = (ql[:, :, :, g % 2, :] >> (4 * (g // 2))) & 0xF
        q[:, :, :, g, :] = nib | (((qh >> (2 * g)) & 3) << 4)
    q = (q - 32).reshape(rows, k // 256, 256).astype(np.float64)
    s = np.repeat(sc, 16, axis=-1)
    return (d[..., None] * s * q).reshape(rows, k)


def dequant(qtype: int, raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    if qtype == Q8_0:
        return dequant_q8_0(raw, rows, k)
    if qtype == Q4_K:
        return dequant_q4_k(raw, rows, k)
    if qtype == 13:
        return dequant_q5_k(raw, rows, k)
    if qtype == 14:
        return dequant_q6_k(raw, rows, k)
    if qtype == F32:
        return np.asarray(raw, dtype=np.uint8).view(np.float32).astype(np.float64).reshape(rows, k)
    raise ValueError(qtype)


# ------------------------------------------------------------------ GGUF reader

def read_gguf(buf: bytes):
    """Minimal GGUF v3 reader: returns (metadata dict, tensors dict name -> (dims, type, data bytes))."""
    mv = memoryview(buf)
    assert bytes(mv[:4]) == b"GGUF"
    ver, nt, nkv = struct.unpack_from("<IQQ", mv, 4)
    pos = 4 + 4 + 16

    def rstr(p):
        n = struct.unpack_from("<Q", mv, p)[0]
        return bytes(mv[p + 8:p + 8 + n]).decode(), p + 8 + n

    scalar = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}

    def rval(t, p):
        if t == 8:
            return rstr(p)
        if t == 9:
            et, n = struct.unpack_from("<IQ", mv, p)
            p += 12
            vals = []
            for _ in range(n):
                v, p = rval(et, p)
                vals.append(v)
            return vals, p
        fmt = scalar[t]
        return struct.unpack_from(fmt, mv, p)[0], p + struct.calcsize(fmt)

    meta = {}
    for _ in range(nkv):
        k, pos = rstr(pos)
        t = struct.unpack_from("<I", mv, pos)[0]
        pos += 4
        meta[k], pos = rval(t, pos)
    infos = []
    for _ in range(nt):
        name, pos = rstr(pos)
        nd = struct.unpack_from("<I", mv, pos)[0]
        pos += 4
        dims = list(struct.unpack_from("<" + "Q" * nd, mv, pos))
        pos += 8 * nd
        typ, off = struct.unpack_from("<IQ", mv, pos)
        pos += 12
        infos.append((name, dims, typ, off))
    align = meta.get("general.alignment", 32)
    start = (pos + align - 1) // align * align
    layout = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
    tensors = {}
    for name, dims, typ, off in infos:
        n = int(np.prod(dims))
        epb, bpb = layout[typ]
        nbytes = n // epb * bpb
        tensors[name] = (dims, typ, np.frombuffer(buf, dtype=np.uint8, count=nbytes, offset=start + off))
    return meta, tensors, start


# ------------------------------------------------------------------ forward

def _r16(a):
    """f64 values rounded to f32, then to f16 (IEEE nearest-even), back as f64."""
    return np.asarray(a).astype(np.float32).astype(np.float16).astype(np.float64)


def attn_cm1(q, K, V, vis):
    """The reference's flash_attn_cm1.slang arithmetic for query rows q [R][hd]
    (f32 values) over f16 keys / values K, V [n][hd] with visibility vis
    [R][n], written with numpy's own float16 / float32 conversions: q staged as
    f16(q * f32(f32(1 / sqrt(hd)) * f32(log2 e))); per 64-key block from key 0
    the row maximum, the f16 output rescaled by f16(exp2(m_old - m_new)),
    P = exp2(S - m) rounded to f16, P V added into an f16 accumulator per
    16-key chunk, that added to the f16 output; out = f32(O) * f32(1 / L)."""
    R, hd = q.shape
    n = K.shape[0]
    qs = np.float32(np.float32(1.0) / np.sqrt(np.float32(hd))) * np.float32(1.4426950408889634)
    q16 = (q.astype(np.float32) * qs).astype(np.float16).astype(np.float64)
    Kf = np.asarray(K, np.float64)
    Vf = np.asarray(V, np.float64)
    M = np.full(R, -1e30, np.float32)
    Lsum = np.zeros(R)
    O = np.zeros((R, hd), np.float16)
    for k0 in range(0, n, 64):
        k1 = min(k0 + 64, n)
        vb = vis[:, k0:k1]
        S = (q16 @ Kf[k0:k1].T).astype(np.float32)
        S = np.where(vb, S, np.float32(-np.inf))
        Mn = np.maximum(np.maximum(S.max(axis=1), np.float32(-1e30)), M)
        e = np.exp2((M - Mn).astype(np.float64)).astype(np.float32)
        Lsum = e.astype(np.float64) * Lsum
        O = (e.astype(np.float16).astype(np.float64)[:, None] * O.astype(np.float64)).astype(np.float16)
        Pm = np.where(vb, np.exp2((S - Mn[:, None]).astype(np.float64)).astype(np.float32), np.float32(0))
        Lsum = Lsum + Pm.astype(np.float64).sum(axis=1)
        P16 = Pm.astype(np.float16).astype(np.float64)
        acc = np.zeros((R, hd), np.float16)
        for c0 in range(0, k1 - k0, 16):
            c1 = min(c0 + 16, k1 - k0)
            acc = (acc.astype(np.float64) + P16[:, c0:c1] @ Vf[k0 + c0:k0 + c1]).astype(np.float16)
        O = (O.astype(np.float64) + acc.astype(np.float64)).astype(np.float16)
        M = Mn
    Lf = Lsum.astype(np.float32)
    inv = np.where(Lf == 0, np.float32(0), np.float32(1) / np.where(Lf == 0, np.float32(1), Lf))
    return (O.astype(np.float32) * inv[:, None]).astype(np.float64)


class RefLlama:
    """float64 Llama forward with f16 K/V storage (same cache rounding as the reference)."""

    def __init__(self, buf: bytes, mm16: bool = False, cm1: bool = False):
        """mm16: the dense matmuls with the reference's wide-GEMM operands
        (mul_mm_cm.slang): f16-rounded f32 weights and f16-rounded inputs.
        cm1: causal calls of more than one column compute attention with the
        reference's cooperative-matrix flash attention arithmetic (attn_cm1)."""
        meta, T, _ = read_gguf(buf)
        self.mm16 = mm16
        self.cm1 = cm1
        self.nl = meta["llama.block_count"]
        self.d = meta["llama.embedding_length"]
        self.nh = meta["llama.attention.head_count"]
        self.nkv = meta.get("llama.attention.head_count_kv", self.nh)
        self.ff = meta["llama.feed_forward_length"]
        self.eps = meta.get("llama.attention.layer_norm_rms_epsilon", 1e-5)
        self.base = meta.get("llama.rope.freq_base", 10000.0)
        self.hd = self.d // self.nh

        def mat(name):
            dims, typ, data = T[name]
            rows = dims[1] if len(dims) > 1 else 1
            return dequant(typ, data, rows, dims[0])

        self.emb = mat("token_embd.weight")
        self.V = self.emb.shape[0]
        self.out = mat("output.weight") if "output.weight" in T else self.emb
        self.onorm = mat("output_norm.weight")[0]
        self.layers = []
        for i in range(self.nl):
            g = lambda s: mat(f"blk.{i}.{s}.weight")  # noqa: E731
            self.layers.append({k: g(k) for k in ["attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                                 "ffn_norm", "ffn_gate", "ffn_up", "ffn_down"]})
        self.K = [np.zeros((0, self.nkv, self.hd)) for _ in range(self.nl)]
        self.Vc = [np.zeros((0, self.nkv, self.hd)) for _ in range(self.nl)]
        if mm16:
            self.out = _r16(self.out)
            for W in self.layers:
                for k in ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]:
                    W[k] = _r16(W[k])

    def mm(self, x, w):
        """x @ w.T; in mm16 mode the input rounded to f16 (w already is) and the
        output stored as f32, as the reference's f32 tensors hold it (the same
        storage points as the C oracle, so both round the same f32 values to f16)."""
        if not self.mm16:
            return x @ w.T
        return (_r16(x) @ w.T).astype(np.float32).astype(np.float64)

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * w[0] if w.ndim == 2 else None

    def rope(self, x, pos):
        # x [L, heads, hd]; adjacent pairs rotated by pos * base^(-i0/hd)
        i0 = np.arange(0, self.hd, 2)
        th = np.asarray(pos, dtype=np.float64)[:, None] * self.base ** (-i0 / self.hd)[None, :]
        c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
        x0, x1 = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2] = x0 * c - x1 * s
        out[..., 1::2] = x0 * s + x1 * c
        return out

    def forward(self, tokens, parents=None):
        """Appends to the cache; returns (logits [L][V], residual [L][d])."""
        L = len(tokens)
        P = self.K[0].shape[0]
        if parents is None:
            parents = [i - 1 for i in range(L)]
        depth = []
        for i in range(L):
            depth.append(0 if parents[i] < 0 else depth[parents[i]] + 1)
        anc = np.zeros((L, L), dtype=bool)
        for j in range(L):
            x = j
            while x >= 0:
                anc[j, x] = True
                x = parents[x]
        pos = P + np.array(depth)
        x = self.emb[np.asarray(tokens)].copy()
        gqa = self.nh // self.nkv
        for li, W in enumerate(self.layers):
            h = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * W["attn_norm"][0]
            q = self.mm(h, W["attn_q"]).reshape(L, self.nh, self.hd)
            k = self.mm(h, W["attn_k"]).reshape(L, self.nkv, self.hd)
            v = self.mm(h, W["attn_v"]).reshape(L, self.nkv, self.hd)
            q = self.rope(q, pos)
            k = self.rope(k, pos)
            k16 = k.astype(np.float32).astype(np.float16).astype(np.float64)
            v16 = v.astype(np.float32).astype(np.float16).astype(np.float64)
            self.K[li] = np.concatenate([self.K[li], k16])
            self.Vc[li] = np.concatenate([self.Vc[li], v16])
            Kc, Vc = self.K[li], self.Vc[li]
            att = np.zeros((L, self.nh, self.hd))
            q32 = q.astype(np.float32).astype(np.float64)
            causal = all(parents[i] == i - 1 for i in range(L))
            for hh in range(self.nh):
                kh = hh // gqa
                if self.cm1 and L > 1 and causal:
                    vis = np.ones((L, P + L), dtype=bool)
                    vis[:, P:] = anc
                    att[:, hh, :] = attn_cm1(q32[:, hh, :], Kc[:, kh, :], Vc[:, kh, :], vis)
                    continue
                s = q32[:, hh, :] @ Kc[:, kh, :].T / np.sqrt(self.hd)  # [L, P+L]
                mask = np.ones_like(s, dtype=bool)
                mask[:, P:] = anc
                s = np.where(mask, s, -np.inf)
                s = s - s.max(axis=1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=1, keepdims=True)
                att[:, hh, :] = p @ Vc[:, kh, :]
            att = att.reshape(L, self.d).astype(np.float32).astype(np.float64)
            x = (x + self.mm(att, W["attn_output"])).astype(np.float32).astype(np.float64)
            h2 = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * W["ffn_norm"][0]
            g = self.mm(h2, W["ffn_gate"])
            u = self.mm(h2, W["ffn_up"])
            a = (g / (1 + np.exp(-g)) * u).astype(np.float32).astype(np.float64)
            x = (x + self.mm(a, W["ffn_down"])).astype(np.float32).astype(np.float64)
        f = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * self.onorm
        return self.mm(f, self.out), x

    def truncate(self, p):
        for li in range(self.nl):
            self.K[li] = self.K[li][:p]
            self.Vc[li] = self.Vc[li][:p]


class RefQwen(RefLlama):
    """float64 Qwen3 / Qwen3-MoE forward: decoupled head_dim (attention.key_length),
    per-head RMSNorm of q and k with learned [head_dim] weights before a
    rotate-half ("NEOX") RoPE that pairs element i with i + head_dim/2, and for
    qwen3moe a routed FFN: softmax router, top-k experts by probability (ties
    to the lower index), weights divided by their sum, weighted sum of
    per-expert SwiGLU FFNs."""

    def __init__(self, buf: bytes):
        meta, T, _ = read_gguf(buf)
        self.arch = meta["general.architecture"]
        A = self.arch + "."
        self.nl = meta[A + "block_count"]
        self.d = meta[A + "embedding_length"]
        self.nh = meta[A + "attention.head_count"]
        self.nkv = meta.get(A + "attention.head_count_kv", self.nh)
        self.hd = meta.get(A + "attention.key_length", self.d // self.nh)
        self.eps = meta.get(A + "attention.layer_norm_rms_epsilon", 1e-6)
        self.base = meta.get(A + "rope.freq_base", 1e6)
        self.moe = self.arch == "qwen3moe"
        if self.moe:
            self.E = meta[A + "expert_count"]
            self.k = meta[A + "expert_used_count"]
            self.ef = meta[A + "expert_feed_forward_length"]

        def mat(name):
            dims, typ, data = T[name]
            rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
            return dequant(typ, data, rows, dims[0])

        self.emb = mat("token_embd.weight")
        self.V = self.emb.shape[0]
        self.out = mat("output.weight") if "output.weight" in T else self.emb
        self.onorm = mat("output_norm.weight")[0]
        self.layers = []
        names = ["attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm", "attn_k_norm", "ffn_norm"]
        names += ["ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"] if self.moe else \
            ["ffn_gate", "ffn_up", "ffn_down"]
        for i in range(self.nl):
            W = {k: mat(f"blk.{i}.{k}.weight") for k in names}
            if self.moe:
                W["ffn_gate_exps"] = W["ffn_gate_exps"].reshape(self.E, self.ef, self.d)
                W["ffn_up_exps"] = W["ffn_up_exps"].reshape(self.E, self.ef, self.d)
                W["ffn_down_exps"] = W["ffn_down_exps"].reshape(self.E, self.d, self.ef)
            self.layers.append(W)
        self.K = [np.zeros((0, self.nkv, self.hd)) for _ in range(self.nl)]
        self.Vc = [np.zeros((0, self.nkv, self.hd)) for _ in range(self.nl)]

    def rope(self, x, pos):
        half = self.hd // 2
        th = np.asarray(pos, dtype=np.float64)[:, None] * self.base ** (-2.0 * np.arange(half) / self.hd)[None, :]
        c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
        a, b = x[..., :half], x[..., half:]
        return np.concatenate([a * c - b * s, a * s + b * c], axis=-1)

    def headnorm(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * w[0]

    def route(self, logits):
        z = np.exp(logits - logits.max())
        p = z / z.sum()
        order = np.argsort(-p, kind="stable")[: self.k]  # descending, lower index first on ties
        return order, p[order] / p[order].sum()

    def ffn(self, W, h2):
        if not self.moe:
            g = h2 @ W["ffn_gate"].T
            u = h2 @ W["ffn_up"].T
            a = (g / (1 + np.exp(-g)) * u).astype(np.float32).astype(np.float64)
            return a @ W["ffn_down"].T
        out = np.zeros_like(h2)
        logits = (h2 @ W["ffn_gate_inp"].T).astype(np.float32).astype(np.float64)
        for c in range(h2.shape[0]):
            ids, w = self.route(logits[c])
            w = w.astype(np.float32).astype(np.float64)
            for e, we in zip(ids, w):
                g = W["ffn_gate_exps"][e] @ h2[c]
                u = W["ffn_up_exps"][e] @ h2[c]
                a = (g / (1 + np.exp(-g)) * u).astype(np.float32).astype(np.float64)
                out[c] += we * (W["ffn_down_exps"][e] @ a).astype(np.float32).astype(np.float64)
        return out

    def forward(self, tokens, parents=None):
        L = len(tokens)
        P = self.K[0].shape[0]
        if parents is None:
            parents = [i - 1 for i in range(L)]
        depth = []
        for i in range(L):
            depth.append(0 if parents[i] < 0 else depth[parents[i]] + 1)
        anc = np.zeros((L, L), dtype=bool)
        for j in range(L):
            x = j
            while x >= 0:
                anc[j, x] = True
                x = parents[x]
        pos = P + np.array(depth)
        x = self.emb[np.asarray(tokens)].copy()
        gqa = self.nh // self.nkv
        for li, W in enumerate(self.layers):
            h = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * W["attn_norm"][0]
            q = (h @ W["attn_q"].T).astype(np.float32).astype(np.float64).reshape(L, self.nh, self.hd)
            k = (h @ W["attn_k"].T).astype(np.float32).astype(np.float64).reshape(L, self.nkv, self.hd)
            v = (h @ W["attn_v"].T).reshape(L, self.nkv, self.hd)
            q = self.rope(self.headnorm(q, W["attn_q_norm"]), pos)
            k = self.rope(self.headnorm(k, W["attn_k_norm"]), pos)
            k16 = k.astype(np.float32).astype(np.float16).astype(np.float64)
            v16 = v.astype(np.float32).astype(np.float16).astype(np.float64)
            self.K[li] = np.concatenate([self.K[li], k16])
            self.Vc[li] = np.concatenate([self.Vc[li], v16])
            Kc, Vc = self.K[li], self.Vc[li]
            att = np.zeros((L, self.nh, self.hd))
            q32 = q.astype(np.float32).astype(np.float64)
            for hh in range(self.nh):
                kh = hh // gqa
                s = q32[:, hh, :] @ Kc[:, kh, :].T / np.sqrt(self.hd)
                mask = np.ones_like(s, dtype=bool)
                mask[:, P:] = anc
                s = np.where(mask, s, -np.inf)
                s = s - s.max(axis=1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=1, keepdims=True)
                att[:, hh, :] = p @ Vc[:, kh, :]
            att = att.reshape(L, self.nh * self.hd).astype(np.float32).astype(np.float64)
            x = (x + att @ W["attn_output"].T).astype(np.float32).astype(np.float64)
            h2 = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * W["ffn_norm"][0]
            x = (x + self.ffn(W, h2)).astype(np.float32).astype(np.float64)
        f = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * self.onorm
        return f @ self.out.T, x
