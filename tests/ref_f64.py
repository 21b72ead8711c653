"""An independent float64 forward of the qwen35 verify round, to pin the oracle.

Written from the reference graph, not from oracle/cpvo_model.c:
- the trunk loop of build_inner (crates/codpiece-model/src/qwen35.rs:2553-2786):
  x += attn(rms(x, attn_norm)); then x += down(silu(gate(n)) * up(n)) with
  n = rms(x, post_attention_norm) (:2783-2795);
- build_attn_block (:3000-3198): attn_q holds, per head, q (hd values) then the
  output gate (hd values) (the views at :3031-3045); q and k get a per-head RMS
  norm with attn_q_norm / attn_k_norm (:3037, :3049); IMROPE over n_rot dims
  with the text position streams (p, p, p, 0) (:3053-3062, :3542-3548); K and V
  go to the f16 cache at rows n_past + i (:3082-3093); flash attention with
  scale 1/sqrt(hd) under the causal mask (:3182-3187); then
  merged * sigmoid(gate) and wo (:3196-3197);
- the head (:2788-2821): h = rms(x, output_norm), logits = output . h (the
  token embedding when output is absent), ids = first argmax;
- the fused MTP chain (:2866-2962), link by link: e = embed(tok);
  cat = [rms(e, enorm) ; rms(h, hnorm)] (concat along the row, e first);
  d = eh_proj . cat; d += attn(rms(d, attn_norm)) on the MTP cache (rows
  mtp_past + i at positions n_past + i + 1, written by the first link only,
  :1858-1876, :2894-2900); d += ffn; h = rms(d, shared_head_norm or
  output_norm); logits = head . h; ids = argmax; conf = softmax(logits)[ids]
  (:2943-2952); the next link embeds ids and takes h (:2957-2958).

ggml's CPU types are kept where they are coarser than float64, since the
reference computes with them: every mul_mat first quantizes its activation
rows to the weight's vec_dot_type (Q8_0 blocks of 32 for Q8_0 weights, Q8_K
blocks of 256 for K-quants), the KV cache holds f16, and the CPU flash
attention converts q to f16 for its f16 dot with K.  Everything else
(norms, rope, softmax, gating, residuals, the GEMM sums) is float64.
Weights are dequantized here from the GGUF block layouts (ggml's published
formats), independently of the oracle's dequantizer.
"""
import numpy as np

Q8_0, Q4_K, Q6_K, F32 = 8, 12, 14, 0


def _f16(b):
    return np.ascontiguousarray(b).view(np.float16).astype(np.float64)[..., 0]


def dequant(t, raw, ne0, ne1):
    """[ne1, ne0] float64 of a GGUF tensor's bytes."""
    b = np.asarray(raw, dtype=np.uint8).reshape(ne1, -1)
    if t == F32:
        return b.view(np.float32).astype(np.float64).reshape(ne1, ne0)
    if t == Q8_0:
        blk = b.reshape(ne1, ne0 // 32, 34)
        d = _f16(blk[..., 0:2])
        q = np.ascontiguousarray(blk[..., 2:]).view(np.int8).astype(np.float64)
        return (d[..., None] * q).reshape(ne1, ne0)
    if t == Q4_K:
        blk = b.reshape(ne1, ne0 // 256, 144)
        d, dmin = _f16(blk[..., 0:2]), _f16(blk[..., 2:4])
        s = blk[..., 4:16].astype(np.int64)
        sc = np.empty(s.shape[:-1] + (8,), np.int64)
        mn = np.empty_like(sc)
        for j in range(4):
            sc[..., j] = s[..., j] & 63
            mn[..., j] = s[..., j + 4] & 63
        for j in range(4, 8):
            sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
        qs = blk[..., 16:144].reshape(ne1, ne0 // 256, 4, 32).astype(np.int64)
        # 64-element chunk c: sub-block 2c = low nibbles, 2c+1 = high nibbles
        codes = np.stack([qs & 15, qs >> 4], axis=3).reshape(ne1, ne0 // 256, 8, 32)
        v = d[..., None, None] * sc[..., None] * codes - dmin[..., None, None] * mn[..., None]
        return v.reshape(ne1, ne0)
    if t == Q6_K:
        blk = b.reshape(ne1, ne0 // 256, 210)
        ql, qh = blk[..., 0:128].astype(np.int64), blk[..., 128:192].astype(np.int64)
        sc = np.ascontiguousarray(blk[..., 192:208]).view(np.int8).astype(np.float64)
        d = _f16(blk[..., 208:210])
        codes = np.empty(blk.shape[:-1] + (256,), np.int64)
        for h in range(2):
            a, b2, hb = ql[..., 64 * h:64 * h + 32], ql[..., 64 * h + 32:64 * h + 64], qh[..., 32 * h:32 * h + 32]
            o = 128 * h
            codes[..., o:o + 32] = (a & 15) | ((hb & 3) << 4)
            codes[..., o + 32:o + 64] = (b2 & 15) | (((hb >> 2) & 3) << 4)
            codes[..., o + 64:o + 96] = (a >> 4) | (((hb >> 4) & 3) << 4)
            codes[..., o + 96:o + 128] = (b2 >> 4) | (((hb >> 6) & 3) << 4)
        v = d[..., None] * np.repeat(sc, 16, axis=-1) * (codes - 32)
        return v.reshape(ne1, ne0)
    raise ValueError(t)


def act_quant(t, x):
    """ggml CPU's activation quantization (quantize_row_q8_0_ref / _q8_K_ref,
    in f32 arithmetic), returned dequantized in float64."""
    x = np.asarray(x, dtype=np.float32)
    T, K = x.shape
    if t == Q8_0:
        b = x.reshape(T, K // 32, 32)
        amax = np.abs(b).max(axis=-1, keepdims=True)
        d = amax / np.float32(127)
        with np.errstate(divide="ignore"):
            idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
        v = (b * idv).astype(np.float64)
        q = np.sign(v) * np.floor(np.abs(v) + 0.5)          # roundf: half away from zero
        dh = d.astype(np.float16).astype(np.float64)
        return (dh * q).reshape(T, K)
    Kp = (K + 255) // 256 * 256
    xp = np.zeros((T, Kp), np.float32)
    xp[:, :K] = x
    b = xp.reshape(T, Kp // 256, 256)
    idx = np.abs(b).argmax(axis=-1)                          # first largest magnitude
    mx = np.take_along_axis(b, idx[..., None], axis=-1)
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = np.where(mx != 0, np.float32(-127) / mx, np.float32(0)).astype(np.float32)
    q = np.minimum(np.rint(b * iscale), 127).astype(np.float64)   # nearest_int: ties to even
    with np.errstate(divide="ignore"):
        d = np.where(iscale != 0, np.float32(1) / iscale, np.float32(0)).astype(np.float32)
    return (d.astype(np.float64) * q).reshape(T, Kp)[:, :K]


def rms(x, w, eps):
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * w


def imrope_theta(pos, n_rot, base, sections):
    """theta of each of the n_rot/2 rotated pairs at text position pos: the
    IMROPE sector rule over the position streams (pos, pos, pos, 0)."""
    streams = (pos, pos, pos, 0)
    tot = sum(sections)
    th = np.empty(n_rot // 2)
    for i in range(n_rot // 2):
        sector = i % tot
        if sector % 3 == 1 and sector < 3 * sections[1]:
            p = streams[1]
        elif sector % 3 == 2 and sector < 3 * sections[2]:
            p = streams[2]
        elif sector % 3 == 0 and sector < 3 * sections[0]:
            p = streams[0]
        else:
            p = streams[3]
        th[i] = p * float(base) ** (-2.0 * i / n_rot)
    return th


def rope(x, pos, n_rot, base, sections):
    """NEOX pairs (i, i + n_rot/2) rotated by theta_i; dims past n_rot kept."""
    y = np.array(x, dtype=np.float64, copy=True)
    th = imrope_theta(pos, n_rot, base, sections)
    c, s = np.cos(th), np.sin(th)
    h = n_rot // 2
    x0, x1 = y[..., :h].copy(), y[..., h:n_rot].copy()
    y[..., :h] = x0 * c - x1 * s
    y[..., h:n_rot] = x0 * s + x1 * c
    return y


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


class RefModel:
    """quant_act=False skips the activation quantization: every mul_mat is then
    a plain float64 product (the smooth form of the round)."""

    def __init__(self, hp, tensors, quant_act=True):
        self.hp = dict(hp)
        self.quant_act = quant_act
        self.raw = {name: (t, data, ne0, ne1) for name, t, data, ne0, ne1 in tensors}
        self._deq = {}

    def has(self, name):
        return name in self.raw

    def w(self, name):
        if name not in self._deq:
            t, data, ne0, ne1 = self.raw[name]
            self._deq[name] = dequant(t, data, ne0, ne1)
        return self._deq[name]

    def vec(self, name):
        return self.w(name)[0]

    def rows(self, name, ids):
        """get_rows of a (quantized) matrix: dequantize only those rows."""
        t, data, ne0, ne1 = self.raw[name]
        b = np.asarray(data, dtype=np.uint8).reshape(ne1, -1)
        sel = b[np.asarray(ids, dtype=np.int64)]
        return dequant(t, sel.ravel(), ne0, len(ids))

    def mm(self, name, x):
        """ggml_mul_mat(w, x): x rows quantized to the weight's vec_dot_type."""
        t = self.raw[name][0]
        xa = act_quant(t, x) if self.quant_act else np.asarray(x, np.float64)
        return xa @ self.w(name).T


class RefSession:
    """The round of qwen35.rs step_fused_cached on float64 state."""

    def __init__(self, model, n_ctx):
        hp = model.hp
        self.m, self.hp = model, hp
        self.n_ctx = n_ctx
        self.mtp_ctx = min(n_ctx, 16384)
        row = hp["n_head_kv"] * hp["head_dim"]
        nl = hp["n_layer"] + (1 if hp["has_mtp"] else 0)
        self.kc = [np.zeros((self.mtp_ctx if il == hp["n_layer"] else n_ctx, row), np.float16) for il in range(nl)]
        self.vc = [np.zeros_like(k) for k in self.kc]
        self.n_past = 0
        self.mtp_past = 0

    def set_pos(self, n_past, mtp_past):
        """The round bookkeeping (engine.rs:2533-2540): rows past n_past are
        stale and are overwritten by the next call."""
        self.n_past, self.mtp_past = n_past, mtp_past

    # one attention block (build_attn_block) on normed rows xn
    def _attn(self, il, xn, pos0, row0, n_vis0, write):
        hp, m = self.hp, self.m
        H, Hkv, hd = hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        T = xn.shape[0]
        b = f"blk.{il}."
        q_full = m.mm(b + "attn_q.weight", xn).reshape(T, H, 2 * hd)
        q = rms(q_full[:, :, :hd], m.vec(b + "attn_q_norm.weight"), hp["rms_eps"])
        gate = q_full[:, :, hd:].reshape(T, H * hd)
        k = rms(m.mm(b + "attn_k.weight", xn).reshape(T, Hkv, hd), m.vec(b + "attn_k_norm.weight"), hp["rms_eps"])
        v = m.mm(b + "attn_v.weight", xn).reshape(T, Hkv, hd)
        for t in range(T):
            q[t] = rope(q[t], pos0 + t, hp["n_rot"], hp["freq_base"], hp["rope_sections"])
            k[t] = rope(k[t], pos0 + t, hp["n_rot"], hp["freq_base"], hp["rope_sections"])
        if write:
            self.kc[il][row0:row0 + T] = k.reshape(T, Hkv * hd).astype(np.float16)
            self.vc[il][row0:row0 + T] = v.reshape(T, Hkv * hd).astype(np.float16)
        K = self.kc[il].astype(np.float64).reshape(-1, Hkv, hd)
        V = self.vc[il].astype(np.float64).reshape(-1, Hkv, hd)
        q16 = q.astype(np.float16).astype(np.float64)
        scale = 1.0 / np.sqrt(np.float32(hd))
        out = np.empty((T, H, hd))
        g = H // Hkv
        for t in range(T):
            n_vis = n_vis0 + t + 1                     # rows [0, n_past + t] are visible
            for h in range(H):
                s = K[:n_vis, h // g] @ q16[t, h] * scale
                p = np.exp(s - s.max())
                out[t, h] = (p / p.sum()) @ V[:n_vis, h // g]
        return m.mm(b + "attn_output.weight", out.reshape(T, H * hd) * sigmoid(gate))

    def _block(self, il, x, pos0, row0, n_vis0, write):
        hp, m = self.hp, self.m
        b = f"blk.{il}."
        x = x + self._attn(il, rms(x, m.vec(b + "attn_norm.weight"), hp["rms_eps"]), pos0, row0, n_vis0, write)
        n = rms(x, m.vec(b + "post_attention_norm.weight"), hp["rms_eps"])
        gt, up = m.mm(b + "ffn_gate.weight", n), m.mm(b + "ffn_up.weight", n)
        return x + m.mm(b + "ffn_down.weight", gt * sigmoid(gt) * up)

    def _trunk(self, tokens):
        x = self.m.rows("token_embd.weight", tokens)
        for il in range(self.hp["n_layer"]):
            x = self._block(il, x, self.n_past, self.n_past, self.n_past, True)
        return x

    def prefill(self, tokens):
        self._trunk(tokens)
        self.n_past += len(tokens)

    def _head_name(self):
        return "output.weight" if self.m.has("output.weight") else "token_embd.weight"

    def _mtp_names(self):
        nl = self.hp["n_layer"]
        nx = f"blk.{nl}.nextn."
        m = self.m
        emb = nx + "embed_tokens.weight" if m.has(nx + "embed_tokens.weight") else "token_embd.weight"
        hn = nx + "shared_head_norm.weight" if m.has(nx + "shared_head_norm.weight") else "output_norm.weight"
        head = nx + "shared_head_head.weight" if m.has(nx + "shared_head_head.weight") else self._head_name()
        return nx, emb, hn, head

    def draft(self, hidden, token, pos):
        """Qwen35::mtp_draft (qwen35.rs:2086-2192) on the graph of
        build_mtp_impl (mtp_graph.rs:123-249): (logits [V], hidden [E]) of one
        link; its K/V at MTP row mtp_past (row_ids, :2177-2181), rows
        0..mtp_past visible (:2163-2174), rope position pos; mtp_past + 1."""
        hp, m = self.hp, self.m
        nx, emb, hn, head = self._mtp_names()
        assert self.mtp_past + 1 <= self.mtp_ctx
        e = m.rows(emb, [int(token)])
        cat = np.concatenate([rms(e, m.vec(nx + "enorm.weight"), hp["rms_eps"]),
                              rms(np.asarray(hidden, np.float64).reshape(1, -1), m.vec(nx + "hnorm.weight"),
                                  hp["rms_eps"])], axis=1)
        d = m.mm(nx + "eh_proj.weight", cat)
        d = self._block(hp["n_layer"], d, pos, self.mtp_past, self.mtp_past, True)
        hs = rms(d, m.vec(hn), hp["rms_eps"])
        self.mtp_past += 1
        return m.mm(head, hs)[0], hs[0]

    def step(self, tokens, depth):
        """(preds, chain [depth][T], conf [depth][T], logits [T][V], hidden [T][E])"""
        hp, m = self.hp, self.m
        T = len(tokens)
        assert self.n_past + T <= self.n_ctx
        if self.mtp_past + T > self.mtp_ctx:
            self.mtp_past = 0
        x = self._trunk(tokens)
        h = rms(x, m.vec("output_norm.weight"), hp["rms_eps"])
        logits = m.mm(self._head_name(), h)
        preds = logits.argmax(axis=1)
        chain, conf = [], []
        nl = hp["n_layer"]
        nx = f"blk.{nl}.nextn."
        emb = nx + "embed_tokens.weight" if m.has(nx + "embed_tokens.weight") else "token_embd.weight"
        hn = nx + "shared_head_norm.weight" if m.has(nx + "shared_head_norm.weight") else "output_norm.weight"
        head = nx + "shared_head_head.weight" if m.has(nx + "shared_head_head.weight") else self._head_name()
        tok, hs = preds, h
        for step in range(depth):
            e = m.rows(emb, tok)
            cat = np.concatenate([rms(e, m.vec(nx + "enorm.weight"), hp["rms_eps"]),
                                  rms(hs, m.vec(nx + "hnorm.weight"), hp["rms_eps"])], axis=1)
            d = m.mm(nx + "eh_proj.weight", cat)
            d = self._block(nl, d, self.n_past + 1, self.mtp_past, self.mtp_past, step == 0)
            hs = rms(d, m.vec(hn), hp["rms_eps"])
            ld = m.mm(head, hs)
            ids = ld.argmax(axis=1)
            p = np.exp(ld - ld.max(axis=1, keepdims=True))
            conf.append(p[np.arange(T), ids] / p.sum(axis=1))
            chain.append(ids)
            tok = ids
        self.n_past += T
        return preds, np.array(chain).reshape(depth, T), np.array(conf).reshape(depth, T), logits, h
