"""Seeded qwen35-layout models for the tests (quantized with the oracle's encoders).

The config-1 model: 4 layers, d_model 512, 8 Q / 2 KV heads x 64, SwiGLU FFN
1536, vocab 151,936, Q8_0 weights ~N(0, 0.02), f32 norm weights ~1 + N(0, 0.1)
(distinct per tensor, so a swapped norm shows), one MTP (nextn)
layer; qwen35 layout with full_attention_interval = 1 (attn_q packs Q and a
per-head output gate, q/k norms, IMROPE sections [11, 11, 10, 0], theta 1e6).
"""
import numpy as np

from oracle import cpvo

TINY = dict(n_layer=4, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=1536, n_vocab=151936,
            n_rot=64, rope_sections=[11, 11, 10, 0], rms_eps=1e-6, freq_base=1e6, has_mtp=1)


def make_tensors(hp, seed=0, qtype=cpvo.Q8_0, head_type=None, std=0.02):
    """Yield (name, type, bytes, ne0, ne1) for every tensor of the model."""
    rng = np.random.default_rng(seed)
    E, H, Hkv, hd, F, V = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"], hp["n_ff"], hp["n_vocab"]
    head_type = head_type or qtype

    def lin(name, rows, k, t=qtype):
        w = rng.normal(0, std, size=(rows, k)).astype(np.float32)
        return (name, t, cpvo.quantize(t, w), k, rows)

    def ones(name, n):
        w = (1.0 + 0.1 * rng.normal(size=n)).astype(np.float32)
        return (name, cpvo.F32, w.view(np.uint8), n, 1)

    out = [lin("token_embd.weight", V, E, head_type), ones("output_norm.weight", E),
           lin("output.weight", V, E, head_type)]
    n_layers = hp["n_layer"] + (1 if hp["has_mtp"] else 0)
    for il in range(n_layers):
        b = f"blk.{il}."
        out += [ones(b + "attn_norm.weight", E), ones(b + "post_attention_norm.weight", E),
                ones(b + "attn_q_norm.weight", hd), ones(b + "attn_k_norm.weight", hd),
                lin(b + "attn_q.weight", 2 * H * hd, E), lin(b + "attn_k.weight", Hkv * hd, E),
                lin(b + "attn_v.weight", Hkv * hd, E), lin(b + "attn_output.weight", E, H * hd),
                lin(b + "ffn_gate.weight", F, E), lin(b + "ffn_up.weight", F, E),
                lin(b + "ffn_down.weight", E, F)]
    if hp["has_mtp"]:
        b = f"blk.{hp['n_layer']}.nextn."
        out += [lin(b + "eh_proj.weight", E, 2 * E), ones(b + "enorm.weight", E), ones(b + "hnorm.weight", E)]
    return out


def load_into(model, tensors):
    for name, t, data, ne0, ne1 in tensors:
        model.set_tensor(name, t, data, ne0, ne1)


class OracleSession:
    """cpvo.Session behind the device Session's interface (FusedOut results),
    so the host loop can drive either."""

    def __init__(self, osess):
        self.s = osess

    @property
    def pos(self):
        return self.s.pos

    def set_pos(self, a, b):
        self.s.set_pos(a, b)

    def prefill(self, tokens):
        self.s.prefill(tokens)

    def step_fused_cached(self, tokens, depth, want_logits=False, noise=None):
        from codpiece_amd.model import FusedOut
        p, ch, cf, lg, hd = self.s.step_fused_cached(tokens, depth, want_logits, _host(noise))
        return FusedOut(p.tolist(), ch.tolist(), cf.tolist(), lg, hd)

    def mtp_draft(self, hidden, token, pos, p_min=0.0, want=False):
        """The oracle's standalone draft link (cpvo_mtp_draft) with its argmax
        and the re-draft gate (cpvo_softmax_peak_seq): the same contract as
        Session.mtp_draft; hidden_ptr is the link's hidden row itself."""
        from codpiece_amd.model import DraftResult
        logits, hout = self.s.mtp_draft(_host(hidden), token, pos)
        keep = not (p_min > 0 and cpvo.softmax_peak_seq(logits) < p_min)
        return DraftResult(cpvo.argmax(logits), keep, hout, logits, hout)

    def accept_round(self, out, drafts, params, mode, noise=None, hist=None, key=0, round=0):
        """The oracle's acceptance (cpvo_spec_accept) with the device's Philox
        uniforms for `key` and `round`: the same contract as Session.accept_round."""
        t, V = out.logits.shape
        u = cpvo.philox_uniforms(int(key), 1, t - 1, round=int(round))
        nz = None if noise is None else _host(noise).reshape(1, t, V)
        h = None if not hist else np.asarray(list(hist), dtype=np.int32).reshape(1, -1)
        tok, n = cpvo.spec_accept(np.asarray(out.logits).reshape(1, t, V), np.asarray(drafts, np.int32).reshape(1, t - 1),
                                  oracle_params(params), mode, u=u, noise_t=nz, hist=h)
        return tok[0, :n[0] + 1].tolist(), int(n[0])


def _host(x):
    """numpy float32 of x (numpy, torch on any device, or None)."""
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def oracle_params(p):
    return cpvo.SamplerParams(p.temp, p.top_k, p.top_p, p.min_p, p.min_keep, p.penalty_repeat, p.penalty_freq,
                              p.penalty_present, p.penalty_last_n)


class PairedSession:
    """A device session and an oracle session in lockstep: every call runs on
    the device with the attention tap on, the oracle continues from the
    device's attention outputs, and everything else must agree exactly.
    Records the worst attention tolerance ratio seen."""

    def __init__(self, gsess, osess, n_attn_floats):
        import torch
        self.g, self.o = gsess, osess
        self.tap = torch.empty(n_attn_floats, dtype=torch.float32, device="cuda")
        self.g.set_attn_tap(self.tap)
        self.worst = 0.0
        self.calls = 0

    @property
    def pos(self):
        assert self.g.pos == self.o.pos
        return self.g.pos

    def set_pos(self, a, b):
        self.g.set_pos(a, b)
        self.o.set_pos(a, b)

    def _inject(self):
        import torch
        torch.cuda.synchronize()
        self.o.inject_attention(self.tap.cpu().numpy())

    def _check(self):
        # the device attention follows the oracle's exact contract: no difference at all
        r = self.o.inject_ratio
        assert r == 0.0, f"attention differs from the oracle (ratio {r}) in call {self.calls}"
        self.worst = max(self.worst, r)
        self.calls += 1

    def prefill(self, tokens):
        self.g.prefill(tokens)
        self._inject()
        self.o.prefill(tokens)
        self._check()

    def step_fused_cached(self, tokens, depth, want_logits=False, noise=None):
        g = self.g.step_fused_cached(tokens, depth, want_logits=True, noise=noise)
        self._inject()
        nz = None if noise is None else noise.cpu().numpy()
        p, ch, cf, lg, hd = self.o.step_fused_cached(tokens, depth, want_logits=True, noise=nz)
        self._check()
        assert np.array_equal(g.logits.cpu().numpy(), lg), "logits differ"
        assert np.array_equal(g.hidden.cpu().numpy(), hd), "hidden differs"
        assert g.preds == p.tolist()
        assert g.chain == ch.tolist()
        # the peak probability is a double sum in another order: 1e-6 relative
        np.testing.assert_allclose(np.asarray(g.conf, dtype=np.float32).reshape(cf.shape), cf, rtol=1e-6)
        return g
