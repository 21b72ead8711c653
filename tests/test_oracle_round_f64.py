"""The oracle's verify round held to an independent float64 forward.

tests/ref_f64.py restates the round from the reference graph
(crates/codpiece-model/src/qwen35.rs:2553-2962, build_attn_block
:3000-3198, positions and cache rows :1851-1876) in numpy float64.  It shares
no code with oracle/cpvo_model.c.

The composition is pinned on the round's smooth form: the oracle runs every
mul_mat on the unquantized activation rows (cpvo.set_smooth) and its
attention in binary64 (cpvo.set_attn_f64), and the float64 forward skips the
activation quantization too.  The leaf arithmetic those switches replace is
pinned on its own (the GEMM contract in test_oracle_quant.py, the attention
contract in test_oracle_glue.py); what is compared here is how the round
wires the leaves together, the code the switches do not touch.  Left between
the two is f32 and f16 rounding (the KV cache and q stay f16 on both sides),
under 1e-4 relative.  The bar:
  * logits, hidden rows and draft confidences within 1e-3 of the row's
    largest value (relative);
  * preds and draft ids equal wherever the float64 top-2 gap exceeds 1e-3 of
    the row's scale (a draft link only while every earlier id agreed).
Every composition mistake the oracle can plant (cpvo.set_fault) fails it by
more than 10x.  In the oracle's normal mode (quantized activations, the
chunked attention contract) a perturbation of 1e-7 can move an activation
code across a rounding boundary, after which a row carries about 2% of
quantization noise; that mode is held to the same forward with ggml's
activation quantization at 5e-2.
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf
import ref_f64 as rf

SMALL = dict(mf.TINY, n_layer=2, n_vocab=4096)
TOL = 1e-3


def _models(hp, tensors, quant_act=False):
    om = cpvo.Model(hp)
    mf.load_into(om, tensors)
    return om, rf.RefModel(hp, tensors, quant_act=quant_act)


@pytest.fixture(scope="module")
def small():
    tensors = mf.make_tensors(SMALL, seed=3)
    om, rm = _models(SMALL, tensors)
    yield om, rm
    om.free()


@pytest.fixture(autouse=True)
def smooth_round():
    cpvo.set_attn_f64(True)
    cpvo.set_smooth(True)
    cpvo.set_fault(0)
    yield
    cpvo.set_fault(0)
    cpvo.set_smooth(False)
    cpvo.set_attn_f64(False)


def _rel_rows(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b).max(axis=-1) / np.maximum(np.abs(b).max(axis=-1), 1e-30)


def _gap_ok(ref_logits, tol):
    s = np.sort(ref_logits, axis=-1)
    return (s[:, -1] - s[:, -2]) > tol * np.abs(ref_logits).max(axis=-1)


def round_errors(o, r, tol=TOL):
    """The bar's worst excess, max over checks of error / tol (<= 1 passes;
    a differing id where the reference is no near tie counts as 1e9).
    o, r: (preds, chain, conf, logits, hidden)."""
    P, C, CF, L, Hd = o
    p, c, cf, l, hd = r
    worst = max(_rel_rows(L, l).max(), _rel_rows(Hd, hd).max()) / tol
    ok = _gap_ok(l, tol)
    if np.any(np.asarray(P)[ok] != np.asarray(p)[ok]):
        worst = max(worst, 1e9)
    alive = np.asarray(P) == np.asarray(p)
    for s in range(c.shape[0]):
        worst = max(worst, (np.abs(CF[s] - cf[s]) / cf[s])[alive].max(initial=0.0) / tol)
        # the draft link's own logits are not returned: a differing id is
        # judged by its confidence (the softmax peak moves with the logits)
        alive &= C[s] == c[s]
    return worst


def _run_rounds(om, rm, prompt, depth=4, rounds=((5, 0), (3, 2))):
    """Prefill, then verify rounds; (n, rewind) = verify n tokens, then rewind
    the last `rewind` rows as a partly rejected round does."""
    n_ctx = 160
    os_, rs = cpvo.Session(om, n_ctx), rf.RefSession(rm, n_ctx)
    cut = len(prompt) - sum(n for n, _ in rounds)
    os_.prefill(prompt[:cut])
    rs.prefill(prompt[:cut])
    out, at = [], cut
    for n, back in rounds:
        toks = prompt[at:at + n]
        at += n
        o = os_.step_fused_cached(toks, depth, want_logits=True)
        r = rs.step(toks, depth)
        out.append((o, r))
        if back:
            npast, mpast = os_.pos
            os_.set_pos(npast - back, mpast + n - back)
            rs.set_pos(npast - back, mpast + n - back)
            assert os_.pos == (rs.n_past, rs.mtp_past)
            at -= back
    os_.free()
    return out


def test_round_matches_independent_f64_forward(small):
    om, rm = small
    prompt = np.random.default_rng(1).integers(0, SMALL["n_vocab"], size=40).tolist()
    for o, r in _run_rounds(om, rm, prompt):
        assert round_errors(o, r) <= 1.0


def test_k_quant_round_matches_independent_f64_forward():
    # the 27B-class weight mix on a small model: Q4_K linears, Q6_K embedding
    # and head (the forward dequantizes both formats itself)
    tensors = mf.make_tensors(SMALL, seed=6, qtype=cpvo.Q4_K, head_type=cpvo.Q6_K)
    om, rm = _models(SMALL, tensors)
    prompt = np.random.default_rng(3).integers(0, SMALL["n_vocab"], size=40).tolist()
    for o, r in _run_rounds(om, rm, prompt):
        assert round_errors(o, r) <= 1.0
    om.free()


def test_config1_round_matches_independent_f64_forward():
    # the config-1 model itself: 4 layers, vocabulary 151,936, a rejected tail
    tensors = mf.make_tensors(mf.TINY, seed=5)
    om, rm = _models(mf.TINY, tensors)
    prompt = np.random.default_rng(2).integers(0, mf.TINY["n_vocab"], size=48).tolist()
    for o, r in _run_rounds(om, rm, prompt, rounds=((5, 3), (5, 0))):
        assert round_errors(o, r) <= 1.0
    om.free()


@pytest.mark.parametrize("fault", [1, 2, 3, 4, 5, 6])
def test_each_planted_composition_mistake_is_caught(small, fault):
    om, rm = small
    prompt = np.random.default_rng(1).integers(0, SMALL["n_vocab"], size=40).tolist()
    cpvo.set_fault(fault)
    worst = max(round_errors(o, r) for o, r in _run_rounds(om, rm, prompt))
    cpvo.set_fault(0)
    assert worst > 10.0, f"planted mistake {fault} passes the f64 check ({worst:.3f})"


def test_quantized_round_stays_near_f64(small):
    # the oracle's normal mode (ggml's activation quantization, the chunked
    # attention contract the device reproduces) against the forward with the
    # same activation quantization: quantization noise only -- a rounding of
    # an activation code that flips amplifies the attention contract's
    # fixed-point differences (worst relative logit error measured 5.2e-2)
    om, _ = small
    cpvo.set_attn_f64(False)
    cpvo.set_smooth(False)
    rq = rf.RefModel(SMALL, mf.make_tensors(SMALL, seed=3), quant_act=True)
    prompt = np.random.default_rng(1).integers(0, SMALL["n_vocab"], size=40).tolist()
    for o, r in _run_rounds(om, rq, prompt):
        assert round_errors(o, r, tol=7e-2) <= 1.0


def _zeroed(tensors, names):
    out = []
    for name, t, data, ne0, ne1 in tensors:
        if name in names:
            data = cpvo.quantize(t, np.zeros((ne1, ne0), np.float32))
        out.append((name, t, data, ne0, ne1))
    return out


def test_zero_output_projections_make_every_layer_the_identity():
    # wo = 0 and ffn_down = 0 in every trunk layer: each block adds exactly 0,
    # so the logits are head . rms(embed) -- bit for bit the oracle's own GEMM
    # and norm on the embedding rows, and the f64 forward's closed form
    hp = dict(SMALL, has_mtp=0)
    names = {f"blk.{i}.{w}" for i in range(hp["n_layer"]) for w in ("attn_output.weight", "ffn_down.weight")}
    tensors = _zeroed(mf.make_tensors(hp, seed=8), names)
    cpvo.set_attn_f64(False)
    cpvo.set_smooth(False)
    om, rm = _models(hp, tensors, quant_act=True)
    toks = np.random.default_rng(3).integers(0, hp["n_vocab"], size=6).tolist()
    s = cpvo.Session(om, 32)
    P, _, _, L, Hd = s.step_fused_cached(toks, 0, want_logits=True)
    tmap = {n: (t, d, a, b) for n, t, d, a, b in tensors}
    t_e, d_e, ne0, _ = tmap["token_embd.weight"]
    rb = cpvo.row_bytes(t_e, ne0)
    emb = cpvo.dequantize(t_e, np.asarray(d_e).reshape(-1, rb)[toks], ne0)
    nw = np.asarray(tmap["output_norm.weight"][1]).view(np.float32)
    h = np.stack([cpvo.rms_norm(e, hp["rms_eps"], nw) for e in emb])
    assert np.array_equal(Hd.view(np.uint32), h.astype(np.float32).view(np.uint32))
    t_o, d_o, _, _ = tmap["output.weight"]
    assert np.array_equal(L.view(np.uint32), cpvo.qgemm(t_o, d_o, h.astype(np.float32)).view(np.uint32))
    ref = rf.RefSession(rm, 32).step(toks, 0)
    assert _rel_rows(L, ref[3]).max() <= 1e-5
    s.free()
    om.free()


def test_zero_attn_q_gives_uniform_attention_at_half_gate():
    # attn_q = 0: q = 0 (every score 0, so attention is the mean of the
    # visible V rows) and gate = 0 (sigmoid 1/2); the f64 forward reduces to
    # that closed form, and the oracle must agree with it
    hp = dict(SMALL, has_mtp=0, n_layer=1)
    tensors = _zeroed(mf.make_tensors(hp, seed=9), {"blk.0.attn_q.weight"})
    om, rm = _models(hp, tensors)
    prompt = np.random.default_rng(4).integers(0, hp["n_vocab"], size=12).tolist()
    s, r = cpvo.Session(om, 32), rf.RefSession(rm, 32)
    s.prefill(prompt[:7])
    r.prefill(prompt[:7])
    o = s.step_fused_cached(prompt[7:], 0, want_logits=True)
    ref = r.step(prompt[7:], 0)
    assert _rel_rows(o[3], ref[3]).max() <= 1e-4
    # the closed form itself, on the f64 side: wo input = 0.5 * mean(V rows 0..n_past+t)
    x = rm.rows("token_embd.weight", prompt)
    xn = rf.rms(x, rm.vec("blk.0.attn_norm.weight"), hp["rms_eps"])
    v = rm.mm("blk.0.attn_v.weight", xn).astype(np.float16).astype(np.float64)
    H, Hkv, hd = hp["n_head"], hp["n_head_kv"], hp["head_dim"]
    wo_in = np.stack([np.repeat(v[:i + 1].reshape(i + 1, Hkv, hd).mean(axis=0), H // Hkv, axis=0).ravel() * 0.5
                      for i in range(7, 12)])
    x1 = x[7:] + rm.mm("blk.0.attn_output.weight", wo_in)
    n = rf.rms(x1, rm.vec("blk.0.post_attention_norm.weight"), hp["rms_eps"])
    g, u = rm.mm("blk.0.ffn_gate.weight", n), rm.mm("blk.0.ffn_up.weight", n)
    x2 = x1 + rm.mm("blk.0.ffn_down.weight", g * rf.sigmoid(g) * u)
    logits = rm.mm("output.weight", rf.rms(x2, rm.vec("output_norm.weight"), hp["rms_eps"]))
    assert _rel_rows(ref[3], logits).max() <= 1e-12
    s.free()
    om.free()
