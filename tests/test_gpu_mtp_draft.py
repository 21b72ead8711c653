"""The standalone draft link (cpv_mtp_draft) and the re-draft gate
(cpv_redraft_gate) on the device, against the oracle.

Bar: bit-exact.  A link's logits and hidden row equal cpvo_mtp_draft's bit
for bit, its draft equals the oracle's argmax and its gate the oracle's
sequential-f32 decision (engine.rs:2598-2606), over chained links after a
round, for the config-1 model (Q8_0, vocabulary 151,936) and the Q4_K / Q6_K
mix; positions advance as the reference's (mtp_past + 1 per link), and a
round after the links still equals the oracle's.  The gate kernel is held to
the oracle at V = 151,936 on random rows and on rows built so that 1 / lse
lies within the f32 sum's rounding of p_min, where the bound pass cannot
decide and the sequential fold runs (the test counts those rows on the CPU
with the same bound).
"""
import numpy as np
import pytest
import torch

from oracle import cpvo

import model_fixtures as mf

pytestmark = pytest.mark.gpu

V = mf.TINY["n_vocab"]


def _models(qtype, head_type, seed):
    from codpiece_amd.model import Model, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    tensors = mf.make_tensors(mf.TINY, seed=seed, qtype=qtype, head_type=head_type)
    gm = Model(ctx, make_hparams(**mf.TINY))
    mf.load_into(gm, tensors)
    gm.ready()
    om = cpvo.Model(mf.TINY)
    mf.load_into(om, tensors)
    return ctx, gm, om


@pytest.fixture(scope="module", params=["q8_0", "q4_k"])
def models(request):
    if request.param == "q8_0":
        ctx, gm, om = _models(cpvo.Q8_0, None, 0)
    else:
        ctx, gm, om = _models(cpvo.Q4_K, cpvo.Q6_K, 2)
    yield ctx, gm, om
    gm.free()
    om.free()
    ctx.close()


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def test_chained_draft_links_equal_the_oracle(models):
    from codpiece_amd.model import Session
    ctx, gm, om = models
    g, o = Session(gm, 256), cpvo.Session(om, 256)
    prompt = np.random.default_rng(31).integers(0, V, size=40).tolist()
    print("case prefill + round", flush=True)
    g.prefill(prompt[:35])
    o.prefill(prompt[:35])
    gr = g.step_fused_cached(prompt[35:], 2, want_logits=True)
    P, C, CF, L, H = o.step_fused_cached(prompt[35:], 2, want_logits=True)
    assert np.array_equal(_bits(gr.hidden.cpu().numpy()), _bits(H))
    # a round that kept two drafts, then a re-draft from row 2
    for s in (g, o):
        s.set_pos(38, 3)
    hg, ho, tok, pos = gr.hidden[2], H[2], 1234, 38
    peaks = []
    for link in range(4):
        print(f"case link {link}", flush=True)
        r = g.mtp_draft(hg, tok, pos, 0.0, want=True)
        lo, hn = o.mtp_draft(ho, tok, pos)
        assert np.array_equal(_bits(r.logits.cpu().numpy()), _bits(lo)), f"link {link} logits"
        assert np.array_equal(_bits(r.hidden.cpu().numpy()), _bits(hn)), f"link {link} hidden"
        assert r.draft == cpvo.argmax(lo) and r.keep
        assert g.pos == o.pos == (38, 4 + link)
        peaks.append(cpvo.softmax_peak_seq(lo))
        hg, ho, tok, pos = r.hidden_ptr, hn, r.draft, pos + 1
    # the gate at thresholds on both sides of each link's peak, on the same link
    for p in sorted(peaks):
        for thr in (np.nextafter(np.float32(p), np.float32(1)), np.float32(p),
                    np.nextafter(np.float32(p), np.float32(0))):
            g.set_pos(38, 3)
            o.set_pos(38, 3)
            r = g.mtp_draft(gr.hidden[2], 1234, 38, float(thr))
            lo, _ = o.mtp_draft(H[2], 1234, 38)
            assert r.keep == (not (cpvo.softmax_peak_seq(lo) < thr))
    # the next round sees the links' MTP rows as the oracle does
    print("case round after links", flush=True)
    g.set_pos(38, 7)
    o.set_pos(38, 7)
    gr = g.step_fused_cached([5, 6, 7], 3, want_logits=True)
    P, C, CF, L, H = o.step_fused_cached([5, 6, 7], 3, want_logits=True)
    assert gr.preds == P.tolist() and gr.chain == C.tolist()
    assert np.array_equal(_bits(gr.logits.cpu().numpy()), _bits(L))
    g.free()
    o.free()


def test_draft_link_errors(models):
    from codpiece_amd.model import CpvError, Session
    _, gm, _ = models
    g = Session(gm, 32)
    h = torch.ones(mf.TINY["n_embd"], dtype=torch.float32, device="cuda")
    for tok, pos, mtp in ((V, 0, 0), (-1, 0, 0), (3, 34, 0), (3, -1, 0), (3, 0, 32)):
        g.set_pos(0, mtp)
        with pytest.raises(CpvError):
            g.mtp_draft(h, tok, pos)
        assert g.pos == (0, mtp)
    g.set_pos(0, 31)
    g.mtp_draft(h, 3, 33)
    assert g.pos == (0, 32)
    g.free()


def _ambiguous(l, p_min):
    """The bound pass's verdict for row l (as gate_fin_kernel computes it):
    True when 1 / lse cannot be placed on one side of p_min without the
    sequential fold."""
    l = np.asarray(l, np.float32)
    n = l.size
    e = cpvo.expf((l - np.float32(l.max())).astype(np.float32)).astype(np.float64)
    S = e.sum()
    W = (e * (n - np.arange(n))).sum()
    B = 1.0625 * 2.0 ** -24 * W + 2.0 ** -40 * S
    p = float(np.float32(p_min))
    below = (1.0 / (S - B)) * (1 + 2.0 ** -40) < p * (1 - 2.0 ** -23)
    keep = (1.0 / (S + B)) * (1 - 2.0 ** -40) >= p
    return not below and not keep


def test_redraft_gate_matches_the_sequential_f32_sum():
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    rng = np.random.default_rng(7)
    rows = []
    # random rows far from the threshold (the bound pass decides them)
    for sc in (0.5, 3.0, 8.0):
        rows.append(rng.normal(0, sc, V).astype(np.float32))
    # a spike over N(0, 1): the peak near 0.75 for spikes near ln(3 sum e^l)
    base = rng.normal(0, 1, V).astype(np.float32)
    s0 = float(np.log(3.0 * np.exp(base.astype(np.float64)).sum()))
    for ds in np.linspace(-0.02, 0.02, 21):
        r = base.copy()
        r[rng.integers(V)] = np.float32(s0 + ds)
        rows.append(r)
    # one term of 1 then V - 1 equal small terms: every add rounds the same
    # way against a sum in [1, 2), so the f32 sum is off the exact one by
    # about half a percent, across the threshold
    c0 = float(np.log((1 / 0.75 - 1) / (V - 1)))
    for dc in np.linspace(-0.012, 0.012, 13):
        r = np.full(V, np.float32(c0 + dc), np.float32)
        r[rng.integers(V)] = 0.0
        rows.append(r)
    x = np.stack(rows)
    for p_min in (0.75, 0.5, 0.0):
        xd = torch.from_numpy(x).cuda()
        am, keep = ctx.redraft_gate(xd, p_min)
        am, keep = am.cpu().numpy(), keep.cpu().numpy()
        want_keep = [not (p_min > 0 and cpvo.softmax_peak_seq(r) < np.float32(p_min)) for r in x]
        assert am.tolist() == [cpvo.argmax(r) for r in x]
        assert keep.astype(bool).tolist() == want_keep, p_min
        if p_min == 0.75:
            amb = [_ambiguous(r, p_min) for r in x]
            assert sum(amb) >= 5, "no row needed the sequential fold"
            sel = np.array(want_keep)[np.array(amb)]
            assert sel.any() and not sel.all(), "the ambiguous rows fall on one side only"
    ctx.close()
