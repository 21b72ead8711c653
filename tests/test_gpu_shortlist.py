"""The MTP draft head over a shortlist (cpv_verify_step_cands) against the oracle.

Each link projects onto the head's candidate rows, takes its argmax and peak
over them, reports cands[argmax] and feeds the argmax itself to the next link
(qwen35.rs:1904-1910, 2925-2958).  The device round must equal the oracle's:
logits, preds and chain bit for bit, the peak confidence to 1e-6, with the
shortlist repeated (the gathered head kept) and changed (gathered again).
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf

pytestmark = pytest.mark.gpu

K_MODEL = dict(mf.TINY, n_layer=2, n_vocab=4096)


@pytest.fixture(scope="module", params=["q4k", "q8_0"])
def models(request):
    from codpiece_amd.model import Model, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    if request.param == "q4k":
        tensors = mf.make_tensors(K_MODEL, seed=9, qtype=cpvo.Q4_K, head_type=cpvo.Q6_K)
    else:
        tensors = mf.make_tensors(K_MODEL, seed=10)
    gm = Model(ctx, make_hparams(**K_MODEL))
    mf.load_into(gm, tensors)
    gm.ready()
    om = cpvo.Model(K_MODEL)
    mf.load_into(om, tensors)
    yield ctx, gm, om
    gm.free()
    om.free()
    ctx.close()


def same_round(a, b):
    assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
    assert a.preds == b[0].tolist()
    assert a.chain == b[1].tolist()
    assert np.allclose(np.asarray(a.conf), b[2], rtol=0, atol=1e-6)


def test_shortlist_rounds_equal_oracle(models):
    from codpiece_amd.model import Session
    ctx, gm, om = models
    V = K_MODEL["n_vocab"]
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, V, size=60).tolist()
    c1 = rng.choice(V, size=700, replace=False).tolist()
    c2 = sorted(rng.choice(V, size=64, replace=False).tolist())
    g, o = Session(gm, 256), cpvo.Session(om, 256)
    g.prefill(prompt[:50])
    o.prefill(prompt[:50])
    for i, (toks, cands) in enumerate([(prompt[50:55], c1), (prompt[55:60], c1), (prompt[45:50], c2)]):
        print("round", i, "with", len(cands), "candidates", flush=True)
        a = g.step_fused_cached(toks, 4, want_logits=True, cands=cands)
        b = o.step_fused_cached(toks, 4, want_logits=True, cands=cands)
        same_round(a, b)
        assert all(v in cands for row in a.chain for v in row)
    # back to the full head
    a = g.step_fused_cached(prompt[:5], 4, want_logits=True)
    b = o.step_fused_cached(prompt[:5], 4, want_logits=True)
    same_round(a, b)
    g.free()
    o.free()


def test_permuted_shortlist_feeds_the_index_to_the_next_link(models):
    # the same candidate set in identity and in permuted order: the first
    # link's drafts agree, the second link embeds the shortlist index
    # (qwen35.rs:2958) and differs; each order equals the oracle's round
    from codpiece_amd.model import Session
    ctx, gm, om = models
    V = K_MODEL["n_vocab"]
    n = 512
    ident = list(range(n))
    perm = np.random.default_rng(23).permutation(n).tolist()
    prompt = np.random.default_rng(24).integers(0, V, size=40).tolist()
    rounds = []
    for cands in (ident, perm):
        g, o = Session(gm, 256), cpvo.Session(om, 256)
        g.prefill(prompt[:35])
        o.prefill(prompt[:35])
        a = g.step_fused_cached(prompt[35:], 2, want_logits=True, cands=cands)
        b = o.step_fused_cached(prompt[35:], 2, want_logits=True, cands=cands)
        same_round(a, b)
        rounds.append(a)
        g.free()
        o.free()
    a0, a1 = rounds
    assert a0.preds == a1.preds and a0.chain[0] == a1.chain[0]
    assert a0.chain[1] != a1.chain[1] or a0.conf[1] != a1.conf[1]


def test_shortlist_of_the_argmax_rows_matches_the_full_head_first_link(models):
    # with every id a candidate, in order, link 0 equals the full head's draft
    from codpiece_amd.model import Session
    ctx, gm, om = models
    V = K_MODEL["n_vocab"]
    rng = np.random.default_rng(22)
    prompt = rng.integers(0, V, size=40).tolist()
    g1, g2 = Session(gm, 256), Session(gm, 256)
    for g in (g1, g2):
        g.prefill(prompt[:35])
    a = g1.step_fused_cached(prompt[35:], 1, cands=list(range(V)))
    b = g2.step_fused_cached(prompt[35:], 1)
    assert a.chain == b.chain and a.preds == b.preds
    g1.free()
    g2.free()


def test_bad_candidates_are_errors(models):
    from codpiece_amd.model import Session
    from codpiece_amd.runtime import CpvError
    ctx, gm, om = models
    V = K_MODEL["n_vocab"]
    g = Session(gm, 256)
    g.prefill(list(range(10)))
    with pytest.raises(CpvError):
        g.step_fused_cached([1, 2], 2, cands=[0, V])
    with pytest.raises(CpvError):
        g.step_fused_cached([1, 2], 2, cands=[-1, 3])
    with pytest.raises(CpvError):
        g.step_fused_cached([1, 2], 2, cands=list(range(V)) + [0])
    assert g.pos[0] == 10
    g.free()
