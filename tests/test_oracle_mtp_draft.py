"""The oracle's standalone draft link and re-draft gate, pinned on the CPU.

cpvo_mtp_draft restates Qwen35::mtp_draft (crates/codpiece-model/src/
qwen35.rs:2086-2192) on the graph of build_mtp_impl (crates/codpiece-model/
src/mtp_graph.rs:123-249).  It is held to:
  * the round's own first chain link (already pinned by the f64 forward) on a
    one-row round, where the two compute the same link: same hidden, token,
    rope position (n_past + 1), K/V row and visible rows -- bit for bit;
  * an independent float64 restatement (tests/ref_f64.py RefSession.draft),
    over three chained links after a round, on the smooth round (unquantized
    activations, binary64 attention), within 1e-3; the three planted
    mistakes that touch a draft link (concat order, enorm/hnorm swapped, the
    hidden handed on before the head norm) each fail that bar by 10x.

cpvo_softmax_peak_seq restates the re-draft gate's value (engine.rs:
2598-2606; main.rs:946-954): 1 / (f32 sum in index order of exp(l - max)).
It is held to numpy's float32 add.accumulate (a sequential sum by
definition) over the pinned expf, to the closed forms of a uniform row (1/V
exactly, V < 2^24) and a single finite logit (1), and to the rounding
behaviour that makes the order matter.
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf
import ref_f64 as rf

SMALL = dict(mf.TINY, n_layer=2, n_vocab=4096)
TOL = 1e-3


def _seq_peak(l):
    l = np.asarray(l, np.float32)
    m = np.float32(np.max(l))
    e = cpvo.expf((l - m).astype(np.float32))
    lse = np.add.accumulate(e, dtype=np.float32)[-1]
    return float(np.float32(1.0) / lse)


@pytest.mark.parametrize("V", [7, 4096, 151936])
def test_peak_seq_is_the_sequential_f32_loop(V):
    rng = np.random.default_rng(V)
    for scale in (0.5, 3.0, 12.0):
        l = (rng.normal(0, scale, V)).astype(np.float32)
        assert cpvo.softmax_peak_seq(l) == _seq_peak(l)


def test_peak_seq_closed_forms():
    V = 151936
    assert cpvo.softmax_peak_seq(np.full(V, 0.25, np.float32)) == float(np.float32(1.0) / np.float32(V))
    l = np.full(V, -np.inf, np.float32)
    l[12345] = 3.0
    assert cpvo.softmax_peak_seq(l) == 1.0


def test_peak_seq_order_matters_and_is_index_order():
    # one large term first, then many small ones: each small add rounds
    # against the large partial sum, so index order and reverse order differ
    V = 151936
    l = np.full(V, np.float32(np.log(np.float32(1e-6))), np.float32)
    l[0] = 0.0
    fwd = cpvo.softmax_peak_seq(l)
    rev = cpvo.softmax_peak_seq(l[::-1].copy())
    assert fwd == _seq_peak(l) and rev == _seq_peak(l[::-1])
    assert fwd != rev
    exact = 1.0 / (1.0 + (V - 1) * float(cpvo.expf(np.array([l[1]], np.float32))[0]))
    assert abs(fwd - exact) < 1e-2 * exact


@pytest.fixture(scope="module")
def small():
    tensors = mf.make_tensors(SMALL, seed=3)
    om = cpvo.Model(SMALL)
    mf.load_into(om, tensors)
    yield om, tensors
    om.free()


def test_draft_link_equals_the_rounds_first_link(small):
    om, _ = small
    prompt = np.random.default_rng(4).integers(0, SMALL["n_vocab"], size=30).tolist()
    a, b = cpvo.Session(om, 64), cpvo.Session(om, 64)
    for s in (a, b):
        s.prefill(prompt[:-1])
        s.set_pos(s.pos[0], 7)
    P, C, CF, L, H = a.step_fused_cached(prompt[-1:], 1, want_logits=True)
    # the round's link 0: hidden h[0], token preds[0], rope position
    # n_past + 1, K/V at mtp_past, rows 0..mtp_past visible
    _, _, _, Lb, Hb = b.step_fused_cached(prompt[-1:], 0, want_logits=True)
    assert np.array_equal(Lb, L) and np.array_equal(Hb, H)
    n_past, mtp_past = b.pos
    logits, hout = b.mtp_draft(Hb[0], int(P[0]), n_past)
    assert b.pos == (n_past, mtp_past + 1)
    assert cpvo.argmax(logits) == C[0][0]
    mx = logits.max()
    conf = np.float32(1.0 / np.sum(cpvo.expf((logits - mx).astype(np.float32)).astype(np.float64)))
    assert abs(conf - CF[0][0]) <= 1e-6 * CF[0][0]
    a.free()
    b.free()


def _draft_chain(session, hidden, token, pos, n):
    out = []
    h, t = hidden, token
    for i in range(n):
        lg, h = session.draft(h, t, pos + i) if isinstance(session, rf.RefSession) else session.mtp_draft(h, t, pos + i)
        t = int(np.argmax(lg)) if isinstance(session, rf.RefSession) else cpvo.argmax(lg)
        out.append((np.asarray(lg, np.float64), np.asarray(h, np.float64), t))
    return out


def _chain_error(o, r):
    worst = 0.0
    for (lo, ho, to), (lr, hr, tr) in zip(o, r):
        worst = max(worst, np.abs(lo - lr).max() / np.abs(lr).max() / TOL, np.abs(ho - hr).max() / np.abs(hr).max() / TOL)
        s = np.sort(lr)
        if s[-1] - s[-2] > TOL * np.abs(lr).max() and to != tr:
            worst = max(worst, 1e9)
        if to != tr:
            break
    return worst


def _run_drafts(om, tensors, quant=False):
    rm = rf.RefModel(SMALL, tensors, quant_act=quant)
    prompt = np.random.default_rng(9).integers(0, SMALL["n_vocab"], size=24).tolist()
    os_, rs = cpvo.Session(om, 64), rf.RefSession(rm, 64)
    os_.prefill(prompt[:20])
    rs.prefill(prompt[:20])
    _, _, _, _, H = os_.step_fused_cached(prompt[20:], 2, want_logits=True)
    _, _, _, _, Hr = rs.step(prompt[20:], 2)
    # the engine's bookkeeping after a round that kept 1 draft, then a
    # re-draft from the kept row's hidden at rope position n_past
    for s in (os_, rs):
        s.set_pos(22, 2)
    tok = 17
    o = _draft_chain(os_, H[1], tok, 22, 3)
    r = _draft_chain(rs, Hr[1], tok, 22, 3)
    assert os_.pos == (22, 5) and (rs.n_past, rs.mtp_past) == (22, 5)
    os_.free()
    return o, r


@pytest.fixture
def smooth():
    cpvo.set_attn_f64(True)
    cpvo.set_smooth(True)
    yield
    cpvo.set_fault(0)
    cpvo.set_smooth(False)
    cpvo.set_attn_f64(False)


def test_draft_links_match_independent_f64_forward(small, smooth):
    om, tensors = small
    o, r = _run_drafts(om, tensors)
    assert _chain_error(o, r) <= 1.0


@pytest.mark.parametrize("fault", [3, 4, 6])
def test_planted_mistakes_in_a_draft_link_are_caught(small, smooth, fault):
    om, tensors = small
    cpvo.set_fault(fault)
    o, r = _run_drafts(om, tensors)
    cpvo.set_fault(0)
    assert _chain_error(o, r) > 10.0


def test_draft_link_refuses_a_full_mtp_cache_and_bad_positions(small):
    om, _ = small
    s = cpvo.Session(om, 16)
    h = np.ones(SMALL["n_embd"], np.float32)
    s.set_pos(0, 16)
    with pytest.raises(AssertionError):
        s.mtp_draft(h, 1, 0)
    s.set_pos(0, 15)
    with pytest.raises(AssertionError):
        s.mtp_draft(h, 1, 18)
    s.mtp_draft(h, 1, 17)
    assert s.pos == (0, 16)
    s.free()
