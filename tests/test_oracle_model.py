"""The oracle's verify round and the host loop, on the CPU (no GPU needed).

Pins: (1) the host loop in codpiece_amd.model.fused_generate, driven over the
oracle session, commits the same tokens and counts as the oracle's C
restatement of cmd_fused (crates/codpiece-cli/src/main.rs:643-931);
(2) batch invariance -- every row's logits depend only on its own token and
the tokens before it (per-row activation quantization, exact GEMMs and per-row
f64 attention), so a verify of T rows equals T single-row steps bit for bit,
which fixes the causal mask, positions and KV writes;
(3) rewind -- after set_pos(n_past - over, .) a redo equals a fresh run;
(4) the MTP cache window restarts at 0 when it would overflow.
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf

SMALL = dict(mf.TINY, n_layer=2, n_vocab=4096)


@pytest.fixture(scope="module")
def om():
    m = cpvo.Model(SMALL)
    mf.load_into(m, mf.make_tensors(SMALL, seed=3))
    yield m
    m.free()


def test_host_loop_matches_oracle_loop(om):
    from codpiece_amd.model import fused_generate
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, SMALL["n_vocab"], size=90).tolist()
    a = cpvo.Session(om, 256)
    b = cpvo.Session(om, 256)
    toks, st = fused_generate(mf.OracleSession(a), prompt, 24, 3, tail=16, bulk=32)
    otoks, ost = b.fused_generate(prompt, 24, 3, tail=16, bulk=32)
    assert toks == otoks
    assert [st.accepted, st.proposed, st.rounds] == ost
    assert a.pos == b.pos
    a.free()
    b.free()


def test_verify_rows_equal_single_steps(om):
    rng = np.random.default_rng(4)
    toks = rng.integers(0, SMALL["n_vocab"], size=12).tolist()
    a = cpvo.Session(om, 64)
    a.prefill(toks[:7])
    _, _, _, la, _ = a.step_fused_cached(toks[7:], 0, want_logits=True)
    b = cpvo.Session(om, 64)
    b.prefill(toks[:7])
    rows = []
    for t in toks[7:]:
        _, _, _, l1, _ = b.step_fused_cached([t], 0, want_logits=True)
        rows.append(l1[0])
    assert np.array_equal(la, np.stack(rows))
    assert a.pos == b.pos == (12, 0)
    a.free()
    b.free()


def test_prefill_equals_verify_trunk(om):
    rng = np.random.default_rng(5)
    toks = rng.integers(0, SMALL["n_vocab"], size=9).tolist()
    a = cpvo.Session(om, 64)
    a.prefill(toks[:8])
    _, _, _, la, _ = a.step_fused_cached(toks[8:], 0, want_logits=True)
    b = cpvo.Session(om, 64)
    b.prefill(toks[:3])
    b.prefill(toks[3:8])
    _, _, _, lb, _ = b.step_fused_cached(toks[8:], 0, want_logits=True)
    assert np.array_equal(la, lb)
    a.free()
    b.free()


def test_rewind_equals_fresh_run(om):
    rng = np.random.default_rng(6)
    toks = rng.integers(0, SMALL["n_vocab"], size=14).tolist()
    alt = rng.integers(0, SMALL["n_vocab"], size=3).tolist()
    a = cpvo.Session(om, 64)
    a.prefill(toks[:9])
    a.step_fused_cached(toks[9:], 2)            # 5 rows, then reject the last 3
    a.set_pos(11, 0)
    pa, ca, _, la, _ = a.step_fused_cached(alt, 2, want_logits=True)
    b = cpvo.Session(om, 64)
    b.prefill(toks[:11])
    pb, cb, _, lb, _ = b.step_fused_cached(alt, 2, want_logits=True)
    assert np.array_equal(la, lb)
    assert np.array_equal(pa, pb)
    assert np.array_equal(ca, cb)
    a.free()
    b.free()


def test_mtp_window_restarts_when_full(om):
    a = cpvo.Session(om, 16)                    # mtp window = min(n_ctx, 16384) = 16
    a.set_pos(0, 14)
    a.step_fused_cached([1, 2, 3], 1)
    # 14 + 3 > 16: the draft head's window restarts at 0 before the round
    assert a.pos == (3, 0)
    a.free()


def test_context_overflow_is_refused(om):
    a = cpvo.Session(om, 8)
    a.prefill(list(range(6)))
    with pytest.raises(AssertionError):
        a.step_fused_cached([1, 2, 3], 0)
    a.free()
