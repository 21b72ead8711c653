"""The sampled speculative loop and the losslessness gate on the device,
config-1 model (4 layers, d 512, vocabulary 151,936, Q8_0), against the oracle.

Bar: bit-exact.  The device round reproduces the oracle's round bit for bit
and cpv_spec_accept reproduces cpvo_spec_accept for the same uniforms, so the
same host loop (codpiece_amd.model) driven over the device session and over
the oracle session must commit the same tokens with the same counts and end at
the same positions: rejection at T = 0.7 / top-p 0.95 (the config-5 sampled
leg's setting), gumbel coupling with and without filters, and penalties, each
with the post-commit re-draft off, at the engine's defaults, at a p_min that
keeps some links, and ungated.  The CLI spec path (standalone draft links then
a verify-only round) likewise.  The
uniforms are Philox4x64-10 by role (key seed, round in the counter); the gumbel noise is
generated once on the host and handed to both.

The losslessness gate (scripts/final-verify.sh:15-30): with drafts taken from
the plain greedy stream (so that rounds accept several drafts) and one wrong
draft every third round, the device streams at depths 1-4 equal its plain
greedy stream (depth 0), which equals the oracle's.
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf

pytestmark = pytest.mark.gpu

V = mf.TINY["n_vocab"]
REJECT, GUMBEL = cpvo.ACCEPT_REJECT, cpvo.ACCEPT_GUMBEL


@pytest.fixture(scope="module")
def models():
    from codpiece_amd.model import Model, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    tensors = mf.make_tensors(mf.TINY, seed=0)
    gm = Model(ctx, make_hparams(**mf.TINY))
    mf.load_into(gm, tensors)
    gm.ready()
    om = cpvo.Model(mf.TINY)
    mf.load_into(om, tensors)
    yield ctx, gm, om
    gm.free()
    om.free()
    ctx.close()


def sessions(models, n_ctx=512):
    from codpiece_amd.model import Session
    _, gm, om = models
    return Session(gm, n_ctx), cpvo.Session(om, n_ctx)


def gumbel_noise(seed, temp):
    def noise(r, rows):
        u = np.random.default_rng([seed, r]).random((rows, V), dtype=np.float32)
        u = np.maximum(u, np.float32(1e-12))
        return (-np.log(-np.log(u)) * np.float32(temp)).astype(np.float32)
    return noise


CASES = [
    ("reject_T0.7_top_p0.95", REJECT, dict(temp=0.7, top_p=0.95)),
    ("reject_penalties", REJECT, dict(temp=0.9, top_k=40, penalty_repeat=1.3, penalty_present=0.4,
                                      penalty_last_n=16)),
    ("gumbel_plain", GUMBEL, dict(temp=0.7)),
    ("gumbel_top_p0.95", GUMBEL, dict(temp=0.7, top_p=0.95)),
]


def mixed_pmin(models):
    """A re-draft gate threshold near the median softmax peak of this model's
    draft links (from the oracle), so that re-drafts keep some links and stop
    at others."""
    _, _, om = models
    s = cpvo.Session(om, 64)
    prompt = np.random.default_rng(12).integers(0, V, size=8).tolist()
    _, _, _, _, H = s.step_fused_cached(prompt, 0, want_logits=True)
    peaks = []
    for i in range(8):
        lg, _ = s.mtp_draft(H[i], prompt[(i + 3) % 8], s.pos[0])
        peaks.append(cpvo.softmax_peak_seq(lg))
    s.free()
    return float(np.median(peaks))


# the post-commit re-draft (engine.rs:2584-2625): off, the engine's defaults
# (depth 3, p_min 0.75), a p_min that keeps some links, ungated
REDRAFTS = [("redraft_off", 0, 0.75), ("redraft_default", 3, 0.75), ("redraft_mixed", 3, None),
            ("redraft_ungated", 3, 0.0)]


@pytest.mark.parametrize("rd", REDRAFTS, ids=[r[0] for r in REDRAFTS])
@pytest.mark.parametrize("name,mode,pk", CASES, ids=[c[0] for c in CASES])
def test_sampled_loop_equals_the_oracle_loop(models, name, mode, pk, rd):
    from codpiece_amd.model import sampled_generate
    from codpiece_amd.runtime import SamplerParams
    _, rdepth, pmin = rd
    if pmin is None:
        pmin = mixed_pmin(models)
    g, o = sessions(models)
    prompt = np.random.default_rng(21).integers(0, V, size=96).tolist()
    noise = gumbel_noise(5, pk["temp"])
    print(f"case {name} {rd[0]}", flush=True)
    toks, st = sampled_generate(g, prompt, 24, 3, SamplerParams(**pk), mode, seed=13, tail=32, bulk=64, noise=noise,
                                redraft_depth=rdepth, redraft_pmin=pmin)
    otoks, ost = sampled_generate(mf.OracleSession(o), prompt, 24, 3, cpvo.SamplerParams(**pk), mode, seed=13,
                                  tail=32, bulk=64, noise=noise, redraft_depth=rdepth, redraft_pmin=pmin)
    assert toks == otoks
    assert (st.accepted, st.proposed, st.rounds) == (ost.accepted, ost.proposed, ost.rounds)
    assert (st.redraft_rounds, st.redraft_links) == (ost.redraft_rounds, ost.redraft_links)
    if rdepth and name != "gumbel_plain":      # (plain gumbel commits the graph's argmax: never divergent)
        assert st.redraft_rounds > 0
    assert g.pos == o.pos
    g.free()
    o.free()


@pytest.mark.parametrize("n_spec,p_min", [(1, 0.75), (3, None), (3, 0.0)])
def test_spec_path_equals_the_oracle(models, n_spec, p_min):
    """The CLI spec path (crates/codpiece-cli/src/main.rs:1040-1160): standalone
    draft links, a verify-only round, greedy acceptance, both positions rewound."""
    from codpiece_amd.model import spec_generate
    if p_min is None:
        p_min = mixed_pmin(models)
    g, o = sessions(models)
    prompt = np.random.default_rng(23).integers(0, V, size=80).tolist()
    print(f"case spec n_spec={n_spec} p_min={p_min}", flush=True)
    toks, st = spec_generate(g, prompt, 24, n_spec, p_min, tail=16, bulk=64)
    otoks, ost = spec_generate(mf.OracleSession(o), prompt, 24, n_spec, p_min, tail=16, bulk=64)
    assert toks == otoks
    assert (st.accepted, st.proposed, st.rounds, st.redraft_links) == (ost.accepted, ost.proposed, ost.rounds,
                                                                         ost.redraft_links)
    assert g.pos == o.pos
    g.free()
    o.free()


def _drafter(stream, depth, spoil_every=3):
    state = {"round": 0}

    def drafter(committed, chain):
        state["round"] += 1
        n = len(committed)
        d = [stream[i] for i in range(n, min(n + depth, len(stream)))]
        if d and state["round"] % spoil_every == 0:
            j = state["round"] % len(d)
            d[j] = (d[j] + 1) % V
        return d
    return drafter


def test_losslessness_gate_on_the_device(models):
    from codpiece_amd.model import fused_generate
    prompt = np.random.default_rng(8).integers(0, V, size=80).tolist()
    g0, o0 = sessions(models)
    plain, st0 = fused_generate(g0, prompt, 32, 0, tail=16, bulk=64)
    oplain, _ = fused_generate(mf.OracleSession(o0), prompt, 32, 0, tail=16, bulk=64)
    assert plain == oplain and st0.rounds == 31
    for depth in (1, 2, 3, 4):
        print(f"case depth={depth}", flush=True)
        g, o = sessions(models)
        toks, st = fused_generate(g, prompt, 32, depth, tail=16, bulk=64, drafter=_drafter(plain, depth))
        otoks, ost = fused_generate(mf.OracleSession(o), prompt, 32, depth, tail=16, bulk=64,
                                    drafter=_drafter(plain, depth))
        assert toks == plain == otoks
        assert st.accepted > st.rounds // 2 and st.accepted < st.proposed
        assert (st.accepted, st.proposed, st.rounds) == (ost.accepted, ost.proposed, ost.rounds)
        assert g.pos == o.pos
        g.free()
        o.free()
    g0.free()
    o0.free()
