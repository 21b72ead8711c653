"""The sampled speculative loop and the losslessness gate, on the CPU.

(1) codpiece_amd.model.sampled_generate, driven over the oracle session (whose
acceptance is cpvo_spec_accept), commits the same tokens and counts as an
independent restatement of the engine's loop written here from
crates/codpiece-server/src/engine.rs:1958-2039 and 2212-2625 with the
codpiece-sample primitives (Sampler::distribution, Dist::prob_of / draw /
draw_excluding, sample_coupled), draft by draft, on the same uniforms by role
(Philox4x64-10, key seed, counter (0, j, role, round)) and the same gumbel
noise.  Rejection, gumbel coupling with and without filters, and penalties;
with the post-commit re-draft (:2584-2625: standalone draft links from the
kept row's hidden, gated by the softmax peak, computed here as a numpy
float32 sequential sum) off, at the engine's default p_min 0.75, at a p_min
that passes some links and stops others, and ungated.  The CLI spec path
(crates/codpiece-cli/src/main.rs:1040-1160) and mtp-probe (:1250-1285) are
restated the same way.
(2) The losslessness gate of scripts/final-verify.sh:15-30: greedy streams at
draft depths 1-4 equal plain greedy decoding (depth 0).  Random MTP drafts are
almost never accepted, so the drafts are taken from the plain greedy stream
itself (every round fully accepted) and, in every third round, with one wrong
token (a partial accept and a rewind); the stream must not change.
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf

SMALL = dict(mf.TINY, n_layer=2, n_vocab=4096)
REJECT, GUMBEL = cpvo.ACCEPT_REJECT, cpvo.ACCEPT_GUMBEL


@pytest.fixture(scope="module")
def om():
    m = cpvo.Model(SMALL)
    mf.load_into(m, mf.make_tensors(SMALL, seed=3))
    yield m
    m.free()


def gumbel_noise(seed, temp, V):
    """T-scaled gumbel noise for round r (the engine's noise thread,
    engine.rs:2098-2114: -ln(-ln(max(u, 1e-12))) * T), from numpy."""
    def noise(r, rows):
        u = np.random.default_rng([seed, r]).random((rows, V), dtype=np.float32)
        u = np.maximum(u, np.float32(1e-12))
        return (-np.log(-np.log(u)) * np.float32(temp)).astype(np.float32)
    return noise


def seq_peak(l):
    """1 / lse, lse the float32 sequential sum of exp(l - max) (engine.rs:2603-2605)."""
    l = np.asarray(l, np.float32)
    e = cpvo.expf((l - np.float32(l.max())).astype(np.float32))
    return np.float32(1.0) / np.add.accumulate(e, dtype=np.float32)[-1]


def engine_restatement(osess, prompt, n_gen, depth, params, mode, seed, tail, bulk, noise=None,
                       redraft_depth=0, redraft_pmin=0.75):
    """engine.rs's single-request sampled loop, draft by draft."""
    sampler = cpvo.Sampler(params)
    plain = (params.temp > 0 and params.top_k == 0 and params.top_p >= 1.0 and params.min_p <= 0.0
             and params.penalty_repeat == 1.0 and params.penalty_freq == 0.0 and params.penalty_present == 0.0)
    for t in prompt:                                   # sampler.accept_all(text_ids)
        sampler.accept(t)
    split = max(0, len(prompt) - tail)
    for c in range(0, split, bulk):
        osess.prefill(prompt[c:min(split, c + bulk)])
    P, C, CF, L, _ = osess.step_fused_cached(prompt[split:], depth, want_logits=True)
    n_past, mtp_past = osess.pos
    osess.set_pos(n_past, mtp_past + len(P))          # session.mtp_past += preds.len()
    at = len(P) - 1
    u0 = cpvo.philox_uniforms(seed, 1, 0)[0]
    nxt = sampler.distribution(L[at]).draw(u0[0][0])   # sampler.draw_from(&d)
    drafts = [int(C[l][at]) for l in range(depth)]
    sampler.accept(nxt)
    committed = [int(nxt)]
    acc = prop = rounds = 0
    while len(committed) < n_gen:
        rounds += 1
        batch = [committed[-1]] + drafts
        k = len(drafts)
        nz = noise(rounds, len(batch)) if mode == GUMBEL else None
        P, C, CF, L, H = osess.step_fused_cached(batch, depth, want_logits=True, noise=nz)
        prop += k
        u = cpvo.philox_uniforms(seed, 1, k, round=rounds)[0]
        n_keep, repl = 0, None
        for j, d in enumerate(drafts):
            if mode == GUMBEL:
                commit = int(P[j]) if plain else sampler.sample_coupled(L[j], nz[j])
                keep = d == commit
                if not keep:
                    repl = commit
            else:
                dist = sampler.distribution(L[j])
                keep = u[j][0] < dist.prob_of(d)
                if not keep:
                    repl = dist.draw_excluding(d, u[j][1])
            if not keep:
                break
            n_keep += 1
            sampler.accept(d)
        acc += n_keep
        done = False
        for d in drafts[:n_keep]:
            committed.append(int(d))
            if len(committed) >= n_gen:
                done = True
                break
        if done:
            break
        if repl is not None:
            nxt = repl
        elif mode == GUMBEL:
            nxt = int(P[n_keep]) if plain else sampler.sample_coupled(L[n_keep], nz[n_keep])
        else:
            nxt = sampler.distribution(L[n_keep]).draw(u[k][0])
        sampler.accept(nxt)
        committed.append(int(nxt))
        drafts = [int(C[l][n_keep]) for l in range(depth)]
        if nxt != P[n_keep]:
            drafts = []
        over = len(batch) - (n_keep + 1)
        n_past, mtp_past = osess.pos
        osess.set_pos(n_past - over, mtp_past + n_keep + 1)
        if not drafts and redraft_depth > 0:            # engine.rs:2584-2625
            h, tok_in, pos = H[n_keep], nxt, osess.pos[0]
            for _ in range(redraft_depth):
                lg, hn = osess.mtp_draft(h, tok_in, pos)
                d = int(np.argmax(lg))                 # first maximum, as qwen35.rs:3659-3669
                if redraft_pmin > 0.0 and seq_peak(lg) < np.float32(redraft_pmin):
                    break
                drafts.append(d)
                tok_in, h, pos = d, hn, pos + 1
            drafts = drafts[:depth]
    return committed, (acc, prop, rounds)


CASES = [
    ("reject", REJECT, dict(temp=0.7, top_p=0.95)),
    ("reject_penalties", REJECT, dict(temp=0.9, top_k=40, penalty_repeat=1.3, penalty_present=0.4,
                                      penalty_last_n=16)),
    ("gumbel_plain", GUMBEL, dict(temp=0.7)),
    ("gumbel_top_p", GUMBEL, dict(temp=0.7, top_p=0.95)),
]


# the re-draft: off; the engine's defaults (on random weights every first link
# is below 0.75, so each divergent round runs one link and stops); a p_min
# between the typical peaks of this model's links (some pass, some stop);
# ungated
REDRAFTS = [("off", 0, 0.75), ("default", 3, 0.75), ("mixed", 3, None), ("ungated", 3, 0.0)]


def mixed_pmin(om):
    """A gate threshold near the median softmax peak of this model's draft
    links, so that a re-draft keeps some links and stops at others."""
    s = cpvo.Session(om, 64)
    prompt = np.random.default_rng(12).integers(0, SMALL["n_vocab"], size=8).tolist()
    _, _, _, _, H = s.step_fused_cached(prompt, 0, want_logits=True)
    peaks = []
    for i in range(8):
        lg, _ = s.mtp_draft(H[i % len(prompt)], prompt[(i + 3) % len(prompt)], s.pos[0])
        peaks.append(float(seq_peak(lg)))
    s.free()
    return float(np.median(peaks))


@pytest.mark.parametrize("rd", REDRAFTS, ids=[r[0] for r in REDRAFTS])
@pytest.mark.parametrize("name,mode,pk", CASES, ids=[c[0] for c in CASES])
def test_sampled_loop_matches_engine_restatement(om, name, mode, pk, rd):
    from codpiece_amd.model import sampled_generate
    _, rdepth, pmin = rd
    if pmin is None:
        pmin = mixed_pmin(om)
    params = cpvo.SamplerParams(**pk)
    prompt = np.random.default_rng(5).integers(0, SMALL["n_vocab"], size=60).tolist()
    noise = gumbel_noise(11, params.temp, SMALL["n_vocab"])
    a, b = cpvo.Session(om, 256), cpvo.Session(om, 256)
    toks, st = sampled_generate(mf.OracleSession(a), prompt, 40, 3, params, mode, seed=9, tail=16, bulk=32,
                                noise=noise, redraft_depth=rdepth, redraft_pmin=pmin)
    rtoks, rst = engine_restatement(b, prompt, 40, 3, params, mode, 9, 16, 32, noise, rdepth, pmin)
    assert toks == rtoks
    assert (st.accepted, st.proposed, st.rounds) == rst
    assert a.pos == b.pos
    if name == "gumbel_plain":
        # the commit is the graph's own gumbel argmax, so no round diverges
        assert st.redraft_rounds == 0
    elif rdepth:
        assert st.redraft_rounds > 0 and st.redraft_links >= st.redraft_rounds
    if rd[0] == "mixed" and name != "gumbel_plain":
        assert st.redraft_rounds < st.redraft_links < 3 * st.redraft_rounds   # some links stop, some pass
    a.free()
    b.free()


def spec_restatement(osess, prompt, n_gen, n_spec, p_min, tail, bulk):
    """cmd_spec (crates/codpiece-cli/src/main.rs:1040-1160) with no context
    oracle, draft by draft."""
    split = max(0, len(prompt) - tail)
    for c in range(0, split, bulk):
        osess.prefill(prompt[c:min(split, c + bulk)])
    P, _, _, _, H = osess.step_fused_cached(prompt[split:], 0, want_logits=True)
    committed, hidden = [int(P[-1])], H[-1]
    acc = prop = rounds = 0
    while len(committed) < n_gen:
        last = committed[-1]
        drafts, h, tok_in, pos = [], hidden, last, osess.pos[0]
        for _ in range(n_spec):
            lg, dh = osess.mtp_draft(h, tok_in, pos)
            d = int(np.argmax(lg))
            if seq_peak(lg) < np.float32(p_min):       # softmax_prob(dl, d) at the argmax
                n_past, mtp_past = osess.pos
                osess.set_pos(n_past, mtp_past - 1)   # the slot is given back
                break
            drafts.append(d)
            tok_in, pos, h = d, pos + 1, dh
        P, _, _, _, H = osess.step_fused_cached([last] + drafts, 0, want_logits=True)
        rounds += 1
        prop += len(drafts)
        n_keep = 0
        while n_keep < len(drafts) and P[n_keep] == drafts[n_keep]:
            n_keep += 1
        acc += n_keep
        stop = False
        for d in drafts[:n_keep]:
            committed.append(d)
            if len(committed) >= n_gen:
                stop = True
                break
        if stop:
            break
        committed.append(int(P[n_keep]))
        hidden = H[n_keep]
        extra = len(drafts) - n_keep
        if extra:
            n_past, mtp_past = osess.pos
            osess.set_pos(n_past - extra, mtp_past - extra)
    return committed, (acc, prop, rounds)


@pytest.mark.parametrize("n_spec,p_min", [(1, 0.75), (3, None), (3, 0.0)])
def test_spec_path_matches_cli_restatement(om, n_spec, p_min):
    from codpiece_amd.model import spec_generate
    if p_min is None:
        p_min = mixed_pmin(om)
    prompt = np.random.default_rng(15).integers(0, SMALL["n_vocab"], size=40).tolist()
    a, b = cpvo.Session(om, 256), cpvo.Session(om, 256)
    toks, st = spec_generate(mf.OracleSession(a), prompt, 30, n_spec, p_min, tail=8, bulk=16)
    rtoks, rst = spec_restatement(b, prompt, 30, n_spec, p_min, 8, 16)
    assert toks == rtoks
    assert (st.accepted, st.proposed, st.rounds) == rst
    assert a.pos == b.pos
    # greedy acceptance: the stream is plain greedy decoding whatever the drafts
    g = cpvo.Session(om, 256)
    plain, _ = g.fused_generate(prompt, 30, 0, tail=8, bulk=16)
    assert toks == plain
    for x in (a, b, g):
        x.free()


def test_mtp_probe_counts_the_links_hits(om):
    from codpiece_amd.model import mtp_probe
    prompt = np.random.default_rng(16).integers(0, SMALL["n_vocab"], size=30).tolist()
    a, b = cpvo.Session(om, 256), cpvo.Session(om, 256)
    stream, hits, total = mtp_probe(mf.OracleSession(a), prompt, 12, tail=8, bulk=16)
    plain, _ = b.fused_generate(prompt, 13, 0, tail=8, bulk=16)
    assert stream == plain and total == 11
    # each link drafts the token after next from (hidden at pos, next): the
    # draft of step i is compared with the greedy token of step i + 1
    assert 0 <= hits <= total
    assert a.pos == (len(prompt) + 12, 12)
    a.free()
    b.free()


def test_sampled_loop_accepts_drafts_with_a_peaked_target(om):
    # at a very low temperature the target is nearly one-hot on the argmax:
    # the plain gumbel commit is the trunk's argmax, drafts from the greedy
    # stream are kept, and the sampled stream is the greedy one
    from codpiece_amd.model import fused_generate, sampled_generate
    prompt = np.random.default_rng(6).integers(0, SMALL["n_vocab"], size=40).tolist()
    g0 = cpvo.Session(om, 256)
    greedy, _ = fused_generate(mf.OracleSession(g0), prompt, 24, 0, tail=8, bulk=32)
    s = cpvo.Session(om, 256)
    params = cpvo.SamplerParams(temp=1e-4)
    noise = gumbel_noise(3, params.temp, SMALL["n_vocab"])
    toks, st = sampled_generate(mf.OracleSession(s), prompt, 24, 3, params, GUMBEL, seed=1, tail=8, bulk=32,
                                noise=noise, drafter=_lossless_drafter(greedy, 3, spoil_every=10 ** 9))
    assert toks == greedy
    assert st.accepted == st.proposed > 0
    g0.free()
    s.free()


def _lossless_drafter(stream, depth, spoil_every=3):
    state = {"round": 0}

    def drafter(committed, chain):
        state["round"] += 1
        n = len(committed)
        d = [stream[i] for i in range(n, min(n + depth, len(stream)))]
        if d and state["round"] % spoil_every == 0:
            j = state["round"] % len(d)
            d[j] = (d[j] + 1) % SMALL["n_vocab"]
        return d
    return drafter


@pytest.mark.parametrize("depth", [1, 2, 3, 4])
def test_losslessness_gate_fused_depths_equal_plain_greedy(om, depth):
    from codpiece_amd.model import fused_generate
    prompt = np.random.default_rng(7).integers(0, SMALL["n_vocab"], size=50).tolist()
    s0 = cpvo.Session(om, 256)
    plain, st0 = fused_generate(mf.OracleSession(s0), prompt, 40, 0, tail=10, bulk=32)
    assert st0.accepted == 0 and st0.rounds == 39
    s = cpvo.Session(om, 256)
    toks, st = fused_generate(mf.OracleSession(s), prompt, 40, depth, tail=10, bulk=32,
                              drafter=_lossless_drafter(plain, depth))
    assert toks == plain
    assert st.accepted > st.rounds // 2          # multi-accept rounds happened
    assert st.accepted < st.proposed             # and rejected drafts were rewound
    # positions: every committed token but the last is in the trunk cache,
    # and the MTP rows are the tail round's plus n_keep + 1 per round, unless
    # the last round ended inside its accepted drafts (no rewind then)
    if s.pos[0] == len(prompt) + len(plain) - 1:
        assert s.pos[1] == 10 + st.accepted + st.rounds
    else:
        assert len(prompt) + len(plain) - 1 < s.pos[0] <= len(prompt) + len(plain) - 1 + depth
    # the MTP drafts of the same loop (never accepted on random weights) give the same stream
    s2 = cpvo.Session(om, 256)
    toks2, _ = fused_generate(mf.OracleSession(s2), prompt, 40, depth, tail=10, bulk=32)
    assert toks2 == plain
    for x in (s0, s, s2):
        x.free()
