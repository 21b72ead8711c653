"""The reference sampler's own tests (crates/codpiece-sample/src/lib.rs:473-718),
re-expressed against the oracle's restatement, plus the acceptance rules."""
import numpy as np
import pytest

from oracle import cpvo
from oracle.cpvo import SamplerParams as P


def s(**kw):
    seed = kw.pop("seed", 0)
    return cpvo.Sampler(P(**kw), seed)


def test_temp_zero_is_argmax():                                  # :481-490
    logits = np.array([0.1, 5.0, -2.0, 4.9], dtype=np.float32)
    for top_k in [0, 1, 2, 4]:
        for top_p in [1.0, 0.5]:
            assert s(top_k=top_k, top_p=top_p).sample(logits) == 1


def test_top_k_one_is_argmax_at_any_temperature():               # :492-499
    smp = s(temp=2.0, top_k=1)
    for _ in range(50):
        assert smp.sample(np.array([1.0, 3.0, 2.0], dtype=np.float32)) == 1


def test_top_p_includes_the_crossing_token():                    # :501-512
    smp = s(temp=1.0, top_p=0.7)
    seen = {smp.sample(np.array([2.0, 1.0, 0.0], dtype=np.float32)) for _ in range(2000)}
    assert seen == {0, 1}


def test_min_p_thresholds_relative_to_the_peak():                # :514-529
    logits = np.array([2.0, 1.0, 0.0], dtype=np.float32)
    smp = s(temp=1.0, min_p=0.5)
    assert all(smp.sample(logits) == 0 for _ in range(500))
    smp = s(temp=1.0, min_p=0.3)
    assert {smp.sample(logits) for _ in range(4000)} == {0, 1}


def test_repeat_penalty_pushes_a_repeated_token_down():          # :531-538
    smp = s(penalty_repeat=2.0)
    logits = np.array([5.0, 4.9], dtype=np.float32)
    assert smp.sample(logits) == 0
    smp.accept(0)
    assert smp.sample(logits) == 1


def test_repeat_penalty_does_not_promote_negative_logits():      # :540-549
    smp = s(penalty_repeat=2.0)
    logits = np.array([-1.0, -1.5], dtype=np.float32)
    assert smp.sample(logits) == 0
    smp.accept(0)
    assert smp.sample(logits) == 1


def test_a_seed_reproduces_a_run():                              # :551-560
    logits = np.array([1.0, 1.1, 0.9, 1.05], dtype=np.float32)

    def run(seed):
        smp = s(temp=1.0, seed=seed)
        return [smp.sample(logits) for _ in range(64)]
    assert run(42) == run(42) and run(42) != run(43)


def test_the_draw_follows_the_distribution():                    # :562-571
    logits = np.array([0.0, np.log(np.float32(3.0))], dtype=np.float32)
    smp = s(temp=1.0, seed=7)
    n = 40000
    frac = sum(smp.sample(logits) == 1 for _ in range(n)) / n
    assert abs(frac - 0.75) < 0.01


def test_temperature_flattens():                                 # :573-586
    logits = np.array([0.0, np.log(np.float32(3.0))], dtype=np.float32)
    hot = s(temp=8.0, seed=3)
    cold = s(temp=0.25, seed=3)
    h = sum(hot.sample(logits) == 1 for _ in range(20000))
    c = sum(cold.sample(logits) == 1 for _ in range(20000))
    assert h < c and c > 19000


def test_a_greedy_distribution_is_a_point_mass():               # :588-597
    d = s().distribution(np.array([1.0, 4.0, 2.0], dtype=np.float32))
    assert len(d) == 1 and d.prob_of(1) == 1.0 and d.prob_of(0) == 0.0


def test_a_filtered_token_has_no_probability():                  # :599-607
    d = s(temp=1.0, top_k=1).distribution(np.array([2.0, 1.0, 0.0], dtype=np.float32))
    assert d.prob_of(0) == 1.0 and d.prob_of(2) == 0.0


def test_draw_excluding_never_returns_the_excluded_token():     # :609-618
    d = s(temp=1.0).distribution(np.array([2.0, 1.0, 0.0], dtype=np.float32))
    for i in range(1000):
        assert d.draw_excluding(0, np.float32(i / 1000)) != 0


def test_the_acceptance_rule_reproduces_the_target_distribution():  # :626-653
    logits = np.array([1.0, 0.5, 0.0, -0.5], dtype=np.float32)
    smp = s(temp=1.0, seed=11)
    target = smp.distribution(logits)
    n = 200000
    counts = np.zeros(4)
    for _ in range(n):
        roll = smp.rng.next_f32()
        if roll < target.prob_of(0):
            tok = 0
        else:
            tok = target.draw_excluding(0, smp.rng.next_f32())
        counts[tok] += 1
    for t in range(4):
        assert abs(counts[t] / n - target.prob_of(t)) < 0.005


@pytest.mark.parametrize("label,params", [
    ("plain", dict(temp=0.9, seed=7)),
    ("filtered", dict(temp=1.1, top_k=3, top_p=0.95, seed=7)),
])
def test_coupled_sampling_emits_the_target_distribution(label, params):  # :655-709
    logits = np.array([1.0, 0.3, -0.5, 0.05], dtype=np.float32)
    smp = s(**params)
    target = smp.distribution(logits)
    n = 200000
    counts = np.zeros(4)
    agree = 0
    T = np.float32(params["temp"])
    for _ in range(n):
        u = np.array([max(smp.rng.next_f32(), 1e-12) for _ in range(4)], dtype=np.float32)
        noise = (-np.log(-np.log(u.astype(np.float64)))).astype(np.float32) * T
        tok = smp.sample_coupled(logits, noise)
        counts[tok] += 1
        graph = int(np.argmax(logits + noise))
        agree += graph == tok
    for t in range(4):
        assert abs(counts[t] / n - target.prob_of(t)) < 0.005, (label, t)
    if label == "plain":
        assert agree == n
    else:
        assert agree / n > 0.8


def test_greedy_when_no_filter_reports():                         # :711-717 (is_greedy)
    # the greedy acceptance path is the raw argmax; with temp <= 0 the
    # distribution's point mass is that same argmax, lowest index on ties
    x = np.array([1.0, 3.0, 3.0, 0.0], dtype=np.float32)
    assert cpvo.argmax(x) == 1
    assert s().distribution(x).ids.tolist() == [1]


# ---- acceptance (crates/codpiece-server/src/engine.rs:2326-2461) ----------------

def _logits(rng, B, k1, V, spike=8.0):
    l = rng.normal(0, 3, size=(B, k1, V)).astype(np.float32)
    for b in range(B):
        for j in range(k1):
            l[b, j, rng.integers(V)] += spike
    return l


def test_role_mapped_uniforms_reproduce_the_sequential_engine_loop():
    rng = np.random.default_rng(0)
    V, k = 2000, 4
    params = P(temp=0.7, top_p=0.95)
    for trial in range(40):
        pl = _logits(rng, 1, k + 1, V)[0]
        # drafts: argmax of the target at some positions (accepted), noise at others
        drafts = np.array([int(np.argmax(pl[j])) if rng.random() < 0.7 else int(rng.integers(V))
                           for j in range(k)], dtype=np.int32)
        r = cpvo.Rng(1000 + trial)
        tok_seq, n_seq, used = cpvo.spec_accept_rng(pl, drafts, params, r)
        u = np.where(np.isnan(used), np.float32(0.5), used).astype(np.float32)[None]
        tok, n = cpvo.spec_accept(pl[None], drafts[None], params, cpvo.ACCEPT_REJECT, u=u)
        assert n[0] == n_seq
        assert tok[0, :n_seq + 1].tolist() == tok_seq[:n_seq + 1].tolist()


def test_greedy_acceptance_is_the_longest_matching_prefix():
    rng = np.random.default_rng(1)
    V, k = 500, 4
    pl = _logits(rng, 3, k + 1, V)
    am = pl.argmax(axis=2)
    drafts = am[:, :k].copy()
    drafts[1, 2] = (drafts[1, 2] + 1) % V          # row 1 rejects at 2
    drafts[2, 0] = (drafts[2, 0] + 1) % V          # row 2 rejects at 0
    tok, n = cpvo.spec_accept(pl, drafts, P(), cpvo.ACCEPT_GREEDY)
    assert n.tolist() == [4, 2, 0]
    assert tok[0].tolist() == am[0].tolist()
    assert tok[1, :3].tolist() == am[1, :3].tolist()
    assert tok[2, 0] == am[2, 0]


def test_general_rule_reduces_to_the_reference_rule_for_one_hot_drafts():
    rng = np.random.default_rng(2)
    V, k, B = 1500, 4, 6
    params = P(temp=0.7, top_p=0.95)
    pl = _logits(rng, B, k + 1, V)
    drafts = rng.integers(V, size=(B, k)).astype(np.int32)
    for b in range(B):
        for j in range(k):
            if rng.random() < 0.6:
                drafts[b, j] = int(np.argmax(pl[b, j]))
    q = np.full((B, k, V), -1e4, dtype=np.float32)
    for b in range(B):
        for j in range(k):
            q[b, j, drafts[b, j]] = 1e4
    u = cpvo.philox_uniforms(99, B, k)
    t1, n1 = cpvo.spec_accept(pl, drafts, params, cpvo.ACCEPT_REJECT, u=u)
    t2, n2 = cpvo.spec_accept(pl, drafts, params, cpvo.ACCEPT_REJECT, u=u, q_logits=q)
    assert np.array_equal(n1, n2)
    for b in range(B):
        assert t1[b, :n1[b] + 1].tolist() == t2[b, :n2[b] + 1].tolist()


def test_general_rule_emits_the_target_distribution():
    # closed form: one draft drawn from q, accepted with min(1, p/q), residual
    # max(0, p - q): the emitted token follows p exactly
    V = 6
    pl = np.array([[[1.0, 0.5, 0.0, -0.5, 0.2, -1.0], [0.0] * 6]], dtype=np.float32)
    ql = np.array([[[0.0, 1.0, 0.5, 0.0, -1.0, 0.3]]], dtype=np.float32)
    params = P(temp=1.0)
    pd = cpvo.Sampler(params).distribution(pl[0, 0])
    qd = cpvo.Sampler(params).distribution(ql[0, 0])
    pv = np.array([pd.prob_of(i) for i in range(V)])
    n = 60000
    counts = np.zeros(V)
    rng = np.random.default_rng(5)
    for i in range(n):
        x = qd.draw(np.float32(rng.random()))
        u = rng.random(size=(1, 2, 2)).astype(np.float32)
        tok, na = cpvo.spec_accept(pl, np.array([[x]]), params, cpvo.ACCEPT_REJECT, u=u, q_logits=ql)
        counts[tok[0, 0]] += 1
    assert np.abs(counts / n - pv).max() < 0.01


def test_gumbel_plain_acceptance_matches_the_in_graph_argmax():
    rng = np.random.default_rng(3)
    V, k, B = 800, 3, 4
    params = P(temp=0.7)
    pl = _logits(rng, B, k + 1, V)
    u = rng.random(size=(B, k + 1, V)).astype(np.float32)
    noise = (-np.log(-np.log(np.maximum(u, 1e-12)))).astype(np.float32) * np.float32(0.7)
    graph = (pl + noise).argmax(axis=2)
    drafts = graph[:, :k].copy()
    drafts[0, 1] = (drafts[0, 1] + 3) % V
    tok, n = cpvo.spec_accept(pl, drafts, params, cpvo.ACCEPT_GUMBEL, noise_t=noise)
    assert n.tolist() == [1, 3, 3, 3]
    assert tok[0, :2].tolist() == graph[0, :2].tolist()
    assert tok[1].tolist() == graph[1].tolist()


def test_penalty_window_grows_with_accepted_drafts():
    # the engine calls sampler.accept(draft) after each kept draft
    # (engine.rs:2368-2369): a repeat penalty then changes later positions
    V = 4
    pl = np.array([[[0.0, 5.0, 4.9, 0.0], [0.0, 5.0, 4.9, 0.0], [0.0, 5.0, 4.9, 0.0]]],
                  dtype=np.float32)
    params = P(temp=0.0, penalty_repeat=2.0)
    u = np.zeros((1, 3, 2), dtype=np.float32)
    drafts = np.array([[1, 2]], dtype=np.int32)
    tok, n = cpvo.spec_accept(pl, drafts, params, cpvo.ACCEPT_REJECT, u=u)
    # position 0: argmax 1 (accepted); position 1: token 1 penalised to 2.5,
    # argmax 2 (accepted); position 2: 1 and 2 penalised, argmax of [0, 2.5, 2.45, 0] = 1
    assert n[0] == 2 and tok[0].tolist() == [1, 2, 1]
