"""GPU parity of the target distributions and of speculative acceptance.

Bar: bit-exact.  The device sampler reproduces the CPU sampler's f32
arithmetic, sequential sums included (crates/codpiece-sample/src/lib.rs:
229-471), so ids, probabilities, accept counts and emitted tokens must equal
the oracle's exactly for the same logits and uniforms.  The headline shapes
are B in {1, 4, 16} sequences x k+1 = 5 rows x V = 151936 logits ~ N(0, 3)
with a +8 spike, T = 0.7, top-p 0.95, uniforms from Philox4x64-10.
"""
import zlib

import numpy as np
import pytest
import torch

from oracle import cpvo

pytestmark = pytest.mark.gpu

V27 = 151936


@pytest.fixture(scope="module")
def ctx():
    from codpiece_amd.runtime import Context
    c = Context(0)
    yield c
    c.close()


def dev_params(p):
    from codpiece_amd.runtime import SamplerParams
    return SamplerParams(p.temp, p.top_k, p.top_p, p.min_p, p.min_keep, p.penalty_repeat, p.penalty_freq,
                         p.penalty_present, p.penalty_last_n)


def spiked(rng, shape, sd=3.0, spike=8.0):
    x = rng.normal(0, sd, size=shape).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    for r in range(flat.shape[0]):
        flat[r, rng.integers(shape[-1])] += np.float32(spike)
    return x


def check_dist(ctx, logits, p, hist=None):
    """Device distribution of each row == oracle distribution, bit for bit."""
    rows, v = logits.shape
    h = None if hist is None else torch.from_numpy(np.ascontiguousarray(hist, dtype=np.int32)).cuda()
    ids, probs, n = ctx.distribution(torch.from_numpy(logits).cuda(), dev_params(p), h)
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        hr = None if hist is None else [t for t in hist[r] if t >= 0][-p.penalty_last_n:] if p.penalty_last_n else []
        rid, rp, _ = cpvo.distribution(p, logits[r], hr)
        assert n[r] == rid.size, (r, n[r], rid.size)
        assert np.array_equal(ids[r, :n[r]], rid), r
        bad = np.flatnonzero(probs[r, :n[r]].view(np.uint32) != rp.view(np.uint32))
        assert bad.size == 0, (r, bad[:5], probs[r, bad[:5]], rp[bad[:5]])
    return n


DIST_CASES = {
    "top_p_0.95_T0.7": dict(temp=0.7, top_p=0.95),
    "no_filter_T0.7": dict(temp=0.7),
    "top_k_40_T0.8": dict(temp=0.8, top_k=40),
    "top_k_50_top_p_0.9_min_p_0.05": dict(temp=1.0, top_k=50, top_p=0.9, min_p=0.05),
    "min_p_0.05_T0.7": dict(temp=0.7, min_p=0.05),
    "min_p_0.002_top_p_0.9": dict(temp=1.3, min_p=0.002, top_p=0.9),
    "temp_0": dict(temp=0.0, top_p=0.95),
    "top_p_0.5_min_keep_3000": dict(temp=0.9, top_p=0.5, min_keep=3000),
    "top_k_20000_two_bands": dict(temp=0.7, top_k=20000),
    "top_p_0.9999_many_bands": dict(temp=0.7, top_p=0.9999),
}


@pytest.mark.parametrize("name", list(DIST_CASES))
def test_distribution_headline_rows(ctx, name):
    print(f"case dist {name}", flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    logits = spiked(rng, (3, V27))
    check_dist(ctx, logits, cpvo.SamplerParams(**DIST_CASES[name]))


@pytest.mark.parametrize("rows", [60, 140])
def test_distribution_top_p_row_counts(ctx, rows):
    # top-p builds: the maximum and exponentials over many workgroups per
    # row, then the index-order sum and the first band side by side when two
    # workgroups per row fit the 256 CUs (60 rows), else one per row (140)
    print(f"case dist top-p rows={rows}", flush=True)
    rng = np.random.default_rng(rows)
    logits = spiked(rng, (rows, 8192))
    check_dist(ctx, logits, cpvo.SamplerParams(temp=0.7, top_p=0.95))


def test_distribution_penalties_with_history(ctx):
    print("case dist penalties", flush=True)
    rng = np.random.default_rng(7)
    logits = spiked(rng, (4, V27))
    hist = rng.integers(0, 300, size=(4, 200)).astype(np.int32)   # repeats inside the window
    hist[:, ::7] = -1                                              # empty slots are skipped
    hist[1, :] = -1
    hist[2, 5] = V27 + 3                                           # out-of-vocabulary ids are ignored
    for p in [cpvo.SamplerParams(temp=0.7, top_p=0.95, penalty_repeat=1.3, penalty_freq=0.1,
                                 penalty_present=0.2, penalty_last_n=64),
              cpvo.SamplerParams(temp=1.0, top_k=30, penalty_repeat=0.7, penalty_last_n=150),
              cpvo.SamplerParams(temp=0.0, penalty_repeat=2.0, penalty_last_n=64)]:
        check_dist(ctx, logits, p, hist)


def test_distribution_equal_logits_order_by_id(ctx):
    # every key ties on the logit: the band selection descends into the id
    # bits and the candidate order is the id order
    print("case dist equal logits", flush=True)
    logits = np.zeros((2, 40000), dtype=np.float32)
    logits[1, ::3] = -np.inf
    for p in [cpvo.SamplerParams(temp=1.0, top_p=0.5), cpvo.SamplerParams(temp=0.5, top_k=17000),
              cpvo.SamplerParams(temp=2.0, min_p=0.5)]:
        check_dist(ctx, logits, p)


def test_distribution_top_p_band_parts_and_fallback(ctx):
    # the split top-p build sorts its first band in parts of whole histogram
    # bins (a part spans at most 2048 keys plus its last bin, and may hold
    # 4096); tied logits share a bin: row 0 ties 5000 top logits, more than a
    # part may hold, so its band is sorted in one workgroup; row 1 ties 1500
    print("case dist band parts", flush=True)
    rng = np.random.default_rng(5)
    logits = rng.normal(0, 1, size=(3, V27)).astype(np.float32)
    logits[0, rng.choice(V27, 5000, replace=False)] = 5.0
    logits[1, rng.choice(V27, 1500, replace=False)] = 5.0
    for p in [cpvo.SamplerParams(temp=0.7, top_p=0.95), cpvo.SamplerParams(temp=1.0, top_p=0.3)]:
        check_dist(ctx, logits, p)


def short_exp_logits():
    """Logits l <= 0 whose expf is a float with at most 3 significant bits,
    from 1 down to 2^-40: their sums round on exact ties all the time."""
    out = []
    for j in range(41):
        for m in (1.0, 1.25, 1.5, 1.75):
            t = np.float32(m * 2.0 ** -j)
            if t > 1:
                continue
            x0 = np.float32(np.log(np.float64(t)))
            cand = [x0]
            up = dn = x0
            for _ in range(300):
                up = np.nextafter(up, np.float32(1))
                dn = np.nextafter(dn, np.float32(-1e9))
                cand += [up, dn]
            cand = np.array([c for c in cand if c <= 0], dtype=np.float32)
            hit = cand[cpvo.expf(cand) == t]
            if hit.size:
                out.append(hit[0])
    return np.array(out, dtype=np.float32)


def count_ties(x):
    """Steps of the sequential f32 sum of x that round an exact halfway case."""
    s, ties = np.float32(0), 0
    for v in x.astype(np.float32):
        exact = np.float64(s) + np.float64(v)         # exact: both terms are short here
        r = np.float32(exact)
        if r != exact:
            lo = np.nextafter(r, np.float32(-np.inf)) if np.float64(r) > exact else r
            hi = np.nextafter(lo, np.float32(np.inf))
            ties += (np.float64(lo) + np.float64(hi)) / 2 == exact
        s = r
    return ties


def test_distribution_sums_with_rounding_ties(ctx):
    print("case dist ties", flush=True)
    pool = short_exp_logits()
    assert pool.size > 40
    rng = np.random.default_rng(11)
    logits = rng.choice(pool, size=(6, 20000)).astype(np.float32)
    logits[:, 0] = 0.0
    logits[3, 1:10000] = pool[np.argmin(pool)]         # a long run of tiny terms first
    assert count_ties(cpvo.expf(logits[0])) > 100       # the softmax sum really meets ties
    check_dist(ctx, logits, cpvo.SamplerParams(temp=1.0))
    check_dist(ctx, logits, cpvo.SamplerParams(temp=1.0, top_p=0.97))


@pytest.mark.parametrize("v", [1, 2, 7, 1000, 1025, 9000])
def test_distribution_small_vocabularies(ctx, v):
    print(f"case dist v={v}", flush=True)
    rng = np.random.default_rng(v)
    logits = spiked(rng, (3, v), sd=2.0, spike=3.0)
    for p in [cpvo.SamplerParams(temp=0.7, top_p=0.95), cpvo.SamplerParams(temp=0.7),
              cpvo.SamplerParams(temp=1.0, top_k=5), cpvo.SamplerParams(temp=1.0, min_p=0.1, top_p=0.8)]:
        check_dist(ctx, logits, p)


# ---------------------------------------------------------------- acceptance
def drafts_for(rng, pl, k, p_argmax=0.7):
    B = pl.shape[0]
    am = pl.argmax(axis=2)
    d = rng.integers(pl.shape[2], size=(B, k)).astype(np.int32)
    take = rng.random(size=(B, k)) < p_argmax
    d[take] = am[:, :k][take]
    return d


def accept(ctx, pl, draft, p, mode, seed=None, u=None, q=None, noise=None, hist=None, rnd=0):
    t = lambda a, dt=np.float32: None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=dt)).cuda()
    tok, n = ctx.spec_accept(t(pl), t(draft, np.int32), dev_params(p), mode, u=t(u), q_logits=t(q),
                             noise=t(noise), hist=t(hist, np.int32), philox_seed=seed or 0, philox_round=rnd)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), n.cpu().numpy()


def same(got, ref):
    gt, gn = got
    rt, rn = ref
    assert np.array_equal(gn, rn), (gn, rn)
    for b in range(gn.size):
        assert np.array_equal(gt[b, :gn[b] + 1], rt[b, :rn[b] + 1]), (b, gt[b], rt[b])


@pytest.mark.parametrize("B", [1, 4, 16])
def test_headline_acceptance(ctx, B):
    # target logits ~N(0,3) + a +8 spike, draft logits = target + N(0,1),
    # drafts sampled from the draft distribution; T = 0.7, top-p 0.95,
    # device Philox uniforms; rejection with the draft distribution, the
    # one-hot rule, and greedy argmax match
    print(f"case accept headline B={B}", flush=True)
    k = 4
    rng = np.random.default_rng(100 + B)
    pl = spiked(rng, (B, k + 1, V27))
    ql = (pl[:, :k] + rng.normal(0, 1, size=(B, k, V27))).astype(np.float32)
    p = cpvo.SamplerParams(temp=0.7, top_p=0.95)
    draft = np.array([[cpvo.Sampler(p).distribution(ql[b, j]).draw(np.float32(rng.random())) for j in range(k)]
                      for b in range(B)], dtype=np.int32)
    seed = 1234 + B
    u = cpvo.philox_uniforms(seed, B, k)
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, seed=seed, q=ql),
         cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u, q_logits=ql))
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, seed=seed),
         cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u))
    # a later round of the same request: the round in the counter's last word
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, seed=seed, rnd=37),
         cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=cpvo.philox_uniforms(seed, B, k, round=37)))
    g = cpvo.SamplerParams()
    same(accept(ctx, pl, draft, g, cpvo.ACCEPT_GREEDY), cpvo.spec_accept(pl, draft, g, cpvo.ACCEPT_GREEDY))


def test_reject_many_rounds_small_vocab(ctx):
    # many seeds: every accept count and both replacement paths occur
    print("case accept reject sweep", flush=True)
    k, B, V = 4, 16, 3000
    seen = set()
    for it in range(12):
        rng = np.random.default_rng(it)
        peaked = it % 3 == 0                  # near-certain drafts: whole windows are kept
        pl = spiked(rng, (B, k + 1, V), sd=1.5, spike=14.0 if peaked else 4.0)
        draft = drafts_for(rng, pl, k, 1.0 if peaked else 0.85)
        p = [cpvo.SamplerParams(temp=0.7, top_p=0.95), cpvo.SamplerParams(temp=1.0),
             cpvo.SamplerParams(temp=0.8, top_k=20), cpvo.SamplerParams(temp=1.0, min_p=0.05)][it % 4]
        u = rng.random(size=(B, k + 1, 2)).astype(np.float32)
        got = accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, u=u)
        ref = cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u)
        same(got, ref)
        seen.update(ref[1].tolist())
    assert seen == set(range(k + 1))


def test_reject_general_rule_with_draft_logits(ctx):
    print("case accept reject q", flush=True)
    k, B, V = 4, 8, 20000
    rng = np.random.default_rng(5)
    pl = spiked(rng, (B, k + 1, V), sd=2.0, spike=5.0)
    q = (pl[:, :k] + rng.normal(0, 1.0, size=(B, k, V))).astype(np.float32)
    draft = q.argmax(axis=2).astype(np.int32)
    for p in [cpvo.SamplerParams(temp=0.7, top_p=0.95), cpvo.SamplerParams(temp=1.0)]:
        for seed in range(3):
            u = cpvo.philox_uniforms(seed, B, k)
            got = accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, seed=seed, q=q)
            ref = cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u, q_logits=q)
            same(got, ref)


def test_reject_draws_deep_in_long_candidate_lists(ctx):
    # near-flat target logits keep ~144k candidates at top-p 0.95, so the
    # replacement draws' cumulative searches end anywhere from the first
    # elements to the last of 18 fold windows (replacement uniforms from
    # 0.001 to 0.999); random drafts are rejected, and with the draft
    # distribution about half the residual terms are 0
    print("case accept reject long lists", flush=True)
    k, B = 4, 4
    rng = np.random.default_rng(17)
    pl = rng.normal(0, 0.05, size=(B, k + 1, V27)).astype(np.float32)
    q = (pl[:, :k] + rng.normal(0, 0.05, size=(B, k, V27))).astype(np.float32)
    draft = rng.integers(0, V27, size=(B, k)).astype(np.int32)
    p = cpvo.SamplerParams(temp=0.7, top_p=0.95)
    u = rng.random(size=(B, k + 1, 2)).astype(np.float32)
    u[:, :, 1] = np.array([0.001, 0.3, 0.6, 0.999], dtype=np.float32)[:, None]
    for ql in (None, q):
        got = accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, u=u, q=ql)
        ref = cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u, q_logits=ql)
        same(got, ref)


def test_reject_penalty_window_grows_with_drafts(ctx):
    print("case accept reject penalties", flush=True)
    k, B, V = 4, 6, 5000
    rng = np.random.default_rng(9)
    pl = spiked(rng, (B, k + 1, V), sd=1.0, spike=3.0)
    draft = drafts_for(rng, pl, k, 0.9)
    hist = rng.integers(0, V, size=(B, 40)).astype(np.int32)
    hist[:, :5] = -1
    hist[0, 10:20] = draft[0, 0]
    p = cpvo.SamplerParams(temp=0.8, top_p=0.9, penalty_repeat=1.5, penalty_freq=0.3, penalty_present=0.1,
                           penalty_last_n=32)
    u = rng.random(size=(B, k + 1, 2)).astype(np.float32)
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, u=u, hist=hist),
         cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u, hist=hist))
    p0 = cpvo.SamplerParams(temp=0.0, penalty_repeat=3.0, penalty_last_n=8)
    same(accept(ctx, pl, draft, p0, cpvo.ACCEPT_REJECT, u=u, hist=hist),
         cpvo.spec_accept(pl, draft, p0, cpvo.ACCEPT_REJECT, u=u, hist=hist))


def test_greedy(ctx):
    print("case accept greedy", flush=True)
    k, B = 4, 16
    rng = np.random.default_rng(3)
    pl = spiked(rng, (B, k + 1, V27))
    draft = drafts_for(rng, pl, k, 0.8)
    p = cpvo.SamplerParams()
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_GREEDY), cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_GREEDY))


def gumbel_noise(rng, shape, T):
    u = rng.random(size=shape).astype(np.float32)
    return (-np.log(-np.log(np.maximum(u, 1e-12)))).astype(np.float32) * np.float32(T)


@pytest.mark.parametrize("filtered", [False, True])
def test_gumbel(ctx, filtered):
    print(f"case accept gumbel filtered={filtered}", flush=True)
    k, B, V = 4, 8, 30000
    rng = np.random.default_rng(21)
    pl = spiked(rng, (B, k + 1, V), sd=2.0, spike=4.0)
    T = 0.7
    noise = gumbel_noise(rng, (B, k + 1, V), T)
    am = (pl + noise).argmax(axis=2)
    draft = am[:, :k].astype(np.int32).copy()
    flip = rng.random(size=(B, k)) < 0.25
    draft[flip] = (draft[flip] + 1) % V
    p = cpvo.SamplerParams(temp=T, top_p=0.9, top_k=0) if filtered else cpvo.SamplerParams(temp=T)
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_GUMBEL, noise=noise),
         cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_GUMBEL, noise_t=noise))


def test_k_zero_draws_the_bonus_token(ctx):
    print("case accept k=0", flush=True)
    rng = np.random.default_rng(4)
    pl = spiked(rng, (3, 1, 4000))
    draft = np.zeros((3, 0), dtype=np.int32)
    p = cpvo.SamplerParams(temp=0.7, top_p=0.95)
    u = rng.random(size=(3, 1, 2)).astype(np.float32)
    same(accept(ctx, pl, draft, p, cpvo.ACCEPT_REJECT, u=u), cpvo.spec_accept(pl, draft, p, cpvo.ACCEPT_REJECT, u=u))


def test_bad_arguments_are_refused(ctx):
    from codpiece_amd.runtime import CpvError
    pl = torch.zeros((1, 2, 10), device="cuda")
    d = torch.zeros((1, 1), dtype=torch.int32, device="cuda")
    with pytest.raises(CpvError):
        ctx.spec_accept(pl, d, dev_params(cpvo.SamplerParams(temp=1.0, min_p=1.5)), cpvo.ACCEPT_REJECT)
    with pytest.raises(CpvError):
        ctx.spec_accept(pl, d, dev_params(cpvo.SamplerParams(temp=1.0)), cpvo.ACCEPT_GUMBEL)
    with pytest.raises(CpvError):
        ctx.spec_accept(pl, d, dev_params(cpvo.SamplerParams(temp=1.0, top_k=-1)), cpvo.ACCEPT_REJECT)
