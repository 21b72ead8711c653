"""GPU parity on randomly drawn shapes: attention over the API's f16 caches,
the quantized GEMM, the target distributions and speculative acceptance,
against the oracle.

Bar: bit-exact, as everywhere else.  The fixed-shape tests pin the model's
shapes and the kernels' thresholds one by one; these draw the shapes the
kernels' dispatch has to get right together, each case from its own seed:
- attention: head dim 64 or 128; 1-8 KV heads; 1, 2, 4, 5 or 8 query heads
  per KV head; 1-64 query rows as a chain or a random tree; contexts near
  the 128-row chunk edges, short, or up to 20000 rows; V strides with slack;
  value scales from 1e-3 to 3000 (the top value limb); all-zero K rows and
  query rows;
- GEMM: Q8_0, Q4_K and Q6_K; K up to 6144 (multiples of the block, so Q8_0
  also takes partial 256-element units); N from 1 to 5120; M at the
  kernels' row thresholds (8/9, 16/17, 32/33, 48/49, 64/65, ...) or anywhere
  up to 256; activation scales 1e-3 to 50; zero weight and activation rows;
- sampler: vocabularies of 1 to 262144 ids; 1-8 rows or 40-140 short ones;
  logits of spread 0.05-10, with spikes, ties and masked (-inf) ids; every
  filter (temperature 0-1.5, top-k past V, top-p, min-p, min_keep 0 to
  5000) and the penalties over a history with empty slots; acceptance for
  1-16 sequences of 0-8 drafts by argmax match, rejection (the one-hot rule
  and the draft distribution, uniforms given or from Philox) and gumbel;
- whole rounds on random small models: 1-3 layers, d_model 256-5120, head
  dim 64 or 128, 1-20 query heads over 1-4 KV heads, FFN 256-3072, Q8_0 or
  Q4_K linears with a Q8_0, Q4_K or Q6_K head, with or without the MTP
  layer; prompts prefilled in random chunks, then three rounds of 1-16 rows
  at depth 0-4, each rewound to a random accepted prefix; random draft
  trees of 1-64 nodes on such models, every leaf's path against the
  oracle's chain of it, then a committed branch and the round after it.
"""
import numpy as np
import pytest
import torch

from oracle import cpvo

import model_fixtures as mf

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from codpiece_amd.runtime import Context
    c = Context(0)
    yield c
    c.close()


def f16(a):
    return cpvo.f32_to_f16_bits(a.astype(np.float32))


@pytest.mark.parametrize("seed", range(40))
def test_attention_random_shape(ctx, seed):
    rng = np.random.default_rng(7000 + seed)
    d = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    h = hkv * int(rng.choice([1, 2, 4, 5, 8]))
    t = int(rng.integers(1, 17)) if rng.random() < 0.7 else int(rng.integers(17, 65))
    r = rng.random()
    if r < 0.3:
        n_past = int(rng.integers(0, 600))
    elif r < 0.6:
        n_past = int(128 * rng.integers(1, 80) - rng.integers(0, 3) * t + rng.integers(-2, 3))
    else:
        n_past = int(rng.integers(600, 20000))
    n_past = max(0, n_past)
    parent = [-1] + [int(rng.integers(-1, j)) for j in range(1, t)] if rng.random() < 0.5 else None
    n_ctx = n_past + t
    vs = (n_ctx + 7) // 8 * 8 + int(rng.choice([0, 8, 64]))
    ks, vsc = float(rng.choice([1.0, 1e-3, 30.0])), float(rng.choice([1.0, 1e-3, 100.0]))
    k = f16(rng.normal(size=(n_ctx, hkv * d)) * ks)
    v = rng.normal(size=(n_ctx, hkv * d)) * vsc
    if rng.random() < 0.3:
        big = (rng.random(n_ctx) < 0.05)[:, None] & (rng.random(hkv * d) < 0.3)[None, :]
        v = np.where(big, rng.normal(size=v.shape) * 3000, v)
    v = f16(v)
    if rng.random() < 0.3:
        hh = int(rng.integers(0, hkv))
        k[rng.random(n_ctx) < 0.1, hh * d:(hh + 1) * d] = 0
    vt = np.zeros((hkv * d, vs), dtype=np.uint16)
    vt[:, :n_ctx] = v.T
    q = rng.normal(size=(t, h, d)).astype(np.float32)
    if rng.random() < 0.2:
        q[int(rng.integers(0, t)), int(rng.integers(0, h))] = 0
    scale = np.float32(1) / np.sqrt(np.float32(d))
    print(f"case t={t} h={h} hkv={hkv} d={d} n_past={n_past} v_stride={vs} tree={parent is not None}", flush=True)
    par = None if parent is None else torch.tensor(parent, dtype=torch.int32, device="cuda")
    got = ctx.attn(torch.from_numpy(q).cuda(), torch.from_numpy(k.view(np.int16)).cuda(),
                   torch.from_numpy(vt.view(np.int16)).cuda(), n_past, par, hkv, float(scale)).cpu().numpy()
    ref = cpvo.attn(q, k, v, n_past, parent, scale)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), np.count_nonzero(got != ref)


EDGE_M = [1, 2, 4, 5, 8, 9, 12, 16, 17, 24, 31, 32, 33, 47, 48, 49, 63, 64, 65, 100, 128, 129, 200, 255, 256]


@pytest.mark.parametrize("seed", range(60))
def test_qgemm_random_shape(ctx, seed):
    rng = np.random.default_rng(9000 + seed)
    ty = (cpvo.Q8_0, cpvo.Q4_K, cpvo.Q6_K)[seed % 3]
    blk = 32 if ty == cpvo.Q8_0 else 256
    k = blk * int(rng.integers(1, 6144 // blk + 1))
    n = int(rng.integers(1, 3000)) if rng.random() < 0.7 else int(rng.choice([64, 128, 4096, 5120]))
    m = int(rng.choice(EDGE_M)) if rng.random() < 0.6 else int(rng.integers(1, 257))
    while m * n * k > 4e8 and n > 64:      # (keeps the oracle's side to a second or so)
        n //= 2
    wf = rng.normal(0, 0.02, size=(n, k)).astype(np.float32)
    if rng.random() < 0.2:
        wf[int(rng.integers(0, n))] = 0
    wq = cpvo.quantize(ty, wf)
    x = (rng.normal(0, 1, size=(m, k)) * float(rng.choice([1.0, 1e-3, 50.0]))).astype(np.float32)
    if rng.random() < 0.3:
        x[int(rng.integers(0, m))] = 0
    print(f"case type={ty} n={n} k={k} m={m}", flush=True)
    w = ctx.upload_weight(ty, wq, n, k)
    y = ctx.qgemm(w, torch.from_numpy(x).cuda()).cpu().numpy()
    w.free()
    ref = cpvo.qgemm(ty, wq, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()


def dev_params(p):
    from codpiece_amd.runtime import SamplerParams
    return SamplerParams(p.temp, p.top_k, p.top_p, p.min_p, p.min_keep, p.penalty_repeat, p.penalty_freq,
                         p.penalty_present, p.penalty_last_n)


def rand_v(rng):
    r = rng.random()
    if r < 0.2:
        return int(rng.integers(1, 64))
    if r < 0.5:
        return int(rng.integers(64, 20000))
    if r < 0.8:
        return 151936
    return int(rng.integers(20000, 262145))


def rand_logits(rng, shape):
    x = rng.normal(0, float(rng.choice([0.05, 1.0, 3.0, 10.0])), size=shape).astype(np.float32)
    flat = x.reshape(-1, shape[-1])
    if rng.random() < 0.5:
        for r in range(flat.shape[0]):
            flat[r, rng.integers(shape[-1])] += np.float32(rng.choice([3.0, 8.0, 20.0]))
    if rng.random() < 0.25:                    # ties
        x = (np.round(x * 2) / 2).astype(np.float32)
    if rng.random() < 0.15:                    # masked ids (id 0 stays)
        x[rng.random(size=shape) < 0.3] = -np.inf
        x.reshape(-1, shape[-1])[:, 0] = 0.0
    return np.ascontiguousarray(x)


def rand_params(rng, V, penalties=True):
    pen = penalties and rng.random() < 0.3
    return cpvo.SamplerParams(
        temp=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])),
        top_k=0 if rng.random() < 0.5 else int(rng.integers(1, V + 6)),
        top_p=1.0 if rng.random() < 0.3 else float(rng.uniform(0.05, 1.0)),
        min_p=0.0 if rng.random() < 0.6 else float(rng.uniform(0.0, 0.3)),
        min_keep=int(rng.choice([1, 0, int(rng.integers(1, 5000))])),
        penalty_repeat=float(rng.choice([0.7, 1.3])) if pen else 1.0,
        penalty_freq=float(rng.uniform(0, 0.5)) if pen else 0.0,
        penalty_present=float(rng.uniform(0, 0.5)) if pen else 0.0,
        penalty_last_n=int(rng.integers(0, 200)) if pen else 64)


def rand_hist(rng, rows, V):
    h = rng.integers(0, min(V, 500), size=(rows, int(rng.integers(1, 300)))).astype(np.int32)
    h[rng.random(size=h.shape) < 0.1] = -1     # empty slots
    return h


def dev(a, dt=np.float32):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=dt)).cuda()


@pytest.mark.parametrize("seed", range(30))
def test_distribution_random(ctx, seed):
    rng = np.random.default_rng(11000 + seed)
    V = rand_v(rng)
    rows = int(rng.integers(1, 9)) if rng.random() < 0.85 else int(rng.integers(40, 141))
    if rows > 20 and V > 20000:
        V = 8192
    logits = rand_logits(rng, (rows, V))
    p = rand_params(rng, V)
    hist = rand_hist(rng, rows, V) if p.penalty_repeat != 1.0 else None
    print(f"case rows={rows} V={V} temp={p.temp} top_k={p.top_k} top_p={p.top_p:.3f} min_p={p.min_p:.3f} "
          f"min_keep={p.min_keep} penalties={hist is not None}", flush=True)
    ids, probs, n = ctx.distribution(dev(logits), dev_params(p), dev(hist, np.int32))
    ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
    for r in range(rows):
        hr = None if hist is None else ([x for x in hist[r] if x >= 0][-p.penalty_last_n:] if p.penalty_last_n else [])
        rid, rp, _ = cpvo.distribution(p, logits[r], hr)
        assert n[r] == rid.size, (r, n[r], rid.size)
        assert np.array_equal(ids[r, :n[r]], rid), r
        assert np.array_equal(probs[r, :n[r]].view(np.uint32), rp.view(np.uint32)), r


@pytest.mark.parametrize("seed", range(30))
def test_acceptance_random(ctx, seed):
    rng = np.random.default_rng(12000 + seed)
    V, B, k = rand_v(rng), int(rng.integers(1, 17)), int(rng.integers(0, 9))
    if B * (k + 1) * V > 4e7:
        V = max(1, int(4e7 // (B * (k + 1))))
    pl = rand_logits(rng, (B, k + 1, V))
    mode = (cpvo.ACCEPT_GREEDY, cpvo.ACCEPT_REJECT, cpvo.ACCEPT_REJECT, cpvo.ACCEPT_GUMBEL)[seed % 4]
    p = rand_params(rng, V, penalties=mode == cpvo.ACCEPT_REJECT)
    if mode == cpvo.ACCEPT_GUMBEL and p.temp == 0.0:
        p.temp = 0.7
    draft = rng.integers(0, V, size=(B, k)).astype(np.int32)
    take = rng.random(size=(B, k)) < 0.7
    draft[take] = pl.argmax(axis=2)[:, :k][take]
    q = None
    if mode == cpvo.ACCEPT_REJECT and rng.random() < 0.5:
        q = (pl[:, :k] + rng.normal(0, 1, size=(B, k, V))).astype(np.float32)
    noise = None
    if mode == cpvo.ACCEPT_GUMBEL:
        g = rng.random(size=(B, k + 1, V)).astype(np.float32)
        noise = (-np.log(-np.log(np.maximum(g, 1e-12)))).astype(np.float32) * np.float32(p.temp)
    hist = rand_hist(rng, B, V) if (mode == cpvo.ACCEPT_REJECT and p.penalty_repeat != 1.0) else None
    philox = rng.random() < 0.5
    ps, pr = int(rng.integers(0, 1 << 30)), int(rng.integers(0, 1000))
    u = cpvo.philox_uniforms(ps, B, k, round=pr) if philox else rng.random(size=(B, k + 1, 2)).astype(np.float32)
    print(f"case B={B} k={k} V={V} mode={mode} temp={p.temp} top_k={p.top_k} top_p={p.top_p:.3f} "
          f"min_p={p.min_p:.3f} q={q is not None} penalties={hist is not None} philox={philox}", flush=True)
    tok, n = ctx.spec_accept(dev(pl), dev(draft, np.int32), dev_params(p), mode, u=None if philox else dev(u),
                             q_logits=dev(q), noise=dev(noise), hist=dev(hist, np.int32),
                             philox_seed=ps if philox else 0, philox_round=pr if philox else 0)
    tok, n = tok.cpu().numpy(), n.cpu().numpy()
    rt, rn = cpvo.spec_accept(pl, draft, p, mode, u=u if mode == cpvo.ACCEPT_REJECT else None, q_logits=q,
                              noise_t=noise, hist=hist)
    assert np.array_equal(n, rn), (n, rn)
    for b in range(B):
        assert np.array_equal(tok[b, :n[b] + 1], rt[b, :rn[b] + 1]), (b, tok[b], rt[b])


def random_models(ctx, rng, qt):
    """A random small layout with its weights: (device model, oracle model, hparams)."""
    from codpiece_amd.model import Model, make_hparams
    while True:
        hd, hkv = int(rng.choice([64, 128])), int(rng.choice([1, 2, 4]))
        H = hkv * int(rng.choice([1, 2, 4, 5]))
        if qt == cpvo.Q8_0 or (H * hd) % 256 == 0:    # (wo's K is H * hd)
            break
    E, F = 256 * int(rng.choice([1, 2, 3, 4, 6, 8, 20])), 256 * int(rng.integers(1, 13))
    while E * F > 5120 * 1536:
        F = max(256, F // 512 * 256)
    hp = dict(mf.TINY, n_layer=int(rng.integers(1, 4)), n_embd=E, n_head=H, n_head_kv=hkv, head_dim=hd, n_rot=hd,
              rope_sections=[11, 11, 10, 0] if hd == 64 else [22, 22, 20, 0], n_ff=F,
              n_vocab=int(rng.integers(300, 6000)), has_mtp=int(rng.random() < 0.8))
    ht = (cpvo.Q8_0, cpvo.Q4_K, cpvo.Q6_K)[int(rng.integers(0, 3))]
    print(f"case {hp} linears={qt} head={ht}", flush=True)
    tensors = mf.make_tensors(hp, seed=int(rng.integers(0, 1 << 20)), qtype=qt, head_type=ht)
    gm = Model(ctx, make_hparams(**hp))
    mf.load_into(gm, tensors)
    gm.ready()
    om = cpvo.Model(hp)
    mf.load_into(om, tensors)
    return gm, om, hp


@pytest.mark.parametrize("seed", range(8))
def test_rounds_on_random_models(ctx, seed):
    from codpiece_amd.model import Session
    rng = np.random.default_rng(13000 + seed)
    gm, om, hp = random_models(ctx, rng, (cpvo.Q8_0, cpvo.Q4_K)[seed % 2])
    g, o = Session(gm, 1024, max_batch=256), cpvo.Session(om, 1024)
    try:
        n_prompt = int(rng.integers(1, 400))
        prompt = rng.integers(0, hp["n_vocab"], size=n_prompt + 64).tolist()
        c = 0
        while c < n_prompt:
            step = min(n_prompt - c, int(rng.choice([1, 5, 17, 64, 256])))
            g.prefill(prompt[c:c + step])
            o.prefill(prompt[c:c + step])
            c += step
        for _ in range(3):
            T = int(rng.integers(1, 17))
            depth = int(rng.integers(0, 5)) if hp["has_mtp"] else 0
            print(f"round n_past={g.pos[0]} T={T} depth={depth}", flush=True)
            a = g.step_fused_cached(prompt[c:c + T], depth, want_logits=True)
            b = o.step_fused_cached(prompt[c:c + T], depth, want_logits=True)
            assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
            assert np.array_equal(a.hidden.cpu().numpy().view(np.uint32), b[4].view(np.uint32))
            assert a.preds == b[0].tolist() and a.chain == b[1].tolist()
            # keep a random accepted prefix; a round without drafts writes no
            # MTP rows, so only a drafting round moves the MTP position
            keep = int(rng.integers(1, T + 1))
            n_past, mtp_past = g.pos
            m2 = mtp_past + keep if depth > 0 else mtp_past
            g.set_pos(n_past - T + keep, m2)
            o.set_pos(n_past - T + keep, m2)
            c += keep
    finally:
        g.free()
        o.free()
        gm.free()
        om.free()


def path_to(parent, v):
    p = []
    while v >= 0:
        p.append(v)
        v = parent[v]
    return p[::-1]


@pytest.mark.parametrize("seed", range(6))
def test_random_trees_on_random_models(ctx, seed):
    # every leaf's root-to-node path of a random tree (1-64 nodes) equals the
    # oracle's chain verify of that path from the same context; then a random
    # node's path is committed and the next round equals the one after the
    # oracle's chain of that path
    from codpiece_amd.model import Session
    rng = np.random.default_rng(14000 + seed)
    gm, om, hp = random_models(ctx, rng, (cpvo.Q8_0, cpvo.Q4_K)[seed % 2])
    V = hp["n_vocab"]
    t = int(rng.integers(1, 65))
    parent = [-1] + [int(rng.integers(-1, j)) for j in range(1, t)]
    n_prompt = int(rng.integers(1, 300))
    prompt = rng.integers(0, V, size=n_prompt).tolist()
    toks = rng.integers(0, V, size=t).tolist()
    g, o = Session(gm, 1024, max_batch=256), cpvo.Session(om, 1024)
    try:
        g.prefill(prompt)
        o.prefill(prompt)
        print(f"tree of {t} after {n_prompt}", flush=True)
        a = g.verify_tree(toks, parent, want_logits=True)
        la, ha = a.logits.cpu().numpy(), a.hidden.cpu().numpy()
        for leaf in [v for v in range(t) if v not in parent]:
            path = path_to(parent, leaf)
            o.set_pos(n_prompt, 0)
            b = o.step_fused_cached([toks[v] for v in path], 0, want_logits=True)
            assert np.array_equal(la[path].view(np.uint32), b[3].view(np.uint32)), ("logits", path)
            assert np.array_equal(ha[path].view(np.uint32), b[4].view(np.uint32)), ("hidden", path)
            assert [a.preds[v] for v in path] == b[0].tolist()
        path = path_to(parent, int(rng.integers(0, t)))
        g.commit_branch(path)
        o.set_pos(n_prompt, 0)
        o.step_fused_cached([toks[v] for v in path], 0)
        assert g.pos[0] == o.pos[0] == n_prompt + len(path)
        nxt = rng.integers(0, V, size=int(rng.integers(1, 9))).tolist()
        a = g.step_fused_cached(nxt, 0, want_logits=True)
        b = o.step_fused_cached(nxt, 0, want_logits=True)
        assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
        assert a.preds == b[0].tolist()
    finally:
        g.free()
        o.free()
        gm.free()
        om.free()
