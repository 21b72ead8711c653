"""The 27B-class model at its workload on the device (config 5).

64 layers, d_model 5120, 40/8 heads x 128, FFN 17408, vocabulary 151,936,
Q4_K linears with a Q6_K embedding and head, one MTP layer, built on the
device as bench.py builds it; a 4096-token random prompt prefilled into a
32,768-row context.  The whole model is too large for the oracle to run, so
the round is held to properties the exact contracts fix, and its head and its
acceptance to the oracle on the round's own data:
  (a) a 5-row verify equals five 1-row verifies bit for bit (logits, hidden,
      preds, draft chain and confidence): every row depends only on its own
      token and the rows before it;
  (b) rewinding and verifying again reproduces the round bit for bit;
  (c) a 16-node draft tree with linear parents equals the 16-token chain;
  (d) the round's logits equal the oracle's Q6_K GEMM of the device's hidden
      rows with the head's bytes, bit for bit, and the preds are their first
      argmax;
  (e) the T = 0.7 / top-p 0.95 leg: cpv_spec_accept on the round's logits
      equals the oracle's acceptance on the same logits and uniforms, in the
      rejection and gumbel modes;
  (f) the sampled loop runs rounds of that leg on the device, each committing
      its accepted drafts and one token.
"""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import cpvo

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402  (the workload's model definition and synthetic weights)

HP = dict(bench.HP)
V, E = HP["n_vocab"], HP["n_embd"]
PROMPT = 4096


@pytest.fixture(scope="module")
def big():
    from codpiece_amd.model import Model, Session, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    print("building the 27B-class model on the device", flush=True)
    m = Model(ctx, make_hparams(**HP))
    gen = torch.Generator(device=ctx.torch_device)
    gen.manual_seed(5)
    head = None
    for name, t, ne0, ne1 in bench.tensor_specs(HP):
        if t == bench.F32:
            data = torch.ones(ne0, dtype=torch.float32, device=ctx.torch_device)
        else:
            data = bench.synth_quant(torch, t, ne1, ne0, gen, ctx.torch_device)
            if name == "output.weight":
                head = data.cpu().numpy()
        m.set_tensor(name, t, data, ne0, ne1)
        del data
    m.ready()
    s = Session(m, 32768, max_batch=512)
    prompt = np.random.default_rng(9).integers(0, V, size=PROMPT).tolist()
    print("prefilling 4096 tokens", flush=True)
    for c in range(0, PROMPT, 512):
        s.prefill(prompt[c:c + 512])
    s.set_pos(PROMPT, 0)
    torch.cuda.synchronize()
    yield ctx, m, s, head
    s.free()
    m.free()
    ctx.close()


def _round(s, toks, depth=4):
    o = s.step_fused_cached(toks, depth, want_logits=True)
    return (o.preds, o.chain, o.conf, o.logits.cpu().numpy(), o.hidden.cpu().numpy())


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


TOKS5 = np.random.default_rng(10).integers(0, V, size=5).tolist()


def test_five_row_verify_equals_five_single_steps(big):
    _, _, s, _ = big
    p0 = s.pos
    print("case 5-row round", flush=True)
    P, C, CF, L, H = _round(s, TOKS5)
    s.set_pos(*p0)
    for i, tok in enumerate(TOKS5):
        print(f"case single step {i}", flush=True)
        n_past, mtp_past = s.pos
        p, c, cf, l, h = _round(s, [tok])
        assert _eq(l[0], L[i]) and _eq(h[0], H[i]), i
        assert p[0] == P[i]
        assert [x[0] for x in c] == [x[i] for x in C]
        assert _eq([x[0] for x in cf], [x[i] for x in CF])
        s.set_pos(n_past + 1, mtp_past + 1)
    s.set_pos(*p0)


def test_rewind_and_redo_is_identical(big):
    _, _, s, _ = big
    p0 = s.pos
    a = _round(s, TOKS5)
    assert s.pos == (p0[0] + 5, p0[1])
    s.set_pos(*p0)
    b = _round(s, TOKS5)
    assert a[0] == b[0] and a[1] == b[1] and _eq(a[2], b[2]) and _eq(a[3], b[3]) and _eq(a[4], b[4])
    s.set_pos(*p0)


def test_linear_tree_equals_the_chain(big):
    _, _, s, _ = big
    p0 = s.pos
    toks = np.random.default_rng(12).integers(0, V, size=16).tolist()
    chain = s.step_fused_cached(toks, 0, want_logits=True)
    s.set_pos(*p0)
    tree = s.verify_tree(toks, [-1] + list(range(15)), want_logits=True)
    assert tree.preds == chain.preds
    assert _eq(tree.logits.cpu().numpy(), chain.logits.cpu().numpy())
    assert _eq(tree.hidden.cpu().numpy(), chain.hidden.cpu().numpy())
    s.set_pos(*p0)


def test_head_logits_equal_the_oracle_gemm(big):
    _, _, s, head = big
    p0 = s.pos
    P, _, _, L, H = _round(s, TOKS5)
    s.set_pos(*p0)
    print("case oracle Q6_K head over 5 rows", flush=True)
    ref = cpvo.qgemm(cpvo.Q6_K, head, H, threads=16)
    assert _eq(L, ref)
    assert P == [int(np.argmax(r)) for r in ref]


def _uniform_noise(seed, temp, rows):
    u = np.random.default_rng(seed).random((rows, V), dtype=np.float32)
    u = np.maximum(u, np.float32(1e-12))
    return (-np.log(-np.log(u)) * np.float32(temp)).astype(np.float32)


@pytest.mark.parametrize("mode,top_p", [(cpvo.ACCEPT_REJECT, 0.95), (cpvo.ACCEPT_GUMBEL, 0.95),
                                        (cpvo.ACCEPT_GUMBEL, 1.0)])
def test_sampled_leg_acceptance_equals_the_oracle(big, mode, top_p):
    from codpiece_amd.runtime import SamplerParams
    ctx, _, s, _ = big
    p0 = s.pos
    nz = _uniform_noise(31, 0.7, 5) if mode == cpvo.ACCEPT_GUMBEL else None
    o = s.step_fused_cached(TOKS5, 4, want_logits=True,
                            noise=None if nz is None else torch.from_numpy(nz).cuda())
    s.set_pos(*p0)
    L = o.logits.cpu().numpy()
    # drafts: the round's own tokens after the first, and then its own preds
    # (so that some are accepted)
    for drafts in (TOKS5[1:], o.preds[:4]):
        print(f"case mode={mode} top_p={top_p} drafts={drafts}", flush=True)
        for seed in range(4):
            dr = torch.tensor([drafts], dtype=torch.int32, device="cuda")
            tok, n = ctx.spec_accept(o.logits.view(1, 5, V), dr, SamplerParams(temp=0.7, top_p=top_p), mode,
                                     noise=None if nz is None else torch.from_numpy(nz).cuda().view(1, 5, V),
                                     philox_seed=seed)
            otok, on = cpvo.spec_accept(L.reshape(1, 5, V), np.array([drafts], np.int32),
                                        cpvo.SamplerParams(temp=0.7, top_p=top_p), mode,
                                        u=cpvo.philox_uniforms(seed, 1, 4),
                                        noise_t=None if nz is None else nz.reshape(1, 5, V))
            n = int(n.cpu()[0])
            assert n == int(on[0])
            assert tok.cpu().numpy()[0, :n + 1].tolist() == otok[0, :n + 1].tolist()


def test_sampled_loop_runs_at_the_workload(big):
    from codpiece_amd.model import sampled_generate
    from codpiece_amd.runtime import SamplerParams
    ctx, m, _, _ = big
    from codpiece_amd.model import Session
    s = Session(m, 32768, max_batch=512)
    prompt = np.random.default_rng(9).integers(0, V, size=PROMPT).tolist()
    print("case sampled loop at T=0.7 top-p 0.95", flush=True)
    toks, st = sampled_generate(s, prompt, 12, 4, SamplerParams(temp=0.7, top_p=0.95), cpvo.ACCEPT_REJECT,
                                seed=3, tail=64, bulk=512)
    assert len(toks) == 12 and all(0 <= t < V for t in toks)
    assert st.rounds >= 1 and st.accepted <= st.proposed
    n_past, _ = s.pos
    # every committed token but the last is in the cache (a last round that
    # ends inside its accepted drafts is not rewound)
    assert PROMPT + len(toks) - 1 <= n_past <= PROMPT + len(toks) - 1 + 4
    s.free()
