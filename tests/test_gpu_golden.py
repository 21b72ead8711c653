"""The device path against the committed golden fixtures (bit-exact).

Same files as tests/test_golden.py, which pins them to the oracle on the CPU;
here each fixture's inputs go through the C ABI on cuda:0.
"""
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as mg  # noqa: E402
import model_fixtures as mf  # noqa: E402

from oracle import cpvo  # noqa: E402

pytestmark = pytest.mark.gpu


def load(name):
    return np.load(os.path.join(HERE, "golden", f"{name}.npz"))


@pytest.fixture(scope="module")
def ctx():
    from codpiece_amd.runtime import Context
    c = Context(0)
    yield c
    c.close()


def dev(a, dt=None):
    return torch.from_numpy(np.ascontiguousarray(a if dt is None else a.astype(dt))).cuda()


def dparams(p):
    from codpiece_amd.runtime import SamplerParams
    return SamplerParams(p.temp, p.top_k, p.top_p, p.min_p, p.min_keep, p.penalty_repeat, p.penalty_freq,
                         p.penalty_present, p.penalty_last_n)


@pytest.mark.parametrize("q", ["q4_k", "q6_k", "q8_0"])
def test_qgemm_fixture(ctx, q):
    f = load("qgemm")
    t, n, k = f[f"{q}_shape"].tolist()
    print(f"case golden qgemm {q} n={n} k={k}", flush=True)
    w = ctx.upload_weight(t, f[f"{q}_w"], n, k)
    y = ctx.qgemm(w, dev(f[f"{q}_x"])).cpu().numpy()
    w.free()
    assert np.array_equal(y.view(np.uint32), f[f"{q}_y"].view(np.uint32))


def test_attn_fixture(ctx):
    f = load("attn")
    n_past, t, h, hkv, d = f["dims"].tolist()
    print("case golden attn tree16", flush=True)
    vs = (n_past + t + 7) // 8 * 8
    vt = np.zeros((hkv * d, vs), dtype=np.uint16)
    vt[:, :n_past + t] = f["v"].T
    out = ctx.attn(dev(f["q"]), dev(f["k"].view(np.int16)), dev(vt.view(np.int16)), n_past,
                   dev(f["parent"]), hkv, float(f["scale"][0])).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), f["out"].view(np.uint32))


def test_sampler_fixture(ctx):
    f = load("sampler")
    print("case golden distributions", flush=True)
    for si, row in enumerate(mg.SAMPLER_SETTINGS):
        p = mg.params(row)
        ids, probs, n = ctx.distribution(dev(f["logits"]), dparams(p), dev(f["hist"]))
        ids, probs, n = ids.cpu().numpy(), probs.cpu().numpy(), n.cpu().numpy()
        assert np.array_equal(n, f[f"s{si}_n"]), si
        for r in range(n.size):
            assert np.array_equal(ids[r, :n[r]], f[f"s{si}_ids"][r, :n[r]]), (si, r)
            assert np.array_equal(probs[r, :n[r]].view(np.uint32), f[f"s{si}_probs"][r, :n[r]].view(np.uint32))


def test_accept_fixture(ctx):
    f = load("accept")
    print("case golden acceptance", flush=True)
    pr = mg.params(mg.SAMPLER_SETTINGS[0])
    cases = {
        "greedy": (cpvo.SamplerParams(), cpvo.ACCEPT_GREEDY, {}),
        "reject": (pr, cpvo.ACCEPT_REJECT, dict(u=dev(f["u"]))),
        "reject_q": (pr, cpvo.ACCEPT_REJECT, dict(u=dev(f["u"]), q_logits=dev(f["q_logits"]))),
        "gumbel_plain": (cpvo.SamplerParams(temp=0.7), cpvo.ACCEPT_GUMBEL, dict(noise=dev(f["noise"]))),
        "gumbel_top_p": (pr, cpvo.ACCEPT_GUMBEL, dict(noise=dev(f["noise"]))),
    }
    for name, (p, mode, kw) in cases.items():
        tok, n = ctx.spec_accept(dev(f["p_logits"]), dev(f["draft"]), dparams(p), mode, **kw)
        tok, n = tok.cpu().numpy(), n.cpu().numpy()
        assert np.array_equal(n, f[f"{name}_n"]), name
        for b in range(n.size):
            assert np.array_equal(tok[b, :n[b] + 1], f[f"{name}_tok"][b, :n[b] + 1]), (name, b)


def test_stream_fixture(ctx):
    from codpiece_amd.model import Model, Session, fused_generate, make_hparams
    f = load("stream")
    print("case golden micro-model stream", flush=True)
    gm = Model(ctx, make_hparams(**mg.MICRO))
    mf.load_into(gm, mf.make_tensors(mg.MICRO, seed=mg.MICRO_SEED))
    gm.ready()
    s = Session(gm, 256)
    toks, st = fused_generate(s, mg.micro_prompt(), mg.MICRO_GEN, mg.MICRO_DEPTH, tail=16, bulk=32)
    s.free()
    gm.free()
    assert toks == f["tokens"].tolist()
    assert [st.accepted, st.proposed, st.rounds] == f["stats"].tolist()
