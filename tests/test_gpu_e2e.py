"""End-to-end parity of the verify round on the config-1 model (device vs oracle).

Two bars.  (1) Lockstep: each device call runs with its attention tap on and
the oracle continues from the device's attention outputs, after checking them
against its own f64 attention (|dev - ref| <= 2e-5 + 2e-4|ref|); everything
else -- embeddings, norms, rope, the exact-window GEMMs, gates, SwiGLU, the LM
head, argmax, the MTP chain, the KV writes and the round bookkeeping -- must
then agree bit for bit (logits, hidden, preds, chain), the peak confidence to
1e-6.  (2) Free-running: attention follows the same exact, order-free contract on
both sides, so without any injection the logits, the greedy streams and the
acceptance counts are bit-identical to the oracle's.
"""
import numpy as np
import pytest
import torch

from oracle import cpvo

import model_fixtures as mf

pytestmark = pytest.mark.gpu

V = mf.TINY["n_vocab"]


@pytest.fixture(scope="module")
def models():
    from codpiece_amd.model import Model, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    hp = make_hparams(**mf.TINY)
    tensors = mf.make_tensors(mf.TINY, seed=0)
    gm = Model(ctx, hp)
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
    ctx, gm, om = models
    return Session(gm, n_ctx), cpvo.Session(om, n_ctx)


def paired(models, n_ctx=512, max_t=160, depth=4):
    g, o = sessions(models, n_ctx)
    hp = mf.TINY
    n = (hp["n_layer"] + depth) * max_t * hp["n_head"] * hp["head_dim"]
    return mf.PairedSession(g, o, n), g, o


def test_lockstep_single_round(models):
    ps, g, o = paired(models)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, V, size=70).tolist()
    print("lockstep: prefill 64 + round of 6 at depth 4", flush=True)
    ps.prefill(prompt[:64])
    ps.step_fused_cached(prompt[64:], 4)
    assert ps.pos == (70, 0)
    print("worst attention ratio", ps.worst, flush=True)
    g.free()
    o.free()


def test_lockstep_fused_loop_config1(models):
    # config 1: 128 random prompt ids, greedy fused speculation at depth 4, 64 new tokens,
    # driven by the host loop; the paired session checks every call
    from codpiece_amd.model import fused_generate
    ps, g, o = paired(models)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, V, size=128).tolist()
    print("lockstep fused generate 64 at depth 4", flush=True)
    toks, st = fused_generate(ps, prompt, 64, 4)
    assert len(toks) == 64 and st.rounds > 0
    print("rounds", st.rounds, "accepted", st.accepted, "worst ratio", ps.worst, flush=True)
    g.free()
    o.free()


def test_lockstep_all_drafts_accepted(models):
    # drafts = the trunk's own greedy continuation, so every draft is kept:
    # the multi-accept path that random MTP drafts never reach
    from codpiece_amd.model import fused_generate  # noqa: F401  (same loop rules below)
    ps, g, o = paired(models)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, V, size=40).tolist()
    ps.prefill(prompt[:-1])
    n0 = ps.pos[0]
    cont = [prompt[-1]]
    for _ in range(5):
        out = ps.step_fused_cached(cont[-1:], 0)
        cont.append(out.preds[0])
    ps.set_pos(n0, 0)
    out = ps.step_fused_cached(cont[:5], 4)
    assert out.preds[:4] == cont[1:5]
    assert out.preds[4] == cont[5]
    g.free()
    o.free()


def test_lockstep_gumbel_noise(models):
    # stochastic argmax: logits + per-token noise, same noise on both sides
    ps, g, o = paired(models)
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, V, size=30).tolist()
    ps.prefill(prompt[:25])
    u = rng.random(size=(5, V)).astype(np.float32)
    noise = torch.from_numpy(-np.log(-np.log(np.maximum(u, 1e-12))).astype(np.float32)).cuda()
    ps.step_fused_cached(prompt[25:], 2, noise=noise)
    g.free()
    o.free()


def test_free_running_round_is_bit_exact(models):
    g, o = sessions(models)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, V, size=70).tolist()
    g.prefill(prompt[:64])
    o.prefill(prompt[:64])
    a = g.step_fused_cached(prompt[64:], 4, want_logits=True)
    p, chain, conf, logits, hidden = o.step_fused_cached(prompt[64:], 4, want_logits=True)
    assert np.array_equal(a.logits.cpu().numpy(), logits)
    assert np.array_equal(a.hidden.cpu().numpy(), hidden)
    assert a.preds == p.tolist() and a.chain == chain.tolist()
    g.free()
    o.free()


def test_free_running_fused_loop_streams(models):
    from codpiece_amd.model import fused_generate
    g, o = sessions(models)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, V, size=128).tolist()
    toks, st = fused_generate(g, prompt, 64, 4)
    otoks, ost = o.fused_generate(prompt, 64, 4)
    same = next((i for i, (x, y) in enumerate(zip(toks, otoks)) if x != y), len(toks))
    print("free-running streams agree on the first", same, "of", len(toks), "tokens", flush=True)
    assert toks == otoks
    assert [st.accepted, st.proposed, st.rounds] == ost
    g.free()
    o.free()


def test_rewind_then_redo_is_deterministic(models):
    g, _ = sessions(models)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, V, size=20).tolist()
    g.prefill(prompt[:15])
    a = g.step_fused_cached(prompt[15:], 4, want_logits=True)
    la = a.logits.cpu()
    g.set_pos(15, 0)
    b = g.step_fused_cached(prompt[15:], 4, want_logits=True)
    assert a.preds == b.preds and a.chain == b.chain
    assert torch.equal(la, b.logits.cpu())
    g.free()


def test_context_overflow_is_an_error(models):
    from codpiece_amd import CpvError
    g, _ = sessions(models, n_ctx=16)
    g.prefill(list(range(12)))
    with pytest.raises(CpvError):
        g.step_fused_cached([1, 2, 3, 4, 5], 4)
    g.free()


def test_lockstep_mtp_window_restart(models):
    # mtp_past + t > min(n_ctx, 16384): the draft head's window restarts at row 0
    ps, g, o = paired(models)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, V, size=25).tolist()
    ps.prefill(prompt[:20])
    ps.set_pos(20, 509)
    ps.step_fused_cached(prompt[20:], 3)
    assert ps.pos == (25, 0)
    g.free()
    o.free()


K_MODEL = dict(mf.TINY, n_layer=2, n_vocab=4096)


@pytest.fixture(scope="module")
def kmodels():
    # the 27B-class mix at small size: Q4_K linears, Q6_K embedding and head
    from codpiece_amd.model import Model, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    tensors = mf.make_tensors(K_MODEL, seed=7, qtype=cpvo.Q4_K, head_type=cpvo.Q6_K)
    gm = Model(ctx, make_hparams(**K_MODEL))
    mf.load_into(gm, tensors)
    gm.ready()
    om = cpvo.Model(K_MODEL)
    mf.load_into(om, tensors)
    yield ctx, gm, om
    gm.free()
    om.free()
    ctx.close()


def test_q4k_model_rounds_and_stream_are_bit_exact(kmodels):
    from codpiece_amd.model import Session, fused_generate
    ctx, gm, om = kmodels
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, K_MODEL["n_vocab"], size=70).tolist()
    g, o = Session(gm, 256), cpvo.Session(om, 256)
    g.prefill(prompt[:60])
    o.prefill(prompt[:60])
    a = g.step_fused_cached(prompt[60:65], 4, want_logits=True)
    b = o.step_fused_cached(prompt[60:65], 4, want_logits=True)
    assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
    assert np.array_equal(a.hidden.cpu().numpy().view(np.uint32), b[4].view(np.uint32))
    assert a.preds == b[0].tolist() and a.chain == b[1].tolist()
    g.free()
    o.free()
    g, o = Session(gm, 256), cpvo.Session(om, 256)
    toks, st = fused_generate(g, prompt, 24, 4, tail=16, bulk=32)
    otoks, ost = o.fused_generate(prompt, 24, 4, tail=16, bulk=32)
    assert toks == otoks
    assert [st.accepted, st.proposed, st.rounds] == ost
    g.free()
    o.free()


def test_q4k_long_prefill_chunks_are_bit_exact(kmodels):
    # the prompt prefill at the chunk sizes the wide Q4_K GEMM takes: 256 rows
    # (four full row blocks), then 37 (a partial one), then a round on top
    from codpiece_amd.model import Session
    ctx, gm, om = kmodels
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, K_MODEL["n_vocab"], size=300).tolist()
    g, o = Session(gm, 512, max_batch=256), cpvo.Session(om, 512)
    for c0, c1 in ((0, 256), (256, 293)):
        print(f"prefill {c0}:{c1}", flush=True)
        g.prefill(prompt[c0:c1])
        o.prefill(prompt[c0:c1])
    a = g.step_fused_cached(prompt[293:298], 4, want_logits=True)
    b = o.step_fused_cached(prompt[293:298], 4, want_logits=True)
    assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
    assert np.array_equal(a.hidden.cpu().numpy().view(np.uint32), b[4].view(np.uint32))
    assert a.preds == b[0].tolist() and a.chain == b[1].tolist()
    g.free()
    o.free()


def test_q4k_prefill_of_600_rows_is_bit_exact(kmodels):
    # one prefill call past the cpv_qgemm row limit: ten 64-row blocks of the
    # wide GEMM, the last one partial (24 rows)
    from codpiece_amd.model import Session
    ctx, gm, om = kmodels
    rng = np.random.default_rng(10)
    prompt = rng.integers(0, K_MODEL["n_vocab"], size=605).tolist()
    g, o = Session(gm, 1024, max_batch=600), cpvo.Session(om, 1024)
    g.prefill(prompt[:600])
    o.prefill(prompt[:600])
    a = g.step_fused_cached(prompt[600:605], 4, want_logits=True)
    b = o.step_fused_cached(prompt[600:605], 4, want_logits=True)
    assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
    assert np.array_equal(a.hidden.cpu().numpy().view(np.uint32), b[4].view(np.uint32))
    assert a.preds == b[0].tolist() and a.chain == b[1].tolist()
    g.free()
    o.free()


W_MODEL = dict(mf.TINY, n_layer=1, n_embd=5120, n_head=40, n_head_kv=8, head_dim=128, n_rot=128,
               rope_sections=[22, 22, 20, 0], n_ff=1536, n_vocab=2048)


@pytest.mark.gpu
def test_wide_rows_round_is_bit_exact():
    # d_model 5120: 20 units per row, so the row kernels' waves take a second
    # unit (the widths above all fit one pass); the 27B-class head layout
    from codpiece_amd.model import Model, Session, make_hparams
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    tensors = mf.make_tensors(W_MODEL, seed=11, qtype=cpvo.Q4_K, head_type=cpvo.Q6_K)
    gm = Model(ctx, make_hparams(**W_MODEL))
    mf.load_into(gm, tensors)
    gm.ready()
    om = cpvo.Model(W_MODEL)
    mf.load_into(om, tensors)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, W_MODEL["n_vocab"], size=45).tolist()
    g, o = Session(gm, 128), cpvo.Session(om, 128)
    g.prefill(prompt[:40])
    o.prefill(prompt[:40])
    a = g.step_fused_cached(prompt[40:45], 4, want_logits=True)
    b = o.step_fused_cached(prompt[40:45], 4, want_logits=True)
    assert np.array_equal(a.hidden.cpu().numpy().view(np.uint32), b[4].view(np.uint32))
    assert np.array_equal(a.logits.cpu().numpy().view(np.uint32), b[3].view(np.uint32))
    assert a.preds == b[0].tolist() and a.chain == b[1].tolist()
    g.free()
    o.free()
    gm.free()
    om.free()
    ctx.close()


def test_wide_query_blocks_at_long_context(models):
    # From 512 (chunk, KV head) units on, a KV head's query rows past 32 run
    # in 48-row blocks over the session's limb caches; the config-1 model (2
    # KV heads) gets there at 32768 cached rows.  Each verify row depends only
    # on its own token and the rows before it, so the first 8 rows of a
    # 16-row verify (64 query rows per KV head: 48-row blocks) equal an 8-row
    # verify (32 rows: one 32-row block) bit for bit, and a 16-node tree with
    # linear parents (48-row blocks, ancestor masks) equals the 16-row chain.
    from codpiece_amd.model import Session
    ctx, gm, om = models
    n = 32768
    s = Session(gm, n + 64, max_batch=512)
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, V, size=n).tolist()
    print("case prefill 32768 rows", flush=True)
    for c in range(0, n, 512):
        s.prefill(prompt[c:c + 512])
    s.set_pos(n, 0)
    toks = rng.integers(0, V, size=16).tolist()
    print("case 16-row chain", flush=True)
    a = s.step_fused_cached(toks, 0, want_logits=True)
    la, ha = a.logits.cpu().numpy(), a.hidden.cpu().numpy()
    s.set_pos(n, 0)
    print("case 8-row chain", flush=True)
    b = s.step_fused_cached(toks[:8], 0, want_logits=True)
    assert b.preds == a.preds[:8]
    assert np.array_equal(b.logits.cpu().numpy().view(np.uint32), la[:8].view(np.uint32))
    assert np.array_equal(b.hidden.cpu().numpy().view(np.uint32), ha[:8].view(np.uint32))
    s.set_pos(n, 0)
    print("case 16-node linear tree", flush=True)
    t = s.verify_tree(toks, [-1] + list(range(15)), want_logits=True)
    assert t.preds == a.preds
    assert np.array_equal(t.logits.cpu().numpy().view(np.uint32), la.view(np.uint32))
    assert np.array_equal(t.hidden.cpu().numpy().view(np.uint32), ha.view(np.uint32))
    s.free()
