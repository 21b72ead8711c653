"""Round replay (per-shape HIP graphs) against eager rounds, on the device.

Bar: bit-exact.  Two sessions over the config-1 model, one replaying
captured rounds (the default) and one launching every kernel, run the same
rounds: a prompt of 960 tokens, then rounds of 5, 1 and 3 tokens at depths 4
and 0 with random rewinds, while n_past crosses the 1024-row boundary (a new
attention grid, so a new capture).  Between rounds the program does other
device work (a GEMM on another weight and a prefill on a third session) and
synchronizes, so each replay follows eager work.  Every round's preds, chain,
confidences, logits and hidden rows must be equal bit for bit, and the
replaying session must have replayed most of its rounds.
"""
import numpy as np
import pytest
import torch

import model_fixtures as mf

pytestmark = pytest.mark.gpu

V = mf.TINY["n_vocab"]


@pytest.fixture(scope="module")
def model():
    from codpiece_amd.model import Model, make_hparams
    from codpiece_amd.runtime import Context
    from oracle import cpvo
    ctx = Context(0)
    gm = Model(ctx, make_hparams(**mf.TINY))
    mf.load_into(gm, mf.make_tensors(mf.TINY, seed=0))
    gm.ready()
    rng = np.random.default_rng(4)
    w = ctx.upload_weight(cpvo.Q8_0, cpvo.quantize(cpvo.Q8_0, rng.normal(0, 0.02, (512, 1024)).astype(np.float32)),
                          512, 1024)
    yield ctx, gm, w
    w.free()
    gm.free()
    ctx.close()


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_replayed_rounds_equal_eager_rounds(model):
    from codpiece_amd.model import Session
    ctx, gm, w = model
    a, b, other = Session(gm, 2048), Session(gm, 2048), Session(gm, 2048)
    b.set_replay(False)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, V, size=960).tolist()
    for s in (a, b):
        for c in range(0, len(prompt), 64):
            s.prefill(prompt[c:c + 64])
    x = torch.randn(5, 1024, device="cuda")
    plan = [(5, 4)] * 12 + [(1, 4)] * 6 + [(5, 0)] * 6 + [(3, 4)] * 6 + [(5, 4)] * 16
    for r, (t, depth) in enumerate(plan):
        toks = rng.integers(0, V, size=t).tolist()
        print(f"case round {r} t={t} depth={depth} n_past={a.pos[0]}", flush=True)
        oa = a.step_fused_cached(toks, depth, want_logits=True)
        ob = b.step_fused_cached(toks, depth, want_logits=True)
        assert oa.preds == ob.preds, r
        assert oa.chain == ob.chain, r
        assert _eq(oa.conf, ob.conf), r
        assert _eq(oa.logits.cpu().numpy(), ob.logits.cpu().numpy()), r
        assert _eq(oa.hidden.cpu().numpy(), ob.hidden.cpu().numpy()), r
        # a rewind as the loop does it: keep + 1 rows stay
        keep = int(rng.integers(0, t))
        n_past, mtp_past = a.pos
        assert (n_past, mtp_past) == b.pos
        for s in (a, b):
            s.set_pos(n_past - (t - keep - 1), mtp_past + keep + 1)
        # other device work between the rounds, then a synchronization
        ctx.qgemm(w, x)
        other.prefill(rng.integers(0, V, size=8).tolist())
        torch.cuda.synchronize()
    assert a.pos[0] > 1024 and a.pos == b.pos
    captured, replayed = a.replay_stats
    assert captured >= 4 and replayed >= len(plan) - 2 * captured, (captured, replayed)
    assert b.replay_stats == (0, 0)
    for s in (a, b, other):
        s.free()


def test_long_context_gate_fold_equals_unfused_attention(model):
    # The gate kernel folds the attention's chunk partials itself, the first
    # 48 chunks from registers and the rest from memory.  At 6600 + 5 rows
    # (52 chunks) a round must equal, bit for bit, the same round through
    # the attention's own fold kernel (an attention tap selects that path).
    from codpiece_amd.model import Session
    ctx, gm, w = model
    a, b = Session(gm, 8192, max_batch=512), Session(gm, 8192, max_batch=512)
    b.set_attn_tap(torch.zeros(16, device="cuda"))   # (too small to hold a copy: only the path changes)
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, V, size=6600).tolist()
    for s in (a, b):
        for c in range(0, len(prompt), 512):
            s.prefill(prompt[c:c + 512])
    for r in range(2):
        toks = rng.integers(0, V, size=5).tolist()
        print(f"case long-context round {r} n_past={a.pos[0]}", flush=True)
        oa = a.step_fused_cached(toks, 4, want_logits=True)
        ob = b.step_fused_cached(toks, 4, want_logits=True)
        assert oa.preds == ob.preds and oa.chain == ob.chain, r
        assert _eq(oa.logits.cpu().numpy(), ob.logits.cpu().numpy()), r
        assert _eq(oa.hidden.cpu().numpy(), ob.hidden.cpu().numpy()), r
    assert a.pos == b.pos and a.pos[0] > 48 * 128
    for s in (a, b):
        s.free()
