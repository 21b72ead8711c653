"""Draft trees end to end: cpv_verify_tree and cpv_session_commit_branch.

The reference verifies linear drafts only, so a tree is held to what a chain
gives.  Every node's logits must equal, bit for bit, those of the oracle's
chain verify of its root-to-node path from the same context; the attention
contract makes a row's result independent of rows it cannot see.  After
committing a path, the next round must equal the one that follows a chain
verify of that path (the compacted K/V rows are the chain's rows).
"""
import numpy as np
import pytest

from oracle import cpvo

import model_fixtures as mf

pytestmark = pytest.mark.gpu

# the canonical 16-node draft tree: 4 children of the context, 3 children each
# of nodes 0 and 1, 3 of node 4 and 3 of node 10 (widths 4, 6, 3, 3)
TREE = [-1, -1, -1, -1, 0, 0, 0, 1, 1, 1, 4, 4, 4, 10, 10, 10]
K_MODEL = dict(mf.TINY, n_layer=2, n_vocab=4096)


def path_to(parent, v):
    p = []
    while v >= 0:
        p.append(v)
        v = parent[v]
    return p[::-1]


def leaves(parent):
    return [v for v in range(len(parent)) if v not in parent]


@pytest.fixture(scope="module")
def kmodels():
    # small 27B-class mix: Q4_K linears, Q6_K embedding and head
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


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("n_prompt", [60, 200])
def test_tree_rows_equal_oracle_chains(kmodels, n_prompt):
    from codpiece_amd.model import Session
    ctx, gm, om = kmodels
    V = K_MODEL["n_vocab"]
    rng = np.random.default_rng(30 + n_prompt)
    prompt = rng.integers(0, V, size=n_prompt).tolist()
    toks = rng.integers(0, V, size=len(TREE)).tolist()
    g, o = Session(gm, 512, max_batch=256), cpvo.Session(om, 512)
    g.prefill(prompt)
    o.prefill(prompt)
    print("tree of", len(TREE), "after", n_prompt, flush=True)
    a = g.verify_tree(toks, TREE, want_logits=True)
    assert g.pos[0] == n_prompt + len(TREE)
    la = a.logits.cpu().numpy()
    ha = a.hidden.cpu().numpy()
    for leaf in leaves(TREE):
        path = path_to(TREE, leaf)
        o.set_pos(n_prompt, 0)
        b = o.step_fused_cached([toks[v] for v in path], 0, want_logits=True)
        assert np.array_equal(bits(la[path]), bits(b[3])), ("logits", path)
        assert np.array_equal(bits(ha[path]), bits(b[4])), ("hidden", path)
        assert [a.preds[v] for v in path] == b[0].tolist()
    g.free()
    o.free()


@pytest.mark.parametrize("path", [[1, 8], [0, 4, 10, 13], [0, 4], [2], []])
def test_commit_branch_then_round_equals_chain(kmodels, path):
    from codpiece_amd.model import Session
    ctx, gm, om = kmodels
    V = K_MODEL["n_vocab"]
    rng = np.random.default_rng(40 + len(path))
    prompt = rng.integers(0, V, size=80).tolist()
    toks = rng.integers(0, V, size=len(TREE)).tolist()
    nxt = rng.integers(0, V, size=5).tolist()
    g, o = Session(gm, 512, max_batch=256), cpvo.Session(om, 512)
    g.prefill(prompt)
    o.prefill(prompt)
    print("commit", path, flush=True)
    g.verify_tree(toks, TREE)
    g.commit_branch(path)
    assert g.pos[0] == 80 + len(path)
    if path:
        o.step_fused_cached([toks[v] for v in path], 0)
    assert o.pos[0] == 80 + len(path)
    a = g.step_fused_cached(nxt, 0, want_logits=True)
    b = o.step_fused_cached(nxt, 0, want_logits=True)
    assert np.array_equal(bits(a.logits.cpu().numpy()), bits(b[3]))
    assert a.preds == b[0].tolist()
    g.free()
    o.free()


def test_two_tree_rounds_in_a_row(kmodels):
    # commit, then a second tree on top of the compacted rows
    from codpiece_amd.model import Session
    ctx, gm, om = kmodels
    V = K_MODEL["n_vocab"]
    rng = np.random.default_rng(50)
    prompt = rng.integers(0, V, size=64).tolist()
    t1 = rng.integers(0, V, size=len(TREE)).tolist()
    t2 = rng.integers(0, V, size=len(TREE)).tolist()
    g, o = Session(gm, 512, max_batch=256), cpvo.Session(om, 512)
    g.prefill(prompt)
    o.prefill(prompt)
    g.verify_tree(t1, TREE)
    p1 = [1, 9]
    g.commit_branch(p1)
    o.step_fused_cached([t1[v] for v in p1], 0)
    a = g.verify_tree(t2, TREE, want_logits=True)
    la = a.logits.cpu().numpy()
    base = 64 + len(p1)
    for leaf in (3, 15):
        path = path_to(TREE, leaf)
        o.set_pos(base, 0)
        b = o.step_fused_cached([t2[v] for v in path], 0, want_logits=True)
        assert np.array_equal(bits(la[path]), bits(b[3]))
    g.free()
    o.free()


def test_tree_arguments_are_checked(kmodels):
    from codpiece_amd.model import Session
    from codpiece_amd.runtime import CpvError
    ctx, gm, om = kmodels
    g = Session(gm, 256, max_batch=128)
    g.prefill(list(range(10)))
    with pytest.raises(CpvError):
        g.verify_tree([1, 2, 3], [-1, 1, 0])          # a node that is its own parent
    with pytest.raises(CpvError):
        g.verify_tree([1, 2, 3], [-1, 2, 0])          # a parent after its child
    with pytest.raises(CpvError):
        g.verify_tree(list(range(65)), [-1] * 65)     # more than 64 nodes
    with pytest.raises(CpvError):
        g.commit_branch([0])                          # no tree pending
    assert g.pos[0] == 10
    g.verify_tree(list(range(16)), TREE)
    with pytest.raises(CpvError):
        g.commit_branch([4])                          # does not start at a root
    with pytest.raises(CpvError):
        g.commit_branch([0, 7])                       # 7 is not a child of 0
    with pytest.raises(CpvError):
        g.commit_branch([0, 4, 10, 13, 13])           # longer than any path
    g.commit_branch([0, 5])
    assert g.pos[0] == 12
    with pytest.raises(CpvError):
        g.commit_branch([0])                          # already committed
    g.verify_tree(list(range(4)), [-1, 0, 1, 2])
    g.step_fused_cached([5], 0)                       # a chain verify ends the pending tree
    with pytest.raises(CpvError):
        g.commit_branch([0])
    g.free()
