"""GPU parity of tree-masked GQA attention against the oracle.

Bar: bit-exact.  Both sides implement the chunked attention contract:
fixed-point scores with exact integer sums; per 128-row chunk the weights
p = rint(expf(w - m_c) 2^22) and the values vq = rint(f16(v) 2^14), whose
products and normaliser are summed exactly in integers; then a fold over the
chunks in chunk order.  So the device result does not depend on its grid or
on the number of query rows per call.  The contract itself is held within
2^-12 max|v| + 2^-15 of binary64 attention by the oracle's own tests.
"""
import numpy as np
import pytest
import torch

from oracle import cpvo

pytestmark = pytest.mark.gpu

TREE16 = [-1, -1, -1, -1, 0, 0, 0, 1, 1, 1, 4, 4, 4, 10, 10, 10]


@pytest.fixture(scope="module")
def ctx():
    from codpiece_amd.runtime import Context
    c = Context(0)
    yield c
    c.close()


def make(rng, n_ctx, hkv, d, v_stride=None):
    k = cpvo.f32_to_f16_bits(rng.normal(size=(n_ctx, hkv * d)).astype(np.float32))
    v = cpvo.f32_to_f16_bits(rng.normal(size=(n_ctx, hkv * d)).astype(np.float32))
    vs = v_stride or (n_ctx + 7) // 8 * 8
    vt = np.zeros((hkv * d, vs), dtype=np.uint16)
    vt[:, :n_ctx] = v.T
    return k, v, vt


def run(ctx, t, h, hkv, d, n_past, parent, seed=0, extra_rows=0):
    rng = np.random.default_rng(seed)
    n_ctx = n_past + t + extra_rows
    k, v, vt = make(rng, n_ctx, hkv, d)
    q = rng.normal(size=(t, h, d)).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(d))
    print(f"case t={t} h={h} hkv={hkv} d={d} n_past={n_past} tree={parent is not None}", flush=True)
    par = None if parent is None else torch.tensor(parent, dtype=torch.int32, device="cuda")
    got = ctx.attn(torch.from_numpy(q).cuda(), torch.from_numpy(k.view(np.int16)).cuda(),
                   torch.from_numpy(vt.view(np.int16)).cuda(), n_past, par, hkv, float(scale)).cpu().numpy()
    ref = cpvo.attn(q, k[:n_past + t], v[:n_past + t], n_past, parent, scale)
    return got, ref


def close(got, ref):
    assert np.array_equal(got, ref), (np.abs(got - ref).max(), np.count_nonzero(got != ref))


@pytest.mark.parametrize("n_past", [0, 1, 37, 300, 1000])
def test_tiny_model_chain(ctx, n_past):
    # 8 Q / 2 KV heads x 64, T = k+1 = 5, causal chain (the reference's mask)
    close(*run(ctx, 5, 8, 2, 64, n_past, None))


@pytest.mark.parametrize("n_past", [4096, 4101, 4123, 4124])
def test_27b_class_chain(ctx, n_past):
    # n = n_past + 5 rows: a final chunk of 5, 10, 32 and 33 rows
    close(*run(ctx, 5, 40, 8, 128, n_past, None))


@pytest.mark.parametrize("n_ctx", [8192, 32768])
def test_tree_verify_config(ctx, n_ctx):
    # 40 Q / 8 KV heads x 128, a 16-node draft tree over n_ctx context rows
    close(*run(ctx, 16, 40, 8, 128, n_ctx, TREE16, seed=n_ctx))


@pytest.mark.parametrize("t,parent", [(13, TREE16[:13]), (11, None)])
def test_80_row_block_with_padding_rows(ctx, t, parent):
    # over the API's caches, 49 to 80 query rows per KV head run as one
    # 80-row block from 512 (chunk, KV head) units on: 65 and 55 rows here,
    # the rest of the block padding
    close(*run(ctx, t, 40, 8, 128, 8192, parent, seed=t))


@pytest.mark.parametrize("t,n_ctx", [(8, 8192), (20, 8192), (16, 4096)])
def test_query_block_shapes(ctx, t, n_ctx):
    # 40 Q / 8 KV heads, random trees: 40 query rows per KV head in one
    # 48-row block, 100 in 48 + 48 + 4, both from 512 units on; and 80 rows
    # below 512 units (4096 rows: 264 units) in 32-row blocks
    rng = np.random.default_rng(t + n_ctx)
    parent = [-1] + [int(rng.integers(-1, i)) for i in range(1, t)]
    close(*run(ctx, t, 40, 8, 128, n_ctx, parent, seed=t))


def test_80_row_block_d64(ctx):
    # d = 64, 2 KV heads: 257 chunks x 2 = 514 units, 64 query rows per KV head
    close(*run(ctx, 16, 8, 2, 64, 32768, TREE16, seed=64))


@pytest.mark.parametrize("n_past", [300, 8192])
def test_large_values_use_the_top_value_limb(ctx, n_past):
    # values of magnitude 512 and up carry a nonzero top limb (|vq| >= 2^23):
    # scattered rows and columns of them, so that some 64-row steps of a
    # wave hold one and others do not, next to small ones
    rng = np.random.default_rng(n_past + 1)
    t, h, hkv, d = 16, 40, 8, 128
    n_ctx = n_past + t
    k, v, vt = make(rng, n_ctx, hkv, d)
    big = cpvo.f32_to_f16_bits((rng.normal(size=(n_ctx, hkv * d)) * 3000).astype(np.float32))
    rows = rng.random(n_ctx) < 0.05
    cols = rng.random(hkv * d) < 0.3
    mask = rows[:, None] & cols[None, :]
    v = np.where(mask, big, v)
    vt[:, :n_ctx] = v.T
    q = rng.normal(size=(t, h, d)).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(d))
    par = torch.tensor(TREE16, dtype=torch.int32, device="cuda")
    got = ctx.attn(torch.from_numpy(q).cuda(), torch.from_numpy(k.view(np.int16)).cuda(),
                   torch.from_numpy(vt.view(np.int16)).cuda(), n_past, par, hkv, float(scale)).cpu().numpy()
    ref = cpvo.attn(q, k, v, n_past, TREE16, scale)
    close(got, ref)


def test_tree_with_linear_parents_equals_chain(ctx):
    a, _ = run(ctx, 8, 8, 2, 64, 200, None, seed=3)
    b, _ = run(ctx, 8, 8, 2, 64, 200, list(range(-1, 7)), seed=3)
    assert np.array_equal(a, b)


def test_rows_past_the_window_are_ignored(ctx):
    # cache rows beyond n_past + t (stale rows of a rolled-back round) never count
    a, ref = run(ctx, 5, 8, 2, 64, 100, None, seed=4, extra_rows=200)
    close(a, ref)


def test_wide_tree_max_nodes(ctx):
    # 64 nodes, one query head per KV head: a bushy random tree
    rng = np.random.default_rng(9)
    parent = [-1] + [int(rng.integers(-1, i)) for i in range(1, 64)]
    close(*run(ctx, 64, 2, 2, 64, 500, parent, seed=5))


def test_bad_shapes_are_rejected(ctx):
    from codpiece_amd import CpvError
    q = torch.zeros((4, 8, 96), device="cuda")
    kc = torch.zeros((16, 2 * 96), dtype=torch.int16, device="cuda")
    with pytest.raises(CpvError):
        ctx.attn(q, kc, kc, 4, None, 2, 0.1)


@pytest.mark.parametrize("split", [1, 7, 40])
def test_chain_in_pieces_equals_whole(ctx, split):
    rng = np.random.default_rng(21)
    n_past, t, h, hkv, d = 600, 40, 8, 2, 64
    k, v, vt = make(rng, n_past + t, hkv, d)
    qn = rng.normal(size=(t, h, d)).astype(np.float32)
    kc = torch.from_numpy(k.view(np.int16)).cuda()
    vtc = torch.from_numpy(vt.view(np.int16)).cuda()
    outs = []
    for t0 in range(0, t, split):
        tn = min(split, t - t0)
        q = torch.from_numpy(qn[t0:t0 + tn]).cuda()
        outs.append(ctx.attn(q, kc, vtc, n_past + t0, None, hkv, 0.125).cpu().numpy())
    got = np.concatenate(outs)
    ref = cpvo.attn(qn, k, v, n_past, None, np.float32(0.125))
    close(got, ref)
