"""GPU parity on randomly drawn shapes: attention over the API's f16 caches
and the quantized GEMM, against the oracle.

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
  up to 256; activation scales 1e-3 to 50; zero weight and activation rows.
"""
import numpy as np
import pytest
import torch

from oracle import cpvo

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
