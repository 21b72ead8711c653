"""GPU parity of the quantized GEMM, get_rows and argmax against the oracle.

Bar: bit-exact.  The GEMM contract sums exact integers, so the HIP kernel must
reproduce the oracle's f32 outputs bit for bit at every shape, including the
27B-class verify shapes (K, N) in {(5120, 7168), (5120, 5120), (5120, 17408),
(17408, 5120)} with M in {1, 5, 8, 16}; up to 16 rows share one pass over
the weights (12 and 24 rows check the partial and split launches; Q4_K above
8 rows runs on the 16x16x32 MFMA kernel).  Above 16 rows (Q4_K) or 8 rows
(Q6_K, Q8_0) every type runs on its wide (prefill) kernel, held to the same
bar.
"""
import numpy as np
import pytest
import torch

from oracle import cpvo

pytestmark = pytest.mark.gpu

TYPES = {"q8_0": cpvo.Q8_0, "q4_k": cpvo.Q4_K, "q6_k": cpvo.Q6_K}


@pytest.fixture(scope="module")
def ctx():
    from codpiece_amd.runtime import Context
    c = Context(0)
    yield c
    c.close()


_weights = {}


def weights(t, n, k, seed=0):
    key = (t, n, k, seed)
    if key not in _weights:
        rng = np.random.default_rng(seed + 1000 * t + n + 7 * k)
        wf = rng.normal(0, 0.02, size=(n, k)).astype(np.float32)
        _weights[key] = cpvo.quantize(t, wf)
    return _weights[key]


def run_case(ctx, t, n, k, m, seed=0, xscale=1.0):
    wq = weights(t, n, k)
    rng = np.random.default_rng(seed)
    x = (rng.normal(0, 1, size=(m, k)) * xscale).astype(np.float32)
    print(f"case type={t} n={n} k={k} m={m}", flush=True)
    w = ctx.upload_weight(t, wq, n, k)
    y = ctx.qgemm(w, torch.from_numpy(x).cuda()).cpu().numpy()
    ref = cpvo.qgemm(t, wq, x)
    w.free()
    return y, ref


@pytest.mark.parametrize("tname", list(TYPES))
@pytest.mark.parametrize("n,k", [(64, 256), (48, 512), (1000, 768), (33, 1024), (160, 4096)])
@pytest.mark.parametrize("m", [1, 3, 5, 9, 12, 13, 16, 24])
def test_qgemm_bit_exact_small(ctx, tname, n, k, m):
    t = TYPES[tname]
    y, ref = run_case(ctx, t, n, k, m)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()


@pytest.mark.parametrize("tname", ["q4_k", "q8_0"])
@pytest.mark.parametrize("k,n", [(5120, 7168), (5120, 5120), (5120, 17408), (17408, 5120)])
@pytest.mark.parametrize("m", [1, 5, 8, 16])
def test_qgemm_bit_exact_verify_shapes(ctx, tname, k, n, m):
    t = TYPES[tname]
    y, ref = run_case(ctx, t, n, k, m)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 16])
def test_qgemm_lm_head_q6_k(ctx, m):
    # the output projection of the 27B-class layout: Q6_K, K = 5120, a slice of
    # the 151,936 vocabulary rows (full vocab is covered by the e2e test); 16
    # rows are a draft tree's; below 8 rows the code-sum term is summed ahead
    # of the group loop, at 8 inside it
    y, ref = run_case(ctx, cpvo.Q6_K, 4096, 5120, m)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tname", ["q4_k", "q6_k"])
@pytest.mark.parametrize("m", [4, 9, 16])
def test_qgemm_extreme_scales_and_zero_rows(ctx, tname, m):
    # 4 rows: the 4x4x4 kernel; 9 and 16: the 16x16x32 ones
    t = TYPES[tname]
    n, k = 32, 1024
    rng = np.random.default_rng(3)
    wf = rng.normal(0, 0.02, size=(n, k)).astype(np.float32)
    wf[5] = 0.0                                   # an all-zero weight row
    wf[7] *= 1e3                                  # a row with huge scales
    wq = cpvo.quantize(t, wf)
    x = rng.normal(0, 1, size=(m, k)).astype(np.float32)
    x[1] = 0.0                                    # an all-zero activation row
    x[2] *= 1e-6
    w = ctx.upload_weight(t, wq, n, k)
    y = ctx.qgemm(w, torch.from_numpy(x).cuda()).cpu().numpy()
    ref = cpvo.qgemm(t, wq, x)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    assert np.all(y[1] == 0) and np.all(y[:, 5] == 0)


# ---- the wide kernels (the prompt prefill's rows; here 32 and more)

@pytest.mark.parametrize("tname", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("n,k", [(64, 256), (1000, 768), (33, 1024), (160, 4096)])
@pytest.mark.parametrize("m", [32, 37, 64, 100, 256])
def test_qgemm_wide_bit_exact_small(ctx, tname, n, k, m):
    y, ref = run_case(ctx, TYPES[tname], n, k, m)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()


@pytest.mark.parametrize("m", [32, 100])
def test_qgemm_wide_q8_0_partial_unit(ctx, m):
    # K = 800: 25 blocks of 32, so the last 256-element unit holds one block
    y, ref = run_case(ctx, cpvo.Q8_0, 40, 800, m)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()


@pytest.mark.parametrize("tname", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("k,n", [(5120, 7168), (5120, 5120), (5120, 17408), (17408, 5120)])
@pytest.mark.parametrize("m", [64, 256])
def test_qgemm_wide_bit_exact_prefill_shapes(ctx, tname, k, n, m):
    y, ref = run_case(ctx, TYPES[tname], n, k, m)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), np.abs(y - ref).max()


@pytest.mark.parametrize("tname", ["q4_k", "q6_k", "q8_0"])
def test_qgemm_wide_rows_match_the_skinny_kernel(ctx, tname):
    # a row's outputs do not depend on the rows batched with it: the wide
    # launch over 96 rows against the skinny kernel on 8-row slices
    t = TYPES[tname]
    n, k = 5120, 17408
    wq = weights(t, n, k)
    x = torch.from_numpy(np.random.default_rng(11).normal(0, 1, size=(96, k)).astype(np.float32)).cuda()
    w = ctx.upload_weight(t, wq, n, k)
    yw = ctx.qgemm(w, x).cpu().numpy()
    for r in range(0, 96, 8):
        ys = ctx.qgemm(w, x[r:r + 8].contiguous()).cpu().numpy()
        assert np.array_equal(yw[r:r + 8].view(np.uint32), ys.view(np.uint32)), r
    w.free()


@pytest.mark.parametrize("tname", ["q4_k", "q6_k", "q8_0"])
def test_qgemm_wide_extreme_scales_and_zero_rows(ctx, tname):
    t = TYPES[tname]
    n, k = 96, 1280
    rng = np.random.default_rng(4)
    wf = rng.normal(0, 0.02, size=(n, k)).astype(np.float32)
    wf[5] = 0.0
    wf[70] *= 1e3
    wq = cpvo.quantize(t, wf)
    x = rng.normal(0, 1, size=(70, k)).astype(np.float32)
    x[1] = 0.0
    x[2] *= 1e-6
    x[65] *= 1e4
    w = ctx.upload_weight(t, wq, n, k)
    y = ctx.qgemm(w, torch.from_numpy(x).cuda()).cpu().numpy()
    ref = cpvo.qgemm(t, wq, x)
    w.free()
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    assert np.all(y[1] == 0) and np.all(y[:, 5] == 0)


def test_qgemm_rejects_bad_shapes(ctx):
    from codpiece_amd import CpvError
    w = ctx.upload_weight(cpvo.Q8_0, weights(cpvo.Q8_0, 16, 64), 16, 64)
    x = torch.zeros((257, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(CpvError):
        ctx.qgemm(w, x)
    with pytest.raises(CpvError):
        ctx.upload_weight(cpvo.Q4_K, np.zeros(144, np.uint8), 1, 100)


@pytest.mark.parametrize("tname,k", [(t, k) for t in TYPES for k in (512, 5120)] + [("q8_0", 800)])
def test_get_rows_matches_ggml_dequant(ctx, tname, k):
    # four elements per thread; 800 = 25 Q8_0 blocks (a partial 256-element
    # unit); ids outside the table give zero rows
    t = TYPES[tname]
    n = 300
    wq = weights(t, n, k)
    w = ctx.upload_weight(t, wq, n, k)
    ids = [0, 7, 299, 150, 7, 64, 63]
    rows = torch.tensor(ids + [-1, n], dtype=torch.int32, device="cuda")
    got = ctx.get_rows(w, rows).cpu().numpy()
    w.free()
    ref = cpvo.dequantize(t, wq, k)[ids]
    assert np.array_equal(got[:len(ids)].view(np.uint32), ref.view(np.uint32))
    assert not got[len(ids):].any()


def test_argmax_first_maximum_and_noise(ctx):
    rng = np.random.default_rng(1)
    x = rng.normal(size=(7, 151936)).astype(np.float32)
    x[0, 100] = x[0, 90000] = 50.0               # tie: the lower index wins
    x[1, :] = -np.inf
    x[1, 12] = -1e30
    nz = rng.normal(size=x.shape).astype(np.float32)
    xt, nt = torch.from_numpy(x).cuda(), torch.from_numpy(nz).cuda()
    got = ctx.argmax_rows(xt).cpu().numpy()
    want = [cpvo.argmax(r) for r in x]
    assert got.tolist() == want and got[0] == 100 and got[1] == 12
    got2 = ctx.argmax_rows(xt, nt).cpu().numpy()
    assert got2.tolist() == [cpvo.argmax((a + b).astype(np.float32)) for a, b in zip(x, nz)]
