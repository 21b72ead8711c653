"""GPU parity of cpv_qgemm_noalloc, the allocation-free GEMM entry point.

Bar: bit-exact against cpv_qgemm (the same kernels, with the activations and
the accumulator in the library's per-device scratch).  Two calls in a row, the
second on a smaller input, so a result left over in the shared scratch would
show.  The limits are refused on the host before anything is launched.
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


def _weight(t, n, k, seed):
    rng = np.random.default_rng(seed)
    return cpvo.quantize(t, rng.normal(0, 0.02, size=(n, k)).astype(np.float32))


def _both(ctx, w, x):
    print(f"case n={w.n} k={w.k} m={x.shape[0]}", flush=True)
    y_ref = ctx.qgemm(w, x)
    y = torch.full_like(y_ref, float("nan"))
    ctx.qgemm_noalloc(w, x, y)
    torch.cuda.synchronize()
    return y.cpu().numpy(), y_ref.cpu().numpy()


@pytest.mark.parametrize("t", [cpvo.Q4_K, cpvo.Q8_0, cpvo.Q6_K])
def test_noalloc_equals_qgemm_on_two_calls(ctx, t):
    rng = np.random.default_rng(7)
    # first call: 16 rows of a 1000 x 2048 weight; second: 3 rows of 200 x 1024
    for n, k, m in [(1000, 2048, 16), (200, 1024, 3)]:
        wq = _weight(t, n, k, seed=n + k + t)
        w = ctx.upload_weight(t, wq, n, k)
        x = torch.from_numpy(rng.normal(0, 1, size=(m, k)).astype(np.float32)).cuda()
        y, y_ref = _both(ctx, w, x)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        assert np.array_equal(y.view(np.uint32), cpvo.qgemm(t, wq, x.cpu().numpy()).view(np.uint32))
        w.free()


def test_noalloc_at_a_verify_shape(ctx):
    # the 27B-class wo projection (5120 x 5120, Q4_K) at 5 rows, then 1 row
    rng = np.random.default_rng(3)
    wq = _weight(cpvo.Q4_K, 5120, 5120, seed=11)
    w = ctx.upload_weight(cpvo.Q4_K, wq, 5120, 5120)
    for m in (5, 1):
        x = torch.from_numpy(rng.normal(0, 1, size=(m, 5120)).astype(np.float32)).cuda()
        y, y_ref = _both(ctx, w, x)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    w.free()


def test_noalloc_limits_are_refused(ctx):
    from codpiece_amd._lib import CPV_EINVAL, CpvError
    wq = _weight(cpvo.Q8_0, 64, 256, seed=5)
    w = ctx.upload_weight(cpvo.Q8_0, wq, 64, 256)
    x = torch.zeros((17, 256), dtype=torch.float32, device="cuda")
    y = torch.zeros((17, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(CpvError) as e:
        ctx.qgemm_noalloc(w, x, y)
    assert e.value.status == CPV_EINVAL
    w.free()
    # 16 rows of a 70,000-row weight need more than the 8 MiB accumulator
    big = ctx.upload_weight(cpvo.Q8_0, np.zeros((70000, 34 * 8), dtype=np.uint8), 70000, 256)
    x = torch.zeros((16, 256), dtype=torch.float32, device="cuda")
    y = torch.zeros((16, 70000), dtype=torch.float32, device="cuda")
    with pytest.raises(CpvError) as e:
        ctx.qgemm_noalloc(big, x, y)
    assert e.value.status == CPV_EINVAL
    big.free()
