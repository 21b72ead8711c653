"""Pins for rms_norm, RoPE and the masked GQA attention oracle."""
import numpy as np
import pytest

from oracle import cpvo


def test_rms_norm_matches_double_reference():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 2, size=(7, 5120)).astype(np.float32)
    w = rng.normal(1, 0.1, size=5120).astype(np.float32)
    y = cpvo.rms_norm(x, 1e-6, w)
    for r in range(7):
        sq = (x[r] * x[r]).astype(np.float64)         # f32 squares, summed in double
        mean = np.float32(sq.sum() / 5120)
        scale = np.float32(1) / np.sqrt(np.float32(mean + np.float32(1e-6)), dtype=np.float32)
        ref = (x[r] * scale).astype(np.float32) * w
        assert np.array_equal(y[r], ref)


def test_rms_norm_is_scale_invariant_and_handles_zero():
    x = np.zeros(64, dtype=np.float32)
    assert np.all(cpvo.rms_norm(x, 1e-6) == 0)
    x = np.arange(1, 65, dtype=np.float32)
    a = cpvo.rms_norm(x, 0.0)
    b = cpvo.rms_norm(x * 4, 0.0)                      # powers of two scale exactly
    assert np.array_equal(a, b)
    np.testing.assert_allclose(np.sqrt((a.astype(np.float64) ** 2).mean()), 1.0, rtol=1e-6)


def test_rope_table_is_ggml_theta_recurrence():
    cs = cpvo.rope_table(64, 64, 1e6)
    assert np.all(cs[0, :, 0] == 1) and np.all(cs[0, :, 1] == 0)
    th_scale = np.float32(np.power(np.float32(1e6), np.float32(-2.0 / 64)))
    th = np.float32(37)
    for i in range(32):
        np.testing.assert_allclose(cs[37, i], [np.cos(th), np.sin(th)], atol=2e-6)
        th = np.float32(th * th_scale)


def test_rope_sections_covering_all_pairs_equal_plain_rope():
    # qwen35 IMROPE with equal text streams and sections that cover every pair
    a = cpvo.rope_table(100, 64, 1e6)
    b = cpvo.rope_table(100, 64, 1e6, sections=[11, 11, 10, 0])
    assert np.array_equal(a, b)
    # sections that leave pairs to the 4th (zero) stream: those pairs do not rotate
    c = cpvo.rope_table(100, 128, 1e6, sections=[22, 22, 20, 0])
    assert np.all(c[50, 62] == [1.0, 0.0])


def test_rope_rotates_neox_pairs_and_preserves_norm():
    rng = np.random.default_rng(1)
    x = rng.normal(size=128).astype(np.float32)
    cs = cpvo.rope_table(200, 128, 1e6)
    y = cpvo.rope_neox(x, 128, cs[123])
    np.testing.assert_allclose(np.linalg.norm(y), np.linalg.norm(x), rtol=1e-6)
    c, s = cs[123, 5]
    np.testing.assert_allclose([y[5], y[5 + 64]], [x[5] * c - x[69] * s, x[5] * s + x[69] * c], rtol=1e-6)
    # partial rotary: dims past n_rot untouched
    z = cpvo.rope_neox(x, 64, cs[123, :32].copy())
    assert np.array_equal(z[64:], x[64:])


def _cache(rng, n, hkv, d):
    k = cpvo.f32_to_f16_bits(rng.normal(size=(n, hkv * d)).astype(np.float32))
    v = cpvo.f32_to_f16_bits(rng.normal(size=(n, hkv * d)).astype(np.float32))
    return k, v


def _brute(q, k, v, n_past, parent, scale, H, Hkv, D):
    """Dense masked softmax over an explicit [T, n] visibility matrix (f64)."""
    T = q.shape[0]
    n = n_past + T
    vis = np.zeros((T, n), dtype=bool)
    vis[:, :n_past] = True
    for t in range(T):
        a = t
        while a >= 0:
            vis[t, n_past + a] = True
            a = parent[a] if parent is not None else a - 1
    kf = cpvo.f16_bits_to_f32(k).astype(np.float64).reshape(-1, Hkv, D)
    vf = cpvo.f16_bits_to_f32(v).astype(np.float64).reshape(-1, Hkv, D)
    qf = cpvo.f16_bits_to_f32(cpvo.f32_to_f16_bits(q)).astype(np.float64)
    out = np.zeros((T, H, D))
    for h in range(H):
        kh = h // (H // Hkv)
        s = qf[:, h] @ kf[:n, kh].T * scale
        s[~vis] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h] = p @ vf[:n, kh]
    return out.reshape(T, H * D)


TREE = [-1, -1, -1, -1, 0, 0, 0, 1, 1, 1, 4, 4, 4, 10, 10, 10]


def test_attention_f64_matches_dense_masked_softmax():
    rng = np.random.default_rng(2)
    H, Hkv, D, n_past = 8, 2, 64, 300
    T = len(TREE)
    k, v = _cache(rng, n_past + T, Hkv, D)
    q = rng.normal(size=(T, H, D)).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(D))
    got = cpvo.attn(q, k, v, n_past, TREE, scale, f64=True)
    ref = _brute(q, k, v, n_past, TREE, float(scale), H, Hkv, D)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("n_past,qmul", [(0, 1.0), (1, 3.0), (300, 1.0), (700, 3.0), (4096, 1.0)])
def test_exact_contract_is_attention_up_to_its_fixed_points(n_past, qmul):
    # the contract rounds the scores to 15-bit fixed point, each weight to a
    # multiple of 2^-22 and each value to a multiple of 2^-14 (so within
    # 2^-15, a weighted mean of which stays within 2^-15):
    # |exact - f64| <= 2^-12 * max|v| + 2^-15 bounds them together (measured:
    # 3e-6 max|v| at qmul 1, 6e-5 max|v| at qmul 3)
    rng = np.random.default_rng(n_past + 7)
    H, Hkv, D = 8, 2, 64
    T = len(TREE)
    k, v = _cache(rng, n_past + T, Hkv, D)
    q = (qmul * rng.normal(size=(T, H, D))).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(D))
    a = cpvo.attn(q, k, v, n_past, TREE, scale)
    b = cpvo.attn(q, k, v, n_past, TREE, scale, f64=True)
    bound = 2.0 ** -12 * np.abs(cpvo.f16_bits_to_f32(v)).max() + 2.0 ** -15
    assert np.abs(a - b).max() <= bound


@pytest.mark.parametrize("vscale,rel", [(1e-3, 4e-3), (2.0 ** -10, 4e-3), (2.0 ** -6, 4e-4), (1.0, 2e-5)])
def test_exact_contract_with_small_values_is_absolute_in_v(vscale, rel):
    # vq = rint(f16(v) 2^14) rounds each value within 2^-15 absolute, not
    # relative: for values far below 2^-4 the bound 2^-12 max|v| + 2^-15 is
    # its absolute term, and the error relative to max|v| grows as the
    # values shrink (measured: 0.17% of max|v| for V ~ N(0, 1e-3), 0.013%
    # at 2^-6, 4e-6 at unit scale).  Each case holds the bound and its
    # measured relative size (with margin).
    rng = np.random.default_rng(int(1 / vscale) if vscale < 1 else 5)
    H, Hkv, D = 8, 2, 64
    T = len(TREE)
    n = 300 + T
    k = cpvo.f32_to_f16_bits(rng.normal(size=(n, Hkv * D)).astype(np.float32))
    v = cpvo.f32_to_f16_bits((vscale * rng.normal(size=(n, Hkv * D))).astype(np.float32))
    q = rng.normal(size=(T, H, D)).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(D))
    a = cpvo.attn(q, k, v, 300, TREE, scale)
    b = cpvo.attn(q, k, v, 300, TREE, scale, f64=True)
    vmax = np.abs(cpvo.f16_bits_to_f32(v)).max()
    err = np.abs(a - b).max()
    assert err <= 2.0 ** -12 * vmax + 2.0 ** -15
    assert err / vmax <= rel


@pytest.mark.parametrize("n_past", [0, 127, 128, 700, 2047])
def test_exact_contract_uniform_weights_closed_form(n_past):
    # q = 0: every visible score is 0, so in every chunk m = 0, e = 1,
    # p = 2^22, Z_c = (rows) 2^22 and the chunk factors are 1; with v = 1
    # (vq = 2^14) each chunk's P_c is its row count and the fold their sum, so
    # out = (float)n * (float)(1/n) exactly.  A dropped or repeated row or
    # chunk, a wrong factor, scale or limb weight, or a missing normalisation
    # breaks the equality.
    rng = np.random.default_rng(n_past)
    H, Hkv, D, T = 4, 2, 32, 3
    n = n_past + T
    k = cpvo.f32_to_f16_bits(rng.normal(size=(n, Hkv * D)).astype(np.float32))
    v = cpvo.f32_to_f16_bits(np.ones((n, Hkv * D), np.float32))
    q = np.zeros((T, H, D), np.float32)
    out = cpvo.attn(q, k, v, n_past, None, 0.5)
    for t in range(T):
        nv = n_past + t + 1
        want = np.float32(np.float32(nv) * np.float32(1.0 / nv))
        assert np.all(out[t] == want), (t, out[t][:3], want)


def test_linear_chain_equals_tree_with_linear_parents():
    rng = np.random.default_rng(3)
    H, Hkv, D, n_past, T = 4, 1, 32, 50, 5
    k, v = _cache(rng, n_past + T, Hkv, D)
    q = rng.normal(size=(T, H, D)).astype(np.float32)
    a = cpvo.attn(q, k, v, n_past, None, 0.2)
    b = cpvo.attn(q, k, v, n_past, list(range(-1, T - 1)), 0.2)
    assert np.array_equal(a, b)


def test_invisible_rows_do_not_matter_and_siblings_differ_only_by_self():
    rng = np.random.default_rng(4)
    H, Hkv, D, n_past = 4, 2, 32, 20
    T = len(TREE)
    k, v = _cache(rng, n_past + T, Hkv, D)
    q = np.repeat(rng.normal(size=(1, H, D)).astype(np.float32), T, axis=0)
    a = cpvo.attn(q, k, v, n_past, TREE, 0.15)
    # change the K/V of node 15 (only node 15 sees it)
    k2, v2 = k.copy(), v.copy()
    k2[n_past + 15] = cpvo.f32_to_f16_bits(rng.normal(size=Hkv * D).astype(np.float32))
    v2[n_past + 15] = cpvo.f32_to_f16_bits(rng.normal(size=Hkv * D).astype(np.float32))
    b = cpvo.attn(q, k2, v2, n_past, TREE, 0.15)
    assert np.array_equal(a[:15], b[:15]) and not np.array_equal(a[15], b[15])


def test_single_visible_row_returns_its_value():
    rng = np.random.default_rng(5)
    H, Hkv, D = 2, 1, 16
    k, v = _cache(rng, 1, Hkv, D)
    q = rng.normal(size=(1, H, D)).astype(np.float32)
    out = cpvo.attn(q, k, v, 0, None, 0.3)
    # weight 1 on the one row: the value at the contract's 2^-14 fixed point
    vv = cpvo.f16_bits_to_f32(v)[0]
    want = (np.rint(vv.astype(np.float64) * 2.0 ** 14) * 2.0 ** -14).astype(np.float32)
    assert np.array_equal(out[0, :D], want) and np.array_equal(out[0, D:], want)

