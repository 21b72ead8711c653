"""Pins for the oracle's block formats and the exact-window GEMM contract."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import cpvo


def test_block_sizes_match_gguf():
    # crates/codpiece-gguf/src/lib.rs:545-550
    assert cpvo.row_bytes(cpvo.Q8_0, 32) == 34
    assert cpvo.row_bytes(cpvo.Q6_K, 512) == 420
    assert cpvo.row_bytes(cpvo.Q4_K, 256) == 144
    with pytest.raises(AssertionError):
        cpvo.row_bytes(cpvo.Q8_0, 33)


def test_mul_mat_convention_known_answer():
    # crates/codpiece-ggml-sys/tests/smoke.rs:18-43: A ne=[2,3], B ne=[2,2] -> [3,7,11,6,14,22]
    a = np.array([[1, 2], [3, 4], [5, 6]], dtype=np.float32)
    b = np.array([[1, 1], [2, 2]], dtype=np.float32)
    assert cpvo.mul_mat_f32(a, b).ravel().tolist() == [3, 7, 11, 6, 14, 22]


def test_qgemm_uses_the_same_convention():
    # small integer operands padded to one Q8_0 block: the weights quantize
    # exactly (amax 127), the activations carry ~1% Q8_0 rounding, which is
    # far below what a transposed layout would produce
    a = np.zeros((3, 32), dtype=np.float32)
    b = np.zeros((2, 32), dtype=np.float32)
    a[:, 0] = [127, -127, 127]
    a[:, 1] = [0, 127, -127]
    b[0, :2] = [1, 2]
    b[1, :2] = [-2, 1]
    w = cpvo.quantize(cpvo.Q8_0, a)
    y = cpvo.qgemm(cpvo.Q8_0, w, b)
    want = b @ a.T
    assert y.shape == (2, 3)
    np.testing.assert_allclose(y, want, rtol=1e-2)


@pytest.mark.parametrize("t", [cpvo.Q8_0, cpvo.Q4_K, cpvo.Q6_K])
def test_dequant_error_is_bounded_by_the_block_step(t):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 0.02, size=(8, 1024)).astype(np.float32)
    q = cpvo.quantize(t, x)
    y = cpvo.dequantize(t, q, 1024)
    err = np.abs(y - x)
    amax = np.abs(x).reshape(8, -1, 32).max(axis=2)
    # half a code step per 32 elements: range/15 (Q4_K), amax/31 (Q6_K),
    # amax/127 (Q8_0), plus the rounding of the 6-bit / int8 sub-scales, which
    # can push an edge element up to one full step away (clamped code); Q8_0
    # codes use the f32 scale but decode with its fp16 rounding: +127 * 2^-11.
    # A layout mistake (a misplaced high bit, a swapped nibble) costs >= 16 steps.
    step = {cpvo.Q8_0: amax / 127, cpvo.Q4_K: 2 * amax / 15, cpvo.Q6_K: amax / 31}[t]
    frac = {cpvo.Q8_0: 0.5 + 127 * 2.0**-11, cpvo.Q4_K: 0.75, cpvo.Q6_K: 2.0}[t]
    bound = np.repeat(step, 32, axis=1) * frac + 1e-7
    assert np.all(err <= bound), (err / bound).max()


def test_q8_0_extreme_element_maps_to_127():
    x = np.linspace(-3, 2, 32, dtype=np.float32)[None]
    q = cpvo.quantize(cpvo.Q8_0, x)[0]
    codes = q[2:].view(np.int8)
    assert codes[0] == -127 and codes.max() < 127
    d = np.frombuffer(q[:2].tobytes(), dtype=np.float16)[0]
    assert d == np.float16(np.float32(3) / np.float32(127))


def _parse_rows(t, w, K):
    """Independent numpy parse of the ggml layouts -> (ints, exact rationals)."""
    rb = cpvo.row_bytes(t, K)
    rows = []
    for r in range(w.shape[0]):
        row = w[r].tobytes()
        vals = []
        for b in range(len(row) // cpvo.SIZE[t]):
            blk = row[b * cpvo.SIZE[t]:(b + 1) * cpvo.SIZE[t]]
            if t == cpvo.Q8_0:
                d = Fraction(float(np.frombuffer(blk[:2], np.float16)[0]))
                q = np.frombuffer(blk[2:], np.int8)
                vals += [d * int(v) for v in q]
            elif t == cpvo.Q4_K:
                d = Fraction(float(np.frombuffer(blk[0:2], np.float16)[0]))
                dm = Fraction(float(np.frombuffer(blk[2:4], np.float16)[0]))
                s = blk[4:16]
                qs = blk[16:]
                sc, mn = [], []
                for j in range(8):
                    if j < 4:
                        sc.append(s[j] & 63)
                        mn.append(s[j + 4] & 63)
                    else:
                        sc.append((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4))
                        mn.append((s[j + 4] >> 4) | ((s[j] >> 6) << 4))
                codes = [0] * 256
                for c in range(4):
                    for l in range(32):
                        codes[c * 64 + l] = qs[c * 32 + l] & 0xF
                        codes[c * 64 + 32 + l] = qs[c * 32 + l] >> 4
                vals += [d * sc[e // 32] * codes[e] - dm * mn[e // 32] for e in range(256)]
            else:
                ql, qh = blk[:128], blk[128:192]
                sc = np.frombuffer(blk[192:208], np.int8)
                d = Fraction(float(np.frombuffer(blk[208:210], np.float16)[0]))
                codes = [0] * 256
                for h in range(2):
                    for l in range(32):
                        a, b2 = ql[h * 64 + l], ql[h * 64 + 32 + l]
                        hb = qh[h * 32 + l]
                        codes[h * 128 + l] = ((a & 0xF) | (((hb >> 0) & 3) << 4)) - 32
                        codes[h * 128 + 32 + l] = ((b2 & 0xF) | (((hb >> 2) & 3) << 4)) - 32
                        codes[h * 128 + 64 + l] = ((a >> 4) | (((hb >> 4) & 3) << 4)) - 32
                        codes[h * 128 + 96 + l] = ((b2 >> 4) | (((hb >> 6) & 3) << 4)) - 32
                vals += [d * int(sc[e // 16]) * codes[e] for e in range(256)]
        rows.append(vals)
    return rows


def _act_rationals(t, x):
    """ggml's activation quantization, restated independently in numpy f32."""
    out = []
    for row in x:
        vals = []
        if t == cpvo.Q8_0:
            for b in range(len(row) // 32):
                blk = row[b * 32:(b + 1) * 32].astype(np.float32)
                amax = np.float32(np.abs(blk).max())
                d = np.float32(amax / np.float32(127))
                idd = np.float32(1) / d if d != 0 else np.float32(0)
                v = (blk * idd).astype(np.float32)
                q = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))  # roundf: half away from 0
                dh = Fraction(float(np.float16(d)))
                vals += [dh * int(c) for c in q]
        else:
            for b in range(len(row) // 256):
                blk = row[b * 256:(b + 1) * 256].astype(np.float32)
                i = int(np.argmax(np.abs(blk)))
                mx = np.float32(blk[i])
                if mx == 0:
                    vals += [Fraction(0)] * 256
                    continue
                isc = np.float32(np.float32(-127) / mx)
                q = np.minimum(np.rint((isc * blk).astype(np.float32)), 127)
                d = Fraction(float(np.float32(np.float32(1) / isc)))
                vals += [d * int(c) for c in q]
        out.append(vals)
    return out


def _f32_rne(fr):
    """Round an exact rational to the nearest float32 (ties to even)."""
    if fr == 0:
        return np.float32(0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return np.float32(sign * float(fl * ulp))


@pytest.mark.parametrize("t,K", [(cpvo.Q8_0, 64), (cpvo.Q4_K, 512), (cpvo.Q6_K, 512)])
def test_qgemm_is_the_correctly_rounded_quantized_dot(t, K):
    # closed form: parse the blocks and the activation codes independently,
    # sum exactly with rationals, round once to f32
    rng = np.random.default_rng(7)
    N, M = 6, 3
    w = cpvo.quantize(t, rng.normal(0, 0.02, size=(N, K)).astype(np.float32))
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    y = cpvo.qgemm(t, w, x)
    W = _parse_rows(t, w, K)
    X = _act_rationals(t, x)
    for m in range(M):
        for n in range(N):
            exact = sum((a * b for a, b in zip(W[n], X[m])), Fraction(0))
            assert y[m, n] == _f32_rne(exact), (m, n, float(exact), y[m, n])


@pytest.mark.parametrize("t", [cpvo.Q8_0, cpvo.Q4_K, cpvo.Q6_K])
def test_qgemm_matches_f64_reference_at_verify_shapes(t):
    rng = np.random.default_rng(3)
    K, N, M = 5120, 64, 5
    w = cpvo.quantize(t, rng.normal(0, 0.02, size=(N, K)).astype(np.float32))
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    y = cpvo.qgemm(t, w, x)
    y64 = cpvo.qgemm_f64(t, w, x)
    # the f64 reference has ~1e-16 relative error; the contract rounds once,
    # after a sum whose grid error is ~1e-11 absolute at these scales (it shows
    # only on outputs that cancel to ~1e-5)
    ulp = np.spacing(np.abs(y64).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(y.astype(np.float64) - y64) <= ulp + 1e-10)
    assert np.mean(np.abs(y.astype(np.float64) - y64) <= ulp / 2) > 0.99


@pytest.mark.parametrize("t", [cpvo.Q8_0, cpvo.Q4_K, cpvo.Q6_K])
def test_qgemm_is_invariant_to_block_order(t):
    # exact integer accumulation: permuting the K blocks of both operands in
    # the same way must not change a single bit
    rng = np.random.default_rng(5)
    K, N, M = 2048, 16, 4
    blk = cpvo.BLOCK[t] if t != cpvo.Q8_0 else 32
    blk_q = 256 if t != cpvo.Q8_0 else 32
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    wf = rng.normal(0, 0.02, size=(N, K)).astype(np.float32)
    w = cpvo.quantize(t, wf)
    perm = rng.permutation(K // blk_q)
    xp = x.reshape(M, -1, blk_q)[:, perm].reshape(M, K)
    wp = w.reshape(N, -1, cpvo.SIZE[t])[:, perm].reshape(N, -1)
    assert np.array_equal(cpvo.qgemm(t, w, x).view(np.uint32), cpvo.qgemm(t, wp, xp).view(np.uint32))
    del blk


def test_qgemm_rows_are_independent():
    rng = np.random.default_rng(9)
    K, N = 1024, 32
    w = cpvo.quantize(cpvo.Q4_K, rng.normal(0, 0.02, size=(N, K)).astype(np.float32))
    x = rng.normal(0, 1, size=(5, K)).astype(np.float32)
    y = cpvo.qgemm(cpvo.Q4_K, w, x)
    for m in range(5):
        assert np.array_equal(cpvo.qgemm(cpvo.Q4_K, w, x[m:m + 1])[0], y[m])


def test_qgemm_zero_activation_row_gives_zero():
    rng = np.random.default_rng(2)
    w = cpvo.quantize(cpvo.Q6_K, rng.normal(0, 0.02, size=(8, 512)).astype(np.float32))
    x = np.zeros((2, 512), dtype=np.float32)
    x[1] = rng.normal(size=512)
    y = cpvo.qgemm(cpvo.Q6_K, w, x)
    assert np.all(y[0] == 0) and np.any(y[1] != 0)
