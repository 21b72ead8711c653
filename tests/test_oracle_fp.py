"""Pins for the oracle's scalar contracts: fp16, exp, Philox, xoshiro."""
import decimal
import struct

import numpy as np
import pytest

from oracle import cpvo


def test_fp16_matches_numpy_on_sampled_bit_patterns():
    # every 97th float32 bit pattern plus the neighbourhoods of the fp16 edges
    bits = np.arange(0, 2**32, 97, dtype=np.uint64).astype(np.uint32)
    edges = []
    for v in [65504.0, 65519.0, 65520.0, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08, 1.0, 0.5]:
        b = np.array([v], dtype=np.float32).view(np.uint32)[0]
        edges.append(np.arange(int(b) - 4096, int(b) + 4096, dtype=np.int64).astype(np.uint32))
    bits = np.concatenate([bits] + edges + [e | np.uint32(0x80000000) for e in edges])
    x = bits.view(np.float32)
    ours = cpvo.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7C00) == 0x7C00) and np.all((ours[nan] & 0x3FF) != 0)


def test_fp16_to_fp32_all_patterns():
    h = np.arange(2**16, dtype=np.uint32).astype(np.uint16)
    ours = cpvo.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(ours[nan]))


def test_exp_table_is_2_pow_i_over_32():
    decimal.getcontext().prec = 60
    tab = cpvo.exp_table()
    for i in range(32):
        d = float(decimal.Decimal(2) ** (decimal.Decimal(i) / 32))
        u = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert int(tab[i]) == (u - (i << 47)) % 2**64


def test_expf_equals_libm_on_every_softmax_input():
    # softmax evaluates exp(l - max) <= 0, tempered or not: the whole negative
    # range down to underflow, every f32 bit pattern
    assert cpvo.expf_vs_libm(-110.0, 0.0, 1) == 0


def test_expf_equals_libm_on_positive_inputs():
    assert cpvo.expf_vs_libm(0.0, 89.0, 1) == 0


def test_expf_special_values():
    x = np.array([0.0, -0.0, -np.inf, np.inf, 1.0, -1.0, 88.72284, -104.0], dtype=np.float32)
    y = cpvo.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0 and y[2] == 0.0 and np.isinf(y[3])
    assert abs(y[4] - np.float32(np.e)) == 0 and y[7] == 0.0
    assert np.isinf(y[6])


def test_philox_matches_numpy_philox4x64():
    # numpy increments its 256-bit counter before each block, so
    # Philox(counter=c-1).random_raw(4) is the block at counter c
    for ctr, key in [((1, 2, 3, 4), (5, 6)), ((0, 0, 0, 0), (0, 0)),
                     ((2**64 - 1, 7, 2**63, 11), (2**64 - 3, 42)), ((0, 0, 9, 1), (1, 2))]:
        c = sum(int(v) << (64 * i) for i, v in enumerate(ctr))
        c = (c - 1) % 2**256
        prev = np.array([(c >> (64 * i)) & (2**64 - 1) for i in range(4)], dtype=np.uint64)
        bg = np.random.Philox(key=np.array(key, dtype=np.uint64), counter=prev)
        want = bg.random_raw(4)
        got = cpvo.philox4x64(ctr, key)
        assert [int(v) for v in got] == [int(v) for v in want]


def test_uniforms_are_24_bit_and_role_addressed():
    u = cpvo.philox_uniforms(1234, 3, 4)
    assert u.shape == (3, 5, 2)
    assert np.all(u >= 0) and np.all(u < 1)
    assert np.all((u * 2**24) == np.floor(u * 2**24))
    # a uniform depends only on (b, j, role), not on the batch it was drawn in
    u2 = cpvo.philox_uniforms(1234, 5, 4)
    assert np.array_equal(u, u2[:3])
    x = cpvo.philox4x64((2, 3, 1, 0), (1234, 0))
    assert u[2, 3, 1] == np.float32(int(x[0]) >> 40) / np.float32(2**24)
    # the round is the counter's last word: round r of seed s is not round 0
    # of another seed (a request keeps one key for all of its rounds)
    u7 = cpvo.philox_uniforms(1234, 3, 4, round=7)
    x7 = cpvo.philox4x64((2, 3, 1, 7), (1234, 0))
    assert u7[2, 3, 1] == np.float32(int(x7[0]) >> 40) / np.float32(2**24)
    assert not np.array_equal(u7, u) and not np.array_equal(u7, cpvo.philox_uniforms(1234 + 7, 3, 4))


def test_splitmix_seeding_known_answer():
    # splitmix64's first output from state 0 is 0xE220A8397B1DCDAF (Steele,
    # Lea, Flood 2014 reference generator); Rng::new(seed) mixes seed + 2*gamma
    gamma = 0x9E3779B97F4A7C15
    r = cpvo.Rng((-gamma) % 2**64)
    assert int(r.s[0]) == 0xE220A8397B1DCDAF


def test_xoshiro256pp_known_answer():
    # xoshiro256++ (Blackman & Vigna) from state {1, 2, 3, 4}: the first
    # output is rotl(1 + 4, 23) + 1, the state update is the published one
    r = cpvo.Rng(0)
    r.s[:] = np.array([1, 2, 3, 4], dtype=np.uint64)
    assert r.next_u64() == (5 << 23) + 1
    # s2 ^= s0, s3 ^= s1, s1 ^= s2, s0 ^= s3, s2 ^= s1_old << 17, s3 = rotl(s3, 45)
    assert [int(v) for v in r.s] == [7, 0, 2 ^ (2 << 17), 6 << 45]


def test_a_seed_reproduces_a_run():
    # crates/codpiece-sample/src/lib.rs:551-560 at the RNG level
    r1, r2, r3 = cpvo.Rng(42), cpvo.Rng(42), cpvo.Rng(43)
    s1 = [r1.next_f32() for _ in range(64)]
    s2 = [r2.next_f32() for _ in range(64)]
    s3 = [r3.next_f32() for _ in range(64)]
    assert s1 == s2 and s1 != s3


def test_next_f32_is_high_24_bits():
    r1, r2 = cpvo.Rng(7), cpvo.Rng(7)
    for _ in range(100):
        u = r1.next_u64()
        f = r2.next_f32()
        assert f == np.float32(u >> 40) / np.float32(2**24)
