"""Pins of the oracle's RMSNorm, RoPE, RoPE table and RNG.

RMSNorm (cpp/tensor.hpp:146-176) and RoPE (cpp/tensor.hpp:201-369) are pinned
bit for bit against the reference's own TensorOps where the reference harness
is built, and by closed forms everywhere: rms(out / w) == 1, rotation
preserves pair norms, pos 0 is the identity, a 90-degree table turns the
pairing into an index permutation (block8 KAT), interleaved == NeoX on the
de-interleaved vector.
"""
import numpy as np
import pytest

import oracle as O

HAVE_REF = O.RefModel.available("B")


def rng_vec(seed, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


@pytest.mark.parametrize("n", [64, 128, 4, 7, 13, 130])
def test_rmsnorm_closed_form(n):
    x = rng_vec(n, n, 3.0)
    w = (1 + 0.02 * rng_vec(n + 1, n)).astype(np.float32)
    out = O.rmsnorm(x, w)
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w64
    assert np.allclose(out, want, rtol=2e-6, atol=1e-7)
    r = out.astype(np.float64) / w64
    assert abs(np.sqrt(np.mean(r * r)) - 1.0) < 1e-5


@pytest.mark.skipif(not HAVE_REF, reason="reference harness not built")
@pytest.mark.parametrize("n", [64, 128, 4, 7, 13, 130])
def test_rmsnorm_matches_reference_bits(n):
    R = O.RefModel.load("B")
    for seed in range(20):
        x = rng_vec(1000 + seed, n, 2.0)
        w = (1 + 0.02 * rng_vec(2000 + seed, n)).astype(np.float32)
        ref = np.empty(n, np.float32)
        R.ref_rmsnorm(ref, x, w, n)
        assert np.array_equal(ref.view(np.uint32), O.rmsnorm(x, w).view(np.uint32))


def _angles(hd, pos, base):
    c, s = O.rope_rows(base, hd, pos, 1)
    return c[0], s[0]


@pytest.mark.parametrize("style", [0, 1, 2])
def test_rope_pos0_identity_and_norm_preserving(style):
    hd, nh, nkv = 128, 4, 2
    q, k = rng_vec(1, nh * hd), rng_vec(2, nkv * hd)
    c, s = _angles(hd, 0, 1e6)
    q2, k2 = O.rope(style, q, k, hd, nh, nkv, c, s)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)
    c, s = _angles(hd, 1234, 1e6)
    q2, _ = O.rope(style, q, k, hd, nh, nkv, c, s)
    # every element's partner: norms of the multiset of pairs are preserved
    assert np.isclose(np.sum(q2.astype(np.float64) ** 2), np.sum(q.astype(np.float64) ** 2), rtol=1e-5)


def test_rope_block8_permutation_kat():
    # cos = 0, sin = 1 turns each rotation into (x, y) -> (-y, x): the output
    # shows which element each position is paired with.
    hd = 24  # half = 12: three full blocks of 4 pairs, no tail
    x = np.arange(1, hd + 1, dtype=np.float32)
    c, s = np.zeros(hd // 2, np.float32), np.ones(hd // 2, np.float32)
    q2, _ = O.rope(1, x, np.zeros(hd, np.float32), hd, 1, 1, c, s)
    want = np.empty(hd, np.float32)
    for b in range(3):
        for j in range(4):
            e0, e1 = 8 * b + j, 8 * b + 4 + j
            want[e0], want[e1] = -x[e1], x[e0]
    assert np.array_equal(q2, want)
    # half = 10: two full blocks then an interleaved tail of 2 pairs
    hd = 20
    x = np.arange(1, hd + 1, dtype=np.float32)
    c, s = np.zeros(hd // 2, np.float32), np.ones(hd // 2, np.float32)
    q2, _ = O.rope(1, x, np.zeros(hd, np.float32), hd, 1, 1, c, s)
    want = np.empty(hd, np.float32)
    for b in range(2):
        for j in range(4):
            e0, e1 = 8 * b + j, 8 * b + 4 + j
            want[e0], want[e1] = -x[e1], x[e0]
    for i in (8, 9):
        want[2 * i], want[2 * i + 1] = -x[2 * i + 1], x[2 * i]
    assert np.array_equal(q2, want)


def test_rope_interleaved_equals_neox_on_deinterleaved_vector():
    hd = 64
    x = rng_vec(7, hd)
    c, s = _angles(hd, 77, 1e4)
    inter, _ = O.rope(2, x, np.zeros(hd, np.float32), hd, 1, 1, c, s)
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])  # (2i, 2i+1) -> (i, i+half)
    neox, _ = O.rope(0, x[perm], np.zeros(hd, np.float32), hd, 1, 1, c, s)
    assert np.array_equal(inter[perm], neox)


@pytest.mark.skipif(not HAVE_REF, reason="reference harness not built")
@pytest.mark.parametrize("qwen", [0, 1])
@pytest.mark.parametrize("hd", [64, 128, 20])
def test_rope_matches_reference_bits(qwen, hd):
    R = O.RefModel.load("B")
    nh, nkv = 3, 2
    for pos in (0, 1, 511, 4095):
        c, s = _angles(hd, pos, 1e6 if qwen else 1e4)
        q, k = rng_vec(pos + 1, nh * hd), rng_vec(pos + 2, nkv * hd)
        rq, rk = q.copy(), k.copy()
        R.ref_rope(qwen, rq, rk, hd, nh, nkv, c, s)
        oq, ok = O.rope(0 if qwen else 1, q, k, hd, nh, nkv, c, s)
        assert np.array_equal(rq.view(np.uint32), oq.view(np.uint32))
        assert np.array_equal(rk.view(np.uint32), ok.view(np.uint32))


def test_rope_table_closed_form():
    hd, base = 128, 1e6
    c, s = O.rope_table(base, hd, 64)
    i = np.arange(hd // 2)
    for pos in (0, 1, 63):
        theta = pos / np.power(base, 2.0 * i / hd)
        assert np.allclose(c[pos], np.cos(theta), atol=2e-6)
        assert np.allclose(s[pos], np.sin(theta), atol=2e-6)
    assert np.array_equal(c[0], np.ones(hd // 2, np.float32)) and np.array_equal(s[0], np.zeros(hd // 2, np.float32))
    rows_c, rows_s = O.rope_rows(base, hd, 17, 5)
    assert np.array_equal(rows_c, c[17:22]) and np.array_equal(rows_s, s[17:22])


@pytest.mark.skipif(not HAVE_REF, reason="reference harness not built")
def test_rope_table_matches_reference_allocation():
    ref = O.RefModel(4, 2, 64, 512, 1e4, False, False, "B")
    rc, rs = ref.rope_rows(0, 512)
    ref.close()
    c, s = O.rope_table(1e4, 64, 512)
    assert np.array_equal(rc.view(np.uint32), c.view(np.uint32))
    assert np.array_equal(rs.view(np.uint32), s.view(np.uint32))


def test_splitmix64_published_sequence():
    # Vigna's splitmix64.c seeded with 1234567
    L = O.lib()
    got = [L.pqo_splitmix64(1234567, i) for i in range(5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def test_normal_generator_moments_and_counter_addressing():
    z = O.normal(9, O.KIND_Q, 0, 0, 1 << 20)
    assert abs(float(z.mean())) < 5e-3 and abs(float(z.std()) - 1.0) < 5e-3
    assert abs(float(np.mean(z.astype(np.float64) ** 4)) - 3.0) < 0.05
    # value i is addressable on its own (counter-based), as the GPU fill needs
    assert np.array_equal(O.normal(9, O.KIND_Q, 0, 777, 10), z[777:787])


def test_synth_rows_outliers_and_rounding():
    k, v = O.synth_kv_rows(3, 5, 64, 0, 4000, 0.01, 4)
    flags = np.array([O.lib().pqo_is_outlier(3, 5, p, 0.01) for p in range(4000)])
    assert 15 < flags.sum() < 70
    kf = O.fp16_to_fp32(k).astype(np.float64)
    assert np.abs(kf[flags == 1]).mean() > 5 * np.abs(kf[flags == 0]).mean()
    z = O.normal(3, O.KIND_KHIST, 5, 0, 4000 * 64).reshape(4000, 64)
    z[flags == 1] *= 8.0
    assert np.array_equal(k, O.fp32_to_fp16(z))
    k2, _ = O.synth_kv_rows(3, 5, 64, 1000, 50, 0.01, 1)
    assert np.array_equal(k2, k[1000:1050])
