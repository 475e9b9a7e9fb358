"""Pins of the oracle's attention loop (cpp/model.hpp:375-418) by closed forms
and float64 brute force, and of its prefill ordering (cpp/model.hpp:493-593)."""
import numpy as np

import oracle as O


def _cache(seed, s, kvd, pos, prob=0.0):
    kc = np.zeros((s, kvd), np.uint16)
    vc = np.zeros((s, kvd), np.uint16)
    kc[:pos], vc[:pos] = O.synth_kv_rows(seed, 0, kvd, 0, pos, prob, 4)
    return kc, vc


def test_ctx1_output_is_v():
    shp = O.shape(8, 2, 64, 8, 0)
    q, k, v = O.step_inputs(1, 0, 0, 8, 2, 64)
    kc, vc = _cache(1, 8, 128, 0)
    c, s = O.rope_rows(1e6, 64, 0, 1)
    out = O.attn_step(shp, 0, q, k, v, None, None, c[0], s[0], kc, vc)
    want = O.fp16_to_fp32(O.fp32_to_fp16(v)).reshape(2, 64)
    assert np.array_equal(out.reshape(8, 64), np.repeat(want, 4, axis=0))


def test_equal_keys_give_mean_of_values():
    shp = O.shape(4, 1, 64, 64, 0)
    kc, vc = _cache(2, 64, 64, 40)
    kc[:40] = kc[0]
    q = np.random.default_rng(0).standard_normal(4 * 64).astype(np.float32)
    out = O.attend(shp, 39, q, kc, vc)
    want = O.fp16_to_fp32(vc[:40]).astype(np.float64).mean(axis=0)
    assert np.allclose(out.reshape(4, 64), want, atol=2e-6)


def test_dominant_key_selects_its_value():
    shp = O.shape(2, 1, 64, 32, 0)
    kc, vc = _cache(3, 32, 64, 20)
    q = np.zeros(2 * 64, np.float32)
    q[:64] = 1.0
    q[64:] = 1.0
    kc[:20] = O.fp32_to_fp16(np.zeros(64, np.float32))
    kc[7] = O.fp32_to_fp16(np.full(64, 30.0, np.float32))  # score 30*64/8 = 240 above the rest
    out = O.attend(shp, 19, q, kc, vc)
    assert np.array_equal(out[:64], O.fp16_to_fp32(vc[7]))


def test_matches_float64_softmax():
    # tolerance: fp32 roundings of the scores (~1e-7 * hd * |q||k|) moved by
    # |v|; x8 outlier keys raise scores to ~24 and values to ~8
    for (nh, nkv, hd, pos, prob, atol) in [(8, 2, 64, 100, 0.0, 1e-5), (16, 8, 128, 300, 0.05, 5e-4),
                                           (6, 3, 128, 33, 0.0, 1e-5)]:
        shp = O.shape(nh, nkv, hd, pos + 1, 0)
        kc, vc = _cache(pos, pos + 1, nkv * hd, pos + 1, prob)
        q = np.random.default_rng(pos).standard_normal(nh * hd).astype(np.float32)
        out = O.attend(shp, pos, q, kc, vc)
        ref = O.attend_f64(shp, pos, q, kc, vc)
        assert np.allclose(out, ref, rtol=1e-4, atol=atol), np.abs(out - ref).max()


def test_thread_split_is_bit_identical():
    shp = O.shape(32, 8, 128, 600, 0)
    kc, vc = _cache(4, 600, 1024, 599, 0.01)
    q = np.random.default_rng(4).standard_normal(32 * 128).astype(np.float32)
    a = O.attend(shp, 599, q, kc, vc, n_threads=1)
    b = O.attend(shp, 599, q, kc, vc, n_threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_prefill_orders_agree_bitwise_and_rows_equal_decode():
    nh, nkv, hd, smax, start, n = 16, 4, 64, 128, 9, 50
    shp = O.shape(nh, nkv, hd, smax, 1)
    cos, sin = O.rope_table(1e4, hd, smax)
    qn, kn = O.qk_norm_weights(5, 0, hd)
    q, k, v = O.batch_inputs(5, 0, 0, n, nh, nkv, hd)
    kc1, vc1 = _cache(5, smax, nkv * hd, start)
    kc2, vc2 = kc1.copy(), vc1.copy()
    a = O.prefill(shp, start, q, k, v, qn, kn, cos, sin, kc1, vc1, serial=True, n_threads=1)
    b = O.prefill(shp, start, q, k, v, qn, kn, cos, sin, kc2, vc2, serial=False, n_threads=8)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)
    kc3, vc3 = _cache(5, smax, nkv * hd, start)
    for i in range(n):
        p = start + i
        o = O.attn_step(shp, p, q[i], k[i], v[i], qn, kn, cos[p], sin[p], kc3, vc3)
        assert np.array_equal(o.view(np.uint32), a[i].view(np.uint32))
