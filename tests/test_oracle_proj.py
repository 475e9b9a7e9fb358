"""The projection oracle (oracle/pqa_oracle_proj.c, restating matmul_bias,
vec_dot and dequantize_row of cpp/tensor.hpp:110-143 and cpp/quant.hpp:176-358)
pinned two ways: bit-equal to the reference's own functions
(oracle/_ref/libref_B.so, compiled without FMA contraction) on every type,
shape class and special scale, and the block formats' closed forms (hand-built
blocks whose values are known integers)."""
import numpy as np
import pytest

import oracle as O
from proj_cases import make_bias, make_rows

TYPES = [O.GGUF_F32, O.GGUF_F16, O.GGUF_Q4_0, O.GGUF_Q8_0, O.GGUF_Q4_K, O.GGUF_Q6_K]
needs_ref = pytest.mark.skipif(not O.RefModel.available("B"), reason="oracle/_ref not built")


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@needs_ref
@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("n", [512, 1536, 4096])
def test_matmul_bias_equals_reference(wtype, n):
    rng = np.random.default_rng(1000 * wtype + n)
    rows = 48
    w = make_rows(rng, wtype, rows, n, special=True)
    x = rng.standard_normal(n).astype(np.float32)
    ref = O.RefProj()
    for btype in (O.GGUF_NONE, O.GGUF_F32, O.GGUF_F16):
        b = None if btype == O.GGUF_NONE else make_bias(rng, btype, rows)
        ours = O.matmul_bias(x, w, wtype, rows, b, btype)
        theirs = ref.matmul_bias(x, w, wtype, rows, b, btype)
        assert bits_equal(ours, theirs), (wtype, n, btype)


@needs_ref
@pytest.mark.parametrize("wtype", TYPES)
def test_dequant_equals_reference(wtype):
    rng = np.random.default_rng(7 + wtype)
    n = 1024
    w = make_rows(rng, wtype, 8, n, special=True)
    ref = O.RefProj()
    for r in range(8):
        assert bits_equal(O.dequant_row(wtype, w[r], n), ref.dequant_row(wtype, w[r], n)), (wtype, r)


@needs_ref
def test_fma_build_differs_only_in_rounding():
    # The shipped flags (build A) may contract d1*q - m1 and the dot products
    # into FMAs; the difference stays at rounding level.
    rng = np.random.default_rng(3)
    n, rows = 4096, 64
    w = make_rows(rng, O.GGUF_Q4_K, rows, n)
    x = rng.standard_normal(n).astype(np.float32)
    a = O.RefProj("A").matmul_bias(x, w, O.GGUF_Q4_K, rows)
    b = O.matmul_bias(x, w, O.GGUF_Q4_K, rows)
    assert np.max(np.abs(a - b)) <= 1e-4 * np.max(np.abs(b))


def f16(v):
    return np.array([v], "<f2").view(np.uint8)


def test_closed_form_q8_0_and_q4_0():
    # d = 2: Q8_0 values are 2 q, Q4_0 values are 2 (nibble - 8)
    q = np.arange(-16, 16, dtype=np.int8)
    blk8 = np.concatenate([f16(2.0), q.view(np.uint8)])
    assert np.array_equal(O.dequant_row(O.GGUF_Q8_0, blk8, 32), 2.0 * q.astype(np.float32))
    nib = np.arange(32) % 16
    packed = (nib[:16] | (nib[16:] << 4)).astype(np.uint8)
    blk4 = np.concatenate([f16(2.0), packed])
    assert np.array_equal(O.dequant_row(O.GGUF_Q4_0, blk4, 32), 2.0 * (nib - 8).astype(np.float32))


def test_closed_form_q4_k():
    # d = 1, dmin = 0.5, sub-block j with scale j + 1 and min 2 j: y = (j+1) q - j
    sc = [j + 1 for j in range(8)]
    mn = [2 * j for j in range(8)]
    s12 = np.zeros(12, np.uint8)
    for j in range(4):
        s12[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s12[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s12[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    q = np.arange(256) % 16
    qs = np.zeros(128, np.uint8)
    for jj in range(4):  # 32 bytes per 64 elements: low nibbles first 32, high nibbles next 32
        lo, hi = q[64 * jj:64 * jj + 32], q[64 * jj + 32:64 * jj + 64]
        qs[32 * jj:32 * jj + 32] = lo | (hi << 4)
    blk = np.concatenate([f16(1.0), f16(0.5), s12, qs])
    y = O.dequant_row(O.GGUF_Q4_K, blk, 256)
    want = np.array([sc[e // 32] * q[e] - 0.5 * mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_q4k_term_magnitudes_closed_form_and_limits():
    # the closed-form block above: |d q| + |m| = (j+1) q + j for sub-block j
    sc = [j + 1 for j in range(8)]
    mn = [2 * j for j in range(8)]
    s12 = np.zeros(12, np.uint8)
    for j in range(4):
        s12[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s12[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s12[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    q = np.arange(256) % 16
    qs = np.zeros(128, np.uint8)
    for jj in range(4):
        lo, hi = q[64 * jj:64 * jj + 32], q[64 * jj + 32:64 * jj + 64]
        qs[32 * jj:32 * jj + 32] = lo | (hi << 4)
    blk = np.concatenate([f16(1.0), f16(0.5), s12, qs])
    got = O.q4k_term_magnitudes(blk[None, :], 256)[0]
    want = np.array([sc[e // 32] * q[e] + 0.5 * mn[e // 32] for e in range(256)], np.float64)
    assert np.array_equal(got, want)
    # random rows against the dequantization: |d q| + |m| >= |w|; equal to |w|
    # when d = 0 (w = -m) and, up to w's fp32 rounding, when dmin = 0 (w = d q)
    rng = np.random.default_rng(77)
    n = 512
    raw = make_rows(rng, O.GGUF_Q4_K, 6, n).reshape(6, n // 256, 144).copy()
    raw[0:2, :, 0:2] = 0   # d = +0
    raw[2:4, :, 2:4] = 0   # dmin = +0
    raw = raw.reshape(6, -1)
    mag = O.q4k_term_magnitudes(raw, n)
    w = np.abs(np.stack([O.dequant_row(O.GGUF_Q4_K, raw[r], n) for r in range(6)]).astype(np.float64))
    assert np.array_equal(mag[0:2], w[0:2])
    assert np.all(np.abs(mag[2:4] - w[2:4]) <= 2.0 ** -24 * w[2:4])
    assert np.all(mag >= w * (1 - 2.0 ** -24))
    assert np.any(mag[4:] > 1.5 * w[4:])  # the general rows do carry cancelling terms


def test_closed_form_q6_k():
    # d = 1, scales s_i = i - 8; 6-bit q from the low/high planes, y = s * (q - 32)
    q6 = (np.arange(256) * 7) % 64
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        for l in range(32):
            v = [q6[128 * h + 32 * quad + l] for quad in range(4)]
            ql[64 * h + l] = (v[0] & 0xF) | ((v[2] & 0xF) << 4)
            ql[64 * h + l + 32] = (v[1] & 0xF) | ((v[3] & 0xF) << 4)
            qh[32 * h + l] = (v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6)
    scales = (np.arange(16) - 8).astype(np.int8)
    blk = np.concatenate([ql, qh, scales.view(np.uint8), f16(1.0)])
    y = O.dequant_row(O.GGUF_Q6_K, blk, 256)
    # element e = 128 h + 32 quad + l uses scale index 8 h + l // 16 + 2 quad
    want = np.array([scales[8 * (e // 128) + (e % 32) // 16 + 2 * ((e % 128) // 32)] * (q6[e] - 32.0)
                     for e in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_sse2_order_is_the_one_restated():
    # Terms chosen so that the SSE2 grouping (8 lanes, then (t0+t2)+(t1+t3))
    # and a plain left-to-right sum give different floats.
    w = np.zeros(16, np.float32)
    w[0], w[1], w[5] = 1.0, 1e8, -1e8  # SSE2: lane 0 keeps the 1; in order it is absorbed by 1e8
    x = np.ones(16, np.float32)
    raw = w.view(np.uint8)
    got = O.vec_dot(O.GGUF_F32, raw, x)
    lanes = [w[l::8].astype(np.float32) for l in range(8)]
    acc = [np.float32(0)] * 8
    for l in range(8):
        for v in lanes[l]:
            acc[l] = np.float32(acc[l] + v)
    t = [np.float32(acc[l] + acc[l + 4]) for l in range(4)]
    want = np.float32(np.float32(t[0] + t[2]) + np.float32(t[1] + t[3]))
    seq = np.float32(0)
    for v in w:
        seq = np.float32(seq + v)
    assert got == want and want != seq


@pytest.mark.parametrize("wtype", TYPES)
def test_matmul_bias_tokens_equals_per_token_calls(wtype):
    # the threaded batched form (the prompt-path checker) gives, for every
    # token, the bits of the per-token matmul_bias pinned to the reference above
    rng = np.random.default_rng(4242 + wtype)
    rows, n, n_tok = 37, 512, 9
    w = make_rows(rng, wtype, rows, n, special=True)
    x = rng.standard_normal((n_tok, n)).astype(np.float32)
    for btype in (O.GGUF_NONE, O.GGUF_F32, O.GGUF_F16):
        b = None if btype == O.GGUF_NONE else make_bias(rng, btype, rows)
        for threads in (1, 4):
            got = O.matmul_bias_tokens(x, w, wtype, rows, b, btype, n_threads=threads)
            for t in range(n_tok):
                assert bits_equal(got[t], O.matmul_bias(x[t], w, wtype, rows, b, btype)), (wtype, btype, threads, t)
