"""Pins of the oracle's fp16 conversions (cpp/quant.hpp:73-100, :102-135).

The narrowing is checked against an independent closed form (numpy's
round-to-nearest-even with exact ties moved away from zero, fp32 subnormals
flushed to signed zero, NaN -> sign|0x7E00) over every sign/exponent/top-10
mantissa pattern with the rounding-relevant low bits, and exhaustively over the
fp16-subnormal band; and bit for bit against the reference's own
fp32_to_fp16 on all 2^32 inputs where the reference harness is built.
"""
import numpy as np
import pytest

import oracle as O


@np.errstate(invalid="ignore", over="ignore")
def closed_form_f32_to_f16(bits):
    """Reference rounding restated from the IEEE view: nearest, ties away."""
    bits = np.asarray(bits, dtype=np.uint32)
    x = bits.view(np.float32)
    sign = ((bits >> 16) & 0x8000).astype(np.uint16)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16)  # RNE
    hb = h.view(np.uint16)
    x64 = x.astype(np.float64)
    r64 = h.astype(np.float64)
    # neighbour away from zero of the RNE result (one fp16 ulp further out)
    away = (hb & 0x7FFF).astype(np.int64) + 1
    away_val = (away.astype(np.uint16)).view(np.float16).astype(np.float64)
    away_val = np.where(x < 0, -away_val, away_val)
    finite = np.isfinite(r64) & np.isfinite(x64) & np.isfinite(away_val)
    half_gap = np.abs(away_val - r64) / 2
    tie = finite & (np.abs(x64 - r64) == half_gap) & (np.abs(r64) < np.abs(x64))
    out = np.where(tie, (away.astype(np.uint16) | sign), hb).astype(np.uint16)
    be = (bits >> 23) & 0xFF
    out = np.where(be == 0, sign, out)  # fp32 zero / subnormal -> signed zero
    nan = (be == 0xFF) & ((bits & 0x7FFFFF) != 0)
    out = np.where(nan, sign | 0x7E00, out)
    return out.astype(np.uint16)


def test_widen_exhaustive_matches_ieee():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.fp16_to_fp32(h).view(np.uint32)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)


def test_narrow_closed_form_structured_exhaustive():
    # every sign x exponent x top-10-mantissa pattern, low 13 bits at the
    # rounding decision points
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    lows = np.array([0, 1, 0x0FFF, 0x1000, 0x1001, 0x1FFF, 0x0800, 0x17FF], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).reshape(-1)
    got = O.fp32_to_fp16(bits.view(np.float32))
    want = closed_form_f32_to_f16(bits)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first bits {bits[bad[0]]:#010x}: {got[bad[0]]:#06x} vs {want[bad[0]]:#06x}"


def test_narrow_closed_form_subnormal_band():
    # fp32 exponents 101..113 cover results from 0 through the fp16 subnormals
    # to the smallest normals: all 2^23 mantissas at the band's edges (101,
    # 102, 112, 113), 2^20 random mantissas (both signs) at the others
    rng = np.random.default_rng(5)
    for be in range(101, 114):
        if be in (101, 102, 112, 113):
            mant = np.arange(1 << 23, dtype=np.uint32)
            sign = np.zeros(mant.size, dtype=np.uint32)
        else:
            mant = rng.integers(0, 1 << 23, size=1 << 20, dtype=np.uint32)
            sign = rng.integers(0, 2, size=mant.size, dtype=np.uint32)
        bits = (sign << np.uint32(31)) | (np.uint32(be) << np.uint32(23)) | mant
        got = O.fp32_to_fp16(bits.view(np.float32))
        want = closed_form_f32_to_f16(bits)
        assert np.array_equal(got, want), f"exponent {be}"


def test_narrow_special_values():
    f = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65519.99, 65520.0, 1e-8, -1e-8,
                  2.0 ** -25, 2.0 ** -24, 2.0 ** -14, 1.0, -2.5, 1.00048828125], dtype=np.float32)
    got = O.fp32_to_fp16(f)
    want = [0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x7BFF, 0x7BFF, 0x7C00, 0x0000, 0x8000,
            0x0001, 0x0001, 0x0400, 0x3C00, 0xC100, 0x3C01]
    assert [int(x) for x in got] == want


def test_ties_round_away_unlike_rne():
    # 1 + 2^-11 is exactly halfway between 1 and 1 + 2^-10: RNE keeps 1.0,
    # the reference rounds away to 0x3C01
    x = np.array([1.0 + 2.0 ** -11, -(1.0 + 2.0 ** -11), 1.0 + 3 * 2.0 ** -11], dtype=np.float32)
    assert [int(v) for v in O.fp32_to_fp16(x)] == [0x3C01, 0xBC01, 0x3C02]
    assert int(x[:1].astype(np.float16).view(np.uint16)[0]) == 0x3C00


@pytest.mark.skipif(not O.RefModel.available("B"), reason="reference harness not built (oracle/_ref)")
def test_narrow_matches_reference_on_all_2_32_inputs():
    R = O.RefModel.load("B")
    chunk = 1 << 27
    for c in range((1 << 32) // chunk):
        a = O.fp32_bits_to_fp16(c * chunk, chunk, 8)
        b = np.empty(chunk, np.uint16)
        R.ref_fp32_bits_to_fp16_range(c * chunk, chunk, b)
        assert np.array_equal(a, b), f"chunk {c}"


@pytest.mark.skipif(not O.RefModel.available("B"), reason="reference harness not built (oracle/_ref)")
def test_widen_matches_reference_exhaustive():
    R = O.RefModel.load("B")
    ref = np.empty(65536, np.float32)
    R.ref_fp16_to_fp32_all(ref)
    got = O.fp16_to_fp32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
