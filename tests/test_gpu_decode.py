"""Decode parity on the GPU: libpqa.so against the CPU oracle on identical
seeded inputs. K/V rows bit-exact, attention output within
max-abs 2e-3 / rel 1e-2."""
import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads
from gpu_util import assert_bits_equal, assert_close

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu

# name, n_heads, n_kv, head_dim, max_seq_len, rope_style, rope_base, qk_norm, pos, outlier_prob
CASES = [
    ("tinyllama_block8_pos511", 32, 4, 64, 512, 1, 1e4, False, 511, 0.0),
    ("qwen25_pos0", 14, 2, 64, 64, 0, 1e6, False, 0, 0.0),
    ("qwen25_pos1", 14, 2, 64, 64, 0, 1e6, False, 1, 0.0),
    ("qwen25_pos77", 14, 2, 64, 128, 0, 1e6, False, 77, 0.0),
    ("qwen3_1p7b_pos1000", 16, 8, 128, 1024, 0, 1e6, True, 1000, 0.0),
    # per-column splits of 128 rows; the owner split holds 40 rows, so the
    # wave that adds the new row after its own rows (wave 3) has none
    ("qwen25_pos936_idle_late_writer", 14, 2, 64, 1024, 0, 1e6, True, 936, 0.0),
    # whole-row workgroups of 4 columns x 2 waves, 32-row splits; the owner
    # split's first waves add the new row after their 16 rows
    ("qwen3_1p7b_pos2000_whole_rows", 16, 8, 128, 2048, 0, 1e6, True, 2000, 0.0),
    ("qwen3_8b_outliers_pos4095", 32, 8, 128, 4096, 0, 1e6, True, 4095, 0.01),
    ("g16_two_chunks", 32, 2, 128, 600, 0, 1e6, True, 555, 0.0),
    ("interleaved_g1", 8, 8, 64, 300, 2, 1e4, False, 299, 0.0),
    ("block8_g3_qknorm", 12, 4, 128, 200, 1, 1e4, True, 150, 0.0),
    ("g5_pos_65", 10, 2, 64, 100, 0, 1e6, True, 65, 0.0),
    ("two_column_groups", 32, 16, 64, 400, 0, 1e6, False, 333, 0.0),
    # whole-row workgroups whose column count is not a power of two: 3
    # columns x 2 waves (waves 6, 7 idle), and 5 columns x 1 wave
    ("whole_rows_three_columns", 6, 3, 128, 4096, 0, 1e6, True, 4000, 0.0),
    ("whole_rows_five_columns", 20, 5, 64, 2048, 0, 1e6, False, 2000, 0.0),
]


def _decode_case(idx, nh, nkv, hd, smax, style, base, qk, pos, prob, split=0):
    seed = 7000 + idx
    kvd = nkv * hd
    cos, sin = O.rope_table(base, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, style, rope_cos=cos, rope_sin=sin)
    if split:
        att.set_decode_split(split)
    qn = kn = None
    if qk:
        qn, kn = O.qk_norm_weights(seed, 0, hd)
        att.set_qk_norm(0, qn, kn)
    att.synth_kv(0, 0, pos, seed, prob)
    kh, vh = O.synth_kv_rows(seed, 0, kvd, 0, pos, prob, cpu_threads())
    if pos:
        gk, gv = att.kv_download(0, 0, pos)
        assert_bits_equal(gk, kh, "synthetic K history")
        assert_bits_equal(gv, vh, "synthetic V history")
    q, k, v = O.step_inputs(seed, 0, 0, nh, nkv, hd)
    dev = torch.device("cuda:0")
    out = att.forward(0, pos, torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                      torch.from_numpy(v).to(dev))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kc = np.zeros((smax, kvd), np.uint16)
    vc = np.zeros((smax, kvd), np.uint16)
    kc[:pos], vc[:pos] = kh, vh
    shp = O.shape(nh, nkv, hd, smax, style)
    want = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc, cpu_threads())
    rk, rv = att.kv_download(0, pos, 1)
    assert_bits_equal(rk[0], kc[pos], "appended K row")
    assert_bits_equal(rv[0], vc[pos], "appended V row")
    err = assert_close(got, want)
    att.close()
    return err


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(case):
    idx = CASES.index(case)
    print(f"decode case {case[0]}", flush=True)
    _decode_case(idx, *case[1:])


@pytest.mark.parametrize("split", [64, 128, 576])
def test_decode_split_sizes(split):
    # same answer for any split of the history (up to fp32 summation order)
    print(f"decode split {split}", flush=True)
    _decode_case(50, 16, 8, 128, 2048, 0, 1e6, True, 2000, 0.0, split=split)


def test_last_table_row_without_qk_norm():
    # Regression: with no QK-norm the kernel once loaded its placeholder norm
    # weights from the RoPE row at pos, reading past the end of the table when
    # pos == max_seq_len - 1 and the table ends on an allocation boundary.
    print("decode last row, no qk-norm, 131072-entry table", flush=True)
    _decode_case(60, 16, 8, 128, 131072, 0, 1e6, False, 131071, 0.0)


def test_pos_ctx1_is_v_exactly():
    # ctx = 1: softmax of one row is 1, so out = fp16(v) exactly (cpp/model.hpp:387-413)
    nh, nkv, hd, smax = 8, 2, 128, 16
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    q, k, v = O.step_inputs(5, 0, 0, nh, nkv, hd)
    out = att.forward(0, 0, q, k, v)
    g = nh // nkv
    want = O.fp16_to_fp32(O.fp32_to_fp16(v)).reshape(nkv, hd)
    for h in range(nh):
        assert np.array_equal(out.reshape(nh, hd)[h], want[h // g])
    att.close()


def test_decode_host_and_device_paths_agree():
    nh, nkv, hd, smax, pos = 16, 8, 128, 512, 300
    cos, sin = O.rope_table(1e6, hd, smax)
    outs = []
    for host in (True, False):
        att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
        att.synth_kv(0, 0, pos, 11, 0.0)
        q, k, v = O.step_inputs(11, 0, 0, nh, nkv, hd)
        if host:
            outs.append(att.forward(0, pos, q, k, v))
        else:
            dev = torch.device("cuda:0")
            o = att.forward(0, pos, *(torch.from_numpy(x).to(dev) for x in (q, k, v)))
            torch.cuda.synchronize()
            outs.append(o.cpu().numpy())
        att.close()
    assert np.array_equal(outs[0], outs[1])


def test_decode_successive_positions():
    # One context, token after token: each call sees the rows the previous
    # calls appended, and the split partials of one call (written by the
    # split pass, read by the combine launch) never leak into the next.
    nh, nkv, hd, smax, pos0, n = 32, 4, 64, 640, 600, 6
    seed = 9100
    cos, sin = O.rope_table(1e4, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 1, rope_cos=cos, rope_sin=sin)
    att.synth_kv(0, 0, pos0, seed, 0.0)
    kh, vh = O.synth_kv_rows(seed, 0, nkv * hd, 0, pos0, 0.0, cpu_threads())
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros((smax, nkv * hd), np.uint16)
    kc[:pos0], vc[:pos0] = kh, vh
    shp = O.shape(nh, nkv, hd, smax, 1)
    for i in range(n):
        pos = pos0 + i
        print(f"decode successive pos {pos}", flush=True)
        q, k, v = O.step_inputs(seed, 0, i, nh, nkv, hd)
        got = att.forward(0, pos, q, k, v)
        want = O.attn_step(shp, pos, q, k, v, None, None, cos[pos], sin[pos], kc, vc, cpu_threads())
        assert_close(got, want)
    gk, gv = att.kv_download(0, pos0, n)
    assert_bits_equal(gk, kc[pos0:pos0 + n], "appended K rows")
    assert_bits_equal(gv, vc[pos0:pos0 + n], "appended V rows")
    att.close()
