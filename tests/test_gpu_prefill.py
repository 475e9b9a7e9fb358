"""Prefill parity on the GPU: causal MFMA flash attention and the batched
append against the oracle's token loop (cpp/model.hpp:493-593)."""
import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads
from gpu_util import assert_bits_equal, assert_close

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402
from picolm_qwen_amd._lib import PQA_ERR_ARG, PQAError, check, lib  # noqa: E402

pytestmark = pytest.mark.gpu

# name, n_heads, n_kv, head_dim, max_seq_len, rope_style, rope_base, qk_norm, start, n_tok, history_outliers
# Every case runs in the default precision (q as fp16 hi + lo). The cases
# without outliers also run with one fp16 q; with x8 outlier rows in the
# history a single fp16 rounding of q moves those scores by ~1e-2.
CASES = [
    ("qwen3_4b_s256", 32, 8, 128, 256, 0, 1e6, True, 0, 256, 0.0),
    ("qwen3_4b_start37_n200", 32, 8, 128, 512, 0, 1e6, True, 37, 200, 0.0),
    ("tinyllama_block8_n1", 32, 4, 64, 64, 1, 1e4, False, 0, 1, 0.0),
    ("tinyllama_block8_n129", 32, 4, 64, 256, 1, 1e4, False, 5, 129, 0.0),
    ("qwen25_g7_n100", 14, 2, 64, 512, 0, 1e6, False, 300, 100, 0.01),
    ("g2_n77", 16, 8, 128, 128, 0, 1e6, True, 0, 77, 0.0),
    ("g16_n40", 32, 2, 128, 128, 2, 1e4, True, 10, 40, 0.0),
    ("g1_interleaved_n65", 4, 4, 64, 96, 2, 1e4, False, 0, 65, 0.0),
    ("block8_hd128_splitq_n150", 16, 4, 128, 200, 1, 1e4, True, 3, 150, 0.01),
    ("interleaved_hd64_splitq_n130", 8, 2, 64, 160, 2, 1e4, True, 0, 130, 0.01),
    # Llama-3.2-1B heads: 8 KV heads at hd 64, 1200 rows in 10 row blocks
    ("llama32_1b_hd64_start20_n300", 32, 8, 64, 512, 0, 5e5, False, 20, 300, 0.0),
    # 4000 rows in 32 row blocks behind a 50-row history
    ("qwen3_4b_start50_n1000", 32, 8, 128, 1100, 0, 1e6, True, 50, 1000, 0.0),
]


def _prefill_case(idx, nh, nkv, hd, smax, style, base, qk, start, n_tok, prob, split_q=None,
                  norm_scale=1.0):
    """split_q None keeps the library's default precision; norm_scale
    multiplies the QK-norm weights (trained ones are not pinned near 1)."""
    seed = 9000 + idx
    kvd = nkv * hd
    cos, sin = O.rope_table(base, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, style, rope_cos=cos, rope_sin=sin)
    if split_q is not None:
        att.set_prefill_precision(split_q)
    qn = kn = None
    if qk:
        qn, kn = O.qk_norm_weights(seed, 0, hd)
        qn, kn = (qn * norm_scale).astype(np.float32), (kn * norm_scale).astype(np.float32)
        att.set_qk_norm(0, qn, kn)
    kc = np.zeros((smax, kvd), np.uint16)
    vc = np.zeros((smax, kvd), np.uint16)
    if start:
        att.synth_kv(0, 0, start, seed, prob)
        kc[:start], vc[:start] = O.synth_kv_rows(seed, 0, kvd, 0, start, prob, cpu_threads())
    q, k, v = O.batch_inputs(seed, 0, 0, n_tok, nh, nkv, hd)
    dev = torch.device("cuda:0")
    out = att.forward_batch(0, start, *(torch.from_numpy(x).to(dev) for x in (q, k, v)))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    shp = O.shape(nh, nkv, hd, smax, style)
    want = O.prefill(shp, start, q, k, v, qn, kn, cos, sin, kc, vc, serial=False, n_threads=cpu_threads())
    gk, gv = att.kv_download(0, start, n_tok)
    assert_bits_equal(gk, kc[start:start + n_tok], "appended K rows")
    assert_bits_equal(gv, vc[start:start + n_tok], "appended V rows")
    err = assert_close(got, want)
    att.close()
    return err


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_prefill_matches_oracle(case):
    print(f"prefill case {case[0]}", flush=True)
    _prefill_case(CASES.index(case), *case[1:])


FP16_Q_CASES = [c for c in CASES if c[-1] == 0.0]


@pytest.mark.parametrize("case", FP16_Q_CASES, ids=[c[0] for c in FP16_Q_CASES])
def test_prefill_fp16_q_mode_matches_oracle(case):
    print(f"prefill fp16-q case {case[0]}", flush=True)
    _prefill_case(CASES.index(case), *case[1:], split_q=False)


@pytest.mark.parametrize("scale", [2.0, 3.0])
def test_prefill_default_with_large_qk_norm_weights(scale):
    # QK-norm weights scaled by 2-3 scale every score by 4-9: the default hi + lo
    # q stays inside the tolerance (one fp16 q misses it from a scale of about 2)
    print(f"prefill qk-norm weights x{scale}", flush=True)
    _prefill_case(60, 32, 8, 128, 300, 0, 1e6, True, 20, 250, 0.0, norm_scale=scale)


def test_prefill_to_last_table_row_without_qk_norm():
    # Same regression as the decode test: the prompt ends on the last row of
    # a table that ends on an allocation boundary, no QK-norm.
    print("prefill to last row, no qk-norm", flush=True)
    _prefill_case(41, 16, 8, 128, 65536, 0, 1e6, False, 65536 - 300, 300, 0.0)


def test_prefill_precision_setting_values():
    # 1 (hi + lo, the default) and 0 (one fp16 q) are the modes; anything else is refused
    att = PicoAttention(1, 16, 4, 2, 64)
    for mode in (False, True):
        att.set_prefill_precision(mode)
    with pytest.raises(PQAError) as e:
        check(lib().pqa_set_prefill_precision(att.handle, 2), att.handle)
    assert e.value.code == PQA_ERR_ARG
    att.close()


def test_prefill_split_q_mode_set_explicitly():
    print("prefill split-q mode set explicitly", flush=True)
    _prefill_case(40, 32, 8, 128, 300, 0, 1e6, True, 20, 250, 0.0, split_q=True)


def test_prefill_row_equals_decode():
    # causal prefill row i == decode at pos start+i over the same cache
    nh, nkv, hd, smax, n = 16, 8, 128, 256, 150
    cos, sin = O.rope_table(1e6, hd, smax)
    qn, kn = O.qk_norm_weights(3, 0, hd)
    q, k, v = O.batch_inputs(3, 0, 0, n, nh, nkv, hd)
    dev = torch.device("cuda:0")
    a = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    a.set_qk_norm(0, qn, kn)
    pre = a.forward_batch(0, 0, *(torch.from_numpy(x).to(dev) for x in (q, k, v)))
    b = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    b.set_qk_norm(0, qn, kn)
    dec = []
    for i in range(n):
        dec.append(b.forward(0, i, q[i], k[i], v[i]))
    torch.cuda.synchronize()
    pre = pre.cpu().numpy()
    assert_close(pre, np.stack(dec), atol=2e-3, rtol=1e-2, what="prefill vs decode")
    ka, va = a.kv_download(0, 0, n)
    kb, vb = b.kv_download(0, 0, n)
    assert_bits_equal(ka, kb, "K rows prefill vs decode")
    assert_bits_equal(va, vb, "V rows prefill vs decode")
    a.close()
    b.close()


def test_prefill_successive_launches_append_every_row():
    # two layers, the prompt in two chunks per layer with the layers
    # interleaved (Qwen3-4B heads): every launch appends all of its rows,
    # bit-equal to the oracle's, and its outputs, which read the previous
    # chunk's rows as history, are within the tolerance
    print("prefill successive launches", flush=True)
    nh, nkv, hd, smax, seed = 32, 8, 128, 640, 9100
    kvd = nkv * hd
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(2, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    norms = [O.qk_norm_weights(seed, layer, hd) for layer in range(2)]
    for layer in range(2):
        att.set_qk_norm(layer, *norms[layer])
    kc = np.zeros((2, smax, kvd), np.uint16)
    vc = np.zeros_like(kc)
    shp = O.shape(nh, nkv, hd, smax, 0)
    dev = torch.device("cuda:0")
    for start, n in ((0, 256), (256, 344)):
        for layer in range(2):
            q, k, v = O.batch_inputs(seed, layer, start, n, nh, nkv, hd)
            out = att.forward_batch(layer, start, *(torch.from_numpy(x).to(dev) for x in (q, k, v)))
            torch.cuda.synchronize()
            want = O.prefill(shp, start, q, k, v, *norms[layer], cos, sin, kc[layer], vc[layer],
                             n_threads=cpu_threads())
            gk, gv = att.kv_download(layer, start, n)
            assert_bits_equal(gk, kc[layer, start:start + n], f"K rows layer {layer} from {start}")
            assert_bits_equal(gv, vc[layer, start:start + n], f"V rows layer {layer} from {start}")
            assert_close(out.cpu().numpy(), want, what=f"layer {layer} from {start}")
    att.close()
