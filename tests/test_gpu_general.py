"""Head sizes other than 64 and 128 (the reference takes any head_dim up to
512, cpp/model.hpp:172): decode and prefill on the general kernels against the
oracle, with all three RoPE pairings (block8 with its interleaved tail, half
not a multiple of 4), QK-norm, GQA groups split into chunks, one or many key
ranges; appended K/V rows bit-exact, outputs within max-abs 2e-3 / rel 1e-2.
Also: the projections-to-attention entry points and the no-allocation decode
at such a size, and prefill row i equal to the decode at i."""
import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads
from gpu_util import assert_bits_equal, assert_close
from proj_cases import make_rows

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# name, n_heads, n_kv, head_dim, max_seq_len, rope_style, rope_base, qk_norm, pos, outlier_prob
DECODE = [
    ("hd80_neox_qknorm_pos700", 16, 4, 80, 1024, 0, 1e6, True, 700, 0.0),
    ("hd96_block8_pos33", 32, 8, 96, 64, 1, 1e4, True, 33, 0.0),
    ("hd100_block8_tail_pos300", 8, 2, 100, 512, 1, 1e4, True, 300, 0.0),
    ("hd256_neox_pos4000", 8, 2, 256, 4096, 0, 1e6, True, 4000, 0.01),
    ("hd512_interleaved_pos129", 4, 1, 512, 256, 2, 1e4, False, 129, 0.0),
    ("hd48_g12_chunks_pos0", 24, 2, 48, 16, 0, 1e6, True, 0, 0.0),
    ("hd2_pos70", 4, 2, 2, 128, 0, 1e4, False, 70, 0.0),
    ("hd72_long_pos20000", 16, 2, 72, 20480, 0, 1e6, False, 20000, 0.0),
]


def _context(nh, nkv, hd, smax, style, base, qk, seed):
    cos, sin = O.rope_table(base, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, style, rope_cos=cos, rope_sin=sin)
    qn = kn = None
    if qk:
        qn, kn = O.qk_norm_weights(seed, 0, hd)
        att.set_qk_norm(0, qn, kn)
    return att, cos, sin, qn, kn


@pytest.mark.parametrize("case", DECODE, ids=[c[0] for c in DECODE])
def test_general_decode_matches_oracle(case):
    name, nh, nkv, hd, smax, style, base, qk, pos, prob = case
    print(f"general decode {name}", flush=True)
    seed = 11000 + DECODE.index(case)
    kvd = nkv * hd
    att, cos, sin, qn, kn = _context(nh, nkv, hd, smax, style, base, qk, seed)
    att.synth_kv(0, 0, pos, seed, prob)
    kc = np.zeros((smax, kvd), np.uint16)
    vc = np.zeros_like(kc)
    kc[:pos], vc[:pos] = O.synth_kv_rows(seed, 0, kvd, 0, pos, prob, cpu_threads())
    q, k, v = O.step_inputs(seed, 0, 0, nh, nkv, hd)
    out = att.forward(0, pos, *(torch.from_numpy(x).to(DEV) for x in (q, k, v)))
    torch.cuda.synchronize()
    want = O.attn_step(O.shape(nh, nkv, hd, smax, style), pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc,
                       cpu_threads())
    rk, rv = att.kv_download(0, pos, 1)
    assert_bits_equal(rk[0], kc[pos], "appended K row")
    assert_bits_equal(rv[0], vc[pos], "appended V row")
    assert_close(out.cpu().numpy(), want)
    # the no-allocation decode runs the same kernels on its own scratch: same bits
    att.kv_upload(0, pos, np.zeros((1, kvd), np.uint16), np.zeros((1, kvd), np.uint16))
    o2 = torch.empty(nh * hd, dtype=torch.float32, device=DEV)
    att.forward_noalloc(0, pos, *(torch.from_numpy(x).to(DEV) for x in (q, k, v)), o2)
    assert_bits_equal(o2.cpu().numpy().view(np.uint32), out.cpu().numpy().view(np.uint32), "noalloc output")
    att.close()


# name, n_heads, n_kv, head_dim, max_seq_len, rope_style, rope_base, qk_norm, start, n_tok
PREFILL = [
    ("hd96_block8_n150", 32, 8, 96, 256, 1, 1e4, True, 0, 150),
    ("hd100_block8_tail_start40_n70", 8, 2, 100, 160, 1, 1e4, True, 40, 70),
    ("hd256_neox_start5_n64", 8, 2, 256, 128, 0, 1e6, True, 5, 64),
    ("hd80_interleaved_g12_n33", 24, 2, 80, 64, 2, 1e4, False, 0, 33),
]


@pytest.mark.parametrize("case", PREFILL, ids=[c[0] for c in PREFILL])
def test_general_prefill_matches_oracle(case):
    name, nh, nkv, hd, smax, style, base, qk, start, n_tok = case
    print(f"general prefill {name}", flush=True)
    seed = 12000 + PREFILL.index(case)
    kvd = nkv * hd
    att, cos, sin, qn, kn = _context(nh, nkv, hd, smax, style, base, qk, seed)
    kc = np.zeros((smax, kvd), np.uint16)
    vc = np.zeros_like(kc)
    if start:
        hk, hv = O.synth_kv_rows(seed, 0, kvd, 0, start, 0.0, cpu_threads())
        kc[:start], vc[:start] = hk, hv
        att.kv_upload(0, 0, hk, hv)
    q, k, v = O.batch_inputs(seed, 0, 0, n_tok, nh, nkv, hd)
    out = att.forward_batch(0, start, *(torch.from_numpy(x).to(DEV) for x in (q, k, v)))
    torch.cuda.synchronize()
    want = O.prefill(O.shape(nh, nkv, hd, smax, style), start, q, k, v, qn, kn, cos, sin, kc, vc,
                     n_threads=cpu_threads())
    assert_close(out.cpu().numpy(), want)
    gk, gv = att.kv_download(0, start, n_tok)
    assert_bits_equal(gk, kc[start:start + n_tok], "prefill K rows")
    assert_bits_equal(gv, vc[start:start + n_tok], "prefill V rows")
    att.close()


def test_general_prefill_row_equals_decode():
    # the last prompt row through pqa_prefill and the same token through
    # pqa_decode read the same cache rows: outputs equal to the tolerance and
    # the rows bit-equal
    print("general prefill row = decode", flush=True)
    nh, nkv, hd, smax, n = 12, 4, 96, 128, 90
    att, cos, sin, qn, kn = _context(nh, nkv, hd, smax, 0, 1e6, True, 5)
    q, k, v = O.batch_inputs(5, 0, 0, n, nh, nkv, hd)
    pre = att.forward_batch(0, 0, *(torch.from_numpy(x).to(DEV) for x in (q, k, v))).cpu().numpy()
    dec, _, _, _, _ = _context(nh, nkv, hd, smax, 0, 1e6, True, 5)
    gk, gv = att.kv_download(0, 0, n - 1)
    dec.kv_upload(0, 0, gk, gv)
    o = dec.forward(0, n - 1, *(torch.from_numpy(x[n - 1]).to(DEV) for x in (q, k, v))).cpu().numpy()
    assert_close(o, pre[n - 1])
    rk, rv = dec.kv_download(0, n - 1, 1)
    ak, av = att.kv_download(0, n - 1, 1)
    assert_bits_equal(rk, ak, "K row")
    assert_bits_equal(rv, av, "V row")
    att.close()
    dec.close()


def test_general_from_xb_paths():
    # head_dim 96 with Q8_0 projections: pqa_decode_x (projections bit-exact,
    # so the appended rows are too) against the oracle, and pqa_prefill_x (the
    # batched GEMM's scaled result read by the general prep kernel) bit-equal
    # to pqa_qkv_project_batch followed by pqa_prefill on a twin context
    print("general head_dim from xb", flush=True)
    rng = np.random.default_rng(96)
    nh, nkv, hd, dim, smax, n_tok = 16, 4, 96, 1024, 128, 50
    wt = O.GGUF_Q8_0
    wq, wk, wv = (make_rows(rng, wt, r, dim) for r in (nh * hd, nkv * hd, nkv * hd))
    ctxs = []
    for _ in range(2):
        att, cos, sin, qn, kn = _context(nh, nkv, hd, smax, 0, 1e6, True, 7)
        att.set_qkv_weights(0, dim, wq, wt, wk, wt, wv, wt)
        ctxs.append(att)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    a = ctxs[0].forward_batch_x(0, 0, torch.from_numpy(x).to(DEV)).cpu().numpy()
    qb, kb, vb = ctxs[1].qkv_project_batch(0, torch.from_numpy(x).to(DEV))
    b = ctxs[1].forward_batch(0, 0, qb, kb, vb).cpu().numpy()
    assert_bits_equal(a.view(np.uint32), b.view(np.uint32), "prefill_x vs project + prefill")
    ka, va = ctxs[0].kv_download(0, 0, n_tok)
    kb2, vb2 = ctxs[1].kv_download(0, 0, n_tok)
    assert_bits_equal(ka, kb2, "K rows")
    assert_bits_equal(va, vb2, "V rows")
    # one more token through pqa_decode_x, against the oracle from the same cache
    pos = n_tok
    xt = rng.standard_normal(dim).astype(np.float32)
    out = ctxs[0].forward_x(0, pos, torch.from_numpy(xt).to(DEV)).cpu().numpy()
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros_like(kc)
    kc[:pos], vc[:pos] = ka, va
    q = O.matmul_bias(xt, wq, wt, nh * hd)
    k = O.matmul_bias(xt, wk, wt, nkv * hd)
    v = O.matmul_bias(xt, wv, wt, nkv * hd)
    want = O.attn_step(O.shape(nh, nkv, hd, smax, 0), pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc)
    assert_close(out, want)
    rk, rv = ctxs[0].kv_download(0, pos, 1)
    assert_bits_equal(rk[0], kc[pos], "appended K row from xb")
    assert_bits_equal(rv[0], vc[pos], "appended V row from xb")
    for c in ctxs:
        c.close()
