"""The prompt path's K and V projections in the reference's summation order
(pqa_exact.hip, the default of pqa_set_batch_projection): k and v from
pqa_qkv_project_batch bit-equal to the projection oracle (bit-equal to the
reference's matmul_bias, per token) for every weight type, bias type, partial
token / row / k tiles and unaligned inputs; the cache rows that pqa_prefill_x
writes byte-equal to the oracle's, at small shapes, at a general head size and
for a whole 2048-token prompt at Qwen3-4B widths (n_embd 2560, 32/8 heads,
head_dim 128), whose sampled outputs are also within max-abs 2e-3 / rel 1e-2."""
import numpy as np
import pytest

import oracle as O
from gpu_util import assert_bits_equal, assert_close
from proj_cases import make_bias, make_rows

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TYPES = [O.GGUF_F32, O.GGUF_F16, O.GGUF_Q4_0, O.GGUF_Q8_0, O.GGUF_Q4_K, O.GGUF_Q6_K]


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("wtype", TYPES)
def test_batch_kv_bit_exact_per_type(wtype):
    # 70 tokens (a full and a partial 64-token tile), kv_dim 192 (3 row tiles),
    # rows of 512 elements (8 k tiles); F32/F16 biases on k and v
    print(f"reference-order batch K/V, type {wtype}", flush=True)
    rng = np.random.default_rng(31000 + wtype)
    nh, nkv, hd, dim, n_tok = 6, 3, 64, 512, 70
    att = PicoAttention(1, 16, nh, nkv, hd)
    rows = (nh * hd, nkv * hd, nkv * hd)
    w = [make_rows(rng, wtype, r, dim, special=True) for r in rows]
    bt = (O.GGUF_NONE, O.GGUF_F32, O.GGUF_F16)
    b = [None, make_bias(rng, bt[1], rows[1]), make_bias(rng, bt[2], rows[2])]
    att.set_qkv_weights(0, dim, w[0], wtype, w[1], wtype, w[2], wtype, b[0], bt[0], b[1], bt[1], b[2], bt[2])
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    q, k, v = (g.cpu().numpy() for g in att.qkv_project_batch(0, torch.from_numpy(x).to(DEV)))
    for name, g, j in (("k", k, 1), ("v", v, 2)):
        want = O.matmul_bias_tokens(x, w[j], wtype, rows[j], b[j], bt[j])
        assert_bits_equal(_bits(g), _bits(want), f"{name} (type {wtype})")
    # q stays on the split GEMM, within its bound
    wf = np.stack([O.dequant_row(wtype, w[0][r], dim) for r in range(rows[0])]).astype(np.float64)
    wq = O.matmul_bias_tokens(x, w[0], wtype, rows[0])
    mag = np.abs(x.astype(np.float64)) @ np.abs(wf).T
    assert np.all(np.abs(q - wq) <= (4 * dim + 13) * 2.0 ** -24 * mag + 1e-30)
    att.close()


@pytest.mark.parametrize("wtype", [O.GGUF_F32, O.GGUF_Q8_0])
def test_batch_kv_padded_width_and_unaligned_input(wtype):
    # F32 rows of 104 elements (the last k tile 40 wide, zero products past the
    # row: +0 added to a chain leaves it unchanged); Q8_0 rows of 192 (six
    # blocks); inputs at a 4-byte offset take the scalar-load kernels and must
    # give the same bits
    print(f"reference-order batch K/V, padded width, type {wtype}", flush=True)
    rng = np.random.default_rng(32000 + wtype)
    nh, nkv, hd, n_tok = 4, 2, 64, 131
    dim = 104 if wtype == O.GGUF_F32 else 192
    att = PicoAttention(1, 16, nh, nkv, hd)
    rows = (nh * hd, nkv * hd, nkv * hd)
    w = [make_rows(rng, wtype, r, dim) for r in rows]
    att.set_qkv_weights(0, dim, w[0], wtype, w[1], wtype, w[2], wtype)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    xd = torch.from_numpy(x).to(DEV)
    flat = torch.empty(n_tok * dim + 1, dtype=torch.float32, device=DEV)
    xu = flat[1:].view(n_tok, dim)
    xu.copy_(xd)
    assert xu.data_ptr() % 16 == 4
    _, k, v = (g.cpu().numpy() for g in att.qkv_project_batch(0, xd))
    _, ku, vu = (g.cpu().numpy() for g in att.qkv_project_batch(0, xu))
    for name, g, gu, j in (("k", k, ku, 1), ("v", v, vu, 2)):
        want = O.matmul_bias_tokens(x, w[j], wtype, rows[j])
        assert_bits_equal(_bits(g), _bits(want), f"{name} aligned")
        assert_bits_equal(_bits(gu), _bits(want), f"{name} unaligned")
    att.close()


def test_batch_kv_equals_per_token_projection():
    # the batched reference-order K/V and pqa_qkv_project (one token, the same
    # order) give the same bits: Q4_K k, Q6_K v, Qwen3-4B width
    print("batch K/V vs per-token projection", flush=True)
    rng = np.random.default_rng(33)
    nh, nkv, hd, dim, n_tok = 8, 2, 128, 2560, 5
    att = PicoAttention(1, 16, nh, nkv, hd)
    w = [make_rows(rng, t, r, dim) for t, r in ((O.GGUF_Q4_K, nh * hd), (O.GGUF_Q4_K, nkv * hd),
                                                (O.GGUF_Q6_K, nkv * hd))]
    att.set_qkv_weights(0, dim, w[0], O.GGUF_Q4_K, w[1], O.GGUF_Q4_K, w[2], O.GGUF_Q6_K)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    _, kb, vb = (g.cpu().numpy() for g in att.qkv_project_batch(0, torch.from_numpy(x).to(DEV)))
    for t in range(n_tok):
        _, k1, v1 = (g.cpu().numpy() for g in att.qkv_project(0, torch.from_numpy(x[t]).to(DEV)))
        assert_bits_equal(_bits(kb[t]), _bits(k1), f"k token {t}")
        assert_bits_equal(_bits(vb[t]), _bits(v1), f"v token {t}")
    att.close()


def test_prefill_x_general_head_dim_rows_exact():
    # head_dim 96 takes the VALU attention kernels; their K/V prep reads the
    # reference-order columns as they are
    print("prefill_x hd 96, reference-order K/V", flush=True)
    rng = np.random.default_rng(3496)
    nh, nkv, hd, dim, n_tok, smax, start = 8, 2, 96, 512, 40, 64, 9
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    qn, kn = O.qk_norm_weights(5, 0, hd)
    att.set_qk_norm(0, qn, kn)
    types = (O.GGUF_Q8_0, O.GGUF_Q4_K, O.GGUF_F16)
    rows = (nh * hd, nkv * hd, nkv * hd)
    w = [make_rows(rng, t, r, dim) for t, r in zip(types, rows)]
    b = [make_bias(rng, O.GGUF_F32, r) for r in rows]
    att.set_qkv_weights(0, dim, w[0], types[0], w[1], types[1], w[2], types[2], b[0], O.GGUF_F32, b[1], O.GGUF_F32,
                        b[2], O.GGUF_F32)
    hk, hv = O.synth_kv_rows(3, 0, nkv * hd, 0, start, 0.0, 4)
    att.kv_upload(0, 0, hk, hv)
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros_like(kc)
    kc[:start], vc[:start] = hk, hv
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    qkv = [O.matmul_bias_tokens(x, w[j], types[j], rows[j], b[j], O.GGUF_F32) for j in range(3)]
    want = O.prefill(O.shape(nh, nkv, hd, smax, 0), start, *qkv, qn, kn, cos, sin, kc, vc)
    out = att.forward_batch_x(0, start, torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert_close(out, want)
    gk, gv = att.kv_download(0, start, n_tok)
    assert_bits_equal(gk, kc[start:start + n_tok], "K rows")
    assert_bits_equal(gv, vc[start:start + n_tok], "V rows")
    att.close()


def test_prompt_path_qwen3_4b_2048_tokens():
    # a whole 2048-token prompt at Qwen3-4B widths through pqa_prefill_x: all
    # 2048 K and V cache rows byte-equal to the oracle's (reference-order
    # projections, the reference's QK-norm, RoPE and fp16 rounding), and the
    # outputs of 48 tokens (the first 16, the last 16, 16 in between) within
    # the attention tolerance of the oracle's attention over that cache
    print("prompt path Qwen3-4B widths, 2048 tokens", flush=True)
    rng = np.random.default_rng(4096)
    nh, nkv, hd, dim, n_tok = 32, 8, 128, 2560, 2048
    smax = n_tok
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    qn, kn = O.qk_norm_weights(17, 0, hd)
    att.set_qk_norm(0, qn, kn)
    types = (O.GGUF_Q4_K, O.GGUF_Q4_K, O.GGUF_Q6_K)
    rows = (nh * hd, nkv * hd, nkv * hd)
    w = [make_rows(rng, t, r, dim) for t, r in zip(types, rows)]
    att.set_qkv_weights(0, dim, w[0], types[0], w[1], types[1], w[2], types[2])
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    out = att.forward_batch_x(0, 0, torch.from_numpy(x).to(DEV)).cpu().numpy()
    gk, gv = att.kv_download(0, 0, n_tok)
    att.close()
    print("  GPU done; oracle projections", flush=True)

    k = O.matmul_bias_tokens(x, w[1], types[1], rows[1], n_threads=16)
    v = O.matmul_bias_tokens(x, w[2], types[2], rows[2], n_threads=16)
    sample = sorted(set(range(16)) | set(range(n_tok - 16, n_tok)) | set(rng.choice(n_tok, 16, replace=False).tolist()))
    q = np.zeros((n_tok, nh * hd), np.float32)
    q[sample] = O.matmul_bias_tokens(x[sample], w[0], types[0], rows[0], n_threads=16)
    shp = O.shape(nh, nkv, hd, smax, 0)
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros_like(kc)
    qr = {}
    for t in range(n_tok):  # norm, RoPE, fp16 append of every row; the sampled q normed and rotated
        qt = O.append(shp, t, q[t], k[t], v[t], qn, kn, cos[t], sin[t], kc, vc)
        if t in sample:
            qr[t] = qt
    assert_bits_equal(gk, kc, "K rows of the 2048-token prompt")
    assert_bits_equal(gv, vc, "V rows of the 2048-token prompt")
    print("  cache rows equal; sampled outputs", flush=True)
    for t in sample:
        want = O.attend(shp, t, qr[t], kc, vc, n_threads=8)
        assert_close(out[t], want, what=f"output of token {t}")
