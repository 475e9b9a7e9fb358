"""Q/K/V projections on the GPU (pqa_qkv_project, pqa_decode_x through
libpqa.so) against the projection oracle, which is bit-equal to the
reference's matmul_bias: k and v bit-exact for every weight type, with and
without biases, at small shapes and at the Qwen3-8B layer shape; q bit-exact
with pqa_set_token_projection(1) and, by default, within the fp32 reordering
bound for the types of the any-order path (F32, F16, Q4_K) and bit-exact for
the others; the attention block from xb (pqa_decode_x) with its appended K/V
rows bit-exact and its output within max-abs 2e-3 / rel 1e-2 of the oracle."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from gpu_util import assert_bits_equal, assert_close
from proj_cases import make_bias, make_rows

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention, _lib  # noqa: E402
from picolm_qwen_amd._lib import PQA_ERR_ARG, PQA_ERR_UNSUPPORTED, PQAError  # noqa: E402

pytestmark = pytest.mark.gpu
TYPES = [O.GGUF_F32, O.GGUF_F16, O.GGUF_Q4_0, O.GGUF_Q8_0, O.GGUF_Q4_K, O.GGUF_Q6_K]


def _project(att, layer, x):
    dev = torch.device("cuda:0")
    q, k, v = att.qkv_project(layer, torch.from_numpy(x).to(dev))
    return q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()


FAST_Q = (O.GGUF_F32, O.GGUF_F16, O.GGUF_Q4_K)  # q types of the any-order path


def _q_within_reordering_bound(g, x, w, wt, rows, b, bt):
    # any summation order over n fused products, then the bias: at most
    # (n + 12) 2^-24 (sum_i |w_i x_i| + |b|) from the reference's sum (F32 and
    # F16 weights enter as they are); Q4_K groups are summed as d sum q x -
    # m sum x, so their terms are |d q_i| and |m| instead of |w_i|
    n = x.shape[0]
    want = O.matmul_bias(x, w, wt, rows, b, bt).astype(np.float64)
    if wt == O.GGUF_Q4_K:
        wf = O.q4k_term_magnitudes(w, n)
    else:
        wf = np.stack([O.dequant_row(wt, w[r], n) for r in range(rows)]).astype(np.float64)
    mag = np.abs(wf) @ np.abs(x.astype(np.float64))
    if b is not None:
        bias = b.view(np.float16) if bt == O.GGUF_F16 else b.view(np.float32)
        mag = mag + np.abs(bias.astype(np.float64))
    err = np.abs(g.astype(np.float64) - want)
    bound = (n + 12) * 2.0 ** -24 * mag + 1e-30
    assert np.all(err <= bound), (wt, float(np.max(err / bound)))
    # and in practice far inside it: a few ulps of sum |w x|
    assert float(np.median(err / (mag + 1e-30))) < 16 * 2.0 ** -24, wt


def _check(att, layer, x, mats, exact_q=False):
    got = _project(att, layer, x)
    for name, g, (w, wt, rows, b, bt) in zip("qkv", got, mats):
        if name == "q" and not exact_q and wt in FAST_Q:
            _q_within_reordering_bound(g, x, w, wt, rows, b, bt)
            continue
        want = O.matmul_bias(x, w, wt, rows, b, bt)
        assert_bits_equal(g.view(np.uint32), want.view(np.uint32), f"{name} (type {wt}, bias {bt})")


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("n", [512, 1536])
def test_projection_bit_exact_per_type(wtype, n):
    print(f"projection type {wtype} n {n}", flush=True)
    rng = np.random.default_rng(500 + 10 * wtype + n)
    nh, nkv, hd = 8, 2, 64
    att = PicoAttention(1, 64, nh, nkv, hd)
    mats = []
    for rows, bt in ((nh * hd, O.GGUF_NONE), (nkv * hd, O.GGUF_F32), (nkv * hd, O.GGUF_F16)):
        b = None if bt == O.GGUF_NONE else make_bias(rng, bt, rows)
        mats.append((make_rows(rng, wtype, rows, n, special=True), wtype, rows, b, bt))
    (wq, _, _, bq, bqt), (wk, _, _, bk, bkt), (wv, _, _, bv, bvt) = mats
    att.set_qkv_weights(0, n, wq, wtype, wk, wtype, wv, wtype, bq, bqt, bk, bkt, bv, bvt)
    x = rng.standard_normal(n).astype(np.float32)
    _check(att, 0, x, mats)
    att.set_token_projection(True)
    _check(att, 0, x, mats, exact_q=True)
    att.set_token_projection(False)
    _check(att, 0, x, mats)
    att.close()


def test_projection_qwen3_8b_layer_mixed_types():
    # Q4_K q/k and Q6_K v, as a Q4_K_M file stores them; 4096-wide rows
    print("projection qwen3-8b layer", flush=True)
    rng = np.random.default_rng(88)
    nh, nkv, hd, n = 32, 8, 128, 4096
    att = PicoAttention(2, 128, nh, nkv, hd)
    mats = [(make_rows(rng, O.GGUF_Q4_K, nh * hd, n), O.GGUF_Q4_K, nh * hd, None, O.GGUF_NONE),
            (make_rows(rng, O.GGUF_Q4_K, nkv * hd, n), O.GGUF_Q4_K, nkv * hd, None, O.GGUF_NONE),
            (make_rows(rng, O.GGUF_Q6_K, nkv * hd, n), O.GGUF_Q6_K, nkv * hd, None, O.GGUF_NONE)]
    att.set_qkv_weights(1, n, mats[0][0], O.GGUF_Q4_K, mats[1][0], O.GGUF_Q4_K, mats[2][0], O.GGUF_Q6_K)
    for seed in range(2):
        x = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
        _check(att, 1, x, mats)
    att.set_token_projection(True)
    _check(att, 1, x, mats, exact_q=True)
    att.close()


@pytest.mark.parametrize("wtype,n", [(O.GGUF_F32, 8), (O.GGUF_F16, 8), (O.GGUF_Q4_K, 256)])
def test_any_order_q_narrowest_rows(wtype, n):
    # the narrowest rows each type allows (one F32 / F16 unit for two lanes,
    # one Q4_K super-block: 4 of the wave's 64 lanes hold a unit) and a single
    # q row, k and v rows of one head
    print(f"any-order q narrow type {wtype} n {n}", flush=True)
    rng = np.random.default_rng(5000 + n + wtype)
    att = PicoAttention(1, 16, 1, 1, 64)
    mats = [(make_rows(rng, wtype, 64, n), wtype, 64, make_bias(rng, O.GGUF_F32, 64), O.GGUF_F32),
            (make_rows(rng, wtype, 64, n), wtype, 64, None, O.GGUF_NONE),
            (make_rows(rng, wtype, 64, n), wtype, 64, None, O.GGUF_NONE)]
    att.set_qkv_weights(0, n, mats[0][0], wtype, mats[1][0], wtype, mats[2][0], wtype, mats[0][3], O.GGUF_F32)
    for seed in range(3):
        x = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
        _check(att, 0, x, mats)
    att.close()


@pytest.mark.parametrize("wtype,n", [(O.GGUF_F32, 8192), (O.GGUF_F16, 8192), (O.GGUF_Q4_K, 8192), (O.GGUF_F32, 520),
                                     (O.GGUF_F16, 2056), (O.GGUF_Q4_K, 2560)])
def test_any_order_q_widths(wtype, n):
    # the any-order q rows at the widest input (8192: several batches of
    # units per lane) and at widths that leave lanes without a unit (F32 520,
    # F16 2056: a partial batch; Q4_K 2560: 40 quarter blocks for 64 lanes);
    # 300 q rows, so the last workgroup has waves past the last row
    print(f"any-order q type {wtype} n {n}", flush=True)
    rng = np.random.default_rng(4000 + n + wtype)
    att = PicoAttention(1, 16, 3, 1, 100)
    q_rows, kv_rows = 300, 100
    mats = [(make_rows(rng, wtype, q_rows, n), wtype, q_rows, make_bias(rng, O.GGUF_F16, q_rows), O.GGUF_F16),
            (make_rows(rng, wtype, kv_rows, n), wtype, kv_rows, None, O.GGUF_NONE),
            (make_rows(rng, wtype, kv_rows, n), wtype, kv_rows, make_bias(rng, O.GGUF_F32, kv_rows), O.GGUF_F32)]
    att.set_qkv_weights(0, n, mats[0][0], wtype, mats[1][0], wtype, mats[2][0], wtype,
                        mats[0][3], O.GGUF_F16, None, 0, mats[2][3], O.GGUF_F32)
    x = rng.standard_normal(n).astype(np.float32)
    _check(att, 0, x, mats)
    att.close()


@pytest.mark.parametrize("wtype", [O.GGUF_Q8_0, O.GGUF_Q4_0, O.GGUF_F16])
def test_projection_qwen25_width_partial_chunk(wtype):
    # Qwen2.5-0.5B: 896-wide rows (14 x 64), the last row chunk is partial
    rng = np.random.default_rng(9 + wtype)
    nh, nkv, hd, n = 14, 2, 64, 896
    att = PicoAttention(1, 32, nh, nkv, hd)
    mats = [(make_rows(rng, wtype, r, n), wtype, r, make_bias(rng, O.GGUF_F32, r), O.GGUF_F32)
            for r in (nh * hd, nkv * hd, nkv * hd)]
    att.set_qkv_weights(0, n, mats[0][0], wtype, mats[1][0], wtype, mats[2][0], wtype,
                        mats[0][3], O.GGUF_F32, mats[1][3], O.GGUF_F32, mats[2][3], O.GGUF_F32)
    x = rng.standard_normal(n).astype(np.float32)
    _check(att, 0, x, mats)
    att.close()


def test_rejected_shapes_and_types():
    att = PicoAttention(1, 16, 4, 2, 64)
    w = np.zeros((256, 1024), np.uint8)
    with pytest.raises(PQAError) as e:
        att.set_qkv_weights(0, 1024, w, 10, w, 10, w, 10)  # Q8_1: not a type the reference dequantizes
    assert e.value.code == PQA_ERR_UNSUPPORTED
    with pytest.raises(PQAError) as e:
        att.set_qkv_weights(0, 300, w, O.GGUF_Q4_K, w, O.GGUF_Q4_K, w, O.GGUF_Q4_K)  # not whole blocks
    assert e.value.code == PQA_ERR_UNSUPPORTED
    with pytest.raises(PQAError) as e:
        att.set_qkv_weights(0, 256, w, O.GGUF_Q6_K, w, O.GGUF_Q6_K, w, O.GGUF_Q6_K)  # Q6_K needs 512
    assert e.value.code == PQA_ERR_UNSUPPORTED
    dev = torch.device("cuda:0")
    xb = torch.zeros(256, device=dev)
    with pytest.raises(ValueError):  # the mirror refuses a layer without weights
        att.qkv_project(0, xb)
    # and so does the library on its own
    out = torch.zeros(4 * 64, device=dev)
    p = [C.c_void_p(t.data_ptr()) for t in (xb, out, out, out)]
    assert _lib.lib().pqa_qkv_project(att.handle, 0, *p) == PQA_ERR_ARG
    assert "no projection weights" in att.last_error()
    for setter, name in ((_lib.lib().pqa_set_token_projection, "exact_q"), (_lib.lib().pqa_set_out_projection, "exact")):
        assert setter(att.handle, 2) == PQA_ERR_ARG and name in att.last_error()
        assert setter(att.handle, 0) == 0 and setter(att.handle, 1) == 0
    att.close()


def test_weight_set_order_keeps_the_widest_lds_limit():
    # Qwen3-4B widths: attn_output rows are 4096 wide (67,584 bytes of LDS per
    # workgroup, above the default 64 KiB), attn_q/k/v rows 2560 (61,440). The
    # kernel's LDS limit is process-wide: setting the narrower q/k/v weights
    # after attn_output must not lower it below what out_project requests.
    print("out weights, then qkv weights, then out_project", flush=True)
    rng = np.random.default_rng(4040)
    nh, nkv, hd, dim = 32, 8, 128, 2560
    att = PicoAttention(1, 16, nh, nkv, hd)
    wo = make_rows(rng, O.GGUF_Q4_K, dim, nh * hd)
    att.set_out_weights(0, dim, wo, O.GGUF_Q4_K)
    mats = [make_rows(rng, O.GGUF_Q4_K, r, dim) for r in (nh * hd, nkv * hd, nkv * hd)]
    att.set_qkv_weights(0, dim, mats[0], O.GGUF_Q4_K, mats[1], O.GGUF_Q4_K, mats[2], O.GGUF_Q4_K)
    dev = torch.device("cuda:0")
    attn = rng.standard_normal(nh * hd).astype(np.float32)
    x0 = rng.standard_normal(dim).astype(np.float32)
    x = torch.from_numpy(x0.copy()).to(dev)
    att.out_project(0, torch.from_numpy(attn).to(dev), x)
    want = x0 + O.matmul_bias(attn, wo, O.GGUF_Q4_K, dim)
    assert_bits_equal(x.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32), "x after residual")
    # a second, narrower context made afterwards does not lower it either
    small = PicoAttention(1, 16, 4, 2, 64)
    sm = [make_rows(rng, O.GGUF_Q4_K, r, 512) for r in (256, 128, 128)]
    small.set_qkv_weights(0, 512, sm[0], O.GGUF_Q4_K, sm[1], O.GGUF_Q4_K, sm[2], O.GGUF_Q4_K)
    x = torch.from_numpy(x0.copy()).to(dev)
    att.out_project(0, torch.from_numpy(attn).to(dev), x)
    assert_bits_equal(x.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32), "x, second call")
    small.close()
    att.close()


@pytest.mark.parametrize("qk_norm", [False, True])
def test_decode_from_xb_matches_oracle(qk_norm):
    print(f"decode_x qk_norm {qk_norm}", flush=True)
    rng = np.random.default_rng(77 + qk_norm)
    nh, nkv, hd, n, smax, pos = 16, 8, 128, 2048, 512, 300
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    qn = kn = None
    if qk_norm:
        qn, kn = O.qk_norm_weights(31, 0, hd)
        att.set_qk_norm(0, qn, kn)
    wq = make_rows(rng, O.GGUF_Q4_K, nh * hd, n)
    wk = make_rows(rng, O.GGUF_Q4_K, nkv * hd, n)
    wv = make_rows(rng, O.GGUF_Q6_K, nkv * hd, n)
    att.set_qkv_weights(0, n, wq, O.GGUF_Q4_K, wk, O.GGUF_Q4_K, wv, O.GGUF_Q6_K)
    att.synth_kv(0, 0, pos, 31, 0.0)
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros((smax, nkv * hd), np.uint16)
    kc[:pos], vc[:pos] = O.synth_kv_rows(31, 0, nkv * hd, 0, pos)
    x = rng.standard_normal(n).astype(np.float32)
    q = O.matmul_bias(x, wq, O.GGUF_Q4_K, nh * hd)
    k = O.matmul_bias(x, wk, O.GGUF_Q4_K, nkv * hd)
    v = O.matmul_bias(x, wv, O.GGUF_Q6_K, nkv * hd)
    shp = O.shape(nh, nkv, hd, smax, 0)
    want = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc)
    out = att.forward_x(0, pos, torch.from_numpy(x).to(torch.device("cuda:0"))).cpu().numpy()
    gk, gv = att.kv_download(0, pos, 1)
    assert_bits_equal(gk[0], kc[pos], "appended K row")
    assert_bits_equal(gv[0], vc[pos], "appended V row")
    assert_close(out, want)
    att.close()


@pytest.mark.parametrize("wtype,bt", [(O.GGUF_Q4_K, O.GGUF_NONE), (O.GGUF_Q8_0, O.GGUF_F32), (O.GGUF_F16, O.GGUF_F16),
                                      (O.GGUF_Q6_K, O.GGUF_NONE)])
def test_out_projection_with_residual_bit_exact(wtype, bt):
    # Qwen3-4B shape: attention output 32 x 128 = 4096 wide, residual 2560
    print(f"out projection type {wtype} bias {bt}", flush=True)
    rng = np.random.default_rng(700 + wtype)
    nh, nkv, hd, dim = 32, 8, 128, 2560
    att = PicoAttention(1, 16, nh, nkv, hd)
    wo = make_rows(rng, wtype, dim, nh * hd)
    bo = None if bt == O.GGUF_NONE else make_bias(rng, bt, dim)
    att.set_out_weights(0, dim, wo, wtype, bo, bt)
    dev = torch.device("cuda:0")
    attn = rng.standard_normal(nh * hd).astype(np.float32)
    x0 = rng.standard_normal(dim).astype(np.float32)
    x = torch.from_numpy(x0.copy()).to(dev)
    att.out_project(0, torch.from_numpy(attn).to(dev), x)
    want = x0 + O.matmul_bias(attn, wo, wtype, dim, bo, bt)  # vec_add: x[i] + xb2[i] in fp32
    assert_bits_equal(x.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32), "x after residual")
    att.close()


@pytest.mark.parametrize("wtype,bt", [(O.GGUF_Q4_K, O.GGUF_NONE), (O.GGUF_F16, O.GGUF_F16), (O.GGUF_F32, O.GGUF_F32)])
def test_out_projection_any_order_within_bound(wtype, bt):
    # pqa_set_out_projection(0): x = x0 + (Wo attn + bo) with the sum in any
    # order, within the reordering bound of the sum, plus the residual add's
    # own rounding; then back to the reference's order, bit-exact again
    print(f"out projection any order type {wtype}", flush=True)
    rng = np.random.default_rng(720 + wtype)
    nh, nkv, hd, dim = 32, 8, 128, 2560
    att = PicoAttention(1, 16, nh, nkv, hd)
    wo = make_rows(rng, wtype, dim, nh * hd)
    bo = None if bt == O.GGUF_NONE else make_bias(rng, bt, dim)
    att.set_out_weights(0, dim, wo, wtype, bo, bt)
    dev = torch.device("cuda:0")
    attn = rng.standard_normal(nh * hd).astype(np.float32)
    x0 = rng.standard_normal(dim).astype(np.float32)
    att.set_out_projection(False)
    x = torch.from_numpy(x0.copy()).to(dev)
    att.out_project(0, torch.from_numpy(attn).to(dev), x)
    got = x.cpu().numpy().astype(np.float64)
    want = (x0 + O.matmul_bias(attn, wo, wtype, dim, bo, bt)).astype(np.float32).astype(np.float64)
    n = nh * hd
    if wtype == O.GGUF_Q4_K:
        wf = O.q4k_term_magnitudes(wo, n)
    else:
        wf = np.stack([O.dequant_row(wtype, wo[r], n) for r in range(dim)]).astype(np.float64)
    mag = np.abs(wf) @ np.abs(attn.astype(np.float64))
    if bo is not None:
        mag = mag + np.abs((bo.view(np.float16) if bt == O.GGUF_F16 else bo.view(np.float32)).astype(np.float64))
    bound = (n + 12) * 2.0 ** -24 * mag + 2.0 ** -23 * np.abs(want) + 1e-30
    err = np.abs(got - want)
    assert np.all(err <= bound), float(np.max(err / bound))
    att.set_out_projection(True)
    x = torch.from_numpy(x0.copy()).to(dev)
    att.out_project(0, torch.from_numpy(attn).to(dev), x)
    assert_bits_equal(x.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32), "x, reference order")
    att.close()


def test_attention_block_from_xb_to_residual():
    # the whole attention half of a Qwen3-4B layer at pos 200: K/V rows
    # bit-exact, x within the output tolerance (it carries the attention output)
    print("attention block", flush=True)
    rng = np.random.default_rng(4242)
    nh, nkv, hd, dim, smax, pos = 32, 8, 128, 2560, 256, 200
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    qn, kn = O.qk_norm_weights(5, 0, hd)
    att.set_qk_norm(0, qn, kn)
    wq = make_rows(rng, O.GGUF_Q4_K, nh * hd, dim)
    wk = make_rows(rng, O.GGUF_Q4_K, nkv * hd, dim)
    wv = make_rows(rng, O.GGUF_Q6_K, nkv * hd, dim)
    wo = make_rows(rng, O.GGUF_Q4_K, dim, nh * hd)
    att.set_qkv_weights(0, dim, wq, O.GGUF_Q4_K, wk, O.GGUF_Q4_K, wv, O.GGUF_Q6_K)
    att.set_out_weights(0, dim, wo, O.GGUF_Q4_K)
    att.synth_kv(0, 0, pos, 5, 0.0)
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros((smax, nkv * hd), np.uint16)
    kc[:pos], vc[:pos] = O.synth_kv_rows(5, 0, nkv * hd, 0, pos)
    xb = rng.standard_normal(dim).astype(np.float32)
    x0 = rng.standard_normal(dim).astype(np.float32)
    q = O.matmul_bias(xb, wq, O.GGUF_Q4_K, nh * hd)
    k = O.matmul_bias(xb, wk, O.GGUF_Q4_K, nkv * hd)
    v = O.matmul_bias(xb, wv, O.GGUF_Q6_K, nkv * hd)
    attn = O.attn_step(O.shape(nh, nkv, hd, smax, 0), pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc)
    want = x0 + O.matmul_bias(attn, wo, O.GGUF_Q4_K, dim)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(x0.copy()).to(dev)
    att.attention_block(0, pos, torch.from_numpy(xb).to(dev), x)
    gk, gv = att.kv_download(0, pos, 1)
    assert_bits_equal(gk[0], kc[pos], "appended K row")
    assert_bits_equal(gv[0], vc[pos], "appended V row")
    assert_close(x.cpu().numpy(), want, what="residual stream")
    att.close()


def test_batched_projection_within_fp32_reordering_bound():
    # Qwen3-4B widths, 37 tokens: the weights are dequantized exactly; the
    # batched path splits w and x (scaled by powers of two) into fp16 hi + lo
    # and sums w_hi x_hi + w_hi x_lo + w_lo x_hi in fp32 over 3n terms in the
    # GEMM's own order. Its error is at most (3n + 12) 2^-24 sum_i |w_i x_i|
    # (2^-22 per product for the split, any summation order over 3n terms);
    # the reference's sequential sums add (n + 1) 2^-24 sum_i |w_i x_i|
    print("batched projection", flush=True)
    rng = np.random.default_rng(31337)
    nh, nkv, hd, dim, n_tok = 32, 8, 128, 2560, 37
    att = PicoAttention(1, 64, nh, nkv, hd)
    mats = [(make_rows(rng, O.GGUF_Q4_K, nh * hd, dim), O.GGUF_Q4_K, nh * hd, make_bias(rng, O.GGUF_F32, nh * hd),
             O.GGUF_F32),
            (make_rows(rng, O.GGUF_Q4_K, nkv * hd, dim), O.GGUF_Q4_K, nkv * hd, None, O.GGUF_NONE),
            (make_rows(rng, O.GGUF_Q6_K, nkv * hd, dim), O.GGUF_Q6_K, nkv * hd, make_bias(rng, O.GGUF_F16, nkv * hd),
             O.GGUF_F16)]
    att.set_qkv_weights(0, dim, mats[0][0], O.GGUF_Q4_K, mats[1][0], O.GGUF_Q4_K, mats[2][0], O.GGUF_Q6_K,
                        mats[0][3], O.GGUF_F32, None, 0, mats[2][3], O.GGUF_F16)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    got = [g.cpu().numpy() for g in att.qkv_project_batch(0, torch.from_numpy(x).to(torch.device("cuda:0")))]
    for name, g, (w, wt, rows, b, bt) in zip("qkv", got, mats):
        wf = np.stack([O.dequant_row(wt, w[r], dim) for r in range(rows)]).astype(np.float64)
        for t in range(0, n_tok, 6):
            want = O.matmul_bias(x[t], w, wt, rows, b, bt)
            mag = np.abs(wf) @ np.abs(x[t].astype(np.float64))
            bound = (4 * dim + 13) * 2.0 ** -24 * mag + 1e-30
            err = np.abs(g[t].astype(np.float64) - want)
            assert np.all(err <= bound), (name, t, float(np.max(err / bound)))
            # and in practice far inside it: a typical error of a few ulps of sum |w x|
            assert float(np.median(err / (mag + 1e-30))) < 64 * 2.0 ** -24, (name, t)
    att.close()


@pytest.mark.parametrize("wtype", TYPES)
def test_batched_projection_every_type(wtype):
    # the batched path over each weight type the reference dequantizes, odd
    # token counts, F32 and F16 biases; same bound as above
    print(f"batched projection type {wtype}", flush=True)
    rng = np.random.default_rng(900 + wtype)
    nh, nkv, hd, dim = 4, 2, 64, 1024  # whole blocks of every type (Q6_K rows: multiples of 512)
    att = PicoAttention(1, 16, nh, nkv, hd)
    mats = [(make_rows(rng, wtype, rows, dim, special=True), make_bias(rng, bt, rows) if bt else None, bt)
            for rows, bt in ((nh * hd, O.GGUF_F16), (nkv * hd, O.GGUF_NONE), (nkv * hd, O.GGUF_F32))]
    att.set_qkv_weights(0, dim, mats[0][0], wtype, mats[1][0], wtype, mats[2][0], wtype,
                        mats[0][1], mats[0][2], None, 0, mats[2][1], mats[2][2])
    for n_tok in (1, 5):
        x = rng.standard_normal((n_tok, dim)).astype(np.float32)
        got = [g.cpu().numpy() for g in att.qkv_project_batch(0, torch.from_numpy(x).to(torch.device("cuda:0")))]
        for name, g, (w, b, bt) in zip("qkv", got, mats):
            wf = np.stack([O.dequant_row(wtype, w[r], dim) for r in range(w.shape[0])]).astype(np.float64)
            for t in range(n_tok):
                want = O.matmul_bias(x[t], w, wtype, w.shape[0], b, bt)
                mag = np.abs(wf) @ np.abs(x[t].astype(np.float64))
                err = np.abs(g[t].astype(np.float64) - want)
                assert np.all(err <= (4 * dim + 13) * 2.0 ** -24 * mag + 1e-30), (name, n_tok, t)
    att.close()


def test_batched_projection_follows_replaced_weights():
    # the batched path keeps a split copy of a layer's rows; replacing the
    # layer's weights must drop it
    print("batched projection after new weights", flush=True)
    rng = np.random.default_rng(4242)
    nh, nkv, hd, dim, n_tok = 4, 2, 64, 512, 9
    att = PicoAttention(2, 16, nh, nkv, hd)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    xd = torch.from_numpy(x).to(torch.device("cuda:0"))
    for rep in range(2):
        ws = [make_rows(rng, O.GGUF_Q8_0, rows, dim) for rows in (nh * hd, nkv * hd, nkv * hd)]
        att.set_qkv_weights(1, dim, ws[0], O.GGUF_Q8_0, ws[1], O.GGUF_Q8_0, ws[2], O.GGUF_Q8_0)
        got = [g.cpu().numpy() for g in att.qkv_project_batch(1, xd)]
        for g, w in zip(got, ws):
            wf = np.stack([O.dequant_row(O.GGUF_Q8_0, w[r], dim) for r in range(w.shape[0])]).astype(np.float64)
            for t in range(n_tok):
                want = O.matmul_bias(x[t], w, O.GGUF_Q8_0, w.shape[0])
                mag = np.abs(wf) @ np.abs(x[t].astype(np.float64))
                assert np.all(np.abs(g[t] - want) <= (4 * dim + 13) * 2.0 ** -24 * mag + 1e-30), (rep, t)
    att.close()


def test_batched_projection_multi_tile_and_k_padding():
    # the GEMM's edges: 600 tokens = 3 row blocks of 256 (the last partial),
    # 640 output rows = 3 column blocks of 192 and a partial one, and F32
    # weights of width 104 (each split half padded with zeros to 128); same bound
    print("batched projection: multi-tile, padded K", flush=True)
    rng = np.random.default_rng(6060)
    nh, nkv, hd, dim, n_tok = 6, 2, 64, 104, 600
    att = PicoAttention(1, 16, nh, nkv, hd)
    mats = [(make_rows(rng, O.GGUF_F32, rows, dim), make_bias(rng, O.GGUF_F32, rows)) for rows in
            (nh * hd, nkv * hd, nkv * hd)]
    att.set_qkv_weights(0, dim, mats[0][0], O.GGUF_F32, mats[1][0], O.GGUF_F32, mats[2][0], O.GGUF_F32,
                        mats[0][1], O.GGUF_F32, mats[1][1], O.GGUF_F32, mats[2][1], O.GGUF_F32)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    got = [g.cpu().numpy() for g in att.qkv_project_batch(0, torch.from_numpy(x).to(torch.device("cuda:0")))]
    for name, g, (w, b) in zip("qkv", got, mats):
        wf = np.stack([O.dequant_row(O.GGUF_F32, w[r], dim) for r in range(w.shape[0])]).astype(np.float64)
        for t in sorted({0, 1, 255, 256, 300, 511, 512, 598, 599} | set(range(3, n_tok, 41))):
            want = O.matmul_bias(x[t], w, O.GGUF_F32, w.shape[0], b, O.GGUF_F32)
            mag = np.abs(wf) @ np.abs(x[t].astype(np.float64))
            err = np.abs(g[t].astype(np.float64) - want)
            assert np.all(err <= (4 * dim + 13) * 2.0 ** -24 * mag + 1e-30), (name, t, float(np.max(err)))
    att.close()


def _check_prompt_rows(got_rows, want_rows, exact_kv):
    """Appended K/V rows of the prompt path: byte-equal with the reference-order
    K/V projection (the default); with the split GEMM a few elements may round
    to the neighbouring fp16 value (the projection's ~1e-6 relative reordering
    carried through norm and RoPE)."""
    for name, g, wnt in zip("KV", got_rows, want_rows):
        if exact_kv:
            assert_bits_equal(g, wnt, f"{name} rows from xb")
            continue
        same = g == wnt
        gf, wf = g.view(np.float16).astype(np.float64), wnt.view(np.float16).astype(np.float64)
        slack = 2.0 ** -10 * np.abs(wf) + 1e-4 * np.abs(wf).max()
        assert same.mean() >= 0.99 and np.all(np.abs(gf - wf) <= slack), (name, float(same.mean()))


@pytest.mark.parametrize("exact_kv", [True, False])
def test_prompt_path_from_xb_with_biases(exact_kv):
    # Qwen2.5-style layer: q/k/v biases (F32 and F16), no QK-norm, hd 64,
    # a prompt continuing at position 40; the prefill kernels read the scaled
    # GEMM result, undo the scale and add the biases themselves (q always; k
    # and v only with the split-GEMM K/V projection). q and k here have std 2
    # (scores up to ~11): the default hi + lo q keeps the scores at fp32 level
    # (one fp16 q would miss the tolerance here)
    print(f"prefill_x with biases, exact_kv {exact_kv}", flush=True)
    rng = np.random.default_rng(1414)
    nh, nkv, hd, dim, n_tok, smax, start = 14, 2, 64, 896, 70, 160, 40
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    if not exact_kv:
        att.set_batch_projection(False)
    mats = [(make_rows(rng, O.GGUF_Q8_0, nh * hd, dim), make_bias(rng, O.GGUF_F32, nh * hd), O.GGUF_F32),
            (make_rows(rng, O.GGUF_Q8_0, nkv * hd, dim), make_bias(rng, O.GGUF_F16, nkv * hd), O.GGUF_F16),
            (make_rows(rng, O.GGUF_Q8_0, nkv * hd, dim), make_bias(rng, O.GGUF_F32, nkv * hd), O.GGUF_F32)]
    att.set_qkv_weights(0, dim, mats[0][0], O.GGUF_Q8_0, mats[1][0], O.GGUF_Q8_0, mats[2][0], O.GGUF_Q8_0,
                        mats[0][1], mats[0][2], mats[1][1], mats[1][2], mats[2][1], mats[2][2])
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros((smax, nkv * hd), np.uint16)
    hk, hv = O.synth_kv_rows(77, 0, nkv * hd, 0, start, 0.0, 4)
    kc[:start], vc[:start] = hk, hv
    att.kv_upload(0, 0, hk, hv)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    qkv = [np.stack([O.matmul_bias(x[t], w, O.GGUF_Q8_0, w.shape[0], b, bt) for t in range(n_tok)])
           for w, b, bt in mats]
    want = O.prefill(O.shape(nh, nkv, hd, smax, 0), start, *qkv, None, None, cos, sin, kc, vc)
    out = att.forward_batch_x(0, start, torch.from_numpy(x).to(torch.device("cuda:0"))).cpu().numpy()
    assert_close(out, want)
    _check_prompt_rows(att.kv_download(0, start, n_tok), (kc[start:start + n_tok], vc[start:start + n_tok]), exact_kv)
    att.close()


@pytest.mark.parametrize("exact_kv", [True, False])
def test_prompt_path_from_xb_matches_oracle(exact_kv):
    # pqa_prefill_x = batched projections + the MFMA prefill: outputs within the
    # attention tolerance; K/V rows byte-equal with the reference-order K/V
    # projection, within one fp16 step (>= 99 % equal) with the split GEMM
    print(f"prefill_x, exact_kv {exact_kv}", flush=True)
    rng = np.random.default_rng(2718)
    nh, nkv, hd, dim, n_tok, smax = 16, 8, 128, 2048, 96, 128
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    if not exact_kv:
        att.set_batch_projection(False)
    qn, kn = O.qk_norm_weights(9, 0, hd)
    att.set_qk_norm(0, qn, kn)
    wq = make_rows(rng, O.GGUF_Q4_K, nh * hd, dim)
    wk = make_rows(rng, O.GGUF_Q4_K, nkv * hd, dim)
    wv = make_rows(rng, O.GGUF_Q6_K, nkv * hd, dim)
    att.set_qkv_weights(0, dim, wq, O.GGUF_Q4_K, wk, O.GGUF_Q4_K, wv, O.GGUF_Q6_K)
    x = rng.standard_normal((n_tok, dim)).astype(np.float32)
    q = np.stack([O.matmul_bias(x[t], wq, O.GGUF_Q4_K, nh * hd) for t in range(n_tok)])
    k = np.stack([O.matmul_bias(x[t], wk, O.GGUF_Q4_K, nkv * hd) for t in range(n_tok)])
    v = np.stack([O.matmul_bias(x[t], wv, O.GGUF_Q6_K, nkv * hd) for t in range(n_tok)])
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros((smax, nkv * hd), np.uint16)
    want = O.prefill(O.shape(nh, nkv, hd, smax, 0), 0, q, k, v, qn, kn, cos, sin, kc, vc)
    out = att.forward_batch_x(0, 0, torch.from_numpy(x).to(torch.device("cuda:0"))).cpu().numpy()
    assert_close(out, want)
    _check_prompt_rows(att.kv_download(0, 0, n_tok), (kc[:n_tok], vc[:n_tok]), exact_kv)
    att.close()


def test_batched_projection_unaligned_input_equals_aligned():
    # X rows that are not 16-byte aligned take the scalar split kernel, aligned
    # ones the float4 kernel; both do the same arithmetic, so q, k and v must
    # agree bit for bit (and with the oracle, through the tests above)
    print("batched projection, unaligned input", flush=True)
    rng = np.random.default_rng(5151)
    nh, nkv, hd, dim, n_tok = 4, 2, 64, 512, 7
    att = PicoAttention(1, 16, nh, nkv, hd)
    ws = [make_rows(rng, O.GGUF_Q4_K, rows, dim) for rows in (nh * hd, nkv * hd, nkv * hd)]
    att.set_qkv_weights(0, dim, ws[0], O.GGUF_Q4_K, ws[1], O.GGUF_Q4_K, ws[2], O.GGUF_Q4_K)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(rng.standard_normal((n_tok, dim)).astype(np.float32)).to(dev)
    flat = torch.empty(n_tok * dim + 1, dtype=torch.float32, device=dev)
    xu = flat[1:].view(n_tok, dim)
    xu.copy_(x)
    assert xu.data_ptr() % 16 == 4
    a = [g.cpu().numpy() for g in att.qkv_project_batch(0, x)]
    b = [g.cpu().numpy() for g in att.qkv_project_batch(0, xu)]
    for name, ga, gb in zip("qkv", a, b):
        assert_bits_equal(gb, ga, f"{name} from unaligned rows")
    att.close()


def test_batched_projection_rejects_unaligned_outputs():
    # q, k and v are stored as float4s: a misaligned output pointer is refused
    # (PQA_ERR_ARG) before any kernel runs, as pqa_decode and pqa_prefill do
    rng = np.random.default_rng(5252)
    nh, nkv, hd, dim, n_tok = 4, 2, 64, 512, 3
    att = PicoAttention(1, 16, nh, nkv, hd)
    ws = [make_rows(rng, O.GGUF_Q4_K, rows, dim) for rows in (nh * hd, nkv * hd, nkv * hd)]
    att.set_qkv_weights(0, dim, ws[0], O.GGUF_Q4_K, ws[1], O.GGUF_Q4_K, ws[2], O.GGUF_Q4_K)
    dev = torch.device("cuda:0")
    x = torch.zeros((n_tok, dim), dtype=torch.float32, device=dev)
    buf = torch.zeros(n_tok * nh * hd + 8, dtype=torch.float32, device=dev)
    kv = torch.zeros(n_tok * nkv * hd + 8, dtype=torch.float32, device=dev)
    L = _lib.lib()
    ptr = lambda t, off=0: C.c_void_p(t.data_ptr() + off)  # noqa: E731
    for qo, ko, vo in ((4, 0, 0), (0, 8, 0), (0, 0, 12)):
        rc = L.pqa_qkv_project_batch(att.handle, 0, n_tok, ptr(x), ptr(buf, qo), ptr(kv, ko), ptr(kv, vo))
        assert rc == PQA_ERR_ARG and "aligned" in att.last_error()
    att.close()
