"""The forward-loop entry points on the GPU: the batched output projection with
its residual add (pqa_out_project_batch) within the split GEMM's bound; the
attention half of a forward_batch layer (pqa_prefill_block) against the oracle's
per-token chain and bit-equal to its two halves called one after the other; the
host-pointer forms bit-equal to the device ones; and the compiled adapter
(include/pqa_forward.hpp through adapter/forward_demo.cpp) running a prompt
and decode tokens through two layers, checked against the reference's layer
loops restated on the oracle."""
import numpy as np
import pytest

import oracle as O
from adapter_cases import Model
from gpu_util import assert_bits_equal, assert_close
from proj_cases import make_bias, make_rows

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _layer(rng, nh, nkv, hd, dim, types=(O.GGUF_Q4_K, O.GGUF_Q4_K, O.GGUF_Q6_K, O.GGUF_Q4_K), bias=False):
    """Q/K/V/O rows of one layer and their biases (F32, or None)."""
    rows = (nh * hd, nkv * hd, nkv * hd, dim)
    widths = (dim, dim, dim, nh * hd)
    w = [make_rows(rng, t, r, n) for t, r, n in zip(types, rows, widths)]
    b = [make_bias(rng, O.GGUF_F32, r) if bias else None for r in rows]
    return w, b


def _set(att, layer, dim, w, b, types):
    bt = [O.GGUF_NONE if x is None else O.GGUF_F32 for x in b]
    att.set_qkv_weights(layer, dim, w[0], types[0], w[1], types[1], w[2], types[2], b[0], bt[0], b[1], bt[1], b[2],
                        bt[2])
    att.set_out_weights(layer, dim, w[3], types[3], b[3], bt[3])


@pytest.mark.parametrize("n_tok", [1, 37, 300])
def test_out_project_batch_within_split_gemm_bound(n_tok):
    # Qwen3-4B widths: attention output 4096 wide, residual 2560. The split fp16
    # GEMM is within (3 q_dim + 12) 2^-24 sum |w a| of exact (the bound the Q/K/V
    # tests use, with the reference's own summation error on top); the bias add
    # and the residual add round once each on both sides
    print(f"out_project_batch n_tok {n_tok}", flush=True)
    rng = np.random.default_rng(9000 + n_tok)
    nh, nkv, hd, dim = 32, 8, 128, 2560
    qd = nh * hd
    att = PicoAttention(1, 16, nh, nkv, hd)
    wo = make_rows(rng, O.GGUF_Q4_K, dim, qd)
    bo = make_bias(rng, O.GGUF_F32, dim)
    att.set_out_weights(0, dim, wo, O.GGUF_Q4_K, bo, O.GGUF_F32)
    attn = rng.standard_normal((n_tok, qd)).astype(np.float32)
    x0 = rng.standard_normal((n_tok, dim)).astype(np.float32)
    x = torch.from_numpy(x0.copy()).to(DEV)
    att.out_project_batch(0, torch.from_numpy(attn).to(DEV), x)
    got = x.cpu().numpy().astype(np.float64)
    wf = np.stack([O.dequant_row(O.GGUF_Q4_K, wo[r], qd) for r in range(dim)]).astype(np.float64)
    bf = bo.view(np.float32).astype(np.float64)
    for t in sorted({0, n_tok // 2, n_tok - 1}):
        want = (x0[t] + O.matmul_bias(attn[t], wo, O.GGUF_Q4_K, dim, bo, O.GGUF_F32)).astype(np.float64)
        mag = np.abs(wf) @ np.abs(attn[t].astype(np.float64)) + np.abs(bf)
        bound = (4 * qd + 13) * 2.0 ** -24 * mag + 2.0 ** -23 * (np.abs(want) + np.abs(x0[t])) + 1e-30
        err = np.abs(got[t] - want)
        assert np.all(err <= bound), (t, float(np.max(err / bound)))
    att.close()


def test_prefill_block_matches_oracle_chain_and_its_halves():
    # a Qwen3-style layer (QK-norm, no biases) at hd 128; a 60-token prompt
    # continuing a 40-row history: x after the block within the attention
    # tolerance of the reference's per-token chain, and bit-equal to
    # pqa_prefill_x followed by pqa_out_project_batch
    print("prefill_block", flush=True)
    rng = np.random.default_rng(5150)
    nh, nkv, hd, dim, n_tok, start, smax = 16, 8, 128, 2048, 60, 40, 128
    types = (O.GGUF_Q4_K, O.GGUF_Q4_K, O.GGUF_Q6_K, O.GGUF_Q8_0)
    w, b = _layer(rng, nh, nkv, hd, dim, types)
    cos, sin = O.rope_table(1e6, hd, smax)
    qn, kn = O.qk_norm_weights(11, 0, hd)
    atts = []
    for _ in range(2):
        a = PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
        a.set_qk_norm(0, qn, kn)
        _set(a, 0, dim, w, b, types)
        atts.append(a)
    hk, hv = O.synth_kv_rows(21, 0, nkv * hd, 0, start, 0.0, 4)
    for a in atts:
        a.kv_upload(0, 0, hk, hv)
    kc = np.zeros((smax, nkv * hd), np.uint16)
    vc = np.zeros_like(kc)
    kc[:start], vc[:start] = hk, hv
    xb = rng.standard_normal((n_tok, dim)).astype(np.float32)
    x0 = rng.standard_normal((n_tok, dim)).astype(np.float32)
    want = np.empty_like(x0)
    shp = O.shape(nh, nkv, hd, smax, 0)
    for i in range(n_tok):
        pos = start + i
        q, k, v = (O.matmul_bias(xb[i], w[j], types[j], r) for j, r in enumerate((nh * hd, nkv * hd, nkv * hd)))
        attn = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc)
        want[i] = x0[i] + O.matmul_bias(attn, w[3], types[3], dim)
    x = torch.from_numpy(x0.copy()).to(DEV)
    atts[0].prefill_block(0, start, torch.from_numpy(xb).to(DEV), x)
    got = x.cpu().numpy()
    assert_close(got, want, what="residual stream")
    gk, gv = atts[0].kv_download(0, start, n_tok)
    # the default reference-order K/V projection: the cache rows are the
    # reference's bytes
    assert_bits_equal(gk, kc[start:start + n_tok], "K rows")
    assert_bits_equal(gv, vc[start:start + n_tok], "V rows")
    # the same two halves through their own entry points
    attn = atts[1].forward_batch_x(0, start, torch.from_numpy(xb).to(DEV))
    x2 = torch.from_numpy(x0.copy()).to(DEV)
    atts[1].out_project_batch(0, attn, x2)
    assert_bits_equal(x2.cpu().numpy().view(np.uint32), got.view(np.uint32), "prefill_block vs its halves")
    for a in atts:
        a.close()


@pytest.mark.parametrize("n_tok", [24, 300, 1100])
def test_host_entry_points_equal_device_ones(n_tok):
    # pqa_prefill_block_host / pqa_attention_block_host against the device
    # forms on a twin context: bit-equal x and cache rows. 24 tokens take the
    # one-copy pinned buffer; 300 tokens of 2048 floats (4.8 MB in, 2.4 MB
    # back) one fill of the two 8 MiB slots each way; 1100 tokens (18 MB in,
    # 9 MB back) three fills in and two back
    print(f"host blocks n_tok {n_tok}", flush=True)
    rng = np.random.default_rng(777 + n_tok)
    nh, nkv, hd, dim = 16, 4, 128, 2048
    smax = max(320, n_tok + 8)
    types = (O.GGUF_Q8_0, O.GGUF_Q8_0, O.GGUF_Q8_0, O.GGUF_Q4_K)
    w, b = _layer(rng, nh, nkv, hd, dim, types, bias=True)
    cos, sin = O.rope_table(1e6, hd, smax)
    host, dev = (PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin) for _ in range(2))
    for a in (host, dev):
        _set(a, 0, dim, w, b, types)
    xb = rng.standard_normal((n_tok, dim)).astype(np.float32)
    x0 = rng.standard_normal((n_tok, dim)).astype(np.float32)
    xh = x0.copy()
    host.prefill_block(0, 0, xb, xh)
    xd = torch.from_numpy(x0.copy()).to(DEV)
    dev.prefill_block(0, 0, torch.from_numpy(xb).to(DEV), xd)
    assert_bits_equal(xh.view(np.uint32), xd.cpu().numpy().view(np.uint32), "prefill block x")
    for pos in (n_tok, n_tok + 1):
        xb1 = rng.standard_normal(dim).astype(np.float32)
        x1 = rng.standard_normal(dim).astype(np.float32)
        h1 = x1.copy()
        host.attention_block(0, pos, xb1, h1)
        d1 = torch.from_numpy(x1.copy()).to(DEV)
        dev.attention_block(0, pos, torch.from_numpy(xb1).to(DEV), d1)
        assert_bits_equal(h1.view(np.uint32), d1.cpu().numpy().view(np.uint32), f"decode block x at {pos}")
    hk, hv = host.kv_download(0, 0, n_tok + 2)
    dk, dv = dev.kv_download(0, 0, n_tok + 2)
    assert_bits_equal(hk, dk, "K rows")
    assert_bits_equal(hv, dv, "V rows")
    for a in (host, dev):
        a.close()


def test_host_attention_block_equals_device_on_the_any_order_paths():
    # Q4_K q and attn_output rows: the host entry takes the same any-order q
    # path (the default) and, switched on, the any-order attn_output path, as
    # the device entry: bit-equal x and cache rows
    print("host attention block, any-order paths", flush=True)
    rng = np.random.default_rng(4711)
    nh, nkv, hd, dim, smax = 16, 4, 128, 2048, 64
    types = (O.GGUF_Q4_K, O.GGUF_Q4_K, O.GGUF_Q6_K, O.GGUF_Q4_K)
    w, b = _layer(rng, nh, nkv, hd, dim, types, bias=True)
    cos, sin = O.rope_table(1e6, hd, smax)
    host, dev = (PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin) for _ in range(2))
    for a in (host, dev):
        _set(a, 0, dim, w, b, types)
        a.synth_kv(0, 0, 20, 3, 0.0)
    for pos, out_exact in ((20, True), (21, False)):
        for a in (host, dev):
            a.set_out_projection(out_exact)
        xb1 = rng.standard_normal(dim).astype(np.float32)
        x1 = rng.standard_normal(dim).astype(np.float32)
        h1 = x1.copy()
        host.attention_block(0, pos, xb1, h1)
        d1 = torch.from_numpy(x1.copy()).to(DEV)
        dev.attention_block(0, pos, torch.from_numpy(xb1).to(DEV), d1)
        assert_bits_equal(h1.view(np.uint32), d1.cpu().numpy().view(np.uint32), f"x at {pos}")
    hk, hv = host.kv_download(0, 0, 22)
    dk, dv = dev.kv_download(0, 0, 22)
    assert_bits_equal(hk, dk, "K rows")
    assert_bits_equal(hv, dv, "V rows")
    for a in (host, dev):
        a.close()


@pytest.mark.parametrize("qk_norm,bias", [(True, False), (False, True)])
def test_compiled_adapter_runs_the_reference_loops(qk_norm, bias):
    # two layers, a 24-token prompt through forward_batch_layers, then 4 tokens
    # through forward_layers, norms and FFN as callbacks; the residual streams
    # after the last layer within the attention tolerance of the reference's
    # loops on the oracle (projections there are sequential F32 dot products)
    print(f"adapter demo qk_norm {qk_norm} bias {bias}", flush=True)
    m = Model(31 + int(qk_norm), qk_norm=qk_norm, bias=bias)
    rng = np.random.default_rng(8)
    xp = rng.standard_normal((24, m.n)).astype(np.float32)
    xd = rng.standard_normal((4, m.n)).astype(np.float32)
    want_p, want_d, _, _ = m.reference_chain(xp, xd)
    rc, msg = m.run_demo(xp, xd)
    assert rc == 0, msg
    assert_close(xp, want_p, what="prompt residual streams")
    assert_close(xd, want_d, what="decode residual streams")
