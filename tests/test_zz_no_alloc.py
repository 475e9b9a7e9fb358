"""pqa_decode_noalloc (split partials in the library's static per-GPU scratch)
against pqa_decode (context workspace), through the C ABI: two calls in a row,
the second over a shorter history (fewer splits, so the scratch still holds
the first call's partials past what the second call writes), then another
context shape on the same GPU. Outputs within max-abs 2e-3 / rel 1e-2 of
pqa_decode's (the same kernels: expected bit-identical) and of the oracle;
appended rows bit-exact."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads
from gpu_util import assert_bits_equal, assert_close

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention, _lib  # noqa: E402

pytestmark = pytest.mark.gpu


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _both(att, layer, pos, q, k, v):
    """pqa_decode, then pqa_decode_noalloc, on the same inputs; both append
    the same row at pos."""
    L = _lib.lib()
    dev = torch.device("cuda:0")
    tq, tk, tv = (torch.from_numpy(x).to(dev) for x in (q, k, v))
    want = torch.empty(att.q_dim, dtype=torch.float32, device=dev)
    got = torch.full((att.q_dim,), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    _lib.check(L.pqa_decode(att.handle, layer, pos, _ptr(tq), _ptr(tk), _ptr(tv), _ptr(want)), att.handle)
    _lib.check(L.pqa_decode_noalloc(att.handle, layer, pos, _ptr(tq), _ptr(tk), _ptr(tv), _ptr(got)), att.handle)
    att.sync()
    return got.cpu().numpy(), want.cpu().numpy()


def _case(nh, nkv, hd, smax, style, base, qk, positions, seed):
    kvd = nkv * hd
    cos, sin = O.rope_table(base, hd, smax)
    att = PicoAttention(1, smax, nh, nkv, hd, style, rope_cos=cos, rope_sin=sin)
    qn = kn = None
    if qk:
        qn, kn = O.qk_norm_weights(seed, 0, hd)
        att.set_qk_norm(0, qn, kn)
    top = max(positions)
    att.synth_kv(0, 0, top, seed, 0.01)
    kh, vh = O.synth_kv_rows(seed, 0, kvd, 0, top, 0.01, cpu_threads())
    shp = O.shape(nh, nkv, hd, smax, style)
    for i, pos in enumerate(positions):
        print(f"noalloc {nh}/{nkv}/{hd} pos {pos}", flush=True)
        q, k, v = O.step_inputs(seed, 0, i, nh, nkv, hd)
        got, want = _both(att, 0, pos, q, k, v)
        assert_close(got, want, what=f"pqa_decode_noalloc vs pqa_decode at pos {pos}")
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "same kernels: expected identical bits"
        kc = np.zeros((pos + 1, kvd), np.uint16)
        vc = np.zeros((pos + 1, kvd), np.uint16)
        kc[:pos], vc[:pos] = kh[:pos], vh[:pos]
        ref = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc, cpu_threads())
        assert_close(got, ref, what=f"pqa_decode_noalloc vs oracle at pos {pos}")
        rk, rv = att.kv_download(0, pos, 1)
        assert_bits_equal(rk[0], kc[pos], "appended K row")
        assert_bits_equal(rv[0], vc[pos], "appended V row")
        # the history rows at pos were overwritten by the append; restore them
        # for the next (shorter) call's oracle
        if pos < top:
            att.kv_upload(0, pos, kh[pos:pos + 1], vh[pos:pos + 1])
    att.close()


def test_noalloc_matches_decode_long_then_short_history():
    # 256 splits (whole-row workgroups), then 6 per-column splits
    _case(32, 8, 128, 32768, 0, 1e6, True, [32767, 700], seed=8801)


def test_noalloc_other_shape_on_the_same_gpu():
    # GQA group of 7, head_dim 64: other partial strides over the same scratch
    _case(14, 2, 64, 4096, 0, 1e6, False, [4095, 1000, 3], seed=8802)


def test_noalloc_runs_one_split_when_partials_exceed_the_scratch():
    # 8192 KV heads x 1 query head x (128 + 2) floats x 2 splits = 8.5 MB > 8 MiB:
    # the call runs as one split (no scratch) instead of being refused, and
    # equals pqa_decode bit for bit (which at this head count takes one split
    # too), at a per-column launch (pos 1) and a whole-row launch (pos 600)
    nh = nkv = 8192
    hd, smax = 128, 601
    att = PicoAttention(1, smax, nh, nkv, hd, 0)
    att.synth_kv(0, 0, smax - 1, 8803, 0.0)
    dev = torch.device("cuda:0")
    L = _lib.lib()
    for pos in (1, 600):
        print(f"noalloc one split, pos {pos}", flush=True)
        q, k, v = (torch.from_numpy(x).to(dev) for x in O.step_inputs(8803, 0, pos, nh, nkv, hd))
        outs = []
        for fn in (L.pqa_decode, L.pqa_decode_noalloc):
            out = torch.zeros(nh * hd, device=dev)
            rc = fn(att.handle, 0, pos, _ptr(q), _ptr(k), _ptr(v), _ptr(out))
            assert rc == _lib.PQA_OK, att.last_error()
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
        assert_bits_equal(outs[1].view(np.uint32), outs[0].view(np.uint32), f"noalloc vs decode at pos {pos}")
    att.close()
