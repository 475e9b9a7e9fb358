"""pqa_decode_noalloc captured into a HIP graph (picolm_qwen_amd.hipgraph) and
replayed: every replay, with eager work and synchronisations of the program
between replays, gives pqa_decode's outputs bit for bit, for one-launch
per-column steps, split + merge steps and whole-row workgroups; and pqa_prefill
(which allocates nothing) the same way."""
import ctypes as C

import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention, _lib  # noqa: E402
from picolm_qwen_amd.hipgraph import Graph  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ptr(t):
    return C.c_void_p(t.data_ptr())


@pytest.mark.parametrize("nh,nkv,hd,pos", [
    (14, 2, 64, 5),        # one split per column, one launch
    (14, 2, 64, 1500),     # per-column splits + the one-wave merge launch
    (16, 8, 128, 8191),    # whole-row workgroups + the merge launch
])
def test_graph_replays_equal_eager_decode(nh, nkv, hd, pos):
    print(f"graph replay {nh}/{nkv}/{hd} pos {pos}", flush=True)
    n_layers, seed = 2, 9100 + pos
    cos, sin = O.rope_table(1e6, hd, pos + 1)
    att = PicoAttention(n_layers, pos + 1, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    for layer in range(n_layers):
        att.set_qk_norm(layer, *O.qk_norm_weights(seed, layer, hd))
        att.synth_kv(layer, 0, pos, seed + layer, 0.01)
    L = _lib.lib()
    ins = [tuple(torch.from_numpy(x).to(DEV) for x in O.step_inputs(seed, layer, pos, nh, nkv, hd))
           for layer in range(n_layers)]
    want = [torch.zeros(nh * hd, device=DEV) for _ in range(n_layers)]
    got = [torch.zeros(nh * hd, device=DEV) for _ in range(n_layers)]
    torch.cuda.synchronize()
    for layer in range(n_layers):
        q, k, v = ins[layer]
        assert L.pqa_decode(att.handle, layer, pos, _ptr(q), _ptr(k), _ptr(v), _ptr(want[layer])) == 0
    att.sync()
    stream = L.pqa_stream(att.handle)

    def step():
        for layer in range(n_layers):
            q, k, v = ins[layer]
            rc = L.pqa_decode_noalloc(att.handle, layer, pos, _ptr(q), _ptr(k), _ptr(v), _ptr(got[layer]))
            assert rc == 0, att.last_error()

    g = Graph(stream, step)
    x = torch.randn(512, 512, device=DEV)
    for rep in range(4):
        for t in got:
            t.zero_()
        y = x @ x  # the program's own eager work between replays
        torch.cuda.synchronize()
        g.launch(stream)
        att.sync()
        torch.cuda.synchronize()
        for layer in range(n_layers):
            assert torch.equal(got[layer].view(torch.int32), want[layer].view(torch.int32)), (rep, layer)
        assert torch.isfinite(y).all()
    g.close()
    att.close()


def test_graph_replays_equal_eager_prefill():
    # pqa_prefill of two layers (Qwen3-4B heads, a 40-row history) captured
    # and replayed with the new cache rows cleared between replays: every
    # replay rewrites them, and its outputs and rows equal the eager call's
    print("graph replay prefill", flush=True)
    nh, nkv, hd, smax, start, n, seed = 32, 8, 128, 512, 40, 300, 9200
    cos, sin = O.rope_table(1e6, hd, smax)
    att = PicoAttention(2, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin)
    for layer in range(2):
        att.set_qk_norm(layer, *O.qk_norm_weights(seed, layer, hd))
        att.synth_kv(layer, 0, start, seed + layer, 0.0)
    L = _lib.lib()
    ins = [tuple(torch.from_numpy(x).to(DEV) for x in O.batch_inputs(seed, layer, start, n, nh, nkv, hd))
           for layer in range(2)]
    want = [torch.zeros(n, nh * hd, device=DEV) for _ in range(2)]
    got = [torch.zeros(n, nh * hd, device=DEV) for _ in range(2)]
    torch.cuda.synchronize()
    for layer in range(2):
        q, k, v = ins[layer]
        assert L.pqa_prefill(att.handle, layer, start, n, _ptr(q), _ptr(k), _ptr(v), _ptr(want[layer])) == 0
    att.sync()
    rows = [att.kv_download(layer, start, n) for layer in range(2)]
    zeros = np.zeros((n, nkv * hd), np.uint16)
    stream = L.pqa_stream(att.handle)

    def step():
        for layer in range(2):
            q, k, v = ins[layer]
            rc = L.pqa_prefill(att.handle, layer, start, n, _ptr(q), _ptr(k), _ptr(v), _ptr(got[layer]))
            assert rc == 0, att.last_error()

    g = Graph(stream, step)
    for rep in range(3):
        for layer in range(2):
            got[layer].zero_()
            att.kv_upload(layer, start, zeros, zeros)
        torch.cuda.synchronize()
        g.launch(stream)
        att.sync()
        for layer in range(2):
            assert torch.equal(got[layer].view(torch.int32), want[layer].view(torch.int32)), (rep, layer)
            gk, gv = att.kv_download(layer, start, n)
            assert np.array_equal(gk, rows[layer][0]) and np.array_equal(gv, rows[layer][1]), (rep, layer)
    g.close()
    att.close()
