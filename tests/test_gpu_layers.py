"""Layers above 0 at their real offsets: a Qwen3-8B-shaped context of 36
layers x 131072 positions (32/8/128, 19.3 GB of fp16 cache), each layer with
its own seed for history, inputs and QK-norm weights. Layer 35's slice starts
35 x 268 MB = 9.4 GB into each cache allocation, past every 32-bit byte
offset. Decode at the last position of layers 35, 34 and 0 against the
oracle (max-abs 2e-3 / rel 1e-2), appended rows bit-exact, and the rows of
the neighbouring layers untouched by those appends."""
import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads
from gpu_util import assert_bits_equal, assert_close

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu

NL, NH, NKV, HD, SMAX = 36, 32, 8, 128, 131072
KVD = NKV * HD
SEED = 0xC0FFEE + 5000


def layer_seed(layer):
    return SEED + 1000 * layer


def test_high_layers_past_4_gib_match_oracle():
    pos = SMAX - 1
    att = PicoAttention(NL, SMAX, NH, NKV, HD, 0, rope_base=1e6)
    layers = (35, 34, 0)
    for layer in layers:
        qn, kn = O.qk_norm_weights(layer_seed(layer), layer, HD)
        att.set_qk_norm(layer, qn, kn)
        att.synth_kv(layer, 0, pos, layer_seed(layer), 0.01)
    cos, sin = O.rope_table(1e6, HD, SMAX)
    shp = O.shape(NH, NKV, HD, SMAX, 0)
    dev = torch.device("cuda:0")
    for layer in layers:
        print(f"layer {layer} decode at pos {pos}", flush=True)
        s = layer_seed(layer)
        qn, kn = O.qk_norm_weights(s, layer, HD)
        q, k, v = O.step_inputs(s, layer, 0, NH, NKV, HD)
        out = att.forward(layer, pos, *(torch.from_numpy(x).to(dev) for x in (q, k, v)))
        torch.cuda.synchronize()
        kc = np.zeros((SMAX, KVD), np.uint16)
        vc = np.zeros((SMAX, KVD), np.uint16)
        kc[:pos], vc[:pos] = O.synth_kv_rows(s, layer, KVD, 0, pos, 0.01, cpu_threads())
        # the device history of this layer is the seeded one (checked at both ends)
        gk, gv = att.kv_download(layer, 0, 64)
        assert_bits_equal(gk, kc[:64], f"layer {layer} K history head")
        gk, gv = att.kv_download(layer, pos - 64, 64)
        assert_bits_equal(gv, vc[pos - 64:pos], f"layer {layer} V history tail")
        want = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc, cpu_threads())
        assert_close(out.cpu().numpy(), want, what=f"layer {layer} output vs oracle")
        rk, rv = att.kv_download(layer, pos, 1)
        assert_bits_equal(rk[0], kc[pos], f"layer {layer} appended K row")
        assert_bits_equal(rv[0], vc[pos], f"layer {layer} appended V row")
    # layer 33 was never written: its rows are still the zeroed cache, so no
    # append or history write of the neighbouring layers landed in it
    zk, zv = att.kv_download(33, pos - 1, 2)
    assert not zk.any() and not zv.any()
    zk, zv = att.kv_download(33, 0, 2)
    assert not zk.any() and not zv.any()
    att.close()
