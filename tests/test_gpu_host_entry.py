"""The host-pointer entry points (pqa_decode_host, pqa_prefill_host), the calls
a CPU forward loop makes per layer in place of cpp/model.hpp:326-418 and
:489-593. Small payloads travel through one pinned host buffer, large ones
through two pinned 8 MiB slots that CPU threads fill while the DMA engine
drains the other; both must give the device-pointer entry's bits exactly, and
the K/V rows they append must be the same."""
import numpy as np
import pytest
import torch

import oracle as O
from picolm_qwen_amd import PicoAttention
from picolm_qwen_amd._lib import PQAError

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _pair(nh, nkv, hd, smax, seed):
    cos, sin = O.rope_table(1e6, hd, smax)
    a = [PicoAttention(1, smax, nh, nkv, hd, 0, rope_cos=cos, rope_sin=sin) for _ in range(2)]
    for att in a:
        att.set_qk_norm(0, *O.qk_norm_weights(seed, 0, hd))
    return a


def _device(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


# 300 x 20 KB of payload: past the 4 MiB one-copy buffer, one slot each way;
# 2400 tokens: 28.8 MB in (four slot fills, both slots reused) and 19.2 MB out
@pytest.mark.parametrize("n_tok", [3, 300, 2400])
def test_prefill_host_matches_device_entry(n_tok):
    nh, nkv, hd, seed = 16, 4, 128, 7301
    smax = max(512, n_tok)
    host, dev = _pair(nh, nkv, hd, smax, seed)
    q, k, v = O.batch_inputs(seed, 0, 0, n_tok, nh, nkv, hd)
    got = host.forward_batch(0, 0, q, k, v)
    want = dev.forward_batch(0, 0, _device(q), _device(k), _device(v))
    torch.cuda.synchronize()
    assert np.array_equal(got, want.cpu().numpy())
    kh, vh = host.kv_download(0, 0, n_tok)
    kd, vd = dev.kv_download(0, 0, n_tok)
    assert np.array_equal(kh, kd) and np.array_equal(vh, vd)
    host.close()
    dev.close()


def test_decode_host_successive_calls_and_a_failed_call():
    # token after token through the pinned buffer, with a prompt (which grows
    # the buffers) and a rejected call in between: every output equals the
    # device entry's, and the rejected call leaves the next one intact
    nh, nkv, hd, smax, seed = 32, 8, 128, 256, 7302
    host, dev = _pair(nh, nkv, hd, smax, seed)
    q, k, v = O.batch_inputs(seed, 0, 0, 40, nh, nkv, hd)
    host.forward_batch(0, 0, q[:32], k[:32], v[:32])
    dev.forward_batch(0, 0, _device(q[:32]), _device(k[:32]), _device(v[:32]))
    for pos in range(32, 40):
        got = host.forward(0, pos, q[pos], k[pos], v[pos])
        want = dev.forward(0, pos, _device(q[pos]), _device(k[pos]), _device(v[pos]))
        torch.cuda.synchronize()
        assert np.array_equal(got, want.cpu().numpy()), pos
        if pos == 35:
            with pytest.raises(PQAError):
                host.forward(0, smax, q[pos], k[pos], v[pos])  # pos out of range
    kh, vh = host.kv_download(0, 0, 40)
    kd, vd = dev.kv_download(0, 0, 40)
    assert np.array_equal(kh, kd) and np.array_equal(vh, vd)
    host.close()
    dev.close()


@pytest.mark.parametrize("nh,nkv,hd,pos", [
    (16, 8, 128, 8191),    # whole-row workgroups, several splits: the merge launch writes out into host memory
    (16, 8, 128, 32767),   # Qwen3-1.7B shape at its full context
    (32, 4, 64, 2047),     # hd 64, several splits
    (8, 2, 96, 3000),      # a general head size (VALU kernels, their own merge)
])
def test_decode_host_multi_split_and_general_equal_device_entry(nh, nkv, hd, pos):
    # the zero-copy host entry (kernels read q/k/v from and write out into the
    # pinned staging buffer) against the device entry at launch shapes the
    # single-split cases above do not reach: bit-equal outputs and rows
    print(f"decode host entry {nh}/{nkv}/{hd} pos {pos}", flush=True)
    seed = 7400 + pos
    host, dev = _pair(nh, nkv, hd, pos + 1, seed)
    for att in (host, dev):
        att.synth_kv(0, 0, pos, seed, 0.01)
    q, k, v = O.step_inputs(seed, 0, pos, nh, nkv, hd)
    got = host.forward(0, pos, q, k, v)
    want = dev.forward(0, pos, _device(q), _device(k), _device(v))
    torch.cuda.synchronize()
    assert np.array_equal(got, want.cpu().numpy())
    kh, vh = host.kv_download(0, pos, 1)
    kd, vd = dev.kv_download(0, pos, 1)
    assert np.array_equal(kh, kd) and np.array_equal(vh, vd)
    host.close()
    dev.close()
