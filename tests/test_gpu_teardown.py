"""Teardown order: a context destroyed while torch tensors that its calls
used are still alive, then those tensors freed, then the device synchronised.
An early build let torch record events on the context's stream for each
tensor (record_stream); freeing a tensor after pqa_destroy then recorded an
event on a destroyed stream and the process died with a segmentation fault at
exit. The calls now order torch's stream after the context stream instead
(wait_stream), so nothing refers to the context stream once it is gone."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu


def _run_and_drop(close_first):
    nh, nkv, hd, smax, pos = 32, 4, 64, 512, 300
    dev = torch.device("cuda:0")
    att = PicoAttention(1, smax, nh, nkv, hd, 1, rope_base=1e4)
    att.synth_kv(0, 0, pos, 3, 0.0)
    q, k, v = (torch.from_numpy(x).to(dev) for x in O.step_inputs(3, 0, 0, nh, nkv, hd))
    out = att.forward(0, pos, q, k, v)
    pre = att.forward_batch(0, pos + 1, q.reshape(1, -1).repeat(3, 1).contiguous(),
                            k.reshape(1, -1).repeat(3, 1).contiguous(), v.reshape(1, -1).repeat(3, 1).contiguous())
    host = out.cpu().numpy().copy()
    if close_first:
        att.close()
        del q, k, v, out, pre
    else:
        del q, k, v, out, pre
        att.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return host


@pytest.mark.parametrize("close_first", [True, False])
def test_tensors_freed_after_destroy(close_first):
    print(f"teardown close_first={close_first}", flush=True)
    a = _run_and_drop(close_first)
    b = _run_and_drop(close_first)
    assert np.isfinite(a).all() and np.array_equal(a, b)
    # the allocator and the default stream still work
    x = torch.ones(1 << 20, device="cuda:0")
    assert float(x.sum()) == float(1 << 20)


def test_context_garbage_collected_without_close():
    dev = torch.device("cuda:0")
    att = PicoAttention(1, 64, 8, 2, 64)
    q, k, v = (torch.from_numpy(x).to(dev) for x in O.step_inputs(4, 0, 0, 8, 2, 64))
    att.forward(0, 5, q, k, v)
    del att  # __del__ destroys the context; the tensors outlive it
    import gc
    gc.collect()
    del q, k, v
    torch.cuda.synchronize()
    assert float(torch.ones(16, device=dev).sum()) == 16.0
