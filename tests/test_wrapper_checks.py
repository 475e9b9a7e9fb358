"""Host-side argument checks of the Python mirror (no GPU): every device
argument is checked for dtype, contiguity, size and device, and host weight
arrays for their byte size, before libpqa.so is called. A tensor that fails
any of these would make a kernel read or write outside its buffer."""
import numpy as np
import pytest

from picolm_qwen_amd import PicoAttention
from picolm_qwen_amd.attention import _dev_ptr, _gguf_row_bytes

torch = pytest.importorskip("torch")

NL, NH, NKV, HD, EMBD = 2, 8, 2, 64, 512
Q_DIM, KV_DIM = NH * HD, NKV * HD


def detached(qkv_layers=(0,), out_layers=(0,)):
    """A PicoAttention whose checks run but which holds no context: a call
    that got past its checks would raise RuntimeError (no handle), never reach
    the library."""
    a = PicoAttention.__new__(PicoAttention)
    a._h = None
    a.n_layers, a.max_seq_len = NL, 64
    a.n_heads, a.n_kv_heads, a.head_dim = NH, NKV, HD
    a.q_dim, a.kv_dim = Q_DIM, KV_DIM
    a.rope_style = 0
    a._qkv_embd = [EMBD if l in qkv_layers else 0 for l in range(NL)]
    a._out_rows = [EMBD if l in out_layers else 0 for l in range(NL)]
    return a


def f32(*shape):
    return torch.zeros(shape, dtype=torch.float32)


def test_dev_ptr_rejects_each_kind_of_bad_tensor():
    with pytest.raises(ValueError, match="float32"):
        _dev_ptr(torch.zeros(8, dtype=torch.float16), "float32", 8)
    with pytest.raises(ValueError, match="contiguous"):
        _dev_ptr(torch.zeros(4, 4).t(), "float32", 16)
    with pytest.raises(ValueError, match="elements"):
        _dev_ptr(f32(7), "float32", 8)
    with pytest.raises(ValueError, match="GPU"):
        _dev_ptr(f32(8), "float32", 8)
    with pytest.raises(ValueError, match="torch tensor"):
        _dev_ptr(np.zeros(8, np.float32), "float32", 8)


@pytest.mark.parametrize("call", [
    lambda a: a.qkv_project(0, f32(EMBD + 1)),                     # wrong width
    lambda a: a.qkv_project(0, torch.zeros(EMBD, dtype=torch.float16)),
    lambda a: a.qkv_project(0, f32(EMBD), q=f32(Q_DIM - 4)),       # short output
    lambda a: a.forward_x(0, 3, f32(2 * EMBD)),
    lambda a: a.out_project(0, f32(Q_DIM), f32(EMBD - 1)),          # short residual
    lambda a: a.out_project(0, f32(Q_DIM + 1), f32(EMBD)),
    lambda a: a.attention_block(0, 3, f32(EMBD), f32(2 * EMBD)),
    lambda a: a.qkv_project_batch(0, f32(4, EMBD + 8)),             # xb.shape[1] != n_embd
    lambda a: a.qkv_project_batch(0, f32(4 * EMBD)),                # not [n_tok][n_embd]
    lambda a: a.forward_batch_x(0, 0, f32(4, EMBD), out=f32(3, Q_DIM)),
    lambda a: a.forward_batch_x(0, 0, torch.zeros(4, 2 * EMBD)[:, ::2]),
    lambda a: a.qkv_project(1, f32(EMBD)),                         # layer without weights
    lambda a: a.out_project(1, f32(Q_DIM), f32(EMBD)),
    lambda a: a.qkv_project(5, f32(EMBD)),                         # layer out of range
    lambda a: a.forward(0, 3, f32(Q_DIM), f32(KV_DIM), f32(KV_DIM + 1)),
    lambda a: a.forward(0, 3, f32(Q_DIM), f32(KV_DIM), f32(KV_DIM), out=f32(Q_DIM - 1)),
    lambda a: a.forward_batch(0, 0, f32(3, Q_DIM), f32(3, KV_DIM), f32(2, KV_DIM)),
    lambda a: a.forward(0, 3, np.zeros(Q_DIM, np.float32), np.zeros(KV_DIM, np.float32),
                        np.zeros(KV_DIM, np.float32), out=np.zeros(Q_DIM - 1, np.float32)),
    lambda a: a.forward(0, 3, np.zeros(Q_DIM, np.float32), np.zeros(KV_DIM, np.float32),
                        np.zeros(KV_DIM, np.float32), out=np.zeros(Q_DIM, np.float64)),
    lambda a: a.fp32_to_fp16(f32(16), torch.zeros(15, dtype=torch.int16)),
], ids=lambda c: None)
def test_device_calls_raise_before_the_library(call):
    with pytest.raises(ValueError):
        call(detached())


def q4k_rows(rows, n):
    return np.zeros((rows, _gguf_row_bytes(13, n)), np.uint8)


def test_weight_arrays_are_checked_against_rows_times_row_bytes():
    a = detached(qkv_layers=(), out_layers=())
    ok = (q4k_rows(Q_DIM, EMBD), 13, q4k_rows(KV_DIM, EMBD), 13, q4k_rows(KV_DIM, EMBD), 13)
    short_q = (q4k_rows(Q_DIM - 1, EMBD),) + ok[1:]
    with pytest.raises(ValueError, match="wq"):
        a.set_qkv_weights(0, EMBD, *short_q)
    narrow_v = ok[:4] + (q4k_rows(KV_DIM, EMBD)[:, :-1].copy(), 13)
    with pytest.raises(ValueError, match="wv"):
        a.set_qkv_weights(0, EMBD, *narrow_v)
    with pytest.raises(ValueError, match="bk"):
        a.set_qkv_weights(0, EMBD, *ok, bk=np.zeros(KV_DIM - 1, np.float32), bk_type=1)
    with pytest.raises(ValueError, match="bq"):
        a.set_qkv_weights(0, EMBD, *ok, bq=np.zeros(Q_DIM // 2 - 1, np.float32), bq_type=2)
    with pytest.raises(ValueError, match="wo"):
        a.set_out_weights(0, EMBD, q4k_rows(EMBD - 1, Q_DIM), 13)
    with pytest.raises(ValueError, match="bo"):
        a.set_out_weights(0, EMBD, q4k_rows(EMBD, Q_DIM), 13, bo=np.zeros(EMBD - 1, np.float32), bo_type=1)
    # well-sized arrays pass every check and reach the (absent) context
    with pytest.raises(RuntimeError, match="destroyed"):
        a.set_qkv_weights(0, EMBD, *ok, bq=np.zeros(Q_DIM, np.float16), bq_type=2)
    with pytest.raises(RuntimeError, match="destroyed"):
        a.set_out_weights(0, EMBD, q4k_rows(EMBD, Q_DIM), 13)


@pytest.mark.parametrize("wtype,n,want", [(1, 64, 256), (2, 64, 128), (3, 64, 36), (9, 64, 68),
                                          (13, 512, 288), (15, 512, 420), (13, 100, None), (7, 64, None)])
def test_gguf_row_bytes(wtype, n, want):
    # block geometry of cpp/quant.hpp:33-63 (Q4_K 144 B, Q6_K 210 B per 256)
    assert _gguf_row_bytes(wtype, n) == want
