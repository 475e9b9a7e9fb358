"""The device fp32 -> fp16 conversion the K/V append uses (f32_to_f16_ref,
exported as pqa_fp32_to_fp16) bit for bit against the oracle's, which is
pinned to the reference's fp32_to_fp16 (cpp/quant.hpp:102-135) on all 2^32
inputs and to a closed form: here on every one of the 2^32 fp32 bit patterns
(overflow to +-inf, NaN -> sign|0x7E00, fp32 subnormals -> +-0, the fp16
subnormal band, exact ties away from zero), plus the named special values."""
import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention  # noqa: E402

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


def _device_narrow(att, bits_i32):
    dst = torch.empty(bits_i32.numel(), dtype=torch.int16, device=bits_i32.device)
    att.fp32_to_fp16(bits_i32.view(torch.float32), dst)
    torch.cuda.synchronize()
    return dst.cpu().numpy().view(np.uint16)


def test_device_narrow_special_values():
    att = PicoAttention(1, 8, 2, 1, 64)
    f = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 65504.0, 65519.99, 65520.0, -65520.0, 1e30,
                  1e-8, -1e-8, 1e-40, -1e-40, 2.0 ** -25, 2.0 ** -24, 2.0 ** -14, 1.0, -2.5,
                  1.0 + 2.0 ** -11, -(1.0 + 2.0 ** -11), 1.0 + 3 * 2.0 ** -11], dtype=np.float32)
    bits = torch.from_numpy(f.view(np.int32).copy()).cuda()
    got = _device_narrow(att, bits)
    want = O.fp32_to_fp16(f)
    assert [int(x) for x in got] == [int(x) for x in want]
    # the named cases, as the reference rounds them
    assert [int(x) for x in got[:11]] == [0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0xFE00, 0x7BFF, 0x7BFF,
                                          0x7C00, 0xFC00, 0x7C00]
    assert [int(x) for x in got[11:15]] == [0x0000, 0x8000, 0x0000, 0x8000]  # fp32 subnormals -> signed zero
    assert [int(x) for x in got[20:]] == [0x3C01, 0xBC01, 0x3C02]  # ties away from zero
    att.close()


def test_device_narrow_all_2_32_inputs():
    att = PicoAttention(1, 8, 2, 1, 64)
    dev = torch.device("cuda:0")
    for c in range((1 << 32) // CHUNK):
        print(f"fp16 narrow chunk {c}", flush=True)
        first = c * CHUNK
        u = torch.arange(first, first + CHUNK, dtype=torch.int64, device=dev)
        bits = torch.where(u >= (1 << 31), u - (1 << 32), u).to(torch.int32)
        got = _device_narrow(att, bits)
        del u, bits
        want = O.fp32_bits_to_fp16(first, CHUNK, cpu_threads())
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (f"{bad.size} mismatches in chunk {c}; first input bits {first + int(bad[0]):#010x}: "
                               f"{int(got[bad[0]]):#06x} vs {int(want[bad[0]]):#06x}")
    att.close()
