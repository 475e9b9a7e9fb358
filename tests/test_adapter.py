"""The forward-loop adapter without a GPU: include/pqa_forward.hpp compiles
warning-free as C++17 against libpqa.so, turns a refused call into
pqa_fwd::Error with the library's code and message, and the compiled demo
(picolm_qwen_amd/adapter/forward_demo.cpp) loads and reports errors through its
C entry point. The GPU half is tests/test_gpu_forward.py."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from adapter_cases import DEMO, Model, demo_lib
from picolm_qwen_amd import _lib
from picolm_qwen_amd._build import LIB

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = r"""
#include "pqa_forward.hpp"
#include <cstdio>
#include <cstring>
#include <vector>

int main() {
    pqa_fwd::Dims d;
    d.n_layers = 2;
    d.n_embd = 512;
    d.n_heads = 8;
    d.n_kv_heads = 2;
    d.head_dim = 514;  // above 512: refused by pqa_create before any device call
    d.max_seq_len = 16;
    try {
        pqa_fwd::Attention a(d);
        std::vector<float> x(512), xb(512);
        auto norm = [](int, float* o, const float* i) { std::memcpy(o, i, 512 * sizeof(float)); };
        auto ffn = [](int, float*) {};
        pqa_fwd::forward_layers(a, 0, x.data(), xb.data(), norm, ffn);
        pqa_fwd::forward_batch_layers(a, 0, 1, x.data(), xb.data(), norm, ffn);
        return 1;
    } catch (const pqa_fwd::Error& e) {
        if (e.code != PQA_ERR_UNSUPPORTED || !std::strstr(e.what(), "head_dim")) return 2;
    }
    std::printf("adapter ok\n");
    return 0;
}
"""


def test_forward_header_compiles_and_reports_errors(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ not installed")
    src = tmp_path / "loop.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "loop"
    libdir = os.path.dirname(LIB)
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{ROOT}/include", str(src),
                    "-o", str(exe), f"-L{libdir}", "-lpqa", f"-Wl,-rpath,{libdir}"], check=True, capture_output=True,
                   text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stderr[-2000:])
    assert "adapter ok" in out.stdout


def test_demo_library_is_built_and_reports_errors():
    assert os.path.exists(DEMO), "run __graft_entry__.build()"
    m = Model(1, n_layers=1, head_dim=514)
    xp = np.zeros((2, m.n), np.float32)
    xd = np.zeros((1, m.n), np.float32)
    rc, msg = m.run_demo(xp, xd)
    assert rc == _lib.PQA_ERR_UNSUPPORTED and "head_dim" in msg, (rc, msg)
    assert hasattr(demo_lib(), "pqaf_demo_run")
