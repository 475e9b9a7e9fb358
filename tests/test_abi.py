"""The C ABI without a GPU: libpqa.so loads, exports every function declared in
include/pqa.h, validates arguments before touching the device, reports errors
through pqa_last_error, and its host-side RoPE table equals the reference's."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle as O
from picolm_qwen_amd import _lib
from picolm_qwen_amd._build import LIB

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "pqa.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pqa_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built_in_tree():
    assert os.path.exists(LIB), "run __graft_entry__.build()"


def test_exports_every_declared_function():
    L = C.CDLL(LIB)
    names = header_functions()
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert sorted(_lib.EXPORTS) == names


def test_create_rejects_bad_shapes_before_any_device_call():
    L = _lib.lib()
    h = C.c_void_p()
    tab = np.zeros(64 * 48, np.float32)
    p = tab.ctypes.data_as(C.c_void_p)
    assert L.pqa_create(C.byref(h), 1, 64, 8, 2, 514, 0, p, p) == _lib.PQA_ERR_UNSUPPORTED
    assert b"head_dim" in L.pqa_last_error(None)
    assert L.pqa_create(C.byref(h), 1, 64, 8, 2, 95, 0, p, p) == _lib.PQA_ERR_UNSUPPORTED
    assert L.pqa_create(C.byref(h), 1, 64, 8, 2, 0, 0, p, p) == _lib.PQA_ERR_UNSUPPORTED
    assert L.pqa_create(C.byref(h), 1, 64, 6, 4, 64, 0, p, p) == _lib.PQA_ERR_ARG
    assert b"multiple" in L.pqa_last_error(None)
    # more query heads per KV head than the decode launch's 16-bit field holds
    assert L.pqa_create(C.byref(h), 1, 64, 65536, 1, 64, 0, p, p) == _lib.PQA_ERR_UNSUPPORTED
    assert not h.value
    assert L.pqa_create(C.byref(h), 1, 64, 8, 2, 64, 3, p, p) == _lib.PQA_ERR_ARG
    assert L.pqa_create(C.byref(h), 0, 64, 8, 2, 64, 0, p, p) == _lib.PQA_ERR_ARG
    assert L.pqa_create(C.byref(h), 1, 64, 8, 2, 64, 0, None, None) == _lib.PQA_ERR_ARG
    assert L.pqa_create(None, 1, 64, 8, 2, 64, 0, p, p) == _lib.PQA_ERR_ARG


def test_null_context_calls_fail_cleanly():
    L = _lib.lib()
    assert L.pqa_decode(None, 0, 0, None, None, None, None) == _lib.PQA_ERR_ARG
    assert L.pqa_prefill(None, 0, 0, 1, None, None, None, None) == _lib.PQA_ERR_ARG
    assert L.pqa_sync(None) == _lib.PQA_ERR_ARG
    assert L.pqa_kvc_save(None, b"/nonexistent/x.kvc", 1) == _lib.PQA_ERR_ARG
    assert L.pqa_kvc_load(None, b"/nonexistent/x.kvc") == 0
    for setter in (L.pqa_set_token_projection, L.pqa_set_out_projection, L.pqa_set_batch_projection,
                   L.pqa_set_prefill_precision):
        assert setter(None, 1) == _lib.PQA_ERR_ARG
    assert b"ctx is NULL" in L.pqa_last_error(None)
    assert L.pqa_stream(None) is None
    L.pqa_destroy(None)


@pytest.mark.parametrize("base,hd", [(1e4, 64), (1e6, 128)])
def test_host_rope_table_equals_oracle_and_reference_formula(base, hd):
    from picolm_qwen_amd import rope_table
    c, s = rope_table(base, hd, 300)
    oc, os_ = O.rope_table(base, hd, 300)
    assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def test_python_wrapper_raises_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from picolm_qwen_amd import PicoAttention, PQAError
    with pytest.raises(PQAError):
        PicoAttention(1, 64, 8, 2, 64)


CALLER = r"""
#include "pqa.h"
#include <stdio.h>
#include <string.h>
#include <math.h>

int main(void) {
    pqa_ctx* ctx = NULL;
    float tab[64 * 48] = {0};
    /* the reference's forward loop would create one context per model; a bad
       head_dim is refused before any device call */
    int rc = pqa_create(&ctx, 1, 64, 8, 2, 514, PQA_ROPE_NEOX_HALF, tab, tab);
    if (rc != PQA_ERR_UNSUPPORTED || ctx != NULL) return 1;
    if (!strstr(pqa_last_error(NULL), "head_dim")) return 2;
    if (pqa_decode(NULL, 0, 0, NULL, NULL, NULL, NULL) != PQA_ERR_ARG) return 3;
    float c[4 * 32], s[4 * 32];
    pqa_rope_table(10000.0f, 64, 4, c, s);
    for (int pos = 0; pos < 4; pos++)
        for (int i = 0; i < 32; i++) {
            float theta = (float)pos / powf(10000.0f, (float)(2 * i) / 64.0f);
            if (c[pos * 32 + i] != cosf(theta) || s[pos * 32 + i] != sinf(theta)) return 4;
        }
    printf("caller ok\n");
    return 0;
}
"""


@pytest.mark.parametrize("compiler,std,ext", [("g++", "-std=c++17", "cpp"), ("gcc", "-std=c11", "c")])
def test_header_compiles_and_links_from_c_and_cpp(tmp_path, compiler, std, ext):
    # The reference's forward loop is C++17; a C caller works too. The header
    # must compile warning-free in both and every call must resolve in libpqa.so.
    import shutil
    import subprocess
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    src = tmp_path / f"caller.{ext}"
    src.write_text(CALLER)
    exe = tmp_path / "caller"
    libdir = os.path.dirname(LIB)
    cmd = [compiler, std, "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{ROOT}/include", str(src), "-o", str(exe),
           f"-L{libdir}", "-lpqa", f"-Wl,-rpath,{libdir}", "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stderr[-2000:])
    assert "caller ok" in out.stdout
