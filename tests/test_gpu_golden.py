"""The HIP path against the golden vectors of the reference's own Model::forward
(tests/golden/). Inputs are regenerated from the recorded seeds; cache history
is filled on the device by the same generator. Every context here takes the
product's RoPE table (pqa_rope_table, computed with this host's libm), so the
goldens pin it end to end. Appended K/V rows and whole caches: bit-exact
(SHA-256). Attention outputs: max-abs 2e-3 / rel 1e-2, on every output row
(the oracle's full output, itself pinned by the goldens' SHA-256, gives the
rows the fixtures do not hold)."""
import functools
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads
from gpu_util import assert_bits_equal, assert_close

torch = pytest.importorskip("torch")
from picolm_qwen_amd import PicoAttention, rope_table  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "goldens.json")) as f:
    CASES = {c["name"]: c for c in json.load(f)["cases"]}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _context(c, n_layers=1):
    """A context whose RoPE table is the product's own (rope_cos=None:
    pqa_rope_table, cpp/model.hpp:1008-1017)."""
    hd = c["hd"]
    att = PicoAttention(n_layers, c["smax"], c["nh"], c["nkv"], hd, 0 if c["qwen"] else 1, rope_base=c["base"])
    if c["qk"]:
        qn, kn = O.qk_norm_weights(c["seed"], 0, hd)
        att.set_qk_norm(0, qn, kn)
    return att


@functools.lru_cache(maxsize=None)
def _oracle_steps(name):
    """The oracle's outputs for every token of a golden step sequence; their
    SHA-256 must be the one the reference's own run recorded."""
    c = CASES[name]
    nh, nkv, hd, smax, seed, start, n = c["nh"], c["nkv"], c["hd"], c["smax"], c["seed"], c["start"], c["n"]
    kvd = nkv * hd
    shp = O.shape(nh, nkv, hd, smax, 0 if c["qwen"] else 1)
    qn = kn = None
    if c["qk"]:
        qn, kn = O.qk_norm_weights(seed, 0, hd)
    kc = np.zeros((smax, kvd), np.uint16)
    vc = np.zeros((smax, kvd), np.uint16)
    if start:
        kc[:start], vc[:start] = O.synth_kv_rows(seed, 0, kvd, 0, start, c["outlier"], cpu_threads())
    cos, sin = O.rope_table(c["base"], hd, smax)
    q, k, v = O.batch_inputs(seed, 0, 0, n, nh, nkv, hd)
    outs = O.prefill(shp, start, q, k, v, qn, kn, cos, sin, kc, vc, serial=False, n_threads=cpu_threads())
    assert sha(outs) == c["outs_sha256"], f"{name}: oracle outputs differ from the reference's"
    return outs


@pytest.mark.parametrize("name", [n for n, c in CASES.items() if c["kind"] == "decode"])
def test_product_rope_table_rows_match_reference(name):
    # the table rows the reference itself used at the golden position, computed
    # here by the product's pqa_rope_table on this host
    c = CASES[name]
    with np.load(os.path.join(GOLDEN, c["file"])) as z:
        crow, srow = z["cos_row"], z["sin_row"]
    cos, sin = rope_table(c["base"], c["hd"], c["pos"] + 1)
    assert_bits_equal(cos[c["pos"]].view(np.uint32), crow.view(np.uint32), "cos row")
    assert_bits_equal(sin[c["pos"]].view(np.uint32), srow.view(np.uint32), "sin row")


@pytest.mark.parametrize("name", [n for n, c in CASES.items() if c["kind"] == "decode"])
def test_decode_matches_reference_golden(name):
    c = CASES[name]
    print(f"golden decode {name}", flush=True)
    with np.load(os.path.join(GOLDEN, c["file"])) as z:
        g = {k: z[k] for k in z.files}
    att = _context(c)
    att.synth_kv(0, 0, c["pos"], c["seed"], c["outlier"])
    q, k, v = O.step_inputs(c["seed"], 0, 0, c["nh"], c["nkv"], c["hd"])
    dev = torch.device("cuda:0")
    out = att.forward(0, c["pos"], *(torch.from_numpy(x).to(dev) for x in (q, k, v)))
    torch.cuda.synchronize()
    kr, vr = att.kv_download(0, c["pos"], 1)
    assert_bits_equal(kr[0], g["k_row"], "appended K row vs reference")
    assert_bits_equal(vr[0], g["v_row"], "appended V row vs reference")
    assert_close(out.cpu().numpy(), g["out"], what=f"{name} output vs reference")
    att.close()


@pytest.mark.parametrize("name", [n for n, c in CASES.items() if c["kind"] == "steps"])
@pytest.mark.parametrize("mode", ["prefill", "decode_steps"])
def test_steps_match_reference_golden(name, mode):
    c = CASES[name]
    print(f"golden {mode} {name}", flush=True)
    with np.load(os.path.join(GOLDEN, c["file"])) as z:
        g = {k: z[k] for k in z.files}
    start, n = c["start"], c["n"]
    att = _context(c)
    if start:
        att.synth_kv(0, 0, start, c["seed"], c["outlier"])
    q, k, v = O.batch_inputs(c["seed"], 0, 0, n, c["nh"], c["nkv"], c["hd"])
    dev = torch.device("cuda:0")
    tq, tk, tv = (torch.from_numpy(x).to(dev) for x in (q, k, v))
    if mode == "prefill":
        out = att.forward_batch(0, start, tq, tk, tv)
    else:
        out = torch.empty((n, c["nh"] * c["hd"]), dtype=torch.float32, device=dev)
        for i in range(n):
            att.forward(0, start + i, tq[i], tk[i], tv[i], out=out[i])
    torch.cuda.synchronize()
    kc, vc = att.kv_download(0, 0, start + n)
    assert sha(kc) == c["k_cache_sha256"], "K cache differs from the reference's"
    assert sha(vc) == c["v_cache_sha256"], "V cache differs from the reference's"
    got = out.cpu().numpy()
    assert_close(got[c["sample"]], g["out_rows"], what=f"{name} sampled rows vs reference")
    assert_close(got, _oracle_steps(name), what=f"{name} all {n} rows vs oracle")
    att.close()
