"""The oracle against golden vectors written by the reference's own Model::forward
(tests/golden/make_goldens.py; the -ffp-contract=off build). Bit-exact:
attention outputs, appended K/V rows, RoPE rows and the SHA-256 of whole
output sets and caches."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
from conftest import cpu_threads

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "goldens.json")) as f:
    INDEX = json.load(f)
CASES = {c["name"]: c for c in INDEX["cases"]}


def load(c):
    with np.load(os.path.join(GOLDEN, c["file"])) as z:
        return {k: z[k] for k in z.files}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), np.asarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


def oracle_case(c):
    """Runs the oracle on a golden case's regenerated inputs."""
    nh, nkv, hd, smax, seed = c["nh"], c["nkv"], c["hd"], c["smax"], c["seed"]
    kvd = nkv * hd
    style = 0 if c["qwen"] else 1
    shp = O.shape(nh, nkv, hd, smax, style)
    qn = kn = None
    if c["qk"]:
        qn, kn = O.qk_norm_weights(seed, 0, hd)
    if c["kind"] == "decode":
        pos = c["pos"]
        kc = np.zeros((pos + 1, kvd), np.uint16)
        vc = np.zeros((pos + 1, kvd), np.uint16)
        kc[:pos], vc[:pos] = O.synth_kv_rows(seed, 0, kvd, 0, pos, c["outlier"], cpu_threads())
        cos, sin = O.rope_rows(c["base"], hd, pos, 1)
        q, k, v = O.step_inputs(seed, 0, 0, nh, nkv, hd)
        out = O.attn_step(shp, pos, q, k, v, qn, kn, cos[0], sin[0], kc, vc, cpu_threads())
        return {"out": out, "k_row": kc[pos], "v_row": vc[pos], "cos_row": cos[0], "sin_row": sin[0]}
    start, n = c["start"], c["n"]
    kc = np.zeros((smax, kvd), np.uint16)
    vc = np.zeros((smax, kvd), np.uint16)
    if start:
        kc[:start], vc[:start] = O.synth_kv_rows(seed, 0, kvd, 0, start, c["outlier"], cpu_threads())
    cos, sin = O.rope_table(c["base"], hd, smax)
    q, k, v = O.batch_inputs(seed, 0, 0, n, nh, nkv, hd)
    outs = O.prefill(shp, start, q, k, v, qn, kn, cos, sin, kc, vc, serial=False, n_threads=cpu_threads())
    return {"outs": outs, "kc": kc[:start + n], "vc": vc[:start + n]}


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_reproduces_reference_goldens(name):
    c = CASES[name]
    g = load(c)
    r = oracle_case(c)
    if c["kind"] == "decode":
        for key in ("out", "k_row", "v_row", "cos_row", "sin_row"):
            assert bits_equal(r[key], g[key]), f"{name}: {key} differs"
    else:
        sample = c["sample"]
        start = c["start"]
        assert bits_equal(r["outs"][sample], g["out_rows"]), f"{name}: sampled output rows differ"
        assert sha(r["outs"]) == c["outs_sha256"], f"{name}: output set hash differs"
        assert sha(r["kc"]) == c["k_cache_sha256"] and sha(r["vc"]) == c["v_cache_sha256"], f"{name}: cache hash"
        assert bits_equal(r["kc"][[start + s for s in sample]], g["k_rows"])


def test_golden_index_records_shipped_build_variance():
    # The reference's shipped flags contract a*b+c into FMAs on this host; the
    # resulting K rows differ from the bit-exact target in a few elements per
    # ten thousand and outputs by < 1e-4. Recorded by the generator.
    for c in INDEX["cases"]:
        d = c["a_vs_b"]
        assert d["out_max_abs"] < 1e-4
        if "k_cache_elems" in d:
            assert d["k_cache_elems_differing"] < 1e-3 * d["k_cache_elems"]
