#!/usr/bin/env python3
"""Writes the golden vectors of tests/golden/ by running the reference's own
attention code (rain1201/picolm_qwen Model::forward, compiled from
/root/reference/cpp by oracle/Makefile into oracle/_ref/libref_{A,B}.so).

Run in the build container only (the GPU host has no reference tree):
    make -C oracle ref && python tests/golden/make_goldens.py

Inputs are not stored: they are regenerated from seeds with the oracle's
SplitMix64/Box-Muller generator (oracle/pqa_oracle.h). Stored per case:
outputs of the -ffp-contract=off build (B, the bit-exact target), the
appended K/V rows, the RoPE rows used, SHA-256 of large arrays, and how far the
reference's shipped-flags build (A, FMA contraction) is from B.
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

# name, n_heads, n_kv, head_dim, max_seq_len, rope_qwen, rope_base, qk_norm, kind, args
CASES = [
    # decode at pos with seeded history rows 0..pos-1
    dict(name="tinyllama_decode_pos511", nh=32, nkv=4, hd=64, smax=512, qwen=False, base=1e4, qk=False,
         kind="decode", pos=511, outlier=0.0, seed=101),
    dict(name="qwen3_1.7b_decode_pos32767", nh=16, nkv=8, hd=128, smax=32768, qwen=True, base=1e6, qk=True,
         kind="decode", pos=32767, outlier=0.0, seed=103),
    dict(name="qwen3_8b_decode_pos131071", nh=32, nkv=8, hd=128, smax=131072, qwen=True, base=1e6, qk=True,
         kind="decode", pos=131071, outlier=0.01, seed=105),
    dict(name="qwen2.5_decode_pos0", nh=14, nkv=2, hd=64, smax=64, qwen=True, base=1e6, qk=False,
         kind="decode", pos=0, outlier=0.0, seed=106),
    dict(name="llama_block8_qknorm_g3_pos150", nh=12, nkv=4, hd=128, smax=200, qwen=False, base=1e4, qk=True,
         kind="decode", pos=150, outlier=0.0, seed=107),
    # token-by-token steps from `start` (history 0..start-1 seeded): the prefill loop
    dict(name="qwen2.5_sweep_4096", nh=14, nkv=2, hd=64, smax=4096, qwen=True, base=1e6, qk=False,
         kind="steps", start=0, n=4096, outlier=0.0, seed=102, sample=[0, 1, 2, 63, 511, 2047, 4095]),
    dict(name="qwen3_4b_prefill_2048", nh=32, nkv=8, hd=128, smax=2048, qwen=True, base=1e6, qk=True,
         kind="steps", start=0, n=2048, outlier=0.0, seed=104, sample=[0, 1, 17, 1000, 2047]),
    dict(name="qwen3_prefill_start37_n200", nh=16, nkv=8, hd=128, smax=512, qwen=True, base=1e6, qk=True,
         kind="steps", start=37, n=200, outlier=0.0, seed=108, sample=[0, 99, 199]),
]


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_case(c, variant):
    nh, nkv, hd, smax = c["nh"], c["nkv"], c["hd"], c["smax"]
    kvd = nkv * hd
    seed = c["seed"]
    ref = O.RefModel(nh, nkv, hd, smax, c["base"], c["qwen"], c["qk"], variant)
    try:
        if c["qk"]:
            qn, kn = O.qk_norm_weights(seed, 0, hd)
            ref.set_qk_norm(qn, kn)
        res = {}
        if c["kind"] == "decode":
            pos = c["pos"]
            kh, vh = O.synth_kv_rows(seed, 0, kvd, 0, pos, c["outlier"], 8)
            ref.set_cache_rows(0, kh, vh)
            del kh, vh
            q, k, v = O.step_inputs(seed, 0, 0, nh, nkv, hd)
            res["out"] = ref.step(pos, q, k, v)
            res["k_row"], res["v_row"] = ref.cache_rows(pos, 1)
            res["cos_row"], res["sin_row"] = ref.rope_rows(pos, 1)
        else:
            start, n = c["start"], c["n"]
            if start:
                kh, vh = O.synth_kv_rows(seed, 0, kvd, 0, start, c["outlier"], 8)
                ref.set_cache_rows(0, kh, vh)
            q, k, v = O.batch_inputs(seed, 0, 0, n, nh, nkv, hd)
            outs = np.empty((n, nh * hd), np.float32)
            for i in range(n):
                outs[i] = ref.step(start + i, q[i], k[i], v[i])
            res["outs_sha256"] = sha(outs)
            res["out_rows"] = outs[c["sample"]]
            kc, vc = ref.cache_rows(0, start + n)
            res["k_cache_sha256"] = sha(kc)
            res["v_cache_sha256"] = sha(vc)
            res["k_rows"] = kc[[start + s for s in c["sample"]]]
            res["v_rows"] = vc[[start + s for s in c["sample"]]]
            res["_outs"], res["_kc"] = outs, kc
        return res
    finally:
        ref.close()


def main():
    if not O.RefModel.available("B") or not O.RefModel.available("A"):
        sys.exit("build the reference harness first: make -C oracle ref")
    index = {"generator": "oracle SplitMix64 + Box-Muller (oracle/pqa_oracle.h)",
             "reference": "rain1201/picolm_qwen cpp/model.hpp Model::forward via oracle/ref_harness.cpp",
             "bit_exact_build": "B: -O3 -std=c++17 -march=native -ffp-contract=off",
             "shipped_build": "A: -O3 -std=c++17 -march=native (GCC default -ffp-contract=fast)",
             "cases": []}
    for c in CASES:
        t0 = time.time()
        b = run_case(c, "B")
        a = run_case(c, "A")
        meta = {k: v for k, v in c.items()}
        arrays = {}
        if c["kind"] == "decode":
            arrays = {"out": b["out"], "k_row": b["k_row"][0], "v_row": b["v_row"][0],
                      "cos_row": b["cos_row"][0], "sin_row": b["sin_row"][0]}
            meta["a_vs_b"] = {"out_max_abs": float(np.abs(a["out"] - b["out"]).max()),
                              "k_row_elems_differing": int((a["k_row"] != b["k_row"]).sum()),
                              "v_row_elems_differing": int((a["v_row"] != b["v_row"]).sum())}
        else:
            arrays = {"out_rows": b["out_rows"], "k_rows": b["k_rows"], "v_rows": b["v_rows"]}
            meta["outs_sha256"] = b["outs_sha256"]
            meta["k_cache_sha256"] = b["k_cache_sha256"]
            meta["v_cache_sha256"] = b["v_cache_sha256"]
            meta["a_vs_b"] = {"out_max_abs": float(np.abs(a["_outs"] - b["_outs"]).max()),
                              "k_cache_elems_differing": int((a["_kc"] != b["_kc"]).sum()),
                              "k_cache_elems": int(b["_kc"].size)}
        fname = c["name"] + ".npz"
        np.savez_compressed(os.path.join(HERE, fname), **arrays)
        meta["file"] = fname
        index["cases"].append(meta)
        print(f"{c['name']}: {time.time() - t0:.1f}s  A-vs-B {meta['a_vs_b']}", flush=True)
    with open(os.path.join(HERE, "goldens.json"), "w") as f:
        json.dump(index, f, indent=1)


if __name__ == "__main__":
    main()
