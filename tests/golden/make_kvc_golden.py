#!/usr/bin/env python3
"""Writes tests/golden/kvc_ref_l2_s8_kv128_pos5.npz: a .kvc file produced by
the reference's own kvcache_save (picolm/model.c:882-921, compiled from
/root/reference/picolm by oracle/Makefile into oracle/_ref/libref_kvc.so),
together with the caches it was written from.

Run in the build container only (the GPU host has no reference tree):
    make -C oracle ref && python tests/golden/make_kvc_golden.py

Stored: key_cache / val_cache uint16 [2][8][128] (every fp16 bit pattern is
fair game, so the rows are uniform uint16 plus NaN, inf, -0 and subnormal
codes), n_pos = 5, n_kv_heads = 2, head_dim = 64, and kvc = the file's bytes.
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "kvc_ref_l2_s8_kv128_pos5.npz")


def main():
    if not O.RefKvc.available():
        sys.exit("oracle/_ref/libref_kvc.so is not built (make -C oracle ref)")
    rng = np.random.default_rng(20260)
    n_layers, max_seq_len, n_kv, hd, n_pos = 2, 8, 2, 64, 5
    shape = (n_layers, max_seq_len, n_kv * hd)
    k = rng.integers(0, 1 << 16, shape, dtype=np.uint16)
    v = rng.integers(0, 1 << 16, shape, dtype=np.uint16)
    specials = np.array([0x7E00, 0xFFFF, 0x7C00, 0xFC00, 0x8000, 0x0001, 0x83FF, 0x0000], np.uint16)
    k[0, 0, :8] = specials
    v[1, n_pos - 1, -8:] = specials
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "golden.kvc")
        rc = O.RefKvc.save(k, v, n_kv, hd, path, n_pos)
        if rc != 0:
            sys.exit(f"kvcache_save returned {rc}")
        data = np.frombuffer(open(path, "rb").read(), np.uint8)
    np.savez(OUT, key_cache=k, val_cache=v, n_pos=n_pos, n_kv_heads=n_kv, head_dim=hd, kvc=data)
    print(f"wrote {OUT} ({data.size} file bytes)")


if __name__ == "__main__":
    main()
