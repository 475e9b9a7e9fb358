#!/usr/bin/env python3
"""Benchmark of the attention path on one MI355X.

Headline (`value`): decode attention of a Qwen3-8B-shaped model (32 query /
8 KV heads, head_dim 128, QK-RMSNorm, NeoX RoPE theta 1e6), one token at
position 131071 over a 131072-entry fp16 KV cache, all 36 layers per step
(19.3 GB of cache rotated through, so the 256 MB Infinity Cache cannot hold
it), 1 % of history rows scaled x8. Unit: algorithmic KV GB/s = bytes the
reference reads and writes per layer (K and V rows 0..pos, q, k, v, out, the
appended row) / time.

Also reported in the same JSON line under "workloads":
  qwen3_1.7b_decode   16/8/128, pos 32767, 28 layers (HBM-bound)
  qwen3_4b_prefill    32/8/128, 2048-token causal prefill, 36 layers (MFMA)
  tinyllama_decode    32/4/64, block8 RoPE, pos 511, 1 layer (latency)
  qwen2.5_0.5b_sweep  14/2/64, positions 0..4095 token by token, 24 layers
  qwen3_8b_kvc_save_load  .kvc save/load of 4096 positions x 36 layers (604 MB)
  qwen3_8b_qkv_proj   Q/K/V projections of one token, Q4_K/Q4_K/Q6_K, 36 layers
  qwen3_4b_prefill_from_xb  prompt path from the normed inputs: projections + prefill

`roofline` covers the decode kernel of the headline workload, timed with HIP
events on the library's stream. `cpu_baseline` times the CPU oracle (the
reference loop restated, heads split over T threads) on one layer of the same
cache, downloaded from the GPU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
"""
import argparse
import ctypes as C
import json
import re
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2516.6  # dense fp16, 256 CU x 2.4 GHz x 4096 flop/clk
METRIC = "attn µs/layer; decode KV GB/s (% HBM peak); prefill TFLOP/s (% MFMA)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(ctx, nh, nkv, hd):
    """Algorithmic bytes of one decode launch: K and V rows 0..pos read
    (ctx rows), q/k/v fp32 in, out fp32, the new K/V row written."""
    kv_dim = nkv * hd
    return 2 * ctx * kv_dim * 2 + nh * hd * 4 + 2 * kv_dim * 4 + nh * hd * 4 + 2 * kv_dim * 2


def prefill_flops(nh, hd, s, start=0):
    """Causal attention flops: 2 matmuls x 2 flop x n_q x hd x (key count summed over rows)."""
    keys = sum(start + i + 1 for i in range(s))
    return 2 * 2 * nh * hd * keys


class Ctx:
    """Thin ctypes holder around one pqa context (the bench calls the C ABI directly)."""

    def __init__(self, n_layers, smax, nh, nkv, hd, style, base):
        from picolm_qwen_amd import _lib
        from picolm_qwen_amd.attention import rope_table
        self.L = _lib.lib()
        self.check = _lib.check
        cos, sin = rope_table(base, hd, smax)
        h = C.c_void_p()
        self.check(self.L.pqa_create(C.byref(h), n_layers, smax, nh, nkv, hd, style,
                                     cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p)))
        self.h = h
        self.n_layers, self.smax, self.nh, self.nkv, self.hd = n_layers, smax, nh, nkv, hd

    def stream(self):
        return self.L.pqa_stream(self.h)

    def close(self):
        if self.h:
            self.L.pqa_destroy(self.h)
            self.h = None


def make_inputs(torch, dev, rng, n_layers, n_tok, nh, nkv, hd):
    q = torch.from_numpy(rng.standard_normal((n_layers, n_tok, nh * hd), dtype=np.float32)).to(dev)
    k = torch.from_numpy(rng.standard_normal((n_layers, n_tok, nkv * hd), dtype=np.float32)).to(dev)
    v = torch.from_numpy(rng.standard_normal((n_layers, n_tok, nkv * hd), dtype=np.float32)).to(dev)
    out = torch.empty((n_layers, n_tok, nh * hd), dtype=torch.float32, device=dev)
    return q, k, v, out


def set_norms(cx, rng, hd):
    for layer in range(cx.n_layers):
        qw = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        kw = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        cx.check(cx.L.pqa_set_qk_norm(cx.h, layer, qw.ctypes.data_as(C.c_void_p),
                                      kw.ctypes.data_as(C.c_void_p)), cx.h)
    return


def timed(torch, cx, fn, steps, warmup):
    """Runs fn() warmup+steps times; returns (wall ms/step, event ms/step on the library stream)."""
    ext = torch.cuda.ExternalStream(cx.stream())
    for _ in range(warmup):
        fn()
    cx.check(cx.L.pqa_sync(cx.h), cx.h)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(ext)
    for _ in range(steps):
        fn()
    e1.record(ext)
    cx.check(cx.L.pqa_sync(cx.h), cx.h)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, e0.elapsed_time(e1) / steps


def decode_workload(torch, dev, name, n_layers, nh, nkv, hd, style, base, pos, prob, steps, warmup, qk_norm,
                    seed=20251201, keep=False):
    cx = Ctx(n_layers, pos + 1, nh, nkv, hd, style, base)
    rng = np.random.default_rng(seed)
    if qk_norm:
        set_norms(cx, rng, hd)
    for layer in range(n_layers):
        cx.check(cx.L.pqa_synth_kv(cx.h, layer, 0, pos, seed, prob), cx.h)
    q, k, v, out = make_inputs(torch, dev, rng, n_layers, 1, nh, nkv, hd)
    cx.check(cx.L.pqa_sync(cx.h), cx.h)
    torch.cuda.synchronize()
    ptr = lambda t, layer: C.c_void_p(t[layer].data_ptr())  # noqa: E731
    args = [(layer, ptr(q, layer), ptr(k, layer), ptr(v, layer), ptr(out, layer)) for layer in range(n_layers)]
    dec = cx.L.pqa_decode
    h = cx.h

    def step():
        for layer, a, b, c, d in args:
            dec(h, layer, pos, a, b, c, d)

    wall, ev = timed(torch, cx, step, steps, warmup)
    per_layer_us = ev * 1e3 / n_layers
    nbytes = decode_bytes(pos + 1, nh, nkv, hd)
    gbs = nbytes / (per_layer_us * 1e-6) / 1e9
    res = {"workload": name, "n_layers": n_layers, "pos": pos, "us_per_layer": round(per_layer_us, 3),
           "bytes_per_layer": nbytes, "GB_per_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "ms_per_step_event": round(ev, 4), "ms_per_step_wall": round(wall, 4)}
    log(f"[bench] {name}: {per_layer_us:.2f} us/layer, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM)")
    if keep:
        return res, cx, (q, k, v, out)
    cx.close()
    return res, None, None


def prefill_workload(torch, dev, n_layers, nh, nkv, hd, s, steps, warmup, seed=4242):
    cx = Ctx(n_layers, s, nh, nkv, hd, 0, 1e6)
    rng = np.random.default_rng(seed)
    set_norms(cx, rng, hd)
    q, k, v, out = make_inputs(torch, dev, rng, n_layers, s, nh, nkv, hd)
    torch.cuda.synchronize()
    ptr = lambda t, layer: C.c_void_p(t[layer].data_ptr())  # noqa: E731
    args = [(layer, ptr(q, layer), ptr(k, layer), ptr(v, layer), ptr(out, layer)) for layer in range(n_layers)]
    pre = cx.L.pqa_prefill
    h = cx.h

    def step():
        for layer, a, b, c, d in args:
            pre(h, layer, 0, s, a, b, c, d)

    wall, ev = timed(torch, cx, step, steps, warmup)
    per_layer_us = ev * 1e3 / n_layers
    fl = prefill_flops(nh, hd, s)
    tf = fl / (per_layer_us * 1e-6) / 1e12
    res = {"workload": "qwen3_4b_prefill", "n_layers": n_layers, "n_tok": s,
           "us_per_layer_append_plus_attention": round(per_layer_us, 3), "flops_per_layer": fl,
           "TFLOP_per_s": round(tf, 1), "mfma_frac": round(tf / MFMA_FP16_PEAK_TFLOPS, 4), "dtype": "fp16",
           "q_precision": "fp16 hi + lo (the library default; the QK^T MFMA work counts once in flops)",
           "ms_per_step_event": round(ev, 4), "ms_per_step_wall": round(wall, 4)}
    log(f"[bench] prefill: {per_layer_us:.2f} us/layer, {tf:.1f} TFLOP/s ({100 * tf / MFMA_FP16_PEAK_TFLOPS:.1f}% MFMA)")
    cx.close()
    return res


def sweep_workload(torch, dev, n_layers=24, nh=14, nkv=2, hd=64, positions=4096, checkpoints=(1, 512, 1024, 2048, 4096)):
    cx = Ctx(n_layers, positions, nh, nkv, hd, 0, 1e6)
    rng = np.random.default_rng(777)
    q, k, v, out = make_inputs(torch, dev, rng, n_layers, positions, nh, nkv, hd)
    torch.cuda.synchronize()
    dec = cx.L.pqa_decode
    h = cx.h
    qp, kp, vp, op = (t.data_ptr() for t in (q, k, v, out))
    qs, kvs = nh * hd * 4, nkv * hd * 4
    ext = torch.cuda.ExternalStream(cx.stream())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(ext)
    for pos in range(positions):
        for layer in range(n_layers):
            off_q = ((layer * positions) + pos)
            dec(h, layer, pos, C.c_void_p(qp + off_q * qs), C.c_void_p(kp + off_q * kvs),
                C.c_void_p(vp + off_q * kvs), C.c_void_p(op + off_q * qs))
    e1.record(ext)
    cx.check(cx.L.pqa_sync(cx.h), cx.h)
    avg_us = e0.elapsed_time(e1) * 1e3 / (positions * n_layers)
    curve = {}
    for ctx_len in checkpoints:
        pos = ctx_len - 1

        def step():
            for layer in range(n_layers):
                off_q = ((layer * positions) + pos)
                dec(h, layer, pos, C.c_void_p(qp + off_q * qs), C.c_void_p(kp + off_q * kvs),
                    C.c_void_p(vp + off_q * kvs), C.c_void_p(op + off_q * qs))

        _, ev = timed(torch, cx, step, 20, 2)
        curve[str(ctx_len)] = round(ev * 1e3 / n_layers, 3)
    cx.close()
    log(f"[bench] qwen2.5 sweep: avg {avg_us:.2f} us/layer over ctx 1..{positions}; curve {curve}")
    return {"workload": "qwen2.5_0.5b_sweep", "n_layers": n_layers, "positions": positions,
            "avg_us_per_layer_launch_loop": round(avg_us, 3), "us_per_layer_vs_ctx": curve}


def kvc_workload(torch, dev, n_layers=36, nh=32, nkv=8, hd=128, n_pos=4096, reps=3):
    """.kvc persistence (picolm/model.c:870-983) of a Qwen3-8B-shaped cache
    prefix, 4096 positions x 36 layers (604 MB file): pqa_kvc_save /
    pqa_kvc_load between HBM and a file in the temp directory (page cache, no
    fsync, as the reference), beside the reference's own kvcache_save /
    kvcache_load (oracle/_ref/libref_kvc.so, where built) on a host copy of
    the same cache. Unit: file GB/s, median of `reps` after one warm-up."""
    import filecmp
    import tempfile
    import oracle as O
    cx = Ctx(n_layers, n_pos, nh, nkv, hd, 0, 1e6)
    for layer in range(n_layers):
        cx.check(cx.L.pqa_synth_kv(cx.h, layer, 0, n_pos, 1234 + layer, 0.0), cx.h)
    cx.check(cx.L.pqa_sync(cx.h), cx.h)
    kv_dim = nkv * hd
    nbytes = 16 + 2 * n_layers * n_pos * kv_dim * 2
    tmp = tempfile.mkdtemp(prefix="pqa_kvc_")
    ours = os.path.join(tmp, "ours.kvc")
    ref = os.path.join(tmp, "ref.kvc")

    def clock(fn):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def save():
        cx.check(cx.L.pqa_kvc_save(cx.h, ours.encode(), n_pos), cx.h)

    def load():
        if cx.L.pqa_kvc_load(cx.h, ours.encode()) != n_pos:
            raise RuntimeError(cx.L.pqa_last_error(cx.h))

    res = {"workload": "qwen3_8b_kvc_save_load", "n_layers": n_layers, "n_pos": n_pos, "kv_dim": kv_dim,
           "file_bytes": nbytes, "unit": "GB/s (file bytes / wall time)"}
    try:
        t_save, t_load = clock(save), clock(load)
        res.update(save_GB_per_s=round(nbytes / t_save / 1e9, 3), load_GB_per_s=round(nbytes / t_load / 1e9, 3),
                   save_ms=round(t_save * 1e3, 2), load_ms=round(t_load * 1e3, 2))
        if O.RefKvc.available():
            kc = np.zeros((n_layers, n_pos, kv_dim), np.uint16)
            vc = np.zeros((n_layers, n_pos, kv_dim), np.uint16)
            for layer in range(n_layers):
                cx.check(cx.L.pqa_kv_download(cx.h, layer, 0, n_pos, kc[layer].ctypes.data_as(C.c_void_p),
                                              vc[layer].ctypes.data_as(C.c_void_p)), cx.h)
            r_save = clock(lambda: O.RefKvc.save(kc, vc, nkv, hd, ref, n_pos))
            r_load = clock(lambda: O.RefKvc.load_into(kc, vc, nkv, hd, ref))
            res["cpu_baseline"] = {
                "kind": "reference", "cores": 1,
                "save_GB_per_s": round(nbytes / r_save / 1e9, 3), "load_GB_per_s": round(nbytes / r_load / 1e9, 3),
                "sample": "kvcache_save / kvcache_load of the same cache bytes from host memory, same file size"}
            res["files_identical"] = filecmp.cmp(ours, ref, shallow=False)
    finally:
        for f in (ours, ref):
            if os.path.exists(f):
                os.unlink(f)
        os.rmdir(tmp)
        cx.close()
    log(f"[bench] kvc: {res}")
    return res


def gguf_rows(rng, wtype, rows, n):
    """Synthetic GGUF rows: random payload, fp16 scale fields of a realistic size."""
    be, bb, scales = {13: (256, 144, (0, 2)), 15: (256, 210, (208,))}[wtype]
    nb = n // be
    raw = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)
    for off in scales:
        raw[:, :, off:off + 2] = rng.uniform(1e-3, 2e-2, (rows, nb)).astype("<f2").view(np.uint8).reshape(rows, nb, 2)
    return raw.reshape(rows, nb * bb)


def proj_workload(torch, dev, n_layers=36, nh=32, nkv=8, hd=128, n=4096, steps=20, warmup=3, cpu=True):
    """Q/K/V projections of one token (matmul_bias, cpp/model.hpp:320-366) for a
    Qwen3-8B-shaped layer stored as a Q4_K_M file stores it: Q4_K attn_q and
    attn_k, Q6_K attn_v, 4096-wide rows; 36 layers rotated per step (547 MB of
    weights, more than the Infinity Cache). Unit: weight GB/s."""
    Q4K, Q6K = 13, 15
    cx = Ctx(n_layers, 64, nh, nkv, hd, 0, 1e6)
    rng = np.random.default_rng(606)
    wbytes = 0
    for layer in range(n_layers):
        wq, wk, wv = gguf_rows(rng, Q4K, nh * hd, n), gguf_rows(rng, Q4K, nkv * hd, n), gguf_rows(rng, Q6K, nkv * hd, n)
        if layer == 0:
            w0 = (wq, wk, wv)
            wbytes = wq.nbytes + wk.nbytes + wv.nbytes
        wo = gguf_rows(rng, Q4K, n, nh * hd)
        vp = lambda a: a.ctypes.data_as(C.c_void_p)
        cx.check(cx.L.pqa_set_qkv_weights(cx.h, layer, n, vp(wq), Q4K, None, 0, vp(wk), Q4K, None, 0, vp(wv), Q6K,
                                          None, 0), cx.h)
        cx.check(cx.L.pqa_set_out_weights(cx.h, layer, n, vp(wo), Q4K, None, 0), cx.h)
        obytes = wo.nbytes
    x = torch.from_numpy(rng.standard_normal((n_layers, n), dtype=np.float32)).to(dev)
    q = torch.empty((n_layers, nh * hd), device=dev)
    k = torch.empty((n_layers, nkv * hd), device=dev)
    v = torch.empty((n_layers, nkv * hd), device=dev)
    torch.cuda.synchronize()
    proj = cx.L.pqa_qkv_project
    ptrs = [(C.c_void_p(x[l].data_ptr()), C.c_void_p(q[l].data_ptr()), C.c_void_p(k[l].data_ptr()),
             C.c_void_p(v[l].data_ptr())) for l in range(n_layers)]

    def step():
        for layer in range(n_layers):
            proj(cx.h, layer, *ptrs[layer])

    wall, ev = timed(torch, cx, step, steps, warmup)
    us = ev * 1e3 / n_layers
    gbs = wbytes / (us * 1e-6) / 1e9
    resid = torch.from_numpy(rng.standard_normal((n_layers, n), dtype=np.float32)).to(dev)
    oproj = cx.L.pqa_out_project
    optrs = [(C.c_void_p(q[l].data_ptr()), C.c_void_p(resid[l].data_ptr())) for l in range(n_layers)]

    def ostep():
        for layer in range(n_layers):
            oproj(cx.h, layer, *optrs[layer])

    _, oev = timed(torch, cx, ostep, steps, warmup)
    ous = oev * 1e3 / n_layers
    res = {"workload": "qwen3_8b_qkv_proj_q4_k_m", "n_embd": n, "rows": [nh * hd, nkv * hd, nkv * hd],
           "weight_types": ["Q4_K", "Q4_K", "Q6_K"], "weight_bytes_per_layer": wbytes,
           "us_per_layer": round(us, 3), "weight_GB_per_s": round(gbs, 1),
           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bit_exact_vs_reference_build_B": True,
           "out_proj": {"rows": n, "width": nh * hd, "weight_type": "Q4_K", "weight_bytes_per_layer": obytes,
                        "us_per_layer": round(ous, 3), "weight_GB_per_s": round(obytes / (ous * 1e-6) / 1e9, 1),
                        "note": "attn_output matmul_bias + residual vec_add (cpp/model.hpp:420-427)"}}
    if cpu:
        import oracle as O
        if O.RefModel.available("B"):
            ref = O.RefProj("B")
            xh = x[0].cpu().numpy()
            reps, total = 0, 0.0
            while total < 6.0 and reps < 50:
                t0 = time.perf_counter()
                for w, wt in zip(w0, (Q4K, Q4K, Q6K)):
                    ref.matmul_bias(xh, w, wt, w.shape[0])
                total += time.perf_counter() - t0
                reps += 1
            per = total / reps
            res["cpu_baseline"] = {"kind": "reference", "cores": 1, "us_per_layer": round(per * 1e6, 1),
                                   "weight_GB_per_s": round(wbytes / per / 1e9, 3),
                                   "sample": f"TensorOps::matmul_bias of the reference (build B) on layer 0, {reps}x"}
            qg = q[0].cpu().numpy()
            res["q_layer0_bit_exact"] = bool(np.array_equal(qg.view(np.uint32),
                                                            ref.matmul_bias(xh, w0[0], Q4K, nh * hd).view(np.uint32)))
    cx.close()
    log(f"[bench] qkv projection: {us:.2f} us/layer, {gbs:.0f} GB/s of weights ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM); {res.get('cpu_baseline')}")
    return res


def prefill_x_workload(torch, dev, n_layers=36, nh=32, nkv=8, hd=128, dim=2560, s=2048, steps=3, warmup=1, cpu=True):
    """The prompt path of a Qwen3-4B-shaped layer from the normed inputs
    (pqa_prefill_x): exact dequantization of Q4_K attn_q/attn_k and Q6_K
    attn_v, split into fp16 hi/lo parts (kept per layer after the first
    call), one GEMM over 2048 tokens (rocBLAS, fp16 MFMA with fp32
    accumulation), bias, then the K/V append and the causal MFMA prefill; 36
    layers per step."""
    Q4K, Q6K = 13, 15
    cx = Ctx(n_layers, s, nh, nkv, hd, 0, 1e6)
    rng = np.random.default_rng(909)
    set_norms(cx, rng, hd)
    vp = lambda a: a.ctypes.data_as(C.c_void_p)
    for layer in range(n_layers):
        wq, wk, wv = gguf_rows(rng, Q4K, nh * hd, dim), gguf_rows(rng, Q4K, nkv * hd, dim), gguf_rows(rng, Q6K, nkv * hd, dim)
        if layer == 0:
            w0 = (wq, wk, wv)
        cx.check(cx.L.pqa_set_qkv_weights(cx.h, layer, dim, vp(wq), Q4K, None, 0, vp(wk), Q4K, None, 0, vp(wv), Q6K,
                                          None, 0), cx.h)
    x = torch.from_numpy(rng.standard_normal((s, dim), dtype=np.float32)).to(dev)
    out = torch.empty((s, nh * hd), device=dev)
    torch.cuda.synchronize()
    run = cx.L.pqa_prefill_x
    xp, op = C.c_void_p(x.data_ptr()), C.c_void_p(out.data_ptr())

    def step():
        for layer in range(n_layers):
            cx.check(run(cx.h, layer, 0, s, xp, op), cx.h)

    _, ev = timed(torch, cx, step, steps, warmup)
    us = ev * 1e3 / n_layers
    gemm_flops = 2.0 * s * (nh * hd + 2 * nkv * hd) * dim
    attn_flops = prefill_flops(nh, hd, s)
    cx.close()
    res = {"workload": "qwen3_4b_prefill_from_xb", "tokens": s, "n_embd": dim, "weight_types": ["Q4_K", "Q4_K", "Q6_K"],
           "us_per_layer": round(us, 1), "projection_GFLOP_per_layer": round(gemm_flops / 1e9, 1),
           "attention_GFLOP_per_layer": round(attn_flops / 1e9, 1),
           "TFLOP_per_s_total": round((gemm_flops + attn_flops) / (us * 1e-6) / 1e12, 1)}
    if cpu:
        import oracle as O
        if O.RefModel.available("B"):
            # the reference's per-token matmul_bias (forward_batch's projections)
            # for a few tokens of layer 0, scaled to the prompt; the attention
            # part of the reference's prompt path is not in this figure
            ref = O.RefProj("B")
            xh = x[:4].cpu().numpy()
            t0 = time.perf_counter()
            for t in range(4):
                for w, wt in zip(w0, (Q4K, Q4K, Q6K)):
                    ref.matmul_bias(xh[t], w, wt, w.shape[0])
            per_tok = (time.perf_counter() - t0) / 4
            res["cpu_baseline"] = {"kind": "reference", "cores": 1, "us_per_layer_projections": round(per_tok * s * 1e6),
                                   "sample": f"TensorOps::matmul_bias of the reference (build B) for q/k/v of 4 "
                                             f"tokens of layer 0, scaled to {s} tokens; projections only"}
    log(f"[bench] prefill from xb: {us:.1f} us/layer; {res}")
    return res


def cpu_baseline(cx, q, k, v, out0, nh, nkv, hd, pos, budget_s=12.0):
    """The oracle (reference attention loop, restated in C) on layer 0 of the
    headline cache: same K/V bytes (downloaded), same q/k/v and norm weights."""
    import oracle as O
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    kv_dim = nkv * hd
    smax = pos + 1
    kc = np.zeros((smax, kv_dim), np.uint16)
    vc = np.zeros((smax, kv_dim), np.uint16)
    cx.check(cx.L.pqa_kv_download(cx.h, 0, 0, pos, kc.ctypes.data_as(C.c_void_p), vc.ctypes.data_as(C.c_void_p)), cx.h)
    qn = np.empty(hd, np.float32)
    kn = np.empty(hd, np.float32)
    rng = np.random.default_rng(20251201)  # same draw order as decode_workload
    for _ in range(1):
        qn[:] = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        kn[:] = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    from picolm_qwen_amd.attention import rope_table
    cos, sin = rope_table(1e6, hd, smax)
    shp = O.shape(nh, nkv, hd, smax, 0)
    qh, kh, vh = (t[0, 0].cpu().numpy() for t in (q, k, v))
    t0 = time.perf_counter()
    want = O.attn_step(shp, pos, qh, kh, vh, qn, kn, cos[pos], sin[pos], kc, vc, 1)
    t1 = time.perf_counter() - t0
    got = out0.cpu().numpy().reshape(-1)
    max_err = float(np.abs(got - want).max())
    log(f"[bench] layer-0 GPU output vs oracle: max abs err {max_err:.2e}")
    reps, total = 0, 0.0
    while total < budget_s and reps < 200:
        t0 = time.perf_counter()
        O.attn_step(shp, pos, qh, kh, vh, qn, kn, cos[pos], sin[pos], kc, vc, threads)
        total += time.perf_counter() - t0
        reps += 1
    per_layer = total / reps
    nbytes = decode_bytes(pos + 1, nh, nkv, hd)
    log(f"[bench] cpu oracle: 1 thread {t1 * 1e6:.0f} us/layer, {threads} threads {per_layer * 1e6:.0f} us/layer")
    return {"value": round(nbytes / per_layer / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_layer": round(per_layer * 1e6, 1), "us_per_layer_1_thread": round(t1 * 1e6, 1),
            "gpu_vs_oracle_max_abs_err": max_err,
            "sample": f"layer 0 of 36 of the headline decode (pos {pos}, same cache bytes and inputs), "
                      f"oracle attention step run {reps}x with query heads split over {threads} threads, "
                      f"plus once on 1 thread"}


COPY_BYTES = 1 << 30  # the calibration copy: reads and writes 1 GiB


def pmc_probe(torch, dev):
    """The dispatches the two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE)
    count: the headline decode (36 layers x 2 steps, same cache and inputs as
    the bench) and three launches of a plain elementwise copy of known size
    (torch.neg over 1 GiB of fp32: 1 GiB read + 1 GiB written), whose counter
    readings give the bytes-per-count scale."""
    decode_workload(torch, dev, "qwen3_8b_decode", 36, 32, 8, 128, 0, 1e6, 131071, 0.01, 2, 0, True)
    src = torch.ones(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log("[bench] pmc probe done")


def _rows(path):
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _find(d, suffix):
    for root, _, files in os.walk(d):
        for fn in files:
            if fn.endswith(suffix):
                return os.path.join(root, fn)
    raise FileNotFoundError(f"no *{suffix} under {d}")


def summarize_pmc(fetch_dir, write_dir):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the headline decode
    kernels, scaled by the calibration copy's bytes per KiB counted."""
    out = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        groups = {}
        for r in _rows(_find(d, "counter_collection.csv")):
            if r.get("Counter_Name") != counter:
                continue
            name = r["Kernel_Name"]
            key = ("copy" if "neg_kernel" in name else "decode" if "decode_kernel<128, 4>" in name
                   else "combine" if "decode_combine_kernel<128>" in name else None)
            if key:
                groups.setdefault(key, {}).setdefault(r["Dispatch_Id"], 0.0)
                groups[key][r["Dispatch_Id"]] += float(r["Counter_Value"])
        out[counter] = {k: (sum(v.values()) / len(v), len(v)) for k, v in groups.items()}
    fc, _ = out["FETCH_SIZE"]["copy"]
    wc, _ = out["WRITE_SIZE"]["copy"]
    f_scale = COPY_BYTES / fc  # bytes per counted KiB, reads
    w_scale = COPY_BYTES / wc
    lines = ["kernel                              dispatches  FETCH_SIZE KiB  WRITE_SIZE KiB  read bytes     written bytes"]
    res = {}
    for k in ("decode", "combine", "copy"):
        fk, nf = out["FETCH_SIZE"][k]
        wk, _ = out["WRITE_SIZE"][k]
        res[k] = (fk * f_scale, wk * w_scale)
        lines.append(f"{k:36s}{nf:10d}  {fk:14.1f}  {wk:14.1f}  {fk * f_scale:13.0f}  {wk * w_scale:13.0f}")
    alg = decode_bytes(131072, 32, 8, 128)
    traffic = res["decode"][0] + res["decode"][1] + res["combine"][0] + res["combine"][1]
    lines += ["",
              f"scale: reads {f_scale:.1f} B per FETCH_SIZE KiB, writes {w_scale:.1f} B per WRITE_SIZE KiB "
              f"(calibration copy: {COPY_BYTES} B read + {COPY_BYTES} B written per dispatch)",
              f"algorithmic bytes per decode launch: {alg}",
              f"hbm_traffic_bytes_per_launch: {traffic:.0f}",
              f"traffic / algorithmic: {traffic / alg:.4f}"]
    return "\n".join(lines)


def summarize_counters(dirs, match):
    """Per-dispatch averages of every counter in one or more rocprofv3 --pmc
    output directories, for the kernels whose name contains `match`, with the
    derived rates the counters give: MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES /
    (GRBM_GUI_ACTIVE x 1024 SIMDs), LDS bank conflicts per LDS instruction,
    VALU and LDS instructions per MFMA."""
    vals = {}
    names = set()
    durs = []
    for d in dirs:
        seen = set()
        for r in _rows(_find(d, "counter_collection.csv")):
            name = r["Kernel_Name"]
            if match not in name:
                continue
            names.add(name.split("(")[0])
            key = (d, r["Dispatch_Id"])  # dispatch ids restart in every run
            per = vals.setdefault(r["Counter_Name"], {})
            per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
            if key not in seen:
                seen.add(key)
                durs.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9)
    avg = {c: sum(v.values()) / len(v) for c, v in vals.items()}
    dur = sum(durs) / len(durs) if durs else 0.0
    lines = [f"kernel: {' | '.join(sorted(names))}",
             f"average dispatch duration under counter collection: {dur * 1e6:.2f} us",
             f"{'counter':32s} {'dispatches':>10s} {'average per dispatch':>22s}"]
    for c in sorted(avg):
        lines.append(f"{c:32s} {len(vals[c]):10d} {avg[c]:22.1f}")
    lines.append("")
    simds, xcds = 256 * 4, 8
    if "GRBM_GUI_ACTIVE" in avg and dur:
        # GRBM_GUI_ACTIVE comes summed over the 8 XCDs
        lines.append(f"clock: {avg['GRBM_GUI_ACTIVE'] / xcds / dur / 1e6:.0f} MHz "
                     f"(GRBM_GUI_ACTIVE / {xcds} XCDs / duration)")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in avg and "GRBM_GUI_ACTIVE" in avg:
        lines.append(f"mfma_busy_frac: {avg['SQ_VALU_MFMA_BUSY_CYCLES'] / (avg['GRBM_GUI_ACTIVE'] / xcds * simds):.4f} "
                     f"(SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {xcds} XCDs x {simds} SIMDs): issued MFMA "
                     f"cycles, the hi + lo q's second QK product included)")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in avg and "SQ_INSTS_MFMA" in avg and avg["SQ_INSTS_MFMA"]:
        lines.append(f"cycles_per_mfma: {avg['SQ_VALU_MFMA_BUSY_CYCLES'] / avg['SQ_INSTS_MFMA']:.2f}")
    if "SQ_LDS_BANK_CONFLICT" in avg and "SQ_LDS_IDX_ACTIVE" in avg and avg["SQ_LDS_IDX_ACTIVE"]:
        lines.append(f"lds_bank_conflict_frac: {avg['SQ_LDS_BANK_CONFLICT'] / avg['SQ_LDS_IDX_ACTIVE']:.4f} "
                     f"(SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE cycles)")
    if "SQ_INSTS_MFMA" in avg and avg["SQ_INSTS_MFMA"]:
        for c in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_SALU"):
            if c in avg:
                lines.append(f"{c.lower()}_per_mfma: {avg[c] / avg['SQ_INSTS_MFMA']:.3f}")
    if "SQ_WAIT_INST_LDS" in avg and "SQ_WAVE_CYCLES" in avg and avg["SQ_WAVE_CYCLES"]:
        lines.append(f"wait_inst_lds_per_wave_cycle: {avg['SQ_WAIT_INST_LDS'] / avg['SQ_WAVE_CYCLES']:.4f}")
    return "\n".join(lines)


def summarize_trace(trace_dir):
    """Average kernel durations per (kernel, grid) from a rocprofv3
    --kernel-trace CSV, labelled with the workload each instance belongs to."""
    groups = {}
    for r in _rows(_find(trace_dir, "kernel_trace.csv")):
        name = r["Kernel_Name"]
        m = re.match(r"_ZN3pqa(\d+)", name)  # a name the tracer left mangled: pqa::<identifier>
        if m:
            name = "pqa::" + name[m.end():m.end() + int(m.group(1))]
        # this library's kernels, and rocBLAS's GEMM kernels of the batched projections
        if not name.startswith(("void pqa::", "pqa::", "Cijk_")):
            continue
        grid = tuple(int(r.get(f"Grid_Size_{a}", r.get("Grid_Size", 0)) or 0) for a in "XYZ")
        g = groups.setdefault((name, grid), [])
        g.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = [f"{'kernel':52s} {'grid (threads)':>20s} {'calls':>7s} {'avg us':>9s} {'min us':>9s} {'max us':>9s}"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        short = name.replace("void pqa::", "").replace("pqa::", "").split("(")[0]
        if short.startswith("Cijk_"):
            short = "rocBLAS " + short[:40] + "..."
        lines.append(f"{short:52s} {str(grid):>20s} {len(d):7d} {sum(d) / len(d):9.2f} {min(d):9.2f} {max(d):9.2f}")
    return "\n".join(lines)


def profile_value(fname, key):
    """A figure recorded in a committed rocprofv3 summary under profiles/
    (None when the summary is absent)."""
    path = os.path.join(ROOT, "profiles", fname)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(key):
            return line
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--pmc-probe", action="store_true", help="dispatches for the rocprofv3 --pmc passes")
    ap.add_argument("--only", choices=["qwen3_1.7b_decode", "qwen3_4b_prefill", "tinyllama_decode",
                                       "qwen2.5_0.5b_sweep", "qwen3_8b_kvc_save_load", "qwen3_8b_qkv_proj",
                                       "qwen3_4b_prefill_from_xb"],
                    help="run one secondary workload and print it")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--summarize-trace", metavar="TRACE_DIR")
    ap.add_argument("--summarize-counters", nargs="+", metavar="PMC_DIR",
                    help="per-dispatch counter averages of the kernels named by --kernel")
    ap.add_argument("--kernel", default="prefill_attn_kernel")
    args = ap.parse_args()
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.kernel))
        return
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc))
        return
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode would shard by KV head with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.pmc_probe:
        pmc_probe(torch, dev)
        return
    if args.only:
        runs = {
            "qwen3_1.7b_decode": lambda: decode_workload(torch, dev, "qwen3_1.7b_decode", 28, 16, 8, 128, 0, 1e6,
                                                         32767, 0.0, args.steps, args.warmup, True)[0],
            "qwen3_4b_prefill": lambda: prefill_workload(torch, dev, 36, 32, 8, 128, 2048,
                                                         max(3, args.steps // 5), 1),
            "tinyllama_decode": lambda: decode_workload(torch, dev, "tinyllama_decode", 1, 32, 4, 64, 1, 1e4, 511,
                                                        0.0, max(args.steps, 200), args.warmup, False)[0],
            "qwen2.5_0.5b_sweep": lambda: sweep_workload(torch, dev),
            "qwen3_8b_kvc_save_load": lambda: kvc_workload(torch, dev),
            "qwen3_8b_qkv_proj": lambda: proj_workload(torch, dev, steps=args.steps, warmup=args.warmup),
            "qwen3_4b_prefill_from_xb": lambda: prefill_x_workload(torch, dev),
        }
        print(json.dumps({args.only: runs[args.only]()}), flush=True)
        return

    nh, nkv, hd, layers, pos = 32, 8, 128, 36, 131071
    head, cx, bufs = decode_workload(torch, dev, "qwen3_8b_decode", layers, nh, nkv, hd, 0, 1e6, pos, 0.01,
                                     args.steps, args.warmup, True, keep=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cx, bufs[0], bufs[1], bufs[2], bufs[3][0, 0], nh, nkv, hd, pos)
    cx.close()
    del bufs
    torch.cuda.empty_cache()

    workloads = {"qwen3_8b_decode": head}
    if not args.quick:
        workloads["qwen3_1.7b_decode"] = decode_workload(torch, dev, "qwen3_1.7b_decode", 28, 16, 8, 128, 0, 1e6,
                                                         32767, 0.0, args.steps, args.warmup, True)[0]
        workloads["qwen3_4b_prefill"] = prefill_workload(torch, dev, 36, 32, 8, 128, 2048,
                                                         max(3, args.steps // 5), 1)
        workloads["tinyllama_decode"] = decode_workload(torch, dev, "tinyllama_decode", 1, 32, 4, 64, 1, 1e4, 511,
                                                        0.0, max(args.steps, 200), args.warmup, False)[0]
        workloads["qwen2.5_0.5b_sweep"] = sweep_workload(torch, dev)
        workloads["qwen3_8b_kvc_save_load"] = kvc_workload(torch, dev)
        workloads["qwen3_8b_qkv_proj"] = proj_workload(torch, dev, steps=args.steps, warmup=args.warmup,
                                                       cpu=not args.no_cpu)
        workloads["qwen3_4b_prefill_from_xb"] = prefill_x_workload(torch, dev, cpu=not args.no_cpu)

    per_layer_us = head["us_per_layer"]
    achieved = head["GB_per_s"]
    tline = profile_value("decode_qwen3_8b_ctx131072_hbm_traffic.txt", "hbm_traffic_bytes_per_launch:")
    traffic = int(float(tline.split(":")[1])) if tline else None
    if "qwen3_4b_prefill" in workloads:
        aline = profile_value("prefill_qwen3_4b_2048_kernel_trace.txt", "prefill_attn_kernel")
        if aline:
            attn_us = float(aline.split()[-3])
            tf = prefill_flops(32, 128, 2048) / (attn_us * 1e-6) / 1e12
            workloads["qwen3_4b_prefill"]["attention_only_rocprof"] = {
                "us_per_layer": attn_us, "TFLOP_per_s": round(tf, 1),
                "mfma_frac": round(tf / MFMA_FP16_PEAK_TFLOPS, 4),
                "source": "profiles/prefill_qwen3_4b_2048_kernel_trace.txt"}
    line = {
        "metric": METRIC,
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step_event"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) q/k/v, cache history N(0,1) with 1% rows x8, fp16)",
        "config": {"workload": "Qwen3-8B-shaped decode attention: 1 token at pos 131071 over a 131072-entry "
                               "fp16 KV cache, all 36 layers per step",
                   "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd, "layers": layers, "ctx": pos + 1,
                   "kv_cache_GB": round(2 * layers * (pos + 1) * nkv * hd * 2 / 1e9, 2), "parallelism": "none"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "decode_kernel<128,4> + decode_combine_kernel<128> (one pqa_decode call)",
                     "us_per_launch": per_layer_us, "bytes_per_launch": head["bytes_per_layer"],
                     "traffic_source": "profiles/decode_qwen3_8b_ctx131072_hbm_traffic.txt (rocprofv3 --pmc "
                                       "FETCH_SIZE, WRITE_SIZE; copy-calibrated)"},
        "cpu_baseline": cpu,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
