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
events on the library's stream. Each attention workload carries a
`cpu_baseline`: the CPU oracle (the reference's attention loop restated; its
timing build uses the reference's -O3 and FP contraction with
-march=x86-64-v4) on the same cache bytes (downloaded) and inputs, on 1
thread and on T = min(usable cores, 16) threads, with the sample it covers
stated; the checker build compares the GPU's output and appended rows on the
layers it lists. `host_entry` times the host-pointer entry points
(pqa_decode_host, pqa_prefill_host) that a CPU forward loop calls, PCIe and
the per-call sync included. `cpu_host` names the host CPU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
"""
import argparse
import ctypes as C
import json
import re
import os
import subprocess
import sys
import time
import warnings

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
    """Thin ctypes holder around one pqa context (the bench calls the C ABI directly).

    While Ctx.deferred is a list, close() only queues the context, and
    close_deferred() destroys the queued ones. The full run keeps every
    workload's context until its end: releasing a large cache makes the
    driver work on the freed memory for seconds, and the next workload's
    kernels then share HBM with that work (C3 measured 26.70 us per layer
    right after C5's 19 GB context was destroyed, 25.35 us with it kept, and
    25.38 us 10 s after the release). A serving process allocates its cache
    once, so the kept-context figures are the ones it sees."""

    deferred = None

    def __init__(self, n_layers, smax, nh, nkv, hd, style, base, L=None):
        from picolm_qwen_amd import _lib
        from picolm_qwen_amd.attention import rope_table
        self.L = L if L is not None else _lib.lib()
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
        if self.h and Ctx.deferred is not None:
            Ctx.deferred.append(self)
        elif self.h:
            self.L.pqa_destroy(self.h)
            self.h = None

    @staticmethod
    def close_deferred():
        queued, Ctx.deferred = Ctx.deferred or [], None
        for cx in queued:
            cx.close()


def make_inputs(torch, dev, rng, n_layers, n_tok, nh, nkv, hd):
    q = torch.from_numpy(rng.standard_normal((n_layers, n_tok, nh * hd), dtype=np.float32)).to(dev)
    k = torch.from_numpy(rng.standard_normal((n_layers, n_tok, nkv * hd), dtype=np.float32)).to(dev)
    v = torch.from_numpy(rng.standard_normal((n_layers, n_tok, nkv * hd), dtype=np.float32)).to(dev)
    out = torch.empty((n_layers, n_tok, nh * hd), dtype=torch.float32, device=dev)
    return q, k, v, out


def set_norms(cx, rng, hd):
    """Per-layer QK-RMSNorm weights near 1; returns them as [(q_w, k_w)] by layer."""
    norms = []
    for layer in range(cx.n_layers):
        qw = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        kw = (1.0 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        cx.check(cx.L.pqa_set_qk_norm(cx.h, layer, qw.ctypes.data_as(C.c_void_p),
                                      kw.ctypes.data_as(C.c_void_p)), cx.h)
        norms.append((qw, kw))
    return norms


def _vp(a):
    return a.ctypes.data_as(C.c_void_p)


def cpu_threads():
    """T = min(usable cores, 16): the reference's thread-pool cap (cpp/tensor.hpp:16)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_host():
    """This host's core count and CPU model, printed beside every CPU figure."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key = line.split(":", 1)[0].strip()
                if key in ("model name", "cpu family", "model", "flags") and key not in info:
                    info[key] = line.split(":", 1)[1].strip()
                if not line.strip():
                    break  # the first processor's block is enough
    except OSError:
        pass
    flags = set(info.get("flags", "").split())
    return {"nproc": os.cpu_count(), "usable_cores": len(os.sched_getaffinity(0)),
            "model": info.get("model name", ""), "family_model": f"{info.get('cpu family')}/{info.get('model')}",
            "avx512": all(x in flags for x in ("avx512f", "avx512bw", "avx512dq", "avx512vl")),
            "threads_T": cpu_threads()}


def median_time(fn, runs):
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_decode(cx, inputs, norms, style, base, pos, time_layers, check_layers, runs_1, runs_t, ref=None):
    """The oracle's decode step (the reference's attention block,
    cpp/model.hpp:326-418, restated) on this run's own cache bytes and inputs.

    check_layers: the checker build (liboracle.so, heads over T threads) runs
    each listed layer; its output is compared with the GPU's and its appended
    K/V row with the row the GPU wrote. time_layers: the timing build
    (liboracle_bench.so) runs each listed layer on 1 thread (median of
    runs_1) and on T threads (median of runs_t). inputs(layer) returns the
    layer's (q, k, v, gpu_out) as host arrays."""
    import oracle as O
    from picolm_qwen_amd.attention import rope_table
    lb, flags = O.bench_lib()
    nt = cpu_threads()
    kv_dim = cx.nkv * cx.hd
    shp = O.shape(cx.nh, cx.nkv, cx.hd, pos + 1, style)
    cos, sin = rope_table(base, cx.hd, pos + 1)
    kc = np.empty((pos + 1, kv_dim), np.uint16)
    vc = np.empty_like(kc)
    t1, tt, err, exact = [], [], 0.0, True
    for layer in sorted(set(time_layers) | set(check_layers)):
        cx.check(cx.L.pqa_kv_download(cx.h, layer, 0, pos + 1, _vp(kc), _vp(vc)), cx.h)
        krow, vrow = kc[pos].copy(), vc[pos].copy()  # the row the GPU appended
        q, k, v, got = inputs(layer)
        qn, kn = norms[layer] if norms else (None, None)
        if layer in check_layers:
            want = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc, nt)
            err = max(err, float(np.abs(got - want).max()))
            exact = exact and bool(np.array_equal(kc[pos], krow) and np.array_equal(vc[pos], vrow))
        if layer in time_layers:
            def step(n):
                O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc, vc, n, L=lb)
            t1.append(median_time(lambda: step(1), runs_1))
            tt.append(median_time(lambda: step(nt), runs_t))
    nbytes = decode_bytes(pos + 1, cx.nh, cx.nkv, cx.hd)
    us1, ust = float(np.mean(t1)) * 1e6, float(np.mean(tt)) * 1e6
    res = {"value": round(nbytes / ust / 1e3, 3), "unit": "GB/s", "cores": nt, "kind": "port",
           "us_per_layer": round(ust, 2), "us_per_layer_1_thread": round(us1, 2),
           "GB_per_s_1_thread": round(nbytes / us1 / 1e3, 3), "build": flags,
           "layers_timed": len(t1), "runs_per_layer": [runs_1, runs_t],
           "layers_checked": sorted(check_layers), "gpu_vs_oracle_max_abs_err": err,
           "appended_kv_rows_bit_exact": exact,
           "sample": f"the oracle's decode step at pos {pos} on {len(t1)} of {cx.n_layers} layers (same cache "
                     f"bytes, downloaded, and the same inputs as the GPU run); median of {runs_1} run(s) on 1 "
                     f"thread and {runs_t} on {nt} threads (query heads split) per layer, mean over layers"}
    log(f"[bench]   cpu oracle: 1 thread {us1:.1f} us/layer, {nt} threads {ust:.1f} us/layer; "
        f"layers {sorted(check_layers)} max abs err {err:.2e}, appended rows bit-exact {exact}")
    if ref is not None:
        # the reference's own attention beside the port, on layer 0 (ref = (seed, outlier prob, runs))
        q, k, v, got = inputs(0)
        r = ref_attention_cpu(cx, style, base, pos, ref[1], ref[0], q, k, v, norms, got, ref[2])
        if r is not None:
            if "us_per_layer_attention" in r:
                r["port_us_per_layer_1_thread_layer0"] = round(t1[0] * 1e6, 1) if t1 else None
            res["reference_attention"] = r
            log(f"[bench]   reference attention (libref_A.so, 1 thread): {r}")
    return res


def ref_attention_cpu(cx, style, base, pos, prob, seed, q, k, v, norms, gpu_out, runs):
    """The reference's own decode step, timed: Model::forward (cpp/model.hpp:311-451)
    built with its shipped flags (oracle/_ref/libref_A.so: -O3 -march=native,
    GCC's default FMA contraction), one token at `pos` over the layer-0 history of
    this run (the same seeded rows the GPU holds, regenerated on the host) on one
    thread (its matmul pool is left at one thread; its attention loop has one).
    The harness's one-layer model has zero-weight F32 projections, so the same
    call at pos 0 (one history row) times everything but the attention loop; the
    difference is the reference's attention. Run in a child process: the build
    targets the container's CPU, and a host without one of its instructions must
    not take the bench down. Returns a dict, or None where the build is absent."""
    import tempfile
    import oracle as O
    if not O.RefModel.available("A"):
        return None
    fd, path = tempfile.mkstemp(suffix=".npz")
    os.close(fd)
    qn, kn = norms[0] if norms else (np.zeros(0, np.float32), np.zeros(0, np.float32))
    np.savez(path, q=q, k=k, v=v, qn=qn, kn=kn, gpu_out=gpu_out,
             shape=np.array([cx.nh, cx.nkv, cx.hd, pos, style, runs, seed], np.int64),
             fl=np.array([base, prob], np.float64))
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--ref-attn-child", path],
                           capture_output=True, text=True, timeout=600)
        line = [x for x in r.stdout.splitlines() if x.startswith("{")]
        if r.returncode != 0 or not line:
            return {"kind": "reference", "error": f"child exited {r.returncode}: {r.stderr[-300:]}"}
        return json.loads(line[-1])
    finally:
        os.unlink(path)


def ref_attention_child(path):
    """Body of ref_attention_cpu's child process (bench.py --ref-attn-child NPZ)."""
    import oracle as O
    d = np.load(path)
    nh, nkv, hd, pos, style, runs, seed = (int(x) for x in d["shape"])
    base, prob = (float(x) for x in d["fl"])
    qk = d["qn"].size > 0
    kv_dim = nkv * hd
    t0 = time.perf_counter()
    R = O.RefModel(nh, nkv, hd, pos + 1, base, style == 0, qk, variant="A")
    if qk:
        R.set_qk_norm(d["qn"], d["kn"])
    kc, vc = O.synth_kv_rows(seed, 0, kv_dim, 0, pos, prob, cpu_threads())
    R.set_cache_rows(0, kc, vc)
    del kc, vc
    setup = time.perf_counter() - t0
    times, out = [], None
    for _ in range(runs):
        t0 = time.perf_counter()
        out = R.step(pos, d["q"], d["k"], d["v"])
        times.append(time.perf_counter() - t0)
    t_pos = float(np.median(times))
    t0 = time.perf_counter()
    R.step(0, d["q"], d["k"], d["v"])  # one history row: the layer without the attention loop
    t_zero = time.perf_counter() - t0
    R.close()
    err = float(np.abs(out - d["gpu_out"]).max())
    nbytes = decode_bytes(pos + 1, nh, nkv, hd)
    print(json.dumps({
        "kind": "reference", "cores": 1, "build": "oracle/_ref/libref_A.so (cpp/Makefile flags: -O3 -std=c++17 "
                                                  "-march=native, built in the build container)",
        "us_per_layer_forward": round(t_pos * 1e6, 1), "us_pos0_forward": round(t_zero * 1e6, 1),
        "us_per_layer_attention": round((t_pos - t_zero) * 1e6, 1),
        "non_attention_share": round(t_zero / t_pos, 4),
        "GB_per_s_attention": round(nbytes / ((t_pos - t_zero) * 1e6) / 1e3, 3),
        "gpu_vs_reference_max_abs_err": err, "runs": runs, "setup_s": round(setup, 1),
        "sample": f"Model::forward of the reference's one-layer harness (zero-weight F32 projections, identity "
                  f"attn_output) for one token at pos {pos} over the layer-0 history of this run, median of "
                  f"{runs} run(s) on 1 thread, minus the same call at pos 0 (projections and the rest of the "
                  f"layer)"}), flush=True)


def host_entry_decode(cx, q, k, v, out, pos, steps):
    """pqa_decode_host, the call a CPU forward loop makes per layer: host
    q/k/v in, host out back, PCIe copies and the per-call stream sync
    included. Returns wall µs per layer and whether its outputs equal the
    device-pointer entry's bit for bit."""
    qh, kh, vh, want = (np.ascontiguousarray(t.cpu().numpy()) for t in (q, k, v, out))
    oh = np.zeros_like(want)
    fn = cx.L.pqa_decode_host
    h = cx.h
    args = [(layer, _vp(qh[layer]), _vp(kh[layer]), _vp(vh[layer]), _vp(oh[layer])) for layer in range(cx.n_layers)]

    def step():
        for layer, a, b, c, d in args:
            rc = fn(h, layer, pos, a, b, c, d)
            if rc:
                cx.check(rc, h)

    step()
    t = median_time(step, max(3, steps // 3))
    return {"entry": "pqa_decode_host", "us_per_layer": round(t * 1e6 / cx.n_layers, 2),
            "equals_device_entry": bool(np.array_equal(oh, want)),
            "note": "the caller's pageable host buffers, copied by the CPU into and out of the library's pinned "
                    "staging buffer, which the decode kernels read and write directly (no DMA copies); "
                    "a stream sync per call"}


# Untimed work before every timed region, at least: after an idle spell (the
# CPU oracles between workloads idle the GPU for seconds) the GPU's clocks ramp
# over the first tens of ms of work. Measured on C3 (28 layers at ctx 32768):
# 3 warmup steps gave 25.4-26.8 us per layer depending on what ran before;
# 150 steps (~110 ms) first gave 25.40-25.45 us in every order tried.
WARMUP_MIN_MS = 150.0


def warm_up(cx, fn):
    """fn() untimed until WARMUP_MIN_MS of wall time have passed."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < WARMUP_MIN_MS:
        for _ in range(8):
            fn()
        cx.check(cx.L.pqa_sync(cx.h), cx.h)


def timed(torch, cx, fn, steps, warmup):
    """Runs fn() warmup times, then more untimed until WARMUP_MIN_MS of wall
    time have passed since the first, then steps times timed; returns (wall
    ms/step, event ms/step on the library stream)."""
    ext = torch.cuda.ExternalStream(cx.stream())
    t_warm = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - t_warm) * 1e3 < WARMUP_MIN_MS:
        for _ in range(max(1, warmup)):
            fn()
            n += 1
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
                    seed=20251201, keep=False, cpu=None, host_entry=False):
    """cpu: None, or (time_layers, check_layers, runs_1, runs_t[, reference runs]) for cpu_decode; with a
    fifth element the reference's own attention (libref_A.so) is timed beside the port on layer 0."""
    cx = Ctx(n_layers, pos + 1, nh, nkv, hd, style, base)
    rng = np.random.default_rng(seed)
    norms = set_norms(cx, rng, hd) if qk_norm else None
    for layer in range(n_layers):
        # the history stream is keyed by (seed, layer): every layer holds its own rows
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
    if host_entry:
        res["host_entry"] = host_entry_decode(cx, q, k, v, out, pos, steps)
        log(f"[bench]   host entry: {res['host_entry']}")
    if cpu is not None:
        def inputs(layer):
            return tuple(t[layer, 0].cpu().numpy() for t in (q, k, v, out))
        ref = (seed, prob, cpu[4]) if len(cpu) > 4 else None  # cpu[4]: reference runs at layer 0
        res["cpu_baseline"] = cpu_decode(cx, inputs, norms, style, base, pos, *cpu[:4], ref=ref)
    if keep:
        return res, cx, (q, k, v, out)
    cx.close()
    return res, None, None


def cpu_prefill(cx, q, k, v, out, norms, s, check_layers, check_rows=512, rows_1=64, rows_t=512):
    """The oracle's causal prefill (cpp/model.hpp:507-593 restated) on this
    run's inputs, over the last rows of the prompt with the GPU-built cache
    of the rows before them (downloaded). The checker build compares the last
    check_rows rows of each check layer (output at tolerance, appended K/V
    rows bit for bit); the timing build runs the last rows_1 rows on 1 thread
    and the last rows_t rows on T threads of layer 0. A row's work is its key
    count, so the full-layer time is the sample time x (keys of all s rows) /
    (keys of the sampled rows)."""
    import oracle as O
    from picolm_qwen_amd.attention import rope_table
    lb, flags = O.bench_lib()
    nt = cpu_threads()
    kv_dim = cx.nkv * cx.hd
    shp = O.shape(cx.nh, cx.nkv, cx.hd, s, 0)
    cos, sin = rope_table(1e6, cx.hd, s)
    kc = np.empty((s, kv_dim), np.uint16)
    vc = np.empty_like(kc)
    keys = lambda r: sum(i + 1 for i in range(s - r, s))  # noqa: E731
    total = keys(s)
    err, exact, times = 0.0, True, {}
    for layer in sorted(set(check_layers) | {0}):
        cx.check(cx.L.pqa_kv_download(cx.h, layer, 0, s, _vp(kc), _vp(vc)), cx.h)
        kg, vg = kc.copy(), vc.copy()
        qh, kh, vh = (t[layer].cpu().numpy() for t in (q, k, v))
        qn, kn = norms[layer]
        if layer in check_layers:
            st = s - check_rows
            want = O.prefill(shp, st, qh[st:], kh[st:], vh[st:], qn, kn, cos, sin, kc, vc, n_threads=nt)
            err = max(err, float(np.abs(out[layer, st:].cpu().numpy() - want).max()))
            exact = exact and bool(np.array_equal(kc, kg) and np.array_equal(vc, vg))
        if layer == 0:
            for n, rows in ((1, rows_1), (nt, rows_t)):
                st = s - rows
                t0 = time.perf_counter()
                O.prefill(shp, st, qh[st:], kh[st:], vh[st:], qn, kn, cos, sin, kc, vc, n_threads=n, L=lb)
                times[n] = (time.perf_counter() - t0) * total / keys(rows)
    fl = prefill_flops(cx.nh, cx.hd, s)
    res = {"value": round(fl / times[nt] / 1e12, 5), "unit": "TFLOP/s", "cores": nt, "kind": "port",
           "us_per_layer": round(times[nt] * 1e6), "us_per_layer_1_thread": round(times[1] * 1e6),
           "build": flags, "layers_checked": sorted(check_layers), "rows_checked_per_layer": check_rows,
           "gpu_vs_oracle_max_abs_err": err, "appended_kv_rows_bit_exact": exact,
           "sample": f"layer 0: the last {rows_1} prompt rows on 1 thread and the last {rows_t} on {nt} threads "
                     f"(rows split), each run once over the GPU-built cache of the rows before them; "
                     f"scaled to all {s} rows by key count ({keys(rows_1)} and {keys(rows_t)} of {total} "
                     f"row-keys). Per layer; the {cx.n_layers}-layer prompt is {cx.n_layers}x."}
    log(f"[bench]   cpu oracle prefill: 1 thread {times[1]:.2f} s/layer, {nt} threads {times[nt]:.2f} s/layer "
        f"(extrapolated); layers {sorted(check_layers)} last {check_rows} rows max abs err {err:.2e}, "
        f"appended rows bit-exact {exact}")
    return res


def host_entry_prefill(cx, q, k, v, out, s):
    """pqa_prefill_host over all layers: host q/k/v in, host out back, PCIe
    copies and the per-call sync included; wall µs per layer and whether the
    outputs equal the device-pointer entry's bit for bit."""
    qh, kh, vh, want = (np.ascontiguousarray(t.cpu().numpy()) for t in (q, k, v, out))
    oh = np.zeros_like(want)
    fn = cx.L.pqa_prefill_host
    h = cx.h

    def step():
        for layer in range(cx.n_layers):
            rc = fn(h, layer, 0, s, _vp(qh[layer]), _vp(kh[layer]), _vp(vh[layer]), _vp(oh[layer]))
            if rc:
                cx.check(rc, h)

    step()
    t = median_time(step, 3)
    return {"entry": "pqa_prefill_host", "us_per_layer": round(t * 1e6 / cx.n_layers, 1),
            "equals_device_entry": bool(np.array_equal(oh, want)),
            "note": "the caller's pageable host buffers (80 MB in, 32 MB out per layer, past the 4 MiB one-copy "
                    "staging): streamed through two 8 MiB pinned slots (CPU threads fill one while the DMA "
                    "engine copies the other), the prefill, the results back the same way, a stream sync per call"}


def prefill_workload(torch, dev, n_layers, nh, nkv, hd, s, steps, warmup, seed=4242, cpu=False, host_entry=False):
    cx = Ctx(n_layers, s, nh, nkv, hd, 0, 1e6)
    rng = np.random.default_rng(seed)
    norms = set_norms(cx, rng, hd)
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
    if host_entry:
        res["host_entry"] = host_entry_prefill(cx, q, k, v, out, s)
        log(f"[bench]   host entry: {res['host_entry']}")
    if cpu:
        res["cpu_baseline"] = cpu_prefill(cx, q, k, v, out, norms, s, (0, n_layers - 1))
    cx.close()
    return res


def sweep_workload(torch, dev, n_layers=24, nh=14, nkv=2, hd=64, positions=4096, checkpoints=(1, 512, 1024, 2048, 4096),
                   cpu=False):
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

    def pos0():  # position 0 of every layer: rewrites row 0 with the bytes the sweep writes there
        for layer in range(n_layers):
            off_q = layer * positions
            dec(h, layer, 0, C.c_void_p(qp + off_q * qs), C.c_void_p(kp + off_q * kvs),
                C.c_void_p(vp + off_q * kvs), C.c_void_p(op + off_q * qs))

    warm_up(cx, pos0)
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
    log(f"[bench] qwen2.5 sweep: avg {avg_us:.2f} us/layer over ctx 1..{positions}; curve {curve}")
    res = {"workload": "qwen2.5_0.5b_sweep", "n_layers": n_layers, "positions": positions,
           "avg_us_per_layer_launch_loop": round(avg_us, 3), "us_per_layer_vs_ctx": curve}
    res.update(sweep_graphs(torch, cx, n_layers, positions, checkpoints, (qp, kp, vp, op), (qs, kvs), out))
    if cpu:
        # the oracle at two points of the curve, all layers, each layer's own inputs at that position
        res["cpu_baseline"] = {}
        for ctx_len in (512, positions):
            pos = ctx_len - 1

            def inputs(layer, pos=pos):
                return tuple(t[layer, pos].cpu().numpy() for t in (q, k, v, out))
            res["cpu_baseline"][str(ctx_len)] = cpu_decode(cx, inputs, None, 0, 1e6, pos, range(n_layers),
                                                           range(n_layers), 5, 5)
    cx.close()
    return res


def sweep_graphs(torch, cx, n_layers, positions, checkpoints, ptrs, sizes, out):
    """The same sweep with each position's 24-layer decode step captured once
    into a HIP graph (pqa_decode_noalloc: no allocation, no memset; captured on
    the library stream, picolm_qwen_amd.hipgraph) and replayed: the device-side
    cost of a step without the host's per-launch cost. Captures every position
    first, then replays positions 0..4095 in order (each replay re-appends the
    row the launch loop appended, same bits), then each checkpoint's graph 20
    times. The outputs of every replayed position are compared with the launch
    loop's bit for bit."""
    from picolm_qwen_amd.hipgraph import Graph
    qp, kp, vp, op = ptrs
    qs, kvs = sizes
    nod, h = cx.L.pqa_decode_noalloc, cx.h
    torch.cuda.synchronize()
    eager = out.clone()

    def step(pos):
        for layer in range(n_layers):
            o = (layer * positions) + pos
            cx.check(nod(h, layer, pos, C.c_void_p(qp + o * qs), C.c_void_p(kp + o * kvs), C.c_void_p(vp + o * kvs),
                         C.c_void_p(op + o * qs)), h)

    t0 = time.perf_counter()
    graphs = [Graph(cx.stream(), lambda pos=pos: step(pos)) for pos in range(positions)]
    capture_s = time.perf_counter() - t0
    ext = torch.cuda.ExternalStream(cx.stream())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out.zero_()
    warm_up(cx, lambda: graphs[0].launch(cx.stream()))  # position 0 again: the same row 0
    torch.cuda.synchronize()
    e0.record(ext)
    for g in graphs:
        g.launch(cx.stream())
    e1.record(ext)
    cx.check(cx.L.pqa_sync(cx.h), cx.h)
    torch.cuda.synchronize()
    avg = e0.elapsed_time(e1) * 1e3 / (positions * n_layers)
    same = bool(torch.equal(out.view(torch.int32), eager.view(torch.int32)))
    curve = {}
    for ctx_len in checkpoints:
        g = graphs[ctx_len - 1]

        def replay(g=g):
            g.launch(cx.stream())

        _, ev = timed(torch, cx, replay, 20, 2)
        curve[str(ctx_len)] = round(ev * 1e3 / n_layers, 3)
    same = same and bool(torch.equal(out.view(torch.int32), eager.view(torch.int32)))
    for g in graphs:
        g.close()
    log(f"[bench] qwen2.5 sweep, graph replay: avg {avg:.2f} us/layer over ctx 1..{positions}; curve {curve}; "
        f"equal to the launch loop {same}; {positions} captures in {capture_s:.1f} s")
    return {"avg_us_per_layer_graph": round(avg, 3), "us_per_layer_vs_ctx_graph": curve,
            "graph_outputs_equal_launch_loop": same,
            "graph": "one HIP graph per position (24 layers of pqa_decode_noalloc, captured on the library stream), "
                     "replayed in position order; the curve replays each checkpoint's graph 20 times"}


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

    # q rows in the reference's order too (pqa_set_token_projection(1)), then
    # the default: q on the any-order path, k and v in the reference's order
    cx.check(cx.L.pqa_set_token_projection(cx.h, 1), cx.h)
    _, ev_exact = timed(torch, cx, step, steps, warmup)
    us_exact = ev_exact * 1e3 / n_layers
    q_exact = q[0].cpu().numpy().copy()
    cx.check(cx.L.pqa_set_token_projection(cx.h, 0), cx.h)
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
    cx.check(cx.L.pqa_set_out_projection(cx.h, 0), cx.h)  # the opt-in any-order rows
    _, oev_any = timed(torch, cx, ostep, steps, warmup)
    cx.check(cx.L.pqa_set_out_projection(cx.h, 1), cx.h)
    ous_any = oev_any * 1e3 / n_layers
    res = {"workload": "qwen3_8b_qkv_proj_q4_k_m", "n_embd": n, "rows": [nh * hd, nkv * hd, nkv * hd],
           "weight_types": ["Q4_K", "Q4_K", "Q6_K"], "weight_bytes_per_layer": wbytes,
           "us_per_layer": round(us, 3), "weight_GB_per_s": round(gbs, 1),
           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "q_rows": "any summation order, one row per wave (the default); k and v in the reference's order",
           "all_reference_order": {"us_per_layer": round(us_exact, 3),
                                   "weight_GB_per_s": round(wbytes / (us_exact * 1e-6) / 1e9, 1),
                                   "note": "pqa_set_token_projection(1): q, k and v bit-identical to matmul_bias"},
           "out_proj": {"rows": n, "width": nh * hd, "weight_type": "Q4_K", "weight_bytes_per_layer": obytes,
                        "us_per_layer": round(ous, 3), "weight_GB_per_s": round(obytes / (ous * 1e-6) / 1e9, 1),
                        "any_order_us_per_layer": round(ous_any, 3),
                        "note": "attn_output matmul_bias + residual vec_add (cpp/model.hpp:420-427), the reference's "
                                "order (default); any_order: pqa_set_out_projection(0)"}}
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
            qr = ref.matmul_bias(xh, w0[0], Q4K, nh * hd)
            res["q_layer0_bit_exact_all_reference_order"] = bool(np.array_equal(q_exact.view(np.uint32),
                                                                                qr.view(np.uint32)))
            qg = q[0].cpu().numpy()
            res["q_layer0_max_abs_err_any_order"] = float(np.max(np.abs(qg.astype(np.float64) - qr)))
            res["q_layer0_max_abs"] = float(np.max(np.abs(qr)))
            res["kv_layer0_bit_exact"] = bool(
                np.array_equal(k[0].cpu().numpy().view(np.uint32), ref.matmul_bias(xh, w0[1], Q4K, nkv * hd).view(np.uint32))
                and np.array_equal(v[0].cpu().numpy().view(np.uint32),
                                   ref.matmul_bias(xh, w0[2], Q6K, nkv * hd).view(np.uint32)))
    cx.close()
    log(f"[bench] qkv projection: {us:.2f} us/layer, {gbs:.0f} GB/s of weights ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM); "
        f"all in the reference's order {us_exact:.2f} us; attn_output {ous:.2f} us (any order {ous_any:.2f} us); "
        f"{res.get('cpu_baseline')}")
    return res


def prefill_x_workload(torch, dev, n_layers=36, nh=32, nkv=8, hd=128, dim=2560, s=2048, steps=3, warmup=1, cpu=True):
    """The prompt path of a Qwen3-4B-shaped layer from the normed inputs
    (pqa_prefill_x): exact dequantization of Q4_K attn_q/attn_k and Q6_K
    attn_v, split into fp16 hi/lo parts (kept per layer after the first
    call), one GEMM over 2048 tokens (gemm_f16x3_nt_kernel, fp16 MFMA with
    fp32 accumulation), bias, then the K/V append and the causal MFMA prefill; 36
    layers per step. Timed in both K/V projection modes: the default (k and v
    in the reference's summation order on ordered_dot_kernel, bit-exact cache
    rows; the GEMM covers q only) and the split GEMM for all three."""
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

    us_mode = {}
    for exact in (1, 0):
        cx.check(cx.L.pqa_set_batch_projection(cx.h, exact), cx.h)
        _, ev = timed(torch, cx, step, steps, warmup)
        us_mode[exact] = ev * 1e3 / n_layers
    us = us_mode[1]
    gemm_flops = 2.0 * s * (nh * hd + 2 * nkv * hd) * dim
    attn_flops = prefill_flops(nh, hd, s)
    cx.close()
    res = {"workload": "qwen3_4b_prefill_from_xb", "tokens": s, "n_embd": dim, "weight_types": ["Q4_K", "Q4_K", "Q6_K"],
           "us_per_layer": round(us, 1), "kv_projection": "reference order (bit-exact cache rows)",
           "us_per_layer_split_gemm_kv": round(us_mode[0], 1),
           "projection_GFLOP_per_layer": round(gemm_flops / 1e9, 1),
           "attention_GFLOP_per_layer": round(attn_flops / 1e9, 1),
           "TFLOP_per_s_total_split_gemm_kv": round((gemm_flops + attn_flops) / (us_mode[0] * 1e-6) / 1e12, 1)}
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


COPY_BYTES = 1 << 30  # the calibration copy: reads and writes 1 GiB


# the decode shapes a --pmc-probe can run: (workload name, n_layers, nh, nkv, hd, pos, outlier prob)
PMC_SHAPES = {"c5": ("qwen3_8b_decode", 36, 32, 8, 128, 131071, 0.01),
              "c3": ("qwen3_1.7b_decode", 28, 16, 8, 128, 32767, 0.0)}


def pmc_probe(torch, dev, which="c5"):
    """The dispatches the rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE, or
    other counters) count: a decode workload (C5, the headline: 36 layers x 2
    steps; or C3: 28 layers x 2 steps; same caches and inputs as the bench) and
    three launches of a plain elementwise copy of known size (torch.neg over 1
    GiB of fp32: 1 GiB read + 1 GiB written), whose counter readings give the
    bytes-per-count scale."""
    name, nl, nh, nkv, hd, pos, prob = PMC_SHAPES[which]
    decode_workload(torch, dev, name, nl, nh, nkv, hd, 0, 1e6, pos, prob, 2, 0, True)
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


def summarize_pmc(fetch_dir, write_dir, which="c5"):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) of the decode kernels of a
    --pmc-probe run (C5: query-head chunk 4; C3: 2), scaled by the calibration
    copy's bytes per KiB counted."""
    _, _, nh, nkv, hd, pos, _ = PMC_SHAPES[which]
    chunk = min(nh // nkv, 8)
    out = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        groups = {}
        for r in _rows(_find(d, "counter_collection.csv")):
            if r.get("Counter_Name") != counter:
                continue
            name = r["Kernel_Name"]
            key = ("copy" if "neg_kernel" in name else
                   "decode" if re.search(rf"decode_kernel<{hd}, {chunk}[,>]", name)
                   else "combine" if re.search(rf"decode_combine(_wave)?_kernel<{hd}>", name) else None)
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
    alg = decode_bytes(pos + 1, nh, nkv, hd)
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
                     f"cycles; for the prefill, the hi + lo q's second QK product included)")
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
        # this library's kernels
        if not name.startswith(("void pqa::", "pqa::")):
            continue
        grid = tuple(int(r.get(f"Grid_Size_{a}", r.get("Grid_Size", 0)) or 0) for a in "XYZ")
        g = groups.setdefault((name, grid), [])
        g.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = [f"{'kernel':52s} {'grid (threads)':>20s} {'calls':>7s} {'avg us':>9s} {'min us':>9s} {'max us':>9s}"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        short = name.replace("void pqa::", "").replace("pqa::", "").split("(")[0]
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


def secondary_workloads(torch, dev, steps, warmup, cpu_on):
    """The workloads reported beside the headline, in run order (name -> thunk)."""
    return {
        # C3: every layer timed on 1 thread once and T threads 3x, every layer checked
        "qwen3_1.7b_decode": lambda: decode_workload(
            torch, dev, "qwen3_1.7b_decode", 28, 16, 8, 128, 0, 1e6, 32767, 0.0, steps, warmup, True,
            cpu=(range(28), range(28), 1, 3, 3) if cpu_on else None, host_entry=True)[0],
        "qwen3_4b_prefill": lambda: prefill_workload(torch, dev, 36, 32, 8, 128, 2048, max(3, steps // 5), 1,
                                                     cpu=cpu_on, host_entry=True),
        "tinyllama_decode": lambda: decode_workload(
            torch, dev, "tinyllama_decode", 1, 32, 4, 64, 1, 1e4, 511, 0.0, max(steps, 200), warmup, False,
            cpu=((0,), (0,), 21, 21) if cpu_on else None, host_entry=True)[0],
        "qwen2.5_0.5b_sweep": lambda: sweep_workload(torch, dev, cpu=cpu_on),
        "qwen3_8b_kvc_save_load": lambda: kvc_workload(torch, dev),
        "qwen3_8b_qkv_proj": lambda: proj_workload(torch, dev, steps=steps, warmup=warmup, cpu=cpu_on),
        "qwen3_4b_prefill_from_xb": lambda: prefill_x_workload(torch, dev, cpu=cpu_on),
    }


# Phase stamps of the decode kernel (the stamped build, libpqa_stamps.so): slot
# offsets as pqa_decode.hip numbers them, in s_memrealtime ticks (100 MHz).
STAMP_SLOTS, STAMP_WGS = 64, 4096
STAMP_PHASES = [("prologue loads issued", 1), ("q ready (norm, RoPE, LDS)", 10), ("history loop starts", 19),
                ("history loop done", 28)]
STAMP_MERGE, STAMP_END, STAMP_NEW0, STAMP_NEW1 = 37, 38, 39, 40


PSTAMP_SLOTS, PSTAMP_WGS = 64, 4096


def prefill_phase_stamps(reps=5):
    """Per-phase timings of the prefill attention kernel from the stamped build:
    the Qwen3-4B prefill of 2048 tokens (one layer, QK-norm, default hi + lo q).
    Per row block (each workgroup runs a long block, then a short one), the
    median over reps launches of the per-workgroup means (µs from the
    workgroup's first stamp)."""
    import torch
    from picolm_qwen_amd import _lib
    L = _lib.stamped_lib()
    dev = torch.device("cuda:0")
    nh, nkv, hd, s = 32, 8, 128, 2048
    cx = Ctx(1, s, nh, nkv, hd, 0, 1e6, L=L)
    rng = np.random.default_rng(4242)
    set_norms(cx, rng, hd)
    q, k, v, out = make_inputs(torch, dev, rng, 1, s, nh, nkv, hd)
    torch.cuda.synchronize()
    args = [C.c_void_p(t[0].data_ptr()) for t in (q, k, v, out)]
    _, ev = timed(torch, cx, lambda: L.pqa_prefill(cx.h, 0, 0, s, *args), 10, 3)
    rows = []
    for _ in range(reps):
        cx.check(L.pqa_prefill_stamps_clear())
        cx.check(L.pqa_prefill(cx.h, 0, 0, s, *args), cx.h)
        cx.check(L.pqa_sync(cx.h), cx.h)
        a = np.zeros(PSTAMP_WGS * PSTAMP_SLOTS, np.uint64)
        cx.check(L.pqa_prefill_stamps_read(a.ctypes.data_as(C.c_void_p), a.size))
        a = a.reshape(PSTAMP_WGS, PSTAMP_SLOTS).astype(np.int64)
        a = a[a[:, 0] > 0]
        t0 = a[:, :1]
        rel = np.where(a > 0, (a - t0) / 100.0, np.nan)
        ends = np.nanmax(np.where(a > 0, a, np.nan), 1)
        rows.append((len(a), rel, (np.nanmax(ends) - a[:, 0].min()) / 100.0,
                     (a[:, 0].max() - a[:, 0].min()) / 100.0))
    with warnings.catch_warnings():  # stamp slots no wave writes are all-NaN columns
        warnings.simplefilter("ignore", RuntimeWarning)
        med = np.nanmedian(np.stack([np.nanmean(r, 0) for _, r, _, _ in rows]), 0)
    span = float(np.median([x[2] for x in rows]))
    spread = float(np.median([x[3] for x in rows]))
    lines = [f"prefill 2048 tokens, 32/8 heads, hd 128, QK-norm, hi + lo q: {rows[0][0]} workgroups; "
             f"{ev * 1e3:.1f} us per call event-timed (stamped build, with the K/V prep launch); "
             f"first start to last stamp {span:.1f} us; workgroup starts spread over {spread:.2f} us",
             f"  us from the workgroup's start (mean over workgroups, median of {reps} launches); "
             "waves 0-3 take even key tiles, 4-7 odd ones"]
    for j, name in ((0, "long block"), (1, "short block")):
        b = 32 * j
        lines.append(f"  {name}: starts {med[b]:6.2f}")
        lines.append(f"    q rows landed {med[b + 22]:6.2f}   (wave 0: q and the first tiles in LDS)")
        lines.append(f"    q math done   {med[b + 23]:6.2f}   (wave 0: normed, rotated, fp16 in LDS)")
        lines.append("    q ready         " + " ".join(f"{x:6.2f}" for x in med[b + 1:b + 9]))
        lines.append("    tile loop done  " + " ".join(f"{x:6.2f}" for x in med[b + 9:b + 17]))
        lines.append(f"    partials merged {med[b + 17]:6.2f}")
        lines.append("    rows stored     " + " ".join(f"{x:6.2f}" for x in med[b + 18:b + 22]))
    cx.close()
    lines += prefill_step_stamps(reps)
    return "\n".join(lines)


SSTAMP_WGS, SSTAMP_STEPS, SSTAMP_EVENTS = 256, 32, 8


def prefill_step_stamps(reps):
    """Per-step phases of the long block's tile loop, from the build with the
    per-step stamps (waves 0 and 4 of the first 256 workgroups), on the same
    prefill: the mean time of each phase of a step, in ns, over every stamped
    step of every workgroup, median of reps launches. The stamps cost time
    themselves, so this build runs slower than the one without them."""
    import torch
    from picolm_qwen_amd import _lib
    L = _lib.stamped_lib(step=True)
    dev = torch.device("cuda:0")
    nh, nkv, hd, s = 32, 8, 128, 2048
    cx = Ctx(1, s, nh, nkv, hd, 0, 1e6, L=L)
    rng = np.random.default_rng(4242)
    set_norms(cx, rng, hd)
    q, k, v, out = make_inputs(torch, dev, rng, 1, s, nh, nkv, hd)
    torch.cuda.synchronize()
    args = [C.c_void_p(t[0].data_ptr()) for t in (q, k, v, out)]
    _, ev = timed(torch, cx, lambda: L.pqa_prefill(cx.h, 0, 0, s, *args), 10, 3)
    names = ["wait for own tile loads", "workgroup barrier", "issue next tile loads", "score MFMAs + row max",
             "exp, fp16 P, row sums", "PV MFMAs issued", "to the next step"]
    per = []
    for _ in range(reps):
        cx.check(L.pqa_prefill_stamps_clear())
        cx.check(L.pqa_prefill(cx.h, 0, 0, s, *args), cx.h)
        cx.check(L.pqa_sync(cx.h), cx.h)
        a = np.zeros(SSTAMP_WGS * 2 * SSTAMP_STEPS * SSTAMP_EVENTS, np.uint64)
        cx.check(L.pqa_prefill_step_stamps_read(a.ctypes.data_as(C.c_void_p), a.size))
        a = a.reshape(SSTAMP_WGS * 2, SSTAMP_STEPS, SSTAMP_EVENTS).astype(np.float64)
        a[a == 0] = np.nan
        nxt = np.concatenate([a[:, 1:, 0], np.full((a.shape[0], 1), np.nan)], 1)  # next step's start
        d = np.diff(np.concatenate([a[:, :, :7], nxt[:, :, None]], 2), axis=2) * 10.0  # 100 MHz ticks -> ns
        per.append(np.nanmean(d.reshape(-1, 7), 0))
    m = np.median(np.stack(per), 0)
    cx.close()
    lines = [f"  long-block tile loop, per step (both waves of a SIMD one 64-key tile each; the build with per-step "
             f"stamps: {ev * 1e3:.1f} us per call event-timed): mean ns per phase over waves 0 and 4 of every "
             f"workgroup, median of {reps} launches"]
    for nm, x in zip(names, m):
        lines.append(f"    {nm:28s} {x:7.1f}")
    lines.append(f"    {'step total':28s} {float(np.nansum(m)):7.1f}")
    return lines


def phase_stamps(cases=None, reps=7):
    """Per-phase timings of single decode launches from the stamped build: for
    each case, the median over reps launches of each wave's stamps relative to
    its workgroup's start, averaged over workgroups (µs)."""
    import torch
    from picolm_qwen_amd import _lib
    L = _lib.stamped_lib()
    dev = torch.device("cuda:0")
    cases = cases or [("tinyllama ctx 512 (32/4 heads, hd 64, block8)", 32, 4, 64, 1, 1e4, 511, False),
                      ("qwen2.5-0.5b ctx 1 (14/2 heads, hd 64)", 14, 2, 64, 0, 1e6, 0, False),
                      ("qwen2.5-0.5b ctx 301 (14/2 heads, hd 64)", 14, 2, 64, 0, 1e6, 300, False),
                      ("qwen3 16/8 heads hd 128, ctx 201, QK-norm", 16, 8, 128, 0, 1e6, 200, True),
                      ("qwen3-1.7b ctx 32768 (16/8 heads, hd 128, QK-norm; whole-row workgroups)",
                       16, 8, 128, 0, 1e6, 32767, True)]
    lines = []
    for name, nh, nkv, hd, style, base, pos, qk in cases:
        cx = Ctx(1, pos + 1, nh, nkv, hd, style, base, L=L)
        rng = np.random.default_rng(1)
        if qk:
            set_norms(cx, rng, hd)
        if pos:
            cx.check(L.pqa_synth_kv(cx.h, 0, 0, pos, 5, 0.0), cx.h)
        q, k, v, out = make_inputs(torch, dev, rng, 1, 1, nh, nkv, hd)
        torch.cuda.synchronize()
        args = [C.c_void_p(t[0].data_ptr()) for t in (q, k, v, out)]
        _, ev = timed(torch, cx, lambda: L.pqa_decode(cx.h, 0, pos, *args), 200, 20)
        per = []
        for _ in range(reps):
            cx.check(L.pqa_decode_stamps_clear())
            cx.check(L.pqa_decode(cx.h, 0, pos, *args), cx.h)
            cx.check(L.pqa_sync(cx.h), cx.h)
            a = np.zeros(STAMP_WGS * STAMP_SLOTS, np.uint64)
            cx.check(L.pqa_decode_stamps_read(a.ctypes.data_as(C.c_void_p), a.size))
            a = a.reshape(STAMP_WGS, STAMP_SLOTS).astype(np.int64)
            a = a[a[:, 0] > 0]
            rel = np.where(a > 0, (a - a[:, :1]) / 100.0, np.nan)
            per.append((len(a), rel, (a[:, STAMP_END].max() - a[:, 0].min()) / 100.0,
                        (a[:, 0] - a[:, 0].min()) / 100.0, (a[:, STAMP_END] - a[:, 0].min()) / 100.0))
        nwg = per[0][0]
        med = np.nanmedian(np.stack([np.nanmean(x[1], 0) for x in per]), 0)
        span = float(np.median([x[2] for x in per]))
        lines.append(f"{name}: {nwg} workgroup(s); {ev * 1e3:.2f} us per call event-timed (stamped build); "
                     f"first start to last end {span:.2f} us")
        if nwg > 8:
            st = np.median(np.stack([np.percentile(x[3], [0, 50, 100]) for x in per]), 0)
            en = np.median(np.stack([np.percentile(x[4], [0, 50, 100]) for x in per]), 0)
            lines.append(f"  workgroup starts (min/median/max, us after the first) {st[0]:.2f} / {st[1]:.2f} / "
                         f"{st[2]:.2f}; ends {en[0]:.2f} / {en[1]:.2f} / {en[2]:.2f}")
        lines.append("  us from the workgroup's start, per wave 0..8 (mean over workgroups, median of "
                     f"{reps} launches; '  -  ': the wave has no such phase)")
        for label, off in STAMP_PHASES:
            lines.append(f"    {label:28s} " + " ".join("  -  " if np.isnan(x) else f"{x:5.2f}"
                                                       for x in med[off:off + 9]))
        lines.append(f"    {'writer wave: new row':28s} {med[STAMP_NEW0]:5.2f} -> {med[STAMP_NEW1]:5.2f}")
        lines.append(f"    {'workgroup merge starts':28s} {med[STAMP_MERGE]:5.2f}")
        lines.append(f"    {'outputs stored':28s} {med[STAMP_END]:5.2f}")
        cx.close()
        torch.cuda.empty_cache()
    return "\n".join(lines)


def sdpa_compare(reps=50):
    """torch's scaled_dot_product_attention on the Qwen3-4B prefill shape
    (1 x 32 heads x 2048 tokens x 128, causal, the 8 KV heads repeated),
    fp16 and bf16, per backend that this torch offers: the vendor attention
    beside which prefill_attn_kernel is measured (event-timed, µs per call)."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import sdpa_kernel, SDPBackend
    dev = torch.device("cuda:0")
    b, h, hk, s, d = 1, 32, 8, 2048, 128
    flops = 4 * b * h * d * (s * (s + 1) / 2)
    lines = []
    for dt in (torch.float16, torch.bfloat16):
        q = torch.randn(b, h, s, d, device=dev, dtype=dt)
        k = torch.randn(b, hk, s, d, device=dev, dtype=dt).repeat_interleave(h // hk, dim=1).contiguous()
        v = torch.randn(b, hk, s, d, device=dev, dtype=dt).repeat_interleave(h // hk, dim=1).contiguous()
        for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
            try:
                with sdpa_kernel(be):
                    for _ in range(5):
                        F.scaled_dot_product_attention(q, k, v, is_causal=True)
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(reps):
                        F.scaled_dot_product_attention(q, k, v, is_causal=True)
                    e1.record()
                    torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / reps
                lines.append(f"[sdpa] {str(dt).split('.')[-1]:9s} {name:10s} {us:8.2f} us/layer "
                             f"{flops / us / 1e6:7.1f} TFLOP/s")
            except RuntimeError as ex:
                lines.append(f"[sdpa] {str(dt).split('.')[-1]:9s} {name:10s} unavailable ({str(ex)[:80]})")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--pmc-probe", nargs="?", const="c5", choices=sorted(PMC_SHAPES),
                    help="dispatches for the rocprofv3 --pmc passes (c5, the default, or c3)")
    ap.add_argument("--pmc-shape", default="c5", choices=sorted(PMC_SHAPES), help="decode shape of --summarize-pmc")
    ap.add_argument("--only", choices=["qwen3_1.7b_decode", "qwen3_4b_prefill", "tinyllama_decode",
                                       "qwen2.5_0.5b_sweep", "qwen3_8b_kvc_save_load", "qwen3_8b_qkv_proj",
                                       "qwen3_4b_prefill_from_xb"],
                    help="run one secondary workload and print it")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--summarize-trace", metavar="TRACE_DIR")
    ap.add_argument("--summarize-counters", nargs="+", metavar="PMC_DIR",
                    help="per-dispatch counter averages of the kernels named by --kernel")
    ap.add_argument("--kernel", default="prefill_attn_kernel")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="per-phase decode and prefill timings from the stamped build (libpqa_stamps.so)")
    ap.add_argument("--ref-attn-child", metavar="NPZ", help=argparse.SUPPRESS)
    ap.add_argument("--sdpa-compare", action="store_true",
                    help="torch scaled_dot_product_attention on the Qwen3-4B prefill shape, for comparison")
    args = ap.parse_args()
    if args.sdpa_compare:
        print(sdpa_compare(), flush=True)
        return
    if args.phase_stamps:
        print(phase_stamps(), flush=True)
        print(prefill_phase_stamps(), flush=True)
        return
    if args.ref_attn_child:
        ref_attention_child(args.ref_attn_child)
        return
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.kernel))
        return
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc, which=args.pmc_shape))
        return
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode would shard by KV head with no exchange)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.pmc_probe:
        pmc_probe(torch, dev, args.pmc_probe)
        return
    cpu_on = not args.no_cpu
    runs = secondary_workloads(torch, dev, args.steps, args.warmup, cpu_on)
    if args.only:
        print(json.dumps({args.only: runs[args.only]()}), flush=True)
        return

    nh, nkv, hd, layers, pos = 32, 8, 128, 36, 131071
    Ctx.deferred = []  # every context lives until the end of the run (see Ctx)
    host = cpu_host()
    log(f"[bench] host CPU: {host}")
    # C5: 1 thread on layer 0 once, T threads 3x; layers 0, 17 and 35 checked (35's slice starts past 4 GiB)
    head = decode_workload(torch, dev, "qwen3_8b_decode", layers, nh, nkv, hd, 0, 1e6, pos, 0.01,
                           args.steps, args.warmup, True, cpu=((0,), (0, 17, 35), 1, 3, 1) if cpu_on else None,
                           host_entry=not args.quick)[0]
    cpu = head.get("cpu_baseline")

    workloads = {"qwen3_8b_decode": head}
    if not args.quick:
        for name, run in runs.items():
            workloads[name] = run()

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
        "warmup_min_ms": WARMUP_MIN_MS,
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
        "cpu_host": host,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)
    Ctx.close_deferred()


if __name__ == "__main__":
    main()
