"""ctypes bindings for the CPU oracle (liboracle.so) and the reference harness
(_ref/libref_{A,B}.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never as a compute path of the product.

Functions restated from the reference (rain1201/picolm_qwen) and the pin of
each one (closed form, exhaustive KAT or golden vector) are listed in
oracle/pqa_oracle.h. q4k_term_magnitudes (the per-element terms of the
any-order Q4_K sums' error bound) is pinned by a closed-form block and by its
limits against the dequantization (tests/test_oracle_proj.py).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
ORACLE_BENCH_SO = os.path.join(HERE, "liboracle_bench.so")
REF_SO = {"A": os.path.join(HERE, "_ref", "libref_A.so"), "B": os.path.join(HERE, "_ref", "libref_B.so"),
          "kvc": os.path.join(HERE, "_ref", "libref_kvc.so")}

ROPE_NEOX_HALF, ROPE_LLAMA_X86_BLOCK8, ROPE_LLAMA_INTERLEAVED = 0, 1, 2
KIND_Q, KIND_K, KIND_V, KIND_KHIST, KIND_VHIST, KIND_QNORM, KIND_KNORM, KIND_OUTLIER = range(1, 9)

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")


class Shape(C.Structure):
    _fields_ = [("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("max_seq_len", C.c_int), ("rope_style", C.c_int)]


_lib = None
_bench_lib = None
_AVX512 = ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")


def lib():
    """Loads liboracle.so (built by `make -C oracle`): the checker."""
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle not built: {ORACLE_SO} missing (run make -C oracle)")
        _lib = _bind(C.CDLL(ORACLE_SO))
    return _lib


def host_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return all(x in flags for x in _AVX512)
    except OSError:
        pass
    return False


def bench_lib():
    """The oracle as the reference builds its own code (-O3, FP contraction,
    x86-64-v4), used only to time the CPU baseline. Returns (library, flags
    description); falls back to the checker build when liboracle_bench.so is
    missing or this CPU lacks AVX-512."""
    global _bench_lib
    if _bench_lib is None:
        if os.path.exists(ORACLE_BENCH_SO) and host_has_avx512():
            _bench_lib = (_bind(C.CDLL(ORACLE_BENCH_SO)), "gcc -O3 -march=x86-64-v4 -ffp-contract=fast")
        else:
            _bench_lib = (lib(), "gcc -O3 -march=x86-64-v3 -ffp-contract=off (checker build; no AVX-512 build here)")
    return _bench_lib


def _bind(L):
    L.pqo_fp16_to_fp32.restype = C.c_float
    L.pqo_fp16_to_fp32.argtypes = [C.c_uint16]
    L.pqo_fp32_to_fp16.restype = C.c_uint16
    L.pqo_fp32_to_fp16.argtypes = [C.c_float]
    L.pqo_fp16_to_fp32_array.argtypes = [_u16p, _f32p, C.c_size_t]
    L.pqo_fp32_to_fp16_array.argtypes = [_f32p, _u16p, C.c_size_t]
    L.pqo_fp32_bits_to_fp16_range.argtypes = [C.c_uint32, C.c_size_t, _u16p, C.c_int]
    L.pqo_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int]
    L.pqo_rope.argtypes = [C.c_int, _f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
    L.pqo_rope_table.argtypes = [C.c_float, C.c_int, C.c_int, _f32p, _f32p]
    L.pqo_rope_rows.argtypes = [C.c_float, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
    vp = C.c_void_p
    L.pqo_attn_step.argtypes = [C.POINTER(Shape), C.c_int, _f32p, _f32p, _f32p, vp, vp, _f32p, _f32p,
                                _u16p, _u16p, _f32p, C.c_int]
    L.pqo_attend.argtypes = [C.POINTER(Shape), C.c_int, _f32p, _u16p, _u16p, _f32p, C.c_int]
    L.pqo_append.argtypes = [C.POINTER(Shape), C.c_int, _f32p, _f32p, _f32p, vp, vp, _f32p, _f32p,
                             _u16p, _u16p]
    L.pqo_prefill.argtypes = [C.POINTER(Shape), C.c_int, C.c_int, _f32p, _f32p, _f32p, vp, vp, _f32p,
                              _f32p, _u16p, _u16p, _f32p, C.c_int, C.c_int]
    L.pqo_attend_f64.argtypes = [C.POINTER(Shape), C.c_int, _f32p, _u16p, _u16p, _f64p]
    L.pqo_splitmix64.restype = C.c_uint64
    L.pqo_splitmix64.argtypes = [C.c_uint64, C.c_uint64]
    L.pqo_stream_key.restype = C.c_uint64
    L.pqo_stream_key.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32]
    L.pqo_normal.restype = C.c_float
    L.pqo_normal.argtypes = [C.c_uint64, C.c_uint64]
    L.pqo_fill_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, _f32p]
    L.pqo_is_outlier.restype = C.c_int
    L.pqo_is_outlier.argtypes = [C.c_uint64, C.c_uint32, C.c_uint64, C.c_float]
    L.pqo_synth_kv_rows.argtypes = [C.c_uint64, C.c_uint32, C.c_int, C.c_int, C.c_int, C.c_float,
                                    _u16p, _u16p, C.c_int]
    L.pqo_row_bytes.restype = C.c_size_t
    L.pqo_row_bytes.argtypes = [C.c_int, C.c_int]
    L.pqo_dequant_row.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_int]
    L.pqo_vec_dot.restype = C.c_float
    L.pqo_vec_dot.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_int]
    L.pqo_matmul_bias.argtypes = [_f32p, _f32p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int]
    L.pqo_matmul_bias_tokens.argtypes = [_f32p, _f32p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int,
                                         C.c_int, C.c_int]
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def shape(n_heads, n_kv_heads, head_dim, max_seq_len, rope_style):
    return Shape(n_heads, n_kv_heads, head_dim, max_seq_len, rope_style)


# ---- numerics -------------------------------------------------------------

def fp32_to_fp16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().pqo_fp32_to_fp16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def fp16_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().pqo_fp16_to_fp32_array(h.reshape(-1), out.reshape(-1), h.size)
    return out


def fp32_bits_to_fp16(first, n, n_threads=8):
    out = np.empty(n, dtype=np.uint16)
    lib().pqo_fp32_bits_to_fp16_range(first, n, out, n_threads)
    return out


def rmsnorm(x, w):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().pqo_rmsnorm(out, x, np.ascontiguousarray(w, dtype=np.float32), x.size)
    return out


def rope(style, q, k, head_dim, n_heads, n_kv_heads, cos_row, sin_row):
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    lib().pqo_rope(style, q.reshape(-1), k.reshape(-1), head_dim, n_heads, n_kv_heads,
                   np.ascontiguousarray(cos_row, dtype=np.float32),
                   np.ascontiguousarray(sin_row, dtype=np.float32))
    return q, k


def rope_table(base, head_dim, max_seq_len):
    half = head_dim // 2
    c = np.empty((max_seq_len, half), dtype=np.float32)
    s = np.empty((max_seq_len, half), dtype=np.float32)
    lib().pqo_rope_table(base, head_dim, max_seq_len, c.reshape(-1), s.reshape(-1))
    return c, s


def rope_rows(base, head_dim, pos0, n):
    half = head_dim // 2
    c = np.empty((n, half), dtype=np.float32)
    s = np.empty((n, half), dtype=np.float32)
    lib().pqo_rope_rows(base, head_dim, pos0, n, c.reshape(-1), s.reshape(-1))
    return c, s


def attn_step(shp, pos, q, k, v, q_norm_w, k_norm_w, cos_row, sin_row, kc, vc, n_threads=1, L=None):
    """Decode block at `pos`; kc/vc (layer slice, uint16 [S_max, kv_dim]) are updated in place.
    L: the library to run (default the checker; bench_lib()[0] for timing)."""
    out = np.empty(shp.n_heads * shp.head_dim, dtype=np.float32)
    qn = None if q_norm_w is None else np.ascontiguousarray(q_norm_w, dtype=np.float32)
    kn = None if k_norm_w is None else np.ascontiguousarray(k_norm_w, dtype=np.float32)
    (L or lib()).pqo_attn_step(C.byref(shp), pos, np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                        np.ascontiguousarray(k, dtype=np.float32).reshape(-1),
                        np.ascontiguousarray(v, dtype=np.float32).reshape(-1), _ptr(qn), _ptr(kn),
                        np.ascontiguousarray(cos_row, dtype=np.float32).reshape(-1),
                        np.ascontiguousarray(sin_row, dtype=np.float32).reshape(-1),
                        kc.reshape(-1), vc.reshape(-1), out, n_threads)
    return out


def attend(shp, pos, q, kc, vc, n_threads=1):
    out = np.empty(shp.n_heads * shp.head_dim, dtype=np.float32)
    lib().pqo_attend(C.byref(shp), pos, np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                     kc.reshape(-1), vc.reshape(-1), out, n_threads)
    return out


def append(shp, pos, q, k, v, q_norm_w, k_norm_w, cos_row, sin_row, kc, vc):
    """Norm + RoPE + fp16 append; returns the normed, roped q."""
    q = np.array(q, dtype=np.float32, copy=True).reshape(-1)
    qn = None if q_norm_w is None else np.ascontiguousarray(q_norm_w, dtype=np.float32)
    kn = None if k_norm_w is None else np.ascontiguousarray(k_norm_w, dtype=np.float32)
    lib().pqo_append(C.byref(shp), pos, q, np.ascontiguousarray(k, dtype=np.float32).reshape(-1),
                     np.ascontiguousarray(v, dtype=np.float32).reshape(-1), _ptr(qn), _ptr(kn),
                     np.ascontiguousarray(cos_row, dtype=np.float32).reshape(-1),
                     np.ascontiguousarray(sin_row, dtype=np.float32).reshape(-1),
                     kc.reshape(-1), vc.reshape(-1))
    return q


def prefill(shp, start, q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, kc, vc, serial=False,
            n_threads=8, L=None):
    n_tok = q.shape[0]
    out = np.empty((n_tok, shp.n_heads * shp.head_dim), dtype=np.float32)
    qn = None if q_norm_w is None else np.ascontiguousarray(q_norm_w, dtype=np.float32)
    kn = None if k_norm_w is None else np.ascontiguousarray(k_norm_w, dtype=np.float32)
    (L or lib()).pqo_prefill(C.byref(shp), start, n_tok, np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                      np.ascontiguousarray(k, dtype=np.float32).reshape(-1),
                      np.ascontiguousarray(v, dtype=np.float32).reshape(-1), _ptr(qn), _ptr(kn),
                      np.ascontiguousarray(cos_tab, dtype=np.float32).reshape(-1),
                      np.ascontiguousarray(sin_tab, dtype=np.float32).reshape(-1),
                      kc.reshape(-1), vc.reshape(-1), out.reshape(-1), 1 if serial else 0, n_threads)
    return out


def attend_f64(shp, pos, q, kc, vc):
    out = np.empty(shp.n_heads * shp.head_dim, dtype=np.float64)
    lib().pqo_attend_f64(C.byref(shp), pos, np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                         kc.reshape(-1), vc.reshape(-1), out)
    return out


# ---- synthetic inputs -------------------------------------------------------

def stream_key(seed, kind, layer):
    return lib().pqo_stream_key(seed, kind, layer)


def normal(seed, kind, layer, first, n, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().pqo_fill_normal(stream_key(seed, kind, layer), first, n, mean, std, out)
    return out


def synth_kv_rows(seed, layer, kv_dim, pos0, n, outlier_prob=0.0, n_threads=8):
    k = np.empty((n, kv_dim), dtype=np.uint16)
    v = np.empty((n, kv_dim), dtype=np.uint16)
    if n > 0:
        lib().pqo_synth_kv_rows(seed, layer, kv_dim, pos0, n, outlier_prob, k.reshape(-1), v.reshape(-1),
                                n_threads)
    return k, v


def step_inputs(seed, layer, token, n_heads, n_kv_heads, head_dim):
    """q/k/v fp32 ~N(0,1) of one token (index `token` of the layer's streams)."""
    q_dim, kv_dim = n_heads * head_dim, n_kv_heads * head_dim
    q = normal(seed, KIND_Q, layer, token * q_dim, q_dim)
    k = normal(seed, KIND_K, layer, token * kv_dim, kv_dim)
    v = normal(seed, KIND_V, layer, token * kv_dim, kv_dim)
    return q, k, v


def batch_inputs(seed, layer, start_token, n_tok, n_heads, n_kv_heads, head_dim):
    q_dim, kv_dim = n_heads * head_dim, n_kv_heads * head_dim
    q = normal(seed, KIND_Q, layer, start_token * q_dim, n_tok * q_dim).reshape(n_tok, q_dim)
    k = normal(seed, KIND_K, layer, start_token * kv_dim, n_tok * kv_dim).reshape(n_tok, kv_dim)
    v = normal(seed, KIND_V, layer, start_token * kv_dim, n_tok * kv_dim).reshape(n_tok, kv_dim)
    return q, k, v


def qk_norm_weights(seed, layer, head_dim):
    """QK-RMSNorm weights ~N(1, 0.02)."""
    return (normal(seed, KIND_QNORM, layer, 0, head_dim, 1.0, 0.02),
            normal(seed, KIND_KNORM, layer, 0, head_dim, 1.0, 0.02))


# ---- Q/K/V projections (cpp/tensor.hpp:110-143, cpp/quant.hpp:176-358) ---------

GGUF_NONE, GGUF_F32, GGUF_F16, GGUF_Q4_0, GGUF_Q8_0, GGUF_Q4_K, GGUF_Q6_K = 0, 1, 2, 3, 9, 13, 15
GGUF_BLOCK = {GGUF_F32: (1, 4), GGUF_F16: (1, 2), GGUF_Q4_0: (32, 18), GGUF_Q8_0: (32, 34),
              GGUF_Q4_K: (256, 144), GGUF_Q6_K: (256, 210)}  # (elements, bytes) per block


def row_bytes(wtype, n):
    return int(lib().pqo_row_bytes(wtype, n))


def _vp(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def dequant_row(wtype, raw, n):
    out = np.empty(n, np.float32)
    if lib().pqo_dequant_row(wtype, _vp(np.ascontiguousarray(raw)), out, n):
        raise ValueError("unsupported type or shape")
    return out


def vec_dot(wtype, raw_row, x):
    x = np.ascontiguousarray(x, np.float32)
    return float(lib().pqo_vec_dot(wtype, _vp(np.ascontiguousarray(raw_row)), x, x.size))


def q4k_term_magnitudes(raw, n):
    """|d q| + |m| per element of Q4_K rows [rows][row bytes] of n elements,
    float64 [rows][n]: w = d q - m with d = d_super * sc and m = dmin * mn of
    the element's 32-element group (get_scale_min_k4 and dequantize_row_q4_K,
    cpp/quant.hpp:210-236). The terms a sum in the form d sum q x - m sum x
    rounds, for its error bound."""
    rows = raw.shape[0]
    blk = np.ascontiguousarray(raw).reshape(rows, n // 256, 144)
    d = blk[:, :, 0:2].copy().view("<f2")[..., 0].astype(np.float32)
    dmin = blk[:, :, 2:4].copy().view("<f2")[..., 0].astype(np.float32)
    sc = blk[:, :, 4:16].astype(np.int64)
    qs = blk[:, :, 16:144].astype(np.int64)
    out = np.zeros((rows, n // 256, 256), np.float64)
    for j in range(8):
        if j < 4:
            s_, m_ = sc[..., j] & 63, sc[..., j + 4] & 63
        else:
            s_ = (sc[..., j + 4] & 0xF) | ((sc[..., j - 4] >> 6) << 4)
            m_ = (sc[..., j + 4] >> 4) | ((sc[..., j] >> 6) << 4)
        d1 = (d * s_.astype(np.float32)).astype(np.float64)
        m1 = (dmin * m_.astype(np.float32)).astype(np.float64)
        jj, hi = j // 2, j % 2
        q = (qs[..., 32 * jj:32 * jj + 32] >> (4 * hi)) & 0xF
        out[..., 64 * jj + 32 * hi:64 * jj + 32 * hi + 32] = np.abs(d1[..., None] * q) + np.abs(m1[..., None])
    return out.reshape(rows, n)


def matmul_bias(x, w_raw, wtype, d, b_raw=None, btype=GGUF_NONE):
    """out[d] = W x (+ b): w_raw uint8 [d][row_bytes], b_raw uint8 bias row or None."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(d, np.float32)
    if lib().pqo_matmul_bias(out, x, _vp(np.ascontiguousarray(w_raw)), wtype,
                             _vp(None if b_raw is None else np.ascontiguousarray(b_raw)), btype, x.size, d):
        raise ValueError("unsupported type or shape")
    return out


def matmul_bias_tokens(x, w_raw, wtype, d, b_raw=None, btype=GGUF_NONE, n_threads=8):
    """matmul_bias of every row of x [n_tok][n] -> [n_tok][d], rows split over threads."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], d), np.float32)
    if lib().pqo_matmul_bias_tokens(out.reshape(-1), x.reshape(-1), x.shape[0], _vp(np.ascontiguousarray(w_raw)),
                                    wtype, _vp(None if b_raw is None else np.ascontiguousarray(b_raw)), btype,
                                    x.shape[1], d, n_threads):
        raise ValueError("unsupported type or shape")
    return out


# ---- reference harness (only where it was built) -----------------------------

class RefModel:
    """The reference's Model::forward driven through oracle/ref_harness.cpp."""

    _libs = {}

    @classmethod
    def available(cls, variant="B"):
        return os.path.exists(REF_SO[variant])

    @classmethod
    def load(cls, variant="B"):
        if variant in cls._libs:
            return cls._libs[variant]
        L = C.CDLL(REF_SO[variant])
        L.ref_open.restype = C.c_void_p
        L.ref_open.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, C.c_int]
        L.ref_set_qk_norm.argtypes = [C.c_void_p, _f32p, _f32p]
        L.ref_set_cache_rows.argtypes = [C.c_void_p, C.c_int, C.c_int, _u16p, _u16p]
        L.ref_get_cache_rows.argtypes = [C.c_void_p, C.c_int, C.c_int, _u16p, _u16p]
        L.ref_get_rope_rows.argtypes = [C.c_void_p, C.c_int, C.c_int, _f32p, _f32p]
        L.ref_step.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p, _f32p, _f32p]
        L.ref_close.argtypes = [C.c_void_p]
        L.ref_fp32_bits_to_fp16_range.argtypes = [C.c_uint32, C.c_size_t, _u16p]
        L.ref_fp16_to_fp32_all.argtypes = [_f32p]
        L.ref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int]
        L.ref_rope.argtypes = [C.c_int, _f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
        L.ref_dequantize_row.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_int]
        L.ref_vec_dot.restype = C.c_float
        L.ref_vec_dot.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_int]
        L.ref_matmul_bias.argtypes = [_f32p, _f32p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int]
        cls._libs[variant] = L
        return L

    def __init__(self, n_heads, n_kv_heads, head_dim, max_seq_len, rope_base, rope_qwen, qk_norm,
                 variant="B", path=None):
        import tempfile
        self.L = self.load(variant)
        self.nh, self.nkv, self.hd, self.smax = n_heads, n_kv_heads, head_dim, max_seq_len
        fd, self.path = tempfile.mkstemp(suffix=".gguf") if path is None else (None, path)
        if fd is not None:
            os.close(fd)
        self.h = self.L.ref_open(self.path.encode(), n_heads, n_kv_heads, head_dim, max_seq_len,
                                 rope_base, int(rope_qwen), int(qk_norm))
        if not self.h:
            raise RuntimeError("reference Model::load failed")

    def set_qk_norm(self, qw, kw):
        self.L.ref_set_qk_norm(self.h, np.ascontiguousarray(qw, np.float32), np.ascontiguousarray(kw, np.float32))

    def set_cache_rows(self, pos0, k, v):
        n = k.shape[0]
        if n:
            self.L.ref_set_cache_rows(self.h, pos0, n, np.ascontiguousarray(k).reshape(-1),
                                      np.ascontiguousarray(v).reshape(-1))

    def cache_rows(self, pos0, n):
        kv = self.nkv * self.hd
        k = np.empty((n, kv), np.uint16)
        v = np.empty((n, kv), np.uint16)
        self.L.ref_get_cache_rows(self.h, pos0, n, k.reshape(-1), v.reshape(-1))
        return k, v

    def rope_rows(self, pos0, n):
        half = self.hd // 2
        c = np.empty((n, half), np.float32)
        s = np.empty((n, half), np.float32)
        self.L.ref_get_rope_rows(self.h, pos0, n, c.reshape(-1), s.reshape(-1))
        return c, s

    def step(self, pos, q, k, v):
        out = np.empty(self.nh * self.hd, np.float32)
        self.L.ref_step(self.h, pos, np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                        np.ascontiguousarray(v, np.float32), out)
        return out

    def close(self):
        if self.h:
            self.L.ref_close(self.h)
            self.h = None
        if self.path and os.path.exists(self.path):
            os.unlink(self.path)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- .kvc KV-cache files (picolm/model.c:870-983) ----------------------------
#
# Restated with numpy on whole caches [n_layers][max_seq_len][kv_dim] uint16.
# Pinned in tests/test_oracle_kvc.py against the reference's compiled
# kvcache_save / kvcache_load (RefKvc below) on every branch of both, against
# a committed file written by kvcache_save, and against the format's closed
# form (length 16 + 4*n_layers*n_pos*kv_dim, the magic bytes "PCVK" on disk).

KVC_MAGIC = 0x4B564350  # picolm/model.h:12


def kvc_file_bytes(key_cache, val_cache, n_pos):
    """kvcache_save (picolm/model.c:882-921): the file for rows [0, n_pos).
    Returns None where the reference returns -1 without writing (n_pos outside
    [1, max_seq_len])."""
    n_layers, max_seq_len, kv_dim = key_cache.shape
    if n_pos <= 0 or n_pos > max_seq_len:
        return None
    header = np.array([KVC_MAGIC, n_pos, n_layers, kv_dim], dtype="<u4")      # :895-901
    body_k = np.ascontiguousarray(key_cache[:, :n_pos], dtype="<u2")            # :905-910
    body_v = np.ascontiguousarray(val_cache[:, :n_pos], dtype="<u2")            # :911-916
    return header.tobytes() + body_k.tobytes() + body_v.tobytes()


def kvc_load_bytes(data, key_cache, val_cache):
    """kvcache_load (picolm/model.c:923-983) of file contents `data` into the
    caches, in place. Returns what the reference returns: the header's n_pos
    (an int32, so a count of 2^31 or more is negative and loads nothing), or 0
    on a short header, bad magic, shape mismatch, n_pos > max_seq_len or a
    short body; a short body leaves the bytes it held in place, as the
    row-by-row fread does (:961-978)."""
    n_layers, max_seq_len, kv_dim = key_cache.shape
    if len(data) < 16:                                                          # :932-935
        return 0
    magic, n_pos_u, file_layers, file_kv_dim = np.frombuffer(data[:16], dtype="<u4").tolist()
    to_i32 = lambda u: u - (1 << 32) if u >= (1 << 31) else u
    n_pos, file_layers, file_kv_dim = to_i32(n_pos_u), to_i32(file_layers), to_i32(file_kv_dim)
    if magic != KVC_MAGIC:                                                      # :937-941
        return 0
    if file_layers != n_layers or file_kv_dim != kv_dim:                        # :947-952
        return 0
    if n_pos > max_seq_len:                                                     # :953-958
        return 0
    if n_pos <= 0:
        return n_pos
    body = memoryview(data)[16:]
    run = n_pos * kv_dim * 2
    off = 0
    for cache in (key_cache, val_cache):
        flat = cache.reshape(n_layers, -1).view(np.uint8)
        for layer in range(n_layers):
            take = max(0, min(run, len(body) - off))
            flat[layer, :take] = np.frombuffer(body[off:off + take], dtype=np.uint8)
            off += take
            if take < run:
                return 0
    return n_pos


class RefKvc:
    """The reference's kvcache_save / kvcache_load via oracle/ref_kvc_harness.c."""

    _lib = None

    @classmethod
    def available(cls):
        return os.path.exists(REF_SO["kvc"])

    @classmethod
    def load(cls):
        if cls._lib is None:
            L = C.CDLL(REF_SO["kvc"])
            args = [_u16p, _u16p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_char_p]
            L.refkvc_save.argtypes = args + [C.c_int]
            L.refkvc_load.argtypes = args
            cls._lib = L
        return cls._lib

    @classmethod
    def save(cls, key_cache, val_cache, n_kv_heads, head_dim, path, n_pos):
        n_layers, max_seq_len, _ = key_cache.shape
        return cls.load().refkvc_save(np.ascontiguousarray(key_cache, np.uint16),
                                      np.ascontiguousarray(val_cache, np.uint16), n_layers, max_seq_len,
                                      n_kv_heads, head_dim, os.fsencode(path), n_pos)

    @classmethod
    def load_into(cls, key_cache, val_cache, n_kv_heads, head_dim, path):
        """Loads in place (caches must be C-contiguous uint16)."""
        assert key_cache.flags.c_contiguous and val_cache.flags.c_contiguous
        n_layers, max_seq_len, _ = key_cache.shape
        return cls.load().refkvc_load(key_cache, val_cache, n_layers, max_seq_len, n_kv_heads, head_dim,
                                      os.fsencode(path))


class RefProj:
    """The reference's dequantize_row / vec_dot / TensorOps::matmul_bias
    (oracle/ref_harness.cpp, build B unless stated)."""

    def __init__(self, variant="B"):
        self.L = RefModel.load(variant)

    def dequant_row(self, wtype, raw, n):
        out = np.empty(n, np.float32)
        self.L.ref_dequantize_row(_vp(np.ascontiguousarray(raw)), out, n, wtype)
        return out

    def vec_dot(self, wtype, raw_row, x):
        x = np.ascontiguousarray(x, np.float32)
        return float(self.L.ref_vec_dot(_vp(np.ascontiguousarray(raw_row)), x, x.size, wtype))

    def matmul_bias(self, x, w_raw, wtype, d, b_raw=None, btype=GGUF_NONE):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(d, np.float32)
        self.L.ref_matmul_bias(out, x, _vp(np.ascontiguousarray(w_raw)),
                               _vp(None if b_raw is None else np.ascontiguousarray(b_raw)), x.size, d, wtype,
                               btype if b_raw is not None else GGUF_NONE)
        return out
