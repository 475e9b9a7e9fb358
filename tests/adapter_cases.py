"""The compiled forward-loop adapter (picolm_qwen_amd/adapter/forward_demo.cpp
over include/pqa_forward.hpp) driven from the tests: a small random Qwen-style
model with F32 weights, the attention RMSNorm and an FFN stand-in passed in as
callbacks, and the reference's own layer loop restated on the oracle to check it
(cpp/model.hpp:311-451 per token, :489-626 per prompt)."""
import ctypes as C
import os

import numpy as np

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEMO = os.path.join(ROOT, "picolm_qwen_amd", "adapter", "libpqa_forward_demo.so")

NORM_FN = C.CFUNCTYPE(None, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_float), C.c_void_p)
FFN_FN = C.CFUNCTYPE(None, C.c_int, C.POINTER(C.c_float), C.c_void_p)

_lib = None


def demo_lib():
    global _lib
    if _lib is None:
        if not os.path.exists(DEMO):
            raise RuntimeError(f"{DEMO} is not built: run __graft_entry__.build()")
        L = C.CDLL(DEMO)
        fp = C.c_void_p
        L.pqaf_demo_run.restype = C.c_int
        L.pqaf_demo_run.argtypes = ([C.c_int] * 6 + [C.c_int, C.c_float] + [fp] * 10 +
                                    [C.c_int, fp, C.c_int, fp, NORM_FN, FFN_FN, fp, C.c_char_p, C.c_int])
        _lib = L
    return _lib


class Model:
    """Random weights of one small Qwen-style attention stack (F32 GGUF rows)."""

    def __init__(self, seed, n_layers=2, n_embd=512, n_heads=8, n_kv_heads=2, head_dim=64, max_seq_len=64,
                 rope_base=1e6, qk_norm=True, bias=True):
        rng = np.random.default_rng(seed)
        self.L, self.n, self.nh, self.nkv, self.hd = n_layers, n_embd, n_heads, n_kv_heads, head_dim
        self.smax, self.base = max_seq_len, rope_base
        qd, kvd = n_heads * head_dim, n_kv_heads * head_dim
        self.qd, self.kvd = qd, kvd
        s = 1.0 / np.sqrt(n_embd)
        f = lambda *shape: (rng.standard_normal(shape) * s).astype(np.float32)  # noqa: E731
        self.wq, self.wk, self.wv = f(n_layers, qd, n_embd), f(n_layers, kvd, n_embd), f(n_layers, kvd, n_embd)
        self.wo = (rng.standard_normal((n_layers, n_embd, qd)) / np.sqrt(qd)).astype(np.float32)
        b = lambda *shape: (rng.standard_normal(shape) * 0.1).astype(np.float32) if bias else None  # noqa: E731
        self.bq, self.bk, self.bv, self.bo = b(n_layers, qd), b(n_layers, kvd), b(n_layers, kvd), b(n_layers, n_embd)
        if qk_norm:
            self.qn = (1.0 + 0.2 * rng.standard_normal((n_layers, head_dim))).astype(np.float32)
            self.kn = (1.0 + 0.2 * rng.standard_normal((n_layers, head_dim))).astype(np.float32)
        else:
            self.qn = self.kn = None
        self.attn_norm_w = (1.0 + 0.1 * rng.standard_normal((n_layers, n_embd))).astype(np.float32)
        self.ffn_w = (0.5 * rng.standard_normal((n_layers, n_embd))).astype(np.float32)

    # the callbacks: the reference's rmsnorm (cpp/model.hpp:314) and an FFN
    # stand-in, the same float32 arithmetic in the demo and in the chain below
    def attn_norm(self, layer, x):
        return O.rmsnorm(x, self.attn_norm_w[layer])

    def ffn(self, layer, x):
        return (x + np.float32(0.25) * np.tanh(x * self.ffn_w[layer])).astype(np.float32)

    def run_demo(self, x_prompt, x_decode):
        """Drives pqaf_demo_run; returns (rc, message); x_prompt and x_decode are
        updated in place."""
        L = demo_lib()
        n = self.n

        def norm_cb(layer, xb, x, _user):
            xs = np.ctypeslib.as_array(x, shape=(n,))
            np.ctypeslib.as_array(xb, shape=(n,))[:] = self.attn_norm(layer, xs)

        def ffn_cb(layer, x, _user):
            xs = np.ctypeslib.as_array(x, shape=(n,))
            xs[:] = self.ffn(layer, xs)

        ncb, fcb = NORM_FN(norm_cb), FFN_FN(ffn_cb)
        p = lambda a: None if a is None else a.ctypes.data_as(C.c_void_p)  # noqa: E731
        err = C.create_string_buffer(512)
        for a in (x_prompt, x_decode):
            assert a.dtype == np.float32 and a.flags.c_contiguous and a.shape[-1] == n
        rc = L.pqaf_demo_run(self.L, n, self.nh, self.nkv, self.hd, self.smax, 0, self.base, p(self.wq), p(self.wk),
                             p(self.wv), p(self.wo), p(self.bq), p(self.bk), p(self.bv), p(self.bo), p(self.qn),
                             p(self.kn), x_prompt.shape[0], p(x_prompt), x_decode.shape[0], p(x_decode), ncb, fcb,
                             None, err, len(err))
        return rc, err.value.decode(errors="replace")

    def reference_chain(self, x_prompt, x_decode):
        """The reference's loops on the oracle: for each layer, each prompt token
        (cpp/model.hpp:489-626), then each decode token through every layer
        (:311-451). Returns the residual streams after the last layer."""
        shp = O.shape(self.nh, self.nkv, self.hd, self.smax, 0)
        cos, sin = O.rope_table(self.base, self.hd, self.smax)
        kc = np.zeros((self.L, self.smax, self.kvd), np.uint16)
        vc = np.zeros_like(kc)
        F32 = O.GGUF_F32
        raw = lambda a: a.view(np.uint8)  # noqa: E731

        def braw(b, layer):
            return (None, O.GGUF_NONE) if b is None else (raw(b[layer]), F32)

        def block(layer, pos, x):
            xb = self.attn_norm(layer, x)
            q = O.matmul_bias(xb, raw(self.wq[layer]), F32, self.qd, *braw(self.bq, layer))
            k = O.matmul_bias(xb, raw(self.wk[layer]), F32, self.kvd, *braw(self.bk, layer))
            v = O.matmul_bias(xb, raw(self.wv[layer]), F32, self.kvd, *braw(self.bv, layer))
            qn = None if self.qn is None else self.qn[layer]
            kn = None if self.kn is None else self.kn[layer]
            attn = O.attn_step(shp, pos, q, k, v, qn, kn, cos[pos], sin[pos], kc[layer], vc[layer])
            x = (x + O.matmul_bias(attn, raw(self.wo[layer]), F32, self.n, *braw(self.bo, layer))).astype(np.float32)
            return self.ffn(layer, x)

        xp = np.array(x_prompt, np.float32, copy=True)
        xd = np.array(x_decode, np.float32, copy=True)
        for layer in range(self.L):
            for i in range(xp.shape[0]):
                xp[i] = block(layer, i, xp[i])
        for t in range(xd.shape[0]):
            for layer in range(self.L):
                xd[t] = block(layer, xp.shape[0] + t, xd[t])
        return xp, xd, kc, vc
