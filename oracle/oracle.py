"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker or the timed CPU baseline. The product (libmlxr, mlx-runner_amd/mlxr.py) never
imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    P, I, F = C.c_void_p, C.c_int, C.c_float
    sig = {
        "orc_bf16_to_f32": (F, [C.c_uint16]), "orc_f32_to_bf16": (C.c_uint16, [F]),
        "orc_f16_to_f32": (F, [C.c_uint16]), "orc_f32_to_f16": (C.c_uint16, [F]), "orc_round_bf16": (F, [F]),
        "orc_pack": (None, [P, C.c_int64, I, P]), "orc_unpack": (None, [P, C.c_int64, I, P]),
        "orc_qlinear_f64": (None, [P, P, I, P]),
        "orc_qlinear_f16": (None, [P, P, I, P]), "orc_qlinear_prefill": (None, [P, P, I, P]),
        "orc_round_f16_d": (C.c_double, [C.c_double]),
        "orc_dequant_row": (None, [P, I, P]),
        "orc_rms_norm": (None, [P, P, P, I, I, F]), "orc_inv_freq": (None, [C.c_double, I, P]),
        "orc_rope": (None, [P, I, I, I, I, P]), "orc_silu_mul": (F, [F, F]),
        "orc_attention": (None, [P, P, P, I, I, I, I, I, F, P]),
        "orc_attention_list": (None, [P, P, P, I, I, I, I, I, F, P, I, I, P]),
        "orc_sparse_make_plan": (I, [I, I, I, I, I, P]), "orc_sparse_clamp": (None, [P, P, P, P, I]),
        "orc_sparse_index": (None, [P, I, I, I, I, I, I, P]),
        "orc_sparse_score": (None, [P, P, I, I, I, I, I, I, P]), "orc_sparse_key": (C.c_uint32, [F]),
        "orc_sparse_select": (None, [P, I, P, P]),
        "orc_argmax": (I, [P, I]),
        "orc_sample_distribution": (I, [P, I, P, I, F, I, F, F, F, P, P, I]),
        "orc_model_load": (P, [C.c_char_p, I]), "orc_model_free": (None, [P]), "orc_last_error": (C.c_char_p, []),
        "orc_model_vocab": (I, [P]), "orc_model_hidden": (I, [P]),
        "orc_forward": (I, [P, P, I, I, I, P]), "orc_model_set_sparse": (None, [P, I, I, I, I, I, I]),
        "orc_model_set_kv": (I, [P, I, P, P, I]), "orc_model_threads": (I, []),
    }
    for n, (r, a) in sig.items():
        f = getattr(lib, n)
        f.restype = r
        f.argtypes = a
    return lib


lib = _load()


class QLinear(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p), ("bias", C.c_void_p),
                ("O", C.c_int), ("K", C.c_int), ("bits", C.c_int), ("gs", C.c_int)]


class SparsePlan(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("pool", "b0", "nb", "p", "sink_end", "win_start", "L", "count")]


def _ptr(a):
    return a.ctypes.data if a is not None else None


def pack(codes, bits):
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    out = np.zeros((codes.size * bits + 7) // 8, np.uint8)
    lib.orc_pack(codes.ctypes.data, codes.size, bits, out.ctypes.data)
    return out


def unpack(packed, n, bits):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(n, np.uint32)
    lib.orc_unpack(packed.ctypes.data, n, bits, out.ctypes.data)
    return out


class QMatrix:
    """Host quantized matrix: packed [O][K*bits/8] bytes, float scales/biases [O][K/gs]."""

    def __init__(self, packed, scales, biases, K, bits, gs, bias=None):
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8)
        self.scales = np.ascontiguousarray(scales, dtype=np.float32)
        self.biases = np.ascontiguousarray(biases, dtype=np.float32)
        self.bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self.O = self.scales.shape[0]
        self.K, self.bits, self.gs = K, bits, gs
        self.s = QLinear(self.packed.ctypes.data, self.scales.ctypes.data, self.biases.ctypes.data, _ptr(self.bias),
                         self.O, K, bits, gs)

    def matmul_f64(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.K)
        y = np.zeros((x.shape[0], self.O), np.float32)
        lib.orc_qlinear_f64(C.byref(self.s), x.ctypes.data, x.shape[0], y.ctypes.data)
        return y

    def matmul_f16(self, x):
        """The 4-bit tile GEMM's precision: per-row power-of-two scaled f16 x, f16(fma(s, q, b)) weights."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.K)
        y = np.zeros((x.shape[0], self.O), np.float32)
        lib.orc_qlinear_f16(C.byref(self.s), x.ctypes.data, x.shape[0], y.ctypes.data)
        return y

    def matmul_prefill(self, x):
        """The model prefill's precision for this matrix (the tile GEMM's f16 operands for 4-bit gs
        32/64/128 with K / gs even, else fp32-level: the double product)."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.K)
        y = np.zeros((x.shape[0], self.O), np.float32)
        lib.orc_qlinear_prefill(C.byref(self.s), x.ctypes.data, x.shape[0], y.ctypes.data)
        return y

    def dequant_row(self, r):
        out = np.zeros(self.K, np.float32)
        lib.orc_dequant_row(C.byref(self.s), r, out.ctypes.data)
        return out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    dim = x.shape[-1]
    y = np.zeros_like(x)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib.orc_rms_norm(x.ctypes.data, y.ctypes.data, w.ctypes.data, dim, x.size // dim, C.c_float(eps))
    return y


def inv_freq(theta, rot_dim):
    out = np.zeros(rot_dim // 2, np.float32)
    lib.orc_inv_freq(theta, rot_dim, out.ctypes.data)
    return out


def rope(v, pos, inv_f, rot_dim=None, traditional=False):
    v = np.array(v, dtype=np.float32, copy=True)
    D = v.size
    lib.orc_rope(v.ctypes.data, D, rot_dim or D, int(traditional), pos, np.ascontiguousarray(inv_f, np.float32).ctypes.data)
    return v


def attention(q, kc, vc, nH, nKV, pos, scale):
    """q [nH][D]; kc/vc [nKV][max_seq][D] float."""
    q = np.ascontiguousarray(q, np.float32); kc = np.ascontiguousarray(kc, np.float32); vc = np.ascontiguousarray(vc, np.float32)
    D = q.shape[-1]
    out = np.zeros((nH, D), np.float32)
    lib.orc_attention(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, D, nH, nKV, kc.shape[1], pos, C.c_float(scale), out.ctypes.data)
    return out


def attention_list(q, kc, vc, nH, nKV, pos, scale, lists, count, list_stride):
    q = np.ascontiguousarray(q, np.float32); kc = np.ascontiguousarray(kc, np.float32); vc = np.ascontiguousarray(vc, np.float32)
    lists = np.ascontiguousarray(lists, np.int32)
    D = q.shape[-1]
    out = np.zeros((nH, D), np.float32)
    lib.orc_attention_list(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, D, nH, nKV, kc.shape[1], pos, C.c_float(scale),
                           lists.ctypes.data, count, list_stride, out.ctypes.data)
    return out


def sparse_plan(top_k, window, sink, min_context, position):
    p = SparsePlan()
    ok = lib.orc_sparse_make_plan(top_k, window, sink, min_context, position, C.byref(p))
    return p if ok else None


def sparse_clamp(top_k, window, sink, min_context=None):
    a, b, c, d = C.c_int(top_k), C.c_int(window), C.c_int(sink), C.c_int(min_context or 0)
    lib.orc_sparse_clamp(C.byref(a), C.byref(b), C.byref(c), C.byref(d), 0 if min_context is None else 1)
    return a.value, b.value, c.value, d.value


def sparse_index(kc, nKV, D, max_seq, b0, nb):
    kc = np.ascontiguousarray(kc, np.float32)
    idx = np.zeros(((max_seq // 4 + 1), nKV, D), np.float32)
    lib.orc_sparse_index(kc.ctypes.data, nKV, D, max_seq, 4, b0, nb, idx.ctypes.data)
    return idx


def sparse_score(q, idx, nH, nKV, D, b0, nb, rows):
    q = np.ascontiguousarray(q, np.float32); idx = np.ascontiguousarray(idx, np.float32)
    out = np.zeros(rows * nb, np.float32)
    lib.orc_sparse_score(q.ctypes.data, idx.ctypes.data, nH, nKV, D, b0, nb, rows, out.ctypes.data)
    return out.reshape(rows, nb)


def sparse_key(f):
    return lib.orc_sparse_key(C.c_float(f))


def sparse_select(scores, plan):
    scores = np.ascontiguousarray(scores, np.float32)
    out = np.zeros(plan.count, np.int32)
    lib.orc_sparse_select(scores.ctypes.data, plan.nb, C.byref(plan), out.ctypes.data)
    return out


def argmax(logits):
    l = np.ascontiguousarray(logits, np.float32)
    return lib.orc_argmax(l.ctypes.data, l.size)


def sample_distribution(logits, recent, temperature, top_k, top_p, min_p, penalty, max_out=4096):
    l = np.array(logits, dtype=np.float32, copy=True)
    r = np.ascontiguousarray(recent, np.int32)
    ids = np.zeros(max_out, np.int32); pr = np.zeros(max_out, np.float32)
    n = lib.orc_sample_distribution(l.ctypes.data, l.size, r.ctypes.data, r.size, C.c_float(temperature), top_k,
                                    C.c_float(top_p), C.c_float(min_p), C.c_float(penalty), ids.ctypes.data, pr.ctypes.data, max_out)
    if n < 0:
        return None
    return ids[:n].copy(), pr[:n].copy()


class Model:
    """The oracle's whole-model forward over an MLX model directory."""

    def __init__(self, directory, max_seq):
        self.h = lib.orc_model_load(directory.encode(), max_seq)
        if not self.h:
            raise RuntimeError(lib.orc_last_error().decode())
        self.vocab = lib.orc_model_vocab(self.h)
        self.max_seq = max_seq

    def forward(self, tokens, offset, small_t=1 << 30):
        """Logits of the last token (fp32 semantics: every product in double precision). small_t is a
        diagnostic: chunks longer than small_t tokens use the GPU GEMM's operand precision instead."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(self.vocab, np.float32)
        rc = lib.orc_forward(self.h, t.ctypes.data, t.size, offset, small_t, out.ctypes.data)
        if rc:
            raise RuntimeError(lib.orc_last_error().decode())
        return out

    def set_sparse(self, enabled, top_k=2048, window=512, sink=4, min_context=0, per_head=True):
        tk, w, s, mc = sparse_clamp(top_k, window, sink, min_context if min_context > 0 else None)
        lib.orc_model_set_sparse(self.h, int(enabled), tk, w, s, mc, int(per_head))

    def set_kv(self, layer, k, v):
        k = np.ascontiguousarray(k, np.float32); v = np.ascontiguousarray(v, np.float32)
        assert lib.orc_model_set_kv(self.h, layer, k.ctypes.data, v.ctypes.data, k.shape[1]) == 0

    def close(self):
        if self.h:
            lib.orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def threads():
    return lib.orc_model_threads()
