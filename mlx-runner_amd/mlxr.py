"""Python host binding of libmlxr (ctypes over include/mlxr.h).

Mirrors the reference's engine surface (Sources/MLXEngine/Transformer.swift:642-1303):
`Transformer(directory, context_length, sparse)` with `forward`, `prefill`, `begin_decode_step`,
`finish`, `reusable_prefix`, `reset_write_tracking`, `seed_sampler`, `sparse`, `last_gpu_time`;
`SparseAttention` (SparseAttention.swift:29-78) and `SamplingParameters` (Engine.swift:3-16).
Errors raise `EngineError` carrying the reference's case name (GPU.swift:4-33).

The library is loaded from this directory (built by build.py); a missing library raises
ImportError — there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MLXR_LIB") or os.path.join(_HERE, "libmlxr.so")

ERRORS = {
    -1: "noMetalDevice", -2: "invalidFile", -3: "missingTensor", -4: "unsupported", -5: "contextFull",
    -6: "outOfMemory", -7: "cancelled", -8: "invalidOutput", -9: "gpuFailure", -10: "invalidArgument",
}


class EngineError(RuntimeError):
    def __init__(self, code: int, message: str):
        self.code = code
        self.case = ERRORS.get(code, f"error{code}")
        super().__init__(f"{self.case}: {message}")


class SparseCfg(C.Structure):
    _fields_ = [("top_k", C.c_int32), ("window", C.c_int32), ("sink", C.c_int32), ("min_context", C.c_int32),
                ("per_head", C.c_int32)]


class SampleParams(C.Structure):
    _fields_ = [("V", C.c_int32), ("pos", C.c_int32), ("window", C.c_int32), ("top_k", C.c_int32),
                ("penalty", C.c_float), ("temperature", C.c_float), ("top_p", C.c_float), ("min_p", C.c_float)]


class Step(C.Structure):
    _fields_ = [("id", C.c_int64), ("offset", C.c_int32)]


class QMat(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p), ("bias", C.c_void_p), ("O", C.c_int32)]


CancelFn = C.CFUNCTYPE(C.c_int, C.c_void_p)   # mlxr_cancel_fn


def _cancel_fn(is_cancelled):
    """A C callback for an isCancelled closure (a null function pointer for None). The caller keeps
    the returned object alive for the duration of the call."""
    if is_cancelled is None:
        return CancelFn()
    return CancelFn(lambda _user: 1 if is_cancelled() else 0)


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run `python mlx-runner_amd/build.py`")
    lib = C.CDLL(LIB_PATH)
    P, I, F, V = C.c_void_p, C.c_int, C.c_float, None
    sig = {
        "mlxr_model_open": (I, [C.c_char_p, I, C.POINTER(SparseCfg), C.POINTER(P)]),
        "mlxr_model_close": (V, [P]),
        "mlxr_vocab_size": (I, [P]), "mlxr_max_seq": (I, [P]), "mlxr_hidden_size": (I, [P]), "mlxr_num_layers": (I, [P]),
        "mlxr_weight_bytes": (C.c_int64, [P]), "mlxr_device_bytes": (C.c_int64, [P]),
        "mlxr_quant_description": (C.c_char_p, [P]), "mlxr_sparse_available": (I, [P]), "mlxr_written_high": (I, [P]),
        "mlxr_forward": (I, [P, P, I, I, I, I, C.POINTER(C.POINTER(F)), CancelFn, P]),
        "mlxr_prefill": (I, [P, P, I, I, C.POINTER(SampleParams), C.POINTER(C.c_int32), CancelFn, P]),
        "mlxr_step_logits": (I, [P, C.POINTER(C.POINTER(F))]),
        "mlxr_begin_decode": (I, [P, I, C.POINTER(SampleParams), C.POINTER(Step)]),
        "mlxr_begin_steps": (I, [P, P, I, I, C.POINTER(SampleParams), C.POINTER(Step)]),
        "mlxr_model_type": (C.c_char_p, [P]), "mlxr_eos_token_ids": (I, [P, P, I]), "mlxr_is_hybrid": (I, [P]),
        "mlxr_supports_batched_verify": (I, [P]), "mlxr_sparse_layer_count": (I, [P]), "mlxr_sparse_off_reason": (C.c_char_p, [P]),
        "mlxr_finish": (I, [P, C.POINTER(Step), C.POINTER(C.c_int32)]),
        "mlxr_reusable_prefix": (I, [P, I, I]), "mlxr_reset_write_tracking": (V, [P]),
        "mlxr_seed_sampler": (I, [P, C.c_uint64]), "mlxr_set_sparse": (I, [P, C.POINTER(SparseCfg)]),
        "mlxr_last_gpu_time": (C.c_double, [P]), "mlxr_read_kv": (I, [P, I, I, P, P]), "mlxr_set_graphs": (I, [P, I]), "mlxr_set_decode_mode": (I, [P, I]), "mlxr_decode_mode": (I, [P]), "mlxr_decode_mode_reason": (C.c_char_p, [P]), "mlxr_profile_decode_phases": (I, [P, I, P, I]), "mlxr_debug_stall_next_step": (I, [P]),
        "mlxr_profile_kernel": (I, [P, C.c_char_p, I, I, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
        "mlxr_synth_write": (I, [C.c_char_p, C.c_uint64, F, C.c_char_p]),
        "mlxr_quantize_row": (I, [P, I, I, I, P, P, P]),
        "mlxr_synth_matrix": (I, [C.c_uint64, C.c_uint64, I, I, I, I, F, P, P, P]),
        "mlxr_device_count": (I, []), "mlxr_device_name": (C.c_char_p, []),
        "mlxr_dev_alloc": (I, [C.POINTER(P), C.c_size_t]), "mlxr_dev_free": (I, [P]),
        "mlxr_memcpy_h2d": (I, [P, P, C.c_size_t]), "mlxr_memcpy_d2h": (I, [P, P, C.c_size_t]),
        "mlxr_memset": (I, [P, I, C.c_size_t]), "mlxr_synchronize": (I, []), "mlxr_last_error": (C.c_char_p, []),
        "mlxr_timer_start": (I, []), "mlxr_timer_stop": (I, [C.POINTER(F)]),
        "mlxr_k_qmv": (I, [C.POINTER(QMat), I, I, I, I, I, P, P, F, P, I]),
        "mlxr_k_qmm": (I, [C.POINTER(QMat), I, I, I, I, I, I, P, I, P, I]),
        "mlxr_k_qgemm": (I, [C.POINTER(QMat), I, I, I, I, I, P, I, P, I]),
        "mlxr_k_qgemm_tiles": (I, [C.POINTER(QMat), I, I, I, I, I, P, I, P, I]),
        "mlxr_k_qmv_tiles": (I, [C.POINTER(QMat), I, I, I, I, P, P, C.c_float, P, I]),
        "mlxr_k_qmm_tiles": (I, [C.POINTER(QMat), I, I, I, I, I, P, I, P, F, P, I]),
        "mlxr_k_qembed": (I, [C.POINTER(QMat), I, I, I, I, P, I, P]),
        "mlxr_k_rms_norm": (I, [P, P, P, P, I, I, F]),
        "mlxr_k_qkv_post": (I, [P, I, P, P, P, I, P, P, I, I, I, I, I, I, I, F]),
        "mlxr_k_attention": (I, [P, I, P, P, I, I, I, I, I, I, F, P, I, P, I, I, I]),
        "mlxr_k_flash_prefill": (I, [P, I, P, P, I, I, I, I, I, I, F, P, I]),
        "mlxr_k_sparse_index": (I, [P, I, I, I, I, I, P]),
        "mlxr_k_sparse_score": (I, [P, P, I, I, I, I, I, I, P]),
        "mlxr_k_sparse_select": (I, [P, I, I, I, I, I, I, I, P, I]),
        "mlxr_k_sample": (I, [P, I, P, P, P, I, C.POINTER(SampleParams)]),
        "mlxr_k_sample_noalloc": (I, [P, I, P, P, P, I, C.POINTER(SampleParams), P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int):
    if rc != 0:
        raise EngineError(rc, lib.mlxr_last_error().decode(errors="replace"))


# --------------------------------------------------------------------------------- device memory
class DeviceArray:
    """A device allocation holding a numpy-described array (upload / download helpers)."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib.mlxr_dev_alloc(C.byref(p), max(self.nbytes, 16)))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(lib.mlxr_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes))
        return d

    @classmethod
    def zeros(cls, shape, dtype):
        d = cls(shape, dtype)
        check(lib.mlxr_memset(d.ptr, 0, d.nbytes))
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(lib.mlxr_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(lib.mlxr_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def free(self):
        if self.ptr:
            lib.mlxr_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    check(lib.mlxr_synchronize())


def device_count() -> int:
    return lib.mlxr_device_count()


# --------------------------------------------------------------------------------- engine types
@dataclasses.dataclass
class SamplingParameters:
    """Engine.swift:3-16 (defaults as the reference)."""
    temperature: float = 0.7
    top_p: float = 0.95
    top_k: int = 40
    min_p: float = 0.0
    repetition_penalty: float = 1.05
    repetition_window: int = 64

    @staticmethod
    def greedy():
        return SamplingParameters(temperature=0.0, repetition_penalty=1.0)

    def params(self, vocab: int) -> SampleParams:
        return SampleParams(vocab, 0, max(0, self.repetition_window), self.top_k, self.repetition_penalty,
                            self.temperature, self.top_p, self.min_p)


@dataclasses.dataclass
class SparseAttention:
    """SparseAttention.swift:29-54: the sparse decode attention budget (clamped by the library)."""
    top_k: int = 2048
    window: int = 512
    sink: int = 4
    min_context: int = 0     # 0: 2 * (sink + top_k + window)
    per_head: bool = True

    def cfg(self) -> SparseCfg:
        return SparseCfg(self.top_k, self.window, self.sink, self.min_context, 1 if self.per_head else 0)

    @staticmethod
    def from_environment(env=None):
        """SparseAttention.parse(environment:) (SparseAttention.swift:62-78)."""
        env = os.environ if env is None else env
        s = env.get("MLXR_SPARSE_ATTN", "").strip().lower()
        if s in ("", "1", "on", "true", "yes"):
            top_k = 2048
        else:
            try:
                top_k = int(s)
            except ValueError:
                return None
            if top_k <= 1:
                return None

        def num(k):
            try:
                return int(env[k].strip())
            except (KeyError, ValueError):
                return None
        w = num("MLXR_SPARSE_WINDOW")
        mc = num("MLXR_SPARSE_MIN")
        return SparseAttention(top_k=top_k, window=512 if w is None else w, sink=4, min_context=mc or 0,
                               per_head=env.get("MLXR_SPARSE_SHARED", "").strip() != "1")


class DecodeStep:
    def __init__(self, step: Step):
        self._s = step
        self.offset = step.offset


class Transformer:
    """A decoder-only transformer on the MI355X (Transformer.swift:642)."""

    def __init__(self, directory: str, context_length: int = 4096, sparse: SparseAttention | None = None):
        h = C.c_void_p()
        cfg = sparse.cfg() if sparse is not None else None
        check(lib.mlxr_model_open(directory.encode(), int(context_length), C.byref(cfg) if cfg is not None else None,
                                  C.byref(h)))
        self._h = h.value
        self._sparse = sparse if sparse is not None and self.sparse_available else None
        self.vocab_size = lib.mlxr_vocab_size(self._h)
        self.max_seq = lib.mlxr_max_seq(self._h)
        self.hidden_size = lib.mlxr_hidden_size(self._h)
        self.num_layers = lib.mlxr_num_layers(self._h)
        self.weight_bytes = lib.mlxr_weight_bytes(self._h)
        self.quant_description = lib.mlxr_quant_description(self._h).decode()

    def close(self):
        if getattr(self, "_h", None):
            lib.mlxr_model_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def sparse_available(self) -> bool:
        return bool(lib.mlxr_sparse_available(self._h))

    @property
    def written_high(self) -> int:
        return lib.mlxr_written_high(self._h)

    @property
    def last_gpu_time(self) -> float:
        return lib.mlxr_last_gpu_time(self._h)

    @property
    def sparse(self) -> SparseAttention | None:
        """The sparse decode attention budget in use (Transformer.sparse, :813), None when off."""
        return self._sparse

    def set_sparse(self, sparse: SparseAttention | None):
        cfg = sparse.cfg() if sparse is not None else None
        check(lib.mlxr_set_sparse(self._h, C.byref(cfg) if cfg is not None else None))
        self._sparse = sparse

    def profile_kernel(self, kind: str, iters: int = 100, context: int = 1):
        """(mean launch ms, algorithmic bytes per launch) of one decode kernel class."""
        ms, b = C.c_double(), C.c_int64()
        check(lib.mlxr_profile_kernel(self._h, kind.encode(), iters, context, C.byref(ms), C.byref(b)))
        return ms.value, b.value

    def set_decode_mode(self, mode):
        """True / 1: the persistent step where the model allows it; False / 0: one kernel per operation
        (repacked tiles where the model has them); 2: one kernel per operation on the MLX layout."""
        check(lib.mlxr_set_decode_mode(self._h, int(mode)))

    @property
    def persistent_decode(self) -> bool:
        return bool(lib.mlxr_decode_mode(self._h))

    @property
    def persistent_decode_reason(self) -> str:
        """Why dense steps run kernel by kernel ("" when the persistent step runs them)."""
        return lib.mlxr_decode_mode_reason(self._h).decode()

    def profile_decode_phases(self, offset: int):
        """[(mean start, mean end, latest end) us] of each interval of one persistent decode step."""
        out = np.zeros(3 * 1024, np.float64)
        n = lib.mlxr_profile_decode_phases(self._h, offset, out.ctypes.data, 1024)
        if n < 0:
            check(n)
        return out[:3 * n].reshape(n, 3)

    def profile_decode_marks(self, offset: int):
        """Raw wall-clock marks (us) of one persistent decode step: [workgroup][mark], -1 unset."""
        out = np.zeros(4096 * 1024, np.float64)
        n = lib.mlxr_profile_decode_phases(self._h, offset, out.ctypes.data, -1)
        if n < 0:
            check(n)
        return out[:n * 1024].reshape(n, 1024)

    def debug_stall_next_step(self):
        """Makes the next persistent decode step's first wait expire (mlxr_debug_stall_next_step)."""
        check(lib.mlxr_debug_stall_next_step(self._h))

    def set_graphs(self, on: bool):
        check(lib.mlxr_set_graphs(self._h, 1 if on else 0))

    def forward(self, tokens, offset: int, all_logits: bool = False, dense: bool = False, is_cancelled=None) -> np.ndarray:
        """forward(_:offset:allLogits:dense:isCancelled:): is_cancelled() is polled between chunks."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = C.POINTER(C.c_float)()
        cb = _cancel_fn(is_cancelled)
        check(lib.mlxr_forward(self._h, t.ctypes.data, len(t), int(offset), int(all_logits), int(dense), C.byref(out), cb, None))
        rows = len(t) if all_logits else 1
        arr = np.ctypeslib.as_array(out, shape=(rows * self.vocab_size,)).copy()
        return arr.reshape(rows, self.vocab_size) if all_logits else arr

    def prefill(self, tokens, offset: int, sample: SamplingParameters, is_cancelled=None) -> int:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        sp = sample.params(self.vocab_size)
        tok = C.c_int32()
        cb = _cancel_fn(is_cancelled)
        check(lib.mlxr_prefill(self._h, t.ctypes.data, len(t), int(offset), C.byref(sp), C.byref(tok), cb, None))
        return tok.value

    def step_logits(self) -> np.ndarray:
        """Logits of the last finished decode step (mlxr_step_logits)."""
        out = C.POINTER(C.c_float)()
        check(lib.mlxr_step_logits(self._h, C.byref(out)))
        return np.ctypeslib.as_array(out, shape=(self.vocab_size,)).copy()

    def begin_decode_step(self, offset: int, sample: SamplingParameters) -> DecodeStep:
        sp = sample.params(self.vocab_size)
        st = Step()
        check(lib.mlxr_begin_decode(self._h, int(offset), C.byref(sp), C.byref(st)))
        return DecodeStep(st)

    def begin_steps(self, tokens, offset: int, sample: SamplingParameters) -> DecodeStep:
        """beginSteps (Transformer.swift:1265-1296): tokens at offset.., one step selecting the
        token after the last, not waited for (finish it like a decode step)."""
        t = np.ascontiguousarray(tokens, np.int32)
        sp = sample.params(self.vocab_size)
        st = Step()
        check(lib.mlxr_begin_steps(self._h, t.ctypes.data, int(t.size), int(offset), C.byref(sp), C.byref(st)))
        return DecodeStep(st)

    @property
    def model_type(self) -> str:
        return lib.mlxr_model_type(self._h).decode()

    @property
    def eos_token_ids(self) -> list:
        n = lib.mlxr_eos_token_ids(self._h, None, 0)
        out = np.zeros(max(n, 1), np.int32)
        lib.mlxr_eos_token_ids(self._h, out.ctypes.data, n)
        return out[:n].tolist()

    @property
    def sparse_layer_count(self) -> int:
        return lib.mlxr_sparse_layer_count(self._h)

    @property
    def sparse_off_reason(self) -> str:
        return lib.mlxr_sparse_off_reason(self._h).decode()

    @property
    def is_hybrid(self) -> bool:
        return bool(lib.mlxr_is_hybrid(self._h))

    @property
    def supports_batched_verify(self) -> bool:
        return bool(lib.mlxr_supports_batched_verify(self._h))

    def finish(self, step: DecodeStep) -> int:
        tok = C.c_int32()
        check(lib.mlxr_finish(self._h, C.byref(step._s), C.byref(tok)))
        return tok.value

    def reusable_prefix(self, common: int, previous_length: int) -> int:
        return lib.mlxr_reusable_prefix(self._h, int(common), int(previous_length))

    def reset_write_tracking(self):
        lib.mlxr_reset_write_tracking(self._h)

    def seed_sampler(self, seed: int):
        check(lib.mlxr_seed_sampler(self._h, C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)))

    def read_kv(self, layer: int, rows: int, nkv: int, head_dim: int):
        k = np.empty((nkv, rows, head_dim), np.float32)
        v = np.empty_like(k)
        check(lib.mlxr_read_kv(self._h, layer, rows, k.ctypes.data, v.ctypes.data))
        return k, v

    def generate(self, prompt, max_tokens: int, sample: SamplingParameters, offset: int = 0, stop=()):
        """The pipelined GPU-sampled loop of InferenceEngine.run (Engine.swift:740-763): step n+1 is
        committed before step n is read back; at most two steps in flight."""
        first = self.prefill(prompt, offset, sample)
        out = [first]
        pos = offset + len(prompt)
        if max_tokens <= 1 or first in stop:
            return out
        cur = self.begin_decode_step(pos, sample)
        while True:
            nxt = None
            if len(out) + 1 < max_tokens and cur.offset + 2 < self.max_seq:
                nxt = self.begin_decode_step(cur.offset + 1, sample)
            tok = self.finish(cur)
            out.append(tok)
            if tok in stop or len(out) >= max_tokens or nxt is None:
                if nxt is not None:
                    self.finish(nxt)
                return out
            cur = nxt


def synth_write(config: dict | str, seed: int, directory: str, std: float = 0.02):
    """Writes a seeded synthetic MLX-format model directory (see mlxr_synth_write)."""
    import json
    text = config if isinstance(config, str) else json.dumps(config)
    check(lib.mlxr_synth_write(text.encode(), C.c_uint64(seed), C.c_float(std), directory.encode()))


def synth_matrix(seed: int, tensor_id: int, O: int, K: int, bits: int, group_size: int, std: float = 0.02):
    """One seeded matrix drawn and quantized as mlxr_synth_write draws its tensors: (codes [O][K*bits/8]
    uint8, bf16 scales [O][K/gs] uint16, bf16 biases [O][K/gs] uint16)."""
    codes = np.zeros((O, K * bits // 8), np.uint8)
    s = np.zeros((O, K // group_size), np.uint16)
    b = np.zeros((O, K // group_size), np.uint16)
    check(lib.mlxr_synth_matrix(C.c_uint64(seed), C.c_uint64(tensor_id), O, K, bits, group_size, C.c_float(std),
                                codes.ctypes.data, s.ctypes.data, b.ctypes.data))
    return codes, s, b


def quantize_row(w: np.ndarray, bits: int, group_size: int):
    w = np.ascontiguousarray(w, dtype=np.float32)
    K = w.size
    codes = np.zeros(K * bits // 8, np.uint8)
    s = np.zeros(K // group_size, np.uint16)
    b = np.zeros(K // group_size, np.uint16)
    check(lib.mlxr_quantize_row(w.ctypes.data, K, bits, group_size, codes.ctypes.data, s.ctypes.data, b.ctypes.data))
    return codes, s, b
