"""mlxr_k_sample_noalloc (the entry point that allocates nothing) against mlxr_k_sample, through
the C ABI: two calls in a row, the second with a smaller vocabulary, greedy and sampled, and the
size limit. Token, status and the sampler state must be bit-identical."""
import ctypes

import numpy as np
import pytest

from qfix import XorShift

pytestmark = pytest.mark.gpu


def _logits(V, seed):
    rng = XorShift(seed)
    l = np.random.default_rng(seed).uniform(-12, -6, V).astype(np.float32)
    for i in range(0, V, 97):
        l[i] += 8 + 4 * rng.float()
    l[V // 3] = l[V - 1] = np.max(l) + 0.5   # a tie at the top: the lower index wins
    return l


def _run(mlxr, fn, logits, params, history, seed):
    V = len(logits)
    hist = np.zeros(len(history) + 2, np.int32)
    hist[:len(history)] = history
    dh = mlxr.DeviceArray.from_numpy(hist)
    st = mlxr.DeviceArray.zeros(len(history) + 2, np.int32)
    rng = mlxr.DeviceArray.from_numpy(np.array([seed, 0], np.uint64))
    dl = mlxr.DeviceArray.from_numpy(logits)
    pos = len(history) - 1
    sp = params.params(V)
    if fn == "noalloc":
        rc = mlxr.lib.mlxr_k_sample_noalloc(dl.ptr, V, dh.ptr, st.ptr, rng.ptr, pos, ctypes.byref(sp), None)
    else:
        rc = mlxr.lib.mlxr_k_sample(dl.ptr, V, dh.ptr, st.ptr, rng.ptr, pos, ctypes.byref(sp))
    mlxr.check(rc)
    mlxr.synchronize()
    return int(dh.numpy()[pos + 1]), int(st.numpy()[pos + 1]), rng.numpy().tobytes(), dl.numpy()


@pytest.mark.parametrize("params", ["greedy", "sampled"])
def test_sample_noalloc_matches_sample(gpu, params):
    p = (gpu.SamplingParameters(temperature=0, repetition_penalty=1.2, repetition_window=16) if params == "greedy"
         else gpu.SamplingParameters(temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.1))
    history = [3, 17, 99, 5, 3]
    for V, seed in ((151936, 11), (1000, 12)):   # the second call smaller: stale partials must not leak
        print(f"[case] noalloc {params} V={V}", flush=True)
        l = _logits(V, seed)
        want = _run(gpu, "alloc", l.copy(), p, history, seed)
        got = _run(gpu, "noalloc", l.copy(), p, history, seed)
        assert got[0] == want[0] and got[1] == want[1] and got[2] == want[2], (V, got[:2], want[:2])
        assert np.array_equal(got[3].view(np.uint32), want[3].view(np.uint32))


def test_sample_noalloc_rejects_oversize(gpu):
    V = 262144 + 256
    dl = gpu.DeviceArray.zeros((16,), np.float32)
    d = gpu.DeviceArray.zeros((4,), np.int32)
    r = gpu.DeviceArray.zeros((2,), np.uint64)
    sp = gpu.SamplingParameters.greedy().params(V)
    rc = gpu.lib.mlxr_k_sample_noalloc(dl.ptr, V, d.ptr, d.ptr, r.ptr, 0, ctypes.byref(sp), None)
    assert rc == -10
    assert "exceeds" in gpu.lib.mlxr_last_error().decode()
