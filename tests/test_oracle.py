"""Pins of the CPU oracle (CPU only). Each check uses something the oracle's own code does not:
closed forms, known answers, invariants, numpy/scipy routines, or the reference tests' own
restatements (Tests/MLXEngineTests). The reference commits no golden vectors for this path.
"""
import math

import numpy as np
import pytest

import oracle
from qfix import QuantFixture, XorShift, bf16_round, bf16_to_f32, pack_codes, unpack_codes


# ---------------------------------------------------------------------------------------- formats
def test_bf16_known_answers():
    f = lambda bits: np.array([bits], np.uint32).view(np.float32)[0]
    assert oracle.lib.orc_f32_to_bf16(1.0) == 0x3F80
    assert oracle.lib.orc_f32_to_bf16(float(f(0x3F808000))) == 0x3F80      # tie -> even
    assert oracle.lib.orc_f32_to_bf16(float(f(0x3F818000))) == 0x3F82      # tie -> even (up)
    assert oracle.lib.orc_f32_to_bf16(float(f(0x3F808001))) == 0x3F81      # above the tie
    assert oracle.lib.orc_f32_to_bf16(-2.0) == 0xC000
    assert oracle.lib.orc_f32_to_bf16(float("inf")) == 0x7F80
    assert (oracle.lib.orc_f32_to_bf16(float("nan")) & 0x7FC0) == 0x7FC0
    assert oracle.lib.orc_bf16_to_f32(0x4049) == np.float32(3.140625)


def test_f16_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.normal(0, 1, 2000), rng.normal(0, 1e-5, 200), [65504.0, 1e-8, -0.0, 6.1e-5]]).astype(np.float32)
    for v in vals:
        h = oracle.lib.orc_f32_to_f16(float(v))
        assert h == np.float32(v).astype(np.float16).view(np.uint16), v
        assert oracle.lib.orc_f16_to_f32(h) == np.float16(v).astype(np.float32)


# ---------------------------------------------------------------------------------------- packing
def test_pack_known_answer():
    # codes 1, 2, 3 at 3 bits: stream bits 100 010 110 -> byte 0 = 0b11010001, byte 1 = 0
    assert oracle.pack([1, 2, 3], 3).tolist() == [0xD1, 0x00]
    # 4 bits: two codes per byte, first code in the low nibble (MLX uint32 little-endian)
    assert oracle.pack([0xA, 0x5, 0xF, 0x0], 4).tolist() == [0x5A, 0x0F]


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_pack_unpack_against_bit_arrays(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, 4096).astype(np.uint32)
    p = oracle.pack(codes, bits)
    assert np.array_equal(p, pack_codes(codes, bits))          # numpy bit arrays (independent)
    assert np.array_equal(oracle.unpack(p, codes.size, bits), codes)
    assert np.array_equal(unpack_codes(p, codes.size, bits), codes)


# ---------------------------------------------------------------------------------------- linear
@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 32), (4, 64), (5, 64), (6, 128), (8, 64)])
def test_qlinear_against_numpy(bits, gs):
    fx = QuantFixture(24, 256, bits, gs, seed=bits)
    x = XorShift(bits).floats(3 * 256).reshape(3, 256)
    q = fx.oracle(oracle)
    ref = x.astype(np.float64) @ fx.dense().astype(np.float64).T     # unpacking via numpy bit arrays
    assert np.allclose(q.matmul_f64(x), ref, rtol=1e-6, atol=1e-6)
    for r in (0, 7, 23):
        assert np.array_equal(q.dequant_row(r), fx.dense()[r])


def test_round_f16_matches_numpy():
    """orc_round_f16_d against numpy's correctly rounded double -> half conversion: normals, ties,
    subnormals, overflow."""
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.normal(0, 1, 4000), rng.normal(0, 1e-5, 2000), rng.normal(0, 1e4, 1000),
                        (np.arange(-2048, 2048) + 0.5) * 2.0 ** -3,        # exact ties at ulp 2^-2 .. 2^-3
                        np.array([0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e6, 2.0 ** -25, 3 * 2.0 ** -25])])
    got = np.array([oracle.lib.orc_round_f16_d(float(a)) for a in v])
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).astype(np.float64)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_qlinear_f16_precision(gs):
    """The 4-bit GEMM precision against a numpy restatement (numpy's own f16 rounding) and the
    rounding bound to the exact product: each operand is within 2^-11 relative of its exact value
    (x scaled so that f16 keeps 11 bits), so |y - exact| <= 2^-10 * sum|w x| (+ subnormal slack)."""
    K, O, T = 512, 40, 5
    fx = QuantFixture(O, K, 4, gs, seed=gs, fast=True)
    x = np.random.default_rng(gs).normal(0, 3, (T, K)).astype(np.float32)
    x[1] *= 1e-3
    x[2, :] = 0.0
    x[3] *= 300.0
    q = fx.oracle(oracle)
    got = q.matmul_f16(x)
    g = np.repeat(np.arange(K // gs), gs)
    s16 = fx.scales.astype(np.float16).astype(np.float64)[:, g]
    b16 = fx.biases.astype(np.float16).astype(np.float64)[:, g]
    w16 = (s16 * fx.codes + b16).astype(np.float16).astype(np.float64)
    mx = np.abs(x).max(axis=1)
    e = np.where(mx > 0, 14 - np.frexp(mx)[1], 0)
    xh = (x.astype(np.float64) * 2.0 ** e[:, None]).astype(np.float16).astype(np.float64)
    ref = (xh @ w16.T) * 2.0 ** -e[:, None]
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-9)
    assert np.all(np.abs(xh * 2.0 ** -e[:, None]).max(axis=1) <= mx * (1 + 2.0 ** -11))
    exact = x.astype(np.float64) @ fx.dense().astype(np.float64).T
    bound = 2.0 ** -10 * (np.abs(x).astype(np.float64) @ np.abs(fx.dense()).astype(np.float64).T) + 1e-6
    assert np.all(np.abs(got - exact) <= bound)
    assert np.array_equal(got[2], np.zeros(O, np.float32))
    assert np.array_equal(q.matmul_prefill(x), got)
    fx3 = QuantFixture(8, 128, 3, 32, seed=1, fast=True)   # other widths: the fp32-level product
    assert np.array_equal(fx3.oracle(oracle).matmul_prefill(x[:, :128]), fx3.oracle(oracle).matmul_f64(x[:, :128]))


def test_qlinear_special_cases():
    """All codes 0: y = sum_g b_g * sum(x in g); scales 0 and biases 0: y = 0; bias added per row."""
    K, O, gs = 128, 4, 64
    packed = np.zeros((O, K // 2), np.uint8)
    s = np.full((O, K // gs), 0.5, np.float32)
    b = np.arange(O * (K // gs), dtype=np.float32).reshape(O, K // gs)
    x = np.linspace(-1, 1, K, dtype=np.float32)
    q = oracle.QMatrix(packed, s, b, K, 4, gs, bias=np.array([1, 2, 3, 4], np.float32))
    exp = np.array([b[o, 0] * x[:64].sum(dtype=np.float64) + b[o, 1] * x[64:].sum(dtype=np.float64) + o + 1 for o in range(O)])
    assert np.allclose(q.matmul_f64(x)[0], exp, atol=1e-5)


# ---------------------------------------------------------------------------------------- norms, rope
def test_rms_norm_invariants():
    x = np.random.default_rng(1).normal(0, 3, (5, 1024)).astype(np.float32)
    y = oracle.rms_norm(x, np.ones(1024, np.float32), 0.0)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-6)
    w = np.linspace(0.5, 2, 1024, dtype=np.float32)
    assert np.allclose(oracle.rms_norm(x, w, 1e-6), x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w,
                       rtol=1e-5)


def test_inv_freq_and_rope_as_complex_rotation():
    D = 128
    f = oracle.inv_freq(1e6, D)
    assert f[0] == 1.0 and np.isclose(f[-1], 1e6 ** (-(D - 2) / D), rtol=1e-6)
    v = np.random.default_rng(2).normal(0, 1, D).astype(np.float32)
    assert np.array_equal(oracle.rope(v, 0, f), v)
    for pos in (1, 17, 4095, 32767):
        got = oracle.rope(v, pos, f)
        # half-split RoPE: (v_i, v_{i+D/2}) is the complex number v_i + i v_{i+D/2} rotated by pos * f_i
        z = (v[:D // 2].astype(np.complex128) + 1j * v[D // 2:]) * np.exp(1j * (np.float32(pos) * f).astype(np.float64))
        assert np.allclose(got[:D // 2], z.real, atol=5e-5) and np.allclose(got[D // 2:], z.imag, atol=5e-5)
        assert np.isclose(np.linalg.norm(got), np.linalg.norm(v), rtol=1e-5)
    # traditional (interleaved) pairs (v_{2i}, v_{2i+1})
    got = oracle.rope(v, 9, f, traditional=True)
    z = (v[0::2].astype(np.complex128) + 1j * v[1::2]) * np.exp(1j * (np.float32(9) * f).astype(np.float64))
    assert np.allclose(got[0::2], z.real, atol=5e-5) and np.allclose(got[1::2], z.imag, atol=5e-5)


def test_silu():
    from scipy.special import expit
    for g, u in ((0.0, 3.0), (1.5, -2.0), (-20.0, 1.0), (7.25, 0.5)):
        assert np.isclose(oracle.lib.orc_silu_mul(g, u), g * expit(g) * u, rtol=1e-6, atol=1e-12)


# ---------------------------------------------------------------------------------------- attention
def numpy_attention(q, kc, vc, nH, nKV, positions, scale):
    out = np.zeros_like(q, dtype=np.float64)
    G = nH // nKV
    for h in range(nH):
        k = kc[h // G, positions].astype(np.float64); v = vc[h // G, positions].astype(np.float64)
        s = (q[h].astype(np.float32) * np.float32(scale)).astype(np.float64) @ k.T
        p = np.exp(s - s.max()); p /= p.sum()
        out[h] = p @ v
    return out


def test_attention_against_softmax():
    nH, nKV, D, S = 8, 2, 128, 64
    rng = np.random.default_rng(3)
    kc, vc = rng.uniform(-1, 1, (nKV, S, D)).astype(np.float32), rng.uniform(-1, 1, (nKV, S, D)).astype(np.float32)
    q = rng.uniform(-1, 1, (nH, D)).astype(np.float32)
    got = oracle.attention(q, kc, vc, nH, nKV, 40, 0.3)
    assert np.allclose(got, numpy_attention(q, kc, vc, nH, nKV, np.arange(41), 0.3), atol=1e-6)
    # invariants: a constant V row gives that constant; one key gives its value
    vc2 = np.broadcast_to(np.arange(D, dtype=np.float32), (nKV, S, D)).copy()
    assert np.allclose(oracle.attention(q, kc, vc2, nH, nKV, 40, 0.3), np.arange(D)[None], atol=1e-4)
    assert np.allclose(oracle.attention(q, kc, vc, nH, nKV, 0, 0.3), vc[np.arange(nH) // 4, 0], atol=1e-6)
    lst = np.array([0, 5, 6, 40, 99, -4], np.int32)      # out-of-range entries clamp to [0, L-1]
    got = oracle.attention_list(q, kc, vc, nH, nKV, 40, 0.3, lst, lst.size, 0)
    assert np.allclose(got, numpy_attention(q, kc, vc, nH, nKV, np.array([0, 5, 6, 40, 40, 0]), 0.3), atol=1e-6)


# ---------------------------------------------------------------------------------------- sparse
def test_sparse_clamp_known_answers():
    """configIsClampedToWholeBlocks (SparseAttentionTests.swift:52-56) and the default minimum context."""
    assert oracle.sparse_clamp(2050, 0, -3, -1) == (2048, 4, 0, 1)
    assert oracle.sparse_clamp(1, 512, 4)[0] == 4
    assert oracle.sparse_clamp(2048, 512, 4) == (2048, 512, 4, 5128)


@pytest.mark.parametrize("cfg", [(2048, 512, 4, None), (64, 16, 4, 1), (8, 5, 1, 1), (1 << 20, 4, 0, 1)])
def test_sparse_plan_partitions_the_context(cfg):
    """planPartitionsTheContext (SparseAttentionTests.swift:14-37)."""
    top_k, window, sink, mc = oracle.sparse_clamp(*cfg)
    for L in (1, 2, 7, 64, 65, 300, 5127, 5128, 5129, 8191, 32768):
        p = oracle.sparse_plan(top_k, window, sink, mc, L - 1)
        sink_end = (sink + 3) // 4 * 4
        if p is None:
            assert L < mc or L - window <= sink_end or (L - window) // 4 * 4 <= sink_end
            continue
        assert L >= mc and p.L == L and p.pool == 4
        assert p.sink_end >= sink and p.sink_end % 4 == 0 and p.b0 * 4 == p.sink_end
        assert p.win_start <= L - window and p.win_start % 4 == 0 and (p.b0 + p.nb) * 4 == p.win_start and p.nb > 0
        assert p.p == min(top_k // 4, p.nb) and p.p >= 1
        assert p.count == p.sink_end + p.p * 4 + (L - p.win_start) and p.count <= L
    assert oracle.sparse_plan(*oracle.sparse_clamp(2048, 512, 4, 1), 100_000 - 1) is not None
    assert oracle.sparse_plan(*oracle.sparse_clamp(2048, 512, 4), 100) is None


def test_sparse_index_score_select():
    nKV, D, S = 2, 128, 64
    k = bf16_to_f32(bf16_round(np.random.default_rng(4).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    idx = oracle.sparse_index(k, nKV, D, S, 3, 7)
    for b in range(3, 10):
        assert np.array_equal(idx[b], bf16_to_f32(bf16_round(k[:, 4 * b:4 * b + 4].astype(np.float32).sum(1) / 4)))
    assert np.all(idx[:3] == 0) and np.all(idx[10:] == 0)
    nH = 8
    q = np.random.default_rng(5).uniform(-1, 1, (nH, D)).astype(np.float32)
    qs = q.reshape(nKV, nH // nKV, D).sum(1)
    per = oracle.sparse_score(q, idx, nH, nKV, D, 3, 7, nKV)
    assert np.allclose(per, np.einsum("hd,bhd->hb", qs, idx[3:10]), rtol=1e-5, atol=1e-5)
    shared = oracle.sparse_score(q, idx, nH, nKV, D, 3, 7, 1)
    assert np.allclose(shared[0], per.sum(0), rtol=1e-5, atol=1e-5)
    # select: the reference test's restatement (sort by key desc then index, keep p, position order)
    for N, p, values, seed in ((1000, 100, None, 1), (5000, 512, [-1, 0, 0.5, 2], 2), (3, 2, [1], 3), (4096, 3, [-3, -2.5], 4)):
        rng = XorShift(seed)
        scores = np.array([rng.float(-10, 10) if values is None else values[rng.next() % len(values)] for _ in range(N)], np.float32)
        plan = oracle.SparsePlan(4, 1, N, p, 4, (1 + N) * 4, (1 + N) * 4 + 37, 4 + 4 * p + 37)
        keys = [oracle.sparse_key(float(s)) for s in scores]
        kept = sorted(sorted(range(N), key=lambda i: (-keys[i], i))[:p])
        exp = list(range(4)) + [(1 + n) * 4 + i for n in kept for i in range(4)] + list(range((1 + N) * 4, (1 + N) * 4 + 37))
        assert oracle.sparse_select(scores, plan).tolist() == exp
    assert oracle.sparse_key(-1.0) < oracle.sparse_key(-0.5) < oracle.sparse_key(0.0) < oracle.sparse_key(2.0)


# ---------------------------------------------------------------------------------------- sampling
def test_argmax_ties_and_non_finite():
    l = np.zeros(1000, np.float32); l[300] = 30; l[9] = 30
    assert oracle.argmax(l) == 9
    l[5] = np.nan
    assert oracle.argmax(l) == 9
    assert oracle.argmax(np.full(10, -np.inf, np.float32)) == -1


def test_sample_distribution_semantics():
    """Engine.swift:112-160 restated independently with numpy: penalty once per distinct recent
    token (positive / p, negative * p), temperature, top-k, min-p, top-p."""
    rng = np.random.default_rng(6)
    V = 3000
    l = rng.normal(0, 2, V).astype(np.float32)
    recent = [5, 9, 9, 5, 77, 2999]
    for T, k, p, mp, pen in ((0.9, 40, 0.95, 0.0, 1.1), (1.0, 0, 1.0, 0.0, 1.0), (0.7, 200, 0.8, 0.05, 1.3), (1.2, 5, 1.0, 0.0, 1.0)):
        ids, probs = oracle.sample_distribution(l, recent, T, k, p, mp, pen)
        x = l.astype(np.float32).copy()
        for t in set(recent):
            x[t] = x[t] / np.float32(pen) if x[t] > 0 else x[t] * np.float32(pen)
        kk = min(k, V) if k > 0 else min(512, V)
        order = np.argsort(-x, kind="stable")[:kk]
        pr = np.exp((x[order].astype(np.float64) - x[order[0]]) / T)
        cut = kk
        if mp > 0:
            below = np.nonzero(pr < mp * pr[0])[0]
            cut = int(below[0]) if below.size else cut
        if p < 1:
            c = np.cumsum(pr[:cut] / pr.sum())
            hit = np.nonzero(c >= p)[0]
            cut = int(hit[0]) + 1 if hit.size else cut
        cut = max(1, cut)
        assert ids.tolist() == order[:cut].tolist()
        assert np.allclose(probs, pr[:cut] / pr[:cut].sum(), rtol=1e-4)
    ids, probs = oracle.sample_distribution(l, recent, 0.0, 40, 1.0, 0.0, 1.3)
    assert ids.size == 1 and probs[0] == 1.0
    bad = l.copy(); bad[3] = np.inf
    assert oracle.sample_distribution(bad, [], 0.9, 40, 1, 0, 1) is None
