"""Kernel parity on the MI355X through libmlxr's C ABI, against the CPU oracle.

Mirrors the reference's kernel tests (Tests/MLXEngineTests/KernelTests.swift,
SparseAttentionTests.swift): same shapes, same generators, the same closeness metric
(|a-b| / max(1, |b|)), with the north-star tolerance 1e-3 for the fp32 matvec paths.
"""
import ctypes

import numpy as np
import pytest

import oracle
from qfix import QuantFixture, SynthMatrix, XorShift, bf16_round, bf16_to_f32, max_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3          # matvec / GEMM vs the oracle in the same declared precision (north star)


def qmv(mlxr, fixtures, x, norm_w=None, eps=1e-6, epi=0, y0=None):
    parts = (mlxr.QMat * len(fixtures))(*[f.device(mlxr) for f in fixtures])
    f0 = fixtures[0]
    O = sum(f.O for f in fixtures) if epi != 2 else f0.O
    dx = mlxr.DeviceArray.from_numpy(np.asarray(x, np.float32))
    dy = mlxr.DeviceArray.from_numpy(np.zeros(O, np.float32) if y0 is None else np.asarray(y0, np.float32))
    dn = mlxr.DeviceArray.from_numpy(np.asarray(norm_w, np.float32)) if norm_w is not None else None
    mlxr.check(mlxr.lib.mlxr_k_qmv(parts, len(fixtures), f0.K, f0.bits, f0.gs, 0 if f0.st == "bf16" else 1, dx.ptr,
                                   dn.ptr if dn else None, eps, dy.ptr, epi))
    mlxr.synchronize()
    return dy.numpy()


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_qmv_all_bits_groups_dtypes(gpu, bits):
    """quantizedMatchesReference at T = 1 (KernelTests.swift:128-146): K 512, O 40."""
    K, O = 512, 40
    for gs in (32, 64, 128):
        for st in ("f16", "bf16"):
            fx = QuantFixture(O, K, bits, gs, st=st)
            rng = XorShift(1 * 31 + bits)
            x = rng.floats(K)
            got = qmv(gpu, [fx], x)
            ref = fx.oracle(oracle).matmul_f64(x)[0]
            assert max_rel_err(got, ref) < TOL, (bits, gs, st)
            # the oracle itself agrees with the float64 numpy product of the dequantized matrix
            assert max_rel_err(ref, fx.reference(x)[0]) < 1e-6


@pytest.mark.parametrize("K", [1152, 1536, 2304, 2560, 896, 1664, 6912])
def test_qmv_partial_passes(gpu, K):
    """fourBitDecodeWithPartialPass (KernelTests.swift:188-199): K not a multiple of 1024."""
    O = 24
    for gs in (32, 64, 128):
        if K % gs:
            continue
        fx = QuantFixture(O, K, 4, gs, seed=K, fast=True)
        x = XorShift(K).floats(K)
        assert max_rel_err(qmv(gpu, [fx], x), fx.oracle(oracle).matmul_f64(x)[0]) < TOL


def test_fused_qkv_with_bias_matches_separate(gpu):
    """fusedDecodeWithBiasMatchesSeparate (KernelTests.swift:214-227)."""
    K = 256
    parts = [QuantFixture(o, K, 4, 64, with_bias=True, seed=s) for o, s in ((64, 1), (16, 2), (16, 3))]
    x = XorShift(99).floats(K)
    got = qmv(gpu, parts, x)
    ref = np.concatenate([p.oracle(oracle).matmul_f64(x)[0] for p in parts])
    assert max_rel_err(got, ref) < TOL


def test_qmv_normalised_input_and_epilogues(gpu):
    """x = RMSNorm(h) * w inside the matvec; accumulate (residual) and SiLU-gated epilogues."""
    K, O = 1024, 96
    rng = np.random.default_rng(3)
    h = rng.normal(0, 1, K).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    fa, fb = QuantFixture(O, K, 4, 64, seed=11, fast=True), QuantFixture(O, K, 4, 64, seed=12, fast=True)
    xn = oracle.rms_norm(h[None], w, 1e-6)[0]
    ref_a = fa.oracle(oracle).matmul_f64(xn)[0]
    assert max_rel_err(qmv(gpu, [fa], h, norm_w=w), ref_a) < TOL
    y0 = rng.normal(0, 1, O).astype(np.float32)
    assert max_rel_err(qmv(gpu, [fa], xn, epi=1, y0=y0), y0 + ref_a) < TOL
    ref_b = fb.oracle(oracle).matmul_f64(xn)[0]
    gated = np.array([oracle.lib.orc_silu_mul(float(g), float(u)) for g, u in zip(ref_a, ref_b)], np.float32)
    assert max_rel_err(qmv(gpu, [fa, fb], h, norm_w=w, epi=2), gated) < TOL


@pytest.mark.parametrize("bits", [3, 4, 6, 8])
def test_qmm_small_batch(gpu, bits):
    """T = 2..8 (qmm / qmvx4, KernelTests.swift:232-252) with padded strides (NaN padding never read)."""
    K, O = 512, 44
    fx = QuantFixture(O, K, bits, 64 if bits != 3 else 32, seed=K + O)
    qm = (gpu.QMat * 1)(fx.device(gpu))
    for T in (2, 3, 4, 5, 8):
        xs, ys = K + 4, O + 3
        x = np.full((T, xs), np.nan, np.float32)
        x[:, :K] = np.random.default_rng(T).uniform(-1, 1, (T, K))
        dx = gpu.DeviceArray.from_numpy(x)
        dy = gpu.DeviceArray.from_numpy(np.zeros((T, ys), np.float32))
        gpu.check(gpu.lib.mlxr_k_qmm(qm, 1, K, bits, fx.gs, 0, T, dx.ptr, xs, dy.ptr, ys))
        gpu.synchronize()
        got = dy.numpy()[:, :O]
        assert max_rel_err(got, fx.oracle(oracle).matmul_f64(x[:, :K])) < TOL, T


@pytest.mark.parametrize("bits,gs,st", [(4, 32, "bf16"), (4, 64, "f16"), (4, 128, "bf16"), (8, 32, "f16"), (8, 64, "bf16"),
                                         (8, 128, "bf16"), (2, 64, "bf16"), (3, 32, "bf16"), (3, 128, "f16"), (6, 64, "f16"),
                                         (6, 128, "bf16")])
def test_qmm_small_batch_wide_loads(gpu, bits, gs, st):
    """The small-batch kernel with wide code loads (32 codes per lane at 2 / 3 / 4 / 6 bits, 16 at 8;
    several groups per load at gs 32 / 64: one MFMA set per group, the other groups' lanes zeroed;
    3- and 6-bit codes straddling dwords): K of several batches per wave (the
    eight-wave launch at 4096 / gs 32), two fused parts with ragged row counts, f16 and bf16
    scales, T = 1..8 with fp32 inputs (x lo parts in use) and bf16-valued inputs (no lo parts);
    1e-3 against the fp64 product. 8-bit gs 128 runs the per-group kernel."""
    K = 4096 if gs == 32 else 2048
    fa = QuantFixture(40, K, bits, gs, st=st, seed=K + bits, fast=True)
    fb = QuantFixture(27, K, bits, gs, st=st, seed=K + bits + 1, fast=True)
    qm = (gpu.QMat * 2)(fa.device(gpu), fb.device(gpu))
    O = fa.O + fb.O
    for T in (1, 3, 4, 8):
        rng = np.random.default_rng(T * 31 + bits)
        for bf16_x in (False, True):
            x = rng.normal(0, 1, (T, K)).astype(np.float32)
            if bf16_x:
                x = bf16_to_f32(bf16_round(x)).reshape(T, K)
            dx = gpu.DeviceArray.from_numpy(x)
            dy = gpu.DeviceArray.from_numpy(np.zeros((T, O), np.float32))
            gpu.check(gpu.lib.mlxr_k_qmm(qm, 2, K, bits, gs, 0 if st == "bf16" else 1, T, dx.ptr, K, dy.ptr, O))
            gpu.synchronize()
            ref = np.concatenate([fa.oracle(oracle).matmul_f64(x), fb.oracle(oracle).matmul_f64(x)], axis=1)
            assert max_rel_err(dy.numpy(), ref) < TOL, (T, bf16_x)


def qgemm(mlxr, fx, x):
    T = x.shape[0]
    qm = (mlxr.QMat * 1)(fx.device(mlxr))
    dx = mlxr.DeviceArray.from_numpy(x)
    dy = mlxr.DeviceArray.from_numpy(np.zeros((T, fx.O), np.float32))
    mlxr.check(mlxr.lib.mlxr_k_qgemm(qm, fx.K, fx.bits, fx.gs, 0 if fx.st == "bf16" else 1, T, dx.ptr, fx.K, dy.ptr, fx.O))
    mlxr.synchronize()
    return dy.numpy()


@pytest.mark.parametrize("bits,gs", [(2, 32), (3, 32), (4, 32), (4, 64), (4, 128), (5, 64), (6, 128), (8, 32)])
def test_qgemm_prefill_tiles(gpu, bits, gs):
    """prefillTilesMatchReference shapes (KernelTests.swift:150-164) for the MLX-layout prefill GEMM
    against the oracle's fp64 product at the 1e-3 matvec / GEMM gate: exact codes, x as f16 hi + lo,
    scale and bias per group in fp32. Ragged T and O, K with an odd number of groups (1088 at gs
    64, 1152 at gs 128), and bf16-valued inputs (whose lo parts are zero: the tile skips them)."""
    shapes = ((64, 41, 1088), (128, 41, 576), (517, 41, 576), (96, 2050, 576), (128, 2050, 576), (517, 520, 576))
    if gs == 128:
        shapes = ((64, 41, 1152), (517, 41, 640), (128, 2050, 640), (300, 520, 1152))
    for T, O, K in shapes:
        fx = QuantFixture(O, K, bits, gs, seed=T + O, fast=True)
        x = np.random.default_rng(T * 7 + bits).uniform(-1, 1, (T, K)).astype(np.float32)
        assert max_rel_err(qgemm(gpu, fx, x), fx.oracle(oracle).matmul_f64(x)) < TOL, (T, O, K)
        xb = bf16_to_f32(bf16_round(x)).reshape(T, K)
        assert max_rel_err(qgemm(gpu, fx, xb), fx.oracle(oracle).matmul_f64(xb)) < TOL, ("bf16 x", T, O, K)
    # a bf16-valued row next to fp32 rows in one token tile: each row keeps its own precision; with
    # bf16 and f16 scales and biases (f16 biases enter the bias products as two bf16 parts)
    x = np.random.default_rng(bits).normal(0, 1, (40, 1024)).astype(np.float32)
    x[::3] = bf16_to_f32(bf16_round(x[::3])).reshape(-1, 1024)
    for st in ("bf16", "f16"):
        fx = QuantFixture(300, 1024, bits, gs, st=st, seed=1, fast=True)
        assert max_rel_err(qgemm(gpu, fx, x), fx.oracle(oracle).matmul_f64(x)) < TOL, st


def test_qgemm_row_scaling(gpu):
    """The prefill GEMM on rows of very different magnitude (the per-row power-of-two scaling keeps
    each row's precision), a zero row, bias, bf16 and f16 scales: every row within 1e-5 of its own
    scale against the fp64 product."""
    O, K, T = 300, 1024, 40
    for st in ("bf16", "f16"):
        fx = QuantFixture(O, K, 4, 64, st=st, seed=5, with_bias=True, fast=True)
        x = np.random.default_rng(9).normal(0, 1, (T, K)).astype(np.float32)
        x *= (10.0 ** np.linspace(-6, 6, T)).astype(np.float32)[:, None]
        x[7] = 0.0
        got = qgemm(gpu, fx, x)
        ref = fx.oracle(oracle).matmul_f64(x)
        scale = np.maximum(np.abs(ref).max(axis=1, keepdims=True), 1e-30)
        assert np.all(np.abs(got - ref) / scale < 1e-5), st
        assert np.all(np.isfinite(got))


def qgemm_tiles(mlxr, fxs, x, gated=False):
    T = x.shape[0]
    qm = (mlxr.QMat * len(fxs))(*[f.device(mlxr) for f in fxs])
    cols = fxs[0].O if gated else sum(f.O for f in fxs)
    dx = mlxr.DeviceArray.from_numpy(x)
    dy = mlxr.DeviceArray.from_numpy(np.full((T, cols), np.nan, np.float32))
    mlxr.check(mlxr.lib.mlxr_k_qgemm_tiles(qm, len(fxs), fxs[0].K, fxs[0].gs, int(gated), T, dx.ptr, x.shape[1], dy.ptr, cols))
    mlxr.synchronize()
    return dy.numpy()


@pytest.mark.parametrize("gs", [32, 64])
def test_qgemm_tiles(gpu, gs):
    """The prefill GEMM over repacked tiles (model prefill's path for 4-bit bf16-scale models):
    fused parts [A|B|C] with per-part bias (or none) and ragged row counts, against the oracle's 4-bit GEMM
    precision per part; T not a multiple of the 128-token tile."""
    K = 512
    for T in (9, 130, 300):
        fxs = [QuantFixture(O, K, 4, gs, seed=O + T, with_bias=T != 130, fast=True) for O in (264, 40, 88)]
        x = np.random.default_rng(T).normal(0, 1, (T, K)).astype(np.float32)
        got = qgemm_tiles(gpu, fxs, x)
        ref = np.concatenate([f.oracle(oracle).matmul_f16(x) for f in fxs], axis=1)
        assert max_rel_err(got, ref) < TOL, T
        assert np.max(np.abs(got - ref)) < 1e-4, T


@pytest.mark.parametrize("gs", [32, 64])
def test_qgemm_tiles_gated(gpu, gs):
    """Gate|up on the repacked tiles with SiLU(gate) * up in the epilogue (silu_mul,
    Kernels.swift:2004-2013) against the oracle's GEMM precision and orc_silu_mul."""
    K, I = 768, 200
    for T in (17, 257):
        g, u = (QuantFixture(I, K, 4, gs, seed=s, fast=True) for s in (1 + T, 2 + T))
        x = np.random.default_rng(T).normal(0, 1, (T, K)).astype(np.float32)
        got = qgemm_tiles(gpu, [g, u], x, gated=True)
        gr, ur = g.oracle(oracle).matmul_f16(x), u.oracle(oracle).matmul_f16(x)
        ref = (gr / (1.0 + np.exp(-gr.astype(np.float64)))).astype(np.float32) * ur
        assert np.all(np.isfinite(got))
        assert max_rel_err(got, ref) < TOL, T


def qmv_tiles(mlxr, fxs, x, mode=0, norm_w=None, eps=1e-6, y0=None):
    qm = (mlxr.QMat * len(fxs))(*[f.device(mlxr) for f in fxs])
    O = fxs[0].O if mode == 2 else sum(f.O for f in fxs)
    dx = mlxr.DeviceArray.from_numpy(np.asarray(x, np.float32))
    dy = mlxr.DeviceArray.from_numpy(np.full(O, np.nan, np.float32) if y0 is None else np.asarray(y0, np.float32))
    dn = mlxr.DeviceArray.from_numpy(np.asarray(norm_w, np.float32)) if norm_w is not None else None
    mlxr.check(mlxr.lib.mlxr_k_qmv_tiles(qm, len(fxs), fxs[0].K, fxs[0].gs, mode, dx.ptr, dn.ptr if dn else None, eps,
                                         dy.ptr, 1))
    mlxr.synchronize()
    return dy.numpy()


@pytest.mark.parametrize("gs", [32, 64])
def test_qmv_tiles_epilogues(gpu, gs):
    """The batch-1 decode projection over the repacked tiles (the persistent step's matvec phases and
    the kernel-per-op step's launches; qmv with its fused RMSNorm input, accumulate and SiLU-gated
    epilogues, Kernels.swift:60-113, 204-318, 2004-2013) against the oracle's fp64 product at the
    1e-3 matvec gate: fused q|k|v parts with bias and ragged row counts, K from one scale group to
    the 32B MLP's 27648, and an input of large magnitude (the power-of-two scaling). x enters the
    matrix cores as an f16 hi + lo pair, so the reference's fp32 input is kept."""
    rng = np.random.default_rng(gs)
    for K, Os in ((128, (40,)), (1024, (264, 40, 88)), (5120, (72,)), (27648, (24,))):
        fxs = [QuantFixture(O, K, 4, gs, seed=O + K, with_bias=len(Os) > 1, fast=True) for O in Os]
        h = rng.normal(0, 1, K).astype(np.float32)
        w = rng.uniform(0.5, 1.5, K).astype(np.float32)
        xn = oracle.rms_norm(h[None], w, 1e-6)[0]
        ref = np.concatenate([f.oracle(oracle).matmul_f64(xn)[0] for f in fxs])
        assert max_rel_err(qmv_tiles(gpu, fxs, h, norm_w=w), ref) < TOL, K
        big = (h * 3e4).astype(np.float32)
        ref_big = np.concatenate([f.oracle(oracle).matmul_f64(big)[0] for f in fxs])
        assert max_rel_err(qmv_tiles(gpu, fxs, big) / 3e4, ref_big / 3e4) < TOL, K   # the gate at the input's scale
        y0 = rng.normal(0, 1, ref.size).astype(np.float32)
        assert max_rel_err(qmv_tiles(gpu, fxs, xn, mode=1, y0=y0), y0 + ref) < TOL, K
        tiny = (h * 1e-20).astype(np.float32)   # scaled up by 2^e before rounding: no f16 underflow
        ref_tiny = np.concatenate([f.oracle(oracle).matmul_f64(tiny)[0] for f in fxs])
        assert max_rel_err(qmv_tiles(gpu, fxs, tiny) * 1e20, ref_tiny * 1e20) < TOL, K
    K, I = 2048, 200
    g, u = (QuantFixture(I, K, 4, gs, seed=s, fast=True) for s in (5, 6))
    h = rng.normal(0, 1, K).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    xn = oracle.rms_norm(h[None], w, 1e-6)[0]
    gr, ur = g.oracle(oracle).matmul_f64(xn)[0], u.oracle(oracle).matmul_f64(xn)[0]
    gated = np.array([oracle.lib.orc_silu_mul(float(a), float(b)) for a, b in zip(gr, ur)], np.float32)
    assert max_rel_err(qmv_tiles(gpu, [g, u], h, mode=2, norm_w=w), gated) < TOL
    zero = qmv_tiles(gpu, [g, u], np.zeros(K, np.float32), mode=2)
    assert np.all(zero == 0.0)


def test_qmv_tiles_input_slices_share_scratch(gpu):
    """The input-sliced matvec (a projection whose tiles are too few for the CUs runs as several
    input slices per tile, the last slice of a tile adding the partials) over one scratch shared by
    launches of different shapes and slice counts: a small projection, a larger one whose partials
    cover the small one's scratch, then the small one again (its per-tile counters must still read
    zero), each against the oracle's fp64 product at the matvec gate, plain and accumulating."""
    rng = np.random.default_rng(3)
    cases = [(16384, 40), (12288, 1024), (16384, 40), (27648, 24), (16384, 40)]   # 2, 2, 2, 8, 2 slices
    fx = {}
    for K, O in cases:
        f = fx.setdefault((K, O), QuantFixture(O, K, 4, 64, seed=K + O, fast=True))
        x = rng.normal(0, 1, K).astype(np.float32)
        ref = f.oracle(oracle).matmul_f64(x)[0]
        assert max_rel_err(qmv_tiles(gpu, [f], x), ref) < TOL, (K, O)
        y0 = rng.normal(0, 1, O).astype(np.float32)
        assert max_rel_err(qmv_tiles(gpu, [f], x, mode=1, y0=y0), y0 + ref) < TOL, (K, O)


def qmm_tiles(mlxr, fxs, x, mode=0, norm_w=None, eps=1e-6, y0=None):
    T, K = x.shape
    qm = (mlxr.QMat * len(fxs))(*[f.device(mlxr) for f in fxs])
    cols = fxs[0].O if mode == 2 else sum(f.O for f in fxs)
    dx = mlxr.DeviceArray.from_numpy(np.ascontiguousarray(x))
    dy = mlxr.DeviceArray.from_numpy(np.full((T, cols), np.nan, np.float32) if y0 is None else np.asarray(y0, np.float32))
    dn = mlxr.DeviceArray.from_numpy(np.asarray(norm_w, np.float32)) if norm_w is not None else None
    mlxr.check(mlxr.lib.mlxr_k_qmm_tiles(qm, len(fxs), K, fxs[0].gs, mode, T, dx.ptr, K, dn.ptr if dn else None, eps,
                                         dy.ptr, cols))
    mlxr.synchronize()
    return dy.numpy()


def _gated_ref(g, u, x):
    gr, ur = g.oracle(oracle).matmul_f64(x), u.oracle(oracle).matmul_f64(x)
    return np.array([[oracle.lib.orc_silu_mul(float(a), float(b)) for a, b in zip(gr[t], ur[t])] for t in range(len(x))],
                    np.float32)


@pytest.mark.parametrize("gs", [32, 64])
def test_qmm_tiles_small_batch(gpu, gs):
    """The verify batch's projections over the repacked tiles (qmm / qmvx4, Kernels.swift:60-113,
    518-622): T = 1..8 tokens in the matrix cores' B columns, every token against the oracle's fp64
    product at the 1e-3 matvec gate: fused parts with bias and ragged rows, inputs from one scale
    group to 12288 values (the long ones in input slices summed across workgroups), rows of very
    different magnitude, a single part of many tiles per workgroup (the lm_head), and the gated
    form."""
    rng = np.random.default_rng(gs)
    for K, Os in ((128, (40,)), (1024, (264, 40, 88)), (4096, (72,)), (12288, (24,)), (27648, (40,))):
        fxs = [QuantFixture(O, K, 4, gs, seed=O + K, with_bias=len(Os) > 1, fast=True) for O in Os]
        for T in ((1, 3, 8) if K < 27648 else (8,)):   # the 32B down: seven input slices at T = 8
            mag = (10.0 ** np.linspace(-3, 3, T)).astype(np.float32)
            x = rng.normal(0, 1, (T, K)).astype(np.float32) * mag[:, None]
            ref = np.concatenate([f.oracle(oracle).matmul_f64(x) for f in fxs], axis=1)
            got = qmm_tiles(gpu, fxs, x)
            for t in range(T):
                assert max_rel_err(got[t] / mag[t], ref[t] / mag[t]) < TOL, (K, T, t)
    f = QuantFixture(16 * 40 * 256 + 40, 256, 4, gs, seed=7, fast=True)
    x = rng.normal(0, 1, (2, 256)).astype(np.float32)
    assert max_rel_err(qmm_tiles(gpu, [f], x), f.oracle(oracle).matmul_f64(x)) < TOL
    # gated: one slice, and two slices summed before the SiLU (x scaled so that gate and up stay
    # O(10): the product's rounding grows with |gate| * |up|, not with the result)
    for K, T in ((2048, 5), (8192, 8)):
        g, u = (QuantFixture(200, K, 4, gs, seed=s + K, fast=True) for s in (5, 6))
        x = rng.normal(0, 1, (T, K)).astype(np.float32) / np.float32(np.sqrt(K / 64))
        assert max_rel_err(qmm_tiles(gpu, [g, u], x, mode=2), _gated_ref(g, u, x)) < TOL, K


def test_qmm_tiles_split_launches_share_scratch(gpu):
    """Input-sliced small-batch launches of different tile counts (all above 64) through the one
    scratch they share, as a verify layer at Qwen2.5-32B width runs them (K = 5120 runs in two
    slices at T = 5): q|k|v-sized (448 tiles), o-sized (320 tiles), then both again, with a
    batch-1 sliced matvec of 128 tiles between them. Every launch's
    per-tile counters must still read zero after the others' partials were written, and every
    token row must match the fp64 product at the matvec gate."""
    rng = np.random.default_rng(11)
    K, T = 5120, 5
    fx = {O: QuantFixture(O, K, 4, 64, seed=O, with_bias=True, fast=True) for O in (7168, 5120)}
    down = QuantFixture(2048, 27648, 4, 64, seed=3, fast=True)   # a batch-1 sliced matvec (128 tiles) in between
    for O in (7168, 5120, 7168, 5120, 7168):
        xd = rng.normal(0, 1, 27648).astype(np.float32)
        assert max_rel_err(qmv_tiles(gpu, [down], xd), down.oracle(oracle).matmul_f64(xd)[0]) < TOL, O
        x = rng.normal(0, 1, (T, K)).astype(np.float32)
        ref = fx[O].oracle(oracle).matmul_f64(x)
        got = qmm_tiles(gpu, [fx[O]], x)
        assert np.all(np.isfinite(got)), O
        assert max_rel_err(got, ref) < TOL, O
        y0 = rng.normal(0, 1, ref.shape).astype(np.float32)
        assert max_rel_err(qmm_tiles(gpu, [fx[O]], x, mode=1, y0=y0), y0 + ref) < TOL, O


@pytest.mark.parametrize("K,T", [(4096, 5), (12288, 8)])
def test_qmm_tiles_norm_and_accumulate(gpu, K, T):
    """The verify batch's fused forms: x[t] := RMSNorm(x[t]) * w inside the launch (the statistics
    over the whole input also when it runs in slices), and the residual add y[t] += W x[t]."""
    rng = np.random.default_rng(K + T)
    fxs = [QuantFixture(O, K, 4, 64, seed=O, with_bias=True, fast=True) for O in (136, 56)]
    h = rng.normal(0, 3, (T, K)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, K).astype(np.float32)
    xn = oracle.rms_norm(h, w, 1e-6)
    ref = np.concatenate([f.oracle(oracle).matmul_f64(xn) for f in fxs], axis=1)
    assert max_rel_err(qmm_tiles(gpu, fxs, h, norm_w=w), ref) < TOL
    y0 = rng.normal(0, 1, ref.shape).astype(np.float32)
    assert max_rel_err(qmm_tiles(gpu, fxs, h, mode=1, y0=y0), y0 + np.concatenate(
        [f.oracle(oracle).matmul_f64(h) for f in fxs], axis=1)) < TOL
    g, u = (QuantFixture(96, K, 4, 64, seed=s, fast=True) for s in (8, 9))
    w = w / np.float32(np.sqrt(K / 64))   # gate and up O(10), as in the gated small-batch check
    assert max_rel_err(qmm_tiles(gpu, [g, u], h, mode=2, norm_w=w), _gated_ref(g, u, oracle.rms_norm(h, w, 1e-6))) < TOL


def _decode_input(kind, K, rng):
    """Inputs as the decode step feeds each projection: RMSNorm'd hidden state (q|k|v, gate|up,
    lm_head: passed raw with the norm weights, the norm runs in the kernel), the attention output
    (o_proj: a softmax-weighted mean of value rows) and SiLU(g) * u (down)."""
    if kind == "norm":
        return rng.normal(0, 1, K).astype(np.float32) * np.float32(3.0)
    if kind == "attn":
        return (rng.normal(0, 1, K) * 0.3).astype(np.float32)
    g, u = rng.normal(0, 1.3, K), rng.normal(0, 1.3, K)
    return (g / (1 + np.exp(-g)) * u).astype(np.float32)


# (name, K, parts' rows, gated, input kind): every batch-1 projection of configs[1] (Qwen3-8B) and
# configs[4] (Qwen2.5-32B), weights N(0, 0.02) quantized 4-bit g64 as the synthetic models are
CONFIG_PROJECTIONS = [
    ("qwen3-8b qkv", 4096, (4096, 1024, 1024), False, "norm"),
    ("qwen3-8b o", 4096, (4096,), False, "attn"),
    ("qwen3-8b gate|up", 4096, (12288, 12288), True, "norm"),
    ("qwen3-8b down", 12288, (4096,), False, "mlp"),
    ("qwen3-8b lm_head", 4096, (151936,), False, "norm"),
    ("qwen2.5-32b qkv", 5120, (5120, 1024, 1024), False, "norm"),
    ("qwen2.5-32b o", 5120, (5120,), False, "attn"),
    ("qwen2.5-32b gate|up", 5120, (27648, 27648), True, "norm"),
    ("qwen2.5-32b down", 27648, (5120,), False, "mlp"),
]


@pytest.mark.parametrize("name,K,Os,gated,kind", CONFIG_PROJECTIONS, ids=[c[0] for c in CONFIG_PROJECTIONS])
def test_decode_matvec_config_shapes(gpu, name, K, Os, gated, kind):
    """The decode matvec at the benchmark models' real projection shapes against the oracle's fp64
    product, 1e-3 relative (|a-b| / max(1, |b|)): the reference's qmv keeps x in fp32
    (Kernels.swift:204-318), and so does the f16 hi + lo operand here."""
    print(f"[case] {name} K={K} rows={Os}", flush=True)
    fxs = [SynthMatrix(gpu, O, K, 4, 64, seed=11, tensor_id=i) for i, O in enumerate(Os)]
    rng = np.random.default_rng(K + sum(Os))
    x = _decode_input(kind, K, rng)
    nw = rng.uniform(0.8, 1.2, K).astype(np.float32) if kind == "norm" else None
    xr = oracle.rms_norm(x[None], nw, 1e-6)[0] if nw is not None else x
    refs = [f.oracle(oracle).matmul_f64(xr)[0] for f in fxs]
    if gated:
        g, u = refs
        ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32)
        got = qmv_tiles(gpu, fxs, x, mode=2, norm_w=nw)
    else:
        ref = np.concatenate(refs)
        got = qmv_tiles(gpu, fxs, x, norm_w=nw)
    err = max_rel_err(got, ref)
    print(f"[case] {name}: max rel err {err:.3g}, max |y| {np.max(np.abs(ref)):.3g}", flush=True)
    assert err < TOL, (name, err)
    if name.endswith("lm_head"):   # the greedy token: bit-exact argmax where the oracle's top-2 margin decides it
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > 2 * TOL * max(1.0, abs(top2[1])):
            assert int(np.argmax(got)) == int(np.argmax(ref))


def test_qgemm_batch_invariant(gpu):
    """prefillTilesAgreeBitwise (KernelTests.swift:168-184): a token's output does not depend on T."""
    O, K = 2050, 1024
    fx = QuantFixture(O, K, 4, 64, seed=3, fast=True)
    x = np.random.default_rng(11).uniform(-1, 1, (256, K)).astype(np.float32)
    full = qgemm(gpu, fx, x)
    for T in (9, 16, 33, 96):
        assert np.array_equal(qgemm(gpu, fx, x[:T]).view(np.uint32), full[:T].view(np.uint32)), T


@pytest.mark.parametrize("bits,gs", [(3, 32), (8, 64)])
def test_qgemm_split_k_batch_invariant(gpu, bits, gs):
    """The MLX-layout GEMM over a long input (128 K steps: four fixed K slices added in order):
    a launch of few tiles runs the slices on workgroups of their own (9 tokens x 40 row tiles), a
    launch of many does not (512 tokens x 40), and a token's result is bit-identical either way
    (prefillTilesAgreeBitwise, KernelTests.swift:168-184), and matches the fp64 product at the
    1e-3 gate; repeated, so the split's tile counters are back at zero."""
    O, K = 5120, 8192
    fx = QuantFixture(O, K, bits, gs, seed=bits, fast=True)
    x = np.random.default_rng(bits).uniform(-1, 1, (512, K)).astype(np.float32)
    full = qgemm(gpu, fx, x)
    for _ in range(2):
        few = qgemm(gpu, fx, x[:9])
        assert np.array_equal(few.view(np.uint32), full[:9].view(np.uint32))
    assert max_rel_err(few, fx.oracle(oracle).matmul_f64(x[:9])) < TOL


def test_qembed(gpu):
    """quantizedEmbeddingLookup (KernelTests.swift:287-296), tol 1e-5."""
    K, V = 128, 16
    fx = QuantFixture(V, K, 4, 64)
    ids = np.array([3, 0, 15, 7], np.int32)
    qm = (gpu.QMat * 1)(fx.device(gpu))
    did = gpu.DeviceArray.from_numpy(ids)
    out = gpu.DeviceArray.zeros((4, K), np.float32)
    gpu.check(gpu.lib.mlxr_k_qembed(qm, K, 4, 64, 0, did.ptr, 4, out.ptr))
    gpu.synchronize()
    q = fx.oracle(oracle)
    ref = np.stack([q.dequant_row(int(i)) for i in ids])
    assert np.max(np.abs(out.numpy() - ref)) <= 1e-5
    bad = gpu.DeviceArray.from_numpy(np.array([16], np.int32))
    with pytest.raises(gpu.EngineError):
        gpu.check(gpu.lib.mlxr_k_qembed(qm, K, 4, 64, 0, bad.ptr, 1, out.ptr))


def test_rms_norm_and_add(gpu):
    rng = np.random.default_rng(5)
    for dim, rows in ((1024, 3), (4096, 2), (5120, 1)):
        x = rng.normal(0, 2, (rows, dim)).astype(np.float32)
        r = rng.normal(0, 1, (rows, dim)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
        dx, dr, dy, dw = (gpu.DeviceArray.from_numpy(a) for a in (x, r, np.zeros_like(x), w))
        gpu.check(gpu.lib.mlxr_k_rms_norm(dx.ptr, None, dy.ptr, dw.ptr, dim, rows, 1e-6))
        gpu.synchronize()
        assert max_rel_err(dy.numpy(), oracle.rms_norm(x, w, 1e-6)) < 1e-5
        gpu.check(gpu.lib.mlxr_k_rms_norm(dx.ptr, dr.ptr, dy.ptr, dw.ptr, dim, rows, 1e-6))
        gpu.synchronize()
        assert max_rel_err(dx.numpy(), x + r) < 1e-6
        assert max_rel_err(dy.numpy(), oracle.rms_norm(x + r, w, 1e-6)) < 1e-5


def to_paged(c, page=64):
    """[nKV][max_seq][D] -> the library's cache layout [max_seq/64][nKV][64][D]."""
    nKV, S, D = c.shape
    return np.ascontiguousarray(c.reshape(nKV, S // page, page, D).transpose(1, 0, 2, 3))


def from_paged(c, nKV, D, page=64):
    pages = c.size // (nKV * page * D)
    return np.ascontiguousarray(c.reshape(pages, nKV, page, D).transpose(1, 0, 2, 3).reshape(nKV, pages * page, D))


@pytest.mark.parametrize("qk_norm,traditional,rot", [(True, False, 128), (False, False, 128), (True, True, 128),
                                                    (True, False, 64)])
def test_qkv_post(gpu, qk_norm, traditional, rot):
    """q/k norm + RoPE + K/V append against the oracle: full rotation (one wave per head) and
    partial rotation (rot_dim 64: the workgroup-per-head kernel)."""
    nH, nKV, D, S, T, off = 4, 2, 128, 128, 5, 37
    rng = np.random.default_rng(7)
    cols = (nH + 2 * nKV) * D
    qkv = rng.normal(0, 1, (T, cols)).astype(np.float32)
    invf = oracle.inv_freq(1e6, rot)
    qn = rng.uniform(0.5, 1.5, D).astype(np.float32) if qk_norm else None
    kn = rng.uniform(0.5, 1.5, D).astype(np.float32) if qk_norm else None
    dq = gpu.DeviceArray.from_numpy(qkv)
    dk = gpu.DeviceArray.zeros(S * nKV * D, np.uint16)
    dv = gpu.DeviceArray.zeros(S * nKV * D, np.uint16)
    di = gpu.DeviceArray.from_numpy(invf)
    dqn = gpu.DeviceArray.from_numpy(qn) if qk_norm else None
    dkn = gpu.DeviceArray.from_numpy(kn) if qk_norm else None
    gpu.check(gpu.lib.mlxr_k_qkv_post(dq.ptr, cols, di.ptr, dk.ptr, dv.ptr, S, dqn.ptr if dqn else None, dkn.ptr if dkn else None,
                                      D, nH, nKV, rot, int(traditional), off, T, 1e-6))
    gpu.synchronize()
    got_q = dq.numpy()
    kc = bf16_to_f32(from_paged(dk.numpy(), nKV, D))
    vc = bf16_to_f32(from_paged(dv.numpy(), nKV, D))
    for t in range(T):
        pos = off + t
        for h in range(nH + nKV):
            v = qkv[t, h * D:(h + 1) * D]
            if qk_norm:
                v = oracle.rms_norm(v[None], qn if h < nH else kn, 1e-6)[0]
            ref = oracle.rope(v, pos, invf, rot_dim=rot, traditional=traditional)
            if h < nH:
                assert np.max(np.abs(got_q[t, h * D:(h + 1) * D] - ref)) < 2e-5
            else:
                assert np.array_equal(kc[h - nH, pos], bf16_to_f32(bf16_round(ref))) or \
                    np.max(np.abs(kc[h - nH, pos] - ref)) <= np.max(np.abs(ref)) * 2 ** -8
        for h in range(nKV):
            assert np.array_equal(vc[h, pos], bf16_to_f32(bf16_round(qkv[t, (nH + nKV + h) * D:(nH + nKV + h + 1) * D])))


def run_attention(mlxr, q, kc, vc, nH, nKV, offset, T, scale, lists=None, count=0, list_stride=0, nsplit=32):
    D = q.shape[-1]
    S = kc.shape[1]
    dq = mlxr.DeviceArray.from_numpy(q.reshape(T, nH * D))
    dk = mlxr.DeviceArray.from_numpy(bf16_round(to_paged(kc)))
    dv = mlxr.DeviceArray.from_numpy(bf16_round(to_paged(vc)))
    out = mlxr.DeviceArray.zeros((T, nH * D), np.float32)
    dl = mlxr.DeviceArray.from_numpy(np.asarray(lists, np.int32)) if lists is not None else None
    mlxr.check(mlxr.lib.mlxr_k_attention(dq.ptr, nH * D, dk.ptr, dv.ptr, S, D, nH, nKV, offset, T, scale, out.ptr, nH * D,
                                         dl.ptr if dl else None, count, list_stride, nsplit))
    mlxr.synchronize()
    return out.numpy().reshape(T, nH, D)


@pytest.mark.parametrize("nH,nKV", [(4, 2), (10, 2), (32, 8), (40, 8)])
def test_attention_decode_and_split(gpu, nH, nKV):
    """kernelsMatchReference (KernelTests.swift:540-586): decode at position 100 of a 128-row cache;
    single-range and split results agree; over a bf16 cache (values rounded as stored)."""
    D, S = 128, 128
    rng = XorShift(D * 31)
    kc = bf16_to_f32(bf16_round(np.random.default_rng(nH).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    vc = bf16_to_f32(bf16_round(np.random.default_rng(nH + 1).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    q = np.random.default_rng(nH + 2).uniform(-1, 1, (nH, D)).astype(np.float32)
    scale = 3 / np.sqrt(D)
    ref = oracle.attention(q, kc, vc, nH, nKV, 100, scale)
    one = run_attention(gpu, q, kc, vc, nH, nKV, 100, 1, scale, nsplit=1)[0]
    split = run_attention(gpu, q, kc, vc, nH, nKV, 100, 1, scale, nsplit=32)[0]
    assert max_rel_err(one, ref) < 2e-5
    assert max_rel_err(split, ref) < 2e-5
    # several query tokens (positions 100..104) run as decode steps
    q5 = np.random.default_rng(9).uniform(-1, 1, (5, nH, D)).astype(np.float32)
    got5 = run_attention(gpu, q5, kc, vc, nH, nKV, 100, 5, scale)
    for t in range(5):
        assert max_rel_err(got5[t], oracle.attention(q5[t], kc, vc, nH, nKV, 100 + t, scale)) < 2e-5
    del rng


@pytest.mark.parametrize("nH,nKV,offset,T,nsplit", [(32, 8, 700, 8, 3), (40, 8, 300, 8, 1), (4, 2, 100, 5, 64),
                                                   (8, 1, 37, 2, 32), (64, 8, 511, 8, 5), (40, 8, 1000, 8, 256)])
def test_attention_verify_batch(gpu, nH, nKV, offset, T, nsplit):
    """The verify batch's attention (attention_split + attention_combine per query, Kernels.swift:
    1317-1374): the T queries of a KV head share one pass over each key range, query t masked past
    its own position offset + t. Every query against the reference attention at its position; keys
    past the batch's last position are NaN (never read); ranges past a query's position (nsplit 64
    over 105 keys), ranges raised to 128 keys at most (nsplit 1 over 308 keys), G T up to 64, and
    the 32B shape's many ranges (G = 5, T = 8, 256 ranges of 4 keys)."""
    D, S = 128, 1024
    kc = bf16_to_f32(bf16_round(np.random.default_rng(nH + T).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    vc = bf16_to_f32(bf16_round(np.random.default_rng(nH + T + 1).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    kc[:, offset + T:] = np.nan
    vc[:, offset + T:] = np.nan
    q = np.random.default_rng(nH + T + 2).uniform(-1, 1, (T, nH, D)).astype(np.float32)
    scale = 3 / np.sqrt(D)
    got = run_attention(gpu, q, kc, vc, nH, nKV, offset, T, scale, nsplit=nsplit)
    assert np.all(np.isfinite(got))
    kref, vref = np.nan_to_num(kc), np.nan_to_num(vc)
    for t in range(T):
        assert max_rel_err(got[t], oracle.attention(q[t], kref, vref, nH, nKV, offset + t, scale)) < 2e-5, t


def run_flash(mlxr, q, kc, vc, nH, nKV, offset, T, scale):
    D = q.shape[-1]
    S = kc.shape[1]
    dq = mlxr.DeviceArray.from_numpy(np.ascontiguousarray(q.reshape(T, nH * D)))
    dk = mlxr.DeviceArray.from_numpy(bf16_round(to_paged(kc)))
    dv = mlxr.DeviceArray.from_numpy(bf16_round(to_paged(vc)))
    out = mlxr.DeviceArray.zeros((T, nH * D), np.float32)
    mlxr.check(mlxr.lib.mlxr_k_flash_prefill(dq.ptr, nH * D, dk.ptr, dv.ptr, S, D, nH, nKV, offset, T, scale, out.ptr, nH * D))
    mlxr.synchronize()
    return out.numpy().reshape(T, nH, D)


@pytest.mark.parametrize("nH,nKV,offset,T", [(4, 2, 0, 1), (4, 2, 0, 45), (32, 8, 37, 200), (40, 8, 64, 130), (16, 2, 5, 96),
                                            (8, 8, 0, 97), (12, 4, 3, 350)])
def test_flash_prefill(gpu, nH, nKV, offset, T):
    """flash_prefill (Kernels.swift:1839-2000): token t of the chunk (position offset + t) attends keys
    0..offset + t; every token's output against the reference attention (oracle), and rows past the
    chunk's last key filled with NaN to check they never reach the result. Tolerance 1e-4 relative:
    q and p enter the bf16 matrix cores as hi + lo pairs (~2^-16), products accumulate in fp32."""
    D, S = 128, 512
    kc = bf16_to_f32(bf16_round(np.random.default_rng(nH + T).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    vc = bf16_to_f32(bf16_round(np.random.default_rng(nH + T + 1).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    kc[:, offset + T:] = np.nan
    vc[:, offset + T:] = np.nan
    q = np.random.default_rng(nH + T + 2).uniform(-1, 1, (T, nH, D)).astype(np.float32)
    scale = 3 / np.sqrt(D)
    got = run_flash(gpu, q, kc, vc, nH, nKV, offset, T, scale)
    assert np.all(np.isfinite(got))
    kref, vref = np.nan_to_num(kc), np.nan_to_num(vc)
    for t in range(T):
        ref = oracle.attention(q[t], kref, vref, nH, nKV, offset + t, scale)
        assert max_rel_err(got[t], ref) < 1e-4, (t, max_rel_err(got[t], ref))


@pytest.mark.parametrize("nH,nKV", [(4, 2), (8, 2), (10, 2)])
def test_attention_over_lists(gpu, nH, nKV):
    """attentionOverTheList (SparseAttentionTests.swift:214-297): the full list is bit-identical to
    split attention; subsets and clamped entries match the reference attention over those positions."""
    D, S, offset = 128, 128, 100
    L = offset + 1
    kc = bf16_to_f32(bf16_round(np.random.default_rng(1).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    vc = bf16_to_f32(bf16_round(np.random.default_rng(2).uniform(-1, 1, (nKV, S, D)).astype(np.float32)))
    q = np.random.default_rng(3).uniform(-1, 1, (nH, D)).astype(np.float32)
    scale = 3 / np.sqrt(D)
    split = run_attention(gpu, q, kc, vc, nH, nKV, offset, 1, scale)
    full = run_attention(gpu, q, kc, vc, nH, nKV, offset, 1, scale, lists=np.arange(L), count=L, list_stride=0)
    assert np.array_equal(full.view(np.uint32), split.view(np.uint32))
    subset = np.array([0, 1, 2, 3, 20, 21, 22, 23, 52, 53, 54, 55] + list(range(90, L)), np.int32)
    got = run_attention(gpu, q, kc, vc, nH, nKV, offset, 1, scale, lists=subset, count=subset.size)[0]
    assert max_rel_err(got, oracle.attention_list(q, kc, vc, nH, nKV, offset, scale, subset, subset.size, 0)) < 2e-5
    clamped = np.concatenate([subset, [L + 5, -3]]).astype(np.int32)
    got_c = run_attention(gpu, q, kc, vc, nH, nKV, offset, 1, scale, lists=clamped, count=clamped.size)[0]
    ref_c = np.sort(np.concatenate([subset, [L - 1, 0]])).astype(np.int32)
    assert max_rel_err(got_c, run_attention(gpu, q, kc, vc, nH, nKV, offset, 1, scale, lists=ref_c, count=ref_c.size)[0]) < 1e-5

    def head_list(kvh):
        lst = [0, 1, 2, 3]
        for b in range(3):
            start = 8 + 4 * (kvh + 5 * b)
            lst += list(range(start, start + 4))
        return lst + list(range(90, L))
    lists = np.stack([np.array(head_list(h), np.int32) for h in range(nKV)])
    cnt = lists.shape[1]
    got_h = run_attention(gpu, q, kc, vc, nH, nKV, offset, 1, scale, lists=lists.reshape(-1), count=cnt, list_stride=cnt)[0]
    ref_h = oracle.attention_list(q, kc, vc, nH, nKV, offset, scale, lists.reshape(-1), cnt, cnt)
    assert max_rel_err(got_h, ref_h) < 2e-5


def test_sparse_index_is_block_mean(gpu):
    """indexIsTheMeanOfEachBlock (SparseAttentionTests.swift:60-85)."""
    nKV, D, S = 2, 128, 64
    k = bf16_to_f32(bf16_round(XorShift(11).floats(nKV * S * D).reshape(nKV, S, D)))
    dk = gpu.DeviceArray.from_numpy(bf16_round(to_paged(k)))
    sentinel = bf16_round(np.array([7.0], np.float32))[0]
    idx = gpu.DeviceArray.from_numpy(np.full(S // 4 * nKV * D, sentinel, np.uint16))
    gpu.check(gpu.lib.mlxr_k_sparse_index(dk.ptr, S, nKV, D, 12, 28, idx.ptr))   # blocks 3 .. 9
    gpu.synchronize()
    got = bf16_to_f32(idx.numpy()).reshape(S // 4, nKV, D)
    ref = oracle.sparse_index(k, nKV, D, S, 3, 7)
    for b in range(S // 4):
        if 3 <= b < 10:
            assert np.array_equal(got[b], ref[b])
        else:
            assert np.all(got[b] == 7.0)


@pytest.mark.parametrize("nH,nKV", [(8, 2), (16, 8), (32, 8), (40, 8), (12, 6)])
def test_sparse_scores(gpu, nH, nKV):
    """scoresSumTheHeadsDotProducts (SparseAttentionTests.swift:88-121), tol 1e-3 * max(1, |s|)."""
    D, b0, nb = 128, 2, 150
    rng = XorShift(nH * 1000 + D)
    q = rng.floats(nH * D).reshape(nH, D)
    idxf = bf16_to_f32(bf16_round(rng.floats((b0 + nb) * nKV * D))).reshape(b0 + nb, nKV, D)
    dq, di = gpu.DeviceArray.from_numpy(q), gpu.DeviceArray.from_numpy(bf16_round(idxf))
    for rows in (1, nKV):
        ds = gpu.DeviceArray.zeros(rows * nb, np.float32)
        gpu.check(gpu.lib.mlxr_k_sparse_score(dq.ptr, di.ptr, nH, nKV, D, b0, nb, rows, ds.ptr))
        gpu.synchronize()
        ref = oracle.sparse_score(q, idxf, nH, nKV, D, b0, nb, rows)
        assert np.all(np.abs(ds.numpy().reshape(rows, nb) - ref) <= 1e-3 * np.maximum(1, np.abs(ref)))


SELECT_CASES = [(1000, 100, None), (777, 777, None), (5000, 512, [-1, 0, 0.5, 2]), (33, 1, None), (4096, 3, [-3, -2.5]),
                (3, 2, [1])]


@pytest.mark.parametrize("N,p,values", SELECT_CASES)
def test_sparse_select_exact(gpu, N, p, values):
    """selectKeepsTheTopBlocksInPositionOrder (SparseAttentionTests.swift:124-166): exact lists."""
    sink_end, b0 = 4, 1
    win_start = (b0 + N) * 4
    L = win_start + 37
    rng = XorShift(N * 7 + p)
    if values is None:
        scores = np.array([rng.float(-10, 10) for _ in range(N)], np.float32)
    else:
        scores = np.array([values[rng.next() % len(values)] for _ in range(N)], np.float32)
    plan = oracle.SparsePlan(4, b0, N, p, sink_end, win_start, L, sink_end + p * 4 + (L - win_start))
    ref = oracle.sparse_select(scores, plan)
    # the reference test's own restatement: sort by (key desc, index asc), keep p, back to position order
    keys = [oracle.sparse_key(float(s)) for s in scores]
    kept = sorted(sorted(range(N), key=lambda i: (-keys[i], i))[:p])
    expect = list(range(sink_end)) + [(b0 + n) * 4 + i for n in kept for i in range(4)] + list(range(win_start, L))
    assert ref.tolist() == expect
    ds = gpu.DeviceArray.from_numpy(scores)
    dl = gpu.DeviceArray.from_numpy(np.full(L + 8, -1, np.int32))
    gpu.check(gpu.lib.mlxr_k_sparse_select(ds.ptr, 1, b0, N, p, sink_end, win_start, L, dl.ptr, 0))
    gpu.synchronize()
    got = dl.numpy()
    assert got[:plan.count].tolist() == expect
    assert np.all(got[plan.count:] == -1)


def test_sparse_select_rows_independent(gpu):
    """selectRowsAreIndependent (SparseAttentionTests.swift:170-209)."""
    N, p, rows = 700, 64, 3
    b0, sink_end = 1, 4
    win_start = (b0 + N) * 4
    L = win_start + 21
    stride = L + 50
    rng = XorShift(77)
    scores = np.array([rng.float(-10, 10) for _ in range(rows * N)], np.float32)
    ds = gpu.DeviceArray.from_numpy(scores)
    dl = gpu.DeviceArray.from_numpy(np.full(rows * stride, -1, np.int32))
    gpu.check(gpu.lib.mlxr_k_sparse_select(ds.ptr, rows, b0, N, p, sink_end, win_start, L, dl.ptr, stride))
    gpu.synchronize()
    got = dl.numpy().reshape(rows, stride)
    count = sink_end + p * 4 + (L - win_start)
    plan = oracle.SparsePlan(4, b0, N, p, sink_end, win_start, L, count)
    for r in range(rows):
        assert got[r, :count].tolist() == oracle.sparse_select(scores[r * N:(r + 1) * N], plan).tolist()
        assert np.all(got[r, count:] == -1)


def sample_gpu(mlxr, logits, params, history=(), draws=1, seed=1):
    V = len(logits)
    hist = np.zeros(len(history) + 2, np.int32)
    hist[:len(history)] = history
    dh = mlxr.DeviceArray.from_numpy(hist)
    st = mlxr.DeviceArray.zeros(len(history) + 2, np.int32)
    rng = mlxr.DeviceArray.from_numpy(np.array([seed, 0], np.uint64))
    pos = max(0, len(history) - 1)
    toks = []
    for _ in range(draws):
        dl = mlxr.DeviceArray.from_numpy(np.asarray(logits, np.float32))
        sp = params.params(V)
        mlxr.check(mlxr.lib.mlxr_k_sample(dl.ptr, V, dh.ptr, st.ptr, rng.ptr, pos, ctypes.byref(sp)))
        mlxr.synchronize()
        toks.append(int(dh.numpy()[pos + 1]))
    return toks, st.numpy()[pos + 1]


def test_logits(V, seed=3):
    rng = XorShift(seed)
    l = np.array([-12 + 6 * rng.float() for _ in range(V)], np.float32)
    for i in range(0, V, 97):
        l[i] += 8 + 4 * rng.float()
    l[5] = 7.25; l[777 % V] = 7.25; l[V - 1] = 7.25
    return l


test_logits.__test__ = False


def test_greedy_ties_and_penalty(gpu):
    """greedyMatchesCPUArgmaxIncludingTiesAndPenalty (KernelTests.swift:355-375)."""
    for V in (1000, 32768, 151936):
        l = test_logits(V)
        l[300] = 30; l[9] = 30
        p = gpu.SamplingParameters(temperature=0, repetition_penalty=1)
        assert sample_gpu(gpu, l, p)[0] == [9]
        assert oracle.argmax(l) == 9
        p = gpu.SamplingParameters(temperature=0, repetition_penalty=1.3, repetition_window=64)
        hist = [1, 2, 9, 9, 4]
        ids, _ = oracle.sample_distribution(l, hist[-64:], 0, 40, 1, 0, 1.3)
        assert ids[0] == 300
        assert sample_gpu(gpu, l, p, history=hist)[0] == [300]


def test_penalty_long_window_and_nan(gpu):
    """The repetition penalty over a window longer than one staging round (5000 of 6000 history
    entries, tokens repeated within and across rounds) penalises each distinct token once: the
    greedy token equals the oracle's penalised argmax, and so does the penalised logits' span
    maximum (a penalised top token loses to the next). A NaN logit is never selected (the
    reference's comparisons skip it)."""
    V = 32768
    l = test_logits(V, seed=5)
    rng = np.random.default_rng(0)
    hist = rng.integers(0, V, 6000).astype(np.int32)
    top = np.argsort(-l)[:12]
    hist[-3:] = top[0]            # the top token in the first round, three times
    hist[-2500] = top[0]          # and again in the second round
    hist[-4000] = top[1]          # the second one only in the second round
    hist[-100] = top[2]; hist[-4100] = top[2]
    for window in (64, 2048, 2049, 5000):
        p = gpu.SamplingParameters(temperature=0, repetition_penalty=1.7, repetition_window=window)
        ids, _ = oracle.sample_distribution(l, hist[-window:], 0, 40, 1, 0, 1.7)
        assert sample_gpu(gpu, l, p, history=hist.tolist())[0] == [int(ids[0])], window
    ln = l.copy()
    best = int(np.argmax(l))
    ln[best - 1] = np.nan
    assert sample_gpu(gpu, ln, gpu.SamplingParameters(temperature=0))[0] == [best]
    toks, _ = sample_gpu(gpu, ln, gpu.SamplingParameters(temperature=5.0, top_k=1000), draws=50)
    assert best - 1 not in toks


def test_non_finite_logits_reported(gpu):
    l = test_logits(4096)
    l[7] = np.inf
    toks, status = sample_gpu(gpu, l, gpu.SamplingParameters())
    assert status == 1 and toks == [0]


@pytest.mark.parametrize("top_k,top_p,min_p", [(40, 0.95, 0.0), (0, 1.0, 0.0), (200, 0.8, 0.05), (5, 1.0, 0.0)])
def test_sampled_distribution(gpu, top_k, top_p, min_p):
    """sampledDistributionMatchesCPU (KernelTests.swift:394-419): same support, frequencies within 4.5 sigma."""
    V = 32768
    l = test_logits(V, seed=11)
    hist = [i * 97 for i in range(40)]
    p = gpu.SamplingParameters(temperature=0.9, top_k=top_k, top_p=top_p, min_p=min_p, repetition_penalty=1.1)
    ids, probs = oracle.sample_distribution(l, hist[-64:], 0.9, top_k, top_p, min_p, 1.1)
    cpu = dict(zip(ids.tolist(), probs.tolist()))
    draws = 3000
    toks, _ = sample_gpu(gpu, l, p, history=hist, draws=draws)
    freq = {}
    for t in toks:
        freq[t] = freq.get(t, 0) + 1
    for t in freq:
        assert t in cpu, t
    for t, pr in cpu.items():
        if pr > 0.01:
            f = freq.get(t, 0) / draws
            assert abs(f - pr) < 4.5 * np.sqrt(pr * (1 - pr) / draws) + 0.002, (t, pr, f)
