"""Test fixtures restating the reference tests' generators (Tests/MLXEngineTests/KernelTests.swift).

- XorShift: `RNG` (KernelTests.swift:8-14), including its `float(lo, hi)`.
- pack_codes: `pack(_:bits:)` (KernelTests.swift:34-43), done here with numpy bit arrays so it is
  independent of the oracle's loop.
- QuantFixture: random codes, scales U(0.001, 0.05), biases U(-0.2, 0.2) rounded to the storage
  dtype (KernelTests.swift:48-100).
"""
import numpy as np

M64 = (1 << 64) - 1


class XorShift:
    def __init__(self, s):
        self.s = s & M64

    def next(self):
        s = self.s
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        self.s = s
        return s

    def float(self, lo=-1.0, hi=1.0):
        # Float arithmetic as in Swift: lo + (hi - lo) * Float(next() % 1_000_000) / 1_000_000
        f = np.float32(self.next() % 1_000_000) / np.float32(1_000_000)
        return np.float32(np.float32(lo) + np.float32(np.float32(hi) - np.float32(lo)) * np.float32(f))

    def floats(self, n, lo=-1.0, hi=1.0):
        return np.array([self.float(lo, hi) for _ in range(n)], np.float32)


def bf16_round(x):
    x = np.ascontiguousarray(x, np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_codes(codes, bits):
    """Little-endian bit stream: bit b of value i at stream bit i*bits+b."""
    codes = np.asarray(codes, np.uint64).reshape(-1)
    bitsarr = ((codes[:, None] >> np.arange(bits, dtype=np.uint64)[None, :]) & 1).astype(np.uint8).reshape(-1)
    pad = (-bitsarr.size) % 8
    if pad:
        bitsarr = np.concatenate([bitsarr, np.zeros(pad, np.uint8)])
    return np.packbits(bitsarr, bitorder="little")


def unpack_codes(packed, n, bits):
    b = np.unpackbits(np.asarray(packed, np.uint8), bitorder="little")[: n * bits].reshape(n, bits).astype(np.uint32)
    return (b << np.arange(bits, dtype=np.uint32)[None, :]).sum(axis=1).astype(np.uint32)


class QuantFixture:
    def __init__(self, O, K, bits, gs, st="bf16", seed=7, with_bias=False, fast=False):
        self.O, self.K, self.bits, self.gs, self.st = O, K, bits, gs, st
        groups = K // gs
        if fast:   # numpy generator for large shapes (not the reference's RNG)
            rs = np.random.default_rng(seed)
            q = rs.integers(0, 1 << bits, size=(O, K), dtype=np.uint64)
            scales = rs.uniform(0.001, 0.05, size=(O, groups)).astype(np.float32)
            biases = rs.uniform(-0.2, 0.2, size=(O, groups)).astype(np.float32)
            bias = rs.uniform(-0.5, 0.5, size=O).astype(np.float32) if with_bias else None
        else:
            rng = XorShift(seed)
            q = np.array([rng.next() % (1 << bits) for _ in range(O * K)], np.uint64).reshape(O, K)
            sb = []
            for _ in range(O * groups):
                sb.append((rng.float(0.001, 0.05), rng.float(-0.2, 0.2)))
            scales = np.array([a for a, _ in sb], np.float32).reshape(O, groups)
            biases = np.array([b for _, b in sb], np.float32).reshape(O, groups)
            bias = np.array([rng.float(-0.5, 0.5) for _ in range(O)], np.float32) if with_bias else None
        self.codes = q.astype(np.uint32)
        if st == "bf16":
            self.s_raw, self.b_raw = bf16_round(scales), bf16_round(biases)
            self.scales, self.biases = bf16_to_f32(self.s_raw), bf16_to_f32(self.b_raw)
            if bias is not None:
                self.bias_raw = bf16_round(bias)
                self.bias = bf16_to_f32(self.bias_raw)
        else:
            self.s_raw, self.b_raw = scales.astype(np.float16).view(np.uint16), biases.astype(np.float16).view(np.uint16)
            self.scales, self.biases = scales.astype(np.float16).astype(np.float32), biases.astype(np.float16).astype(np.float32)
            if bias is not None:
                self.bias_raw = bias.astype(np.float16).view(np.uint16)
                self.bias = bias.astype(np.float16).astype(np.float32)
        if bias is None:
            self.bias_raw = None
            self.bias = None
        self.packed = np.stack([pack_codes(self.codes[r], bits) for r in range(O)]) if not fast else self._pack_fast()

    def _pack_fast(self):
        return pack_codes(self.codes.reshape(-1), self.bits).reshape(self.O, self.K * self.bits // 8)

    def dense(self):
        """Dequantized weights [O][K] (fp32 `s*q+b`)."""
        g = np.repeat(np.arange(self.K // self.gs), self.gs)
        return (self.codes.astype(np.float32) * self.scales[:, g] + self.biases[:, g]).astype(np.float32)

    def reference(self, x):
        """QuantFixture.reference (KernelTests.swift:102-113): float64 accumulate."""
        y = np.asarray(x, np.float64).reshape(-1, self.K) @ self.dense().astype(np.float64).T
        if self.bias is not None:
            y = y.astype(np.float32) + self.bias
        return y.astype(np.float32)

    def device(self, mlxr):
        self.d_w = mlxr.DeviceArray.from_numpy(self.packed)
        self.d_s = mlxr.DeviceArray.from_numpy(self.s_raw)
        self.d_b = mlxr.DeviceArray.from_numpy(self.b_raw)
        self.d_bias = mlxr.DeviceArray.from_numpy(self.bias_raw) if self.bias_raw is not None else None
        return mlxr.QMat(self.d_w.ptr, self.d_s.ptr, self.d_b.ptr, self.d_bias.ptr if self.d_bias else None, self.O)

    def oracle(self, oracle):
        return oracle.QMatrix(self.packed, self.scales, self.biases, self.K, self.bits, self.gs, bias=self.bias)


class SynthMatrix:
    """A matrix at a real model shape, N(0, std) weights quantized exactly as the synthetic models are
    (mlxr_synth_matrix: MLX affine, bf16 scale / bias). Exposes the QuantFixture members the kernel
    tests use (packed bytes, raw and float scales / biases, device and oracle views)."""

    def __init__(self, mlxr, O, K, bits, gs, seed=1, tensor_id=0, std=0.02):
        self.O, self.K, self.bits, self.gs, self.st = O, K, bits, gs, "bf16"
        self.packed, self.s_raw, self.b_raw = mlxr.synth_matrix(seed, tensor_id, O, K, bits, gs, std)
        self.scales, self.biases = bf16_to_f32(self.s_raw), bf16_to_f32(self.b_raw)
        self.bias_raw = self.bias = None

    def rows(self, r0, r1):
        """Rows [r0, r1) as a matrix of their own."""
        sub = object.__new__(SynthMatrix)
        sub.O, sub.K, sub.bits, sub.gs, sub.st = r1 - r0, self.K, self.bits, self.gs, self.st
        sub.packed, sub.s_raw, sub.b_raw = self.packed[r0:r1], self.s_raw[r0:r1], self.b_raw[r0:r1]
        sub.scales, sub.biases = self.scales[r0:r1], self.biases[r0:r1]
        sub.bias_raw = sub.bias = None
        return sub

    device = QuantFixture.device
    oracle = QuantFixture.oracle


def max_rel_err(a, b):
    """assertClose's metric (KernelTests.swift:116-124): |a-b| / max(1, |b|)."""
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(1.0, np.abs(b)))) if a.size else 0.0


def read_safetensors(path):
    """Minimal reader (header JSON + raw little-endian data): bf16 tensors come back as uint16."""
    import json
    import struct
    raw = open(path, "rb").read()
    (hl,) = struct.unpack("<Q", raw[:8])
    hdr = json.loads(raw[8:8 + hl])
    data = memoryview(raw)[8 + hl:]
    dt = {"U32": np.uint32, "BF16": np.uint16, "F16": np.float16, "F32": np.float32, "U8": np.uint8, "I32": np.int32}
    out = {}
    for k, v in hdr.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        out[k] = np.frombuffer(data[a:b], dtype=dt[v["dtype"]]).reshape(v["shape"]).copy()
    return out


def write_safetensors(path, tensors, dtypes):
    import json
    import struct
    hdr, off, blobs = {}, 0, []
    for k, a in tensors.items():
        b = np.ascontiguousarray(a).tobytes()
        hdr[k] = {"dtype": dtypes[k], "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    h = json.dumps(hdr).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))
