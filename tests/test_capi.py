"""The C ABI on the CPU: libmlxr loads, exports every function include/mlxr.h declares, and rejects
bad files and arguments before any device work (GPU.swift:214-272 validation, EngineTests.swift:125-209)."""
import json
import os
import re
import struct

import numpy as np
import pytest

import configs
import mlxr
from qfix import read_safetensors, write_safetensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "mlxr.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlxr_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 40
    for n in names:
        assert hasattr(mlxr.lib, n), n


def test_library_is_built_for_gfx950():
    import subprocess
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                          f"--input={mlxr.LIB_PATH}"], capture_output=True, text=True)
    if out.returncode == 0 and out.stdout:
        assert "gfx950" in out.stdout


def write_st(path, header, data=b""):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


@pytest.fixture
def model_dir(tmp_path):
    d = str(tmp_path / "m")
    mlxr.synth_write(configs.tiny("qwen3", layers=1), seed=1, directory=d)
    return d


def open_err(d):
    with pytest.raises(mlxr.EngineError) as e:
        mlxr.Transformer(d, 256)
    return e.value


def test_valid_model_reaches_the_device_check(model_dir):
    if mlxr.device_count() == 0:
        assert open_err(model_dir).case == "noMetalDevice"


def test_malformed_safetensors(tmp_path, model_dir):
    cfg = open(os.path.join(model_dir, "config.json")).read()
    cases = {
        "truncated": lambda p: open(p, "wb").write(b"\x01\x02"),
        "header length": lambda p: open(p, "wb").write(struct.pack("<Q", 1 << 40) + b"{}"),
        "bad json": lambda p: open(p, "wb").write(struct.pack("<Q", 5) + b"{nope"),
        "out of bounds": lambda p: write_st(p, {"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8),
        "size mismatch": lambda p: write_st(p, {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 16]}}, b"\0" * 16),
        "negative shape": lambda p: write_st(p, {"x": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}}),
        # the reference's rejectsMalformedHeaders cases (EngineTests.swift:164-178), 16 payload bytes
        "past end": lambda p: write_st(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 1000]}}, b"\0" * 16),
        "start after end": lambda p: write_st(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [8, 0]}}, b"\0" * 16),
        "negative offset": lambda p: write_st(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [-16, 0]}}, b"\0" * 16),
        "shape bytes": lambda p: write_st(p, {"a": {"dtype": "F32", "shape": [5], "data_offsets": [0, 16]}}, b"\0" * 16),
        "shape overflow": lambda p: write_st(p, {"a": {"dtype": "F32", "shape": [4611686018427387904, 4],
                                                       "data_offsets": [0, 16]}}, b"\0" * 16),
        "negative dim": lambda p: write_st(p, {"a": {"dtype": "F32", "shape": [-4], "data_offsets": [0, 16]}}, b"\0" * 16),
        "not json": lambda p: open(p, "wb").write(struct.pack("<Q", 8) + b"not json" + b"\0" * 16),
        # rejectsHugeHeaderLength (EngineTests.swift:186-197)
        "huge header": lambda p: open(p, "wb").write(struct.pack("<Q", (1 << 64) - 5) + b"\0" * 64),
        "entry not an object": lambda p: write_st(p, {"a": 3}, b"\0" * 16),
    }
    for name, make in cases.items():
        d = tmp_path / name.replace(" ", "_")
        d.mkdir()
        (d / "config.json").write_text(cfg)
        make(str(d / "model.safetensors"))
        assert open_err(str(d)).case == "invalidFile", name


def test_index_lists_the_shards(tmp_path, model_dir):
    """WeightStore.shardFiles (GPU.swift:316-330): with model.safetensors.index.json, only the files
    its weight_map names load, so an unrelated sidecar (here a corrupt one) is never opened; without
    the index every .safetensors file loads and the corrupt one is rejected. An index that names no
    existing file falls back to every file."""
    import shutil
    def layout(name, index):
        d = tmp_path / name
        shutil.copytree(model_dir, d)
        (d / "optiq_vision.safetensors").write_bytes(struct.pack("<Q", 5) + b"{nope")
        if index is not None:
            (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": index}))
        return str(d)
    ok = layout("indexed", {"model.embed_tokens.weight": "model.safetensors"})
    bad = layout("plain", None)
    stale = layout("stale", {"model.embed_tokens.weight": "model-00001-of-00002.safetensors"})
    assert open_err(bad).case == "invalidFile"
    assert open_err(stale).case == "invalidFile"
    if mlxr.device_count() == 0:
        assert open_err(ok).case == "noMetalDevice"   # past the loader: only the device is missing
    else:
        with mlxr.Transformer(ok, 256) as m:
            assert m.vocab_size > 0


def test_config_validation(tmp_path, model_dir):
    st = open(os.path.join(model_dir, "model.safetensors"), "rb").read()
    base = json.load(open(os.path.join(model_dir, "config.json")))
    cases = [({"model_type": "gemma3"}, "unsupported"), ({"hidden_size": 0}, "invalidFile"),
             ({"num_key_value_heads": 3}, "invalidFile"), ({"rope_theta": -1}, "invalidFile")]
    for i, (patch, case) in enumerate(cases):
        d = tmp_path / f"c{i}"
        d.mkdir()
        c = dict(base); c.update(patch)
        (d / "config.json").write_text(json.dumps(c))
        (d / "model.safetensors").write_bytes(st)
        assert open_err(str(d)).case == case, patch
    empty = tmp_path / "empty"
    empty.mkdir()
    assert open_err(str(empty)).case == "invalidFile"


def test_missing_tensor(tmp_path, model_dir):
    import json as _j, struct as _s
    raw = open(os.path.join(model_dir, "model.safetensors"), "rb").read()
    hdr = _j.loads(raw[8:8 + _s.unpack("<Q", raw[:8])[0]])
    dtypes = {k: v["dtype"] for k, v in hdr.items() if k != "__metadata__"}
    t = read_safetensors(os.path.join(model_dir, "model.safetensors"))
    del t["model.layers.0.mlp.down_proj.scales"]
    d = tmp_path / "miss"
    d.mkdir()
    write_safetensors(str(d / "model.safetensors"), t, dtypes)
    (d / "config.json").write_text(open(os.path.join(model_dir, "config.json")).read())
    e = open_err(str(d))
    assert e.case in ("missingTensor", "unsupported")


def test_kernel_entry_points_reject_bad_shapes():
    qm = (mlxr.QMat * 1)(mlxr.QMat(None, None, None, None, 0))
    rc = mlxr.lib.mlxr_k_qmv(qm, 1, 512, 4, 64, 0, None, None, 1e-6, None, 0)
    assert rc != 0
    rc = mlxr.lib.mlxr_k_sparse_select(None, 1, 1, 10, 11, 4, 44, 50, None, 0)
    assert rc != 0


def test_sparse_environment_parsing():
    """SparseAttention.parse(environment:) (SparseAttentionTests.swift:40-50)."""
    std = mlxr.SparseAttention()
    assert mlxr.SparseAttention.from_environment({}) == std
    for on in ["", "1", "on", "ON", " true ", "yes"]:
        assert mlxr.SparseAttention.from_environment({"MLXR_SPARSE_ATTN": on}) == std, on
    for off in ["0", "off", "false", "no", "maybe", "-5"]:
        assert mlxr.SparseAttention.from_environment({"MLXR_SPARSE_ATTN": off}) is None, off
    assert mlxr.SparseAttention.from_environment({"MLXR_SPARSE_ATTN": "4096"}).top_k == 4096
    env = {"MLXR_SPARSE_WINDOW": "256", "MLXR_SPARSE_MIN": "2000", "MLXR_SPARSE_SHARED": "1"}
    c = mlxr.SparseAttention.from_environment(env)
    assert c.top_k == 2048 and c.window == 256 and c.min_context == 2000 and not c.per_head
