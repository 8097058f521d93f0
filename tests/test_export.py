"""Checkpoint -> runtime export (minimind-orangepi_amd/export_minimind_runtime.py)
and the checkpoint inspector, on the CPU.

The strongest check is a round trip through the fixture-pinned file: the
runtime weights of the `mini` golden case (sha256 in tests/golden/mini.json,
the file the reference build reads to produce the golden tokens) are turned
into a HuggingFace-style checkpoint (config.json + model.safetensors) and
exported again; the output must be byte-identical.
"""
from __future__ import annotations

import hashlib
import json
import struct
import sys

import numpy as np
import pytest

from conftest import ROOT, load_golden

sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
import export_minimind_runtime as ex  # noqa: E402
import inspect_minimind_checkpoint as insp  # noqa: E402

HF_KEYS = ("hidden_size", "num_hidden_layers", "vocab_size", "num_attention_heads", "num_key_value_heads",
           "intermediate_size", "max_position_embeddings", "rms_norm_eps", "rope_theta", "tie_word_embeddings")


def write_safetensors(path, tensors: dict, dtype: str = "F32") -> None:
    """Minimal safetensors writer (header JSON + raw little-endian data)."""
    header, blobs, off = {}, [], 0
    for name, arr in tensors.items():
        a = np.asarray(arr, np.float32)
        if dtype == "F32":
            raw = a.astype("<f4").tobytes()
        elif dtype == "F16":
            raw = a.astype("<f2").tobytes()
        elif dtype == "BF16":
            raw = (a.view(np.uint32) >> 16).astype("<u2").tobytes()  # truncation: exact for bf16-valued inputs
        else:
            raw = a.astype("<i4").tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def make_checkpoint(mmr, tmp_path, case="mini", overrides=None, drop=(), dtype="F32", cast=None):
    g = load_golden(case)
    cfg_dict = {**g["config"], **(overrides or {})}
    rt = tmp_path / "runtime_src"
    mmr.write_synthetic_model(rt, mmr.make_config(**cfg_dict), g["seed"], g["std"], g["round_fp16"])
    ck = tmp_path / "checkpoint"
    ck.mkdir()
    (ck / "config.json").write_text(json.dumps({k: cfg_dict[k] for k in HF_KEYS if k in cfg_dict}))
    c = ex.load_config(ck)
    state = ex.read_runtime_weights(rt / "weights.bin", c)
    shapes = ex.expected_shapes(c)
    tensors = {n: (cast(v) if cast else v).reshape(shapes[n][0]) for n, v in state.items() if n not in drop}
    write_safetensors(ck / "model.safetensors", tensors, dtype)
    return g, rt, ck, c


def test_export_reproduces_the_fixture_file(mmr, tmp_path):
    g, rt, ck, _ = make_checkpoint(mmr, tmp_path)
    out = tmp_path / "out"
    assert ex.main(["--model", str(ck), "--output", str(out)]) == 0
    data = (out / "weights.bin").read_bytes()
    assert data == (rt / "weights.bin").read_bytes()
    assert hashlib.sha256(data).hexdigest() == g["weights_sha256"]
    c = mmr.load_config(out / "minimind_runtime_config.txt")
    for k in ("hidden_size", "num_hidden_layers", "vocab_size", "num_attention_heads", "num_key_value_heads",
              "head_dim", "intermediate_size", "max_position_embeddings"):
        assert getattr(c, k) == g["config"].get(k, getattr(c, k)), k
    assert c.rms_norm_eps == pytest.approx(g["config"]["rms_norm_eps"])
    assert mmr.has_runtime_model(out)


def test_export_fills_tied_lm_head(mmr, tmp_path):
    _, rt, ck, _ = make_checkpoint(mmr, tmp_path, overrides={"tie_word_embeddings": 1}, drop=("lm_head.weight",))
    out = tmp_path / "out"
    ex.export_weights(ck, out)
    assert (out / "weights.bin").read_bytes() == (rt / "weights.bin").read_bytes()


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
def test_export_half_precision_checkpoints(mmr, tmp_path, dtype):
    # F16 / BF16 safetensors widen exactly to fp32 (export_minimind_runtime.py:29-56)
    if dtype == "F16":
        cast = lambda v: v.astype(np.float16).astype(np.float32)  # noqa: E731
    else:
        cast = lambda v: (v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)  # noqa: E731
    _, _, ck, c = make_checkpoint(mmr, tmp_path, dtype=dtype, cast=cast)
    out = tmp_path / "out"
    ex.export_weights(ck, out)
    got = ex.read_runtime_weights(out / "weights.bin", c)
    src = ex.read_safetensors(ck / "model.safetensors")
    for name, v in got.items():
        np.testing.assert_array_equal(v, src[name].reshape(-1))


def test_export_fp16_payload(mmr, tmp_path):
    g, rt, ck, c = make_checkpoint(mmr, tmp_path)
    out = tmp_path / "out"
    ex.export_weights(ck, out, dtype="f16")
    data = (out / "weights.bin").read_bytes()
    assert data[:8] == b"MMRTH001"
    full = (rt / "weights.bin").stat().st_size
    assert len(data) < 0.55 * full
    got, ref = ex.read_runtime_weights(out / "weights.bin", c), ex.read_runtime_weights(rt / "weights.bin", c)
    for name in ref:  # the fixture's weights are fp16-representable: the payload is exact
        np.testing.assert_array_equal(got[name], ref[name])


def test_export_torch_checkpoint(mmr, tmp_path):
    torch = pytest.importorskip("torch")
    _, rt, ck, c = make_checkpoint(mmr, tmp_path)
    state = ex.read_safetensors(ck / "model.safetensors")
    (ck / "model.safetensors").unlink()
    torch.save({"model": {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in state.items()}}, ck / "model.pth")
    out = tmp_path / "out"
    ex.export_weights(ck, out)
    assert (out / "weights.bin").read_bytes() == (rt / "weights.bin").read_bytes()


def test_export_errors(mmr, tmp_path):
    _, _, ck, _ = make_checkpoint(mmr, tmp_path, drop=("model.layers.1.mlp.up_proj.weight",))
    with pytest.raises(RuntimeError, match="missing tensor: model.layers.1.mlp.up_proj.weight"):
        ex.export_weights(ck, tmp_path / "o1")
    state = ex.read_safetensors(ck / "model.safetensors")
    state["model.layers.1.mlp.up_proj.weight"] = np.zeros((3, 4), np.float32)
    write_safetensors(ck / "model.safetensors", state)
    with pytest.raises(RuntimeError, match=r"shape mismatch for model.layers.1.mlp.up_proj.weight"):
        ex.export_weights(ck, tmp_path / "o2")
    cfg = json.loads((ck / "config.json").read_text())
    (ck / "config.json").write_text(json.dumps({**cfg, "head_dim": 7}))
    with pytest.raises(RuntimeError, match="head_dim must equal"):
        ex.export_weights(ck, tmp_path / "o3")
    (ck / "config.json").write_text(json.dumps(cfg))
    write_safetensors(ck / "model.safetensors", {"x": np.zeros(2, np.float32)}, "I32")
    with pytest.raises(RuntimeError, match="unsupported safetensors dtype"):
        ex.export_weights(ck, tmp_path / "o4")
    with pytest.raises(FileNotFoundError):
        ex.export_weights(tmp_path / "empty_dir_that_does_not_exist", tmp_path / "o5")


def test_config_defaults_and_reference_keys(mmr, tmp_path):
    # inspect_minimind_checkpoint.py:32-67: head_dim = hidden / heads,
    # intermediate = ceil(hidden * pi / 64) * 64
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 512, "num_attention_heads": 8}))
    c = ex.load_config(tmp_path)
    assert c.head_dim == 64 and c.intermediate_size == 1664 and c.num_key_value_heads == 4
    assert ex.default_intermediate_size(768) == 2432
    ref = ex.runtime_config_text(c, reference_keys=True)
    keys = [line.split("=")[0] for line in ref.splitlines()]
    assert keys == list(ex.REFERENCE_CONFIG_KEYS) and "rms_norm_eps" not in ref
    full = ex.runtime_config_text(c)
    assert full.startswith(ref) and "rms_norm_eps=1e-06" in full and "rope_theta=1000000.0" in full
    for text in (ref, full):
        p = tmp_path / "minimind_runtime_config.txt"
        p.write_text(text)
        rc = mmr.load_config(p)
        assert (rc.hidden_size, rc.head_dim, rc.intermediate_size) == (512, 64, 1664)


def test_inspect_cli(mmr, tmp_path, capsys):
    _, _, ck, _ = make_checkpoint(mmr, tmp_path)
    assert insp.main([str(ck)]) == 0
    assert "tensors validated" in capsys.readouterr().out
    assert insp.main([str(ck), "--skip-weights"]) == 0
    state = ex.read_safetensors(ck / "model.safetensors")
    del state["model.norm.weight"]
    write_safetensors(ck / "model.safetensors", state)
    assert insp.main([str(ck)]) == 1
    assert "weight error: missing tensor: model.norm.weight" in capsys.readouterr().err
