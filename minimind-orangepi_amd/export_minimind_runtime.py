#!/usr/bin/env python3
"""Export a MiniMind checkpoint directory into the runtime format.

    python export_minimind_runtime.py --model CHECKPOINT_DIR --output RUNTIME_DIR
                                      [--dtype f32|f16] [--reference-keys]

Drop-in for the reference's src/python/tools/export_minimind_runtime.py
(export_weights, :185-226, same CLI flags and output files):
  * reads config.json with the reference defaults (inspect_minimind_checkpoint.py:
    36-67) and validates it (:70-108);
  * reads every *.safetensors file (F32 / F16 / BF16), else pytorch_model.bin,
    model.pth or the first *.pth, unwrapping a nested "model" / "state_dict";
  * fills lm_head.weight from the embedding when it is absent and tied;
  * checks every tensor of the runtime order for presence and shape;
  * writes minimind_runtime_config.txt (key=value) and weights.bin: magic
    "MMRTW001", then per tensor in the fixed order (runtime_loader.cpp:133-163)
    u64 name length, name, u64 element count, the values as little-endian fp32;
  * copies tokenizer.json when present.

Differences, each deliberate:
  * the config file also carries rms_norm_eps and rope_theta from config.json
    (the reference runtime ignores unknown keys; without them it falls back to
    eps 1e-6 whatever the checkpoint says); --reference-keys writes exactly
    the reference's key set;
  * --dtype f16 writes magic "MMRTH001" with IEEE fp16 payloads (round to
    nearest even): half the file, and exactly the weights the GPU runtime
    uploads;
  * .pth / .bin checkpoints load with torch.load(weights_only=True), which
    executes nothing from the file;
  * arrays are converted with numpy instead of per-value Python loops.

This module needs only numpy (plus torch for .pth/.bin inputs); it does not
load the GPU library.
"""
from __future__ import annotations

import argparse
import json
import math
import shutil
import struct
import sys
from dataclasses import dataclass
from pathlib import Path

import numpy as np

RUNTIME_MAGIC_F32 = b"MMRTW001"
RUNTIME_MAGIC_F16 = b"MMRTH001"


@dataclass(frozen=True)
class CheckpointConfig:
    """config.json fields the runtime uses, with the reference's defaults."""
    hidden_size: int = 768
    num_hidden_layers: int = 8
    use_moe: bool = False
    vocab_size: int = 6400
    num_attention_heads: int = 8
    num_key_value_heads: int = 4
    head_dim: int = 96
    intermediate_size: int = 2432
    max_position_embeddings: int = 32768
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    tie_word_embeddings: bool = True
    hidden_act: str = "silu"
    num_experts: int = 4
    num_experts_per_tok: int = 1
    moe_intermediate_size: int = 2432


def default_intermediate_size(hidden_size: int) -> int:
    """ceil(hidden * pi / 64) * 64 (inspect_minimind_checkpoint.py:32-33)."""
    return math.ceil(hidden_size * math.pi / 64) * 64


def load_config(model_dir: Path) -> CheckpointConfig:
    path = Path(model_dir) / "config.json"
    data = json.loads(path.read_text()) if path.exists() else {}
    hidden = int(data.get("hidden_size", 768))
    heads = int(data.get("num_attention_heads", 8))
    inter = int(data.get("intermediate_size", default_intermediate_size(hidden)))
    use_moe = bool(data["use_moe"]) if "use_moe" in data else ("moe_intermediate_size" in data or
                                                               "num_experts_per_tok" in data)
    return CheckpointConfig(
        hidden_size=hidden,
        num_hidden_layers=int(data.get("num_hidden_layers", data.get("n_layers", 8))),
        use_moe=use_moe,
        vocab_size=int(data.get("vocab_size", 6400)),
        num_attention_heads=heads,
        num_key_value_heads=int(data.get("num_key_value_heads", 4)),
        head_dim=int(data.get("head_dim", hidden // heads)),
        intermediate_size=inter,
        max_position_embeddings=int(data.get("max_position_embeddings", 32768)),
        rms_norm_eps=float(data.get("rms_norm_eps", 1e-6)),
        rope_theta=float(data.get("rope_theta", 1_000_000.0)),
        tie_word_embeddings=bool(data.get("tie_word_embeddings", True)),
        hidden_act=str(data.get("hidden_act", "silu")),
        num_experts=int(data.get("num_experts", 4)),
        num_experts_per_tok=int(data.get("num_experts_per_tok", 1)),
        moe_intermediate_size=int(data.get("moe_intermediate_size", data.get("intermediate_size", inter))),
    )


def validate_config(c: CheckpointConfig) -> list[str]:
    errors = []
    for field in ("hidden_size", "num_hidden_layers", "vocab_size", "num_attention_heads", "num_key_value_heads",
                  "head_dim", "intermediate_size", "max_position_embeddings"):
        if getattr(c, field) <= 0:
            errors.append(f"{field} must be positive")
    if c.num_attention_heads > 0 and c.hidden_size % c.num_attention_heads != 0:
        errors.append("hidden_size must be divisible by num_attention_heads")
    if c.num_attention_heads > 0 and c.head_dim != c.hidden_size // c.num_attention_heads:
        errors.append("head_dim must equal hidden_size / num_attention_heads")
    if c.num_key_value_heads > 0 and c.num_attention_heads % c.num_key_value_heads != 0:
        errors.append("num_attention_heads must be divisible by num_key_value_heads")
    if c.hidden_act != "silu":
        errors.append("only silu hidden_act is currently supported")
    if c.rms_norm_eps <= 0:
        errors.append("rms_norm_eps must be positive")
    if c.rope_theta <= 0:
        errors.append("rope_theta must be positive")
    if c.use_moe:
        if c.num_experts <= 0:
            errors.append("num_experts must be positive")
        if c.num_experts_per_tok != 1:
            errors.append("only top-1 MoE routing is currently supported")
        if c.moe_intermediate_size <= 0:
            errors.append("moe_intermediate_size must be positive")
    return errors


def tensor_order(c: CheckpointConfig) -> list[str]:
    """Runtime tensor order (runtime_loader.cpp:133-163)."""
    names = ["model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"]
    for layer in range(c.num_hidden_layers):
        p = f"model.layers.{layer}."
        names += [p + "input_layernorm.weight", p + "post_attention_layernorm.weight",
                  p + "self_attn.q_norm.weight", p + "self_attn.k_norm.weight",
                  p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                  p + "self_attn.v_proj.weight", p + "self_attn.o_proj.weight"]
        if c.use_moe:
            names.append(p + "mlp.gate.weight")
            for e in range(c.num_experts):
                q = p + f"mlp.experts.{e}."
                names += [q + "gate_proj.weight", q + "up_proj.weight", q + "down_proj.weight"]
        else:
            names += [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", p + "mlp.down_proj.weight"]
    return names


def expected_shapes(c: CheckpointConfig) -> dict[str, tuple[tuple[int, ...], bool]]:
    """name -> (shape, required) (inspect_minimind_checkpoint.py:111-139)."""
    q_out, kv_out, H = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim, c.hidden_size
    out = {"model.embed_tokens.weight": ((c.vocab_size, H), True),
           "model.norm.weight": ((H,), True),
           "lm_head.weight": ((c.vocab_size, H), not c.tie_word_embeddings)}
    for layer in range(c.num_hidden_layers):
        p = f"model.layers.{layer}."
        out[p + "input_layernorm.weight"] = ((H,), True)
        out[p + "post_attention_layernorm.weight"] = ((H,), True)
        out[p + "self_attn.q_proj.weight"] = ((q_out, H), True)
        out[p + "self_attn.k_proj.weight"] = ((kv_out, H), True)
        out[p + "self_attn.v_proj.weight"] = ((kv_out, H), True)
        out[p + "self_attn.o_proj.weight"] = ((H, q_out), True)
        out[p + "self_attn.q_norm.weight"] = ((c.head_dim,), True)
        out[p + "self_attn.k_norm.weight"] = ((c.head_dim,), True)
        if c.use_moe:
            out[p + "mlp.gate.weight"] = ((c.num_experts, H), True)
            for e in range(c.num_experts):
                q = p + f"mlp.experts.{e}."
                out[q + "gate_proj.weight"] = ((c.moe_intermediate_size, H), True)
                out[q + "up_proj.weight"] = ((c.moe_intermediate_size, H), True)
                out[q + "down_proj.weight"] = ((H, c.moe_intermediate_size), True)
        else:
            out[p + "mlp.gate_proj.weight"] = ((c.intermediate_size, H), True)
            out[p + "mlp.up_proj.weight"] = ((c.intermediate_size, H), True)
            out[p + "mlp.down_proj.weight"] = ((H, c.intermediate_size), True)
    return out


# ---------------------------------------------------------------- loading ----

def read_safetensors(path: Path) -> dict[str, np.ndarray]:
    """The safetensors container (u64 header size, JSON header, raw data),
    F32 / F16 / BF16 tensors returned as float32 arrays (exact)."""
    path = Path(path)
    with path.open("rb") as f:
        header_size = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(header_size))
    data = np.memmap(path, dtype=np.uint8, mode="r")
    base = 8 + header_size
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        start, end = meta["data_offsets"]
        raw = np.asarray(data[base + start: base + end])
        shape = tuple(int(v) for v in meta["shape"])
        dtype = meta["dtype"]
        if dtype == "F32":
            arr = raw.view("<f4")
        elif dtype == "F16":
            arr = raw.view("<f2").astype(np.float32)
        elif dtype == "BF16":
            arr = (raw.view("<u2").astype(np.uint32) << 16).view("<f4")
        else:
            raise RuntimeError(f"unsupported safetensors dtype: {dtype}")
        out[name] = np.array(arr, dtype=np.float32).reshape(shape)
    return out


def _torch_state(path: Path) -> dict:
    try:
        import torch
    except ImportError as exc:
        raise RuntimeError("PyTorch checkpoint export requires torch to be installed") from exc
    loaded = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(loaded, dict) and isinstance(loaded.get("model"), dict):
        loaded = loaded["model"]
    if isinstance(loaded, dict) and isinstance(loaded.get("state_dict"), dict):
        loaded = loaded["state_dict"]
    if not isinstance(loaded, dict):
        raise RuntimeError("unsupported checkpoint format")
    return {k: v.detach().cpu().float().numpy() if hasattr(v, "detach") else np.asarray(v, np.float32)
            for k, v in loaded.items() if hasattr(v, "shape")}


def load_state_dict(model_dir: Path) -> dict[str, np.ndarray]:
    model_dir = Path(model_dir)
    files = sorted(model_dir.glob("*.safetensors"))
    if files:
        state = {}
        for f in files:
            state.update(read_safetensors(f))
        return state
    for name in ("pytorch_model.bin", "model.pth"):
        if (model_dir / name).exists():
            return _torch_state(model_dir / name)
    pth = sorted(model_dir.glob("*.pth"))
    if not pth:
        raise FileNotFoundError(f"no safetensors, pytorch_model.bin, or .pth checkpoint found in {model_dir}")
    return _torch_state(pth[0])


def validate_weights(actual: dict[str, tuple[int, ...]], c: CheckpointConfig) -> list[str]:
    """Presence and shape of every tensor (inspect_minimind_checkpoint.py:193-203)."""
    errors = []
    for name, (shape, required) in expected_shapes(c).items():
        if name not in actual:
            if required:
                errors.append(f"missing tensor: {name}")
            continue
        if tuple(actual[name]) != shape:
            errors.append(f"shape mismatch for {name}: expected {shape}, got {tuple(actual[name])}")
    return errors


# ---------------------------------------------------------------- writing ----

REFERENCE_CONFIG_KEYS = ("hidden_size", "num_hidden_layers", "use_moe", "vocab_size", "num_attention_heads",
                         "num_key_value_heads", "head_dim", "intermediate_size", "max_position_embeddings",
                         "tie_word_embeddings", "num_experts", "num_experts_per_tok", "moe_intermediate_size")


def runtime_config_text(c: CheckpointConfig, reference_keys: bool = False) -> str:
    """minimind_runtime_config.txt: the reference's keys (export_minimind_runtime.py:
    174-190) in its order, then rms_norm_eps and rope_theta unless reference_keys."""
    def fmt(key):
        v = getattr(c, key)
        return str(int(v)) if isinstance(v, bool) else str(v)
    lines = [f"{k}={fmt(k)}" for k in REFERENCE_CONFIG_KEYS]
    if not reference_keys:
        lines += [f"rms_norm_eps={c.rms_norm_eps!r}", f"rope_theta={c.rope_theta!r}"]
    return "\n".join(lines) + "\n"


def export_weights(model_dir: Path, output_dir: Path, dtype: str = "f32", reference_keys: bool = False) -> None:
    model_dir, output_dir = Path(model_dir), Path(output_dir)
    if dtype not in ("f32", "f16"):
        raise ValueError("dtype must be f32 or f16")
    c = load_config(model_dir)
    errors = validate_config(c)
    if errors:
        raise RuntimeError("invalid config: " + errors[0])
    if c.use_moe and c.num_experts_per_tok != 1:
        raise RuntimeError("runtime export currently supports top-1 MoE checkpoints only")
    state = load_state_dict(model_dir)
    if "lm_head.weight" not in state and c.tie_word_embeddings and "model.embed_tokens.weight" in state:
        state["lm_head.weight"] = state["model.embed_tokens.weight"]
    order = tensor_order(c)
    expected = expected_shapes(c)
    errors = []
    for name in order:
        if name not in state:
            errors.append(f"missing tensor: {name}")
        elif tuple(state[name].shape) != expected[name][0]:
            errors.append(f"shape mismatch for {name}: expected {expected[name][0]}, got {tuple(state[name].shape)}")
    if errors:
        raise RuntimeError("\n".join(errors[:20]))
    output_dir.mkdir(parents=True, exist_ok=True)
    (output_dir / "minimind_runtime_config.txt").write_text(runtime_config_text(c, reference_keys))
    payload = np.dtype("<f2") if dtype == "f16" else np.dtype("<f4")
    with (output_dir / "weights.bin").open("wb") as f:
        f.write(RUNTIME_MAGIC_F16 if dtype == "f16" else RUNTIME_MAGIC_F32)
        for name in order:
            values = np.ascontiguousarray(np.asarray(state[name], dtype=np.float32).reshape(-1))
            encoded = name.encode("utf-8")
            f.write(struct.pack("<Q", len(encoded)))
            f.write(encoded)
            f.write(struct.pack("<Q", values.size))
            f.write(values.astype(payload).tobytes())
    tokenizer = model_dir / "tokenizer.json"
    if tokenizer.exists():
        shutil.copy2(tokenizer, output_dir / "tokenizer.json")


def read_runtime_weights(path: Path, c: CheckpointConfig) -> dict[str, np.ndarray]:
    """weights.bin (either payload) -> name -> flat float32 array, in file order."""
    data = Path(path).read_bytes()
    magic = data[:8]
    if magic not in (RUNTIME_MAGIC_F32, RUNTIME_MAGIC_F16):
        raise RuntimeError("unsupported runtime weight format")
    item = np.dtype("<f2") if magic == RUNTIME_MAGIC_F16 else np.dtype("<f4")
    off, out = 8, {}
    for expected in tensor_order(c):
        (n,) = struct.unpack_from("<Q", data, off)
        name = data[off + 8: off + 8 + n].decode("utf-8")
        if name != expected:
            raise RuntimeError(f"expected tensor {expected}, got {name}")
        off += 8 + n
        (count,) = struct.unpack_from("<Q", data, off)
        off += 8
        out[name] = np.frombuffer(data, dtype=item, count=count, offset=off).astype(np.float32)
        off += count * item.itemsize
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Export dense MiniMind weights into the local runtime format")
    ap.add_argument("--model", type=Path, required=True)
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--dtype", choices=("f32", "f16"), default="f32",
                    help="payload of weights.bin: f32 (MMRTW001, the reference format) or f16 (MMRTH001)")
    ap.add_argument("--reference-keys", action="store_true",
                    help="write exactly the reference exporter's config keys (no rms_norm_eps / rope_theta)")
    args = ap.parse_args(argv)
    export_weights(args.model, args.output, args.dtype, args.reference_keys)
    print(f"exported runtime weights to {args.output}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
