#!/usr/bin/env python3
"""Inspect and validate a MiniMind checkpoint directory.

    python inspect_minimind_checkpoint.py MODEL_DIR [--skip-weights]

Drop-in for the reference's src/python/tools/inspect_minimind_checkpoint.py
(main, :206-232): validates config.json, then every tensor's presence and
shape.  Safetensors shapes come from the file headers only; .pth / .bin
checkpoints load with torch.load(weights_only=True).  Exit status 0 when
valid, 1 otherwise, with the same messages.
"""
from __future__ import annotations

import argparse
import json
import struct
import sys
from pathlib import Path

from export_minimind_runtime import load_config, load_state_dict, validate_config, validate_weights


def safetensors_shapes(path: Path) -> dict[str, tuple[int, ...]]:
    with Path(path).open("rb") as f:
        header_size = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(header_size))
    return {k: tuple(int(v) for v in m["shape"]) for k, m in header.items() if k != "__metadata__"}


def load_weight_shapes(model_dir: Path) -> dict[str, tuple[int, ...]]:
    files = sorted(Path(model_dir).glob("*.safetensors"))
    if files:
        shapes = {}
        for f in files:
            shapes.update(safetensors_shapes(f))
        return shapes
    return {k: tuple(v.shape) for k, v in load_state_dict(model_dir).items()}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Inspect and validate a MiniMind checkpoint directory")
    ap.add_argument("model_dir", type=Path)
    ap.add_argument("--skip-weights", action="store_true")
    args = ap.parse_args(argv)
    config = load_config(args.model_dir)
    errors = validate_config(config)
    if errors:
        for e in errors:
            print(f"config error: {e}", file=sys.stderr)
        return 1
    print(f"config: hidden={config.hidden_size} layers={config.num_hidden_layers} vocab={config.vocab_size} "
          f"moe={config.use_moe}")
    if args.skip_weights:
        return 0
    actual = load_weight_shapes(args.model_dir)
    errors = validate_weights(actual, config)
    if errors:
        for e in errors[:50]:
            print(f"weight error: {e}", file=sys.stderr)
        if len(errors) > 50:
            print(f"... {len(errors) - 50} more errors", file=sys.stderr)
        return 1
    print(f"weights: {len(actual)} tensors validated")
    return 0


if __name__ == "__main__":
    sys.exit(main())
