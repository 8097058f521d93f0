#!/usr/bin/env python3
"""Generate the golden fixtures in tests/golden/ from the reference's own CPU path.

Runs in the build container only (it needs /root/reference to build
oracle/_ref/ref_driver).  For every case it
  1. writes a synthetic model directory (minimind_runtime_config.txt +
     weights.bin) with the runtime's seeded generator,
  2. runs the reference build (oracle/_ref/ref_driver, the unmodified reference
     sources) for greedy generation and per-step logits,
  3. re-runs the C restatement (oracle/build/liboracle.so) and requires
     bit-identical tokens and logits,
  4. stores tokens, logit digests, top-2 margins and selected logit rows.

The fixtures are data only (inputs and expected outputs); no reference source
is copied.

    python tests/golden/make_golden.py [case ...]
"""
from __future__ import annotations

import hashlib
import json
import sys
import tempfile
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

import mmr  # noqa: E402  (writes the synthetic model files)
import oracle  # noqa: E402

GOLDEN = Path(__file__).resolve().parent

MINIMIND2 = dict(hidden_size=768, num_hidden_layers=16, num_attention_heads=8, num_key_value_heads=2, head_dim=96,
                 intermediate_size=2048, vocab_size=6400, max_position_embeddings=32768, rms_norm_eps=1e-5,
                 rope_theta=1e6, tie_word_embeddings=1)
MINIMIND2_SMALL = dict(hidden_size=512, num_hidden_layers=8, num_attention_heads=8, num_key_value_heads=2,
                       head_dim=64, intermediate_size=1408, vocab_size=6400, max_position_embeddings=32768,
                       rms_norm_eps=1e-5, rope_theta=1e6, tie_word_embeddings=1)
# configs[2]'s attention shape (8 query / 2 KV heads, head_dim 96, theta 1e6)
# in a one-layer model, and a head_dim 128 variant: long-context decode cases
# the CPU path finishes in about a minute
ATTN96 = dict(hidden_size=768, num_hidden_layers=1, num_attention_heads=8, num_key_value_heads=2, head_dim=96,
              intermediate_size=512, vocab_size=512, max_position_embeddings=16384, rms_norm_eps=1e-5,
              rope_theta=1e6, tie_word_embeddings=0)
ATTN128 = dict(hidden_size=1024, num_hidden_layers=1, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
               intermediate_size=512, vocab_size=512, max_position_embeddings=16384, rms_norm_eps=1e-5,
               rope_theta=1e6, tie_word_embeddings=0)
MINI = dict(hidden_size=256, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
            intermediate_size=512, vocab_size=512, max_position_embeddings=4096, rms_norm_eps=1e-5, rope_theta=1e4,
            tie_word_embeddings=0)

CASES = {
    # small untied model, every step's logits: quick GPU parity
    "mini": dict(config=MINI, seed=7, round_fp16=True, prompt_seed=3, prompt_len=7, max_new=24,
                 logit_steps=list(range(24)), hash_weights=True),
    # same weights, config file without rms_norm_eps / rope_theta, run through the
    # reference's own loader (load_runtime_language_model): pins the file formats
    "mini_loader": dict(config=MINI, seed=7, round_fp16=True, prompt_seed=3, prompt_len=7, max_new=12,
                        logit_steps=[], loader=True, strip_keys=("rms_norm_eps", "rope_theta")),
    # MiniMind2-small, fp32 weights, 5-token prompt, 16 tokens
    "cfg0": dict(config=MINIMIND2_SMALL, seed=0, round_fp16=False, prompt_seed=1, prompt_len=5, max_new=16,
                 logit_steps=[0, 15], hash_weights=True),
    # MiniMind2 with fp16-representable weights, short prompt (fast GPU parity)
    "cfg3_short": dict(config=MINIMIND2, seed=0, round_fp16=True, prompt_seed=1, prompt_len=8, max_new=32,
                       logit_steps=[0, 31]),
    # 512-token prompt, 256 greedy steps
    "cfg3": dict(config=MINIMIND2, seed=0, round_fp16=True, prompt_seed=1, prompt_len=512, max_new=256,
                 logit_steps=[0, 64, 128, 192, 255]),
    # BASELINE configs[4], sequence 0 of the batch: MiniMind2, 256-token prompt
    # (seed 1000 + sequence index), greedy to a 4096-token context with no EOS
    # stop (the batched step decodes a fixed number of steps)
    "cfg4_seq0": dict(config=MINIMIND2, seed=0, round_fp16=True, prompt_seed=1000, prompt_len=256, max_new=3840,
                      logit_steps=[0, 1280, 2560, 3839], stream=True),
    # decode steps whose context crosses 4096 and 8192 keys (d 96) and 2048 keys
    # (d 128): the split attention with the fused q/k postprocess and the
    # separate combine kernel
    "long4k": dict(config=ATTN96, seed=21, round_fp16=True, prompt_seed=22, prompt_len=4090, max_new=16,
                   logit_steps=list(range(16)), stream=True),
    "long8k": dict(config=ATTN96, seed=21, round_fp16=True, prompt_seed=23, prompt_len=8185, max_new=16,
                   logit_steps=list(range(16)), stream=True),
    "long_d128": dict(config=ATTN128, seed=24, round_fp16=True, prompt_seed=25, prompt_len=2040, max_new=16,
                      logit_steps=list(range(16)), stream=True),
}


def sha256_file(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 22), b""):
            h.update(chunk)
    return h.hexdigest()


def oracle_replay(model_dir: Path, prompt, max_new: int, steps, stop_at_eos: bool = True):
    """C restatement, step by step: greedy tokens with generate's EOS rule
    (language_model.cpp:389-395) unless stop_at_eos is False, and the logits
    rows at `steps`."""
    m = oracle.OracleModel(model_dir)
    eos = int(m.config.eos_token_id)
    st = m.new_state()
    lg = None
    for t in prompt:
        lg = st.forward_token(int(t))
    ids, rows = [], []
    for i in range(max_new):
        nxt = oracle.argmax(lg)
        ids.append(nxt)
        if i in steps:
            rows.append(lg.copy())
        if (stop_at_eos and nxt == eos) or i + 1 == max_new:
            break
        lg = st.forward_token(nxt)
    return ids, np.array(rows, np.float32).reshape(len(rows), m.vocab)


def make_case(name: str, spec: dict, workdir: Path) -> dict:
    cfg = mmr.make_config(**spec["config"])
    model_dir = workdir / name
    mmr.write_synthetic_model(model_dir, cfg, spec["seed"], 0.02, spec["round_fp16"])
    if spec.get("strip_keys"):
        cfg_path = model_dir / "minimind_runtime_config.txt"
        lines = [l for l in cfg_path.read_text().splitlines() if l.split("=")[0] not in spec["strip_keys"]]
        cfg_path.write_text("\n".join(lines) + "\n")
    prompt = mmr.synthesize_prompt(spec["prompt_seed"], spec["prompt_len"], spec["config"]["vocab_size"]).tolist()
    t0 = time.time()
    steps = spec["logit_steps"]
    if spec.get("loader"):
        ref = oracle.ref_run("loader", model_dir, prompt, spec["max_new"])
        logits = np.zeros((0, spec["config"]["vocab_size"]), np.float32)
        ora = oracle.OracleModel(model_dir).generate(prompt, spec["max_new"])
        if ora != ref["generated"]:
            raise SystemExit(f"{name}: restatement tokens differ from the reference loader run")
    else:
        lpath = workdir / f"{name}_logits.bin"
        mode = "stream" if spec.get("stream") else "generate"
        with ThreadPoolExecutor(1) as ex:  # reference process and restatement run concurrently
            fut_ref = ex.submit(oracle.ref_run, mode, model_dir, prompt, spec["max_new"], lpath, steps)
            ora_ids, ora_rows = oracle_replay(model_dir, prompt, spec["max_new"], steps,
                                              stop_at_eos=not spec.get("stream"))
            ref = fut_ref.result()
        logits = np.fromfile(lpath, np.float32).reshape(len(steps), spec["config"]["vocab_size"])
        if mode == "generate" and ref["generated"] != ref["replay"]:
            raise SystemExit(f"{name}: reference generate and forward_token replay disagree")
        if ora_ids != ref["generated"]:
            raise SystemExit(f"{name}: restatement tokens differ from the reference build")
        if not np.array_equal(ora_rows, logits):
            raise SystemExit(f"{name}: restatement logits are not bit-identical to the reference build")
    elapsed = time.time() - t0
    out = {
        "case": name,
        "config": spec["config"],
        "seed": spec["seed"],
        "std": 0.02,
        "round_fp16": spec["round_fp16"],
        "prompt_seed": spec["prompt_seed"],
        "prompt": prompt,
        "max_new": spec["max_new"],
        "generated": ref["generated"],
        "stop_at_eos": not spec.get("stream"),
        "margin": ref.get("margin", []),
        "runner_up": ref.get("runner_up", []),
        "logit_sum": ref.get("logit_sum", []),
        "logit_sumsq": ref.get("logit_sumsq", []),
        "logit_steps": steps,
        "eps_used": ref["eps"],
        "strip_keys": list(spec.get("strip_keys", ())),
        "source": "oracle/_ref/ref_driver (reference CPU path), cross-checked bit-exact against oracle/cpu_ref.c",
        "reference_seconds": round(elapsed, 2),
    }
    if spec.get("hash_weights"):
        out["weights_sha256"] = sha256_file(model_dir / "weights.bin")
    (GOLDEN / f"{name}.json").write_text(json.dumps(out, indent=1) + "\n")
    if len(steps):
        np.save(GOLDEN / f"{name}_logits.npy", logits)
    print(f"[golden] {name}: {len(ref['generated'])} tokens, min margin "
          f"{min(out['margin']) if out['margin'] else float('nan'):.4g}, {elapsed:.1f}s", flush=True)
    return out


def main(argv) -> int:
    if not oracle.ref_available():
        oracle.build()
    if not oracle.ref_available():
        print("oracle/_ref/ref_driver is not built (needs /root/reference)", file=sys.stderr)
        return 1
    names = argv or list(CASES)
    with tempfile.TemporaryDirectory() as tmp:
        for n in names:
            make_case(n, CASES[n], Path(tmp))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
