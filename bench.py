#!/usr/bin/env python3
"""Decode throughput of the MiniMind2 gfx950 runtime.

    python bench.py [--gpus 1] [--steps 256] [--warmup 1] [--kv f32|f16] [--no-cpu-baseline]

Workload: MiniMind2 dense (hidden 768, 16 layers, 8/2 heads, d 96, FFN 2048,
vocab 6400), fp16 weights drawn N(0, 0.02) from seed 0, a 512-token uniform
prompt from seed 1, then `--steps` greedy decode steps replayed from the
captured hipGraph with the token fed forward on the device.  A "step" is one
decode step (one token); `value` is decode tok/s = steps / time of the steps,
measured with HIP events on the decode stream between two device syncs.

The same line carries
  * roofline: the dominant kernel (gate_up GEMV + SwiGLU) launched alone
    `--kernel-reps` times over the 16 layers' weights, timed with HIP events on
    the stream it runs on; achieved = algorithmic bytes / average duration;
  * kernels: the same measurement for every kernel of the step;
  * cpu_baseline: the reference's own CPU path (oracle/_ref/ref_driver, built
    from the unmodified reference sources) on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))

METRIC = "decode tok/s at batch 1 (MiniMind2, 1 GPU) + GEMV/attn HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
MINIMIND2 = dict(hidden_size=768, num_hidden_layers=16, num_attention_heads=8, num_key_value_heads=2, head_dim=96,
                 intermediate_size=2048, vocab_size=6400, max_position_embeddings=32768, rms_norm_eps=1e-5,
                 rope_theta=1e6, tie_word_embeddings=1)
PROMPT_LEN = 512


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_bytes(c: dict, kernel: str, n_keys: int, kv_bytes: int) -> int:
    """Algorithmic HBM bytes of one launch: weights read once, inputs read once,
    outputs written once (fp16 weights, fp32 activations)."""
    H, D, F, V = c["hidden_size"], c["head_dim"], c["intermediate_size"], c["vocab_size"]
    Hq, Hkv = c["num_attention_heads"], c["num_key_value_heads"]
    qkv_rows = (Hq + 2 * Hkv) * D
    if kernel == "qkv":      # W, h, norm gain, qkv out
        return qkv_rows * H * 2 + H * 4 + H * 4 + qkv_rows * 4
    if kernel == "attention":  # K/V of n_keys tokens, qkv in, new k/v append, out
        return 2 * Hkv * n_keys * D * kv_bytes + qkv_rows * 4 + 2 * Hkv * D * kv_bytes + Hq * D * 4
    if kernel == "o":        # W, attn in, residual read + write
        return H * Hq * D * 2 + Hq * D * 4 + 2 * H * 4
    if kernel == "gate_up":  # W (2F x H), h, norm gain, act out
        return 2 * F * H * 2 + H * 4 + H * 4 + F * 4
    if kernel == "down":     # W, act in, residual read + write
        return H * F * 2 + F * 4 + 2 * H * 4
    if kernel == "lm_head":  # W, h, norm gain, logits out (argmax partials are a few KB)
        return V * H * 2 + H * 4 + H * 4 + V * 4
    if kernel == "finalize":  # argmax partials in, token out
        return 0
    raise KeyError(kernel)


def cpu_baseline(mmr, cfg, prompt, sample_steps: int) -> dict | None:
    """The reference CPU path (single-threaded, as shipped) on a bounded sample."""
    ref = ROOT / "oracle" / "_ref" / "ref_driver"
    if not ref.exists():
        log("oracle/_ref/ref_driver not built: cpu_baseline omitted")
        return None
    with tempfile.TemporaryDirectory() as tmp:
        mmr.write_synthetic_model(tmp, cfg, 0, 0.02, True)
        short = [int(t) for t in prompt[:8]]
        cmd = [str(ref), "bench", tmp, ",".join(map(str, short)), str(sample_steps + 1)]
        try:
            cmd = ["taskset", "-c", str(sorted(os.sched_getaffinity(0))[0])] + cmd
        except (AttributeError, OSError):
            pass
        t0 = time.time()
        proc = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        if proc.returncode != 0:
            log(f"ref_driver failed: {proc.stderr.strip()}")
            return None
        out = json.loads(proc.stdout)
        log(f"cpu baseline: {out['decode_tokens_per_second']:.2f} tok/s ({time.time() - t0:.1f}s)")
    return {
        "value": round(out["decode_tokens_per_second"], 3),
        "unit": "tok/s",
        "cores": 1,
        "kind": "reference",
        "sample": f"MiniMind2 same weights, 8-token prompt fed token by token, then {out['decode_steps']} greedy "
                  f"decode steps (positions 8..{8 + out['decode_steps']}); reference CPU path, single thread",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--kv", choices=["f32", "f16"], default="f32")
    ap.add_argument("--kernel-reps", type=int, default=320)
    ap.add_argument("--cpu-sample-steps", type=int, default=48)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): batch-1 decode "
              f"of a 104M-parameter model has no cross-GPU work; see DESIGN.md for how it would shard.",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.steps + PROMPT_LEN > MINIMIND2["max_position_embeddings"]:
        print("--steps out of range", file=sys.stderr)
        return 2

    import mmr  # noqa: E402  (fails loudly if libmmr.so is not built)

    if mmr.device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        return 1
    cfg = mmr.make_config(**MINIMIND2)
    t0 = time.time()
    model = mmr.Model.synthetic(cfg, 0, 0.02, True)
    log(f"model ready ({model.weight_bytes() / 1e6:.1f} MB fp16 weights, {time.time() - t0:.1f}s)")
    prompt = mmr.synthesize_prompt(1, PROMPT_LEN, MINIMIND2["vocab_size"])
    kv = mmr.KV_F16 if args.kv == "f16" else mmr.KV_F32
    state = model.make_state(PROMPT_LEN + args.steps + 8, kv)
    stream = state.stream
    ev = [mmr.Event() for _ in range(4)]

    def run_once():
        state.reset()
        mmr.synchronize()
        ev[0].record(stream)
        state.enqueue_prefill(prompt)
        ev[1].record(stream)
        state.enqueue_decode(args.steps)
        ev[2].record(stream)
        state.synchronize()
        mmr.synchronize()
        return ev[0].elapsed_ms(ev[1]), ev[1].elapsed_ms(ev[2])

    for w in range(args.warmup):
        run_once()
        log(f"warmup {w + 1}/{args.warmup} done")
    prefill_ms, decode_ms = run_once()
    tok_s = args.steps / (decode_ms / 1e3)
    prefill_tok_s = PROMPT_LEN / (prefill_ms / 1e3)
    log(f"decode: {args.steps} steps in {decode_ms:.3f} ms -> {tok_s:.1f} tok/s; prefill {prefill_tok_s:.1f} tok/s")

    generated = state.read_sequence(PROMPT_LEN, args.steps + 1).tolist()
    parity = None
    golden = ROOT / "tests" / "golden" / "cfg3.json"
    if golden.exists():
        ref_tokens = json.loads(golden.read_text())["generated"]
        n = min(len(ref_tokens), len(generated))
        parity = bool(generated[:n] == ref_tokens[:n])
        log(f"tokens vs reference CPU path: {'identical' if parity else 'DIFFERENT'} over {n} tokens")

    # Per-kernel timing: each kernel launched alone, cycling over the 16 layers.
    n_keys = PROMPT_LEN + args.steps
    kv_bytes = 2 if kv == mmr.KV_F16 else 4
    kernels = {}
    names = ["qkv", "attention", "o", "gate_up", "down", "lm_head", "finalize"]
    state.reset()
    state.enqueue_prefill(prompt)
    state.enqueue_decode(args.steps - 1)
    state.synchronize()
    for kid, name in enumerate(names):
        state.launch_step_kernel(kid, 0, 32)  # warm
        mmr.synchronize()
        ev[0].record(stream)
        state.launch_step_kernel(kid, 0, args.kernel_reps)
        ev[1].record(stream)
        state.synchronize()
        avg_us = ev[0].elapsed_ms(ev[1]) * 1e3 / args.kernel_reps
        b = kernel_bytes(MINIMIND2, name, n_keys, kv_bytes)
        kernels[name] = {"avg_us": round(avg_us, 3), "bytes": b, "gbs": round(b / (avg_us * 1e-6) / 1e9, 1)}
        if name == "attention":
            kernels[name]["splits_note"] = "split kernel only; the combine runs in the o-projection prologue"
        log(f"kernel {name:9s} {avg_us:8.3f} us  {kernels[name]['gbs']:8.1f} GB/s")
    per_step_us = sum(kernels[n]["avg_us"] for n in names[:5]) * MINIMIND2["num_hidden_layers"] + \
        kernels["lm_head"]["avg_us"] + kernels["finalize"]["avg_us"]
    step_bytes = sum(kernels[n]["bytes"] for n in names[:5]) * MINIMIND2["num_hidden_layers"] + \
        kernels["lm_head"]["bytes"]
    dom = "gate_up"
    ach = kernels[dom]["gbs"]

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(mmr, cfg, prompt, args.cpu_sample_steps)

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(decode_ms / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (fp16 weights)" if kv == mmr.KV_F32 else "f32 (fp16 weights, fp16 KV)",
        "data": "synthetic: N(0,0.02) fp16 weights seed 0, uniform 512-token prompt seed 1",
        "config": {"workload": "configs[3] MiniMind2 dense batch-1 greedy decode after a 512-token prompt",
                   "prompt_tokens": PROMPT_LEN, "decode_steps": args.steps, "kv_cache": args.kv,
                   "parallelism": "single GPU"},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "prefill_mode": "token-by-token through the decode graph",
        "tokens_match_reference": parity,
        "step_bytes": step_bytes,
        "step_gbs": round(step_bytes / (decode_ms / args.steps * 1e-3) / 1e9, 1),
        "sum_kernel_us_per_step": round(per_step_us, 2),
        "kernels": kernels,
        "roofline": {"bound": "hbm", "kernel": "gemv gate_up+SwiGLU (4096x768 fp16, RMSNorm prologue)",
                     "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
