#!/usr/bin/env python3
"""Decode throughput of the MiniMind2 gfx950 runtime.

    python bench.py [--gpus 1] [--steps 256] [--warmup 1] [--kv f16|f32] [--no-other-kv] [--no-cpu-baseline]
                    [--no-graph] [--copy-probe-mib 256] [--no-gemv-sweep] [--no-attention-sweep]
                    [--no-context-sweep] [--batch 32] [--batch-context 4096] [--kernel-reps 320]
    python bench.py --traffic-probe N [--traffic-kernel layer|attention|gate_up]   (counter-run workload)
    python bench.py [--no-graph] --context-probe T | --sweep-probe | --batch-probe  (kernel-trace workloads)

Workload: MiniMind2 dense (hidden 768, 16 layers, 8/2 heads, d 96, FFN 2048,
vocab 6400), fp16 weights drawn N(0, 0.02) from seed 0, a 512-token uniform
prompt from seed 1, then `--steps` greedy decode steps replayed from the
captured hipGraph with the token fed forward on the device.  The KV cache is
fp16 by default, as the reference's device cache (CustomAttentionCache,
ascend_custom_ops.cpp:59-65,126-139); `other_kv_cache` records the same decode
with the other dtype (fp32, the reference CPU path's).  A "step" is one
decode step (one token); `value` is decode tok/s = steps / time of the steps,
measured with HIP events on the decode stream between two device syncs.

The same line carries
  * roofline: the kernel with the largest share of the step (decode
    attention at 768 keys, KERNEL_CONTEXT; the other step kernels under
    `secondary`) launched alone `--kernel-reps` times over the 16 layers as
    one hipGraph chain (eager launches with --no-graph), timed with HIP events
    on the stream it runs on; achieved = algorithmic bytes / average time per
    launch;
  * kernels: the same measurement for every kernel of the step;
  * gemv_sweep / attention_sweep: BASELINE configs[1] GEMV shapes and
    configs[2] attention contexts alone through the C ABI, MALL-resident and
    HBM-streaming;
  * decode_context_sweep: the whole decode step at the configs[2] context
    lengths (1024 / 4096 / 8192 tokens);
  * batched: BASELINE configs[4], 32 sequences with 256-token prompts decoded
    in lockstep to 4096 positions over a paged fp16 KV cache (aggregate tok/s,
    p50 / p90 step latency);
  * launch_floor: per-kernel time of a hipGraph chain of 80 trivial kernels
    (empty, and one dependent load + store), the latency every kernel of the
    82-kernel step pays before it moves a byte;
  * copy_probe: a device-to-device copy of --copy-probe-mib MiB (HIP's blit
    kernel), the achievable-bandwidth yardstick and the calibration dispatch
    of the FETCH_SIZE / WRITE_SIZE counter runs;
  * roofline.traffic: L2-to-memory bytes per launch of each step kernel at
    the same 768 keys, from the committed counter summary TRAFFIC_FILE
    (written from `bench.py --traffic-probe 48 --traffic-kernel layer` runs),
    null when that file is absent;
  * cpu_baseline: the reference's own CPU path (oracle/_ref/ref_driver, built
    from the unmodified reference sources) on a bounded sample on this host.

--no-graph launches the step kernels one by one instead of replaying the
hipGraph (same kernels); rocprofv3's kernel tracing needs it.
"""
from __future__ import annotations

import argparse
import json
import os
import re
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


KERNEL_LABELS = {
    "qkv": "gemv qkv (1152x768 fp16, RMSNorm prologue)",
    "attention": "decode attention (q/k norm + RoPE + KV append + split partials, 8/2 heads, d 96, fp16 KV)",
    "o": "gemv o (768x768 fp16, split combine prologue, residual epilogue)",
    "gate_up": "gemv gate_up+SwiGLU (4096x768 fp16, RMSNorm prologue)",
    "down": "gemv down (768x2048 fp16, residual epilogue)",
    "lm_head": "gemv lm_head (6400x768 fp16, final RMSNorm prologue, argmax partials)",
    "finalize": "argmax finalize",
}
# Committed FETCH_SIZE / WRITE_SIZE summary of every step kernel (from
# `bench.py --traffic-probe N --traffic-kernel layer` at KERNEL_CONTEXT keys):
# one `traffic_bytes_per_launch[<kernel>]: <bytes>` line per kernel.
TRAFFIC_FILE = "profiles/decode_step_kernels_minimind2_768keys_traffic.md"

# Context of the per-kernel timings, the roofline and the counter probes: the
# end of configs[3]'s decode (512-token prompt + 256 steps), whatever --steps.
KERNEL_CONTEXT = PROMPT_LEN + 256

GEMV_SHAPES = [("qkv", 1152, 768), ("o", 768, 768), ("gate_up", 4096, 768), ("down", 768, 2048),
               ("lm_head_argmax", 6400, 768)]


def timed_chain(mmr, stream, ev, reps: int, launch, graph: bool) -> float:
    """Mean us per launch of launch(0) .. launch(reps - 1): replayed as one
    hipGraph chain (graph=True; host launch cost never paces them), or
    launched one by one between the events (graph=False, what rocprofv3's
    kernel trace can follow)."""
    if graph:
        with mmr.Graph(stream) as g:
            for i in range(reps):
                launch(i)
        g.launch()
        ev[0].record(stream)
        g.launch()
        ev[1].record(stream)
        stream.synchronize()
        g.free()
    else:
        ev[0].record(stream)
        for i in range(reps):
            launch(i)
        ev[1].record(stream)
        stream.synchronize()
    return ev[0].elapsed_ms(ev[1]) * 1e3 / reps


def gemv_sweep(mmr, stream, ev, reps: int = 256, graph: bool = True, labels=("mall", "hbm")) -> dict:
    """BASELINE configs[1] shapes with its input format (x fp16 [K] ~ N(0,1))
    through the C ABI (mmr_matvec_f16x and mmr_matvec_argmax_f16x), each timed
    over rotated weight copies: `mall` keeps the rotation at <= 160 MiB
    (resident in the 256 MB Infinity Cache), `hbm` at >= 640 MiB (every launch
    streams from HBM).  GB/s = algorithmic bytes (W fp16 + x fp16 + y fp32, or
    the int32 token for argmax: the per-shape bytes of the configs[1] table) /
    mean launch time of `reps` launches replayed as one hipGraph chain (eager
    launches with graph=False: a host-paced rate, for the kernel trace)."""
    lib = mmr.lib()
    out = {}
    rng = np.random.default_rng(7)
    for name, n, k in GEMV_SHAPES:
        x = mmr.DeviceArray.from_numpy(rng.standard_normal(k).astype(np.float16).view(np.uint16))
        y = mmr.DeviceArray(n, np.float32)
        tok = mmr.DeviceArray(1, np.int32)
        ws_bytes = mmr.matvec_argmax_workspace_size(n, k)
        ws = mmr.DeviceArray(max(ws_bytes, 1), np.uint8)
        wbytes = n * k * 2
        argmax = name.endswith("argmax")
        alg = wbytes + k * 2 + (4 if argmax else n * 4)
        res = {"rows": n, "cols": k, "bytes": alg}
        for label, budget in [b for b in (("mall", 160 << 20), ("hbm", 640 << 20)) if b[0] in labels]:
            copies = max(2, budget // wbytes) if label == "mall" else max(2, -(-budget // wbytes))
            big = mmr.DeviceArray(copies * wbytes, np.uint8, zero=True)

            def launch(i):
                w = big.ptr + (i % copies) * wbytes
                if argmax:
                    mmr.check(lib.mmr_matvec_argmax_f16x(w, n, k, x.ptr, None, tok.ptr, ws.ptr, ws_bytes,
                                                         stream.handle))
                else:
                    mmr.check(lib.mmr_matvec_f16x(w, n, k, x.ptr, None, y.ptr, stream.handle))

            for i in range(copies):
                launch(i)
            us = timed_chain(mmr, stream, ev, reps, launch, graph)
            res[label] = {"avg_us": round(us, 3), "gbs": round(alg / (us * 1e-6) / 1e9, 1),
                          "rotation_mib": round(copies * wbytes / 2**20, 1)}
            big.free()
        log(f"gemv {name:15s} {n}x{k}: " + " | ".join(f"{lb} {res[lb]['avg_us']:.3f} us {res[lb]['gbs']:.0f} GB/s"
                                                      for lb in labels))
        out[name] = res
    return out


ATTN_CONTEXTS = (128, 1024, 4096, 8192)


def attention_sweep(mmr, stream, ev, reps: int = 200, graph: bool = True) -> dict:
    """decode attention over T cached tokens plus the new
    one (T + 1 keys), 8 q / 2 kv heads, d 96, fp16 K/V ~ N(0, 1), through the
    C ABI (mmr_attention_from_cache: attention kernel + log-sum-exp combine, split
    count chosen by the library).  `resident`: every launch reads the same
    cache (MALL/L2-resident after the first); `hbm` (T >= 4096): launches
    rotate over caches totalling >= 640 MiB.  GB/s = algorithmic bytes
    (K + V of T + 1 tokens, fp32 q in and out) / mean time per call of `reps`
    calls replayed as one hipGraph chain."""
    hq, hkv, d = 8, 2, 96
    rng = np.random.default_rng(11)
    q = mmr.DeviceArray.from_numpy(rng.standard_normal(hq * d).astype(np.float32))
    o = mmr.DeviceArray(hq * d, np.float32)
    ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, 0), np.uint8)
    out = {}
    for T in ATTN_CONTEXTS:
        n = T + 1
        alg = 2 * hkv * d * 2 * n + 2 * hq * d * 4
        caches = [mmr.KvCache(hkv, d, n, mmr.KV_F16)]
        rows = caches[0].rows
        caches[0].upload(rng.standard_normal((hkv, rows, d)).astype(np.float16),
                         rng.standard_normal((hkv, rows, d)).astype(np.float16))
        res = {"keys": n, "bytes": alg}
        labels = [("resident", 1)]
        if T >= 4096:
            labels.append(("hbm", -(-(640 << 20) // (2 * hkv * rows * d * 2))))
        for label, copies in labels:
            while len(caches) < copies:
                caches.append(mmr.KvCache(hkv, d, n, mmr.KV_F16))  # zero-filled
            for i in range(copies):
                mmr.attention_from_cache(q, caches[i], n, hq, hkv, d, o, ws, stream=stream)
            us = timed_chain(mmr, stream, ev, reps,
                             lambda i: mmr.attention_from_cache(q, caches[i % copies], n, hq, hkv, d, o, ws,
                                                                stream=stream), graph)
            res[label] = {"avg_us": round(us, 3), "gbs": round(alg / (us * 1e-6) / 1e9, 1),
                          "frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "caches": copies}
        log(f"attention T={T}: " + " | ".join(f"{k} {res[k]['avg_us']:.2f} us {res[k]['gbs']:.0f} GB/s"
                                              for k, _ in labels))
        out[str(T)] = res
        del caches
    return out


DECODE_CONTEXTS = (1024, 4096, 8192)


def other_kv_decode(mmr, model, prompt, steps: int, kv_name: str) -> dict:
    """The same decode with the other KV cache dtype (one warm and one timed
    run): the value line uses --kv, this records the alternative's rate and
    whether its tokens also equal the reference CPU path's."""
    kv = mmr.KV_F16 if kv_name == "f16" else mmr.KV_F32
    st = model.make_state(PROMPT_LEN + steps + 8, kv)
    ev = [mmr.Event() for _ in range(2)]
    for _ in range(2):
        st.reset()
        st.enqueue_prefill(prompt)
        ev[0].record(st.stream)
        st.enqueue_decode(steps)
        ev[1].record(st.stream)
        st.synchronize()
    ms = ev[0].elapsed_ms(ev[1])
    generated = st.read_sequence(PROMPT_LEN, steps + 1).tolist()
    golden = ROOT / "tests" / "golden" / "cfg3.json"
    match = None
    if golden.exists():
        ref = json.loads(golden.read_text())["generated"]
        n = min(len(ref), len(generated))
        match = bool(generated[:n] == ref[:n])
    st.free()
    log(f"decode with {kv_name} KV: {steps / (ms / 1e3):.1f} tok/s, tokens match reference: {match}")
    return {"kv_cache": kv_name, "tok_s": round(steps / (ms / 1e3), 1), "ms_per_step": round(ms / steps, 5),
            "tokens_match_reference": match}


def decode_context_sweep(mmr, model, kv, steps: int = 64) -> dict:
    """The batch-1 decode step at the configs[2] context lengths: a prompt of T
    uniform tokens (chunked GEMM prefill), 8 warm steps, then `steps` timed
    hipGraph-replayed steps (HIP events on the decode stream)."""
    rng = np.random.default_rng(12)
    out = {}
    for T in DECODE_CONTEXTS:
        prompt = [int(t) for t in rng.integers(0, MINIMIND2["vocab_size"], T)]
        st = model.make_state(T + steps + 16, kv)
        st.enqueue_prefill(prompt)
        st.enqueue_decode(8)
        st.synchronize()
        ev = [mmr.Event() for _ in range(2)]
        ev[0].record(st.stream)
        st.enqueue_decode(steps)
        ev[1].record(st.stream)
        st.synchronize()
        ms = ev[0].elapsed_ms(ev[1])
        out[str(T)] = {"us_per_step": round(ms * 1e3 / steps, 1), "tok_s": round(steps / (ms * 1e-3), 1)}
        log(f"decode at context {T}: {out[str(T)]['us_per_step']} us/step, {out[str(T)]['tok_s']} tok/s")
        del st
    return out


def context_probe(mmr, context: int, steps: int, kv) -> int:
    """Workload of the long-context kernel-trace profiles: MiniMind2 with the
    bench's synthetic weights, a uniform prompt of `context` tokens (chunked
    GEMM prefill), then `steps` decode steps.  With --no-graph every step's
    kernels are launched one by one, which is what rocprofv3's kernel trace
    can follow on this image."""
    cfg = mmr.make_config(**MINIMIND2)
    model = mmr.Model.synthetic(cfg, 0, 0.02, True)
    prompt = mmr.synthesize_prompt(1, context, MINIMIND2["vocab_size"]).tolist()
    st = model.make_state(context + steps + 8, kv)
    st.enqueue_prefill(prompt)
    st.synchronize()
    ev = [mmr.Event() for _ in range(2)]
    ev[0].record(st.stream)
    st.enqueue_decode(steps)
    ev[1].record(st.stream)
    st.synchronize()
    ms = ev[0].elapsed_ms(ev[1])
    print(json.dumps({"context_probe": {"context": context, "steps": steps, "us_per_step": round(ms * 1e3 / steps, 1),
                                        "launch_mode": "eager" if os.environ.get("MMR_NO_GRAPH") else "hipGraph"}}),
          flush=True)
    return 0


def traffic_probe(mmr, launches: int, copy_mib: int, kernel: str) -> int:
    """Workload of the FETCH_SIZE / WRITE_SIZE counter runs: one kernel of the
    decode step launched alone, eagerly (rocprofv3's counter collection is
    run on eager dispatches only), then one device-to-device copy of
    `copy_mib` MiB, the calibration dispatch whose bytes are known.

    gate_up: the GEMV (4096 x 768 fp16, RMSNorm prologue, SwiGLU epilogue, the
    step's launch plan: 32-lane groups, two rows per group) through the C ABI
    over a 16-copy weight rotation like the 16 layers of the step.
    attention: the decode step's attention kernel (q/k norm + RoPE + KV append
    + split partials, attention_head_kernel at 768 keys, 12 splits, fp16 KV)
    through mmr_decode_attention_fused, cycling over 16 caches like the 16
    layers of a step."""
    H, F, layers = MINIMIND2["hidden_size"], MINIMIND2["intermediate_size"], MINIMIND2["num_hidden_layers"]
    rng = np.random.default_rng(3)
    if kernel == "layer":
        # Every kernel of the decode step's layers as the step launches them,
        # through mmr_decoder_layer_forward (qkv GEMV + RMSNorm, fused
        # attention at KERNEL_CONTEXT keys over an fp16 cache with 12 splits,
        # O GEMV with the split-combine prologue + residual, gate_up + SwiGLU,
        # down + residual: the step's launch plans) over the 16 layers of a
        # MiniMind2 model, one layer per call; then the lm_head GEMV with the
        # final RMSNorm and argmax partials (+ finalize), 16 times.  The step's
        # attention launch also carries L2-warming blocks; this one does not.
        cfg = mmr.make_config(**MINIMIND2)
        model = mmr.Model.synthetic(cfg, 0, 0.02, True)
        hkv, d, V = MINIMIND2["num_key_value_heads"], MINIMIND2["head_dim"], MINIMIND2["vocab_size"]
        n_keys = KERNEL_CONTEXT
        splits = 12  # the decode step's split count at 768 keys (12 tiles of 64)
        views = [mmr.LayerWeights.of_model(model, l) for l in range(layers)]
        caches = []
        for _ in range(layers):
            c = mmr.KvCache(hkv, d, n_keys, mmr.KV_F16)
            c.upload(rng.standard_normal((hkv, n_keys, d)).astype(np.float16),
                     rng.standard_normal((hkv, n_keys, d)).astype(np.float16))
            caches.append(c)
        x = mmr.DeviceArray.from_numpy(rng.standard_normal(H).astype(np.float32))
        y = mmr.DeviceArray(H, np.float32)
        pos = mmr.DeviceArray.from_numpy(np.array([n_keys - 1], np.int32))
        err = mmr.DeviceArray(1, np.int32, zero=True)
        ws = mmr.DeviceArray(views[0].workspace_size(splits), np.uint8)
        lm = mmr.DeviceArray.from_numpy(
            (rng.standard_normal((V, H)) * 0.02).astype(np.float16).reshape(-1).view(np.uint16))
        fnorm = mmr.DeviceArray.from_numpy(np.ones(H, np.float32))
        tok = mmr.DeviceArray(1, np.int32)
        lws = mmr.DeviceArray(mmr.matvec_argmax_workspace_size(V, H), np.uint8)
        stream = mmr.Stream()
        for i in range(launches):
            views[i % layers].forward(caches[i % layers], x, pos, y, ws, splits, err, stream=stream)
        for i in range(layers):
            mmr.matvec_argmax_f16(lm, V, H, y, tok, lws, norm_w=fnorm, eps=MINIMIND2["rms_norm_eps"], stream=stream)
        stream.synchronize()
        assert int(err.numpy()[0]) == 0
        alg = {name: kernel_bytes(MINIMIND2, name, n_keys, 2) for name in ("qkv", "attention", "o", "gate_up", "down",
                                                                          "lm_head")}
    elif kernel == "prefill":
        # One 512-token chunked prefill of MiniMind2 (the configs[3] prompt):
        # the GEMMs, attention, q/k rows and residual + norm kernels of 16
        # layers once each, then the head.
        cfg = mmr.make_config(**MINIMIND2)
        model = mmr.Model.synthetic(cfg, 0, 0.02, True)
        st = model.make_state(PROMPT_LEN + 8, mmr.KV_F16)
        st.enqueue_prefill(mmr.synthesize_prompt(1, PROMPT_LEN, MINIMIND2["vocab_size"]).tolist())
        st.synchronize()
        stream = mmr.Stream(st.stream)
        H, Fi, V = MINIMIND2["hidden_size"], MINIMIND2["intermediate_size"], MINIMIND2["vocab_size"]
        qkv_rows = (MINIMIND2["num_attention_heads"] + 2 * MINIMIND2["num_key_value_heads"]) * MINIMIND2["head_dim"]
        alg = {"qkv_w": qkv_rows * H * 2, "o_w": H * H * 2, "gate_up_w": 2 * Fi * H * 2, "down_w": H * Fi * 2,
               "note": "weight bytes per launch; activations per launch are listed in the profile"}
    elif kernel == "batch":
        # configs[4]'s batch of 32 sequences, one prompt token each, then 3
        # decode steps: the batched step's split-K GEMMs (M = 32), paged
        # attention and residual + norm kernels, 4 steps of 16 layers.
        cfg = mmr.make_config(**MINIMIND2)
        model = mmr.Model.synthetic(cfg, 0, 0.02, True)
        bs = model.make_batch_state(32, 64, mmr.KV_F16)
        bs.prefill([[1 + b] for b in range(32)])
        bs.decode(3)
        bs.synchronize()
        stream = mmr.Stream(bs.stream)
        H, Fi = MINIMIND2["hidden_size"], MINIMIND2["intermediate_size"]
        qkv_rows = (MINIMIND2["num_attention_heads"] + 2 * MINIMIND2["num_key_value_heads"]) * MINIMIND2["head_dim"]
        alg = {"qkv_w": qkv_rows * H * 2, "o_w": H * H * 2, "gate_up_w": 2 * Fi * H * 2, "down_w": H * Fi * 2,
               "lm_head_w": MINIMIND2["vocab_size"] * H * 2}
    elif kernel == "attention":
        hq, hkv, d = MINIMIND2["num_attention_heads"], MINIMIND2["num_key_value_heads"], MINIMIND2["head_dim"]
        n_keys = KERNEL_CONTEXT
        caches = []
        for _ in range(layers):
            c = mmr.KvCache(hkv, d, n_keys, mmr.KV_F16)
            c.upload(rng.standard_normal((hkv, c.rows, d)).astype(np.float16),
                     rng.standard_normal((hkv, c.rows, d)).astype(np.float16))
            caches.append(c)
        rope = mmr.RopeTable(n_keys, d, MINIMIND2["rope_theta"])
        qkv = mmr.DeviceArray.from_numpy(rng.standard_normal((hq + 2 * hkv) * d).astype(np.float32))
        ones = mmr.DeviceArray.from_numpy(np.ones(d, np.float32))
        pos = mmr.DeviceArray.from_numpy(np.array([n_keys - 1], np.int32))
        err = mmr.DeviceArray(1, np.int32, zero=True)
        splits = 12  # the decode step's split count at 768 keys (12 tiles of 64)
        ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, splits), np.uint8)
        out = mmr.DeviceArray(hq * d, np.float32)
        stream = mmr.Stream()
        for i in range(launches):
            mmr.decode_attention_fused(qkv, ones, ones, MINIMIND2["rms_norm_eps"], rope, pos, caches[i % layers], hq,
                                       hkv, d, out, ws, splits, err, stream=stream)
        stream.synchronize()
        alg = kernel_bytes(MINIMIND2, "attention", n_keys, 2)
    else:
        wbytes = 2 * F * H * 2
        w = mmr.DeviceArray(layers * wbytes, np.uint8, zero=True)
        x = mmr.DeviceArray.from_numpy(rng.standard_normal(H).astype(np.float32))
        g = mmr.DeviceArray.from_numpy(np.ones(H, np.float32))
        y = mmr.DeviceArray(F, np.float32)
        stream = mmr.Stream()
        lib = mmr.lib()
        for i in range(launches):
            mmr.check(lib.mmr_matvec_f16_ex(w.ptr + (i % layers) * wbytes, 2 * F, H, x.ptr, g.ptr, 1e-5,
                                            mmr.PRO_RMSNORM, mmr.EPI_SWIGLU, None, y.ptr, 32, 2, stream.handle))
        stream.synchronize()
        alg = kernel_bytes(MINIMIND2, "gate_up", 0, 0)
    n = copy_mib << 20
    src, dst = mmr.DeviceArray(n, np.uint8, zero=True), mmr.DeviceArray(n, np.uint8)
    dst.copy_from(src, stream)
    stream.synchronize()
    print(json.dumps({"traffic_probe": {"kernel": kernel, "launches": launches, "alg_bytes": alg,
                                        "copy_bytes": n}}), flush=True)
    return 0


def batched_decode(mmr, model, batch: int, prompt_len: int, context: int) -> dict:
    """`batch` independent sequences with random prompts of
    `prompt_len` tokens, decoded in lockstep to `context` positions over the
    paged fp16 KV cache.  Aggregate tok/s = batch * decode steps / decode time;
    per-step latency from an event after every step."""
    rng = np.random.default_rng(4)
    prompts = [[int(t) for t in rng.integers(0, MINIMIND2["vocab_size"], prompt_len)] for _ in range(batch)]
    bs = model.make_batch_state(batch, context, mmr.KV_F16)
    steps = context - prompt_len
    ev = [mmr.Event() for _ in range(steps + 2)]
    ev[0].record(bs.stream)
    bs.prefill(prompts)
    ev[1].record(bs.stream)
    for i in range(steps):
        bs.decode(1)
        ev[i + 2].record(bs.stream)
    bs.synchronize()
    step_ms = np.array([ev[i + 1].elapsed_ms(ev[i + 2]) for i in range(steps)])
    decode_ms = ev[1].elapsed_ms(ev[-1])
    out = {"batch": batch, "prompt_tokens": prompt_len, "context": context, "kv_cache": "f16 paged (64-token pages)",
           "prefill_ms": round(ev[0].elapsed_ms(ev[1]), 2), "prefill_mode": "batched decode steps over the prompts",
           "decode_steps": steps, "decode_ms": round(decode_ms, 2),
           "aggregate_tok_s": round(batch * steps / (decode_ms * 1e-3), 1),
           "p50_step_ms": round(float(np.median(step_ms)), 4), "p90_step_ms": round(float(np.percentile(step_ms, 90)), 4),
           "first_step_ms": round(float(step_ms[0]), 4), "last_step_ms": round(float(step_ms[-1]), 4)}
    log(f"batched decode B={batch} {prompt_len}->{context}: {out['aggregate_tok_s']} tok/s aggregate, "
        f"p50 step {out['p50_step_ms']} ms")
    bs.free()
    return out


def host_cpu() -> dict:
    """Host CPU model and the cores this process may use (the GPU box's share)."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count()
    return {"cpu_model": model, "cores_available": avail, "cores_online": os.cpu_count()}


def cpu_baseline(mmr, cfg, prompt, sample_steps: int, gpu_steps: int) -> dict | None:
    """The reference CPU path (oracle/_ref/ref_driver, the unmodified reference
    sources; single-threaded as shipped) at the GPU line's context: the same
    512-token prompt fed token by token (the reference's CPU prefill,
    language_model.cpp:339-341 needs Ascend), then `sample_steps` greedy decode
    steps timed as bench_decode.cpp:86-113 does, pinned to one core."""
    ref = ROOT / "oracle" / "_ref" / "ref_driver"
    if not ref.exists():
        log("oracle/_ref/ref_driver not built: cpu_baseline omitted")
        return None
    host = host_cpu()
    with tempfile.TemporaryDirectory() as tmp:
        mmr.write_synthetic_model(tmp, cfg, 0, 0.02, True)
        cmd = [str(ref), "bench", tmp, ",".join(str(int(t)) for t in prompt), str(sample_steps + 1)]
        try:
            cmd = ["taskset", "-c", str(sorted(os.sched_getaffinity(0))[0])] + cmd
        except (AttributeError, OSError):
            pass
        t0 = time.time()
        proc = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
        if proc.returncode != 0:
            log(f"ref_driver failed: {proc.stderr.strip()}")
            return None
        out = json.loads(proc.stdout)
        log(f"cpu baseline: {out['decode_tokens_per_second']:.2f} tok/s decode, prompt "
            f"{out['prefill_tokens'] / out['prefill_seconds']:.2f} tok/s ({time.time() - t0:.1f}s)")
    P, n = len(prompt), out["decode_steps"]
    return {
        "value": round(out["decode_tokens_per_second"], 3),
        "unit": "tok/s",
        "cores": 1,
        "cores_available": host["cores_available"],
        "cores_online": host["cores_online"],
        "cpu_model": host["cpu_model"],
        "kind": "reference",
        "prompt_tok_s": round(out["prefill_tokens"] / out["prefill_seconds"], 3),
        "sample": f"MiniMind2, the GPU line's weights and 512-token prompt, fed token by token "
                  f"({out['prefill_seconds']:.1f} s), then {n} greedy decode steps at positions {P}..{P + n} "
                  f"(the GPU line decodes {P}..{P + gpu_steps}); reference CPU path, one thread pinned to one core",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--kv", choices=["f32", "f16"], default="f16")
    ap.add_argument("--no-other-kv", action="store_true", help="skip the decode with the other KV cache dtype")
    ap.add_argument("--kernel-reps", type=int, default=320)
    ap.add_argument("--cpu-sample-steps", type=int, default=128)  # ~25 s of one core with the prompt
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=256)
    ap.add_argument("--no-gemv-sweep", action="store_true")
    ap.add_argument("--no-attention-sweep", action="store_true")
    ap.add_argument("--no-context-sweep", action="store_true")
    ap.add_argument("--batch", type=int, default=32, help="configs[4] batch size (0: skip the batched run)")
    ap.add_argument("--batch-context", type=int, default=4096)
    ap.add_argument("--traffic-probe", type=int, default=0, metavar="LAUNCHES",
                    help="run only the counter-run workload (kernel launches + one copy) and exit")
    ap.add_argument("--traffic-kernel", choices=["layer", "attention", "gate_up", "prefill", "batch"], default="layer")
    ap.add_argument("--context-probe", type=int, default=0, metavar="TOKENS",
                    help="run only a prefill of TOKENS prompt tokens + --context-probe-steps decode steps and exit")
    ap.add_argument("--context-probe-steps", type=int, default=24)
    ap.add_argument("--batch-probe", action="store_true",
                    help="run only the configs[4] batched decode (--batch, --batch-context), then exit")
    ap.add_argument("--sweep-probe", action="store_true",
                    help="run only the GEMV sweep (HBM rotation) and the attention sweep, then exit")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): batch-1 decode "
              f"of a 104M-parameter model has no cross-GPU work (it would shard by sequence: one weight replica "
              f"and its own requests per GPU, no collective on the decode path).",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.steps + PROMPT_LEN > MINIMIND2["max_position_embeddings"]:
        print("--steps out of range", file=sys.stderr)
        return 2

    if args.no_graph or args.traffic_probe > 0:
        os.environ["MMR_NO_GRAPH"] = "1"  # read when the decode state is created
    import mmr  # noqa: E402  (fails loudly if libmmr.so is not built)

    if args.traffic_probe > 0:
        return traffic_probe(mmr, args.traffic_probe, max(args.copy_probe_mib, 1), args.traffic_kernel)
    if args.sweep_probe:
        # configs[1] GEMV shapes over the HBM rotation and the configs[2]
        # attention op, launched one by one (the kernel-trace workload)
        stream = mmr.Stream()
        ev = [mmr.Event() for _ in range(2)]
        sweep = gemv_sweep(mmr, stream, ev, graph=not args.no_graph, labels=("hbm",))
        attn = attention_sweep(mmr, stream, ev, graph=not args.no_graph)
        print(json.dumps({"sweep_probe": {"launch_mode": "eager" if args.no_graph else "hipGraph",
                                          "gemv_sweep": sweep, "attention_sweep": attn}}), flush=True)
        return 0
    if args.batch_probe:
        # configs[4] alone: the batched leg of the default run (the kernel-trace workload with --no-graph)
        model = mmr.Model.synthetic(mmr.make_config(**MINIMIND2), 0, 0.02, True)
        res = batched_decode(mmr, model, max(args.batch, 1), 256, args.batch_context)
        print(json.dumps({"batch_probe": res, "launch_mode": "eager" if args.no_graph else "hipGraph"}), flush=True)
        return 0
    if args.context_probe > 0:
        return context_probe(mmr, args.context_probe, args.context_probe_steps,
                             mmr.KV_F16 if args.kv == "f16" else mmr.KV_F32)

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

    # Per-kernel timing: each kernel launched alone, cycling over the 16
    # layers, at KERNEL_CONTEXT keys (the context of configs[3]'s last step and
    # of the committed counter probes), whatever --steps.
    n_keys = KERNEL_CONTEXT
    kv_bytes = 2 if kv == mmr.KV_F16 else 4
    kernels = {}
    names = ["qkv", "attention", "o", "gate_up", "down", "lm_head", "finalize"]
    kstate = model.make_state(KERNEL_CONTEXT + 8, kv)
    kstate.enqueue_prefill(prompt)
    kstate.enqueue_decode(KERNEL_CONTEXT - PROMPT_LEN - 1)
    kstate.synchronize()
    for kid, name in enumerate(names):
        # kernel_reps launches as one hipGraph chain (eager with --no-graph),
        # timed with HIP events on the decode stream
        avg_us = kstate.time_step_kernel(kid, 0, args.kernel_reps)
        b = kernel_bytes(MINIMIND2, name, n_keys, kv_bytes)
        kernels[name] = {"avg_us": round(avg_us, 3), "bytes": b, "gbs": round(b / (avg_us * 1e-6) / 1e9, 1)}
        if name == "attention":
            kernels[name]["splits_note"] = ("attention kernel only (one block per query head and split at this "
                                            "context); the split combine runs in the o-projection prologue")
        log(f"kernel {name:9s} {avg_us:8.3f} us  {kernels[name]['gbs']:8.1f} GB/s")
    # The step's attention launch also carries L2-warming blocks that load
    # the layer's O, gate_up and down weights (bytes the next three kernels
    # then read from L2).  The same kernel without them, on a state made with
    # warming off at the same context:
    c = MINIMIND2
    warm_bytes = 2 * (c["hidden_size"] * c["num_attention_heads"] * c["head_dim"] +
                      3 * c["hidden_size"] * c["intermediate_size"])
    caller_warm = os.environ.get("MMR_L2_WARM_BLOCKS")
    os.environ["MMR_L2_WARM_BLOCKS"] = "0"
    cold = model.make_state(KERNEL_CONTEXT + 8, kv)
    if caller_warm is None:
        del os.environ["MMR_L2_WARM_BLOCKS"]
    else:
        os.environ["MMR_L2_WARM_BLOCKS"] = caller_warm  # the caller's setting holds for the later legs
    cold.enqueue_prefill(prompt)
    cold.enqueue_decode(KERNEL_CONTEXT - PROMPT_LEN - 1)
    cold.synchronize()
    a = kernels["attention"]
    a["avg_us_without_warm_blocks"] = round(cold.time_step_kernel(names.index("attention"), 0, args.kernel_reps), 3)
    a["warm_bytes_per_launch"] = warm_bytes
    a["warm_note"] = ("avg_us is the launch as the step runs it, with extra blocks on the idle CUs loading the layer's O, "
                      "gate_up and down weights into the L2s of the XCDs that read them next; "
                      "avg_us_without_warm_blocks is the attention work alone")
    log(f"kernel attention without warming blocks {a['avg_us_without_warm_blocks']:.3f} us")
    del cold, kstate
    per_step_us = sum(kernels[n]["avg_us"] for n in names[:5]) * MINIMIND2["num_hidden_layers"] + \
        kernels["lm_head"]["avg_us"] + kernels["finalize"]["avg_us"]
    step_bytes = sum(kernels[n]["bytes"] for n in names[:5]) * MINIMIND2["num_hidden_layers"] + \
        kernels["lm_head"]["bytes"]
    # The roofline kernel is the one with the largest share of the step:
    # time per launch x launches per step (16 for the layer kernels).
    per_step = {n: kernels[n]["avg_us"] * (MINIMIND2["num_hidden_layers"] if n in names[:5] else 1) for n in names}
    for n in names:
        kernels[n]["us_per_step"] = round(per_step[n], 2)
    dom = max(per_step, key=per_step.get)
    log(f"dominant kernel: {dom} ({per_step[dom]:.1f} us per step)")
    # The chain's per-kernel floor: trivial kernels replayed from a hipGraph.
    floor = {"kernels_in_chain": 80, "blocks": 256,
             "empty_us": round(mmr.launch_floor_us(80, 256, False, 20), 3),
             "load_store_us": round(mmr.launch_floor_us(80, 256, True, 20), 3)}
    log(f"launch floor: empty {floor['empty_us']:.3f} us, dependent load + store {floor['load_store_us']:.3f} us "
        f"per kernel (graph chain of 80)")

    copy_probe = None
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib << 20
        src, dst = mmr.DeviceArray(n, np.uint8, zero=True), mmr.DeviceArray(n, np.uint8)
        dst.copy_from(src, stream)  # warm
        reps = 4
        ev[0].record(stream)
        for _ in range(reps):
            dst.copy_from(src, stream)
        ev[1].record(stream)
        state.synchronize()
        ms = ev[0].elapsed_ms(ev[1]) / reps
        copy_probe = {"bytes_per_copy": n, "ms": round(ms, 4), "gbs": round(2 * n / (ms * 1e-3) / 1e9, 1),
                      "note": "read + write bytes / time of one device-to-device copy"}
        log(f"copy probe: {args.copy_probe_mib} MiB d2d in {ms:.3f} ms -> {copy_probe['gbs']} GB/s (read+write)")
        src.free()
        dst.free()

    # Prefill alone, repeated on the reset state (its decode results were read
    # above): the median of 8 runs, since one run varies by a few percent.
    pf = []
    for _ in range(8):
        state.reset()
        mmr.synchronize()
        ev[0].record(stream)
        state.enqueue_prefill(prompt)
        ev[1].record(stream)
        state.synchronize()
        pf.append(ev[0].elapsed_ms(ev[1]))
    prefill_tok_s = PROMPT_LEN / (float(np.median(pf)) / 1e3)
    log(f"prefill: median of 8 runs {np.median(pf):.3f} ms -> {prefill_tok_s:.1f} tok/s")

    sweep = None if args.no_gemv_sweep else gemv_sweep(mmr, mmr.Stream(stream), ev, graph=not args.no_graph)
    attn_sweep = None if args.no_attention_sweep else attention_sweep(mmr, mmr.Stream(stream), ev,
                                                                      graph=not args.no_graph)
    ctx_sweep = None if args.no_context_sweep else decode_context_sweep(mmr, model, kv)
    other_kv = None if args.no_other_kv else other_kv_decode(mmr, model, prompt, args.steps,
                                                             "f32" if args.kv == "f16" else "f16")
    batched = batched_decode(mmr, model, args.batch, 256, args.batch_context) if args.batch > 0 else None

    def roofline_of(name: str) -> dict:
        """HBM roofline entry of one step kernel; traffic (L2-to-memory bytes
        per launch) from its committed counter summary, null without one."""
        traffic, tsrc = None, TRAFFIC_FILE
        if (ROOT / tsrc).exists():
            m = re.search(r"traffic_bytes_per_launch\[" + name + r"\]:\s*(\d+)", (ROOT / tsrc).read_text())
            traffic = int(m.group(1)) if m else None
        ach = kernels[name]["gbs"]
        return {"bound": "hbm", "kernel": KERNEL_LABELS[name], "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": tsrc if traffic is not None else None,
                "traffic_over_algorithmic": round(traffic / kernels[name]["bytes"], 3) if traffic else None,
                "context_keys": KERNEL_CONTEXT,
                "bytes_per_launch": kernels[name]["bytes"], "avg_us": kernels[name]["avg_us"],
                "us_per_step": kernels[name]["us_per_step"],
                **{k: kernels[name][k] for k in ("avg_us_without_warm_blocks", "warm_bytes_per_launch")
                   if k in kernels[name]},
                **({"traffic_scope": "the attention work alone (the --traffic-probe launch has no warming blocks); "
                                     "the step's launch also fetches warm_bytes_per_launch"}
                   if traffic is not None and "warm_bytes_per_launch" in kernels[name] else {})}

    roofline = roofline_of(dom)
    roofline["secondary"] = {n: roofline_of(n) for n in names[:6] if n != dom}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(mmr, cfg, prompt, args.cpu_sample_steps, args.steps)

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
        "prefill_mode": "chunked batched kernels (fp16-MFMA GEMMs with hi/lo fp32 activations, fp16-MFMA causal "
                        "attention with hi/lo q and p for the fp16 KV cache), 512-token chunks",
        "tokens_match_reference": parity,
        "step_bytes": step_bytes,
        "step_gbs": round(step_bytes / (decode_ms / args.steps * 1e-3) / 1e9, 1),
        "sum_kernel_us_per_step": round(per_step_us, 2),
        "kernels": kernels,
        "copy_probe": copy_probe,
        "gemv_sweep": sweep,
        "attention_sweep": attn_sweep,
        "launch_floor": floor,
        "decode_context_sweep": ctx_sweep,
        "other_kv_cache": other_kv,
        "batched": batched,
        "launch_mode": "eager (--no-graph)" if args.no_graph else "hipGraph replay",
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
