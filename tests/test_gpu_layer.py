"""GPU parity of the decoder-layer boundary (mmr_decoder_layer_forward, the
counterpart of run_dense_decoder_layer_device, decoder_layer.cpp:617-659, over
a LayerKvCache, decoder_layer.h:40-48) against the oracle's decoder layer
(oracle/cpu_ref.c orc_decoder_layer: the layer_step the model-level
bit-exact test pins to the reference build, decoder_layer.cpp:312-407).

Bar: layer outputs within max|d| / max|ref| <= 2e-3 (the observed error is
printed; fp16 weights are exact on both sides, the difference is summation
order); cached keys/values within 1e-5 relative (fp32 cache) or equal to the
oracle's rounded to fp16 (fp16 cache, 1 ulp allowed for keys).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from conftest import ROOT, load_golden, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3


def host_layer(model_dir, cfg_dict, layer):
    sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
    import export_minimind_runtime as ex
    cc = ex.CheckpointConfig(**{k: v for k, v in cfg_dict.items() if k in ex.CheckpointConfig.__dataclass_fields__})
    w = ex.read_runtime_weights(model_dir / "weights.bin", cc)
    p = f"model.layers.{layer}."
    names = {"input_norm": "input_layernorm.weight", "post_attention_norm": "post_attention_layernorm.weight",
             "q_norm": "self_attn.q_norm.weight", "k_norm": "self_attn.k_norm.weight",
             "q_proj": "self_attn.q_proj.weight", "k_proj": "self_attn.k_proj.weight",
             "v_proj": "self_attn.v_proj.weight", "o_proj": "self_attn.o_proj.weight",
             "gate_proj": "mlp.gate_proj.weight", "up_proj": "mlp.up_proj.weight", "down_proj": "mlp.down_proj.weight"}
    return {k: w[p + v] for k, v in names.items()}


@pytest.fixture(scope="module")
def mini(gpu, oracle, tmp_path_factory):
    mmr = gpu
    g = load_golden("mini")
    d = tmp_path_factory.mktemp("layer_mini")
    cfg = mmr.make_config(**g["config"])
    mmr.write_synthetic_model(d, cfg, g["seed"], g["std"], g["round_fp16"])
    return mmr, oracle, g, d, mmr.Model.load(d), oracle.OracleModel(d)


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("splits", [0, 32])
def test_decoder_layer_matches_oracle(mini, kv, splits):
    # splits 0: automatic (one per 64-token tile of the capacity: merged in the
    # O projection's prologue); 32: the separate combine kernel
    mmr, oracle, g, d, model, ref = mini
    print(f"[case] decoder layer kv={kv} splits={splits}", flush=True)
    c = g["config"]
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    layer, steps = 1, 140
    lw = mmr.LayerWeights.of_model(model, layer)
    kvd = mmr.KV_F16 if kv == "f16" else mmr.KV_F32
    cache = mmr.KvCache(Hkv, D, steps, kvd)
    n_split = splits or -(-steps // 64)
    ws = mmr.DeviceArray(lw.workspace_size(n_split), np.uint8)
    pos = mmr.DeviceArray(1, np.int32)
    err = mmr.DeviceArray(1, np.int32, zero=True)
    x, y = mmr.DeviceArray(H, np.float32), mmr.DeviceArray(H, np.float32)
    st = ref.new_state()
    rng = np.random.default_rng(5)
    worst = 0.0
    for p in range(steps):
        h = rng.standard_normal(H).astype(np.float32)
        x.upload(h)
        pos.upload(np.array([p], np.int32))
        lw.forward(cache, x, pos, y, ws, splits, err)
        want = st.decoder_layer(layer, h, p)
        e = rel_err(y.numpy(), want)
        worst = max(worst, e)
        assert e < TOL, (p, e)
    assert int(err.numpy()[0]) == 0
    print(f"[result] {steps} positions, worst layer-output error {worst:.2e}", flush=True)
    keys, values = cache.download()
    rk, rv = st.layer_cache(layer)  # [tokens][kv][d]
    rk, rv = rk.transpose(1, 0, 2), rv.transpose(1, 0, 2)
    gk, gv = keys[:, :steps].astype(np.float32), values[:, :steps].astype(np.float32)
    if kv == "f32":
        assert rel_err(gk, rk) < 1e-5 and rel_err(gv, rv) < 1e-5
    else:
        assert rel_err(gk, rk.astype(np.float16).astype(np.float32)) < 2e-3
        assert rel_err(gv, rv.astype(np.float16).astype(np.float32)) < 2e-3


def test_uploaded_layer_equals_model_view_and_captures(mini):
    # mmr_layer_weights_create from the host arrays of layer 0 gives the same
    # bits as the model's own layer; the call replays from a hipGraph with the
    # position advanced in device memory between replays
    mmr, oracle, g, d, model, ref = mini
    c = g["config"]
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    up = mmr.LayerWeights.create(model.config, **host_layer(d, c, 0))
    view = mmr.LayerWeights.of_model(model, 0)
    steps = 40
    stream = mmr.Stream()
    ca, cb = mmr.KvCache(Hkv, D, steps, mmr.KV_F16), mmr.KvCache(Hkv, D, steps, mmr.KV_F16)
    ws_a, ws_b = (mmr.DeviceArray(up.workspace_size(4), np.uint8) for _ in range(2))
    pos_a, pos_b = mmr.DeviceArray(1, np.int32), mmr.DeviceArray(1, np.int32)
    err = mmr.DeviceArray(1, np.int32, zero=True)
    xa, xb = mmr.DeviceArray(H, np.float32), mmr.DeviceArray(H, np.float32)
    ya, yb = mmr.DeviceArray(H, np.float32), mmr.DeviceArray(H, np.float32)
    with mmr.Graph(stream) as graph:
        view.forward(cb, xb, pos_b, yb, ws_b, 4, err, stream=stream)
    rng = np.random.default_rng(9)
    for p in range(steps):
        h = rng.standard_normal(H).astype(np.float32)
        xa.upload(h)
        xb.upload(h)
        pos_a.upload(np.array([p], np.int32))
        pos_b.upload(np.array([p], np.int32))
        up.forward(ca, xa, pos_a, ya, ws_a, 4, err, stream=stream)
        graph.launch()
        stream.synchronize()
        np.testing.assert_array_equal(ya.numpy(), yb.numpy())
    ka, va = ca.download()
    kb, vb = cb.download()
    np.testing.assert_array_equal(ka, kb)
    np.testing.assert_array_equal(va, vb)
    assert int(err.numpy()[0]) == 0


def test_decoder_layer_errors(mini):
    mmr, oracle, g, d, model, ref = mini
    c = g["config"]
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    lw = mmr.LayerWeights.of_model(model, 0)
    with pytest.raises(mmr.OutOfRange):
        mmr.LayerWeights.of_model(model, c["num_hidden_layers"])
    x, y = mmr.DeviceArray(H, np.float32), mmr.DeviceArray(H, np.float32)
    x.upload(np.ones(H, np.float32))
    pos = mmr.DeviceArray.from_numpy(np.array([8], np.int32))
    err = mmr.DeviceArray(1, np.int32, zero=True)
    ws = mmr.DeviceArray(lw.workspace_size(1), np.uint8)
    with pytest.raises(mmr.InvalidArgument, match="cache shape"):
        lw.forward(mmr.KvCache(Hkv, D * 2, 8), x, pos, y, ws, 1, err)
    with pytest.raises(mmr.InvalidArgument, match="workspace"):
        lw.forward(mmr.KvCache(Hkv, D, 8), x, pos, y, ws, 8, err)
    # position 8 in an 8-position cache: flagged by the kernel, nothing written
    small = mmr.KvCache(Hkv, D, 8)
    lw.forward(small, x, pos, y, ws, 1, err)
    mmr.synchronize()
    assert int(err.numpy()[0]) == 1
    bad = mmr.make_config(**{**c, "head_dim": 48})  # rejected before any array is read
    with pytest.raises(mmr.InvalidArgument, match="head_dim"):
        mmr.LayerWeights.create(bad, **{k: np.zeros(1, np.float32) for k in mmr.LayerWeights.NAMES})


@pytest.fixture(scope="module")
def mm2(gpu, oracle, tmp_path_factory):
    # MiniMind2 (BASELINE configs[3] shape): hidden 768, 8 / 2 heads of 96,
    # FFN 2048; the qkv GEMV's 2-row plan and the 16-split combine prologue
    mmr = gpu
    g = load_golden("cfg3")
    d = tmp_path_factory.mktemp("layer_mm2")
    mmr.write_synthetic_model(d, mmr.make_config(**g["config"]), g["seed"], g["std"], g["round_fp16"])
    return mmr, oracle, g, d, mmr.Model.load(d), oracle.OracleModel(d)


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("splits", [0, 16])
def test_minimind2_decoder_layer_in_place(mm2, kv, splits):
    # out aliasing hidden (include/mmr.h allows it): every residual GEMV reads
    # residual[row] before it stores y[row], so the in-place call gives the
    # same bits as the call with separate buffers; both match the oracle
    mmr, oracle, g, d, model, ref = mm2
    print(f"[case] MiniMind2 layer in place kv={kv} splits={splits}", flush=True)
    c = g["config"]
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    layer, steps = 5, 200
    lw = mmr.LayerWeights.of_model(model, layer)
    kvd = mmr.KV_F16 if kv == "f16" else mmr.KV_F32
    ca, cb = mmr.KvCache(Hkv, D, 4096, kvd, reserve=False), mmr.KvCache(Hkv, D, 4096, kvd, reserve=False)
    n_split = splits or 8  # automatic: one split per 64-token tile of the 512 backed rows
    ws_a, ws_b = (mmr.DeviceArray(lw.workspace_size(n_split), np.uint8) for _ in range(2))
    pos = mmr.DeviceArray(1, np.int32)
    err = mmr.DeviceArray(1, np.int32, zero=True)
    xa, xb, yb = (mmr.DeviceArray(H, np.float32) for _ in range(3))
    st = ref.new_state()
    rng = np.random.default_rng(15)
    worst = 0.0
    for p in range(steps):
        h = rng.standard_normal(H).astype(np.float32)
        xa.upload(h)
        xb.upload(h)
        pos.upload(np.array([p], np.int32))
        lw.forward(ca, xa, pos, xa, ws_a, splits, err)  # in place
        lw.forward(cb, xb, pos, yb, ws_b, splits, err)
        got = xa.numpy()
        np.testing.assert_array_equal(got, yb.numpy())
        e = rel_err(got, st.decoder_layer(layer, h, p))
        worst = max(worst, e)
        assert e < TOL, (p, e)
    assert int(err.numpy()[0]) == 0
    print(f"[result] {steps} positions, worst layer-output error {worst:.2e}", flush=True)
    np.testing.assert_array_equal(ca.download(steps)[0], cb.download(steps)[0])


_PREFILL_REF = {}


def prefill_reference(ref, layer, hs, start, h_next):
    """The oracle's layer applied position by position from an empty cache:
    row i at RoPE position start + i, cached at row i (the reference's
    prefill layer semantics, decoder_layer.cpp:409-527); then one decode
    step of h_next at position start + T on that cache."""
    key = (layer, hs.shape[0], start, float(hs[0, 0]))
    if key not in _PREFILL_REF:
        st = ref.new_state()
        outs = np.stack([st.decoder_layer(layer, hs[i], start + i) for i in range(hs.shape[0])])
        cache = st.layer_cache(layer)
        _PREFILL_REF[key] = (outs, cache, st.decoder_layer(layer, h_next, start + hs.shape[0]))
    return _PREFILL_REF[key]


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("T", [1, 17, 512])
def test_minimind2_prefill_layer_matches_oracle(mm2, kv, T):
    # mmr_prefill_layer_forward (run_dense_prefill_layer_device,
    # decoder_layer.cpp:661-734): T rows through one layer on the matrix cores
    mmr, oracle, g, d, model, ref = mm2
    print(f"[case] MiniMind2 prefill layer kv={kv} T={T}", flush=True)
    c = g["config"]
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    layer = 7
    lw = mmr.LayerWeights.of_model(model, layer)
    kvd = mmr.KV_F16 if kv == "f16" else mmr.KV_F32
    hs = np.random.default_rng(100 + T).standard_normal((T, H)).astype(np.float32)
    h1 = np.random.default_rng(7).standard_normal(H).astype(np.float32)
    want, (rk, rv), want_next = prefill_reference(ref, layer, hs, 0, h1)
    cache = mmr.KvCache(Hkv, D, T + 8, kvd)
    x, y = mmr.DeviceArray.from_numpy(hs.reshape(-1)), mmr.DeviceArray(T * H, np.float32)
    ws = mmr.DeviceArray(lw.prefill_workspace_size(T), np.uint8)
    lw.prefill(cache, x, 0, T, y, ws)
    got = y.numpy().reshape(T, H)
    e = rel_err(got, want)
    print(f"[result] prefill layer T={T} kv={kv}: error {e:.2e}", flush=True)
    assert e < TOL
    for i in (0, T // 2, T - 1):
        assert rel_err(got[i], want[i]) < TOL, i
    keys, values = cache.download(T)
    gk, gv = keys.astype(np.float32), values.astype(np.float32)
    rk, rv = rk.transpose(1, 0, 2), rv.transpose(1, 0, 2)
    if kv == "f32":
        assert rel_err(gk, rk) < 1e-5 and rel_err(gv, rv) < 1e-5
    else:
        assert rel_err(gk, rk.astype(np.float16).astype(np.float32)) < 2e-3
        assert rel_err(gv, rv.astype(np.float16).astype(np.float32)) < 2e-3
    # the cache now holds T rows: a second prefill is refused (decoder_layer.cpp:416-418)
    with pytest.raises(mmr.InvalidArgument, match="empty KV cache"):
        lw.prefill(cache, x, 0, T, y, ws)
    # decode continues from the prefilled cache: position T attends rows 0..T
    pos = mmr.DeviceArray.from_numpy(np.array([T], np.int32))
    err = mmr.DeviceArray(1, np.int32, zero=True)
    xd, yd = mmr.DeviceArray.from_numpy(h1), mmr.DeviceArray(H, np.float32)
    dws = mmr.DeviceArray(lw.workspace_size(4), np.uint8)
    lw.forward(cache, xd, pos, yd, dws, 4, err)
    assert rel_err(yd.numpy(), want_next) < TOL
    assert int(err.numpy()[0]) == 0


def test_minimind2_prefill_layer_in_place_rope_offset_and_capture(mm2):
    # start_position shifts only the rotation (rows still go to cache rows
    # 0..T-1); out may alias hidden_seq; the call replays from a hipGraph
    # after the cache is reset, with the same bits every replay
    mmr, oracle, g, d, model, ref = mm2
    c = g["config"]
    H, D, Hkv = c["hidden_size"], c["head_dim"], c["num_key_value_heads"]
    layer, T, start = 2, 40, 300
    lw = mmr.LayerWeights.of_model(model, layer)
    hs = np.random.default_rng(41).standard_normal((T, H)).astype(np.float32)
    want, _, _ = prefill_reference(ref, layer, hs, start, np.zeros(H, np.float32))
    cache = mmr.KvCache(Hkv, D, 64, mmr.KV_F16)
    ws = mmr.DeviceArray(lw.prefill_workspace_size(T), np.uint8)
    x = mmr.DeviceArray.from_numpy(hs.reshape(-1))
    lw.prefill(cache, x, start, T, x, ws)  # in place
    first = x.numpy().reshape(T, H)
    assert rel_err(first, want) < TOL
    stream = mmr.Stream()
    cache.reset()
    x.upload(hs.reshape(-1))
    xin = mmr.DeviceArray.from_numpy(hs.reshape(-1))
    with mmr.Graph(stream) as graph:
        lw.prefill(cache, xin, start, T, x, ws, stream=stream)
    for _ in range(3):
        graph.launch()
        stream.synchronize()
        np.testing.assert_array_equal(x.numpy().reshape(T, H), first)
    with pytest.raises(mmr.LengthError, match="not backed"):
        short = mmr.KvCache(Hkv, D, 4096, mmr.KV_F16, reserve=False)  # 512 rows backed
        lw.prefill(short, mmr.DeviceArray(600 * H, np.float32), 0, 600, mmr.DeviceArray(600 * H, np.float32),
                   mmr.DeviceArray(lw.prefill_workspace_size(600), np.uint8))
