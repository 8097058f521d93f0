"""The KV cache's paging: 64-token pages in doubling segments (segment 0 =
positions [0, 512), segment s >= 1 = [512 << (s - 1), 512 << s)), backed as
the context reaches them.  This replaces the reference's resident cache,
which reallocates and drops its rows when a longer context arrives
(ensure_attention_cache, ascend_custom_ops.cpp:126-139).

Checks: the backed extent and device bytes follow the segment rule exactly;
rows written across segment boundaries read back bit for bit; attention over
rows spread across segments equals the oracle's (decoder_layer.cpp:184-234)
within 2e-3; op-level calls on unbacked rows fail instead of allocating; a
model state backs one segment at creation and grows without moving a row
(its tokens stay those of a fully backed run).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_golden, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3


def page_bytes(hkv, d, elem):
    return 64 * hkv * d * elem  # one layer's keys (or values) of one page


def test_op_cache_grows_by_segments(gpu, oracle):
    mmr = gpu
    hq, hkv, d = 8, 2, 96
    cache = mmr.KvCache(hkv, d, 4096, mmr.KV_F16, reserve=False)
    assert cache.rows == 512  # segment 0 only
    assert cache.device_bytes == 2 * 8 * page_bytes(hkv, d, 2)
    k0, v0, first, n = cache.segment(0)
    assert k0 and v0 and (first, n) == (0, 512)
    assert cache.segment(1)[0] == 0 and cache.segment(1)[3] == 0  # unbacked
    rng = np.random.default_rng(31)
    q = rng.standard_normal(hq * d).astype(np.float32)
    T = 1000
    keys = rng.standard_normal((hkv, T, d)).astype(np.float16)
    vals = rng.standard_normal((hkv, T, d)).astype(np.float16)
    dq, out = mmr.DeviceArray.from_numpy(q), mmr.DeviceArray(hq * d, np.float32)
    ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, 0), np.uint8)
    cache.upload(keys[:, :500], vals[:, :500])
    with pytest.raises(mmr.LengthError, match="not backed"):  # op-level calls never allocate
        mmr.attention_from_cache(dq, cache, 600, hq, hkv, d, out, ws)
    cache.reserve(600)
    assert cache.rows == 1024 and cache.device_bytes == 2 * 16 * page_bytes(hkv, d, 2)
    assert cache.segment(1)[2:] == (512, 512)
    cache.upload(keys[:, 500:], vals[:, 500:], first=500)  # rows 500..999 straddle segments 0 and 1
    gk, gv = cache.download(T)
    np.testing.assert_array_equal(gk, keys)
    np.testing.assert_array_equal(gv, vals)
    # attention over all 1000 rows (tiles in both segments), any split count
    kref = keys.transpose(1, 0, 2).reshape(-1).astype(np.float32)
    vref = vals.transpose(1, 0, 2).reshape(-1).astype(np.float32)
    want = oracle.attention_step(q, kref, vref, T, hq, hkv, d)
    for splits in (0, 1, 5, 16, 40):
        mmr.attention_from_cache(dq, cache, T, hq, hkv, d, out, ws, splits=splits)
        assert rel_err(out.numpy(), want) < TOL, splits
    with pytest.raises(mmr.LengthError):
        cache.reserve(4097)
    cache.reserve(4096)  # segments 2 (1024..2047) and 3 (2048..4095)
    assert cache.rows == 4096 and cache.device_bytes == 2 * 64 * page_bytes(hkv, d, 2)
    np.testing.assert_array_equal(cache.download(T)[0], keys)  # growth moved nothing
    cache.reset()
    assert cache.rows == 512 and cache.segment(1)[0] == 0
    assert cache.device_bytes == 2 * 8 * page_bytes(hkv, d, 2)
    np.testing.assert_array_equal(cache.download(500)[0], keys[:, :500])  # segment 0 kept


def test_op_cache_short_capacity_backs_whole_pages(gpu):
    mmr = gpu
    cache = mmr.KvCache(2, 64, 100, mmr.KV_F32, reserve=False)
    assert cache.rows == 100  # usable positions: the capacity
    assert cache.device_bytes == 2 * 2 * page_bytes(2, 64, 4)  # two 64-token pages
    with pytest.raises(mmr.MmrError):
        cache.upload(np.zeros((2, 101, 64), np.float32), np.zeros((2, 101, 64), np.float32))


def test_state_backs_one_segment_and_grows_with_the_context(gpu, oracle, tmp_path):
    # make_state backs segment 0 only; the prompt and the decode steps add
    # segments as the context reaches them (a decode graph's split bucket is
    # backed whole before it is captured).  Tokens equal a fully backed run's.
    mmr = gpu
    g = load_golden("mini")
    cfg = mmr.make_config(**g["config"])
    mmr.write_synthetic_model(tmp_path, cfg, g["seed"], g["std"], g["round_fp16"])
    model = mmr.Model.load(tmp_path)
    L, hkv, d = g["config"]["num_hidden_layers"], g["config"]["num_key_value_heads"], g["config"]["head_dim"]
    seg_bytes = lambda pages: 2 * L * pages * page_bytes(hkv, d, 2)  # noqa: E731
    st = model.make_state(0, mmr.KV_F16)  # capacity = max_position_embeddings (4096)
    assert st.kv_backed() == (512, seg_bytes(8))
    prompt = mmr.synthesize_prompt(77, 600, g["config"]["vocab_size"]).tolist()
    st.enqueue_prefill(prompt)
    st.synchronize()
    assert st.kv_backed() == (1024, seg_bytes(16))  # the prompt's 600 rows: segments 0 and 1
    st.enqueue_decode(8)  # context 601..608: 10 tiles, the 12-split bucket, up to 12 tiles (768)
    st.synchronize()
    assert st.kv_backed() == (1024, seg_bytes(16))
    st.enqueue_decode(1500)  # context past 2048 (33+ tiles): the 40-split bucket reaches 2560, segment 3
    st.synchronize()
    assert st.kv_backed() == (4096, seg_bytes(64))
    got = st.read_sequence(600, 1509).tolist()
    # the same decode on a state whose whole capacity is backed from the start
    ref = model.make_state(0, mmr.KV_F16)
    ref.reserve(4096)
    assert ref.kv_backed() == (4096, seg_bytes(64))
    ref.enqueue_prefill(prompt)
    ref.enqueue_decode(1508)
    ref.synchronize()
    assert ref.read_sequence(600, 1509).tolist() == got
    with pytest.raises(mmr.LengthError):
        ref.reserve(4097)
