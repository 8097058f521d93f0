"""GPU test of mmr_attention_from_cache_noalloc, the entry point that
allocates nothing (split partials in the library's static device scratch):
its output must equal mmr_attention_from_cache's (same kernels, same split
count, caller workspace) bit for bit, on two calls in a row, the second with
a smaller input, and a request beyond the scratch must fail cleanly.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _cache(mmr, rng, hkv, d, tokens, kv):
    c = mmr.KvCache(hkv, d, tokens, kv)
    dt = np.float16 if kv == mmr.KV_F16 else np.float32
    c.upload(rng.standard_normal((hkv, c.rows, d)).astype(dt), rng.standard_normal((hkv, c.rows, d)).astype(dt))
    return c


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_noalloc_attention_equals_workspace_entry(gpu, kv):
    mmr = gpu
    print(f"[case] noalloc attention kv={kv}", flush=True)
    kvd = mmr.KV_F16 if kv == "f16" else mmr.KV_F32
    rng = np.random.default_rng(17)
    hq, hkv, d = 8, 2, 96
    for tokens, splits in ((3001, 0), (130, 0), (700, 40)):  # second call smaller than the first
        cache = _cache(mmr, rng, hkv, d, tokens, kvd)
        q = mmr.DeviceArray.from_numpy(rng.standard_normal(hq * d).astype(np.float32))
        want, got = mmr.DeviceArray(hq * d, np.float32), mmr.DeviceArray(hq * d, np.float32)
        n = splits or -(-tokens // 64)
        ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, n), np.uint8)
        mmr.attention_from_cache(q, cache, tokens, hq, hkv, d, want, ws, splits)
        mmr.attention_from_cache_noalloc(q, cache, tokens, hq, hkv, d, got, splits)
        mmr.synchronize()
        np.testing.assert_array_equal(got.numpy(), want.numpy(), err_msg=f"tokens {tokens}")
        assert np.isfinite(got.numpy()).all()


def test_noalloc_attention_rejects_partials_beyond_scratch(gpu):
    mmr = gpu
    hq, hkv, d = 8, 2, 96
    cache = mmr.KvCache(hkv, d, 4096, mmr.KV_F16)
    q, out = mmr.DeviceArray(hq * d, np.float32, zero=True), mmr.DeviceArray(hq * d, np.float32)
    assert mmr.attention_workspace_size(hq, hkv, d, 4096) > mmr.NOALLOC_SCRATCH_BYTES
    with pytest.raises(mmr.InvalidArgument, match="static scratch"):
        mmr.attention_from_cache_noalloc(q, cache, 4096, hq, hkv, d, out, 4096)
