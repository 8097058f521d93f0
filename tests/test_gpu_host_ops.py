"""GPU parity of the host-vector operator twins (cube_matvec, cube_matmul,
cube_matvec_argmax, ascend_matmul.h:116-133; custom_attention,
custom_prefill_attention, custom_attention_cached, ascend_custom_ops.h:33-55)
and the availability probes, through the C ABI, against the oracle's CPU
restatement (oracle/cpu_ref.c: orc_matvec decoder_layer.cpp:65-90,
orc_attention_step decoder_layer.cpp:184-234, orc_argmax
language_model.cpp:408-413).

Bar: matrices are fp16-representable, so the projections differ from the
oracle only by summation order: max|d| / max|ref| < 1e-5; attention within
2e-3 (observed ~1e-7); argmax indices exact, ties to the first index.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def fp16_exact(rng, *shape, std=0.05):
    return (rng.standard_normal(shape) * std).astype(np.float16).astype(np.float32)


def test_probes(gpu):
    assert gpu.cube_matvec_available() and gpu.cube_matmul_available() and gpu.custom_ops_available()


def test_cube_matvec_matmul_argmax(gpu, oracle):
    mmr = gpu
    rng = np.random.default_rng(21)
    for rows, cols in ((300, 256), (1152, 768), (7, 64)):
        w = fp16_exact(rng, rows, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        assert rel_err(mmr.cube_matvec(w, x), oracle.matvec(w, x)) < 1e-5
        X = rng.standard_normal((5, cols)).astype(np.float32)
        got = mmr.cube_matmul(w, X)
        for b in range(5):
            assert rel_err(got[b], oracle.matvec(w, X[b])) < 1e-5
        assert mmr.cube_matvec_argmax(w, x) == oracle.argmax(oracle.matvec(w, x))
    # duplicate maximal rows: the first index wins (std::max_element)
    w = fp16_exact(rng, 64, 64)
    w[40] = w[9] = np.abs(w[9]) + 0.25
    x = np.ones(64, np.float32)
    assert mmr.cube_matvec_argmax(w, x) == 9
    with pytest.raises(mmr.InvalidArgument):
        mmr.cube_matvec(fp16_exact(rng, 4, 12), np.ones(12, np.float32))  # cols not a multiple of 8


def test_custom_attention_forms(gpu, oracle):
    mmr = gpu
    rng = np.random.default_rng(22)
    hq, hkv, d = 8, 2, 64
    T = 37
    q = rng.standard_normal(hq * d).astype(np.float32)
    keys = rng.standard_normal((T, hkv, d)).astype(np.float32)
    values = rng.standard_normal((T, hkv, d)).astype(np.float32)
    got = mmr.custom_attention(q, keys, values, T, hq, hkv, d)
    assert rel_err(got, oracle.attention_step(q, keys, values, T, hq, hkv, d)) < 2e-3
    # cached: one key/value per call, attention over the growing cache
    cache = mmr.HostAttentionCache()
    for t in range(1, 30):
        out = mmr.custom_attention_cached(q, keys[t - 1], values[t - 1], cache, t, hq, hkv, d)
        assert rel_err(out, oracle.attention_step(q, keys[:t], values[:t], t, hq, hkv, d)) < 2e-3, t
    assert cache.info()[:3] == (hkv, d, 2048)  # the reference's 2048-token floor
    # prefill: causal attention of every row over its prefix
    S = 40
    Q = rng.standard_normal((S, hq * d)).astype(np.float32)
    K = rng.standard_normal((S, hkv, d)).astype(np.float32)
    Vv = rng.standard_normal((S, hkv, d)).astype(np.float32)
    out = mmr.custom_prefill_attention(Q, K, Vv, cache, S, hq, hkv, d).reshape(S, hq * d)
    for i in (0, 1, 17, S - 1):
        assert rel_err(out[i], oracle.attention_step(Q[i], K[: i + 1], Vv[: i + 1], i + 1, hq, hkv, d)) < 2e-3, i
    # a cache of another shape is replaced
    other = mmr.custom_attention_cached(q[: 4 * 32], keys[0, :, :32].copy(), values[0, :, :32].copy(), cache, 1,
                                        4, hkv, 32)
    assert cache.info()[:2] == (hkv, 32)
    np.testing.assert_allclose(other, np.repeat(values[0, :, :32], 2, axis=0).reshape(-1), rtol=1e-6)


def test_cached_attention_grows_and_keeps_rows(gpu, oracle):
    # prefill fills the 2048-row cache; the next cached call needs row 2048:
    # the cache grows and rows 0..2047 stay (the reference would start empty)
    mmr = gpu
    rng = np.random.default_rng(23)
    hq, hkv, d, S = 4, 2, 32, 2048
    Q = rng.standard_normal((S, hq * d)).astype(np.float32)
    K = rng.standard_normal((S + 1, hkv, d)).astype(np.float32)
    Vv = rng.standard_normal((S + 1, hkv, d)).astype(np.float32)
    cache = mmr.HostAttentionCache()
    mmr.custom_prefill_attention(Q, K[:S], Vv[:S], cache, S, hq, hkv, d)
    assert cache.info()[2] == 2048
    q = rng.standard_normal(hq * d).astype(np.float32)
    out = mmr.custom_attention_cached(q, K[S], Vv[S], cache, S + 1, hq, hkv, d)
    assert cache.info()[2] >= S + 1
    assert rel_err(out, oracle.attention_step(q, K, Vv, S + 1, hq, hkv, d)) < 2e-3


def test_cached_attention_forms_keep_a_callers_fp16_cache(gpu, oracle):
    # A caller may hand the twins an fp16 cache (the reference's device cache
    # dtype, ascend_custom_ops.cpp:126-139): rows are stored rounded to fp16,
    # for every KV head, and the dtype survives growth.  The oracle sees the
    # same fp16-rounded keys/values.
    mmr = gpu
    rng = np.random.default_rng(24)
    hq, hkv, d, S = 8, 2, 64, 300
    Q = rng.standard_normal((S, hq * d)).astype(np.float32)
    K = rng.standard_normal((S + 2, hkv, d)).astype(np.float32)
    Vv = rng.standard_normal((S + 2, hkv, d)).astype(np.float32)
    Kh, Vh = (a.astype(np.float16).astype(np.float32) for a in (K, Vv))
    cache = mmr.HostAttentionCache.create(hkv, d, S, mmr.KV_F16)
    out = mmr.custom_prefill_attention(Q, K[:S], Vv[:S], cache, S, hq, hkv, d).reshape(S, hq * d)
    for i in (0, 5, S - 1):
        want = oracle.attention_step(Q[i], Kh[: i + 1], Vh[: i + 1], i + 1, hq, hkv, d)
        assert rel_err(out[i], want) < 2e-3, i
    q = rng.standard_normal(hq * d).astype(np.float32)
    for t in (S + 1, S + 2):  # the second call outgrows the 300-row cache
        got = mmr.custom_attention_cached(q, K[t - 1], Vv[t - 1], cache, t, hq, hkv, d)
        assert rel_err(got, oracle.attention_step(q, Kh[:t], Vh[:t], t, hq, hkv, d)) < 2e-3, t
    kvh, dd, cap, dtype = cache.info()
    assert (kvh, dd, dtype) == (hkv, d, mmr.KV_F16) and cap >= S + 2
