"""GPU parity of each op-level entry point of the C ABI against the oracle.

Tolerance for floating-point outputs: max |gpu - oracle| / max |oracle| <= 2e-3
(the north-star bound for logits and attention outputs), fp32 accumulation on
both sides.  Integer outputs (argmax indices, cache appends into fp32) are
compared exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3


def f16_weights(rng, rows, cols, std=0.02):
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float16)
    return w, w.astype(np.float32)


# MiniMind2 GEMV sweep shapes (N x K), plus ragged ones
GEMV_SHAPES = [(1152, 768), (768, 768), (4096, 768), (768, 2048), (6400, 768), (1408, 512), (512, 1408), (13, 24)]


@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_matvec_matches_oracle(gpu, oracle, rows, cols):
    mmr = gpu
    print(f"[case] matvec {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    w16, w32 = f16_weights(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float16).astype(np.float32)  # x ~ N(0,1), fp16-representable
    dw = mmr.DeviceArray.from_numpy(w16.view(np.uint16))
    dx = mmr.DeviceArray.from_numpy(x)
    dy = mmr.DeviceArray(rows, np.float32)
    mmr.matvec_f16(dw, rows, cols, dx, dy)
    ref = oracle.matvec(w32, x)
    assert rel_err(dy.numpy(), ref) < TOL
    # configs[1]'s fp16 x: widened exactly, the same products and sums, the same bits
    dxh = mmr.DeviceArray.from_numpy(x.astype(np.float16).view(np.uint16))
    dyh = mmr.DeviceArray(rows, np.float32)
    mmr.matvec_f16x(dw, rows, cols, dxh, dyh)
    np.testing.assert_array_equal(dyh.numpy(), dy.numpy())
    ws = mmr.DeviceArray(mmr.matvec_argmax_workspace_size(rows, cols), np.uint8)
    tok, lg = mmr.DeviceArray(1, np.int32), mmr.DeviceArray(rows, np.float32)
    mmr.matvec_argmax_f16x(dw, rows, cols, dxh, tok, ws, logits=lg)
    np.testing.assert_array_equal(lg.numpy(), dy.numpy())
    assert int(tok.numpy()[0]) == oracle.argmax(dy.numpy())
    # residual epilogue (device_matmul_add)
    res = rng.standard_normal(rows).astype(np.float32)
    dr = mmr.DeviceArray.from_numpy(res)
    mmr.matvec_f16(dw, rows, cols, dx, dr, residual=dr)
    assert rel_err(dr.numpy(), res + ref) < TOL


@pytest.mark.parametrize("lanes", [16, 32, 64])
@pytest.mark.parametrize("rpg", [1, 2, 4])
def test_matvec_launch_shapes_agree(gpu, oracle, lanes, rpg):
    mmr = gpu
    rng = np.random.default_rng(lanes + rpg)
    rows, cols = 1000, 768
    w16, w32 = f16_weights(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    dw, dx, dy = mmr.DeviceArray.from_numpy(w16.view(np.uint16)), mmr.DeviceArray.from_numpy(x), mmr.DeviceArray(rows, np.float32)
    mmr.matvec_f16_ex(dw, rows, cols, dx, dy, lanes_per_row=lanes, rows_per_group=rpg)
    assert rel_err(dy.numpy(), oracle.matvec(w32, x)) < TOL


def test_fused_rmsnorm_prologue_and_swiglu(gpu, oracle):
    mmr = gpu
    rng = np.random.default_rng(11)
    H, F, eps = 768, 2048, 1e-5
    h = (rng.standard_normal(H) * 0.3).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    g16, g32 = f16_weights(rng, F, H)
    u16, u32 = f16_weights(rng, F, H)
    inter = np.empty((2 * F, H), np.float16)
    inter[0::2], inter[1::2] = g16, u16  # device layout: gate_i, up_i interleaved
    dw = mmr.DeviceArray.from_numpy(inter.view(np.uint16))
    dh, dn = mmr.DeviceArray.from_numpy(h), mmr.DeviceArray.from_numpy(nw)
    dy = mmr.DeviceArray(F, np.float32)
    mmr.matvec_f16_ex(dw, 2 * F, H, dh, dy, norm_w=dn, eps=eps, prologue=mmr.PRO_RMSNORM, epilogue=mmr.EPI_SWIGLU)
    xn = oracle.rms_norm_layer(h, nw, eps)
    gu = np.concatenate([oracle.matvec(g32, xn), oracle.matvec(u32, xn)])
    assert rel_err(dy.numpy(), oracle.swiglu_from_gate_up(gu)) < TOL
    # plain RMSNorm prologue into a store
    dq = mmr.DeviceArray(F, np.float32)
    dg = mmr.DeviceArray.from_numpy(g16.view(np.uint16))
    mmr.matvec_f16_ex(dg, F, H, dh, dq, norm_w=dn, eps=eps, prologue=mmr.PRO_RMSNORM)
    assert rel_err(dq.numpy(), oracle.matvec(g32, xn)) < TOL


def test_argmax_matches_oracle_and_first_index(gpu, oracle):
    mmr = gpu
    rng = np.random.default_rng(5)
    V, H, eps = 6400, 768, 1e-5
    w16, w32 = f16_weights(rng, V, H)
    h = rng.standard_normal(H).astype(np.float32)
    nw = np.ones(H, np.float32)
    dw, dh, dn = (mmr.DeviceArray.from_numpy(a) for a in (w16.view(np.uint16), h, nw))
    logits, tok = mmr.DeviceArray(V, np.float32), mmr.DeviceArray(1, np.int32)
    ws = mmr.DeviceArray(mmr.matvec_argmax_workspace_size(V, H), np.uint8)
    mmr.matvec_argmax_f16(dw, V, H, dh, tok, ws, logits=logits, norm_w=dn, eps=eps)
    ref = oracle.matvec(w32, oracle.rms_norm_final(h, nw, eps))
    assert rel_err(logits.numpy(), ref) < TOL
    assert int(tok.numpy()[0]) == int(np.argmax(logits.numpy())) == oracle.argmax(ref)
    # exact ties resolve to the lowest index: duplicate the winning row further down and earlier
    win = int(tok.numpy()[0])
    for dup in (V - 1, 17):
        w2 = w16.copy()
        w2[dup] = w16[win]
        dw.upload(w2.view(np.uint16))
        for rep in range(3):  # repeated calls on the same workspace stay correct
            mmr.matvec_argmax_f16(dw, V, H, dh, tok, ws, norm_w=dn, eps=eps)
            assert int(tok.numpy()[0]) == min(win, dup)


def cache_layout(keys_ref, tokens, hkv, d, rows):
    """[token][kv_head][d] (reference) -> [kv_head][rows][d] (cache)."""
    out = np.zeros((hkv, rows, d), keys_ref.dtype)
    out[:, :tokens, :] = keys_ref.reshape(tokens, hkv, d).transpose(1, 0, 2)
    return out


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("tokens", [1, 5, 63, 64, 65, 128, 1024, 4097, 8193])
def test_attention_from_cache_matches_oracle(gpu, oracle, kv, tokens):
    # 8 q / 2 kv heads, d 96, K/V ~ N(0,1); T cached + the new token
    mmr = gpu
    print(f"[case] attention kv={kv} tokens={tokens}", flush=True)
    hq, hkv, d = 8, 2, 96
    rng = np.random.default_rng(tokens)
    np_kv = np.float16 if kv == "f16" else np.float32
    q = rng.standard_normal(hq * d).astype(np.float32)
    k = rng.standard_normal(tokens * hkv * d).astype(np_kv).astype(np.float32)
    v = rng.standard_normal(tokens * hkv * d).astype(np_kv).astype(np.float32)
    cap = tokens + 3
    cache = mmr.KvCache(hkv, d, cap, mmr.KV_F16 if kv == "f16" else mmr.KV_F32)
    cache.upload(cache_layout(k, tokens, hkv, d, cache.rows), cache_layout(v, tokens, hkv, d, cache.rows))
    dq, out = mmr.DeviceArray.from_numpy(q), mmr.DeviceArray(hq * d, np.float32)
    ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, 4096), np.uint8)
    ref = oracle.attention_step(q, k, v, tokens, hq, hkv, d)
    mmr.attention_from_cache(dq, cache, tokens, hq, hkv, d, out, ws)
    got = out.numpy()
    assert rel_err(got, ref) < TOL
    # any split count (up to the limit) gives the same result.  The combine kernel takes 16 groups x R loads per
    # thread, R the smallest of 2, 4, ..., 16, 20, ..., 32 covering the splits: every R is reached here (32 / 33,
    # 128 / 129, 256 / 257 and 512 / 513 on either side of a variant's limit), and 4096 takes the multi-round one
    for splits in (1, 3, 7, 32, 33, 65, 100, 128, 129, 180, 200, 240, 256, 257, 300, 350, 400, 512, 513, 4096):
        mmr.attention_from_cache(dq, cache, tokens, hq, hkv, d, out, ws, splits=splits)
        assert rel_err(out.numpy(), got) < 1e-5


def test_attention_reference_patterned_case(gpu, oracle):
    # test_ascend_custom_ops.cpp:91-136 (T 5, 4/2 heads, d 16), at the tighter bound
    mmr = gpu
    T, hq, hkv, d = 5, 4, 2, 16
    q = ((np.arange(hq * d) % 13) - 6).astype(np.float32) * 0.03125
    i = np.arange(T * hkv * d)
    k = ((i % 17) - 8).astype(np.float32) * 0.025
    v = ((i % 11) - 5).astype(np.float32) * 0.0375
    cache = mmr.KvCache(hkv, d, 8, mmr.KV_F32)
    cache.upload(cache_layout(k, T, hkv, d, cache.rows), cache_layout(v, T, hkv, d, cache.rows))
    dq, out = mmr.DeviceArray.from_numpy(q), mmr.DeviceArray(hq * d, np.float32)
    ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, 0), np.uint8)
    mmr.attention_from_cache(dq, cache, T, hq, hkv, d, out, ws)
    assert rel_err(out.numpy(), oracle.attention_step(q, k, v, T, hq, hkv, d)) < TOL


@pytest.mark.parametrize("d", [64, 96, 128])
def test_qkv_postprocess_and_append(gpu, oracle, d):
    mmr = gpu
    hq, hkv, pos, eps, theta = 8, 2, 7, 1e-5, 1e6
    rng = np.random.default_rng(d)
    qkv = rng.standard_normal((hq + 2 * hkv) * d).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    rope = mmr.RopeTable(64, d, theta)
    cache = mmr.KvCache(hkv, d, 16, mmr.KV_F32)
    dqkv, dqn, dkn = (mmr.DeviceArray.from_numpy(a) for a in (qkv, qn, kn))
    query = mmr.DeviceArray(hq * d, np.float32)
    tokens = 4  # append at cache index 3
    mmr.decode_qkv_postprocess(dqkv, dqn, dkn, cache, tokens, hq, hkv, d, pos, rope, eps, query)
    q_ref, k_ref = oracle.qk_norm_rope(qkv[: hq * d], qkv[hq * d: (hq + hkv) * d], qn, kn, hq, hkv, d, pos, eps, theta)
    assert rel_err(query.numpy(), q_ref) < 1e-5
    keys, vals = cache.download()
    assert rel_err(keys[:, tokens - 1, :].reshape(-1), k_ref) < 1e-5
    np.testing.assert_array_equal(vals[:, tokens - 1, :].reshape(-1), qkv[(hq + hkv) * d:])
    assert not keys[:, tokens:, :].any() and not keys[:, : tokens - 1, :].any()
    assert cache.rows == 16 and cache.device_bytes == 2 * hkv * 64 * d * 4  # one 64-token page of K and of V


@pytest.mark.parametrize("splits", [8, 129])
@pytest.mark.parametrize("d", [32, 64, 96, 128])
@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_fused_append_attention_matches_oracle(gpu, oracle, kv, d, splits):
    # regression: the appended key must be the rotated one for every head_dim
    # (d = 64 once stored a half-rotated key: a missing barrier between RoPE
    # and the rounding of the new key).  8 splits run the per-head kernel;
    # 129 (more blocks than the per-head and per-group kernels take) the
    # split-K kernel, on the fp16 matrix cores for an fp16 cache and d <= 96.
    mmr = gpu
    print(f"[case] fused attention kv={kv} d={d} splits={splits}", flush=True)
    hq, hkv, eps, theta = 8, 2, 1e-5, 1e6
    rng = np.random.default_rng(21)
    np_kv = np.float16 if kv == "f16" else np.float32
    cap = 300
    rope = mmr.RopeTable(1024, d, theta)
    cache = mmr.KvCache(hkv, d, cap, mmr.KV_F16 if kv == "f16" else mmr.KV_F32)
    qn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    dqn, dkn = mmr.DeviceArray.from_numpy(qn), mmr.DeviceArray.from_numpy(kn)
    ws = mmr.DeviceArray(mmr.attention_workspace_size(hq, hkv, d, splits), np.uint8)
    err = mmr.DeviceArray(1, np.int32, zero=True)
    pos_d = mmr.DeviceArray(1, np.int32)
    out = mmr.DeviceArray(hq * d, np.float32)
    keys_ref, vals_ref = [], []
    for pos in range(cap):  # decode a whole sequence: append then attend each step
        qkv = rng.standard_normal((hq + 2 * hkv) * d).astype(np.float32)
        pos_d.upload(np.array([pos], np.int32))
        mmr.decode_attention_fused(mmr.DeviceArray.from_numpy(qkv), dqn, dkn, eps, rope, pos_d, cache, hq, hkv, d,
                                   out, ws, splits, err)
        q_ref, k_ref = oracle.qk_norm_rope(qkv[: hq * d], qkv[hq * d: (hq + hkv) * d], qn, kn, hq, hkv, d, pos,
                                           eps, theta)
        keys_ref.append(k_ref.astype(np_kv).astype(np.float32))
        vals_ref.append(qkv[(hq + hkv) * d:].astype(np_kv).astype(np.float32))
        if pos in (0, 1, 2, 3, 63, 64, 200, cap - 1):
            ref = oracle.attention_step(q_ref, np.concatenate(keys_ref), np.concatenate(vals_ref), pos + 1, hq, hkv, d)
            assert rel_err(out.numpy(), ref) < TOL, pos
            keys, _ = cache.download()
            stored = keys[:, : pos + 1, :].transpose(1, 0, 2).reshape(-1).astype(np.float32)
            # fp32 cache: fp32 rounding only; fp16 cache: a key within 1e-7 of an
            # fp16 rounding boundary may land on the neighbouring value (2^-11 rel)
            key_tol = 1e-5 if kv == "f32" else 1e-3
            assert rel_err(stored, np.concatenate(keys_ref)) < key_tol, pos
    assert int(err.numpy()[0]) == 0
    pos_d.upload(np.array([cap], np.int32))  # out of range: flagged, nothing written
    mmr.decode_attention_fused(mmr.DeviceArray.from_numpy(qkv), dqn, dkn, eps, rope, pos_d, cache, hq, hkv, d, out,
                               ws, splits, err)
    assert int(err.numpy()[0]) == 1


def test_support_ops(gpu, oracle):
    mmr = gpu
    # rms_norm_rows 3 x 128 (test_ascend_custom_ops.cpp:195-220)
    rows, cols, eps = 3, 128, 1e-5
    x = ((np.arange(rows * cols) % 23) - 11).astype(np.float32) * 0.0625
    w = (0.75 + (np.arange(cols) % 5) * 0.03125).astype(np.float32)
    dx, dw, dy = mmr.DeviceArray.from_numpy(x), mmr.DeviceArray.from_numpy(w), mmr.DeviceArray(rows * cols, np.float32)
    mmr.rms_norm_rows(dx, dw, eps, rows, cols, dy)
    ref = np.concatenate([oracle.rms_norm_layer(x[r * cols:(r + 1) * cols], w, eps) for r in range(rows)])
    assert rel_err(dy.numpy(), ref) < 1e-5
    # swiglu_rows 3 x 64 (test_ascend_custom_ops.cpp:222-245)
    sr, sc = 3, 64
    gu = np.zeros((sr, 2 * sc), np.float32)
    idx = np.arange(sr * sc).reshape(sr, sc)
    gu[:, :sc] = ((idx % 13) - 6) * 0.125
    gu[:, sc:] = ((idx % 11) - 5) * 0.0625
    dgu, dout = mmr.DeviceArray.from_numpy(gu), mmr.DeviceArray(sr * sc, np.float32)
    mmr.swiglu_rows(dgu, sr, sc, dout)
    ref = np.concatenate([oracle.swiglu_from_gate_up(gu[r]) for r in range(sr)])
    assert rel_err(dout.numpy(), ref) < 1e-5
    # add (test_ascend_custom_ops.cpp:20-30)
    a = ((np.arange(128) % 17) - 8).astype(np.float32) * 0.03125
    b = ((np.arange(128) % 13) - 6).astype(np.float32) * 0.0625
    da, db, dc = mmr.DeviceArray.from_numpy(a), mmr.DeviceArray.from_numpy(b), mmr.DeviceArray(128, np.float32)
    mmr.add(da, db, 128, dc)
    np.testing.assert_array_equal(dc.numpy(), a + b)
    # embedding gather with an out-of-range id flagged, not read
    table = np.random.default_rng(0).standard_normal((10, 16)).astype(np.float16)
    ids = np.array([3, 0, 9, 10], np.int32)
    dt, di = mmr.DeviceArray.from_numpy(table.view(np.uint16)), mmr.DeviceArray.from_numpy(ids)
    de, derr = mmr.DeviceArray(4 * 16, np.float32), mmr.DeviceArray(1, np.int32, zero=True)
    mmr.embedding_gather(dt, di, 4, 10, 16, de, derr)
    e = de.numpy().reshape(4, 16)
    np.testing.assert_array_equal(e[:3], table[[3, 0, 9]].astype(np.float32))
    assert not e[3].any() and int(derr.numpy()[0]) == 1


def test_launch_floor_probe(gpu):
    # the bench's per-kernel floor: both chains run and report a plausible time
    mmr = gpu
    empty = mmr.launch_floor_us(16, 64, False, 4)
    dep = mmr.launch_floor_us(16, 64, True, 4)
    assert 0.1 < empty < 100.0 and 0.1 < dep < 100.0
    with pytest.raises(mmr.InvalidArgument):
        mmr.launch_floor_us(0, 64, True, 4)


def test_graph_capture_replays_the_captured_calls(gpu, oracle):
    # mmr.Graph: calls enqueued inside the block are captured, not run; each
    # replay runs them again and matches the eager result.
    mmr = gpu
    rng = np.random.default_rng(5)
    w, w32 = f16_weights(rng, 768, 768)
    x = rng.standard_normal(768).astype(np.float32)
    dw, dx = mmr.DeviceArray.from_numpy(w.view(np.uint16)), mmr.DeviceArray.from_numpy(x)
    y_eager, y_graph = mmr.DeviceArray(768, np.float32), mmr.DeviceArray(768, np.float32, zero=True)
    stream = mmr.Stream()
    mmr.matvec_f16(dw, 768, 768, dx, y_eager, stream=stream)
    with mmr.Graph(stream) as graph:
        mmr.matvec_f16(dw, 768, 768, dx, y_graph, stream=stream)
    stream.synchronize()
    assert not y_graph.numpy().any()  # captured, not executed
    for _ in range(3):
        graph.launch()
        stream.synchronize()
        np.testing.assert_array_equal(y_graph.numpy(), y_eager.numpy())
        y_graph.upload(np.zeros(768, np.float32))
    graph.free()
    assert rel_err(y_eager.numpy(), oracle.matvec(w32, x)) < TOL
