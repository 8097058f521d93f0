"""Pins the CPU oracle (oracle/cpu_ref.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (dropped
eps, swapped RoPE sign or pair index, transposed matrix, wrong GQA head
mapping, softmax without max subtraction or normalisation, last-instead-of-
first argmax) fails it:
  * closed forms and patterned inputs of the reference's own tests
    (test_ops.cpp, test_rope.cpp, test_ascend_custom_ops.cpp) checked against
    an independent float64 computation at tight tolerance;
  * invariants (RoPE at position 0, norm preservation, one-key attention);
  * the golden fixtures produced by the reference build (oracle/_ref), which
    the oracle must reproduce bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_golden, rel_err


# ---- closed forms from the reference's unit tests --------------------------------

def test_rms_norm_eps0_closed_form(oracle):
    # test_ops.cpp:23-36: rows [3, 4] and [1, 2], weight [1, 2], eps 0
    w = np.array([1.0, 2.0], np.float32)
    out = oracle.rms_norm_layer([3.0, 4.0], w, 0.0)
    s = 1.0 / np.sqrt((9.0 + 16.0) / 2.0)
    assert abs(out[0] - 3.0 * s) < 1e-6 and abs(out[1] - 4.0 * s * 2.0) < 1e-6
    out2 = oracle.rms_norm_layer([1.0, 2.0], w, 0.0)
    s2 = 1.0 / np.sqrt((1.0 + 4.0) / 2.0)
    assert abs(out2[0] - s2) < 1e-6 and abs(out2[1] - 4.0 * s2) < 1e-6


def test_swiglu_closed_form(oracle):
    # test_ops.cpp:38-49: gate [0, 1, -1], up [2, 3, 4]
    out = oracle.swiglu_from_gate_up([0.0, 1.0, -1.0, 2.0, 3.0, 4.0])
    expect = [0.0, 3.0 / (1.0 + np.exp(-1.0)), -4.0 / (1.0 + np.exp(1.0))]
    np.testing.assert_allclose(out, expect, atol=1e-6)


def test_rms_norm_patterned_128(oracle):
    # test_ascend_custom_ops.cpp:32-51 patterned input, eps 1e-5
    i = np.arange(128)
    x = ((i % 17) - 8).astype(np.float32) * 0.125
    w = (0.5 + (i % 7) * 0.03125).astype(np.float32)
    xd = x.astype(np.float64)
    expect = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w
    out = oracle.rms_norm_layer(x, w, 1e-5)
    assert rel_err(out, expect) < 1e-6
    # the final-norm association differs only in rounding
    assert rel_err(oracle.rms_norm_final(x, w, 1e-5), expect) < 1e-6
    # eps matters: dropping it changes the result measurably for a tiny input
    tiny = x * 1e-3
    with_eps = oracle.rms_norm_layer(tiny, w, 1e-5)
    no_eps = oracle.rms_norm_layer(tiny, w, 0.0)
    assert rel_err(with_eps, no_eps) > 1e-3


def test_rope_table_values(oracle):
    # test_rope.cpp:39-44: theta 1e4, d 4, position 1 -> (cos 1, cos 0.01)
    c, s = oracle.rope_row(1, 4, 1e4)
    np.testing.assert_allclose(c, [np.cos(1.0), np.cos(0.01)], atol=1e-6)
    np.testing.assert_allclose(s, [np.sin(1.0), np.sin(0.01)], atol=1e-6)
    c0, s0 = oracle.rope_row(0, 4, 1e4)
    np.testing.assert_array_equal(c0, [1.0, 1.0])
    np.testing.assert_array_equal(s0, [0.0, 0.0])


def rope_f64(x, heads, d, pos, theta):
    x = np.asarray(x, np.float64).reshape(heads, d).copy()
    half = d // 2
    inv = 1.0 / theta ** (np.arange(half) * 2.0 / d)
    ang = pos * inv
    a, b = x[:, :half].copy(), x[:, half:].copy()
    x[:, :half] = a * np.cos(ang) - b * np.sin(ang)
    x[:, half:] = b * np.cos(ang) + a * np.sin(ang)
    return x.reshape(-1)


def test_rope_patterned_2x96(oracle):
    # test_ascend_custom_ops.cpp:67-89: 2 heads, d 96, position 7, theta 1e6
    x = ((np.arange(192) % 19) - 9).astype(np.float32) * 0.03125
    out = oracle.apply_rope(x, 2, 96, 7, 1e6)
    assert rel_err(out, rope_f64(x, 2, 96, 7, 1e6)) < 1e-5
    # rotate-half pairs (i, i + d/2): swapping the pairing or the sign fails
    wrong = rope_f64(x[::-1].copy(), 2, 96, 7, 1e6)[::-1]
    assert rel_err(out, wrong) > 1e-2


def test_rope_invariants(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(8 * 96).astype(np.float32)
    np.testing.assert_array_equal(oracle.apply_rope(x, 8, 96, 0, 1e6), x)
    y = oracle.apply_rope(x, 8, 96, 1234, 1e6).reshape(8, 2, 48)
    xr = x.reshape(8, 2, 48)
    np.testing.assert_allclose(np.hypot(y[:, 0], y[:, 1]), np.hypot(xr[:, 0], xr[:, 1]), rtol=1e-5)


def attention_f64(q, k, v, tokens, hq, hkv, d):
    q = np.asarray(q, np.float64).reshape(hq, d)
    k = np.asarray(k, np.float64).reshape(tokens, hkv, d)
    v = np.asarray(v, np.float64).reshape(tokens, hkv, d)
    out = np.zeros((hq, d))
    rep = hq // hkv
    for h in range(hq):
        s = k[:, h // rep, :] @ q[h] / np.sqrt(d)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, h // rep, :]
    return out.reshape(-1)


def test_attention_patterned_reference_case(oracle):
    # test_ascend_custom_ops.cpp:91-136: T 5, 4 q heads / 2 kv heads, d 16
    T, hq, hkv, d = 5, 4, 2, 16
    q = ((np.arange(hq * d) % 13) - 6).astype(np.float32) * 0.03125
    i = np.arange(T * hkv * d)
    k = ((i % 17) - 8).astype(np.float32) * 0.025
    v = ((i % 11) - 5).astype(np.float32) * 0.0375
    out = oracle.attention_step(q, k, v, T, hq, hkv, d)
    assert rel_err(out, attention_f64(q, k, v, T, hq, hkv, d)) < 1e-5


def test_attention_invariants(oracle):
    rng = np.random.default_rng(1)
    hq, hkv, d = 8, 2, 96
    q = rng.standard_normal(hq * d).astype(np.float32)
    k = rng.standard_normal(1 * hkv * d).astype(np.float32)
    v = rng.standard_normal(1 * hkv * d).astype(np.float32)
    out = oracle.attention_step(q, k, v, 1, hq, hkv, d).reshape(hq, d)
    for h in range(hq):  # one key: output is that key's value row (GQA head h // 4)
        np.testing.assert_allclose(out[h], v.reshape(hkv, d)[h // 4], rtol=1e-6)
    T = 300
    k = (rng.standard_normal(T * hkv * d) * 3).astype(np.float32)  # large scores: needs max subtraction
    v = rng.standard_normal(T * hkv * d).astype(np.float32)
    out = oracle.attention_step(q, k, v, T, hq, hkv, d)
    assert rel_err(out, attention_f64(q, k, v, T, hq, hkv, d)) < 1e-5
    assert np.all(np.isfinite(out))


def test_matvec_brute_force(oracle):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((37, 24)).astype(np.float32)
    x = rng.standard_normal(24).astype(np.float32)
    out = oracle.matvec(w, x)
    assert rel_err(out, w.astype(np.float64) @ x.astype(np.float64)) < 1e-6
    assert rel_err(out[:24], w.T[:24, :24].astype(np.float64) @ x) > 1e-2  # transposed operand fails


def test_argmax_first_maximum(oracle):
    assert oracle.argmax([1.0, 3.0, 2.0, 3.0]) == 1
    assert oracle.argmax([-1.0, -1.0]) == 0
    assert oracle.argmax([0.0, 0.0, 5.0]) == 2


def test_fp16_conversion_matches_ieee_rne(oracle):
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 0.02,
        rng.standard_normal(20000).astype(np.float32) * 1000,
        (rng.random(2000).astype(np.float32) * 2 ** -14),          # subnormal halves
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2 ** -25, 2 ** -24, 3 * 2 ** -25], np.float32),
    ])
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, vals.astype(np.float16).view(np.uint16))
    back = np.array([oracle.f16_bits_to_f32(int(h)) for h in got[:5000]], np.float32)
    np.testing.assert_array_equal(back, got[:5000].view(np.float16).astype(np.float32))


# ---- model-level: bit-identical to the reference build ----------------------------

def _model_dir(mmr, tmp_path, g):
    cfg = mmr.make_config(**g["config"])
    d = tmp_path / g["case"]
    mmr.write_synthetic_model(d, cfg, g["seed"], g["std"], g["round_fp16"])
    if g["strip_keys"]:
        p = d / "minimind_runtime_config.txt"
        p.write_text("\n".join(l for l in p.read_text().splitlines() if l.split("=")[0] not in g["strip_keys"]) + "\n")
    return d


@pytest.mark.parametrize("case", ["mini", "cfg0", "cfg3_short"])
def test_oracle_reproduces_reference_build(mmr, oracle, tmp_path, case):
    g = load_golden(case)
    d = _model_dir(mmr, tmp_path, g)
    m = oracle.OracleModel(d)
    assert m.generate(g["prompt"], g["max_new"]) == g["generated"]
    st = m.new_state()
    lg = None
    for t in g["prompt"]:
        lg = st.forward_token(t)
    rows = []
    for i, tok in enumerate(g["generated"]):
        if i in g["logit_steps"]:
            rows.append(lg)
        if i + 1 < len(g["generated"]):
            lg = st.forward_token(tok)
    np.testing.assert_array_equal(np.array(rows), g["logits"])  # bit-identical
    assert st.position == len(g["prompt"]) + len(g["generated"]) - 1


def test_oracle_loader_defaults(mmr, oracle, tmp_path):
    # config file without rms_norm_eps / rope_theta -> reference defaults (1e-6, 1e6)
    g = load_golden("mini_loader")
    d = _model_dir(mmr, tmp_path, g)
    m = oracle.OracleModel(d)
    assert abs(m.config.rms_norm_eps - 1e-6) < 1e-12
    assert g["eps_used"] == pytest.approx(1e-6)
    assert m.generate(g["prompt"], g["max_new"]) == g["generated"]


def test_oracle_rejects_bad_token(mmr, oracle, tmp_path):
    g = load_golden("mini")
    m = oracle.OracleModel(_model_dir(mmr, tmp_path, g))
    with pytest.raises(IndexError):
        m.new_state().forward_token(g["config"]["vocab_size"])


def test_fp16_weight_rounding_keeps_configs0(mmr, oracle, tmp_path):
    # configs[0]'s fixture has fp32 weights; the GPU runtime stores weights as
    # fp16 (RNE).  On the reference's own CPU arithmetic (the oracle, pinned
    # bit-exact to the reference build above) the rounding keeps every golden
    # token and moves the logits of every step by at most 1e-3 of max|logit|:
    # the GPU's configs[0] test can hold the fp32 golden to the 2e-3 bar.
    g = load_golden("cfg0")
    cfg = mmr.make_config(**g["config"])
    a, b = tmp_path / "fp32", tmp_path / "fp16"
    mmr.write_synthetic_model(a, cfg, g["seed"], g["std"], False)
    mmr.write_synthetic_model(b, cfg, g["seed"], g["std"], True)
    ra, rb = oracle.OracleModel(a), oracle.OracleModel(b)
    assert rb.generate(g["prompt"], g["max_new"]) == g["generated"]
    sa, sb = ra.new_state(), rb.new_state()
    worst = 0.0
    for t in (g["prompt"] + g["generated"])[:-1]:
        la, lb = sa.forward_token(t), sb.forward_token(t)
        worst = max(worst, float(np.max(np.abs(la - lb)) / np.max(np.abs(la))))
    assert 0.0 < worst < 1e-3, worst
