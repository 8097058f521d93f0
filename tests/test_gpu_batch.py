"""GPU parity of batched decode: a batch of independent
sequences in lockstep over a paged KV cache must produce, for every sequence,
the token ids the single-sequence path produces for it alone (which equal the
reference CPU path), with logits within the bound.

Bound: max |batch - single| / max |single| <= 1e-4 for logits (the batch runs
its projections as split-K GEMMs on the fp16 matrix cores with a hi/lo split
of the fp32 activations, the single path as GEMVs); token ids exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import load_golden, rel_err

pytestmark = pytest.mark.gpu


def synth_model(mmr, g, **overrides):
    return mmr.Model.synthetic(mmr.make_config(**{**g["config"], **overrides}), g["seed"], g["std"], g["round_fp16"])


def single_sequence(mmr, m, prompt, last_index, capacity, kv):
    """seq[0 .. last_index] and last-step logits of one sequence decoded alone."""
    st = m.make_state(capacity, kv)
    st.enqueue_prefill(prompt)
    st.enqueue_decode(last_index - len(prompt))
    st.synchronize()
    return st.read_sequence(0, last_index + 1), st.read_logits()


@pytest.mark.parametrize("kv", ["f16", "f32"])
def test_batch_matches_single_sequences(gpu, kv):
    # prompts of different lengths; positions cross 64-token pages and reach
    # more than four attention tiles (two splits per sequence)
    mmr = gpu
    print(f"[case] batch mini kv={kv}", flush=True)
    g = load_golden("mini")
    m = synth_model(mmr, g)
    kvd = mmr.KV_F16 if kv == "f16" else mmr.KV_F32
    rng = np.random.default_rng(11)
    lengths = [70, 5, 130, 33]
    prompts = [[int(t) for t in rng.integers(0, g["config"]["vocab_size"], n)] for n in lengths]
    cap, steps = 320, 170
    bs = m.make_batch_state(len(prompts), cap, kvd)
    bs.prefill(prompts)
    bs.decode(steps)
    bs.synchronize()
    last = max(lengths) + steps
    assert bs.steps == last
    for b, p in enumerate(prompts):
        ref_seq, ref_logits = single_sequence(mmr, m, p, last, cap, kvd)
        got = bs.read_sequence(b, 0, last + 1)
        np.testing.assert_array_equal(got, ref_seq, err_msg=f"sequence {b}")
        assert rel_err(bs.read_logits(b), ref_logits) < 1e-4, b


def test_batch_wide_hidden_takes_eight_qkv_partials(gpu):
    # hidden 1024: no chunk of up to 256 columns tiles K in three, so the QKV
    # projection hands the attention eight split-K partials (the prologue's
    # full variant; MiniMind2 and the mini model take the three-part one)
    mmr = gpu
    print("[case] batch hidden 1024, 16/2 heads of 64, 8 QKV partials", flush=True)
    g = load_golden("mini")
    m = synth_model(mmr, g, hidden_size=1024, num_attention_heads=16, num_key_value_heads=2, head_dim=64,
                    intermediate_size=1024)
    rng = np.random.default_rng(3)
    lengths = [40, 9, 75]
    prompts = [[int(t) for t in rng.integers(0, g["config"]["vocab_size"], n)] for n in lengths]
    cap, steps = 200, 90
    bs = m.make_batch_state(len(prompts), cap, mmr.KV_F16)
    bs.prefill(prompts)
    bs.decode(steps)
    bs.synchronize()
    last = max(lengths) + steps
    for b, p in enumerate(prompts):
        ref_seq, ref_logits = single_sequence(mmr, m, p, last, cap, mmr.KV_F16)
        np.testing.assert_array_equal(bs.read_sequence(b, 0, last + 1), ref_seq, err_msg=f"sequence {b}")
        assert rel_err(bs.read_logits(b), ref_logits) < 1e-4, b


def test_batch_long_context_split_paths(gpu):
    # positions up to 1150: the attention split count per sequence steps
    # through 1, 2, 4, 8 and 16, so the O projection's staging merges 1-4 and
    # 5-8 split partials itself and hands 16 to the combine kernel
    mmr = gpu
    print("[case] batch mini long context", flush=True)
    g = load_golden("mini")
    m = synth_model(mmr, g)
    rng = np.random.default_rng(5)
    lengths = [20, 3]
    prompts = [[int(t) for t in rng.integers(0, g["config"]["vocab_size"], n)] for n in lengths]
    cap, steps = 1200, 1130
    bs = m.make_batch_state(len(prompts), cap, mmr.KV_F16)
    bs.prefill(prompts)
    bs.decode(steps)
    bs.synchronize()
    last = max(lengths) + steps
    for b, p in enumerate(prompts):
        ref_seq, ref_logits = single_sequence(mmr, m, p, last, cap, mmr.KV_F16)
        np.testing.assert_array_equal(bs.read_sequence(b, 0, last + 1), ref_seq, err_msg=f"sequence {b}")
        assert rel_err(bs.read_logits(b), ref_logits) < 1e-4, b


@pytest.mark.parametrize("batch", [17, 40])
def test_batch_sizes_across_gemm_paths(gpu, batch):
    # 17 rows: the split-K GEMMs' second 16-row tile is partly filled; 40 rows
    # (over 32): the projections fall back to the dense GEMM, whose single
    # "partial" the consumers add, with the separate combine and SwiGLU kernels
    mmr = gpu
    print(f"[case] batch mini B={batch}", flush=True)
    g = load_golden("mini")
    m = synth_model(mmr, g)
    rng = np.random.default_rng(batch)
    lengths = [int(n) for n in rng.integers(1, 40, batch)]
    prompts = [[int(t) for t in rng.integers(0, g["config"]["vocab_size"], n)] for n in lengths]
    cap, steps = 96, 50
    bs = m.make_batch_state(batch, cap, mmr.KV_F16)
    bs.prefill(prompts)
    bs.decode(steps)
    bs.synchronize()
    last = max(lengths) + steps
    for b in (0, batch // 2, batch - 1):
        ref_seq, ref_logits = single_sequence(mmr, m, prompts[b], last, cap, mmr.KV_F16)
        np.testing.assert_array_equal(bs.read_sequence(b, 0, last + 1), ref_seq, err_msg=f"sequence {b}")
        assert rel_err(bs.read_logits(b), ref_logits) < 1e-4, b


def test_batch_reproduces_reference_golden(gpu):
    # MiniMind2 (configs[3] weights): sequence 0 holds the cfg3_short prompt,
    # whose greedy continuation is the reference CPU path's golden output
    mmr = gpu
    g = load_golden("cfg3_short")
    m = synth_model(mmr, g)
    rng = np.random.default_rng(3)
    prompts = [g["prompt"], [int(t) for t in rng.integers(0, 6400, 40)], [int(t) for t in rng.integers(0, 6400, 3)]]
    bs = m.make_batch_state(len(prompts), 128, mmr.KV_F32)
    bs.prefill(prompts)
    bs.decode(len(g["generated"]) - 1 + 40 - len(g["prompt"]))
    got = bs.read_sequence(0, len(g["prompt"]), len(g["generated"])).tolist()
    assert got == g["generated"]
    for b in (1, 2):
        last = bs.steps
        ref_seq, _ = single_sequence(mmr, m, prompts[b], last, 128, mmr.KV_F32)
        np.testing.assert_array_equal(bs.read_sequence(b, 0, last + 1), ref_seq)


def test_batch_graph_replays_match_eager(gpu, monkeypatch):
    mmr = gpu
    g = load_golden("mini")
    m = synth_model(mmr, g)
    prompts = [[1, 2, 3], [4, 5, 6, 7, 8, 9], [10]]
    graph = m.make_batch_state(3, 96)
    monkeypatch.setenv("MMR_NO_GRAPH", "1")
    eager = m.make_batch_state(3, 96)
    monkeypatch.delenv("MMR_NO_GRAPH")
    for st in (graph, eager):
        st.prefill(prompts)
        st.decode(80)
        st.synchronize()
    for b in range(3):
        np.testing.assert_array_equal(graph.read_sequence(b, 0, 87), eager.read_sequence(b, 0, 87))
        np.testing.assert_array_equal(graph.read_logits(b), eager.read_logits(b))


def test_batch_l2_warming_leaves_the_step_unchanged(gpu, monkeypatch):
    # The residual + norm launches' L2-warming blocks (MMR_L2_WARM_BLOCKS; off
    # by default in the batched step) only load the next GEMMs' weights: the
    # batched decode with them equals the decode without, bit for bit, on
    # MiniMind2's shapes (split-K GEMMs for qkv, gate_up, down and lm_head).
    mmr = gpu
    print("[case] batch cfg3 B=8, warming on / off", flush=True)
    g = load_golden("cfg3")
    m = synth_model(mmr, g)
    rng = np.random.default_rng(21)
    prompts = [[int(t) for t in rng.integers(0, g["config"]["vocab_size"], n)] for n in (40, 64, 17, 90, 8, 33, 71, 50)]
    states = []
    for warm in ("128", "0"):
        monkeypatch.setenv("MMR_L2_WARM_BLOCKS", warm)
        bs = m.make_batch_state(len(prompts), 160)
        monkeypatch.delenv("MMR_L2_WARM_BLOCKS")
        bs.prefill(prompts)
        bs.decode(60)
        bs.synchronize()
        states.append(bs)
    last = max(len(p) for p in prompts) + 60
    for b in range(len(prompts)):
        np.testing.assert_array_equal(states[0].read_sequence(b, 0, last + 1), states[1].read_sequence(b, 0, last + 1))
        np.testing.assert_array_equal(states[0].read_logits(b), states[1].read_logits(b))


def test_batch_error_behaviour(gpu):
    mmr = gpu
    g = load_golden("mini")
    m = synth_model(mmr, g)
    V = g["config"]["vocab_size"]
    bs = m.make_batch_state(2, 16)
    with pytest.raises(mmr.InvalidArgument, match="one prompt per sequence"):
        bs.prefill([[1, 2]])
    with pytest.raises(mmr.InvalidArgument, match="cannot be empty"):
        bs.prefill([[1], []])
    with pytest.raises(mmr.OutOfRange):
        bs.prefill([[1], [V]])
    with pytest.raises(mmr.InvalidArgument, match="needs prompts"):
        bs.decode(1)
    with pytest.raises(mmr.LengthError):
        bs.prefill([[1] * 17, [2]])
    bs.prefill([[1, 2, 3], [4]])
    with pytest.raises(mmr.LengthError):
        bs.decode(14)  # 3 + 14 > 16 positions
    bs.decode(13)
    bs.synchronize()
    assert bs.steps == 16
    with pytest.raises(mmr.InvalidArgument, match="empty KV caches"):
        bs.prefill([[1], [2]])
    with pytest.raises(mmr.InvalidArgument):
        m.make_batch_state(0, 16)
    with pytest.raises(mmr.OutOfRange):
        bs.read_sequence(2, 0, 1)
