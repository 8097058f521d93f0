"""The reference's built-in toy model (make_toy_language_model,
language_model.cpp:415-470: hidden 4, head_dim 2, vocab 8) on the GPU's
small-model step kernel, and the callers that fall back to it when no model
directory is given: minimind_generate, bench_decode, run_text.py and
TextSession.  Cases re-expressed from the reference's
tests/unit/test_language_model.cpp:14-33,
tests/integration/test_text_generate.py:7-65 and
tests/integration/test_text_session.py:107-124.

Parity: tokens identical to the oracle (the reference CPU path's arithmetic)
on the same toy weights; logits within max|d| / max|ref| <= 2e-3 (the GPU
holds the weights in fp16, so the toy's 0.2 and 0.1 entries round by up to
2.4e-4 relative).
"""
from __future__ import annotations

import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT, rel_err

pytestmark = pytest.mark.gpu
BIN = ROOT / "minimind-orangepi_amd" / "bin"
sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
from minimind_orangepi.session import TextSession  # noqa: E402


@pytest.fixture(scope="module")
def toy(gpu, oracle, tmp_path_factory):
    d = tmp_path_factory.mktemp("toy")
    gpu.write_toy_model(d)
    return gpu.Model.toy(), oracle.OracleModel(d), d


def run(argv):
    return subprocess.run([str(a) for a in argv], check=True, capture_output=True, text=True, timeout=120).stdout


def test_toy_model_generates_like_the_reference(toy):
    # test_language_model.cpp:14-33: generate({1, 2}, 4) gives 1..4 in-vocabulary ids;
    # an empty prompt raises invalid_argument
    mmr = sys.modules["mmr"]
    model, ref, _ = toy
    assert model.config.hidden_size == 4 and model.config.head_dim == 2 and model.config.vocab_size == 8
    got = model.generate([1, 2], 4)
    assert 1 <= len(got) <= 4 and all(0 <= t < 8 for t in got)
    assert got == ref.generate([1, 2], 4)
    with pytest.raises(mmr.InvalidArgument):
        model.generate([], 1)


@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_toy_model_logits_and_tokens_match_oracle(toy, kv):
    mmr = sys.modules["mmr"]
    model, ref, _ = toy
    for prompt in ([1, 2], [0, 1], [5, 1, 6, 1, 5, 1, 6, 4], [1, 2, 3, 4, 5, 6, 7], [3] * 12):
        assert model.generate(prompt, 8) == ref.generate(prompt, 8), prompt
        st = model.make_state(len(prompt) + 8, mmr.KV_F16 if kv == "f16" else mmr.KV_F32)
        rs = ref.new_state()
        tok = prompt
        for t in prompt + [7, 6, 5, 4]:
            e = rel_err(st.forward_token(t), rs.forward_token(t))
            assert e < 2e-3, (prompt, t, e)
    # the device loop (hipGraph steps) past the toy's nominal 16 positions:
    # the small-model kernel evaluates RoPE at any position, as the CPU path does
    st = model.make_state(40)
    st.enqueue_prefill([1, 2, 3])
    st.enqueue_decode(30)
    st.synchronize()
    rs = ref.new_state()
    for t in [1, 2]:
        rs.forward_token(t)
    want, lg = [], rs.forward_token(3)
    for _ in range(31):
        want.append(int(np.argmax(lg)))
        lg = rs.forward_token(want[-1])
    assert st.read_sequence(3, 31).tolist() == want


def test_toy_model_errors(toy):
    mmr = sys.modules["mmr"]
    model, _, _ = toy
    st = model.make_state(4)
    with pytest.raises(mmr.OutOfRange):
        st.forward_next_token(8)
    for t in range(4):
        st.forward_next_token(t)
    with pytest.raises(mmr.LengthError):
        st.forward_next_token(1)
    with pytest.raises(mmr.InvalidArgument):
        model.make_batch_state(2, 8)
    with pytest.raises(mmr.InvalidArgument):
        model.make_state(4096)


def test_minimind_generate_without_model_explicit_tokens(toy):
    # test_text_generate.py:26-45
    out = run([BIN / "minimind_generate", "--tokens", "1,2", "--max-new-tokens", "2"])
    assert "prompt_tokens: 1 2" in out
    assert "token: " not in out
    assert "generated_tokens:" in out
    gen = [int(t) for t in next(l for l in out.splitlines() if l.startswith("generated_tokens:")).split(":")[1].split()]
    assert gen == toy[1].generate([1, 2], 2)


def test_minimind_generate_without_model_streams(toy):
    # test_text_generate.py:48-65
    out = run([BIN / "minimind_generate", "--tokens", "1,2", "--max-new-tokens", "2", "--stream"])
    token_lines = [l for l in out.splitlines() if l.startswith("token: ")]
    generated = next(l for l in out.splitlines() if l.startswith("generated_tokens:")).split(":", 1)[1].split()
    assert "prompt_tokens: 1 2" in out
    assert token_lines and len(token_lines) == len(generated)


def test_run_text_without_model(toy):
    # test_text_generate.py:7-23
    out = run([sys.executable, ROOT / "minimind-orangepi_amd" / "run_text.py", "--prompt", "hi",
               "--max-new-tokens", "2"])
    assert "generated_tokens:" in out
    assert "prompt_tokens: 0 1" in out  # the bytes of "hi" folded into the toy's 8 ids


def test_session_toy_stream_matches_blocking(toy):
    # test_text_session.py:107-114
    session = TextSession(BIN / "minimind_generate", None)
    streamed = list(session.stream_generate_result("hi", 3))
    blocking = session.generate_result("hi", 3)
    assert streamed
    assert streamed[-1].generated_tokens == blocking.generated_tokens
    assert streamed[-1].prompt_tokens == blocking.prompt_tokens


def test_session_toy_streams_chat_history(toy):
    # test_text_session.py:117-124
    session = TextSession(BIN / "minimind_generate", None)
    streamed = list(session.stream_generate_chat_result([("hi", "hello"), ("who are you", "")], 3))
    assert streamed
    assert streamed[-1].generated_tokens
    assert streamed[-1].prompt_tokens


def test_bench_decode_without_model(toy):
    # bench_decode.cpp:117-151 with the toy fallback and its defaults
    # (prompt "hello", 16 tokens): the eight keys, decode_steps = tokens - 1
    out = run([BIN / "bench_decode"])
    kv = dict(line.split("=", 1) for line in out.splitlines() if "=" in line)
    assert kv["prompt_tokens"] == "5" and kv["generated_tokens"] == "16" and kv["decode_steps"] == "15"
    assert float(kv["decode_tokens_per_second"]) > 0


@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_check_prefill_consistency_tool(gpu, tmp_path, kv):
    # bench/check_prefill_consistency.cpp:9-57 on exported model directories:
    # the GEMM prefill path (mini) and a configs[2]-shaped layer (d 96)
    from conftest import load_golden
    for case, n in (("mini", "40"), ("long4k", "510")):  # ids (i % 1000) + 1 stay inside vocab 512
        g = load_golden(case)
        d = tmp_path / f"{case}_{kv}"
        gpu.write_synthetic_model(d, gpu.make_config(**g["config"]), g["seed"], g["std"], g["round_fp16"])
        out = run([BIN / "check_prefill_consistency", d, n, "--kv", kv])
        assert "prefill consistency ok" in out
    with pytest.raises(subprocess.CalledProcessError):
        run([BIN / "check_prefill_consistency"])
