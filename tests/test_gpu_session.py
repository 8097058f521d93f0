"""minimind_generate and the Python session on a real model directory: the
tool's stdout protocol (the reference's tests/integration/test_text_generate.py
cases) and TextSession's results against the in-process model."""
from __future__ import annotations

import subprocess
import sys

import pytest

from conftest import ROOT, load_golden

pytestmark = pytest.mark.gpu
sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
from minimind_orangepi.session import DEFAULT_EXECUTABLE, TextSession  # noqa: E402


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory, gpu):
    g = load_golden("mini")
    d = tmp_path_factory.mktemp("mini_model")
    gpu.write_synthetic_model(d, gpu.make_config(**g["config"]), g["seed"], g["std"], g["round_fp16"])
    return d


def run_tool(*args):
    return subprocess.run([str(DEFAULT_EXECUTABLE), *args], check=True, capture_output=True, text=True,
                          timeout=120).stdout


def test_tool_explicit_tokens_blocking_and_streaming(gpu, model_dir):
    g = load_golden("mini")
    toks = ",".join(map(str, g["prompt"]))
    out = run_tool("--model", str(model_dir), "--tokens", toks, "--max-new-tokens", "6")
    assert f"prompt_tokens: {' '.join(map(str, g['prompt']))}" in out and "token: " not in out
    gen = [int(t) for t in next(l for l in out.splitlines() if l.startswith("generated_tokens:")).split(":")[1].split()]
    assert gen == g["generated"][:6]
    out = run_tool("--model", str(model_dir), "--tokens", toks, "--max-new-tokens", "6", "--stream")
    streamed = [int(l.split(":")[1]) for l in out.splitlines() if l.startswith("token: ")]
    assert streamed == gen


def test_session_stream_matches_blocking_and_model(gpu, model_dir):
    session = TextSession(model=model_dir)
    streamed = list(session.stream_generate_result("hi", 5))
    blocking = session.generate_result("hi", 5)
    assert streamed and streamed[-1].generated_tokens == blocking.generated_tokens
    assert streamed[-1].prompt_tokens == blocking.prompt_tokens
    assert [r.generated_tokens for r in streamed[:-1]] == [blocking.generated_tokens[: i + 1] for i in range(5)]
    m = gpu.Model.load(model_dir)
    assert m.generate(blocking.prompt_tokens, 5) == blocking.generated_tokens
    chat = list(session.stream_generate_chat_result([("hi", "hello"), ("who are you", "")], 3))
    assert chat[-1].generated_tokens and chat[-1].prompt_tokens


def test_session_with_tokenizer(gpu, model_dir, tmp_path):
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import Tokenizer, models, pre_tokenizers
    words = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "user", "assistant", "hello", "world", "\n"]
    vocab = {w: i for i, w in enumerate(words)}
    tok = Tokenizer(models.WordLevel(vocab, unk_token="<|endoftext|>"))
    tok.pre_tokenizer = pre_tokenizers.Split(pattern=tokenizers.Regex(r"<\|[a-z_]+\|>|\n|[a-z]+"),
                                             behavior="isolated")
    d = tmp_path / "model"
    d.mkdir()
    for f in ("minimind_runtime_config.txt", "weights.bin"):
        (d / f).write_bytes((model_dir / f).read_bytes())
    tok.save(str(d / "tokenizer.json"))
    session = TextSession(model=d)
    r = session.generate_result("hello world", 4)
    expect = tok.encode("<|im_start|>user\nhello world<|im_end|>\n<|im_start|>assistant\n").ids
    assert r.prompt_tokens == expect
    assert r.generated_text == tok.decode(r.generated_tokens)
    raw = session.generate_result("hello world", 4, raw_prompt=True)
    assert raw.prompt_tokens == tok.encode("hello world").ids


def test_run_text_cli(gpu, model_dir):
    out = subprocess.run([sys.executable, str(ROOT / "minimind-orangepi_amd" / "run_text.py"), "--model",
                          str(model_dir), "--prompt", "hi", "--max-new-tokens", "2"],
                         check=True, capture_output=True, text=True, timeout=120).stdout
    assert "generated_tokens:" in out


@pytest.mark.parametrize("device_loop", ["0", "1"])
def test_bench_decode_tool(gpu, model_dir, device_loop):
    # bench_decode.cpp:61-151: flags --input-tokens / --tokens / --warmup and the
    # eight key=value output lines, decode_steps = tokens - 1
    out = subprocess.run([str(ROOT / "minimind-orangepi_amd" / "bin" / "bench_decode"), "--model", str(model_dir),
                          "--input-tokens", "1,2,3", "--tokens", "8", "--warmup", "1", "--device-loop", device_loop],
                         check=True, capture_output=True, text=True, timeout=120).stdout
    kv = dict(line.split("=", 1) for line in out.splitlines() if "=" in line)
    assert list(kv) == ["prompt_tokens", "generated_tokens", "prefill_tokens", "prefill_seconds",
                        "prefill_tokens_per_second", "decode_steps", "decode_seconds", "decode_tokens_per_second"]
    assert kv["prompt_tokens"] == "3" and kv["generated_tokens"] == "8" and kv["decode_steps"] == "7"
    assert float(kv["decode_tokens_per_second"]) > 0
