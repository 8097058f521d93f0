"""The Python caller of minimind_generate (minimind_orangepi.session), on the
CPU: chat markers, token-line parsing and model-directory validation, with
the cases of the reference's tests/integration/test_text_session.py."""
from __future__ import annotations

import sys

import pytest

from conftest import ROOT

sys.path.insert(0, str(ROOT / "minimind-orangepi_amd"))
from minimind_orangepi.session import (  # noqa: E402
    GenerationResult, chat_prompt, chat_prompt_from_history,
    parse_stream_token_line, parse_token_line, validate_runtime_model_dir)


def test_parse_token_line():
    out = "prompt_tokens: 1 2\ngenerated_tokens: 3 4\n"
    assert parse_token_line(out, "prompt_tokens") == [1, 2]
    assert parse_token_line(out, "generated_tokens") == [3, 4]
    assert parse_token_line("generated_tokens:\n", "generated_tokens") == []
    with pytest.raises(ValueError, match="missing prompt_tokens"):
        parse_token_line("generated_tokens: 1\n", "prompt_tokens")


def test_parse_stream_token_line():
    assert parse_stream_token_line("token: 42") == 42
    with pytest.raises(ValueError):
        parse_stream_token_line("generated_tokens: 42")
    with pytest.raises(ValueError):
        parse_stream_token_line("token: 1 2")


def test_generation_result_format():
    r = GenerationResult("prompt_tokens: 1\ngenerated_tokens: 2\n", [1], [2], "hello")
    assert r.format().endswith("generated_text: hello\n")
    assert GenerationResult("x\n", [1], [2]).format() == "x\n"


def test_chat_markers():
    assert chat_prompt("你好") == "<|im_start|>user\n你好<|im_end|>\n<|im_start|>assistant\n"
    assert chat_prompt("你好", open_thinking=True).endswith("assistant\n<think>\n")
    assert chat_prompt_from_history([("你好", "")]) == chat_prompt("你好")
    assert chat_prompt_from_history([("你好", "您好"), ("你是谁", "")]) == (
        "<|im_start|>user\n你好<|im_end|>\n<|im_start|>assistant\n您好<|im_end|>\n"
        "<|im_start|>user\n你是谁<|im_end|>\n<|im_start|>assistant\n")
    thinking = chat_prompt_from_history([("你好", "您好"), ("继续", "")], open_thinking=True)
    assert thinking.count("<think>") == 1 and thinking.endswith("<|im_start|>assistant\n<think>\n")
    closed = chat_prompt_from_history([("a", "b")])
    assert closed.endswith("<|im_start|>assistant\nb<|im_end|>\n<|im_start|>assistant\n")
    with pytest.raises(ValueError, match="history cannot be empty"):
        chat_prompt_from_history([])
    with pytest.raises(ValueError, match="empty user message"):
        chat_prompt_from_history([(" ", "x")])


def test_validate_runtime_model_dir(tmp_path):
    validate_runtime_model_dir(None)
    with pytest.raises(FileNotFoundError):
        validate_runtime_model_dir(tmp_path / "missing")
    f = tmp_path / "file"
    f.write_text("x")
    with pytest.raises(NotADirectoryError):
        validate_runtime_model_dir(f)
    d = tmp_path / "model"
    d.mkdir()
    with pytest.raises(ValueError, match="minimind_runtime_config.txt"):
        validate_runtime_model_dir(d)
    (d / "minimind_runtime_config.txt").write_text("hidden_size=4\n")
    with pytest.raises(ValueError, match="weights.bin"):
        validate_runtime_model_dir(d)
    (d / "weights.bin").write_bytes(b"MMRTW001")
    validate_runtime_model_dir(d)
