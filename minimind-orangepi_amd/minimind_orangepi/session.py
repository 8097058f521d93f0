"""Text generation session over the runtime's `minimind_generate` tool.

Same API and protocol as the reference's src/python/minimind_orangepi/session.py
(GenerationResult :9-19, chat_prompt :22-25, chat_prompt_from_history :28-49,
validate_runtime_model_dir :52-61, the token-line parsers :64-81, TextSession
:84-213), so existing callers switch by pointing `executable` at this
runtime's bin/minimind_generate (the default here).

Protocol of the tool: "prompt_tokens: ..." first, then with --stream one
"token: N" line per generated token as it is produced, then
"generated_tokens: ...".  With a tokenizer.json in the model directory the
prompt is wrapped in the MiniMind chat markers (unless raw) and encoded here;
otherwise the raw text goes to the tool, which maps its bytes into the
vocabulary.

Difference: the gfx950 tool has no built-in toy model (its shapes, hidden 4
and head_dim 2, are below what the device kernels implement), so `model` must
name a runtime model directory; None makes the tool exit with status 2, which
surfaces as subprocess.CalledProcessError.
"""
from __future__ import annotations

import subprocess
from dataclasses import dataclass
from pathlib import Path
from typing import Iterator, Sequence

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
DEFAULT_EXECUTABLE = PACKAGE_ROOT / "bin" / "minimind_generate"


@dataclass(frozen=True)
class GenerationResult:
    raw_output: str
    prompt_tokens: list[int]
    generated_tokens: list[int]
    generated_text: str | None = None

    def format(self) -> str:
        if self.generated_text is None:
            return self.raw_output
        return f"{self.raw_output}generated_text: {self.generated_text}\n"


def chat_prompt(prompt: str, open_thinking: bool = False) -> str:
    """One user turn in the MiniMind chat markers, opening the assistant turn."""
    head = f"<|im_start|>user\n{prompt}<|im_end|>\n<|im_start|>assistant\n"
    return head + "<think>\n" if open_thinking else head


def chat_prompt_from_history(history: Sequence[tuple[str, str | None]], open_thinking: bool = False) -> str:
    """Several turns; the last turn's assistant text (if any) is closed and a
    new assistant turn is opened (with <think> when open_thinking)."""
    if not history:
        raise ValueError("history cannot be empty")
    out = []
    last = len(history) - 1
    for i, (user, assistant) in enumerate(history):
        if not user.strip():
            raise ValueError("history contains an empty user message")
        out.append(f"<|im_start|>user\n{user}<|im_end|>\n")
        if assistant:
            out.append(f"<|im_start|>assistant\n{assistant}<|im_end|>\n")
        if i == last:
            out.append("<|im_start|>assistant\n<think>\n" if open_thinking else "<|im_start|>assistant\n")
    return "".join(out)


def validate_runtime_model_dir(model: Path | None) -> None:
    if model is None:
        return
    model = Path(model)
    if not model.exists():
        raise FileNotFoundError(f"model directory does not exist: {model}")
    if not model.is_dir():
        raise NotADirectoryError(f"model path is not a directory: {model}")
    missing = [n for n in ("minimind_runtime_config.txt", "weights.bin") if not (model / n).exists()]
    if missing:
        raise ValueError(f"invalid MiniMind text runtime model directory {model}; missing: {', '.join(missing)}")


def parse_token_values(value: str) -> list[int]:
    return [int(v) for v in value.split()]


def parse_token_line(output: str, label: str) -> list[int]:
    prefix = label + ":"
    for line in output.splitlines():
        if line.startswith(prefix):
            return parse_token_values(line[len(prefix):])
    raise ValueError(f"missing {label} in runtime output")


def parse_stream_token_line(line: str) -> int:
    if not line.startswith("token:"):
        raise ValueError("missing token line")
    values = parse_token_values(line[len("token:"):])
    if len(values) != 1:
        raise ValueError("stream token line must contain exactly one token")
    return values[0]


class TextSession:
    def __init__(self, executable: Path | None = None, model: Path | None = None) -> None:
        self.executable = Path(executable) if executable else DEFAULT_EXECUTABLE
        self.model = Path(model) if model is not None else None
        validate_runtime_model_dir(self.model)

    def _load_tokenizer(self):
        if self.model is None or not (self.model / "tokenizer.json").exists():
            return None
        try:
            from tokenizers import Tokenizer
        except ImportError as exc:
            raise RuntimeError("tokenizer.json requires the tokenizers package") from exc
        return Tokenizer.from_file(str(self.model / "tokenizer.json"))

    def _command(self, prompt: str, max_new_tokens: int, raw_prompt: bool, open_thinking: bool, stream: bool):
        cmd = [str(self.executable), "--max-new-tokens", str(max_new_tokens)]
        if stream:
            cmd.append("--stream")
        if self.model is not None:
            cmd += ["--model", str(self.model)]
        tokenizer = self._load_tokenizer()
        if tokenizer is None:
            cmd += ["--prompt", prompt]
        else:
            text = prompt if raw_prompt else chat_prompt(prompt, open_thinking)
            cmd += ["--tokens", ",".join(str(t) for t in tokenizer.encode(text).ids)]
        return cmd, tokenizer

    @staticmethod
    def _result(raw: str, prompt_tokens: list[int], generated: list[int], tokenizer) -> GenerationResult:
        text = tokenizer.decode(generated) if tokenizer is not None else None
        return GenerationResult(raw, list(prompt_tokens), list(generated), text)

    def generate_result(self, prompt: str, max_new_tokens: int = 8, raw_prompt: bool = False,
                        open_thinking: bool = False) -> GenerationResult:
        cmd, tokenizer = self._command(prompt, max_new_tokens, raw_prompt, open_thinking, False)
        done = subprocess.run(cmd, check=True, capture_output=True, text=True)
        return self._result(done.stdout, parse_token_line(done.stdout, "prompt_tokens"),
                            parse_token_line(done.stdout, "generated_tokens"), tokenizer)

    def stream_generate_result(self, prompt: str, max_new_tokens: int = 8, raw_prompt: bool = False,
                               open_thinking: bool = False) -> Iterator[GenerationResult]:
        """Yields a result after every streamed token and after the final line."""
        cmd, tokenizer = self._command(prompt, max_new_tokens, raw_prompt, open_thinking, True)
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, bufsize=1)
        raw: list[str] = []
        prompt_tokens: list[int] = []
        generated: list[int] = []
        try:
            for line in proc.stdout:
                raw.append(line)
                s = line.strip()
                if s.startswith("prompt_tokens:"):
                    prompt_tokens = parse_token_values(s.split(":", 1)[1])
                elif s.startswith("token:"):
                    generated.append(parse_stream_token_line(s))
                    yield self._result("".join(raw), prompt_tokens, generated, tokenizer)
                elif s.startswith("generated_tokens:"):
                    generated = parse_token_values(s.split(":", 1)[1])
                    yield self._result("".join(raw), prompt_tokens, generated, tokenizer)
            stderr = proc.stderr.read() if proc.stderr is not None else ""
            code = proc.wait()
        except BaseException:
            proc.kill()
            proc.wait()
            raise
        if code != 0:
            raise subprocess.CalledProcessError(code, cmd, output="".join(raw), stderr=stderr)

    def stream_generate_chat_result(self, history: Sequence[tuple[str, str | None]], max_new_tokens: int = 8,
                                    open_thinking: bool = False) -> Iterator[GenerationResult]:
        yield from self.stream_generate_result(chat_prompt_from_history(history, open_thinking), max_new_tokens,
                                               True, False)

    def generate(self, prompt: str, max_new_tokens: int = 8, raw_prompt: bool = False,
                 open_thinking: bool = False) -> str:
        return self.generate_result(prompt, max_new_tokens, raw_prompt, open_thinking).format()
