"""Python front end of the runtime's `minimind_generate` tool.

The public names are the ones callers of the reference use
(src/python/minimind_orangepi/session.py:9-213): GenerationResult,
chat_prompt, chat_prompt_from_history, validate_runtime_model_dir,
parse_token_values, parse_token_line, parse_stream_token_line and
TextSession with generate / generate_result / stream_generate_result /
stream_generate_chat_result.  What they exchange with the tool is its stdout
protocol:

    prompt_tokens: 1 2 3          always first
    token: 17                     one per generated id, only with --stream
    generated_tokens: 17 42 ...   always last

Prompt text reaches the tool in one of two ways.  When the model directory
holds a tokenizer.json (and the `tokenizers` package is importable) the text
is wrapped in the MiniMind chat template unless raw, encoded here, and passed
as --tokens; the generated ids are decoded back into `generated_text`.
Otherwise the text goes as --prompt and the tool folds its bytes into the
vocabulary.  Without a model directory the tool runs the reference's built-in
toy model (on the GPU, like any other model).
"""
from __future__ import annotations

import subprocess
from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterator, Sequence

DEFAULT_EXECUTABLE = Path(__file__).resolve().parents[1] / "bin" / "minimind_generate"
RUNTIME_FILES = ("minimind_runtime_config.txt", "weights.bin")

# MiniMind chat template: every turn is <|im_start|>ROLE\nTEXT<|im_end|>\n and
# the prompt ends with an open assistant turn (optionally already thinking).
_TURN_START, _TURN_END = "<|im_start|>", "<|im_end|>"


def _closed_turn(role: str, text: str) -> str:
    return f"{_TURN_START}{role}\n{text}{_TURN_END}\n"


def _open_assistant(open_thinking: bool) -> str:
    return f"{_TURN_START}assistant\n" + ("<think>\n" if open_thinking else "")


def chat_prompt(prompt: str, open_thinking: bool = False) -> str:
    """A single user message followed by the opened assistant turn."""
    return _closed_turn("user", prompt) + _open_assistant(open_thinking)


def chat_prompt_from_history(history: Sequence[tuple[str, str | None]], open_thinking: bool = False) -> str:
    """A conversation of (user, assistant-or-empty) pairs: each user message,
    each non-empty assistant reply as a closed turn, then one opened
    assistant turn (the only place <think> may appear)."""
    if not history:
        raise ValueError("history cannot be empty")
    text = []
    for user, reply in history:
        if not user.strip():
            raise ValueError("history contains an empty user message")
        text.append(_closed_turn("user", user))
        if reply:
            text.append(_closed_turn("assistant", reply))
    text.append(_open_assistant(open_thinking))
    return "".join(text)


def validate_runtime_model_dir(model: Path | None) -> None:
    """None is allowed (the tool's toy model); a path must be a directory
    holding both runtime files."""
    if model is None:
        return
    model = Path(model)
    if not model.exists():
        raise FileNotFoundError(f"model directory does not exist: {model}")
    if not model.is_dir():
        raise NotADirectoryError(f"model path is not a directory: {model}")
    absent = [name for name in RUNTIME_FILES if not (model / name).is_file()]
    if absent:
        raise ValueError(f"{model} is not a MiniMind text runtime model directory; missing: {', '.join(absent)}")


def parse_token_values(value: str) -> list[int]:
    """Whitespace-separated token ids."""
    return [int(tok) for tok in value.split()]


def parse_token_line(output: str, label: str) -> list[int]:
    """Ids of the first `label:` line of the tool's output."""
    prefix = label + ":"
    for line in output.splitlines():
        if line.startswith(prefix):
            return parse_token_values(line[len(prefix):])
    raise ValueError(f"missing {label} in runtime output")


def parse_stream_token_line(line: str) -> int:
    """The id of one streamed `token: N` line."""
    if not line.startswith("token:"):
        raise ValueError(f"not a streamed token line: {line!r}")
    ids = parse_token_values(line[len("token:"):])
    if len(ids) != 1:
        raise ValueError(f"a streamed token line carries exactly one id, got {len(ids)}")
    return ids[0]


@dataclass(frozen=True)
class GenerationResult:
    raw_output: str
    prompt_tokens: list[int]
    generated_tokens: list[int]
    generated_text: str | None = None

    def format(self) -> str:
        """The tool's output, plus a generated_text line when text was decoded."""
        if self.generated_text is None:
            return self.raw_output
        return f"{self.raw_output}generated_text: {self.generated_text}\n"


@dataclass
class _Transcript:
    """What has been read of one run of the tool so far."""
    lines: list[str] = field(default_factory=list)
    prompt: list[int] = field(default_factory=list)
    generated: list[int] = field(default_factory=list)

    def take(self, line: str) -> bool:
        """Record one stdout line; True when it changed the generated ids."""
        self.lines.append(line)
        body = line.strip()
        if body.startswith("prompt_tokens:"):
            self.prompt = parse_token_values(body.split(":", 1)[1])
        elif body.startswith("token:"):
            self.generated.append(parse_stream_token_line(body))
            return True
        elif body.startswith("generated_tokens:"):
            self.generated = parse_token_values(body.split(":", 1)[1])
            return True
        return False


class TextSession:
    """Greedy generation through `minimind_generate` (one process per call)."""

    def __init__(self, executable: Path | None = None, model: Path | None = None) -> None:
        self.executable = Path(executable) if executable is not None else DEFAULT_EXECUTABLE
        self.model = Path(model) if model is not None else None
        self._tokenizer_cache: tuple[bool, object] = (False, None)

    # ---- tool invocation -------------------------------------------------

    def _tokenizer(self):
        loaded, tok = self._tokenizer_cache
        if loaded:
            return tok
        path = self.model / "tokenizer.json" if self.model is not None else None
        if path is not None and path.is_file():
            try:
                from tokenizers import Tokenizer
            except ImportError as exc:
                raise RuntimeError("tokenizer.json requires the tokenizers package") from exc
            tok = Tokenizer.from_file(str(path))
        self._tokenizer_cache = (True, tok)
        return tok

    def _argv(self, prompt: str, max_new_tokens: int, raw_prompt: bool, open_thinking: bool, stream: bool):
        argv = [str(self.executable), "--max-new-tokens", str(int(max_new_tokens))]
        if self.model is not None:
            argv += ["--model", str(self.model)]
        if stream:
            argv.append("--stream")
        tok = self._tokenizer()
        if tok is None:
            argv += ["--prompt", prompt]
        else:
            text = prompt if raw_prompt else chat_prompt(prompt, open_thinking)
            argv += ["--tokens", ",".join(map(str, tok.encode(text).ids))]
        return argv, tok

    @staticmethod
    def _result(raw: str, prompt: list[int], generated: list[int], tok) -> GenerationResult:
        text = tok.decode(generated) if tok is not None else None
        return GenerationResult(raw, list(prompt), list(generated), text)

    # ---- public API ---------------------------------------------------------

    def generate_result(self, prompt: str, max_new_tokens: int = 8, raw_prompt: bool = False,
                        open_thinking: bool = False) -> GenerationResult:
        argv, tok = self._argv(prompt, max_new_tokens, raw_prompt, open_thinking, stream=False)
        done = subprocess.run(argv, check=True, capture_output=True, text=True)
        return self._result(done.stdout, parse_token_line(done.stdout, "prompt_tokens"),
                            parse_token_line(done.stdout, "generated_tokens"), tok)

    def stream_generate_result(self, prompt: str, max_new_tokens: int = 8, raw_prompt: bool = False,
                               open_thinking: bool = False) -> Iterator[GenerationResult]:
        """One result per streamed token and one for the closing
        generated_tokens line, each with all output read so far."""
        argv, tok = self._argv(prompt, max_new_tokens, raw_prompt, open_thinking, stream=True)
        seen = _Transcript()
        with subprocess.Popen(argv, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, bufsize=1) as proc:
            try:
                for line in proc.stdout:
                    if seen.take(line):
                        yield self._result("".join(seen.lines), seen.prompt, seen.generated, tok)
                err = proc.stderr.read()
                code = proc.wait()
            except BaseException:
                proc.kill()
                raise
        if code != 0:
            raise subprocess.CalledProcessError(code, argv, output="".join(seen.lines), stderr=err)

    def stream_generate_chat_result(self, history: Sequence[tuple[str, str | None]], max_new_tokens: int = 8,
                                    open_thinking: bool = False) -> Iterator[GenerationResult]:
        """The conversation rendered with chat_prompt_from_history, then
        streamed as a raw prompt."""
        yield from self.stream_generate_result(chat_prompt_from_history(history, open_thinking), max_new_tokens,
                                               raw_prompt=True)

    def generate(self, prompt: str, max_new_tokens: int = 8, raw_prompt: bool = False,
                 open_thinking: bool = False) -> str:
        return self.generate_result(prompt, max_new_tokens, raw_prompt, open_thinking).format()
