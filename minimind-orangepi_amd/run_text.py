#!/usr/bin/env python3
"""Command-line text generation on the gfx950 runtime.

Flags are the reference tool's (src/python/tools/run_text.py): --model,
--prompt, --max-new-tokens, --raw-prompt, --open-thinking, --executable.  The
output is the generation tool's stdout protocol, with a generated_text line
when the model directory carries a tokenizer.  Without --model the tool runs
the reference's built-in toy model.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

from minimind_orangepi.session import TextSession  # noqa: E402


def parse_args(argv=None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(prog="run_text.py",
                                 description="Greedy MiniMind text generation through minimind_generate")
    ap.add_argument("--model", type=Path, default=None,
                    help="directory with minimind_runtime_config.txt and weights.bin (default: the toy model)")
    ap.add_argument("--prompt", default="MiniMind", help="prompt text (default: %(default)s)")
    ap.add_argument("--max-new-tokens", type=int, default=8, help="tokens to generate (default: %(default)s)")
    ap.add_argument("--raw-prompt", action="store_true", help="send the text as is, no chat template")
    ap.add_argument("--open-thinking", action="store_true", help="open the assistant turn with <think>")
    ap.add_argument("--executable", type=Path, default=None, help="minimind_generate to run (default: this runtime's)")
    return ap.parse_args(argv)


def main(argv=None) -> int:
    opts = parse_args(argv)
    session = TextSession(opts.executable, opts.model)
    sys.stdout.write(session.generate(opts.prompt, opts.max_new_tokens, opts.raw_prompt, opts.open_thinking))
    return 0


if __name__ == "__main__":
    sys.exit(main())
