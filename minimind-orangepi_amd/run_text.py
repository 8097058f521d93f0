#!/usr/bin/env python3
"""Run MiniMind text generation on the gfx950 runtime.

    python run_text.py --model RUNTIME_DIR [--prompt TEXT] [--max-new-tokens N]
                       [--raw-prompt] [--open-thinking] [--executable PATH]

Same flags and output as the reference's src/python/tools/run_text.py; the
default executable is this runtime's bin/minimind_generate.
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

from minimind_orangepi.session import TextSession  # noqa: E402


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Run MiniMind text generation on the local runtime")
    ap.add_argument("--model", type=Path, default=None, help="Runtime model directory exported by export_minimind_runtime.py")
    ap.add_argument("--prompt", default="MiniMind")
    ap.add_argument("--max-new-tokens", type=int, default=8)
    ap.add_argument("--raw-prompt", action="store_true", help="Do not wrap the prompt in MiniMind chat markers")
    ap.add_argument("--open-thinking", action="store_true", help="Start the assistant response with a <think> marker")
    ap.add_argument("--executable", type=Path, default=None)
    args = ap.parse_args(argv)
    session = TextSession(args.executable, args.model)
    print(session.generate(args.prompt, args.max_new_tokens, args.raw_prompt, args.open_thinking), end="")
    return 0


if __name__ == "__main__":
    sys.exit(main())
