#!/usr/bin/env python3
"""Command-line entry of the verify.py scoring contract for this library.

    python verify.py --op silu --case-module NKIBench/reference/silu_....py
    python verify.py --pilot --nkibench-root ../AccelOpt/NKIBench

Same options and output as ``python -m kda.verify`` (kda-for-trainium_amd/kda/verify.py).
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent / "kda-for-trainium_amd"))

from kda.verify import main  # noqa: E402

if __name__ == "__main__":
    sys.exit(main())
