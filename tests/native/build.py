"""Builds the native test drivers under tests/native/ (test infrastructure, like
the oracle): each ``<name>.cpp`` becomes the executable ``<name>`` beside it.
They bind the product libraries with dlopen at run time and link nothing of
them."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent


def build() -> None:
    for src in sorted(HERE.glob("*.cpp")):
        subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", str(src), "-ldl",
                        "-o", str(src.with_suffix(""))], check=True)


if __name__ == "__main__":
    build()
