"""The interface identity of include/cairn_gemm.h.

CAIRN's header generator names a library's identity symbol cairn_interface_<library>_<h>, where h is the first 16
hex digits of the SHA-256 of the interface the header states (src/cairn/compiler/lower/header.py:280-285); the
library defines the symbol and the header refers to it, so a program built against another version of the header
fails to link. This header's stated interface is its text between the `cairn:stated-begin` and `cairn:stated-end`
markers, byte for byte (declarations, types and the comments that state their meaning).

    python -m cairn_amd.identity           print the identity the header's text gives
    python -m cairn_amd.identity --write   rewrite the header's CAIRN_GEMM_IDENTITY line to it
"""

from __future__ import annotations

import hashlib
import re
import sys
from pathlib import Path

HEADER = Path(__file__).resolve().parents[1] / "include" / "cairn_gemm.h"
LIBRARY_NAME = "gemm_gfx950"
BEGIN, END = "/* cairn:stated-begin */\n", "/* cairn:stated-end */\n"
DEFINE = re.compile(r"^#define CAIRN_GEMM_IDENTITY (\w+)$", re.M)


def stated(text: str) -> str:
    """The header's stated interface: the text strictly between the two markers."""
    first = text.index(BEGIN) + len(BEGIN)
    return text[first : text.index(END, first)]


def derived(text: str | None = None) -> str:
    """The identity the header's stated interface gives."""
    text = HEADER.read_text() if text is None else text
    return f"cairn_interface_{LIBRARY_NAME}_{hashlib.sha256(stated(text).encode()).hexdigest()[:16]}"


def declared(text: str | None = None) -> str:
    """The identity the header's CAIRN_GEMM_IDENTITY line names."""
    text = HEADER.read_text() if text is None else text
    found = DEFINE.search(text)
    if not found:
        raise ValueError(f"{HEADER}: no CAIRN_GEMM_IDENTITY line")
    return found.group(1)


def check() -> str:
    """The identity, or an error if the header's line is stale (its declarations changed since it was written)."""
    want, have = derived(), declared()
    if want != have:
        raise RuntimeError(f"{HEADER.name}: CAIRN_GEMM_IDENTITY is {have}, its stated interface gives {want}: "
                           "run python -m cairn_amd.identity --write")  # fmt: skip
    return have


def write() -> str:
    text = HEADER.read_text()
    want = derived(text)
    HEADER.write_text(DEFINE.sub(f"#define CAIRN_GEMM_IDENTITY {want}", text, count=1))
    return want


if __name__ == "__main__":
    print(write() if "--write" in sys.argv[1:] else derived())
