"""Writes tests/golden/reference_ffi_symbols.txt: the C symbols the reference's
ctypes wrapper binds for the YOLO model path (NativeCppYoloModel._configure,
src/aexrt/cpp_runtime.py:543-662), one per line.

The names are read from the wrapper's source text (every ``self.lib.<name>``
in that method); nothing of the reference is imported or run.  The library
built here must export every one of them (tests/test_packing_abi.py).
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = Path("/root/reference/src/aexrt/cpp_runtime.py")


def main() -> int:
    text = SOURCE.read_text(encoding="utf-8")
    start = text.index("    def _configure(self) -> None:", text.index("class NativeCppYoloModel"))
    end = text.index("\ndef ", start)
    names = sorted(set(re.findall(r"self\.lib\.(\w+)\.", text[start:end])))
    (HERE / "reference_ffi_symbols.txt").write_text("\n".join(names) + "\n")
    print(f"{len(names)} symbols")
    return 0


if __name__ == "__main__":
    sys.exit(main())
