"""Writes the integration guide's hip_variants.cpp (the translation unit a tiny-llm maintainer
adds: the TINYQWEN_*_VARIANT registrations and the gpu_decode engine adapter) from the C++
blocks of INTEGRATION.md, so what the tests compile and link is the text the guide shows.

usage: python3 extract_binding.py INTEGRATION.md out.cpp   (test infrastructure only)
"""
import re
import sys


def binding_source(text: str) -> str:
    """The guide's C++ blocks that register variants (the registry block and the gpu_decode block)."""
    blocks = [re.sub(r"^  ", "", b, flags=re.M) for b in re.findall(r"```cpp\n(.*?)```", text, flags=re.S)]
    parts = [b for b in blocks if "TINYQWEN_" in b and "VARIANT" in b]
    if len(parts) != 2:
        raise SystemExit(f"expected the registry block and the gpu_decode block, found {len(parts)}")
    return "\n".join(parts)


if __name__ == "__main__":
    src = binding_source(open(sys.argv[1]).read())
    with open(sys.argv[2], "w") as f:
        f.write(src)
