"""Writes the GGUF fixtures of tests/golden/.

gguf_model_file.gguf and gguf_model_file_legacy.gguf are the two files the
reference's GgufModelFileTests.CreateModel builds
(SharpInference.Gguf.Tests/GgufModelFileTests.cs:56-84): metadata
general.architecture = "test" and test.values = [0.5, 0.25, -1] (f32
array, with a 64-bit count, or a 32-bit count in the legacy file), one
Float16 tensor "weight" of dims [2] holding 1 and 2 at offset 0 of a
32-byte aligned data section.  The expected parse results are asserted in
tests/test_gguf.py (GgufModelFileTests.cs:14-24).

    python tests/golden/make_gguf_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from sharpinference_amd import gguf  # noqa: E402


def main():
    meta = {"general.architecture": (gguf.STRING, "test"),
            "test.values": (gguf.ARRAY, gguf.F32, [0.5, 0.25, -1.0])}
    weight = np.array([1.0, 2.0], np.float16)
    for name, legacy in (("gguf_model_file.gguf", False), ("gguf_model_file_legacy.gguf", True)):
        gguf.write_gguf(os.path.join(HERE, name), meta, [("weight", 1, [2], weight)], legacy_array_count=legacy)


if __name__ == "__main__":
    main()
