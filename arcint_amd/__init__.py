"""arcint_amd: ggml's quantized MUL_MAT / MUL_MAT_ID for MI355X (gfx950).

The product is libqmm.so (HIP kernels + a C ABI, include/qmm.h); this
package holds its sources (csrc/), the in-tree build (build.py), the ctypes
binding shaped like a ggml backend (qmm.py) and the seeded synthetic inputs
the benchmarks use (synth.py).
"""
from . import synth  # noqa: F401

__all__ = ["synth"]
