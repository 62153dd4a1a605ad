"""exl3r: Python plumbing over the MI355X (gfx950) fused row-op library.

`exl3r.ffi` mirrors the reference's src/ffi.rs wrappers on torch tensors; `exl3r._lib` loads the
C ABI declared in include/exl3r/rowops.h.  All compute runs in the HIP library."""
from ._lib import (BF16, EDTYPE, EINVAL, F16, F32, I32, I64, OK, ROPE_GPTJ, ROPE_NEOX, ROPE_NONE,
                   Exl3rError, LIB_PATH, NAIVE_PATH, load, load_naive)

__all__ = ["F32", "F16", "BF16", "I32", "I64", "OK", "EINVAL", "EDTYPE", "ROPE_NONE", "ROPE_GPTJ", "ROPE_NEOX",
           "Exl3rError", "LIB_PATH", "NAIVE_PATH", "load", "load_naive"]
