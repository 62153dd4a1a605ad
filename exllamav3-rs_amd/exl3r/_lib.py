"""ctypes loading of the gfx950 row-op library (lib/libexl3rowops.so) and its prototypes.

The library is the product; this module is plumbing.  `load()` raises when the shared object is
missing -- there is no fallback implementation of any op."""
import contextlib
import ctypes
import os

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(_PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libexl3rowops.so")
NAIVE_PATH = os.path.join(LIB_DIR, "libexl3r_naive.so")
TUNE_PATH = os.path.join(LIB_DIR, "libexl3rowops_tune.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_ROOT), "include", "exl3r", "rowops.h")

F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
OK, EINVAL, EDTYPE = 0, -1, -2
ROPE_NONE, ROPE_GPTJ, ROPE_NEOX = 0, 1, 2
HAD_EXACT = 16   # EXL3R_HAD_EXACT: the fused Hadamard entry points' reference butterfly

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i32 = ctypes.c_int32


class RopeDesc(ctypes.Structure):
    """exl3r_rope_desc of include/exl3r/rowops.h, field for field (exl3r_rope_run)."""
    _fields_ = [("struct_size", _i32), ("dtype", _i32), ("bsz", _i64), ("seq_len", _i64), ("head_dim", _i32),
                ("rotary_dim", _i32), ("rope_mode", _i32), ("attn_factor", _f), ("q", _vp), ("out_q", _vp),
                ("q_tok_stride", _i64), ("q_head_stride", _i64), ("out_q_tok_stride", _i64),
                ("out_q_head_stride", _i64), ("num_heads_q", _i32), ("num_heads_k", _i32), ("k", _vp),
                ("out_k", _vp), ("k_tok_stride", _i64), ("k_head_stride", _i64), ("inv_freq", _vp),
                ("angle_table", _vp), ("table_rows", _i64), ("table_batch_stride", _i64), ("cs_table", _vp),
                ("positions", _vp), ("position_ids", _vp), ("position", _i32), ("norm_dtype", _i32),
                ("q_norm", _vp), ("k_norm", _vp), ("norm_eps", _f), ("norm_constant_bias", _f),
                ("rotate", _i32), ("page_size", _i32), ("q_post_scale", _vp), ("k_post_scale", _vp),
                ("v_post_scale", _vp), ("v", _vp), ("v_tok_stride", _i64), ("v_head_stride", _i64),
                ("k_cache", _vp), ("v_cache", _vp), ("num_pages", _i64), ("max_blocks_per_seq", _i64),
                ("block_table", _vp), ("cache_seqlens", _vp), ("err_flag", _vp)]


PROTOTYPES = {
    "exl3r_rope_run": (_i, [ctypes.POINTER(RopeDesc), _vp]),
    "exl3r_version": (_i, []),
    "exl3r_last_error": (ctypes.c_char_p, []),
    "exl3r_rms_norm": (_i, [_vp, _i, _i64, _vp, _i, _vp, _i, _i64, _i64, _i64, _f, _f, _f, _vp]),
    "exl3r_rms_norm_res_in": (_i, [_vp, _i, _i64, _vp, _i, _vp, _i, _i64, _vp, _i, _i64, _i64, _i64, _f, _f, _f, _vp]),
    "exl3r_silu_mul": (_i, [_vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _i64, _i64, _f, _vp]),
    "exl3r_gelu_mul": (_i, [_vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _i64, _i64, _f, _vp]),
    "exl3r_rope": (_i, [_vp, _vp, _i64, _i64, _i, _vp, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _i,
                        _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _vp]),
    "exl3r_rope_had": (_i, [_vp, _vp, _i64, _i, _vp, _vp, _i64, _i, _i, _i64, _i64, _i, _vp, _i,
                            _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _vp, _vp, _vp, _vp]),
    "exl3r_rope_table": (_i, [_vp, _vp, _i64, _i64, _i, _vp, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _i64, _i64,
                              _i, _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _vp, _vp]),
    "exl3r_rope_qg": (_i, [_vp, _i64, _vp, _i, _vp, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _i, _i32, _vp, _vp, _vp,
                           _vp, _i, _f, _f, _i, _f, _vp]),
    "exl3r_rope_cs_table": (_i, [_i64, _i64, _vp, _i, _i32, _vp, _vp, _f, _vp, _vp]),
    "exl3r_rope_cs": (_i, [_vp, _vp, _i64, _i64, _i, _vp, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _i, _vp, _vp, _i,
                           _f, _f, _i, _vp]),
    "exl3r_gated_rms_norm": (_i, [_vp, _i, _i64, _vp, _i, _i, _vp, _i, _i64, _vp, _i, _i64, _i64, _i64, _f, _f, _i, _i,
                                  _vp]),
    "exl3r_gated_rms_norm_had": (_i, [_vp, _i, _i64, _vp, _i, _i, _vp, _i, _i64, _vp, _i64, _vp, _i, _vp, _i64, _i64,
                                      _i64, _f, _f, _i, _i, _f, _vp]),
    "exl3r_mul_sigmoid": (_i, [_vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _i64, _i64, _vp]),
    "exl3r_deinterleave_qg": (_i, [_vp, _i64, _vp, _i64, _vp, _i64, _i, _i64, _i, _i, _vp]),
    "exl3r_argmax_sample": (_i, [_vp, _i, _i64, _i64, _i64, _i, _vp, _vp]),
    "exl3r_gumbel_sample": (_i, [_vp, _i, _i64, _i64, _i64, _i, ctypes.c_uint32, _vp, _vp]),
    "exl3r_sample_workspace_bytes": (ctypes.c_size_t, []),
    "exl3r_argmax_sample_ws": (_i, [_vp, _i, _i64, _i64, _i64, _i, _vp, _vp, ctypes.c_size_t, _vp]),
    "exl3r_gumbel_sample_ws": (_i, [_vp, _i, _i64, _i64, _i64, _i, ctypes.c_uint32, _vp, _vp, ctypes.c_size_t, _vp]),
    "exl3r_argmax_sample_noalloc": (_i, [_vp, _i, _i64, _i64, _i64, _i, _vp, _vp]),
    "exl3r_rms_norm_had": (_i, [_vp, _i, _i64, _vp, _i, _vp, _i, _i64, _vp, _i64, _i, _vp, _vp, _i64, _i64, _i64,
                                _f, _f, _f, _f, _i, _vp, _vp]),
    "exl3r_had_r_128": (_i, [_vp, _i, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _f, _vp]),
    "exl3r_had_r_128_mfma": (_i, [_vp, _i, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _f, _vp]),
    "exl3r_act_mul_had": (_i, [_i, _vp, _vp, _i, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _f, _f, _i, _vp,
                               _vp, _vp]),
    "exl3r_gumbel_noise": (_i, [_vp, _i, _i64, _vp, _i, _i64, _i64, _i64, ctypes.c_uint32, _vp]),
    "exl3r_rope_paged_kv": (_i, [_vp, _vp, _i64, _i64, _i, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i, _i, _i64, _i64,
                                 _i, _vp, _i, _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _vp, _vp, _i, _i64,
                                 _vp, _i64, _vp, _vp, _vp, _vp]),
    "exl3r_rope_paged_kv_had": (_i, [_vp, _vp, _i64, _i, _vp, _vp, _i64, _vp, _i64, _i, _i, _i64, _i64, _i, _vp, _i,
                                     _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _vp, _vp, _i, _i64,
                                     _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "exl3r_embedding": (_i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _i64, _vp, _vp]),
    "exl3r_embedding_rms_norm": (_i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _i64, _vp, _i,
                                      _vp, _i, _i64, _f, _f, _f, _vp, _vp]),
}

# Launch-shape overrides of the sweep/test build only (csrc/tuning.h); the product library has none.
TUNE_PROTOTYPES = {
    "exl3r_tune_rms": (None, [_i, _i]),
    "exl3r_tune_rms_rows": (None, [_i]),
    "exl3r_tune_rms_split": (None, [_i, _i]),
    "exl3r_tune_rms_mode": (None, [_i, _i, _i, _i]),
    "exl3r_tune_act": (None, [_i, _i, _i]),
    "exl3r_tune_rope": (None, [_i]),
    "exl3r_tune_rope_tok": (None, [_i, _i, _i]),
    "exl3r_tune_rope_nx": (None, [_i]),
    "exl3r_tune_rope_nx_run": (None, [_i]),
    "exl3r_tune_rope_ss32": (None, [_i]),
    "exl3r_tune_sample": (None, [_i, _i]),
    "exl3r_tune_had": (None, [_i]),
    "exl3r_tune_had_mfma": (None, [_i, _i]),
    "exl3r_tune_had_threads": (None, [_i]),
    "exl3r_tune_embed": (None, [_i]),
}

NAIVE_PROTOTYPES = {
    "naive_add_f16": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "naive_rms_norm_f16": (_i, [_vp, _vp, _vp, _i64, _i, _f, _vp]),
    "naive_head_norm_f16": (_i, [_vp, _vp, _i64, _i, _i, _f, _vp]),
    "naive_rope_neox_f16": (_i, [_vp, _vp, _vp, _i64, _i64, _i, _i, _vp]),
    "naive_silu_f16": (_i, [_vp, _vp, _i64, _vp]),
    "naive_mul_f16": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "naive_paged_kv_update_f16": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i, _i, _i64, _i, _vp]),
    "calib_copy": (_i, [_vp, _vp, _i64, _vp]),
    "calib_copy_cached": (_i, [_vp, _vp, _i64, _vp]),
}

_lib = None
_naive = None
_tune = None


def _bind(path, protos):
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() (make -C exllamav3-rs_amd)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in protos.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load():
    """The row-op library (ctypes.CDLL with prototypes set)."""
    global _lib
    if _lib is None:
        _lib = _bind(LIB_PATH, PROTOTYPES)
    return _lib


def load_naive():
    """The naive unfused baseline library (bench only)."""
    global _naive
    if _naive is None:
        _naive = _bind(NAIVE_PATH, NAIVE_PROTOTYPES)
    return _naive


def load_tune():
    """The sweep/test build of the library (lib/libexl3rowops_tune.so): the same sources compiled with
    EXL3R_TUNING, which adds the process-global exl3r_tune_* launch-shape overrides.  Tests only."""
    global _tune
    if _tune is None:
        _tune = _bind(TUNE_PATH, {**PROTOTYPES, **TUNE_PROTOTYPES})
    return _tune


@contextlib.contextmanager
def tuned():
    """Within the block, the ffi wrappers call the sweep/test build (load_tune()), whose handle is
    yielded to set its overrides; on exit every override is reset and the product library restored."""
    global _lib
    saved = load()
    lib = load_tune()
    _lib = lib
    try:
        yield lib
    finally:
        lib.exl3r_tune_rms(0, 0)
        lib.exl3r_tune_rms_rows(0)
        lib.exl3r_tune_rms_split(0, 1)
        lib.exl3r_tune_rms_mode(0, 0, 0, 0)
        lib.exl3r_tune_act(0, 0, 0)
        lib.exl3r_tune_rope(0)
        lib.exl3r_tune_rope_tok(0, 0, 0)
        lib.exl3r_tune_rope_nx(0)
        lib.exl3r_tune_rope_nx_run(0)
        lib.exl3r_tune_rope_ss32(0)
        lib.exl3r_tune_sample(0, 0)
        lib.exl3r_tune_had(0)
        lib.exl3r_tune_had_mfma(0, 0)
        lib.exl3r_tune_had_threads(0)
        lib.exl3r_tune_embed(0)
        _lib = saved


class Exl3rError(RuntimeError):
    """A non-zero status from a C-ABI entry point (message from exl3r_last_error())."""

    def __init__(self, code, message):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def check(rc):
    if rc != OK:
        raise Exl3rError(rc, load().exl3r_last_error().decode(errors="replace"))
    return rc
