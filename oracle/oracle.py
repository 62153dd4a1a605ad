"""ctypes binding of the CPU oracle (rowops_oracle.c) over numpy arrays -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker or the timed
CPU baseline; never by the product path.  16-bit floats are passed as raw uint16 bit patterns."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "liboracle_rowops.so")

F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
ROPE_GPTJ, ROPE_NEOX = 1, 2
ACT_SILU, ACT_GELU, ACT_SIGMOID = 0, 1, 2

_vp, _i, _i64, _f, _i32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_int32
_PROTOS = {
    "oracle_f32_to_f16": (ctypes.c_uint16, [_f]),
    "oracle_f16_to_f32": (_f, [ctypes.c_uint16]),
    "oracle_f32_to_bf16": (ctypes.c_uint16, [_f]),
    "oracle_bf16_to_f32": (_f, [ctypes.c_uint16]),
    "oracle_round": (ctypes.c_double, [ctypes.c_double, _i]),
    "oracle_f32_to_f16_array": (None, [_vp, _vp, _i64]),
    "oracle_f32_to_bf16_array": (None, [_vp, _vp, _i64]),
    "oracle_rms_norm": (_i, [_vp, _i, _i64, _vp, _i, _vp, _i, _i64, _vp, _i, _i64, _i64, _i64, _f, _f, _f, _i]),
    "oracle_act_mul": (_i, [_i, _vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _i64, _i64, _f, _i]),
    "oracle_rope": (_i, [_vp, _vp, _i64, _i64, _i, _vp, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _i,
                         _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _i]),
    "oracle_rope_table": (_i, [_vp, _vp, _i64, _i64, _i, _vp, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _i64, _i64,
                               _i, _i32, _vp, _vp, _vp, _vp, _i, _f, _f, _i, _f, _vp, _i]),
    "oracle_embedding": (_i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _i64, _vp, _i]),
    "oracle_gated_rms_norm": (_i, [_vp, _i, _i64, _vp, _i, _i, _vp, _i, _i64, _vp, _i, _i64, _i64, _i64, _f, _f, _i,
                                   _i, _i]),
    "oracle_deinterleave_qg": (_i, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i, _i, _i]),
    "oracle_argmax": (_i, [_vp, _i, _i64, _i64, _i64, _i, _vp, _i]),
    "oracle_philox4x32_10": (None, [_vp, _vp, _vp]),
    "oracle_had_r_128": (_i, [_vp, _i, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _f, _i]),
    "oracle_log_f32": (ctypes.c_float, [_f]),
    "oracle_gumbel_of_bits": (None, [_vp, _vp, _i64]),
    "oracle_gumbel_noise": (_i, [_vp, _i, _i64, _vp, _i, _i64, _i64, _i64, ctypes.c_uint32, _i]),
    "oracle_gumbel_sample": (_i, [_vp, _i, _i64, _i64, _i64, _i, ctypes.c_uint32, _vp, _i]),
    "oracle_paged_kv_append": (_i, [_vp, _i64, _i64, _vp, _i64, _i64, _i, _i, _i64, _i64, _i, _vp, _vp, _i, _i64,
                                    _vp, _i64, _vp, _vp, _i]),
    "oracle_embedding_rms_norm": (_i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _i64, _vp, _i,
                                       _vp, _i, _i64, _f, _f, _f, _vp, _i]),
}

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def set_mutation(m):
    ctypes.c_int.in_dll(load(), "oracle_mutation").value = int(m)


def get_mutation():
    return ctypes.c_int.in_dll(load(), "oracle_mutation").value


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"] or a.ndim <= 1, "oracle arrays must be C-contiguous"
    return a.ctypes.data


def storage_dtype(code):
    return {F32: np.float32, F16: np.uint16, BF16: np.uint16, I32: np.int32, I64: np.int64}[code]


def f32_to_f16_bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    load().oracle_f32_to_f16_array(_p(a), _p(out), a.size)
    return out


def f32_to_bf16_bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    load().oracle_f32_to_bf16_array(_p(a), _p(out), a.size)
    return out


def to_bits(a, code):
    """fp32 values -> storage array of dtype `code` (RNE)."""
    if code == F32:
        return np.ascontiguousarray(a, dtype=np.float32)
    return f32_to_f16_bits(a) if code == F16 else f32_to_bf16_bits(a)


def to_f32(a, code):
    """Storage array of dtype `code` -> exact fp32 values."""
    if code == F32:
        return np.asarray(a, dtype=np.float32)
    if code == F16:
        return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float32)
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _check(rc, name):
    if rc != 0:
        raise ValueError(f"{name} returned {rc}")


def rms_norm(x, xt, w, wt, yt, eps, cb=0.0, cs=1.0, r=None, rt=F32, nthreads=1):
    """y (new array) = RMSNorm of x [rows, dim]; with r: r is updated in place (RES_IN)."""
    rows, dim = x.shape
    y = np.zeros((rows, dim), storage_dtype(yt))
    _check(load().oracle_rms_norm(_p(x), xt, dim, _p(w), wt, _p(y), yt, dim, _p(r), rt, dim, rows, dim,
                                  eps, cb, cs, nthreads), "oracle_rms_norm")
    return y


def act_mul(act, x, y, it, zt, limit=0.0, nthreads=1):
    rows, cols = x.shape
    z = np.zeros((rows, cols), storage_dtype(zt))
    _check(load().oracle_act_mul(act, _p(x), _p(y), it, _p(z), zt, rows, cols, cols, cols, cols, limit, nthreads),
           "oracle_act_mul")
    return z


def mul_sigmoid(x, y, it, zt, nthreads=1):
    """z = x * sigmoid(y) (fp32 product, one rounding): act_mul with the operands' roles swapped."""
    return act_mul(ACT_SIGMOID, y, x, it, zt, nthreads=nthreads)


def gated_rms_norm(x, xt, g, gt, yt, w=None, wt=F32, w_groups=1, eps=1e-6, cb=0.0, gate_first=False, gate_act=0,
                   nthreads=1):
    """x, g: [rows, dim] storage arrays; w: [w_groups * dim] or None.  Returns y."""
    rows, dim = x.shape
    y = np.zeros((rows, dim), storage_dtype(yt))
    _check(load().oracle_gated_rms_norm(_p(x), xt, dim, _p(w), wt, w_groups, _p(y), yt, dim, _p(g), gt, dim, rows,
                                        dim, eps, cb, int(gate_first), gate_act, nthreads), "oracle_gated_rms_norm")
    return y


def argmax(logits, dt, max_logit=0, nthreads=1):
    """logits: [rows, vocab] storage array.  Returns int64 [rows]: first maximal index below max_logit."""
    rows, vocab = logits.shape
    ids = np.zeros(rows, np.int64)
    _check(load().oracle_argmax(_p(logits), dt, rows, vocab, vocab, max_logit, _p(ids), nthreads), "oracle_argmax")
    return ids


def had_r_128(x, dt, pre=None, post=None, scale=1.0, nthreads=1):
    """x: [rows, cols] storage (f16 bits or f32).  Returns the random-Hadamard transform (same dtype)."""
    rows, cols = x.shape
    out = np.zeros_like(x)
    pre = None if pre is None else np.ascontiguousarray(pre, np.uint16)
    post = None if post is None else np.ascontiguousarray(post, np.uint16)
    _check(load().oracle_had_r_128(_p(np.ascontiguousarray(x)), dt, cols, _p(out), cols, rows, cols, _p(pre), _p(post),
                                   scale, nthreads), "oracle_had_r_128")
    return out


def philox4x32_10(ctr, key):
    """One Philox4x32-10 block: ctr 4 x uint32, key 2 x uint32 -> 4 x uint32."""
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(4, np.uint32)
    load().oracle_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def log_f32(x):
    return np.float32(load().oracle_log_f32(float(x)))


def gumbel_of_bits(bits):
    """Gumbel noise -log(-log(u)) for raw uint32 Philox words (u = ((b >> 9) + 0.5) * 2^-23)."""
    b = np.ascontiguousarray(bits, np.uint32)
    g = np.zeros(b.shape, np.float32)
    load().oracle_gumbel_of_bits(_p(b), _p(g), b.size)
    return g


def gumbel_noise(x, xt, seed, out_dt=F32, nthreads=1):
    """x: [rows, cols] storage.  Returns x + Gumbel noise of (seed, row, column), rounded to out_dt."""
    rows, cols = x.shape
    out = np.zeros((rows, cols), np.float32 if out_dt == F32 else np.uint16)
    _check(load().oracle_gumbel_noise(_p(x), xt, cols, _p(out), out_dt, cols, rows, cols, seed, nthreads),
           "oracle_gumbel_noise")
    return out


def gumbel_sample(logits, dt, seed, max_logit=0, nthreads=1):
    """Gumbel-max draw per row: argmax over the first max_logit columns of logits + noise."""
    rows, vocab = logits.shape
    ids = np.zeros(rows, np.int64)
    _check(load().oracle_gumbel_sample(_p(logits), dt, rows, vocab, vocab, max_logit, seed, _p(ids), nthreads),
           "oracle_gumbel_sample")
    return ids


def deinterleave_qg(qg, heads, hd, nthreads=1):
    """qg: [rows, heads * 2 * hd] 16-bit storage.  Returns (q [rows, heads * hd], g [rows, heads * hd])."""
    rows = qg.shape[0]
    q = np.zeros((rows, heads * hd), qg.dtype)
    g = np.zeros((rows, heads * hd), qg.dtype)
    _check(load().oracle_deinterleave_qg(_p(qg), heads * 2 * hd, _p(q), heads * hd, _p(g), heads * hd, rows, heads, hd,
                                         nthreads), "oracle_deinterleave_qg")
    return q, g


def rope(q, k, dt, inv_freq, mode, position=0, positions=None, position_ids=None, q_norm=None, k_norm=None,
         nwt=F16, eps=1e-6, cb=0.0, attn=1.0, nthreads=1):
    """q: [bsz, seq, hq, hd], k: [bsz, seq, hk, hd] or None (storage arrays). Returns (out_q, out_k)."""
    bsz, seq, hq, hd = q.shape
    oq = np.empty_like(q)
    ok, hk = None, 0
    if k is not None:
        hk = k.shape[2]
        ok = np.empty_like(k)
    inv_freq = np.ascontiguousarray(inv_freq, dtype=np.float32)
    _check(load().oracle_rope(_p(q), _p(oq), hq * hd, hd, hq, _p(k), _p(ok), hk * hd, hd, hk, dt, bsz, seq, hd,
                              _p(inv_freq), inv_freq.size * 2, int(position), _p(positions), _p(position_ids),
                              _p(q_norm), _p(k_norm), nwt, eps, cb, mode, attn, nthreads), "oracle_rope")
    return oq, ok


def rope_table(q, k, dt, table, mode, table_bstride=None, position=0, positions=None, position_ids=None, q_norm=None,
               k_norm=None, nwt=F16, eps=1e-6, cb=0.0, attn=1.0, nthreads=1):
    """rope() with angles read from `table` ([rows, R/2], one table for every sequence, or
    [bsz, rows, R/2], one per sequence).  Returns (out_q, out_k, err)."""
    bsz, seq, hq, hd = q.shape
    oq = np.empty_like(q)
    ok, hk = None, 0
    if k is not None:
        hk = k.shape[2]
        ok = np.empty_like(k)
    table = np.ascontiguousarray(table, dtype=np.float32)
    rows, half = table.shape[-2], table.shape[-1]
    if table_bstride is None:
        table_bstride = rows * half if table.ndim == 3 else 0
    err = np.zeros(1, np.int32)
    _check(load().oracle_rope_table(_p(q), _p(oq), hq * hd, hd, hq, _p(k), _p(ok), hk * hd, hd, hk, dt, bsz, seq, hd,
                                    _p(table), rows, table_bstride, half * 2, int(position), _p(positions),
                                    _p(position_ids), _p(q_norm), _p(k_norm), nwt, eps, cb, mode, attn, _p(err),
                                    nthreads), "oracle_rope_table")
    return oq, ok, int(err[0])


def embedding(table, tt, ids, idt, ot, nthreads=1):
    vocab, hidden = table.shape
    n = ids.size
    out = np.zeros((n, hidden), storage_dtype(ot))
    err = np.zeros(1, np.int32)
    _check(load().oracle_embedding(_p(table), tt, vocab, hidden, hidden, _p(ids), idt, n, _p(out), ot, hidden,
                                   _p(err), nthreads), "oracle_embedding")
    return out, int(err[0])


def paged_kv_append(k, v, dt, k_cache, v_cache, block_table, cache_seqlens, nthreads=1):
    """k, v: [bsz, seq, hk, hd] storage arrays (either may be None); k_cache / v_cache:
    [pages, page_size, hk, hd], updated in place; block_table int32 [bsz, max_blocks];
    cache_seqlens int32 [bsz].  Returns the error flag."""
    src = k if k is not None else v
    bsz, seq, hk, hd = src.shape
    pages, page_size = (k_cache if k_cache is not None else v_cache).shape[:2]
    bt = np.ascontiguousarray(block_table, np.int32)
    cl = np.ascontiguousarray(cache_seqlens, np.int32)
    err = np.zeros(1, np.int32)
    k = None if k is None else np.ascontiguousarray(k)
    v = None if v is None else np.ascontiguousarray(v)
    _check(load().oracle_paged_kv_append(_p(k), hk * hd, hd, _p(v), hk * hd, hd, hk, dt, bsz, seq, hd,
                                         _p(k_cache), _p(v_cache), page_size, pages, _p(bt), bt.shape[1], _p(cl),
                                         _p(err), nthreads), "oracle_paged_kv_append")
    return int(err[0])


def embedding_rms_norm(table, tt, ids, idt, w, wt, yt, ht=None, eps=1e-6, cb=0.0, cs=1.0, nthreads=1):
    vocab, hidden = table.shape
    n = ids.size
    y = np.zeros((n, hidden), storage_dtype(yt))
    h = None if ht is None else np.zeros((n, hidden), storage_dtype(ht))
    err = np.zeros(1, np.int32)
    _check(load().oracle_embedding_rms_norm(_p(table), tt, vocab, hidden, hidden, _p(ids), idt, n,
                                            _p(h), ht if ht is not None else F32, hidden, _p(w), wt, _p(y), yt,
                                            hidden, eps, cb, cs, _p(err), nthreads), "oracle_embedding_rms_norm")
    return h, y, int(err[0])
