"""Torch-tensor wrappers over the C ABI, with the names and argument meaning of the reference's
`src/ffi.rs` wrappers (rms_norm ffi.rs:293-296, rms_norm_res_in 464-468, silu_mul 492-495,
gelu_mul 496-499, rope 298-333) plus the embedding gather that replaces Embedding::forward's
index_select (src/modules.rs:430-436).

Tensors must live on the GPU; every wrapper launches on the current torch stream (the reference's
kernels use the current torch stream too, kernels/norm.cu:328) unless `stream` is given, and raises
Exl3rError on a non-zero status (the reference's TORCH_CHECK raises)."""
import ctypes
import math

import torch

from ._lib import BF16, F16, F32, HAD_EXACT, I32, I64, RopeDesc, check, load

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int32: I32, torch.int64: I64}


def dtype_code(t):
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(t, stream):
    if stream is not None:
        return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream
    return torch.cuda.current_stream(t.device).cuda_stream


def _rows(t):
    """[..., dim] tensor as (rows, dim, row_stride); the last dim must be dense and the leading dims
    must collapse into one stride."""
    if t.dim() == 0:
        raise ValueError("expected at least 1-D tensor")
    dim = t.shape[-1]
    if t.dim() == 1:
        return 1, dim, dim
    if dim == 0:
        return math.prod(t.shape[:-1]), 0, 0
    if dim > 1 and t.stride(-1) != 1:
        raise ValueError("last dimension must be contiguous")
    try:
        v = t.view(-1, dim)
    except RuntimeError as e:
        raise ValueError("leading dimensions must collapse to one row stride") from e
    rows = v.shape[0]
    return rows, dim, max(dim, v.stride(0)) if rows > 1 else dim


def rms_norm(x, w, y, eps, constant_bias=0.0, constant_scale=1.0, stream=None):
    """y = RMSNorm(x) * (w + constant_bias) * constant_scale over the last dim (w may be None)."""
    rows, dim, ldx = _rows(x)
    ry, dy, ldy = _rows(y)
    if (ry, dy) != (rows, dim):
        raise ValueError("x and y shapes differ")
    check(load().exl3r_rms_norm(_ptr(x), dtype_code(x), ldx, _ptr(w), dtype_code(w) if w is not None else F16,
                                _ptr(y), dtype_code(y), ldy, rows, dim, eps, constant_bias, constant_scale,
                                _stream(x, stream)))


def rms_norm_res_in(x, w, y, r, eps, constant_bias=0.0, constant_scale=1.0, stream=None):
    """r += x (in place, rounded to r's dtype), y = RMSNorm(r) * (w + constant_bias) * constant_scale."""
    rows, dim, ldx = _rows(x)
    ry, dy, ldy = _rows(y)
    rr, dr, ldr = _rows(r)
    if (ry, dy) != (rows, dim) or (rr, dr) != (rows, dim):
        raise ValueError("x, y and r shapes differ")
    check(load().exl3r_rms_norm_res_in(_ptr(x), dtype_code(x), ldx, _ptr(w), dtype_code(w) if w is not None else F16,
                                       _ptr(y), dtype_code(y), ldy, _ptr(r), dtype_code(r), ldr, rows, dim,
                                       eps, constant_bias, constant_scale, _stream(x, stream)))


def _act(fn, x, y, z, act_limit, stream):
    rows, cols, ldx = _rows(x)
    ry, cy, ldy = _rows(y)
    rz, cz, ldz = _rows(z)
    if (ry, cy) != (rows, cols) or (rz, cz) != (rows, cols):
        raise ValueError("x, y and z shapes differ")
    if x.dtype != y.dtype:
        raise TypeError("x and y must share a dtype")
    check(fn(_ptr(x), _ptr(y), dtype_code(x), _ptr(z), dtype_code(z), rows, cols, ldx, ldy, ldz, act_limit,
             _stream(x, stream)))


def silu_mul(x, y, z, act_limit=0.0, stream=None):
    """z = silu(x) * y (SwiGLU); act_limit 0 disables clamping."""
    _act(load().exl3r_silu_mul, x, y, z, act_limit, stream)


def gelu_mul(x, y, z, act_limit=0.0, stream=None):
    """z = gelu_tanh(x) * y."""
    _act(load().exl3r_gelu_mul, x, y, z, act_limit, stream)


def gated_rms_norm(x, w, y, g, eps, constant_bias=0.0, w_groups=1, gate_first=False, gate_act=0, stream=None):
    """y = RMSNorm(x) * (w + constant_bias) * act(g), or RMSNorm(x * act(g)) * (w + constant_bias) with
    gate_first; act = silu (gate_act 0) or sigmoid (1); w may be None or hold w_groups rows of dim
    (src/ffi.rs:479-483)."""
    rows, dim, ldx = _rows(x)
    ry, dy, ldy = _rows(y)
    rg, dg, ldg = _rows(g)
    if (ry, dy) != (rows, dim) or (rg, dg) != (rows, dim):
        raise ValueError("x, y and g shapes differ")
    if w is not None and w.numel() != w_groups * dim:
        raise ValueError("w must hold w_groups * dim values")
    check(load().exl3r_gated_rms_norm(_ptr(x), dtype_code(x), ldx, _ptr(w), dtype_code(w) if w is not None else F32,
                                      w_groups, _ptr(y), dtype_code(y), ldy, _ptr(g), dtype_code(g), ldg, rows, dim, eps,
                                      constant_bias, int(bool(gate_first)), int(gate_act), _stream(x, stream)))



def gated_rms_norm_had(x, w, g, out, eps, pre_scale=None, y=None, constant_bias=0.0, w_groups=1, gate_first=False,
                       gate_act=0, had_scale=1.0, pre_rows=1, stream=None, exact=False):
    """One pass: the gated norm of gated_rms_norm into an f16 y (written only if given), then
    out = had_r_128(y, pre_scale) (f16, dim % 128 == 0): o_proj's input rotation.  Norm row r uses
    pre_scale[(r % pre_rows) * dim:]: with rows = tokens * heads of head_dim, pre_rows = heads.  Rows of
    128 run the transform on the matrix cores; exact=True: the reference's butterfly (EXL3R_HAD_EXACT in
    gate_act)."""
    rows, dim, ldx = _rows(x)
    rg, dg, ldg = _rows(g)
    ro, do, ldo = _rows(out)
    if (rg, dg) != (rows, dim) or (ro, do) != (rows, dim) or out.dtype != torch.float16:
        raise ValueError("g like x; out f16 shaped like x")
    ldy = 0
    if y is not None:
        ry, dy, ldy = _rows(y)
        if (ry, dy) != (rows, dim) or y.dtype != torch.float16:
            raise ValueError("y is the f16 norm output shaped like x")
    if w is not None and w.numel() != w_groups * dim:
        raise ValueError("w must hold w_groups * dim values")
    check(load().exl3r_gated_rms_norm_had(_ptr(x), dtype_code(x), ldx, _ptr(w), dtype_code(w) if w is not None else F32,
                                          w_groups, _ptr(g), dtype_code(g), ldg, _ptr(y), ldy, _ptr(pre_scale),
                                          int(pre_rows), _ptr(out), ldo, rows, dim, eps, constant_bias,
                                          int(bool(gate_first)),
                                          int(gate_act) | (HAD_EXACT if exact else 0), float(had_scale),
                                          _stream(x, stream)))

def mul_sigmoid(x, y, z, stream=None):
    """z = x * sigmoid(y) (fp32, one rounding); z may be x."""
    rows, cols, ldx = _rows(x)
    ry, cy, ldy = _rows(y)
    rz, cz, ldz = _rows(z)
    if (ry, cy) != (rows, cols) or (rz, cz) != (rows, cols):
        raise ValueError("x, y and z shapes differ")
    if x.dtype != y.dtype:
        raise TypeError("x and y must share a dtype")
    check(load().exl3r_mul_sigmoid(_ptr(x), _ptr(y), dtype_code(x), _ptr(z), dtype_code(z), rows, cols, ldx, ldy, ldz,
                                   _stream(x, stream)))


def mul_sigmoid_(x, y, stream=None):
    """x *= sigmoid(y) in place (src/ffi.rs:616-618)."""
    mul_sigmoid(x, y, x, stream)


def deinterleave_qg(qg, q, g, head_dim, stream=None):
    """Split [.., heads * 2 * head_dim] per-head interleaved (q | g) rows into q [.., heads, head_dim] and
    g [.., heads * head_dim] (src/ffi.rs:622-624)."""
    width = qg.shape[-1]
    if width % (2 * head_dim):
        raise ValueError("qg's last dim must be heads * 2 * head_dim")
    heads = width // (2 * head_dim)
    rows, _, ldqg = _rows(qg)
    q2 = q.reshape(rows, heads * head_dim) if q.is_contiguous() else q.view(rows, heads * head_dim)
    rq, cq, ldq = _rows(q2)
    rg, cg, ldg = _rows(g.reshape(rows, heads * head_dim) if g.is_contiguous() else g)
    if (rq, cq) != (rows, heads * head_dim) or (rg, cg) != (rows, heads * head_dim):
        raise ValueError("q and g must hold heads * head_dim values per row")
    if q.dtype != qg.dtype or g.dtype != qg.dtype:
        raise TypeError("qg, q and g must share a dtype")
    check(load().exl3r_deinterleave_qg(_ptr(qg), ldqg, _ptr(q), ldq, _ptr(g), ldg, dtype_code(qg), rows, heads, head_dim,
                                       _stream(qg, stream)))


def rope(q, out_q, k, out_k, inv_freq, position, positions, q_norm, k_norm, norm_eps, norm_constant_bias,
         rope_mode, attn_factor, position_ids=None, stream=None, err_flag=None):
    """Fused (optional) q/k head RMSNorm + RoPE.  q, k: (bsz, seq_len, heads, head_dim); `positions`
    (int32 [bsz], device) or `position_ids` (int32 [bsz, seq_len], device) override `position`.
    As in the reference (rope.cu:340-347), a 2-D [max_pos, R/2] or 3-D [bsz, max_pos, R/2] inv_freq
    is a table of precomputed angles (RoPE::apply's freq_table, src/rope.rs:225-260): the 2-D table
    is shared by every sequence; a position outside it sets err_flag (int32, device) if given."""
    if q.dim() != 4:
        raise ValueError("q must be (bsz, seq_len, heads, head_dim)")
    bsz, seq, hq, hd = q.shape
    if q.stride(3) != 1 or out_q.stride() != q.stride() or out_q.shape != q.shape:
        raise ValueError("q innermost dim must be dense and out_q must share q's layout")
    if seq > 1 and q.stride(0) != seq * q.stride(1) and bsz > 1:
        raise ValueError("q batch stride must be seq_len * token stride")
    hk, k_ts, k_hs = 0, 0, 0
    if k is not None:
        if k.dim() != 4 or k.shape[0] != bsz or k.shape[1] != seq or k.shape[3] != hd:
            raise ValueError("k is incorrect shape")
        if k.stride(3) != 1 or out_k is None or out_k.stride() != k.stride():
            raise ValueError("k innermost dim must be dense and out_k must share k's layout")
        if seq > 1 and k.stride(0) != seq * k.stride(1) and bsz > 1:
            raise ValueError("k batch stride must be seq_len * token stride")
        hk, k_ts, k_hs = k.shape[2], k.stride(1), k.stride(2)
    for t in (positions, position_ids):
        if t is not None and t.dtype != torch.int32:
            raise TypeError("positions / position_ids must be int32")
    nw = q_norm if q_norm is not None else k_norm
    if inv_freq.dim() > 1:
        if inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous() or inv_freq.dim() > 3:
            raise ValueError("an angle table must be a contiguous float32 [max_pos, R/2] or [bsz, max_pos, R/2]")
        if inv_freq.dim() == 3 and inv_freq.shape[0] < bsz:
            raise ValueError("a per-sequence angle table needs bsz rows of tables")
        rows, half = inv_freq.shape[-2], inv_freq.shape[-1]
        bstride = rows * half if inv_freq.dim() == 3 else 0
        check(load().exl3r_rope_table(_ptr(q), _ptr(out_q), q.stride(1), q.stride(2), hq,
                                      _ptr(k), _ptr(out_k), k_ts, k_hs, hk,
                                      dtype_code(q), bsz, seq, hd, _ptr(inv_freq), rows, bstride, half * 2,
                                      int(position), _ptr(positions), _ptr(position_ids),
                                      _ptr(q_norm), _ptr(k_norm), dtype_code(nw) if nw is not None else F16,
                                      norm_eps, norm_constant_bias, rope_mode, attn_factor, _ptr(err_flag),
                                      _stream(q, stream)))
        return
    check(load().exl3r_rope(_ptr(q), _ptr(out_q), q.stride(1), q.stride(2), hq,
                            _ptr(k), _ptr(out_k), k_ts, k_hs, hk,
                            dtype_code(q), bsz, seq, hd, _ptr(inv_freq), inv_freq.shape[-1] * 2,
                            int(position), _ptr(positions), _ptr(position_ids),
                            _ptr(q_norm), _ptr(k_norm), dtype_code(nw) if nw is not None else F16,
                            norm_eps, norm_constant_bias, rope_mode, attn_factor, _stream(q, stream)))


def _rotary_dim(inv_freq, cs_table, tokens, device):
    """rotary_dim of the entry points that take inv_freq [R/2] and / or a rope_cs_table() {cos, sin} table
    [tokens, R/2, 2] (tokens = bsz * seq_len).  These kernels index the table by token, so a table built for
    fewer tokens (one reused across forward passes of different lengths) is rejected here; an angle table
    (2-D / 3-D inv_freq) is rope()'s input only."""
    if inv_freq is not None and (inv_freq.dim() != 1 or inv_freq.dtype != torch.float32):
        raise ValueError("inv_freq must be float32 [R/2]; an angle table (RoPE::apply's freq_table) takes rope()")
    if cs_table is not None:
        if (cs_table.dtype != torch.float32 or not cs_table.is_contiguous() or cs_table.dim() != 3
                or cs_table.shape[0] != tokens or cs_table.shape[2] != 2):
            raise ValueError(f"cs_table must be a contiguous float32 [bsz * seq_len = {tokens}, R/2, 2], "
                             f"got {tuple(cs_table.shape)} {cs_table.dtype}")
        if cs_table.device != device:
            raise ValueError("cs_table must be on the device of q")
        if inv_freq is not None and inv_freq.shape[0] != cs_table.shape[1]:
            raise ValueError("cs_table and inv_freq disagree on rotary_dim")
        return cs_table.shape[1] * 2
    if inv_freq is None:
        raise ValueError("inv_freq or cs_table is required")
    return inv_freq.shape[0] * 2


def rope_qg(qg, out_q, k, out_k, inv_freq, position, positions, q_norm, k_norm, norm_eps, norm_constant_bias,
            rope_mode, attn_factor, position_ids=None, stream=None):
    """deinterleave_qg() then rope() on its q, in one pass (gated attention, src/modules.rs:637-646 then
    669-681): qg (bsz, seq_len, heads, 2 * head_dim) holds each head's [q | g]; out_q (bsz, seq_len, heads,
    head_dim) dense receives the roped q.  The gate stays in qg: qg[..., head_dim:] as rows of head_dim with
    row stride 2 * head_dim (mul_sigmoid's y)."""
    if qg.dim() != 4 or out_q.dim() != 4:
        raise ValueError("qg must be (bsz, seq_len, heads, 2 * head_dim) and out_q (bsz, seq_len, heads, head_dim)")
    bsz, seq, hq, hd2 = qg.shape
    hd = hd2 // 2
    if hd2 % 2 or tuple(out_q.shape) != (bsz, seq, hq, hd) or not out_q.is_contiguous():
        raise ValueError("out_q must be a dense (bsz, seq_len, heads, head_dim)")
    if qg.stride(3) != 1 or qg.stride(2) != hd2 or (bsz > 1 and seq > 1 and qg.stride(0) != seq * qg.stride(1)):
        raise ValueError("qg must hold dense [q | g] heads with batch stride seq_len * token stride")
    hk, k_ts, k_hs = 0, 0, 0
    if k is not None:
        if k.dim() != 4 or k.shape[0] != bsz or k.shape[1] != seq or k.shape[3] != hd:
            raise ValueError("k is incorrect shape")
        if k.stride(3) != 1 or out_k is None or out_k.stride() != k.stride():
            raise ValueError("k innermost dim must be dense and out_k must share k's layout")
        if seq > 1 and k.stride(0) != seq * k.stride(1) and bsz > 1:
            raise ValueError("k batch stride must be seq_len * token stride")
        hk, k_ts, k_hs = k.shape[2], k.stride(1), k.stride(2)
    for t in (positions, position_ids):
        if t is not None and t.dtype != torch.int32:
            raise TypeError("positions / position_ids must be int32")
    nw = q_norm if q_norm is not None else k_norm
    check(load().exl3r_rope_qg(_ptr(qg), qg.stride(1), _ptr(out_q), hq, _ptr(k), _ptr(out_k), k_ts, k_hs, hk,
                               dtype_code(qg), bsz, seq, hd, _ptr(inv_freq), _rotary_dim(inv_freq, None, 0, qg.device),
                               int(position),
                               _ptr(positions), _ptr(position_ids), _ptr(q_norm), _ptr(k_norm),
                               dtype_code(nw) if nw is not None else F16, norm_eps, norm_constant_bias, rope_mode,
                               attn_factor, _stream(qg, stream)))


def rope_cs_table(bsz, seq_len, inv_freq, position, positions=None, position_ids=None, attn_factor=1.0, out=None,
                  stream=None):
    """{cos, sin} * attn_factor of every token's rotary frequencies (float32 [bsz * seq_len, R/2, 2]), as
    rope() evaluates them for the same positions: built once per forward pass, read by every layer's
    rope_cs().  `out`, if given, is filled in place."""
    if inv_freq.dim() != 1 or inv_freq.dtype != torch.float32:
        raise ValueError("inv_freq must be float32 [R/2]")
    for t in (positions, position_ids):
        if t is not None and t.dtype != torch.int32:
            raise TypeError("positions / position_ids must be int32")
    half = inv_freq.shape[0]
    if out is None:
        out = torch.empty((bsz * seq_len, half, 2), device=inv_freq.device, dtype=torch.float32)
    elif out.dtype != torch.float32 or not out.is_contiguous() or out.shape != (bsz * seq_len, half, 2):
        raise ValueError("out must be a contiguous float32 [bsz * seq_len, R/2, 2]")
    check(load().exl3r_rope_cs_table(bsz, seq_len, _ptr(inv_freq), half * 2, int(position), _ptr(positions),
                                     _ptr(position_ids), attn_factor, _ptr(out), _stream(inv_freq, stream)))
    return out


def rope_cs(q, out_q, k, out_k, cs_table, q_norm, k_norm, norm_eps, norm_constant_bias, rope_mode, stream=None):
    """rope() with the rotary pairs read from a rope_cs_table() of the same positions: bit-identical to
    rope(), the per-layer sin / cos evaluation replaced by a table row copy.  q, k: as rope()."""
    if q.dim() != 4:
        raise ValueError("q must be (bsz, seq_len, heads, head_dim)")
    bsz, seq, hq, hd = q.shape
    if q.stride(3) != 1 or out_q.stride() != q.stride() or out_q.shape != q.shape:
        raise ValueError("q innermost dim must be dense and out_q must share q's layout")
    if seq > 1 and q.stride(0) != seq * q.stride(1) and bsz > 1:
        raise ValueError("q batch stride must be seq_len * token stride")
    hk, k_ts, k_hs = 0, 0, 0
    if k is not None:
        if k.dim() != 4 or k.shape[0] != bsz or k.shape[1] != seq or k.shape[3] != hd:
            raise ValueError("k is incorrect shape")
        if k.stride(3) != 1 or out_k is None or out_k.stride() != k.stride():
            raise ValueError("k innermost dim must be dense and out_k must share k's layout")
        if seq > 1 and k.stride(0) != seq * k.stride(1) and bsz > 1:
            raise ValueError("k batch stride must be seq_len * token stride")
        hk, k_ts, k_hs = k.shape[2], k.stride(1), k.stride(2)
    if (cs_table.dtype != torch.float32 or not cs_table.is_contiguous() or cs_table.dim() != 3
            or cs_table.shape[0] != bsz * seq or cs_table.shape[2] != 2):
        raise ValueError("cs_table must be a contiguous float32 [bsz * seq_len, R/2, 2]")
    nw = q_norm if q_norm is not None else k_norm
    check(load().exl3r_rope_cs(_ptr(q), _ptr(out_q), q.stride(1), q.stride(2), hq, _ptr(k), _ptr(out_k), k_ts, k_hs,
                               hk, dtype_code(q), bsz, seq, hd, _ptr(cs_table), cs_table.shape[1] * 2,
                               _ptr(q_norm), _ptr(k_norm), dtype_code(nw) if nw is not None else F16,
                               norm_eps, norm_constant_bias, rope_mode, _stream(q, stream)))


def rope_had(q, out_q, k, out_k, inv_freq, position, positions, q_norm, k_norm, norm_eps, norm_constant_bias,
             rope_mode, attn_factor, q_post_scale=None, k_post_scale=None, position_ids=None, stream=None,
             cs_table=None, exact=False):
    """rope() on the raw f16 outputs of the q / k projections, each first given its projection's output
    rotation had_r_128(y, y, None, svh) (src/modules.rs:231).  q, k: (bsz, seq_len, heads, head_dim) with
    heads packed; q_post_scale / k_post_scale: f16 [heads * head_dim] or None.  The fused launch runs the
    rotations on the matrix cores; exact=True: the reference's butterfly (EXL3R_HAD_EXACT in rope_mode)."""
    if q.dim() != 4:
        raise ValueError("q must be (bsz, seq_len, heads, head_dim)")
    bsz, seq, hq, hd = q.shape
    if q.stride(3) != 1 or q.stride(2) != hd or out_q.stride() != q.stride() or out_q.shape != q.shape:
        raise ValueError("q heads must be packed and out_q must share q's layout")
    if seq > 1 and bsz > 1 and q.stride(0) != seq * q.stride(1):
        raise ValueError("q batch stride must be seq_len * token stride")
    hk, k_ts = 0, 0
    if k is not None:
        if k.dim() != 4 or k.shape[:2] != q.shape[:2] or k.shape[3] != hd or k.stride(3) != 1 or k.stride(2) != hd:
            raise ValueError("k must be (bsz, seq_len, kv_heads, head_dim) with packed heads")
        if out_k is None or out_k.stride() != k.stride() or out_k.shape != k.shape:
            raise ValueError("out_k must share k's layout")
        if seq > 1 and bsz > 1 and k.stride(0) != seq * k.stride(1):
            raise ValueError("k batch stride must be seq_len * token stride")
        hk, k_ts = k.shape[2], k.stride(1)
    nw = q_norm if q_norm is not None else k_norm
    check(load().exl3r_rope_had(_ptr(q), _ptr(out_q), q.stride(1), hq, _ptr(k), _ptr(out_k), k_ts, hk,
                                dtype_code(q), bsz, seq, hd, _ptr(inv_freq), _rotary_dim(inv_freq, cs_table, bsz * seq, q.device),
                                int(position), _ptr(positions), _ptr(position_ids),
                                _ptr(q_norm), _ptr(k_norm), dtype_code(nw) if nw is not None else F16,
                                norm_eps, norm_constant_bias, rope_mode | (HAD_EXACT if exact else 0), attn_factor,
                                _ptr(q_post_scale), _ptr(k_post_scale), _ptr(cs_table), _stream(q, stream)))


def rope_paged_kv(q, out_q, k, out_k, v, inv_freq, position, positions, q_norm, k_norm, norm_eps, norm_constant_bias,
                  rope_mode, attn_factor, k_cache, v_cache, block_table, cache_seqlens, position_ids=None,
                  err_flag=None, stream=None, cs_table=None):
    """rope() on q and k fused with the paged KV-cache append that follows it (paged_kv_cache_update):
    the roped k (also written to out_k unless it is None) and v go to k_cache / v_cache
    [pages, page_size, kv_heads, head_dim] at cache_seqlens[b] + s through block_table
    (int32 [bsz, max_blocks]).  cs_table: a rope_cs_table() of the same positions, read in place of
    evaluating sin / cos (inv_freq may then be None)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be (bsz, seq_len, heads, head_dim)")
    bsz, seq, hq, hd = q.shape
    hk = k.shape[2]
    if k.shape != v.shape or k.shape[0] != bsz or k.shape[1] != seq or k.shape[3] != hd:
        raise ValueError("k and v must be (bsz, seq_len, kv_heads, head_dim) like q")
    if q.stride(3) != 1 or out_q.stride() != q.stride() or out_q.shape != q.shape:
        raise ValueError("q innermost dim must be dense and out_q must share q's layout")
    for t in (k, v) + ((out_k,) if out_k is not None else ()):
        if t.stride(3) != 1 or (seq > 1 and bsz > 1 and t.stride(0) != seq * t.stride(1)):
            raise ValueError("k / v / out_k: dense innermost dim and batch stride seq_len * token stride")
    if out_k is not None and out_k.stride() != k.stride():
        raise ValueError("out_k must share k's layout")
    if seq > 1 and bsz > 1 and q.stride(0) != seq * q.stride(1):
        raise ValueError("q batch stride must be seq_len * token stride")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.shape[2:] != (hk, hd) or not k_cache.is_contiguous() \
            or not v_cache.is_contiguous():
        raise ValueError("caches must be contiguous (pages, page_size, kv_heads, head_dim)")
    if block_table.dim() != 2 or block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32:
        raise TypeError("block_table (bsz, max_blocks) and cache_seqlens (bsz) must be int32")
    for t in (positions, position_ids):
        if t is not None and t.dtype != torch.int32:
            raise TypeError("positions / position_ids must be int32")
    nw = q_norm if q_norm is not None else k_norm
    check(load().exl3r_rope_paged_kv(_ptr(q), _ptr(out_q), q.stride(1), q.stride(2), hq,
                                     _ptr(k), _ptr(out_k), k.stride(1), k.stride(2),
                                     _ptr(v), v.stride(1), v.stride(2), hk,
                                     dtype_code(q), bsz, seq, hd, _ptr(inv_freq), _rotary_dim(inv_freq, cs_table, bsz * seq, q.device),
                                     int(position), _ptr(positions), _ptr(position_ids),
                                     _ptr(q_norm), _ptr(k_norm), dtype_code(nw) if nw is not None else F16,
                                     norm_eps, norm_constant_bias, rope_mode, attn_factor,
                                     _ptr(k_cache), _ptr(v_cache), k_cache.shape[1], k_cache.shape[0],
                                     _ptr(block_table), block_table.shape[1], _ptr(cache_seqlens),
                                     _ptr(err_flag), _ptr(cs_table), _stream(q, stream)))


def rope_paged_kv_had(q, out_q, k, out_k, v, inv_freq, position, positions, q_norm, k_norm, norm_eps,
                      norm_constant_bias, rope_mode, attn_factor, k_cache, v_cache, block_table, cache_seqlens,
                      q_post_scale=None, k_post_scale=None, v_post_scale=None, position_ids=None, err_flag=None,
                      stream=None, cs_table=None, exact=False):
    """rope_paged_kv() on the raw f16 outputs of the q / k / v projections (heads packed), each first given
    its projection's output rotation had_r_128(y, y, None, svh) (src/modules.rs:231).  Outside the fused
    launch (head_dim 128, 16-byte aligned) v, and k when out_k is None, are rotated in place.  The fused
    launch runs the rotations on the matrix cores; exact=True: the reference's butterfly."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be (bsz, seq_len, heads, head_dim)")
    bsz, seq, hq, hd = q.shape
    hk = k.shape[2]
    if k.shape != v.shape or k.shape[:2] != q.shape[:2] or k.shape[3] != hd:
        raise ValueError("k and v must be (bsz, seq_len, kv_heads, head_dim) like q")
    for t in (q, k, v) + ((out_k,) if out_k is not None else ()):
        if t.stride(3) != 1 or t.stride(2) != hd or (seq > 1 and bsz > 1 and t.stride(0) != seq * t.stride(1)):
            raise ValueError("q / k / v / out_k: packed heads and batch stride seq_len * token stride")
    if out_q.stride() != q.stride() or out_q.shape != q.shape or (out_k is not None and out_k.stride() != k.stride()):
        raise ValueError("out_q / out_k must share q's / k's layout")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.shape[2:] != (hk, hd) or \
            not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("caches must be contiguous (pages, page_size, kv_heads, head_dim)")
    if block_table.dim() != 2 or block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32:
        raise TypeError("block_table (bsz, max_blocks) and cache_seqlens (bsz) must be int32")
    nw = q_norm if q_norm is not None else k_norm
    check(load().exl3r_rope_paged_kv_had(_ptr(q), _ptr(out_q), q.stride(1), hq, _ptr(k), _ptr(out_k), k.stride(1),
                                         _ptr(v), v.stride(1), hk, dtype_code(q), bsz, seq, hd, _ptr(inv_freq),
                                         _rotary_dim(inv_freq, cs_table, bsz * seq, q.device), int(position), _ptr(positions),
                                         _ptr(position_ids),
                                         _ptr(q_norm), _ptr(k_norm), dtype_code(nw) if nw is not None else F16,
                                         norm_eps, norm_constant_bias, rope_mode | (HAD_EXACT if exact else 0),
                                         attn_factor, _ptr(k_cache), _ptr(v_cache), k_cache.shape[1], k_cache.shape[0],
                                         _ptr(block_table), block_table.shape[1], _ptr(cache_seqlens), _ptr(err_flag),
                                         _ptr(q_post_scale), _ptr(k_post_scale), _ptr(v_post_scale),
                                         _ptr(cs_table), _stream(q, stream)))


def rope_run(stream=None, **fields):
    """exl3r_rope_run: every RoPE variant through one descriptor (exl3r_rope_desc).  Fields by name;
    tensors pass their device pointers, None a null pointer, the rest their values; struct_size is set
    here.  The variant and its checks follow from the fields that are set (see the header).
    attn_factor defaults to 1.0 (the unscaled rotation), as the Rust binding's Default does."""
    d = RopeDesc()
    d.struct_size = ctypes.sizeof(RopeDesc)
    d.attn_factor = 1.0
    names = {f[0] for f in RopeDesc._fields_}
    first = None
    for key, val in fields.items():
        if key not in names or key == "struct_size":
            raise TypeError(f"rope_run: unknown field {key}")
        if isinstance(val, torch.Tensor):
            first = first if first is not None else val
            val = val.data_ptr()
        elif val is None:
            val = 0
        setattr(d, key, val)
    s = _stream(first, stream) if first is not None else (stream or 0)
    check(load().exl3r_rope_run(ctypes.byref(d), s))


def argmax_sample(logits, ids, max_logit=0, stream=None):
    """ids[i] = first index of the maximum of logits[i, :max_logit] (NaN maximal), int64
    (src/ffi.rs:521-525; the generator's batched argmax)."""
    rows, vocab, ld = _rows(logits)
    if ids.dtype != torch.int64 or ids.numel() != rows:
        raise ValueError("ids must be int64 with one entry per row")
    check(load().exl3r_argmax_sample(_ptr(logits), dtype_code(logits), rows, vocab, ld, int(max_logit), _ptr(ids),
                                     _stream(logits, stream)))


def gumbel_sample(logits, ids, max_logit=0, random=0, stream=None):
    """ids[i] = argmax of logits[i, :max_logit] + Gumbel(0, 1) noise of (random, i, column): a draw from
    softmax(logits[i, :max_logit]) (src/ffi.rs:526-530)."""
    rows, vocab, ld = _rows(logits)
    if ids.dtype != torch.int64 or ids.numel() != rows:
        raise ValueError("ids must be int64 with one entry per row")
    check(load().exl3r_gumbel_sample(_ptr(logits), dtype_code(logits), rows, vocab, ld, int(max_logit),
                                     int(random) & 0xFFFFFFFF, _ptr(ids), _stream(logits, stream)))


def sample_workspace_bytes():
    """Bytes of the workspace argmax_sample_ws / gumbel_sample_ws take (any shape up to 384 rows)."""
    return int(load().exl3r_sample_workspace_bytes())


def _workspace(ws, logits):
    if ws is None or ws.device != logits.device or not ws.is_contiguous() or ws.data_ptr() % 256:
        raise ValueError("workspace must be a contiguous 256-byte aligned tensor on the logits' device")
    return _ptr(ws), ws.numel() * ws.element_size()


def argmax_sample_ws(logits, ids, workspace, max_logit=0, stream=None):
    """argmax_sample in one launch below 128 rows, the row counters and slots in `workspace` (at least
    sample_workspace_bytes() bytes, zero before the first use; every call leaves it zero).  The ids are
    identical to argmax_sample's."""
    rows, vocab, ld = _rows(logits)
    if ids.dtype != torch.int64 or ids.numel() != rows:
        raise ValueError("ids must be int64 with one entry per row")
    wp, wb = _workspace(workspace, logits)
    check(load().exl3r_argmax_sample_ws(_ptr(logits), dtype_code(logits), rows, vocab, ld, int(max_logit), _ptr(ids),
                                        wp, wb, _stream(logits, stream)))


def gumbel_sample_ws(logits, ids, workspace, max_logit=0, random=0, stream=None):
    """gumbel_sample in one launch below 384 rows, with the workspace of argmax_sample_ws; the same draws."""
    rows, vocab, ld = _rows(logits)
    if ids.dtype != torch.int64 or ids.numel() != rows:
        raise ValueError("ids must be int64 with one entry per row")
    wp, wb = _workspace(workspace, logits)
    check(load().exl3r_gumbel_sample_ws(_ptr(logits), dtype_code(logits), rows, vocab, ld, int(max_logit),
                                        int(random) & 0xFFFFFFFF, _ptr(ids), wp, wb, _stream(logits, stream)))


def gumbel_noise(x, out, random=0, stream=None):
    """out = x + the Gumbel noise of gumbel_sample (src/ffi.rs:531-535); out may be x."""
    rows, cols, ldx = _rows(x)
    ro, co, ldo = _rows(out)
    if (ro, co) != (rows, cols):
        raise ValueError("x and out must have the same shape")
    check(load().exl3r_gumbel_noise(_ptr(x), dtype_code(x), ldx, _ptr(out), dtype_code(out), ldo, rows, cols,
                                    int(random) & 0xFFFFFFFF, _stream(x, stream)))


def had_r_128(x, out, pre_scale=None, post_scale=None, scale=1.0, stream=None, mfma=False):
    """Random-Hadamard transform of [rows, k] f16 / f32 x into out (k % 128 == 0), with an optional f16
    per-column pre_scale (before) or post_scale (after) (src/ffi.rs:604-608).  mfma=True: the transform on
    the matrix cores (exl3r_had_r_128_mfma, f16 only; within the stated rounding tolerance)."""
    rows, cols, ldx = _rows(x)
    ro, co, ldo = _rows(out)
    if (ro, co) != (rows, cols) or out.dtype != x.dtype:
        raise ValueError("x and out must share shape and dtype")
    for t in (pre_scale, post_scale):
        if t is not None and (t.dtype != torch.float16 or t.numel() != cols or not t.is_contiguous()):
            raise ValueError("scales must be contiguous f16 with one entry per column")
    fn = load().exl3r_had_r_128_mfma if mfma else load().exl3r_had_r_128
    check(fn(_ptr(x), dtype_code(x), ldx, _ptr(out), ldo, rows, cols, _ptr(pre_scale), _ptr(post_scale), float(scale),
             _stream(x, stream)))


def rms_norm_had(x, w, outs, pre_scales, eps, constant_bias=0.0, constant_scale=1.0, r=None, y=None, had_scale=1.0,
                 rotate_x=False, x_post_scale=None, stream=None, exact=False):
    """One pass: y = RMSNorm(x) (or r += x; y = RMSNorm(r)) in f16, then outs[i] = had_r_128(y, pre_scales[i])
    for each projection (1..4 f16 outputs shaped like x; y is written only if given).  rotate_x: x (f16) is
    first taken through its producer's output rotation had_r_128(x, post_scale=x_post_scale).  The
    transforms run on the matrix cores; exact=True: the reference's butterfly (EXL3R_HAD_EXACT)."""
    rows, dim, ldx = _rows(x)
    if not 1 <= len(outs) <= 4 or len(pre_scales) != len(outs):
        raise ValueError("1..4 outputs, one pre_scale (or None) each")
    ldo = None
    for o in outs:
        ro, co, lo = _rows(o)
        if (ro, co) != (rows, dim) or o.dtype != torch.float16 or (ldo is not None and lo != ldo):
            raise ValueError("outputs must be f16 shaped like x with one row stride")
        ldo = lo
    ldr = _rows(r)[2] if r is not None else 0
    ldy = _rows(y)[2] if y is not None else 0
    if y is not None and y.dtype != torch.float16:
        raise ValueError("y is the f16 norm output")
    arr = ctypes.c_void_p * len(outs)
    pre = arr(*[_ptr(p) for p in pre_scales])
    out = arr(*[_ptr(o) for o in outs])
    check(load().exl3r_rms_norm_had(_ptr(x), dtype_code(x), ldx, _ptr(w), dtype_code(w) if w is not None else F16,
                                    _ptr(r), dtype_code(r) if r is not None else F16, ldr, _ptr(y), ldy, len(outs),
                                    pre, out, ldo, rows, dim, eps, constant_bias, constant_scale, float(had_scale),
                                    (1 if rotate_x else 0) | (HAD_EXACT if exact else 0), _ptr(x_post_scale),
                                    _stream(x, stream)))


ACT_CODES = {"silu": 0, "gelu": 1, "mul_sigmoid": 2}


def act_mul_had(act, x, y, out, pre_scale=None, z=None, act_limit=0.0, had_scale=1.0, rotate_x=False, rotate_y=False,
                x_post_scale=None, y_post_scale=None, stream=None, exact=False):
    """One pass: z = silu(x) * y, gelu(x) * y or x * sigmoid(y) in f16, then out = had_r_128(z, pre_scale)
    (f16 [rows, cols], cols % 128 == 0); z is written only if given.  rotate_x / rotate_y: the f16 input is
    first given its projection's output rotation had_r_128(v, post_scale=x_post_scale / y_post_scale).
    The transforms run on the matrix cores; exact=True: the reference's butterfly (EXL3R_HAD_EXACT),
    bit-identical to the unfused calls."""
    rows, cols, ldx = _rows(x)
    ry, cy, ldy = _rows(y)
    ro, co, ldo = _rows(out)
    if (ry, cy) != (rows, cols) or (ro, co) != (rows, cols) or y.dtype != x.dtype or out.dtype != torch.float16:
        raise ValueError("y like x; out f16 shaped like x")
    ldz = 0
    if z is not None:
        rz, cz, ldz = _rows(z)
        if (rz, cz) != (rows, cols) or z.dtype != torch.float16:
            raise ValueError("z is the f16 activation shaped like x")
    check(load().exl3r_act_mul_had(ACT_CODES[act], _ptr(x), _ptr(y), dtype_code(x), ldx, ldy, _ptr(z), ldz,
                                   _ptr(pre_scale), _ptr(out), ldo, rows, cols, act_limit, float(had_scale),
                                   (1 if rotate_x else 0) | (2 if rotate_y else 0) | (HAD_EXACT if exact else 0),
                                   _ptr(x_post_scale),
                                   _ptr(y_post_scale), _stream(x, stream)))


def embedding(table, ids, out, err_flag=None, stream=None):
    """out[i] = table[ids[i]] (bit-exact, or exact upcast to f32)."""
    vocab, hidden = table.shape
    n = ids.numel()
    ro, ho, ldo = _rows(out)
    if (ro, ho) != (n, hidden):
        raise ValueError("out must be [ids.numel(), hidden]")
    check(load().exl3r_embedding(_ptr(table), dtype_code(table), vocab, hidden, table.stride(0),
                                 _ptr(ids), dtype_code(ids), n, _ptr(out), dtype_code(out), ldo,
                                 _ptr(err_flag), _stream(table, stream)))


def embedding_rms_norm(table, ids, h, w, y, eps, constant_bias=0.0, constant_scale=1.0, err_flag=None,
                       stream=None):
    """h[i] = table[ids[i]] (h may be None), y = RMSNorm(h) * (w + constant_bias) * constant_scale."""
    vocab, hidden = table.shape
    n = ids.numel()
    ry, hy, ldy = _rows(y)
    if (ry, hy) != (n, hidden):
        raise ValueError("y must be [ids.numel(), hidden]")
    ldh, ht = hidden, F32
    if h is not None:
        rh, hh, ldh = _rows(h)
        if (rh, hh) != (n, hidden):
            raise ValueError("h must be [ids.numel(), hidden]")
        ht = dtype_code(h)
    check(load().exl3r_embedding_rms_norm(_ptr(table), dtype_code(table), vocab, hidden, table.stride(0),
                                          _ptr(ids), dtype_code(ids), n, _ptr(h), ht, ldh,
                                          _ptr(w), dtype_code(w) if w is not None else F16,
                                          _ptr(y), dtype_code(y), ldy, eps, constant_bias, constant_scale,
                                          _ptr(err_flag), _stream(table, stream)))
