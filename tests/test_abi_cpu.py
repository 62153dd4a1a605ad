"""CPU-side checks of the drop-in boundary: the HIP library loads without a GPU, exports every
symbol include/exl3r/rowops.h declares, and rejects invalid arguments with the documented status
codes and a message before touching the GPU (no compute is launched here)."""
import ctypes
import re

import pytest

import exl3r
from exl3r import _lib


def declared_symbols():
    text = open(_lib.HEADER_PATH).read()
    return sorted(set(re.findall(r"EXL3R_API\s+[\w\s\*]+?\b(exl3r_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("exl3r_rms_norm", "exl3r_rms_norm_res_in", "exl3r_silu_mul", "exl3r_gelu_mul", "exl3r_rope",
              "exl3r_embedding", "exl3r_embedding_rms_norm", "exl3r_last_error", "exl3r_version"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared_symbols()) <= set(_lib.PROTOTYPES)


def test_version():
    assert exl3r.load().exl3r_version() >= 10000


def _err():
    return exl3r.load().exl3r_last_error().decode()


FAKE = 0x1000   # never dereferenced: every call below fails validation first
F32, F16, BF16, I32, I64 = exl3r.F32, exl3r.F16, exl3r.BF16, exl3r.I32, exl3r.I64


def test_rms_norm_validation():
    lib = exl3r.load()
    assert lib.exl3r_rms_norm(None, F16, 64, None, F16, FAKE, F16, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EINVAL
    assert "non-null" in _err()
    assert lib.exl3r_rms_norm(FAKE, 7, 64, None, F16, FAKE, F16, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EDTYPE
    assert lib.exl3r_rms_norm(FAKE, F16, 32, None, F16, FAKE + 4096, F16, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EINVAL
    assert "stride" in _err()
    assert lib.exl3r_rms_norm(FAKE, F16, 64, None, F16, FAKE, F32, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EINVAL
    assert "in-place" in _err()
    assert lib.exl3r_rms_norm(FAKE, F16, 64, None, F16, FAKE + 64, F16, 64, 0, 64, 1e-6, 0.0, 1.0, None) == exl3r.OK


def test_rms_norm_res_in_validation():
    lib = exl3r.load()
    args = [FAKE, F16, 64, None, F16, FAKE + 4096, F16, 64]
    assert lib.exl3r_rms_norm_res_in(*args, None, F32, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EINVAL
    assert lib.exl3r_rms_norm_res_in(*args, FAKE + 4096, F32, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EINVAL
    assert "alias" in _err()
    assert lib.exl3r_rms_norm_res_in(*args, FAKE + 8192, I32, 64, 4, 64, 1e-6, 0.0, 1.0, None) == exl3r.EDTYPE


@pytest.mark.parametrize("name", ["exl3r_silu_mul", "exl3r_gelu_mul"])
def test_act_validation(name):
    fn = getattr(exl3r.load(), name)
    assert fn(FAKE, None, F16, FAKE, F16, 2, 8, 8, 8, 8, 0.0, None) == exl3r.EINVAL
    assert fn(FAKE, FAKE, I64, FAKE + 64, F16, 2, 8, 8, 8, 8, 0.0, None) == exl3r.EDTYPE
    assert fn(FAKE, FAKE + 64, F16, FAKE, F32, 2, 8, 8, 8, 8, 0.0, None) == exl3r.EINVAL
    assert fn(FAKE, FAKE + 64, F16, FAKE + 128, F16, 3, 8, 4, 8, 8, 0.0, None) == exl3r.EINVAL
    assert fn(FAKE, FAKE + 64, F16, FAKE + 128, F16, 0, 8, 8, 8, 8, 0.0, None) == exl3r.OK


def _rope(**kw):
    a = dict(q=FAKE, oq=FAKE, qts=4 * 64, qhs=64, hq=4, k=FAKE + 65536, ok=FAKE + 65536, kts=2 * 64, khs=64, hk=2,
             dt=F16, bsz=1, seq=3, hd=64, inv=FAKE + 131072, R=64, pos=0, positions=None, ids=None,
             qn=None, kn=None, nwt=F16, eps=1e-6, cb=0.0, mode=exl3r.ROPE_NEOX, attn=1.0)
    a.update(kw)
    return exl3r.load().exl3r_rope(*a.values(), None)


def test_rope_validation():
    assert _rope(mode=exl3r.ROPE_NONE) == exl3r.EINVAL
    assert "rope_mode" in _err()
    assert _rope(dt=F32) == exl3r.EDTYPE
    assert _rope(R=66) == exl3r.EINVAL
    assert _rope(R=0) == exl3r.EINVAL
    assert _rope(hd=63, qhs=63) == exl3r.EINVAL
    assert _rope(positions=FAKE, ids=FAKE) == exl3r.EINVAL
    assert _rope(qn=FAKE) == exl3r.EINVAL
    assert "k_norm" in _err()
    assert _rope(kn=FAKE) == exl3r.EINVAL
    assert _rope(qn=FAKE, kn=FAKE, nwt=I32) == exl3r.EDTYPE
    assert _rope(inv=None) == exl3r.EINVAL
    assert _rope(qts=64) == exl3r.EINVAL
    assert _rope(seq=0) == exl3r.OK


def test_embedding_validation():
    lib = exl3r.load()
    assert lib.exl3r_embedding(None, BF16, 10, 16, 16, FAKE, I32, 4, FAKE, BF16, 16, None, None) == exl3r.EINVAL
    assert lib.exl3r_embedding(FAKE, BF16, 10, 16, 16, FAKE, F32, 4, FAKE, BF16, 16, None, None) == exl3r.EDTYPE
    assert lib.exl3r_embedding(FAKE, F32, 10, 16, 16, FAKE, I32, 4, FAKE, BF16, 16, None, None) == exl3r.EDTYPE
    assert "exact" in _err()
    assert lib.exl3r_embedding(FAKE, BF16, 10, 16, 8, FAKE, I32, 4, FAKE, BF16, 16, None, None) == exl3r.EINVAL
    assert lib.exl3r_embedding(FAKE, BF16, 10, 16, 16, FAKE, I32, 0, FAKE, BF16, 16, None, None) == exl3r.OK
    assert lib.exl3r_embedding_rms_norm(FAKE, BF16, 10, 16, 16, FAKE, I32, 4, FAKE, F16, 16, None, BF16,
                                        FAKE + 4096, BF16, 16, 1e-6, 0.0, 1.0, None, None) == exl3r.EINVAL


def test_errors_are_thread_local():
    import threading
    lib = exl3r.load()
    lib.exl3r_rms_norm(None, F16, 64, None, F16, FAKE, F16, 64, 4, 64, 1e-6, 0.0, 1.0, None)
    seen = []

    def other():
        seen.append(lib.exl3r_last_error().decode())

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen == [""] and "non-null" in _err()


def test_zero_size_calls_accept_null_data():
    """Empty tensors carry null data pointers: a call with no rows / tokens / ids validates its
    shapes and dtypes, launches nothing and succeeds (no GPU needed)."""
    lib = exl3r.load()
    assert lib.exl3r_rms_norm(None, F16, 64, None, F16, None, F16, 64, 0, 64, 1e-6, 0.0, 1.0, None) == exl3r.OK
    assert lib.exl3r_rms_norm(None, 9, 64, None, F16, None, F16, 64, 0, 64, 1e-6, 0.0, 1.0, None) == exl3r.EDTYPE
    assert lib.exl3r_rms_norm_res_in(None, F16, 64, None, F16, None, F16, 64, None, F32, 64, 0, 64,
                                     1e-6, 0.0, 1.0, None) == exl3r.OK
    for fn in (lib.exl3r_silu_mul, lib.exl3r_gelu_mul):
        assert fn(None, None, BF16, None, BF16, 0, 17408, 17408, 17408, 17408, 0.0, None) == exl3r.OK
        assert fn(None, None, I32, None, BF16, 0, 8, 8, 8, 8, 0.0, None) == exl3r.EDTYPE
    assert _rope(q=None, oq=None, k=None, ok=None, seq=0) == exl3r.OK
    assert _rope(q=None, oq=None, k=None, ok=None, seq=0, mode=0) == exl3r.EINVAL
    assert lib.exl3r_embedding(FAKE, BF16, 10, 16, 16, None, I64, 0, None, F32, 16, None, None) == exl3r.OK
    assert lib.exl3r_embedding_rms_norm(FAKE, BF16, 10, 16, 16, None, I64, 0, None, BF16, 16, None, BF16,
                                        None, BF16, 16, 1e-6, 0.0, 1.0, None, None) == exl3r.OK


def test_rope_paged_kv_validation():
    lib = exl3r.load()
    inv, kc, vc, bt, sl = FAKE + 131072, FAKE + 262144, FAKE + 393216, FAKE + 524288, FAKE + 528384

    def call(**kw):
        a = dict(q=FAKE, oq=FAKE, qts=4 * 64, qhs=64, hq=4, k=FAKE + 65536, ok=None, kts=2 * 64, khs=64,
                 v=FAKE + 98304, vts=2 * 64, vhs=64, hkv=2, dt=F16, bsz=1, seq=3, hd=64, inv=inv, R=64, pos=0,
                 positions=None, ids=None, qn=None, kn=None, nwt=F16, eps=1e-6, cb=0.0, mode=exl3r.ROPE_NEOX, attn=1.0,
                 kc=kc, vc=vc, page=256, pages=4, bt=bt, mb=2, sl=sl, err=None)
        cs = kw.pop("cs", None)
        a.update(kw)
        return lib.exl3r_rope_paged_kv(*a.values(), cs, None)
    assert call(page=100) == exl3r.EINVAL
    assert call(pages=0) == exl3r.EINVAL
    assert call(v=None) == exl3r.EINVAL
    assert call(kc=None) == exl3r.EINVAL
    assert call(bt=None) == exl3r.EINVAL
    assert call(vhs=32) == exl3r.EINVAL
    assert call(dt=F32) == exl3r.EDTYPE
    assert call(hkv=0) == exl3r.EINVAL
    assert call(cs=FAKE + 65540) == exl3r.EINVAL and "cs_table" in _err()    # misaligned {cos, sin} table
    assert call(inv=None) == exl3r.EINVAL                                      # no rotation source
    assert call(q=None, oq=None, k=None, v=None, kc=None, vc=None, bt=None, sl=None, seq=0) == exl3r.OK


def test_gated_and_gate_ops_validation():
    lib = exl3r.load()
    # exl3r_gated_rms_norm(x, xt, ldx, w, wt, w_groups, y, yt, ldy, g, gt, ldg, rows, dim, eps, cb, gate_first, gate_act)
    base = [FAKE, BF16, 128, None, F32, 1, FAKE + 65536, F16, 128, FAKE + 131072, F32, 128, 4, 128, 1e-6, 0.0, 0, 0]
    def gated(**kw):
        a = list(base)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lib.exl3r_gated_rms_norm(*a, None)
    assert gated(a10=7) == exl3r.EDTYPE
    assert gated(a11=64) == exl3r.EINVAL and "gate row stride" in _err()
    assert gated(a5=0) == exl3r.EINVAL and "w_groups" in _err()
    assert gated(a17=2) == exl3r.EINVAL and "gate_act" in _err()
    assert gated(a9=None) == exl3r.EINVAL
    assert gated(a9=FAKE + 65536) == exl3r.EINVAL and "alias" in _err()
    assert gated(a12=0) == exl3r.OK
    # exl3r_mul_sigmoid(x, y, in_dtype, z, z_dtype, rows, cols, ldx, ldy, ldz)
    assert lib.exl3r_mul_sigmoid(FAKE, FAKE + 4096, 7, FAKE + 8192, F16, 2, 8, 8, 8, 8, None) == exl3r.EDTYPE
    assert lib.exl3r_mul_sigmoid(FAKE, FAKE + 4096, F16, FAKE + 8192, F16, 2, 8, 4, 8, 8, None) == exl3r.EINVAL
    assert lib.exl3r_mul_sigmoid(FAKE, FAKE + 4096, F16, FAKE + 8192, F16, 0, 8, 8, 8, 8, None) == exl3r.OK
    # exl3r_deinterleave_qg(qg, ld_qg, q, ld_q, g, ld_g, dtype, rows, heads, head_dim)
    assert lib.exl3r_deinterleave_qg(FAKE, 512, FAKE + 4096, 256, FAKE + 8192, 256, I32, 2, 2, 128, None) == exl3r.EDTYPE
    assert lib.exl3r_deinterleave_qg(FAKE, 256, FAKE + 4096, 256, FAKE + 8192, 256, F16, 2, 2, 128, None) == exl3r.EINVAL
    assert lib.exl3r_deinterleave_qg(FAKE, 512, FAKE, 256, FAKE + 8192, 256, F16, 2, 2, 128, None) == exl3r.EINVAL
    assert "alias" in _err()
    assert lib.exl3r_deinterleave_qg(None, 512, None, 256, None, 256, F16, 0, 2, 128, None) == exl3r.OK


def test_sampling_validation():
    lib = exl3r.load()
    for fn, extra in ((lib.exl3r_argmax_sample, ()), (lib.exl3r_gumbel_sample, (7,))):
        # (logits, dtype, rows, vocab, ld, max_logit[, random], ids)
        assert fn(FAKE, I64, 2, 100, 100, 0, *extra, FAKE + 4096, None) == exl3r.EDTYPE
        assert fn(FAKE, F16, 2, 0, 100, 0, *extra, FAKE + 4096, None) == exl3r.EINVAL
        assert fn(FAKE, F16, 2, 100, 50, 0, *extra, FAKE + 4096, None) == exl3r.EINVAL and "ld" in _err()
        assert fn(FAKE, F16, 2, 100, 100, 0, *extra, None, None) == exl3r.EINVAL and "non-null" in _err()
        assert fn(None, F16, 0, 100, 100, 0, *extra, None, None) == exl3r.OK
    # the one-launch forms: (..., ids, workspace, workspace_bytes)
    need = lib.exl3r_sample_workspace_bytes()
    assert need == 384 * (4 + 8)                            # a counter and a slot per row, up to 384 rows
    for fn, extra in ((lib.exl3r_argmax_sample_ws, ()), (lib.exl3r_gumbel_sample_ws, (7,))):
        ws = FAKE + (1 << 20)
        assert fn(FAKE, F16, 2, 151936, 151936, 0, *extra, FAKE + 4096, None, need, None) == exl3r.EINVAL
        assert "workspace" in _err()
        assert fn(FAKE, F16, 2, 151936, 151936, 0, *extra, FAKE + 4096, ws, need - 8, None) == exl3r.EINVAL
        assert "workspace" in _err() and str(need) in _err()
        assert fn(FAKE, F16, 2, 151936, 151936, 0, *extra, FAKE + 4096, ws + 128, need, None) == exl3r.EINVAL
        assert "aligned" in _err()
        assert fn(FAKE, I64, 2, 100, 100, 0, *extra, FAKE + 4096, ws, need, None) == exl3r.EDTYPE
        assert fn(None, F16, 0, 100, 100, 0, *extra, None, ws, need, None) == exl3r.OK
    # the allocation-free argmax validates before it looks up its scratch
    assert lib.exl3r_argmax_sample_noalloc(FAKE, I64, 2, 100, 100, 0, FAKE + 4096, None) == exl3r.EDTYPE
    assert lib.exl3r_argmax_sample_noalloc(FAKE, F16, 2, 100, 50, 0, FAKE + 4096, None) == exl3r.EINVAL
    assert lib.exl3r_argmax_sample_noalloc(FAKE, F16, 2, 100, 100, 0, None, None) == exl3r.EINVAL
    assert lib.exl3r_argmax_sample_noalloc(None, F16, 0, 100, 100, 0, None, None) == exl3r.OK
    # exl3r_gumbel_noise(x, x_dtype, ldx, out, out_dtype, ldo, rows, cols, random)
    assert lib.exl3r_gumbel_noise(FAKE, F16, 64, FAKE + 8192, I32, 64, 2, 64, 1, None) == exl3r.EDTYPE
    assert lib.exl3r_gumbel_noise(FAKE, F16, 32, FAKE + 8192, F32, 64, 2, 64, 1, None) == exl3r.EINVAL
    assert lib.exl3r_gumbel_noise(None, F16, 64, None, F32, 64, 2, 0, 1, None) == exl3r.OK


def test_rope_table_validation():
    lib = exl3r.load()
    def call(rows=16, bstride=0, table=FAKE + 65536):
        return lib.exl3r_rope_table(FAKE, FAKE, 4 * 64, 64, 4, None, None, 0, 64, 0, F16, 1, 3, 64, table, rows,
                                    bstride, 64, 0, None, None, None, None, F16, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0,
                                    None, None)
    assert call(rows=0) == exl3r.EINVAL and "table_rows" in _err()
    assert call(bstride=-1) == exl3r.EINVAL
    assert call(table=None) == exl3r.EINVAL and "angle table" in _err()


def test_rope_qg_validation():
    lib = exl3r.load()
    def rope_qg(**kw):
        # (qg, qg_ts, oq, hq, k, ok, k_ts, k_hs, hk, dtype, bsz, seq, hd, inv, R, pos, positions, ids, qn, kn, nwt, eps,
        #  cb, mode, attn)
        a = dict(qg=FAKE, qts=4 * 256, oq=FAKE + 65536, hq=4, k=None, ok=None, kts=0, khs=128, hk=0, dt=F16, bsz=1,
                 seq=3, hd=128, inv=FAKE + 131072, R=128, pos=0, positions=None, ids=None, qn=None, kn=None, nwt=F16,
                 eps=1e-6, cb=0.0, mode=exl3r.ROPE_NEOX, attn=1.0)
        a.update(kw)
        return lib.exl3r_rope_qg(*a.values(), None)
    assert rope_qg(oq=FAKE + 1024) == exl3r.EINVAL and "overlaps" in _err()
    assert rope_qg(dt=F32) == exl3r.EDTYPE
    assert rope_qg(qts=4 * 256 - 8) == exl3r.EINVAL                  # token stride below heads * 2 * head_dim
    assert rope_qg(hd=0) == exl3r.EINVAL
    assert rope_qg(seq=0) == exl3r.OK


def test_rope_cs_validation():
    lib = exl3r.load()
    # exl3r_rope_cs_table(bsz, seq, inv_freq, R, position, positions, position_ids, attn, cs_table)
    assert lib.exl3r_rope_cs_table(1, 3, FAKE, 63, 0, None, None, 1.0, FAKE + 65536, None) == exl3r.EINVAL
    assert lib.exl3r_rope_cs_table(1, 3, FAKE, 64, 0, FAKE, FAKE, 1.0, FAKE + 65536, None) == exl3r.EINVAL
    assert "at most one" in _err()
    assert lib.exl3r_rope_cs_table(1, 3, FAKE, 64, 0, None, None, 1.0, FAKE + 65540, None) == exl3r.EINVAL
    assert "aligned" in _err()
    assert lib.exl3r_rope_cs_table(1, 3, None, 64, 0, None, None, 1.0, FAKE + 65536, None) == exl3r.EINVAL
    assert lib.exl3r_rope_cs_table(0, 3, None, 64, 0, None, None, 1.0, None, None) == exl3r.OK

    def rope_cs(**kw):
        # (q, oq, q_ts, q_hs, hq, k, ok, k_ts, k_hs, hk, dtype, bsz, seq, hd, cs, R, qn, kn, nwt, eps, cb, mode)
        a = dict(q=FAKE, oq=FAKE, qts=4 * 64, qhs=64, hq=4, k=None, ok=None, kts=0, khs=64, hk=0, dt=F16, bsz=1,
                 seq=3, hd=64, cs=FAKE + 65536, R=64, qn=None, kn=None, nwt=F16, eps=1e-6, cb=0.0,
                 mode=exl3r.ROPE_NEOX)
        a.update(kw)
        return lib.exl3r_rope_cs(*a.values(), None)
    assert rope_cs(dt=F32) == exl3r.EDTYPE
    assert rope_cs(cs=None) == exl3r.EINVAL
    assert rope_cs(cs=FAKE + 65540) == exl3r.EINVAL and "aligned" in _err()
    assert rope_cs(R=128) == exl3r.EINVAL
    assert rope_cs(mode=3) == exl3r.EINVAL
    assert rope_cs(seq=0) == exl3r.OK


def test_hadamard_validation():
    lib = exl3r.load()
    # exl3r_had_r_128(x, dtype, ldx, out, ldo, rows, cols, pre, post, scale)
    assert lib.exl3r_had_r_128(FAKE, BF16, 256, FAKE + 8192, 256, 2, 256, None, None, 1.0, None) == exl3r.EDTYPE
    assert lib.exl3r_had_r_128(FAKE, F16, 200, FAKE + 8192, 200, 2, 200, None, None, 1.0, None) == exl3r.EINVAL
    assert "multiple of 128" in _err()
    assert lib.exl3r_had_r_128(FAKE, F16, 256, FAKE + 8192, 256, 2, 256, FAKE, FAKE, 1.0, None) == exl3r.EINVAL
    assert "at most one" in _err()
    assert lib.exl3r_had_r_128(None, F16, 256, None, 256, 0, 256, None, None, 1.0, None) == exl3r.OK
    # the matrix-core form: f16 only, same shape and scale checks
    assert lib.exl3r_had_r_128_mfma(FAKE, F32, 256, FAKE + 8192, 256, 2, 256, None, None, 1.0, None) == exl3r.EDTYPE
    assert lib.exl3r_had_r_128_mfma(FAKE, F16, 200, FAKE + 8192, 200, 2, 200, None, None, 1.0, None) == exl3r.EINVAL
    assert lib.exl3r_had_r_128_mfma(FAKE, F16, 256, FAKE + 8192, 256, 2, 256, FAKE, FAKE, 1.0, None) == exl3r.EINVAL
    assert "exl3r_had_r_128_mfma" in _err()
    assert lib.exl3r_had_r_128_mfma(None, F16, 256, None, 256, 0, 256, None, None, 1.0, None) == exl3r.OK

    arr = ctypes.c_void_p * 4
    outs, pres = arr(FAKE + 65536, FAKE + 131072, 0, 0), arr(0, 0, 0, 0)
    def norm_had(**kw):
        # (x, xt, ldx, w, wt, r, rt, ldr, y, ldy, n_out, pres, outs, ldo, rows, dim, eps, cb, cs, had_scale,
        #  rotate_x, x_post)
        a = dict(x=FAKE, xt=F16, ldx=256, w=None, wt=F16, r=None, rt=F32, ldr=256, y=None, ldy=256, n=2, pres=pres,
                 outs=outs, ldo=256, rows=4, dim=256, eps=1e-6, cb=0.0, cs=1.0, hs=1.0, rot=0, xpost=None)
        a.update(kw)
        return lib.exl3r_rms_norm_had(*a.values(), None)
    assert norm_had(dim=200, ldx=200, ldo=200) == exl3r.EINVAL
    assert norm_had(n=5) == exl3r.EINVAL and "n_out" in _err()
    assert norm_had(xt=7) == exl3r.EDTYPE
    assert norm_had(rot=1, xt=BF16) == exl3r.EDTYPE and "rotate_x" in _err()
    assert norm_had(xpost=FAKE) == exl3r.EINVAL and "rotate_x" in _err()
    assert norm_had(rot=2) == exl3r.EINVAL and "rotate_x" in _err()
    assert norm_had(outs=arr(FAKE, FAKE + 131072, 0, 0)) == exl3r.EINVAL and "alias" in _err()
    assert norm_had(outs=arr(FAKE + 65536, FAKE + 65536, 0, 0)) == exl3r.EINVAL and "alias" in _err()
    assert norm_had(rows=0) == exl3r.OK

    def act_had(**kw):
        # (act, x, y, in_dtype, ldx, ldy, z, ldz, pre, out, ldo, rows, cols, act_limit, had_scale, rotate_in,
        #  x_post, y_post)
        a = dict(act=0, x=FAKE, y=FAKE + 8192, it=F16, ldx=256,
                 ldy=256, z=None, ldz=256, pre=None, out=FAKE + 65536, ldo=256, rows=4, cols=256, lim=0.0, hs=1.0,
                 rot=0, xp=None, yp=None)
        a.update(kw)
        return lib.exl3r_act_mul_had(*a.values(), None)
    assert act_had(act=9) == exl3r.EINVAL and "unknown act" in _err()
    assert act_had(cols=200, ldx=200, ldy=200, ldo=200) == exl3r.EINVAL
    assert act_had(out=FAKE) == exl3r.EINVAL and "alias" in _err()
    assert act_had(rot=4) == exl3r.EINVAL
    assert act_had(rot=1, it=BF16) == exl3r.EDTYPE
    assert act_had(yp=FAKE) == exl3r.EINVAL and "post-scale" in _err()
    assert act_had(act=2, lim=1.0) == exl3r.EINVAL and "act_limit" in _err()
    assert act_had(rows=0) == exl3r.OK


def test_rope_had_validation():
    lib = exl3r.load()
    def rope_had(**kw):
        # (q, oq, q_ts, hq, k, ok, k_ts, hk, dtype, bsz, seq, hd, inv, R, pos, positions, ids, qn, kn, nwt, eps, cb,
        #  mode, attn, q_post, k_post)
        a = dict(q=FAKE, oq=FAKE, qts=4 * 128, hq=4, k=None, ok=None, kts=0, hk=0, dt=F16, bsz=1, seq=3, hd=128,
                 inv=FAKE + 65536, R=128, pos=0, positions=None, ids=None, qn=None, kn=None, nwt=F16, eps=1e-6, cb=0.0,
                 mode=exl3r.ROPE_NEOX, attn=1.0, qp=None, kp=None)
        cs = kw.pop("cs", None)
        a.update(kw)
        return lib.exl3r_rope_had(*a.values(), cs, None)
    assert rope_had(dt=BF16) == exl3r.EDTYPE
    assert rope_had(hq=3, hd=64, R=64, qts=3 * 64) == exl3r.EINVAL and "multiple of 128" in _err()
    assert rope_had(kp=FAKE) == exl3r.EINVAL
    assert rope_had(inv=None, cs=FAKE + 65540) == exl3r.EINVAL and "cs_table" in _err()
    assert rope_had(inv=None) == exl3r.EINVAL
    assert rope_had(seq=0) == exl3r.OK

    def paged_had(**kw):
        a = dict(q=FAKE, oq=FAKE, qts=4 * 128, hq=4, k=FAKE + 65536, ok=None, kts=2 * 128, v=FAKE + 98304,
                 vts=2 * 128, hkv=2, dt=F16, bsz=1, seq=3, hd=128, inv=FAKE + 131072, R=128, pos=0, positions=None,
                 ids=None, qn=None, kn=None, nwt=F16, eps=1e-6, cb=0.0, mode=exl3r.ROPE_NEOX, attn=1.0,
                 kc=FAKE + 262144, vc=FAKE + 393216, page=256, pages=4, bt=FAKE + 524288, mb=2, sl=FAKE + 528384,
                 err=None, qp=None, kp=None, vp=None)
        cs = kw.pop("cs", None)
        a.update(kw)
        return lib.exl3r_rope_paged_kv_had(*a.values(), cs, None)
    assert paged_had(dt=BF16) == exl3r.EDTYPE
    assert paged_had(page=100) == exl3r.EINVAL
    assert paged_had(cs=FAKE + 65540) == exl3r.EINVAL and "cs_table" in _err()
    assert paged_had(v=None) == exl3r.EINVAL
    assert paged_had(hkv=0) == exl3r.EINVAL
    assert paged_had(seq=0, q=None, oq=None, k=None, v=None, kc=None, vc=None, bt=None, sl=None) == exl3r.OK


def test_gated_rms_norm_had_validation():
    lib = exl3r.load()
    def call(**kw):
        # (x, xt, ldx, w, wt, w_groups, g, gt, ldg, y, ldy, pre, pre_rows, out, ldo, rows, dim, eps, cb, first, act, hs)
        a = dict(x=FAKE, xt=BF16, ldx=128, w=None, wt=F32, wg=1, g=FAKE + 65536, gt=F32, ldg=128, y=None, ldy=128,
                 pre=None, pre_rows=1, out=FAKE + 131072, ldo=128, rows=4, dim=128, eps=1e-6, cb=0.0, first=0, act=0,
                 hs=1.0)
        a.update(kw)
        return lib.exl3r_gated_rms_norm_had(*a.values(), None)
    assert call(dim=100, ldx=100, ldg=100, ldo=100) == exl3r.EINVAL and "multiple of 128" in _err()
    assert call(gt=7) == exl3r.EDTYPE
    assert call(pre_rows=0) == exl3r.EINVAL
    assert call(pre_rows=3) == exl3r.EINVAL and "pre_rows" in _err()
    assert call(act=2) == exl3r.EINVAL
    assert call(out=FAKE, xt=F16) == exl3r.EINVAL and "alias" in _err()
    assert call(out=FAKE + 65536) == exl3r.EINVAL and "alias" in _err()
    assert call(g=None) == exl3r.EINVAL
    assert call(rows=0) == exl3r.OK
