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
        a.update(kw)
        return lib.exl3r_rope_paged_kv(*a.values(), None)
    assert call(page=100) == exl3r.EINVAL
    assert call(pages=0) == exl3r.EINVAL
    assert call(v=None) == exl3r.EINVAL
    assert call(kc=None) == exl3r.EINVAL
    assert call(bt=None) == exl3r.EINVAL
    assert call(vhs=32) == exl3r.EINVAL
    assert call(dt=F32) == exl3r.EDTYPE
    assert call(hkv=0) == exl3r.EINVAL
    assert call(q=None, oq=None, k=None, v=None, kc=None, vc=None, bt=None, sl=None, seq=0) == exl3r.OK
