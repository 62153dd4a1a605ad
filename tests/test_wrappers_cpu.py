"""CPU checks of the host-side boundary beyond the C ABI: the product library carries no launch-shape
hooks (they live in the sweep/test build only), and the Python wrappers reject a {cos, sin} table that
does not cover the call's tokens, or an angle table where only inv_freq [R/2] is read, before anything
is launched (the kernels index the table by token and read inv_freq's first R/2 values)."""
import ctypes

import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from exl3r import _lib

from test_abi_cpu import declared_symbols


def test_product_library_has_no_tuning_hooks():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    present = [n for n in _lib.TUNE_PROTOTYPES if hasattr(lib, n)]
    assert not present, present


def test_tuning_build_exports_the_abi_and_its_hooks():
    lib = ctypes.CDLL(_lib.TUNE_PATH)
    missing = [n for n in list(_lib.TUNE_PROTOTYPES) + declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_tuned_context_restores_the_product_library():
    prod = _lib.load()
    with _lib.tuned() as tl:
        assert _lib.load() is tl and tl is not prod
    assert _lib.load() is prod


F16 = torch.float16


def qkv(bsz=1, seq=3, hq=4, hk=2, hd=128):
    q = torch.zeros((bsz, seq, hq, hd), dtype=F16)
    k = torch.zeros((bsz, seq, hk, hd), dtype=F16)
    v = torch.zeros((bsz, seq, hk, hd), dtype=F16)
    return q, k, v


def paged_args(hk=2, hd=128):
    kc = torch.zeros((4, 256, hk, hd), dtype=F16)
    return kc, kc.clone(), torch.zeros((1, 2), dtype=torch.int32), torch.zeros(1, dtype=torch.int32)


INV = torch.ones(64, dtype=torch.float32)


def call(op, inv_freq, cs_table):
    q, k, v = qkv()
    if op == "rope_had":
        ffi.rope_had(q, q.clone(), k, k.clone(), inv_freq, 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0,
                     cs_table=cs_table)
    elif op == "rope_paged_kv":
        kc, vc, bt, sl = paged_args()
        ffi.rope_paged_kv(q, q.clone(), k, k.clone(), v, inv_freq, 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX,
                          1.0, kc, vc, bt, sl, cs_table=cs_table)
    elif op == "rope_paged_kv_had":
        kc, vc, bt, sl = paged_args()
        ffi.rope_paged_kv_had(q, q.clone(), k, k.clone(), v, inv_freq, 0, None, None, None, 1e-6, 0.0,
                              exl3r.ROPE_NEOX, 1.0, kc, vc, bt, sl, cs_table=cs_table)
    else:
        qg = torch.zeros((1, 3, 4, 256), dtype=F16)
        ffi.rope_qg(qg, q.clone(), k, k.clone(), inv_freq, 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)


TABLE_OPS = ["rope_had", "rope_paged_kv", "rope_paged_kv_had"]


@pytest.mark.parametrize("op", TABLE_OPS)
def test_short_cs_table_is_rejected(op):
    """A table built for 2 tokens, passed to a 3-token call (a table kept across forward passes)."""
    with pytest.raises(ValueError, match="cs_table"):
        call(op, None, torch.zeros((2, 64, 2), dtype=torch.float32))


@pytest.mark.parametrize("op", TABLE_OPS)
@pytest.mark.parametrize("bad", ["f16", "strided", "pairs3", "rdim"])
def test_malformed_cs_table_is_rejected(op, bad):
    t = torch.zeros((3, 64, 2), dtype=torch.float32)
    if bad == "f16":
        t = t.to(F16)
    elif bad == "strided":
        t = torch.zeros((3, 64, 4), dtype=torch.float32)[..., :2]
    elif bad == "pairs3":
        t = torch.zeros((3, 64, 3), dtype=torch.float32)
    with pytest.raises(ValueError):
        call(op, torch.ones(32, dtype=torch.float32) if bad == "rdim" else None, t)


@pytest.mark.parametrize("op", TABLE_OPS)
def test_cs_table_on_another_device_is_rejected(op):
    with pytest.raises(ValueError, match="device"):
        call(op, None, torch.zeros((3, 64, 2), dtype=torch.float32, device="meta"))


@pytest.mark.parametrize("op", TABLE_OPS + ["rope_qg"])
def test_angle_table_as_inv_freq_is_rejected(op):
    """Only rope() reads a 2-D / 3-D angle table (RoPE::apply's freq_table); these entry points read
    inv_freq[0 .. R/2) and would take the table's first row (all zeros: nothing rotated)."""
    with pytest.raises(ValueError, match="inv_freq"):
        call(op, torch.zeros((16, 64), dtype=torch.float32), None)


@pytest.mark.parametrize("op", TABLE_OPS)
def test_no_frequency_source_is_rejected(op):
    with pytest.raises(ValueError, match="inv_freq or cs_table"):
        call(op, None, None)


@pytest.mark.skipif(torch.cuda.is_available(), reason="would launch on host tensors")
@pytest.mark.parametrize("op", TABLE_OPS)
def test_well_formed_table_passes_validation(op):
    """Control for the rejections above: a table that covers the call gets past every wrapper check and
    fails only where the launch needs a GPU."""
    with pytest.raises(RuntimeError, match="GPU"):
        call(op, INV, torch.zeros((3, 64, 2), dtype=torch.float32))
