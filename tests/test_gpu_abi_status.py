"""An entry point's status covers its own launches only: a HIP error that another caller left pending
on the thread is neither reported as the entry point's nor cleared by it.  The pending error comes from
hipSetDevice with an ordinal past the device count (refused on the host; nothing reaches the GPU), and
the entry points are called through the C ABI directly, so no torch call runs in between."""
import ctypes

import pytest
import torch

import exl3r
from exl3r import _lib


def hip():
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipGetErrorName.restype = ctypes.c_char_p
    return lib


@pytest.mark.gpu
def test_pending_error_is_left_to_its_owner():
    lib, h = exl3r.load(), hip()
    torch.cuda.set_device(0)
    g = torch.randn(64, 1024, device="cuda").half()
    u = torch.randn(64, 1024, device="cuda").half()
    z = torch.empty_like(g)
    torch.cuda.synchronize()
    h.hipGetLastError()   # start from a clear slot (torch may have left something)
    n = ctypes.c_int()
    assert h.hipGetDeviceCount(ctypes.byref(n)) == 0
    assert h.hipSetDevice(n.value + 7) != 0
    pending = h.hipPeekAtLastError()
    assert pending != 0, "hipSetDevice past the device count left no pending error"
    print("pending:", h.hipGetErrorName(pending).decode(), flush=True)
    rc = lib.exl3r_silu_mul(ctypes.c_void_p(g.data_ptr()), ctypes.c_void_p(u.data_ptr()), _lib.F16,
                            ctypes.c_void_p(z.data_ptr()), _lib.F16, 64, 1024, 1024, 1024, 1024,
                            ctypes.c_float(0.0), None)
    assert rc == 0, lib.exl3r_last_error()
    after = h.hipPeekAtLastError()
    assert after == pending, f"pending error changed: {h.hipGetErrorName(after).decode()}"
    assert h.hipGetLastError() == pending     # the owner reads (and clears) it
    assert h.hipGetLastError() == 0
    torch.cuda.synchronize()
    ref = torch.nn.functional.silu(g.float()) * u.float()
    assert torch.allclose(z.float(), ref, rtol=2e-3, atol=1e-3)


@pytest.mark.gpu
def test_validation_error_leaves_hip_state_alone():
    """A refused call (negative status, nothing launched) touches no HIP state either."""
    lib, h = exl3r.load(), hip()
    torch.cuda.set_device(0)
    torch.cuda.synchronize()
    h.hipGetLastError()
    rc = lib.exl3r_silu_mul(ctypes.c_void_p(16), ctypes.c_void_p(16), 99, ctypes.c_void_p(16), _lib.F16,
                            4, 64, 64, 64, 64, ctypes.c_float(0.0), None)
    assert rc == _lib.EDTYPE
    assert h.hipPeekAtLastError() == 0
