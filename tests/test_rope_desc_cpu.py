"""CPU checks of exl3r_rope_run, the descriptor form of the RoPE entry points: the Python mirror of
exl3r_rope_desc has the C header's size and field offsets (a C program compiled here prints them), and
the router rejects descriptors that name no variant or several before anything reaches the GPU."""
import ctypes
import os
import subprocess
import tempfile

import pytest

import exl3r
import exl3r.ffi as ffi
from exl3r import _lib

FAKE = 0x1000   # never dereferenced: every call below fails validation first


def c_layout():
    names = [f[0] for f in _lib.RopeDesc._fields_]
    src = "#include <stddef.h>\n#include <stdio.h>\n#include \"exl3r/rowops.h\"\nint main(void) {\n"
    src += '  printf("size %zu\\n", sizeof(exl3r_rope_desc));\n'
    for n in names:
        src += f'  printf("{n} %zu\\n", offsetof(exl3r_rope_desc, {n}));\n'
    src += "  return 0;\n}\n"
    inc = os.path.dirname(os.path.dirname(_lib.HEADER_PATH))
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-I", inc, c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (line.split() for line in out.strip().splitlines())}


def test_python_mirror_matches_the_header():
    lay = c_layout()
    assert lay.pop("size") == ctypes.sizeof(_lib.RopeDesc)
    for name, off in lay.items():
        assert getattr(_lib.RopeDesc, name).offset == off, name


def base(**kw):
    d = dict(dtype=exl3r.F16, bsz=1, seq_len=4, head_dim=128, rotary_dim=128, rope_mode=exl3r.ROPE_NEOX,
             attn_factor=1.0, q=FAKE, out_q=FAKE, q_tok_stride=256, q_head_stride=128, num_heads_q=2,
             inv_freq=FAKE)
    d.update(kw)
    return d


@pytest.mark.parametrize("case,kw", [
    ("no source", dict(inv_freq=None)),
    ("two sources", dict(angle_table=FAKE, table_rows=8)),
    ("table and cs", dict(inv_freq=None, angle_table=FAKE, table_rows=8, cs_table=FAKE)),
    ("post-scale without rotate", dict(q_post_scale=FAKE)),
    ("v without k_cache", dict(v=FAKE)),
    ("angle table with the cache", dict(inv_freq=None, angle_table=FAKE, table_rows=8, k_cache=FAKE)),
    ("own out_q layout with cs", dict(inv_freq=None, cs_table=FAKE, out_q_head_stride=64)),
    ("own out_q layout that is not the q|g split", dict(out_q_head_stride=64)),
    ("rotate with padded heads", dict(rotate=1, q_head_stride=192, q_tok_stride=384)),
    ("rotate 2", dict(rotate=2)),
    ("EXL3R_HAD_EXACT without rotate", dict(rotate=16)),
])
def test_router_rejects(case, kw):
    with pytest.raises(exl3r.Exl3rError) as e:
        ffi.rope_run(stream=0, **base(**kw))
    assert e.value.code == _lib.EINVAL, case
    assert "exl3r_rope_run" in str(e.value), case


def test_selected_entry_point_checks_apply():
    """A descriptor that names a variant is checked by that variant's entry point (its message)."""
    with pytest.raises(exl3r.Exl3rError) as e:
        ffi.rope_run(stream=0, **base(dtype=exl3r.F32))
    assert "exl3r_rope:" in str(e.value)
    with pytest.raises(exl3r.Exl3rError) as e:
        ffi.rope_run(stream=0, **base(rotate=1, dtype=exl3r.BF16))
    assert "exl3r_rope_had" in str(e.value)


def test_struct_size_and_null():
    lib = exl3r.load()
    d = _lib.RopeDesc()
    for k, v in base().items():
        setattr(d, k, v)
    d.struct_size = ctypes.sizeof(d) - 8
    assert lib.exl3r_rope_run(ctypes.byref(d), None) == _lib.EINVAL
    assert "struct_size" in lib.exl3r_last_error().decode()
    assert lib.exl3r_rope_run(None, None) == _lib.EINVAL


def test_attn_factor_default_and_zero():
    """rope_run sets attn_factor = 1.0 unless given (the Rust binding's Default): a descriptor without it
    reaches the selected entry point's own checks.  A raw zero-initialised descriptor (attn_factor 0)
    or a NaN attn_factor is refused before any launch."""
    kw = base(dtype=exl3r.F32)
    del kw["attn_factor"]
    with pytest.raises(exl3r.Exl3rError) as e:
        ffi.rope_run(stream=0, **kw)
    assert "exl3r_rope:" in str(e.value)
    lib = exl3r.load()
    for bad in (0.0, -0.0, float("nan")):
        d = _lib.RopeDesc()
        for k, v in base(attn_factor=bad).items():
            setattr(d, k, v)
        d.struct_size = ctypes.sizeof(d)
        assert lib.exl3r_rope_run(ctypes.byref(d), None) == _lib.EINVAL, bad
        assert "attn_factor" in lib.exl3r_last_error().decode(), bad


def test_unknown_field():
    with pytest.raises(TypeError):
        ffi.rope_run(stream=0, no_such_field=1)
