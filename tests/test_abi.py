"""The C ABI without a GPU: libeii.so loads, exports every entry point include/eii.h declares
(with the ctypes signatures eii/lib.py binds), and rejects bad arguments and malformed model
files with the documented status codes before touching a device."""
import ctypes as C
import os
import re
import shutil

import numpy as np
import pytest

from eii import lib as L
from eii import modelbin

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "eii.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eii_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    names = declared()
    assert len(names) >= 20
    assert set(names) == set(L.SIGNATURES), set(names) ^ set(L.SIGNATURES)


def test_library_exports_every_entry_point():
    lib = L.load()
    for n in declared():
        assert hasattr(lib, n), n


def test_argument_errors_need_no_device():
    lib = L.load()
    assert lib.eii_gemm_i8(None, 16, None, 4, 4, 64, None, None) == L.EII_E_ARG
    a = (C.c_int16 * 64)()
    w = (C.c_int8 * 256)()
    assert lib.eii_gemm_i8(a, 12, w, 1, 4, 64, a, None) == L.EII_E_ARG         # a_bits
    assert lib.eii_gemm_i8(a, 8, w, 1, 4, 64, None, None) == L.EII_E_ARG        # no output
    assert lib.eii_gemm_i8(a, 16, w, 1, 4, 200000, a, None) == L.EII_E_BOUND    # K past 131072
    assert b"131072" in lib.eii_last_error()
    assert lib.eii_linear(a, 16, w, None, None, None, 1, 4, 64, 16, None, None) == L.EII_E_ARG
    assert lib.eii_rmsnorm(None, 1, None, 14, 11, 16, None, None) == L.EII_E_ARG
    assert lib.eii_attention(None, None, 1, 4, None, 10, 10, 11, 11, 16, None, None) == L.EII_E_ARG
    assert lib.eii_rope(None, None, 1, None, None, 512, 10, 11, 16, 10, 11, 16, None) == L.EII_E_ARG
    g = (C.c_int16 * 1536)()
    t = (C.c_int32 * 65536)()
    assert lib.eii_rope(g, t, 1, t, t, 512, 10, 11, 32, 10, 11, 16, None) == L.EII_E_ARG      # int16 out
    assert lib.eii_rope(g, t, 1, t, t, 512, 10, 60, 16, 10, 11, 16, None) == L.EII_E_BOUND    # shift -20
    assert lib.eii_silu_gate(None, None, 1, None, 12, 12, 13, 16, None, None) == L.EII_E_ARG
    assert lib.eii_silu_gate(g, g, 1, t, 12, 12, 13, 8, g, None) == L.EII_E_ARG                # bits_m
    assert lib.eii_silu_gate(g, g, 1, t, 12, 12, 60, 16, g, None) == L.EII_E_BOUND             # shift -36
    h = C.c_void_p()
    assert lib.eii_model_load(None, 0, C.byref(h)) == L.EII_E_ARG
    assert lib.eii_forward(None, None, 1, 1, None, None, None, None, None) == L.EII_E_ARG
    assert lib.eii_model_rope_rows(None) == 0


def test_model_file_errors(tmp_path, model_path):
    lib = L.load()
    h = C.c_void_p()
    missing = str(tmp_path / "none.bin").encode()
    assert lib.eii_model_load(missing, 0, C.byref(h)) == L.EII_E_IO
    short = tmp_path / "short.bin"
    short.write_bytes(b"\0" * 1000)
    assert lib.eii_model_load(str(short).encode(), 0, C.byref(h)) == L.EII_E_IO
    assert b"bytes" in lib.eii_last_error()
    # a requantization shift n + f_in - f_out below 1 (python/intref.py:49 asserts >= 1)
    bad = tmp_path / "bad.bin"
    shutil.copyfile(model_path, bad)
    off = modelbin.matrix_offset(0, "q") + 576 * 576 + 8 * 576    # n[0] of layer 0's q_proj
    with open(bad, "r+b") as f:
        f.seek(off)
        f.write(np.array([-40], dtype="<i8").tobytes())
    assert lib.eii_model_load(str(bad).encode(), 0, C.byref(h)) == L.EII_E_BOUND
    assert not h.value


def test_model_gain_outside_int16(tmp_path, model_path):
    """RMSNorm gains are int16 (quant_vec_int16, python/intref.py:126-130): a wider one is a bound
    violation at load, before any device work."""
    lib = L.load()
    h = C.c_void_p()
    for layer, which in ((0, 0), (17, 1)):
        bad = tmp_path / f"gain{layer}.bin"
        shutil.copyfile(model_path, bad)
        off = modelbin.HEADER_BYTES + layer * modelbin.LAYER_BYTES + 24 * 8 + which * (576 * 8 + 8) + 8 * 5
        with open(bad, "r+b") as f:
            f.seek(off)
            f.write(np.array([1 << 20], dtype="<i8").tobytes())
        assert lib.eii_model_load(str(bad).encode(), 0, C.byref(h)) == L.EII_E_BOUND
        assert b"ln%d" % (which + 1) in lib.eii_last_error()
        assert not h.value
    bad = tmp_path / "final.bin"
    shutil.copyfile(model_path, bad)
    off = 49152 * 576 + 2 * 49152 * 8 + 8 * 100        # final gain entry 100
    with open(bad, "r+b") as f:
        f.seek(off)
        f.write(np.array([-32769], dtype="<i8").tobytes())
    assert lib.eii_model_load(str(bad).encode(), 0, C.byref(h)) == L.EII_E_BOUND
    assert b"final gain" in lib.eii_last_error()
