"""The C-ABI library (include/espalier.h) on the CPU: it loads without a GPU, exports every declared entry point,
and its argument checks fail with an error code and a message before any HIP call (the reference's TORCH_CHECKs,
dense.cu:281-296, experts.cu:405-438, route.cu:190-193)."""
import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "espalier.h"
PKG = REPO / "vllm-espalier_amd" / "vllm_espalier"
LIB = PKG / "libespalier_hip.so"


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        subprocess.run([sys.executable, str(PKG / "csrc" / "build.py"), "--only", "lib"], check=True)
    L = ctypes.CDLL(str(LIB))
    L.esp_last_error.restype = ctypes.c_char_p
    return L


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\s*\*)\s+(esp_[a-z0-9_]+)\s*\(", text, re.M)))


def test_header_declares_the_reference_surface():
    names = declared()
    # the 13 functions of the reference's espalier_ext module (experts.cpp:44-232) plus the error / version calls
    ref = {"had", "route_group", "dense", "group_shared", "down_combine2", "grouped", "dequant", "group", "rot_in",
           "gateup_epilogue", "down_epilogue", "combine", "down_combine"}
    assert {f"esp_{n}" for n in ref} <= set(names)
    assert "esp_last_error" in names and "esp_abi_version" in names


def test_every_declared_symbol_is_exported(lib):
    for n in declared():
        assert hasattr(lib, n), n


def test_abi_version(lib):
    lib.esp_abi_version.restype = ctypes.c_int
    assert lib.esp_abi_version() == 1


def _dense(lib, **over):
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    f = lib.esp_dense
    f.restype = ctypes.c_int
    f.argtypes = [P, ctypes.c_int, I64, I64, I64, I64, ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(P),
                  ctypes.POINTER(I64), ctypes.POINTER(I64), P, ctypes.c_int, I64, I64, P, I64, P, I64, P, I64, I64,
                  I64, I64, I64, I64, I64, P]
    a = dict(M=1, K=2048, n=1, ncols=2048, col0=0, y_cols=2048, k2=8, cb=7, SK=1, W=4, z_numel=1 << 30, x=16, y=16,
             t=16, x_stride=None)
    a.update(over)
    one = (P * 1)(16)                                   # non-null, never dereferenced: the checks fail first
    tp = (P * 1)(a["t"])
    nc, c0 = (I64 * 1)(a["ncols"]), (I64 * 1)(a["col0"])
    rc = f(a["x"], 1, a["x_stride"] or a["K"], a["M"], a["K"], a["n"], tp, one, one, nc, c0, a["y"], 1, a["y_cols"],
           a["y_cols"], 16, 1 << 30, 16, a["z_numel"], 16, 1 << 20, a["k2"], a["cb"], a["SK"], a["W"], 2, 0, None)
    return rc, lib.esp_last_error().decode()


@pytest.mark.parametrize("over,needle", [
    (dict(M=0), "rows"), (dict(M=33), "rows"), (dict(n=5), "matrices"), (dict(K=2000), "K"),
    (dict(W=6), "W"), (dict(ncols=100), "shape"), (dict(col0=100), "past y"), (dict(SK=65), "SK"), (dict(SK=0), "SK"),
    # the split-K partials are addressed by 32-bit byte offsets from Z (16-byte buffer accesses): at most 4 GiB
    (dict(M=32, SK=64, ncols=4160 * 128, y_cols=4160 * 128, z_numel=1 << 40), "4 GiB"),
    # the kernels move 4 elements of a row and 16-byte trellis units at a time: misaligned operands are refused
    (dict(x=18), "aligned"), (dict(y=20), "aligned"), (dict(x_stride=2050), "aligned"), (dict(t=24), "aligned"),
    (dict(col0=2, y_cols=4096), "multiple of 4"),
])
def test_dense_argument_errors(lib, over, needle):
    rc, msg = _dense(lib, **over)
    assert rc == 1, msg                                  # ESP_ERR_ARG
    assert needle in msg


def test_dense_unsupported_codebook(lib):
    rc, msg = _dense(lib, cb=3, k2=8)                    # E2M1 has no 4-bit kernel (experts_grouped.cuh:227-229)
    assert rc == 2 and "cb=3" in msg                     # ESP_ERR_UNSUPPORTED


def test_dequant_errors(lib):
    f = lib.esp_dequant
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                  ctypes.c_void_p]
    assert f(16, 16, 40, 32, 8, 7, None) == 1            # K not a multiple of 16
    assert "multiples of 16" in lib.esp_last_error().decode()
    assert f(16, 16, 32, 32, 9, 7, None) == 2            # odd K2: no instance
    assert f(None, 16, 32, 32, 8, 7, None) == 1


def _dense_rmsnorm(lib, **over):
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    f = lib.esp_dense_rmsnorm
    f.restype = ctypes.c_int
    f.argtypes = [P, P, P, P, ctypes.c_double, P, ctypes.c_int, I64, I64, I64, I64, ctypes.POINTER(P),
                  ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(I64), ctypes.POINTER(I64), P, ctypes.c_int, I64,
                  I64, P, I64, P, I64, I64, I64, I64, I64, I64, P]
    a = dict(M=1, K=2048, W=16, SK=8, h=16, w=16, h_out=16, d1=None, x_dtype=1, rot_smem=64 * 1024)
    a.update(over)
    one = (P * 1)(16)
    nc, c0 = (I64 * 1)(2048), (I64 * 1)(0)
    rc = f(a["h"], a["d1"], None, a["w"], 1e-6, a["h_out"], a["x_dtype"], a["K"], a["M"], a["K"], 1, one, one, one, nc,
           c0, 16, 1, 2048, 2048, 16, 1 << 30, 16, 1 << 20, 8, 7, a["SK"], a["W"], a["rot_smem"], None)
    return rc, lib.esp_last_error().decode()


@pytest.mark.parametrize("over,needle", [
    (dict(M=5), "rows"), (dict(W=8, M=3), "rows"), (dict(h_out=None), "null"), (dict(x_dtype=2), "bf16"),
    (dict(d1=8), "aligned"), (dict(rot_smem=0), "shared memory"),
])
def test_dense_rmsnorm_argument_errors(lib, over, needle):
    """The fused-norm dense entry point refuses, before any HIP call, what its in-launch norm cannot do: more rows than
    four waves each, unaligned rows, fp32 rows, rows that do not fit the fused rotation."""
    rc, msg = _dense_rmsnorm(lib, **over)
    assert rc == 1, msg
    assert needle in msg


def test_route_group_rmsnorm_argument_errors(lib):
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    f = lib.esp_route_group_rmsnorm
    f.restype = ctypes.c_int
    f.argtypes = [P, P, P, ctypes.c_double, P, P, ctypes.c_int, I64, I64, I64, P, I64, P, I64, I64, ctypes.c_void_p,
                  I64, P, P, P, P, I64, P, P, I64, P]
    args = lambda R, h_out: (16, None, 16, 1e-6, h_out, 16, 1, 2048, R, 2048, 16, 256, 16, 8, 256, 16, 1 << 20, 16,  # noqa
                             16, 16, 16, 257, 16, 16, 32, None)
    assert f(*args(5, 16)) == 1 and "4 rows" in lib.esp_last_error().decode()
    assert f(*args(1, None)) == 1 and "null" in lib.esp_last_error().decode()
