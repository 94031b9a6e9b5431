"""esp_dense_noalloc (scratch in the library's device array) against esp_dense (caller scratch), through the C ABI:
the same bits on two calls in a row, the second with a smaller input, and a clear error for a launch whose scratch
would not fit the array. Both calls of a pair run on torch's current stream."""
import ctypes
from pathlib import Path

import pytest
import torch

from vllm_espalier import dense as Dn
from vllm_espalier import experts as G
from vllm_espalier import workloads as WL

pytestmark = pytest.mark.gpu
LIB = Path(__file__).resolve().parent.parent / "vllm-espalier_amd" / "vllm_espalier" / "libespalier_hip.so"
P, I64, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
ESP_BF16 = 1


@pytest.fixture(scope="module")
def lib(ext):                                   # ext: the package's extension, which loads this same library
    L = ctypes.CDLL(str(LIB))
    L.esp_last_error.restype = ctypes.c_char_p
    head = [P, INT, I64, I64, I64, I64, ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(I64),
            ctypes.POINTER(I64), P, INT, I64, I64]
    L.esp_dense.restype = INT
    L.esp_dense.argtypes = head + [P, I64, P, I64, P, I64, I64, I64, I64, I64, I64, I64, P]
    L.esp_dense_noalloc.restype = INT
    L.esp_dense_noalloc.argtypes = head + [I64, I64, I64, I64, I64, I64, P]
    return L


def _ptrs(ts):
    return (P * len(ts))(*[t.data_ptr() for t in ts])


def _i64(vals):
    return (I64 * len(vals))(*vals)


def _call(lib, noalloc, mats, x, y, plan, scratch=None):
    """One launch of the matrices (one launch group) into y through esp_dense or esp_dense_noalloc."""
    sk, w, pf = plan
    M, K = x.shape
    m0 = mats[0]
    k2, cb = 2 * m0.K, G.KERNEL_CB[m0.cb]
    ncols = [m.out_features for m in mats]
    col0 = [sum(ncols[:i]) for i in range(len(mats))]
    head = (x.data_ptr(), ESP_BF16, K, M, K, len(mats), _ptrs([m.trellis for m in mats]),
            _ptrs([m.suh for m in mats]), _ptrs([m.svh for m in mats]), _i64(ncols), _i64(col0), y.data_ptr(),
            ESP_BF16, y.shape[1], y.shape[1])
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.esp_dense_noalloc(*head, k2, cb, sk, w, pf, Dn.ROT_SMEM, stream)
    else:
        z, xh, counters = scratch
        rc = lib.esp_dense(*head, xh.data_ptr(), xh.numel(), z.data_ptr(), z.numel(), counters.data_ptr(),
                           counters.numel(), k2, cb, sk, w, pf, Dn.ROT_SMEM, stream)
    return rc


def test_noalloc_equals_dense_twice_then_smaller(dev, lib):
    gen = torch.Generator().manual_seed(12)
    cases = [  # (matrices, rows, plan): the larger first, then a smaller input
        ([WL.matrix(2048, 4096, 4, "int6", gen, dev), WL.matrix(2048, 512, 4, "int6", gen, dev),
          WL.matrix(2048, 512, 4, "int6", gen, dev)], 32, (6, 16, 2)),
        ([WL.matrix(512, 2048, 4, "int5", gen, dev)], 1, (4, 8, 2)),
    ]
    for i, (mats, M, plan) in enumerate(cases):
        print(f"noalloc call {i}: M={M}, {sum(m.out_features for m in mats)} columns, plan {plan}", flush=True)
        K, N = mats[0].in_features, sum(m.out_features for m in mats)
        x = torch.randn((M, K), generator=gen).to(torch.bfloat16).to(dev)
        want = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        scratch = (torch.empty(plan[0] * M * N, dtype=torch.float32, device=dev),
                   torch.empty(len(mats) * M * K, dtype=torch.half, device=dev),
                   torch.zeros(32 * (N // 128), dtype=torch.int32, device=dev))
        assert _call(lib, False, mats, x, want, plan, scratch) == 0, lib.esp_last_error()
        assert _call(lib, True, mats, x, got, plan) == 0, lib.esp_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}"


def test_noalloc_rejects_a_launch_beyond_its_array(dev, lib):
    """32 rows, 8 splits and 16384 columns: 16 MiB of partials, more than the array holds beside its counters; the
    call fails before launching anything and names the sizes."""
    gen = torch.Generator().manual_seed(13)
    mats = [WL.matrix(2048, 16384, 2, "mcg", gen, dev)]
    x = torch.randn((32, 2048), generator=gen).to(torch.bfloat16).to(dev)
    y = torch.zeros((32, 16384), dtype=torch.bfloat16, device=dev)
    rc = _call(lib, True, mats, x, y, (8, 16, 2))
    assert rc == 1
    msg = lib.esp_last_error().decode()
    assert "scratch" in msg and "16777216" in msg, msg
    torch.cuda.synchronize()
    assert int(y.view(torch.int16).abs().sum()) == 0
