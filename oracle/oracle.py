"""CPU oracle for the vllm-espalier trellis kernel layer -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and only as the checker
(or as the timed CPU baseline). The product path (vllm-espalier_amd/) never imports it.

ctypes bindings of liboracle.so (espalier_oracle.c, the C restatement of the reference's arithmetic) plus numpy
references for the float-tolerance parts (dense / MoE forwards in fp64). Every function cites the reference
file:line it restates; paths are relative to the reference repository root.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
HAD_SCALE = np.float32(0.08838834764831845)        # dense.cu:23
KERNEL_CB = {0: 1, 1: 3, 3: 6, 4: 7}                 # experts.py:34 (grid code -> kernel codebook)
COMPILED = {(1, k2) for k2 in range(2, 17, 2)} | {(3, 2), (3, 4), (3, 6), (6, 4), (6, 6), (6, 8), (7, 6), (7, 8),
                                                   (7, 10)}   # experts_grouped.cuh:227-229, experts.py:36-37
GRID_C = {6: np.float32(3.94921875) / np.float32(15.0), 7: np.float32(3.94921875) / np.float32(31.0)}

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        u16p, i16p, i32p = (np.ctypeslib.ndpointer(t, flags="C_CONTIGUOUS") for t in (np.uint16, np.int16, np.int32))
        f32p, f64p, u32p = (np.ctypeslib.ndpointer(t, flags="C_CONTIGUOUS") for t in (np.float32, np.float64, np.uint32))
        L.eo_f32_to_f16.restype = ctypes.c_uint16
        L.eo_f32_to_f16.argtypes = [ctypes.c_float]
        L.eo_f16_to_f32.restype = ctypes.c_float
        L.eo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.eo_f32_to_bf16.restype = ctypes.c_uint16
        L.eo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.eo_f64_to_bf16.restype = ctypes.c_uint16
        L.eo_f64_to_bf16.argtypes = [ctypes.c_double]
        for f in ("eo_mcg", "eo_e2m1"):
            getattr(L, f).restype = ctypes.c_uint16
            getattr(L, f).argtypes = [ctypes.c_uint32]
        L.eo_grid_q.restype = ctypes.c_int
        L.eo_grid_q.argtypes = [ctypes.c_uint32, ctypes.c_int]
        L.eo_decode.restype = ctypes.c_uint16
        L.eo_decode.argtypes = [ctypes.c_uint32, ctypes.c_int]
        L.eo_supported.restype = ctypes.c_int
        L.eo_supported.argtypes = [ctypes.c_int, ctypes.c_int]
        L.eo_state.restype = ctypes.c_uint32
        L.eo_state.argtypes = [u32p, ctypes.c_int, ctypes.c_int]
        L.eo_position.restype = None
        L.eo_position.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
        L.eo_dequant.restype = ctypes.c_int
        L.eo_dequant.argtypes = [i16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, u16p, ctypes.c_int]
        L.eo_dequant_f32.restype = ctypes.c_int
        L.eo_dequant_f32.argtypes = [i16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, f32p, ctypes.c_int]
        L.eo_fwht128.restype = None
        L.eo_fwht128.argtypes = [f32p]
        L.eo_had.restype = None
        L.eo_had.argtypes = [u16p, ctypes.c_void_p, ctypes.c_void_p, u16p, ctypes.c_int, ctypes.c_int]
        L.eo_rotate.restype = None
        L.eo_rotate.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, u16p, u16p, ctypes.c_int, ctypes.c_int]
        L.eo_group.restype = ctypes.c_int
        L.eo_group.argtypes = [i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, i32p, i32p]
        L.eo_route.restype = None
        L.eo_route.argtypes = [u16p, u16p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, i32p, f64p, u16p, f64p]
        L.eo_dot_bf16_exact.restype = ctypes.c_double
        L.eo_dot_bf16_exact.argtypes = [u16p, u16p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        L.eo_gateup_epilogue.restype = None
        L.eo_gateup_epilogue.argtypes = [f32p, i32p, u16p, u16p, u16p, u16p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int]
        L.eo_down_combine2.restype = None
        L.eo_down_combine2.argtypes = [f32p, i32p, u16p, f32p, f32p, f32p, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int]
        _lib = L
    return _lib


# ---------------------------------------------------------------------------------------------------------------
# codebooks and trellis (experts_grouped.cuh:23-154, 321-340)
# ---------------------------------------------------------------------------------------------------------------

def codebook_table(cb: int) -> np.ndarray:
    """uint16 value bits of all 65536 states for kernel codebook cb."""
    L = lib()
    return np.array([L.eo_decode(s, cb) for s in range(65536)], dtype=np.uint16)


def grid_q_table(cb: int) -> np.ndarray:
    L = lib()
    return np.array([L.eo_grid_q(s, cb) for s in range(65536)], dtype=np.int32)


def state(words: np.ndarray, k2: int, p: int) -> int:
    return int(lib().eo_state(np.ascontiguousarray(words, dtype=np.uint32), k2, p))


def position(p: int) -> tuple[int, int]:
    k, n = ctypes.c_int(), ctypes.c_int()
    lib().eo_position(p, ctypes.byref(k), ctypes.byref(n))
    return k.value, n.value


def dequant(trellis: np.ndarray, k2: int, cb: int, threads: int = 0) -> np.ndarray:
    """W [K, N] as fp16 bit patterns (uint16): the reference dequantisation (experts_grouped.cuh:321-340)."""
    t = np.ascontiguousarray(trellis, dtype=np.int16)
    K, N = t.shape[0] * 16, t.shape[1] * 16
    out = np.empty((K, N), dtype=np.uint16)
    if lib().eo_dequant(t, K, N, k2, cb, out, threads) != 0:
        raise ValueError(f"no decode for codebook {cb} at K2 {k2}")
    return out


def dequant_f32(trellis: np.ndarray, k2: int, cb: int, threads: int = 0) -> np.ndarray:
    t = np.ascontiguousarray(trellis, dtype=np.int16)
    K, N = t.shape[0] * 16, t.shape[1] * 16
    out = np.empty((K, N), dtype=np.float32)
    if lib().eo_dequant_f32(t, K, N, k2, cb, out, threads) != 0:
        raise ValueError(f"no decode for codebook {cb} at K2 {k2}")
    return out


def f16(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """RNE float32 -> bf16 bits."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---------------------------------------------------------------------------------------------------------------
# Hadamard (experts.cu:79-90, dense.cu:92-128, 242-265)
# ---------------------------------------------------------------------------------------------------------------

def fwht128_f32(v: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().eo_fwht128(a)
    return a


def had(x_bits: np.ndarray, pre: np.ndarray | None = None, post: np.ndarray | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x.shape
    y = np.empty_like(x)
    pre_a = None if pre is None else np.ascontiguousarray(pre, dtype=np.uint16)
    post_a = None if post is None else np.ascontiguousarray(post, dtype=np.uint16)
    lib().eo_had(x, None if pre_a is None else pre_a.ctypes.data, None if post_a is None else post_a.ctypes.data,
                 y, M, K)
    return y


DT = {np.float16: 0, "bf16": 1, np.float32: 2}


def rotate(x: np.ndarray, x_dtype: str, suh_bits: np.ndarray) -> np.ndarray:
    """fp16 bits of H(x * suh) / sqrt(128) (dense.cu:92-108). x_dtype 'f16' | 'bf16' | 'f32'; x holds bit patterns
    (uint16) for the 16-bit types, float32 values for 'f32'."""
    code = {"f16": 0, "bf16": 1, "f32": 2}[x_dtype]
    xa = np.ascontiguousarray(x, dtype=np.float32 if code == 2 else np.uint16)
    M, K = xa.shape
    out = np.empty((M, K), dtype=np.uint16)
    lib().eo_rotate(xa.ctypes.data, code, K, np.ascontiguousarray(suh_bits, dtype=np.uint16), out, M, K)
    return out


def sylvester(n: int = 128) -> np.ndarray:
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def had64(x: np.ndarray) -> np.ndarray:
    """x @ blockdiag(H128) / sqrt(128) in fp64 (the float reference of gpu_dense.py:66-73)."""
    H = sylvester() / np.sqrt(128.0)
    s = x.shape
    return (x.reshape(*s[:-1], -1, 128) @ H).reshape(s)


# ---------------------------------------------------------------------------------------------------------------
# float references of the forwards (fp64)
# ---------------------------------------------------------------------------------------------------------------

def dense_ref(xh_bits: np.ndarray, W: np.ndarray, svh_bits: np.ndarray, scale: float = 1.0) -> np.ndarray:
    """y = H(xh @ W) * scale * svh in fp64, from the fp16 rotated input xh (the bits the kernels multiply) and the
    decoded W (dense.cu:120-128: finish)."""
    xh = f16(xh_bits).astype(np.float64)
    return had64(xh @ W.astype(np.float64)) * scale * f16(svh_bits).astype(np.float64)


def linear_ref(x: np.ndarray, W: np.ndarray, suh_bits: np.ndarray, svh_bits: np.ndarray) -> np.ndarray:
    """H(H(x * suh) @ W) * svh entirely in fp64 (gpu_dense.py:76-77)."""
    return had64(had64(x.astype(np.float64) * f16(suh_bits)) @ W.astype(np.float64)) * f16(svh_bits)


# ---------------------------------------------------------------------------------------------------------------
# grouping and routing (experts.cu:19-76, route.cu:35-181)
# ---------------------------------------------------------------------------------------------------------------

def group(pick: np.ndarray, R: int, slots: int, E: int, maxm: int):
    p = np.ascontiguousarray(pick, dtype=np.int32).reshape(-1)
    uids = np.zeros(max(1, min(R * slots, E)), dtype=np.int32)
    members = np.full((max(1, min(R * slots, E)), maxm), -1, dtype=np.int32)
    cnt = lib().eo_group(p, R, slots, E, maxm, uids, members)
    return cnt, uids[:cnt].copy(), members[:cnt].copy()


def route(x_bits: np.ndarray, gate_bits: np.ndarray, k: int, sgate_bits: np.ndarray | None = None,
          shared_id: int = -1):
    """Exact routing: (pick [R, k+has] int32, wts [R, k+has] fp64, logits bf16 bits [R, E], shared logit [R])."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    g = np.ascontiguousarray(gate_bits, dtype=np.uint16)
    R, H = x.shape
    E = g.shape[0]
    has = shared_id >= 0
    slots = k + has
    pick = np.zeros((R, slots), dtype=np.int32)
    wts = np.zeros((R, slots), dtype=np.float64)
    logits = np.zeros((R, E), dtype=np.uint16)
    sl = np.zeros(R, dtype=np.float64)
    sg = None if sgate_bits is None else np.ascontiguousarray(sgate_bits, dtype=np.uint16)
    lib().eo_route(x, g, None if sg is None else sg.ctypes.data, R, H, E, k, shared_id, pick, wts, logits, sl)
    return pick, wts, logits, sl


def gateup_epilogue(Z, pick, svh_g, svh_u, suh_d, P, N, SK, E, limit=float("inf"), act_mode=1):
    xd = np.zeros((P, N), dtype=np.uint16)
    lib().eo_gateup_epilogue(np.ascontiguousarray(Z, dtype=np.float32), np.ascontiguousarray(pick, dtype=np.int32),
                             np.ascontiguousarray(svh_g, dtype=np.uint16), np.ascontiguousarray(svh_u, dtype=np.uint16),
                             np.ascontiguousarray(suh_d, dtype=np.uint16), xd, P, N, SK, E, limit, act_mode)
    return xd


def down_combine2(Z, pick, svh_d, y, wts, rows, P, D, SK, E, slots, n_routed, shared=True):
    y = np.ascontiguousarray(y, dtype=np.float32).copy()
    out = np.zeros((rows, D), dtype=np.float32)
    osh = np.zeros((rows, D), dtype=np.float32) if shared else None
    lib().eo_down_combine2(np.ascontiguousarray(Z, dtype=np.float32), np.ascontiguousarray(pick, dtype=np.int32),
                           np.ascontiguousarray(svh_d, dtype=np.uint16), y, np.ascontiguousarray(wts, dtype=np.float32),
                           out, None if osh is None else osh.ctypes.data, rows, P, D, SK, E, slots, n_routed)
    return out, osh, y


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-300))


def rel_max_above_floor(got: np.ndarray, ref: np.ndarray, out_dtype=np.float16) -> float:
    """The reference's own gate (gpu_dense.py:217-223): max|got-ref|/max|ref| minus the same for ref rounded to the
    output dtype ('bf16' or a numpy float type)."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    m = np.abs(ref).max()
    if out_dtype == "bf16":
        rr = bf16_to_f32(f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    else:
        rr = ref.astype(out_dtype).astype(np.float64)
    return float(np.abs(got - ref).max() / m - np.abs(rr - ref).max() / m)


os.environ.setdefault("OMP_NUM_THREADS", str(os.cpu_count() or 1))
