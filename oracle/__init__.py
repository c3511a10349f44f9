"""ctypes binding of the CPU oracle (oracle/libah_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker (or the host baseline that is timed).  The product path
(apeiron_amd) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libah_oracle.so")

_lib = None

c_size = ctypes.c_size_t
c_ptr = ctypes.c_void_p


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.aho_f16_to_fixed.argtypes = [ctypes.c_uint16, ctypes.POINTER(ctypes.c_int64)]
        L.aho_to_q32.argtypes = [ctypes.c_uint32, ctypes.POINTER(ctypes.c_int64)]
        L.aho_act_scale.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]
        L.aho_quant_act.argtypes = [c_ptr, c_size, c_ptr, c_ptr]
        L.aho_quant_act_f32.argtypes = [c_ptr, c_size, c_ptr, c_ptr]
        L.aho_dequant_act.argtypes = [c_ptr, c_ptr, c_size, c_ptr]
        L.aho_dequant_row.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_ptr]
        L.aho_matvec_fixed.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_size, c_ptr, c_size, c_ptr]
        L.aho_matvec_q8act.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_size, c_ptr, c_ptr, c_size, c_ptr]
        L.aho_block_dots.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_ptr, c_ptr, c_ptr]
        L.aho_row_absdot.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_size, c_ptr, c_ptr, c_ptr]
        L.aho_matvec_q8act_fast.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_size, c_ptr, c_ptr, c_ptr, ctypes.c_int]
        L.aho_matmat_q8act_fast.argtypes = [ctypes.c_uint32, c_ptr, c_size, c_size, c_size, c_size, c_ptr, c_ptr, c_ptr, ctypes.c_int]
        L.aho_set_cpu_path.argtypes = [ctypes.c_int]
        L.aho_row_bytes.argtypes = [ctypes.c_uint32, c_size, ctypes.POINTER(c_size)]
        L.aho_fixed_exp.argtypes = [ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]
        L.aho_silu_fixed.argtypes = [ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]
        L.aho_swiglu.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]
        L.aho_swiglu_quant_f32.argtypes = [c_ptr, c_ptr, c_size, c_ptr, c_ptr, c_ptr]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(c_ptr)


def f16_to_fixed(h: int) -> tuple[int, int]:
    v = ctypes.c_int64(0)
    st = lib().aho_f16_to_fixed(h, ctypes.byref(v))
    return st, v.value


def to_q32(bits: int) -> tuple[int, int]:
    v = ctypes.c_int64(0)
    st = lib().aho_to_q32(bits, ctypes.byref(v))
    return st, v.value


def act_scale(absmax: int):
    v = ctypes.c_uint64(0)
    st = lib().aho_act_scale(absmax, ctypes.byref(v))
    return None if st else v.value


def quant_act(x) -> tuple[int, np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.int64)
    n = x.shape[0]
    codes = np.zeros(max(n, 1), dtype=np.int8)
    scales = np.zeros(max(-(-n // 32), 1), dtype=np.int64)
    st = lib().aho_quant_act(_p(x), n, _p(codes), _p(scales))
    return st, codes[:n], scales[: -(-n // 32)]


def quant_act_f32(x) -> tuple[int, np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[0]
    codes = np.zeros(max(n, 1), dtype=np.int8)
    scales = np.zeros(max(-(-n // 32), 1), dtype=np.int64)
    st = lib().aho_quant_act_f32(_p(x), n, _p(codes), _p(scales))
    return st, codes[:n], scales[: -(-n // 32)]


def quant_act_f32_batch(x2d: np.ndarray) -> tuple[int, np.ndarray, np.ndarray]:
    x2d = np.ascontiguousarray(x2d, dtype=np.float32)
    n_tok, n = x2d.shape
    nb = -(-n // 32)
    codes = np.zeros((n_tok, n), dtype=np.int8)
    scales = np.zeros((n_tok, nb), dtype=np.int64)
    for c in range(n_tok):
        st, codes[c], scales[c] = quant_act_f32(x2d[c])
        if st:
            return st, codes, scales
    return 0, codes, scales


def dequant_act(codes, scales) -> tuple[int, np.ndarray]:
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.int64)
    out = np.zeros(max(codes.shape[0], 1), dtype=np.int64)
    st = lib().aho_dequant_act(_p(codes), _p(scales), codes.shape[0], _p(out))
    return st, out[: codes.shape[0]]


def dequant_row(t: int, row, n: int) -> tuple[int, np.ndarray]:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.zeros(max(n, 1), dtype=np.int64)
    st = lib().aho_dequant_row(t, _p(row), row.shape[0], n, _p(out))
    return st, out[:n]


def matvec_fixed(t: int, raw, n_out: int, n_in: int, x) -> tuple[int, np.ndarray]:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.int64)
    y = np.zeros(max(n_out, 1), dtype=np.int64)
    st = lib().aho_matvec_fixed(t, _p(raw), raw.shape[0], n_out, n_in, _p(x), x.shape[0], _p(y))
    return st, y[:n_out]


def matvec_q8act(t: int, raw, n_out: int, n_in: int, codes, scales) -> tuple[int, np.ndarray]:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.int64)
    y = np.zeros(max(n_out, 1), dtype=np.int64)
    st = lib().aho_matvec_q8act(t, _p(raw), raw.shape[0], n_out, n_in, _p(codes), _p(scales),
                                codes.shape[0], _p(y))
    return st, y[:n_out]


def matvec_q8act_fast(t: int, raw, n_out: int, n_in: int, codes, scales, threads: int = 8):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.int64)
    y = np.zeros(max(n_out, 1), dtype=np.int64)
    st = lib().aho_matvec_q8act_fast(t, _p(raw), raw.shape[0], n_out, n_in, _p(codes), _p(scales),
                                     _p(y), threads)
    return st, y[:n_out]


def matmat_q8act_fast(t: int, raw, n_out: int, n_in: int, codes2d, scales2d, threads: int = 8):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    codes2d = np.ascontiguousarray(codes2d, dtype=np.int8)
    scales2d = np.ascontiguousarray(scales2d, dtype=np.int64)
    n_tok = codes2d.shape[0]
    y = np.zeros((max(n_tok, 1), max(n_out, 1)), dtype=np.int64)
    st = lib().aho_matmat_q8act_fast(t, _p(raw), raw.shape[0], n_out, n_in, n_tok, _p(codes2d),
                                     _p(scales2d), _p(y), threads)
    return st, y[:n_tok, :n_out]


def block_dots(t: int, row, n_in: int, codes) -> tuple[int, np.ndarray, np.ndarray]:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    nd = -(-n_in // 16) if t in (10, 11, 14) else -(-n_in // 32)  # per-16 groups: Q2_K, Q3_K, Q6_K
    dots = np.zeros(max(nd, 1), dtype=np.int32)
    xs = np.zeros(max(-(-n_in // 32), 1), dtype=np.int32)
    st = lib().aho_block_dots(t, _p(row), row.shape[0], n_in, _p(codes), _p(dots), _p(xs))
    return st, dots[:nd], xs[: -(-n_in // 32)]


def row_absdot(t: int, raw, n_out: int, n_in: int, codes, scales) -> tuple[int, np.ndarray]:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.int64)
    out = np.zeros(max(n_out, 1), dtype=np.float64)
    st = lib().aho_row_absdot(t, _p(raw), raw.shape[0], n_out, n_in, _p(codes), _p(scales), _p(out))
    return st, out[:n_out]


def fixed_exp(x: int):
    v = ctypes.c_int64(0)
    st = lib().aho_fixed_exp(int(x), ctypes.byref(v))
    return st, v.value


def silu_fixed(x: int):
    v = ctypes.c_int64(0)
    st = lib().aho_silu_fixed(int(x), ctypes.byref(v))
    return st, v.value


def swiglu(gate: int, up: int):
    v = ctypes.c_int64(0)
    st = lib().aho_swiglu(int(gate), int(up), ctypes.byref(v))
    return st, v.value


def swiglu_quant_f32(gate, up):
    """to_q32 + SwiGLU + quant_act of f32 gate/up: (status, codes, scales, hidden Q32.32)."""
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    n = gate.shape[0]
    codes = np.zeros(max(n, 1), dtype=np.int8)
    scales = np.zeros(max(-(-n // 32), 1), dtype=np.int64)
    h = np.zeros(max(n, 1), dtype=np.int64)
    st = lib().aho_swiglu_quant_f32(_p(gate), _p(up), n, _p(codes), _p(scales), _p(h))
    return st, codes[:n], scales[: -(-n // 32)], h[:n]


def q32_to_real(y: np.ndarray) -> np.ndarray:
    """Q32.32 integers as real values (float64; exact for |y| < 2^53)."""
    return np.asarray(y, dtype=np.float64) / 4294967296.0


CPU_PORTABLE, CPU_AVX2, CPU_VNNI = 0, 1, 2


def set_cpu_path(path: int) -> int:
    """Forces the fast path's cores (clamped to what the host has; -1: the host's best) and
    returns the path now in use."""
    return lib().aho_set_cpu_path(path)


def cpu_path() -> int:
    return lib().aho_cpu_path()
