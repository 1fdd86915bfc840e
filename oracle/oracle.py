"""ctypes front-end of the CPU oracle (lp_oracle.c) and of the reference's
own layout oracle built into ``oracle/_ref`` (ref_glue.cpp).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module. The product package ``laplace_amd`` never does.

Every function here forwards to C; the arithmetic and its reference
citations live in ``lp_oracle.c``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

F32, F16, Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 6, 8, 10, 11, 12, 13, 14, 30
INT_TYPES = (Q8_0, Q4_0, Q5_0, Q4_K, Q6_K)
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q2_K: "Q2_K",
              Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", BF16: "BF16"}

_lib = None
_ref = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i16p = np.ctypeslib.ndpointer(np.int16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> None:
    """Compile liboracle.so (and _ref/libref.so where the reference exists)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.check_call(["make", "-s", "-C", HERE, "all"])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.or_bytes_per_block.restype = C.c_size_t
        L.or_bytes_per_block.argtypes = [C.c_int]
        L.or_elements_per_block.restype = C.c_int
        L.or_elements_per_block.argtypes = [C.c_int]
        L.or_row_bytes.restype = C.c_size_t
        L.or_row_bytes.argtypes = [C.c_int, C.c_int]
        L.or_fp16_to_fp32.restype = C.c_float
        L.or_fp16_to_fp32.argtypes = [C.c_uint16]
        L.or_fp32_to_fp16.restype = C.c_uint16
        L.or_fp32_to_fp16.argtypes = [C.c_float]
        L.or_bf16_to_fp32.restype = C.c_float
        L.or_bf16_to_fp32.argtypes = [C.c_uint16]
        L.or_fp32_to_bf16.restype = C.c_uint16
        L.or_fp32_to_bf16.argtypes = [C.c_float]
        L.or_get_scale_min_k4.argtypes = [C.c_int, _u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.or_quantize_act.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _f32p, _i16p, _i16p, _i8p]
        L.or_n_subsums.restype = C.c_int
        L.or_n_subsums.argtypes = [C.c_int, C.c_int]
        L.or_block_sums_row.restype = C.c_int
        L.or_block_sums_row.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
        L.or_dot_int_row.restype = C.c_float
        L.or_dot_int_row.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.or_gemm_int.restype = C.c_int
        L.or_gemm_int.argtypes = [C.c_int, _f32p, _u8p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.or_moe_gemv_int.restype = C.c_int
        L.or_moe_gemv_int.argtypes = [C.c_int, _f32p, _u8p, _i32p, C.c_int, _f32p,
                                      C.c_int, C.c_int, C.c_int, C.c_int]
        L.or_dot_scalar_row.restype = C.c_float
        L.or_dot_scalar_row.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        L.or_gemm_scalar.restype = C.c_int
        L.or_gemm_scalar.argtypes = [C.c_int, _f32p, _u8p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.or_dequantize.restype = C.c_int
        L.or_dequantize.argtypes = [C.c_int, _u8p, _f32p, C.c_int]
        L.or_ref_test_weights.restype = C.c_int
        L.or_ref_test_weights.argtypes = [C.c_int, C.c_int, C.c_int, _u8p]
        L.or_moe_ffn.restype = C.c_int
        L.or_moe_ffn.argtypes = [_f32p, C.c_int, C.c_int, _u8p, C.c_int, _f32p, _f32p, C.c_float,
                                 _u8p, C.c_int, _u8p, C.c_int, _f32p, C.c_int, C.c_int, C.c_int,
                                 _f32p, _i32p, _f32p]
        L.or_ref_test_x.argtypes = [C.c_int, C.c_int, _f32p]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own header-only layout oracle (oracle/_ref/libref.so)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(REF_PATH)
        R = C.CDLL(REF_PATH)
        R.ref_fp16_to_fp32.restype = C.c_float
        R.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        R.ref_fp32_to_fp16.restype = C.c_uint16
        R.ref_fp32_to_fp16.argtypes = [C.c_float]
        R.ref_bf16_to_fp32.restype = C.c_float
        R.ref_bf16_to_fp32.argtypes = [C.c_uint16]
        R.ref_fp32_to_bf16.restype = C.c_uint16
        R.ref_fp32_to_bf16.argtypes = [C.c_float]
        R.ref_get_scale_min_k4.argtypes = [C.c_int, _u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        R.ref_dequant.restype = C.c_int
        R.ref_dequant.argtypes = [C.c_int, _u8p, C.c_long, _f32p]
        R.ref_xorshift_u32.argtypes = [C.c_uint32, C.c_long, _u32p]
        R.ref_xorshift_float.argtypes = [C.c_uint32, C.c_long, _f32p]
        vp, cp = C.c_void_p, C.c_char_p
        R.ref_gguf_new.restype = vp
        R.ref_gguf_free.argtypes = [vp]
        R.ref_gguf_kv_u32.argtypes = [vp, cp, C.c_uint32]
        R.ref_gguf_kv_i32.argtypes = [vp, cp, C.c_int32]
        R.ref_gguf_kv_f32.argtypes = [vp, cp, C.c_float]
        R.ref_gguf_kv_bool.argtypes = [vp, cp, C.c_int]
        R.ref_gguf_kv_str.argtypes = [vp, cp, cp]
        R.ref_gguf_kv_arr_str.argtypes = [vp, cp, C.POINTER(cp), C.c_long]
        R.ref_gguf_kv_arr_u8.argtypes = [vp, cp, _u8p, C.c_long]
        R.ref_gguf_kv_arr_i16.argtypes = [vp, cp, _i16p, C.c_long]
        R.ref_gguf_kv_arr_bool.argtypes = [vp, cp, _u8p, C.c_long]
        R.ref_gguf_kv_arr_i32.argtypes = [vp, cp, _i32p, C.c_long]
        R.ref_gguf_add_tensor.argtypes = [vp, cp, C.POINTER(C.c_uint64), C.c_int, C.c_uint32, _u8p, C.c_long]
        R.ref_gguf_write.restype = C.c_int
        R.ref_gguf_write.argtypes = [vp, cp, C.c_long]
        _ref = R
    return _ref


class RefGGUFWriter:
    """The reference's GGUF test-file writer (tests/gguf_writer.h, compiled
    into oracle/_ref): metadata and tensors are handed to it one by one, and
    it writes the file exactly as the reference's tests do (GGUF v3, tensor
    data 32-byte aligned)."""

    def __init__(self):
        self.R = ref()
        self.h = self.R.ref_gguf_new()

    def __del__(self):
        if getattr(self, "h", None):
            self.R.ref_gguf_free(self.h)
            self.h = None

    def kv(self, kind: str, key: str, value):
        k = key.encode()
        R, h = self.R, self.h
        if kind == "u32":
            R.ref_gguf_kv_u32(h, k, value)
        elif kind == "i32":
            R.ref_gguf_kv_i32(h, k, value)
        elif kind == "f32":
            R.ref_gguf_kv_f32(h, k, value)
        elif kind == "bool":
            R.ref_gguf_kv_bool(h, k, 1 if value else 0)
        elif kind == "str":
            R.ref_gguf_kv_str(h, k, value.encode())
        elif kind == "arr_str":
            arr = (C.c_char_p * len(value))(*[v.encode() for v in value])
            R.ref_gguf_kv_arr_str(h, k, arr, len(value))
        elif kind == "arr_u8":
            a = np.ascontiguousarray(value, np.uint8)
            R.ref_gguf_kv_arr_u8(h, k, a, a.size)
        elif kind == "arr_i16":
            a = np.ascontiguousarray(value, np.int16)
            R.ref_gguf_kv_arr_i16(h, k, a, a.size)
        elif kind == "arr_bool":
            a = np.ascontiguousarray(value, np.uint8)
            R.ref_gguf_kv_arr_bool(h, k, a, a.size)
        elif kind == "arr_i32":
            a = np.ascontiguousarray(value, np.int32)
            R.ref_gguf_kv_arr_i32(h, k, a, a.size)
        else:
            raise ValueError(kind)

    def tensor(self, name: str, dims, type_: int, data: np.ndarray):
        d = (C.c_uint64 * len(dims))(*dims)
        a = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        self.R.ref_gguf_add_tensor(self.h, name.encode(), d, len(dims), type_, a, a.size)

    def write(self, path: str, truncate: int = 0):
        if self.R.ref_gguf_write(self.h, path.encode(), truncate):
            raise OSError(f"reference writer failed on {path}")


# --------------------------------------------------------------------------
# numpy conveniences

def row_bytes(t: int, K: int) -> int:
    return int(lib().or_row_bytes(t, K))


def block_elems(t: int) -> int:
    return int(lib().or_elements_per_block(t))


def quantize_act(x: np.ndarray):
    """ActQ8 blocks of x[M, K] as (d, sum, sum_lo, sum_hi, qs)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    nb = K // 32
    d = np.zeros((M, nb), np.float32)
    s = np.zeros((M, nb), np.float32)
    lo = np.zeros((M, nb), np.int16)
    hi = np.zeros((M, nb), np.int16)
    qs = np.zeros((M, K), np.int8)
    lib().or_quantize_act(x, M, K, d, s, lo, hi, qs)
    return d, s, lo, hi, qs


def block_sums(t: int, w: np.ndarray, qs: np.ndarray, K: int, N: int) -> np.ndarray:
    """Per-sub-block int32 dots, shape [M, N, n_subsums]."""
    qs = np.ascontiguousarray(qs, dtype=np.int8).reshape(-1, K)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    M = qs.shape[0]
    ns = lib().or_n_subsums(t, K)
    rb = row_bytes(t, K)
    out = np.zeros((M, N, ns), np.int32)
    wp = w.ctypes.data
    for m in range(M):
        for j in range(N):
            rc = lib().or_block_sums_row(t, wp + j * rb, qs[m].ctypes.data, K, out[m, j].ctypes.data)
            if rc != 0:
                raise ValueError(f"unsupported type {t}")
    return out


def gemm_int(t: int, x: np.ndarray, w: np.ndarray, N: int, nthreads: int = 8) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    y = np.zeros((M, N), np.float32)
    if lib().or_gemm_int(t, x, np.ascontiguousarray(w, dtype=np.uint8), y, M, K, N, nthreads):
        raise ValueError(f"unsupported type {t}")
    return y


def gemm_scalar(t: int, x: np.ndarray, w: np.ndarray, N: int, nthreads: int = 8) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    M, K = x.shape
    y = np.zeros((M, N), np.float32)
    if lib().or_gemm_scalar(t, x, np.ascontiguousarray(w, dtype=np.uint8), y, M, K, N, nthreads):
        raise ValueError(f"unsupported type {t}")
    return y


def moe_gemv_int(t: int, x: np.ndarray, w: np.ndarray, expert_idx, K: int, N: int,
                 multi: bool, nthreads: int = 8) -> np.ndarray:
    idx = np.ascontiguousarray(expert_idx, dtype=np.int32)
    n = idx.shape[0]
    y = np.zeros((n, N), np.float32)
    rc = lib().or_moe_gemv_int(t, np.ascontiguousarray(x, dtype=np.float32).reshape(-1),
                               np.ascontiguousarray(w, dtype=np.uint8), idx, n, y, K, N,
                               1 if multi else 0, nthreads)
    if rc:
        raise ValueError(f"unsupported type {t}")
    return y


def moe_ffn(x, router_w, router_type, router_scale, pre_norm, eps, gu_w, gu_type, dn_w, dn_type,
            down_scale, n_exp, top_k, inter):
    """Gemma4 MoE feed-forward of x [T, H]; returns (out [T, H], idx, w [T, top_k])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    out = np.zeros((T, H), np.float32)
    idx = np.zeros((T, top_k), np.int32)
    wts = np.zeros((T, top_k), np.float32)
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32)
    u = lambda a: np.ascontiguousarray(a, dtype=np.uint8)
    rc = lib().or_moe_ffn(x, T, H, u(router_w), router_type, f(router_scale), f(pre_norm), eps,
                          u(gu_w), gu_type, u(dn_w), dn_type, f(down_scale), n_exp, top_k, inter,
                          out, idx, wts)
    if rc:
        raise ValueError("unsupported type or top_k")
    return out, idx, wts


def dequantize(t: int, w: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    if lib().or_dequantize(t, np.ascontiguousarray(w, dtype=np.uint8), out, n):
        raise ValueError(f"unsupported type {t}")
    return out


def ref_test_weights(t: int, K: int, N: int) -> np.ndarray:
    out = np.zeros(row_bytes(t, K) * N, np.uint8)
    if lib().or_ref_test_weights(t, K, N, out):
        raise ValueError(f"no reference test generator for type {t}")
    return out


def ref_test_x(t: int, K: int) -> np.ndarray:
    out = np.zeros(K, np.float32)
    lib().or_ref_test_x(t, K, out)
    return out
