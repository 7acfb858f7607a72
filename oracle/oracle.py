"""ctypes wrapper of oracle/liboracle_kv.so — TEST INFRASTRUCTURE ONLY.

The oracle is the checker for the HIP path: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module, never the product.
All arrays are numpy (C-contiguous); fp16 data is passed as its uint16 bits.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_kv.so")
F32, F16, FP8 = 0, 1, 2

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run make -C oracle")
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_to_f32.restype = ctypes.c_float
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        lib.oracle_fp8_decode.argtypes = [ctypes.c_uint8]
        lib.oracle_fp8_decode.restype = ctypes.c_float
        lib.oracle_fp8_encode.argtypes = [ctypes.c_float]
        lib.oracle_fp8_encode.restype = ctypes.c_uint8
        lib.oracle_fp8_scale.argtypes = [ctypes.c_float]
        lib.oracle_fp8_scale.restype = ctypes.c_float
        P = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        lib.oracle_reshape_and_cache.argtypes = [P, P, i64, i64, P, P, P, P, P, i32, i32, i32, i32, i32, i32, i32]
        lib.oracle_reshape_and_cache.restype = None
        lib.oracle_fp8_quantise_rows.argtypes = [P, i64, i32, i32, P, P, i32]
        lib.oracle_fp8_quantise_rows.restype = None
        lib.oracle_paged_decode.argtypes = [P, P, P, P, P, P, P, P, i32, i32, i32, i32, i32, i32, i32, f32, i32, i32]
        lib.oracle_paged_decode.restype = None
        lib.oracle_paged_prefill.argtypes = [P, P, P, P, P, P, P, P, P, i32, i32, i32, i32, i32, i32, f32, i32, i32]
        lib.oracle_paged_prefill.restype = None
        lib.oracle_rope.argtypes = [P, P, i64, i64, P, P, i32, i32, i32, i32, i32, i32, i32]
        lib.oracle_rope.restype = None
        lib.oracle_copy_blocks.argtypes = [P, i32, i32, i32, P, i32]
        lib.oracle_copy_blocks.restype = None
        lib.oracle_swap_blocks.argtypes = [P, i32, i32, i32, P, i32, P, i32, i32]
        lib.oracle_swap_blocks.restype = None
        _lib = lib
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return F32
    if a.dtype in (np.float16, np.uint16):
        return F16
    if a.dtype == np.uint8:
        return FP8
    raise TypeError(a.dtype)


def f16_to_f32(bits: int) -> float:
    return load().oracle_f16_to_f32(bits)


def f32_to_f16(x: float) -> int:
    return load().oracle_f32_to_f16(x)


def fp8_decode(code: int) -> float:
    return load().oracle_fp8_decode(code)


def fp8_encode(x: float) -> int:
    return load().oracle_fp8_encode(x)


def fp8_scale(amax: float) -> float:
    return load().oracle_fp8_scale(amax)


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, key_scales=None, value_scales=None):
    """In place on key_cache/value_cache ([N, bs, Hkv, D]) and scales ([N, bs, Hkv])."""
    N, bs, Hkv, D = key_cache.shape
    T = key.shape[0]
    slot_mapping = np.ascontiguousarray(slot_mapping, dtype=np.int32)
    key = np.ascontiguousarray(key)
    value = np.ascontiguousarray(value)
    load().oracle_reshape_and_cache(_p(key), _p(value), 0, 0, _p(key_cache), _p(value_cache),
                                    _p(key_scales), _p(value_scales), _p(slot_mapping), T, Hkv, D, bs, N,
                                    dtype_code(key), dtype_code(key_cache))


def fp8_quantise_rows(x, nthreads=1):
    """x [..., D] fp32, or fp16 bits as uint16 -> (codes uint8 [..., D], scales fp32 [...]):
    the FP8 quantisation reshape_and_cache applies per (token, kv head) vector."""
    x = np.ascontiguousarray(x)
    D = x.shape[-1]
    rows = x.size // D
    codes = np.empty(x.shape, np.uint8)
    scales = np.empty(x.shape[:-1], np.float32)
    load().oracle_fp8_quantise_rows(_p(x), rows, D, dtype_code(x), _p(codes), _p(scales), nthreads)
    return codes, scales


def rope(query, key, cos_sin, positions=None, start_pos=0):
    """In place on query [T, H, D] and key [T, Hkv, D] (fp32 or fp16 bits as uint16);
    cos_sin fp32 [P, D/2, 2]."""
    T, H, D = query.shape
    Hkv = key.shape[1]
    cs = np.ascontiguousarray(cos_sin, dtype=np.float32)
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    load().oracle_rope(_p(query), _p(key), 0, 0, _p(cs), _p(pos), start_pos, cs.shape[0], T, H, Hkv, D,
                       dtype_code(query))


def paged_decode(query, key_cache, value_cache, block_tables, context_lens, scale, key_scales=None,
                 value_scales=None, max_context_len=None, out=None, nthreads=1):
    """query fp32 [S, H, D]; returns fp32 [S, H, D] (accumulated into `out` if given)."""
    query = np.ascontiguousarray(query, dtype=np.float32)
    S, H, D = query.shape
    N, bs, Hkv, _ = key_cache.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    if out is None:
        out = np.zeros((S, H, D), np.float32)
    mcl = bt.shape[1] * bs if max_context_len is None else max_context_len
    load().oracle_paged_decode(_p(out), _p(query), _p(key_cache), _p(value_cache), _p(key_scales),
                               _p(value_scales), _p(bt), _p(cl), S, H, Hkv, D, bs, mcl, bt.shape[1],
                               scale, dtype_code(key_cache), nthreads)
    return out


def paged_prefill(query, key_cache, value_cache, block_tables, context_lens, query_start_loc, scale,
                  key_scales=None, value_scales=None, nthreads=1):
    query = np.ascontiguousarray(query, dtype=np.float32)
    Tq, H, D = query.shape
    N, bs, Hkv, _ = key_cache.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    out = np.zeros((Tq, H, D), np.float32)
    load().oracle_paged_prefill(_p(out), _p(query), _p(key_cache), _p(value_cache), _p(key_scales),
                                _p(value_scales), _p(bt), _p(cl), _p(qsl), cl.shape[0], H, Hkv, D, bs,
                                bt.shape[1], scale, dtype_code(key_cache), nthreads)
    return out


class _Plane(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("layer_stride_bytes", ctypes.c_int64),
                ("block_bytes", ctypes.c_int64)]


def _planes(arrays):
    arr = (_Plane * len(arrays))()
    for i, a in enumerate(arrays):
        assert a.flags["C_CONTIGUOUS"]
        arr[i].base = a.ctypes.data
        arr[i].layer_stride_bytes = a.strides[0]
        arr[i].block_bytes = a.strides[1]
    return arr


def copy_blocks(layer_arrays, block_pairs):
    L, N = layer_arrays[0].shape[:2]
    pairs = np.ascontiguousarray(block_pairs, dtype=np.int32)
    load().oracle_copy_blocks(_planes(layer_arrays), len(layer_arrays), L, N, _p(pairs), pairs.shape[0])


def swap_blocks(layer_arrays, host, num_host_blocks, block_pairs, direction):
    L, N = layer_arrays[0].shape[:2]
    pairs = np.ascontiguousarray(block_pairs, dtype=np.int32)
    load().oracle_swap_blocks(_planes(layer_arrays), len(layer_arrays), L, N, _p(host), num_host_blocks,
                              _p(pairs), pairs.shape[0], direction)
