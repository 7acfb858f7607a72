"""ctypes binding of libvllm_kv_amd.so (the C ABI in include/vllm_kv_amd.h).

Torch tensors are used only as device memory and streams: every call passes raw
pointers and sizes to the C ABI, which launches the HIP kernels.  There is no
fallback: if the library is missing or no GPU is present the calls raise.

Entry points and the reference interfaces they replace:
  reshape_and_cache  -> per-token cudaMemcpyAsync pair, src/layers/attention.cpp:84-102
  rope_reshape_and_cache -> rope_forward (src/kernels/rotary_embedding.cu:37-45) + that append
  paged_decode       -> vllm::paged_attention_forward, src/attention/paged_attention.cu:85-93
  paged_prefill      -> token-by-token prefill through decode, src/core/engine.cpp:157-164
  copy_blocks / swap_blocks -> no reference counterpart (fork / offload)
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(os.path.dirname(_HERE))          # vllm-cpp_amd/
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libvllm_kv_amd.so")

ABI_VERSION = 4  # vkv_abi_version() of the library this binding's structs match
DTYPE_F32, DTYPE_F16, DTYPE_FP8 = 0, 1, 2
SWAP_OUT, SWAP_IN = 0, 1

ERRORS = {
    -1: "VKV_ERR_NULL", -2: "VKV_ERR_SHAPE", -3: "VKV_ERR_UNSUPPORTED",
    -4: "VKV_ERR_WORKSPACE", -5: "VKV_ERR_ALIGN", -6: "VKV_ERR_DEVICE",
}

# Every symbol the C header declares; tests check the library exports them all.
EXPORTED = [
    "vkv_last_error", "vkv_abi_version", "vkv_reshape_and_cache", "vkv_slot_mapping_host",
    "vkv_paged_decode_workspace_size", "vkv_paged_decode", "vkv_paged_decode_noalloc", "vkv_paged_decode_append",
    "vkv_paged_prefill_workspace_size",
    "vkv_paged_prefill",
    "vkv_copy_blocks", "vkv_check_block_pairs_host", "vkv_swap_host_block_bytes",
    "vkv_swap_blocks", "vkv_rope_reshape_and_cache", "vkv_rope_cos_sin_host",
    "vkv_kv_block_bytes", "vkv_kv_pool_num_blocks", "vkv_release_workspace", "vkv_prefill_work_list_host",
]


class VkvError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERRORS.get(code, 'hipError %d' % code)}: {message}")
        self.code = code


class AppendParams(ctypes.Structure):
    _fields_ = [
        ("key", ctypes.c_void_p), ("value", ctypes.c_void_p),
        ("key_stride", ctypes.c_int64), ("value_stride", ctypes.c_int64),
        ("key_cache", ctypes.c_void_p), ("value_cache", ctypes.c_void_p),
        ("key_scales", ctypes.c_void_p), ("value_scales", ctypes.c_void_p),
        ("slot_mapping", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32), ("src_dtype", ctypes.c_int32),
        ("cache_dtype", ctypes.c_int32),
    ]


class RopeAppendParams(ctypes.Structure):
    _fields_ = [
        ("query", ctypes.c_void_p), ("key", ctypes.c_void_p), ("value", ctypes.c_void_p),
        ("query_stride", ctypes.c_int64), ("key_stride", ctypes.c_int64), ("value_stride", ctypes.c_int64),
        ("cos_sin", ctypes.c_void_p), ("positions", ctypes.c_void_p),
        ("start_pos", ctypes.c_int32), ("max_position", ctypes.c_int32),
        ("key_cache", ctypes.c_void_p), ("value_cache", ctypes.c_void_p),
        ("key_scales", ctypes.c_void_p), ("value_scales", ctypes.c_void_p),
        ("slot_mapping", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int32), ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32), ("num_blocks", ctypes.c_int32),
        ("src_dtype", ctypes.c_int32), ("cache_dtype", ctypes.c_int32),
    ]


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("output", ctypes.c_void_p), ("query", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p), ("value_cache", ctypes.c_void_p),
        ("key_scales", ctypes.c_void_p), ("value_scales", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p), ("context_lens", ctypes.c_void_p),
        ("query_stride", ctypes.c_int64),
        ("num_seqs", ctypes.c_int32), ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32), ("max_context_len", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32), ("num_blocks", ctypes.c_int32),
        ("scale", ctypes.c_float), ("io_dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32), ("accumulate", ctypes.c_int32),
        ("partition_size", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class PrefillParams(ctypes.Structure):
    _fields_ = [
        ("output", ctypes.c_void_p), ("query", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p), ("value_cache", ctypes.c_void_p),
        ("key_scales", ctypes.c_void_p), ("value_scales", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p), ("context_lens", ctypes.c_void_p),
        ("query_start_loc", ctypes.c_void_p),
        ("query_stride", ctypes.c_int64),
        ("num_seqs", ctypes.c_int32), ("num_query_tokens", ctypes.c_int32),
        ("max_query_len", ctypes.c_int32), ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32), ("max_blocks_per_seq", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32), ("scale", ctypes.c_float),
        ("io_dtype", ctypes.c_int32), ("kv_dtype", ctypes.c_int32),
        ("max_context_len", ctypes.c_int32), ("multi_token_only", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("work_list", ctypes.c_void_p), ("work_list_words", ctypes.c_int32),
    ]


class BlockPlane(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("layer_stride_bytes", ctypes.c_int64),
                ("block_bytes", ctypes.c_int64)]


_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with __graft_entry__.build() "
                           "(make -C vllm-cpp_amd)")
    # torch ships its own libamdhip64.so.7.  Loading torch first makes the
    # library bind to that runtime (same soname); loading it first would map a
    # second HIP runtime into the process, which then sees no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    lib.vkv_last_error.restype = ctypes.c_char_p
    lib.vkv_abi_version.restype = ctypes.c_int
    if lib.vkv_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {lib.vkv_abi_version()}, this binding's structs are "
                           f"version {ABI_VERSION}: rebuild it (make -C vllm-cpp_amd)")
    for name, ptype in (("vkv_reshape_and_cache", AppendParams), ("vkv_paged_decode", DecodeParams),
                        ("vkv_paged_decode_noalloc", DecodeParams),
                        ("vkv_paged_prefill", PrefillParams),
                        ("vkv_rope_reshape_and_cache", RopeAppendParams)):
        f = getattr(lib, name)
        f.argtypes = [ctypes.POINTER(ptype), ctypes.c_void_p]
        f.restype = ctypes.c_int
    lib.vkv_paged_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeParams)]
    lib.vkv_paged_decode_workspace_size.restype = ctypes.c_size_t
    lib.vkv_paged_prefill_workspace_size.argtypes = [ctypes.POINTER(PrefillParams)]
    lib.vkv_paged_prefill_workspace_size.restype = ctypes.c_size_t
    lib.vkv_slot_mapping_host.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.vkv_slot_mapping_host.restype = ctypes.c_int
    lib.vkv_rope_cos_sin_host.argtypes = [ctypes.c_float, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.vkv_rope_cos_sin_host.restype = ctypes.c_int
    i32 = ctypes.c_int32
    lib.vkv_kv_block_bytes.argtypes = [i32, i32, i32, i32, i32]
    lib.vkv_kv_block_bytes.restype = ctypes.c_int64
    lib.vkv_kv_pool_num_blocks.argtypes = [ctypes.c_uint64, ctypes.c_uint64, i32, i32, i32, i32, i32, i32, i32]
    lib.vkv_kv_pool_num_blocks.restype = ctypes.c_int64
    lib.vkv_copy_blocks.argtypes = [ctypes.POINTER(BlockPlane), ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
    lib.vkv_copy_blocks.restype = ctypes.c_int
    lib.vkv_check_block_pairs_host.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32]
    lib.vkv_check_block_pairs_host.restype = ctypes.c_int
    lib.vkv_swap_host_block_bytes.argtypes = [ctypes.POINTER(BlockPlane), ctypes.c_int32, ctypes.c_int32]
    lib.vkv_swap_host_block_bytes.restype = ctypes.c_size_t
    lib.vkv_swap_blocks.argtypes = [ctypes.POINTER(BlockPlane), ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p,
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.vkv_swap_blocks.restype = ctypes.c_int
    lib.vkv_paged_decode_append.argtypes = [ctypes.POINTER(AppendParams), ctypes.POINTER(DecodeParams), ctypes.c_void_p]
    lib.vkv_paged_decode_append.restype = ctypes.c_int
    lib.vkv_release_workspace.argtypes = [ctypes.c_void_p]
    lib.vkv_release_workspace.restype = ctypes.c_int
    lib.vkv_prefill_work_list_host.argtypes = [ctypes.POINTER(PrefillParams), ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p, ctypes.c_int64]
    lib.vkv_prefill_work_list_host.restype = ctypes.c_int64
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        raise VkvError(rc, load().vkv_last_error().decode())


# ---------------------------------------------------------------- torch helpers

def _torch():
    import torch
    return torch


def _dtype_code(t) -> int:
    torch = _torch()
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.uint8 or t.dtype == getattr(torch, "float8_e4m3fn", None):
        return DTYPE_FP8
    raise TypeError(f"unsupported dtype {t.dtype}")


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


STREAM_PER_THREAD = 2  # the value of the hipStreamPerThread handle


def _stream(stream) -> Optional[int]:
    """A torch stream (None: the current one) or a raw stream handle (int)."""
    if isinstance(stream, int):
        return stream
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def release_workspace(stream=None) -> None:
    """vkv_release_workspace: free the library's workspace buffers of `stream`
    on the current device (after synchronising it)."""
    check(load().vkv_release_workspace(_stream(stream)))


def _require_cuda(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("all tensors must be on the GPU")


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping,
                      key_scales=None, value_scales=None, stream=None) -> None:
    """key/value [T, Hkv, D] (token stride from the tensor); caches [N, bs, Hkv, D];
    slot_mapping int32 [T]; FP8 caches (uint8) need key_scales/value_scales [N, bs, Hkv]."""
    _require_cuda(key, value, key_cache, value_cache, slot_mapping, key_scales, value_scales)
    p = append_params(key, value, key_cache, value_cache, slot_mapping, key_scales, value_scales)
    check(load().vkv_reshape_and_cache(ctypes.byref(p), _stream(stream)))


def append_params(key, value, key_cache, value_cache, slot_mapping, key_scales=None,
                  value_scales=None) -> AppendParams:
    T = key.shape[0]
    N, bs, Hkv, D = key_cache.shape
    return AppendParams(
        key=_ptr(key), value=_ptr(value), key_stride=key.stride(0), value_stride=value.stride(0),
        key_cache=_ptr(key_cache), value_cache=_ptr(value_cache),
        key_scales=_ptr(key_scales), value_scales=_ptr(value_scales),
        slot_mapping=_ptr(slot_mapping), num_tokens=T, num_kv_heads=Hkv, head_dim=D,
        block_size=bs, num_blocks=N, src_dtype=_dtype_code(key), cache_dtype=_dtype_code(key_cache))


def kv_pool_num_blocks(budget_bytes: int, non_kv_bytes: int, num_layers: int, block_size: int,
                       num_kv_heads: int, head_dim: int, kv_dtype: int, max_num_seqs: int,
                       max_model_len: int) -> int:
    """KV blocks that fit the budget (the reference's pool sizing with the element type)."""
    n = load().vkv_kv_pool_num_blocks(budget_bytes, non_kv_bytes, num_layers, block_size, num_kv_heads,
                                      head_dim, kv_dtype, max_num_seqs, max_model_len)
    if n < 0:
        check(int(n))
    return int(n)


def kv_block_bytes(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int, kv_dtype: int) -> int:
    n = load().vkv_kv_block_bytes(num_layers, block_size, num_kv_heads, head_dim, kv_dtype)
    if n < 0:
        check(int(n))
    return int(n)


def rope_cos_sin_host(theta: float, head_dim: int, max_position: int):
    """The reference's RoPE table [max_position, head_dim/2, 2] fp32 (numpy), built by the library."""
    import numpy as np
    t = np.zeros((max_position, head_dim // 2, 2), np.float32)
    check(load().vkv_rope_cos_sin_host(theta, head_dim, max_position, t.ctypes.data))
    return t


def rope_reshape_and_cache(query, key, value, cos_sin, positions=None, start_pos=0,
                           key_cache=None, value_cache=None, slot_mapping=None,
                           key_scales=None, value_scales=None, stream=None) -> None:
    """query [T, H, D], key/value [T, Hkv, D] (f32 or f16); cos_sin [P, D/2, 2] fp32 on the GPU;
    positions int32 [T] or None (start_pos + t).  With caches: query rotated in place, rotated
    key and value stored through slot_mapping.  Without: query and key rotated in place."""
    _require_cuda(query, key, value, cos_sin, positions, key_cache, value_cache, slot_mapping,
                  key_scales, value_scales)
    T, H, D = query.shape
    Hkv = key.shape[1]
    N = bs = 0
    cache_dtype = DTYPE_F16
    if key_cache is not None:
        N, bs = key_cache.shape[0], key_cache.shape[1]
        cache_dtype = _dtype_code(key_cache)
    p = RopeAppendParams(
        query=_ptr(query), key=_ptr(key), value=_ptr(value), query_stride=query.stride(0),
        key_stride=key.stride(0), value_stride=0 if value is None else value.stride(0),
        cos_sin=_ptr(cos_sin), positions=_ptr(positions), start_pos=start_pos,
        max_position=cos_sin.shape[0], key_cache=_ptr(key_cache), value_cache=_ptr(value_cache),
        key_scales=_ptr(key_scales), value_scales=_ptr(value_scales), slot_mapping=_ptr(slot_mapping),
        num_tokens=T, num_heads=H, num_kv_heads=Hkv, head_dim=D, block_size=bs, num_blocks=N,
        src_dtype=_dtype_code(query), cache_dtype=cache_dtype)
    check(load().vkv_rope_reshape_and_cache(ctypes.byref(p), _stream(stream)))


def decode_params(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                  key_scales=None, value_scales=None, max_context_len=None,
                  accumulate=False, partition_size=0, workspace=None) -> DecodeParams:
    S, H, D = out.shape
    N, bs, Hkv, _ = key_cache.shape
    MB = block_tables.shape[1]
    return DecodeParams(
        output=_ptr(out), query=_ptr(query), key_cache=_ptr(key_cache), value_cache=_ptr(value_cache),
        key_scales=_ptr(key_scales), value_scales=_ptr(value_scales),
        block_tables=_ptr(block_tables), context_lens=_ptr(context_lens),
        query_stride=query.stride(0), num_seqs=S, num_heads=H, num_kv_heads=Hkv, head_dim=D,
        block_size=bs, max_context_len=MB * bs if max_context_len is None else max_context_len,
        max_blocks_per_seq=MB, num_blocks=N, scale=scale, io_dtype=_dtype_code(out),
        kv_dtype=_dtype_code(key_cache), accumulate=int(accumulate), partition_size=partition_size,
        workspace=_ptr(workspace), workspace_bytes=0 if workspace is None else workspace.numel() * workspace.element_size())


def paged_decode(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                 key_scales=None, value_scales=None, max_context_len=None, accumulate=False,
                 partition_size=0, workspace=None, stream=None) -> None:
    """out/query [S, H, D] (f32 or f16); caches [N, bs, Hkv, D]; block_tables int32 [S, MB];
    context_lens int32 [S]."""
    _require_cuda(out, query, key_cache, value_cache, block_tables, context_lens, key_scales,
                  value_scales, workspace)
    p = decode_params(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                      key_scales, value_scales, max_context_len, accumulate, partition_size, workspace)
    check(load().vkv_paged_decode(ctypes.byref(p), _stream(stream)))


def paged_decode_append(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                        key, value, slot_mapping, key_scales=None, value_scales=None,
                        max_context_len=None, accumulate=False, partition_size=0, workspace=None,
                        stream=None) -> None:
    """vkv_paged_decode_append: reshape_and_cache(key, value, ..., slot_mapping) then
    paged_decode(...), the append fused into the decode when the shapes allow (key/value
    [num_seqs, Hkv, D], token s being sequence s's new token)."""
    _require_cuda(out, query, key_cache, value_cache, block_tables, context_lens, key, value, slot_mapping,
                  key_scales, value_scales, workspace)
    ap = append_params(key, value, key_cache, value_cache, slot_mapping, key_scales, value_scales)
    dp = decode_params(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                       key_scales, value_scales, max_context_len, accumulate, partition_size, workspace)
    check(load().vkv_paged_decode_append(ctypes.byref(ap), ctypes.byref(dp), _stream(stream)))


def paged_decode_noalloc(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                         key_scales=None, value_scales=None, max_context_len=None, accumulate=False,
                         partition_size=0, stream=None) -> None:
    """paged_decode with the split-K workspace in the library's fixed device array
    (no allocation; overlapping calls on one device race)."""
    _require_cuda(out, query, key_cache, value_cache, block_tables, context_lens, key_scales, value_scales)
    p = decode_params(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                      key_scales, value_scales, max_context_len, accumulate, partition_size, None)
    check(load().vkv_paged_decode_noalloc(ctypes.byref(p), _stream(stream)))


def decode_workspace_size(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                          key_scales=None, value_scales=None, max_context_len=None,
                          partition_size=0) -> int:
    p = decode_params(out, query, key_cache, value_cache, block_tables, context_lens, scale,
                      key_scales, value_scales, max_context_len, False, partition_size, None)
    return int(load().vkv_paged_decode_workspace_size(ctypes.byref(p)))


def prefill_params(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                   max_query_len, scale, key_scales=None, value_scales=None, max_context_len=0,
                   workspace=None, multi_token_only=False) -> PrefillParams:
    Tq, H, D = out.shape
    N, bs, Hkv, _ = key_cache.shape
    return PrefillParams(
        output=_ptr(out), query=_ptr(query), key_cache=_ptr(key_cache), value_cache=_ptr(value_cache),
        key_scales=_ptr(key_scales), value_scales=_ptr(value_scales),
        block_tables=_ptr(block_tables), context_lens=_ptr(context_lens),
        query_start_loc=_ptr(query_start_loc), query_stride=query.stride(0),
        num_seqs=context_lens.shape[0], num_query_tokens=Tq, max_query_len=max_query_len,
        num_heads=H, num_kv_heads=Hkv, head_dim=D, block_size=bs,
        max_blocks_per_seq=block_tables.shape[1], num_blocks=N, scale=scale,
        io_dtype=_dtype_code(out), kv_dtype=_dtype_code(key_cache), max_context_len=max_context_len,
        multi_token_only=1 if multi_token_only else 0, workspace=_ptr(workspace),
        workspace_bytes=0 if workspace is None else workspace.numel() * workspace.element_size())


def paged_prefill(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                  max_query_len, scale, key_scales=None, value_scales=None, max_context_len=0,
                  workspace=None, stream=None, multi_token_only=False, work_list=None) -> None:
    """out/query [Tq, H, D]; query_start_loc int32 [S+1]; context_lens counts the step's tokens.
    max_context_len > 0 clamps every row's keys; workspace (optional) as for paged_decode;
    multi_token_only: the caller's promise that no sequence has exactly one query token
    (skips the decode pass that serves those); work_list: a device int32 copy of
    prefill_work_list()'s words for this call (optional)."""
    _require_cuda(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                  key_scales, value_scales, workspace, work_list)
    p = prefill_params(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                       max_query_len, scale, key_scales, value_scales, max_context_len, workspace,
                       multi_token_only)
    if work_list is not None and work_list.numel() > 0:
        p.work_list = work_list.data_ptr()
        p.work_list_words = int(work_list.numel())
    check(load().vkv_paged_prefill(ctypes.byref(p), _stream(stream)))


def prefill_work_list(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                      max_query_len, scale, host_query_start_loc, host_context_lens, key_scales=None,
                      value_scales=None, max_context_len=0):
    """vkv_prefill_work_list_host for the call these arguments describe, from host (numpy)
    copies of its query_start_loc and context_lens: int32 numpy words (empty when the
    call's shape runs without a list)."""
    import numpy as np
    p = prefill_params(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                       max_query_len, scale, key_scales, value_scales, max_context_len, None)
    hq = np.ascontiguousarray(host_query_start_loc, dtype=np.int32)
    hc = np.ascontiguousarray(host_context_lens, dtype=np.int32)
    n = int(load().vkv_prefill_work_list_host(ctypes.byref(p), hq.ctypes.data, hc.ctypes.data, None, 0))
    if n < 0:
        raise VkvError(n, "vkv_prefill_work_list_host failed")
    words = np.zeros(n, np.int32)
    if n:
        r = int(load().vkv_prefill_work_list_host(ctypes.byref(p), hq.ctypes.data, hc.ctypes.data,
                                                  words.ctypes.data, n))
        if r != n:
            raise VkvError(r, "vkv_prefill_work_list_host failed")
    return words


def prefill_workspace_size(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                           max_query_len, scale, key_scales=None, value_scales=None, max_context_len=0) -> int:
    p = prefill_params(out, query, key_cache, value_cache, block_tables, context_lens, query_start_loc,
                       max_query_len, scale, key_scales, value_scales, max_context_len, None)
    return int(load().vkv_paged_prefill_workspace_size(ctypes.byref(p)))


def planes_of(tensors: Sequence, num_layers: int):
    """Plane descriptors for per-layer arrays stacked as [L, N, ...] tensors."""
    arr = (BlockPlane * len(tensors))()
    for i, t in enumerate(tensors):
        assert t.shape[0] == num_layers
        arr[i].base = t.data_ptr()
        arr[i].layer_stride_bytes = t.stride(0) * t.element_size()
        arr[i].block_bytes = t.stride(1) * t.element_size()
    return arr


def copy_blocks(layer_tensors: Sequence, block_pairs, stream=None) -> None:
    """layer_tensors: [L, N, ...] tensors (K, V[, K scales, V scales]); block_pairs int32 [P, 2] on GPU."""
    _require_cuda(*layer_tensors, block_pairs)
    L, N = layer_tensors[0].shape[:2]
    planes = planes_of(layer_tensors, L)
    check(load().vkv_copy_blocks(planes, len(layer_tensors), L, N, _ptr(block_pairs),
                                 block_pairs.shape[0], _stream(stream)))


def swap_blocks(layer_tensors: Sequence, host_buffer, num_host_blocks: int, block_pairs,
                direction: int, stream=None) -> None:
    """host_buffer: pinned CPU tensor of num_host_blocks * host_block_bytes bytes."""
    _require_cuda(*layer_tensors, block_pairs)
    L, N = layer_tensors[0].shape[:2]
    planes = planes_of(layer_tensors, L)
    check(load().vkv_swap_blocks(planes, len(layer_tensors), L, N, host_buffer.data_ptr(),
                                 num_host_blocks, _ptr(block_pairs), block_pairs.shape[0],
                                 direction, _stream(stream)))


def host_block_bytes(layer_tensors: Sequence) -> int:
    L = layer_tensors[0].shape[0]
    return int(load().vkv_swap_host_block_bytes(planes_of(layer_tensors, L), len(layer_tensors), L))
