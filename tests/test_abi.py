"""CPU checks of the C ABI library: it loads without a GPU, exports every symbol
the header declares, and rejects bad arguments on the host before any launch."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vllm_kv_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vkv_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_binding_list(vkv):
    assert declared_functions() == sorted(vkv.EXPORTED)


def test_library_exports_every_declared_symbol(vkv):
    lib = vkv.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.vkv_abi_version() == vkv.ABI_VERSION == 4


def test_struct_sizes_match_header_layout(vkv):
    # int64 after 8 pointers etc.: sizes fixed by the C layout rules (x86-64 SysV)
    assert ctypes.sizeof(vkv.AppendParams) == 9 * 8 + 7 * 4 + 4  # trailing pad to 8
    assert ctypes.sizeof(vkv.DecodeParams) == 8 * 8 + 8 + 14 * 4 + 8 + 8
    assert ctypes.sizeof(vkv.BlockPlane) == 24
    assert ctypes.sizeof(vkv.RopeAppendParams) == 3 * 8 + 3 * 8 + 2 * 8 + 2 * 4 + 5 * 8 + 8 * 4
    # 9 pointers, query_stride, 14 int32/float, workspace pointer and size
    assert ctypes.sizeof(vkv.PrefillParams) == 9 * 8 + 8 + 14 * 4 + 8 + 8 + 8 + 8  # work_list, words + pad
    assert vkv.PrefillParams.work_list.offset == 152
    assert vkv.PrefillParams.multi_token_only.offset == 132
    assert vkv.PrefillParams.workspace.offset == 136


def _decode_params(vkv, **over):
    p = vkv.DecodeParams(output=16, query=16, key_cache=16, value_cache=16, block_tables=16, context_lens=16,
                         num_seqs=2, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                         max_context_len=4096, max_blocks_per_seq=256, num_blocks=1000, scale=0.088,
                         io_dtype=1, kv_dtype=1)
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code", [
    (dict(num_heads=30), -2),            # not a multiple of num_kv_heads
    (dict(head_dim=0), -2),
    (dict(head_dim=1025), -3),           # beyond the generic kernel's largest head_dim
    (dict(block_size=0), -2),
    (dict(io_dtype=1, kv_dtype=0), -3),  # fp32 KV with fp16 io
    (dict(kv_dtype=2), -1),              # fp8 without scales
    (dict(query=0), -1),
    (dict(key_cache=25), -5),            # not even fp16-aligned
    (dict(max_blocks_per_seq=0), -2),
])
def test_decode_argument_errors(vkv, over, code):
    lib = vkv.load()
    p = _decode_params(vkv, **over)
    assert lib.vkv_paged_decode(ctypes.byref(p), None) == code
    assert lib.vkv_last_error()


def test_decode_zero_sequences_is_noop(vkv):
    lib = vkv.load()
    p = _decode_params(vkv, num_seqs=0)
    assert lib.vkv_paged_decode(ctypes.byref(p), None) == 0


def test_workspace_size_formula(vkv):
    lib = vkv.load()
    p = _decode_params(vkv, num_seqs=64, max_context_len=4112, max_blocks_per_seq=257)
    # 1 KiB of claim counters, then partials of (D + 2) floats per (seq, head, partition).  The
    # default size is 768 tokens, but the kernels may pick a size per call from 3/4 of that
    # (576 tokens, a multiple of the 16-token block) upwards: ceil(4112/576) = 8 partitions
    assert lib.vkv_paged_decode_workspace_size(ctypes.byref(p)) == 1024 + 64 * 32 * 8 * (128 + 2) * 4
    p.partition_size = 512  # ceil(4112/512) = 9
    assert lib.vkv_paged_decode_workspace_size(ctypes.byref(p)) == 1024 + 64 * 32 * 9 * (128 + 2) * 4


def test_decode_append_argument_errors(vkv):
    """vkv_paged_decode_append checks both parameter blocks first (no GPU)."""
    lib = vkv.load()
    dp = _decode_params(vkv)
    ap = vkv.AppendParams(key=16, value=16, key_cache=16, value_cache=16, slot_mapping=16, num_tokens=2,
                          num_kv_heads=8, head_dim=128, block_size=16, num_blocks=1000, src_dtype=1, cache_dtype=1)
    assert lib.vkv_paged_decode_append(None, ctypes.byref(dp), None) == -1
    assert lib.vkv_paged_decode_append(ctypes.byref(ap), None, None) == -1
    ap.num_kv_heads = 0
    assert lib.vkv_paged_decode_append(ctypes.byref(ap), ctypes.byref(dp), None) == -2
    ap.num_kv_heads = 8
    dp.num_heads = 30
    assert lib.vkv_paged_decode_append(ctypes.byref(ap), ctypes.byref(dp), None) == -2
    # nothing to append and nothing to decode: nothing launched
    ap.num_tokens = 0
    dp.num_seqs = 0
    assert lib.vkv_paged_decode_append(ctypes.byref(ap), ctypes.byref(dp), None) == 0


def test_append_argument_errors(vkv):
    lib = vkv.load()
    base = dict(key=16, value=16, key_cache=16, value_cache=16, slot_mapping=16, num_tokens=4, num_kv_heads=8,
                head_dim=128, block_size=16, num_blocks=10, src_dtype=1, cache_dtype=1)
    p = vkv.AppendParams(**base)
    p.key_stride = 3  # smaller than a row
    assert lib.vkv_reshape_and_cache(ctypes.byref(p), None) == -2
    p = vkv.AppendParams(**{**base, "cache_dtype": 2})
    assert lib.vkv_reshape_and_cache(ctypes.byref(p), None) == -1  # fp8 needs scales
    p = vkv.AppendParams(**{**base, "src_dtype": 1, "cache_dtype": 0})
    assert lib.vkv_reshape_and_cache(ctypes.byref(p), None) == -3
    p = vkv.AppendParams(**{**base, "key": 17})
    assert lib.vkv_reshape_and_cache(ctypes.byref(p), None) == -5  # not fp16-aligned
    p = vkv.AppendParams(**{**base, "num_tokens": 0})
    assert lib.vkv_reshape_and_cache(ctypes.byref(p), None) == 0


def test_slot_mapping_host_matches_reference_placement(vkv):
    """slot = block_table[pos/bs]*bs + pos%bs (src/layers/attention.cpp:85-94); a
    position beyond the table is an error (the reference aborts, :87-90)."""
    lib = vkv.load()
    table = np.array([7, 2, 9], np.int32)
    out = np.zeros(5, np.int32)
    assert lib.vkv_slot_mapping_host(table.ctypes.data, 3, 16, 14, 5, out.ctypes.data) == 0
    assert out.tolist() == [7 * 16 + 14, 7 * 16 + 15, 2 * 16 + 0, 2 * 16 + 1, 2 * 16 + 2]
    assert lib.vkv_slot_mapping_host(table.ctypes.data, 3, 16, 46, 5, out.ctypes.data) == -2


def test_copy_pairs_check(vkv):
    lib = vkv.load()
    ok = np.array([[0, 5], [1, 6], [2, 7]], np.int32)
    assert lib.vkv_check_block_pairs_host(ok.ctypes.data, 3, 8) == 0
    bad = np.array([[0, 5], [5, 6]], np.int32)
    assert lib.vkv_check_block_pairs_host(bad.ctypes.data, 2, 8) == -2
    oob = np.array([[0, 8]], np.int32)
    assert lib.vkv_check_block_pairs_host(oob.ctypes.data, 1, 8) == -2


def test_rope_argument_errors(vkv):
    lib = vkv.load()
    base = dict(query=16, key=16, value=16, cos_sin=16, max_position=100, key_cache=16, value_cache=16,
                slot_mapping=16, num_tokens=4, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                num_blocks=10, src_dtype=1, cache_dtype=1)

    def call(**over):
        p = vkv.RopeAppendParams(**{**base, **over})
        return lib.vkv_rope_reshape_and_cache(ctypes.byref(p), None)

    assert call(head_dim=96) == -3
    assert call(cos_sin=0) == -1
    assert call(max_position=0) == -2
    assert call(cache_dtype=2) == -1              # FP8 needs scales
    assert call(cache_dtype=0) == -3              # fp32 cache from fp16 source
    assert call(query=24) == -5                   # misaligned
    assert call(query_stride=100) == -2           # shorter than a token's heads
    assert call(value=0) == -1                    # fused mode needs the value rows
    assert call(num_tokens=0) == 0
    # rope-only mode ignores the value and cache fields
    p = vkv.RopeAppendParams(**{**base, "key_cache": 0, "value": 0, "slot_mapping": 0, "num_tokens": 0})
    assert lib.vkv_rope_reshape_and_cache(ctypes.byref(p), None) == 0


def test_kv_pool_sizing_with_element_type(vkv):
    """src/model/qwen.cpp:72-73,94-104 restated: fp32 equals the reference's formula exactly;
    fp16 / FP8 use their element bytes (FP8 + one fp32 scale per slot and kv head)."""
    L, bs, Hkv, D = 32, 16, 8, 128
    ref_per_block = 2 * bs * Hkv * D * 4 * L  # sizeof(float) in the reference
    assert vkv.kv_block_bytes(L, bs, Hkv, D, vkv.DTYPE_F32) == ref_per_block
    assert vkv.kv_block_bytes(L, bs, Hkv, D, vkv.DTYPE_F16) == ref_per_block // 2
    assert vkv.kv_block_bytes(L, bs, Hkv, D, vkv.DTYPE_FP8) == 2 * bs * Hkv * (D + 4) * L
    budget, non_kv = 250 * 2**30, 20 * 2**30
    for dt in (vkv.DTYPE_F32, vkv.DTYPE_F16, vkv.DTYPE_FP8):
        per = vkv.kv_block_bytes(L, bs, Hkv, D, dt)
        want = min(256 * ((32768 + bs - 1) // bs), (budget - non_kv) // per)
        assert vkv.kv_pool_num_blocks(budget, non_kv, L, bs, Hkv, D, dt, 256, 32768) == want
    f32 = vkv.kv_pool_num_blocks(budget, non_kv, L, bs, Hkv, D, vkv.DTYPE_F32, 10**6, 10**6)
    f16 = vkv.kv_pool_num_blocks(budget, non_kv, L, bs, Hkv, D, vkv.DTYPE_F16, 10**6, 10**6)
    fp8 = vkv.kv_pool_num_blocks(budget, non_kv, L, bs, Hkv, D, vkv.DTYPE_FP8, 10**6, 10**6)
    assert f16 in (2 * f32, 2 * f32 + 1) and 3.8 * f32 < fp8 < 4 * f32 + 4
    assert vkv.kv_pool_num_blocks(non_kv, non_kv, L, bs, Hkv, D, vkv.DTYPE_F16, 8, 4096) == 0
    assert vkv.kv_pool_num_blocks(budget, non_kv, L, bs, Hkv, D, vkv.DTYPE_F16, 2, 100) == 2 * 7
    with pytest.raises(vkv.VkvError):
        vkv.kv_block_bytes(L, bs, Hkv, D, 7)


def _prefill_params(vkv, **over):
    p = vkv.PrefillParams(output=16, query=16, key_cache=16, value_cache=16, block_tables=16, context_lens=16,
                          query_start_loc=16, num_seqs=3, num_query_tokens=600, max_query_len=512, num_heads=28,
                          num_kv_heads=4, head_dim=128, block_size=32, max_blocks_per_seq=80, num_blocks=1000,
                          scale=0.088, io_dtype=1, kv_dtype=1)
    for k, v in over.items():
        setattr(p, k, v)
    return p


def test_prefill_argument_errors_and_workspace(vkv):
    lib = vkv.load()
    assert lib.vkv_paged_prefill(ctypes.byref(_prefill_params(vkv, query_start_loc=0)), None) == -1
    assert lib.vkv_paged_prefill(ctypes.byref(_prefill_params(vkv, max_query_len=0)), None) == -2
    assert lib.vkv_paged_prefill(ctypes.byref(_prefill_params(vkv, max_context_len=-1)), None) == -2
    assert lib.vkv_paged_prefill(ctypes.byref(_prefill_params(vkv, multi_token_only=2)), None) == -2
    assert lib.vkv_paged_prefill(ctypes.byref(_prefill_params(vkv, num_query_tokens=0)), None) == 0
    need = lib.vkv_paged_prefill_workspace_size(ctypes.byref(_prefill_params(vkv)))
    # at least the 1 KiB header and the partials of the 3 sequences' decode rows
    assert need >= 1024 + 3 * 28 * (128 + 2) * 4
    p = _prefill_params(vkv, workspace=256, workspace_bytes=need - 16)
    assert lib.vkv_paged_prefill(ctypes.byref(p), None) == -4       # too small
    p = _prefill_params(vkv, workspace=8, workspace_bytes=need)
    assert lib.vkv_paged_prefill(ctypes.byref(p), None) == -5       # misaligned
    assert lib.vkv_paged_prefill_workspace_size(ctypes.byref(_prefill_params(vkv, head_dim=0))) == 0


@pytest.mark.parametrize("shape", [(28, 4, 128, 32, 1, 1), (32, 8, 128, 16, 1, 2), (16, 8, 64, 16, 1, 1),
                                   (32, 2, 128, 16, 1, 1)])
def test_prefill_work_list_host(vkv, shape):
    """vkv_prefill_work_list_host (no GPU): every work item (sequence, row block,
    kv head) of the call exactly once, with its sequence's query rows and prior
    context, dealt to one list per workgroup longest first, each to the least
    loaded list; no list for shapes the matrix-core kernels do not run;
    capacity and argument errors."""
    import numpy as np
    H, Hkv, D, bs, io, kv = shape
    rng = np.random.default_rng(H + D)
    q_lens = np.concatenate([rng.integers(2, 700, 9), [1, 1, 1]]).astype(np.int32)
    prior = rng.integers(0, 3000, q_lens.size).astype(np.int32)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    ctx = (prior + q_lens).astype(np.int32)
    mb = int((ctx.max() + bs - 1) // bs)
    p = _prefill_params(vkv, num_seqs=q_lens.size, num_query_tokens=int(qsl[-1]), max_query_len=int(q_lens.max()),
                        num_heads=H, num_kv_heads=Hkv, head_dim=D, block_size=bs, max_blocks_per_seq=mb,
                        io_dtype=io, kv_dtype=kv)
    lib = vkv.load()
    n = lib.vkv_prefill_work_list_host(ctypes.byref(p), qsl.ctypes.data, ctx.ctypes.data, None, 0)
    G = H // Hkv
    rows = 256 if D == 128 else 512
    want = {}
    for s in range(q_lens.size):
        if q_lens[s] < 2:
            continue
        nb = (int(q_lens[s]) * G + rows - 1) // rows
        for b in range(nb):
            last = min(int(q_lens[s]), ((b + 1) * rows - 1) // G + 1)
            t = (int(prior[s]) + last + 63) // 64
            for k in range(Hkv):
                want[(s, b, k)] = (int(qsl[s]), int(q_lens[s]), int(prior[s]), t)
    # one list per CU (256 on this device, and without a device), at most one
    # per item; slot k of list w at k W + w, 8 words each, s = -1 past its end
    lists = min(256, len(want))
    words = np.zeros(n, np.int32)
    assert lib.vkv_prefill_work_list_host(ctypes.byref(p), qsl.ctypes.data, ctx.ctypes.data,
                                          words.ctypes.data, n - 1) == -2
    assert lib.vkv_prefill_work_list_host(ctypes.byref(p), qsl.ctypes.data, ctx.ctypes.data,
                                          words.ctypes.data, n) == n
    assert words[0] == lists and words[2] == 3 and words[3] == len(want)
    L = int(words[1])
    assert n == 32 + 8 * lists * L
    slots = words[32:].reshape(L, lists, 8)
    got = {}
    per_list = []
    for w in range(lists):
        col = [slots[k, w] for k in range(L) if slots[k, w, 0] >= 0]
        assert all(slots[k, w, 0] == -1 for k in range(len(col), L))  # the list ends once
        per_list.append(col)
        for e in col:
            got[(int(e[0]), int(e[1]), int(e[2]))] = (int(e[3]), int(e[4]), int(e[5]), int(e[6]))
    assert got == want and sum(len(c) for c in per_list) == len(want)
    assert L == max(len(c) for c in per_list)
    # the deal, replayed: longest first (ties in (s, b, kvh) order), each item
    # to the least loaded list (ties: the lowest), an item costing its key
    # tiles + 5; each list holds its items in the order dealt
    order = sorted(want, key=lambda k: (-want[k][3], k))
    load = [0] * lists
    dealt = [[] for _ in range(lists)]
    for key in order:
        w = min(range(lists), key=lambda x: (load[x], x))
        load[w] += want[key][3] + 5
        dealt[w].append(key)
    assert dealt == [[(int(e[0]), int(e[1]), int(e[2])) for e in c] for c in per_list]
    # shapes without the list: fp32 queries, FP8 at head_dim 64, and fp16 at
    # head_dim 64 with groups of 4 heads or more (the register-staged kernel)
    p32 = _prefill_params(vkv, io_dtype=0, kv_dtype=0)
    assert lib.vkv_prefill_work_list_host(ctypes.byref(p32), qsl.ctypes.data, ctx.ctypes.data, None, 0) == 0
    p8 = _prefill_params(vkv, head_dim=64, kv_dtype=2)
    assert lib.vkv_prefill_work_list_host(ctypes.byref(p8), qsl.ctypes.data, ctx.ctypes.data, None, 0) == 0
    p64 = _prefill_params(vkv, num_seqs=q_lens.size, num_query_tokens=int(qsl[-1]), max_query_len=int(q_lens.max()),
                          num_heads=16, num_kv_heads=4, head_dim=64, block_size=16, max_blocks_per_seq=mb)
    assert lib.vkv_prefill_work_list_host(ctypes.byref(p64), qsl.ctypes.data, ctx.ctypes.data, None, 0) == 0
    assert lib.vkv_prefill_work_list_host(ctypes.byref(p), None, ctx.ctypes.data, None, 0) == -1
    # a negative length is refused before any launch
    assert lib.vkv_paged_prefill(ctypes.byref(_prefill_params(vkv, work_list_words=-1)), None) == -2
