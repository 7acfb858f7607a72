"""GPU parity of paged decode attention against the oracle.

The oracle restates src/attention/paged_attention.cu:13-82.  fp16 outputs must be
within 2e-3 abs + 1e-2 rel of it; the fp32 reference-API path within
2e-5 abs + 1e-4 rel.  FP8-KV outputs are compared with the oracle run on the
same FP8 cache (codes and scales), at the fp16 bound, which is tighter than the
3e-2 relative the FP8 contract allows; their distance to the unquantised fp16
result (quantisation error, not parity) is only bounded loosely.
"""
import numpy as np
import pytest

from helpers import (F16_ATOL, F16_RTOL, F32_ATOL, F32_RTOL, assert_close, to_dev, to_np)

pytestmark = pytest.mark.gpu


def _pool(rng, N, bs, Hkv, D, sigma):
    k = (rng.standard_normal((N, bs, Hkv, D), dtype=np.float32) * sigma).astype(np.float16)
    v = (rng.standard_normal((N, bs, Hkv, D), dtype=np.float32) * sigma).astype(np.float16)
    return k, v


def _layout(rng, ctx, bs, extra_blocks=3):
    from vllm_kv_amd import workloads
    need = int(sum((c + bs - 1) // bs for c in ctx))
    return workloads.make_layout(np.asarray(ctx, np.int32), bs, rng, num_blocks=max(need + extra_blocks, 1),
                                 max_blocks_per_seq=max(1, max((c + bs - 1) // bs for c in ctx)))


def _run_decode(vkv, cuda, q, k, v, lay, scale, io, **kw):
    import torch
    tdt = torch.float16 if io == np.float16 else torch.float32
    S, H, D = q.shape
    out = torch.zeros((S, H, D), dtype=tdt, device=cuda)
    vkv.paged_decode(out, to_dev(q.astype(io), cuda), to_dev(k, cuda), to_dev(v, cuda),
                     to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda), scale, **kw)
    torch.cuda.synchronize()
    return to_np(out).astype(np.float32)


CASES = [
    # (H, Hkv, D, bs, contexts)
    (14, 2, 64, 16, [1, 17, 255, 256, 257, 600]),
    (32, 8, 128, 16, [1, 2, 16, 100, 511, 512, 513, 1300]),
    (28, 4, 128, 32, [31, 32, 33, 700]),
    (8, 8, 128, 16, [5, 300]),
    (16, 8, 256, 8, [9, 64, 520]),
    (24, 4, 64, 64, [1, 63, 64, 65, 1000]),
    (40, 5, 128, 16, [77, 290]),
    (24, 8, 128, 16, [0, 7, 33]),
]


@pytest.mark.parametrize("H,Hkv,D,bs,ctx", CASES)
def test_decode_f16_vs_oracle(vkv, oracle, cuda, H, Hkv, D, bs, ctx):
    rng = np.random.default_rng(H * 1000 + D + bs)
    lay = _layout(rng, ctx, bs)
    k, v = _pool(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    q = (rng.standard_normal((len(ctx), H, D), dtype=np.float32) * 0.5).astype(np.float16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    ref = oracle.paged_decode(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                              lay.context_lens, scale)
    got = _run_decode(vkv, cuda, q, k, v, lay, scale, np.float16)
    assert_close(got, ref, F16_ATOL, F16_RTOL, "fp16 decode")


# Shapes outside the fixed-shape kernels (head_dim 64/128/256, group <= 8,
# power-of-two blocks) run on the generic variant: any head_dim up to 1024
# (whole 16-byte vectors or single elements), any group size (query heads in
# chunks), any block size.  (H, Hkv, D, bs, contexts, io dtype, kv dtype)
GENERIC_CASES = [
    (32, 2, 80, 12, [1, 13, 300, 1000], "f16", "f16"),    # group 16, head_dim 80
    (64, 2, 96, 24, [5, 24, 25, 777], "f16", "f16"),      # group 32
    (64, 1, 128, 16, [3, 200, 1500], "f16", "f16"),       # MQA, group 64
    (16, 16, 112, 16, [9, 400], "f16", "f16"),            # group 1, head_dim 112
    (12, 4, 100, 10, [1, 11, 250], "f16", "f16"),         # 200-byte heads: element loads
    (8, 8, 33, 5, [1, 6, 77], "f16", "f16"),              # odd head_dim and block size
    (8, 2, 64, 1, [1, 2, 100], "f16", "f16"),             # one-token blocks
    (4, 1, 576, 16, [2, 300], "f16", "f16"),              # head_dim 576 (two vectors per lane)
    (8, 2, 1024, 8, [17, 129], "f16", "f16"),             # the largest head_dim
    (20, 5, 128, 48, [47, 48, 49, 2000], "f16", "f16"),   # power-of-two head_dim, block 48
    (32, 2, 80, 12, [1, 40, 900], "f32", "f32"),          # the reference API's dtype
    (6, 3, 98, 7, [3, 70], "f32", "f32"),                 # fp32 element loads
    (20, 2, 96, 24, [8, 333], "f32", "f16"),
    (32, 2, 96, 16, [1, 130, 600], "f16", "fp8"),         # FP8 cache, group 16
    (24, 8, 64, 12, [12, 13, 500], "f16", "fp8"),         # FP8, non-power-of-two blocks
    (16, 4, 104, 8, [5, 300], "f32", "fp8"),              # FP8 104-byte heads: element loads
]


@pytest.mark.parametrize("H,Hkv,D,bs,ctx,io,kv", GENERIC_CASES)
def test_decode_generic_shapes_vs_oracle(vkv, oracle, cuda, H, Hkv, D, bs, ctx, io, kv):
    import torch
    rng = np.random.default_rng(H * 7 + D * 3 + bs)
    lay = _layout(rng, ctx, bs)
    N = lay.num_blocks
    kf = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32) * 0.5
    vf = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32) * 0.5
    q = rng.standard_normal((len(ctx), H, D), dtype=np.float32) * 0.5
    scale = float(1.0 / np.sqrt(np.float32(D)))
    ks = vs = hks = hvs = None
    if kv == "f32":
        hk, hv, kc, vc = kf, vf, to_dev(kf, cuda), to_dev(vf, cuda)
    elif kv == "f16":
        hk, hv = kf.astype(np.float16).view(np.uint16), vf.astype(np.float16).view(np.uint16)
        kc, vc = to_dev(hk.view(np.float16), cuda), to_dev(hv.view(np.float16), cuda)
    else:  # FP8 codes and scales from the oracle's quantisation of the fp16 pool
        k16, v16 = kf.astype(np.float16).view(np.uint16), vf.astype(np.float16).view(np.uint16)
        hk = np.zeros((N, bs, Hkv, D), np.uint8)
        hv = np.zeros_like(hk)
        hks = np.zeros((N, bs, Hkv), np.float32)
        hvs = np.zeros_like(hks)
        oracle.reshape_and_cache(k16.reshape(-1, Hkv, D), v16.reshape(-1, Hkv, D), hk, hv,
                                 np.arange(N * bs, dtype=np.int32), hks, hvs)
        kc, vc, ks, vs = (to_dev(x, cuda) for x in (hk, hv, hks, hvs))
    if io == "f16":
        q = q.astype(np.float16).astype(np.float32)
    ref = oracle.paged_decode(q, hk, hv, lay.block_tables, lay.context_lens, scale, key_scales=hks,
                              value_scales=hvs)
    out = torch.zeros((len(ctx), H, D), dtype=torch.float16 if io == "f16" else torch.float32, device=cuda)
    qd = to_dev(q.astype(np.float16) if io == "f16" else q, cuda)
    vkv.paged_decode(out, qd, kc, vc, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda), scale,
                     key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    tol = {"f16": (F16_ATOL, F16_RTOL), "f32": (F32_ATOL, F32_RTOL if kv == "f32" else 1e-3)}[io]
    assert_close(to_np(out).astype(np.float32), ref, *tol, f"generic decode {H}/{Hkv}/{D}/bs{bs} {io}/{kv}")


def test_decode_generic_unaligned_cache(vkv, oracle, cuda):
    """Caches that are only element-aligned (an fp16 pool starting 2 bytes into
    its allocation) at a fixed-kernel shape take the generic variant with
    element loads; same result as the oracle."""
    import torch
    rng = np.random.default_rng(41)
    H, Hkv, D, bs, ctx = 32, 8, 128, 16, [3, 300, 1100]
    lay = _layout(rng, ctx, bs)
    k, v = _pool(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    q = (rng.standard_normal((len(ctx), H, D), dtype=np.float32) * 0.5).astype(np.float16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    ref = oracle.paged_decode(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                              lay.context_lens, scale)
    flat_k = torch.zeros(k.size + 8, dtype=torch.float16, device=cuda)
    flat_v = torch.zeros(v.size + 8, dtype=torch.float16, device=cuda)
    flat_k[1:1 + k.size] = to_dev(k.reshape(-1), cuda)
    flat_v[1:1 + v.size] = to_dev(v.reshape(-1), cuda)
    kc = flat_k[1:1 + k.size].view(k.shape)
    vc = flat_v[1:1 + v.size].view(v.shape)
    assert kc.data_ptr() % 16 == 2
    got = torch.zeros((len(ctx), H, D), dtype=torch.float16, device=cuda)
    vkv.paged_decode(got, to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda),
                     scale)
    torch.cuda.synchronize()
    assert_close(to_np(got).astype(np.float32), ref, F16_ATOL, F16_RTOL, "unaligned fp16 cache")


@pytest.mark.parametrize("partition_size", [16, 64, 128, 512])
def test_decode_partition_sizes(vkv, oracle, cuda, partition_size):
    """Split-K merging is independent of where the context is cut."""
    rng = np.random.default_rng(5)
    ctx = [1, 15, 16, 17, 300, 1025]
    lay = _layout(rng, ctx, 16)
    k, v = _pool(rng, lay.num_blocks, 16, 4, 128, 0.5)
    q = (rng.standard_normal((len(ctx), 16, 128), dtype=np.float32) * 0.5).astype(np.float16)
    scale = 1.0 / np.sqrt(128.0)
    ref = oracle.paged_decode(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                              lay.context_lens, scale)
    got = _run_decode(vkv, cuda, q, k, v, lay, scale, np.float16, partition_size=partition_size)
    assert_close(got, ref, F16_ATOL, F16_RTOL, f"partition {partition_size}")


def test_decode_f32_reference_api_semantics(vkv, oracle, cuda):
    """fp32 Q/K/V/output, output accumulated into (reference `out +=`), ctx clamp
    to max_context_len, ctx 0 leaves the output untouched."""
    import torch
    rng = np.random.default_rng(9)
    H, Hkv, D, bs = 14, 2, 64, 16
    ctx = [0, 1, 40, 300, 513]
    lay = _layout(rng, ctx, bs)
    k = rng.standard_normal((lay.num_blocks, bs, Hkv, D), dtype=np.float32) * 0.5
    v = rng.standard_normal((lay.num_blocks, bs, Hkv, D), dtype=np.float32) * 0.5
    q = rng.standard_normal((len(ctx), H, D), dtype=np.float32) * 0.5
    prior = rng.standard_normal((len(ctx), H, D), dtype=np.float32)
    scale = 0.125
    max_ctx = 257
    ref = oracle.paged_decode(q, k, v, lay.block_tables, lay.context_lens, scale,
                              max_context_len=max_ctx, out=prior.copy())
    out = to_dev(prior, cuda)
    vkv.paged_decode(out, to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                     to_dev(lay.context_lens, cuda), scale, max_context_len=max_ctx, accumulate=True)
    torch.cuda.synchronize()
    got = to_np(out)
    assert np.array_equal(got[0], prior[0])  # ctx 0
    assert_close(got, ref, F32_ATOL, F32_RTOL, "fp32 decode")


# scale 0 weighs every key e^0 = 1 in the reference (the mean of V); each
# kernel family: fixed fp16 D 128 (matrix-core QK^T), fixed D 64 (VALU),
# generic (head_dim 80, group 16), FP8 cache, fp32 reference types.
@pytest.mark.parametrize("H,Hkv,D,bs,io,kv", [(32, 8, 128, 16, "f16", "f16"), (14, 2, 64, 16, "f16", "f16"),
                                              (32, 2, 80, 12, "f16", "f16"), (32, 8, 128, 16, "f16", "fp8"),
                                              (14, 2, 64, 16, "f32", "f32")])
def test_decode_scale_zero(vkv, oracle, cuda, H, Hkv, D, bs, io, kv):
    import torch
    rng = np.random.default_rng(77 + D)
    ctx = [1, 16, 300, 1100]
    lay = _layout(rng, ctx, bs)
    N = lay.num_blocks
    kf = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32)
    vf = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32)
    q = (rng.standard_normal((len(ctx), H, D), dtype=np.float32) * 4).astype(np.float16).astype(np.float32)
    ks = vs = hks = hvs = None
    if kv == "f32":
        hk, hv, kc, vc = kf, vf, to_dev(kf, cuda), to_dev(vf, cuda)
    elif kv == "f16":
        hk, hv = kf.astype(np.float16).view(np.uint16), vf.astype(np.float16).view(np.uint16)
        kc, vc = to_dev(hk.view(np.float16), cuda), to_dev(hv.view(np.float16), cuda)
    else:
        kc = torch.zeros((N, bs, Hkv, D), dtype=torch.uint8, device=cuda)
        vc = torch.zeros_like(kc)
        ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=cuda)
        vs = torch.zeros_like(ks)
        vkv.reshape_and_cache(to_dev(kf.astype(np.float16).reshape(-1, Hkv, D), cuda),
                              to_dev(vf.astype(np.float16).reshape(-1, Hkv, D), cuda), kc, vc,
                              to_dev(np.arange(N * bs, dtype=np.int32), cuda), ks, vs)
        torch.cuda.synchronize()
        hk, hv, hks, hvs = to_np(kc), to_np(vc), to_np(ks), to_np(vs)
    ref = oracle.paged_decode(q, hk, hv, lay.block_tables, lay.context_lens, 0.0, key_scales=hks, value_scales=hvs)
    out = torch.zeros((len(ctx), H, D), dtype=torch.float16 if io == "f16" else torch.float32, device=cuda)
    vkv.paged_decode(out, to_dev(q.astype(np.float16) if io == "f16" else q, cuda), kc, vc,
                     to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda), 0.0, key_scales=ks,
                     value_scales=vs)
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float32)
    assert np.isfinite(got).all()
    tol = (F16_ATOL, F16_RTOL) if io == "f16" else (F32_ATOL, F32_RTOL)
    assert_close(got, ref, *tol, f"scale 0 decode {H}/{Hkv}/{D} {io}/{kv}")


def test_decode_f32_io_f16_kv(vkv, oracle, cuda):
    rng = np.random.default_rng(21)
    ctx = [3, 200, 700]
    lay = _layout(rng, ctx, 16)
    k, v = _pool(rng, lay.num_blocks, 16, 8, 128, 0.3)
    q = rng.standard_normal((3, 32, 128), dtype=np.float32) * 0.3
    scale = 1.0 / np.sqrt(128.0)
    ref = oracle.paged_decode(q, k.view(np.uint16), v.view(np.uint16), lay.block_tables, lay.context_lens, scale)
    got = _run_decode(vkv, cuda, q, k, v, lay, scale, np.float32)
    assert_close(got, ref, F32_ATOL, 1e-3, "fp32-io fp16-kv decode")


def test_decode_config1_golden(vkv, cuda):
    """C1 (Qwen2.5-0.5B layer): append one token per sequence, then decode; compare
    with the committed golden output of the oracle (tests/golden/config1.npz)."""
    import os
    import sys
    import torch
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_config1
    g = np.load(make_config1.PATH)
    inp = make_config1.generate()
    assert make_config1.digest(inp["key_cache"], inp["value_cache"], inp["new_k"], inp["new_v"],
                               inp["query"]) == str(g["inputs_sha256"]), "C1 input generator drifted"
    kc = to_dev(inp["key_cache"], cuda)
    vc = to_dev(inp["value_cache"], cuda)
    vkv.reshape_and_cache(to_dev(inp["new_k"], cuda), to_dev(inp["new_v"], cuda), kc, vc,
                          to_dev(g["slot_mapping"], cuda))
    q = to_dev(inp["query"], cuda)
    out = torch.zeros(q.shape, dtype=torch.float16, device=cuda)
    vkv.paged_decode(out, q, kc, vc, to_dev(g["block_tables"], cuda), to_dev(g["context_lens"], cuda),
                     float(g["scale"]))
    torch.cuda.synchronize()
    assert make_config1.digest(to_np(kc), to_np(vc)) == str(g["after_sha256"])
    assert_close(to_np(out).astype(np.float32), g["output"], F16_ATOL, F16_RTOL, "C1 golden")


def _fp8_case(rng, ctx, H, Hkv, D, bs):
    lay = _layout(rng, ctx, bs)
    N = lay.num_blocks
    k = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32)
    v = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32)
    out_mask = rng.random(k.shape) < 0.01
    k[out_mask] *= 8
    v[rng.random(v.shape) < 0.01] *= 8
    return lay, k.astype(np.float16), v.astype(np.float16)


@pytest.mark.parametrize("H,Hkv,D,bs,ctx", [(32, 8, 128, 16, [1, 130, 600, 2000]), (14, 2, 64, 16, [5, 257]),
                                            (28, 4, 128, 32, [33, 900]),
                                            # kv-head pairs at groups 1-3 and with two kv heads, and an odd
                                            # kv-head count (single kv heads per item)
                                            (8, 8, 128, 16, [17, 800, 3]), (16, 8, 128, 16, [1, 1500]),
                                            (12, 4, 128, 16, [40, 777, 16]), (8, 2, 128, 64, [65, 2100]),
                                            (12, 3, 128, 16, [300, 31])])
def test_decode_fp8(vkv, oracle, cuda, H, Hkv, D, bs, ctx):
    import torch
    rng = np.random.default_rng(4 + D)
    lay, k16, v16 = _fp8_case(rng, ctx, H, Hkv, D, bs)
    N = lay.num_blocks
    q = rng.standard_normal((len(ctx), H, D), dtype=np.float32).astype(np.float16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    # quantise the whole pool with the GPU append (its bit-exactness is tested separately)
    slots = np.arange(N * bs, dtype=np.int32)
    kc = torch.zeros((N, bs, Hkv, D), dtype=torch.uint8, device=cuda)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=cuda)
    vs = torch.zeros_like(ks)
    vkv.reshape_and_cache(to_dev(k16.reshape(-1, Hkv, D), cuda), to_dev(v16.reshape(-1, Hkv, D), cuda),
                          kc, vc, to_dev(slots, cuda), ks, vs)
    torch.cuda.synchronize()
    out = torch.zeros((len(ctx), H, D), dtype=torch.float16, device=cuda)
    vkv.paged_decode(out, to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda),
                     scale, key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float32)
    ref8 = oracle.paged_decode(q.astype(np.float32), to_np(kc), to_np(vc), lay.block_tables, lay.context_lens,
                               scale, key_scales=to_np(ks), value_scales=to_np(vs))
    assert_close(got, ref8, F16_ATOL, F16_RTOL, "fp8 decode vs oracle on the same fp8 cache")
    ref16 = oracle.paged_decode(q.astype(np.float32), k16.view(np.uint16), v16.view(np.uint16), lay.block_tables,
                                lay.context_lens, scale)
    # The quantisation itself: e4m3 keeps 3 mantissa bits and a row's scale follows
    # its largest element (x8 outliers), so against the unquantised fp16 result the
    # per-(seq, head) relative error is a few percent; bound it loosely.
    num = np.linalg.norm(got - ref16, axis=-1)
    den = np.linalg.norm(ref16, axis=-1)
    assert (num <= 0.15 * den + 1e-6).all(), f"fp8 vs fp16 relative error {float((num / den).max()):.4f}"


@pytest.mark.parametrize("D", [128, 64])
def test_decode_fp8_single_key_is_exact(vkv, oracle, cuda, D):
    """ctx 1 with value scale 1: every output element is its e4m3 code's value
    exactly (the weight is 1), so the value path's code-to-fp16 conversion is
    checked for all 254 finite codes (matrix-core variant at D=128, VALU at 64)."""
    import torch
    H, Hkv, bs, S = 32, 8, 16, 3
    G = H // Hkv
    rng = np.random.default_rng(77)
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    N = S + 1
    kc = rng.integers(0, 0x70, (N, bs, Hkv, D), dtype=np.uint8)      # any finite keys
    vc = np.zeros((N, bs, Hkv, D), np.uint8)
    for s in range(S):
        vc[s + 1, 0] = np.resize(rng.permutation(finite), Hkv * D).reshape(Hkv, D)
    ks = np.full((N, bs, Hkv), 0.5, np.float32)
    vs = np.ones((N, bs, Hkv), np.float32)
    bt = np.arange(1, S + 1, dtype=np.int32)[:, None]
    cl = np.ones(S, np.int32)
    q = rng.standard_normal((S, H, D)).astype(np.float16)
    out = torch.zeros((S, H, D), dtype=torch.float16, device=cuda)
    vkv.paged_decode(out, to_dev(q, cuda), to_dev(kc, cuda), to_dev(vc, cuda), to_dev(bt, cuda), to_dev(cl, cuda),
                     float(1.0 / np.sqrt(D)), key_scales=to_dev(ks, cuda), value_scales=to_dev(vs, cuda))
    torch.cuda.synchronize()
    table = np.array([oracle.fp8_decode(int(c)) for c in range(256)], np.float32)
    want = table[vc[1:S + 1, 0]]                                   # [S, Hkv, D]
    want = np.repeat(want, G, axis=1)                               # head h reads kv head h // G
    assert np.array_equal(to_np(out).astype(np.float32), want)


def _c2_inputs(cuda, seed_shift=0):
    import torch
    from vllm_kv_amd import workloads
    cfg = workloads.config2()
    lay = cfg.layout
    S, H, Hkv, D, bs = cfg.num_seqs, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    g = torch.Generator(device=cuda).manual_seed(cfg.seed + seed_shift)
    shape = (lay.num_blocks, bs, Hkv, D)
    kc = (torch.randn(shape, generator=g, device=cuda) * cfg.sigma).half()
    vc = (torch.randn(shape, generator=g, device=cuda) * cfg.sigma).half()
    q = (torch.randn((S, H, D), generator=g, device=cuda) * cfg.sigma).half()
    nk = (torch.randn((S, Hkv, D), generator=g, device=cuda) * cfg.sigma).half()
    nv = (torch.randn((S, Hkv, D), generator=g, device=cuda) * cfg.sigma).half()
    return cfg, kc, vc, q, nk, nv


def test_decode_config2_all_rows(vkv, oracle, cuda):
    """Full C2 (Llama-3-8B shape, B=64, ctx U[512,4096]): append + decode on the GPU;
    every sequence and head is recomputed by the oracle on the whole pool (the
    same block tables); a second decode over a re-permuted pool (same contents,
    other block ids) must give bit-identical output."""
    import torch
    cfg, kc, vc, q, nk, nv = _c2_inputs(cuda)
    lay = cfg.layout
    S = cfg.num_seqs
    slots = to_dev(lay.slots(cfg.prev_lens, np.arange(S)), cuda)
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    vkv.reshape_and_cache(nk, nv, kc, vc, slots)
    out = torch.zeros_like(q)
    vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np(q).astype(np.float32), to_np(kc).view(np.uint16), to_np(vc).view(np.uint16),
                              lay.block_tables, lay.context_lens, cfg.scale, nthreads=_threads())
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, "C2, all 64 sequences")
    # relabel every physical block: contents move, tables follow; output must not change
    perm = torch.from_numpy(np.random.default_rng(77).permutation(lay.num_blocks)).long().to(cuda)
    kc2 = torch.empty_like(kc)
    vc2 = torch.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    bt2 = torch.where(bt >= 0, perm[bt.long().clamp(min=0)], bt.long()).int()
    out2 = torch.zeros_like(out)
    vkv.paged_decode(out2, q, kc2, vc2, bt2, cl, cfg.scale)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def _threads():
    import os
    return max(1, min(16, os.cpu_count() or 1))


def test_decode_concurrent_streams_library_workspace(vkv, cuda):
    """Two streams decode different batches at the same time, both on the
    library's workspace (workspace=None): each output equals its solo run bit
    for bit (the library keeps one workspace per stream)."""
    import torch
    cfg, kc, vc, qa, _, _ = _c2_inputs(cuda)
    _, kc_b, vc_b, qb, _, _ = _c2_inputs(cuda, seed_shift=5)
    lay = cfg.layout
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    solo_a = torch.zeros_like(qa)
    solo_b = torch.zeros_like(qb)
    vkv.paged_decode(solo_a, qa, kc, vc, bt, cl, cfg.scale)
    vkv.paged_decode(solo_b, qb, kc_b, vc_b, bt, cl, cfg.scale)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs_a = [torch.full_like(qa, float("nan")) for _ in range(6)]
    outs_b = [torch.full_like(qb, float("nan")) for _ in range(6)]
    torch.cuda.synchronize()
    for i in range(6):
        vkv.paged_decode(outs_a[i], qa, kc, vc, bt, cl, cfg.scale, stream=s1)
        vkv.paged_decode(outs_b[i], qb, kc_b, vc_b, bt, cl, cfg.scale, stream=s2)
    s1.synchronize()
    s2.synchronize()
    for i in range(6):
        assert torch.equal(outs_a[i].view(torch.int16), solo_a.view(torch.int16)), ("stream 1", i)
        assert torch.equal(outs_b[i].view(torch.int16), solo_b.view(torch.int16)), ("stream 2", i)


def test_decode_per_thread_stream_and_release(vkv, cuda):
    """hipStreamPerThread names a different stream in each thread: two threads
    decoding on it at the same time each get their own library workspace, and
    every output equals its solo run bit for bit.  vkv_release_workspace frees
    a stream's buffers; the next call on that stream allocates afresh and gives
    the same result, and releasing a stream without buffers is a no-op."""
    import threading
    import torch
    cfg, kc, vc, qa, _, _ = _c2_inputs(cuda)
    _, kc_b, vc_b, qb, _, _ = _c2_inputs(cuda, seed_shift=5)
    lay = cfg.layout
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    solo = [torch.zeros_like(qa), torch.zeros_like(qb)]
    vkv.paged_decode(solo[0], qa, kc, vc, bt, cl, cfg.scale)
    vkv.paged_decode(solo[1], qb, kc_b, vc_b, bt, cl, cfg.scale)
    torch.cuda.synchronize()
    outs = [[torch.full_like(qa, float("nan")) for _ in range(6)], [torch.full_like(qb, float("nan")) for _ in range(6)]]
    args = [(qa, kc, vc), (qb, kc_b, vc_b)]
    errors = []
    start = threading.Barrier(2)

    def worker(w):
        try:
            torch.cuda.set_device(cuda)
            q_, k_, v_ = args[w]
            start.wait()
            for i in range(6):
                vkv.paged_decode(outs[w][i], q_, k_, v_, bt, cl, cfg.scale, stream=vkv.STREAM_PER_THREAD)
            torch.cuda.synchronize()
            vkv.release_workspace(vkv.STREAM_PER_THREAD)
        except Exception as e:  # reported below
            errors.append(e)

    torch.cuda.synchronize()  # the fills of outs run on torch's stream
    ths = [threading.Thread(target=worker, args=(w,)) for w in range(2)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    assert not errors, errors
    for w in range(2):
        for i in range(6):
            assert torch.equal(outs[w][i].view(torch.int16), solo[w].view(torch.int16)), ("thread", w, i)
    s1 = torch.cuda.Stream()
    vkv.release_workspace(s1)  # nothing allocated yet
    again = torch.full_like(qa, float("nan"))
    vkv.paged_decode(again, qa, kc, vc, bt, cl, cfg.scale, stream=s1)
    vkv.release_workspace(s1)
    again2 = torch.full_like(qa, float("nan"))
    vkv.paged_decode(again2, qa, kc, vc, bt, cl, cfg.scale, stream=s1)
    s1.synchronize()
    vkv.release_workspace(s1)
    assert torch.equal(again.view(torch.int16), solo[0].view(torch.int16))
    assert torch.equal(again2.view(torch.int16), solo[0].view(torch.int16))


def test_decode_library_workspace_capture_rules(vkv, cuda):
    """A capture that would have to grow the stream's library workspace fails
    with VKV_ERR_WORKSPACE instead of allocating inside the capture; after one
    eager call of that size the same call captures, and the graph replays to
    the eager result with eager calls (and a larger call, which grows the
    buffer again) between the replays."""
    import torch
    cfg, kc, vc, q, _, _ = _c2_inputs(cuda)
    lay = cfg.layout
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    ref = torch.zeros_like(q)
    vkv.paged_decode(ref, q, kc, vc, bt, cl, cfg.scale)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.zeros_like(q)
    err = None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out.zero_()
            try:
                vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=s)
            except vkv.VkvError as e:
                err = e
    assert err is not None and err.code == -4, err
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=s)  # eager: sizes the stream's buffer
    s.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g2, stream=s):
            vkv.paged_decode(out, q, kc, vc, bt, cl, cfg.scale, stream=s)
    torch.cuda.synchronize()
    # a call over longer tables on the same stream grows (and retires) the buffer
    big_bt = torch.full((bt.shape[0], 4 * bt.shape[1]), -1, dtype=torch.int32, device=cuda)
    big_bt[:, :bt.shape[1]] = bt
    for i in range(3):
        out.fill_(float("nan"))
        scratch = torch.zeros_like(out)
        with torch.cuda.stream(s):
            vkv.paged_decode(scratch, q, kc, vc, big_bt if i == 1 else bt, cl, cfg.scale, stream=s)
        s.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), i
        assert torch.equal(scratch.view(torch.int16), ref.view(torch.int16)), i


def test_decode_rows_beyond_one_launch(vkv, oracle, cuda):
    """More sequences than one partition launch holds (8192 rows): the library
    splits the call into consecutive row ranges; every row against the oracle."""
    import torch
    S, H, Hkv, D, bs = 17000, 8, 2, 64, 16
    rng = np.random.default_rng(8)
    ctx = rng.integers(1, 40, size=S).astype(np.int32)
    lay = _layout(rng, ctx, bs)
    k, v = _pool(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    q = (rng.standard_normal((S, H, D), dtype=np.float32) * 0.5).astype(np.float16)
    ref = oracle.paged_decode(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                              lay.context_lens, 0.125, nthreads=_threads())
    got = _run_decode(vkv, cuda, q, k, v, lay, 0.125, np.float16)
    assert_close(got, ref, F16_ATOL, F16_RTOL, "17000 sequences")


@pytest.mark.parametrize("H,Hkv,D", [(8, 8, 64), (32, 8, 128)])
def test_decode_more_groups_than_grid(vkv, oracle, cuda, H, Hkv, D):
    """A batch with many more work groups (4 kv-head items each) than the grid,
    which holds one workgroup per resident slot (at most 8 per CU): the groups
    past the grid are dealt to the workgroups in later rounds (matrix-core
    kernel, D 128) or claimed through the workspace counters (VALU kernel,
    D 64).  Sampled sequences against the oracle; a second call must agree bit
    for bit (the counters return to zero)."""
    import torch
    S, bs, P = 2048, 16, 64
    rng = np.random.default_rng(D + H)
    ctx = rng.integers(150, 260, size=S).astype(np.int32)
    lay = _layout(rng, ctx, bs)
    groups = int(sum((c + P - 1) // P for c in ctx)) * Hkv // 4
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    assert groups > 16 * cus, (groups, cus)
    g = torch.Generator(device=cuda).manual_seed(11)
    shape = (lay.num_blocks, bs, Hkv, D)
    kc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    vc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    q = (torch.randn((S, H, D), generator=g, device=cuda) * 0.5).half()
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    out = torch.zeros((S, H, D), dtype=torch.float16, device=cuda)
    vkv.paged_decode(out, q, kc, vc, bt, cl, scale, partition_size=P)
    out2 = torch.zeros_like(out)
    vkv.paged_decode(out2, q, kc, vc, bt, cl, scale, partition_size=P)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    got = to_np(out).astype(np.float32)
    qn = to_np(q).astype(np.float32)
    for s in [0, 1, 777, 1500, 2046, 2047]:
        n = int(lay.context_lens[s])
        nblk = (n + bs - 1) // bs
        ids = torch.from_numpy(lay.block_tables[s, :nblk]).long().to(cuda)
        kk = to_np(kc[ids]).view(np.uint16)
        vv = to_np(vc[ids]).view(np.uint16)
        ref = oracle.paged_decode(qn[s:s + 1], kk, vv, np.arange(nblk, dtype=np.int32)[None, :],
                                  np.array([n], np.int32), scale)
        assert_close(got[s:s + 1], ref, F16_ATOL, F16_RTOL, f"sequence {s}")


def test_decode_caller_workspace_and_errors(vkv, cuda):
    import torch
    rng = np.random.default_rng(3)
    ctx = [40, 900]
    lay = _layout(rng, ctx, 16)
    k, v = _pool(rng, lay.num_blocks, 16, 2, 64, 0.5)
    q = (rng.standard_normal((2, 4, 64), dtype=np.float32)).astype(np.float16)
    args = (to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
            to_dev(lay.context_lens, cuda), 0.125)
    out_a = torch.zeros((2, 4, 64), dtype=torch.float16, device=cuda)
    vkv.paged_decode(out_a, *args)
    need = vkv.decode_workspace_size(out_a, *args)
    assert need > 0
    ws = torch.zeros(need // 4 + 4, dtype=torch.float32, device=cuda)  # header must start zeroed
    out_b = torch.zeros_like(out_a)
    vkv.paged_decode(out_b, *args, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    small = torch.zeros(16, dtype=torch.float32, device=cuda)
    with pytest.raises(vkv.VkvError) as e:
        vkv.paged_decode(out_b, *args, workspace=small)
    assert e.value.code == -4


def test_decode_default_partition_choice(vkv, oracle, cuda):
    """Partition size left to the library on a batch whose default-size items
    fill between one and two rounds of resident waves (C3's 120 decode rows:
    G = 7, contexts U[1024, 8192]): the kernels pick the size on the device
    and record it in the workspace header (int 1).  The result must equal an
    explicit call at the recorded size bit for bit (same partitions, so the
    merge kernel read the size right), and sampled rows match the oracle."""
    import torch
    from vllm_kv_amd import workloads
    cfg = workloads.config3()
    npf = int((cfg.q_lens > 1).sum())
    lay = cfg.layout
    H, Hkv, D, bs = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    bt = to_dev(np.ascontiguousarray(lay.block_tables[npf:]), cuda)
    cl = to_dev(np.ascontiguousarray(lay.context_lens[npf:]), cuda)
    S = bt.shape[0]
    g = torch.Generator(device=cuda).manual_seed(21)
    shape = (lay.num_blocks, bs, Hkv, D)
    kc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    vc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    q = (torch.randn((S, H, D), generator=g, device=cuda) * 0.5).half()
    scale = cfg.scale
    out = torch.zeros((S, H, D), dtype=torch.float16, device=cuda)
    need = vkv.decode_workspace_size(out, q, kc, vc, bt, cl, scale)
    ws = torch.zeros(need // 4 + 4, dtype=torch.int32, device=cuda)
    vkv.paged_decode(out, q, kc, vc, bt, cl, scale, workspace=ws)
    torch.cuda.synchronize()
    chosen = int(ws[1].item())
    # candidates: 3/4, 7/8, 1, 5/4, 5/3 and 2 x 768 tokens, in 32-token blocks.  On a
    # 256-CU device (1 024 waves per level, 2 048 resident at this group size) 768
    # tokens give 3 216 items (4 levels) and 1 280 tokens 2 044 (2 levels), the least
    # levels x (P + 128) of the six.
    assert int(((cl.cpu().numpy().astype(np.int64) + 1279) // 1280).sum()) * Hkv == 2044
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:
        assert chosen == 1280, chosen
    assert chosen in (576, 672, 768, 960, 1280, 1536), chosen
    out2 = torch.zeros_like(out)
    vkv.paged_decode(out2, q, kc, vc, bt, cl, scale, partition_size=chosen)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), chosen
    got = to_np(out).astype(np.float32)
    qn = to_np(q).astype(np.float32)
    for s in [0, 1, 57, 118, 119]:
        n = int(lay.context_lens[npf + s])
        nblk = (n + bs - 1) // bs
        ids = torch.from_numpy(lay.block_tables[npf + s, :nblk]).long().to(cuda)
        kk = to_np(kc[ids]).view(np.uint16)
        vv = to_np(vc[ids]).view(np.uint16)
        ref = oracle.paged_decode(qn[s:s + 1], kk, vv, np.arange(nblk, dtype=np.int32)[None, :],
                                  np.array([n], np.int32), scale)
        assert_close(got[s:s + 1], ref, F16_ATOL, F16_RTOL, f"row {s} (partition {chosen})")


def test_decode_partition_choice_below_default(vkv, cuda):
    """C2's batch (64 rows, 8 kv heads, contexts U[513, 4097]) gives 1 784
    items at the default 768 tokens: two waves on the busiest SIMDs of a
    256-CU device.  656 tokens keep two (2 016 items, computed from the
    context lengths here) with shorter partitions, so the kernels pick it and
    record it; the output equals an explicit call at that size bit for bit."""
    import torch
    from vllm_kv_amd import workloads
    cfg = workloads.config2()
    lay = cfg.layout
    H, Hkv, D, bs = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    cl_np = np.asarray(lay.context_lens, np.int64)
    assert int(((cl_np + 767) // 768).sum()) * Hkv == 1784
    assert int(((cl_np + 655) // 656).sum()) * Hkv == 2016
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    S = bt.shape[0]
    g = torch.Generator(device=cuda).manual_seed(22)
    shape = (lay.num_blocks, bs, Hkv, D)
    kc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    vc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    q = (torch.randn((S, H, D), generator=g, device=cuda) * 0.5).half()
    scale = float(1.0 / np.sqrt(np.float32(D)))
    out = torch.zeros((S, H, D), dtype=torch.float16, device=cuda)
    need = vkv.decode_workspace_size(out, q, kc, vc, bt, cl, scale)
    ws = torch.zeros(need // 4 + 4, dtype=torch.int32, device=cuda)
    vkv.paged_decode(out, q, kc, vc, bt, cl, scale, workspace=ws)
    torch.cuda.synchronize()
    chosen = int(ws[1].item())
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:
        assert chosen == 656, chosen
    # 3/4, 7/8, 1, 5/4 x 768 and 64 blocks (5/3 and 2 x 768 capped), and 55/64 x 768 in the freed slot
    assert chosen in (576, 656, 672, 768, 960, 1024), chosen
    out2 = torch.zeros_like(out)
    vkv.paged_decode(out2, q, kc, vc, bt, cl, scale, partition_size=chosen)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), chosen


# (rows, context range, kv dtype, the size a 256-CU device picks)
_CHOICE_BATCHES = [
    (64, 1000, 2600, "f16", 576), (64, 512, 4096, "f16", 768), (48, 2000, 4096, "f16", 656),
    (96, 300, 2000, "f16", 576), (64, 2600, 4096, "f16", 960), (64, 2800, 4096, "f16", 1024),
    (64, 1000, 2600, "fp8", 576), (48, 2000, 4096, "fp8", 656), (64, 2600, 4096, "fp8", 960),
]


@pytest.mark.parametrize("idx", range(len(_CHOICE_BATCHES)))
def test_decode_partition_choice_batches(vkv, oracle, cuda, idx):
    """Batches of 48-96 rows (8 kv heads, G = 4, D = 128, 16-token blocks, the
    matrix-core kernels; enough rows that the default stays 768 tokens) whose
    default-size items lie beyond one level of waves and within two rounds,
    so the kernels pick a size among 576, 656, 672, 768, 960 and 1 024
    tokens.  The one they record must give an output bit-identical to an
    explicit call at that size (the merge read the same size).  On a
    256-CU device it must be the least ceil(items / 1 024) x (P + 128), with
    the items counted here from the context lengths.  Two rows are checked
    against the oracle."""
    import torch
    from vllm_kv_amd import workloads
    S, lo, hi, kv, want = _CHOICE_BATCHES[idx]
    H, Hkv, D, bs = 32, 8, 128, 16
    rng = np.random.default_rng(100 + [b[:3] for b in _CHOICE_BATCHES].index((S, lo, hi)))
    ctx = rng.integers(lo, hi + 1, size=S).astype(np.int32)
    lay = workloads.make_layout(ctx, bs, rng, slack=0.05)
    cl_np = lay.context_lens.astype(np.int64)
    cands = (576, 656, 672, 768, 960, 1024)
    items = {c: int(((cl_np + c - 1) // c).sum()) * Hkv for c in cands}
    assert 1024 < items[768] <= 4096  # beyond one level, within two rounds of a 256-CU device
    assert min(cands, key=lambda c: (-(-items[c] // 1024) * (c + 128), c)) == want
    g = torch.Generator(device=cuda).manual_seed(idx)
    shape = (lay.num_blocks, bs, Hkv, D)
    ks = vs = None
    if kv == "fp8":
        kc = torch.empty(shape, dtype=torch.uint8, device=cuda)
        vc = torch.empty_like(kc)
        ks = torch.empty(shape[:3], dtype=torch.float32, device=cuda)
        vs = torch.empty_like(ks)
        x = torch.randn((2, lay.num_blocks * bs, Hkv, D), generator=g, device=cuda).half()
        vkv.reshape_and_cache(x[0], x[1], kc, vc, torch.arange(lay.num_blocks * bs, dtype=torch.int32,
                                                                device=cuda), ks, vs)
        del x
    else:
        kc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
        vc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    q = (torch.randn((S, H, D), generator=g, device=cuda) * 0.5).half()
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    out = torch.zeros((S, H, D), dtype=torch.float16, device=cuda)
    need = vkv.decode_workspace_size(out, q, kc, vc, bt, cl, scale, key_scales=ks, value_scales=vs)
    ws = torch.zeros(need // 4 + 4, dtype=torch.int32, device=cuda)
    vkv.paged_decode(out, q, kc, vc, bt, cl, scale, key_scales=ks, value_scales=vs, workspace=ws)
    torch.cuda.synchronize()
    chosen = int(ws[1].item())
    assert chosen in cands, chosen
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:
        assert chosen == want, (chosen, want)
    out2 = torch.zeros_like(out)
    vkv.paged_decode(out2, q, kc, vc, bt, cl, scale, key_scales=ks, value_scales=vs, partition_size=chosen)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), chosen
    got = to_np(out).astype(np.float32)
    qn = to_np(q).astype(np.float32)
    for s_ in (0, S - 1):
        n = int(lay.context_lens[s_])
        nblk = (n + bs - 1) // bs
        ids = torch.from_numpy(lay.block_tables[s_, :nblk]).long().to(cuda)
        tab = np.arange(nblk, dtype=np.int32)[None, :]
        if kv == "fp8":
            ref = oracle.paged_decode(qn[s_:s_ + 1], to_np(kc[ids]), to_np(vc[ids]), tab, np.array([n], np.int32),
                                      scale, key_scales=to_np(ks[ids]), value_scales=to_np(vs[ids]))
        else:
            ref = oracle.paged_decode(qn[s_:s_ + 1], to_np(kc[ids]).view(np.uint16), to_np(vc[ids]).view(np.uint16),
                                      tab, np.array([n], np.int32), scale)
        assert_close(got[s_:s_ + 1], ref, F16_ATOL, F16_RTOL, f"row {s_} (partition {chosen}, {kv})")


def test_decode_config5_all_rows(vkv, oracle, cuda):
    """Full C5 (Llama-3-8B shape, FP8 e4m3 cache with per-(token, head) scales, B=256,
    lognormal contexts up to 22.6k tokens): the pool, N(0,1) with 1 % of the values
    x8 (the outliers that set the scales), is quantised by the GPU append; one
    decode call covers every sequence (items claimed past the grid), and every
    sequence and head is recomputed by the oracle on the same FP8 codes and scales."""
    import torch
    from vllm_kv_amd import workloads
    cfg = workloads.config5()
    lay = cfg.layout
    S, H, Hkv, D, bs = cfg.num_seqs, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    N = lay.num_blocks
    g = torch.Generator(device=cuda).manual_seed(4)  # the pool and queries bench.py's C5 row draws
    kc = torch.empty((N, bs, Hkv, D), dtype=torch.uint8, device=cuda)
    vc = torch.empty_like(kc)
    ks = torch.empty((N, bs, Hkv), dtype=torch.float32, device=cuda)
    vs = torch.empty_like(ks)
    slots = torch.arange(N * bs, dtype=torch.int32, device=cuda)
    chunk = 1 << 20
    for s0 in range(0, N * bs, chunk):
        n = min(chunk, N * bs - s0)
        x = torch.randn((2, n, Hkv, D), generator=g, device=cuda)
        x = torch.where(torch.rand(x.shape, generator=g, device=cuda) < 0.01, x * 8, x).half()
        vkv.reshape_and_cache(x[0], x[1], kc, vc, slots[s0:s0 + n], ks, vs)
        del x
    q = torch.randn((S, H, D), generator=g, device=cuda).half()
    out = torch.zeros((S, H, D), dtype=torch.float16, device=cuda)
    vkv.paged_decode(out, q, kc, vc, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda), cfg.scale,
                     key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(to_np(q).astype(np.float32), to_np(kc), to_np(vc), lay.block_tables,
                              lay.context_lens, cfg.scale, key_scales=to_np(ks), value_scales=to_np(vs),
                              nthreads=_threads())
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, "C5, all 256 sequences")


@pytest.mark.parametrize("mix", ["mixed", "exact"])
def test_decode_multi_round_claim_order(vkv, oracle, cuda, mix):
    """A call whose items take several rounds of the resident waves, with at
    most 512 rows, claims its items longest first: full partitions, then the
    rows' short final partitions by length class.  480 sequences (H32/Hkv8/D128
    fp16, bs16) whose contexts mix empty rows, exact multiples of the 768-token
    partition (no short partition), single short partitions and long rows
    ("mixed"), or are all exact multiples ("exact": no short partitions at all);
    every sequence and head against the oracle."""
    import torch
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(77 if mix == "mixed" else 78)
    S, H, Hkv, D, bs = 480, 32, 8, 128, 16
    if mix == "mixed":
        kind = rng.integers(0, 4, S)
        ctx = np.where(kind == 0, 0,
              np.where(kind == 1, 768 * rng.integers(1, 5, S),
              np.where(kind == 2, rng.integers(1, 768, S), rng.integers(769, 4000, S)))).astype(np.int32)
    else:
        ctx = (768 * rng.integers(1, 4, S)).astype(np.int32)
    lay = workloads.make_layout(ctx, bs, rng, slack=0.05)
    N = lay.num_blocks
    g = torch.Generator(device=cuda).manual_seed(5)
    kc = (torch.randn((N, bs, Hkv, D), generator=g, device=cuda) * 0.5).half()
    vc = (torch.randn((N, bs, Hkv, D), generator=g, device=cuda) * 0.5).half()
    q = (torch.randn((S, H, D), generator=g, device=cuda) * 0.5).half()
    scale = float(1.0 / np.sqrt(D))
    out = torch.full((S, H, D), float("nan"), dtype=torch.float16, device=cuda)
    vkv.paged_decode(out, q, kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda), scale)
    torch.cuda.synchronize()
    items = int(((ctx.astype(np.int64) + 767) // 768).sum()) * Hkv
    assert items > 3 * 1024, "the call must take more than one round of resident waves"
    ref = oracle.paged_decode(to_np(q).astype(np.float32), to_np(kc).view(np.uint16), to_np(vc).view(np.uint16),
                              lay.block_tables, ctx, scale, nthreads=_threads())
    got = to_np(out).astype(np.float32)
    # (empty rows: zero, as the reference's zeroed output would hold)
    assert_close(got, ref, F16_ATOL, F16_RTOL, f"multi-round claim order ({mix})")
