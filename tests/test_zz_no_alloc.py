"""GPU test of vkv_paged_decode_noalloc, the decode entry point that allocates
nothing (split-K workspace in a fixed device array of the library).

Called through the C ABI (ctypes), its output must equal vkv_paged_decode's on
the same inputs bit for bit (same kernels, same partitions), on two calls in a
row of which the second is smaller, and it must reject a call whose workspace
would exceed the array, leaving the next call correct.
"""
import ctypes

import numpy as np
import pytest

from helpers import to_dev

pytestmark = pytest.mark.gpu


def _inputs(cuda, S, H, Hkv, D, bs, lo, hi, seed, fp8=False):
    import torch
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, size=S).astype(np.int32)
    lay = workloads.make_layout(ctx, bs, rng, slack=0.1)
    g = torch.Generator(device=cuda).manual_seed(seed)
    shape = (lay.num_blocks, bs, Hkv, D)
    q = (torch.randn((S, H, D), generator=g, device=cuda) * 0.5).half()
    ks = vs = None
    if fp8:
        import vllm_kv_amd as vkv
        kc = torch.empty(shape, dtype=torch.uint8, device=cuda)
        vc = torch.empty_like(kc)
        ks = torch.empty(shape[:3], dtype=torch.float32, device=cuda)
        vs = torch.empty_like(ks)
        x = torch.randn((2, lay.num_blocks * bs, Hkv, D), generator=g, device=cuda).half()
        slots = torch.arange(lay.num_blocks * bs, dtype=torch.int32, device=cuda)
        vkv.reshape_and_cache(x[0], x[1], kc, vc, slots, ks, vs)
    else:
        kc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
        vc = (torch.randn(shape, generator=g, device=cuda) * 0.5).half()
    bt = to_dev(lay.block_tables, cuda)
    cl = to_dev(lay.context_lens, cuda)
    return q, kc, vc, bt, cl, ks, vs, float(1.0 / np.sqrt(np.float32(D)))


def _noalloc(vkv, lib, out, q, kc, vc, bt, cl, scale, ks, vs, stream):
    p = vkv.decode_params(out, q, kc, vc, bt, cl, scale, ks, vs)
    return lib.vkv_paged_decode_noalloc(ctypes.byref(p), ctypes.c_void_p(stream.cuda_stream))


def test_noalloc_decode_matches_paged_decode(vkv, cuda):
    import torch
    lib = vkv.load()
    lib.vkv_paged_decode_noalloc.argtypes = [ctypes.POINTER(vkv.DecodeParams), ctypes.c_void_p]
    lib.vkv_paged_decode_noalloc.restype = ctypes.c_int
    stream = torch.cuda.current_stream()
    cases = [
        # C2's shape (matrix-core variant), then a smaller call of another variant
        dict(S=64, H=32, Hkv=8, D=128, bs=16, lo=512, hi=4096, seed=1),
        dict(S=5, H=14, Hkv=2, D=64, bs=16, lo=1, hi=700, seed=2),
        dict(S=40, H=32, Hkv=8, D=128, bs=16, lo=100, hi=3000, seed=3, fp8=True),
        dict(S=3, H=32, Hkv=8, D=128, bs=16, lo=10, hi=300, seed=4),
    ]
    for c in cases:
        q, kc, vc, bt, cl, ks, vs, scale = _inputs(cuda, **c)
        want = torch.zeros_like(q)
        vkv.paged_decode(want, q, kc, vc, bt, cl, scale, key_scales=ks, value_scales=vs)
        got = torch.full_like(q, float("nan"))
        rc = _noalloc(vkv, lib, got, q, kc, vc, bt, cl, scale, ks, vs, stream)
        assert rc == 0, (c, rc, lib.vkv_last_error())
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), c

    # A call whose split-K workspace would exceed the array is refused on the
    # host (256 sequences whose tables allow 64k tokens); the next call is right.
    q, kc, vc, bt, cl, ks, vs, scale = _inputs(cuda, S=256, H=32, Hkv=8, D=128, bs=16, lo=100, hi=200, seed=5)
    big_bt = torch.zeros((256, 4096), dtype=torch.int32, device=cuda)
    big_bt[:, :bt.shape[1]] = bt
    out = torch.zeros_like(q)
    assert _noalloc(vkv, lib, out, q, kc, vc, big_bt, cl, scale, None, None, stream) == -4
    assert b"scratch" in lib.vkv_last_error()
    want = torch.zeros_like(q)
    vkv.paged_decode(want, q, kc, vc, bt, cl, scale)
    assert _noalloc(vkv, lib, out, q, kc, vc, bt, cl, scale, None, None, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
