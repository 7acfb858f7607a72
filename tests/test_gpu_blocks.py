"""GPU parity of copy_blocks and swap_blocks: bit-exact against the oracle's memcpy.

Neither operation exists in the reference; the contract (distinct destinations,
no destination that is also a source, ids outside the pool skipped) is the one
declared in include/vllm_kv_amd.h.
"""
import numpy as np
import pytest

from helpers import to_dev, to_np

pytestmark = pytest.mark.gpu


def _planes(rng, L, N, bs, Hkv, D, fp8):
    if fp8:
        k = rng.integers(0, 256, size=(L, N, bs, Hkv, D), dtype=np.uint8)
        v = rng.integers(0, 256, size=(L, N, bs, Hkv, D), dtype=np.uint8)
        ks = rng.random((L, N, bs, Hkv), dtype=np.float32)
        vs = rng.random((L, N, bs, Hkv), dtype=np.float32)
        return [k, v, ks, vs]
    # fp16 planes carried as int16 bit patterns (torch indexes int16, not uint16)
    k = rng.integers(-(1 << 15), 1 << 15, size=(L, N, bs, Hkv, D), dtype=np.int16)
    v = rng.integers(-(1 << 15), 1 << 15, size=(L, N, bs, Hkv, D), dtype=np.int16)
    return [k, v]


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("L,N,bs,Hkv,D,P", [(3, 40, 16, 2, 64, 13), (2, 24, 64, 8, 128, 9), (1, 300, 8, 1, 64, 100)])
def test_copy_blocks_bitexact(vkv, oracle, cuda, fp8, L, N, bs, Hkv, D, P):
    import torch
    rng = np.random.default_rng(L * 100 + N + P + fp8)
    arrs = _planes(rng, L, N, bs, Hkv, D, fp8)
    ids = rng.permutation(N)
    pairs = np.stack([ids[:P], ids[P:2 * P]], axis=1).astype(np.int32)
    pairs = np.concatenate([pairs, [[N + 3, 0], [0, -1]]]).astype(np.int32)  # out of range: skipped
    dev = [to_dev(a, cuda) for a in arrs]
    ref = [a.copy() for a in arrs]
    oracle.copy_blocks(ref, pairs)
    vkv.copy_blocks(dev, to_dev(pairs, cuda))
    torch.cuda.synchronize()
    for d, r in zip(dev, ref):
        assert np.array_equal(to_np(d).view(np.uint8), r.view(np.uint8))


def test_copy_blocks_host_check(vkv):
    lib = vkv.load()
    ok = np.array([[1, 2], [3, 4]], np.int32)
    assert lib.vkv_check_block_pairs_host(ok.ctypes.data, 2, 8) == 0
    dup = np.array([[1, 2], [3, 2]], np.int32)
    assert lib.vkv_check_block_pairs_host(dup.ctypes.data, 2, 8) == -2
    chain = np.array([[1, 2], [2, 4]], np.int32)
    assert lib.vkv_check_block_pairs_host(chain.ctypes.data, 2, 8) == -2


@pytest.mark.parametrize("fp8", [False, True])
def test_swap_roundtrip_bitexact(vkv, oracle, cuda, fp8):
    import torch
    rng = np.random.default_rng(31 + fp8)
    L, N, bs, Hkv, D = 3, 30, 16, 2, 64
    arrs = _planes(rng, L, N, bs, Hkv, D, fp8)
    dev = [to_dev(a, cuda) for a in arrs]
    hbb = vkv.host_block_bytes(dev)
    assert hbb == sum(a[0, 0].nbytes for a in arrs) * L
    H = 12
    host = torch.zeros(H * hbb, dtype=torch.uint8).pin_memory()
    out_pairs = np.stack([rng.permutation(N)[:H], rng.permutation(H)], axis=1).astype(np.int32)
    # swap out, compare host bytes with the oracle's layout
    vkv.swap_blocks(dev, host, H, to_dev(out_pairs, cuda), vkv.SWAP_OUT)
    torch.cuda.synchronize()
    ref_host = np.zeros(H * hbb, np.uint8)
    oracle.swap_blocks([a.copy() for a in arrs], ref_host, H, out_pairs, 0)
    assert np.array_equal(host.numpy(), ref_host)
    # clobber the device blocks, swap back in, the pool is restored
    for d in dev:
        d[:, torch.from_numpy(out_pairs[:, 0]).long()] = 0
    in_pairs = out_pairs[:, ::-1].copy()
    vkv.swap_blocks(dev, host, H, to_dev(in_pairs, cuda), vkv.SWAP_IN)
    torch.cuda.synchronize()
    for d, a in zip(dev, arrs):
        assert np.array_equal(to_np(d), a)
