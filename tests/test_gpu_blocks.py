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


def _c4_planes(cuda, seed):
    """configs[3]'s pool: 32 layers x (K, V) of [8192, 64, 8, 128] fp16 (random
    bit patterns, carried as int16), 68.7 GB on the device."""
    import torch
    from vllm_kv_amd import workloads
    cfg = workloads.config4()
    shape = (cfg.num_layers, cfg.num_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim)
    g = torch.Generator(device=cuda).manual_seed(seed)
    planes = [torch.empty(shape, dtype=torch.int16, device=cuda) for _ in range(2)]
    for pl in planes:
        for layer in range(cfg.num_layers):
            pl[layer].random_(-32768, 32767, generator=g)
    return cfg, planes


def _block_sums(layer):
    """A position-weighted checksum per block of one layer [N, ...] (int64, wrapping)."""
    import torch
    w = layer.reshape(layer.shape[0], -1).view(torch.int32).long()
    return (w * torch.arange(1, w.shape[1] + 1, device=w.device)).sum(1)


def test_copy_blocks_config4_full(vkv, oracle, cuda):
    """configs[3] copy_blocks at full size: 4096 (src, dst) pairs over 32 layers x
    (K, V) of 128 KiB blocks (68.7 GB moved).  Every destination equals its
    source bit for bit, every other block keeps its checksum, and the blocks of
    the first 64 pairs over all layers equal the oracle's copy of their
    pre-call contents."""
    import torch
    cfg, planes = _c4_planes(cuda, 3)
    L = cfg.num_layers
    pairs = cfg.copy_pairs
    assert vkv.load().vkv_check_block_pairs_host(pairs.ctypes.data, pairs.shape[0], cfg.num_blocks) == 0
    sub = np.unique(pairs[:64].ravel())
    remap = {int(b): i for i, b in enumerate(sub)}
    sub_pairs = np.array([[remap[int(a)], remap[int(b)]] for a, b in pairs[:64]], np.int32)
    sid = torch.from_numpy(sub).long().to(cuda)
    before_sub = [np.ascontiguousarray(to_np(pl[:, sid])) for pl in planes]
    before_sums = [[_block_sums(pl[layer]) for layer in range(L)] for pl in planes]
    vkv.copy_blocks(planes, to_dev(pairs, cuda))
    torch.cuda.synchronize()
    src = torch.from_numpy(pairs[:, 0]).long().to(cuda)
    dst = torch.from_numpy(pairs[:, 1]).long().to(cuda)
    keep = torch.ones(cfg.num_blocks, dtype=torch.bool, device=cuda)
    keep[dst] = False
    for p, pl in enumerate(planes):
        for layer in range(L):
            assert torch.equal(pl[layer][dst], pl[layer][src]), (p, layer)
            after = _block_sums(pl[layer])
            assert torch.equal(after[keep], before_sums[p][layer][keep]), (p, layer)
    oracle.copy_blocks(before_sub, sub_pairs)
    for pl, ref in zip(planes, before_sub):
        assert np.array_equal(to_np(pl[:, sid]), ref)


def test_swap_blocks_config4_full_side_stream(vkv, oracle, cuda):
    """configs[3] swap at full size: 2048 blocks (8 MiB each over 32 layers x K, V)
    swapped out to pinned host memory and back into other device blocks on a
    side stream while decodes run on the default stream.  The round trip is bit
    exact, the host layout of four blocks equals the oracle's, and every decode
    output equals a decode run alone."""
    import torch
    from vllm_kv_amd import workloads
    cfg, planes = _c4_planes(cuda, 4)
    L, N = cfg.num_layers, cfg.num_blocks
    blocks = cfg.swap_blocks
    nsw = int(blocks.shape[0])
    hb = vkv.host_block_bytes(planes)
    assert hb == 2 * L * cfg.block_bytes
    host = torch.empty(nsw * hb, dtype=torch.uint8, pin_memory=True)
    free = np.setdiff1d(np.arange(N, dtype=np.int32), blocks)[:nsw]
    out_pairs = to_dev(np.stack([blocks, np.arange(nsw, dtype=np.int32)], 1), cuda)
    in_pairs = to_dev(np.stack([np.arange(nsw, dtype=np.int32), free], 1), cuda)
    # a decode batch for the default stream (C2's shape)
    c2 = workloads.config2()
    lay = c2.layout
    gq = torch.Generator(device=cuda).manual_seed(9)
    kc = (torch.randn((lay.num_blocks, 16, 8, 128), generator=gq, device=cuda) * 0.3).half()
    vc = (torch.randn((lay.num_blocks, 16, 8, 128), generator=gq, device=cuda) * 0.3).half()
    q = (torch.randn((c2.num_seqs, 32, 128), generator=gq, device=cuda) * 0.3).half()
    bt, cl = to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda)
    solo = torch.zeros_like(q)
    vkv.paged_decode(solo, q, kc, vc, bt, cl, c2.scale)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    outs = [torch.full_like(q, float("nan")) for _ in range(20)]
    vkv.swap_blocks(planes, host, nsw, out_pairs, vkv.SWAP_OUT, stream=side)
    for o in outs[:10]:
        vkv.paged_decode(o, q, kc, vc, bt, cl, c2.scale)
    side.synchronize()
    vkv.swap_blocks(planes, host, nsw, in_pairs, vkv.SWAP_IN, stream=side)
    for o in outs[10:]:
        vkv.paged_decode(o, q, kc, vc, bt, cl, c2.scale)
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o.view(torch.int16), solo.view(torch.int16)), i
    a = torch.from_numpy(blocks).long().to(cuda)
    b = torch.from_numpy(free).long().to(cuda)
    for p, pl in enumerate(planes):
        for layer in range(L):
            assert torch.equal(pl[layer][b], pl[layer][a]), (p, layer)
    # host layout [host block][plane][layer][block bytes] of four blocks vs the oracle
    pick = [0, 1, 777, nsw - 1]
    sub = [np.ascontiguousarray(to_np(pl[:, torch.from_numpy(blocks[pick]).long().to(cuda)])) for pl in planes]
    ref_host = np.zeros(len(pick) * hb, np.uint8)
    oracle.swap_blocks(sub, ref_host, len(pick), np.stack([np.arange(4), np.arange(4)], 1).astype(np.int32), 0)
    got = host.numpy().reshape(nsw, hb)[pick].reshape(-1)
    assert np.array_equal(got, ref_host)
