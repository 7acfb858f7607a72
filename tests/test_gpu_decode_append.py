"""vkv_paged_decode_append against the two calls it stands for.

The reference's decode step copies each new token's K/V rows into their slots
and then runs paged attention (src/layers/attention.cpp:81-127).  The library
fuses the append into the decode launches when the shapes allow; the outputs
and both caches must then be bit-identical to vkv_reshape_and_cache followed by
vkv_paged_decode on the same inputs (which the decode tests pin to the oracle).
"""
import numpy as np
import pytest

from helpers import to_dev

pytestmark = pytest.mark.gpu


def _case(rng, H, Hkv, D, bs, prev, extra_blocks=4, sigma=0.5):
    from vllm_kv_amd import workloads
    prev = np.asarray(prev, np.int32)
    ctx = prev + 1
    need = int(sum((c + bs - 1) // bs for c in ctx))
    lay = workloads.make_layout(ctx, bs, rng, num_blocks=need + extra_blocks)
    N = lay.num_blocks
    k = (rng.standard_normal((N, bs, Hkv, D), dtype=np.float32) * sigma).astype(np.float16)
    v = (rng.standard_normal((N, bs, Hkv, D), dtype=np.float32) * sigma).astype(np.float16)
    S = len(prev)
    q = (rng.standard_normal((S, H, D), dtype=np.float32) * sigma).astype(np.float16)
    nk = (rng.standard_normal((S, Hkv, D), dtype=np.float32) * sigma).astype(np.float16)
    nv = (rng.standard_normal((S, Hkv, D), dtype=np.float32) * sigma).astype(np.float16)
    slots = lay.slots(prev, np.arange(S)).astype(np.int32)
    return lay, k, v, q, nk, nv, slots


def _run(vkv, cuda, lay, k, v, q, nk, nv, slots, fused, io=np.float16, accumulate=False, out0=None):
    import torch
    kc, vc = to_dev(k, cuda), to_dev(v, cuda)
    qd = to_dev(q.astype(io), cuda)
    out = to_dev(out0.astype(io), cuda) if out0 is not None else torch.zeros(
        q.shape, dtype=torch.float16 if io == np.float16 else torch.float32, device=cuda)
    bt, cl = to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda)
    nkd, nvd, sd = to_dev(nk, cuda), to_dev(nv, cuda), to_dev(slots, cuda)
    scale = 1.0 / np.sqrt(q.shape[2])
    if fused:
        vkv.paged_decode_append(out, qd, kc, vc, bt, cl, scale, nkd, nvd, sd, accumulate=accumulate)
    else:
        vkv.reshape_and_cache(nkd, nvd, kc, vc, sd)
        vkv.paged_decode(out, qd, kc, vc, bt, cl, scale, accumulate=accumulate)
    torch.cuda.synchronize()
    return out.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy()


def _assert_same(vkv, cuda, case, **kw):
    a = _run(vkv, cuda, *case, fused=False, **kw)
    b = _run(vkv, cuda, *case, fused=True, **kw)
    for x, y, what in zip(a, b, ("output", "key cache", "value cache")):
        assert x.tobytes() == y.tobytes(), f"{what} differs from the two-call sequence"


CASES = [
    # (H, Hkv, D, bs, previous context per sequence): kernels reached
    (32, 8, 128, 16, None),                        # C2's 64 sequences: matrix-core claim loop
    (14, 2, 64, 16, [0, 15, 16, 300]),             # small call: static grid, VALU items at D 64
    (28, 4, 128, 32, [0, 31, 32, 700, 2047]),      # new token opening a block; bs 32
    (16, 8, 256, 8, [8, 64, 519]),                 # D 256, blocks of 8 (VALU items), wave merge of 4 per lane
    (8, 8, 128, 16, list(range(5, 3000, 75))),     # group 1, many partitions per row
    (32, 4, 128, 64, [3, 900, 4000]),              # group 8, blocks larger than a chunk
]


@pytest.mark.parametrize("H,Hkv,D,bs,prev", CASES)
def test_decode_append_matches_two_calls(vkv, cuda, H, Hkv, D, bs, prev):
    rng = np.random.default_rng(H * 100 + D + bs)
    if prev is None:
        from vllm_kv_amd import workloads
        prev = workloads.config2().prev_lens
    _assert_same(vkv, cuda, _case(rng, H, Hkv, D, bs, prev))


@pytest.mark.parametrize("H,Hkv,D,bs,prev", [(32, 8, 128, 16, [4, 299, 1000]), (14, 2, 64, 16, [0, 15, 16, 300]),
                                               (16, 8, 256, 8, [8, 64, 519])])
def test_decode_append_f32_cache(vkv, cuda, H, Hkv, D, bs, prev):
    """The reference's own dtype: fp32 query, rows, cache and output (VALU items)."""
    rng = np.random.default_rng(H + D)
    lay, k, v, q, nk, nv, slots = _case(rng, H, Hkv, D, bs, prev)
    case = (lay, k.astype(np.float32), v.astype(np.float32), q.astype(np.float32), nk.astype(np.float32),
            nv.astype(np.float32), slots)
    _assert_same(vkv, cuda, case, io=np.float32)


def test_decode_append_f32_io_and_accumulate(vkv, cuda):
    """fp32 query / output over the fp16 cache (VALU items), and accumulate = 1."""
    rng = np.random.default_rng(7)
    case = _case(rng, 32, 8, 128, 16, [4, 299, 1000])
    _assert_same(vkv, cuda, case, io=np.float32)
    out0 = rng.standard_normal(case[3].shape).astype(np.float32)
    _assert_same(vkv, cuda, case, accumulate=True, out0=out0)


def test_decode_append_slots_elsewhere(vkv, cuda):
    """A skipped token (slot -1) and a token bound for an unused slot (not the
    sequence's last position): that position reads the cache as it was, as in
    the two calls."""
    rng = np.random.default_rng(11)
    lay, k, v, q, nk, nv, slots = _case(rng, 32, 8, 128, 16, [40, 300, 17, 900], extra_blocks=4)
    used = set(int(b) for b in lay.block_tables.ravel() if b >= 0)
    spare = next(b for b in range(lay.num_blocks) if b not in used)
    slots = slots.copy()
    slots[0] = -1
    slots[2] = spare * 16 + 5
    _assert_same(vkv, cuda, (lay, k, v, q, nk, nv, slots))


def test_decode_append_fp8_cache_runs_both_calls(vkv, cuda):
    """FP8 caches are not fused: the call is the append then the decode."""
    import torch
    rng = np.random.default_rng(13)
    lay, k, v, q, nk, nv, slots = _case(rng, 32, 8, 128, 16, [5, 200, 777])
    N, bs, Hkv, D = k.shape
    res = []
    for fused in (False, True):
        k8 = torch.zeros((N, bs, Hkv, D), dtype=torch.uint8, device=cuda)
        v8 = torch.zeros_like(k8)
        ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=cuda)
        vs = torch.zeros_like(ks)
        all_slots = torch.arange(N * bs, dtype=torch.int32, device=cuda)
        vkv.reshape_and_cache(to_dev(k, cuda).reshape(-1, Hkv, D), to_dev(v, cuda).reshape(-1, Hkv, D), k8, v8,
                              all_slots, ks, vs)
        out = torch.zeros(q.shape, dtype=torch.float16, device=cuda)
        args = (out, to_dev(q, cuda), k8, v8, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda),
                1.0 / np.sqrt(D))
        nkd, nvd, sd = to_dev(nk, cuda), to_dev(nv, cuda), to_dev(slots, cuda)
        if fused:
            vkv.paged_decode_append(*args, nkd, nvd, sd, key_scales=ks, value_scales=vs)
        else:
            vkv.reshape_and_cache(nkd, nvd, k8, v8, sd, ks, vs)
            vkv.paged_decode(*args, key_scales=ks, value_scales=vs)
        torch.cuda.synchronize()
        res.append([t.cpu().numpy().tobytes() for t in (out, k8, v8, ks, vs)])
    assert res[0] == res[1]


@pytest.mark.parametrize("prev", [[100, 50, 300], [100, 50] + list(range(300, 1060, 20))])  # static grid, claim loop
def test_decode_append_is_fused(vkv, cuda, prev):
    """The fused form reads an appended slot from the new rows only at its own
    sequence's last position: a token bound for a slot inside another
    sequence's context (outside what a decode step does) is seen there by the
    two calls but not by the fused call.  So the outputs differ exactly for
    that other sequence, which shows the fused launches ran."""
    rng = np.random.default_rng(17)
    lay, k, v, q, nk, nv, slots = _case(rng, 32, 8, 128, 16, prev)
    slots = slots.copy()
    slots[1] = int(lay.block_tables[0, 2]) * 16 + 3  # position 35 of sequence 0
    a = _run(vkv, cuda, lay, k, v, q, nk, nv, slots, fused=False)
    b = _run(vkv, cuda, lay, k, v, q, nk, nv, slots, fused=True)
    assert a[1].tobytes() == b[1].tobytes() and a[2].tobytes() == b[2].tobytes()
    assert a[0][0].tobytes() != b[0][0].tobytes()          # sequence 0 read the slot before the store
    assert a[0][1:].tobytes() == b[0][1:].tobytes()


def test_decode_append_rows_beyond_one_launch(vkv, cuda):
    """More sequences than one launch takes (consecutive row ranges): the new
    rows and slots follow each range."""
    rng = np.random.default_rng(19)
    prev = rng.integers(0, 40, 8300).astype(np.int32)
    _assert_same(vkv, cuda, _case(rng, 4, 2, 64, 16, prev))


@pytest.mark.parametrize("prev", [[3, 60, 300], [100, 50] + list(range(300, 1060, 20))])  # static grid, claim loop
def test_decode_append_graph_replays(vkv, cuda, prev):
    """The fused call captured in a HIP graph replays to the eager result (the
    append stores the same rows each time), with eager calls on the capture
    stream's library workspace and synchronisations between the replays."""
    import torch
    rng = np.random.default_rng(23)
    lay, k, v, q, nk, nv, slots = _case(rng, 32, 8, 128, 16, prev)
    kc, vc = to_dev(k, cuda), to_dev(v, cuda)
    args = (to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda),
            1.0 / np.sqrt(128), to_dev(nk, cuda), to_dev(nv, cuda), to_dev(slots, cuda))
    out = torch.zeros(q.shape, dtype=torch.float16, device=cuda)
    vkv.paged_decode_append(out, *args)
    torch.cuda.synchronize()
    ref, kref, vref = out.clone(), kc.clone(), vc.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        vkv.paged_decode_append(torch.empty_like(out), *args, stream=s)  # sizes the capture stream's workspace
        with torch.cuda.graph(g, stream=s):
            vkv.paged_decode_append(out, *args, stream=s)
    torch.cuda.synchronize()
    for i in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(s):
            vkv.paged_decode_append(torch.empty_like(out), *args, stream=s)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), i
        assert torch.equal(kref, kc) and torch.equal(vref, vc), i
