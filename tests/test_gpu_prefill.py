"""GPU parity of causal chunked-prefill attention.

The reference prefills one token per forward pass (src/core/engine.cpp:157-164),
so query row j of a sequence with q_len rows and ctx keys equals decode over
ctx - q_len + j + 1 keys; the oracle computes exactly that.
"""
import numpy as np
import pytest

from helpers import F16_ATOL, F16_RTOL, assert_close, to_dev, to_np

pytestmark = pytest.mark.gpu


def _case(H, Hkv, D, bs, q_lens, prior, seed):
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(seed)
    q_lens = np.asarray(q_lens, np.int32)
    ctx = np.asarray(prior, np.int32) + q_lens
    lay = workloads.make_layout(ctx, bs, rng, slack=0.2)
    k, v = workloads.fill_pool_numpy(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    Tq = int(qsl[-1])
    q = (rng.standard_normal((Tq, H, D), dtype=np.float32) * 0.5).astype(np.float16)
    return lay, ctx, qsl, q, k, v, float(1.0 / np.sqrt(np.float32(D)))


def _quantise(vkv, cuda, k, v):
    """FP8 cache (codes + per-(slot, head) scales) of fp16 pools [N, bs, Hkv, D],
    quantised by the GPU append; returns device tensors and their host copies."""
    import torch
    N, bs, Hkv, D = k.shape
    kc = torch.zeros((N, bs, Hkv, D), dtype=torch.uint8, device=cuda)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=cuda)
    vs = torch.zeros_like(ks)
    slots = to_dev(np.arange(N * bs, dtype=np.int32), cuda)
    vkv.reshape_and_cache(to_dev(k.reshape(-1, Hkv, D), cuda), to_dev(v.reshape(-1, Hkv, D), cuda), kc, vc, slots,
                          ks, vs)
    torch.cuda.synchronize()
    return (kc, vc, ks, vs), (to_np(kc), to_np(vc), to_np(ks), to_np(vs))


def _cache(vkv, cuda, kvt, k, v):
    """(device K, V, K scales, V scales), (host copies for the oracle) of a pool."""
    if kvt == "f16":
        return (to_dev(k, cuda), to_dev(v, cuda), None, None), (k.view(np.uint16), v.view(np.uint16), None, None)
    return _quantise(vkv, cuda, k, v)


def _threads():
    import os
    return max(1, min(16, os.cpu_count() or 1))


# fp16 queries at head_dim 64/128 run sequences with >= 2 query tokens on the
# matrix-core kernels and single-token ones through split-K decode; each case
# runs over an fp16 cache and over its FP8 quantisation (against the oracle
# on the same codes and scales).
@pytest.mark.parametrize("kvt", ["f16", "fp8"])
@pytest.mark.parametrize("H,Hkv,D,bs,q_lens,prior", [
    (32, 8, 128, 16, [5, 1, 17], [0, 30, 40]),
    (28, 4, 128, 32, [64, 1, 1, 33], [100, 500, 0, 7]),
    (14, 2, 64, 16, [40], [0]),
    (16, 2, 128, 16, [40, 3, 1], [10, 0, 77]),      # group 8
    (8, 8, 64, 8, [70, 2], [9000, 5]),              # MHA; 1131 blocks: FP8 D 64 kernel's 1024-id window reloads
    (8, 8, 64, 8, [40, 3], [17000, 9]),             # 2130 blocks: the wide kernels' 2048-id window refills
    (8, 2, 128, 8, [20, 1], [16500, 40]),           # the same at D 128
    (16, 4, 128, 64, [33, 1, 100], [64, 0, 129]),   # blocks larger than a key tile
    (12, 4, 128, 16, [2, 31, 32, 65], [0, 1, 15, 300]),
    # groups 5 and 6: 256-row work items end inside a token's heads
    (10, 2, 128, 16, [77, 1, 300, 52], [3, 40, 129, 0]),
    (24, 4, 64, 32, [129, 7, 1, 250], [600, 0, 33, 64]),
    # groups above 8 (a token brings G rows to a work item): 16 and 32
    (32, 2, 128, 16, [300, 1, 40], [100, 50, 0]),
    (32, 1, 64, 16, [200, 2], [30, 0]),
])
def test_prefill_vs_oracle(vkv, oracle, cuda, kvt, H, Hkv, D, bs, q_lens, prior):
    """Against the oracle, with the kernels' own work ordering and with the
    host-built work list (vkv_prefill_work_list_host) of the same call."""
    import torch
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, q_lens, prior, sum(q_lens) + H)
    Tq = q.shape[0]
    (kc, vc, ks, vs), (hk, hv, hks, hvs) = _cache(vkv, cuda, kvt, k, v)
    ref = oracle.paged_prefill(q.astype(np.float32), hk, hv, lay.block_tables, ctx, qsl, scale,
                               key_scales=hks, value_scales=hvs, nthreads=_threads())
    args = (to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda), to_dev(qsl, cuda),
            int(max(q_lens)), scale)
    for listed in (False, True):
        out = torch.zeros((Tq, H, D), dtype=torch.float16, device=cuda)
        wl = None
        if listed:
            words = vkv.prefill_work_list(out, *args, qsl, ctx, key_scales=ks, value_scales=vs)
            wl = to_dev(words, cuda) if words.size else None
        vkv.paged_prefill(out, *args, key_scales=ks, value_scales=vs, work_list=wl)
        torch.cuda.synchronize()
        assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL,
                     f"prefill ({kvt} cache, {'host' if listed else 'in-kernel'} work list)")


@pytest.mark.parametrize("kvt", ["f16", "fp8"])
def test_prefill_work_list_relaid(vkv, oracle, cuda, kvt):
    """A host-built schedule re-laid into more lists than the grid has
    workgroups (each workgroup then runs its extra lists in turn), with entries
    the kernels must skip mixed in (a sequence, kv head or row block past the
    call's, a single-token or out-of-range query span): every row still
    matches the oracle."""
    import torch
    H, Hkv, D, bs, q_lens, prior = 28, 4, 128, 32, [300, 1, 200, 64], [100, 500, 0, 7]
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, q_lens, prior, 91)
    Tq = q.shape[0]
    (kc, vc, ks, vs), (hk, hv, hks, hvs) = _cache(vkv, cuda, kvt, k, v)
    ref = oracle.paged_prefill(q.astype(np.float32), hk, hv, lay.block_tables, ctx, qsl, scale,
                               key_scales=hks, value_scales=hvs, nthreads=_threads())
    args = (to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda), to_dev(qsl, cuda),
            int(max(q_lens)), scale)
    out = torch.zeros((Tq, H, D), dtype=torch.float16, device=cuda)
    words = vkv.prefill_work_list(out, *args, qsl, ctx, key_scales=ks, value_scales=vs)
    lists, L = int(words[0]), int(words[1])
    slots = words[32:].reshape(L, lists, 8)
    items = [slots[kk, w].copy() for w in range(lists) for kk in range(L) if slots[kk, w, 0] >= 0]
    assert len(items) == int(words[3])
    bad = [[9, 0, 0, 0, 300, 100, 1, 0],                 # sequence past the call's
           [0, 0, 9, 0, 300, 100, 1, 0],                 # kv head past the call's
           [0, 1 << 24, 0, 0, 300, 100, 1, 0],           # row block past the sequence's rows
           [1, 0, 0, 300, 1, 499, 1, 0],                 # a single query token
           [0, 0, 0, Tq - 10, 300, 100, 1, 0]]           # query rows past the call's
    entries = items + [np.array(e, np.int32) for e in bad]
    W2 = 300  # more lists than the device's CUs
    L2 = (len(entries) + W2 - 1) // W2
    relaid = np.zeros(32 + 8 * W2 * L2, np.int32)
    relaid[:4] = [W2, L2, words[2], len(entries)]
    sl = relaid[32:].reshape(L2, W2, 8)
    sl[:, :, 0] = -1
    for n, e in enumerate(entries):
        sl[n // W2, n % W2] = e
    vkv.paged_prefill(out, *args, key_scales=ks, value_scales=vs, work_list=to_dev(relaid, cuda))
    torch.cuda.synchronize()
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, f"prefill, re-laid list ({kvt} cache)")


@pytest.mark.parametrize("bs", [1, 2])
def test_prefill_small_blocks_vs_oracle(vkv, oracle, cuda, bs):
    """fp16 D = 128 caches with one- and two-token blocks (a direct load's
    four key rows then span blocks: per-lane block ids)."""
    H, Hkv, D = 8, 2, 128
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, [40, 1, 9], [10, 3, 0], 41 + bs)
    import torch
    ref = oracle.paged_prefill(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                               ctx, qsl, scale)
    out = torch.zeros(q.shape, dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                      to_dev(ctx, cuda), to_dev(qsl, cuda), int(np.diff(qsl).max()), scale)
    torch.cuda.synchronize()
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, f"prefill bs{bs}")


@pytest.mark.parametrize("H,Hkv,D,bs", [(28, 4, 128, 32), (16, 2, 64, 16)])  # groups 7 and 8
def test_prefill_fp8_vs_oracle(vkv, oracle, cuda, H, Hkv, D, bs):
    """FP8 cache (quantised by the GPU append): against the oracle on the same codes and scales."""
    import torch
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, [48, 1, 130], [20, 300, 64], 9)
    (kc, vc, ks, vs), (hk, hv, hks, hvs) = _quantise(vkv, cuda, k, v)
    out = torch.zeros((q.shape[0], H, D), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda),
                      to_dev(qsl, cuda), 130, scale, key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    ref = oracle.paged_prefill(q.astype(np.float32), hk, hv, lay.block_tables, ctx, qsl, scale,
                               key_scales=hks, value_scales=hvs)
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, "fp8 prefill")


@pytest.mark.parametrize("kvt", ["f16", "fp8"])
@pytest.mark.parametrize("H,Hkv,D,bs", [(28, 4, 128, 32), (14, 2, 64, 16)])
def test_prefill_scale_zero(vkv, oracle, cuda, kvt, H, Hkv, D, bs):
    """scale 0 (every key weighs e^0 = 1 in the reference: row j is the mean of
    V over its prior + j + 1 keys) on the matrix-core kernels and the decode rows."""
    import torch
    lay, ctx, qsl, q, k, v, _ = _case(H, Hkv, D, bs, [70, 1, 200], [30, 90, 0], 19)
    (kc, vc, ks, vs), (hk, hv, hks, hvs) = _cache(vkv, cuda, kvt, k, v)
    ref = oracle.paged_prefill(q.astype(np.float32), hk, hv, lay.block_tables, ctx, qsl, 0.0,
                               key_scales=hks, value_scales=hvs, nthreads=_threads())
    out = torch.zeros((q.shape[0], H, D), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda),
                      to_dev(qsl, cuda), 200, 0.0, key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float32)
    assert np.isfinite(got).all()
    assert_close(got, ref, F16_ATOL, F16_RTOL, f"scale 0 prefill ({kvt} cache)")


def test_prefill_many_items(vkv, oracle, cuda):
    """More work items than persistent workgroups (items claimed in turn), ragged lengths."""
    import torch
    rng = np.random.default_rng(11)
    S = 24  # ~290 items of 256 (token, head) rows
    q_lens = rng.integers(2, 200, S).tolist()
    prior = rng.integers(0, 300, S).tolist()
    H, Hkv, D, bs = 28, 4, 128, 16
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, q_lens, prior, 5)
    ref = oracle.paged_prefill(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                               ctx, qsl, scale, nthreads=8)
    out = torch.zeros((q.shape[0], H, D), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                      to_dev(ctx, cuda), to_dev(qsl, cuda), int(max(q_lens)), scale)
    torch.cuda.synchronize()
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, "prefill")


@pytest.mark.parametrize("kvt", ["f16", "fp8"])
def test_prefill_mixed_config3(vkv, oracle, cuda, kvt):
    """C3's mixed call at its full size and with its stated inputs (pool and
    queries 0.3 N(0,1) from seed 2, drawn as bench.py's C3 rows draw them):
    8 chunks of 512 query tokens (prior U[0, 2048]) on the matrix-core kernels
    and 120 single-token sequences (contexts U[1024, 8192]) through split-K
    decode with the partition size picked on the device, over an fp16 cache
    and over its FP8 quantisation.  Every one of the 4 216 query rows (4 096
    chunk rows, 120 decode rows) against the oracle, where row j of a chunk is
    decode over prior + j + 1 keys (src/core/engine.cpp:157-164)."""
    import torch
    from vllm_kv_amd import workloads
    cfg = workloads.config3()
    lay = cfg.layout
    H, Hkv, D, bs = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    qsl = cfg.query_start_loc
    Tq = int(qsl[-1])
    g = torch.Generator(device=cuda).manual_seed(2)
    shape = (lay.num_blocks, bs, Hkv, D)
    k16 = (torch.randn(shape, generator=g, device=cuda) * 0.3).half()
    v16 = (torch.randn(shape, generator=g, device=cuda) * 0.3).half()
    q = (torch.randn((Tq, H, D), generator=g, device=cuda) * 0.3).half()
    if kvt == "f16":
        kc, vc, ks, vs = k16, v16, None, None
        hk, hv, hks, hvs = to_np(kc).view(np.uint16), to_np(vc).view(np.uint16), None, None
    else:
        kc = torch.empty(shape, dtype=torch.uint8, device=cuda)
        vc = torch.empty_like(kc)
        ks = torch.empty(shape[:3], dtype=torch.float32, device=cuda)
        vs = torch.empty_like(ks)
        slots = torch.arange(lay.num_blocks * bs, dtype=torch.int32, device=cuda)
        vkv.reshape_and_cache(k16.view(-1, Hkv, D), v16.view(-1, Hkv, D), kc, vc, slots, ks, vs)
        hk, hv, hks, hvs = to_np(kc), to_np(vc), to_np(ks), to_np(vs)
    del k16, v16
    out = torch.zeros((Tq, H, D), dtype=torch.float16, device=cuda)
    args = (q, kc, vc, to_dev(lay.block_tables, cuda), to_dev(lay.context_lens, cuda), to_dev(qsl, cuda),
            int(cfg.q_lens.max()), cfg.scale)
    vkv.paged_prefill(out, *args, key_scales=ks, value_scales=vs)
    # the same call with the host-built work list
    out2 = torch.zeros_like(out)
    words = vkv.prefill_work_list(out2, *args, qsl, lay.context_lens, key_scales=ks, value_scales=vs)
    assert words.size > 0
    vkv.paged_prefill(out2, *args, key_scales=ks, value_scales=vs, work_list=to_dev(words, cuda))
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float32)
    ref = oracle.paged_prefill(to_np(q).astype(np.float32), hk, hv, lay.block_tables, lay.context_lens, qsl,
                               cfg.scale, key_scales=hks, value_scales=hvs, nthreads=_threads())
    npf = int((cfg.q_lens > 1).sum())
    assert int(qsl[npf]) == 4096 and Tq == 4216
    assert_close(got, ref, F16_ATOL, F16_RTOL, f"C3 ({kvt} cache): all 4096 chunk rows and 120 decode rows")
    # the work list changes the order of the items, not a single result bit
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


@pytest.mark.parametrize("kvt", ["f16", "fp8"])
def test_prefill_large_call_list_kernel(vkv, oracle, cuda, kvt):
    """A call with more row blocks than the fp16 kernel orders in LDS (here 720
    blocks of 256 (token, head) rows, 80 sequences of 300 tokens at group 7):
    the separate list kernel builds the longest-first order (the FP8 kernel
    always uses it).  Sampled rows against the oracle (row j of a sequence is
    decode over prior + j + 1 keys), on the same codes and scales for FP8."""
    import torch
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(17)
    H, Hkv, D, bs, S, qn_ = 28, 4, 128, 16, 80, 300
    q_lens = np.full(S, qn_, np.int32)
    prior = rng.integers(0, 700, S).astype(np.int32)
    ctx = prior + q_lens
    lay = workloads.make_layout(ctx, bs, rng, slack=0.1)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    Tq = int(qsl[-1])
    k, v = workloads.fill_pool_numpy(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    (kc, vc, ks, vs), (hk, hv, hks, hvs) = _cache(vkv, cuda, kvt, k, v)
    q = (rng.standard_normal((Tq, H, D), dtype=np.float32) * 0.5).astype(np.float16)
    out = torch.zeros((Tq, H, D), dtype=torch.float16, device=cuda)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    vkv.paged_prefill(out, to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda),
                      to_dev(qsl, cuda), qn_, scale, key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float32)
    seqs = [0, 31, 79, int(np.argmax(prior))]
    rows = np.concatenate([np.arange(qsl[s], qsl[s + 1]) for s in seqs])
    sub_qsl = np.concatenate([[0], np.cumsum([qsl[s + 1] - qsl[s] for s in seqs])]).astype(np.int32)
    ref = oracle.paged_prefill(q[rows].astype(np.float32), hk, hv, np.ascontiguousarray(lay.block_tables[seqs]),
                               np.ascontiguousarray(ctx[seqs]), sub_qsl, scale, key_scales=hks, value_scales=hvs,
                               nthreads=_threads())
    assert_close(got[rows], ref, F16_ATOL, F16_RTOL, f"720-block call ({kvt} cache), every row of 4 sequences")


def _mixed_inputs(cuda):
    import torch
    rng = np.random.default_rng(31)
    H, Hkv, D, bs = 28, 4, 128, 32
    q_lens = [300, 1, 1, 77, 1, 1, 1, 200] + [1] * 40
    prior = rng.integers(0, 3000, len(q_lens)).tolist()
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, q_lens, prior, 9)
    args = [to_dev(x, cuda) for x in (q, k, v, lay.block_tables, ctx, qsl)]
    out = torch.zeros((q.shape[0], H, D), dtype=torch.float16, device=cuda)
    return out, args, int(max(q_lens)), scale


def test_prefill_mixed_on_caller_stream(vkv, cuda):
    """A mixed call (matrix-core rows and single-token decode rows) issued on a
    non-default stream: after synchronising only that stream the output is
    complete and equals a call on the default stream bit for bit."""
    import torch
    out, args, mql, scale = _mixed_inputs(cuda)
    vkv.paged_prefill(out, *args, mql, scale)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    for _ in range(3):
        out2 = torch.full_like(out, float("nan"))
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            vkv.paged_prefill(out2, *args, mql, scale, stream=s)
            out2.record_stream(s)
        s.synchronize()
        assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def test_prefill_mixed_graph_replays(vkv, cuda):
    """A mixed call captured in a graph (work-list, prefill, decode and merge
    kernels; the claim counters are reset by kernels, not memsets) replays to
    the eager result, with eager calls on the capture stream's library
    workspace and synchronisations between the replays.  The capture stream's
    workspace is sized by one eager call first (it cannot grow under capture)."""
    import torch
    out, args, mql, scale = _mixed_inputs(cuda)
    vkv.paged_prefill(out, *args, mql, scale)
    torch.cuda.synchronize()
    ref = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        vkv.paged_prefill(torch.empty_like(out), *args, mql, scale, stream=s)
        out.zero_()
        with torch.cuda.graph(g, stream=s):
            vkv.paged_prefill(out, *args, mql, scale, stream=s)
    torch.cuda.synchronize()
    for i in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(s):
            vkv.paged_prefill(torch.empty_like(out), *args, mql, scale, stream=s)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), i


def test_prefill_context_shorter_than_chunk(vkv, oracle, cuda):
    """context_lens below q_len (invalid input): rows whose position sees no key
    are zeros, the others attend the keys there are, and nothing is read out of
    range (the second sequence's items have no keys at all)."""
    import torch
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(17)
    H, Hkv, D, bs = 28, 4, 128, 16
    q_lens = np.array([40, 33, 5], np.int32)
    ctx = np.array([10, 0, 60], np.int32)  # prior -30, -33, 55
    lay = workloads.make_layout(np.maximum(ctx, 1), bs, rng, slack=0.2)
    k, v = workloads.fill_pool_numpy(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = (rng.standard_normal((int(qsl[-1]), H, D), dtype=np.float32) * 0.5).astype(np.float16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    ref = oracle.paged_prefill(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                               ctx, qsl, scale)
    assert not ref[:29].any() and not ref[40:73].any()  # no key before position 0
    out = torch.full((q.shape[0], H, D), 7.0, dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                      to_dev(ctx, cuda), to_dev(qsl, cuda), int(q_lens.max()), scale)
    torch.cuda.synchronize()
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, "prefill")


def test_prefill_f32_rows(vkv, oracle, cuda):
    """fp32 queries take the per-row decode path (reference precision)."""
    import torch
    from helpers import F32_ATOL, F32_RTOL
    H, Hkv, D, bs = 8, 2, 64, 16
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, [9, 1, 20], [3, 40, 0], 21)
    q32 = q.astype(np.float32)
    ref = oracle.paged_prefill(q32, k.view(np.uint16), v.view(np.uint16), lay.block_tables, ctx, qsl, scale)
    out = torch.zeros((q.shape[0], H, D), dtype=torch.float32, device=cuda)
    vkv.paged_prefill(out, to_dev(q32, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                      to_dev(ctx, cuda), to_dev(qsl, cuda), 20, scale)
    torch.cuda.synchronize()
    assert_close(to_np(out), ref, F32_ATOL, F32_RTOL, "fp32 prefill")


@pytest.mark.parametrize("kvt", ["f16", "fp8"])
def test_prefill_growing_logits(vkv, oracle, cuda, kvt):
    """Large logits whose running maximum keeps growing along the keys (key norms
    ramp up with position): every rescale of the online softmax, and the
    cross-lane row maximum, must be right for the weights to stay finite."""
    import torch
    rng = np.random.default_rng(31)
    H, Hkv, D, bs = 28, 4, 128, 16
    q_lens = np.array([96, 40], np.int32)
    prior = np.array([700, 130], np.int32)
    ctx = prior + q_lens
    from vllm_kv_amd import workloads
    lay = workloads.make_layout(ctx, bs, rng, slack=0.2)
    N = lay.num_blocks
    k = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32)
    v = rng.standard_normal((N, bs, Hkv, D), dtype=np.float32)
    # key norm grows with the token's position in its sequence: logits up to ~150
    for s in range(len(ctx)):
        for t in range(int(ctx[s])):
            blk = lay.block_tables[s, t // bs]
            k[blk, t % bs] *= 0.2 + 2.5 * t / int(ctx[s])
    k, v = k.astype(np.float16), v.astype(np.float16)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = rng.standard_normal((int(qsl[-1]), H, D)).astype(np.float16)
    scale = 0.35
    tq = to_dev(q, cuda)
    if kvt == "f16":
        kc, vc, ks, vs = to_dev(k, cuda), to_dev(v, cuda), None, None
        hk, hv, hks, hvs = k.view(np.uint16), v.view(np.uint16), None, None
    else:
        kc = torch.zeros((N, bs, Hkv, D), dtype=torch.uint8, device=cuda)
        vc = torch.zeros_like(kc)
        ks = torch.zeros((N, bs, Hkv), dtype=torch.float32, device=cuda)
        vs = torch.zeros_like(ks)
        slots = to_dev(np.arange(N * bs, dtype=np.int32), cuda)
        vkv.reshape_and_cache(to_dev(k.reshape(-1, Hkv, D), cuda), to_dev(v.reshape(-1, Hkv, D), cuda), kc, vc,
                              slots, ks, vs)
        torch.cuda.synchronize()
        hk, hv, hks, hvs = to_np(kc), to_np(vc), to_np(ks), to_np(vs)
    out = torch.zeros((q.shape[0], H, D), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, tq, kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda), to_dev(qsl, cuda),
                      int(q_lens.max()), scale, key_scales=ks, value_scales=vs)
    torch.cuda.synchronize()
    ref = oracle.paged_prefill(q.astype(np.float32), hk, hv, lay.block_tables, ctx, qsl, scale,
                               key_scales=hks, value_scales=hvs)
    got = to_np(out).astype(np.float32)
    assert np.isfinite(got).all()
    if kvt == "f16":
        assert_close(got, ref, F16_ATOL, F16_RTOL, "prefill with growing logits")
    else:
        # The kernel stages dequantised keys as fp16 (2^-12 relative), which at
        # logits near 50 moves single weights by about 1 %: held to the FP8
        # contract (3e-2 relative) per output row instead of element-wise.
        err = np.linalg.norm(got - ref, axis=-1) / np.maximum(np.linalg.norm(ref, axis=-1), 1e-6)
        assert err.max() <= 3e-2, f"FP8 prefill with growing logits: row error {err.max():.3e}"


def test_prefill_caller_workspace(vkv, cuda):
    """A caller workspace of vkv_paged_prefill_workspace_size() bytes (header
    zeroed) gives the library workspace's result bit for bit, twice in a row."""
    import torch
    out, args, mql, scale = _mixed_inputs(cuda)
    vkv.paged_prefill(out, *args, mql, scale)
    need = vkv.prefill_workspace_size(out, *args, mql, scale)
    assert need > 1024
    ws = torch.zeros(need // 4 + 4, dtype=torch.int32, device=cuda)
    for _ in range(2):
        out2 = torch.full_like(out, float("nan"))
        vkv.paged_prefill(out2, *args, mql, scale, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    small = torch.zeros(64, dtype=torch.int32, device=cuda)
    with pytest.raises(vkv.VkvError) as e:
        vkv.paged_prefill(out, *args, mql, scale, workspace=small)
    assert e.value.code == -4


@pytest.mark.parametrize("io", ["f16", "f32"])
def test_prefill_max_context_len_clamp(vkv, oracle, cuda, io):
    """max_context_len clamps every row's key count as decode does (the
    reference's min(ctx, max_context_len), paged_attention.cu:20): row j of a
    sequence attends keys 0 .. min(prior + j + 1, max_context_len) - 1, on the
    matrix-core path (fp16) and the per-row decode path (fp32), with the
    single-token rows of the call clamped the same way."""
    import torch
    from helpers import F32_ATOL, F32_RTOL
    H, Hkv, D, bs = 28, 4, 128, 16
    q_lens, prior = [100, 1, 60, 1], [150, 300, 20, 40]
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, q_lens, prior, 77)
    max_ctx = 180
    # per-row reference: each query row is a decode over its clamped causal context
    seq_of = np.repeat(np.arange(len(q_lens)), q_lens)
    j = np.arange(q.shape[0]) - qsl[seq_of]
    row_ctx = np.asarray(prior)[seq_of] + j + 1
    qf = q.astype(np.float32)
    ref = oracle.paged_decode(qf, k.view(np.uint16), v.view(np.uint16),
                              np.ascontiguousarray(lay.block_tables[seq_of]), row_ctx.astype(np.int32), scale,
                              max_context_len=max_ctx)
    if io == "f16":
        qd, out = to_dev(q, cuda), torch.zeros((q.shape[0], H, D), dtype=torch.float16, device=cuda)
        tol = (F16_ATOL, F16_RTOL)
    else:
        qd, out = to_dev(qf, cuda), torch.zeros((q.shape[0], H, D), dtype=torch.float32, device=cuda)
        tol = (F32_ATOL, 1e-3)
    vkv.paged_prefill(out, qd, to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda), to_dev(ctx, cuda),
                      to_dev(qsl, cuda), max(q_lens), scale, max_context_len=max_ctx)
    torch.cuda.synchronize()
    assert_close(to_np(out).astype(np.float32), ref, *tol, f"prefill clamped to {max_ctx} keys ({io})")


def test_prefill_group16_list_kernel(vkv, oracle, cuda):
    """Group 16 in a call large enough for the separate list kernel (more than
    512 row blocks): each sequence brings ceil(q G / 256) row blocks per kv
    head, twice what one per 32 query tokens would allow, and the work list
    must hold them all.  Every row of three sequences against the oracle."""
    import torch
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(29)
    H, Hkv, D, bs, S, qn_ = 16, 1, 128, 16, 24, 360
    q_lens = np.full(S, qn_, np.int32)
    prior = rng.integers(0, 200, S).astype(np.int32)
    ctx = prior + q_lens
    lay = workloads.make_layout(ctx, bs, rng, slack=0.1)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    Tq = int(qsl[-1])
    assert Tq * (H // Hkv) // 256 > 512  # the list-kernel path
    k, v = workloads.fill_pool_numpy(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    q = (rng.standard_normal((Tq, H, D), dtype=np.float32) * 0.5).astype(np.float16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    out = torch.zeros((Tq, H, D), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                      to_dev(ctx, cuda), to_dev(qsl, cuda), qn_, scale)
    torch.cuda.synchronize()
    got = to_np(out).astype(np.float32)
    seqs = [0, 11, S - 1]
    rows = np.concatenate([np.arange(qsl[s], qsl[s + 1]) for s in seqs])
    sub_qsl = np.concatenate([[0], np.cumsum([qsl[s + 1] - qsl[s] for s in seqs])]).astype(np.int32)
    ref = oracle.paged_prefill(q[rows].astype(np.float32), k.view(np.uint16), v.view(np.uint16),
                               np.ascontiguousarray(lay.block_tables[seqs]), np.ascontiguousarray(ctx[seqs]), sub_qsl,
                               scale, nthreads=_threads())
    assert_close(got[rows], ref, F16_ATOL, F16_RTOL, "group-16 prefill through the list kernel")


@pytest.mark.parametrize("kvt", ["f16", "fp8"])
def test_prefill_multi_token_only(vkv, oracle, cuda, kvt):
    """multi_token_only = 1 (no sequence has one query token) skips the decode
    pass: on such a batch the output equals the default call's bit for bit and
    the oracle's; a mixed call on the same workspace afterwards is still right
    (the skipped pass leaves no counter behind)."""
    import torch
    H, Hkv, D, bs = 28, 4, 128, 16
    lay, ctx, qsl, q, k, v, scale = _case(H, Hkv, D, bs, [40, 3, 77, 2], [100, 0, 513, 31], 200)
    (kc, vc, ks, vs), (hk, hv, hks, hvs) = _cache(vkv, cuda, kvt, k, v)
    args = (to_dev(q, cuda), kc, vc, to_dev(lay.block_tables, cuda), to_dev(ctx, cuda), to_dev(qsl, cuda), 77, scale)
    out_a = torch.full((q.shape[0], H, D), float("nan"), dtype=torch.float16, device=cuda)
    out_b = torch.full_like(out_a, float("nan"))
    vkv.paged_prefill(out_a, *args, key_scales=ks, value_scales=vs)
    vkv.paged_prefill(out_b, *args, key_scales=ks, value_scales=vs, multi_token_only=True)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
    ref = oracle.paged_prefill(q.astype(np.float32), hk, hv, lay.block_tables, ctx, qsl, scale,
                               key_scales=hks, value_scales=hvs, nthreads=_threads())
    assert_close(to_np(out_b).astype(np.float32), ref, F16_ATOL, F16_RTOL, f"multi-token-only prefill ({kvt})")
    # then a mixed call (single-token sequences among them) on the same library workspace
    lay2, ctx2, qsl2, q2, k2, v2, _ = _case(H, Hkv, D, bs, [1, 30, 1, 1], [300, 7, 0, 900], 200)
    (kc2, vc2, ks2, vs2), (hk2, hv2, hks2, hvs2) = _cache(vkv, cuda, kvt, k2, v2)
    out_c = torch.full((q2.shape[0], H, D), float("nan"), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out_c, to_dev(q2, cuda), kc2, vc2, to_dev(lay2.block_tables, cuda), to_dev(ctx2, cuda),
                      to_dev(qsl2, cuda), 30, scale, key_scales=ks2, value_scales=vs2)
    torch.cuda.synchronize()
    ref2 = oracle.paged_prefill(q2.astype(np.float32), hk2, hv2, lay2.block_tables, ctx2, qsl2, scale,
                                key_scales=hks2, value_scales=hvs2, nthreads=_threads())
    assert_close(to_np(out_c).astype(np.float32), ref2, F16_ATOL, F16_RTOL, f"mixed prefill after ({kvt})")
