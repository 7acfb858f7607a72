"""GPU parity of causal chunked-prefill attention.

The reference prefills one token per forward pass (src/core/engine.cpp:157-164),
so query row j of a sequence with q_len rows and ctx keys equals decode over
ctx - q_len + j + 1 keys; the oracle computes exactly that.
"""
import numpy as np
import pytest

from helpers import F16_ATOL, F16_RTOL, assert_close, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,Hkv,D,bs,q_lens,prior", [
    (32, 8, 128, 16, [5, 1, 17], [0, 30, 40]),
    (28, 4, 128, 32, [64, 1, 1, 33], [100, 500, 0, 7]),
    (14, 2, 64, 16, [40], [0]),
])
def test_prefill_vs_oracle(vkv, oracle, cuda, H, Hkv, D, bs, q_lens, prior):
    import torch
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(sum(q_lens) + H)
    q_lens = np.asarray(q_lens, np.int32)
    ctx = np.asarray(prior, np.int32) + q_lens
    lay = workloads.make_layout(ctx, bs, rng, slack=0.2)
    k, v = workloads.fill_pool_numpy(rng, lay.num_blocks, bs, Hkv, D, 0.5)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    Tq = int(qsl[-1])
    q = (rng.standard_normal((Tq, H, D), dtype=np.float32) * 0.5).astype(np.float16)
    scale = float(1.0 / np.sqrt(np.float32(D)))
    ref = oracle.paged_prefill(q.astype(np.float32), k.view(np.uint16), v.view(np.uint16), lay.block_tables,
                               ctx, qsl, scale)
    out = torch.zeros((Tq, H, D), dtype=torch.float16, device=cuda)
    vkv.paged_prefill(out, to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda), to_dev(lay.block_tables, cuda),
                      to_dev(ctx, cuda), to_dev(qsl, cuda), int(q_lens.max()), scale)
    torch.cuda.synchronize()
    assert_close(to_np(out).astype(np.float32), ref, F16_ATOL, F16_RTOL, "prefill")
