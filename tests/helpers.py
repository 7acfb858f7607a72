"""Shared helpers of the test suite (numpy <-> torch, tolerances, random layouts)."""
import numpy as np

# fp16 attention outputs: |gpu - ref| <= ATOL + RTOL*|ref|
F16_ATOL, F16_RTOL = 2e-3, 1e-2
# fp32 path (reference API): fp32 accumulation with hardware exp2, ~1e-6 relative
F32_ATOL, F32_RTOL = 2e-5, 1e-4


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_np(t):
    return t.detach().cpu().numpy()


def assert_close(got, ref, atol, rtol, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        idx = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; worst at {idx}: "
                             f"got {got[idx]!r} ref {ref[idx]!r} (atol {atol}, rtol {rtol})")


def softmax_attention_f64(q, k, v, scale):
    """Textbook softmax(q k^T * scale) v in float64; q [D], k/v [T, D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    if k.shape[0] == 0:
        return np.zeros(q.shape[-1])
    logits = (k @ q) * scale
    w = np.exp(logits - logits.max())
    return (w / w.sum()) @ v


def gather_tokens(cache, table, ctx, bs):
    """K or V rows [ctx, Hkv, D] of one sequence from a [N, bs, Hkv, D] pool."""
    pos = np.arange(ctx)
    return cache[table[pos // bs], pos % bs]
