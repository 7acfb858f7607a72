"""The generic decode kernel divides token indices by the block size with a
multiplier (vllm-cpp_amd/csrc/decode_common.hpp, block_div / set_block_div):
q = (n + mulhi(n, m)) >> s with s = ceil(log2 d), m = ceil(2^(32+s) / d) - 2^32.
Checked here against integer division for every block size up to 4096 at the
boundaries of every quotient range the kernels can reach, and at random
indices below 2^31 (no GPU)."""
import numpy as np


def _consts(d):
    s = 0
    while (1 << s) < d:
        s += 1
    m = ((1 << (32 + s)) + d - 1) // d
    return m - (1 << 32), s


def _div(n, m, s):
    n = n.astype(np.uint64)
    hi = (n * np.uint64(m)) >> np.uint64(32)
    return ((n + hi) & np.uint64(0xFFFFFFFF)) >> np.uint64(s)


def test_block_div_small_block_sizes_exhaustive_near_multiples():
    for d in range(1, 4097):
        m, s = _consts(d)
        assert 0 <= m < (1 << 32)
        k = np.arange(0, 20000, dtype=np.int64)
        n = np.concatenate([k * d, k * d + d - 1, np.maximum(k * d - 1, 0)])
        n = n[n < (1 << 31)]
        assert np.array_equal(_div(n, m, s), (n // d).astype(np.uint64)), d


def test_block_div_large_indices():
    rng = np.random.default_rng(0)
    for d in list(range(1, 300)) + [1000, 1023, 1024, 1025, 4095, 65535, 65536, 1 << 20]:
        m, s = _consts(d)
        n = rng.integers(0, 1 << 31, 20000, dtype=np.int64)
        top = np.arange((1 << 31) - 5000, 1 << 31, dtype=np.int64)
        n = np.concatenate([n, top, (top // d) * d, (top // d) * d - 1])
        assert np.array_equal(_div(n, m, s), (n // d).astype(np.uint64)), d
