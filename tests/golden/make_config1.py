"""Writes tests/golden/config1.npz: the C1 golden case (Qwen2.5-0.5B attention layer).

H14 / Hkv2 / D64 fp16, block_size 16, a pool of 256 blocks, 4 sequences with
context U[1,512] (seed 0, workloads.config1()).  Pool contents, the appended
token's K/V and Q are N(0, 0.5) fp16 drawn from numpy default_rng([0, 1]).
One token per sequence is appended through slot_mapping (reshape_and_cache),
then decode attention runs over ctx+1 keys with scale 1/sqrt(64).  The expected
output (fp32) comes from the CPU oracle (oracle/kv_oracle.c), itself pinned by
tests/test_oracle.py.

To stay small the fixture holds the metadata, SHA-256 digests of the generated
inputs and of the caches after the append, and the output; generate() rebuilds
the inputs and the digests catch any drift of the generator.

Run from the repository root after `make -C oracle`:  python tests/golden/make_config1.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for p in (ROOT, os.path.join(ROOT, "vllm-cpp_amd", "python")):
    if p not in sys.path:
        sys.path.insert(0, p)

from vllm_kv_amd import workloads  # noqa: E402

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1.npz")


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def generate():
    """Inputs of the C1 case: dict of fp16 arrays plus the layout."""
    cfg = workloads.config1()
    lay = cfg.layout
    rng = np.random.default_rng([0, 1])
    S, H, Hkv, D, bs = cfg.num_seqs, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.block_size
    kc, vc = workloads.fill_pool_numpy(rng, lay.num_blocks, bs, Hkv, D, cfg.sigma)
    new_k = (rng.standard_normal((S, Hkv, D), dtype=np.float32) * cfg.sigma).astype(np.float16)
    new_v = (rng.standard_normal((S, Hkv, D), dtype=np.float32) * cfg.sigma).astype(np.float16)
    q = (rng.standard_normal((S, H, D), dtype=np.float32) * cfg.sigma).astype(np.float16)
    slots = lay.slots(cfg.prev_lens, np.arange(S))
    return dict(cfg=cfg, key_cache=kc, value_cache=vc, new_k=new_k, new_v=new_v, query=q, slot_mapping=slots)


def main():
    from oracle import oracle
    g = generate()
    cfg, lay = g["cfg"], g["cfg"].layout
    kc_after = g["key_cache"].copy()
    vc_after = g["value_cache"].copy()
    oracle.reshape_and_cache(g["new_k"].view(np.uint16), g["new_v"].view(np.uint16), kc_after.view(np.uint16),
                             vc_after.view(np.uint16), g["slot_mapping"])
    out = oracle.paged_decode(g["query"].astype(np.float32), kc_after.view(np.uint16), vc_after.view(np.uint16),
                              lay.block_tables, lay.context_lens, cfg.scale)
    np.savez_compressed(
        PATH, slot_mapping=g["slot_mapping"], block_tables=lay.block_tables, context_lens=lay.context_lens,
        scale=np.float32(cfg.scale),
        inputs_sha256=digest(g["key_cache"], g["value_cache"], g["new_k"], g["new_v"], g["query"]),
        after_sha256=digest(kc_after, vc_after), output=out)
    print(f"wrote {PATH}: contexts {lay.context_lens.tolist()}, output |max| {np.abs(out).max():.4f}")


if __name__ == "__main__":
    main()
