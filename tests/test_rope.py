"""RoPE and the fused RoPE + KV append.

CPU tests pin the oracle's rope (oracle/kv_oracle.c, restating
src/kernels/rotary_embedding.cu:13-34) against a float64 numpy rotation with
the reference's pairing (d, d + D/2), position 0 = identity and preserved pair
norms; and the library's host table builder against the formula of
src/model/qwen.cpp:119-128 evaluated in float64.

GPU tests compare vkv_rope_reshape_and_cache with the oracle composition
rope (in place) followed by reshape_and_cache, bit for bit: the rotated
queries, the cache bytes and the FP8 scales.
"""
import numpy as np
import pytest

from helpers import to_dev, to_np


def rope_f64(x, cos_sin, pos):
    """x [T, heads, D] -> rotated in float64 (pairs d, d + D/2)."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    half = D // 2
    c = cos_sin[pos, :, 0].astype(np.float64)[:, None, :]
    s = cos_sin[pos, :, 1].astype(np.float64)[:, None, :]
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


def table_f64(theta, D, P):
    """qwen.cpp:121-127 in float64: (cos f, sin f) with f = pos / theta^(2d/D), and f itself."""
    d = np.arange(D // 2, dtype=np.float64)
    f = np.arange(P, dtype=np.float64)[:, None] / np.power(float(theta), 2.0 * d / D)[None, :]
    return np.stack([np.cos(f), np.sin(f)], axis=-1), f


def random_table(rng, P, D):
    ang = rng.random((P, D // 2)) * 2 * np.pi
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


# ---------------------------------------------------------------- oracle pinning (CPU)

@pytest.mark.parametrize("D", [64, 128])
def test_oracle_rope_vs_f64(oracle, D):
    rng = np.random.default_rng(5)
    T, H, Hkv, P = 9, 6, 2, 40
    cs = random_table(rng, P, D)
    pos = rng.integers(0, P, T).astype(np.int32)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    rq, rk = rope_f64(q, cs, pos), rope_f64(k, cs, pos)
    oracle.rope(q, k, cs, positions=pos)
    # one fma over one rounded product: within 2 ulp of the fp32 result scale
    assert (np.abs(q - rq) <= 3e-7 * (np.abs(rq) + 1.0)).all()
    assert (np.abs(k - rk) <= 3e-7 * (np.abs(rk) + 1.0)).all()


def test_oracle_rope_identity_and_norm(oracle):
    rng = np.random.default_rng(6)
    T, H, Hkv, D, P = 4, 3, 1, 64, 8
    cs = random_table(rng, P, D)
    cs[0, :, 0], cs[0, :, 1] = 1.0, 0.0  # position 0 of any real table
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    oracle.rope(q, k, cs, positions=np.zeros(T, np.int32))
    assert np.array_equal(q, q0) and np.array_equal(k, k0)
    oracle.rope(q, k, cs, start_pos=3)  # positions 3..6
    half = D // 2
    n_before = q0[..., :half] ** 2 + q0[..., half:] ** 2
    n_after = q[..., :half] ** 2 + q[..., half:] ** 2
    assert np.allclose(n_after, n_before, rtol=2e-6, atol=1e-6)
    assert not np.array_equal(q, q0)


def test_oracle_rope_f16_rounds_once(oracle):
    rng = np.random.default_rng(7)
    T, H, Hkv, D, P = 5, 4, 2, 128, 16
    cs = random_table(rng, P, D)
    q = (rng.standard_normal((T, H, D)) * 0.5).astype(np.float16)
    k = (rng.standard_normal((T, Hkv, D)) * 0.5).astype(np.float16)
    pos = np.arange(T, dtype=np.int32) + 7
    rq = rope_f64(q.astype(np.float32), cs, pos)
    qb = q.view(np.uint16).copy()
    kb = k.view(np.uint16).copy()
    oracle.rope(qb, kb, cs, positions=pos)
    got = qb.view(np.float16).astype(np.float64)
    # fp16 result of an fp32 rotation: within half an fp16 ulp plus the fp32 error
    assert (np.abs(got - rq) <= np.abs(rq) * 2.0 ** -11 + 2.0 ** -24 + 1e-6).all()


def test_host_cos_sin_table(vkv):
    theta, D, P = 10000.0, 64, 4096
    got = vkv.rope_cos_sin_host(theta, D, P)
    ref, f = table_f64(theta, D, P)
    assert got.shape == (P, D // 2, 2)
    # the reference evaluates f in fp32 (powf, then one division): a few ulp of f
    # move cos/sin by at most that much; the functions themselves add < 1e-7
    tol = 4.0 * np.spacing(f.astype(np.float32)).astype(np.float64) + 2e-7
    assert (np.abs(got - ref) <= tol[..., None]).all()
    assert np.array_equal(got[0, :, 0], np.ones(D // 2, np.float32)) and not got[0, :, 1].any()


# ---------------------------------------------------------------- GPU parity

CASES = [  # (H, Hkv, D, src, cache)
    (14, 2, 64, np.float16, "f16"),
    (32, 8, 128, np.float16, "f16"),
    (28, 4, 128, np.float16, "fp8"),
    (8, 2, 256, np.float16, "f16"),
    (8, 2, 64, np.float32, "f32"),
    (16, 4, 128, np.float32, "f16"),
    (14, 2, 64, np.float32, "fp8"),
    (4, 1, 256, np.float16, "fp8"),
]


def _inputs(rng, T, H, Hkv, D, src):
    q = (rng.standard_normal((T, H, D)) * 0.7).astype(src)
    k = (rng.standard_normal((T, Hkv, D)) * 0.7).astype(src)
    v = (rng.standard_normal((T, Hkv, D)) * 0.7).astype(src)
    if src == np.float16:
        k[0, 0, :] = 0  # an all-zero key head (FP8 scale rule)
    return q, k, v


def _bits(a):
    """fp16 arrays as their uint16 bits (the oracle's fp16 currency); others unchanged."""
    return a.view(np.uint16) if a.dtype == np.float16 else a


@pytest.mark.gpu
@pytest.mark.parametrize("H,Hkv,D,src,cache", CASES)
def test_fused_rope_append_bit_exact(vkv, oracle, cuda, H, Hkv, D, src, cache):
    import torch
    rng = np.random.default_rng(H * 1000 + D)
    T, N, bs, P = 37, 16, 16, 300
    q, k, v = _inputs(rng, T, H, Hkv, D, src)
    cs = random_table(rng, P, D)
    pos = rng.integers(0, P, T).astype(np.int32)
    slots = rng.permutation(N * bs)[:T].astype(np.int32)
    slots[3] = -1  # padding token: nothing stored
    cdt = {"f32": np.float32, "f16": np.float16, "fp8": np.uint8}[cache]
    kc = rng.integers(0, 255, (N, bs, Hkv, D * np.dtype(cdt).itemsize), dtype=np.uint8).view(cdt).copy()
    vc = rng.integers(0, 255, (N, bs, Hkv, D * np.dtype(cdt).itemsize), dtype=np.uint8).view(cdt).copy()
    ks = vs = None
    if cache == "fp8":
        ks = np.full((N, bs, Hkv), -1.0, np.float32)
        vs = np.full((N, bs, Hkv), -1.0, np.float32)
    print(f"case H{H} Hkv{Hkv} D{D} src {np.dtype(src).name} cache {cache}", flush=True)

    tq, tk, tv = to_dev(q, cuda), to_dev(k, cuda), to_dev(v, cuda)
    tkc, tvc = to_dev(kc, cuda), to_dev(vc, cuda)
    tks = None if ks is None else to_dev(ks, cuda)
    tvs = None if vs is None else to_dev(vs, cuda)
    vkv.rope_reshape_and_cache(tq, tk, tv, to_dev(cs, cuda), positions=to_dev(pos, cuda), key_cache=tkc,
                               value_cache=tvc, slot_mapping=to_dev(slots, cuda), key_scales=tks,
                               value_scales=tvs)
    torch.cuda.synchronize()

    oq, ok = _bits(q.copy()), _bits(k.copy())
    oracle.rope(oq, ok, cs, positions=pos)
    okc, ovc = _bits(kc.copy()), _bits(vc.copy())
    oracle.reshape_and_cache(ok, _bits(v), okc, ovc, slots, ks, vs)

    raw = lambda a: np.ascontiguousarray(a).view(np.uint8)  # caches hold random bytes (NaN patterns too)
    assert np.array_equal(raw(to_np(tq)), raw(oq)), "rotated queries differ"
    assert np.array_equal(raw(to_np(tk)), raw(k)), "the fused op must not write the key source"
    assert np.array_equal(raw(to_np(tkc)), raw(okc)), "key cache differs"
    assert np.array_equal(raw(to_np(tvc)), raw(ovc)), "value cache differs"
    if cache == "fp8":
        assert np.array_equal(to_np(tks), ks) and np.array_equal(to_np(tvs), vs), "FP8 scales differ"


@pytest.mark.gpu
@pytest.mark.parametrize("D,src", [(64, np.float32), (128, np.float16), (256, np.float32)])
def test_rope_only_in_place(vkv, oracle, cuda, D, src):
    """key_cache None: the reference's rope_forward (q and k rotated in place), start_pos form."""
    import torch
    rng = np.random.default_rng(D)
    T, H, Hkv, P = 21, 14, 2, 64
    q, k, _ = _inputs(rng, T, H, Hkv, D, src)
    cs = random_table(rng, P, D)
    tq, tk = to_dev(q, cuda), to_dev(k, cuda)
    vkv.rope_reshape_and_cache(tq, tk, None, to_dev(cs, cuda), start_pos=11)
    torch.cuda.synchronize()
    oq, ok = _bits(q.copy()), _bits(k.copy())
    oracle.rope(oq, ok, cs, start_pos=11)
    assert np.array_equal(_bits(to_np(tq)), oq)
    assert np.array_equal(_bits(to_np(tk)), ok)


@pytest.mark.gpu
def test_fused_equals_unfused_llama_step(vkv, cuda):
    """C2-shaped step (64 tokens, H32/Hkv8/D128 fp16, reference table): fused op == GPU rope
    then GPU append, and both equal the f64 rotation within fp16 rounding."""
    import torch
    rng = np.random.default_rng(11)
    T, H, Hkv, D, N, bs = 64, 32, 8, 128, 300, 16
    cs = vkv.rope_cos_sin_host(500000.0, D, 4200)
    pos = rng.integers(512, 4096, T).astype(np.int32)
    q, k, v = _inputs(rng, T, H, Hkv, D, np.float16)
    slots = rng.permutation(N * bs)[:T].astype(np.int32)
    tcs, tpos, tsl = to_dev(cs, cuda), to_dev(pos, cuda), to_dev(slots, cuda)
    kc1 = torch.zeros((N, bs, Hkv, D), dtype=torch.float16, device=cuda)
    vc1, kc2, vc2 = kc1.clone(), kc1.clone(), kc1.clone()
    q1, q2 = to_dev(q, cuda), to_dev(q, cuda)
    k1, k2, v1 = to_dev(k, cuda), to_dev(k, cuda), to_dev(v, cuda)
    vkv.rope_reshape_and_cache(q1, k1, v1, tcs, positions=tpos, key_cache=kc1, value_cache=vc1, slot_mapping=tsl)
    vkv.rope_reshape_and_cache(q2, k2, None, tcs, positions=tpos)
    vkv.reshape_and_cache(k2, v1, kc2, vc2, tsl)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    ref = rope_f64(q.astype(np.float32), cs, pos)
    got = to_np(q1).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-4).all()
