"""Pins the CPU oracle (oracle/kv_oracle.c) against checks that do not restate it.

- fp16 conversions: every bit pattern against numpy.float16.
- e4m3fn decode: all 256 codes against torch.float8_e4m3fn; encode: every fp16
  value and a dense fp32 sweep against torch's round-to-nearest-even cast, plus
  the saturation rule by closed form.
- decode attention: fp64 textbook softmax(q K^T s) V (numpy) with distinct
  keys per kv head (a wrong GQA map, scale, or token order fails), and closed
  forms: ctx 1 -> V0 exactly, equal keys -> mean V, one dominant logit -> its V,
  ctx 0 -> output untouched, clamp to max_context_len.
- prefill: fp64 causal masked attention.
- append / copy / swap: numpy scatter and fancy-index copies; FP8 append
  through torch's e4m3 cast of the fp32 quotient.
"""
import numpy as np
import pytest

from helpers import gather_tokens, softmax_attention_f64


def torch_fp8_encode(x_f32):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x_f32, np.float32)).to(torch.float8_e4m3fn)
    return t.view(torch.uint8).numpy()


def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_rne(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        (rng.random(20000) * 70000 - 35000).astype(np.float32),
        np.ldexp(rng.random(5000), rng.integers(-30, -10, 5000)).astype(np.float32),  # subnormal range
        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e9, -1e9, np.inf, -np.inf], np.float32),
        # exact ties between fp16 neighbours
        (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
    ])
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


def test_fp8_decode_all_codes(oracle):
    import torch
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.fp8_decode(int(c)) for c in codes], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    assert nan.sum() == 2 and got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9


def test_fp8_encode_every_fp16_value(oracle):
    vals = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) < 464.0)]  # torch overflows to NaN beyond; saturation below
    got = np.array([oracle.fp8_encode(float(v)) for v in vals], np.uint8)
    assert np.array_equal(got, torch_fp8_encode(vals))


def test_fp8_encode_fp32_sweep_and_saturation(oracle):
    rng = np.random.default_rng(1)
    mags = np.ldexp(1.0 + rng.random(30000), rng.integers(-12, 9, 30000)).astype(np.float32)
    x = mags * rng.choice([-1.0, 1.0], 30000).astype(np.float32)
    x = x[np.abs(x) < 464.0]
    got = np.array([oracle.fp8_encode(float(v)) for v in x], np.uint8)
    assert np.array_equal(got, torch_fp8_encode(x))
    for v, code in [(448.0, 0x7E), (463.9, 0x7E), (464.0, 0x7E), (1e6, 0x7E), (np.inf, 0x7E),
                    (-1e6, 0xFE), (-np.inf, 0xFE), (np.nan, 0x7F), (-0.0, 0x80), (2.0 ** -10, 0x00),
                    (3 * 2.0 ** -11, 0x01)]:
        assert oracle.fp8_encode(v) == code, v


def test_fp8_scale_rule(oracle):
    assert oracle.fp8_scale(0.0) == 1.0
    for a in [448.0, 1.0, 3.5, 1e-5, 65504.0]:
        assert oracle.fp8_scale(a) == np.float32(np.float32(a) / np.float32(448.0))


def _random_case(rng, H, Hkv, D, bs, ctx, N=None):
    from vllm_kv_amd import workloads
    need = sum((c + bs - 1) // bs for c in ctx)
    lay = workloads.make_layout(np.asarray(ctx, np.int32), bs, rng, num_blocks=N or need + 2)
    k = rng.standard_normal((lay.num_blocks, bs, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((lay.num_blocks, bs, Hkv, D)).astype(np.float32)
    q = rng.standard_normal((len(ctx), H, D)).astype(np.float32)
    return lay, q, k, v


@pytest.mark.parametrize("H,Hkv,D,bs,ctx", [(14, 2, 64, 16, [1, 33, 300]), (8, 8, 32, 4, [7, 19]),
                                            (12, 3, 128, 32, [65, 2]), (4, 1, 64, 16, [100])])
def test_decode_matches_fp64_textbook(oracle, H, Hkv, D, bs, ctx):
    rng = np.random.default_rng(H + D + bs)
    lay, q, k, v = _random_case(rng, H, Hkv, D, bs, ctx)
    scale = 1.0 / np.sqrt(D)
    got = oracle.paged_decode(q, k, v, lay.block_tables, lay.context_lens, scale)
    G = H // Hkv
    for s, n in enumerate(ctx):
        kk = gather_tokens(k, lay.block_tables[s], n, bs)
        vv = gather_tokens(v, lay.block_tables[s], n, bs)
        for h in range(H):
            ref = softmax_attention_f64(q[s, h], kk[:, h // G], vv[:, h // G], scale)
            np.testing.assert_allclose(got[s, h], ref, rtol=2e-5, atol=2e-6)


def test_decode_threads_agree(oracle):
    rng = np.random.default_rng(3)
    lay, q, k, v = _random_case(rng, 16, 4, 64, 16, [50, 400, 3, 129])
    a = oracle.paged_decode(q, k, v, lay.block_tables, lay.context_lens, 0.125, nthreads=1)
    b = oracle.paged_decode(q, k, v, lay.block_tables, lay.context_lens, 0.125, nthreads=5)
    assert np.array_equal(a, b)


def test_decode_closed_forms(oracle):
    rng = np.random.default_rng(4)
    H, Hkv, D, bs = 4, 2, 64, 16
    lay, q, k, v = _random_case(rng, H, Hkv, D, bs, [1, 40, 40, 0, 70])
    # seq 1: all its keys equal -> uniform weights -> mean of V
    t1 = lay.block_tables[1]
    k[t1[:3]] = k[t1[0], 0]
    # seq 2: one key aligned with the query of every head of kv head 0, scaled up
    t2 = lay.block_tables[2]
    k[t2[1], 5, 0] = q[2, 0] * 50.0
    q[2, 1] = q[2, 0]
    prior = rng.standard_normal((5, H, D)).astype(np.float32)
    out = oracle.paged_decode(q, k, v, lay.block_tables, lay.context_lens, 0.125, max_context_len=64,
                              out=prior.copy())
    # ctx 1: the single V row, exactly (weight e^0 / (1 + 1e-10) == 1 in fp32)
    t0 = lay.block_tables[0]
    for h in range(H):
        assert np.array_equal(out[0, h], prior[0, h] + v[t0[0], 0, h // 2]) or \
            np.allclose(out[0, h], prior[0, h] + v[t0[0], 0, h // 2], rtol=0, atol=1e-6)
    vv = gather_tokens(v, t1, 40, bs)
    for h in range(H):
        np.testing.assert_allclose(out[1, h] - prior[1, h], vv[:, h // 2].mean(0), atol=2e-6)
    for h in (0, 1):
        np.testing.assert_allclose(out[2, h] - prior[2, h], v[t2[1], 5, 0], atol=1e-5)
    assert np.array_equal(out[3], prior[3])  # ctx 0 leaves the accumulator untouched
    # ctx 70 clamped to max_context_len 64
    ref = oracle.paged_decode(q[4:5], k, v, lay.block_tables[4:5], np.array([64], np.int32), 0.125,
                              out=prior[4:5].copy())
    np.testing.assert_array_equal(out[4], ref[0])


def test_decode_single_value_exact(oracle):
    """ctx 1 with a zero accumulator returns V0 bit for bit."""
    rng = np.random.default_rng(5)
    lay, q, k, v = _random_case(rng, 2, 1, 64, 16, [1])
    out = oracle.paged_decode(q, k, v, lay.block_tables, lay.context_lens, 0.125)
    assert np.array_equal(out[0, 0], v[lay.block_tables[0, 0], 0, 0])


def test_decode_fp8_dequantises_code_times_scale(oracle):
    rng = np.random.default_rng(6)
    H, Hkv, D, bs = 4, 2, 32, 8
    lay, q, k, v = _random_case(rng, H, Hkv, D, bs, [9, 20])
    kc = rng.integers(0, 0x7F, size=k.shape, dtype=np.uint8) | (rng.integers(0, 2, size=k.shape, dtype=np.uint8) << 7)
    vc = rng.integers(0, 0x7F, size=v.shape, dtype=np.uint8)
    ks = rng.random(k.shape[:3], dtype=np.float32) + 0.1
    vs = rng.random(v.shape[:3], dtype=np.float32) + 0.1
    got = oracle.paged_decode(q, kc, vc, lay.block_tables, lay.context_lens, 0.2, key_scales=ks, value_scales=vs)
    import torch
    deq = lambda c: torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()  # noqa: E731
    kf = deq(kc) * ks[..., None]
    vf = deq(vc) * vs[..., None]
    ref = oracle.paged_decode(q, kf, vf, lay.block_tables, lay.context_lens, 0.2)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_prefill_matches_causal_fp64(oracle):
    from vllm_kv_amd import workloads
    rng = np.random.default_rng(7)
    H, Hkv, D, bs = 6, 2, 32, 8
    q_lens = np.array([5, 1, 9], np.int32)
    prior = np.array([0, 12, 3], np.int32)
    ctx = prior + q_lens
    lay = workloads.make_layout(ctx, bs, rng, slack=0.5)
    k = rng.standard_normal((lay.num_blocks, bs, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((lay.num_blocks, bs, Hkv, D)).astype(np.float32)
    qsl = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = rng.standard_normal((int(qsl[-1]), H, D)).astype(np.float32)
    got = oracle.paged_prefill(q, k, v, lay.block_tables, ctx, qsl, 0.3)
    for s in range(3):
        kk = gather_tokens(k, lay.block_tables[s], ctx[s], bs)
        vv = gather_tokens(v, lay.block_tables[s], ctx[s], bs)
        for j in range(q_lens[s]):
            n = prior[s] + j + 1
            for h in range(H):
                ref = softmax_attention_f64(q[qsl[s] + j, h], kk[:n, h // 3], vv[:n, h // 3], 0.3)
                np.testing.assert_allclose(got[qsl[s] + j, h], ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_append_is_a_row_scatter(oracle, dtype):
    rng = np.random.default_rng(8)
    N, bs, Hkv, D, T = 10, 4, 3, 16, 25
    kc = np.zeros((N, bs, Hkv, D), dtype)
    vc = np.zeros_like(kc)
    slots = rng.permutation(N * bs)[:T].astype(np.int32)
    slots[0] = -1
    slots[1] = N * bs
    k = rng.standard_normal((T, Hkv, D)).astype(dtype)
    v = rng.standard_normal((T, Hkv, D)).astype(dtype)
    view = (lambda a: a.view(np.uint16)) if dtype == np.float16 else (lambda a: a)
    oracle.reshape_and_cache(view(k), view(v), view(kc), view(vc), slots)
    ek = np.zeros_like(kc).reshape(N * bs, Hkv, D)
    ev = np.zeros_like(vc).reshape(N * bs, Hkv, D)
    ok = (slots >= 0) & (slots < N * bs)
    ek[slots[ok]] = k[ok]
    ev[slots[ok]] = v[ok]
    assert np.array_equal(kc.reshape(N * bs, Hkv, D), ek)
    assert np.array_equal(vc.reshape(N * bs, Hkv, D), ev)


def test_append_fp8_matches_torch_quantisation(oracle):
    rng = np.random.default_rng(9)
    N, bs, Hkv, D, T = 8, 4, 2, 32, 20
    k = (rng.standard_normal((T, Hkv, D)) * 3).astype(np.float16)
    k[::5] *= 8
    k[2, 1] = 0
    v = (rng.standard_normal((T, Hkv, D)) * 1e-3).astype(np.float16)
    slots = rng.permutation(N * bs)[:T].astype(np.int32)
    kc = np.zeros((N, bs, Hkv, D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros((N, bs, Hkv), np.float32)
    vs = np.zeros_like(ks)
    oracle.reshape_and_cache(k.view(np.uint16), v.view(np.uint16), kc, vc, slots, ks, vs)
    for x, codes, scales in ((k, kc, ks), (v, vc, vs)):
        xf = x.astype(np.float32)
        amax = np.abs(xf).max(-1)
        sc = np.where(amax == 0, np.float32(1), amax / np.float32(448)).astype(np.float32)
        q = torch_fp8_encode(xf / sc[..., None])
        assert np.array_equal(scales.reshape(-1, Hkv)[slots], sc)
        assert np.array_equal(codes.reshape(-1, Hkv, D)[slots], q)


@pytest.mark.parametrize("src", [np.float16, np.float32])
def test_fp8_quantise_rows_matches_append_and_torch(oracle, src):
    """The dense quantiser (the checker of the large FP8 append test) against
    the append's own scatter and against torch's e4m3 cast of x / (amax / 448),
    on C5's input distribution (N(0,1) with 1 % outliers x8, seed 4), with an
    all-zero vector and a 448-saturating one."""
    rng = np.random.default_rng(4)
    T, Hkv, D = 512, 8, 128
    x = rng.standard_normal((T, Hkv, D), dtype=np.float32)
    x = np.where(rng.random(x.shape) < 0.01, x * 8, x).astype(src)
    x[3, 2] = 0
    x[7, 1, 5] = 900
    bits = x.view(np.uint16) if src == np.float16 else x
    codes, scales = oracle.fp8_quantise_rows(bits, nthreads=4)
    N, bs = T // 4 + 3, 4
    slots = rng.permutation(N * bs)[:T].astype(np.int32)
    kc = np.zeros((N, bs, Hkv, D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros((N, bs, Hkv), np.float32)
    vs = np.zeros_like(ks)
    oracle.reshape_and_cache(bits, bits, kc, vc, slots, ks, vs)
    assert np.array_equal(kc.reshape(-1, Hkv, D)[slots], codes)
    assert np.array_equal(ks.reshape(-1, Hkv)[slots], scales)
    xf = x.astype(np.float32)
    amax = np.abs(xf).max(-1)
    sc = np.where(amax == 0, np.float32(1), amax / np.float32(448)).astype(np.float32)
    assert np.array_equal(scales, sc)
    assert np.array_equal(codes, torch_fp8_encode(xf / sc[..., None]))
    assert scales[3, 2] == 1.0 and not codes[3, 2].any()


def test_decode_scale_zero_is_mean_of_v(oracle):
    """scale 0: every key weighs e^0 = 1 (the reference's m0 = -1e30 start makes
    the first max 0), so each output is the mean of V over the context."""
    rng = np.random.default_rng(12)
    H, Hkv, D, bs = 6, 2, 32, 8
    lay, q, k, v = _random_case(rng, H, Hkv, D, bs, [1, 9, 40])
    out = oracle.paged_decode(q * 30, k, v, lay.block_tables, lay.context_lens, 0.0)
    for s, n in enumerate(lay.context_lens):
        vv = gather_tokens(v, lay.block_tables[s], int(n), bs)
        for h in range(H):
            np.testing.assert_allclose(out[s, h], vv[:, h // 3].mean(0), rtol=1e-6, atol=1e-6)


def test_copy_and_swap_blocks(oracle):
    rng = np.random.default_rng(10)
    L, N = 3, 12
    k = rng.integers(0, 255, (L, N, 4, 2, 8), dtype=np.uint8)
    s = rng.random((L, N, 4, 2), dtype=np.float32)
    pairs = np.array([[0, 5], [3, 7], [11, 1], [20, 2]], np.int32)  # last pair out of range
    k2, s2 = k.copy(), s.copy()
    oracle.copy_blocks([k2, s2], pairs)
    ek, es = k.copy(), s.copy()
    for a, b in pairs[:3]:
        ek[:, b] = k[:, a]
        es[:, b] = s[:, a]
    assert np.array_equal(k2, ek) and np.array_equal(s2, es)
    hbb = L * (k[0, 0].nbytes + s[0, 0].nbytes)
    host = np.zeros(4 * hbb, np.uint8)
    out_pairs = np.array([[4, 0], [9, 3]], np.int32)
    oracle.swap_blocks([k, s], host, 4, out_pairs, 0)
    blk = host[3 * hbb:4 * hbb]
    assert np.array_equal(blk[:L * k[0, 0].nbytes].reshape(L, -1), k[:, 9].reshape(L, -1))
    k3, s3 = np.zeros_like(k), np.zeros_like(s)
    oracle.swap_blocks([k3, s3], host, 4, out_pairs[:, ::-1].copy(), 1)
    assert np.array_equal(k3[:, 4], k[:, 4]) and np.array_equal(s3[:, 9], s[:, 9])
