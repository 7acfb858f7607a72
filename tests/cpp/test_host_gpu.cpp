// test_host_gpu.cpp — the C++ host API on a GPU: KVCache geometry (the
// reference's tests/unit/test_kv_cache.cpp:4-16, restated), KVCache::append and
// vllm::paged_attention_forward against a direct host computation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "check.hpp"
#include "vllm/attention/paged_attention.hpp"
#include "vllm/memory/kv_cache.hpp"
#include "vllm/utils/hip_utils.hpp"

using vllm::KVCache;

TEST_CASE(kv_cache_basic_allocation) {  // reference test_kv_cache.cpp:4-10
    KVCache cache(4, 16, 16, 8, 128);
    CHECK_EQ(cache.num_layers(), 4u);
    CHECK_EQ(cache.num_blocks(), 16u);
    CHECK_EQ(cache.block_size(), 16u);
    CHECK(cache.total_bytes() > 0);
    CHECK_EQ(cache.total_bytes(), 2u * 4 * 16 * 16 * 8 * 128 * 4);  // fp32 by default, as in the reference
}

TEST_CASE(kv_cache_pointers_valid) {  // reference test_kv_cache.cpp:12-16
    KVCache cache(2, 4, 8, 4, 64);
    CHECK(cache.k_ptr(0, 0) != nullptr);
    CHECK(cache.v_ptr(0, 0) != nullptr);
    // per-layer and per-block strides of [L][N][bs][Hkv][D] floats
    auto* k00 = static_cast<char*>(cache.k_ptr(0, 0));
    CHECK_EQ(static_cast<char*>(cache.k_ptr(0, 1)) - k00, 8 * 4 * 64 * 4);
    CHECK_EQ(static_cast<char*>(cache.k_ptr(1, 0)) - k00, 4 * 8 * 4 * 64 * 4);
}

TEST_CASE(kv_cache_fp8_geometry) {
    KVCache cache(2, 10, 16, 8, 128, nullptr, nullptr, vllm::KVDtype::kFP8E4M3);
    CHECK_EQ(cache.block_bytes(), 16u * 8 * 128);
    CHECK_EQ(cache.scale_block_bytes(), 16u * 8 * 4);
    CHECK_EQ(cache.host_block_bytes(), 2u * 2 * (16 * 8 * 128 + 16 * 8 * 4));
    CHECK(cache.k_scale_ptr(1, 3) != nullptr);
}

TEST_CASE(append_and_paged_attention_forward_fp32) {
    // One sequence, the reference's per-token loop replaced by KVCache::append,
    // then vllm::paged_attention_forward with `out +=` on a zeroed output.
    const int L = 2, N = 8, bs = 16, Hkv = 2, D = 64, H = 4, ctx = 37, layer = 1;
    KVCache cache(L, N, bs, Hkv, D);
    std::mt19937 gen(3);
    std::normal_distribution<float> nd(0.f, 0.5f);
    std::vector<float> k(ctx * Hkv * D), v(ctx * Hkv * D), q(H * D);
    for (auto& x : k) x = nd(gen);
    for (auto& x : v) x = nd(gen);
    for (auto& x : q) x = nd(gen);
    std::vector<int32_t> table = {5, 2, 7};  // 3 blocks cover 37 tokens
    std::vector<int32_t> slots(ctx);
    VLLM_KV_CHECK(vkv_slot_mapping_host(table.data(), 3, bs, 0, ctx, slots.data()));
    float *dk, *dv, *dq, *dout;
    int32_t *dslots, *dtable, *dctx;
    VLLM_HIP_CHECK(hipMalloc(&dk, k.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dv, v.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dq, q.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dout, q.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dslots, ctx * 4));
    VLLM_HIP_CHECK(hipMalloc(&dtable, 3 * 4));
    VLLM_HIP_CHECK(hipMalloc(&dctx, 4));
    VLLM_HIP_CHECK(hipMemcpy(dk, k.data(), k.size() * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dv, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dq, q.data(), q.size() * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dslots, slots.data(), ctx * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dtable, table.data(), 3 * 4, hipMemcpyHostToDevice));
    const int32_t c = ctx;
    VLLM_HIP_CHECK(hipMemcpy(dctx, &c, 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemset(dout, 0, q.size() * 4));
    cache.append(layer, dk, dv, dslots, ctx, vllm::KVDtype::kF32, nullptr);

    // the appended rows sit where the reference's memcpy loop puts them
    std::vector<float> row(Hkv * D);
    VLLM_HIP_CHECK(hipMemcpy(row.data(), static_cast<float*>(cache.k_ptr(layer, 2)) + 4 * Hkv * D, row.size() * 4,
                             hipMemcpyDeviceToHost));  // position 20 = block 1 (id 2), slot 4
    bool same = true;
    for (int i = 0; i < Hkv * D; ++i) same &= row[i] == k[20 * Hkv * D + i];
    CHECK(same);

    vllm::PagedAttentionParams p{};
    p.output = dout;
    p.query = dq;
    p.key_cache = static_cast<const float*>(cache.k_ptr(layer, 0));
    p.value_cache = static_cast<const float*>(cache.v_ptr(layer, 0));
    p.block_tables = dtable;
    p.context_lens = dctx;
    p.num_seqs = 1;
    p.num_heads = H;
    p.num_kv_heads = Hkv;
    p.head_dim = D;
    p.block_size = bs;
    p.max_context_len = N * bs;
    p.max_blocks_per_seq = 3;
    p.scale = 1.0f / std::sqrt(float(D));
    p.stream = nullptr;
    vllm::paged_attention_forward(p);
    std::vector<float> out(q.size());
    VLLM_HIP_CHECK(hipMemcpy(out.data(), dout, out.size() * 4, hipMemcpyDeviceToHost));

    double worst = 0;
    int printed = 0;
    for (int h = 0; h < H; ++h) {
        const int kvh = h / (H / Hkv);
        std::vector<double> logit(ctx);
        double m = -1e300, sum = 0;
        for (int t = 0; t < ctx; ++t) {
            double d = 0;
            for (int i = 0; i < D; ++i) d += double(q[h * D + i]) * k[(t * Hkv + kvh) * D + i];
            logit[t] = d * p.scale;
            m = std::max(m, logit[t]);
        }
        for (int t = 0; t < ctx; ++t) sum += std::exp(logit[t] - m);
        for (int i = 0; i < D; ++i) {
            double o = 0;
            for (int t = 0; t < ctx; ++t) o += std::exp(logit[t] - m) / sum * v[(t * Hkv + kvh) * D + i];
            const double r = std::fabs(o - out[h * D + i]) / (2e-5 + 1e-4 * std::fabs(o));
            if (r > 1.0 && printed < 6) {
                std::printf("  head %d dim %d: got %.6f expected %.6f\n", h, i, out[h * D + i], o);
                ++printed;
            }
            worst = std::max(worst, r);
        }
    }
    CHECK(worst <= 1.0);
    if (worst > 1.0) std::printf("  worst error ratio %.3f\n", worst);
    (void)hipFree(dk);
    (void)hipFree(dv);
    (void)hipFree(dq);
    (void)hipFree(dout);
    (void)hipFree(dslots);
    (void)hipFree(dtable);
    (void)hipFree(dctx);
}

// vllm::paged_attention_forward (fp32, the reference's types) at shapes the
// reference kernel accepts beyond the fixed-shape kernels: head_dim 80 / 96 /
// 98, groups 16 / 32 / 64 (MQA), block sizes 12 / 24 / 7.  Several sequences
// over randomly permuted blocks, `out +=` on a zeroed output, against an fp64
// host computation of softmax(scale q K^T) V.
namespace {
struct Shape {
    int H, Hkv, D, bs;
    std::vector<int> ctx;
};

double forward_case(const Shape& c, unsigned seed) {
    const int S = int(c.ctx.size());
    int MB = 1, need = 0;
    for (int n : c.ctx) {
        MB = std::max(MB, (n + c.bs - 1) / c.bs);
        need += (n + c.bs - 1) / c.bs;
    }
    const int N = need + 3;
    std::mt19937 gen(seed);
    std::normal_distribution<float> nd(0.f, 0.5f);
    const size_t pool = size_t(N) * c.bs * c.Hkv * c.D;
    std::vector<float> k(pool), v(pool), q(size_t(S) * c.H * c.D);
    for (auto& x : k) x = nd(gen);
    for (auto& x : v) x = nd(gen);
    for (auto& x : q) x = nd(gen);
    std::vector<int32_t> perm(N);
    for (int i = 0; i < N; ++i) perm[i] = i;
    std::shuffle(perm.begin(), perm.end(), gen);
    std::vector<int32_t> table(size_t(S) * MB, 0), ctx(c.ctx.begin(), c.ctx.end());
    int next = 0;
    for (int s = 0; s < S; ++s)
        for (int b = 0; b < (c.ctx[s] + c.bs - 1) / c.bs; ++b) table[size_t(s) * MB + b] = perm[next++];
    float *dk, *dv, *dq, *dout;
    int32_t *dtable, *dctx;
    VLLM_HIP_CHECK(hipMalloc(&dk, pool * 4));
    VLLM_HIP_CHECK(hipMalloc(&dv, pool * 4));
    VLLM_HIP_CHECK(hipMalloc(&dq, q.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dout, q.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dtable, table.size() * 4));
    VLLM_HIP_CHECK(hipMalloc(&dctx, S * 4));
    VLLM_HIP_CHECK(hipMemcpy(dk, k.data(), pool * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dv, v.data(), pool * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dq, q.data(), q.size() * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dtable, table.data(), table.size() * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dctx, ctx.data(), S * 4, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemset(dout, 0, q.size() * 4));
    vllm::PagedAttentionParams p{};
    p.output = dout;
    p.query = dq;
    p.key_cache = dk;
    p.value_cache = dv;
    p.block_tables = dtable;
    p.context_lens = dctx;
    p.num_seqs = S;
    p.num_heads = c.H;
    p.num_kv_heads = c.Hkv;
    p.head_dim = c.D;
    p.block_size = c.bs;
    p.max_context_len = MB * c.bs;
    p.max_blocks_per_seq = MB;
    p.scale = 1.0f / std::sqrt(float(c.D));
    p.stream = nullptr;
    vllm::paged_attention_forward(p);
    std::vector<float> out(q.size());
    VLLM_HIP_CHECK(hipMemcpy(out.data(), dout, out.size() * 4, hipMemcpyDeviceToHost));
    double worst = 0;
    const int G = c.H / c.Hkv;
    for (int s = 0; s < S; ++s) {
        for (int h = 0; h < c.H; ++h) {
            const int kvh = h / G;
            auto row = [&](const std::vector<float>& x, int t) {
                const int blk = table[size_t(s) * MB + t / c.bs];
                return &x[((size_t(blk) * c.bs + t % c.bs) * c.Hkv + kvh) * c.D];
            };
            const float* qh = &q[(size_t(s) * c.H + h) * c.D];
            std::vector<double> w(c.ctx[s]);
            double m = -1e300, sum = 0;
            for (int t = 0; t < c.ctx[s]; ++t) {
                const float* kr = row(k, t);
                double d = 0;
                for (int i = 0; i < c.D; ++i) d += double(qh[i]) * kr[i];
                w[t] = d * p.scale;
                m = std::max(m, w[t]);
            }
            for (int t = 0; t < c.ctx[s]; ++t) sum += (w[t] = std::exp(w[t] - m));
            for (int i = 0; i < c.D; ++i) {
                double o = 0;
                for (int t = 0; t < c.ctx[s]; ++t) o += w[t] / sum * row(v, t)[i];
                const double got = out[(size_t(s) * c.H + h) * c.D + i];
                worst = std::max(worst, std::fabs(o - got) / (2e-5 + 1e-4 * std::fabs(o)));
            }
        }
    }
    (void)hipFree(dk);
    (void)hipFree(dv);
    (void)hipFree(dq);
    (void)hipFree(dout);
    (void)hipFree(dtable);
    (void)hipFree(dctx);
    return worst;
}
}  // namespace

TEST_CASE(paged_attention_forward_any_shape) {
    const Shape shapes[] = {
        {32, 2, 80, 12, {1, 12, 13, 250}},    // head_dim 80, group 16, block 12
        {64, 2, 96, 24, {7, 24, 300}},        // head_dim 96, group 32, block 24
        {64, 1, 80, 24, {2, 100}},            // MQA: group 64
        {6, 3, 98, 7, {1, 8, 90}},            // element loads, block 7
    };
    unsigned seed = 11;
    for (const Shape& c : shapes) {
        const double worst = forward_case(c, seed++);
        if (worst > 1.0)
            std::printf("  H%d Hkv%d D%d bs%d: worst error ratio %.3f\n", c.H, c.Hkv, c.D, c.bs, worst);
        CHECK(worst <= 1.0);
    }
}

TEST_CASE(copy_blocks_through_kv_cache) {
    KVCache cache(3, 6, 16, 2, 64, nullptr, nullptr, vllm::KVDtype::kF16);
    const size_t bytes = cache.block_bytes();
    std::vector<uint8_t> pattern(bytes);
    for (size_t i = 0; i < bytes; ++i) pattern[i] = uint8_t(i * 7 + 3);
    for (int l = 0; l < 3; ++l) VLLM_HIP_CHECK(hipMemcpy(cache.k_ptr(l, 1), pattern.data(), bytes, hipMemcpyHostToDevice));
    int32_t pairs[2] = {1, 4};
    int32_t* dpairs;
    VLLM_HIP_CHECK(hipMalloc(&dpairs, sizeof(pairs)));
    VLLM_HIP_CHECK(hipMemcpy(dpairs, pairs, sizeof(pairs), hipMemcpyHostToDevice));
    cache.copy_blocks(dpairs, 1, nullptr);
    VLLM_HIP_CHECK(hipDeviceSynchronize());
    std::vector<uint8_t> got(bytes);
    bool same = true;
    for (int l = 0; l < 3; ++l) {
        VLLM_HIP_CHECK(hipMemcpy(got.data(), cache.k_ptr(l, 4), bytes, hipMemcpyDeviceToHost));
        same &= got == pattern;
    }
    CHECK(same);
    (void)hipFree(dpairs);
}

int main() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        std::printf("no GPU\n");
        return 2;
    }
    return check::run_all();
}
