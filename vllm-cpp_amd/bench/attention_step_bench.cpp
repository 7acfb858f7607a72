// attention_step_bench.cpp — one decode step of every layer of a Llama-3-8B-
// shaped model's attention (32 layers, H32/Hkv8/D128, fp16 KV, bs16, 64
// sequences with contexts U[512,4096] as in C2), run two ways on the GPU:
//
//   batched   AttentionMetadata::build once per step, then per layer one
//             PagedAttentionLayer::forward (fused RoPE + append, one decode
//             launch for all sequences);
//   per-token the reference's call pattern (src/layers/attention.cpp:78-129
//             run per sequence, as src/core/engine.cpp:176-186 does): per
//             layer and sequence a RoPE launch, two device copies placing K
//             and V, two pageable host->device uploads (context length, block
//             table), a memset of the output and a one-sequence decode.
//
// Both use this library's kernels, so the difference is the host/launch
// structure of the step.  Prints one JSON line; the last layer's outputs of
// the two runs are compared (same inputs, fp16 tolerance).
//
//   bench_attention_step [layers=32] [batched_steps=20] [per_token_steps=2]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "vllm/attention/attention_step.hpp"
#include "vllm/core/block_manager.hpp"
#include "vllm/memory/kv_cache.hpp"
#include "vllm/utils/hip_utils.hpp"
#include "vllm_kv_amd.h"

namespace {

constexpr int H = 32, Hkv = 8, D = 128, BS = 16, S = 64;

uint16_t f16_bits(float x) {
    _Float16 h = static_cast<_Float16>(x);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

float f16_value(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return static_cast<float>(h);
}

}  // namespace

int main(int argc, char** argv) {
    const int L = argc > 1 ? std::atoi(argv[1]) : 32;
    const int batched_steps = argc > 2 ? std::atoi(argv[2]) : 20;
    const int per_token_steps = argc > 3 ? std::atoi(argv[3]) : 2;
    std::mt19937 gen(1);
    std::uniform_int_distribution<int> ctx_dist(512, 4096);
    std::vector<int> ctx(S);
    int64_t need = 0;
    for (int s = 0; s < S; ++s) {
        ctx[s] = ctx_dist(gen);
        need += (ctx[s] + 1 + BS - 1) / BS;
    }
    const int N = int(need * 11 / 10);
    const int MB = (4096 + 1 + BS - 1) / BS;
    const int P = 8192;

    vllm::KVCache cache(L, N, BS, Hkv, D, nullptr, nullptr, vllm::KVDtype::kF16);
    const size_t layer_bytes = cache.layer_bytes();
    for (int l = 0; l < L; ++l) {  // any finite fp16 content (0x3333 = 0.2249)
        VLLM_HIP_CHECK(hipMemset(cache.k_ptr(l, 0), 0x33, layer_bytes));
        VLLM_HIP_CHECK(hipMemset(cache.v_ptr(l, 0), 0x33, layer_bytes));
    }
    // block tables from the pool in a random order (BlockManager ids, permuted)
    vllm::BlockManager bm(BS, N, 0);
    std::vector<std::vector<int32_t>> tables(S);
    for (int s = 0; s < S; ++s) tables[s] = bm.allocate_for_sequence(size_t(ctx[s] + 1));
    std::vector<int32_t> perm(N);
    for (int i = 0; i < N; ++i) perm[i] = i;
    std::shuffle(perm.begin(), perm.end(), gen);
    for (auto& t : tables)
        for (auto& id : t) id = perm[id];

    std::vector<float> cs(size_t(P) * D);
    VLLM_KV_CHECK(vkv_rope_cos_sin_host(500000.0f, D, P, cs.data()));
    float* dcs;
    VLLM_HIP_CHECK(hipMalloc(&dcs, cs.size() * 4));
    VLLM_HIP_CHECK(hipMemcpy(dcs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));

    // q/k/v of every layer (post-projection), fp16
    std::normal_distribution<float> nd(0.f, 0.3f);
    const size_t qn = size_t(S) * H * D, kn = size_t(S) * Hkv * D;
    std::vector<uint16_t> hq(qn * L), hk(kn * L), hv(kn * L);
    for (auto& x : hq) x = f16_bits(nd(gen));
    for (auto& x : hk) x = f16_bits(nd(gen));
    for (auto& x : hv) x = f16_bits(nd(gen));
    uint16_t *dq0, *dq, *dk, *dv, *dout, *dout_ref;
    VLLM_HIP_CHECK(hipMalloc(&dq0, hq.size() * 2));
    VLLM_HIP_CHECK(hipMalloc(&dq, hq.size() * 2));
    VLLM_HIP_CHECK(hipMalloc(&dk, hk.size() * 2));
    VLLM_HIP_CHECK(hipMalloc(&dv, hv.size() * 2));
    VLLM_HIP_CHECK(hipMalloc(&dout, qn * L * 2));
    VLLM_HIP_CHECK(hipMalloc(&dout_ref, qn * L * 2));
    VLLM_HIP_CHECK(hipMemcpy(dq0, hq.data(), hq.size() * 2, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dk, hk.data(), hk.size() * 2, hipMemcpyHostToDevice));
    VLLM_HIP_CHECK(hipMemcpy(dv, hv.data(), hv.size() * 2, hipMemcpyHostToDevice));

    hipStream_t st;
    VLLM_HIP_CHECK(hipStreamCreate(&st));
    hipEvent_t e0, e1;
    VLLM_HIP_CHECK(hipEventCreate(&e0));
    VLLM_HIP_CHECK(hipEventCreate(&e1));

    // ---------------- batched
    vllm::AttentionMetadata md(S, S, MB, BS);
    vllm::PagedAttentionLayer attn(H, Hkv, D, P);
    attn.attach_rope_table(dcs, P);
    std::vector<vllm::StepSequence> step(S);
    for (int s = 0; s < S; ++s) step[s] = {tables[s].data(), int32_t(tables[s].size()), ctx[s], 1};
    auto batched = [&]() {
        // queries are rotated in place: start every step from the same inputs
        VLLM_HIP_CHECK(hipMemcpyAsync(dq, dq0, hq.size() * 2, hipMemcpyDeviceToDevice, st));
        md.build(step, st);
        for (int l = 0; l < L; ++l)
            attn.forward(dout + qn * l, dq + qn * l, dk + kn * l, dv + kn * l, vllm::KVDtype::kF16, cache, md,
                         size_t(l), st);
    };
    batched();  // warm-up (and the workspace allocation)
    VLLM_HIP_CHECK(hipStreamSynchronize(st));
    VLLM_HIP_CHECK(hipEventRecord(e0, st));
    for (int i = 0; i < batched_steps; ++i) batched();
    VLLM_HIP_CHECK(hipEventRecord(e1, st));
    VLLM_HIP_CHECK(hipEventSynchronize(e1));
    float ms_b = 0;
    VLLM_HIP_CHECK(hipEventElapsedTime(&ms_b, e0, e1));
    // subtract the query restore copies (not part of the step)
    VLLM_HIP_CHECK(hipEventRecord(e0, st));
    for (int i = 0; i < batched_steps; ++i)
        VLLM_HIP_CHECK(hipMemcpyAsync(dq, dq0, hq.size() * 2, hipMemcpyDeviceToDevice, st));
    VLLM_HIP_CHECK(hipEventRecord(e1, st));
    VLLM_HIP_CHECK(hipEventSynchronize(e1));
    float ms_copy = 0;
    VLLM_HIP_CHECK(hipEventElapsedTime(&ms_copy, e0, e1));
    const double us_batched = (ms_b - ms_copy) * 1e3 / batched_steps;

    // ---------------- per-token (the reference's structure)
    int32_t *ctx_d, *bt_d;
    VLLM_HIP_CHECK(hipMalloc(&ctx_d, 4));
    VLLM_HIP_CHECK(hipMalloc(&bt_d, MB * 4));
    const size_t row_bytes = size_t(Hkv) * D * 2;
    auto per_token = [&]() {
        VLLM_HIP_CHECK(hipMemcpyAsync(dq, dq0, hq.size() * 2, hipMemcpyDeviceToDevice, st));
        for (int l = 0; l < L; ++l) {
            for (int s = 0; s < S; ++s) {
                uint16_t* q = dq + qn * l + size_t(s) * H * D;
                uint16_t* k = dk + kn * l + size_t(s) * Hkv * D;
                const uint16_t* v = dv + kn * l + size_t(s) * Hkv * D;
                vkv_rope_append_params rp{};
                rp.query = q;
                rp.key = k;  // rotated in place, as rope_forward does
                rp.cos_sin = dcs;
                rp.start_pos = ctx[s];
                rp.max_position = P;
                rp.num_tokens = 1;
                rp.num_heads = H;
                rp.num_kv_heads = Hkv;
                rp.head_dim = D;
                rp.src_dtype = VKV_DTYPE_F16;
                VLLM_KV_CHECK(vkv_rope_reshape_and_cache(&rp, reinterpret_cast<vkv_stream_t>(st)));
                const int pos = ctx[s];
                const int32_t blk = tables[s][pos / BS];
                char* kslot = static_cast<char*>(cache.k_ptr(l, blk)) + size_t(pos % BS) * row_bytes;
                char* vslot = static_cast<char*>(cache.v_ptr(l, blk)) + size_t(pos % BS) * row_bytes;
                VLLM_HIP_CHECK(hipMemcpyAsync(kslot, k, row_bytes, hipMemcpyDeviceToDevice, st));
                VLLM_HIP_CHECK(hipMemcpyAsync(vslot, v, row_bytes, hipMemcpyDeviceToDevice, st));
                const int32_t c = ctx[s] + 1;
                VLLM_HIP_CHECK(hipMemcpyAsync(ctx_d, &c, 4, hipMemcpyHostToDevice, st));
                VLLM_HIP_CHECK(hipMemcpyAsync(bt_d, tables[s].data(), tables[s].size() * 4, hipMemcpyHostToDevice, st));
                uint16_t* o = dout_ref + qn * l + size_t(s) * H * D;
                VLLM_HIP_CHECK(hipMemsetAsync(o, 0, size_t(H) * D * 2, st));
                vkv_decode_params dp{};
                dp.output = o;
                dp.query = q;
                dp.key_cache = cache.k_ptr(l, 0);
                dp.value_cache = cache.v_ptr(l, 0);
                dp.block_tables = bt_d;
                dp.context_lens = ctx_d;
                dp.num_seqs = 1;
                dp.num_heads = H;
                dp.num_kv_heads = Hkv;
                dp.head_dim = D;
                dp.block_size = BS;
                dp.max_context_len = std::min(P, N * BS);
                dp.max_blocks_per_seq = int32_t(tables[s].size());
                dp.num_blocks = N;
                dp.scale = 1.0f / std::sqrt(float(D));
                dp.io_dtype = VKV_DTYPE_F16;
                dp.kv_dtype = VKV_DTYPE_F16;
                dp.accumulate = 1;
                VLLM_KV_CHECK(vkv_paged_decode(&dp, reinterpret_cast<vkv_stream_t>(st)));
            }
        }
    };
    // the per-token key rotation is in place: restore k before each run
    std::vector<uint16_t> hk_keep = hk;
    per_token();  // warm-up
    VLLM_HIP_CHECK(hipStreamSynchronize(st));
    double us_per_token = 0;
    for (int i = 0; i < per_token_steps; ++i) {
        VLLM_HIP_CHECK(hipMemcpy(dk, hk_keep.data(), hk_keep.size() * 2, hipMemcpyHostToDevice));
        VLLM_HIP_CHECK(hipStreamSynchronize(st));
        const auto t0 = std::chrono::steady_clock::now();
        per_token();
        VLLM_HIP_CHECK(hipStreamSynchronize(st));
        const auto t1 = std::chrono::steady_clock::now();
        us_per_token += std::chrono::duration<double, std::micro>(t1 - t0).count();
    }
    us_per_token /= per_token_steps;

    // last layer: same inputs, same caches (the append rewrote the same slots)
    std::vector<uint16_t> a(qn), b(qn);
    VLLM_HIP_CHECK(hipMemcpy(a.data(), dout + qn * (L - 1), qn * 2, hipMemcpyDeviceToHost));
    VLLM_HIP_CHECK(hipMemcpy(b.data(), dout_ref + qn * (L - 1), qn * 2, hipMemcpyDeviceToHost));
    double worst = 0;
    for (size_t i = 0; i < qn; ++i) {
        const double x = f16_value(a[i]), y = f16_value(b[i]);
        worst = std::max(worst, std::fabs(x - y) / (2e-3 + 1e-2 * std::fabs(y)));
    }
    int64_t kv_tokens = 0;
    for (int s = 0; s < S; ++s) kv_tokens += ctx[s] + 1;
    const double kv_bytes = double(kv_tokens) * Hkv * D * 2 * 2 * L;
    std::printf(
        "{\"row\": \"batched attention step\", \"workload\": \"Llama-3-8B attention, %d layers, H32/Hkv8/D128 fp16 KV, "
        "bs16, B=64, ctx U[512,4096], one decode token per sequence\", \"layers\": %d, "
        "\"batched_us_per_step\": %.1f, \"per_token_us_per_step\": %.1f, \"speedup\": %.1f, "
        "\"batched_decode_tokens_per_s\": %.0f, \"batched_kv_gbs\": %.1f, \"outputs_match\": %s, "
        "\"max_error_ratio\": %.3f}\n",
        L, L, us_batched, us_per_token, us_per_token / us_batched, S / (us_batched * 1e-6),
        kv_bytes / (us_batched * 1e-6) / 1e9, worst <= 1.0 ? "true" : "false", worst);
    return worst <= 1.0 ? 0 : 1;
}
