/*
 * kv_oracle.c — CPU restatement of the reference's paged KV-cache path.
 * TEST INFRASTRUCTURE ONLY (see kv_oracle.h): the product never links this.
 *
 * Built with -ffp-contract=off so that every fused multiply-add below is an
 * explicit fmaf() and every other operation rounds on its own, on any host.
 */
#include "kv_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 */

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    float mag;
    if (exp == 0x1F) {
        mag = man ? NAN : INFINITY;
    } else if (exp == 0) {
        mag = ldexpf((float)man, -24); /* subnormal: man * 2^-24, exact */
    } else {
        mag = ldexpf((float)(man | 0x400u), (int)exp - 25); /* 1.man * 2^(exp-15) */
    }
    return sign ? -mag : mag;
}

uint16_t oracle_f32_to_f16(float f) {
    /* Round to nearest even through an exact double computation. */
    uint16_t sign = signbit(f) ? 0x8000u : 0u;
    if (isnan(f)) return (uint16_t)(sign | 0x7E00u);
    double a = fabs((double)f);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
    if (a < ldexp(1.0, -14)) {
        /* subnormal grid: multiples of 2^-24 */
        double q = a * ldexp(1.0, 24);
        double r = nearbyint(q); /* default rounding mode: nearest even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    int e;
    double m = frexp(a, &e); /* a = m * 2^e, m in [0.5,1) */
    /* 11 significant bits: scale so that the integer part has 11 bits */
    double q = ldexp(m, 11);
    double r = nearbyint(q);
    if (r >= 2048.0) { r = 1024.0; e += 1; }
    int exp16 = e - 1 + 15; /* value = r * 2^(e-11) = (r/1024) * 2^(e-1) */
    if (exp16 >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(exp16 << 10) | (uint16_t)((uint32_t)r - 1024u));
}

/* ---------------------------------------------------------------- fp8 */

float oracle_fp8_decode(uint8_t code) {
    int sign = code >> 7;
    int exp = (code >> 3) & 0xF;
    int man = code & 0x7;
    float mag;
    if (exp == 0xF && man == 0x7) {
        mag = NAN;
    } else if (exp == 0) {
        mag = ldexpf((float)man, -9); /* man/8 * 2^(1-7) */
    } else {
        mag = ldexpf((float)(8 + man), exp - 10); /* (1+man/8) * 2^(exp-7) */
    }
    return sign ? -mag : mag;
}

uint8_t oracle_fp8_encode(float x) {
    uint8_t sign = signbit(x) ? 0x80u : 0u;
    if (isnan(x)) return (uint8_t)(sign | 0x7Fu);
    double a = fabs((double)x);
    if (a >= 448.0) return (uint8_t)(sign | 0x7Eu);
    int best = 0;
    double best_err = a; /* distance to code 0 */
    for (int c = 1; c <= 0x7E; ++c) {
        double v = (double)oracle_fp8_decode((uint8_t)c);
        double err = fabs(v - a);
        if (err < best_err || (err == best_err && (c & 1) == 0 && (best & 1) == 1)) {
            best = c;
            best_err = err;
        }
    }
    return (uint8_t)(sign | (uint8_t)best);
}

float oracle_fp8_scale(float amax) {
    if (amax == 0.0f) return 1.0f;
    return amax / 448.0f;
}

/* ---------------------------------------------------------------- helpers */

/* Decode tables filled once from the scalar definitions above, so that the
 * attention loops do not call ldexpf per element. */
static float g_f16_table[65536];
static float g_fp8_table[256];
static pthread_once_t g_tables_once = PTHREAD_ONCE_INIT;

static void fill_tables(void) {
    for (uint32_t i = 0; i < 65536u; ++i) g_f16_table[i] = oracle_f16_to_f32((uint16_t)i);
    for (uint32_t i = 0; i < 256u; ++i) g_fp8_table[i] = oracle_fp8_decode((uint8_t)i);
}

static float load_elem(const void* base, int64_t i, int32_t dtype) {
    switch (dtype) {
        case OR_F32: return ((const float*)base)[i];
        case OR_F16: return g_f16_table[((const uint16_t*)base)[i]];
        default: return g_fp8_table[((const uint8_t*)base)[i]];
    }
}

static size_t dtype_bytes(int32_t dtype) {
    return dtype == OR_F32 ? 4u : dtype == OR_F16 ? 2u : 1u;
}

/* ---------------------------------------------------------------- rope */

static void store_elem(void* base, int64_t i, int32_t dtype, float x) {
    if (dtype == OR_F32) ((float*)base)[i] = x;
    else ((uint16_t*)base)[i] = oracle_f32_to_f16(x);
}

/* src/kernels/rotary_embedding.cu:13-34, one (token, head, dim pair) at a time:
 * x0 = x[d], x1 = x[d + D/2], c/s from the interleaved table row of pos;
 * x[d] = x0*c - x1*s, x[d+D/2] = x0*s + x1*c, each evaluated as one fused
 * multiply-add over a rounded product (fmaf(x0, c, -(x1*s)), fmaf(x0, s, x1*c)). */
static void rope_vec(void* base, int64_t off, int32_t head_dim, const float* row, int32_t dtype) {
    const int32_t half = head_dim / 2;
    for (int32_t d = 0; d < half; ++d) {
        const float c = row[2 * d], s = row[2 * d + 1];
        const float x0 = load_elem(base, off + d, dtype);
        const float x1 = load_elem(base, off + d + half, dtype);
        store_elem(base, off + d, dtype, fmaf(x0, c, -(x1 * s)));
        store_elem(base, off + d + half, dtype, fmaf(x0, s, x1 * c));
    }
}

void oracle_rope(void* query, void* key, int64_t query_stride, int64_t key_stride,
                 const float* cos_sin, const int32_t* positions, int32_t start_pos,
                 int32_t max_position, int32_t num_tokens, int32_t num_heads,
                 int32_t num_kv_heads, int32_t head_dim, int32_t src_dtype) {
    pthread_once(&g_tables_once, fill_tables);
    if (query_stride == 0) query_stride = (int64_t)num_heads * head_dim;
    if (key_stride == 0) key_stride = (int64_t)num_kv_heads * head_dim;
    for (int32_t t = 0; t < num_tokens; ++t) {
        int32_t pos = positions ? positions[t] : start_pos + t;
        if (pos < 0) pos = 0;
        if (pos >= max_position) pos = max_position - 1;
        const float* row = cos_sin + (int64_t)pos * head_dim;
        for (int32_t h = 0; h < num_heads; ++h) {
            rope_vec(query, t * query_stride + (int64_t)h * head_dim, head_dim, row, src_dtype);
            if (h < num_kv_heads) rope_vec(key, t * key_stride + (int64_t)h * head_dim, head_dim, row, src_dtype);
        }
    }
}

/* ---------------------------------------------------------------- append */

/* One (token, kv head) vector of head_dim source elements at element offset
 * s0 -> head_dim e4m3 codes; returns the vector's scale (amax / 448, 1 for an
 * all-zero vector).  Each code is the nearest e4m3 value of x / scale. */
static float quantise_row_fp8(const void* src, int64_t s0, int32_t head_dim, int32_t src_dtype, uint8_t* codes) {
    float amax = 0.0f;
    for (int d = 0; d < head_dim; ++d) {
        float a = fabsf(load_elem(src, s0 + d, src_dtype));
        if (a > amax) amax = a;
    }
    float sc = oracle_fp8_scale(amax);
    for (int d = 0; d < head_dim; ++d) codes[d] = oracle_fp8_encode(load_elem(src, s0 + d, src_dtype) / sc);
    return sc;
}

typedef struct quant_job {
    const void* src;
    uint8_t* codes;
    float* scales;
    int32_t head_dim, src_dtype;
    int64_t begin, end;
} quant_job;

static void* quant_worker(void* p) {
    const quant_job* j = (const quant_job*)p;
    for (int64_t r = j->begin; r < j->end; ++r)
        j->scales[r] = quantise_row_fp8(j->src, r * j->head_dim, j->head_dim, j->src_dtype,
                                        j->codes + r * j->head_dim);
    return NULL;
}

void oracle_fp8_quantise_rows(const void* src, int64_t num_rows, int32_t head_dim, int32_t src_dtype,
                              uint8_t* codes, float* scales, int32_t nthreads) {
    pthread_once(&g_tables_once, fill_tables);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t)nthreads > num_rows) nthreads = (int32_t)(num_rows > 0 ? num_rows : 1);
    quant_job jobs[256];
    pthread_t th[256];
    for (int i = 0; i < nthreads; ++i) {
        jobs[i] = (quant_job){src, codes, scales, head_dim, src_dtype, num_rows * i / nthreads,
                              num_rows * (i + 1) / nthreads};
        if (nthreads > 1) pthread_create(&th[i], NULL, quant_worker, &jobs[i]);
    }
    if (nthreads == 1) quant_worker(&jobs[0]);
    else
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
}

void oracle_reshape_and_cache(const void* key, const void* value, int64_t key_stride,
                              int64_t value_stride, void* key_cache, void* value_cache,
                              float* key_scales, float* value_scales,
                              const int32_t* slot_mapping, int32_t num_tokens,
                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                              int32_t num_blocks, int32_t src_dtype, int32_t cache_dtype) {
    pthread_once(&g_tables_once, fill_tables);
    const int64_t row = (int64_t)num_kv_heads * head_dim;
    if (key_stride == 0) key_stride = row;
    if (value_stride == 0) value_stride = row;
    const int64_t num_slots = (int64_t)num_blocks * block_size;
    for (int32_t t = 0; t < num_tokens; ++t) {
        const int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= num_slots) continue;
        for (int kv = 0; kv < 2; ++kv) {
            const void* src = kv ? value : key;
            const int64_t stride = kv ? value_stride : key_stride;
            void* dst = kv ? value_cache : key_cache;
            float* scales = kv ? value_scales : key_scales;
            if (cache_dtype == src_dtype) {
                size_t eb = dtype_bytes(src_dtype);
                memcpy((char*)dst + (size_t)(slot * row) * eb,
                       (const char*)src + (size_t)(t * stride) * eb, (size_t)row * eb);
                continue;
            }
            for (int h = 0; h < num_kv_heads; ++h) {
                const int64_t s0 = t * stride + (int64_t)h * head_dim;
                const int64_t d0 = slot * row + (int64_t)h * head_dim;
                if (cache_dtype == OR_F16) {
                    for (int d = 0; d < head_dim; ++d)
                        ((uint16_t*)dst)[d0 + d] = oracle_f32_to_f16(load_elem(src, s0 + d, src_dtype));
                } else { /* FP8 */
                    scales[slot * num_kv_heads + h] =
                        quantise_row_fp8(src, s0, head_dim, src_dtype, (uint8_t*)dst + d0);
                }
            }
        }
    }
}

/* ---------------------------------------------------------------- decode */

typedef struct decode_job {
    float* out;
    const float* query;
    const void* kc;
    const void* vc;
    const float* ks;
    const float* vs;
    const int32_t* bt;
    const int32_t* cl;
    int32_t S, H, Hkv, D, bs, max_ctx, MB, kv_dtype;
    float scale;
    int64_t pair_begin, pair_end;
    /* prefill mode: per-pair context override */
    const int32_t* ctx_override; /* [S*H] or NULL */
    const int32_t* seq_of_row;   /* prefill: row -> sequence, else NULL */
} decode_job;

static float kv_value(const void* cache, const float* scales, int64_t elem, int64_t scale_idx,
                      int32_t dtype) {
    float v = load_elem(cache, elem, dtype);
    if (dtype == OR_FP8) v = v * scales[scale_idx];
    return v;
}

/* One (row, head) of paged_attention_kernel (src/attention/paged_attention.cu:13-82). */
static void decode_one(const decode_job* j, int64_t row, int32_t seq, int32_t head, int32_t ctx) {
    const int32_t D = j->D;
    const int32_t group = j->H / j->Hkv;
    const int32_t kvh = head / group;                                   /* :19 */
    const int32_t nblk = (ctx + j->bs - 1) / j->bs;                     /* :21 */
    const float* q = j->query + (row * j->H + head) * (int64_t)D;       /* :23 */
    float* out = j->out + (row * j->H + head) * (int64_t)D;
    float acc = 0.0f;                                                    /* :25 */
    float max_logit = -1e30f;                                            /* :26 */
    float lanes[32];
    for (int pass = 0; pass < 2; ++pass) {                               /* :29 / :57 */
        for (int32_t b = 0; b < nblk; ++b) {
            const int32_t phys = j->bt[(int64_t)seq * j->MB + b];        /* :30 */
            int32_t tokens = ctx - b * j->bs;                            /* :31 */
            if (tokens > j->bs) tokens = j->bs;
            for (int32_t t = 0; t < tokens; ++t) {
                const int64_t slot = (int64_t)phys * j->bs + t;
                const int64_t off = (slot * j->Hkv + kvh) * (int64_t)D;  /* :34-35 */
                const int64_t sidx = slot * j->Hkv + kvh;
                for (int l = 0; l < 32; ++l) {                           /* :37-40 */
                    float dot = 0.0f;
                    for (int d = l; d < D; d += 32)
                        dot = fmaf(q[d], kv_value(j->kc, j->ks, off + d, sidx, j->kv_dtype), dot);
                    lanes[l] = dot;
                }
                for (int o = 16; o > 0; o >>= 1) {                       /* :43-45 */
                    float nxt[32];
                    for (int l = 0; l < 32; ++l) nxt[l] = lanes[l] + (l + o < 32 ? lanes[l + o] : lanes[l]);
                    memcpy(lanes, nxt, sizeof(nxt));
                }
                float dot = lanes[0];
                if (pass == 0) {                                         /* :47-52 */
                    dot *= j->scale;
                    float prev = max_logit;
                    max_logit = fmaxf(max_logit, dot);
                    acc = acc * expf(prev - max_logit) + expf(dot - max_logit);
                } else {                                                 /* :74-79 */
                    float w = expf(dot * j->scale - max_logit) / (acc + 1e-10f);
                    for (int d = 0; d < D; ++d)
                        out[d] = fmaf(w, kv_value(j->vc, j->vs, off + d, sidx, j->kv_dtype), out[d]);
                }
            }
        }
    }
}

static void* decode_worker(void* arg) {
    const decode_job* j = (const decode_job*)arg;
    for (int64_t p = j->pair_begin; p < j->pair_end; ++p) {
        const int64_t row = p / j->H;
        const int32_t head = (int32_t)(p % j->H);
        int32_t seq, ctx;
        if (j->seq_of_row) {
            seq = j->seq_of_row[row];
            ctx = j->ctx_override[row];
        } else {
            seq = (int32_t)row;
            ctx = j->cl[row];
            if (ctx > j->max_ctx) ctx = j->max_ctx;                      /* :20 */
        }
        if (ctx <= 0) continue;
        decode_one(j, row, seq, head, ctx);
    }
    return NULL;
}

static void run_jobs(decode_job proto, int64_t num_pairs, int32_t nthreads) {
    pthread_once(&g_tables_once, fill_tables);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t)nthreads > num_pairs) nthreads = (int32_t)(num_pairs > 0 ? num_pairs : 1);
    if (nthreads == 1) {
        proto.pair_begin = 0;
        proto.pair_end = num_pairs;
        decode_worker(&proto);
        return;
    }
    pthread_t th[256];
    decode_job jobs[256];
    for (int i = 0; i < nthreads; ++i) {
        jobs[i] = proto;
        jobs[i].pair_begin = num_pairs * i / nthreads;
        jobs[i].pair_end = num_pairs * (i + 1) / nthreads;
        pthread_create(&th[i], NULL, decode_worker, &jobs[i]);
    }
    for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
}

void oracle_paged_decode(float* out, const float* query, const void* key_cache,
                         const void* value_cache, const float* key_scales,
                         const float* value_scales, const int32_t* block_tables,
                         const int32_t* context_lens, int32_t num_seqs, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int32_t max_context_len, int32_t max_blocks_per_seq, float scale,
                         int32_t kv_dtype, int32_t nthreads) {
    decode_job j;
    memset(&j, 0, sizeof(j));
    j.out = out; j.query = query; j.kc = key_cache; j.vc = value_cache;
    j.ks = key_scales; j.vs = value_scales; j.bt = block_tables; j.cl = context_lens;
    j.S = num_seqs; j.H = num_heads; j.Hkv = num_kv_heads; j.D = head_dim; j.bs = block_size;
    j.max_ctx = max_context_len; j.MB = max_blocks_per_seq; j.kv_dtype = kv_dtype; j.scale = scale;
    run_jobs(j, (int64_t)num_seqs * num_heads, nthreads);
}

void oracle_paged_prefill(float* out, const float* query, const void* key_cache,
                          const void* value_cache, const float* key_scales,
                          const float* value_scales, const int32_t* block_tables,
                          const int32_t* context_lens, const int32_t* query_start_loc,
                          int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                          float scale, int32_t kv_dtype, int32_t nthreads) {
    const int32_t rows = query_start_loc[num_seqs];
    int32_t* seq_of_row = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    int32_t* ctx_of_row = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    for (int32_t s = 0; s < num_seqs; ++s) {
        const int32_t q0 = query_start_loc[s], q1 = query_start_loc[s + 1];
        const int32_t qlen = q1 - q0;
        for (int32_t r = q0; r < q1; ++r) {
            seq_of_row[r] = s;
            ctx_of_row[r] = context_lens[s] - qlen + (r - q0) + 1; /* decode at position p sees p+1 keys */
        }
    }
    memset(out, 0, sizeof(float) * (size_t)rows * (size_t)num_heads * (size_t)head_dim);
    decode_job j;
    memset(&j, 0, sizeof(j));
    j.out = out; j.query = query; j.kc = key_cache; j.vc = value_cache;
    j.ks = key_scales; j.vs = value_scales; j.bt = block_tables; j.cl = context_lens;
    j.S = num_seqs; j.H = num_heads; j.Hkv = num_kv_heads; j.D = head_dim; j.bs = block_size;
    j.max_ctx = 0x7FFFFFFF; j.MB = max_blocks_per_seq; j.kv_dtype = kv_dtype; j.scale = scale;
    j.seq_of_row = seq_of_row; j.ctx_override = ctx_of_row;
    run_jobs(j, (int64_t)rows * num_heads, nthreads);
    free(seq_of_row);
    free(ctx_of_row);
}

/* ---------------------------------------------------------------- block ops */

void oracle_copy_blocks(const oracle_plane* planes, int32_t num_planes, int32_t num_layers,
                        int32_t num_blocks, const int32_t* block_pairs, int32_t num_pairs) {
    for (int32_t i = 0; i < num_pairs; ++i) {
        const int32_t src = block_pairs[2 * i], dst = block_pairs[2 * i + 1];
        if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) continue;
        for (int32_t p = 0; p < num_planes; ++p) {
            for (int32_t l = 0; l < num_layers; ++l) {
                char* layer = (char*)planes[p].base + (int64_t)l * planes[p].layer_stride_bytes;
                memmove(layer + (int64_t)dst * planes[p].block_bytes,
                        layer + (int64_t)src * planes[p].block_bytes, (size_t)planes[p].block_bytes);
            }
        }
    }
}

void oracle_swap_blocks(const oracle_plane* planes, int32_t num_planes, int32_t num_layers,
                        int32_t num_dev_blocks, void* host_base, int32_t num_host_blocks,
                        const int32_t* block_pairs, int32_t num_pairs, int32_t direction) {
    int64_t host_block_bytes = 0;
    for (int32_t p = 0; p < num_planes; ++p) host_block_bytes += (int64_t)num_layers * planes[p].block_bytes;
    for (int32_t i = 0; i < num_pairs; ++i) {
        const int32_t src = block_pairs[2 * i], dst = block_pairs[2 * i + 1];
        const int32_t dev = direction == 0 ? src : dst;
        const int32_t host = direction == 0 ? dst : src;
        if (dev < 0 || dev >= num_dev_blocks || host < 0 || host >= num_host_blocks) continue;
        char* h = (char*)host_base + (int64_t)host * host_block_bytes;
        for (int32_t p = 0; p < num_planes; ++p) {
            for (int32_t l = 0; l < num_layers; ++l) {
                char* d = (char*)planes[p].base + (int64_t)l * planes[p].layer_stride_bytes +
                          (int64_t)dev * planes[p].block_bytes;
                if (direction == 0) memcpy(h, d, (size_t)planes[p].block_bytes);
                else memcpy(d, h, (size_t)planes[p].block_bytes);
                h += planes[p].block_bytes;
            }
        }
    }
}
