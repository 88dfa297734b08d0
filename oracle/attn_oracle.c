/*
 * attn_oracle.c -- CPU restatement of diffuse-rs's denoise-step attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker.  The product library never links
 * or calls it; it has no GPU fallback to this code.
 *
 * The reference (agalimova/diffuse-rs v0.4.0) is Rust and cannot be built in
 * this image (no cargo/rustc), so this is a restatement, not a build of it.
 * Each function names the reference lines it follows:
 *
 *   or_visible              src/model/attention.rs:29-57   (visible)
 *   or_attention_row_scalar src/model/attention.rs:140-186 (attention_row_scalar)
 *   or_attention_row_avx2   src/model/attention.rs:267-345 (attention_row_avx2)
 *   hsum_avx2               src/model/ops.rs:352-362       (hsum_avx2)
 *   or_attention            src/model/attention.rs:101-133 (attention: rayon over
 *                           n_head*nq tasks, head = task / nq)
 *   or_rms_norm_inplace     src/model/ops.rs:106-114       (f64 sum of f32 squares)
 *   or_norm_heads           src/model/ops.rs:384-389
 *   or_rms_norm_noscale     src/model/ops.rs:116-124       (Gemma V heads)
 *   or_add_bias             src/model/ops.rs:373-382
 *   or_rope_table           src/model/ops.rs:390-417       (build_rope_cache[_ff])
 *   or_rotate_rows          src/model/ops.rs:419-452       (apply_rope / rotate_rows)
 *   or_cache_store/gather   src/model/cache.rs:62-82       (StepCache::store/gather)
 *   or_split_active         src/model/cache.rs:85-114      (StepCache::split_active)
 *   or_f16_to_f32           src/kernels.rs:46-69           (f16_to_f32)
 *   or_quantize_q8k         src/kernels.rs:79-122          (quantize_rows_q8_k)
 *   or_dequant_q4k          src/kernels.rs:186-215         (dequantize_q4k_row)
 *   or_dequant_q6k          src/kernels.rs:129-163         (dequantize_q6k_row)
 *   or_vec_dot_q4k_q8k      src/kernels.rs:228-308         (the scalar Q4_K x Q8_K
 *                           dot of the reference's tests, candle-core 0.8.4's
 *                           BlockQ4K::vec_dot_unopt)
 *   or_vec_dot_q6k_q8k      src/kernels.rs:313-347         (ggml's generic Q6_K dot)
 *   or_qmatmul              src/model/matmul.rs:120-148    (native_matmul:
 *                           out[t*rows + r] = vec_dot(weight row r, act row t)),
 *                           plus residual_add, src/model/ops.rs:365-370; the
 *                           legacy types' dispatch of matmul.rs:103-106,192-194
 *   or_dequant_q4_0         src/kernels.rs:165-173         (dequantize_q4_0_row)
 *   or_dequant_q8_0         src/kernels.rs:176-183         (dequantize_q8_0_row)
 *   or_dequant_q5_0         ggml's Q5_0 layout (d, qh[4], qs[16]), which
 *                           candle-core 0.8.4's BlockQ5_0 holds
 *   or_quantize_q8_0        ActScratch::q80 (matmul.rs:73-82) ->
 *                           candle-core 0.8.4 BlockQ8_0::from_float, ggml's
 *                           quantize_row_q8_0 (candle is not vendored: the
 *                           published algorithm, restated)
 *   or_vec_dot_q4_0_q8_0,   the generic block dots of ggml / candle-core
 *   or_vec_dot_q5_0_q8_0,   0.8.4 (vec_dot_unopt): per block sumi of the
 *   or_vec_dot_q8_0_q8_0    integer products, sumf += sumi * d_w * d_a
 *   or_post_norm_residual   forward.rs:346-350: norm_rows_inplace
 *                           (ops.rs:141-145 -> rms_norm_inplace :106-114) of
 *                           Wo's output, then residual_add (ops.rs:365-370)
 *
 * Numerics follow Rust semantics: no FMA contraction outside the explicit
 * _mm256_fmadd_ps calls (build with -ffp-contract=off), f32::exp = libm expf,
 * f32::max = fmaxf, iterator .sum() = left fold.
 *
 * Pinning (see tests/test_oracle.py): the reference's own closed-form tests
 * (src/model/tests.rs:55-237), a float64 three-pass brute force, GQA ==
 * repeated-KV MHA, block-diagonal == separate runs, key-permutation
 * invariance, torch scaled_dot_product_attention on CPU, and the committed
 * golden fixtures in tests/golden/.
 */
#include <immintrin.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* AttnShape (attention.rs:10-27).  Option<usize> -> (value, present). */
typedef struct {
    size_t nq, nk, n_head, n_head_kv, head_dim;
    size_t window;
    int has_window;
    size_t prefix;
    int has_prefix;
    float scale;
} or_shape;

/* Rows (attention.rs:65-70).  Empty slice == NULL pointer. */
typedef struct {
    const size_t* pos;
    const size_t* seq;    /* NULL: every row has sequence id 0 (attention.rs:74-76) */
    const size_t* prefix; /* NULL: fall back to the shape's causal_prefix (:151) */
} or_rows;

/* visible() -- attention.rs:36-57. */
int or_visible(size_t qpos, size_t kpos, size_t qseq, size_t kseq, int has_window, size_t window,
               int has_prefix, size_t prefix) {
    if (qseq != kseq) return 0;
    if (has_window) {
        size_t diff = qpos > kpos ? qpos - kpos : kpos - qpos; /* usize::abs_diff */
        if (diff >= window) return 0;
    }
    if (has_prefix && qpos < prefix) return kpos <= qpos;
    return 1;
}

static inline size_t seq_at(const or_rows* r, size_t i) { return r->seq ? r->seq[i] : 0; }

/* Per-(head, query) setup shared by both row kernels (attention.rs:143-152). */
typedef struct {
    size_t hd, qo, kv_stride, kv_off, qpos, qseq, prefix;
    int has_prefix;
} row_ctx;

static row_ctx row_setup(const or_shape* s, const or_rows* qr, size_t head, size_t i) {
    row_ctx c;
    c.hd = s->head_dim;
    c.qo = i * s->n_head * c.hd + head * c.hd;
    c.kv_stride = s->n_head_kv * c.hd;
    c.kv_off = (head / (s->n_head / s->n_head_kv)) * c.hd;
    c.qpos = qr->pos[i];
    c.qseq = seq_at(qr, i);
    if (qr->prefix) {
        c.has_prefix = 1;
        c.prefix = qr->prefix[i];
    } else {
        c.has_prefix = s->has_prefix;
        c.prefix = s->prefix;
    }
    return c;
}

/* attention_row_scalar -- attention.rs:140-186.  Heap accumulator for hd > 256
 * mirrors ACC_STACK (:135-138); the arithmetic is the same either way. */
void or_attention_row_scalar(float* out, const float* q, const float* k, const float* v,
                             const or_shape* s, const or_rows* qr, const or_rows* kr, size_t head,
                             size_t i) {
    row_ctx c = row_setup(s, qr, head, i);
    float acc_stack[256];
    float* acc = c.hd <= 256 ? acc_stack : (float*)malloc(c.hd * sizeof(float));
    for (size_t d = 0; d < c.hd; d++) acc[d] = 0.0f;
    float max = -INFINITY;
    float sum = 0.0f;
    for (size_t j = 0; j < s->nk; j++) {
        if (!or_visible(c.qpos, kr->pos[j], c.qseq, seq_at(kr, j), s->has_window, s->window,
                        c.has_prefix, c.prefix))
            continue;
        size_t ko = j * c.kv_stride + c.kv_off;
        float dot = -0.0f; /* Rust's f32 Sum folds from -0.0 */
        for (size_t d = 0; d < c.hd; d++) dot = dot + q[c.qo + d] * k[ko + d];
        float score = dot * s->scale;
        float new_max = fmaxf(max, score);
        float correction = expf(max - new_max);
        float w = expf(score - new_max);
        sum = sum * correction + w;
        for (size_t d = 0; d < c.hd; d++) acc[d] = acc[d] * correction + w * v[ko + d];
        max = new_max;
    }
    float inv = 1.0f / sum;
    for (size_t d = 0; d < c.hd; d++) out[c.qo + d] = acc[d] * inv;
    if (acc != acc_stack) free(acc);
}

/* hsum_avx2 -- ops.rs:352-362: ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)). */
__attribute__((target("avx2,fma"))) static inline float hsum_avx2(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 a = _mm_add_ps(lo, hi);
    __m128 b = _mm_add_ps(a, _mm_shuffle_ps(a, a, 0xB1)); /* pairs (1,0,3,2) */
    __m128 r = _mm_add_ps(b, _mm_shuffle_ps(b, b, 0x4E)); /* halves (2,3,0,1) */
    return _mm_cvtss_f32(r);
}

/* attention_row_avx2 -- attention.rs:267-345. */
__attribute__((target("avx2,fma"))) void or_attention_row_avx2(
    float* out, const float* q, const float* k, const float* v, const or_shape* s,
    const or_rows* qr, const or_rows* kr, size_t head, size_t i) {
    row_ctx c = row_setup(s, qr, head, i);
    float acc_stack[256];
    float* acc = c.hd <= 256 ? acc_stack : (float*)malloc(c.hd * sizeof(float));
    for (size_t d = 0; d < c.hd; d++) acc[d] = 0.0f;
    float max = -INFINITY;
    float sum = 0.0f;
    for (size_t j = 0; j < s->nk; j++) {
        if (!or_visible(c.qpos, kr->pos[j], c.qseq, seq_at(kr, j), s->has_window, s->window,
                        c.has_prefix, c.prefix))
            continue;
        size_t ko = j * c.kv_stride + c.kv_off;
        __m256 dv = _mm256_setzero_ps();
        size_t d = 0;
        for (; d + 8 <= c.hd; d += 8)
            dv = _mm256_fmadd_ps(_mm256_loadu_ps(q + c.qo + d), _mm256_loadu_ps(k + ko + d), dv);
        float dot = hsum_avx2(dv);
        for (; d < c.hd; d++) dot = dot + q[c.qo + d] * k[ko + d];
        float score = dot * s->scale;
        float new_max = fmaxf(max, score);
        float correction = expf(max - new_max);
        float w = expf(score - new_max);
        sum = sum * correction + w;
        __m256 cv = _mm256_set1_ps(correction);
        __m256 wv = _mm256_set1_ps(w);
        d = 0;
        for (; d + 8 <= c.hd; d += 8) {
            __m256 av = _mm256_loadu_ps(acc + d);
            __m256 vv = _mm256_loadu_ps(v + ko + d);
            _mm256_storeu_ps(acc + d, _mm256_fmadd_ps(wv, vv, _mm256_mul_ps(av, cv)));
        }
        for (; d < c.hd; d++) acc[d] = acc[d] * correction + w * v[ko + d];
        max = new_max;
    }
    __m256 inv = _mm256_set1_ps(1.0f / sum);
    size_t d = 0;
    for (; d + 8 <= c.hd; d += 8)
        _mm256_storeu_ps(out + c.qo + d, _mm256_mul_ps(_mm256_loadu_ps(acc + d), inv));
    for (; d < c.hd; d++) out[c.qo + d] = acc[d] / sum;
    if (acc != acc_stack) free(acc);
}

/* attention() -- attention.rs:101-133.  Tasks 0..n_head*nq, head = task / nq,
 * i = task % nq; each task owns the hd-wide band of out it writes.
 * nthreads <= 0 means "all OpenMP threads".  use_avx2 selects the row kernel
 * the reference dispatches to on an AVX2 host (:113-114). */
void or_attention(float* out, const float* q, const float* k, const float* v, const or_shape* s,
                  const or_rows* qr, const or_rows* kr, int nthreads, int use_avx2) {
    long ntask = (long)(s->n_head * s->nq);
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 16) num_threads(nt)
#endif
    for (long task = 0; task < ntask; task++) {
        size_t head = (size_t)task / s->nq, i = (size_t)task % s->nq;
        if (use_avx2)
            or_attention_row_avx2(out, q, k, v, s, qr, kr, head, i);
        else
            or_attention_row_scalar(out, q, k, v, s, qr, kr, head, i);
    }
    (void)nthreads;
}

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* rms_norm_inplace -- ops.rs:106-114: ss accumulated in f64 over f32 squares,
 * scale = 1 / (sqrt(ss/n + eps) as f32), x = x * scale * w. */
void or_rms_norm_inplace(float* x, const float* w, size_t n, float eps) {
    double ss = 0.0;
    for (size_t i = 0; i < n; i++) {
        float sq = x[i] * x[i];
        ss += (double)sq;
    }
    float scale = 1.0f / (float)sqrt(ss / (double)n + (double)eps);
    for (size_t i = 0; i < n; i++) x[i] = x[i] * scale * w[i];
}

/* norm_heads -- ops.rs:384-389: every hd-wide group of x with the same gain. */
void or_norm_heads(float* x, size_t len, const float* w, size_t hd, float eps) {
    for (size_t o = 0; o + hd <= len; o += hd) or_rms_norm_inplace(x + o, w, hd, eps);
}

/* rms_norm_noscale -- ops.rs:116-124: RMSNorm without a gain (Gemma's V heads,
 * forward.rs:303-308). */
void or_rms_norm_noscale(float* x, size_t n, float eps) {
    double ss = 0.0;
    for (size_t i = 0; i < n; i++) {
        float sq = x[i] * x[i];
        ss += (double)sq;
    }
    float scale = 1.0f / (float)sqrt(ss / (double)n + (double)eps);
    for (size_t i = 0; i < n; i++) x[i] *= scale;
}

/* add_bias -- ops.rs:373-382: the stride-long bias added to each of n rows. */
void or_add_bias(float* x, const float* b, size_t stride, size_t n) {
    for (size_t t = 0; t < n; t++)
        for (size_t i = 0; i < stride; i++) x[t * stride + i] += b[i];
}

/* build_rope_cache_ff -- ops.rs:396-417 (build_rope_cache, :391-393, is ff =
 * NULL): for position t < max_len and i < rope_dim/2, freq_i = 1 /
 * theta^(2i/rope_dim), divided by ff[i] when given, and (sin, cos) of t*freq_i,
 * all in f32 (Rust's f32::powf / sin / cos are libm's powf / sinf / cosf).
 * out[(t*half + i)*2] = sin, out[(t*half + i)*2 + 1] = cos. */
void or_rope_table(float* out, size_t max_len, size_t rope_dim, float theta, const float* ff) {
    size_t half = rope_dim / 2;
    for (size_t t = 0; t < max_len; t++)
        for (size_t i = 0; i < half; i++) {
            float e = 2.0f * (float)i / (float)rope_dim;
            float freq = 1.0f / powf(theta, e);
            if (ff) freq /= ff[i];
            float ang = (float)t * freq;
            out[(t * half + i) * 2] = sinf(ang);
            out[(t * half + i) * 2 + 1] = cosf(ang);
        }
}

/* rotate_rows -- ops.rs:433-452 (apply_rope, :419-431, runs it over Q with
 * n_head and over K with n_head_kv): row t at position pos[t], each head's
 * first rot dims rotate in pairs (i, i + rot/2). */
void or_rotate_rows(float* x, const float* table, const size_t* pos, size_t n, size_t heads,
                    size_t hd, size_t rot) {
    size_t half = rot / 2;
    for (size_t t = 0; t < n; t++)
        for (size_t head = 0; head < heads; head++) {
            float* row = x + t * heads * hd + head * hd;
            for (size_t i = 0; i < half; i++) {
                float sn = table[(pos[t] * half + i) * 2], cs = table[(pos[t] * half + i) * 2 + 1];
                float a = row[i], b = row[half + i];
                row[i] = a * cs - b * sn;
                row[half + i] = a * sn + b * cs;
            }
        }
}

/* StepCache::store -- cache.rs:62-71: row r goes to position positions[r]. */
void or_cache_store(float* ck, float* cv, size_t stride, const size_t* positions, size_t n,
                    const float* k, const float* v) {
    for (size_t r = 0; r < n; r++) {
        memcpy(ck + positions[r] * stride, k + r * stride, stride * sizeof(float));
        memcpy(cv + positions[r] * stride, v + r * stride, stride * sizeof(float));
    }
}

/* StepCache::gather -- cache.rs:73-82. */
void or_cache_gather(const float* ck, const float* cv, size_t stride, const size_t* positions,
                     size_t n, float* out_k, float* out_v) {
    for (size_t r = 0; r < n; r++) {
        memcpy(out_k + r * stride, ck + positions[r] * stride, stride * sizeof(float));
        memcpy(out_v + r * stride, cv + positions[r] * stride, stride * sizeof(float));
    }
}

/* StepCache::split_active -- cache.rs:85-114 with EXTRA_ACTIVE_STEPS = 2
 * (cache.rs:23).  prev_seq/last_changed are the cache's state arrays (length
 * n); active/cached receive ascending positions. */
#define OR_EXTRA_ACTIVE_STEPS 2
void or_split_active(const int32_t* prev_seq, int32_t* last_changed, const int32_t* seq,
                     const uint8_t* is_masked, size_t n, size_t step, size_t vicinity,
                     size_t* active, size_t* n_active, size_t* cached, size_t* n_cached) {
    uint8_t* act = (uint8_t*)calloc(n ? n : 1, 1);
    for (size_t i = 0; i < n; i++) {
        int changed = seq[i] != prev_seq[i];
        if (changed) last_changed[i] = (int32_t)step;
        int recently = last_changed[i] >= 0 &&
                       ((int32_t)step - last_changed[i]) <= (int32_t)OR_EXTRA_ACTIVE_STEPS;
        act[i] = (uint8_t)(changed || is_masked[i] || recently);
    }
    if (vicinity > 0) {
        for (size_t m = 0; m < n; m++) {
            if (!is_masked[m]) continue;
            size_t lo = m > vicinity ? m - vicinity : 0;
            size_t hi = m + vicinity + 1 < n ? m + vicinity + 1 : n;
            for (size_t i = lo; i < hi; i++) act[i] = 1;
        }
    }
    size_t na = 0, nc = 0;
    for (size_t i = 0; i < n; i++) {
        if (act[i])
            active[na++] = i;
        else
            cached[nc++] = i;
    }
    *n_active = na;
    *n_cached = nc;
    free(act);
}


/* ---------------------------------------------------------------------------
 * Quantized matmul: Q4_K / Q6_K weight rows against Q8_K activation rows.
 * Block layouts (src/kernels.rs:9-41): Q4_K 144 bytes {u16 d, u16 dmin,
 * u8 scales[12], u8 qs[128]}; Q6_K 210 bytes {u8 ql[128], u8 qh[64],
 * i8 scales[16], u16 d}; Q8_K 292 bytes {f32 d, i8 qs[256], i16 bsums[16]}.
 * ------------------------------------------------------------------------- */
#define OR_QK 256

typedef struct {
    float d;
    int8_t qs[OR_QK];
    int16_t bsums[OR_QK / 16];
} or_q8k_t;

/* f16_to_f32 -- src/kernels.rs:46-69 (subnormals normalised by shifting). */
float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t e = 0, m = mant;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                e++;
            }
            bits = (sign << 31) | ((113u - e) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | (0xFFu << 23) | (mant ? 0x7FFFFFu : 0u);
    } else {
        bits = (sign << 31) | ((ex + 127u - 15u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* quantize_rows_q8_k -- src/kernels.rs:79-122: per 256-value block, the
 * first value of largest magnitude sets iscale = -128 / max; q = round(iscale
 * x) (half away from zero, as f32::round) capped at 127; d = 1 / iscale;
 * bsums are the sums of 16 consecutive q.  An all-zero block has d = 0. */
void or_quantize_q8k(const float* src, size_t n, size_t cols, or_q8k_t* dst) {
    const size_t nb = cols / OR_QK;
    for (size_t t = 0; t < n; t++)
        for (size_t b = 0; b < nb; b++) {
            const float* xs = src + t * cols + b * OR_QK;
            or_q8k_t* blk = dst + t * nb + b;
            float mx = 0.0f, amax = 0.0f;
            for (int j = 0; j < OR_QK; j++)
                if (amax < fabsf(xs[j])) {
                    amax = fabsf(xs[j]);
                    mx = xs[j];
                }
            memset(blk, 0, sizeof(*blk));
            if (amax == 0.0f) continue;
            const float iscale = -128.0f / mx;
            for (int j = 0; j < OR_QK; j++) {
                float v = roundf(iscale * xs[j]);
                blk->qs[j] = (int8_t)(v < 127.0f ? v : 127.0f);
            }
            for (int j = 0; j < OR_QK / 16; j++) {
                int32_t sm = 0;
                for (int i = 0; i < 16; i++) sm += blk->qs[j * 16 + i];
                blk->bsums[j] = (int16_t)sm;
            }
            blk->d = 1.0f / iscale;
        }
}

/* The 6-bit scales and mins of a Q4_K block (src/kernels.rs:193-201): the 12
 * packed bytes unpacked into sc[8] and mn[8]. */
static void q4k_scales(const uint8_t* packed, uint8_t sc[8], uint8_t mn[8]) {
    uint32_t u[4];
    memcpy(u, packed, 12);
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
    u[3] = ((u[2] >> 4) & k2) | (((u[1] >> 6) & k3) << 4);
    const uint32_t aux = u[1] & k1;
    u[1] = (u[2] & k2) | (((u[0] >> 6) & k3) << 4);
    u[2] = aux;
    u[0] &= k1;
    memcpy(sc, u, 8);
    memcpy(mn, (const uint8_t*)u + 8, 8);
}

/* dequantize_q4k_row -- src/kernels.rs:186-215. */
void or_dequant_q4k(const uint8_t* blocks, size_t nb, float* out) {
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* x = blocks + b * 144;
        uint16_t hd, hm;
        memcpy(&hd, x, 2);
        memcpy(&hm, x + 2, 2);
        const float d = or_f16_to_f32(hd), dmin = or_f16_to_f32(hm);
        uint8_t sc[8], mn[8];
        q4k_scales(x + 4, sc, mn);
        const uint8_t* qs = x + 16;
        for (int j = 0; j < 4; j++)
            for (int k = 0; k < 32; k++) {
                const uint8_t q = qs[j * 32 + k];
                out[b * OR_QK + 64 * j + k] = d * (float)sc[2 * j] * (float)(q & 0xF) - dmin * (float)mn[2 * j];
                out[b * OR_QK + 64 * j + 32 + k] =
                    d * (float)sc[2 * j + 1] * (float)(q >> 4) - dmin * (float)mn[2 * j + 1];
            }
    }
}

/* The 256 signed 6-bit values of a Q6_K block (src/kernels.rs:135-147). */
static void q6k_values(const uint8_t* x, int8_t a[OR_QK]) {
    const uint8_t *ql = x, *qh = x + 128;
    for (int half = 0; half < 2; half++) {
        const uint8_t *l8 = ql + 64 * half, *h8 = qh + 32 * half;
        int8_t* o = a + 128 * half;
        for (int l = 0; l < 32; l++) {
            o[l] = (int8_t)((l8[l] & 0xF) | ((h8[l] & 3) << 4)) - 32;
            o[l + 32] = (int8_t)((l8[l + 32] & 0xF) | (((h8[l] >> 2) & 3) << 4)) - 32;
            o[l + 64] = (int8_t)((l8[l] >> 4) | (((h8[l] >> 4) & 3) << 4)) - 32;
            o[l + 96] = (int8_t)((l8[l + 32] >> 4) | (((h8[l] >> 6) & 3) << 4)) - 32;
        }
    }
}

/* dequantize_q6k_row -- src/kernels.rs:129-163: d * scale[j / 16] * value. */
void or_dequant_q6k(const uint8_t* blocks, size_t nb, float* out) {
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* x = blocks + b * 210;
        uint16_t hd;
        memcpy(&hd, x + 208, 2);
        const float d = or_f16_to_f32(hd);
        const int8_t* sc = (const int8_t*)(x + 192);
        int8_t a[OR_QK];
        q6k_values(x, a);
        for (int j = 0; j < OR_QK; j++) out[b * OR_QK + j] = d * (float)sc[j / 16] * (float)a[j];
    }
}

/* Q4_K x Q8_K (src/kernels.rs:228-308): integer products gathered into eight
 * lanes (element i of the block goes to lane i % 8), each sub-block of 32
 * times its scale; per block sums[l] += d * aux32[l] and sumf -= dmin * sumi
 * (sumi = bsums . mins), with d = f16(x.d) * y.d and dmin = f16(x.dmin) *
 * y.d; finally sumf + sums[0] + ... + sums[7]. */
float or_vec_dot_q4k_q8k(const uint8_t* x, const or_q8k_t* y, size_t nb) {
    float sums[8] = {0}, sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* xb = x + b * 144;
        const or_q8k_t* yb = y + b;
        int8_t a[OR_QK];
        const uint8_t* q4 = xb + 16;
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                a[64 * j + l] = (int8_t)(q4[32 * j + l] & 0xF);
                a[64 * j + 32 + l] = (int8_t)(q4[32 * j + l] >> 4);
            }
        uint8_t sc[8], mn[8];
        q4k_scales(xb + 4, sc, mn);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)yb->bsums[j] * (int32_t)mn[j / 2];
        int32_t aux32[8] = {0};
        for (int i = 0; i < OR_QK; i++) aux32[i % 8] += (int32_t)sc[i / 32] * ((int32_t)yb->qs[i] * a[i]);
        uint16_t hd, hm;
        memcpy(&hd, xb, 2);
        memcpy(&hm, xb + 2, 2);
        const float d = or_f16_to_f32(hd) * yb->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        const float dmin = or_f16_to_f32(hm) * yb->d;
        sumf -= dmin * (float)sumi;
    }
    float tot = 0.0f;  /* sums.iter().sum(): a left fold from zero, added last */
    for (int l = 0; l < 8; l++) tot += sums[l];
    return sumf + tot;
}

/* Q6_K x Q8_K (src/kernels.rs:313-347): per block sumf += d * sumi with d =
 * f16(x.d) * y.d and sumi = sum_j scale[j] * sum of 16 products. */
float or_vec_dot_q6k_q8k(const uint8_t* x, const or_q8k_t* y, size_t nb) {
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* xb = x + b * 210;
        const or_q8k_t* yb = y + b;
        int8_t a[OR_QK];
        q6k_values(xb, a);
        const int8_t* sc = (const int8_t*)(xb + 192);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++)
            for (int k = 0; k < 16; k++) sumi += (int32_t)sc[j] * (int32_t)a[16 * j + k] * (int32_t)yb->qs[16 * j + k];
        uint16_t hd;
        memcpy(&hd, xb + 208, 2);
        sumf += or_f16_to_f32(hd) * yb->d * (float)sumi;
    }
    return sumf;
}

/* ---- the legacy 32-value block types: Q4_0 (18 bytes: f16 d, 16 bytes of
 * nibbles), Q5_0 (22 bytes: f16 d, 32 high bits, 16 bytes of nibbles), Q8_0
 * (34 bytes: f16 d, 32 int8), and Q8_0 activations. */
#define OR_Q0 32

typedef struct {
    uint16_t d;
    int8_t qs[OR_Q0];
} or_q80_t; /* packed: 34 bytes */

/* Value j (0..31) of a legacy block, before the scale: Q4_0 nibble j of
 * byte j % 16 (low nibble for j < 16, high for j >= 16) - 8
 * (kernels.rs:168-170); Q5_0 the same nibble with bit j of qh as bit 4,
 * - 16; Q8_0 the int8 itself (kernels.rs:179-180). */
static int legacy_value(int wtype, const uint8_t* blk, int j) {
    if (wtype == 2) {
        const uint8_t q = blk[2 + (j & 15)];
        return (int)(j < 16 ? (q & 0x0F) : (q >> 4)) - 8;
    }
    if (wtype == 6) {
        uint32_t qh;
        memcpy(&qh, blk + 2, 4);
        const uint8_t q = blk[6 + (j & 15)];
        const int nib = j < 16 ? (q & 0x0F) : (q >> 4);
        return (nib | (int)(((qh >> j) & 1u) << 4)) - 16;
    }
    return (int)(int8_t)blk[2 + j];
}

static size_t legacy_bytes(int wtype) { return wtype == 2 ? 18 : (wtype == 6 ? 22 : 34); }

static void dequant_legacy(int wtype, const uint8_t* blocks, size_t nb, float* out) {
    const size_t bb = legacy_bytes(wtype);
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* x = blocks + b * bb;
        uint16_t hd;
        memcpy(&hd, x, 2);
        const float d = or_f16_to_f32(hd);
        for (int j = 0; j < OR_Q0; j++) out[b * OR_Q0 + j] = d * (float)legacy_value(wtype, x, j);
    }
}
void or_dequant_q4_0(const uint8_t* blocks, size_t nb, float* out) { dequant_legacy(2, blocks, nb, out); }
void or_dequant_q5_0(const uint8_t* blocks, size_t nb, float* out) { dequant_legacy(6, blocks, nb, out); }
void or_dequant_q8_0(const uint8_t* blocks, size_t nb, float* out) { dequant_legacy(8, blocks, nb, out); }

/* f32 -> f16, round to nearest even (the half crate's f16::from_f32);
 * finite inputs below 65520 in magnitude, as a block scale amax / 127 is. */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to inf */
    if (ax < 0x38800000u) {                                     /* f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;            /* below half the smallest subnormal */
        /* |f| = m * 2^(e - 150); in units of the smallest subnormal 2^-24
         * that is m >> (126 - e), rounded to nearest even (a round-up to
         * 1024 is the smallest normal's encoding) */
        const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t sh = 126u - e; /* 14 .. 24 */
        const uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        const uint32_t r = q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
        return (uint16_t)(sign | r);
    }
    const uint32_t e = (ax >> 23) - 112, m = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* (a carry into the exponent is right) */
    return (uint16_t)(sign | h);
}
uint16_t or_f32_to_f16(float f) { return f32_to_f16(f); }

/* quantize_row_q8_0 (candle-core 0.8.4 BlockQ8_0::from_float, as ggml):
 * per 32 values amax = max |x| (f32::max, which ignores a NaN), d = amax /
 * 127, id = d != 0 ? 1 / d : 0, q = round(x * id) (half away from zero,
 * saturating to int8 as Rust's `as i8`), stored d = f16(d). */
void or_quantize_q8_0(const float* src, size_t n, size_t cols, or_q80_t* dst) {
    const size_t nb = cols / OR_Q0;
    for (size_t t = 0; t < n; t++)
        for (size_t b = 0; b < nb; b++) {
            const float* xs = src + t * cols + b * OR_Q0;
            or_q80_t* y = dst + t * nb + b;
            float amax = 0.0f;
            for (int j = 0; j < OR_Q0; j++) amax = fmaxf(amax, fabsf(xs[j]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            y->d = f32_to_f16(d);
            for (int j = 0; j < OR_Q0; j++) {
                float v = roundf(xs[j] * id);
                if (v != v) v = 0.0f;
                v = v > 127.0f ? 127.0f : (v < -128.0f ? -128.0f : v);
                y->qs[j] = (int8_t)v;
            }
        }
}

/* The generic legacy block dots (ggml / candle-core 0.8.4 vec_dot_unopt):
 * sumf += (float)sumi * d_w * d_a per block, in block order. */
static float vec_dot_legacy_q8_0(int wtype, const uint8_t* x, const or_q80_t* y, size_t nb) {
    const size_t bb = legacy_bytes(wtype);
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* xb = x + b * bb;
        int32_t sumi = 0;
        for (int j = 0; j < OR_Q0; j++) sumi += legacy_value(wtype, xb, j) * (int32_t)y[b].qs[j];
        uint16_t hd;
        memcpy(&hd, xb, 2);
        sumf += (float)sumi * or_f16_to_f32(hd) * or_f16_to_f32(y[b].d);
    }
    return sumf;
}
float or_vec_dot_q4_0_q8_0(const uint8_t* x, const or_q80_t* y, size_t nb) { return vec_dot_legacy_q8_0(2, x, y, nb); }
float or_vec_dot_q5_0_q8_0(const uint8_t* x, const or_q80_t* y, size_t nb) { return vec_dot_legacy_q8_0(6, x, y, nb); }
float or_vec_dot_q8_0_q8_0(const uint8_t* x, const or_q80_t* y, size_t nb) { return vec_dot_legacy_q8_0(8, x, y, nb); }

/* Gemma's step after Wo (forward.rs:346-350): each of the n rows of cur
 * ([n][e]) RMS-normalised in place with gain w and eps (norm_rows_inplace,
 * ops.rs:141-145 -> rms_norm_inplace :106-114), then residual_add
 * (ops.rs:365-370): cur += residual. */
void or_post_norm_residual(float* cur, const float* w, const float* residual, size_t n, size_t e, float eps) {
    for (size_t t = 0; t < n; t++) {
        or_rms_norm_inplace(cur + t * e, w, e, eps);
        if (residual)
            for (size_t i = 0; i < e; i++) cur[t * e + i] = cur[t * e + i] + residual[t * e + i];
    }
}

/* native_matmul (src/model/matmul.rs:120-148) over f32 activations quantized
 * to Q8_K (ActScratch::q8k, matmul.rs:64-71): out[t*rows + r] = vec_dot(weight
 * row r, activation row t); with residual (non-NULL), then residual_add
 * (ops.rs:365-370): out += residual.  wtype 12 = Q4_K, 14 = Q6_K (GGML ids). */
void or_qmatmul(int wtype, const uint8_t* w, size_t rows, size_t cols, const float* act, size_t n,
                float* out, const float* residual) {
    if (wtype == 2 || wtype == 6 || wtype == 8) {
        /* Q4_0 / Q5_0 / Q8_0 weights over Q8_0 activations (matmul.rs:103-106,
         * 192-194: ActScratch::q80) */
        const size_t nb0 = cols / OR_Q0, bb0 = legacy_bytes(wtype);
        or_q80_t* q0 = (or_q80_t*)malloc((n * nb0 > 0 ? n * nb0 : 1) * sizeof(or_q80_t));
        or_quantize_q8_0(act, n, cols, q0);
#pragma omp parallel for schedule(static)
        for (long long r = 0; r < (long long)rows; r++)
            for (size_t t = 0; t < n; t++) {
                float v = vec_dot_legacy_q8_0(wtype, w + (size_t)r * nb0 * bb0, q0 + t * nb0, nb0);
                if (residual) v += residual[t * rows + (size_t)r];
                out[t * rows + (size_t)r] = v;
            }
        free(q0);
        return;
    }
    const size_t nb = cols / OR_QK, bb = wtype == 12 ? 144 : 210;
    or_q8k_t* q = (or_q8k_t*)malloc((n * nb > 0 ? n * nb : 1) * sizeof(or_q8k_t));
    or_quantize_q8k(act, n, cols, q);
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < (long long)rows; r++)
        for (size_t t = 0; t < n; t++) {
            const uint8_t* wr = w + (size_t)r * nb * bb;
            float v = wtype == 12 ? or_vec_dot_q4k_q8k(wr, q + t * nb, nb) : or_vec_dot_q6k_q8k(wr, q + t * nb, nb);
            if (residual) v += residual[t * rows + (size_t)r];
            out[t * rows + (size_t)r] = v;
        }
    free(q);
}
