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
