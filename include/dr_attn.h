/*
 * dr_attn.h -- C ABI of the MI355X (gfx950) denoise-step attention library.
 *
 * This is the drop-in boundary for diffuse-rs's per-denoise-step attention
 * (agalimova/diffuse-rs v0.4.0).  Each entry point names the reference
 * interface it replaces.  Plain pointers and sizes only: Rust binds
 * `usize` as `size_t`, `Option<usize>` as `dr_opt_usize`, and an empty slice
 * as (NULL, 0).
 *
 * Status codes: every fallible entry point returns DR_OK (0) or a nonzero
 * dr_status; dr_last_error() gives a message for the calling thread.  The
 * reference's attention() is infallible and panics on bad input; a Rust shim
 * maps a nonzero status to panic!().
 *
 * Threading: a dr_ctx owns one HIP stream and serves one host thread at a
 * time (mirrors the reference's single-threaded `&mut Model` discipline,
 * server.rs:350-351): an entry point that uses its workspaces, split tickets
 * or launch record (attention, step, qmatmul, dr_ctx_set_stream) returns
 * DR_ERR_BUSY to a second thread that calls while the first is inside.
 * dr_attention() uses one process-wide context, serialised internally.
 */
#ifndef DR_ATTN_H
#define DR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    DR_OK = 0,
    DR_ERR_INVALID = 1,     /* bad shape, length or argument */
    DR_ERR_NO_DEVICE = 2,   /* no HIP device visible */
    DR_ERR_OOM = 3,         /* device allocation failed */
    DR_ERR_HIP = 4,         /* a HIP runtime call failed */
    DR_ERR_UNSUPPORTED = 5, /* valid for the reference, not built here (e.g. head_dim > 512) */
    DR_ERR_BUSY = 6         /* the context is in use by another host thread */
} dr_status;

/* Option<usize>: present == 0 means None. */
typedef struct {
    size_t value;
    uint8_t present;
} dr_opt_usize;

/* AttnShape -- src/model/attention.rs:10-27. */
typedef struct {
    size_t nq;
    size_t nk;
    size_t n_head;
    size_t n_head_kv;
    size_t head_dim;
    dr_opt_usize sliding_window; /* key visible iff |qpos - kpos| < window */
    dr_opt_usize causal_prefix;  /* queries with qpos < prefix see kpos <= qpos */
    float scale;
} dr_attn_shape;

/* Rows -- src/model/attention.rs:65-70.  pos has one entry per row; seq and
 * prefix may be empty ((NULL, 0)): empty seq = every row in sequence 0
 * (:74-76), empty prefix = the shape's causal_prefix (:151). */
typedef struct {
    const size_t* pos;
    size_t pos_len;
    const size_t* seq;
    size_t seq_len;
    const size_t* prefix;
    size_t prefix_len;
} dr_rows;

/* Message for the last failing call on this thread ("" if none). */
const char* dr_last_error(void);

/* Library and ABI version, "MAJOR.MINOR.PATCH". */
const char* dr_version(void);

/* Number of visible HIP devices (0 on a host without a GPU; never fails). */
int dr_device_count(void);

/*
 * Literal drop-in for
 *   pub(crate) fn attention(out: &mut [f32], q: &[f32], k: &[f32], v: &[f32],
 *                           s: AttnShape, qr: Rows, kr: Rows)
 * at src/model/attention.rs:106 (caller: src/model/forward.rs:343).
 *
 * Host pointers, synchronous: uploads q/k/v and row metadata, runs the fused
 * kernel on device 0, downloads out.  The kernel takes Q, K and V as bf16
 * hi + lo halves (the hi/lo kernel of DR_PRECISION_HILO layers): scores and
 * values are f32-accurate, so out matches the reference's f32 attention to
 * the bar of the f32 computation under every mask, also where a row sees
 * only a few keys.  The host copies dominate the call.  Layouts as the reference:
 * q [nq][n_head][head_dim], k and v [nk][n_head_kv][head_dim], out
 * [nq][n_head * head_dim], all f32 row-major; out is fully overwritten.
 * Lengths are checked as the reference's debug_asserts (:107-109) and
 * slicing would; a query that sees no key yields NaN, as the reference's
 * 0 * (1/0) does (:181-185).
 */
int dr_attention(float* out, size_t out_len, const float* q, size_t q_len, const float* k,
                 size_t k_len, const float* v, size_t v_len, dr_attn_shape s, dr_rows qr,
                 dr_rows kr);

/* ------------------------------------------------------------------------- *
 * Device-resident path: a context (device + stream), the inter-step KV cache
 * kept in HBM as bf16, per-pass row metadata, and attention that reads the
 * cache directly.  All float* below are DEVICE pointers (hipMalloc'd or torch
 * tensors); work is enqueued on the context's stream and is asynchronous
 * unless stated otherwise.
 * ------------------------------------------------------------------------- */

typedef struct dr_ctx dr_ctx;

/* Create a context on `device` with its own (default-priority) stream. */
int dr_ctx_create(int device, dr_ctx** out);
/* Use the caller's hipStream_t (cast to void*; NULL: the context's own) for
 * later calls.  The new stream first waits (on the device) for the work
 * already queued on the old one, so the context's workspaces and split
 * tickets are never in use on both; the old stream must still exist.  (When
 * either stream is under graph capture, no wait is inserted: the graph's own
 * dependencies order the calls.) */
int dr_ctx_set_stream(dr_ctx* ctx, void* stream);
/* The hipStream_t the context enqueues on. */
void* dr_ctx_stream(dr_ctx* ctx);
int dr_ctx_synchronize(dr_ctx* ctx);
/* Release the caller's hold on ctx.  Every pass, cache and RoPE table made on
 * ctx holds it too: its stream and workspaces are freed once ctx and all of
 * them have been destroyed, in any order (a garbage collector may finalize
 * the context first).  Workspaces that grew are freed only here, never while
 * a captured hipGraph could still use them. */
void dr_ctx_destroy(dr_ctx* ctx);

/*
 * PassRows -- src/model/attention.rs:79-85, built once per forward pass in
 * src/model/forward.rs:87-101: the active (recomputed) sequence positions,
 * ascending, copied to the device once and reused by every layer's
 * dr_cache_store and dr_attention_cached.  Queries are the active rows.
 */
typedef struct dr_pass dr_pass;
int dr_pass_create(dr_ctx* ctx, const size_t* active, size_t n_active, dr_pass** out);
/* Replace the positions (e.g. for the next denoise step); synchronous upload. */
int dr_pass_set(dr_pass* pass, const size_t* active, size_t n_active);
size_t dr_pass_len(const dr_pass* pass);
/* Copy the pass's positions (ascending) into out (host, room for cap
 * entries, cap >= dr_pass_len); waits for the context's stream.  Reads back
 * what dr_cache_split_active_dev wrote (ActiveSplit's lists, cache.rs:7-10). */
int dr_pass_positions(const dr_pass* pass, size_t* out, size_t cap);
void dr_pass_destroy(dr_pass* pass);

/*
 * StepCache -- src/model/cache.rs:25-115.  Per layer, per batch slot, K and V
 * for every sequence position 0..n_total, stored as bf16 in HBM (K row-major
 * per KV head, V transposed per KV head).  StepCache::new (:44-54) takes
 * per-layer strides n_head_kv * head_dim (forward.rs:267); here the two
 * factors are given separately.  n_batch > 1 holds several independent
 * streams (e.g. the conditional and unconditional CFG streams, each of which
 * has its own StepCache in sampler.rs:432-434) so one launch serves both.
 * Storage is zero-initialised.  vicinity starts at 0 (cache.rs:40).
 */
typedef struct dr_step_cache dr_step_cache;
int dr_cache_create(dr_ctx* ctx, size_t n_total, size_t n_layer, const size_t* n_head_kv,
                    const size_t* head_dim, size_t n_batch, dr_step_cache** out);
void dr_cache_destroy(dr_step_cache* cache);

/* Score precision of one cache layer; no counterpart in the reference, whose
 * StepCache holds f32 K (cache.rs:25-54) and whose attention forms f32 scores
 * (attention.rs:289-331).  DR_PRECISION_BF16 (the default): K is kept as
 * bf16 and the scores come from bf16 Q and K, within 1e-2 of the reference
 * at the usual 1/sqrt(head_dim) scale.  DR_PRECISION_HILO: the layer also
 * keeps the lo halves bf16(x - bf16(x)) of K and V in two more planes (twice
 * the layer's cache memory, written by every later store), and its attention
 * forms S = Qh.Kh + Qh.Kl + Ql.Kh from the bf16 hi/lo halves of Q and K and
 * P.(Vh + Vl): scores accurate to ~2^-16 and values to ~2^-17, for layers
 * whose scale makes bf16 too coarse -- Gemma's kq_scale 1.0
 * (forward.rs:338-341), where the softmax is nearly one-hot and bf16 moves
 * outputs by ~0.15.  Set it before storing the layer's rows (rows stored
 * earlier have zero lo halves); DR_PRECISION_BF16 frees the planes.  Hi/lo
 * layers run without masks or with position masks (window, causal prefix,
 * query sequence ids). */
#define DR_PRECISION_BF16 0
#define DR_PRECISION_HILO 1
int dr_cache_set_precision(dr_step_cache* cache, size_t layer, int precision);
/* dr_cache_create with each layer's score precision given up front
 * (precision: n_layer entries, DR_PRECISION_BF16 or DR_PRECISION_HILO; NULL =
 * all bf16), so a binding sets it from the layer's attention scale when it
 * builds the cache: DiffusionGemma, whose layers all use kq_scale 1.0
 * (forward.rs:338-341), takes DR_PRECISION_HILO for every layer.  A cached
 * attention call (dr_attention_cached, _noalloc, _step, _step_epi) on a
 * DR_PRECISION_BF16 layer with |scale| * sqrt(head_dim) > 2 fails with
 * DR_ERR_UNSUPPORTED, since bf16 scores miss the 1e-2 bar there (outputs move
 * by ~0.24 at Gemma's 1.0), unless a kernel family was forced with
 * dr_ctx_set_kernel (then the caller accepts bf16 scores). */
int dr_cache_create_layers(dr_ctx* ctx, size_t n_total, size_t n_layer, const size_t* n_head_kv,
                           const size_t* head_dim, const int* precision, size_t n_batch,
                           dr_step_cache** out);

/* StepCache::store (cache.rs:62-71) for the pass's active positions: row r of
 * k/v ([n_active][n_head_kv][head_dim] f32, device) goes to position
 * active[r].  If k_norm_w (device, head_dim f32) is non-NULL each K head is
 * first RMS-normalised with that gain and eps (norm_heads, ops.rs:384-389, as
 * forward.rs:300-302 does before the store). */
int dr_cache_store(dr_step_cache* cache, size_t layer, size_t batch, const dr_pass* pass,
                   const float* k, const float* v, const float* k_norm_w, float eps);

/* StepCache::gather (cache.rs:73-82): rows at `positions` (host array) into
 * out_k/out_v (device, f32, [n][n_head_kv][head_dim]).  Values are the bf16
 * cache contents widened to f32. */
int dr_cache_gather(dr_step_cache* cache, size_t layer, size_t batch, const size_t* positions,
                    size_t n, float* out_k, float* out_v);

/* StepCache::update_seq (cache.rs:56-59) for one batch slot (host data). */
int dr_cache_update_seq(dr_step_cache* cache, size_t batch, const int32_t* seq, size_t n);
/* StepCache::split_active (cache.rs:85-114) for one batch slot.  active and
 * cached must each have room for n entries; both come back ascending. */
int dr_cache_split_active(dr_step_cache* cache, size_t batch, const int32_t* seq,
                          const uint8_t* is_masked, size_t n, size_t step, size_t* active,
                          size_t* n_active, size_t* cached, size_t* n_cached);
/* The same split on caller-owned state, with no device involved: prev_seq and
 * last_changed are StepCache's arrays (cache.rs:29-31, initially all -1),
 * length n; last_changed is updated in place. */
int dr_split_active(const int32_t* prev_seq, int32_t* last_changed, const int32_t* seq,
                    const uint8_t* is_masked, size_t n, size_t step, size_t vicinity,
                    size_t* active, size_t* n_active, size_t* cached, size_t* n_cached);
/* StepCache::update_seq (cache.rs:56-59) from a device array seq [n_total]
 * (int32), ordered on the context's stream. */
int dr_cache_update_seq_dev(dr_step_cache* cache, size_t batch, const int32_t* seq, size_t n);
/* StepCache::split_active (cache.rs:85-114) computed on the device from
 * device arrays seq [n] (int32) and is_masked [n] (uint8): the active
 * positions are written into pass `active` and the cached ones into pass
 * `cached` (their device position arrays, ascending), ready for
 * dr_attention_cached / dr_cache_store / dr_attention_step, with no host
 * loop and no upload of index lists.  The two counts come back through one
 * small device-to-host copy (the launches that follow are sized by them).
 * The slot's split state (cache.rs:29-31) moves to the device on first use
 * and back on the next host-side dr_cache_split_active / dr_cache_update_seq,
 * so the two kinds of call may be mixed on one slot. */
int dr_cache_split_active_dev(dr_step_cache* cache, size_t batch, const int32_t* seq,
                              const uint8_t* is_masked, size_t n, size_t step, dr_pass* active,
                              dr_pass* cached, size_t* n_active, size_t* n_cached);
/* StepCache.vicinity (cache.rs:37-41). */
int dr_cache_set_vicinity(dr_step_cache* cache, size_t batch, size_t vicinity);
/* StepCache.initialized (cache.rs:33). */
int dr_cache_initialized(const dr_step_cache* cache, size_t batch);

/* One batch slot of a cached attention call. */
typedef struct {
    const float* q; /* device, [n_active][n_head][head_dim] f32 */
    float* out;     /* device, [n_active][n_head * head_dim] f32, overwritten */
    const dr_pass* pass;
} dr_batch_item;

/*
 * Cached attention: the attention() call of attention_block
 * (src/model/forward.rs:312-343) with the gather/concatenate of
 * :312-317 removed.  Item b's queries (its pass's active positions) attend
 * to cache slot b's keys at every position 0..n_total; call dr_cache_store
 * for the active rows first, as forward.rs:318-320 does.  The reference's
 * key order [cached | active] and this one differ only in summation order:
 * masking is by position (attention.rs:29-35).  sliding_window,
 * causal_prefix and scale are AttnShape's (forward.rs:327-342).  If q_norm_w
 * (device, head_dim f32) is non-NULL each query head is RMS-normalised with
 * it first (forward.rs:297-299).  n_items <= the cache's n_batch and <= 8.
 */
int dr_attention_cached(dr_step_cache* cache, size_t layer, const dr_batch_item* items,
                        size_t n_items, size_t n_head, dr_opt_usize sliding_window,
                        dr_opt_usize causal_prefix, float scale, const float* q_norm_w,
                        float q_norm_eps);

/*
 * dr_attention_cached without allocating: the same arguments, checks,
 * kernels and results, but the device memory the call uses beyond its
 * inputs and outputs (the key-split partials, and on a DR_PRECISION_HILO
 * layer whose Q epilogue runs as a pass of its own, the Q copy it writes)
 * goes to a fixed 64 MiB device array that the library holds on every GPU it
 * runs on until the process ends, instead of the context's growing
 * workspaces.  No hipMalloc, hipFree
 * or allocating library routine runs in the call, so it can be made under
 * hipGraph capture, in serving loops and in harnesses that forbid
 * allocation.  A plan that needs more than 64 MiB (far beyond the
 * configurations here: DiffusionGemma's 512-wide global layer needs 34 MB)
 * returns DR_ERR_INVALID.  Nothing in the array needs to start at zero.
 * Every call on a GPU shares that GPU's array: a call on another stream than
 * the previous call on that GPU (from any context) first waits, on the
 * device, for that call's kernels, through an event made at dr_ctx_create,
 * so no two calls use the array at once.  Calls captured into a hipGraph are
 * ordered by the graph alone: two captured calls on one GPU must not run
 * concurrently.
 * This entry point has no counterpart in the reference; it is for callers
 * that cannot allocate.
 */
int dr_attention_cached_noalloc(dr_step_cache* cache, size_t layer, const dr_batch_item* items,
                                size_t n_items, size_t n_head, dr_opt_usize sliding_window,
                                dr_opt_usize causal_prefix, float scale, const float* q_norm_w,
                                float q_norm_eps);

/* One batch slot of a denoise-step layer: queries and the active K/V rows. */
typedef struct {
    const float* q; /* device, [n_active][n_head][head_dim] f32 */
    float* out;     /* device, [n_active][n_head * head_dim] f32, overwritten */
    const dr_pass* pass;
    const float* k; /* device, [n_active][n_head_kv][head_dim] f32 (RoPE applied) */
    const float* v; /* device, [n_active][n_head_kv][head_dim] f32 */
} dr_step_item;

/*
 * One denoise-step attention layer with its cache update: the per-layer block
 * of attention_block (src/model/forward.rs:296-343), norm_heads(k, k_norm) +
 * cache.store(active) + gather(cached) ++ active + attention().  For item b
 * (cache batch slot b) the active rows k / v are RMS-normalised with
 * k_norm_w when it is non-NULL (K only), stored into the cache at the
 * pass's positions, and the queries attend over every position 0..n_total,
 * the active ones with the rows just given.  This is dr_cache_store per item
 * followed by dr_attention_cached.  Other arguments as dr_attention_cached.
 */
int dr_attention_step(dr_step_cache* cache, size_t layer, const dr_step_item* items,
                      size_t n_items, size_t n_head, dr_opt_usize sliding_window,
                      dr_opt_usize causal_prefix, float scale, const float* q_norm_w,
                      float q_norm_eps, const float* k_norm_w, float k_norm_eps);

/*
 * The Q/K/V epilogue of attention_block (src/model/forward.rs:291-310), on
 * device rows and in place, before dr_attention_step / dr_cache_store +
 * dr_attention_cached (which are then called without norms):
 *   add_bias(q, bq), (k, bk), (v, bv)           ops.rs:373-382 (NULL: none)
 *   norm_heads(q, q_norm_w), (k, k_norm_w)       ops.rs:384-389 (NULL: none)
 *   Gemma: rms_norm_noscale of each V head       ops.rs:116-124 (v_norm != 0)
 *   apply_rope(q, k, rope, pass positions)       ops.rs:419-452 (rope NULL: none)
 * q is [n][n_head][head_dim], k and v [n][n_head_kv][head_dim] f32 (device),
 * row t at the pass's t-th position; the biases are [heads * head_dim] and
 * the norm gains [head_dim] (device); eps is rms_norm_eps.  head_dim <= 512.
 */
typedef struct dr_rope dr_rope;
/* build_rope_cache_ff (src/model/ops.rs:396-417; build_rope_cache :391-393
 * when freq_factors is NULL): the f32 (sin, cos) table of positions
 * 0..max_len and the rope_dim/2 frequency pairs, built on the host exactly
 * as the reference builds it and kept on the device.  freq_factors: host,
 * rope_dim/2 floats, or NULL. */
int dr_rope_create(dr_ctx* ctx, size_t max_len, size_t rope_dim, float theta,
                   const float* freq_factors, dr_rope** out);
void dr_rope_destroy(dr_rope* rope);
int dr_qkv_epilogue(dr_ctx* ctx, const dr_pass* pass, float* q, float* k, float* v, size_t n_head,
                    size_t n_head_kv, size_t head_dim, const float* bq, const float* bk,
                    const float* bv, const float* q_norm_w, const float* k_norm_w, int v_norm,
                    float eps, const dr_rope* rope);

/* The operands of the Q/K/V epilogue (all device pointers, NULL = none). */
typedef struct {
    const float* bq;       /* [n_head * head_dim] */
    const float* bk;       /* [n_head_kv * head_dim] */
    const float* bv;       /* [n_head_kv * head_dim] */
    const float* q_norm_w; /* [head_dim] */
    const float* k_norm_w; /* [head_dim] */
    int v_norm;            /* Gemma: unweighted RMSNorm of each V head */
    float eps;             /* rms_norm_eps */
    const dr_rope* rope;   /* rope_dim a multiple of 8 */
} dr_epilogue;
/* dr_attention_step with the Q/K/V epilogue of attention_block
 * (src/model/forward.rs:291-343) folded into its passes: each item's k / v
 * rows get bias, norm and (K) RoPE inside the cache store, and its q rows get
 * bias, QK-norm and RoPE where the attention reads them, at the pass's
 * positions.  No separate pass over q, k or v; the item buffers are read,
 * never written.  Same result as dr_qkv_epilogue followed by
 * dr_attention_step. */
int dr_attention_step_epi(dr_step_cache* cache, size_t layer, const dr_step_item* items,
                          size_t n_items, size_t n_head, dr_opt_usize sliding_window,
                          dr_opt_usize causal_prefix, float scale, const dr_epilogue* epi);

/* One batch slot of a denoise-step layer whose Q, K and V rows lie at row
 * strides: the rows of a fused QKV projection (Qkv::Fused,
 * src/model/forward.rs:281-289), [n][n_head*hd + 2*n_head_kv*hd], are read
 * in place with q = row, k = row + n_head*hd, v = k + n_head_kv*hd and both
 * strides the fused row length -- no copy into separate Q / K / V buffers. */
typedef struct {
    const float* q;   /* device, row t at q + t * q_stride: [n_head][head_dim] f32 */
    float* out;       /* device, [n_active][n_head * head_dim] f32, overwritten */
    const dr_pass* pass;
    const float* k;   /* device, row t at k + t * kv_stride: [n_head_kv][head_dim] f32 */
    const float* v;   /* device, row t at v + t * kv_stride */
    size_t q_stride;  /* elements between Q rows, a multiple of 4 (0: n_head * head_dim) */
    size_t kv_stride; /* elements between K rows and between V rows (0: n_head_kv * head_dim) */
} dr_step_item_rows;
/* dr_attention_step_epi on strided rows (every item with the same strides);
 * epi may be NULL (no epilogue: dr_attention_step without norms).  Same
 * results as copying the rows apart and calling dr_attention_step_epi. */
int dr_attention_step_rows(dr_step_cache* cache, size_t layer, const dr_step_item_rows* items,
                           size_t n_items, size_t n_head, dr_opt_usize sliding_window,
                           dr_opt_usize causal_prefix, float scale, const dr_epilogue* epi);

/* ---- the projection after the attention: Wo on GGUF quantized weights */
#define DR_WTYPE_Q4K 12 /* GGML type ids */
#define DR_WTYPE_Q6K 14
#define DR_WTYPE_Q4_0 2 /* the legacy 32-value block types, over Q8_0 activations */
#define DR_WTYPE_Q5_0 6
#define DR_WTYPE_Q8_0 8
/* MatWeight::forward for Q4_K / Q6_K weights (src/model/matmul.rs:94-106):
 * the activations are quantized to Q8_K (ActScratch::q8k, matmul.rs:64-71,
 * quantize_rows_q8_k of src/kernels.rs:79-122) and native_matmul
 * (matmul.rs:120-148) takes out[t*rows + r] = vec_dot(weight row r,
 * activation row t); with residual non-NULL, residual_add (ops.rs:365-370)
 * follows, as attention_block does after Wo (src/model/forward.rs:345-350).
 * w: rows x cols/256 GGUF blocks (144 bytes for Q4_K, 210 for Q6_K), act
 * [n][cols], out and residual [n][rows] f32, all device pointers on the
 * context's stream; residual may equal out.  cols must be a multiple of 256,
 * and Q4_K blocks must start 16-byte aligned.
 * The integer part of each block dot (src/kernels.rs:228-347) is exact; the
 * f32 combine of the per-block integers with the block scales rounds in its
 * own order, so each output is within (nb + 12) * 2^-24 * S of the exact dot
 * (nb = cols / 256, S the sum over blocks of |d * scaled dot| + |dmin *
 * mins dot|), as the reference's scalar dot is. */
int dr_qmatmul(dr_ctx* ctx, int wtype, const void* w, size_t rows, size_t cols, const float* act,
               size_t n, float* out, const float* residual);
/* The same for MatWeight::Q40 (matmul.rs:103-106, Q4_0 weights) and the
 * expert types of ExpertMat (matmul.rs:156-158, 192-194: Q4_0, Q5_0, Q8_0):
 * wtype DR_WTYPE_Q4_0 / _Q5_0 / _Q8_0, weights rows x cols/32 GGUF blocks of
 * 18 / 22 / 34 bytes (2-byte aligned), cols a multiple of 32; the
 * activations are quantized to Q8_0 (ActScratch::q80, matmul.rs:73-82:
 * candle-core 0.8.4's BlockQ8_0::from_float, see dr_quantize_q8_0) and each
 * output is vec_dot(weight row r, activation row t): per block d_w * d_a times
 * the exact integer dot, summed over blocks in f32; within (cols / 32 + 12) *
 * 2^-24 * sum_i |w_i a_i| of the exact value, as the reference's own f32
 * sum is.  act must be 16-byte aligned. */

/* Wo with Gemma's post-attention RMSNorm (src/model/forward.rs:346-350): out =
 * rms_norm_inplace(act . W^T, norm_w, eps) (ops.rs:106-114, each of the n
 * output rows of `rows` values, f64 sum of f32 squares) + residual (NULL:
 * none).  Any weight type of dr_qmatmul; norm_w: [rows] device floats.  One
 * more launch after the matmul (a row's norm needs the whole row). */
int dr_qmatmul_post_norm(dr_ctx* ctx, int wtype, const void* w, size_t rows, size_t cols, const float* act,
                         size_t n, float* out, const float* residual, const float* norm_w, float eps);

/* ExpertMat::forward_expert (src/model/matmul.rs:176-213): dr_qmatmul on
 * expert `expert`'s slice of a [n_expert][rows][cols] stack of Q4_K / Q6_K
 * blocks (expert_matmul, matmul.rs:201-213).  expert >= n_expert is
 * DR_ERR_INVALID ("expert index out of range", matmul.rs:208). */
int dr_qmatmul_expert(dr_ctx* ctx, int wtype, const void* w, size_t n_expert, size_t expert, size_t rows,
                      size_t cols, const float* act, size_t n, float* out, const float* residual);

/* quantize_rows_q8_k (src/kernels.rs:79-122), the quantization dr_qmatmul
 * applies to its activations: act [n][cols] f32 (cols a multiple of 256) ->
 * out, n * cols / 256 blocks of the reference's BlockQ8K (292 bytes: f32 d,
 * int8 qs[256], int16 bsums[16]; kernels.rs:37-41), 4-byte aligned. */
int dr_quantize_q8k(dr_ctx* ctx, const float* act, size_t n, size_t cols, void* out);

/* quantize_row_q8_0 (candle-core 0.8.4 BlockQ8_0::from_float, which
 * ActScratch::q80 calls, src/model/matmul.rs:73-82), the quantization
 * dr_qmatmul applies to its activations for the legacy weight types: act
 * [n][cols] f32 (cols a multiple of 32, 16-byte aligned) -> out, n * cols /
 * 32 blocks of 34 bytes (f16 d = amax / 127 rounded to nearest even, int8
 * qs[32] = round(x / d) half away from zero), 2-byte aligned. */
int dr_quantize_q8_0(dr_ctx* ctx, const float* act, size_t n, size_t cols, void* out);

/* Launch configuration of the last attention kernel this context enqueued
 * (for measurement): key splits across workgroups, workgroups, waves per
 * workgroup, keys per tile, head-dim tile, 32-row query blocks and key
 * groups per workgroup. */
typedef struct {
    int n_split;
    int n_workgroups;
    int waves_per_wg;
    int block_n;
    int head_dim_tile;
    int row_blocks;
    int key_groups;
    int rows_per_wave; /* query rows per compute wave: 32, or 16 (STAGED: two waves per row
                        * block; STREAMS at head dim 256: one 16-row block per workgroup) */
    int kernel; /* DR_KERNEL_STAGED, DR_KERNEL_STREAMS or DR_KERNEL_HILO: which attention kernel ran */
    int split_merge; /* key splits merged: 0 no split, 1 by a second kernel, 2 in-kernel */
} dr_launch_info;
int dr_ctx_last_launch(const dr_ctx* ctx, dr_launch_info* info);

/* Override the key-split heuristic for later calls on ctx (0 = automatic). */
int dr_ctx_set_split(dr_ctx* ctx, int n_split);
/* Query rows per compute wave for later calls on ctx: 16 or 32 where the
 * head-dim tile builds both, 0 = automatic.  With DR_KERNEL_STREAMS at head
 * dim 256, 16 selects the 16-row-wave stream kernel (no key split). */
int dr_ctx_set_wave_rows(dr_ctx* ctx, int rows);
/* Attention kernel families, for dr_ctx_set_kernel and dr_launch_info.kernel.
 * STAGED: the workgroup's waves share K/V super-tiles staged in LDS (every
 * head dim and mask, the Q bias / RoPE epilogue).  STREAMS: head dims 128
 * and 256; each wave streams its own key tiles into LDS with no workgroup
 * barrier in the key loop (no mask or position masks, Q norm). */
#define DR_KERNEL_AUTO 0
#define DR_KERNEL_STAGED 1
#define DR_KERNEL_STREAMS 2
/* HILO: layers kept at DR_PRECISION_HILO and the drop-in dr_attention
 * (f32-accurate scores and values from bf16 hi/lo halves of Q, K and V; see
 * dr_cache_set_precision). */
#define DR_KERNEL_HILO 3
/* Pick the kernel family for later calls on ctx: DR_KERNEL_AUTO (the
 * planner: HILO on hi/lo layers, else STREAMS wherever it applies), or force
 * STAGED / STREAMS (STREAMS falls back to STAGED where it does not apply; on
 * a hi/lo layer both ignore the lo half).  A tuning knob, for measurement
 * and tests. */
int dr_ctx_set_kernel(dr_ctx* ctx, int kernel);
/* The element type of the Q rows that later dr_attention_cached /
 * _cached_noalloc / _step / _step_epi calls on ctx read (no counterpart in
 * the reference, whose attention() takes f32; for callers whose projections
 * produce bf16).  DR_DTYPE_F32 (the default): q points at float rows.
 * DR_DTYPE_BF16: q points at bf16 rows of the same shape (uint16 bit
 * patterns), read by the per-wave-stream kernel, which applies the Q
 * epilogue and the scale to them as to f32 rows.  Calls that that kernel
 * cannot run (head dims other than 128 / 256, hi/lo layers, RoPE below full
 * rotary, forced tile shapes) fail with DR_ERR_UNSUPPORTED before any
 * store. */
#define DR_DTYPE_F32 0
#define DR_DTYPE_BF16 1
int dr_ctx_set_q_dtype(dr_ctx* ctx, int dtype);
/* The element type of the output rows that later dr_attention_cached /
 * _cached_noalloc / _step / _step_epi calls on ctx write (no counterpart in
 * the reference, whose attention() writes f32; for callers whose Wo
 * projection reads bf16).  DR_DTYPE_F32 (the default): out points at float
 * rows.  DR_DTYPE_BF16: out points at bf16 rows of the same shape (uint16
 * bit patterns), each the f32 result rounded to nearest even; written by the
 * per-wave-stream kernel, with the same restrictions and errors as
 * dr_ctx_set_q_dtype's bf16 rows. */
int dr_ctx_set_o_dtype(dr_ctx* ctx, int dtype);
/* How key splits of the STREAMS kernel are merged on later calls on ctx (a
 * tuning knob with no counterpart in the reference, for measurement and
 * tests).  1 (the default): in-kernel; the last split of each 32-row block
 * to finish merges the others' partials, which every split writes and reads
 * with agent-scope (L2-coherent) accesses, counted by per-block tickets that
 * dr_ctx_create allocates and zeroes and each merge resets.  0: a second
 * kernel merges them, as for the other kernel families.  Both give the same
 * bits.  A context's calls never overlap on the device (one stream at a
 * time, ordered across dr_ctx_set_stream), so its tickets and split
 * workspace are used by one call at a time. */
int dr_ctx_set_split_merge(dr_ctx* ctx, int in_kernel);
/* Override the workgroup shape (32-row query blocks x key groups) and the
 * key split for later calls on ctx; 0 = automatic, unbuilt shapes fall back
 * to the automatic one. */
int dr_ctx_set_tuning(dr_ctx* ctx, int row_blocks, int key_groups, int n_split);

/* ---- diagnostics (no counterpart in the reference; for tests) */
/* Device and pinned host allocations the library has made in this process
 * (every hipMalloc / hipHostMalloc it calls).  Host-only, never fails. */
long dr_debug_alloc_count(void);
/* The key tiles the STREAMS kernel's waves request for one workgroup of a
 * head_dim 128 / 256 problem: nk keys in a cache of cap positions (a
 * multiple of 64), queries at positions qmin..qmax under a sliding window
 * (window < 0: none), n_split key splits, every row group and every wave
 * count the kernel is built with (4 and 8 waves per workgroup at head_dim
 * 128, 4 at 256).  Computed on the host by the same code the kernel runs.  min_tile / max_tile: the extremes
 * of every tile index any wave issues a DMA for (including a wave without
 * tiles); partition_ok: 1 if each split's waves multiply each tile of its
 * range exactly once and the splits cover the workgroup's range once. */
int dr_debug_ring_tiles(size_t head_dim, size_t nk, size_t cap, long long window, long long qmin,
                        long long qmax, size_t n_split, int* min_tile, int* max_tile,
                        int* partition_ok);

#ifdef __cplusplus
}
#endif

#endif /* DR_ATTN_H */
