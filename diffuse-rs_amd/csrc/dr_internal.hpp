// dr_internal.hpp -- kernel argument blocks and launcher declarations shared by
// the HIP kernels (attn_fwd.hip, kv_cache.hip) and the C ABI (dr_api.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dr {

// Key tiles are padded to this many rows in every K / V^T buffer, so a tile
// load never leaves the allocation.
constexpr int KEY_ALIGN = 64;
constexpr int MAX_BATCH = 8;
// V^T is stored key-tile-major: [n_head_kv][cap / VT_KEYS][HD][VT_KEYS], so
// the V^T tile of keys [32 t, 32 t + 32) is one contiguous HD x 32 block
// (whole cache lines for the DMA) and element (g, d, p) sits at
// (g * cap + (p / 32) * 32) * HD + d * 32 + p % 32.
constexpr int VT_KEYS = 32;

// One batch slot of an attention launch.  K is [n_head_kv][cap][HD] bf16
// (row = key index), VT is V transposed in 32-key tiles,
// [n_head_kv][cap / 32][HD][32] bf16 (a tile's d-row holds its 32 keys).
// Key index j has sequence position kpos[j] (kpos == nullptr: position j)
// and sequence id kseq[j] (nullptr: 0).
struct AttnSlot {
    const void* q;        // [nq][q_rstride] f32 (bf16 with AttnArgs::q_bf16), head h at h*hd
    float* out;           // [nq][o_rstride] f32 (bf16 with AttnArgs::o_bf16)
    const int* qpos;      // [nq] sequence positions of the queries (device)
    const int* qseq;      // [nq] or nullptr
    const int* qprefix;   // [nq] per-row causal prefix or nullptr
    const uint16_t* k;    // bf16 bits
    const uint16_t* vt;   // bf16 bits
    const uint16_t* klo;  // K's lo half, bf16(k - bf16(k)), K's layout (the hi/lo kernel) or nullptr
    const uint16_t* vlo;  // V's lo half in V^T's layout (with klo) or nullptr
    const int* kpos;      // [nk] or nullptr
    const int* kseq;      // [nk] or nullptr
    int nq;
    int nk;
    int qpos_sorted;      // qpos strictly ascending (a dr_pass): key ranges from endpoints
    int qpos0;            // >= 0: qpos[i] == qpos0 + i (contiguous), read without a load
};

struct AttnArgs {
    // The scalars of the workgroup decode and of the first loads fill the
    // first 64 bytes, with batch slot 0 right behind, so the kernel fetches
    // them with a few wide scalar loads and one wait.
    int n_batch;
    int n_head_kv, group;          // group = n_head / n_head_kv
    int hd;                        // actual head_dim (<= the kernel's HD tile)
    int cap;                       // key capacity of K/VT (multiple of KEY_ALIGN)
    int q_rstride;                 // elements between query rows
    int rowgroups;                 // workgroup row groups per (batch, kv head)
    int n_split;                   // key splits; > 1 writes partials
    uint32_t mg_split, mg_rowgroups, mg_hkv;  // division magic for the workgroup decode
    float c;                       // scale * log2(e), folded into Q
    int n_wg;                      // workgroups in the grid
    int window;                    // < 0: no sliding window
    int prefix;                    // < 0: no causal prefix (scalar)
    int o_rstride;                 // elements between output rows
    AttnSlot slot[MAX_BATCH];
    int n_head;
    const float* qn_w;             // QK-norm gain for Q heads or nullptr
    float qn_eps;
    float* part_o;                 // [split][batch*kv head][row][HD] partial accumulators
    float* part_ml;                // [split][batch*kv head][row][2] partial (max, sum)
    int part_rows;                 // rows per (batch, kv head) in a split plane
    // Per-row-block arrival counters [batch*kv head][rowgroups], zero between
    // calls, or nullptr.  Set: the last split of each row block to finish
    // merges the partials in-kernel (agent-scope accesses) and resets its
    // counter; no split_merge_kernel follows.  The per-wave-stream kernel only.
    int* ticket;
    int q_bf16;                    // Q rows are bf16 (the per-wave-stream kernel reads them)
    int o_bf16;                    // output rows are bf16 (the per-wave-stream kernel writes them)
    // the Q/K/V epilogue's Q part (forward.rs:291-310): bias before the
    // QK-norm, RoPE after it, at the query rows' positions (qpos)
    const float* qb;               // [n_head*hd] or nullptr
    const float* rope;             // [max_len][rot/2][2] (sin, cos) table or nullptr
    int rot;                       // rotated dims (a multiple of 8)
    // (host planning only) an upper bound on the keys any row block can see
    // (the union of the query rows' sliding-window bands), 0: not known
    int key_band;
    int ring_rot;  // the per-wave-stream kernel rotates each row group's tile walk
};
static_assert(offsetof(AttnArgs, slot) == 64, "scalar block of AttnArgs is one 64-byte line");

struct StoreArgs {
    const float* k;      // [n][rstride] f32 rows, kv head g at g * hd
    const float* v;
    int rstride;         // elements between rows (0: n_head_kv * hd)
    const int* pos;      // [n] strictly ascending destination positions (device);
                         // nullptr: row r -> r
    int n;
    int n_head_kv;
    int hd;              // actual head_dim (<= HD tile; tail zero-filled)
    int cap;
    uint16_t* kc;        // [n_head_kv][cap][HD] bf16 bits
    uint16_t* vtc;       // [n_head_kv][cap / VT_KEYS][HD][VT_KEYS] bf16 bits
    uint16_t* klo;       // nullptr, or K's lo half bf16(k - bf16(k)) in K's layout
    uint16_t* vlo;       // with klo: V's lo half in V^T's layout
    const float* kn_w;   // K-norm gain or nullptr
    float kn_eps;
    int vec;             // rows may be read as 16-byte pieces (hd == HD tile, aligned)
    int batch, n_batch;  // batch slot of the cache (n_batch 0 counts as 1): picks the XCDs
    // set by launch_store: workgroup -> (kv head, head-dim chunk, row block)
    int n_rb, per_xcd, xcd_lo, xcd_n;
    // the Q/K/V epilogue's K / V part (forward.rs:291-310), all optional
    const float* kb;     // [n_head_kv*hd] K bias
    const float* vb;     // [n_head_kv*hd] V bias
    int v_norm;          // Gemma: unweighted RMSNorm of each V head (eps kn_eps)
    const float* rope;   // [max_len][rot/2][2] (sin, cos) table, or nullptr
    int rot;             // rotated dims per head
    int pos0;            // >= 0: pos[r] == pos0 + r (contiguous rows), read without a load
};

struct GatherArgs {
    const uint16_t* kc;
    const uint16_t* vtc;
    const uint16_t* klo;  // nullptr, or K's lo half (added back)
    const uint16_t* vlo;  // with klo: V's lo half (added back)
    const int* pos;      // [n] device
    int n;
    int n_head_kv;
    int hd;
    int cap;
    float* out_k;        // [n][n_head_kv][hd] f32
    float* out_v;
};

// The Q/K/V epilogue of attention_block (forward.rs:291-310), in place on
// device rows: q [n][n_head*hd], k and v [n][n_head_kv*hd] f32.
struct EpiArgs {
    float* q;
    float* k;
    float* v;
    const int* pos;       // [n] sequence positions of the rows (device)
    int pos0;             // >= 0: pos[r] == pos0 + r (contiguous rows), read without a load
    int n, n_head, n_head_kv, hd;
    const float* bq;      // [n_head*hd] or nullptr (add_bias)
    const float* bk;      // [n_head_kv*hd] or nullptr
    const float* bv;
    const float* qn_w;    // [hd] QK-norm gains or nullptr
    const float* kn_w;
    int v_norm;           // Gemma: unweighted RMSNorm of each V head
    float eps;
    const float* rope;    // [max_len][rot/2][2] (sin, cos) or nullptr
    int rot;              // rotated dims per head (even, <= hd)
    int vec;              // q, k, v 16-byte aligned and hd a multiple of 4: vector loads
};

// StepCache::split_active (cache.rs:85-114) of one batch slot on the device.
struct SplitArgs {
    const int* seq;        // [n] this step's tokens
    const uint8_t* is_masked;  // [n]
    const int* prev_seq;   // [n] the tokens of the last update_seq
    int* last_changed;     // [n] step of each position's last change (-1: never); updated
    int* active;           // [n] out: active positions, ascending
    int* cached;           // [n] out: cached positions, ascending
    int* meta;             // [6] out: n_active, n_cached, first/last active, first/last cached
    int n;
    int step;
    int vicinity;
};

// A Q8_K block (src/kernels.rs:37-41): 292 bytes.
struct Q8KBlock {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
static_assert(sizeof(Q8KBlock) == 292, "Q8_K block layout");

// Activation rows of dr_qmatmul's workspace: a multiple of the 128 rows of a
// qmm workgroup (the pad rows are quantized as zeros).
__host__ __device__ inline int qmm_rows_padded(int n) { return (n + 127) / 128 * 128; }

// dr_qmatmul's workspace: the Q8_K activations in the order the int8 MFMA
// reads them, so every operand load of a wave is one contiguous run.  Rows
// are grouped in 32-row tiles; lane (c, g) of a tile's operands (c = row % 32,
// g = 0, 1) holds values 32 s + 16 g .. + 15 of sub-block slab s:
//   qs    int8 [n_pad/32][nb][8 slabs][64 lanes][16]
//   bmin  bf16 [n_pad/32][nb][64 lanes][8]  lane (c, 0): bsum_s & 63, lane
//         (c, 1): bsum_s - (bsum_s & 63), s = 0..7 (bsum_s = sum of values
//         32 s .. 32 s + 31 of row c)
//   xd    f32  [n_pad/32][nb][32]  the Q8_K d of each row
struct QmmLayout {
    int8_t* qs;
    uint16_t* bmin;
    float* xd;
    int nb;
    __host__ __device__ QmmLayout(void* ws, int n_pad, int cols) {
        nb = cols / 256;
        qs = static_cast<int8_t*>(ws);
        bmin = reinterpret_cast<uint16_t*>(qs + (size_t)n_pad * cols);
        xd = reinterpret_cast<float*>(bmin + (size_t)n_pad * nb * 16);
    }
    // (tile, block) index of row-tile t32 = t / 32 and block b
    __host__ __device__ size_t tb(int t32, int b) const { return (size_t)t32 * nb + b; }
};

// dr_qmatmul's workspace for the legacy 32-value block types (Q4_0, Q5_0,
// Q8_0 weights): the Q8_0 activations in the order the int8 MFMA reads them.
//   qs  int8 [n_pad/32][nb][64 lanes][16]  lane (c, g): values 16 g .. + 15
//       of block b of row c of the 32-row tile
//   xd  f32  [n_pad/32][nb][32]  the f16 d of each row's block, as f32
struct Q0Layout {
    int8_t* qs;
    float* xd;
    int nb;
    __host__ __device__ Q0Layout(void* ws, int n_pad, int cols) {
        nb = cols / 32;
        qs = static_cast<int8_t*>(ws);
        xd = reinterpret_cast<float*>(qs + (size_t)n_pad * cols);
    }
};

// native_matmul (src/model/matmul.rs:120-148) + residual_add (ops.rs:365-370):
// out[t * rows + r] = vec_dot(w row r, q8k(act row t)) (+ residual).
struct QmmArgs {
    int wtype;               // 12 = Q4_K, 14 = Q6_K; 2 = Q4_0, 6 = Q5_0, 8 = Q8_0 (Q8_0 activations)
    const void* w;           // rows * cols/256 blocks
    int rows, cols;          // cols a multiple of 256
    const float* act;        // [n][cols]
    int n;
    int n_pad;               // qmm_rows_padded(n)
    void* ws;                // workspace of qmm_workspace_bytes(n, cols) bytes (QmmLayout)
    float* out;              // [n][rows]
    const float* residual;   // [n][rows] or nullptr (may alias out)
    // Gemma's post-attention RMSNorm of each output row before the residual
    // add (forward.rs:346-350): gain [rows] or nullptr
    const float* norm_w;
    float norm_eps;
    float* norm_tmp;         // with norm_w: [n][rows] f32 for the rows before the norm
};

// The 32-key tiles [kt_lo, kt_hi) that a block of queries at positions
// qmin..qmax can see through a sliding window (|qpos - kpos| < window,
// attention.rs:43-47) among nk keys at positions 0..nk-1.
__host__ __device__ inline void band_tile_range(int nk, int window, int qmin, int qmax, int& kt_lo,
                                                int& kt_hi) {
    long lo = (long)qmin - window + 1, hi = (long)qmax + window;
    if (lo < 0) lo = 0;
    if (hi > nk) hi = nk;
    if (hi <= lo) {
        kt_lo = kt_hi = 0;
    } else {
        kt_lo = (int)(lo / 32);
        kt_hi = (int)((hi + 31) / 32);
    }
}

// Key tiles [t0, t1) of split `split` of n_split over a workgroup's key tile
// range [kt_lo, kt_hi): ceil-sized consecutive pieces, the last ones possibly
// empty.
__host__ __device__ inline void split_tile_range(int kt_lo, int kt_hi, int n_split, int split, int& t0,
                                                 int& t1) {
    t0 = kt_lo;
    t1 = kt_hi;
    if (n_split > 1) {
        const int ntiles = kt_hi - kt_lo;
        const int per = (ntiles + n_split - 1) / n_split;
        const int a = split * per, b = (split + 1) * per;
        t0 = kt_lo + (a < ntiles ? a : ntiles);
        t1 = kt_lo + (b < ntiles ? b : ntiles);
    }
}

// The key tiles one wave of attn_ring_kernel requests.  Wave w of a workgroup
// whose key range is tiles [t0, t0 + nt) owns tiles t0 + w, t0 + w + rw, ...
// (kw of them) and walks them from its krot-th on, krot = rot mod kw with rot
// the row group when the launch rotates (else 0).  Rotated, the row groups of
// one kv head, which share an XCD, first request different tiles, so the
// head's K/V comes from HBM in one round and later tiles hit in L2 -- right
// while a head's K/V fits that L2 (C2: the 32-layer step 15.34 -> 15.16 us);
// beyond it the rotated walks keep the whole head in play and the L2
// thrashes (C5's global layer fetched 128 MB per call rotated, 44 unrotated),
// so the planner turns it off there (LaunchPlan::rotate).  A wave with no
// tile still issues one K and one V^T DMA (the compiler's vmcnt accounting
// assumes them); that DMA reads tile min(t0 + w, cap_tiles - 1), which lies
// inside the cache plane: the tile base is the DMA's scalar offset, which the
// buffer range check does not cover.  Kernel and host (dr_debug_ring_tiles)
// both use this.
struct RingWaveTiles {
    int t0, wave, rw, kw, krot, idle_tile;
    __host__ __device__ RingWaveTiles(int t0_, int nt, int wave_, int rw_, int rot, int cap_tiles)
        : t0(t0_), wave(wave_), rw(rw_) {
        kw = wave < nt ? (nt - wave + rw - 1) / rw : 0;
        krot = kw > 1 ? rot % kw : 0;
        idle_tile = t0 + wave < cap_tiles - 1 ? t0 + wave : cap_tiles - 1;
    }
    // the k-th tile this wave multiplies, k < kw
    __host__ __device__ int at(int k) const {
        const int kk = k + krot;
        return t0 + wave + rw * (kk >= kw ? kk - kw : kk);
    }
    // the tile of the wave's first K and V^T DMA
    __host__ __device__ int first_dma() const { return kw > 0 ? at(0) : idle_tile; }
};

// Masking mode of an attention launch.
enum MaskMode : int {
    MASK_NONE = 0,  // every key visible (only the key tail is masked)
    MASK_POS = 1,   // window / causal prefix / query sequence ids; key j at position j
    MASK_KEYS = 2,  // arbitrary key positions and/or key sequence ids (per-key metadata)
};

struct LaunchPlan {
    int hd_tile;     // 64, 128, 256 or 512
    int block_n;     // keys per tile (one MFMA key block is 32)
    int rb;          // row blocks (32 query rows each) per workgroup
    int kq;          // key groups per workgroup (merged in LDS)
    int waves;       // rb * kq
    int stages;      // LDS pipeline depth (super-tiles of kq tiles)
    int n_split;     // key splits across workgroups (merged by the last one to finish)
    int rowgroups;   // workgroups per (batch, kv head) and split
    int n_workgroups;
    int mask;        // MaskMode
    bool qepi;       // Q epilogue compiled in: bias, QK-norm, RoPE, each where its operand is given
    bool w16;        // two 16-row compute waves per (row block, key group)
    int kernel;      // KernelKind
    int merge;       // set at launch: 0 no split, 1 split_merge_kernel, 2 in-kernel
    bool rotate;     // KERNEL_STREAMS: rotate the row groups' tile walks (RingWaveTiles)
};

// Attention kernel families.  STAGED: attn_fwd_kernel, the workgroup's waves
// share super-tiles of K/V staged in LDS (every head dim, mask mode and the
// Q epilogue).  STREAMS: attn_ring_kernel, head dims 128 and 256, each wave
// streams its own key tiles (no mask or MASK_POS, Q norm only).  HILO:
// attn_hilo_kernel, f32-accurate scores and values from bf16 hi/lo halves of
// Q, K and V (layers whose cache holds the lo halves, and the drop-in; every
// mask mode, plain Q).
enum KernelKind : int {
    KERNEL_AUTO = 0,
    KERNEL_STAGED = 1,
    KERNEL_STREAMS = 2,
    KERNEL_HILO = 3,
};

// What of the Q/K/V epilogue the attention prologue applies to Q: nothing,
// the QK-norm only, or also the bias and RoPE.
enum QEpilogue : int {
    QEPI_NONE = 0,
    QEPI_NORM = 1,
    QEPI_FULL = 2,
};

// Chooses tile sizes and the key split for a problem on a device with n_cu
// compute units (window: the sliding window, < 0 for none; rot: the rotary
// dims of a RoPE in the Q epilogue, 0 for none).  force_rb /
// force_kq / force_split > 0 override the heuristic (tuning); force_rows 16
// or 32 picks the query rows per compute wave where both are built (0:
// automatic).  merge_in_kernel: the per-wave-stream kernel's key splits (up
// to ring_merge_splits) will be merged in-kernel, which makes them cheaper.
LaunchPlan plan_attention(int hd, int n_batch, int n_head_kv, int group, int max_nq, int max_nk,
                          int mask, int qepi, int window, int rot, int n_cu, int force_rb, int force_kq,
                          int force_split, int force_rows, int force_kernel, bool merge_in_kernel,
                          int key_band = 0);

// Bytes of split workspace a plan needs (part_o + part_ml).
size_t split_workspace_bytes(const LaunchPlan& p, int n_batch, int n_head_kv);

hipError_t launch_attention(const LaunchPlan& p, AttnArgs& a, hipStream_t st);

// The fixed device workspace of the allocation-free entry point
// (scratch.hip): its size, the set-up that takes this device's address of it
// (once per device, with the device current), and that address (nullptr
// before scratch_init succeeded on the device).
size_t scratch_bytes();
hipError_t scratch_init(int device);
void* scratch_ptr(int device);
hipError_t launch_ring(const LaunchPlan& p, const AttnArgs& a, hipStream_t st);
// waves per workgroup of attn_ring_kernel for a workgroup streaming `tiles`
// key tiles (0: head dim not built), and whether a wave count is built
int ring_waves(int hd, int tiles);
bool ring_waves_built(int hd, int waves);
int ring_merge_splits(int hd);  // most key splits attn_ring_kernel merges in-kernel
hipError_t launch_hilo(const LaunchPlan& p, const AttnArgs& a, hipStream_t st);
int hilo_rows();  // query rows per workgroup of attn_hilo_kernel
hipError_t launch_store(int hd_tile, const StoreArgs& a, hipStream_t st);
hipError_t launch_gather(int hd_tile, const GatherArgs& a, hipStream_t st);
hipError_t launch_epilogue(const EpiArgs& a, hipStream_t st);
hipError_t launch_split_active(const SplitArgs& a, hipStream_t st);
size_t qmm_workspace_bytes(int n, int cols);
size_t qmm0_workspace_bytes(int n, int cols);  // the legacy block types
hipError_t launch_qmatmul(const QmmArgs& a, hipStream_t st);
// quantize_row_q8_0 into the reference's BlockQ8_0 layout (34 bytes each)
hipError_t launch_quantize_q80(const float* act, int n, int cols, void* out, hipStream_t st);
// quantize_rows_q8_k into the reference's BlockQ8K layout
hipError_t launch_quantize_q8k(const float* act, int n, int cols, Q8KBlock* out, hipStream_t st);

}  // namespace dr
