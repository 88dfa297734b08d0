// attn_ring.hip -- denoise-step attention at head dim 128 with per-wave key
// streams (gfx950, MI355X).
//
// Computes the reference's attention() (src/model/attention.rs:101-186) for
// one row block of 32 query rows per workgroup: every (query row, head) of the
// block against the keys visible to it (visible(), :36-57), with an online
// softmax.  Same operands, cache layout and numerics as attn_fwd_kernel; the
// difference is how the K/V stream reaches the matrix cores.
//
// A workgroup of 32 query rows reads every K/V byte of its key range from L2
// once, 384 KB per call at LLaDA-8B's 768 keys, so the L2 -> CU stream (64 B
// per clock per CU on MI355X) bounds the call, not the MFMAs.  The stream
// reaches that rate only with several waves issuing loads independently.
// So each of the workgroup's 4 waves is a key group of its own: wave w owns the
// 32-key tiles w, w + 4, w + 8, ... of the range and runs all 32 query rows
// against them.  It moves each of its tiles into its own slice of LDS with
// buffer_load ... lds (K tile and V^T tile in separate 8 KB buffers) and
// waits on its own vmcnt, so no workgroup barrier sits in the key loop.  The
// next K tile is requested as soon as the QK^T product has read the current
// one, the next V^T tile as soon as the PV product has.  The 4 partial softmax
// states of each row are merged through LDS at the end, which also stages
// coalesced full-row output stores.
//
// Per wave and tile (32 keys x 32 query rows), on v_mfma_f32_32x32x16_bf16:
//   S^T = K Q^T - m   A = K (LDS rows permuted by sigma), B = Q^T (registers)
//   O^T += V^T P^T    A = V^T (LDS), B = P^T straight from the S^T registers
// Lane (col, half) owns query row col and keys 16*half .. 16*half + 15 of the
// tile, so the softmax row statistics need one exchange with lane ^ 32.
// Softmax runs in the log2 domain with the lazily moved maximum of
// attn_fwd.hip (m moves only when a score exceeds it by more than 8); l sums
// the bf16-rounded p that the PV product multiplies.  A row with no visible
// key ends with l = 0 and writes NaN, as attention.rs:181-185 does.
#include "attn_common.hpp"

#include <limits.h>
#include <math.h>

namespace dr {
namespace {

// Geometry per head dim and wave count W (each wave streams its own tiles).
// hd 256: 4 waves, one per SIMD (a wave's O^T, 128 registers, and Q^T
// fragments, 64, fill most of a SIMD's register file; its K + V^T tiles take
// 32 KB of LDS).  hd 128: 4 or 8 waves, chosen by the planner from the tiles
// a workgroup streams (ring_waves).  Short streams take 4: at LLaDA-8B's 768
// keys (24 tiles) 8 waves, two per SIMD, took 11.4 us per call over a 32-layer
// cache against 10.9 for 4, since their first tiles made a larger start burst
// through HBM and they leave twice the partial rows to merge.  Long streams
// take 8, whose loads keep twice the bytes in flight: at 40 - 80 tiles 4 waves
// were 1 - 6 % slower.
template <int HD, int W>
struct Ring {
    static constexpr int RW = W;                  // waves (key groups) per workgroup
    static constexpr int RT = BN * HD;            // bf16 elements per K tile (and per V^T tile)
    static constexpr int KCH = HD / 8;            // 16-byte chunks per K row
    static constexpr int VCH = BN / 8;            // 16-byte chunks per V^T row
    static constexpr int NDMA = RT * 2 / 1024;    // 1 KB DMA instructions per tile
    static constexpr int KS = HD / 16;            // contraction steps of QK^T
    static constexpr int DB = HD / 32;            // 32-dim blocks of O^T
    static constexpr int TPR = RW * 64 / 32;      // threads per query row (Q load, final pass)
    static constexpr int QP = HD / 4 / TPR;       // f32x4 pieces per thread and row
    static constexpr int RING_BYTES = RW * 2 * RT * 2;   // per wave: K tile + V^T tile
    static constexpr int Q_BYTES = 32 * HD * 2;          // the block's Q rows, bf16
    static constexpr int ML_OFF = RING_BYTES + Q_BYTES;  // [RW][32] max, then [RW][32] sum
    static constexpr int LDS = ML_OFF + 2 * RW * 32 * 4;
    static constexpr int MS = HD == 128 ? 4 : 2;  // most key splits merged in-kernel (registers)
    static_assert(32 * HD * 4 == 2 * RT * 2, "a wave's O^T partial fills its K + V^T buffers");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NDMA < 32, "two tiles of DMA fit the vmcnt counter");
};

template <int HD, int MODE, int W>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4)))
void attn_ring_kernel(const AttnArgs a) {
    using G = Ring<HD, W>;
    constexpr int RW = G::RW, RT = G::RT, R_KCH = G::KCH, R_VCH = G::VCH, NDMA = G::NDMA;
    constexpr int RHD = HD, TPR = G::TPR, QP = G::QP, KS = G::KS, DB = G::DB;
    constexpr int RING_BYTES = G::RING_BYTES, ML_OFF = G::ML_OFF;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_red[3];

    AttnSlot S = a.slot[0];
    const float* qn_w = a.qn_w;
    // (every argument the Q load depends on is fetched in this first batch:
    // fetched where first used, each cost a dependent scalar round trip)
    int q_bf16 = a.q_bf16;
    const float* qb = a.qb;
    const float* rope = a.rope;
    asm volatile("" : "+s"(S.q), "+s"(S.out), "+s"(S.qpos), "+s"(S.qseq), "+s"(S.qprefix),
                 "+s"(S.k), "+s"(S.vt), "+s"(S.nq), "+s"(S.nk), "+s"(S.qpos_sorted), "+s"(qn_w),
                 "+s"(S.qpos0), "+s"(q_bf16), "+s"(qb), "+s"(rope)
                 : "s"(a.n_batch), "s"(a.n_head_kv), "s"(a.group), "s"(a.cap),
                   "s"(a.q_rstride), "s"(a.rowgroups), "s"(a.n_split), "s"(a.mg_split),
                   "s"(a.mg_rowgroups), "s"(a.mg_hkv), "s"(a.c), "s"(a.n_wg), "s"(a.window),
                   "s"(a.prefix));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, hf = lane >> 5;

    // Workgroup -> (batch, kv head, row group, split); consecutive logical
    // ids (the row groups of one kv head) share an XCD and its L2.
    const int nwg = a.n_wg;
    const int hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    int split = 0, rg, b = 0, g;
    if (a.n_split == 1 && a.n_batch == 1) {
        g = udiv(lid, a.rowgroups, a.mg_rowgroups);
        rg = lid - g * a.rowgroups;
    } else {
        const int q1 = udiv(lid, a.n_split, a.mg_split);
        split = lid - q1 * a.n_split;
        const int q2 = udiv(q1, a.rowgroups, a.mg_rowgroups);
        rg = q1 - q2 * a.rowgroups;
        b = udiv(q2, a.n_head_kv, a.mg_hkv);
        g = q2 - b * a.n_head_kv;
        if (a.n_batch > 1) S = a.slot[b];
    }

    const int rows_total = a.group * S.nq;
    const int wg_row0 = rg * 32;
    if (wg_row0 >= rows_total) return;  // uniform over the workgroup and all its splits
    const float inv_nq = __builtin_amdgcn_rcpf((float)S.nq);
    // (head in group, query index) of packed row r; MHA rows are the queries
    auto split_row = [&](int r, int& hgo, int& qio) __attribute__((always_inline)) {
        if (a.group == 1) {
            hgo = 0;
            qio = r;
        } else {
            row_split(r, S.nq, inv_nq, a.group, hgo, qio);
        }
    };

    // ---- Q rows first: they gate the first MFMA.  Thread tid holds the QP
    // f32x4 pieces d0 + (HD / QP) p of workgroup row tid / TPR (rows past the
    // block load row 0 and are zeroed later: no branch, so nothing issued
    // below waits for these loads).
    constexpr int QSTR = HD / QP;
    const int qlr = tid / TPR;
    const int qd0 = (tid % TPR) * 4;
    const int qr = wg_row0 + qlr;
    const bool qok = qr < rows_total;
    // The Q part of the Q/K/V epilogue (forward.rs:291-310) when the caller
    // folds it in: the bias (add_bias, ops.rs:373-382) before the QK-norm,
    // RoPE (rotate_rows, ops.rs:433-452) after it.  Full rotary only (rot ==
    // HD, checked at launch): dim d < HD/2 and its partner d + HD/2 are then
    // pieces p and p + QP/2 of the same thread, and the (sin, cos) pairs of
    // the row's position are those of the thread's first QP/2 pieces.
    f32x4 xq[QP], wq[QP], bq4[QP];
    u32x2 xq16[QP];  // bf16 rows: the raw pieces, widened after the first DMA is issued
    f32x4 tab[QP / 2][2];
    int tab_pos = 0;  // RoPE on a pass with scattered positions: the row's position
    auto load_tab = [&](int pos) __attribute__((always_inline)) {
        const float* trow = rope + ((size_t)pos * (RHD / 2) + qd0) * 2;
#pragma unroll
        for (int p = 0; p < QP / 2; ++p) {
            tab[p][0] = gload<f32x4>(trow + 2 * QSTR * p);
            tab[p][1] = gload<f32x4>(trow + 2 * QSTR * p + 4);
        }
    };
    {
        int qhg, qqi;
        split_row(qok ? qr : 0, qhg, qqi);
        const size_t qoff = (size_t)qqi * a.q_rstride + (size_t)(g * a.group + qhg) * RHD + qd0;
        if (q_bf16) {
            // bf16 rows: 8-byte pieces, kept raw here (a vector type, not
            // HIP's uint2 struct, whose copy made a flat load; widening them
            // here made the wave wait for them before any K/V DMA)
            const uint16_t* qrow = static_cast<const uint16_t*>(S.q) + qoff;
#pragma unroll
            for (int p = 0; p < QP; ++p) xq16[p] = gload<u32x2>(qrow + QSTR * p);
        } else {
            const float* qrow = static_cast<const float*>(S.q) + qoff;
#pragma unroll
            for (int p = 0; p < QP; ++p) xq[p] = gload<f32x4>(qrow + QSTR * p);
        }
        if (qn_w) {  // the QK-norm gains of these dims
#pragma unroll
            for (int p = 0; p < QP; ++p) wq[p] = gload<f32x4>(qn_w + qd0 + QSTR * p);
        }
        if (qb) {
            const float* bq = qb + (size_t)(g * a.group + qhg) * RHD;
#pragma unroll
            for (int p = 0; p < QP; ++p) bq4[p] = gload<f32x4>(bq + qd0 + QSTR * p);
        }
        if (rope) {
            // the row's position, then the table row (pairs j = qd0 + QSTR p,
            // 2 floats each).  Contiguous passes know the position and load
            // the row here.  Other passes load the position here and the row
            // after the first K/V DMA: a table address that depends on a load
            // made the compiler wait for every load so far (the Q rows too)
            // before the first DMA.
            if (S.qpos0 >= 0)
                load_tab(S.qpos0 + qqi);
            else
                tab_pos = gload<int>(S.qpos + qqi);
        }
    }

    // ---- the query row of this lane's column, its mask state, and the
    // workgroup's key-tile range (MASK_POS: the band its rows can see)
    const int r = wg_row0 + col;
    const bool rvalid = r < rows_total;
    int hg = 0, qi = 0;
    if (rvalid) split_row(r, hg, qi);
    int kt_lo = 0, kt_hi = (S.nk + BN - 1) / BN;
    int my_qpos = 0, my_qseq = 0, my_pref = -1;
    int qmin = 0, qmax = 0;
    bool tiles_can_be_full = MODE == MASK_NONE;
    if constexpr (MODE == MASK_POS) {
        // (contiguous passes: positions without a load, so the key range,
        // and the first K/V DMA behind it, wait for nothing)
        my_qpos = S.qpos0 >= 0 ? S.qpos0 + (rvalid ? qi : 0) : gload<int>(S.qpos + (rvalid ? qi : 0));
        if (S.qseq) my_qseq = gload<int>(S.qseq + (rvalid ? qi : 0));
        my_pref = S.qprefix ? (rvalid ? gload<int>(S.qprefix + qi) : -1) : a.prefix;
        bool prefix_free;
        if (S.qpos_sorted && S.qprefix == nullptr) {
            // ascending positions: the extremes sit at the ends of the block
            // (the whole pass if it spans heads), read with scalar loads
            const int r1 = min(wg_row0 + 32, rows_total) - 1;
            const int h0 = wg_row0 / S.nq, h1 = r1 / S.nq;
            const int lo = h0 == h1 ? wg_row0 - h0 * S.nq : 0;
            const int hi = h0 == h1 ? r1 - h0 * S.nq : S.nq - 1;
            if (S.qpos0 >= 0) {
                qmin = S.qpos0 + lo;
                qmax = S.qpos0 + hi;
            } else {
                qmin = *(const __attribute__((address_space(4))) int*)(S.qpos + lo);
                qmax = *(const __attribute__((address_space(4))) int*)(S.qpos + hi);
            }
            prefix_free = a.prefix < 0 || qmin >= a.prefix;
        } else {
            int vmin = rvalid ? my_qpos : INT_MAX;
            int vmax = rvalid ? my_qpos : INT_MIN;
            int pref_row = (rvalid && my_pref >= 0 && my_qpos < my_pref) ? 1 : 0;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                vmin = min(vmin, __shfl_xor(vmin, off));
                vmax = max(vmax, __shfl_xor(vmax, off));
                pref_row |= __shfl_xor(pref_row, off);
            }
            // every wave holds the same 32 rows: wave 0's reduction is the workgroup's
            if (wave == 0 && lane == 0) {
                s_red[0] = vmin;
                s_red[1] = vmax;
                s_red[2] = pref_row;
            }
            __syncthreads();
            qmin = s_red[0];
            qmax = s_red[1];
            prefix_free = s_red[2] == 0;
        }
        tiles_can_be_full = prefix_free && S.qseq == nullptr;
        if (a.window >= 0) band_tile_range(S.nk, a.window, qmin, qmax, kt_lo, kt_hi);
    }
    int t0, t1;
    split_tile_range(kt_lo, kt_hi, a.n_split, split, t0, t1);
    const int nt = t1 - t0;  // tiles of this workgroup: t0 + j, j < nt

    // ---- the K / V^T planes of kv head g, and this wave's DMA offsets.
    // K tile t is rows [32t, 32t + 32) of [cap][128]; the V^T tile of the
    // same keys is the 128 x 32 block at the same byte offset of the V^T
    // plane.  LDS row R of a K tile holds key sigma(R) with its 16-byte
    // chunks XOR-swizzled by R, V^T row d its chunks swizzled by d; lane i of
    // DMA instruction j fills LDS chunk 64 j + i, so it reads the global
    // chunk that belongs there.  Each instruction reads 1 KB of whole rows.
    const uint32_t plane_bytes = (uint32_t)a.cap * RHD * 2;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(S.k + (size_t)g * a.cap * RHD, plane_bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(S.vt + (size_t)g * RHD * a.cap, plane_bytes);
    int kvo[NDMA], vvo[NDMA];
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
        const int idx = j * 64 + lane;
        const int R = idx / R_KCH, pk = idx % R_KCH;
        kvo[j] = (sigma(R) * RHD + ((pk ^ swz<R_KCH>(R)) << 3)) * 2;
        const int d = idx / R_VCH, pv = idx % R_VCH;
        vvo[j] = (d * BN + ((pv ^ swz<R_VCH>(d)) << 3)) * 2;
    }
    uint16_t* const kbuf = smem + wave * 2 * RT;
    uint16_t* const vbuf = kbuf + RT;
    auto issue_k = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma16(rk, kbuf + j * 512, kvo[j], t * (BN * RHD * 2));
    };
    auto issue_v = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma16(rv, vbuf + j * 512, vvo[j], t * (BN * RHD * 2));
    };
    auto issue_v_to_k = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma16(rv, kbuf + j * 512, vvo[j], t * (BN * RHD * 2));
    };
    // Wave w takes tiles t0 + w, t0 + w + RW, ...: a fixed assignment, so
    // every call sums each row's keys in the same order (bit-identical
    // results run to run; claiming tiles dynamically balanced the waves'
    // finishing times but made the summation order depend on timing).  Row
    // group rg starts its walk at a rotated point when the launch asks
    // (RingWaveTiles).
    // (The first DMA is issued even when the wave has no tile, unconditional
    // for the compiler's wait accounting; its data is never used, and it reads
    // a tile clamped into the cache plane, since the tile base goes in the
    // DMA's scalar offset, which the descriptor's range check excludes.)
    const RingWaveTiles wt(t0, nt, wave, RW, a.ring_rot ? rg : 0, a.cap / BN);
    const int kw = wt.kw;  // this wave's tiles
    auto tile_at = [&](int k) __attribute__((always_inline)) { return wt.at(k); };
    issue_k(wt.first_dma());

    if (rope && S.qpos0 < 0) load_tab(tab_pos);
    if (q_bf16) {  // widened exactly to f32
#pragma unroll
        for (int p = 0; p < QP; ++p) {
            const u32x2 w = xq16[p];
            xq[p] = f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                          __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
        }
    }

    if (qb) {
#pragma unroll
        for (int p = 0; p < QP; ++p) xq[p] += bq4[p];
    }
    // QK-norm (rms_norm_inplace, ops.rs:106-114): f32 squares summed in f64
    // over the TPR lanes of the row, then x * scale * w.
    if (qn_w) {
        double ss = 0.0;
#pragma unroll
        for (int p = 0; p < QP; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sq = xq[p][e] * xq[p][e];
                ss += (double)sq;
            }
#pragma unroll
        for (int off = 1; off < TPR; off <<= 1) ss += __shfl_xor(ss, off);
        const float sc = 1.0f / (float)sqrt(ss / (double)RHD + (double)a.qn_eps);
#pragma unroll
        for (int p = 0; p < QP; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
                xq[p][e] = xq[p][e] * sc * wq[p][e];
            }
    }
    if (rope) {
#pragma unroll
        for (int p = 0; p < QP / 2; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sn = tab[p][e >> 1][2 * (e & 1)], cs = tab[p][e >> 1][2 * (e & 1) + 1];
                const float lo = xq[p][e], hi = xq[p + QP / 2][e];
                xq[p][e] = rope_lo(lo, hi, sn, cs);
                xq[p + QP / 2][e] = rope_hi(lo, hi, sn, cs);
            }
    }
    uint16_t* const qs = smem + RING_BYTES / 2;
#pragma unroll
    for (int p = 0; p < QP; ++p) {
        const int d = qd0 + QSTR * p;
        bf16x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (__bf16)(qok ? xq[p][e] * a.c : 0.0f);
        *reinterpret_cast<bf16x4*>(qs + qlr * RHD + (((d >> 3) ^ swz<R_KCH>(qlr)) << 3) + (d & 7)) = y;
    }
    lds_barrier();  // (the first K tile stays in flight)
    // The first V^T tile, first needed by the PV product of step 1, is
    // requested only now: at kernel start every CU asks for its Q rows and
    // first tiles at once, and the smaller that burst, the sooner Q and the
    // first K tile land.  (DMA order stays K0, V0, K1, ...)
    issue_v(wt.first_dma());
    // Q^T fragments, held for the whole key loop: lane (col, hf) supplies
    // row col, dims 16 c + 8 hf .. + 8 of contraction step c
    bf16x8 qf[KS];
#pragma unroll
    for (int c = 0; c < KS; ++c)
        qf[c] = *reinterpret_cast<const bf16x8*>(qs + col * RHD + (((2 * c + hf) ^ swz<R_KCH>(col)) << 3));

    f32x16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x16{};
    float mu = 0.0f;        // running max m (log2 units), valid once m_set
    bool m_set = false;
    float thr = -INFINITY;  // a score above mu + thr moves m
    float l_acc = 0.0f;     // this lane's share (its 16 keys per tile) of the row's sum
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

    // V^T fragments of a tile: lane (col, hf) supplies row d = 32 db + col,
    // keys 16 hf + 8 sl .. + 8 of key slice sl (the P^T slice it holds)
    auto read_v = [&](const uint16_t* vsrc, bf16x8 (&vf)[DB][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int d = 32 * db + col;
            const uint16_t* vrow = vsrc + d * BN;
            const int sw = swz<R_VCH>(d);
            vf[db][0] = *reinterpret_cast<const bf16x8*>(vrow + (((2 * hf) ^ sw) << 3));
            vf[db][1] = *reinterpret_cast<const bf16x8*>(vrow + (((2 * hf + 1) ^ sw) << 3));
        }
    };
    auto pv = [&](const bf16x8 (&vf)[DB][2], const bf16x8 (&pp)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][0], pp[0], o[db], 0, 0, 0);
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][1], pp[1], o[db], 0, 0, 0);
        }
    };

    // Software pipeline over this wave's tiles: step i runs QK^T of tile i
    // and its softmax, and the PV product of tile i - 1 interleaved with the
    // exponentials (one MFMA per few VALU instructions, in one basic block),
    // so the matrix core and the VALU overlap inside the wave.  O holds tile
    // i - 1's product relative to the max before tile i; it is rescaled
    // after that product when tile i moves the max.  DMA order: K0 V0 | K1 |
    // K2 V1 | K3 V2 | ... (the next K tile once QK^T has read the buffer, the
    // next V^T tile once PV has); the last tile's V^T goes to the K buffer as
    // soon as its QK^T has read that, so its latency overlaps the last
    // softmax instead of trailing it.  Step 0 has no PV and is peeled off.
    f32x16 negm;  // -m in every slot: the accumulator input of QK^T
#pragma unroll
    for (int e = 0; e < 16; ++e) negm[e] = 0.0f;
    // S^T = K Q^T - m of the tile in the K buffer
    auto qk = [&]() __attribute__((always_inline)) {
        const uint16_t* krow = kbuf + col * RHD;
        const int sw = swz<R_KCH>(col);
        f32x16 sacc = negm;
#pragma unroll
        for (int h = 0; h < KS / 4; ++h) {
            bf16x8 kf[4];
#pragma unroll
            for (int c = 0; c < 4; ++c)
                kf[c] = *reinterpret_cast<const bf16x8*>(krow + (((2 * (4 * h + c) + hf) ^ sw) << 3));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[c], qf[4 * h + c], sacc, 0, 0, 0);
        }
        return sacc;
    };
    // masking, and the lazily moved max: returns whether m moved (then O
    // must be scaled by alpha once the pending PV product is in)
    auto mask_and_max = [&](f32x16& sv, int tt, float& alpha) __attribute__((always_inline)) {
        // slot e is key 32 tt + 16 hf + e
        const int kbase = tt * BN;
        bool full = kbase + BN <= S.nk;
        if constexpr (MODE == MASK_POS) {
            const bool win_ok =
                a.window < 0 || (qmax - kbase < a.window && kbase + BN - 1 - qmin < a.window);
            full = full && tiles_can_be_full && win_ok;
        }
        if (!full) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int kidx = kbase + 16 * hf + e;
                bool vis = kidx < S.nk;
                if constexpr (MODE == MASK_POS)
                    vis = vis & visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
                sv[e] = vis ? sv[e] : -INFINITY;
            }
        }
        float mx = max3(sv[0], sv[1], sv[2]);
        mx = max3(mx, sv[3], sv[4]);
        mx = max3(mx, sv[5], sv[6]);
        mx = max3(mx, sv[7], sv[8]);
        mx = max3(mx, sv[9], sv[10]);
        mx = max3(mx, sv[11], sv[12]);
        mx = max3(mx, sv[13], sv[14]);
        mx = __builtin_fmaxf(mx, sv[15]);
        const bool moved = __builtin_amdgcn_ballot_w64(mx > thr) != 0;
        alpha = 1.0f;
        if (moved) {
            const float cm = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
            const bool upd = cm > thr;
            const float delta = upd ? cm : 0.0f;
            alpha = upd ? (m_set ? __builtin_amdgcn_exp2f(-delta) : 0.0f) : 1.0f;
            mu += delta;
            m_set = m_set | upd;
            thr = m_set ? RESCALE_THRESHOLD : -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                sv[e] -= delta;
                negm[e] = -mu;
            }
            l_acc *= alpha;
        }
        return moved;
    };
    // p = exp2(s) rounded to bf16 in pairs (P^T slice sl = slots 8 sl ..
    // 8 sl + 7), l += the rounded p
    auto softmax_p = [&](const f32x16& sv, u32x4 (&pw)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int sl = 0; sl < 2; ++sl)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bf16x2 pr = {(__bf16)__builtin_amdgcn_exp2f(sv[8 * sl + 2 * j]),
                                   (__bf16)__builtin_amdgcn_exp2f(sv[8 * sl + 2 * j + 1])};
                pw[sl][j] = __builtin_bit_cast(uint32_t, pr);
                l_acc = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_acc, false);
            }
    };
    // (keeps p and l computed before this point: the exponentials stay in
    // the block of the PV product they are interleaved with)
    auto pin = [&](const u32x4 (&pw)[2]) __attribute__((always_inline)) {
        asm volatile("" ::"v"(pw[0][0]), "v"(pw[0][1]), "v"(pw[0][2]), "v"(pw[0][3]), "v"(pw[1][0]),
                     "v"(pw[1][1]), "v"(pw[1][2]), "v"(pw[1][3]), "v"(l_acc));
    };

    u32x4 pprev[2];
    bool last_in_k = false;  // the last tile's V^T is in the K buffer
    int t = kw > 0 ? tile_at(0) : -1;  // the current tile (uniform over the wave)
    if (t >= 0) {
        // step 0: K tile 0 has landed when only V^T tile 0 is outstanding
        wait_vmcnt<NDMA>();
        f32x16 sv = qk();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const int tn = kw > 1 ? tile_at(1) : -1;
        if (tn >= 0) issue_k(tn);
        float alpha;
        mask_and_max(sv, t, alpha);  // (O is still zero: no rescale)
        softmax_p(sv, pprev);
        t = tn;
    }
    for (int i = 1; t >= 0; ++i) {
        // K tile i has landed: outstanding after it is V^T tile i - 1 (NDMA
        // instructions), except at i = 1, where V^T 0 was issued before K 1
        if (i == 1)
            wait_vmcnt<0>();
        else
            wait_vmcnt<NDMA>();
        f32x16 sv = qk();
        // every K fragment is in registers: the K buffer takes the next tile,
        // or this last tile's V^T
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const int tn = i + 1 < kw ? tile_at(i + 1) : -1;
        if (tn >= 0)
            issue_k(tn);
        else
            issue_v_to_k(t);
        // V^T tile i - 1 (the pending PV product's operand) has landed: after
        // it only the DMA just issued is outstanding
        wait_vmcnt<NDMA>();
        bf16x8 vf[DB][2];
        read_v(vbuf, vf);
        float alpha;
        const bool moved = mask_and_max(sv, t, alpha);
        // the PV product of tile i - 1, interleaved with tile i's exponentials
        u32x4 pcur[2];
        softmax_p(sv, pcur);
        {
            const bf16x8 pp[2] = {__builtin_bit_cast(bf16x8, pprev[0]), __builtin_bit_cast(bf16x8, pprev[1])};
            pv(vf, pp);
        }
#pragma unroll
        for (int k = 0; k < 2 * DB; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);            // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x402, 16 / DB, 0);  // VALU / transcendental
        }
        pin(pcur);
        __builtin_amdgcn_sched_barrier(0);
        if (moved) {
#pragma unroll
            for (int db = 0; db < DB; ++db) o[db] *= alpha;
        }
        pprev[0] = pcur[0];
        pprev[1] = pcur[1];
        // the V^T buffer is free once its fragments are in registers: it
        // takes this tile's V^T (the last tile's went to the K buffer)
        if (tn >= 0) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue_v(t);
        }
        last_in_k = true;
        t = tn;
    }
    // the last tile's PV product (a wave without tiles has none: its buffer
    // holds a tile past its range, whose values it must not multiply, even
    // by zero)
    wait_vmcnt<0>();
    if (kw > 0) {
        bf16x8 vf[DB][2];
        read_v(last_in_k ? kbuf : vbuf, vf);
        const bf16x8 pp[2] = {__builtin_bit_cast(bf16x8, pprev[0]), __builtin_bit_cast(bf16x8, pprev[1])};
        pv(vf, pp);
    }

    // ---- merge the RW key groups of each row.  A wave's K and V^T buffers
    // are its own and free once its last PV product has read them: its O^T
    // (32 rows x HD f32) goes there right away, while other waves
    // may still be in their loops, with (m, l) beside the other rows'
    // statistics.  After one barrier every thread finishes a row: wave w's
    // partial is weighted by exp2(m_w - M), M the row's largest m, and
    // O = sum_w w_w O_w / sum_w w_w l_w.  16-byte chunk c of row q sits at
    // chunk c ^ q of its row, so both the writes (lanes spread over
    // rows) and the reads (lanes spread over chunks) hit distinct banks.
    float* const sm = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + ML_OFF);  // [RW][32]
    float* const sl = sm + RW * 32;                                                    // [RW][32]
    const float l_tot = l_acc + __shfl_xor(l_acc, 32);
    if (hf == 0) {
        sm[wave * 32 + col] = m_set ? mu : -INFINITY;
        sl[wave * 32 + col] = l_tot;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // (the last V^T fragments are read)
    {
        // o[db][e] is O^T[d = 32 db + 8 (e / 4) + 4 hf + e % 4][col]: chunk
        // 8 db + 2 (e / 4) + hf of row col
        float* myrow = reinterpret_cast<float*>(kbuf) + col * RHD;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(myrow + 4 * ((8 * db + 2 * j + hf) ^ col)) =
                    f32x4{o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]};
    }
    lds_barrier();
    // thread tid: row rr = tid / TPR, chunks cidx(k) = ch + TPR k', k < CPT,
    // where k' = k except with 8 threads per row: there a wave's 64 lanes are
    // 8 rows of 8 and every read below would take the same 8-chunk block of 8
    // rows (half of a bank sweep, 4 lanes per bank), so odd rows take the
    // blocks in the other order (k' = k ^ 1).  Every access of the final pass
    // uses the same mapping.
    constexpr int CPT = HD / 4 / TPR;
    const int rr = tid / TPR, ch = tid % TPR;
    auto cidx = [&](int k) __attribute__((always_inline)) {
        return ch + TPR * (TPR == 8 ? (k ^ (rr & 1)) : k);
    };
    const int row = wg_row0 + rr;
    const bool row_ok = row < rows_total;
    f32x4 acc[CPT];
    float M = -INFINITY, L = 0.0f;
    if (row_ok) {
        float mw[RW];
#pragma unroll
        for (int w = 0; w < RW; ++w) {
            mw[w] = sm[w * 32 + rr];
            M = __builtin_fmaxf(M, mw[w]);
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < RW; ++w) {
            const float wt = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - M);
            const float* prow = reinterpret_cast<const float*>(smem + w * 2 * RT) + rr * RHD;
#pragma unroll
            for (int k = 0; k < CPT; ++k)
                acc[k] += wt * *reinterpret_cast<const f32x4*>(prow + 4 * (cidx(k) ^ rr));
            L += wt * sl[w * 32 + rr];
        }
    }
    auto store_rows = [&](const f32x4 (&val)[CPT], float l) __attribute__((always_inline)) {
        int ohg, oqi;
        split_row(row, ohg, oqi);
        const size_t o0 = (size_t)oqi * a.o_rstride + (size_t)(g * a.group + ohg) * RHD;
        const float il = __builtin_amdgcn_rcpf(l);
        if (a.o_bf16) {  // rounded to nearest even, 8-byte pieces
            uint16_t* orow = reinterpret_cast<uint16_t*>(S.out) + o0;
#pragma unroll
            for (int k = 0; k < CPT; ++k) {
                const f32x4 v = val[k] * il;
                const bf16x4 y = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
                gstore(orow + 4 * cidx(k), y);
            }
        } else {
            float* orow = S.out + o0;
#pragma unroll
            for (int k = 0; k < CPT; ++k) gstore(orow + 4 * cidx(k), val[k] * il);
        }
    };
    if (a.n_split == 1) {
        if (row_ok) store_rows(acc, L);
        return;
    }
    // This split's partial row: the sum relative to the row max M, and (M, L).
    const size_t plane = (size_t)a.n_batch * a.n_head_kv * a.part_rows;
    const size_t prow0 = (size_t)(b * a.n_head_kv + g) * a.part_rows + row;  // in split plane 0
    if (!a.ticket) {
        // for split_merge_kernel, launched next
        if (row_ok) {
            const size_t prow = (size_t)split * plane + prow0;
#pragma unroll
            for (int k = 0; k < CPT; ++k) gstore(a.part_o + prow * RHD + 4 * cidx(k), acc[k]);
            if (ch == 0) gstore(a.part_ml + prow * 2, make_float2(M, L));
        }
        return;
    }
    // In-kernel merge.  Each split stores its partial with agent-scope
    // stores and waits until they are complete; one thread then takes the
    // row block's ticket.  The split that draws n_split - 1 arrives last: the
    // others' stores are complete, and its agent-scope loads see them.  It
    // merges the splits in split order (the same bits whichever split
    // arrives last, and those of split_merge_kernel) and resets the ticket
    // for the next call.  No workgroup waits for another.
    // (Byte offsets of a row plane fit 32 bits: the host checks the size.)
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.part_o, 0xffffffffu);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.part_ml, 0xffffffffu);
    if (row_ok) {
        const int po = (int)(((size_t)split * plane + prow0) * RHD * 4);
#pragma unroll
        for (int k = 0; k < CPT; ++k) store_sc1(ro, po + 16 * cidx(k), acc[k]);
        if (ch == 0) store2_sc1(rm, (int)(((size_t)split * plane + prow0) * 8), M, L);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* const tk = a.ticket + (b * a.n_head_kv + g) * a.rowgroups + rg;
    if (tid == 0) s_red[0] = __hip_atomic_fetch_add(tk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_red[0] != a.n_split - 1) return;
    if (tid == 0) __hip_atomic_store(tk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!row_ok) return;
    // one group of G::MS states (n_split <= MS, checked on the host), the
    // own one from registers; past n_split, weight 0
    constexpr int MS = G::MS;
    float Mx = -INFINITY, Ls = 0.0f;
    f32x4 macc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) macc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m[MS], l[MS];
    f32x4 so[MS][CPT];
#pragma unroll
    for (int j = 0; j < MS; ++j) {
        const int sp = min(j, a.n_split - 1);
        if (sp == split) {
            m[j] = M;
            l[j] = L;
#pragma unroll
            for (int k = 0; k < CPT; ++k) so[j][k] = acc[k];
        } else {
            const float2 ml = load2_sc1(rm, (int)(((size_t)sp * plane + prow0) * 8));
            m[j] = ml.x;
            l[j] = ml.y;
            const int po = (int)(((size_t)sp * plane + prow0) * RHD * 4);
#pragma unroll
            for (int k = 0; k < CPT; ++k) so[j][k] = load_sc1(ro, po + 16 * cidx(k));
        }
        if (j >= a.n_split) m[j] = -INFINITY;
    }
    merge_split_states<MS, CPT>(Mx, Ls, macc, m, l, so);
    store_rows(macc, Ls);
}

// ---------------------------------------------------------------------------
// 16-row waves at head dim 256: one 16-row block per workgroup, 4 waves, each
// a key group streaming its own tiles as attn_ring_kernel does, on
// v_mfma_f32_16x16x32_bf16 (the lane mappings of attn_fwd_kernel's 16-row
// waves: lane (n16, g16) = query row n16, contraction / key group g16; LDS
// row R of a K tile holds key kappa(R), so that the S^T accumulators of the
// two 16-key blocks give each lane the keys 8 g16 .. 8 g16 + 7 that the PV
// product wants from it).  A wave's O^T takes 64 registers instead of the
// 128 of a 32-row wave, and half the rows per workgroup give twice the
// workgroups: a short key band fills the chip without a key split, so no
// split partials go through memory and no merge tail follows the loop.  No
// key splits, no Q epilogue beyond the QK-norm, bias and RoPE of the 32-row
// kernel's Q load.
template <int HD>
struct Ring16 {
    static constexpr int RW = 4;                  // waves (key groups) per workgroup
    static constexpr int ROWS = 16;               // query rows per workgroup
    static constexpr int RT = BN * HD;            // bf16 elements per K tile (and per V^T tile)
    static constexpr int KCH = HD / 8;            // 16-byte chunks per K row
    static constexpr int VCH = BN / 8;            // 16-byte chunks per V^T row
    static constexpr int NDMA = RT * 2 / 1024;    // 1 KB DMA instructions per tile
    static constexpr int NC = HD / 32;            // contraction steps of QK^T (32 dims each)
    static constexpr int ND = HD / 16;            // 16-dim blocks of O^T
    static constexpr int TPR = RW * 64 / ROWS;    // threads per query row (Q load, final pass)
    static constexpr int QP = HD / 4 / TPR;       // f32x4 pieces per thread and row
    static constexpr int RING_BYTES = RW * 2 * RT * 2;
    static constexpr int Q_BYTES = ROWS * HD * 2;
    static constexpr int ML_OFF = RING_BYTES + Q_BYTES;  // [RW][16] max, then [RW][16] sum
    static constexpr int LDS = ML_OFF + 2 * RW * ROWS * 4;
    static_assert(HD == 256, "built for head dim 256");
    static_assert(ROWS * HD * 4 <= 2 * RT * 2, "a wave's O^T partial fits its K + V^T buffers");
    static_assert(QP % 2 == 0, "RoPE pairs sit in one thread");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NDMA < 32, "two tiles of DMA fit the vmcnt counter");
};

template <int HD, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attn_ring16_kernel(const AttnArgs a) {
    using G = Ring16<HD>;
    constexpr int RW = G::RW, RT = G::RT, R_KCH = G::KCH, R_VCH = G::VCH, NDMA = G::NDMA;
    constexpr int RHD = HD, TPR = G::TPR, QP = G::QP, NC = G::NC, ND = G::ND, ROWS = G::ROWS;
    constexpr int RING_BYTES = G::RING_BYTES, ML_OFF = G::ML_OFF;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_red[3];

    AttnSlot S = a.slot[0];
    const float* qn_w = a.qn_w;
    int q_bf16 = a.q_bf16;
    const float* qb = a.qb;
    const float* rope = a.rope;
    asm volatile("" : "+s"(S.q), "+s"(S.out), "+s"(S.qpos), "+s"(S.qseq), "+s"(S.qprefix),
                 "+s"(S.k), "+s"(S.vt), "+s"(S.nq), "+s"(S.nk), "+s"(S.qpos_sorted), "+s"(qn_w),
                 "+s"(S.qpos0), "+s"(q_bf16), "+s"(qb), "+s"(rope)
                 : "s"(a.n_batch), "s"(a.n_head_kv), "s"(a.group), "s"(a.cap),
                   "s"(a.q_rstride), "s"(a.rowgroups), "s"(a.mg_rowgroups), "s"(a.mg_hkv), "s"(a.c),
                   "s"(a.n_wg), "s"(a.window), "s"(a.prefix));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, g16 = lane >> 4;

    // Workgroup -> (batch, kv head, row group); consecutive logical ids (the
    // row groups of one kv head) share an XCD and its L2.
    const int nwg = a.n_wg;
    const int hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int q2 = udiv(lid, a.rowgroups, a.mg_rowgroups);
    const int rg = lid - q2 * a.rowgroups;
    const int b = udiv(q2, a.n_head_kv, a.mg_hkv);
    const int g = q2 - b * a.n_head_kv;
    if (a.n_batch > 1) S = a.slot[b];

    const int rows_total = a.group * S.nq;
    const int wg_row0 = rg * ROWS;
    if (wg_row0 >= rows_total) return;  // uniform over the workgroup
    const float inv_nq = __builtin_amdgcn_rcpf((float)S.nq);
    auto split_row = [&](int r, int& hgo, int& qio) __attribute__((always_inline)) {
        if (a.group == 1) {
            hgo = 0;
            qio = r;
        } else {
            row_split(r, S.nq, inv_nq, a.group, hgo, qio);
        }
    };

    // ---- Q rows (as attn_ring_kernel): thread tid holds the QP f32x4 pieces
    // d0 + (HD / QP) p of workgroup row tid / TPR
    constexpr int QSTR = HD / QP;
    const int qlr = tid / TPR;
    const int qd0 = (tid % TPR) * 4;
    const int qr = wg_row0 + qlr;
    const bool qok = qr < rows_total;
    f32x4 xq[QP], wq[QP], bq4[QP];
    u32x2 xq16[QP];
    f32x4 tab[QP / 2][2];
    int tab_pos = 0;
    auto load_tab = [&](int pos) __attribute__((always_inline)) {
        const float* trow = rope + ((size_t)pos * (RHD / 2) + qd0) * 2;
#pragma unroll
        for (int p = 0; p < QP / 2; ++p) {
            tab[p][0] = gload<f32x4>(trow + 2 * QSTR * p);
            tab[p][1] = gload<f32x4>(trow + 2 * QSTR * p + 4);
        }
    };
    {
        int qhg, qqi;
        split_row(qok ? qr : 0, qhg, qqi);
        const size_t qoff = (size_t)qqi * a.q_rstride + (size_t)(g * a.group + qhg) * RHD + qd0;
        if (q_bf16) {
            const uint16_t* qrow = static_cast<const uint16_t*>(S.q) + qoff;
#pragma unroll
            for (int p = 0; p < QP; ++p) xq16[p] = gload<u32x2>(qrow + QSTR * p);
        } else {
            const float* qrow = static_cast<const float*>(S.q) + qoff;
#pragma unroll
            for (int p = 0; p < QP; ++p) xq[p] = gload<f32x4>(qrow + QSTR * p);
        }
        if (qn_w) {
#pragma unroll
            for (int p = 0; p < QP; ++p) wq[p] = gload<f32x4>(qn_w + qd0 + QSTR * p);
        }
        if (qb) {
            const float* bq = qb + (size_t)(g * a.group + qhg) * RHD;
#pragma unroll
            for (int p = 0; p < QP; ++p) bq4[p] = gload<f32x4>(bq + qd0 + QSTR * p);
        }
        if (rope) {
            if (S.qpos0 >= 0)
                load_tab(S.qpos0 + qqi);
            else
                tab_pos = gload<int>(S.qpos + qqi);
        }
    }

    // ---- this lane's query row (n16), its mask state, the key-tile range
    const int r = wg_row0 + n16;
    const bool rvalid = r < rows_total;
    int hg = 0, qi = 0;
    if (rvalid) split_row(r, hg, qi);
    int kt_lo = 0, kt_hi = (S.nk + BN - 1) / BN;
    int my_qpos = 0, my_qseq = 0, my_pref = -1;
    int qmin = 0, qmax = 0;
    bool tiles_can_be_full = MODE == MASK_NONE;
    if constexpr (MODE == MASK_POS) {
        my_qpos = S.qpos0 >= 0 ? S.qpos0 + (rvalid ? qi : 0) : gload<int>(S.qpos + (rvalid ? qi : 0));
        if (S.qseq) my_qseq = gload<int>(S.qseq + (rvalid ? qi : 0));
        my_pref = S.qprefix ? (rvalid ? gload<int>(S.qprefix + qi) : -1) : a.prefix;
        bool prefix_free;
        if (S.qpos_sorted && S.qprefix == nullptr) {
            const int r1 = min(wg_row0 + ROWS, rows_total) - 1;
            const int h0 = wg_row0 / S.nq, h1 = r1 / S.nq;
            const int lo = h0 == h1 ? wg_row0 - h0 * S.nq : 0;
            const int hi = h0 == h1 ? r1 - h0 * S.nq : S.nq - 1;
            if (S.qpos0 >= 0) {
                qmin = S.qpos0 + lo;
                qmax = S.qpos0 + hi;
            } else {
                qmin = *(const __attribute__((address_space(4))) int*)(S.qpos + lo);
                qmax = *(const __attribute__((address_space(4))) int*)(S.qpos + hi);
            }
            prefix_free = a.prefix < 0 || qmin >= a.prefix;
        } else {
            int vmin = rvalid ? my_qpos : INT_MAX;
            int vmax = rvalid ? my_qpos : INT_MIN;
            int pref_row = (rvalid && my_pref >= 0 && my_qpos < my_pref) ? 1 : 0;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                vmin = min(vmin, __shfl_xor(vmin, off));
                vmax = max(vmax, __shfl_xor(vmax, off));
                pref_row |= __shfl_xor(pref_row, off);
            }
            if (wave == 0 && lane == 0) {
                s_red[0] = vmin;
                s_red[1] = vmax;
                s_red[2] = pref_row;
            }
            __syncthreads();
            qmin = s_red[0];
            qmax = s_red[1];
            prefix_free = s_red[2] == 0;
        }
        tiles_can_be_full = prefix_free && S.qseq == nullptr;
        if (a.window >= 0) band_tile_range(S.nk, a.window, qmin, qmax, kt_lo, kt_hi);
    }
    const int t0 = kt_lo, nt = kt_hi - kt_lo;

    // ---- K / V^T planes of kv head g and this wave's DMA offsets: LDS row R
    // of a K tile holds key kappa(R), chunks swizzled by R; V^T row d chunks
    // swizzled by swz_v16(d)
    const uint32_t plane_bytes = (uint32_t)a.cap * RHD * 2;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(S.k + (size_t)g * a.cap * RHD, plane_bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(S.vt + (size_t)g * RHD * a.cap, plane_bytes);
    int kvo[NDMA], vvo[NDMA];
#pragma unroll
    for (int j = 0; j < NDMA; ++j) {
        const int idx = j * 64 + lane;
        const int R = idx / R_KCH, pk = idx % R_KCH;
        kvo[j] = (kappa(R) * RHD + ((pk ^ swz<R_KCH>(R)) << 3)) * 2;
        const int d = idx / R_VCH, pv = idx % R_VCH;
        vvo[j] = (d * BN + ((pv ^ swz_v16(d)) << 3)) * 2;
    }
    uint16_t* const kbuf = smem + wave * 2 * RT;
    uint16_t* const vbuf = kbuf + RT;
    auto issue_k = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma16(rk, kbuf + j * 512, kvo[j], t * (BN * RHD * 2));
    };
    auto issue_v = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma16(rv, vbuf + j * 512, vvo[j], t * (BN * RHD * 2));
    };
    auto issue_v_to_k = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma16(rv, kbuf + j * 512, vvo[j], t * (BN * RHD * 2));
    };
    // wave w takes tiles t0 + w, t0 + w + RW, ... (a fixed assignment: the
    // same summation order every call)
    const RingWaveTiles wt(t0, nt, wave, RW, 0, a.cap / BN);
    const int kw = wt.kw;
    auto tile_at = [&](int k) __attribute__((always_inline)) { return wt.at(k); };
    issue_k(wt.first_dma());

    if (rope && S.qpos0 < 0) load_tab(tab_pos);
    if (q_bf16) {
#pragma unroll
        for (int p = 0; p < QP; ++p) {
            const u32x2 w = xq16[p];
            xq[p] = f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                          __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
        }
    }
    if (qb) {
#pragma unroll
        for (int p = 0; p < QP; ++p) xq[p] += bq4[p];
    }
    if (qn_w) {
        double ss = 0.0;
#pragma unroll
        for (int p = 0; p < QP; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sq = xq[p][e] * xq[p][e];
                ss += (double)sq;
            }
#pragma unroll
        for (int off = 1; off < TPR; off <<= 1) ss += __shfl_xor(ss, off);
        const float sc = 1.0f / (float)sqrt(ss / (double)RHD + (double)a.qn_eps);
#pragma unroll
        for (int p = 0; p < QP; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
                xq[p][e] = xq[p][e] * sc * wq[p][e];
            }
    }
    if (rope) {
#pragma unroll
        for (int p = 0; p < QP / 2; ++p)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sn = tab[p][e >> 1][2 * (e & 1)], cs = tab[p][e >> 1][2 * (e & 1) + 1];
                const float lo = xq[p][e], hi = xq[p + QP / 2][e];
                xq[p][e] = rope_lo(lo, hi, sn, cs);
                xq[p + QP / 2][e] = rope_hi(lo, hi, sn, cs);
            }
    }
    uint16_t* const qs = smem + RING_BYTES / 2;
#pragma unroll
    for (int p = 0; p < QP; ++p) {
        const int d = qd0 + QSTR * p;
        bf16x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (__bf16)(qok ? xq[p][e] * a.c : 0.0f);
        *reinterpret_cast<bf16x4*>(qs + qlr * RHD + (((d >> 3) ^ swz<R_KCH>(qlr)) << 3) + (d & 7)) = y;
    }
    lds_barrier();  // (the first K tile stays in flight)
    issue_v(wt.first_dma());
    // Q^T fragments: lane (n16, g16) supplies row n16, dims 32 c + 8 g16 .. + 8
    bf16x8 qf[NC];
    {
        const uint16_t* qrow = qs + n16 * RHD;
        const int sw = swz<R_KCH>(n16);
#pragma unroll
        for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const bf16x8*>(qrow + (((4 * c + g16) ^ sw) << 3));
    }

    f32x4 o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f32x4{};
    float mu = 0.0f;
    bool m_set = false;
    float thr = -INFINITY;
    float l_acc = 0.0f;
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    float negm = 0.0f;  // -m: the accumulator init of QK^T

    // V^T fragments of a tile: lane (n16, g16) supplies row d = 16 db + n16,
    // keys 8 g16 .. + 8 (the keys of the P^T operand it holds)
    auto read_v = [&](const uint16_t* vsrc, bf16x8 (&vf)[ND]) __attribute__((always_inline)) {
#pragma unroll
        for (int db = 0; db < ND; ++db) {
            const int d = 16 * db + n16;
            vf[db] = *reinterpret_cast<const bf16x8*>(vsrc + d * BN + ((g16 ^ swz_v16(d)) << 3));
        }
    };
    auto pv = [&](const bf16x8 (&vf)[ND], const bf16x8& pp) __attribute__((always_inline)) {
#pragma unroll
        for (int db = 0; db < ND; ++db) o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[db], pp, o[db], 0, 0, 0);
    };
    // S^T = K Q^T - m of the tile in the K buffer: block b holds LDS rows
    // 16 b + n16; slot i of block b is key 8 g16 + 4 b + i
    auto qk = [&](f32x4& s0, f32x4& s1) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s0[i] = s1[i] = negm;
        const uint16_t* kr0 = kbuf + n16 * RHD;
        const uint16_t* kr1 = kbuf + (16 + n16) * RHD;
        const int sw0 = swz<R_KCH>(n16), sw1 = swz<R_KCH>(16 + n16);
        constexpr int NKH = 2, NCH = NC / NKH;
#pragma unroll
        for (int h = 0; h < NKH; ++h) {
            bf16x8 kf0[NCH], kf1[NCH];
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int cc = h * NCH + c;
                kf0[c] = *reinterpret_cast<const bf16x8*>(kr0 + (((4 * cc + g16) ^ sw0) << 3));
                kf1[c] = *reinterpret_cast<const bf16x8*>(kr1 + (((4 * cc + g16) ^ sw1) << 3));
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf0[c], qf[h * NCH + c], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf1[c], qf[h * NCH + c], s1, 0, 0, 0);
            }
        }
    };
    // masking and the lazily moved max; a row's 32 scores sit in the four
    // lanes n16 + 16 g16
    auto mask_and_max = [&](f32x4& s0, f32x4& s1, int tt, float& alpha) __attribute__((always_inline)) {
        const int kbase = tt * BN;
        bool full = kbase + BN <= S.nk;
        if constexpr (MODE == MASK_POS) {
            const bool win_ok =
                a.window < 0 || (qmax - kbase < a.window && kbase + BN - 1 - qmin < a.window);
            full = full && tiles_can_be_full && win_ok;
        }
        if (!full) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int kidx = kbase + 8 * g16 + j;
                bool vis = kidx < S.nk;
                if constexpr (MODE == MASK_POS)
                    vis = vis & visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
                if (j < 4)
                    s0[j] = vis ? s0[j] : -INFINITY;
                else
                    s1[j - 4] = vis ? s1[j - 4] : -INFINITY;
            }
        }
        float mx = max3(s0[0], s0[1], s0[2]);
        mx = max3(mx, s0[3], s1[0]);
        mx = max3(mx, s1[1], s1[2]);
        mx = __builtin_fmaxf(mx, s1[3]);
        const bool moved = __builtin_amdgcn_ballot_w64(mx > thr) != 0;
        alpha = 1.0f;
        if (moved) {
            float cm = __builtin_fmaxf(mx, __shfl_xor(mx, 16));
            cm = __builtin_fmaxf(cm, __shfl_xor(cm, 32));
            const bool upd = cm > thr;
            const float delta = upd ? cm : 0.0f;
            alpha = upd ? (m_set ? __builtin_amdgcn_exp2f(-delta) : 0.0f) : 1.0f;
            mu += delta;
            m_set = m_set | upd;
            thr = m_set ? RESCALE_THRESHOLD : -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s0[i] -= delta;
                s1[i] -= delta;
            }
            negm = -mu;
            l_acc *= alpha;
        }
        return moved;
    };
    // p = exp2(s) rounded to bf16 in pairs, l += the rounded p
    auto softmax_p = [&](const f32x4& s0, const f32x4& s1, u32x4& pw) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float x0 = j < 2 ? s0[2 * j] : s1[2 * j - 4];
            const float x1 = j < 2 ? s0[2 * j + 1] : s1[2 * j - 3];
            const bf16x2 pr = {(__bf16)__builtin_amdgcn_exp2f(x0), (__bf16)__builtin_amdgcn_exp2f(x1)};
            pw[j] = __builtin_bit_cast(uint32_t, pr);
            l_acc = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_acc, false);
        }
    };
    auto pin = [&](const u32x4& pw) __attribute__((always_inline)) {
        asm volatile("" ::"v"(pw[0]), "v"(pw[1]), "v"(pw[2]), "v"(pw[3]), "v"(l_acc));
    };

    // Software pipeline and DMA order as attn_ring_kernel: step i runs QK^T
    // of tile i and its softmax, and the PV product of tile i - 1 under the
    // exponentials.  K0 V0 | K1 | K2 V1 | K3 V2 | ...; the last tile's V^T
    // goes to the K buffer once its QK^T has read that.
    u32x4 pprev;
    bool last_in_k = false;
    int t = kw > 0 ? tile_at(0) : -1;
    if (t >= 0) {
        wait_vmcnt<NDMA>();
        f32x4 s0, s1;
        qk(s0, s1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const int tn = kw > 1 ? tile_at(1) : -1;
        if (tn >= 0) issue_k(tn);
        float alpha;
        mask_and_max(s0, s1, t, alpha);  // (O is still zero: no rescale)
        softmax_p(s0, s1, pprev);
        t = tn;
    }
    for (int i = 1; t >= 0; ++i) {
        if (i == 1)
            wait_vmcnt<0>();
        else
            wait_vmcnt<NDMA>();
        f32x4 s0, s1;
        qk(s0, s1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const int tn = i + 1 < kw ? tile_at(i + 1) : -1;
        if (tn >= 0)
            issue_k(tn);
        else
            issue_v_to_k(t);
        wait_vmcnt<NDMA>();
        bf16x8 vf[ND];
        read_v(vbuf, vf);
        float alpha;
        const bool moved = mask_and_max(s0, s1, t, alpha);
        u32x4 pcur;
        softmax_p(s0, s1, pcur);
        pv(vf, __builtin_bit_cast(bf16x8, pprev));
#pragma unroll
        for (int k = 0; k < ND; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x402, 1, 0);  // VALU / transcendental
        }
        pin(pcur);
        __builtin_amdgcn_sched_barrier(0);
        if (moved) {
#pragma unroll
            for (int db = 0; db < ND; ++db) o[db] *= alpha;
        }
        pprev = pcur;
        if (tn >= 0) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue_v(t);
        }
        last_in_k = true;
        t = tn;
    }
    wait_vmcnt<0>();
    if (kw > 0) {
        bf16x8 vf[ND];
        read_v(last_in_k ? kbuf : vbuf, vf);
        pv(vf, __builtin_bit_cast(bf16x8, pprev));
    }

    // ---- merge the RW key groups of each row through LDS (as
    // attn_ring_kernel): wave w's O^T (16 rows x HD f32) into its own K and
    // V^T buffers, 16-byte chunk c of row n at chunk c ^ n, then every thread
    // finishes its share of a row
    float* const sm = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + ML_OFF);  // [RW][16]
    float* const sl = sm + RW * ROWS;                                                  // [RW][16]
    float l_tot = l_acc + __shfl_xor(l_acc, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (g16 == 0) {
        sm[wave * ROWS + n16] = m_set ? mu : -INFINITY;
        sl[wave * ROWS + n16] = l_tot;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    {
        // o[db][i] is O^T[d = 16 db + 4 g16 + i][n16]: chunk 4 db + g16 of row n16
        float* myrow = reinterpret_cast<float*>(kbuf) + n16 * RHD;
#pragma unroll
        for (int db = 0; db < ND; ++db)
            *reinterpret_cast<f32x4*>(myrow + 4 * ((4 * db + g16) ^ n16)) = o[db];
    }
    lds_barrier();
    // thread tid: row rr = tid / TPR (TPR = 16: a read's 16 lanes are one
    // row's 16 chunk slots), chunks ch + TPR k
    constexpr int CPT = HD / 4 / TPR;
    const int rr = tid / TPR, ch = tid % TPR;
    const int row = wg_row0 + rr;
    if (row >= rows_total) return;
    float mw[RW];
    float M = -INFINITY, L = 0.0f;
#pragma unroll
    for (int w = 0; w < RW; ++w) {
        mw[w] = sm[w * ROWS + rr];
        M = __builtin_fmaxf(M, mw[w]);
    }
    f32x4 acc[CPT];
#pragma unroll
    for (int k = 0; k < CPT; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < RW; ++w) {
        const float wt_w = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - M);
        const float* prow = reinterpret_cast<const float*>(smem + w * 2 * RT) + rr * RHD;
#pragma unroll
        for (int k = 0; k < CPT; ++k)
            acc[k] += wt_w * *reinterpret_cast<const f32x4*>(prow + 4 * ((ch + TPR * k) ^ rr));
        L += wt_w * sl[w * ROWS + rr];
    }
    int ohg, oqi;
    split_row(row, ohg, oqi);
    const size_t o0 = (size_t)oqi * a.o_rstride + (size_t)(g * a.group + ohg) * RHD;
    const float il = __builtin_amdgcn_rcpf(L);
    if (a.o_bf16) {
        uint16_t* orow = reinterpret_cast<uint16_t*>(S.out) + o0;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const f32x4 v = acc[k] * il;
            const bf16x4 y = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
            gstore(orow + 4 * (ch + TPR * k), y);
        }
    } else {
        float* orow = S.out + o0;
#pragma unroll
        for (int k = 0; k < CPT; ++k) gstore(orow + 4 * (ch + TPR * k), acc[k] * il);
    }
}

template <int HD, int MODE>
hipError_t launch_ring16_mode(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    static bool attr_set = false;
    auto fn = attn_ring16_kernel<HD, MODE>;
    constexpr int lds = Ring16<HD>::LDS;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3(p.n_workgroups), dim3(256), lds, st, a);
    return hipGetLastError();
}

template <int HD, int MODE, int W>
hipError_t launch_ring_mode(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    static bool attr_set = false;
    auto fn = attn_ring_kernel<HD, MODE, W>;
    constexpr int lds = Ring<HD, W>::LDS;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3(p.n_workgroups), dim3(W * 64), lds, st, a);
    return hipGetLastError();
}

template <int HD, int W>
hipError_t launch_ring_hd(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    switch (p.mask) {
        case MASK_NONE: return launch_ring_mode<HD, MASK_NONE, W>(p, a, st);
        case MASK_POS: return launch_ring_mode<HD, MASK_POS, W>(p, a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// The tiles one workgroup streams above which head dim 128 takes 8 waves.
constexpr int RING8_MIN_TILES = 33;

int ring_waves(int hd, int tiles) {
    if (hd == 128) return tiles >= RING8_MIN_TILES ? 8 : 4;
    return hd == 256 ? 4 : 0;
}

bool ring_waves_built(int hd, int waves) {
    return (hd == 128 && (waves == 4 || waves == 8)) || (hd == 256 && waves == 4);
}

int ring_merge_splits(int hd) {
    return hd == 128 ? Ring<128, 4>::MS : (hd == 256 ? Ring<256, 4>::MS : 0);
}

hipError_t launch_ring(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    // (RoPE on Q only at full rotary: see the Q load)
    if (p.w16) {  // 16-row waves: head dim 256, one 16-row block per workgroup, no key split
        if ((a.rope && a.rot != a.hd) || a.hd != 256 || p.hd_tile != 256 || p.n_split != 1 || p.waves != 4)
            return hipErrorInvalidValue;
        switch (p.mask) {
            case MASK_NONE: return launch_ring16_mode<256, MASK_NONE>(p, a, st);
            case MASK_POS: return launch_ring16_mode<256, MASK_POS>(p, a, st);
            default: return hipErrorInvalidValue;
        }
    }
    if ((a.rope && a.rot != a.hd) || a.hd != p.hd_tile || !ring_waves_built(a.hd, p.waves))
        return hipErrorInvalidValue;
    if (a.ticket && a.n_split > ring_merge_splits(a.hd)) return hipErrorInvalidValue;
    if (a.hd == 128) return p.waves == 8 ? launch_ring_hd<128, 8>(p, a, st) : launch_ring_hd<128, 4>(p, a, st);
    return launch_ring_hd<256, 4>(p, a, st);
}

}  // namespace dr
