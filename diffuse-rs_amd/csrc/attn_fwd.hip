// attn_fwd.hip -- fused denoise-step attention for gfx950 (MI355X, CDNA4).
//
// Computes, for every (query row i, head h), the reference's
//   out[i][h] = sum_j softmax_j(scale * q[i][h] . k[j][h/group]) * v[j][h/group]
// over the keys j visible to i (src/model/attention.rs:101-186, visible() at
// :36-57), in one pass over the keys with an online softmax.
//
// Work decomposition.  Query rows of one KV head are cut into "row blocks"
// of 32 rows (GQA: the `group` query heads of a KV head are packed into the
// row dimension, so a K/V tile is read once for all of them).  A workgroup
// owns RB row blocks and a range of 32-key tiles, and runs RB x KQ waves:
// wave (rb, kq) computes row block rb against every KQ-th tile of the range.
// The KQ tiles of a "super-tile" sit side by side in LDS, each shared by the
// RB waves of its key group, so one CU pulls each K/V byte from L2 once per
// RB*32 query rows (L2 -> CU bandwidth is ~59 B/clk per CU on MI355X; with
// 64 rows that is what the MFMAs consume).  At the end the KQ partial
// softmax states of a row block are merged through LDS, which also stages
// the output for full-row, coalesced stores.  When there are too few
// workgroups to fill the chip the key range is also split across
// workgroups (n_split > 1): each writes its partial rows, and a second,
// small kernel (split_merge_kernel) combines them.
//
// Per wave and 32-key block:
//   S^T[key][q] = K Q^T - m  via v_mfma_f32_32x32x16_bf16, A = K (LDS),
//                            B = Q^T fragments (registers), C = -m
//   O^T[d][q]  += V^T P^T    via the same MFMA, A = V^T (LDS),
//                            B = P^T straight from the S^T accumulators.
// Computing the transposed products makes each lane own one query column, so
// the softmax row statistics are per lane (lane and lane^32 share a column),
// and P never leaves registers.  K rows are placed in LDS in a permuted order
// (sigma below) chosen so that lane half `hf` ends up holding keys
// 16*hf .. 16*hf+15 of every 32-key block, which is exactly the contiguous
// 8-key run each half must supply as the B operand of the PV product.
//
// Softmax, log2 domain: Q is multiplied by scale*log2(e) before rounding to
// bf16, and the running max m enters the QK^T product as its accumulator
// init, so p = exp2(S) needs no subtraction.  m is only moved when a score
// exceeds it by more than 8 (p <= 256 is exact enough in bf16/f32), which
// skips the O rescale on almost every tile; O / l does not depend on the
// choice of m.  The first visible key of a column always sets m.  l sums the
// bf16-rounded p that the PV product multiplies (v_dot2 with (1, 1)), so the
// weights normalise exactly.  A row with no visible key ends with l = 0 and
// writes 0 * (1/0) = NaN, like the reference (attention.rs:181-185).
//
// Memory: K is [kv head][key][HD] and V is stored transposed [kv head][d][key]
// (the KV-cache layout written by kv_cache.hip).  Tiles move HBM -> LDS with
// buffer_load_dwordx4 ... lds (16 bytes per lane, no VGPR staging), NS
// super-tiles deep; the per-lane source offsets are loop invariant and the
// tile base travels in a scalar register.  Each lane picks the global chunk
// that belongs at its LDS slot, so the linear DMA writes produce the
// permuted, XOR-swizzled tile image that keeps the MFMA operand reads
// (16 B per lane) free of bank conflicts.  Q is loaded once per workgroup
// (coalesced f32 rows, RMS-normalised when asked, scaled, rounded to bf16)
// into the LDS of the last pipeline stage, before that stage is first used.
#include "attn_common.hpp"

#include <type_traits>

#include <limits.h>
#include <math.h>

namespace dr {
namespace {

template <int HD, int RB, int KQ, int NS, int NP, bool W16 = false>
struct Geometry {
    // W16: two compute waves of 16 query rows per (row block, key group).
    // DS (head dim 512): two compute waves per (row block, key group) that
    // split the head dim: each holds Q and O for its 256-wide half, and the
    // two halves of every score are summed through LDS.
    static constexpr bool DS = HD > 256;
    static constexpr int NE = RB * KQ;         // (row block, key group) pairs: merge entries
    static constexpr int NW = NE * (W16 ? 2 : 1) * (DS ? 2 : 1);  // compute waves per workgroup
    static constexpr int NWT = NW + NP;        // all waves (NP: DMA-only producer waves)
    static constexpr int NT = NWT * 64;
    static constexpr int NDMA = NP > 0 ? NP : NW;  // waves that issue the K/V DMA
    static constexpr int NC = HD / 16;         // QK^T contraction steps
    static constexpr int ND = HD / 32;         // 32-row blocks of O^T
    static constexpr int KCH = HD / 8;         // 16-byte chunks per K row
    static constexpr int VCH = BN / 8;         // 16-byte chunks per V^T row
    static constexpr int TILE = BN * HD;       // bf16 elements per K (or V^T) tile
    static constexpr int SLOT = 2 * TILE;      // K tile then V^T tile
    static constexpr int STAGE = KQ * SLOT;    // one super-tile
    static constexpr int CPT = TILE / 8;       // 16-byte chunks per tile
    static constexpr int NLDW = STAGE / 8 / (NDMA * 64);  // DMA instructions per DMA wave
                                                          // and super-tile
    static constexpr int QROWS = RB * 32;      // query rows per workgroup
    // DS: each compute wave's partial scores (32 x 32 f32), after the stages
    static constexpr size_t XCH_BYTES = DS ? (size_t)NW * 64 * (W16 ? 8 : 16) * 4 : 0;
    static constexpr size_t STAGE_BYTES = (size_t)NS * STAGE * 2 + XCH_BYTES;
    // Q fragments are held in registers for the whole kernel; Q is staged
    // once, through the first slot of the last pipeline stage.
    static constexpr int ROWF = HD + 4;        // f32 row pitch of the merge area
    static constexpr size_t MERGE_BYTES = ((size_t)NE * 32 * ROWF + 2 * NE * 32) * 4;
    static constexpr size_t LDS_BYTES = STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES;
    static constexpr int WAVES_PER_SIMD = (NWT + 3) / 4;
    static_assert(CPT % 64 == 0, "a DMA instruction must stay inside one tile");
    static_assert(STAGE / 8 % (NDMA * 64) == 0, "super-tile must split evenly over the waves");
    static_assert(NLDW * (NS - 1) < 64, "vmcnt range");
    static_assert(QROWS * HD <= SLOT, "Q staging must fit in one tile slot");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(!W16 || HD <= 256 || DS, "16-row waves: head dim up to 256, or split");
    static_assert(!DS || (HD == 512 && NP == 0 && KQ == 1),
                  "head-dim split: head dim 512, one key group, no DMA waves");
};

template <int HD, int RB, int KQ, int NS, int NP, int MODE, bool QEPI, bool W16>
__attribute__((amdgpu_waves_per_eu(Geometry<HD, RB, KQ, NS, NP, W16>::WAVES_PER_SIMD,
                                   Geometry<HD, RB, KQ, NS, NP, W16>::WAVES_PER_SIMD))) __global__
__launch_bounds__((RB * KQ * (W16 ? 2 : 1) * (HD > 256 ? 2 : 1) + NP) * 64) void attn_fwd_kernel(const AttnArgs a) {
    using G = Geometry<HD, RB, KQ, NS, NP, W16>;
    constexpr int NW = G::NW, NWT = G::NWT, NT = G::NT, NC = G::NC, ND = G::ND;
    constexpr int KCH = G::KCH, VCH = G::VCH, TILE = G::TILE, SLOT = G::SLOT;
    constexpr int CPT = G::CPT, NLDW = G::NLDW, ROWF = G::ROWF, QROWS = G::QROWS;

    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_red[3][NWT];

    // Every scalar of the decode and the first loads, and batch slot 0, is
    // requested here at once (wide scalar loads, one wait) rather than by one
    // dependent load at each first use.  The empty asm also keeps the
    // compiler from turning "slot 0 or slot b" below into a pointer select
    // and a second, dependent load.
    AttnSlot S = a.slot[0];
    asm volatile("" : "+s"(S.q), "+s"(S.out), "+s"(S.qpos), "+s"(S.qseq), "+s"(S.qprefix),
                 "+s"(S.k), "+s"(S.vt), "+s"(S.kpos), "+s"(S.kseq), "+s"(S.nq), "+s"(S.nk),
                 "+s"(S.qpos_sorted)
                 : "s"(a.n_batch), "s"(a.n_head_kv), "s"(a.group), "s"(a.hd), "s"(a.cap),
                   "s"(a.q_rstride), "s"(a.rowgroups), "s"(a.n_split), "s"(a.mg_split),
                   "s"(a.mg_rowgroups), "s"(a.mg_hkv), "s"(a.c), "s"(a.n_wg), "s"(a.window),
                   "s"(a.prefix));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, hf = lane >> 5;
    // waves [0, NW) compute (row block rb, key group kq); with NP > 0 waves
    // [NW, NW+NP) only move K/V tiles into LDS, so no compute wave ever
    // stalls behind a memory instruction that the memory system cannot take
    const bool compute = wave < NW;
    const bool dma = NP == 0 || !compute;
    const int dwave = NP > 0 ? wave - NW : wave;  // index among the DMA waves
    const int rb = wave % RB, kq = (wave / RB) % KQ;
    // W16: the wave's half of the row block (rows rh*16 .. rh*16 + 15)
    const int rh = W16 ? (wave / (RB * KQ)) % 2 : 0;

    // Workgroup -> (batch, kv head, row group, split).  The hardware deals
    // workgroups round-robin over the 8 XCDs; remapping keeps consecutive
    // logical ids (same row group, its splits) on one XCD's L2.
    const int nwg = a.n_wg;
    const int hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int q1 = udiv(lid, a.n_split, a.mg_split);
    const int split = lid - q1 * a.n_split;
    const int q2 = udiv(q1, a.rowgroups, a.mg_rowgroups);
    const int rg = q1 - q2 * a.rowgroups;
    const int b = udiv(q2, a.n_head_kv, a.mg_hkv);
    const int g = q2 - b * a.n_head_kv;
    if (a.n_batch > 1) S = a.slot[b];

    const int rows_total = a.group * S.nq;
    const int wg_row0 = rg * QROWS;
    if (wg_row0 >= rows_total) return;  // uniform over the workgroup and all its splits
    const int r = wg_row0 + rb * 32 + (W16 ? rh * 16 + (lane & 15) : col);
    const bool rvalid = r < rows_total;
    const float inv_nq = __builtin_amdgcn_rcpf((float)S.nq);
    int hg = 0, qi = 0;
    if (rvalid) row_split(r, S.nq, inv_nq, a.group, hg, qi);

    // ---- masking state and the key tile range of this workgroup
    int kt_lo = 0, kt_hi = (S.nk + BN - 1) / BN;
    int my_qpos = 0, my_qseq = 0, my_pref = -1;
    int qmin = 0, qmax = 0;
    bool tiles_can_be_full = MODE == MASK_NONE;
    if constexpr (MODE != MASK_NONE) {
        my_qpos = rvalid ? (S.qpos0 >= 0 ? S.qpos0 + qi : S.qpos[qi]) : 0;  // (contiguous: no load)
        my_qseq = (rvalid && S.qseq) ? S.qseq[qi] : 0;
        my_pref = S.qprefix ? (rvalid ? S.qprefix[qi] : -1) : a.prefix;
    }
    if constexpr (MODE == MASK_POS) {
        bool prefix_free;
        if (S.qpos_sorted && S.qprefix == nullptr) {
            // ascending positions: the extremes sit at the ends of the
            // workgroup's query range (the whole range if it spans heads)
            const int r1 = min(wg_row0 + QROWS, rows_total) - 1;
            const int h0 = wg_row0 / S.nq, h1 = r1 / S.nq;
            const int lo = h0 == h1 ? wg_row0 - h0 * S.nq : 0;
            const int hi = h0 == h1 ? r1 - h0 * S.nq : S.nq - 1;
            qmin = S.qpos0 >= 0 ? S.qpos0 + lo : S.qpos[lo];
            qmax = S.qpos0 >= 0 ? S.qpos0 + hi : S.qpos[hi];
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
            if (lane == 0) {
                s_red[0][wave] = vmin;
                s_red[1][wave] = vmax;
                s_red[2][wave] = pref_row;
            }
            __syncthreads();
            qmin = INT_MAX;
            qmax = INT_MIN;
            int anyp = 0;
#pragma unroll
            for (int w = 0; w < NWT; ++w) {
                qmin = min(qmin, s_red[0][w]);
                qmax = max(qmax, s_red[1][w]);
                anyp |= s_red[2][w];
            }
            prefix_free = anyp == 0;
        }
        tiles_can_be_full = prefix_free && S.qseq == nullptr;
        if (a.window >= 0) {
            // keys k with |q - k| < window for some q in [qmin, qmax]
            const long lo = max(0L, (long)qmin - a.window + 1);
            const long hi = min((long)S.nk, (long)qmax + a.window);
            if (hi <= lo) {
                kt_lo = kt_hi = 0;
            } else {
                kt_lo = (int)(lo / BN);
                kt_hi = (int)((hi + BN - 1) / BN);
            }
        }
    }
    const int ntiles = kt_hi - kt_lo;
    const int per = (ntiles + a.n_split - 1) / a.n_split;
    const int t0 = kt_lo + min(split * per, ntiles);
    const int t1 = kt_lo + min((split + 1) * per, ntiles);
    const int nsup = (t1 - t0 + KQ - 1) / KQ;  // super-tiles

    // Tile of slot u (super-tile u) of this wave's key group.
    const int kg = compute ? kq : dwave;  // this wave's key group
    auto tile_at = [&](int u) __attribute__((always_inline)) { return t0 + u * KQ + kg; };

    // ---- DMA plan: instruction j of this wave fills 64 chunks of one tile
    // region (region 2*i is K tile i of the super-tile, 2*i+1 its V^T tile).
    // A wave's instructions cover whole regions or part of one, so the
    // region of instruction j is the wave's first region plus a compile-time
    // offset; the per-lane source offset (bytes from the tile base) is loop
    // invariant and the tile base is a scalar.
    constexpr bool WHOLE = (NLDW * 64) % CPT == 0;
    static_assert(WHOLE || CPT % (NLDW * 64) == 0, "DMA split");
    const int wreg0 = (dwave * NLDW * 64) / CPT;
    auto voff_of = [&](int j, int ln) __attribute__((always_inline)) -> int {
        const int jreg = WHOLE ? (j * 64) / CPT : 0;
        const int idx = (WHOLE ? (j * 64) % CPT : (dwave * NLDW * 64) % CPT + j * 64) + ln;
        if (((wreg0 + jreg) & 1) == 0) {
            const int R = idx / KCH, pk = idx % KCH;
            return (((R & ~31) + kperm<W16>(R & 31)) * HD + ((pk ^ swz<KCH>(R)) << 3)) * 2;
        }
        const int d = idx / VCH, pv = idx % VCH;
        return (d * BN + ((pv ^ (W16 ? swz_v16(d) : swz<VCH>(d))) << 3)) * 2;  // within the V^T tile
    };
    // Compute waves that also issue DMA keep the offsets in registers; DMA
    // waves recompute them per super-tile (they have the issue slots to
    // spare, and the compute waves' registers stay free of them).
    int voff[NP > 0 ? 1 : NLDW];
    if constexpr (NP == 0) {
#pragma unroll
        for (int j = 0; j < NLDW; ++j) voff[j] = voff_of(j, lane);
    }
    const uint32_t plane_bytes = (uint32_t)a.cap * HD * 2;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(S.k + (size_t)g * a.cap * HD, plane_bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(S.vt + (size_t)g * HD * a.cap, plane_bytes);

    // DMA instructions [j0, j1) of super-tile u into stage st.
    auto issue_range = [&](int u, int st, int j0, int j1) __attribute__((always_inline)) {
        const int cofs = WHOLE ? 0 : (dwave * NLDW * 64) % CPT;  // first chunk in the region
        const int ln = lane;
#pragma unroll
        for (int j = 0; j < NLDW; ++j) {
            if (j < j0 || j >= j1) continue;
            const int reg = wreg0 + (WHOLE ? (j * 64) / CPT : 0);
            const int kqr = reg >> 1;
            uint16_t* dst = smem + (kqr * NS + st) * SLOT + (reg & 1) * TILE +
                            ((WHOLE ? (j * 64) % CPT : cofs + j * 64) << 3);
            // slots past the range reload the last tile: in bounds, unused
            const int t = min(t0 + u * KQ + kqr, t1 - 1);
            const int vo = NP > 0 ? voff_of(j, ln) : voff[NP > 0 ? 0 : j];
            // (K tile t and V^T tile t both start at byte t * BN * HD * 2)
            if (reg & 1)
                dma16(rv, dst, vo, t * (BN * HD * 2));
            else
                dma16(rk, dst, vo, t * (BN * HD * 2));
        }
    };
    auto issue = [&](int u, int st) __attribute__((always_inline)) { issue_range(u, st, 0, NLDW); };

    // What a DMA wave does for super-tile u into stage st before the main
    // loop: the DMA.
    auto fill = [&](int u, int st) __attribute__((always_inline)) { issue(u, st); };

    // ---- Q: the workgroup's rows, loaded once (coalesced f32x4 row pieces,
    // requested before the first K/V DMA: they gate the first MFMA),
    // RMS-normalised when asked, times scale*log2(e), rounded to bf16 and
    // stored in the B-operand layout in stage NS-1 (first written by the DMA
    // of super-tile NS-1, issued after the barrier at the top of the loop).
    // A lane holds PPL f32x4 pieces of a row, at d0 + p*HW (head dim 512:
    // two, so that a row fits one wave).
    constexpr int PPL = HD > 256 ? 2 : 1;
    constexpr int HW = HD / PPL;
    constexpr int LPR = HW / 4;       // lanes per row
    constexpr int RPI = 64 / LPR;     // rows per wave instruction
    constexpr int QIT = (QROWS + NWT * RPI - 1) / (NWT * RPI);  // row groups per wave
    const int d0 = (lane % LPR) * 4;
    // workgroup row of this lane in iteration it (rows past QROWS are idle)
    auto q_lrow = [&](int it) __attribute__((always_inline)) {
        return (it * NWT + wave) * RPI + lane / LPR;
    };
    // The epilogue's Q part (QEPI kernels only; bias, QK-norm and RoPE each
    // where its operand is given): its operands are requested with the rows.
    // Kernels without QEPI carry none of this code.  Rows are loaded and
    // written in batches of QB iterations (all at once except with the
    // epilogue at head dim 512, whose operands would not fit the registers).
    constexpr int QB = (QEPI && PPL > 1) ? (QIT < 4 ? QIT : 4) : QIT;
    const int rhalf = QEPI ? a.rot / 2 : 0;
    const bool qbias = QEPI && a.qb != nullptr;
    const bool qrope = QEPI && a.rope != nullptr;
    uint16_t* const qs = smem + (NS - 1) * SLOT;
    // The QK-norm gains of this lane's dims, the same for every row it
    // normalises: loaded once, through the global address space (a generic
    // load inside the row loop may alias the LDS stores of the rows before
    // it, so each one waited for the previous row's store and its own
    // round trip).
    f32x4 wqv[PPL];
    if constexpr (QEPI) {
        if (a.qn_w) {
#pragma unroll
            for (int pc = 0; pc < PPL; ++pc) {
                const int dp = d0 + pc * HW;
                if (a.hd == HD) {
                    wqv[pc] = gload<f32x4>(a.qn_w + dp);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) wqv[pc][e] = dp + e < a.hd ? gload<float>(a.qn_w + dp + e) : 0.0f;
                }
            }
        }
    }
    auto q_batch = [&](const int ib) __attribute__((always_inline)) {
        // Loads first, all of them unconditional and unmasked (rows past the
        // block read row 0, dims past the head a clamped in-row piece, both
        // zeroed after the first K/V DMA is issued): a load on some lanes, or
        // a select of a loaded value before the DMA, made each row wait for
        // the previous row's loads (the branches write the same registers).
        f32x4 xq[QB][PPL];
        f32x4 bq4[QB][PPL];
        f32x4 tq[QB][PPL][2];  // RoPE: the (sin, cos) pairs of a piece's four dims, raw
        bool okq[QB];
        int qp[QB];  // the rows' positions, requested before the rows (RoPE's table index)
#pragma unroll
        for (int ii = 0; ii < QB; ++ii) {
            const int it = ib + ii;
            qp[ii] = 0;
            if constexpr (QEPI) {
                const int rr = wg_row0 + q_lrow(it);
                const bool ok = it < QIT && q_lrow(it) < QROWS && rr < rows_total;
                int hgq = 0, qiq = 0;
                if (ok) row_split(rr, S.nq, inv_nq, a.group, hgq, qiq);
                if (qrope) qp[ii] = S.qpos0 >= 0 ? S.qpos0 + qiq : gload<int>(S.qpos + qiq);
            }
        }
        // (two copies of the loop, picked once: a head dim that is a multiple
        // of 4 loads whole pieces, any other one element by element; one
        // loop holding both kept a wait between them on every row)
        auto load_rows = [&](auto vec_tag) __attribute__((always_inline)) {
            constexpr bool VEC = decltype(vec_tag)::value;
#pragma unroll
        for (int ii = 0; ii < QB; ++ii) {
            const int it = ib + ii;
            const int rr = wg_row0 + q_lrow(it);
            const bool ok = it < QIT && q_lrow(it) < QROWS && rr < rows_total;
            okq[ii] = ok;
            int hgq = 0, qiq = 0;
            if (ok) row_split(rr, S.nq, inv_nq, a.group, hgq, qiq);
            const int qh = g * a.group + hgq;
            const float* qrow = static_cast<const float*>(S.q) + (size_t)qiq * a.q_rstride +
                                (size_t)qh * a.hd;
#pragma unroll
            for (int pc = 0; pc < PPL; ++pc) {
                const int dp = d0 + pc * HW;
                if constexpr (VEC) {
                    const int dpc = min(dp, a.hd - 4);
                    xq[ii][pc] = gload<f32x4>(qrow + dpc);
                    if (qbias) bq4[ii][pc] = gload<f32x4>(a.qb + (size_t)qh * a.hd + dpc);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) xq[ii][pc][e] = (ok && dp + e < a.hd) ? qrow[dp + e] : 0.0f;
                    if (qbias) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            bq4[ii][pc][e] = (ok && dp + e < a.hd) ? a.qb[(size_t)qh * a.hd + dp + e] : 0.0f;
                    }
                }
                if (qrope) {
                    // dims dp .. dp+3 lie on one side of rot/2 (a multiple of 4):
                    // their four (sin, cos) pairs are 32 contiguous bytes of the
                    // table (a piece past rot reads the last in-range one, unused)
                    const int dr = min(dp, a.rot - 4);
                    const int j0 = dr < rhalf ? dr : dr - rhalf;
                    const float* t = a.rope + ((size_t)qp[ii] * rhalf + j0) * 2;
                    tq[ii][pc][0] = gload<f32x4>(t);
                    tq[ii][pc][1] = gload<f32x4>(t + 4);
                }
            }
        }
        };
        if (a.hd % 4 == 0)
            load_rows(std::true_type{});
        else
            load_rows(std::false_type{});

        if (ib == 0 && dma) {  // (first batch only)
#pragma unroll
            for (int i = 0; i < NS - 1; ++i)
                if (i < nsup) fill(i, i);
        }

#pragma unroll
        for (int ii = 0; ii < QB; ++ii) {
            const int it = ib + ii;
            f32x4 x[PPL];
#pragma unroll
            for (int pc = 0; pc < PPL; ++pc) {
                const bool in = okq[ii] && d0 + pc * HW < a.hd;
                x[pc] = in ? xq[ii][pc] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (qbias && in) x[pc] += bq4[ii][pc];  // add_bias (ops.rs:373-382)
            }
            if (QEPI && a.qn_w) {
                // rms_norm_inplace (ops.rs:106-114): f32 squares summed in f64.
                double ss = 0.0;
#pragma unroll
                for (int pc = 0; pc < PPL; ++pc)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float sq = x[pc][e] * x[pc][e];
                        ss += (double)sq;
                    }
#pragma unroll
                for (int off = 1; off < LPR; off <<= 1) ss += __shfl_xor(ss, off);
                const float sc = 1.0f / (float)sqrt(ss / (double)a.hd + (double)a.qn_eps);
#pragma unroll
                for (int pc = 0; pc < PPL; ++pc)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + pc * HW + e < a.hd) x[pc][e] = x[pc][e] * sc * wqv[pc][e];
            }
            if (qrope) {
                // rotate_rows (ops.rs:433-452): dim d < rot pairs with d +- rot/2,
                // held by piece (d +- rot/2) / HW of this row's lane
                // ((d +- rot/2) % HW) / 4 (rot is a multiple of 8)
                f32x4 xp[PPL];
#pragma unroll
                for (int pc = 0; pc < PPL; ++pc) {
                    const int dp = d0 + pc * HW;
                    const int dq = dp < rhalf ? dp + rhalf : dp - rhalf;
                    const int src = dp < a.rot ? lane - lane % LPR + (dq % HW) / 4 : lane;
                    const int pq = dp < a.rot ? dq / HW : pc;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float v = __shfl(x[0][e], src);
                        if constexpr (PPL > 1) {
                            const float v1 = __shfl(x[1][e], src);
                            v = pq == 0 ? v : v1;
                        }
                        xp[pc][e] = v;
                    }
                }
#pragma unroll
                for (int pc = 0; pc < PPL; ++pc) {
                    const int dp = d0 + pc * HW;
                    if (dp < a.rot) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            x[pc][e] = dp < rhalf
                                           ? rope_lo(x[pc][e], xp[pc][e], tq[ii][pc][e >> 1][2 * (e & 1)],
                                                     tq[ii][pc][e >> 1][2 * (e & 1) + 1])
                                           : rope_hi(xp[pc][e], x[pc][e], tq[ii][pc][e >> 1][2 * (e & 1)],
                                                     tq[ii][pc][e >> 1][2 * (e & 1) + 1]);
                    }
                }
            }
            const int lr = q_lrow(it);  // row within the workgroup
            const int rl = lr & 31;     // row within its row block (the swizzle key)
#pragma unroll
            for (int pc = 0; pc < PPL; ++pc) {
                const int dp = d0 + pc * HW;
                bf16x4 y;
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = (__bf16)(x[pc][e] * a.c);
                if (it < QIT && lr < QROWS)
                    *reinterpret_cast<bf16x4*>(qs + lr * HD + (((dp >> 3) ^ swz<KCH>(rl)) << 3) +
                                               (dp & 7)) = y;
            }
        }
    };
    if constexpr (QB == QIT) {
        q_batch(0);
    } else {
#pragma unroll
        for (int ib = 0; ib < QIT; ib += QB) q_batch(ib);
    }
    __syncthreads();
    const uint16_t* qrow_l = qs + (rb * 32 + col) * HD;
    auto qfrag = [&](int c) __attribute__((always_inline)) {
        return *reinterpret_cast<const bf16x8*>(qrow_l + (((2 * c + hf) ^ swz<KCH>(col)) << 3));
    };
    // The merge area of the epilogue (it overlays the tile stages).
    // One entry per (row block, key group) = k * RB + rb.
    constexpr int NE = G::NE;
    float* mrows = reinterpret_cast<float*>(smem);  // [NE][32][ROWF]
    float* sm = mrows + NE * 32 * ROWF;             // [NE][32] running max
    float* sl = sm + NE * 32;                       // [NE][32] scaled sum

    // Compute waves and DMA-only waves run separate loops with the same
    // number of barriers, so that none of the compute state (O, P, V^T and Q
    // fragments) is live in the DMA waves' code.
    if (W16 && compute) {
        if constexpr (W16) {
            // 16 query rows per wave on 16x16x32 MFMAs: two compute waves per
            // SIMD, so the softmax of one overlaps the matrix products of the
            // other.  Lane (g16, n16): query row n16, contraction / key group
            // g16.  Same transposed products as the 32-row waves: S^T = K Q^T
            // in two 16-key blocks, O^T += V^T P^T.
            // Head dim 512 (WDS): the head dim is also split, as in the
            // 32-row head-dim-split branch below: wave dh holds Q and O^T of
            // dims [256 dh, 256 dh + 256), and the two halves of the scores
            // meet in LDS after the QK^T product.
            constexpr bool WDS = G::DS;
            constexpr int NC16 = HD / 32;  // contraction steps of 32 along d
            constexpr int ND16 = HD / 16;  // 16-row blocks of O^T
            constexpr int NCW = WDS ? NC16 / 2 : NC16;  // this wave's contraction steps
            constexpr int NDW = WDS ? ND16 / 2 : ND16;  // this wave's 16-row blocks of O^T
            const int dh = WDS ? wave / (RB * KQ * 2) : 0;
            const int c0 = dh * NCW, db0 = dh * NDW;
            const int n16 = lane & 15, g16 = lane >> 4;
            const int qr = rb * 32 + rh * 16 + n16;  // query row within the workgroup
            bf16x8 qf[NCW];
            {
                const uint16_t* qrow = qs + qr * HD;
                const int sw = swz<KCH>(qr & 31);
#pragma unroll
                for (int c = 0; c < NCW; ++c)
                    qf[c] = *reinterpret_cast<const bf16x8*>(qrow + (((4 * (c0 + c) + g16) ^ sw) << 3));
            }
            f32x4 o[NDW];
#pragma unroll
            for (int db = 0; db < NDW; ++db) o[db] = f32x4{};
            float mu = 0.0f;  // running max m (log2 units), valid once m_set
            bool m_set = false;
            float thr = -INFINITY;  // a score above mu + thr moves m
            float l_acc = 0.0f;     // this lane's share of the row's weight sum
            const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

            // O^T += V^T P^T; contraction slot 8*g16 + j is key 8*g16 + j in
            // both operands.
            auto pv = [&](const bf16x8 (&vf)[NDW], const bf16x8& pf) __attribute__((always_inline)) {
#pragma unroll
                for (int db = 0; db < NDW; ++db)
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[db], pf, o[db], 0, 0, 0);
            };
            // One super-tile, software-pipelined like the 32-row step: the
            // previous tile's PV product is interleaved with this tile's
            // softmax, and this tile's V^T fragments replace vf afterwards.
            // Without DMA waves (NP == 0, head dim 256) the compute waves wait
            // for and issue the K/V DMA themselves, in three parts spread over
            // the step as the 32-row step does.
            constexpr int J1 = NLDW / 4, J2 = NLDW / 2;
            // Head dim 256 has no registers for V^T fragments held across a
            // step: its PV product runs in the tile's own step, the fragments
            // read in two halves (PIPE16 false).
            constexpr bool PIPE16 = HD <= 128;
            auto step = [&](int u, bf16x8 (&vf)[NDW], const bf16x8& pin, bf16x8& pout)
                __attribute__((always_inline)) {
                const int st = u % NS;
                if constexpr (NP == 0) wait_tiles<NLDW, NS>(min(NS - 2, nsup - 1 - u));
                __syncthreads();  // super-tile u visible to all waves; u-1 (and Q) fully consumed
                const int un = u + NS - 1, stn = (u + NS - 1) % NS;
                const bool pf = NP == 0 && un < nsup;
                if (t0 + u * KQ + kq >= t1) {  // this key group has no tile in the last super-tile
                    if (pf) issue(un, stn);
                    if constexpr (PIPE16) pv(vf, pin);
                    pout = bf16x8{};
                    return;
                }
                if (pf) issue_range(un, stn, 0, J1);
                const int t = t0 + u * KQ + kq;
                const uint16_t* ks = smem + (kq * NS + st) * SLOT;
                const uint16_t* vs = ks + TILE;
                const int kbase_t = t * BN;

                // score j = 4*b + i of this lane is key kbase_t + 8*g16 + j
                int kp[8], kqs[8];
                if constexpr (MODE == MASK_KEYS) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int kidx = min(kbase_t + 8 * g16 + j, S.nk - 1);
                        kp[j] = S.kpos ? S.kpos[kidx] : kidx;
                        kqs[j] = S.kseq ? S.kseq[kidx] : 0;
                    }
                }

                // S^T = K Q^T - m: block b holds LDS rows 16*b + n16 (keys
                // kappa of them), -m as the accumulator init.
                f32x4 s0, s1;
#pragma unroll
                for (int i = 0; i < 4; ++i) s0[i] = s1[i] = (WDS && dh != 0) ? 0.0f : -mu;
                {
                    // (head dim 256: the K fragments in two halves, the second
                    // read while the MFMAs of the first run)
                    constexpr int NKH = HD > 128 ? 2 : 1, NCH = NCW / NKH;
                    const uint16_t* kr0 = ks + n16 * HD;
                    const uint16_t* kr1 = ks + (16 + n16) * HD;
                    const int sw0 = swz<KCH>(n16), sw1 = swz<KCH>(16 + n16);
#pragma unroll
                    for (int h = 0; h < NKH; ++h) {
                        bf16x8 kf0[NCH], kf1[NCH];
#pragma unroll
                        for (int c = 0; c < NCH; ++c) {
                            const int cc = c0 + h * NCH + c;
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
                }
                __builtin_amdgcn_sched_barrier(0);
                if (pf) issue_range(un, stn, J1, J2);
                if constexpr (WDS) {
                    // both halves of every score through LDS; the pair adds
                    // them (IEEE addition commutes: both get the same sums)
                    float* xch = reinterpret_cast<float*>(smem + NS * G::STAGE);
                    f32x4* mine = reinterpret_cast<f32x4*>(xch) + wave * 128;
                    mine[lane] = s0;
                    mine[64 + lane] = s1;
                    __syncthreads();
                    const f32x4* theirs =
                        reinterpret_cast<const f32x4*>(xch) + ((wave + RB * KQ * 2) % NW) * 128;
                    s0 += theirs[lane];
                    s1 += theirs[64 + lane];
                }

                bool full = kbase_t + BN <= S.nk;
                if constexpr (MODE == MASK_POS) {
                    const bool win_ok = a.window < 0 || (qmax - kbase_t < a.window &&
                                                         kbase_t + BN - 1 - qmin < a.window);
                    full = full && tiles_can_be_full && win_ok;
                } else if constexpr (MODE == MASK_KEYS) {
                    full = false;
                }
                if (!full) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int kidx = kbase_t + 8 * g16 + j;
                        bool vis = kidx < S.nk;
                        if constexpr (MODE == MASK_POS) {
                            vis = vis & visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
                        } else if constexpr (MODE == MASK_KEYS) {
                            vis = vis & visible(my_qpos, kp[j], my_qseq, kqs[j], a.window, my_pref);
                        }
                        if (j < 4)
                            s0[j] = vis ? s0[j] : -INFINITY;
                        else
                            s1[j - 4] = vis ? s1[j - 4] : -INFINITY;
                    }
                }

                // Online softmax with a lazily moved max; a row's 32 scores sit
                // in the four lanes n16 + 16*g16.
                float mx = max3(s0[0], s0[1], s0[2]);
                mx = max3(mx, s0[3], s1[0]);
                mx = max3(mx, s1[1], s1[2]);
                mx = __builtin_fmaxf(mx, s1[3]);
                const bool moved = __builtin_amdgcn_ballot_w64(mx > thr) != 0;
                float alpha = 1.0f;
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
                    l_acc *= alpha;
                }

                // p = exp2(s) rounded to bf16 in pairs; l sums the rounded
                // values (what the PV product multiplies).
                u32x4 w4;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float x0 = j < 2 ? s0[2 * j] : s1[2 * j - 4];
                    const float x1 = j < 2 ? s0[2 * j + 1] : s1[2 * j - 3];
                    const bf16x2 pr = {(__bf16)__builtin_amdgcn_exp2f(x0),
                                       (__bf16)__builtin_amdgcn_exp2f(x1)};
                    w4[j] = __builtin_bit_cast(uint32_t, pr);
                    l_acc = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_acc, false);
                }
                pout = __builtin_bit_cast(bf16x8, w4);
                if constexpr (PIPE16) {
                    pv(vf, pin);
#pragma unroll
                    for (int i = 0; i < ND16; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                        __builtin_amdgcn_sched_group_barrier(0x402, 2, 0);  // two VALU / transcendental
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (moved) {
#pragma unroll
                    for (int db = 0; db < NDW; ++db) o[db] *= alpha;
                }
                if (pf) issue_range(un, stn, J2, NLDW);
                // this tile's V^T fragments: rows 16*(db0 + db) + n16, keys 8*g16 ..
                auto vfrag = [&](int db) __attribute__((always_inline)) {
                    const int d = 16 * (db0 + db) + n16;
                    return *reinterpret_cast<const bf16x8*>(vs + d * BN + ((g16 ^ swz_v16(d)) << 3));
                };
                if constexpr (PIPE16) {
#pragma unroll
                    for (int db = 0; db < NDW; ++db) vf[db] = vfrag(db);
                } else {
                    constexpr int NVH = NDW / 2;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        bf16x8 vh[NVH];
#pragma unroll
                        for (int i = 0; i < NVH; ++i) vh[i] = vfrag(h * NVH + i);
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int i = 0; i < NVH; ++i)
                            o[h * NVH + i] =
                                __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh[i], pout, o[h * NVH + i], 0, 0, 0);
                    }
                }
            };

            {
                bf16x8 vf[NDW], pa, pb;
#pragma unroll
                for (int db = 0; db < NDW; ++db) vf[db] = bf16x8{};
                pa = bf16x8{};
                int u = 0;
                for (; u + 1 < nsup; u += 2) {
                    step(u, vf, pa, pb);
                    step(u + 1, vf, pb, pa);
                }
                if (u < nsup) {
                    step(u, vf, pa, pb);
                    if constexpr (PIPE16) pv(vf, pb);
                } else if constexpr (PIPE16) {
                    pv(vf, pa);
                }
            }

            // ---- merge the KQ key groups: entry kq * RB + rb, rows rh*16 + n16
            float l_tot = l_acc + __shfl_xor(l_acc, 16);
            l_tot += __shfl_xor(l_tot, 32);
            const float m_fin = m_set ? mu : -INFINITY;
            const int e = kq * RB + rb, row32 = rh * 16 + n16;
            __syncthreads();  // every wave is done with the tile stages
            if (g16 == 0 && dh == 0) sm[e * 32 + row32] = m_fin;
            __syncthreads();
            {
                float M = -INFINITY;
#pragma unroll
                for (int k = 0; k < KQ; ++k) M = __builtin_fmaxf(M, sm[(k * RB + rb) * 32 + row32]);
                const float sc = (m_fin == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_fin - M);
                // o[db][i] is O^T[d = 16*(db0 + db) + 4*g16 + i][n16]
                float* myrow = mrows + (e * 32 + row32) * ROWF + 16 * db0;
#pragma unroll
                for (int db = 0; db < NDW; ++db)
                    *reinterpret_cast<f32x4*>(myrow + 16 * db + 4 * g16) = o[db] * sc;
                if (g16 == 0 && dh == 0) sl[e * 32 + row32] = l_tot * sc;
            }
        }
    } else if (G::DS && compute) {
        if constexpr (G::DS && !W16) {
            // Head dim 512: the wave pair (rb, dh = 0 / 1) shares 32 query rows
            // and splits the head dim.  Wave dh holds the Q fragments and the
            // O^T rows of dims [256 dh, 256 dh + 256): it computes its half of
            // every score, the two halves meet in LDS, and both waves add them
            // (IEEE addition commutes, so both hold the same scores and take
            // the same softmax steps) before each multiplies P into its half
            // of V^T.  One key group, so every wave reads every tile.
            static_assert(KQ == 1, "head-dim split: one key group");
            constexpr int NCH = NC / 2;  // contraction steps of this wave's half
            constexpr int NDH = ND / 2;  // 32-row blocks of this wave's half of O^T
            const int dh = wave / (RB * KQ);
            const int partner = (wave + RB * KQ) % NW;
            float* xch = reinterpret_cast<float*>(smem + NS * G::STAGE);  // [NW][4][64] f32x4
            bf16x8 qf[NCH];
#pragma unroll
            for (int c = 0; c < NCH; ++c) qf[c] = qfrag(dh * NCH + c);

            f32x16 o[NDH];
#pragma unroll
            for (int db = 0; db < NDH; ++db) o[db] = f32x16{};
            float mu = 0.0f;  // running max m (log2 units), valid once m_set
            bool m_set = false;
            float thr = -INFINITY;  // a score above mu + thr moves m
            float l_lo = 0.0f, l_hi = 0.0f;
            const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
            constexpr int J1 = NLDW / 4, J2 = NLDW / 2;

            for (int u = 0; u < nsup; ++u) {
                const int st = u % NS;
                wait_tiles<NLDW, NS>(min(NS - 2, nsup - 1 - u));
                __syncthreads();  // super-tile u visible to all waves; u-1 (and Q) fully consumed
                const int un = u + NS - 1, stn = (u + NS - 1) % NS;
                const bool pf = un < nsup;
                const int t = t0 + u;
                const uint16_t* ks = smem + st * SLOT;
                const uint16_t* vs = ks + TILE;
                const int kbase_t = t * BN;
                int kp[16], kqs[16];
                if constexpr (MODE == MASK_KEYS) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int kidx = min(kbase_t + 16 * hf + i, S.nk - 1);
                        kp[i] = S.kpos ? S.kpos[kidx] : kidx;
                        kqs[i] = S.kseq ? S.kseq[kidx] : 0;
                    }
                }
                if (pf) issue_range(un, stn, 0, J1);
                __builtin_amdgcn_sched_barrier(0);

                // this half of S^T = K Q^T; wave 0 of the pair starts from -m
                f32x16 s;
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = dh == 0 ? -mu : 0.0f;
                {
                    constexpr int NH = NCH / 2;
                    const uint16_t* krow = ks + col * HD;
                    const int sw = swz<KCH>(col);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        bf16x8 kf[NH];
#pragma unroll
                        for (int c = 0; c < NH; ++c)
                            kf[c] = *reinterpret_cast<const bf16x8*>(
                                krow + (((2 * (dh * NCH + h * NH + c) + hf) ^ sw) << 3));
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int c = 0; c < NH; ++c)
                            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[c], qf[h * NH + c], s, 0, 0, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                {
                    f32x4* mine = reinterpret_cast<f32x4*>(xch) + wave * 256;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        mine[j * 64 + lane] = f32x4{s[4 * j], s[4 * j + 1], s[4 * j + 2], s[4 * j + 3]};
                }
                // this half of V^T, read while the partner finishes its scores
                bf16x8 vf[NDH][2];
#pragma unroll
                for (int db = 0; db < NDH; ++db) {
                    const int d = (dh * NDH + db) * 32 + col;
                    const uint16_t* vrow = vs + d * BN;
                    const int sw = swz<VCH>(d);
                    vf[db][0] = *reinterpret_cast<const bf16x8*>(vrow + (((2 * hf) ^ sw) << 3));
                    vf[db][1] = *reinterpret_cast<const bf16x8*>(vrow + (((2 * hf + 1) ^ sw) << 3));
                }
                if (pf) issue_range(un, stn, J1, J2);
                __syncthreads();  // both halves of every score are in LDS
                {
                    const f32x4* theirs = reinterpret_cast<const f32x4*>(xch) + partner * 256;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const f32x4 x = theirs[j * 64 + lane];
#pragma unroll
                        for (int e = 0; e < 4; ++e) s[4 * j + e] += x[e];
                    }
                }

                // Masking: s[i] is the score of key t*BN + 16*hf + i.
                bool full = kbase_t + BN <= S.nk;
                if constexpr (MODE == MASK_POS) {
                    const bool win_ok = a.window < 0 || (qmax - kbase_t < a.window &&
                                                         kbase_t + BN - 1 - qmin < a.window);
                    full = full && tiles_can_be_full && win_ok;
                } else if constexpr (MODE == MASK_KEYS) {
                    full = false;
                }
                if (!full) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int kidx = kbase_t + 16 * hf + i;
                        bool vis = kidx < S.nk;
                        if constexpr (MODE == MASK_POS) {
                            vis = vis & visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
                        } else if constexpr (MODE == MASK_KEYS) {
                            vis = vis & visible(my_qpos, kp[i], my_qseq, kqs[i], a.window, my_pref);
                        }
                        s[i] = vis ? s[i] : -INFINITY;
                    }
                }

                // Online softmax with a lazily moved max, as in the 32-row step.
                float mx = max3(s[0], s[1], s[2]);
#pragma unroll
                for (int i = 3; i < 15; i += 2) mx = max3(mx, s[i], s[i + 1]);
                mx = __builtin_fmaxf(mx, s[15]);
                const bool moved = __builtin_amdgcn_ballot_w64(mx > thr) != 0;
                if (moved) {
                    const float cm = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
                    const bool upd = cm > thr;
                    const float delta = upd ? cm : 0.0f;
                    const float alpha = upd ? (m_set ? __builtin_amdgcn_exp2f(-delta) : 0.0f) : 1.0f;
                    mu += delta;
                    m_set = m_set | upd;
                    thr = m_set ? RESCALE_THRESHOLD : -INFINITY;
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[i] -= delta;
                    l_lo *= alpha;
                    l_hi *= alpha;
#pragma unroll
                    for (int db = 0; db < NDH; ++db) o[db] *= alpha;
                }
                bf16x8 pw[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    u32x4 w4;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float p0 = __builtin_amdgcn_exp2f(s[8 * hh + 2 * j]);
                        const float p1 = __builtin_amdgcn_exp2f(s[8 * hh + 2 * j + 1]);
                        const bf16x2 pr = {(__bf16)p0, (__bf16)p1};
                        w4[j] = __builtin_bit_cast(uint32_t, pr);
                        if (hh == 0)
                            l_lo = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_lo, false);
                        else
                            l_hi = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_hi, false);
                    }
                    pw[hh] = __builtin_bit_cast(bf16x8, w4);
                }
                __builtin_amdgcn_sched_barrier(0);
                if (pf) issue_range(un, stn, J2, NLDW);
#pragma unroll
                for (int db = 0; db < NDH; ++db) {
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][0], pw[0], o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][1], pw[1], o[db], 0, 0, 0);
                }
            }

            // ---- merge: the pair's two halves form one entry's row
            const float l_run = l_lo + l_hi;
            const float l_tot = l_run + __shfl_xor(l_run, 32);
            const float m_fin = m_set ? mu : -INFINITY;
            const int ent = kq * RB + rb;
            __syncthreads();  // every wave is done with the tile stages and the exchange
            if (hf == 0 && dh == 0) sm[ent * 32 + col] = m_fin;
            __syncthreads();
            {
                float M = -INFINITY;
#pragma unroll
                for (int k = 0; k < KQ; ++k) M = __builtin_fmaxf(M, sm[(k * RB + rb) * 32 + col]);
                const float sc = (m_fin == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_fin - M);
                // o[db][4j + e] is O^T[d = 256 dh + db*32 + 8j + 4hf + e][col]
                float* myrow = mrows + (ent * 32 + col) * ROWF + dh * (HD / 2);
#pragma unroll
                for (int db = 0; db < NDH; ++db)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        f32x4 val;
#pragma unroll
                        for (int e = 0; e < 4; ++e) val[e] = o[db][4 * j + e] * sc;
                        *reinterpret_cast<f32x4*>(myrow + db * 32 + 8 * j + 4 * hf) = val;
                    }
                if (hf == 0 && dh == 0) sl[ent * 32 + col] = l_tot * sc;
            }
        }
    } else if (NP == 0 || compute) {
        // (16-row and head-dim-split builds never reach this branch: every
        // compute wave took one of the two above)
        if constexpr (!G::DS && !W16) {
            bf16x8 qf[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) qf[c] = qfrag(c);

            // ---- main loop over super-tiles
            f32x16 o[ND];
#pragma unroll
            for (int db = 0; db < ND; ++db) o[db] = f32x16{};
            float mu = 0.0f;          // running max m (log2 units), valid once m_set
            bool m_set = false;
            float thr = -INFINITY;    // a score above mu + thr moves m
            float l_lo = 0.0f, l_hi = 0.0f;
            const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

            // O^T += V^T P^T for one tile whose V^T fragments and P are in registers.
            // Contraction slot 8*hf + j of MFMA hh is key 16*hf + 8*hh + j, in both
            // operands.
            auto pv = [&](const bf16x8 (&vf)[ND][2], const bf16x8 (&pf)[2]) __attribute__((always_inline)) {
#pragma unroll
                for (int db = 0; db < ND; ++db) {
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][0], pf[0], o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][1], pf[1], o[db], 0, 0, 0);
                }
            };

            // One super-tile.  A compute wave software-pipelines its tiles: the PV
            // product of its previous tile (V^T fragments vf and P pin, in registers)
            // is issued in program order between the VALU instructions of this
            // tile's softmax, so the matrix core and the VALU work at the same time
            // (with one compute wave per SIMD nothing else would fill either).  This
            // tile's P goes to pout, and its V^T fragments replace vf once those
            // MFMAs have read them (one set of V^T registers, which leaves room for
            // Q's); the first step multiplies zero fragments.  Without DMA waves (NP == 0)
            // the DMA of super-tile u+NS-1 is issued in three parts spread over the
            // compute, so that no wave stalls on a burst of memory instructions in
            // front of its MFMAs.  Head dim 256 has no registers for a second set of
            // V^T fragments (Q stays in registers there): its PV product is issued
            // in the step of its tile, after the softmax (PIPE false).
            constexpr bool PIPE = HD <= 128;
            constexpr int J1 = NLDW / 4, J2 = NLDW / 2;
            auto step = [&](int u, bf16x8 (&vf)[ND][2], const bf16x8 (&pin)[2], bf16x8 (&pout)[2])
                __attribute__((always_inline)) {
                const int st = u % NS;
                if (dma) wait_tiles<NLDW, NS>(min(NS - 2, nsup - 1 - u));
                __syncthreads();  // super-tile u visible to all waves; u-1 (and Q) fully consumed
                const int un = u + NS - 1, stn = (u + NS - 1) % NS;
                const bool pf = NP == 0 && un < nsup;

                if (t0 + u * KQ + kq >= t1) {  // this key group has no tile in the last super-tile
                    if (pf) issue(un, stn);
                    if constexpr (PIPE) pv(vf, pin);
                    pout[0] = pout[1] = bf16x8{};  // vf holds finite values: nothing is added
                    return;
                }
                const int t = tile_at(u);
                const uint16_t* ks = smem + (kq * NS + st) * SLOT;
                const uint16_t* vs = ks + TILE;
                const int kbase_t = t * BN;

                // per-key metadata (arbitrary key positions / ids): loaded per tile
                int kp[16], kqs[16];
                if constexpr (MODE == MASK_KEYS) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int kidx = min(kbase_t + 16 * hf + i, S.nk - 1);
                        kp[i] = S.kpos ? S.kpos[kidx] : kidx;
                        kqs[i] = S.kseq ? S.kseq[kidx] : 0;
                    }
                }
                if (pf) issue_range(un, stn, 0, J1);
                __builtin_amdgcn_sched_barrier(0);

                // S^T = K Q^T - m: -m enters as the accumulator init, so the scores
                // come out relative to m.  The K fragments are requested in two
                // halves, the second while the MFMAs of the first run.
                f32x16 s;
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = -mu;
                {
                    constexpr int NH = NC / 2;
                    const uint16_t* krow = ks + col * HD;
                    const int sw = swz<KCH>(col);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        bf16x8 kf[NH];
#pragma unroll
                        for (int c = 0; c < NH; ++c)
                            kf[c] = *reinterpret_cast<const bf16x8*>(
                                krow + (((2 * (h * NH + c) + hf) ^ sw) << 3));
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int c = 0; c < NH; ++c)
                            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[c], qf[h * NH + c], s, 0, 0, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);

                // this tile's V^T fragments
                auto read_v = [&]() __attribute__((always_inline)) {
#pragma unroll
                    for (int db = 0; db < ND; ++db) {
                        const int d = db * 32 + col;
                        const uint16_t* vrow = vs + d * BN;
                        const int sw = swz<VCH>(d);
                        vf[db][0] = *reinterpret_cast<const bf16x8*>(vrow + (((2 * hf) ^ sw) << 3));
                        vf[db][1] = *reinterpret_cast<const bf16x8*>(vrow + (((2 * hf + 1) ^ sw) << 3));
                    }
                };
                if constexpr (!PIPE) read_v();
                if (pf) issue_range(un, stn, J1, J2);

                // Masking: s[i] is the score of key t*BN + 16*hf + i.
                bool full = kbase_t + BN <= S.nk;
                if constexpr (MODE == MASK_POS) {
                    const bool win_ok = a.window < 0 || (qmax - kbase_t < a.window &&
                                                         kbase_t + BN - 1 - qmin < a.window);
                    full = full && tiles_can_be_full && win_ok;
                } else if constexpr (MODE == MASK_KEYS) {
                    full = false;
                }
                if (!full) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int kidx = kbase_t + 16 * hf + i;
                        bool vis = kidx < S.nk;
                        if constexpr (MODE == MASK_POS) {
                            vis = vis & visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
                        } else if constexpr (MODE == MASK_KEYS) {
                            vis = vis & visible(my_qpos, kp[i], my_qseq, kqs[i], a.window, my_pref);
                        }
                        s[i] = vis ? s[i] : -INFINITY;
                    }
                }

                // Online softmax with a lazily moved max (scores are relative to mu).
                float mx = max3(s[0], s[1], s[2]);
#pragma unroll
                for (int i = 3; i < 15; i += 2) mx = max3(mx, s[i], s[i + 1]);
                mx = __builtin_fmaxf(mx, s[15]);
                // The column max over both lane halves decides, so lane and lane^32
                // move m together.  O is rescaled after the previous tile's PV
                // product (whose P is relative to the old m) has gone into it, and
                // before this tile's.
                const bool moved = __builtin_amdgcn_ballot_w64(mx > thr) != 0;
                float alpha = 1.0f;
                if (moved) {
                    const float cm = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
                    const bool upd = cm > thr;
                    const float delta = upd ? cm : 0.0f;
                    alpha = upd ? (m_set ? __builtin_amdgcn_exp2f(-delta) : 0.0f) : 1.0f;
                    mu += delta;
                    m_set = m_set | upd;
                    thr = m_set ? RESCALE_THRESHOLD : -INFINITY;
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[i] -= delta;
                    l_lo *= alpha;
                    l_hi *= alpha;
                }

                // p = exp2(s) rounded to bf16 in pairs; l sums the rounded values
                // (what the PV product multiplies), so the weights normalise exactly.
                // The previous tile's PV MFMAs are interleaved with this VALU work.
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    u32x4 w4;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float p0 = __builtin_amdgcn_exp2f(s[8 * hh + 2 * j]);
                        const float p1 = __builtin_amdgcn_exp2f(s[8 * hh + 2 * j + 1]);
                        const bf16x2 pr = {(__bf16)p0, (__bf16)p1};
                        w4[j] = __builtin_bit_cast(uint32_t, pr);
                        if (hh == 0)
                            l_lo = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_lo, false);
                        else
                            l_hi = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l_hi, false);
                    }
                    pout[hh] = __builtin_bit_cast(bf16x8, w4);
                }
                if constexpr (PIPE) {
                    pv(vf, pin);
#pragma unroll
                    for (int i = 0; i < 2 * ND; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                        __builtin_amdgcn_sched_group_barrier(0x402, 4, 0);  // four VALU / transcendental
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (moved) {
#pragma unroll
                    for (int db = 0; db < ND; ++db) o[db] *= alpha;
                }
                if constexpr (PIPE) read_v();
                if (pf) issue_range(un, stn, J2, NLDW);
                if constexpr (!PIPE) pv(vf, pout);
            };

            {
                bf16x8 vf[ND][2], pfa[2], pfb[2];
#pragma unroll
                for (int db = 0; db < ND; ++db) vf[db][0] = vf[db][1] = bf16x8{};
                pfa[0] = pfa[1] = bf16x8{};
                int u = 0;
                for (; u + 1 < nsup; u += 2) {
                    step(u, vf, pfa, pfb);
                    step(u + 1, vf, pfb, pfa);
                }
                if (u < nsup) {
                    step(u, vf, pfa, pfb);
                    if (PIPE) pv(vf, pfb);
                } else if (PIPE) {
                    pv(vf, pfa);
                }
            }

            // ---- merge the KQ key groups of each row block through LDS
            const float l_run = l_lo + l_hi;
            const float l_tot = l_run + __shfl_xor(l_run, 32);
            const float m_fin = m_set ? mu : -INFINITY;
            __syncthreads();  // every wave is done with the tile stages
            if (hf == 0) sm[wave * 32 + col] = m_fin;
            __syncthreads();
            {
                float M = -INFINITY;
#pragma unroll
                for (int k = 0; k < KQ; ++k) M = __builtin_fmaxf(M, sm[(k * RB + rb) * 32 + col]);
                const float sc = (m_fin == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_fin - M);
                // o[db][4j + e] is O^T[d = db*32 + 8j + 4hf + e][col]
                float* myrow = mrows + (wave * 32 + col) * ROWF;
#pragma unroll
                for (int db = 0; db < ND; ++db)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        f32x4 val;
#pragma unroll
                        for (int e = 0; e < 4; ++e) val[e] = o[db][4 * j + e] * sc;
                        *reinterpret_cast<f32x4*>(myrow + db * 32 + 8 * j + 4 * hf) = val;
                    }
                if (hf == 0) sl[wave * 32 + col] = l_tot * sc;
            }
        }
    } else {
        for (int u = 0; u < nsup; ++u) {
            wait_tiles<NLDW, NS>(min(NS - 2, nsup - 1 - u));
            __syncthreads();
            const int un = u + NS - 1;
            if (un < nsup) issue(un, un % NS);
        }
        __syncthreads();  // the two barriers of the compute waves' merge
        __syncthreads();
    }
    __syncthreads();

    constexpr int CHUNKS = HD / 4;
    const size_t rows_pad = (size_t)a.rowgroups * QROWS;
    const size_t bg = (size_t)b * a.n_head_kv + g;
    if (a.n_split == 1) {
        for (int item = tid; item < QROWS * CHUNKS; item += NT) {
            const int rr = item / CHUNKS, ch = item % CHUNKS;
            const int rbi = rr >> 5, ci = rr & 31;
            const int rglob = wg_row0 + rr;
            if (rglob >= rows_total) continue;
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            float L = 0.0f;
#pragma unroll
            for (int k = 0; k < KQ; ++k) {
                const int wi = k * RB + rbi;
                acc += *reinterpret_cast<const f32x4*>(mrows + (wi * 32 + ci) * ROWF + ch * 4);
                L += sl[wi * 32 + ci];
            }
            const int c0 = ch * 4;
            int hgi, qii;
            row_split(rglob, S.nq, inv_nq, a.group, hgi, qii);
            float* orow = S.out + (size_t)qii * a.o_rstride + (size_t)(g * a.group + hgi) * a.hd;
            const f32x4 val = acc * __builtin_amdgcn_rcpf(L);
            if (a.hd == HD) {
                *reinterpret_cast<f32x4*>(orow + c0) = val;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c0 + e < a.hd) orow[c0 + e] = val[e];
            }
        }
        return;
    }

    // ---- key split: this split's partial rows (the sum over its key groups,
    // relative to the row max M, with M and the sum of weights L) go to the
    // split workspace; split_merge_kernel, launched next on the same stream,
    // combines the splits.  The kernel boundary orders the writes before the
    // merge's reads, so no cross-workgroup protocol is needed here.
    const size_t plane = (size_t)a.n_batch * a.n_head_kv * rows_pad;  // rows per split
    float* po = a.part_o + (size_t)split * plane * HD;
    float* pml = a.part_ml + (size_t)split * plane * 2;
    for (int item = tid; item < QROWS * CHUNKS; item += NT) {
        const int rr = item / CHUNKS, ch = item % CHUNKS;
        const int rbi = rr >> 5, ci = rr & 31;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f, Mrow = -INFINITY;
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
            const int wi = k * RB + rbi;
            acc += *reinterpret_cast<const f32x4*>(mrows + (wi * 32 + ci) * ROWF + ch * 4);
            L += sl[wi * 32 + ci];
            Mrow = __builtin_fmaxf(Mrow, sm[wi * 32 + ci]);
        }
        const size_t prow = bg * rows_pad + wg_row0 + rr;  // row within a split plane
        *reinterpret_cast<f32x4*>(po + prow * HD + ch * 4) = acc;
        if (ch == 0) *reinterpret_cast<float2*>(pml + prow * 2) = make_float2(Mrow, L);
    }
}

// Combines the key splits of an attention launch: one thread per (row of a
// split plane, 16-byte chunk of HD).  Row r of (batch b, kv head g) merges the
// n_split partial states (M_s, L_s, acc_s) as softmax states merge:
// out = sum_s w_s acc_s / sum_s w_s L_s with w_s = exp2(M_s - max_s M_s) (a
// split with no visible key has M_s = -inf and weight 0; a row with none at
// all ends 0 * (1/0) = NaN, as in the unsplit kernel).
template <int HD>
__global__ __launch_bounds__(256) void split_merge_kernel(const AttnArgs a) {
    constexpr int CHUNKS = HD / 4;
    const size_t plane = (size_t)a.n_batch * a.n_head_kv * a.part_rows;
    const size_t item = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (item >= plane * CHUNKS) return;
    const size_t prow = item / CHUNKS;
    const int ch = (int)(item % CHUNKS);
    const int bg = (int)(prow / a.part_rows), r = (int)(prow % a.part_rows);
    const int b = bg / a.n_head_kv, g = bg % a.n_head_kv;
    // (a row past the slot's rows is merged from whatever its workspace row
    // holds and not stored: testing first put a wait for the slot's row
    // count, a dynamically indexed argument, in front of every partial load)
    float Mx = -INFINITY, Ls = 0.0f;
    f32x4 acc[1] = {{0.0f, 0.0f, 0.0f, 0.0f}};
    // Partials within 2^31 bytes (the usual case) are read with buffer loads:
    // one per-thread offset and the split's plane offset as a scalar, so the
    // SG loads of a group need no address registers of their own (with 64-bit
    // addresses the compiler held back loads until earlier ones returned).
    // SG, the splits whose loads are issued together: 4 up to 4 splits, else
    // 8.  (Slots past n_split reload the last split and weigh 0; at 4 splits
    // a group of 8 doubled the loads the address unit handles.)
    auto groups = [&](auto buffered, auto sgc) __attribute__((always_inline)) {
        constexpr bool BUF = decltype(buffered)::value;
        constexpr int SG = decltype(sgc)::value;
        const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.part_o, 0xffffffffu);
        const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.part_ml, 0xffffffffu);
        const int vo = (int)((prow * HD + ch * 4) * 4), vm = (int)(prow * 8);
        for (int s0 = 0; s0 < a.n_split; s0 += SG) {
            float m[SG], l[SG];
            f32x4 o[SG][1];
#pragma unroll
            for (int j = 0; j < SG; ++j) {
                const int sp = min(s0 + j, a.n_split - 1);
                float2 ml;
                if constexpr (BUF) {
                    const auto w = __builtin_amdgcn_raw_buffer_load_b64(rm, vm, (int)((size_t)sp * plane * 8), 0);
                    ml = make_float2(__uint_as_float(w[0]), __uint_as_float(w[1]));
                    o[j][0] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, vo, (int)((size_t)sp * plane * HD * 4), 0));
                } else {
                    ml = *reinterpret_cast<const float2*>(a.part_ml + ((size_t)sp * plane + prow) * 2);
                    o[j][0] = *reinterpret_cast<const f32x4*>(a.part_o + ((size_t)sp * plane + prow) * HD + ch * 4);
                }
                const bool in = s0 + j < a.n_split;
                m[j] = in ? ml.x : -INFINITY;
                l[j] = ml.y;
            }
            __builtin_amdgcn_sched_barrier(0);  // (every load above before any wait)
            merge_split_states<SG, 1>(Mx, Ls, acc, m, l, o);
        }
    };
    const bool buffered = (size_t)a.n_split * plane * HD * 4 <= 0x7fffffffu;  // (uniform)
    if (a.n_split <= 4) {
        if (buffered)
            groups(std::integral_constant<bool, true>{}, std::integral_constant<int, 4>{});
        else
            groups(std::integral_constant<bool, false>{}, std::integral_constant<int, 4>{});
    } else {
        if (buffered)
            groups(std::integral_constant<bool, true>{}, std::integral_constant<int, 8>{});
        else
            groups(std::integral_constant<bool, false>{}, std::integral_constant<int, 8>{});
    }
    const AttnSlot& S = a.slot[b];
    if (r >= a.group * S.nq) return;
    int hg, qi;
    row_split(r, S.nq, __builtin_amdgcn_rcpf((float)S.nq), a.group, hg, qi);
    const size_t o0 = (size_t)qi * a.o_rstride + (size_t)(g * a.group + hg) * a.hd;
    float* orow = S.out + o0;
    const f32x4 val = acc[0] * __builtin_amdgcn_rcpf(Ls);
    const int c0 = ch * 4;
    if (a.o_bf16) {  // (the per-wave-stream kernel's launches only: hd == HD)
        const bf16x4 y = {(__bf16)val[0], (__bf16)val[1], (__bf16)val[2], (__bf16)val[3]};
        *reinterpret_cast<bf16x4*>(reinterpret_cast<uint16_t*>(S.out) + o0 + c0) = y;
    } else if (a.hd == HD) {
        *reinterpret_cast<f32x4*>(orow + c0) = val;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (c0 + e < a.hd) orow[c0 + e] = val[e];
    }
}

template <int HD, int RB, int KQ, int NS, int NP, int MODE, bool QEPI, bool W16 = false>
hipError_t launch_fwd(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    using G = Geometry<HD, RB, KQ, NS, NP, W16>;
    constexpr size_t lds = G::LDS_BYTES;
    static bool attr_set = false;
    auto fn = attn_fwd_kernel<HD, RB, KQ, NS, NP, MODE, QEPI, W16>;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3(p.n_workgroups), dim3(G::NT), lds, st, a);
    return hipGetLastError();
}

// The 16-row-wave builds.
template <int HD, int RB, int KQ, int NS, int NP>
hipError_t launch_modes16(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    switch (p.mask) {
        case MASK_NONE:
            return p.qepi ? launch_fwd<HD, RB, KQ, NS, NP, MASK_NONE, true, true>(p, a, st)
                           : launch_fwd<HD, RB, KQ, NS, NP, MASK_NONE, false, true>(p, a, st);
        case MASK_POS:
            return p.qepi ? launch_fwd<HD, RB, KQ, NS, NP, MASK_POS, true, true>(p, a, st)
                           : launch_fwd<HD, RB, KQ, NS, NP, MASK_POS, false, true>(p, a, st);
        default:
            if (p.qepi) return hipErrorInvalidValue;
            return launch_fwd<HD, RB, KQ, NS, NP, MASK_KEYS, false, true>(p, a, st);
    }
}

template <int HD, int RB, int KQ, int NS, int NP>
hipError_t launch_modes(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    switch (p.mask) {
        case MASK_NONE:
            return p.qepi ? launch_fwd<HD, RB, KQ, NS, NP, MASK_NONE, true>(p, a, st)
                           : launch_fwd<HD, RB, KQ, NS, NP, MASK_NONE, false>(p, a, st);
        case MASK_POS:
            return p.qepi ? launch_fwd<HD, RB, KQ, NS, NP, MASK_POS, true>(p, a, st)
                           : launch_fwd<HD, RB, KQ, NS, NP, MASK_POS, false>(p, a, st);
        default:
            if (p.qepi) return hipErrorInvalidValue;
            return launch_fwd<HD, RB, KQ, NS, NP, MASK_KEYS, false>(p, a, st);
    }
}

// The workgroup shapes built for each head-dim tile: RB row blocks x KQ key
// groups of compute waves, NP DMA-only waves, NS pipeline stages (super-tiles
// of KQ x (K + V^T) tiles of 32 keys).
struct Shape {
    int hd, rb, kq, ns, np;
    bool w16;  // two 16-row compute waves per (row block, key group)
};
constexpr Shape SHAPES[] = {
    {64, 1, 4, 3, 4, false}, {64, 2, 2, 4, 4, false}, {64, 2, 4, 3, 0, false},
    {128, 1, 4, 2, 4, false}, {128, 2, 2, 4, 4, false}, {128, 2, 4, 2, 0, false},
    {128, 1, 4, 2, 4, true}, {256, 2, 2, 2, 0, true},
    {256, 2, 2, 2, 0, false}, {256, 1, 2, 2, 0, false},  // 32-row waves: one per SIMD, 512 VGPRs
    {512, 2, 1, 2, 0, false},  // head-dim split, 32-row waves: a pair per row block, one per SIMD
    {512, 2, 1, 2, 0, true},   // ... and with 16-row waves: 8 compute waves, two per SIMD
};

const Shape* find_shape(int hd_tile, int rb, int kq, bool w16) {
    for (const Shape& s : SHAPES)
        if (s.hd == hd_tile && s.rb == rb && s.kq == kq && s.w16 == w16) return &s;
    return nullptr;
}

hipError_t launch_shape(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    if (p.w16) {
        if (p.hd_tile == 128 && p.rb == 1 && p.kq == 4) return launch_modes16<128, 1, 4, 2, 4>(p, a, st);
        if (p.hd_tile == 256 && p.rb == 2 && p.kq == 2) return launch_modes16<256, 2, 2, 2, 0>(p, a, st);
        if (p.hd_tile == 512 && p.rb == 2 && p.kq == 1) return launch_modes16<512, 2, 1, 2, 0>(p, a, st);
        return hipErrorInvalidValue;
    }
    const int key = p.hd_tile * 100 + p.rb * 10 + p.kq;
    switch (key) {
        case 6414: return launch_modes<64, 1, 4, 3, 4>(p, a, st);
        case 6422: return launch_modes<64, 2, 2, 4, 4>(p, a, st);
        case 6424: return launch_modes<64, 2, 4, 3, 0>(p, a, st);
        case 12814: return launch_modes<128, 1, 4, 2, 4>(p, a, st);
        case 12822: return launch_modes<128, 2, 2, 4, 4>(p, a, st);
        case 12824: return launch_modes<128, 2, 4, 2, 0>(p, a, st);
        case 25622: return launch_modes<256, 2, 2, 2, 0>(p, a, st);
        case 25612: return launch_modes<256, 1, 2, 2, 0>(p, a, st);
        case 51221: return launch_modes<512, 2, 1, 2, 0>(p, a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// Longest key band (32-key tiles) for which head dim 256 takes 16-row waves.
constexpr int RING16_MAX_TILES = 44;

LaunchPlan plan_attention(int hd, int n_batch, int n_head_kv, int group, int max_nq, int max_nk,
                          int mask, int qepi, int window, int rot, int n_cu, int force_rb, int force_kq,
                          int force_split, int force_rows, int force_kernel, bool merge_in_kernel,
                          int key_band) {
    LaunchPlan p{};
    p.hd_tile = hd <= 64 ? 64 : (hd <= 128 ? 128 : (hd <= 256 ? 256 : 512));
    p.block_n = BN;
    p.mask = mask;
    p.qepi = qepi != QEPI_NONE;  // (no key-masked build carries the Q epilogue: its launch fails)
    p.kernel = KERNEL_STAGED;
    const int cus = n_cu > 0 ? n_cu : 256;
    const int row_blocks = (group * max_nq + 31) / 32;  // per (batch, kv head)
    const int ntiles = (max_nk + BN - 1) / BN;
    // Head dim exactly 128 or 256 without per-key metadata, with a Q
    // epilogue of at most the bias, the QK-norm and a full-rotary RoPE: the
    // per-wave key streams of attn_ring_kernel (one 32-row
    // block per workgroup, 8 or 4 key groups).  A 32-row workgroup pulls
    // every K/V byte of its key range through its CU, so the call is bound by
    // that stream; independent per-wave DMA keeps it nearer the CU's rate
    // than the staged kernel's shared super-tiles.  Picked when the one-block
    // workgroups fit one round of the CUs, and at head dim 256 when each
    // workgroup's key band is short: a sliding window of at most 1024 (a band
    // of at most ~2k keys, where the staged kernel's 64-row blocks would need
    // a key split: DiffusionGemma's sliding layers take 21.6 against
    // 28.7 us), or a band of at most 4608 keys that two in-kernel-merged
    // splits fill the chip with (16/8 heads, 256 queries, no window: 18.3
    // against 28.9 us at 1280 keys, 23.2 against 30.1 at 2304, a tie at
    // 4352; at 8448 and 16640 keys the staged kernel's 64-row split blocks
    // win, 57.0 against 62.2 and 94.4 against 109.4; window 2500 over 6256
    // keys, canvas rows at the end, a 2755-key band: 27.4 against 34.3).  When one-block
    // workgroups would take more than one round of the CUs (C3's GQA rows:
    // 448 blocks on 256 CUs), the staged kernel's 64-row workgroups read each
    // K/V tile once for twice the rows and keep them.
    const int ring_blocks = n_batch * n_head_kv * row_blocks;
    // keys of the widest band a workgroup reads: from the query rows'
    // positions when the caller knows them, else the window's worst case
    // (plus a tile for the band's alignment)
    int band = window >= 0 && 2 * window + BN < max_nk ? 2 * window + BN : max_nk;
    if (key_band > 0 && key_band + BN < band) band = key_band + BN;
    const int band_tiles = ((band < max_nk ? band : max_nk) + BN - 1) / BN;
    // waves per workgroup for the unsplit band (the split below is sized with
    // it; the final count follows from the tiles a split workgroup streams)
    const int rw = ring_waves(hd, band_tiles);
    const bool ring_ok = rw > 0 && mask != MASK_KEYS && (qepi != QEPI_FULL || rot == 0 || rot == hd);
    const bool ring_short_band = hd == 256 && merge_in_kernel && 2 * ring_blocks <= cus && band <= 4608 &&
                                 ntiles >= 2 * rw;
    const bool ring_auto =
        ring_blocks <= cus && (hd == 128 || (window >= 0 && window <= 1024) || ring_short_band);
    // 16-row waves at head dim 256 (attn_ring16_kernel): one 16-row block
    // per workgroup, no key split.  Twice the workgroups of the 32-row
    // kernel, each streaming its whole band for half the rows, so it wins
    // where the 32-row kernel needs a key split and the band is short (16/8
    // heads, 256 queries, auto plan against 16-row waves, µs: window 256
    // 13.2 / 10.7, 512 15.0 / 12.9, 1024 17.4 / 16.5, 1536 20.2 / 20.6, 2048
    // 22.7 / 24.1; no window, 512 keys 12.7 / 10.0, 1280 16.8 / 16.5, 2304
    // 22.2 / 23.6).  Picked for bands up to RING16_MAX_TILES tiles when its
    // workgroups fill more than half the CUs in one round.
    const int r16_blocks = n_batch * n_head_kv * ((group * max_nq + 15) / 16);
    const bool r16_forced = force_kernel == KERNEL_STREAMS && force_rows == 16;
    // (the planner's choice within the stream family too: bf16 Q or output
    // rows ask for that family)
    const bool r16_auto = (force_kernel == KERNEL_AUTO || force_kernel == KERNEL_STREAMS) && force_rows <= 0 &&
                          force_split <= 0 &&
                          band_tiles <= RING16_MAX_TILES && 2 * r16_blocks > cus && r16_blocks <= cus;
    if (ring_ok && hd == 256 && (r16_forced || r16_auto) && force_rb <= 0 && force_kq <= 0) {
        p.kernel = KERNEL_STREAMS;
        p.w16 = true;
        p.rb = 1;
        p.stages = 1;
        p.qepi = false;
        p.rowgroups = (group * max_nq + 15) / 16;
        if (p.rowgroups < 1) p.rowgroups = 1;
        p.n_split = 1;
        p.n_workgroups = n_batch * n_head_kv * p.rowgroups;
        p.waves = 4;
        p.kq = 4;
        p.rotate = false;
        return p;
    }
    if (ring_ok && (force_kernel == KERNEL_STREAMS || (force_kernel == KERNEL_AUTO && ring_auto)) &&
        force_rb <= 0 && force_kq <= 0 && force_rows <= 0) {
        p.kernel = KERNEL_STREAMS;
        p.rb = 1;
        p.w16 = false;
        p.stages = 1;
        p.qepi = false;  // the Q bias, norm and RoPE are runtime operands of the kernel
        p.rowgroups = row_blocks < 1 ? 1 : row_blocks;
        const int base = n_batch * n_head_kv * p.rowgroups;
        int split = 1;
        if (force_split > 0) {
            split = force_split;
        } else if (hd == 256 && merge_in_kernel && 2 * base <= cus && ntiles >= 2 * rw) {
            // A half-filled chip at head dim 256: two key splits merged
            // in-kernel (DiffusionGemma's sliding layers: 18.1 against 21.8 us
            // unsplit; with the separate merge kernel the split lost, 22.9).
            split = 2;
        } else if ((hd == 128 ? 2 : 4) * base <= cus) {
            // too few workgroups for the CUs: split the keys, keeping a tile
            // for each of a split's waves
            split = cus / base;
            const int max_split = ntiles / rw > 1 ? ntiles / rw : 1;
            if (split > max_split) split = max_split;
        }
        if (split < 1) split = 1;
        p.n_split = split;
        p.n_workgroups = base * split;
        // (a split only shortens a workgroup's stream: never more waves than rw,
        // so the split's cap of a tile per wave still holds)
        p.waves = ring_waves(hd, (band_tiles + split - 1) / split);
        p.kq = p.waves;
        // rotated tile walks while the K/V that one XCD's workgroups read fits
        // its L2 (4 MB, part of it left to Q, O and partials): the kv heads an
        // XCD holds (consecutive workgroups: a head's row groups and splits)
        // times a head's keys (its band) times 4 * head dim bytes
        const int per_head = p.rowgroups * split;
        const int per_xcd = (p.n_workgroups + 7) / 8;
        const long long heads = per_xcd <= per_head ? 1 : (per_xcd + per_head - 1) / per_head;
        p.rotate = heads * (long long)(band < max_nk ? band : max_nk) * hd * 4 <= (3LL << 20);
        return p;
    }
    // Head dims up to 128: one row block of four key groups with four DMA
    // waves (two waves per SIMD).  256: two row blocks of two key groups,
    // one 32-row wave per SIMD (the accumulators need the whole register
    // file), or the 16-row form (below).
    // 512: two row blocks, each a wave pair that splits the head dim.
    int rb = 1;
    int kq = p.hd_tile == 256 ? 2 : (p.hd_tile == 512 ? 1 : 4);
    if ((p.hd_tile == 256 && row_blocks >= 2) || p.hd_tile == 512) rb = 2;
    // Head dim 128 without a mask: two 16-row compute waves per key group
    // (two compute waves per SIMD; 1-3 % faster on C2-C4, whose loop is bound
    // by the K/V stream).  The masked builds of that shape spill, so masked
    // launches keep 32-row waves unless asked.
    // Head dim 256 (two row blocks, two key groups): 16-row waves under every
    // mask (200-222 VGPRs, so two compute waves per SIMD, which issue their
    // own DMA): C5's sliding and global layers take 29.0 and 36.3 us against
    // 33.7 and 41.4 with one 32-row wave per SIMD.
    // Head dim 512: 16-row waves that also split the head dim (8 compute
    // waves, 204-232 VGPRs): the G512 global layer takes 74.3 us against 93.2.
    bool w16 = (p.hd_tile == 128 && mask == MASK_NONE) || (p.hd_tile == 256 && rb == 2 && kq == 2) ||
               p.hd_tile == 512;
    // Head dims up to 128 with more one-row-block workgroups than CUs (C3's
    // 448 on 256): two row blocks of 32-row waves and four key groups, with
    // the compute waves issuing the DMA (RB 2, KQ 4, NP 0).  That fills the
    // chip in one round instead of leaving a partial second one, and each
    // K/V tile serves 64 query rows (C3: 18.8 against 23.6 us).
    if (p.hd_tile <= 128 && n_batch * n_head_kv * row_blocks > cus && row_blocks >= 2) {
        rb = 2;
        kq = 4;
        w16 = false;
    }
    if (force_rb > 0) rb = force_rb;
    if (force_kq > 0) kq = force_kq;
    if (force_rows == 16) w16 = true;
    if (force_rows == 32) w16 = false;
    const Shape* sh = find_shape(p.hd_tile, rb, kq, w16);
    if (!sh) {
        rb = (p.hd_tile == 256 && row_blocks >= 2) || p.hd_tile == 512 ? 2 : 1;
        kq = p.hd_tile == 256 ? 2 : (p.hd_tile == 512 ? 1 : 4);
        w16 = false;
        sh = find_shape(p.hd_tile, rb, kq, w16);
    }
    p.rb = rb;
    p.kq = kq;
    p.w16 = w16;
    p.waves = rb * kq * (w16 ? 2 : 1) * (p.hd_tile == 512 ? 2 : 1) + sh->np;
    p.stages = sh->ns;
    p.rowgroups = (row_blocks + rb - 1) / rb;
    if (p.rowgroups < 1) p.rowgroups = 1;
    const int base = n_batch * n_head_kv * p.rowgroups;
    int split = 1;
    if (force_split > 0) {
        split = force_split;
    } else if (2 * base <= cus) {
        // Too few workgroups to fill the chip (one workgroup per CU): split
        // the keys, keeping at least one super-tile per split.
        split = cus / base;
        const int max_split = ntiles / kq > 1 ? ntiles / kq : 1;
        if (split > max_split) split = max_split;
    }
    if (split < 1) split = 1;
    p.n_split = split;
    p.n_workgroups = base * split;
    return p;
}

size_t split_workspace_bytes(const LaunchPlan& p, int n_batch, int n_head_kv) {
    if (p.n_split <= 1) return 0;
    const size_t rows = (size_t)n_batch * n_head_kv * p.rowgroups * p.rb * 32;
    return (size_t)p.n_split * rows * ((size_t)p.hd_tile + 2) * sizeof(float);
}

// ceil(2^32 / d) when n * d < 2^32 for every n < n_max, else 0.
static uint32_t div_magic(int d, int n_max) {
    if (d < 2 || (uint64_t)n_max * (uint64_t)d >= ((uint64_t)1 << 32)) return 0;
    return (uint32_t)((((uint64_t)1 << 32) + (uint64_t)d - 1) / (uint64_t)d);
}

hipError_t launch_attention(const LaunchPlan& p, AttnArgs& a, hipStream_t st) {
    a.n_wg = p.n_workgroups;
    a.rowgroups = p.rowgroups;
    a.n_split = p.n_split;
    if (p.n_split > 1) {
        const size_t rows = (size_t)a.n_batch * a.n_head_kv * p.rowgroups * p.rb * 32;
        a.part_ml = a.part_o + (size_t)p.n_split * rows * p.hd_tile;
    }
    a.mg_split = div_magic(a.n_split, p.n_workgroups);
    a.mg_rowgroups = div_magic(a.rowgroups, p.n_workgroups);
    a.mg_hkv = div_magic(a.n_head_kv, p.n_workgroups);
    a.part_rows = p.rowgroups * p.rb * 32;
    a.ring_rot = p.rotate ? 1 : 0;
    if (p.kernel != KERNEL_STREAMS) a.ticket = nullptr;  // (the others always merge in a second kernel)
    hipError_t e = p.kernel == KERNEL_STREAMS ? launch_ring(p, a, st)
                   : p.kernel == KERNEL_HILO  ? launch_hilo(p, a, st)
                                              : launch_shape(p, a, st);
    if (e != hipSuccess || p.n_split <= 1 || a.ticket) return e;
    const size_t items = (size_t)a.n_batch * a.n_head_kv * a.part_rows * (p.hd_tile / 4);
    const dim3 grid((unsigned)((items + 255) / 256));
    switch (p.hd_tile) {
        case 64: hipLaunchKernelGGL(split_merge_kernel<64>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(split_merge_kernel<128>, grid, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(split_merge_kernel<256>, grid, dim3(256), 0, st, a); break;
        case 512: hipLaunchKernelGGL(split_merge_kernel<512>, grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dr
