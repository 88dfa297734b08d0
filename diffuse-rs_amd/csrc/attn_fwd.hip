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
// owns RB row blocks and a range of key tiles, and runs RB x KQ waves: wave
// (rb, kq) computes row block rb against every KQ-th tile of the range.  The
// KQ tiles of a "super-tile" sit side by side in LDS, each shared by the RB
// waves of its key group; at the end the KQ partial softmax states of a row
// block are merged through LDS, which also stages the output so that it is
// written with full-row, coalesced stores.  Optionally the key range is also
// split across workgroups (n_split > 1), merged by attn_combine_kernel.
//
// Per wave and 32-key block:
//   S^T[key][q] = K Q^T    via v_mfma_f32_32x32x16_bf16, A = K (LDS),
//                          B = the wave's Q^T fragments (registers)
//   O^T[d][q]  += V^T P^T  via the same MFMA, A = V^T (LDS),
//                          B = P^T straight from the S^T accumulators.
// Computing the transposed products makes each lane own one query column, so
// the softmax row statistics are per lane (plus one exchange with lane^32),
// and P never leaves registers.  K rows are placed in LDS in a permuted order
// (sigma below) chosen so that lane half `hf` ends up holding keys
// 16*hf .. 16*hf+15 of every 32-key block, which is exactly the contiguous
// 8-key run each half must supply as the B operand of the PV product.
//
// The softmax works in the log2 domain: Q is multiplied by scale*log2(e)
// before rounding to bf16, p = exp2(s - m).  The running max is only moved
// when it grows by more than 8 (p <= 256 is exact enough in bf16/f32), which
// skips the O rescale on almost every tile; O / l does not depend on the
// choice of m.  l sums the bf16-rounded p that the PV product uses, so the
// weights normalise exactly.  A row with no visible key ends with l = 0 and
// writes 0 * (1/0) = NaN, like the reference (attention.rs:181-185).
//
// Memory: K is [kv head][key][HD] and V is stored transposed [kv head][d][key]
// (the KV-cache layout written by kv_cache.hip).  Tiles move HBM -> LDS with
// gfx950's global_load_lds_dwordx4 (16 bytes per lane, no VGPR staging),
// NS super-tiles deep.  Each lane picks the global chunk that belongs at its
// LDS slot, so the linear DMA writes produce the permuted, XOR-swizzled tile
// image that keeps the MFMA operand reads (16 B per lane) free of bank
// conflicts.
#include "dr_internal.hpp"

#include <limits.h>
#include <math.h>

namespace dr {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float RESCALE_THRESHOLD = 8.0f;  // log2 units

// 16-byte-chunk swizzle for an LDS row holding CH chunks.  Keeps 8 (32-bank
// LDS) or 16 (64-bank LDS) consecutive rows read at the same logical chunk on
// distinct banks.
template <int CH>
__device__ __forceinline__ int swz(int row) {
    if constexpr (CH >= 16) {
        return row & 15;
    } else if constexpr (CH == 8) {
        return (row & 7) ^ ((row >> 3) & 1);
    } else {
        static_assert(CH == 4, "unsupported row width");
        return ((row >> 1) ^ (row >> 3)) & 3;
    }
}

// Key offset (within a 32-key block) stored in LDS row R of the block.  The
// MFMA puts A-row R in accumulator slot i of lane half hf with
// R = 8*(i/4) + 4*hf + (i%4); sigma(R) = 16*hf + i places key 16*hf + i there.
__device__ __forceinline__ int sigma(int R) {
    return 16 * ((R >> 2) & 1) + 4 * (R >> 3) + (R & 3);
}

// visible() of attention.rs:36-57, evaluated without branches (bitwise
// and/or of the three rules) so the per-element mask is a straight-line
// compare + select; a short-circuit version compiled into divergent control
// flow that lost masked elements.
__device__ __forceinline__ bool visible(int qpos, int kpos, int qseq, int kseq, int window,
                                        int prefix) {
    const bool same_seq = qseq == kseq;
    const bool in_band = (window < 0) | (abs(qpos - kpos) < window);
    const bool causal_ok = (prefix < 0) | (qpos >= prefix) | (kpos <= qpos);
    return same_seq & in_band & causal_ok;
}

// 16 bytes per lane global -> LDS (global_load_lds_dwordx4): lane i of the
// wave writes lds_base + 16*i.  Kept in a __device__ helper: used directly in
// a kernel body, the builtin makes the host compilation pass drop the
// kernel's launch stub.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
    __builtin_amdgcn_global_load_lds(
        (const __attribute__((address_space(1))) void*)src,
        (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most `pending` super-tiles (each NI vector-memory
// instructions) issued after the current one are still in flight.
template <int NI, int NS>
__device__ __forceinline__ void wait_tiles(int pending) {
    if constexpr (NS >= 3) {
        if (pending >= 1) {
            wait_vmcnt<NI>();
            return;
        }
    }
    wait_vmcnt<0>();
}

template <int HD, int BN, int RB, int KQ, int NS>
struct Geometry {
    static constexpr int NW = RB * KQ;         // waves per workgroup
    static constexpr int NT = NW * 64;
    static constexpr int NB = BN / 32;         // 32-key blocks per tile
    static constexpr int NC = HD / 16;         // QK^T contraction steps
    static constexpr int ND = HD / 32;         // 32-row blocks of O^T
    static constexpr int KCH = HD / 8;         // 16-byte chunks per K row
    static constexpr int VCH = BN / 8;         // 16-byte chunks per V^T row
    static constexpr int TILE = BN * HD;       // bf16 elements per K (or V^T) tile
    static constexpr int SLOT = 2 * TILE;      // K tile then V^T tile
    static constexpr int STAGE = KQ * SLOT;    // one super-tile
    static constexpr int CPT = TILE / 8;       // 16-byte chunks per tile
    static constexpr int NLDW = STAGE / 8 / NT;  // DMA instructions per wave per super-tile
    static constexpr int ROWF = HD + 4;        // f32 row pitch of the merge area
    static constexpr size_t STAGE_BYTES = (size_t)NS * STAGE * 2;
    static constexpr size_t MERGE_BYTES = ((size_t)NW * 32 * ROWF + 2 * NW * 32) * 4;
    static constexpr size_t LDS_BYTES = STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES;
    static_assert(CPT % 64 == 0, "a DMA instruction must stay inside one tile");
    static_assert(STAGE / 8 % NT == 0, "super-tile must split evenly over the waves");
    static_assert(NLDW < 64, "vmcnt range");
};

template <int HD, int BN, int RB, int KQ, int NS, int MODE, bool QNORM>
__attribute__((amdgpu_waves_per_eu((RB * KQ + 3) / 4, (RB * KQ + 3) / 4))) __global__
__launch_bounds__(RB * KQ * 64) void attn_fwd_kernel(const AttnArgs a) {
    using G = Geometry<HD, BN, RB, KQ, NS>;
    constexpr int NW = G::NW, NT = G::NT, NB = G::NB, NC = G::NC, ND = G::ND;
    constexpr int KCH = G::KCH, VCH = G::VCH, TILE = G::TILE, SLOT = G::SLOT, STAGE = G::STAGE;
    constexpr int CPT = G::CPT, NLDW = G::NLDW, ROWF = G::ROWF;

    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_red[3][NW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, hf = lane >> 5;
    const int rb = wave % RB, kq = wave / RB;

    // Workgroup -> (batch, kv head, row group, split).  The hardware deals
    // workgroups round-robin over the 8 XCDs; remapping keeps consecutive
    // logical ids (same KV head, neighbouring splits) on one XCD's L2.
    const int nwg = gridDim.x;
    const int hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int split = lid % a.n_split;
    int rest = lid / a.n_split;
    const int rg = rest % a.rowgroups;
    rest /= a.rowgroups;
    const int g = rest % a.n_head_kv;
    const int b = rest / a.n_head_kv;
    const AttnSlot& S = a.slot[b];

    const int rows_total = a.group * S.nq;
    const int wg_row0 = rg * RB * 32;
    if (wg_row0 >= rows_total) return;  // uniform over the workgroup and all splits
    const int r = wg_row0 + rb * 32 + col;
    const bool rvalid = r < rows_total;
    const int hg = rvalid ? r / S.nq : 0;
    const int qi = rvalid ? r - hg * S.nq : 0;
    const int head = g * a.group + hg;

    // ---- Q loads first (their latency overlaps the key-range work and DMA)
    float x[NC][8];
    {
        const float* qrow =
            static_cast<const float*>(S.q) + (size_t)qi * a.q_rstride + (size_t)head * a.hd;
        if (rvalid && a.hd == HD) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const f32x4* p = reinterpret_cast<const f32x4*>(qrow + 16 * c + 8 * hf);
                const f32x4 u = p[0], w = p[1];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[c][j] = u[j];
                    x[c][4 + j] = w[j];
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = 16 * c + 8 * hf + j;
                    x[c][j] = (rvalid && d < a.hd) ? qrow[d] : 0.0f;
                }
        }
    }

    // ---- masking state and the key tile range of this workgroup
    int kt_lo = 0, kt_hi = (S.nk + BN - 1) / BN;
    int my_qpos = 0, my_qseq = 0, my_pref = -1;
    int qmin = 0, qmax = 0;
    bool tiles_can_be_full = MODE == MASK_NONE;
    if constexpr (MODE != MASK_NONE) {
        my_qpos = rvalid ? S.qpos[qi] : 0;
        my_qseq = (rvalid && S.qseq) ? S.qseq[qi] : 0;
        my_pref = S.qprefix ? (rvalid ? S.qprefix[qi] : -1) : a.prefix;
    }
    if constexpr (MODE == MASK_POS) {
        bool prefix_free;
        if (S.qpos_sorted && S.qprefix == nullptr) {
            // ascending positions: the extremes sit at the ends of the
            // workgroup's query range (the whole range if it spans heads)
            const int r1 = min(wg_row0 + RB * 32, rows_total) - 1;
            const int h0 = wg_row0 / S.nq, h1 = r1 / S.nq;
            const int lo = h0 == h1 ? wg_row0 - h0 * S.nq : 0;
            const int hi = h0 == h1 ? r1 - h0 * S.nq : S.nq - 1;
            qmin = S.qpos[lo];
            qmax = S.qpos[hi];
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
            for (int w = 0; w < NW; ++w) {
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

    // ---- DMA plan of this lane: instruction j fills 64 chunks of one tile
    // slot; slot and K/V side are uniform per instruction.
    int doff[NLDW], dslot[NLDW];
    bool disv[NLDW];
#pragma unroll
    for (int j = 0; j < NLDW; ++j) {
        const int c0 = (wave * NLDW + j) * 64;  // first stage chunk of the instruction
        const int region = c0 / CPT;
        dslot[j] = region >> 1;
        disv[j] = region & 1;
        const int idx = c0 % CPT + lane;  // chunk within the tile
        if (!disv[j]) {
            const int R = idx / KCH, pk = idx % KCH;
            doff[j] = ((R & ~31) + sigma(R & 31)) * HD + ((pk ^ swz<KCH>(R)) << 3);
        } else {
            const int d = idx / VCH, pv = idx % VCH;
            doff[j] = d * a.cap + ((pv ^ swz<VCH>(d)) << 3);
        }
    }
    const uint16_t* kbase = S.k + (size_t)g * a.cap * HD;
    const uint16_t* vbase = S.vt + (size_t)g * HD * a.cap;

    auto issue = [&](int u, int st) {
        uint16_t* stage = smem + st * STAGE + wave * NLDW * 512;
#pragma unroll
        for (int j = 0; j < NLDW; ++j) {
            // slots past the range reload the last tile: in bounds, unused
            const int t = min(t0 + u * KQ + dslot[j], t1 - 1);
            const uint16_t* src = disv[j] ? vbase + (size_t)t * BN : kbase + (size_t)t * BN * HD;
            dma16(src + doff[j], stage + j * 512);
        }
    };

#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < nsup) issue(i, i);

    // ---- Q fragments (B operand of S^T = K Q^T), scale*log2e folded in
    bf16x8 qf[NC];
    {
        if constexpr (QNORM) {
            // rms_norm_inplace (ops.rs:106-114): f32 squares summed in f64.
            double ss = 0.0;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float sq = x[c][j] * x[c][j];
                    ss += (double)sq;
                }
            ss += __shfl_xor(ss, 32);
            const float sc = 1.0f / (float)sqrt(ss / (double)a.hd + (double)a.qn_eps);
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = 16 * c + 8 * hf + j;
                    if (d < a.hd) x[c][j] = x[c][j] * sc * a.qn_w[d];
                }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j) qf[c][j] = (__bf16)(x[c][j] * a.c);
    }

    // ---- main loop over super-tiles
    f32x16 o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    for (int u = 0; u < nsup; ++u) {
        const int st = u % NS;
        wait_tiles<NLDW, NS>(min(NS - 2, nsup - 1 - u));
        __syncthreads();  // super-tile u visible to all waves; u-1 fully consumed
        if (u + NS - 1 < nsup) issue(u + NS - 1, (u + NS - 1) % NS);

        const int t = t0 + u * KQ + kq;
        if (t >= t1) continue;  // this key group has no tile in the last super-tile
        const uint16_t* ks = smem + st * STAGE + kq * SLOT;
        const uint16_t* vs = ks + TILE;
        const int kbase_t = t * BN;

        // per-key metadata (arbitrary key positions / ids): loaded per tile
        int kp[NB][16], kqs[NB][16];
        if constexpr (MODE == MASK_KEYS) {
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kidx = min(kbase_t + kb * 32 + 16 * hf + i, S.nk - 1);
                    kp[kb][i] = S.kpos ? S.kpos[kidx] : kidx;
                    kqs[kb][i] = S.kseq ? S.kseq[kidx] : 0;
                }
        }

        // S^T = K Q^T.  All K fragments of a 32-key block are read before its
        // MFMAs so the LDS latency is paid once per block, not per MFMA.
        f32x16 sacc[NB];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            const int R = kb * 32 + col;
            const uint16_t* krow = ks + R * HD;
            const int sw = swz<KCH>(R);
            bf16x8 kf[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c)
                kf[c] = *reinterpret_cast<const bf16x8*>(krow + (((2 * c + hf) ^ sw) << 3));
            sacc[kb] = f32x16{};
#pragma unroll
            for (int c = 0; c < NC; ++c)
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[c], qf[c], sacc[kb], 0, 0, 0);
        }

        // Masking: sacc[kb][i] is the score of key t*BN + kb*32 + 16*hf + i.
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
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kidx = kbase_t + kb * 32 + 16 * hf + i;
                    bool vis = kidx < S.nk;
                    if constexpr (MODE == MASK_POS) {
                        vis = vis & visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
                    } else if constexpr (MODE == MASK_KEYS) {
                        vis = vis & visible(my_qpos, kp[kb][i], my_qseq, kqs[kb][i], a.window,
                                            my_pref);
                    }
                    sacc[kb][i] = vis ? sacc[kb][i] : -INFINITY;
                }
        }

        // Online softmax with a lazily moved max.
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[kb][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const bool need = (m_new - m_run) > RESCALE_THRESHOLD;
        if (__builtin_amdgcn_ballot_w64(need)) {
            if (need) {
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < ND; ++db) o[db] *= alpha;
                m_run = m_new;
            }
        }
        const float mu = (m_run == -INFINITY) ? 0.0f : m_run;
        // p = exp2(s - m) rounded to bf16 in pairs; l sums the rounded values
        // (what the PV product multiplies), so the weights normalise exactly.
        bf16x8 pf[NB][2];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                u32x4 w4;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p0 = __builtin_amdgcn_exp2f(sacc[kb][8 * hh + 2 * j] - mu);
                    const float p1 = __builtin_amdgcn_exp2f(sacc[kb][8 * hh + 2 * j + 1] - mu);
                    const bf16x2 pr = {(__bf16)p0, (__bf16)p1};
                    w4[j] = __builtin_bit_cast(uint32_t, pr);
                    l_run += __uint_as_float(w4[j] << 16) + __uint_as_float(w4[j] & 0xffff0000u);
                }
                pf[kb][hh] = __builtin_bit_cast(bf16x8, w4);
            }

        // O^T += V^T P^T.  Contraction slot 8*hf + j of MFMA (kb, hh) is key
        // kb*32 + 16*hf + 8*hh + j, in both operands.
#pragma unroll
        for (int db = 0; db < ND; ++db) {
            const int d = db * 32 + col;
            const uint16_t* vrow = vs + d * BN;
            const int sw = swz<VCH>(d);
            bf16x8 vf[NB][2];
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
                    vf[kb][hh] = *reinterpret_cast<const bf16x8*>(
                        vrow + (((4 * kb + 2 * hf + hh) ^ sw) << 3));
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[kb][hh], pf[kb][hh], o[db],
                                                                    0, 0, 0);
        }
    }

    // ---- merge the KQ key groups of each row block through LDS and write
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    __syncthreads();  // every wave is done with the tile stages
    float* mrows = reinterpret_cast<float*>(smem);  // [NW][32][ROWF]
    float* sm = mrows + NW * 32 * ROWF;             // [NW][32] running max
    float* sl = sm + NW * 32;                       // [NW][32] scaled sum
    if (hf == 0) sm[wave * 32 + col] = m_run;
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < KQ; ++k) M = fmaxf(M, sm[(k * RB + rb) * 32 + col]);
    const float sc = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - M);
    {
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
    __syncthreads();

    constexpr int CHUNKS = HD / 4;
    const size_t rows_pad = (size_t)a.rowgroups * RB * 32;
    const size_t bg = (size_t)b * a.n_head_kv + g;
    for (int item = tid; item < RB * 32 * CHUNKS; item += NT) {
        const int rr = item / CHUNKS, ch = item % CHUNKS;
        const int rbi = rr >> 5, ci = rr & 31;
        const int rglob = wg_row0 + rr;
        if (rglob >= rows_total) continue;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f, Mrow = -INFINITY;
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
            const int wi = k * RB + rbi;
            acc += *reinterpret_cast<const f32x4*>(mrows + (wi * 32 + ci) * ROWF + ch * 4);
            L += sl[wi * 32 + ci];
            Mrow = fmaxf(Mrow, sm[wi * 32 + ci]);
        }
        const int d0 = ch * 4;
        if (a.n_split == 1) {
            const int hgi = rglob / S.nq, qii = rglob - hgi * S.nq;
            float* orow = S.out + (size_t)qii * a.o_rstride + (size_t)(g * a.group + hgi) * a.hd;
            const f32x4 val = acc * (1.0f / L);
            if (a.hd == HD) {
                *reinterpret_cast<f32x4*>(orow + d0) = val;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d0 + e < a.hd) orow[d0 + e] = val[e];
            }
        } else {
            const size_t prow =
                ((size_t)split * a.n_batch * a.n_head_kv + bg) * rows_pad + rglob;
            *reinterpret_cast<f32x4*>(a.part_o + prow * HD + d0) = acc;
            if (ch == 0) {
                a.part_ml[prow * 2] = Mrow;
                a.part_ml[prow * 2 + 1] = L;
            }
        }
    }
}

// Merges the key-split partials: M = max m_s, L = sum l_s 2^(m_s - M),
// O = sum O_s 2^(m_s - M) / L.  One thread per 4 consecutive output values;
// the workgroups of a row group run on the XCD whose L2 holds its partials.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const CombineArgs a, int rows_per_rg) {
    constexpr int CH = HD / 4;
    const int nwg = gridDim.x;
    const int hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int c_in_rg = lid % a.wg_per_rowgroup;
    const int rgi = lid / a.wg_per_rowgroup;  // (batch, kv head, row group)
    const int rg = rgi % a.rowgroups;
    const int bg = rgi / a.rowgroups;
    const int b = bg / a.n_head_kv, g = bg % a.n_head_kv;
    const int item = c_in_rg * 256 + threadIdx.x;
    if (item >= rows_per_rg * CH) return;
    const int r = rg * rows_per_rg + item / CH;
    const int chunk = item % CH;
    const AttnSlot& S = a.slot[b];
    if (r >= a.group * S.nq) return;
    const int hg = r / S.nq, qi = r - hg * S.nq;
    const int head = g * a.group + hg;

    const size_t plane = (size_t)a.n_batch * a.n_head_kv * a.rows_pad;  // rows per split
    const size_t prow = (size_t)bg * a.rows_pad + r;
    float M = -INFINITY;
    for (int s = 0; s < a.n_split; ++s) M = fmaxf(M, a.part_ml[(s * plane + prow) * 2]);
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    float L = 0.0f;
    for (int s = 0; s < a.n_split; ++s) {
        const float ms = a.part_ml[(s * plane + prow) * 2];
        const float w = (ms == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
        L += w * a.part_ml[(s * plane + prow) * 2 + 1];
        const f32x4 v = *reinterpret_cast<const f32x4*>(a.part_o + (s * plane + prow) * HD +
                                                        chunk * 4);
        o += w * v;
    }
    const float inv = 1.0f / L;
    float* orow = S.out + (size_t)qi * a.o_rstride + (size_t)head * a.hd;
    const int d0 = chunk * 4;
    if (a.hd == HD) {
        *reinterpret_cast<f32x4*>(orow + d0) = o * inv;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (d0 + e < a.hd) orow[d0 + e] = o[e] * inv;
    }
}

template <int HD, int BN, int RB, int KQ, int NS, int MODE, bool QNORM>
hipError_t launch_fwd(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    constexpr size_t lds = Geometry<HD, BN, RB, KQ, NS>::LDS_BYTES;
    static bool attr_set = false;
    auto fn = attn_fwd_kernel<HD, BN, RB, KQ, NS, MODE, QNORM>;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3(p.n_workgroups), dim3(RB * KQ * 64), lds, st, a);
    return hipGetLastError();
}

template <int HD, int BN, int RB, int KQ, int NS>
hipError_t launch_modes(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    switch (p.mask) {
        case MASK_NONE:
            return p.qnorm ? launch_fwd<HD, BN, RB, KQ, NS, MASK_NONE, true>(p, a, st)
                           : launch_fwd<HD, BN, RB, KQ, NS, MASK_NONE, false>(p, a, st);
        case MASK_POS:
            return p.qnorm ? launch_fwd<HD, BN, RB, KQ, NS, MASK_POS, true>(p, a, st)
                           : launch_fwd<HD, BN, RB, KQ, NS, MASK_POS, false>(p, a, st);
        default:
            return launch_fwd<HD, BN, RB, KQ, NS, MASK_KEYS, false>(p, a, st);
    }
}

// The (RB, KQ) shapes built for each head-dim tile (all with 32-key tiles).
// LDS per workgroup: NS super-tiles of KQ x (K + V^T) tiles.
//   HD  64: (1,4) (2,4)  NS 3     HD 128: (1,4) (2,4) (2,2)  NS 2
//   HD 256: (1,2) (2,2)  NS 2
bool shape_built(int hd_tile, int rb, int kq) {
    switch (hd_tile) {
        case 64: return (rb == 1 || rb == 2) && kq == 4;
        case 128: return (rb == 1 && kq == 4) || (rb == 2 && (kq == 4 || kq == 2));
        case 256: return (rb == 1 || rb == 2) && kq == 2;
        default: return false;
    }
}

hipError_t launch_shape(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    const int key = p.hd_tile * 100 + p.rb * 10 + p.kq;
    switch (key) {
        case 6414: return launch_modes<64, 32, 1, 4, 3>(p, a, st);
        case 6424: return launch_modes<64, 32, 2, 4, 3>(p, a, st);
        case 12814: return launch_modes<128, 32, 1, 4, 2>(p, a, st);
        case 12824: return launch_modes<128, 32, 2, 4, 2>(p, a, st);
        case 12822: return launch_modes<128, 32, 2, 2, 2>(p, a, st);
        case 25612: return launch_modes<256, 32, 1, 2, 2>(p, a, st);
        case 25622: return launch_modes<256, 32, 2, 2, 2>(p, a, st);
        default: return hipErrorInvalidValue;
    }
}

template <int HD>
hipError_t launch_combine(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    CombineArgs c;
    for (int i = 0; i < MAX_BATCH; ++i) c.slot[i] = a.slot[i];
    c.n_batch = a.n_batch;
    c.n_head_kv = a.n_head_kv;
    c.group = a.group;
    c.hd = a.hd;
    c.o_rstride = a.o_rstride;
    c.rows_pad = a.rowgroups * p.rb * 32;
    c.rowgroups = a.rowgroups;
    c.n_split = a.n_split;
    c.part_o = a.part_o;
    c.part_ml = a.part_ml;
    const int rows_per_rg = p.rb * 32;
    c.wg_per_rowgroup = (rows_per_rg * (HD / 4) + 255) / 256;
    const int nwg = a.n_batch * a.n_head_kv * a.rowgroups * c.wg_per_rowgroup;
    hipLaunchKernelGGL(attn_combine_kernel<HD>, dim3(nwg), dim3(256), 0, st, c, rows_per_rg);
    return hipGetLastError();
}

}  // namespace

LaunchPlan plan_attention(int hd, int n_batch, int n_head_kv, int group, int max_nq, int max_nk,
                          int mask, bool qnorm, int n_cu, int force_rb, int force_kq,
                          int force_split) {
    LaunchPlan p;
    p.hd_tile = hd <= 64 ? 64 : (hd <= 128 ? 128 : 256);
    p.block_n = 32;
    p.mask = mask;
    p.qnorm = qnorm && mask != MASK_KEYS;
    const int cus = n_cu > 0 ? n_cu : 256;
    const int row_blocks = (group * max_nq + 31) / 32;  // per (batch, kv head)
    const int ntiles = (max_nk + p.block_n - 1) / p.block_n;
    const int kq_full = p.hd_tile == 256 ? 2 : 4;
    // Prefer two row blocks per workgroup (halves the K/V traffic per row)
    // when that still gives every CU a workgroup; otherwise one.
    int rb = (n_batch * n_head_kv * ((row_blocks + 1) / 2) >= cus) ? 2 : 1;
    int kq = kq_full;
    if (force_rb > 0) rb = force_rb;
    if (force_kq > 0) kq = force_kq;
    if (!shape_built(p.hd_tile, rb, kq)) {
        rb = 1;
        kq = kq_full;
    }
    p.rb = rb;
    p.kq = kq;
    p.waves = rb * kq;
    p.stages = p.hd_tile == 64 ? 3 : 2;
    p.rowgroups = (row_blocks + rb - 1) / rb;
    if (p.rowgroups < 1) p.rowgroups = 1;
    const int base = n_batch * n_head_kv * p.rowgroups;
    int split = 1;
    if (force_split > 0) {
        split = force_split;
    } else if (base < cus / 2) {
        // Too few workgroups to fill the chip: split the keys, keeping at
        // least two super-tiles per split.
        split = (cus + base - 1) / base;
        const int max_split = ntiles / (2 * kq) > 1 ? ntiles / (2 * kq) : 1;
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

hipError_t launch_attention(const LaunchPlan& p, AttnArgs& a, hipStream_t st) {
    a.rowgroups = p.rowgroups;
    a.n_split = p.n_split;
    if (p.n_split > 1) {
        const size_t rows = (size_t)a.n_batch * a.n_head_kv * p.rowgroups * p.rb * 32;
        a.part_ml = a.part_o + (size_t)p.n_split * rows * p.hd_tile;
    }
    hipError_t e = launch_shape(p, a, st);
    if (e != hipSuccess || p.n_split == 1) return e;
    switch (p.hd_tile) {
        case 64: return launch_combine<64>(p, a, st);
        case 128: return launch_combine<128>(p, a, st);
        default: return launch_combine<256>(p, a, st);
    }
}

}  // namespace dr
