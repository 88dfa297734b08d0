// attn_hilo.hip -- the denoise-step attention of attention.rs:101-186 with
// f32-accurate scores, for layers whose score scale is large enough that bf16
// operands are not (Gemma runs every layer at kq_scale 1.0 after QK-norm,
// src/model/forward.rs:338-341: at head dim 256 the scores have a standard
// deviation of ~16, the softmax is nearly one-hot, and the 2^-9 rounding of
// bf16 Q and K moves the outputs by ~0.15).
//
// Scores.  Q (times scale * log2 e, in f32) and K are each split into bf16
// halves, x = hi + lo with hi = bf16(x) and lo = bf16(x - hi), and
//   S = Qh.Kh + Qh.Kl + Ql.Kh
// on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, f32 accumulation); the
// dropped Ql.Kl and the rounding of lo leave a relative error of ~2^-16 per
// product.  Values: O += P.Vh + P.Vl, V to ~2^-17.  At such a scale the
// softmax is nearly one-hot, so an output is essentially one V row and bf16
// V alone would move it by up to 2^-9 of that row.  P stays bf16: the
// dominant key's p is exactly 1 and l sums the same rounded p.  The cache
// holds the lo halves of K and V^T in planes of their own, written by the
// store next to the hi halves (dr_cache_set_precision).  The drop-in
// dr_attention() runs every call here on its f32 inputs, with the per-key
// positions and sequence ids of its arbitrary key order (MASK_KEYS).
//
// Work decomposition.  A workgroup owns 64 query rows of one (batch slot, kv
// head) -- four 16-row blocks, GQA heads packed into rows as in attn_fwd.hip --
// and a range of 32-key tiles (a key split when the chip would otherwise be
// under-filled; split_merge_kernel combines the splits).  Every wave takes
// every tile of the range for its rows: K hi, K lo, V^T hi and V^T lo of a
// tile sit in LDS once for all of them.  At head dim 512 two waves share a row block,
// each holding Q and O for half the head dims; their partial scores meet in
// LDS.  Per tile: the next tile's K halves stream in while this tile's
// softmax and P.V run, its V^T halves while the next QK^T runs.
//
// Per wave and tile, S^T = K Q^T (A = K rows from LDS, B = Q^T from
// registers): K rows sit in LDS in the order kappa of attn_common.hpp, so the
// lane that holds query q and slot group g ends up with the scores of keys
// 8 g .. 8 g + 7, exactly the B operand of O^T += V^T P^T.  Online softmax in
// the log2 domain with the lazily moved maximum of the other kernels; l sums
// the bf16-rounded p that the P.V product multiplies.
#include "attn_common.hpp"

#include <limits.h>
#include <math.h>

namespace dr {
namespace {

template <int HD>
struct HiloGeom {
    static constexpr int DSPLIT = HD > 256 ? 2 : 1;  // waves per 16-row block
    static constexpr int HDW = HD / DSPLIT;          // head dims per wave
    static constexpr int RBW = 4;                    // 16-row blocks per workgroup
    static constexpr int NW = RBW * DSPLIT;
    static constexpr int NT = NW * 64;
    static constexpr int QROWS = RBW * 16;
    static constexpr int KCH = HD / 8;               // 16-byte chunks per K row
    static constexpr int TILE = BN * HD;             // bf16 elements of a K, K lo or V^T tile
    static constexpr int CPT = TILE / 8;             // 16-byte chunks per tile
    static constexpr int NST = HDW / 32;             // QK^T contraction steps per wave
    static constexpr int NDB = HDW / 16;             // 16-row blocks of a wave's O^T
    static constexpr int KDMA = 2 * CPT / 64 / NW;   // K hi + K lo DMA instructions per wave
    static constexpr int VDMA = 2 * CPT / 64 / NW;   // V^T hi + lo DMA instructions per wave
    static constexpr size_t XCH_BYTES = DSPLIT > 1 ? (size_t)NW * 8 * 64 * 4 : 0;
    static constexpr size_t LDS_BYTES = (size_t)4 * TILE * 2 + XCH_BYTES;
    static_assert(CPT % (64 * NW) == 0, "a tile must split evenly over the waves' DMA");
    static_assert(KDMA + VDMA < 64, "vmcnt range");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

template <int HD, int MODE>
__global__ __launch_bounds__(HiloGeom<HD>::NT) void attn_hilo_kernel(const AttnArgs a) {
    using G = HiloGeom<HD>;
    constexpr int NW = G::NW, RBW = G::RBW, HDW = G::HDW, KCH = G::KCH, TILE = G::TILE;
    constexpr int CPT = G::CPT, NST = G::NST, NDB = G::NDB, KDMA = G::KDMA, VDMA = G::VDMA;
    constexpr int QROWS = G::QROWS;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_red[3][NW];
    uint16_t* const lk = smem;              // K hi tile (rows in kappa order, chunks swizzled)
    uint16_t* const lkl = smem + TILE;      // K lo tile (same layout)
    uint16_t* const lv = smem + 2 * TILE;   // V^T tile [HD][32] (chunks swizzled by swz_v16)
    uint16_t* const lvl = smem + 3 * TILE;  // V^T lo tile (same layout)
    float* const xch = reinterpret_cast<float*>(smem + 4 * TILE);  // [NW][8][64] partial scores

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rbw = wave % RBW, dh = wave / RBW;  // row block, head-dim half
    const int qc = lane & 15, gq = lane >> 4;     // query column, slot group

    // ---- workgroup -> (batch, kv head, split, row group), XCD-grouped as in
    // attn_fwd.hip but with the row group fastest: an XCD then holds every
    // row group of a few (head, split) key ranges, so each key range's hi and
    // lo planes are fetched into one L2 instead of four. At hd 512 (16/2
    // heads, 4 splits, 4352 keys) that cuts the kernel's fetches from 151 to
    // 69 MB per call at the same time within 1 %. attn_fwd.hip keeps the
    // split fastest, measured 3 % faster there.
    const int nwg = a.n_wg, hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int q1 = udiv(lid, a.rowgroups, a.mg_rowgroups);
    const int rg = lid - q1 * a.rowgroups;
    const int q2 = udiv(q1, a.n_split, a.mg_split);
    const int split = q1 - q2 * a.n_split;
    const int b = udiv(q2, a.n_head_kv, a.mg_hkv);
    const int g = q2 - b * a.n_head_kv;
    const AttnSlot S = a.slot[b];
    const int rows_total = a.group * S.nq;
    const int wg_row0 = rg * QROWS;
    if (wg_row0 >= rows_total) return;  // uniform over the workgroup and all its splits
    const int r = wg_row0 + rbw * 16 + qc;
    const bool rvalid = r < rows_total;
    int hg = 0, qi = 0;
    if (rvalid) row_split(r, S.nq, __builtin_amdgcn_rcpf((float)S.nq), a.group, hg, qi);

    // ---- masking state and the key tile range (attn_fwd.hip's rules)
    int kt_lo = 0, kt_hi = (S.nk + BN - 1) / BN;
    int my_qpos = 0, my_qseq = 0, my_pref = -1;
    if constexpr (MODE != MASK_NONE) {
        my_qpos = rvalid ? (S.qpos0 >= 0 ? S.qpos0 + qi : gload<int>(S.qpos + qi)) : 0;  // (contiguous: no load)
        my_qseq = (rvalid && S.qseq) ? gload<int>(S.qseq + qi) : 0;
        my_pref = S.qprefix ? (rvalid ? gload<int>(S.qprefix + qi) : -1) : a.prefix;
    }
    if constexpr (MODE == MASK_POS) {
        if (a.window >= 0) {
            int vmin = rvalid ? my_qpos : INT_MAX, vmax = rvalid ? my_qpos : INT_MIN;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                vmin = min(vmin, __shfl_xor(vmin, off));
                vmax = max(vmax, __shfl_xor(vmax, off));
            }
            if (lane == 0) {
                s_red[0][wave] = vmin;
                s_red[1][wave] = vmax;
            }
            __syncthreads();
            int qmin = INT_MAX, qmax = INT_MIN;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                qmin = min(qmin, s_red[0][w]);
                qmax = max(qmax, s_red[1][w]);
            }
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

    // ---- Q of this lane's row: hi and lo bf16 halves of q * scale * log2 e
    // at head dims dh HDW + 32 st + 8 gq + (0..7)
    bf16x8 qh[NST], ql[NST];
    {
        const float* qrow = static_cast<const float*>(S.q) + (size_t)qi * a.q_rstride +
                            (size_t)(g * a.group + hg) * a.hd;
        float x[NST][8];
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            const int d0 = dh * HDW + 32 * st + 8 * gq;
            if (rvalid && a.hd == HD) {
                const f32x4 u = gload<f32x4>(qrow + d0), w = gload<f32x4>(qrow + d0 + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[st][e] = u[e];
                    x[st][4 + e] = w[e];
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    x[st][e] = (rvalid && d0 + e < a.hd) ? gload<float>(qrow + d0 + e) : 0.0f;
            }
        }
        // QK-norm of the row (rms_norm_inplace, ops.rs:106-114), when the
        // host leaves it to this kernel (no bias or RoPE, hd == HD): f32
        // squares summed in f64 over the row's four lanes (slot groups gq)
        // and, at hd 512, over the two waves of the row block (half 0's sum
        // first on both), then x * scale * w
        if (a.qn_w) {
            double ss = 0.0;
#pragma unroll
            for (int st = 0; st < NST; ++st)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float sq = x[st][e] * x[st][e];
                    ss += (double)sq;
                }
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if constexpr (G::DSPLIT > 1) {
                __shared__ double s_ss[NW][16];
                if (gq == 0) s_ss[wave][qc] = ss;
                __syncthreads();
                const double other = s_ss[wave ^ RBW][qc];
                ss = dh == 0 ? ss + other : other + ss;
            }
            {
                const float sc = 1.0f / (float)sqrt(ss / (double)HD + (double)a.qn_eps);
#pragma unroll
                for (int st = 0; st < NST; ++st) {
                    const int d0 = dh * HDW + 32 * st + 8 * gq;
                    const f32x4 w0 = gload<f32x4>(a.qn_w + d0), w1 = gload<f32x4>(a.qn_w + d0 + 4);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
#pragma clang fp contract(off)
                        x[st][e] = x[st][e] * sc * (e < 4 ? w0[e] : w1[e - 4]);
                    }
                }
            }
        }
#pragma unroll
        for (int st = 0; st < NST; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xs = x[st][e] * a.c;
                const __bf16 h = (__bf16)xs;
                qh[st][e] = h;
                ql[st][e] = (__bf16)(xs - (float)h);
            }
    }

    // ---- DMA: instruction j of this wave moves 64 chunks (1 KB) of a tile
    const uint32_t plane_bytes = (uint32_t)a.cap * HD * 2;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(S.k + (size_t)g * a.cap * HD, plane_bytes);
    const __amdgpu_buffer_rsrc_t rkl = make_rsrc(S.klo + (size_t)g * a.cap * HD, plane_bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(S.vt + (size_t)g * HD * a.cap, plane_bytes);
    const __amdgpu_buffer_rsrc_t rvl = make_rsrc(S.vlo + (size_t)g * HD * a.cap, plane_bytes);
    // K hi / lo: LDS chunk idx of the 2-tile K region holds key kappa(R),
    // head-dim chunk pc ^ swz(R) of plane idx / CPT
    int kvo[KDMA];
#pragma unroll
    for (int j = 0; j < KDMA; ++j) {
        const int idx = ((wave * KDMA + j) * 64 + lane) % CPT;
        const int R = idx / KCH, pc = idx % KCH;
        kvo[j] = (kappa(R) * HD + ((pc ^ swz<KCH>(R)) << 3)) * 2;
    }
    auto issue_k = [&](int t) __attribute__((always_inline)) {
        const int soff = t * BN * HD * 2;  // (K tile t starts at key 32 t)
#pragma unroll
        for (int j = 0; j < KDMA; ++j) {
            const int first = (wave * KDMA + j) * 64;  // first chunk of the instruction
            uint16_t* dst = lk + first * 8;            // (the two K tiles are contiguous)
            if (first < CPT)
                dma16(rk, dst, kvo[j], soff);
            else
                dma16(rkl, dst, kvo[j], soff);
        }
    };
    // V^T hi / lo: LDS chunk (d, pv) of a tile holds chunk pv ^ swz_v16(d)
    // of row d
    auto issue_v = [&](int t) __attribute__((always_inline)) {
        const int soff = t * BN * HD * 2;  // V^T tile t: HD x 32 contiguous
#pragma unroll
        for (int j = 0; j < VDMA; ++j) {
            const int first = (wave * VDMA + j) * 64;  // (the two V^T tiles are contiguous)
            const int idx = (first + lane) % CPT, d = idx / (BN / 8), pv = idx % (BN / 8);
            const int voff = (d * (BN / 8) + (pv ^ swz_v16(d))) * 16;
            if (first < CPT)
                dma16(rv, lv + first * 8, voff, soff);
            else
                dma16(rvl, lv + first * 8, voff, soff);
        }
    };

    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    if (t0 < t1) {
        issue_k(t0);
        issue_v(t0);
    }
    for (int t = t0; t < t1; ++t) {
        // K of tile t has landed (the V^T DMA issued after it may be in flight)
        wait_vmcnt<VDMA>();
        lds_barrier();
        // per-key positions and sequence ids of this lane's 8 keys
        // (MASK_KEYS; identity positions / one sequence where absent).  Loads
        // issued here complete before the vmcnt(0) below, so the counted DMA
        // waits stay exact or wait longer, never less.
        int kp[8], kqs[8];
        if constexpr (MODE == MASK_KEYS) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int kidx = t * BN + 8 * gq + i;
                const int kc = min(kidx, S.nk - 1);
                kp[i] = S.kpos ? gload<int>(S.kpos + kc) : kidx;
                kqs[i] = S.kseq ? gload<int>(S.kseq + kc) : 0;
            }
        }
        // ---- S^T = K Q^T over this wave's head dims, hi/lo split
        f32x4 s[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            const int R = 16 * kh + qc;
#pragma unroll
            for (int st = 0; st < NST; ++st) {
                const int pc = dh * (HDW / 8) + 4 * st + gq;
                const int off = R * HD + ((pc ^ swz<KCH>(R)) << 3);
                const bf16x8 kf = *reinterpret_cast<const bf16x8*>(lk + off);
                const bf16x8 kl = *reinterpret_cast<const bf16x8*>(lkl + off);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qh[st], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, ql[st], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[st], acc, 0, 0, 0);
            }
            s[kh] = acc;
        }
        if constexpr (G::DSPLIT > 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) xch[(wave * 8 + i) * 64 + lane] = s[i >> 2][i & 3];
        }
        // V^T of tile t has landed; every wave is done with the K tiles
        wait_vmcnt<0>();
        lds_barrier();
        if (t + 1 < t1) issue_k(t + 1);
        if constexpr (G::DSPLIT > 1) {
            const int pw = wave ^ RBW;  // the other head-dim half of this row block
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float other = xch[(pw * 8 + i) * 64 + lane];
                s[i >> 2][i & 3] = dh == 0 ? s[i >> 2][i & 3] + other : other + s[i >> 2][i & 3];
            }
        }
        // ---- mask, tile maximum of the row, lazy rescale
        // slot (kh, i) of this lane is key 32 t + 8 gq + 4 kh + i
        float sv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kidx = t * BN + 8 * gq + i;
            bool vis = rvalid && kidx < S.nk;
            if constexpr (MODE == MASK_POS) vis = vis && visible(my_qpos, kidx, my_qseq, 0, a.window, my_pref);
            if constexpr (MODE == MASK_KEYS) vis = vis && visible(my_qpos, kp[i], my_qseq, kqs[i], a.window, my_pref);
            sv[i] = vis ? s[i >> 2][i & 3] : -INFINITY;
        }
        float mt = max3(sv[0], sv[1], sv[2]);
        mt = max3(mt, sv[3], sv[4]);
        mt = max3(mt, sv[5], sv[6]);
        mt = __builtin_fmaxf(mt, sv[7]);
        mt = __builtin_fmaxf(mt, __shfl_xor(mt, 16));
        mt = __builtin_fmaxf(mt, __shfl_xor(mt, 32));
        if (mt > m + RESCALE_THRESHOLD || (m == -INFINITY && mt > -INFINITY)) {
            const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mt);
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db] *= f;
            l *= f;
            m = mt;
        }
        // ---- p = 2^(s - m) as bf16, its sum, and O^T += V^T P^T
        bf16x8 pb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[i] - m);
            pb[i] = (__bf16)p;
            l += (float)pb[i];
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = dh * HDW + 16 * db + qc;
            const bf16x8 vf = *reinterpret_cast<const bf16x8*>(lv + d * BN + ((gq ^ swz_v16(d)) << 3));
            const bf16x8 vl = *reinterpret_cast<const bf16x8*>(lvl + d * BN + ((gq ^ swz_v16(d)) << 3));
            o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pb, o[db], 0, 0, 0);
            o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, pb, o[db], 0, 0, 0);
        }
        // every wave is done with V^T (and with the partial scores)
        lds_barrier();
        if (t + 1 < t1) issue_v(t + 1);
    }

    // ---- the row's sum over its four slot groups; out or the split partial
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (!rvalid) return;
    if (a.n_split <= 1) {
        float* orow = S.out + (size_t)qi * a.o_rstride + (size_t)(g * a.group + hg) * a.hd;
        const float il = __builtin_amdgcn_rcpf(l);  // no visible key: 0 * inf = NaN (attention.rs:181-185)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d0 = dh * HDW + 16 * db + 4 * gq;
            const f32x4 val = o[db] * il;
            if (a.hd == HD) {
                gstore(orow + d0, val);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d0 + e < a.hd) orow[d0 + e] = val[e];
            }
        }
    } else {
        const size_t plane = (size_t)a.n_batch * a.n_head_kv * a.part_rows;
        const size_t prow = (size_t)(b * a.n_head_kv + g) * a.part_rows + r;
        float* po = a.part_o + (size_t)split * plane * HD + prow * HD;
#pragma unroll
        for (int db = 0; db < NDB; ++db) gstore(po + dh * HDW + 16 * db + 4 * gq, o[db]);
        if (dh == 0 && gq == 0) gstore(a.part_ml + ((size_t)split * plane + prow) * 2, make_float2(m, l));
    }
}

template <int HD>
hipError_t launch_hilo_hd(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    using G = HiloGeom<HD>;
    constexpr size_t lds = G::LDS_BYTES;
    if (p.mask == MASK_NONE) {
        auto k = attn_hilo_kernel<HD, MASK_NONE>;
        hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k, dim3(p.n_workgroups), dim3(G::NT), lds, st, a);
    } else if (p.mask == MASK_POS) {
        auto k = attn_hilo_kernel<HD, MASK_POS>;
        hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k, dim3(p.n_workgroups), dim3(G::NT), lds, st, a);
    } else if (p.mask == MASK_KEYS) {
        auto k = attn_hilo_kernel<HD, MASK_KEYS>;
        hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k, dim3(p.n_workgroups), dim3(G::NT), lds, st, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

// Rows per workgroup of the hi/lo kernel (four 16-row blocks).
int hilo_rows() { return HiloGeom<256>::QROWS; }

hipError_t launch_hilo(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    if (a.hd > p.hd_tile) return hipErrorInvalidValue;
    for (int i = 0; i < a.n_batch; ++i)
        if (!a.slot[i].klo || !a.slot[i].vlo) return hipErrorInvalidValue;  // no lo planes
    switch (p.hd_tile) {
        case 64: return launch_hilo_hd<64>(p, a, st);
        case 128: return launch_hilo_hd<128>(p, a, st);
        case 256: return launch_hilo_hd<256>(p, a, st);
        case 512: return launch_hilo_hd<512>(p, a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dr
