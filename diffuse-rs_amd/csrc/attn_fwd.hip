// attn_fwd.hip -- fused denoise-step attention for gfx950 (MI355X, CDNA4).
//
// Computes, for every (query row i, head h), the reference's
//   out[i][h] = sum_j softmax_j(scale * q[i][h] . k[j][h/group]) * v[j][h/group]
// over the keys j visible to i (src/model/attention.rs:101-186, visible() at
// :36-57), in one pass over the keys with an online softmax.
//
// Work decomposition.  A workgroup owns NW "row blocks" of 32 rows that share
// one KV head (GQA: the `group` query heads of a KV head are packed into the
// row dimension, so each K/V tile is read once for all of them) and a range
// of key tiles (its split).  Each wave owns one row block:
//   S^T[key][q] = K Q^T    via v_mfma_f32_32x32x16_bf16, A = K tile (LDS),
//                          B = the wave's Q^T fragments (registers)
//   O^T[d][q]  += V^T P^T  via the same MFMA, A = V^T tile (LDS),
//                          B = P^T straight from the S^T accumulators.
// Computing the transposed products makes each lane own one query column, so
// the softmax row statistics are per lane (plus one exchange with lane^32),
// and P never leaves registers.  K rows are loaded into LDS in a permuted
// order (sigma below) chosen so that lane half `hf` ends up holding keys
// 16*hf .. 16*hf+15 of every 32-key block, which is exactly the contiguous
// 8-key run each half must supply as the B operand of the PV product.
//
// The softmax works in the log2 domain: Q is multiplied by scale*log2(e)
// before rounding to bf16, p = exp2(s - m).  The running max is only moved
// when it grows by more than 8 (p <= 256 fits bf16/f32 exactly as well), which
// skips the O rescale on almost every tile; O / l is unchanged by the choice
// of m.  A row with no visible key ends with l = 0 and writes 0 * (1/0) = NaN,
// like the reference (attention.rs:181-185).
//
// Memory: K is [kv head][key][HD] and V is stored transposed [kv head][d][key]
// (the KV-cache layout written by kv_cache.hip), so both tiles arrive in LDS
// with plain 16-byte row loads.  LDS rows are XOR-swizzled in 16-byte chunks so
// the MFMA operand reads (16 B per lane) are bank-conflict free.  Two LDS
// stages: the global loads of tile t+1 are in flight while tile t computes.
#include "dr_internal.hpp"

#include <limits.h>
#include <math.h>

namespace dr {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// LDS row (within a 32-row block) that receives key offset kk (0..31).  The
// MFMA puts A-row R of the block in accumulator slot i of lane half hf with
// R = 8*(i/4) + 4*hf + (i%4); sigma(R) = 16*hf + i places key 16*hf + i there.
__device__ __forceinline__ int sigma_inv(int kk) {
    return ((kk >> 2) & 3) * 8 + (kk >> 4) * 4 + (kk & 3);
}

__device__ __forceinline__ bool visible(int qpos, int kpos, int qseq, int kseq, int window,
                                        int prefix) {
    if (qseq != kseq) return false;
    if (window >= 0 && abs(qpos - kpos) >= window) return false;
    if (prefix >= 0 && qpos < prefix) return kpos <= qpos;
    return true;
}

template <int HD, int BN, int NW, bool MASKED, bool QNORM>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const AttnArgs a) {
    constexpr int NB = BN / 32;       // 32-key blocks per tile
    constexpr int NC = HD / 16;       // QK^T contraction steps
    constexpr int ND = HD / 32;       // 32-row blocks of O^T
    constexpr int KCH = HD / 8;       // 16-byte chunks per K row
    constexpr int VCH = BN / 8;       // 16-byte chunks per V^T row
    constexpr int TILE = BN * HD;     // bf16 elements per K (or V^T) tile
    constexpr int NT = NW * 64;
    constexpr int NLD = TILE / 8 / NT;  // 16-byte chunks per thread per tile
    static_assert(TILE / 8 % NT == 0, "tile must split evenly over the workgroup");

    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_kmeta[2][2][BN];
    __shared__ int s_red[3][NW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, hf = lane >> 5;

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
    const int wg_row0 = rg * NW * 32;
    if (wg_row0 >= rows_total) return;  // uniform over the workgroup and all splits
    const int r = wg_row0 + wave * 32 + col;
    const bool rvalid = r < rows_total;
    const int hg = rvalid ? r / S.nq : 0;
    const int qi = rvalid ? r - hg * S.nq : 0;
    const int head = g * a.group + hg;

    // ---- Q fragments: lane holds Q[qi][head][16c + 8hf .. +7] for every c.
    bf16x8 qf[NC];
    {
        float x[NC][8];
        const float* qrow =
            static_cast<const float*>(S.q) + (size_t)qi * a.q_rstride + (size_t)head * a.hd;
        if (rvalid && a.hd == HD) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const f32x4* p = reinterpret_cast<const f32x4*>(qrow + 16 * c + 8 * hf);
                f32x4 u = p[0], w = p[1];
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

    // ---- key tile range of this workgroup and split
    int kt_lo = 0, kt_hi = (S.nk + BN - 1) / BN;
    int my_qpos = 0, my_qseq = 0, my_pref = -1;
    int qmin = 0, qmax = 0;
    bool prefix_free = true;
    if constexpr (MASKED) {
        my_qpos = rvalid ? S.qpos[qi] : 0;
        my_qseq = (rvalid && S.qseq) ? S.qseq[qi] : 0;
        my_pref = S.qprefix ? (rvalid ? S.qprefix[qi] : -1) : a.prefix;
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
        if (a.window >= 0 && S.kpos == nullptr) {
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

    // ---- main loop
    f32x16 o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    const size_t kv_base = (size_t)g * a.cap;      // K row base of this kv head
    const size_t vt_base = (size_t)g * HD;         // V^T row base of this kv head
    u32x4 kreg[NLD], vreg[NLD];
    int kmeta0 = 0, kmeta1 = 0;

    auto gload = [&](int t) {
        const int k0 = t * BN;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int idx = tid + i * NT;
            const int key = idx / KCH, c = idx % KCH;
            kreg[i] = *reinterpret_cast<const u32x4*>(S.k + (kv_base + k0 + key) * HD + c * 8);
        }
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int idx = tid + i * NT;
            const int d = idx / VCH, kc = idx % VCH;
            vreg[i] = *reinterpret_cast<const u32x4*>(S.vt + (vt_base + d) * a.cap + k0 + kc * 8);
        }
        if constexpr (MASKED) {
            if (tid < BN) {
                const int kidx = k0 + tid;
                kmeta0 = (S.kpos && kidx < S.nk) ? S.kpos[kidx] : kidx;
                kmeta1 = (S.kseq && kidx < S.nk) ? S.kseq[kidx] : 0;
            }
        }
    };
    auto lstore = [&](int st) {
        uint16_t* ks = smem + st * 2 * TILE;
        uint16_t* vs = ks + TILE;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int idx = tid + i * NT;
            const int key = idx / KCH, c = idx % KCH;
            const int R = (key & ~31) + sigma_inv(key & 31);
            *reinterpret_cast<u32x4*>(ks + R * HD + ((c ^ swz<KCH>(R)) << 3)) = kreg[i];
        }
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int idx = tid + i * NT;
            const int d = idx / VCH, kc = idx % VCH;
            *reinterpret_cast<u32x4*>(vs + d * BN + ((kc ^ swz<VCH>(d)) << 3)) = vreg[i];
        }
        if constexpr (MASKED) {
            if (tid < BN) {
                s_kmeta[st][0][tid] = kmeta0;
                s_kmeta[st][1][tid] = kmeta1;
            }
        }
    };

    auto compute = [&](int st, int t) {
        const uint16_t* ks = smem + st * 2 * TILE;
        const uint16_t* vs = ks + TILE;
        f32x16 sacc[NB];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            sacc[kb] = f32x16{};
            const int R = kb * 32 + col;
            const uint16_t* krow = ks + R * HD;
            const int sw = swz<KCH>(R);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const bf16x8 af =
                    *reinterpret_cast<const bf16x8*>(krow + (((2 * c + hf) ^ sw) << 3));
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[c], sacc[kb], 0, 0, 0);
            }
        }

        // Masking: sacc[kb][i] is the score of key t*BN + kb*32 + 16*hf + i.
        const int kbase = t * BN;
        bool full = kbase + BN <= S.nk;
        if constexpr (MASKED) {
            const bool ident = S.kpos == nullptr && S.kseq == nullptr && S.qseq == nullptr;
            const bool win_ok =
                a.window < 0 || (qmax - kbase < a.window && kbase + BN - 1 - qmin < a.window);
            full = full && ident && prefix_free && win_ok;
        }
        if (!full) {
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kl = kb * 32 + 16 * hf + i;
                    bool vis = kbase + kl < S.nk;
                    if constexpr (MASKED) {
                        vis = vis && visible(my_qpos, s_kmeta[st][0][kl], my_qseq,
                                             s_kmeta[st][1][kl], a.window, my_pref);
                    }
                    if (!vis) sacc[kb][i] = -INFINITY;
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
        bf16x8 pf[NB][2];
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(sacc[kb][8 * hh + j] - mu);
                    l_run += p;
                    pf[kb][hh][j] = (__bf16)p;
                }

        // O^T += V^T P^T.  Contraction slot 8*hf + j of MFMA (kb, hh) is key
        // kb*32 + 16*hf + 8*hh + j, in both operands.
#pragma unroll
        for (int db = 0; db < ND; ++db) {
            const int d = db * 32 + col;
            const uint16_t* vrow = vs + d * BN;
            const int sw = swz<VCH>(d);
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const bf16x8 vf = *reinterpret_cast<const bf16x8*>(
                        vrow + (((4 * kb + 2 * hf + hh) ^ sw) << 3));
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[kb][hh], o[db], 0, 0,
                                                                    0);
                }
        }
    };

    if (t0 < t1) {
        gload(t0);
        lstore(0);
        __syncthreads();
        for (int t = t0; t < t1; ++t) {
            const int st = (t - t0) & 1;
            if (t + 1 < t1) gload(t + 1);
            compute(st, t);
            if (t + 1 < t1) lstore(st ^ 1);
            __syncthreads();
        }
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);

    if (a.n_split == 1) {
        if (!rvalid) return;
        const float inv = 1.0f / l_tot;
        float* orow = S.out + (size_t)qi * a.o_rstride + (size_t)head * a.hd;
        // o[db][4j + e] is O^T[d = db*32 + 8j + 4hf + e][col]
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d0 = db * 32 + 8 * j + 4 * hf;
                f32x4 val;
#pragma unroll
                for (int e = 0; e < 4; ++e) val[e] = o[db][4 * j + e] * inv;
                if (a.hd == HD) {
                    *reinterpret_cast<f32x4*>(orow + d0) = val;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < a.hd) orow[d0 + e] = val[e];
                }
            }
        return;
    }

    // Split partials, in accumulator layout (coalesced: lane-fastest).
    const size_t nrb = (size_t)a.n_batch * a.n_head_kv * a.rowgroups * NW;
    const size_t rb = ((size_t)(b * a.n_head_kv + g) * a.rowgroups + rg) * NW + wave;
    float* po = a.part_o + ((size_t)split * nrb + rb) * (size_t)(HD * 32);
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) po[(db * 16 + i) * 64 + lane] = o[db][i];
    float* pml = a.part_ml + ((size_t)split * nrb + rb) * 128;
    pml[lane] = m_run;
    pml[64 + lane] = l_tot;
}

// Merges the key-split partials of one 32-row block per wave:
// M = max m_s, L = sum l_s 2^(m_s - M), O = sum O_s 2^(m_s - M) / L.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const CombineArgs a, int rb_per_bg,
                                                           int n_rb) {
    constexpr int ND = HD / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, hf = lane >> 5;
    const int rb = blockIdx.x * 4 + wave;
    if (rb >= n_rb) return;
    const int bg = rb / rb_per_bg, rbk = rb % rb_per_bg;
    const int b = bg / a.n_head_kv, g = bg % a.n_head_kv;
    const AttnSlot& S = a.slot[b];
    const int r = rbk * 32 + col;
    if (r >= a.group * S.nq) return;
    const int hg = r / S.nq, qi = r - hg * S.nq;
    const int head = g * a.group + hg;

    float M = -INFINITY;
    for (int s = 0; s < a.n_split; ++s)
        M = fmaxf(M, a.part_ml[((size_t)s * n_rb + rb) * 128 + lane]);
    f32x16 o[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = f32x16{};
    float L = 0.0f;
    for (int s = 0; s < a.n_split; ++s) {
        const float* pml = a.part_ml + ((size_t)s * n_rb + rb) * 128;
        const float ms = pml[lane];
        const float w = (ms == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
        L += w * pml[64 + lane];
        const float* po = a.part_o + ((size_t)s * n_rb + rb) * (size_t)(HD * 32);
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] += w * po[(db * 16 + i) * 64 + lane];
    }
    const float inv = 1.0f / L;
    float* orow = S.out + (size_t)qi * a.o_rstride + (size_t)head * a.hd;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d0 = db * 32 + 8 * j + 4 * hf;
            f32x4 val;
#pragma unroll
            for (int e = 0; e < 4; ++e) val[e] = o[db][4 * j + e] * inv;
            if (a.hd == HD) {
                *reinterpret_cast<f32x4*>(orow + d0) = val;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d0 + e < a.hd) orow[d0 + e] = val[e];
            }
        }
}

template <int HD, int BN, int NW, bool MASKED, bool QNORM>
hipError_t launch_fwd(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    constexpr size_t lds = (size_t)4 * BN * HD * sizeof(uint16_t);
    static bool attr_set = false;
    auto fn = attn_fwd_kernel<HD, BN, NW, MASKED, QNORM>;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(fn, dim3(p.n_workgroups), dim3(NW * 64), lds, st, a);
    return hipGetLastError();
}

template <int HD, int BN, int NW>
hipError_t launch_variant(const LaunchPlan& p, const AttnArgs& a, hipStream_t st) {
    if (p.masked) {
        return p.qnorm ? launch_fwd<HD, BN, NW, true, true>(p, a, st)
                       : launch_fwd<HD, BN, NW, true, false>(p, a, st);
    }
    return p.qnorm ? launch_fwd<HD, BN, NW, false, true>(p, a, st)
                   : launch_fwd<HD, BN, NW, false, false>(p, a, st);
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
    c.rowgroups = a.rowgroups;
    c.n_split = a.n_split;
    c.part_o = a.part_o;
    c.part_ml = a.part_ml;
    const int rb_per_bg = a.rowgroups * p.waves;
    const int n_rb = a.n_batch * a.n_head_kv * rb_per_bg;
    hipLaunchKernelGGL(attn_combine_kernel<HD>, dim3((n_rb + 3) / 4), dim3(256), 0, st, c,
                       rb_per_bg, n_rb);
    return hipGetLastError();
}

}  // namespace

LaunchPlan plan_attention(int hd, int n_batch, int n_head_kv, int group, int max_nq, int max_nk,
                          bool masked, bool qnorm, int n_cu, int force_split) {
    LaunchPlan p;
    p.hd_tile = hd <= 64 ? 64 : (hd <= 128 ? 128 : 256);
    p.block_n = p.hd_tile == 256 ? 32 : 64;
    p.waves = 4;
    p.masked = masked;
    p.qnorm = qnorm;
    const int rows = group * max_nq;
    p.rowgroups = (rows + p.waves * 32 - 1) / (p.waves * 32);
    if (p.rowgroups < 1) p.rowgroups = 1;
    const int base = n_batch * n_head_kv * p.rowgroups;
    const int ntiles = (max_nk + p.block_n - 1) / p.block_n;
    int split = 1;
    if (force_split > 0) {
        split = force_split;
    } else {
        // Fill the chip with about one workgroup per CU while keeping at
        // least two key tiles per split.
        const int target = n_cu > 0 ? n_cu : 256;
        split = (target + base - 1) / base;
        const int max_split = ntiles / 2 > 1 ? ntiles / 2 : 1;
        if (split > max_split) split = max_split;
    }
    if (split < 1) split = 1;
    p.n_split = split;
    p.n_workgroups = base * split;
    return p;
}

size_t split_workspace_bytes(const LaunchPlan& p, int n_batch, int n_head_kv) {
    if (p.n_split <= 1) return 0;
    const size_t nrb = (size_t)n_batch * n_head_kv * p.rowgroups * p.waves;
    return (size_t)p.n_split * nrb * ((size_t)p.hd_tile * 32 + 128) * sizeof(float);
}

hipError_t launch_attention(const LaunchPlan& p, AttnArgs& a, hipStream_t st) {
    a.rowgroups = p.rowgroups;
    a.n_split = p.n_split;
    if (p.n_split > 1) {
        const size_t nrb = (size_t)a.n_batch * a.n_head_kv * p.rowgroups * p.waves;
        a.part_ml = a.part_o + (size_t)p.n_split * nrb * p.hd_tile * 32;
    }
    hipError_t e;
    switch (p.hd_tile) {
        case 64: e = launch_variant<64, 64, 4>(p, a, st); break;
        case 128: e = launch_variant<128, 64, 4>(p, a, st); break;
        case 256: e = launch_variant<256, 32, 4>(p, a, st); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || p.n_split == 1) return e;
    switch (p.hd_tile) {
        case 64: return launch_combine<64>(p, a, st);
        case 128: return launch_combine<128>(p, a, st);
        default: return launch_combine<256>(p, a, st);
    }
}

}  // namespace dr
