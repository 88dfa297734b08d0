// qkv_epilogue.hip -- the per-layer Q/K/V epilogue of attention_block
// (src/model/forward.rs:291-310) on device rows, in place:
//   add_bias of q, k, v                      ops.rs:373-382
//   QK-norm: norm_heads(q, q_norm), (k, ...)  ops.rs:384-389 -> rms_norm_inplace :106-114
//   Gemma: rms_norm_noscale of each V head    ops.rs:116-124 (forward.rs:303-308)
//   apply_rope(q, k) at the rows' positions   ops.rs:419-452, with the f32
//                                             (sin, cos) table of build_rope_cache_ff
//                                             (ops.rs:396-417) built on the host
// in that order, the reference's.  HBM-bound: each head row is read and
// written once.
#include "dr_internal.hpp"

#include <math.h>

namespace dr {
namespace {

constexpr int EPI_WAVES = 4;  // waves per workgroup
constexpr int SPW = 4;        // head rows per wave, processed in lockstep

// Head row s of the launch: one of q / k / v of one row.
struct Seg {
    float* x;
    const float* bias;
    int r;      // row (position index)
    int kind;   // 0: q, 1: k, 2: v
    bool valid;
};

__device__ __forceinline__ Seg seg_of(const EpiArgs& a, int s) {
    Seg g{};
    const int per_row = a.n_head + 2 * a.n_head_kv;
    g.valid = s < a.n * per_row;
    if (!g.valid) return g;
    const int r = s / per_row, j = s - r * per_row;
    g.r = r;
    const int hd = a.hd;
    if (j < a.n_head) {
        g.x = a.q + ((size_t)r * a.n_head + j) * hd;
        g.bias = a.bq ? a.bq + (size_t)j * hd : nullptr;
        g.kind = 0;
    } else if (j < a.n_head + a.n_head_kv) {
        const int gk = j - a.n_head;
        g.x = a.k + ((size_t)r * a.n_head_kv + gk) * hd;
        g.bias = a.bk ? a.bk + (size_t)gk * hd : nullptr;
        g.kind = 1;
    } else {
        const int gv = j - a.n_head - a.n_head_kv;
        g.x = a.v + ((size_t)r * a.n_head_kv + gv) * hd;
        g.bias = a.bv ? a.bv + (size_t)gv * hd : nullptr;
        g.kind = 2;
    }
    return g;
}

// One wave per SPW consecutive head rows, taken through every phase
// together (loads, bias, norm sums and their cross-lane reduction, RoPE,
// stores), so the latency chains of the rows overlap.  Lane l holds the EPL
// contiguous elements l*EPL .. l*EPL + EPL - 1 of a row (vector loads).
template <int EPL>  // elements per lane: hd <= 64 * EPL
__global__ __launch_bounds__(EPI_WAVES * 64) void qkv_epilogue_kernel(const EpiArgs a) {
    // Rust evaluates a*cos - b*sin and the norms' products without fused
    // multiply-adds; so does this kernel.
#pragma clang fp contract(off)
    __shared__ float row_lds[EPI_WAVES][SPW][64 * EPL];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int s0 = (blockIdx.x * EPI_WAVES + wave) * SPW;
    const int hd = a.hd, half = a.rot / 2, d0 = lane * EPL;
    const bool whole = a.vec && d0 + EPL <= hd;  // this lane's chunk: vector loads
    Seg sg[SPW];
    float y[SPW][EPL], bb[SPW][EPL], wq[EPL], wk[EPL];
    float2 sc2[SPW][EPL];

    // ---- every global load first: values, biases, gains; then the table
    // entries at the rows' positions
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int d = d0 + e;
        wq[e] = (a.qn_w && d < hd) ? a.qn_w[d] : 1.0f;
        wk[e] = (a.kn_w && d < hd) ? a.kn_w[d] : 1.0f;
    }
    int pos[SPW];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        sg[i] = seg_of(a, s0 + i);
        // (contiguous rows: the table row follows from the row index, so the
        // table loads need not wait for a position load)
        pos[i] = (sg[i].valid && sg[i].kind < 2 && a.rope) ? (a.pos0 >= 0 ? a.pos0 + sg[i].r : a.pos[sg[i].r]) : 0;
        if (sg[i].valid && whole && EPL % 4 == 0) {
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                const float4 t = *reinterpret_cast<const float4*>(sg[i].x + d0 + e);
                y[i][e] = t.x; y[i][e + 1] = t.y; y[i][e + 2] = t.z; y[i][e + 3] = t.w;
            }
        } else if (sg[i].valid && whole && EPL == 2) {
            const float2 t = *reinterpret_cast<const float2*>(sg[i].x + d0);
            y[i][0] = t.x;
            y[i][1] = t.y;
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e) y[i][e] = (sg[i].valid && d0 + e < hd) ? sg[i].x[d0 + e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e)
            bb[i][e] = (sg[i].valid && sg[i].bias && d0 + e < hd) ? sg[i].bias[d0 + e] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < SPW; ++i)
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int d = d0 + e;
            const int j = d < half ? d : d - half;
            sc2[i][e] = (sg[i].valid && sg[i].kind < 2 && a.rope && d < a.rot)
                            ? *reinterpret_cast<const float2*>(a.rope + ((size_t)pos[i] * half + j) * 2)
                            : make_float2(0.0f, 1.0f);
        }

    // ---- bias (add_bias)
#pragma unroll
    for (int i = 0; i < SPW; ++i)
        if (sg[i].bias) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) y[i][e] += bb[i][e];
        }

    // ---- RMSNorm: f32 squares summed in f64, scale = 1 / (f32) sqrt(ss/n + eps)
    bool nrm[SPW];
    double ss[SPW];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        nrm[i] = sg[i].valid && ((sg[i].kind == 0 && a.qn_w) || (sg[i].kind == 1 && a.kn_w) ||
                                 (sg[i].kind == 2 && a.v_norm));
        ss[i] = 0.0;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float sq = y[i][e] * y[i][e];
            if (d0 + e < hd) ss[i] += (double)sq;
        }
    }
    if (nrm[0] || nrm[1] || nrm[2] || nrm[3]) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
#pragma unroll
            for (int i = 0; i < SPW; ++i) ss[i] += __shfl_xor(ss[i], off);
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            if (!nrm[i]) continue;
            const float sc = 1.0f / (float)sqrt(ss[i] / (double)hd + (double)a.eps);
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                y[i][e] = sg[i].kind == 2 ? y[i][e] * sc : y[i][e] * sc * (sg[i].kind == 0 ? wq[e] : wk[e]);
        }
    }

    // ---- RoPE on q and k rows: dims (j, j + rot/2), j < rot/2, rotate by
    // the angle of (position, j); a dim's partner sits in another lane, so
    // the rows go through this wave's LDS
    if (a.rope) {
#pragma unroll
        for (int i = 0; i < SPW; ++i)
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                if (d0 + e < hd) row_lds[wave][i][d0 + e] = y[i][e];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            if (!sg[i].valid || sg[i].kind == 2) continue;
            const float* b = row_lds[wave][i];
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int d = d0 + e;
                if (d >= a.rot) continue;
                const float sn = sc2[i][e].x, cs = sc2[i][e].y;
                if (d < half)
                    y[i][e] = b[d] * cs - b[d + half] * sn;
                else
                    y[i][e] = b[d - half] * sn + b[d] * cs;
            }
        }
    }

    // ---- stores
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        if (!sg[i].valid) continue;
        if (whole && EPL % 4 == 0) {
#pragma unroll
            for (int e = 0; e < EPL; e += 4)
                *reinterpret_cast<float4*>(sg[i].x + d0 + e) =
                    make_float4(y[i][e], y[i][e + 1], y[i][e + 2], y[i][e + 3]);
        } else if (whole && EPL == 2) {
            *reinterpret_cast<float2*>(sg[i].x + d0) = make_float2(y[i][0], y[i][1]);
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e)
                if (d0 + e < hd) sg[i].x[d0 + e] = y[i][e];
        }
    }
}

template <int EPL>
hipError_t launch_epi(const EpiArgs& a, hipStream_t st) {
    const long segs = (long)a.n * (a.n_head + 2 * a.n_head_kv);
    const long per_wg = (long)EPI_WAVES * SPW;
    const long grid = (segs + per_wg - 1) / per_wg;
    hipLaunchKernelGGL(qkv_epilogue_kernel<EPL>, dim3((unsigned)grid), dim3(EPI_WAVES * 64), 0, st,
                       a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_epilogue(const EpiArgs& a, hipStream_t st) {
    if (a.n <= 0) return hipSuccess;
    if (a.hd <= 64) return launch_epi<1>(a, st);
    if (a.hd <= 128) return launch_epi<2>(a, st);
    if (a.hd <= 256) return launch_epi<4>(a, st);
    if (a.hd <= 512) return launch_epi<8>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace dr
