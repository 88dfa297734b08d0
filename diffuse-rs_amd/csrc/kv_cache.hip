// kv_cache.hip -- the inter-step KV cache in HBM (StepCache,
// src/model/cache.rs:25-115), bf16, position-indexed.
//
// Layout per (layer, batch slot), for n_head_kv heads and capacity `cap`
// positions (a multiple of 64), HD = the head-dim tile (64/128/256):
//   K  : [n_head_kv][cap][HD]   row = sequence position
//   V^T: [n_head_kv][HD][cap]   V transposed: a d-row holds all positions
// The attention kernel stages both as 16-byte row loads; V^T is exactly the
// operand orientation the P.V MFMA needs, so the transpose is paid once per
// stored row instead of once per attention tile.
//
// store:  StepCache::store (cache.rs:62-71) -- f32 rows -> bf16 at their
//         positions, optionally after per-head RMSNorm of K (norm_heads,
//         ops.rs:384-389, applied before the store in forward.rs:300-302).
//         One launch: workgroups [0, n_kblocks) write K rows (one wave per
//         (row, kv head)); the rest transpose 64x64 blocks of V through LDS.
// gather: StepCache::gather (cache.rs:73-82) -- bf16 back to f32 rows.
#include "dr_internal.hpp"

#include <math.h>

namespace dr {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint16_t f2bf(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

constexpr int VT_ROWS = 64;  // positions per V^T block
constexpr int VT_D = 64;     // head-dim entries per V^T block

template <int HD>
__global__ __launch_bounds__(256) void kv_store_kernel(const StoreArgs a, int n_kblocks) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if ((int)blockIdx.x < n_kblocks) {
        // ---- K: one wave per (row, kv head); EPL consecutive values per lane
        constexpr int EPL = HD / 64;
        const int pair = blockIdx.x * 4 + wave;
        if (pair >= a.n * a.n_head_kv) return;
        const int r = pair / a.n_head_kv, g = pair % a.n_head_kv;
        const int pos = a.pos ? a.pos[r] : r;
        const float* src = a.k + (size_t)pair * a.hd;
        float x[EPL];
        if (a.hd == HD) {
            if constexpr (EPL == 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(src + lane * 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = v[e];
            } else {
#pragma unroll
                for (int e = 0; e < EPL; ++e) x[e] = src[lane * EPL + e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int d = lane * EPL + e;
                x[e] = d < a.hd ? src[d] : 0.0f;
            }
        }
        if (a.kn_w) {
            // rms_norm_inplace (ops.rs:106-114): f32 squares summed in f64.
            double ss = 0.0;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float sq = x[e] * x[e];
                ss += (double)sq;
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            const float sc = 1.0f / (float)sqrt(ss / (double)a.hd + (double)a.kn_eps);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int d = lane * EPL + e;
                if (d < a.hd) x[e] = x[e] * sc * a.kn_w[d];
            }
        }
        uint16_t* dst = a.kc + ((size_t)g * a.cap + pos) * HD + lane * EPL;
#pragma unroll
        for (int e = 0; e < EPL; ++e) dst[e] = f2bf(x[e]);
        return;
    }

    // ---- V^T: a block of 64 rows x 64 d of one kv head, transposed via LDS
    __shared__ uint16_t tile[VT_D][VT_ROWS + 2];
    constexpr int NDC = HD / VT_D;
    const int nrc = (a.n + VT_ROWS - 1) / VT_ROWS;
    int t = blockIdx.x - n_kblocks;
    const int rc = t % nrc;
    t /= nrc;
    const int dc = t % NDC;
    const int g = t / NDC;
    {
        const int row = tid >> 2, d0 = (tid & 3) * 16;
        const int r = rc * VT_ROWS + row;
        const int dbase = dc * VT_D + d0;
        const float* src = a.v + ((size_t)r * a.n_head_kv + g) * a.hd + dbase;
        float x[16];
        if (r < a.n && a.hd == HD) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * q4);
#pragma unroll
                for (int e = 0; e < 4; ++e) x[4 * q4 + e] = v[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) x[e] = (r < a.n && dbase + e < a.hd) ? src[e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) tile[d0 + e][row] = f2bf(x[e]);
    }
    __syncthreads();
    {
        const int d = tid >> 2, r0 = (tid & 3) * 16;
        const int rfirst = rc * VT_ROWS + r0;
        if (rfirst >= a.n) return;
        const int nr = min(16, a.n - rfirst);
        uint16_t* drow = a.vtc + ((size_t)g * HD + dc * VT_D + d) * a.cap;
        const int p0 = a.pos ? a.pos[rfirst] : rfirst;
        const bool contiguous =
            nr == 16 && (a.pos == nullptr || a.pos[rfirst + 15] - p0 == 15) && (p0 & 7) == 0;
        if (contiguous) {
            u32x4 w[2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[h][e] = (uint32_t)tile[d][r0 + 8 * h + 2 * e] |
                              ((uint32_t)tile[d][r0 + 8 * h + 2 * e + 1] << 16);
            *reinterpret_cast<u32x4*>(drow + p0) = w[0];
            *reinterpret_cast<u32x4*>(drow + p0 + 8) = w[1];
        } else {
            for (int e = 0; e < nr; ++e) {
                const int pos = a.pos ? a.pos[rfirst + e] : rfirst + e;
                drow[pos] = tile[d][r0 + e];
            }
        }
    }
}

// One thread per (row, kv head, d).
template <int HD>
__global__ __launch_bounds__(256) void kv_gather_kernel(const GatherArgs a) {
    const size_t total = (size_t)a.n * a.n_head_kv * a.hd;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * 256) {
        const int d = (int)(idx % a.hd);
        const size_t rg = idx / a.hd;
        const int g = (int)(rg % a.n_head_kv);
        const int r = (int)(rg / a.n_head_kv);
        const int pos = a.pos[r];
        a.out_k[idx] = bf2f(a.kc[((size_t)g * a.cap + pos) * HD + d]);
        a.out_v[idx] = bf2f(a.vtc[((size_t)g * HD + d) * a.cap + pos]);
    }
}

}  // namespace

hipError_t launch_store(int hd_tile, const StoreArgs& a, hipStream_t st) {
    if (a.n <= 0) return hipSuccess;
    const int n_kblocks = (a.n * a.n_head_kv + 3) / 4;
    const int n_vblocks = (a.n + VT_ROWS - 1) / VT_ROWS * (hd_tile / VT_D) * a.n_head_kv;
    dim3 grid(n_kblocks + n_vblocks);
    switch (hd_tile) {
        case 64: hipLaunchKernelGGL(kv_store_kernel<64>, grid, dim3(256), 0, st, a, n_kblocks); break;
        case 128: hipLaunchKernelGGL(kv_store_kernel<128>, grid, dim3(256), 0, st, a, n_kblocks); break;
        case 256: hipLaunchKernelGGL(kv_store_kernel<256>, grid, dim3(256), 0, st, a, n_kblocks); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gather(int hd_tile, const GatherArgs& a, hipStream_t st) {
    const size_t total = (size_t)a.n * a.n_head_kv * a.hd;
    if (total == 0) return hipSuccess;
    size_t blocks = (total + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    switch (hd_tile) {
        case 64: hipLaunchKernelGGL(kv_gather_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(kv_gather_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(kv_gather_kernel<256>, dim3((unsigned)blocks), dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dr
