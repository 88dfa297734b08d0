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
// gather: StepCache::gather (cache.rs:73-82) -- bf16 back to f32 rows.
#include "dr_internal.hpp"

#include <math.h>

namespace dr {
namespace {

__device__ __forceinline__ uint16_t f2bf(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

constexpr int STORE_ROWS = 32;  // rows per workgroup

// grid (ceil(n / 32), n_head_kv); 256 threads.
template <int HD>
__global__ __launch_bounds__(256) void kv_store_kernel(const StoreArgs a) {
    constexpr int EPL = HD / 64;  // K elements per lane per row
    __shared__ uint16_t vtile[STORE_ROWS][HD + 2];
    const int g = blockIdx.y;
    const int r0 = blockIdx.x * STORE_ROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // K: each wave normalises, converts and stores 8 rows.
    for (int rr = 0; rr < STORE_ROWS / 4; ++rr) {
        const int r = r0 + wave * (STORE_ROWS / 4) + rr;
        if (r >= a.n) break;
        const int pos = a.pos ? a.pos[r] : r;
        const float* src = a.k + ((size_t)r * a.n_head_kv + g) * a.hd;
        float x[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int d = lane * EPL + e;
            x[e] = d < a.hd ? src[d] : 0.0f;
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
    }

    // V: stage 32 rows in LDS, then write them transposed.
    for (int idx = tid; idx < STORE_ROWS * HD; idx += 256) {
        const int rr = idx / HD, d = idx % HD;
        const int r = r0 + rr;
        const float x = (r < a.n && d < a.hd) ? a.v[((size_t)r * a.n_head_kv + g) * a.hd + d] : 0.0f;
        vtile[rr][d] = f2bf(x);
    }
    __syncthreads();
    for (int idx = tid; idx < STORE_ROWS * HD; idx += 256) {
        const int rr = idx % STORE_ROWS, d = idx / STORE_ROWS;
        const int r = r0 + rr;
        if (r < a.n) {
            const int pos = a.pos ? a.pos[r] : r;
            a.vtc[((size_t)g * HD + d) * a.cap + pos] = vtile[rr][d];
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
    dim3 grid((a.n + STORE_ROWS - 1) / STORE_ROWS, a.n_head_kv);
    switch (hd_tile) {
        case 64: hipLaunchKernelGGL(kv_store_kernel<64>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(kv_store_kernel<128>, grid, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(kv_store_kernel<256>, grid, dim3(256), 0, st, a); break;
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
