// qmatmul.hip -- the projection after the attention (Wo, src/model/forward.rs:
// 345-350) on GGUF k-quant weights: native_matmul (src/model/matmul.rs:120-148)
// quantizes the f32 activations to Q8_K (ActScratch::q8k, matmul.rs:64-71) and
// takes, for every (activation row t, weight row r), the Q4_K or Q6_K x Q8_K
// block dot product; residual_add (ops.rs:365-370) follows.
//
// Every output runs the reference's scalar dot in its own order (the test
// module's vec_dot of src/kernels.rs:228-347): the integer parts are exact
// whatever the grouping, and the f32 operations are the same ones in the same
// sequence, without fused multiply-adds.  So each output matches that
// restatement bit for bit.
#include "dr_internal.hpp"

namespace dr {
namespace {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144, Q6K_BYTES = 210;

// f16_to_f32 of src/kernels.rs:46-69 (bit for bit, NaN payload included).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            const uint32_t lz = __builtin_clz(mant) - 21;  // shifts until bit 10 is set
            bits = (sign << 31) | ((113u - lz) << 23) | (((mant << lz) & 0x3FFu) << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | (0xFFu << 23) | (mant ? 0x7FFFFFu : 0u);
    } else {
        bits = (sign << 31) | ((ex + 112u) << 23) | (mant << 13);
    }
    return __uint_as_float(bits);
}

// quantize_rows_q8_k (src/kernels.rs:79-122): one workgroup per 256-value
// block, thread i owns value i.  The first value of largest magnitude gives
// iscale = -128 / max; q = round(iscale x) capped at 127; d = 1 / iscale;
// bsums = sums of 16.  NaN values never win the scan (amax < |x| is false).
__global__ __launch_bounds__(256) void q8k_quantize_kernel(const float* __restrict__ x, int cols,
                                                           int nb, Q8KBlock* __restrict__ out) {
    __shared__ float s_a[4];
    __shared__ int s_i[4];
    __shared__ float s_mx;
    const int blk = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = blk / nb, b = blk - t * nb;
    const float v = x[(size_t)t * cols + (size_t)b * QK + tid];
    float a = v != v ? -1.0f : fabsf(v);
    int idx = tid;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(a, off);
        const int oi = __shfl_xor(idx, off);
        if (oa > a || (oa == a && oi < idx)) {
            a = oa;
            idx = oi;
        }
    }
    if (lane == 0) {
        s_a[wave] = a;
        s_i[wave] = idx;
    }
    __syncthreads();
    float amax = s_a[0];
    int imax = s_i[0];
#pragma unroll
    for (int w = 1; w < 4; ++w)
        if (s_a[w] > amax) {  // waves in index order: a tie keeps the earlier one
            amax = s_a[w];
            imax = s_i[w];
        }
    if (tid == imax) s_mx = v;
    __syncthreads();
    Q8KBlock* o = out + blk;
    int q = 0;
    if (amax > 0.0f) {
#pragma clang fp contract(off)
        const float iscale = -128.0f / s_mx;
        const float r = fminf(roundf(iscale * v), 127.0f);
        q = (int)r;
        if (tid == 0) o->d = 1.0f / iscale;
    } else if (tid == 0) {
        o->d = 0.0f;
    }
    o->qs[tid] = (int8_t)q;
    int s = q;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off);
    if ((tid & 15) == 0) o->bsums[tid >> 4] = (int16_t)s;
}

// Tile of one workgroup: TR weight rows x TT activation rows; thread (rg, tg)
// owns weight rows 2 rg, 2 rg + 1 and activation rows 4 tg .. 4 tg + 3.
constexpr int TR = 64, TT = 32;

// Q4_K: the 6-bit scales and mins of a block (src/kernels.rs:193-201).
__device__ __forceinline__ void q4k_unpack_scales(const uint8_t* p, uint8_t sc[8], uint8_t mn[8]) {
    uint32_t u[4];
    u[0] = p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
    u[1] = p[4] | (p[5] << 8) | (p[6] << 16) | ((uint32_t)p[7] << 24);
    u[2] = p[8] | (p[9] << 8) | (p[10] << 16) | ((uint32_t)p[11] << 24);
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
    u[3] = ((u[2] >> 4) & k2) | (((u[1] >> 6) & k3) << 4);
    const uint32_t aux = u[1] & k1;
    u[1] = (u[2] & k2) | (((u[0] >> 6) & k3) << 4);
    u[2] = aux;
    u[0] &= k1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        sc[i] = (u[i / 4] >> (8 * (i % 4))) & 0xFF;
        mn[i] = (u[2 + i / 4] >> (8 * (i % 4))) & 0xFF;
    }
}

// WT: 12 = Q4_K, 14 = Q6_K (GGML type ids).
//
// LDS per 256-value block: the weight values as int8 and the activation
// values, both as 64 dwords per row.  For Q4_K dword 8 j + l holds the four
// values 32 j + 8 g + l (g = 0..3) of sub-block j: the reference's eight
// lanes gather element i into lane i % 8, so one sdot4 per (j, l) gives
// exactly lane l's share of sub-block j.  For Q6_K the 16-value groups are
// summed whole, so the values stay in order.
template <int WT>
__global__ __launch_bounds__(256) void qmm_kernel(const QmmArgs a) {
#pragma clang fp contract(off)
    constexpr bool Q4 = WT == 12;
    constexpr int WB = Q4 ? Q4K_BYTES : Q6K_BYTES;
    // (weight-row arrays padded by one word: a wave's 32 lanes read 32
    // different rows at the same column, which would otherwise share a bank)
    __shared__ uint32_t s_w[TR][65];
    __shared__ uint32_t s_x[TT][64];
    __shared__ int s_sc[TR][17];    // Q4_K: sc[0..7], mn[8..15]; Q6_K: scales[16]
    __shared__ float s_wd[TR][3];   // f16 d (and dmin) of the weight block
    __shared__ float s_xd[TT];      // Q8_K d
    __shared__ int s_bs[TT][16];    // Q8_K bsums

    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * TR, t0 = blockIdx.y * TT;
    const int rg = tid & 31, tg = tid >> 5;
    const int nb = a.cols / QK;
    const uint8_t* W = static_cast<const uint8_t*>(a.w);

    float sums[8][8];  // [output][lane] (Q4_K); Q6_K uses sumf only
    float sumf[8];
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        sumf[o] = 0.0f;
#pragma unroll
        for (int l = 0; l < 8; ++l) sums[o][l] = 0.0f;
    }

    for (int b = 0; b < nb; ++b) {
        __syncthreads();  // the previous block's tiles are consumed
        // ---- stage the weight rows: 4 threads per row, each 1/4 of the block
        {
            const int rr = tid >> 2, part = tid & 3, r = r0 + rr;
            const uint8_t* blk = W + ((size_t)min(r, a.rows - 1) * nb + b) * WB;
            if constexpr (Q4) {
                // qs bytes 32 part .. 32 part + 31 (two 16-byte loads: blocks
                // are 144 bytes, so 16-byte aligned): sub-blocks 2 part (low
                // nibbles) and 2 part + 1 (high nibbles); byte 8 g + l goes to
                // byte g of dword l
                const uint4* q = reinterpret_cast<const uint4*>(blk + 16 + 32 * part);
                const uint4 v0 = q[0], v1 = q[1];
                const uint32_t qd[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    uint32_t lo = 0, hi = 0;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int k = 8 * g + l;
                        const uint32_t byte = (qd[k >> 2] >> (8 * (k & 3))) & 0xFF;
                        lo |= (byte & 0xF) << (8 * g);
                        hi |= (byte >> 4) << (8 * g);
                    }
                    s_w[rr][8 * (2 * part) + l] = lo;
                    s_w[rr][8 * (2 * part + 1) + l] = hi;
                }
                if (part == 0) {
                    const uint4 h = *reinterpret_cast<const uint4*>(blk);  // d, dmin, scales[12]
                    uint8_t hb[16];
                    const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
                    for (int i = 0; i < 16; ++i) hb[i] = (hw[i >> 2] >> (8 * (i & 3))) & 0xFF;
                    uint8_t sc[8], mn[8];
                    q4k_unpack_scales(hb + 4, sc, mn);
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        s_sc[rr][i] = sc[i];
                        s_sc[rr][8 + i] = mn[i];
                    }
                    s_wd[rr][0] = f16_bits_to_f32(h.x & 0xFFFF);
                    s_wd[rr][1] = f16_bits_to_f32(h.x >> 16);
                }
            } else {
                // values 64 part .. 64 part + 63 (src/kernels.rs:135-147):
                // half h = part / 2, quarter q = part % 2 of 32 ql bytes
                const uint8_t* ql = blk + 64 * (part >> 1);
                const uint8_t* qh = blk + 128 + 32 * (part >> 1);
                const int qq = part & 1;  // values 128 h + 64 qq + [0, 64)
#pragma unroll
                for (int k = 0; k < 16; ++k) {  // dword k of the 64 values
                    uint32_t wv = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * k + e;           // 0..63 within the quarter
                        const int sub = i >> 5, l = i & 31;  // 32-value run, index in it
                        const int run = 2 * qq + sub;        // aux8[l + 32 run] of the half
                        int val;
                        if (run == 0) val = (ql[l] & 0xF) | ((qh[l] & 3) << 4);
                        else if (run == 1) val = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
                        else if (run == 2) val = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
                        else val = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
                        wv |= (uint32_t)((val - 32) & 0xFF) << (8 * e);
                    }
                    s_w[rr][16 * part + k] = wv;
                }
                if (part == 0) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) s_sc[rr][i] = (int8_t)blk[192 + i];
                    s_wd[rr][0] = f16_bits_to_f32(blk[208] | (blk[209] << 8));
                }
            }
        }
        // ---- stage the activation rows: 8 threads per row, one sub-block each
        {
            const int tt = tid >> 3, j = tid & 7, t = t0 + tt;
            const Q8KBlock* xb = a.q8 + (size_t)min(t, a.n - 1) * nb + b;
            // sub-block j's 32 values as 8 dword loads (Q8_K blocks are 292
            // bytes: 4-byte aligned)
            const uint32_t* qw = reinterpret_cast<const uint32_t*>(xb->qs + 32 * j);
            uint32_t qd[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) qd[i] = qw[i];
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                uint32_t v = 0;
                if constexpr (Q4) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int k = 8 * g + l;
                        v |= ((qd[k >> 2] >> (8 * (k & 3))) & 0xFF) << (8 * g);
                    }
                } else {
                    v = qd[l];
                }
                s_x[tt][8 * j + l] = v;
            }
            const uint32_t bs = *reinterpret_cast<const uint32_t*>(xb->bsums + 2 * j);
            s_bs[tt][2 * j] = (int16_t)(bs & 0xFFFF);
            s_bs[tt][2 * j + 1] = (int16_t)(bs >> 16);
            if (j == 0) s_xd[tt] = xb->d;
        }
        __syncthreads();

        // ---- this block's contribution to the thread's 8 outputs
        if constexpr (Q4) {
            int aux[8][8];
#pragma unroll
            for (int o = 0; o < 8; ++o)
#pragma unroll
                for (int l = 0; l < 8; ++l) aux[o][l] = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int sc0 = s_sc[2 * rg][j], sc1 = s_sc[2 * rg + 1][j];
                // the sub-block's 64 independent dot4s first, then their
                // scaling (a scaled product right behind its dot4 stalls)
                int p[8][8];
#pragma unroll
                for (int l = 0; l < 8; ++l) {
                    const int w0 = s_w[2 * rg][8 * j + l], w1 = s_w[2 * rg + 1][8 * j + l];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int xv = s_x[4 * tg + k][8 * j + l];
                        p[k][l] = __builtin_amdgcn_sdot4(w0, xv, 0, false);
                        p[4 + k][l] = __builtin_amdgcn_sdot4(w1, xv, 0, false);
                    }
                }
                // (scales <= 63 and |dot4| <= 4 * 15 * 128: exact in the
                // full-rate 24-bit multiply)
#pragma unroll
                for (int o = 0; o < 8; ++o)
#pragma unroll
                    for (int l = 0; l < 8; ++l) aux[o][l] += __mul24(o < 4 ? sc0 : sc1, p[o][l]);
            }
#pragma unroll
            for (int o = 0; o < 8; ++o) {
                const int rr = 2 * rg + (o >> 2), tt = 4 * tg + (o & 3);
                int sumi = 0;
#pragma unroll
                for (int j = 0; j < 16; ++j) sumi += s_bs[tt][j] * s_sc[rr][8 + j / 2];
                const float d = s_wd[rr][0] * s_xd[tt];
#pragma unroll
                for (int l = 0; l < 8; ++l) sums[o][l] += d * (float)aux[o][l];
                const float dmin = s_wd[rr][1] * s_xd[tt];
                sumf[o] -= dmin * (float)sumi;
            }
        } else {
#pragma unroll
            for (int o = 0; o < 8; ++o) {
                const int rr = 2 * rg + (o >> 2), tt = 4 * tg + (o & 3);
                int sumi = 0;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    int p = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) p = __builtin_amdgcn_sdot4(s_w[rr][4 * j + k], s_x[tt][4 * j + k], p, false);
                    sumi += __mul24(s_sc[rr][j], p);  // |scale| <= 128, |p| <= 4 * 32 * 128
                }
                const float d = s_wd[rr][0] * s_xd[tt];
                sumf[o] += d * (float)sumi;
            }
        }
    }

    // ---- write: sumf + (sums[0] + ... + sums[7]) (+ residual)
#pragma unroll
    for (int o = 0; o < 8; ++o) {
        const int r = r0 + 2 * rg + (o >> 2), t = t0 + 4 * tg + (o & 3);
        if (r >= a.rows || t >= a.n) continue;
        float v = sumf[o];
        if constexpr (Q4) {
            float tot = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; ++l) tot += sums[o][l];
            v = v + tot;
        }
        const size_t idx = (size_t)t * a.rows + r;
        if (a.residual) v += a.residual[idx];
        a.out[idx] = v;
    }
}

}  // namespace

hipError_t launch_qmatmul(const QmmArgs& a, hipStream_t st) {
    if (a.n <= 0 || a.rows <= 0) return hipSuccess;
    const int nb = a.cols / QK;
    hipLaunchKernelGGL(q8k_quantize_kernel, dim3((unsigned)(a.n * nb)), dim3(256), 0, st, a.act, a.cols, nb,
                       a.q8);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)((a.rows + TR - 1) / TR), (unsigned)((a.n + TT - 1) / TT));
    if (a.wtype == 12)
        hipLaunchKernelGGL(qmm_kernel<12>, grid, dim3(256), 0, st, a);
    else if (a.wtype == 14)
        hipLaunchKernelGGL(qmm_kernel<14>, grid, dim3(256), 0, st, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace dr
