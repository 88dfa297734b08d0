// qmatmul.hip -- the projection after the attention (Wo, src/model/forward.rs:
// 345-350) on GGUF k-quant weights: native_matmul (src/model/matmul.rs:120-148)
// quantizes the f32 activations to Q8_K (ActScratch::q8k, matmul.rs:64-71) and
// takes, for every (activation row t, weight row r), the Q4_K or Q6_K x Q8_K
// block dot product; residual_add (ops.rs:365-370) follows.
//
// The integer part of every block dot runs on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8).  A block dot is
//   Q4_K:  d_x * (d_w * sum_s sc_s sum_{i in s} q_i x_i  -  dmin_w * sum_s mn_s bsum_s)
//   Q6_K:  d_x *  d_w * sum_s sc_s sum_{i in s} (q_i - 32) x_i
// with 6-bit (Q4_K, sub-blocks of 32) or int8 (Q6_K, sub-blocks of 16)
// scales sc_s.  The scale is folded into the weight operand: sc_s * q_i does
// not fit in int8, so it is split as hi * 2^k + lo with both parts in int8 and
// run as two MFMA chains over the whole 256-value block, aux = (acc_hi << k)
// + acc_lo, exact in int32.  The Q4_K min term is one exact bf16 MFMA per
// block (mn_s <= 63 and the 32-value sums bsum_s split as lo + 64 hi are bf16
// integers; every partial sum stays below 2^24).  Per block and output the f32
// combine is fma(fma(aux, d_w, -dmin_w * mins), d_x, sum).
//
// Numerics: every integer is exact; each output differs from the reference's
// scalar vec_dot (src/kernels.rs:228-347) only in the rounding of the f32
// combine: both are within (nb + 12) * 2^-24 of sum_b (|d aux_b| +
// |dmin sumi_b|) of the exact value, nb = cols / 256.
#include "dr_internal.hpp"

namespace dr {
namespace {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144, Q6K_BYTES = 210;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

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

template <typename T>
__device__ __forceinline__ T gld(const void* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}
// 16 bytes from a 2-byte-aligned address (Q6_K blocks are 210 bytes)
__device__ __forceinline__ u32x4 gld16_a2(const uint8_t* p) {
    const uint8_t* q = static_cast<const uint8_t*>(__builtin_assume_aligned(p, 2));
    u32x4 v;
    __builtin_memcpy(&v, q, 16);
    return v;
}

__device__ __forceinline__ uint32_t pk_mul_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}
__device__ __forceinline__ uint32_t pk_ashr_i16(uint32_t a, int s) {
    const i16x2 v = __builtin_bit_cast(i16x2, a);
    return __builtin_bit_cast(uint32_t, v >> (short)s);
}
// bytes b0 b1 b2 b3 -> the two u16 lanes {b_lo, b_lo + 1} of the pair
__device__ __forceinline__ uint32_t bytes01_u16(uint32_t x) { return __builtin_amdgcn_perm(x, x, 0x0c010c00u); }
__device__ __forceinline__ uint32_t bytes23_u16(uint32_t x) { return __builtin_amdgcn_perm(x, x, 0x0c030c02u); }
// low bytes of the four u16 lanes of (lo, hi) -> one dword
__device__ __forceinline__ uint32_t pack_lo_bytes(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x06040200u);
}
// byte j of x in both u16 lanes
__device__ __forceinline__ uint32_t rep_byte_u16(uint32_t x, int j) {
    const uint32_t b = (x >> (8 * j)) & 0xFFu;
    return b | (b << 16);
}
// bf16 of the small non-negative integers in bytes 0..3 of x, as two dwords
__device__ __forceinline__ void bytes_to_bf16(uint32_t x, uint32_t& lo, uint32_t& hi) {
    const uint32_t f0 = __float_as_uint((float)(x & 0xFFu)), f1 = __float_as_uint((float)((x >> 8) & 0xFFu));
    const uint32_t f2 = __float_as_uint((float)((x >> 16) & 0xFFu)), f3 = __float_as_uint((float)(x >> 24));
    lo = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
    hi = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
}

// ---------------------------------------------------------------------------
// Q8_K quantization (quantize_rows_q8_k, src/kernels.rs:79-122): one
// workgroup per 256-value block, thread i owns value i.  The first value of
// largest magnitude gives iscale = -128 / max; q = round(iscale x) capped at
// 127; d = 1 / iscale.  NaN values never win the scan (amax < |x| is false).
//
// REF = true writes the reference's BlockQ8K (d, qs[256], bsums[16]); REF =
// false writes the matrix-core layout of the workspace (QmmLayout): qs with
// value 32 s + 16 g + j of a block at byte 128 g + 16 s + j, so the 16-value
// operand of lane group g for sub-block s is one 16-byte run and a lane's
// eight runs are one 128-byte line; the 32-value sums as bf16 lo / 64 hi;
// d as [block][row].  Rows n .. n_pad - 1 are written as zeros.
template <bool REF>
__global__ __launch_bounds__(256) void q8k_quantize_kernel(const float* __restrict__ x, int cols, int nb,
                                                           int n, int n_pad, void* __restrict__ out) {
    __shared__ float s_a[4];
    __shared__ int s_i[4];
    __shared__ float s_mx;
    const int blk = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = blk / nb, b = blk - t * nb;
    const float v = t < n ? x[(size_t)t * cols + (size_t)b * QK + tid] : 0.0f;
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
    int q = 0;
    float d = 0.0f;
    if (amax > 0.0f) {
#pragma clang fp contract(off)
        const float iscale = -128.0f / s_mx;
        const float r = fminf(roundf(iscale * v), 127.0f);
        q = (int)r;
        d = 1.0f / iscale;
    }
    if constexpr (REF) {
        Q8KBlock* o = static_cast<Q8KBlock*>(out) + blk;
        if (tid == 0) o->d = d;
        o->qs[tid] = (int8_t)q;
        int s = q;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off);
        if ((tid & 15) == 0) o->bsums[tid >> 4] = (int16_t)s;
    } else {
        const QmmLayout L(out, n_pad, cols);
        // four neighbouring values land in one dword of the permuted block
        const uint32_t q0 = q & 0xFF, q1 = __shfl_down(q, 1) & 0xFF, q2 = __shfl_down(q, 2) & 0xFF,
                       q3 = __shfl_down(q, 3) & 0xFF;
        if ((tid & 3) == 0) {
            const int pos = 128 * ((tid >> 4) & 1) + 16 * (tid >> 5) + (tid & 15);
            *reinterpret_cast<uint32_t*>(L.qs + (size_t)t * cols + (size_t)b * QK + pos) =
                q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
        }
        int s = q;
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) s += __shfl_xor(s, off);
        if ((tid & 31) == 0) {
            const int lo = s & 63, hi = s - lo;  // |s| <= 4096: both exact in bf16
            uint16_t* bm = L.bmin + ((size_t)t * nb + b) * 16;
            bm[tid >> 5] = (uint16_t)(__float_as_uint((float)lo) >> 16);
            bm[8 + (tid >> 5)] = (uint16_t)(__float_as_uint((float)hi) >> 16);
        }
        if (tid == 0) L.xd[(size_t)b * n_pad + t] = d;
    }
}

// ---------------------------------------------------------------------------
// The block dots.  A workgroup owns 32 weight rows x 128 activation rows (four
// 32 x 32 MFMA tiles); its four waves split the 256-value blocks of a row into
// four contiguous ranges and their partial sums meet in LDS in wave order, so
// every output is summed in the same order on every call.
//
// MFMA operands (A = activations: row t; B = weights: column r): lane (c, g),
// c = lane % 32, g = lane / 32, holds values 32 s + 16 g .. + 15 of sub-block
// slab s of row c; accumulator slot i of that lane is output (t = 8 (i / 4) +
// 4 g + i % 4, r = c).
//
// Weight operand of a Q4_K block: slab s = sub-block s.  sc_s = 8 sh + sl with
// sh, sl <= 7, so sh * q and sl * q (q <= 15) are bytes and a 16-bit packed
// multiply scales two nibble bytes at once without carries.  Q6_K: slab s is
// sub-blocks 2 s (g = 0) and 2 s + 1 (g = 1); w = sc * (q - 32) in
// [-4064, 4096] is formed in 16-bit lanes and split as 64 hi + lo.
template <int WT>
struct WeightOps {
    i32x4 hi[8], lo[8];
    bf16x8 mn;        // Q4_K: the eight 6-bit mins
    float wd, wdmin;  // f16 d (and dmin) of the block
};

__device__ __forceinline__ void prep_q4k(const uint8_t* blk, int g, WeightOps<12>& o) {
    const u32x4 h = gld<u32x4>(blk);  // d, dmin, scales[12]
    o.wd = f16_bits_to_f32(h.x & 0xFFFF);
    o.wdmin = f16_bits_to_f32(h.x >> 16);
    // the 12 packed bytes (src/kernels.rs:193-201): sc 0..3, sc 4..7, mn 0..3, mn 4..7
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
    const uint32_t sc03 = h.y & k1, mn03 = h.z & k1;
    const uint32_t sc47 = (h.w & k2) | (((h.y >> 6) & k3) << 4);
    const uint32_t mn47 = ((h.w >> 4) & k2) | (((h.z >> 6) & k3) << 4);
    const uint32_t sh[2] = {(sc03 >> 3) & 0x07070707u, (sc47 >> 3) & 0x07070707u};
    const uint32_t sl[2] = {sc03 & 0x07070707u, sc47 & 0x07070707u};
    uint32_t m0, m1, m2, m3;
    bytes_to_bf16(mn03, m0, m1);
    bytes_to_bf16(mn47, m2, m3);
    o.mn = __builtin_bit_cast(bf16x8, u32x4{m0, m1, m2, m3});
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // qs bytes 32 j + 16 g ..: sub-blocks 2 j (low), 2 j + 1 (high)
        const u32x4 raw = gld<u32x4>(blk + 16 + 32 * j + 16 * g);
#pragma unroll
        for (int hn = 0; hn < 2; ++hn) {
            const int s = 2 * j + hn;
            const uint32_t fh = rep_byte_u16(sh[s >> 2], s & 3), fl = rep_byte_u16(sl[s >> 2], s & 3);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t nib = hn ? (raw[c] >> 4) & 0x0F0F0F0Fu : raw[c] & 0x0F0F0F0Fu;
                o.hi[s][c] = (int)pk_mul_u16(nib, fh);
                o.lo[s][c] = (int)pk_mul_u16(nib, fl);
            }
        }
    }
}

__device__ __forceinline__ void prep_q6k(const uint8_t* blk, int g, WeightOps<14>& o) {
    o.wd = f16_bits_to_f32(blk[208] | (blk[209] << 8));
    o.wdmin = 0.0f;
    const u32x4 scv = gld16_a2(blk + 192);  // int8 scales of the 16 sub-blocks
    u32x4 ql[2][2], qh[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        qh[h] = gld16_a2(blk + 128 + 32 * h + 16 * g);
#pragma unroll
        for (int a = 0; a < 2; ++a) ql[h][a] = gld16_a2(blk + 64 * h + 32 * a + 16 * g);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        // values 128 h + 32 quarter + 16 g + j (src/kernels.rs:135-147)
        const int h = s >> 2, quarter = s & 3, a = quarter & 1;
        const int sb = 2 * s + g;  // sub-block of 16
        const int scb = (int)(int8_t)((scv[sb >> 2] >> (8 * (sb & 3))) & 0xFF);
        const uint32_t f = ((uint32_t)scb & 0xFFFFu) * 0x10001u;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t nib = (quarter >> 1) ? (ql[h][a][c] >> 4) & 0x0F0F0F0Fu : ql[h][a][c] & 0x0F0F0F0Fu;
            const uint32_t q6 = nib | (((qh[h][c] >> (2 * quarter)) & 0x03030303u) << 4);
            const uint32_t w01 = pk_mul_u16(pk_sub_u16(bytes01_u16(q6), 0x00200020u), f);
            const uint32_t w23 = pk_mul_u16(pk_sub_u16(bytes23_u16(q6), 0x00200020u), f);
            o.hi[s][c] = (int)pack_lo_bytes(pk_ashr_i16(w01, 6), pk_ashr_i16(w23, 6));
            o.lo[s][c] = (int)pack_lo_bytes(w01 & 0x003F003Fu, w23 & 0x003F003Fu);
        }
    }
}

template <int WT>
__global__ __launch_bounds__(256) void qmm_kernel(const QmmArgs a) {
    constexpr bool Q4 = WT == 12;
    constexpr int WB = Q4 ? Q4K_BYTES : Q6K_BYTES;
    constexpr int SHIFT = Q4 ? 3 : 6;
    // partial sums of the three other waves for each wave's tile:
    // [tile][source wave, own skipped][slot][lane]
    __shared__ float s_part[4][3][16][64];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, g = lane >> 5;
    const int nb = a.cols / QK;
    const int n_rt = (a.rows + 31) / 32, n_tt = a.n_pad / 128;
    const int nwg = n_rt * n_tt, hw = blockIdx.x;
    // the 128-row tiles of one weight tile on one XCD: the weights (the larger
    // operand) are read into each XCD's L2 once
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int rt = lid / n_tt, tt = lid - rt * n_tt;
    const int r = min(rt * 32 + col, a.rows - 1);
    const int t0 = tt * 128;
    const QmmLayout L(a.ws, a.n_pad, a.cols);
    const uint8_t* wrow = static_cast<const uint8_t*>(a.w) + (size_t)r * nb * WB;

    f32x16 sum[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) sum[c][i] = 0.0f;

    const int b_begin = wave * nb / 4, b_end = (wave + 1) * nb / 4;
    for (int b = b_begin; b < b_end; ++b) {
        WeightOps<WT> wo;
        if constexpr (Q4)
            prep_q4k(wrow + (size_t)b * WB, g, wo);
        else
            prep_q6k(wrow + (size_t)b * WB, g, wo);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int tr = t0 + 32 * c + col;  // this lane's A row
            const int8_t* ap = L.qs + (size_t)tr * a.cols + (size_t)b * QK + 128 * g;
            i32x4 av[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) av[s] = gld<i32x4>(ap + 16 * s);
            f32x4 xd[4];
            const float* xp = L.xd + (size_t)b * a.n_pad + t0 + 32 * c + 4 * g;
#pragma unroll
            for (int k = 0; k < 4; ++k) xd[k] = gld<f32x4>(xp + 8 * k);
            i32x16 ah = {}, al = {};
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                ah = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[s], wo.hi[s], ah, 0, 0, 0);
                al = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[s], wo.lo[s], al, 0, 0, 0);
            }
            f32x16 mins = {};
            if constexpr (Q4) {
                const bf16x8 bm = gld<bf16x8>(L.bmin + ((size_t)tr * nb + b) * 16 + 8 * g);
                f32x16 z;
#pragma unroll
                for (int i = 0; i < 16; ++i) z[i] = 0.0f;
                mins = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bm, wo.mn, z, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float f = (float)(ah[i] * (1 << SHIFT) + al[i]);
                const float inner = Q4 ? __builtin_fmaf(f, wo.wd, -(mins[i] * wo.wdmin)) : f * wo.wd;
                sum[c][i] = __builtin_fmaf(inner, xd[i >> 2][i & 3], sum[c][i]);
            }
        }
    }

    // ---- the four partial sums of each tile, in wave order; wave w writes tile w
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c == wave) continue;
        const int src = wave < c ? wave : wave - 1;
#pragma unroll
        for (int i = 0; i < 16; ++i) s_part[c][src][i][lane] = sum[c][i];
    }
    __syncthreads();
    const int c = wave;
    f32x16 own;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
        if (cc == c) own = sum[cc];
    const int rr = rt * 32 + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float p = w == c ? own[i] : s_part[c][w < c ? w : (w > c ? w - 1 : 0)][i][lane];
            v = w == 0 ? p : v + p;
        }
        const int t = t0 + 32 * c + 8 * (i >> 2) + 4 * g + (i & 3);
        if (t < a.n && rr < a.rows) {
            const size_t idx = (size_t)t * a.rows + rr;
            if (a.residual) v += a.residual[idx];
            a.out[idx] = v;
        }
    }
}

}  // namespace

size_t qmm_workspace_bytes(int n, int cols) {
    const size_t n_pad = (size_t)qmm_rows_padded(n), nb = (size_t)cols / QK;
    return n_pad * nb * (QK + 16 * sizeof(uint16_t) + sizeof(float));
}

hipError_t launch_qmatmul(const QmmArgs& a, hipStream_t st) {
    if (a.n <= 0 || a.rows <= 0) return hipSuccess;
    if (a.n_pad != qmm_rows_padded(a.n) || a.cols % QK != 0) return hipErrorInvalidValue;
    const int nb = a.cols / QK;
    hipLaunchKernelGGL(q8k_quantize_kernel<false>, dim3((unsigned)(a.n_pad * nb)), dim3(256), 0, st, a.act,
                       a.cols, nb, a.n, a.n_pad, a.ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned nwg = (unsigned)(((a.rows + 31) / 32) * (a.n_pad / 128));
    if (a.wtype == 12)
        hipLaunchKernelGGL(qmm_kernel<12>, dim3(nwg), dim3(256), 0, st, a);
    else if (a.wtype == 14)
        hipLaunchKernelGGL(qmm_kernel<14>, dim3(nwg), dim3(256), 0, st, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_quantize_q8k(const float* act, int n, int cols, Q8KBlock* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int nb = cols / QK;
    hipLaunchKernelGGL(q8k_quantize_kernel<true>, dim3((unsigned)(n * nb)), dim3(256), 0, st, act, cols, nb, n,
                       n, static_cast<void*>(out));
    return hipGetLastError();
}

}  // namespace dr
