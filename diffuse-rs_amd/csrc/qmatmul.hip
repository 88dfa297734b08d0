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
// integers; every partial sum stays below 2^24).  The block scales d = d_x d_w
// and dmin = d_x dmin_w of every output come out of a K = 2 f32 MFMA in the
// accumulator layout, each one rounded product as in the reference; per
// block and output the combine is sum = fma(-dmin, mins, fma(d, aux, sum)).
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

// A workgroup barrier that waits only for this wave's LDS operations (the
// global loads in flight stay in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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
// Q8_K quantization (quantize_rows_q8_k, src/kernels.rs:79-122): one wave per
// 256-value block (four per workgroup), lane l owns values 4 l .. 4 l + 3.
// The first value of largest magnitude gives iscale = -128 / max; q =
// round(iscale x) capped at 127; d = 1 / iscale.  NaN values never win the
// scan (amax < |x| is false).  Only max's sign needs the first index: the
// magnitude is a wave maximum, the first holder a ballot.
//
// REF = true writes the reference's BlockQ8K (d, qs[256], bsums[16]); REF =
// false writes the matrix-core operand order of the workspace (QmmLayout).
// Rows n .. n_pad - 1 are written as zeros.
// DPP steps of the wave reductions below (gfx9 row / quad patterns).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// Maximum over the wave, in lane 63 and broadcast through a scalar.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));        // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_f<0x4E>(v));        // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_f<0x141>(v));       // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));       // row_mirror: every lane holds its row's maximum
    v = fmaxf(v, dpp_f<0x142, 0xA>(v));  // row_bcast:15 into rows 1 and 3
    v = fmaxf(v, dpp_f<0x143, 0xC>(v));  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Quantizes the 256 values of one row-block held by a wave (lane l: values
// 4 l .. 4 l + 3): q (four values), d, and the lane's share of the sums.
struct RowQ {
    uint32_t packed;  // the lane's four q as bytes
    int sum4;         // their sum
    float d;
};
__device__ __forceinline__ RowQ quantize_row_block(const f32x4 v) {
    // the largest |x| (a NaN never wins: it counts as -1), then the first
    // value that has it: the lowest lane holding one, its first element
    float ae[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) ae[e] = v[e] != v[e] ? -1.0f : fabsf(v[e]);
    const float amax = wave_max(fmaxf(fmaxf(ae[0], ae[1]), fmaxf(ae[2], ae[3])));
    const float mine = ae[0] == amax ? v[0] : ae[1] == amax ? v[1] : ae[2] == amax ? v[2] : v[3];
    const unsigned long long hit = __ballot(ae[0] == amax || ae[1] == amax || ae[2] == amax || ae[3] == amax);
    const int first = hit ? (int)__builtin_ctzll(hit) : 0;
    const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), first));
    int q[4] = {0, 0, 0, 0};
    RowQ o;
    o.d = 0.0f;
    if (amax > 0.0f) {
#pragma clang fp contract(off)
        const float iscale = -128.0f / mx;
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = (int)fminf(roundf(iscale * v[e]), 127.0f);
        o.d = 1.0f / iscale;
    }
    o.packed = (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | ((uint32_t)q[3] << 24);
    o.sum4 = q[0] + q[1] + q[2] + q[3];
    return o;
}

// The reference's BlockQ8K (d, qs[256], bsums[16]): one wave per block, four
// per workgroup.
__global__ __launch_bounds__(256) void q8k_quantize_ref_kernel(const float* __restrict__ x, int cols, int nb, int n,
                                                               Q8KBlock* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= n * nb) return;  // (no barriers below: a whole wave leaves)
    const int t = blk / nb, b = blk - t * nb;
    const RowQ rq = quantize_row_block(gld<f32x4>(x + (size_t)t * cols + (size_t)b * QK + 4 * lane));
    Q8KBlock* o = out + blk;
    if (lane == 0) o->d = rq.d;
    *reinterpret_cast<uint32_t*>(o->qs + 4 * lane) = rq.packed;
    int s = rq.sum4;
    s += dpp_i<0xB1>(s);  // the quad: 16 values
    s += dpp_i<0x4E>(s);
    if ((lane & 3) == 0) o->bsums[lane >> 2] = (int16_t)s;
}

// The matrix-core operand order of the workspace (QmmLayout): one workgroup
// (8 waves) per 32-row tile and block, wave w quantizes rows 4 w .. 4 w + 3.
// The tile's operands are assembled in LDS and leave as whole 16-byte runs
// (8 KB of qs, 1 KB of min operands, 128 bytes of d).  Rows n .. n_pad - 1
// are written as zeros.
__global__ __launch_bounds__(512) void q8k_quantize_tiles_kernel(const float* __restrict__ x, int cols, int nb,
                                                                 int n, int n_pad, void* __restrict__ ws) {
    // qs chunks [slab * 2 + g][33, one pad][16 bytes]: the 16 lane quads of a
    // row write distinct banks
    __shared__ __attribute__((aligned(16))) uint32_t s_q[16 * 33 * 4];
    __shared__ __attribute__((aligned(16))) uint16_t s_bm[64 * 8];
    __shared__ __attribute__((aligned(16))) float s_xd[32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t32 = blockIdx.x / nb, b = blockIdx.x - t32 * nb;
    // every load unconditional (rows past n read row n - 1, then count as
    // zeros): a load behind a branch made the compiler wait for the loads
    // before it, two round trips instead of one
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int t = t32 * 32 + 4 * wave + k;
        v[k] = gld<f32x4>(x + (size_t)min(t, n - 1) * cols + (size_t)b * QK + 4 * lane);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (t32 * 32 + 4 * wave + k >= n) v[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int c = 4 * wave + k;
        const RowQ rq = quantize_row_block(v[k]);
        // values 4 lane .. + 3: slab lane / 8, lane group (lane / 4) % 2
        s_q[((lane >> 2) * 33 + c) * 4 + (lane & 3)] = rq.packed;
        int s = rq.sum4;
        s += dpp_i<0xB1>(s);   // the quad
        s += dpp_i<0x4E>(s);
        s += dpp_i<0x141>(s);  // and its half row: 32 values
        if ((lane & 7) == 0) {
            const int lo = s & 63, hi = s - lo;  // |s| <= 4096: both exact in bf16
            s_bm[c * 8 + (lane >> 3)] = (uint16_t)(__float_as_uint((float)lo) >> 16);
            s_bm[(32 + c) * 8 + (lane >> 3)] = (uint16_t)(__float_as_uint((float)hi) >> 16);
        }
        if (lane == 0) s_xd[c] = rq.d;
    }
    __syncthreads();
    const QmmLayout L(ws, n_pad, cols);
    const size_t tb = L.tb(t32, b);
    const int q = threadIdx.x;  // chunk (slab * 2 + g) * 32 + row of the tile's 8 KB
    *reinterpret_cast<u32x4*>(L.qs + tb * 8192 + (size_t)q * 16) =
        *reinterpret_cast<const u32x4*>(&s_q[((q >> 5) * 33 + (q & 31)) * 4]);
    if (q < 64)
        *reinterpret_cast<u32x4*>(L.bmin + (tb * 64 + q) * 8) = *reinterpret_cast<const u32x4*>(&s_bm[q * 8]);
    else if (q < 72)
        *reinterpret_cast<f32x4*>(L.xd + tb * 32 + 4 * (q - 64)) = *reinterpret_cast<const f32x4*>(&s_xd[4 * (q - 64)]);
}

// ---------------------------------------------------------------------------
// The block dots.  A workgroup (8 waves, two per SIMD) owns 32 weight rows x
// 128 activation rows: wave w computes the 32 x 32 MFMA tile c = w % 4 over
// half h = w / 4 of the 256-value blocks of a row (the two halves' partial
// sums meet in LDS, so every output is summed in one fixed order).  The
// weight operands of a block are formed once per workgroup: each wave of a
// half converts two of the eight sub-block slabs of its half's block into
// LDS, double-buffered, one block ahead of the MFMAs; one barrier per block.
//
// MFMA operands (A = activations: row t; B = weights: column r): lane (c, g),
// c = lane % 32, g = lane / 32, holds values 32 s + 16 g .. + 15 of sub-block
// slab s of row c; accumulator slot i of that lane is output (t = 8 (i / 4) +
// 4 g + i % 4, r = c).
//
// Weight operand of a Q4_K block: slab s = sub-block s.  sc_s = 8 sh + sl with
// sh, sl <= 7, so sh * q and sl * q (q <= 15) are bytes and a 16-bit packed
// multiply scales two nibble bytes at once without carries; the two parts
// run as one accumulator chain: acc = 8 * (A . hi) + A . lo.  Q6_K: slab s is
// sub-blocks 2 s (g = 0) and 2 s + 1 (g = 1); w = sc * (q - 32) in
// [-4064, 4096] is formed in 16-bit lanes and split as 64 hi + lo.

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    // exact for every finite and infinite f16 (src/kernels.rs:46-69); a NaN
    // stays a NaN
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// The raw bytes a wave needs of one block: the 16-byte Q4_K header (d, dmin,
// scales) and the 16 qs bytes of its two slabs; for Q6_K the scales, the ql
// and qh runs of its two slabs, and d.
template <int WT>
struct RawBlock;
template <>
struct RawBlock<12> {
    u32x4 h, q;
};
template <>
struct RawBlock<14> {
    u32x4 sc, ql[2], qh;
    uint32_t d;
};

// slabs 2 c and 2 c + 1 of a Q4_K block: qs bytes 32 c + 16 g .. + 15
__device__ __forceinline__ void load_raw(const uint8_t* blk, int c, int g, RawBlock<12>& r) {
    r.h = gld<u32x4>(blk);
    r.q = gld<u32x4>(blk + 16 + 32 * c + 16 * g);
}
// slabs 2 c, 2 c + 1 of a Q6_K block: half c / 2, quarters 2 (c % 2), + 1
// (src/kernels.rs:135-147): ql runs 64 h + 32 a + 16 g, qh run 32 h + 16 g
__device__ __forceinline__ void load_raw(const uint8_t* blk, int c, int g, RawBlock<14>& r) {
    const int h = c >> 1;
    r.sc = gld16_a2(blk + 192);
    r.ql[0] = gld16_a2(blk + 64 * h + 16 * g);
    r.ql[1] = gld16_a2(blk + 64 * h + 32 + 16 * g);
    r.qh = gld16_a2(blk + 128 + 32 * h + 16 * g);
    r.d = gld<uint16_t>(blk + 208);
}

// What the combine of a block needs besides the MFMA results.
struct BlockScale {
    float wd, wdmin;
    bf16x8 mn;  // Q4_K: the eight 6-bit mins (B operand of the min MFMA)
};

// Scales of a block, and this wave's two slabs of B operands into LDS
// (dst[slab][hi / lo][lane]).
__device__ __forceinline__ void prep(const RawBlock<12>& r, int c, int lane, u32x4* dst, BlockScale& o) {
    const u32x4 h = r.h;
    o.wd = f16_to_f32(h.x & 0xFFFF);
    o.wdmin = f16_to_f32(h.x >> 16);
    // the 12 packed bytes (src/kernels.rs:193-201): sc 0..3, sc 4..7, mn 0..3, mn 4..7
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
    const uint32_t sc03 = h.y & k1, mn03 = h.z & k1;
    const uint32_t sc47 = (h.w & k2) | (((h.y >> 6) & k3) << 4);
    const uint32_t mn47 = ((h.w >> 4) & k2) | (((h.z >> 6) & k3) << 4);
    uint32_t m0, m1, m2, m3;
    bytes_to_bf16(mn03, m0, m1);
    bytes_to_bf16(mn47, m2, m3);
    o.mn = __builtin_bit_cast(bf16x8, u32x4{m0, m1, m2, m3});
    const uint32_t sc = c < 2 ? sc03 : sc47;  // bytes 2 c % 4, 2 c % 4 + 1
    const uint32_t sh = (sc >> 3) & 0x07070707u, sl = sc & 0x07070707u;
#pragma unroll
    for (int hn = 0; hn < 2; ++hn) {  // low nibbles: slab 2 c; high: 2 c + 1
        const int byte = 2 * (c & 1) + hn;
        const uint32_t fh = rep_byte_u16(sh, byte), fl = rep_byte_u16(sl, byte);
        u32x4 vh, vl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t nib = hn ? (r.q[k] >> 4) & 0x0F0F0F0Fu : r.q[k] & 0x0F0F0F0Fu;
            vh[k] = pk_mul_u16(nib, fh);
            vl[k] = pk_mul_u16(nib, fl);
        }
        dst[((2 * c + hn) * 2 + 0) * 64 + lane] = vh;
        dst[((2 * c + hn) * 2 + 1) * 64 + lane] = vl;
    }
}

__device__ __forceinline__ void prep(const RawBlock<14>& r, int c, int lane, u32x4* dst, BlockScale& o) {
    o.wd = f16_to_f32(r.d);
    o.wdmin = 0.0f;
    const int g = lane >> 5;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
        const int s = 2 * c + k2;
        const int quarter = s & 3;        // ql run a = quarter & 1, nibble quarter >> 1
        const int sb = 2 * s + g;         // sub-block of 16
        // (selects, not indexing: the indices differ between waves)
        const uint32_t scw = (sb >> 2) == 0 ? r.sc.x : (sb >> 2) == 1 ? r.sc.y : (sb >> 2) == 2 ? r.sc.z : r.sc.w;
        const int scb = (int)(int8_t)((scw >> (8 * (sb & 3))) & 0xFF);
        const uint32_t f = ((uint32_t)scb & 0xFFFFu) * 0x10001u;
        const u32x4 qrun = (quarter & 1) ? r.ql[1] : r.ql[0];
        const int nshift = (quarter >> 1) * 4;
        u32x4 vh, vl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t nib = (qrun[k] >> nshift) & 0x0F0F0F0Fu;
            const uint32_t q6 = nib | (((r.qh[k] >> (2 * quarter)) & 0x03030303u) << 4);
            const uint32_t w01 = pk_mul_u16(pk_sub_u16(bytes01_u16(q6), 0x00200020u), f);
            const uint32_t w23 = pk_mul_u16(pk_sub_u16(bytes23_u16(q6), 0x00200020u), f);
            vh[k] = pack_lo_bytes(pk_ashr_i16(w01, 6), pk_ashr_i16(w23, 6));
            vl[k] = pack_lo_bytes(w01 & 0x003F003Fu, w23 & 0x003F003Fu);
        }
        dst[(s * 2 + 0) * 64 + lane] = vh;
        dst[(s * 2 + 1) * 64 + lane] = vl;
    }
}

// The residual of a lane's 16 outputs (activation rows t0 + 8 (i / 4) + 4 g
// + i % 4, weight row rr), every index clamped in bounds so that all 16
// loads are in flight together: a load behind a per-lane bounds check would
// be waited for before the next one issues.
__device__ __forceinline__ void load_residual(const QmmArgs& a, int t0, int g, int rr, float (&rv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) rv[i] = 0.0f;
    if (!a.residual) return;
    const int rc = min(rr, a.rows - 1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = min(t0 + 8 * (i >> 2) + 4 * g + (i & 3), a.n - 1);
        rv[i] = gld<float>(a.residual + (size_t)t * a.rows + rc);
    }
}
// out[t][rr] = sum (+ residual) for the lane's outputs inside the problem.
__device__ __forceinline__ void store_tile(const QmmArgs& a, int t0, int g, int rr, const f32x16& sum,
                                           const float (&rv)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = t0 + 8 * (i >> 2) + 4 * g + (i & 3);
        float v = sum[i];
        if (a.residual) v += rv[i];
        if (t < a.n && rr < a.rows) a.out[(size_t)t * a.rows + rr] = v;
    }
}

template <int WT>
__global__ __launch_bounds__(512) void qmm_kernel(const QmmArgs a) {
    constexpr bool Q4 = WT == 12;
    constexpr int WB = Q4 ? Q4K_BYTES : Q6K_BYTES;
    constexpr int SHIFT = Q4 ? 3 : 6;
    // B operands [buffer][half][slab][hi / lo][lane] (64 KB); after the loop
    // the first 16 KB carry half 1's partial sums [tile][slot][lane]
    __shared__ u32x4 s_b[2][2][8][2][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // (uniform: scalar branches)
    const int c = wave & 3, kh = wave >> 2;
    const int nb = a.cols / QK;
    const int n_rt = (a.rows + 31) / 32, n_tt = a.n_pad / 128;
    const int nwg = n_rt * n_tt, hw = blockIdx.x;
    // the 128-row tiles of one weight tile on one XCD: the weights (the larger
    // operand) are read into each XCD's L2 once
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int rt = lid / n_tt, tt = lid - rt * n_tt;
    const int col = lane & 31, g = lane >> 5;
    const int r = min(rt * 32 + col, a.rows - 1);
    const int tc = tt * 128 + 32 * c;  // first row of this wave's tile
    const QmmLayout L(a.ws, a.n_pad, a.cols);
    const uint8_t* wrow = static_cast<const uint8_t*>(a.w) + (size_t)r * nb * WB;

    const int nh = (nb + 1) / 2;                 // iterations (blocks of half 0)
    const int kb0 = kh ? nh : 0, kcnt = kh ? nb - nh : nh;
    const int8_t* abase = L.qs + (size_t)(tc >> 5) * nb * 8 * 1024 + lane * 16;
    const float* xbase = L.xd + (size_t)(tc >> 5) * nb * 32 + col;
    const uint16_t* mbase = L.bmin + ((size_t)(tc >> 5) * nb * 64 + lane) * 8;

    f32x16 sum;
#pragma unroll
    for (int i = 0; i < 16; ++i) sum[i] = 0.0f;

    // Per block: the A operands, the rows' Q8_K d and the min operand.  Two
    // sets (the block being multiplied, the next one) and two raw weight sets
    // (the block being formed into LDS, the one after), used alternately by
    // an unrolled pair of iterations, so nothing is copied between registers.
    // Prefetches past the wave's last block reload that block (in bounds,
    // unused): no load sits behind a branch.
    struct Stage {
        i32x4 av[8];
        float xd;  // lane (c, 0): the Q8_K d of row c (A operand of the scale MFMAs)
        bf16x8 bm;
    };
    Stage S[2];
    RawBlock<WT> R[2];
    BlockScale bsc;
    const int blast = kb0 + (kcnt > 0 ? kcnt - 1 : 0);
    auto load_stage = [&](int b, Stage& st) __attribute__((always_inline)) {
        // (in order of need: loads complete in issue order)
#pragma unroll
        for (int s = 0; s < 8; ++s) st.av[s] = gld<i32x4>(abase + ((size_t)b * 8 + s) * 1024);
        st.xd = gld<float>(xbase + (size_t)b * 32);
        if constexpr (Q4) st.bm = gld<bf16x8>(mbase + (size_t)b * 64 * 8);
    };
    // The combine of a block runs in the next iteration, under that block's
    // MFMA chains: the products of the previous block wait in registers.
    struct Products {
        i32x16 acc;
        f32x16 mins, dd, dm;
    };
    Products P;
    bool pending = false;  // P holds a block not yet added into sum (uniform)
    auto combine = [&](const Products& pr) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sum[i] = __builtin_fmaf(pr.dd[i], (float)pr.acc[i], sum[i]);
            if constexpr (Q4) sum[i] = __builtin_fmaf(-pr.dm[i], pr.mins[i], sum[i]);
        }
    };
    auto body = [&](int it, Stage& cur, Stage& nxt, RawBlock<WT>& rprep, RawBlock<WT>& rload, int buf)
        __attribute__((always_inline)) {
        if (it < kcnt) {
            load_stage(min(kb0 + it + 1, blast), nxt);
            load_raw(wrow + (size_t)min(kb0 + it + 2, blast) * WB, c, g, rload);
            // (the scheduler would otherwise sink the prefetches to their use)
            __builtin_amdgcn_sched_barrier(0);
            // ---- MFMAs of this block: acc = 2^SHIFT (A . hi) + A . lo
            const u32x4* bsrc = &s_b[buf][kh][0][0][lane];
            Products np;
            i32x16 acc = {};
#pragma unroll
            for (int s = 0; s < 8; ++s)
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.av[s], __builtin_bit_cast(i32x4, bsrc[(s * 2) * 64]),
                                                            acc, 0, 0, 0);
            // ---- under the first chain: the previous block's combine
            if (pending) combine(P);
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] *= (1 << SHIFT);
#pragma unroll
            for (int s = 0; s < 8; ++s)
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                    cur.av[s], __builtin_bit_cast(i32x4, bsrc[(s * 2 + 1) * 64]), acc, 0, 0, 0);
            np.acc = acc;
            np.mins = f32x16{};
            if constexpr (Q4) np.mins = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.bm, bsc.mn, np.mins, 0, 0, 0);
            // the block scales d_x d_w (and d_x dmin_w) of every slot, each one
            // f32 product, on a K = 2 f32 MFMA with the second K row zero
            const float xa = g == 0 ? cur.xd : 0.0f;
            const f32x16 z = {};
            np.dd = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, g == 0 ? bsc.wd : 0.0f, z, 0, 0, 0);
            np.dm = f32x16{};
            if constexpr (Q4) np.dm = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, g == 0 ? bsc.wdmin : 0.0f, z, 0, 0, 0);
            // ---- under the second chain: the next block's B operands into the
            // other buffer (past the last block: a repeat nobody reads)
            prep(rprep, c, lane, &s_b[buf ^ 1][kh][0][0][0], bsc);
            P = np;
            pending = true;
        }
        lds_barrier();
    };
    if (kcnt > 0) {
        RawBlock<WT> raw0;
        load_raw(wrow + (size_t)kb0 * WB, c, g, raw0);
        load_stage(kb0, S[0]);
        load_raw(wrow + (size_t)min(kb0 + 1, blast) * WB, c, g, R[1]);
        prep(raw0, c, lane, &s_b[0][kh][0][0][0], bsc);
    }
    lds_barrier();
    int it = 0;
    for (; it + 1 < nh; it += 2) {
        body(it, S[0], S[1], R[1], R[0], 0);
        body(it + 1, S[1], S[0], R[0], R[1], 1);
    }
    if (it < nh) body(it, S[0], S[1], R[1], R[0], 0);
    const int rr = rt * 32 + col;
    float rv[16];
    if (kh == 0) load_residual(a, tc, g, rr, rv);
    if (pending) combine(P);

    // ---- half 1's partial sums to LDS; half 0 adds them (and the residual)
    float* red = reinterpret_cast<float*>(&s_b[0][0][0][0][0]);
    if (kh == 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) red[(c * 16 + i) * 64 + lane] = sum[i];
    }
    lds_barrier();
    if (kh == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sum[i] = sum[i] + red[(c * 16 + i) * 64 + lane];
        store_tile(a, tc, g, rr, sum, rv);
    }
}

// ---------------------------------------------------------------------------
// The legacy 32-value block types: Q4_0, Q5_0 and Q8_0 weights over Q8_0
// activations (MatWeight::Q40 and ExpertMat::{Q40, Q50, Q80},
// src/model/matmul.rs:103-106, 192-194; ActScratch::q80, :73-82).  A block
// dot is d_w * d_a * sumi with sumi = sum_j w_j a_j over 32 int8 values, so
// one v_mfma_i32_32x32x32_i8 per block gives the exact sumi of a 32 x 32
// (activation row x weight row) tile, and a K = 2 f32 MFMA the d_w d_a of
// every slot (each one f32 product); the combine is sum = fma(sumi, d, sum)
// in block order.  Every integer is exact, so each output is within
// (nb + 12) * 2^-24 * sum_i |w_i a_i| of the exact dot, as the reference's
// own f32 accumulation is (nb = cols / 32).

// quantize_row_q8_0 (candle-core 0.8.4 BlockQ8_0::from_float, ggml's
// reference): per 32 values of a row, amax = max |x| (a NaN never wins), d =
// amax / 127, id = d != 0 ? 1 / d : 0 (IEEE divisions, as the reference's),
// q = round(x * id) half away from zero, saturated to int8; the block's scale
// is f16(d), round to nearest even.  One wave per (32-row tile, block): lane
// (c, g) holds values 16 g .. 16 g + 15 of row c.  REF = false writes the
// operand order of the workspace (Q0Layout), REF = true the reference's
// BlockQ8_0 (34 bytes: f16 d, int8 qs[32]).  Rows n .. n_pad - 1 are zeros.
template <bool REF>
__global__ __launch_bounds__(256) void q80_quantize_kernel(const float* __restrict__ x, int cols, int nb, int n,
                                                           int n_pad, void* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);  // (tile, block)
    if (item >= (n_pad / 32) * nb) return;  // (no barrier below: a whole wave leaves)
    const int t32 = item / nb, b = item - t32 * nb;
    const int c = lane & 31, g = lane >> 5;
    const int t = t32 * 32 + c;
    // (unconditional loads, as in q8k_quantize_tiles_kernel)
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = gld<f32x4>(x + (size_t)min(t, n - 1) * cols + (size_t)b * 32 + 16 * g + 4 * k);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (t >= n) v[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) am = fmaxf(am, fabsf(v[k][e]));
    am = fmaxf(am, __shfl_xor(am, 32));
    float d, id;
    {
#pragma clang fp contract(off)
        d = am / 127.0f;
        id = d != 0.0f ? 1.0f / d : 0.0f;
    }
    uint32_t pk[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float q;
            {
#pragma clang fp contract(off)
                q = roundf(v[k][e] * id);
            }
            q = q != q ? 0.0f : fminf(fmaxf(q, -128.0f), 127.0f);
            w |= ((uint32_t)(int)q & 0xFFu) << (8 * e);
        }
        pk[k] = w;
    }
    const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16)d);
    if constexpr (REF) {
        if (t >= n) return;
        uint8_t* blk = static_cast<uint8_t*>(out) + ((size_t)t * nb + b) * 34;
        if (g == 0) *reinterpret_cast<uint16_t*>(blk) = dh;
        uint16_t* q16 = reinterpret_cast<uint16_t*>(blk + 2 + 16 * g);  // (2-byte aligned)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            q16[2 * k] = (uint16_t)(pk[k] & 0xFFFFu);
            q16[2 * k + 1] = (uint16_t)(pk[k] >> 16);
        }
    } else {
        const Q0Layout L(out, n_pad, cols);
        const size_t tb = (size_t)t32 * nb + b;
        *reinterpret_cast<u32x4*>(L.qs + (tb * 64 + lane) * 16) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        if (g == 0) L.xd[tb * 32 + c] = (float)__builtin_bit_cast(_Float16, dh);
    }
}

// A signed int8 in each byte of x (each in [0, 255 - off]) minus off, without
// carries between bytes: (x + 128 - off) stays in 0..255, then flip bit 7.
__device__ __forceinline__ uint32_t bytes_minus(uint32_t x, uint32_t off4) {
    return ((x | 0x80808080u) - off4) ^ 0x80808080u;
}
// bits 0..3 of b to bit 4 of bytes 0..3
__device__ __forceinline__ uint32_t bits_to_byte_bit4(uint32_t b) { return ((b * 0x00204081u) & 0x01010101u) << 4; }

// The raw bytes of one legacy block that lane (c, g) needs: the f16 d, the
// 16 value bytes of its half (Q8_0), or the 16 nibble bytes (Q4_0, Q5_0)
// and the 32 high bits (Q5_0).
template <int WT>
struct LegacyRaw {
    u32x4 q;
    uint32_t dh, qh;
};
template <int WT>
__device__ __forceinline__ void load_legacy(const uint8_t* blk, int g, LegacyRaw<WT>& r) {
    r.dh = gld<uint16_t>(blk);
    if constexpr (WT == 8) {
        r.q = gld16_a2(blk + 2 + 16 * g);
        r.qh = 0;
    } else if constexpr (WT == 2) {
        r.q = gld16_a2(blk + 2);
        r.qh = 0;
    } else {
        r.qh = (uint32_t)gld<uint16_t>(blk + 2) | ((uint32_t)gld<uint16_t>(blk + 4) << 16);
        r.q = gld16_a2(blk + 6);
    }
}
// The weight operand of lane (c, g): values 16 g .. 16 g + 15 of the block
// as int8 (Q8_0: the bytes; Q4_0: nibble of byte j % 16 (high for j >= 16)
// - 8; Q5_0: that nibble | bit j of qh << 4, - 16).
template <int WT>
__device__ __forceinline__ i32x4 legacy_operand(const LegacyRaw<WT>& r, int g) {
    if constexpr (WT == 8) {
        return __builtin_bit_cast(i32x4, r.q);
    } else if constexpr (WT == 2) {
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = bytes_minus((g ? r.q[k] >> 4 : r.q[k]) & 0x0F0F0F0Fu, 0x08080808u);
        return __builtin_bit_cast(i32x4, o);
    } else {
        static_assert(WT == 6, "legacy weight type");
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t nib = (g ? r.q[k] >> 4 : r.q[k]) & 0x0F0F0F0Fu;
            const uint32_t hi = bits_to_byte_bit4((r.qh >> (16 * g + 4 * k)) & 0xFu);
            o[k] = bytes_minus(nib | hi, 0x10101010u);
        }
        return __builtin_bit_cast(i32x4, o);
    }
}

// A workgroup (8 waves, two per SIMD) owns 32 weight rows x 128 activation
// rows: wave w the 32 x 32 tile of activation rows 32 (w % 4) .. + 31 over
// half w / 4 of the blocks (the halves' partial sums meet in LDS, so every
// output is summed in one fixed order).  Lane (c, g): weight row c of the
// tile (B operand) and activation row c (A operand), values 16 g .. 16 g +
// 15 of each block; accumulator slot i is output (activation row 8 (i / 4) +
// 4 g + i % 4, weight row c).
//
// The four waves of a half need the same weight operands.  Loaded by each
// wave, 16 bytes per lane from 32 rows a row apart, they kept the texture
// address unit busy for almost the whole kernel; so the blocks go in groups
// of QG: wave w % 4 of a half loads block w % 4 of the next group and forms
// its operand (and d) into LDS, double-buffered, one barrier per group, and
// every wave reads its operands from there.  Each wave keeps the activation
// operands of its next QG blocks in flight (a ring of registers, unrolled so
// that nothing is copied and every wait counts only the loads it needs), and
// a block's combine runs after the next block's MFMAs are issued.
constexpr int QG = 4;
template <int WT>
__global__ __launch_bounds__(512) void qmm0_kernel(const QmmArgs a) {
    constexpr int BB = WT == 2 ? 18 : (WT == 6 ? 22 : 34);
    __shared__ u32x4 s_w[2][2][QG][64];  // [buffer][half][block of the group][lane]: B operands
    __shared__ float s_d[2][2][QG][32];  // the weight rows' d
    __shared__ float s_red[4][16][64];   // half 1's partial sums
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // (uniform: scalar branches)
    const int w4 = wave & 3, kh = wave >> 2;
    const int c = lane & 31, g = lane >> 5;
    const int nb = a.cols / 32;
    const int n_rt = (a.rows + 31) / 32, n_tt = a.n_pad / 128;
    const int nwg = n_rt * n_tt, hw = blockIdx.x;
    const int lid = (nwg & 7) == 0 ? (hw & 7) * (nwg >> 3) + (hw >> 3) : hw;
    const int rt = lid / n_tt, tt = lid - rt * n_tt;
    const int r = min(rt * 32 + c, a.rows - 1);
    const int t32 = tt * 4 + w4;  // this wave's 32-row activation tile
    const Q0Layout L(a.ws, a.n_pad, a.cols);
    const uint8_t* wrow = static_cast<const uint8_t*>(a.w) + (size_t)r * nb * BB;
    const int8_t* abase = L.qs + ((size_t)t32 * nb * 64 + lane) * 16;
    const float* xbase = L.xd + (size_t)t32 * nb * 32 + c;
    const int nh = (nb + 1) / 2;
    const int kb0 = kh ? nh : 0, kcnt = kh ? nb - nh : nh;
    const int blast = kb0 + (kcnt > 0 ? kcnt - 1 : 0);
    const int ngroups = (nh + QG - 1) / QG;  // the same for both halves: every wave meets every barrier

    struct Stage {
        i32x4 av;
        float xd;  // lane (c, 0): the Q8_0 d of activation row c
    };
    // (blocks past the wave's last reload that block: in bounds, unused)
    auto load_a = [&](int j, Stage& st) __attribute__((always_inline)) {
        const int b = min(kb0 + j, blast);
        st.av = gld<i32x4>(abase + (size_t)b * 1024);
        st.xd = gld<float>(xbase + (size_t)b * 32);
    };
    auto load_w = [&](int grp, LegacyRaw<WT>& raw) __attribute__((always_inline)) {
        load_legacy<WT>(wrow + (size_t)min(kb0 + grp * QG + w4, blast) * BB, g, raw);
    };
    auto form = [&](int buf, const LegacyRaw<WT>& raw) __attribute__((always_inline)) {
        s_w[buf][kh][w4][lane] = __builtin_bit_cast(u32x4, legacy_operand<WT>(raw, g));
        if (g == 0) s_d[buf][kh][w4][c] = f16_to_f32(raw.dh);
    };
    struct Products {
        i32x16 acc;
        f32x16 dd;
    };
    f32x16 sum;
#pragma unroll
    for (int i = 0; i < 16; ++i) sum[i] = 0.0f;
    const f32x16 z = {};
    Products P;
    bool pending = false;  // (uniform)
    auto combine = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sum[i] = __builtin_fmaf((float)P.acc[i], P.dd[i], sum[i]);
    };

    LegacyRaw<WT> raw;
    load_w(0, raw);
    Stage S[QG];
#pragma unroll
    for (int j = 0; j < QG; ++j) load_a(j, S[j]);
    form(0, raw);
    lds_barrier();
    for (int grp = 0; grp < ngroups; ++grp) {
        const int buf = grp & 1;
        load_w(grp + 1, raw);  // (past the last group: a reload nobody reads)
#pragma unroll
        for (int j = 0; j < QG; ++j) {
            const int it = grp * QG + j;
            if (it < kcnt) {
                const i32x4 bv = __builtin_bit_cast(i32x4, s_w[buf][kh][j][lane]);
                const float wd = s_d[buf][kh][j][c];
                Products np;
                np.acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(S[j].av, bv, i32x16{}, 0, 0, 0);
                np.dd = __builtin_amdgcn_mfma_f32_32x32x2f32(g == 0 ? S[j].xd : 0.0f, g == 0 ? wd : 0.0f, z, 0, 0,
                                                             0);
                if (pending) combine();
                P = np;
                pending = true;
            }
            load_a(it + QG, S[j]);
        }
        form(buf ^ 1, raw);
        lds_barrier();
    }
    const int rr = rt * 32 + c;
    float rv[16];
    if (kh == 0) load_residual(a, t32 * 32, g, rr, rv);
    if (pending) combine();
    if (kh == 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s_red[w4][i][lane] = sum[i];
    }
    lds_barrier();
    if (kh == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sum[i] = sum[i] + s_red[w4][i][lane];
        store_tile(a, t32 * 32, g, rr, sum, rv);
    }
}

// Gemma's post-attention RMSNorm before the residual add (forward.rs:346-350):
// row t of x ([n][e], the matmul's output) becomes out = x * scale * w +
// residual, scale = 1 / (float)sqrt(ss / e + eps) with ss the f64 sum of the
// row's f32 squares (norm_rows_inplace -> rms_norm_inplace, ops.rs:106-114,
// 141-145; the sum in another order than the reference's left fold, which
// may move scale by an ulp).  residual may alias out (not x).  One workgroup
// per row; rows whose length is a multiple of 4 (with 16-byte aligned
// buffers) are read as 16-byte pieces,
// PN_PIECES per thread issued together, so a row costs one round trip per
// 4 * 256 * PN_PIECES values rather than one per 256.
constexpr int PN_PIECES = 4;
__global__ __launch_bounds__(256) void post_norm_kernel(const float* __restrict__ x, float* out,
                                                        const float* __restrict__ w, const float* residual, int e,
                                                        float eps) {
    __shared__ double s_part[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* row = x + (size_t)t * e;
    const bool vec = (e & 3) == 0 &&
                     (((uintptr_t)x | (uintptr_t)out | (uintptr_t)w | (uintptr_t)residual) & 15) == 0;
    double ss = 0.0;
    if (vec) {
        const int e4 = e >> 2;
        for (int i0 = 0; i0 < e4; i0 += 256 * PN_PIECES) {
            f32x4 v[PN_PIECES];
#pragma unroll
            for (int k = 0; k < PN_PIECES; ++k) {
                const int i = i0 + tid + 256 * k;
                v[k] = gld<f32x4>(row + 4 * (size_t)min(i, e4 - 1));
                if (i >= e4) v[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int k = 0; k < PN_PIECES; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma clang fp contract(off)
                    const float sq = v[k][j] * v[k][j];
                    ss += (double)sq;
                }
        }
    } else {
        for (int i = tid; i < e; i += 256) {
#pragma clang fp contract(off)
            const float sq = row[i] * row[i];
            ss += (double)sq;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    const double tot = ((s_part[0] + s_part[1]) + s_part[2]) + s_part[3];
    const float scale = 1.0f / (float)sqrt(tot / (double)e + (double)eps);
    float* orow = out + (size_t)t * e;
    const float* rrow = residual ? residual + (size_t)t * e : nullptr;
    if (vec) {
        const int e4 = e >> 2;
        for (int i0 = 0; i0 < e4; i0 += 256 * PN_PIECES) {
            f32x4 v[PN_PIECES], g[PN_PIECES], r[PN_PIECES];
#pragma unroll
            for (int k = 0; k < PN_PIECES; ++k) {
                const size_t i = 4 * (size_t)min(i0 + tid + 256 * k, e4 - 1);
                v[k] = gld<f32x4>(row + i);
                g[k] = gld<f32x4>(w + i);
                r[k] = rrow ? gld<f32x4>(rrow + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int k = 0; k < PN_PIECES; ++k) {
                const int i = i0 + tid + 256 * k;
                if (i < e4) {
                    f32x4 o;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
#pragma clang fp contract(off)
                        float y = v[k][j] * scale * g[k][j];
                        if (rrow) y = y + r[k][j];
                        o[j] = y;
                    }
                    *(__attribute__((address_space(1))) f32x4*)(orow + 4 * (size_t)i) = o;
                }
            }
        }
    } else {
        for (int i = tid; i < e; i += 256) {
#pragma clang fp contract(off)
            float y = row[i] * scale * w[i];
            if (rrow) y = y + rrow[i];
            orow[i] = y;
        }
    }
}

}  // namespace

size_t qmm_workspace_bytes(int n, int cols) {
    const size_t n_pad = (size_t)qmm_rows_padded(n), nb = (size_t)cols / QK;
    return n_pad * nb * (QK + 16 * sizeof(uint16_t) + sizeof(float));
}

size_t qmm0_workspace_bytes(int n, int cols) {
    const size_t n_pad = (size_t)qmm_rows_padded(n), nb = (size_t)cols / 32;
    return n_pad * cols + n_pad * nb * sizeof(float);
}

static bool legacy_wtype(int wt) { return wt == 2 || wt == 6 || wt == 8; }

hipError_t launch_qmatmul(const QmmArgs& a, hipStream_t st) {
    if (a.n <= 0 || a.rows <= 0) return hipSuccess;
    if (legacy_wtype(a.wtype)) {
        if (a.n_pad != qmm_rows_padded(a.n) || a.cols % 32 != 0) return hipErrorInvalidValue;
        const int nb = a.cols / 32;
        const unsigned items = (unsigned)(a.n_pad / 32 * nb);
        hipLaunchKernelGGL(q80_quantize_kernel<false>, dim3((items + 3) / 4), dim3(256), 0, st, a.act, a.cols, nb,
                           a.n, a.n_pad, a.ws);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const unsigned nwg = (unsigned)(((a.rows + 31) / 32) * (a.n_pad / 128));
        QmmArgs b = a;
        if (a.norm_w) {  // the raw rows to norm_tmp; the residual comes after the norm
            b.residual = nullptr;
            b.out = a.norm_tmp;
        }
        switch (a.wtype) {
            case 2: hipLaunchKernelGGL(qmm0_kernel<2>, dim3(nwg), dim3(512), 0, st, b); break;
            case 6: hipLaunchKernelGGL(qmm0_kernel<6>, dim3(nwg), dim3(512), 0, st, b); break;
            default: hipLaunchKernelGGL(qmm0_kernel<8>, dim3(nwg), dim3(512), 0, st, b); break;
        }
        e = hipGetLastError();
        if (e != hipSuccess || !a.norm_w) return e;
        hipLaunchKernelGGL(post_norm_kernel, dim3((unsigned)a.n), dim3(256), 0, st, a.norm_tmp, a.out, a.norm_w,
                           a.residual, a.rows, a.norm_eps);
        return hipGetLastError();
    }
    if (a.n_pad != qmm_rows_padded(a.n) || a.cols % QK != 0) return hipErrorInvalidValue;
    const int nb = a.cols / QK;
    hipLaunchKernelGGL(q8k_quantize_tiles_kernel, dim3((unsigned)(a.n_pad / 32 * nb)), dim3(512), 0, st, a.act,
                       a.cols, nb, a.n, a.n_pad, a.ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned nwg = (unsigned)(((a.rows + 31) / 32) * (a.n_pad / 128));
    QmmArgs b = a;
    if (a.norm_w) {  // the raw rows to norm_tmp; the residual comes after the norm
        b.residual = nullptr;
        b.out = a.norm_tmp;
    }
    if (a.wtype == 12)
        hipLaunchKernelGGL(qmm_kernel<12>, dim3(nwg), dim3(512), 0, st, b);
    else if (a.wtype == 14)
        hipLaunchKernelGGL(qmm_kernel<14>, dim3(nwg), dim3(512), 0, st, b);
    else
        return hipErrorInvalidValue;
    e = hipGetLastError();
    if (e != hipSuccess || !a.norm_w) return e;
    hipLaunchKernelGGL(post_norm_kernel, dim3((unsigned)a.n), dim3(256), 0, st, a.norm_tmp, a.out, a.norm_w,
                       a.residual, a.rows, a.norm_eps);
    return hipGetLastError();
}

hipError_t launch_quantize_q80(const float* act, int n, int cols, void* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int nb = cols / 32, n_pad = (n + 31) / 32 * 32;
    const unsigned items = (unsigned)(n_pad / 32 * nb);
    hipLaunchKernelGGL(q80_quantize_kernel<true>, dim3((items + 3) / 4), dim3(256), 0, st, act, cols, nb, n, n_pad,
                       out);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k(const float* act, int n, int cols, Q8KBlock* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int nb = cols / QK;
    hipLaunchKernelGGL(q8k_quantize_ref_kernel, dim3((unsigned)((n * nb + 3) / 4)), dim3(256), 0, st, act, cols, nb,
                       n, out);
    return hipGetLastError();
}

}  // namespace dr
