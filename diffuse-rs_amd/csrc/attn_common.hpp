// attn_common.hpp -- device helpers shared by the attention kernels
// (attn_fwd.hip, attn_ring.hip): vector types, the LDS tile swizzle and key
// permutations of the 32-key K tiles, LDS-DMA, visible() of attention.rs:36-57,
// and the packed-row decode of GQA query rows.
#pragma once

#include "dr_internal.hpp"

namespace dr {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int BN = 32;                     // keys per tile (one MFMA key block)
static_assert(BN == VT_KEYS, "a key tile is one V^T tile of the cache");
constexpr float RESCALE_THRESHOLD = 8.0f;  // log2 units

// 16-byte-chunk swizzle for an LDS row holding CH chunks, so that the rows
// that one MFMA operand read takes at the same logical chunk sit on distinct
// banks.  The 64-byte rows of a V^T tile (CH 4; the read takes row d = 32 db
// + col, chunks 2 hf + s) use (d >> 2) & 3, which SQ_LDS_BANK_CONFLICT
// measures conflict-free on MI355X.  ((d >> 1) ^ (d >> 3)) & 3, conflict-free
// for a 32-bank LDS read 8 lanes at a time, cost 32 conflict cycles per wave
// and tile there, 17-32 % of the LDS-active cycles at C2, C4 and C5's global
// layer, and ((d >> 2) ^ (d >> 4)) & 3 as many.)
template <int CH>
__device__ __forceinline__ int swz(int row) {
    if constexpr (CH >= 16) {
        return row & 15;
    } else if constexpr (CH == 8) {
        return (row & 7) ^ ((row >> 3) & 1);
    } else {
        static_assert(CH == 4, "unsupported row width");
        return (row >> 2) & 3;
    }
}

// The 64-byte V^T rows read by 16-row waves (16x16x32 MFMA: lane (g, n)
// reads chunk g of row 16 k + n) take (d >> 1) & 3, which
// SQ_LDS_BANK_CONFLICT measures conflict-free on MI355X; swz<4> above cost
// 0.28 of the LDS-active cycles there, and five other forms as much.
__device__ __forceinline__ int swz_v16(int d) { return (d >> 1) & 3; }

// RoPE's rotation of one pair (ops.rs:447-448), without fused multiply-adds
// as Rust evaluates it.
__device__ __forceinline__ float rope_lo(float a, float b, float sn, float cs) {
#pragma clang fp contract(off)
    return a * cs - b * sn;
}
__device__ __forceinline__ float rope_hi(float a, float b, float sn, float cs) {
#pragma clang fp contract(off)
    return a * sn + b * cs;
}

// Key offset (within a 32-key block) stored in LDS row R of the block.  The
// MFMA puts A-row R in accumulator slot i of lane half hf with
// R = 8*(i/4) + 4*hf + (i%4); sigma(R) = 16*hf + i places key 16*hf + i there.
__device__ __forceinline__ int sigma(int R) {
    return 16 * ((R >> 2) & 1) + 4 * (R >> 3) + (R & 3);
}

// The same for 16-row waves (16x16x32 MFMA, two 16-key blocks b): A-row R
// of block b lands in accumulator slot i of lane group g with R = 4*g + i,
// and the PV product wants lane group g to hold keys 8*g .. 8*g + 7, so
// kappa(16*b + 4*g + i) = 8*g + 4*b + i.
__device__ __forceinline__ int kappa(int R) {
    return 8 * ((R & 15) >> 2) + 4 * (R >> 4) + (R & 3);
}
template <bool W16>
__device__ __forceinline__ int kperm(int R) {
    if constexpr (W16)
        return kappa(R);
    else
        return sigma(R);
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

// Raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit
// data format, no swizzle).  Loads at offsets >= bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// 16 bytes per lane, buffer -> LDS (buffer_load_dwordx4 ... lds): lane i
// reads rsrc + soff + voff and writes lds_base + 16*i.  Kept in a __device__
// helper: used directly in a kernel body, an LDS-DMA builtin made the host
// compilation pass drop the kernel's launch stub.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds_base, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base,
                                             16, voff, soff, 0, 0);
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
    if constexpr (NS >= 4) {
        if (pending >= 2) {
            wait_vmcnt<2 * NI>();
            return;
        }
    }
    if constexpr (NS >= 3) {
        if (pending >= 1) {
            wait_vmcnt<NI>();
            return;
        }
    }
    wait_vmcnt<0>();
}

// (head in group, query index) of packed row r = hg * nq + qi.  MHA rows are
// the queries themselves; otherwise a float reciprocal estimate (exact to +-1
// for r < 2^24) is corrected once, instead of an integer division.
__device__ __forceinline__ void row_split(int r, int nq, float inv_nq, int group, int& hg,
                                          int& qi) {
    if (group == 1) {
        hg = 0;
        qi = r;
        return;
    }
    int h = (int)((float)r * inv_nq);
    int q = r - h * nq;
    if (q < 0) {
        --h;
        q += nq;
    } else if (q >= nq) {
        ++h;
        q -= nq;
    }
    hg = h;
    qi = q;
}

// n / d for the workgroup decode: mul-high by m = ceil(2^32 / d), exact when
// n * d < 2^32 (the host passes m = 0 where that is not guaranteed).
__device__ __forceinline__ int udiv(int n, int d, uint32_t m) {
    return m ? (int)__umulhi((uint32_t)n, m) : n / d;
}

// Loads and stores through the global address space.  Pointers that come
// from kernel-argument structs are generic to the compiler, which then emits
// flat instructions; a pending flat load makes every later wait a full
// vmcnt(0) (it may be an LDS access), which would also wait for in-flight
// K/V tile DMA.
// (The host compilation pass, which only parses device code, has no
// address spaces.)
template <typename T>
__device__ __forceinline__ T gload(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(1))) T*)p;
#else
    return *static_cast<const T*>(p);
#endif
}
template <typename T>
__device__ __forceinline__ void gstore(void* p, const T& v) {
#if defined(__HIP_DEVICE_COMPILE__)
    *(__attribute__((address_space(1))) T*)p = v;
#else
    *static_cast<T*>(p) = v;
#endif
}

// Workgroup barrier that orders only this wave's LDS instructions
// (ds_read / ds_write) before it.  __syncthreads() is a workgroup release
// fence, which must also wait for in-flight buffer_load ... lds DMA (it
// writes LDS), i.e. vmcnt(0); a wave that keeps its own K/V DMA in flight
// across the barrier uses this instead.  The "memory" clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float max3(float a, float b, float c) {
    return __builtin_fmaxf(__builtin_fmaxf(a, b), c);
}

// Folds SG key-split softmax states (m_j, l_j, o_j: row max in log2 units,
// weight sum, C 4-float chunks of the unnormalised row) into the running
// state (Mx, Ls, acc) as softmax states merge: weights exp2(m_j - max), a
// state with m_j = -inf weighs 0.  Every kernel that merges splits calls this,
// with the operations spelled out (no contraction), so they agree bit for bit.
// No branch: when every state so far has m = -inf the running state is (-inf,
// 0, 0), f and every weight are 0, and it stays so (an early return let the
// compiler sink the l and o loads behind the m loads' wait).
template <int SG, int C>
__device__ __forceinline__ void merge_split_states(float& Mx, float& Ls, f32x4 (&acc)[C],
                                                   const float (&m)[SG], const float (&l)[SG],
                                                   const f32x4 (&o)[SG][C]) {
#pragma clang fp contract(off)
    float nm = Mx;
#pragma unroll
    for (int j = 0; j < SG; ++j) nm = __builtin_fmaxf(nm, m[j]);
    const float f = Mx == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(Mx - nm);
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = acc[c] * f;
    Ls = Ls * f;
#pragma unroll
    for (int j = 0; j < SG; ++j) {
        const float w = m[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[j] - nm);
        Ls = __builtin_fmaf(w, l[j], Ls);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[c][e] = __builtin_fmaf(w, o[j][c][e], acc[c][e]);
    }
    Mx = nm;
}

// Agent-scope (sc1) accesses: coherent across the XCDs' separate L2s without
// a cache-wide writeback or invalidate.  The key-split partials that a
// workgroup merges in-kernel (the last split of a row block to finish, by an
// atomic ticket) are written and read only through these; the 16-byte forms
// are buffer instructions with the sc1 cache-policy bit.
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ void store_sc1(__amdgpu_buffer_rsrc_t r, int voff, const f32x4& v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, 0, CPOL_SC1);
}
__device__ __forceinline__ f32x4 load_sc1(__amdgpu_buffer_rsrc_t r, int voff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, CPOL_SC1));
}
__device__ __forceinline__ void store2_sc1(__amdgpu_buffer_rsrc_t r, int voff, float x, float y) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) uint32_t,
                                                             (float __attribute__((ext_vector_type(2)))){x, y}),
                                          r, voff, 0, CPOL_SC1);
}
__device__ __forceinline__ float2 load2_sc1(__amdgpu_buffer_rsrc_t r, int voff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, CPOL_SC1);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

}  // namespace
}  // namespace dr
