// kv_cache.hip -- the inter-step KV cache in HBM (StepCache,
// src/model/cache.rs:25-115), bf16, position-indexed.
//
// Layout per (layer, batch slot), for n_head_kv heads and capacity `cap`
// positions (a multiple of 64), HD = the head-dim tile (64/128/256/512):
//   K  : [n_head_kv][cap][HD]              row = sequence position
//   V^T: [n_head_kv][cap/32][HD][32]       V transposed per 32-key tile: a
//                                          tile's d-row holds its 32 positions
// The attention kernel stages both as 16-byte loads; V^T is exactly the
// operand orientation the P.V MFMA needs, so the transpose is paid once per
// stored row instead of once per attention tile, and a key tile of either is
// one contiguous block (whole cache lines for the DMA).
//
// store:  StepCache::store (cache.rs:62-71) -- f32 rows -> bf16 at their
//         positions, optionally after per-head RMSNorm of K (norm_heads,
//         ops.rs:384-389, applied before the store in forward.rs:300-302).
//         A layer kept at hi/lo precision also gets the lo halves,
//         bf16(x - bf16(x)), of K and V in planes laid out like K and V^T.
//         One launch, one workgroup per (64-row block, 64-wide head-dim
//         chunk, kv head): K converted in registers, V transposed through LDS.
//         Rows that fill whole 32-key tiles at contiguous positions, without
//         RoPE or lo halves (the denoise step's canvas rows), take a second
//         kernel: one workgroup per (kv head, tile), whole-line loads and
//         stores.
// gather: StepCache::gather (cache.rs:73-82) -- bf16 back to f32 rows (hi +
//         lo where the layer keeps the lo halves).
#include <algorithm>

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

constexpr int SR = 64;   // rows per store workgroup: one 128-byte line of a V^T row
constexpr int SD = 64;   // head-dim entries per store workgroup: one 128-byte line of a K row
constexpr int SPT = 16;  // consecutive values per thread (4 threads per row, 256 threads)

// One workgroup per (64-row block, 64-wide head-dim chunk, kv head), so that
// every 128-byte line of K and of V^T it writes is written whole by it.  All
// loads of the block (16 K and 16 V floats per thread) are issued before any
// store.  K: optional per-head RMSNorm, whose sum of squares covers the whole
// row (the other chunks' values are loaded for it), then bf16 at the row's
// position.  V: bf16 into an LDS tile transposed to [d][row]; each thread then
// writes 16 positions of one d-row of V^T (16-byte stores when the positions
// are contiguous and aligned).
template <int HD>
__global__ __launch_bounds__(256) void kv_store_kernel(const StoreArgs a) {
    constexpr int NDC = HD / SD;
    constexpr int V4 = SPT / 4;
    __shared__ __align__(16) uint16_t tile[SD][SR + 8];
    __shared__ __align__(16) uint16_t tile_lo[SD][SR + 8];  // V's lo half, when kept

    // Workgroup -> (kv head g, chunk dc, row block).  The hardware deals
    // workgroups round-robin over the 8 XCDs (XCD = blockIdx & 7); each XCD in
    // [xcd_lo, xcd_lo + xcd_n) takes a contiguous run of per_xcd logical ids,
    // so kv head g is written through the L2 of the XCD on which the attention
    // launch reads it (it deals heads to XCDs in the same contiguous way).
    const int x = blockIdx.x & 7;
    if (x < a.xcd_lo || x >= a.xcd_lo + a.xcd_n) return;
    const int lid = (x - a.xcd_lo) * a.per_xcd + (int)(blockIdx.x >> 3);
    if (lid >= a.n_head_kv * NDC * a.n_rb) return;
    const int hc = lid / a.n_rb;
    const int g = hc / NDC, dc = hc - g * NDC;
    const int r0 = (lid - hc * a.n_rb) * SR;
    const int tid = threadIdx.x, rl = tid >> 2, part = tid & 3;
    const int r = r0 + rl;
    const bool ok = r < a.n;
    const int d0 = dc * SD + part * SPT;  // first head-dim entry of this thread
    const size_t row = (size_t)(ok ? r : 0) * a.rstride + (size_t)g * a.hd;
    f32x4 xk[V4], xv[V4];
    if (ok && a.vec) {
#pragma unroll
        for (int i = 0; i < V4; ++i) {
            xk[i] = *reinterpret_cast<const f32x4*>(a.k + row + d0 + 4 * i);
            xv[i] = *reinterpret_cast<const f32x4*>(a.v + row + d0 + 4 * i);
        }
    } else {
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = d0 + 4 * i + e;
                const bool in = ok && d < a.hd;
                xk[i][e] = in ? a.k[row + d] : 0.0f;
                xv[i][e] = in ? a.v[row + d] : 0.0f;
            }
    }
    // The K-norm gains of this thread's dims and, with RoPE, of their
    // partners (d +- rot/2), requested with the rows: read where they are
    // used, after the row's norm, they cost a dependent round trip.
    f32x4 kw[V4], kwp[V4];
    if (a.kn_w) {
        const int hr = a.rot / 2;
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = d0 + 4 * i + e;
                kw[i][e] = d < a.hd ? a.kn_w[d] : 0.0f;
                kwp[i][e] = (a.rope && d < a.rot) ? a.kn_w[d < hr ? d + hr : d - hr] : 0.0f;
            }
    }
    const int pos = ok ? (a.pos0 >= 0 ? a.pos0 + r : (a.pos ? a.pos[r] : r)) : 0;
    // RoPE's (sin, cos) pairs of this thread's 16 dims, requested with the
    // rows: when rot/2 is a multiple of 16 they lie on one side of it, 32
    // contiguous floats of the position's table row
    const int rhalf = a.rot / 2;
    const bool tab_vec = a.rope && rhalf % SPT == 0 && d0 < a.rot;
    f32x4 tv[SPT / 2];
    if (tab_vec && ok) {
        const int j0 = d0 < rhalf ? d0 : d0 - rhalf;
        const f32x4* t = reinterpret_cast<const f32x4*>(a.rope + ((size_t)pos * rhalf + j0) * 2);
#pragma unroll
        for (int i = 0; i < SPT / 2; ++i) tv[i] = t[i];
    }

    // The Q/K/V epilogue's K and V part (forward.rs:291-310), when asked:
    // add_bias (ops.rs:373-382), then K's RMSNorm with the gain / V's
    // without one (Gemma, ops.rs:116-124), then RoPE on K (ops.rs:433-452).
    const float* kb = a.kb ? a.kb + (size_t)g * a.hd : nullptr;
    const float* vb = a.vb ? a.vb + (size_t)g * a.hd : nullptr;
    if (kb || vb) {
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = d0 + 4 * i + e;
                if (d < a.hd) {
                    if (kb) xk[i][e] += kb[d];
                    if (vb) xv[i][e] += vb[d];
                }
            }
    }
    // The row's other 64-wide chunks at this thread's 16 entries (bias
    // added), read once: the norms sum over the whole row, and with RoPE a
    // dim's partner (d +- rot/2) lies in one of them when rot/2 is a multiple
    // of 64.
    const bool need_ko = a.kn_w || a.rope;
    f32x4 ko[NDC][V4], vo[NDC][V4];
    auto load_other = [&](f32x4 (&xo)[NDC][V4], const float* src, const float* bias)
        __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NDC; ++c) {
            if (c == dc) continue;
            const int e0 = c * SD + part * SPT;
            if (ok && a.vec) {
#pragma unroll
                for (int i = 0; i < V4; ++i) {
                    xo[c][i] = *reinterpret_cast<const f32x4*>(src + row + e0 + 4 * i);
                    if (bias) xo[c][i] += *reinterpret_cast<const f32x4*>(bias + e0 + 4 * i);
                }
            } else {
#pragma unroll
                for (int i = 0; i < V4; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int d = e0 + 4 * i + e;
                        float v = (ok && d < a.hd) ? src[row + d] : 0.0f;
                        if (bias && d < a.hd) v += bias[d];
                        xo[c][i][e] = v;
                    }
            }
        }
    };
    if (need_ko) load_other(ko, a.k, kb);
    if (a.v_norm) load_other(vo, a.v, vb);
    // rms_norm_inplace (ops.rs:106-114) / rms_norm_noscale: f32 squares
    // summed in f64 over the whole row
    auto row_scale = [&](const f32x4 (&x)[V4], const f32x4 (&xo)[NDC][V4], float eps)
        __attribute__((always_inline)) {
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < NDC; ++c)
#pragma unroll
            for (int i = 0; i < V4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float xv = c == dc ? x[i][e] : xo[c][i][e];
                    const float sq = xv * xv;
                    ss += (double)sq;
                }
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        return 1.0f / (float)sqrt(ss / (double)a.hd + (double)eps);
    };
    float ksc = 1.0f;
    if (a.kn_w) {
        ksc = row_scale(xk, ko, a.kn_eps);
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = d0 + 4 * i + e;
                if (d < a.hd) xk[i][e] = xk[i][e] * ksc * kw[i][e];
            }
    }
    if (a.v_norm) {
        const float vsc = row_scale(xv, vo, a.kn_eps);
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[i][e] *= vsc;
    }
    if (a.rope && ok) {
        // the partner's value with the same bias and norm, then the pair
        // rotates (rotate_rows, ops.rs:433-452)
        const int half = a.rot / 2;
        const float* tab = a.rope + (size_t)pos * half * 2;
        const bool chunked = half % SD == 0;  // partner = same entry of chunk dc +- half/SD
        // (the thread's 16 dims lie on one side of half, so one chunk)
        const int pc = chunked ? (d0 < half ? dc + half / SD : dc - half / SD) : 0;
        f32x4 yk[V4];
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = d0 + 4 * i + e;
                yk[i][e] = xk[i][e];
                if (d >= a.rot) continue;
                const int pd = d < half ? d + half : d - half;
                float xp;
                if (chunked) {
                    xp = 0.0f;
#pragma unroll
                    for (int c = 0; c < NDC; ++c)
                        if (c == pc) xp = ko[c][i][e];  // pc != dc
                } else {
                    xp = a.k[row + pd];
                    if (kb) xp += kb[pd];
                }
                if (a.kn_w) xp = xp * ksc * kwp[i][e];
                const int j = d < half ? d : pd;
                float2 t;
                if (tab_vec) {
                    const int k4 = 4 * i + e;  // pair k4 of the 16: floats 2*k4, 2*k4+1
                    t = make_float2(tv[k4 / 2][2 * (k4 % 2)], tv[k4 / 2][2 * (k4 % 2) + 1]);
                } else {
                    t = *reinterpret_cast<const float2*>(tab + 2 * j);
                }
                yk[i][e] = d < half ? rope_lo(xk[i][e], xp, t.x, t.y) : rope_hi(xp, xk[i][e], t.x, t.y);
            }
#pragma unroll
        for (int i = 0; i < V4; ++i) xk[i] = yk[i];
    }
    if (ok) {
        uint16_t* dst = a.kc + ((size_t)g * a.cap + pos) * HD + d0;
#pragma unroll
        for (int i = 0; i < V4; i += 2) {
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                w[2 * j] = (uint32_t)f2bf(xk[i + j][0]) | ((uint32_t)f2bf(xk[i + j][1]) << 16);
                w[2 * j + 1] = (uint32_t)f2bf(xk[i + j][2]) | ((uint32_t)f2bf(xk[i + j][3]) << 16);
            }
            *reinterpret_cast<u32x4*>(dst + 4 * i) = w;
        }
        if (a.klo) {
            // the lo half: bf16 of what bf16 rounding dropped
            uint16_t* dlo = a.klo + ((size_t)g * a.cap + pos) * HD + d0;
#pragma unroll
            for (int i = 0; i < V4; i += 2) {
                u32x4 w;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    uint16_t lo[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) lo[e] = f2bf(xk[i + j][e] - bf2f(f2bf(xk[i + j][e])));
                    w[2 * j] = (uint32_t)lo[0] | ((uint32_t)lo[1] << 16);
                    w[2 * j + 1] = (uint32_t)lo[2] | ((uint32_t)lo[3] << 16);
                }
                *reinterpret_cast<u32x4*>(dlo + 4 * i) = w;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < V4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) tile[part * SPT + 4 * i + e][rl] = f2bf(xv[i][e]);
    if (a.vlo) {
#pragma unroll
        for (int i = 0; i < V4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                tile_lo[part * SPT + 4 * i + e][rl] = f2bf(xv[i][e] - bf2f(f2bf(xv[i][e])));
    }
    // (a pass without pos0: the position of row tid % 64 of the block, for
    // the V^T stores below, requested before the barrier)
    const bool known = a.pos0 >= 0 || a.pos == nullptr;
    const int my_row = r0 + (tid & 63);
    const int my_pos = (!known && my_row < a.n) ? a.pos[my_row] : 0;
    __syncthreads();

    if (!known) {
        // Positions from a list: the 64 lanes of a wave take the block's 64
        // rows of one d-row, so each store instruction's 2-byte writes fall
        // into the few 32-key tiles that the sorted positions span and merge
        // into a few segment writes.  (Lanes over 16 d-rows x 4 row groups
        // made 64 separate writes per instruction: 12.9 against 4.1 us for
        // C2's 256 rows.)
        if (my_row >= a.n) return;
        const size_t pofs = (size_t)(my_pos / VT_KEYS) * (HD * VT_KEYS) + my_pos % VT_KEYS;
        const size_t vbase = (size_t)g * HD * a.cap + (size_t)(dc * SD) * VT_KEYS + pofs;
        const int rr = tid & 63;
#pragma unroll
        for (int k = 0; k < SD / 4; ++k) {
            const int d = (tid >> 6) + 4 * k;
            a.vtc[vbase + (size_t)d * VT_KEYS] = tile[d][rr];
        }
        if (a.vlo) {
#pragma unroll
            for (int k = 0; k < SD / 4; ++k) {
                const int d = (tid >> 6) + 4 * k;
                a.vlo[vbase + (size_t)d * VT_KEYS] = tile_lo[d][rr];
            }
        }
        return;
    }

    // V^T: thread -> (d-row dl, positions p0 + [0,16)).
    const int dl = tid >> 2, p0 = (tid & 3) * SPT;
    const int rfirst = r0 + p0;
    if (rfirst >= a.n) return;
    const int cnt = min(SPT, a.n - rfirst);
    const int dv = dc * SD + dl;  // this thread's d-row
    // V^T element (g, dv, p): tile p / VT_KEYS, offset p % VT_KEYS in its d-row
    const size_t vrow = (size_t)g * HD * a.cap + (size_t)dv * VT_KEYS;
    auto vt_in = [&](uint16_t* plane, int p) __attribute__((always_inline)) {
        return plane + vrow + (size_t)(p / VT_KEYS) * (HD * VT_KEYS) + p % VT_KEYS;
    };
    auto vt_at = [&](int p) __attribute__((always_inline)) { return vt_in(a.vtc, p); };
    // (contiguous rows, pos0 >= 0: positions without a load)
    const int pbase = a.pos0 >= 0 ? a.pos0 : 0;
    const int q0 = pbase + rfirst;
    const bool contiguous = cnt == SPT && (q0 & 7) == 0;
    const uint16_t* t = &tile[dl][p0];
    if (contiguous) {
        // 8 positions from a multiple of 8 never cross a 32-key tile
#pragma unroll
        for (int h = 0; h < SPT / 8; ++h)
            *reinterpret_cast<u32x4*>(vt_at(q0 + 8 * h)) = *reinterpret_cast<const u32x4*>(t + 8 * h);
    } else {
        for (int e = 0; e < cnt; ++e) *vt_at(q0 + e) = t[e];
    }
    if (a.vlo) {
        // the same positions of the lo plane (V^T's layout)
        const uint16_t* tl = &tile_lo[dl][p0];
        if (contiguous) {
#pragma unroll
            for (int h = 0; h < SPT / 8; ++h)
                *reinterpret_cast<u32x4*>(vt_in(a.vlo, q0 + 8 * h)) = *reinterpret_cast<const u32x4*>(tl + 8 * h);
        } else {
            for (int e = 0; e < cnt; ++e) *vt_in(a.vlo, q0 + e) = tl[e];
        }
    }
}

// The store of rows that fill whole 32-key V^T tiles at contiguous positions
// (pos0 and n multiples of 32), head dim == HD (64, 128 or 256), without lo
// halves: the canvas rows of every denoise step.  One workgroup per (kv
// head, tile); thread (rg, dc), rg fastest, holds the 4 dims 4 dc .. 4 dc + 3
// of the tile's rows RPG rg .. RPG rg + RPG - 1.
// - Loads: per instruction the wave reads whole 128-byte lines (hd 128: 8
//   rows x 128 B), against 64-byte pieces at a 64-byte lane stride in
//   kv_store_kernel.
// - The K / V biases, the K norm and Gemma's V norm of the epilogue, as in
//   kv_store_kernel: a row's f32 squares summed in f64, over the 4 dims of
//   each thread, then across the lanes of the row in the wave (shuffles),
//   then across the 4 waves in wave order (LDS).  RoPE on K (rotate_rows,
//   ops.rs:433-452; rot a multiple of 8, so a thread's 4 dims lie on one side
//   of rot / 2) reads the partner dim d +- rot / 2 of the normed row from LDS
//   and the (sin, cos) pairs of the row's position, loaded with the rows.
// - K: bf16 of the 4 dims, 8 bytes per row.
// - V^T: at step e the thread writes the RPG keys of its rows in d-row
//   4 dc + e of the tile; the NRG lanes of one dc together write that
//   d-row's 64 bytes whole, so no LDS transpose and no barrier is needed.
// Same values as kv_store_kernel: bf16 (round to nearest even) of each f32.
// EPI: the epilogue (biases, norms, RoPE) is compiled in; the plain build
// keeps it out, since its conditional updates of the loaded rows made the K
// stores wait for every load.
template <int HD, bool EPI>
__global__ __launch_bounds__(256) void kv_store_tiles_kernel(const StoreArgs a) {
    constexpr int CPR = HD / 4;     // 4-dim pieces per row
    constexpr int NRG = 256 / CPR;  // row groups
    constexpr int RPG = VT_KEYS / NRG;  // rows per row group
    static_assert(NRG * RPG == VT_KEYS && RPG >= 2 && RPG <= 8, "tile geometry");

    const int x = blockIdx.x & 7;  // (XCD placement as kv_store_kernel)
    if (x < a.xcd_lo || x >= a.xcd_lo + a.xcd_n) return;
    const int lid = (x - a.xcd_lo) * a.per_xcd + (int)(blockIdx.x >> 3);
    const int ntl = a.n / VT_KEYS;
    if (lid >= a.n_head_kv * ntl) return;
    const int g = lid / ntl, tb = lid - g * ntl;
    const int tid = threadIdx.x;
    const int rg = tid % NRG, dc = tid / NRG;
    const int r0 = tb * VT_KEYS + rg * RPG;  // first row of this thread
    const size_t rstride = (size_t)a.rstride;
    const size_t src = (size_t)r0 * rstride + (size_t)g * HD + 4 * dc;
    f32x4 xk[RPG], xv[RPG];
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
        xk[j] = *reinterpret_cast<const f32x4*>(a.k + src + j * rstride);
        xv[j] = *reinterpret_cast<const f32x4*>(a.v + src + j * rstride);
    }
    if constexpr (EPI) {
        const int half = a.rot / 2;
        const int d0 = 4 * dc;
        const bool rot_me = a.rope && d0 < a.rot;
        f32x4 tab[RPG][2];  // (sin, cos) of pairs jj .. jj + 3 at each row's position
        if (rot_me) {
            const int jj = d0 < half ? d0 : d0 - half;
            const int pp = (a.pos0 >= 0 ? a.pos0 : 0) + r0;
#pragma unroll
            for (int j = 0; j < RPG; ++j) {
                const float* t = a.rope + ((size_t)(pp + j) * half + jj) * 2;
                tab[j][0] = *reinterpret_cast<const f32x4*>(t);
                tab[j][1] = *reinterpret_cast<const f32x4*>(t + 4);
            }
        }
        f32x4 kw4 = {}, kb4 = {}, vb4 = {};
        if (a.kn_w) kw4 = *reinterpret_cast<const f32x4*>(a.kn_w + 4 * dc);
        if (a.kb) kb4 = *reinterpret_cast<const f32x4*>(a.kb + (size_t)g * HD + 4 * dc);
        if (a.vb) vb4 = *reinterpret_cast<const f32x4*>(a.vb + (size_t)g * HD + 4 * dc);
        // (each bias only where given: adding a zero would turn -0.0 into +0.0)
        if (a.kb) {
#pragma unroll
            for (int j = 0; j < RPG; ++j) xk[j] += kb4;
        }
        if (a.vb) {
#pragma unroll
            for (int j = 0; j < RPG; ++j) xv[j] += vb4;
        }
        if (a.kn_w || a.v_norm) {
            // rms_norm_inplace (ops.rs:106-114) / rms_norm_noscale: sum of the
            // row's f32 squares in f64; the row's lanes in this wave are lanes
            // rg + NRG i, the other CPR / (64 / NRG) - 1 shares are in the
            // other waves
            __shared__ double s_ss[2][4][VT_KEYS];  // [K, V][wave][row of the tile]
            const int wave = tid >> 6;
            auto row_ss = [&](const f32x4 (&x)[RPG], double (&ss)[RPG]) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < RPG; ++j) {
                    double t = 0.0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float sq = x[j][e] * x[j][e];
                        t += (double)sq;
                    }
#pragma unroll
                    for (int off = NRG; off < 64; off <<= 1) t += __shfl_xor(t, off);
                    ss[j] = t;
                }
            };
            double ssk[RPG], ssv[RPG];
            if (a.kn_w) row_ss(xk, ssk);
            if (a.v_norm) row_ss(xv, ssv);
            if ((tid & 63) < NRG) {
#pragma unroll
                for (int j = 0; j < RPG; ++j) {
                    if (a.kn_w) s_ss[0][wave][rg * RPG + j] = ssk[j];
                    if (a.v_norm) s_ss[1][wave][rg * RPG + j] = ssv[j];
                }
            }
            __syncthreads();
            auto scale_of = [&](int kv, int j) __attribute__((always_inline)) {
                const double t = ((s_ss[kv][0][rg * RPG + j] + s_ss[kv][1][rg * RPG + j]) + s_ss[kv][2][rg * RPG + j]) +
                                 s_ss[kv][3][rg * RPG + j];
                return 1.0f / (float)sqrt(t / (double)HD + (double)a.kn_eps);
            };
#pragma unroll
            for (int j = 0; j < RPG; ++j) {
                if (a.kn_w) {
                    const float sc = scale_of(0, j);
#pragma unroll
                    for (int e = 0; e < 4; ++e) xk[j][e] = xk[j][e] * sc * kw4[e];
                }
                if (a.v_norm) {
                    const float sc = scale_of(1, j);
#pragma unroll
                    for (int e = 0; e < 4; ++e) xv[j][e] *= sc;
                }
            }
        }
        if (a.rope) {
            __shared__ __align__(16) float s_k[VT_KEYS][HD + 4];  // the tile's normed K rows
#pragma unroll
            for (int j = 0; j < RPG; ++j) *reinterpret_cast<f32x4*>(&s_k[rg * RPG + j][d0]) = xk[j];
            __syncthreads();
            if (rot_me) {
                const int pd0 = d0 < half ? d0 + half : d0 - half;
#pragma unroll
                for (int j = 0; j < RPG; ++j) {
                    const f32x4 xp = *reinterpret_cast<const f32x4*>(&s_k[rg * RPG + j][pd0]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float sn = tab[j][e >> 1][2 * (e & 1)], cs = tab[j][e >> 1][2 * (e & 1) + 1];
                        xk[j][e] = d0 < half ? rope_lo(xk[j][e], xp[e], sn, cs) : rope_hi(xp[e], xk[j][e], sn, cs);
                    }
                }
            }
        }
    }
    const int p0 = a.pos0 >= 0 ? a.pos0 : 0;  // (host: pos0 >= 0, or no position list)
    uint16_t* kdst = a.kc + ((size_t)g * a.cap + p0 + r0) * HD + 4 * dc;
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
        uint32_t w0 = (uint32_t)f2bf(xk[j][0]) | ((uint32_t)f2bf(xk[j][1]) << 16);
        uint32_t w1 = (uint32_t)f2bf(xk[j][2]) | ((uint32_t)f2bf(xk[j][3]) << 16);
        *reinterpret_cast<uint2*>(kdst + (size_t)j * HD) = make_uint2(w0, w1);
    }
    uint16_t* vdst = a.vtc + (size_t)g * HD * a.cap + (size_t)(p0 / VT_KEYS + tb) * (HD * VT_KEYS) +
                     (size_t)(4 * dc) * VT_KEYS + rg * RPG;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t w[RPG / 2];
#pragma unroll
        for (int j = 0; j < RPG / 2; ++j)
            w[j] = (uint32_t)f2bf(xv[2 * j][e]) | ((uint32_t)f2bf(xv[2 * j + 1][e]) << 16);
        uint16_t* row = vdst + e * VT_KEYS;
        if constexpr (RPG == 2) {
            *reinterpret_cast<uint32_t*>(row) = w[0];
        } else if constexpr (RPG == 4) {
            *reinterpret_cast<uint2*>(row) = make_uint2(w[0], w[1]);
        } else {
            *reinterpret_cast<u32x4*>(row) = u32x4{w[0], w[1], w[2], w[3]};
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
        const size_t ki = ((size_t)g * a.cap + pos) * HD + d;
        a.out_k[idx] = a.klo ? bf2f(a.kc[ki]) + bf2f(a.klo[ki]) : bf2f(a.kc[ki]);
        const size_t vi = ((size_t)g * a.cap + (size_t)(pos / VT_KEYS) * VT_KEYS) * HD + (size_t)d * VT_KEYS +
                          pos % VT_KEYS;
        a.out_v[idx] = a.vlo ? bf2f(a.vtc[vi]) + bf2f(a.vlo[vi]) : bf2f(a.vtc[vi]);
    }
}

}  // namespace

hipError_t launch_store(int hd_tile, const StoreArgs& args, hipStream_t st) {
    if (args.n <= 0) return hipSuccess;
    if (hd_tile != 64 && hd_tile != 128 && hd_tile != 256 && hd_tile != 512) return hipErrorInvalidValue;
    StoreArgs a = args;
    if (a.rstride == 0) a.rstride = a.n_head_kv * a.hd;  // (packed rows)
    if (a.rstride < a.n_head_kv * a.hd) return hipErrorInvalidValue;
    // Batch slot b of nb: the attention launch puts the slot's kv heads on
    // XCDs [8b/nb, 8(b+1)/nb).
    const int nb = a.n_batch > 0 ? a.n_batch : 1;
    a.xcd_lo = 8 * a.batch / nb;
    a.xcd_n = std::max(1, 8 * (a.batch + 1) / nb - a.xcd_lo);
    // whole tiles at contiguous positions, no epilogue: the tile kernel
    const int p0 = a.pos0 >= 0 ? a.pos0 : (a.pos == nullptr ? 0 : -1);
    const bool tiles = a.vec && a.hd == hd_tile && hd_tile <= 256 && p0 >= 0 && p0 % VT_KEYS == 0 &&
                       a.n % VT_KEYS == 0 && !a.klo && !a.vlo && (!a.rope || (a.rot % 8 == 0 && a.rot <= a.hd)) &&
                       (((uintptr_t)a.kn_w | (uintptr_t)a.kb | (uintptr_t)a.vb | (uintptr_t)a.rope) & 15) == 0;
    if (tiles) {
        a.pos0 = p0;
        const int work = a.n_head_kv * (a.n / VT_KEYS);
        a.per_xcd = (work + a.xcd_n - 1) / a.xcd_n;
        const dim3 grid((unsigned)(8 * a.per_xcd));
        const bool epi = a.kn_w || a.kb || a.vb || a.v_norm || a.rope;
        switch (hd_tile * 2 + (epi ? 1 : 0)) {
            case 128: hipLaunchKernelGGL((kv_store_tiles_kernel<64, false>), grid, dim3(256), 0, st, a); break;
            case 129: hipLaunchKernelGGL((kv_store_tiles_kernel<64, true>), grid, dim3(256), 0, st, a); break;
            case 256: hipLaunchKernelGGL((kv_store_tiles_kernel<128, false>), grid, dim3(256), 0, st, a); break;
            case 257: hipLaunchKernelGGL((kv_store_tiles_kernel<128, true>), grid, dim3(256), 0, st, a); break;
            case 512: hipLaunchKernelGGL((kv_store_tiles_kernel<256, false>), grid, dim3(256), 0, st, a); break;
            default: hipLaunchKernelGGL((kv_store_tiles_kernel<256, true>), grid, dim3(256), 0, st, a); break;
        }
        return hipGetLastError();
    }
    a.n_rb = (a.n + SR - 1) / SR;
    const int work = a.n_head_kv * (hd_tile / SD) * a.n_rb;
    a.per_xcd = (work + a.xcd_n - 1) / a.xcd_n;
    const dim3 grid((unsigned)(8 * a.per_xcd));
    switch (hd_tile) {
        case 64: hipLaunchKernelGGL(kv_store_kernel<64>, grid, dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL(kv_store_kernel<128>, grid, dim3(256), 0, st, a); break;
        case 256: hipLaunchKernelGGL(kv_store_kernel<256>, grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(kv_store_kernel<512>, grid, dim3(256), 0, st, a); break;
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
        case 512: hipLaunchKernelGGL(kv_gather_kernel<512>, dim3((unsigned)blocks), dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dr
