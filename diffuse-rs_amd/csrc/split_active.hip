// split_active.hip -- StepCache::split_active (src/model/cache.rs:85-114) on
// the device: the per-position active test and the two ascending position
// lists, written straight into the passes' device position arrays, so that a
// denoise step whose token sequence lives on the device needs no host loop
// and no upload of index lists.
#include "dr_internal.hpp"

namespace dr {
namespace {

constexpr int ST = 1024;                // threads: one position each per chunk
constexpr int EXTRA_ACTIVE_STEPS = 2;   // cache.rs:23

// One workgroup.  Chunk by chunk (ST positions), every thread decides its
// position (cache.rs:88-97: changed, still masked, or changed within
// EXTRA_ACTIVE_STEPS steps; :98-104: within `vicinity` of a masked position),
// then its rank among the chunk's active positions comes from the wave's
// ballot and the waves' counts in LDS.  Active position i goes to
// active[rank], a cached one to cached[i - rank] (the positions are 0..n-1,
// so i - rank cached positions precede it): both lists ascend.  meta gets
// {n_active, n_cached, first active, last active, first cached, last cached}.
__global__ __launch_bounds__(ST) void split_active_kernel(const SplitArgs a) {
    __shared__ int s_wave[ST / 64];
    __shared__ int s_meta[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 4) s_meta[tid] = 0;
    int na = 0;  // active positions before this chunk (uniform)
    for (int base = 0; base < a.n; base += ST) {
        const int i = base + tid;
        bool act = false;
        if (i < a.n) {
            const bool changed = a.seq[i] != a.prev_seq[i];
            int lc = a.last_changed[i];
            if (changed) {
                lc = a.step;
                a.last_changed[i] = lc;
            }
            const bool recent = lc >= 0 && a.step - lc <= EXTRA_ACTIVE_STEPS;
            act = changed || a.is_masked[i] != 0 || recent;
            if (!act && a.vicinity > 0) {
                // some masked m with |i - m| <= vicinity fills i
                const int lo = i > a.vicinity ? i - a.vicinity : 0;
                const int hi = min(a.n - 1, i + a.vicinity);
                for (int m = lo; m <= hi && !act; ++m) act = a.is_masked[m] != 0;
            }
        }
        const uint64_t bal = __ballot(act);
        const int before = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) s_wave[wave] = __popcll(bal);
        __syncthreads();
        int wbase = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < ST / 64; ++w) {
            const int c = s_wave[w];
            wbase += w < wave ? c : 0;
            tot += c;
        }
        const int chunk_n = min(ST, a.n - base);
        if (i < a.n) {
            const int ra = na + wbase + before;  // rank among the active positions
            if (act) {
                a.active[ra] = i;
                if (ra == 0) s_meta[0] = i;
                if (ra == na + tot - 1) s_meta[1] = i;
            } else {
                const int rc = i - ra;
                a.cached[rc] = i;
                if (rc == 0) s_meta[2] = i;
                if (rc == base + chunk_n - (na + tot) - 1) s_meta[3] = i;
            }
        }
        na += tot;
        __syncthreads();  // s_wave is rewritten by the next chunk
    }
    __syncthreads();  // (n == 0: the initial s_meta)
    if (tid == 0) {
        a.meta[0] = na;
        a.meta[1] = a.n - na;
        a.meta[2] = s_meta[0];
        a.meta[3] = s_meta[1];
        a.meta[4] = s_meta[2];
        a.meta[5] = s_meta[3];
    }
}

}  // namespace

hipError_t launch_split_active(const SplitArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(split_active_kernel, dim3(1), dim3(ST), 0, st, a);
    return hipGetLastError();
}

}  // namespace dr
