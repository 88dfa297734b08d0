// dr_internal.hpp -- kernel argument blocks and launcher declarations shared by
// the HIP kernels (attn_fwd.hip, kv_cache.hip) and the C ABI (dr_api.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dr {

// Key tiles are padded to this many rows in every K / V^T buffer, so a tile
// load never leaves the allocation.
constexpr int KEY_ALIGN = 64;
constexpr int MAX_BATCH = 8;

// One batch slot of an attention launch.  K is [n_head_kv][cap][HD] bf16
// (row = key index), VT is [n_head_kv][HD][cap] bf16 (V transposed so that a
// d-row holds consecutive keys).  Key index j has sequence position kpos[j]
// (kpos == nullptr: position j) and sequence id kseq[j] (nullptr: 0).
struct AttnSlot {
    const void* q;        // [nq][q_rstride] f32, head h at h*hd
    float* out;           // [nq][o_rstride] f32
    const int* qpos;      // [nq] sequence positions of the queries (device)
    const int* qseq;      // [nq] or nullptr
    const int* qprefix;   // [nq] per-row causal prefix or nullptr
    const uint16_t* k;    // bf16 bits
    const uint16_t* vt;   // bf16 bits
    const int* kpos;      // [nk] or nullptr
    const int* kseq;      // [nk] or nullptr
    int nq;
    int nk;
};

struct AttnArgs {
    AttnSlot slot[MAX_BATCH];
    int n_batch;
    int n_head, n_head_kv, group;  // group = n_head / n_head_kv
    int hd;                        // actual head_dim (<= the kernel's HD tile)
    int cap;                       // key capacity of K/VT (multiple of KEY_ALIGN)
    int q_rstride, o_rstride;      // elements between query / output rows
    float c;                       // scale * log2(e), folded into Q
    int window;                    // < 0: no sliding window
    int prefix;                    // < 0: no causal prefix (scalar)
    const float* qn_w;             // QK-norm gain for Q heads or nullptr
    float qn_eps;
    int rowgroups;                 // workgroup row groups per (batch, kv head)
    int n_split;                   // key splits; > 1 writes partials
    float* part_o;                 // split partial accumulators
    float* part_ml;                // split partial (max, sum)
};

// Row geometry used by both the attention and the combine kernel.
struct CombineArgs {
    AttnSlot slot[MAX_BATCH];
    int n_batch;
    int n_head_kv, group, hd;
    int o_rstride;
    int rowgroups;
    int n_split;
    const float* part_o;
    const float* part_ml;
};

struct StoreArgs {
    const float* k;      // [n][n_head_kv][hd] f32 rows
    const float* v;
    const int* pos;      // [n] destination positions (device); nullptr: row r -> r
    int n;
    int n_head_kv;
    int hd;              // actual head_dim (<= HD tile; tail zero-filled)
    int cap;
    uint16_t* kc;        // [n_head_kv][cap][HD] bf16 bits
    uint16_t* vtc;       // [n_head_kv][HD][cap] bf16 bits
    const float* kn_w;   // K-norm gain or nullptr
    float kn_eps;
};

struct GatherArgs {
    const uint16_t* kc;
    const uint16_t* vtc;
    const int* pos;      // [n] device
    int n;
    int n_head_kv;
    int hd;
    int cap;
    float* out_k;        // [n][n_head_kv][hd] f32
    float* out_v;
};

struct LaunchPlan {
    int hd_tile;     // 64, 128 or 256
    int block_n;     // keys per LDS tile
    int waves;       // waves per workgroup (32 query rows each)
    int n_split;
    int rowgroups;
    int n_workgroups;
    bool masked;
    bool qnorm;
};

// Chooses tile sizes and the key split for a problem on a device with n_cu
// compute units.  force_split > 0 overrides the split heuristic.
LaunchPlan plan_attention(int hd, int n_batch, int n_head_kv, int group, int max_nq, int max_nk,
                          bool masked, bool qnorm, int n_cu, int force_split);

// Bytes of split workspace a plan needs (part_o + part_ml).
size_t split_workspace_bytes(const LaunchPlan& p, int n_batch, int n_head_kv);

hipError_t launch_attention(const LaunchPlan& p, AttnArgs& a, hipStream_t st);
hipError_t launch_store(int hd_tile, const StoreArgs& a, hipStream_t st);
hipError_t launch_gather(int hd_tile, const GatherArgs& a, hipStream_t st);

}  // namespace dr
