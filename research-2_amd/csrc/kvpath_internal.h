// Host-side declarations shared by the kvpath translation units: the argument blocks the
// kernels take by value, and the launchers each .hip file exports to the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvpath.h"

namespace kvpath {

// A cache member as the kernels see it (strides in elements, D stride 1).
struct CacheView {
    void* base;
    float* scale;  // fp8 only: f32[pages, 2, Hkv]
    int64_t num_pages, block, s_page, s_kv, s_row, s_head;
    int32_t hkv, d, dt;
};

struct AppendArgs {
    const void* k;
    const void* v;
    int64_t k_srow, k_shead, v_srow, v_shead;
    int32_t in_dt;
    CacheView c;
    const int32_t* slots;
    int64_t T;
};

struct GatherArgs {
    CacheView c;
    const int32_t* table;
    int64_t table_stride, R, width;
    void* out_k;
    void* out_v;
};

struct CopyArgs {
    CacheView c;
    const int32_t* src;
    const int32_t* dst;
    int64_t n;
};

// Everything the attention partition and reduce kernels read.
struct AttnArgs {
    const void* q;
    int64_t q_srow, q_shead;
    int32_t q_dt;
    CacheView c;
    const int32_t* row_request;
    const int32_t* qsl;
    const int32_t* seq_lens;
    const int32_t* table;
    int64_t table_stride, table_width;
    int32_t T, R, H, G;  // G = H / Hkv, q heads per kv head
    int32_t window, causal;
    const float* sinks;
    float score_scale_log2;  // log2(e) / sqrt(D)
    int32_t part;            // partition length in keys (multiple of 32): every entry's when
                             // part_fixed, else the floor of each entry's own split
    int32_t part_fixed;
    int32_t n_parts;         // partition slots per entry (the workspace's partition dimension)
    int32_t grid_parts;      // partition slots per entry in the grid: n_parts, or with a window
                             // only as many as one entry's window can reach, from its first
                             // visible key
    int32_t tile_groups;     // grid columns per partition (row tiles split across workgroups)
    // Partial outputs [n_parts, T, H, D]: with a bf16 q (part_bf16), each partition's output
    // normalized by its own sum and rounded to bf16 (the format vLLM's paged_attention_v2 and
    // FlashInfer's split-KV decode keep); otherwise un-normalized f32. Either way part_ml holds
    // (running max in log2 units, sum of weights) in f32.
    void* part_o;
    float* part_ml;          // [n_parts, T, H, 2]
    int32_t part_bf16;
    void* out;
    int64_t out_srow, out_shead;
    int32_t out_dt;
    // Fused append (bf16 k/v into a bf16 cache): this step's rows, read for the new keys and
    // written to the cache by the partition that holds them. k_new == nullptr: no append.
    const void* k_new;
    const void* v_new;
    int64_t kn_srow, kn_shead, vn_srow, vn_shead;
    const int32_t* slots;
    // Set by launch_attention when one partition holds every row's keys: the multi-row kernel
    // normalizes and writes `out` itself, an extra grid slice (z == R) zeroes the rows no entry
    // owns, and no reduce runs.
    int32_t direct;
    // The plan check (kvpath_plan::positions; nullptr: unchecked): the output writers write a row
    // that breaks the plan as NaN and set bit 0 of *status (nullptr: no status word).
    const int32_t* positions;
    int32_t* status;
    int32_t check_slots;     // also check a fused-append row's slot against its table slot
};

hipError_t launch_append(const AppendArgs& a, hipStream_t s);
hipError_t launch_append_fp8(const AppendArgs& a, hipStream_t s);
hipError_t launch_gather(const GatherArgs& a, hipStream_t s);
hipError_t launch_copy_blocks(const CopyArgs& a, hipStream_t s);
// Whether some attention kernel serves these dtypes, head dim, block size and alignments.
bool attention_supported(const AttnArgs& a);
// Returns hipErrorNotSupported (without launching) when attention_supported(a) is false.
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);  // partitions, then reduce
// Whether the partition kernels can take this step's append in (k_new).
bool attention_fuses(const AttnArgs& a);
// How a step's keys are split into partitions: `part` keys each (fixed) or each entry's own
// split with floor length `part` (split_entry, on the device), into at most `slots` per entry.
struct SplitChoice {
    int32_t part, slots, fixed;
};
// The split for a step of this shape; `partition` > 0 is a caller's fixed length.
SplitChoice choose_split(int64_t n_tokens, int64_t n_reqs, int64_t q_heads, int64_t kv_heads,
                         int64_t width, int64_t block, int32_t partition);
// The largest T * slots of any step with T <= max_tokens rows and R <= max_reqs entries of this
// shape (a workspace for it serves every such step; T * slots alone is not monotone in T or R).
int64_t max_token_slots(int64_t max_tokens, int64_t max_reqs, int64_t q_heads, int64_t kv_heads,
                        int64_t width, int64_t block, int32_t partition);
// Partition slots per entry the grid holds (AttnArgs::grid_parts): all `slots`, or with a window
// only as many as an entry's window reaches. The partition and reduce kernels both derive each
// entry's split from it, so it is set once with the rest of the arguments.
int32_t grid_slots(int32_t window, int64_t n_tokens, int32_t part, int32_t slots);
hipError_t launch_partitions(const AttnArgs& a, hipStream_t s);
hipError_t launch_reduce(const AttnArgs& a, hipStream_t s);

}  // namespace kvpath
