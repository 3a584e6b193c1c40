/*
 * kvpath.h -- C ABI of the MI355X (gfx950) paged-KV library `libkvpath.so`.
 *
 * The library implements Kelpie's paged-KV hot path: append this step's K/V rows into 16-token
 * pages through the int32 slot mapping (with optional e4m3 quantize-on-append), read pages
 * through the int32 block table, and paged attention for decode and for multi-row (DFlash
 * verify) steps.  Every entry point takes plain device pointers, element strides and sizes, and a
 * `hipStream_t`, launches asynchronously on that stream, never allocates, never synchronizes and
 * never reads device memory from the host, so every call can be captured in a hipGraph.
 *
 * Every entry point returns a status: KVPATH_OK (0), or a negative code with a message that
 * `kvpath_last_error()` returns (thread-local, valid until the next call on that thread).
 *
 * Reference interfaces replaced (arb8020/research-2, paths under kelpie/kelpie-models/kelpie_models):
 *   kvpath_kv_append          kernels/ops/paged_attention.py:44-54    write_kv
 *   kvpath_paged_attention    kernels/ops/paged_attention.py:67-140   paged_attention (op body)
 *   kvpath_attend             kernels/ops/paged_attention.py:160-183  _attend (+ :186-240 mask,
 *                                                                      softmax with sinks)
 *   kvpath_attend_partitions  + kvpath_attend_reduce: the two halves of kvpath_attend
 *   kvpath_kv_gather          kernels/ops/paged_attention.py:172-177  the gather inside _attend
 *   kvpath_copy_blocks        no counterpart (the reference never copies pages; the fork /
 *                             compaction primitive this library adds, bit-exact page copies)
 *   kvpath_workspace_bytes    no counterpart (the reference allocates its scratch inside torch;
 *                             here the caller allocates it, so graph capture sees no allocation)
 *   kvpath_workspace_bytes_max  the same, bounded over every step up to a bucket's size
 *   kvpath_split_plan         no counterpart in kelpie's op (it does not split a row's keys); the
 *                             per-sequence split follows kernels/vendored/cuda/vllm_attention/
 *                             triton_unified_attention.py:335-355
 *   kvpath_paged_attention_noalloc  no counterpart: the whole op for callers that cannot
 *                             allocate (see its declaration)
 */
#ifndef KVPATH_H
#define KVPATH_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A stream handle as HIP declares it (`hipStream_t` is `struct ihipStream_t*`). NULL is the
 * null stream. */
typedef struct ihipStream_t* kvpath_stream_t;

enum kvpath_status {
    KVPATH_OK = 0,
    KVPATH_EINVAL = -1,       /* an argument violates the contract (null pointer, shape, stride) */
    KVPATH_EUNSUPPORTED = -2, /* a valid case this library does not serve (caller may refuse it
                                 the way kelpie adapters do: NotImplementedError) */
    KVPATH_ELAUNCH = -3,      /* the HIP runtime refused a launch */
};

enum kvpath_dtype {
    KVPATH_F32 = 0,
    KVPATH_F16 = 1,
    KVPATH_BF16 = 2,
    KVPATH_FP8_E4M3 = 3, /* OCP e4m3fn (bias 7, max 448, 0x7f/0xff NaN, no infinities) */
};

/*
 * One layer's cache member, the view `kv_member` of shape [pages, 2, block, Hkv, D]
 * (kernels/ops/paged_attention.py:3-8; strides as sdk/kv.py:163-224 lays them out: page
 * stride = bytes_per_page, K/V stride = Hkv*D, row stride = the whole unit of all layers).
 * Strides are in elements of `dtype`; the D stride must be 1.  Offsets are computed in 64 bits.
 * `scale` is used only when dtype is KVPATH_FP8_E4M3: f32[pages, 2, Hkv] contiguous, the
 * per-(page, K/V, kv-head) dequant scale (value = e4m3 * scale).
 */
typedef struct kvpath_cache {
    void* base;
    int64_t num_pages, block_size, num_kv_heads, head_dim;
    int64_t stride_page, stride_kv, stride_row, stride_head;
    int32_t dtype;
    float* scale;
} kvpath_cache;

/* A [rows, heads, D] tensor (q, k, v or an output), D stride 1, strides in elements. */
typedef struct kvpath_rows {
    void* data;
    int64_t rows, heads, head_dim;
    int64_t stride_row, stride_head;
    int32_t dtype;
} kvpath_rows;

/*
 * The step's plan, exactly the int32 device tensors kelpie-core hands down
 * (sdk/device.py:62-78, kelpie-core/src/scheduler.zig:1330-1383, c_api.zig:1085-1153):
 *   row_request i32[T]  owning entry of each padded row, -1 for a pad row
 *   query_start_loc i32[R+1]  entry r owns rows [qsl[r], qsl[r+1]); pad entries are empty
 *   seq_lens i32[R]     context length of each entry including this step's rows
 *   block_table i32[R, P]  page ids, row stride `table_stride` (elements); 0 = null page
 *   slot_mapping i32[T] flat slot page*block + offset for each row's K/V
 *   positions i32[T]    each row's position (NULL: the plan is not checked)
 * The kernels derive a row's position as seq_lens[r] - rows_r + i (its entry's newest
 * positions).  With `positions` given, attention checks that invariant on every row, as
 * kernels/ops/paged_attention.py:128, 143-157 asserts it on every call: a row that names an
 * entry (row_request >= 0) must lie in that entry's rows, its entry's seq_len must fit the
 * table row, positions[t] must be seq_lens[r] - rows_r + (t - qsl[r]), and when the attention
 * launch appends the row itself (kvpath_paged_attention's fused append) and opts->check_slots
 * is set, slot_mapping[t] must be that position's slot in the entry's table row.  A row that
 * breaks the plan is written as NaN (every head) instead of its output, and bit 0 of
 * *opts->plan_status is set; nothing traps.  The position check adds no dependent load to the
 * output writers; the slot check adds one (a table read), so it is opt-in.
 */
typedef struct kvpath_plan {
    const int32_t* row_request;
    const int32_t* query_start_loc;
    const int32_t* seq_lens;
    const int32_t* block_table;
    const int32_t* slot_mapping;
    int64_t num_tokens, num_reqs, table_width, table_stride;
    const int32_t* positions;
} kvpath_plan;

/* Attention options: `window` > 0 keeps keys (pos - window, pos] (0: no window; negative is
 * refused with KVPATH_EINVAL); `sinks` is NULL or f32[H]
 * per-head sink logits (kernels/ops/paged_attention.py:215-240); `causal` = 0 lets every row
 * see its entry's whole context (the DFlash drafter). `partition_tokens` is a fixed split-KV
 * partition length for every entry, a multiple of 32; 0 lets the library split each entry by its
 * own length on the device (kvpath_split_plan).  `plan_status` is NULL or a device int32 that
 * the plan check ORs 1 into when a row breaks the plan (kvpath_plan; the caller clears it, and
 * reads it whenever it syncs); `check_slots` != 0 adds the fused append's slot check to it. */
typedef struct kvpath_attn_opts {
    int32_t window;
    const float* sinks;
    int32_t causal;
    int32_t partition_tokens;
    int32_t* plan_status;
    int32_t check_slots;
} kvpath_attn_opts;

/* Version of the ABI above (bumped on any change to a struct or signature). */
int32_t kvpath_abi_version(void);

/* The message of the last failing call on this thread ("" when none). */
const char* kvpath_last_error(void);

/*
 * KV append (replaces write_kv, kernels/ops/paged_attention.py:44-54):
 *   K[slot_mapping[t]] = k[t], V[slot_mapping[t]] = v[t] for t < plan->num_tokens,
 * converted to the cache dtype (round to nearest even).  With an fp8 cache, the rows are
 * quantized on append: for every page a step touches, the per-(page, K/V, kv-head) scale grows
 * to max(old, absmax(new rows)/448), rows already in the page are requantized to the new scale,
 * and a step that writes a page's row 0 starts the page afresh (old scale and rows discarded).
 * Only `slot_mapping` and `num_tokens` of `plan` are read.  Rows with a slot outside the pool are
 * skipped.  Rows of one step that share a page must be consecutive (true of every kelpie plan).
 */
int32_t kvpath_kv_append(const kvpath_cache* cache, const kvpath_rows* k, const kvpath_rows* v,
                         const kvpath_plan* plan, kvpath_stream_t stream);

/*
 * Gather (the gather inside _attend, kernels/ops/paged_attention.py:172-177):
 *   out_k[r, j] = K[block_table[r, j / block] * block + j % block] for j < width * block,
 * likewise V, for r < plan->num_reqs.  out_k and out_v are dense [R, width*block, Hkv, D] in the
 * cache dtype.  Bit-exact copies; a page id outside the pool yields zeros.
 */
int32_t kvpath_kv_gather(const kvpath_cache* cache, const kvpath_plan* plan, int64_t width,
                         void* out_k, void* out_v, kvpath_stream_t stream);

/*
 * copy_blocks: page dst[i] <- page src[i] for i < n_pairs, every row, K and V (and, for an fp8
 * cache, the page's scales).  dst ids must be distinct and disjoint from the src ids.
 */
int32_t kvpath_copy_blocks(const kvpath_cache* cache, const int32_t* src, const int32_t* dst,
                           int64_t n_pairs, kvpath_stream_t stream);

/*
 * How kvpath_attend splits a step's keys into split-KV partitions (no counterpart in kelpie's op,
 * which attends each row in one pass).  With partition_tokens 0 the library chooses from the
 * step's shape: each entry's keys (from its anchor: key 0, or with a window its first visible
 * key rounded down to 32) are cut on the device, from its own seq_len, into
 * min(slots, ceil(span / partition_tokens)) partitions of equal length rounded up to 32 keys, so
 * the split does not depend on how wide the block table is beyond the slots an entry could fill
 * (kelpie sizes tables for max_seq_len).  A decode step over a table of at most 768 keys gets
 * one slot: one partition per entry, written to `out` with no reduce.  With partition_tokens > 0
 * (a multiple of 32) every
 * partition has that length and slots = ceil(table_width * block / partition_tokens).
 */
typedef struct kvpath_split {
    int32_t partition_tokens; /* per_entry: the floor of each entry's length; else every one's */
    int32_t slots;            /* partitions per entry at most: the workspace's partition dim */
    int32_t per_entry;        /* 1: sized per entry on the device; 0: fixed length */
} kvpath_split;

int32_t kvpath_split_plan(int64_t num_tokens, int64_t num_reqs, int64_t num_heads,
                          int64_t kv_heads, int64_t table_width, int64_t block_size,
                          int32_t partition_tokens, kvpath_split* out);

/*
 * Scratch bytes kvpath_attend / kvpath_paged_attention need for a step of exactly this shape and
 * partition_tokens (the split-KV partials: per row, q head and partition slot, D values and 2
 * floats; sized for f32 values, which a bf16 q halves in use).  The size is per exact shape: it
 * does not grow monotonically with num_tokens or num_reqs (the split gives a step of more rows
 * fewer partition slots per entry), so a workspace sized for one step may be too small for a
 * smaller one; kvpath_workspace_bytes_max sizes one workspace for every step up to a bound.
 * -1 for a shape the library refuses: a negative size, num_tokens / table_width / block_size of
 * 2^31 or more (or a table spanning 2^31 keys), more than 65535 entries, more than 2^16 heads or
 * head dims, q heads not a multiple of kv heads, a partition that is not a multiple of 32.
 */
int64_t kvpath_workspace_bytes(int64_t num_tokens, int64_t num_reqs, int64_t num_heads,
                               int64_t kv_heads, int64_t head_dim, int64_t table_width,
                               int64_t block_size, int32_t partition_tokens);

/*
 * No counterpart in the reference (its scratch lives in torch's allocator).  Scratch bytes that
 * serve every step of at most max_tokens rows and max_reqs entries with these heads, head dim,
 * table width, block size and partition_tokens: the largest kvpath_workspace_bytes over those
 * steps, so a caller that allocates once for its largest bucket covers its smaller buckets too.
 * Non-decreasing in max_tokens and max_reqs.  Host arithmetic only (up to ~65 split choices per
 * entry count), -1 for a shape kvpath_workspace_bytes refuses.
 */
int64_t kvpath_workspace_bytes_max(int64_t max_tokens, int64_t max_reqs, int64_t num_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t table_width,
                                   int64_t block_size, int32_t partition_tokens);

/*
 * Attention only (replaces _attend and its mask/softmax, kernels/ops/paged_attention.py:
 * 160-240, over the whole plan): out[t] = softmax(q[t] K^T / sqrt(D) [+ sink]) V over the keys
 * row t may see; pad rows (row_request < 0) are written as exact zeros.  q and out are
 * [T, H, D]; H must be a multiple of the cache's Hkv.  `workspace` holds at least
 * kvpath_workspace_bytes(...) bytes.
 */
int32_t kvpath_attend(const kvpath_rows* q, const kvpath_cache* cache, const kvpath_plan* plan,
                      const kvpath_attn_opts* opts, kvpath_rows* out, void* workspace,
                      int64_t workspace_bytes, kvpath_stream_t stream);

/*
 * The two halves of kvpath_attend, for callers that schedule or time them apart (same
 * arguments; the partitions half does not read `out`).
 *   kvpath_attend_partitions  split-KV pass: for every row, q head and partition (as
 *                             kvpath_split_plan describes), the partial (o[D], max, sum) into
 *                             `workspace`; with a bf16 q, o is normalized by the partition's sum
 *                             and stored in bf16 (as vLLM's paged_attention_v2 keeps its
 *                             partials), else un-normalized f32 (vLLM's segment kernel,
 *                             kernels/vendored/cuda/vllm_attention/triton_unified_attention.py:
 *                             206-709, is the reference design point; kelpie's op has no split)
 *   kvpath_attend_reduce      combine each row's partitions (and the sink logit) into `out`;
 *                             pad rows exactly 0 (triton_unified_attention.py:712-800 likewise)
 */
int32_t kvpath_attend_partitions(const kvpath_rows* q, const kvpath_cache* cache,
                                 const kvpath_plan* plan, const kvpath_attn_opts* opts,
                                 void* workspace, int64_t workspace_bytes, kvpath_stream_t stream);

int32_t kvpath_attend_reduce(const kvpath_rows* q, const kvpath_cache* cache,
                             const kvpath_plan* plan, const kvpath_attn_opts* opts,
                             kvpath_rows* out, void* workspace, int64_t workspace_bytes,
                             kvpath_stream_t stream);

/*
 * The whole op (replaces paged_attention, kernels/ops/paged_attention.py:67-140): append k/v
 * at slot_mapping, then attend, on one stream. For a decode-shaped step of bf16 rows into a bf16
 * cache, or into an fp8 cache with 32 % block_size == 0, and for a verify- or drafter-sized step
 * (a few row tiles per entry) of bf16 rows into a bf16 cache, the append runs inside the
 * attention kernel with the same bytes, scales and output (pad rows are then not written to the
 * scratch slot, which nothing reads); that relies on each real row's slot_mapping being its
 * position's slot in its entry's block table, as the engine's plans give it.
 */
int32_t kvpath_paged_attention(const kvpath_rows* q, const kvpath_rows* k, const kvpath_rows* v,
                               const kvpath_cache* cache, const kvpath_plan* plan,
                               const kvpath_attn_opts* opts, kvpath_rows* out, void* workspace,
                               int64_t workspace_bytes, kvpath_stream_t stream);

/*
 * The whole op without a workspace argument.  No counterpart in the reference: it is for callers
 * that cannot allocate -- code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments and results as kvpath_paged_attention; the split-KV partials go to
 * the library's own 64 MiB device scratch (one per GPU, held until the process ends), so a step
 * whose kvpath_workspace_bytes exceeds 64 MiB is refused with KVPATH_EINVAL before any device
 * call.  No memory is allocated.  Every call on a GPU shares that GPU's scratch: calls that
 * overlap on one GPU (on different streams, or from different threads) race and must not.  The
 * scratch keeps the last call's partials; nothing in it needs to start at zero.
 */
int32_t kvpath_paged_attention_noalloc(const kvpath_rows* q, const kvpath_rows* k,
                                       const kvpath_rows* v, const kvpath_cache* cache,
                                       const kvpath_plan* plan, const kvpath_attn_opts* opts,
                                       kvpath_rows* out, kvpath_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KVPATH_H */
