// The C ABI (include/kvpath.h): argument validation, then the launches.
//
// Validation runs on the host from the shapes and strides alone -- no device memory is read, so
// a call stays asynchronous and capturable.  A violated contract returns KVPATH_EINVAL (or
// KVPATH_EUNSUPPORTED for a valid case no kernel serves) with a message, before any launch.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "kvpath_internal.h"

namespace {

// ---- the no-allocation entry point's scratch ---------------------------------------------------

// Split-KV partials of kvpath_paged_attention_noalloc: one file-scope device array, which each GPU
// the library runs on holds (64 MiB) until the process ends. Host code never passes `scratch`
// itself to a kernel or a copy -- in host code the name is a stand-in, not a device address --
// only the address hipGetSymbolAddress returns for the current device (scratch_ptr below).
constexpr int64_t kScratchBytes = int64_t{64} << 20;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device (with that device
// current) and kept. Returns a HIP error when the device or the lookup fails.
// The first call on a device may come while a stream is being captured (the entry point is for
// code under hipGraph capture). The lookup is no stream operation, but it may load the code
// object that holds `scratch`, which a capture in global or thread-local mode forbids; so this
// thread's capture mode is relaxed for the lookup alone and restored after it, which leaves the
// capture valid and records nothing into it.
hipError_t scratch_ptr(void** out) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        err = hipThreadExchangeStreamCaptureMode(&mode);
        if (err != hipSuccess) return err;
        void* p = nullptr;
        const hipError_t lookup = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        err = hipThreadExchangeStreamCaptureMode(&mode);
        if (lookup != hipSuccess) return lookup;
        if (err != hipSuccess) return err;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

thread_local std::string g_error;

int32_t fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int32_t ok() {
    g_error.clear();
    return KVPATH_OK;
}

int32_t launched(hipError_t err, const char* what) {
    if (err == hipSuccess) return ok();
    if (err == hipErrorNotSupported)
        return fail(KVPATH_EUNSUPPORTED, "%s: no kernel serves this shape/dtype", what);
    return fail(KVPATH_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
}

bool valid_dtype(int32_t dt) { return dt >= KVPATH_F32 && dt <= KVPATH_FP8_E4M3; }

// Head counts and head dims beyond this are refused, so every product below stays in int64 and
// the kernels' int32 fields hold them.
constexpr int64_t kMaxHeads = 1 << 16, kMaxDim = 1 << 16;

int32_t check_cache(const kvpath_cache* c, const char* what, kvpath::CacheView* out) {
    if (c == nullptr || c->base == nullptr) return fail(KVPATH_EINVAL, "%s: null cache", what);
    if (!valid_dtype(c->dtype)) return fail(KVPATH_EINVAL, "%s: bad cache dtype %d", what, c->dtype);
    if (c->num_pages < 1 || c->block_size < 1 || c->num_kv_heads < 1 || c->head_dim < 1)
        return fail(KVPATH_EINVAL, "%s: cache dims must be positive (pages %lld block %lld Hkv %lld D %lld)",
                    what, (long long)c->num_pages, (long long)c->block_size,
                    (long long)c->num_kv_heads, (long long)c->head_dim);
    if (c->stride_page < 0 || c->stride_kv < 0 || c->stride_row < 0 || c->stride_head < 0)
        return fail(KVPATH_EINVAL, "%s: negative cache stride", what);
    if (c->num_kv_heads > kMaxHeads || c->head_dim > kMaxDim)
        return fail(KVPATH_EINVAL, "%s: %lld kv heads of dim %lld exceed %lld / %lld", what,
                    (long long)c->num_kv_heads, (long long)c->head_dim, (long long)kMaxHeads,
                    (long long)kMaxDim);
    if (c->num_pages >= (1ll << 31) || c->block_size >= (1ll << 31) ||
        c->num_pages * c->block_size >= (1ll << 31))
        return fail(KVPATH_EINVAL, "%s: %lld pages of %lld slots do not fit the int32 slot mapping",
                    what, (long long)c->num_pages, (long long)c->block_size);
    if (c->dtype == KVPATH_FP8_E4M3 && c->scale == nullptr)
        return fail(KVPATH_EINVAL, "%s: an fp8 cache needs its scale tensor", what);
    out->base = c->base;
    out->scale = c->dtype == KVPATH_FP8_E4M3 ? c->scale : nullptr;
    out->num_pages = c->num_pages;
    out->block = c->block_size;
    out->s_page = c->stride_page;
    out->s_kv = c->stride_kv;
    out->s_row = c->stride_row;
    out->s_head = c->stride_head;
    out->hkv = static_cast<int32_t>(c->num_kv_heads);
    out->d = static_cast<int32_t>(c->head_dim);
    out->dt = c->dtype;
    return KVPATH_OK;
}

int32_t check_rows(const kvpath_rows* x, const char* name, const char* what, int64_t rows,
                   int64_t heads, int64_t dim, bool allow_fp8) {
    if (x == nullptr) return fail(KVPATH_EINVAL, "%s: %s is null", what, name);
    if (!valid_dtype(x->dtype) || (!allow_fp8 && x->dtype == KVPATH_FP8_E4M3))
        return fail(KVPATH_EINVAL, "%s: %s has bad dtype %d", what, name, x->dtype);
    if (x->rows != rows || (heads >= 0 && x->heads != heads) || x->head_dim != dim)
        return fail(KVPATH_EINVAL, "%s: %s is [%lld, %lld, %lld], want [%lld, %lld, %lld]", what,
                    name, (long long)x->rows, (long long)x->heads, (long long)x->head_dim,
                    (long long)rows, (long long)heads, (long long)dim);
    if (rows > 0 && x->data == nullptr) return fail(KVPATH_EINVAL, "%s: %s data is null", what, name);
    if (x->stride_row < 0 || x->stride_head < 0)
        return fail(KVPATH_EINVAL, "%s: %s has a negative stride", what, name);
    return KVPATH_OK;
}

struct WorkspaceLayout {
    int64_t o_bytes, ml_offset, total;
};

// The split-KV workspace: f32-sized partials [slots, T, H, D], then (m, l) [slots, T, H, 2].
// total is -1 when a size overflows int64 (the caller refuses the call). Takes T below 2^31 and
// H, D below 2^16.
WorkspaceLayout workspace_layout(int64_t T, int64_t H, int64_t D, int64_t slots) {
    WorkspaceLayout w{0, 0, -1};
    int64_t rows, o_vals, ml_vals;
    if (__builtin_mul_overflow(T * H, slots, &rows) || __builtin_mul_overflow(rows, D * 4, &o_vals) ||
        __builtin_mul_overflow(rows, static_cast<int64_t>(8), &ml_vals) ||
        o_vals > (int64_t{1} << 62) || ml_vals > (int64_t{1} << 62))
        return w;
    w.o_bytes = o_vals;
    w.ml_offset = (w.o_bytes + 255) / 256 * 256;
    w.total = w.ml_offset + ml_vals;
    return w;
}

// The shape limits every attention entry point and size query shares: sizes below 2^31 (a
// table spanning fewer than 2^31 keys), heads and head dims up to 2^16, a partition length that
// is a multiple of 32 (0: the library's choice). Returns a message, or nullptr when the shape is
// acceptable.
const char* shape_problem(int64_t T, int64_t R, int64_t H, int64_t hkv, int64_t D, int64_t width,
                          int64_t block, int32_t partition) {
    if (T < 0 || R < 0 || H < 0 || hkv < 0 || D < 0 || width < 0 || block < 1)
        return "negative or zero size";
    if (T >= (1ll << 31) || R > 65535) return "plan too large";
    if (H > kMaxHeads || hkv > kMaxHeads || D > kMaxDim) return "too many heads or head dims";
    if (width >= (1ll << 31) || block >= (1ll << 31) || width * block >= (1ll << 31))
        return "table spans too many keys";
    if (partition < 0 || partition % 32 != 0) return "partition_tokens is not a multiple of 32";
    return nullptr;
}

// Validates an append and fills its kernel arguments; launches nothing.
int32_t append_args(const kvpath::CacheView& c, const kvpath_rows* k, const kvpath_rows* v,
                    const kvpath_plan* plan, const char* what, kvpath::AppendArgs* out) {
    if (plan == nullptr) return fail(KVPATH_EINVAL, "%s: null plan", what);
    const int64_t T = plan->num_tokens;
    if (T < 0) return fail(KVPATH_EINVAL, "%s: negative num_tokens", what);
    int32_t st;
    if ((st = check_rows(k, "k", what, T, c.hkv, c.d, false)) != KVPATH_OK) return st;
    if ((st = check_rows(v, "v", what, T, c.hkv, c.d, false)) != KVPATH_OK) return st;
    if (k->dtype != v->dtype) return fail(KVPATH_EINVAL, "%s: k and v dtypes differ", what);
    if (T > 0 && plan->slot_mapping == nullptr) return fail(KVPATH_EINVAL, "%s: null slot_mapping", what);
    if (T > (1ll << 31) - 1) return fail(KVPATH_EINVAL, "%s: too many rows", what);
    if (c.dt == KVPATH_FP8_E4M3 && c.block > 64)
        return fail(KVPATH_EUNSUPPORTED, "%s: fp8 append supports block <= 64, got %lld", what,
                    (long long)c.block);
    kvpath::AppendArgs& a = *out;
    a = kvpath::AppendArgs{};
    a.k = k->data;
    a.v = v->data;
    a.k_srow = k->stride_row;
    a.k_shead = k->stride_head;
    a.v_srow = v->stride_row;
    a.v_shead = v->stride_head;
    a.in_dt = k->dtype;
    a.c = c;
    a.slots = plan->slot_mapping;
    a.T = T;
    return KVPATH_OK;
}

int32_t append_launch(const kvpath::AppendArgs& a, hipStream_t stream, const char* what) {
    const hipError_t err = a.c.dt == KVPATH_FP8_E4M3 ? kvpath::launch_append_fp8(a, stream)
                                                     : kvpath::launch_append(a, stream);
    return launched(err, what);
}

int32_t append_impl(const kvpath::CacheView& c, const kvpath_rows* k, const kvpath_rows* v,
                    const kvpath_plan* plan, hipStream_t stream, const char* what) {
    kvpath::AppendArgs a;
    int32_t st = append_args(c, k, v, plan, what, &a);
    if (st != KVPATH_OK) return st;
    return append_launch(a, stream, what);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Whether this step's append can run inside the attention kernel: bf16 rows, 16-byte aligned,
// into a bf16 cache (16-byte chunks) or an fp8 one (8-byte e4m3 chunks), on the decode-shaped
// path.
bool append_fuses(const kvpath::AppendArgs& ap, const kvpath::AttnArgs& a) {
    const bool cache_ok = a.c.dt == KVPATH_BF16 ||
                          (a.c.dt == KVPATH_FP8_E4M3 && a.c.scale != nullptr &&
                           (reinterpret_cast<uintptr_t>(a.c.base) & 7) == 0);
    return cache_ok && ap.in_dt == KVPATH_BF16 && ap.T == a.T && aligned16(ap.k) &&
           aligned16(ap.v) && ap.k_srow % 8 == 0 && ap.k_shead % 8 == 0 && ap.v_srow % 8 == 0 &&
           ap.v_shead % 8 == 0 && (a.c.s_page % 8 == 0) && (a.c.s_row % 8 == 0) &&
           (a.c.s_kv % 8 == 0) && (a.c.s_head % 8 == 0) && kvpath::attention_fuses(a);
}

// Validates an attention call and fills its kernel arguments; launches nothing.
int32_t attend_args(const kvpath_rows* q, const kvpath::CacheView& c, const kvpath_plan* plan,
                    const kvpath_attn_opts* opts, kvpath_rows* out, void* ws, int64_t ws_bytes,
                    const char* what, kvpath::AttnArgs* args, bool allow_null_out = false) {
    if (plan == nullptr) return fail(KVPATH_EINVAL, "%s: null plan", what);
    const int64_t T = plan->num_tokens, R = plan->num_reqs;
    if (T < 0 || R < 0) return fail(KVPATH_EINVAL, "%s: negative plan size", what);
    int32_t st;
    if ((st = check_rows(q, "q", what, T, -1, c.d, false)) != KVPATH_OK) return st;
    const int64_t H = q->heads;
    if (H > kMaxHeads)
        return fail(KVPATH_EINVAL, "%s: %lld q heads exceed %lld", what, (long long)H, (long long)kMaxHeads);
    if (H < 1 || H % c.hkv != 0)
        return fail(KVPATH_EINVAL, "%s: %lld q heads is not a multiple of %d kv heads", what,
                    (long long)H, c.hkv);
    if (out != nullptr || !allow_null_out)
        if ((st = check_rows(out, "out", what, T, H, c.d, false)) != KVPATH_OK) return st;
    if (T == 0) {
        *args = kvpath::AttnArgs{};
        return ok();
    }
    if (R < 1) return fail(KVPATH_EINVAL, "%s: rows but no entries", what);
    if (plan->row_request == nullptr || plan->query_start_loc == nullptr ||
        plan->seq_lens == nullptr || plan->block_table == nullptr)
        return fail(KVPATH_EINVAL, "%s: null plan tensor", what);
    if (plan->table_width < 1 || plan->table_stride < plan->table_width)
        return fail(KVPATH_EINVAL, "%s: block table width %lld / stride %lld", what,
                    (long long)plan->table_width, (long long)plan->table_stride);
    // Entries index the partition grid's z dimension (at most 65535).
    if (T > (1ll << 31) - 1 || R > 65535)
        return fail(KVPATH_EINVAL, "%s: plan too large", what);
    const int32_t req_part = opts ? opts->partition_tokens : 0;
    if (req_part < 0 || req_part % 32 != 0)
        return fail(KVPATH_EINVAL, "%s: partition_tokens %d is not a multiple of 32", what, req_part);
    if (plan->table_width >= (1ll << 31) || plan->table_width * c.block >= (1ll << 31))
        return fail(KVPATH_EINVAL, "%s: table spans too many keys", what);
    const kvpath::SplitChoice split =
        kvpath::choose_split(T, R, H, c.hkv, plan->table_width, c.block, req_part);
    // The grid's x dimension holds partition slots x row-tile groups (at most 64).
    if (static_cast<int64_t>(split.slots) * 64 >= (1ll << 31))
        return fail(KVPATH_EINVAL, "%s: table spans too many keys", what);
    if (opts && opts->window < 0)
        return fail(KVPATH_EINVAL, "%s: negative window %d", what, opts->window);
    const WorkspaceLayout w = workspace_layout(T, H, c.d, split.slots);
    if (w.total < 0) return fail(KVPATH_EINVAL, "%s: workspace size overflows", what);
    if (ws == nullptr || ws_bytes < w.total)
        return fail(KVPATH_EINVAL, "%s: workspace of %lld bytes, need %lld", what,
                    (long long)ws_bytes, (long long)w.total);
    if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0)
        return fail(KVPATH_EINVAL, "%s: workspace must be 256-byte aligned", what);
    kvpath::AttnArgs& a = *args;
    a = kvpath::AttnArgs{};
    a.q = q->data;
    a.q_srow = q->stride_row;
    a.q_shead = q->stride_head;
    a.q_dt = q->dtype;
    a.c = c;
    a.row_request = plan->row_request;
    a.qsl = plan->query_start_loc;
    a.seq_lens = plan->seq_lens;
    a.table = plan->block_table;
    a.table_stride = plan->table_stride;
    a.table_width = plan->table_width;
    a.T = static_cast<int32_t>(T);
    a.R = static_cast<int32_t>(R);
    a.H = static_cast<int32_t>(H);
    a.G = static_cast<int32_t>(H / c.hkv);
    a.window = opts ? opts->window : 0;
    a.causal = opts ? (opts->causal != 0) : 1;
    a.sinks = opts ? opts->sinks : nullptr;
    a.positions = plan->positions;
    a.status = opts ? opts->plan_status : nullptr;
    a.check_slots = opts ? (opts->check_slots != 0) : 0;
    a.score_scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(c.d)));
    a.part = split.part;
    a.part_fixed = split.fixed;
    a.n_parts = split.slots;
    a.grid_parts = kvpath::grid_slots(a.window, T, split.part, split.slots);
    a.tile_groups = 1;
    a.part_o = ws;
    // The partial format follows q alone, so kvpath_attend_partitions and kvpath_attend_reduce
    // always agree on it (the workspace is sized for f32 partials either way).
    a.part_bf16 = q->dtype == KVPATH_BF16 ? 1 : 0;
    a.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + w.ml_offset);
    if (out != nullptr) {
        a.out = out->data;
        a.out_srow = out->stride_row;
        a.out_shead = out->stride_head;
        a.out_dt = out->dtype;
    }
    if (!kvpath::attention_supported(a))
        return fail(KVPATH_EUNSUPPORTED,
                    "%s: no kernel serves q dtype %d with cache dtype %d, D %d, block %lld", what,
                    a.q_dt, c.dt, c.d, (long long)c.block);
    return ok();
}

// The whole op over a given workspace: validate the attention half before the append launches,
// so a refused call writes nothing; fuse the append into the partition kernels when they take it.
int32_t paged_attention_impl(const kvpath_rows* q, const kvpath_rows* k, const kvpath_rows* v,
                             const kvpath_cache* cache, const kvpath_plan* plan,
                             const kvpath_attn_opts* opts, kvpath_rows* out, void* workspace,
                             int64_t workspace_bytes, kvpath_stream_t stream, const char* what) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, what, &c);
    if (st != KVPATH_OK) return st;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    kvpath::AttnArgs a;
    if ((st = attend_args(q, c, plan, opts, out, workspace, workspace_bytes, what, &a)) != KVPATH_OK)
        return st;
    kvpath::AppendArgs ap;
    if ((st = append_args(c, k, v, plan, what, &ap)) != KVPATH_OK) return st;
    if (a.T > 0 && append_fuses(ap, a)) {
        // One launch: the partitions that hold this step's rows write them.
        a.k_new = ap.k;
        a.v_new = ap.v;
        a.kn_srow = ap.k_srow;
        a.kn_shead = ap.k_shead;
        a.vn_srow = ap.v_srow;
        a.vn_shead = ap.v_shead;
        a.slots = ap.slots;
    } else if ((st = append_launch(ap, s, what)) != KVPATH_OK) {
        return st;
    }
    return launched(kvpath::launch_attention(a, s), what);
}

}  // namespace

extern "C" {

int32_t kvpath_abi_version(void) { return 4; }

const char* kvpath_last_error(void) { return g_error.c_str(); }

int32_t kvpath_kv_append(const kvpath_cache* cache, const kvpath_rows* k, const kvpath_rows* v,
                         const kvpath_plan* plan, kvpath_stream_t stream) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, "kv_append", &c);
    if (st != KVPATH_OK) return st;
    return append_impl(c, k, v, plan, reinterpret_cast<hipStream_t>(stream), "kv_append");
}

int32_t kvpath_kv_gather(const kvpath_cache* cache, const kvpath_plan* plan, int64_t width,
                         void* out_k, void* out_v, kvpath_stream_t stream) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, "kv_gather", &c);
    if (st != KVPATH_OK) return st;
    if (plan == nullptr || plan->num_reqs < 0) return fail(KVPATH_EINVAL, "kv_gather: bad plan");
    if (width < 0 || width > plan->table_width || plan->table_stride < plan->table_width)
        return fail(KVPATH_EINVAL, "kv_gather: width %lld outside the table (%lld)",
                    (long long)width, (long long)plan->table_width);
    if (plan->num_reqs > 0 && width > 0 &&
        (plan->block_table == nullptr || out_k == nullptr || out_v == nullptr))
        return fail(KVPATH_EINVAL, "kv_gather: null pointer");
    kvpath::GatherArgs a{};
    a.c = c;
    a.table = plan->block_table;
    a.table_stride = plan->table_stride;
    a.R = plan->num_reqs;
    a.width = width;
    a.out_k = out_k;
    a.out_v = out_v;
    return launched(kvpath::launch_gather(a, reinterpret_cast<hipStream_t>(stream)), "kv_gather");
}

int32_t kvpath_copy_blocks(const kvpath_cache* cache, const int32_t* src, const int32_t* dst,
                           int64_t n_pairs, kvpath_stream_t stream) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, "copy_blocks", &c);
    if (st != KVPATH_OK) return st;
    if (n_pairs < 0) return fail(KVPATH_EINVAL, "copy_blocks: negative pair count");
    if (n_pairs > 0 && (src == nullptr || dst == nullptr))
        return fail(KVPATH_EINVAL, "copy_blocks: null pair list");
    kvpath::CopyArgs a{};
    a.c = c;
    a.src = src;
    a.dst = dst;
    a.n = n_pairs;
    return launched(kvpath::launch_copy_blocks(a, reinterpret_cast<hipStream_t>(stream)),
                    "copy_blocks");
}

int32_t kvpath_split_plan(int64_t num_tokens, int64_t num_reqs, int64_t num_heads,
                          int64_t kv_heads, int64_t table_width, int64_t block_size,
                          int32_t partition_tokens, kvpath_split* out) {
    if (out == nullptr) return fail(KVPATH_EINVAL, "split_plan: null output");
    if (const char* why = shape_problem(num_tokens, num_reqs, num_heads, kv_heads, 1, table_width,
                                        block_size, partition_tokens))
        return fail(KVPATH_EINVAL, "split_plan: %s", why);
    if (kv_heads < 1 || num_heads % kv_heads != 0)
        return fail(KVPATH_EINVAL, "split_plan: %lld q heads is not a multiple of %lld kv heads",
                    (long long)num_heads, (long long)kv_heads);
    const kvpath::SplitChoice sp = kvpath::choose_split(num_tokens, num_reqs, num_heads, kv_heads,
                                                        table_width, block_size, partition_tokens);
    out->partition_tokens = sp.part;
    out->slots = sp.slots;
    out->per_entry = sp.fixed ? 0 : 1;
    return ok();
}

int64_t kvpath_workspace_bytes(int64_t num_tokens, int64_t num_reqs, int64_t num_heads,
                               int64_t kv_heads, int64_t head_dim, int64_t table_width,
                               int64_t block_size, int32_t partition_tokens) {
    if (shape_problem(num_tokens, num_reqs, num_heads, kv_heads, head_dim, table_width, block_size,
                      partition_tokens) != nullptr ||
        kv_heads < 1 || num_heads % kv_heads != 0)
        return -1;
    const kvpath::SplitChoice sp = kvpath::choose_split(num_tokens, num_reqs, num_heads, kv_heads,
                                                        table_width, block_size, partition_tokens);
    return workspace_layout(num_tokens, num_heads, head_dim, sp.slots).total;
}

int64_t kvpath_workspace_bytes_max(int64_t max_tokens, int64_t max_reqs, int64_t num_heads,
                                   int64_t kv_heads, int64_t head_dim, int64_t table_width,
                                   int64_t block_size, int32_t partition_tokens) {
    if (shape_problem(max_tokens, max_reqs, num_heads, kv_heads, head_dim, table_width, block_size,
                      partition_tokens) != nullptr ||
        kv_heads < 1 || num_heads % kv_heads != 0)
        return -1;
    const int64_t token_slots = kvpath::max_token_slots(max_tokens, max_reqs, num_heads, kv_heads,
                                                        table_width, block_size, partition_tokens);
    // T * H * slots partial rows at most: the layout of one row with that many slots bounds every
    // step's (its sizes grow with T * slots alone).
    return workspace_layout(1, num_heads, head_dim, token_slots).total;
}

int32_t kvpath_attend(const kvpath_rows* q, const kvpath_cache* cache, const kvpath_plan* plan,
                      const kvpath_attn_opts* opts, kvpath_rows* out, void* workspace,
                      int64_t workspace_bytes, kvpath_stream_t stream) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, "attend", &c);
    if (st != KVPATH_OK) return st;
    kvpath::AttnArgs a;
    if ((st = attend_args(q, c, plan, opts, out, workspace, workspace_bytes, "attend", &a)) != KVPATH_OK)
        return st;
    return launched(kvpath::launch_attention(a, reinterpret_cast<hipStream_t>(stream)), "attend");
}

int32_t kvpath_attend_partitions(const kvpath_rows* q, const kvpath_cache* cache,
                                 const kvpath_plan* plan, const kvpath_attn_opts* opts,
                                 void* workspace, int64_t workspace_bytes, kvpath_stream_t stream) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, "attend_partitions", &c);
    if (st != KVPATH_OK) return st;
    kvpath::AttnArgs a;
    if ((st = attend_args(q, c, plan, opts, nullptr, workspace, workspace_bytes,
                          "attend_partitions", &a, true)) != KVPATH_OK)
        return st;
    return launched(kvpath::launch_partitions(a, reinterpret_cast<hipStream_t>(stream)),
                    "attend_partitions");
}

int32_t kvpath_attend_reduce(const kvpath_rows* q, const kvpath_cache* cache,
                             const kvpath_plan* plan, const kvpath_attn_opts* opts,
                             kvpath_rows* out, void* workspace, int64_t workspace_bytes,
                             kvpath_stream_t stream) {
    kvpath::CacheView c;
    int32_t st = check_cache(cache, "attend_reduce", &c);
    if (st != KVPATH_OK) return st;
    kvpath::AttnArgs a;
    if ((st = attend_args(q, c, plan, opts, out, workspace, workspace_bytes, "attend_reduce", &a)) !=
        KVPATH_OK)
        return st;
    return launched(kvpath::launch_reduce(a, reinterpret_cast<hipStream_t>(stream)),
                    "attend_reduce");
}

int32_t kvpath_paged_attention(const kvpath_rows* q, const kvpath_rows* k, const kvpath_rows* v,
                               const kvpath_cache* cache, const kvpath_plan* plan,
                               const kvpath_attn_opts* opts, kvpath_rows* out, void* workspace,
                               int64_t workspace_bytes, kvpath_stream_t stream) {
    return paged_attention_impl(q, k, v, cache, plan, opts, out, workspace, workspace_bytes, stream,
                                "paged_attention");
}

int32_t kvpath_paged_attention_noalloc(const kvpath_rows* q, const kvpath_rows* k,
                                       const kvpath_rows* v, const kvpath_cache* cache,
                                       const kvpath_plan* plan, const kvpath_attn_opts* opts,
                                       kvpath_rows* out, kvpath_stream_t stream) {
    const char* what = "paged_attention_noalloc";
    // The step's workspace size first, from the shapes alone: a step that needs more than the
    // scratch holds is refused before any device call.
    if (q == nullptr || cache == nullptr || plan == nullptr)
        return fail(KVPATH_EINVAL, "%s: null argument", what);
    const int64_t need = kvpath_workspace_bytes(plan->num_tokens, plan->num_reqs, q->heads,
                                                cache->num_kv_heads, cache->head_dim,
                                                plan->table_width, cache->block_size,
                                                opts ? opts->partition_tokens : 0);
    if (need < 0)
        return fail(KVPATH_EINVAL, "%s: a shape the library refuses (see kvpath_workspace_bytes)",
                    what);
    if (need > kScratchBytes)
        return fail(KVPATH_EINVAL,
                    "%s: this step needs %lld bytes of split-KV scratch, more than the %lld the "
                    "no-allocation entry point holds; call kvpath_paged_attention with a workspace",
                    what, (long long)need, (long long)kScratchBytes);
    void* ws = nullptr;
    const hipError_t err = scratch_ptr(&ws);
    if (err != hipSuccess)
        return fail(KVPATH_ELAUNCH, "%s: the scratch's device address: %s", what,
                    hipGetErrorString(err));
    return paged_attention_impl(q, k, v, cache, plan, opts, out, ws, kScratchBytes, stream, what);
}

}  // extern "C"
