// Native launch and graph capture of the whole op, with no Python and no torch: a C++ host
// program over the C ABI (include/kvpath.h) and the HIP runtime, as a non-Python caller (kelpie's
// Zig step loop, a C launcher) would drive it.
//
// One decode-shaped step (32 entries of 1 row, one pad row, 32/8 heads, D 128, 16-token pages) is
// captured once into a hipGraph -- a device-to-device restore of the pool, then
// kvpath_paged_attention (append + split-KV attention + reduce) -- and replayed on four plans of
// the same shape written into the captured plan buffers between replays (as kelpie rewrites its
// static plan tensors, sdk/captured.py). Each replay must equal an eager call on the same plan
// bit for bit, output and pool; the pad row must be exactly zero.
//
// Exit status: 0 pass, 1 fail, 77 no GPU (the test runner treats it as skipped).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kvpath.h"

namespace {

constexpr int kEntries = 32, kRows = kEntries + 1;  // one pad row
constexpr int kHeads = 32, kKvHeads = 8, kDim = 128, kBlock = 16;
constexpr int kPages = 4096, kWidth = 128;  // table width: 2048 keys
constexpr int kMinLen = 100, kMaxLen = 2000;  // 32 entries x at most 125 pages < 4095 pages
constexpr int kReplays = 4;

#define CHECK_HIP(x)                                                                     \
    do {                                                                                 \
        hipError_t err_ = (x);                                                           \
        if (err_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,               \
                         hipGetErrorString(err_));                                       \
            std::exit(1);                                                                \
        }                                                                                \
    } while (0)

#define CHECK_KV(x)                                                                      \
    do {                                                                                 \
        int32_t st_ = (x);                                                               \
        if (st_ != KVPATH_OK) {                                                          \
            std::fprintf(stderr, "%s:%d %s: status %d: %s\n", __FILE__, __LINE__, #x,    \
                         st_, kvpath_last_error());                                      \
            std::exit(1);                                                                \
        }                                                                                \
    } while (0)

struct Rng {  // splitmix64
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    int below(int n) { return static_cast<int>(next() % static_cast<uint64_t>(n)); }
    float unit() { return static_cast<float>((next() >> 40) * (1.0 / 16777216.0)) * 2.0f - 1.0f; }
};

uint16_t to_bf16(float f) {  // round to nearest even (finite inputs)
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

float from_bf16(uint16_t h) {
    const uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

struct Plan {
    std::vector<int32_t> row_request, qsl, seq_lens, table, slots;
};

// Entry r: context U[kMinLen, kMaxLen] including its new row, distinct random pages (none shared
// between entries, never the null page 0); the pad row writes page 0's last slot.
Plan make_plan(Rng& rng) {
    Plan p;
    p.row_request.resize(kRows);
    p.qsl.resize(kEntries + 2);
    p.seq_lens.resize(kEntries + 1);
    p.table.assign(static_cast<size_t>(kEntries + 1) * kWidth, 0);
    p.slots.resize(kRows);
    std::vector<int32_t> pages(kPages - 1);
    for (int i = 0; i < kPages - 1; ++i) pages[i] = i + 1;
    for (int i = kPages - 2; i > 0; --i) std::swap(pages[i], pages[rng.below(i + 1)]);
    int next_page = 0;
    for (int r = 0; r < kEntries; ++r) {
        const int len = kMinLen + rng.below(kMaxLen - kMinLen + 1);
        const int n_pages = (len + kBlock - 1) / kBlock;
        if (next_page + n_pages > kPages - 1 || n_pages > kWidth) {
            std::fprintf(stderr, "plan does not fit the pool\n");
            std::exit(1);
        }
        for (int j = 0; j < n_pages; ++j) p.table[static_cast<size_t>(r) * kWidth + j] = pages[next_page++];
        p.seq_lens[r] = len;
        p.qsl[r] = r;
        p.row_request[r] = r;
        const int pos = len - 1;
        p.slots[r] = p.table[static_cast<size_t>(r) * kWidth + pos / kBlock] * kBlock + pos % kBlock;
    }
    // Pad entry (empty query, seq_len 1, null table) and pad row (scratch slot of page 0).
    p.qsl[kEntries] = kEntries;
    p.qsl[kEntries + 1] = kEntries;
    p.seq_lens[kEntries] = 1;
    p.row_request[kEntries] = -1;
    p.slots[kEntries] = kBlock - 1;
    return p;
}

template <class T>
T* device_copy(const std::vector<T>& h) {
    T* d = nullptr;
    CHECK_HIP(hipMalloc(&d, h.size() * sizeof(T)));
    CHECK_HIP(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <class T>
void upload(T* d, const std::vector<T>& h) {
    CHECK_HIP(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
}

}  // namespace

int main() {
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || n_dev < 1) {
        std::printf("no GPU: skipped\n");
        return 77;
    }
    CHECK_HIP(hipSetDevice(0));
    Rng rng{2024};

    // Pool [pages, 2, block, Hkv, D] bf16, contiguous; a pristine copy restores it per step.
    const size_t pool_elems = static_cast<size_t>(kPages) * 2 * kBlock * kKvHeads * kDim;
    std::vector<uint16_t> pool_h(pool_elems);
    for (auto& x : pool_h) x = to_bf16(rng.unit());
    uint16_t* pristine = device_copy(pool_h);
    uint16_t *pool_g = nullptr, *pool_e = nullptr;
    CHECK_HIP(hipMalloc(&pool_g, pool_elems * 2));
    CHECK_HIP(hipMalloc(&pool_e, pool_elems * 2));

    std::vector<uint16_t> q_h(static_cast<size_t>(kRows) * kHeads * kDim), k_h(static_cast<size_t>(kRows) * kKvHeads * kDim),
        v_h(k_h.size());
    for (auto& x : q_h) x = to_bf16(rng.unit());
    for (auto& x : k_h) x = to_bf16(rng.unit());
    for (auto& x : v_h) x = to_bf16(rng.unit());
    uint16_t* q = device_copy(q_h);
    uint16_t* k = device_copy(k_h);
    uint16_t* v = device_copy(v_h);
    uint16_t *out_g = nullptr, *out_e = nullptr;
    CHECK_HIP(hipMalloc(&out_g, q_h.size() * 2));
    CHECK_HIP(hipMalloc(&out_e, q_h.size() * 2));

    Plan plan0 = make_plan(rng);
    int32_t* rr = device_copy(plan0.row_request);
    int32_t* qsl = device_copy(plan0.qsl);
    int32_t* lens = device_copy(plan0.seq_lens);
    int32_t* table = device_copy(plan0.table);
    int32_t* slots = device_copy(plan0.slots);

    auto cache_of = [&](uint16_t* pool) {
        kvpath_cache c{};
        c.base = pool;
        c.num_pages = kPages;
        c.block_size = kBlock;
        c.num_kv_heads = kKvHeads;
        c.head_dim = kDim;
        c.stride_kv = static_cast<int64_t>(kBlock) * kKvHeads * kDim;
        c.stride_page = 2 * c.stride_kv;
        c.stride_row = static_cast<int64_t>(kKvHeads) * kDim;
        c.stride_head = kDim;
        c.dtype = KVPATH_BF16;
        c.scale = nullptr;
        return c;
    };
    auto rows_of = [](void* data, int heads) {
        kvpath_rows r{};
        r.data = data;
        r.rows = kRows;
        r.heads = heads;
        r.head_dim = kDim;
        r.stride_row = static_cast<int64_t>(heads) * kDim;
        r.stride_head = kDim;
        r.dtype = KVPATH_BF16;
        return r;
    };
    kvpath_plan plan{};
    plan.row_request = rr;
    plan.query_start_loc = qsl;
    plan.seq_lens = lens;
    plan.block_table = table;
    plan.slot_mapping = slots;
    plan.num_tokens = kRows;
    plan.num_reqs = kEntries + 1;
    plan.table_width = kWidth;
    plan.table_stride = kWidth;
    kvpath_attn_opts opts{};  // no window, no sinks, causal, the library's partition
    opts.causal = 1;
    opts.partition_tokens = 0;
    const int64_t ws_bytes =
        kvpath_workspace_bytes(kRows, kEntries + 1, kHeads, kKvHeads, kDim, kWidth, kBlock, opts.partition_tokens);
    void *ws_g = nullptr, *ws_e = nullptr;
    CHECK_HIP(hipMalloc(&ws_g, ws_bytes));
    CHECK_HIP(hipMalloc(&ws_e, ws_bytes));

    kvpath_cache cache_g = cache_of(pool_g), cache_e = cache_of(pool_e);
    kvpath_rows qr = rows_of(q, kHeads), kr = rows_of(k, kKvHeads), vr = rows_of(v, kKvHeads);
    kvpath_rows og = rows_of(out_g, kHeads), oe = rows_of(out_e, kHeads);

    hipStream_t stream;
    CHECK_HIP(hipStreamCreate(&stream));
    // Capture: restore the pool (a copy node; no memset nodes), then the whole op.
    hipGraph_t graph;
    hipGraphExec_t exec;
    CHECK_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    CHECK_HIP(hipMemcpyAsync(pool_g, pristine, pool_elems * 2, hipMemcpyDeviceToDevice, stream));
    CHECK_KV(kvpath_paged_attention(&qr, &kr, &vr, &cache_g, &plan, &opts, &og, ws_g, ws_bytes, stream));
    CHECK_HIP(hipStreamEndCapture(stream, &graph));
    CHECK_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));

    std::vector<uint16_t> got(q_h.size()), want(q_h.size()), pg(pool_elems), pe(pool_elems);
    int failures = 0;
    for (int rep = 0; rep < kReplays; ++rep) {
        const Plan p = rep == 0 ? plan0 : make_plan(rng);
        upload(rr, p.row_request);
        upload(qsl, p.qsl);
        upload(lens, p.seq_lens);
        upload(table, p.table);
        upload(slots, p.slots);
        CHECK_HIP(hipGraphLaunch(exec, stream));
        CHECK_HIP(hipMemcpyAsync(pool_e, pristine, pool_elems * 2, hipMemcpyDeviceToDevice, stream));
        CHECK_KV(kvpath_paged_attention(&qr, &kr, &vr, &cache_e, &plan, &opts, &oe, ws_e, ws_bytes, stream));
        CHECK_HIP(hipStreamSynchronize(stream));
        CHECK_HIP(hipMemcpy(got.data(), out_g, got.size() * 2, hipMemcpyDeviceToHost));
        CHECK_HIP(hipMemcpy(want.data(), out_e, want.size() * 2, hipMemcpyDeviceToHost));
        CHECK_HIP(hipMemcpy(pg.data(), pool_g, pool_elems * 2, hipMemcpyDeviceToHost));
        CHECK_HIP(hipMemcpy(pe.data(), pool_e, pool_elems * 2, hipMemcpyDeviceToHost));
        const bool out_same = std::memcmp(got.data(), want.data(), got.size() * 2) == 0;
        const bool pool_same = std::memcmp(pg.data(), pe.data(), pool_elems * 2) == 0;
        bool pad_zero = true, finite = true;
        float max_abs = 0.0f;
        for (size_t i = 0; i < got.size(); ++i) {
            const float f = from_bf16(got[i]);
            if (i >= static_cast<size_t>(kEntries) * kHeads * kDim) pad_zero = pad_zero && got[i] == 0;
            finite = finite && std::isfinite(f);
            max_abs = std::fmax(max_abs, std::fabs(f));
        }
        // The appended rows landed: entry 0's new K row equals k[0] in the pool.
        const int32_t slot0 = p.slots[0];
        const size_t kpos = (static_cast<size_t>(slot0 / kBlock) * 2 * kBlock + slot0 % kBlock) * kKvHeads * kDim;
        const bool appended = std::memcmp(pg.data() + kpos, k_h.data(), kKvHeads * kDim * 2) == 0;
        if (!pool_same || !out_same) {  // where do they differ, and which matches the host's append?
            std::vector<uint16_t> expect(pool_h);
            for (int t = 0; t < kEntries; ++t) {
                const int32_t sl = p.slots[t];
                for (int m = 0; m < 2; ++m) {
                    const size_t base = ((static_cast<size_t>(sl / kBlock) * 2 + m) * kBlock + sl % kBlock) * kKvHeads * kDim;
                    std::memcpy(expect.data() + base, (m ? v_h : k_h).data() + static_cast<size_t>(t) * kKvHeads * kDim,
                                kKvHeads * kDim * 2);
                }
            }
            size_t dg = 0, de = 0, dge = 0, first = pool_elems;
            for (size_t i = 0; i < pool_elems; ++i) {
                dg += pg[i] != expect[i];
                de += pe[i] != expect[i];
                if (pg[i] != pe[i]) { ++dge; if (first == pool_elems) first = i; }
            }
            size_t dout = 0, first_out = got.size();
            for (size_t i = 0; i < got.size(); ++i) if (got[i] != want[i]) { ++dout; if (first_out == got.size()) first_out = i; }
            std::printf("  pool: graph vs host %zu, eager vs host %zu, graph vs eager %zu (first %zu); out diffs %zu (first %zu)\n",
                        dg, de, dge, first, dout, first_out);
        }
        const bool ok = out_same && pool_same && pad_zero && finite && appended && max_abs > 0.0f;
        std::printf("replay %d: out %s eager, pool %s eager, pad row %s, appended %s, max|out| %.4f: %s\n",
                    rep, out_same ? "==" : "!=", pool_same ? "==" : "!=", pad_zero ? "zero" : "NONZERO",
                    appended ? "yes" : "NO", max_abs, ok ? "ok" : "FAIL");
        failures += ok ? 0 : 1;
    }
    CHECK_HIP(hipGraphExecDestroy(exec));
    CHECK_HIP(hipGraphDestroy(graph));
    CHECK_HIP(hipStreamDestroy(stream));
    std::printf("%s\n", failures == 0 ? "PASS" : "FAIL");
    return failures == 0 ? 0 : 1;
}
