// torch.ops.kvpath.paged_attention and paged_attention_fp8 -- kelpie's op
// (kelpie/kelpie-models/kelpie_models/kernels/ops/paged_attention.py:67-140) -- and write_kv /
// write_kv_fp8 (its append, :44-54, which DFlash's context injection also calls,
// models/torch/dflash.py:197), registered with the torch dispatcher in C++ over the C ABI of
// libkvpath.so (include/kvpath.h).
//
// An eager call from Python then costs the dispatcher's argument handling plus this file's
// checks and one C-ABI call, with no Python frame between the caller and the launch (kelpie runs
// prefill eagerly, sdk/captured.py:13-17, so this is paid once per layer per prefill step).
// The argument contract, error types and messages are those of the Python layer it replaces
// (research-2_amd/kvpath/paged_attention.py): tensors on one ROCm device (no CPU path), int32
// plan tensors, `sinks` empty or f32[H], an fp8 member with its f32[pages, 2, Hkv] scales; a
// case no kernel serves raises NotImplementedError (kelpie's refusal convention,
// kernels/adapters/paged_attention_vllm.py:69-74), a broken contract ValueError or RuntimeError.
// The op is inference-only, as kelpie's is (ops/paged_attention.py:380-385): its Autograd kernel
// runs it below autograd and, when an input requires grad, gives the output a node whose backward
// raises NotImplementedError.
#include <ATen/ATen.h>
#include <c10/hip/HIPException.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/function.h>
#include <torch/csrc/autograd/functions/utils.h>
#include <torch/csrc/autograd/variable.h>
#include <torch/library.h>

#include <array>
#include <atomic>
#include <mutex>

#include "../../include/kvpath.h"

namespace {

constexpr int64_t kMembers = 2;

int32_t dtype_code(const at::Tensor& t, const char* what) {
    switch (t.scalar_type()) {
        case at::kFloat: return KVPATH_F32;
        case at::kHalf: return KVPATH_F16;
        case at::kBFloat16: return KVPATH_BF16;
        case at::kFloat8_e4m3fn: return KVPATH_FP8_E4M3;
        default:
            TORCH_CHECK_NOT_IMPLEMENTED(false, "kvpath: ", what, " dtype ", t.scalar_type(),
                                        " (serves f32, f16, bf16, float8_e4m3fn caches)");
    }
}

// Every tensor on the same ROCm device; returns it.
at::Device one_device(std::initializer_list<const at::Tensor*> tensors) {
    const at::Device dev = (*tensors.begin())->device();
    for (const at::Tensor* t : tensors)
        TORCH_CHECK(t->device().is_cuda() && t->device() == dev,
                    "kvpath: every tensor must be on one ROCm device, got ", t->device(), " (and ",
                    dev, "); there is no CPU path");
    return dev;
}

kvpath_cache cache_of(const at::Tensor& m, const at::Tensor* scale) {
    TORCH_CHECK_VALUE(m.dim() == 5 && m.size(1) == kMembers,
                      "kv_member must be [pages, 2, block, Hkv, D], got ", m.sizes());
    TORCH_CHECK_NOT_IMPLEMENTED(m.stride(4) == 1, "kvpath: kv_member's D stride is ", m.stride(4),
                                ", kernels need D innermost");
    const int32_t code = dtype_code(m, "kv_member");
    kvpath_cache c{};
    c.base = m.data_ptr();
    c.num_pages = m.size(0);
    c.block_size = m.size(2);
    c.num_kv_heads = m.size(3);
    c.head_dim = m.size(4);
    c.stride_page = m.stride(0);
    c.stride_kv = m.stride(1);
    c.stride_row = m.stride(2);
    c.stride_head = m.stride(3);
    c.dtype = code;
    c.scale = nullptr;
    if (code == KVPATH_FP8_E4M3) {
        TORCH_CHECK_VALUE(scale != nullptr, "kvpath: an fp8 kv_member needs kv_scale (new_kv_scale)");
        TORCH_CHECK_VALUE(scale->scalar_type() == at::kFloat && scale->dim() == 3 &&
                              scale->size(0) == c.num_pages && scale->size(1) == kMembers &&
                              scale->size(2) == c.num_kv_heads && scale->is_contiguous(),
                          "kvpath: kv_scale must be contiguous f32[", c.num_pages, ", 2, ",
                          c.num_kv_heads, "], got ", scale->scalar_type(), " ", scale->sizes());
        c.scale = scale->data_ptr<float>();
    }
    return c;
}

// A [T, heads, D] tensor as kvpath_rows (copied when D is not innermost; `keep` holds it).
kvpath_rows rows_of(const at::Tensor& x, const char* what, at::Tensor& keep) {
    TORCH_CHECK_VALUE(x.dim() == 3, "kvpath: ", what, " must be [T, heads, D], got ", x.sizes());
    keep = x.stride(2) == 1 ? x : x.contiguous();
    return kvpath_rows{keep.data_ptr(), keep.size(0), keep.size(1), keep.size(2), keep.stride(0),
                       keep.stride(1), dtype_code(keep, what)};
}

// An int32 plan tensor, contiguous (block_table: unit column stride, row stride >= its width).
const int32_t* plan_ptr(const at::Tensor& t, const char* what, at::Tensor& keep, bool table = false) {
    TORCH_CHECK_VALUE(t.scalar_type() == at::kInt, "kvpath: ", what,
                      " must be int32 (sdk/device.py casts the plan to i32), got ", t.scalar_type());
    if (table) {
        TORCH_CHECK_VALUE(t.dim() == 2, "kvpath: block_table must be [R, P], got ", t.sizes());
        keep = (t.stride(1) == 1 && t.stride(0) >= t.size(1)) ? t : t.contiguous();
    } else {
        keep = t.is_contiguous() ? t : t.contiguous();
    }
    return keep.data_ptr<int32_t>();
}

// The plan's lengths (kelpie's contract, ops/paged_attention.py:90-101): row_request, positions
// and slot_mapping i32[T], query_start_loc i32[R+1], seq_lens i32[R], block_table i32[R, P]. The
// kernels read them through bare pointers, so a tensor of another length is refused here instead
// of being read past its end.
void check_rows_of_plan(const at::Tensor& t, const char* what, int64_t T) {
    TORCH_CHECK_VALUE(t.dim() == 1 && t.size(0) == T, "kvpath: ", what, " must be i32[T = ", T,
                      "], got ", t.sizes());
}

void check_plan_lengths(int64_t T, const at::Tensor& row_request, const at::Tensor& positions,
                        const at::Tensor& query_start_loc, const at::Tensor& seq_lens,
                        const at::Tensor& block_table, const at::Tensor& slot_mapping) {
    check_rows_of_plan(row_request, "row_request", T);
    check_rows_of_plan(positions, "positions", T);
    check_rows_of_plan(slot_mapping, "slot_mapping", T);
    TORCH_CHECK_VALUE(seq_lens.dim() == 1, "kvpath: seq_lens must be i32[R], got ", seq_lens.sizes());
    const int64_t R = seq_lens.size(0);
    TORCH_CHECK_VALUE(query_start_loc.dim() == 1 && query_start_loc.size(0) == R + 1,
                      "kvpath: query_start_loc must be i32[R + 1 = ", R + 1, "], got ",
                      query_start_loc.sizes());
    TORCH_CHECK_VALUE(block_table.dim() == 2 && block_table.size(0) == R,
                      "kvpath: block_table must be i32[R = ", R, ", P], got ", block_table.sizes());
}

// One plan-status word per device (an int32 the kernels' plan check ORs 1 into), created zeroed
// by the first call on the device outside stream capture and kept for the process; a call
// captured before it exists passes none (its bad rows are still written as NaN). The tensors
// are never destroyed, so no device memory is freed after the runtime has gone at exit.
constexpr int kMaxDevices = 64;
std::mutex g_status_mutex;
std::array<at::Tensor*, kMaxDevices> g_status{};

at::Tensor* status_word(at::Device dev) {
    const int idx = dev.index();
    TORCH_CHECK(idx >= 0 && idx < kMaxDevices, "kvpath: device index ", idx);
    std::lock_guard<std::mutex> lock(g_status_mutex);
    if (g_status[idx] == nullptr) {
        const c10::hip::HIPStream stream = c10::hip::getCurrentHIPStream(idx);
        hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
        C10_HIP_CHECK(hipStreamIsCapturing(stream.stream(), &capturing));
        if (capturing != hipStreamCaptureStatusNone) return nullptr;
        auto* word = new at::Tensor(at::zeros({1}, at::TensorOptions().dtype(at::kInt).device(dev)));
        stream.synchronize();
        g_status[idx] = word;
    }
    return g_status[idx];
}

void check(int32_t status, const char* entry) {
    if (status == KVPATH_OK) return;
    const char* message = kvpath_last_error();
    TORCH_CHECK_NOT_IMPLEMENTED(status != KVPATH_EUNSUPPORTED, "kvpath ", entry, ": ", message);
    TORCH_CHECK(false, "kvpath ", entry, ": status ", status, ": ", message);
}

std::atomic<bool> g_check_slots{false};  // the plan check's opt-in slot comparison

at::Tensor paged_attention_any(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                               const at::Tensor& kv_member, const at::Tensor& row_request,
                               const at::Tensor& positions, const at::Tensor& query_start_loc,
                               const at::Tensor& seq_lens, const at::Tensor& block_table,
                               const at::Tensor& slot_mapping, int64_t window,
                               const at::Tensor& sinks, bool causal, const at::Tensor* kv_scale,
                               int64_t partition) {
    const at::Device dev = one_device({&q, &k, &v, &kv_member, &row_request, &positions,
                                       &query_start_loc, &seq_lens, &block_table, &slot_mapping});
    const c10::hip::HIPGuard device_guard(dev.index());
    const kvpath_cache cache = cache_of(kv_member, kv_scale);
    at::Tensor qk, kk, vk;
    kvpath_rows qr = rows_of(q, "q", qk), kr = rows_of(k, "k", kk), vr = rows_of(v, "v", vk);
    const int64_t T = q.size(0), H = q.size(1), D = q.size(2);
    check_plan_lengths(T, row_request, positions, query_start_loc, seq_lens, block_table, slot_mapping);
    at::Tensor out = at::empty({T, H * D}, q.options());
    kvpath_rows outr{out.data_ptr(), T, H, D, out.stride(0), D, dtype_code(out, "out")};
    at::Tensor rr_k, pos_k, qsl_k, len_k, table_k, slot_k;
    kvpath_plan plan{};
    plan.row_request = plan_ptr(row_request, "row_request", rr_k);
    plan.positions = plan_ptr(positions, "positions", pos_k);
    plan.query_start_loc = plan_ptr(query_start_loc, "query_start_loc", qsl_k);
    plan.seq_lens = plan_ptr(seq_lens, "seq_lens", len_k);
    plan.block_table = plan_ptr(block_table, "block_table", table_k, true);
    plan.slot_mapping = plan_ptr(slot_mapping, "slot_mapping", slot_k);
    plan.num_tokens = T;
    plan.num_reqs = seq_lens.size(0);
    plan.table_width = table_k.size(1);
    plan.table_stride = std::max<int64_t>(table_k.stride(0), plan.table_width);
    at::Tensor sinks_k;
    kvpath_attn_opts opts{};
    opts.window = static_cast<int32_t>(window);
    opts.causal = causal ? 1 : 0;
    opts.partition_tokens = static_cast<int32_t>(std::max<int64_t>(0, partition));
    opts.check_slots = g_check_slots ? 1 : 0;
    if (sinks.numel() > 0) {
        TORCH_CHECK_VALUE(sinks.dim() == 1 && sinks.size(0) == H, "kvpath: sinks must be f32[", H,
                          "], got ", sinks.sizes());
        one_device({&q, &sinks});
        sinks_k = sinks.to(at::kFloat).contiguous();
        opts.sinks = sinks_k.data_ptr<float>();
    }
    at::Tensor* word = status_word(dev);
    opts.plan_status = word != nullptr ? word->data_ptr<int32_t>() : nullptr;
    const int64_t ws_bytes = kvpath_workspace_bytes(T, plan.num_reqs, H, cache.num_kv_heads, D,
                                                    plan.table_width, cache.block_size,
                                                    opts.partition_tokens);
    TORCH_CHECK_VALUE(ws_bytes >= 0, "kvpath: bad workspace shape");
    // 256-byte aligned scratch from torch's allocator (graph-pool safe under capture).
    at::Tensor ws = at::empty({ws_bytes + 256}, at::TensorOptions().dtype(at::kByte).device(dev));
    char* base = static_cast<char*>(ws.data_ptr());
    char* aligned = base + ((256 - reinterpret_cast<uintptr_t>(base) % 256) % 256);
    const hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();
    check(kvpath_paged_attention(&qr, &kr, &vr, &cache, &plan, &opts, &outr, aligned, ws_bytes,
                                 reinterpret_cast<kvpath_stream_t>(stream)),
          "paged_attention");
    return out;
}

at::Tensor paged_attention_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                               at::Tensor& kv_member, const at::Tensor& row_request,
                               const at::Tensor& positions, const at::Tensor& query_start_loc,
                               const at::Tensor& seq_lens, const at::Tensor& block_table,
                               const at::Tensor& slot_mapping, int64_t window,
                               const at::Tensor& sinks, bool causal, int64_t partition) {
    return paged_attention_any(q, k, v, kv_member, row_request, positions, query_start_loc,
                               seq_lens, block_table, slot_mapping, window, sinks, causal, nullptr,
                               partition);
}

at::Tensor paged_attention_fp8_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                   at::Tensor& kv_member, const at::Tensor& row_request,
                                   const at::Tensor& positions, const at::Tensor& query_start_loc,
                                   const at::Tensor& seq_lens, const at::Tensor& block_table,
                                   const at::Tensor& slot_mapping, int64_t window,
                                   const at::Tensor& sinks, bool causal, at::Tensor& kv_scale,
                                   int64_t partition) {
    one_device({&q, &kv_scale});
    return paged_attention_any(q, k, v, kv_member, row_request, positions, query_start_loc,
                               seq_lens, block_table, slot_mapping, window, sinks, causal,
                               &kv_scale, partition);
}

// write_kv (kernels/ops/paged_attention.py:44-54): k, v [T, Hkv, D] into the member at the flat
// slots, converted to the cache dtype; an fp8 member quantizes on append and updates kv_scale.
void write_kv_any(const at::Tensor& kv_member, const at::Tensor& k, const at::Tensor& v,
                  const at::Tensor& slot_mapping, const at::Tensor* kv_scale) {
    const at::Device dev = one_device({&kv_member, &k, &v, &slot_mapping});
    const c10::hip::HIPGuard device_guard(dev.index());
    const kvpath_cache cache = cache_of(kv_member, kv_scale);
    at::Tensor kk, vk, slot_k;
    kvpath_rows kr = rows_of(k, "k", kk), vr = rows_of(v, "v", vk);
    check_rows_of_plan(slot_mapping, "slot_mapping", k.size(0));
    kvpath_plan plan{};
    plan.slot_mapping = plan_ptr(slot_mapping, "slot_mapping", slot_k);
    plan.num_tokens = k.size(0);
    const hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();
    check(kvpath_kv_append(&cache, &kr, &vr, &plan, reinterpret_cast<kvpath_stream_t>(stream)),
          "kv_append");
}

void write_kv_hip(at::Tensor& kv_member, const at::Tensor& k, const at::Tensor& v,
                  const at::Tensor& slot_mapping) {
    write_kv_any(kv_member, k, v, slot_mapping, nullptr);
}

void write_kv_fp8_hip(at::Tensor& kv_member, const at::Tensor& k, const at::Tensor& v,
                      const at::Tensor& slot_mapping, at::Tensor& kv_scale) {
    one_device({&kv_member, &kv_scale});
    write_kv_any(kv_member, k, v, slot_mapping, &kv_scale);
}

void write_kv_cpu(at::Tensor& kv_member, const at::Tensor&, const at::Tensor&, const at::Tensor&) {
    TORCH_CHECK(false, "kvpath: every tensor must be on one ROCm device, got ", kv_member.device(),
                "; there is no CPU path");
}

void write_kv_fp8_cpu(at::Tensor& kv_member, const at::Tensor&, const at::Tensor&,
                      const at::Tensor&, at::Tensor&) {
    TORCH_CHECK(false, "kvpath: every tensor must be on one ROCm device, got ", kv_member.device(),
                "; there is no CPU path");
}

// CPU tensors (dispatched here when no argument is on a ROCm device): refused, as the Python
// layer refused them.
at::Tensor paged_attention_cpu(const at::Tensor& q, const at::Tensor&, const at::Tensor&,
                               at::Tensor&, const at::Tensor&, const at::Tensor&,
                               const at::Tensor&, const at::Tensor&, const at::Tensor&,
                               const at::Tensor&, int64_t, const at::Tensor&, bool, int64_t) {
    TORCH_CHECK(false, "kvpath: every tensor must be on one ROCm device, got ", q.device(),
                "; there is no CPU path");
}

at::Tensor paged_attention_fp8_cpu(const at::Tensor& q, const at::Tensor&, const at::Tensor&,
                                   at::Tensor&, const at::Tensor&, const at::Tensor&,
                                   const at::Tensor&, const at::Tensor&, const at::Tensor&,
                                   const at::Tensor&, int64_t, const at::Tensor&, bool,
                                   at::Tensor&, int64_t) {
    TORCH_CHECK(false, "kvpath: every tensor must be on one ROCm device, got ", q.device(),
                "; there is no CPU path");
}

// The backward of an inference-only op.
struct NoBackward final : torch::autograd::Node {
    explicit NoBackward(std::string op) : op_(std::move(op)) {}
    torch::autograd::variable_list apply(torch::autograd::variable_list&&) override {
        TORCH_CHECK_NOT_IMPLEMENTED(false, op_,
                                    " has no backward: the paged-KV path is inference-only (kelpie "
                                    "defers training to its train-step branch)");
    }
    std::string name() const override { return "KvpathNoBackward"; }
    std::string op_;
};

// The Autograd kernels: run the op below autograd (kv_member's, and kv_scale's, version bumped
// as an in-place write), then, when a floating input requires grad, hang the output on a
// NoBackward node.
void attach_no_backward(at::Tensor& out, const char* op, const at::Tensor& q, const at::Tensor& k,
                        const at::Tensor& v, const at::Tensor& sinks) {
    if (!torch::autograd::compute_requires_grad(q, k, v, sinks)) return;
    auto node = std::shared_ptr<NoBackward>(new NoBackward(op), torch::autograd::deleteNode);
    node->set_next_edges(torch::autograd::collect_next_edges(q, k, v, sinks));
    torch::autograd::set_history(out, node);
}

at::Tensor paged_attention_autograd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                    at::Tensor& kv_member, const at::Tensor& row_request,
                                    const at::Tensor& positions, const at::Tensor& query_start_loc,
                                    const at::Tensor& seq_lens, const at::Tensor& block_table,
                                    const at::Tensor& slot_mapping, int64_t window,
                                    const at::Tensor& sinks, bool causal, int64_t partition) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("kvpath::paged_attention", "")
                         .typed<decltype(paged_attention_hip)>();
    at::Tensor out;
    {
        at::AutoDispatchBelowADInplaceOrView guard;
        out = op.call(q, k, v, kv_member, row_request, positions, query_start_loc, seq_lens,
                      block_table, slot_mapping, window, sinks, causal, partition);
    }
    torch::autograd::impl::bump_version(kv_member);
    attach_no_backward(out, "kvpath::paged_attention", q, k, v, sinks);
    return out;
}

at::Tensor paged_attention_fp8_autograd(const at::Tensor& q, const at::Tensor& k,
                                        const at::Tensor& v, at::Tensor& kv_member,
                                        const at::Tensor& row_request, const at::Tensor& positions,
                                        const at::Tensor& query_start_loc,
                                        const at::Tensor& seq_lens, const at::Tensor& block_table,
                                        const at::Tensor& slot_mapping, int64_t window,
                                        const at::Tensor& sinks, bool causal, at::Tensor& kv_scale,
                                        int64_t partition) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("kvpath::paged_attention_fp8", "")
                         .typed<decltype(paged_attention_fp8_hip)>();
    at::Tensor out;
    {
        at::AutoDispatchBelowADInplaceOrView guard;
        out = op.call(q, k, v, kv_member, row_request, positions, query_start_loc, seq_lens,
                      block_table, slot_mapping, window, sinks, causal, kv_scale, partition);
    }
    torch::autograd::impl::bump_version(kv_member);
    torch::autograd::impl::bump_version(kv_scale);
    attach_no_backward(out, "kvpath::paged_attention_fp8", q, k, v, sinks);
    return out;
}

// The plan-status word of a device (created if absent and no capture is running), for
// kvpath.plan_status / clear_plan_status / check_plan_status.
at::Tensor plan_status_word(int64_t device) {
    const at::Device dev(at::kCUDA, static_cast<c10::DeviceIndex>(device));
    at::Tensor* word = status_word(dev);
    TORCH_CHECK(word != nullptr, "kvpath: the plan-status word cannot be created during capture");
    return *word;
}

// The plan check's slot comparison for later calls; returns the previous setting.
bool set_check_slots(bool on) { return g_check_slots.exchange(on); }

}  // namespace

TORCH_LIBRARY(kvpath, m) {
    m.def("paged_attention(Tensor q, Tensor k, Tensor v, Tensor(a3!) kv_member, Tensor row_request, "
          "Tensor positions, Tensor query_start_loc, Tensor seq_lens, Tensor block_table, "
          "Tensor slot_mapping, int window, Tensor sinks, bool causal=True, int partition=0) "
          "-> Tensor");
    m.def("paged_attention_fp8(Tensor q, Tensor k, Tensor v, Tensor(a3!) kv_member, "
          "Tensor row_request, Tensor positions, Tensor query_start_loc, Tensor seq_lens, "
          "Tensor block_table, Tensor slot_mapping, int window, Tensor sinks, bool causal, "
          "Tensor(a13!) kv_scale, int partition=0) -> Tensor");
    m.def("write_kv(Tensor(a!) kv_member, Tensor k, Tensor v, Tensor slot_mapping) -> ()");
    m.def("write_kv_fp8(Tensor(a!) kv_member, Tensor k, Tensor v, Tensor slot_mapping, "
          "Tensor(b!) kv_scale) -> ()");
    m.def("plan_status_word(int device) -> Tensor", plan_status_word);
    m.def("set_check_slots(bool on) -> bool", set_check_slots);
}

TORCH_LIBRARY_IMPL(kvpath, CUDA, m) {
    m.impl("paged_attention", paged_attention_hip);
    m.impl("paged_attention_fp8", paged_attention_fp8_hip);
    m.impl("write_kv", write_kv_hip);
    m.impl("write_kv_fp8", write_kv_fp8_hip);
}

TORCH_LIBRARY_IMPL(kvpath, CPU, m) {
    m.impl("paged_attention", paged_attention_cpu);
    m.impl("paged_attention_fp8", paged_attention_fp8_cpu);
    m.impl("write_kv", write_kv_cpu);
    m.impl("write_kv_fp8", write_kv_fp8_cpu);
}

namespace {

// write_kv only writes its cache (no output to differentiate): below autograd, with the written
// tensors' versions bumped as in-place writes.
void write_kv_autograd(at::Tensor& kv_member, const at::Tensor& k, const at::Tensor& v,
                       const at::Tensor& slot_mapping) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("kvpath::write_kv", "")
                         .typed<decltype(write_kv_hip)>();
    {
        at::AutoDispatchBelowADInplaceOrView guard;
        op.call(kv_member, k, v, slot_mapping);
    }
    torch::autograd::impl::bump_version(kv_member);
}

void write_kv_fp8_autograd(at::Tensor& kv_member, const at::Tensor& k, const at::Tensor& v,
                           const at::Tensor& slot_mapping, at::Tensor& kv_scale) {
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("kvpath::write_kv_fp8", "")
                         .typed<decltype(write_kv_fp8_hip)>();
    {
        at::AutoDispatchBelowADInplaceOrView guard;
        op.call(kv_member, k, v, slot_mapping, kv_scale);
    }
    torch::autograd::impl::bump_version(kv_member);
    torch::autograd::impl::bump_version(kv_scale);
}

}  // namespace

TORCH_LIBRARY_IMPL(kvpath, Autograd, m) {
    m.impl("paged_attention", paged_attention_autograd);
    m.impl("paged_attention_fp8", paged_attention_fp8_autograd);
    m.impl("write_kv", write_kv_autograd);
    m.impl("write_kv_fp8", write_kv_fp8_autograd);
}
