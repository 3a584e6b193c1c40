// Paged attention over kelpie's plan: split-KV partition kernels and the reduce.
//
// Replaces _attend and its mask / softmax (kelpie/kelpie-models/kelpie_models/kernels/ops/
// paged_attention.py:160-240).  Semantics, per padded row t of entry r = row_request[t]:
//   pos_t   = seq_lens[r] - rows_r + (t - qsl[r])          (an entry's rows are its newest)
//   key j is visible iff j < seq_lens[r], and j <= pos_t when causal, and j > pos_t - window
//   when window > 0;
//   out[t, hq] = sum_j softmax_j(q.k_j / sqrt(D) [, sink_hq]) v_j over visible keys, where a
//   sink logit competes in the softmax and is dropped; a row with no visible key, and every pad
//   row, is exactly 0.
//
// Work decomposition (split-KV, "flash decoding"): workgroup = (entry r, kv head h, partition p
// of `part` keys, row-tile group).  The q rows of one kv head are the entry's rows x its G q
// heads ("q-rows", qrow = row * G + head-in-group), taken 16 at a time as MFMA tiles.  Each
// workgroup writes, per q-row, a partial (o[D], running max m, weight sum l) for its partition
// (o normalized by l and rounded to bf16 when q is bf16, else un-normalized f32); the reduce
// kernel combines the partitions of each row.
//
// MFMA kernel (bf16 or fp8 cache, bf16 q, D a multiple of 32, block a multiple of 16).  With
// v_mfma_f32_16x16x32_bf16, one 16-key slice of a page against a 16-q-row tile is
//   S^T[key, qrow] = K[key, :] . Q^T[:, qrow]       A = K (16 keys x 32 dims per instruction)
// so lane (c = lane % 16, g = lane / 16) loads key c's dims [32kk + 8g, +8) straight from HBM
// (16 contiguous bytes, no transpose) and receives S^T[4g + i, c], i < 4.  Two slices (32 keys)
// then feed the output product in transposed form,
//   O^T[d, qrow] += V^T[d, key] . P^T[key, qrow]     B = P^T, taken from S^T in registers
// where lane (c, g) holds q-row c's probabilities for keys {4g..4g+3} of both slices: those 8
// values ARE its B operand, with the reduction index k = 8g + j mapped to key 4g + j (j < 4) of
// slice 0 and key 4g + j - 4 of slice 1.  The A operand V^T needs V's columns, so V passes
// through the wave's own LDS tile (row-major, read back one bf16 per key).  The output lands as
// O^T[16nb + 4g + i, c]: q-row c is owned by lanes c, c+16, c+32, c+48 -- the same lanes that own
// its scores -- so the online-softmax rescale is a per-lane multiply with no shuffles.
// Four waves split the partition's 32-key blocks round-robin and merge through LDS at the end.
//
// fp8 cache: e4m3 bytes convert exactly to bf16; the per-(page, kv head) scales are applied to
// the scores (K) and to the probabilities (V) of each 16-key slice, which lies in one page.
#include <algorithm>
#include <type_traits>

#include "kvpath_device.h"
#include "kvpath_fp8.h"
#include "kvpath_internal.h"

namespace kvpath {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kNegInf = -__builtin_huge_valf();

// ---- the plan, per workgroup -------------------------------------------------------------------

struct Entry {
    int32_t q0, n_rows, seq_len, n_q;  // first row, rows, context length, q-rows
    int32_t anchor, part;              // partition 0's first key, partition length (split_entry)
};

// r must be in [0, R). All three scalars are loaded before any test, so they travel together
// (one memory latency, not two).
__device__ __forceinline__ bool load_entry(const AttnArgs& a, int r, Entry& e) {
    const int32_t q0 = a.qsl[r], q1 = a.qsl[r + 1];
    int32_t len32 = a.seq_lens[r];
    // An empty asm consuming all three keeps the compiler from sinking the seq_lens load below
    // the test (it would otherwise wait for qsl first).
    asm volatile("" ::"s"(q0), "s"(q1), "s"(len32));
    int64_t len = len32;
    e.q0 = q0;
    e.n_rows = q1 - q0;
    if (e.n_rows <= 0 || e.q0 < 0 || e.q0 + e.n_rows > a.T) return false;
    // Not a plan: its rows must be its newest positions, and its keys must fit its table row
    // (kelpie-core sizes tables for max_seq_len). Such an entry's rows are left to the dead-row
    // writers (zeros, or NaN under the plan check).
    if (len < e.n_rows || len > a.table_width * a.c.block) return false;
    e.seq_len = static_cast<int32_t>(len);
    e.n_q = e.n_rows * a.G;
    return true;
}

// A workgroup's partition slot: blockIdx.x = slot + grid_parts * tg. Partition-fastest order keeps
// an entry's partitions together, and workgroup i runs on XCD i % 8. With an odd x extent the
// slots of successive grid rows land on rotating XCDs by themselves; with an even one every XCD
// would see few slot indices everywhere (with 8 partitions, one XCD all first partitions, another
// only tails, most of them empty: 64-entry Llama-3-8B decode over a 4096-key table, 156 us
// against 114), so there the slot
// is rotated by the (kv head, entry) coordinates (120 us). Each (tile group, kv head, entry)
// still covers each slot once.
__device__ __forceinline__ int part_slot(const AttnArgs& a, unsigned bx, unsigned by, unsigned bz) {
    const unsigned rot = (gridDim.x & 1u) ? 0u : by + bz;
    return static_cast<int>((bx % a.grid_parts + rot) % a.grid_parts);
}

__device__ __forceinline__ int part_slot(const AttnArgs& a) {
    return part_slot(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Multi-row grids with several tile groups per partition: the workgroups of one (entry, kv head,
// partition) read the same K/V. Workgroup i runs on XCD i % 8, each XCD behind its own L2, so
// such a grid is renumbered to hand each XCD a contiguous run of the work list (work item
// x + X * (y + Y * z), x = slot + grid_parts * tile group fastest): the tile groups of one
// partition then share one L2's copy instead of fetching it on every XCD. The z == R slice of a
// direct-output grid keeps its coordinates.
// A grid that fills the GPU's two workgroups per CU once places workgroups i and i + 256 on one
// CU (read back from HW_ID on MI355X), i.e. items j and j + 32 of an XCD's run. Causal rows make
// a partition's later tile groups read more keys (chunked prefill, 512 rows after 2k keys: 65
// blocks for the first, 80 for the last), so the pairs in the second half of each XCD's run take
// their tile groups in reverse order, and each CU holds a long and a short one (145 blocks)
// instead of two alike (130 to 160): 1.7% on that step.
struct WgCoord {
    unsigned x, y, z;
};

__device__ __forceinline__ WgCoord work_coord(const AttnArgs& a) {
    WgCoord w{blockIdx.x, blockIdx.y, blockIdx.z};
    if (a.tile_groups > 1 && w.z < static_cast<unsigned>(a.R)) {
        const unsigned X = gridDim.x, Y = gridDim.y;
        const unsigned n = X * Y * static_cast<unsigned>(a.R);
        const unsigned lin = w.x + X * (w.y + Y * w.z);
        const unsigned xcd = lin % 8u, j = lin / 8u;
        const unsigned item = xcd * (n / 8u) + min(xcd, n % 8u) + j;
        w.x = item % X;
        // Reversal is per (entry, kv head) pair, so the renumbering stays a bijection.
        const unsigned pairs_half_run = max(1u, n / 8u / X / 2u);
        if ((item / X / pairs_half_run) & 1u) w.x = X - 1u - w.x;
        w.y = (item / X) % Y;
        w.z = item / (X * Y);
    }
    return w;
}

// Partitions are counted from an entry's anchor: key 0 without a window; with one, the entry's
// first visible key (its first row's) rounded down to a 32-key block. Partition p holds keys
// [anchor + p * part, + part), block-aligned, and is slot p of the workspace. A window's keys
// then start at partition 0, so the grid holds only as many partitions as a window can reach
// (one, when it fits a partition: decode then writes its output directly), and a long context
// adds no workgroups that find nothing to do.
//
// The partition length is the step's fixed length (a.part_fixed: a caller's explicit choice), or
// each entry's own split of its span (keys from the anchor to the end of its context), decided
// here from its seq_len alone: ceil(span / a.part) partitions (a.part is the floor length), at
// most the grid's slots per entry, of equal 32-key-aligned length. A short entry then takes few
// slots and a long one all of them, whatever the block table's width (kelpie sizes it for
// max_seq_len: kelpie-core/src/scheduler.zig:1577-1578), as the reference design point splits
// each sequence by its own length under a fixed grid (kernels/vendored/cuda/vllm_attention/
// triton_unified_attention.py:335-355).
__device__ __forceinline__ void split_entry(const AttnArgs& a, Entry& e) {
    e.anchor = a.window > 0 ? max(0, e.seq_len - e.n_rows - a.window + 1) / 32 * 32 : 0;
    if (a.part_fixed) {
        e.part = a.part;
        return;
    }
    const int span = e.seq_len - e.anchor;
    const int n = min(max((span + a.part - 1) / a.part, 1), a.grid_parts);
    e.part = ((span + n - 1) / n + 31) / 32 * 32;
}

// The first key of partition p of a split entry.
__device__ __forceinline__ int part_start(const Entry& e, int p) { return e.anchor + p * e.part; }

// Keys [lo, hi) some q-row in [qr0, qr1) of the entry can see.
__device__ __forceinline__ void visible_span(const AttnArgs& a, const Entry& e, int qr0, int qr1,
                                             int& lo, int& hi) {
    const int pos_lo = e.seq_len - e.n_rows + qr0 / a.G;
    const int pos_hi = e.seq_len - e.n_rows + (qr1 - 1) / a.G;
    hi = a.causal ? pos_hi + 1 : e.seq_len;
    lo = a.window > 0 ? max(0, pos_lo - a.window + 1) : 0;
}

// Row t is live when row_request names an entry whose rows include t; every other row (pads)
// is written as exact zeros.
__device__ __forceinline__ bool row_live(const AttnArgs& a, int t, Entry& e) {
    const int r = a.row_request[t];
    return r >= 0 && r < a.R && load_entry(a, r, e) && t >= e.q0 && t < e.q0 + e.n_rows;
}

// The plan check, on every row an output writer writes when the plan carries `positions`: a row
// that names an entry (row_request >= 0) must be one of that entry's rows (row_live: the entry
// holds it, and its seq_len covers its rows and fits its table row), at its newest position
// (positions[t] == seq_lens[r] - rows_r + (t - qsl[r]), the invariant kelpie's op asserts,
// ops/paged_attention.py:143-157). With a.check_slots, a row this launch appends itself (k_new)
// must also have slot_mapping[t] at that position's slot in the entry's table row (the slot the
// kernels' reads of it assume; one more dependent load per row, so opt-in). `pos_t` is
// positions[t], loaded by the caller beside its other per-row loads (plan_position); `live` and
// `e` are row_live's result for t. A row that breaks the plan is written as NaN instead of its
// attention output and sets bit 0 of *a.status (broken_plan).
__device__ __forceinline__ int32_t plan_position(const AttnArgs& a, int t) {
    return a.positions != nullptr ? a.positions[t] : 0;
}

__device__ __forceinline__ bool row_breaks_plan(const AttnArgs& a, int t, int32_t pos_t, bool live,
                                                const Entry& e) {
    if (a.positions == nullptr) return false;
    if (!live) return a.row_request[t] >= 0;
    const int pos = e.seq_len - e.n_rows + (t - e.q0);
    if (pos_t != pos) return true;
    if (!a.check_slots || a.k_new == nullptr) return false;
    const int64_t page = a.table[static_cast<int64_t>(a.row_request[t]) * a.table_stride + pos / a.c.block];
    return static_cast<int64_t>(a.slots[t]) != page * a.c.block + pos % a.c.block;
}

__device__ __forceinline__ void broken_plan(const AttnArgs& a) {
    if (a.status != nullptr) __hip_atomic_fetch_or(a.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr uint32_t kNanBf16x2 = 0x7fc07fc0u;  // two quiet-NaN bf16 values

__device__ __forceinline__ bool key_visible(const AttnArgs& a, const Entry& e, int qrow, int key) {
    const int pos = e.seq_len - e.n_rows + qrow / a.G;
    bool ok = qrow < e.n_q && key < e.seq_len;
    if (a.causal) ok = ok && key <= pos;
    if (a.window > 0) ok = ok && key > pos - a.window;
    return ok;
}

// Page id of page index `pi` of entry r, or -1 when outside the table or the pool.
__device__ __forceinline__ int64_t page_id(const AttnArgs& a, int r, int64_t pi) {
    if (pi >= a.table_width) return -1;
    const int64_t id = a.table[r * a.table_stride + pi];
    return (id >= 0 && id < a.c.num_pages) ? id : -1;
}

// Partials are partition-major, [n_parts, T, H, D]: a workgroup's rows of one partition (its
// tokens' q heads of one kv head group) lie in runs of G * D values, so its stores are 1 KiB
// runs at D 128 and G 4 instead of 256-byte pieces n_parts apart (measured: the verify kernel
// 1.3%, decode 0.8% faster); the reduce reads each partition's heads of a row as one run.
__device__ __forceinline__ int64_t part_index(const AttnArgs& a, int t, int hq, int p) {
    return ((static_cast<int64_t>(p) * a.T + t) * a.H + hq) * a.c.d;
}

// The partial output of (row t, q head hq, partition p): f32, un-normalized ...
__device__ __forceinline__ float* part_o_f32(const AttnArgs& a, int t, int hq, int p) {
    return static_cast<float*>(a.part_o) + part_index(a, t, hq, p);
}

// ... or, with a bf16 q, normalized by the partition's own sum and rounded to bf16.
__device__ __forceinline__ uint16_t* part_o_bf16(const AttnArgs& a, int t, int hq, int p) {
    return static_cast<uint16_t*>(a.part_o) + part_index(a, t, hq, p);
}

__device__ __forceinline__ float* part_ml_ptr(const AttnArgs& a, int t, int hq, int p) {
    return a.part_ml + ((static_cast<int64_t>(p) * a.T + t) * a.H + hq) * 2;
}

// ---- MFMA partition kernel ---------------------------------------------------------------------

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// Eight e4m3 values as eight bf16, exact (bf16 holds every e4m3 value): gfx950's scaled
// conversion, two values per instruction, with scale 1.0 (it applies only the scale's
// power-of-two exponent, so 1.0 is the identity; checked on the GPU for all 256 bytes).
__device__ __forceinline__ u32x4 widen_fp8(u32x2 w) {
    u32x4 out;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        out[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                                      static_cast<int>(w[i]), 1.0f, false));
        out[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                                          static_cast<int>(w[i]), 1.0f, true));
    }
    return out;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// Two probabilities as a bf16 pair with gfx950's v_cvt_pk_bf16_f32 (round to nearest even, as
// pack_bf16; one instruction instead of a dozen). Probabilities are finite, in [0, 2^8].
__device__ __forceinline__ uint32_t pack_prob(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Two normalized partial outputs as a bf16 pair, the same conversion (a NaN stays a NaN).
__device__ __forceinline__ uint32_t pack_partial(float lo, float hi) { return pack_prob(lo, hi); }

// One (row, q head, partition)'s partial from an MFMA kernel (whose q is bf16, so its partials
// are bf16): dims [d, d + 4) of the un-normalized output `o` over its sum of weights `l` (0 when
// the partition saw no key), 8 bytes. The caller writes (m, l) to part_ml.
__device__ __forceinline__ void store_partial4(const AttnArgs& a, int t, int hq, int p, int d, f32x4 o,
                                               float l) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    *reinterpret_cast<u32x2*>(part_o_bf16(a, t, hq, p) + d) =
        u32x2{pack_partial(o[0] * inv, o[1] * inv), pack_partial(o[2] * inv, o[3] * inv)};
}

// Dims [d, d + 4) of a partial as stored: four bf16 (8 bytes) or four f32. widen_partial turns
// them into f32; times partial_scale<BF16P>(l) that is the partition's un-normalized output.
// (The reduce kernels load them with untracked loads and widen them after one wait, so a batch
// of loads is issued before any wait.)
template <bool BF16P>
using PartialRaw = std::conditional_t<BF16P, u32x2, f32x4>;

template <bool BF16P>
__device__ __forceinline__ f32x4 widen_partial(PartialRaw<BF16P> w) {
    if constexpr (BF16P)
        return f32x4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                     __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u)};
    else
        return w;
}

template <bool BF16P>
__device__ __forceinline__ float load_partial1(const AttnArgs& a, int t, int hq, int p, int d) {
    if constexpr (BF16P)
        return bf16_to_f32(part_o_bf16(a, t, hq, p)[d]);
    else
        return part_o_f32(a, t, hq, p)[d];
}

template <bool BF16P>
__device__ __forceinline__ float partial_scale(float l) { return BF16P ? l : 1.0f; }

typedef short v4s __attribute__((ext_vector_type(4)));

// The online softmax keeps each q-row's running max m and rescales its accumulators only when a
// block's max exceeds m by more than kRescaleLog2 (log2 units); probabilities 2^(s - m) then stay
// below 2^kRescaleLog2, which fp32 sums and bf16 operands carry without loss of range.
constexpr float kRescaleLog2 = 8.0f;

// One K/V block in flight: a bf16 K in registers as loaded (V goes straight to LDS); an fp8
// block goes to LDS whole (K and V), so it holds nothing here.
template <int KK, bool FP8>
struct BlockRegs {
    u32x4 k[2][FP8 ? 1 : KK];
};

// Register loads the compiler does not track (inline asm). The block loop waits for them with
// counted s_waitcnt, so the next block's loads stay outstanding while this one is used; the
// compiler's own tracking of these loads would wait for every outstanding load instead. Each
// register is then passed through after_wait(), so no use can move above the wait.
__device__ __forceinline__ u32x4 load_x4_async(const char* p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}

__device__ __forceinline__ u32x2 load_x2_async(const char* p) {
    u32x2 v;
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}

template <typename T>
__device__ __forceinline__ void after_wait(T& x) {
    asm volatile("" : "+v"(x));
}

// Reductions over the four 16-lane rows of a wave (lane l gets the result over lanes
// l % 16 + 16k), in registers: v_permlane16_swap exchanges rows 1 and 3 of one operand with rows
// 0 and 2 of the other, v_permlane32_swap the upper half of one with the lower half of the
// other, so with both operands equal to x the two results hold the row pairs to combine. The
// s_nops cover the hazard between a VALU write and the swap reading it (without them the swap
// read stale values on the GPU). The compiler builtins are not used: with them the compiler
// dropped the combine.
__device__ __forceinline__ float rows_max(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    x = fmaxf(a, b);
    a = x;
    b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}

__device__ __forceinline__ float rows_sum(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    x = a + b;
    a = x;
    b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Four bf16 of a staged V tile, transposed across the lane group (ds_read_b64_tr_b16): lane
// 4a + b of each 16-lane group receives element b of the 8-byte rows addressed by lanes a,
// a + 4, a + 8, a + 12 of its group. Issued as inline asm the compiler does not track: it would
// otherwise wait for every outstanding global_load_lds before the first LDS read (it cannot tell
// which LDS bytes they write). The caller waits (wait_lds_ops) and passes the result through
// after_wait() before use.
__device__ __forceinline__ v4s lds_read_tr16_async(uint32_t addr) {
    v4s v;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// 16 bytes of LDS, untracked like lds_read_tr16_async.
__device__ __forceinline__ u32x4 lds_read_b128_async(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// 8 bytes of LDS, untracked like lds_read_tr16_async.
__device__ __forceinline__ u32x2 lds_read_b64_async(uint32_t addr) {
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// ds_read_b128 / ds_read_b64_tr_b16, untracked like lds_read_b128_async / lds_read_tr16_async,
// at a compile-time byte offset from the address register: a ring slot's offset goes into the
// instruction's 16-bit offset field, so one address register serves every slot (a register
// operand per slot and read would cost the multi-row kernels dozens of VGPRs).
// (Offsets past the field's 16 bits, from D 256's larger slots, go into the address instead.)
template <int Off>
__device__ __forceinline__ u32x4 lds_read_b128_at(uint32_t addr) {
    static_assert(Off >= 0, "LDS offsets are unsigned");
    u32x4 v;
    if constexpr (Off < 65536)
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(Off) : "memory");
    else
        v = lds_read_b128_async(addr + Off);
    return v;
}

template <int Off>
__device__ __forceinline__ v4s lds_read_tr16_at(uint32_t addr) {
    static_assert(Off >= 0, "LDS offsets are unsigned");
    v4s v;
    if constexpr (Off < 65536)
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(Off) : "memory");
    else
        v = lds_read_tr16_async(addr + Off);
    return v;
}

// ds_read_b64_tr_b8, untracked: lane 8a + b of each 16-lane group receives byte b of the 8-byte
// rows addressed by lanes a, a + 2, ..., a + 14 of its group (probed on the GPU), so one read
// gives a lane eight keys' bytes of one column.
__device__ __forceinline__ u32x2 lds_read_tr8_async(uint32_t addr) {
    u32x2 v;
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// The decode kernel's fp8 tiles (K, then V, per 32-key block): key k's D bytes at k * D, its
// 16-byte chunk q at slot q ^ fp8_swizzle(k). Loads are whole rows per instruction (full
// 128-byte lines). The swizzle spreads the 16 keys of a K operand read, and the 32 keys of a
// transposed V read, so that every LDS bank is touched exactly twice (the minimum for 512 B).
template <int D>
__device__ __forceinline__ int fp8_swizzle(int key) {
    constexpr int CPK = D / 16;                     // chunks per key row
    constexpr int KPB = D >= 256 ? 1 : 256 / D;     // keys per 256-byte bank period
    return (key / KPB) % CPK;
}

template <int KK, bool FP8>
__device__ __forceinline__ void after_wait(BlockRegs<KK, FP8>& st) {
    if constexpr (!FP8) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) after_wait(st.k[s][kk]);
    }
}

template <int D, int W>
struct MfmaLdsV2 {
    // Per wave: two V buffers of 2 slices x (D/32) blocks of 1 KiB (16 rows x 64 bytes).
    static constexpr int kBuf = 2 * (D / 32) * 1024;
    static constexpr int kStageWave = 2 * kBuf;
    static constexpr int kStage = W * kStageWave;
    static constexpr int kOPitch = D + 4;
    static constexpr int kMerge = W * 16 * kOPitch * 4 + W * 16 * 2 * 4;
    static constexpr int kBytes = kStage > kMerge ? kStage : kMerge;
};

typedef __attribute__((address_space(3))) void lds_void;

// Cache-policy operand of global_load_lds: plain, or NT (non-temporal, streaming). KV bytes are
// read once per step; the streaming hint pays when an instruction covers whole 128-byte lines
// (measured on gfx950: a random-page decode read goes from ~5.7 to ~6.5 TB/s) and costs when it
// covers half lines, so only whole-row loads use it.
constexpr int kPolicyPlain = 0;
constexpr int kPolicyStream = 2;

// 16 bytes per lane from global memory straight into LDS at dst + 16 * lane (gfx950).
template <int Policy = kPolicyPlain>
__device__ __forceinline__ void load_lds16(const void* src, char* dst_wave_base) {
    __builtin_amdgcn_global_load_lds(
        src, reinterpret_cast<lds_void*>(reinterpret_cast<uintptr_t>(dst_wave_base) & 0xffffffffu),
        16, 0, Policy);
}

// The decode kernel's V tile: per 32-key block, key k's D values are one row of 2D bytes at
// k * 2D, and its 16-byte chunk q sits at slot q ^ v_swizzle(k). A bf16 V block is loaded whole
// rows per instruction (512 / D keys; full 128-byte lines). The swizzle keeps each 32-byte pair
// of chunks together and spreads the 16 keys of a transposed read over the banks so that every
// bank is touched exactly twice (the minimum for 512 bytes).
template <int D>
__device__ __forceinline__ int v_swizzle(int key) {
    return D == 64 ? 2 * ((key >> 1) & 3) : 2 * (key & 7);
}

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N vector memory operations of this wave are outstanding. Loads complete in
// issue order, so this waits for everything but the last N loads issued.
template <int N>
__device__ __forceinline__ void wait_vmem() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void wait_lds_ops() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Wait until at most N LDS operations of this wave are outstanding. LDS operations complete in
// issue order (scalar memory loads, which share the counter, only make it wait longer), so this
// waits for everything but the last N LDS operations issued.
template <int N>
__device__ __forceinline__ void wait_lds() {
    static_assert(N >= 0 && N < 16, "lgkmcnt is four bits");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}

// Direct output, grid slice z == R: every row that is not live gets exact zeros (what the reduce
// writes for it), or NaN when it names an entry it does not belong to under the plan check
// (row_breaks_plan). Threads test one row each; the workgroup then writes the rows it found
// together, 8 bytes (four bf16) per store. `list` holds NTH + 1 ints of LDS (NTH threads).
template <int NTH>
__device__ void zero_dead_rows(const AttnArgs& a, int* list) {
    const int n_wg = static_cast<int>(gridDim.x * gridDim.y);
    const int wg = static_cast<int>(blockIdx.x + gridDim.x * blockIdx.y);
    const int vecs = a.c.d / 4;
    uint16_t* out = static_cast<uint16_t*>(a.out);
    for (int base = wg * NTH; base < a.T; base += n_wg * NTH) {
        if (threadIdx.x == 0) list[NTH] = 0;
        __syncthreads();
        const int t = base + static_cast<int>(threadIdx.x);
        Entry e;
        if (t < a.T && !row_live(a, t, e)) {
            const bool broken = row_breaks_plan(a, t, 0, false, e);
            if (broken) broken_plan(a);
            list[atomicAdd(&list[NTH], 1)] = broken ? ~t : t;
        }
        __syncthreads();
        const int n = list[NTH];
        for (int k = 0; k < n; ++k) {
            const int tk = list[k];
            const uint32_t fill = tk < 0 ? kNanBf16x2 : 0u;
            const int64_t row = static_cast<int64_t>(tk < 0 ? ~tk : tk) * a.out_srow;
            for (int idx = static_cast<int>(threadIdx.x); idx < a.H * vecs; idx += NTH) {
                const int hq = idx / vecs, v = idx - hq * vecs;
                *reinterpret_cast<u32x2*>(out + row + static_cast<int64_t>(hq) * a.out_shead + 4 * v) =
                    u32x2{fill, fill};
            }
        }
        __syncthreads();  // the list is rewritten next round
    }
}

// Fused append: this step's rows i in [i_lo, i_hi) of entry e (the entry's last n_rows keys)
// get their K and V for kv head h written to their slots, 16 bytes per thread and step, by the
// NTH threads of one workgroup. Rows whose slot lies outside the pool are skipped (pad rows
// belong to no entry). Readers of these keys in the same kernel take them from k_new / v_new,
// so no workgroup reads a slot this kernel writes.
template <int D, int NTH>
__device__ __forceinline__ void append_rows_of_entry(const AttnArgs& a, const Entry& e, int h, int i_lo,
                                                     int i_hi) {
    constexpr int kChunks = D / 8;  // 16-byte chunks per (row, member, head)
    const int64_t pool = a.c.num_pages * a.c.block;
    const int64_t head_bytes = static_cast<int64_t>(h) * a.c.s_head * 2;
    for (int idx = static_cast<int>(threadIdx.x); idx < (i_hi - i_lo) * 2 * kChunks; idx += NTH) {
        const int i = i_lo + idx / (2 * kChunks);
        const int rem = idx - (i - i_lo) * 2 * kChunks;
        const int m = rem / kChunks, cc = rem - m * kChunks;
        const int t = e.q0 + i;
        const int64_t slot = a.slots[t];
        if (slot < 0 || slot >= pool) continue;
        const char* src = static_cast<const char*>(m ? a.v_new : a.k_new) +
                          (static_cast<int64_t>(t) * (m ? a.vn_srow : a.kn_srow) +
                           static_cast<int64_t>(h) * (m ? a.vn_shead : a.kn_shead)) * 2 + cc * 16;
        char* dst = static_cast<char*>(a.c.base) +
                    ((slot / a.c.block) * a.c.s_page + m * a.c.s_kv + (slot % a.c.block) * a.c.s_row) * 2 +
                    head_bytes + cc * 16;
        *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
    }
}

// Fused fp8 append: this step's rows i in [i_lo, i_hi) of entry e (the entry's last n_rows
// keys), for kv head h, under the quantize-on-append rule of kvpath_fp8.h, by the workgroup whose
// partition holds them. Partitions start on 32-key boundaries and a page holds `block` keys with
// 32 % block == 0, so every page these rows land in lies inside this partition: no other
// workgroup of the launch reads its head-h bytes or scales, and this one reads them only after
// the barrier that follows the call. (The rows' slots are their positions' slots in the entry's
// table, as the engine's plans give them.) Each run of rows in one page becomes two units (K, V);
// a group of D / 8 lanes takes a unit, a lane 8 dims. The first kRunKeep rows of a run stay in
// registers between the absmax and the quantize pass (a decode entry's rows: n_rows * G <= 16,
// so at most 4 rows when G >= 4); longer runs read theirs twice. Rows whose slot lies outside the
// pool are skipped. The bytes and scales equal append_fp8_runs' (the clamped conversion it uses
// for non-finite runs gives its unclamped one's result on finite ones).
constexpr int kRunKeep = 4;

template <int D, int NTH>
__device__ __forceinline__ void append_fp8_rows_of_entry(const AttnArgs& a, const Entry& e, int h, int i_lo,
                                                         int i_hi) {
    constexpr int L = D / 8;
    constexpr int kGroups = NTH / L;
    const int n = i_hi - i_lo;
    if (n <= 0) return;
    const int64_t block = a.c.block, pool = a.c.num_pages * block;
    const int lane = static_cast<int>(threadIdx.x) % L;
    uint8_t* cache = static_cast<uint8_t*>(a.c.base);
    for (int u = static_cast<int>(threadIdx.x) / L; u < 2 * n; u += kGroups) {
        const int j = u >> 1, m = u & 1;
        const int64_t t0 = e.q0 + i_lo + j;
        const int64_t slot0 = a.slots[t0];
        const int64_t page = page_of(slot0, block, pool);
        if (page < 0) continue;
        if (j > 0 && page_of(a.slots[t0 - 1], block, pool) == page) continue;  // not a run's first row
        int len = 1;
        uint64_t written = 1ull << (slot0 - page * block);
        while (j + len < n) {
            const int64_t s2 = a.slots[t0 + len];
            if (page_of(s2, block, pool) != page) break;
            written |= 1ull << (s2 - page * block);
            ++len;
        }
        const bool fresh = written & 1ull;
        const uint16_t* src = static_cast<const uint16_t*>(m ? a.v_new : a.k_new) +
                              h * (m ? a.vn_shead : a.kn_shead) + 8 * lane;
        const int64_t s_row = m ? a.vn_srow : a.kn_srow;
        float* scale_slot = a.c.scale + (page * 2 + m) * a.c.hkv + h;
        const float s_old = fresh ? 0.0f : *scale_slot;
        u32x4 keep[kRunKeep];
#pragma unroll
        for (int r = 0; r < kRunKeep; ++r)
            keep[r] = r < len ? *reinterpret_cast<const u32x4*>(src + (t0 + r) * s_row) : u32x4{0, 0, 0, 0};
        float amax = 0.0f;
#pragma unroll
        for (int r = 0; r < kRunKeep; ++r) {
            float x[8];
            widen_bf16x8(keep[r], x);
            amax = fmaxf(amax, absmax8(x));
        }
        for (int r = kRunKeep; r < len; ++r) {
            float x[8];
            widen_bf16x8(*reinterpret_cast<const u32x4*>(src + (t0 + r) * s_row), x);
            amax = fmaxf(amax, absmax8(x));
        }
#pragma unroll
        for (int o = L / 2; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, L));
        int k;
        const float s_new = grow_scale(s_old, __fdiv_rn(amax, kFp8Max), k);
        const float r_new = s_new > 0.0f ? __fdiv_rn(1.0f, s_new) : 0.0f;
        const int64_t head_base = page * a.c.s_page + m * a.c.s_kv + h * a.c.s_head + 8 * lane;
        if (k > 0) {  // the page's other rows: an exponent shift
            for (int64_t row = 0; row < block; ++row) {
                if (written >> row & 1ull) continue;
                u32x2* p = reinterpret_cast<u32x2*>(cache + head_base + row * a.c.s_row);
                *p = requant8(*p, k);
            }
        }
        for (int r = 0; r < len; ++r) {
            float x[8];
            u32x4 w = keep[0];
#pragma unroll
            for (int q = 1; q < kRunKeep; ++q)
                if (r == q) w = keep[q];
            if (r >= kRunKeep) w = *reinterpret_cast<const u32x4*>(src + (t0 + r) * s_row);
            widen_bf16x8(w, x);
            const int64_t row = static_cast<int64_t>(a.slots[t0 + r]) - page * block;
            *reinterpret_cast<u32x2*>(cache + head_base + row * a.c.s_row) =
                r_new > 0.0f ? quantize8(x, r_new) : u32x2{0, 0};
        }
        if (lane == 0) *scale_slot = s_new;
    }
}

// DIRECT: this launch writes `out` itself (one partition holds every row's keys) and its grid has
// the z == R slice that zeroes dead rows; a separate instantiation, so the split-KV kernel carries
// none of it.
template <int D, int NT, bool FP8, int W, bool DIRECT = false>
__device__ __forceinline__ void partition_body(const AttnArgs& a, char* lds) {
    // bf16 multi-row steps run attn_partition_verify; this body's bf16 path is kept for one
    // row tile per wave (decode) only, the case its LDS layout, page-offset preload and merge
    // are built and tested for. (An experiment that re-enabled bf16 with four tiles per wave
    // faulted the GPU on the DFlash verify workload.)
    static_assert(FP8 || NT == 1, "bf16 multi-row steps use attn_partition_verify");
    constexpr int KK = D / 32;  // MFMA steps over the head dim
    constexpr int NB = D / 16;  // 16-wide output column blocks
    constexpr int ES = FP8 ? 1 : 2;
    // bf16 K goes to registers with loads the compiler does not track (its own tracking would
    // drain the pipeline at the first LDS read). That needs the compiler to leave a load's
    // destination untouched until the explicit wait; under high register pressure (D 256, or
    // four row tiles per wave) it copies the destinations into AGPRs right after the load and
    // reuses them (read before the data lands; the late data then overwrites the reuse), so
    // only one-tile instances at D <= 128 keep them. The build scans the ISA for such uses and
    // refuses to link the library when it finds one (kvpath.isa_scan).
    constexpr bool kAsyncK = D <= 128 && NT == 1;
    constexpr int kWaves = W;   // waves per workgroup
    constexpr int kThreads = 64 * W;
    using L = MfmaLdsV2<D, W>;

    const int r = blockIdx.z, h = blockIdx.y;
    if constexpr (DIRECT) {
        if (r == a.R) {
            zero_dead_rows<kThreads>(a, reinterpret_cast<int*>(lds));
            return;
        }
    }
    const int p_rel = part_slot(a);
    const int tg0 = blockIdx.x / a.grid_parts;
    // The wave index is uniform; readfirstlane tells the compiler so, which keeps the block loop's
    // control flow scalar.
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int64_t table_row = static_cast<int64_t>(r) * a.table_stride;
    const int block = static_cast<int>(a.c.block);

    Entry e;
    if (!load_entry(a, r, e)) return;
    split_entry(a, e);
    const int p = p_rel;
    const int part_lo = part_start(e, p);
    if (part_lo >= e.seq_len) return;
    // The page ids of this wave's first 32 blocks when its keys start at the partition's first
    // key (always so without a window), loaded right after the entry's scalars, before anything
    // else, so the first K/V loads wait for as little as possible. (Loaded before the entry check
    // they cost more: a workgroup whose partition lies past its entry would wait for them before
    // retiring.) Lane l holds block l/2, slice l%2; an id past the table is 0 and is checked
    // against the entry below.
    const int spec_kb0 = part_lo / 32 + wave;
    int spec_pid = 0;
    {
        const int64_t pi = ((spec_kb0 + kWaves * (lane >> 1)) * 32 + (lane & 1) * 16) / block;
        if (pi < a.table_width) spec_pid = a.table[table_row + pi];
    }
    const int part_hi = min(part_lo + e.part, e.seq_len);

    const char* cache = static_cast<const char*>(a.c.base);
    const int64_t head_bytes = static_cast<int64_t>(h) * a.c.s_head * ES;

    // Fused append: this step's rows are the entry's last n_rows keys. The partition holding a
    // row writes its K and V for head h (16-byte chunks); the attention below reads those keys
    // from k_new / v_new, so no workgroup reads a slot this kernel writes.
    const int first_new = e.seq_len - e.n_rows;
    const bool fused_append = !FP8 && a.k_new != nullptr;
    if (fused_append && tg0 == 0)
        append_rows_of_entry<D, kThreads>(a, e, h, max(0, part_lo - first_new),
                                          min(e.n_rows, part_hi - first_new));
    // An fp8 cache's fused append quantizes into the pages this partition holds, and the
    // attention below then reads them from the cache like every other key (after the barrier,
    // which also orders the stores: workgroup scope suffices, every reader is in this workgroup).
    if constexpr (FP8 && NT == 1) {
        if (a.k_new != nullptr) {
            append_fp8_rows_of_entry<D, kThreads>(a, e, h, max(0, part_lo - first_new),
                                                  min(e.n_rows, part_hi - first_new));
            __syncthreads();
        }
    }
    const char* k_new_head = fused_append ? static_cast<const char*>(a.k_new) +
                                                static_cast<int64_t>(h) * a.kn_shead * 2 : nullptr;
    const char* v_new_head = fused_append ? static_cast<const char*>(a.v_new) +
                                                static_cast<int64_t>(h) * a.vn_shead * 2 : nullptr;
    const int64_t kv_bytes = a.c.s_kv * ES;
    // K: lane (c, g) reads key row c, dims [32kk + 8g, +8) -- its MFMA A operand.
    const uint32_t k_lane_off = static_cast<uint32_t>(c * a.c.s_row * ES + g * 8 * ES);
    // V (bf16, straight to LDS): instruction j of a 16-key slice loads keys j * KPI + l / CPK,
    // lane l taking slot l % CPK of its key's row, i.e. dims chunk (l % CPK) ^ v_swizzle(key).
    // fp8 V takes K's lane layout and is written to the tile after widening.
    constexpr int CPK = D / 8;     // 16-byte chunks per key row
    constexpr int KPI = 64 / CPK;  // keys per load instruction
    int v_key[KK];
    uint32_t v_chunk_off[KK], v_lane_off[KK];
#pragma unroll
    for (int j = 0; j < KK; ++j) {
        v_key[j] = j * KPI + lane / CPK;
        v_chunk_off[j] = static_cast<uint32_t>(((lane % CPK) ^ v_swizzle<D>(v_key[j])) * 16);
        v_lane_off[j] = static_cast<uint32_t>(v_key[j] * a.c.s_row * ES) + v_chunk_off[j];
    }
    char* vst = lds + wave * L::kStageWave;
    // fp8 tiles: instruction j of a 16-key slice loads keys j * F_KPI + l / F_CPK of the slice,
    // lane l taking slot l % F_CPK of its key's row, i.e. chunk (l % F_CPK) ^ fp8_swizzle(key).
    constexpr int F_CPK = D / 16;           // 16-byte chunks per fp8 key row
    constexpr int F_KPI = 64 / F_CPK;       // keys per load instruction
    constexpr int F_IPS = 16 / F_KPI;       // load instructions per slice
    uint32_t f_lane_off[FP8 ? F_IPS : 1] = {};
    // K operand reads: lane (c, g) takes key 16s + c, bytes [32kk + 8g, +8).
    uint32_t f_krd[FP8 ? 2 : 1][FP8 ? KK : 1] = {};
    // Transposed V reads: lane m of 16-lane group g addresses key_j = (j < 4 ? 4g + j :
    // 16 + 4g + j - 4), j = m / 2, bytes [16nb + 8(m % 2), +8); byte j of every lane of the group
    // then belongs to key_j -- the P^T operand's key order.
    int f_vkey[FP8 ? 8 : 1] = {};
    uint32_t f_vrd_row = 0;
    int f_vsw = 0;
    if constexpr (FP8) {
#pragma unroll
        for (int j = 0; j < F_IPS; ++j) {
            const int key = j * F_KPI + lane / F_CPK;
            f_lane_off[j] = static_cast<uint32_t>(key * a.c.s_row +
                                                  ((lane % F_CPK) ^ fp8_swizzle<D>(key)) * 16);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk)
                f_krd[s][kk] = static_cast<uint32_t>(
                    (16 * s + c) * D + (((2 * kk + (g >> 1)) ^ fp8_swizzle<D>(c)) * 16) + (g & 1) * 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) f_vkey[j] = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
        const int m = lane & 15;
        const int my_key = f_vkey[m >> 1];
        f_vrd_row = static_cast<uint32_t>(my_key * D + (m & 1) * 8);
        f_vsw = fp8_swizzle<D>(my_key);
    }
    const int n_tiles = (e.n_q + 15) / 16;
    const int n_pages_seq = (e.seq_len + block - 1) / block;
    const int r_row = 4 * g + (c >> 2);  // transposed-read source key (within a slice)

    for (int tg = tg0; tg * NT < n_tiles; tg += a.tile_groups) {
        const int qr0 = tg * NT * 16;
        const int qr1 = min(qr0 + NT * 16, e.n_q);
        int lo, hi;
        visible_span(a, e, qr0, qr1, lo, hi);
        lo = max(lo, part_lo);
        hi = min(hi, part_hi);
        if (lo >= hi) continue;  // no q-row of this group reads this partition
        // Keys every q-row of the group sees: blocks inside [full_lo, full_hi) need no mask.
        const int pos_first = e.seq_len - e.n_rows + qr0 / a.G;
        const int pos_last = e.seq_len - e.n_rows + (qr1 - 1) / a.G;
        const int full_hi = a.causal ? pos_first + 1 : e.seq_len;
        const int full_lo = a.window > 0 ? pos_last - a.window + 1 : 0;

        // Q^T operands: lane (c, g) holds q-row (tile*16 + c), dims [32kk + 8g, +8). Rows past
        // the group are zero: their scores are finite and never written out.
        u32x4 qb[NT][KK];
#pragma unroll
        for (int ti = 0; ti < NT; ++ti) {
            const int qrow = qr0 + ti * 16 + c;
            const bool ok = qrow < e.n_q;
            const int t = e.q0 + (ok ? qrow / a.G : 0);
            const int hq = h * a.G + (ok ? qrow % a.G : 0);
            const char* qp = static_cast<const char*>(a.q) +
                             (static_cast<int64_t>(t) * a.q_srow + static_cast<int64_t>(hq) * a.q_shead) * 2;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                const u32x4 x = *reinterpret_cast<const u32x4*>(qp + (32 * kk + 8 * g) * 2);
                qb[ti][kk] = ok ? x : u32x4{0, 0, 0, 0};
            }
        }

        f32x4 acc[NT][NB];
        float m_run[NT], l_run[NT];
#pragma unroll
        for (int ti = 0; ti < NT; ++ti) {
            m_run[ti] = kNegInf;
            l_run[ti] = 0.0f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[ti][nb] = f32x4{0, 0, 0, 0};
        }

        // This wave's 32-key blocks: kb0 + 4i, i < n_kb.
        const int kb_first = lo / 32, kb_last = (hi - 1) / 32;
        const int kb0 = kb_first + wave;
        const int n_kb = kb0 <= kb_last ? (kb_last - kb0) / kWaves + 1 : 0;

        for (int chunk = 0; chunk < n_kb; chunk += 32) {
            // Page ids (and fp8 scales) of the next 32 blocks, one (block, slice) per lane:
            // lane l -> block chunk + l/2, slice l%2. A missing page reads the null page 0; its
            // keys are past the context and masked.
            // With each, the byte offset of the slice (page, row in the page, kv head), so issuing
            // a block is two lane reads per slice.
            int my_pid = 0;
            float my_ks = 0.0f, my_vs = 0.0f;
            uint32_t off_lo, off_hi;
            {
                const int i = chunk + (lane >> 1);
                const int key0 = (kb0 + kWaves * i) * 32 + (lane & 1) * 16;
                if (i < n_kb && key0 < e.seq_len) {
                    const int pi = key0 / block;
                    if (pi < n_pages_seq) {
                        const int id = chunk == 0 && kb0 == spec_kb0 ? spec_pid : a.table[table_row + pi];
                        if (id >= 0 && id < a.c.num_pages) my_pid = id;
                    }
                }
                if constexpr (FP8) {
                    my_ks = a.c.scale[(static_cast<int64_t>(my_pid) * 2 + 0) * a.c.hkv + h];
                    my_vs = a.c.scale[(static_cast<int64_t>(my_pid) * 2 + 1) * a.c.hkv + h];
                }
                const uint64_t off = static_cast<uint64_t>(static_cast<int64_t>(my_pid) * a.c.s_page * ES +
                                                           static_cast<int64_t>(key0 % block) * a.c.s_row * ES +
                                                           head_bytes);
                off_lo = static_cast<uint32_t>(off);
                off_hi = static_cast<uint32_t>(off >> 32);
            }
            const int n_here = min(32, n_kb - chunk);

            // Issue block i's loads into LDS buffer `buf` (= i % 2, a compile-time constant at
            // every call): a bf16 K into registers and V into LDS; an fp8 K and V into LDS.
            auto load_block = [&](BlockRegs<KK, FP8>& st, int i, int buf) {
                const int kb = kb0 + kWaves * (chunk + i);
                char* vbuf = vst + buf * L::kBuf;
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const int sel = 2 * i + s;
                    const int key0 = kb * 32 + s * 16;
                    const uint32_t lo32 = __builtin_amdgcn_readlane(off_lo, sel);
                    const uint32_t hi32 = __builtin_amdgcn_readlane(off_hi, sel);
                    const char* kbase = cache + ((static_cast<uint64_t>(hi32) << 32) | lo32);
                    const char* kp = kbase + k_lane_off;
                    // This step's keys come from its own k/v rows.
                    const bool new_keys = fused_append && key0 + 16 > first_new;
                    if (new_keys) {
                        const int kkey = key0 + c;
                        if (kkey >= first_new && kkey < e.seq_len)
                            kp = k_new_head + static_cast<int64_t>(e.q0 + kkey - first_new) * a.kn_srow * 2 + g * 16;
                    }
                    if constexpr (FP8) {
                        // K and V tiles, whole key rows per instruction, streaming.
#pragma unroll
                        for (int j = 0; j < F_IPS; ++j) {
                            load_lds16<kPolicyStream>(kbase + f_lane_off[j],
                                                      vbuf + (s * F_IPS + j) * 1024);
                            load_lds16<kPolicyStream>(kbase + kv_bytes + f_lane_off[j],
                                                      vbuf + 32 * D + (s * F_IPS + j) * 1024);
                        }
                        continue;
                    }
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) {
                        {
                            st.k[s][kk] = kAsyncK ? load_x4_async(kp + kk * 64)
                                                  : *reinterpret_cast<const u32x4*>(kp + kk * 64);
                            const char* vp = kbase + kv_bytes + v_lane_off[kk];
                            if (new_keys) {
                                const int vkey = key0 + v_key[kk];
                                if (vkey >= first_new && vkey < e.seq_len)
                                    vp = v_new_head + static_cast<int64_t>(e.q0 + vkey - first_new) * a.vn_srow * 2 +
                                         v_chunk_off[kk];
                            }
                            load_lds16<kPolicyStream>(vp, vbuf + (s * KK + kk) * 1024);
                        }
                    }
                }
            };

            auto compute_block = [&](BlockRegs<KK, FP8>& st, int i, int buf) {
                const int kb = kb0 + kWaves * (chunk + i);
                // fp8 scales are read here, not when the block's loads are issued, so those loads
                // do not wait for the scale lookups.
                float ks[2] = {1.0f, 1.0f}, vs[2] = {1.0f, 1.0f};
                if constexpr (FP8) {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        ks[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                            __builtin_bit_cast(int, my_ks), 2 * i + s));
                        vs[s] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                            __builtin_bit_cast(int, my_vs), 2 * i + s));
                    }
                }
                const char* vbuf = vst + buf * L::kBuf;
                const bool tail = kb * 32 + 32 > e.seq_len;
                // fp8: every K operand of the block, read from the tile and widened below.
                u32x2 k8[FP8 ? 2 : 1][FP8 ? KK : 1];
                if constexpr (FP8) {
                    const uint32_t kt = lds_addr(vbuf);
#pragma unroll
                    for (int s = 0; s < 2; ++s)
#pragma unroll
                        for (int kk = 0; kk < KK; ++kk) k8[s][kk] = lds_read_b64_async(kt + f_krd[s][kk]);
                    wait_lds_ops();
#pragma unroll
                    for (int s = 0; s < 2; ++s)
#pragma unroll
                        for (int kk = 0; kk < KK; ++kk) after_wait(k8[s][kk]);
                } else if (tail) {
                    // Keys past the context may hold anything (NaN included); zero their V rows
                    // in LDS so a zero probability cannot turn into NaN in the product. The tail
                    // block is this wave's last, so nothing else of its is in flight.
                    wave_sync_lds();
#pragma unroll
                    for (int s = 0; s < 2; ++s)
#pragma unroll
                        for (int kk = 0; kk < KK; ++kk)
                            if (kb * 32 + s * 16 + c >= e.seq_len)
                                *reinterpret_cast<u32x4*>(const_cast<char*>(vbuf) + s * KK * 1024 + c * 2 * D +
                                                          (((4 * kk + g) ^ v_swizzle<D>(c)) * 16)) = u32x4{0, 0, 0, 0};
                }
                const bool masked = kb * 32 < full_lo || kb * 32 + 32 > full_hi;
                u32x4 pb[NT];
#pragma unroll
                for (int ti = 0; ti < NT; ++ti) {
                    float sc[2][4];
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        f32x4 acc_s = {0, 0, 0, 0};
#pragma unroll
                        for (int kk = 0; kk < KK; ++kk) {
                            u32x4 kop;
                            if constexpr (FP8)
                                kop = widen_fp8(k8[s][kk]);
                            else
                                kop = st.k[s][kk];
                            acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, kop),
                                __builtin_bit_cast(bf16x8, qb[ti][kk]), acc_s, 0, 0, 0);
                        }
                        const float mul = FP8 ? a.score_scale_log2 * ks[s] : a.score_scale_log2;
#pragma unroll
                        for (int j = 0; j < 4; ++j) sc[s][j] = acc_s[j] * mul;
                    }
                    if (masked) {
                        const int qrow = qr0 + ti * 16 + c;
                        const int pos = e.seq_len - e.n_rows + qrow / a.G;
                        const int vis_hi = a.causal ? min(pos + 1, e.seq_len) : e.seq_len;
                        const int vis_lo = a.window > 0 ? pos - a.window + 1 : 0;
#pragma unroll
                        for (int s = 0; s < 2; ++s)
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const int key = kb * 32 + s * 16 + 4 * g + j;
                                if (key >= vis_hi || key < vis_lo) sc[s][j] = kNegInf;
                            }
                    }
                    float mx = kNegInf;
#pragma unroll
                    for (int s = 0; s < 2; ++s)
#pragma unroll
                        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, sc[s][j]);
                    mx = rows_max(mx);
                    // Rescale only when some q-row's max grew past the slack (wave-uniform).
                    if (__builtin_amdgcn_ballot_w64(mx > m_run[ti] + kRescaleLog2)) {
                        const float m_new = fmaxf(m_run[ti], mx);
                        const float alpha = m_new == kNegInf ? 1.0f
                                                             : __builtin_amdgcn_exp2f(m_run[ti] - m_new);
                        l_run[ti] *= alpha;
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) acc[ti][nb] *= alpha;
                        m_run[ti] = m_new;
                    }
                    const float m_use = m_run[ti] == kNegInf ? 0.0f : m_run[ti];
                    float pr[2][4];
                    float sum = 0.0f;
#pragma unroll
                    for (int s = 0; s < 2; ++s)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            pr[s][j] = __builtin_amdgcn_exp2f(sc[s][j] - m_use);
                            sum += pr[s][j];
                        }
                    l_run[ti] += sum;
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const float vm = FP8 ? vs[s] : 1.0f;
                        pb[ti][2 * s] = pack_prob(pr[s][0] * vm, pr[s][1] * vm);
                        pb[ti][2 * s + 1] = pack_prob(pr[s][2] * vm, pr[s][3] * vm);
                    }
                }

                // O^T += V^T . P^T: two transposed reads give lane (c, g) column 16nb + c of
                // keys 4g..4g+3 of slice 0 and of slice 1 (lane m of a 16-lane group addresses
                // key 4g + m/4, dims 16nb + 4(m%4) .. +3). Reads go in batches of kBatch column
                // blocks, each batch waited for once.
                if constexpr (FP8) {
                    // O^T += V^T . P^T from the fp8 V tile: one transposed byte read per column
                    // block gives lane (c, g) the eight keys of its P^T operand for column
                    // 16nb + c; bytes of keys past the context are zeroed (they may hold NaN).
                    uint32_t live_lo = 0xffffffffu, live_hi = 0xffffffffu;
                    if (tail) {
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            if (kb * 32 + f_vkey[j] >= e.seq_len) {
                                if (j < 4) live_lo &= ~(0xffu << (8 * j));
                                else live_hi &= ~(0xffu << (8 * (j - 4)));
                            }
                    }
                    const uint32_t vt = lds_addr(vbuf) + 32 * D + f_vrd_row;
                    constexpr int kBatch8 = NB < 8 ? NB : 8;
#pragma unroll
                    for (int nb0 = 0; nb0 < NB; nb0 += kBatch8) {
                        u32x2 vraw[kBatch8];
#pragma unroll
                        for (int j = 0; j < kBatch8; ++j)
                            vraw[j] = lds_read_tr8_async(vt + (((nb0 + j) ^ f_vsw) * 16));
                        wait_lds_ops();
#pragma unroll
                        for (int j = 0; j < kBatch8; ++j) {
                            after_wait(vraw[j]);
                            vraw[j][0] &= live_lo;
                            vraw[j][1] &= live_hi;
                            const u32x4 va = widen_fp8(vraw[j]);
#pragma unroll
                            for (int ti = 0; ti < NT; ++ti)
                                acc[ti][nb0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    __builtin_bit_cast(bf16x8, va), __builtin_bit_cast(bf16x8, pb[ti]),
                                    acc[ti][nb0 + j], 0, 0, 0);
                        }
                    }
                    return;
                }
                wave_sync_lds();
                constexpr int kBatch = NB < 4 ? NB : 4;
                const uint32_t v_row_addr = lds_addr(vbuf) + r_row * 2 * D + (c & 1) * 8;
                const int v_sw = v_swizzle<D>(r_row);
#pragma unroll
                for (int nb0 = 0; nb0 < NB; nb0 += kBatch) {
                v4s lo_b[kBatch], hi_b[kBatch];
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    const int q = 2 * (nb0 + j) + ((c & 3) >> 1);
                    const uint32_t addr = v_row_addr + ((q ^ v_sw) * 16);
                    lo_b[j] = lds_read_tr16_async(addr);
                    hi_b[j] = lds_read_tr16_async(addr + KK * 1024);
                }
                wait_lds_ops();
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    after_wait(lo_b[j]);
                    after_wait(hi_b[j]);
                }
#pragma unroll
                for (int j = 0; j < kBatch; ++j) {
                    const int nb = nb0 + j;
                    const u32x2 lo2 = __builtin_bit_cast(u32x2, lo_b[j]), hi2 = __builtin_bit_cast(u32x2, hi_b[j]);
                    const u32x4 va = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
                    for (int ti = 0; ti < NT; ++ti)
                        acc[ti][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, va), __builtin_bit_cast(bf16x8, pb[ti]),
                            acc[ti][nb], 0, 0, 0);
                }
                }
            };

            // Two blocks in flight: block i+2's loads are issued as soon as block i's math is done
            // (into the registers and LDS buffer block i used), and the wait before block i's
            // math leaves block i+1's loads outstanding. kOps = vector memory operations per
            // block: bf16, K and V, two slices of KK each; fp8, the K and V tiles, KK each.
            constexpr int kOps = FP8 ? 2 * KK : 4 * KK;
            BlockRegs<KK, FP8> sa, sb;
            load_block(sa, 0, 0);
            if (n_here > 1) load_block(sb, 1, 1);
            for (int i = 0; i < n_here; i += 2) {
                if (i + 1 < n_here) wait_vmem<kOps>(); else wait_vmem<0>();
                after_wait(sa);
                wave_sync_lds();
                compute_block(sa, i, 0);
                if (i + 2 < n_here) {
                    wait_lds_ops();  // block i's LDS reads are done before its buffer refills
                    load_block(sa, i + 2, 0);
                }
                if (i + 1 >= n_here) break;
                if (i + 2 < n_here) wait_vmem<kOps>(); else wait_vmem<0>();
                after_wait(sb);
                wave_sync_lds();
                compute_block(sb, i + 1, 1);
                if (i + 3 < n_here) {
                    wait_lds_ops();
                    load_block(sb, i + 3, 1);
                }
            }
            wait_vmem_all();  // nothing may still be writing this wave's LDS
        }

        // Merge the four waves, one tile at a time, and write the partials.
        float* om = reinterpret_cast<float*>(lds);
        float* mls = om + kWaves * 16 * L::kOPitch;
#pragma unroll
        for (int ti = 0; ti < NT; ++ti) {
            float l = l_run[ti];
            l = rows_sum(l);
            __syncthreads();  // every wave is done with its V tile / the previous merge
            float* mine = om + wave * 16 * L::kOPitch + c * L::kOPitch;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                *reinterpret_cast<f32x4*>(mine + 16 * nb + 4 * g) = acc[ti][nb];
            if (g == 0) {
                mls[(wave * 16 + c) * 2] = m_run[ti];
                mls[(wave * 16 + c) * 2 + 1] = l;
            }
            __syncthreads();
            const int rows_here = min(16, qr1 - (qr0 + ti * 16));
            constexpr int QD = D / 4;  // four dims per thread and step
            for (int idx = threadIdx.x; idx < rows_here * QD; idx += kThreads) {
                const int qc = idx / QD, d = 4 * (idx - qc * QD);
                const int qrow = qr0 + ti * 16 + qc;
                float mmax = kNegInf;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) mmax = fmaxf(mmax, mls[(w * 16 + qc) * 2]);
                f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
                float lsum = 0.0f;
                if (mmax != kNegInf) {
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) {
                        const float mw = mls[(w * 16 + qc) * 2];
                        const float f = mw == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(mw - mmax);
                        o += *reinterpret_cast<const f32x4*>(om + (w * 16 + qc) * L::kOPitch + d) * f;
                        lsum += mls[(w * 16 + qc) * 2 + 1] * f;
                    }
                }
                const int t = e.q0 + qrow / a.G, hq = h * a.G + qrow % a.G;
                if constexpr (DIRECT) {
                    // One partition holds the row's keys: the reduce's arithmetic here, written
                    // only where the reduce would write it (row_request names this entry).
                    // positions[t] is loaded beside row_request[t] (independent loads, one wait).
                    const int32_t owner = a.row_request[t];
                    const int32_t pos_t = plan_position(a, t);
                    if (owner != r) continue;
                    float scale = 0.0f;  // no visible key: exact zeros
                    if (lsum > 0.0f) {
                        if (a.sinks != nullptr) {
                            const float sink = a.sinks[hq] * kLog2e;
                            const float top = fmaxf(mmax, sink);
                            const float f = __builtin_amdgcn_exp2f(mmax - top);
                            scale = f / (lsum * f + __builtin_amdgcn_exp2f(sink - top));
                        } else {
                            scale = 1.0f / lsum;
                        }
                    }
                    o *= scale;
                    u32x2 packed{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])};
                    if (row_breaks_plan(a, t, pos_t, true, e)) {
                        broken_plan(a);
                        packed = u32x2{kNanBf16x2, kNanBf16x2};
                    }
                    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + static_cast<int64_t>(t) * a.out_srow +
                                              static_cast<int64_t>(hq) * a.out_shead + d) = packed;
                    continue;
                }
                store_partial4(a, t, hq, p, d, o, lsum);
                if (d == 0) {
                    float* ml = part_ml_ptr(a, t, hq, p);
                    ml[0] = mmax;
                    ml[1] = lsum;
                }
            }
        }
    }

}

// ---- multi-row partition kernel (verify, prefill) -----------------------------------------------

// The workgroup's waves share every 32-key block: the workgroup stages K and V once per block in
// an LDS ring of kStages blocks (the waves split each block's global_load_lds instructions, whole
// key rows per instruction, streaming), and each wave owns its own 16-q-row tiles. Block
// i+kStages-1 is issued as soon as every wave is done with block i-1, so kStages-1 blocks are in
// flight per workgroup. K tiles keep key k's row at k * 2D with chunk q at slot q ^ k_swizzle(k),
// so a wave's MFMA A operand reads (16 keys, one chunk each) touch distinct banks; V tiles use
// the decode kernel's layout and transposed reads. No cross-wave merge: a wave writes its tiles'
// partials, or with direct output the normalized rows.
template <int D>
struct VerifyLds {
    static constexpr int kTile = 32 * D * 2;     // one member of one 32-key block, bf16
    static constexpr int kStage = 2 * kTile;     // K then V
    static constexpr int kStages = 3;
    static constexpr int kBytes = kStages * kStage;
};

template <int D>
__device__ __forceinline__ int k_swizzle(int key) {
    // D 64: two keys per 256 bytes, eight chunks a row; D >= 128: one key or more per 256 bytes.
    return D == 64 ? (key >> 1) & 7 : key & 15;
}

// The multi-row kernel's waves take TPW 16-row tiles each: one for verify-sized steps (a step of
// 16 rows x G heads is four tiles, one per wave), two for prefill-sized ones, where every K and V
// operand a wave reads from LDS then feeds two MFMAs and each wave carries two independent
// dependency chains.
// TPW 1: three workgroups per CU (LDS 3 x 48 KiB at D 128; at most 168 VGPRs per lane, which the
// kernel fits without spilling): measured 78 -> 68 us on DFlash verify (16 entries x 16 rows)
// against the compiler's 184-VGPR
// two-per-CU choice. TPW 2: two per CU (the second tile's q operand and accumulators). Four
// tiles per wave (one wave per SIMD) measured 169 us on chunked prefill (4 x 512 rows after 2k
// keys) against 119 us with two.
template <int TPW>
constexpr int verify_waves_per_eu() { return TPW == 1 ? 3 : 2; }

template <int D, int TPW, int W>
__global__ __launch_bounds__(64 * W)
__attribute__((amdgpu_waves_per_eu(verify_waves_per_eu<TPW>(), verify_waves_per_eu<TPW>())))
void attn_partition_verify(AttnArgs a) {
    constexpr int KK = D / 32;
    constexpr int NB = D / 16;
    constexpr int CPK = D / 8;     // 16-byte chunks per key row
    constexpr int KPI = 64 / CPK;  // keys per load instruction
    constexpr int kWaves = W;
    constexpr int kThreads = 64 * W;
    constexpr int kLoads = 4 * KK / W;  // 1 KiB DMA instructions per wave per block
    constexpr int kRowsWg = kWaves * TPW * 16;
    using L = VerifyLds<D>;
    constexpr int S = L::kStages;
    __shared__ __attribute__((aligned(16))) char lds[L::kBytes];
    // Staged partial rows (the epilogue): D bf16 and 16 bytes of padding, which spreads the
    // rows' 8-byte writes over the LDS banks.
    constexpr int kStagePitch = 2 * D + 16;
    static_assert(kWaves * TPW * 16 * kStagePitch <= L::kBytes, "the staged partials fit the ring");

    const WgCoord wc = work_coord(a);
    const int r = static_cast<int>(wc.z), h = static_cast<int>(wc.y);
    if (r == a.R) {  // only in a direct-output grid
        zero_dead_rows<kThreads>(a, reinterpret_cast<int*>(lds));
        return;
    }
    const int tg0 = static_cast<int>(wc.x) / a.grid_parts;
    Entry e;
    if (!load_entry(a, r, e)) return;
    split_entry(a, e);
    const int p = part_slot(a, wc.x, wc.y, wc.z);
    const int part_lo = part_start(e, p);
    if (part_lo >= e.seq_len) return;
    const int part_hi = min(part_lo + e.part, e.seq_len);
    // Fused append (at most four tile groups per partition): this step's rows are the entry's
    // last n_rows keys; every workgroup whose partition holds a row writes its K and V for head h
    // before anything is loaded, and the barrier orders its own stores before its ring's loads of
    // the same slots. The partition's other tile groups write the same bytes to the same slots,
    // so whichever store a load sees, it reads the new row.
    if (a.k_new != nullptr) {
        const int first_new = e.seq_len - e.n_rows;
        append_rows_of_entry<D, 64 * W>(a, e, h, max(0, part_lo - first_new),
                                        min(e.n_rows, part_hi - first_new));
        __syncthreads();
    }

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int c = lane & 15, g = lane >> 4;
    const char* cache = static_cast<const char*>(a.c.base);
    const int64_t head_bytes = static_cast<int64_t>(h) * a.c.s_head * 2;
    const int64_t kv_bytes = a.c.s_kv * 2;
    const int n_tiles = (e.n_q + 15) / 16;
    const int64_t table_row = static_cast<int64_t>(r) * a.table_stride;
    const int block = static_cast<int>(a.c.block);
    const int n_pages_seq = (e.seq_len + block - 1) / block;

    // Loading: a stage is 4 * KK instructions of 1 KiB, (member, slice s, j) in that order; wave
    // w issues instructions w, w + W, ... Instruction j of a slice covers keys j * KPI + l / CPK,
    // lane l taking slot l % CPK of its key's row.
    uint32_t ld_src[kLoads], ld_dst[kLoads];
#pragma unroll
    for (int bi = 0; bi < kLoads; ++bi) {
        const int b = wave + kWaves * bi;
        const int member = b / (2 * KK), s = (b / KK) & 1, j = b % KK;
        const int key = j * KPI + lane / CPK;
        const int sw = member == 0 ? k_swizzle<D>(key) : v_swizzle<D>(key);
        ld_src[bi] = static_cast<uint32_t>(member * kv_bytes + key * a.c.s_row * 2 +
                                           ((lane % CPK) ^ sw) * 16);
        ld_dst[bi] = static_cast<uint32_t>(member * L::kTile + (s * KK + j) * 1024);
    }
    // LDS read addresses within a ring slot (the slot's offset is an immediate of each read).
    // K operand reads: lane (c, g) takes key 16s + c, chunk 4kk + g.
    const uint32_t lds0 = lds_addr(lds);
    uint32_t k_rd[2][KK];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
            k_rd[s2][kk] = lds0 + static_cast<uint32_t>((16 * s2 + c) * 2 * D + (((4 * kk + g) ^ k_swizzle<D>(c)) * 16));
    // V operand reads (transposed): lane (c, g) reads key row 4g + c/4 of each slice, column
    // block nb's chunk 2nb + (c & 3)/2 at its swizzled slot.
    uint32_t v_rd[NB];
    {
        const int r_row = 4 * g + (c >> 2);
        const int v_sw = v_swizzle<D>(r_row);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            v_rd[nb] = lds0 + static_cast<uint32_t>(r_row * 2 * D + (c & 1) * 8 +
                                                    (((2 * nb + ((c & 3) >> 1)) ^ v_sw) * 16));
    }

    for (int tg = tg0; tg * kWaves * TPW < n_tiles; tg += a.tile_groups) {
        const int qr0 = tg * kRowsWg;
        const int qr1 = min(qr0 + kRowsWg, e.n_q);
        int lo, hi;
        visible_span(a, e, qr0, qr1, lo, hi);
        lo = max(lo, part_lo);
        hi = min(hi, part_hi);
        if (lo >= hi) continue;  // uniform: no q-row of this group reads this partition
        // This wave's tiles: q-rows tq0 + 16t + c, t < TPW.
        const int tq0 = qr0 + wave * TPW * 16;
        const bool has_tile = tq0 < qr1;
        const int pos_first = e.seq_len - e.n_rows + min(tq0, e.n_q - 1) / a.G;
        const int pos_last = e.seq_len - e.n_rows + (min(tq0 + TPW * 16, qr1) - 1) / a.G;
        const int full_hi = a.causal ? pos_first + 1 : e.seq_len;
        const int full_lo = a.window > 0 ? pos_last - a.window + 1 : 0;

        u32x4 qb[TPW][KK];
        // Direct output writes a row only where the reduce would (row_request names this entry);
        // the row's position for the plan check is loaded here, so the load overlaps the blocks.
        bool own[TPW];
        int32_t own_pos[TPW];
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const int qrow = tq0 + 16 * t + c;
            const bool ok = qrow < qr1;
            const int tok = e.q0 + (ok ? qrow / a.G : 0);
            own[t] = ok && (!a.direct || a.row_request[tok] == r);
            own_pos[t] = a.direct ? plan_position(a, tok) : 0;
            const int hq = h * a.G + (ok ? qrow % a.G : 0);
            const char* qp = static_cast<const char*>(a.q) +
                             (static_cast<int64_t>(tok) * a.q_srow + static_cast<int64_t>(hq) * a.q_shead) * 2;
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                const u32x4 x = *reinterpret_cast<const u32x4*>(qp + (32 * kk + 8 * g) * 2);
                qb[t][kk] = ok ? x : u32x4{0, 0, 0, 0};
            }
        }
        f32x4 acc[TPW][NB];
        float m_run[TPW], l_run[TPW];
        // Two tiles per wave sum each row's probabilities on the matrix unit, which has room (the
        // vector unit has less): one more PV MFMA per tile and block against an all-ones V block
        // gives every lane of row c its sum over the block's keys, in place of eight adds a tile
        // and the final cross-lane sum. (It sums the bf16 probabilities the PV MFMAs use.)
        constexpr bool kSumMfma = TPW == 2;
        f32x4 acc_l[kSumMfma ? TPW : 1];
        // m_thr: the raw score (before the log2-unit scale) above which a row rescales.
        float m_thr[TPW];
        float neg_m[TPW];  // -m_run (0 while no key is visible): the exp argument's offset
        const float inv_scale = 1.0f / a.score_scale_log2;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[t][nb] = f32x4{0, 0, 0, 0};
            m_run[t] = kNegInf;
            m_thr[t] = kNegInf;
            neg_m[t] = 0.0f;
            l_run[t] = 0.0f;
            if constexpr (kSumMfma) acc_l[t] = f32x4{0, 0, 0, 0};
        }

        const int kb_first = lo / 32, kb_last = (hi - 1) / 32;
        const int n_kb = kb_last - kb_first + 1;

        for (int chunk = 0; chunk < n_kb; chunk += 32) {
            // Byte offsets of the next 32 blocks' slices (page, row in the page, kv head), one
            // (block, slice) per lane of every wave, so issuing a block is two lane reads per
            // slice. A missing page reads the null page 0; its keys are past the context.
            uint64_t my_off = 0;
            {
                const int i = chunk + (lane >> 1);
                const int key0 = (kb_first + i) * 32 + (lane & 1) * 16;
                int pid = 0;
                if (i < n_kb && key0 < e.seq_len) {
                    const int pi = key0 / block;
                    if (pi < n_pages_seq) {
                        const int id = a.table[table_row + pi];
                        if (id >= 0 && id < a.c.num_pages) pid = id;
                    }
                }
                my_off = static_cast<uint64_t>(static_cast<int64_t>(pid) * a.c.s_page * 2 +
                                               static_cast<int64_t>(key0 % block) * a.c.s_row * 2 + head_bytes);
            }
            const uint32_t off_lo = static_cast<uint32_t>(my_off), off_hi = static_cast<uint32_t>(my_off >> 32);
            const int n_here = min(32, n_kb - chunk);

            // This wave's quarter of block i, into ring slot `slot`.
            auto load_stage = [&](int i, int slot) {
                char* stage = lds + slot * L::kStage;
                const char* base[2];
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const uint32_t lo32 = __builtin_amdgcn_readlane(off_lo, 2 * i + s2);
                    const uint32_t hi32 = __builtin_amdgcn_readlane(off_hi, 2 * i + s2);
                    base[s2] = cache + ((static_cast<uint64_t>(hi32) << 32) | lo32);
                }
#pragma unroll
                for (int bi = 0; bi < kLoads; ++bi) {
                    const int b = wave + kWaves * bi;
                    const int s2 = (b / KK) & 1;
                    load_lds16<kPolicyStream>(base[s2] + ld_src[bi], stage + ld_dst[bi]);
                }
            };

            auto compute_stage = [&](int i, auto slot_c) {
                const int kb = kb_first + chunk + i;
                constexpr int kOff = decltype(slot_c)::value * L::kStage;
                u32x4 kop[2][KK];
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) kop[s2][kk] = lds_read_b128_at<kOff>(k_rd[s2][kk]);
                // Two tiles per wave (the registers allow it): the block's V operand reads go out
                // right behind K's and land while QK^T and the softmax run; the wait lets them stay
                // outstanding. One tile per wave reads V in batches after the softmax.
                constexpr bool kEarlyV = TPW == 2;
                v4s vlo[kEarlyV ? NB : 1], vhi[kEarlyV ? NB : 1];
                if constexpr (kEarlyV) {
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        vlo[nb] = lds_read_tr16_at<kOff + L::kTile>(v_rd[nb]);
                        vhi[nb] = lds_read_tr16_at<kOff + L::kTile + KK * 1024>(v_rd[nb]);
                    }
                    wait_lds<(2 * NB < 15 ? 2 * NB : 15)>();
                } else {
                    wait_lds_ops();
                }
                float sc[TPW][2][4];
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    f32x4 acc_s[TPW];
#pragma unroll
                    for (int t = 0; t < TPW; ++t) acc_s[t] = f32x4{0, 0, 0, 0};
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) {
                        after_wait(kop[s2][kk]);
#pragma unroll
                        for (int t = 0; t < TPW; ++t)
                            acc_s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, kop[s2][kk]), __builtin_bit_cast(bf16x8, qb[t][kk]),
                                acc_s[t], 0, 0, 0);
                    }
#pragma unroll
                    for (int t = 0; t < TPW; ++t)
#pragma unroll
                        for (int j = 0; j < 4; ++j) sc[t][s2][j] = acc_s[t][j];  // raw: scaled in exp2's fma
                }
                if (kb * 32 < full_lo || kb * 32 + 32 > full_hi) {
#pragma unroll
                    for (int t = 0; t < TPW; ++t) {
                        const int qrow = tq0 + 16 * t + c;
                        const int pos = e.seq_len - e.n_rows + qrow / a.G;
                        const int vis_hi = a.causal ? min(pos + 1, e.seq_len) : e.seq_len;
                        const int vis_lo = a.window > 0 ? pos - a.window + 1 : 0;
#pragma unroll
                        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const int key = kb * 32 + s2 * 16 + 4 * g + j;
                                if (key >= vis_hi || key < vis_lo) sc[t][s2][j] = kNegInf;
                            }
                    }
                }
                u32x4 pb[TPW];
#pragma unroll
                for (int t = 0; t < TPW; ++t) {
                    // This lane's raw maximum against the row's threshold: a row rescales when
                    // its block maximum exceeds its running one by more than kRescaleLog2, i.e.
                    // when one of its lanes' maxima does. Only then is the row maximum formed
                    // (cross-lane), so most blocks skip it.
                    float mx = kNegInf;
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, sc[t][s2][j]);
                    if (__builtin_amdgcn_ballot_w64(mx > m_thr[t])) {
                        const float m_new = fmaxf(m_run[t], rows_max(mx) * a.score_scale_log2);
                        const float alpha = m_new == kNegInf ? 1.0f : __builtin_amdgcn_exp2f(m_run[t] - m_new);
                        if constexpr (kSumMfma)
                            acc_l[t] *= alpha;
                        else
                            l_run[t] *= alpha;
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb) acc[t][nb] *= alpha;
                        m_run[t] = m_new;
                        m_thr[t] = (m_new + kRescaleLog2) * inv_scale;
                        neg_m[t] = m_new == kNegInf ? 0.0f : -m_new;
                    }
                    float pr[2][4];
                    float sum = 0.0f;
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            pr[s2][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][s2][j], a.score_scale_log2, neg_m[t]));
                            sum += pr[s2][j];
                        }
                    if constexpr (!kSumMfma) l_run[t] += sum;
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2) {
                        pb[t][2 * s2] = pack_prob(pr[s2][0], pr[s2][1]);
                        pb[t][2 * s2 + 1] = pack_prob(pr[s2][2], pr[s2][3]);
                    }
                }
                if constexpr (kSumMfma) {
                    constexpr uint32_t kOnes = 0x3f803f80u;  // a bf16 pair of 1.0
                    const u32x4 ones = {kOnes, kOnes, kOnes, kOnes};
#pragma unroll
                    for (int t = 0; t < TPW; ++t)
                        acc_l[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, ones), __builtin_bit_cast(bf16x8, pb[t]), acc_l[t], 0, 0, 0);
                }
                if constexpr (kEarlyV) {
                    wait_lds_ops();
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        after_wait(vlo[nb]);
                        after_wait(vhi[nb]);
                        const u32x2 lo2 = __builtin_bit_cast(u32x2, vlo[nb]), hi2 = __builtin_bit_cast(u32x2, vhi[nb]);
                        const u32x4 va = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
                        for (int t = 0; t < TPW; ++t)
                            acc[t][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, va), __builtin_bit_cast(bf16x8, pb[t]), acc[t][nb], 0, 0, 0);
                    }
                    return;
                }
                constexpr int kBatch = NB < 4 ? NB : 4;
#pragma unroll
                for (int nb0 = 0; nb0 < NB; nb0 += kBatch) {
                    v4s lo_b[kBatch], hi_b[kBatch];
#pragma unroll
                    for (int j = 0; j < kBatch; ++j) {
                        lo_b[j] = lds_read_tr16_at<kOff + L::kTile>(v_rd[nb0 + j]);
                        hi_b[j] = lds_read_tr16_at<kOff + L::kTile + KK * 1024>(v_rd[nb0 + j]);
                    }
                    wait_lds_ops();
#pragma unroll
                    for (int j = 0; j < kBatch; ++j) {
                        after_wait(lo_b[j]);
                        after_wait(hi_b[j]);
                        const v4s lo4 = lo_b[j], hi4 = hi_b[j];
                        u32x4 va;
                        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo4), hi2 = __builtin_bit_cast(u32x2, hi4);
                        va = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
#pragma unroll
                        for (int t = 0; t < TPW; ++t)
                            acc[t][nb0 + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, va), __builtin_bit_cast(bf16x8, pb[t]), acc[t][nb0 + j],
                                0, 0, 0);
                    }
                }
            };

            // Ring: blocks 0 .. S-2 in flight first; at block i, wait for this wave's loads of
            // block i (the S-2 later blocks stay outstanding), a barrier (every wave's loads of
            // block i have landed, and every wave is done with block i-1), then issue block
            // i+S-1 into block i-1's slot and compute block i. The barrier carries no memory
            // fence: LDS needs none, and a fence would wait for every outstanding load.
#pragma unroll
            for (int i = 0; i < S - 1; ++i)
                if (i < n_here) load_stage(i, i);
            // One block per step, unrolled by S so every ring slot is a compile-time offset.
            auto step = [&](auto u_c, int i) {
                constexpr int u = decltype(u_c)::value;
                if (i + S - 2 < n_here) wait_vmem<(S - 2) * kLoads>(); else wait_vmem<0>();
                __builtin_amdgcn_s_barrier();
                if (i + S - 1 < n_here) load_stage(i + S - 1, (u + S - 1) % S);
                const int kb = kb_first + chunk + i;
                if (kb * 32 + 32 > e.seq_len) {
                    // V rows past the context may hold anything (NaN included): zero them so a
                    // zero probability cannot turn into NaN. This is the workgroup's last
                    // block, so nothing else is in flight; all threads share the rows, then
                    // a barrier before anyone reads the tile.
                    char* vt = lds + u * L::kStage + L::kTile;
                    for (int idx = static_cast<int>(threadIdx.x); idx < 32 * CPK; idx += kThreads) {
                        const int key = idx / CPK;
                        if (kb * 32 + key >= e.seq_len)
                            *reinterpret_cast<u32x4*>(vt + key * 2 * D + (idx % CPK) * 16) = u32x4{0, 0, 0, 0};
                    }
                    __syncthreads();
                }
                if (has_tile) compute_stage(i, u_c);
            };
            static_assert(S == 3, "the step loop below is unrolled by three");
            for (int i0 = 0; i0 < n_here; i0 += S) {
                step(std::integral_constant<int, 0>{}, i0);
                if (i0 + 1 >= n_here) break;
                step(std::integral_constant<int, 1>{}, i0 + 1);
                if (i0 + 2 >= n_here) break;
                step(std::integral_constant<int, 2>{}, i0 + 2);
            }
            wait_vmem_all();
            __builtin_amdgcn_s_barrier();  // the next chunk / tile group reuses the ring
        }

        // This wave's tile partials: lane (c, g) holds q-row tq0 + 16t + c, dims 16nb + 4g + i.
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            float l;
            if constexpr (kSumMfma)
                l = acc_l[t][0];
            else
                l = rows_sum(l_run[t]);
            const int qrow = tq0 + 16 * t + c;
            if (a.direct) {
                // The reduce's arithmetic for a row with a single partition, in bf16.
                if (!has_tile || !own[t]) continue;
                const int tok = e.q0 + qrow / a.G, hq = h * a.G + qrow % a.G;
                float scale = 0.0f;  // no visible key: exact zeros
                if (l > 0.0f) {
                    if (a.sinks != nullptr) {
                        const float sink = a.sinks[hq] * kLog2e;
                        const float top = fmaxf(m_run[t], sink);
                        const float f = __builtin_amdgcn_exp2f(m_run[t] - top);
                        scale = f / (l * f + __builtin_amdgcn_exp2f(sink - top));
                    } else {
                        scale = 1.0f / l;
                    }
                }
                uint16_t* po = static_cast<uint16_t*>(a.out) + static_cast<int64_t>(tok) * a.out_srow +
                               static_cast<int64_t>(hq) * a.out_shead;
                const bool broken = row_breaks_plan(a, tok, own_pos[t], true, e);
                if (broken) broken_plan(a);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const f32x4 o = acc[t][nb] * scale;
                    *reinterpret_cast<u32x2*>(po + 16 * nb + 4 * g) =
                        broken ? u32x2{kNanBf16x2, kNanBf16x2} : u32x2{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])};
                }
                continue;
            }
            // Partials, staged through this wave's share of the ring (idle since the last
            // chunk's closing barrier): a lane holds 8-byte pieces of 16 rows, so storing from
            // registers writes 32 bytes of each of 16 rows per instruction; from the staged
            // tile, 16 lanes write one row's D values whole, 16 bytes each. (Measured on
            // DFlash verify: the scattered stores cost 4.4 us of a 58.6 us kernel.) The same
            // values as store_partial4.
            if (has_tile) {
                char* row_st = lds + (wave * TPW * 16 + 16 * t + c) * kStagePitch;
                const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const f32x4 o = acc[t][nb];
                    *reinterpret_cast<u32x2*>(row_st + (16 * nb + 4 * g) * 2) =
                        u32x2{pack_partial(o[0] * inv, o[1] * inv), pack_partial(o[2] * inv, o[3] * inv)};
                }
                if (g == 0 && qrow < qr1) {
                    const int tok = e.q0 + qrow / a.G, hq = h * a.G + qrow % a.G;
                    float* ml = part_ml_ptr(a, tok, hq, p);
                    ml[0] = m_run[t];
                    ml[1] = l;
                }
            }
        }
        if (!a.direct) {
            if (has_tile) {
                wave_sync_lds();  // this wave's staged rows are written
                constexpr int kRowsPerStore = 64 / CPK;
#pragma unroll
                for (int r0 = 0; r0 < TPW * 16; r0 += kRowsPerStore) {
                    const int row = r0 + lane / CPK, ch = lane % CPK;
                    const int qrow = tq0 + row;
                    const u32x4 val = *reinterpret_cast<const u32x4*>(
                        lds + (wave * TPW * 16 + row) * kStagePitch + ch * 16);
                    if (qrow < qr1) {
                        const int tok = e.q0 + qrow / a.G, hq = h * a.G + qrow % a.G;
                        *reinterpret_cast<u32x4*>(part_o_bf16(a, tok, hq, p) + ch * 8) = val;
                    }
                }
            }
            __syncthreads();  // the next tile group's ring loads may land on the staged rows
        }
    }
}

// Decode (one row tile per group): sized for two waves per SIMD. An fp8 block is half the
// bytes of a bf16 one, so fp8 workgroups are two waves, each walking twice as many blocks; so
// are D 64 ones (a quarter of D 128's per-key bytes: measured 4% faster than four waves on
// gpt-oss decode, while at D 128 four waves are 1-3% faster). A one-partition (direct-output)
// D 64 launch takes four: its keys are few (a 128-key window spans at most five blocks), and
// with a wave keeping two blocks in flight, four waves have them all in flight at once (gpt-oss
// sliding-window decode: 9.25 against 9.34 us).
template <int D, bool FP8, bool DIRECT = false>
constexpr int decode_waves() { return FP8 || (D == 64 && !DIRECT) ? 2 : 4; }

template <int D, bool FP8, bool DIRECT>
__global__ __launch_bounds__((64 * decode_waves<D, FP8, DIRECT>())) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_partition_mfma_decode(AttnArgs a) {
    constexpr int W = decode_waves<D, FP8, DIRECT>();
    __shared__ __attribute__((aligned(16))) char lds[MfmaLdsV2<D, W>::kBytes];
    partition_body<D, 1, FP8, W, DIRECT>(a, lds);
}

// Multi-row fp8 steps: NT row tiles per wave, K/V read once per group.
template <int D, int NT, bool FP8>
__global__ __launch_bounds__(kThreads) void attn_partition_mfma(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) char lds[MfmaLdsV2<D, kWaves>::kBytes];
    partition_body<D, NT, FP8, kWaves>(a, lds);
}

// ---- generic partition kernel (VALU, f32 math; any float dtype, D <= 512) -----------------------

constexpr int kGenMaxD = 512;

__global__ __launch_bounds__(kThreads) void attn_partition_generic(AttnArgs a) {
    __shared__ float qs[kWaves][kGenMaxD];
    const int r = blockIdx.z, h = blockIdx.y;
    const int tg = blockIdx.x / a.grid_parts;
    Entry e;
    if (!load_entry(a, r, e)) return;
    split_entry(a, e);
    const int p = part_slot(a);
    const int part_lo = part_start(e, p);
    if (part_lo >= e.seq_len) return;
    const int part_hi = min(part_lo + e.part, e.seq_len);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int D = a.c.d;
    constexpr int kPer = kGenMaxD / 64;

    for (int qrow = tg * kWaves + wave; qrow < e.n_q; qrow += a.tile_groups * kWaves) {
        int lo, hi;
        visible_span(a, e, qrow, qrow + 1, lo, hi);
        lo = max(lo, part_lo);
        hi = min(hi, part_hi);
        const int t = e.q0 + qrow / a.G, hq = h * a.G + qrow % a.G;
        const int64_t qoff = static_cast<int64_t>(t) * a.q_srow + static_cast<int64_t>(hq) * a.q_shead;
        wave_sync_lds();  // the previous q-row's reads of qs are done
        for (int d = lane; d < D; d += 64) qs[wave][d] = load_as_f32(a.q, qoff + d, a.q_dt);
        wave_sync_lds();

        float m_run = kNegInf, l_run = 0.0f;
        float o[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) o[i] = 0.0f;
        for (int k0 = lo; k0 < hi; k0 += 64) {
            const int key = k0 + lane;
            float s = kNegInf;
            int64_t krow = -1;
            if (key < hi && key_visible(a, e, qrow, key)) {
                const int64_t pid = page_id(a, r, key / a.c.block);
                if (pid >= 0) {
                    krow = pid * a.c.s_page + (key % a.c.block) * a.c.s_row +
                           static_cast<int64_t>(h) * a.c.s_head;
                    float dot = 0.0f;
                    for (int d = 0; d < D; ++d)
                        dot = fmaf(qs[wave][d], load_as_f32(a.c.base, krow + d, a.c.dt), dot);
                    s = dot * a.score_scale_log2;
                }
            }
            const float m_new = fmaxf(m_run, wave_max(s));
            if (m_new == kNegInf) continue;
            const float alpha = exp2f(m_run - m_new);
            const float pr = exp2f(s - m_new);
            l_run = l_run * alpha + wave_sum(pr);
            m_run = m_new;
#pragma unroll
            for (int i = 0; i < kPer; ++i) o[i] *= alpha;
            const int n = min(64, hi - k0);
            for (int j = 0; j < n; ++j) {
                const float pj = __shfl(pr, j, 64);
                const int64_t vrow = __shfl(krow, j, 64);
                if (vrow < 0) continue;
#pragma unroll
                for (int i = 0; i < kPer; ++i) {
                    const int d = lane + 64 * i;
                    if (d < D) o[i] = fmaf(pj, load_as_f32(a.c.base, vrow + a.c.s_kv + d, a.c.dt), o[i]);
                }
            }
        }
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int d = lane + 64 * i;
            if (d >= D) continue;
            if (a.part_bf16)
                part_o_bf16(a, t, hq, p)[d] = f32_to_bf16(o[i] * inv);
            else
                part_o_f32(a, t, hq, p)[d] = o[i];
        }
        if (lane == 0) {
            float* ml = part_ml_ptr(a, t, hq, p);
            ml[0] = m_run;
            ml[1] = l_run;
        }
    }
}

// ---- reduce --------------------------------------------------------------------------------------

// One workgroup per (row, q head), any number of partitions; it reads exactly the partitions the
// row's visible keys fall in (the partition kernels wrote each of them). Threads are [partition
// lane][vector of D]; each thread folds partitions p_lo + pl, + n_pl, ... in one pass with a
// running max (eight loads in flight per batch), then the partition lanes merge through LDS.
constexpr int kReduceThreads = 256;
constexpr int kReduceBatch = 8;

template <bool BF16P>
__global__ __launch_bounds__(kReduceThreads) void attn_reduce(AttnArgs a) {
    __shared__ float red_o[kReduceThreads * 4];
    __shared__ float red_m[kReduceThreads];
    __shared__ float red_l[kReduceThreads];
    const int t = blockIdx.x, hq = blockIdx.y;
    const int D = a.c.d;
    const int vec = (D % 4 == 0) ? 4 : 1;
    const int n_vec = D / vec;
    const int lanes_d = min(n_vec, kReduceThreads);
    const int n_pl = kReduceThreads / lanes_d;  // partition lanes
    const int pl = threadIdx.x / lanes_d, vi = threadIdx.x % lanes_d;

    const int32_t pos_t = plan_position(a, t);
    Entry e;
    const bool live = row_live(a, t, e);
    const bool broken = row_breaks_plan(a, t, pos_t, live, e);
    int p_lo = 0, p_hi = -1;
    if (live) {
        int lo, hi;
        const int qrow = (t - e.q0) * a.G;
        visible_span(a, e, qrow, qrow + 1, lo, hi);
        hi = min(hi, e.seq_len);
        split_entry(a, e);
        p_lo = (lo - e.anchor) / e.part;
        p_hi = (hi - 1 - e.anchor) / e.part;
    }

    const int64_t out_base = static_cast<int64_t>(t) * a.out_srow + static_cast<int64_t>(hq) * a.out_shead;
    for (int v0 = 0; v0 < n_vec; v0 += lanes_d) {
        const int v = v0 + vi;
        float m = kNegInf, l = 0.0f;
        f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
        if (pl < n_pl && v < n_vec) {
            for (int b = p_lo + pl; b <= p_hi; b += kReduceBatch * n_pl) {
                float mp[kReduceBatch], lp[kReduceBatch];
                f32x4 xp[kReduceBatch];
                if (vec == 4) {
                    // The batch's loads all go out before one wait (untracked loads, as in
                    // attn_reduce_few); partitions past p_hi re-read partition b, masked below.
                    u32x2 mlr[kReduceBatch];
                    PartialRaw<BF16P> xr[kReduceBatch];
#pragma unroll
                    for (int j = 0; j < kReduceBatch; ++j) {
                        const int p = b + j * n_pl <= p_hi ? b + j * n_pl : b;
                        mlr[j] = load_x2_async(reinterpret_cast<const char*>(part_ml_ptr(a, t, hq, p)));
                        if constexpr (BF16P)
                            xr[j] = load_x2_async(reinterpret_cast<const char*>(part_o_bf16(a, t, hq, p) + v * 4));
                        else
                            xr[j] = __builtin_bit_cast(f32x4, load_x4_async(reinterpret_cast<const char*>(
                                                                  part_o_f32(a, t, hq, p) + v * 4)));
                    }
                    wait_vmem_all();
#pragma unroll
                    for (int j = 0; j < kReduceBatch; ++j) {
                        after_wait(mlr[j]);
                        after_wait(xr[j]);
                        const bool in = b + j * n_pl <= p_hi;
                        mp[j] = in ? __uint_as_float(mlr[j][0]) : kNegInf;
                        lp[j] = in ? __uint_as_float(mlr[j][1]) : 0.0f;
                        xp[j] = widen_partial<BF16P>(xr[j]);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < kReduceBatch; ++j) {
                        const int p = b + j * n_pl;
                        if (p <= p_hi) {
                            const float* ml = part_ml_ptr(a, t, hq, p);
                            mp[j] = ml[0];
                            lp[j] = ml[1];
                            xp[j] = f32x4{load_partial1<BF16P>(a, t, hq, p, v), 0.0f, 0.0f, 0.0f};
                        } else {
                            mp[j] = kNegInf;
                            lp[j] = 0.0f;
                            xp[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < kReduceBatch; ++j) {
                    const bool use = mp[j] != kNegInf;
                    const float mj = use ? mp[j] : kNegInf;
                    if (mj > m) {
                        const float f = m == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m - mj);
                        o *= f;
                        l *= f;
                        m = mj;
                    }
                    const float w = use ? __builtin_amdgcn_exp2f(mj - m) : 0.0f;
                    o += (use ? xp[j] : f32x4{0.0f, 0.0f, 0.0f, 0.0f}) * (w * partial_scale<BF16P>(lp[j]));
                    l += (use ? lp[j] : 0.0f) * w;
                }
            }
        }
        if (n_pl > 1) {
            __syncthreads();  // the previous vector chunk's merge reads are done
            red_o[threadIdx.x * 4 + 0] = o[0];
            red_o[threadIdx.x * 4 + 1] = o[1];
            red_o[threadIdx.x * 4 + 2] = o[2];
            red_o[threadIdx.x * 4 + 3] = o[3];
            red_m[threadIdx.x] = m;
            red_l[threadIdx.x] = l;
            __syncthreads();
            if (pl == 0) {
                for (int j = 1; j < n_pl; ++j) {
                    const int src = j * lanes_d + vi;
                    const float mj = red_m[src];
                    if (mj == kNegInf) continue;
                    const float top = fmaxf(m, mj);
                    const float fa = m == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m - top);
                    const float fb = __builtin_amdgcn_exp2f(mj - top);
                    const f32x4 ob = {red_o[src * 4], red_o[src * 4 + 1], red_o[src * 4 + 2], red_o[src * 4 + 3]};
                    o = o * fa + ob * fb;
                    l = l * fa + red_l[src] * fb;
                    m = top;
                }
            }
        }
        if (pl != 0 || v >= n_vec) continue;
        float scale = 0.0f;  // a dead row, or no visible key: exact zeros
        if (live && l > 0.0f) {
            if (a.sinks != nullptr) {
                const float sink = a.sinks[hq] * kLog2e;
                const float top = fmaxf(m, sink);
                const float f = __builtin_amdgcn_exp2f(m - top);
                scale = f / (l * f + __builtin_amdgcn_exp2f(sink - top));
            } else {
                scale = 1.0f / l;
            }
        }
        if (broken) {
            scale = __builtin_nanf("");  // every product NaN, zeros included
            if (vi == 0) broken_plan(a);
        }
        for (int i = 0; i < vec; ++i)
            store_from_f32(a.out, out_base + v * vec + i, a.out_dt, o[i] * scale);
    }
}

// Few partitions per row (at most kFewParts): one thread per (row, q head, 4 floats of D) folds
// all of its partitions; every load is issued up front (fully unrolled, predicated), so the
// whole reduce is two memory latencies with no synchronization. 256 threads = 256 / (D / 4)
// q heads of one row.
constexpr int kFewParts = 16;

template <bool BF16P>
__global__ __launch_bounds__(kReduceThreads) void attn_reduce_few(AttnArgs a) {
    const int D = a.c.d;
    const int n_vec = D / 4;
    const int heads_per_wg = kReduceThreads / n_vec;
    const int t = blockIdx.x;
    const int hq = blockIdx.y * heads_per_wg + static_cast<int>(threadIdx.x) / n_vec;
    const int v = static_cast<int>(threadIdx.x) % n_vec;
    if (hq >= a.H) return;
    const int32_t pos_t = plan_position(a, t);
    Entry e;
    const bool live = row_live(a, t, e);
    const bool broken = row_breaks_plan(a, t, pos_t, live, e);
    const int64_t out_base = static_cast<int64_t>(t) * a.out_srow + static_cast<int64_t>(hq) * a.out_shead + 4 * v;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    float scale = 0.0f;  // a dead row, or no visible key: exact zeros
    if (live) {
        int lo, hi;
        const int qrow = (t - e.q0) * a.G;
        visible_span(a, e, qrow, qrow + 1, lo, hi);
        hi = min(hi, e.seq_len);
        split_entry(a, e);
        const int p_lo = (lo - e.anchor) / e.part, n_p = (hi - 1 - e.anchor) / e.part - p_lo + 1;
        // Every (m, l) and partial load is issued before one wait: slots past n_p re-read slot
        // p_lo (L1 hits) and are masked after the loads. The loads are inline asm the compiler
        // does not track (it would otherwise wait for the maxima before issuing the partials).
        // Slots past the table's partition count are never loaded (a uniform, scalar bound).
        const int n_all = min(a.n_parts, kFewParts);
        u32x2 mlv[kFewParts];
        PartialRaw<BF16P> pv[kFewParts];
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) {
            mlv[i] = u32x2{0, 0};
            pv[i] = PartialRaw<BF16P>{};
            if (i >= n_all) break;
            const int p = p_lo + (i < n_p ? i : 0);
            mlv[i] = load_x2_async(reinterpret_cast<const char*>(part_ml_ptr(a, t, hq, p)));
            if constexpr (BF16P)
                pv[i] = load_x2_async(reinterpret_cast<const char*>(part_o_bf16(a, t, hq, p) + 4 * v));
            else
                pv[i] = __builtin_bit_cast(f32x4, load_x4_async(reinterpret_cast<const char*>(
                                                      part_o_f32(a, t, hq, p) + 4 * v)));
        }
        wait_vmem_all();
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) {
            after_wait(mlv[i]);
            after_wait(pv[i]);
        }
        float mv[kFewParts], lv[kFewParts];
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) {
            mv[i] = i < n_p ? __uint_as_float(mlv[i][0]) : kNegInf;
            lv[i] = i < n_p ? __uint_as_float(mlv[i][1]) : 0.0f;
        }
        float m = kNegInf;
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) m = fmaxf(m, mv[i]);
        float l = 0.0f;
        if (m != kNegInf) {
#pragma unroll
            for (int i = 0; i < kFewParts; ++i) {
                const float w = mv[i] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(mv[i] - m);
                const f32x4 x = i < n_p ? widen_partial<BF16P>(pv[i]) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                o += x * (w * partial_scale<BF16P>(lv[i]));
                l += lv[i] * w;
            }
        }
        if (l > 0.0f) {
            if (a.sinks != nullptr) {
                const float sink = a.sinks[hq] * kLog2e;
                const float top = fmaxf(m, sink);
                const float f = __builtin_amdgcn_exp2f(m - top);
                scale = f / (l * f + __builtin_amdgcn_exp2f(sink - top));
            } else {
                scale = 1.0f / l;
            }
        }
    }
    if (broken) {
        scale = __builtin_nanf("");  // every product NaN, zeros included
        if (threadIdx.x == 0) broken_plan(a);
    }
    if (a.out_dt == DT_BF16) {
        u32x2 w;
        w[0] = static_cast<uint32_t>(f32_to_bf16(o[0] * scale)) | (static_cast<uint32_t>(f32_to_bf16(o[1] * scale)) << 16);
        w[1] = static_cast<uint32_t>(f32_to_bf16(o[2] * scale)) | (static_cast<uint32_t>(f32_to_bf16(o[3] * scale)) << 16);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + out_base) = w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) store_from_f32(a.out, out_base + i, a.out_dt, o[i] * scale);
    }
}

// Few partitions with bf16 partials and a bf16 output (every MFMA step): attn_reduce_few with
// eight dims per thread, so 16-byte partial loads and output stores and half the threads.
__global__ __launch_bounds__(kReduceThreads) void attn_reduce_few_bf16x8(AttnArgs a) {
    const int D = a.c.d;
    const int n_vec = D / 8;
    const int heads_per_wg = kReduceThreads / n_vec;
    const int t = blockIdx.x;
    const int hq = blockIdx.y * heads_per_wg + static_cast<int>(threadIdx.x) / n_vec;
    const int v = static_cast<int>(threadIdx.x) % n_vec;
    if (hq >= a.H) return;
    const int32_t pos_t = plan_position(a, t);
    Entry e;
    const bool live = row_live(a, t, e);
    const bool broken = row_breaks_plan(a, t, pos_t, live, e);
    const int64_t out_base = static_cast<int64_t>(t) * a.out_srow + static_cast<int64_t>(hq) * a.out_shead + 8 * v;
    f32x4 o0 = {0.0f, 0.0f, 0.0f, 0.0f}, o1 = {0.0f, 0.0f, 0.0f, 0.0f};
    float scale = 0.0f;  // a dead row, or no visible key: exact zeros
    if (live) {
        int lo, hi;
        const int qrow = (t - e.q0) * a.G;
        visible_span(a, e, qrow, qrow + 1, lo, hi);
        hi = min(hi, e.seq_len);
        split_entry(a, e);
        const int p_lo = (lo - e.anchor) / e.part, n_p = (hi - 1 - e.anchor) / e.part - p_lo + 1;
        // As attn_reduce_few: every load issued before one wait, slots past n_p re-reading slot
        // p_lo and masked after.
        const int n_all = min(a.n_parts, kFewParts);
        u32x2 mlv[kFewParts];
        u32x4 pv[kFewParts];
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) {
            mlv[i] = u32x2{0, 0};
            pv[i] = u32x4{0, 0, 0, 0};
            if (i >= n_all) break;
            const int p = p_lo + (i < n_p ? i : 0);
            mlv[i] = load_x2_async(reinterpret_cast<const char*>(part_ml_ptr(a, t, hq, p)));
            pv[i] = load_x4_async(reinterpret_cast<const char*>(part_o_bf16(a, t, hq, p) + 8 * v));
        }
        wait_vmem_all();
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) {
            after_wait(mlv[i]);
            after_wait(pv[i]);
        }
        float mv[kFewParts], lv[kFewParts];
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) {
            mv[i] = i < n_p ? __uint_as_float(mlv[i][0]) : kNegInf;
            lv[i] = i < n_p ? __uint_as_float(mlv[i][1]) : 0.0f;
        }
        float m = kNegInf;
#pragma unroll
        for (int i = 0; i < kFewParts; ++i) m = fmaxf(m, mv[i]);
        float l = 0.0f;
        if (m != kNegInf) {
#pragma unroll
            for (int i = 0; i < kFewParts; ++i) {
                const float w = mv[i] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(mv[i] - m);
                // The same arithmetic as attn_reduce_few, element for element.
                const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
                const f32x4 x0 = i < n_p ? widen_partial<true>(u32x2{pv[i][0], pv[i][1]}) : zero;
                const f32x4 x1 = i < n_p ? widen_partial<true>(u32x2{pv[i][2], pv[i][3]}) : zero;
                const float f = w * partial_scale<true>(lv[i]);
                o0 += x0 * f;
                o1 += x1 * f;
                l += lv[i] * w;
            }
        }
        if (l > 0.0f) {
            if (a.sinks != nullptr) {
                const float sink = a.sinks[hq] * kLog2e;
                const float top = fmaxf(m, sink);
                const float f = __builtin_amdgcn_exp2f(m - top);
                scale = f / (l * f + __builtin_amdgcn_exp2f(sink - top));
            } else {
                scale = 1.0f / l;
            }
        }
    }
    if (broken) {
        scale = __builtin_nanf("");  // every product NaN, zeros included
        if (threadIdx.x == 0) broken_plan(a);
    }
    const f32x4 a0 = o0 * scale, a1 = o1 * scale;
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out) + out_base) =
        u32x4{pack_bf16(a0[0], a0[1]), pack_bf16(a0[2], a0[3]), pack_bf16(a1[0], a1[1]), pack_bf16(a1[2], a1[3])};
}

template <int D, bool FP8>
hipError_t launch_mfma(const AttnArgs& a, int nt, dim3 grid, hipStream_t s) {
    if (nt == 1) {
        if (a.direct)
            hipLaunchKernelGGL((attn_partition_mfma_decode<D, FP8, true>), grid,
                               dim3(64 * decode_waves<D, FP8, true>()), 0, s, a);
        else
            hipLaunchKernelGGL((attn_partition_mfma_decode<D, FP8, false>), grid,
                               dim3(64 * decode_waves<D, FP8>()), 0, s, a);
    } else if constexpr (!FP8) {
        // Multi-row bf16 steps: the verify kernel (K/V staged once per workgroup), four waves of
        // one row tile, or of two for prefill-sized steps (nt 8, D <= 128). (Two waves of two
        // tiles for verify-sized steps measured 3% slower on DFlash verify than four of one, and
        // still 1.5% slower with the two-tile kernel's early V reads and MFMA row sums.)
        if constexpr (D <= 128) {
            if (nt == 8) {
                hipLaunchKernelGGL((attn_partition_verify<D, 2, 4>), grid, dim3(256), 0, s, a);
                return hipGetLastError();
            }

        }
        hipLaunchKernelGGL((attn_partition_verify<D, 1, 4>), grid, dim3(256), 0, s, a);
    } else if (nt == 2) {
        hipLaunchKernelGGL((attn_partition_mfma<D, 2, FP8>), grid, dim3(kThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL((attn_partition_mfma<D, 4, FP8>), grid, dim3(kThreads), 0, s, a);
    }
    return hipGetLastError();
}

// The MFMA kernel's requirements: bf16 q over a bf16 or fp8 cache, D in {64, 128, 256}, blocks of
// whole 16-key slices, and the alignments of its 16-byte (bf16) / 8-byte (fp8) loads.
bool mfma_serves(const AttnArgs& a) {
    const bool mfma_dtypes = a.q_dt == DT_BF16 && (a.c.dt == DT_BF16 || a.c.dt == DT_FP8);
    const bool mfma_shape = (a.c.d == 64 || a.c.d == 128 || a.c.d == 256) && a.c.block % 16 == 0 &&
                            a.q_shead % 8 == 0 && a.q_srow % 8 == 0 &&
                            (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 &&
                            (a.c.dt == DT_FP8 ? (a.c.s_page % 8 == 0 && a.c.s_row % 8 == 0 &&
                                                 a.c.s_kv % 8 == 0 && a.c.s_head % 8 == 0 &&
                                                 (reinterpret_cast<uintptr_t>(a.c.base) & 7) == 0)
                                              : (a.c.s_page % 8 == 0 && a.c.s_row % 8 == 0 &&
                                                 a.c.s_kv % 8 == 0 && a.c.s_head % 8 == 0 &&
                                                 (reinterpret_cast<uintptr_t>(a.c.base) & 15) == 0));
    return mfma_dtypes && mfma_shape;
}

}  // namespace

bool attention_supported(const AttnArgs& a) {
    if (mfma_serves(a)) return true;
    // The generic kernel: any non-fp8 dtypes, D <= 512.
    return a.c.dt != DT_FP8 && a.q_dt != DT_FP8 && a.c.d <= kGenMaxD;
}

namespace {

// 16-row tiles per entry (rounded up over the step's average) and, for multi-row steps, the
// workgroups one (entry, kv head, partition) is spread over: each takes four tiles, at most 64.
int64_t tiles_per_entry(int64_t T, int64_t R, int64_t G) {
    return ((T * G + R - 1) / R + 15) / 16;
}

int64_t tile_groups_for(int64_t tiles) { return tiles <= 1 ? 1 : std::min<int64_t>(64, (tiles + 3) / 4); }

}  // namespace

SplitChoice choose_split(int64_t n_tokens, int64_t n_reqs, int64_t q_heads, int64_t kv_heads,
                         int64_t width, int64_t block, int32_t partition) {
    const int64_t keys = width * block;
    const auto cdiv = [](int64_t x, int64_t y) { return (x + y - 1) / y; };
    if (partition > 0)  // the caller's length, every entry alike
        return SplitChoice{partition, static_cast<int32_t>(std::max<int64_t>(1, cdiv(keys, partition))), 1};
    constexpr int32_t kBase = 512;
    if (n_tokens <= 0 || n_reqs <= 0 || kv_heads <= 0 || width <= 0 || block <= 0)
        return SplitChoice{kBase, 1, 0};
    const int64_t tiles = tiles_per_entry(n_tokens, n_reqs, q_heads / kv_heads);
    const int64_t groups = tile_groups_for(tiles);
    // Each entry is split on the device by its own length (split_entry): ceil(span / base)
    // partitions of equal length, at most `slots` of them. The slots bound the grid
    // (R x Hkv x tile groups x slots workgroups, the empty ones retire at once) and the
    // workspace; they are chosen from the step's shape, never from how wide the block table is
    // beyond what one entry could fill at the floor length. Every partition a workgroup serves
    // costs a fixed start (entry and table loads before its first K/V bytes) and end (partial
    // stores, whose HBM writes interleaved with the K/V stream cost far more per byte than the
    // reads); longer partitions amortize both, fewer workgroups balance worse. Measured on
    // MI355X:
    //  - decode: 512-key floor, slots for 2048+ workgroups over the grid and at least nine (64
    //    entries of 1-4k keys: partitions of <= 512 keys, nine slots; 4 entries of 128k: 65
    //    slots of 2048 keys);
    //  - multi-row steps of one row group per entry (verify, drafter) write a partial per row:
    //    896-key floor (16 entries of 16 rows over 0.5-8k keys: 512-key partitions averaged
    //    89.3 us a step, 800-1000 keys 85.0-85.7), slots for 1024+ workgroups, at least nine;
    //  - prefill-sized steps (8+ workgroups per partition from their rows alone) fill the grid
    //    with rows: slots only up to 1024 workgroups (4 x 512-row chunks after 2k keys: one
    //    partition, 124 us, against 155-176 us split).
    //  - decode over a table of at most 768 keys: one slot, so each entry is one partition and
    //    the kernel writes `out` with no reduce launch. Per layer of a 24-call graph: gpt-oss
    //    decode of 2-8 entries over <= 700 keys 7.0-8.6 us against 10.8-12.5 split; Llama-3-8B
    //    decode at 512 keys 9.5-16.4 us against 12.4-24.9 for 1-32 entries. At 1024 keys the
    //    split still wins up to 8 entries (13.7-19.4 against 12.4-16.4 us).
    // An odd slot count keeps the grid's x extent odd, which spreads each entry's partitions
    // over consecutive XCDs (part_slot).
    const int64_t wgs = n_reqs * kv_heads * groups;
    const bool prefill = groups >= 8;
    const bool multi_row = tiles > 1;
    constexpr int64_t kOnePartitionKeys = 768;
    if (!multi_row && keys <= kOnePartitionKeys) return SplitChoice{kBase, 1, 0};
    const int64_t base = prefill ? 512 : (multi_row ? 896 : kBase);
    int64_t cap = prefill ? std::max<int64_t>(1, 1024 / wgs)
                          : std::max<int64_t>(9, cdiv(multi_row ? 1024 : 2048, wgs));
    if (cap > 1 && cap % 2 == 0) cap += 1;
    const int64_t slots = std::min<int64_t>(cap, std::max<int64_t>(1, cdiv(keys, base)));
    return SplitChoice{static_cast<int32_t>(base), static_cast<int32_t>(slots), 0};
}

int64_t max_token_slots(int64_t max_tokens, int64_t max_reqs, int64_t q_heads, int64_t kv_heads,
                        int64_t width, int64_t block, int32_t partition) {
    if (max_tokens <= 0) return 0;
    if (partition > 0 || max_reqs <= 0)  // the slots do not depend on the step's rows
        return max_tokens * choose_split(max_tokens, std::max<int64_t>(1, max_reqs), q_heads, kv_heads,
                                         width, block, partition).slots;
    // choose_split reads a step's rows only through its row tiles per entry,
    // ceil(T * G / (16 * R)): slots are constant while the tiles stay within one of the ranges
    // {1}, [2, 4], [4g - 3, 4g] (g = 2..63) and [253, inf), so T * slots peaks at the largest T
    // of each range, T <= 16 * t_hi * R / G, or at max_tokens.
    const int64_t G = std::max<int64_t>(1, q_heads / std::max<int64_t>(1, kv_heads));
    int64_t best = 0;
    for (int64_t R = 1; R <= max_reqs; ++R) {
        const auto at = [&](int64_t T) {
            if (T >= 1 && T <= max_tokens)
                best = std::max(best, T * choose_split(T, R, q_heads, kv_heads, width, block, 0).slots);
        };
        at(max_tokens);
        at(16 * R / G);
        for (int64_t g = 1; g < 64; ++g) at(64 * g * R / G);
    }
    return best;
}

int32_t grid_slots(int32_t window, int64_t n_tokens, int32_t part, int32_t slots) {
    // With a window, an entry's visible keys span at most window + rows - 1 keys (rows <= T)
    // from its anchor's block, so at most window + T + 30 keys from the anchor; a split entry's
    // span from its anchor is at most that many keys too, so its share of the floor length
    // needs no more slots either.
    if (window <= 0) return slots;
    return static_cast<int32_t>(
        std::min<int64_t>(slots, (static_cast<int64_t>(window) + n_tokens + 30 + part - 1) / part));
}

// Row tiles per entry from which a bf16 multi-row step takes two tiles per wave.
constexpr int64_t kTwoTileMin = 16;

// The partition kernels' grid and row-tile choice for this shape.
void partition_shape(AttnArgs& a, int& nt, dim3& grid) {
    // Row tiles per workgroup: a step whose entries average one row (decode) needs one tile;
    // multi-row steps (verify) take up to four so K/V is read once for all of an entry's rows.
    const int64_t tiles = tiles_per_entry(a.T, a.R, a.G);
    nt = tiles <= 1 ? 1 : (tiles <= 2 ? 2 : 4);
    // Prefill-sized bf16 steps (two full workgroups of eight tiles or more): two tiles per wave.
    // (D 256 would spill the second tile's registers.)
    if (nt == 4 && tiles >= kTwoTileMin && a.c.d <= 128 && mfma_serves(a) && a.c.dt == DT_BF16) nt = 8;
    // Multi-row steps: a workgroup takes nt row tiles; long steps (prefill) spread the rest
    // over more workgroups, each reading the partition's K/V again (from L2 when they share it).
    a.tile_groups = nt > 1 ? static_cast<int>(std::min<int64_t>(64, (tiles + nt - 1) / nt)) : 1;
    grid = dim3(static_cast<unsigned>(a.grid_parts * a.tile_groups), static_cast<unsigned>(a.c.hkv),
                static_cast<unsigned>(a.R));
}

bool attention_fuses(const AttnArgs& a) {
    // Decode-shaped steps, bf16 or fp8 cache, and bf16 multi-row steps of one workgroup per
    // partition. An fp8 cache needs every page inside one partition (32 % block == 0): its
    // append rewrites whole pages' scales. (An earlier multi-row form that read the new keys
    // from k/v inside its block loop spilled past three waves per SIMD; the verify kernel writes
    // them to the cache before its loop instead, which costs no registers there.)
    if (!mfma_serves(a) || a.c.d % 8 != 0) return false;
    if (a.c.dt != DT_BF16 && !(a.c.dt == DT_FP8 && a.c.block > 0 && 32 % a.c.block == 0)) return false;
    AttnArgs b = a;
    int nt;
    dim3 grid;
    partition_shape(b, nt, grid);
    // Multi-row bf16 steps of at most four workgroups per partition (verify, drafter; gpt-oss's
    // 1 + 15 rows x 8 q heads take two): each of the partition's workgroups writes the
    // partition's new rows before reading its keys. Another workgroup of the partition may be
    // writing the same slots meanwhile, but with the same bytes, and a workgroup's own stores
    // are complete before its loads (its barrier), so every read sees the new row. Timed per
    // layer in a 24-call graph, gpt-oss decode_extra (1-8 entries of 16 rows) went from
    // 8.7-18.3 us with the append launch to 6.7-15.9. (Prefill-sized steps spread a
    // partition's rows over 8+ workgroups: the copies would cost more than the launch.)
    return nt == 1 || (a.c.dt == DT_BF16 && nt != 8 && b.tile_groups <= 4);
}

// Whether the partition kernel can write `out` itself: one partition holds every row's keys
// (the reduce would fold a single term; a window that fits a partition, or a short table), bf16
// out in 8-byte runs, and room in the grid's z dimension for the slice that zeroes dead rows.
// The decode body (bf16 or fp8 cache) and the bf16 multi-row kernel do; the fp8 multi-row
// kernel does not.
bool writes_direct(const AttnArgs& a, int nt) {
    return a.grid_parts == 1 && a.R < 65535 && a.out != nullptr && a.out_dt == DT_BF16 &&
           a.out_shead % 4 == 0 && a.out_srow % 4 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 7) == 0 &&
           mfma_serves(a) && (nt == 1 || a.c.dt == DT_BF16);
}

hipError_t launch_partitions(const AttnArgs& in, hipStream_t s) {
    AttnArgs a = in;
    if (a.T <= 0) return hipSuccess;
    if (!attention_supported(a)) return hipErrorNotSupported;
    int nt;
    dim3 grid;
    partition_shape(a, nt, grid);
    if (a.direct) {
        if (!writes_direct(a, nt)) return hipErrorInvalidValue;  // set only by launch_attention
        grid.z += 1;
    }
    if (a.k_new != nullptr && !attention_fuses(a)) return hipErrorInvalidValue;  // checked by the caller
    if (mfma_serves(a)) {
        if (!a.part_bf16) return hipErrorInvalidValue;  // MFMA kernels write bf16 partials (bf16 q)
        const bool fp8 = a.c.dt == DT_FP8;
        switch (a.c.d) {
            case 64: return fp8 ? launch_mfma<64, true>(a, nt, grid, s) : launch_mfma<64, false>(a, nt, grid, s);
            case 128: return fp8 ? launch_mfma<128, true>(a, nt, grid, s) : launch_mfma<128, false>(a, nt, grid, s);
            default: return fp8 ? launch_mfma<256, true>(a, nt, grid, s) : launch_mfma<256, false>(a, nt, grid, s);
        }
    }
    hipLaunchKernelGGL(attn_partition_generic, grid, dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_reduce(const AttnArgs& a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    const bool few = a.n_parts <= kFewParts && a.c.d % 4 == 0 && a.c.d / 4 <= kReduceThreads &&
                     (a.out_dt != DT_BF16 || (a.out_shead % 4 == 0 && a.out_srow % 4 == 0 &&
                                              (reinterpret_cast<uintptr_t>(a.out) & 7) == 0));
    if (few && a.part_bf16 && a.out_dt == DT_BF16 && a.c.d % 8 == 0 && a.c.d / 8 <= kReduceThreads &&
        a.out_shead % 8 == 0 && a.out_srow % 8 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
        const int heads_per_wg = kReduceThreads / (a.c.d / 8);
        const dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>((a.H + heads_per_wg - 1) / heads_per_wg));
        hipLaunchKernelGGL(attn_reduce_few_bf16x8, grid, dim3(kReduceThreads), 0, s, a);
    } else if (few) {
        const int heads_per_wg = kReduceThreads / (a.c.d / 4);
        const dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>((a.H + heads_per_wg - 1) / heads_per_wg));
        if (a.part_bf16)
            hipLaunchKernelGGL(attn_reduce_few<true>, grid, dim3(kReduceThreads), 0, s, a);
        else
            hipLaunchKernelGGL(attn_reduce_few<false>, grid, dim3(kReduceThreads), 0, s, a);
    } else {
        const dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>(a.H));
        if (a.part_bf16)
            hipLaunchKernelGGL(attn_reduce<true>, grid, dim3(kReduceThreads), 0, s, a);
        else
            hipLaunchKernelGGL(attn_reduce<false>, grid, dim3(kReduceThreads), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& in, hipStream_t s) {
    AttnArgs a = in;
    if (a.T > 0 && mfma_serves(a)) {
        AttnArgs b = a;
        int nt;
        dim3 grid;
        partition_shape(b, nt, grid);
        a.direct = writes_direct(b, nt) ? 1 : 0;
    }
    const hipError_t err = launch_partitions(a, s);
    if (err != hipSuccess || a.direct) return err;
    return launch_reduce(a, s);
}

}  // namespace kvpath
