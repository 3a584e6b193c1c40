// fp8 (e4m3fn) quantize-on-append with a per-(page, K/V, kv-head) fp32 scale.
//
// The rule (no reference counterpart: the reference's KV dtype is the model dtype,
// sdk/kv.py:76-143) and its helpers are in kvpath_fp8.h.
//
// append_fp8_runs (bf16 rows, D of 64, 128 or 256): a workgroup takes a chunk of consecutive
// rows; each of them that leads a run becomes 2 * Hkv units (member, kv head), and the
// workgroup's lane groups (D / 8 lanes: a lane owns 8 dims, 16 bytes of a bf16 row and 8 bytes of
// its e4m3 row) take the units round-robin. A unit loads its run's rows (the first 16 kept in
// registers, every load issued before the first use), reduces the absmax across its lanes,
// requantizes the page's other rows when the scale grew, and stores the run's rows as packed
// e4m3. Whole-page (prefill-shaped) appends take chunks of 16 rows, so each workgroup serves one
// page of every (member, head); decode-shaped ones take one row per workgroup, so every
// (row, member, head) unit runs in parallel.
//
// append_fp8_generic (any input dtype, any D or alignment): one workgroup per row, only run
// leaders work; a (member, head) pair is owned by a group of 16 lanes.
#include <algorithm>

#include "kvpath_device.h"
#include "kvpath_fp8.h"
#include "kvpath_internal.h"

namespace kvpath {
namespace {

constexpr int kThreads = 256;

// Eight values times r as eight e4m3 bytes, for a run whose inputs are all finite: then
// |x * r| <= 448 (1 + 3 * 2^-24) < 464 (r rounds 1 / s_new with s_new >= absmax / 448), which the
// conversion rounds to at most 448, so the clamp of quantize8 changes no result and is left out.
__device__ __forceinline__ u32x2 quantize8_finite(const float (&x)[8], float r) {
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[0] * r, x[1] * r, 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(x[2] * r, x[3] * r, lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(x[4] * r, x[5] * r, 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(x[6] * r, x[7] * r, hi, true);
    return u32x2{static_cast<uint32_t>(lo), static_cast<uint32_t>(hi)};
}

// Eight run values as stored: zeros when r = 0, else the finite or the clamped conversion.
// (r and finite are uniform over the unit's lanes.)
__device__ __forceinline__ u32x2 quantize_run8(const float (&x)[8], float r, bool finite) {
    if (!(r > 0.0f)) return u32x2{0, 0};
    return finite ? quantize8_finite(x, r) : quantize8(x, r);
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// The running maximum of |x| over 16 bytes of bf16, as bit patterns: with the sign bit cleared a
// bf16 orders as its 16-bit pattern (zeros, subnormals, normals, then inf at 0x7f80 and NaNs
// above), so two values take one packed integer maximum.
__device__ __forceinline__ u16x2 absmax_bits(u16x2 m, u32x4 w) {
#pragma unroll
    for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7fff7fffu));
    return m;
}

constexpr int kMaxChunk = 64;  // rows per workgroup at most
constexpr int kWindow = kMaxChunk + 64;  // slots staged in LDS: the chunk and the runs it leads
constexpr int kKeep = 16;  // run rows a unit keeps in registers between its two passes

template <int D>
__global__ __launch_bounds__(kThreads) void append_fp8_runs(AppendArgs a, int chunk) {
    constexpr int L = D / 8;             // lanes per unit
    constexpr int G = kThreads / L;      // units in flight per workgroup
    __shared__ int64_t s_slot[kWindow + 1];  // slots of rows c0 - 1 .. c0 + kWindow - 1
    __shared__ int s_lead[kMaxChunk];
    __shared__ int s_len[kMaxChunk];
    __shared__ uint64_t s_written[kMaxChunk];
    __shared__ int s_n;

    const int64_t block = a.c.block;
    const int64_t pool = a.c.num_pages * block;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * chunk;
    const int tid = static_cast<int>(threadIdx.x);
    if (tid == 0) s_n = 0;
    for (int i = tid; i < kWindow + 1; i += kThreads) {
        const int64_t t = c0 - 1 + i;
        s_slot[i] = (t >= 0 && t < a.T) ? static_cast<int64_t>(a.slots[t]) : -1;
    }
    __syncthreads();
    // Leaders of this chunk, with their runs: the rows after them in the same page.
    if (tid < chunk && c0 + tid < a.T) {
        const int64_t slot = s_slot[tid + 1];
        const int64_t page = page_of(slot, block, pool);
        if (page >= 0 && page_of(s_slot[tid], block, pool) != page) {
            uint64_t written = 1ull << (slot - page * block);
            int n = 1;
            for (;;) {
                const int64_t t = c0 + tid + n;
                if (t >= a.T) break;
                const int w = tid + n + 1;
                const int64_t s2 = w <= kWindow ? s_slot[w] : static_cast<int64_t>(a.slots[t]);
                if (page_of(s2, block, pool) != page) break;
                written |= 1ull << (s2 - page * block);
                ++n;
            }
            const int at = atomicAdd(&s_n, 1);
            s_lead[at] = static_cast<int>(c0 + tid);
            s_len[at] = n;
            s_written[at] = written;
        }
    }
    __syncthreads();

    const int hkv = a.c.hkv;
    const int n_units = s_n * 2 * hkv;
    const int grp = tid / L, lane = tid % L;
    uint8_t* cache = static_cast<uint8_t*>(a.c.base);
    for (int u = grp; u < n_units; u += G) {
        const int li = u / (2 * hkv), pair = u - li * 2 * hkv;
        const int m = pair / hkv, h = pair - m * hkv;
        const int64_t t0 = s_lead[li];
        const int n = s_len[li];
        const uint64_t written = s_written[li];
        const bool fresh = written & 1ull;
        const int64_t page = s_slot[t0 - c0 + 1] / block;
        const uint16_t* src = static_cast<const uint16_t*>(m ? a.v : a.k) +
                              h * (m ? a.v_shead : a.k_shead) + 8 * lane;
        const int64_t s_row = m ? a.v_srow : a.k_srow;
        float* scale_slot = a.c.scale + (page * 2 + m) * hkv + h;
        const int64_t head_base = page * a.c.s_page + m * a.c.s_kv + h * a.c.s_head + 8 * lane;

        // Pass 1: the run's absmax; its first kKeep rows stay in registers.
        u32x4 keep[kKeep];
#pragma unroll
        for (int j = 0; j < kKeep; ++j)
            keep[j] = j < n ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (t0 + j) * s_row))
                            : u32x4{0, 0, 0, 0};
        const float s_stored = *scale_slot;
        u16x2 mb = {0, 0};
#pragma unroll
        for (int j = 0; j < kKeep; ++j) mb = absmax_bits(mb, keep[j]);
        for (int j = kKeep; j < n; ++j)
            mb = absmax_bits(mb, *reinterpret_cast<const u32x4*>(src + (t0 + j) * s_row));
        uint32_t bits = max(static_cast<uint32_t>(mb[0]), static_cast<uint32_t>(mb[1]));
#pragma unroll
        for (int o = L / 2; o >= 1; o >>= 1) bits = max(bits, static_cast<uint32_t>(__shfl_xor(static_cast<int>(bits), o, L)));
        // All finite (the usual case): the bit maximum is the absmax. An inf or NaN takes the f32
        // rule (fmaxf skips NaNs) and the clamped conversion.
        const bool finite = bits < 0x7f80u;
        float amax = __uint_as_float(bits << 16);
        if (!finite) {
            amax = 0.0f;
            for (int j = 0; j < n; ++j) {
                float x[8];
                widen_bf16x8(*reinterpret_cast<const u32x4*>(src + (t0 + j) * s_row), x);
                amax = fmaxf(amax, absmax8(x));
            }
#pragma unroll
            for (int o = L / 2; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, L));
        }

        int k;
        const float s_new = grow_scale(fresh ? 0.0f : s_stored, __fdiv_rn(amax, kFp8Max), k);
        const float r_new = s_new > 0.0f ? __fdiv_rn(1.0f, s_new) : 0.0f;

        // The page's other rows, when the scale grew: f32(q) * 2^-k, requantized.
        if (k > 0) {
            for (int64_t row0 = 0; row0 < block; row0 += kKeep) {
                u32x2 q[kKeep];
#pragma unroll
                for (int j = 0; j < kKeep; ++j) {
                    const int64_t row = row0 + j;
                    q[j] = row < block && !(written >> row & 1ull)
                               ? *reinterpret_cast<const u32x2*>(cache + head_base + row * a.c.s_row)
                               : u32x2{0, 0};
                }
#pragma unroll
                for (int j = 0; j < kKeep; ++j) {
                    const int64_t row = row0 + j;
                    if (row >= block || (written >> row & 1ull)) continue;
                    *reinterpret_cast<u32x2*>(cache + head_base + row * a.c.s_row) = requant8(q[j], k);
                }
            }
        }

        // Pass 2: the run's rows, x * r_new. (The kept rows pass through an empty asm first, so
        // they are widened again here from their packed bf16 rather than pass 1's f32 copies
        // being held in registers across the requantization.)
#pragma unroll
        for (int j = 0; j < kKeep; ++j) asm volatile("" : "+v"(keep[j]));
#pragma unroll
        for (int j = 0; j < kKeep; ++j) {
            if (j < n) {
                float x[8];
                widen_bf16x8(keep[j], x);
                // The first kKeep rows of a run that starts in the chunk lie in the LDS window.
                const int64_t row = s_slot[t0 - c0 + 1 + j] - page * block;
                __builtin_nontemporal_store(quantize_run8(x, r_new, finite),
                                            reinterpret_cast<u32x2*>(cache + head_base + row * a.c.s_row));
            }
        }
        for (int j = kKeep; j < n; ++j) {
            float x[8];
            widen_bf16x8(*reinterpret_cast<const u32x4*>(src + (t0 + j) * s_row), x);
            const int64_t row = static_cast<int64_t>(a.slots[t0 + j]) - page * block;
            *reinterpret_cast<u32x2*>(cache + head_base + row * a.c.s_row) = quantize_run8(x, r_new, finite);
        }
        if (lane == 0) *scale_slot = s_new;
    }
}

constexpr int kGroup = 16;  // lanes per (member, head) in the generic kernel

__global__ __launch_bounds__(kThreads) void append_fp8_generic(AppendArgs a) {
    const int64_t t = blockIdx.x;
    const int64_t pool = a.c.num_pages * a.c.block;
    const int64_t page = page_of(a.slots[t], a.c.block, pool);
    if (page < 0) return;
    if (t > 0 && page_of(a.slots[t - 1], a.c.block, pool) == page) return;  // not the leader
    int64_t end = t + 1;
    while (end < a.T && page_of(a.slots[end], a.c.block, pool) == page) ++end;

    // Which rows of the page this run writes (block <= 64), and whether it starts the page.
    uint64_t written = 0;
    for (int64_t r = t; r < end; ++r) written |= 1ull << (a.slots[r] - page * a.c.block);
    const bool fresh = written & 1ull;

    uint8_t* cache = static_cast<uint8_t*>(a.c.base);
    const int lane = threadIdx.x % kGroup;
    const int n_pairs = 2 * a.c.hkv;
    for (int pair = threadIdx.x / kGroup; pair < n_pairs; pair += kThreads / kGroup) {
        const int m = pair / a.c.hkv;
        const int h = pair - m * a.c.hkv;
        const void* src = m ? a.v : a.k;
        const int64_t s_row = m ? a.v_srow : a.k_srow;
        const int64_t s_head = m ? a.v_shead : a.k_shead;

        float amax = 0.0f;
        for (int64_t r = t; r < end; ++r)
            for (int d = lane; d < a.c.d; d += kGroup)
                amax = fmaxf(amax, fabsf(load_as_f32(src, r * s_row + h * s_head + d, a.in_dt)));
#pragma unroll
        for (int o = kGroup / 2; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kGroup));

        float* scale_slot = a.c.scale + (page * 2 + m) * a.c.hkv + h;
        int k;
        const float s_new = grow_scale(fresh ? 0.0f : *scale_slot, __fdiv_rn(amax, kFp8Max), k);
        const float r_new = s_new > 0.0f ? __fdiv_rn(1.0f, s_new) : 0.0f;
        const int64_t head_base = page * a.c.s_page + m * a.c.s_kv + h * a.c.s_head;

        if (k > 0) {
            for (int64_t row = 0; row < a.c.block; ++row) {
                if (written >> row & 1ull) continue;
                uint8_t* p = cache + head_base + row * a.c.s_row;
                for (int d = lane; d < a.c.d; d += kGroup)
                    p[d] = f32_to_fp8(__builtin_amdgcn_ldexpf(fp8_to_f32(p[d]), -k));
            }
        }
        for (int64_t r = t; r < end; ++r) {
            uint8_t* p = cache + head_base + (a.slots[r] - page * a.c.block) * a.c.s_row;
            for (int d = lane; d < a.c.d; d += kGroup) {
                const float x = load_as_f32(src, r * s_row + h * s_head + d, a.in_dt);
                p[d] = r_new > 0.0f ? f32_to_fp8(__fmul_rn(x, r_new)) : 0;
            }
        }
        if (lane == 0) *scale_slot = s_new;
    }
}

// Whether append_fp8_runs serves this append: bf16 rows of D 64, 128 or 256 whose 16-byte
// chunks and 8-byte e4m3 chunks are aligned.
bool runs_serve(const AppendArgs& a) {
    const int d = a.c.d;
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return a.in_dt == DT_BF16 && (d == 64 || d == 128 || d == 256) && a16(a.k) && a16(a.v) &&
           a.k_srow % 8 == 0 && a.k_shead % 8 == 0 && a.v_srow % 8 == 0 && a.v_shead % 8 == 0 &&
           (reinterpret_cast<uintptr_t>(a.c.base) & 7) == 0 && a.c.s_page % 8 == 0 &&
           a.c.s_kv % 8 == 0 && a.c.s_row % 8 == 0 && a.c.s_head % 8 == 0;
}

}  // namespace

hipError_t launch_append_fp8(const AppendArgs& a, hipStream_t s) {
    if (a.T <= 0) return hipSuccess;
    if (runs_serve(a)) {
        // Rows per workgroup: one for decode-sized steps (every unit in parallel), growing with
        // the step to a page's 16 rows (one page of every (member, head) per workgroup).
        const int chunk = static_cast<int>(std::min<int64_t>(16, std::max<int64_t>(1, a.T / 2048)));
        const dim3 grid(static_cast<unsigned>((a.T + chunk - 1) / chunk));
        switch (a.c.d) {
            case 64: hipLaunchKernelGGL(append_fp8_runs<64>, grid, dim3(kThreads), 0, s, a, chunk); break;
            case 128: hipLaunchKernelGGL(append_fp8_runs<128>, grid, dim3(kThreads), 0, s, a, chunk); break;
            default: hipLaunchKernelGGL(append_fp8_runs<256>, grid, dim3(kThreads), 0, s, a, chunk); break;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(append_fp8_generic, dim3(static_cast<unsigned>(a.T)), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace kvpath
