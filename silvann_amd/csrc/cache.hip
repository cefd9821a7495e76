// cache.hip — the page-aware cache writer (appended row 141 `attention_cache_write_paged`): new key and value rows
// into their positions' slots of a paged (or contiguous) cache, keys turned by RoPE on the way.
//
// The reference has no writer: its rows verb points `rope_rows` at the cache row of the chunk's first position and
// the value projection at the value plane (engine/src/packages/nn/cpu/opcodes/attention__abi.cuh:13-14 P2, 398-406),
// which needs the cache to be contiguous. This door is that `rope_rows` (kernels.cuh:1710-1726) and that placement,
// with each row's slot looked up through its sequence's page table. HBM-bound byte work: every element is read and
// written once; no LDS, no matrix cores.
#include <algorithm>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

// The reference's own in-kernel bounds fault word "NPBN" (packages/nn/contracts/objects/primitives.cuh:5): a row
// whose position is at or past the cache's capacity is written nowhere and leaves it in the fault word.
constexpr unsigned int kFaultBounds = 0x4E50424Eu;

struct CacheArgs {
    uint16_t* kc;
    uint16_t* vc;
    const uint32_t* pages;
    uint64_t pages_row;
    uint64_t page_size;
    uint64_t capacity;
    const uint32_t* positions;
    uint64_t rows_per_seq;
    const uint16_t* k;
    const uint16_t* v;
    const float* cs;
    uint64_t rot;       // 0 when cs is NULL
    uint64_t rows, kv_heads, head_dim;
    uint64_t rope_units, k_units, units;   // per (row, kv head): RoPE units, key units, key + value units
    unsigned int* over;
};

// Halves from the cache plane's start to row r's slot; false when the row's position is past the capacity.
__device__ __forceinline__ bool slot_of(const CacheArgs& a, uint64_t r, uint64_t& at) {
    const uint64_t u = r / a.rows_per_seq;
    const uint64_t p = (uint64_t)a.positions[u] + r % a.rows_per_seq;
    if (p >= a.capacity) return false;
    const uint64_t slot = a.pages ? (uint64_t)a.pages[u * a.pages_row + p / a.page_size] * a.page_size + p % a.page_size
                                  : u * a.capacity + p;
    at = slot * a.kv_heads * a.head_dim;
    return true;
}

template <int W> struct Lanes;
template <> struct Lanes<8> {
    typedef u32x4 T;   // 8 halves
    static __device__ __forceinline__ void widen(T x, float* f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = half_bits_to_float((uint16_t)(x[i] & 0xFFFFu));
            f[2 * i + 1] = half_bits_to_float((uint16_t)(x[i] >> 16));
        }
    }
    static __device__ __forceinline__ T narrow(const float* f, bool& hit) {
        T x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = (uint32_t)to_half(f[2 * i], hit) | ((uint32_t)to_half(f[2 * i + 1], hit) << 16);
        return x;
    }
};
template <> struct Lanes<1> {
    typedef uint16_t T;
    static __device__ __forceinline__ void widen(T x, float* f) { f[0] = half_bits_to_float(x); }
    static __device__ __forceinline__ T narrow(const float* f, bool& hit) { return to_half(f[0], hit); }
};

// One unit a lane, W elements wide: of a (row, kv head), units [0, rope_units) turn elements j .. j+W-1 with their
// partners j+rot/2 .. (the reference's pair k: x[k], x[k + rot/2]), units up to k_units copy the key's unturned
// tail, the rest copy the value. The turn is the reference's arithmetic as its host family is built and runs it —
// a·c − b·s and b·c + a·s in fp32 contracted to fma(a, c, −(b·s)) and fma(b, c, a·s) (GCC's default contraction of
// kernels.cuh:1720-1724, matched bit for bit) — then RNE to fp16 with the overflow flag. Nothing else is contracted.
template <int W>
__global__ __launch_bounds__(256) void cache_write(CacheArgs a) {
#pragma clang fp contract(off)
    typedef typename Lanes<W>::T T;
    const uint64_t total = a.rows * a.kv_heads * a.units;
    const uint64_t pairs = a.rot / 2;
    bool hit = false, out = false;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256) {
        const uint64_t item = i / a.units, unit = i - item * a.units;
        const uint64_t r = item / a.kv_heads, h = item - r * a.kv_heads;
        uint64_t at;
        if (!slot_of(a, r, at)) {
            out = true;
            continue;
        }
        const uint64_t src = item * a.head_dim, dst = at + h * a.head_dim;
        if (unit < a.rope_units) {
            const uint64_t j = unit * W;
            float x0[W], x1[W], o0[W], o1[W];
            Lanes<W>::widen(*(const T*)(a.k + src + j), x0);
            Lanes<W>::widen(*(const T*)(a.k + src + j + pairs), x1);
            const float* c = a.cs + r * a.rot + j;
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const float co = c[e], si = c[pairs + e];
                o0[e] = __builtin_fmaf(x0[e], co, -(x1[e] * si));
                o1[e] = __builtin_fmaf(x1[e], co, x0[e] * si);
            }
            *(T*)(a.kc + dst + j) = Lanes<W>::narrow(o0, hit);
            *(T*)(a.kc + dst + j + pairs) = Lanes<W>::narrow(o1, hit);
        } else if (unit < a.k_units) {
            const uint64_t j = a.rot + (unit - a.rope_units) * W;
            *(T*)(a.kc + dst + j) = *(const T*)(a.k + src + j);
        } else {
            const uint64_t j = (unit - a.k_units) * W;
            *(T*)(a.vc + dst + j) = *(const T*)(a.v + src + j);
        }
    }
    // A row past the capacity outranks an overflow, whatever order the lanes get here in: the bounds fault is
    // stored, the overflow only goes into a clear word.
    if (hit) atomicCAS(a.over, 0u, kFaultOverflow);
    if (out) *a.over = kFaultBounds;
}

// `rope_rows` itself (kernels.cuh:1710-1726), every row's heads turned in place or into `o`: a lane a pair, the
// same two FMAs as the writer. Rows row_stride apart, heads head_stride apart, any alignment.
__global__ __launch_bounds__(256) void rope_rows_kernel(uint16_t* o, const uint16_t* x, const float* cs, uint64_t rows,
                                                        uint64_t heads, uint64_t head_stride, uint64_t row_stride,
                                                        uint64_t rot, unsigned int* over) {
#pragma clang fp contract(off)
    const uint64_t pairs = rot / 2, per_row = heads * pairs, n = rows * per_row;
    bool hit = false;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint64_t r = i / per_row, rest = i - r * per_row, e = rest / pairs, k = rest - e * pairs;
        const uint64_t at = r * row_stride + e * head_stride + k;
        const float a = half_bits_to_float(x[at]), b = half_bits_to_float(x[at + pairs]);
        const float c = cs[r * rot + k], s = cs[r * rot + pairs + k];
        o[at] = to_half(__builtin_fmaf(a, c, -(b * s)), hit);
        o[at + pairs] = to_half(__builtin_fmaf(b, c, a * s), hit);
    }
    if (hit) *over = kFaultOverflow;
}

}  // namespace
}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_attention_cache_write_paged(uint16_t* k_cache, uint16_t* v_cache,
                                                               const uint32_t* pages, uint64_t pages_row,
                                                               uint64_t page_size, uint64_t capacity,
                                                               const uint32_t* positions, uint64_t rows_per_seq,
                                                               const uint16_t* k, const uint16_t* v, const float* cs,
                                                               uint64_t rot, uint64_t rows, uint64_t kv_heads,
                                                               uint64_t head_dim, unsigned int* over) {
    silvann::flush_deferred();
    using namespace silvann;
    const uint64_t turn = cs ? rot : 0;
    const bool ok = k_cache && v_cache && positions && k && v && over && rows > 0 && rows < (1ull << 32) &&
                    kv_heads > 0 && kv_heads <= (1u << 20) && head_dim > 0 && head_dim <= (1u << 20) &&
                    rows_per_seq > 0 && capacity > 0 && capacity < (1ull << 32) && turn % 2 == 0 &&
                    turn <= head_dim && (!pages || (page_size > 0 && pages_row >= (capacity + page_size - 1) / page_size));
    if (!ok) {
        refuse("attention_cache_write_paged");
        return;
    }
    CacheArgs a;
    a.kc = k_cache; a.vc = v_cache; a.pages = pages; a.pages_row = pages_row; a.page_size = page_size;
    a.capacity = capacity; a.positions = positions; a.rows_per_seq = rows_per_seq; a.k = k; a.v = v; a.cs = cs;
    a.rot = turn; a.rows = rows; a.kv_heads = kv_heads; a.head_dim = head_dim; a.over = over;
    // 16-byte units when every row, head, turned half and pointer allows them
    const auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const bool vec = head_dim % 8 == 0 && turn % 16 == 0 && al16(k_cache) && al16(v_cache) && al16(k) && al16(v) &&
                     (!cs || al16(cs));
    const uint64_t w = vec ? 8 : 1;
    a.rope_units = turn / 2 / w;
    a.k_units = a.rope_units + (head_dim - turn) / w;
    a.units = a.k_units + head_dim / w;
    const uint64_t total = rows * kv_heads * a.units;
    const uint64_t blocks = std::min<uint64_t>((total + 255) / 256, 8192);
    prof_begin(kProfCacheWrite);
    if (vec) cache_write<8><<<dim3((unsigned)blocks), 256, 0, stream()>>>(a);
    else cache_write<1><<<dim3((unsigned)blocks), 256, 0, stream()>>>(a);
    prof_end(kProfCacheWrite);
    check_launch("attention_cache_write_paged");
}

SILVANN_EXPORT void silvann_gfx950_rope_rows(uint16_t* o, const uint16_t* x, const float* cs, uint64_t rows,
                                             uint64_t heads, uint64_t head_stride, uint64_t row_stride, uint64_t rot,
                                             unsigned int* over) {
    silvann::flush_deferred();
    using namespace silvann;
    if (rows == 0 || heads == 0 || rot < 2) return;   // nothing to turn (the reference's loop runs no item)
    const uint64_t n = rows * heads * (rot / 2);
    const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 8192);
    rope_rows_kernel<<<dim3((unsigned)blocks), 256, 0, stream()>>>(o, x, cs, rows, heads, head_stride, row_stride, rot,
                                                                   over);
    check_launch("rope_rows");
}
