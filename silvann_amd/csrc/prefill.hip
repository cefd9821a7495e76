// prefill.hip — causal attention of a chunk of new positions over a (paged or contiguous) fp16 cache, on
// CDNA4 fp16 MFMA with fp32 accumulation: the fused form of the reference's
// `attention_causal_scores_grouped` → `attention_causal_softmax` → `attention_causal_mix`
// (kernels.cuh:1028-1081, 2051-2060), which materialise every row's weights in `p`; nothing is materialised
// here.
//
// A workgroup is 4 waves over the same rows, each a query head of one kv head's group (or, for a group not a
// multiple of 4, fewer heads over more rows), so a K/V tile in LDS serves four heads. A wave owns 32 query
// rows of one head. Per 32-key tile:
//   S^T = K · Q^T      v_mfma_f32_32x32x16_f16: keys as M, the wave's rows as N, head dims as K; Q^T stays
//                      in registers, K comes from LDS; one accumulator chain
//   online softmax     a lane owns one row (its column of S^T, 16 keys); the row's other 16 keys are in lane
//                      l ^ 32, one exchange away; exponents in base 2 with the scale folded in
//   O^T += V^T · P^T   the same MFMA with keys as K: P^T is the S^T registers narrowed to fp16; V^T is read
//                      from the row-major tile with the transposing LDS read (ds_read_b64_tr_b16), two a
//                      k-step
// K and V tiles move HBM → LDS directly (16 bytes a lane, from a scalar base plus a 32-bit lane offset)
// through a ring of four stages: tile t + 1 is resident and tiles t + 2 and t + 3 are in flight while tile t
// computes, one barrier a tile. Tile t + 1's scores are issued to the matrix cores before tile t's softmax,
// so the exponentials run while the MFMAs do. Rows are XOR-swizzled in 16-byte chunks so both operand reads
// are free of bank conflicts. Causal: keys past a row's position are masked in the diagonal tiles only;
// tiles past the workgroup's last row are never loaded. With a short prefix, a workgroup takes row tiles i
// and N-1-i, so every workgroup has the same work. Positions are 32-bit (first + rows < 2^31); a tile's
// page comes from a cursor that advances a tile a load, so the loop has no 64-bit division.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

#ifndef SILVANN_PREFILL_KA
#define SILVANN_PREFILL_KA 4
#endif
#ifndef SILVANN_PREFILL_VA
#define SILVANN_PREFILL_VA 2
#endif
#ifndef SILVANN_PREFILL_UNIFORM_WAVE
#define SILVANN_PREFILL_UNIFORM_WAVE 0
#endif
#ifndef SILVANN_DUO_KA   // causal_duo's operand read-ahead in MFMAs (-D in experiment builds; deeper spills at head_dim 256)
#define SILVANN_DUO_KA 1
#endif
#ifndef SILVANN_DUO_VA
#define SILVANN_DUO_VA 1
#endif
#ifndef SILVANN_DUO_PIN   // 0: the compiler schedules causal_duo's operand reads (an experiment build's comparison)
#define SILVANN_DUO_PIN 1
#endif
#ifndef SILVANN_PREFILL_XCD_ORDER   // 0: workgroups in launch order (an experiment build's comparison)
#define SILVANN_PREFILL_XCD_ORDER 1
#endif

constexpr int kKT = 32;      // keys a tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

typedef short s16x4 __attribute__((ext_vector_type(4)));

struct CausalArgs {
    uint16_t* o;
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint32_t* pages;
    uint32_t page_size;
    uint32_t q_heads, kv_heads, group;
    uint32_t hw;        // heads a workgroup (4, 2 or 1)
    uint32_t hblocks;   // group / hw
    uint32_t rt;        // rows a workgroup: 32 · (4 / hw)
    uint32_t rtiles;    // ceil(rows / rt)
    uint32_t first, rows;   // first + rows < 2^31: positions and key counts are 32-bit
    float scale_log2;   // 1/sqrt(head_dim) · log2(e)
    unsigned int* over;
    float* res;         // the residual form: row r, head h at res + (r·q_heads + h)·(head_dim + 2)
};

// Tile chunk swizzles (16-byte chunks, CPR of them a row). K: the S^T A-operand read takes one chunk from
// 32 rows; XOR by the row spreads them over the banks. V: the transposing read takes 64 bytes (4 chunks)
// from 8 rows, rows 4 apart in the same bank set; XOR by 4·(row % 4) puts a chunk group's rows apart.
template <int CPR> __device__ __forceinline__ int kslot(int row, int c) { return c ^ (row & (CPR < 16 ? CPR - 1 : 15)); }
template <int CPR> __device__ __forceinline__ int vslot(int row, int c) {
    return c ^ ((row & (CPR >= 16 ? 3 : (CPR / 4 - 1))) << 2);
}

// Page-table entries a workgroup keeps in LDS (16 KB); a longer table is read through the scalar cache.
constexpr uint32_t kPagesInLds = 4096;

template <int HD>
struct Stage {
    _Float16 k[kKT * HD];
    _Float16 v[kKT * HD];
};
constexpr int kStages = 4;
// How far (log2 units) a row's max may pass the max its exponents are taken against before the
// accumulator is rescaled.
constexpr float kRescale = 8.0f;

typedef __attribute__((address_space(3))) void* lds_ptr;

// s_waitcnt's immediate for "vector-memory count <= n" alone (n < 64): the count's low four bits sit in
// bits 3:0 and its high two in bits 15:14; expcnt and lgkmcnt are left at their maxima (no wait).
constexpr int vmcnt_only(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }

// A uniform 32-bit load through the scalar cache (a read; the page table is never written by the kernel).
__device__ __forceinline__ uint32_t scalar_load(const uint32_t* p) {
    uint32_t x;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(x) : "s"(p) : "memory");
    return x;
}

// dma16s with one wait state after the load, so the next write of M0 (the next load's LDS address) is never
// the very next instruction: the spacing the compiler's own schedules keep for this instruction.
__device__ __forceinline__ void dma16s_gap(const void* base, uint32_t off, lds_ptr lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    asm volatile("global_load_lds_dwordx4 %0, %1\n\ts_nop 0" : : "v"(off), "s"(sb), "{m0}"(m0) : "memory");
}

// x *= c for an accumulator element held in an accumulation register, in place.
__device__ __forceinline__ void scale_acc(float& x, float c) {
    float tmp;
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(tmp)
                 : "v"(c));
}

// XCD-aware workgroup order. The hardware deals a launch's workgroups to the 8 XCDs round robin (linear id % 8),
// and each XCD has its own L2. The logical index M = (id % 8)·(N / 8) + id / 8 gives each XCD a contiguous range
// of logical workgroups, which run x-fastest: the row tiles of one head block, so the K/V tiles they all stream
// are fetched into one XCD's L2 instead of every XCD's. A bijection when N is a multiple of 8 (else the identity).
struct Block { uint32_t x, y; };
__device__ __forceinline__ Block xcd_block() {
    const uint32_t n = gridDim.x * gridDim.y, id = blockIdx.x + blockIdx.y * gridDim.x;
    const uint32_t m = SILVANN_PREFILL_XCD_ORDER && n % 8 == 0 ? (id % 8) * (n / 8) + id / 8 : id;
    return {m % gridDim.x, m / gridDim.x};
}

// PTL: the page table fits LDS (kPagesInLds entries) and tiles look their page up there.
// RES: write each row's residual {m, l, acc} (the reference's `attention_weights` + `attention_residual_mix`
// contract, kernels.cuh:1186-1238: m the row's largest scaled score, l = Σ e^(s − m), acc = Σ e^(s − m)·v)
// instead of its fp16 answer.
template <int HD, bool PAIRED, bool PTL, bool RES = false>
__global__ __launch_bounds__(kThreads) void causal_mfma(CausalArgs a) {
    constexpr int CPR = HD / 8;        // 16-byte chunks in a key row
    constexpr int KSTEPS = HD / 16;    // k-steps of S^T (16 dims each)
    constexpr int DT = HD / 32;        // 32-dim tiles of O^T
    constexpr int LOADS = kKT * CPR / kThreads;   // 16-byte direct loads a thread issues a plane a tile
    constexpr uint32_t RB = 2 * HD;    // bytes a key row in a stage
    __shared__ __attribute__((aligned(16))) Stage<HD> ring[kStages];
    __shared__ uint32_t pt[PTL ? kPagesInLds : 1];   // the sequence's page table, off the memory counter

    // SILVANN_PREFILL_UNIFORM_WAVE=1 (an experiment build): the wave index through readfirstlane, so every
    // loop bound and branch derived from it is lowered as wave-uniform, the generic tile loop's too
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = SILVANN_PREFILL_UNIFORM_WAVE ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const Block blk = xcd_block();
    const uint32_t g = blk.y / a.hblocks, hb = blk.y % a.hblocks;
    const uint32_t head = g * a.group + hb * a.hw + (w % a.hw);
    const uint32_t row = a.kv_heads * HD;   // elements a cache position
    bool hit = false;

    // Loop-invariant offsets. Direct loads: thread slot s = tid + 256·i is key row s / CPR, physical chunk
    // s % CPR, which holds logical chunk (s % CPR) ^ swizzle(row) — byte offsets from the tile's key 0 (and
    // from key 0 itself for the last tile's keys past the cache, which are masked).
    uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int s = tid + kThreads * i, r = s / CPR, pc = s % CPR;
        koff[i] = (uint32_t)r * row * 2u + 16u * kslot<CPR>(r, pc);
        voff[i] = (uint32_t)r * row * 2u + 16u * vslot<CPR>(r, pc);
    }
    // S^T A operand: key row col, logical chunk 2·kk + half; the swizzle touches the chunk's low four bits,
    // so k-steps kk and kk + 8 differ by 16 chunks (an immediate). O^T A operand (the transposing read), per
    // dim tile n: lane 4·jj + rr of a 16-lane block points at key 4·half + jj (+ 16·s2 + 8·hh, immediates),
    // dims d0 .. d0+3 with d0 = 32·n + 16·(block & 1) + 4·rr; the swizzle touches bits 2-3 of the chunk, so
    // dim tiles n and n + 4 differ by 16 chunks.
    constexpr int KR = KSTEPS < 8 ? KSTEPS : 8, VR = DT < 4 ? DT : 4;
    uint32_t kread[KR], vread[VR];
    {
        const int blk = lane >> 4, li = lane & 15, jj = li >> 2, rr = li & 3, key = 4 * half + jj;
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) kread[kk] = col * RB + 16u * kslot<CPR>(col, 2 * kk + half);
#pragma unroll
        for (int n = 0; n < VR; ++n) {
            const int d0 = 32 * n + 16 * (blk & 1) + 4 * rr;
            vread[n] = key * RB + 16u * vslot<CPR>(key, d0 >> 3) + 2u * (d0 & 7);
        }
    }

    f32x16 acc[DT];
    f16x8 qb[KSTEPS];

    // S^T (32 keys × 32 rows) of stage `st`: lane holds keys 8·(r/4) + 4·half + r%4 of row col.
    auto scores = [&](int st) __attribute__((always_inline)) -> f32x16 {
        const char* S = (const char*)ring[st].k;
        f32x16 c = (f32x16)0.0f;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk)
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const f16x8*)(S + kread[kk % 8] + 256 * (kk / 8)), qb[kk], c,
                                                        0, 0, 0);
        return c;
    };

    // O^T (32 dims × 32 rows) += V^T · P^T for stage `st`, per dim tile n and k-step s2 (16 keys): the A
    // operand is V^T at dims 32·n + col, keys 16·s2 + 8·(j/4) + 4·half + j%4 — the keys register 8·s2 + j of
    // P^T holds. The transposing read: in each 16-lane block, lane 4·jj + rr points at row (key) jj, dims
    // d0 + 4·rr .. +3, and lane i gets that row's dim d0 + i; two reads (keys +0 and +8) make the 8 halves.
    auto mix = [&](int st, const f16x8* pb) __attribute__((always_inline)) {
        const char* S = (const char*)ring[st].v;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int n = 0; n < DT; ++n) {
                const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(S + vread[n % 4] + 256 * (n / 4) + (16 * s2) * RB));
                const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(S + vread[n % 4] + 256 * (n / 4) + (16 * s2 + 8) * RB));
                const f16x8 va = __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[s2], acc[n], 0, 0, 0);
            }
    };

    auto process = [&](uint32_t rtile) __attribute__((always_inline)) {
        const uint32_t wg_r0 = rtile * a.rt;
        const uint32_t r0 = wg_r0 + (w / a.hw) * 32;   // the wave's first row
        const uint32_t wg_rlast = min(a.rows, wg_r0 + a.rt) - 1;
        const uint32_t nkeys = a.first + wg_rlast + 1;   // keys the workgroup's last row sees
        const uint32_t ntiles = (nkeys + kKT - 1) / kKT;
        const uint32_t myrow = r0 + col;
        const bool row_ok = myrow < a.rows;
        {
            const uint16_t* qr = a.q + ((uint64_t)(row_ok ? myrow : 0) * a.q_heads + head) * HD;
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) qb[kk] = *(const f16x8*)(qr + 16 * kk + 8 * half);
        }
        const uint32_t mypos = a.first + (row_ok ? myrow : 0);
        const uint32_t diag_from = a.first + r0;   // tile t is diagonal for the wave when 32·t + 31 > diag_from
#pragma unroll
        for (int n = 0; n < DT; ++n) acc[n] = (f32x16)0.0f;
        float m = -INFINITY, l = 0.0f;
        float mt = -INFINITY;   // RES: the row's true running max (m lags it by up to kRescale)

        // The load cursor: tiles are loaded in order, so the page and the offset in it advance by a tile
        // each load (page_size is a multiple of the tile).
        uint32_t lt = 0, lj = 0, loff = 0, page = 0;
        auto load_tile = [&]() __attribute__((always_inline)) {
            uint64_t base;   // elements from the plane's start to the tile's key 0, kv head g
            if (!a.pages) {
                base = (uint64_t)lt * kKT * row;
            } else {
                if (loff == 0) {
                    if constexpr (PTL) page = __builtin_amdgcn_readfirstlane(pt[lj]);
                    else page = scalar_load(a.pages + lj);
                }
                base = ((uint64_t)page * a.page_size + loff) * row;
                loff += kKT;
                if (loff == a.page_size) { loff = 0; ++lj; }
            }
            base += (uint64_t)g * HD;
            const bool full = (lt + 1) * kKT <= nkeys;
            char* S = (char*)&ring[lt % kStages];
            ++lt;
            const uint16_t* kb = a.k + base;
            const uint16_t* vb = a.v + base;
            if (full) {
#pragma unroll
                for (int i = 0; i < LOADS; ++i) {
                    const uint32_t at = 16u * (kThreads * i + (tid & ~63));
                    dma16s(kb, koff[i], (lds_ptr)(S + at));
                    dma16s(vb, voff[i], (lds_ptr)(S + sizeof(_Float16) * kKT * HD + at));
                }
            } else {   // the last tile: keys past the cache bring the tile's key 0 (masked)
                const uint32_t left = nkeys - (lt - 1) * kKT;
#pragma unroll
                for (int i = 0; i < LOADS; ++i) {
                    const uint32_t at = 16u * (kThreads * i + (tid & ~63));
                    const uint32_t r = (uint32_t)(tid + kThreads * i) / CPR, back = r < left ? 0u : r * row * 2u;
                    dma16s(kb, koff[i] - back, (lds_ptr)(S + at));
                    dma16s(vb, voff[i] - back, (lds_ptr)(S + sizeof(_Float16) * kKT * HD + at));
                }
            }
        };

        // the ring: tile t in stage t % 4; tile t + 1 resident (its scores are computed during tile t), tiles
        // t + 2 and t + 3 in flight
        __syncthreads();   // the ring and the page table are free (a previous row tile's last reads are done)
        if (PTL && a.pages) {
            const uint32_t npages = (nkeys + a.page_size - 1) / a.page_size;
            for (uint32_t j = tid; j < npages; j += kThreads) pt[j] = a.pages[j];
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the entries are in registers
            __syncthreads();                      // and in LDS for every wave
        }
        load_tile();
        if (ntiles > 1) load_tile();
        if (ntiles > 2) {
            load_tile();
            __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LOADS));   // tiles 0 and 1 landed; tile 2 may fly
        } else {
            __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        __syncthreads();

        f32x16 sc = scores(0), scn;
        float sv[16], mx;
        // First half of tile t: tile t + 3's loads, tile t + 1's scores to the matrix cores, then this tile's
        // masked scores and their row max (log2 units) beside them.
        auto front = [&](uint32_t t) __attribute__((always_inline)) {
            if (t + 3 < ntiles) load_tile();
            if (t + 1 < ntiles) scn = scores((t + 1) % kStages);
            if (t * kKT + kKT - 1 > diag_from) {   // some key of the tile is past some row of the wave
                const int lim = (int)(mypos - t * kKT) - 4 * half;
#pragma unroll
                for (int r = 0; r < 16; ++r) sv[r] = 8 * (r / 4) + (r % 4) > lim ? -INFINITY : sc[r];
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) sv[r] = sc[r];
            }
            float x = sv[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) x = fmaxf(x, sv[r]);
            x = max_xor32(x);
            mx = x * a.scale_log2;   // the scale is positive: max and scale commute
        };
        // Second half: the weights 2^(s·scale − m) as fp16 P^T, their row sum, P·V, and the ring's turn.
        auto back = [&](uint32_t t) __attribute__((always_inline)) {
            float lsum = 0.0f;
            f16x8 pb[2];
            const float nm = -m;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(fmaf(sv[r], a.scale_log2, nm));
                lsum += p;
                pb[r / 8][r % 8] = (_Float16)p;
            }
            l += lsum;
            mix(t % kStages, pb);
            if (t + 1 < ntiles) {
                sc = scn;
                // this wave's part of tile t + 2 landed (the next iteration computes its scores); tile t + 3's
                // 2·LOADS loads, issued after it, may still fly — the vector-memory counter retires in order
                if (t + 3 < ntiles) __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LOADS));
                else __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();   // everyone's part has; everyone is done with stage st
            }
        };

        // Lazy rescale: the exponents stay against the running max m unless some row's new max passes it by
        // more than kRescale (log2 units); then the weights are at most 2^kRescale, exact enough in fp16,
        // and the accumulator keeps its scale. The rescale — the whole accumulator times 2^(m − m') — runs
        // only when some lane needs it (always on the first tile, rarely after), in place on the matrix
        // cores' accumulator registers, so the accumulator keeps one register assignment through the loop.
        auto rescale = [&]() __attribute__((always_inline)) {
            if constexpr (RES) mt = fmaxf(mt, mx);
            if (__builtin_amdgcn_ballot_w64(mx > m + kRescale)) {
                const float mnew = fmaxf(m, mx);
                const float corr = __builtin_amdgcn_exp2f(m - mnew);
                l *= corr;
#pragma unroll
                for (int n = 0; n < DT; ++n)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        float x = acc[n][i];
                        scale_acc(x, corr);
                        acc[n][i] = x;
                    }
                m = mnew;
            }
        };

        // Steady state: tiles wholly below the wave's diagonal whose load three tiles ahead is a full tile.
        // One branch-free block a tile, in the order the matrix cores want it: tile t + 1's scores (16
        // MFMAs) with tile t's exponentials, sums and fp16 packing between them, then tile t's P·V (16
        // MFMAs) with tile t + 1's row max between them; the instruction groups are pinned so each MFMA has
        // vector work to hide behind and its LDS operand was read a few MFMAs earlier.
        // Built for head_dim 256 only (the other widths keep the generic loop). steady_end is wave-uniform
        // by construction (the wave's rows); readfirstlane says so to the compiler, which otherwise lowers
        // this loop and the tail after it as divergent, with the tile cursor in vector registers.
        uint32_t t = 0;
        if constexpr (HD == 256) {
        const uint32_t below = (diag_from + 1) / kKT;   // tiles t with 32·t + 31 <= diag_from
        const uint32_t steady_end = __builtin_amdgcn_readfirstlane(min(ntiles > 4 ? ntiles - 4 : 0u, below));
        if (steady_end > 0) {
            float x = sc[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) x = fmaxf(x, sc[r]);
            x = max_xor32(x);
            mx = x * a.scale_log2;
        }
        for (; t < steady_end; ++t) {
            rescale();
            load_tile();
            const char* SK = (const char*)ring[(t + 1) % kStages].k;
            const char* SV = (const char*)ring[t % kStages].v;
            auto kread_at = [&](int kk) __attribute__((always_inline)) {
                return *(const f16x8*)(SK + kread[kk % 8] + 256 * (kk / 8));
            };
            auto vread_at = [&](int i) __attribute__((always_inline)) {   // MFMA i: k-step i / DT, dim tile i % DT
                const int s2 = i / DT, n = i % DT;
                const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(SV + vread[n % 4] + 256 * (n / 4) + (16 * s2) * RB));
                const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(SV + vread[n % 4] + 256 * (n / 4) + (16 * s2 + 8) * RB));
                return __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
            };
            // operand reads ahead of their MFMA (K operands KA MFMAs ahead, V^T operands VA; experiment builds set
            // them with -D, the defaults are the measured choice)
            constexpr int KA = SILVANN_PREFILL_KA, VA = SILVANN_PREFILL_VA;
            static_assert(VA >= 1 && VA <= KA && KA + 1 <= KSTEPS, "V reads take the last K-read slots");
            f16x8 kb[KA + 1], vb[VA + 2];
            f32x16 c = (f32x16)0.0f;
            float lsum = 0.0f;
            f16x8 pb[2];
            const float nm = -m;
#pragma unroll
            for (int kk = 0; kk < KA && kk < KSTEPS; ++kk) kb[kk] = kread_at(kk);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) {
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb[kk % (KA + 1)], qb[kk], c, 0, 0, 0);
                if (kk + KA < KSTEPS) kb[(kk + KA) % (KA + 1)] = kread_at(kk + KA);
                // the S^T loop's last KA steps read no K: their slots bring the first VA V^T operands
                if (kk + KA >= KSTEPS && kk + KA - KSTEPS < VA) vb[kk + KA - KSTEPS] = vread_at(kk + KA - KSTEPS);
                // the weights of tile t, spread over the MFMAs (one each when KSTEPS is 16)
#pragma unroll
                for (int r = kk * 16 / KSTEPS; r < (kk + 1) * 16 / KSTEPS; ++r) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(sc[r], a.scale_log2, nm));
                    lsum += p;
                    pb[r / 8][r % 8] = (_Float16)p;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            l += lsum;
            float x = 0.0f;
#pragma unroll
            for (int i = 0; i < 2 * DT; ++i) {
                acc[i % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb[i % (VA + 2)], pb[i / DT], acc[i % DT], 0, 0, 0);
                if (i + VA < 2 * DT) vb[(i + VA) % (VA + 2)] = vread_at(i + VA);
                // tile t + 1's row max, once its scores are out of the matrix cores
                if (i == 2) x = fmaxf(c[0], c[1]);
                if (i >= 3 && i < 10) x = fmaxf(x, fmaxf(c[2 * (i - 2)], c[2 * (i - 2) + 1]));
                __builtin_amdgcn_sched_barrier(0);
            }
            if (2 * DT < 11) {
                x = c[0];
#pragma unroll
                for (int r = 1; r < 16; ++r) x = fmaxf(x, c[r]);
            }
            sc = c;
            x = max_xor32(x);
            mx = x * a.scale_log2;
            __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LOADS));   // tile t + 2 landed; tile t + 3 may fly
            __syncthreads();
        }
        }
        for (; t < ntiles; ++t) {
            front(t);
            rescale();
            back(t);
        }

        l = sum_xor32(l);
        if (!row_ok) return;
        if constexpr (RES) {
            // against the true max: every weight 2^(s·scale − mt) <= 1, and m in the scores' own units
            const float corr = __builtin_amdgcn_exp2f(m - mt);
            float* rrow = a.res + ((uint64_t)myrow * a.q_heads + head) * (HD + 2);
            if (half == 0) *(float2*)rrow = make_float2(mt * kLn2, l * corr);
#pragma unroll
            for (int n = 0; n < DT; ++n)
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    float* at = rrow + 2 + 32 * n + 8 * qd + 4 * half;
                    *(float2*)at = make_float2(acc[n][4 * qd] * corr, acc[n][4 * qd + 1] * corr);
                    *(float2*)(at + 2) = make_float2(acc[n][4 * qd + 2] * corr, acc[n][4 * qd + 3] * corr);
                }
            return;
        }
        const float inv_l = 1.0f / l;
        uint16_t* orow = a.o + ((uint64_t)myrow * a.q_heads + head) * HD;
#pragma unroll
        for (int n = 0; n < DT; ++n)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                // register 4·qd + i holds dim 32·n + 8·qd + 4·half + i
                uint16_t hv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) hv[i] = to_half(acc[n][4 * qd + i] * inv_l, hit);
                const uint64_t packed = (uint64_t)hv[0] | ((uint64_t)hv[1] << 16) | ((uint64_t)hv[2] << 32) |
                                        ((uint64_t)hv[3] << 48);
                *(uint64_t*)(orow + 32 * n + 8 * qd + 4 * half) = packed;
            }
    };

    if (PAIRED) {
        // row tiles N-1-x (heavy) then x (light): the same work for every workgroup
        const uint32_t heavy = a.rtiles - 1 - blk.x, light = blk.x;
        process(heavy);
        if (light < heavy) process(light);
    } else {
        process(a.rtiles - 1 - blk.x);   // heaviest first
    }
    if (hit) *a.over = kFaultOverflow;
}

// ── causal_pipe: the head_dim-256 kernel, software-pipelined two tiles deep ────────────────────────────
//
// The same workgroup shape, operand layouts, swizzles and online softmax as causal_mfma, scheduled so that
// no step of a tile waits on the step before it. Iteration t of a wave:
//   matrix cores   S(t + 2) = K(t + 2) · Q^T (16 MFMAs, one accumulator chain) alternating one for one
//                  with O^T += V(t)^T · P(t)^T (16 MFMAs over the 8 accumulator tiles), each operand read
//                  from LDS two MFMAs ahead into rotating registers
//   vector unit    tile t + 1's softmax between them: its row max (the partner half of the row by one
//                  v_permlane32_swap), the lazy max update, and its weights 2^(s·scale − m) narrowed to
//                  fp16 as P(t + 1)
//   memory         K(t + 5) and V(t + 3) straight into LDS, so every tile has two iterations to land
// The max update only decides: a changed max rescales l at once and the accumulator at the top of the next
// iteration, after P(t)·V has gone in at the old scale. K and V have rings of their own, four stages each;
// tile j lives in stage j % 4 of each. While K(t + 5) exists every iteration issues the same loads and one
// vmcnt count serves them all; the last iterations load what exists and wait for everything. Iterations
// whose tile t + 1 is diagonal or that are among the last five take a general path with the mask and the
// bounds.
template <int HD, bool PAIRED, bool PTL>
__global__ __launch_bounds__(kThreads) void causal_pipe(CausalArgs a) {
    constexpr int CPR = HD / 8;
    constexpr int KSTEPS = HD / 16;   // S MFMAs a tile; also the P·V MFMAs a tile (2 k-steps × HD / 32)
    constexpr int DT = HD / 32;
    constexpr int LOADS = kKT * CPR / kThreads;
    constexpr uint32_t RB = 2 * HD;
    constexpr int NS = 4;                              // stages of each ring
    constexpr int GROUP = 2 * LOADS;                   // direct loads a thread issues an iteration
    static_assert(2 * DT == KSTEPS, "one P·V MFMA for each S MFMA");
    __shared__ __attribute__((aligned(16))) _Float16 kring[NS][kKT * HD];
    __shared__ __attribute__((aligned(16))) _Float16 vring[NS][kKT * HD];
    __shared__ uint32_t pt[PTL ? kPagesInLds : 1];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const uint32_t g = blockIdx.y / a.hblocks, hb = blockIdx.y % a.hblocks;
    const uint32_t head = g * a.group + hb * a.hw + (w % a.hw);
    const uint32_t row = a.kv_heads * HD;
    bool hit = false;

    uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int s = tid + kThreads * i, r = s / CPR, pc = s % CPR;
        koff[i] = (uint32_t)r * row * 2u + 16u * kslot<CPR>(r, pc);
        voff[i] = (uint32_t)r * row * 2u + 16u * vslot<CPR>(r, pc);
    }
    constexpr int KR = KSTEPS < 8 ? KSTEPS : 8, VR = DT < 4 ? DT : 4;
    uint32_t kread[KR], vread[VR];
    {
        const int blk = lane >> 4, li = lane & 15, jj = li >> 2, rr = li & 3, key = 4 * half + jj;
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) kread[kk] = col * RB + 16u * kslot<CPR>(col, 2 * kk + half);
#pragma unroll
        for (int n = 0; n < VR; ++n) {
            const int d0 = 32 * n + 16 * (blk & 1) + 4 * rr;
            vread[n] = key * RB + 16u * vslot<CPR>(key, d0 >> 3) + 2u * (d0 & 7);
        }
    }

    f32x16 acc[DT];
    f16x8 qb[KSTEPS];

    // S^T operand k of the tile in K stage `ks`; V^T operand i (k-step i / DT, dim tile i % DT) of V stage `vs`
    auto kop = [&](int ks, int kk) __attribute__((always_inline)) {
        return *(const f16x8*)((const char*)kring[ks] + kread[kk % 8] + 256 * (kk / 8));
    };
    auto vop = [&](int vs, int i) __attribute__((always_inline)) {
        const char* S = (const char*)vring[vs];
        const int s2 = i / DT, n = i % DT;
        const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(S + vread[n % 4] + 256 * (n / 4) + (16 * s2) * RB));
        const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(S + vread[n % 4] + 256 * (n / 4) + (16 * s2 + 8) * RB));
        return __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
    };

    auto process = [&](uint32_t rtile) __attribute__((always_inline)) {
        const uint32_t wg_r0 = rtile * a.rt;
        const uint32_t r0 = wg_r0 + (w / a.hw) * 32;
        const uint32_t wg_rlast = min(a.rows, wg_r0 + a.rt) - 1;
        const uint32_t nkeys = a.first + wg_rlast + 1;
        const uint32_t ntiles = (nkeys + kKT - 1) / kKT;
        const uint32_t myrow = r0 + col;
        const bool row_ok = myrow < a.rows;
        {
            const uint16_t* qr = a.q + ((uint64_t)(row_ok ? myrow : 0) * a.q_heads + head) * HD;
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) qb[kk] = *(const f16x8*)(qr + 16 * kk + 8 * half);
        }
        const uint32_t mypos = a.first + (row_ok ? myrow : 0);
        const uint32_t diag_from = a.first + r0;
#pragma unroll
        for (int n = 0; n < DT; ++n) acc[n] = (f32x16)0.0f;
        float m = -INFINITY, l = 0.0f, corr = 1.0f;
        uint64_t rescale = 0;   // lanes whose max moved: the accumulator waits for its factor `corr`

        __syncthreads();   // both rings and the page table are free
        if (PTL && a.pages) {
            const uint32_t npages = (nkeys + a.page_size - 1) / a.page_size;
            for (uint32_t j = tid; j < npages; j += kThreads) pt[j] = a.pages[j];
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __syncthreads();
        }

        // Load cursors, one a plane: the next tile to load, its page and the offset in it (page_size is a
        // multiple of the tile).
        struct Cursor { uint32_t j, lj, loff, page; };
        auto lookup = [&](uint32_t lj) __attribute__((always_inline)) -> uint32_t {
            if constexpr (PTL) return __builtin_amdgcn_readfirstlane(pt[lj]);
            else return scalar_load(a.pages + lj);
        };
        Cursor ck{0, 0, 0, 0}, cv{0, 0, 0, 0};
        if (a.pages) ck.page = cv.page = lookup(0);
        // Tile c.j of K (ISK) or V into its stage, 16 bytes a lane, LOADS a thread; in the last (partial)
        // tile keys past the cache bring the tile's key 0 (masked). The cursor then moves to the next tile.
        // Only tiles that exist are loaded, so no two loads in flight ever target the same bytes.
        auto issue = [&](auto isk, Cursor& c) __attribute__((always_inline)) {
            constexpr bool ISK = decltype(isk)::value;
            uint64_t base = a.pages ? ((uint64_t)c.page * a.page_size + c.loff) * row : (uint64_t)c.j * kKT * row;
            base += (uint64_t)g * HD;
            const uint16_t* pb = (ISK ? a.k : a.v) + base;
            const uint32_t* off = ISK ? koff : voff;
            char* S = ISK ? (char*)kring[c.j % NS] : (char*)vring[c.j % NS];
            if ((c.j + 1) * kKT <= nkeys) {
#pragma unroll
                for (int i = 0; i < LOADS; ++i) dma16s_gap(pb, off[i], (lds_ptr)(S + 16u * (kThreads * i + (tid & ~63))));
            } else {
                const uint32_t left = nkeys - c.j * kKT;
#pragma unroll
                for (int i = 0; i < LOADS; ++i) {
                    const uint32_t r = (uint32_t)(tid + kThreads * i) / CPR, back = r < left ? 0u : r * row * 2u;
                    dma16s_gap(pb, off[i] - back, (lds_ptr)(S + 16u * (kThreads * i + (tid & ~63))));
                }
            }
            ++c.j;
            if (a.pages && c.j < ntiles) {
                c.loff += kKT;
                if (c.loff == a.page_size) {
                    c.loff = 0;
                    ++c.lj;
                    c.page = lookup(c.lj);
                }
            }
        };
        using KT = std::integral_constant<bool, true>;
        using VT = std::integral_constant<bool, false>;
        auto issue_k = [&]() __attribute__((always_inline)) { if (ck.j < ntiles) issue(KT{}, ck); };
        auto issue_v = [&]() __attribute__((always_inline)) { if (cv.j < ntiles) issue(VT{}, cv); };

        // S^T of the K tile in stage ks, one accumulator chain
        auto scores = [&](int ks) __attribute__((always_inline)) -> f32x16 {
            f32x16 c = (f32x16)0.0f;
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) c = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop(ks, kk), qb[kk], c, 0, 0, 0);
            return c;
        };
        // Softmax of raw scores s (tile j): the lazy max update, the weights as fp16 P^T, l at the new scale.
        // MASK: keys past the row's position are -inf (a diagonal tile).
        auto softmax = [&](f32x16 s, uint32_t j, bool mask, f16x8* pbn) __attribute__((always_inline)) {
            float sv[16];
            if (mask) {
                const int lim = (int)(mypos - j * kKT) - 4 * half;
#pragma unroll
                for (int r = 0; r < 16; ++r) sv[r] = 8 * (r / 4) + (r % 4) > lim ? -INFINITY : s[r];
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) sv[r] = s[r];
            }
            float x = sv[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) x = fmaxf(x, sv[r]);
            const float mx = max_xor32(x) * a.scale_log2;
            const float mnew = mx > m + kRescale ? fmaxf(m, mx) : m;
            const float c = mnew == m ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
            rescale = __builtin_amdgcn_ballot_w64(mnew != m);
            corr = c;
            m = mnew;
            float lsum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(fmaf(sv[r], a.scale_log2, -mnew));
                lsum += p;
                pbn[r / 8][r % 8] = (_Float16)p;
            }
            l = fmaf(l, c, lsum);
        };
        auto apply_rescale = [&]() __attribute__((always_inline)) {
            if (rescale) {
#pragma unroll
                for (int n = 0; n < DT; ++n)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        float x = acc[n][i];
                        scale_acc(x, corr);
                        acc[n][i] = x;
                    }
                rescale = 0;
            }
        };

        // Prologue. K 0..3, V 0 and 1 go out first; once K 0 and K 1 have given S(0) and S(1) (and P(0)),
        // K 4 and V 2 follow — K 4's stage is K 0's. Then iteration t issues K(t + 5) and V(t + 3), each
        // into a stage whose tile every wave has finished with (the barrier closing iteration t - 1).
        const bool full = ntiles >= 6;   // every prologue and steady group exists: exact vmcnt counts
        issue_k(); issue_k(); issue_k(); issue_v();
        issue_k(); issue_v();
        if (full) __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * LOADS));   // K 0..2 and V 0 landed; K 3, V 1 fly
        else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        __syncthreads();
        f32x16 sc0 = scores(0);
        f32x16 sc = ntiles > 1 ? scores(1) : sc0;
        f16x8 pb[2];
        softmax(sc0, 0, kKT - 1 > diag_from, pb);
        __syncthreads();   // K 0 is read by every wave
        issue_k(); issue_v();

        // steady: tile t + 1 wholly below the wave's diagonal and S(t + 2) inside the sequence
        // steady: K(t + 5) exists (so S(t + 2) does) and tile t + 1 lies wholly below the wave's diagonal
        const uint32_t below = (diag_from + 1) / kKT;   // tiles j with 32·j + 31 <= diag_from
        const uint32_t steady_end = __builtin_amdgcn_readfirstlane(
            min(ntiles > 5 ? ntiles - 5 : 0u, below > 1 ? below - 1 : 0u));
        uint32_t t = 0;
        for (; t < steady_end; ++t) {
            apply_rescale();
            issue_k();
            issue_v();
            const int ks = (t + 2) % NS, vs = t % NS;
            f32x16 c = (f32x16)0.0f;
            f16x8 pbn[2];
            f16x8 kb[3], vb[3];
            kb[0] = kop(ks, 0);
            vb[0] = vop(vs, 0);
            kb[1] = kop(ks, 1);
            vb[1] = vop(vs, 1);
            // tile t + 1's softmax, spread over the 16 MFMA pairs: the max over 4 of them, the update at the
            // fifth, the weights over the rest
            float x = 0.0f, mnew = 0.0f, cf = 1.0f, lsum = 0.0f;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < KSTEPS; ++k) {
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb[k % 3], qb[k], c, 0, 0, 0);
                if (k + 2 < KSTEPS) kb[(k + 2) % 3] = kop(ks, k + 2);
                acc[k % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb[k % 3], pb[k / DT], acc[k % DT], 0, 0, 0);
                if (k + 2 < KSTEPS) vb[(k + 2) % 3] = vop(vs, k + 2);
                constexpr int MAXS = KSTEPS / 4 > 0 ? KSTEPS / 4 : 1;   // steps the max takes
                if (k < MAXS) {
#pragma unroll
                    for (int r = k * 16 / MAXS; r < (k + 1) * 16 / MAXS; ++r) x = r == 0 ? sc[0] : fmaxf(x, sc[r]);
                }
                if (k == MAXS) {
                    const float mx = max_xor32(x) * a.scale_log2;
                    mnew = mx > m + kRescale ? fmaxf(m, mx) : m;
                    cf = mnew == m ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
                    rescale = __builtin_amdgcn_ballot_w64(mnew != m);
                }
                if (k > MAXS) {
                    constexpr int SPAN = KSTEPS - 1 - MAXS;   // steps left for the 16 weights
                    const int e = k - MAXS - 1;
#pragma unroll
                    for (int r = e * 16 / SPAN; r < (e + 1) * 16 / SPAN; ++r) {
                        const float p = __builtin_amdgcn_exp2f(fmaf(sc[r], a.scale_log2, -mnew));
                        lsum += p;
                        pbn[r / 8][r % 8] = (_Float16)p;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            corr = cf;
            m = mnew;
            l = fmaf(l, cf, lsum);
            pb[0] = pbn[0];
            pb[1] = pbn[1];
            sc = c;
            __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * GROUP));   // K(t + 3), V(t + 1) landed
            __syncthreads();
        }
        // the last iterations: diagonal tiles masked, no scores past the sequence
        for (; t < ntiles; ++t) {
            apply_rescale();
            issue_k();
            issue_v();
            f32x16 c = sc;
            if (t + 2 < ntiles) c = scores((t + 2) % NS);
            {
                const int vs = t % NS;
#pragma unroll
                for (int i = 0; i < KSTEPS; ++i)
                    acc[i % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop(vs, i), pb[i / DT], acc[i % DT], 0, 0, 0);
            }
            if (t + 1 < ntiles) {
                f16x8 pbn[2];
                softmax(sc, t + 1, (t + 1) * kKT + kKT - 1 > diag_from, pbn);
                pb[0] = pbn[0];
                pb[1] = pbn[1];
            }
            sc = c;
            __builtin_amdgcn_s_waitcnt(vmcnt_only(0));   // groups shrink at the end: wait for all
            __syncthreads();
        }

        l = sum_xor32(l);
        if (!row_ok) return;
        const float inv_l = 1.0f / l;
        uint16_t* orow = a.o + ((uint64_t)myrow * a.q_heads + head) * HD;
#pragma unroll
        for (int n = 0; n < DT; ++n)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                uint16_t hv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) hv[i] = to_half(acc[n][4 * qd + i] * inv_l, hit);
                const uint64_t packed = (uint64_t)hv[0] | ((uint64_t)hv[1] << 16) | ((uint64_t)hv[2] << 32) |
                                        ((uint64_t)hv[3] << 48);
                *(uint64_t*)(orow + 32 * n + 8 * qd + 4 * half) = packed;
            }
    };

    if (PAIRED) {
        const uint32_t heavy = a.rtiles - 1 - blockIdx.x, light = blockIdx.x;
        process(heavy);
        if (light < heavy) process(light);
    } else {
        process(a.rtiles - 1 - blockIdx.x);
    }
    if (hit) *a.over = kFaultOverflow;
}


// ── causal_duo: two waves a SIMD, each taking every other key tile ─────────────────────────────────────
//
// causal_mfma runs one wave a SIMD: a wave's softmax and every wait on its operands leave the matrix cores
// idle, since no other wave on the SIMD has MFMAs to issue. causal_duo gives each (query head, 32 rows) two
// waves, on the same SIMD (waves w and w + 4), which take the even and the odd key tiles: while one waits or
// runs its exponentials the other's MFMAs go to the matrix cores. A workgroup is 8 waves: 4 query heads of
// one kv head's group over the same 32 rows, so a K/V tile in LDS still serves four heads. The ring holds
// two pairs of tiles: pair j (tiles 2j, 2j + 1) is read while pair j + 1 lands, one barrier a pair. Each
// wave keeps its own running max, sum and O^T; at the end the two waves of a head exchange halves of O^T
// through LDS (the ring's bytes, free by then) and each merges and writes half the head dims:
//   m = max(m0, m1),  l = l0·2^(m0 − m) + l1·2^(m1 − m),  O = (O0·2^(m0 − m) + O1·2^(m1 − m)) / l
// — the reference's merge of two residuals (kernels.cuh:1243-1267) in base 2. The register budget is half
// causal_mfma's (256 a lane: O^T's 128 in accumulation registers, Q^T's 64 and the tile's scores, weights
// and operands in the rest), so there is no read-ahead of a next tile's scores.
constexpr int kDuoWaves = 8;
constexpr int kDuoThreads = 64 * kDuoWaves;

// RES: each row's residual {m, l, acc} (row 140) in place of its fp16 answer, as causal_mfma<…, RES>.
template <int HD, bool PAIRED, bool PTL, bool RES = false>
__global__ __launch_bounds__(kDuoThreads) void causal_duo(CausalArgs a) {
    static_assert(HD == 128 || HD == 256, "a tile's loads split evenly over 512 threads");
    constexpr int CPR = HD / 8;
    constexpr int KSTEPS = HD / 16;
    constexpr int DT = HD / 32;
    constexpr int LOADS = kKT * CPR / kDuoThreads;
    constexpr uint32_t RB = 2 * HD;
    __shared__ __attribute__((aligned(16))) Stage<HD> ring[kStages];
    __shared__ uint32_t pt[PTL ? kPagesInLds : 1];
    __shared__ float ml[kDuoWaves][3][64];   // the merge: each wave's running max, sum and (RES) true max
    static_assert(sizeof(ring) == kDuoWaves * (DT / 2) * 16 * 64 * sizeof(float), "the exchange fills the ring");

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = w & 3, par = w >> 2;   // head of the workgroup's four; tile parity
    const int col = lane & 31, half = lane >> 5;
    const Block blk = xcd_block();
    const uint32_t g = blk.y / a.hblocks, hb = blk.y % a.hblocks;
    const uint32_t head = g * a.group + hb * 4 + hi;
    const uint32_t row = a.kv_heads * HD;
    bool hit = false;

    uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int s = tid + kDuoThreads * i, r = s / CPR, pc = s % CPR;
        koff[i] = (uint32_t)r * row * 2u + 16u * kslot<CPR>(r, pc);
        voff[i] = (uint32_t)r * row * 2u + 16u * vslot<CPR>(r, pc);
    }
    // The operand reads' LDS offsets, one register each: the swizzles touch chunk bits the k-step (K: bits 1-3
    // of the chunk) or the dim tile (V: bits 2-3) sets, so k-step kk's offset is kread ^ 32·(kk % 8) (+ 256 for
    // kk >= 8, an immediate) and dim tile n's is vread ^ 64·(n % 4) (+ 256 for n >= 4).
    static_assert(CPR >= 16, "the k-step and dim-tile bits are below the swizzle's reach");
    uint32_t kread, vread;
    {
        const int b16 = lane >> 4, li = lane & 15, jj = li >> 2, rr = li & 3, key = 4 * half + jj;
        kread = col * RB + 16u * kslot<CPR>(col, half);
        const int d0 = 16 * (b16 & 1) + 4 * rr;
        vread = key * RB + 16u * vslot<CPR>(key, d0 >> 3) + 2u * (d0 & 7);
    }

    f32x16 acc[DT];
    f16x8 qb[KSTEPS];

    auto process = [&](uint32_t rtile) __attribute__((always_inline)) {
        const uint32_t r0 = rtile * 32;
        const uint32_t rlast = min(a.rows, r0 + 32) - 1;
        const uint32_t nkeys = a.first + rlast + 1;
        const uint32_t ntiles = (nkeys + kKT - 1) / kKT;
        const uint32_t myrow = r0 + col;
        const bool row_ok = myrow < a.rows;
        {
            const uint16_t* qr = a.q + ((uint64_t)(row_ok ? myrow : 0) * a.q_heads + head) * HD;
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) qb[kk] = *(const f16x8*)(qr + 16 * kk + 8 * half);
        }
        const uint32_t mypos = a.first + (row_ok ? myrow : 0);
        const uint32_t diag_from = a.first + r0;
#pragma unroll
        for (int n = 0; n < DT; ++n) acc[n] = (f32x16)0.0f;
        float m = -INFINITY, l = 0.0f;
        float mt = -INFINITY;   // RES: the row's true running max (m lags it by up to kRescale)

        uint32_t lt = 0, lj = 0, loff = 0, page = 0;
        auto load_tile = [&]() __attribute__((always_inline)) {
            uint64_t base;
            if (!a.pages) {
                base = (uint64_t)lt * kKT * row;
            } else {
                if (loff == 0) {
                    if constexpr (PTL) page = __builtin_amdgcn_readfirstlane(pt[lj]);
                    else page = scalar_load(a.pages + lj);
                }
                base = ((uint64_t)page * a.page_size + loff) * row;
                loff += kKT;
                if (loff == a.page_size) { loff = 0; ++lj; }
            }
            base += (uint64_t)g * HD;
            const bool full = (lt + 1) * kKT <= nkeys;
            char* S = (char*)&ring[lt % kStages];
            const uint32_t left = nkeys - lt * kKT;
            ++lt;
            const uint16_t* kb = a.k + base;
            const uint16_t* vb = a.v + base;
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const uint32_t at = 16u * (kDuoThreads * i + (tid & ~63));
                // the last tile: keys past the cache bring the tile's key 0 (masked)
                const uint32_t r = (uint32_t)(tid + kDuoThreads * i) / CPR, back = full || r < left ? 0u : r * row * 2u;
                dma16s(kb, koff[i] - back, (lds_ptr)(S + at));
                dma16s(vb, voff[i] - back, (lds_ptr)(S + sizeof(_Float16) * kKT * HD + at));
            }
        };

        __syncthreads();   // the ring, the page table and the exchange area are free
        if (PTL && a.pages) {
            const uint32_t npages = (nkeys + a.page_size - 1) / a.page_size;
            for (uint32_t j = tid; j < npages; j += kDuoThreads) pt[j] = a.pages[j];
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __syncthreads();
        }
        load_tile();
        if (ntiles > 1) load_tile();

        for (uint32_t t0 = 0; t0 < ntiles; t0 += 2) {
            __builtin_amdgcn_s_waitcnt(0x0F70);   // this thread's part of pair t0 / 2 landed
            __syncthreads();                      // everyone's has; pair t0 / 2 - 1's stages are free
            if (t0 + 2 < ntiles) load_tile();
            if (t0 + 3 < ntiles) load_tile();
            const uint32_t t = t0 + par;
            if (t >= ntiles) continue;   // the odd wave of a last, lone tile
            const int st = t % kStages;
            // S^T (32 keys × 32 rows): lane holds keys 8·(r/4) + 4·half + r%4 of row col
            // operands read KA (K) and VA (V^T) MFMAs ahead into rotating registers, the groups pinned in order
            constexpr int KA = SILVANN_DUO_KA, VA = SILVANN_DUO_VA;
            f32x16 c = (f32x16)0.0f;
            {
                const char* S = (const char*)ring[st].k;
                auto kread_at = [&](int kk) __attribute__((always_inline)) {
                    return *(const f16x8*)(S + (kread ^ (32u * (kk % 8))) + 256 * (kk / 8));
                };
                f16x8 kb[KA + 1];
#pragma unroll
                for (int kk = 0; kk < KA; ++kk) kb[kk] = kread_at(kk);
#pragma unroll
                for (int kk = 0; kk < KSTEPS; ++kk) {
                    if (kk + KA < KSTEPS) kb[(kk + KA) % (KA + 1)] = kread_at(kk + KA);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb[kk % (KA + 1)], qb[kk], c, 0, 0, 0);
                    if constexpr (SILVANN_DUO_PIN != 0) __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (t * kKT + kKT - 1 > diag_from) {
                const int lim = (int)(mypos - t * kKT) - 4 * half;
#pragma unroll
                for (int r = 0; r < 16; ++r) c[r] = 8 * (r / 4) + (r % 4) > lim ? -INFINITY : c[r];
            }
            float x = c[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) x = fmaxf(x, c[r]);
            const float mx = max_xor32(x) * a.scale_log2;
            if constexpr (RES) mt = fmaxf(mt, mx);
            if (__builtin_amdgcn_ballot_w64(mx > m + kRescale)) {   // the lazy rescale of causal_mfma
                const float mnew = fmaxf(m, mx);
                // a row that has still seen no key (m and mnew -inf) keeps its zeros
                const float corr = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
                l *= corr;
#pragma unroll
                for (int n = 0; n < DT; ++n) acc[n] *= corr;
                m = mnew;
            }
            float lsum = 0.0f;
            f16x8 pb[2];
            // A row may have seen no key yet: the odd wave's first tile can lie wholly past a row's position (the
            // even wave's tile 0 always holds key 0). Its max is still -inf; its weights must be 0, not
            // 2^(-inf + inf), and a rescale that other rows of the wave ask for must leave it at 0 (above).
            const float nm = m == -INFINITY ? 0.0f : -m;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(fmaf(c[r], a.scale_log2, nm));
                lsum += p;
                pb[r / 8][r % 8] = (_Float16)p;
            }
            l += lsum;
            // O^T += V^T · P^T, V^T through the transposing LDS read (as causal_mfma's mix); MFMA i is k-step i / DT,
            // dim tile i % DT
            const char* S = (const char*)ring[st].v;
            auto vread_at = [&](int i) __attribute__((always_inline)) {
                const int s2 = i / DT, n = i % DT;
                const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(S + (vread ^ (64u * (n % 4))) + 256 * (n / 4) + (16 * s2) * RB));
                const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(S + (vread ^ (64u * (n % 4))) + 256 * (n / 4) +
                                                               (16 * s2 + 8) * RB));
                return __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
            };
            f16x8 vb[VA + 1];
#pragma unroll
            for (int i = 0; i < VA; ++i) vb[i] = vread_at(i);
#pragma unroll
            for (int i = 0; i < 2 * DT; ++i) {
                if (i + VA < 2 * DT) vb[(i + VA) % (VA + 1)] = vread_at(i + VA);
                acc[i % DT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb[i % (VA + 1)], pb[i / DT], acc[i % DT], 0, 0, 0);
                if constexpr (SILVANN_DUO_PIN != 0) __builtin_amdgcn_sched_barrier(0);
            }
        }

        // The merge. Wave par keeps dim tiles [par·DT/2, par·DT/2 + DT/2) and hands the other half to its partner
        // (wave w ^ 4) through the ring's bytes: exchange slot (wave, tile, register) holds 64 lanes' floats.
        l = sum_xor32(l);
        __syncthreads();   // every wave is done with the ring
        float* X = (float*)ring;
        const int pw = w ^ 4;
        ml[w][0][lane] = m;
        ml[w][1][lane] = l;
        ml[w][2][lane] = mt;
        // Which half a wave keeps is chosen by value, tile by tile (par is wave-uniform): an index or a branch on
        // par would let the compiler address O^T in memory, putting it in scratch.
#pragma unroll
        for (int n = 0; n < DT / 2; ++n) {
            const f32x16 gv = par ? acc[n] : acc[n + DT / 2];
#pragma unroll
            for (int i = 0; i < 16; ++i) X[((w * (DT / 2) + n) * 16 + i) * 64 + lane] = gv[i];
        }
        __syncthreads();
        const float m1 = ml[pw][0][lane], l1 = ml[pw][1][lane];
        if constexpr (RES) {
            // against the true max of both waves: every weight 2^(s·scale − M) <= 1, m in the scores' own units
            const float M = fmaxf(mt, ml[pw][2][lane]);
            const float c0 = __builtin_amdgcn_exp2f(m - M), c1 = __builtin_amdgcn_exp2f(m1 - M);
            if (!row_ok) return;
            float* rrow = a.res + ((uint64_t)myrow * a.q_heads + head) * (HD + 2);
            if (par == 0 && half == 0) *(float2*)rrow = make_float2(M * kLn2, l * c0 + l1 * c1);
#pragma unroll
            for (int n = 0; n < DT / 2; ++n) {
                const f32x16 kv = par ? acc[n + DT / 2] : acc[n];
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    float v4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        v4[i] = kv[4 * qd + i] * c0 + X[((pw * (DT / 2) + n) * 16 + 4 * qd + i) * 64 + lane] * c1;
                    float* at = rrow + 2 + par * (HD / 2) + 32 * n + 8 * qd + 4 * half;
                    *(float2*)at = make_float2(v4[0], v4[1]);
                    *(float2*)(at + 2) = make_float2(v4[2], v4[3]);
                }
            }
            return;
        }
        const float mm = fmaxf(m, m1);
        const float c0 = __builtin_amdgcn_exp2f(m - mm), c1 = __builtin_amdgcn_exp2f(m1 - mm);
        const float inv_l = 1.0f / (l * c0 + l1 * c1);
        if (!row_ok) return;
        const float a0 = c0 * inv_l, a1 = c1 * inv_l;
        uint16_t* orow = a.o + ((uint64_t)myrow * a.q_heads + head) * HD + par * (HD / 2);
#pragma unroll
        for (int n = 0; n < DT / 2; ++n) {
            const f32x16 kv = par ? acc[n + DT / 2] : acc[n];
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                // register 4·qd + i holds dim 32·n' + 8·qd + 4·half + i of dim tile n'
                uint16_t hv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float o1 = X[((pw * (DT / 2) + n) * 16 + 4 * qd + i) * 64 + lane];
                    hv[i] = to_half(kv[4 * qd + i] * a0 + o1 * a1, hit);
                }
                const uint64_t packed = (uint64_t)hv[0] | ((uint64_t)hv[1] << 16) | ((uint64_t)hv[2] << 32) |
                                        ((uint64_t)hv[3] << 48);
                *(uint64_t*)(orow + 32 * n + 8 * qd + 4 * half) = packed;
            }
        }
    };

    if (PAIRED) {
        const uint32_t heavy = a.rtiles - 1 - blk.x, light = blk.x;
        process(heavy);
        if (light < heavy) process(light);
    } else {
        process(a.rtiles - 1 - blk.x);
    }
    if (hit) *a.over = kFaultOverflow;
}

}  // namespace

// Which head_dim-256 kernel runs: causal_mfma (the default) or causal_pipe, chosen once a process by
// SILVANN_GFX950_PREFILL=pipe. causal_pipe has been checked against the oracle in the CPU emulation of the
// kernels (tests/emu) and has not yet run on a GPU, so it is not the default.
static bool prefill_pipe() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_PREFILL");
        return e && strcmp(e, "pipe") == 0;
    }();
    return on;
}
// causal_duo (two waves a SIMD) for the fp16 answers at head_dim 128 and 256 when the group is a multiple of 4,
// chosen by SILVANN_GFX950_PREFILL=duo; checked in the CPU emulation, not yet timed on a GPU.
static bool prefill_duo() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_PREFILL");
        return e && strcmp(e, "duo") == 0;
    }();
    return on;
}

// The shapes causal_mfma takes (pages NULL or `page_size` positions a page).
bool causal_shape_ok(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows,
                     bool paged, uint64_t page_size) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && kv_heads > 0 && q_heads > 0 &&
           q_heads % kv_heads == 0 &&
           rows > 0 && first + rows < (1ull << 31) &&
           (!paged || (page_size > 0 && page_size < (1ull << 31) && page_size % kKT == 0));
}

// o (with over) for the fp16 answers, or res for the residuals; what = the entry point's name
void causal_paged_launch(uint16_t* o, float* res, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const uint32_t* pages, uint64_t page_size, uint64_t q_heads, uint64_t kv_heads,
                         uint64_t head_dim, uint64_t first, uint64_t rows, unsigned int* over, const char* what) {
    if (!causal_shape_ok(q_heads, kv_heads, head_dim, first, rows, pages != nullptr, page_size)) {
        refuse(what);
        return;
    }
    if (!vec_aligned(q, k, v)) {
        fprintf(stderr, "silvann_gfx950: %s: q, k and v must be 16-byte aligned\n", what);
        refuse(what);
        return;
    }
    CausalArgs a;
    a.o = o; a.res = res; a.q = q; a.k = k; a.v = v; a.pages = pages; a.page_size = (uint32_t)page_size;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hw = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
    a.hblocks = a.group / a.hw;
    a.rt = 32 * (4 / a.hw);
    a.rtiles = (uint32_t)((rows + a.rt - 1) / a.rt);
    a.first = (uint32_t)first; a.rows = (uint32_t)rows;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
    a.over = over;
    // pair row tiles when the causal part dominates the work (a prefix shorter than the chunk)
    const bool paired = first < rows && a.rtiles > 1;
    const dim3 grid(paired ? (a.rtiles + 1) / 2 : a.rtiles, a.kv_heads * a.hblocks);
    const bool duo = prefill_duo() && a.hw == 4 && head_dim >= 128;
    const uint64_t threads = duo ? kDuoThreads : kThreads;
    if ((uint64_t)grid.x * grid.y * threads >= (1ull << 32) || grid.y > 65535) {   // work-items below 2^32
        refuse(what);
        return;
    }
    hipStream_t st = stream();
    prof_begin(kProfCausal);
    const bool ptl = pages && (first + rows + page_size - 1) / page_size <= kPagesInLds;
#define SILVANN_CAUSAL_RES(HDV) \
    if (paired) { \
        if (ptl) causal_mfma<HDV, true, true, true><<<grid, kThreads, 0, st>>>(a); \
        else causal_mfma<HDV, true, false, true><<<grid, kThreads, 0, st>>>(a); \
    } else { \
        if (ptl) causal_mfma<HDV, false, true, true><<<grid, kThreads, 0, st>>>(a); \
        else causal_mfma<HDV, false, false, true><<<grid, kThreads, 0, st>>>(a); \
    }
#define SILVANN_CAUSAL(HDV) \
    if (paired) { \
        if (ptl) causal_mfma<HDV, true, true><<<grid, kThreads, 0, st>>>(a); \
        else causal_mfma<HDV, true, false><<<grid, kThreads, 0, st>>>(a); \
    } else { \
        if (ptl) causal_mfma<HDV, false, true><<<grid, kThreads, 0, st>>>(a); \
        else causal_mfma<HDV, false, false><<<grid, kThreads, 0, st>>>(a); \
    }
    if (duo) {
        const dim3 g2 = grid;
#define SILVANN_CAUSAL_DUO(HDV, R) \
    if (paired) { \
        if (ptl) causal_duo<HDV, true, true, R><<<g2, kDuoThreads, 0, st>>>(a); \
        else causal_duo<HDV, true, false, R><<<g2, kDuoThreads, 0, st>>>(a); \
    } else { \
        if (ptl) causal_duo<HDV, false, true, R><<<g2, kDuoThreads, 0, st>>>(a); \
        else causal_duo<HDV, false, false, R><<<g2, kDuoThreads, 0, st>>>(a); \
    }
        if (res) {
            if (head_dim == 128) { SILVANN_CAUSAL_DUO(128, true) } else { SILVANN_CAUSAL_DUO(256, true) }
        } else {
            if (head_dim == 128) { SILVANN_CAUSAL_DUO(128, false) } else { SILVANN_CAUSAL_DUO(256, false) }
        }
#undef SILVANN_CAUSAL_DUO
    } else if (res) {
        switch (head_dim) {
            case 64: SILVANN_CAUSAL_RES(64) break;
            case 128: SILVANN_CAUSAL_RES(128) break;
            default: SILVANN_CAUSAL_RES(256) break;
        }
    } else switch (head_dim) {
        case 64: SILVANN_CAUSAL(64) break;
        case 128: SILVANN_CAUSAL(128) break;
        default:
            if (prefill_pipe()) {
                if (paired) {
                    if (ptl) causal_pipe<256, true, true><<<grid, kThreads, 0, st>>>(a);
                    else causal_pipe<256, true, false><<<grid, kThreads, 0, st>>>(a);
                } else {
                    if (ptl) causal_pipe<256, false, true><<<grid, kThreads, 0, st>>>(a);
                    else causal_pipe<256, false, false><<<grid, kThreads, 0, st>>>(a);
                }
            } else {
                SILVANN_CAUSAL(256)
            }
            break;
    }
#undef SILVANN_CAUSAL
#undef SILVANN_CAUSAL_RES
    prof_end(kProfCausal);
    check_launch(what);
}

}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_attention_causal_paged(uint16_t* o, const uint16_t* q, const uint16_t* k,
                                                          const uint16_t* v, const uint32_t* pages, uint64_t page_size,
                                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                          uint64_t first, uint64_t rows, unsigned int* over) {
    silvann::flush_deferred();
    silvann::causal_paged_launch(o, nullptr, q, k, v, pages, page_size, q_heads, kv_heads, head_dim, first, rows, over,
                                 "attention_causal_paged");
}

SILVANN_EXPORT void silvann_gfx950_attention_causal_residual_paged(float* res, const uint16_t* q, const uint16_t* k,
                                                                   const uint16_t* v, const uint32_t* pages,
                                                                   uint64_t page_size, uint64_t q_heads,
                                                                   uint64_t kv_heads, uint64_t head_dim, uint64_t first,
                                                                   uint64_t rows) {
    silvann::flush_deferred();
    if (!res) {
        silvann::refuse("attention_causal_residual_paged");
        return;
    }
    silvann::causal_paged_launch(nullptr, res, q, k, v, pages, page_size, q_heads, kv_heads, head_dim, first, rows,
                                 nullptr, "attention_causal_residual_paged");
}
