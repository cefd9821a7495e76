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
//                      in registers, K comes from LDS; four independent accumulator chains
//   online softmax     a lane owns one row (its column of S^T, 16 keys); the row's other 16 keys are in lane
//                      l ^ 32, one exchange away; exponents in base 2 with the scale folded in
//   O^T += V^T · P^T   the same MFMA with keys as K: P^T is the S^T registers narrowed to fp16; V^T is read
//                      from the row-major tile with the transposing LDS read (ds_read_b64_tr_b16), two a
//                      k-step
// K and V tiles move HBM → LDS directly (16 bytes a lane) through a ring of four stages: tile t + 1 is
// resident and tiles t + 2 and t + 3 are in flight while tile t computes, one barrier a tile. Tile t + 1's scores are issued to the matrix
// cores before tile t's softmax, so the exponentials run while the MFMAs do. Rows are XOR-swizzled in 16-byte chunks so both operand reads are
// free of bank conflicts. Causal: keys past a row's position are masked in the diagonal tiles; tiles past
// the workgroup's last row are never loaded. With a short prefix, a workgroup takes row tiles i and N-1-i,
// so every workgroup has the same work.
#include <math.h>
#include <stdio.h>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

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
    uint64_t page_size;
    uint32_t q_heads, kv_heads, group;
    uint32_t hw;        // heads a workgroup (4, 2 or 1)
    uint32_t hblocks;   // group / hw
    uint32_t rt;        // rows a workgroup: 32 · (4 / hw)
    uint32_t rtiles;    // ceil(rows / rt)
    uint64_t first, rows;
    float scale_log2;   // 1/sqrt(head_dim) · log2(e)
    unsigned int* over;
};

// Tile chunk swizzles (16-byte chunks, CPR of them a row). K: the S^T A-operand read takes one chunk from
// 32 rows; XOR by the row spreads them over the banks. V: the transposing read takes 64 bytes (4 chunks)
// from 8 rows, rows 4 apart in the same bank set; XOR by 4·(row % 4) puts a chunk group's rows apart.
template <int CPR> __device__ __forceinline__ int kslot(int row, int c) { return c ^ (row & (CPR < 16 ? CPR - 1 : 15)); }
template <int CPR> __device__ __forceinline__ int vslot(int row, int c) {
    return c ^ ((row & (CPR >= 16 ? 3 : (CPR / 4 - 1))) << 2);
}

// Page-table entries a workgroup keeps in LDS (16 KB); a longer table is read from memory.
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

// PTL: the page table fits LDS (kPagesInLds entries) and tiles look their page up there.
template <int HD, bool PAIRED, bool PTL>
__global__ __launch_bounds__(kThreads) void causal_mfma(CausalArgs a) {
    constexpr int CPR = HD / 8;        // 16-byte chunks in a key row
    constexpr int KSTEPS = HD / 16;    // k-steps of S^T (16 dims each)
    constexpr int DT = HD / 32;        // 32-dim tiles of O^T
    constexpr int LOADS = kKT * CPR / kThreads;   // 16-byte direct loads a thread issues a plane a tile
    __shared__ __attribute__((aligned(16))) Stage<HD> ring[kStages];
    __shared__ uint32_t pt[PTL ? kPagesInLds : 1];   // the sequence's page table, off the memory counter

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const uint32_t g = blockIdx.y / a.hblocks, hb = blockIdx.y % a.hblocks;
    const uint32_t head = g * a.group + hb * a.hw + (w % a.hw);
    const uint64_t row = (uint64_t)a.kv_heads * HD;
    bool hit = false;

    // One 32-key tile of K and V into stage `st`: thread slot s = tid + 256·i is row s / CPR, physical chunk
    // s % CPR, which holds logical chunk (s % CPR) ^ swizzle(row). Keys past `nkeys` bring key 0 of the
    // tile (masked).
    auto tile_row = [&](const uint16_t* plane, uint64_t t0) __attribute__((always_inline)) -> const uint16_t* {
        if (!a.pages) return plane + t0 * row;
        const uint32_t j = (uint32_t)(t0 / a.page_size);
        uint32_t page;
        if constexpr (PTL) page = pt[j];
        else page = a.pages[j];
        return plane + ((uint64_t)page * a.page_size + t0 % a.page_size) * row;
    };
    auto load_tile = [&](int st, uint32_t t, uint64_t nkeys) __attribute__((always_inline)) {
        const uint64_t t0 = (uint64_t)t * kKT;
        const uint16_t* kb = tile_row(a.k, t0) + (uint64_t)g * HD;
        const uint16_t* vb = tile_row(a.v, t0) + (uint64_t)g * HD;
        Stage<HD>& S = ring[st];
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int s = tid + kThreads * i, r = s / CPR, pc = s % CPR;
            const uint64_t rr = t0 + r < nkeys ? (uint64_t)r : 0;
            dma16(kb + rr * row + 8 * kslot<CPR>(r, pc),
                  (__attribute__((address_space(3))) void*)(&S.k[8 * kThreads * i + 8 * (tid & ~63)]));
            dma16(vb + rr * row + 8 * vslot<CPR>(r, pc),
                  (__attribute__((address_space(3))) void*)(&S.v[8 * kThreads * i + 8 * (tid & ~63)]));
        }
    };

    f32x16 acc[DT];
    f16x8 qb[KSTEPS];

    // S^T (32 keys × 32 rows) of stage `st`: lane holds keys 8·(r/4) + 4·half + r%4 of row col; two chains.
    auto scores = [&](int st) __attribute__((always_inline)) -> f32x16 {
        const Stage<HD>& S = ring[st];
        f32x16 c0 = (f32x16)0.0f, c1 = (f32x16)0.0f;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; kk += 2) {
            const f16x8 k0 = *(const f16x8*)(&S.k[col * HD + 8 * kslot<CPR>(col, 2 * kk + half)]);
            const f16x8 k1 = *(const f16x8*)(&S.k[col * HD + 8 * kslot<CPR>(col, 2 * kk + 2 + half)]);
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, qb[kk], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(k1, qb[kk + 1], c1, 0, 0, 0);
        }
        return c0 + c1;
    };

    // O^T (32 dims × 32 rows) += V^T · P^T for stage `st`, per dim tile n and k-step s2 (16 keys): the A
    // operand is V^T at dims 32·n + col, keys 16·s2 + 8·(j/4) + 4·half + j%4 — the keys register 8·s2 + j of
    // P^T holds. The transposing read: in each 16-lane block, lane 4·jj + rr points at row (key) jj, dims
    // d0 + 4·rr .. +3, and lane i gets that row's dim d0 + i; two reads (keys +0 and +8) make the 8 halves.
    auto mix = [&](int st, const f16x8* pb) __attribute__((always_inline)) {
        const Stage<HD>& S = ring[st];
        const int blk = lane >> 4, li = lane & 15, jj = li >> 2, rr = li & 3;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int n = 0; n < DT; ++n) {
                const int d0 = 32 * n + 16 * (blk & 1) + 4 * rr;
                f16x8 va;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int key = 16 * s2 + 8 * hh + 4 * half + jj;
                    const _Float16* src = &S.v[key * HD + 8 * vslot<CPR>(key, d0 >> 3) + (d0 & 7)];
                    const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4*)(src));
                    const f16x4 xh = __builtin_bit_cast(f16x4, x);
                    va[4 * hh + 0] = xh[0];
                    va[4 * hh + 1] = xh[1];
                    va[4 * hh + 2] = xh[2];
                    va[4 * hh + 3] = xh[3];
                }
                acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[s2], acc[n], 0, 0, 0);
            }
    };

    auto process = [&](uint32_t rtile) __attribute__((always_inline)) {
        const uint64_t r0 = (uint64_t)rtile * a.rt + (uint64_t)(w / a.hw) * 32;   // the wave's first row
        const uint64_t wg_r0 = (uint64_t)rtile * a.rt;
        const uint64_t wg_rlast = min(a.rows, wg_r0 + a.rt) - 1;
        const uint64_t nkeys = a.first + wg_rlast + 1;             // keys the workgroup's last row sees
        const uint32_t ntiles = (uint32_t)((nkeys + kKT - 1) / kKT);
        const uint64_t myrow = r0 + col;
        const bool row_ok = myrow < a.rows;
        {
            const uint16_t* qr = a.q + ((row_ok ? myrow : 0) * a.q_heads + head) * HD;
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) qb[kk] = *(const f16x8*)(qr + 16 * kk + 8 * half);
        }
        const uint64_t mypos = a.first + (row_ok ? myrow : 0);
#pragma unroll
        for (int n = 0; n < DT; ++n) acc[n] = (f32x16)0.0f;
        float m = -INFINITY, l = 0.0f;

        // the ring: tile t in stage t % 4; tile t + 1 resident (its scores are computed during tile t), tiles
        // t + 2 and t + 3 in flight
        __syncthreads();   // the ring and the page table are free (a previous row tile's last reads are done)
        if (PTL && a.pages) {
            const uint32_t npages = (uint32_t)((nkeys + a.page_size - 1) / a.page_size);
            for (uint32_t j = tid; j < npages; j += kThreads) pt[j] = a.pages[j];
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the entries are in registers
            __syncthreads();                      // and in LDS for every wave
        }
        load_tile(0, 0, nkeys);
        if (ntiles > 1) load_tile(1, 1, nkeys);
        if (ntiles > 2) {
            load_tile(2, 2, nkeys);
            __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LOADS));   // tiles 0 and 1 landed; tile 2 may fly
        } else {
            __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        __syncthreads();
        f32x16 sc = scores(0);
        for (uint32_t t = 0; t < ntiles; ++t) {
            const int st = t % kStages, st1 = (t + 1) % kStages, st3 = (t + 3) % kStages;
            // tile t + 3 into the stage tile t - 1 used (every wave left it at the last barrier)
            const bool ahead = t + 3 < ntiles;
            if (ahead) load_tile(st3, t + 3, nkeys);
            // the next tile's scores go to the matrix cores first; this tile's softmax runs beside them
            f32x16 scn;
            if (t + 1 < ntiles) scn = scores(st1);
            const uint64_t t0 = (uint64_t)t * kKT;
            float sv[16];
            float mx = -INFINITY;
            const bool diag = t0 + kKT - 1 > a.first + r0;   // some key of the tile is past some row of the wave
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t key = t0 + 8 * (r / 4) + 4 * half + (r % 4);
                float x = sc[r] * a.scale_log2;
                if (diag && key > mypos) x = -INFINITY;
                sv[r] = x;
                mx = fmaxf(mx, x);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            // Lazy rescale: the exponents stay against the running max m unless some row's new max passes
            // it by more than kRescale (log2 units); then the weights are at most 2^kRescale, exact enough
            // in fp16, and the accumulator keeps its scale. The rescale — the whole accumulator times
            // e^(m - m') — runs only when some lane needs it (always on the first tile, rarely after).
            if (__builtin_amdgcn_ballot_w64(mx > m + kRescale)) {
                const float mnew = fmaxf(m, mx);
                const float corr = __builtin_amdgcn_exp2f(m - mnew);
                l *= corr;
#pragma unroll
                for (int n = 0; n < DT; ++n) acc[n] *= corr;
                m = mnew;
            }
            float lsum = 0.0f;
            f16x8 pb[2];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = __builtin_amdgcn_exp2f(sv[r] - m);
                lsum += p;
                pb[r / 8][r % 8] = (_Float16)p;
            }
            l += lsum;
            mix(st, pb);
            if (t + 1 < ntiles) {
                sc = scn;
                // this wave's part of tile t + 2 landed (the next iteration computes its scores); tile t + 3's
                // 2·LOADS loads, issued after it, may still fly — the vector-memory counter retires in order
                if (ahead) __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LOADS));
                else __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();   // everyone's part has; everyone is done with stage st
            }
        }

        l += __shfl_xor(l, 32);
        if (!row_ok) return;
        const float inv_l = 1.0f / l;
        uint16_t* orow = a.o + (myrow * a.q_heads + head) * HD;
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
        const uint32_t heavy = a.rtiles - 1 - blockIdx.x, light = blockIdx.x;
        process(heavy);
        if (light < heavy) process(light);
    } else {
        process(a.rtiles - 1 - blockIdx.x);   // heaviest first
    }
    if (hit) *a.over = kFaultOverflow;
}

}  // namespace

void causal_paged_launch(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* pages,
                         uint64_t page_size, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t first,
                         uint64_t rows, unsigned int* over) {
    const bool ok = (head_dim == 64 || head_dim == 128 || head_dim == 256) && kv_heads > 0 && q_heads % kv_heads == 0 &&
                    rows > 0 && first + rows < (1ull << 40) && (!pages || (page_size > 0 && page_size % kKT == 0));
    if (!ok) {
        refuse("attention_causal_paged");
        return;
    }
    CausalArgs a;
    a.o = o; a.q = q; a.k = k; a.v = v; a.pages = pages; a.page_size = page_size;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hw = a.group % 4 == 0 ? 4 : (a.group % 2 == 0 ? 2 : 1);
    a.hblocks = a.group / a.hw;
    a.rt = 32 * (4 / a.hw);
    a.rtiles = (uint32_t)((rows + a.rt - 1) / a.rt);
    a.first = first; a.rows = rows;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
    a.over = over;
    // pair row tiles when the causal part dominates the work (a prefix shorter than the chunk)
    const bool paired = first < rows && a.rtiles > 1;
    const dim3 grid(paired ? (a.rtiles + 1) / 2 : a.rtiles, a.kv_heads * a.hblocks);
    hipStream_t st = stream();
    prof_begin(kProfCausal);
    const bool ptl = pages && (first + rows + page_size - 1) / page_size <= kPagesInLds;
#define SILVANN_CAUSAL(HDV) \
    if (paired) { \
        if (ptl) causal_mfma<HDV, true, true><<<grid, kThreads, 0, st>>>(a); \
        else causal_mfma<HDV, true, false><<<grid, kThreads, 0, st>>>(a); \
    } else { \
        if (ptl) causal_mfma<HDV, false, true><<<grid, kThreads, 0, st>>>(a); \
        else causal_mfma<HDV, false, false><<<grid, kThreads, 0, st>>>(a); \
    }
    switch (head_dim) {
        case 64: SILVANN_CAUSAL(64) break;
        case 128: SILVANN_CAUSAL(128) break;
        default: SILVANN_CAUSAL(256) break;
    }
#undef SILVANN_CAUSAL
    prof_end(kProfCausal);
    check_launch("attention_causal_paged");
}

}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_attention_causal_paged(uint16_t* o, const uint16_t* q, const uint16_t* k,
                                                          const uint16_t* v, const uint32_t* pages, uint64_t page_size,
                                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                          uint64_t first, uint64_t rows, unsigned int* over) {
    silvann::causal_paged_launch(o, q, k, v, pages, page_size, q_heads, kv_heads, head_dim, first, rows, over);
}
