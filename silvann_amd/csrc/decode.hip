// decode.hip — split-K flash decoding for grouped-query attention over a paged (or contiguous) fp16 cache.
//
// The reference's decode is two doors: `attention_scores` writes every query head's softmax weights into
// `p`, `attention_mix` reads them back (kernels.cuh:885-915, 1133-1164). Here one pass reads each key and
// value once for all the query heads that share their kv head, and the reference's own residual contract
// (kernels.cuh:1180-1267: per head [m, l, acc], merged exactly by e^(m_a - m), e^(m_b - m)) joins the splits:
//
//   plan    decode_plan: each row's split count, prefix-summed, and the work counter zeroed — in the
//           scratch's header
//   pass 1  decode_split: one workgroup of 4 waves a work item — (split of `chunk` positions of a row, kv
//           head, head block of up to 16 query heads) — flattened over the rows by the plan's prefix sums,
//           so a short row costs only its own splits and no workgroup idles (one workgroup an item measured
//           faster than a persistent grid taking items from a counter: C2 5.17 vs 4.87 TB/s, C5 6.2 vs
//           5.1). Each wave walks
//           32 KB tiles of K and V (32 keys at head_dim 256, 64 at 128, 128 at 64) of the split:
//             S^T = K · Q^T     v_mfma_f32_16x16x32_f16, keys as M, the group's query heads as N (a group of
//                               8 fills half the columns; the other half is zero — the decode is HBM-bound,
//                               and the MFMA has 50x the throughput it needs)
//             online softmax    in registers: a lane owns one query head's column; its tile max is folded
//                               over the column's four 16-lane groups
//             O^T += V^T · P^T  the same MFMA, keys as K: P comes straight from the S^T registers, V^T from
//                               the tile staged in LDS and read transposed
//           then the four waves' (m, l, O) merge in LDS and the split's residual goes to `part`.
//   pass 2  decode_merge: a workgroup per (row, query head, 64 dims) merges that head's split residuals and writes
//           acc / l as fp16, flagging overflow (kernels.cuh:1258-1267).
//
// K loads are 16 bytes a lane (8 halves of one key row: the MFMA A operand's own layout) into registers; V
// goes straight from HBM into LDS (16 bytes a lane, consecutive lanes on consecutive bytes of a row), so it
// takes no registers and two workgroups fit on a CU at head_dim 256.
//
// Other forms of the same kernels:
//   head_dim 512     32-key tiles, one wave a SIMD; SHARED when k == v (latent attention: each tile comes into LDS
//                    once and both operands are read from there), its workgroups in an XCD-aware order
//   fused finish     (SILVANN_GFX950_DECODE_FUSED=1) the last split of a row and head block merges the others
//   decode_one       one query of a deferred door pair (scores → mix, weights → residual_mix, the grouped chains
//                    with a softmax or a sink), its scratch the pair's weights buffer; decode_merge_res writes the
//                    residual, decode_merge<…, SINK> folds the sink in
//   decode_causal    a deferred causal chain at head_dim 512: each row a decode over the same cache
#include <math.h>
#include <atomic>
#include <random>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kMaxSplits = 65536;  // splits a row: the split grid's x extent stays small

struct DecodeArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint32_t* pages;
    uint64_t pages_row;
    uint64_t page_size;
    uint64_t k_row;
    const uint32_t* lens;
    uint32_t q_heads, kv_heads, group, hblocks;
    uint32_t chunk, nsplit;
    float scale;
    float* part;
    const uint32_t* plan;   // decode_plan's: full splits of rows before u, all splits, the short splits' rows
    uint32_t* counter;      // the next work item
    uint32_t rows;
    // the fused finish: a count of finished splits a (row, kv head, head block), the answers, the fault word
    uint32_t* done;
    uint32_t* gdone = nullptr;   // rows of more than kFinishGroup splits: a count a group of them, maxng a unit
    uint32_t maxng = 0;
    uint16_t* o;
    unsigned int* over;
    // the inline plan with lens null: row u's length is len_first + u·len_step, and workgroup 0 writes the lengths
    // to lens_out for the merge
    uint32_t len_first, len_step;
    uint32_t* lens_out;
    uint64_t tag;   // the fused finish with the inline plan: this call's tag for the counts (below kTagMask)
};

// The scratch: the work counter, the plan (2·rows + 2 words, below), the finished-split counts (rows · kv heads · head blocks, 8 bytes each:
// 32-bit counts, or the inline plan's tagged 64-bit words), then the partial residuals
// [row][q head][split][head_dim + 2].
constexpr uint64_t kPlanAt = 64;
uint64_t done_at(uint64_t rows) { return (kPlanAt + 4 * (2 * rows + 2) + 7) / 8 * 8; }
// The fused finish's groups: a row of more than kFinishGroup splits finishes in two levels (decode_split).
constexpr uint32_t kFinishGroup = 32;
uint64_t groups_at(uint64_t rows, uint64_t units) { return done_at(rows) + 8 * rows * units; }
// `maxng` count words a (row, kv head, head block) after the finished-split counts: the groups' (row 137's scratch)
uint64_t part_at(uint64_t rows, uint64_t units, uint64_t maxng = 0) {
    return (groups_at(rows, units) + 8 * rows * units * maxng + 255) / 256 * 256;
}
// A tagged finished-split count: the call's tag in the top 40 bits, the count below. A word holding another tag
// (an earlier call's, or whatever the scratch held) counts as zero, so no launch has to clear the counts first.
constexpr int kTagShift = 24;
constexpr uint64_t kTagMask = (1ull << (64 - kTagShift)) - 1;
// A launch's work-items (workgroups × 256) must stay below 2^32: the most workgroups a split grid may have.
constexpr uint64_t kMaxGroups = (1ull << 32) / kThreads - 8;

// The grid of the shared-tile form: its XCD-aware order covers the splits in groups of 8.
uint32_t shared_grid(uint64_t splits, uint64_t units) { return (uint32_t)((splits + 7) / 8 * 8 * units); }

// The plan: each row's full splits (len / chunk) prefix-summed into plan[0..rows] (plan[rows] = F, every row's full
// splits), the count of all splits at plan[rows + 1], and after it, plan[rows + 2 ..], the rows whose last split is
// shorter than a chunk, longest remainder first (by 64 buckets of chunk / 64). decode_split takes its items in that
// order — every full split, then the short ones from the longest — so the last round of work items, the one the
// chip is not full for, is made of the shortest ones. One workgroup; the counter zeroed. FUSED: also the
// finished-split counts zeroed, and the answers of rows with no positions written as zeros (no split of theirs
// will finish them).
constexpr uint32_t kRemBuckets = 64;
__device__ __forceinline__ uint32_t rem_bucket(uint32_t rem, uint32_t chunk) {
    return kRemBuckets - 1 - (uint32_t)((uint64_t)rem * kRemBuckets / chunk);   // bucket 0: the longest remainders
}
template <bool FUSED = false>
__global__ __launch_bounds__(256) void decode_plan(const uint32_t* lens, uint32_t rows, uint32_t chunk, uint32_t* plan,
                                                   uint32_t* counter, uint32_t* done = nullptr, uint32_t units = 0,
                                                   uint16_t* o = nullptr, uint32_t row_halves = 0,
                                                   uint32_t* gdone = nullptr, uint32_t maxng = 0) {
    if constexpr (FUSED) {
        for (uint32_t i = threadIdx.x; i < rows * units; i += 256) done[i] = 0;
        for (uint32_t i = threadIdx.x; i < rows * units * maxng; i += 256) gdone[i] = 0;
        for (uint32_t u = 0; u < rows; ++u)
            if (lens[u] == 0)
                for (uint32_t i = threadIdx.x; i < row_halves; i += 256) o[(uint64_t)u * row_halves + i] = 0;
    }
    __shared__ uint32_t scan[256];
    __shared__ uint32_t carry;
    __shared__ uint32_t bucket[kRemBuckets];
    if (threadIdx.x == 0) {
        counter[0] = 0;
        carry = 0;
    }
    if (threadIdx.x < kRemBuckets) bucket[threadIdx.x] = 0;
    __syncthreads();
    for (uint32_t base = 0; base < rows; base += 256) {
        const uint32_t u = base + threadIdx.x;
        const uint32_t len = u < rows ? lens[u] : 0;
        const uint32_t n = len / chunk, rem = len % chunk;
        if (rem) atomicAdd(&bucket[rem_bucket(rem, chunk)], 1u);
        scan[threadIdx.x] = n;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {   // inclusive scan
            const uint32_t add = threadIdx.x >= (unsigned)off ? scan[threadIdx.x - off] : 0;
            __syncthreads();
            scan[threadIdx.x] += add;
            __syncthreads();
        }
        if (u < rows) plan[u] = carry + scan[threadIdx.x] - n;
        __syncthreads();
        if (threadIdx.x == 255) carry += scan[255];
        __syncthreads();
    }
    if (threadIdx.x == 0) {   // the buckets' starts, longest first
        uint32_t at = 0;
        for (uint32_t b = 0; b < kRemBuckets; ++b) {
            const uint32_t c = bucket[b];
            bucket[b] = at;
            at += c;
        }
        plan[rows] = carry;
        plan[rows + 1] = carry + at;
    }
    __syncthreads();
    for (uint32_t u = threadIdx.x; u < rows; u += 256) {
        const uint32_t rem = lens[u] % chunk;
        if (rem) plan[rows + 2 + atomicAdd(&bucket[rem_bucket(rem, chunk)], 1u)] = u;
    }
}

// Where the 16 keys from position `t` of row `u`, kv head `g` start in a plane: through the page table (a
// page holds a multiple of 16 positions, so 16 keys from a multiple of 16 never straddle two), or contiguous.
__device__ __forceinline__ const uint16_t* group_base(const uint16_t* plane, const DecodeArgs& a, uint32_t u,
                                                      uint32_t g, uint32_t t, uint64_t row, int hd) {
    if (a.pages) {
        const uint32_t ps = (uint32_t)a.page_size;
        const uint64_t phys = (uint64_t)a.pages[(uint64_t)u * a.pages_row + t / ps] * ps + t % ps;
        return plane + phys * row + (uint64_t)g * hd;
    }
    return plane + (uint64_t)u * a.k_row + (uint64_t)t * row + (uint64_t)g * hd;
}

// A value tile in LDS: 32 rows of HD halves, no padding (the direct-to-LDS load writes 16 bytes a lane,
// consecutively). Row `key`'s 16-byte chunk `c` sits at chunk slot c ^ f(key), f(key) = 2·((key / 4) % 4):
// the transposed read takes one dim from keys 4·grp + j of the four lane groups, and the swizzle puts the
// four groups' chunks in different banks.
__device__ __forceinline__ int vslot(int key, int chunk) { return chunk ^ (((key >> 2) & 3) << 1); }

// Keys a wave takes a step: 32 KB of K and V (16 KB each) up to head_dim 256; at 512, 32 keys (64 KB), the least a
// P·V k-step takes.
constexpr int tile_keys(int hd) { return 8192 / hd < 32 ? 32 : 8192 / hd; }
// Cache policy of the streamed K/V loads: non-temporal (read once, kept out of the caches' way).
constexpr int kCacheStream = 2;
// Which of decode_split's cache-policy variants runs (SILVANN_GFX950_DECODE_VARIANT overrides).
constexpr int kDefaultVariant = 2;

// VARIANT bit 0: non-temporal K loads; bit 1: non-temporal value loads into LDS. GROUPED: pages shorter than
// a tile, so each 16-key group of a tile is looked up on its own; otherwise one lookup a tile.
// One workgroup an item: workgroup x is item x; past the last item it returns at once.
// SHARED: the keys are the values (k == v: multi-head latent attention, where one cache of latents is both,
// engine/src/packages/ai_z__glm_5_3/cpu/opcodes/layer__abi.cuh:283-289): each tile comes into LDS once and the
// S^T A operand is read from there. Two waves a SIMD up to head_dim 256; one at 512 (its accumulator alone is
// 128 registers a lane).
// FUSED: the split that finishes last for its (row, kv head, head block) — it counts the finished splits — merges
// them and writes the answers, as decode_merge does; no second launch.
// VTR: the V^T operand read with the transposing LDS read (two a MFMA) rather than element by element (eight) —
// at head_dim 512, where the P·V MFMAs are the most a tile has.
template <int HD, int VARIANT, bool GROUPED, bool SHARED = false, bool FUSED = false, bool VTR = (HD >= 512),
          bool INLINE = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(HD >= 512 ? 1 : 2, HD >= 512 ? 1 : 2)))
void decode_split(DecodeArgs a) {
    static_assert(!(FUSED && INLINE) || kMaxSplits < (1u << kTagShift), "a tagged count holds every split");
    constexpr int TK = tile_keys(HD);  // keys a wave takes a step: 32 KB of K and V whatever the head width
    constexpr int MT = TK / 16;      // 16-key M tiles of S^T
    constexpr int KS = HD / 32;      // k-steps of the S^T MFMA (32 dims each)
    constexpr int NT = HD / 16;      // d-tiles of the O^T accumulator
    constexpr int VCH = TK * HD / 512;  // 16-byte value chunks a lane brings in a tile
    constexpr int CPR = HD / 8;      // 16-byte chunks in one value row
    constexpr int kStageBytes = kWaves * TK * HD * 2;
    constexpr int kMergeBytes = kWaves * 16 * HD * 4 + 2 * kWaves * 16 * 4;
    constexpr int kSmem = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSmem];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const uint64_t row = (uint64_t)a.kv_heads * HD;
    const uint32_t GH = a.kv_heads * a.hblocks;
    // INLINE (at most 64 rows): every wave makes the plan itself — lane u holds row u's length and the splits of the
    // rows before it (a butterfly scan), and an item's row is the last lane whose splits-before are at most its
    // split index — so no plan launch goes first.
    uint32_t lane_len = 0, lane_before = 0, inline_total = 0;
    if constexpr (INLINE) {
        if (a.lens) {
            lane_len = lane < (int)a.rows ? a.lens[lane] : 0u;
        } else {
            lane_len = lane < (int)a.rows ? a.len_first + (uint32_t)lane * a.len_step : 0u;
            if (blockIdx.x == 0 && w == 0 && lane < (int)a.rows) a.lens_out[lane] = lane_len;
        }
        const uint32_t n = (lane_len + a.chunk - 1) / a.chunk;
        uint32_t incl = n, sum = n;
#pragma unroll
        for (int b = 1; b < 64; b <<= 1) {
            const uint32_t t = __shfl_xor(sum, b);
            if (lane & b) incl += t;
            sum += t;
        }
        lane_before = incl - n;
        inline_total = __builtin_amdgcn_readfirstlane(sum) * GH;
        if constexpr (FUSED) {
            // rows with no positions have no split to finish them: workgroup 0 writes their zero answers
            if (blockIdx.x == 0) {
                uint64_t empty = __builtin_amdgcn_ballot_w64(lane < (int)a.rows && lane_len == 0);
                const uint32_t halves = a.q_heads * HD;
                while (empty) {
                    const uint32_t e = (uint32_t)__builtin_ctzll(empty);
                    empty &= empty - 1;
                    for (uint32_t i = threadIdx.x; i < halves; i += kThreads) a.o[(uint64_t)e * halves + i] = 0;
                }
            }
        }
    }
    const uint32_t total = INLINE ? inline_total : a.plan[a.rows + 1] * GH;
    __shared__ uint32_t is_last;
    // the workgroup's item: its own index
    uint32_t item = blockIdx.x;
    if constexpr (SHARED) {
        // XCD-aware order: workgroups go to the 8 XCDs round robin (workgroup b to XCD b % 8), and the head blocks of
        // one split read the same latents, so they take blocks 8·j + x for one x — one XCD and its L2 — and
        // consecutive j. A block past the last split gets an item past the last and returns.
        const uint32_t x = blockIdx.x & 7u, j = blockIdx.x >> 3;
        item = ((j / GH) * 8u + x) * GH + j % GH;
    }
    if (item >= total) return;
    const uint32_t sidx = item / GH, gh = item % GH;
    uint32_t lo = 0, hi = a.rows, s;
    if constexpr (INLINE) {
        // lane 0 (no splits before it) always counts, so lo is a row
        lo = (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < (int)a.rows && lane_before <= sidx)) - 1u;
        s = sidx - (uint32_t)__builtin_amdgcn_readlane((int)lane_before, (int)lo);
    } else {
        const uint32_t full = a.plan[a.rows];
        if (sidx < full) {   // a full split: the row whose full splits hold index sidx
            while (hi - lo > 1) {
                const uint32_t mid = (lo + hi) >> 1;
                if (a.plan[mid] <= sidx) lo = mid;
                else hi = mid;
            }
            s = sidx - a.plan[lo];
        } else {             // a row's shorter last split, after every full one
            lo = a.plan[a.rows + 2 + (sidx - full)];
            s = a.plan[lo + 1] - a.plan[lo];
        }
    }
    const uint32_t u = lo;
    const uint32_t g = gh / a.hblocks, hb = gh % a.hblocks;
    const uint32_t len = INLINE ? (uint32_t)__builtin_amdgcn_readlane((int)lane_len, (int)u) : a.lens[u];
    const uint32_t start = s * a.chunk;
    const uint32_t end = min(len, start + a.chunk);
    const uint32_t h0 = g * a.group + hb * 16;
    const int nh = min(16, (int)(a.group - hb * 16));

    // Q^T as the B operand: lane (col, grp) holds head col's dims 32·ks + 8·grp .. +8; heads past the block are 0.
    f16x8 qb[KS];
    {
        const uint16_t* qh = a.q + ((uint64_t)u * a.q_heads + h0 + (col < nh ? col : 0)) * HD;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            f16x8 x = *(const f16x8*)(qh + 32 * ks + 8 * grp);
            qb[ks] = col < nh ? x : (f16x8)0;
        }
    }

    float m = -INFINITY, l = 0.0f;
    f32x4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = (f32x4)0.0f;
    _Float16* vs = (_Float16*)smem + w * TK * HD;

    const uint32_t ntiles = (end - start + TK - 1) / TK;
    constexpr int NG = GROUPED ? MT : 1;
    // key `key` (< TK) of the current tile in a plane whose group bases are `gb`
    auto at = [&](const uint16_t* const* gb, int key) -> const uint16_t* {
        if constexpr (GROUPED) return gb[key >> 4] + (uint64_t)(key & 15) * row;
        else return gb[0] + (uint64_t)key * row;
    };
    for (uint32_t j = w; j < ntiles; j += kWaves) {
        const uint32_t t0 = start + j * TK;
        const uint32_t nvalid = min((uint32_t)TK, end - t0);
        // the tile's bases: one page-table lookup a tile, or one a 16-key group when pages are shorter
        const uint16_t* kg[NG];
        const uint16_t* vg[NG];
        // (groups past the split's last key, never read from — their keys take key 0 — alias its last group, so no
        // page-table entry past the row's is looked up)
        const uint32_t last_group = (nvalid - 1) / 16;
#pragma unroll
        for (int p = 0; p < NG; ++p) {
            const uint32_t t = t0 + 16 * min((uint32_t)p, last_group);
            kg[p] = group_base(a.k, a, u, g, t, row, HD);
            vg[p] = group_base(a.v, a, u, g, t, row, HD);
        }

        // K as the A operand: lane (col, grp) reads key 16·p + col, dims 32·ks + 8·grp .. +8. Keys past the
        // split read key 0 of the tile (their scores are masked). Streamed once: non-temporal. (SHARED: from
        // the tile in LDS, below.)
        f16x8 kr[MT][KS];
        if constexpr (!SHARED) {
#pragma unroll
            for (int p = 0; p < MT; ++p) {
                const int key = 16 * p + col;
                const f16x8* kk = (const f16x8*)at(kg, key < (int)nvalid ? key : 0) + grp;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    kr[p][ks] = (VARIANT & 1) ? __builtin_nontemporal_load(kk + 4 * ks) : kk[4 * ks];
            }
        }
        // V straight into LDS: the load of step i writes slots 64·i .. 64·i + 63, one a lane; slot (key, c)
        // holds the row's chunk c ^ f(key). Keys past the split bring key 0 of the tile (weight 0).
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int slot = lane + 64 * i, key = slot / CPR, c = vslot(key, slot % CPR);
            const uint16_t* src = at(vg, key < (int)nvalid ? key : 0) + 8 * c;
            __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(vs + 64 * 8 * i),
                                             16, 0, (VARIANT & 2) ? kCacheStream : 0);
        }

        if constexpr (SHARED) {
            // the tile landed; key 16·p + col's chunk 4·ks + grp sits at slot chunk ^ f(key) of its row
            __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int p = 0; p < MT; ++p) {
                const int key = 16 * p + col;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) kr[p][ks] = *(const f16x8*)(vs + (key * CPR + vslot(key, 4 * ks + grp)) * 8);
            }
        }
        // S^T: lane holds keys 16·p + 4·grp + r of head col.
        float sv[MT * 4];
#pragma unroll
        for (int p = 0; p < MT; ++p) {
            f32x4 st = (f32x4)0.0f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[p][ks], qb[ks], st, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = 16 * p + 4 * grp + r;
                sv[4 * p + r] = key < (int)nvalid ? st[r] * a.scale : -INFINITY;
            }
        }
        float mx = sv[0];
#pragma unroll
        for (int r = 1; r < MT * 4; ++r) mx = fmaxf(mx, sv[r]);
        mx = groups_max(mx);
        const float mnew = fmaxf(m, mx);
        const float corr = fast_exp(m - mnew);
        float lsum = 0.0f;
        // P^T as the B operand of k-step sp (32 keys): keys 32·sp + 4·grp + jj and 32·sp + 16 + 4·grp + jj —
        // the S^T registers of M tiles 2·sp and 2·sp + 1
        f16x8 pb[MT / 2];
#pragma unroll
        for (int r = 0; r < MT * 4; ++r) {
            const float pr = fast_exp(sv[r] - mnew);
            lsum += pr;
            pb[r / 8][r % 8] = (_Float16)pr;
        }
        l = l * corr + lsum;
        m = mnew;
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] *= corr;

        // The value tile landed (the direct loads count as vector memory); read it transposed as the A
        // operand: lane (col, grp) takes dim 16·n + col of the keys its P^T column holds.
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int sp = 0; sp < MT / 2; ++sp)
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const int d = 16 * n + col;
                f16x8 va;
                if constexpr (VTR) {
                    // lane 4·jj + rr of 16-lane block grp points at key 32·sp + 4·grp + jj (+ 16), dims
                    // 16·n + 4·rr .. +3; lane col of the block gets dim 16·n + col of its four keys
                    const int li = lane & 15, jj = li >> 2, d0 = 16 * n + 4 * (li & 3);
                    const int k0 = 32 * sp + 4 * grp + jj, k1 = k0 + 16;
                    typedef short s16x4 __attribute__((ext_vector_type(4)));
                    const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4*)(vs + (k0 * CPR + vslot(k0, d0 >> 3)) * 8 + (d0 & 7)));
                    const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4*)(vs + (k1 * CPR + vslot(k1, d0 >> 3)) * 8 + (d0 & 7)));
                    va = __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
                } else {
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const int key = 32 * sp + (jj < 4 ? 4 * grp + jj : 16 + 4 * grp + (jj - 4));
                        va[jj] = vs[(key * CPR + vslot(key, d >> 3)) * 8 + (d & 7)];
                    }
                }
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[sp], acc[n], 0, 0, 0);
            }
        // every lane's reads of this tile are done before the next tile's loads overwrite it
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
    }
    l = groups_sum(l);

    // The four waves' residuals, merged in LDS into the split's one.
    __syncthreads();
    float* os = (float*)smem;                 // [wave][head][HD]
    float* ms = os + kWaves * 16 * HD;        // [wave][head]
    float* ls = ms + kWaves * 16;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) os[(w * 16 + col) * HD + 16 * n + 4 * grp + r] = acc[n][r];
    if (grp == 0) {
        ms[w * 16 + col] = m;
        ls[w * 16 + col] = l;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nh * HD; idx += kThreads) {
        const int hh = idx / HD, d = idx % HD;
        float mm = ms[hh];
#pragma unroll
        for (int ww = 1; ww < kWaves; ++ww) mm = fmaxf(mm, ms[ww * 16 + hh]);
        float sum = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
            const float f = fast_exp(ms[ww * 16 + hh] - mm);
            sum += os[(ww * 16 + hh) * HD + d] * f;
            lsum += ls[ww * 16 + hh] * f;
        }
        float* pr = a.part + (((uint64_t)u * a.q_heads + h0 + hh) * a.nsplit + s) * (HD + 2);
        pr[2 + d] = sum;
        if (d == 0) {
            pr[0] = mm;
            pr[1] = lsum;
        }
    }
    if constexpr (FUSED) {
        // Release this split's residual device-wide, then count it in. A row of at most kFinishGroup splits: the
        // split that makes the row's count whole acquires the others' residuals and finishes the heads. A longer
        // row finishes in two levels, so no one workgroup reads every split's residual: the split that completes
        // its group of kFinishGroup merges the group, exactly, into the group's first slot, then counts the group
        // in, and the group that completes the row finishes the heads from the group slots.
        __threadfence();
        __syncthreads();
        const uint32_t ns = (len + a.chunk - 1) / a.chunk;
        const uint32_t ng = (ns + kFinishGroup - 1) / kFinishGroup;
        const uint32_t gi = s / kFinishGroup, g0 = gi * kFinishGroup, gsz = min(kFinishGroup, ns - g0);
        const uint64_t unit = (uint64_t)u * GH + gh;
        const float* base = a.part + ((uint64_t)u * a.q_heads + h0) * a.nsplit * (HD + 2);
        // count one in at entry i of a plane of counts; answers whether that made `total`
        auto count_in = [&](uint32_t* plane, uint64_t i, uint32_t total) -> bool {
            if constexpr (INLINE) {
                // no plan launch cleared the count: a word of another tag is a count of zero
                unsigned long long* word = (unsigned long long*)plane + i;
                unsigned long long seen = *(volatile unsigned long long*)word, was;   // a guess the CAS corrects
                uint32_t count;
                do {
                    was = seen;
                    count = (was >> kTagShift) == a.tag ? (uint32_t)(was & ((1u << kTagShift) - 1)) : 0u;
                    seen = atomicCAS(word, was, (a.tag << kTagShift) | (count + 1u));
                } while (seen != was);
                return count == total - 1;
            } else {
                return atomicAdd(plane + i, 1u) == total - 1;
            }
        };
        // the answers from `count` residuals, slot q at q·stride: a wave a head for the largest m and
        // l = Σ e^(m_s - M)·l_s, then a lane a (head, dim) for acc / l
        auto finish = [&](uint32_t count, uint32_t stride) {
            for (int hh = w; hh < nh; hh += kWaves) {
                const float* ph = base + (uint64_t)hh * a.nsplit * (HD + 2);
                float mm = -INFINITY;
                for (uint32_t q = lane; q < count; q += 64) mm = fmaxf(mm, ph[(uint64_t)q * stride * (HD + 2)]);
                mm = wave_max(mm);
                float ll = 0.0f;
                for (uint32_t q = lane; q < count; q += 64)
                    ll += fast_exp(ph[(uint64_t)q * stride * (HD + 2)] - mm) * ph[(uint64_t)q * stride * (HD + 2) + 1];
                ll = wave_sum(ll);
                if (lane == 0) {
                    ms[hh] = mm;
                    ls[hh] = ll;
                }
            }
            __syncthreads();
            bool hit = false;
            for (int idx = threadIdx.x; idx < nh * HD; idx += kThreads) {
                const int hh = idx / HD, d = idx % HD;
                const float* ph = base + (uint64_t)hh * a.nsplit * (HD + 2);
                const float mm = ms[hh];
                float acc = 0.0f;
                for (uint32_t q = 0; q < count; ++q)
                    acc += fast_exp(ph[(uint64_t)q * stride * (HD + 2)] - mm) * ph[(uint64_t)q * stride * (HD + 2) + 2 + d];
                a.o[((uint64_t)u * a.q_heads + h0 + hh) * HD + d] = to_half(acc / ls[hh], hit);
            }
            if (hit) *a.over = kFaultOverflow;
        };
        if (threadIdx.x == 0)
            is_last = ng == 1 ? count_in(a.done, unit, ns) : count_in(a.gdone, unit * a.maxng + gi, gsz);
        __syncthreads();
        if (is_last) {
            __threadfence();
            if (ng == 1) {
                finish(ns, 1);
            } else {
                // the group's residual into slot g0: each split's weight e^(m_s - M) a head (a lane a split), then
                // a lane a (head, dim) sums its column in place, then the head's M and l
                __shared__ float gw[16 * kFinishGroup];
                for (int hh = w; hh < nh; hh += kWaves) {
                    const float* ph = base + (uint64_t)hh * a.nsplit * (HD + 2) + (uint64_t)g0 * (HD + 2);
                    const float m_s = lane < (int)gsz ? ph[(uint64_t)lane * (HD + 2)] : -INFINITY;
                    const float mm = wave_max(m_s);
                    const float wt = lane < (int)gsz ? fast_exp(m_s - mm) : 0.0f;
                    const float ll = wave_sum(lane < (int)gsz ? wt * ph[(uint64_t)lane * (HD + 2) + 1] : 0.0f);
                    if (lane < (int)gsz) gw[hh * kFinishGroup + lane] = wt;
                    if (lane == 0) {
                        ms[hh] = mm;
                        ls[hh] = ll;
                    }
                }
                __syncthreads();
                for (int idx = threadIdx.x; idx < nh * HD; idx += kThreads) {
                    const int hh = idx / HD, d = idx % HD;
                    float* ph = (float*)base + (uint64_t)hh * a.nsplit * (HD + 2) + (uint64_t)g0 * (HD + 2);
                    float acc = 0.0f;
                    for (uint32_t j = 0; j < gsz; ++j) acc += gw[hh * kFinishGroup + j] * ph[(uint64_t)j * (HD + 2) + 2 + d];
                    ph[2 + d] = acc;
                }
                __syncthreads();
                if ((int)threadIdx.x < nh) {
                    float* ph = (float*)base + (uint64_t)threadIdx.x * a.nsplit * (HD + 2) + (uint64_t)g0 * (HD + 2);
                    ph[0] = ms[threadIdx.x];
                    ph[1] = ls[threadIdx.x];
                }
                // release the group's residual, then count the group in; the group that completes the row finishes
                __threadfence();
                __syncthreads();
                if (threadIdx.x == 0) is_last = count_in(a.done, unit, ng);
                __syncthreads();
                if (is_last) {
                    __threadfence();
                    finish(ng, kFinishGroup);
                }
            }
        }
    }
}

// head_dim 512 with the keys the values (latent attention), opt-in (SILVANN_GFX950_DECODE_LATENT=wide): one
// workgroup a (split, kv head, four head blocks), its four waves each a head block of up to 16 query heads, so each
// latent tile comes from L2 into LDS once for up to 64 heads — where decode_split<512, …, SHARED> brings it once for
// each head block's workgroup. The tiles (32 latents, 32 KB) go HBM → LDS directly through a ring of four stages,
// every wave loading an eighth of each: tile t + 3 is in flight while tile t computes, one barrier a tile. A wave
// past the group's head blocks loads and meets the barriers but computes nothing. No merge across the waves: each
// writes its head block's residual, which decode_merge joins as decode_split's.
constexpr int kLatentBlocks = 4;   // head blocks a workgroup
constexpr int kLatentStages = 4;
constexpr int vmcnt_only(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }
template <bool GROUPED>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void decode_latent(DecodeArgs a) {
    constexpr int HD = 512, TK = 32, MT = TK / 16, KS = HD / 32, NT = HD / 16, CPR = HD / 8;
    constexpr int kStage = TK * HD;                 // halves a stage
    constexpr int LOADS = TK * CPR / kThreads;      // 16-byte loads a thread a tile
    __shared__ __attribute__((aligned(16))) _Float16 ring[kLatentStages * kStage];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const uint64_t row = (uint64_t)a.kv_heads * HD;
    const uint32_t units = (a.hblocks + kLatentBlocks - 1) / kLatentBlocks, GH = a.kv_heads * units;
    const uint32_t item = blockIdx.x;
    if (item >= a.plan[a.rows + 1] * GH) return;
    const uint32_t sidx = item / GH, gh = item % GH;
    uint32_t u, s;
    {
        const uint32_t full = a.plan[a.rows];
        if (sidx < full) {
            uint32_t lo = 0, hi = a.rows;
            while (hi - lo > 1) {
                const uint32_t mid = (lo + hi) >> 1;
                if (a.plan[mid] <= sidx) lo = mid;
                else hi = mid;
            }
            u = lo;
            s = sidx - a.plan[lo];
        } else {
            u = a.plan[a.rows + 2 + (sidx - full)];
            s = a.plan[u + 1] - a.plan[u];
        }
    }
    const uint32_t g = gh / units, hb = (gh % units) * kLatentBlocks + w;
    const bool active = hb < a.hblocks;
    const uint32_t len = a.lens[u], start = s * a.chunk, end = min(len, start + a.chunk);
    const uint32_t h0 = g * a.group + hb * 16;
    const int nh = active ? min(16, (int)(a.group - hb * 16)) : 0;

    f16x8 qb[KS];
    {
        const uint16_t* qh = a.q + ((uint64_t)u * a.q_heads + (active ? h0 : 0) + (col < nh ? col : 0)) * HD;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            f16x8 x = *(const f16x8*)(qh + 32 * ks + 8 * grp);
            qb[ks] = col < nh ? x : (f16x8)0;
        }
    }
    float m = -INFINITY, l = 0.0f;
    f32x4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = (f32x4)0.0f;

    const uint32_t ntiles = (end - start + TK - 1) / TK;
    // tile t into its stage: this wave's slots w·LOADS·64 .. , slot (key, physical chunk) holding the key's logical
    // chunk chunk ^ f(key); latents past the split bring the tile's latent 0 (masked)
    auto load_tile = [&](uint32_t t) __attribute__((always_inline)) {
        const uint32_t t0 = start + t * TK, nvalid = min((uint32_t)TK, end - t0);
        const uint16_t* gb[GROUPED ? 2 : 1];
#pragma unroll
        for (int p = 0; p < (GROUPED ? 2 : 1); ++p)
            gb[p] = group_base(a.k, a, u, g, t0 + 16 * min((uint32_t)p, (nvalid - 1) / 16), row, HD);
        _Float16* st = ring + (t % kLatentStages) * kStage;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int slot = (w * LOADS + i) * 64 + lane, key = slot / CPR, c = vslot(key, slot % CPR);
            const int kk = key < (int)nvalid ? key : 0;
            const uint16_t* src = (GROUPED ? gb[kk >> 4] + (uint64_t)(kk & 15) * row : gb[0] + (uint64_t)kk * row) + 8 * c;
            dma16_nt(src, (__attribute__((address_space(3))) void*)(st + (w * LOADS + i) * 64 * 8));
        }
    };
    // vector-memory count <= (tiles issued after tile t + 1)·LOADS: tile t + 1 landed
    auto wait_next = [&](uint32_t t) __attribute__((always_inline)) {
        const uint32_t after = ntiles > t + 2 ? min(ntiles - t - 2, 2u) : 0u;
        if (after == 2) __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * LOADS));
        else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS));
        else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    };

    load_tile(0);
    if (ntiles > 1) load_tile(1);
    if (ntiles > 2) load_tile(2);
    if (ntiles > 2) __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * LOADS));
    else if (ntiles > 1) __builtin_amdgcn_s_waitcnt(vmcnt_only(LOADS));
    else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    __syncthreads();
    for (uint32_t t = 0; t < ntiles; ++t) {
        // stage (t + 3) % 4 held tile t - 1, which every wave finished before the last barrier
        if (t + 3 < ntiles) load_tile(t + 3);
        if (active) {
            const _Float16* vs = ring + (t % kLatentStages) * kStage;
            const uint32_t nvalid = min((uint32_t)TK, end - (start + t * TK));
            // S^T: lane holds latents 16·p + 4·grp + r of head col
            float sv[MT * 4];
#pragma unroll
            for (int p = 0; p < MT; ++p) {
                const int key = 16 * p + col;
                f32x4 st4 = (f32x4)0.0f;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    st4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8*)(vs + (key * CPR + vslot(key, 4 * ks + grp)) * 8),
                                                                qb[ks], st4, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int k2 = 16 * p + 4 * grp + r;
                    sv[4 * p + r] = k2 < (int)nvalid ? st4[r] * a.scale : -INFINITY;
                }
            }
            float mx = sv[0];
#pragma unroll
            for (int r = 1; r < MT * 4; ++r) mx = fmaxf(mx, sv[r]);
            mx = groups_max(mx);
            const float mnew = fmaxf(m, mx);
            const float corr = fast_exp(m - mnew);
            float lsum = 0.0f;
            f16x8 pb[MT / 2];
#pragma unroll
            for (int r = 0; r < MT * 4; ++r) {
                const float pr = fast_exp(sv[r] - mnew);
                lsum += pr;
                pb[r / 8][r % 8] = (_Float16)pr;
            }
            l = l * corr + lsum;
            m = mnew;
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] *= corr;
            // O^T += V^T · P^T, V^T through the transposing read: lane 4·jj + rr of block grp points at latent
            // 32·sp + 4·grp + jj (+ 16), dims 16·n + 4·rr .. +3
#pragma unroll
            for (int sp = 0; sp < MT / 2; ++sp)
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const int li = lane & 15, jj = li >> 2, d0 = 16 * n + 4 * (li & 3);
                    const int k0 = 32 * sp + 4 * grp + jj, k1 = k0 + 16;
                    typedef short s16x4 __attribute__((ext_vector_type(4)));
                    const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4*)(vs + (k0 * CPR + vslot(k0, d0 >> 3)) * 8 + (d0 & 7)));
                    const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4*)(vs + (k1 * CPR + vslot(k1, d0 >> 3)) * 8 + (d0 & 7)));
                    const f16x8 va = __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[sp], acc[n], 0, 0, 0);
                }
        }
        if (t + 1 < ntiles) {
            wait_next(t);
            __syncthreads();   // tile t + 1 is in LDS for every wave; every wave is done reading tile t
        }
    }
    if (!active) return;
    l = groups_sum(l);
    if (col < nh) {
        float* pr = a.part + (((uint64_t)u * a.q_heads + h0 + col) * a.nsplit + s) * (HD + 2);
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) pr[2 + 16 * n + 4 * grp + r] = acc[n][r];
        if (grp == 0) {
            pr[0] = m;
            pr[1] = l;
        }
    }
}

// Pass 2: a workgroup of 4 or 16 waves (by the split count) per (row, query head, 64 dims). Wave w takes
// splits w, w + waves, …, eight
// at a time with eight independent sums (their loads in flight together); a lane holds one dim; the waves'
// sums meet in LDS. Every split's weight e^(m_s - M) needs the head's largest m first, folded over the
// whole workgroup.
// SINK: each head's sum takes one more term, e^(sink[h] - M) with M over the sink too (attention_softmax_sink's
// weights, kernels.cuh:1115-1131, mixed: one query row).
template <int HD, int kMergeWaves, bool SINK = false>
__global__ __launch_bounds__(64 * kMergeWaves) void decode_merge(uint16_t* o, const float* part, const uint32_t* lens,
                                                                 uint32_t q_heads, uint32_t chunk, uint32_t nsplit,
                                                                 unsigned int* over, const uint16_t* sink) {
    __shared__ float red[kMergeWaves];
    __shared__ float accs[kMergeWaves][64];
    __shared__ float ls[kMergeWaves];
    const uint32_t h = blockIdx.x, u = blockIdx.y;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int d = blockIdx.z * 64 + lane;
    const uint32_t len = lens[u];
    uint16_t* out = o + ((uint64_t)u * q_heads + h) * HD;
    if (len == 0) {
        if (w == 0) out[d] = 0;
        return;
    }
    const uint32_t ns = (len + chunk - 1) / chunk;
    const float* pr = part + ((uint64_t)u * q_heads + h) * nsplit * (HD + 2);

    float mx = -INFINITY;
    for (uint32_t s = threadIdx.x; s < ns; s += 64 * kMergeWaves) mx = fmaxf(mx, pr[(uint64_t)s * (HD + 2)]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int k = 1; k < kMergeWaves; ++k) M = fmaxf(M, red[k]);
    float sk = 0.0f;
    if constexpr (SINK) {
        sk = half_bits_to_float(sink[h]);
        M = fmaxf(M, sk);
    }

    constexpr int U = 8;
    float accu[U], lsu[U];
#pragma unroll
    for (int k = 0; k < U; ++k) accu[k] = lsu[k] = 0.0f;
    uint32_t s = w;
    for (; s + kMergeWaves * (U - 1) < ns; s += kMergeWaves * U) {
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const float* a = pr + (uint64_t)(s + kMergeWaves * k) * (HD + 2);
            const float f = fast_exp(a[0] - M);
            accu[k] += f * a[2 + d];
            lsu[k] += f * a[1];
        }
    }
    for (; s < ns; s += kMergeWaves) {
        const float* a = pr + (uint64_t)s * (HD + 2);
        const float f = fast_exp(a[0] - M);
        accu[0] += f * a[2 + d];
        lsu[0] += f * a[1];
    }
    float acc = 0.0f, lsum = 0.0f;
#pragma unroll
    for (int k = 0; k < U; ++k) {
        acc += accu[k];
        lsum += lsu[k];
    }
    accs[w][lane] = acc;
    if (lane == 0) ls[w] = lsum;
    __syncthreads();
    if (w != 0) return;
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int k = 0; k < kMergeWaves; ++k) {
        L += ls[k];
        A += accs[k][lane];
    }
    if constexpr (SINK) L += fast_exp(sk - M);
    bool hit = false;
    out[d] = to_half(A / L, hit);
    if (hit) *over = kFaultOverflow;
}

// One row of a uniform length: its length where decode_split reads it, its one-row plan (as decode_plan lays it
// out), the counter zeroed — the plan of the deferred door pairs, whose one query's length is a host value.
__global__ void decode_plan_one(uint32_t* lens, uint32_t length, uint32_t chunk, uint32_t* plan, uint32_t* counter) {
    if (threadIdx.x == 0) {
        lens[0] = length;
        plan[0] = 0;
        plan[1] = length / chunk;                  // the full splits
        plan[2] = (length + chunk - 1) / chunk;    // all splits
        plan[3] = 0;                               // the row of the shorter last split, if there is one
        counter[0] = 0;
    }
}

// Row u of a causal chunk attends positions 0 .. first + u: its length, where decode_plan and decode_split read it.
__global__ void causal_lens(uint32_t* lens, uint32_t first, uint32_t rows) {
    for (uint32_t u = blockIdx.x * blockDim.x + threadIdx.x; u < rows; u += gridDim.x * blockDim.x) lens[u] = first + u + 1;
}

// decode_merge's arithmetic into the reference's residual instead of an answer: res[h] = {M, Σ e^(m_s - M)·l_s,
// Σ e^(m_s - M)·acc_s} (kernels.cuh:1243-1255 over the splits), a workgroup per (query head, 64 dims), one row.
template <int HD>
__global__ __launch_bounds__(256) void decode_merge_res(float* res, const float* part, uint32_t nsplit) {
    __shared__ float red[4];
    __shared__ float accs[4][64];
    __shared__ float lss[4];
    const uint32_t h = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int d = blockIdx.z * 64 + lane;
    const float* pr = part + (uint64_t)h * nsplit * (HD + 2);
    float* out = res + (uint64_t)h * (HD + 2);
    float mx = -INFINITY;
    for (uint32_t s = threadIdx.x; s < nsplit; s += 256) mx = fmaxf(mx, pr[(uint64_t)s * (HD + 2)]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float acc = 0.0f, lsum = 0.0f;
    for (uint32_t s = w; s < nsplit; s += 4) {
        const float* x = pr + (uint64_t)s * (HD + 2);
        const float f = fast_exp(x[0] - M);
        acc += f * x[2 + d];
        lsum += f * x[1];
    }
    accs[w][lane] = acc;
    if (lane == 0) lss[w] = lsum;
    __syncthreads();
    if (w != 0) return;
    out[2 + d] = accs[0][lane] + accs[1][lane] + accs[2][lane] + accs[3][lane];
    if (d == 0) {
        out[0] = M;
        out[1] = lss[0] + lss[1] + lss[2] + lss[3];
    }
}

// The split length: a multiple of the 4 waves' tiles, sized so the items (splits × kv heads × head blocks,
// over the longest row for every row) about fill the chip once — more would re-pay the per-item merge,
// fewer would leave CUs idle — and never past 1024 positions, past which the measured rate falls.
// SILVANN_GFX950_DECODE_CHUNK overrides.
uint64_t resident_groups();
uint32_t choose_chunk(uint64_t head_dim, uint64_t kv_heads, uint64_t hblocks, uint64_t most, uint64_t rows) {
    const uint64_t step = (uint64_t)tile_keys((int)head_dim) * kWaves;
    uint64_t c = 0;
    if (const char* e = getenv("SILVANN_GFX950_DECODE_CHUNK")) c = strtoull(e, nullptr, 10);
    if (c == 0) {
        const uint64_t work = most * rows * kv_heads * hblocks;
        c = (work + resident_groups() - 1) / resident_groups();
        if (c > 1024) c = 1024;
    }
    c = (c + step - 1) / step * step;
    if (c < step) c = step;
    while ((most + c - 1) / c > kMaxSplits) c += step;
    return (uint32_t)c;
}

// Workgroups of decode_split the current device holds at once: two a CU (64 KB of LDS and two waves a SIMD
// each). SILVANN_GFX950_DECODE_GROUPS overrides.
uint64_t resident_groups() {
    static thread_local int dev_cached = -1;
    static thread_local uint64_t groups = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (dev != dev_cached) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        groups = 2ull * (uint64_t)cus;
        if (const char* e = getenv("SILVANN_GFX950_DECODE_GROUPS")) {
            const uint64_t g = strtoull(e, nullptr, 10);
            if (g > 0) groups = g;
        }
        dev_cached = dev;
    }
    return groups;
}

bool vtr() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_DECODE_VTR");
        return e && strtol(e, nullptr, 10) > 0;
    }();
    return on;
}

// The fused finish (SILVANN_GFX950_DECODE_FUSED=1): checked in the CPU emulation, not yet measured on a GPU.
bool fused_finish() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_DECODE_FUSED");
        return e && strtol(e, nullptr, 10) > 0;
    }();
    return on;
}

// This call's tag for the fused finish's tagged counts: a process-wide serial from a random start, 40 bits, so a
// count word left by another call (or any earlier contents of the scratch) shows another tag but by a 2^-40 chance.
uint64_t next_tag() {
    static std::atomic<uint64_t> serial{[] {
        std::random_device rd;
        return ((uint64_t)rd() << 32) ^ (uint64_t)rd();
    }()};
    return serial.fetch_add(1, std::memory_order_relaxed) & kTagMask;
}

// The plan made inside decode_split at batches of at most 64 rows (SILVANN_GFX950_DECODE_INLINE=1): checked in the
// CPU emulation, not yet measured on a GPU.
bool inline_plan() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_DECODE_INLINE");
        return e && strtol(e, nullptr, 10) > 0;
    }();
    return on;
}

// Latent attention's wide form (SILVANN_GFX950_DECODE_LATENT=wide): checked in the CPU emulation, not yet
// measured on a GPU.
bool latent_wide() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_DECODE_LATENT");
        return e && strcmp(e, "wide") == 0;
    }();
    return on;
}

// decode_split over contiguous caches, one workgroup an item, `splits` = rows · splits a row: head_dim 64-512, the
// keys-are-values form at 512 when `shared`; INL makes the plan inside the kernel.
template <bool INL>
void split_contiguous(const DecodeArgs& a, uint64_t head_dim, bool shared, uint64_t splits, hipStream_t st) {
    const uint64_t gh = (uint64_t)a.kv_heads * a.hblocks;
    const dim3 grid((uint32_t)(splits * gh));
    if (head_dim == 512) {
        if (shared) decode_split<512, 2, false, true, false, true, INL><<<dim3(shared_grid(splits, gh)), kThreads, 0, st>>>(a);
        else decode_split<512, 2, false, false, false, true, INL><<<grid, kThreads, 0, st>>>(a);
    } else if (head_dim == 256) {
        decode_split<256, kDefaultVariant, false, false, false, false, INL><<<grid, kThreads, 0, st>>>(a);
    } else if (head_dim == 128) {
        decode_split<128, kDefaultVariant, false, false, false, false, INL><<<grid, kThreads, 0, st>>>(a);
    } else {
        decode_split<64, kDefaultVariant, false, false, false, false, INL><<<grid, kThreads, 0, st>>>(a);
    }
}

uint32_t head_blocks(uint64_t q_heads, uint64_t kv_heads) { return (uint32_t)((q_heads / kv_heads + 15) / 16); }

bool decode_shape_ok(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512) && kv_heads > 0 && q_heads > 0 && q_heads % kv_heads == 0 &&
           rows > 0 && rows <= 65535 && most > 0 && most < (1ull << 31) && kv_heads * head_blocks(q_heads, kv_heads) <= 65535;
}

}  // namespace

void decode_paged_launch(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* pages,
                         uint64_t pages_row, uint64_t page_size, uint64_t k_row, const uint32_t* lens,
                         uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows,
                         float* scratch, unsigned int* over) {
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, most, rows) || (pages && (page_size == 0 || page_size % 16 || page_size > 0x7FFFFFFFull))) {
        fprintf(stderr, "silvann_gfx950: attention_decode_paged: unsupported shape (q_heads %llu kv_heads %llu "
                        "head_dim %llu most %llu rows %llu page_size %llu)\n",
                (unsigned long long)q_heads, (unsigned long long)kv_heads, (unsigned long long)head_dim,
                (unsigned long long)most, (unsigned long long)rows, (unsigned long long)page_size);
        refuse("attention_decode_paged");
        return;
    }
    if (!vec_aligned(q, k, v) || !scratch_aligned(scratch) || k_row % 8 != 0) {
        fprintf(stderr, "silvann_gfx950: attention_decode_paged: q, k and v must be 16-byte aligned, k_row a multiple "
                        "of 8 elements and scratch 8-byte aligned\n");
        refuse("attention_decode_paged");
        return;
    }
    DecodeArgs a;
    a.q = q; a.k = k; a.v = v; a.pages = pages; a.pages_row = pages_row; a.page_size = page_size; a.k_row = k_row;
    a.lens = lens;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hblocks = head_blocks(q_heads, kv_heads);
    // latent attention's wide form: a workgroup takes four head blocks, so a quarter of the units share the chip
    const bool latent = head_dim == 512 && k == v && latent_wide();
    const uint32_t lunits = (a.hblocks + kLatentBlocks - 1) / kLatentBlocks;
    a.chunk = choose_chunk(head_dim, kv_heads, latent ? lunits : a.hblocks, most, rows);
    a.nsplit = (uint32_t)((most + a.chunk - 1) / a.chunk);
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.counter = (uint32_t*)scratch;
    a.plan = (const uint32_t*)((char*)scratch + kPlanAt);
    a.done = (uint32_t*)((char*)scratch + done_at(rows));
    a.maxng = (a.nsplit + kFinishGroup - 1) / kFinishGroup;
    a.gdone = (uint32_t*)((char*)scratch + groups_at(rows, kv_heads * a.hblocks));
    a.part = (float*)((char*)scratch + part_at(rows, kv_heads * a.hblocks, a.maxng));
    a.rows = (uint32_t)rows;
    a.o = o;
    a.over = over;
    a.len_first = a.len_step = 0;
    a.lens_out = nullptr;
    a.tag = 0;
    const dim3 mgrid((uint32_t)q_heads, (uint32_t)rows, (uint32_t)(head_dim / 64));
    hipStream_t st = stream();
    static const int variant = [] {
        const char* e = getenv("SILVANN_GFX950_DECODE_VARIANT");
        return e ? (int)(strtol(e, nullptr, 10) & 3) : kDefaultVariant;
    }();
    const bool grouped = pages && page_size % tile_keys((int)head_dim) != 0;
    // as many workgroups as the chip holds at once (two a CU: LDS and registers allow no more), never more
    // than there are work items
    const uint64_t items = rows * a.nsplit * kv_heads * a.hblocks;   // at least the items there are
    if (items + 8 * kv_heads * a.hblocks > kMaxGroups) {   // (the shared form rounds its splits up to 8)
        refuse("attention_decode_paged");
        return;
    }
    const dim3 igrid((uint32_t)items);
    const bool fused = fused_finish();
    if (fused && head_dim <= 256 && inline_plan() && rows <= 64) {
        // one launch: the plan made in the kernel, the counts tagged with this call's tag
        a.tag = next_tag();
        prof_begin(kProfDecodeSplit);
        const uint32_t hv = (uint32_t)head_dim;
        if (grouped) {
            if (hv == 64) decode_split<64, kDefaultVariant, true, false, true, false, true><<<igrid, kThreads, 0, st>>>(a);
            else if (hv == 128) decode_split<128, kDefaultVariant, true, false, true, false, true><<<igrid, kThreads, 0, st>>>(a);
            else decode_split<256, kDefaultVariant, true, false, true, false, true><<<igrid, kThreads, 0, st>>>(a);
        } else {
            if (hv == 64) decode_split<64, kDefaultVariant, false, false, true, false, true><<<igrid, kThreads, 0, st>>>(a);
            else if (hv == 128) decode_split<128, kDefaultVariant, false, false, true, false, true><<<igrid, kThreads, 0, st>>>(a);
            else decode_split<256, kDefaultVariant, false, false, true, false, true><<<igrid, kThreads, 0, st>>>(a);
        }
        prof_end(kProfDecodeSplit);
        check_launch("attention_decode_paged");
        return;
    }
    if (fused && head_dim <= 256) {
        const uint32_t units = a.kv_heads * a.hblocks;
        decode_plan<true><<<1, 256, 0, st>>>(lens, a.rows, a.chunk, (uint32_t*)a.plan, a.counter, a.done, units, o,
                                             a.q_heads * (uint32_t)head_dim, a.gdone, a.maxng);
        prof_begin(kProfDecodeSplit);
        const uint32_t hv = (uint32_t)head_dim;
        if (grouped) {
            if (hv == 64) decode_split<64, kDefaultVariant, true, false, true><<<igrid, kThreads, 0, st>>>(a);
            else if (hv == 128) decode_split<128, kDefaultVariant, true, false, true><<<igrid, kThreads, 0, st>>>(a);
            else decode_split<256, kDefaultVariant, true, false, true><<<igrid, kThreads, 0, st>>>(a);
        } else {
            if (hv == 64) decode_split<64, kDefaultVariant, false, false, true><<<igrid, kThreads, 0, st>>>(a);
            else if (hv == 128) decode_split<128, kDefaultVariant, false, false, true><<<igrid, kThreads, 0, st>>>(a);
            else decode_split<256, kDefaultVariant, false, false, true><<<igrid, kThreads, 0, st>>>(a);
        }
        prof_end(kProfDecodeSplit);
        check_launch("attention_decode_paged");
        return;
    }
    // the plan made inside decode_split at batches of at most 64 rows: one launch fewer a step
    const bool inlined = inline_plan() && rows <= 64 && head_dim <= 256 && !vtr();
    if (!inlined) decode_plan<<<1, 256, 0, st>>>(lens, a.rows, a.chunk, (uint32_t*)a.plan, a.counter);
    prof_begin(kProfDecodeSplit);
    // head_dim 512: one workgroup an item; the shared-tile form when the keys are the values
    const bool shared = k == v;
    if (head_dim == 512) {
        if (shared && latent) {
            const dim3 lgrid((uint32_t)(rows * a.nsplit * kv_heads * lunits));
            if (grouped) decode_latent<true><<<lgrid, kThreads, 0, st>>>(a);
            else decode_latent<false><<<lgrid, kThreads, 0, st>>>(a);
        } else if (shared) {
            const dim3 sgrid(shared_grid(rows * a.nsplit, kv_heads * a.hblocks));
            if (grouped) decode_split<512, 2, true, true><<<sgrid, kThreads, 0, st>>>(a);
            else decode_split<512, 2, false, true><<<sgrid, kThreads, 0, st>>>(a);
        } else {
            if (grouped) decode_split<512, 2, true><<<igrid, kThreads, 0, st>>>(a);
            else decode_split<512, 2, false><<<igrid, kThreads, 0, st>>>(a);
        }
    } else if (inlined) {
        switch (head_dim) {
#define SILVANN_DECODE_INLINE(HDV) \
            case HDV: \
                if (grouped) decode_split<HDV, kDefaultVariant, true, false, false, false, true><<<igrid, kThreads, 0, st>>>(a); \
                else decode_split<HDV, kDefaultVariant, false, false, false, false, true><<<igrid, kThreads, 0, st>>>(a); \
                break;
            SILVANN_DECODE_INLINE(64) SILVANN_DECODE_INLINE(128) SILVANN_DECODE_INLINE(256)
#undef SILVANN_DECODE_INLINE
            default: break;
        }
    } else if (vtr()) {
        // the transposing V^T read at head_dim <= 256 (SILVANN_GFX950_DECODE_VTR=1): checked in the CPU emulation,
        // not yet measured against the element reads these widths run by default
        switch (head_dim) {
#define SILVANN_DECODE_VTR(HDV) \
            case HDV: \
                if (grouped) decode_split<HDV, kDefaultVariant, true, false, false, true><<<igrid, kThreads, 0, st>>>(a); \
                else decode_split<HDV, kDefaultVariant, false, false, false, true><<<igrid, kThreads, 0, st>>>(a); \
                break;
            SILVANN_DECODE_VTR(64) SILVANN_DECODE_VTR(128) SILVANN_DECODE_VTR(256)
#undef SILVANN_DECODE_VTR
            default: break;
        }
    } else switch (head_dim * 4 + variant) {
#define SILVANN_DECODE_CASE(HDV, VAR) \
        case HDV * 4 + VAR: \
            if (grouped) decode_split<HDV, VAR, true><<<igrid, kThreads, 0, st>>>(a); \
            else decode_split<HDV, VAR, false><<<igrid, kThreads, 0, st>>>(a); \
            break;
        SILVANN_DECODE_CASE(64, 0) SILVANN_DECODE_CASE(64, 1) SILVANN_DECODE_CASE(64, 2) SILVANN_DECODE_CASE(64, 3)
        SILVANN_DECODE_CASE(128, 0) SILVANN_DECODE_CASE(128, 1) SILVANN_DECODE_CASE(128, 2) SILVANN_DECODE_CASE(128, 3)
        SILVANN_DECODE_CASE(256, 0) SILVANN_DECODE_CASE(256, 1) SILVANN_DECODE_CASE(256, 2) SILVANN_DECODE_CASE(256, 3)
#undef SILVANN_DECODE_CASE
        default: break;
    }
    prof_end(kProfDecodeSplit);
    prof_begin(kProfDecodeMerge);
    const bool wide = a.nsplit > 64;
#define SILVANN_MERGE(HDV) \
    if (wide) decode_merge<HDV, 16><<<mgrid, 1024, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr); \
    else decode_merge<HDV, 4><<<mgrid, 256, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr);
    switch (head_dim) {
        case 64: SILVANN_MERGE(64) break;
        case 128: SILVANN_MERGE(128) break;
        case 256: SILVANN_MERGE(256) break;
        default: SILVANN_MERGE(512) break;
    }
#undef SILVANN_MERGE
    prof_end(kProfDecodeMerge);
    check_launch("attention_decode_paged");
}

// One query over a contiguous cache — the deferred door pairs' fused form (attention_scores + attention_mix into
// `o`; attention_weights + attention_residual_mix into `res`). Its scratch is the pair's own weights buffer, `cap`
// bytes, which the fused form never fills with weights: the splits are made long enough for their residuals to fit
// it. Answers false, launching nothing, when the shape is not one decode_split takes or no split length fits.
bool decode_one(uint16_t* o, float* res, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint64_t q_heads,
                uint64_t kv_heads, uint64_t head_dim, uint64_t length, void* scratch, uint64_t cap, unsigned int* over,
                const uint16_t* sink) {
    if (sink && !o) return false;   // a sink weighs the answer's sum; the residual form has none
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, length, 1) || !vec_aligned(q, k, v) || !scratch_aligned(scratch))
        return false;
    const uint32_t hblocks = head_blocks(q_heads, kv_heads);
    const uint64_t head = part_at(1, kv_heads * hblocks), per_split = q_heads * (head_dim + 2) * sizeof(float);
    if (cap <= head || (cap - head) / per_split == 0) return false;
    const uint64_t fit = (cap - head) / per_split;   // splits the scratch holds
    const uint64_t step = (uint64_t)tile_keys((int)head_dim) * kWaves;
    uint64_t chunk = choose_chunk(head_dim, kv_heads, hblocks, length, 1);
    if ((length + chunk - 1) / chunk > fit) chunk = ((length + fit - 1) / fit + step - 1) / step * step;
    const uint64_t nsplit = (length + chunk - 1) / chunk;
    if (nsplit > fit || nsplit > kMaxSplits || (nsplit + 8) * kv_heads * hblocks > kMaxGroups) return false;
    DecodeArgs a;
    a.q = q; a.k = k; a.v = v; a.pages = nullptr; a.pages_row = 0; a.page_size = 0; a.k_row = 0;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hblocks = hblocks;
    a.chunk = (uint32_t)chunk;
    a.nsplit = (uint32_t)nsplit;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.counter = (uint32_t*)scratch;
    uint32_t* lens = (uint32_t*)((char*)scratch + 32);
    a.lens = lens;
    a.plan = (const uint32_t*)((char*)scratch + kPlanAt);
    a.done = (uint32_t*)((char*)scratch + done_at(1));
    a.part = (float*)((char*)scratch + head);
    a.rows = 1;
    a.o = o;
    a.over = over;
    a.len_first = a.len_step = 0;
    a.lens_out = nullptr;
    a.tag = 0;
    hipStream_t st = stream();
    prof_begin(kProfDecodeSplit);
    if (o && !sink && head_dim <= 256 && inline_plan() && fused_finish() && nsplit <= kFinishGroup) {
        // one launch: the last split of each head block finishes the answers, its counts tagged
        a.lens = nullptr;
        a.len_first = (uint32_t)length;
        a.lens_out = lens;
        a.tag = next_tag();
        const dim3 grid((uint32_t)(nsplit * kv_heads * hblocks));
        if (head_dim == 256) decode_split<256, kDefaultVariant, false, false, true, false, true><<<grid, kThreads, 0, st>>>(a);
        else if (head_dim == 128) decode_split<128, kDefaultVariant, false, false, true, false, true><<<grid, kThreads, 0, st>>>(a);
        else decode_split<64, kDefaultVariant, false, false, true, false, true><<<grid, kThreads, 0, st>>>(a);
        prof_end(kProfDecodeSplit);
        return true;
    }
    if (inline_plan()) {   // the length from the host, written out for the merge by the split kernel
        a.lens = nullptr;
        a.len_first = (uint32_t)length;
        a.lens_out = lens;
        split_contiguous<true>(a, head_dim, k == v, nsplit, st);
    } else {
        decode_plan_one<<<1, 64, 0, st>>>(lens, (uint32_t)length, a.chunk, (uint32_t*)a.plan, a.counter);
        split_contiguous<false>(a, head_dim, k == v, nsplit, st);
    }
    prof_end(kProfDecodeSplit);
    const dim3 mgrid((uint32_t)q_heads, 1, (uint32_t)(head_dim / 64));
    if (o) {
        const bool wide = nsplit > 64;
#define SILVANN_MERGE_ONE(HDV) \
        if (sink) { \
            if (wide) decode_merge<HDV, 16, true><<<mgrid, 1024, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, sink); \
            else decode_merge<HDV, 4, true><<<mgrid, 256, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, sink); \
        } else if (wide) decode_merge<HDV, 16><<<mgrid, 1024, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr); \
        else decode_merge<HDV, 4><<<mgrid, 256, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr);
        switch (head_dim) {
            case 64: SILVANN_MERGE_ONE(64) break;
            case 128: SILVANN_MERGE_ONE(128) break;
            case 256: SILVANN_MERGE_ONE(256) break;
            default: SILVANN_MERGE_ONE(512) break;
        }
#undef SILVANN_MERGE_ONE
    } else {
        switch (head_dim) {
            case 64: decode_merge_res<64><<<mgrid, 256, 0, st>>>(res, a.part, a.nsplit); break;
            case 128: decode_merge_res<128><<<mgrid, 256, 0, st>>>(res, a.part, a.nsplit); break;
            case 256: decode_merge_res<256><<<mgrid, 256, 0, st>>>(res, a.part, a.nsplit); break;
            default: decode_merge_res<512><<<mgrid, 256, 0, st>>>(res, a.part, a.nsplit); break;
        }
    }
    return true;
}

// Causal attention of `rows` rows over one contiguous cache as the split-K decode: row u attends positions 0 ..
// first + u (every row's cache is the same, k_row 0) — the deferred causal chain's fused form where causal_mfma
// takes no such shape (head_dim 512: latent attention's block prefill, where the latents are the keys and the
// values). Its scratch is the chain's weights buffer, `cap` bytes. Answers false, launching nothing, when the shape
// is not one decode_split takes or the scratch is too small.
bool decode_causal(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint64_t q_heads,
                   uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows, void* scratch, uint64_t cap,
                   unsigned int* over) {
    const uint64_t most = first + rows;
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, most, rows) || !vec_aligned(q, k, v) || !scratch_aligned(scratch))
        return false;
    const uint32_t hblocks = head_blocks(q_heads, kv_heads);
    const uint64_t lens_at = part_at(rows, kv_heads * hblocks);
    const uint64_t head = lens_at + (4 * rows + 255) / 256 * 256;
    const uint64_t per_split = rows * q_heads * (head_dim + 2) * sizeof(float);
    if (cap <= head || (cap - head) / per_split == 0) return false;
    const uint64_t fit = (cap - head) / per_split;   // splits a row the scratch holds
    const uint64_t step = (uint64_t)tile_keys((int)head_dim) * kWaves;
    uint64_t chunk = choose_chunk(head_dim, kv_heads, hblocks, most, rows);
    if ((most + chunk - 1) / chunk > fit) chunk = ((most + fit - 1) / fit + step - 1) / step * step;
    DecodeArgs a;
    a.chunk = (uint32_t)chunk;
    a.nsplit = (uint32_t)((most + chunk - 1) / chunk);
    if (a.nsplit > fit || a.nsplit > kMaxSplits || (rows * a.nsplit + 8) * kv_heads * hblocks > kMaxGroups) return false;
    a.q = q; a.k = k; a.v = v; a.pages = nullptr; a.pages_row = 0; a.page_size = 0; a.k_row = 0;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hblocks = hblocks;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.counter = (uint32_t*)scratch;
    uint32_t* lens = (uint32_t*)((char*)scratch + lens_at);
    a.lens = lens;
    a.plan = (const uint32_t*)((char*)scratch + kPlanAt);
    a.done = (uint32_t*)((char*)scratch + done_at(rows));
    a.part = (float*)((char*)scratch + head);
    a.rows = (uint32_t)rows;
    a.o = o;
    a.over = over;
    a.len_first = a.len_step = 0;
    a.lens_out = nullptr;
    a.tag = 0;
    hipStream_t st = stream();
    prof_begin(kProfDecodeSplit);
    if (inline_plan() && rows <= 64) {   // row u's length first + u + 1, written out for the merge by the split kernel
        a.lens = nullptr;
        a.len_first = (uint32_t)first + 1u;
        a.len_step = 1;
        a.lens_out = lens;
        split_contiguous<true>(a, head_dim, k == v, rows * a.nsplit, st);
    } else {
        causal_lens<<<(uint32_t)((rows + 255) / 256), 256, 0, st>>>(lens, (uint32_t)first, (uint32_t)rows);
        decode_plan<<<1, 256, 0, st>>>(lens, a.rows, a.chunk, (uint32_t*)a.plan, a.counter);
        split_contiguous<false>(a, head_dim, k == v, rows * a.nsplit, st);
    }
    prof_end(kProfDecodeSplit);
    const dim3 mgrid((uint32_t)q_heads, (uint32_t)rows, (uint32_t)(head_dim / 64));
    const bool wide = a.nsplit > 64;
#define SILVANN_MERGE_C(HDV) \
    if (wide) decode_merge<HDV, 16><<<mgrid, 1024, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr); \
    else decode_merge<HDV, 4><<<mgrid, 256, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr);
    switch (head_dim) {
        case 64: SILVANN_MERGE_C(64) break;
        case 128: SILVANN_MERGE_C(128) break;
        case 256: SILVANN_MERGE_C(256) break;
        default: SILVANN_MERGE_C(512) break;
    }
#undef SILVANN_MERGE_C
    return true;
}

// Rows over their own contiguous caches (row u's keys and values at k + u·k_row, lens[u] of them, lens on the device)
// — the deferred many-row grouped chain's fused form (scores_grouped_rows + softmax_lens + mix_rows, GLM 5.3's
// block of rows over their gathered latents). Its scratch is the chain's weights buffer, `cap` bytes, the split
// length raised until the splits fit it. Answers false, launching nothing, when the shape is not one decode_split
// takes or no split length fits.
bool decode_rows_fit(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* lens,
                     uint64_t k_row, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most,
                     uint64_t rows, void* scratch, uint64_t cap, unsigned int* over) {
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, most, rows) || !vec_aligned(q, k, v) || !scratch_aligned(scratch) ||
        k_row % 8 != 0)
        return false;
    const uint32_t hblocks = head_blocks(q_heads, kv_heads);
    const uint64_t head = part_at(rows, kv_heads * hblocks);
    const uint64_t per_split = rows * q_heads * (head_dim + 2) * sizeof(float);
    if (cap <= head || (cap - head) / per_split == 0) return false;
    const uint64_t fit = (cap - head) / per_split;   // splits a row the scratch holds
    const uint64_t step = (uint64_t)tile_keys((int)head_dim) * kWaves;
    uint64_t chunk = choose_chunk(head_dim, kv_heads, hblocks, most, rows);
    if ((most + chunk - 1) / chunk > fit) chunk = ((most + fit - 1) / fit + step - 1) / step * step;
    DecodeArgs a;
    a.chunk = (uint32_t)chunk;
    a.nsplit = (uint32_t)((most + chunk - 1) / chunk);
    if (a.nsplit > fit || a.nsplit > kMaxSplits || (rows * a.nsplit + 8) * kv_heads * hblocks > kMaxGroups) return false;
    a.q = q; a.k = k; a.v = v; a.pages = nullptr; a.pages_row = 0; a.page_size = 0; a.k_row = k_row;
    a.lens = lens;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hblocks = hblocks;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.counter = (uint32_t*)scratch;
    a.plan = (const uint32_t*)((char*)scratch + kPlanAt);
    a.done = (uint32_t*)((char*)scratch + done_at(rows));
    a.part = (float*)((char*)scratch + head);
    a.rows = (uint32_t)rows;
    a.o = o;
    a.over = over;
    a.len_first = a.len_step = 0;
    a.lens_out = nullptr;
    a.tag = 0;
    hipStream_t st = stream();
    prof_begin(kProfDecodeSplit);
    if (inline_plan() && rows <= 64) {
        split_contiguous<true>(a, head_dim, k == v, rows * a.nsplit, st);
    } else {
        decode_plan<<<1, 256, 0, st>>>(lens, a.rows, a.chunk, (uint32_t*)a.plan, a.counter);
        split_contiguous<false>(a, head_dim, k == v, rows * a.nsplit, st);
    }
    prof_end(kProfDecodeSplit);
    const dim3 mgrid((uint32_t)q_heads, (uint32_t)rows, (uint32_t)(head_dim / 64));
    const bool wide = a.nsplit > 64;
#define SILVANN_MERGE_R(HDV) \
    if (wide) decode_merge<HDV, 16><<<mgrid, 1024, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr); \
    else decode_merge<HDV, 4><<<mgrid, 256, 0, st>>>(o, a.part, lens, a.q_heads, a.chunk, a.nsplit, over, nullptr);
    switch (head_dim) {
        case 64: SILVANN_MERGE_R(64) break;
        case 128: SILVANN_MERGE_R(128) break;
        case 256: SILVANN_MERGE_R(256) break;
        default: SILVANN_MERGE_R(512) break;
    }
#undef SILVANN_MERGE_R
    return true;
}

uint64_t decode_paged_scratch(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows) {
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, most, rows)) return 0;
    const uint32_t hb = head_blocks(q_heads, kv_heads);
    auto need = [&](uint64_t units) {   // the chunk a grid of `units` workgroups a split takes
        const uint32_t chunk = choose_chunk(head_dim, kv_heads, units, most, rows);
        const uint64_t nsplit = (most + chunk - 1) / chunk;
        const uint64_t maxng = (nsplit + kFinishGroup - 1) / kFinishGroup;
        return part_at(rows, kv_heads * hb, maxng) + rows * q_heads * nsplit * (head_dim + 2) * sizeof(float);
    };
    // head_dim 512: enough for latent attention's wide form too (its splits are shorter), which the caller may take
    // (keys the values) or not
    const uint64_t n = need(hb);
    if (head_dim != 512) return n;
    const uint64_t nw = need((hb + kLatentBlocks - 1) / kLatentBlocks);
    return n > nw ? n : nw;
}

}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_attention_decode_paged(uint16_t* o, const uint16_t* q, const uint16_t* k,
                                                          const uint16_t* v, const uint32_t* pages, uint64_t pages_row,
                                                          uint64_t page_size, uint64_t k_row, const uint32_t* lens,
                                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                          uint64_t most, uint64_t rows, float* scratch,
                                                          unsigned int* over) {
    silvann::flush_deferred();
    silvann::decode_paged_launch(o, q, k, v, pages, pages_row, page_size, k_row, lens, q_heads, kv_heads, head_dim,
                                 most, rows, scratch, over);
}

SILVANN_EXPORT uint64_t silvann_gfx950_attention_decode_paged_scratch(uint64_t q_heads, uint64_t kv_heads,
                                                                      uint64_t head_dim, uint64_t most, uint64_t rows) {
    return silvann::decode_paged_scratch(q_heads, kv_heads, head_dim, most, rows);
}
