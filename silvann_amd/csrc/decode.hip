// decode.hip — split-K flash decoding for grouped-query attention over a paged (or contiguous) fp16 cache.
//
// The reference's decode is two doors: `attention_scores` writes every query head's softmax weights into
// `p`, `attention_mix` reads them back (kernels.cuh:885-915, 1133-1164). Here one pass reads each key and
// value once for all the query heads that share their kv head, and the reference's own residual contract
// (kernels.cuh:1180-1267: per head [m, l, acc], merged exactly by e^(m_a - m), e^(m_b - m)) joins the splits:
//
//   pass 1  decode_split: a workgroup of 4 waves per (row, kv head, head block of up to 16 query heads,
//           split of `chunk` positions). Each wave walks 32-key tiles of the split:
//             S^T = K · Q^T     v_mfma_f32_16x16x32_f16, keys as M, the group's query heads as N (a group of
//                               8 fills half the columns; the other half is zero — the decode is HBM-bound,
//                               and the MFMA has 50x the throughput it needs)
//             online softmax    in registers: a lane owns one query head's column; its tile max is folded
//                               over the column's four 16-lane groups
//             O^T += V^T · P^T  the same MFMA, keys as K: P comes straight from the S^T registers, V^T from
//                               the tile staged in LDS and read transposed
//           then the four waves' (m, l, O) merge in LDS and the split's residual goes to `part`.
//   pass 2  decode_merge: a workgroup per (row, query head) merges that head's split residuals and writes
//           acc / l as fp16, flagging overflow (kernels.cuh:1258-1267).
//
// K loads are 16 bytes a lane (8 halves of one key row: the MFMA A operand's own layout); V loads are
// 16 bytes a lane with consecutive lanes on consecutive bytes of a row.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

constexpr int kTile = 32;   // keys a wave takes a step
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kMaxSplits = 8192;  // the merge keeps a weight a split in LDS

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
};

// Where tile `t0` of row `u`, kv head `g` starts in a plane: through the page table, or contiguous.
__device__ __forceinline__ const uint16_t* tile_base(const uint16_t* plane, const DecodeArgs& a, uint32_t u,
                                                     uint32_t g, uint32_t t0, uint64_t row, int hd) {
    if (a.pages) {
        const uint64_t phys = (uint64_t)a.pages[(uint64_t)u * a.pages_row + t0 / a.page_size] * a.page_size +
                              t0 % a.page_size;
        return plane + phys * row + (uint64_t)g * hd;
    }
    return plane + (uint64_t)u * a.k_row + (uint64_t)t0 * row + (uint64_t)g * hd;
}

template <int HD>
__global__ __launch_bounds__(kThreads) void decode_split(DecodeArgs a) {
    constexpr int KS = HD / 32;      // k-steps of the S^T MFMA (32 dims each)
    constexpr int NT = HD / 16;      // d-tiles of the O^T accumulator
    constexpr int VP = HD + 16;      // LDS pitch of a staged value row, in halves (HD·2 + 32 bytes)
    constexpr int VCH = HD / 16;     // 16-byte value chunks a lane loads a tile
    constexpr int CPR = HD / 8;      // 16-byte chunks in one value row
    constexpr int kStageBytes = kWaves * kTile * VP * 2;
    constexpr int kMergeBytes = kWaves * 16 * HD * 4 + 2 * kWaves * 16 * 4;
    constexpr int kSmem = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSmem];

    const uint32_t s = blockIdx.x, u = blockIdx.z;
    const uint32_t g = blockIdx.y / a.hblocks, hb = blockIdx.y % a.hblocks;
    const uint32_t len = a.lens[u];
    const uint32_t start = s * a.chunk;
    if (start >= len) return;  // the whole workgroup: this split is past the row's length
    const uint32_t end = min(len, start + a.chunk);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const uint32_t h0 = g * a.group + hb * 16;
    const int nh = min(16, (int)(a.group - hb * 16));
    const uint64_t row = (uint64_t)a.kv_heads * HD;

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
    _Float16* vs = (_Float16*)smem + w * kTile * VP;

    const uint32_t ntiles = (end - start + kTile - 1) / kTile;
    for (uint32_t j = w; j < ntiles; j += kWaves) {
        const uint32_t t0 = start + j * kTile;
        const uint32_t nvalid = min((uint32_t)kTile, end - t0);
        const uint16_t* kb = tile_base(a.k, a, u, g, t0, row, HD);
        const uint16_t* vb = tile_base(a.v, a, u, g, t0, row, HD);

        // K as the A operand: lane (col, grp) reads key 16·p + col, dims 32·ks + 8·grp .. +8. Keys past the
        // split read key 0 of the tile (their scores are masked).
        f16x8 kr[2][KS];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int key = 16 * p + col;
            const uint16_t* kk = kb + (uint64_t)(key < (int)nvalid ? key : 0) * row;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kr[p][ks] = *(const f16x8*)(kk + 32 * ks + 8 * grp);
        }
        // V rows, 16 bytes a lane, consecutive lanes along a row.
        f16x8 vr[VCH];
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int c = lane + 64 * i, key = c / CPR, part = c % CPR;
            vr[i] = *(const f16x8*)(vb + (uint64_t)(key < (int)nvalid ? key : 0) * row + 8 * part);
        }

        // S^T: lane holds keys 16·p + 4·grp + r of head col.
        float sv[8];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
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
        for (int r = 1; r < 8; ++r) mx = fmaxf(mx, sv[r]);
        mx = groups_max(mx);
        const float mnew = fmaxf(m, mx);
        const float corr = fast_exp(m - mnew);
        float lsum = 0.0f;
        f16x8 pb;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const float pr = fast_exp(sv[r] - mnew);
            lsum += pr;
            pb[r] = (_Float16)pr;
        }
        l = l * corr + lsum;
        m = mnew;
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[n] *= corr;

        // Stage the value tile, then read it transposed as the A operand: lane (col, grp) takes dim
        // 16·n + col of keys 4·grp .. +4 and 16 + 4·grp .. +4 — the keys its P^T column holds.
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int c = lane + 64 * i, key = c / CPR, part = c % CPR;
            *(f16x8*)(vs + key * VP + 8 * part) = vr[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            f16x8 va;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int key = jj < 4 ? 4 * grp + jj : 16 + 4 * grp + (jj - 4);
                va[jj] = vs[key * VP + 16 * n + col];
            }
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, acc[n], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
}

template <int HD>
__global__ __launch_bounds__(256) void decode_merge(uint16_t* o, const float* part, const uint32_t* lens,
                                                    uint32_t q_heads, uint32_t chunk, uint32_t nsplit,
                                                    unsigned int* over) {
    __shared__ float wts[kMaxSplits];
    __shared__ float red[8];
    const uint32_t h = blockIdx.x, u = blockIdx.y;
    const uint32_t len = lens[u];
    uint16_t* out = o + ((uint64_t)u * q_heads + h) * HD;
    if (len == 0) {
        for (int d = threadIdx.x; d < HD; d += blockDim.x) out[d] = 0;
        return;
    }
    const uint32_t ns = (len + chunk - 1) / chunk;
    const float* pr = part + ((uint64_t)u * q_heads + h) * nsplit * (HD + 2);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;

    float mx = -INFINITY;
    for (uint32_t s = threadIdx.x; s < ns; s += blockDim.x) mx = fmaxf(mx, pr[(uint64_t)s * (HD + 2)]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float lsum = 0.0f;
    for (uint32_t s = threadIdx.x; s < ns; s += blockDim.x) {
        const float f = fast_exp(pr[(uint64_t)s * (HD + 2)] - M);
        wts[s] = f;
        lsum += f * pr[(uint64_t)s * (HD + 2) + 1];
    }
    lsum = wave_sum(lsum);
    if (lane == 0) red[4 + w] = lsum;
    __syncthreads();
    const float L = red[4] + red[5] + red[6] + red[7];
    bool hit = false;
    for (int d = threadIdx.x; d < HD; d += blockDim.x) {
        float acc = 0.0f;
        for (uint32_t s = 0; s < ns; ++s) acc += wts[s] * pr[(uint64_t)s * (HD + 2) + 2 + d];
        out[d] = to_half(acc / L, hit);
    }
    if (hit) *over = kFaultOverflow;
}

// The split length: a multiple of the 4 waves' 32-key tiles, sized so the grid is about 1024 workgroups
// over the rows' longest length, and at most kMaxSplits splits a row. SILVANN_GFX950_DECODE_CHUNK overrides.
uint32_t choose_chunk(uint64_t kv_heads, uint64_t hblocks, uint64_t most, uint64_t rows) {
    const uint64_t step = (uint64_t)kTile * kWaves;
    if (const char* e = getenv("SILVANN_GFX950_DECODE_CHUNK")) {
        const uint64_t c = strtoull(e, nullptr, 10);
        if (c >= step) {
            uint64_t cc = (c + step - 1) / step * step;
            while ((most + cc - 1) / cc > kMaxSplits) cc += step;
            return (uint32_t)cc;
        }
    }
    const uint64_t work = most * rows * kv_heads * hblocks;
    uint64_t c = (work + 1023) / 1024;
    c = (c + step - 1) / step * step;
    if (c < step) c = step;
    while ((most + c - 1) / c > kMaxSplits) c += step;
    if (c > 0xFFFFFFFFull - step) c = 0xFFFFFFFFull / step * step;
    return (uint32_t)c;
}

uint32_t head_blocks(uint64_t q_heads, uint64_t kv_heads) { return (uint32_t)((q_heads / kv_heads + 15) / 16); }

bool decode_shape_ok(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && kv_heads > 0 && q_heads % kv_heads == 0 &&
           rows > 0 && rows <= 65535 && most > 0 && most < (1ull << 31) && kv_heads * head_blocks(q_heads, kv_heads) <= 65535;
}

}  // namespace

// Launched by the door below and by the deferred scores+mix pair in doors.hip.
void decode_paged_launch(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* pages,
                         uint64_t pages_row, uint64_t page_size, uint64_t k_row, const uint32_t* lens,
                         uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows,
                         float* scratch, unsigned int* over) {
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, most, rows) || (pages && (page_size == 0 || page_size % kTile))) {
        fprintf(stderr, "silvann_gfx950: attention_decode_paged: unsupported shape (q_heads %llu kv_heads %llu "
                        "head_dim %llu most %llu rows %llu page_size %llu)\n",
                (unsigned long long)q_heads, (unsigned long long)kv_heads, (unsigned long long)head_dim,
                (unsigned long long)most, (unsigned long long)rows, (unsigned long long)page_size);
        refuse("attention_decode_paged");
        return;
    }
    DecodeArgs a;
    a.q = q; a.k = k; a.v = v; a.pages = pages; a.pages_row = pages_row; a.page_size = page_size; a.k_row = k_row;
    a.lens = lens;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hblocks = head_blocks(q_heads, kv_heads);
    a.chunk = choose_chunk(kv_heads, a.hblocks, most, rows);
    a.nsplit = (uint32_t)((most + a.chunk - 1) / a.chunk);
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.part = scratch;
    const dim3 grid(a.nsplit, (uint32_t)(kv_heads * a.hblocks), (uint32_t)rows);
    const dim3 mgrid((uint32_t)q_heads, (uint32_t)rows);
    hipStream_t st = stream();
    prof_begin(kProfDecodeSplit);
    switch (head_dim) {
        case 64: decode_split<64><<<grid, kThreads, 0, st>>>(a); break;
        case 128: decode_split<128><<<grid, kThreads, 0, st>>>(a); break;
        default: decode_split<256><<<grid, kThreads, 0, st>>>(a); break;
    }
    prof_end(kProfDecodeSplit);
    prof_begin(kProfDecodeMerge);
    switch (head_dim) {
        case 64: decode_merge<64><<<mgrid, 256, 0, st>>>(o, scratch, lens, a.q_heads, a.chunk, a.nsplit, over); break;
        case 128: decode_merge<128><<<mgrid, 256, 0, st>>>(o, scratch, lens, a.q_heads, a.chunk, a.nsplit, over); break;
        default: decode_merge<256><<<mgrid, 256, 0, st>>>(o, scratch, lens, a.q_heads, a.chunk, a.nsplit, over); break;
    }
    prof_end(kProfDecodeMerge);
    check_launch("attention_decode_paged");
}

uint64_t decode_paged_scratch(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows) {
    if (!decode_shape_ok(q_heads, kv_heads, head_dim, most, rows)) return 0;
    const uint32_t chunk = choose_chunk(kv_heads, head_blocks(q_heads, kv_heads), most, rows);
    const uint64_t nsplit = (most + chunk - 1) / chunk;
    return rows * q_heads * nsplit * (head_dim + 2) * sizeof(float);
}

}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_attention_decode_paged(uint16_t* o, const uint16_t* q, const uint16_t* k,
                                                          const uint16_t* v, const uint32_t* pages, uint64_t pages_row,
                                                          uint64_t page_size, uint64_t k_row, const uint32_t* lens,
                                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                          uint64_t most, uint64_t rows, float* scratch,
                                                          unsigned int* over) {
    silvann::decode_paged_launch(o, q, k, v, pages, pages_row, page_size, k_row, lens, q_heads, kv_heads, head_dim,
                                 most, rows, scratch, over);
}

SILVANN_EXPORT uint64_t silvann_gfx950_attention_decode_paged_scratch(uint64_t q_heads, uint64_t kv_heads,
                                                                      uint64_t head_dim, uint64_t most, uint64_t rows) {
    return silvann::decode_paged_scratch(q_heads, kv_heads, head_dim, most, rows);
}
