// prefill.hip — causal attention of a chunk of new positions over a (paged or contiguous) fp16 cache, on
// CDNA4 fp16 MFMA with fp32 accumulation: the fused form of the reference's
// `attention_causal_scores_grouped` → `attention_causal_softmax` → `attention_causal_mix`
// (kernels.cuh:1028-1081, 2051-2060), which materialise every row's weights in `p`; nothing is materialised
// here.
//
// A workgroup is 4 waves over the same rows, each a query head of one kv head's group (or, for a group not a
// multiple of 4, fewer heads over more rows). A wave owns 32 query rows of one head. Per 32-key tile:
//   S^T = K · Q^T      v_mfma_f32_32x32x16_f16: keys as M, the wave's rows as N, head dims as K. K comes
//                      from the tile staged in LDS (row layout), Q^T from registers loaded once.
//   online softmax     a lane owns one row (its column of S^T, 16 keys); the row's other 16 keys are in lane
//                      l ^ 32, one exchange away.
//   O^T += V^T · P^T   the same MFMA with keys as K: P^T is the S^T registers narrowed to fp16, V^T is the
//                      value tile staged in LDS transposed ([dim][key]), read 4 keys at a time.
// K and V tiles are double-buffered: the next tile's global loads are in flight while this tile computes.
// Causal: keys past a row's position are masked in the diagonal tiles; tiles past the workgroup's last
// row are never loaded. Workgroups are issued heaviest (latest rows) first.
#include <math.h>
#include <stdio.h>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

constexpr int kKT = 32;      // keys a tile
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

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
    float scale;
    unsigned int* over;
};

__device__ __forceinline__ const uint16_t* key_row(const uint16_t* plane, const CausalArgs& a, uint64_t t,
                                                   uint64_t row) {
    if (a.pages) return plane + ((uint64_t)a.pages[t / a.page_size] * a.page_size + t % a.page_size) * row;
    return plane + t * row;
}

template <int HD>
__global__ __launch_bounds__(kThreads) void causal_mfma(CausalArgs a) {
    constexpr int KP = HD + 8;         // LDS pitch of a key row, halves
    constexpr int VTP = kKT + 4;       // LDS pitch of a transposed value row (one dim, 32 keys), halves
    constexpr int KSTEPS = HD / 16;    // k-steps of S^T (16 dims each)
    constexpr int DT = HD / 32;        // 32-dim tiles of O^T
    constexpr int CPR = HD / 8;        // 16-byte chunks in a key row
    constexpr int CHUNKS = kKT * CPR / kThreads;  // chunks a thread stages per plane per tile
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][kKT * KP];
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][HD * VTP];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    // Heaviest first: blockIdx.x 0 takes the last row tile.
    const uint32_t rtile = a.rtiles - 1 - blockIdx.x;
    const uint32_t g = blockIdx.y / a.hblocks, hb = blockIdx.y % a.hblocks;
    const uint32_t head = g * a.group + hb * a.hw + (w % a.hw);
    const uint64_t r0 = (uint64_t)rtile * a.rt + (uint64_t)(w / a.hw) * 32;   // the wave's first row
    const uint64_t wg_r0 = (uint64_t)rtile * a.rt;
    const uint64_t wg_rlast = min(a.rows, wg_r0 + a.rt) - 1;
    const uint64_t row = (uint64_t)a.kv_heads * HD;
    const uint64_t nkeys = a.first + wg_rlast + 1;            // keys the workgroup's last row sees
    const uint32_t ntiles = (uint32_t)((nkeys + kKT - 1) / kKT);

    // Q^T as the B operand: lane (col, half) holds row r0 + col's dims 16·kk + 8·half .. +8.
    const uint64_t myrow = r0 + col;
    const bool row_ok = myrow < a.rows;
    f16x8 qb[KSTEPS];
    {
        const uint16_t* qr = a.q + ((row_ok ? myrow : 0) * a.q_heads + head) * HD;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) qb[kk] = *(const f16x8*)(qr + 16 * kk + 8 * half);
    }
    const uint64_t mypos = a.first + (row_ok ? myrow : 0);

    f32x16 acc[DT];
#pragma unroll
    for (int n = 0; n < DT; ++n) acc[n] = (f32x16)0.0f;
    float m = -INFINITY, l = 0.0f;

    // Staging: thread chunk c = tid + kThreads·i is key c / CPR, dims 8·(c % CPR) .. +8.
    f16x8 kreg[CHUNKS], vreg[CHUNKS];
    auto load_tile = [&](uint32_t t) {
        const uint64_t t0 = (uint64_t)t * kKT;
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + kThreads * i, key = c / CPR, part = c % CPR;
            uint64_t kt = t0 + key;
            if (kt >= nkeys) kt = t0;   // past the last key: any valid key (masked)
            kreg[i] = *(const f16x8*)(key_row(a.k, a, kt, row) + (uint64_t)g * HD + 8 * part);
            vreg[i] = *(const f16x8*)(key_row(a.v, a, kt, row) + (uint64_t)g * HD + 8 * part);
        }
    };
    auto store_tile = [&](int b) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = tid + kThreads * i, key = c / CPR, part = c % CPR;
            *(f16x8*)(&ks[b][key * KP + 8 * part]) = kreg[i];
            // transposed, keys swizzled in groups of 4 by the dim's 8-block so a chunk's 8 writes spread banks
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = 8 * part + e;
                const int kp = key ^ (((d >> 3) & 7) << 2);
                vt[b][d * VTP + kp] = vreg[i][e];
            }
        }
    };

    load_tile(0);
    store_tile(0);
    __syncthreads();

    for (uint32_t t = 0; t < ntiles; ++t) {
        const int b = t & 1;
        if (t + 1 < ntiles) load_tile(t + 1);
        const uint64_t t0 = (uint64_t)t * kKT;

        // S^T (32 keys × 32 rows): lane holds keys 8·(r/4) + 4·half + r%4 of row col.
        f32x16 st = (f32x16)0.0f;
        const _Float16* kb = ks[b];
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
            const f16x8 ka = *(const f16x8*)(&kb[col * KP + 16 * kk + 8 * half]);
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb[kk], st, 0, 0, 0);
        }
        float sv[16];
        float mx = -INFINITY;
        const bool diag = t0 + kKT - 1 > a.first + r0;   // some key of the tile is past some row of the wave
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint64_t key = t0 + 8 * (r / 4) + 4 * half + (r % 4);
            float x = st[r] * a.scale;
            if (diag && key > mypos) x = -INFINITY;
            sv[r] = x;
            mx = fmaxf(mx, x);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = fmaxf(m, mx);
        const float corr = fast_exp(m - mnew);
        float lsum = 0.0f;
        f16x8 pb[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = fast_exp(sv[r] - mnew);
            lsum += p;
            pb[r / 8][r % 8] = (_Float16)p;
        }
        l = l * corr + lsum;
        m = mnew;
#pragma unroll
        for (int n = 0; n < DT; ++n) acc[n] *= corr;

        // O^T (32 dims × 32 rows) per dim tile n, two k-steps of 16 keys: the A operand is V^T at dim
        // 32·n + col, keys 16·s + 8·(j/4) + 4·half + j%4 — the keys register 8·s + j of P^T holds.
        const _Float16* vb = vt[b];
#pragma unroll
        for (int n = 0; n < DT; ++n) {
            const int d = 32 * n + col;
            const int sw = ((d >> 3) & 7) << 2;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int k0 = (16 * s2 + 4 * half) ^ sw, k1 = (16 * s2 + 8 + 4 * half) ^ sw;
                const f16x4 lo = *(const f16x4*)(&vb[d * VTP + k0]);
                const f16x4 hi = *(const f16x4*)(&vb[d * VTP + k1]);
                const f16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[s2], acc[n], 0, 0, 0);
            }
        }
        if (t + 1 < ntiles) store_tile(b ^ 1);
        __syncthreads();
    }

    l += __shfl_xor(l, 32);
    if (!row_ok) return;
    const float inv_l = 1.0f / l;
    bool hit = false;
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
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.over = over;
    const dim3 grid(a.rtiles, a.kv_heads * a.hblocks);
    hipStream_t st = stream();
    prof_begin(kProfCausal);
    switch (head_dim) {
        case 64: causal_mfma<64><<<grid, kThreads, 0, st>>>(a); break;
        case 128: causal_mfma<128><<<grid, kThreads, 0, st>>>(a); break;
        default: causal_mfma<256><<<grid, kThreads, 0, st>>>(a); break;
    }
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
