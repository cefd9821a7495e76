// tq_decode.hip — split-K attention over TurboQuant keys and values on CDNA4 fp16 MFMA: the fused form of
// `attention_weights_tq` + `attention_residual_mix_tq` (kernels.cuh:2963-3026), which materialise every
// weight in `p`. Each code is read once; the answer is the same residual {m, l, acc} a query head, so a
// tier's residual joins the others through `attention_merge` as the tiers' verbs do (mixer__abi.cuh:392-412).
//
// A row is ceil(head_dim / (16/D)) 16-bit containers, value c at bit D·(c % (16/D)) of container c / (16/D),
// meaning kTqLevels<D>[code] · the row's fp16 scale (kernels.cuh:2957-2961). Key row t of kv head g is row
// t·kv_heads + g of the codes and scales (kernels.cuh:2972-2974).
//
//   pass 1  tq_split: one workgroup of 4 waves a work item — (query row, split of `chunk` keys, kv head, block
//           of up to 16 query heads). Each wave walks tiles of TK keys (TK = 8192 / head_dim):
//             K         decoded straight into the MFMA A operand: lane (col, grp) takes key 16·p + col, dims
//                       32·ks + 8·grp .. +8 — eight consecutive codes, one 32-bit (D = 4) or 64-bit (D = 8)
//                       load — through the levels held in LDS, times the row's scale, to fp16
//             S^T       v_mfma_f32_16x16x32_f16, keys as M, the block's query heads as N
//             softmax   online, in registers, as decode_split does
//             V         decoded into the wave's LDS tile (fp16, rows swizzled in 16-byte chunks), then read
//                       with the transposing LDS read as the A operand of O^T += V^T · P^T
//           then the four waves' (m, l, O) merge in LDS and the split's residual goes to the scratch.
//   pass 2  tq_merge: a workgroup per (query row, query head, 64 dims) merges the splits exactly
//           (kernels.cuh:1243-1255) into the residual res[h] = {m, l, acc}.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "common.hpp"
#include "tq_levels.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kMaxSplits = 65536;
// Workgroups one launch of tq_split may have: its item index and the grid's thread count stay 32-bit.
constexpr uint64_t kMaxGroups = (1ull << 32) / kThreads - 1;

struct TqArgs {
    const uint16_t* q;
    const uint8_t* kc;
    const uint16_t* ks;
    const uint8_t* vc;
    const uint16_t* vs;
    uint32_t q_heads, kv_heads, group, hblocks;
    uint32_t length, chunk, nsplit, rows;
    uint32_t row_bytes;
    float scale;
    float* part;   // [row][q head][split][head_dim + 2]
};

template <int D> __device__ __forceinline__ uint16_t level_bits(uint32_t c) {
    if constexpr (D == 4) return kTqLevels4[c];
    else return kTqLevels8[c];
}

// Keys a wave takes a step: a decoded 16 KB value tile at every head width.
constexpr int tile_keys(int hd) { return 8192 / hd; }
__device__ __forceinline__ int vslot(int key, int chunk) { return chunk ^ (((key >> 2) & 3) << 1); }

// Eight consecutive codes of a row from value `c0` (a multiple of 8): D = 4 two containers, D = 8 four.
template <int D> __device__ __forceinline__ uint64_t codes8(const uint8_t* row, uint32_t c0) {
    if constexpr (D == 4) return *(const uint32_t*)(row + c0 / 2);
    else return *(const uint64_t*)(row + c0);
}

// Eight values from their codes: level × the row's scale, rounded once to fp16. D = 8: a level (fp32, from the fp16
// table) a code. D = 4: a byte of two codes is one read of `lev2`, its two levels as fp16 pair, scaled with one packed
// fp16 multiply — the same bits, since a product of two fp16 values is exact in fp32 before its one rounding.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <int D> __device__ __forceinline__ f16x8 decode8(uint64_t bits, float scale, const float* lev,
                                                          const uint32_t* lev2) {
    f16x8 x;
    if constexpr (D == 4) {
        const _Float16 sh = (_Float16)scale;   // exact: the scale is an fp16 value
        const f16x2 s2 = {sh, sh};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const f16x2 v = __builtin_bit_cast(f16x2, lev2[(bits >> (8 * b)) & 0xFFu]) * s2;
            x[2 * b] = v[0];
            x[2 * b + 1] = v[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = (_Float16)(scale * lev[(bits >> (D * i)) & ((1u << D) - 1u)]);
    }
    return x;
}

template <int HD, int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void tq_split(TqArgs a) {
    constexpr int TK = tile_keys(HD);
    constexpr int MT = TK / 16;       // 16-key M tiles of S^T
    constexpr int KS = HD / 32;       // k-steps of S^T
    constexpr int NT = HD / 16;       // d-tiles of O^T
    constexpr int CPR = HD / 8;       // 16-byte chunks in a decoded value row
    constexpr int VCH = TK * CPR / 64;   // value chunks a lane decodes a tile
    constexpr int kStageBytes = kWaves * TK * HD * 2;
    constexpr int kMergeBytes = kWaves * 16 * HD * 4 + 2 * kWaves * 16 * 4;
    constexpr int kSmem = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSmem];
    __shared__ float lev[1 << D];
    __shared__ uint32_t lev2[D == 4 ? 256 : 1];   // D = 4: byte b's two levels, low nibble's in the low half

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const uint32_t GH = a.kv_heads * a.hblocks;
    const uint32_t item = blockIdx.x;
    const uint32_t u = item / (a.nsplit * GH), rest = item % (a.nsplit * GH);
    const uint32_t s = rest / GH, gh = rest % GH;
    const uint32_t g = gh / a.hblocks, hb = gh % a.hblocks;
    const uint32_t start = s * a.chunk, end = min(a.length, start + a.chunk);
    const uint32_t h0 = g * a.group + hb * 16;
    const int nh = min(16, (int)(a.group - hb * 16));

    for (uint32_t c = threadIdx.x; c < (1u << D); c += kThreads) lev[c] = half_bits_to_float(level_bits<D>(c));
    if constexpr (D == 4)
        for (uint32_t b = threadIdx.x; b < 256; b += kThreads)
            lev2[b] = (uint32_t)level_bits<4>(b & 15u) | ((uint32_t)level_bits<4>(b >> 4) << 16);

    f16x8 qb[KS];
    {
        const uint16_t* qh = a.q + ((uint64_t)u * a.q_heads + h0 + (col < nh ? col : 0)) * HD;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            f16x8 x = *(const f16x8*)(qh + 32 * ks + 8 * grp);
            qb[ks] = col < nh ? x : (f16x8)0;
        }
    }
    __syncthreads();   // the levels are in LDS

    float m = -INFINITY, l = 0.0f;
    f32x4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = (f32x4)0.0f;
    _Float16* vt = (_Float16*)smem + w * TK * HD;
    const uint32_t ntiles = (end - start + TK - 1) / TK;
    const uint64_t rb = a.row_bytes;

    for (uint32_t j = w; j < ntiles; j += kWaves) {
        const uint32_t t0 = start + j * TK;
        const uint32_t nvalid = min((uint32_t)TK, end - t0);
        // K codes as the A operand's source; keys past the split read key t0 (their scores are masked). The codes
        // are held raw (a 32- or 64-bit word a k-step) and decoded one 16-key M tile at a time, just before its
        // MFMAs, so the decoded fp16 operands of only one M tile are live at once.
        uint64_t kcodes[MT][KS];
        float kscale[MT];
#pragma unroll
        for (int p = 0; p < MT; ++p) {
            const int key = 16 * p + col;
            const uint64_t krow = (uint64_t)(t0 + (key < (int)nvalid ? key : 0)) * a.kv_heads + g;
            const uint8_t* row = a.kc + krow * rb;
            kscale[p] = half_bits_to_float(a.ks[krow]);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kcodes[p][ks] = codes8<D>(row, 32 * ks + 8 * grp);
        }
        // V decoded into the wave's tile: slot (key, c) holds chunk c ^ f(key) of the key's row; keys past the
        // split bring key t0 (weight 0)
#pragma unroll
        for (int i = 0; i < VCH; ++i) {
            const int slot = lane + 64 * i, key = slot / CPR, c = slot % CPR;
            const uint64_t vrow = (uint64_t)(t0 + (key < (int)nvalid ? key : 0)) * a.kv_heads + g;
            const f16x8 x = decode8<D>(codes8<D>(a.vc + vrow * rb, 8 * c), half_bits_to_float(a.vs[vrow]), lev, lev2);
            *(f16x8*)(vt + (key * CPR + vslot(key, c)) * 8) = x;
        }

        float sv[MT * 4];
#pragma unroll
        for (int p = 0; p < MT; ++p) {
            f32x4 st = (f32x4)0.0f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                st = __builtin_amdgcn_mfma_f32_16x16x32_f16(decode8<D>(kcodes[p][ks], kscale[p], lev, lev2), qb[ks], st, 0, 0, 0);
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

        __builtin_amdgcn_wave_barrier();   // the wave's decoded values are in its tile
#pragma unroll
        for (int sp = 0; sp < MT / 2; ++sp)
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                // V^T as the A operand through the transposing read: lane 4·jj + rr of 16-lane block grp points at
                // key 32·sp + 4·grp + jj (+ 16), dims 16·n + 4·rr .. +3; lane col of the block gets dim 16·n + col
                // of its four keys
                const int li = lane & 15, jj = li >> 2, d0 = 16 * n + 4 * (li & 3);
                const int k0 = 32 * sp + 4 * grp + jj, k1 = k0 + 16;
                typedef short s16x4 __attribute__((ext_vector_type(4)));
                const s16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(vt + (k0 * CPR + vslot(k0, d0 >> 3)) * 8 + (d0 & 7)));
                const s16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4*)(vt + (k1 * CPR + vslot(k1, d0 >> 3)) * 8 + (d0 & 7)));
                const f16x8 va = __builtin_bit_cast(f16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[sp], acc[n], 0, 0, 0);
            }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this tile's reads are done before the next overwrites it
        __builtin_amdgcn_wave_barrier();
    }
    l = groups_sum(l);

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
        if (mm != -INFINITY) {
#pragma unroll
            for (int ww = 0; ww < kWaves; ++ww) {
                const float f = fast_exp(ms[ww * 16 + hh] - mm);
                sum += os[(ww * 16 + hh) * HD + d] * f;
                lsum += ls[ww * 16 + hh] * f;
            }
        }
        float* pr = a.part + (((uint64_t)u * a.q_heads + h0 + hh) * a.nsplit + s) * (HD + 2);
        pr[2 + d] = sum;
        if (d == 0) {
            pr[0] = mm;
            pr[1] = lsum;
        }
    }
}

// A workgroup per (query row, query head, 64 dims): the splits' residuals merged exactly, each by e^(m_s - M)
// (kernels.cuh:1243-1255), into res = {M, l, acc}.
template <int HD>
__global__ __launch_bounds__(256) void tq_merge(float* res, const float* part, uint32_t q_heads, uint32_t nsplit) {
    __shared__ float red[4];
    __shared__ float accs[4][64];
    __shared__ float lss[4];
    const uint32_t h = blockIdx.x, u = blockIdx.y;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int d = blockIdx.z * 64 + lane;
    const float* pr = part + ((uint64_t)u * q_heads + h) * nsplit * (HD + 2);
    float* out = res + ((uint64_t)u * q_heads + h) * (HD + 2);
    float mx = -INFINITY;
    for (uint32_t s = threadIdx.x; s < nsplit; s += 256) mx = fmaxf(mx, pr[(uint64_t)s * (HD + 2)]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float acc = 0.0f, lsum = 0.0f;
    if (M != -INFINITY)
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

uint32_t tq_hblocks(uint64_t q_heads, uint64_t kv_heads) { return (uint32_t)((q_heads / kv_heads + 15) / 16); }

bool tq_shape_ok(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length, uint64_t d, uint64_t rows) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && (d == 4 || d == 8) && kv_heads > 0 &&
           q_heads > 0 && q_heads % kv_heads == 0 && length < (1ull << 31) && rows > 0 && rows <= 65535 &&
           kv_heads * tq_hblocks(q_heads, kv_heads) <= 65535;
}

// The split length: a multiple of the 4 waves' tiles, sized so the items about fill the chip (two workgroups
// a CU on 256 CUs), at most 1024 keys.
uint32_t tq_chunk(uint64_t head_dim, uint64_t kv_heads, uint64_t hblocks, uint64_t length, uint64_t rows) {
    const uint64_t step = (uint64_t)tile_keys((int)head_dim) * kWaves;
    const uint64_t groups = 512;
    uint64_t c = (length * rows * kv_heads * hblocks + groups - 1) / groups;
    if (c > 1024) c = 1024;
    c = (c + step - 1) / step * step;
    if (c < step) c = step;
    while ((length + c - 1) / c > kMaxSplits) c += step;
    return (uint32_t)c;
}

}  // namespace

uint64_t residual_tq_scratch(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length, uint64_t d,
                             uint64_t rows) {
    if (!tq_shape_ok(q_heads, kv_heads, head_dim, length, d, rows)) return 0;
    const uint32_t chunk = tq_chunk(head_dim, kv_heads, tq_hblocks(q_heads, kv_heads), length, rows);
    const uint64_t nsplit = length == 0 ? 0 : (length + chunk - 1) / chunk;
    return rows * q_heads * (nsplit > 0 ? nsplit : 1) * (head_dim + 2) * sizeof(float);
}

// The launch with a given split length (a multiple of the waves' tiles).
void residual_tq_run(float* res, const uint16_t* q, const uint8_t* kc, const uint16_t* ks, const uint8_t* vc,
                     const uint16_t* vs, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                     uint64_t d, uint64_t rows, float* scratch, uint32_t chunk) {
    TqArgs a;
    a.q = q; a.kc = kc; a.ks = ks; a.vc = vc; a.vs = vs;
    a.q_heads = (uint32_t)q_heads; a.kv_heads = (uint32_t)kv_heads; a.group = (uint32_t)(q_heads / kv_heads);
    a.hblocks = tq_hblocks(q_heads, kv_heads);
    a.length = (uint32_t)length; a.rows = (uint32_t)rows;
    a.chunk = chunk;
    a.nsplit = (uint32_t)((length + a.chunk - 1) / a.chunk);
    a.row_bytes = (uint32_t)((head_dim + 16 / d - 1) / (16 / d) * 2);
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.part = scratch;
    hipStream_t st = stream();
    const dim3 mgrid((uint32_t)q_heads, (uint32_t)rows, (uint32_t)(head_dim / 64));
    prof_begin(kProfTqSplit);
    if (a.nsplit > 0) {
        const dim3 grid(a.nsplit * a.kv_heads * a.hblocks * a.rows);
#define SILVANN_TQ(HDV, DV) \
        if (head_dim == HDV && d == DV) tq_split<HDV, DV><<<grid, kThreads, 0, st>>>(a);
        SILVANN_TQ(64, 4) SILVANN_TQ(64, 8) SILVANN_TQ(128, 4) SILVANN_TQ(128, 8) SILVANN_TQ(256, 4) SILVANN_TQ(256, 8)
#undef SILVANN_TQ
    }
    prof_end(kProfTqSplit);
    switch (head_dim) {
        case 64: tq_merge<64><<<mgrid, 256, 0, st>>>(res, scratch, a.q_heads, a.nsplit); break;
        case 128: tq_merge<128><<<mgrid, 256, 0, st>>>(res, scratch, a.q_heads, a.nsplit); break;
        default: tq_merge<256><<<mgrid, 256, 0, st>>>(res, scratch, a.q_heads, a.nsplit); break;
    }
    check_launch("attention_residual_tq");
}

void residual_tq_launch(float* res, const uint16_t* q, const uint8_t* kc, const uint16_t* ks, const uint8_t* vc,
                        const uint16_t* vs, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                        uint64_t d, uint64_t rows, float* scratch) {
    if (!tq_shape_ok(q_heads, kv_heads, head_dim, length, d, rows) || (((uintptr_t)kc | (uintptr_t)vc) & 7u) != 0 ||
        (((uintptr_t)q) & 15u) != 0) {
        refuse("attention_residual_tq");
        return;
    }
    const uint32_t chunk = tq_chunk(head_dim, kv_heads, tq_hblocks(q_heads, kv_heads), length, rows);
    if ((length + chunk - 1) / chunk * kv_heads * tq_hblocks(q_heads, kv_heads) * rows > kMaxGroups) {
        refuse("attention_residual_tq");
        return;
    }
    residual_tq_run(res, q, kc, ks, vc, vs, q_heads, kv_heads, head_dim, length, d, rows, scratch, chunk);
}

// The deferred TurboQuant pairs' fused form: weights_tq(_rows) + residual_mix_tq(_rows) as row 139, its scratch the
// pair's own weights buffer (`cap` bytes), the splits made long enough for their residuals to fit it. Answers false,
// launching nothing, when the operands are not ones row 139 takes or no split length fits.
bool residual_tq_fit(float* res, const uint16_t* q, const uint8_t* kc, const uint16_t* ks, const uint8_t* vc,
                     const uint16_t* vs, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                     uint64_t d, uint64_t rows, void* scratch, uint64_t cap) {
    if (!tq_shape_ok(q_heads, kv_heads, head_dim, length, d, rows) || length == 0 ||
        (((uintptr_t)kc | (uintptr_t)vc) & 7u) != 0 || (((uintptr_t)q) & 15u) != 0 ||
        !scratch_aligned(scratch))
        return false;
    const uint64_t per_split = rows * q_heads * (head_dim + 2) * sizeof(float);
    const uint64_t fit = cap / per_split;
    if (fit == 0) return false;
    const uint32_t hb = tq_hblocks(q_heads, kv_heads);
    const uint64_t step = (uint64_t)tile_keys((int)head_dim) * kWaves;
    uint64_t chunk = tq_chunk(head_dim, kv_heads, hb, length, rows);
    if ((length + chunk - 1) / chunk > fit) chunk = ((length + fit - 1) / fit + step - 1) / step * step;
    const uint64_t nsplit = (length + chunk - 1) / chunk;
    if (nsplit > fit || nsplit > kMaxSplits || nsplit * kv_heads * hb * rows > kMaxGroups) return false;
    residual_tq_run(res, q, kc, ks, vc, vs, q_heads, kv_heads, head_dim, length, d, rows, (float*)scratch,
                    (uint32_t)chunk);
    return true;
}

}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_attention_residual_tq(float* res, const uint16_t* q, const uint8_t* k_codes,
                                                         const uint16_t* k_scales, const uint8_t* v_codes,
                                                         const uint16_t* v_scales, uint64_t q_heads,
                                                         uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                                                         uint64_t d, uint64_t rows, float* scratch) {
    silvann::flush_deferred();
    silvann::residual_tq_launch(res, q, k_codes, k_scales, v_codes, v_scales, q_heads, kv_heads, head_dim, length, d,
                                rows, scratch);
}

SILVANN_EXPORT uint64_t silvann_gfx950_attention_residual_tq_scratch(uint64_t q_heads, uint64_t kv_heads,
                                                                     uint64_t head_dim, uint64_t length, uint64_t d,
                                                                     uint64_t rows) {
    return silvann::residual_tq_scratch(q_heads, kv_heads, head_dim, length, d, rows);
}
