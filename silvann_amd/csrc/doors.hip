// doors.hip — the reference's nn attention door rows, each with its exact signature, on gfx950.
//
// The reference splits attention into doors that hand fp32 weights `p` between them (scores → mix,
// weights → residual_mix, causal scores → softmax → mix). Every door here keeps that contract bit-for-bit in
// layout: what it writes into `p` and `res` is where and what the reference's body writes
// (kernels.cuh:885-1267, 2036-2060; doors.cuh:414-432), within fp32 rounding. Four kernels serve all 17 rows,
// each told the row geometry of its door:
//   scores_raw    a workgroup per (row, kv head, 16-head block, 256 keys); a thread per key computes the
//                 dots of all the block's query heads (held in LDS) with its key: the key is read once for the
//                 group (kernels.cuh:917-948's point), and the scaled scores go to `p`
//   softmax_rows  a workgroup per weight row: its max, e^(x - max), their sum; normalised, or left
//                 unnormalised with {m, l} into the residual (the weights doors)
//   mix_rows      a workgroup per (row, kv head, 64 dims): 4 waves split the keys, a lane a dim, every query
//                 head of the group accumulated from one read of each value; the waves meet in LDS
//   merge/finish  a thread per head / per element.
// plus the TurboQuant rows' kernels (tq_scores, tq_mix_part, tq_mix_reduce) and softmax_sink_rows.
//
// The chains' first doors are deferred (common.hpp, `Deferred`): attention_scores, attention_weights,
// attention_causal_scores_grouped, attention_scores_grouped, attention_weights_rows and the TurboQuant weights
// doors record their operands instead of launching, and their continuation runs the chain as one fused kernel
// (decode.hip, prefill.hip, tq_decode.hip) when it arrives with the same operands. Every other export here first
// runs what is recorded (flush_deferred, below) with the bodies the deferred doors run on their own. These
// kernels are then the reference's contract for every other order of calls, and for callers that read `p` or
// `res` themselves.
#include <math.h>
#include <stdio.h>

#include "common.hpp"
#include "tq_levels.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

// How a door's rows lie in its operands.
enum Mode : int {
    kSingle = 0,       // one query (scores, mix, weights, residual_mix): length, p[h·length + t]
    kCausal = 1,       // rows r at first + r (causal_*): len first+r+1, q row r·qh·hd, p (r·qh+h)·span, k/v shared
    kLens = 2,         // rows u with their own keys (*_rows of NN-115): len lens[u], q u·q_row, k/v u·k_row,
                       //   p u·p_row + h·len, o u·o_row
    kByRow = 3,        // the one-row door a row at a time (weights_rows, residual_mix_rows, doors.cuh:417-432):
                       //   len first+r+1, q row r·qh·hd, p r·qh·span + h·len, res (r·qh+h)·(hd+2)
    kTqRows = 4,       // the TurboQuant rows (weights_tq_rows, residual_mix_tq_rows, doors.cuh:433-450): every row
                       //   over the same `length` keys; q row r·qh·hd, p r·qh·len + h·len, res (r·qh+h)·(hd+2)
};

struct Geom {
    int mode;
    uint64_t length, first, span;
    uint64_t q_row, k_row, p_row, o_row;
    const uint32_t* lens;
    uint32_t q_heads, kv_heads, head_dim;
};

struct RowAt {
    uint64_t len, q, k, p, hstride, o;
};

template <int MODE>
__device__ __forceinline__ RowAt row_at(const Geom& G, uint64_t u) {
    RowAt r;
    const uint64_t qh = G.q_heads, hd = G.head_dim;
    if constexpr (MODE == kCausal) {
        r.len = G.first + u + 1; r.q = u * qh * hd; r.k = 0; r.p = u * qh * G.span; r.hstride = G.span;
        r.o = u * qh * hd;
    } else if constexpr (MODE == kLens) {
        r.len = G.lens[u]; r.q = u * G.q_row; r.k = u * G.k_row; r.p = u * G.p_row; r.hstride = r.len;
        r.o = u * G.o_row;
    } else if constexpr (MODE == kByRow) {
        r.len = G.first + u + 1; r.q = u * qh * hd; r.k = 0; r.p = u * qh * G.span; r.hstride = r.len;
        r.o = u * qh * (hd + 2);
    } else if constexpr (MODE == kTqRows) {
        r.len = G.length; r.q = u * qh * hd; r.k = 0; r.p = u * qh * G.length; r.hstride = G.length;
        r.o = u * qh * (hd + 2);
    } else {
        static_assert(MODE == kSingle, "row geometry");
        r.len = G.length; r.q = 0; r.k = 0; r.p = 0; r.hstride = G.length; r.o = 0;
    }
    return r;
}

constexpr int kHB = 16;   // query heads a block of scores_raw / mix_rows holds

// Scaled dots of a block of query heads with 256 keys; the query heads' rows in LDS as floats.
template <int MODE>
__global__ __launch_bounds__(256) void scores_raw(float* p, const uint16_t* q, const uint16_t* k, Geom G,
                                                  uint32_t hblocks, uint32_t nheads, float scale) {
    extern __shared__ float qs[];   // [nheads][head_dim]
    const uint64_t u = blockIdx.z;
    const uint32_t g = blockIdx.y / hblocks, hb = blockIdx.y % hblocks;
    const uint32_t group = G.q_heads / G.kv_heads, hd = G.head_dim;
    const uint32_t h0 = g * group + hb * nheads;
    const int nh = (int)min(nheads, group - hb * nheads);
    const RowAt R = row_at<MODE>(G, u);
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if ((uint64_t)blockIdx.x * 256 >= R.len) return;
    for (uint32_t i = threadIdx.x; i < (uint32_t)nh * hd; i += 256)
        qs[i] = half_bits_to_float(q[R.q + (uint64_t)(h0 + i / hd) * hd + i % hd]);
    __syncthreads();
    if (t >= R.len) return;
    const uint64_t row = (uint64_t)G.kv_heads * hd;
    const uint16_t* kr = k + R.k + t * row + (uint64_t)g * hd;
    float dot[kHB];
#pragma unroll
    for (int j = 0; j < kHB; ++j) dot[j] = 0.0f;
    if ((hd & 1u) == 0 && (((uintptr_t)kr) & 3u) == 0) {
        const uint32_t* k2 = (const uint32_t*)kr;
        for (uint32_t e = 0; e < hd / 2; ++e) {
            const uint32_t pair = k2[e];
            const float k0 = half_bits_to_float((uint16_t)(pair & 0xFFFFu));
            const float k1 = half_bits_to_float((uint16_t)(pair >> 16));
#pragma unroll
            for (int j = 0; j < kHB; ++j)
                if (j < nh) dot[j] += qs[j * hd + 2 * e] * k0 + qs[j * hd + 2 * e + 1] * k1;
        }
    } else {
        for (uint32_t e = 0; e < hd; ++e) {
            const float kv = half_bits_to_float(kr[e]);
#pragma unroll
            for (int j = 0; j < kHB; ++j)
                if (j < nh) dot[j] += qs[j * hd + e] * kv;
        }
    }
#pragma unroll
    for (int j = 0; j < kHB; ++j)
        if (j < nh) p[R.p + (uint64_t)(h0 + j) * R.hstride + t] = dot[j] * scale;
}

// A weight row's softmax in place. `res` non-null: unnormalised e^(x - m), {m, l} into res (the weights
// doors); else normalised by 1 / l (kernels.cuh:1085-1094).
template <int MODE>
__global__ __launch_bounds__(256) void softmax_rows(float* p, float* res, Geom G, uint64_t nrows) {
    __shared__ float red[8];
    const uint64_t i = blockIdx.x + (uint64_t)blockIdx.y * gridDim.x;
    if (i >= nrows) return;
    uint64_t len, off, roff = 0;
    const uint64_t qh = G.q_heads;
    if constexpr (MODE == kCausal) {
        len = G.first + i / qh + 1; off = i * G.span;
    } else if constexpr (MODE == kLens) {
        const uint64_t u = i / qh, h = i % qh;
        len = G.lens[u]; off = u * G.p_row + h * len;
    } else if constexpr (MODE == kByRow) {
        const uint64_t r = i / qh, h = i % qh;
        len = G.first + r + 1; off = r * qh * G.span + h * len; roff = i * (G.head_dim + 2ull);
    } else {
        static_assert(MODE == kSingle, "row geometry");
        len = G.length; off = i * G.length; roff = i * (G.head_dim + 2ull);
    }
    float* ph = p + off;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float mx = -INFINITY;
    for (uint64_t t = threadIdx.x; t < len; t += 256) mx = fmaxf(mx, ph[t]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    const float top = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float part = 0.0f;
    for (uint64_t t = threadIdx.x; t < len; t += 256) {
        const float e = expf(ph[t] - top);
        ph[t] = e;
        part += e;
    }
    part = wave_sum(part);
    if (lane == 0) red[4 + w] = part;
    __syncthreads();
    const float sum = red[4] + red[5] + red[6] + red[7];
    if (res) {
        if (threadIdx.x == 0) {
            res[roff] = top;
            res[roff + 1] = sum;
        }
        return;
    }
    const float inv = 1.0f / sum;
    for (uint64_t t = threadIdx.x; t < len; t += 256) ph[t] *= inv;
}

// Row r's softmax with a sink (kernels.cuh:1115-1131): the top over sink[r] and the row, e^(x - top), normalised by
// their sum plus e^(sink[r] - top) — weight a row may give to none of its positions. A workgroup a row.
__global__ __launch_bounds__(256) void softmax_sink_rows(float* p, const uint16_t* sink, uint64_t rows,
                                                         uint64_t length) {
    __shared__ float red[8];
    const uint64_t r = blockIdx.x + (uint64_t)blockIdx.y * gridDim.x;
    if (r >= rows) return;
    float* ph = p + r * length;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float sk = half_bits_to_float(sink[r]);
    float mx = sk;
    for (uint64_t t = threadIdx.x; t < length; t += 256) mx = fmaxf(mx, ph[t]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    const float top = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float part = 0.0f;
    for (uint64_t t = threadIdx.x; t < length; t += 256) {
        const float e = expf(ph[t] - top);
        ph[t] = e;
        part += e;
    }
    part = wave_sum(part);
    if (lane == 0) red[4 + w] = part;
    __syncthreads();
    const float inv = 1.0f / (red[4] + red[5] + red[6] + red[7] + expf(sk - top));
    for (uint64_t t = threadIdx.x; t < length; t += 256) ph[t] *= inv;
}

// o[h][d] = Σ_t p[h][t] v_t[d] for a block of query heads of one kv head and 64 dims; into fp16 `o` (with
// the overflow flag) or, `acc_out` set, into the fp32 residual's acc.
template <int MODE>
__global__ __launch_bounds__(256) void mix_rows(uint16_t* o, float* acc_out, const float* p, const uint16_t* v,
                                                Geom G, uint32_t hblocks, uint32_t dblocks, unsigned int* over) {
    __shared__ float part[4][kHB][64];
    const uint64_t u = blockIdx.z;
    const uint32_t g = blockIdx.y / hblocks, hb = blockIdx.y % hblocks;
    const uint32_t group = G.q_heads / G.kv_heads, hd = G.head_dim;
    const uint32_t h0 = g * group + hb * kHB;
    const int nh = (int)min((uint32_t)kHB, group - hb * kHB);
    const uint32_t d = (blockIdx.x % dblocks) * 64 + (threadIdx.x & 63);
    const int w = threadIdx.x >> 6;
    const RowAt R = row_at<MODE>(G, u);
    const uint64_t row = (uint64_t)G.kv_heads * hd;
    float acc[kHB];
#pragma unroll
    for (int j = 0; j < kHB; ++j) acc[j] = 0.0f;
    if (d < hd) {
        const uint16_t* vc = v + R.k + (uint64_t)g * hd + d;
        const float* pb = p + R.p + (uint64_t)h0 * R.hstride;
        for (uint64_t t = w; t < R.len; t += 4) {
            const float vv = half_bits_to_float(vc[t * row]);
#pragma unroll
            for (int j = 0; j < kHB; ++j)
                if (j < nh) acc[j] += pb[(uint64_t)j * R.hstride + t] * vv;
        }
    }
#pragma unroll
    for (int j = 0; j < kHB; ++j) part[w][j][threadIdx.x & 63] = acc[j];
    __syncthreads();
    if (w != 0 || d >= hd) return;
    bool hit = false;
    for (int j = 0; j < nh; ++j) {
        const float s = part[0][j][threadIdx.x] + part[1][j][threadIdx.x] + part[2][j][threadIdx.x] +
                        part[3][j][threadIdx.x];
        if (acc_out) {
            acc_out[R.o + (uint64_t)(h0 + j) * (hd + 2) + 2 + d] = s;
        } else {
            o[R.o + (uint64_t)(h0 + j) * hd + d] = to_half(s, hit);
        }
    }
    if (hit) *over = kFaultOverflow;
}

// kernels.cuh:1243-1255: a thread a head; a head's m and l are read before anything of it is written.
__global__ void merge_heads(float* into, const float* a, const float* b, uint64_t q_heads, uint64_t head_dim) {
    const uint64_t h = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= q_heads) return;
    const uint64_t w = head_dim + 2;
    const float ma = a[h * w], la = a[h * w + 1], mb = b[h * w], lb = b[h * w + 1];
    const float m = fmaxf(ma, mb);
    const float fa = expf(ma - m), fb = expf(mb - m);
    for (uint64_t e = 0; e < head_dim; ++e) into[h * w + 2 + e] = a[h * w + 2 + e] * fa + b[h * w + 2 + e] * fb;
    into[h * w] = m;
    into[h * w + 1] = la * fa + lb * fb;
}

// kernels.cuh:1258-1267
__global__ void finish_heads(uint16_t* o, const float* res, uint64_t q_heads, uint64_t head_dim, unsigned int* over) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= q_heads * head_dim) return;
    const uint64_t h = i / head_dim, w = head_dim + 2;
    bool hit = false;
    o[i] = to_half(res[h * w + 2 + i % head_dim] / res[h * w + 1], hit);
    if (hit) *over = kFaultOverflow;
}

Geom geom(int mode, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim) {
    Geom G = {};
    G.mode = mode;
    G.q_heads = (uint32_t)q_heads;
    G.kv_heads = (uint32_t)kv_heads;
    G.head_dim = (uint32_t)head_dim;
    return G;
}

bool heads_ok(const char* door, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t rows) {
    if (kv_heads == 0 || q_heads == 0 || head_dim == 0 || q_heads % kv_heads != 0 || head_dim > 8192 ||
        q_heads > 65535 || rows > 65535) {
        refuse(door);
        return false;
    }
    return true;
}

uint32_t dims_for(uint32_t head_dim) {
    // query heads a scores_raw block holds: 16, fewer where 16 rows of head_dim floats would pass 64 KB
    uint32_t n = kHB;
    while (n > 1 && (uint64_t)n * head_dim * 4 > 65536) n >>= 1;
    return n;
}

void launch_scores(float* p, const uint16_t* q, const uint16_t* k, const Geom& G, uint64_t rows, uint64_t most) {
    if (rows == 0 || most == 0) return;
    const uint32_t group = G.q_heads / G.kv_heads;
    const uint32_t nheads = dims_for(G.head_dim);
    const uint32_t hblocks = (group + nheads - 1) / nheads;
    const dim3 grid((uint32_t)((most + 255) / 256), G.kv_heads * hblocks, (uint32_t)rows);
    const float scale = 1.0f / sqrtf((float)G.head_dim);
    const size_t lds = nheads * G.head_dim * sizeof(float);
    hipStream_t st = stream();
    switch (G.mode) {
        case kCausal: scores_raw<kCausal><<<grid, 256, lds, st>>>(p, q, k, G, hblocks, nheads, scale); break;
        case kLens: scores_raw<kLens><<<grid, 256, lds, st>>>(p, q, k, G, hblocks, nheads, scale); break;
        case kByRow: scores_raw<kByRow><<<grid, 256, lds, st>>>(p, q, k, G, hblocks, nheads, scale); break;
        default: scores_raw<kSingle><<<grid, 256, lds, st>>>(p, q, k, G, hblocks, nheads, scale); break;
    }
}

void launch_softmax(float* p, float* res, const Geom& G, uint64_t nrows) {
    if (nrows == 0) return;
    const uint32_t x = (uint32_t)(nrows < 65535 ? nrows : 65535);
    const dim3 grid(x, (uint32_t)((nrows + x - 1) / x));
    hipStream_t st = stream();
    switch (G.mode) {
        case kCausal: softmax_rows<kCausal><<<grid, 256, 0, st>>>(p, res, G, nrows); break;
        case kLens: softmax_rows<kLens><<<grid, 256, 0, st>>>(p, res, G, nrows); break;
        case kByRow: softmax_rows<kByRow><<<grid, 256, 0, st>>>(p, res, G, nrows); break;
        default: softmax_rows<kSingle><<<grid, 256, 0, st>>>(p, res, G, nrows); break;
    }
}

void launch_mix(uint16_t* o, float* acc_out, const float* p, const uint16_t* v, const Geom& G, uint64_t rows,
                unsigned int* over) {
    if (rows == 0) return;
    const uint32_t group = G.q_heads / G.kv_heads;
    const uint32_t hblocks = (group + kHB - 1) / kHB;
    const uint32_t dblocks = (G.head_dim + 63) / 64;
    const dim3 grid(dblocks, G.kv_heads * hblocks, (uint32_t)rows);
    hipStream_t st = stream();
    switch (G.mode) {
        case kCausal: mix_rows<kCausal><<<grid, 256, 0, st>>>(o, acc_out, p, v, G, hblocks, dblocks, over); break;
        case kLens: mix_rows<kLens><<<grid, 256, 0, st>>>(o, acc_out, p, v, G, hblocks, dblocks, over); break;
        case kByRow: mix_rows<kByRow><<<grid, 256, 0, st>>>(o, acc_out, p, v, G, hblocks, dblocks, over); break;
        default: mix_rows<kSingle><<<grid, 256, 0, st>>>(o, acc_out, p, v, G, hblocks, dblocks, over); break;
    }
}


// ── TurboQuant rows: keys and values as d-bit codes, one fp16 scale a row (kernels.cuh:2957-3026) ─────
//
// A row of head_dim values is ceil(head_dim / (16 / D)) 16-bit containers, value c in container c / (16 / D)
// at bit D·(c % (16 / D)); it means kTqLevels<D>[code] (fp16) times the row's scale. Key row t of kv head g
// is row t·kv_heads + g of `codes` / `scales` (kernels.cuh:2972-2974).
//   tq_scores      a workgroup per (row, kv head, 16-head block, 256 keys); a thread per key decodes its
//                  row once for all the block's query heads (held in LDS), as scores_raw does for fp16 keys;
//                  then softmax_rows writes e^(s - m) and {m, l} (kernels.cuh:2963-3000)
//   tq_mix_part    a workgroup per (row, kv head, 16-head block, split of the keys); a wave per 64 dims, a
//                  lane per dim, every head of the block from one decode of each value; the split's sums go
//                  into the workgroup's own stretch of `p` — weights it has finished reading, which the
//                  reference hands the pass to keep its sums in (kernels.cuh:3001-3003) — or straight into
//                  the residual when there is one split
//   tq_mix_reduce  the splits' sums, in split order, into the residual's acc

// Level c of width D as fp16 bits (the tables are device read-only data; each workgroup copies its width's
// into LDS as floats).
template <int D> __device__ __forceinline__ uint16_t tq_level_bits(uint32_t c) {
    if constexpr (D == 1) return kTqLevels1[c];
    else if constexpr (D == 2) return kTqLevels2[c];
    else if constexpr (D == 3) return kTqLevels3[c];
    else if constexpr (D == 4) return kTqLevels4[c];
    else if constexpr (D == 5) return kTqLevels5[c];
    else return kTqLevels8[c];
}

constexpr uint32_t kTqSplit = 1024;   // keys a split of tq_mix_part at least (and at least head_dim: the sums' room)

template <int MODE, int D>
__global__ __launch_bounds__(256) void tq_scores(float* p, const uint16_t* q, const uint16_t* codes16,
                                                 const uint16_t* scales, Geom G, uint32_t hblocks, uint32_t nheads,
                                                 uint32_t row_units, float inv) {
    constexpr uint32_t PER = 16 / D, MASK = (1u << D) - 1u;
    extern __shared__ float qs[];   // [nheads][head_dim], then the 2^D levels
    float* lev = qs + nheads * G.head_dim;
    const uint64_t u = blockIdx.z;
    const uint32_t g = blockIdx.y / hblocks, hb = blockIdx.y % hblocks;
    const uint32_t group = G.q_heads / G.kv_heads, hd = G.head_dim;
    const uint32_t h0 = g * group + hb * nheads;
    const int nh = (int)min(nheads, group - hb * nheads);
    const RowAt R = row_at<MODE>(G, u);
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if ((uint64_t)blockIdx.x * 256 >= R.len) return;
    for (uint32_t i = threadIdx.x; i < (uint32_t)nh * hd; i += 256)
        qs[i] = half_bits_to_float(q[R.q + (uint64_t)(h0 + i / hd) * hd + i % hd]);
    for (uint32_t c = threadIdx.x; c < (1u << D); c += 256) lev[c] = half_bits_to_float(tq_level_bits<D>(c));
    __syncthreads();
    if (t >= R.len) return;
    const uint64_t krow = t * G.kv_heads + g;
    const uint16_t* kr = codes16 + krow * row_units;
    const float scale = half_bits_to_float(scales[krow]);
    float dot[kHB];
#pragma unroll
    for (int j = 0; j < kHB; ++j) dot[j] = 0.0f;
    for (uint32_t w = 0; w < row_units; ++w) {
        const uint32_t unit = kr[w];
#pragma unroll
        for (uint32_t s = 0; s < PER; ++s) {
            const uint32_t e = w * PER + s;
            if (e >= hd) break;
            const float kv = scale * lev[(unit >> (D * s)) & MASK];
#pragma unroll
            for (int j = 0; j < kHB; ++j)
                if (j < nh) dot[j] += qs[j * hd + e] * kv;
        }
    }
#pragma unroll
    for (int j = 0; j < kHB; ++j)
        if (j < nh) p[R.p + (uint64_t)(h0 + j) * R.hstride + t] = dot[j] * inv;
}

// `direct`: one split, its sums straight into the residual; else into p at the split's start (then the
// launch has head_dim <= 256: one pass of lanes holds every dim, and every lane has read its weights before
// any lane writes over them).
template <int MODE, int D>
__global__ __launch_bounds__(256) void tq_mix_part(float* res, float* p, const uint16_t* codes16,
                                                   const uint16_t* scales, Geom G, uint32_t hblocks,
                                                   uint32_t row_units, uint32_t nsplit, uint64_t split, bool direct) {
    constexpr uint32_t PER = 16 / D, MASK = (1u << D) - 1u;
    __shared__ float lev[1 << D];
    const uint64_t u = blockIdx.z;
    const uint32_t s = blockIdx.x;
    const uint32_t g = blockIdx.y / hblocks, hb = blockIdx.y % hblocks;
    const uint32_t group = G.q_heads / G.kv_heads, hd = G.head_dim;
    const uint32_t h0 = g * group + hb * kHB;
    const int nh = (int)min((uint32_t)kHB, group - hb * kHB);
    const RowAt R = row_at<MODE>(G, u);
    const uint64_t t0 = (uint64_t)s * split, t1 = s + 1 == nsplit ? R.len : t0 + split;
    for (uint32_t c = threadIdx.x; c < (1u << D); c += 256) lev[c] = half_bits_to_float(tq_level_bits<D>(c));
    __syncthreads();
    const float* pb = p + R.p + (uint64_t)h0 * R.hstride;
    for (uint32_t base = 0; base < hd; base += 256) {   // a lane a dim, 256 dims a pass
        const uint32_t d = base + threadIdx.x;
        float acc[kHB];
#pragma unroll
        for (int j = 0; j < kHB; ++j) acc[j] = 0.0f;
        if (d < hd) {
            const uint32_t wunit = d / PER, shift = D * (d % PER);
            for (uint64_t t = t0; t < t1; ++t) {
                const uint64_t vrow = t * G.kv_heads + g;
                const float vv =
                    half_bits_to_float(scales[vrow]) * lev[(codes16[vrow * row_units + wunit] >> shift) & MASK];
#pragma unroll
                for (int j = 0; j < kHB; ++j)
                    if (j < nh) acc[j] += pb[(uint64_t)j * R.hstride + t] * vv;
            }
        }
        __syncthreads();
        if (d < hd)
            for (int j = 0; j < nh; ++j) {
                if (direct) res[R.o + (uint64_t)(h0 + j) * (hd + 2) + 2 + d] = acc[j];
                else p[R.p + (uint64_t)(h0 + j) * R.hstride + t0 + d] = acc[j];
            }
    }
}

template <int MODE>
__global__ __launch_bounds__(256) void tq_mix_reduce(float* res, const float* p, Geom G, uint32_t nsplit,
                                                     uint64_t split) {
    const uint64_t u = blockIdx.z;
    const uint32_t h = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
    const uint32_t hd = G.head_dim;
    if (d >= hd) return;
    const RowAt R = row_at<MODE>(G, u);
    const float* ph = p + R.p + (uint64_t)h * R.hstride + d;
    float sum = 0.0f;
    for (uint32_t s = 0; s < nsplit; ++s) sum += ph[(uint64_t)s * split];
    res[R.o + (uint64_t)h * (hd + 2) + 2 + d] = sum;
}


bool tq_ok(const char* door, const uint8_t* codes, uint64_t head_dim, uint64_t d) {
    if (!(d == 1 || d == 2 || d == 3 || d == 4 || d == 5 || d == 8) || (((uintptr_t)codes) & 1u) != 0 || head_dim == 0) {
        refuse(door);
        return false;
    }
    return true;
}

uint32_t tq_row_units(uint64_t d, uint64_t head_dim) { return (uint32_t)((head_dim + 16 / d - 1) / (16 / d)); }

template <int MODE>
void launch_tq_scores(float* p, const uint16_t* q, const uint8_t* codes, const uint16_t* scales, const Geom& G,
                      uint64_t rows, uint64_t d) {
    if (rows == 0 || G.length == 0) return;
    const uint32_t group = G.q_heads / G.kv_heads;
    uint32_t nheads = kHB;   // query heads a block holds, with the levels, in 64 KB of LDS
    while (nheads > 1 && (uint64_t)nheads * G.head_dim * 4 + (4u << d) > 65536) nheads >>= 1;
    const uint32_t hblocks = (group + nheads - 1) / nheads;
    const dim3 grid((uint32_t)((G.length + 255) / 256), G.kv_heads * hblocks, (uint32_t)rows);
    const size_t lds = (size_t)nheads * G.head_dim * 4 + (4u << d);
    const float inv = 1.0f / sqrtf((float)(uint32_t)G.head_dim);
    const uint32_t units = tq_row_units(d, G.head_dim);
    const uint16_t* c16 = (const uint16_t*)codes;
    hipStream_t st = stream();
    switch (d) {
        case 1: tq_scores<MODE, 1><<<grid, 256, lds, st>>>(p, q, c16, scales, G, hblocks, nheads, units, inv); break;
        case 2: tq_scores<MODE, 2><<<grid, 256, lds, st>>>(p, q, c16, scales, G, hblocks, nheads, units, inv); break;
        case 3: tq_scores<MODE, 3><<<grid, 256, lds, st>>>(p, q, c16, scales, G, hblocks, nheads, units, inv); break;
        case 4: tq_scores<MODE, 4><<<grid, 256, lds, st>>>(p, q, c16, scales, G, hblocks, nheads, units, inv); break;
        case 5: tq_scores<MODE, 5><<<grid, 256, lds, st>>>(p, q, c16, scales, G, hblocks, nheads, units, inv); break;
        default: tq_scores<MODE, 8><<<grid, 256, lds, st>>>(p, q, c16, scales, G, hblocks, nheads, units, inv); break;
    }
}

template <int MODE>
void launch_tq_mix(float* res, float* p, const uint8_t* codes, const uint16_t* scales, const Geom& G, uint64_t rows,
                   uint64_t d) {
    if (rows == 0) return;
    const uint32_t group = G.q_heads / G.kv_heads;
    const uint32_t hblocks = (group + kHB - 1) / kHB;
    // splits of `split` keys, the last taking the remainder (so each has at least `split` >= head_dim keys of
    // room for its sums); at most 65535 of them. Splitting needs head_dim <= 256 (one pass of lanes).
    uint64_t split = kTqSplit;
    while (G.length / split > 65535) split *= 2;
    const uint32_t nsplit = G.head_dim <= 256 && G.length >= 2 * split ? (uint32_t)(G.length / split) : 1u;
    const bool direct = nsplit == 1;
    const dim3 grid(nsplit, G.kv_heads * hblocks, (uint32_t)rows);
    const uint32_t units = tq_row_units(d, G.head_dim);
    const uint16_t* c16 = (const uint16_t*)codes;
    hipStream_t st = stream();
    switch (d) {
        case 1: tq_mix_part<MODE, 1><<<grid, 256, 0, st>>>(res, p, c16, scales, G, hblocks, units, nsplit, split, direct); break;
        case 2: tq_mix_part<MODE, 2><<<grid, 256, 0, st>>>(res, p, c16, scales, G, hblocks, units, nsplit, split, direct); break;
        case 3: tq_mix_part<MODE, 3><<<grid, 256, 0, st>>>(res, p, c16, scales, G, hblocks, units, nsplit, split, direct); break;
        case 4: tq_mix_part<MODE, 4><<<grid, 256, 0, st>>>(res, p, c16, scales, G, hblocks, units, nsplit, split, direct); break;
        case 5: tq_mix_part<MODE, 5><<<grid, 256, 0, st>>>(res, p, c16, scales, G, hblocks, units, nsplit, split, direct); break;
        default: tq_mix_part<MODE, 8><<<grid, 256, 0, st>>>(res, p, c16, scales, G, hblocks, units, nsplit, split, direct); break;
    }
    if (!direct) {
        const dim3 rgrid((G.head_dim + 255) / 256, G.q_heads, (uint32_t)rows);
        tq_mix_reduce<MODE><<<rgrid, 256, 0, st>>>(res, p, G, nsplit, split);
    }
}
// The chain doors' bodies: what each door launches when it runs on its own (and what a flush runs).
void scores_body(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads, uint64_t kv_heads,
                 uint64_t head_dim, uint64_t length) {
    if (!heads_ok("attention_scores", q_heads, kv_heads, head_dim, 1)) return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_scores(p, q, k, G, 1, length);
    launch_softmax(p, nullptr, G, q_heads);
    check_launch("attention_scores");
}

void weights_body(float* p, float* res, const uint16_t* q, const uint16_t* k, uint64_t q_heads, uint64_t kv_heads,
                  uint64_t head_dim, uint64_t length) {
    if (!heads_ok("attention_weights", q_heads, kv_heads, head_dim, 1)) return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_scores(p, q, k, G, 1, length);
    launch_softmax(p, res, G, q_heads);
    check_launch("attention_weights");
}

void causal_scores_grouped_body(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads, uint64_t kv_heads,
                                uint64_t head_dim, uint64_t first, uint64_t rows) {
    if (!heads_ok("attention_causal_scores_grouped", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kCausal, q_heads, kv_heads, head_dim);
    G.first = first;
    G.span = first + rows;
    launch_scores(p, q, k, G, rows, first + rows);
    check_launch("attention_causal_scores_grouped");
}

void causal_softmax_body(float* p, uint64_t q_heads, uint64_t first, uint64_t rows) {
    if (q_heads == 0) return;
    Geom G = geom(kCausal, q_heads, 1, 1);
    G.first = first;
    G.span = first + rows;
    launch_softmax(p, nullptr, G, rows * q_heads);
    check_launch("attention_causal_softmax");
}

void weights_rows_body(float* p, float* res, const uint16_t* q, const uint16_t* k, uint64_t q_heads, uint64_t kv_heads,
                       uint64_t head_dim, uint64_t first, uint64_t rows) {
    if (!heads_ok("attention_weights_rows", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kByRow, q_heads, kv_heads, head_dim);
    G.first = first;
    G.span = first + rows;
    launch_scores(p, q, k, G, rows, first + rows);
    launch_softmax(p, res, G, rows * q_heads);
    check_launch("attention_weights_rows");
}

void weights_tq_body(float* p, float* res, const uint16_t* q, const uint8_t* codes, const uint16_t* scales,
                     uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length, uint64_t d) {
    if (!heads_ok("attention_weights_tq", q_heads, kv_heads, head_dim, 1) ||
        !tq_ok("attention_weights_tq", codes, head_dim, d))
        return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_tq_scores<kSingle>(p, q, codes, scales, G, 1, d);
    launch_softmax(p, res, G, q_heads);
    check_launch("attention_weights_tq");
}

void weights_tq_rows_body(float* p, float* res, const uint16_t* q, const uint8_t* codes, const uint16_t* scales,
                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length, uint64_t d,
                          uint64_t rows) {
    if (!heads_ok("attention_weights_tq_rows", q_heads, kv_heads, head_dim, rows) ||
        !tq_ok("attention_weights_tq_rows", codes, head_dim, d))
        return;
    Geom G = geom(kTqRows, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_tq_scores<kTqRows>(p, q, codes, scales, G, rows, d);
    Geom S = geom(kSingle, q_heads, kv_heads, head_dim);   // weight row i at i·length, its residual at i·(hd + 2)
    S.length = length;
    launch_softmax(p, res, S, rows * q_heads);
    check_launch("attention_weights_tq_rows");
}

void scores_grouped_body(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads, uint64_t kv_heads,
                         uint64_t head_dim, uint64_t length) {
    if (!heads_ok("attention_scores_grouped", q_heads, kv_heads, head_dim, 1)) return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_scores(p, q, k, G, 1, length);
    check_launch("attention_scores_grouped");
}

void softmax_rows_body(float* p, uint64_t rows, uint64_t length) {
    Geom G = geom(kSingle, 1, 1, 1);   // row r at r·length, `length` long: the one-query geometry
    G.length = length;
    if (length == 0) return;
    launch_softmax(p, nullptr, G, rows);
    check_launch("attention_softmax_rows");
}

void softmax_sink_body(float* p, const uint16_t* sink, uint64_t rows, uint64_t length) {
    if (rows == 0) return;
    const dim3 grid((uint32_t)(rows < 65535 ? rows : 65535), (uint32_t)((rows + 65534) / 65535));
    softmax_sink_rows<<<grid, 256, 0, stream()>>>(p, sink, rows, length);
    check_launch("attention_softmax_sink");
}

void scores_grouped_rows_body(float* p, uint64_t p_row, const uint16_t* q, uint64_t q_row, const uint16_t* k,
                              uint64_t k_row, const uint32_t* lens, uint64_t q_heads, uint64_t kv_heads,
                              uint64_t head_dim, uint64_t most, uint64_t rows) {
    if (!heads_ok("attention_scores_grouped_rows", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kLens, q_heads, kv_heads, head_dim);
    G.p_row = p_row; G.q_row = q_row; G.k_row = k_row; G.lens = lens;
    launch_scores(p, q, k, G, rows, most);
    check_launch("attention_scores_grouped_rows");
}

void softmax_lens_body(float* p, uint64_t p_row, const uint32_t* lens, uint64_t heads, uint64_t rows) {
    if (heads == 0) return;
    Geom G = geom(kLens, heads, 1, 1);
    G.p_row = p_row; G.lens = lens;
    launch_softmax(p, nullptr, G, rows * heads);
    check_launch("attention_softmax_lens");
}

// A door records its chain's first step only when a fused form could take the chain (and the shape is valid:
// an invalid one runs at once, to be refused).
bool decode_chain_shape(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512) && kv_heads > 0 &&
           q_heads > 0 && q_heads % kv_heads == 0 && length > 0 && length < (1ull << 31);
}

}  // namespace

void flush_deferred() {
    Deferred& d = deferred();
    if (d.kind == kDeferNone) return;
    const Deferred r = d;
    d = Deferred();
    switch (r.kind) {
        case kDeferScores: scores_body(r.p, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.length); break;
        case kDeferWeights: weights_body(r.p, r.res, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.length); break;
        case kDeferCausal:
            causal_scores_grouped_body(r.p, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.first, r.rows);
            break;
        case kDeferCausalSoftmax:
            causal_scores_grouped_body(r.p, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.first, r.rows);
            causal_softmax_body(r.p, r.q_heads, r.first, r.rows);
            break;
        case kDeferWeightsRows:
            weights_rows_body(r.p, r.res, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.first, r.rows);
            break;
        case kDeferWeightsTq:
            weights_tq_body(r.p, r.res, r.q, r.codes, r.scales, r.q_heads, r.kv_heads, r.head_dim, r.length, r.d);
            break;
        case kDeferGrouped: scores_grouped_body(r.p, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.length); break;
        case kDeferGroupedSoftmax:
            scores_grouped_body(r.p, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.length);
            softmax_rows_body(r.p, r.q_heads, r.length);
            break;
        case kDeferGroupedSink:
            scores_grouped_body(r.p, r.q, r.k, r.q_heads, r.kv_heads, r.head_dim, r.length);
            softmax_sink_body(r.p, r.sink, r.q_heads, r.length);
            break;
        case kDeferGroupedRows:
            scores_grouped_rows_body(r.p, r.p_row, r.q, r.q_row, r.k, r.k_row, r.lens, r.q_heads, r.kv_heads,
                                     r.head_dim, r.length, r.rows);
            break;
        case kDeferGroupedRowsSoftmax:
            scores_grouped_rows_body(r.p, r.p_row, r.q, r.q_row, r.k, r.k_row, r.lens, r.q_heads, r.kv_heads,
                                     r.head_dim, r.length, r.rows);
            softmax_lens_body(r.p, r.p_row, r.lens, r.q_heads, r.rows);
            break;
        case kDeferWeightsTqRows:
            weights_tq_rows_body(r.p, r.res, r.q, r.codes, r.scales, r.q_heads, r.kv_heads, r.head_dim, r.length, r.d,
                                 r.rows);
            break;
        default: break;
    }
}

}  // namespace silvann

using namespace silvann;

// gpu.cuh:119 — kernels.cuh:1133-1141
// Deferred when it may be a chain's first step (see common.hpp); its mix then runs the split-K decode.
SILVANN_EXPORT void silvann_gfx950_attention_scores(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                                    uint64_t kv_heads, uint64_t head_dim, uint64_t length) {
    flush_deferred();
    if (defer_enabled() && decode_chain_shape(q_heads, kv_heads, head_dim, length)) {
        Deferred& d = deferred();
        d.kind = kDeferScores; d.p = p; d.q = q; d.k = k;
        d.q_heads = q_heads; d.kv_heads = kv_heads; d.head_dim = head_dim; d.length = length; d.st = stream();
        return;
    }
    scores_body(p, q, k, q_heads, kv_heads, head_dim, length);
}

// gpu.cuh:120 — kernels.cuh:1156-1164
SILVANN_EXPORT void silvann_gfx950_attention_mix(uint16_t* o, const float* p, const uint16_t* v, uint64_t q_heads,
                                                 uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                                                 unsigned int* over) {
    Deferred& d = deferred();
    const bool chain = d.kind == kDeferScores || d.kind == kDeferGroupedSoftmax || d.kind == kDeferGroupedSink;
    if (chain && d.p == p && d.q_heads == q_heads && d.kv_heads == kv_heads && d.head_dim == head_dim &&
        d.length == length && d.st == stream() &&
        decode_one(o, nullptr, d.q, d.k, v, q_heads, kv_heads, head_dim, length, (void*)p,
                   q_heads * length * sizeof(float), over, d.kind == kDeferGroupedSink ? d.sink : nullptr)) {
        d = Deferred();   // the chain ran fused: p holds the splits' residuals, not weights
        check_launch("attention_mix");
        return;
    }
    flush_deferred();
    if (!heads_ok("attention_mix", q_heads, kv_heads, head_dim, 1)) return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_mix(o, nullptr, p, v, G, 1, over);
    check_launch("attention_mix");
}

// gpu.cuh:122 — kernels.cuh:1190-1221
// Deferred when it may be a chain's first step; its residual_mix then runs the split-K decode into `res`.
SILVANN_EXPORT void silvann_gfx950_attention_weights(float* p, float* res, const uint16_t* q, const uint16_t* k,
                                                     uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                     uint64_t length) {
    flush_deferred();
    if (defer_enabled() && decode_chain_shape(q_heads, kv_heads, head_dim, length)) {
        Deferred& d = deferred();
        d.kind = kDeferWeights; d.p = p; d.res = res; d.q = q; d.k = k;
        d.q_heads = q_heads; d.kv_heads = kv_heads; d.head_dim = head_dim; d.length = length; d.st = stream();
        return;
    }
    weights_body(p, res, q, k, q_heads, kv_heads, head_dim, length);
}

// gpu.cuh:123 — kernels.cuh:1224-1238
SILVANN_EXPORT void silvann_gfx950_attention_residual_mix(float* res, const float* p, const uint16_t* v,
                                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                          uint64_t length) {
    Deferred& d = deferred();
    if (d.kind == kDeferWeights && d.p == p && d.res == res && d.q_heads == q_heads && d.kv_heads == kv_heads &&
        d.head_dim == head_dim && d.length == length && d.st == stream() &&
        decode_one(nullptr, res, d.q, d.k, v, q_heads, kv_heads, head_dim, length, (void*)p,
                   q_heads * length * sizeof(float), nullptr)) {
        d = Deferred();
        check_launch("attention_residual_mix");
        return;
    }
    flush_deferred();
    if (!heads_ok("attention_residual_mix", q_heads, kv_heads, head_dim, 1)) return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_mix(nullptr, res, p, v, G, 1, nullptr);
    check_launch("attention_residual_mix");
}

// gpu.cuh:124 — kernels.cuh:1243-1255
SILVANN_EXPORT void silvann_gfx950_attention_merge(float* into, const float* a, const float* b, uint64_t q_heads,
                                                   uint64_t head_dim) {
    silvann::flush_deferred();
    if (q_heads == 0) return;
    merge_heads<<<(uint32_t)((q_heads + 63) / 64), 64, 0, stream()>>>(into, a, b, q_heads, head_dim);
    check_launch("attention_merge");
}

// gpu.cuh:125 — kernels.cuh:1258-1267
SILVANN_EXPORT void silvann_gfx950_attention_finish(uint16_t* o, const float* res, uint64_t q_heads,
                                                    uint64_t head_dim, unsigned int* over) {
    silvann::flush_deferred();
    const uint64_t n = q_heads * head_dim;
    if (n == 0) return;
    finish_heads<<<(uint32_t)((n + 255) / 256), 256, 0, stream()>>>(o, res, q_heads, head_dim, over);
    check_launch("attention_finish");
}

// gpu.cuh:155 — kernels.cuh:2039-2049
SILVANN_EXPORT void silvann_gfx950_attention_causal_scores(float* p, const uint16_t* q, const uint16_t* k,
                                                           uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                           uint64_t first, uint64_t rows) {
    silvann::flush_deferred();
    if (!heads_ok("attention_causal_scores", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kCausal, q_heads, kv_heads, head_dim);
    G.first = first;
    G.span = first + rows;
    launch_scores(p, q, k, G, rows, first + rows);
    launch_softmax(p, nullptr, G, rows * q_heads);
    check_launch("attention_causal_scores");
}

// gpu.cuh:156 — kernels.cuh:2051-2060
SILVANN_EXPORT void silvann_gfx950_attention_causal_mix(uint16_t* o, const float* p, const uint16_t* v,
                                                        uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                        uint64_t first, uint64_t rows, unsigned int* over) {
    Deferred& d = deferred();
    if (d.kind == kDeferCausalSoftmax && d.p == p && d.q_heads == q_heads && d.kv_heads == kv_heads &&
        d.head_dim == head_dim && d.first == first && d.rows == rows && d.st == stream()) {
        const Deferred r = d;
        if (causal_shape_ok(q_heads, kv_heads, head_dim, first, rows, false, 0) && vec_aligned(r.q, r.k, v)) {
            d = Deferred();   // the chain runs fused on the matrix cores: p is never written
            causal_paged_launch(o, nullptr, r.q, r.k, v, nullptr, 0, q_heads, kv_heads, head_dim, first, rows, over,
                                "attention_causal_mix");
            return;
        }
        // other shapes (head_dim 512): each row a decode over the same cache, p the scratch
        const uint64_t cap = rows * q_heads * (first + rows) * sizeof(float);
        if (decode_causal(o, r.q, r.k, v, q_heads, kv_heads, head_dim, first, rows, r.p, cap, over)) {
            d = Deferred();
            check_launch("attention_causal_mix");
            return;
        }
    }
    flush_deferred();
    if (!heads_ok("attention_causal_mix", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kCausal, q_heads, kv_heads, head_dim);
    G.first = first;
    G.span = first + rows;
    launch_mix(o, nullptr, p, v, G, rows, over);
    check_launch("attention_causal_mix");
}

// gpu.cuh:189 — kernels.cuh:928-948
SILVANN_EXPORT void silvann_gfx950_attention_scores_grouped(float* p, const uint16_t* q, const uint16_t* k,
                                                            uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                            uint64_t length) {
    flush_deferred();
    if (defer_enabled() && decode_chain_shape(q_heads, kv_heads, head_dim, length)) {
        Deferred& d = deferred();   // with softmax_rows or softmax_sink, then mix: the split-K decode
        d.kind = kDeferGrouped; d.p = p; d.q = q; d.k = k;
        d.q_heads = q_heads; d.kv_heads = kv_heads; d.head_dim = head_dim; d.length = length; d.st = stream();
        return;
    }
    scores_grouped_body(p, q, k, q_heads, kv_heads, head_dim, length);
}

// gpu.cuh:190 — kernels.cuh:1095-1097
SILVANN_EXPORT void silvann_gfx950_attention_softmax_rows(float* p, uint64_t rows, uint64_t length) {
    Deferred& d = deferred();
    if (d.kind == kDeferGrouped && d.p == p && d.q_heads == rows && d.length == length && d.st == stream()) {
        d.kind = kDeferGroupedSoftmax;   // the chain's second step, recorded too
        return;
    }
    flush_deferred();
    softmax_rows_body(p, rows, length);
}

// gpu.cuh:201 — kernels.cuh:1115-1131
SILVANN_EXPORT void silvann_gfx950_attention_softmax_sink(float* p, const uint16_t* sink, uint64_t rows,
                                                          uint64_t length) {
    Deferred& d = deferred();
    if (d.kind == kDeferGrouped && d.p == p && d.q_heads == rows && d.length == length && d.st == stream()) {
        d.kind = kDeferGroupedSink;   // the chain's second step, recorded with its sink
        d.sink = sink;
        return;
    }
    flush_deferred();
    softmax_sink_body(p, sink, rows, length);
}

// gpu.cuh:191 — kernels.cuh:1028-1061
// Deferred when it may be a chain's first step; its causal_softmax and causal_mix then run causal_mfma.
SILVANN_EXPORT void silvann_gfx950_attention_causal_scores_grouped(float* p, const uint16_t* q, const uint16_t* k,
                                                                   uint64_t q_heads, uint64_t kv_heads,
                                                                   uint64_t head_dim, uint64_t first, uint64_t rows) {
    flush_deferred();
    if (defer_enabled() && (causal_shape_ok(q_heads, kv_heads, head_dim, first, rows, false, 0) ||
                            (decode_chain_shape(q_heads, kv_heads, head_dim, first + rows) && rows <= 65535))) {
        Deferred& d = deferred();
        d.kind = kDeferCausal; d.p = p; d.q = q; d.k = k;
        d.q_heads = q_heads; d.kv_heads = kv_heads; d.head_dim = head_dim; d.first = first; d.rows = rows;
        d.st = stream();
        return;
    }
    causal_scores_grouped_body(p, q, k, q_heads, kv_heads, head_dim, first, rows);
}

// gpu.cuh:192 — kernels.cuh:1065-1081
SILVANN_EXPORT void silvann_gfx950_attention_causal_softmax(float* p, uint64_t q_heads, uint64_t first, uint64_t rows) {
    Deferred& d = deferred();
    if (d.kind == kDeferCausal && d.p == p && d.q_heads == q_heads && d.first == first && d.rows == rows &&
        d.st == stream()) {
        d.kind = kDeferCausalSoftmax;   // the chain's second step, recorded too
        return;
    }
    flush_deferred();
    causal_softmax_body(p, q_heads, first, rows);
}

// gpu.cuh:195 — doors.cuh:417-424
SILVANN_EXPORT void silvann_gfx950_attention_weights_rows(float* p, float* res, const uint16_t* q, const uint16_t* k,
                                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                          uint64_t first, uint64_t rows) {
    flush_deferred();
    if (defer_enabled() && causal_shape_ok(q_heads, kv_heads, head_dim, first, rows, false, 0)) {
        Deferred& d = deferred();   // with its residual_mix_rows: the causal residual (row 140)
        d.kind = kDeferWeightsRows; d.p = p; d.res = res; d.q = q; d.k = k;
        d.q_heads = q_heads; d.kv_heads = kv_heads; d.head_dim = head_dim; d.first = first; d.rows = rows;
        d.st = stream();
        return;
    }
    weights_rows_body(p, res, q, k, q_heads, kv_heads, head_dim, first, rows);
}

// gpu.cuh:196 — doors.cuh:425-432
SILVANN_EXPORT void silvann_gfx950_attention_residual_mix_rows(float* res, const float* p, const uint16_t* v,
                                                               uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                               uint64_t first, uint64_t rows) {
    Deferred& d = deferred();
    if (d.kind == kDeferWeightsRows && d.p == p && d.res == res && d.q_heads == q_heads && d.kv_heads == kv_heads &&
        d.head_dim == head_dim && d.first == first && d.rows == rows && d.st == stream() && vec_aligned(d.q, d.k, v)) {
        const Deferred r = d;
        d = Deferred();   // the pair runs fused: p is never written
        causal_paged_launch(nullptr, res, r.q, r.k, v, nullptr, 0, q_heads, kv_heads, head_dim, first, rows, nullptr,
                            "attention_residual_mix_rows");
        return;
    }
    flush_deferred();
    if (!heads_ok("attention_residual_mix_rows", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kByRow, q_heads, kv_heads, head_dim);
    G.first = first;
    G.span = first + rows;
    launch_mix(nullptr, res, p, v, G, rows, nullptr);
    check_launch("attention_residual_mix_rows");
}

// gpu.cuh:222 — kernels.cuh:953-972
SILVANN_EXPORT void silvann_gfx950_attention_scores_grouped_rows(float* p, uint64_t p_row, const uint16_t* q,
                                                                 uint64_t q_row, const uint16_t* k, uint64_t k_row,
                                                                 const uint32_t* lens, uint64_t q_heads,
                                                                 uint64_t kv_heads, uint64_t head_dim, uint64_t most,
                                                                 uint64_t rows) {
    flush_deferred();
    if (defer_enabled() && decode_chain_shape(q_heads, kv_heads, head_dim, most) && rows > 0 && rows <= 65535 &&
        q_row == q_heads * head_dim) {
        Deferred& d = deferred();   // with softmax_lens and mix_rows: the split-K decode of every row
        d.kind = kDeferGroupedRows; d.p = p; d.p_row = p_row; d.q = q; d.q_row = q_row; d.k = k; d.k_row = k_row;
        d.lens = lens; d.q_heads = q_heads; d.kv_heads = kv_heads; d.head_dim = head_dim; d.length = most;
        d.rows = rows; d.st = stream();
        return;
    }
    scores_grouped_rows_body(p, p_row, q, q_row, k, k_row, lens, q_heads, kv_heads, head_dim, most, rows);
}

// gpu.cuh:223 — kernels.cuh:1104-1110
SILVANN_EXPORT void silvann_gfx950_attention_softmax_lens(float* p, uint64_t p_row, const uint32_t* lens,
                                                          uint64_t heads, uint64_t rows) {
    Deferred& d = deferred();
    if (d.kind == kDeferGroupedRows && d.p == p && d.p_row == p_row && d.lens == lens && d.q_heads == heads &&
        d.rows == rows && d.st == stream()) {
        d.kind = kDeferGroupedRowsSoftmax;   // the chain's second step, recorded too
        return;
    }
    flush_deferred();
    softmax_lens_body(p, p_row, lens, heads, rows);
}

// gpu.cuh:224 — kernels.cuh:1169-1178
SILVANN_EXPORT void silvann_gfx950_attention_mix_rows(uint16_t* o, uint64_t o_row, const float* p, uint64_t p_row,
                                                      const uint16_t* v, uint64_t v_row, const uint32_t* lens,
                                                      uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                      uint64_t rows, unsigned int* over) {
    Deferred& d = deferred();
    if (d.kind == kDeferGroupedRowsSoftmax && d.p == p && d.p_row == p_row && d.lens == lens &&
        d.q_heads == q_heads && d.kv_heads == kv_heads && d.head_dim == head_dim && d.rows == rows &&
        o_row == q_heads * head_dim && v_row == d.k_row && d.st == stream() &&
        decode_rows_fit(o, d.q, d.k, v, lens, d.k_row, q_heads, kv_heads, head_dim, d.length, rows,
                        const_cast<float*>(p), rows * p_row * sizeof(float), over)) {
        d = Deferred();   // the chain ran fused: p holds the splits' residuals, not weights
        check_launch("attention_mix_rows");
        return;
    }
    flush_deferred();
    if (!heads_ok("attention_mix_rows", q_heads, kv_heads, head_dim, rows)) return;
    Geom G = geom(kLens, q_heads, kv_heads, head_dim);
    G.p_row = p_row; G.k_row = v_row; G.o_row = o_row; G.lens = lens;
    launch_mix(o, nullptr, p, v, G, rows, over);
    check_launch("attention_mix_rows");
}

// gpu.cuh:163 attention_weights_tq — kernels.cuh:2963-3000: e^(s - m) unnormalised into p, {m, l} into res
SILVANN_EXPORT void silvann_gfx950_attention_weights_tq(float* p, float* res, const uint16_t* q, const uint8_t* codes,
                                                        const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads,
                                                        uint64_t head_dim, uint64_t length, uint64_t d) {
    flush_deferred();
    if (defer_enabled() && (d == 4 || d == 8)) {
        Deferred& r = deferred();   // with its residual_mix_tq: the fused TurboQuant residual (row 139)
        r.kind = kDeferWeightsTq; r.p = p; r.res = res; r.q = q; r.codes = codes; r.scales = scales;
        r.q_heads = q_heads; r.kv_heads = kv_heads; r.head_dim = head_dim; r.length = length; r.d = d; r.rows = 1;
        r.st = stream();
        return;
    }
    weights_tq_body(p, res, q, codes, scales, q_heads, kv_heads, head_dim, length, d);
}

// gpu.cuh:164 attention_residual_mix_tq — kernels.cuh:3005-3026. The weights are the pass's once read: its
// splits keep their sums in p (kernels.cuh:3001-3003), so p holds no weights after it.
SILVANN_EXPORT void silvann_gfx950_attention_residual_mix_tq(float* res, const float* p, const uint8_t* codes,
                                                             const uint16_t* scales, uint64_t q_heads,
                                                             uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                                                             uint64_t d) {
    Deferred& r = deferred();
    if (r.kind == kDeferWeightsTq && r.p == p && r.res == res && r.q_heads == q_heads && r.kv_heads == kv_heads &&
        r.head_dim == head_dim && r.length == length && r.d == d && r.st == stream() &&
        residual_tq_fit(res, r.q, r.codes, r.scales, codes, scales, q_heads, kv_heads, head_dim, length, d, 1,
                        const_cast<float*>(p), q_heads * length * sizeof(float))) {
        r = Deferred();   // the pair ran fused: p holds the splits' residuals, not weights
        return;
    }
    flush_deferred();
    if (!heads_ok("attention_residual_mix_tq", q_heads, kv_heads, head_dim, 1) ||
        !tq_ok("attention_residual_mix_tq", codes, head_dim, d))
        return;
    Geom G = geom(kSingle, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_tq_mix<kSingle>(res, const_cast<float*>(p), codes, scales, G, 1, d);
    check_launch("attention_residual_mix_tq");
}

// gpu.cuh:197 attention_weights_tq_rows — doors.cuh:203,433-441: weights_tq a row at a time, in one launch
SILVANN_EXPORT void silvann_gfx950_attention_weights_tq_rows(float* p, float* res, const uint16_t* q,
                                                             const uint8_t* codes, const uint16_t* scales,
                                                             uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                             uint64_t length, uint64_t d, uint64_t rows) {
    flush_deferred();
    if (defer_enabled() && (d == 4 || d == 8)) {
        Deferred& r = deferred();   // with its residual_mix_tq_rows: row 139 over all the rows
        r.kind = kDeferWeightsTqRows; r.p = p; r.res = res; r.q = q; r.codes = codes; r.scales = scales;
        r.q_heads = q_heads; r.kv_heads = kv_heads; r.head_dim = head_dim; r.length = length; r.d = d; r.rows = rows;
        r.st = stream();
        return;
    }
    weights_tq_rows_body(p, res, q, codes, scales, q_heads, kv_heads, head_dim, length, d, rows);
}

// gpu.cuh:198 attention_residual_mix_tq_rows — doors.cuh:204,442-450
SILVANN_EXPORT void silvann_gfx950_attention_residual_mix_tq_rows(float* res, const float* p, const uint8_t* codes,
                                                                  const uint16_t* scales, uint64_t q_heads,
                                                                  uint64_t kv_heads, uint64_t head_dim,
                                                                  uint64_t length, uint64_t d, uint64_t rows) {
    Deferred& r = deferred();
    if (r.kind == kDeferWeightsTqRows && r.p == p && r.res == res && r.q_heads == q_heads && r.kv_heads == kv_heads &&
        r.head_dim == head_dim && r.length == length && r.d == d && r.rows == rows && r.st == stream() &&
        residual_tq_fit(res, r.q, r.codes, r.scales, codes, scales, q_heads, kv_heads, head_dim, length, d, rows,
                        const_cast<float*>(p), rows * q_heads * length * sizeof(float))) {
        r = Deferred();
        return;
    }
    flush_deferred();
    if (!heads_ok("attention_residual_mix_tq_rows", q_heads, kv_heads, head_dim, rows) ||
        !tq_ok("attention_residual_mix_tq_rows", codes, head_dim, d))
        return;
    Geom G = geom(kTqRows, q_heads, kv_heads, head_dim);
    G.length = length;
    launch_tq_mix<kTqRows>(res, const_cast<float*>(p), codes, scales, G, rows, d);
    check_launch("attention_residual_mix_tq_rows");
}
