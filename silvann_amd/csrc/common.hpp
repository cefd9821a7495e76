// common.hpp — what every kernel file of the gfx950 attention library shares: the fp16 vector types the
// MFMA builtins take, the fault word, the wave-level folds, and the launch bookkeeping (stream and the
// remembered launch failure).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SILVANN_EXPORT extern "C" __attribute__((visibility("default")))

namespace silvann {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The fault a door stores when an fp16 answer overflows: "NPOV" (reference
// packages/nn/contracts/objects/primitives.cuh:57, kernels.cuh:29-40).
constexpr unsigned int kFaultOverflow = 0x4E504F56u;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// fp32 -> fp16 with round-to-nearest-even, subnormals kept: the hardware conversion gives the bits of the
// reference's hand-written one (kernels.cuh:2763-2808) for every finite input. A finite input whose answer
// is infinite overflowed — past 65504 or carried there by the rounding — and is flagged; an input that was
// already inf or NaN passes through unflagged, as the reference does.
__device__ __forceinline__ uint16_t to_half(float f, bool& hit) {
    _Float16 h = (_Float16)f;
    uint16_t b = __builtin_bit_cast(uint16_t, h);
    if ((b & 0x7FFFu) == 0x7C00u && __builtin_isfinite(f)) hit = true;
    return b;
}

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// e^x as 2^(x·log2 e) on the transcendental unit; -inf gives 0.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// Cross-lane folds: DPP within a row of 16 lanes (row_ror 8 and 4, then the quad permutations that swap lane
// pairs 2 apart and 1 apart), ds_swizzle in its bitmask mode for lane ^ 16 (no LDS bank access), and
// v_permlane32_swap between the wave's halves — where __shfl_xor would be a ds_bpermute a step. Each step combines
// a lane with a partner that combines it back, with a commutative operation, so every lane of the group ends with
// the same bits.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124, kDppXor2 = 0x4E, kDppXor1 = 0xB1;
// ds_swizzle offset, bitmask mode (bit 15 clear): and_mask 0x1F, or_mask 0, xor_mask 0x10 — lane l reads l ^ 16
constexpr int kSwizzleXor16 = 0x401F;
__device__ __forceinline__ float xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), kSwizzleXor16));
}
__device__ __forceinline__ float max_xor16(float v) { return fmaxf(v, xor16(v)); }
__device__ __forceinline__ float sum_xor16(float v) { return v + xor16(v); }
// {lane l's value, lane l ^ 32's}, lower half first: v_permlane32_swap of a register with itself
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float row_max(float v) {   // over the lane's row of 16
    v = fmaxf(v, dpp_mov<kDppRor8>(v));
    v = fmaxf(v, dpp_mov<kDppRor4>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    return fmaxf(v, dpp_mov<kDppXor1>(v));
}
__device__ __forceinline__ float row_sum(float v) {
    v += dpp_mov<kDppRor8>(v);
    v += dpp_mov<kDppRor4>(v);
    v += dpp_mov<kDppXor2>(v);
    return v + dpp_mov<kDppXor1>(v);
}
// Folds over the whole wave (64 lanes; every lane active) and over the four 16-lane groups of a lane's column.
__device__ __forceinline__ float wave_max(float v) { return max_xor32(max_xor16(row_max(v))); }
__device__ __forceinline__ float wave_sum(float v) { return sum_xor32(sum_xor16(row_sum(v))); }
// Over lanes l, l^16, l^32, l^48: the four row-groups of an MFMA 16x16 tile's column.
__device__ __forceinline__ float groups_max(float v) { return max_xor32(max_xor16(v)); }
__device__ __forceinline__ float groups_sum(float v) { return sum_xor32(sum_xor16(v)); }

// 16 bytes a lane from global memory straight into LDS: lane l's data lands at `lds` + 16·l (`lds` must be
// the same for the whole wave). Written as its own instruction, not the builtin, so the compiler does not
// make every later LDS read wait for it: the caller orders it with explicit vmcnt waits and barriers.
__device__ __forceinline__ void dma16(const void* src, __attribute__((address_space(3))) void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(m0) : "memory");
}
// The same from a wave-uniform base (scalar registers) plus a 32-bit per-lane byte offset: no 64-bit
// address arithmetic in the vector unit.
__device__ __forceinline__ void dma16s(const void* base, uint32_t off, __attribute__((address_space(3))) void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    const uint64_t b = (uint64_t)(uintptr_t)base;
    // readfirstlane returns a signed int: widen through uint32_t, or the low word sign-extends over the high
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(sb), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void dma16_nt(const void* src, __attribute__((address_space(3))) void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("global_load_lds_dwordx4 %0, off nt" : : "v"(src), "{m0}"(m0) : "memory");
}

// ── launch bookkeeping ─────────────────────────────────────────────────────────────────────────────
hipStream_t stream();
// Records a failed launch (printed once, remembered until silvann_gfx950_launch_failed reads it).
void check_launch(const char* what);
// Live kernel timing for the benchmark: when enabled on this thread, a door brackets its named kernel
// with hipEvents on its stream; silvann_gfx950_profile_read sums them.
void prof_begin(int kernel);
void prof_end(int kernel);
enum ProfKernel : int { kProfDecodeSplit = 0, kProfDecodeMerge = 1, kProfCausal = 2, kProfTqSplit = 3, kProfCacheWrite = 4,
                       kProfKernels = 5 };
// Records a door that refused its operands without launching (printed, remembered the same way).
void refuse(const char* what);

// ── deferred doors ──────────────────────────────────────────────────────────────────────────────────────
// The reference's verbs call some doors only as chains, back to back on one thread: attention_scores then
// attention_mix (attention__abi.cuh:155-158), attention_weights then attention_residual_mix (203-206),
// attention_causal_scores_grouped, attention_causal_softmax, attention_causal_mix (407-414), the TurboQuant pair
// attention_weights_tq then attention_residual_mix_tq (266-269, mixer__abi.cuh:395-407), the tiered prefill
// window's many-row pairs (prefill__abi.cuh:430-440), and latent attention's attention_scores_grouped then
// attention_softmax_rows (GLM 5.3, ai_z__glm_5_3/cpu/opcodes/layer__abi.cuh:283-289) or attention_softmax_sink
// (DeepSeek V4, ai_deepseek_4/cpu/opcodes/layer__abi.cuh:299-301), then attention_mix, and its many-row form
// attention_scores_grouped_rows, attention_softmax_lens, attention_mix_rows (GLM's block of rows, 1037-1043). The first door of a
// chain is recorded, not launched; when its continuation arrives with the same operands the chain runs as one fused
// kernel and the weights are never written. Any other door of this library first flushes what is recorded — runs
// the recorded door as it would have run — so every other order keeps the reference's semantics.
enum DeferKind : int {
    kDeferNone = 0, kDeferScores, kDeferWeights, kDeferCausal, kDeferCausalSoftmax, kDeferWeightsRows, kDeferWeightsTq,
    kDeferWeightsTqRows, kDeferGrouped, kDeferGroupedSoftmax, kDeferGroupedSink, kDeferGroupedRows,
    kDeferGroupedRowsSoftmax
};
struct Deferred {
    int kind = kDeferNone;
    float* p = nullptr;
    float* res = nullptr;
    const uint16_t* q = nullptr;
    const uint16_t* k = nullptr;      // keys (fp16), or
    const uint8_t* codes = nullptr;   // TurboQuant key codes
    const uint16_t* scales = nullptr;
    const uint16_t* sink = nullptr;   // attention_softmax_sink's, one a head
    const uint32_t* lens = nullptr;   // the many-row grouped chain's: rows' lengths, rows' strides
    uint64_t p_row = 0, q_row = 0, k_row = 0;
    uint64_t q_heads = 0, kv_heads = 0, head_dim = 0, length = 0, first = 0, rows = 0, d = 0;
    hipStream_t st = nullptr;
};
Deferred& deferred();     // this thread's
bool defer_enabled();     // this thread's switch (SILVANN_GFX950_DEFER=0 turns the default off)
void flush_deferred();    // launch what is recorded, if anything, and clear it
// the fused forms the continuations launch (decode.hip, prefill.hip)
bool decode_one(uint16_t* o, float* res, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint64_t q_heads,
                uint64_t kv_heads, uint64_t head_dim, uint64_t length, void* scratch, uint64_t cap, unsigned int* over,
                const uint16_t* sink = nullptr);
bool decode_rows_fit(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint32_t* lens,
                     uint64_t k_row, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t most,
                     uint64_t rows, void* scratch, uint64_t cap, unsigned int* over);
bool decode_causal(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint64_t q_heads,
                   uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows, void* scratch, uint64_t cap,
                   unsigned int* over);
bool residual_tq_fit(float* res, const uint16_t* q, const uint8_t* kc, const uint16_t* ks, const uint8_t* vc,
                     const uint16_t* vs, uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                     uint64_t d, uint64_t rows, void* scratch, uint64_t cap);
// The fused kernels read q and the K and V rows in 16-byte vectors (and V through 16-byte LDS-DMA), and keep 64-bit
// counters in their scratch: a fused form runs only on operands aligned for that, else the doors run one by one.
inline bool vec_aligned(const void* q, const void* k, const void* v) {
    return (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15u) == 0;
}
inline bool scratch_aligned(const void* s) { return (((uintptr_t)s) & 7u) == 0; }
bool causal_shape_ok(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows,
                     bool paged, uint64_t page_size);
void causal_paged_launch(uint16_t* o, float* res, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const uint32_t* pages, uint64_t page_size, uint64_t q_heads, uint64_t kv_heads,
                         uint64_t head_dim, uint64_t first, uint64_t rows, unsigned int* over, const char* what);

}  // namespace silvann
