// emu_rt.hpp — TEST INFRASTRUCTURE: a CPU emulation of the gfx950 execution model, enough to run this
// library's kernel sources on the host and check them against the oracle without a GPU.
//
// Each lane is a host thread. Lanes meet in waves of 64 and workgroups of blockDim.x at real barriers;
// the cross-lane builtins (MFMA, the transposing LDS read, readfirstlane, ballot, permlane32 swap,
// shuffles) exchange through per-wave scratch with the operand layouts the hardware documents. One
// workgroup runs at a time, so a kernel's __shared__ arrays are function statics. Direct-to-LDS loads land
// late (see dma_issue), so a missing wait or barrier shows up as NaN in the answer. Global buffers are
// placed against guard pages by the harness, so an out-of-bounds access stops the run with its address.
#pragma once
#include <atomic>
#include <barrier>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

struct EmuDim3 { uint32_t x = 0, y = 0, z = 0; };
inline thread_local EmuDim3 threadIdx, blockIdx;
inline EmuDim3 blockDim, gridDim;
struct dim3 { uint32_t x, y, z; dim3(uint32_t a = 1, uint32_t b = 1, uint32_t c = 1) : x(a), y(b), z(c) {} };
typedef void* hipStream_t;
struct float2 { float x, y; };
inline float2 make_float2(float x, float y) { return {x, y}; }

namespace emu {
constexpr int kScratch = 256;
struct Wave {
    std::barrier<> bar{64};
    alignas(64) unsigned char slot[64][kScratch];
};
struct Group {
    std::barrier<>* bar;
    Wave* waves;
    int nw;
};
inline Group* G = nullptr;
inline thread_local int tl_lane = 0, tl_wave = 0;
inline std::atomic<long> ops{0};

// deposit `mine`, meet, let every lane compute from all 64 deposits, meet again (the slots are free)
template <class T, class F>
inline auto wave_op(const T& mine, F f) {
    static_assert(sizeof(T) <= kScratch, "slot too small");
    Wave& W = G->waves[tl_wave];
    std::memcpy(W.slot[tl_lane], &mine, sizeof(T));
    W.bar.arrive_and_wait();
    auto r = f([&](int l) { T x; std::memcpy(&x, W.slot[l], sizeof(T)); return x; });
    W.bar.arrive_and_wait();
    ++ops;
    return r;
}
// Direct-to-LDS loads land late: the destination holds NaN halves from issue until the issuing lane's
// s_waitcnt lets the load retire (loads retire in order), so a read before landing or a load over bytes
// another wave still reads shows up as NaN in the answer. EMU_SYNC=1 lands them at once instead.
struct PendingDma { char* dst; unsigned char data[16]; };
inline thread_local std::vector<PendingDma> tl_dma;
inline thread_local size_t tl_dma_head = 0;
inline bool async_dma = !getenv("EMU_SYNC");
inline void dma_issue(const char* src, char* dst) {
    PendingDma p; p.dst = dst; std::memcpy(p.data, src, 16);
    if (async_dma) { std::memset(dst, 0xFF, 16); tl_dma.push_back(p); }
    else std::memcpy(dst, src, 16);
}
inline void waitcnt(int imm) {
    const size_t vm = (imm & 0xF) | (((imm >> 14) & 3) << 4);
    while (tl_dma.size() - tl_dma_head > vm) { auto& p = tl_dma[tl_dma_head++]; std::memcpy(p.dst, p.data, 16); }
    if (tl_dma_head == tl_dma.size()) { tl_dma.clear(); tl_dma_head = 0; }
}
inline void launch(dim3 grid, uint32_t threads, std::function<void()> body, const char* name = "") {
    static const bool log = getenv("EMU_LAUNCHES") != nullptr;
    if (log) std::fprintf(stderr, "emu launch %s\n", name);
    gridDim = {grid.x, grid.y, grid.z};
    blockDim = {threads, 1, 1};
    const int nw = (threads + 63) / 64;
    for (uint32_t z = 0; z < grid.z; ++z)
        for (uint32_t y = 0; y < grid.y; ++y)
            for (uint32_t x = 0; x < grid.x; ++x) {
                std::barrier<> bar(threads);
                std::vector<Wave> waves(nw);
                Group g{&bar, waves.data(), nw};
                G = &g;
                std::vector<std::thread> th;
                th.reserve(threads);
                for (uint32_t t = 0; t < threads; ++t)
                    th.emplace_back([&, t] {
                        threadIdx = {t, 0, 0};
                        blockIdx = {x, y, z};
                        tl_lane = t & 63;
                        tl_wave = t >> 6;
                        body();
                        waitcnt(0);
                        // a lane that finished still arrives at the barriers of the lanes still running
                        G->bar->arrive_and_drop();
                        G->waves[tl_wave].bar.arrive_and_drop();
                    });
                for (auto& h : th) h.join();
                G = nullptr;
            }
}
}  // namespace emu

inline void __syncthreads() { emu::G->bar->arrive_and_wait(); }

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static

template <class T> inline T min(T a, T b) { return a < b ? a : b; }
template <class T> inline T max(T a, T b) { return a > b ? a : b; }
inline uint32_t __float_as_uint(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float __uint_as_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

template <class T> inline T emu_readfirstlane(T v) {
    return emu::wave_op(v, [](auto get) { return get(0); });
}
#define __builtin_amdgcn_readfirstlane(v) emu_readfirstlane(v)
inline uint64_t __builtin_amdgcn_ballot_w64(bool p) {
    return emu::wave_op(p, [](auto get) { uint64_t m = 0; for (int l = 0; l < 64; ++l) if (get(l)) m |= 1ull << l; return m; });
}
inline int __builtin_amdgcn_readlane(int v, int l) {
    return emu::wave_op(v, [&](auto get) { return get(l); });
}
template <class T> inline T __shfl_xor(T v, int mask, int width = 64) {
    const int me = emu::tl_lane;
    return emu::wave_op(v, [&](auto get) { int src = me ^ mask; if ((src & ~(width - 1)) != (me & ~(width - 1))) src = me; return get(src); });
}
typedef uint32_t emu_u32x2 __attribute__((ext_vector_type(2)));
inline emu_u32x2 __builtin_amdgcn_permlane32_swap(uint32_t vdst, uint32_t src, bool, bool) {
    struct P { uint32_t d, s; };
    const int me = emu::tl_lane;
    return emu::wave_op(P{vdst, src}, [&](auto get) {
        emu_u32x2 r;
        if (me < 32) { r[0] = get(me).d; r[1] = get(me + 32).d; }   // vdst low unchanged; src low <- vdst high
        else { r[0] = get(me - 32).s; r[1] = get(me).s; }          // vdst high <- src low; src high unchanged
        return r;
    });
}
// ds_swizzle, bitmask mode only (offset bit 15 clear): lane l of each 32 reads ((l & and) | or) ^ xor
inline int __builtin_amdgcn_ds_swizzle(int v, int offset) {
    const int me = emu::tl_lane;
    if (offset & 0x8000) {
        std::fprintf(stderr, "emu: ds_swizzle offset %#x\n", offset);
        std::abort();
    }
    const int andm = offset & 31, orm = (offset >> 5) & 31, xorm = (offset >> 10) & 31;
    return emu::wave_op(v, [&](auto get) { return get((me & ~31) | ((((me & 31) & andm) | orm) ^ xorm)); });
}
// DPP moves: quad_perm (ctrl < 0x100, lane i of a quad reads lane (ctrl >> 2i) & 3) and row_ror (0x121-0x12F,
// lane i of a row of 16 reads lane (i - n) mod 16); every lane active, masks full
inline int __builtin_amdgcn_mov_dpp(int v, int ctrl, int, int, bool) {
    const int me = emu::tl_lane;
    if (!(ctrl < 0x100 || (ctrl >= 0x121 && ctrl <= 0x12F))) {
        std::fprintf(stderr, "emu: dpp control %#x\n", ctrl);
        std::abort();
    }
    return emu::wave_op(v, [&](auto get) {
        const int src = ctrl < 0x100 ? (me & ~3) | ((ctrl >> (2 * (me & 3))) & 3) : (me & ~15) | ((me - (ctrl & 15)) & 15);
        return get(src);
    });
}
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_s_waitcnt(x) emu::waitcnt(x)
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
// lanes of a wave are not in lockstep here: a wave barrier is a real meeting of the wave's 64 lanes
inline void __builtin_amdgcn_wave_barrier() { emu::G->waves[emu::tl_wave].bar.arrive_and_wait(); }
// global_load_lds: each lane's `size` bytes from its own address land at (the first lane's lds) + lane·size
inline void __builtin_amdgcn_global_load_lds(const void* src, void* lds, int size, int, int) {
    if (size != 16) { std::fprintf(stderr, "emu: global_load_lds size %d\n", size); std::abort(); }
    char* dst = (char*)emu_readfirstlane(lds) + 16 * emu::tl_lane;
    emu::dma_issue((const char*)src, dst);
}
inline uint32_t atomicAdd(uint32_t* p, uint32_t v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline void __threadfence() { __atomic_thread_fence(__ATOMIC_SEQ_CST); }
inline unsigned int atomicCAS(unsigned int* p, unsigned int cmp, unsigned int val) {
    __atomic_compare_exchange_n(p, &cmp, val, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
    return cmp;
}
inline unsigned long long atomicCAS(unsigned long long* p, unsigned long long cmp, unsigned long long val) {
    __atomic_compare_exchange_n(p, &cmp, val, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
    return cmp;
}
typedef int hipError_t;
constexpr hipError_t hipSuccess = 0;
enum { hipDeviceAttributeMultiprocessorCount = 0 };
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, int, int) { *v = 256; return hipSuccess; }
#define __builtin_amdgcn_sched_group_barrier(a, b, c) ((void)0)

typedef _Float16 emu_f16x8 __attribute__((ext_vector_type(8)));
typedef float emu_f32x16 __attribute__((ext_vector_type(16)));
typedef short emu_s16x4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_32x32x16_f16: lane l holds A[m = l % 32][k = 8·(l / 32) + i], B[k = 8·(l / 32) + i][n = l % 32],
// and D register r at m = 8·(r / 4) + 4·(l / 32) + r % 4, n = l % 32.
inline emu_f32x16 __builtin_amdgcn_mfma_f32_32x32x16_f16(emu_f16x8 a, emu_f16x8 b, emu_f32x16 c, int, int, int) {
    struct In { emu_f16x8 a, b; };
    const int me = emu::tl_lane;
    return emu::wave_op(In{a, b}, [&](auto get) {
        float A[32][16], B[16][32];
        for (int l = 0; l < 64; ++l) {
            In x = get(l);
            for (int i = 0; i < 8; ++i) { A[l % 32][8 * (l / 32) + i] = (float)x.a[i]; B[8 * (l / 32) + i][l % 32] = (float)x.b[i]; }
        }
        emu_f32x16 d;
        const int n = me % 32;
        for (int r = 0; r < 16; ++r) {
            const int m = 8 * (r / 4) + 4 * (me / 32) + r % 4;
            double s = c[r];
            for (int k = 0; k < 16; ++k) s += (double)A[m][k] * (double)B[k][n];
            d[r] = (float)s;
        }
        return d;
    });
}
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
// v_mfma_f32_16x16x32_f16: lane l holds A[m = l % 16][k = 8·(l / 16) + i], B[k = 8·(l / 16) + i][n = l % 16],
// and D register r at m = 4·(l / 16) + r, n = l % 16.
inline emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x32_f16(emu_f16x8 a, emu_f16x8 b, emu_f32x4 c, int, int, int) {
    struct In { emu_f16x8 a, b; };
    const int me = emu::tl_lane;
    return emu::wave_op(In{a, b}, [&](auto get) {
        float A[16][32], B[32][16];
        for (int l = 0; l < 64; ++l) {
            In x = get(l);
            for (int i = 0; i < 8; ++i) { A[l % 16][8 * (l / 16) + i] = (float)x.a[i]; B[8 * (l / 16) + i][l % 16] = (float)x.b[i]; }
        }
        emu_f32x4 d;
        const int n = me % 16;
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * (me / 16) + r;
            double s = c[r];
            for (int k = 0; k < 32; ++k) s += (double)A[m][k] * (double)B[k][n];
            d[r] = (float)s;
        }
        return d;
    });
}
// ds_read_b64_tr_b16: in each block of 16 lanes, lane 4·j + q reads halves (row j, columns 4·q .. 4·q + 3) of
// a 4 × 16 tile; lane i of the block receives column i: (row 0, i), (row 1, i), (row 2, i), (row 3, i).
inline emu_s16x4 __builtin_amdgcn_ds_read_tr16_b64_v4i16(emu_s16x4* p) {
    const int me = emu::tl_lane;
    const emu_s16x4 mine = *p;
    return emu::wave_op(mine, [&](auto get) {
        const int b = me & ~15, i = me & 15;
        emu_s16x4 r;
        for (int j = 0; j < 4; ++j) r[j] = get(b + 4 * j + i / 4)[i % 4];
        return r;
    });
}
