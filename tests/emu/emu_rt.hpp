// emu_rt.hpp — TEST INFRASTRUCTURE: a CPU emulation of the gfx950 execution model, enough to run this
// library's kernel sources on the host and check them against the oracle without a GPU.
//
// Each lane is a fiber: one host thread runs every lane of a workgroup, switching lanes only where a lane waits
// at a barrier (a workgroup barrier, a wave barrier, or the meeting inside a cross-lane op). Lanes meet in waves
// of 64 and workgroups of blockDim.x; the cross-lane builtins (MFMA, the transposing LDS read, readfirstlane,
// ballot, the lane swaps, DPP, swizzles, shuffles) exchange through per-wave scratch with the operand layouts the
// hardware documents. One workgroup runs at a time, so a kernel's __shared__ arrays are function statics.
// Direct-to-LDS loads land late (see dma_issue), so a missing wait or barrier shows up as NaN in the answer.
// Global buffers are placed against guard pages by the harness, so an out-of-bounds access stops the run with
// its address. Lanes that can all never run again (a barrier some lanes never reach) stop the run too. Between
// barriers the lanes run in a seeded random order (EMU_SEED), fresh each time they all have run.
#pragma once
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <vector>

#include <unistd.h>

struct EmuDim3 { uint32_t x = 0, y = 0, z = 0; };
inline EmuDim3 threadIdx, blockIdx;   // the running lane's (set at every switch to it)
inline EmuDim3 blockDim, gridDim;
struct dim3 { uint32_t x, y, z; dim3(uint32_t a = 1, uint32_t b = 1, uint32_t c = 1) : x(a), y(b), z(c) {} };
typedef void* hipStream_t;
struct float2 { float x, y; };
inline float2 make_float2(float x, float y) { return {x, y}; }

// Saves the callee-saved registers and the stack pointer of the running context in *save_sp and resumes the one
// whose stack pointer is load_sp (harness.cpp, x86-64 System V).
extern "C" void emu_ctx_switch(void** save_sp, void* load_sp);

namespace emu {
constexpr int kScratch = 256;
// A barrier of `count` lanes: the last to arrive completes the phase (a new generation) and runs on; the others
// wait until their phase's generation has passed. A lane that ends drops out of every later phase.
struct Barrier {
    int count = 0, arrived = 0;
    unsigned gen = 0;
};
struct Wave {
    Barrier bar;
    alignas(64) unsigned char slot[64][kScratch];
    // a cross-lane op whose 64 answers one lane computes for all: computed once an op
    bool computed = false;
    alignas(64) unsigned char result[64][64];
};
struct Group {
    Barrier* bar;
    Wave* waves;
    int nw;
};
inline Group* G = nullptr;
inline int tl_lane = 0, tl_wave = 0;   // the running lane's
inline std::atomic<long> ops{0};

struct PendingDma { char* dst; unsigned char data[16]; };
struct Lane {
    void* sp = nullptr;
    std::unique_ptr<char[]> stack;
    uint32_t t = 0;
    std::vector<PendingDma> dma;
    size_t dma_head = 0;
    Barrier* wait = nullptr;
    unsigned wait_gen = 0;
    bool done = false;
};
constexpr size_t kStackBytes = 1 << 20;   // a lane's stack (the kernels keep whole tiles of operands in locals)
inline std::vector<Lane> lanes;
inline Lane* cur = nullptr;
inline void* sched_sp = nullptr;
inline const std::function<void()>* body = nullptr;

inline void yield() { emu_ctx_switch(&cur->sp, sched_sp); }
inline void arrive_and_wait(Barrier& b) {
    if (++b.arrived == b.count) {   // the last: the phase completes, this lane runs on
        b.arrived = 0;
        ++b.gen;
        return;
    }
    cur->wait = &b;
    cur->wait_gen = b.gen;
    yield();
}
inline void arrive_and_drop(Barrier& b) {
    --b.count;
    if (b.count > 0 && b.arrived == b.count) {
        b.arrived = 0;
        ++b.gen;
    }
}

// deposit `mine`, meet, let every lane compute from all 64 deposits, meet again (the slots are free)
template <class T, class F>
inline auto wave_op(const T& mine, F f) {
    static_assert(sizeof(T) <= kScratch, "slot too small");
    Wave& W = G->waves[tl_wave];
    std::memcpy(W.slot[tl_lane], &mine, sizeof(T));
    arrive_and_wait(W.bar);
    auto r = f([&](int l) { T x; std::memcpy(&x, W.slot[l], sizeof(T)); return x; });
    arrive_and_wait(W.bar);
    ++ops;
    return r;
}
// The same, for ops whose answers come from one computation over all 64 deposits: `all(get, out)` fills every
// lane's answer once an op (the first lane past the meeting runs it), each lane takes its own.
template <class R, class T, class F>
inline R wave_op_all(const T& mine, F all) {
    static_assert(sizeof(T) <= kScratch && sizeof(R) <= 64, "slot too small");
    Wave& W = G->waves[tl_wave];
    std::memcpy(W.slot[tl_lane], &mine, sizeof(T));
    arrive_and_wait(W.bar);
    if (!W.computed) {
        R out[64];
        all([&](int l) { T x; std::memcpy(&x, W.slot[l], sizeof(T)); return x; }, out);
        for (int l = 0; l < 64; ++l) std::memcpy(W.result[l], &out[l], sizeof(R));
        W.computed = true;
    }
    R r;
    std::memcpy(&r, W.result[tl_lane], sizeof(R));
    arrive_and_wait(W.bar);
    W.computed = false;   // every lane has its answer: the next op computes afresh
    ++ops;
    return r;
}
// Direct-to-LDS loads land late: the destination holds NaN halves from issue until the issuing lane's
// s_waitcnt lets the load retire (loads retire in order), so a read before landing or a load over bytes
// another wave still reads shows up as NaN in the answer. EMU_SYNC=1 lands them at once instead.
inline bool async_dma = !getenv("EMU_SYNC");
inline void dma_issue(const char* src, char* dst) {
    PendingDma p; p.dst = dst; std::memcpy(p.data, src, 16);
    if (async_dma) { std::memset(dst, 0xFF, 16); cur->dma.push_back(p); }
    else std::memcpy(dst, src, 16);
}
inline void waitcnt(int imm) {
    auto& q = cur->dma;
    size_t& head = cur->dma_head;
    const size_t vm = (imm & 0xF) | (((imm >> 14) & 3) << 4);
    while (q.size() - head > vm) { auto& p = q[head++]; std::memcpy(p.dst, p.data, 16); }
    if (head == q.size()) { q.clear(); head = 0; }
}

// a lane's first instructions: its body, its loads landed, out of every later barrier phase, back to the scheduler
[[noreturn]] inline void lane_entry() {
    (*body)();
    waitcnt(0);
    arrive_and_drop(*G->bar);
    arrive_and_drop(G->waves[tl_wave].bar);
    cur->done = true;
    yield();
    std::abort();   // a finished lane is never resumed
}
inline void lane_start(Lane& L) {
    if (!L.stack) L.stack.reset(new char[kStackBytes]);
    uintptr_t top = ((uintptr_t)L.stack.get() + kStackBytes) & ~(uintptr_t)15;
    void** sp = (void**)top;
    *--sp = nullptr;                      // lane_entry's return address (it never returns): entry rsp = 8 mod 16
    *--sp = (void*)&lane_entry;           // emu_ctx_switch's `ret` goes here
    for (int i = 0; i < 6; ++i) *--sp = nullptr;   // rbp, rbx, r12-r15
    L.sp = sp;
}

inline void launch(dim3 grid, uint32_t threads, std::function<void()> fn, const char* name = "") {
    static const bool log = getenv("EMU_LAUNCHES") != nullptr;
    if (log) std::fprintf(stderr, "emu launch %s\n", name);
    gridDim = {grid.x, grid.y, grid.z};
    blockDim = {threads, 1, 1};
    const int nw = (threads + 63) / 64;
    if (lanes.size() < threads) lanes.resize(threads);
    std::vector<Wave> waves(nw);
    std::vector<uint32_t> order(threads);
    static const uint64_t seed = getenv("EMU_SEED") ? strtoull(getenv("EMU_SEED"), nullptr, 10) : 1;
    body = &fn;
    for (uint32_t z = 0; z < grid.z; ++z)
        for (uint32_t y = 0; y < grid.y; ++y)
            for (uint32_t x = 0; x < grid.x; ++x) {
                Barrier bar;
                bar.count = (int)threads;
                for (int w = 0; w < nw; ++w) {
                    waves[w].bar = Barrier();
                    waves[w].bar.count = (int)(threads - 64u * w < 64u ? threads - 64u * w : 64u);
                    waves[w].computed = false;
                }
                Group g{&bar, waves.data(), nw};
                G = &g;
                blockIdx = {x, y, z};
                for (uint32_t t = 0; t < threads; ++t) {
                    Lane& L = lanes[t];
                    L.t = t;
                    L.dma.clear();
                    L.dma_head = 0;
                    L.wait = nullptr;
                    L.done = false;
                    lane_start(L);
                }
                // each sweep visits the lanes in a fresh order (seeded: EMU_SEED, the workgroup), so no wave is
                // always the first to reach shared memory: a missing barrier between one wave's LDS writes and
                // another's reads shows up whichever wave writes
                uint64_t rng = seed ^ (0x9E3779B97F4A7C15ull * (1 + x + (uint64_t)gridDim.x * (y + (uint64_t)gridDim.y * z)));
                for (uint32_t t = 0; t < threads; ++t) order[t] = t;
                // and only a random half of the waves runs in a sweep, so waves drift apart as far as their
                // barriers let them: a wave that overwrites shared memory another wave still reads does so here
                uint32_t running = threads;
                while (running) {
                    bool moved = false, ready = false;
                    auto next = [&] { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return rng; };
                    for (uint32_t i = threads - 1; i > 0; --i) {   // Fisher-Yates with xorshift64
                        const uint32_t j = (uint32_t)(next() % (i + 1));
                        const uint32_t tmp = order[i]; order[i] = order[j]; order[j] = tmp;
                    }
                    uint64_t runs = next();
                    if (nw > 1 && (runs & ((nw < 64 ? 1ull << nw : 0ull) - 1)) == 0) runs |= 1ull << (next() % nw);
                    if (nw == 1) runs = 1;
                    for (uint32_t i = 0; i < threads; ++i) {
                        const uint32_t t = order[i];
                        Lane& L = lanes[t];
                        if (L.done || (L.wait && L.wait->gen == L.wait_gen)) continue;
                        ready = true;
                        if (!((runs >> (t >> 6)) & 1)) continue;
                        L.wait = nullptr;
                        cur = &L;
                        threadIdx = {t, 0, 0};
                        tl_lane = (int)(t & 63);
                        tl_wave = (int)(t >> 6);
                        emu_ctx_switch(&sched_sp, L.sp);
                        moved = true;
                        if (L.done) --running;
                    }
                    if (!moved && !ready) {
                        const char m[] = "EMU DEADLOCK (a barrier some lanes never reach)\n";
                        (void)!write(2, m, sizeof m - 1);
                        _exit(4);
                    }
                }
                cur = nullptr;
                G = nullptr;
            }
}
}  // namespace emu

inline void __syncthreads() { emu::arrive_and_wait(*emu::G->bar); }

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
inline void __builtin_amdgcn_wave_barrier() { emu::arrive_and_wait(emu::G->waves[emu::tl_wave].bar); }
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
    struct In { emu_f16x8 a, b; emu_f32x16 c; };
    return emu::wave_op_all<emu_f32x16>(In{a, b, c}, [](auto get, emu_f32x16* out) {
        float A[32][16], B[16][32];
        for (int l = 0; l < 64; ++l) {
            In x = get(l);
            for (int i = 0; i < 8; ++i) { A[l % 32][8 * (l / 32) + i] = (float)x.a[i]; B[8 * (l / 32) + i][l % 32] = (float)x.b[i]; }
        }
        for (int me = 0; me < 64; ++me) {
            const emu_f32x16 cc = get(me).c;
            const int n = me % 32;
            for (int r = 0; r < 16; ++r) {
                const int m = 8 * (r / 4) + 4 * (me / 32) + r % 4;
                double s = cc[r];
                for (int k = 0; k < 16; ++k) s += (double)A[m][k] * (double)B[k][n];
                out[me][r] = (float)s;
            }
        }
    });
}
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
// v_mfma_f32_16x16x32_f16: lane l holds A[m = l % 16][k = 8·(l / 16) + i], B[k = 8·(l / 16) + i][n = l % 16],
// and D register r at m = 4·(l / 16) + r, n = l % 16.
inline emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x32_f16(emu_f16x8 a, emu_f16x8 b, emu_f32x4 c, int, int, int) {
    struct In { emu_f16x8 a, b; emu_f32x4 c; };
    return emu::wave_op_all<emu_f32x4>(In{a, b, c}, [](auto get, emu_f32x4* out) {
        float A[16][32], B[32][16];
        for (int l = 0; l < 64; ++l) {
            In x = get(l);
            for (int i = 0; i < 8; ++i) { A[l % 16][8 * (l / 16) + i] = (float)x.a[i]; B[8 * (l / 16) + i][l % 16] = (float)x.b[i]; }
        }
        for (int me = 0; me < 64; ++me) {
            const emu_f32x4 cc = get(me).c;
            const int n = me % 16;
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * (me / 16) + r;
                double s = cc[r];
                for (int k = 0; k < 32; ++k) s += (double)A[m][k] * (double)B[k][n];
                out[me][r] = (float)s;
            }
        }
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
