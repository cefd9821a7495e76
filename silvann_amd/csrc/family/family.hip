// family.hip — this library as a SiLVANN silicon family of its own: libsilvann_gfx950_family.so, which exports one
// symbol, `silvann_silicon_family_get`, as every family does (engine/src/silicon_families/entry.cuh:69-81;
// engine/scripts/build_silicon_families.sh:69-79 checks that nothing else of ours is exported).
//
// The table it answers for ABI version 9 (packages/sys/contracts/abi/silicon_family.cuh:33, 48-55) carries one door
// table a package, in the engine's package order (packages/manifest__header.cuh:162-169):
//   sys (0)    the 31 doors of packages/sys/contracts/abi/gpu.cuh:47-77 on the HIP runtime, for the gfx950 cards
//              only (a family numbers only the cards it takes)
//   nn (1)     the 137 rows of packages/nn/contracts/abi/gpu.cuh:93-241 and this library's five appended rows: its
//              attention rows and rope_rows are this library's doors; every other row refuses (the launch is
//              remembered as refused, so the next compute_completed answers false and the engine raises the
//              fault) — this family runs attention, not the whole of nn
//   2-6        the model packages' tables, which hold only their size (ai_qwen_3/contracts/abi/gpu.cuh:10)
// The library's deferred door chains run through the sys doors too: every one of them first runs what a chain has
// recorded, so a program that reads a weights buffer with memory_read sees its weights.
#include <fcntl.h>
#include <string.h>
#include <unistd.h>

#include <memory>
#include <new>

#include "../common.hpp"
#include "../../../include/silvann_gfx950_attention.h"

namespace silvann {
namespace {

constexpr uint32_t kAbiVersion = 9;       // silicon_family.cuh:33
constexpr uint32_t kFamilyId = 275;       // between amd_rocm10 (250) and nvidia_cuda12 (300): roster.cuh:55-66
constexpr uint32_t kSysRows = 31;         // sys/contracts/abi/gpu.cuh:47-77
constexpr uint32_t kNnRows = SILVANN_GFX950_NN_ROWS + 5;   // the reference's 137 and the appended 137-141
constexpr uint32_t kPackages = 7;         // manifest__header.cuh:162-169

struct FamilyTable {   // silicon_family.cuh:48-55
    uint32_t abi_version, size, id, package_count;
    const char* name;
    const void* const* package_doors;
};
struct SysDoors { uint32_t size; void* row[kSysRows]; };
struct NnDoors { uint32_t size; void* row[kNnRows]; };
struct SizeOnly { uint32_t size; };

// ── which cards: the gfx950 ones, numbered in the runtime's order ────────────────────────────────────────────
bool takes(int ordinal) {
    hipDeviceProp_t p;
    return hipGetDeviceProperties(&p, ordinal) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0;
}
int shown() {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0 ? n : 0;
}
int ordinal_of(uint32_t index) {   // the runtime's number for this family's device `index`, or -1
    uint32_t mine = 0;
    for (int o = 0; o < shown(); ++o)
        if (takes(o) && mine++ == index) return o;
    return -1;
}

// ── the sys doors, in the order of the contract's list ───────────────────────────────────────────────────────
bool memory_allocate(void** at, size_t bytes) { flush_deferred(); return hipMalloc(at, bytes) == hipSuccess; }
void memory_free(void* at) { flush_deferred(); if (at) (void)hipFree(at); }
bool memory_zerofill(void* at, size_t bytes) {
    flush_deferred();
    return hipMemsetAsync(at, 0, bytes, stream()) == hipSuccess && hipStreamSynchronize(stream()) == hipSuccess;
}
// card -> RAM and RAM -> card, after the work queued before them, and waited for
bool memory_read(void* to, const void* from, size_t bytes) {
    flush_deferred();
    return hipMemcpyAsync(to, from, bytes, hipMemcpyDeviceToHost, stream()) == hipSuccess &&
           hipStreamSynchronize(stream()) == hipSuccess;
}
bool memory_write(void* to, const void* from, size_t bytes) {
    flush_deferred();
    return hipMemcpyAsync(to, from, bytes, hipMemcpyHostToDevice, stream()) == hipSuccess &&
           hipStreamSynchronize(stream()) == hipSuccess;
}
// Every door this thread queued has finished — and none was refused: a refused launch answers false once
// (amd_rocm_base/sys.cuh:39-62's rule, kept per device by silvann_gfx950_launch_failed).
bool compute_completed() {
    flush_deferred();
    const bool waited = hipStreamSynchronize(stream()) == hipSuccess;
    if (silvann_gfx950_launch_failed()) return false;
    return waited;
}
bool side_open(void** channel) {   // a queue whose copies do not wait behind compute (default priority)
    flush_deferred();
    return hipStreamCreateWithFlags((hipStream_t*)channel, hipStreamNonBlocking) == hipSuccess;
}
void side_close(void* channel) { if (channel) (void)hipStreamDestroy((hipStream_t)channel); }
bool side_memory_read(void* to, const void* from, size_t bytes, void* channel) {
    flush_deferred();
    return hipMemcpyAsync(to, from, bytes, hipMemcpyDeviceToHost, (hipStream_t)channel) == hipSuccess &&
           hipStreamSynchronize((hipStream_t)channel) == hipSuccess;
}
bool side_memory_write(void* to, const void* from, size_t bytes, void* channel) {
    flush_deferred();
    return hipMemcpyAsync(to, from, bytes, hipMemcpyHostToDevice, (hipStream_t)channel) == hipSuccess &&
           hipStreamSynchronize((hipStream_t)channel) == hipSuccess;
}
bool memory_allocate_host_ram_mapped(void** at, void** card_at, size_t bytes) {
    if (hipHostMalloc(at, bytes, hipHostMallocMapped) != hipSuccess) return false;
    if (hipHostGetDevicePointer(card_at, *at, 0) == hipSuccess) return true;
    (void)hipHostFree(*at);
    *at = nullptr;
    return false;
}
void memory_free_host_ram(void* at) { if (at) (void)hipHostFree(at); }
uint32_t device_count() {
    uint32_t mine = 0;
    for (int o = 0; o < shown(); ++o)
        if (takes(o)) ++mine;
    return mine;
}
uint32_t bind_device(uint32_t index) {   // per thread, as the runtime binds: 1 when bound
    flush_deferred();
    const int o = ordinal_of(index);
    return o >= 0 && hipSetDevice(o) == hipSuccess ? 1u : 0u;
}
uint32_t bound_device() {   // this family's number for the thread's card, or 0xFFFFFFFF
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || !takes(d)) return 0xFFFFFFFFu;
    uint32_t mine = 0;
    for (int o = 0; o < d; ++o)
        if (takes(o)) ++mine;
    return mine;
}
// RAM the program already holds cannot be pinned in place here: the runtime's host registration is not offered on
// these machines, so the door answers no and the program takes memory_allocate_host_ram_mapped instead.
bool memory_register_host(void* at, size_t bytes, void** card_at) {
    (void)at; (void)bytes; (void)card_at;
    return false;
}
void memory_unregister_host(void* at) { (void)at; }
// A handle is the descriptor plus one, so 0 is never a file (file.cuh:25-38's convention).
bool file_open(const char* path, uint64_t* handle) {
    if (!path || !handle) return false;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return false;
    *handle = (uint64_t)(uint32_t)fd + 1u;
    return true;
}
void file_close(uint64_t handle) {
    if (handle != 0) (void)close((int)(handle - 1));
}
// `bytes` of the file from `offset` into card memory at `to`, through a host bounce buffer of up to 64 MiB, each
// piece written as memory_write writes (after the work queued before it); false on a short file or a failed copy
// (file.cuh:89-102's contract)
bool file_read(uint64_t handle, uint64_t offset, uint64_t bytes, void* to) {
    if (handle == 0 || (!to && bytes != 0)) return false;
    const int fd = (int)(handle - 1);
    const uint64_t piece = bytes < (64ull << 20) ? bytes : (64ull << 20);
    std::unique_ptr<char[]> bounce(piece ? new (std::nothrow) char[piece] : nullptr);
    if (piece && !bounce) return false;
    for (uint64_t done = 0; done < bytes;) {
        const uint64_t want = bytes - done < piece ? bytes - done : piece;
        uint64_t got = 0;
        while (got < want) {
            const ssize_t n = pread(fd, bounce.get() + got, want - got, (off_t)(offset + done + got));
            if (n <= 0) return false;
            got += (uint64_t)n;
        }
        if (!memory_write((char*)to + done, bounce.get(), want)) return false;
        done += want;
    }
    return true;
}
// A card's memory is not the machine's to map a file into (amd_rocm_base/sys.cuh:205-209's answer).
bool memory_map_file(void* at, size_t bytes, uint64_t handle, uint64_t offset) {
    (void)at; (void)bytes; (void)handle; (void)offset;
    return false;
}
bool memory_prefetch(const void* at, size_t bytes) { (void)at; (void)bytes; return true; }   // always resident
bool peer_access(uint32_t other) {
    flush_deferred();
    int here = -1;
    const int there = ordinal_of(other);
    if (hipGetDevice(&here) != hipSuccess || here < 0 || there < 0) return false;
    if (here == there) return true;
    int can = 0;
    if (hipDeviceCanAccessPeer(&can, here, there) != hipSuccess || can == 0) return false;
    const hipError_t on = hipDeviceEnablePeerAccess(there, 0);
    if (on == hipErrorPeerAccessAlreadyEnabled) {
        (void)hipGetLastError();
        return true;
    }
    return on == hipSuccess;
}
// marks: events on the thread's stream, only ever waited for
bool mark_open(void** mark) { return hipEventCreateWithFlags((hipEvent_t*)mark, hipEventDisableTiming) == hipSuccess; }
void mark_close(void* mark) { if (mark) (void)hipEventDestroy((hipEvent_t)mark); }
bool mark_record(void* mark) { flush_deferred(); return hipEventRecord((hipEvent_t)mark, stream()) == hipSuccess; }
bool mark_wait(void* mark) { flush_deferred(); return hipStreamWaitEvent(stream(), (hipEvent_t)mark, 0) == hipSuccess; }
bool side_memory_write_queued(void* to, const void* from, size_t bytes, void* channel) {
    flush_deferred();
    return hipMemcpyAsync(to, from, bytes, hipMemcpyHostToDevice, (hipStream_t)channel) == hipSuccess;
}
bool side_memory_read_queued(void* to, const void* from, size_t bytes, void* channel) {
    flush_deferred();
    return hipMemcpyAsync(to, from, bytes, hipMemcpyDeviceToHost, (hipStream_t)channel) == hipSuccess;
}
bool side_mark_record(void* mark, void* channel) {
    return hipEventRecord((hipEvent_t)mark, (hipStream_t)channel) == hipSuccess;
}
bool mark_reached(void* mark) { return hipEventSynchronize((hipEvent_t)mark) == hipSuccess; }

// An nn row this family does not run: remembered as a refused launch (every nn door returns nothing, so one
// function stands for every signature).
void nn_unanswered() { refuse("an nn row outside attention (this family runs attention only)"); }

struct Tables {
    SysDoors sys;
    NnDoors nn;
    SizeOnly models[kPackages - 2];
    const void* packages[kPackages];
    FamilyTable family;
    Tables() {
        sys.size = (uint32_t)sizeof(SysDoors);
        void* const rows[kSysRows] = {
            (void*)&memory_allocate, (void*)&memory_free, (void*)&memory_zerofill, (void*)&memory_read,
            (void*)&memory_write, (void*)&compute_completed, (void*)&side_open, (void*)&side_close,
            (void*)&side_memory_read, (void*)&side_memory_write, (void*)&memory_allocate_host_ram_mapped,
            (void*)&memory_free_host_ram, (void*)&device_count, (void*)&bind_device, (void*)&bound_device,
            (void*)&memory_register_host, (void*)&memory_unregister_host, (void*)&file_open, (void*)&file_close,
            (void*)&file_read, (void*)&memory_map_file, (void*)&memory_prefetch, (void*)&peer_access,
            (void*)&mark_open, (void*)&mark_close, (void*)&mark_record, (void*)&mark_wait,
            (void*)&side_memory_write_queued, (void*)&side_memory_read_queued, (void*)&side_mark_record,
            (void*)&mark_reached,
        };
        for (uint32_t i = 0; i < kSysRows; ++i) sys.row[i] = rows[i];
        nn.size = (uint32_t)sizeof(NnDoors);
        for (uint32_t i = 0; i < kNnRows; ++i) nn.row[i] = (void*)&nn_unanswered;
        (void)silvann_gfx950_attention_install(&nn);   // this library's rows over the refusing ones
        for (auto& m : models) m.size = (uint32_t)sizeof(SizeOnly);
        packages[0] = &sys;
        packages[1] = &nn;
        for (uint32_t i = 2; i < kPackages; ++i) packages[i] = &models[i - 2];
        family = FamilyTable{kAbiVersion, (uint32_t)sizeof(FamilyTable), kFamilyId, kPackages,
                             "amd_gfx950_attention", packages};
    }
};

}  // namespace
}  // namespace silvann

// The one exported function: the table for the version this family speaks, nothing for another
// (entry.cuh:69-81: a program reading a table of another shape would call through the wrong pointers).
extern "C" __attribute__((visibility("default"))) const void* silvann_silicon_family_get(uint32_t abi_version) {
    static const silvann::Tables tables;
    return abi_version == silvann::kAbiVersion ? (const void*)&tables.family : nullptr;
}
