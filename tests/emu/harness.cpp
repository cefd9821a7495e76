// harness.cpp — TEST INFRASTRUCTURE: runs one call of one of the library's entry points (causal prefill, its
// residual form, paged decode, the reference's generic rows, the TurboQuant rows, the cache writer) in the CPU emulation, on inputs and parameters a test
// wrote to a directory, and writes the answer back there. Every buffer sits against an inaccessible page, so an out-of-bounds read or write stops the
// run with the buffer, the offset and the lane that made it; a run that outlives its time limit (a lost
// barrier) stops too.
#include <vector>
#include <execinfo.h>
#include <signal.h>
#include <sys/mman.h>
#include <unistd.h>

#include <string>

#include "emu_rt.hpp"
#include "silvann_gfx950_attention.h"

// The lanes' context switch (emu_rt.hpp): push the callee-saved registers, keep the stack pointer in *save_sp (rdi),
// take load_sp (rsi) as the stack pointer, pop that context's callee-saved registers and return into it.
asm(R"(
    .text
    .globl emu_ctx_switch
    .type emu_ctx_switch, @function
emu_ctx_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size emu_ctx_switch, .-emu_ctx_switch
)");

namespace silvann {
extern int emu_refused;
void flush_deferred();
}
// library.hip is not part of the emulation: its flush entry point, here
extern "C" void silvann_gfx950_flush(void) { silvann::flush_deferred(); }

namespace {
struct Guarded { char* map; size_t len; char* p; size_t n; const char* name; };
std::vector<Guarded> bufs;

char* guarded(size_t n, const char* name) {
    const size_t pg = 4096, body = (n + pg - 1) / pg * pg, len = body + 2 * pg;
    char* m = (char*)mmap(nullptr, len, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (m == MAP_FAILED) abort();
    mprotect(m, pg, PROT_NONE);
    mprotect(m + pg + body, pg, PROT_NONE);
    char* p = m + pg + body - n;   // the buffer ends at the upper guard page
    bufs.push_back({m, len, p, n, name});
    return p;
}

void on_fault(int sig, siginfo_t* si, void*) {
    char msg[512];
    const char* who = "no buffer";
    long rel = 0;
    for (auto& b : bufs)
        if ((char*)si->si_addr >= b.map && (char*)si->si_addr < b.map + b.len) {
            who = b.name;
            rel = (char*)si->si_addr - b.p;
        }
    const int k = snprintf(msg, sizeof msg, "EMU FAULT signal %d at %p (%s, offset %ld) lane %u block (%u,%u,%u)\n",
                           sig, si->si_addr, who, rel, threadIdx.x, blockIdx.x, blockIdx.y, blockIdx.z);
    (void)!write(2, msg, k);
    void* bt[64];
    backtrace_symbols_fd(bt, backtrace(bt, 64), 2);
    _exit(3);
}

void on_alarm(int) {
    const char m[] = "EMU TIMEOUT (a barrier some lanes never reach?)\n";
    (void)!write(2, m, sizeof m - 1);
    _exit(4);
}

char* load(const std::string& f, const char* name, size_t* n = nullptr) {
    FILE* fp = fopen(f.c_str(), "rb");
    if (!fp) return nullptr;
    fseek(fp, 0, SEEK_END);
    const size_t len = ftell(fp);
    fseek(fp, 0, SEEK_SET);
    char* p = guarded(len, name);
    if (fread(p, 1, len, fp) != len) abort();
    fclose(fp);
    if (n) *n = len;
    return p;
}

void save(const std::string& f, const void* p, size_t n) {
    FILE* fp = fopen(f.c_str(), "wb");
    fwrite(p, 1, n, fp);
    fclose(fp);
}
}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) return 2;
    struct sigaction sa {};
    sa.sa_sigaction = on_fault;
    sa.sa_flags = SA_SIGINFO;
    sigaction(SIGSEGV, &sa, nullptr);
    sigaction(SIGBUS, &sa, nullptr);
    signal(SIGALRM, on_alarm);
    const std::string d = argv[1];
    auto d_dir = [&](unsigned long) { return d; };
    char mode[16];
    unsigned long qh, kvh, hd, a0, a1, ps, pages_row, k_row, timeout;
    FILE* fp = fopen((d + "/params.txt").c_str(), "r");
    if (!fp || fscanf(fp, "%15s %lu %lu %lu %lu %lu %lu %lu %lu %lu", mode, &qh, &kvh, &hd, &a0, &a1, &ps, &pages_row,
                      &k_row, &timeout) != 10)
        return 2;
    fclose(fp);
    alarm((unsigned)timeout);
    size_t qn = 0;
    char* q = load(d + "/q.bin", "q", &qn);
    // EMU_MISALIGN=q: q moved to an address 2 mod 16; =p: the chains' weights buffer at 4 mod 8
    const char* mis = getenv("EMU_MISALIGN");
    const bool mis_q = mis && std::string(mis) == "q", mis_p = mis && std::string(mis) == "p";
    if (mis_q && q) {
        char* m = guarded(qn + 2, "q");   // ends 2 bytes short of the page: starts at 2 mod 16 for qn a multiple of 16
        memcpy(m, q, qn);
        q = m;
    }
    char* k = load(d + "/k.bin", "k");
    char* v = load(d + "/v.bin", "v");
    if (!v) v = k;   // no values of their own: the keys are the values (latent attention)
    char* pages = load(d + "/pages.bin", "pages");
    unsigned int* over = (unsigned int*)guarded(4, "over");
    *over = 0;
    size_t on = 0;
    char* o = nullptr;
    if (std::string(mode) == "causal") {   // a0 = first, a1 = rows
        on = a1 * qh * hd * 2;
        o = guarded(on, "o");
        memset(o, 0xFF, on);   // NaN halves: every answer must be written
        silvann_gfx950_attention_causal_paged((uint16_t*)o, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                                              (const uint32_t*)pages, ps, qh, kvh, hd, a0, a1, over);
    } else if (std::string(mode) == "fp16" || std::string(mode) == "fp16_rows") {
        // fp16: weights then residual_mix over a0 = length keys (one row). fp16_rows: weights_rows then
        // residual_mix_rows, rows a1 from a0 = first. p, the residual after the first door, and after the second.
        const bool many = std::string(mode) == "fp16_rows";
        const unsigned long rows = many ? a1 : 1, rf = hd + 2, span = many ? a0 + a1 : a0;
        float* p = (float*)guarded(rows * qh * span * 4, "p");
        memset(p, 0xFF, rows * qh * span * 4);
        float* res = (float*)guarded(rows * qh * rf * 4, "res");
        memset(res, 0xFF, rows * qh * rf * 4);
        if (many) silvann_gfx950_attention_weights_rows(p, res, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, a0, a1);
        else silvann_gfx950_attention_weights(p, res, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, a0);
        save(d + "/p.bin", p, rows * qh * span * 4);
        save(d + "/res_w.bin", res, rows * qh * rf * 4);
        if (many) silvann_gfx950_attention_residual_mix_rows(res, p, (const uint16_t*)v, qh, kvh, hd, a0, a1);
        else silvann_gfx950_attention_residual_mix(res, p, (const uint16_t*)v, qh, kvh, hd, a0);
        save(d + "/res.bin", res, rows * qh * rf * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "grouped" || std::string(mode) == "grouped_rows") {
        // grouped: scores_grouped, softmax_rows, mix over a0 = length keys. grouped_rows: scores_grouped_rows,
        // softmax_lens, mix_rows, a1 rows over their own lens (file lens) at k + u·k_row, p rows q_heads·a0 apart.
        const bool many = std::string(mode) == "grouped_rows";
        const unsigned long rows = many ? a1 : 1, most = a0;
        const unsigned long p_row = qh * most, o_row = qh * hd;
        float* p = (float*)guarded(rows * p_row * 4, "p");
        memset(p, 0xFF, rows * p_row * 4);
        uint16_t* o16 = (uint16_t*)guarded(rows * o_row * 2, "o");
        memset(o16, 0xFF, rows * o_row * 2);
        if (many) {
            char* lens = load(d + "/lens.bin", "lens");
            silvann_gfx950_attention_scores_grouped_rows(p, p_row, (const uint16_t*)q, o_row, (const uint16_t*)k, k_row,
                                                         (const uint32_t*)lens, qh, kvh, hd, most, rows);
            save(d + "/p.bin", p, rows * p_row * 4);
            silvann_gfx950_attention_softmax_lens(p, p_row, (const uint32_t*)lens, qh, rows);
            save(d + "/p_soft.bin", p, rows * p_row * 4);
            silvann_gfx950_attention_mix_rows(o16, o_row, p, p_row, (const uint16_t*)v, k_row, (const uint32_t*)lens, qh,
                                              kvh, hd, rows, over);
        } else {
            silvann_gfx950_attention_scores_grouped(p, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, most);
            save(d + "/p.bin", p, rows * p_row * 4);
            silvann_gfx950_attention_softmax_rows(p, qh, most);
            save(d + "/p_soft.bin", p, rows * p_row * 4);
            silvann_gfx950_attention_mix(o16, p, (const uint16_t*)v, qh, kvh, hd, most, over);
        }
        save(d + "/o.bin", o16, rows * o_row * 2);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "rope") {
        // rope_rows in place: q holds x, k the angles; qh = heads, hd = head_stride, a1 = rows, ps = rot,
        // k_row = row_stride
        size_t xn = 0;
        char* x = load(d + "/q.bin", "x", &xn);
        silvann_gfx950_rope_rows((uint16_t*)x, (const uint16_t*)x, (const float*)k, a1, qh, hd, k_row, ps, over);
        save(d + "/o.bin", x, xn);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "chain_decode" || std::string(mode) == "chain_weights") {
        // The reference verbs' door chains over a0 = length keys, as the verbs call them (deferred unless
        // SILVANN_GFX950_DEFER=0): scores then mix into o, or weights then residual_mix into res. a1 = 1 puts a
        // merge of an unrelated pair of residuals between the two doors (which must run the first door as it was).
        const unsigned long length = a0, rf = hd + 2;
        float* p = (float*)guarded(qh * length * 4 + (mis_p ? 4 : 0), "p");
        memset(p, 0xFF, qh * length * 4);
        float* res = (float*)guarded(qh * rf * 4, "res");
        memset(res, 0xFF, qh * rf * 4);
        float* other = (float*)guarded(2 * rf * 4, "other");
        memset(other, 0, 2 * rf * 4);
        const bool decode = std::string(mode) == "chain_decode";
        const unsigned long on = qh * hd * 2;
        uint16_t* o16 = (uint16_t*)guarded(on, "o");
        memset(o16, 0xFF, on);
        if (decode) silvann_gfx950_attention_scores(p, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, length);
        else silvann_gfx950_attention_weights(p, res, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, length);
        if (a1 == 1) silvann_gfx950_attention_merge(other, other, other + rf, 1, hd);
        if (decode) silvann_gfx950_attention_mix(o16, p, (const uint16_t*)v, qh, kvh, hd, length, over);
        else silvann_gfx950_attention_residual_mix(res, p, (const uint16_t*)v, qh, kvh, hd, length);
        silvann_gfx950_flush();
        save(d + "/o.bin", o16, on);
        save(d + "/p.bin", p, qh * length * 4);
        save(d + "/res.bin", res, qh * rf * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode).rfind("cres_", 0) == 0) {
        // the residual chains (a0 = first or length, a1 = rows, ps = d, pages_row = 1: another door in between);
        // TurboQuant: k / v the codes, pages / lens the key / value scales
        const std::string kind = std::string(mode).substr(5);   // rows, tq or tqr
        const unsigned long rows = a1, rf = hd + 2, span = kind == "rows" ? a0 + a1 : a0;
        float* p = (float*)guarded(rows * qh * span * 4, "p");
        memset(p, 0xFF, rows * qh * span * 4);
        float* res = (float*)guarded(rows * qh * rf * 4, "res");
        memset(res, 0xFF, rows * qh * rf * 4);
        char* vs = load(d + "/lens.bin", "v_scales");
        if (kind == "rows")
            silvann_gfx950_attention_weights_rows(p, res, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, a0, rows);
        else if (kind == "tq")
            silvann_gfx950_attention_weights_tq(p, res, (const uint16_t*)q, (const uint8_t*)k, (const uint16_t*)pages, qh,
                                                kvh, hd, a0, ps);
        else
            silvann_gfx950_attention_weights_tq_rows(p, res, (const uint16_t*)q, (const uint8_t*)k,
                                                     (const uint16_t*)pages, qh, kvh, hd, a0, ps, rows);
        if (pages_row == 1) silvann_gfx950_attention_finish(nullptr, nullptr, 0, hd, over);
        if (kind == "rows")
            silvann_gfx950_attention_residual_mix_rows(res, p, (const uint16_t*)v, qh, kvh, hd, a0, rows);
        else if (kind == "tq")
            silvann_gfx950_attention_residual_mix_tq(res, p, (const uint8_t*)v, (const uint16_t*)vs, qh, kvh, hd, a0, ps);
        else
            silvann_gfx950_attention_residual_mix_tq_rows(res, p, (const uint8_t*)v, (const uint16_t*)vs, qh, kvh, hd, a0,
                                                          ps, rows);
        silvann_gfx950_flush();
        save(d + "/p.bin", p, rows * qh * span * 4);
        save(d + "/res.bin", res, rows * qh * rf * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "chain_grp") {
        // scores_grouped, softmax_rows (a1 = 0) or softmax_sink (a1 = 1, the sink in lens.bin), mix over a0 keys;
        // ps = 1 puts another door between the softmax and the mix
        const unsigned long length = a0;
        float* p = (float*)guarded(qh * length * 4, "p");
        memset(p, 0xFF, qh * length * 4);
        char* sink = a1 ? load(d + "/lens.bin", "sink") : nullptr;
        const unsigned long on = qh * hd * 2;
        uint16_t* o16 = (uint16_t*)guarded(on, "o");
        memset(o16, 0xFF, on);
        silvann_gfx950_attention_scores_grouped(p, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, length);
        if (a1) silvann_gfx950_attention_softmax_sink(p, (const uint16_t*)sink, qh, length);
        else silvann_gfx950_attention_softmax_rows(p, qh, length);
        if (ps == 1) silvann_gfx950_attention_finish(nullptr, nullptr, 0, hd, over);
        silvann_gfx950_attention_mix(o16, p, (const uint16_t*)v, qh, kvh, hd, length, over);
        silvann_gfx950_flush();
        save(d + "/o.bin", o16, on);
        save(d + "/p.bin", p, qh * length * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "chain_grows") {
        // scores_grouped_rows, softmax_lens, mix_rows: a1 rows over their own lens (lens.bin) of at most a0 keys, at
        // k + u·k_row; ps = 1 puts another door between the softmax and the mix
        const unsigned long rows = a1, most = a0, p_row = qh * most, o_row = qh * hd;
        char* lens = load(d + "/lens.bin", "lens");
        float* p = (float*)guarded(rows * p_row * 4, "p");
        memset(p, 0xFF, rows * p_row * 4);
        const unsigned long on = rows * o_row * 2;
        uint16_t* o16 = (uint16_t*)guarded(on, "o");
        memset(o16, 0xFF, on);
        silvann_gfx950_attention_scores_grouped_rows(p, p_row, (const uint16_t*)q, o_row, (const uint16_t*)k, k_row,
                                                     (const uint32_t*)lens, qh, kvh, hd, most, rows);
        silvann_gfx950_attention_softmax_lens(p, p_row, (const uint32_t*)lens, qh, rows);
        if (ps == 1) silvann_gfx950_attention_finish(nullptr, nullptr, 0, hd, over);
        silvann_gfx950_attention_mix_rows(o16, o_row, p, p_row, (const uint16_t*)v, k_row, (const uint32_t*)lens, qh,
                                          kvh, hd, rows, over);
        silvann_gfx950_flush();
        save(d + "/o.bin", o16, on);
        save(d + "/p.bin", p, rows * p_row * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "chain_causal") {
        // causal_scores_grouped, causal_softmax, causal_mix from a0 = first over a1 = rows, as nn__attention__rows
        // calls them; ps = 1 puts another door (a finish of nothing) between the softmax and the mix
        const unsigned long first = a0, rows = a1, span = first + rows;
        float* p = (float*)guarded(rows * qh * span * 4, "p");
        memset(p, 0xFF, rows * qh * span * 4);
        const unsigned long on = rows * qh * hd * 2;
        uint16_t* o16 = (uint16_t*)guarded(on, "o");
        memset(o16, 0xFF, on);
        silvann_gfx950_attention_causal_scores_grouped(p, (const uint16_t*)q, (const uint16_t*)k, qh, kvh, hd, first,
                                                       rows);
        silvann_gfx950_attention_causal_softmax(p, qh, first, rows);
        if (ps == 1) silvann_gfx950_attention_finish(nullptr, nullptr, 0, hd, over);
        silvann_gfx950_attention_causal_mix(o16, p, (const uint16_t*)v, qh, kvh, hd, first, rows, over);
        silvann_gfx950_flush();
        save(d + "/o.bin", o16, on);
        save(d + "/p.bin", p, rows * qh * span * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "cache") {
        // qh = rot, a0 = rows_per_seq, a1 = rows, k_row = capacity; q holds the angles (fp32), lens the positions,
        // kc / vc the caches as they were
        size_t kn = 0, vn = 0;
        char* kc = load(d + "/kc.bin", "k_cache", &kn);
        char* vc = load(d + "/vc.bin", "v_cache", &vn);
        char* lens = load(d + "/lens.bin", "positions");
        silvann_gfx950_attention_cache_write_paged((uint16_t*)kc, (uint16_t*)vc, (const uint32_t*)pages, pages_row, ps,
                                                   k_row, (const uint32_t*)lens, a0, (const uint16_t*)k,
                                                   (const uint16_t*)v, (const float*)q, qh, a1, kvh, hd, over);
        save(d + "/kc_out.bin", kc, kn);
        save(d + "/vc_out.bin", vc, vn);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "causal_res") {   // a0 = first, a1 = rows
        const unsigned long rf = hd + 2;
        float* res = (float*)guarded(a1 * qh * rf * 4, "res");
        memset(res, 0xFF, a1 * qh * rf * 4);   // whatever the caller's residual held
        silvann_gfx950_attention_causal_residual_paged(res, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                                                       (const uint32_t*)pages, ps, qh, kvh, hd, a0, a1);
        save(d + "/res.bin", res, a1 * qh * rf * 4);
        save(d + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "tq_fused") {
        // a0 = length, a1 = rows, ps = d; k / v the codes, pages / lens the key / value scales
        const unsigned long length = a0, rows = a1, d = ps, rf = hd + 2;
        char* ksc = pages;
        char* vsc = load(d_dir(0) + "/lens.bin", "v_scales");
        float* res = (float*)guarded(rows * qh * rf * 4, "res");
        memset(res, 0xFF, rows * qh * rf * 4);
        const uint64_t sb = silvann_gfx950_attention_residual_tq_scratch(qh, kvh, hd, length, d, rows);
        float* scratch = (float*)guarded(sb ? sb : 4, "scratch");
        memset(scratch, 0xFF, sb ? sb : 4);
        silvann_gfx950_attention_residual_tq(res, (const uint16_t*)q, (const uint8_t*)k, (const uint16_t*)ksc,
                                             (const uint8_t*)v, (const uint16_t*)vsc, qh, kvh, hd, length, d, rows,
                                             scratch);
        save(d_dir(0) + "/res.bin", res, rows * qh * rf * 4);
        save(d_dir(0) + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else if (std::string(mode) == "tq" || std::string(mode) == "tq_rows") {
        // a0 = length, a1 = rows, ps = d; k holds the codes, v the scales
        const unsigned long length = a0, rows = a1, d = ps, rf = hd + 2;
        float* p = (float*)guarded((rows * qh * length + 1) * 4, "p");
        float* res = (float*)guarded(rows * qh * rf * 4, "res");
        memset(res, 0xFF, rows * qh * rf * 4);   // whatever the caller's residual held
        if (std::string(mode) == "tq")
            silvann_gfx950_attention_weights_tq(p, res, (const uint16_t*)q, (const uint8_t*)k, (const uint16_t*)v, qh, kvh,
                                                hd, length, d);
        else
            silvann_gfx950_attention_weights_tq_rows(p, res, (const uint16_t*)q, (const uint8_t*)k, (const uint16_t*)v,
                                                     qh, kvh, hd, length, d, rows);
        save(d_dir(d) + "/p.bin", p, rows * qh * length * 4);
        save(d_dir(d) + "/res_w.bin", res, rows * qh * rf * 4);
        if (std::string(mode) == "tq")
            silvann_gfx950_attention_residual_mix_tq(res, p, (const uint8_t*)k, (const uint16_t*)v, qh, kvh, hd, length, d);
        else
            silvann_gfx950_attention_residual_mix_tq_rows(res, p, (const uint8_t*)k, (const uint16_t*)v, qh, kvh, hd, length,
                                                          d, rows);
        save(d_dir(d) + "/res.bin", res, rows * qh * rf * 4);
        save(d_dir(d) + "/over.bin", over, 4);
        fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
        return silvann::emu_refused ? 5 : 0;
    } else {                               // a0 = most, a1 = rows
        char* lens = load(d + "/lens.bin", "lens");
        on = a1 * qh * hd * 2;
        o = guarded(on, "o");
        memset(o, 0xFF, on);   // NaN halves: every answer must be written
        const uint64_t sb = silvann_gfx950_attention_decode_paged_scratch(qh, kvh, hd, a0, a1);
        float* scratch = (float*)guarded(sb ? sb : 4, "scratch");
        memset(scratch, 0xFF, sb ? sb : 4);   // whatever a caller's scratch held before
        // EMU_REPEAT: a first call with every query negated, then the call whose answers are kept, over the scratch
        // the first left (its partials differ from the second's), the answers cleared between
        const int calls = getenv("EMU_REPEAT") ? 2 : 1;
        std::vector<uint16_t> decoy((const uint16_t*)q, (const uint16_t*)q + a1 * qh * hd);
        for (uint16_t& h : decoy) h ^= 0x8000u;
        for (int c = 0; c < calls; ++c) {
            if (c) memset(o, 0xFF, on);
            const uint16_t* qc = c + 1 < calls ? decoy.data() : (const uint16_t*)q;
            silvann_gfx950_attention_decode_paged((uint16_t*)o, qc, (const uint16_t*)k, (const uint16_t*)v,
                                                  (const uint32_t*)pages, pages_row, ps, k_row, (const uint32_t*)lens, qh,
                                                  kvh, hd, a0, a1, scratch, over);
        }
    }
    save(d + "/o.bin", o, on);
    save(d + "/over.bin", over, 4);
    fprintf(stderr, "emu done: refused %d, wave exchanges %ld\n", silvann::emu_refused, (long)emu::ops);
    return silvann::emu_refused ? 5 : 0;
}
