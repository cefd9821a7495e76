/* silvann_gfx950_attention.h — the C ABI of the MI355X (gfx950) attention library.
 *
 * Every entry point takes plain device pointers and sizes. All device pointers are addresses in the
 * calling thread's current HIP device; every door is asynchronous on the library's stream for the calling
 * thread (the legacy null stream unless `silvann_gfx950_set_stream` named another), returns once its kernels
 * are queued, and allocates nothing the caller can see (the reference doors' rule).
 *
 * Layouts are the reference's:
 *   q      [q_heads][head_dim] fp16 (decode), [rows][q_heads][head_dim] (causal)
 *   k, v   [position][kv_heads][head_dim] fp16, query head h reading kv head h / (q_heads / kv_heads)
 *   p      fp32 weights, a query head's row `length` long
 *   res    fp32 residual a query head: [m, l, acc[head_dim]]  (head_dim + 2 floats)
 *   over   the worker's fault word: a door whose fp16 answer overflows stores 0x4E504F56 ("NPOV") there
 *
 * The first block of doors has exactly the signature of a row of the reference's nn door table
 * (engine/src/packages/nn/contracts/abi/gpu.cuh, `nn__CONTRACT__DOORS`); each comment cites the row
 * and the generic body whose arithmetic it reproduces (engine/src/packages/nn/gpu/kernels/kernels.cuh).
 * `SILVANN_GFX950_ROW_*` is that row's index in the table (a pointer slot after the table's uint32 size). */
#ifndef SILVANN_GFX950_ATTENTION_H
#define SILVANN_GFX950_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── rows of the reference's nn door table ─────────────────────────────────────────────────────── */

/* gpu.cuh:119 attention_scores — kernels.cuh:1133-1141 (+ scores_head 894-915): p[h][t] = softmax_t(q_h·k_t / sqrt(hd)) */
#define SILVANN_GFX950_ROW_ATTENTION_SCORES 25u
void silvann_gfx950_attention_scores(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                     uint64_t kv_heads, uint64_t head_dim, uint64_t length);
/* gpu.cuh:120 attention_mix — kernels.cuh:1156-1164 (+ mix_head 1144-1154): o[h][e] = fp16(Σ_t p[h][t] v_t[e]) */
#define SILVANN_GFX950_ROW_ATTENTION_MIX 26u
void silvann_gfx950_attention_mix(uint16_t* o, const float* p, const uint16_t* v, uint64_t q_heads,
                                  uint64_t kv_heads, uint64_t head_dim, uint64_t length, unsigned int* over);
/* gpu.cuh:122 attention_weights — kernels.cuh:1190-1221: p = e^(s - m) unnormalised, res[h] = {m, l} */
#define SILVANN_GFX950_ROW_ATTENTION_WEIGHTS 28u
void silvann_gfx950_attention_weights(float* p, float* res, const uint16_t* q, const uint16_t* k,
                                      uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length);
/* gpu.cuh:123 attention_residual_mix — kernels.cuh:1224-1238: res[h].acc[e] = Σ_t p[h][t] v_t[e] */
#define SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX 29u
void silvann_gfx950_attention_residual_mix(float* res, const float* p, const uint16_t* v, uint64_t q_heads,
                                           uint64_t kv_heads, uint64_t head_dim, uint64_t length);
/* gpu.cuh:124 attention_merge — kernels.cuh:1243-1255: two residuals into one; `into` may be `a` or `b` */
#define SILVANN_GFX950_ROW_ATTENTION_MERGE 30u
void silvann_gfx950_attention_merge(float* into, const float* a, const float* b, uint64_t q_heads,
                                    uint64_t head_dim);
/* gpu.cuh:125 attention_finish — kernels.cuh:1258-1267: o = fp16(acc / l) */
#define SILVANN_GFX950_ROW_ATTENTION_FINISH 31u
void silvann_gfx950_attention_finish(uint16_t* o, const float* res, uint64_t q_heads, uint64_t head_dim,
                                     unsigned int* over);
/* gpu.cuh:155 attention_causal_scores — kernels.cuh:2039-2049: row r (position first + r) over keys 0..first+r,
 * weights at p + (r·q_heads + h)·(first + rows) */
#define SILVANN_GFX950_ROW_ATTENTION_CAUSAL_SCORES 61u
void silvann_gfx950_attention_causal_scores(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                            uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows);
/* gpu.cuh:156 attention_causal_mix — kernels.cuh:2051-2060 */
#define SILVANN_GFX950_ROW_ATTENTION_CAUSAL_MIX 62u
void silvann_gfx950_attention_causal_mix(uint16_t* o, const float* p, const uint16_t* v, uint64_t q_heads,
                                         uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows,
                                         unsigned int* over);
/* gpu.cuh:163 attention_weights_tq — kernels.cuh:2963-3000: attention_weights over TurboQuant keys. Key row t of kv
 * head g is row t·kv_heads + g of `codes` (ceil(head_dim / (16/d)) 16-bit containers, little-endian, value c at
 * bit d·(c % (16/d)) of container c / (16/d)) and `scales` (fp16); value c means level_d[code] · scale, level_d the
 * reference's table for width d (kernels.cuh:2264-2354, 2650-2653). d is 1, 2, 3, 4, 5 or 8; `codes` 2-byte
 * aligned; other operands are refused. `q` is already rotated (the caller's). */
#define SILVANN_GFX950_ROW_ATTENTION_WEIGHTS_TQ 69u
void silvann_gfx950_attention_weights_tq(float* p, float* res, const uint16_t* q, const uint8_t* codes,
                                         const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads,
                                         uint64_t head_dim, uint64_t length, uint64_t d);
/* gpu.cuh:164 attention_residual_mix_tq — kernels.cuh:3005-3026: res[h].acc[e] = Σ_t p[h][t] · value_t[e] over
 * TurboQuant values. As the reference allows (kernels.cuh:3001-3003), the door keeps partial sums in `p` once it has
 * read it: `p` holds no weights afterwards. */
#define SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX_TQ 70u
void silvann_gfx950_attention_residual_mix_tq(float* res, const float* p, const uint8_t* codes,
                                              const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads,
                                              uint64_t head_dim, uint64_t length, uint64_t d);
/* gpu.cuh:189 attention_scores_grouped — kernels.cuh:928-948: raw scaled scores, no softmax */
#define SILVANN_GFX950_ROW_ATTENTION_SCORES_GROUPED 95u
void silvann_gfx950_attention_scores_grouped(float* p, const uint16_t* q, const uint16_t* k, uint64_t q_heads,
                                             uint64_t kv_heads, uint64_t head_dim, uint64_t length);
/* gpu.cuh:190 attention_softmax_rows — kernels.cuh:1085-1100: each of `rows` rows (`length` apart) its softmax */
#define SILVANN_GFX950_ROW_ATTENTION_SOFTMAX_ROWS 96u
void silvann_gfx950_attention_softmax_rows(float* p, uint64_t rows, uint64_t length);
/* gpu.cuh:191 attention_causal_scores_grouped — kernels.cuh:1028-1061: raw scaled causal scores */
#define SILVANN_GFX950_ROW_ATTENTION_CAUSAL_SCORES_GROUPED 97u
void silvann_gfx950_attention_causal_scores_grouped(float* p, const uint16_t* q, const uint16_t* k,
                                                    uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                    uint64_t first, uint64_t rows);
/* gpu.cuh:192 attention_causal_softmax — kernels.cuh:1065-1081 */
#define SILVANN_GFX950_ROW_ATTENTION_CAUSAL_SOFTMAX 98u
void silvann_gfx950_attention_causal_softmax(float* p, uint64_t q_heads, uint64_t first, uint64_t rows);
/* gpu.cuh:201 attention_softmax_sink — kernels.cuh:1115-1131: each of `rows` rows (`length` apart) its softmax with
 * a sink, the sum taking one more term e^(sink[r]) (fp16) that weighs no position (DeepSeek V4's attention) */
#define SILVANN_GFX950_ROW_ATTENTION_SOFTMAX_SINK 107u
void silvann_gfx950_attention_softmax_sink(float* p, const uint16_t* sink, uint64_t rows, uint64_t length);
/* gpu.cuh:195 attention_weights_rows — doors.cuh:201-204,417-424 (attention_weights a row at a time) */
#define SILVANN_GFX950_ROW_ATTENTION_WEIGHTS_ROWS 101u
void silvann_gfx950_attention_weights_rows(float* p, float* res, const uint16_t* q, const uint16_t* k,
                                           uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                           uint64_t first, uint64_t rows);
/* gpu.cuh:196 attention_residual_mix_rows — doors.cuh:425-432 */
#define SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX_ROWS 102u
void silvann_gfx950_attention_residual_mix_rows(float* res, const float* p, const uint16_t* v, uint64_t q_heads,
                                                uint64_t kv_heads, uint64_t head_dim, uint64_t first,
                                                uint64_t rows);
/* gpu.cuh:197 attention_weights_tq_rows — doors.cuh:203,433-441: weights_tq for `rows` queries over the same keys,
 * row r's q at q + r·q_heads·head_dim, weights at p + r·q_heads·length, residuals at res + r·q_heads·(head_dim + 2) */
#define SILVANN_GFX950_ROW_ATTENTION_WEIGHTS_TQ_ROWS 103u
void silvann_gfx950_attention_weights_tq_rows(float* p, float* res, const uint16_t* q, const uint8_t* codes,
                                              const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads,
                                              uint64_t head_dim, uint64_t length, uint64_t d, uint64_t rows);
/* gpu.cuh:198 attention_residual_mix_tq_rows — doors.cuh:204,442-450 (p holds no weights afterwards, as above) */
#define SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX_TQ_ROWS 104u
void silvann_gfx950_attention_residual_mix_tq_rows(float* res, const float* p, const uint8_t* codes,
                                                   const uint16_t* scales, uint64_t q_heads, uint64_t kv_heads,
                                                   uint64_t head_dim, uint64_t length, uint64_t d, uint64_t rows);
/* gpu.cuh:222 attention_scores_grouped_rows — kernels.cuh:953-972: row u's lens[u] keys at k + u·k_row */
#define SILVANN_GFX950_ROW_ATTENTION_SCORES_GROUPED_ROWS 128u
void silvann_gfx950_attention_scores_grouped_rows(float* p, uint64_t p_row, const uint16_t* q, uint64_t q_row,
                                                  const uint16_t* k, uint64_t k_row, const uint32_t* lens,
                                                  uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                  uint64_t most, uint64_t rows);
/* gpu.cuh:223 attention_softmax_lens — kernels.cuh:1104-1110 */
#define SILVANN_GFX950_ROW_ATTENTION_SOFTMAX_LENS 129u
void silvann_gfx950_attention_softmax_lens(float* p, uint64_t p_row, const uint32_t* lens, uint64_t heads,
                                           uint64_t rows);
/* gpu.cuh:224 attention_mix_rows — kernels.cuh:1169-1178 */
#define SILVANN_GFX950_ROW_ATTENTION_MIX_ROWS 130u
void silvann_gfx950_attention_mix_rows(uint16_t* o, uint64_t o_row, const float* p, uint64_t p_row,
                                       const uint16_t* v, uint64_t v_row, const uint32_t* lens, uint64_t q_heads,
                                       uint64_t kv_heads, uint64_t head_dim, uint64_t rows, unsigned int* over);

/* gpu.cuh:140 rope_rows — kernels.cuh:1710-1726: each of `rows` rows (row_stride halves apart) has its `heads` heads
 * (head_stride apart) turned by its own angles at cs + r·rot (rot/2 cosines, then rot/2 sines): elements k and
 * k + rot/2 of a head become a·c − b·s and b·c + a·s — as the reference's host build computes them, fma(a, c, −(b·s))
 * and fma(b, c, a·s) — rounded to fp16, overflow storing NPOV in `over`. `o` may be `x`. The RoPE the rows verb
 * turns its chunk's queries and keys with (attention__abi.cuh:403-406). */
#define SILVANN_GFX950_ROW_ROPE_ROWS 46u
void silvann_gfx950_rope_rows(uint16_t* o, const uint16_t* x, const float* cs, uint64_t rows, uint64_t heads,
                              uint64_t head_stride, uint64_t row_stride, uint64_t rot, unsigned int* over);

/* The nn door table's row count at ABI version 9 (gpu.cuh:93-230): new rows are appended after it. */
#define SILVANN_GFX950_NN_ROWS 137u

/* ── rows appended after the reference's table (gpu.cuh:86-88: rows are only ever appended) ──────────
 * The reference has no paged cache (its KV is one contiguous `[position][kv_head][head_dim]` plane a layer).
 * These rows take a cache pool of pages, each `page_size` positions × kv_heads × head_dim fp16 (K and V in
 * pools of their own), and a page table: logical page `j` of row `u` is physical page `pages[u·pages_row + j]`.
 * `pages` NULL means the cache is contiguous, as the reference's (then `k`/`v` for row u start at
 * `u·k_row` halves; `page_size` and `pages_row` are ignored). Their answers are the reference's attention over
 * the gathered-contiguous cache (decode: `attention_scores` + `attention_mix`; causal: `causal_scores` +
 * `causal_mix`). */

/* One query position a row over its own cache: row u's q_heads at q + u·q_heads·head_dim attend positions
 * 0 .. lens[u]-1; out o + u·q_heads·head_dim. Split-K flash decoding: `scratch` holds the partial residuals,
 * `silvann_gfx950_attention_decode_paged_scratch` bytes (0 if it needs none). `page_size` a multiple of 16
 * positions (of 32 for the causal row). `most` is the largest lens[u]
 * (a bound the grid is sized by; lens[u] <= most is the caller's promise). A row with lens[u] == 0 answers 0.
 * q, k and v 16-byte aligned, k_row a multiple of 8 halves and scratch 8-byte aligned; other operands are
 * refused (nothing launched, the refusal remembered for silvann_gfx950_launch_failed).
 * Split-K form of the reference's decode verb (engine/src/packages/nn/cpu/opcodes/attention__abi.cuh:129-160),
 * many rows as `attention_scores_grouped_rows` (gpu.cuh:222) takes them. */
#define SILVANN_GFX950_ROW_ATTENTION_DECODE_PAGED 137u
void silvann_gfx950_attention_decode_paged(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const uint32_t* pages, uint64_t pages_row, uint64_t page_size,
                                           uint64_t k_row, const uint32_t* lens, uint64_t q_heads,
                                           uint64_t kv_heads, uint64_t head_dim, uint64_t most, uint64_t rows,
                                           float* scratch, unsigned int* over);
uint64_t silvann_gfx950_attention_decode_paged_scratch(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                       uint64_t most, uint64_t rows);

/* Causal prefill of `rows` new positions first .. first+rows-1 over the cache, which already holds their
 * keys and values and the `first` before them: row r's q_heads at q + r·q_heads·head_dim attend positions
 * 0 .. first + r; out o + r·q_heads·head_dim. One sequence (page table `pages`, `pages` NULL for a contiguous
 * cache). The fused form of `attention_causal_scores_grouped` + `attention_causal_softmax` +
 * `attention_causal_mix` (gpu.cuh:191,192,156) as the reference's `nn__attention__rows` runs them
 * (attention__abi.cuh:407-414), on fp16 MFMA with fp32 accumulation; no weights are materialised.
 * first + rows < 2^31, page_size a multiple of 32 below 2^31, q, k and v 16-byte aligned; other shapes are
 * refused (nothing launched,
 * the refusal remembered for silvann_gfx950_launch_failed). */
#define SILVANN_GFX950_ROW_ATTENTION_CAUSAL_PAGED 138u
void silvann_gfx950_attention_causal_paged(uint16_t* o, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const uint32_t* pages, uint64_t page_size, uint64_t q_heads,
                                           uint64_t kv_heads, uint64_t head_dim, uint64_t first, uint64_t rows,
                                           unsigned int* over);

/* The causal residual of row 138: what `attention_weights_rows` + `attention_residual_mix_rows` (gpu.cuh:195-196;
 * doors.cuh:201-204,417-432, a row at a time) leave in `res` with `first` — row r's q_heads at
 * q + r·q_heads·head_dim over positions 0 .. first + r, its residuals {m, l, acc[head_dim]} at
 * res + r·q_heads·(head_dim + 2) — over a paged or contiguous cache as row 138 takes it. The tiered prefill
 * window's part (prefill__abi.cuh:420-435, part 0) in one MFMA launch and without the weights. m is the row's
 * largest scaled score. Shapes as row 138; other operands (and a NULL res) are refused. */
#define SILVANN_GFX950_ROW_ATTENTION_CAUSAL_RESIDUAL_PAGED 140u
void silvann_gfx950_attention_causal_residual_paged(float* res, const uint16_t* q, const uint16_t* k,
                                                    const uint16_t* v, const uint32_t* pages, uint64_t page_size,
                                                    uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                    uint64_t first, uint64_t rows);

/* New key and value rows into their cache slots, the keys turned by RoPE: the reference's `rope_rows` (gpu.cuh:140,
 * kernels.cuh:1710-1726) pointed at the cache rows, and the value projection's placement, as its rows verb does them
 * (attention__abi.cuh:398-406; the reference has no writer verb, 13-14 P2) — over a paged cache. Row r (k and v at
 * + r·kv_heads·head_dim) belongs to sequence u = r / rows_per_seq at position positions[u] + r % rows_per_seq
 * (`positions` a device array of a uint32 a sequence: a prefill chunk is one sequence of `rows` rows; a decode batch is
 * `rows` sequences of one row). Its slot is page pages[u·pages_row + position / page_size], offset position %
 * page_size, of pools laid out as rows 137-138 take them; `pages` NULL: sequence u's cache is contiguous at
 * u·capacity positions. The key's first `rot` elements are turned by row r's angles at cs + r·rot (rot/2 cosines,
 * then rot/2 sines; the pairs x[k], x[k + rot/2]): a·c − b·s and b·c + a·s in fp32, rounded to fp16, overflow storing
 * NPOV in `over`; the rest of the key and the value are copied bit for bit. `cs` NULL: no turn. A row at or past
 * `capacity` positions is written nowhere and stores NPBN ("NPBN", primitives.cuh:5) in `over`. Refused (nothing
 * launched): rot odd or past head_dim, pages_row < ⌈capacity / page_size⌉, a NULL operand. */
#define SILVANN_GFX950_ROW_ATTENTION_CACHE_WRITE_PAGED 141u
void silvann_gfx950_attention_cache_write_paged(uint16_t* k_cache, uint16_t* v_cache, const uint32_t* pages,
                                                uint64_t pages_row, uint64_t page_size, uint64_t capacity,
                                                const uint32_t* positions, uint64_t rows_per_seq, const uint16_t* k,
                                                const uint16_t* v, const float* cs, uint64_t rot, uint64_t rows,
                                                uint64_t kv_heads, uint64_t head_dim, unsigned int* over);

/* The TurboQuant residual in one pass: what `attention_weights_tq` + `attention_residual_mix_tq` (gpu.cuh:163-164)
 * leave in `res`, for `rows` query rows over the same `length` TurboQuant key and value rows — row u's q_heads at
 * q + u·q_heads·head_dim, its residuals at res + u·q_heads·(head_dim + 2) — as `attention_weights_tq_rows` +
 * `attention_residual_mix_tq_rows` (gpu.cuh:197-198) give them. Codes as in row 69; d is 4 or 8 (the tiers' widths,
 * attention__abi.cuh:258); head_dim 64, 128 or 256; the code planes 8-byte and q 16-byte aligned; other operands
 * are refused.
 * Split-K on MFMA: no weights are materialised and every code is read once. `scratch` holds the splits' residuals,
 * `silvann_gfx950_attention_residual_tq_scratch` bytes. The tiers' verbs call weights_tq then residual_mix_tq then
 * merge (mixer__abi.cuh:395-410); this row replaces the first two. */
#define SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_TQ 139u
void silvann_gfx950_attention_residual_tq(float* res, const uint16_t* q, const uint8_t* k_codes,
                                          const uint16_t* k_scales, const uint8_t* v_codes, const uint16_t* v_scales,
                                          uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim, uint64_t length,
                                          uint64_t d, uint64_t rows, float* scratch);
uint64_t silvann_gfx950_attention_residual_tq_scratch(uint64_t q_heads, uint64_t kv_heads, uint64_t head_dim,
                                                      uint64_t length, uint64_t d, uint64_t rows);

/* Puts this library's rows into an nn door table: `nn_doors` is the reference's `nn__doors` (a uint32 `size`
 * in bytes, then one function pointer a row from byte 8, gpu.cuh:93-241; entry.cuh:33-45 fills it). Every row
 * above whose index the table's size reaches is overwritten with this library's door, as a family's
 * override step does (amd_rocm_base/overrides/doors.cuh:20 `amd_rocm_base__override_doors`, called once
 * from entry.cuh:72-78); rows past its size are left alone — an older table does not grow. Answers the number
 * of rows written; 0 for a NULL table. */
uint32_t silvann_gfx950_attention_install(void* nn_doors);

/* ── library control (no reference counterpart: the reference family's launch and sys doors do this) ── */

/* The stream the calling thread's doors are queued on (a hipStream_t; NULL is the legacy null stream, the
 * reference family's choice, amd_rocm_base/nn.cuh:25-34). Thread-local, as a runner thread is a worker's. */
void silvann_gfx950_set_stream(void* stream);
void* silvann_gfx950_get_stream(void);
/* Deferred chains. The reference's verbs call some doors only back to back on one thread — attention_scores then
 * attention_mix (attention__abi.cuh:155-158), attention_weights then attention_residual_mix (203-206),
 * attention_causal_scores_grouped then attention_causal_softmax then attention_causal_mix (407-414). By default this
 * library records such a chain's first doors instead of launching them; when the continuation arrives on the same
 * thread and stream with the same operands, the chain runs as one fused kernel (the split-K decode of row 137, the
 * causal prefill of row 138) and the weights buffer `p` never holds weights (the decode pairs use it as their
 * scratch; the fused forms run only when q, k and v are 16-byte aligned and `p` 8-byte aligned, else the doors run
 * one by one). Any other door of this library — and set_stream, launch_failed, flush — first runs what is recorded
 * exactly as the door would have run, so any other order of calls keeps the reference's semantics. A caller that
 * reads `p` itself after a chain's first door, or that calls a door of another library in between, calls
 * silvann_gfx950_flush() first, or switches deferral off for its thread; so does a family's wait (compute_completed)
 * before it synchronises, and a thread before it ends. SILVANN_GFX950_DEFER=0 makes off the process default. (No
 * counterpart in the reference: the fusion its door ABI leaves no single door for.) */
void silvann_gfx950_flush(void);
void silvann_gfx950_set_defer(int on);
/* Nonzero if a door on the current device refused its operands or failed to launch since the last call; clears
 * it. Kept per device, not per thread, as the reference family keeps it (the next compute_completed on that
 * device answers false, amd_rocm_base/sys.cuh:39-62 and amd_rocm_base/nn.cuh:29-33). */
int silvann_gfx950_launch_failed(void);
/* Live kernel timing: with profiling on, this thread's doors bracket their main kernels with hipEvents on
 * their stream. `kernel` is "decode_split", "decode_merge", "causal_mfma", "tq_split" or "cache_write"; read synchronises, answers the
 * summed milliseconds and the launch count since the last read, and clears them. Answers -1 for an unknown
 * name or a failed event. */
void silvann_gfx950_profile_enable(int on);
int silvann_gfx950_profile_read(const char* kernel, double* total_ms, uint64_t* launches);
/* The library's build: "gfx950 <kernels> <version>". */
const char* silvann_gfx950_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SILVANN_GFX950_ATTENTION_H */
