/* mc_kv.h - C ABI of the paged KV-cache hot path in libminicpm_native.so
 * (MI355X / gfx950 build).
 *
 * These entry points are the plain-pointer equivalents of the reference's
 * internal launcher boundary (native/kernels/sm120/kernels.h) and of its
 * PagedKvAllocator (native/runtime/kv_cache.h:68-104). Each declaration cites
 * the reference interface it replaces. Conventions kept from the reference:
 *   - bf16 values travel as uint16_t bit patterns;
 *   - positions / decode limits are read from a DEVICE address at kernel run
 *     time (so a captured graph replays with new positions);
 *   - argument checks return MC_E_INVALID_ARGUMENT, launch failures MC_E_CUDA,
 *     and set the thread-local message returned by mc_last_error();
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *
 * Model geometry is fixed as in the reference (generated_model_config.h):
 * 16 query heads, 2 KV heads (GQA group 8), head_dim 128. A qkv row is 2560
 * bf16: q in columns 0..2047, k in 2048..2303, v in 2304..2559.
 *
 * Pool layout (reference kv_cache.h:29-66 with the page size as a parameter):
 *   element offset = (((layer*max_pages + page)*P + slot)*512 + kv*256
 *                     + head*128 + d)           (bf16 elements)
 *   pos -> page = page_table[pos / P], slot = pos % P.
 */
#ifndef MC_KV_H_
#define MC_KV_H_

#include <stddef.h>
#include <stdint.h>

#include "minicpm_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Exported even when the library is built with -fvisibility=hidden. */
#pragma GCC visibility push(default)

#define MC_KV_Q_HEADS 16u
#define MC_KV_KV_HEADS 2u
#define MC_KV_HEAD_DIM 128u
#define MC_KV_QKV_ROW 2560u
#define MC_KV_PARTIAL_STRIDE 130u /* {m, l, acc[128]} fp32 (kernels.h:277) */
#define MC_KV_MERGE_SPLIT2 32u    /* level-2 merge splits (kernels.h:283) */

/* Pool geometry passed by value. The reference fixes tokens_per_page = 32 and
 * num_layers = 42 at compile time (kv_cache.h:30, :63-65); here both are
 * runtime values. tokens_per_page must be a power of two in [1, 4096]. */
typedef struct mc_kv_layout_t {
    uint32_t max_pages;       /* pages per layer */
    uint32_t tokens_per_page; /* P */
    uint32_t num_layers;      /* L */
    uint32_t reserved;        /* must be 0 */
} mc_kv_layout_t;

/* ---- addressing (host-only, integer) ---- */

/* KvLayout::elem_offset (kv_cache.h:40-45). Returns UINT64_MAX on a bad layout. */
uint64_t mc_kv_elem_offset(mc_kv_layout_t layout, uint32_t layer, uint32_t page,
                           uint32_t slot, uint32_t kv, uint32_t head, uint32_t d);
/* KvLayout::total_elems (kv_cache.h:60-65): max_pages*P*512*num_layers. */
uint64_t mc_kv_total_elems(mc_kv_layout_t layout);
/* attention_decode_chunk_pos tier table (kernels.h:295-304, 512 tier off). */
uint32_t mc_kv_decode_chunk_pos(uint32_t max_ctx);
/* attention_decode_max_chunks (kernels.h:308-311). */
uint32_t mc_kv_decode_max_chunks(uint32_t max_ctx, uint32_t chunk_pos);
/* prefill_flash_split_kv (kernels.h:517-521). */
uint32_t mc_kv_prefill_split_kv(uint32_t tokens);

/* ---- per-session page allocator (PagedKvAllocator, kv_cache.cpp:8-91) ---- */
typedef struct mc_kv_allocator mc_kv_allocator_t;

/* PagedKvAllocator::init (kv_cache.cpp:8-22): d_table is a device
 * u32[max_pages], or NULL for a host-only allocator (same page choices and pages_synced accounting, no
 * copies; used to plan or test tables without a device). */
mc_status_t mc_kv_allocator_create(uint32_t* d_table, uint32_t max_pages,
                                   uint32_t tokens_per_page,
                                   mc_kv_allocator_t** out);
/* Frees the allocator object (the reference's is a session member). */
void mc_kv_allocator_destroy(mc_kv_allocator_t* a);
/* PagedKvAllocator::ensure_pages_for (kv_cache.cpp:47-84): lowest-free-page growth to
 * ceil(total_tokens/P) pages; H2D of the table prefix only when it grew;
 * MC_E_OUT_OF_MEMORY when the pool is too small. */
mc_status_t mc_kv_allocator_ensure_pages_for(mc_kv_allocator_t* a,
                                             uint32_t total_tokens, void* stream);
/* PagedKvAllocator::release_all (kv_cache.cpp:85-91): clears ownership,
 * keeps device table. */
void mc_kv_allocator_release_all(mc_kv_allocator_t* a);
/* pages_owned() and the pages_synced_ count (kv_cache.h:84,100). */
uint32_t mc_kv_allocator_pages_owned(const mc_kv_allocator_t* a);
uint32_t mc_kv_allocator_pages_synced(const mc_kv_allocator_t* a);
/* Copies min(n, pages_owned) entries of the host shadow table (shadow_,
 * kv_cache.h:102). */
uint32_t mc_kv_allocator_host_table(const mc_kv_allocator_t* a, uint32_t* out,
                                    uint32_t n);

/* ---- shared page pool (several sessions in one pool; per-session free) ----
 * No reference counterpart: the reference gives each session a private pool
 * (session.cpp:227-231). This pool serves the interleaved batched-decode and
 * churn workloads. Allocation takes the lowest free page id (same rule as
 * PagedKvAllocator::first_free_page, kv_cache.cpp:24-36); a session's pages
 * are returned by mc_kv_pool_release and become reusable. */
typedef struct mc_kv_pool mc_kv_pool_t;

mc_status_t mc_kv_pool_create(uint32_t max_pages, uint32_t tokens_per_page,
                              uint32_t max_sessions, mc_kv_pool_t** out);
void mc_kv_pool_destroy(mc_kv_pool_t* p);
/* Grows session `sid` to cover total_tokens; appends new page ids to its host
 * table and, if d_table != NULL and the table grew, uploads the grown suffix
 * to d_table (device u32[max pages per session]) on `stream`. */
mc_status_t mc_kv_pool_ensure(mc_kv_pool_t* p, uint32_t sid,
                              uint32_t total_tokens, uint32_t* d_table,
                              void* stream);
/* Frees every page of session `sid`. */
mc_status_t mc_kv_pool_release(mc_kv_pool_t* p, uint32_t sid);
uint32_t mc_kv_pool_pages_free(const mc_kv_pool_t* p);
uint32_t mc_kv_pool_session_pages(const mc_kv_pool_t* p, uint32_t sid);
uint32_t mc_kv_pool_session_table(const mc_kv_pool_t* p, uint32_t sid,
                                  uint32_t* out, uint32_t n);

/* ---- RoPE + K/V append ---- */

/* launch_rope_inv_freq_init (kernels.h:229-230, rope_kv.cu:104-124):
 * d_table[p] = (float)pow(theta, -p/64), p < 64. */
mc_status_t mc_kv_rope_inv_freq_init(float* d_table, double rope_theta,
                                     void* stream);

/* launch_rope_kv (kernels.h:214-225, rope_kv.cu:30-96,126-148): for token t
 * at pos = *d_base_pos + t, rotate q (in place, 16 heads), rotate k and store
 * it to the pool (kv=0), copy v to the pool (kv=1). d_inv_freq may be NULL
 * (then computed from rope_theta in the kernel). */
mc_status_t mc_kv_rope_append(uint16_t* d_qkv, uint32_t tokens,
                              const uint32_t* d_base_pos, uint32_t layer,
                              const uint32_t* d_page_table, uint16_t* d_kv_pool,
                              mc_kv_layout_t layout, double rope_theta,
                              const float* d_inv_freq, void* stream);

/* ---- decode attention (split-KV flash decoding) ---- */

/* launch_attention_decode (kernels.h:369-388, attention_decode.cu:1840-1964).
 * Attends positions 0..limit (limit = *d_pos) of one session and writes
 * d_out [2048] bf16. d_partials [16][max_chunks][130] fp32 is scratch: the
 * chunk kernel folds each workgroup's range of ceil(max_chunks / 256) chunks
 * (one chunk when max_chunks <= 256, or when chunk_pos is not a multiple of
 * 64) into one record {m, l, acc[128]} per query head, and a merge kernel
 * folds the records (fixed order). With 33..256 records per head each head's
 * records are stored split (acc[n][128], then {m, l}[n]) in the same space;
 * d_partials' contents are then not the reference's partial layout. Beyond 256 records per head (chunk_pos
 * not a multiple of 64 and more than 256 chunks) the reference's merges run
 * instead: two-level through d_partials2 ([16][32][130]) when it is not NULL
 * and there are more than 32 records, else one-level. If limit < the range
 * size the single workgroup writes d_out directly.
 * d_inv_freq != NULL enables phase0: q and k of position `limit` are rotated
 * from d_q_rows, K/V of `limit` are written to the pool (pool may be written
 * only in that case). chunk_pos must be a multiple of 16. d_page_table is
 * read at entries 0..limit/P. */
mc_status_t mc_kv_attention_decode(const uint16_t* d_q_rows, const uint32_t* d_pos,
                                   uint32_t layer, const uint32_t* d_page_table,
                                   uint16_t* d_kv_pool, mc_kv_layout_t layout,
                                   float* d_partials, uint32_t max_chunks,
                                   uint16_t* d_out, void* stream,
                                   const float* d_inv_freq, uint32_t chunk_pos,
                                   float* d_partials2);

/* Allocation-free decode. No counterpart in the reference: it is for callers
 * that cannot allocate or pass scratch (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). Same computation and
 * output as mc_kv_attention_decode (bit-identical), but the records live in
 * a library-owned device array of 16 x 256 x 130 floats (2.13 MB per device,
 * held until the process ends), so no d_partials / d_partials2 are taken and
 * nothing is allocated. Limit: at most 256 records per head, i.e. chunk_pos a
 * multiple of 64 or max_chunks <= 256 (else MC_E_INVALID_ARGUMENT). All calls
 * on one device share the array: calls that overlap on a device (e.g. on two
 * streams) race and must be serialized by the caller. */
mc_status_t mc_kv_attention_decode_noalloc(const uint16_t* d_q_rows, const uint32_t* d_pos,
                                           uint32_t layer, const uint32_t* d_page_table,
                                           uint16_t* d_kv_pool, mc_kv_layout_t layout,
                                           uint32_t max_chunks, uint16_t* d_out, void* stream,
                                           const float* d_inv_freq, uint32_t chunk_pos);

/* launch_attention_decode_merge (kernels.h:394-400): merge only, from given
 * level-1 partials. */
mc_status_t mc_kv_attention_decode_merge(const float* d_partials,
                                         const uint32_t* d_pos,
                                         uint32_t max_chunks, uint32_t chunk_pos,
                                         float* d_partials2, uint16_t* d_out,
                                         void* stream);

/* Chunk kernel only (no merge): the test/bench twin of launch_attn_kv_h_test
 * (kernels.h:441-450) without the score scratch. Writes the per-chunk
 * partials [16][max_chunks][130] of chunks 0..limit/chunk_pos (one record
 * per chunk), or d_out directly when limit < chunk_pos. */
mc_status_t mc_kv_attention_decode_chunks(const uint16_t* d_q_rows,
                                          const uint32_t* d_pos, uint32_t layer,
                                          const uint32_t* d_page_table,
                                          uint16_t* d_kv_pool,
                                          mc_kv_layout_t layout,
                                          float* d_partials, uint32_t max_chunks,
                                          uint16_t* d_out, void* stream,
                                          const float* d_inv_freq,
                                          uint32_t chunk_pos);

/* launch_attention_decode_batch (kernels.h:465-480,
 * attention_decode.cu:2120-2170). Slot s uses q row d_q_rows + s*2560,
 * limit *d_slot_pos[s], page table d_slot_pt[s], pool d_slot_kv[s]; writes
 * d_out + s*2048 and uses d_partials (B*16*max_chunks*130 floats) and
 * d_partials2 (B*16*32*130) as scratch, as mc_kv_attention_decode does per
 * slot. Outputs are bit-identical to B single-session calls. The three
 * pointer tables live in device memory. B <= 64. */
mc_status_t mc_kv_attention_decode_batch(const uint16_t* d_q_rows,
                                         const uint32_t* const* d_slot_pos,
                                         uint32_t B, uint32_t layer,
                                         const uint32_t* const* d_slot_pt,
                                         uint16_t* const* d_slot_kv,
                                         mc_kv_layout_t layout, float* d_partials,
                                         uint32_t max_chunks, uint16_t* d_out,
                                         void* stream, const float* d_inv_freq,
                                         uint32_t chunk_pos, float* d_partials2);

/* ---- prefill attention over the paged cache ---- */

/* launch_attn_prefill_flash (kernels.h:575-585, attention_prefill.cu:291-729):
 * causal attention of T query rows (absolute positions *d_base_pos + t) over
 * pool positions 0..*d_base_pos + t gathered through the page table.
 * S_kv in 1..8 key splits; S_kv > 1 needs d_partials of
 * T*16*S_kv*130 floats and runs the split merge. Writes d_out [T][2048]. */
mc_status_t mc_kv_attention_prefill(const uint16_t* d_q_rows, uint32_t tokens,
                                    const uint32_t* d_base_pos, uint32_t layer,
                                    const uint32_t* d_page_table,
                                    const uint16_t* d_kv_pool,
                                    mc_kv_layout_t layout, uint16_t* d_out,
                                    float* d_partials, uint32_t S_kv,
                                    void* stream);

/* ---- device-side sequence advance ---- */

/* launch_decode_advance (kernels.h:632-635, sampling.cu:58-67):
 * d_seq[*d_seq_len] = *d_next_token; *d_seq_len += 1. */
mc_status_t mc_kv_decode_advance(int32_t* d_seq, const int32_t* d_next_token,
                                 uint32_t* d_seq_len, void* stream);

/* launch_batch_advance (kernels.h:651-655, sampling.cu:241-251): per slot s,
 * d_slot_seq[s][*d_slot_pos[s]] = *d_slot_tok[s]; *d_slot_pos[s] += 1. */
mc_status_t mc_kv_batch_advance(int32_t* const* d_slot_seq,
                                const int32_t* const* d_slot_tok,
                                uint32_t* const* d_slot_pos, uint32_t n,
                                void* stream);

/* ---- debug hooks (additive, outside the frozen ABI; the reference keeps
 * similar mc_debug_* hooks outside it, session.cpp:631-723) ---- */

/* Session state: host seq_len, owned pages, pool layout and the device
 * addresses of the pool and page table (any pointer may be NULL). No
 * reference counterpart (test access to a session's KV state). */
mc_status_t mc_debug_session_info(mc_session_t session, uint32_t* seq_len,
                                  uint32_t* pages_owned, mc_kv_layout_t* layout,
                                  void** d_pool, void** d_page_table);
/* Copies the first n token ids of the device sequence (n <= seq_len). No
 * reference counterpart. */
mc_status_t mc_debug_session_seq(mc_session_t session, int32_t* out, uint32_t n);

/* Session arena bytes (one device allocation per session, sized at create;
 * reference session.cpp:651-654) and the decode chunk tier chosen for the
 * session's context (session.cpp:659-662). 0 for a NULL session. */
size_t mc_debug_session_arena_bytes(mc_session_t session);
uint32_t mc_debug_session_attn_chunk(mc_session_t session);

/* Graph A/B switch (reference session.cpp:636-641): enabled = 0 makes the
 * session's decode steps run eagerly although graph mode is on; enabled != 0
 * returns to graph replay, which only takes effect when the model was
 * loaded with enable_cuda_graph (the graph is captured at the first graph
 * step). NULL session: no effect. */
void mc_debug_session_set_graph_enabled(mc_session_t session, int enabled);
/* Nodes of the session's captured decode-step graph (hipGraphGetNodes;
 * reference session.cpp:644-647); 0 when none has been captured yet or for a
 * NULL session. */
size_t mc_debug_session_graph_nodes(mc_session_t session);
/* Regression guard of the RoPE frequency table (reference session.cpp:
 * 668-686): 1 when the session's 64 inv_freq words on the device are
 * bit-identical to the snapshot taken at mc_session_create, 0 when they were
 * overwritten, -1 for a NULL session (or no snapshot), -2 on a HIP error.
 * Call after the last mc_prefill / mc_decode_one / mc_batch_step returned
 * (they synchronize the session's stream). */
int mc_debug_session_rope_intact(mc_session_t session);

/* Decode-step breakdown (reference session.cpp:686-723): when MC_BREAKDOWN
 * is set at mc_session_create, every eager mc_decode_one records events at
 * its segment boundaries (a step replayed as a HIP graph records none; the
 * hooks then report -2). Raw segments, in order:
 * per layer {synthetic qkv row, phase0 decode attention}, then the tail
 * (token write + sequence advance). raw_segments returns their count (0 when
 * off); bucket_count / bucket_name / bucket_of describe the aggregation
 * (qkv, attention, tail); collect writes the last step's segment times (ms)
 * into out_ms[0..n) with n == raw_segments and returns n; 0 = off,
 * -1 = bad arguments, -2 = no complete step recorded yet, -3 = HIP error.
 * Call after the step returned (it synchronizes its stream). */
int mc_debug_breakdown_raw_segments(mc_session_t session);   /* session.cpp:686 */
int mc_debug_breakdown_bucket_count(void);                    /* session.cpp:692 */
const char* mc_debug_breakdown_bucket_name(int i);            /* session.cpp:696 */
int mc_debug_breakdown_bucket_of(int raw);                    /* no counterpart */
int mc_debug_breakdown_collect(mc_session_t session, double* out_ms, int n); /* :705 */

/* Debug dump step limit (reference debug_dump.cpp:152-157, debug_dump.h:
 * 1-12): with MC_DEBUG_DUMP_DIR set in the environment (read once, with
 * MC_DEBUG_DUMP_STEPS = N, default 0) forward number t < N of a session with
 * weights (its counter restarts at mc_session_create / mc_session_reset; each
 * prefill chunk and each mc_decode_one is one forward) writes, into that
 * directory, step{t}.logits.f32 (130560 values), step{t}.final_hidden.f32
 * (the last row after final_norm, 2048) and step{t}.token (int32, the greedy
 * prediction); the first chunk of a prefill also writes layer{i}.hidden_in,
 * .attn_out and .mlp_out.f32 (the last row of the residual at the layer's
 * input, after the o projection's add and after the down projection's add).
 * Values are the bf16 tensors widened to fp32. A decode step that dumps runs
 * eagerly (not from the captured graph). This call changes N at run time
 * (0 stops further dumps); without MC_DEBUG_DUMP_DIR it has no effect. */
void mc_debug_dump_set_steps(int steps);
/* Window seed hook of the reference (debug_dump.cpp:159-199): copies rows x
 * 2048 bf16 host values into the session's residual rows. The reference's
 * windowed loading (MC_LOAD_LAYERS_MIN/MAX), whose forward starts from such a
 * seed, is not supported here, so the next mc_prefill's embedding gather
 * overwrites the rows, as with a fully loaded model in the reference.
 * MC_E_UNSUPPORTED without weights (as the reference), MC_E_INVALID_ARGUMENT
 * for rows outside 1..(the session's prefill chunk rows). */
mc_status_t mc_debug_seed_residual(mc_session_t session, const void* host_bf16_rows,
                                   uint32_t rows);

/* Batch-group statistics (reference batch_group.cpp:869-886): steps run,
 * their summed wall time (us) and the current member count. */
mc_status_t mc_debug_batch_group_stats(mc_batch_group_t group, uint64_t* steps,
                                       uint64_t* decode_us, uint32_t* members);

/* Last mc_batch_step's time per bucket (ms) when MC_BATCH_BREAKDOWN was set
 * at mc_batch_group_create (reference batch_group.cpp:888-927; buckets as
 * mc_debug_breakdown_bucket_name). n must equal the bucket count; returns it,
 * 0 = off, -1 = bad arguments, -2 = no complete step, -3 = HIP error. */
int mc_debug_batch_breakdown_collect(mc_batch_group_t group, double* out_ms, int n);

/* Prefill workgroup shape: 0 = 32 query rows on 8 waves, 1 = 16 rows on 4
 * waves, 2 = 16 rows on two 4-wave halves taking alternate key steps,
 * 0xFFFFFFFF = chosen per launch (default). All compute the same softmax;
 * shapes differ in tile boundaries (key splits) and summation order, within
 * the attention tolerance. The previous value is stored to *previous when
 * that is not NULL. Process-wide; for tests that run every shape. No
 * reference counterpart. */
mc_status_t mc_kv_debug_prefill_shape(uint32_t shape, uint32_t* previous);

/* Prefill job packing: with key splits off, two to three 32-row jobs per CU
 * and a prefix of at least T/4, one workgroup per CU runs a fixed 2-3 job
 * packing instead of greedy dispatch (identical results). enable = 0 turns it
 * off (default on). The previous setting is stored to *previous when that is
 * not NULL. Process-wide; for tests that compare both schedules. No
 * reference counterpart. */
mc_status_t mc_kv_debug_prefill_packing(uint32_t enable, uint32_t* previous);

/* Prefill status of the current device: *barrier_timeouts receives the
 * number of per-half waits of the two-half prefill shape that ran out of
 * their bound (about 0.1 s of polling) since the last reset; each such wait
 * may have left wrong values in that launch's output, so any non-zero value
 * is an error. reset != 0 clears the counter after reading. Synchronous:
 * waits for work queued on the device's blocking streams. No reference
 * counterpart (the reference's prefill uses workgroup barriers only). */
mc_status_t mc_kv_debug_prefill_status(uint32_t* barrier_timeouts, uint32_t reset);

/* Sets the current device's half-barrier timeout count to `count` from the
 * host (no kernel runs): lets a test check that the session prefill path
 * (mc_prefill, which reads and clears the count after each chunk and returns
 * MC_E_INTERNAL when it is non-zero) reports a timeout without making any
 * wait time out. No reference counterpart. */
mc_status_t mc_kv_debug_prefill_force_timeouts(uint32_t count);

/* Decode P.V precision (process-wide): 0 = P rounded to bf16 before P.V
 * (default, the reference's HMMA path), 1 = fp32 P (the reference's
 * MC_ATTN_HMMA_OFF fallback, attention_decode.cu:506-878), 0xFFFFFFFF = from
 * the environment (MC_ATTN_HMMA_OFF set -> fp32 P, read once, as
 * kernels.h:355-367 does). The previous value goes to *previous when not
 * NULL. Switch between launches only: a captured graph keeps the kernels it
 * was captured with. */
mc_status_t mc_kv_debug_decode_fp32p(uint32_t fp32_p, uint32_t* previous);

/* Measurement switch (process-wide, default 0): with enable != 0,
 * mc_kv_attention_decode and mc_kv_attention_decode_batch launch only the
 * chunk kernel (records written, d_out not produced), so a benchmark can
 * time that kernel alone in its production configuration. The previous
 * value goes to *previous when not NULL. No reference counterpart. */
mc_status_t mc_kv_debug_decode_records_only(uint32_t enable, uint32_t* previous);

/* Debug timeline (process-wide, default off): attaches a device buffer of
 * launches * MC_KV_TIMELINE_WORDS uint64 words. Each later decode
 * (mc_kv_attention_decode, _batch, _noalloc) takes the next region of the
 * ring; in its region, chunk-kernel workgroup w (w < 8192, linear block
 * index) writes words 4w..4w+3 = {entry clock, exit clock (latest wave),
 * XCC id, 0} and merge workgroup m (m < 2048) writes words 32768 + 2m..+1 =
 * {entry, exit}. The clock is s_memrealtime, 100 MHz. The caller zeroes the
 * buffer; unwritten words stay 0. A captured graph keeps the regions it was
 * captured with. d_stamps = NULL with launches = 0 detaches (the region
 * counter restarts at 0 on every call). Detached, the kernels only test a
 * null pointer. No reference counterpart. */
#define MC_KV_TIMELINE_WORDS 36864u
mc_status_t mc_kv_debug_decode_timeline(uint64_t* d_stamps, uint32_t launches);

/* Library build identity, e.g. "minicpm-kv gfx950". No reference
 * counterpart. */
const char* mc_kv_build_info(void);

#pragma GCC visibility pop

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MC_KV_H_ */
