/* mc_model.h - C ABI of the weight path in libminicpm_native.so (MI355X /
 * gfx950 build): the kernels around the paged KV cache that a MiniCPM5
 * forward needs once real weights are loaded (embedding, RMSNorm, SwiGLU,
 * GEMV, greedy argmax) and a check of a model.wpk weight package.
 *
 * Each declaration cites the reference launcher it replaces
 * (native/kernels/sm120/kernels.h, native/runtime/weight_loader.h). The
 * conventions are those of mc_kv.h: bf16 as uint16_t bit patterns, device
 * pointers, `stream` a hipStream_t as void*, MC_E_INVALID_ARGUMENT for bad
 * arguments, MC_E_CUDA for launch failures, message in mc_last_error().
 *
 * mc_model_load (minicpm_runtime.h) uses these when the model directory holds
 * model.wpk: prefill runs the GEMMs through rocBLAS (bf16 in/out, fp32
 * compute), decode and batch steps run the GEMV kernels below.
 */
#ifndef MC_MODEL_H_
#define MC_MODEL_H_

#include <stddef.h>
#include <stdint.h>

#include "minicpm_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

#define MC_MODEL_GEMV_MAX_ROWS 8u /* activation rows per GEMV launch (batch steps) */

/* launch_embedding_gather (kernels.h:156) and
 * launch_embedding_gather_indirect (kernels.h:197): d_out[r] =
 * d_table[id_r] for r < rows, id_r = d_ids[r], or *d_slot_tok[r] (a device
 * table of per-slot token addresses) when d_ids is NULL. Exactly one of d_ids
 * / d_slot_tok. hidden must be a multiple of 8; ids must lie in the table. */
mc_status_t mc_model_embedding_gather(const uint16_t* d_table, const int32_t* d_ids,
                                      const int32_t* const* d_slot_tok, uint16_t* d_out,
                                      uint32_t hidden, uint32_t rows, void* stream);

/* launch_rmsnorm_rows (kernels.h:172) when d_add is NULL, and
 * launch_residual_add_rmsnorm (kernels.h:185) when it is not: per row,
 * optionally d_res = bf16(d_res + d_add) (stored), then
 * d_out = bf16(d_res * inv * d_weight), inv = 1/sqrt(mean(d_res^2) + eps),
 * all in fp32. n must be a multiple of 8. */
mc_status_t mc_model_rmsnorm_rows(uint16_t* d_res, const uint16_t* d_add,
                                  const uint16_t* d_weight, uint16_t* d_out, uint32_t rows,
                                  uint32_t n, float eps, void* stream);

/* launch_swiglu_gated (kernels.h:589): d_src [rows][2*inter] holds gate |
 * up; d_out[r][i] = bf16(silu(g) * u), silu(g) = g / (1 + exp(-g)) in fp32. */
mc_status_t mc_model_swiglu_rows(const uint16_t* d_src, uint16_t* d_out, uint32_t rows,
                                 uint32_t inter, void* stream);

/* launch_decode_gemv (kernels.h:666), extended to M <= 8 activation rows
 * (batch steps): d_y[m][n] = bf16(sum_k d_w[n][k] * d_x[m][k]) with fp32
 * accumulation, d_w row-major [N][K], row strides ldx / ldy (elements).
 * K is 2048 or 6144 (the model's projections). */
mc_status_t mc_model_gemv(const uint16_t* d_w, const uint16_t* d_x, uint32_t ldx,
                          uint16_t* d_y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                          void* stream);

/* launch_gemv_rows_prologue (kernels.h:743), for M <= 8 rows of 2048:
 * r = bf16(d_res_in + d_add) (d_add may be NULL: r = d_res_in), stored to
 * d_res_out when that is not NULL (it must not alias the inputs), x =
 * bf16(r * inv * d_norm_w) as mc_model_rmsnorm_rows, then d_y = GEMV(d_w, x)
 * with K = 2048. Row stride of the residual buffers: ldr. */
mc_status_t mc_model_gemv_resnorm(const uint16_t* d_w, const uint16_t* d_res_in,
                                  const uint16_t* d_add, const uint16_t* d_norm_w,
                                  uint16_t* d_res_out, uint32_t ldr, uint16_t* d_y, uint32_t ldy,
                                  uint32_t M, uint32_t N, float eps, void* stream);

/* launch_gemv_rows_prologue (kernels.h:743) followed by launch_swiglu_gated
 * (kernels.h:589) in one launch: with the prologue of
 * mc_model_gemv_resnorm, output column i < I of row m is
 * bf16(silu(g) * u) where g = bf16(d_w[i] . x_m) and u = bf16(d_w[I + i] . x_m)
 * (d_w: the gate_up matrix [2I][2048], gate rows then up rows), i.e. the
 * gate_up projection rounded to bf16 and then the SwiGLU, without writing
 * the projection. d_y rows hold I values (stride ldy). */
mc_status_t mc_model_gemv_resnorm_swiglu(const uint16_t* d_w, const uint16_t* d_res_in,
                                         const uint16_t* d_add, const uint16_t* d_norm_w,
                                         uint16_t* d_res_out, uint32_t ldr, uint16_t* d_y,
                                         uint32_t ldy, uint32_t M, uint32_t I, float eps,
                                         void* stream);

/* launch_gemv_rows_swiglu (kernels.h:760), for M <= 8 rows: x =
 * swiglu(d_gate_up rows [M][ldx], gate in columns 0..K-1, up in K..2K-1) as
 * mc_model_swiglu_rows, then d_y = GEMV(d_w, x). K is 2048 or 6144. */
mc_status_t mc_model_gemv_swiglu(const uint16_t* d_w, const uint16_t* d_gate_up, uint32_t ldx,
                                 uint16_t* d_y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                                 void* stream);

/* Row GEMM of a prefill chunk of MC_MODEL_GEMM_ROWS_MIN..MAX rows: d_y[m][n] =
 * bf16(sum_k d_w[n][k] * d_x[m][k]) with fp32 accumulation (swiglu = 0), or,
 * with swiglu = 1, d_y[m][n] = bf16(silu(g) * u) where g and u are the rows
 * n and N + n of d_w ([2N][K]: gate rows, then up rows) dotted with x_m and
 * rounded to bf16 (the gate_up projection followed by the SwiGLU, as
 * mc_model_gemv_resnorm_swiglu). N a multiple of 16, K 2048 or 6144 (2048
 * with swiglu), row strides ldx (multiple of 8) and ldy (multiple of 4) in
 * elements, d_w and d_x 16-byte and d_y 8-byte aligned. No
 * reference counterpart: the reference runs every multi-token chunk through
 * cuBLAS (forward.cpp:200-420); this replaces the library GEMM where its
 * per-call cost dominates. */
#define MC_MODEL_GEMM_ROWS_MIN 9u
#define MC_MODEL_GEMM_ROWS_MAX 32u
mc_status_t mc_model_gemm_rows(const uint16_t* d_w, const uint16_t* d_x, uint32_t ldx,
                               uint16_t* d_y, uint32_t ldy, uint32_t M, uint32_t N, uint32_t K,
                               uint32_t swiglu, void* stream);

/* ---- FP8 projections (precision MC_FP8: single-token forwards) ----
 * d_w: e4m3 codes [N][K] (uint8, 16-byte aligned rows), d_scale: fp32 [N]
 * row scales; d_y[n] = bf16(d_scale[n] * sum_k e4m3(d_w[n][k]) * x[k])
 * with fp32 accumulation, the scale applied after the sum (gemv_fp8.cu:3-7);
 * e4m3 is s.eeee.mmm with bias 7, subnormals m/8 * 2^-6, and S.1111.111
 * read as +-480 (kernels.h:120-148). One activation row (bf16); K is 2048
 * or 6144. */

/* launch_gemv_fp8 (kernels.h:721-726): x = d_x [K]. */
mc_status_t mc_model_gemv_fp8(const uint8_t* d_w, const float* d_scale, const uint16_t* d_x,
                              uint16_t* d_y, uint32_t N, uint32_t K, void* stream);

/* launch_gemv_fp8_swiglu (kernels.h:753-758): x = SwiGLU of the gate|up row
 * d_gate_up [2K], rounded to bf16. */
mc_status_t mc_model_gemv_fp8_swiglu(const uint8_t* d_w, const float* d_scale,
                                     const uint16_t* d_gate_up, uint16_t* d_y, uint32_t N,
                                     uint32_t K, void* stream);

/* launch_gemv_fp8_prologue (kernels.h:735-741): r = bf16(d_res_in + d_add)
 * (d_add may be NULL), stored to d_res_out when not NULL (not aliasing the
 * inputs), x = bf16(r * inv * d_norm_w) over 2048 dims, K = 2048. */
mc_status_t mc_model_gemv_fp8_resnorm(const uint8_t* d_w, const float* d_scale,
                                      const uint16_t* d_res_in, const uint16_t* d_add,
                                      const uint16_t* d_norm_w, uint16_t* d_res_out,
                                      uint16_t* d_y, uint32_t N, float eps, void* stream);

/* The norm prologue with the SwiGLU epilogue of mc_model_gemv_resnorm_swiglu:
 * d_w holds 2I rows (gate rows, then up rows) and d_scale 2I scales;
 * d_y[n] = bf16(silu(g) * u) with g, u the two projections rounded to bf16
 * (a gate_up projection, then the SwiGLU kernel). No reference counterpart
 * (the reference fuses the SwiGLU into the down projection instead). */
mc_status_t mc_model_gemv_fp8_resnorm_swiglu(const uint8_t* d_w, const float* d_scale,
                                             const uint16_t* d_res_in, const uint16_t* d_add,
                                             const uint16_t* d_norm_w, uint16_t* d_res_out,
                                             uint16_t* d_y, uint32_t I, float eps,
                                             void* stream);

/* launch_sampling_greedy_bf16 (kernels.h:610) for rows == 1 and
 * launch_batch_argmax_bf16 (kernels.h:641): per row of n bf16 logits the
 * index of the largest value compared in fp32, ties to the lowest index,
 * written to d_out[r] or to *d_slot_tok[r]. Exactly one of the two. With
 * stage buffers (MC_MODEL_ARGMAX_SLICES floats / ints per row, as the
 * reference's d_stage_v / d_stage_i) the row is scanned by that many
 * workgroups and the slices reduced by a second launch; with NULL one
 * workgroup scans the row. */
#define MC_MODEL_ARGMAX_SLICES 64u
mc_status_t mc_model_argmax_bf16(const uint16_t* d_logits, uint32_t n, uint32_t rows,
                                 int32_t* d_out, int32_t* const* d_slot_tok, float* d_stage_v,
                                 int32_t* d_stage_i, void* stream);

/* WeightLoader::load_wpk's checks (weight_loader.h:120-137,
 * weight_loader.cpp:201-360) without a device: reads the model.wpk at
 * `path` (header, TOC, every section the full model needs, the sizes and
 * offsets within the file) and returns MC_OK with the bytes the device arena
 * would hold in *arena_bytes, or MC_E_IO / MC_E_MODEL_MISMATCH with the
 * reason in mc_last_error(). No reference counterpart as a separate call. */
mc_status_t mc_model_wpk_check(const char* path, uint64_t* arena_bytes);

/* WeightLoader::load_wpk_fp8's checks (weight_loader.cpp:470-620) of a
 * model_fp8.wpk without a device: the header rules of model.wpk, unique
 * name hashes, the 42 x {qkv, o, gate_up, down} sections (plus "lm_head"
 * when the package holds a dtype-2 one and MC_FP8_LMHEAD_OFF is unset) as
 * dtype 2 (e4m3) row-major [N][K] with N * K code bytes and 4N scale bytes
 * inside the file; other sections are ignored. *arena_bytes = the device
 * bytes the codes and scales take. MC_E_MODEL_MISMATCH for a missing file
 * or a failed check, MC_E_IO for a short read. */
mc_status_t mc_model_wpk_fp8_check(const char* path, uint64_t* arena_bytes);

/* Debug hooks of a model loaded with weights (outside the frozen ABI):
 * the bf16 logits (as fp32) of the last forward of a session (its last
 * prefill chunk's last row or its last decode), and of `slot` in the last
 * mc_batch_step of a group (mc_debug_batch_last_logits,
 * batch_group.cpp:929-955; MC_E_INVALID_ARGUMENT when the slot was not in
 * that step). out_f32 holds 130560 floats. */
mc_status_t mc_debug_session_last_logits(mc_session_t session, float* out_f32);
mc_status_t mc_debug_batch_last_logits(mc_batch_group_t group, uint32_t slot, float* out_f32);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* MC_MODEL_H_ */
