/* minicpm_runtime.h - stable host/GPU C ABI of libminicpm_native.so (v0.1,
 * ABI 0x00020000), declared for the MI355X build.
 *
 * Every declaration below keeps the name, argument order, types and struct
 * layout of the reference ABI (native/include/minicpm_runtime.h:28-199) so that
 * the Rust host crates (rust/minicpm-runtime-sys/src/lib.rs:61-190, which
 * resolve these symbols by name through dlopen in
 * rust/minicpm-runtime/src/native.rs:90-94) load this library unchanged.
 *
 * Contract (unchanged from the reference):
 *   - extern "C", fixed-width integers, POD structs, opaque handles;
 *   - structs that may evolve carry struct_size (and abi_version);
 *   - a model is immutable and may be shared; a session is not thread-safe;
 *   - every entry point returns mc_status_t; mc_last_error() returns the
 *     calling thread's last English diagnostic.
 */
#ifndef MINICPM_RUNTIME_H_
#define MINICPM_RUNTIME_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Exported even when the library is built with -fvisibility=hidden. */
#pragma GCC visibility push(default)

#define MC_ABI_VERSION 0x00020000u

typedef struct mc_model mc_model_t;
typedef struct mc_session mc_session_t;

typedef enum mc_status_t {
    MC_OK = 0,
    MC_E_INVALID_ARGUMENT = 1,
    MC_E_IO = 2,
    MC_E_CUDA = 3, /* device runtime error (HIP on this build) */
    MC_E_MODEL_MISMATCH = 4,
    MC_E_OUT_OF_MEMORY = 5,
    MC_E_GRAPH = 6,
    MC_E_UNSUPPORTED = 7,
    MC_E_INTERNAL = 100
} mc_status_t;

typedef enum mc_precision_t {
    MC_BF16 = 0,
    MC_FP16 = 1,
    MC_FP8 = 2,
    MC_NVFP4 = 3
} mc_precision_t;

typedef enum mc_kv_precision_t {
    MC_KV_BF16 = 0,
    MC_KV_FP8 = 1
} mc_kv_precision_t;

/* 40 bytes on x86_64. */
typedef struct mc_model_options_t {
    uint32_t struct_size;
    uint32_t abi_version;
    int32_t device_id;
    uint32_t max_sessions;
    uint32_t max_context_tokens;
    mc_precision_t precision;
    mc_kv_precision_t kv_precision;
    uint32_t enable_cuda_graph;
    uint64_t reserve_vram_bytes;
} mc_model_options_t;

/* 32 bytes on x86_64. */
typedef struct mc_generation_config_t {
    uint32_t struct_size;
    uint32_t max_new_tokens;
    float temperature;
    float top_p;
    uint32_t top_k;
    float repetition_penalty;
    uint64_t seed;
} mc_generation_config_t;

typedef struct mc_runtime_stats_t {
    uint64_t prompt_tokens;
    uint64_t generated_tokens;
    uint64_t prefill_us;
    uint64_t decode_us;
    uint64_t peak_vram_bytes;
    uint64_t cuda_graph_launches;
} mc_runtime_stats_t;

/* ---- lifecycle ---- */
mc_status_t mc_model_load(const char* model_dir,
                          const mc_model_options_t* options,
                          mc_model_t* out_model);
void mc_model_destroy(mc_model_t model);
mc_status_t mc_session_create(mc_model_t model, mc_session_t* out_session);
mc_status_t mc_session_reset(mc_session_t session);
void mc_session_destroy(mc_session_t session);

/* ---- inference ---- */
mc_status_t mc_prefill(mc_session_t session, const int32_t* token_ids,
                       uint32_t token_count);
mc_status_t mc_decode_one(mc_session_t session,
                          const mc_generation_config_t* config,
                          int32_t* out_token);

/* ---- observability ---- */
mc_status_t mc_get_stats(mc_session_t session, mc_runtime_stats_t* out_stats);
const char* mc_last_error(void);

/* ---- batched decode (additive surface) ---- */
typedef struct mc_batch_group mc_batch_group_t;

/* 32 bytes on x86_64; reserved[] must be zero. */
typedef struct mc_batch_options_t {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t max_slots;          /* 1..8 */
    uint32_t max_context_tokens; /* must match the member sessions' tier */
    uint32_t reserved[4];
} mc_batch_options_t;

mc_status_t mc_batch_group_create(mc_model_t model,
                                  const mc_batch_options_t* options,
                                  mc_batch_group_t* out_group);
mc_status_t mc_batch_group_add(mc_batch_group_t group, mc_session_t session,
                               uint32_t* slot_id);
mc_status_t mc_batch_group_remove(mc_batch_group_t group, uint32_t slot_id);
mc_status_t mc_batch_step(mc_batch_group_t group, const uint32_t* slot_ids,
                          uint32_t n, const mc_generation_config_t* cfgs,
                          int32_t* out_tokens);
void mc_batch_group_destroy(mc_batch_group_t group);

#pragma GCC visibility pop

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MINICPM_RUNTIME_H_ */
