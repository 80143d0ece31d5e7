// model_internal.h - weight package and model constants shared by the host
// translation units of the weight path (wpk.cpp, forward.cpp, abi_shell.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mc_kv.h"
#include "mc_model.h"

namespace mckv {

// MiniCPM5-2B geometry (native/runtime/generated_model_config.h:13-23).
constexpr uint32_t kModelLayers = 42;
constexpr uint32_t kHidden = 2048;
constexpr uint32_t kInter = 6144;
constexpr uint32_t kVocabSize = 130560;
constexpr uint32_t kQkvCols = 2560;  // q (16 x 128) | k (2 x 128) | v (2 x 128)
constexpr float kRmsEps = 1e-6f;

// Device pointers into one weight allocation (row-major bf16, [out][in]).
struct ModelWeights {
    void* arena = nullptr;
    uint64_t bytes = 0;
    const uint16_t* embedding = nullptr;   // [vocab][hidden]
    const uint16_t* lm_head = nullptr;     // [vocab][hidden]
    const uint16_t* final_norm = nullptr;  // [hidden]
    const uint16_t* norm1[kModelLayers] = {};
    const uint16_t* qkv[kModelLayers] = {};      // [2560][2048]
    const uint16_t* o[kModelLayers] = {};        // [2048][2048]
    const uint16_t* norm2[kModelLayers] = {};
    const uint16_t* gate_up[kModelLayers] = {};  // [12288][2048], gate rows then up rows
    const uint16_t* down[kModelLayers] = {};     // [2048][6144]
    // FP8 copies (model_fp8.wpk, precision MC_FP8): e4m3 codes [N][K] and
    // fp32 row scales [N] of the four projections, and of the lm_head when
    // the package holds one; fp8_arena == nullptr when not loaded.
    void* fp8_arena = nullptr;
    uint64_t fp8_bytes = 0;
    const uint8_t* q_qkv[kModelLayers] = {};
    const float* s_qkv[kModelLayers] = {};
    const uint8_t* q_o[kModelLayers] = {};
    const float* s_o[kModelLayers] = {};
    const uint8_t* q_gate_up[kModelLayers] = {};
    const float* s_gate_up[kModelLayers] = {};
    const uint8_t* q_down[kModelLayers] = {};
    const float* s_down[kModelLayers] = {};
    const uint8_t* q_lm_head = nullptr;
    const float* s_lm_head = nullptr;
};

// Reads and checks `path` (a model.wpk). With `w` != nullptr the sections
// are uploaded into one device allocation on the current device (stream
// `st`), otherwise only checked; *arena_bytes receives the allocation size.
mc_status_t wpk_load(const char* path, ModelWeights* w, uint64_t* arena_bytes, hipStream_t st);
// The same for model_fp8.wpk into w's FP8 members (its own allocation).
mc_status_t wpk_load_fp8(const char* path, ModelWeights* w, uint64_t* arena_bytes,
                         hipStream_t st);
void wpk_free(ModelWeights* w);

}  // namespace mckv

namespace mckv {

// Device buffers and KV state one forward works on. Activation buffers hold
// `rows` rows; res_a / res_b are the two residual buffers the fused decode
// chain alternates between.
struct Forward {
    const ModelWeights* w = nullptr;
    hipStream_t st = nullptr;
    void* blas = nullptr;  // prefill GEMM libraries (prefill_blas_create)
    // KV cache of a session (prefill and solo decode)
    uint16_t* pool = nullptr;
    const uint32_t* d_pt = nullptr;
    mc_kv_layout_t layout{};
    const uint32_t* d_seq_len = nullptr;  // positions are read here at run time
    const float* inv_freq = nullptr;
    float* partials = nullptr;
    float* partials2 = nullptr;
    float* pf_partials = nullptr;
    uint32_t max_chunks = 0, chunk_pos = 64;
    // activations
    uint16_t *res_a = nullptr, *res_b = nullptr, *normed = nullptr, *qkv = nullptr,
             *attn = nullptr, *o_out = nullptr, *gate_up = nullptr, *mlp = nullptr,
             *down = nullptr, *logits = nullptr;
    float* stage_v = nullptr;    // argmax slice results
    int32_t* stage_i = nullptr;
    uint32_t rows = 0;
    // debug dump (MC_DEBUG_DUMP_DIR): the session's forward counter for this
    // forward and whether it may dump per-layer rows (the first prefill chunk)
    uint32_t dump_step = 0;
    bool dump_layers = false;
    // prefill: positions the chunk's last row attends (base + n; 0 = not
    // known), which caps the prefill attention's key splits
    uint32_t keys = 0;
};

// Debug dump of the reference (debug_dump.h:1-12): with MC_DEBUG_DUMP_DIR set
// (read once) and MC_DEBUG_DUMP_STEPS = N, forward number t < N of a session
// writes step{t}.logits.f32 / step{t}.final_hidden.f32 / step{t}.token, and a
// first prefill chunk also layer{i}.hidden_in / attn_out / mlp_out.f32 (the
// last row), bf16 values widened to fp32, in the golden fixtures' layout.
bool dump_due(uint32_t step);

// Device bytes of the activation buffers of a Forward with `rows` rows and
// `logit_rows` logits rows, and their carving from `base` (256-aligned).
size_t forward_act_bytes(uint32_t rows, uint32_t logit_rows);
void forward_carve(Forward& f, char* base, uint32_t rows, uint32_t logit_rows);

// GEMM library state of a session's prefill projections (a rocBLAS handle
// and a hipBLASLt handle with its matmul descriptor) and the size of the
// device workspace it is to be given (*ws_bytes); prefill_blas_workspace then
// hands it that much caller memory (carved from the session arena), after
// which neither library allocates. On failure *h is null (and nothing is
// held). prefill_blas_destroy(nullptr) does nothing.
mc_status_t prefill_blas_create(void** h, size_t* ws_bytes);
mc_status_t prefill_blas_workspace(void* h, void* ws, size_t ws_bytes);
void prefill_blas_destroy(void* h);

// Prefill of n <= rows tokens at positions *d_seq_len.. (ids on the device):
// K/V of every layer appended, the greedy next token written to *d_next.
mc_status_t forward_prefill(const Forward& f, const int32_t* d_ids, uint32_t n, int32_t* d_next);

// Called at segment boundaries of a decode step (after each layer's qkv
// projection and after the rest of the layer).
struct Marker {
    void (*fn)(void*) = nullptr;
    void* ctx = nullptr;
    void operator()() const {
        if (fn != nullptr) fn(ctx);
    }
};

// Decode of the token *d_tok at position *d_seq_len (K/V appended), the greedy
// next token written to *d_next (may be d_tok).
mc_status_t forward_decode(const Forward& f, const int32_t* d_tok, int32_t* d_next,
                           const Marker& mark);

// Batch decode of n <= 8 sessions: tokens *d_slot_tok[s], positions
// *d_slot_pos[s], page tables d_slot_pt[s], pools d_slot_kv[s]; the next
// tokens are written back to *d_slot_tok[s]. Activations of f (rows >= n).
struct BatchKv {
    const uint32_t* const* d_slot_pos;
    const uint32_t* const* d_slot_pt;
    uint16_t* const* d_slot_kv;
    int32_t* const* d_slot_tok;
    uint32_t n;
};
mc_status_t forward_batch(const Forward& f, const BatchKv& b, const Marker& mark);

}  // namespace mckv
