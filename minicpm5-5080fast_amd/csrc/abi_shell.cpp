// abi_shell.cpp - the stable mc_* ABI (include/minicpm_runtime.h) on HIP:
// model / session / batch-group lifecycle around the paged KV cache.
//
// Semantics follow the reference runtime: option validation and device
// selection (native/runtime/model.cpp:100-200), one device arena per session
// sized at create time (session.cpp:58-135,161-318), reset keeps memory and
// clears ownership (session.cpp:510-544), prefill validation and chunking by
// 8448 tokens (prefill_executor.cpp:27,55-157), decode validation, the
// max_new_tokens EOS sentinel and the mock token rule of the weight-free mode
// (decode_executor.cpp:35-40,70-150,431-553; sampling.cu:50-56), and the batch
// group's validation / slot rules (batch_group.cpp:223-612,614-859).
//
// A model directory holding model.wpk loads the weights (wpk.cpp) and runs
// the MiniCPM5 forward (forward.cpp) with greedy decoding: the token returned
// by a decode is the one the previous forward predicted, and the forward on
// it predicts the next (decode_executor.cpp:171-230); non-greedy configs are
// rejected with MC_E_UNSUPPORTED (sampling is outside this build). Any other
// directory loads in weight-free mode. Unlike the reference's mock (which
// skips the forward), that mode runs the real KV path every layer on
// synthetic qkv rows (synth.hip): prefill appends with RoPE and runs the
// paged prefill attention, decode runs the phase0 decode attention, batch
// steps run the batched decode attention with per-slot pointer tables.
// Emitted tokens follow the reference mock rule token = 100 + ((seq_len *
// 2654435761) ^ rng) % 1000, rng advanced by xorshift32, seeded from the
// first decode config's seed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <sys/stat.h>
#include <vector>

#include <rocblas/rocblas.h>

#include "error.h"
#include "kv_common.h"
#include "kv_internal.h"
#include "model_internal.h"
#include "trace.h"

namespace mckv {
namespace {

constexpr uint32_t kLayers = 42;            // generated_model_config.h:13
constexpr uint32_t kTokensPerPage = 32;     // kv_cache.h:30
constexpr uint32_t kVocab = 130560;         // generated_model_config.h
constexpr int32_t kEos = 130073;            // generated_model_config.h:30
constexpr uint32_t kMaxCtx = 131072;        // generated_model_config.h
constexpr uint32_t kPrefillChunk = 8448;    // prefill_executor.cpp:27
constexpr uint32_t kPrefillChunkMax = 65535;  // prefill_executor.cpp:28

// Tokens per prefill forward: MC_PREFILL_CHUNK, read once per process,
// overrides the 8448 default within [8448, 65535]; any other value keeps
// the default with a warning on stderr (prefill_executor.cpp:30-50).
uint32_t prefill_chunk_tokens() {
    static const uint32_t chunk = [] {
        const char* env = std::getenv("MC_PREFILL_CHUNK");
        if (env == nullptr) return kPrefillChunk;
        char* end = nullptr;
        const unsigned long v = std::strtoul(env, &end, 10);
        if (end == env || *end != '\0' || v < kPrefillChunk || v > kPrefillChunkMax) {
            std::fprintf(stderr,
                         "libminicpm_native: ignoring MC_PREFILL_CHUNK '%s' (a token count "
                         "%u..%u is expected); prefill forwards take %u tokens\n",
                         env, kPrefillChunk, kPrefillChunkMax, kPrefillChunk);
            return kPrefillChunk;
        }
        return (uint32_t)v;
    }();
    return chunk;
}
constexpr uint32_t kMaxSlots = 8;           // batch_group.cpp:52
constexpr double kTheta = 5.0e6;            // generated_model_config.h:23

uint32_t xorshift32(uint32_t x) {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return x;
}
int32_t mock_token(uint32_t seq_len, uint32_t rng) {
    const uint32_t h = (seq_len * 2654435761u) ^ rng;
    return (int32_t)(100u + h % 1000u);
}

struct DevState {
    uint32_t seq_len;
    int32_t next_token;
};

// Per-segment timing of a decode step (the reference's MC_BREAKDOWN /
// MC_BATCH_BREAKDOWN diagnostics, internal_state.h:177-207 and
// batch_group.cpp:55-63): with the variable set when a session (group) is
// created, events are recorded at every segment boundary of an eager step
// and the debug hooks read the segment times of the last step. Steps that
// run as a captured graph record nothing (elapsed times between event nodes
// of a HIP graph are not available), so the hooks then report no step.
// Segments of a step: per layer the qkv row (synthetic, or with weights the
// residual add + norm1 + qkv projection) and the rest of the layer (the phase0
// decode attention: RoPE + K/V write + chunk kernel + merge; with weights also
// the o projection and the MLP), then the tail (with weights the lm_head and
// argmax; token write + sequence advance).
constexpr uint32_t kBdLayerSegs = 2;
constexpr uint32_t kBdEvents = 1 + kLayers * kBdLayerSegs + 1;  // start, boundaries, end
constexpr uint32_t kBdRawSegs = kBdEvents - 1;
constexpr uint32_t kBdBuckets = 3;
const char* const kBdNames[kBdBuckets] = {"qkv(synthetic or norm1+projection)",
                                          "layer(attention[+o+mlp])",
                                          "tail([lm_head+argmax+]token+advance)"};
uint32_t bd_bucket(uint32_t raw) {
    return raw == kBdRawSegs - 1u ? kBdBuckets - 1u : raw % kBdLayerSegs;
}

struct Breakdown {
    bool enabled = false;
    uint32_t used = 0;
    hipEvent_t ev[kBdEvents] = {};

    void init(const char* env) {
        if (std::getenv(env) == nullptr) return;
        for (uint32_t i = 0; i < kBdEvents; ++i)
            if (hipEventCreate(&ev[i]) != hipSuccess) {
                (void)hipGetLastError();
                destroy();  // a diagnostic: silently off when events are unavailable
                return;
            }
        enabled = true;
    }
    void destroy() {
        for (auto& e : ev)
            if (e) {
                (void)hipEventDestroy(e);
                e = nullptr;
            }
        enabled = false;
    }
    void mark(hipStream_t st) {
        if (enabled && used < kBdEvents) (void)hipEventRecord(ev[used++], st);
    }

    // Raw segment k = ev[k] -> ev[k + 1] (ms); false on a HIP error.
    bool segment(uint32_t k, double* ms) const {
        float f = 0.f;
        if (hipEventElapsedTime(&f, ev[k], ev[k + 1]) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        *ms = (double)f;
        return true;
    }
};

size_t align256(size_t x) { return (x + 255u) & ~size_t(255); }

// One captured decode step: the per-layer launches of a step are recorded
// into a HIP graph once and replayed; positions and tokens are read from
// device memory, so replays need no re-capture.
struct StepGraph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

void destroy_graph(StepGraph& g) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
    g = StepGraph{};
}

struct ModelImpl {
    bool weights = false;     // model.wpk loaded: real forward
    ModelWeights w;
    bool use_graphs = false;  // mc_model_options_t::enable_cuda_graph
    int device_id = 0;
    uint32_t max_sessions = 0;
    uint32_t max_ctx = 0;
    std::atomic<uint32_t> live_sessions{0};
    uint64_t total_vram = 0;
};

struct SessionImpl {
    ModelImpl* model = nullptr;
    hipStream_t stream = nullptr;
    void* arena = nullptr;
    size_t arena_bytes = 0;
    // carved buffers
    uint16_t* pool = nullptr;
    uint32_t* d_pt = nullptr;
    int32_t* d_seq = nullptr;
    DevState* d_state = nullptr;
    float* inv_freq = nullptr;
    uint16_t* qkv = nullptr;       // [chunk][2560]
    uint16_t* attn_out = nullptr;  // [chunk][2048]
    float* partials = nullptr;     // decode level-1
    float* partials2 = nullptr;    // decode level-2
    float* pf_partials = nullptr;  // prefill split partials
    mc_kv_allocator_t* kv = nullptr;
    mc_kv_layout_t layout{};
    uint32_t chunk_pos = 64, max_chunks = 0, act_rows = 0;
    // host state
    uint32_t seq_len = 0;
    uint32_t rng = 0;
    bool rng_seeded = false;
    bool in_group = false;
    DevState h_state{};
    int32_t h_tok = 0;
    mc_runtime_stats_t total{}, since_reset{};
    uint64_t min_free = ~0ull;
    StepGraph step_graph;
    uint64_t graph_launches = 0;
    bool graph_off = false;  // mc_debug_session_set_graph_enabled(s, 0)
    uint32_t debug_step = 0;  // forwards since create / reset (debug dump step numbers)
    uint32_t rope_snapshot[64] = {};  // inv_freq words at create
    bool rope_snapshot_valid = false;
    Breakdown bd;
    // with weights
    Forward fwd;
    void* blas = nullptr;  // prefill GEMM libraries (prefill_blas_create)
    int32_t* h_emit = nullptr;  // pinned: the token a decode returns
};

struct GroupImpl {
    ModelImpl* model = nullptr;
    hipStream_t stream = nullptr;
    uint32_t max_slots = 0, max_ctx = 0, chunk_pos = 64, max_chunks = 0;
    SessionImpl* members[kMaxSlots] = {};
    void* arena = nullptr;
    // device tables (fixed addresses) of the current step's members
    uint32_t** d_pos = nullptr;
    uint32_t** d_pt = nullptr;
    uint16_t** d_kv = nullptr;
    int32_t** d_tok = nullptr;
    int32_t** d_seq = nullptr;
    uint16_t* qkv = nullptr;
    uint16_t* out = nullptr;
    float* partials = nullptr;
    float* partials2 = nullptr;
    float* inv_freq = nullptr;
    void* h_tables = nullptr;  // pinned staging: 5 x kMaxSlots pointers
    int32_t* h_tok = nullptr;  // pinned staging of the step's tokens
    hipEvent_t ev = nullptr;
    mc_kv_layout_t layout{};
    StepGraph step_graph[kMaxSlots + 1];  // by the number of slots in the step
    uint64_t steps = 0, decode_us = 0;
    Breakdown bd;
    Forward fwd;  // with weights: activation rows of a step
    int32_t last_row[kMaxSlots];  // logits row of each slot in the last step, or -1
};

mc_status_t set_device(int id, const char* who) {
    const hipError_t e = hipSetDevice(id);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error("%s: hipSetDevice(%d) failed: %s", who, id, hipGetErrorString(e));
        return MC_E_CUDA;
    }
    return MC_OK;
}

#define HIP_OR_RETURN(call, what)                          \
    do {                                                   \
        const hipError_t _e = (call);                      \
        if (_e != hipSuccess) return check_hip(_e, what);  \
    } while (0)
#define MC_OR_RETURN(call)                 \
    do {                                   \
        const mc_status_t _s = (call);     \
        if (_s != MC_OK) return _s;        \
    } while (0)

// Runs `body` (launches on st): eagerly, or through a graph captured at the
// first call and replayed afterwards.
template <class F>
mc_status_t run_step(bool use_graph, StepGraph& sg, hipStream_t st, F&& body) {
    if (!use_graph) return body();
    if (sg.exec == nullptr) {
        HIP_OR_RETURN(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal),
                      "decode step: hipStreamBeginCapture failed");
        const mc_status_t bs = body();
        hipGraph_t graph = nullptr;
        const hipError_t e = hipStreamEndCapture(st, &graph);
        if (bs != MC_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return bs;
        }
        if (e != hipSuccess) return check_hip(e, "decode step: hipStreamEndCapture failed");
        const hipError_t e2 = hipGraphInstantiate(&sg.exec, graph, nullptr, nullptr, 0);
        if (e2 != hipSuccess) {
            (void)hipGraphDestroy(graph);
            sg.exec = nullptr;
            return check_hip(e2, "decode step: hipGraphInstantiate failed");
        }
        sg.graph = graph;
    }
    HIP_OR_RETURN(hipGraphLaunch(sg.exec, st), "decode step: hipGraphLaunch failed");
    return MC_OK;
}

void release_session(SessionImpl* s) {
    if (s == nullptr) return;
    (void)hipSetDevice(s->model->device_id);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    destroy_graph(s->step_graph);
    s->bd.destroy();
    prefill_blas_destroy(s->blas);
    if (s->h_emit) (void)hipHostFree(s->h_emit);
    if (s->kv) mc_kv_allocator_destroy(s->kv);
    if (s->arena) (void)hipFree(s->arena);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    s->model->live_sessions.fetch_sub(1);
    delete s;
}

void release_group(GroupImpl* g) {
    if (g == nullptr) return;
    (void)hipSetDevice(g->model->device_id);
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    for (uint32_t i = 0; i < kMaxSlots; ++i)
        if (g->members[i]) {
            // remove semantics: group work visible to the member's stream
            if (g->ev) {
                (void)hipEventRecord(g->ev, g->stream);
                (void)hipStreamWaitEvent(g->members[i]->stream, g->ev, 0);
            }
            g->members[i]->in_group = false;
            g->members[i] = nullptr;
        }
    if (g->ev) (void)hipEventDestroy(g->ev);
    for (auto& sg : g->step_graph) destroy_graph(sg);
    g->bd.destroy();
    if (g->h_tables) (void)hipHostFree(g->h_tables);
    if (g->h_tok) (void)hipHostFree(g->h_tok);
    if (g->arena) (void)hipFree(g->arena);
    if (g->stream) (void)hipStreamDestroy(g->stream);
    delete g;
}

// Runs the synthetic forward of one prefill chunk: per layer synthetic rows,
// RoPE + K/V append, paged prefill attention.
mc_status_t prefill_chunk(SessionImpl& s, uint32_t base, uint32_t n, bool first) {
    hipStream_t st = s.stream;
    s.h_state.seq_len = base;
    HIP_OR_RETURN(hipMemcpyAsync(&s.d_state->seq_len, &s.h_state.seq_len, sizeof(uint32_t),
                                 hipMemcpyHostToDevice, st),
                  "mc_prefill: d_state H2D failed");
    if (s.model->weights) {
        // the greedy prediction after the chunk's last token goes to
        // d_state.next_token, the token the first decode returns
        s.fwd.dump_step = s.debug_step;
        s.fwd.dump_layers = first;  // layer rows: the first chunk of the prefill
        s.fwd.keys = base + n;
        const mc_status_t fs =
            forward_prefill(s.fwd, s.d_seq + base, n, &s.d_state->next_token);
        s.debug_step += 1;
        MC_OR_RETURN(fs);
        HIP_OR_RETURN(hipStreamSynchronize(st), "mc_prefill: stream sync failed");
        return prefill_barrier_check("mc_prefill");
    }
    const uint32_t S = mc_kv_prefill_split_kv(n);
    for (uint32_t l = 0; l < kLayers; ++l) {
        MC_OR_RETURN(launch_synth_qkv(s.qkv, n, s.d_seq + base, &s.d_state->seq_len, l, st));
        MC_OR_RETURN(mc_kv_rope_append(s.qkv, n, &s.d_state->seq_len, l, s.d_pt, s.pool,
                                       s.layout, kTheta, s.inv_freq, st));
        MC_OR_RETURN(mc_kv_attention_prefill(s.qkv, n, &s.d_state->seq_len, l, s.d_pt,
                                             s.pool, s.layout, s.attn_out,
                                             S > 1u ? s.pf_partials : nullptr, S, st));
    }
    // The stream still reads h_state.seq_len's copy source asynchronously; keep
    // the host value stable until the caller synchronizes.
    HIP_OR_RETURN(hipStreamSynchronize(st), "mc_prefill: stream sync failed");
    return prefill_barrier_check("mc_prefill");
}

}  // namespace
}  // namespace mckv

using namespace mckv;

struct mc_model {
    ModelImpl* impl;
};
struct mc_session {
    SessionImpl* impl;
};
struct mc_batch_group {
    GroupImpl* impl;
};

extern "C" {

mc_status_t mc_model_load(const char* model_dir, const mc_model_options_t* options,
                          mc_model_t* out_model) {
    MC_GUARD_BEGIN
    if (out_model) *out_model = mc_model{nullptr};
    if (model_dir == nullptr || options == nullptr || out_model == nullptr) {
        set_error("mc_model_load: a required pointer argument (model_dir, options, out_model) is null");
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->struct_size != sizeof(mc_model_options_t)) {
        set_error("mc_model_load: options struct is %u bytes, this library expects %zu",
                  options->struct_size, sizeof(mc_model_options_t));
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->abi_version != MC_ABI_VERSION) {
        set_error("mc_model_load: caller built against ABI 0x%08x, library implements 0x%08x",
                  options->abi_version, MC_ABI_VERSION);
        return MC_E_INVALID_ARGUMENT;
    }
    // Order and status codes of the reference's checks (model.cpp:58-100):
    // weight and cache precision first (MC_E_UNSUPPORTED), then device,
    // sessions and a zero context (MC_E_INVALID_ARGUMENT), then a context
    // beyond the model's limit (MC_E_UNSUPPORTED).
    // MC_FP8 is the reference's dual copy (model.cpp:68-80,198-230): bf16
    // weights for prefill and batch steps, e4m3 ones for single-token decode
    if (options->precision != MC_BF16 && options->precision != MC_FP8) {
        set_error("mc_model_load: weight precision %d not supported (MC_BF16, or MC_FP8 with the "
                  "bf16 package for prefill)",
                  (int)options->precision);
        return MC_E_UNSUPPORTED;
    }
    if (options->kv_precision != MC_KV_BF16) {
        set_error("mc_model_load: KV cache precision %d not supported (MC_KV_BF16 only)",
                  (int)options->kv_precision);
        return MC_E_UNSUPPORTED;
    }
    if (options->device_id < 0) {
        set_error("mc_model_load: device_id %d is negative", options->device_id);
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->max_sessions == 0) {
        set_error("mc_model_load: max_sessions is 0 (at least one session is needed)");
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->max_context_tokens == 0) {
        set_error("mc_model_load: max_context_tokens is 0");
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->max_context_tokens > kMaxCtx) {
        set_error("mc_model_load: max_context_tokens %u is beyond the model's %u positions",
                  options->max_context_tokens, kMaxCtx);
        return MC_E_UNSUPPORTED;
    }
    struct stat st {};
    if (stat(model_dir, &st) != 0 || !S_ISDIR(st.st_mode)) {
        set_error("mc_model_load: cannot open model directory '%s'", model_dir);
        return MC_E_IO;
    }
    const std::string wpk = std::string(model_dir) + "/model.wpk";
    const bool has_wpk = stat(wpk.c_str(), &st) == 0;
    const std::string wpk8 = std::string(model_dir) + "/model_fp8.wpk";
    const bool fp8 = options->precision == MC_FP8;
    if (fp8 && (!has_wpk || stat(wpk8.c_str(), &st) != 0)) {
        // FP8 has no weight-free form (model.cpp:203-213)
        set_error("mc_model_load: precision MC_FP8 needs model.wpk (bf16 weights for prefill) "
                  "and model_fp8.wpk (e4m3 weights and row scales) in '%s'",
                  model_dir);
        return MC_E_MODEL_MISMATCH;
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return check_hip(e, "mc_model_load: hipGetDeviceCount failed");
    if (options->device_id >= count) {
        set_error("mc_model_load: no device %d (%d visible)",
                  options->device_id, count);
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(options->device_id, "mc_model_load"));
    hipDeviceProp_t prop{};
    e = hipGetDeviceProperties(&prop, options->device_id);
    if (e != hipSuccess) return check_hip(e, "mc_model_load: hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("mc_model_load: device %d reports architecture '%s'; the kernels are built for gfx950 (MI355X)",
                  options->device_id, prop.gcnArchName);
        return MC_E_MODEL_MISMATCH;
    }
    auto* m = new ModelImpl();
    m->device_id = options->device_id;
    m->max_sessions = options->max_sessions;
    m->max_ctx = options->max_context_tokens;
    m->use_graphs = options->enable_cuda_graph != 0u;
    m->total_vram = prop.totalGlobalMem;
    if (has_wpk) {
        hipStream_t ls = nullptr;
        e = hipStreamCreate(&ls);
        if (e != hipSuccess) {
            delete m;
            return check_hip(e, "mc_model_load: hipStreamCreate failed");
        }
        uint64_t bytes = 0;
        mc_status_t rs = wpk_load(wpk.c_str(), &m->w, &bytes, ls);
        if (rs == MC_OK && fp8) {
            rs = wpk_load_fp8(wpk8.c_str(), &m->w, &bytes, ls);
            if (rs != MC_OK) wpk_free(&m->w);
        }
        (void)hipStreamDestroy(ls);
        if (rs != MC_OK) {
            delete m;
            return rs;
        }
        m->weights = true;
    }
    *out_model = mc_model{m};
    return MC_OK;
    MC_GUARD_END
}

void mc_model_destroy(mc_model_t model) {
    ModelImpl* m = model.impl;
    if (m == nullptr) return;
    if (m->weights) {
        (void)hipSetDevice(m->device_id);
        wpk_free(&m->w);
    }
    delete m;
}

mc_status_t mc_session_create(mc_model_t model, mc_session_t* out_session) {
    MC_GUARD_BEGIN
    if (out_session) *out_session = mc_session{nullptr};
    if (model.impl == nullptr || out_session == nullptr) {
        set_error("mc_session_create: model handle or out_session is null");
        return MC_E_INVALID_ARGUMENT;
    }
    ModelImpl* m = model.impl;
    MC_OR_RETURN(set_device(m->device_id, "mc_session_create"));
    if (m->live_sessions.fetch_add(1) + 1 > m->max_sessions) {
        m->live_sessions.fetch_sub(1);
        set_error("mc_session_create: the model already has its max_sessions (%u) live sessions",
                  m->max_sessions);
        return MC_E_UNSUPPORTED;
    }
    auto* s = new SessionImpl();
    s->model = m;
    hipError_t e = hipStreamCreate(&s->stream);
    if (e != hipSuccess) {
        release_session(s);
        return check_hip(e, "mc_session_create: hipStreamCreate failed");
    }
    s->bd.init("MC_BREAKDOWN");
    const uint32_t max_pages = (m->max_ctx + kTokensPerPage - 1u) / kTokensPerPage;
    s->layout = mc_kv_layout_t{max_pages, kTokensPerPage, kLayers, 0};
    s->chunk_pos = mc_kv_decode_chunk_pos(m->max_ctx);
    s->max_chunks = mc_kv_decode_max_chunks(m->max_ctx, s->chunk_pos);
    s->act_rows = std::min(m->max_ctx, prefill_chunk_tokens());
    const size_t pool_b = (size_t)mc_kv_total_elems(s->layout) * 2u;
    // With weights: the prefill projections' rocBLAS and hipBLASLt handles get
    // their device workspace from the arena, so neither allocates after create.
    size_t blas_ws = 0;
    if (m->weights) {
        const mc_status_t bs = prefill_blas_create(&s->blas, &blas_ws);
        if (bs != MC_OK) {
            release_session(s);
            return bs;
        }
    }
    const size_t sizes[] = {
        pool_b,
        (size_t)max_pages * 4u,
        (size_t)m->max_ctx * 4u,
        sizeof(DevState),
        64u * 4u,
        (size_t)s->act_rows * kRow * 2u,
        (size_t)s->act_rows * 2048u * 2u,
        (size_t)kHq * s->max_chunks * kPartial * 4u,
        (size_t)kHq * kSplit2 * kPartial * 4u,
        (size_t)4096u * kHq * kPartial * 4u,  // prefill: T * S_kv <= 4096
        m->weights ? forward_act_bytes(s->act_rows, 1u) : 0u,
        blas_ws,
    };
    size_t total = 0;
    for (size_t b : sizes) total += align256(b);
    e = hipMalloc(&s->arena, total);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        size_t fr = 0, tt = 0;
        (void)hipMemGetInfo(&fr, &tt);
        set_error("mc_session_create: session arena allocation failed: need %zu bytes but "
                  "free VRAM is %zu bytes (max_context_tokens=%u)",
                  total, fr, m->max_ctx);
        release_session(s);
        return MC_E_OUT_OF_MEMORY;
    }
    s->arena_bytes = total;
    char* p = static_cast<char*>(s->arena);
    void* bufs[12];
    for (int i = 0; i < 12; ++i) {
        bufs[i] = p;
        p += align256(sizes[i]);
    }
    s->pool = (uint16_t*)bufs[0];
    s->d_pt = (uint32_t*)bufs[1];
    s->d_seq = (int32_t*)bufs[2];
    s->d_state = (DevState*)bufs[3];
    s->inv_freq = (float*)bufs[4];
    s->qkv = (uint16_t*)bufs[5];
    s->attn_out = (uint16_t*)bufs[6];
    s->partials = (float*)bufs[7];
    s->partials2 = (float*)bufs[8];
    s->pf_partials = (float*)bufs[9];
    mc_status_t rs = mc_kv_allocator_create(s->d_pt, max_pages, kTokensPerPage, &s->kv);
    if (rs == MC_OK) rs = mc_kv_rope_inv_freq_init(s->inv_freq, kTheta, s->stream);
    if (rs == MC_OK && m->weights) {
        Forward& f = s->fwd;
        forward_carve(f, static_cast<char*>(bufs[10]), s->act_rows, 1u);
        f.w = &m->w;
        f.st = s->stream;
        f.pool = s->pool;
        f.d_pt = s->d_pt;
        f.layout = s->layout;
        f.d_seq_len = &s->d_state->seq_len;
        f.inv_freq = s->inv_freq;
        f.partials = s->partials;
        f.partials2 = s->partials2;
        f.pf_partials = s->pf_partials;
        f.max_chunks = s->max_chunks;
        f.chunk_pos = s->chunk_pos;
        rs = prefill_blas_workspace(s->blas, bufs[11], blas_ws);
        if (rs == MC_OK) {
            f.blas = s->blas;
            e = hipHostMalloc((void**)&s->h_emit, sizeof(int32_t));
            if (e != hipSuccess) rs = check_hip(e, "mc_session_create: pinned token buffer");
        }
    }
    if (rs == MC_OK) {
        e = hipMemsetAsync(s->d_state, 0, sizeof(DevState), s->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
        // create-time snapshot of the RoPE table (mc_debug_session_rope_intact)
        if (e == hipSuccess)
            e = hipMemcpy(s->rope_snapshot, s->inv_freq, sizeof(s->rope_snapshot),
                          hipMemcpyDeviceToHost);
        if (e != hipSuccess) rs = check_hip(e, "mc_session_create: init failed");
        else s->rope_snapshot_valid = true;
    }
    if (rs != MC_OK) {
        release_session(s);
        return rs;
    }
    *out_session = mc_session{s};
    return MC_OK;
    MC_GUARD_END
}

mc_status_t mc_session_reset(mc_session_t session) {
    MC_GUARD_BEGIN
    SessionImpl* s = session.impl;
    if (s == nullptr) {
        set_error("mc_session_reset: null session handle");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_session_reset"));
    mc_kv_allocator_release_all(s->kv);
    s->seq_len = 0;
    s->debug_step = 0;
    s->rng_seeded = false;
    s->since_reset = mc_runtime_stats_t{};
    s->h_state = DevState{};
    HIP_OR_RETURN(hipMemcpyAsync(s->d_state, &s->h_state, sizeof(DevState),
                                 hipMemcpyHostToDevice, s->stream),
                  "mc_session_reset: d_state H2D failed");
    HIP_OR_RETURN(hipStreamSynchronize(s->stream), "mc_session_reset: sync failed");
    return MC_OK;
    MC_GUARD_END
}

void mc_session_destroy(mc_session_t session) { release_session(session.impl); }

mc_status_t mc_prefill(mc_session_t session, const int32_t* token_ids,
                       uint32_t token_count) {
    MC_GUARD_BEGIN
    SessionImpl* s = session.impl;
    if (s == nullptr) {
        set_error("mc_prefill: null session handle");
        return MC_E_INVALID_ARGUMENT;
    }
    if (token_ids == nullptr || token_count == 0) {
        set_error("mc_prefill: empty prompt (token_ids null or token_count 0)");
        return MC_E_INVALID_ARGUMENT;
    }
    if (s->in_group) {
        set_error("mc_prefill: session is attached to a batch group; remove it before solo use");
        return MC_E_UNSUPPORTED;
    }
    const uint32_t max_ctx = s->model->max_ctx;
    if (token_count > max_ctx - s->seq_len) {
        set_error("mc_prefill: %u more tokens do not fit the %u-token context "
                  "(%u already cached)",
                  token_count, max_ctx, s->seq_len);
        return MC_E_OUT_OF_MEMORY;
    }
    for (uint32_t i = 0; i < token_count; ++i)
        if (token_ids[i] < 0 || (uint32_t)token_ids[i] >= kVocab) {
            set_error("mc_prefill: token %u has id %d, outside the vocabulary (size %u)", i, token_ids[i],
                      kVocab);
            return MC_E_INVALID_ARGUMENT;
        }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_prefill"));
    const auto t0 = std::chrono::steady_clock::now();
    TraceRange trace_range("mc_prefill");
    const uint32_t base = s->seq_len;
    HIP_OR_RETURN(hipMemcpyAsync(s->d_seq + base, token_ids, (size_t)token_count * 4u,
                                 hipMemcpyHostToDevice, s->stream),
                  "mc_prefill: token H2D copy failed");
    MC_OR_RETURN(mc_kv_allocator_ensure_pages_for(s->kv, base + token_count, s->stream));
    for (uint32_t off = 0; off < token_count;) {
        const uint32_t n =
            token_count - off > s->act_rows ? s->act_rows : token_count - off;
        MC_OR_RETURN(prefill_chunk(*s, base + off, n, off == 0u));
        off += n;
    }
    s->seq_len = base + token_count;
    s->h_state.seq_len = s->seq_len;
    // weight-free mode: the next decode continues from the last prompt token;
    // with weights the prefill wrote its prediction to d_state.next_token
    if (!s->model->weights) s->h_state.next_token = token_ids[token_count - 1];
    HIP_OR_RETURN(hipMemcpyAsync(s->d_state, &s->h_state,
                                 s->model->weights ? sizeof(uint32_t) : sizeof(DevState),
                                 hipMemcpyHostToDevice, s->stream),
                  "mc_prefill: d_state H2D update failed");
    HIP_OR_RETURN(hipStreamSynchronize(s->stream), "mc_prefill: stream sync failed");
    const uint64_t us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                            std::chrono::steady_clock::now() - t0)
                            .count();
    s->total.prompt_tokens += token_count;
    s->since_reset.prompt_tokens += token_count;
    s->total.prefill_us += us;
    s->since_reset.prefill_us += us;
    return MC_OK;
    MC_GUARD_END
}

mc_status_t mc_decode_one(mc_session_t session, const mc_generation_config_t* config,
                          int32_t* out_token) {
    MC_GUARD_BEGIN
    SessionImpl* s = session.impl;
    if (s == nullptr || config == nullptr || out_token == nullptr) {
        set_error("mc_decode_one: a required pointer argument (session, config, out_token) is null");
        return MC_E_INVALID_ARGUMENT;
    }
    if (config->struct_size != sizeof(*config)) {
        set_error("mc_decode_one: generation config is %u bytes, this library expects %zu",
                  config->struct_size, sizeof(*config));
        return MC_E_INVALID_ARGUMENT;
    }
    if (config->max_new_tokens == 0) {
        set_error("mc_decode_one: max_new_tokens is 0");
        return MC_E_INVALID_ARGUMENT;
    }
    if (s->in_group) {
        set_error("mc_decode_one: session is attached to a batch group; remove it before solo use");
        return MC_E_UNSUPPORTED;
    }
    if (s->model->weights && config->temperature > 0.f && config->top_k != 1u) {
        set_error("mc_decode_one: the config asks for sampling; this build decodes greedily "
                  "(temperature <= 0 or top_k == 1)");
        return MC_E_UNSUPPORTED;
    }
    if (s->seq_len == 0) {
        set_error("mc_decode_one: nothing to continue: prefill a prompt first");
        return MC_E_INVALID_ARGUMENT;
    }
    if (s->seq_len >= s->model->max_ctx) {
        set_error("mc_decode_one: no room for another token (%u of %u positions used)", s->seq_len,
                  s->model->max_ctx);
        return MC_E_OUT_OF_MEMORY;
    }
    if (s->since_reset.generated_tokens >= config->max_new_tokens) {
        *out_token = kEos;
        return MC_OK;
    }
    if (!s->rng_seeded) {
        s->rng = (uint32_t)config->seed;
        s->rng_seeded = true;
    }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_decode_one"));
    const auto t0 = std::chrono::steady_clock::now();
    hipStream_t st = s->stream;
    MC_OR_RETURN(mc_kv_allocator_ensure_pages_for(s->kv, s->seq_len + 1u, st));
    TraceRange trace_range("mc_decode_one");
    // a step that writes debug dump files runs eagerly (the files are written
    // from the host between its kernels)
    const bool dumping = s->model->weights && dump_due(s->debug_step);
    const bool graph = s->model->use_graphs && !s->graph_off && !dumping;
    if (s->model->weights) {
        s->fwd.dump_step = s->debug_step;
        s->fwd.dump_layers = false;
        // returns the token the previous forward predicted; the forward on it
        // (position seq_len) predicts the next one into d_state.next_token
        HIP_OR_RETURN(hipMemcpyAsync(s->h_emit, &s->d_state->next_token, 4u,
                                     hipMemcpyDeviceToHost, st),
                      "mc_decode_one: token D2H failed");
        s->bd.used = graph ? kBdEvents + 1u : 0u;
        const Marker mark{[](void* c) {
                              auto* ss = static_cast<SessionImpl*>(c);
                              ss->bd.mark(ss->stream);
                          },
                          s};
        MC_OR_RETURN(run_step(graph, s->step_graph, st, [&]() -> mc_status_t {
            s->bd.mark(st);
            return forward_decode(s->fwd, &s->d_state->next_token, &s->d_state->next_token,
                                  mark);
        }));
        s->debug_step += 1;
        if (graph) s->graph_launches += 1;
        MC_OR_RETURN(mc_kv_decode_advance(s->d_seq, &s->d_state->next_token,
                                          &s->d_state->seq_len, st));
        s->bd.mark(st);
        HIP_OR_RETURN(hipStreamSynchronize(st), "mc_decode_one: stream sync failed");
        const int32_t emitted = *s->h_emit;
        if (emitted < 0 || (uint32_t)emitted >= kVocab) {
            set_error("mc_decode_one: the forward produced token id %d, outside the vocabulary",
                      emitted);
            return MC_E_INTERNAL;
        }
        s->seq_len += 1;
        s->h_state.seq_len = s->seq_len;
        s->rng = xorshift32(s->rng);
        const uint64_t us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                                std::chrono::steady_clock::now() - t0)
                                .count();
        s->total.generated_tokens += 1;
        s->since_reset.generated_tokens += 1;
        s->total.decode_us += us;
        s->since_reset.decode_us += us;
        *out_token = emitted;
        return MC_OK;
    }
    // Per layer: synthetic row of (d_next_token, seq_len), phase0 decode
    // attention at limit = seq_len (appends K/V of that position).
    s->bd.used = graph ? kBdEvents + 1u : 0u;  // graph steps: nothing recorded
    MC_OR_RETURN(run_step(graph, s->step_graph, st, [&]() -> mc_status_t {
        s->bd.mark(st);
        for (uint32_t l = 0; l < kLayers; ++l) {
            MC_OR_RETURN(launch_synth_qkv(s->qkv, 1, &s->d_state->next_token,
                                          &s->d_state->seq_len, l, st));
            s->bd.mark(st);
            MC_OR_RETURN(mc_kv_attention_decode(s->qkv, &s->d_state->seq_len, l, s->d_pt,
                                                s->pool, s->layout, s->partials,
                                                s->max_chunks, s->attn_out, st, s->inv_freq,
                                                s->chunk_pos, s->partials2));
            s->bd.mark(st);
        }
        return MC_OK;
    }));
    if (graph) s->graph_launches += 1;
    s->h_tok = mock_token(s->seq_len, s->rng);
    HIP_OR_RETURN(hipMemcpyAsync(&s->d_state->next_token, &s->h_tok, 4u,
                                 hipMemcpyHostToDevice, st),
                  "mc_decode_one: token H2D failed");
    MC_OR_RETURN(mc_kv_decode_advance(s->d_seq, &s->d_state->next_token,
                                      &s->d_state->seq_len, st));
    s->bd.mark(st);
    HIP_OR_RETURN(hipStreamSynchronize(st), "mc_decode_one: stream sync failed");
    s->seq_len += 1;
    s->h_state.seq_len = s->seq_len;
    s->h_state.next_token = s->h_tok;
    s->rng = xorshift32(s->rng);
    const uint64_t us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                            std::chrono::steady_clock::now() - t0)
                            .count();
    s->total.generated_tokens += 1;
    s->since_reset.generated_tokens += 1;
    s->total.decode_us += us;
    s->since_reset.decode_us += us;
    *out_token = s->h_tok;
    return MC_OK;
    MC_GUARD_END
}

mc_status_t mc_get_stats(mc_session_t session, mc_runtime_stats_t* out_stats) {
    MC_GUARD_BEGIN
    SessionImpl* s = session.impl;
    if (s == nullptr || out_stats == nullptr) {
        set_error("mc_get_stats: session handle or out_stats is null");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_get_stats"));
    size_t fr = 0, tt = 0;
    HIP_OR_RETURN(hipMemGetInfo(&fr, &tt), "mc_get_stats: hipMemGetInfo failed");
    if (fr < s->min_free) s->min_free = fr;
    *out_stats = s->total;
    out_stats->peak_vram_bytes = s->model->total_vram - s->min_free;
    out_stats->cuda_graph_launches = s->graph_launches;
    return MC_OK;
    MC_GUARD_END
}

// ---------------- batch group ----------------

mc_status_t mc_batch_group_create(mc_model_t model, const mc_batch_options_t* options,
                                  mc_batch_group_t* out_group) {
    MC_GUARD_BEGIN
    if (out_group) *out_group = mc_batch_group{nullptr};
    if (model.impl == nullptr) {
        set_error("mc_batch_group_create: null model handle");
        return MC_E_INVALID_ARGUMENT;
    }
    if (options == nullptr || out_group == nullptr) {
        set_error("mc_batch_group_create: options or out_group is null");
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->struct_size != sizeof(mc_batch_options_t)) {
        set_error("mc_batch_group_create: options struct is %u bytes, this library expects %zu",
                  options->struct_size, sizeof(mc_batch_options_t));
        return MC_E_INVALID_ARGUMENT;
    }
    if (options->abi_version != MC_ABI_VERSION) {
        set_error("mc_batch_group_create: caller built against ABI 0x%08x, library implements 0x%08x",
                  options->abi_version, MC_ABI_VERSION);
        return MC_E_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < 4; ++i)
        if (options->reserved[i] != 0) {
            set_error("mc_batch_group_create: options->reserved[%u] is set; reserved words must be 0", i);
            return MC_E_INVALID_ARGUMENT;
        }
    if (options->max_slots == 0 || options->max_slots > kMaxSlots) {
        set_error("mc_batch_group_create: max_slots %u not supported (allowed 1..%u)",
                  options->max_slots, kMaxSlots);
        return MC_E_UNSUPPORTED;
    }
    ModelImpl* m = model.impl;
    if (options->max_context_tokens != m->max_ctx) {
        set_error("mc_batch_group_create: group context %u differs from the model's %u tokens",
                  options->max_context_tokens, m->max_ctx);
        return MC_E_UNSUPPORTED;
    }
    MC_OR_RETURN(set_device(m->device_id, "mc_batch_group_create"));
    auto* g = new GroupImpl();
    g->model = m;
    for (auto& r : g->last_row) r = -1;
    g->max_slots = options->max_slots;
    g->max_ctx = m->max_ctx;
    g->chunk_pos = mc_kv_decode_chunk_pos(m->max_ctx);
    g->max_chunks = mc_kv_decode_max_chunks(m->max_ctx, g->chunk_pos);
    hipError_t e = hipStreamCreate(&g->stream);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&g->ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        release_group(g);
        return check_hip(e, "mc_batch_group_create: stream/event creation failed");
    }
    g->bd.init("MC_BATCH_BREAKDOWN");
    const uint32_t B = kMaxSlots;
    const size_t sizes[] = {
        5u * B * sizeof(void*),
        (size_t)B * kRow * 2u,
        (size_t)B * 2048u * 2u,
        (size_t)B * kHq * g->max_chunks * kPartial * 4u,
        (size_t)B * kHq * kSplit2 * kPartial * 4u,
        64u * 4u,
        m->weights ? forward_act_bytes(B, B) : 0u,
    };
    size_t total = 0;
    for (size_t b : sizes) total += align256(b);
    e = hipMalloc(&g->arena, total);
    if (e == hipSuccess) e = hipHostMalloc(&g->h_tables, 5u * B * sizeof(void*));
    if (e == hipSuccess) e = hipHostMalloc((void**)&g->h_tok, B * sizeof(int32_t));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error("mc_batch_group_create: could not allocate the group's %zu-byte device arena", total);
        release_group(g);
        return MC_E_OUT_OF_MEMORY;
    }
    char* p = static_cast<char*>(g->arena);
    void** tables = reinterpret_cast<void**>(p);
    g->d_pos = reinterpret_cast<uint32_t**>(tables);
    g->d_pt = reinterpret_cast<uint32_t**>(tables + B);
    g->d_kv = reinterpret_cast<uint16_t**>(tables + 2u * B);
    g->d_tok = reinterpret_cast<int32_t**>(tables + 3u * B);
    g->d_seq = reinterpret_cast<int32_t**>(tables + 4u * B);
    p += align256(sizes[0]);
    g->qkv = (uint16_t*)p;
    p += align256(sizes[1]);
    g->out = (uint16_t*)p;
    p += align256(sizes[2]);
    g->partials = (float*)p;
    p += align256(sizes[3]);
    g->partials2 = (float*)p;
    p += align256(sizes[4]);
    g->inv_freq = (float*)p;
    p += align256(sizes[5]);
    if (m->weights) {
        Forward& f = g->fwd;
        forward_carve(f, p, B, B);
        f.w = &m->w;
        f.st = g->stream;
        f.inv_freq = g->inv_freq;
        f.partials = g->partials;
        f.partials2 = g->partials2;
        f.max_chunks = g->max_chunks;
        f.chunk_pos = g->chunk_pos;
    }
    mc_status_t rs = mc_kv_rope_inv_freq_init(g->inv_freq, kTheta, g->stream);
    if (rs == MC_OK) {
        e = hipStreamSynchronize(g->stream);
        if (e != hipSuccess) rs = check_hip(e, "mc_batch_group_create: init sync failed");
    }
    if (rs != MC_OK) {
        release_group(g);
        return rs;
    }
    *out_group = mc_batch_group{g};
    return MC_OK;
    MC_GUARD_END
}

mc_status_t mc_batch_group_add(mc_batch_group_t group, mc_session_t session,
                               uint32_t* slot_id) {
    MC_GUARD_BEGIN
    GroupImpl* g = group.impl;
    if (g == nullptr) {
        set_error("mc_batch_group_add: null group handle");
        return MC_E_INVALID_ARGUMENT;
    }
    SessionImpl* s = session.impl;
    if (s == nullptr || slot_id == nullptr) {
        set_error("mc_batch_group_add: session handle or slot_id is null");
        return MC_E_INVALID_ARGUMENT;
    }
    if (s->model != g->model) {
        set_error("mc_batch_group_add: session was created from another model than the group");
        return MC_E_UNSUPPORTED;
    }
    if (s->chunk_pos != g->chunk_pos || s->max_chunks != g->max_chunks) {
        set_error("mc_batch_group_add: session and group use different decode chunk tiers");
        return MC_E_UNSUPPORTED;
    }
    if (s->in_group) {
        set_error("mc_batch_group_add: session is attached to a batch group already");
        return MC_E_UNSUPPORTED;
    }
    uint32_t slot = g->max_slots;
    for (uint32_t i = 0; i < g->max_slots; ++i)
        if (g->members[i] == nullptr) {
            slot = i;
            break;
        }
    if (slot == g->max_slots) {
        set_error("mc_batch_group_add: all %u slots are taken", g->max_slots);
        return MC_E_UNSUPPORTED;
    }
    MC_OR_RETURN(set_device(g->model->device_id, "mc_batch_group_add"));
    // member -> group: the member's earlier prefill/KV writes are visible.
    HIP_OR_RETURN(hipEventRecord(g->ev, s->stream),
                  "mc_batch_group_add: event chain (member->group) failed");
    HIP_OR_RETURN(hipStreamWaitEvent(g->stream, g->ev, 0),
                  "mc_batch_group_add: event chain (member->group) failed");
    g->members[slot] = s;
    s->in_group = true;
    *slot_id = slot;
    return MC_OK;
    MC_GUARD_END
}

mc_status_t mc_batch_group_remove(mc_batch_group_t group, uint32_t slot_id) {
    MC_GUARD_BEGIN
    GroupImpl* g = group.impl;
    if (g == nullptr) {
        set_error("mc_batch_group_remove: null group handle");
        return MC_E_INVALID_ARGUMENT;
    }
    if (slot_id >= g->max_slots || g->members[slot_id] == nullptr) {
        set_error("mc_batch_group_remove: slot %u is empty", slot_id);
        return MC_E_INVALID_ARGUMENT;
    }
    SessionImpl* s = g->members[slot_id];
    MC_OR_RETURN(set_device(g->model->device_id, "mc_batch_group_remove"));
    // group -> member: the group's KV / sequence writes are visible to solo use.
    HIP_OR_RETURN(hipEventRecord(g->ev, g->stream),
                  "mc_batch_group_remove: event chain (group->member) failed");
    HIP_OR_RETURN(hipStreamWaitEvent(s->stream, g->ev, 0),
                  "mc_batch_group_remove: event chain (group->member) failed");
    s->in_group = false;
    g->members[slot_id] = nullptr;
    return MC_OK;
    MC_GUARD_END
}

mc_status_t mc_batch_step(mc_batch_group_t group, const uint32_t* slot_ids, uint32_t n,
                          const mc_generation_config_t* cfgs, int32_t* out_tokens) {
    MC_GUARD_BEGIN
    GroupImpl* g = group.impl;
    if (g == nullptr) {
        set_error("mc_batch_step: null group handle");
        return MC_E_INVALID_ARGUMENT;
    }
    if (slot_ids == nullptr || cfgs == nullptr || out_tokens == nullptr) {
        set_error("mc_batch_step: a required array (slot_ids, cfgs, out_tokens) is null");
        return MC_E_INVALID_ARGUMENT;
    }
    if (n == 0 || n > g->max_slots) {
        set_error("mc_batch_step: step size %u not supported (allowed 1..%u)", n, g->max_slots);
        return MC_E_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t sid = slot_ids[i];
        if (sid >= g->max_slots || g->members[sid] == nullptr) {
            set_error("mc_batch_step: entry %u names slot %u, which is empty", i, sid);
            return MC_E_INVALID_ARGUMENT;
        }
        for (uint32_t j = 0; j < i; ++j)
            if (slot_ids[j] == sid) {
                set_error("mc_batch_step: slot %u is listed twice", sid);
                return MC_E_INVALID_ARGUMENT;
            }
        if (cfgs[i].struct_size != sizeof(cfgs[i])) {
            set_error("mc_batch_step: config %u is %u bytes, this library expects %zu", i,
                      cfgs[i].struct_size, sizeof(cfgs[i]));
            return MC_E_INVALID_ARGUMENT;
        }
        if (cfgs[i].temperature > 0.f && cfgs[i].top_k != 1u) {
            set_error("mc_batch_step: config %u asks for sampling; batch steps decode greedily", i);
            return MC_E_UNSUPPORTED;
        }
    }
    MC_OR_RETURN(set_device(g->model->device_id, "mc_batch_step"));
    hipStream_t st = g->stream;
    for (uint32_t i = 0; i < n; ++i) {
        SessionImpl* s = g->members[slot_ids[i]];
        if (s->seq_len == 0) {
            set_error("mc_batch_step: slot %u has nothing to continue: prefill it first",
                      slot_ids[i]);
            return MC_E_INVALID_ARGUMENT;
        }
        if (s->seq_len >= g->max_ctx) {
            set_error("mc_batch_step: slot %u has no room for another token (%u positions used)", slot_ids[i],
                      s->seq_len);
            return MC_E_OUT_OF_MEMORY;
        }
    }
    for (uint32_t i = 0; i < n; ++i)
        MC_OR_RETURN(mc_kv_allocator_ensure_pages_for(g->members[slot_ids[i]]->kv,
                                                      g->members[slot_ids[i]]->seq_len + 1u,
                                                      st));
    const auto t0 = std::chrono::steady_clock::now();
    // Step tables (compacted to the n members of this step).
    void** h = static_cast<void**>(g->h_tables);
    const uint32_t B = kMaxSlots;
    for (uint32_t i = 0; i < n; ++i) {
        SessionImpl* s = g->members[slot_ids[i]];
        h[i] = &s->d_state->seq_len;
        h[B + i] = s->d_pt;
        h[2u * B + i] = s->pool;
        h[3u * B + i] = &s->d_state->next_token;
        h[4u * B + i] = s->d_seq;
    }
    HIP_OR_RETURN(hipMemcpyAsync(g->d_pos, h, 5u * B * sizeof(void*),
                                 hipMemcpyHostToDevice, st),
                  "mc_batch_step: slot pointer table H2D failed");
    const mc_kv_layout_t lay = g->members[slot_ids[0]]->layout;
    TraceRange trace_range("mc_batch_step");
    if (g->model->weights) {
        // each slot returns the token its previous forward predicted; the
        // step predicts the next ones into the members' d_state.next_token
        for (uint32_t i = 0; i < n; ++i)
            HIP_OR_RETURN(hipMemcpyAsync(&g->h_tok[i], &g->members[slot_ids[i]]->d_state->next_token,
                                         4u, hipMemcpyDeviceToHost, st),
                          "mc_batch_step: token D2H failed");
        g->fwd.layout = lay;
        g->bd.used = g->model->use_graphs ? kBdEvents + 1u : 0u;
        const Marker mark{[](void* c) {
                              auto* gg = static_cast<GroupImpl*>(c);
                              gg->bd.mark(gg->stream);
                          },
                          g};
        const BatchKv kv{g->d_pos, g->d_pt, g->d_kv, g->d_tok, n};
        for (auto& r : g->last_row) r = -1;
        for (uint32_t i = 0; i < n; ++i) g->last_row[slot_ids[i]] = (int32_t)i;
        MC_OR_RETURN(run_step(g->model->use_graphs, g->step_graph[n], st, [&]() -> mc_status_t {
            g->bd.mark(st);
            return forward_batch(g->fwd, kv, mark);
        }));
        if (g->model->use_graphs)
            for (uint32_t i = 0; i < n; ++i) g->members[slot_ids[i]]->graph_launches += 1;
    }
    if (!g->model->weights) {
        g->bd.used = g->model->use_graphs ? kBdEvents + 1u : 0u;  // graph steps: nothing recorded
        MC_OR_RETURN(run_step(g->model->use_graphs, g->step_graph[n], st, [&]() -> mc_status_t {
            g->bd.mark(st);
            for (uint32_t l = 0; l < kLayers; ++l) {
                MC_OR_RETURN(launch_synth_qkv_batch(g->qkv, n, g->d_tok, g->d_pos, l, st));
                g->bd.mark(st);
                MC_OR_RETURN(mc_kv_attention_decode_batch(
                    g->qkv, g->d_pos, n, l, g->d_pt, g->d_kv, lay, g->partials, g->max_chunks,
                    g->out, st, g->inv_freq, g->chunk_pos, g->partials2));
                g->bd.mark(st);
            }
            return MC_OK;
        }));
        if (g->model->use_graphs)
            for (uint32_t i = 0; i < n; ++i) g->members[slot_ids[i]]->graph_launches += 1;
        for (uint32_t i = 0; i < n; ++i) {
            SessionImpl* s = g->members[slot_ids[i]];
            if (!s->rng_seeded) {
                s->rng = (uint32_t)cfgs[i].seed;
                s->rng_seeded = true;
            }
            g->h_tok[i] = mock_token(s->seq_len, s->rng);
            HIP_OR_RETURN(hipMemcpyAsync(&s->d_state->next_token, &g->h_tok[i], 4u,
                                         hipMemcpyHostToDevice, st),
                          "mc_batch_step: token H2D failed");
        }
    }
    MC_OR_RETURN(mc_kv_batch_advance(g->d_seq, g->d_tok, g->d_pos, n, st));
    g->bd.mark(st);
    HIP_OR_RETURN(hipStreamSynchronize(st), "mc_batch_step: stream sync failed");
    for (uint32_t i = 0; i < n; ++i)
        if (g->h_tok[i] < 0 || (uint32_t)g->h_tok[i] >= kVocab) {
            set_error("mc_batch_step: slot %u produced token id %d, outside the vocabulary",
                      slot_ids[i], g->h_tok[i]);
            return MC_E_INTERNAL;
        }
    const uint64_t us = (uint64_t)std::chrono::duration_cast<std::chrono::microseconds>(
                            std::chrono::steady_clock::now() - t0)
                            .count();
    g->steps += 1;
    g->decode_us += us;
    for (uint32_t i = 0; i < n; ++i) {
        SessionImpl* s = g->members[slot_ids[i]];
        s->seq_len += 1;
        s->h_state.seq_len = s->seq_len;
        s->h_state.next_token = g->h_tok[i];
        s->rng = xorshift32(s->rng);
        s->total.generated_tokens += 1;
        s->since_reset.generated_tokens += 1;
        s->total.decode_us += us;
        s->since_reset.decode_us += us;
        out_tokens[i] = g->h_tok[i];
    }
    return MC_OK;
    MC_GUARD_END
}

void mc_batch_group_destroy(mc_batch_group_t group) { release_group(group.impl); }

// ---------------- debug hooks (outside the frozen ABI) ----------------

mc_status_t mc_debug_session_info(mc_session_t session, uint32_t* seq_len,
                                  uint32_t* pages_owned, mc_kv_layout_t* layout,
                                  void** d_pool, void** d_page_table) {
    SessionImpl* s = session.impl;
    if (s == nullptr) {
        set_error("mc_debug_session_info: session is NULL");
        return MC_E_INVALID_ARGUMENT;
    }
    if (seq_len) *seq_len = s->seq_len;
    if (pages_owned) *pages_owned = mc_kv_allocator_pages_owned(s->kv);
    if (layout) *layout = s->layout;
    if (d_pool) *d_pool = s->pool;
    if (d_page_table) *d_page_table = s->d_pt;
    return MC_OK;
}

size_t mc_debug_session_arena_bytes(mc_session_t session) {
    return session.impl ? session.impl->arena_bytes : 0u;
}

uint32_t mc_debug_session_attn_chunk(mc_session_t session) {
    return session.impl ? session.impl->chunk_pos : 0u;
}

void mc_debug_session_set_graph_enabled(mc_session_t session, int enabled) {
    if (session.impl == nullptr) return;
    session.impl->graph_off = enabled == 0;
}

size_t mc_debug_session_graph_nodes(mc_session_t session) {
    SessionImpl* s = session.impl;
    if (s == nullptr || s->step_graph.graph == nullptr) return 0u;
    size_t n = 0;
    if (hipGraphGetNodes(s->step_graph.graph, nullptr, &n) != hipSuccess) {
        (void)hipGetLastError();
        return 0u;
    }
    return n;
}

int mc_debug_session_rope_intact(mc_session_t session) {
    SessionImpl* s = session.impl;
    if (s == nullptr || !s->rope_snapshot_valid || s->inv_freq == nullptr) return -1;
    if (hipSetDevice(s->model->device_id) != hipSuccess) {
        (void)hipGetLastError();
        return -2;
    }
    uint32_t cur[64];
    if (hipMemcpy(cur, s->inv_freq, sizeof(cur), hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return -2;
    }
    return std::memcmp(cur, s->rope_snapshot, sizeof(cur)) == 0 ? 1 : 0;
}

mc_status_t mc_debug_seed_residual(mc_session_t session, const void* host_bf16_rows,
                                   uint32_t rows) {
    MC_GUARD_BEGIN
    SessionImpl* s = session.impl;
    if (s == nullptr || host_bf16_rows == nullptr) {
        set_error("mc_debug_seed_residual: session/rows pointer is NULL");
        return MC_E_INVALID_ARGUMENT;
    }
    if (!s->model->weights) {
        set_error("mc_debug_seed_residual: requires a session of a model loaded with weights "
                  "(model.wpk)");
        return MC_E_UNSUPPORTED;
    }
    if (rows == 0u || rows > s->fwd.rows) {
        set_error("mc_debug_seed_residual: rows=%u out of range (1..%u, the prefill chunk rows)",
                  rows, s->fwd.rows);
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_debug_seed_residual"));
    HIP_OR_RETURN(hipMemcpy(s->fwd.res_a, host_bf16_rows, (size_t)rows * kHidden * 2u,
                            hipMemcpyHostToDevice),
                  "mc_debug_seed_residual: H2D copy failed");
    return MC_OK;
    MC_GUARD_END
}

int mc_debug_breakdown_raw_segments(mc_session_t session) {
    return (session.impl && session.impl->bd.enabled) ? (int)kBdRawSegs : 0;
}

int mc_debug_breakdown_bucket_count(void) { return (int)kBdBuckets; }

const char* mc_debug_breakdown_bucket_name(int i) {
    return (i < 0 || (uint32_t)i >= kBdBuckets) ? nullptr : kBdNames[i];
}

int mc_debug_breakdown_bucket_of(int raw) {
    return (raw < 0 || (uint32_t)raw >= kBdRawSegs) ? -1 : (int)bd_bucket((uint32_t)raw);
}

int mc_debug_breakdown_collect(mc_session_t session, double* out_ms, int n) {
    SessionImpl* s = session.impl;
    if (s == nullptr) return -1;
    if (!s->bd.enabled) return 0;
    if (out_ms == nullptr || n != (int)kBdRawSegs) return -1;
    if (s->bd.used != kBdEvents) return -2;
    if (hipSetDevice(s->model->device_id) != hipSuccess) return -3;
    for (uint32_t k = 0; k < kBdRawSegs; ++k)
        if (!s->bd.segment(k, &out_ms[k])) return -3;
    return (int)kBdRawSegs;
}

mc_status_t mc_debug_batch_group_stats(mc_batch_group_t group, uint64_t* steps,
                                       uint64_t* decode_us, uint32_t* members) {
    GroupImpl* g = group.impl;
    if (g == nullptr || steps == nullptr || decode_us == nullptr || members == nullptr) {
        set_error("mc_debug_batch_group_stats: null group or output pointer");
        return MC_E_INVALID_ARGUMENT;
    }
    uint32_t cnt = 0;
    for (uint32_t i = 0; i < g->max_slots; ++i) cnt += g->members[i] != nullptr;
    *steps = g->steps;
    *decode_us = g->decode_us;
    *members = cnt;
    return MC_OK;
}

int mc_debug_batch_breakdown_collect(mc_batch_group_t group, double* out_ms, int n) {
    GroupImpl* g = group.impl;
    if (g == nullptr || out_ms == nullptr || n != (int)kBdBuckets) return -1;
    if (!g->bd.enabled) return 0;
    if (g->bd.used != kBdEvents) return -2;
    if (hipSetDevice(g->model->device_id) != hipSuccess) return -3;
    double b[kBdBuckets] = {};
    for (uint32_t k = 0; k < kBdRawSegs; ++k) {
        double ms = 0.0;
        if (!g->bd.segment(k, &ms)) return -3;
        b[bd_bucket(k)] += ms;
    }
    for (uint32_t i = 0; i < kBdBuckets; ++i) out_ms[i] = b[i];
    return (int)kBdBuckets;
}

namespace {
mc_status_t logits_to_host(const uint16_t* d_row, float* out, const char* who) {
    std::vector<uint16_t> h(kVocabSize);
    const hipError_t e =
        hipMemcpy(h.data(), d_row, (size_t)kVocabSize * 2u, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return check_hip(e, who);
    for (uint32_t i = 0; i < kVocabSize; ++i) out[i] = bf16_to_f32(h[i]);
    return MC_OK;
}
}  // namespace

mc_status_t mc_debug_session_last_logits(mc_session_t session, float* out_f32) {
    SessionImpl* s = session.impl;
    if (s == nullptr || out_f32 == nullptr || !s->model->weights) {
        set_error("mc_debug_session_last_logits: needs a session of a model with weights and "
                  "an output array");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_debug_session_last_logits"));
    HIP_OR_RETURN(hipStreamSynchronize(s->stream), "mc_debug_session_last_logits: sync failed");
    return logits_to_host(s->fwd.logits, out_f32, "mc_debug_session_last_logits: D2H failed");
}

mc_status_t mc_debug_batch_last_logits(mc_batch_group_t group, uint32_t slot, float* out_f32) {
    GroupImpl* g = group.impl;
    if (g == nullptr || out_f32 == nullptr || !g->model->weights || slot >= kMaxSlots ||
        g->last_row[slot] < 0) {
        set_error("mc_debug_batch_last_logits: needs a group of a model with weights, an output "
                  "array and a slot of the last step");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(g->model->device_id, "mc_debug_batch_last_logits"));
    HIP_OR_RETURN(hipStreamSynchronize(g->stream), "mc_debug_batch_last_logits: sync failed");
    return logits_to_host(g->fwd.logits + (size_t)g->last_row[slot] * kVocabSize, out_f32,
                          "mc_debug_batch_last_logits: D2H failed");
}

mc_status_t mc_debug_session_seq(mc_session_t session, int32_t* out, uint32_t n) {
    SessionImpl* s = session.impl;
    if (s == nullptr || out == nullptr || n > s->seq_len) {
        set_error("mc_debug_session_seq: bad arguments");
        return MC_E_INVALID_ARGUMENT;
    }
    MC_OR_RETURN(set_device(s->model->device_id, "mc_debug_session_seq"));
    HIP_OR_RETURN(hipMemcpy(out, s->d_seq, (size_t)n * 4u, hipMemcpyDeviceToHost),
                  "mc_debug_session_seq: D2H failed");
    return MC_OK;
}

}  // extern "C"
