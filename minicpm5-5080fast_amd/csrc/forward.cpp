// forward.cpp - the MiniCPM5 forward over the paged KV cache when real
// weights are loaded (model.wpk).
//
// Layer graph of the reference (native/runtime/forward.cpp:200-420):
//   residual -> RMSNorm(norm1) -> qkv projection -> RoPE (q in place, k/v
//   into the pages) -> paged causal GQA attention -> o projection ->
//   residual add -> RMSNorm(norm2) -> gate_up projection -> SwiGLU -> down
//   projection -> residual add -> RMSNorm(next layer's norm1, or final_norm
//   after the last layer); logits of the last row through lm_head, greedy
//   argmax into the next token. Every rounding point of the reference is kept:
//   the residual is stored in bf16 after each add, norms, projections, SwiGLU
//   and logits are bf16.
//
// MI355X mapping:
//   * prefill (T rows): projections through rocBLAS GEMM (bf16 in/out, fp32
//     compute), RMSNorm / residual-add kernels, SwiGLU, the paged prefill
//     attention; the lm_head of the last row through the GEMV;
//   * decode (one row) and batch steps (n <= 8 rows): every projection is the
//     HBM-streaming GEMV of model_kernels.hip, with the residual add + RMSNorm
//     fused into the GEMV that consumes it (qkv, gate_up, lm_head) and the
//     SwiGLU fused into the gate_up projection's output (each output column
//     streams its gate and up rows together; the reference fuses it into the
//     down projection's input, forward.cpp:348-375, which would repeat the
//     SwiGLU in every workgroup); the residual alternates between two
//     buffers so that the workgroup writing the new residual never races the
//     workgroups still reading the old one. Attention is the phase0 decode
//     (RoPE + K/V append + split-KV attention in one chunk kernel).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "error.h"
#include "kv_common.h"
#include "mc_kv.h"
#include "model_internal.h"
#include "prefill_gemm_table.h"
#include "trace.h"

namespace mckv {
namespace {

constexpr double kTheta = 5.0e6;  // generated_model_config.h:23

// MC_ROPE_TABLE_OFF (read once per process, forward.cpp:248-262): the RoPE
// kernel computes its frequencies itself instead of reading the table, and
// a decode step runs it before the attention instead of the attention's
// phase0 append (the same values bit for bit: the kernel evaluates the
// table's own expression, and phase0 equals rope-then-attend).
bool rope_table_off() {
    static const bool off = std::getenv("MC_ROPE_TABLE_OFF") != nullptr;
    return off;
}

size_t a256(size_t x) { return (x + 255u) & ~size_t(255); }

#define FWD_OR_RETURN(call)             \
    do {                                \
        const mc_status_t _s = (call);  \
        if (_s != MC_OK) return _s;     \
    } while (0)

// The tuned table of the rocBLAS this process resolved (by its version
// string), or null.
bool gemm_defaults_only() {
    static const bool on = std::getenv("MC_PREFILL_GEMM_DEFAULT") != nullptr;
    return on;
}

const PrefillGemmTable* gemm_table() {
    static const PrefillGemmTable* t = []() -> const PrefillGemmTable* {
        if (gemm_defaults_only()) return nullptr;
        char ver[256] = {0};
        if (rocblas_get_version_string(ver, sizeof(ver)) != rocblas_status_success)
            return nullptr;
        for (const PrefillGemmTable& e : kPrefillGemmTables)
            if (std::strcmp(e.rocblas_version, ver) == 0) return &e;
        return nullptr;
    }();
    return t;
}

static_assert(sizeof(kPrefillGemmRocm) / sizeof(kPrefillGemmRocm[0]) <= 64u &&
                  sizeof(kPrefillGemmTorch) / sizeof(kPrefillGemmTorch[0]) <= 64u,
              "a table row is one bit of gemm_bf16's rejection mask");

// Row of the tuned table for an M x N x K projection: the largest tuned M not
// above M; -1 below the smallest, for other shapes or without a table.
int gemm_row(const PrefillGemmTable* t, uint32_t M, uint32_t N, uint32_t K) {
    int row = -1;
    if (t == nullptr) return row;
    for (uint32_t i = 0; i < t->count; ++i) {
        const PrefillGemmSolution& e = t->rows[i];
        if (e.n == N && e.k == K && e.m <= M) row = (int)i;
    }
    return row;
}

// The prefill projections' GEMM libraries of one session.
struct PrefillBlas {
    rocblas_handle rb = nullptr;
    hipblasLtHandle_t lt = nullptr;
    hipblasLtMatmulDesc_t desc = nullptr;  // y^T = W^T(op T) . x^T, fp32 compute
    void* ws = nullptr;
    size_t ws_bytes = 0;
};

// hipBLASLt rows: chunks of kLtMinRows..kLtMaxRows rows without a tuned
// rocBLAS solution go through hipBLASLt with the heuristic's first algorithm,
// looked up once per (M, N, K) per process. Through PyTorch's libraries a
// rocblas_gemm_ex call takes ~16 us of host time whatever the size, a
// hipblasLtMatmul call ~9 us, with kernels of the same speed; measured, the
// prefill of 17..256 tokens is 3-11% faster this way. Larger chunks stay on
// rocBLAS (its tuned table; the host time is hidden behind the kernels).
constexpr uint32_t kLtMinRows = 17u, kLtMaxRows = 1023u;

struct LtAlgoCache {
    std::mutex mu;
    std::unordered_map<uint64_t, hipblasLtMatmulAlgo_t> algos;
    std::unordered_map<uint64_t, bool> failed;
};
LtAlgoCache& lt_cache() {
    static LtAlgoCache c;
    return c;
}

// y[M][N] = x[M][K] . W[N][K]^T through hipBLASLt; false (nothing launched)
// when hipBLASLt has no algorithm for the shape or rejects the call.
bool gemm_lt(const PrefillBlas& b, hipStream_t st, const uint16_t* x, uint32_t M,
             const uint16_t* W, uint32_t N, uint32_t K, uint16_t* y) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    const uint64_t key = ((uint64_t)(uint32_t)dev << 56) ^ ((uint64_t)M << 32) ^
                         ((uint64_t)N << 16) ^ (uint64_t)K;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    bool ok = hipblasLtMatrixLayoutCreate(&la, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&lb, HIP_R_16BF, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&lc, HIP_R_16BF, N, M, N) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulAlgo_t algo{};
    if (ok) {
        LtAlgoCache& c = lt_cache();
        std::lock_guard<std::mutex> lk(c.mu);
        auto it = c.algos.find(key);
        if (it != c.algos.end()) {
            algo = it->second;
        } else if (c.failed.count(key)) {
            ok = false;
        } else {
            hipblasLtMatmulPreference_t pref = nullptr;
            hipblasLtMatmulHeuristicResult_t res{};
            int n = 0;
            uint64_t wsz = b.ws_bytes;
            ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatmulPreferenceSetAttribute(
                     pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz, sizeof(wsz)) ==
                     HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatmulAlgoGetHeuristic(b.lt, b.desc, la, lb, lc, lc, pref, 1, &res,
                                                 &n) == HIPBLAS_STATUS_SUCCESS &&
                 n > 0 && res.state == HIPBLAS_STATUS_SUCCESS && res.workspaceSize <= b.ws_bytes;
            if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
            if (ok) {
                algo = res.algo;
                c.algos.emplace(key, algo);
            } else {
                c.failed.emplace(key, true);
            }
        }
    }
    if (ok) {
        const float alpha = 1.f, beta = 0.f;
        ok = hipblasLtMatmul(b.lt, b.desc, &alpha, W, la, x, lb, &beta, y, lc, y, lc, &algo, b.ws,
                             b.ws_bytes, st) == HIPBLAS_STATUS_SUCCESS;
    }
    if (la) (void)hipblasLtMatrixLayoutDestroy(la);
    if (lb) (void)hipblasLtMatrixLayoutDestroy(lb);
    if (lc) (void)hipblasLtMatrixLayoutDestroy(lc);
    return ok;
}

// y[M][N] = x[M][K] . W[N][K]^T (column-major view: C(N x M) = W^T(N x K) .
// x^T(K x M)). A shape with a tuned rocBLAS solution runs it; an index that
// rocBLAS rejects (it checks one against the problem before launching) reruns
// the call on the default heuristic and leaves that table row on it for the
// rest of the process. Other shapes of kLtMinRows..kLtMaxRows rows go through
// hipBLASLt, the rest (and whatever hipBLASLt declines) through rocBLAS's
// default heuristic. MC_PREFILL_GEMM_DEFAULT=1 sends every projection to
// rocBLAS's default heuristic (the measured A/B of the tables and the
// hipBLASLt rows).
mc_status_t gemm_bf16(const Forward& f, const uint16_t* x, uint32_t M, const uint16_t* W,
                      uint32_t N, uint32_t K, uint16_t* y) {
    const PrefillBlas& b = *static_cast<const PrefillBlas*>(f.blas);
    const PrefillGemmTable* t = gemm_table();
    const int row = gemm_row(t, M, N, K);
    // rows whose index this process's rocBLAS rejected
    static std::atomic<uint64_t> rejected{0};
    const uint64_t bit = row >= 0 ? uint64_t(1) << row : 0u;
    const int32_t idx = row >= 0 && !(rejected.load(std::memory_order_relaxed) & bit)
                            ? t->rows[row].index
                            : 0;
    if (idx == 0 && M >= kLtMinRows && M <= kLtMaxRows && !gemm_defaults_only() &&
        gemm_lt(b, f.st, x, M, W, N, K, y))
        return MC_OK;
    rocblas_handle h = b.rb;
    if (rocblas_set_stream(h, f.st) != rocblas_status_success) {
        set_error("prefill GEMM: rocblas_set_stream failed");
        return MC_E_CUDA;
    }
    const float alpha = 1.f, beta = 0.f;
    auto run = [&](int32_t i) {
        return rocblas_gemm_ex(
            h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)N,
            (rocblas_int)M, (rocblas_int)K, &alpha, W, rocblas_datatype_bf16_r, (rocblas_int)K, x,
            rocblas_datatype_bf16_r, (rocblas_int)K, &beta, y, rocblas_datatype_bf16_r,
            (rocblas_int)N, y, rocblas_datatype_bf16_r, (rocblas_int)N, rocblas_datatype_f32_r,
            i ? rocblas_gemm_algo_solution_index : rocblas_gemm_algo_standard, i, 0);
    };
    rocblas_status s = run(idx);
    if (s != rocblas_status_success && idx != 0) {
        rejected.fetch_or(bit, std::memory_order_relaxed);
        s = run(0);
    }
    if (s != rocblas_status_success) {
        set_error("prefill GEMM (%u x %u x %u): rocblas_gemm_ex failed: %s", M, N, K,
                  rocblas_status_to_string(s));
        return MC_E_CUDA;
    }
    return MC_OK;
}

// Device workspace handed to the prefill projections' rocBLAS handle. With a
// caller-owned workspace rocBLAS only selects GEMM solutions whose scratch
// fits in it and never allocates on its own.
constexpr size_t kBlasWorkspace = size_t(32) << 20;

// ---- debug dump ----
struct DumpConfig {
    bool on = false;
    int steps = 0;
    std::string dir;
};
DumpConfig& dump_config() {
    static DumpConfig c = [] {
        DumpConfig d;
        const char* dir = std::getenv("MC_DEBUG_DUMP_DIR");
        if (dir != nullptr && dir[0] != '\0') {
            const char* n = std::getenv("MC_DEBUG_DUMP_STEPS");
            d.on = true;
            d.dir = dir;
            d.steps = n != nullptr ? std::atoi(n) : 0;
            std::fprintf(stderr, "[minicpm-native] debug dump enabled: dir=%s steps=%d\n", dir,
                         d.steps);
        }
        return d;
    }();
    return c;
}

// Writes n bf16 values of device memory as fp32 to <dir>/<name> (synchronous).
mc_status_t dump_bf16(const std::string& name, const uint16_t* d, size_t n, hipStream_t st) {
    std::vector<uint16_t> h(n);
    hipError_t e = hipMemcpyAsync(h.data(), d, n * 2u, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error("debug dump %s: copy failed: %s", name.c_str(), hipGetErrorString(e));
        return MC_E_CUDA;
    }
    std::vector<float> f(n);
    for (size_t i = 0; i < n; ++i) f[i] = bf16_to_f32(h[i]);
    const std::string path = dump_config().dir + "/" + name;
    FILE* fp = std::fopen(path.c_str(), "wb");
    if (fp == nullptr) {
        set_error("debug dump: cannot open %s", path.c_str());
        return MC_E_IO;
    }
    const size_t w = std::fwrite(f.data(), sizeof(float), n, fp);
    std::fclose(fp);
    if (w != n) {
        set_error("debug dump: short write to %s", path.c_str());
        return MC_E_IO;
    }
    return MC_OK;
}

mc_status_t dump_token(const std::string& name, const int32_t* d_tok, hipStream_t st) {
    int32_t t = -1;
    hipError_t e = hipMemcpyAsync(&t, d_tok, 4u, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error("debug dump %s: copy failed: %s", name.c_str(), hipGetErrorString(e));
        return MC_E_CUDA;
    }
    const std::string path = dump_config().dir + "/" + name;
    FILE* fp = std::fopen(path.c_str(), "wb");
    if (fp == nullptr) {
        set_error("debug dump: cannot open %s", path.c_str());
        return MC_E_IO;
    }
    const size_t w = std::fwrite(&t, sizeof(t), 1, fp);
    std::fclose(fp);
    if (w != 1u) {
        set_error("debug dump: short write to %s", path.c_str());
        return MC_E_IO;
    }
    return MC_OK;
}

std::string dump_name(const char* kind, uint32_t i, const char* what) {
    char b[64];
    std::snprintf(b, sizeof(b), "%s%u.%s", kind, i, what);
    return b;
}

// The residual r = bf16(cur + add) of one row into `tmp` (cur unchanged);
// `normed` receives a normalized copy that is not used.
mc_status_t residual_row(const uint16_t* cur, const uint16_t* add, uint16_t* tmp,
                         const uint16_t* norm_w, uint16_t* normed, hipStream_t st) {
    if (hipMemcpyAsync(tmp, cur, (size_t)kHidden * 2u, hipMemcpyDeviceToDevice, st) !=
        hipSuccess) {
        (void)hipGetLastError();
        set_error("debug dump: residual copy failed");
        return MC_E_CUDA;
    }
    if (add == nullptr) return MC_OK;
    return mc_model_rmsnorm_rows(tmp, add, norm_w, normed, 1, kHidden, kRmsEps, st);
}

}  // namespace

bool dump_due(uint32_t step) {
    const DumpConfig& c = dump_config();
    return c.on && (int64_t)step < (int64_t)c.steps;
}

mc_status_t prefill_blas_create(void** out, size_t* ws_bytes) {
    *out = nullptr;
    *ws_bytes = kBlasWorkspace;
    PrefillBlas* b = new (std::nothrow) PrefillBlas;
    if (b == nullptr) {
        set_error("mc_session_create: out of host memory");
        return MC_E_OUT_OF_MEMORY;
    }
    if (rocblas_create_handle(&b->rb) != rocblas_status_success) {
        b->rb = nullptr;
        prefill_blas_destroy(b);
        set_error("mc_session_create: rocblas_create_handle failed");
        return MC_E_CUDA;
    }
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (hipblasLtCreate(&b->lt) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescCreate(&b->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(b->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(b->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) !=
            HIPBLAS_STATUS_SUCCESS) {
        prefill_blas_destroy(b);
        set_error("mc_session_create: hipBLASLt handle or matmul descriptor creation failed");
        return MC_E_CUDA;
    }
    *out = b;
    return MC_OK;
}

mc_status_t prefill_blas_workspace(void* hv, void* ws, size_t ws_bytes) {
    PrefillBlas* b = static_cast<PrefillBlas*>(hv);
    const rocblas_status st = rocblas_set_workspace(b->rb, ws, ws_bytes);
    if (st != rocblas_status_success) {
        set_error("mc_session_create: rocblas_set_workspace failed: %s",
                  rocblas_status_to_string(st));
        return MC_E_CUDA;
    }
    b->ws = ws;  // hipBLASLt takes it per call
    b->ws_bytes = ws_bytes;
    return MC_OK;
}

void prefill_blas_destroy(void* hv) {
    PrefillBlas* b = static_cast<PrefillBlas*>(hv);
    if (b == nullptr) return;
    if (b->desc) (void)hipblasLtMatmulDescDestroy(b->desc);
    if (b->lt) (void)hipblasLtDestroy(b->lt);
    if (b->rb) (void)rocblas_destroy_handle(b->rb);
    delete b;
}

size_t forward_act_bytes(uint32_t rows, uint32_t logit_rows) {
    const size_t r = rows;
    return a256(r * kHidden * 2u) * 2u      // res_a, res_b
           + a256(r * kHidden * 2u)         // normed
           + a256(r * kQkvCols * 2u)        // qkv
           + a256(r * kHidden * 2u) * 2u    // attn, o_out
           + a256(r * 2u * kInter * 2u)     // gate_up
           + a256(r * kInter * 2u)          // mlp
           + a256(r * kHidden * 2u)         // down
           + a256((size_t)logit_rows * kVocabSize * 2u)
           + a256((size_t)logit_rows * MC_MODEL_ARGMAX_SLICES * 4u) * 2u;  // argmax stages
}

void forward_carve(Forward& f, char* p, uint32_t rows, uint32_t logit_rows) {
    const size_t r = rows;
    auto take = [&](size_t bytes) {
        uint16_t* q = reinterpret_cast<uint16_t*>(p);
        p += a256(bytes);
        return q;
    };
    f.res_a = take(r * kHidden * 2u);
    f.res_b = take(r * kHidden * 2u);
    f.normed = take(r * kHidden * 2u);
    f.qkv = take(r * kQkvCols * 2u);
    f.attn = take(r * kHidden * 2u);
    f.o_out = take(r * kHidden * 2u);
    f.gate_up = take(r * 2u * kInter * 2u);
    f.mlp = take(r * kInter * 2u);
    f.down = take(r * kHidden * 2u);
    f.logits = take((size_t)logit_rows * kVocabSize * 2u);
    f.stage_v = reinterpret_cast<float*>(take((size_t)logit_rows * MC_MODEL_ARGMAX_SLICES * 4u));
    f.stage_i = reinterpret_cast<int32_t*>(take((size_t)logit_rows * MC_MODEL_ARGMAX_SLICES * 4u));
    f.rows = rows;
}

// Key splits of a prefill chunk's attention: the reference's count for n
// rows (kernels.h:517-521: 4096 / n, 1..8), capped so that each split gets
// at least kSplitKeysMin keys of the chunk's last row. A split of a few
// 64-key steps gains nothing and costs the merge kernel (a 32-token prompt:
// 8 splits of 4 keys, attention 8.7 us + merge 5.0 us per layer). Splits
// change the result's rounding only.
constexpr uint32_t kSplitKeysMin = 512u;
uint32_t prefill_splits(uint32_t n, uint32_t keys) {
    const uint32_t s = mc_kv_prefill_split_kv(n);
    if (keys == 0u) return s;
    const uint32_t cap = keys / kSplitKeysMin;
    return s < cap ? s : (cap < 1u ? 1u : cap);
}

// Projections of short prefill chunks (whole model, 42 layers, best of 5;
// library GEMMs in parentheses): 2..8 tokens through forward_prefill_rows
// 1.74-2.16 ms (3.60-3.67), 9..32 tokens through the row GEMM 2.45-3.31 ms
// (3.30-3.74); at 33-64 tokens the row GEMM measured slower than hipBLASLt
// (its activation reads grow with the rows on each of the N / 16
// workgroups). MC_PREFILL_ROWS_GEMV_OFF=1 sends chunks of 2..32 tokens
// through the GEMM libraries as well (the measured A/B).
bool prefill_rows_gemv_off() {
    static const bool off = std::getenv("MC_PREFILL_ROWS_GEMV_OFF") != nullptr;
    return off;
}

// A prefill chunk of 2..MC_MODEL_GEMV_MAX_ROWS tokens: the projections as
// M-row GEMVs (each weight byte read once for all rows, the residual add +
// RMSNorm as their prologue, the SwiGLU as the gate_up epilogue; the batch
// step's kernels), the RoPE append and the prefill attention of the GEMM
// path, the lm_head on the last row. The same forward as the GEMM path up to
// the projections' fp32 summation order (reference: forward.cpp:200-420
// runs every T > 1 chunk through its GEMMs). The residual is kept as
// cur + pending as in forward_decode.
mc_status_t forward_prefill_rows(const Forward& f, const int32_t* d_ids, uint32_t n,
                                 int32_t* d_next) {
    TraceRange trace_range("forward_prefill_rows");
    const ModelWeights& w = *f.w;
    hipStream_t st = f.st;
    const size_t last = (size_t)(n - 1u) * kHidden;  // the last row's offset
    uint16_t* cur = f.res_a;
    uint16_t* other = f.res_b;
    const uint16_t* pending = nullptr;
    const bool step_dump = dump_due(f.dump_step);
    const bool layer_dump = step_dump && f.dump_layers;
    const uint32_t S = prefill_splits(n, f.keys);
    FWD_OR_RETURN(mc_model_embedding_gather(w.embedding, d_ids, nullptr, cur, kHidden, n, st));
    for (uint32_t l = 0; l < kModelLayers; ++l) {
        if (layer_dump) {
            FWD_OR_RETURN(residual_row(cur + last, pending ? pending + last : nullptr, f.attn,
                                       w.norm1[l], f.normed, st));
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "hidden_in.f32"), f.attn, kHidden, st));
        }
        uint16_t* res_out = pending != nullptr ? other : nullptr;
        FWD_OR_RETURN(mc_model_gemv_resnorm(w.qkv[l], cur, pending, w.norm1[l], res_out, kHidden,
                                            f.qkv, kQkvCols, n, kQkvCols, kRmsEps, st));
        if (pending != nullptr) std::swap(cur, other);
        FWD_OR_RETURN(mc_kv_rope_append(f.qkv, n, f.d_seq_len, l, f.d_pt, f.pool, f.layout, kTheta,
                                        rope_table_off() ? nullptr : f.inv_freq, st));
        FWD_OR_RETURN(mc_kv_attention_prefill(f.qkv, n, f.d_seq_len, l, f.d_pt, f.pool, f.layout,
                                              f.attn, S > 1u ? f.pf_partials : nullptr, S, st));
        FWD_OR_RETURN(mc_model_gemv(w.o[l], f.attn, kHidden, f.o_out, kHidden, n, kHidden,
                                    kHidden, st));
        FWD_OR_RETURN(mc_model_gemv_resnorm_swiglu(w.gate_up[l], cur, f.o_out, w.norm2[l], other,
                                                   kHidden, f.mlp, kInter, n, kInter, kRmsEps,
                                                   st));
        std::swap(cur, other);
        FWD_OR_RETURN(mc_model_gemv(w.down[l], f.mlp, kInter, f.down, kHidden, n, kHidden, kInter,
                                    st));
        pending = f.down;
        if (layer_dump) {  // cur: the residual after the o projection
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "attn_out.f32"), cur + last, kHidden,
                                    st));
            FWD_OR_RETURN(residual_row(cur + last, pending + last, f.attn, w.norm1[0], f.normed,
                                       st));
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "mlp_out.f32"), f.attn, kHidden, st));
        }
    }
    if (step_dump) {  // final_hidden = final_norm(cur + pending), last row
        FWD_OR_RETURN(residual_row(cur + last, pending + last, f.attn, w.final_norm, f.normed,
                                   st));
        FWD_OR_RETURN(mc_model_rmsnorm_rows(f.attn, nullptr, w.final_norm, f.normed, 1, kHidden,
                                            kRmsEps, st));
        FWD_OR_RETURN(dump_bf16(dump_name("step", f.dump_step, "final_hidden.f32"), f.normed,
                                kHidden, st));
    }
    FWD_OR_RETURN(mc_model_gemv_resnorm(w.lm_head, cur + last, pending + last, w.final_norm,
                                        nullptr, kHidden, f.logits, kVocabSize, 1, kVocabSize,
                                        kRmsEps, st));
    FWD_OR_RETURN(mc_model_argmax_bf16(f.logits, kVocabSize, 1, d_next, nullptr, f.stage_v,
                                       f.stage_i, st));
    if (step_dump) {
        FWD_OR_RETURN(dump_bf16(dump_name("step", f.dump_step, "logits.f32"), f.logits,
                                kVocabSize, st));
        FWD_OR_RETURN(dump_token(dump_name("step", f.dump_step, "token"), d_next, st));
    }
    return MC_OK;
}

mc_status_t forward_prefill(const Forward& f, const int32_t* d_ids, uint32_t n, int32_t* d_next) {
    TraceRange trace_range("forward_prefill");
    const ModelWeights& w = *f.w;
    hipStream_t st = f.st;
    if (n == 0u || n > f.rows) {
        set_error("forward_prefill: %u rows for buffers of %u", n, f.rows);
        return MC_E_INTERNAL;
    }
    // A one-token chunk is a T = 1 forward, which the reference runs through
    // its decode path (GEMV projections, FP8 ones in FP8 mode, the phase-0
    // decode attention and the FP8 lm_head: forward.cpp:117-130,252-282,
    // 444-456), not through the GEMMs and prefill attention.
    if (n == 1u) return forward_decode(f, d_ids, d_next, Marker{});
    if (n <= MC_MODEL_GEMV_MAX_ROWS && !prefill_rows_gemv_off())
        return forward_prefill_rows(f, d_ids, n, d_next);
    uint16_t* res = f.res_a;
    const bool step_dump = dump_due(f.dump_step);
    const bool layer_dump = step_dump && f.dump_layers;
    const uint16_t* res_last = res + (size_t)(n - 1u) * kHidden;
    FWD_OR_RETURN(mc_model_embedding_gather(w.embedding, d_ids, nullptr, res, kHidden, n, st));
    FWD_OR_RETURN(mc_model_rmsnorm_rows(res, nullptr, w.norm1[0], f.normed, n, kHidden, kRmsEps, st));
    const uint32_t S = prefill_splits(n, f.keys);
    // 9..32 rows: the projections through the row GEMM (the gate_up one with
    // the SwiGLU as its epilogue), larger chunks through the GEMM libraries
    const bool rows = n >= MC_MODEL_GEMM_ROWS_MIN && n <= MC_MODEL_GEMM_ROWS_MAX &&
                      !prefill_rows_gemv_off();
    auto proj = [&](const uint16_t* x, const uint16_t* W, uint32_t N, uint32_t K, uint16_t* y) {
        return rows ? mc_model_gemm_rows(W, x, K, y, N, n, N, K, 0u, st)
                    : gemm_bf16(f, x, n, W, N, K, y);
    };
    for (uint32_t l = 0; l < kModelLayers; ++l) {
        if (layer_dump)
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "hidden_in.f32"), res_last, kHidden, st));
        FWD_OR_RETURN(proj(f.normed, w.qkv[l], kQkvCols, kHidden, f.qkv));
        FWD_OR_RETURN(mc_kv_rope_append(f.qkv, n, f.d_seq_len, l, f.d_pt, f.pool, f.layout, kTheta,
                                        rope_table_off() ? nullptr : f.inv_freq, st));
        FWD_OR_RETURN(mc_kv_attention_prefill(f.qkv, n, f.d_seq_len, l, f.d_pt, f.pool, f.layout,
                                              f.attn, S > 1u ? f.pf_partials : nullptr, S, st));
        FWD_OR_RETURN(proj(f.attn, w.o[l], kHidden, kHidden, f.o_out));
        FWD_OR_RETURN(
            mc_model_rmsnorm_rows(res, f.o_out, w.norm2[l], f.normed, n, kHidden, kRmsEps, st));
        if (layer_dump)
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "attn_out.f32"), res_last, kHidden, st));
        if (rows) {
            FWD_OR_RETURN(mc_model_gemm_rows(w.gate_up[l], f.normed, kHidden, f.mlp, kInter, n,
                                             kInter, kHidden, 1u, st));
        } else {
            FWD_OR_RETURN(gemm_bf16(f, f.normed, n, w.gate_up[l], 2u * kInter, kHidden, f.gate_up));
            FWD_OR_RETURN(mc_model_swiglu_rows(f.gate_up, f.mlp, n, kInter, st));
        }
        FWD_OR_RETURN(proj(f.mlp, w.down[l], kHidden, kInter, f.down));
        const uint16_t* next_norm = l + 1u < kModelLayers ? w.norm1[l + 1u] : w.final_norm;
        FWD_OR_RETURN(
            mc_model_rmsnorm_rows(res, f.down, next_norm, f.normed, n, kHidden, kRmsEps, st));
        if (layer_dump)
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "mlp_out.f32"), res_last, kHidden, st));
    }
    FWD_OR_RETURN(mc_model_gemv(w.lm_head, f.normed + (size_t)(n - 1u) * kHidden, kHidden,
                                f.logits, kVocabSize, 1, kVocabSize, kHidden, st));
    FWD_OR_RETURN(mc_model_argmax_bf16(f.logits, kVocabSize, 1, d_next, nullptr, f.stage_v,
                                       f.stage_i, st));
    if (step_dump) {
        FWD_OR_RETURN(dump_bf16(dump_name("step", f.dump_step, "final_hidden.f32"),
                                f.normed + (size_t)(n - 1u) * kHidden, kHidden, st));
        FWD_OR_RETURN(dump_bf16(dump_name("step", f.dump_step, "logits.f32"), f.logits,
                                kVocabSize, st));
        FWD_OR_RETURN(dump_token(dump_name("step", f.dump_step, "token"), d_next, st));
    }
    return MC_OK;
}

mc_status_t forward_decode(const Forward& f, const int32_t* d_tok, int32_t* d_next,
                           const Marker& mark) {
    TraceRange trace_range("forward_decode");
    const ModelWeights& w = *f.w;
    hipStream_t st = f.st;
    // cur: the residual as of the current point; pending: the projection
    // still to be added to it (none at layer 0).
    uint16_t* cur = f.res_a;
    uint16_t* other = f.res_b;
    const uint16_t* pending = nullptr;
    // FP8 mode (the FP8 package loaded): the four projections and, when the
    // package has one, the lm_head on e4m3 weights (forward.cpp:117-130,
    // 444-456)
    const bool q8 = w.fp8_arena != nullptr;
    // debug dump (eager steps only): residual rows are formed in f.attn (free
    // between a layer's o projection and the next attention) and normalized
    // into f.normed (unused by this path)
    const bool step_dump = dump_due(f.dump_step);
    const bool layer_dump = step_dump && f.dump_layers;
    FWD_OR_RETURN(mc_model_embedding_gather(w.embedding, d_tok, nullptr, cur, kHidden, 1, st));
    for (uint32_t l = 0; l < kModelLayers; ++l) {
        if (layer_dump) {
            FWD_OR_RETURN(residual_row(cur, pending, f.attn, w.norm1[l], f.normed, st));
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "hidden_in.f32"), f.attn, kHidden, st));
        }
        // qkv = W_qkv . norm1(cur + pending); the sum becomes the residual
        uint16_t* res_out = pending != nullptr ? other : nullptr;
        if (q8)
            FWD_OR_RETURN(mc_model_gemv_fp8_resnorm(w.q_qkv[l], w.s_qkv[l], cur, pending,
                                                    w.norm1[l], res_out, f.qkv, kQkvCols,
                                                    kRmsEps, st));
        else
            FWD_OR_RETURN(mc_model_gemv_resnorm(w.qkv[l], cur, pending, w.norm1[l], res_out,
                                                kHidden, f.qkv, kQkvCols, 1, kQkvCols, kRmsEps,
                                                st));
        if (pending != nullptr) std::swap(cur, other);
        mark();
        if (rope_table_off())
            FWD_OR_RETURN(mc_kv_rope_append(f.qkv, 1, f.d_seq_len, l, f.d_pt, f.pool, f.layout,
                                            kTheta, nullptr, st));
        FWD_OR_RETURN(mc_kv_attention_decode(f.qkv, f.d_seq_len, l, f.d_pt, f.pool, f.layout,
                                             f.partials, f.max_chunks, f.attn, st,
                                             rope_table_off() ? nullptr : f.inv_freq,
                                             f.chunk_pos, f.partials2));
        if (q8) {
            FWD_OR_RETURN(mc_model_gemv_fp8(w.q_o[l], w.s_o[l], f.attn, f.o_out, kHidden, kHidden,
                                            st));
            FWD_OR_RETURN(mc_model_gemv_fp8_resnorm_swiglu(w.q_gate_up[l], w.s_gate_up[l], cur,
                                                           f.o_out, w.norm2[l], other, f.mlp,
                                                           kInter, kRmsEps, st));
            std::swap(cur, other);
            FWD_OR_RETURN(mc_model_gemv_fp8(w.q_down[l], w.s_down[l], f.mlp, f.down, kHidden,
                                            kInter, st));
        } else {
            FWD_OR_RETURN(mc_model_gemv(w.o[l], f.attn, kHidden, f.o_out, kHidden, 1, kHidden,
                                        kHidden, st));
            FWD_OR_RETURN(mc_model_gemv_resnorm_swiglu(w.gate_up[l], cur, f.o_out, w.norm2[l],
                                                       other, kHidden, f.mlp, kInter, 1, kInter,
                                                       kRmsEps, st));
            std::swap(cur, other);
            FWD_OR_RETURN(mc_model_gemv(w.down[l], f.mlp, kInter, f.down, kHidden, 1, kHidden,
                                        kInter, st));
        }
        pending = f.down;
        if (layer_dump) {  // cur: the residual after the o projection
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "attn_out.f32"), cur, kHidden, st));
            FWD_OR_RETURN(residual_row(cur, pending, f.attn, w.norm1[0], f.normed, st));
            FWD_OR_RETURN(dump_bf16(dump_name("layer", l, "mlp_out.f32"), f.attn, kHidden, st));
        }
        mark();
    }
    if (step_dump) {  // final_hidden = final_norm(cur + pending)
        FWD_OR_RETURN(residual_row(cur, pending, f.attn, w.final_norm, f.normed, st));
        FWD_OR_RETURN(mc_model_rmsnorm_rows(f.attn, nullptr, w.final_norm, f.normed, 1, kHidden,
                                            kRmsEps, st));
        FWD_OR_RETURN(dump_bf16(dump_name("step", f.dump_step, "final_hidden.f32"), f.normed,
                                kHidden, st));
    }
    if (q8 && w.q_lm_head != nullptr)
        FWD_OR_RETURN(mc_model_gemv_fp8_resnorm(w.q_lm_head, w.s_lm_head, cur, pending,
                                                w.final_norm, nullptr, f.logits, kVocabSize,
                                                kRmsEps, st));
    else
        FWD_OR_RETURN(mc_model_gemv_resnorm(w.lm_head, cur, pending, w.final_norm, nullptr,
                                            kHidden, f.logits, kVocabSize, 1, kVocabSize,
                                            kRmsEps, st));
    FWD_OR_RETURN(mc_model_argmax_bf16(f.logits, kVocabSize, 1, d_next, nullptr, f.stage_v,
                                       f.stage_i, st));
    if (step_dump) {
        FWD_OR_RETURN(dump_bf16(dump_name("step", f.dump_step, "logits.f32"), f.logits,
                                kVocabSize, st));
        FWD_OR_RETURN(dump_token(dump_name("step", f.dump_step, "token"), d_next, st));
    }
    return MC_OK;
}

mc_status_t forward_batch(const Forward& f, const BatchKv& b, const Marker& mark) {
    TraceRange trace_range("forward_batch");
    const ModelWeights& w = *f.w;
    hipStream_t st = f.st;
    const uint32_t n = b.n;
    if (n == 0u || n > f.rows || n > MC_MODEL_GEMV_MAX_ROWS) {
        set_error("forward_batch: %u rows for buffers of %u", n, f.rows);
        return MC_E_INTERNAL;
    }
    uint16_t* cur = f.res_a;
    uint16_t* other = f.res_b;
    const uint16_t* pending = nullptr;
    FWD_OR_RETURN(mc_model_embedding_gather(w.embedding, nullptr, b.d_slot_tok, cur, kHidden, n, st));
    for (uint32_t l = 0; l < kModelLayers; ++l) {
        FWD_OR_RETURN(mc_model_gemv_resnorm(w.qkv[l], cur, pending, w.norm1[l],
                                            pending != nullptr ? other : nullptr, kHidden, f.qkv,
                                            kQkvCols, n, kQkvCols, kRmsEps, st));
        if (pending != nullptr) std::swap(cur, other);
        mark();
        FWD_OR_RETURN(mc_kv_attention_decode_batch(f.qkv, b.d_slot_pos, n, l, b.d_slot_pt,
                                                   b.d_slot_kv, f.layout, f.partials, f.max_chunks,
                                                   f.attn, st, f.inv_freq, f.chunk_pos,
                                                   f.partials2));
        FWD_OR_RETURN(mc_model_gemv(w.o[l], f.attn, kHidden, f.o_out, kHidden, n, kHidden, kHidden,
                                    st));
        FWD_OR_RETURN(mc_model_gemv_resnorm_swiglu(w.gate_up[l], cur, f.o_out, w.norm2[l], other,
                                                   kHidden, f.mlp, kInter, n, kInter, kRmsEps,
                                                   st));
        std::swap(cur, other);
        FWD_OR_RETURN(mc_model_gemv(w.down[l], f.mlp, kInter, f.down, kHidden, n, kHidden, kInter,
                                    st));
        pending = f.down;
        mark();
    }
    FWD_OR_RETURN(mc_model_gemv_resnorm(w.lm_head, cur, pending, w.final_norm, nullptr, kHidden,
                                        f.logits, kVocabSize, n, kVocabSize, kRmsEps, st));
    return mc_model_argmax_bf16(f.logits, kVocabSize, n, nullptr, b.d_slot_tok, f.stage_v,
                                f.stage_i, st);
}

}  // namespace mckv

extern "C" void mc_debug_dump_set_steps(int steps) {
    mckv::DumpConfig& c = mckv::dump_config();
    if (c.on) c.steps = steps;
}
