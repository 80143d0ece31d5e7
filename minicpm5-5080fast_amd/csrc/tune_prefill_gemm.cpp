// tune_prefill_gemm.cpp - measures every rocBLAS solution of the prefill
// projections (y[M][N] = x[M][K] . W[N][K]^T, bf16 in/out, fp32 compute, the
// call forward.cpp's gemm_bf16 makes) at a set of row counts M and prints the
// fastest solution index per (M, N, K) as the table prefill_gemm_table.h
// holds. Run on the target GPU with the ROCm image the library ships with
// (solution indices belong to that rocBLAS build):
//   make -C minicpm5-5080fast_amd/csrc tune && ../tune_prefill_gemm > table.h
// Search: every solution timed once (after one warm-up call, which also loads
// its code object), then the 8 fastest re-timed over 20 calls; the default
// solution (index 0) is timed the same way and kept when nothing beats it by
// 3%.
#define ROCBLAS_BETA_FEATURES_API
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <utility>
#include <vector>

namespace {
void check_hip(hipError_t e, int line) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e), line);
        std::exit(1);
    }
}
#define CK(x) check_hip((x), __LINE__)
}  // namespace

extern "C" __attribute__((visibility("default"))) int tune_prefill_gemm_run() {
    rocblas_handle h;
    if (rocblas_create_handle(&h) != rocblas_status_success) return 1;
    hipStream_t st;
    CK(hipStreamCreate(&st));
    rocblas_set_stream(h, st);
    const size_t ws_bytes = size_t(32) << 20;  // the session's rocBLAS workspace
    void* ws;
    CK(hipMalloc(&ws, ws_bytes));
    rocblas_set_workspace(h, ws, ws_bytes);
    // Chunks below 256 rows run the library's own row kernels (up to 32 rows)
    // or hipBLASLt, so the tables start at 256 rows.
    const int Ms[] = {256, 512, 1024, 2048, 3072, 4096, 5120, 6144, 7168, 8448};
    const int NK[][2] = {{2560, 2048}, {2048, 2048}, {12288, 2048}, {2048, 6144}};
    void *W, *X, *Y;
    CK(hipMalloc(&W, (size_t)12288 * 6144 * 2));
    CK(hipMalloc(&X, (size_t)8448 * 6144 * 2));
    CK(hipMalloc(&Y, (size_t)8448 * 12288 * 2));
    {
        // Random operands: MFMA power (and so clocks) depends on the data, and
        // a zero-filled problem runs well above the rate real weights reach.
        auto fill = [](void* d, size_t n) {
            std::vector<uint16_t> h(n);
            uint32_t r = 0x2545F491u;
            for (size_t i = 0; i < n; ++i) {
                r = r * 1664525u + 1013904223u;
                // bf16 of magnitude 2^-8..2^-1 with a random sign
                h[i] = (uint16_t)(((r >> 31) << 15) | ((0x77u + ((r >> 24) & 7u)) << 7) |
                                  ((r >> 9) & 0x7Fu));
            }
            CK(hipMemcpy(d, h.data(), n * 2, hipMemcpyHostToDevice));
        };
        fill(W, (size_t)12288 * 6144);
        fill(X, (size_t)8448 * 6144);
    }
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const float alpha = 1.f, beta = 0.f;
    char ver[256] = {0};
    rocblas_get_version_string(ver, sizeof(ver));
    std::printf("// rocBLAS %s\n", ver);
    for (int M : Ms)
        for (const auto& nk : NK) {
            const int N = nk[0], K = nk[1];
            auto run = [&](rocblas_gemm_algo algo, int idx) {
                return rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, N,
                                       M, K, &alpha, W, rocblas_datatype_bf16_r, K, X,
                                       rocblas_datatype_bf16_r, K, &beta, Y,
                                       rocblas_datatype_bf16_r, N, Y, rocblas_datatype_bf16_r,
                                       N, rocblas_datatype_f32_r, algo, idx, 0);
            };
            auto timeit = [&](rocblas_gemm_algo algo, int idx, int reps) -> float {
                if (run(algo, idx) != rocblas_status_success) return -1.f;
                CK(hipEventRecord(e0, st));
                for (int r = 0; r < reps; ++r) run(algo, idx);
                CK(hipEventRecord(e1, st));
                CK(hipEventSynchronize(e1));
                float ms = 0.f;
                CK(hipEventElapsedTime(&ms, e0, e1));
                return ms * 1000.f / (float)reps;
            };
            rocblas_int n = 0;
            rocblas_gemm_ex_get_solutions(
                h, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &alpha, W,
                rocblas_datatype_bf16_r, K, X, rocblas_datatype_bf16_r, K, &beta, Y,
                rocblas_datatype_bf16_r, N, Y, rocblas_datatype_bf16_r, N,
                rocblas_datatype_f32_r, rocblas_gemm_algo_solution_index, 0, nullptr, &n);
            std::vector<rocblas_int> list((size_t)std::max(n, 1));
            if (n > 0)
                rocblas_gemm_ex_get_solutions(
                    h, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &alpha, W,
                    rocblas_datatype_bf16_r, K, X, rocblas_datatype_bf16_r, K, &beta, Y,
                    rocblas_datatype_bf16_r, N, Y, rocblas_datatype_bf16_r, N,
                    rocblas_datatype_f32_r, rocblas_gemm_algo_solution_index, 0, list.data(),
                    &n);
            std::vector<std::pair<float, int>> t1;
            for (int i = 0; i < n; ++i) {
                const float t = timeit(rocblas_gemm_algo_solution_index, list[(size_t)i], 1);
                if (t > 0.f) t1.emplace_back(t, list[(size_t)i]);
            }
            std::sort(t1.begin(), t1.end());
            const float t_def = timeit(rocblas_gemm_algo_standard, 0, 20);
            float best = t_def;
            int bi = 0;
            for (size_t i = 0; i < t1.size() && i < 8u; ++i) {
                const float t = timeit(rocblas_gemm_algo_solution_index, t1[i].second, 20);
                if (t > 0.f && t < best) {
                    best = t;
                    bi = t1[i].second;
                }
            }
            if (best > 0.97f * t_def) bi = 0;
            std::printf("    {%d, %d, %d, %d},  // default %.1f us, chosen %.1f us\n", M, N, K, bi,
                        t_def, bi ? best : t_def);
            std::fflush(stdout);
        }
    return 0;
}
