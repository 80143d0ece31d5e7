// prefill_gemm_table.h - rocBLAS solution index per prefill projection shape.
//
// Rows y[M][N] = x[M][K] . W[N][K]^T of the four projections (qkv 2560x2048,
// o 2048x2048, gate_up 12288x2048, down 2048x6144), bf16 in/out, fp32
// compute. rocBLAS's default heuristic picks a solution per shape; timing
// every solution it lists for the shape (rocblas_gemm_ex_get_solutions)
// finds faster ones for some shapes. Solution indices belong to one rocBLAS
// build, and a process resolves whichever librocblas it loaded first: the one
// under /opt/rocm for a plain C/C++ caller, the one PyTorch bundles once torch
// is imported. So there is one table per rocBLAS version string; another
// build gets no table and runs the default heuristic.
//
// Written by tune_prefill_gemm.cpp (run by tune_prefill_gemm.py, plain and
// with --torch) on an MI355X, on random operands. Index 0 keeps the default
// heuristic (no solution measured 3% faster). A row count between two tuned
// ones uses the row of the lower one; below the smallest, the default.
#pragma once
#include <cstdint>

namespace mckv {

struct PrefillGemmSolution {
    uint32_t m, n, k;
    int32_t index;
};

struct PrefillGemmTable {
    const char* rocblas_version;
    const PrefillGemmSolution* rows;
    uint32_t count;
};

// /opt/rocm rocBLAS 5.2.0.5b515cf1bc. Ascending m within each (n, k).
inline constexpr PrefillGemmSolution kPrefillGemmRocm[] = {
    {256, 2560, 2048, 0},  // default 9.6 us, chosen 9.6 us
    {256, 2048, 2048, 0},  // default 8.9 us, chosen 8.9 us
    {256, 12288, 2048, 438638},  // default 20.0 us, chosen 15.3 us
    {256, 2048, 6144, 439289},  // default 50.3 us, chosen 17.8 us
    {512, 2560, 2048, 438699},  // default 12.8 us, chosen 11.4 us
    {512, 2048, 2048, 438490},  // default 10.3 us, chosen 9.9 us
    {512, 12288, 2048, 438908},  // default 25.9 us, chosen 23.8 us
    {512, 2048, 6144, 438490},  // default 22.1 us, chosen 21.1 us
    {1024, 2560, 2048, 438498},  // default 16.4 us, chosen 15.2 us
    {1024, 2048, 2048, 439044},  // default 13.9 us, chosen 12.6 us
    {1024, 12288, 2048, 0},  // default 39.4 us, chosen 39.4 us
    {1024, 2048, 6144, 438703},  // default 52.3 us, chosen 31.3 us
    {2048, 2560, 2048, 438991},  // default 23.0 us, chosen 21.9 us
    {2048, 2048, 2048, 438649},  // default 23.3 us, chosen 18.3 us
    {2048, 12288, 2048, 0},  // default 74.7 us, chosen 74.7 us
    {2048, 2048, 6144, 439119},  // default 56.5 us, chosen 46.5 us
    {4096, 2560, 2048, 0},  // default 35.8 us, chosen 35.8 us
    {4096, 2048, 2048, 0},  // default 27.8 us, chosen 27.8 us
    {4096, 12288, 2048, 0},  // default 129.4 us, chosen 129.4 us
    {4096, 2048, 6144, 439189},  // default 92.3 us, chosen 71.8 us
    {8448, 2560, 2048, 438853},  // default 73.0 us, chosen 70.6 us
    {8448, 2048, 2048, 439422},  // default 65.4 us, chosen 57.0 us
    {8448, 12288, 2048, 440238},  // default 341.6 us, chosen 282.4 us
    {8448, 2048, 6144, 439217},  // default 164.6 us, chosen 156.1 us
};

// PyTorch's bundled rocBLAS 5.0.2.20250912-42-1199-g2584e35062.
inline constexpr PrefillGemmSolution kPrefillGemmTorch[] = {
    {256, 2560, 2048, 0},  // default 17.0 us, chosen 17.0 us
    {256, 2048, 2048, 0},  // default 16.0 us, chosen 16.0 us
    {256, 12288, 2048, 618501},  // default 22.8 us, chosen 20.3 us
    {256, 2048, 6144, 0},  // default 19.0 us, chosen 19.0 us
    {512, 2560, 2048, 0},  // default 16.3 us, chosen 16.3 us
    {512, 2048, 2048, 0},  // default 16.2 us, chosen 16.2 us
    {512, 12288, 2048, 0},  // default 26.6 us, chosen 26.6 us
    {512, 2048, 6144, 0},  // default 21.8 us, chosen 21.8 us
    {1024, 2560, 2048, 0},  // default 19.0 us, chosen 19.0 us
    {1024, 2048, 2048, 0},  // default 15.3 us, chosen 15.3 us
    {1024, 12288, 2048, 0},  // default 42.1 us, chosen 42.1 us
    {1024, 2048, 6144, 0},  // default 35.0 us, chosen 35.0 us
    {2048, 2560, 2048, 0},  // default 25.7 us, chosen 25.7 us
    {2048, 2048, 2048, 0},  // default 20.9 us, chosen 20.9 us
    {2048, 12288, 2048, 0},  // default 81.9 us, chosen 81.9 us
    {2048, 2048, 6144, 0},  // default 48.6 us, chosen 48.6 us
    {4096, 2560, 2048, 618612},  // default 40.0 us, chosen 38.0 us
    {4096, 2048, 2048, 0},  // default 31.2 us, chosen 31.2 us
    {4096, 12288, 2048, 0},  // default 138.0 us, chosen 138.0 us
    {4096, 2048, 6144, 0},  // default 77.4 us, chosen 77.4 us
    {8448, 2560, 2048, 0},  // default 75.4 us, chosen 75.4 us
    {8448, 2048, 2048, 0},  // default 65.6 us, chosen 65.6 us
    {8448, 12288, 2048, 618612},  // default 608.6 us, chosen 300.5 us
    {8448, 2048, 6144, 618468},  // default 352.7 us, chosen 167.3 us
};

inline constexpr PrefillGemmTable kPrefillGemmTables[] = {
    {"5.2.0.5b515cf1bc", kPrefillGemmRocm, sizeof(kPrefillGemmRocm) / sizeof(kPrefillGemmRocm[0])},
    {"5.0.2.20250912-42-1199-g2584e35062", kPrefillGemmTorch, sizeof(kPrefillGemmTorch) / sizeof(kPrefillGemmTorch[0])},
};

}  // namespace mckv
