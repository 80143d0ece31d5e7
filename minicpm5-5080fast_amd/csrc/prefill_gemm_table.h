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
    {256, 2048, 2048, 0},  // default 8.8 us, chosen 8.8 us
    {256, 12288, 2048, 438638},  // default 20.0 us, chosen 15.5 us
    {256, 2048, 6144, 439289},  // default 50.5 us, chosen 17.9 us
    {512, 2560, 2048, 438699},  // default 12.7 us, chosen 11.3 us
    {512, 2048, 2048, 438490},  // default 10.4 us, chosen 9.7 us
    {512, 12288, 2048, 438908},  // default 26.4 us, chosen 24.1 us
    {512, 2048, 6144, 438490},  // default 22.2 us, chosen 21.3 us
    {1024, 2560, 2048, 438829},  // default 16.5 us, chosen 15.3 us
    {1024, 2048, 2048, 439044},  // default 13.8 us, chosen 12.8 us
    {1024, 12288, 2048, 0},  // default 40.0 us, chosen 40.0 us
    {1024, 2048, 6144, 438703},  // default 52.4 us, chosen 32.0 us
    {2048, 2560, 2048, 438280},  // default 23.6 us, chosen 21.9 us
    {2048, 2048, 2048, 438785},  // default 23.4 us, chosen 18.4 us
    {2048, 12288, 2048, 0},  // default 77.4 us, chosen 77.4 us
    {2048, 2048, 6144, 438785},  // default 56.6 us, chosen 47.6 us
    {3072, 2560, 2048, 439190},  // default 30.6 us, chosen 27.1 us
    {3072, 2048, 2048, 438994},  // default 26.6 us, chosen 23.1 us
    {3072, 12288, 2048, 0},  // default 116.9 us, chosen 116.9 us
    {3072, 2048, 6144, 438280},  // default 85.3 us, chosen 60.7 us
    {4096, 2560, 2048, 438853},  // default 36.6 us, chosen 35.0 us
    {4096, 2048, 2048, 0},  // default 28.5 us, chosen 28.5 us
    {4096, 12288, 2048, 0},  // default 131.8 us, chosen 131.8 us
    {4096, 2048, 6144, 439189},  // default 93.5 us, chosen 73.5 us
    {5120, 2560, 2048, 438973},  // default 45.3 us, chosen 40.2 us
    {5120, 2048, 2048, 0},  // default 33.3 us, chosen 33.3 us
    {5120, 12288, 2048, 439306},  // default 191.6 us, chosen 175.4 us
    {5120, 2048, 6144, 439046},  // default 93.7 us, chosen 86.6 us
    {6144, 2560, 2048, 0},  // default 44.3 us, chosen 44.3 us
    {6144, 2048, 2048, 438853},  // default 41.1 us, chosen 38.6 us
    {6144, 12288, 2048, 440238},  // default 263.7 us, chosen 211.8 us
    {6144, 2048, 6144, 439306},  // default 107.8 us, chosen 102.2 us
    {7168, 2560, 2048, 439434},  // default 67.4 us, chosen 57.7 us
    {7168, 2048, 2048, 0},  // default 43.6 us, chosen 43.6 us
    {7168, 12288, 2048, 439080},  // default 272.5 us, chosen 252.3 us
    {7168, 2048, 6144, 439285},  // default 121.8 us, chosen 113.4 us
    {8448, 2560, 2048, 438853},  // default 75.1 us, chosen 71.5 us
    {8448, 2048, 2048, 439422},  // default 68.4 us, chosen 58.2 us
    {8448, 12288, 2048, 440238},  // default 365.5 us, chosen 292.0 us
    {8448, 2048, 6144, 439253},  // default 168.5 us, chosen 159.2 us
};

// PyTorch's bundled rocBLAS 5.0.2.20250912-42-1199-g2584e35062.
inline constexpr PrefillGemmSolution kPrefillGemmTorch[] = {
    {256, 2560, 2048, 0},  // default 16.0 us, chosen 16.0 us
    {256, 2048, 2048, 0},  // default 19.9 us, chosen 19.9 us
    {256, 12288, 2048, 618509},  // default 22.9 us, chosen 20.7 us
    {256, 2048, 6144, 0},  // default 18.6 us, chosen 18.6 us
    {512, 2560, 2048, 0},  // default 16.3 us, chosen 16.3 us
    {512, 2048, 2048, 0},  // default 17.4 us, chosen 17.4 us
    {512, 12288, 2048, 0},  // default 26.7 us, chosen 26.7 us
    {512, 2048, 6144, 0},  // default 22.0 us, chosen 22.0 us
    {1024, 2560, 2048, 0},  // default 18.9 us, chosen 18.9 us
    {1024, 2048, 2048, 0},  // default 16.1 us, chosen 16.1 us
    {1024, 12288, 2048, 0},  // default 42.7 us, chosen 42.7 us
    {1024, 2048, 6144, 0},  // default 34.9 us, chosen 34.9 us
    {2048, 2560, 2048, 0},  // default 25.5 us, chosen 25.5 us
    {2048, 2048, 2048, 0},  // default 20.8 us, chosen 20.8 us
    {2048, 12288, 2048, 0},  // default 82.7 us, chosen 82.7 us
    {2048, 2048, 6144, 0},  // default 49.3 us, chosen 49.3 us
    {3072, 2560, 2048, 0},  // default 30.6 us, chosen 30.6 us
    {3072, 2048, 2048, 0},  // default 26.2 us, chosen 26.2 us
    {3072, 12288, 2048, 0},  // default 125.2 us, chosen 125.2 us
    {3072, 2048, 6144, 0},  // default 65.2 us, chosen 65.2 us
    {4096, 2560, 2048, 618613},  // default 40.7 us, chosen 38.4 us
    {4096, 2048, 2048, 0},  // default 31.5 us, chosen 31.5 us
    {4096, 12288, 2048, 0},  // default 140.6 us, chosen 140.6 us
    {4096, 2048, 6144, 0},  // default 80.1 us, chosen 80.1 us
    {5120, 2560, 2048, 0},  // default 42.2 us, chosen 42.2 us
    {5120, 2048, 2048, 0},  // default 37.4 us, chosen 37.4 us
    {5120, 12288, 2048, 618614},  // default 193.3 us, chosen 185.7 us
    {5120, 2048, 6144, 0},  // default 95.5 us, chosen 95.5 us
    {6144, 2560, 2048, 0},  // default 45.5 us, chosen 45.5 us
    {6144, 2048, 2048, 0},  // default 42.2 us, chosen 42.2 us
    {6144, 12288, 2048, 618614},  // default 470.5 us, chosen 227.1 us
    {6144, 2048, 6144, 0},  // default 109.1 us, chosen 109.1 us
    {7168, 2560, 2048, 618468},  // default 74.5 us, chosen 70.4 us
    {7168, 2048, 2048, 0},  // default 43.9 us, chosen 43.9 us
    {7168, 12288, 2048, 618612},  // default 278.8 us, chosen 258.0 us
    {7168, 2048, 6144, 0},  // default 116.8 us, chosen 116.8 us
    {8448, 2560, 2048, 0},  // default 75.0 us, chosen 75.0 us
    {8448, 2048, 2048, 0},  // default 65.8 us, chosen 65.8 us
    {8448, 12288, 2048, 618612},  // default 565.3 us, chosen 300.3 us
    {8448, 2048, 6144, 618468},  // default 353.7 us, chosen 169.6 us
};

inline constexpr PrefillGemmTable kPrefillGemmTables[] = {
    {"5.2.0.5b515cf1bc", kPrefillGemmRocm, sizeof(kPrefillGemmRocm) / sizeof(kPrefillGemmRocm[0])},
    {"5.0.2.20250912-42-1199-g2584e35062", kPrefillGemmTorch, sizeof(kPrefillGemmTorch) / sizeof(kPrefillGemmTorch[0])},
};

}  // namespace mckv
