"""Runs the prefill GEMM solution tuner (tune_prefill_gemm.cpp) in this process.

The rocBLAS a process resolves decides which solution indices exist: a
process that imported torch first uses the librocblas PyTorch bundles, a
plain C/C++ caller the one under /opt/rocm. prefill_gemm_table.h keeps one
table per rocBLAS version string, so tune under each loader:

    make -C minicpm5-5080fast_amd/csrc tune
    python3 minicpm5-5080fast_amd/csrc/tune_prefill_gemm.py            # /opt/rocm
    python3 minicpm5-5080fast_amd/csrc/tune_prefill_gemm.py --torch    # torch's

Needs the GPU the table is for; prints the table rows on stdout.
"""
import ctypes
import os
import sys


def main() -> int:
    if "--torch" in sys.argv[1:]:
        import torch  # noqa: F401  (loads torch's rocBLAS first)

        torch.cuda.init()
    here = os.path.dirname(os.path.abspath(__file__))
    lib = ctypes.CDLL(os.path.join(here, "..", "tune_prefill_gemm.so"))
    sys.stdout.flush()
    return int(lib.tune_prefill_gemm_run())


if __name__ == "__main__":
    sys.exit(main())
