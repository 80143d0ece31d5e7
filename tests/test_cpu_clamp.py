"""Bounds of the clamped page addressing the kernels use (kv_common.h
`table_index`, `clamp_page`, `token_base`): for any position and any table
entry, the page-table read stays inside the table's max_pages entries and the
token row addressed stays inside the pool; in-range values pass unchanged.
The header is compiled for the host (hipcc, no device code) into a small
checker that sweeps corner cases and random values."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "minicpm5-5080fast_amd", "csrc")

HARNESS = r"""
#include "kv_common.h"
#include <cstdio>
#include <random>
using namespace mckv;
int main() {
    std::mt19937_64 rng(12345);
    const uint32_t corner[] = {0u, 1u, 31u, 32u, 63u, 64u, 65u, 1000u, 0x7FFFFFFFu,
                               0xFFFFFFFEu, 0xFFFFFFFFu};
    long checks = 0;
    for (uint32_t log2p = 0; log2p <= 7; ++log2p)
        for (uint32_t maxp : {1u, 2u, 3u, 33u, 2048u, 4096u}) {
            DevLayout ly{maxp, log2p, (1u << log2p) - 1u, 3u};
            const uint64_t total = (uint64_t)3 * maxp * (1u << log2p) * kSlotElems;
            auto check = [&](uint32_t pos, uint32_t entry, uint32_t layer) {
                const uint32_t ti = table_index(ly, pos);
                if (ti >= maxp) return 1;
                if ((pos >> log2p) < maxp && ti != (pos >> log2p)) return 2;
                const uint32_t pg = clamp_page(ly, entry);
                if (pg >= maxp) return 3;
                if (entry < maxp && pg != entry) return 4;
                const uint64_t row = token_base(ly, layer, pg, pos & ly.pmask);
                if (row + kSlotElems > total) return 5;
                ++checks;
                return 0;
            };
            for (uint32_t a : corner)
                for (uint32_t b : corner)
                    for (uint32_t l = 0; l < 3; ++l)
                        if (int e = check(a, b, l)) { printf("fail %d %u %u\n", e, a, b); return 1; }
            for (int i = 0; i < 20000; ++i)
                if (int e = check((uint32_t)rng(), (uint32_t)rng() % (3u * maxp + 2u),
                                  (uint32_t)(rng() % 3u))) {
                    printf("fail %d\n", e);
                    return 1;
                }
        }
    printf("ok %ld\n", checks);
    return 0;
}
"""


def test_clamped_page_addressing_stays_in_pool(tmp_path):
    src = tmp_path / "clamp_check.cpp"
    src.write_text(HARNESS)
    exe = tmp_path / "clamp_check"
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    subprocess.run([hipcc, "-O1", "-std=c++17", "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
