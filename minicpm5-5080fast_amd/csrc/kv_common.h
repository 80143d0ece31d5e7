// kv_common.h - shared device/host definitions of the MI355X KV-cache path.
//
// Geometry constants follow the reference model config
// (native/runtime/generated_model_config.h:13-33): 16 query heads, 2 KV heads,
// head_dim 128, qkv row of 2560 bf16 (q | k | v).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mc_kv.h"

namespace mckv {

constexpr uint32_t kHq = 16;
constexpr uint32_t kHkv = 2;
constexpr uint32_t kGroup = kHq / kHkv;  // 8 query heads per KV head
constexpr uint32_t kD = 128;
constexpr uint32_t kRow = 2560;          // qkv row (bf16 elements)
constexpr uint32_t kKCol = 2048;         // first k column
constexpr uint32_t kVCol = 2304;         // first v column
constexpr uint32_t kSlotElems = 512;     // K|V x 2 heads x 128 per token
constexpr uint32_t kPartial = MC_KV_PARTIAL_STRIDE;  // {m, l, acc[128]}
constexpr uint32_t kSplit2 = MC_KV_MERGE_SPLIT2;
// 1/sqrt(128) rounded to fp32, the score scale of the reference
// (attention_decode.cu:116).
constexpr float kScoreScale = 0.08838834764831845f;

// Device view of mc_kv_layout_t with log2(P) precomputed.
struct DevLayout {
    uint32_t max_pages;
    uint32_t log2p;
    uint32_t pmask;
    uint32_t num_layers;
};

// Page-table index of position pos and a page id read from the table, both
// clamped to the pool's max_pages (a corrupt table entry or position then
// addresses a wrong page of the pool instead of memory outside it).
__host__ __device__ __forceinline__ uint32_t table_index(const DevLayout& ly, uint32_t pos) {
    const uint32_t i = pos >> ly.log2p;
    return i < ly.max_pages ? i : ly.max_pages - 1u;
}
__host__ __device__ __forceinline__ uint32_t clamp_page(const DevLayout& ly, uint32_t page) {
    return page < ly.max_pages ? page : ly.max_pages - 1u;
}

// Element offset of (layer, page, slot) token row (kv=0, head=0, d=0).
__host__ __device__ __forceinline__ uint64_t token_base(const DevLayout& ly,
                                                        uint32_t layer,
                                                        uint32_t page,
                                                        uint32_t slot) {
    return ((((uint64_t)layer * ly.max_pages + page) << ly.log2p) + slot) *
           (uint64_t)kSlotElems;
}

// ---- bf16 <-> fp32 ----
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)b << 16;
    return c.f;
}

// Round-to-nearest-even fp32 -> bf16; NaN keeps a quiet NaN payload.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    union { uint32_t u; float f; } c;
    c.f = f;
    const uint32_t u = c.u;
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u)
        return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// ---- RoPE angle -> (cos, sin) ----
// Deterministic fp64 evaluation rounded to fp32, shared by the append kernel
// and the decode phase0 so both write identical K bits. Method: Cody-Waite
// reduction by pi/2 with the three-part split of fdlibm's __ieee754_rem_pio2
// (each k*part exact for |k| < 2^20), then the Taylor series of sin/cos on
// [-pi/4, pi/4] through degree 17/18 in Horner form (truncation < 5e-17), then
// quadrant selection. Only IEEE fma/mul/add/rint are used, so a CPU build with
// the same operation sequence produces the same bits.
__host__ __device__ __forceinline__ void rope_sincos(float angle, float* c_out,
                                                     float* s_out) {
#pragma clang fp contract(off)
    const double x = (double)angle;
    const double k = __builtin_rint(x * 0.6366197723675814);
    double r = __builtin_fma(-k, 1.57079632673412561417e+00, x);
    r = __builtin_fma(-k, 6.07710050630396597660e-11, r);
    r = __builtin_fma(-k, 2.02226624879595063154e-21, r);
    const double r2 = r * r;
    double ps = 2.8114572543455206e-15;
    ps = __builtin_fma(ps, r2, -7.647163731819816e-13);
    ps = __builtin_fma(ps, r2, 1.6059043836821613e-10);
    ps = __builtin_fma(ps, r2, -2.505210838544172e-08);
    ps = __builtin_fma(ps, r2, 2.7557319223985893e-06);
    ps = __builtin_fma(ps, r2, -0.0001984126984126984);
    ps = __builtin_fma(ps, r2, 0.008333333333333333);
    ps = __builtin_fma(ps, r2, -0.16666666666666666);
    const double s = __builtin_fma(ps * r2, r, r);
    double pc = -1.5619206968586225e-16;
    pc = __builtin_fma(pc, r2, 4.779477332387385e-14);
    pc = __builtin_fma(pc, r2, -1.1470745597729725e-11);
    pc = __builtin_fma(pc, r2, 2.08767569878681e-09);
    pc = __builtin_fma(pc, r2, -2.755731922398589e-07);
    pc = __builtin_fma(pc, r2, 2.48015873015873e-05);
    pc = __builtin_fma(pc, r2, -0.001388888888888889);
    pc = __builtin_fma(pc, r2, 0.041666666666666664);
    pc = __builtin_fma(pc, r2, -0.5);
    const double c = __builtin_fma(pc, r2, 1.0);
    const int q = (int)((int64_t)k & 3);
    double cs, sn;
    if (q == 0) { cs = c; sn = s; }
    else if (q == 1) { cs = -s; sn = c; }
    else if (q == 2) { cs = -c; sn = -s; }
    else { cs = s; sn = -c; }
    *c_out = (float)cs;
    *s_out = (float)sn;
}

// rotate_half (non-interleaved) of one element: lower half d<64 gives
// x*c - x2*s, upper half x*c + x2*s, evaluated as t = s*x2 (rounded) followed
// by one fused multiply-add, the evaluation order the reference fixes for its
// rope store (attention_decode.cu:104-113).
__host__ __device__ __forceinline__ float rope_rotate(float x, float x2, float c,
                                                      float s, bool lower) {
#pragma clang fp contract(off)
    const float t = s * x2;
    return lower ? __builtin_fmaf(c, x, -t) : __builtin_fmaf(c, x, t);
}

}  // namespace mckv
