// model_kernels.hip - weight-path kernels of the MiniCPM5 forward for gfx950:
// embedding gather, RMSNorm, residual add + RMSNorm, SwiGLU, bf16 GEMV for 1-8
// activation rows (plain, with a fused residual + RMSNorm prologue, or with a
// fused SwiGLU prologue) and greedy argmax.
//
// Semantics follow the reference kernels (native/kernels/sm120/kernels.h):
//   * embedding: out[t] = table[id[t]] (kernels.h:156, :197 for the per-slot
//     token pointers of a batch step);
//   * RMSNorm: inv = 1/sqrt(sum(x^2)/n + eps) in fp32, out = bf16(x * inv * w)
//     (kernels.h:172); residual add + RMSNorm first stores res = bf16(res + x)
//     and normalizes the rounded residual (kernels.h:185);
//   * SwiGLU on the gate|up row: out = bf16(silu(g) * u), silu(g) =
//     g / (1 + exp(-g)) in fp32 (kernels.h:589);
//   * GEMV: y[m][n] = bf16(sum_k W[n][k] x[m][k]), W row-major [N][K], fp32
//     accumulation (kernels.h:666, the prologue forms :743 and :760);
//   * greedy argmax over bf16 logits compared in fp32, ties to the lowest
//     index (kernels.h:610, :641).
//
// MI355X design of the GEMV (decode is HBM-bound: every weight byte is read
// once per token): a workgroup first stages its activation rows
// (after the fused prologue) into LDS, then each wave streams whole weight
// rows, one row at a time, with the next row's loads issued before the
// current row is reduced. Lane l reads the 16-byte chunks l, l + 64, ... of
// the row (K / 512 of them; whole 1 KB per wave instruction, non-temporal),
// multiplies them with the matching LDS chunks of each activation row through
// v_dot2c_f32_bf16 (two bf16 products accumulated in fp32 per instruction),
// and the lane sums of all activation rows (and of the gate and up rows) of a
// column are combined by one reduce-scatter over the 64 lanes with a fixed
// pairing order (lane_reduce_scatter).
#include <hip/hip_runtime.h>

#include "error.h"
#include "kv_common.h"
#include "mc_model.h"
#include "trace.h"

namespace mckv {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kThreads = 256;
constexpr uint32_t kMaxRows = MC_MODEL_GEMV_MAX_ROWS;  // activation rows per GEMV
// GEMV grids. One activation row: workgroups of 4 waves, up to 1024 of them
// (one output column per wave for the 2560-column qkv projection); the
// prologue is short. Several rows: every workgroup stages all rows (and runs
// the norm prologue for each) before streaming columns, so the staging is
// paid once per workgroup: one 8-wave workgroup per CU (measured against
// 4 waves x 512 and 16 waves x 256: 8.7 / 9.3 / 16.9 us for the 8-row qkv
// projection; 16 waves spill).
constexpr uint32_t kSoloWaves = 4, kSoloBlocks = 1024;
constexpr uint32_t kMultiWaves = 8, kMultiBlocks = 256;

__device__ __forceinline__ uint4 ld_stream(const uint16_t* p) {
    return __builtin_bit_cast(uint4,
                              __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}
__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ float lo_f(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_f(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
// Two fp32 -> bf16 round-to-nearest-even conversions in one v_cvt_pk_bf16_f32
// (a in the low half).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// Sum over the 64 lanes, every lane receiving the total: xor 1 and xor 2
// within quads, the 8- and 16-lane mirrors, then the 16- and 32-lane row
// swaps. The same operands meet in the same order on every call.
__device__ __forceinline__ float wave_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));
    {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                         false, false);
        x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    }
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sum over a 256-thread workgroup (waves in order 0..3), returned to all.
__device__ __forceinline__ float block_sum(float x, float* s4) {
    x = wave_sum(x);
    const uint32_t wave = threadIdx.x >> 6;
    __syncthreads();  // s4 may still be read by a previous call
    if ((threadIdx.x & 63u) == 0u) s4[wave] = x;
    __syncthreads();
    return ((s4[0] + s4[1]) + s4[2]) + s4[3];
}

// Sums of V (a power of two, at most 16) per-lane values over the 64 lanes,
// one value per lane group: value j ends in the 64 / V lanes l with
// l / (64 / V) == j. The pairings run in one fixed order (lanes l and l ^ 32,
// l ^ 16, the 16-lane mirror, the 8-lane mirror, l ^ 2, l ^ 1); the first
// log2(V) of them halve the set of values a lane carries (each side keeps
// one half and adds the partner's copy of it), the rest finish the sum of
// the one value left. Every value therefore goes through the same addition
// tree whatever V is, so a column's result does not depend on how many
// activation rows the launch has.
// one pairing stage K of lane_reduce_scatter over the first C values
template <uint32_t K, uint32_t C, uint32_t V>
__device__ __forceinline__ void lane_pair_stage(float (&v)[V], uint32_t lane) {
    constexpr uint32_t H = C > 1u ? C / 2u : 1u;  // values after this stage
#pragma unroll
    for (uint32_t i = 0; i < H; ++i) {
        const float u = v[i], w = C > 1u ? v[i + H] : v[i];
        if constexpr (K < 2u) {
            // swap: row-even lanes end with (own u, partner u), row-odd lanes
            // with (partner w, own w); the sum is even + odd
            const auto a = K == 0u ? __builtin_amdgcn_permlane32_swap(__float_as_uint(u),
                                                                     __float_as_uint(w), false,
                                                                     false)
                                   : __builtin_amdgcn_permlane16_swap(__float_as_uint(u),
                                                                     __float_as_uint(w), false,
                                                                     false);
            v[i] = __uint_as_float(a[0]) + __uint_as_float(a[1]);
        } else {
            constexpr int kCtl = K == 2u ? 0x140 : K == 3u ? 0x141 : K == 4u ? 0x4E : 0xB1;
            const bool right = ((lane >> (5u - K)) & 1u) != 0u;
            const float keep = right ? w : u, send = right ? u : w;
            v[i] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), kCtl, 0xF,
                                                                   0xF, false));
        }
    }
}

template <uint32_t V>
__device__ __forceinline__ float lane_reduce_scatter(float (&v)[V]) {
    static_assert(V >= 1u && V <= 16u && (V & (V - 1u)) == 0u, "power of two up to 16");
    const uint32_t lane = threadIdx.x & 63u;
    // 0: permlane32 swap, 1: permlane16 swap, 2: row mirror, 3: half-row
    // mirror, 4: quad xor 2, 5: quad xor 1
    constexpr uint32_t C1 = V > 1u ? V / 2u : 1u, C2 = C1 > 1u ? C1 / 2u : 1u;
    constexpr uint32_t C3 = C2 > 1u ? C2 / 2u : 1u, C4 = C3 > 1u ? C3 / 2u : 1u;
    constexpr uint32_t C5 = C4 > 1u ? C4 / 2u : 1u;
    lane_pair_stage<0u, V>(v, lane);
    lane_pair_stage<1u, C1>(v, lane);
    lane_pair_stage<2u, C2>(v, lane);
    lane_pair_stage<3u, C3>(v, lane);
    lane_pair_stage<4u, C4>(v, lane);
    lane_pair_stage<5u, C5>(v, lane);
    return v[0];
}

// ---- embedding gather ----
// grid = rows, block = 256; 16-byte chunks of the hidden row per thread.
__global__ void __launch_bounds__(kThreads)
    embed_kernel(const uint16_t* __restrict__ table, const int32_t* __restrict__ ids,
                 const int32_t* const* __restrict__ slot_tok, uint16_t* __restrict__ out,
                 uint32_t hidden) {
    const uint32_t row = blockIdx.x;
    const int64_t id = slot_tok != nullptr ? *slot_tok[row] : ids[row];
    const uint16_t* src = table + id * (int64_t)hidden;
    uint16_t* dst = out + (size_t)row * hidden;
    for (uint32_t c = threadIdx.x; c < hidden / 8u; c += kThreads)
        *reinterpret_cast<uint4*>(dst + 8u * c) = ld16(src + 8u * c);
}

// ---- RMSNorm rows, optionally after the residual add ----
// grid = rows, block = 256. Each thread owns the same 8-element chunks in
// both passes, so re-reading its own residual stores needs no barrier.
__global__ void __launch_bounds__(kThreads)
    resnorm_kernel(uint16_t* __restrict__ res, const uint16_t* __restrict__ delta,
                   const uint16_t* __restrict__ w, uint16_t* __restrict__ out, uint32_t n,
                   float eps) {
    __shared__ float s4[4];
    uint16_t* r = res + (size_t)blockIdx.x * n;
    const uint16_t* d = delta != nullptr ? delta + (size_t)blockIdx.x * n : nullptr;
    uint16_t* o = out + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (uint32_t c = threadIdx.x; c < n / 8u; c += kThreads) {
        uint4 v = ld16(r + 8u * c);
        if (d != nullptr) {
            const uint4 a = ld16(d + 8u * c);
            v.x = pack2(lo_f(v.x) + lo_f(a.x), hi_f(v.x) + hi_f(a.x));
            v.y = pack2(lo_f(v.y) + lo_f(a.y), hi_f(v.y) + hi_f(a.y));
            v.z = pack2(lo_f(v.z) + lo_f(a.z), hi_f(v.z) + hi_f(a.z));
            v.w = pack2(lo_f(v.w) + lo_f(a.w), hi_f(v.w) + hi_f(a.w));
            *reinterpret_cast<uint4*>(r + 8u * c) = v;
        }
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = lo_f(u[i]), b = hi_f(u[i]);
            ss = fmaf(a, a, ss);
            ss = fmaf(b, b, ss);
        }
    }
    const float inv = 1.0f / sqrtf(block_sum(ss, s4) / (float)n + eps);
    for (uint32_t c = threadIdx.x; c < n / 8u; c += kThreads) {
        const uint4 v = ld16(r + 8u * c), g = ld16(w + 8u * c);
        uint4 y;
        y.x = pack2(lo_f(v.x) * inv * lo_f(g.x), hi_f(v.x) * inv * hi_f(g.x));
        y.y = pack2(lo_f(v.y) * inv * lo_f(g.y), hi_f(v.y) * inv * hi_f(g.y));
        y.z = pack2(lo_f(v.z) * inv * lo_f(g.z), hi_f(v.z) * inv * hi_f(g.z));
        y.w = pack2(lo_f(v.w) * inv * lo_f(g.w), hi_f(v.w) * inv * hi_f(g.w));
        *reinterpret_cast<uint4*>(o + 8u * c) = y;
    }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    return g / (1.0f + expf(-g)) * u;
}
__device__ __forceinline__ uint4 swiglu8(const uint4& g, const uint4& u) {
    uint4 y;
    y.x = pack2(silu_mul(lo_f(g.x), lo_f(u.x)), silu_mul(hi_f(g.x), hi_f(u.x)));
    y.y = pack2(silu_mul(lo_f(g.y), lo_f(u.y)), silu_mul(hi_f(g.y), hi_f(u.y)));
    y.z = pack2(silu_mul(lo_f(g.z), lo_f(u.z)), silu_mul(hi_f(g.z), hi_f(u.z)));
    y.w = pack2(silu_mul(lo_f(g.w), lo_f(u.w)), silu_mul(hi_f(g.w), hi_f(u.w)));
    return y;
}

// ---- SwiGLU rows: src [rows][2*inter] (gate | up) -> out [rows][inter] ----
// grid = (ceil(inter / 8 / 256), rows), block = 256.
__global__ void __launch_bounds__(kThreads)
    swiglu_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ out,
                  uint32_t inter) {
    const uint32_t c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= inter / 8u) return;
    const uint16_t* s = src + (size_t)blockIdx.y * 2u * inter;
    *reinterpret_cast<uint4*>(out + (size_t)blockIdx.y * inter + 8u * c) =
        swiglu8(ld16(s + 8u * c), ld16(s + inter + 8u * c));
}

// ---- GEMV ----
enum : uint32_t { kProNone = 0, kProResnorm = 1, kProSwiglu = 2 };

struct GemvArgs {
    const uint16_t* w;  // [N][K]
    uint32_t N;
    const uint16_t* x;  // kProNone: rows [M][ldx]; kProSwiglu: gate|up rows [M][ldx]
    uint32_t ldx;
    const uint16_t* res_in;  // kProResnorm: [M][ldr]
    const uint16_t* addend;  // kProResnorm: [M][ldr] or nullptr
    const uint16_t* norm_w;  // kProResnorm: [K]
    uint16_t* res_out;       // kProResnorm: [M][ldr] (written by workgroup 0) or nullptr
    uint32_t ldr;
    float eps;
    uint16_t* y;  // [M][ldy]
    uint32_t ldy;
};

// Stages M activation rows of K bf16 into LDS sx[M][K / 8] (16-byte chunks)
// with block T threads: plain (x rows of stride ldx), SwiGLU of gate|up rows,
// or residual add + RMSNorm (K = 2048: r = bf16(res_in + addend) stored to
// res_out by workgroup 0 when not null, x = bf16(r * inv * norm_w); all M
// rows' sums of squares in one workgroup reduction). All of a thread's row
// loads are issued first, then issue() (the caller's first weight loads),
// then the rest: vector loads complete in issue order, so waiting for the
// rows does not wait for the weights, and the prologue runs under the weight
// latency. The caller synchronizes before reading sx.
template <uint32_t M, uint32_t PRO, uint32_t K, uint32_t T, typename Issue>
__device__ __forceinline__ void stage_rows(const uint16_t* x, uint32_t ldx,
                                           const uint16_t* res_in, const uint16_t* addend,
                                           const uint16_t* norm_w, uint16_t* res_out,
                                           uint32_t ldr, float eps, uint4* sx, Issue issue) {
    constexpr uint32_t NCH = K / 8u;
    static_assert(PRO != kProResnorm || K == 2048u, "the norm prologue covers 2048 dims");
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    if constexpr (PRO == kProResnorm) {
        // Item i = 256 m + c is the 16-byte chunk c of row m; a row's 256
        // items are four whole waves, so each wave sums one row's part and
        // all M rows' sums of squares come out of one workgroup barrier.
        constexpr uint32_t IT = (M * 256u + T - 1u) / T;
        __shared__ float s_part[M][4];
        uint4 v[IT], d[IT], g[IT];
#pragma unroll
        for (uint32_t it = 0; it < IT; ++it) {
            const uint32_t i = tid + it * T;
            if (i >= M * 256u) break;  // wave-uniform
            const uint32_t m = i >> 8, c = i & 255u;
            // (unconditional loads keep the compiler's wait counts exact;
            // without an addend the residual row is read twice and not added)
            v[it] = ld16(res_in + (size_t)m * ldr + 8u * c);
            d[it] = ld16((addend != nullptr ? addend : res_in) + (size_t)m * ldr + 8u * c);
            g[it] = ld16(norm_w + 8u * c);
        }
        issue();
#pragma unroll
        for (uint32_t it = 0; it < IT; ++it) {
            const uint32_t i = tid + it * T;
            if (i >= M * 256u) break;  // wave-uniform
            const uint32_t m = i >> 8, c = i & 255u;
            if (addend != nullptr) {
                v[it].x = pack2(lo_f(v[it].x) + lo_f(d[it].x), hi_f(v[it].x) + hi_f(d[it].x));
                v[it].y = pack2(lo_f(v[it].y) + lo_f(d[it].y), hi_f(v[it].y) + hi_f(d[it].y));
                v[it].z = pack2(lo_f(v[it].z) + lo_f(d[it].z), hi_f(v[it].z) + hi_f(d[it].z));
                v[it].w = pack2(lo_f(v[it].w) + lo_f(d[it].w), hi_f(v[it].w) + hi_f(d[it].w));
            }
            if (res_out != nullptr && blockIdx.x == 0u)
                *reinterpret_cast<uint4*>(res_out + (size_t)m * ldr + 8u * c) = v[it];
            const uint32_t u[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
            float t = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = lo_f(u[j]), q = hi_f(u[j]);
                t = fmaf(p, p, t);
                t = fmaf(q, q, t);
            }
            t = wave_sum(t);
            if (lane == 0u) s_part[m][c >> 6] = t;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t it = 0; it < IT; ++it) {
            const uint32_t i = tid + it * T;
            if (i >= M * 256u) break;
            const uint32_t m = i >> 8, c = i & 255u;
            const float tot = ((s_part[m][0] + s_part[m][1]) + s_part[m][2]) + s_part[m][3];
            const float inv = 1.0f / sqrtf(tot / (float)K + eps);
            const uint4 gw = g[it];
            uint4 o;
            o.x = pack2(lo_f(v[it].x) * inv * lo_f(gw.x), hi_f(v[it].x) * inv * hi_f(gw.x));
            o.y = pack2(lo_f(v[it].y) * inv * lo_f(gw.y), hi_f(v[it].y) * inv * hi_f(gw.y));
            o.z = pack2(lo_f(v[it].z) * inv * lo_f(gw.z), hi_f(v[it].z) * inv * hi_f(gw.z));
            o.w = pack2(lo_f(v[it].w) * inv * lo_f(gw.w), hi_f(v[it].w) * inv * hi_f(gw.w));
            sx[m * NCH + c] = o;
        }
    } else {
        constexpr uint32_t IT = (M * NCH + T - 1u) / T;
        constexpr uint32_t H = PRO == kProSwiglu ? 2u : 1u;  // gate, up
        uint4 t[IT][H];
#pragma unroll
        for (uint32_t it = 0; it < IT; ++it) {
            const uint32_t i = tid + it * T;
            if (i >= M * NCH) break;
            const uint32_t m = i / NCH, c = i % NCH;
            const uint16_t* xr = x + (size_t)m * ldx + 8u * c;
#pragma unroll
            for (uint32_t h = 0; h < H; ++h) t[it][h] = ld16(xr + h * K);
        }
        issue();
#pragma unroll
        for (uint32_t it = 0; it < IT; ++it) {
            const uint32_t i = tid + it * T;
            if (i >= M * NCH) break;
            if constexpr (PRO == kProSwiglu) sx[i] = swiglu8(t[it][0], t[it][1]);
            else sx[i] = t[it][0];
        }
    }
}

// K = 512 * KC (16-byte chunks per lane per row); WV waves per workgroup,
// one output column per wave at a time. kProResnorm needs K = 2048.
// SWI: SwiGLU epilogue. Output column n (n < a.N) takes the weight rows n
// (gate) and a.N + n (up) of a [2 a.N][K] matrix: y = bf16(silu(g) * u) with
// g, u the two dot products rounded to bf16 first (the projection's output
// rounding), as a gate_up projection followed by the SwiGLU kernel.
template <uint32_t M, uint32_t PRO, uint32_t KC, bool SWI, uint32_t WV>
__global__ void __launch_bounds__(64u * WV)
    gemv_kernel(const uint16_t* w, const uint16_t* x, const uint16_t* res_in,
                const uint16_t* addend, const uint16_t* norm_w, uint32_t N, uint32_t ldx,
                const GemvArgs args) {
    // The pointers and sizes needed before the first loads come as leading
    // scalar arguments, which this file's build preloads into SGPRs at wave
    // launch (no argument load round before the weight and activation
    // requests); the rest of the arguments is read from the struct.
    GemvArgs a = args;
    a.w = w;
    a.x = x;
    a.res_in = res_in;
    a.addend = addend;
    a.norm_w = norm_w;
    a.N = N;
    a.ldx = ldx;
    constexpr uint32_t K = 512u * KC, NCH = K / 8u, T = 64u * WV;
    static_assert(PRO != kProResnorm || K == 2048u, "the norm prologue covers 2048 dims");
    __shared__ uint4 sx[M * NCH];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // The row is streamed in groups of kG chunks per lane (K / (512 kG) groups
    // per row); the next group's loads (of this row or the next one) are
    // issued before the current group is multiplied, so each lane keeps 2 kG
    // 16-byte loads in flight whatever K is. The first group is requested
    // before the activation prologue: the weights do not depend on it, so the
    // two memory latencies overlap instead of adding up.
    // one activation row: the whole weight row is requested at once (12
    // loads per lane for K = 6144); several rows: groups of 4 chunks
    constexpr uint32_t kG = M == 1u ? KC : 4u, NG = KC / kG;
    constexpr uint32_t R = SWI ? 2u : 1u;  // weight rows per output column
    static_assert(KC % kG == 0u, "whole chunk groups");
    const uint32_t stride = gridDim.x * WV;
    uint32_t n = blockIdx.x * WV + wave, g = 0u;
    const bool active = n < a.N;  // wave-uniform
    auto load = [&](uint4 (&dst)[R][kG], uint32_t col, uint32_t grp) {
#pragma unroll
        for (uint32_t r = 0; r < R; ++r)
#pragma unroll
            for (uint32_t c = 0; c < kG; ++c)
                dst[r][c] = ld_stream(a.w + (size_t)(col + r * a.N) * K +
                                      8u * (lane + 64u * (grp * kG + c)));
    };
    uint4 wc[R][kG];
    stage_rows<M, PRO, K, T>(a.x, a.ldx, a.res_in, a.addend, a.norm_w, a.res_out, a.ldr, a.eps,
                             sx, [&] {
                                 // an inactive wave loads the last row (exact
                                 // wait counts; the values are never used)
                                 load(wc, active ? n : a.N - 1u, g);
                             });
    __syncthreads();
    if (!active) return;  // wave-uniform; no barrier follows
    float acc[R][M];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r)
#pragma unroll
        for (uint32_t m = 0; m < M; ++m) acc[r][m] = 0.f;
    while (true) {
        uint32_t g2 = g + 1u, n2 = n;
        if (g2 == NG) {
            g2 = 0u;
            n2 = n + stride;
        }
        const bool more = n2 < a.N;
        uint4 wn[R][kG];
        if (more) load(wn, n2, g2);
#pragma unroll
        for (uint32_t c = 0; c < kG; ++c) {
            const uint32_t ch = lane + 64u * (g * kG + c);
#pragma unroll
            for (uint32_t m = 0; m < M; ++m) {
                const uint4 xv = sx[m * NCH + ch];
#pragma unroll
                for (uint32_t r = 0; r < R; ++r) {
                    const uint4 wv = wc[r][c];
                    float t = acc[r][m];
                    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.x),
                                                        __builtin_bit_cast(bf16x2_t, xv.x), t,
                                                        false);
                    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.y),
                                                        __builtin_bit_cast(bf16x2_t, xv.y), t,
                                                        false);
                    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.z),
                                                        __builtin_bit_cast(bf16x2_t, xv.z), t,
                                                        false);
                    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wv.w),
                                                        __builtin_bit_cast(bf16x2_t, xv.w), t,
                                                        false);
                    acc[r][m] = t;
                }
            }
        }
        if (g == NG - 1u) {  // column complete (wave-uniform)
            // value j = r * MP + m (zero for m >= M), summed over the lanes
            // at once: value j ends in lanes l >> (6 - log2 V) == j
            constexpr uint32_t MP = M <= 1u ? 1u : M <= 2u ? 2u : M <= 4u ? 4u : 8u;
            constexpr uint32_t V = R * MP;
            constexpr uint32_t kShift = V == 1u ? 6u : V == 2u ? 5u : V == 4u ? 4u
                                      : V == 8u ? 3u : 2u;
            float vals[V];
#pragma unroll
            for (uint32_t r = 0; r < R; ++r)
#pragma unroll
                for (uint32_t m = 0; m < MP; ++m) vals[r * MP + m] = m < M ? acc[r][m] : 0.f;
            float v = lane_reduce_scatter<V>(vals);
            const uint32_t j = kShift == 6u ? 0u : lane >> kShift;
            if constexpr (SWI) {
                // gate (r = 0) in lanes < 32, up (r = 1) in the lane 32 above
                const auto gu = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                                 __float_as_uint(v), false, false);
                const float gt = bf16_to_f32(f32_to_bf16(__uint_as_float(gu[0])));
                const float up = bf16_to_f32(f32_to_bf16(__uint_as_float(gu[1])));
                v = silu_mul(gt, up);
            }
            const uint32_t m = j % MP;
            if ((kShift == 6u || (lane & ((1u << kShift) - 1u)) == 0u) && j < MP && m < M)
                a.y[(size_t)m * a.ldy + n] = f32_to_bf16(v);
#pragma unroll
            for (uint32_t r = 0; r < R; ++r)
#pragma unroll
                for (uint32_t m2 = 0; m2 < M; ++m2) acc[r][m2] = 0.f;
        }
        if (!more) break;
#pragma unroll
        for (uint32_t r = 0; r < R; ++r)
#pragma unroll
            for (uint32_t c = 0; c < kG; ++c) wc[r][c] = wn[r][c];
        n = n2;
        g = g2;
    }
}

// ---- FP8 GEMV (one activation row) ----
// y[n] = bf16(scale[n] * sum_k e4m3(w[n][k]) x[k]) with fp32 accumulation,
// the row scale applied after the sum. Weights: uint8 e4m3 [N][K] rows
// (K / 16 16-byte chunks), lane l of a wave reading chunks l, l + 64, ...
// of each row it takes (KC8 = K / 1024 per lane; 1 KB per wave load). The
// activation row is staged once per workgroup through the prologue into LDS
// (stage_rows, as the bf16 GEMV) when the norm prologue runs, and read by
// each lane directly otherwise; a lane's chunks are the same for every row,
// so it keeps its K / 64 activation values in registers (fp32) and every
// row is one weight load round and 16 FMAs per chunk. e4m3 -> fp32 is v_cvt_pk_f32_fp8 (exact); the codes S.1111.111,
// which it reads as NaN, are decoded by the bit layout instead (+-480) in a
// rarely taken branch, so every code has the meaning of the oracle's decoder.
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float e4m3_bits_to_f32(uint32_t b) {
    // exponent field e, mantissa m: e = 0 -> m/8 * 2^-6, else (1 + m/8) 2^(e-7)
    // (the fp32 with the 7 magnitude bits at bit 20 is that value * 2^-120)
    const float mag = __uint_as_float((b & 0x7Fu) << 20) * 0x1p120f;
    return (b & 0x80u) ? -mag : mag;
}

__device__ __forceinline__ void fp8x16_fma(const uint4& w, const float* x, float& s0,
                                           float& s1) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
    uint32_t nan_code = 0u;  // a byte 0x7F or 0xFF in the chunk
#pragma unroll
    for (int i = 0; i < 4; ++i) nan_code |= ((u[i] & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u;
    if (nan_code == 0u) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)u[i], false);
            const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)u[i], true);
            s0 = fmaf(lo[0], x[4 * i + 0], s0);
            s1 = fmaf(lo[1], x[4 * i + 1], s1);
            s0 = fmaf(hi[0], x[4 * i + 2], s0);
            s1 = fmaf(hi[1], x[4 * i + 3], s1);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0 = fmaf(e4m3_bits_to_f32(u[i] & 0xFFu), x[4 * i + 0], s0);
            s1 = fmaf(e4m3_bits_to_f32((u[i] >> 8) & 0xFFu), x[4 * i + 1], s1);
            s0 = fmaf(e4m3_bits_to_f32((u[i] >> 16) & 0xFFu), x[4 * i + 2], s0);
            s1 = fmaf(e4m3_bits_to_f32(u[i] >> 24), x[4 * i + 3], s1);
        }
    }
}

struct Gemv8Args {
    const uint8_t* w;      // [N][K] (SwiGLU epilogue: [2N][K], gate rows then up rows)
    const float* scale;    // [N] ([2N])
    uint32_t N;
    const uint16_t* x;     // kProNone: [K]; kProSwiglu: gate|up [2K]
    const uint16_t* res_in;  // kProResnorm: [2048]
    const uint16_t* addend;  // kProResnorm: [2048] or nullptr
    const uint16_t* norm_w;  // kProResnorm: [2048]
    uint16_t* res_out;       // kProResnorm: [2048] (workgroup 0) or nullptr
    float eps;
    uint16_t* y;  // [N]
};

// Waves (output rows in flight) per workgroup: 8 with the norm prologue,
// whose staging is shared by the workgroup's waves; 4 otherwise (measured:
// 8-row qkv-shape norm prologue 3.98 us with 8 waves against 4.24 with 4;
// plain o 2.85 us with direct loads against 3.10 staged).
template <uint32_t PRO>
constexpr uint32_t f8_waves() { return PRO == kProResnorm ? 8u : 4u; }
// Grids: at most 4096 waves (one or two output rows each for the layer
// projections), and kF8WideWaves for the lm_head-sized launches (N >=
// kF8WideRows), whose waves walk many rows: more waves keep more rows in
// flight (measured: lm_head 61.1 us with 4096 waves, 46.6 with 8192).
constexpr uint32_t kF8WideRows = 65536, kF8WideWaves = 8192;

template <uint32_t PRO, uint32_t KC8, bool SWI>
__global__ void __launch_bounds__(64u * f8_waves<PRO>()) gemv8_kernel(const Gemv8Args a) {
    constexpr uint32_t kF8Waves = f8_waves<PRO>();
    constexpr uint32_t K = 1024u * KC8;
    constexpr uint32_t R = SWI ? 2u : 1u;
    static_assert(PRO != kProResnorm || K == 2048u, "the norm prologue covers 2048 dims");
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t stride = gridDim.x * kF8Waves;
    uint32_t n = blockIdx.x * kF8Waves + wave;
    const bool active = n < a.N;  // wave-uniform
    auto load = [&](uint4 (&dst)[R][KC8], uint32_t col) {
#pragma unroll
        for (uint32_t r = 0; r < R; ++r)
#pragma unroll
            for (uint32_t c = 0; c < KC8; ++c)
                dst[r][c] = ld_stream(reinterpret_cast<const uint16_t*>(
                    a.w + (size_t)(col + r * a.N) * K + 16u * (lane + 64u * c)));
    };
    // this lane's activation values k = 16 (lane + 64 c) + j, as fp32: with
    // the norm prologue from the row staged once per workgroup in LDS, else
    // read directly (the SwiGLU applied per lane). The activation loads go
    // out before the first row's weight loads, so waiting for them does not
    // wait for the weights (vector loads complete in issue order).
    uint4 wc[R][KC8];
    __shared__ uint4 sx[PRO == kProResnorm ? K / 8u : 1u];
    constexpr uint32_t XH = PRO == kProSwiglu ? 2u : 1u;  // gate, up
    uint4 xraw[PRO == kProResnorm ? 1u : KC8][2][XH];
    if constexpr (PRO == kProResnorm) {
        stage_rows<1u, PRO, K, 64u * kF8Waves>(nullptr, 0u, a.res_in, a.addend, a.norm_w,
                                               a.res_out, 0u, a.eps, sx, [&] {
                                                   load(wc, active ? n : a.N - 1u);
                                               });
        __syncthreads();
    } else {
#pragma unroll
        for (uint32_t c = 0; c < KC8; ++c)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h)
#pragma unroll
                for (uint32_t e = 0; e < XH; ++e)
                    xraw[c][h][e] = ld16(a.x + 16u * (lane + 64u * c) + 8u * h + e * K);
        load(wc, active ? n : a.N - 1u);
    }
    if (!active) return;  // wave-uniform; no barrier follows
    float x[KC8][16];
#pragma unroll
    for (uint32_t c = 0; c < KC8; ++c)
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h) {
            uint4 t;
            if constexpr (PRO == kProResnorm) {
                t = sx[2u * (lane + 64u * c) + h];
            } else if constexpr (PRO == kProSwiglu) {
                t = swiglu8(xraw[c][h][0], xraw[c][h][1]);
            } else {
                t = xraw[c][h][0];
            }
            const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[c][8 * h + 2 * i] = lo_f(u[i]);
                x[c][8 * h + 2 * i + 1] = hi_f(u[i]);
            }
        }

    while (true) {
        const uint32_t n2 = n + stride;
        const bool more = n2 < a.N;
        uint4 wn[R][KC8];
        if (more) load(wn, n2);
        float acc[R];
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (uint32_t c = 0; c < KC8; ++c) fp8x16_fma(wc[r][c], x[c], s0, s1);
            acc[r] = wave_sum(s0 + s1);
        }
        float v = acc[0] * a.scale[n];
        if constexpr (SWI) {
            const float gt = bf16_to_f32(f32_to_bf16(v));
            const float up = bf16_to_f32(f32_to_bf16(acc[1] * a.scale[a.N + n]));
            v = silu_mul(gt, up);
        }
        if (lane == 0u) a.y[n] = f32_to_bf16(v);
        if (!more) break;
#pragma unroll
        for (uint32_t r = 0; r < R; ++r)
#pragma unroll
            for (uint32_t c = 0; c < KC8; ++c) wc[r][c] = wn[r][c];
        n = n2;
    }
}

// One wave per output row, 4 per workgroup; at most 1024 workgroups (the
// 130560-row lm_head: ~32 rows per wave, the next row's loads in flight).
template <uint32_t PRO, uint32_t KC8, bool SWI>
void launch_gemv8(const Gemv8Args& a, hipStream_t st) {
    constexpr uint32_t kF8Waves = f8_waves<PRO>();
    uint32_t blocks = (a.N + kF8Waves - 1u) / kF8Waves;
    const uint32_t cap = (a.N >= kF8WideRows ? kF8WideWaves : 4096u) / kF8Waves;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL((gemv8_kernel<PRO, KC8, SWI>), dim3(blocks), dim3(64u * kF8Waves), 0, st,
                       a);
}

// ---- greedy argmax over bf16 logits ----
// grid = rows, block = 1024. fp32 comparison, ties to the lowest index.
__device__ __forceinline__ void better(float& bv, uint32_t& bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}
// Stage 1 of the two-stage argmax: grid = (kArgSlices, rows), block 256;
// block s scans slice s of the row and writes its (value, index).
constexpr uint32_t kArgSlices = 64;
__global__ void __launch_bounds__(256)
    argmax_slices_kernel(const uint16_t* __restrict__ logits, uint32_t n,
                         float* __restrict__ stage_v, int32_t* __restrict__ stage_i) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const uint16_t* l = logits + (size_t)blockIdx.y * n;
    const uint32_t per = (n + kArgSlices - 1u) / kArgSlices;
    const uint32_t lo = blockIdx.x * per, hi = min(lo + per, n);
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = lo + threadIdx.x; i < hi; i += 256u) better(bv, bi, bf16_to_f32(l[i]), i);
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const float ov = __shfl_xor(bv, (int)off);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, (int)off);
        better(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63u) == 0u) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0u) {
        for (uint32_t w = 1; w < 4u; ++w) better(bv, bi, sv[w], si[w]);
        stage_v[blockIdx.y * kArgSlices + blockIdx.x] = bv;
        stage_i[blockIdx.y * kArgSlices + blockIdx.x] = (int32_t)bi;
    }
}

// Stage 2: grid = rows, block 64 (one slice result per lane).
__global__ void __launch_bounds__(64)
    argmax_final_kernel(const float* __restrict__ stage_v, const int32_t* __restrict__ stage_i,
                        int32_t* out_tok, int32_t* const* __restrict__ slot_tok) {
    float bv = stage_v[blockIdx.x * kArgSlices + threadIdx.x];
    uint32_t bi = (uint32_t)stage_i[blockIdx.x * kArgSlices + threadIdx.x];
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const float ov = __shfl_xor(bv, (int)off);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, (int)off);
        better(bv, bi, ov, oi);
    }
    if (threadIdx.x == 0u) {
        const int32_t tok = bi == 0xFFFFFFFFu ? 0 : (int32_t)bi;
        if (slot_tok != nullptr) *slot_tok[blockIdx.x] = tok;
        else out_tok[blockIdx.x] = tok;
    }
}

__global__ void __launch_bounds__(1024)
    argmax_kernel(const uint16_t* __restrict__ logits, uint32_t n, int32_t* out_tok,
                  int32_t* const* __restrict__ slot_tok) {
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    const uint16_t* l = logits + (size_t)blockIdx.x * n;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < n; i += 1024u) better(bv, bi, bf16_to_f32(l[i]), i);
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const float ov = __shfl_xor(bv, (int)off);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, (int)off);
        better(bv, bi, ov, oi);
    }
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0u) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0u) {
        for (uint32_t w = 1; w < 16u; ++w) better(bv, bi, sv[w], si[w]);
        // all logits NaN: report index 0, as a scan that never improves would
        const int32_t tok = bi == 0xFFFFFFFFu ? 0 : (int32_t)bi;
        if (slot_tok != nullptr) *slot_tok[blockIdx.x] = tok;
        else out_tok[blockIdx.x] = tok;
    }
}

template <uint32_t M, uint32_t PRO, uint32_t KC, bool SWI>
void launch_gemv_t(const GemvArgs& a, hipStream_t st) {
    constexpr uint32_t WV = M == 1u ? kSoloWaves : kMultiWaves;
    constexpr uint32_t cap = M == 1u ? kSoloBlocks : kMultiBlocks;
    uint32_t blocks = (a.N + WV - 1u) / WV;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL((gemv_kernel<M, PRO, KC, SWI, WV>), dim3(blocks), dim3(64u * WV), 0, st,
                       a.w, a.x, a.res_in, a.addend, a.norm_w, a.N, a.ldx, a);
}

template <uint32_t PRO, uint32_t KC, bool SWI = false>
bool launch_gemv_m(uint32_t M, const GemvArgs& a, hipStream_t st) {
    switch (M) {
        case 1: launch_gemv_t<1, PRO, KC, SWI>(a, st); return true;
        case 2: launch_gemv_t<2, PRO, KC, SWI>(a, st); return true;
        case 3: launch_gemv_t<3, PRO, KC, SWI>(a, st); return true;
        case 4: launch_gemv_t<4, PRO, KC, SWI>(a, st); return true;
        case 5: launch_gemv_t<5, PRO, KC, SWI>(a, st); return true;
        case 6: launch_gemv_t<6, PRO, KC, SWI>(a, st); return true;
        case 7: launch_gemv_t<7, PRO, KC, SWI>(a, st); return true;
        case 8: launch_gemv_t<8, PRO, KC, SWI>(a, st); return true;
        default: return false;
    }
}

// ---- row GEMM for prefill chunks of MC_MODEL_GEMM_ROWS_MIN..MAX rows ----
// y[m][n] = bf16(sum_k W[n][k] x[m][k]) (or, SWI, bf16(silu(g) * u) of the
// gate row n and up row N + n, each rounded to bf16 first, as the GEMV
// epilogue) for 9..32 activation rows. The library kernels stream the
// weights slowly at these sizes (hipBLASLt: a 32-row qkv projection in
// 12 us, 0.85 TB/s); this kernel reads each weight byte once, at 1.1-3.8
// TB/s (5.3-7.7 us for qkv, 13-18 us for gate_up + SwiGLU at 9-32 rows).
// Its activation reads grow with the rows, which bounds it above 32.
// Workgroup = 4 waves (8 for K = 6144) on one 16-row block of W (two
// with SWI: gate and up) and every activation row; the waves split K in
// slices, so a workgroup needs only 16 (32) weight rows and the grid has
// N / 16 workgroups. Per 64-element K step a wave uses its W block (lane:
// row l % 16, 16 bytes at k = 8 (l / 16) and 32 + 8 (l / 16): the A operands
// of two v_mfma_f32_16x16x32_bf16), all of which it requests up front, and
// the same k range of each 16-row activation block (B operands, from L2:
// the rows are small and shared by all workgroups), 3 to 6 steps of which
// are in flight. The slice sums are added in LDS in wave order, so the result
// does not depend on timing.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <uint32_t MB, bool SWI, uint32_t KC>
__global__ void __launch_bounds__(KC == 1u ? 256u : 512u)
    gemm_rows_kernel(const uint16_t* w, const uint16_t* x, uint32_t ldx, uint16_t* y,
                     uint32_t ldy, uint32_t M, uint32_t N) {
    constexpr uint32_t WV = KC == 1u ? 4u : 8u;  // waves: K split in WV slices
    constexpr uint32_t K = 2048u * KC, KW = K / WV, NS = KW / 64u;
    constexpr uint32_t R = SWI ? 2u : 1u;
    __shared__ f32x4_t red[WV][R][MB][64];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = blockIdx.x * 16u;
    const uint32_t r16 = lane & 15u, kq = 8u * (lane >> 4);
    const uint32_t k0 = wave * KW + kq;
    // The whole weight slice of the wave is requested first (NS * 2 loads
    // per row block and lane): the small projections have few workgroups, and
    // only all of a matrix in flight at once covers the memory latency.
    uint4 wa[NS][R][2];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
        const uint16_t* wr = w + (size_t)(n0 + r * N + r16) * K + k0;
#pragma unroll
        for (uint32_t st = 0; st < NS; ++st)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) wa[st][r][h] = ld16(wr + 64u * st + 32u * h);
    }
    // activation rows past M read row M - 1 (never stored); XD steps of them
    // in flight (each step waits for one L2 round trip otherwise)
    constexpr uint32_t XD0 = 96u / (8u * MB), XD = XD0 < NS ? XD0 : NS;
    const uint16_t* xr[MB];
#pragma unroll
    for (uint32_t b = 0; b < MB; ++b) xr[b] = x + (size_t)min(16u * b + r16, M - 1u) * ldx + k0;
    uint4 xb[XD][MB][2];
    auto load_x = [&](uint32_t st, uint32_t slot) {
#pragma unroll
        for (uint32_t b = 0; b < MB; ++b)
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) xb[slot][b][h] = ld16(xr[b] + 64u * st + 32u * h);
    };
#pragma unroll
    for (uint32_t st = 0; st + 1u < XD; ++st) load_x(st, st);
    __builtin_amdgcn_sched_barrier(0);
    f32x4_t acc[R][MB];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r)
#pragma unroll
        for (uint32_t b = 0; b < MB; ++b) acc[r][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t st = 0; st < NS; ++st) {
        const uint32_t cur = st % XD;
        if (st + XD - 1u < NS) load_x(st + XD - 1u, (st + XD - 1u) % XD);
#pragma unroll
        for (uint32_t h = 0; h < 2u; ++h)
#pragma unroll
            for (uint32_t r = 0; r < R; ++r)
#pragma unroll
                for (uint32_t b = 0; b < MB; ++b)
                    acc[r][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, wa[st][r][h]),
                        __builtin_bit_cast(bf16x8_t, xb[cur][b][h]), acc[r][b], 0, 0, 0);
    }
#pragma unroll
    for (uint32_t r = 0; r < R; ++r)
#pragma unroll
        for (uint32_t b = 0; b < MB; ++b) red[wave][r][b][lane] = acc[r][b];
    __syncthreads();
    if (wave >= MB) return;  // wave b writes activation block b
    const uint32_t b = wave;
    const uint32_t m = 16u * b + r16;  // D layout: lane -> column m, rows 4 (l / 16) + j
    f32x4_t t[R];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
        t[r] = red[0][r][b][lane];
#pragma unroll
        for (uint32_t v = 1; v < WV; ++v) t[r] += red[v][r][b][lane];  // wave order
    }
    if (m >= M) return;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if constexpr (SWI) {
            const float g = bf16_to_f32(f32_to_bf16(t[0][j]));
            const float u = bf16_to_f32(f32_to_bf16(t[1][j]));
            v[j] = silu_mul(g, u);
        } else {
            v[j] = t[0][j];
        }
    }
    *reinterpret_cast<uint2*>(y + (size_t)m * ldy + n0 + 4u * (lane >> 4)) =
        make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
}

template <bool SWI, uint32_t KC>
void launch_gemm_rows(const uint16_t* w, const uint16_t* x, uint32_t ldx, uint16_t* y,
                      uint32_t ldy, uint32_t M, uint32_t N, hipStream_t st) {
    const dim3 grid(N / 16u), block(KC == 1u ? 256u : 512u);
    if (M <= 16u)
        hipLaunchKernelGGL((gemm_rows_kernel<1, SWI, KC>), grid, block, 0, st, w, x, ldx, y, ldy,
                           M, N);
    else
        hipLaunchKernelGGL((gemm_rows_kernel<2, SWI, KC>), grid, block, 0, st, w, x, ldx, y, ldy,
                           M, N);
}

}  // namespace
}  // namespace mckv

using namespace mckv;

extern "C" mc_status_t mc_model_embedding_gather(const uint16_t* d_table, const int32_t* d_ids,
                                                 const int32_t* const* d_slot_tok,
                                                 uint16_t* d_out, uint32_t hidden,
                                                 uint32_t rows, void* stream) {
    TraceRange trace_range("mc_model_embedding_gather");
    if (d_table == nullptr || d_out == nullptr || (d_ids == nullptr) == (d_slot_tok == nullptr) ||
        hidden == 0u || hidden % 8u != 0u || rows == 0u) {
        set_error("mc_model_embedding_gather: invalid args (hidden=%u rows=%u, exactly one of "
                  "ids / slot_tok must be given)",
                  hidden, rows);
        return MC_E_INVALID_ARGUMENT;
    }
    hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, d_table,
                       d_ids, d_slot_tok, d_out, hidden);
    return check_launch("embedding gather launch failed");
}

extern "C" mc_status_t mc_model_rmsnorm_rows(uint16_t* d_res, const uint16_t* d_add,
                                             const uint16_t* d_weight, uint16_t* d_out,
                                             uint32_t rows, uint32_t n, float eps,
                                             void* stream) {
    TraceRange trace_range("mc_model_rmsnorm_rows");
    if (d_res == nullptr || d_weight == nullptr || d_out == nullptr || rows == 0u || n == 0u ||
        n % 8u != 0u || !(eps >= 0.f)) {
        set_error("mc_model_rmsnorm_rows: invalid args (rows=%u n=%u eps=%g)", rows, n,
                  (double)eps);
        return MC_E_INVALID_ARGUMENT;
    }
    hipLaunchKernelGGL(resnorm_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, d_res,
                       d_add, d_weight, d_out, n, eps);
    return check_launch("rmsnorm launch failed");
}

extern "C" mc_status_t mc_model_swiglu_rows(const uint16_t* d_src, uint16_t* d_out,
                                            uint32_t rows, uint32_t inter, void* stream) {
    TraceRange trace_range("mc_model_swiglu_rows");
    if (d_src == nullptr || d_out == nullptr || rows == 0u || inter == 0u || inter % 8u != 0u ||
        rows > 65535u) {
        set_error("mc_model_swiglu_rows: invalid args (rows=%u inter=%u)", rows, inter);
        return MC_E_INVALID_ARGUMENT;
    }
    const uint32_t bx = (inter / 8u + kThreads - 1u) / kThreads;
    hipLaunchKernelGGL(swiglu_kernel, dim3(bx, rows), dim3(kThreads), 0, (hipStream_t)stream,
                       d_src, d_out, inter);
    return check_launch("swiglu launch failed");
}

extern "C" mc_status_t mc_model_gemv(const uint16_t* d_w, const uint16_t* d_x, uint32_t ldx,
                                     uint16_t* d_y, uint32_t ldy, uint32_t M, uint32_t N,
                                     uint32_t K, void* stream) {
    TraceRange trace_range("mc_model_gemv");
    if (d_w == nullptr || d_x == nullptr || d_y == nullptr || M == 0u || M > kMaxRows ||
        N == 0u || (K != 2048u && K != 6144u) || ldx < K || ldy < N) {
        set_error("mc_model_gemv: invalid args (M=%u N=%u K=%u ldx=%u ldy=%u; M 1..%u, "
                  "K 2048 or 6144)",
                  M, N, K, ldx, ldy, kMaxRows);
        return MC_E_INVALID_ARGUMENT;
    }
    GemvArgs a{};
    a.w = d_w;
    a.N = N;
    a.x = d_x;
    a.ldx = ldx;
    a.y = d_y;
    a.ldy = ldy;
    const bool ok = K == 2048u ? launch_gemv_m<kProNone, 4>(M, a, (hipStream_t)stream)
                               : launch_gemv_m<kProNone, 12>(M, a, (hipStream_t)stream);
    (void)ok;
    return check_launch("gemv launch failed");
}

extern "C" mc_status_t mc_model_gemv_resnorm(const uint16_t* d_w, const uint16_t* d_res_in,
                                             const uint16_t* d_add, const uint16_t* d_norm_w,
                                             uint16_t* d_res_out, uint32_t ldr, uint16_t* d_y,
                                             uint32_t ldy, uint32_t M, uint32_t N, float eps,
                                             void* stream) {
    TraceRange trace_range("mc_model_gemv_resnorm");
    if (d_w == nullptr || d_res_in == nullptr || d_norm_w == nullptr || d_y == nullptr ||
        M == 0u || M > kMaxRows || N == 0u || ldr < 2048u || ldy < N || !(eps >= 0.f) ||
        (d_res_out != nullptr && (d_res_out == d_res_in || d_res_out == d_add))) {
        set_error("mc_model_gemv_resnorm: invalid args (M=%u N=%u ldr=%u ldy=%u; the residual "
                  "output must not alias its inputs)",
                  M, N, ldr, ldy);
        return MC_E_INVALID_ARGUMENT;
    }
    GemvArgs a{};
    a.w = d_w;
    a.N = N;
    a.res_in = d_res_in;
    a.addend = d_add;
    a.norm_w = d_norm_w;
    a.res_out = d_res_out;
    a.ldr = ldr;
    a.eps = eps;
    a.y = d_y;
    a.ldy = ldy;
    launch_gemv_m<kProResnorm, 4>(M, a, (hipStream_t)stream);
    return check_launch("gemv (residual + rmsnorm prologue) launch failed");
}

extern "C" mc_status_t mc_model_gemv_resnorm_swiglu(
    const uint16_t* d_w, const uint16_t* d_res_in, const uint16_t* d_add,
    const uint16_t* d_norm_w, uint16_t* d_res_out, uint32_t ldr, uint16_t* d_y, uint32_t ldy,
    uint32_t M, uint32_t I, float eps, void* stream) {
    TraceRange trace_range("mc_model_gemv_resnorm_swiglu");
    if (d_w == nullptr || d_res_in == nullptr || d_norm_w == nullptr || d_y == nullptr ||
        M == 0u || M > kMaxRows || I == 0u || ldr < 2048u || ldy < I || !(eps >= 0.f) ||
        (d_res_out != nullptr && (d_res_out == d_res_in || d_res_out == d_add))) {
        set_error("mc_model_gemv_resnorm_swiglu: invalid args (M=%u I=%u ldr=%u ldy=%u; the "
                  "residual output must not alias its inputs)",
                  M, I, ldr, ldy);
        return MC_E_INVALID_ARGUMENT;
    }
    GemvArgs a{};
    a.w = d_w;
    a.N = I;
    a.res_in = d_res_in;
    a.addend = d_add;
    a.norm_w = d_norm_w;
    a.res_out = d_res_out;
    a.ldr = ldr;
    a.eps = eps;
    a.y = d_y;
    a.ldy = ldy;
    launch_gemv_m<kProResnorm, 4, true>(M, a, (hipStream_t)stream);
    return check_launch("gemv (residual + rmsnorm prologue, swiglu epilogue) launch failed");
}

extern "C" mc_status_t mc_model_gemv_swiglu(const uint16_t* d_w, const uint16_t* d_gate_up,
                                            uint32_t ldx, uint16_t* d_y, uint32_t ldy,
                                            uint32_t M, uint32_t N, uint32_t K, void* stream) {
    TraceRange trace_range("mc_model_gemv_swiglu");
    if (d_w == nullptr || d_gate_up == nullptr || d_y == nullptr || M == 0u || M > kMaxRows ||
        N == 0u || (K != 2048u && K != 6144u) || ldx < 2u * K || ldy < N) {
        set_error("mc_model_gemv_swiglu: invalid args (M=%u N=%u K=%u ldx=%u ldy=%u)", M, N, K,
                  ldx, ldy);
        return MC_E_INVALID_ARGUMENT;
    }
    GemvArgs a{};
    a.w = d_w;
    a.N = N;
    a.x = d_gate_up;
    a.ldx = ldx;
    a.y = d_y;
    a.ldy = ldy;
    if (K == 2048u) launch_gemv_m<kProSwiglu, 4>(M, a, (hipStream_t)stream);
    else launch_gemv_m<kProSwiglu, 12>(M, a, (hipStream_t)stream);
    return check_launch("gemv (swiglu prologue) launch failed");
}

extern "C" mc_status_t mc_model_argmax_bf16(const uint16_t* d_logits, uint32_t n,
                                            uint32_t rows, int32_t* d_out,
                                            int32_t* const* d_slot_tok, float* d_stage_v,
                                            int32_t* d_stage_i, void* stream) {
    TraceRange trace_range("mc_model_argmax_bf16");
    if (d_logits == nullptr || n == 0u || rows == 0u || rows > 65535u ||
        (d_out == nullptr) == (d_slot_tok == nullptr) ||
        (d_stage_v == nullptr) != (d_stage_i == nullptr)) {
        set_error("mc_model_argmax_bf16: invalid args (n=%u rows=%u, exactly one of out / "
                  "slot_tok must be given, stage buffers both or neither)",
                  n, rows);
        return MC_E_INVALID_ARGUMENT;
    }
    hipStream_t st = (hipStream_t)stream;
    if (d_stage_v == nullptr) {
        hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, st, d_logits, n, d_out,
                           d_slot_tok);
    } else {
        hipLaunchKernelGGL(argmax_slices_kernel, dim3(kArgSlices, rows), dim3(256), 0, st,
                           d_logits, n, d_stage_v, d_stage_i);
        hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, st, d_stage_v, d_stage_i,
                           d_out, d_slot_tok);
    }
    return check_launch("argmax launch failed");
}

extern "C" mc_status_t mc_model_gemv_fp8(const uint8_t* d_w, const float* d_scale,
                                         const uint16_t* d_x, uint16_t* d_y, uint32_t N,
                                         uint32_t K, void* stream) {
    TraceRange trace_range("mc_model_gemv_fp8");
    if (d_w == nullptr || d_scale == nullptr || d_x == nullptr || d_y == nullptr || N == 0u ||
        (K != 2048u && K != 6144u) || ((uintptr_t)d_w & 15u) != 0u) {
        set_error("mc_model_gemv_fp8: invalid args (N=%u K=%u; K 2048 or 6144, weights "
                  "16-byte aligned)",
                  N, K);
        return MC_E_INVALID_ARGUMENT;
    }
    Gemv8Args a{};
    a.w = d_w;
    a.scale = d_scale;
    a.N = N;
    a.x = d_x;
    a.y = d_y;
    if (K == 2048u) launch_gemv8<kProNone, 2, false>(a, (hipStream_t)stream);
    else launch_gemv8<kProNone, 6, false>(a, (hipStream_t)stream);
    return check_launch("fp8 gemv launch failed");
}

extern "C" mc_status_t mc_model_gemv_fp8_swiglu(const uint8_t* d_w, const float* d_scale,
                                                const uint16_t* d_gate_up, uint16_t* d_y,
                                                uint32_t N, uint32_t K, void* stream) {
    TraceRange trace_range("mc_model_gemv_fp8_swiglu");
    if (d_w == nullptr || d_scale == nullptr || d_gate_up == nullptr || d_y == nullptr ||
        N == 0u || (K != 2048u && K != 6144u) || ((uintptr_t)d_w & 15u) != 0u) {
        set_error("mc_model_gemv_fp8_swiglu: invalid args (N=%u K=%u)", N, K);
        return MC_E_INVALID_ARGUMENT;
    }
    Gemv8Args a{};
    a.w = d_w;
    a.scale = d_scale;
    a.N = N;
    a.x = d_gate_up;
    a.y = d_y;
    if (K == 2048u) launch_gemv8<kProSwiglu, 2, false>(a, (hipStream_t)stream);
    else launch_gemv8<kProSwiglu, 6, false>(a, (hipStream_t)stream);
    return check_launch("fp8 gemv (swiglu prologue) launch failed");
}

extern "C" mc_status_t mc_model_gemv_fp8_resnorm(const uint8_t* d_w, const float* d_scale,
                                                 const uint16_t* d_res_in,
                                                 const uint16_t* d_add,
                                                 const uint16_t* d_norm_w,
                                                 uint16_t* d_res_out, uint16_t* d_y,
                                                 uint32_t N, float eps, void* stream) {
    TraceRange trace_range("mc_model_gemv_fp8_resnorm");
    if (d_w == nullptr || d_scale == nullptr || d_res_in == nullptr || d_norm_w == nullptr ||
        d_y == nullptr || N == 0u || !(eps >= 0.f) || ((uintptr_t)d_w & 15u) != 0u ||
        (d_res_out != nullptr && (d_res_out == d_res_in || d_res_out == d_add))) {
        set_error("mc_model_gemv_fp8_resnorm: invalid args (N=%u eps=%g; res_out must not "
                  "alias res_in or add)",
                  N, (double)eps);
        return MC_E_INVALID_ARGUMENT;
    }
    Gemv8Args a{};
    a.w = d_w;
    a.scale = d_scale;
    a.N = N;
    a.res_in = d_res_in;
    a.addend = d_add;
    a.norm_w = d_norm_w;
    a.res_out = d_res_out;
    a.eps = eps;
    a.y = d_y;
    launch_gemv8<kProResnorm, 2, false>(a, (hipStream_t)stream);
    return check_launch("fp8 gemv (norm prologue) launch failed");
}

extern "C" mc_status_t mc_model_gemv_fp8_resnorm_swiglu(
    const uint8_t* d_w, const float* d_scale, const uint16_t* d_res_in, const uint16_t* d_add,
    const uint16_t* d_norm_w, uint16_t* d_res_out, uint16_t* d_y, uint32_t I, float eps,
    void* stream) {
    TraceRange trace_range("mc_model_gemv_fp8_resnorm_swiglu");
    if (d_w == nullptr || d_scale == nullptr || d_res_in == nullptr || d_norm_w == nullptr ||
        d_y == nullptr || I == 0u || !(eps >= 0.f) || ((uintptr_t)d_w & 15u) != 0u ||
        (d_res_out != nullptr && (d_res_out == d_res_in || d_res_out == d_add))) {
        set_error("mc_model_gemv_fp8_resnorm_swiglu: invalid args (I=%u eps=%g)", I,
                  (double)eps);
        return MC_E_INVALID_ARGUMENT;
    }
    Gemv8Args a{};
    a.w = d_w;
    a.scale = d_scale;
    a.N = I;
    a.res_in = d_res_in;
    a.addend = d_add;
    a.norm_w = d_norm_w;
    a.res_out = d_res_out;
    a.eps = eps;
    a.y = d_y;
    launch_gemv8<kProResnorm, 2, true>(a, (hipStream_t)stream);
    return check_launch("fp8 gemv (norm prologue, swiglu epilogue) launch failed");
}

extern "C" mc_status_t mc_model_gemm_rows(const uint16_t* d_w, const uint16_t* d_x, uint32_t ldx,
                                          uint16_t* d_y, uint32_t ldy, uint32_t M, uint32_t N,
                                          uint32_t K, uint32_t swiglu, void* stream) {
    TraceRange trace_range("mc_model_gemm_rows");
    if (d_w == nullptr || d_x == nullptr || d_y == nullptr || M < MC_MODEL_GEMM_ROWS_MIN ||
        M > MC_MODEL_GEMM_ROWS_MAX || N == 0u || N % 16u != 0u || (K != 2048u && K != 6144u) ||
        swiglu > 1u || (swiglu && K != 2048u) || ldx < K || ldy < N || ldx % 8u != 0u ||
        ldy % 4u != 0u || (reinterpret_cast<uintptr_t>(d_w) | reinterpret_cast<uintptr_t>(d_x)) % 16u ||
        reinterpret_cast<uintptr_t>(d_y) % 8u) {
        set_error("mc_model_gemm_rows: invalid args (M=%u N=%u K=%u ldx=%u ldy=%u swiglu=%u; M "
                  "%u..%u, N a multiple of 16, K 2048 or 6144 (2048 with swiglu), ldx a "
                  "multiple of 8 and ldy of 4, w and x 16-byte and y 8-byte aligned)",
                  M, N, K, ldx, ldy, swiglu, MC_MODEL_GEMM_ROWS_MIN, MC_MODEL_GEMM_ROWS_MAX);
        return MC_E_INVALID_ARGUMENT;
    }
    hipStream_t st = (hipStream_t)stream;
    if (swiglu) {
        launch_gemm_rows<true, 1>(d_w, d_x, ldx, d_y, ldy, M, N, st);
    } else {
        if (K == 2048u) launch_gemm_rows<false, 1>(d_w, d_x, ldx, d_y, ldy, M, N, st);
        else launch_gemm_rows<false, 3>(d_w, d_x, ldx, d_y, ldy, M, N, st);
    }
    return check_launch("row GEMM launch failed");
}
