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
// and the 64 lane sums are combined by a fixed butterfly.
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

// K = 512 * KC (16-byte chunks per lane per row); WV waves per workgroup,
// one output column per wave at a time. kProResnorm needs K = 2048.
// SWI: SwiGLU epilogue. Output column n (n < a.N) takes the weight rows n
// (gate) and a.N + n (up) of a [2 a.N][K] matrix: y = bf16(silu(g) * u) with
// g, u the two dot products rounded to bf16 first (the projection's output
// rounding), as a gate_up projection followed by the SwiGLU kernel.
template <uint32_t M, uint32_t PRO, uint32_t KC, bool SWI, uint32_t WV>
__global__ void __launch_bounds__(64u * WV) gemv_kernel(const GemvArgs a) {
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
    if (active) load(wc, n, g);

    // Stage the activation rows (after the prologue) into LDS.
    if constexpr (PRO == kProResnorm) {
        // Item i = 256 m + c is the 16-byte chunk c of row m; a row's 256
        // items are four whole waves, so each wave sums one row's part and
        // all M rows' sums of squares come out of one workgroup barrier.
        constexpr uint32_t IT = (M * 256u + T - 1u) / T;
        __shared__ float s_part[M][4];
        uint4 v[IT];
#pragma unroll
        for (uint32_t it = 0; it < IT; ++it) {
            const uint32_t i = tid + it * T;
            if (i >= M * 256u) break;  // wave-uniform
            const uint32_t m = i >> 8, c = i & 255u;
            v[it] = ld16(a.res_in + (size_t)m * a.ldr + 8u * c);
            if (a.addend != nullptr) {
                const uint4 d = ld16(a.addend + (size_t)m * a.ldr + 8u * c);
                v[it].x = pack2(lo_f(v[it].x) + lo_f(d.x), hi_f(v[it].x) + hi_f(d.x));
                v[it].y = pack2(lo_f(v[it].y) + lo_f(d.y), hi_f(v[it].y) + hi_f(d.y));
                v[it].z = pack2(lo_f(v[it].z) + lo_f(d.z), hi_f(v[it].z) + hi_f(d.z));
                v[it].w = pack2(lo_f(v[it].w) + lo_f(d.w), hi_f(v[it].w) + hi_f(d.w));
            }
            if (a.res_out != nullptr && blockIdx.x == 0u)
                *reinterpret_cast<uint4*>(a.res_out + (size_t)m * a.ldr + 8u * c) = v[it];
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
            const uint4 g = ld16(a.norm_w + 8u * c);
            const float tot = ((s_part[m][0] + s_part[m][1]) + s_part[m][2]) + s_part[m][3];
            const float inv = 1.0f / sqrtf(tot / (float)K + a.eps);
            uint4 o;
            o.x = pack2(lo_f(v[it].x) * inv * lo_f(g.x), hi_f(v[it].x) * inv * hi_f(g.x));
            o.y = pack2(lo_f(v[it].y) * inv * lo_f(g.y), hi_f(v[it].y) * inv * hi_f(g.y));
            o.z = pack2(lo_f(v[it].z) * inv * lo_f(g.z), hi_f(v[it].z) * inv * hi_f(g.z));
            o.w = pack2(lo_f(v[it].w) * inv * lo_f(g.w), hi_f(v[it].w) * inv * hi_f(g.w));
            sx[m * NCH + c] = o;
        }
    } else {
        for (uint32_t i = tid; i < M * NCH; i += T) {
            const uint32_t m = i / NCH, c = i % NCH;
            const uint16_t* xr = a.x + (size_t)m * a.ldx + 8u * c;
            if constexpr (PRO == kProSwiglu) sx[i] = swiglu8(ld16(xr), ld16(xr + K));
            else sx[i] = ld16(xr);
        }
    }
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
#pragma unroll
            for (uint32_t m = 0; m < M; ++m) {
                float v = wave_sum(acc[0][m]);
                if constexpr (SWI) {
                    const float gt = bf16_to_f32(f32_to_bf16(v));
                    const float up = bf16_to_f32(f32_to_bf16(wave_sum(acc[1][m])));
                    v = silu_mul(gt, up);
                }
                if (lane == m) a.y[(size_t)m * a.ldy + n] = f32_to_bf16(v);
#pragma unroll
                for (uint32_t r = 0; r < R; ++r) acc[r][m] = 0.f;
            }
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
                       a);
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
