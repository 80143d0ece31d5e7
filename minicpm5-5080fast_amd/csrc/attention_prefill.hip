// attention_prefill.hip - causal attention of a prefill chunk over the paged
// KV cache (page gather + flash attention), with optional key splits.
//
// Contract of the reference path (native/kernels/sm120/attention_prefill.cu:
// 291-729, kernels.h:517-521,575-585):
//   * query row t (t < T) has absolute position base_pos + t, base_pos =
//     *d_base_pos, and attends pool positions 0..base_pos + t through the page
//     table (causal mask pos > base_pos + t -> -inf);
//   * keys are streamed in 16-position tiles; the tiles needed by a 16-row q
//     tile are 0..(base_pos + last row) >> 4; with S_kv key splits, split s
//     takes tiles [s*qsp, min(s*qsp + qsp - 1, last)], qsp = ceil(ntiles/S_kv);
//   * online softmax per 16-position tile (p fp32 for l, bf16 for P.V), a fully
//     masked tile leaves the state unchanged;
//   * S_kv == 1 writes out[t*2048 + qh*128 + d] = bf16(acc/l); S_kv > 1 writes
//     partial {m, l, acc} at partials[((t*16 + qh)*S_kv + s)*130] and a merge
//     kernel (block per (t, qh)) folds the S_kv partials in ascending order.
//
// MI355X design: one 256-thread workgroup (4 wave64) per (kv head, 16-row q
// tile, key split). The 16 rows x 8 query heads of a KV head form 128 query
// vectors; wave w owns rows 4w..4w+3 as two 16-column groups (column n =
// head n%8 of row 4w + 2*group + n/8), so every MFMA column is a real query.
// The key tile is gathered once per workgroup into LDS (double buffered, two
// 16-byte global loads per thread); each wave then computes
// S^T = K x Q^T (v_mfma_f32_16x16x32_bf16), the online softmax per column,
// transposes V with an identity MFMA and accumulates O^T += V^T x P^T
// (v_mfma_f32_16x16x16bf16_1k), the same operand scheme as the decode kernel.
#include <hip/hip_runtime.h>

#include <cmath>

#include "error.h"
#include "kv_common.h"
#include "kv_internal.h"

namespace mckv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kThreads = 256;
constexpr uint32_t kPitch = 136;  // LDS row pitch (bf16) of a 128-dim row

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& u) {
    return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ s16x4 as_s16x4(const uint2& u) {
    return __builtin_bit_cast(s16x4, u);
}
__device__ __forceinline__ s16x4 trunc_bf16x4(const f32x4& t) {
    uint2 r;
    r.x = (__float_as_uint(t[0]) >> 16) | (__float_as_uint(t[1]) & 0xFFFF0000u);
    r.y = (__float_as_uint(t[2]) >> 16) | (__float_as_uint(t[3]) & 0xFFFF0000u);
    return __builtin_bit_cast(s16x4, r);
}

__global__ void __launch_bounds__(kThreads) prefill_attn_kernel(
    const uint16_t* __restrict__ q_rows, uint32_t T,
    const uint32_t* __restrict__ d_base_pos, uint32_t layer,
    const uint32_t* __restrict__ pt, const uint16_t* __restrict__ pool, DevLayout ly,
    uint16_t* __restrict__ out, float* __restrict__ partials, uint32_t S) {
    __shared__ __align__(16) uint16_t sK[2][16 * kPitch];
    __shared__ __align__(16) uint16_t sV[2][16 * kPitch];

    const uint32_t ntq = (T + 15u) / 16u;
    const uint32_t s = blockIdx.x % S;
    const uint32_t qt = (blockIdx.x / S) % ntq;
    const uint32_t kvh = (blockIdx.x / S) / ntq;
    const uint32_t tb = qt * 16u;
    const uint32_t base_pos = *d_base_pos;
    const uint32_t key_end = base_pos + tb + min(15u, T - 1u - tb);  // last key
    const uint32_t last = key_end >> 4;
    const uint32_t qsp = (last + S) / S;  // ceil((last+1)/S)
    const uint32_t jt0 = s * qsp;
    const uint32_t jt1 = min(jt0 + qsp - 1u, last);

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t col = lane & 15u;
    const uint32_t grp = lane >> 4;

    // Query columns: group g, column col -> head col%8, row 4*wave + 2g + col/8.
    uint32_t row[2];
    bf16x8 qb[2][4];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        row[g] = tb + 4u * wave + 2u * g + (col >> 3);
        const bool ok = row[g] < T;
        const uint16_t* q =
            q_rows + (size_t)(ok ? row[g] : 0u) * kRow + (kvh * kGroup + (col & 7u)) * kD +
            8u * grp;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            qb[g][m] = as_bf16x8(ok ? *reinterpret_cast<const uint4*>(q + 32u * m)
                                    : make_uint4(0u, 0u, 0u, 0u));
    }
    s16x4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        ident[i] = (4u * grp + (uint32_t)i == col) ? (short)0x3F80 : (short)0;

    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    f32x4 acc[2][4][2];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h) acc[g][m][h] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Cooperative gather: element idx = tid + 256*r covers (pos sp, K/V, 8 dims).
    uint4 stage[2];
    auto gather = [&](uint32_t jt) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t idx = tid + 256u * r;
            const uint32_t sp = idx >> 5, w4 = idx & 31u;
            const uint32_t pos = jt * 16u + sp;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (pos <= key_end) {
                const uint32_t page = pt[pos >> ly.log2p];
                v = *reinterpret_cast<const uint4*>(
                    pool + token_base(ly, layer, page, pos & ly.pmask) +
                    (w4 >> 4) * 256u + kvh * kD + (w4 & 15u) * 8u);
            }
            stage[r] = v;
        }
    };
    auto put = [&](int b) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t idx = tid + 256u * r;
            const uint32_t sp = idx >> 5, w4 = idx & 31u;
            uint16_t* dst = ((w4 >> 4) ? sV[b] : sK[b]) + sp * kPitch + (w4 & 15u) * 8u;
            *reinterpret_cast<uint4*>(dst) = stage[r];
        }
    };

    if (jt0 <= jt1) gather(jt0);
    int b = 0;
    for (uint32_t jt = jt0; jt <= jt1; ++jt, b ^= 1) {
        put(b);
        __syncthreads();
        if (jt < jt1) gather(jt + 1u);
        const uint16_t* K = sK[b];
        const uint16_t* V = sV[b];
        // K tile as A operand: lane (pos = col, grp) holds dims 32m + 8*grp + 0..7.
        bf16x8 ka[4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
            ka[m] = as_bf16x8(*reinterpret_cast<const uint4*>(K + col * kPitch + 32u * m +
                                                              8u * grp));
        // V^T blocks via identity MFMA (shared by both column groups).
        s16x4 vt[4][2];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint2 raw = *reinterpret_cast<const uint2*>(
                    V + col * kPitch + 32u * m + 8u * grp + 4u * h);
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                vt[m][h] = trunc_bf16x4(
                    __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(as_s16x4(raw), ident, z, 0,
                                                              0, 0));
            }
        const uint32_t pos0 = jt * 16u + 4u * grp;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < 4; ++m)
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[m], qb[g][m], sacc, 0, 0,
                                                               0);
            const uint32_t lim = base_pos + row[g];
            float sc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v;
                {
#pragma clang fp contract(off)
                    v = sacc[j] * kScoreScale;
                }
                sc[j] = (pos0 + (uint32_t)j <= lim) ? v : -INFINITY;
            }
            float tm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            tm = fmaxf(tm, __shfl_xor(tm, 16));
            tm = fmaxf(tm, __shfl_xor(tm, 32));
            float mn = fmaxf(m_run[g], tm);
            const float renew = (m_run[g] == -INFINITY) ? 0.f : __expf(m_run[g] - mn);
            const float mnext = mn;
            if (mn == -INFINITY) mn = 0.f;  // fully masked so far: p = 0, state kept
            float p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = __expf(sc[j] - mn);
            float ls = (p[0] + p[1]) + (p[2] + p[3]);
            ls += __shfl_xor(ls, 16);
            ls += __shfl_xor(ls, 32);
            l_run[g] = l_run[g] * renew + ls;
            m_run[g] = mnext;
            s16x4 pb;
#pragma unroll
            for (int j = 0; j < 4; ++j) pb[j] = (short)f32_to_bf16(p[j]);
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    acc[g][m][h] = acc[g][m][h] * renew;
                    acc[g][m][h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        vt[m][h], pb, acc[g][m][h], 0, 0, 0);
                }
        }
    }

    // Epilogue: lane holds dims 32m + 8*grp + 4h + j of column (head, row).
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        if (row[g] >= T) continue;
        const uint32_t qh = kvh * kGroup + (col & 7u);
        if (S == 1u) {
            uint16_t* o = out + (size_t)row[g] * 2048u + qh * kD + 8u * grp;
            const float L = l_run[g];
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint16_t w[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        w[j] = f32_to_bf16(L > 0.f ? acc[g][m][h][j] / L : 0.f);
                    *reinterpret_cast<uint2*>(o + 32u * m + 4u * h) =
                        make_uint2((uint32_t)w[0] | ((uint32_t)w[1] << 16),
                                   (uint32_t)w[2] | ((uint32_t)w[3] << 16));
                }
        } else {
            float* pw = partials + ((size_t)(row[g] * 16u + qh) * S + s) * kPartial;
            if (grp == 0u) {
                pw[0] = m_run[g];
                pw[1] = l_run[g];
            }
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float* d = pw + 2u + 32u * m + 8u * grp + 4u * h;
                    *reinterpret_cast<float2*>(d) =
                        make_float2(acc[g][m][h][0], acc[g][m][h][1]);
                    *reinterpret_cast<float2*>(d + 2) =
                        make_float2(acc[g][m][h][2], acc[g][m][h][3]);
                }
        }
    }
}

// grid = T*16 (block = (t, qh)), block = 128 (thread = dim).
__global__ void __launch_bounds__(128) prefill_merge_kernel(
    const float* __restrict__ partials, uint32_t S, uint32_t T,
    uint16_t* __restrict__ out) {
    const uint32_t bh = blockIdx.x;
    const uint32_t t = bh >> 4;
    if (t >= T) return;
    const uint32_t d = threadIdx.x;
    const float* base = partials + (size_t)bh * S * kPartial;
    float M = -INFINITY;
    for (uint32_t i = 0; i < S; ++i) {
        const float* p = base + (size_t)i * kPartial;
        if (p[1] != 0.f) M = fmaxf(M, p[0]);
    }
    float L = 0.f, A = 0.f;
    for (uint32_t i = 0; i < S; ++i) {
        const float* p = base + (size_t)i * kPartial;
        if (p[1] == 0.f) continue;
        const float f = expf(p[0] - M);
        L += p[1] * f;
        A += p[2 + d] * f;
    }
    out[(size_t)t * 2048u + (bh & 15u) * kD + d] = f32_to_bf16(L > 0.f ? A / L : 0.f);
}

}  // namespace
}  // namespace mckv

using namespace mckv;

extern "C" mc_status_t mc_kv_attention_prefill(const uint16_t* d_q_rows, uint32_t tokens,
                                               const uint32_t* d_base_pos, uint32_t layer,
                                               const uint32_t* d_page_table,
                                               const uint16_t* d_kv_pool,
                                               mc_kv_layout_t layout, uint16_t* d_out,
                                               float* d_partials, uint32_t S_kv,
                                               void* stream) {
    DevLayout ly;
    if (d_q_rows == nullptr || d_base_pos == nullptr || d_page_table == nullptr ||
        d_kv_pool == nullptr || d_out == nullptr || tokens == 0 || S_kv == 0u ||
        S_kv > 8u || (S_kv > 1u && d_partials == nullptr) ||
        !layout_valid(layout, &ly) || layer >= layout.num_layers) {
        set_error("mc_kv_attention_prefill: invalid args (tokens=%u S_kv=%u "
                  "partials=%p)",
                  tokens, S_kv, (void*)d_partials);
        return MC_E_INVALID_ARGUMENT;
    }
    const uint32_t ntq = (tokens + 15u) / 16u;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(kHkv * ntq * S_kv), dim3(kThreads), 0,
                       st, d_q_rows, tokens, d_base_pos, layer, d_page_table, d_kv_pool,
                       ly, d_out, d_partials, S_kv);
    if (S_kv > 1u)
        hipLaunchKernelGGL(prefill_merge_kernel, dim3(tokens * 16u), dim3(128), 0, st,
                           d_partials, S_kv, tokens, d_out);
    return check_launch("prefill attention launch failed");
}
