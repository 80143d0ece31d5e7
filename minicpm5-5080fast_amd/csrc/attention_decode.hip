// attention_decode.hip - paged split-KV flash decoding for one new token per
// session (single session and batched), with the two-level partial merge.
//
// Contract of the reference path (native/kernels/sm120/attention_decode.cu:
// 966-1368 chunk kernel, 1494-1595 merge_a/merge_b, 1389-1407/1602-1626
// batched twins, 1840-1964/2120-2170 launchers):
//   * limit = *d_pos is the query position; keys/values 0..limit are attended.
//   * Work is split in chunks of chunk_pos positions; chunk c covers
//     [c*C, min(c*C+C-1, limit)]; chunks starting after limit do nothing.
//   * Scores are fp32 dot(q, k) * (1/sqrt(128) as fp32); softmax runs online in
//     16-position batches: mn = max(m, batch max), renew = exp(m - mn) (0 when
//     m = -inf), p = exp(score - mn) in fp32 feeds l, and p rounded to bf16
//     (RNE) feeds the P.V product.
//   * A chunk writes the partial {m, l, acc[128]} at
//     partials[(qh*max_chunks + c)*130]; when limit < C (single chunk) it writes
//     out[qh*128 + d] = bf16(acc/l) directly instead.
//   * merge_a: n_valid = min(limit/C + 1, max_chunks), nothing when 1; block
//     (qh, s) folds chunks c = s mod 32 (ascending, skipping l == 0) into level-2
//     partial s, an empty split (s >= n_valid) stores {-inf, 0}. merge_b folds
//     the 32 level-2 partials and writes bf16(A/L).
//   * Phase0 (inv_freq != NULL): the block owning position `limit` rotates that
//     token's k from the qkv row, writes K and V of `limit` to the pool and uses
//     the fresh values; q is rotated in registers and never written back.
//
// MI355X design (one 256-thread workgroup = 4 wave64 per (slot, kv head,
// chunk)). Each wave walks 16-position tiles t = wave, wave+4, ... of its chunk
// and keeps its own online-softmax state for all 8 query heads of the KV head;
// the 4 wave states are folded through LDS at the end. Per tile a lane
// (token = lane%16, group = lane/16) issues eight 16-byte global loads: K and V
// dims [32m + 8*group, +8) for m = 0..3 of its token, i.e. each instruction
// reads 64 contiguous bytes of 16 rows; the next tile's loads are in flight
// while the current tile computes.
//   * QK: S^T[16 pos][16 heads] = K (A operand, exactly the loaded registers)
//     x Q^T (B operand, preloaded; heads 8..15 are zero padding) with four
//     v_mfma_f32_16x16x32_bf16.
//   * The D layout gives each lane 4 positions of one head; the batch max/sum
//     need two cross-lane xor steps (16, 32).
//   * P.V needs V with positions along the contraction, but the loaded V has
//     dims along lanes. Multiplying the loaded 16x16 V block by an identity
//     B operand (v_mfma_f32_16x16x16bf16_1k) transposes it exactly (every D
//     element is one bf16 value times 1.0); the truncated result is the A
//     operand of O^T += V^T x P^T, whose B operand (P^T) is the softmax output
//     already in the right lanes. acc ends up as 32 fp32 per lane: head
//     lane%16, dims [32m + 8*group, +8) - the dims the lane loaded.
// Arithmetic intensity is ~8 flop/byte, so the kernel is HBM-bound; MFMA keeps
// the VALU free for addressing and softmax.
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
constexpr uint32_t kWaves = 4;
constexpr uint32_t kTile = 16;

struct Tile {
    uint4 k[4];
    uint4 v[4];
};

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& u) {
    return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ s16x4 half_s16x4(const uint4& u, int h) {
    const uint2 x = h ? make_uint2(u.z, u.w) : make_uint2(u.x, u.y);
    return __builtin_bit_cast(s16x4, x);
}
// fp32 -> bf16 by truncation; exact for values that are bf16 already.
__device__ __forceinline__ s16x4 trunc_bf16x4(const f32x4& t) {
    uint2 r;
    r.x = (__float_as_uint(t[0]) >> 16) | (__float_as_uint(t[1]) & 0xFFFF0000u);
    r.y = (__float_as_uint(t[2]) >> 16) | (__float_as_uint(t[3]) & 0xFFFF0000u);
    return __builtin_bit_cast(s16x4, r);
}

struct DecodeArgs {
    const uint16_t* q_row;  // [2560] of this slot
    uint32_t limit;
    const uint32_t* pt;
    uint16_t* pool;
    float* partials;  // this slot: [16][NC][130]
    uint16_t* out;    // this slot: [2048]
};

template <bool PH0>
__device__ __forceinline__ void decode_chunk_body(const DecodeArgs a, uint32_t layer,
                                                  DevLayout ly, uint32_t NC,
                                                  const float* __restrict__ inv_freq,
                                                  uint32_t C, uint32_t kvh,
                                                  uint32_t chunk) {
    __shared__ float s_cs[64], s_sn[64];
    __shared__ float s_m[kWaves][kGroup], s_l[kWaves][kGroup];
    __shared__ __align__(16) float s_acc[kWaves][kGroup][kD];

    const uint32_t limit = a.limit;
    const uint32_t start = chunk * C;
    if (start > limit) return;  // uniform over the block
    const uint32_t end = min(start + C - 1u, limit);
    const uint32_t ntiles = (end - start) / kTile + 1u;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63u;
    const uint32_t tok = lane & 15u;  // row within a 16-position tile / head col
    const uint32_t grp = lane >> 4;   // 0..3

    const uint16_t* __restrict__ q_row = a.q_row;
    const uint32_t* __restrict__ pt = a.pt;
    uint16_t* __restrict__ pool = a.pool;
    const uint32_t kvcol = kvh * kD + 8u * grp;  // within a token's K or V half

    // Fresh K/V of position `limit` (phase0): this lane's 4x8 dims.
    auto fresh_kv = [&](Tile& T) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            T.k[m] = *reinterpret_cast<const uint4*>(q_row + kKCol + kvcol + 32u * m);
            T.v[m] = *reinterpret_cast<const uint4*>(q_row + kVCol + kvcol + 32u * m);
        }
    };
    auto load_tile = [&](Tile& T, uint32_t t) {
        const uint32_t p = min(start + t * kTile + tok, end);
        if (PH0 && p == limit) {
            fresh_kv(T);  // rotated below, after the cos/sin table exists
            return;
        }
        const uint32_t page = pt[p >> ly.log2p];
        const uint16_t* src = pool + token_base(ly, layer, page, p & ly.pmask) + kvcol;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            T.k[m] = *reinterpret_cast<const uint4*>(src + 32u * m);
            T.v[m] = *reinterpret_cast<const uint4*>(src + 256u + 32u * m);
        }
    };

    Tile cur;
    uint32_t t = wave;
    if (t < ntiles) load_tile(cur, t);

    if (PH0) {
        if (tid < 64u) {
            float c, s;
            rope_sincos((float)limit * inv_freq[tid], &c, &s);
            s_cs[tid] = c;
            s_sn[tid] = s;
        }
        __syncthreads();
    }

    // Rotates the k half of a fresh tile in place and stores K/V of `limit`.
    auto finish_fresh = [&](Tile& T, uint32_t tt) {
        if (!PH0) return;
        const uint32_t p = min(start + tt * kTile + tok, end);
        if (p != limit) return;
        uint4 rk[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint16_t* x = reinterpret_cast<const uint16_t*>(&T.k[m]);
            const uint16_t* x2 = reinterpret_cast<const uint16_t*>(&T.k[m ^ 2]);
            uint16_t* o = reinterpret_cast<uint16_t*>(&rk[m]);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t pr = 32u * (m & 1) + 8u * grp + i;
                o[i] = f32_to_bf16(rope_rotate(bf16_to_f32(x[i]), bf16_to_f32(x2[i]),
                                               s_cs[pr], s_sn[pr], m < 2));
            }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) T.k[m] = rk[m];
        if (start + tt * kTile + tok == limit) {  // the real row writes the pool
            const uint32_t page = pt[limit >> ly.log2p];
            uint16_t* dst =
                pool + token_base(ly, layer, page, limit & ly.pmask) + kvcol;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                *reinterpret_cast<uint4*>(dst + 32u * m) = T.k[m];
                *reinterpret_cast<uint4*>(dst + 256u + 32u * m) = T.v[m];
            }
        }
    };

    // Q^T B operand: lane holds q[head = tok][32m + 8*grp + i]; heads >= 8 zero.
    bf16x8 qb[4];
    {
        uint4 qr[4];
        const bool real = tok < kGroup;
        const uint16_t* qsrc = q_row + (kvh * kGroup + (real ? tok : 0u)) * kD + 8u * grp;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            qr[m] = real ? *reinterpret_cast<const uint4*>(qsrc + 32u * m)
                         : make_uint4(0u, 0u, 0u, 0u);
        if (PH0 && real) {
            uint4 rq[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint16_t* x = reinterpret_cast<const uint16_t*>(&qr[m]);
                const uint16_t* x2 = reinterpret_cast<const uint16_t*>(&qr[m ^ 2]);
                uint16_t* o = reinterpret_cast<uint16_t*>(&rq[m]);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t pr = 32u * (m & 1) + 8u * grp + i;
                    o[i] = f32_to_bf16(rope_rotate(bf16_to_f32(x[i]),
                                                   bf16_to_f32(x2[i]), s_cs[pr],
                                                   s_sn[pr], m < 2));
                }
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) qr[m] = rq[m];
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) qb[m] = as_bf16x8(qr[m]);
    }

    // Identity B operand for the transpose: B[k][c] = (k == c), k = 4*grp + i.
    s16x4 ident;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        ident[i] = (4u * grp + (uint32_t)i == tok) ? (short)0x3F80 : (short)0;

    float m_run = -INFINITY, l_run = 0.f;
    f32x4 acc[4][2];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[m][h] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (; t < ntiles; t += kWaves) {
        const bool has_next = t + kWaves < ntiles;
        Tile nxt;
        if (has_next) load_tile(nxt, t + kWaves);
        finish_fresh(cur, t);

        // S^T = K x Q^T
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m)
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(cur.k[m]), qb[m], s,
                                                        0, 0, 0);
        const uint32_t pos0 = start + t * kTile + 4u * grp;
        float sc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v;
            {
#pragma clang fp contract(off)
                v = s[j] * kScoreScale;
            }
            sc[j] = (pos0 + (uint32_t)j <= end) ? v : -INFINITY;
        }
        float tm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float mn = fmaxf(m_run, tm);
        const float renew = (m_run == -INFINITY) ? 0.f : __expf(m_run - mn);
        float p[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = __expf(sc[j] - mn);
        float ls = (p[0] + p[1]) + (p[2] + p[3]);
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        l_run = l_run * renew + ls;
        m_run = mn;
        s16x4 pb;
#pragma unroll
        for (int j = 0; j < 4; ++j) pb[j] = (short)f32_to_bf16(p[j]);

#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                const f32x4 vt = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                    half_s16x4(cur.v[m], h), ident, z, 0, 0, 0);
                acc[m][h] = acc[m][h] * renew;
                acc[m][h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                    trunc_bf16x4(vt), pb, acc[m][h], 0, 0, 0);
            }
        if (has_next) cur = nxt;
    }

    // Fold the 4 wave states (fixed wave order) through LDS.
    if (tok < kGroup) {
        if (grp == 0u) {
            s_m[wave][tok] = m_run;
            s_l[wave][tok] = l_run;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                *reinterpret_cast<f32x4*>(&s_acc[wave][tok][32u * m + 8u * grp + 4u * h]) =
                    acc[m][h];
    }
    __syncthreads();
    const uint32_t head = tid >> 5;         // 0..7
    const uint32_t d4 = (tid & 31u) * 4u;   // 4 dims
    float M = -INFINITY;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w)
        if (s_l[w][head] != 0.f) M = fmaxf(M, s_m[w][head]);
    float L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) {
        const float lw = s_l[w][head];
        if (lw == 0.f) continue;
        const float f = __expf(s_m[w][head] - M);
        L += lw * f;
        A += *reinterpret_cast<const f32x4*>(&s_acc[w][head][d4]) * f;
    }
    const uint32_t qh = kvh * kGroup + head;
    if (limit < C) {
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f32_to_bf16(L > 0.f ? A[i] / L : 0.f);
        *reinterpret_cast<uint2*>(a.out + qh * kD + d4) =
            make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16),
                       (uint32_t)o[2] | ((uint32_t)o[3] << 16));
    } else {
        float* pw = a.partials + ((size_t)qh * NC + chunk) * kPartial;
        if (d4 == 0u) {
            pw[0] = M;
            pw[1] = L;
        }
        *reinterpret_cast<float2*>(pw + 2 + d4) = make_float2(A[0], A[1]);
        *reinterpret_cast<float2*>(pw + 4 + d4) = make_float2(A[2], A[3]);
    }
}

// grid = (NC, 2 kv heads, B slots). Single-session launches pass B = 1 and the
// direct pointers; batched launches resolve per-slot pointers from tables.
template <bool PH0, bool BATCH>
__global__ void __launch_bounds__(kThreads) decode_chunk_kernel(
    const uint16_t* __restrict__ q_rows, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t layer,
    const uint32_t* pt, const uint32_t* const* __restrict__ slot_pt,
    uint16_t* pool, uint16_t* const* __restrict__ slot_kv, DevLayout ly,
    float* __restrict__ partials, uint32_t NC, uint16_t* __restrict__ out,
    const float* __restrict__ inv_freq, uint32_t C) {
    const uint32_t slot = blockIdx.z;
    DecodeArgs a;
    a.q_row = q_rows + (size_t)slot * kRow;
    a.limit = BATCH ? *slot_pos[slot] : *d_pos;
    a.pt = BATCH ? slot_pt[slot] : pt;
    a.pool = BATCH ? slot_kv[slot] : pool;
    a.partials = partials + (size_t)slot * kHq * NC * kPartial;
    a.out = out + (size_t)slot * kHq * kD;
    decode_chunk_body<PH0>(a, layer, ly, NC, inv_freq, C, blockIdx.y, blockIdx.x);
}

__device__ __forceinline__ uint32_t n_valid_chunks(uint32_t limit, uint32_t C,
                                                   uint32_t NC) {
    const uint32_t n = limit / C + 1u;
    return n > NC ? NC : n;
}

// Level-1 -> level-2 merge. grid = (B*16, 32), block = 128 (thread = dim).
template <bool BATCH>
__global__ void __launch_bounds__(128) merge_a_kernel(
    const float* __restrict__ partials, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NC, uint32_t C,
    float* __restrict__ partials2) {
    const uint32_t slot = blockIdx.x >> 4, qh = blockIdx.x & 15u, s = blockIdx.y;
    const uint32_t d = threadIdx.x;
    const uint32_t limit = BATCH ? *slot_pos[slot] : *d_pos;
    const uint32_t nv = n_valid_chunks(limit, C, NC);
    if (nv == 1u) return;
    const float* P = partials + ((size_t)slot * kHq + qh) * NC * kPartial;
    float* pw2 = partials2 + (((size_t)slot * kHq + qh) * kSplit2 + s) * kPartial;
    if (s >= nv) {
        if (d == 0u) {
            pw2[0] = -INFINITY;
            pw2[1] = 0.f;
        }
        return;
    }
    float mloc = -INFINITY;
    for (uint32_t c = s; c < nv; c += kSplit2) {
        const float* p = P + (size_t)c * kPartial;
        if (p[1] != 0.f) mloc = fmaxf(mloc, p[0]);
    }
    float L = 0.f, A = 0.f;
    for (uint32_t c = s; c < nv; c += kSplit2) {
        const float* p = P + (size_t)c * kPartial;
        if (p[1] == 0.f) continue;
        const float f = expf(p[0] - mloc);
        L += p[1] * f;
        A += p[2 + d] * f;
    }
    if (d == 0u) {
        pw2[0] = mloc;
        pw2[1] = L;
    }
    pw2[2 + d] = A;
}

// Fold of `n` partials with stride kPartial (fixed ascending order) -> bf16.
__device__ __forceinline__ void fold_to_out(const float* __restrict__ P, uint32_t n,
                                            uint32_t d, uint16_t* __restrict__ o) {
    float M = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) {
        const float* p = P + (size_t)i * kPartial;
        if (p[1] != 0.f) M = fmaxf(M, p[0]);
    }
    float L = 0.f, A = 0.f;
    for (uint32_t i = 0; i < n; ++i) {
        const float* p = P + (size_t)i * kPartial;
        if (p[1] == 0.f) continue;
        const float f = expf(p[0] - M);
        L += p[1] * f;
        A += p[2 + d] * f;
    }
    *o = f32_to_bf16(L > 0.f ? A / L : 0.f);
}

// Level-2 -> out. grid = B*16, block = 128.
template <bool BATCH>
__global__ void __launch_bounds__(128) merge_b_kernel(
    const float* __restrict__ partials2, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NC, uint32_t C,
    uint16_t* __restrict__ out) {
    const uint32_t slot = blockIdx.x >> 4, qh = blockIdx.x & 15u;
    const uint32_t limit = BATCH ? *slot_pos[slot] : *d_pos;
    if (n_valid_chunks(limit, C, NC) == 1u) return;
    fold_to_out(partials2 + ((size_t)slot * kHq + qh) * kSplit2 * kPartial, kSplit2,
                threadIdx.x, out + ((size_t)slot * kHq + qh) * kD + threadIdx.x);
}

// One-level merge of all valid level-1 partials (used when no level-2 buffer
// is given). grid = B*16, block = 128.
template <bool BATCH>
__global__ void __launch_bounds__(128) merge_p_kernel(
    const float* __restrict__ partials, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NC, uint32_t C,
    uint16_t* __restrict__ out) {
    const uint32_t slot = blockIdx.x >> 4, qh = blockIdx.x & 15u;
    const uint32_t limit = BATCH ? *slot_pos[slot] : *d_pos;
    const uint32_t nv = n_valid_chunks(limit, C, NC);
    if (nv == 1u) return;
    fold_to_out(partials + ((size_t)slot * kHq + qh) * NC * kPartial, nv, threadIdx.x,
                out + ((size_t)slot * kHq + qh) * kD + threadIdx.x);
}

template <bool BATCH>
mc_status_t launch_chunks(const uint16_t* q, const uint32_t* d_pos,
                          const uint32_t* const* slot_pos, uint32_t B, uint32_t layer,
                          const uint32_t* pt, const uint32_t* const* slot_pt,
                          uint16_t* pool, uint16_t* const* slot_kv, DevLayout ly,
                          float* partials, uint32_t NC, uint16_t* out,
                          hipStream_t st, const float* inv_freq, uint32_t C) {
    const dim3 grid(NC, kHkv, B);
    if (inv_freq != nullptr)
        hipLaunchKernelGGL((decode_chunk_kernel<true, BATCH>), grid, dim3(kThreads), 0,
                           st, q, d_pos, slot_pos, layer, pt, slot_pt, pool, slot_kv, ly,
                           partials, NC, out, inv_freq, C);
    else
        hipLaunchKernelGGL((decode_chunk_kernel<false, BATCH>), grid, dim3(kThreads),
                           0, st, q, d_pos, slot_pos, layer, pt, slot_pt, pool, slot_kv,
                           ly, partials, NC, out, inv_freq, C);
    return check_launch("decode attention chunk launch failed");
}

template <bool BATCH>
mc_status_t launch_merge(const float* partials, const uint32_t* d_pos,
                         const uint32_t* const* slot_pos, uint32_t B, uint32_t NC,
                         uint32_t C, float* partials2, uint16_t* out, hipStream_t st) {
    if (partials2 != nullptr) {
        hipLaunchKernelGGL((merge_a_kernel<BATCH>), dim3(B * kHq, kSplit2), dim3(128), 0,
                           st, partials, d_pos, slot_pos, NC, C, partials2);
        hipLaunchKernelGGL((merge_b_kernel<BATCH>), dim3(B * kHq), dim3(128), 0, st,
                           partials2, d_pos, slot_pos, NC, C, out);
    } else {
        hipLaunchKernelGGL((merge_p_kernel<BATCH>), dim3(B * kHq), dim3(128), 0, st,
                           partials, d_pos, slot_pos, NC, C, out);
    }
    return check_launch("decode attention merge launch failed");
}

bool chunk_args_ok(uint32_t max_chunks, uint32_t chunk_pos) {
    return max_chunks > 0 && max_chunks <= 65535u && chunk_pos >= 16u &&
           chunk_pos % 16u == 0u;
}

}  // namespace
}  // namespace mckv

using namespace mckv;

extern "C" mc_status_t mc_kv_attention_decode_chunks(
    const uint16_t* d_q_rows, const uint32_t* d_pos, uint32_t layer,
    const uint32_t* d_page_table, uint16_t* d_kv_pool, mc_kv_layout_t layout,
    float* d_partials, uint32_t max_chunks, uint16_t* d_out, void* stream,
    const float* d_inv_freq, uint32_t chunk_pos) {
    DevLayout ly;
    if (d_q_rows == nullptr || d_pos == nullptr || d_page_table == nullptr ||
        d_kv_pool == nullptr || d_partials == nullptr || d_out == nullptr ||
        !layout_valid(layout, &ly) || layer >= layout.num_layers ||
        !chunk_args_ok(max_chunks, chunk_pos)) {
        set_error("mc_kv_attention_decode: invalid args (layer=%u max_chunks=%u "
                  "chunk_pos=%u)",
                  layer, max_chunks, chunk_pos);
        return MC_E_INVALID_ARGUMENT;
    }
    return launch_chunks<false>(d_q_rows, d_pos, nullptr, 1, layer, d_page_table,
                                nullptr, d_kv_pool, nullptr, ly, d_partials, max_chunks,
                                d_out, (hipStream_t)stream, d_inv_freq, chunk_pos);
}

extern "C" mc_status_t mc_kv_attention_decode(
    const uint16_t* d_q_rows, const uint32_t* d_pos, uint32_t layer,
    const uint32_t* d_page_table, uint16_t* d_kv_pool, mc_kv_layout_t layout,
    float* d_partials, uint32_t max_chunks, uint16_t* d_out, void* stream,
    const float* d_inv_freq, uint32_t chunk_pos, float* d_partials2) {
    const mc_status_t st = mc_kv_attention_decode_chunks(
        d_q_rows, d_pos, layer, d_page_table, d_kv_pool, layout, d_partials,
        max_chunks, d_out, stream, d_inv_freq, chunk_pos);
    if (st != MC_OK) return st;
    return launch_merge<false>(d_partials, d_pos, nullptr, 1, max_chunks, chunk_pos,
                               d_partials2, d_out, (hipStream_t)stream);
}

extern "C" mc_status_t mc_kv_attention_decode_merge(
    const float* d_partials, const uint32_t* d_pos, uint32_t max_chunks,
    uint32_t chunk_pos, float* d_partials2, uint16_t* d_out, void* stream) {
    if (d_partials == nullptr || d_pos == nullptr || d_out == nullptr ||
        !chunk_args_ok(max_chunks, chunk_pos)) {
        set_error("mc_kv_attention_decode_merge: invalid args (max_chunks=%u "
                  "chunk_pos=%u)",
                  max_chunks, chunk_pos);
        return MC_E_INVALID_ARGUMENT;
    }
    return launch_merge<false>(d_partials, d_pos, nullptr, 1, max_chunks, chunk_pos,
                               d_partials2, d_out, (hipStream_t)stream);
}

extern "C" mc_status_t mc_kv_attention_decode_batch(
    const uint16_t* d_q_rows, const uint32_t* const* d_slot_pos, uint32_t B,
    uint32_t layer, const uint32_t* const* d_slot_pt, uint16_t* const* d_slot_kv,
    mc_kv_layout_t layout, float* d_partials, uint32_t max_chunks, uint16_t* d_out,
    void* stream, const float* d_inv_freq, uint32_t chunk_pos, float* d_partials2) {
    DevLayout ly;
    if (d_q_rows == nullptr || d_slot_pos == nullptr || d_slot_pt == nullptr ||
        d_slot_kv == nullptr || d_partials == nullptr || d_out == nullptr || B == 0 ||
        B > 64u || !layout_valid(layout, &ly) || layer >= layout.num_layers ||
        !chunk_args_ok(max_chunks, chunk_pos)) {
        set_error("mc_kv_attention_decode_batch: invalid args (B=%u layer=%u "
                  "max_chunks=%u chunk_pos=%u)",
                  B, layer, max_chunks, chunk_pos);
        return MC_E_INVALID_ARGUMENT;
    }
    const mc_status_t st = launch_chunks<true>(
        d_q_rows, nullptr, d_slot_pos, B, layer, nullptr, d_slot_pt, nullptr, d_slot_kv,
        ly, d_partials, max_chunks, d_out, (hipStream_t)stream, d_inv_freq, chunk_pos);
    if (st != MC_OK) return st;
    return launch_merge<true>(d_partials, nullptr, d_slot_pos, B, max_chunks, chunk_pos,
                              d_partials2, d_out, (hipStream_t)stream);
}
