// attention_decode.hip - host side of the paged split-KV flash decoding
// (single session and batched) and the stand-alone merge kernels.
//
// The decode kernels themselves live in decode_kernels.h (instantiated in
// decode_bf16p.hip and decode_fp32p.hip). This file holds:
//   * the reference's two-level merge of per-chunk partials (merge_a: split
//     s folds chunks c = s mod 32 ascending, skipping l == 0, into level-2
//     partial s; an empty split stores {-inf, 0}; merge_b folds the 32
//     level-2 partials; merge_p the one-level fold) - native/kernels/sm120/
//     attention_decode.cu:1494-1595, 1602-1626;
//   * the launch policy: the chunk kernel writes one record per workgroup
//     range, merge_r_kernel folds them (the reference's merges serve the
//     stand-alone merge entry point and more than 256 records per head);
//   * the extern "C" entry points of include/mc_kv.h.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <mutex>

#include "decode_kernels.h"
#include "error.h"
#include "trace.h"
#include "kv_common.h"
#include "kv_internal.h"

namespace mckv {
namespace {

constexpr uint32_t kMaxFold = 2048;

// Folds n partials {m, l, acc[128]} at base + i*stride (i ascending) with the
// reference merge rule: M = max m over l != 0; f_i = exp(m_i - M);
// L = sum l_i f_i; A[d] = sum acc_i[d] f_i (ascending, l == 0 skipped). The
// (m, l) pairs are loaded by all threads at once and the acc loads are
// independent, so the fold costs a few memory latencies instead of n.
// Block = 128 threads, thread = dim. Returns A for dim threadIdx.x; M, L
// through references. n <= kMaxFold.
__device__ __forceinline__ float fold_partials(const float* __restrict__ base,
                                               size_t stride, uint32_t n, float& M_out,
                                               float& L_out) {
    __shared__ float s_m[kMaxFold], s_l[kMaxFold], s_red[4];
    const uint32_t d = threadIdx.x;
    float mx = -INFINITY;
    for (uint32_t i = d; i < n; i += 128u) {
        const float2 ml = *reinterpret_cast<const float2*>(base + i * stride);
        s_m[i] = ml.x;
        s_l[i] = ml.y;
        if (ml.y != 0.f) mx = fmaxf(mx, ml.x);
    }
    mx = wave_max(mx);
    if ((d & 63u) == 0u) s_red[d >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(s_red[0], s_red[1]);
    for (uint32_t i = d; i < n; i += 128u)
        s_m[i] = (s_l[i] != 0.f) ? expf(s_m[i] - M) : 0.f;  // s_m now holds f_i
    __syncthreads();
    // Branch-free accumulation: every load is issued unconditionally (the
    // select keeps an l == 0 partial, whatever its acc holds, out of the sum),
    // so 16 loads are in flight at once.
    float L = 0.f, A = 0.f;
#pragma unroll 16
    for (uint32_t i = 0; i < n; ++i) {
        const float v = base[i * stride + 2u + d];
        const float f = s_m[i];
        const bool live = s_l[i] != 0.f;
        L += live ? s_l[i] * f : 0.f;
        A += live ? v * f : 0.f;
    }
    M_out = M;
    L_out = L;
    return A;
}

// Folds of at most NMAX <= 128 partials in ONE memory round, split in two
// steps so that the loads can be issued before the decode limit is known:
// load_partials reads `nload` partials (everything the buffer holds for this
// fold; never more than it holds), fold_loaded then keeps the first n of
// them. Same arithmetic and order as fold_partials (bit-identical results).
// Block = 128 threads, thread = dim.
template <uint32_t NMAX>
struct Loaded {
    float v[NMAX];  // acc[d] of partial i
    float m, l;     // (m, l) of partial threadIdx.x
};

template <uint32_t NMAX>
__device__ __forceinline__ void load_partials(const float* __restrict__ base, size_t stride,
                                              uint32_t nload, Loaded<NMAX>& x) {
    static_assert(NMAX <= 128u, "one (m, l) pair per thread");
    const uint32_t d = threadIdx.x;
#pragma unroll
    for (uint32_t i = 0; i < NMAX; ++i)  // past nload: a repeated (never kept) load
        x.v[i] = base[(i < nload ? i : nload - 1u) * stride + 2u + d];
    const uint32_t di = d < nload ? d : nload - 1u;
    const float2 ml = *reinterpret_cast<const float2*>(base + di * stride);
    x.m = ml.x;
    x.l = ml.y;
}

template <uint32_t NMAX>
__device__ __forceinline__ float fold_loaded(const Loaded<NMAX>& x, uint32_t n, float& M_out,
                                             float& L_out) {
    __shared__ float s_f[NMAX], s_l[NMAX], s_red[2];
    const uint32_t d = threadIdx.x;
    const float m = x.m;
    const float l = d < n ? x.l : 0.f;
    float mx = (l != 0.f) ? m : -INFINITY;
    mx = wave_max(mx);
    if ((d & 63u) == 0u) s_red[d >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(s_red[0], s_red[1]);
    if (d < NMAX) {
        s_f[d] = (l != 0.f) ? expf(m - M) : 0.f;
        s_l[d] = l;
    }
    __syncthreads();
    float L = 0.f, A = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < NMAX; ++i) {
        const float f = s_f[i];
        const bool live = s_l[i] != 0.f;
        L += live ? s_l[i] * f : 0.f;
        A += live ? x.v[i] * f : 0.f;
    }
    M_out = M;
    L_out = L;
    return A;
}

// Level-1 -> level-2 merge. grid = (B*16, 32), block = 128 (thread = dim).
// NMAX >= ceil(NC / 32). Single session: the partial loads are issued before
// the limit is read; no block returns early (stores are predicated), so the
// compiler cannot sink the loads behind the limit.
template <bool BATCH, uint32_t NMAX>
__global__ void __launch_bounds__(128) merge_a_kernel(
    const float* __restrict__ partials, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NC, uint32_t C,
    float* __restrict__ partials2) {
    const uint32_t slot = blockIdx.x >> 4, qh = blockIdx.x & 15u, s = blockIdx.y;
    const uint32_t d = threadIdx.x;
    const float* P = partials + (((size_t)slot * kHq + qh) * NC + s) * kPartial;
    Loaded<NMAX> x;
    uint32_t nv, n;
    if constexpr (BATCH) {
        // Ragged slots: read the limit first and load only the valid chunks
        // (a short slot would otherwise pull its whole stale buffer).
        nv = n_valid_chunks(*slot_pos[slot], C, NC);
        n = s < nv ? (nv - s + kSplit2 - 1u) / kSplit2 : 0u;
        load_partials<NMAX>(P, (size_t)kSplit2 * kPartial, n > 0u ? n : 1u, x);
    } else {
        load_partials<NMAX>(P, (size_t)kSplit2 * kPartial, (NC - s + kSplit2 - 1u) / kSplit2,
                            x);
        nv = n_valid_chunks(*d_pos, C, NC);
        n = s < nv ? (nv - s + kSplit2 - 1u) / kSplit2 : 0u;
    }
    float M, L;
    const float A = fold_loaded<NMAX>(x, n, M, L);
    float* pw2 = partials2 + (((size_t)slot * kHq + qh) * kSplit2 + s) * kPartial;
    if (nv > 1u) {
        if (d == 0u) {  // an empty split (s >= nv) stores {-inf, 0}
            pw2[0] = M;
            pw2[1] = L;
        }
        if (s < nv) pw2[2 + d] = A;
    }
}

// Level-2 -> out. grid = B*16, block = 128.
template <bool BATCH>
__global__ void __launch_bounds__(128) merge_b_kernel(
    const float* __restrict__ partials2, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NC, uint32_t C,
    uint16_t* __restrict__ out, unsigned long long* stamps) {
    const WgStamp stamp(stamps, 2u, kTlMergeWgs, false);
    const uint32_t slot = blockIdx.x >> 4, qh = blockIdx.x & 15u;
    Loaded<kSplit2> x;
    const float* base = partials2 + ((size_t)slot * kHq + qh) * kSplit2 * kPartial;
    // The 32 rows lie inside the caller's buffer for every slot, so they are
    // loaded before the limit (an inactive slot's rows are never used).
    load_partials<kSplit2>(base, kPartial, kSplit2, x);
    const bool active = n_valid_chunks(BATCH ? *slot_pos[slot] : *d_pos, C, NC) > 1u;
    float M, L;
    const float A = fold_loaded<kSplit2>(x, kSplit2, M, L);
    if (active)
        out[((size_t)slot * kHq + qh) * kD + threadIdx.x] = f32_to_bf16(L > 0.f ? A / L : 0.f);
}

// One-level merge of all valid level-1 partials (used when no level-2 buffer
// is given, or when NC <= 32). grid = B*16, block = 128. NMAX >= NC selects
// the one-round fold (loads before the limit, as in merge_a); 0 the generic
// fold over up to kMaxFold partials.
template <bool BATCH, uint32_t NMAX>
__global__ void __launch_bounds__(128) merge_p_kernel(
    const float* __restrict__ partials, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NC, uint32_t C,
    uint16_t* __restrict__ out, unsigned long long* stamps) {
    const WgStamp stamp(stamps, 2u, kTlMergeWgs, false);
    const uint32_t slot = blockIdx.x >> 4, qh = blockIdx.x & 15u;
    const float* base = partials + ((size_t)slot * kHq + qh) * NC * kPartial;
    float M, L, A;
    bool active;
    if constexpr (NMAX > 0u) {
        Loaded<NMAX> x;
        uint32_t nv;
        if constexpr (BATCH) {
            // loads after the limit: measured faster for the batched launch
            nv = n_valid_chunks(*slot_pos[slot], C, NC);
            load_partials<NMAX>(base, kPartial, nv, x);
        } else {
            load_partials<NMAX>(base, kPartial, NC, x);
            nv = n_valid_chunks(*d_pos, C, NC);
        }
        active = nv > 1u;
        A = fold_loaded<NMAX>(x, nv, M, L);
    } else {
        const uint32_t limit = BATCH ? *slot_pos[slot] : *d_pos;
        const uint32_t nv = n_valid_chunks(limit, C, NC);
        if (nv == 1u) return;
        active = true;
        A = fold_partials(base, kPartial, nv, M, L);
    }
    if (active)
        out[((size_t)slot * kHq + qh) * kD + threadIdx.x] = f32_to_bf16(L > 0.f ? A / L : 0.f);
}

template <bool BATCH>
mc_status_t launch_merge(const float* partials, const uint32_t* d_pos,
                         const uint32_t* const* slot_pos, uint32_t B, uint32_t NC,
                         uint32_t C, float* partials2, uint16_t* out, hipStream_t st,
                         unsigned long long* stamps) {
    // With at most 32 chunks every level-2 split holds one chunk, merge_a would
    // copy it exactly (m, l * 1, acc * 1), and merge_b's ascending fold equals
    // the one-level fold: a single kernel gives the identical result.
    if (partials2 != nullptr && NC > kSplit2) {
        const dim3 ga(B * kHq, kSplit2);
        static_assert(kMaxFold <= 64u * kSplit2, "merge_a folds at most 64 per split");
        if (NC <= 16u * kSplit2)
            hipLaunchKernelGGL((merge_a_kernel<BATCH, 16u>), ga, dim3(128), 0, st, partials,
                               d_pos, slot_pos, NC, C, partials2);
        else
            hipLaunchKernelGGL((merge_a_kernel<BATCH, 64u>), ga, dim3(128), 0, st, partials,
                               d_pos, slot_pos, NC, C, partials2);
        hipLaunchKernelGGL((merge_b_kernel<BATCH>), dim3(B * kHq), dim3(128), 0, st,
                           partials2, d_pos, slot_pos, NC, C, out, stamps);
    } else if (NC <= kSplit2) {
        hipLaunchKernelGGL((merge_p_kernel<BATCH, kSplit2>), dim3(B * kHq), dim3(128), 0, st,
                           partials, d_pos, slot_pos, NC, C, out, stamps);
    } else {
        hipLaunchKernelGGL((merge_p_kernel<BATCH, 0u>), dim3(B * kHq), dim3(128), 0, st,
                           partials, d_pos, slot_pos, NC, C, out, stamps);
    }
    return check_launch("decode attention merge launch failed");
}


// Fold of the decode records (split layout) of one (slot, query head,
// slice of 4Q dims) per 256-thread block: record lane rl = t / Q (of
// 256 / Q lanes) holds records rl + k * lanes, k < RPT, dim quad q = t % Q
// dims 4q..4q+3 of the slice. Every record slot of the buffer is loaded
// before the limit arrives (they all lie in the caller's buffer; the ones
// past the limit's record count are masked), so the fold costs one memory
// round. M = max m over records with l != 0, f = exp(m - M); each lane sums
// l f and acc f over its records in k order, then the lanes are combined by
// a fixed tree (xor-shuffles within a wave, then waves 0..3 in order), so
// the result is deterministic and the same for batched and single launches.
// out = bf16(A / L). grid = (16 * 32 / Q slices, B slots).
template <bool BATCH, uint32_t Q, uint32_t RPT>
__global__ void __launch_bounds__(256) merge_r_kernel(
    const float* rec, const uint32_t* d_pos,
    const uint32_t* const* __restrict__ slot_pos, uint32_t NR, uint32_t C_rng,
    uint32_t pos_max, uint16_t* __restrict__ out, unsigned long long* stamps) {
    const WgStamp stamp(stamps, 2u, kTlMergeWgs, false);
    static_assert(Q == 1u || Q == 2u || Q == 4u || Q == 8u, "dim quads per block");
    constexpr uint32_t kSlices = 32u / Q;  // blocks per head
    constexpr uint32_t kLanes = 256u / Q;
    __shared__ float s_mx[4];
    __shared__ float s_sum[4][Q][5];
    const uint32_t t = threadIdx.x, wave = t >> 6;
    const uint32_t slot = blockIdx.y;
    const uint32_t head = blockIdx.x / kSlices;
    const uint32_t q = t % Q, rl = t / Q;
    const uint32_t d = (blockIdx.x % kSlices) * 4u * Q + 4u * q;
    // Split layout: the head's acc rows [NR][128], then its {m, l} pairs.
    const float* hb = rec + ((size_t)slot * kHq + head) * NR * kPartial;
    const float* hml = hb + (size_t)NR * kD;
    // Record group k of this lane: records rl + k * kLanes. Single sessions
    // request every group before the limit (one memory round; a long context
    // uses them all). Batched slots are ragged and often far shorter than the
    // buffer (C5: ~2.4 of 17 MB valid), so they request the first group with
    // the limit and the others only where the limit says they exist.
    constexpr uint32_t K0 = BATCH ? 1u : RPT;
    float2 ml[RPT], a01[RPT], a23[RPT];
    auto load_group = [&](uint32_t k) {
        const uint32_t r = min(rl + k * kLanes, NR - 1u);
        ml[k] = *reinterpret_cast<const float2*>(hml + 2u * r);
        a01[k] = *reinterpret_cast<const float2*>(hb + (size_t)r * kD + d);  // 8-byte aligned
        a23[k] = *reinterpret_cast<const float2*>(hb + (size_t)r * kD + d + 2);
    };
#pragma unroll
    for (uint32_t k = 0; k < K0; ++k) load_group(k);
    const uint32_t limit_raw = BATCH ? *slot_pos[slot] : *d_pos;
    // The record loads above stay ahead of the limit test (rec is not
    // restrict-qualified, so they are ordinary reads that the compiler may not
    // sink below this clobber): one memory round for records and limit.
    asm volatile("" ::: "memory");
    const uint32_t limit = min(limit_raw, pos_max);  // as the chunk kernel
    const uint32_t nr = n_valid_chunks(limit, C_rng, NR);
    if (nr <= 1u) return;  // the chunk kernel wrote the output directly (uniform)
#pragma unroll
    for (uint32_t k = K0; k < RPT; ++k) {
        if (k * kLanes < nr) {  // uniform over the block
            load_group(k);
        } else {  // no record of this group exists; never read below
            ml[k] = make_float2(0.f, 0.f);
            a01[k] = a23[k] = make_float2(0.f, 0.f);
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t k = 0; k < RPT; ++k)
        if (rl + k * kLanes < nr && ml[k].y != 0.f) mx = fmaxf(mx, ml[k].x);
    mx = wave_max(mx);
    if ((t & 63u) == 0u) s_mx[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3]));
    float L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t k = 0; k < RPT; ++k) {
        if (rl + k * kLanes < nr && ml[k].y != 0.f) {
            const float f = expf(ml[k].x - M);
            L += ml[k].y * f;
            A += f32x4{a01[k].x, a01[k].y, a23[k].x, a23[k].y} * f;
        }
    }
#pragma unroll
    for (uint32_t x = Q; x < 64u; x <<= 1) {
        L += __shfl_xor(L, (int)x);
#pragma unroll
        for (int k = 0; k < 4; ++k) A[k] += __shfl_xor(A[k], (int)x);
    }
    if ((t & 63u) < Q) {
        s_sum[wave][q][0] = L;
#pragma unroll
        for (int k = 0; k < 4; ++k) s_sum[wave][q][1 + k] = A[k];
    }
    __syncthreads();
    if (t < Q) {
        float Lt = 0.f;
        f32x4 At = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t w = 0; w < 4u; ++w) {
            Lt += s_sum[w][t][0];
#pragma unroll
            for (int k = 0; k < 4; ++k) At[k] += s_sum[w][t][1 + k];
        }
        uint16_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = f32_to_bf16(Lt > 0.f ? At[k] / Lt : 0.f);
        *reinterpret_cast<uint2*>(out + ((size_t)slot * kHq + head) * kD + d) =
            make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16),
                       (uint32_t)o[2] | ((uint32_t)o[3] << 16));
    }
}

// Block shape of the record merge: 8 dim quads (32 dims, whole 128-byte
// lines of a record per lane) and 32 record lanes with RPT = ceil(NR / 32)
// records each; 64 blocks per slot. Measured at C4 (256 records per head):
// merge span 2.8 us against 3.4 / 3.0 / 4.2 us for 64 / 128 / 256 record
// lanes per block (more blocks, fewer records per lane).
template <bool BATCH>
void launch_merge_r(const ChunkLaunch& L, uint32_t NR) {
    const uint32_t Q = 8u, lanes = 32u;
    const uint32_t rpt = (NR + lanes - 1u) / lanes;
    const dim3 grid(kHq * 32u / Q, L.B);
    const uint32_t C_rng = L.C * L.cpw, pmax = pool_pos_max(L.ly);
#define MC_MERGE_R(QQ, RR)                                                                  \
    hipLaunchKernelGGL((merge_r_kernel<BATCH, QQ, RR>), grid, dim3(256), 0, L.st, L.partials, \
                       L.d_pos, L.slot_pos, NR, C_rng, pmax, L.out, merge_stamps(L.stamps))
    if (rpt <= 1u) MC_MERGE_R(8u, 1u);
    else if (rpt <= 2u) MC_MERGE_R(8u, 2u);
    else if (rpt <= 4u) MC_MERGE_R(8u, 4u);
    else MC_MERGE_R(8u, 8u);
#undef MC_MERGE_R
}

bool chunk_args_ok(uint32_t max_chunks, uint32_t chunk_pos) {
    return max_chunks > 0 && max_chunks <= kMaxFold && chunk_pos >= 16u &&
           chunk_pos % 16u == 0u;
}

// Chunks per workgroup range: enough ranges for ~512 workgroups (2 per CU on
// 256 CUs) for one session whose context fills all NC chunks, and at most
// kMaxRanges ranges (the fused merge folds up to that many records per
// head). The slot count is deliberately left out: batched limits are ragged
// and read on the device, and sizing for B full sessions would give a long
// session a few very long workgroups. cpw > 1 needs C % 64 == 0 (all 4 waves
// then cross chunk boundaries together).
uint32_t chunks_per_range(uint32_t NC, uint32_t C) {
    if (C % 64u != 0u) return 1u;
    return NC > kMaxRanges ? (NC + kMaxRanges - 1u) / kMaxRanges : 1u;
}

// P.V precision: 0 = bf16 P (default), 1 = fp32 P; kFromEnv = read
// MC_ATTN_HMMA_OFF once, like the reference (kernels.h:355-367: set ->
// the fp32-P SIMT kernel). Process-wide and static across launches, so a
// captured graph replays the kernel it was captured with.
constexpr uint32_t kFromEnv = 0xFFFFFFFFu;
std::atomic<uint32_t> g_fp32p{kFromEnv};
bool fp32p_on() {
    uint32_t v = g_fp32p.load(std::memory_order_relaxed);
    if (v == kFromEnv) {
        static const bool env = std::getenv("MC_ATTN_HMMA_OFF") != nullptr;
        v = env ? 1u : 0u;
    }
    return v != 0u;
}
// Measurement switch (debug hook): decode launches stop after the chunk
// kernel, so its time can be taken alone in the production configuration.
std::atomic<uint32_t> g_records_only{0u};

// Debug timeline buffer: run_decode gives each decode the next of `launches`
// regions of kTlWordsPerLaunch words, in a ring (mc_kv_debug_decode_timeline).
// A captured graph keeps the regions it was captured with.
std::mutex g_tl_mu;
unsigned long long* g_tl_buf = nullptr;
uint32_t g_tl_launches = 0u, g_tl_next = 0u;
static_assert(kTlWordsPerLaunch == MC_KV_TIMELINE_WORDS, "timeline region size in mc_kv.h");
unsigned long long* next_timeline_region() {
    std::lock_guard<std::mutex> lk(g_tl_mu);
    if (g_tl_buf == nullptr) return nullptr;
    unsigned long long* r = g_tl_buf + (size_t)g_tl_next * kTlWordsPerLaunch;
    g_tl_next = (g_tl_next + 1u) % g_tl_launches;
    return r;
}

// Runs one decode: the chunk kernel writes one record per (range, query
// head), or the output when the context fits one range; a merge kernel folds
// the records: merge_p for at most 32 records per head, merge_r_kernel up to
// kMaxRanges, beyond (chunk sizes that are not a multiple of 64 with more than
// 256 chunks) the reference's two-level merge when partials2 is given.
template <bool BATCH>
mc_status_t run_decode(ChunkLaunch L, float* partials2) {
    L.batched = BATCH;
    L.cpw = chunks_per_range(L.NC, L.C);
    const uint32_t nr_max = (L.NC + L.cpw - 1u) / L.cpw;
    L.rec_stride = nr_max;
    L.split = nr_max > kSplit2 && nr_max <= kMaxRanges;  // the records merge_r reads
    L.stamps = next_timeline_region();
    const mc_status_t st =
        fp32p_on() ? launch_chunk_kernel<true>(L) : launch_chunk_kernel<false>(L);
    if (st != MC_OK || g_records_only.load(std::memory_order_relaxed) != 0u) return st;
    // Records of a range count as chunks of chunk_pos * cpw positions.
    // Up to 32 records per head the reference's one-level fold (merge_p, one
    // 128-thread block per (slot, head), thread = dim) is the faster merge
    // (C3: 13.5 against 14.4 us/layer with merge_r); beyond, merge_r.
    if (nr_max > kSplit2 && nr_max <= kMaxRanges) {
        launch_merge_r<BATCH>(L, nr_max);
        return check_launch("decode attention merge launch failed");
    }
    return launch_merge<BATCH>(L.partials, L.d_pos, L.slot_pos, L.B, nr_max, L.C * L.cpw,
                               partials2, L.out, L.st, merge_stamps(L.stamps));
}

// ---- allocation-free decode: records in a library-owned device array ----
//
// mc_kv_attention_decode_noalloc keeps its records in `scratch`, a file-scope
// device array of kScratchFloats floats (16 heads x 256 records x 130 =
// 2.13 MB on every device the library runs on, held until the process ends).
// The array's name is only a host-side stand-in: the device address is taken
// once per device with hipGetSymbolAddress (device current) and that pointer
// is what the kernels receive. Every call on one device shares the array, so
// calls that overlap on a device race; the records need no clearing (a merge
// reads only the records its call wrote).
constexpr size_t kScratchFloats = (size_t)kHq * kMaxRanges * kPartial;
__device__ __align__(256) float scratch[kScratchFloats];

// Device address of `scratch` on the current device, looked up once per
// device; nullptr (error set) when the lookup fails.
float* scratch_ptr() {
    static std::mutex mu;
    static float* ptrs[64] = {};
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) {
        if (e != hipSuccess) (void)hipGetLastError();
        set_error("mc_kv_attention_decode_noalloc: no usable current device (%d)", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            set_error("mc_kv_attention_decode_noalloc: hipGetSymbolAddress(scratch) failed on "
                      "device %d: %s",
                      dev, hipGetErrorString(e));
            return nullptr;
        }
        ptrs[dev] = static_cast<float*>(p);
    }
    return ptrs[dev];
}

}  // namespace
}  // namespace mckv

using namespace mckv;

extern "C" mc_status_t mc_kv_attention_decode_noalloc(
    const uint16_t* d_q_rows, const uint32_t* d_pos, uint32_t layer,
    const uint32_t* d_page_table, uint16_t* d_kv_pool, mc_kv_layout_t layout,
    uint32_t max_chunks, uint16_t* d_out, void* stream, const float* d_inv_freq,
    uint32_t chunk_pos) {
    mckv::TraceRange trace_range("mc_kv_attention_decode_noalloc");
    DevLayout ly;
    if (d_q_rows == nullptr || d_pos == nullptr || d_page_table == nullptr ||
        d_kv_pool == nullptr || d_out == nullptr || !layout_valid(layout, &ly) ||
        layer >= layout.num_layers || !chunk_args_ok(max_chunks, chunk_pos)) {
        set_error("mc_kv_attention_decode_noalloc: invalid args (layer=%u max_chunks=%u "
                  "chunk_pos=%u)",
                  layer, max_chunks, chunk_pos);
        return MC_E_INVALID_ARGUMENT;
    }
    const uint32_t cpw = chunks_per_range(max_chunks, chunk_pos);
    const uint32_t nr = (max_chunks + cpw - 1u) / cpw;
    if (nr > kMaxRanges) {
        set_error("mc_kv_attention_decode_noalloc: %u records per head exceed the %u the "
                  "built-in scratch holds (chunk_pos=%u is not a multiple of 64 and "
                  "max_chunks=%u > %u); use mc_kv_attention_decode",
                  nr, kMaxRanges, chunk_pos, max_chunks, kMaxRanges);
        return MC_E_INVALID_ARGUMENT;
    }
    float* rec = scratch_ptr();
    if (rec == nullptr) return MC_E_CUDA;
    ChunkLaunch L{d_q_rows, d_pos, nullptr, 1u, layer, d_page_table, nullptr, d_kv_pool,
                  nullptr, ly, rec, max_chunks, 0u, d_out, (hipStream_t)stream,
                  d_inv_freq, chunk_pos, 0u, false};
    return run_decode<false>(L, nullptr);
}

extern "C" mc_status_t mc_kv_attention_decode_chunks(
    const uint16_t* d_q_rows, const uint32_t* d_pos, uint32_t layer,
    const uint32_t* d_page_table, uint16_t* d_kv_pool, mc_kv_layout_t layout,
    float* d_partials, uint32_t max_chunks, uint16_t* d_out, void* stream,
    const float* d_inv_freq, uint32_t chunk_pos) {
    mckv::TraceRange trace_range("mc_kv_attention_decode_chunks");
    DevLayout ly;
    if (d_q_rows == nullptr || d_pos == nullptr || d_page_table == nullptr ||
        d_kv_pool == nullptr || d_partials == nullptr || d_out == nullptr ||
        !layout_valid(layout, &ly) || layer >= layout.num_layers ||
        !chunk_args_ok(max_chunks, chunk_pos)) {
        set_error("mc_kv_attention_decode_chunks: invalid args (layer=%u max_chunks=%u "
                  "chunk_pos=%u)",
                  layer, max_chunks, chunk_pos);
        return MC_E_INVALID_ARGUMENT;
    }
    // One chunk per range: the records are the per-chunk partials
    // [16][max_chunks][130] of the reference's chunk kernel.
    ChunkLaunch L{d_q_rows, d_pos, nullptr, 1u, layer, d_page_table, nullptr, d_kv_pool,
                  nullptr, ly, d_partials, max_chunks, max_chunks, d_out, (hipStream_t)stream,
                  d_inv_freq, chunk_pos, 1u, false};
    return fp32p_on() ? launch_chunk_kernel<true>(L) : launch_chunk_kernel<false>(L);
}

extern "C" mc_status_t mc_kv_attention_decode(
    const uint16_t* d_q_rows, const uint32_t* d_pos, uint32_t layer,
    const uint32_t* d_page_table, uint16_t* d_kv_pool, mc_kv_layout_t layout,
    float* d_partials, uint32_t max_chunks, uint16_t* d_out, void* stream,
    const float* d_inv_freq, uint32_t chunk_pos, float* d_partials2) {
    mckv::TraceRange trace_range("mc_kv_attention_decode");
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
    ChunkLaunch L{d_q_rows, d_pos, nullptr, 1u, layer, d_page_table, nullptr, d_kv_pool,
                  nullptr, ly, d_partials, max_chunks, 0u, d_out, (hipStream_t)stream,
                  d_inv_freq, chunk_pos, 0u, false};
    return run_decode<false>(L, d_partials2);
}

extern "C" mc_status_t mc_kv_attention_decode_merge(
    const float* d_partials, const uint32_t* d_pos, uint32_t max_chunks,
    uint32_t chunk_pos, float* d_partials2, uint16_t* d_out, void* stream) {
    mckv::TraceRange trace_range("mc_kv_attention_decode_merge");
    if (d_partials == nullptr || d_pos == nullptr || d_out == nullptr ||
        !chunk_args_ok(max_chunks, chunk_pos)) {
        set_error("mc_kv_attention_decode_merge: invalid args (max_chunks=%u "
                  "chunk_pos=%u)",
                  max_chunks, chunk_pos);
        return MC_E_INVALID_ARGUMENT;
    }
    return launch_merge<false>(d_partials, d_pos, nullptr, 1, max_chunks, chunk_pos,
                               d_partials2, d_out, (hipStream_t)stream, nullptr);
}

extern "C" mc_status_t mc_kv_attention_decode_batch(
    const uint16_t* d_q_rows, const uint32_t* const* d_slot_pos, uint32_t B,
    uint32_t layer, const uint32_t* const* d_slot_pt, uint16_t* const* d_slot_kv,
    mc_kv_layout_t layout, float* d_partials, uint32_t max_chunks, uint16_t* d_out,
    void* stream, const float* d_inv_freq, uint32_t chunk_pos, float* d_partials2) {
    mckv::TraceRange trace_range("mc_kv_attention_decode_batch");
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
    ChunkLaunch L{d_q_rows, nullptr, d_slot_pos, B, layer, nullptr, d_slot_pt, nullptr,
                  d_slot_kv, ly, d_partials, max_chunks, 0u, d_out, (hipStream_t)stream,
                  d_inv_freq, chunk_pos, 0u, true};
    return run_decode<true>(L, d_partials2);
}

extern "C" mc_status_t mc_kv_debug_decode_fp32p(uint32_t fp32_p, uint32_t* previous) {
    if (fp32_p > 1u && fp32_p != kFromEnv) {
        set_error("mc_kv_debug_decode_fp32p: fp32_p must be 0, 1 or 0xFFFFFFFF (got %u)", fp32_p);
        return MC_E_INVALID_ARGUMENT;
    }
    const uint32_t prev = g_fp32p.exchange(fp32_p);
    if (previous != nullptr) *previous = prev;
    return MC_OK;
}

extern "C" mc_status_t mc_kv_debug_decode_timeline(uint64_t* d_stamps, uint32_t launches) {
    if ((d_stamps == nullptr) != (launches == 0u)) {
        set_error("mc_kv_debug_decode_timeline: stamps=%p with launches=%u (both or neither)",
                  (void*)d_stamps, launches);
        return MC_E_INVALID_ARGUMENT;
    }
    MC_GUARD_BEGIN
    std::lock_guard<std::mutex> lk(g_tl_mu);
    g_tl_buf = reinterpret_cast<unsigned long long*>(d_stamps);
    g_tl_launches = launches;
    g_tl_next = 0u;
    return MC_OK;
    MC_GUARD_END
}

extern "C" mc_status_t mc_kv_debug_decode_records_only(uint32_t enable, uint32_t* previous) {
    const uint32_t prev = g_records_only.exchange(enable ? 1u : 0u);
    if (previous != nullptr) *previous = prev;
    return MC_OK;
}
