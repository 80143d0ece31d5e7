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
// MI355X design: one 512-thread workgroup (8 wave64, 2 per SIMD) per (kv
// head, 32-row q tile, key split); heavy (late) q tiles are launched first,
// and where greedy dispatch would leave a third round of similar-size jobs on
// a few CUs, one workgroup per CU runs a fixed two/three-job packing.
// Launches with fewer than 512 such workgroups use 16-row tiles instead: as
// two 4-wave halves that take alternate key steps and merge their softmax
// states in LDS (no key splits, at most two tiles per CU: the heaviest
// causal tile sets the time; each half waits only for its own waves, so the
// halves run out of phase), else as 256-thread workgroups two per CU.
// The 32 rows x 8 query heads of a KV head are 256 query vectors: wave w owns
// two 16-column groups, group g holding rows 4w + 2g + {0, 1} x heads 0..7.
// Keys stream in 64-position steps gathered through the page table into LDS
// (three buffers, register-staged prefetch of the next step, page ids one
// step ahead), K and V row-major. Per step and column group:
//   * S^T = K x Q^T: 4 key blocks x 4 v_mfma_f32_16x16x32_bf16 (Q^T in
//     registers for the whole kernel);
//   * online softmax per column over the 64 keys (lane holds 16 scores; the
//     column max across the 4 lane groups with two row-swap permutes), exp2
//     with the scale folded into one FMA, p fp32 for l, bf16
//     (v_cvt_pk_bf16_f32) for P.V;
//   * O^T += V^T x P^T: 2 halves x 8 v_mfma_f32_16x16x32_bf16, V^T read from
//     the row-major tile with gfx950's transposing LDS read, the contraction
//     index permuted identically on both operands so that P^T is exactly the
//     lanes' softmax output.
// The online-softmax update runs per 64 keys (the reference updates per 16)
// with a lazily moved reference max; both are exact restatements of softmax
// and differ only in rounding.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>

#include "error.h"
#include "trace.h"
#include "kv_common.h"
#include "kv_internal.h"

namespace mckv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Workgroup shapes (template parameter SH):
//   kRows32: 512 threads, 8 waves, 32 q rows, three LDS buffers, ping-pong
//            P.V; one workgroup per CU (107 KB LDS);
//   kRows16: 256 threads, 4 waves, 16 q rows, two LDS buffers; two per CU;
//   kHalves: 512 threads, 16 q rows, two 4-wave halves on alternate key steps
//            (two LDS buffers each) merged in LDS at the end; one per CU.
constexpr uint32_t kRows32 = 0u, kRows16 = 1u, kHalves16 = 2u;
// 32-row workgroup count (2 per CU) below which the 16-row shapes are used.
constexpr uint32_t kSmallBelow = 512u;
// Polls of a per-half barrier before it gives up (s_sleep 1 = 64 clocks each,
// about 2^22 * 64 / 2.4 GHz = 0.1 s): far beyond any legal wait, so it only
// ends a wait that can never complete. A timed-out wait is counted in
// g_barrier_timeouts (read by mc_kv_debug_prefill_status).
constexpr uint32_t kHalfBarrierSpins = 1u << 22;
__device__ uint32_t g_barrier_timeouts;
// Forced shape (debug hook; kAutoShape = chosen per launch) and job packing.
constexpr uint32_t kAutoShape = 0xFFFFFFFFu;
std::atomic<uint32_t> g_shape{kAutoShape};
std::atomic<uint32_t> g_packing{1u};

// Compute units of the current device (cached per device; 0 if unknown).
uint32_t cu_count() {
    static std::atomic<uint32_t> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0u;
    uint32_t v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0u) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            return 0u;
        v = static_cast<uint32_t>(n);
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

template <uint32_t SH>
struct PfShape {
    static constexpr uint32_t kThreads = SH == kRows16 ? 256u : 512u;
    static constexpr uint32_t kHalves = SH == kHalves16 ? 2u : 1u;  // key-step sets
    static constexpr uint32_t kQRows = kThreads / kHalves / 16u;  // q rows (4 per wave)
    static constexpr uint32_t kBufs = SH == kRows32 ? 3u : 2u;  // LDS K/V buffers per half
};

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& u) {
    return __builtin_bit_cast(bf16x8, u);
}
// Max over the 4 lanes l, l^16, l^32, l^48 with gfx950's row-swap permutes
// (VALU, no LDS round trip): permlane16_swap(x, x) yields rows (0,0,2,2) and
// (1,1,3,3) of x, permlane32_swap(y, y) the halves (lo,lo) and (hi,hi).
__device__ __forceinline__ float max_across_groups(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y),
                                                    false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

constexpr uint32_t kStep = 64;   // keys per step (32-key steps measured slower)
constexpr int kNKB = kStep / 16;  // 16-key blocks per step
constexpr int kNH = kStep / 32;   // 32-key halves per step (one PV MFMA each)
// Page-id modes of the K/V gather: per row, one page per 64-key step
// (P >= 64), one page per 32-key half (P = 32).
constexpr uint32_t kPageRow = 0, kPageStep = 1, kPageHalf = 2;
constexpr uint32_t kKPitch = 144;  // sK row pitch (bf16): 128 dims + 16 (conflict-free K reads)
constexpr uint32_t kVPitch = 144;  // sV row pitch (bf16): 128 dims + 16 (conflict-free tr reads)
// LDS operand reads issued this many MFMA blocks ahead of their use (software
// pipelining written out in the source; 6-16 measured alike, 2% faster than
// reading each operand right before its MFMAs).
constexpr int kOperandAhead = 8;

// One job = (query tile, kv head, key split), numbered heavy tile first.
template <uint32_t PM, uint32_t SH>
__device__ __forceinline__ void prefill_job(
    const uint16_t* __restrict__ q_rows, uint32_t T, uint32_t base_pos, uint32_t layer,
    const uint32_t* __restrict__ pt, const uint16_t* __restrict__ pool, DevLayout ly,
    uint16_t* __restrict__ out, float* __restrict__ partials, uint32_t S, uint32_t job) {
    constexpr uint32_t kThreads = PfShape<SH>::kThreads;
    constexpr uint32_t kQRows = PfShape<SH>::kQRows;
    constexpr uint32_t kBufs = PfShape<SH>::kBufs;
    constexpr uint32_t kH = PfShape<SH>::kHalves;
    constexpr uint32_t kKeysPerPass = kThreads / kH / 16u;  // keys one gather pass covers
    constexpr int kPass = 32 / (int)kKeysPerPass;      // passes per 32-key half
    constexpr int kStage = 2 * kNH * kPass;            // 16-byte chunks per thread and step
    __shared__ __align__(16) uint16_t sK[kH * kBufs][kStep * kKPitch];
    __shared__ __align__(16) uint16_t sV[kH * kBufs][kStep * kVPitch];

    const uint32_t ntq = (T + kQRows - 1u) / kQRows;
    const uint32_t s = job % S;
    const uint32_t kvh = (job / S) % kHkv;
    const uint32_t qt = ntq - 1u - job / (S * kHkv);  // heavy tiles first
    const uint32_t tb = qt * kQRows;
    const uint32_t key_end = base_pos + tb + min(kQRows - 1u, T - 1u - tb);  // last key
    const uint32_t last = key_end / kStep;
    const uint32_t qsp = (last + S) / S;  // ceil((last+1)/S)
    const uint32_t js0 = s * qsp;
    const uint32_t js1 = min(js0 + qsp - 1u, last);

    const uint32_t tid = threadIdx.x;
    const uint32_t wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
    // kHalves16: waves w and w + 4 own the same query columns; half h takes
    // the steps js0 + h, js0 + h + 2, ... into its own LDS buffers.
    const uint32_t half = kH == 2u ? wave_id >> 2 : 0u;
    const uint32_t wave = kH == 2u ? wave_id & 3u : wave_id;
    const uint32_t hb = half * kBufs;  // this half's first LDS buffer
    const uint32_t lane = tid & 63u;
    const uint32_t col = lane & 15u;
    const uint32_t grp = lane >> 4;
    constexpr int G = 2;

    // Query columns: group g, column col -> head col%8, row 4*wave + 2g + col/8.
    uint32_t row[G];
    bf16x8 qb[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        row[g] = tb + 4u * wave + 2u * g + (col >> 3);
        const bool ok = row[g] < T;
        const uint16_t* q =
            q_rows + (size_t)(ok ? row[g] : tb) * kRow + (kvh * kGroup + (col & 7u)) * kD +
            8u * grp;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint4 v = *reinterpret_cast<const uint4*>(q + 32u * m);
            qb[g][m] = as_bf16x8(ok ? v : make_uint4(0u, 0u, 0u, 0u));
        }
    }

    // Per column: running reference max m_run (raw score units), the score
    // above which it moves (thr = m_run + 8 / kC) and nmc = -m_run * kC
    // (0 while m_run is -inf), all updated only when the reference moves.
    float m_run[G], l_run[G], ren[G], thr[G], nmc[G];
    f32x4 acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_run[g] = -INFINITY;
        thr[g] = -INFINITY;
        nmc[g] = 0.f;
        l_run[g] = 0.f;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[g][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Cooperative gather: per 32-key half, thread tid moves the 16-byte K and
    // V chunks of key tid/16, dims 8*(tid%16) (16 threads per 256-byte row).
    // [K chunks of each half and pass, then V chunks]; zero until the first
    // gather (a half without steps stores zeros)
    uint4 stage[kStage];
#pragma unroll
    for (int r = 0; r < kStage; ++r) stage[r] = make_uint4(0u, 0u, 0u, 0u);
    const uint32_t gtid = tid & (kThreads / kH - 1u);  // gather thread within the half
    const uint32_t kkey = gtid >> 4, kdb = gtid & 15u;
    // key (within the step) and K/V half of stage slot r
    auto key_of = [&](int r) {
        const int rem = r % (kNH * kPass);
        return 32u * (uint32_t)(rem / kPass) + kKeysPerPass * (uint32_t)(rem % kPass) + kkey;
    };
    // Page ids are fetched one step ahead of the K/V loads that use them, so
    // a gather waits for one memory latency, not two. With P >= kStep a step lies
    // in one page, with P = 32 each 32-key half of a step does: their ids are
    // read through the scalar path (row r lies in half (r mod 2 kPass) / kPass).
    auto page_ids = [&](uint32_t js, uint32_t (&pg)[kStage]) {
        if constexpr (PM != kPageRow) {
            uint32_t id[kNH];
#pragma unroll
            for (int h = 0; h < kNH; ++h) {
                const uint32_t pos = js * kStep + (PM == kPageHalf ? 32u * (uint32_t)h : 0u);
                id[h] = (PM == kPageHalf || h == 0) && pos <= key_end
                            ? clamp_page(ly, ((const __attribute__((address_space(4))) uint32_t*)(
                                                 pt))[__builtin_amdgcn_readfirstlane(
                                                 table_index(ly, pos))])
                            : 0u;
            }
#pragma unroll
            for (int r = 0; r < kStage; ++r)
                pg[r] = PM == kPageHalf ? id[(r % (kNH * kPass)) / kPass] : id[0];
        } else {
#pragma unroll
            for (int r = 0; r < kStage; ++r) {
                const uint32_t pos = js * kStep + key_of(r);
                pg[r] = pos <= key_end ? clamp_page(ly, pt[table_index(ly, pos)]) : 0u;
            }
        }
    };
    auto gather = [&](uint32_t js, const uint32_t (&pg)[kStage]) {
        if constexpr (PM != kPageRow) {
            // The step (or each 32-key half) lies in one page: scalar page
            // base, 32-bit lane offsets, and no per-lane range test unless the
            // step passes key_end.
            const uint16_t* pbases[kNH];
#pragma unroll
            for (int h = 0; h < kNH; ++h)
                pbases[h] = pool + token_base(ly, layer, pg[PM == kPageHalf ? h * kPass : 0], 0u);
            const uint32_t step0 = js * kStep;
            const bool full = step0 + kStep - 1u <= key_end;  // wave-uniform
#pragma unroll
            for (int r = 0; r < kStage; ++r) {
                const uint32_t key = key_of(r);
                const uint16_t* pbase =
                    pbases[PM == kPageHalf ? (r % (kNH * kPass)) / kPass : 0];
                const uint32_t off = ((step0 + key) & ly.pmask) * kSlotElems +
                                     (r >= kNH * kPass ? 256u : 0u) + kvh * kD + kdb * 8u;
                if (full) {
                    stage[r] = *reinterpret_cast<const uint4*>(pbase + off);
                } else {
                    uint4 v = make_uint4(0u, 0u, 0u, 0u);
                    if (step0 + key <= key_end) v = *reinterpret_cast<const uint4*>(pbase + off);
                    stage[r] = v;
                }
            }
            return;
        }
#pragma unroll
        for (int r = 0; r < kStage; ++r) {
            const bool isv = r >= kNH * kPass;
            const uint32_t key = key_of(r);
            const uint32_t dblk = kdb;
            const uint32_t pos = js * kStep + key;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (pos <= key_end) {
                v = *reinterpret_cast<const uint4*>(
                    pool + token_base(ly, layer, pg[r], pos & ly.pmask) + (isv ? 256u : 0u) +
                    kvh * kD + dblk * 8u);
            }
            stage[r] = v;
        }
    };
    auto put = [&](int b) {
#pragma unroll
        for (int r = 0; r < kNH * kPass; ++r) {
            const uint32_t key = key_of(r);
            *reinterpret_cast<uint4*>(&sK[hb + b][key * kKPitch + kdb * 8u]) = stage[r];
            *reinterpret_cast<uint4*>(&sV[hb + b][key * kVPitch + kdb * 8u]) =
                stage[kNH * kPass + r];
        }
    };

    // exp(score - m) = exp2(s*c - m*c) with s the raw dot product, c = scale *
    // log2(e): one FMA and one v_exp per score. m_run is the running max of the
    // raw scores (c > 0). l is kept per lane (its own 8 keys per step) and
    // summed across the 4 lane groups at the end.
    constexpr float kC = kScoreScale * 1.4426950408889634f;
    constexpr float kMoveSlack = 8.f / kC;  // 8 in log2 units, in raw score units
    constexpr float kSumCap = 256.f;        // lane sum of p that still bounds p by 2^8
    uint32_t pgn[kStage] = {};
    const uint32_t jsf = js0 + half;  // this half's first step
    if (jsf <= js1) {
        page_ids(jsf, pgn);
        gather(jsf, pgn);
        if (jsf + kH <= js1) page_ids(jsf + kH, pgn);
    }
    // Ping-pong: waves 4..7 (the second wave on each SIMD) add step j's P.V
    // at the start of step j+1, so that on every SIMD one wave runs MFMA
    // while the other runs the softmax. Three LDS buffers keep step j's V
    // intact until then (a wave that writes step j+1's buffer has passed the
    // barrier of step j, so all waves have finished step j-1).
    const bool late_pv = SH == kRows32 && wave >= 4u;
    // P of the current step; late waves consume it at the start of the next
    // step, before that step's softmax overwrites it.
    bf16x8 pb[G][kNH];
    int bprev = 0;
    // V^T operand straight from the row-major V tile with the transposing LDS
    // read: within each 16-lane group, ds_read_b64_tr_b16 gives lane x the
    // element x%4 of the 8-byte rows addressed by lanes 4j + x/4 (j < 4). With
    // lane (4j + r) of group grp addressing key 4*grp + j, dims 16*db + 4r,
    // lane x receives dim 16*db + x of keys 4*grp + j: the A operand of
    // O^T += V^T x P^T. Contraction index i of lane group grp <-> key
    // 32h + 16*(i/4) + 4*grp + i%4 on both operands.
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const uint32_t tr_row = 4u * grp + (col >> 2), tr_col = 4u * (col & 3u);
    auto vread = [&](const uint16_t* Vs, int h, int db) {
        const uint16_t* vr = Vs + (32u * h + tr_row) * kVPitch + 16u * db + tr_col;
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) bf16x4*)(vr));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (__attribute__((address_space(3))) bf16x4*)(vr + 16u * kVPitch));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    auto pv = [&](const uint16_t* Vs, const bf16x8 (&pbv)[G][kNH]) {
        // V^T operands read kOperandAhead blocks ahead of the MFMAs using them
        constexpr int kN = 8 * kNH, kAhead = kOperandAhead;
        bf16x8 va[kN];
#pragma unroll
        for (int i = 0; i < kAhead && i < kN; ++i) va[i] = vread(Vs, i / 8, i % 8);
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            if (i + kAhead < kN) va[i + kAhead] = vread(Vs, (i + kAhead) / 8, (i + kAhead) % 8);
#pragma unroll
            for (int g = 0; g < G; ++g)
                acc[g][i % 8] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[i], pbv[g][i / 8],
                                                                        acc[g][i % 8], 0, 0, 0);
        }
    };
    int b = 0;
    // iterations: the same count for both halves (barriers). A half whose
    // step is past js1 in the last one (act false) stores its last staged
    // data (or zeros) and masks every key, which leaves its state unchanged.
    const uint32_t nit = js0 <= js1 ? (js1 - js0) / kH + 1u : 0u;
    // kHalves16: each half reads and writes only its own LDS buffers, so per
    // iteration it waits only for its own 4 waves (a counter in LDS), and the
    // halves drift apart like two workgroups (one runs MFMA while the other
    // runs the softmax). The wait is bounded so that it cannot hang the
    // kernel; a wait that runs out (the half would then race on LDS buffers
    // still in use, so its output is unreliable) increments the device word
    // g_barrier_timeouts with a vector atomic, which the host reads back.
    constexpr bool kHalfBar = kH == 2u;
    __shared__ uint32_t s_bar[2];
    if constexpr (kHalfBar) {
        if (tid < 2u) s_bar[tid] = 0u;
        __syncthreads();
    }
    auto half_barrier = [&](uint32_t target) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0u) __hip_atomic_fetch_add(&s_bar[half], 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
        bool done = false;
        for (uint32_t spin = 0; spin < kHalfBarrierSpins; ++spin) {
            const uint32_t v = __builtin_amdgcn_readfirstlane(__hip_atomic_load(
                &s_bar[half], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            if (v >= target) {
                done = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!done && lane == 0u)
            __hip_atomic_fetch_add(&g_barrier_timeouts, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    for (uint32_t it = 0; it < nit; ++it, bprev = b, b = (b + 1 == (int)kBufs) ? 0 : b + 1) {
        const uint32_t js = js0 + it * kH + half;
        const bool act = kH == 1u || js <= js1;  // wave-uniform
        put(b);
        if constexpr (kHalfBar) half_barrier(4u * (it + 1u));
        else __syncthreads();
        if (js + kH <= js1) {
            gather(js + kH, pgn);
            if (js + 2u * kH <= js1) page_ids(js + 2u * kH, pgn);
        }
        const uint16_t* K = sK[hb + b];
        const uint16_t* Vt = sV[hb + b];
        if (late_pv && js > js0) pv(sV[hb + bprev], pb);
        // S^T blocks: key block kb (keys 16kb + row), lane col = query column.
        f32x4 sacc[kNKB][G];
        {
            // K operands read kOperandAhead blocks ahead of the MFMAs using them.
            // Operand o is dim slice m = o / kNKB of key block kb = o % kNKB:
            // the MFMAs run slice-major, so consecutive MFMAs feed kNKB * G
            // different accumulators and a chain's next MFMA comes 8 issues
            // after its previous one (a dependent 16x16x32 MFMA otherwise
            // waits for its predecessor's result); every accumulator still
            // sums its slices in order m = 0..3.
            constexpr int kN = 4 * kNKB, kAhead = kOperandAhead;
            bf16x8 ka[kN];
            auto kread = [&](int o) {
                const int kb = o % kNKB, m = o / kNKB;
                const uint16_t* kp = K + (16u * kb + col) * kKPitch + 32u * m + 8u * grp;
                return as_bf16x8(*reinterpret_cast<const uint4*>(kp));
            };
#pragma unroll
            for (int i = 0; i < kAhead && i < kN; ++i) ka[i] = kread(i);
#pragma unroll
            for (int i = 0; i < kN; ++i) {
                if (i + kAhead < kN) ka[i + kAhead] = kread(i + kAhead);
                const int kb = i % kNKB, m = i / kNKB;
#pragma unroll
                for (int g = 0; g < G; ++g)
                    sacc[kb][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        ka[i], qb[g][m], m == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : sacc[kb][g], 0, 0,
                        0);
            }
        }
        // Keys of this lane: 32*js + 16*kb + 4*grp + j. Only steps that reach
        // past the tile's first row can hold masked keys (wave-uniform test).
        if (!act || js * kStep + kStep - 1u > base_pos + tb) {
            const uint32_t pos0 = js * kStep + 4u * grp;
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int kb = 0; kb < kNKB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (!act || pos0 + 16u * kb + (uint32_t)j > base_pos + row[g])
                            sacc[kb][g][j] = -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            // Fast path: once every column has a reference, p is computed
            // against it directly; a lane sum of at most kSumCap bounds every
            // p by 2^8 as the max test below would, so the max is needed only
            // when the sum says the reference may have to move (wave-uniform).
            if (__builtin_amdgcn_ballot_w64(m_run[g] == -INFINITY) == 0u) {
                float ls = 0.f;
#pragma unroll
                for (int kb = 0; kb < kNKB; ++kb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float p =
                            __builtin_amdgcn_exp2f(fmaf(sacc[kb][g][j], kC, nmc[g]));
                        ls += p;
                        pb[g][kb >> 1][4 * (kb & 1) + j] = (__bf16)p;
                    }
                if (__builtin_amdgcn_ballot_w64(ls > kSumCap) == 0u) {
                    l_run[g] += ls;
                    continue;
                }
            }
            float tm = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < kNKB; ++kb)
                tm = fmaxf(tm, fmaxf(fmaxf(sacc[kb][g][0], sacc[kb][g][1]),
                                     fmaxf(sacc[kb][g][2], sacc[kb][g][3])));
            tm = max_across_groups(tm);
            // Lazy reference point: m_run moves only when the new max exceeds
            // it by more than 8 in log2 units (p <= 2^8 otherwise) or when it
            // is still -inf (thr = -inf: any finite max moves it); softmax is
            // invariant to the reference point, so this changes rounding only
            // and leaves most steps without the acc rescale. Column-uniform
            // (tm, m_run agree across lane groups). A moving max exceeds
            // m_run, so the new reference is tm itself; from m_run = -inf the
            // factor exp2(-inf) is 0.
            ren[g] = 1.f;
            if (tm > thr[g]) {
                const float renew = __builtin_amdgcn_exp2f((m_run[g] - tm) * kC);
                l_run[g] *= renew;
                m_run[g] = tm;
                thr[g] = tm + kMoveSlack;
                nmc[g] = -tm * kC;
                ren[g] = renew;
            }
            // fully masked so far (m_run = -inf, nmc = 0): every score is -inf,
            // p = 0 and the state is kept
            float ls = 0.f;
#pragma unroll
            for (int kb = 0; kb < kNKB; ++kb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][g][j], kC, nmc[g]));
                    ls += p;
                    pb[g][kb >> 1][4 * (kb & 1) + j] = (__bf16)p;
                }
            l_run[g] += ls;
            if (__builtin_amdgcn_ballot_w64(ren[g] != 1.f) != 0u) {
#pragma unroll
                for (int db = 0; db < 8; ++db) acc[g][db] = acc[g][db] * ren[g];
            }
        }
        if (!late_pv) pv(Vt, pb);
    }
    if (late_pv && js0 <= js1) pv(sV[hb + bprev], pb);
    if constexpr (kH == 2u) {
        // Fold half 1's state into half 0 through LDS (the K buffers, free
        // after the barrier): per column M = max(m0, m1), factors
        // exp2((m_h - M) * c) (0 for a half that saw no key), l and acc scaled
        // and summed. Per lane: G (m, l) pairs and G * 8 acc quads.
        static_assert(sizeof(float2) * G * 64u * 4u + sizeof(f32x4) * G * 8u * 64u * 4u <=
                          sizeof(sK),
                      "state fits the K buffers");
        f32x4* sa = reinterpret_cast<f32x4*>(&sK[0][0]) + wave * (G * 8u * 64u) + lane;
        float2* sml = reinterpret_cast<float2*>(reinterpret_cast<f32x4*>(&sK[0][0]) +
                                                4u * G * 8u * 64u) +
                      wave * (G * 64u) + lane;
        __syncthreads();
        if (half == 1u) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                sml[g * 64] = make_float2(m_run[g], l_run[g]);
#pragma unroll
                for (int db = 0; db < 8; ++db) sa[(g * 8 + db) * 64] = acc[g][db];
            }
        }
        __syncthreads();
        if (half == 1u) return;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float2 ml = sml[g * 64];
            const float M = fmaxf(m_run[g], ml.x);
            const float f0 =
                m_run[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_run[g] - M) * kC);
            const float f1 = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((ml.x - M) * kC);
            m_run[g] = M;
            l_run[g] = l_run[g] * f0 + ml.y * f1;
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                acc[g][db] = acc[g][db] * f0 + sa[(g * 8 + db) * 64] * f1;
                __builtin_amdgcn_sched_barrier(0);  // one quad in flight: no register peak
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        l_run[g] += __shfl_xor(l_run[g], 16);
        l_run[g] += __shfl_xor(l_run[g], 32);
    }

    // Epilogue: lane holds dims 16*db + 4*grp + j of column (head, row).
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (row[g] >= T) continue;
        const uint32_t qh = kvh * kGroup + (col & 7u);
        if (S == 1u) {
            uint16_t* o = out + (size_t)row[g] * 2048u + qh * kD + 4u * grp;
            const float L = l_run[g];
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                uint16_t w[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    w[j] = f32_to_bf16(L > 0.f ? acc[g][db][j] / L : 0.f);
                *reinterpret_cast<uint2*>(o + 16u * db) =
                    make_uint2((uint32_t)w[0] | ((uint32_t)w[1] << 16),
                               (uint32_t)w[2] | ((uint32_t)w[3] << 16));
            }
        } else {
            float* pw = partials + ((size_t)(row[g] * 16u + qh) * S + s) * kPartial;
            if (grp == 0u) {  // m of the record is in score units (raw * scale)
                pw[0] = m_run[g] * kScoreScale;
                pw[1] = l_run[g];
            }
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                float* d = pw + 2u + 16u * db + 4u * grp;
                *reinterpret_cast<float2*>(d) = make_float2(acc[g][db][0], acc[g][db][1]);
                *reinterpret_cast<float2*>(d + 2) = make_float2(acc[g][db][2], acc[g][db][3]);
            }
        }
    }
}

// grid = one workgroup per job. Jobs are dispatched to CUs as they free up,
// heavy first, which packs well while the jobs are many or of very different
// sizes. With S == 1, between two and three jobs per resident workgroup slot
// (`slots`, 0 = off) and a prefix of at least T/4 (jobs of similar size),
// that greedy order leaves a third round of jobs on a few CUs; there the
// last `slots` workgroups run a fixed packing instead and the others exit at
// once: t = n - 2*slots slots take three of the 3t lightest jobs each
// (snake order), the others two of the remaining ones (heaviest with
// lightest). Every job is computed the same way in both modes.
template <uint32_t PM, uint32_t SH>
__global__ void __launch_bounds__(PfShape<SH>::kThreads)
    __attribute__((amdgpu_waves_per_eu(2))) prefill_attn_kernel(
    const uint16_t* __restrict__ q_rows, uint32_t T,
    const uint32_t* __restrict__ d_base_pos, uint32_t layer,
    const uint32_t* __restrict__ pt, const uint16_t* __restrict__ pool, DevLayout ly,
    uint16_t* __restrict__ out, float* __restrict__ partials, uint32_t S, uint32_t slots) {
    const uint32_t base_pos = *d_base_pos;
    const uint32_t n = gridDim.x;
    uint32_t jobs[3] = {blockIdx.x, 0u, 0u}, nj = 1u;
    if constexpr (SH == kRows32) {
        if (S == 1u && slots > 0u && n > 2u * slots && n <= 3u * slots &&
            4ull * base_pos >= T) {
            if (blockIdx.x < n - slots) return;
            const uint32_t w = blockIdx.x - (n - slots);
            const uint32_t t = n - 2u * slots, pairs = slots - t, b0 = 2u * pairs;
            if (w < pairs) {
                jobs[0] = w;
                jobs[1] = b0 - 1u - w;
                nj = 2u;
            } else {
                const uint32_t u = w - pairs;
                jobs[0] = b0 + u;
                jobs[1] = b0 + 2u * t - 1u - u;
                jobs[2] = b0 + 2u * t + u;
                nj = 3u;
            }
        }
    }
    for (uint32_t i = 0; i < nj; ++i) {
        if (i > 0u) __syncthreads();  // LDS buffers are reused by the next job
        prefill_job<PM, SH>(q_rows, T, base_pos, layer, pt, pool, ly, out, partials,
                                      S, jobs[i]);
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

extern "C" mc_status_t mc_kv_debug_prefill_shape(uint32_t shape, uint32_t* previous) {
    if (shape > mckv::kHalves16 && shape != mckv::kAutoShape) {
        set_error("mc_kv_debug_prefill_shape: shape %u is not 0, 1, 2 or 0xFFFFFFFF", shape);
        return MC_E_INVALID_ARGUMENT;
    }
    const uint32_t prev = mckv::g_shape.exchange(shape);
    if (previous != nullptr) *previous = prev;
    return MC_OK;
}

extern "C" mc_status_t mc_kv_debug_prefill_packing(uint32_t enable, uint32_t* previous) {
    const uint32_t prev = mckv::g_packing.exchange(enable ? 1u : 0u);
    if (previous != nullptr) *previous = prev;
    return MC_OK;
}

extern "C" mc_status_t mc_kv_debug_prefill_status(uint32_t* barrier_timeouts, uint32_t reset) {
    if (barrier_timeouts == nullptr) {
        set_error("mc_kv_debug_prefill_status: barrier_timeouts is NULL");
        return MC_E_INVALID_ARGUMENT;
    }
    // Synchronous on the null stream: waits for prefill launches in flight on
    // blocking streams of the current device.
    hipError_t e = hipMemcpyFromSymbol(barrier_timeouts, HIP_SYMBOL(mckv::g_barrier_timeouts),
                                       sizeof(uint32_t), 0, hipMemcpyDeviceToHost);
    if (e == hipSuccess && reset) {
        const uint32_t zero = 0u;
        e = hipMemcpyToSymbol(HIP_SYMBOL(mckv::g_barrier_timeouts), &zero, sizeof(zero), 0,
                              hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        set_error("mc_kv_debug_prefill_status: %s", hipGetErrorString(e));
        return MC_E_CUDA;
    }
    return MC_OK;
}

namespace mckv {
// Reads and clears the device's half-barrier timeout count after the caller
// synchronized its prefill work; a non-zero count means some launch's output
// may be wrong, reported as MC_E_INTERNAL with the count in the message.
mc_status_t prefill_barrier_check(const char* who) {
    uint32_t n = 0u;
    hipError_t e = hipMemcpyFromSymbol(&n, HIP_SYMBOL(g_barrier_timeouts), sizeof(n), 0,
                                       hipMemcpyDeviceToHost);
    if (e == hipSuccess && n != 0u) {
        const uint32_t zero = 0u;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_barrier_timeouts), &zero, sizeof(zero), 0,
                              hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        set_error("%s: prefill status read failed: %s", who, hipGetErrorString(e));
        return MC_E_CUDA;
    }
    if (n != 0u) {
        set_error("%s: %u prefill half-barrier wait(s) ran out of their bound; the prefill "
                  "output is unreliable",
                  who, n);
        return MC_E_INTERNAL;
    }
    return MC_OK;
}
}  // namespace mckv

extern "C" mc_status_t mc_kv_debug_prefill_force_timeouts(uint32_t count) {
    const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(mckv::g_barrier_timeouts), &count,
                                           sizeof(count), 0, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        set_error("mc_kv_debug_prefill_force_timeouts: %s", hipGetErrorString(e));
        return MC_E_CUDA;
    }
    return MC_OK;
}

extern "C" mc_status_t mc_kv_attention_prefill(const uint16_t* d_q_rows, uint32_t tokens,
                                               const uint32_t* d_base_pos, uint32_t layer,
                                               const uint32_t* d_page_table,
                                               const uint16_t* d_kv_pool,
                                               mc_kv_layout_t layout, uint16_t* d_out,
                                               float* d_partials, uint32_t S_kv,
                                               void* stream) {
    mckv::TraceRange trace_range("mc_kv_attention_prefill");
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
    hipStream_t st = (hipStream_t)stream;
    // Shape: 32-row tiles while they give at least two workgroups per CU;
    // below that 16-row tiles, as two halves on alternate key steps when the
    // launch has no key splits and at most two 16-row jobs per CU (the
    // heaviest causal tile then sets the time, and the halves take it at
    // twice the rate), else as 4-wave workgroups two per CU. Measured
    // (base 0): T=2048 67 -> 60 (16 rows) -> 47.5 us (halves), T=4096
    // 125 -> 118 -> 99.7 us; T=6144 178.5 us with 4-wave workgroups against
    // 210 with halves. With S_kv > 1 a tile's split boundaries follow its
    // last row, so they differ between 32- and 16-row tiles.
    const uint32_t ntq32 = (tokens + 31u) / 32u, ntq16 = (tokens + 15u) / 16u;
    const uint32_t cus = cu_count();
    uint32_t shape = g_shape.load(std::memory_order_relaxed);
    if (shape == kAutoShape) {
        if (kHkv * ntq32 * S_kv >= kSmallBelow) shape = kRows32;
        else if (S_kv == 1u && kHkv * ntq16 <= 2u * (cus ? cus : 256u)) shape = kHalves16;
        else shape = kRows16;
    }
#define MC_PF_LAUNCH(PG, SM)                                                                 \
    hipLaunchKernelGGL((prefill_attn_kernel<PG, SM>),                                        \
                       dim3(kHkv * ((tokens + PfShape<SM>::kQRows - 1u) / PfShape<SM>::kQRows) * \
                            S_kv),                                                           \
                       dim3(PfShape<SM>::kThreads), 0, st, d_q_rows, tokens, d_base_pos, layer, \
                       d_page_table, d_kv_pool, ly, d_out, d_partials, S_kv, slots)
    // resident 32-row workgroup slots: one per CU (LDS-limited)
    const uint32_t slots =
        shape == kRows32 && g_packing.load(std::memory_order_relaxed) ? cus : 0u;
    const uint32_t P = 1u << ly.log2p;
    const uint32_t pm = P >= kStep ? kPageStep : P == 32u ? kPageHalf : kPageRow;
#define MC_PF_PM(SM)                                             \
    if (pm == kPageStep) MC_PF_LAUNCH(kPageStep, SM);            \
    else if (pm == kPageHalf) MC_PF_LAUNCH(kPageHalf, SM);       \
    else MC_PF_LAUNCH(kPageRow, SM);
    switch (shape) {
        case kRows32: MC_PF_PM(kRows32) break;
        case kRows16: MC_PF_PM(kRows16) break;
        default: MC_PF_PM(kHalves16) break;
    }
#undef MC_PF_PM
#undef MC_PF_LAUNCH
    if (S_kv > 1u)
        hipLaunchKernelGGL(prefill_merge_kernel, dim3(tokens * 16u), dim3(128), 0, st,
                           d_partials, S_kv, tokens, d_out);
    return check_launch("prefill attention launch failed");
}
