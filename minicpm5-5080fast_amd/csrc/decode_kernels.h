// decode_kernels.h - device code of the paged split-KV flash decoding for one
// new token per session (single session and batched), shared by the two
// translation units that instantiate it (bf16-P and fp32-P).
//
// Contract of the reference path (native/kernels/sm120/attention_decode.cu:
// 966-1368 chunk kernel, 506-878 fp32-P SIMT variant, 1494-1595 merge_a /
// merge_b, 1389-1407/1602-1626 batched twins, 1840-1964/2120-2170 launchers):
//   * limit = *d_pos is the query position; keys/values 0..limit are attended.
//   * Work is split in chunks of chunk_pos positions; chunk c covers
//     [c*C, min(c*C+C-1, limit)]; chunks starting after limit do nothing.
//   * Scores are fp32 dot(q, k) * (1/sqrt(128) as fp32); softmax runs online in
//     16-position batches: mn = max(m, batch max), renew = exp(m - mn) (0 when
//     m = -inf), p = exp(score - mn) in fp32 feeds l, and p rounded to bf16
//     (RNE) feeds the P.V product (fp32-P mode: p itself feeds P.V, the
//     reference's MC_ATTN_HMMA_OFF fallback).
//   * A partial record is {m, l, acc[128]}; the merge folds records with
//     M = max m over l != 0, f = exp(m - M), L = sum l f, A = sum acc f and
//     writes bf16(A / L). A single record is written as the output directly.
//   * Phase0 (inv_freq != NULL): the block owning position `limit` rotates that
//     token's k from the qkv row, writes K and V of `limit` to the pool and uses
//     the fresh values; q is rotated on the fly (LDS) and never written back.
//
// MI355X design (one 256-thread workgroup = 4 wave64 per (slot, kv head,
// range of chunks); single-session 256/512-position tiers with at least 256
// workgroups put both KV heads in one 512-thread workgroup, and batched
// launches number their workgroups densely over the slots' existing chunk
// groups). Each wave walks 16-position tiles t = wave, wave+4, ...
// of each chunk and keeps one online-softmax state for all 8 query heads
// of the KV head over the whole range; the 4 wave states are folded through
// LDS once, into one record per query head; a second launch (merge_task)
// folds the records. The next tile's loads are in flight while the current
// tile computes.
//   * Loads: K in operand layout - a lane (token = lane%16, group = lane/16)
//     reads K dims [32m + 8*group, +8), m < 4, i.e. each instruction reads 64
//     contiguous bytes of 16 rows. V as whole 256-byte head rows (16 lanes per
//     row) into a wave-private, XOR-swizzled LDS tile. For the 64-position
//     chunk tier K is row-loaded the same way and read back from LDS in the
//     operand layout.
//   * QK: S^T[16 pos][16 heads] = K (A operand) x Q^T (B operand, preloaded;
//     heads 8..15 are zero padding) with four v_mfma_f32_16x16x32_bf16.
//   * The D layout gives each lane 4 positions of one head; the batch max/sum
//     combine the 4 lane groups with two row-swap permutes (16, 32).
//   * P.V: O^T += V^T x P^T (v_mfma_f32_16x16x16bf16_1k; fp32-P: four
//     v_mfma_f32_16x16x4f32). The V^T A operand comes from the LDS tile
//     through the transposing read ds_read_b64_tr_b16; P^T (B operand) is the
//     softmax output already in the right lanes. (The generic schedule for
//     chunk sizes that are not a multiple of 64 keeps V in operand layout and
//     transposes each 16x16 block exactly by an MFMA with an identity B
//     operand.) acc ends up as 32 fp32 per lane: head lane%16, dims
//     [32m + 8*group, +8).
// Arithmetic intensity is ~8 flop/byte, so the kernel is HBM-bound; MFMA keeps
// the VALU free for addressing and softmax.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "error.h"
#include "kv_common.h"

namespace mckv {
namespace {
// Cross-lane reductions without an LDS round trip. gfx950's row-swap
// permutes applied to (x, x): permlane16_swap gives the 16-lane rows
// (r0, r0, r2, r2) and (r1, r1, r3, r3), permlane32_swap the halves (lo, lo)
// and (hi, hi). Combining the two results reduces lanes l, l^16 (then l^32)
// with the same operands, in the same order, as xor shuffles would.
__device__ __forceinline__ float swap16_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float swap32_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float swap16_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float swap32_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
// Max over all 64 lanes: DPP within quads, 8- and 16-lane mirrors, then the
// row swaps (max is exact in any order).
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF,
                                                         false)));  // quad_perm 1,0,3,2
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF,
                                                         false)));  // quad_perm 2,3,0,1
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF,
                                                         false)));  // row_half_mirror
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF,
                                                         false)));  // row_mirror
    return swap32_max(swap16_max(x));
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kThreads = 256;
constexpr uint32_t kWaves = 4;
constexpr uint32_t kTile = 16;
constexpr uint32_t kPageCache = 128;  // page ids staged in LDS per block
// Smallest single-session grid that takes two-head (512-thread) workgroups.
constexpr uint32_t kKv2MinBlocks = 256;
// Register tiles in each wave's load ring (one load group ahead).
constexpr uint32_t kRing = 2;

// K/V rows are read once per launch: non-temporal loads keep them from
// displacing cached data (page tables, records) on their way through
// (C4 30.8 -> 30.0, C3 13.5 -> 12.6, C1 8.35 -> 7.9 us/layer).
// Pool and page-table pointers of batched launches are loaded from the slot
// tables, so the compiler cannot tell they address global memory and would
// emit FLAT accesses, which count against the LDS wait counter as well: every
// LDS wait of the V transpose would then also wait for the next tile's loads
// in flight. All of them point into device global memory; the casts below
// make the accesses global_load / global_store.
#define MCKV_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const MCKV_GLOBAL T* gptr(const T* p) {
    return (const MCKV_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ MCKV_GLOBAL T* gptr(T* p) {
    return (MCKV_GLOBAL T*)p;
}
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
    return __builtin_bit_cast(
        uint4, __builtin_nontemporal_load(reinterpret_cast<const MCKV_GLOBAL u32x4_t*>(gptr(p))));
}

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

// V tile swizzle of token row t (see xpose in decode_range_body).
__device__ __forceinline__ uint32_t vswz(uint32_t t) { return ((t >> 1) & 3u) * 4u + (t & 1u); }
// Dim of rows 4g..4g+3 of the P.V block (m, h) (A operand row 4g + i and
// accumulator row 4g + i hold dim vdim(m, h, g) + i): the 8-byte half read
// by lane group g is h ^ (g & 1).
__device__ __forceinline__ uint32_t vdim(uint32_t m, uint32_t h, uint32_t g) {
    return 32u * m + 8u * g + 4u * (h ^ (g & 1u));
}

// The entry clock is read at once and stored at exit, together with the
// workgroup's index (computed only then: it needs the grid size, one more
// argument load), so that nothing of the stamp buffer is waited for at entry.
struct WgStamp {
    unsigned long long* stamps;
    uint32_t words, cap;
    bool grid3;  // index over a 3-D grid (else blockIdx.x + gridDim.x * blockIdx.y)
    unsigned long long t_entry;
    uint32_t xcc;
    __device__ __forceinline__ WgStamp(unsigned long long* stamps_, uint32_t words_,
                                       uint32_t cap_, bool grid3_)
        : stamps(stamps_), words(words_), cap(cap_), grid3(grid3_),
          t_entry(__builtin_amdgcn_s_memrealtime()),
          xcc((uint32_t)__builtin_amdgcn_s_getreg(6164)) {}
    __device__ __forceinline__ unsigned long long* slot() const {
        if (stamps == nullptr) return nullptr;
        const uint32_t wg = grid3 ? blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)
                                  : blockIdx.x + gridDim.x * blockIdx.y;
        return wg < cap ? stamps + (size_t)words * wg : nullptr;
    }
    __device__ __forceinline__ ~WgStamp() {
        unsigned long long* p = slot();
        if (p == nullptr) return;
        if (threadIdx.x == 0u) {
            p[0] = t_entry;
            if (words > 2u) p[2] = (unsigned long long)xcc;
        }
        if ((threadIdx.x & 63u) == 0u)
            atomicMax(p + 1, (unsigned long long)__builtin_amdgcn_s_memrealtime());
    }
};

struct DecodeArgs {
    const uint16_t* q_row;  // [2560] of this slot
    uint32_t limit;
    const uint32_t* pt;
    uint16_t* pool;
    float* rec;       // this slot's records: 16 heads x rec_stride x 130 floats
    uint32_t rec_stride;
    bool split;       // record layout per head: false {m, l, acc[128]} rows,
                      // true acc[rec_stride][128] then {m, l}[rec_stride]
    uint16_t* out;    // this slot: [2048]
    const struct WgStamp* stamp;  // debug timeline (the first tile's arrival goes to word 3)
    const uint32_t* limit_src;  // the limit's device word, read by the body when the
                                // body's LSRC is set (else `limit` holds the limit)
    uint32_t pos_max;           // limits are clamped to this (the pool's last position)
};


// 256 threads process chunks [c_first, c_end) of one (slot, kv head) as ONE
// range: every wave keeps a single online-softmax state across all chunks of
// the range, the 4 wave states are folded once at the end and written as one
// record per query head, {m, l, acc[128]} at rec[(qh * rec_stride + group)]
// (the reference's partial layout) or, split, acc at row `group` and {m, l}
// at pair `group` of the head's block (see DecodeArgs), or, when the range is the only one (nvalid <= cpw), as the output
// bf16(acc / l). With KV2 the workgroup has 512 threads and threads 256-511
// run the same body for the second KV head over the same chunks (own LDS).
// Waves take tiles j = wave, wave+4, ... of each chunk (a chunk still bounds
// the tile grid, so with cpw = 1 a record is exactly the chunk partial of
// the reference's chunk kernel); the next tile's loads are issued before the
// current tile computes, also across chunk boundaries. cpw > 1 requires
// C % 64 == 0.
template <bool PH0, bool PAGE16, uint32_t TPW, bool KV2, bool FP32P, bool LSRC>
__device__ __forceinline__ void decode_range_body(const DecodeArgs a, uint32_t layer,
                                                  DevLayout ly, uint32_t NC,
                                                  const float* inv_freq,
                                                  uint32_t C, uint32_t kvh, uint32_t group,
                                                  uint32_t cpw) {
    constexpr uint32_t NH = KV2 ? 2u : 1u;  // kv heads per workgroup
    const uint32_t half = KV2 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 8) : 0u;
    // Load layouts per chunk tier. ROWS (64-position tier): K and V as whole
    // head rows, both transposed through LDS (measured faster for 2K
    // contexts). VROWS (all tiers of the straight-line schedule): V as head
    // rows read back with the transposing LDS read, K in operand layout
    // (row-loading K too measured equal at C = 256). The generic schedule
    // keeps both in operand layout.
    constexpr bool ROWS = TPW == 1u;
    constexpr bool VROWS = TPW >= 1u;
    // Row pitches of the rotated q rows (144 bf16 = 288 B) and the fold's acc
    // rows (132 fp32 = 528 B): with these the 16-byte reads of q (one row per
    // lane of a 16-lane group) and the fold's 16-byte writes and reads hit no
    // LDS bank twice (measured with an LDS probe on gfx950; the unpadded 256 B
    // and 512 B rows made every such access a 16- to 28-cycle conflict).
    constexpr uint32_t kQPitch = 144, kAccPitch = kD + 4u;
    __shared__ __align__(16) uint16_t s_q_[NH][PH0 ? kGroup * kQPitch : 1];  // rotated q rows
    __shared__ __align__(16) uint16_t s_fresh_[NH][256];  // K | V of `limit`
    __shared__ uint32_t s_pages_[NH][kPageCache];         // page ids of this block's range
    // per wave: K and V tile, 16 x 256 B (row loads only)
    __shared__ uint4 s_x_[NH][VROWS ? kWaves : 1u][VROWS ? 2u * 16u * 16u : 1u];
    __shared__ float s_m_[NH][kWaves][kGroup], s_l_[NH][kWaves][kGroup];
    __shared__ __align__(16) float s_acc_[NH][kWaves][kGroup][kAccPitch];
    auto& s_q = s_q_[half];
    auto& s_fresh = s_fresh_[half];
    auto& s_pages = s_pages_[half];
    auto& s_x = s_x_[half];
    auto& s_m = s_m_[half];
    auto& s_l = s_l_[half];
    auto& s_acc = s_acc_[half];

    const uint32_t tid = threadIdx.x & 255u;
    // Wave index made provably wave-uniform so every tile / chunk decision
    // below compiles to scalar branches.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63u;
    const uint32_t tok = lane & 15u;  // row within a 16-position tile / head col
    const uint32_t grp = lane >> 4;   // 0..3

    // q_row, inv_freq and pt are not restrict-qualified: loads through them
    // then count as ordinary memory reads, which the start-up's memory
    // clobbers keep in their round (invariant loads may be sunk past them).
    const uint16_t* q_row = a.q_row;
    const uint32_t* pt = a.pt;
    uint16_t* __restrict__ pool = a.pool;
    const uint32_t kvcol = kvh * kD + 8u * grp;  // within a token's K or V half
    // Page ids are clamped to the pool and table indices to the table's
    // max_pages entries (a corrupt entry reads a wrong page instead of
    // faulting the GPU).
    const uint32_t page_max = ly.max_pages - 1u;
    // A 16-position tile starts 16-aligned, so with P >= 16 (PAGE16) it lies in
    // one page and the page id is wave-uniform: it is read through the scalar
    // path and does not serialize behind the vector loads in flight.
    auto table_page = [&](uint32_t t0) {
        return min(((const __attribute__((address_space(4))) uint32_t*)(pt))
                       [__builtin_amdgcn_readfirstlane(min(t0 >> ly.log2p, page_max))],
                   page_max);
    };
    // Loads the tile of rows t0..t0+15, rows past `cend` replaced by row
    // `cend` (so no masked row reads memory past the context); page_u is the
    // page of t0 (PAGE16).
    auto load_rows = [&](Tile& T, uint32_t t0, uint32_t cend, uint32_t page_u) {
        if constexpr (ROWS) {
            // Row loads: lane (q = lane/16, x = lane%16) reads the 16-byte chunk x
            // of the K and V head rows of tokens t0 + q + 4r (r < 4), so every 16
            // lanes read one whole 256-byte head row (whole 128-byte lines per
            // request). xpose() restores the MFMA operand layout through LDS.
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t p = min(t0 + grp + 4u * r, cend);
                const uint32_t page = PAGE16 ? page_u : min(gptr(pt)[p >> ly.log2p], page_max);
                const uint16_t* src =
                    pool + token_base(ly, layer, page, p & ly.pmask) + kvh * kD + 8u * tok;
                T.k[r] = ld16(src);
                T.v[r] = ld16(src + 256u);
            }
            return;
        }
        const uint32_t p = min(t0 + tok, cend);
        const uint32_t page = PAGE16 ? page_u : min(gptr(pt)[p >> ly.log2p], page_max);
        const uint16_t* src = pool + token_base(ly, layer, page, p & ly.pmask) + kvcol;
        if constexpr (VROWS) {  // K in operand layout, V as row loads
#pragma unroll
            for (int m = 0; m < 4; ++m) T.k[m] = ld16(src + 32u * m);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t pr = min(t0 + grp + 4u * r, cend);
                const uint32_t pg = PAGE16 ? page : min(gptr(pt)[pr >> ly.log2p], page_max);
                T.v[r] = ld16(pool + token_base(ly, layer, pg, pr & ly.pmask) + 256u +
                              kvh * kD + 8u * tok);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                T.k[m] = ld16(src + 32u * m);
                T.v[m] = ld16(src + 256u + 32u * m);
            }
        }
    };

    constexpr uint32_t RING = kRing;
    Tile R[RING];
    const uint32_t c_first = group * cpw;
    // Start-up in three memory rounds (the compiler otherwise loads kernel
    // arguments lazily, after the limit test, and waits for the staged page
    // ids with everything else: about six dependent rounds before the first
    // K/V request). Round 1: kernel arguments (the caller has them). Round 2,
    // all issued together: the limit, the page id of this wave's first tile
    // (its position does not depend on the limit), the page ids of the
    // range, q and the phase0 inputs. Round 3: the first K/V tile. The empty
    // asm statements with a memory clobber keep each round's requests ahead
    // of everything after them.
    const uint32_t t0_first = c_first * C + wave * kTile;
    uint32_t page_first_raw = 0u;  // clamped only after round 2 (no early wait)
    if constexpr (PAGE16 && TPW > 0u)
        page_first_raw = ((const __attribute__((address_space(4))) uint32_t*)(pt))
            [__builtin_amdgcn_readfirstlane(min(t0_first >> ly.log2p, page_max))];
    const uint32_t limit_raw =
        LSRC ? *(const __attribute__((address_space(4))) uint32_t*)(a.limit_src) : a.limit;
    // Page ids of the block's position range, staged once into LDS (read by
    // all tiles with a short LDS latency instead of a scalar-cache miss in
    // front of every tile's loads). Loaded for the range's full extent (cpw
    // chunks, indices clamped to the table) before the limit is known; only
    // entries below the range's last position are used.
    const uint32_t page0 = (c_first * C) >> ly.log2p;
    const uint32_t npages_full = ((c_first * C + cpw * C - 1u) >> ly.log2p) - page0 + 1u;
    uint32_t staged_raw = 0u;  // clamped at its LDS store
    if constexpr (PAGE16)
        staged_raw = gptr(pt)[min(page0 + min(tid, npages_full - 1u), page_max)];
    const bool real = tok < kGroup;
    // q: without phase0 each lane loads its Q^T operand directly; with phase0
    // thread tid loads dims p and p + 64 (p = tid % 64) of heads 2w, 2w + 1
    // (w = tid / 64) of this KV head, rotates them with pair p and stages the
    // rotated rows in LDS (4 rotations per thread instead of 32 per lane).
    uint4 qr[4];
    uint16_t qx[2][2];  // phase0: [head 2w + hh][dim p, p + 64]
    if constexpr (!PH0) {
        const uint16_t* qsrc = q_row + (kvh * kGroup + (real ? tok : 0u)) * kD + 8u * grp;
#pragma unroll
        for (int m = 0; m < 4; ++m) qr[m] = *reinterpret_cast<const uint4*>(qsrc + 32u * m);
    } else {
        const uint16_t* qh0 = q_row + (kvh * kGroup + 2u * wave) * kD + (tid & 63u);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            qx[hh][0] = qh0[hh * kD];
            qx[hh][1] = qh0[hh * kD + 64u];
        }
    }
    const uint32_t t64 = tid & 63u;
    float invf = 0.f;
    uint16_t kx = 0, kx2 = 0;
    uint32_t fresh_v = 0u;
    if (PH0) {  // every block reads the new token's k/v (a few cached bytes)
        invf = inv_freq[t64];
        const uint16_t* kr = q_row + kKCol + kvh * kD;
        kx = kr[t64];
        kx2 = kr[t64 + 64u];
        fresh_v = *reinterpret_cast<const uint32_t*>(q_row + kVCol + kvh * kD + 2u * t64);
    }
    // the limit, the first page id and the remaining arguments the K/V
    // addresses need arrive together (one wait, at the limit test below)
    asm volatile("" ::"s"(limit_raw), "s"(page_first_raw), "s"(pool), "s"(ly.pmask), "s"(layer)
                 : "memory");
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t page_first = min(page_first_raw, page_max);

    const uint32_t limit = min(limit_raw, a.pos_max);
    const uint32_t nvalid = min(limit / C + 1u, NC);
    if (c_first >= nvalid) return;  // uniform over the block
    const uint32_t c_end = min(c_first + cpw, nvalid);
    const bool direct = nvalid <= cpw;  // the only range: write the output

    // Position `limit` is kept out of the streamed tiles and added as one extra
    // tile from LDS by wave 0 of the owning block: with phase0 its K/V come
    // from the qkv row, otherwise from the pool. Both modes therefore run the
    // same arithmetic (phase0 output == append-then-attend output, bitwise) and
    // the streaming loop never patches registers.
    const uint32_t last_pos = limit - 1u;  // last streamed position
    auto chunk_end = [&](uint32_t c) { return min(c * C + C - 1u, last_pos); };
    auto chunk_tiles = [&](uint32_t c) {
        const uint32_t cs = c * C;
        return (limit == 0u || last_pos < cs) ? 0u : (chunk_end(c) - cs) / kTile + 1u;
    };
    const bool cached_pages = PAGE16 && npages_full <= kPageCache;
    // `from_table` reads the page id from the table itself (scalar path for
    // PAGE16) instead of the LDS copy; the first tiles use it so that they
    // do not wait for the staging barrier.
    auto load_tile = [&](Tile& T, uint32_t c, uint32_t j, bool from_table) {
        const uint32_t t0 = c * C + j * kTile;
        uint32_t page_u = 0u;
        if constexpr (PAGE16)
            page_u = (cached_pages && !from_table)
                         ? s_pages[__builtin_amdgcn_readfirstlane((t0 >> ly.log2p) - page0)]
                     : (TPW > 0u && (t0 >> ly.log2p) == (t0_first >> ly.log2p))
                         ? page_first
                         : table_page(t0);
        load_rows(T, t0, chunk_end(c), page_u);
    };
    // Row-loaded tile -> operand layout through this wave's LDS tile. A wave
    // reads only what it wrote, in order: no barrier is needed.
    //  * K (64-position tier): chunk x of token t at slot x ^ t of row t; the
    //    operand read (lane (row, group) takes dims [32m + 8*group, +8) of
    //    token row) touches one chunk of 16 rows per 16 lanes, all banks.
    //  * V: chunk x of token t at slot x ^ vswz(t), vswz(t) = 4*((t/2)%4) +
    //    t%2. Every 16-byte store instruction covers whole rows (conflict
    //    free for any per-row permutation); the 8-byte transposing reads of
    //    one instruction address tokens 4*grp + j and chunks 4m + a, and with
    //    this swizzle plus the half choice below the 32 lanes of rows 0..7
    //    hit 32 distinct 8-byte bank pairs (all 64 banks once; with 32 banks,
    //    the 16 lanes of rows 0..3 hit 16 distinct pairs). The former x ^ t
    //    swizzle put 8 rows on 8 slots and one half: a 4-way conflict.
    auto xpose = [&](const Tile& T) -> Tile {
        if constexpr (!VROWS) return T;
        uint4* xs = s_x[wave];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t t = grp + 4u * r;
            if constexpr (ROWS) xs[t * 16u + (tok ^ t)] = T.k[r];
            xs[256u + t * 16u + (tok ^ vswz(t))] = T.v[r];
        }
        __builtin_amdgcn_wave_barrier();
        Tile O;
        // V^T operands with the transposing LDS read: within each 16-lane
        // group, ds_read_b64_tr_b16 gives lane x the element x%4 of the 8-byte
        // rows addressed by lanes 4j + x/4 (j < 4). Lane 4j + a of group grp
        // addresses token 4*grp + j, chunk 4m + a, half h ^ (a & 1), so lane
        // x receives dim vdim(m, h, x/4) + x%4 of tokens 4*grp + j: the A
        // operand of O^T += V^T x P^T, row x of block (m, h) being dim
        // vdim(m, h, x/4) + x%4 (the accumulator rows follow the same map).
        const uint32_t vt_tok = 4u * grp + (tok >> 2);
        const uint32_t a4 = tok & 3u;
        const uint16_t* vs = reinterpret_cast<const uint16_t*>(xs + 256u) + vt_tok * 128u;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t x = (4u * m + grp) ^ tok;
            O.k[m] = ROWS ? xs[tok * 16u + x] : T.k[m];
            const uint16_t* vr = vs + (((4u * m + a4) ^ vswz(vt_tok)) * 8u);
            const uint32_t h0 = (a4 & 1u) * 4u;  // element offset of half 0
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(vr + h0));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(vr + (4u - h0)));
            const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
            O.v[m] = make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
        __builtin_amdgcn_wave_barrier();
        return O;
    };
    // Next (chunk, tile) of this wave after (c, j); false past the range.
    auto advance = [&](uint32_t& c, uint32_t& j) {
        j += kWaves;
        while (c < c_end && j >= chunk_tiles(c)) {
            ++c;
            j = wave;
        }
        return c < c_end;
    };
    // Straight-line schedule helper: tile i (0..TPW-1) of this wave in chunk
    // c, clamped to an existing tile past the end of the range (the clamped
    // load re-reads a tile and is never accumulated).
    auto clamp_load = [&](Tile& T, uint32_t c, uint32_t i, bool from_table) {
        const uint32_t cl = c < c_end ? c : c_end - 1u;
        const uint32_t nt = chunk_tiles(cl);
        uint32_t j = wave + 4u * i;
        if (c >= c_end) j = wave + 4u * (TPW - 1u);
        if (nt == 0u) j = 0u;
        else if (j >= nt) j = nt - 1u;
        load_tile(T, cl, j, from_table);
    };

    // Phase0: cos/sin of position `limit`; the block owning `limit` builds
    // the rotated K and the V of that token in LDS and stores both to the
    // pool. Without phase0 the owner reads K|V of `limit` from the pool.
    const bool owner = limit / C < c_end && limit < NC * C;
    uint2 fresh_kv = make_uint2(0u, 0u);
    uint32_t limit_page = 0u;
    Tile& A = R[0];
    Tile& B = R[RING > 1u ? 1u : 0u];
    uint32_t ac = c_first, aj = wave;
    bool a_ok = false;
    if constexpr (TPW > 0) {
#pragma unroll
        for (uint32_t g = 0; g + 1u < RING; ++g)
            clamp_load(R[g], c_first + g / TPW, g % TPW, true);
    } else {
        a_ok = wave < chunk_tiles(c_first) || advance(ac, aj);
        if (a_ok) load_tile(A, ac, aj, true);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (owner)
        limit_page =
            min(((const __attribute__((address_space(4))) uint32_t*)(pt))[limit >> ly.log2p],
                page_max);
    if (!PH0 && owner) {  // K|V of `limit` from the pool, 32 lanes per half
        const uint16_t* src =
            pool + token_base(ly, layer, limit_page, limit & ly.pmask) + kvh * kD;
        typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
        fresh_kv = __builtin_bit_cast(uint2, *reinterpret_cast<const MCKV_GLOBAL u32x2_t*>(
                                                 gptr(src + 256u * (t64 >> 5) + (t64 & 31u) * 4u)));
    }

    if (cached_pages && tid < npages_full) s_pages[tid] = min(staged_raw, page_max);
    if (PH0) {
        // cos/sin of pair p = tid % 64 (every wave evaluates the same 64)
        float c, sn;
        rope_sincos((float)limit * invf, &c, &sn);
        const uint32_t p = tid & 63u;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const float x = bf16_to_f32(qx[hh][0]), x2 = bf16_to_f32(qx[hh][1]);
            uint16_t* qd = &s_q[(2u * wave + hh) * kQPitch + p];
            qd[0] = f32_to_bf16(rope_rotate(x, x2, c, sn, true));
            qd[64] = f32_to_bf16(rope_rotate(x2, x, c, sn, false));
        }
        if (owner && tid < 64u) {  // pair tid rotates dims tid and tid + 64 of k
            const float x = bf16_to_f32(kx), x2 = bf16_to_f32(kx2);
            const uint16_t lo = f32_to_bf16(rope_rotate(x, x2, c, sn, true));
            const uint16_t hi = f32_to_bf16(rope_rotate(x2, x, c, sn, false));
            s_fresh[tid] = lo;
            s_fresh[tid + 64u] = hi;
            *reinterpret_cast<uint32_t*>(&s_fresh[128u + 2u * tid]) = fresh_v;
            MCKV_GLOBAL uint16_t* dst =
                gptr(pool + token_base(ly, layer, limit_page, limit & ly.pmask) + kvh * kD);
            dst[tid] = lo;
            dst[tid + 64u] = hi;
            *reinterpret_cast<MCKV_GLOBAL uint32_t*>(dst + 256u + 2u * tid) = fresh_v;
        }
    } else if (owner && tid < 64u) {
        const uint32_t h = tid >> 5, d = (tid & 31u) * 4u;
        *reinterpret_cast<uint2*>(&s_fresh[128u * h + d]) = fresh_kv;
    }
    __syncthreads();

    // Q^T B operand: lane holds q[head = tok][32m + 8*grp + i]; heads >= 8 zero.
    bf16x8 qb[4];
    if constexpr (PH0) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
            qr[m] = *reinterpret_cast<const uint4*>(
                &s_q[(real ? tok : 0u) * kQPitch + 32u * m + 8u * grp]);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) qb[m] = as_bf16x8(real ? qr[m] : make_uint4(0u, 0u, 0u, 0u));

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

    // Accumulates the tile starting at position `tstart` (rows after `tend`
    // masked) into the wave's state.
    auto accumulate = [&](const Tile& T, uint32_t tstart, uint32_t tend) {
        // S^T = K x Q^T
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m)
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(T.k[m]), qb[m], s, 0, 0, 0);
        const uint32_t pos0 = tstart + 4u * grp;
        float sc[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            float v;
            {
#pragma clang fp contract(off)
                v = s[jj] * kScoreScale;
            }
            sc[jj] = (pos0 + (uint32_t)jj <= tend) ? v : -INFINITY;
        }
        float tm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        tm = swap32_max(swap16_max(tm));
        const float mn = fmaxf(m_run, tm);
        const float renew = (m_run == -INFINITY) ? 0.f : __expf(m_run - mn);
        float p[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) p[jj] = __expf(sc[jj] - mn);
        float ls = (p[0] + p[1]) + (p[2] + p[3]);
        ls = swap32_sum(swap16_sum(ls));
        l_run = l_run * renew + ls;
        m_run = mn;
        s16x4 pb;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) pb[jj] = (short)f32_to_bf16(p[jj]);
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                s16x4 vop;
                if constexpr (VROWS) {  // T.v already holds the V^T operands
                    vop = half_s16x4(T.v[m], h);
                } else {
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    vop = trunc_bf16x4(__builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                        half_s16x4(T.v[m], h), ident, z, 0, 0, 0));
                }
                acc[m][h] = acc[m][h] * renew;
                if constexpr (FP32P) {
                    // fp32 P: four 16x16x4 fp32 MFMAs contract the positions
                    // {4g + i : g < 4} for i = 0..3. Lane (dim row r, g) holds
                    // V^T[r][4g + i] as element i of its V^T operand and
                    // P^T[4g + i][head] as p[i]; the output layout is the one
                    // of the bf16 16x16x16 product.
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[m][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            bf16_to_f32((uint16_t)vop[i]), p[i], acc[m][h], 0, 0, 0);
                } else {
                    acc[m][h] =
                        __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vop, pb, acc[m][h], 0, 0, 0);
                }
            }
    };

    if constexpr (TPW > 0) {
        // Straight-line schedule (C == 64 * TPW): wave w owns tiles
        // j = w + 4i, i < TPW, of every chunk. Chunks are walked with the tile
        // loop fully unrolled, so the ring slot of every tile is a
        // compile-time constant and the load of the next tile is issued
        // before the current one computes; the wait before each compute then
        // covers only the older load group. Loads for chunks past the range
        // are skipped (scalar branch; the compiler's wait counts stay
        // conservative across it), tiles past a chunk's end within the range
        // are clamped to an already-fetched tile and never accumulated.
        // U chunks are unrolled per loop trip so that U * TPW is a multiple
        // of the ring size and every slot index is a compile-time constant.
        constexpr uint32_t U = (TPW % RING == 0u) ? 1u : RING;
        static_assert((U * TPW) % RING == 0u, "ring slots must repeat per loop trip");
        for (uint32_t c = c_first; c < c_end; c += U) {
#pragma clang loop unroll(full)
            for (uint32_t h = 0; h < U; ++h) {
                const uint32_t cc2 = c + h;
#pragma clang loop unroll(full)
                for (uint32_t i = 0; i < TPW; ++i) {
                    const uint32_t g = h * TPW + i;
                    const uint32_t ga = g + RING - 1u;  // tile to prefetch
                    if (c + ga / TPW < c_end)
                        clamp_load(R[ga % RING], c + ga / TPW, ga % TPW, false);
                    const uint32_t j = wave + 4u * i;
                    if (h == 0u && i == 0u && a.stamp->stamps != nullptr && c == c_first &&
                        threadIdx.x < 64u) {
                        // timeline: clock at which the first tile's K/V are in
                        // registers (the wait the accumulate below needs anyway)
                        uint32_t k0 = R[0].k[0].x;
                        asm volatile("" : "+v"(k0));
                        if (threadIdx.x == 0u)
                            if (unsigned long long* p = a.stamp->slot())
                                p[3] = __builtin_amdgcn_s_memrealtime() + (k0 & 0u);
                    }
                    if (cc2 < c_end && j < chunk_tiles(cc2))
                        accumulate(xpose(R[g % RING]), cc2 * C + j * kTile, chunk_end(cc2));
                }
            }
        }
    } else {
        // Generic schedule (any C multiple of 16): ping-pong over two tiles.
        while (a_ok) {
            uint32_t bc = ac, bj = aj;
            const bool b_ok = advance(bc, bj);
            if (b_ok) load_tile(B, bc, bj, false);
            accumulate(xpose(A), ac * C + aj * kTile, chunk_end(ac));
            if (!b_ok) break;
            uint32_t nc = bc, nj = bj;
            a_ok = advance(nc, nj);
            if (a_ok) load_tile(A, nc, nj, false);
            accumulate(xpose(B), bc * C + bj * kTile, chunk_end(bc));
            ac = nc;
            aj = nj;
        }
    }
    if (owner && wave == 0u) {  // position `limit` from LDS
        Tile F;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            F.k[m] = *reinterpret_cast<const uint4*>(&s_fresh[32u * m + 8u * grp]);
            if constexpr (VROWS) {  // V^T operand: dim d of the token in every k slot
                uint32_t w[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t d = vdim(m, h, tok >> 2) + (tok & 3u);
                    w[h] = (uint32_t)s_fresh[128u + d] * 0x10001u;
                }
                F.v[m] = make_uint4(w[0], w[0], w[1], w[1]);
            } else {
                F.v[m] = *reinterpret_cast<const uint4*>(&s_fresh[128u + 32u * m + 8u * grp]);
            }
        }
        accumulate(F, limit, limit);
    }

    // Fold the 4 wave states in fixed wave order and write the record (or
    // the output).
    if (tok < kGroup) {
        if (grp == 0u) {
            s_m[wave][tok] = m_run;
            s_l[wave][tok] = l_run;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                *reinterpret_cast<f32x4*>(
                    &s_acc[wave][tok][VROWS ? vdim(m, h, grp) : 32u * m + 8u * grp + 4u * h]) =
                    acc[m][h];
    }
    __syncthreads();
    const uint32_t head = tid >> 5;        // 0..7
    const uint32_t d4 = (tid & 31u) * 4u;  // 4 dims
    const uint32_t qh = kvh * kGroup + head;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w)
        if (s_l[w][head] != 0.f) M = fmaxf(M, s_m[w][head]);
    float L = 0.f;
    f32x4 Acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) {
        const float lw = s_l[w][head];
        if (lw == 0.f) continue;
        const float f = __expf(s_m[w][head] - M);
        L += lw * f;
        Acc += *reinterpret_cast<const f32x4*>(&s_acc[w][head][d4]) * f;
    }
    if (direct) {
        uint16_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f32_to_bf16(L > 0.f ? Acc[i] / L : 0.f);
        *reinterpret_cast<uint2*>(a.out + qh * kD + d4) =
            make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16),
                       (uint32_t)o[2] | ((uint32_t)o[3] << 16));
        return;
    }
    if (a.split) {
        float* blk = a.rec + (size_t)qh * a.rec_stride * kPartial;
        float* pa = blk + (size_t)group * kD + d4;
        *reinterpret_cast<float2*>(pa) = make_float2(Acc[0], Acc[1]);
        *reinterpret_cast<float2*>(pa + 2) = make_float2(Acc[2], Acc[3]);
        if (d4 == 0u)
            *reinterpret_cast<float2*>(blk + (size_t)a.rec_stride * kD + 2u * group) =
                make_float2(M, L);
        return;
    }
    float* pw = a.rec + ((size_t)qh * a.rec_stride + group) * kPartial;
    if (d4 == 0u) *reinterpret_cast<float2*>(pw) = make_float2(M, L);
    *reinterpret_cast<float2*>(pw + 2 + d4) = make_float2(Acc[0], Acc[1]);
    *reinterpret_cast<float2*>(pw + 4 + d4) = make_float2(Acc[2], Acc[3]);
}

// Debug timeline (mc_kv_debug_decode_timeline): with a stamp buffer attached,
// workgroup w of a launch writes, at 4 * w of the launch's chunk region,
// {entry clock, exit clock, XCC id, first data clock}: the last is the clock
// at which the workgroup's first K/V tile reached registers (straight-line
// schedule; 0 otherwise); thread 0 stores the entry when the
// workgroup starts and every wave raises the exit to the clock at which it
// leaves (a vector atomic max). The clock is s_memrealtime (100 MHz, one
// count per 10 ns, common to all CUs). Workgroups past kTlChunkWgs are not
// recorded. stamps == nullptr (the default) costs one uniform branch at
// entry and at exit.
constexpr uint32_t kTlChunkWgs = 8192;
constexpr uint32_t kTlMergeWgs = 2048;
constexpr uint32_t kTlWordsPerLaunch = 4u * kTlChunkWgs + 2u * kTlMergeWgs;

// Merge region of a launch's timeline stamps (after the chunk region).
inline unsigned long long* merge_stamps(unsigned long long* chunk_stamps) {
    return chunk_stamps != nullptr ? chunk_stamps + 4u * kTlChunkWgs : nullptr;
}

// Records per head the record merge folds (chunks_per_range keeps ranges
// at or below it).
constexpr uint32_t kMaxRanges = 256;

// Last position the pool can hold (max_pages * P - 1, saturated to 32 bits).
__host__ __device__ __forceinline__ uint32_t pool_pos_max(const DevLayout& ly) {
    const uint64_t cap = (uint64_t)ly.max_pages << ly.log2p;
    return cap > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)(cap - 1u);
}

__device__ __forceinline__ uint32_t n_valid_chunks(uint32_t limit, uint32_t C,
                                                   uint32_t NC) {
    const uint32_t n = limit / C + 1u;
    return n > NC ? NC : n;
}

// grid = (ceil(NC / cpw), 2 kv heads (1 with KV2), B slots), one workgroup
// per range. Single-session launches pass B = 1 and the direct pointers;
// batched launches resolve per-slot pointers from device tables. Records of
// slot s start at partials + s * 16 * rec_stride * 130 with a per-head stride
// of rec_stride records (rec_stride >= the number of ranges, ceil(NC / cpw)).
template <bool PH0, bool BATCH, bool PAGE16, uint32_t TPW, bool KV2, bool FP32P, bool FIXED>
__global__ void __launch_bounds__(KV2 ? 2 * kThreads : kThreads)
    __attribute__((amdgpu_waves_per_eu(2))) decode_chunk_kernel(
    // The first 14 dwords (d_pos .. layer) are what a single-session
    // workgroup needs before its first K/V request; the decode translation
    // units are built with kernel-argument preloading, so these arrive in
    // SGPRs with the wave instead of through a scalar load round (the rest is
    // requested at entry and needed only later).
    const uint32_t* d_pos, const uint32_t* pt, const uint16_t* q_rows, const float* inv_freq,
    uint32_t ly_max_pages, uint32_t ly_log2p, uint32_t C, uint32_t cpw, uint32_t NC,
    uint32_t layer, uint16_t* pool, uint32_t ly_pmask, uint32_t ly_layers,
    const uint32_t* const* __restrict__ slot_pos, const uint32_t* const* __restrict__ slot_pt,
    uint16_t* const* __restrict__ slot_kv, float* __restrict__ partials, uint32_t rec_stride,
    uint16_t* __restrict__ out, uint32_t B, bool split, unsigned long long* stamps) {
    // Batched launches: every pointer argument is requested at entry, in one
    // round (the compiler otherwise loads some of them only where first used,
    // one dependent round each on the way to the first K/V request). Single
    // sessions find theirs preloaded.
    if constexpr (BATCH)
        asm volatile("" ::"s"(q_rows), "s"(slot_pos), "s"(slot_pt), "s"(slot_kv), "s"(inv_freq),
                     "s"(layer), "s"(ly_max_pages), "s"(ly_log2p), "s"(ly_pmask), "s"(C),
                     "s"(cpw), "s"(NC));
    const WgStamp stamp(stamps, 4u, kTlChunkWgs, true);
    const DevLayout ly{ly_max_pages, ly_log2p, ly_pmask, ly_layers};
    // Positions beyond the pool's capacity do not exist: a limit past it is
    // clamped, so page-table reads stay within its max_pages entries.
    const uint32_t pos_max = pool_pos_max(ly);
    const uint32_t kvh = KV2 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 8) : blockIdx.y;
    // lsrc: std::true_type when the body reads the limit from limit_src
    auto run = [&](auto lsrc, uint32_t slot, uint32_t group, uint32_t limit,
                   const uint32_t* limit_src) {
        DecodeArgs a;
        a.q_row = q_rows + (size_t)slot * kRow;
        a.limit = limit;
        a.pt = BATCH ? slot_pt[slot] : pt;
        a.pool = BATCH ? slot_kv[slot] : pool;
        a.rec = partials + (size_t)slot * kHq * rec_stride * kPartial;
        a.rec_stride = rec_stride;
        a.split = split;
        a.out = out + (size_t)slot * kHq * kD;
        a.stamp = &stamp;
        a.limit_src = limit_src;
        a.pos_max = pos_max;
        decode_range_body<PH0, PAGE16, TPW, KV2, FP32P, decltype(lsrc)::value>(
            a, layer, ly, NC, inv_freq, C, kvh, group, cpw);
    };
    if constexpr (BATCH) {
        if constexpr (FIXED) {
            // Small grids (every workgroup resident at once): workgroup
            // (slot, head, range) = (x, y, z), so the workgroup knows its slot
            // without reading every slot's limit first (one dependent load
            // round and the scan fewer before its first K/V; measured C3
            // 12.3 against 12.8 us/layer). Slot is the fastest index so the
            // early ranges of all slots are dispatched first.
            run(std::true_type{}, blockIdx.x, blockIdx.z, 0u, slot_pos[blockIdx.x]);
            return;
        }
        // Work compaction: the (x, slot) workgroups are numbered densely over
        // the chunk groups that exist (slot by slot, ascending), so ragged
        // slots leave their idle workgroups at the end of the grid instead of
        // between the working ones. Every wave derives the same mapping from
        // all slots' limits: lane s reads slot s's limit, a DPP scan gives
        // the running total of chunk groups, and the slot is the first one
        // whose total exceeds this workgroup's number. (A grid of one
        // residency round whose workgroups stride over the work was measured
        // slower: whole ranges are too coarse to balance that way.)
        const uint32_t Cc = TPW > 0u ? 64u * TPW : C;  // 64 * TPW: a shift
        const bool cpw_pow2 = (cpw & (cpw - 1u)) == 0u;
        const uint32_t cpw_log2 = (uint32_t)__builtin_ctz(cpw);
        auto groups = [&](uint32_t nv) {
            return cpw_pow2 ? (nv + cpw - 1u) >> cpw_log2 : (nv + cpw - 1u) / cpw;
        };
        const uint32_t lane = threadIdx.x & 63u;
        uint32_t lim = 0u, cnt = 0u;
        if (lane < B) {
            lim = min(*slot_pos[lane], pos_max);
            cnt = groups(n_valid_chunks(lim, Cc, NC));
        }
        // inclusive scan over the 64 lanes: row_shr 1, 2, 4, 8 within each
        // 16-lane row, then row_bcast 15 (into rows 1, 3) and 31 (rows 2, 3)
        uint32_t incl = cnt;
        incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, 0x111, 0xF, 0xF, false);
        incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, 0x112, 0xF, 0xF, false);
        incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, 0x114, 0xF, 0xF, false);
        incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, 0x118, 0xF, 0xF, false);
        incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, 0x142, 0xA, 0xF, false);
        incl += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)incl, 0x143, 0xC, 0xF, false);
        const uint32_t n = blockIdx.x + gridDim.x * blockIdx.z;
        const uint32_t slot = (uint32_t)__builtin_popcountll(
            __builtin_amdgcn_ballot_w64(lane < B && incl <= n));
        if (slot >= B) return;  // past the last existing chunk group (uniform)
        const uint32_t end = (uint32_t)__builtin_amdgcn_readlane((int)incl, (int)slot);
        const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)cnt, (int)slot);
        run(std::false_type{}, slot, n - (end - c),
            (uint32_t)__builtin_amdgcn_readlane((int)lim, (int)slot), nullptr);
    } else {
        run(std::true_type{}, 0u, blockIdx.x, 0u, d_pos);
    }
}

}  // namespace

// One chunk-kernel launch (records, or the output when there is one range).
struct ChunkLaunch {
    const uint16_t* q;
    const uint32_t* d_pos;
    const uint32_t* const* slot_pos;
    uint32_t B;
    uint32_t layer;
    const uint32_t* pt;
    const uint32_t* const* slot_pt;
    uint16_t* pool;
    uint16_t* const* slot_kv;
    DevLayout ly;
    float* partials;
    uint32_t NC;
    uint32_t rec_stride;
    uint16_t* out;
    hipStream_t st;
    const float* inv_freq;
    uint32_t C;
    uint32_t cpw;
    bool batched;
    bool split;                  // split record layout (DecodeArgs)
    unsigned long long* stamps;  // debug timeline: this launch's region, or nullptr
};

// Both KV heads in one 512-thread workgroup when that still gives every CU a
// workgroup: the 8 waves of a CU then stream the same token rows at the same
// pace (two independent workgroups per CU finish several us apart, and the
// later one runs alone at half the loads in flight). Batched launches keep
// one head per workgroup: their ragged slots leave many workgroups short,
// and finer ones balance better (measured).
inline bool use_kv2(const ChunkLaunch& L) {
    const uint32_t nx = (L.NC + L.cpw - 1u) / L.cpw;
    return !L.batched && (L.C == 256u || L.C == 512u) && nx >= kKv2MinBlocks;
}

// Batched grids of at most this many workgroups (two per CU) map workgroups
// to (slot, range) directly; larger ones, whose ragged slots leave many
// ranges idle, number the existing ranges densely (a direct mapping was
// measured 38 -> 111 us/layer at C5, idle workgroups delaying the long
// sessions' ranges).
constexpr uint32_t kFixedMapMaxWgs = 512;

template <bool PH0, bool BATCH, bool PAGE16, uint32_t TPW, bool KV2, bool FP32P>
void launch_one(const ChunkLaunch& L) {
    const uint32_t nx = (L.NC + L.cpw - 1u) / L.cpw;
    const uint32_t heads = KV2 ? 1u : kHkv;
    const bool fixed_map = BATCH && (uint64_t)nx * heads * L.B <= kFixedMapMaxWgs;
    const dim3 block(KV2 ? kHkv * kThreads : kThreads);
#define MC_CHUNK_LAUNCH(FX, GRID)                                                            \
    hipLaunchKernelGGL((decode_chunk_kernel<PH0, BATCH, PAGE16, TPW, KV2, FP32P, FX>), GRID,  \
                       block, 0, L.st, L.d_pos, L.pt, L.q, L.inv_freq, L.ly.max_pages,        \
                       L.ly.log2p, L.C, L.cpw, L.NC, L.layer, L.pool, L.ly.pmask,             \
                       L.ly.num_layers, L.slot_pos, L.slot_pt, L.slot_kv, L.partials,         \
                       L.rec_stride, L.out, L.B, L.split, L.stamps)
    if constexpr (BATCH && !KV2) {
        if (fixed_map) {
            MC_CHUNK_LAUNCH(true, dim3(L.B, heads, nx));
            return;
        }
    }
    MC_CHUNK_LAUNCH(false, dim3(nx, heads, L.B));
#undef MC_CHUNK_LAUNCH
}

template <bool PH0, bool BATCH, bool PAGE16, bool FP32P>
void launch_tiers(const ChunkLaunch& L) {
    bool kv2 = false;
    if constexpr (!BATCH) kv2 = use_kv2(L);
    switch (L.C) {
        case 64: launch_one<PH0, BATCH, PAGE16, 1u, false, FP32P>(L); break;
        case 128: launch_one<PH0, BATCH, PAGE16, 2u, false, FP32P>(L); break;
        case 256:
            if constexpr (!BATCH)
                if (kv2) { launch_one<PH0, BATCH, PAGE16, 4u, true, FP32P>(L); break; }
            launch_one<PH0, BATCH, PAGE16, 4u, false, FP32P>(L);
            break;
        case 512:
            if constexpr (!BATCH)
                if (kv2) { launch_one<PH0, BATCH, PAGE16, 8u, true, FP32P>(L); break; }
            launch_one<PH0, BATCH, PAGE16, 8u, false, FP32P>(L);
            break;
        default: launch_one<PH0, BATCH, PAGE16, 0u, false, FP32P>(L); break;
    }
}

// Launches the chunk kernel of L (instantiated once per P.V precision, each in
// its own translation unit).
template <bool FP32P>
mc_status_t launch_chunk_kernel(const ChunkLaunch& L) {
    const bool page16 = L.ly.log2p >= 4u;
    const bool ph0 = L.inv_freq != nullptr;
    if (L.batched) {
        if (ph0) {
            if (page16) launch_tiers<true, true, true, FP32P>(L);
            else launch_tiers<true, true, false, FP32P>(L);
        } else {
            if (page16) launch_tiers<false, true, true, FP32P>(L);
            else launch_tiers<false, true, false, FP32P>(L);
        }
    } else {
        if (ph0) {
            if (page16) launch_tiers<true, false, true, FP32P>(L);
            else launch_tiers<true, false, false, FP32P>(L);
        } else {
            if (page16) launch_tiers<false, false, true, FP32P>(L);
            else launch_tiers<false, false, false, FP32P>(L);
        }
    }
    return check_launch("decode attention launch failed");
}

extern template mc_status_t launch_chunk_kernel<false>(const ChunkLaunch&);
extern template mc_status_t launch_chunk_kernel<true>(const ChunkLaunch&);

}  // namespace mckv
