// rope_append.hip - RoPE-fused K/V append for prefill chunks (and any T).
//
// Semantics of the reference rope_kv_kernel (native/kernels/sm120/rope_kv.cu:
// 30-96): token t sits at pos = *d_base_pos + t; q (16 heads) is rotated in
// place in its qkv row, k (2 heads) is rotated and stored to pool slot kv=0,
// v is copied bit-exactly to kv=1. rotate_half is non-interleaved: pair
// p = d mod 64, angle = (float)pos * inv_freq[p].
//
// MI355X mapping: one wave64 per token at a time. The 64 lanes first
// evaluate the 64 (cos, sin) pairs of the token once (lane = pair) into LDS.
// The token row (20 heads of 128 dims: 16 q, 2 k, 2 v) is moved as five 1 KB
// blocks, lane l holding 16 bytes of each; the rotate partner (dim d ^ 64) is
// 8 lanes away and comes through a DPP row rotate. A token's loads all
// precede its stores, so the in-place q update has no cross-lane hazard.
#include <hip/hip_runtime.h>

#include "error.h"
#include "trace.h"
#include "kv_common.h"
#include "kv_internal.h"

namespace mckv {
namespace {

constexpr uint32_t kWaves = 4;  // tokens per 256-thread block

// Partner lane of a rotate pair: dims d and d ^ 64 of a head sit 8 lanes
// apart within a 16-lane DPP row (row_ror:8 swaps lane i and i + 8).
__device__ __forceinline__ uint4 partner8(const uint4& v) {
    uint4 r;
    r.x = (uint32_t)__builtin_amdgcn_mov_dpp((int)v.x, 0x128, 0xF, 0xF, false);
    r.y = (uint32_t)__builtin_amdgcn_mov_dpp((int)v.y, 0x128, 0xF, 0xF, false);
    r.z = (uint32_t)__builtin_amdgcn_mov_dpp((int)v.z, 0x128, 0xF, 0xF, false);
    r.w = (uint32_t)__builtin_amdgcn_mov_dpp((int)v.w, 0x128, 0xF, 0xF, false);
    return r;
}

// Streaming 16-byte accesses: every qkv row and pool row is touched once per
// launch, so loads and stores are non-temporal (no cache allocation for
// data that is not re-read). Measured at C2 (8448 tokens): 19.4 us per
// launch with cached loads, 17.0 us with both non-temporal.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint16_t* p) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}
__device__ __forceinline__ void st_stream(uint16_t* p, const uint4& v) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(p));
}

// Grid cap: 2048 blocks x 4 waves = 8192 waves, one per SIMD slot of the
// 256 CUs at full occupancy (the kernel fits 8 waves per SIMD); larger
// chunks loop. An 8448-token chunk with one wave per token spills 256 waves
// into a second round (20.4 us); the capped, pipelined grid takes 17.0 us.
constexpr uint32_t kMaxBlocks = 2048;

// Each wave walks tokens t, t + W, ... (W = waves in the grid) and issues
// the next token's row loads before rotating and storing the current one,
// so the reads of one token overlap the writes of the previous.
__global__ void __launch_bounds__(256) rope_append_kernel(
    uint16_t* __restrict__ qkv, uint32_t tokens,
    const uint32_t* __restrict__ d_base_pos, uint32_t layer,
    const uint32_t* __restrict__ page_table, uint16_t* __restrict__ pool,
    DevLayout ly, float theta, const float* __restrict__ inv_freq) {
    __shared__ __align__(16) float s_cs[kWaves][64];
    __shared__ __align__(16) float s_sn[kWaves][64];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t W = gridDim.x * kWaves;
    uint32_t t = blockIdx.x * kWaves + wave;
    if (t >= tokens) return;  // wave-uniform; no block-wide barrier follows
    // Lane l covers bytes [16l, 16l + 16) of each 1 KB block b of the token
    // row: head 4b + l/16, dims 8*(l%16) .. +7. Every load and store
    // instruction moves 1 KB contiguous (the K/V block b = 4 is the pool's
    // 1 KB token row [K h0 | K h1 | V h0 | V h1]).
    const uint32_t x = lane & 15u;         // 8-dim block within the head
    const uint32_t pb = 8u * (x & 7u);     // first rotate pair of the lane
    const bool lo_half = x < 8u;           // dims < 64 of the head
    typedef const __attribute__((address_space(4))) uint32_t* scalar_u32p;
    const float f = inv_freq != nullptr ? inv_freq[lane]
                                        : (float)pow((double)theta, -(double)lane / 64.0);
    const uint32_t base = *(scalar_u32p)d_base_pos;
    uint4 v[5];
    {
        const uint16_t* row = qkv + (size_t)t * kRow;
#pragma unroll
        for (int b = 0; b < 5; ++b) v[b] = ld_stream(row + 512u * b + 8u * lane);
    }
    uint32_t page = clamp_page(ly, ((scalar_u32p)page_table)[table_index(ly, base + t)]);
    while (true) {
        const uint32_t tn = t + W;
        const bool more = tn < tokens;
        uint4 vn[5];
        uint32_t page_n = 0u;
        if (more) {
            const uint16_t* rown = qkv + (size_t)tn * kRow;
#pragma unroll
            for (int b = 0; b < 5; ++b) vn[b] = ld_stream(rown + 512u * b + 8u * lane);
            page_n = clamp_page(ly, ((scalar_u32p)page_table)[table_index(ly, base + tn)]);
        }
        const uint32_t pos = base + t;
        {  // (cos, sin) of pair `lane`, shared through this wave's LDS row
            float c, s;
            rope_sincos((float)pos * f, &c, &s);
            s_cs[wave][lane] = c;
            s_sn[wave][lane] = s;
        }
        __builtin_amdgcn_wave_barrier();
        float cs[8], sn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            cs[i] = s_cs[wave][pb + i];
            sn[i] = s_sn[wave][pb + i];
        }
        __builtin_amdgcn_wave_barrier();
        uint16_t* row = qkv + (size_t)t * kRow;
        uint16_t* dst = pool + token_base(ly, layer, page, pos & ly.pmask);
#pragma unroll
        for (int b = 0; b < 5; ++b) {
            const uint4 p2 = partner8(v[b]);
            uint4 o = v[b];
            if (b < 4 || lane < 32u) {  // q heads, k heads: rotate; v heads: copy
                const uint16_t* a = reinterpret_cast<const uint16_t*>(&v[b]);
                const uint16_t* a2 = reinterpret_cast<const uint16_t*>(&p2);
                uint16_t* oo = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    oo[i] = f32_to_bf16(rope_rotate(bf16_to_f32(a[i]), bf16_to_f32(a2[i]), cs[i],
                                                    sn[i], lo_half));
            }
            st_stream((b < 4 ? row + 512u * b : dst) + 8u * lane, o);
        }
        if (!more) break;
#pragma unroll
        for (int b = 0; b < 5; ++b) v[b] = vn[b];
        page = page_n;
        t = tn;
    }
}

__global__ void inv_freq_init_kernel(float* __restrict__ table, double theta) {
    const uint32_t p = threadIdx.x;
    if (p < 64u) table[p] = (float)pow(theta, -(double)p / 64.0);
}

}  // namespace
}  // namespace mckv

extern "C" mc_status_t mc_kv_rope_inv_freq_init(float* d_table, double rope_theta,
                                                void* stream) {
    mckv::TraceRange trace_range("mc_kv_rope_inv_freq_init");
    if (d_table == nullptr || !(rope_theta > 0.0)) {
        mckv::set_error("mc_kv_rope_inv_freq_init: table=%p theta=%g",
                        (void*)d_table, rope_theta);
        return MC_E_INVALID_ARGUMENT;
    }
    hipLaunchKernelGGL(mckv::inv_freq_init_kernel, dim3(1), dim3(64), 0,
                       (hipStream_t)stream, d_table, (double)(float)rope_theta);
    return mckv::check_launch("rope inv_freq init launch failed");
}

extern "C" mc_status_t mc_kv_rope_append(uint16_t* d_qkv, uint32_t tokens,
                                         const uint32_t* d_base_pos, uint32_t layer,
                                         const uint32_t* d_page_table,
                                         uint16_t* d_kv_pool, mc_kv_layout_t layout,
                                         double rope_theta, const float* d_inv_freq,
                                         void* stream) {
    mckv::TraceRange trace_range("mc_kv_rope_append");
    mckv::DevLayout ly;
    if (d_qkv == nullptr || d_base_pos == nullptr || d_page_table == nullptr ||
        d_kv_pool == nullptr || tokens == 0 || !mckv::layout_valid(layout, &ly) ||
        layer >= layout.num_layers ||
        (d_inv_freq == nullptr && !(rope_theta > 0.0))) {
        mckv::set_error("mc_kv_rope_append: invalid args (tokens=%u layer=%u)",
                        tokens, layer);
        return MC_E_INVALID_ARGUMENT;
    }
    uint32_t blocks = (tokens + mckv::kWaves - 1u) / mckv::kWaves;
    if (blocks > mckv::kMaxBlocks) blocks = mckv::kMaxBlocks;
    hipLaunchKernelGGL(mckv::rope_append_kernel, dim3(blocks), dim3(256), 0,
                       (hipStream_t)stream, d_qkv, tokens, d_base_pos, layer,
                       d_page_table, d_kv_pool, ly, (float)rope_theta, d_inv_freq);
    return mckv::check_launch("rope_append launch failed");
}
