// rope_append.hip - RoPE-fused K/V append for prefill chunks (and any T).
//
// Semantics of the reference rope_kv_kernel (native/kernels/sm120/rope_kv.cu:
// 30-96): token t sits at pos = *d_base_pos + t; q (16 heads) is rotated in
// place in its qkv row, k (2 heads) is rotated and stored to pool slot kv=0,
// v is copied bit-exactly to kv=1. rotate_half is non-interleaved: pair
// p = d mod 64, angle = (float)pos * inv_freq[p].
//
// MI355X mapping: one wave64 per token. The 64 lanes first evaluate the 64
// (cos, sin) pairs of the token once (lane = pair) into LDS. Then lane
// (g = lane/8, j = lane%8) owns dims [8j, 8j+8) and their rotate partners
// [64+8j, 64+8j+8) of "head" g, g+8, g+16 (20 heads = 16 q + 2 k + 2 v), so
// every global access is a 16-byte load/store and 8 lanes cover one 128-byte
// half-head: fully coalesced. A lane reads both halves before writing either,
// so the in-place q update has no cross-lane hazard.
#include <hip/hip_runtime.h>

#include "error.h"
#include "kv_common.h"
#include "kv_internal.h"

namespace mckv {
namespace {

constexpr uint32_t kWaves = 4;  // tokens per 256-thread block

__device__ __forceinline__ void rotate8(const uint4& lo, const uint4& hi,
                                        const float* cs, const float* sn,
                                        uint4& olo, uint4& ohi) {
    const uint16_t* a = reinterpret_cast<const uint16_t*>(&lo);
    const uint16_t* b = reinterpret_cast<const uint16_t*>(&hi);
    uint16_t* oa = reinterpret_cast<uint16_t*>(&olo);
    uint16_t* ob = reinterpret_cast<uint16_t*>(&ohi);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x = bf16_to_f32(a[i]);
        const float x2 = bf16_to_f32(b[i]);
        oa[i] = f32_to_bf16(rope_rotate(x, x2, cs[i], sn[i], true));
        ob[i] = f32_to_bf16(rope_rotate(x2, x, cs[i], sn[i], false));
    }
}

__global__ void __launch_bounds__(256) rope_append_kernel(
    uint16_t* __restrict__ qkv, uint32_t tokens,
    const uint32_t* __restrict__ d_base_pos, uint32_t layer,
    const uint32_t* __restrict__ page_table, uint16_t* __restrict__ pool,
    DevLayout ly, float theta, const float* __restrict__ inv_freq) {
    __shared__ __align__(16) float s_cs[kWaves][64];
    __shared__ __align__(16) float s_sn[kWaves][64];
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * kWaves + wave;
    const bool active = t < tokens;
    const uint32_t g = lane >> 3;  // head group 0..7
    const uint32_t j = lane & 7u;  // 8-dim block within the half head
    // Loads are issued in the order their results are needed and none waits
    // for another: inv_freq (vector), then the row (6 x 16 bytes per lane;
    // an inactive wave reads token 0's row, lanes past head 19 re-read head
    // 19), while the base position and the page id come through the scalar
    // path. The cos/sin evaluation then overlaps the row loads.
    typedef const __attribute__((address_space(4))) uint32_t* scalar_u32p;
    const float f = inv_freq != nullptr ? inv_freq[lane]
                                        : (float)pow((double)theta, -(double)lane / 64.0);
    uint16_t* row = qkv + (size_t)(active ? t : 0u) * kRow;
    uint4 lo[3], hi[3];
#pragma unroll
    for (uint32_t it = 0; it < 3; ++it) {
        const uint32_t h = min(g + 8u * it, 19u);  // 0..15 q, 16..17 k, 18..19 v
        const uint16_t* src = row + h * 128u;  // q, k and v heads are contiguous
        lo[it] = *reinterpret_cast<const uint4*>(src + 8u * j);
        hi[it] = *reinterpret_cast<const uint4*>(src + 64u + 8u * j);
    }
    const uint32_t base = *(scalar_u32p)d_base_pos;
    const uint32_t pos = base + t;
    const uint32_t tok_pos = __builtin_amdgcn_readfirstlane(active ? pos : base);
    const uint32_t page = ((scalar_u32p)page_table)[tok_pos >> ly.log2p];
    {
        float c, s;
        rope_sincos((float)pos * f, &c, &s);
        s_cs[wave][lane] = c;
        s_sn[wave][lane] = s;
    }
    __syncthreads();
    if (!active) return;

    float cs[8], sn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        cs[i] = s_cs[wave][8u * j + i];
        sn[i] = s_sn[wave][8u * j + i];
    }
    uint16_t* dst = pool + token_base(ly, layer, page, pos & ly.pmask);

#pragma unroll
    for (uint32_t it = 0; it < 3; ++it) {
        const uint32_t h = g + 8u * it;
        if (h >= 20u) break;
        uint16_t* src = row + h * 128u;
        if (h < 18u) {
            uint4 olo, ohi;
            rotate8(lo[it], hi[it], cs, sn, olo, ohi);
            uint16_t* o = (h < 16u) ? src : dst + (h - 16u) * 128u;
            *reinterpret_cast<uint4*>(o + 8u * j) = olo;
            *reinterpret_cast<uint4*>(o + 64u + 8u * j) = ohi;
        } else {
            uint16_t* o = dst + 256u + (h - 18u) * 128u;
            *reinterpret_cast<uint4*>(o + 8u * j) = lo[it];
            *reinterpret_cast<uint4*>(o + 64u + 8u * j) = hi[it];
        }
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
    mckv::DevLayout ly;
    if (d_qkv == nullptr || d_base_pos == nullptr || d_page_table == nullptr ||
        d_kv_pool == nullptr || tokens == 0 || !mckv::layout_valid(layout, &ly) ||
        layer >= layout.num_layers ||
        (d_inv_freq == nullptr && !(rope_theta > 0.0))) {
        mckv::set_error("mc_kv_rope_append: invalid args (tokens=%u layer=%u)",
                        tokens, layer);
        return MC_E_INVALID_ARGUMENT;
    }
    const uint32_t blocks = (tokens + mckv::kWaves - 1u) / mckv::kWaves;
    hipLaunchKernelGGL(mckv::rope_append_kernel, dim3(blocks), dim3(256), 0,
                       (hipStream_t)stream, d_qkv, tokens, d_base_pos, layer,
                       d_page_table, d_kv_pool, ly, (float)rope_theta, d_inv_freq);
    return mckv::check_launch("rope_append launch failed");
}
