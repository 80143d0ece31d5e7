// synth.hip - deterministic synthetic qkv rows for the weight-free runtime.
//
// The model weights (qkv projection) are outside this build, so the session
// shell derives each qkv row from (token id, position, layer) with an integer
// hash. This lets mc_prefill / mc_decode_one / mc_batch_step drive the real KV
// path (append, paged attention, merge, advance) end to end. Values are
// uniform in [-1, 1) scaled by 1/2 and rounded to bf16.
#include <hip/hip_runtime.h>

#include "error.h"
#include "kv_common.h"
#include "kv_internal.h"

namespace mckv {
namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    // Murmur3 32-bit finalizer.
    x ^= x >> 16;
    x *= 0x85EBCA6Bu;
    x ^= x >> 13;
    x *= 0xC2B2AE35u;
    x ^= x >> 16;
    return x;
}

// Row r: token = tokens[r] (or *slot_tok[r]), pos = *base_pos + r (or
// *slot_pos[r]). grid = (rows), block = 320 threads x 8 columns.
template <bool BATCH>
__global__ void __launch_bounds__(320) synth_qkv_kernel(
    uint16_t* __restrict__ rows, const int32_t* __restrict__ tokens,
    const uint32_t* __restrict__ base_pos, const int32_t* const* __restrict__ slot_tok,
    const uint32_t* const* __restrict__ slot_pos, uint32_t layer) {
    const uint32_t r = blockIdx.x;
    const uint32_t tok = (uint32_t)(BATCH ? *slot_tok[r] : tokens[r]);
    const uint32_t pos = BATCH ? *slot_pos[r] : *base_pos + r;
    const uint32_t seed = mix32(tok * 0x9E3779B1u ^ mix32(pos + 0x632BE5ABu) ^
                                (layer * 0x85EBCA77u));
    const uint32_t c0 = threadIdx.x * 8u;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t h = mix32(seed ^ ((c0 + i) * 0x27D4EB2Fu));
        const float u = (float)(h >> 8) * (1.0f / 16777216.0f);  // [0, 1)
        v[i] = f32_to_bf16(u - 0.5f);
    }
    *reinterpret_cast<uint4*>(rows + (size_t)r * kRow + c0) =
        *reinterpret_cast<const uint4*>(v);
}

}  // namespace

mc_status_t launch_synth_qkv(uint16_t* rows, uint32_t n, const int32_t* tokens,
                             const uint32_t* base_pos, uint32_t layer, hipStream_t st) {
    hipLaunchKernelGGL(synth_qkv_kernel<false>, dim3(n), dim3(320), 0, st, rows, tokens,
                       base_pos, nullptr, nullptr, layer);
    return check_launch("synth_qkv launch failed");
}

mc_status_t launch_synth_qkv_batch(uint16_t* rows, uint32_t n,
                                   const int32_t* const* slot_tok,
                                   const uint32_t* const* slot_pos, uint32_t layer,
                                   hipStream_t st) {
    hipLaunchKernelGGL(synth_qkv_kernel<true>, dim3(n), dim3(320), 0, st, rows, nullptr,
                       nullptr, slot_tok, slot_pos, layer);
    return check_launch("synth_qkv_batch launch failed");
}

}  // namespace mckv
