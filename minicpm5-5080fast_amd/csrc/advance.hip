// advance.hip - device-side sequence advance after a decode step, so the next
// step's `limit` moves without host involvement (reference sampling.cu:58-67
// decode_advance_kernel and :241-251 batch_advance_kernel).
#include <hip/hip_runtime.h>

#include "error.h"
#include "trace.h"
#include "kv_common.h"

namespace mckv {
namespace {

__global__ void decode_advance_kernel(int32_t* __restrict__ seq,
                                      const int32_t* __restrict__ next_token,
                                      uint32_t* __restrict__ seq_len) {
    const uint32_t p = *seq_len;
    seq[p] = *next_token;
    *seq_len = p + 1u;
}

__global__ void batch_advance_kernel(int32_t* const* __restrict__ slot_seq,
                                     const int32_t* const* __restrict__ slot_tok,
                                     uint32_t* const* __restrict__ slot_pos,
                                     uint32_t n) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const uint32_t p = *slot_pos[s];
    slot_seq[s][p] = *slot_tok[s];
    *slot_pos[s] = p + 1u;
}

}  // namespace
}  // namespace mckv

extern "C" mc_status_t mc_kv_decode_advance(int32_t* d_seq, const int32_t* d_next_token,
                                            uint32_t* d_seq_len, void* stream) {
    mckv::TraceRange trace_range("mc_kv_decode_advance");
    if (d_seq == nullptr || d_next_token == nullptr || d_seq_len == nullptr) {
        mckv::set_error("mc_kv_decode_advance: NULL argument");
        return MC_E_INVALID_ARGUMENT;
    }
    hipLaunchKernelGGL(mckv::decode_advance_kernel, dim3(1), dim3(1), 0,
                       (hipStream_t)stream, d_seq, d_next_token, d_seq_len);
    return mckv::check_launch("decode_advance launch failed");
}

extern "C" mc_status_t mc_kv_batch_advance(int32_t* const* d_slot_seq,
                                           const int32_t* const* d_slot_tok,
                                           uint32_t* const* d_slot_pos, uint32_t n,
                                           void* stream) {
    mckv::TraceRange trace_range("mc_kv_batch_advance");
    if (d_slot_seq == nullptr || d_slot_tok == nullptr || d_slot_pos == nullptr ||
        n == 0) {
        mckv::set_error("mc_kv_batch_advance: invalid args (n=%u)", n);
        return MC_E_INVALID_ARGUMENT;
    }
    hipLaunchKernelGGL(mckv::batch_advance_kernel, dim3((n + 63u) / 64u), dim3(64), 0,
                       (hipStream_t)stream, d_slot_seq, d_slot_tok, d_slot_pos, n);
    return mckv::check_launch("batch_advance launch failed");
}
