// kv_internal.h - declarations shared by the host-side translation units.
#pragma once

#include "kv_common.h"

namespace mckv {

// Validates an mc_kv_layout_t (power-of-two page size, non-zero sizes) and
// fills the device view.
bool layout_valid(const mc_kv_layout_t& l, DevLayout* out);

}  // namespace mckv

namespace mckv {

// Deterministic synthetic qkv rows (synth.hip).
mc_status_t launch_synth_qkv(uint16_t* rows, uint32_t n, const int32_t* tokens,
                             const uint32_t* base_pos, uint32_t layer, hipStream_t st);
mc_status_t launch_synth_qkv_batch(uint16_t* rows, uint32_t n,
                                   const int32_t* const* slot_tok,
                                   const uint32_t* const* slot_pos, uint32_t layer,
                                   hipStream_t st);

// Prefill half-barrier status (attention_prefill.hip): after the caller's
// prefill work has been synchronized, reads and clears the device's timeout
// count; MC_E_INTERNAL (with a message) when it is non-zero.
mc_status_t prefill_barrier_check(const char* who);

}  // namespace mckv
