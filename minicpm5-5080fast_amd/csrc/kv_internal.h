// kv_internal.h - declarations shared by the host-side translation units.
#pragma once

#include "kv_common.h"

namespace mckv {

// Validates an mc_kv_layout_t (power-of-two page size, non-zero sizes) and
// fills the device view.
bool layout_valid(const mc_kv_layout_t& l, DevLayout* out);

}  // namespace mckv
