// decode_fp32p.hip - instantiates the decode kernels with fp32 P (the reference's MC_ATTN_HMMA_OFF semantics, P not rounded before P.V).
#include "decode_kernels.h"

namespace mckv {
template mc_status_t launch_chunk_kernel<true>(const ChunkLaunch&);
}  // namespace mckv
