// decode_bf16p.hip - instantiates the decode kernels with bf16 P (P rounded to bf16 before P.V, the reference's default HMMA path).
#include "decode_kernels.h"

namespace mckv {
template mc_status_t launch_chunk_kernel<false>(const ChunkLaunch&);
}  // namespace mckv
