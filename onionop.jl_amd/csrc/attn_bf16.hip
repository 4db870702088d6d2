// attn_bf16.hip -- forward and backward attention kernels for element type bf16
// (one translation unit per element type so the library builds in parallel).
#include "attn_fwd.inc"
#include "attn_bwd.inc"

namespace onionop {
template bool fwd_dispatch<bf16>(hipStream_t, const AttnArgs&);
template bool bwd_dispatch<bf16, false>(hipStream_t, const AttnArgs&, int);
}  // namespace onionop
