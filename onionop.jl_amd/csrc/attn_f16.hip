// attn_f16.hip -- forward and backward attention kernels for element type f16
// (one translation unit per element type so the library builds in parallel).
#include "attn_fwd.inc"
#include "attn_bwd.inc"

namespace onionop {
template bool fwd_dispatch<f16>(hipStream_t, const AttnArgs&);
template bool bwd_dispatch<f16, false>(hipStream_t, const AttnArgs&, int);
}  // namespace onionop
