// attn_f32.hip -- forward and backward attention kernels for element type float
// (one translation unit per element type so the library builds in parallel).
#include "attn_fwd.inc"
#include "attn_bwd.inc"

namespace onionop {
template bool fwd_dispatch<float>(hipStream_t, const AttnArgs&);
template bool bwd_dispatch<float, false>(hipStream_t, const AttnArgs&, int);
template bool bwd_dispatch<float, true>(hipStream_t, const AttnArgs&, int);
}  // namespace onionop
