// attn_f32x6.hip -- the float32 attention kernels with every MFMA product computed as six
// bf16 products of an exact three-way bf16 split (Mfma<float> under ONIONOP_X6,
// attn_common.h): element type code ONIONOP_F32_BF16X6.  The kernels are the float32
// ones, compiled a second time inside namespace onionop_x6 so that the two policies never
// share a symbol.
#include "launch.h"  // onionop::AttnArgs and the launcher interface

namespace onionop_base = onionop;

#define ONIONOP_X6 1
#define onionop onionop_x6
namespace onionop {
using namespace onionop_base;
}
#include "attn_fwd.inc"
#include "attn_bwd.inc"

namespace onionop {
bool fwd_f32x6(hipStream_t s, const AttnArgs& a) { return fwd_dispatch<float>(s, a); }
bool bwd_f32x6(hipStream_t s, const AttnArgs& a, int stages) {
    return a.qk_fp16 ? bwd_dispatch<float, true>(s, a, stages) : bwd_dispatch<float, false>(s, a, stages);
}
}  // namespace onionop
#undef onionop
