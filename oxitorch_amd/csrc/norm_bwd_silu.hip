// The norm VJPs with a SiLU folded in.
#include "norm_bwd_impl.h"

namespace oxi {

int norm_bwd_silu(bool ln, int mode, const NormBwdArgs& a) { return norm_bwd_dispatch<OXI_ACT_SILU>(ln, mode, a); }

}  // namespace oxi
