// The norm VJPs without a folded activation.
#include "norm_bwd_impl.h"

namespace oxi {

int norm_bwd_none(bool ln, int mode, const NormBwdArgs& a) { return norm_bwd_dispatch<OXI_ACT_NONE>(ln, mode, a); }

}  // namespace oxi
