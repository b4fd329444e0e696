// The norm VJPs with a tanh or erf GELU folded in.
#include "norm_bwd_impl.h"

namespace oxi {

int norm_bwd_gelu(int act, bool ln, int mode, const NormBwdArgs& a) {
  return act == OXI_ACT_GELU_TANH ? norm_bwd_dispatch<OXI_ACT_GELU_TANH>(ln, mode, a)
                                  : norm_bwd_dispatch<OXI_ACT_GELU_ERF>(ln, mode, a);
}

}  // namespace oxi
