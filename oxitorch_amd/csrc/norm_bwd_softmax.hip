// The norm VJPs with a softmax or log_softmax over the row folded in.
#include "norm_bwd_impl.h"

namespace oxi {

int norm_bwd_softmax(int act, bool ln, int mode, const NormBwdArgs& a) {
  return act == OXI_ACT_SOFTMAX ? norm_bwd_dispatch<OXI_ACT_SOFTMAX>(ln, mode, a)
                                : norm_bwd_dispatch<OXI_ACT_LOG_SOFTMAX>(ln, mode, a);
}

}  // namespace oxi
