// Row-contiguous matrix-core kernels of format 8 (the template is in qgemm_rc.h).
#include "qgemm_rc.h"

namespace vq {

VQ_RC_PICK(8)
rc_fn rc_pick_tl8(const RcShape& s, int senc) { return rc_pick_tl<8>(s, senc); }

}  // namespace vq
