// Row-contiguous matrix-core kernels of format 4 (the template is in qgemm_rc.h).
#include "qgemm_rc.h"

namespace vq {

VQ_RC_PICK(4)
rc_fn rc_pick_tl4(const RcShape& s, int senc) { return rc_pick_tl<4>(s, senc); }

}  // namespace vq
