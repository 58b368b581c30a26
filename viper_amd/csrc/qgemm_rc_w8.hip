// Row-contiguous matrix-core kernels of format 8 (the template is in qgemm_rc.h).
#include "qgemm_rc.h"

namespace vq {

VQ_RC_PICK(8)

}  // namespace vq
