// Row-contiguous matrix-core kernels of format 5 (the template is in qgemm_rc.h).
#include "qgemm_rc.h"

namespace vq {

VQ_RC_PICK(5)

}  // namespace vq
