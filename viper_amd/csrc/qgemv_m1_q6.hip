// M = 1 GEMV kernels of format 6 (the template is in qgemv_m1.h).
#include "qgemv_m1.h"

namespace vq {

VQ_M1_PICK(6)

}  // namespace vq
