// M = 1 GEMV kernels of format 4, rmsnorm and swiglu prologues (the template is in qgemv_m1.h).
#include "qgemv_m1.h"

namespace vq {

VQ_M1_FOLDED(4)

}  // namespace vq
