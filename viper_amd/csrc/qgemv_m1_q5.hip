// M = 1 GEMV kernels of format 5, quantize and int8 prologues (the template is in qgemv_m1.h).
#include "qgemv_m1.h"

namespace vq {

VQ_M1_PLAIN(5)

}  // namespace vq
