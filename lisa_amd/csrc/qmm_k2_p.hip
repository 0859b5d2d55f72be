// Instantiations of the qmm kernel for 2-bit codes, plain output
// (one of four translation units compiled in parallel; the kernel is in qmm_kernel.h).
#include "qmm_kernel.h"

namespace lisaq {

template <>
qmm_fn qmm_get<2, false>(int gs, int MT, int* lds) {
  return qmm_get_impl<2, false>(gs, MT, lds);
}

}  // namespace lisaq
