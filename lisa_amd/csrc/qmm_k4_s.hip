// Instantiations of the qmm kernel for 4-bit codes, split-K partial output
// (one of four translation units compiled in parallel; the kernel is in qmm_kernel.h).
#include "qmm_kernel.h"

namespace lisaq {

template <>
qmm_fn qmm_get<4, true>(int gs, int MT, int* lds) {
  return qmm_get_impl<4, true>(gs, MT, lds);
}

}  // namespace lisaq
