// gemv_fp8.hip -- the OCP e4m3-weight half of the decode GEMV kernel family
// (template in gemv_valu.h, launcher in gemv.hip), compiled as its own
// translation unit so the two halves build in parallel.
#include "gemv_valu.h"

namespace dbk {

GemvFn gemv_pick_fp8(GemvMode mode, int nb, int u) { return gemv_pick<true>(mode, nb, u); }

}  // namespace dbk
