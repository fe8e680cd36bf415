// gemv_fp8.hip -- the OCP e4m3-weight half of the decode GEMV kernel family
// (template in gemv_valu.h, launcher in gemv.hip), compiled as its own
// translation unit so the two halves build in parallel.
#include "gemv_valu.h"

namespace dbk {

GemvFn gemv_pick_fp8(GemvMode mode, int nb, int u) { return gemv_pick<true>(mode, nb, u); }

GemvFn gemv_pick_fp8_plain_long(int u) {
  switch (u) {
    case 1: return gemv_kernel<kGemvPlain, 1, 1, 1, true, kWavesFp8PlainLong>;
    case 2: return gemv_kernel<kGemvPlain, 1, 1, 2, true, kWavesFp8PlainLong>;
    case 4: return gemv_kernel<kGemvPlain, 1, 1, 4, true, kWavesFp8PlainLong>;
    case 7: return gemv_kernel<kGemvPlain, 1, 1, 7, true, kWavesFp8PlainLong>;
    default: return gemv_kernel<kGemvPlain, 1, 1, 8, true, kWavesFp8PlainLong>;
  }
}

}  // namespace dbk
