// gfx950 MFMA matmul tiles (f16 / bf16 operands, f32 accumulation).
#include "ktir_common.h"

int ktir_launch_matmul_mfma(const ktir_mm_t* d, bool* handled) {
  (void)d;
  *handled = false;
  return KTIR_OK;
}
