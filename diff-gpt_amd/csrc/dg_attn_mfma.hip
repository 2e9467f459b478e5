// bf16 MFMA prefill attention (gfx950).  Placeholder until the tiled kernel
// lands: every shape goes to the vector kernel.
#include "dg_common.h"

namespace dg {

bool mfma_prefill_applicable(int, int, int, int, int, int, const void*, const dg_stride3*,
                             const void*, const dg_stride3*, const void*, const dg_stride3*,
                             const void*, const dg_stride3*) {
  return false;
}

int mfma_prefill(int, int, int, int, int, int, const void*, const dg_stride3*, const void*,
                 const dg_stride3*, const void*, const dg_stride3*, void*, const dg_stride3*, float,
                 hipStream_t) {
  set_error("mfma_prefill: not built");
  return DG_EUNSUPPORTED;
}

}  // namespace dg
