// ir_block_f16.hip -- fused inverted-residual block instantiations, f16 storage.
#include "ir_block_impl.h"

namespace aih {

hipError_t launch_ir_block_f16(const IrArgs &a, uint32_t lds, uint32_t grid, hipStream_t st) {
  return ir_launch_dt<DT_F16>(a, lds, grid, st);
}

int ir_occ_f16(uint32_t nob, uint32_t npw, bool cl, uint32_t lds) {
  return ir_occ_dt<DT_F16>(nob, npw, cl, lds);
}

}  // namespace aih
