// ir_split_f16.hip -- f16 instantiations of the split fused block (one tile per workgroup).
#include "ir_split_impl.h"

namespace aih {

hipError_t launch_ir_split_f16(const IrWaveArgs &a, uint32_t npi, bool deep, uint32_t waves, uint32_t lds,
                              uint32_t grid, hipStream_t st) {
  return irs_launch_dt<DT_F16>(a, npi, deep, waves, lds, grid, st);
}

int ir_split_occ_f16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, bool deep, uint32_t waves, uint32_t lds) {
  return irs_occ_dt<DT_F16>(ke, npi, nob, rl, deep, waves, lds);
}

}  // namespace aih
