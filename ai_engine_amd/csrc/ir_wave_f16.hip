// ir_wave_f16.hip -- f16 instantiations of the one-tile-per-wavefront fused block.
#include "ir_wave_impl.h"

namespace aih {

hipError_t launch_ir_wave_f16(const IrWaveArgs &a, uint32_t npi, uint32_t waves, uint32_t lds, uint32_t grid,
                              hipStream_t st) {
  return irw_launch_dt<DT_F16>(a, npi, waves, lds, grid, st);
}

int ir_wave_occ_f16(uint32_t ke, uint32_t npi, uint32_t nob, bool rl, uint32_t waves, uint32_t lds) {
  return irw_occ_dt<DT_F16>(ke, npi, nob, rl, waves, lds);
}

hipError_t launch_ir_wave_stem_f16(const IrWaveArgs &a, uint32_t waves, uint32_t lds, uint32_t grid, hipStream_t st) {
  return irw_stem_launch<DT_F16>(a, waves, lds, grid, st);
}

int ir_wave_stem_occ_f16(uint32_t waves, uint32_t lds) { return irw_stem_occ<DT_F16>(waves, lds); }

}  // namespace aih
