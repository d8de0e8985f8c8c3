// dw_pw_bf16.hip -- the bf16 instantiations of the fused depthwise ->
// pointwise kernel (dw_pw_impl.h), a translation unit of their own so the
// dtypes build in parallel.
#include "dw_pw_impl.h"

namespace aih {

hipError_t launch_dw_pw_bf16(const DwPwArgs &a, uint32_t k, uint32_t s, uint32_t rows, uint32_t waves, uint32_t lds,
                            uint32_t grid, hipStream_t st) {
  return dp_launch_dt<DT_BF16>(a, k, s, rows, waves, lds, grid, st);
}

int dw_pw_occ_bf16(uint32_t k, uint32_t s, uint32_t no, uint32_t rows, bool cl, uint32_t waves, uint32_t lds) {
  return dp_occ_dt<DT_BF16>(k, s, no, rows, cl, waves, lds);
}

}  // namespace aih
