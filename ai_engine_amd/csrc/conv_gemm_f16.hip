// conv_gemm_f16.hip -- conv-GEMM instantiations for f16 activations and
// weights (f16 MFMA, fp32 accumulation); PAIR selects 16-byte A loads.
#include "conv_gemm_launch.h"

namespace aih {

hipError_t launch_conv_gemm_f16(const GemmArgs &a, int bn, bool igemm, bool pair, hipStream_t st) {
  if (igemm) {
    if (pair) {
      AIH_GEMM_BN_SWITCH(DT_F16, DT_F16, true, true, bn, a, st)
    } else {
      AIH_GEMM_BN_SWITCH(DT_F16, DT_F16, true, false, bn, a, st)
    }
  } else {
    if (pair) {
      AIH_GEMM_BN_SWITCH(DT_F16, DT_F16, false, true, bn, a, st)
    } else {
      AIH_GEMM_BN_SWITCH(DT_F16, DT_F16, false, false, bn, a, st)
    }
  }
}

}  // namespace aih
