// conv_gemm_bf16.hip -- conv-GEMM instantiations for bf16 activations and
// weights (bf16 MFMA, fp32 accumulation); PAIR selects 16-byte A loads.
#include "conv_gemm_launch.h"

namespace aih {

hipError_t launch_conv_gemm_bf16(const GemmArgs &a, int bn, bool igemm, bool pair, hipStream_t st) {
  if (igemm) {
    if (pair) {
      AIH_GEMM_BN_SWITCH(DT_BF16, DT_BF16, true, true, bn, a, st)
    } else {
      AIH_GEMM_BN_SWITCH(DT_BF16, DT_BF16, true, false, bn, a, st)
    }
  } else {
    if (pair) {
      AIH_GEMM_BN_SWITCH(DT_BF16, DT_BF16, false, true, bn, a, st)
    } else {
      AIH_GEMM_BN_SWITCH(DT_BF16, DT_BF16, false, false, bn, a, st)
    }
  }
}

}  // namespace aih
