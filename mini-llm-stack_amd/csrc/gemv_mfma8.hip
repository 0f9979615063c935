// The skinny MFMA GEMM's INT8 kernels (gemv_mfma.h), compiled without the code generation
// option of the INT4 kernels (csrc/build.py): with MFMA results in VGPRs they ran slower.
#include "gemv_mfma.h"

namespace mls {

int launch_gemv_mfma_int8(const WqArgs& p) {
  return p.a_dt == MLS_BF16 ? launch_st<8, __bf16>(p) : launch_st<8, _Float16>(p);
}

int launch_gemv_mfma_split_int8(const WqArgs& q) { return launch_st<8, __bf16, false, true>(q); }

int launch_gemv_mfma_f32_int8(const WqArgs& p) { return launch_st<8, __bf16, false, true, true>(p); }

}  // namespace mls
