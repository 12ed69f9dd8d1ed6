// gemm16_f16.hip — instantiates the direct-to-LDS MFMA GEMM (gemm16_impl.hpp)
// for f16 operands.
#include "gemm16_impl.hpp"

namespace mlxhip {

int gemm16_f16(int c_dtype, int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s) {
    using namespace gemm16;
    if (c_dtype == MLXHIP_DTYPE_F32) return dispatch<MLXHIP_DTYPE_F16, MLXHIP_DTYPE_F32>(a, batch, ta, tb, cfg, s);
    if (c_dtype == MLXHIP_DTYPE_F16) return dispatch<MLXHIP_DTYPE_F16, MLXHIP_DTYPE_F16>(a, batch, ta, tb, cfg, s);
    return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: output dtype %d unsupported for f16 inputs", c_dtype);
}

}  // namespace mlxhip
