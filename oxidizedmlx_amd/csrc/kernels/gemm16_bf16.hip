// gemm16_bf16.hip — instantiates the direct-to-LDS MFMA GEMM (gemm16_impl.hpp)
// for bf16 operands.
#include "gemm16_impl.hpp"

namespace mlxhip {

int gemm16_bf16(int c_dtype, int ta, int tb, const gemm16::Args& a, int64_t batch, int cfg, hipStream_t s) {
    using namespace gemm16;
    if (c_dtype == MLXHIP_DTYPE_F32) return dispatch<MLXHIP_DTYPE_BF16, MLXHIP_DTYPE_F32>(a, batch, ta, tb, cfg, s);
    if (c_dtype == MLXHIP_DTYPE_BF16) return dispatch<MLXHIP_DTYPE_BF16, MLXHIP_DTYPE_BF16>(a, batch, ta, tb, cfg, s);
    return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: output dtype %d unsupported for bf16 inputs", c_dtype);
}

}  // namespace mlxhip
