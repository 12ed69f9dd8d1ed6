// gemm_f32.hip — instantiates the MFMA GEMM (gemm_impl.hpp) for f32 inputs.
#include "gemm_impl.hpp"

namespace mlxhip {

int gemm_f32(int c_dtype, int ta, int tb, const gemm_detail::GemmArgs& a, int64_t batch,
               bool aligned, int wt, hipStream_t s) {
    using namespace gemm_detail;
    if (c_dtype == MLXHIP_DTYPE_F32) return dispatch_trans<MLXHIP_DTYPE_F32, MLXHIP_DTYPE_F32>(a, batch, ta, tb, aligned, wt, s);
    return fail(MLXHIP_ERR_INVALID_ARGUMENT, "gemm: output dtype %d unsupported for f32 inputs", c_dtype);
}

}  // namespace mlxhip
