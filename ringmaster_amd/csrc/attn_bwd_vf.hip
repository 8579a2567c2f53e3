// Head-dim-64 and -128 instantiations of the block-attention backward (kernels and
// launch planning: attn_bwd_kernels.h). This unit is built with VGPR-form MFMAs
// (-mllvm -amdgpu-mfma-vgpr-form=1): the S and dP' tiles that the dK/dV kernel's VALU
// reads then need no v_accvgpr_read, and its K and -V operands are pinned to AGPRs.
#include "attn_bwd_kernels.h"

namespace rmx {

template hipError_t launch_bwd_t<64, RMX_DTYPE_BF16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<64, RMX_DTYPE_BF16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<64, RMX_DTYPE_F16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<64, RMX_DTYPE_F16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<128, RMX_DTYPE_BF16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<128, RMX_DTYPE_BF16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<128, RMX_DTYPE_F16, false>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);
template hipError_t launch_bwd_t<128, RMX_DTYPE_F16, true>(const rmx_attn_layout&,
    const rmx_bwd_problem*, int, hipStream_t);

}  // namespace rmx
