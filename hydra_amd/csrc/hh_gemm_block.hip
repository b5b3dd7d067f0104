// hh_gemm_block.hip — the FFN block's MXFP4 decode gate-up kernels with the fused router
// (up_small_mx with FR = 2), compiled apart from hh_gemm.hip's other kernels. See hh_gemm.hip.
#define HH_GEMM_KERNELS_ONLY
#include "hh_gemm.hip"
