// fa_bwd_wide.hip - backward kernels instantiated in a translation unit of their own so that they
// are compiled with LLVM's iterative ILP machine scheduler (-mllvm
// -amdgpu-sched-strategy=iterative-ilp, see the Makefile), with bitwise the same results:
//  * D = 128 dQ (with and without the sink rows) and dK/dV: about 6% faster than with the default
//    scheduler (c5: dQ 428 -> 402 us, dK/dV 429 -> 400 us);
//  * D = 64 dQ without sink rows (full causal layers): about 2% faster (c3: 1023 -> 1004 us).
// The other kernels stay in fa_bwd.hip with the default, which suits them better (the D = 64
// dK/dV kernel, for one, is slower with this scheduler).
#define FA_BWD_WIDE_TU
#include "fa_bwd.hip"

namespace fa {
template __global__ void bwd_dq_kernel<BF16, 64, false>(const Args);
template __global__ void bwd_dq_kernel<F16, 64, false>(const Args);
template __global__ void bwd_dq_kernel<BF16, 128, false>(const Args);
template __global__ void bwd_dq_kernel<BF16, 128, true>(const Args);
template __global__ void bwd_dq_kernel<F16, 128, false>(const Args);
template __global__ void bwd_dq_kernel<F16, 128, true>(const Args);
template __global__ void bwd_dkdv_kernel<BF16, 128>(const Args);
template __global__ void bwd_dkdv_kernel<F16, 128>(const Args);
}  // namespace fa
