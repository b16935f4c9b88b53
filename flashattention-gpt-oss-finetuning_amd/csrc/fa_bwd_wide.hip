// fa_bwd_wide.hip - the D = 128 backward kernels (dQ, with and without the sink rows, and dK/dV),
// instantiated in a translation unit of their own so that they are compiled with LLVM's
// iterative ILP machine scheduler (-mllvm -amdgpu-sched-strategy=iterative-ilp, see the
// Makefile).  At D = 128 it schedules both kernels about 6% faster than the default scheduler
// (c5: dQ 428 -> 402 us, dK/dV 429 -> 400 us, bitwise the same results); at D = 64 it makes the
// dK/dV kernel slower, so the other head dims stay in fa_bwd.hip with the default.
#define FA_BWD_WIDE_TU
#include "fa_bwd.hip"

namespace fa {
template __global__ void bwd_dq_kernel<BF16, 128, false>(const Args);
template __global__ void bwd_dq_kernel<BF16, 128, true>(const Args);
template __global__ void bwd_dq_kernel<F16, 128, false>(const Args);
template __global__ void bwd_dq_kernel<F16, 128, true>(const Args);
template __global__ void bwd_dkdv_kernel<BF16, 128>(const Args);
template __global__ void bwd_dkdv_kernel<F16, 128>(const Args);
}  // namespace fa
