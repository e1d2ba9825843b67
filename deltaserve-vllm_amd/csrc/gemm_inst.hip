// Translation unit that owns the generic GEMM instantiations shared by the
// single-op entry points (the cycle's own instantiations live next to their
// callers; the template is header-only).
#include "gemm_nt.h"

namespace dsb {
template __global__ void gemm_nt_kernel<256, 256, 2, 2, EpiBF16>(GemmProblem, EpiBF16);
template __global__ void gemm_nt_kernel<128, 128, 2, 2, EpiBF16>(GemmProblem, EpiBF16);
template __global__ void gemm_nt_kernel<64, 64, 2, 2, EpiBF16>(GemmProblem, EpiBF16);
template __global__ void gemm_nt_kernel<256, 256, 2, 2, EpiF32>(GemmProblem, EpiF32);
template __global__ void gemm_nt_kernel<128, 128, 2, 2, EpiF32>(GemmProblem, EpiF32);
template __global__ void gemm_nt_kernel<64, 64, 2, 2, EpiF32>(GemmProblem, EpiF32);
}  // namespace dsb
