// LoRA factor plumbing:
//  * lora_cast: per-cycle fp32 master → bf16 operand copies in the layouts the
//    NT GEMM consumes (A, Aᵀ, s·B into block-diagonal K-concat slabs, (s·B)ᵀ).
//    The reference casts the masters inline per call (ops.py:103-146:
//    `A.to(xin.dtype)`, `B.to(xin.dtype)`); here one multi-tensor launch does it.
//  * lora_tn: the rank-r weight gradients that reduce over tokens,
//      gA = gZᵀ·X   (ops.py:143, grad_A = grad_Z.t() @ xin)
//      gB = s·Gᵀ·Z  (ops.py:144, grad_B = scaling * (gy.t() @ Z))
//    as a token-split fp32 FMA reduction (each thread: 4 columns × 16 ranks)
//    followed by a fixed-order reduction over splits into the fp32 grads.
#include "kernels.h"

namespace dsb {

__global__ __launch_bounds__(256) void lora_cast_kernel(const CastJob* __restrict__ jobs,
                                                        const int2* __restrict__ chunks) {
  const int2 ck = chunks[blockIdx.x];
  const CastJob j = jobs[ck.x];
  const long tot = (long)j.rows * j.cols;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const long idx = (long)ck.y + threadIdx.x + e * 256;
    if (idx >= tot) break;
    const int r = (int)(idx / j.cols), c = (int)(idx % j.cols);
    const float v = j.src[(long)r * j.ld_src + c] * j.scale;
    const long d = j.transpose ? (long)c * j.ld_dst + r : (long)r * j.ld_dst + c;
    j.dst[d] = (bf16)v;
  }
}

hipError_t lora_cast(const CastJob* jobs_dev, const int2* chunks_dev, int nchunks,
                     hipStream_t s) {
  if (nchunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(lora_cast_kernel, dim3(nchunks), dim3(256), 0, s, jobs_dev, chunks_dev);
  return hipGetLastError();
}

namespace {
constexpr int TN_CPT = 4;   // columns per thread
constexpr int TN_RB = 16;   // ranks per block
}  // namespace

__global__ __launch_bounds__(256) void lora_tn_partial_kernel(TnArgs a) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int c = (blockIdx.x * 256 + threadIdx.x) * TN_CPT;
  const int j0 = blockIdx.z * TN_RB;
  const int sp = blockIdx.y;
  const int per = (N + a.nsplit - 1) / a.nsplit;
  const int t0 = min(N, sp * per), t1 = min(N, t0 + per);
  float acc[TN_RB][TN_CPT];
#pragma unroll
  for (int j = 0; j < TN_RB; ++j)
#pragma unroll
    for (int e = 0; e < TN_CPT; ++e) acc[j][e] = 0.f;
  const int nj = min(TN_RB, a.R - j0);
  if (c < a.C) {
#pragma unroll 2
    for (int t = t0; t < t1; ++t) {
      const bf16x4 xv = *reinterpret_cast<const bf16x4*>(a.X + (long)t * a.ldx + c);
      const float* pr = a.P + (long)t * a.ldp + j0;
      float x[TN_CPT];
#pragma unroll
      for (int e = 0; e < TN_CPT; ++e) x[e] = (float)xv[e];
#pragma unroll
      for (int j = 0; j < TN_RB; ++j) {
        const float pv = pr[j < nj ? j : nj - 1];  // clamped: never reads past row t
        const float pj = j < nj ? pv : 0.f;
#pragma unroll
        for (int e = 0; e < TN_CPT; ++e) acc[j][e] += pj * x[e];
      }
    }
#pragma unroll
    for (int j = 0; j < TN_RB; ++j) {
      if (j >= nj) break;
      float* w = a.work + ((long)sp * a.R + j0 + j) * a.C + c;
      *reinterpret_cast<f32x4*>(w) = f32x4{acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
    }
  }
}

__global__ __launch_bounds__(256) void lora_tn_reduce_kernel(TnArgs a) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)a.R * a.C) return;
  const int j = (int)(idx / a.C), c = (int)(idx % a.C);
  float s = 0.f;
  for (int sp = 0; sp < a.nsplit; ++sp) s += a.work[((long)sp * a.R + j) * a.C + c];
  const int grp = j / a.rg, jj = j % a.rg;
  float* o = a.outs[grp];
  if (a.transpose_out)
    o[(long)c * a.rg + jj] = s;
  else
    o[(long)jj * a.C + c] = s;
}

hipError_t lora_tn(const TnArgs& a, hipStream_t s) {
  if (a.R <= 0 || a.C <= 0) return hipSuccess;
  const int cb = (a.C + 256 * TN_CPT - 1) / (256 * TN_CPT);
  const int rb = (a.R + TN_RB - 1) / TN_RB;
  hipLaunchKernelGGL(lora_tn_partial_kernel, dim3(cb, a.nsplit, rb), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long tot = (long)a.R * a.C;
  hipLaunchKernelGGL(lora_tn_reduce_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0,
                     s, a);
  return hipGetLastError();
}

}  // namespace dsb
