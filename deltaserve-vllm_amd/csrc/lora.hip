// LoRA factor plumbing:
//  * lora_cast: per-cycle fp32 master → bf16 operand copies in the layouts the
//    NT GEMM consumes (A, Aᵀ, s·B into block-diagonal K-concat slabs, (s·B)ᵀ).
//    The reference casts the masters inline per call (ops.py:103-146:
//    `A.to(xin.dtype)`, `B.to(xin.dtype)`); here one multi-tensor launch does it.
//  * lora_skinny: the rank-r products that keep the token dimension,
//      Z = X·Aᵀ (ops.py:141) and gZ = G·(s·B) (ops.py:142), [n, R] bf16 out.
//  * lora_tn: the rank-r weight gradients that reduce over tokens,
//      gA = gZᵀ·X   (ops.py:143, grad_A = grad_Z.t() @ xin)
//      gB = s·Gᵀ·Z  (ops.py:144, grad_B = scaling * (gy.t() @ Z))
//
// Both rank-r products are HBM-bound (they stream an [n, width] activation
// once for a few flops per byte), so neither stages through LDS: lanes load
// 16-byte row segments straight into MFMA operand registers. For the TN
// reduction the token dimension is the MFMA K, which the row-major
// activation does not hold contiguously per column; each lane therefore
// loads 8 columns × 8 tokens (eight 16-byte loads) and regroups them in
// registers into 8 operands of 8 tokens each, one per column.
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

// ------------------------------------------------------------------ skinny NT
// Block: 32 tokens, 4 waves splitting K; wave w covers K-slices of 128
// (lane half h takes k0 + 64h + 8kk, kk < 8). MFMA rows = tokens, cols =
// ranks, so each lane ends with 16 tokens × 1 rank per 32-rank block.
template <int RB>
__global__ __launch_bounds__(256) void lora_skinny_kernel(SkinnyArgs a) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int t0 = blockIdx.x * 32;
  if (t0 >= N) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 31, lh = lane >> 5;
  const int j0 = blockIdx.y * RB * 32;
  __shared__ float red[4][RB][32 * 33];
  f32x16 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[rb][r] = 0.f;
  const int t = t0 + li;
  const bool tok = t < N;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int kb = wave * 128; kb < a.K; kb += 4 * 128) {
    u32x4 xv[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int k = kb + 64 * lh + 8 * kk;
      const bool ok = tok && k < a.K;
      const u32x4 v = ldg128(a.X + (ok ? (long)t * a.ldx + k : 0L));
      xv[kk] = ok ? v : zero;
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int j = j0 + rb * 32 + li;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = kb + 64 * lh + 8 * kk;
        const bool ok = j < a.R && k < a.K;
        u32x4 bv = ldg128(a.B + (ok ? (long)j * a.ldb + k : 0L));
        bv = ok ? bv : zero;
        acc[rb] = mfma32(__builtin_bit_cast(bf16x8, xv[kk]), __builtin_bit_cast(bf16x8, bv),
                         acc[rb]);
      }
    }
  }
  // acc[rb][r]: token t0 + 8(r/4) + 4lh + r%4, rank j0 + rb*32 + li
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      red[wave][rb][(8 * (r >> 2) + 4 * lh + (r & 3)) * 33 + li] = acc[rb][r];
  __syncthreads();
  for (int idx = threadIdx.x; idx < RB * 32 * 32; idx += 256) {
    const int rb = idx / 1024, rem = idx % 1024, tt = rem / 32, jj = rem % 32;
    const int tk = t0 + tt, j = j0 + rb * 32 + jj;
    if (tk >= N || j >= a.R) continue;
    const float v = red[0][rb][tt * 33 + jj] + red[1][rb][tt * 33 + jj] +
                    red[2][rb][tt * 33 + jj] + red[3][rb][tt * 33 + jj];
    a.Z[(long)tk * a.ldz + j] = (bf16)v;
  }
}

hipError_t lora_skinny(const SkinnyArgs& a, hipStream_t s) {
  if (a.R <= 0 || a.n <= 0) return hipSuccess;
  const int nrb = (a.R + 31) / 32;
  const dim3 grid((a.n + 31) / 32, (nrb + 1) / 2);
  if (nrb == 1)
    hipLaunchKernelGGL(lora_skinny_kernel<1>, dim3(grid.x, 1), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(lora_skinny_kernel<2>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ TN
// Block: 4 waves × (32 lanes × CPL columns); one token split; RB rank blocks.
// Per 16-token step, lane (li, lh) loads CPL columns c0 + CPL·li .. of tokens
// t + 8lh + e (e < 8), and MFMA #cc consumes column c0 + CPL·li + cc across
// those 8 tokens. Output lane: rank j0 + 32rb + li, columns
// c0 + CPL·(8(r/4) + 4lh + r%4) + cc. Partials go to work[split][C][R].
template <int RB, int CPL>
__global__ __launch_bounds__(256) void lora_tn_partial_kernel(TnArgs a) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 31, lh = lane >> 5;
  const int c0 = (blockIdx.x * 4 + wave) * 32 * CPL;
  const int j0 = blockIdx.z * RB * 32;
  const int sp = blockIdx.y;
  int per = (N + a.nsplit - 1) / a.nsplit;
  per = (per + 15) & ~15;
  const int ta = min(N, sp * per), tb = min(N, ta + per);
  f32x16 acc[RB][CPL];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][cc][r] = 0.f;
  const int cl = c0 + CPL * li;
  const bool cok = cl < a.C;
  for (int t = ta; t < tb; t += 16) {
    bf16 xs[8][CPL];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tt = t + 8 * lh + e;
      const bool ok = cok && tt < tb;
      if constexpr (CPL == 8) {
        u32x4 v = ldg128(a.X + (ok ? (long)tt * a.ldx + cl : 0L));
        if (!ok) v = u32x4{0u, 0u, 0u, 0u};
        const bf16x8 b = __builtin_bit_cast(bf16x8, v);
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) xs[e][cc] = b[cc];
      } else {
        u32x2 v = *reinterpret_cast<const u32x2*>(a.X + (ok ? (long)tt * a.ldx + cl : 0L));
        if (!ok) v = u32x2{0u, 0u};
        const bf16x4 b = __builtin_bit_cast(bf16x4, v);
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) xs[e][cc] = b[cc];
      }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int j = j0 + rb * 32 + li;
      bf16x8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tt = t + 8 * lh + e;
        const bool ok = j < a.R && tt < tb;
        const bf16 v = a.P[ok ? (long)tt * a.ldp + j : 0L];
        pb[e] = ok ? v : (bf16)0.f;
      }
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc) {
        bf16x8 av;
#pragma unroll
        for (int e = 0; e < 8; ++e) av[e] = xs[e][cc];
        acc[rb][cc] = mfma32(av, pb, acc[rb][cc]);
      }
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int j = j0 + rb * 32 + li;
    if (j >= a.R) continue;
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int col = c0 + CPL * (8 * (r >> 2) + 4 * lh + (r & 3)) + cc;
        if (col < a.C) a.work[((long)sp * a.C + col) * a.R + j] = acc[rb][cc][r];
      }
  }
}

__global__ __launch_bounds__(256) void lora_tn_reduce_kernel(TnArgs a) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)a.R * a.C) return;
  const int c = (int)(idx / a.R), j = (int)(idx % a.R);
  float s = 0.f;
  for (int sp = 0; sp < a.nsplit; ++sp) s += a.work[((long)sp * a.C + c) * a.R + j];
  s *= a.scale;
  const int grp = j / a.rg, jj = j % a.rg;
  float* o = a.outs[grp];
  if (a.transpose_out)
    o[(long)c * a.rg + jj] = s;
  else
    o[(long)jj * a.C + c] = s;
}

hipError_t lora_tn(const TnArgs& a, hipStream_t s) {
  if (a.R <= 0 || a.C <= 0) return hipSuccess;
  const int nrb = (a.R + 31) / 32;
  hipError_t e;
  if (nrb == 1) {
    const int cb = (a.C + 4 * 256 - 1) / (4 * 256);
    hipLaunchKernelGGL((lora_tn_partial_kernel<1, 8>), dim3(cb, a.nsplit, 1), dim3(256), 0, s, a);
  } else {
    const int cb = (a.C + 4 * 128 - 1) / (4 * 128);
    hipLaunchKernelGGL((lora_tn_partial_kernel<2, 4>), dim3(cb, a.nsplit, (nrb + 1) / 2),
                       dim3(256), 0, s, a);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const long tot = (long)a.R * a.C;
  hipLaunchKernelGGL(lora_tn_reduce_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0,
                     s, a);
  return hipGetLastError();
}

}  // namespace dsb
