// Bandwidth-bound per-row kernels of the backward: RMSNorm forward/backward,
// RoPE (NeoX rotate-half) forward/backward with the optional per-head q/k
// RMSNorm of Qwen3, the RoPE cos/sin table, and h = silu(gate)·up.
//
// Semantics follow deltaserve-plugin/deltaserve/bwd_services/common/ops.py:
//   rmsnorm            ops.py:84-88   (fp32 internals, output in the input dtype)
//   rmsnorm_backward   ops.py:91-100
//   rope_cos_sin       ops.py:60-65
//   apply_rope         ops.py:68-73
//   rope_backward      ops.py:76-81
//   q/k-norm fwd/bwd   bwd_services/qwen3.py:96-107, :133-144
// All arithmetic is fp32 with one rounding to bf16 at the store.
#include "kernels.h"

namespace dsb {

// One 256-thread block per row; each thread keeps up to RPT 8-wide chunks.
constexpr int NORM_NT = 256;
constexpr int NORM_RPT = 4;  // D <= 256 * 8 * 4 = 8192

__global__ __launch_bounds__(NORM_NT) void rmsnorm_fwd_kernel(
    const bf16* __restrict__ x, long ldx, const bf16* __restrict__ w,
    bf16* __restrict__ y, long ldy, int rows, const int* rows_dev, int D, float eps) {
  int R = rows;
  if (rows_dev) R = min(R, *rows_dev);
  const int row = blockIdx.x;
  if (row >= R) return;
  __shared__ float red[NORM_NT / 64];
  const bf16* xr = x + (long)row * ldx;
  const int nch = D >> 3;
  // the weight chunks are loaded with the row, so their latency overlaps the
  // row's and the block reduction's
  float v[NORM_RPT][8], wv[NORM_RPT][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_RPT; ++i) {
    const int c = threadIdx.x + i * NORM_NT;
    if (c < nch) {
      unpack8(ldg128(xr + c * 8), v[i]);
      unpack8(ldg128(w + c * 8), wv[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
    }
  }
  ss = block_sum<NORM_NT>(ss, red);
  const float inv = rsqrtf(ss / (float)D + eps);
  bf16* yr = y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < NORM_RPT; ++i) {
    const int c = threadIdx.x + i * NORM_NT;
    if (c < nch) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[i][e] * inv) * wv[i][e];
      stg128(yr + c * 8, pack8(o));
    }
  }
}

// The same, one wave per row (4 rows per block) for D = 512·CPL: a lane
// keeps CPL 8-wide chunks of x and of the weight in flight and the row sum is
// a wave reduction (no block barriers). Used for short rows (D = 1024, 2048),
// where the block-per-row kernel's barriers dominate; at D = 4096 the
// block-per-row kernel measured faster.
template <int CPL>
__global__ __launch_bounds__(256) void rmsnorm_fwd_wave_kernel(
    const bf16* __restrict__ x, long ldx, const bf16* __restrict__ w,
    bf16* __restrict__ y, long ldy, int rows, const int* rows_dev, int D, float eps) {
  int R = rows;
  if (rows_dev) R = min(R, *rows_dev);
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= R) return;
  const bf16* xr = x + (long)row * ldx;
  u32x4 xv[CPL], wv[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    xv[i] = ldg128(xr + (lane + 64 * i) * 8);
    wv[i] = ldg128(w + (lane + 64 * i) * 8);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    float v[8];
    unpack8(xv[i], v);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
  bf16* yr = y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    float v[8], wf[8], o[8];
    unpack8(xv[i], v);
    unpack8(wv[i], wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (v[e] * inv) * wf[e];
    stg128(yr + (lane + 64 * i) * 8, pack8(o));
  }
}

// o = rmsnorm_backward(x, g, w) + resid (g fp32 or bf16; resid bf16, fp32
// resid32, or none) → out = bf16(o) and, when out32 is set, the fp32 o (the
// residual-stream gradient the next layer adds to, kept unrounded).
template <typename GT>
__global__ __launch_bounds__(NORM_NT) void rmsnorm_bwd_kernel(
    const bf16* __restrict__ x, long ldx, const GT* __restrict__ g, long ldg,
    const bf16* __restrict__ w, const bf16* __restrict__ resid,
    const float* __restrict__ resid32, long ldr, bf16* __restrict__ out,
    float* __restrict__ out32, long ldo, int rows, const int* rows_dev, int D, float eps) {
  int R = rows;
  if (rows_dev) R = min(R, *rows_dev);
  const int row = blockIdx.x;
  if (row >= R) return;
  __shared__ float red[NORM_NT / 64];
  const bf16* xr = x + (long)row * ldx;
  const GT* gr = g + (long)row * ldg;
  const int nch = D >> 3;
  float xv[NORM_RPT][8], gw[NORM_RPT][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_RPT; ++i) {
    const int c = threadIdx.x + i * NORM_NT;
    if (c < nch) {
      unpack8(ldg128(xr + c * 8), xv[i]);
      float wf[8];
      unpack8(ldg128(w + c * 8), wf);
      if constexpr (sizeof(GT) == 4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(gr + c * 8);
        const f32x4 b = *reinterpret_cast<const f32x4*>(gr + c * 8 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { gw[i][e] = a[e] * wf[e]; gw[i][e + 4] = b[e] * wf[e + 4]; }
      } else {
        float gf[8];
        unpack8(ldg128(gr + c * 8), gf);
#pragma unroll
        for (int e = 0; e < 8; ++e) gw[i][e] = gf[e] * wf[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += xv[i][e] * xv[i][e];
    }
  }
  ss = block_sum<NORM_NT>(ss, red);
  const float inv = rsqrtf(ss / (float)D + eps);
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_RPT; ++i) {
    const int c = threadIdx.x + i * NORM_NT;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += gw[i][e] * (xv[i][e] * inv);
    }
  }
  dot = block_sum<NORM_NT>(dot, red);
  const float k = dot / (float)D;
  bf16* orow = out + (long)row * ldo;
#pragma unroll
  for (int i = 0; i < NORM_RPT; ++i) {
    const int c = threadIdx.x + i * NORM_NT;
    if (c < nch) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (gw[i][e] - (xv[i][e] * inv) * k) * inv;
      if (resid) {
        float rf[8];
        unpack8(ldg128(resid + (long)row * ldr + c * 8), rf);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += rf[e];
      } else if (resid32) {
        const float* rp = resid32 + (long)row * ldr + c * 8;
        const f32x4 a = *reinterpret_cast<const f32x4*>(rp);
        const f32x4 b = *reinterpret_cast<const f32x4*>(rp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { o[e] += a[e]; o[e + 4] += b[e]; }
      }
      stg128(orow + c * 8, pack8(o));
      if (out32) {
        float* op = out32 + (long)row * ldo + c * 8;
        *reinterpret_cast<f32x4*>(op) = f32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<f32x4*>(op + 4) = f32x4{o[4], o[5], o[6], o[7]};
      }
    }
  }
}

// cos/sin[t, i] = cos/sin(float(pos[t]) * inv_freq[i]), i < half.
__global__ void rope_table_kernel(const int* __restrict__ pos, int n, const int* n_dev,
                                  const float* __restrict__ inv_freq, int half,
                                  float* __restrict__ cosb, float* __restrict__ sinb) {
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)N * half) return;
  const int t = (int)(idx / half), i = (int)(idx % half);
  const float a = (float)pos[t] * inv_freq[i];
  float s, c;
  sincosf(a, &s, &c);
  cosb[idx] = c;
  sinb[idx] = s;
}

// HD/16 lanes per head (8 at head_dim 128, 4 at 64): lane i of a head's
// group owns the rotate-half pairs (8i + e, HD/2 + 8i + e), e = 0..7, moved as
// 16-byte vectors; one wave covers 64/(HD/16) heads of one token (q heads,
// then k heads), and per-head sums reduce over the group's lanes.
//   in : the q heads of a row at in (stride ldin) and its k heads at ink
//        (stride ldk): pre-norm, pre-RoPE projection outputs, either the
//        [q | k | v] rows of the recompute or separate saved q / k buffers
//   out: qk row [q | k] after (optional per-head RMSNorm, rounded to bf16) + RoPE
template <int LPH>
DSB_DEV float group_sum(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  if constexpr (LPH == 8) v += __shfl_xor(v, 4, 64);
  return v;
}

template <int HD>
__global__ __launch_bounds__(256) void rope_fwd_kernel(
    const bf16* __restrict__ in, long ldin, const bf16* __restrict__ ink, long ldk,
    bf16* __restrict__ out, long ldout,
    const float* __restrict__ cosb, const float* __restrict__ sinb, int n,
    const int* n_dev, int Hq, int Hkv, const bf16* __restrict__ qn_w,
    const bf16* __restrict__ kn_w, float eps) {
  constexpr int LPH = HD / 16, HPW = 64 / LPH, HALF = HD / 2;
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  const int H = Hq + Hkv, HG = (H + HPW - 1) / HPW;
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (long)N * HG) return;
  const int t = (int)(item / HG), l = threadIdx.x & 63, i = l % LPH;
  const int hh = (int)(item % HG) * HPW + l / LPH;
  const bool live = hh < H;
  const int h = live ? hh : H - 1;
  const bf16* src = h < Hq ? in + (long)t * ldin + h * HD + 8 * i
                            : ink + (long)t * ldk + (h - Hq) * HD + 8 * i;
  float x1[8], x2[8];
  unpack8(ldg128(src), x1);
  unpack8(ldg128(src + HALF), x2);
  const bf16* nw = h < Hq ? qn_w : kn_w;
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x1[e] * x1[e] + x2[e] * x2[e];
    const float inv = rsqrtf(group_sum<LPH>(ss) / (float)HD + eps);
    float w1[8], w2[8];
    unpack8(ldg128(nw + 8 * i), w1);
    unpack8(ldg128(nw + HALF + 8 * i), w2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x1[e] = (float)(bf16)((x1[e] * inv) * w1[e]);
      x2[e] = (float)(bf16)((x2[e] * inv) * w2[e]);
    }
  }
  const f32x4* cp = reinterpret_cast<const f32x4*>(cosb + (long)t * HALF + 8 * i);
  const f32x4* sp = reinterpret_cast<const f32x4*>(sinb + (long)t * HALF + 8 * i);
  const f32x4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  float o1[8], o2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o1[e] = x1[e] * c[e] - x2[e] * sn[e];
    o2[e] = x2[e] * c[e] + x1[e] * sn[e];
  }
  if (live) {
    bf16* dst = out + (long)t * ldout + h * HD + 8 * i;
    stg128(dst, pack8(o1));
    stg128(dst + HALF, pack8(o2));
  }
}

// In-place RoPE backward on g[:, :(Hq+Hkv)*HD] (then the per-head RMSNorm
// backward against the pre-norm projection output when norm weights are given);
// same lane layout as the forward.
template <int HD>
__global__ __launch_bounds__(256) void rope_bwd_kernel(
    bf16* __restrict__ g, long ldg, const bf16* __restrict__ pre, long ldp,
    const bf16* __restrict__ prek, long ldpk,
    const float* __restrict__ cosb, const float* __restrict__ sinb, int n,
    const int* n_dev, int Hq, int Hkv, const bf16* __restrict__ qn_w,
    const bf16* __restrict__ kn_w, float eps) {
  constexpr int LPH = HD / 16, HPW = 64 / LPH, HALF = HD / 2;
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  const int H = Hq + Hkv, HG = (H + HPW - 1) / HPW;
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (long)N * HG) return;
  const int t = (int)(item / HG), l = threadIdx.x & 63, i = l % LPH;
  const int hh = (int)(item % HG) * HPW + l / LPH;
  const bool live = hh < H;
  const int h = live ? hh : H - 1;
  bf16* gp = g + (long)t * ldg + h * HD + 8 * i;
  float g1[8], g2[8];
  unpack8(ldg128(gp), g1);
  unpack8(ldg128(gp + HALF), g2);
  const f32x4* cp = reinterpret_cast<const f32x4*>(cosb + (long)t * HALF + 8 * i);
  const f32x4* sp = reinterpret_cast<const f32x4*>(sinb + (long)t * HALF + 8 * i);
  const f32x4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  float r1[8], r2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r1[e] = g1[e] * c[e] + g2[e] * sn[e];
    r2[e] = -g1[e] * sn[e] + g2[e] * c[e];
  }
  const bf16* nw = h < Hq ? qn_w : kn_w;
  if (nw) {
    const bf16* xp = h < Hq ? pre + (long)t * ldp + h * HD + 8 * i
                            : prek + (long)t * ldpk + (h - Hq) * HD + 8 * i;
    float x1[8], x2[8], w1[8], w2[8];
    unpack8(ldg128(xp), x1);
    unpack8(ldg128(xp + HALF), x2);
    unpack8(ldg128(nw + 8 * i), w1);
    unpack8(ldg128(nw + HALF + 8 * i), w2);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x1[e] * x1[e] + x2[e] * x2[e];
    const float inv = rsqrtf(group_sum<LPH>(ss) / (float)HD + eps);
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r1[e] *= w1[e];
      r2[e] *= w2[e];
      dot += r1[e] * (x1[e] * inv) + r2[e] * (x2[e] * inv);
    }
    const float k = group_sum<LPH>(dot) / (float)HD;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r1[e] = (r1[e] - (x1[e] * inv) * k) * inv;
      r2[e] = (r2[e] - (x2[e] * inv) * k) * inv;
    }
  }
  if (live) {
    stg128(gp, pack8(r1));
    stg128(gp + HALF, pack8(r2));
  }
}

// h[m, j] = bf16(silu(gate) * up) with gate = GU[m, j], up = GU[m, I + j].
__global__ __launch_bounds__(256) void swiglu_h_kernel(const bf16* __restrict__ gu, long ldgu,
                                                       bf16* __restrict__ h, long ldh, int n,
                                                       const int* n_dev, int I) {
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  const int cpr = I >> 3;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)N * cpr) return;
  const int m = (int)(idx / cpr), c = (int)(idx % cpr);
  float g[8], u[8], o[8];
  unpack8(ldg128(gu + (long)m * ldgu + c * 8), g);
  unpack8(ldg128(gu + (long)m * ldgu + I + c * 8), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = g[e] * sigmoid(g[e]) * u[e];
  stg128(h + (long)m * ldh + c * 8, pack8(o));
}

// ------------------------------------------------------------------ launchers

hipError_t rmsnorm_fwd(const bf16* x, long ldx, const bf16* w, bf16* y, long ldy, int rows,
                       const int* rows_dev, int D, float eps, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const dim3 wg((rows + 3) / 4);
  switch (D % 512 == 0 ? D / 512 : 0) {
    case 2: hipLaunchKernelGGL(rmsnorm_fwd_wave_kernel<2>, wg, dim3(256), 0, s, x, ldx, w, y, ldy, rows, rows_dev, D, eps); break;
    case 4: hipLaunchKernelGGL(rmsnorm_fwd_wave_kernel<4>, wg, dim3(256), 0, s, x, ldx, w, y, ldy, rows, rows_dev, D, eps); break;
    default:
      hipLaunchKernelGGL(rmsnorm_fwd_kernel, dim3(rows), dim3(NORM_NT), 0, s, x, ldx, w, y, ldy,
                         rows, rows_dev, D, eps);
  }
  return hipGetLastError();
}

hipError_t rmsnorm_bwd(const bf16* x, long ldx, const void* g, bool g_f32, long ldg,
                       const bf16* w, const bf16* resid, long ldr, bf16* out, long ldo,
                       int rows, const int* rows_dev, int D, float eps, hipStream_t s,
                       const float* resid32, float* out32) {
  if (rows <= 0) return hipSuccess;
  if (g_f32)
    hipLaunchKernelGGL(rmsnorm_bwd_kernel<float>, dim3(rows), dim3(NORM_NT), 0, s, x, ldx,
                       (const float*)g, ldg, w, resid, resid32, ldr, out, out32, ldo, rows,
                       rows_dev, D, eps);
  else
    hipLaunchKernelGGL(rmsnorm_bwd_kernel<bf16>, dim3(rows), dim3(NORM_NT), 0, s, x, ldx,
                       (const bf16*)g, ldg, w, resid, resid32, ldr, out, out32, ldo, rows,
                       rows_dev, D, eps);
  return hipGetLastError();
}

hipError_t rope_table(const int* pos, int n, const int* n_dev, const float* inv_freq,
                      int half, float* cosb, float* sinb, hipStream_t s) {
  const long tot = (long)n * half;
  if (tot <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s,
                     pos, n, n_dev, inv_freq, half, cosb, sinb);
  return hipGetLastError();
}

hipError_t rope_fwd(const bf16* in, long ldin, bf16* out, long ldout, const float* cosb,
                    const float* sinb, int n, const int* n_dev, int Hq, int Hkv, int hd,
                    const bf16* qn_w, const bf16* kn_w, float eps, hipStream_t s,
                    const bf16* ink, long ldk) {
  if (hd != 128 && hd != 64) return hipErrorInvalidValue;
  const int hpw = 64 / (hd / 16);
  const long items = (long)n * ((Hq + Hkv + hpw - 1) / hpw);
  if (items <= 0) return hipSuccess;
  if (!ink) {
    ink = in + (long)Hq * hd;
    ldk = ldin;
  }
  const dim3 grid((unsigned)((items + 3) / 4));
  if (hd == 128)
    hipLaunchKernelGGL(rope_fwd_kernel<128>, grid, dim3(256), 0, s, in, ldin, ink, ldk, out,
                       ldout, cosb, sinb, n, n_dev, Hq, Hkv, qn_w, kn_w, eps);
  else
    hipLaunchKernelGGL(rope_fwd_kernel<64>, grid, dim3(256), 0, s, in, ldin, ink, ldk, out,
                       ldout, cosb, sinb, n, n_dev, Hq, Hkv, qn_w, kn_w, eps);
  return hipGetLastError();
}

hipError_t rope_bwd(bf16* g, long ldg, const bf16* pre, long ldp, const float* cosb,
                    const float* sinb, int n, const int* n_dev, int Hq, int Hkv, int hd,
                    const bf16* qn_w, const bf16* kn_w, float eps, hipStream_t s,
                    const bf16* prek, long ldpk) {
  if (hd != 128 && hd != 64) return hipErrorInvalidValue;
  const int hpw = 64 / (hd / 16);
  const long items = (long)n * ((Hq + Hkv + hpw - 1) / hpw);
  if (items <= 0) return hipSuccess;
  if (!prek) {
    prek = pre + (long)Hq * hd;
    ldpk = ldp;
  }
  const dim3 grid((unsigned)((items + 3) / 4));
  if (hd == 128)
    hipLaunchKernelGGL(rope_bwd_kernel<128>, grid, dim3(256), 0, s, g, ldg, pre, ldp, prek, ldpk,
                       cosb, sinb, n, n_dev, Hq, Hkv, qn_w, kn_w, eps);
  else
    hipLaunchKernelGGL(rope_bwd_kernel<64>, grid, dim3(256), 0, s, g, ldg, pre, ldp, prek, ldpk,
                       cosb, sinb, n, n_dev, Hq, Hkv, qn_w, kn_w, eps);
  return hipGetLastError();
}

hipError_t swiglu_h(const bf16* gu, long ldgu, bf16* h, long ldh, int n, const int* n_dev,
                    int I, hipStream_t s) {
  const long tot = (long)n * (I >> 3);
  if (tot <= 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_h_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, gu,
                     ldgu, h, ldh, n, n_dev, I);
  return hipGetLastError();
}

}  // namespace dsb
