// Packed varlen causal GQA attention (head_dim 128) on gfx950 MFMA:
// forward recompute (ctx, fp32 ctx copy, row log-sum-exp) and the FA2-style
// backward split into a dK/dV pass (one block per 128 keys of one kv head,
// summing its q-head group in registers, no atomics) and a dQ pass (one block
// per 128 queries of one q head). Softmax statistics, P and dS stay fp32 in
// registers; P and dS are rounded to bf16 only as MFMA operands.
//
// Semantics: deltaserve-plugin/deltaserve/bwd_services/common/attention.py
//   attn_forward_core   :20-45   (scale 1/sqrt(Hd), causal mask, fp32 softmax)
//   attn_backward_core  :48-112  (dS = P∘(dP − rowsum(dP∘P)), GQA group sums)
// rowsum(dP∘P) is computed as rowsum(dO∘O) with the fp32 O of the forward.
//
// Register tiles: an MFMA with A = rows of X and B = rows of Y gives
// lane l the Y-row (l%32) and X-rows 8(r/4)+4(l/32)+r%4. A register tile used
// again as the B operand of a product that reduces over those X-rows is fed
// as acc[8c .. 8c+7] for each 16-row chunk c; the matching A operand is read
// from a transposed LDS tile at rows {16c + 4(l/32) + 0..3, +8..+11}.
#include "kernels.h"

namespace dsb {

namespace {
constexpr int HD = 128;
constexpr int SN = 136;  // padded row stride (elements) of [tok][dim] LDS tiles
constexpr int ST = 72;   // padded row stride of [dim][tok] LDS tiles (64 tokens)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kScale = 0.08838834764831845f;  // 1/sqrt(128)

DSB_DEV bf16x8 cat44(bf16x4 lo, bf16x4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

DSB_DEV bf16x8 read_t_frag(const bf16* sT, int row, int col) {
  const bf16* p = sT + row * ST + col;
  return cat44(*reinterpret_cast<const bf16x4*>(p), *reinterpret_cast<const bf16x4*>(p + 8));
}

DSB_DEV bf16x8 read_n_frag(const bf16* sN, int row, int col) {
  return *reinterpret_cast<const bf16x8*>(sN + row * SN + col);
}

// Stage a 64-token × 128-dim tile (rows tok0 .. tok0+63 of a packed sequence
// starting at global row `st`, valid below `L`) into LDS, normal and/or
// transposed. Token-fastest thread mapping keeps the transposed b16 writes
// on consecutive addresses.
DSB_DEV void stage_tile(const bf16* base, long ld, int col0, int st, int tok0, int L, bf16* sN,
                        bf16* sT) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + i * 256;
    const int tok = c & 63, ch = c >> 6;
    const int t = tok0 + tok;
    const bool ok = t < L;
    u32x4 v = ldg128(base + (ok ? (long)(st + t) * ld + col0 + ch * 8 : 0L));
    if (!ok) v = u32x4{0u, 0u, 0u, 0u};
    if (sN) *reinterpret_cast<u32x4*>(sN + tok * SN + ch * 8) = v;
    if (sT) {
      const bf16x8 b = __builtin_bit_cast(bf16x8, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) sT[(ch * 8 + e) * ST + tok] = b[e];
    }
  }
}

DSB_DEV void load_row_frags(const bf16* base, long ld, long row, int col0, bool ok, int lh,
                            bf16x8 (&f)[8]) {
  const bf16* p = base + (ok ? row * ld + col0 : 0L);
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    f[kk] = *reinterpret_cast<const bf16x8*>(p + kk * 16 + lh * 8);
    if (!ok) f[kk] = bf16x8{};
  }
}
}  // namespace

__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  const int tile = blockIdx.x;
  if (tile >= *a.ntiles_dev) return;
  const int h = blockIdx.y, kvh = h / (a.Hq / a.Hkv);
  const int4 tl = a.tiles[tile];
  const int st = tl.x, L = tl.y, q0 = tl.z;
  __shared__ __attribute__((aligned(16))) bf16 sK[64 * SN];
  __shared__ __attribute__((aligned(16))) bf16 sVt[HD * ST];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, lh = lane >> 5;
  const int qpos = q0 + w * 32 + lr;
  const bool qok = qpos < L;

  bf16x8 qf[8];
  load_row_frags(a.q, a.ldq, st + qpos, h * HD, qok, lh, qf);

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_i = -INFINITY, l_i = 0.f;
  const float sl2 = kScale * kLog2e;
  const int kv_end = min(L, q0 + 128);

  for (int k0 = 0; k0 < kv_end; k0 += 64) {
    __syncthreads();
    stage_tile(a.k, a.ldk, kvh * HD, st, k0, L, sK, nullptr);
    stage_tile(a.v, a.ldv, kvh * HD, st, k0, L, nullptr, sVt);
    __syncthreads();

    f32x16 s[2];
#pragma unroll
    for (int kf = 0; kf < 2; ++kf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kf][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        s[kf] = mfma32(read_n_frag(sK, kf * 32 + lr, kk * 16 + lh * 8), qf[kk], s[kf]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + kf * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        float x = s[kf][r] * sl2;
        if (key > qpos || key >= L) x = -INFINITY;
        s[kf][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_i, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_i - m_use);
    float rs = 0.f;
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2f(s[kf][r] - m_use);
        s[kf][r] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32, 64);
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int df = 0; df < 4; ++df)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[df][r] *= alpha;

#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int kf = kc >> 1, c = kc & 1;
      bf16x8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = (bf16)s[kf][8 * c + e];
#pragma unroll
      for (int df = 0; df < 4; ++df)
        o[df] = mfma32(read_t_frag(sVt, df * 32 + lr, kf * 32 + 16 * c + 4 * lh), pb, o[df]);
    }
  }

  if (qok) {
    const float inv_l = 1.f / l_i;
    const long row = st + qpos;
#pragma unroll
    for (int df = 0; df < 4; ++df)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dim = df * 32 + 8 * g + 4 * lh;
        bf16x4 ob;
        f32x4 of;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          of[t] = o[df][4 * g + t] * inv_l;
          ob[t] = (bf16)of[t];
        }
        *reinterpret_cast<bf16x4*>(a.ctx + row * a.ldc + h * HD + dim) = ob;
        if (a.o32) *reinterpret_cast<f32x4*>(a.o32 + row * a.ldo32 + h * HD + dim) = of;
      }
    if (lh == 0) a.lse[(long)h * a.ld_stat + row] = m_i + log2f(l_i);
  }
}

// dsum[h, t] = sum_d dO[t, h*128 + d] * O[t, h*128 + d]
__global__ __launch_bounds__(256) void attn_dsum_kernel(AttnArgs a) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (long)N * a.Hq) return;
  const int t = (int)(item / a.Hq), h = (int)(item % a.Hq), l = threadIdx.x & 63;
  const bf16* d = a.dout + (long)t * a.lddo + h * HD;
  const float* o = a.o32 + (long)t * a.ldo32 + h * HD;
  float v = (float)d[l] * o[l] + (float)d[l + 64] * o[l + 64];
  v = wave_sum(v);
  if (l == 0) a.dsum[(long)h * a.ld_stat + t] = v;
}

__global__ __launch_bounds__(256) void attn_dq_kernel(AttnArgs a) {
  const int tile = blockIdx.x;
  if (tile >= *a.ntiles_dev) return;
  const int h = blockIdx.y, kvh = h / (a.Hq / a.Hkv);
  const int4 tl = a.tiles[tile];
  const int st = tl.x, L = tl.y, q0 = tl.z;
  __shared__ __attribute__((aligned(16))) bf16 sK[64 * SN];
  __shared__ __attribute__((aligned(16))) bf16 sKt[HD * ST];
  __shared__ __attribute__((aligned(16))) bf16 sV[64 * SN];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, lh = lane >> 5;
  const int qpos = q0 + w * 32 + lr;
  const bool qok = qpos < L;

  bf16x8 qf[8], df_[8];
  load_row_frags(a.q, a.ldq, st + qpos, h * HD, qok, lh, qf);
  load_row_frags(a.dout, a.lddo, st + qpos, h * HD, qok, lh, df_);
  const float lse2 = qok ? a.lse[(long)h * a.ld_stat + st + qpos] : 0.f;
  const float dsum = qok ? a.dsum[(long)h * a.ld_stat + st + qpos] : 0.f;

  f32x16 dq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  const float sl2 = kScale * kLog2e;
  const int kv_end = min(L, q0 + 128);

  for (int k0 = 0; k0 < kv_end; k0 += 64) {
    __syncthreads();
    stage_tile(a.k, a.ldk, kvh * HD, st, k0, L, sK, sKt);
    stage_tile(a.v, a.ldv, kvh * HD, st, k0, L, sV, nullptr);
    __syncthreads();

    f32x16 s[2], dp[2];
#pragma unroll
    for (int kf = 0; kf < 2; ++kf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[kf][r] = 0.f; dp[kf][r] = 0.f; }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        s[kf] = mfma32(read_n_frag(sK, kf * 32 + lr, kk * 16 + lh * 8), qf[kk], s[kf]);
        dp[kf] = mfma32(read_n_frag(sV, kf * 32 + lr, kk * 16 + lh * 8), df_[kk], dp[kf]);
      }
    }
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + kf * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        const bool ok = qok && key <= qpos && key < L;
        const float p = ok ? exp2f(s[kf][r] * sl2 - lse2) : 0.f;
        s[kf][r] = p * (dp[kf][r] - dsum);
      }
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int kf = kc >> 1, c = kc & 1;
      bf16x8 sb;
#pragma unroll
      for (int e = 0; e < 8; ++e) sb[e] = (bf16)s[kf][8 * c + e];
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4)
        dq[d4] = mfma32(read_t_frag(sKt, d4 * 32 + lr, kf * 32 + 16 * c + 4 * lh), sb, dq[d4]);
    }
  }

  if (qok) {
    const long row = st + qpos;
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dim = d4 * 32 + 8 * g + 4 * lh;
        bf16x4 ob;
#pragma unroll
        for (int t = 0; t < 4; ++t) ob[t] = (bf16)(dq[d4][4 * g + t] * kScale);
        *reinterpret_cast<bf16x4*>(a.dq + row * a.lddq + h * HD + dim) = ob;
      }
  }
}

__global__ __launch_bounds__(256) void attn_dkdv_kernel(AttnArgs a) {
  const int tile = blockIdx.x;
  if (tile >= *a.ntiles_dev) return;
  const int kvh = blockIdx.y, G = a.Hq / a.Hkv;
  const int4 tl = a.tiles[tile];
  const int st = tl.x, L = tl.y, k0 = tl.z;
  __shared__ __attribute__((aligned(16))) bf16 sQ[64 * SN];
  __shared__ __attribute__((aligned(16))) bf16 sQt[HD * ST];
  __shared__ __attribute__((aligned(16))) bf16 sO[64 * SN];
  __shared__ __attribute__((aligned(16))) bf16 sOt[HD * ST];
  __shared__ float sL[64], sD[64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 31, lh = lane >> 5;
  const int key = k0 + w * 32 + lr;
  const bool kok = key < L;

  bf16x8 kf_[8], vf_[8];
  load_row_frags(a.k, a.ldk, st + key, kvh * HD, kok, lh, kf_);
  load_row_frags(a.v, a.ldv, st + key, kvh * HD, kok, lh, vf_);

  f32x16 dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[i][r] = 0.f; dv[i][r] = 0.f; }
  const float sl2 = kScale * kLog2e;

  for (int hq = kvh * G; hq < kvh * G + G; ++hq) {
    for (int q0 = k0; q0 < L; q0 += 64) {
      __syncthreads();
      stage_tile(a.q, a.ldq, hq * HD, st, q0, L, sQ, sQt);
      stage_tile(a.dout, a.lddo, hq * HD, st, q0, L, sO, sOt);
      if (tid < 64) {
        const bool ok = q0 + tid < L;
        sL[tid] = ok ? a.lse[(long)hq * a.ld_stat + st + q0 + tid] : 0.f;
        sD[tid] = ok ? a.dsum[(long)hq * a.ld_stat + st + q0 + tid] : 0.f;
      }
      __syncthreads();

      f32x16 s[2], dp[2];
#pragma unroll
      for (int qf = 0; qf < 2; ++qf) {
#pragma unroll
        for (int r = 0; r < 16; ++r) { s[qf][r] = 0.f; dp[qf][r] = 0.f; }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          s[qf] = mfma32(read_n_frag(sQ, qf * 32 + lr, kk * 16 + lh * 8), kf_[kk], s[qf]);
          dp[qf] = mfma32(read_n_frag(sO, qf * 32 + lr, kk * 16 + lh * 8), vf_[kk], dp[qf]);
        }
      }
#pragma unroll
      for (int qf = 0; qf < 2; ++qf)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = qf * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          const int query = q0 + qi;
          const bool ok = kok && query < L && query >= key;
          const float p = ok ? exp2f(s[qf][r] * sl2 - sL[qi]) : 0.f;
          s[qf][r] = p;
          dp[qf][r] = p * (dp[qf][r] - sD[qi]);
        }
#pragma unroll
      for (int qc = 0; qc < 4; ++qc) {
        const int qf = qc >> 1, c = qc & 1;
        bf16x8 pb, sb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pb[e] = (bf16)s[qf][8 * c + e];
          sb[e] = (bf16)dp[qf][8 * c + e];
        }
        const int col = qf * 32 + 16 * c + 4 * lh;
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) {
          dv[d4] = mfma32(read_t_frag(sOt, d4 * 32 + lr, col), pb, dv[d4]);
          dk[d4] = mfma32(read_t_frag(sQt, d4 * 32 + lr, col), sb, dk[d4]);
        }
      }
    }
  }

  if (kok) {
    const long row = st + key;
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dim = d4 * 32 + 8 * g + 4 * lh;
        bf16x4 kb, vb;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          kb[t] = (bf16)(dk[d4][4 * g + t] * kScale);
          vb[t] = (bf16)dv[d4][4 * g + t];
        }
        *reinterpret_cast<bf16x4*>(a.dk + row * a.lddk + kvh * HD + dim) = kb;
        *reinterpret_cast<bf16x4*>(a.dv + row * a.lddv + kvh * HD + dim) = vb;
      }
  }
}

hipError_t attn_fwd(const AttnArgs& a, hipStream_t s) {
  if (a.max_tiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(a.max_tiles, a.Hq), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t attn_bwd_prep(const AttnArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const long items = (long)a.n * a.Hq;
  hipLaunchKernelGGL(attn_dsum_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t attn_bwd_dkdv(const AttnArgs& a, hipStream_t s) {
  if (a.max_tiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_dkdv_kernel, dim3(a.max_tiles, a.Hkv), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t attn_bwd_dq(const AttnArgs& a, hipStream_t s) {
  if (a.max_tiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_dq_kernel, dim3(a.max_tiles, a.Hq), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t attn_bwd(const AttnArgs& a, hipStream_t s) {
  hipError_t e;
  if ((e = attn_bwd_prep(a, s)) != hipSuccess) return e;
  if ((e = attn_bwd_dkdv(a, s)) != hipSuccess) return e;
  return attn_bwd_dq(a, s);
}

}  // namespace dsb
