// bf16 "NT" GEMM for gfx950: C[M,N] = A[M,K1]·B[N,K1]ᵀ (+ A2[M,K2]·B2[N,K2]ᵀ)
// with a pluggable epilogue.
//
// Every dense contraction of the backward is phrased in this one form (both
// operands K-contiguous): forward recompute uses the frozen weight [out,in] as
// is, the dX products use the transposed copy made once at bind time, and the
// LoRA factor rides along as a second K segment (K-concatenation), so
// y = x·Wᵀ + (x·Aᵀ)·(s·B)ᵀ is one kernel with K = in + r.
//
// Tiling: BM×BN block tile, BK = 64, WM×WN waves, each wave owns a
// (BM/WM)×(BN/WN) sub-tile of 32×32 MFMA fragments. Global→LDS staging is
// double-buffered through registers (one barrier per K step) with buffer
// loads: rows past M/N fall outside the descriptor and read as zero, and the
// first use of a loaded value is the LDS store after the MFMAs of the current
// step, so the loads overlap the math. LDS rows are 128 B with a 16-byte-chunk
// XOR swizzle so fragment reads of 16 consecutive rows hit distinct banks.
// Block ids are remapped so each XCD (round-robin dispatch over 8 XCDs) gets a
// contiguous run of tiles, grouped 8 deep along M for L2 reuse.
#pragma once

#include "dsb_common.h"

namespace dsb {

struct GemmProblem {
  const bf16* A;
  long lda;
  const bf16* B;
  long ldb;
  const bf16* A2;  // optional second K segment (LoRA); K2 = 0 disables
  long lda2;
  const bf16* B2;
  long ldb2;
  int M, N, K1, K2;
  const int* M_dev;  // optional device-resident row count (min with M)
};

DSB_DEV void tile_map(int bid, int nbm, int nbn, int& pm, int& pn) {
  const int total = nbm * nbn;
  int lid = bid;
  if ((total & 7) == 0) lid = (bid & 7) * (total >> 3) + (bid >> 3);
  constexpr int GM = 8;
  const int per_group = GM * nbn;
  const int gid = lid / per_group;
  const int first_m = gid * GM;
  const int gsz = min(nbm - first_m, GM);
  const int r = lid - gid * per_group;
  pm = first_m + r % gsz;
  pn = r / gsz;
}

// Visit the accumulator as runs of 4 consecutive output columns of one row.
template <int FM, int FN, class F>
DSB_DEV void for_each_quad(const f32x16 (&acc)[FM][FN], int mw, int nw, int M,
                           int lane, F&& f) {
  const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = mw + fm * 32 + lr;
    if (m >= M) continue;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = nw + fn * 32 + 8 * g + 4 * lh;
        float v[4] = {acc[fm][fn][4 * g], acc[fm][fn][4 * g + 1],
                      acc[fm][fn][4 * g + 2], acc[fm][fn][4 * g + 3]};
        f(m, n, v);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, class Epi>
__global__ __launch_bounds__(WM* WN * 64)
__attribute__((amdgpu_waves_per_eu(WM* WN / 4, WM* WN / 4))) void gemm_nt_kernel(GemmProblem p, Epi epi) {
  constexpr int BK = 64, CH = 8;
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int LA = BM * CH / NT, LB = BN * CH / NT;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be 32-aligned");
  static_assert((BM * CH) % NT == 0 && (BN * CH) % NT == 0, "loader split");
  constexpr int SA = BM * BK, SB = BN * BK;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * (SA + SB)];

  int M = p.M;
  if (p.M_dev) M = min(M, *p.M_dev);
  const int nbm = (p.M + BM - 1) / BM, nbn = (p.N + BN - 1) / BN;
  int pm, pn;
  tile_map(blockIdx.x, nbm, nbn, pm, pn);
  const int m0 = pm * BM, n0 = pn * BN;
  if (m0 >= M) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int nk1 = (p.K1 + BK - 1) / BK;
  const int nk2 = p.K2 > 0 ? (p.K2 + BK - 1) / BK : 0;
  const int nk = nk1 + nk2;

  // Buffer resources over this tile's rows of each operand: rows past M (N)
  // fall outside num_records and load as zeros. Thread t loads 16-byte chunk
  // ch = t % 8 of rows t/8 + i·(NT/8); the row step goes in the scalar offset.
  constexpr int RSTEP = NT / CH;
  const int ch = tid % CH, r0 = tid / CH;
  const int rowsA = min(M - m0, BM), rowsB = min(p.N - n0, BN);
  auto rsrc = [](const bf16* base, long ld, int rows, int K) {
    const long bytes = rows > 0 ? (((long)(rows - 1) * ld + K) * 2) : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
  };
  const __amdgpu_buffer_rsrc_t ra1 = rsrc(p.A + (long)m0 * p.lda, p.lda, rowsA, p.K1);
  const __amdgpu_buffer_rsrc_t rb1 = rsrc(p.B + (long)n0 * p.ldb, p.ldb, rowsB, p.K1);
  const __amdgpu_buffer_rsrc_t ra2 = rsrc(p.A2 ? p.A2 + (long)m0 * p.lda2 : p.A, p.lda2, nk2 ? rowsA : 0, p.K2);
  const __amdgpu_buffer_rsrc_t rb2 = rsrc(p.B2 ? p.B2 + (long)n0 * p.ldb2 : p.B, p.ldb2, nk2 ? rowsB : 0, p.K2);
  const int voffA1 = (int)(r0 * p.lda * 2 + ch * 16), voffB1 = (int)(r0 * p.ldb * 2 + ch * 16);
  const int voffA2 = (int)(r0 * p.lda2 * 2 + ch * 16), voffB2 = (int)(r0 * p.ldb2 * 2 + ch * 16);

  u32x4 ra[LA], rb[LB];
  bool kok = true;  // this thread's chunk lies below K (only the last K step can fail)
  auto gload = [&](int kt) {
    if (kt < nk1) {
      const int k0 = kt * BK;
      kok = k0 + ch * 8 < p.K1;
#pragma unroll
      for (int i = 0; i < LA; ++i)
        ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra1, voffA1, (int)(i * RSTEP * p.lda * 2 + k0 * 2), 0);
#pragma unroll
      for (int i = 0; i < LB; ++i)
        rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb1, voffB1, (int)(i * RSTEP * p.ldb * 2 + k0 * 2), 0);
    } else {
      const int k0 = (kt - nk1) * BK;
      kok = k0 + ch * 8 < p.K2;
#pragma unroll
      for (int i = 0; i < LA; ++i)
        ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra2, voffA2, (int)(i * RSTEP * p.lda2 * 2 + k0 * 2), 0);
#pragma unroll
      for (int i = 0; i < LB; ++i)
        rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb2, voffB2, (int)(i * RSTEP * p.ldb2 * 2 + k0 * 2), 0);
    }
  };
  // LDS: [row][8 × 16-byte chunks], chunk slot = ch ^ ((row >> 1) & 7) so that
  // 16 consecutive rows read at one logical chunk hit 16 distinct bank groups.
  auto slot = [](int row, int c) { return row * BK + ((c ^ ((row >> 1) & 7)) << 3); };
  auto sstore = [&](int buf) {
    bf16* sA = smem + buf * (SA + SB);
    bf16* sB = sA + SA;
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < LA; ++i)
      *reinterpret_cast<u32x4*>(sA + slot(r0 + i * RSTEP, ch)) = kok ? ra[i] : zero;
#pragma unroll
    for (int i = 0; i < LB; ++i)
      *reinterpret_cast<u32x4*>(sB + slot(r0 + i * RSTEP, ch)) = kok ? rb[i] : zero;
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int lr = lane & 31, lh = lane >> 5;
  // Fragments double-buffered across the four 16-deep K slices of a step: the
  // LDS reads of slice kk+1 are issued before the MFMAs of slice kk.
  bf16x8 af[2][FM], bfr[2][FN];
  auto load_frags = [&](const bf16* sA, const bf16* sB, int kk, int b) {
    const int kc = kk * 2 + lh;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
      af[b][fm] = *reinterpret_cast<const bf16x8*>(sA + slot(wm * TM + fm * 32 + lr, kc));
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
      bfr[b][fn] = *reinterpret_cast<const bf16x8*>(sB + slot(wn * TN + fn * 32 + lr, kc));
  };
  auto compute = [&](int buf) {
    const bf16* sA = smem + buf * (SA + SB);
    const bf16* sB = sA + SA;
    load_frags(sA, sB, 0, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) load_frags(sA, sB, kk + 1, (kk + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] = mfma32(bfr[kk & 1][fn], af[kk & 1][fm], acc[fm][fn]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    compute(cur);
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  epi.template run<FM, FN, WM, WN>(acc, m0 + wm * TM, n0 + wn * TN, M, lane, wave,
                                   (void*)smem);
}

// ---------------------------------------------------------------- epilogues

// C = acc (+ R), bf16 out. R (optional) is a bf16 residual of the same shape.
struct EpiBF16 {
  bf16* C;
  long ldc;
  int N;
  const bf16* R;
  long ldr;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x16 (&acc)[FM][FN], int mw, int nw, int M, int lane,
                   int, void*) const {
    for_each_quad(acc, mw, nw, M, lane, [&](int m, int n, float* v) {
      if (n + 3 < N) {
        if (R) {
          const bf16x4 r = *reinterpret_cast<const bf16x4*>(R + (long)m * ldr + n);
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] += (float)r[i];
        }
        bf16x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (bf16)v[i];
        *reinterpret_cast<bf16x4*>(C + (long)m * ldc + n) = o;
      } else {
        for (int i = 0; i < 4 && n + i < N; ++i) {
          float x = v[i];
          if (R) x += (float)R[(long)m * ldr + n + i];
          C[(long)m * ldc + n + i] = (bf16)x;
        }
      }
    });
  }
};

// C (+)= acc, fp32 out.
struct EpiF32 {
  float* C;
  long ldc;
  int N;
  int accumulate;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x16 (&acc)[FM][FN], int mw, int nw, int M, int lane,
                   int, void*) const {
    for_each_quad(acc, mw, nw, M, lane, [&](int m, int n, float* v) {
      float* c = C + (long)m * ldc + n;
      if (n + 3 < N) {
        f32x4 o = {v[0], v[1], v[2], v[3]};
        if (accumulate) o += *reinterpret_cast<const f32x4*>(c);
        *reinterpret_cast<f32x4*>(c) = o;
      } else {
        for (int i = 0; i < 4 && n + i < N; ++i) c[i] = accumulate ? c[i] + v[i] : v[i];
      }
    });
  }
};

// SwiGLU backward fused into the down-projection dX product:
//   gh = acc (grad wrt h = silu(gate)·up), gate = GU[m, n], up = GU[m, I + n]
//   G[m, n] = gh·up·silu'(gate), G[m, I + n] = gh·silu(gate)
// with silu'(g) = σ(g)·(1 + g·(1 − σ(g))).
struct EpiSwiGLUBwd {
  const bf16* GU;
  long ldgu;
  bf16* G;
  long ldg;
  int I;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x16 (&acc)[FM][FN], int mw, int nw, int M, int lane,
                   int, void*) const {
    for_each_quad(acc, mw, nw, M, lane, [&](int m, int n, float* v) {
      if (n >= I) return;
      const bf16x4 g4 = *reinterpret_cast<const bf16x4*>(GU + (long)m * ldgu + n);
      const bf16x4 u4 = *reinterpret_cast<const bf16x4*>(GU + (long)m * ldgu + I + n);
      bf16x4 og, ou;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = (float)g4[i], u = (float)u4[i];
        const float sg = 1.f / (1.f + __expf(-g));
        const float silu = g * sg;
        const float dsilu = sg * (1.f + g * (1.f - sg));
        og[i] = (bf16)(v[i] * u * dsilu);
        ou[i] = (bf16)(v[i] * silu);
      }
      *reinterpret_cast<bf16x4*>(G + (long)m * ldg + n) = og;
      *reinterpret_cast<bf16x4*>(G + (long)m * ldg + I + n) = ou;
    });
  }
};

// Skinny LoRA products (N = r or a few r): Zf = sf·acc (fp32), Zb = bf16(sb·acc).
struct EpiLoraZ {
  float* Zf;
  long ldzf;
  float sf;
  bf16* Zb;
  long ldzb;
  float sb;
  int N;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x16 (&acc)[FM][FN], int mw, int nw, int M, int lane,
                   int, void*) const {
    for_each_quad(acc, mw, nw, M, lane, [&](int m, int n, float* v) {
      for (int i = 0; i < 4 && n + i < N; ++i) {
        if (Zf) Zf[(long)m * ldzf + n + i] = sf * v[i];
        if (Zb) Zb[(long)m * ldzb + n + i] = (bf16)(sb * v[i]);
      }
    });
  }
};

// Tile configurations. Big: 256×256, 4 waves of 128×128 (256 accumulators per
// lane). Mid: 128×128, 4 waves of 64×64. Skinny: 64×64, 4 waves of 32×32.
enum GemmCfg { GEMM_BIG = 0, GEMM_MID = 1, GEMM_SKINNY = 2 };

template <int BM, int BN, int WM, int WN, class Epi>
hipError_t launch_gemm_cfg(const GemmProblem& p, const Epi& e, hipStream_t s) {
  const int nbm = (p.M + BM - 1) / BM, nbn = (p.N + BN - 1) / BN;
  if (nbm == 0 || nbn == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, WM, WN, Epi>), dim3(nbm * nbn),
                     dim3(WM * WN * 64), 0, s, p, e);
  return hipGetLastError();
}

inline GemmCfg pick_gemm_cfg(int M, int N) {
  if (N <= 64) return GEMM_SKINNY;
  const long big_tiles = (long)((M + 255) / 256) * ((N + 255) / 256);
  if (big_tiles >= 192) return GEMM_BIG;
  return GEMM_MID;
}

template <class Epi>
hipError_t launch_gemm(const GemmProblem& p, const Epi& e, hipStream_t s, int cfg = -1) {
  if (cfg < 0) cfg = pick_gemm_cfg(p.M, p.N);
  switch (cfg) {
    case GEMM_BIG: return launch_gemm_cfg<256, 256, 2, 2>(p, e, s);
    case GEMM_MID: return launch_gemm_cfg<128, 128, 2, 2>(p, e, s);
    default: return launch_gemm_cfg<64, 64, 2, 2>(p, e, s);
  }
}

}  // namespace dsb
