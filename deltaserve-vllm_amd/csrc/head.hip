// Final-norm output → LM head → shifted cross-entropy → dH, streaming the
// vocabulary in chunks: no [rows, vocab] logits, probabilities or dlogits
// ever exist in memory, only a bf16 [rows, chunk] probability tile per chunk.
//
// Semantics: deltaserve-plugin/deltaserve/bwd_services/common/head.py:42-100
//   loss = sum_rows CE(logits, target) / n_valid, dlogits = (softmax - onehot)/n_valid,
//   grad_rows = dlogits · W. Rows that predict nothing (the last token of each
//   sequence) carry label -1 and contribute neither loss nor gradient.
//
// Two vocabulary-wide products, with the softmax normalised online across
// chunks as flash attention normalises across key tiles:
//   per chunk c: logits = H·W_cᵀ (GEMM; its epilogue writes, per 256-column
//     vocabulary tile t, the reference m_t = max(the tile's row max, the
//     running max M of the earlier chunks) and Σ exp(logit − m_t), the target
//     logit where the tile holds it, and P = bf16(exp(logit − m_t)));
//   ce_rescale: per row, the chunk max M_c = max_t m_t, the running max M and
//     sum L updated (M' = max(M, M_c), L' = L·e^(M−M') + Σ_t s_t·e^(m_t−M')),
//     α = e^(M−M'), and P scaled in place by e^(m_t − M') (P = exp(logit − M'))
//     on the rows where some m_t differs from M' (every row of the first
//     chunk; later, only the rows whose maximum lies in the chunk);
//   dH = dH·α + P·W_c (GEMM, fp32 accumulate with the per-row α);
//   after the last chunk: dH = (dH/L − W[target]) / n_valid (the onehot term
//   exactly, in fp32), LSE = M + ln L, loss_row = LSE − target logit, and a
//   single-block deterministic sum gives the cycle loss.
// Against the reference's 2 passes (logits for the LSE, then dlogits, both
// chunked, head.py:78-80, :92-94) this keeps its 2·M·D·V of logits and
// 2·M·D·V of dH and needs no third product. P passes through bf16 (the MFMA
// operand type) where the reference keeps probabilities in fp32; dH
// accumulates in fp32. The chunk is the reference's VOCAB_CHUNK unit; the
// caller can pause between a chunk's two products and between chunks.
#include "gemm_nt.h"
#include "kernels.h"

namespace dsb {

namespace {
constexpr int CE_BN = 256;

// Per vocab tile (ce_bn columns) of chunk [c0, c0 + Vc): (reference m_t, sum
// exp(logit − m_t)) per row into stats[m, c0/ce_bn + tile], m_t being the
// tile's row max or, from the second chunk on, the running max when that is
// larger; the target logit
// where the tile holds it, and P[m, j] = bf16(exp(logit[m, c0 + j] − m_t)) for
// the chunk's columns j < Vc; columns [Vc, Nc8) (Nc8 = round_up(Vc, 8)) are
// written as zero so the dH product runs its K loop over whole 16-byte chunks.
struct EpiCEProb {
  const int* labels;
  float2* stats;
  int ntn;
  float* tgt_logit;
  bf16* P;
  long ldp;
  int c0, Vc, Nc8;
  // the running max over the earlier chunks (null for the first chunk): each
  // tile's reference is max(tile max, running max), so a row whose maximum is
  // not in this chunk has one reference for all its tiles and needs no rescale
  const float* run_m;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    constexpr int TM = FM * 16, TN = FN * 16, BMl = WM * TM;
    constexpr int PITCH = TN + 4, CG = TN / 8, RPI = 64 / CG;
    constexpr int STG = WM * WN * 32 * PITCH;  // for the staging rows of every wave
    static_assert((STG + 2 * BMl + WN * BMl) * 4 <= 2 * (WM * TM + WN * TN) * 64 * 2,
                  "epilogue scratch fits the stages");
    const int wn = wave % WN, wm = wave / WN;
    const int n0 = nw - wn * TN;
    const int pn = c0 / (WN * TN) + n0 / (WN * TN);
    // lane l holds row l%16 of each 16-row block, columns 4(l/16) .. +3 of
    // each 16-column block: a row's values of the wave tile sit in the four
    // lanes l%16 + 16q, combined with two shuffles
    const int l16 = lane & 15, lq = lane >> 4;
    float* fs = reinterpret_cast<float*>(smem);
    float* red = fs;               // [WN][BMl] per-wave row maxima, before the staging rows
    float* rowmax = fs + STG;      // [BMl] the tile's row maxima
    float* rowsum = rowmax + BMl;  // [WN][BMl] per-wave row sums of exp(logit − max)
    int* tcol = reinterpret_cast<int*>(rowsum + WN * BMl);  // [BMl] target column in the chunk, or -1
    // 1) row maxima over the tile's live columns (every column of the wave
    //    tile is live except in the chunk's last tile: one wave-uniform test)
    const bool whole = nw + TN <= Vc;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      float v = -INFINITY;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = acc[fm][fn][i];
          v = (whole || nw + fn * 16 + 4 * lq + i < Vc) ? fmaxf(v, x) : v;
        }
      v = fmaxf(v, __shfl_xor(v, 16, 64));
      v = fmaxf(v, __shfl_xor(v, 32, 64));
      if (lq == 0) red[wn * BMl + wm * TM + fm * 16 + l16] = v;
    }
    // The accumulators' copies read above die here: the empty asm claims to
    // rewrite each one in its AGPRs, so phase 2 reads them from there again
    // instead of the compiler keeping VGPR copies across the barriers.
    auto& accw = const_cast<f32x4 (&)[FM][FN]>(acc);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) asm volatile("" : "+a"(accw[fm][fn]));
    __syncthreads();
    if (wn == 0 && lq == 0) {
      // the rows' labels and running maxima, all loaded before the first is
      // used (rows past M read row M − 1 and are not used): loads behind a
      // per-row test would each wait for the one before
      int lab[FM];
      float rmx[FM];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) lab[fm] = labels[min(mw + fm * 16 + l16, M - 1)];
      if (run_m) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) rmx[fm] = run_m[min(mw + fm * 16 + l16, M - 1)];
      } else {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) rmx[fm] = -INFINITY;
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * TM + fm * 16 + l16, m = mw + fm * 16 + l16;
        float b = red[row];
#pragma unroll
        for (int j = 1; j < WN; ++j) b = fmaxf(b, red[j * BMl + row]);
        if (run_m) b = fmaxf(b, rmx[fm]);
        rowmax[row] = b;
        const int t = m < M ? lab[fm] - c0 : -1;
        tcol[row] = t >= 0 && t < Vc ? t : -1;
      }
    }
    // the maxima are visible, and every wave is past its reads of `red`,
    // before the staging rows overwrite it
    __syncthreads();
    // 2) P = bf16(exp(logit − max)) through the staging rows (one exp per
    //    logit), each row's sum of the fp32 values reduced on the way: the
    //    CG lanes of a staged row are consecutive
    const int m0 = mw - wm * TM;
    float* buf = fs + wave * 32 * PITCH;
    const int rsub = lane / CG, cg = lane % CG;
    const int n = nw + cg * 8;
#pragma unroll
    for (int b = 0; b < FM / 2; ++b) {
      if (mw + b * 32 >= M) break;  // uniform: the rest of the wave tile is past M
      stage32<FM, FN, PITCH>(acc, b, buf, lane);
#pragma unroll
      for (int it = 0; it < 32 / RPI; ++it) {
        const int row = it * RPI + rsub, lrow = wm * TM + b * 32 + row, m = m0 + lrow;
        const f32x4 x = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8);
        const f32x4 y = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8 + 4);
        const float v[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
        const float bm = rowmax[lrow];
        // the target logit, where the row's target column is one of these 8
        const int tj = tcol[lrow] - n;
        if (m < M && (unsigned)tj < 8u) {
          float x = v[0];
#pragma unroll
          for (int i = 1; i < 8; ++i) x = tj == i ? v[i] : x;
          tgt_logit[m] = x;
        }
        float e[8], part = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          e[i] = (whole || n + i < Vc) ? __expf(v[i] - bm) : 0.f;
          part += e[i];
        }
#pragma unroll
        for (int o = 1; o < CG; o <<= 1) part += __shfl_xor(part, o, 64);
        if (cg == 0) rowsum[wn * BMl + lrow] = part;
        const int lim = Nc8 - n;
        if (m < M && lim > 0) {
          bf16* d = P + (long)m * ldp + n;
          if (lim >= 8) {
            stg128(d, pack8(e));
          } else {
            for (int i = 0; i < lim; ++i) d[i] = (bf16)e[i];
          }
        }
      }
    }
    __syncthreads();
    // 3) the tile's (max, sum) per row
    if (wn == 0 && lq == 0) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * TM + fm * 16 + l16;
        const int m = mw + fm * 16 + l16;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < WN; ++j) s += rowsum[j * BMl + row];
        if (m < M) stats[(long)m * ntn + pn] = make_float2(rowmax[row], s);
      }
    }
  }
};

}  // namespace

// Chunk [c0, c0 + Vc) after its logits product, one wave per live row: the
// chunk max M_c of the tile references m_t and its sum, the running max M and
// sum L (first chunk: M = −inf, L = 0) moved to M' = max(M, M_c), α = e^(M − M')
// for the dH accumulator, and P scaled in place by e^(m_t − M') per tile, so
// P = bf16(exp(logit − M')). After the first chunk every m_t is at least M, so
// a row whose maximum is not in this chunk has m_t = M = M' for every tile and
// its P is left as it is; so are the rows without a target, whose dH the
// finalize sets to zero whatever the product accumulated (P <= 1: finite).
__global__ __launch_bounds__(256) void ce_rescale_kernel(HeadArgs a, int c0, int first) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (m >= N) return;
  const int bn = a.ce_bn, Vc = min(a.vchunk, a.V - c0), Nc8 = (Vc + 7) / 8 * 8;
  const int nt = (Vc + bn - 1) / bn;
  const float2* st = a.stats + (long)m * a.ntn + c0 / bn;
  float mc = -INFINITY;
  for (int j = l; j < nt; j += 64) mc = fmaxf(mc, st[j].x);
  mc = wave_max(mc);
  const float mo = first ? -INFINITY : a.run_m[m];
  const float mn = fmaxf(mo, mc);
  float sc = 0.f;
  for (int j = l; j < nt; j += 64) sc += st[j].y * __expf(st[j].x - mn);
  sc = wave_sum(sc);
  if (l == 0) {
    const float al = first ? 0.f : __expf(mo - mn);
    a.run_m[m] = mn;
    a.run_l[m] = (first ? 0.f : a.run_l[m] * al) + sc;
    a.alpha[m] = al;
  }
  if (a.labels[m] < 0) return;
  bool scaled = false;
  for (int j = l; j < nt; j += 64) scaled |= st[j].x != mn;
  if (!__any(scaled)) return;
  bf16* pr = a.dlog + (long)m * a.vchunk;
#pragma unroll 4
  for (int k = l; k < Nc8 / 8; k += 64) {
    u32x4* q = reinterpret_cast<u32x4*>(pr + 8 * k);
    const float f = __expf(st[(8 * k) / bn].x - mn);
    float v[8];
    unpack8(*q, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= f;
    *q = pack8(v);
  }
}

// After the last chunk, one wave per live row: LSE = M + ln L, loss_row =
// LSE − target logit, dH = (dH/L − W[target]) / n_valid; rows without a target
// get dH = 0 and no loss.
__global__ __launch_bounds__(256) void ce_finalize_kernel(HeadArgs a) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (m >= N) return;
  const int t = a.labels[m];
  float* dr = a.dH + (long)m * a.D;
  if (t < 0) {
    for (int k = l; k < a.D / 4; k += 64)
      reinterpret_cast<f32x4*>(dr)[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (l == 0) a.loss_row[m] = 0.f;
    return;
  }
  const float L = a.run_l[m], lse = a.run_m[m] + __logf(L);
  if (l == 0) {
    a.lse[m] = lse;
    a.loss_row[m] = lse - a.tgt_logit[m];
  }
  const float inv = 1.f / L, sc = *a.inv_nvalid;
  const bf16* w = a.W + (long)t * a.D;
  for (int k = l; k < a.D / 8; k += 64) {
    float wf[8];
    unpack8(ldg128(w + 8 * k), wf);
    f32x4* d = reinterpret_cast<f32x4*>(dr + 8 * k);
    const f32x4 x0 = d[0], x1 = d[1];
    d[0] = f32x4{(x0[0] * inv - wf[0]) * sc, (x0[1] * inv - wf[1]) * sc,
                 (x0[2] * inv - wf[2]) * sc, (x0[3] * inv - wf[3]) * sc};
    d[1] = f32x4{(x1[0] * inv - wf[4]) * sc, (x1[1] * inv - wf[5]) * sc,
                 (x1[2] * inv - wf[6]) * sc, (x1[3] * inv - wf[7]) * sc};
  }
}

// Deterministic single-block sum of loss_row[0:n) times 1/n_valid.
__global__ __launch_bounds__(1024) void ce_loss_kernel(const float* __restrict__ loss_row,
                                                       int n, const int* n_dev,
                                                       const float* inv_nvalid,
                                                       float* __restrict__ out) {
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  __shared__ float red[16];
  float s = 0.f;
  for (int i = threadIdx.x; i < N; i += 1024) s += loss_row[i];
  s = block_sum<1024>(s, red);
  if (threadIdx.x == 0) out[0] = s * (*inv_nvalid);
}

int head_num_chunks(const HeadArgs& a) { return (a.V + a.vchunk - 1) / a.vchunk; }

static GemmProblem chunk_logits_problem(const HeadArgs& a, int c0) {
  const int Vc = min(a.vchunk, a.V - c0);
  return GemmProblem{a.normed, a.ldh, a.W + (long)c0 * a.D, (long)a.D, nullptr, 0, nullptr, 0,
                     a.n, Vc, a.D, 0, a.n_dev};
}

hipError_t head_prob(const HeadArgs& a, int c0, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const int Vc = min(a.vchunk, a.V - c0), Nc8 = (Vc + 7) / 8 * 8;
  EpiCEProb epi{a.labels, a.stats, a.ntn, a.tgt_logit, a.dlog, (long)a.vchunk, c0, Vc, Nc8,
                c0 > 0 ? a.run_m : nullptr};
  if (a.ce_bn == 128) return launch_gemm_cfg<256, 128, 2, 2>(chunk_logits_problem(a, c0), epi, s);
  return launch_gemm_cfg<256, CE_BN, 2, 2>(chunk_logits_problem(a, c0), epi, s);
}

hipError_t head_rescale(const HeadArgs& a, int c0, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(ce_rescale_kernel, dim3((a.n + 3) / 4), dim3(256), 0, s, a, c0,
                     c0 == 0 ? 1 : 0);
  return hipGetLastError();
}

hipError_t head_finalize(const HeadArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(ce_finalize_kernel, dim3((a.n + 3) / 4), dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ce_loss_kernel, dim3(1), dim3(1024), 0, s, a.loss_row, a.n, a.n_dev,
                     a.inv_nvalid, a.loss_out);
  return hipGetLastError();
}

int head_dh_split(const HeadArgs& a, int c0) {
  if (a.gemm_cfg >= 0 || !a.part) return 1;
  const int Nc8 = (min(a.vchunk, a.V - c0) + 7) / 8 * 8;
  const int ks = gemm_split_count(a.n, a.D, Nc8);
  return ks > 1 && (long)ks * a.n * a.D <= a.part_elems ? ks : 1;
}

int head_dh_tail(const HeadArgs& a, int c0, int* tail) {
  *tail = 0;
  if (a.gemm_cfg >= 0 || !a.part || head_dh_split(a, c0) > 1) return 1;
  const int Nc8 = (min(a.vchunk, a.V - c0) + 7) / 8 * 8;
  const int kt = gemm_tail_split(a.n, a.D, Nc8, a.ncu, tail);
  return kt > 1 && (long)kt * *tail * 65536 <= a.part_elems ? kt : 1;
}

hipError_t head_chunk_dh(const HeadArgs& a, int c0, hipStream_t s) {
  const int Nc8 = (min(a.vchunk, a.V - c0) + 7) / 8 * 8;
  // dH = dH·α + P[:, chunk] · W[chunk, :]: the head read in place as the
  // [K, N] operand, rows past the vocabulary loading as zeros
  GemmProblem q{a.dlog, (long)a.vchunk, a.W + (long)c0 * a.D, (long)a.D, nullptr, 0, nullptr, 0,
                a.n, a.D, Nc8, 0, a.n_dev};
  q.b_kn = 1;
  q.kb_rows = min(a.vchunk, a.V - c0);
  EpiF32 ef{a.dH, (long)a.D, a.D, c0 > 0 ? 1 : 0, a.alpha};
  const int ks = head_dh_split(a, c0);
  if (ks > 1) {
    q.part = a.part;
    return launch_gemm_split(q, ef, ks, s);
  }
  int tail = 0;
  const int kt = head_dh_tail(a, c0, &tail);
  if (kt > 1) return launch_gemm_tail(q, ef, kt, tail, a.part, s);
  return launch_gemm(q, ef, s, a.gemm_cfg);
}

hipError_t head_fwd_bwd(const HeadArgs& a, hipStream_t s) {
  hipError_t e;
  if (a.n <= 0) return hipSuccess;
  for (int c0 = 0; c0 < a.V; c0 += a.vchunk) {
    if ((e = head_prob(a, c0, s)) != hipSuccess) return e;
    if ((e = head_rescale(a, c0, s)) != hipSuccess) return e;
    if ((e = head_chunk_dh(a, c0, s)) != hipSuccess) return e;
  }
  return head_finalize(a, s);
}

}  // namespace dsb
