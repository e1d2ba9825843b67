// Final-norm output → LM head → shifted cross-entropy → dH, streaming the
// vocabulary in chunks: no [rows, vocab] logits, probabilities or dlogits
// ever exist in memory, only a bf16 [rows, chunk] dlogits tile per chunk.
//
// Semantics: deltaserve-plugin/deltaserve/bwd_services/common/head.py:42-100
//   loss = sum_rows CE(logits, target) / n_valid, dlogits = (softmax - onehot)/n_valid,
//   grad_rows = dlogits · W. Rows that predict nothing (the last token of each
//   sequence) carry label -1 and contribute neither loss nor gradient.
//
// Pass 1 (LSE), one launch per vocab chunk: an MFMA GEMM logits tile whose
//   epilogue reduces each 256-wide vocab tile to (max, sum exp) per row and
//   picks out the target logit; nothing else is stored.
// Reduce: combine the per-tile statistics into the row LSE and the row loss;
//   a single-block deterministic sum gives the cycle loss.
// Pass 2, per vocab chunk: the same GEMM recomputes the chunk's logits (bit
//   for bit those of pass 1: same kernel, same K order) and its epilogue
//   writes bf16 (exp(logit - lse) - onehot)/n_valid into the chunk's dlogits
//   tile; then dH += dlogits_chunk · W_chunk with the transposed head copy
//   (fp32 accumulate in the epilogue).
// The recompute costs one more 2·M·D·V product than keeping the logits
// (4.2 GB of fp32 at 8192 rows × 128256 vocab), which is what the reference
// does (head.py:84-96); the chunk is the reference's VOCAB_CHUNK unit, so
// the caller can pause between chunks in both passes (head.py:78-80, :92-94).
// dlogits pass through bf16 (the MFMA operand type) where the reference keeps
// them in fp32; the dH product accumulates in fp32.
#include "gemm_nt.h"
#include "kernels.h"

namespace dsb {

namespace {
constexpr int CE_BN = 256;

// Per 256-column vocab tile of chunk [c0, c0 + Vc): (max, sum exp) per row
// into stats[m, c0/256 + tile] and the target logit where the tile holds it.
struct EpiCEStats {
  const int* labels;
  float2* stats;
  int ntn;
  float* tgt_logit;
  int c0, Vc;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    constexpr int TM = FM * 16, TN = FN * 16, BMl = WM * TM;
    static_assert(WN * BMl * 4 <= 2 * (WM * TM + WN * TN) * 64 * 2, "reduction scratch fits");
    const int wn = wave % WN, wm = wave / WN;
    const int n0 = nw - wn * TN;
    const int pn = c0 / (WN * TN) + n0 / (WN * TN);
    // lane l holds row l%16 of each 16-row block, columns 4(l/16) .. +3 of
    // each 16-column block: a row's values of the wave tile sit in the four
    // lanes l%16 + 16q, combined with two shuffles
    const int l16 = lane & 15, lq = lane >> 4;
    float* red = reinterpret_cast<float*>(smem);  // [WN][BMl]
    float mx[FM];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int m = mw + fm * 16 + l16;
      const int t = (m < M) ? labels[m] - c0 : -1;
      float v = -INFINITY;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = nw + fn * 16 + 4 * lq + i;
          const float x = acc[fm][fn][i];
          if (n < Vc) v = fmaxf(v, x);
          if (n == t) tgt_logit[m] = x;
        }
      v = fmaxf(v, __shfl_xor(v, 16, 64));
      mx[fm] = fmaxf(v, __shfl_xor(v, 32, 64));
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
      if (lq == 0) red[wn * BMl + wm * TM + fm * 16 + l16] = mx[fm];
    __syncthreads();
    float sm[FM];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int row = wm * TM + fm * 16 + l16;
      float b = red[row];
#pragma unroll
      for (int j = 1; j < WN; ++j) b = fmaxf(b, red[j * BMl + row]);
      mx[fm] = b;
      float s = 0.f;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = nw + fn * 16 + 4 * lq + i;
          if (n < Vc) s += __expf(acc[fm][fn][i] - b);
        }
      s += __shfl_xor(s, 16, 64);
      sm[fm] = s + __shfl_xor(s, 32, 64);
    }
    __syncthreads();
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
      if (lq == 0) red[wn * BMl + wm * TM + fm * 16 + l16] = sm[fm];
    __syncthreads();
    if (wn == 0 && lq == 0) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * TM + fm * 16 + l16;
        const int m = mw + fm * 16 + l16;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < WN; ++j) s += red[j * BMl + row];
        if (m < M) stats[(long)m * ntn + pn] = make_float2(mx[fm], s);
      }
    }
  }
};

// dlog[m, j] = bf16((exp(logit[m, c0 + j] - lse[m]) - [c0 + j == t_m]) / n_valid)
// for the chunk's columns j < Vc (0 for rows without a target); columns
// [Vc, Nc8) (Nc8 = round_up(Vc, 8)) are written as zero so the dH product
// runs its K loop over whole 16-byte chunks.
struct EpiCEGrad {
  const int* labels;
  const float* lse;
  const float* inv_nvalid;
  bf16* D;
  long ldd;
  int c0, Vc, Nc8;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    const float sc = *inv_nvalid;
    for_each_row8(acc, mw, nw, M, lane, wave, smem, [&](int m, int n, float* v) {
      const int lim = Nc8 - n;
      if (lim <= 0) return;
      const int t = labels[m];
      const float l = lse[m];
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int j = n + i;
        const float e = __expf(v[i] - l) - ((c0 + j) == t ? 1.f : 0.f);
        p[i] = (t >= 0 && j < Vc) ? e * sc : 0.f;
      }
      bf16* d = D + (long)m * ldd + n;
      if (lim >= 8) {
        stg128(d, pack8(p));
      } else {
        for (int i = 0; i < lim; ++i) d[i] = (bf16)p[i];
      }
    });
  }
};

}  // namespace

// One wave per row: combine the per-tile (max, sumexp) pairs.
__global__ __launch_bounds__(256) void ce_reduce_kernel(const float2* __restrict__ stats,
                                                        int ntn, const int* __restrict__ labels,
                                                        const float* __restrict__ tgt_logit,
                                                        float* __restrict__ lse,
                                                        float* __restrict__ loss_row, int n,
                                                        const int* n_dev) {
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (m >= N) return;
  const float2* st = stats + (long)m * ntn;
  float mx = -INFINITY;
  for (int j = l; j < ntn; j += 64) mx = fmaxf(mx, st[j].x);
  mx = wave_max(mx);
  float s = 0.f;
  for (int j = l; j < ntn; j += 64) s += st[j].y * __expf(st[j].x - mx);
  s = wave_sum(s);
  if (l == 0) {
    const float v = mx + __logf(s);
    lse[m] = v;
    loss_row[m] = labels[m] >= 0 ? v - tgt_logit[m] : 0.f;
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

hipError_t head_stats(const HeadArgs& a, int c0, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const int Vc = min(a.vchunk, a.V - c0);
  EpiCEStats epi{a.labels, a.stats, a.ntn, a.tgt_logit, c0, Vc};
  if (a.ce_bn == 128) return launch_gemm_cfg<256, 128, 2, 2>(chunk_logits_problem(a, c0), epi, s);
  return launch_gemm_cfg<256, CE_BN, 2, 2>(chunk_logits_problem(a, c0), epi, s);
}

hipError_t head_reduce(const HeadArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(ce_reduce_kernel, dim3((a.n + 3) / 4), dim3(256), 0, s, a.stats, a.ntn,
                     a.labels, a.tgt_logit, a.lse, a.loss_row, a.n, a.n_dev);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ce_loss_kernel, dim3(1), dim3(1024), 0, s, a.loss_row, a.n, a.n_dev,
                     a.inv_nvalid, a.loss_out);
  return hipGetLastError();
}

hipError_t head_chunk_grad(const HeadArgs& a, int c0, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const int Vc = min(a.vchunk, a.V - c0), Nc8 = (Vc + 7) / 8 * 8;
  EpiCEGrad epi{a.labels, a.lse, a.inv_nvalid, a.dlog, (long)a.vchunk, c0, Vc, Nc8};
  if (a.ce_bn == 128) return launch_gemm_cfg<256, 128, 2, 2>(chunk_logits_problem(a, c0), epi, s);
  return launch_gemm_cfg<256, CE_BN, 2, 2>(chunk_logits_problem(a, c0), epi, s);
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
  // dH += dlogits[:, chunk] · W[chunk, :]: the head read in place as the
  // [K, N] operand, rows past the vocabulary loading as zeros
  GemmProblem q{a.dlog, (long)a.vchunk, a.W + (long)c0 * a.D, (long)a.D, nullptr, 0, nullptr, 0,
                a.n, a.D, Nc8, 0, a.n_dev};
  q.b_kn = 1;
  q.kb_rows = min(a.vchunk, a.V - c0);
  EpiF32 ef{a.dH, (long)a.D, a.D, c0 > 0 ? 1 : 0};
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
  for (int c0 = 0; c0 < a.V; c0 += a.vchunk)
    if ((e = head_stats(a, c0, s)) != hipSuccess) return e;
  if ((e = head_reduce(a, s)) != hipSuccess) return e;
  for (int c0 = 0; c0 < a.V; c0 += a.vchunk) {
    if ((e = head_chunk_grad(a, c0, s)) != hipSuccess) return e;
    if ((e = head_chunk_dh(a, c0, s)) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace dsb
