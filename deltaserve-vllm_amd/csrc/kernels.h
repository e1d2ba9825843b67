// Internal launch API of the backward's HIP kernels (not part of the C-ABI).
#pragma once

#include "../../include/dsb.h"
#include "dsb_common.h"

namespace dsb {

// ---- norm_rope.hip
hipError_t rmsnorm_fwd(const bf16* x, long ldx, const bf16* w, bf16* y, long ldy, int rows,
                       const int* rows_dev, int D, float eps, hipStream_t s);
// out = bf16(o), o = rmsnorm_backward(x, g, w) + (resid | resid32), and the
// fp32 o into out32 when set (resid and resid32 share the row stride ldr,
// out and out32 the row stride ldo).
hipError_t rmsnorm_bwd(const bf16* x, long ldx, const void* g, bool g_f32, long ldg,
                       const bf16* w, const bf16* resid, long ldr, bf16* out, long ldo,
                       int rows, const int* rows_dev, int D, float eps, hipStream_t s,
                       const float* resid32 = nullptr, float* out32 = nullptr);
hipError_t rope_table(const int* pos, int n, const int* n_dev, const float* inv_freq,
                      int half, float* cosb, float* sinb, hipStream_t s);
// q heads of a row at in / pre (row stride ldin / ldp); k heads at ink / prek
// (stride ldk / ldpk), by default right after the q heads of the same row.
// hd: head_dim, 128 or 64 (cos/sin rows of hd/2).
hipError_t rope_fwd(const bf16* in, long ldin, bf16* out, long ldout, const float* cosb,
                    const float* sinb, int n, const int* n_dev, int Hq, int Hkv, int hd,
                    const bf16* qn_w, const bf16* kn_w, float eps, hipStream_t s,
                    const bf16* ink = nullptr, long ldk = 0);
hipError_t rope_bwd(bf16* g, long ldg, const bf16* pre, long ldp, const float* cosb,
                    const float* sinb, int n, const int* n_dev, int Hq, int Hkv, int hd,
                    const bf16* qn_w, const bf16* kn_w, float eps, hipStream_t s,
                    const bf16* prek = nullptr, long ldpk = 0);
hipError_t swiglu_h(const bf16* gu, long ldgu, bf16* h, long ldh, int n, const int* n_dev,
                    int I, hipStream_t s);

// ---- attention.hip
// Packed varlen causal GQA attention, head_dim 128 or 64. `tiles` holds one int4
// (seq_start, seq_len, tile_start, 0) per 128-token tile of every sequence;
// `ntiles_dev` is the live tile count (grid is sized for `max_tiles`).
struct AttnArgs {
  const bf16* q; long ldq;   // [n, Hq*hd] (post-RoPE)
  const bf16* k; long ldk;   // [n, Hkv*hd] (post-RoPE)
  const bf16* v; long ldv;   // [n, Hkv*hd]
  bf16* ctx; long ldc;       // fwd out [n, Hq*hd]
  float* o32;                // fwd out fp32 copy of ctx, ld = ldo32; null: none
  long ldo32;
  bf16* ores;                // fwd out bf16(O − bf16(O)), the rounding residual of
                             // ctx (ld = ldc); dsum then takes O = ctx + ores.
                             // With neither copy dsum takes O from the bf16 ctx.
  float* lse;                // [Hq, ld_stat] log2-domain row log-sum-exp
  float* dsum;               // [Hq, ld_stat] rowsum(dO ∘ O), written by attn_dsum
  long ld_stat;
  const bf16* dout; long lddo;  // bwd in: grad of ctx
  bf16* dq; long lddq;       // bwd out
  bf16* dk; long lddk;
  bf16* dv; long lddv;
  const int4* tiles;          // {start, L, t0, 0} per 128-row tile, heaviest query tile first
  const int4* tiles_k;        // the same tiles, heaviest key tile first (dK/dV pass)
  const int* ntiles_dev;
  int max_tiles;
  int Hq, Hkv;
  int hd = 128;                          // head_dim: 128 or 64
  float scale = 0.08838834764831845f;    // 1/sqrt(hd)
  const int* n_dev;  // live token count (the dK/dV head-split sum reads it)
  int n;
  // fp32 workspace for the dK/dV pass's head split (null: none), at least
  // (Hq / Hkv) · n · 2 · Hkv·hd floats when the split applies
  float* kv_part = nullptr;
  long kv_part_elems = 0;
};
hipError_t attn_fwd(const AttnArgs& a, hipStream_t s);
hipError_t attn_bwd(const AttnArgs& a, hipStream_t s);  // attn_dsum, dQ, dK/dV in order
// dsum for every live row and q-head; the dQ and dK/dV passes read it
hipError_t attn_dsum(const AttnArgs& a, hipStream_t s);
hipError_t attn_bwd_dkdv(const AttnArgs& a, hipStream_t s);
// q-head slices the dK/dV pass splits into (1: none) when kv_part_elems
// holds the partials; attn_bwd_dkdv takes the split when kv_part is set
int attn_dkdv_head_split(const AttnArgs& a);
hipError_t attn_bwd_dq(const AttnArgs& a, hipStream_t s);

// ---- lora.hip
struct CastJob {
  const float* src;
  bf16* dst;
  int rows, cols;   // source shape
  int ld_src, ld_dst;
  int transpose;    // dst[c, r] = src[r, c]
  float scale;
  float clamp;      // > 0: clamp the scaled value to [-clamp, clamp] before the cast
};
hipError_t lora_cast(const CastJob* jobs_dev, const int2* chunks_dev, int nchunks,
                     hipStream_t s);
// Z[t, j] = sum_k X[t, k] · B[j, k] for t < n, j < R; bf16 out.
struct SkinnyArgs {
  const bf16* X; long ldx;
  const bf16* B; long ldb;
  int R, K;
  bf16* Z; long ldz;
  int n; const int* n_dev;
  // fp32 workspace of part_elems floats for a K split (null: no split)
  float* part = nullptr;
  long part_elems = 0;
};
// K slices for a (1: none): short token ranges whose blocks would leave most
// CUs idle split K when part_elems holds slices · n · R partials; lora_skinny
// takes the split when a.part is set
int lora_skinny_split(const SkinnyArgs& a);
hipError_t lora_skinny(const SkinnyArgs& a, hipStream_t s);
// out[j, c] (or out[c, j] when transposed) = scale · sum_t P[t, j] * X[t, c],
// t < n. Output rows j are split into groups of `rg` written to outs[j / rg].
struct TnArgs {
  const bf16* P; long ldp;
  const bf16* X; long ldx;
  int R, C;
  int n; const int* n_dev;
  float* work;     // [nsplit, C, R]
  int nsplit;
  float* outs[3];
  int rg;
  int transpose_out;
  float scale;
  // rows of each group that are stored (0: rg) and, transposed, the output
  // row pitch: a rank padded to a multiple of 8 stores only the adapter's r
  int rv = 0;
};
hipError_t lora_tn(const TnArgs& a, hipStream_t s);
// Up to kTnBatch TN passes (each its own P, X, R, C, outputs and work region;
// one token-split count) in one launch plus one reduction launch.
constexpr int kTnBatch = 12;
struct TnBatch {
  TnArgs a[kTnBatch];
  int count;
  int b0[kTnBatch + 1];
  long r0[kTnBatch + 1];
};
hipError_t lora_tn_batch(const TnArgs* a, int count, hipStream_t s);
// One pass over G [n, C] for the two rank-r products that read it
// (ops.py:142 grad_Z = gy @ (s·B) and ops.py:144 grad_B = s · gy.t() @ Z):
//   Y[t, j] = bf16(sum_c G[t, c]·W[j, c])          (W = (s·B)ᵀ [R2, C])
//   out[c, j] = scale · sum_t P[t, j]·G[t, c]      (P = Z [n, R1], out = grad_B)
// The same pass serves grad_A = grad_Zᵀ·h with Z = h·Aᵀ (W = A, P = grad_Z,
// out[j, c] when transpose_out = 0).
// R1 = 16·RB1 and R2 = 16·RB2 with RB1, RB2 in {1, 2}; C a multiple of 8.
// work holds ceil(C/512)·n_alloc·R2 + nsplit·C·R1 floats.
struct DualArgs {
  const bf16* X; long ldx;  // G
  const bf16* P; long ldp;  // Z
  const bf16* W; long ldw;  // (s·B)ᵀ
  int R1, R2, C;
  int n; const int* n_dev;
  int n_alloc;              // row stride of the Y partials (n <= n_alloc)
  int nsplit;
  float* work;
  bf16* Y; long ldy;
  float* out; float scale;  // out[c, j] (row pitch rv), or out[j, c] when !transpose_out
  int transpose_out;
  int rv = 0;               // rows j < rv are stored (0: R1)
};
// Up to 3 passes with the same R1, R2, n and nsplit in one launch (plus one
// launch for all their reductions); each a[i].work is its own region.
hipError_t lora_dual(const DualArgs* a, int count, hipStream_t s);
bool lora_dual_supported(int R1, int R2, int C);

// ---- head.hip
struct HeadArgs {
  const bf16* normed; long ldh;   // [n, D]
  const bf16* W;                  // [V, D]
  const int* labels;              // [n] target id or -1
  int n; const int* n_dev;
  int D, V;
  float2* stats;                  // [n_cap, ntn] per vocab tile (max, sum exp)
  int ntn;                        // ceil(V / ce_bn)
  int ce_bn = 256;                // vocab tile width of the CE passes (256 or 128)
  float* tgt_logit;               // [n_cap]
  float* lse;                     // [n_cap] row LSE (natural log), after the last chunk
  float* run_m;                   // [n_cap] running row max across chunks
  float* run_l;                   // [n_cap] running Σ exp(logit − run_m)
  float* alpha;                   // [n_cap] the dH accumulator's factor for the chunk
  float* loss_row;                // [n_cap]
  float* loss_out;                // scalar: sum(loss_row)/n_valid
  const float* inv_nvalid;        // device scalar 1/n_valid (0 when none)
  bf16* dlog; int vchunk;         // [n_cap, vchunk] bf16 probabilities of one vocab
                                  // chunk; vchunk a multiple of 256
  float* dH;                      // [n, D] fp32
  int gemm_cfg;                   // tile of the dH product (-1: by shape)
  float* part = nullptr;          // split-K partials for the dH product (null: no split)
  long part_elems = 0;
  int ncu = 0;                    // compute units (tail split of the dH product; 0: none)
};
// Chunk c0 (a multiple of vchunk): head_prob (logits, tile statistics and
// probabilities), head_rescale (online-softmax reference), head_chunk_dh
// (dH·α + P·W); head_finalize after the last chunk (dH, LSE, loss).
int head_num_chunks(const HeadArgs& a);
hipError_t head_fwd_bwd(const HeadArgs& a, hipStream_t s);
hipError_t head_prob(const HeadArgs& a, int c0, hipStream_t s);
hipError_t head_rescale(const HeadArgs& a, int c0, hipStream_t s);
hipError_t head_chunk_dh(const HeadArgs& a, int c0, hipStream_t s);
hipError_t head_finalize(const HeadArgs& a, hipStream_t s);
// K splits head_chunk_dh uses for chunk c0 (1: none), over the whole product
// or (head_dh_tail) over the tiles of its partly filled last round
int head_dh_split(const HeadArgs& a, int c0);
int head_dh_tail(const HeadArgs& a, int c0, int* tail);

// ---- optim.hip
struct OptTensor {
  float* w;
  float* g;
  float* m;
  float* v;
  int numel;
  int layer;
};
struct OptHyper {
  float lr, beta1, beta2, eps, wd, bc1, bc2, max_norm;
};
hipError_t clip_adamw(const OptTensor* tensors_dev, const int2* chunks_dev, int nchunks,
                      const int2* layer_chunks_dev, int nlayers, float* partial,
                      float* sq_layer, const OptHyper* hyper_dev, int do_clip, hipStream_t s);

// ---- capture.hip (forward-side save into the activation store)
hipError_t save_rows(const void* x, long ldx, const void* r, long ldr, long x_rows, int dtype,
                     const int64_t* src, const int64_t* dst, int count, int width, bf16* buf,
                     long ldbuf, long buf_rows, hipStream_t s);
hipError_t save_ids(const int64_t* ids, long ids_len, const int64_t* src, const int64_t* dst, int count,
                    int64_t* out, long out_len, hipStream_t s);

// ---- misc (dsb_api.hip)
hipError_t build_labels(const int64_t* ids, const int* pred_flag, int* labels, int n,
                        const int* n_dev, int V, int* err, hipStream_t s);

}  // namespace dsb
