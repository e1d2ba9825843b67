/* dsb.h — C-ABI of the MI355X (gfx950) DeltaServe LoRA-SFT backward.
 *
 * One shared library, libdsb.so, loaded by ctypes into the backward child
 * (PyTorch-ROCm owns device memory and the LoRA master tensors). Plain
 * pointers and sizes only; every device pointer is a HIP device address.
 * Every function returns 0 on success and non-zero on failure, with the
 * message available from dsb_last_error().
 *
 * Reference interface replaced (paths relative to the reference checkout):
 *   the cycle  LoraSftTrainerService.process_backward
 *              deltaserve-plugin/deltaserve/bwd_services/common/trainer.py:503-678
 *   its state  LoraSftTrainerService._build_state           trainer.py:112-296
 *   its math   bwd_services/llama3.py:62-219, qwen3.py:68-204,
 *              common/{ops,attention,ffn,head}.py
 */
#ifndef DSB_H_
#define DSB_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSB_ABI_VERSION 5

enum { DSB_FAMILY_LLAMA3 = 0, DSB_FAMILY_QWEN3 = 1 };
enum { DSB_ROPE_DEFAULT = 0, DSB_ROPE_LINEAR = 1, DSB_ROPE_LLAMA3 = 2 };
enum {
  DSB_PROJ_Q = 0, DSB_PROJ_K = 1, DSB_PROJ_V = 2, DSB_PROJ_O = 3,
  DSB_PROJ_GATE = 4, DSB_PROJ_UP = 5, DSB_PROJ_DOWN = 6, DSB_NUM_PROJ = 7
};
/* element types of the capture entry points */
enum { DSB_DT_BF16 = 0, DSB_DT_F16 = 1, DSB_DT_F32 = 2 };
/* dsb_desc.flags */
/* DSB_FLAG_SERIAL_LAYERS: run each layer's recompute right before its
   backward on the cycle's stream, instead of beside the previous layer's
   backward on a second stream (the default for models of more than one layer
   whose s_max · hidden is at most 2^24; results are the same either way). */
enum { DSB_FLAG_GRAPH = 1u, DSB_FLAG_NO_CLIP = 2u, DSB_FLAG_KTIMING = 4u,
       DSB_FLAG_SERIAL_LAYERS = 8u };

typedef struct dsb_handle dsb_handle;

/* Model and trainer constants: the backward `meta` dict of
 * deltaserve-plugin/deltaserve/ft_meta.py:131-213 plus the AdamW settings of
 * trainer.py:252-256. head_dim 128 or 64; lora_rank in [1, 64] (the rank-r
 * kernels run at the rank rounded up to a multiple of 8, on zero-padded bf16
 * copies of A and B, and store the adapter's own r rows of each gradient);
 * hidden <= 8192. */
typedef struct dsb_desc {
  int32_t abi_version;       /* DSB_ABI_VERSION */
  int32_t family;            /* DSB_FAMILY_* (Qwen3 adds per-head q/k RMSNorm) */
  int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab;
  int32_t lora_rank;
  float lora_scaling;        /* alpha / r */
  float rms_eps;
  float rope_theta;
  int32_t rope_type;         /* DSB_ROPE_* (ops.py:26-57) */
  float rope_factor, rope_low_freq_factor, rope_high_freq_factor, rope_orig_max_pos;
  int32_t s_max;             /* token capacity of one cycle (max_saved_finetuning_tokens) */
  int32_t max_seqs;          /* sequence capacity of one cycle (s_max admits any packing) */
  float beta1, beta2, adam_eps, weight_decay, max_grad_norm;
  uint32_t flags;            /* DSB_FLAG_* */
  int32_t vocab_chunk;       /* LM-head vocab columns per chunk and pause point, a multiple
                                of 256 (0: 16384, the reference's VOCAB_CHUNK, head.py:25) */
  int32_t gemm_tile;         /* dense-product tile: 0 by shape, else 256, 128 or 64 */
} dsb_desc;

/* Frozen bf16 base weights of one decoder layer, borrowed (the IPC-shared
 * vLLM tensors of trainer.py:201-218: fused qkv_proj and gate_up_proj). */
typedef struct dsb_layer_weights {
  const void* qkv;      /* [q + 2kv, D] */
  const void* o;        /* [D, q] */
  const void* gate_up;  /* [2I, D] (gate rows first) */
  const void* down;     /* [D, I] */
  const void* in_ln;    /* [D] */
  const void* post_ln;  /* [D] */
  const void* q_norm;   /* [head_dim] (Qwen3) or NULL */
  const void* k_norm;   /* [head_dim] (Qwen3) or NULL */
} dsb_layer_weights;

/* One LoRA projection: fp32 PEFT masters A [r, in], B [out, r] and their
 * gradient buffers (torch-owned; the cycle writes the clipped gradient). */
typedef struct dsb_lora_tensors {
  float* A;
  float* B;
  float* gA;
  float* gB;
} dsb_lora_tensors;

/* The captured-activation store (accumulate.py:236-252): per-layer residual
 * inputs and the pre-final-norm residual, bf16 [s_max + 1, D] rows of stride
 * `ld`, and the token ids int64 [s_max]. Only rows [0, n) are read.
 * mlp_gate_up (NULL when not captured): the optional per-layer gate‖up save
 * point, bf16 [s_max + 1, 2·intermediate] (gate columns first) of row stride
 * ld_gate_up; when bound, the cycle takes gate and up from it instead of
 * recomputing the gate_up product (llama3.py:63-72, ffn.py:18-26). */
typedef struct dsb_activations {
  const void* const* layer_in;  /* n_layers pointers */
  const void* final_in;
  const int64_t* input_ids;
  int64_t ld;
  const void* const* mlp_gate_up;  /* n_layers pointers, or NULL */
  int64_t ld_gate_up;
  /* The optional q/k/v save point (all three or none; accumulate.py:213-226):
   * bf16 [s_max + 1, q | kv | kv] per layer, row strides ld_q / ld_k / ld_v.
   * Llama-3 saves q and k after RoPE, Qwen3 before its q/k-norm
   * (family.py:75-84). When bound, the Q/K/V projection is not recomputed
   * (llama3.py:118-126, qwen3.py:90-96): Llama-3 attends the saved rows
   * directly, Qwen3 re-applies the q/k-norm and RoPE to them. The callers
   * pass them only when the worker's save_attn_qkv is on (trainer.py:539-544). */
  const void* const* attn_q;
  const void* const* attn_k;
  const void* const* attn_v;
  int64_t ld_q, ld_k, ld_v;
  /* The optional attention-context save point, bf16 [s_max + 1, q]: the O
   * projection's input (llama3.py:128-132). The attention forward still
   * runs, since the backward takes its softmax statistics and rowsum(dO∘O)
   * from it. */
  const void* const* attn_ctx;
  int64_t ld_ctx;
  /* The optional post-attention residual save point, bf16 [s_max + 1, D]:
   * used in place of the O projection and the residual add
   * (llama3.py:134-141; passed when save_resid_mid is on, trainer.py:552). */
  const void* const* resid_mid;
  int64_t ld_resid_mid;
} dsb_activations;

/* Per-cycle device timing (ms), filled by dsb_step when requested. */
typedef struct dsb_cycle_info {
  float gpu_ms;
  int32_t graph;       /* 1 if the cycle replayed the captured hipGraph */
  int32_t n_valid;
} dsb_cycle_info;

/* Creates the backward state (replaces _build_state's dims/optimizer part,
 * trainer.py:112-256). */
int dsb_create(const dsb_desc* desc, dsb_handle** out);
void dsb_destroy(dsb_handle* h);
/* Message of the last failure on this thread (h may be NULL). */
const char* dsb_last_error(const dsb_handle* h);

/* Binds layer `layer`'s base weights (trainer.py:201-218). Makes the
 * transposed copies the dX products read, once, after waiting for all work
 * already issued to the device (the weights may still be in flight on the
 * caller's streams). */
int dsb_bind_weights(dsb_handle* h, int layer, const dsb_layer_weights* w);
/* Binds the LM head [vocab, D] and the final RMSNorm weight [D] (trainer.py:194-195);
 * waits for the device like dsb_bind_weights. */
int dsb_bind_head(dsb_handle* h, const void* lm_head, const void* final_norm);
/* Binds one LoRA projection (trainer.py:231-243); proj is DSB_PROJ_*. Any
 * subset of the seven projections may be bound per layer (the reference's
 * ld.get(proj) may be None, trainer.py:457-460); unbound ones stay frozen. */
int dsb_bind_lora(dsb_handle* h, int layer, int proj, const dsb_lora_tensors* t);
/* Binds the shared activation buffers (base.py:438-461 share_activations). */
int dsb_bind_activations(dsb_handle* h, const dsb_activations* a);

/* One backward cycle + AdamW step (+ the served-slot publish when slots are
 * bound, dsb_bind_served): trainer.py:503-678.
 * seq_lens: host int32[nseq] in request order, summing to n <= s_max.
 * lr: this cycle's learning rate; step: the optimizer step count t >= 1.
 * stream: the caller's hipStream_t (work is ordered after it and it waits
 * for the cycle). Writes the mean loss and the number of predicting rows. */
int dsb_step(dsb_handle* h, const int32_t* seq_lens, int nseq, int n, float lr, int64_t step,
             void* stream, float* loss, int* n_valid, dsb_cycle_info* info);

/* The same cycle in segments, for the GPU-yield contract of the reference's
 * BackwardService._maybe_pause (bwd_services/base.py:148-208), which the
 * reference calls once per vocab chunk in both LM-head passes (head.py:78-80,
 * :92-94) and at every layer boundary (llama3.py:342-344). With C =
 * ceil(vocab / vocab_chunk): segments 0 .. C-1 are the head's LSE pass, one
 * vocab chunk each; C .. 2C-1 its gradient pass; 2C .. 2C+L-1 the decoder
 * layers from the last to the first; 2C+L (the last) the clip, AdamW and
 * publish. dsb_step_begin stages the
 * cycle (like dsb_step's first half); dsb_step_segment launches segment `seg`
 * (in order, each its own captured graph) and, when run_ahead > 0, keeps the
 * host at most run_ahead segments ahead of the GPU: the reference's
 * backward_run_ahead_boundaries event ring (base.py:155-183). dsb_step_end
 * waits for the cycle and reports like dsb_step. The caller's pause check
 * runs between dsb_step_segment calls, outside any captured region. Results
 * equal dsb_step's bit for bit (same kernels, same order). */
int dsb_num_segments(const dsb_handle* h);
int dsb_step_begin(dsb_handle* h, const int32_t* seq_lens, int nseq, int n, float lr,
                   int64_t step, void* stream);
int dsb_step_segment(dsb_handle* h, int seg, int run_ahead);
int dsb_step_end(dsb_handle* h, void* stream, float* loss, int* n_valid, dsb_cycle_info* info);

/* Served-slot publish, replacing LoraSftTrainerService._publish_to_served
 * (trainer.py:760-802): binds the bf16 rows of vLLM's stacked LoRA buffers
 * for one projection, a_slot = lora_a_stacked[slot, 0] ([r, in], row stride
 * lda) and b_slot = lora_b_stacked[slot, 0] ([out, r], row stride ldb).
 * Every cycle then ends by writing clamp(A, ±6.5e4) and clamp(s·B, ±6.5e4),
 * cast to bf16, into every bound slot, inside its graph after AdamW. NULL
 * slots unbind. dsb_publish writes them once outside a cycle (the
 * switch_adapter path, trainer.py:721-724). */
int dsb_bind_served(dsb_handle* h, int layer, int proj, void* a_slot, int64_t lda, void* b_slot,
                    int64_t ldb);
int dsb_publish(dsb_handle* h, void* stream);

/* Per-kernel-class timing. While enabled (DSB_FLAG_KTIMING at create, or
 * dsb_set_kernel_timing), each cycle replays the captured kernel sequence
 * eagerly on its stream with a HIP event pair around every kernel, and adds
 * the elapsed time and the launch's algorithmic flops / HBM bytes (evaluated
 * for the cycle's live n and packing) to its class. dsb_kernel_stats returns
 * the number of classes (idx < 0 only counts). No counterpart in the
 * reference (it times whole cycles with CUDA events, base.py:528-534); used
 * by bench.py for per-class rooflines. */
int dsb_set_kernel_timing(dsb_handle* h, int on);
int dsb_kernel_stats(const dsb_handle* h, int idx, char* name, int name_len, int64_t* calls,
                     double* total_ms, double* flops, double* bytes);
int dsb_kernel_stats_reset(dsb_handle* h);

/* Zeroes the AdamW moments and sets the weight decay: the fresh optimizer
 * of LoraSftTrainerService.switch_adapter (trainer.py:725-731). The masters
 * keep their addresses, so a captured graph stays valid. */
int dsb_reset_optimizer(dsb_handle* h, float weight_decay);

/* Integer packing of a cycle, host only (trainer.py:510-518, head.py:63-72):
 * positions[n], pred[n] (1 if row t predicts ids[t+1]), returns n_valid or -1. */
int dsb_pack(const int32_t* seq_lens, int nseq, int n, int32_t* positions, int32_t* pred);

/* RoPE inverse frequencies [head_dim/2] (ops.py:26-57), host only. */
int dsb_rope_inv_freq(int head_dim, float theta, int rope_type, float factor, float low,
                      float high, float orig_max, float* out);

/* ---- the forward-side capture (the serving worker's half of the handoff) ----
 *
 * dsb_capture_index replaces ActivationAccumulator.arm_op_step
 * (accumulate.py:324-343), host only: for a step whose finetuning rows sit at
 * `positions` [num_ft] of the flat batch, fills the fixed-length index pair
 * src/dst [max_saved] (n = min(num_ft, max_saved - offset) rows: src[i] =
 * positions[i], dst[i] = offset + i; the rest src 0, dst max_saved, the
 * scratch row). Returns n, or -1 on bad arguments.
 *
 * dsb_save_rows replaces the save op torch.ops.vllm.dserve_save_rows
 * (ft_save_op.py:72-93): buf[dst[i]] = bf16(x[src[i]] (+ r[src[i]], added in
 * x's dtype)) for i < count, x/r of element type x_dtype (DSB_DT_*), rows of
 * `width` elements; buf is a bf16 store [buf_rows = max_saved + 1, ldbuf].
 * Slots pointing at the scratch row (dst == buf_rows - 1), and slots whose
 * src lies outside x's x_rows rows (where the reference's index_select would
 * raise a device-side assert), are skipped. Only
 * enqueues on `stream` (no host synchronisation), so it can be captured in a
 * graph and replayed with refreshed device indices.
 *
 * dsb_save_ids: the final save point's token ids (accumulate.py:598-622):
 * out[dst[i]] = ids[src[i]] for dst[i] < out_len and src[i] < ids_len;
 * stream-ordered likewise. */
int dsb_capture_index(const int64_t* positions, int num_ft, int offset, int max_saved,
                      int64_t* src, int64_t* dst);
int dsb_save_rows(const void* x, int64_t ldx, const void* r, int64_t ldr, int64_t x_rows,
                  int x_dtype, const int64_t* src, const int64_t* dst, int count, int width,
                  void* buf, int64_t ldbuf, int64_t buf_rows, void* stream);
int dsb_save_ids(const int64_t* ids, int64_t ids_len, const int64_t* src, const int64_t* dst,
                 int count, int64_t* out, int64_t out_len, void* stream);

/* ---- single-op entry points (parity tests; synchronous on `stream`) ---- */

/* C = A·Bᵀ (+ A2·B2ᵀ) [+ R]; out_f32 selects fp32 C (accumulate adds to C).
 * b_kn: B and B2 are stored [K, N] (a weight in its own [out, in] layout read
 * by the backward's C = dY·W; N a multiple of 8) instead of [N, K].
 * cfg: -1 tile by shape, 0/1/2 force 256/128/64-wide tiles, -2 split K over
 * the grid as the cycle does when the problem has too few 256-wide tiles,
 * -3 split K over the tiles of a partly filled last round of the device's
 * compute units, as the cycle does (plain launch when there is no such tail). */
int dsb_op_gemm(const void* A, int64_t lda, const void* B, int64_t ldb, const void* A2,
                int64_t lda2, const void* B2, int64_t ldb2, int M, int N, int K1, int K2,
                void* C, int64_t ldc, int out_f32, int accumulate, const void* R, int64_t ldr,
                int b_kn, int cfg, void* stream);
/* Gate‖up product with the SwiGLU forward in its epilogue (the recompute of
 * ffn.py:25-26, frozen gate_up_proj plus its LoRA term; silu as ffn.py:40-41): GU[m, :] = bf16(A·Bᵀ + A2·B2ᵀ)
 * with B [2I, K1] = gate rows then up rows (GU = [gate | up], ld ldgu), and,
 * when H is non-null, H[m, f] = bf16(silu(gate)·up) of the bf16-rounded
 * halves. I a multiple of 64. */
int dsb_op_gemm_glu(const void* A, int64_t lda, const void* B, int64_t ldb, const void* A2,
                    int64_t lda2, const void* B2, int64_t ldb2, int M, int I, int K1, int K2,
                    void* GU, int64_t ldgu, void* H, int64_t ldh, void* stream);
/* ops.py:84-88 */
int dsb_op_rmsnorm(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int rows,
                   int D, float eps, void* stream);
/* ops.py:91-100, plus the bf16 residual add of llama3.py:205 / ffn.py:47-48. */
int dsb_op_rmsnorm_bwd(const void* x, int64_t ldx, const void* g, int g_f32, int64_t ldg,
                       const void* w, const void* resid, int64_t ldr, void* out, int64_t ldo,
                       int rows, int D, float eps, void* stream);
/* ops.py:60-65 cos/sin table [n, head_dim/2] fp32 from int32 positions. */
int dsb_op_rope_table(const int32_t* pos, int n, const float* inv_freq, int half, float* cos_out,
                      float* sin_out, void* stream);
/* ops.py:68-73 (+ qwen3.py:96-107 when norm weights are given). */
int dsb_op_rope(const void* qkv_pre, int64_t ldin, void* qk_out, int64_t ldout,
                const float* cos_t, const float* sin_t, int n, int Hq, int Hkv, int head_dim,
                const void* q_norm, const void* k_norm, float eps, void* stream);
/* ops.py:76-81 (+ qwen3.py:133-144), in place on g. */
int dsb_op_rope_bwd(void* g, int64_t ldg, const void* qkv_pre, int64_t ldp, const float* cos_t,
                    const float* sin_t, int n, int Hq, int Hkv, int head_dim, const void* q_norm,
                    const void* k_norm, float eps, void* stream);
/* attention.py:20-45; o32 [n, Hq*head_dim] fp32 and lse [Hq, n] (log2 domain)
 * out; head_dim 128 or 64. */
int dsb_op_attn_fwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                    int64_t ldv, void* ctx, int64_t ldc, float* o32, float* lse,
                    const int32_t* seq_lens, int nseq, int Hq, int Hkv, int head_dim,
                    void* stream);
/* attention.py:48-112 given the forward's o32/lse. */
int dsb_op_attn_bwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                    int64_t ldv, const float* o32, const float* lse, const void* dout,
                    int64_t lddo, void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv,
                    int64_t lddv, const int32_t* seq_lens, int nseq, int Hq, int Hkv,
                    int head_dim, void* stream);
/* head.py:42-100 from the normed rows: loss, n_valid and dH [n, D] fp32
 * (grad wrt the normed rows; the final-norm backward is dsb_op_rmsnorm_bwd),
 * streaming the vocabulary in chunks of vocab_chunk columns (a multiple of
 * 256; 0: 16384). */
int dsb_op_head(const void* normed, int64_t ldh, const void* lm_w, const int64_t* ids,
                const int32_t* seq_lens, int nseq, int n, int D, int V, int vocab_chunk,
                float* dH, float* loss, int* n_valid, void* stream);
/* grad_A / grad_B of ops.py:143-144: out = scale · Pᵀ·X over n rows, P bf16
 * [n, R] (rows of out in groups of rg written to outs[j / rg]; transpose_out
 * writes out[c, j]). */
int dsb_op_lora_tn(const void* P, int64_t ldp, const void* X, int64_t ldx, int n, int R, int C,
                   float scale, float* out0, float* out1, float* out2, int rg, int transpose_out,
                   void* stream);
/* Z / grad_Z of ops.py:141-142: Z = bf16(X·Bᵀ), X [n, K], B [R, K]. */
int dsb_op_lora_skinny(const void* X, int64_t ldx, const void* B, int64_t ldb, int n, int R, int K,
                       void* Z, int64_t ldz, void* stream);
/* One pass of dsb_op_lora_dual: grad_Z and grad_B of ops.py:142 and :144
 * from one pass over gy = G [n, C]: gZ = bf16(G·BTᵀ) with BT = (s·B)ᵀ [r, C]
 * (ld ldbt), and gB[c, j] = scale · sum_t G[t, c]·Z[t, j] (fp32 [C, r], or
 * [r, C] when transpose_out = 0; the same pass over xin with BT = A and
 * Z = grad_Z gives ops.py:141 Z and :143 grad_A). C, ldg, ldbt multiples of 8. */
typedef struct dsb_dual_pass {
  const void* G; int64_t ldg;
  const void* Z; int64_t ldz;
  const void* BT; int64_t ldbt;
  int32_t C;
  float scale;
  void* gZ; int64_t ldgz;
  float* gB;
  int32_t transpose_out;
} dsb_dual_pass;
/* 1 to 3 passes of rank r in {16, 32} over n rows in one launch (the cycle
 * batches q, k and v this way). The row count is read from device memory,
 * as in the cycle, and the token-split partials are laid out for n_alloc >= n
 * rows. Allocates its partial-sum workspace. */
int dsb_op_lora_dual(const dsb_dual_pass* passes, int count, int n, int n_alloc, int r,
                     void* stream);
/* dsb_op_lora_dual without any allocation, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops). No
 * counterpart in the reference. The row count n is a launch argument, the
 * partial sums live in a 64 MiB device array of the library (one per GPU,
 * held until the process ends; a request needing more fails with an error),
 * and the call only enqueues on `stream` (no synchronisation). Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU race. */
int dsb_op_lora_dual_noalloc(const dsb_dual_pass* passes, int count, int n, int n_alloc, int r,
                             void* stream);
/* trainer.py:624-636 + :668 on a flat tensor list: per-group clip then AdamW. */
int dsb_op_clip_adamw(float* const* w, float* const* g, float* const* m, float* const* v,
                      const int32_t* numel, const int32_t* group, int ntensors, int ngroups,
                      float lr, float beta1, float beta2, float eps, float wd, int64_t step,
                      float max_norm, int do_clip, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSB_H_ */
