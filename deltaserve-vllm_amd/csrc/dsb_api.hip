// C-ABI of the MI355X LoRA-SFT backward: handle, bindings, the per-cycle
// kernel sequence (captured once as a hipGraph), and single-op entry points.
//
// The cycle follows LoraSftTrainerService.process_backward
// (deltaserve-plugin/deltaserve/bwd_services/common/trainer.py:503-678):
//   head_backward (common/head.py:42-100)
//   for i in reversed(range(L)):  layer_forward (llama3.py:62-146 / qwen3.py:68-130)
//                                 layer_backward (llama3.py:149-219 / qwen3.py:147-204)
//   per-layer clip (trainer.py:624-636), AdamW step (trainer.py:668)
// extended to LoRA on all seven projections (q, k, v, o, gate, up, down).
//
// Everything the kernels need per cycle (n, tile tables, positions, label
// flags, optimizer scalars) lives in one device block refreshed by a single
// host→device copy before the graph launch, so one captured graph serves any
// n <= s_max and any packing.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <array>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/dsb.h"
#include "gemm_nt.h"
#include "kernels.h"

namespace dsb {

static thread_local char g_err[2048];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
const char* get_error() { return g_err; }

// ------------------------------------------------------------ small kernels

// labels[t] = pred[t] ? ids[t + 1] : -1; out-of-range ids raise err bit 1.
__global__ void labels_kernel(const int64_t* __restrict__ ids, const int* __restrict__ pred,
                              int* __restrict__ labels, int n, const int* n_dev, int V,
                              int* err) {
  int N = n;
  if (n_dev) N = min(N, *n_dev);
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  int lab = -1;
  if (pred[t]) {
    const int64_t id = ids[t + 1];
    if (id < 0 || id >= V) {
      atomicOr(err, 1);
    } else {
      lab = (int)id;
    }
  }
  labels[t] = lab;
}

hipError_t build_labels(const int64_t* ids, const int* pred, int* labels, int n,
                        const int* n_dev, int V, int* err, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(labels_kernel, dim3((n + 255) / 256), dim3(256), 0, s, ids, pred, labels, n,
                     n_dev, V, err);
  return hipGetLastError();
}

// ------------------------------------------------------------ host helpers

// Integer packing of a cycle (trainer.py:510-518, head.py:63-72).
static int pack_cycle(const int32_t* seq_lens, int nseq, int n, int32_t* pos, int32_t* pred,
                      std::vector<int4>* tiles) {
  long acc = 0;
  for (int i = 0; i < nseq; ++i) {
    if (seq_lens[i] < 0) return -1;
    acc += seq_lens[i];
  }
  if (acc != n) return -1;
  int st = 0, n_valid = 0;
  for (int i = 0; i < nseq; ++i) {
    const int L = seq_lens[i];
    for (int p = 0; p < L; ++p) {
      if (pos) pos[st + p] = p;
      if (pred) pred[st + p] = (p < L - 1) ? 1 : 0;
    }
    if (L >= 2) n_valid += L - 1;
    if (tiles)
      for (int t0 = 0; t0 < L; t0 += 128) tiles->push_back(int4{st, L, t0, 0});
    st += L;
  }
  return n_valid;
}

// Attention tiles of a cycle: one per 128 tokens of each sequence, so at
// most ceil(n/128) + (sequences - 1) <= ceil(s_max/128) + max_seqs.
static int max_tiles_for(int s_max, int max_seqs) { return (s_max + 127) / 128 + max_seqs; }

// Grid capacity (tiles) of the attention launches of a captured graph: the
// smallest of ceil(s_max/128) + 32·2^b (b = 0, 1, ...) that holds the cycle's
// tiles, capped at the handle's bound. A graph is captured per capacity in
// use, so a packing of many short sequences does not make every cycle launch
// its worst-case grid.
static int tile_capacity(int s_max, int bound, int ntiles) {
  const int base = (s_max + 127) / 128;
  long cap = base + 32;
  while (cap < ntiles && cap < bound) cap = base + 2 * (cap - base);
  return (int)std::min<long>(cap, bound);
}

// Tile dispatch orders, heaviest first so the last blocks of a launch are
// short (blocks start roughly in index order): a query tile t0 of the causal
// pass attends to t0 + 128 keys; a key tile is attended by the L - t0 queries
// at or after it. Any order gives the same results (tiles write disjoint rows).
static void order_tiles(const std::vector<int4>& tiles, std::vector<int4>& by_q,
                        std::vector<int4>& by_k) {
  by_q = tiles;
  by_k = tiles;
  std::stable_sort(by_q.begin(), by_q.end(), [](const int4& a, const int4& b) { return a.z > b.z; });
  std::stable_sort(by_k.begin(), by_k.end(),
                   [](const int4& a, const int4& b) { return a.y - a.z > b.y - b.z; });
}

static void rope_inv_freq_host(int hd, float theta, int type, float factor, float low,
                               float high, float orig, float* out) {
  const int half = hd / 2;
  for (int i = 0; i < half; ++i) {
    const float ex = (float)(2 * i) / (float)hd;
    float inv = 1.0f / powf(theta, ex);
    if (type == DSB_ROPE_LINEAR) {
      inv = inv / factor;
    } else if (type == DSB_ROPE_LLAMA3) {
      const double low_wl = (double)orig / low, high_wl = (double)orig / high;
      const float wl = (float)(2.0 * M_PI) / inv;
      if (wl < high_wl) {
        // keep inv
      } else if (wl > low_wl) {
        inv = inv / factor;
      } else {
        const float smooth = (low != high) ? (orig / wl - low) / (high - low) : 0.f;
        inv = (1.f - smooth) * inv / factor + smooth * inv;
      }
    }
    out[i] = inv;
  }
}

}  // namespace dsb

using namespace dsb;

// ------------------------------------------------------------ the handle

namespace {

struct StepHdr {  // device-resident per-cycle scalars (64 bytes)
  int n;
  int ntiles;
  int n_valid;
  int err;
  float inv_nvalid;
  float loss;
  int pad[2];
  OptHyper hyper;
};
static_assert(sizeof(StepHdr) == 64, "StepHdr layout");

struct KRec {
  int cls;
  double fa, fb, fc, ba, bb, bc;
  hipEvent_t e0, e1;
};
struct KClass {
  std::string name;
  long calls = 0;
  double ms = 0, flops = 0, bytes = 0;
};

struct LayerState {
  dsb_layer_weights w{};
  bool bound = false;
  // LoRA groups: q/k/v share one K-concatenated operand slab, gate/up another;
  // a projection of a group that is not bound has zero slices (frozen).
  dsb_lora_tensors lora[DSB_NUM_PROJ]{};
  bool has[DSB_NUM_PROJ]{};
  bf16 *Aqkv, *B2qkv, *BTq, *BTk, *BTv;
  bf16 *Ao, *Bo, *BTo;
  bf16 *Agu, *B2gu, *BTg, *BTu;
  bf16 *Ad, *Bd, *BTd;
};

}  // namespace

// Every non-null pointer 16-byte aligned (the vectorized kernels' contract).
template <class... P>
bool aligned16(const P*... ps) {
  bool ok = true;
  ((ok = ok && ((reinterpret_cast<uintptr_t>(ps) & 15) == 0)), ...);
  return ok;
}

struct GraphSet {  // the cycle's graphs for one attention grid capacity
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<hipGraph_t> seg_graph;
  std::vector<hipGraphExec_t> seg_exec;
};

struct dsb_handle {
  dsb_desc d{};
  int D, Hq, Hkv, hd, q, kv, W3, I, V, r, L, N, max_tiles, ntn, vchunk, nvc, ce_bn;
  // the adapter's rank (rv) and the rank the kernels run at (r: rv rounded up
  // to a multiple of 8; the padded rows of A and columns of B are zeros in the
  // bf16 operands, so they add nothing, and their gradients are not stored)
  int rv;
  int gemm_cfg = -1;  // forced dense-product tile (GEMM_*), -1 by shape
  int tile_cap = 0;   // attention grid capacity of the current cycle
  float s;
  bool qwen = false;
  hipStream_t hs = nullptr;
  hipEvent_t ev_in = nullptr, ev_out = nullptr, ev_t0 = nullptr, ev_t1 = nullptr;
  // second stream (default priority) for the attention backward's dK/dV pass,
  // forked from and joined back into the cycle's stream by these events
  hipStream_t hs2 = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  // Layer overlap: layer li's recompute writes buffer set li & 1, so the
  // recompute of the layer processed next (li − 1) runs on a third stream
  // beside layer li's backward, forked and joined inside layer li's segment.
  // The side stream's products take their own split-K and skinny-slice
  // scratch (part2, tn_work2). Off under per-kernel timing, with
  // DSB_FLAG_SERIAL_LAYERS, with one layer, or for large cycles (see
  // dsb_create); set 1 then aliases set 0.
  struct RecSet {
    bf16 *xn1, *qkv_pre, *qk, *ctx, *ores, *resid, *xn2, *gu, *hb, *Zqkv_b, *Zo_b, *Zgu_b, *Zd_b;
    float* lse;
  };
  RecSet rset[2] = {};
  bool overlap = false;
  hipStream_t hs3 = nullptr;
  hipEvent_t ev_fork3 = nullptr, ev_join3 = nullptr;
  float *part2 = nullptr, *tn_work2 = nullptr;
  std::vector<LayerState> layers;
  const bf16* lm_w = nullptr;
  const bf16* norm_w = nullptr;
  std::vector<const bf16*> layer_in;
  std::vector<const bf16*> gate_up_in;  // saved gate‖up per layer (empty: recompute)
  long ld_gate_up = 0;
  // the other optional save points per layer (empty: recomputed)
  std::vector<const bf16*> q_in, k_in, v_in, ctx_in, rm_in;
  long ld_q_in = 0, ld_k_in = 0, ld_v_in = 0, ld_ctx_in = 0, ld_rm_in = 0;
  const bf16* final_in = nullptr;
  const int64_t* ids = nullptr;
  long act_ld = 0;
  bool finalized = false;
  std::vector<void*> allocs;
  // workspace
  bf16 *xn1, *qkv_pre, *qk, *ctx, *resid, *xn2, *gu, *hb;
  float *lse, *dsum;
  bf16 *Zqkv_b, *Zo_b, *Zgu_b, *Zd_b;
  bf16 *gZd_b, *gZgu_b, *gZo_b, *gZqkv_b;
  bf16 *g0, *g1, *Ggu, *grm, *gctx, *gqkv;
  // the FFN / attention input gradients, fp32 GEMM outputs: each layer's
  // increment of the fp32 residual-stream gradient keeps its accumulator
  // precision into the RMSNorm backward (bf16 here cost 0.5 % per layer of
  // LoRA-gradient error at 32 layers)
  float *gxn2, *gxn1;
  // the residual-stream gradient in fp32 (g32[2] alternate by layer like g0 /
  // g1, which hold its bf16 copies for the MFMA and LoRA operands; grm32 the
  // post-attention residual's): rounding it to bf16 at every layer would
  // compound over the layers
  float *g32[2], *grm32;
  bf16* ores;  // bf16 rounding residual of the attention output: rowsum(dO∘O) from ctx + ores
  bf16 *normed, *dlog;
  float2* stats;
  float *tgt_logit, *lse_h, *loss_row, *dH, *run_m, *run_l, *alpha;
  float* tn_work;
  long tn_work_elems;
  float* part = nullptr;  // split-K partials of the products with too few 256×256 tiles
  long part_elems = 0;
  int ncu = 0;  // compute units of the device (wave-quantisation tails)
  std::vector<TnArgs> tn_pending;  // TN passes of the current layer (see tn_flush)
  float *cosb, *sinb, *inv_freq;
  int* labels;
  // step staging
  void* h_stage = nullptr;  // pinned
  void* d_stage = nullptr;
  size_t stage_bytes = 0;
  StepHdr* d_hdr = nullptr;
  int* d_pos = nullptr;
  int* d_pred = nullptr;
  int4* d_tiles = nullptr;
  int4* d_tiles_k = nullptr;
  // optimizer
  CastJob* d_jobs = nullptr;
  int2* d_cast_chunks = nullptr;
  int ncast_chunks = 0;
  OptTensor* d_opt = nullptr;
  int2* d_opt_chunks = nullptr;
  int nopt_chunks = 0;
  int nopt_tensors = 0;
  int2* d_layer_chunks = nullptr;
  float *d_opt_partial = nullptr, *d_sq = nullptr;
  long cast_elems = 0;
  long opt_elems = 0;
  // per-kernel-class timing (DSB_FLAG_KTIMING)
  bool ktiming = false;
  std::vector<KRec> krec;
  size_t kpos = 0, kcount = 0;
  std::vector<KClass> kcls;
  // publish into the served LoRA slots (trainer.py:760-802)
  struct Served {
    void* a = nullptr;
    long lda = 0;
    void* b = nullptr;
    long ldb = 0;
  };
  std::vector<std::array<Served, DSB_NUM_PROJ>> served;
  CastJob* d_pub_jobs = nullptr;
  int2* d_pub_chunks = nullptr;
  int npub_chunks = 0;
  long pub_elems = 0;
  // graphs, one set per attention grid capacity; the pause-point path
  // captures one graph per segment
  std::vector<std::pair<int, GraphSet>> graphs;
  bool graph_failed = false;
  std::vector<hipEvent_t> ring;  // run-ahead event ring of the pause-point path
  bool in_step = false;
  bool seg_graphed = false;  // the last segment launched replayed its graph
  int seg_next = 0;
  int step_nseq = 0;
  std::vector<int32_t> step_lens;
  std::mutex mu;
  std::string err;
};

namespace {

int fail(dsb_handle* h, const char* msg) {
  set_error("%s", msg);
  if (h) h->err = get_error();
  return -1;
}

template <class T>
int dalloc(dsb_handle* h, T** p, size_t count) {
  void* v = nullptr;
  const size_t bytes = count * sizeof(T) + 256;
  hipError_t e = hipMalloc(&v, bytes);
  if (e != hipSuccess) {
    set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    h->err = get_error();
    return -1;
  }
  h->allocs.push_back(v);
  *p = reinterpret_cast<T*>(v);
  return 0;
}

#define CK(expr)                                                                     \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess) {                                                          \
      set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, __LINE__); \
      h->err = get_error();                                                          \
      return -1;                                                                     \
    }                                                                                \
  } while (0)

#define CKR(expr)            \
  do {                       \
    if ((expr) != 0) return -1; \
  } while (0)

template <class T>
int dalloc_zero(dsb_handle* h, T** p, size_t count) {
  if (dalloc(h, p, count)) return -1;
  CK(hipMemset(*p, 0, count * sizeof(T)));
  return 0;
}

bool has_qkv(const LayerState& ls) {
  return ls.has[DSB_PROJ_Q] || ls.has[DSB_PROJ_K] || ls.has[DSB_PROJ_V];
}
bool has_gu(const LayerState& ls) { return ls.has[DSB_PROJ_GATE] || ls.has[DSB_PROJ_UP]; }

// Gradient outputs of projection p of layer i: its torch-owned buffers, or
// null when p is an untrained member of a trained q/k/v or gate/up group.
// Such a member has zero factor slices: its rank-r passes are skipped (its
// grad_Z columns keep the zeros they were allocated with, so the group's dX
// product adds nothing for it), and the grouped grad_A pass, which computes
// all of the group's rows in one tile, stores no result for it.
float* grad_a(dsb_handle*, const LayerState& ls, int p) {
  return ls.has[p] ? ls.lora[p].gA : nullptr;
}
float* grad_b(dsb_handle*, const LayerState& ls, int p) {
  return ls.has[p] ? ls.lora[p].gB : nullptr;
}

int finalize(dsb_handle* h) {
  if (h->finalized) return 0;
  for (int i = 0; i < h->L; ++i)
    if (!h->layers[i].bound) {
      set_error("layer %d weights not bound", i);
      h->err = get_error();
      return -1;
    }
  if (!h->lm_w || !h->norm_w) return fail(h, "LM head / final norm not bound");
  if (!h->final_in || !h->ids || (int)h->layer_in.size() != h->L)
    return fail(h, "activations not bound");
  const int N = h->N, D = h->D, q = h->q, kv = h->kv, W3 = h->W3, I = h->I, r = h->r;
  const int rv = h->rv;
  const long NN = N + 1;
  CKR(dalloc(h, &h->xn1, NN * D));
  CKR(dalloc(h, &h->qkv_pre, NN * W3));
  CKR(dalloc(h, &h->qk, NN * (q + kv)));
  CKR(dalloc(h, &h->ctx, NN * q));
  CKR(dalloc(h, &h->lse, (long)h->Hq * NN));
  CKR(dalloc(h, &h->dsum, (long)h->Hq * NN));
  CKR(dalloc(h, &h->resid, NN * D));
  CKR(dalloc(h, &h->xn2, NN * D));
  CKR(dalloc(h, &h->gu, NN * 2 * I));
  CKR(dalloc(h, &h->hb, NN * I));
  CKR(dalloc(h, &h->Zqkv_b, NN * 3 * r));
  CKR(dalloc(h, &h->Zo_b, NN * r));
  CKR(dalloc(h, &h->Zgu_b, NN * 2 * r));
  CKR(dalloc(h, &h->Zd_b, NN * r));
  CKR(dalloc(h, &h->gZd_b, NN * r));
  CKR(dalloc_zero(h, &h->gZgu_b, NN * 2 * r));
  CKR(dalloc(h, &h->gZo_b, NN * r));
  CKR(dalloc_zero(h, &h->gZqkv_b, NN * 3 * r));
  CKR(dalloc(h, &h->g0, NN * D));
  CKR(dalloc(h, &h->g1, NN * D));
  CKR(dalloc(h, &h->Ggu, NN * 2 * I));
  CKR(dalloc(h, &h->grm, NN * D));
  CKR(dalloc(h, &h->gctx, NN * q));
  CKR(dalloc(h, &h->gqkv, NN * W3));
  CKR(dalloc(h, &h->gxn2, NN * D));
  CKR(dalloc(h, &h->gxn1, NN * D));
  CKR(dalloc(h, &h->g32[0], NN * D));
  CKR(dalloc(h, &h->g32[1], NN * D));
  CKR(dalloc(h, &h->grm32, NN * D));
  CKR(dalloc(h, &h->ores, NN * q));
  CKR(dalloc(h, &h->normed, NN * D));
  CKR(dalloc(h, &h->stats, NN * h->ntn));
  CKR(dalloc(h, &h->tgt_logit, NN));
  CKR(dalloc(h, &h->lse_h, NN));
  CKR(dalloc(h, &h->loss_row, NN));
  CKR(dalloc(h, &h->run_m, NN));
  CKR(dalloc(h, &h->run_l, NN));
  CKR(dalloc(h, &h->alpha, NN));
  CKR(dalloc(h, &h->dlog, NN * h->vchunk));
  CKR(dalloc(h, &h->dH, NN * D));
  h->tn_work_elems = 32L << 20;
  CKR(dalloc(h, &h->tn_work, h->tn_work_elems));
  {
    int dev = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&h->ncu, hipDeviceAttributeMultiprocessorCount, dev));
    // split-K partials: the largest ks·M·N over the cycle's bf16/fp32 products
    // that gemm_split_count splits, and the largest ks·tail tile partials of
    // those gemm_tail_split splits. Each product is (output width, base
    // reduction depth, LoRA segment): qkv and o recompute, gh, gxn2, gctx,
    // gxn1, the head's dH. A layer with the projection's LoRA reduces over
    // base + segment, one without over the base alone; both are sized, so the
    // split a product takes at run time always fits.
    const int shapes[][3] = {{W3, D, 3 * r}, {D, q, r},  {I, D, r},         {D, 2 * I, 2 * r},
                             {q, D, r},      {D, W3, 3 * r}, {D, h->vchunk, 0}};
    long need = 0;
    for (const auto& sh : shapes) {
      for (const int K : {sh[1], sh[1] + sh[2]}) {
        const int ks = gemm_split_count(N, sh[0], K);
        if (ks > 1) need = std::max(need, (long)ks * N * sh[0]);
        int tail = 0;
        const int kt = gemm_tail_split(N, sh[0], K, h->ncu, &tail);
        if (ks == 1 && kt > 1) need = std::max(need, (long)kt * tail * 65536);
      }
    }
    h->part_elems = need;
    if (need > 0) CKR(dalloc(h, &h->part, need));
  }
  {
    dsb_handle::RecSet& s0 = h->rset[0];
    s0 = {h->xn1, h->qkv_pre, h->qk, h->ctx, h->ores, h->resid, h->xn2, h->gu, h->hb,
          h->Zqkv_b, h->Zo_b, h->Zgu_b, h->Zd_b, h->lse};
    h->rset[1] = s0;
    if (h->overlap) {
      dsb_handle::RecSet& s1 = h->rset[1];
      CKR(dalloc(h, &s1.xn1, NN * D));
      CKR(dalloc(h, &s1.qkv_pre, NN * W3));
      CKR(dalloc(h, &s1.qk, NN * (q + kv)));
      CKR(dalloc(h, &s1.ctx, NN * q));
      CKR(dalloc(h, &s1.ores, NN * q));
      CKR(dalloc(h, &s1.resid, NN * D));
      CKR(dalloc(h, &s1.xn2, NN * D));
      CKR(dalloc(h, &s1.gu, NN * 2 * I));
      CKR(dalloc(h, &s1.hb, NN * I));
      CKR(dalloc(h, &s1.Zqkv_b, NN * 3 * r));
      CKR(dalloc(h, &s1.Zo_b, NN * r));
      CKR(dalloc(h, &s1.Zgu_b, NN * 2 * r));
      CKR(dalloc(h, &s1.Zd_b, NN * r));
      CKR(dalloc(h, &s1.lse, (long)h->Hq * NN));
      CKR(dalloc(h, &h->tn_work2, h->tn_work_elems));
      if (h->part_elems > 0) CKR(dalloc(h, &h->part2, h->part_elems));
    }
  }
  CKR(dalloc(h, &h->cosb, NN * (h->hd / 2)));
  CKR(dalloc(h, &h->sinb, NN * (h->hd / 2)));
  CKR(dalloc(h, &h->inv_freq, 64));
  CKR(dalloc(h, &h->labels, NN));
  {
    float inv[64] = {};
    rope_inv_freq_host(h->hd, h->d.rope_theta, h->d.rope_type, h->d.rope_factor,
                       h->d.rope_low_freq_factor, h->d.rope_high_freq_factor,
                       h->d.rope_orig_max_pos, inv);
    CK(hipMemcpy(h->inv_freq, inv, sizeof(inv), hipMemcpyHostToDevice));
  }
  // step staging: header | positions | pred | tiles
  const size_t off_pos = 64, off_pred = off_pos + ((size_t)N * 4 + 63) / 64 * 64;
  const size_t off_tiles = off_pred + ((size_t)N * 4 + 63) / 64 * 64;
  h->stage_bytes = off_tiles + 2 * (size_t)h->max_tiles * sizeof(int4);  // query, key orders
  CK(hipHostMalloc(&h->h_stage, h->stage_bytes, hipHostMallocDefault));
  memset(h->h_stage, 0, h->stage_bytes);
  char* ds = nullptr;
  CKR(dalloc(h, &ds, h->stage_bytes));
  h->d_stage = ds;
  h->d_hdr = reinterpret_cast<StepHdr*>(ds);
  h->d_pos = reinterpret_cast<int*>(ds + off_pos);
  h->d_pred = reinterpret_cast<int*>(ds + off_pred);
  h->d_tiles = reinterpret_cast<int4*>(ds + off_tiles);
  h->d_tiles_k = h->d_tiles + h->max_tiles;

  // LoRA bf16 operand copies + cast jobs + optimizer tensor table. Operand
  // slabs start zeroed; only bound projections get cast jobs, so an unbound
  // member of a group keeps zero slices and contributes nothing.
  std::vector<CastJob> jobs;
  std::vector<OptTensor> opt;
  std::vector<int2> layer_chunks;
  std::vector<int2> opt_chunks;
  const float s = h->s;
  auto job = [&](const float* src, int rows, int cols, int lds, bf16* dst, int ldd, int tr,
                 float sc) { jobs.push_back(CastJob{src, dst, rows, cols, lds, ldd, tr, sc, 0.f}); };
  for (int i = 0; i < h->L; ++i) {
    LayerState& ls = h->layers[i];
    if (has_qkv(ls)) {
      CKR(dalloc_zero(h, &ls.Aqkv, 3L * r * D));
      CKR(dalloc_zero(h, &ls.B2qkv, (long)W3 * 3 * r));
      CKR(dalloc_zero(h, &ls.BTq, (long)r * q));
      CKR(dalloc_zero(h, &ls.BTk, (long)r * kv));
      CKR(dalloc_zero(h, &ls.BTv, (long)r * kv));
      const int outs[3] = {q, kv, kv}, rowoff[3] = {0, q, q + kv};
      bf16* bts[3] = {ls.BTq, ls.BTk, ls.BTv};
      for (int p = 0; p < 3; ++p) {
        if (!ls.has[p]) continue;
        const dsb_lora_tensors& t = ls.lora[p];
        job(t.A, rv, D, D, ls.Aqkv + (long)p * r * D, D, 0, 1.f);
        job(t.B, outs[p], rv, rv, ls.B2qkv + (long)rowoff[p] * 3 * r + p * r, 3 * r, 0, s);
        job(t.B, outs[p], rv, rv, bts[p], outs[p], 1, s);
      }
    }
    if (ls.has[DSB_PROJ_O]) {
      CKR(dalloc_zero(h, &ls.Ao, (long)r * q));
      CKR(dalloc_zero(h, &ls.Bo, (long)D * r));
      CKR(dalloc_zero(h, &ls.BTo, (long)r * D));
      const dsb_lora_tensors& t = ls.lora[DSB_PROJ_O];
      job(t.A, rv, q, q, ls.Ao, q, 0, 1.f);
      job(t.B, D, rv, rv, ls.Bo, r, 0, s);
      job(t.B, D, rv, rv, ls.BTo, D, 1, s);
    }
    if (has_gu(ls)) {
      CKR(dalloc_zero(h, &ls.Agu, 2L * r * D));
      CKR(dalloc_zero(h, &ls.B2gu, 2L * I * 2 * r));
      CKR(dalloc_zero(h, &ls.BTg, (long)r * I));
      CKR(dalloc_zero(h, &ls.BTu, (long)r * I));
      if (ls.has[DSB_PROJ_GATE]) {
        const dsb_lora_tensors& tg = ls.lora[DSB_PROJ_GATE];
        job(tg.A, rv, D, D, ls.Agu, D, 0, 1.f);
        job(tg.B, I, rv, rv, ls.B2gu, 2 * r, 0, s);
        job(tg.B, I, rv, rv, ls.BTg, I, 1, s);
      }
      if (ls.has[DSB_PROJ_UP]) {
        const dsb_lora_tensors& tu = ls.lora[DSB_PROJ_UP];
        job(tu.A, rv, D, D, ls.Agu + (long)r * D, D, 0, 1.f);
        job(tu.B, I, rv, rv, ls.B2gu + (long)I * 2 * r + r, 2 * r, 0, s);
        job(tu.B, I, rv, rv, ls.BTu, I, 1, s);
      }
    }
    if (ls.has[DSB_PROJ_DOWN]) {
      CKR(dalloc_zero(h, &ls.Ad, (long)r * I));
      CKR(dalloc_zero(h, &ls.Bd, (long)D * r));
      CKR(dalloc_zero(h, &ls.BTd, (long)r * D));
      const dsb_lora_tensors& t = ls.lora[DSB_PROJ_DOWN];
      job(t.A, rv, I, I, ls.Ad, I, 0, 1.f);
      job(t.B, D, rv, rv, ls.Bd, r, 0, s);
      job(t.B, D, rv, rv, ls.BTd, D, 1, s);
    }
    // optimizer tensors of this layer (A then B per bound projection, q..down)
    const int first_chunk = (int)opt_chunks.size();
    const int ins[7] = {D, D, D, q, D, D, I}, outsz[7] = {q, kv, kv, D, I, I, D};
    for (int p = 0; p < DSB_NUM_PROJ; ++p) {
      if (!ls.has[p]) continue;
      const dsb_lora_tensors& t = ls.lora[p];
      const int na = rv * ins[p], nb = outsz[p] * rv;
      float *mA, *vA, *mB, *vB;
      CKR(dalloc_zero(h, &mA, na));
      CKR(dalloc_zero(h, &vA, na));
      CKR(dalloc_zero(h, &mB, nb));
      CKR(dalloc_zero(h, &vB, nb));
      const int ia = (int)opt.size();
      opt.push_back(OptTensor{t.A, t.gA, mA, vA, na, i});
      opt.push_back(OptTensor{t.B, t.gB, mB, vB, nb, i});
      for (int st = 0; st < na; st += 4096) opt_chunks.push_back(int2{ia, st});
      for (int st = 0; st < nb; st += 4096) opt_chunks.push_back(int2{ia + 1, st});
    }
    layer_chunks.push_back(int2{first_chunk, (int)opt_chunks.size() - first_chunk});
  }
  std::vector<int2> cast_chunks;
  for (int j = 0; j < (int)jobs.size(); ++j) {
    const long tot = (long)jobs[j].rows * jobs[j].cols;
    for (long st = 0; st < tot; st += 1024) cast_chunks.push_back(int2{j, (int)st});
  }
  h->ncast_chunks = (int)cast_chunks.size();
  for (const CastJob& j : jobs) h->cast_elems += (long)j.rows * j.cols;
  for (const OptTensor& t : opt) h->opt_elems += t.numel;
  h->nopt_chunks = (int)opt_chunks.size();
  h->nopt_tensors = (int)opt.size();
  if (!jobs.empty()) {
    CKR(dalloc(h, &h->d_jobs, jobs.size()));
    CK(hipMemcpy(h->d_jobs, jobs.data(), jobs.size() * sizeof(CastJob), hipMemcpyHostToDevice));
    CKR(dalloc(h, &h->d_cast_chunks, cast_chunks.size()));
    CK(hipMemcpy(h->d_cast_chunks, cast_chunks.data(), cast_chunks.size() * sizeof(int2),
                 hipMemcpyHostToDevice));
  }
  if (!opt.empty()) {
    CKR(dalloc(h, &h->d_opt, opt.size()));
    CK(hipMemcpy(h->d_opt, opt.data(), opt.size() * sizeof(OptTensor), hipMemcpyHostToDevice));
    CKR(dalloc(h, &h->d_opt_chunks, opt_chunks.size()));
    CK(hipMemcpy(h->d_opt_chunks, opt_chunks.data(), opt_chunks.size() * sizeof(int2),
                 hipMemcpyHostToDevice));
    CKR(dalloc(h, &h->d_opt_partial, opt_chunks.size()));
  }
  CKR(dalloc(h, &h->d_layer_chunks, layer_chunks.size()));
  CK(hipMemcpy(h->d_layer_chunks, layer_chunks.data(), layer_chunks.size() * sizeof(int2),
               hipMemcpyHostToDevice));
  CKR(dalloc(h, &h->d_sq, h->L));
  CK(hipDeviceSynchronize());
  h->finalized = true;
  return 0;
}

#define LK(expr)                                                                 \
  do {                                                                           \
    hipError_t _e = (expr);                                                      \
    if (_e != hipSuccess) {                                                      \
      set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, __LINE__); \
      h->err = get_error();                                                      \
      return -1;                                                                 \
    }                                                                            \
  } while (0)

// ---- per-kernel-class timing: event pairs recorded on the launch stream
// around each kernel (captured into the graph as event nodes). Each record
// carries its algorithmic work as  a·n + b·S + c  (n = live tokens,
// S = sum_i L_i(L_i + 1)), evaluated with the cycle's actual packing.
int kclass(dsb_handle* h, const std::string& name) {
  for (size_t i = 0; i < h->kcls.size(); ++i)
    if (h->kcls[i].name == name) return (int)i;
  h->kcls.push_back(KClass{name});
  return (int)h->kcls.size() - 1;
}

struct KScope {
  dsb_handle* h;
  hipStream_t s;
  long idx = -1;
  KScope(dsb_handle* h_, hipStream_t s_, const std::string& name, double fa, double fb,
         double fc, double ba, double bb, double bc)
      : h(h_), s(s_) {
    if (!h->ktiming) return;
    if (h->kpos == h->krec.size()) {
      KRec r{};
      if (hipEventCreate(&r.e0) != hipSuccess || hipEventCreate(&r.e1) != hipSuccess) return;
      h->krec.push_back(r);
    }
    idx = (long)h->kpos++;
    KRec& r = h->krec[idx];
    r.cls = kclass(h, name);
    r.fa = fa; r.fb = fb; r.fc = fc; r.ba = ba; r.bb = bb; r.bc = bc;
    (void)hipEventRecord(r.e0, s);
  }
  ~KScope() {
    if (idx >= 0) (void)hipEventRecord(h->krec[idx].e1, s);
  }
};

const char* cfg_name(int cfg) {
  return cfg == GEMM_BIG ? "gemm256" : cfg == GEMM_MID ? "gemm128" : "gemm64";
}

// One NT GEMM launch of the cycle (M = live tokens), timed under
// "<tile>_<epilogue>". Algorithmic flops 2·n·N·(K1+K2); bytes: A, B once,
// C once at `ob` bytes per element, plus `xrow` extra bytes per output row.
template <class Epi>
int gemm(dsb_handle* h, const char* epi, const GemmProblem& p, const Epi& e, hipStream_t st,
         double ob, double xrow) {
  const double K = (double)p.K1 + p.K2;
  if constexpr (std::is_same<Epi, EpiBF16>::value || std::is_same<Epi, EpiSwiGLUBwd>::value ||
                std::is_same<Epi, EpiF32>::value) {
    // too few 256×256 tiles for the chip: split K (unless a tile is forced)
    const int ksplit = h->gemm_cfg >= 0 ? 1 : gemm_split_count(p.M, p.N, p.K1 + p.K2);
    if (ksplit > 1 && (long)ksplit * p.M * p.N <= h->part_elems) {
      const bool t128 = gemm_split_tile(p.M, p.N, p.K1 + p.K2) == 128;
      KScope ks(h, st, std::string(t128 ? "gemm128sk_" : "gemm256sk_") + epi, 2.0 * p.N * K, 0, 0,
                2.0 * K + ob * p.N + xrow, 0, 2.0 * p.N * K);
      GemmProblem q = p;
      q.part = h->part;
      LK(launch_gemm_split(q, e, ksplit, st));
      return 0;
    }
    // a partly filled last round of tiles: split K over the tail tiles
    int tail = 0;
    const int kt = h->gemm_cfg >= 0 || ksplit > 1
                       ? 1
                       : gemm_tail_split(p.M, p.N, p.K1 + p.K2, h->ncu, &tail);
    if (kt > 1 && (long)kt * tail * 65536 <= h->part_elems) {
      KScope ks(h, st, std::string("gemm256t_") + epi, 2.0 * p.N * K, 0, 0,
                2.0 * K + ob * p.N + xrow, 0, 2.0 * p.N * K);
      LK(launch_gemm_tail(p, e, kt, tail, h->part, st));
      return 0;
    }
  }
  const int cfg = h->gemm_cfg >= 0 ? h->gemm_cfg : pick_gemm_cfg(p.M, p.N);
  KScope ks(h, st, std::string(cfg_name(cfg)) + "_" + epi, 2.0 * p.N * K, 0, 0,
            2.0 * K + ob * p.N + xrow, 0, 2.0 * p.N * K);
  LK(launch_gemm(p, e, st, cfg));
  return 0;
}

// Rank-r product keeping tokens: Z = bf16(X·Bᵀ) (B [R, K]).
int skinny(dsb_handle* h, const bf16* X, long ldx, const bf16* B, int R, int K, bf16* Z,
           long ldz, hipStream_t s) {
  SkinnyArgs a{X, ldx, B, (long)K, R, K, Z, ldz, h->N, &h->d_hdr->n};
  // K-split partials (short token ranges) in the TN workspace, which holds
  // nothing between the launches that use it
  a.part = h->tn_work;
  a.part_elems = h->tn_work_elems;
  KScope ks(h, s, "lora_skinny", 2.0 * R * K, 0, 0, 2.0 * K + 2.0 * R, 0, 2.0 * R * K);
  LK(lora_skinny(a, s));
  return 0;
}

// A TN pass (grad_A = grad_Zᵀ·X or grad_B = s·Gᵀ·Z) of the layer being
// processed. Nothing in the layer reads these gradients (the optimizer does,
// after the last layer) and their inputs stay valid until the next layer's
// recompute, so the layer's passes are collected here and issued together
// by tn_flush at the end of the layer: one partial launch and one reduction
// for all of them instead of two launches each.
int tn(dsb_handle* h, const bf16* P, long ldp, const bf16* X, long ldx, int R, int C,
       float* o0, float* o1, float* o2, int rg, int transpose, float scale, hipStream_t) {
  TnArgs a{};
  a.P = P; a.ldp = ldp; a.X = X; a.ldx = ldx; a.R = R; a.C = C;
  a.n = h->N; a.n_dev = &h->d_hdr->n;
  a.outs[0] = o0; a.outs[1] = o1; a.outs[2] = o2;
  a.rg = rg; a.transpose_out = transpose; a.scale = scale;
  a.rv = rg == h->r ? h->rv : 0;  // rank-structured outputs: the adapter's rows
  h->tn_pending.push_back(a);
  return 0;
}

int tn_flush(dsb_handle* h, hipStream_t s) {
  std::vector<TnArgs>& pend = h->tn_pending;
  for (size_t i0 = 0; i0 < pend.size(); i0 += kTnBatch) {
    const int cnt = (int)std::min<size_t>(kTnBatch, pend.size() - i0);
    TnArgs* a = pend.data() + i0;
    long blocks = 0, cols = 0;
    double fa = 0, ba = 0, bc = 0;
    for (int i = 0; i < cnt; ++i) {
      blocks += (long)((a[i].C + 127) / 128) * ((a[i].R + 63) / 64);
      cols += (long)a[i].R * a[i].C;
      fa += 2.0 * a[i].R * a[i].C;
      ba += 2.0 * a[i].C + 2.0 * a[i].R;
      bc += 4.0 * a[i].R * a[i].C;
    }
    // (column block, rank group) blocks × token splits: about one block per
    // CU over the whole batch
    int ns = (int)std::max<long>(1, 256 / std::max<long>(blocks, 1));
    ns = std::min(ns, 32);
    ns = std::min(ns, std::max(1, h->N / 64));
    ns = (int)std::max<long>(1, std::min<long>(ns, h->tn_work_elems / std::max<long>(cols, 1)));
    if ((long)ns * cols > h->tn_work_elems) {
      pend.clear();
      return fail(h, "tn: partial sums exceed the workspace");
    }
    float* w = h->tn_work;
    for (int i = 0; i < cnt; ++i) {
      a[i].nsplit = ns;
      a[i].work = w;
      w += (long)ns * a[i].R * a[i].C;
    }
    KScope ks(h, s, "lora_tn", fa, 0, 0, ba, 0, bc);
    const hipError_t e = lora_tn_batch(a, cnt, s);
    if (e != hipSuccess) {
      pend.clear();
      set_error("lora_tn_batch: %s", hipGetErrorString(e));
      h->err = get_error();
      return -1;
    }
  }
  pend.clear();
  return 0;
}

// One lora_dual pass over X [n, C]: Y = bf16(X·Wᵀ) [n, r] and
// out = scale·Pᵀ·X, as [C, r] (transpose) or [r, C]. For an adapter's output
// gradient G: W = (s·B)ᵀ, P = Z gives grad_Z and grad_B (scale s, [C, r]).
struct DualSpec {
  const bf16* X; long ldx; int C;
  const bf16* P; long ldp;
  const bf16* W;
  bf16* Y; long ldy;
  float* out; float scale; int transpose;
};

// Token splits for passes over the given column counts at rank r in one
// launch, or 0 when the shape is outside what the fused kernel handles (the
// caller then runs lora_skinny and lora_tn).
int dual_splits(const dsb_handle* h, const int* C, int count, int r) {
  int ncb = 0;
  long ywork = 0, cols = 0;
  for (int i = 0; i < count; ++i) {
    if (!lora_dual_supported(r, r, C[i])) return 0;
    ncb += (C[i] + 511) / 512;
    ywork += (long)((C[i] + 511) / 512) * h->N * r;
    cols += C[i];
  }
  int ns = std::max(1, std::min(256 / ncb, h->N / 64));
  while (ns > 1 && ywork + (long)ns * cols * r > h->tn_work_elems) --ns;
  return ywork + (long)ns * cols * r > h->tn_work_elems ? 0 : ns;
}

// The passes of `sp` (count <= 3, rank r each) in one launch. Returns 1 when
// the shapes need the separate kernels.
int dual(dsb_handle* h, const DualSpec* sp, int count, int r, hipStream_t s) {
  int C[3];
  for (int i = 0; i < count; ++i) C[i] = sp[i].C;
  const int ns = dual_splits(h, C, count, r);
  if (ns == 0) return 1;
  DualArgs a[3] = {};
  float* work = h->tn_work;
  double flops_n = 0, bytes_n = 0, bytes_c = 0;
  for (int i = 0; i < count; ++i) {
    DualArgs& x = a[i];
    x.X = sp[i].X; x.ldx = sp[i].ldx; x.P = sp[i].P; x.ldp = sp[i].ldp; x.W = sp[i].W;
    x.ldw = sp[i].C; x.R1 = r; x.R2 = r; x.C = sp[i].C;
    x.n = h->N; x.n_dev = &h->d_hdr->n; x.n_alloc = h->N; x.nsplit = ns;
    x.work = work; x.Y = sp[i].Y; x.ldy = sp[i].ldy; x.out = sp[i].out; x.scale = sp[i].scale;
    x.transpose_out = sp[i].transpose;
    x.rv = h->rv;
    work += (long)((x.C + 511) / 512) * h->N * r + (long)ns * x.C * r;
    flops_n += 4.0 * r * x.C;
    bytes_n += 2.0 * x.C + 4.0 * r;
    bytes_c += 6.0 * r * x.C;
  }
  KScope ks(h, s, "lora_dual", flops_n, 0, 0, bytes_n, 0, bytes_c);
  LK(lora_dual(a, count, s));
  return 0;
}

HeadArgs head_args(dsb_handle* h) {
  HeadArgs ha{};
  ha.normed = h->normed; ha.ldh = h->D; ha.W = h->lm_w;
  ha.labels = h->labels;
  ha.n = h->N; ha.n_dev = &h->d_hdr->n; ha.D = h->D; ha.V = h->V; ha.stats = h->stats;
  ha.ntn = h->ntn; ha.ce_bn = h->ce_bn;
  ha.tgt_logit = h->tgt_logit; ha.lse = h->lse_h; ha.loss_row = h->loss_row;
  ha.run_m = h->run_m; ha.run_l = h->run_l; ha.alpha = h->alpha;
  ha.loss_out = &h->d_hdr->loss; ha.inv_nvalid = &h->d_hdr->inv_nvalid;
  ha.dlog = h->dlog; ha.vchunk = h->vchunk; ha.dH = h->dH; ha.gemm_cfg = h->gemm_cfg;
  ha.part = h->part; ha.part_elems = h->part_elems; ha.ncu = h->ncu;
  return ha;
}

// One segment of the cycle on stream st. With C vocab chunks: segments
// 2c and 2c+1 run the LM head's chunk c — its logits product with the tile
// statistics and probabilities, then the rescale to the row's running
// softmax reference and the dH product (segment 0 first builds the RoPE
// table, the LoRA operand casts, the final norm and the labels; segment 2C-1
// ends with dH, the LSE and the loss and the final-norm backward); then one
// segment per decoder layer, last layer first (forward recompute +
// backward); the last segment runs the per-layer clip, AdamW and the publish
// into the served LoRA slots. The cycle is the segments in order (captured
// as one graph); the pause-point path (reference base.py:148-208,
// _maybe_pause per vocab chunk and per layer) launches them one graph per
// segment.
// One decoder layer of the cycle: its forward recompute (rec) into the
// current buffer set and/or its backward (bwd) from it. lo counts the layers
// processed before this one (the incoming gradient buffers alternate by it).
int enqueue_layer(dsb_handle* h, int li, int lo, hipStream_t st, bool rec, bool bwd) {
  const int N = h->N, D = h->D, q = h->q, kv = h->kv, W3 = h->W3, I = h->I, r = h->r;
  const int* nd = &h->d_hdr->n;
  const float eps = h->d.rms_eps;
  const double Hq = h->Hq;
  {
    if (bwd) h->tn_pending.clear();
    // the incoming gradient alternates between the two g buffers layer by layer
    bf16* g = (lo & 1) ? h->g1 : h->g0;
    bf16* gnext = (lo & 1) ? h->g0 : h->g1;
    const float* g32 = h->g32[lo & 1];
    float* gnext32 = h->g32[(lo & 1) ^ 1];
    AttnArgs at{};
    at.q = h->qk; at.ldq = q + kv;
    at.k = h->qk + q; at.ldk = q + kv;
    at.v = h->qkv_pre + q + kv; at.ldv = W3;
    at.ctx = h->ctx; at.ldc = q; at.ores = h->ores;
    at.lse = h->lse; at.dsum = h->dsum; at.ld_stat = N + 1;
    at.dout = h->gctx; at.lddo = q;
    at.dq = h->gqkv; at.lddq = W3;
    at.dk = h->gqkv + q; at.lddk = W3;
    at.dv = h->gqkv + q + kv; at.lddv = W3;
    at.tiles = h->d_tiles; at.tiles_k = h->d_tiles_k; at.ntiles_dev = &h->d_hdr->ntiles;
    at.max_tiles = h->tile_cap;
    at.Hq = h->Hq; at.Hkv = h->Hkv; at.n_dev = nd; at.n = N;
    at.hd = h->hd; at.scale = 1.f / std::sqrt((float)h->hd);
    // dK/dV head-split partials (short cycles) in the TN workspace, which
    // holds nothing while the attention passes run
    at.kv_part = h->tn_work; at.kv_part_elems = h->tn_work_elems;
    // one causal attention matmul = Hq·Hd·S flops (S = sum L(L+1), unmasked pairs ×2)
    const double au = (double)Hq * h->hd;
    const double arow = 2.0 * (q + 2.0 * kv);
    LayerState& ls = h->layers[li];
    const bf16* x = h->layer_in[li];
    const long ldx = h->act_ld;
    const bool hq = has_qkv(ls), ho = ls.has[DSB_PROJ_O], hg = has_gu(ls),
               hd = ls.has[DSB_PROJ_DOWN];
    // gate‖up: the saved forward activations when the store carries them
    // (ffn.py:18-26, llama3.py:63-72), else recomputed into h->gu
    const bool saved_gu = !h->gate_up_in.empty();
    const bf16* gu = saved_gu ? h->gate_up_in[li] : h->gu;
    const long ldgu = saved_gu ? h->ld_gate_up : 2L * I;
    const bf16* wqkv = (const bf16*)ls.w.qkv;
    const bf16* wo = (const bf16*)ls.w.o;
    const bf16* wgu = (const bf16*)ls.w.gate_up;
    const bf16* qnw = (const bf16*)ls.w.q_norm;
    const bf16* knw = (const bf16*)ls.w.k_norm;
    // The optional save points (trainer.py:532-552). Saved q/k/v: Llama-3's
    // q/k are post-RoPE, attended in place; Qwen3's are pre-norm and go
    // through the q/k-norm + RoPE pass into qk. v is attended in place.
    const bool sqkv = !h->q_in.empty(), sctx = !h->ctx_in.empty(), srm = !h->rm_in.empty();
    if (sqkv) {
      if (!h->qwen) {
        at.q = h->q_in[li]; at.ldq = h->ld_q_in;
        at.k = h->k_in[li]; at.ldk = h->ld_k_in;
      }
      at.v = h->v_in[li]; at.ldv = h->ld_v_in;
    }
    // the O projection's input: the saved context, else the recomputed one
    // (the recomputed ctx and its residual still feed rowsum(dO∘O))
    const bf16* cx = sctx ? h->ctx_in[li] : h->ctx;
    const long ldcx = sctx ? h->ld_ctx_in : (long)q;
    // the post-attention residual: saved, or recomputed by the O projection
    const bf16* rs = srm ? h->rm_in[li] : h->resid;
    const long ldrs = srm ? h->ld_rm_in : (long)D;

    const bool hdual = hd && dual_splits(h, &I, 1, r) > 0;

    // ================= forward recompute (llama3.py:62-146, qwen3.py:68-130)
    if (rec) {
    {
      KScope ks(h, st, "rmsnorm_fwd", 0, 0, 0, 4.0 * D, 0, 2.0 * D);
      LK(rmsnorm_fwd(x, ldx, (const bf16*)ls.w.in_ln, h->xn1, D, N, nd, D, eps, st));
    }
    if (hq) CKR(skinny(h, h->xn1, D, ls.Aqkv, 3 * r, D, h->Zqkv_b, 3 * r, st));
    if (!sqkv) {
      GemmProblem p{h->xn1, (long)D, wqkv, (long)D, hq ? h->Zqkv_b : nullptr, 3L * r,
                    hq ? ls.B2qkv : nullptr, 3L * r, N, W3, D, hq ? 3 * r : 0, nd};
      EpiBF16 e{h->qkv_pre, (long)W3, W3, nullptr, 0};
      CKR(gemm(h, "bf16", p, e, st, 2.0, 0.0));
    }
    if (!sqkv || h->qwen) {
      KScope ks(h, st, "rope_fwd", 0, 0, 0, 2.0 * (q + kv) * 2 + 512.0, 0, 0);
      if (sqkv)
        LK(rope_fwd(h->q_in[li], h->ld_q_in, h->qk, q + kv, h->cosb, h->sinb, N, nd, h->Hq,
                    h->Hkv, h->hd, qnw, knw, eps, st, h->k_in[li], h->ld_k_in));
      else
        LK(rope_fwd(h->qkv_pre, W3, h->qk, q + kv, h->cosb, h->sinb, N, nd, h->Hq, h->Hkv,
                    h->hd, h->qwen ? qnw : nullptr, h->qwen ? knw : nullptr, eps, st));
    }
    {
      KScope ks(h, st, "attn_fwd", 0, 2.0 * au, 0, arow + 4.0 * q + 4.0 * Hq, 0, 0);
      LK(attn_fwd(at, st));
    }
    if (ho) CKR(skinny(h, cx, ldcx, ls.Ao, r, q, h->Zo_b, r, st));
    if (!srm) {
      GemmProblem p{cx, ldcx, wo, (long)q, ho ? h->Zo_b : nullptr, (long)r,
                    ho ? ls.Bo : nullptr, (long)r, N, D, q, ho ? r : 0, nd};
      EpiBF16 e{h->resid, (long)D, D, x, ldx};
      CKR(gemm(h, "bf16", p, e, st, 2.0, 2.0 * D));
    }
    {
      KScope ks(h, st, "rmsnorm_fwd", 0, 0, 0, 4.0 * D, 0, 2.0 * D);
      LK(rmsnorm_fwd(rs, ldrs, (const bf16*)ls.w.post_ln, h->xn2, D, N, nd, D, eps, st));
    }
    if (hg) CKR(skinny(h, h->xn2, D, ls.Agu, 2 * r, D, h->Zgu_b, 2 * r, st));
    if (saved_gu) {
      if (hd) {
        KScope ks(h, st, "swiglu_h", 0, 0, 0, 6.0 * I, 0, 0);
        LK(swiglu_h(gu, ldgu, h->hb, I, N, nd, I, st));
      }
    } else {
      // gate‖up (ffn.py:25-26) with h = silu(gate)·up in the epilogue; h is the
      // down projection's input and only feeds its LoRA terms. The fused form
      // needs I to be a multiple of 64 (whole 32-column fragments per half).
      GemmProblem p{h->xn2, (long)D, wgu, (long)D, hg ? h->Zgu_b : nullptr, 2L * r,
                    hg ? ls.B2gu : nullptr, 2L * r, N, 2 * I, D, hg ? 2 * r : 0, nd};
      if (I % 64 == 0) {
        p.glu_half = I;
        EpiGLU e{h->gu, 2L * I, hd ? h->hb : nullptr, (long)I, I};
        CKR(gemm(h, "glu", p, e, st, 2.0, hd ? 2.0 * I : 0.0));
      } else {
        EpiBF16 e{h->gu, 2L * I, 2 * I, nullptr, 0};
        CKR(gemm(h, "bf16", p, e, st, 2.0, 0.0));
        if (hd) {
          KScope ks(h, st, "swiglu_h", 0, 0, 0, 6.0 * I, 0, 0);
          LK(swiglu_h(h->gu, 2L * I, h->hb, I, N, nd, I, st));
        }
      }
    }
    // Z_d = h·A_dᵀ feeds only grad_B of down (the down product itself is not
    // recomputed): when the fused kernel fits, it is computed in the backward
    // together with grad_A_d from one pass over h
    if (hd && !hdual) CKR(skinny(h, h->hb, I, ls.Ad, r, I, h->Zd_b, r, st));
    }  // rec
    if (!bwd) return 0;

    // ================= backward (llama3.py:149-219, qwen3.py:147-204, ffn.py:29-48)
    if (hd) CKR(skinny(h, g, D, ls.BTd, r, D, h->gZd_b, r, st));
    {
      // gh = g·W_down (+ gZ_d·A_d), the gradient wrt h = silu(gate)·up; the
      // epilogue turns it into d_gate ‖ d_up (reads gate ‖ up, writes Ggu),
      // so gh itself is never stored
      GemmProblem p{g, (long)D, (const bf16*)ls.w.down, (long)I, hd ? h->gZd_b : nullptr, (long)r,
                    hd ? ls.Ad : nullptr, (long)I, N, I, D, hd ? r : 0, nd};
      p.b_kn = 1;
      EpiSwiGLUBwd e{gu, ldgu, h->Ggu, 2L * I, I};
      CKR(gemm(h, "dswiglu", p, e, st, 8.0, 0.0));
    }
    // gate, up and down adapters all present and the three passes (each over
    // I columns) fit one fused launch: one launch and one reduction for all
    // three instead of three of each (C3: 84 column blocks × 3 token splits)
    bool mlp3 = false;
    if (hd && hdual && ls.has[DSB_PROJ_GATE] && ls.has[DSB_PROJ_UP]) {
      const int C3c[3] = {I, I, I};
      mlp3 = dual_splits(h, C3c, 3, r) > 0;
    }
    if (mlp3) {
      const DualSpec d[3] = {
          {h->hb, I, I, h->gZd_b, r, ls.Ad, h->Zd_b, r, ls.lora[DSB_PROJ_DOWN].gA, 1.f, 0},
          {h->Ggu, 2L * I, I, h->Zgu_b, 2L * r, ls.BTg, h->gZgu_b, 2L * r,
           grad_b(h, ls, DSB_PROJ_GATE), h->s, 1},
          {h->Ggu + I, 2L * I, I, h->Zgu_b + r, 2L * r, ls.BTu, h->gZgu_b + r, 2L * r,
           grad_b(h, ls, DSB_PROJ_UP), h->s, 1}};
      const int rc = dual(h, d, 3, r, st);
      if (rc != 0) return -1;
    }
    if (hd) {
      const dsb_lora_tensors& t = ls.lora[DSB_PROJ_DOWN];
      if (mlp3) {
        // Z_d and grad_A_d came from the three-pass launch above
      } else if (hdual) {
        // Z_d = bf16(h·A_dᵀ) and grad_A_d = grad_Z_dᵀ·h [r, I] in one pass over h
        const DualSpec d{h->hb, I, I, h->gZd_b, r, ls.Ad, h->Zd_b, r, t.gA, 1.f, 0};
        const int rc = dual(h, &d, 1, r, st);
        if (rc != 0) return -1;
      } else {
        CKR(tn(h, h->gZd_b, r, h->hb, I, r, I, t.gA, nullptr, nullptr, r, 0, 1.f, st));
      }
      CKR(tn(h, h->Zd_b, r, g, D, r, D, t.gB, nullptr, nullptr, r, 1, h->s, st));
    }
    // 1: the member's grad_Z / grad_B still need the separate kernels
    int rest_g = 0, rest_u = 0;
    if (hg && !mlp3) {
      const bool tg = ls.has[DSB_PROJ_GATE], tu = ls.has[DSB_PROJ_UP];
      const DualSpec d[2] = {
          {h->Ggu, 2L * I, I, h->Zgu_b, 2L * r, ls.BTg, h->gZgu_b, 2L * r,
           grad_b(h, ls, DSB_PROJ_GATE), h->s, 1},
          {h->Ggu + I, 2L * I, I, h->Zgu_b + r, 2L * r, ls.BTu, h->gZgu_b + r, 2L * r,
           grad_b(h, ls, DSB_PROJ_UP), h->s, 1}};
      // Two launches when each fills more of the CUs than one launch of
      // both would (C3: one pass gives 28 column blocks × 9 token splits,
      // both together 56 × 4); one launch when the token count caps the
      // splits anyway (256-token cycles: 34 × 4 per pass, 68 × 3 together)
      const int Cg[2] = {I, I};
      const int ns1 = dual_splits(h, Cg, 1, r), ns2 = dual_splits(h, Cg, 2, r);
      if (tg && tu && ns1 > 0 && ns2 > 0 && 2 * ns2 >= ns1) {
        rest_g = rest_u = dual(h, d, 2, r, st);
      } else {
        if (tg) rest_g = dual(h, &d[0], 1, r, st);
        if (tu) rest_u = dual(h, &d[1], 1, r, st);
      }
      if (rest_g < 0 || rest_u < 0) return -1;
      if (rest_g) CKR(skinny(h, h->Ggu, 2L * I, ls.BTg, r, I, h->gZgu_b, 2 * r, st));
      if (rest_u) CKR(skinny(h, h->Ggu + I, 2L * I, ls.BTu, r, I, h->gZgu_b + r, 2 * r, st));
    }
    {
      GemmProblem p{h->Ggu, 2L * I, wgu, (long)D, hg ? h->gZgu_b : nullptr, 2L * r,
                    hg ? ls.Agu : nullptr, (long)D, N, D, 2 * I, hg ? 2 * r : 0, nd};
      p.b_kn = 1;
      EpiF32 e{h->gxn2, (long)D, D, 0};
      CKR(gemm(h, "dx32", p, e, st, 4.0, 0.0));
    }
    if (hg) {
      float* gAg = grad_a(h, ls, DSB_PROJ_GATE);
      float* gAu = grad_a(h, ls, DSB_PROJ_UP);
      CKR(tn(h, h->gZgu_b, 2 * r, h->xn2, D, 2 * r, D, gAg, gAu, nullptr, r, 0, 1.f, st));
      if (rest_g)
        CKR(tn(h, h->Zgu_b, 2 * r, h->Ggu, 2L * I, r, I, grad_b(h, ls, DSB_PROJ_GATE), nullptr,
               nullptr, r, 1, h->s, st));
      if (rest_u)
        CKR(tn(h, h->Zgu_b + r, 2 * r, h->Ggu + I, 2L * I, r, I, grad_b(h, ls, DSB_PROJ_UP),
               nullptr, nullptr, r, 1, h->s, st));
    }
    {
      KScope ks(h, st, "rmsnorm_bwd", 0, 0, 0, 18.0 * D, 0, 2.0 * D);
      LK(rmsnorm_bwd(rs, ldrs, h->gxn2, true, D, (const bf16*)ls.w.post_ln, nullptr, D,
                     h->grm, D, N, nd, D, eps, st, g32, h->grm32));
    }
    int dual_o = 1;
    if (ho) {
      const DualSpec d{h->grm, D, D, h->Zo_b, r, ls.BTo, h->gZo_b, r, ls.lora[DSB_PROJ_O].gB,
                       h->s, 1};
      dual_o = dual(h, &d, 1, r, st);
      if (dual_o < 0) return -1;
      if (dual_o) CKR(skinny(h, h->grm, D, ls.BTo, r, D, h->gZo_b, r, st));
    }
    {
      GemmProblem p{h->grm, (long)D, wo, (long)q, ho ? h->gZo_b : nullptr, (long)r,
                    ho ? ls.Ao : nullptr, (long)q, N, q, D, ho ? r : 0, nd};
      p.b_kn = 1;
      EpiBF16 e{h->gctx, (long)q, q, nullptr, 0};
      CKR(gemm(h, "bf16", p, e, st, 2.0, 0.0));
    }
    if (ho) {
      const dsb_lora_tensors& t = ls.lora[DSB_PROJ_O];
      CKR(tn(h, h->gZo_b, r, cx, ldcx, r, q, t.gA, nullptr, nullptr, r, 0, 1.f, st));
      if (dual_o) CKR(tn(h, h->Zo_b, r, h->grm, D, r, D, t.gB, nullptr, nullptr, r, 1, h->s, st));
    }
    {
      // dsum = rowsum(dO∘O) (reads dO, ctx and its residual) for both passes
      KScope ks(h, st, "attn_dsum", 0, 0, 0, 6.0 * q + 4.0 * Hq, 0, 0);
      LK(attn_dsum(at, st));
    }
    {
      // The dQ and dK/dV passes share only inputs: dK/dV runs on the second
      // stream, concurrently with dQ, so each pass's blocks fill the CUs the
      // other leaves idle (short sequences leave both latency-bound). Under
      // per-kernel timing they run in order, each timed alone.
      const bool fork = !h->ktiming;
      hipStream_t sk = fork ? h->hs2 : st;
      if (fork) {
        CK(hipEventRecord(h->ev_fork, st));
        CK(hipStreamWaitEvent(h->hs2, h->ev_fork, 0));
      }
      {
        KScope ks(h, sk, "attn_dkdv", 0, 4.0 * au, 0, arow + 2.0 * q + 4.0 * kv, 0, 0);
        LK(attn_bwd_dkdv(at, sk));
      }
      {
        KScope ks(h, st, "attn_dq", 0, au, 0, arow + 2.0 * q + 2.0 * q + 8.0 * Hq, 0, 0);
        LK(attn_bwd_dq(at, st));
      }
      if (fork) {
        CK(hipEventRecord(h->ev_join, h->hs2));
        CK(hipStreamWaitEvent(st, h->ev_join, 0));
      }
    }
    {
      KScope ks(h, st, "rope_bwd", 0, 0, 0, 4.0 * (q + kv) + 512.0, 0, 0);
      // the q/k-norm backward (Qwen3) reads the pre-norm q/k: saved or recomputed
      if (sqkv && h->qwen)
        LK(rope_bwd(h->gqkv, W3, h->q_in[li], h->ld_q_in, h->cosb, h->sinb, N, nd, h->Hq,
                    h->Hkv, h->hd, qnw, knw, eps, st, h->k_in[li], h->ld_k_in));
      else
        LK(rope_bwd(h->gqkv, W3, h->qkv_pre, W3, h->cosb, h->sinb, N, nd, h->Hq, h->Hkv,
                    h->hd, h->qwen ? qnw : nullptr, h->qwen ? knw : nullptr, eps, st));
    }
    int rest_qkv[3] = {0, 0, 0};
    if (hq) {
      const DualSpec all[3] = {
          {h->gqkv, W3, q, h->Zqkv_b, 3L * r, ls.BTq, h->gZqkv_b, 3L * r,
           grad_b(h, ls, DSB_PROJ_Q), h->s, 1},
          {h->gqkv + q, W3, kv, h->Zqkv_b + r, 3L * r, ls.BTk, h->gZqkv_b + r, 3L * r,
           grad_b(h, ls, DSB_PROJ_K), h->s, 1},
          {h->gqkv + q + kv, W3, kv, h->Zqkv_b + 2 * r, 3L * r, ls.BTv, h->gZqkv_b + 2 * r, 3L * r,
           grad_b(h, ls, DSB_PROJ_V), h->s, 1}};
      // the trained members in one launch
      DualSpec d[3];
      int member[3], cnt = 0;
      for (int p = 0; p < 3; ++p)
        if (ls.has[p]) { d[cnt] = all[p]; member[cnt++] = p; }
      const int rest = dual(h, d, cnt, r, st);
      if (rest < 0) return -1;
      for (int i = 0; i < cnt; ++i) rest_qkv[member[i]] = rest;
      if (rest_qkv[0]) CKR(skinny(h, h->gqkv, W3, ls.BTq, r, q, h->gZqkv_b, 3 * r, st));
      if (rest_qkv[1]) CKR(skinny(h, h->gqkv + q, W3, ls.BTk, r, kv, h->gZqkv_b + r, 3 * r, st));
      if (rest_qkv[2])
        CKR(skinny(h, h->gqkv + q + kv, W3, ls.BTv, r, kv, h->gZqkv_b + 2 * r, 3 * r, st));
    }
    {
      GemmProblem p{h->gqkv, (long)W3, wqkv, (long)D, hq ? h->gZqkv_b : nullptr, 3L * r,
                    hq ? ls.Aqkv : nullptr, (long)D, N, D, W3, hq ? 3 * r : 0, nd};
      p.b_kn = 1;
      EpiF32 e{h->gxn1, (long)D, D, 0};
      CKR(gemm(h, "dx32", p, e, st, 4.0, 0.0));
    }
    if (hq) {
      CKR(tn(h, h->gZqkv_b, 3 * r, h->xn1, D, 3 * r, D, grad_a(h, ls, DSB_PROJ_Q),
             grad_a(h, ls, DSB_PROJ_K), grad_a(h, ls, DSB_PROJ_V), r, 0, 1.f, st));
      if (rest_qkv[0])
        CKR(tn(h, h->Zqkv_b, 3 * r, h->gqkv, W3, r, q, grad_b(h, ls, DSB_PROJ_Q), nullptr, nullptr,
               r, 1, h->s, st));
      if (rest_qkv[1])
        CKR(tn(h, h->Zqkv_b + r, 3 * r, h->gqkv + q, W3, r, kv, grad_b(h, ls, DSB_PROJ_K), nullptr,
               nullptr, r, 1, h->s, st));
      if (rest_qkv[2])
        CKR(tn(h, h->Zqkv_b + 2 * r, 3 * r, h->gqkv + q + kv, W3, r, kv, grad_b(h, ls, DSB_PROJ_V),
               nullptr, nullptr, r, 1, h->s, st));
    }
    {
      KScope ks(h, st, "rmsnorm_bwd", 0, 0, 0, 18.0 * D, 0, 2.0 * D);
      LK(rmsnorm_bwd(x, ldx, h->gxn1, true, D, (const bf16*)ls.w.in_ln, nullptr, D, gnext, D,
                     N, nd, D, eps, st, h->grm32, gnext32));
    }
    CKR(tn_flush(h, st));
    return 0;
  }
  return 0;
}

void use_set(dsb_handle* h, int k) {
  const dsb_handle::RecSet& s = h->rset[k];
  h->xn1 = s.xn1; h->qkv_pre = s.qkv_pre; h->qk = s.qk; h->ctx = s.ctx; h->ores = s.ores;
  h->resid = s.resid; h->xn2 = s.xn2; h->gu = s.gu; h->hb = s.hb; h->Zqkv_b = s.Zqkv_b;
  h->Zo_b = s.Zo_b; h->Zgu_b = s.Zgu_b; h->Zd_b = s.Zd_b; h->lse = s.lse;
}

// Layer li's recompute on the third stream (into set li & 1, with the side
// scratch), forked from st; the caller joins it back before its segment ends.
int fork_recompute(dsb_handle* h, int li, hipStream_t st) {
  CK(hipEventRecord(h->ev_fork3, st));
  CK(hipStreamWaitEvent(h->hs3, h->ev_fork3, 0));
  use_set(h, li & 1);
  std::swap(h->part, h->part2);
  std::swap(h->tn_work, h->tn_work2);
  const int rc = enqueue_layer(h, li, h->L - 1 - li, h->hs3, true, false);
  std::swap(h->part, h->part2);
  std::swap(h->tn_work, h->tn_work2);
  return rc;
}

int join_recompute(dsb_handle* h, hipStream_t st) {
  CK(hipEventRecord(h->ev_join3, h->hs3));
  CK(hipStreamWaitEvent(st, h->ev_join3, 0));
  return 0;
}

int enqueue_segment(dsb_handle* h, int seg, hipStream_t st) {
  const int N = h->N, D = h->D;
  const int* nd = &h->d_hdr->n;
  const float eps = h->d.rms_eps;
  const int C = h->nvc;
  if (seg < 2 * C) {
    // ---- head: loss and grad wrt final_in (head.py:42-100)
    const HeadArgs ha = head_args(h);
    if (seg == 0) {
      h->kpos = 0;  // kernel-timing records restart with every cycle
      {
        KScope ks(h, st, "rope_table", 0, 0, 0, 4.0 + 64 * 8.0, 0, 0);
        LK(rope_table(h->d_pos, N, nd, h->inv_freq, h->hd / 2, h->cosb, h->sinb, st));
      }
      {
        KScope ks(h, st, "lora_cast", 0, 0, 0, 0, 0, (double)h->cast_elems * 6.0);
        LK(lora_cast(h->d_jobs, h->d_cast_chunks, h->ncast_chunks, st));
      }
      // with the layer overlap, the last layer's recompute (which needs the
      // RoPE tables and the bf16 LoRA operands just written) runs beside the
      // rest of this segment: the final norm, the labels and the first
      // vocabulary chunk's logits
      if (h->overlap && !h->ktiming) CKR(fork_recompute(h, h->L - 1, st));
      {
        KScope ks(h, st, "rmsnorm_fwd", 0, 0, 0, 4.0 * D, 0, 2.0 * D);
        LK(rmsnorm_fwd(h->final_in, h->act_ld, h->norm_w, h->normed, D, N, nd, D, eps, st));
      }
      {
        KScope ks(h, st, "labels", 0, 0, 0, 16, 0, 0);
        LK(build_labels(h->ids, h->d_pred, h->labels, N, nd, h->V, &h->d_hdr->err, st));
      }
    }
    const int c = seg / 2;
    const int c0 = c * h->vchunk, Vc = std::min(h->vchunk, h->V - c0);
    if ((seg & 1) == 0) {
      {
        // 2·n·Vc·D of the head's algorithmic 4·M·D·V (the logits product)
        KScope ks(h, st, h->ce_bn == 128 ? "gemm256x128_ce_prob" : "gemm256_ce_prob",
                  2.0 * Vc * D, 0, 0, 2.0 * D + 8.0 * Vc / h->ce_bn, 0,
                  2.0 * Vc * D + 2.0 * Vc);
        LK(head_prob(ha, c0, st));
      }
      {
        // bytes: the tile statistics and running state of every row, and the
        // P pass over every row (4·Vc bytes) in the first chunk; later chunks
        // scale only the rows whose maximum lies in them, which the count
        // leaves out (a lower bound)
        KScope ks(h, st, "ce_rescale", 0, 0, 0, 8.0 * Vc / h->ce_bn + 12 + (c0 == 0 ? 4.0 * Vc : 0.0),
                  0, 0);
        LK(head_rescale(ha, c0, st));
      }
      if (seg == 0 && h->overlap && !h->ktiming) CKR(join_recompute(h, st));
      return 0;
    }
    {
      // the other 2·n·Vc·D: dH = dH·α + P·W_chunk
      const int cfg = h->gemm_cfg >= 0 ? h->gemm_cfg : pick_gemm_cfg(N, D);
      const bool split = head_dh_split(ha, c0) > 1;
      int tail = 0;
      const bool tsplit = head_dh_tail(ha, c0, &tail) > 1;
      KScope ks(h, st,
                std::string(split ? "gemm256sk" : tsplit ? "gemm256t" : cfg_name(cfg)) + "_f32",
                2.0 * Vc * D, 0, 0, 2.0 * Vc + 8.0 * D, 0, 2.0 * Vc * D);
      LK(head_chunk_dh(ha, c0, st));
    }
    if (c == C - 1) {
      {
        KScope ks(h, st, "ce_finalize", 0, 0, 0, 10.0 * D + 24, 0, 0);
        LK(head_finalize(ha, st));
      }
      KScope ks(h, st, "rmsnorm_bwd", 0, 0, 0, 12.0 * D, 0, 2.0 * D);
      LK(rmsnorm_bwd(h->final_in, h->act_ld, h->dH, true, D, h->norm_w, nullptr, 0, h->g0, D,
                     N, nd, D, eps, st, nullptr, h->g32[0]));
    }
    return 0;
  }
  if (seg < 2 * C + h->L) {
    const int lo = seg - 2 * C;  // layers done before this one in the cycle
    const int li = h->L - 1 - lo;
    // with the overlap, this layer's recompute ran in the previous segment
    // (the first layer's beside the head's first chunk)
    const bool ov = h->overlap && !h->ktiming;
    if (!ov) {
      use_set(h, li & 1);
      CKR(enqueue_layer(h, li, lo, st, true, false));
    }
    // the next layer's recompute (into the other set) beside this backward
    const bool fork = ov && li >= 1;
    if (fork) CKR(fork_recompute(h, li - 1, st));
    use_set(h, li & 1);
    CKR(enqueue_layer(h, li, lo, st, false, true));
    if (fork) CKR(join_recompute(h, st));
    return 0;
  }
  // ---- per-layer clip + AdamW (trainer.py:624-636, :668)
  {
    KScope ks(h, st, "clip_adamw", 0, 0, 0, 0, 0, (double)h->opt_elems * 28.0);
    LK(clip_adamw(h->d_opt, h->d_opt_chunks, h->nopt_chunks, h->d_layer_chunks, h->L,
                  h->d_opt_partial, h->d_sq, &h->d_hdr->hyper,
                  (h->d.flags & DSB_FLAG_NO_CLIP) ? 0 : 1, st));
  }
  if (h->npub_chunks > 0) {
    KScope ks(h, st, "lora_publish", 0, 0, 0, 0, 0, (double)h->pub_elems * 6.0);
    LK(lora_cast(h->d_pub_jobs, h->d_pub_chunks, h->npub_chunks, st));
  }
  h->kcount = h->kpos;
  return 0;
}

int num_segments(const dsb_handle* h) { return 2 * h->nvc + h->L + 1; }

// The whole cycle on stream st.
int enqueue(dsb_handle* h, hipStream_t st) {
  for (int sgi = 0; sgi < num_segments(h); ++sgi) CKR(enqueue_segment(h, sgi, st));
  return 0;
}

// Drops every captured graph (pointers baked into them changed).
void drop_graphs(dsb_handle* h) {
  for (auto& kv : h->graphs) {
    GraphSet& g = kv.second;
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
    for (auto& e : g.seg_exec)
      if (e) (void)hipGraphExecDestroy(e);
    for (auto& x : g.seg_graph)
      if (x) (void)hipGraphDestroy(x);
  }
  h->graphs.clear();
}

// The graph set of the current cycle's attention grid capacity.
GraphSet& graph_set(dsb_handle* h) {
  for (auto& kv : h->graphs)
    if (kv.first == h->tile_cap) return kv.second;
  h->graphs.emplace_back(h->tile_cap, GraphSet{});
  return h->graphs.back().second;
}

// Publish jobs (trainer.py:760-802): A -> a_slot[:r, :in] and s·B ->
// b_slot[:out, :r], both clamped to ±6.5e4 and cast to bf16, for every
// projection with a bound served slot. Rebuilt whenever a slot is bound.
int rebuild_publish(dsb_handle* h) {
  const int D = h->D, q = h->q, kv = h->kv, I = h->I, r = h->rv;
  const int ins[7] = {D, D, D, q, D, D, I}, outs[7] = {q, kv, kv, D, I, I, D};
  std::vector<CastJob> jobs;
  for (int i = 0; i < h->L; ++i)
    for (int p = 0; p < DSB_NUM_PROJ; ++p) {
      const auto& sv = h->served[i][p];
      if (!sv.a || !h->layers[i].has[p]) continue;
      const dsb_lora_tensors& t = h->layers[i].lora[p];
      jobs.push_back(CastJob{t.A, (bf16*)sv.a, r, ins[p], ins[p], (int)sv.lda, 0, 1.f, 6.5e4f});
      jobs.push_back(CastJob{t.B, (bf16*)sv.b, outs[p], r, r, (int)sv.ldb, 0, h->s, 6.5e4f});
    }
  std::vector<int2> chunks;
  long elems = 0;
  for (int j = 0; j < (int)jobs.size(); ++j) {
    const long tot = (long)jobs[j].rows * jobs[j].cols;
    elems += tot;
    for (long st = 0; st < tot; st += 1024) chunks.push_back(int2{j, (int)st});
  }
  CK(hipStreamSynchronize(h->hs));
  if (h->d_pub_jobs) CK(hipFree(h->d_pub_jobs));
  if (h->d_pub_chunks) CK(hipFree(h->d_pub_chunks));
  h->d_pub_jobs = nullptr;
  h->d_pub_chunks = nullptr;
  h->npub_chunks = 0;
  h->pub_elems = elems;
  if (!jobs.empty()) {
    CK(hipMalloc(&h->d_pub_jobs, jobs.size() * sizeof(CastJob)));
    CK(hipMemcpy(h->d_pub_jobs, jobs.data(), jobs.size() * sizeof(CastJob), hipMemcpyHostToDevice));
    CK(hipMalloc(&h->d_pub_chunks, chunks.size() * sizeof(int2)));
    CK(hipMemcpy(h->d_pub_chunks, chunks.data(), chunks.size() * sizeof(int2),
                 hipMemcpyHostToDevice));
    h->npub_chunks = (int)chunks.size();
  }
  drop_graphs(h);
  return 0;
}

// Validates and packs a cycle, stages its device block (one H2D copy on the
// library stream, ordered after the caller's stream) and records the start.
int step_prepare(dsb_handle* h, const int32_t* seq_lens, int nseq, int n, float lr, int64_t step,
                 hipStream_t cs) {
  h->err.clear();
  if (n <= 0 || n > h->N) return fail(h, "dsb_step: n must be in [1, s_max]");
  if (nseq <= 0 || nseq > h->d.max_seqs)
    return fail(h, "dsb_step: nseq must be in [1, max_seqs]");
  if (step < 1) return fail(h, "dsb_step: step must be >= 1");
  if (!seq_lens) return fail(h, "dsb_step: null seq_lens");
  if (finalize(h)) return -1;
  const size_t off_pos = 64, off_pred = off_pos + ((size_t)h->N * 4 + 63) / 64 * 64;
  const size_t off_tiles = off_pred + ((size_t)h->N * 4 + 63) / 64 * 64;
  char* hs = (char*)h->h_stage;
  std::vector<int4> tiles;
  const int nv = pack_cycle(seq_lens, nseq, n, (int32_t*)(hs + off_pos), (int32_t*)(hs + off_pred),
                            &tiles);
  if (nv < 0) return fail(h, "dsb_step: seq_lens must be non-negative and sum to n");
  if ((int)tiles.size() > h->max_tiles) return fail(h, "dsb_step: too many attention tiles");
  h->tile_cap = tile_capacity(h->N, h->max_tiles, (int)tiles.size());
  std::vector<int4> by_q, by_k;
  order_tiles(tiles, by_q, by_k);
  memcpy(hs + off_tiles, by_q.data(), by_q.size() * sizeof(int4));
  memcpy(hs + off_tiles + (size_t)h->max_tiles * sizeof(int4), by_k.data(),
         by_k.size() * sizeof(int4));
  StepHdr hdr{};
  hdr.n = n;
  hdr.ntiles = (int)tiles.size();
  hdr.n_valid = nv;
  hdr.inv_nvalid = nv > 0 ? 1.f / (float)nv : 0.f;
  hdr.hyper.lr = lr;
  hdr.hyper.beta1 = h->d.beta1;
  hdr.hyper.beta2 = h->d.beta2;
  hdr.hyper.eps = h->d.adam_eps;
  hdr.hyper.wd = h->d.weight_decay;
  hdr.hyper.bc1 = (float)(1.0 - pow((double)h->d.beta1, (double)step));
  hdr.hyper.bc2 = (float)(1.0 - pow((double)h->d.beta2, (double)step));
  hdr.hyper.max_norm = h->d.max_grad_norm;
  memcpy(hs, &hdr, sizeof(hdr));
  h->step_lens.assign(seq_lens, seq_lens + nseq);
  h->step_nseq = nseq;
  CK(hipEventRecord(h->ev_in, cs));
  CK(hipStreamWaitEvent(h->hs, h->ev_in, 0));
  CK(hipMemcpyAsync(h->d_stage, h->h_stage, h->stage_bytes, hipMemcpyHostToDevice, h->hs));
  CK(hipEventRecord(h->ev_t0, h->hs));
  return 0;
}

// Copies the 64-byte result header back, orders the caller's stream after
// the cycle, waits for it and reports loss / n_valid / timing.
int step_finish(dsb_handle* h, hipStream_t cs, bool used_graph, float* loss, int* n_valid,
                dsb_cycle_info* info) {
  CK(hipEventRecord(h->ev_t1, h->hs));
  CK(hipMemcpyAsync(h->h_stage, h->d_stage, sizeof(StepHdr), hipMemcpyDeviceToHost, h->hs));
  CK(hipEventRecord(h->ev_out, h->hs));
  CK(hipStreamWaitEvent(cs, h->ev_out, 0));
  CK(hipEventSynchronize(h->ev_out));
  StepHdr back;
  memcpy(&back, h->h_stage, sizeof(back));
  if (h->ktiming) {
    double S = 0;
    for (int i = 0; i < h->step_nseq; ++i)
      S += (double)h->step_lens[i] * (h->step_lens[i] + 1);
    const int n = back.n;
    for (size_t i = 0; i < h->kcount && i < h->krec.size(); ++i) {
      const KRec& rr = h->krec[i];
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, rr.e0, rr.e1) != hipSuccess) continue;
      KClass& c = h->kcls[rr.cls];
      c.calls += 1;
      c.ms += ms;
      c.flops += rr.fa * n + rr.fb * S + rr.fc;
      c.bytes += rr.ba * n + rr.bb * S + rr.bc;
    }
  }
  if (back.err & 1) return fail(h, "dsb_step: a target token id is outside [0, vocab)");
  if (loss) *loss = back.loss;
  if (n_valid) *n_valid = back.n_valid;
  if (info) {
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, h->ev_t0, h->ev_t1));
    info->gpu_ms = ms;
    info->graph = used_graph ? 1 : 0;
    info->n_valid = back.n_valid;
  }
  return 0;
}

// Captures the kernel sequence `fn` issues on the library stream into an
// executable graph; returns 0 and sets *out, or marks capture as failed.
template <class F>
int capture(dsb_handle* h, F&& fn, hipGraph_t* g_out, hipGraphExec_t* x_out) {
  hipError_t e = hipStreamBeginCapture(h->hs, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    const int rc = fn();
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(h->hs, &g);
    if (rc != 0) {
      if (g) (void)hipGraphDestroy(g);
      return -1;
    }
    if (e == hipSuccess) {
      e = hipGraphInstantiate(x_out, g, nullptr, nullptr, 0);
      *g_out = g;
    }
  }
  if (e != hipSuccess) {
    h->graph_failed = true;
    (void)hipGetLastError();
    fprintf(stderr, "[dsb] hipGraph capture failed (%s); running the cycle eagerly\n",
            hipGetErrorString(e));
  }
  return 0;
}

}  // namespace

// ------------------------------------------------------------ C-ABI

extern "C" {

const char* dsb_last_error(const dsb_handle* h) {
  if (h && !h->err.empty()) return h->err.c_str();
  return get_error();
}

int dsb_create(const dsb_desc* d, dsb_handle** out) {
  if (!d || !out) return fail(nullptr, "dsb_create: null argument");
  if (d->abi_version != DSB_ABI_VERSION) return fail(nullptr, "dsb_create: ABI version mismatch");
  if (d->head_dim != 128 && d->head_dim != 64)
    return fail(nullptr, "dsb_create: head_dim must be 128 or 64");
  if (d->n_heads <= 0 || d->n_kv_heads <= 0 || d->n_heads % d->n_kv_heads)
    return fail(nullptr, "dsb_create: n_heads must be a positive multiple of n_kv_heads");
  if (d->lora_rank <= 0 || d->lora_rank > 64)
    return fail(nullptr, "dsb_create: lora_rank must be in [1, 64]");
  if (d->hidden % 8 || d->hidden > 8192 || d->intermediate % 8 || d->vocab <= 0)
    return fail(nullptr, "dsb_create: hidden (<= 8192) and intermediate must be multiples of 8, vocab positive");
  if (d->s_max <= 0 || d->max_seqs <= 0 || d->n_layers <= 0)
    return fail(nullptr, "dsb_create: s_max, max_seqs, n_layers must be positive");
  if (d->vocab_chunk < 0 || d->vocab_chunk % 256)
    return fail(nullptr, "dsb_create: vocab_chunk must be 0 or a positive multiple of 256");
  if (d->gemm_tile != 0 && d->gemm_tile != 256 && d->gemm_tile != 128 && d->gemm_tile != 64)
    return fail(nullptr, "dsb_create: gemm_tile must be 0, 256, 128 or 64");
  if (d->family != DSB_FAMILY_LLAMA3 && d->family != DSB_FAMILY_QWEN3)
    return fail(nullptr, "dsb_create: unknown family");
  auto* h = new dsb_handle();
  h->d = *d;
  h->D = d->hidden; h->Hq = d->n_heads; h->Hkv = d->n_kv_heads;
  h->hd = d->head_dim;
  h->q = h->Hq * h->hd; h->kv = h->Hkv * h->hd; h->W3 = h->q + 2 * h->kv;
  h->I = d->intermediate; h->V = d->vocab; h->L = d->n_layers;
  h->rv = d->lora_rank; h->r = (d->lora_rank + 7) / 8 * 8;
  h->N = d->s_max; h->s = d->lora_scaling; h->qwen = d->family == DSB_FAMILY_QWEN3;
  h->max_tiles = max_tiles_for(d->s_max, std::min(d->max_seqs, d->s_max));
  // LM-head vocab chunk: one pause point per chunk in each pass, and the
  // width of the bf16 dlogits tile (16384 columns: 268 MB at 8192 rows)
  h->vchunk = d->vocab_chunk > 0 ? d->vocab_chunk : 16384;
  h->vchunk = (int)std::min<long>(h->vchunk, ((long)h->V + 255) / 256 * 256);
  // CE passes: 128-wide vocab tiles when 256-wide ones would leave a chunk's
  // launch with under 192 tiles (short cycles: 256 tokens give 64), so the
  // launch streams the head's weights over twice the CUs
  h->ce_bn = (long)((h->N + 255) / 256) * (h->vchunk / 256) < 192 ? 128 : 256;
  h->ntn = (h->V + h->ce_bn - 1) / h->ce_bn;
  h->nvc = (h->V + h->vchunk - 1) / h->vchunk;
  h->gemm_cfg = d->gemm_tile == 256 ? GEMM_BIG
              : d->gemm_tile == 128 ? GEMM_MID
              : d->gemm_tile == 64  ? GEMM_SKINNY : -1;
  h->layers.resize(h->L);
  h->ktiming = (d->flags & DSB_FLAG_KTIMING) != 0;
  // Layer overlap pays where the products leave CUs idle: 256-token to
  // 4.7 K-token cycles at 1–5 K hidden (C1, C2, the 256-token Qwen3-14B
  // cycle: 9–24 % shorter) but not at 8192 tokens × 4096 (C3: 0.1–0.3 %
  // longer), whose products fill every CU for several rounds; it is on up to
  // s_max · hidden = 2^24.
  h->overlap = !(d->flags & DSB_FLAG_SERIAL_LAYERS) && h->L > 1 &&
               (long)d->s_max * d->hidden <= (16L << 20);
  hipError_t e = hipStreamCreateWithFlags(&h->hs, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&h->hs2, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&h->hs3, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ev_fork3, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ev_join3, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ev_fork, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ev_join, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ev_in, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&h->ev_out, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreate(&h->ev_t0);
  if (e == hipSuccess) e = hipEventCreate(&h->ev_t1);
  if (e != hipSuccess) {
    set_error("dsb_create: %s", hipGetErrorString(e));
    dsb_destroy(h);
    return -1;
  }
  *out = h;
  return 0;
}

void dsb_destroy(dsb_handle* h) {
  if (!h) return;
  if (h->hs) (void)hipStreamSynchronize(h->hs);
  if (h->hs2) (void)hipStreamSynchronize(h->hs2);
  if (h->hs3) (void)hipStreamSynchronize(h->hs3);
  drop_graphs(h);
  for (hipEvent_t e : h->ring) (void)hipEventDestroy(e);
  if (h->d_pub_jobs) (void)hipFree(h->d_pub_jobs);
  if (h->d_pub_chunks) (void)hipFree(h->d_pub_chunks);
  for (KRec& r : h->krec) {
    (void)hipEventDestroy(r.e0);
    (void)hipEventDestroy(r.e1);
  }
  for (void* p : h->allocs) (void)hipFree(p);
  if (h->h_stage) (void)hipHostFree(h->h_stage);
  if (h->ev_in) (void)hipEventDestroy(h->ev_in);
  if (h->ev_out) (void)hipEventDestroy(h->ev_out);
  if (h->ev_t0) (void)hipEventDestroy(h->ev_t0);
  if (h->ev_t1) (void)hipEventDestroy(h->ev_t1);
  if (h->ev_fork) (void)hipEventDestroy(h->ev_fork);
  if (h->ev_join) (void)hipEventDestroy(h->ev_join);
  if (h->hs2) (void)hipStreamDestroy(h->hs2);
  if (h->ev_fork3) (void)hipEventDestroy(h->ev_fork3);
  if (h->ev_join3) (void)hipEventDestroy(h->ev_join3);
  if (h->hs3) (void)hipStreamDestroy(h->hs3);
  if (h->hs) (void)hipStreamDestroy(h->hs);
  delete h;
}

int dsb_bind_weights(dsb_handle* h, int layer, const dsb_layer_weights* w) {
  if (!h || !w) return fail(h, "dsb_bind_weights: null argument");
  std::lock_guard<std::mutex> lk(h->mu);
  if (layer < 0 || layer >= h->L) return fail(h, "dsb_bind_weights: layer out of range");
  if (h->finalized) return fail(h, "dsb_bind_weights: state already finalized");
  if (!w->qkv || !w->o || !w->gate_up || !w->down || !w->in_ln || !w->post_ln)
    return fail(h, "dsb_bind_weights: missing base weight");
  if (h->qwen && (!w->q_norm || !w->k_norm))
    return fail(h, "dsb_bind_weights: qwen3 needs q_norm and k_norm");
  LayerState& ls = h->layers[layer];
  // The weights are read in place, in their own [out, in] layout, by every
  // product (no copy). They may still be being written by work the caller
  // issued on its own streams (a dtype conversion, an IPC copy): finish all
  // of it before the library's stream reads them.
  CK(hipDeviceSynchronize());
  ls.w = *w;
  ls.bound = true;
  return 0;
}

int dsb_bind_head(dsb_handle* h, const void* lm_head, const void* final_norm) {
  if (!h || !lm_head || !final_norm) return fail(h, "dsb_bind_head: null argument");
  std::lock_guard<std::mutex> lk(h->mu);
  if (h->finalized) return fail(h, "dsb_bind_head: state already finalized");
  CK(hipDeviceSynchronize());  // as in dsb_bind_weights: the head may still be in flight
  h->lm_w = (const bf16*)lm_head;
  h->norm_w = (const bf16*)final_norm;
  return 0;
}

int dsb_bind_lora(dsb_handle* h, int layer, int proj, const dsb_lora_tensors* t) {
  if (!h || !t) return fail(h, "dsb_bind_lora: null argument");
  std::lock_guard<std::mutex> lk(h->mu);
  if (layer < 0 || layer >= h->L || proj < 0 || proj >= DSB_NUM_PROJ)
    return fail(h, "dsb_bind_lora: layer/proj out of range");
  if (h->finalized) return fail(h, "dsb_bind_lora: state already finalized");
  if (!t->A || !t->B || !t->gA || !t->gB) return fail(h, "dsb_bind_lora: null tensor");
  h->layers[layer].lora[proj] = *t;
  h->layers[layer].has[proj] = true;
  return 0;
}

int dsb_bind_activations(dsb_handle* h, const dsb_activations* a) {
  if (!h || !a || !a->layer_in || !a->final_in || !a->input_ids)
    return fail(h, "dsb_bind_activations: null argument");
  std::lock_guard<std::mutex> lk(h->mu);
  if (h->in_step) return fail(h, "dsb_bind_activations: a segmented cycle is in progress");
  if (a->ld < h->D || a->ld % 8) return fail(h, "dsb_bind_activations: bad row stride");
  if (a->mlp_gate_up && (a->ld_gate_up < 2L * h->I || a->ld_gate_up % 8))
    return fail(h, "dsb_bind_activations: mlp_gate_up row stride must be a multiple of 8 and "
                   ">= 2*intermediate");
  std::vector<const bf16*> gu;
  if (a->mlp_gate_up) {
    for (int i = 0; i < h->L; ++i) {
      if (!a->mlp_gate_up[i] || ((uintptr_t)a->mlp_gate_up[i] & 15))
        return fail(h, "dsb_bind_activations: mlp_gate_up pointers must be non-null, 16-byte "
                       "aligned");
      gu.push_back((const bf16*)a->mlp_gate_up[i]);
    }
  }
  // the optional save points: per-layer bf16 rows of at least `width`
  // columns, 16-byte aligned with a stride that is a multiple of 8
  auto saved = [&](const void* const* ptrs, int64_t ld, int width, const char* what,
                   std::vector<const bf16*>& out) -> int {
    out.clear();
    if (!ptrs) return 0;
    if (ld < width || ld % 8) {
      set_error("dsb_bind_activations: %s row stride must be a multiple of 8 and >= %d", what,
                width);
      h->err = get_error();
      return -1;
    }
    for (int i = 0; i < h->L; ++i) {
      if (!ptrs[i] || ((uintptr_t)ptrs[i] & 15)) {
        set_error("dsb_bind_activations: %s pointers must be non-null, 16-byte aligned", what);
        h->err = get_error();
        return -1;
      }
      out.push_back((const bf16*)ptrs[i]);
    }
    return 0;
  };
  if ((a->attn_q != nullptr) != (a->attn_k != nullptr) ||
      (a->attn_q != nullptr) != (a->attn_v != nullptr))
    return fail(h, "dsb_bind_activations: attn_q, attn_k and attn_v are bound together");
  std::vector<const bf16*> qv, kv_, vv, cv, rv;
  CKR(saved(a->attn_q, a->ld_q, h->q, "attn_q", qv));
  CKR(saved(a->attn_k, a->ld_k, h->kv, "attn_k", kv_));
  CKR(saved(a->attn_v, a->ld_v, h->kv, "attn_v", vv));
  CKR(saved(a->attn_ctx, a->ld_ctx, h->q, "attn_ctx", cv));
  CKR(saved(a->resid_mid, a->ld_resid_mid, h->D, "resid_mid", rv));
  h->layer_in.assign(h->L, nullptr);
  for (int i = 0; i < h->L; ++i) {
    if (!a->layer_in[i]) return fail(h, "dsb_bind_activations: null layer_in");
    h->layer_in[i] = (const bf16*)a->layer_in[i];
  }
  h->gate_up_in = gu;
  h->ld_gate_up = a->mlp_gate_up ? (long)a->ld_gate_up : 0;
  h->q_in = qv; h->k_in = kv_; h->v_in = vv; h->ctx_in = cv; h->rm_in = rv;
  h->ld_q_in = a->ld_q; h->ld_k_in = a->ld_k; h->ld_v_in = a->ld_v;
  h->ld_ctx_in = a->ld_ctx; h->ld_rm_in = a->ld_resid_mid;
  h->final_in = (const bf16*)a->final_in;
  h->ids = a->input_ids;
  h->act_ld = a->ld;
  // Rebinding activations after capture changes baked pointers: drop the graphs.
  drop_graphs(h);
  return 0;
}

int dsb_reset_optimizer(dsb_handle* h, float weight_decay) {
  if (!h) return fail(nullptr, "dsb_reset_optimizer: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  h->d.weight_decay = weight_decay;
  if (!h->finalized) return 0;  // moments are created zeroed at finalize
  std::vector<OptTensor> T(h->nopt_tensors);
  if (!T.empty()) {
    CK(hipMemcpy(T.data(), h->d_opt, T.size() * sizeof(OptTensor), hipMemcpyDeviceToHost));
    for (const OptTensor& t : T) {
      CK(hipMemsetAsync(t.m, 0, (size_t)t.numel * 4, h->hs));
      CK(hipMemsetAsync(t.v, 0, (size_t)t.numel * 4, h->hs));
    }
  }
  CK(hipStreamSynchronize(h->hs));
  return 0;
}

int dsb_kernel_stats(const dsb_handle* h, int idx, char* name, int name_len, int64_t* calls,
                     double* total_ms, double* flops, double* bytes) {
  if (!h) return fail(nullptr, "dsb_kernel_stats: null handle");
  const int nc = (int)h->kcls.size();
  if (idx < 0) return nc;
  if (idx >= nc) return fail(nullptr, "dsb_kernel_stats: index out of range");
  const KClass& c = h->kcls[idx];
  if (name && name_len > 0) snprintf(name, name_len, "%s", c.name.c_str());
  if (calls) *calls = c.calls;
  if (total_ms) *total_ms = c.ms;
  if (flops) *flops = c.flops;
  if (bytes) *bytes = c.bytes;
  return nc;
}

int dsb_set_kernel_timing(dsb_handle* h, int on) {
  if (!h) return fail(nullptr, "dsb_set_kernel_timing: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  h->ktiming = on != 0;
  return 0;
}

int dsb_kernel_stats_reset(dsb_handle* h) {
  if (!h) return fail(nullptr, "dsb_kernel_stats_reset: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  for (KClass& c : h->kcls) {
    c.calls = 0;
    c.ms = c.flops = c.bytes = 0;
  }
  return 0;
}

int dsb_pack(const int32_t* seq_lens, int nseq, int n, int32_t* positions, int32_t* pred) {
  if (nseq < 0 || n < 0 || (nseq > 0 && !seq_lens)) return -1;
  return pack_cycle(seq_lens, nseq, n, positions, pred, nullptr);
}

int dsb_rope_inv_freq(int head_dim, float theta, int rope_type, float factor, float low,
                      float high, float orig_max, float* out) {
  if (head_dim <= 0 || head_dim % 2 || !out) return -1;
  rope_inv_freq_host(head_dim, theta, rope_type, factor, low, high, orig_max, out);
  return 0;
}

int dsb_step(dsb_handle* h, const int32_t* seq_lens, int nseq, int n, float lr, int64_t step,
             void* stream, float* loss, int* n_valid, dsb_cycle_info* info) {
  if (!h) return fail(nullptr, "dsb_step: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  if (h->in_step) return fail(h, "dsb_step: a segmented cycle is in progress");
  hipStream_t cs = (hipStream_t)stream;
  CKR(step_prepare(h, seq_lens, nseq, n, lr, step, cs));
  bool used_graph = false;
  // Kernel timing needs an elapsed time per kernel: HIP reports none for
  // event pairs recorded inside a captured graph, so timed cycles replay the
  // same kernel sequence eagerly on the same stream.
  if ((h->d.flags & DSB_FLAG_GRAPH) && !h->graph_failed && !h->ktiming) {
    GraphSet& gs = graph_set(h);
    if (!gs.exec) CKR(capture(h, [&] { return enqueue(h, h->hs); }, &gs.graph, &gs.exec));
    if (gs.exec) {
      CK(hipGraphLaunch(gs.exec, h->hs));
      used_graph = true;
    }
  }
  if (!used_graph && enqueue(h, h->hs)) return -1;
  return step_finish(h, cs, used_graph, loss, n_valid, info);
}

int dsb_num_segments(const dsb_handle* h) {
  if (!h) return fail(nullptr, "dsb_num_segments: null handle");
  return num_segments(h);
}

int dsb_step_begin(dsb_handle* h, const int32_t* seq_lens, int nseq, int n, float lr,
                   int64_t step, void* stream) {
  if (!h) return fail(nullptr, "dsb_step_begin: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  if (h->in_step) return fail(h, "dsb_step_begin: a segmented cycle is already in progress");
  CKR(step_prepare(h, seq_lens, nseq, n, lr, step, (hipStream_t)stream));
  h->in_step = true;
  h->seg_next = 0;
  return 0;
}

int dsb_step_segment(dsb_handle* h, int seg, int run_ahead) {
  if (!h) return fail(nullptr, "dsb_step_segment: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  if (!h->in_step) return fail(h, "dsb_step_segment: no cycle begun (dsb_step_begin)");
  if (seg != h->seg_next) return fail(h, "dsb_step_segment: segments must run in order");
  if (run_ahead < 0 || run_ahead > 64) return fail(h, "dsb_step_segment: run_ahead must be in [0, 64]");
  const int ns = num_segments(h);
  bool launched = false;
  if ((h->d.flags & DSB_FLAG_GRAPH) && !h->graph_failed && !h->ktiming) {
    GraphSet& gs = graph_set(h);
    if ((int)gs.seg_exec.size() != ns) {
      gs.seg_exec.assign(ns, nullptr);
      gs.seg_graph.assign(ns, nullptr);
    }
    if (!gs.seg_exec[seg])
      CKR(capture(h, [&] { return enqueue_segment(h, seg, h->hs); }, &gs.seg_graph[seg],
                  &gs.seg_exec[seg]));
    if (gs.seg_exec[seg]) {
      CK(hipGraphLaunch(gs.seg_exec[seg], h->hs));
      launched = true;
    }
  }
  h->seg_graphed = launched;
  if (!launched && enqueue_segment(h, seg, h->hs)) return -1;
  h->seg_next = seg + 1;
  // Run-ahead bound (base.py:155-183): record this boundary and wait for the
  // one recorded run_ahead boundaries ago, so the host stays at most
  // run_ahead segments ahead of the GPU.
  if (run_ahead > 0) {
    if ((int)h->ring.size() != run_ahead + 1) {
      for (hipEvent_t e : h->ring) (void)hipEventDestroy(e);
      h->ring.assign(run_ahead + 1, nullptr);
      for (auto& e : h->ring) CK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    const int R = run_ahead + 1;
    CK(hipEventRecord(h->ring[seg % R], h->hs));
    if (seg >= run_ahead) CK(hipEventSynchronize(h->ring[(seg - run_ahead) % R]));
  }
  return 0;
}

int dsb_step_end(dsb_handle* h, void* stream, float* loss, int* n_valid, dsb_cycle_info* info) {
  if (!h) return fail(nullptr, "dsb_step_end: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  if (!h->in_step) return fail(h, "dsb_step_end: no cycle begun");
  h->in_step = false;
  if (h->seg_next != num_segments(h))
    return fail(h, "dsb_step_end: not every segment ran; the cycle's results are incomplete");
  return step_finish(h, (hipStream_t)stream, h->seg_graphed, loss, n_valid, info);
}

int dsb_bind_served(dsb_handle* h, int layer, int proj, void* a_slot, int64_t lda, void* b_slot,
                    int64_t ldb) {
  if (!h) return fail(nullptr, "dsb_bind_served: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  if (layer < 0 || layer >= h->L || proj < 0 || proj >= DSB_NUM_PROJ)
    return fail(h, "dsb_bind_served: layer/proj out of range");
  if (h->in_step) return fail(h, "dsb_bind_served: a segmented cycle is in progress");
  if (!h->layers[layer].has[proj]) return fail(h, "dsb_bind_served: projection has no LoRA bound");
  const int D = h->D, q = h->q, r = h->rv, I = h->I;
  const int ins[7] = {D, D, D, q, D, D, I};
  if ((a_slot == nullptr) != (b_slot == nullptr))
    return fail(h, "dsb_bind_served: bind both slots or neither");
  if (a_slot && (lda < ins[proj] || ldb < r))
    return fail(h, "dsb_bind_served: slot row stride smaller than the row");
  if ((int)h->served.size() != h->L) h->served.assign(h->L, {});
  h->served[layer][proj] = dsb_handle::Served{a_slot, (long)lda, b_slot, (long)ldb};
  return rebuild_publish(h);
}

int dsb_publish(dsb_handle* h, void* stream) {
  if (!h) return fail(nullptr, "dsb_publish: null handle");
  std::lock_guard<std::mutex> lk(h->mu);
  if (h->in_step) return fail(h, "dsb_publish: a segmented cycle is in progress");
  if (h->npub_chunks <= 0) return 0;
  hipStream_t cs = (hipStream_t)stream;
  CK(hipEventRecord(h->ev_in, cs));
  CK(hipStreamWaitEvent(h->hs, h->ev_in, 0));
  LK(lora_cast(h->d_pub_jobs, h->d_pub_chunks, h->npub_chunks, h->hs));
  CK(hipEventRecord(h->ev_out, h->hs));
  CK(hipStreamWaitEvent(cs, h->ev_out, 0));
  CK(hipEventSynchronize(h->ev_out));
  return 0;
}

// ------------------------------------------------------------ single ops

#define OPCK(expr)                                                                   \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess) {                                                          \
      set_error("%s: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, __LINE__); \
      return -1;                                                                     \
    }                                                                                \
  } while (0)

// ------------------------------------------------------------ capture

int dsb_capture_index(const int64_t* positions, int num_ft, int offset, int max_saved,
                      int64_t* src, int64_t* dst) {
  if (max_saved <= 0 || offset < 0 || num_ft < 0 || !src || !dst || (num_ft > 0 && !positions))
    return fail(nullptr, "dsb_capture_index: bad arguments");
  const int n = std::max(0, std::min(num_ft, max_saved - offset));
  for (int i = 0; i < max_saved; ++i) {
    src[i] = i < n ? positions[i] : 0;
    dst[i] = i < n ? (int64_t)offset + i : (int64_t)max_saved;
  }
  return n;
}

int dsb_save_rows(const void* x, int64_t ldx, const void* r, int64_t ldr, int64_t x_rows,
                  int x_dtype, const int64_t* src, const int64_t* dst, int count, int width,
                  void* buf, int64_t ldbuf, int64_t buf_rows, void* stream) {
  if (!x || !src || !dst || !buf || count < 0 || width <= 0 || ldx < width || ldbuf < width ||
      (r && ldr < width) || buf_rows < 1 || x_rows < 0)
    return fail(nullptr, "dsb_save_rows: bad arguments");
  if (x_dtype != DSB_DT_BF16 && x_dtype != DSB_DT_F16 && x_dtype != DSB_DT_F32)
    return fail(nullptr, "dsb_save_rows: x_dtype must be DSB_DT_BF16, DSB_DT_F16 or DSB_DT_F32");
  OPCK(save_rows(x, ldx, r, ldr, x_rows, x_dtype, src, dst, count, width, (bf16*)buf, ldbuf, buf_rows,
                 (hipStream_t)stream));
  return 0;
}

int dsb_save_ids(const int64_t* ids, int64_t ids_len, const int64_t* src, const int64_t* dst,
                 int count, int64_t* out, int64_t out_len, void* stream) {
  if (!ids || !src || !dst || !out || count < 0 || out_len < 0 || ids_len < 0)
    return fail(nullptr, "dsb_save_ids: bad arguments");
  OPCK(save_ids(ids, ids_len, src, dst, count, out, out_len, (hipStream_t)stream));
  return 0;
}

int dsb_op_gemm(const void* A, int64_t lda, const void* B, int64_t ldb, const void* A2,
                int64_t lda2, const void* B2, int64_t ldb2, int M, int N, int K1, int K2, void* C,
                int64_t ldc, int out_f32, int accumulate, const void* R, int64_t ldr, int b_kn,
                int cfg, void* stream) {
  if (K1 % 8 || K2 % 8 || lda % 8 || ldb % 8 || (K2 && (lda2 % 8 || ldb2 % 8)) || ldc % 4)
    return fail(nullptr, "dsb_op_gemm: K and leading dims must be multiples of 8 (ldc of 4)");
  if (b_kn && N % 8)
    return fail(nullptr, "dsb_op_gemm: a [K, N] B needs N a multiple of 8");
  hipStream_t s = (hipStream_t)stream;
  GemmProblem p{(const bf16*)A, lda, (const bf16*)B, ldb, (const bf16*)A2, lda2,
                (const bf16*)B2, ldb2, M, N, K1, K2, nullptr};
  p.b_kn = b_kn ? 1 : 0;
  // cfg -2: split K as the cycle does for problems with too few 256-wide
  // tiles; cfg -3: split K over the tiles of a partly filled last round, as
  // the cycle does (partials in a buffer allocated for the call); by shape
  // otherwise
  if (cfg == -3) {
    int dev = 0, ncu = 0, tail = 0;
    OPCK(hipGetDevice(&dev));
    OPCK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    const int kt = gemm_tail_split(M, N, K1 + K2, ncu, &tail);
    if (kt > 1) {
      float* tp = nullptr;
      OPCK(hipMalloc((void**)&tp, sizeof(float) * (size_t)kt * tail * 65536));
      hipError_t e1;
      if (out_f32) e1 = launch_gemm_tail(p, EpiF32{(float*)C, ldc, N, accumulate}, kt, tail, tp, s);
      else e1 = launch_gemm_tail(p, EpiBF16{(bf16*)C, ldc, N, (const bf16*)R, ldr}, kt, tail, tp, s);
      const hipError_t e2 = e1 == hipSuccess ? hipStreamSynchronize(s) : e1;
      (void)hipFree(tp);
      OPCK(e2);
      return 0;
    }
    cfg = -1;
  }
  const int ks = cfg == -2 ? gemm_split_count(M, N, K1 + K2) : 1;
  if (cfg == -2) cfg = -1;
  if (ks > 1) {
    OPCK(hipMalloc((void**)&p.part, sizeof(float) * (size_t)ks * M * N));
    hipError_t e1;
    if (out_f32) e1 = launch_gemm_split(p, EpiF32{(float*)C, ldc, N, accumulate}, ks, s);
    else e1 = launch_gemm_split(p, EpiBF16{(bf16*)C, ldc, N, (const bf16*)R, ldr}, ks, s);
    const hipError_t e2 = e1 == hipSuccess ? hipStreamSynchronize(s) : e1;
    (void)hipFree(p.part);
    OPCK(e2);
    return 0;
  }
  if (out_f32) {
    EpiF32 e{(float*)C, ldc, N, accumulate};
    OPCK(launch_gemm(p, e, s, cfg));
  } else {
    EpiBF16 e{(bf16*)C, ldc, N, (const bf16*)R, ldr};
    OPCK(launch_gemm(p, e, s, cfg));
  }
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_gemm_glu(const void* A, int64_t lda, const void* B, int64_t ldb, const void* A2,
                    int64_t lda2, const void* B2, int64_t ldb2, int M, int I, int K1, int K2,
                    void* GU, int64_t ldgu, void* H, int64_t ldh, void* stream) {
  if (K1 % 8 || K2 % 8 || lda % 8 || ldb % 8 || (K2 && (lda2 % 8 || ldb2 % 8)) || ldgu % 8 ||
      (H && ldh % 8) || I % 64 || I <= 0 || M < 0 ||
      !aligned16(A, B, A2, B2, GU, H))
    return fail(nullptr, "dsb_op_gemm_glu: I a multiple of 64; K, leading dims multiples of 8");
  GemmProblem p{(const bf16*)A, lda, (const bf16*)B, ldb, (const bf16*)A2, lda2,
                (const bf16*)B2, ldb2, M, 2 * I, K1, K2, nullptr};
  p.glu_half = I;
  EpiGLU e{(bf16*)GU, ldgu, (bf16*)H, ldh, I};
  hipStream_t s = (hipStream_t)stream;
  OPCK(launch_gemm(p, e, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_rmsnorm(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int rows,
                   int D, float eps, void* stream) {
  if (D % 8 || D > 8192) return fail(nullptr, "dsb_op_rmsnorm: D must be a multiple of 8, <= 8192");
  hipStream_t s = (hipStream_t)stream;
  OPCK(rmsnorm_fwd((const bf16*)x, ldx, (const bf16*)w, (bf16*)y, ldy, rows, nullptr, D, eps, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_rmsnorm_bwd(const void* x, int64_t ldx, const void* g, int g_f32, int64_t ldg,
                       const void* w, const void* resid, int64_t ldr, void* out, int64_t ldo,
                       int rows, int D, float eps, void* stream) {
  if (D % 8 || D > 8192) return fail(nullptr, "dsb_op_rmsnorm_bwd: D must be a multiple of 8, <= 8192");
  hipStream_t s = (hipStream_t)stream;
  OPCK(rmsnorm_bwd((const bf16*)x, ldx, g, g_f32 != 0, ldg, (const bf16*)w, (const bf16*)resid,
                   ldr, (bf16*)out, ldo, rows, nullptr, D, eps, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_rope_table(const int32_t* pos, int n, const float* inv_freq, int half, float* cos_out,
                      float* sin_out, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  OPCK(rope_table(pos, n, nullptr, inv_freq, half, cos_out, sin_out, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_rope(const void* qkv_pre, int64_t ldin, void* qk_out, int64_t ldout, const float* cos_t,
                const float* sin_t, int n, int Hq, int Hkv, int head_dim, const void* q_norm,
                const void* k_norm, float eps, void* stream) {
  if (ldin % 8 || ldout % 8 || !aligned16(qkv_pre, qk_out, q_norm, k_norm, cos_t, sin_t))
    return fail(nullptr, "dsb_op_rope: row strides must be multiples of 8, pointers 16-byte aligned");
  if (head_dim != 128 && head_dim != 64) return fail(nullptr, "dsb_op_rope: head_dim 128 or 64");
  hipStream_t s = (hipStream_t)stream;
  OPCK(rope_fwd((const bf16*)qkv_pre, ldin, (bf16*)qk_out, ldout, cos_t, sin_t, n, nullptr, Hq,
                Hkv, head_dim, (const bf16*)q_norm, (const bf16*)k_norm, eps, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_rope_bwd(void* g, int64_t ldg, const void* qkv_pre, int64_t ldp, const float* cos_t,
                    const float* sin_t, int n, int Hq, int Hkv, int head_dim, const void* q_norm,
                    const void* k_norm, float eps, void* stream) {
  if (ldg % 8 || ldp % 8 || !aligned16(g, qkv_pre, q_norm, k_norm, cos_t, sin_t))
    return fail(nullptr, "dsb_op_rope_bwd: row strides must be multiples of 8, pointers 16-byte aligned");
  if (head_dim != 128 && head_dim != 64)
    return fail(nullptr, "dsb_op_rope_bwd: head_dim 128 or 64");
  hipStream_t s = (hipStream_t)stream;
  OPCK(rope_bwd((bf16*)g, ldg, (const bf16*)qkv_pre, ldp, cos_t, sin_t, n, nullptr, Hq, Hkv,
                head_dim, (const bf16*)q_norm, (const bf16*)k_norm, eps, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

}  // extern "C"

namespace {
struct TmpDev {
  std::vector<void*> ptrs;
  ~TmpDev() {
    for (void* p : ptrs) (void)hipFree(p);
  }
  template <class T>
  T* alloc(size_t count) {
    void* p = nullptr;
    if (hipMalloc(&p, count * sizeof(T) + 256) != hipSuccess) return nullptr;
    ptrs.push_back(p);
    return (T*)p;
  }
};

int attn_setup(const int32_t* seq_lens, int nseq, TmpDev& tmp, AttnArgs& a, int* n_out) {
  std::vector<int4> tiles;
  long n = 0;
  for (int i = 0; i < nseq; ++i) n += seq_lens[i];
  if (pack_cycle(seq_lens, nseq, (int)n, nullptr, nullptr, &tiles) < 0)
    return fail(nullptr, "attention: bad seq_lens");
  std::vector<int4> by_q, by_k;
  order_tiles(tiles, by_q, by_k);
  int4* dt = tmp.alloc<int4>(2 * tiles.size() + 2);
  int* dn = tmp.alloc<int>(2);
  if (!dt || !dn) return fail(nullptr, "attention: hipMalloc failed");
  int hv[2] = {(int)tiles.size(), (int)n};
  if (!tiles.empty() &&
      (hipMemcpy(dt, by_q.data(), by_q.size() * sizeof(int4), hipMemcpyHostToDevice) != hipSuccess ||
       hipMemcpy(dt + tiles.size(), by_k.data(), by_k.size() * sizeof(int4),
                 hipMemcpyHostToDevice) != hipSuccess))
    return fail(nullptr, "attention: copy failed");
  if (hipMemcpy(dn, hv, sizeof(hv), hipMemcpyHostToDevice) != hipSuccess)
    return fail(nullptr, "attention: copy failed");
  a.tiles = dt;
  a.tiles_k = dt + tiles.size();
  a.ntiles_dev = dn;
  a.max_tiles = (int)tiles.size();
  a.n_dev = dn + 1;
  a.n = (int)n;
  *n_out = (int)n;
  return 0;
}
}  // namespace

extern "C" {

int dsb_op_attn_fwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                    int64_t ldv, void* ctx, int64_t ldc, float* o32, float* lse,
                    const int32_t* seq_lens, int nseq, int Hq, int Hkv, int head_dim,
                    void* stream) {
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv) return fail(nullptr, "attn: bad head counts");
  if (head_dim != 128 && head_dim != 64) return fail(nullptr, "attn: head_dim 128 or 64");
  hipStream_t s = (hipStream_t)stream;
  TmpDev tmp;
  AttnArgs a{};
  int n = 0;
  if (attn_setup(seq_lens, nseq, tmp, a, &n)) return -1;
  a.q = (const bf16*)q; a.ldq = ldq; a.k = (const bf16*)k; a.ldk = ldk;
  a.v = (const bf16*)v; a.ldv = ldv; a.ctx = (bf16*)ctx; a.ldc = ldc;
  a.o32 = o32; a.ldo32 = (long)Hq * head_dim; a.lse = lse; a.ld_stat = n; a.Hq = Hq; a.Hkv = Hkv;
  a.hd = head_dim; a.scale = 1.f / std::sqrt((float)head_dim);
  OPCK(attn_fwd(a, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_attn_bwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                    int64_t ldv, const float* o32, const float* lse, const void* dout,
                    int64_t lddo, void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv,
                    int64_t lddv, const int32_t* seq_lens, int nseq, int Hq, int Hkv,
                    int head_dim, void* stream) {
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv) return fail(nullptr, "attn: bad head counts");
  if (head_dim != 128 && head_dim != 64) return fail(nullptr, "attn: head_dim 128 or 64");
  if (!o32 || !lse) return fail(nullptr, "attn: o32 and lse from the forward are required");
  if (ldq % 8 || ldk % 8 || ldv % 8 || lddo % 8 ||
      (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dout | (uintptr_t)o32) & 15))
    return fail(nullptr, "attn: rows must be 16-byte aligned (ld multiple of 8)");
  hipStream_t s = (hipStream_t)stream;
  TmpDev tmp;
  AttnArgs a{};
  int n = 0;
  if (attn_setup(seq_lens, nseq, tmp, a, &n)) return -1;
  float* dsum = tmp.alloc<float>((size_t)Hq * (n + 1));
  if (!dsum) return fail(nullptr, "attn: hipMalloc failed");
  a.q = (const bf16*)q; a.ldq = ldq; a.k = (const bf16*)k; a.ldk = ldk;
  a.v = (const bf16*)v; a.ldv = ldv; a.o32 = (float*)o32; a.ldo32 = (long)Hq * head_dim;
  a.hd = head_dim; a.scale = 1.f / std::sqrt((float)head_dim);
  a.lse = (float*)lse; a.dsum = dsum; a.ld_stat = n; a.dout = (const bf16*)dout; a.lddo = lddo;
  a.dq = (bf16*)dq; a.lddq = lddq; a.dk = (bf16*)dk; a.lddk = lddk; a.dv = (bf16*)dv;
  a.lddv = lddv; a.Hq = Hq; a.Hkv = Hkv;
  // the dK/dV head split the cycle takes for short token counts, partials in
  // a buffer allocated for the call
  a.kv_part_elems = (long)(Hq / Hkv) * n * 2 * Hkv * head_dim;
  if (attn_dkdv_head_split(a) > 1) {
    a.kv_part = tmp.alloc<float>((size_t)a.kv_part_elems);
    if (!a.kv_part) return fail(nullptr, "attn: hipMalloc failed");
  }
  OPCK(attn_bwd(a, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_head(const void* normed, int64_t ldh, const void* lm_w, const int64_t* ids,
                const int32_t* seq_lens, int nseq, int n, int D, int V, int vocab_chunk,
                float* dH, float* loss, int* n_valid, void* stream) {
  if (D % 8 || V <= 0 || ldh % 8 || n < 0 || vocab_chunk < 0 || vocab_chunk % 256)
    return fail(nullptr, "dsb_op_head: D and ldh multiples of 8, V positive, vocab_chunk a "
                         "multiple of 256");
  hipStream_t s = (hipStream_t)stream;
  std::vector<int32_t> pred(n > 0 ? n : 1);
  const int nv = pack_cycle(seq_lens, nseq, n, nullptr, pred.data(), nullptr);
  if (nv < 0) return fail(nullptr, "dsb_op_head: seq_lens must sum to n");
  TmpDev tmp;
  const int ntn = (V + 255) / 256;
  const int vchunk = std::min(vocab_chunk > 0 ? vocab_chunk : 16384, ((V + 255) / 256) * 256);
  int* dpred = tmp.alloc<int>(n + 1);
  int* labels = tmp.alloc<int>(n + 1);
  float2* stats = tmp.alloc<float2>((size_t)(n + 1) * ntn);
  float* tl = tmp.alloc<float>(n + 1);
  float* lse = tmp.alloc<float>(n + 1);
  float* lr = tmp.alloc<float>(n + 1);
  float* rm = tmp.alloc<float>(n + 1);
  float* rl = tmp.alloc<float>(n + 1);
  float* al = tmp.alloc<float>(n + 1);
  float* scal = tmp.alloc<float>(4);
  int* err = tmp.alloc<int>(1);
  bf16* dlog = tmp.alloc<bf16>((size_t)(n + 1) * vchunk);
  if (!dpred || !labels || !stats || !tl || !lse || !lr || !rm || !rl || !al || !scal || !err ||
      !dlog)
    return fail(nullptr, "dsb_op_head: hipMalloc failed");
  float hsc[4] = {nv > 0 ? 1.f / nv : 0.f, 0.f, 0.f, 0.f};
  OPCK(hipMemcpy(scal, hsc, sizeof(hsc), hipMemcpyHostToDevice));
  if (n > 0) OPCK(hipMemcpy(dpred, pred.data(), n * sizeof(int32_t), hipMemcpyHostToDevice));
  OPCK(hipMemset(err, 0, sizeof(int)));
  OPCK(build_labels(ids, dpred, labels, n, nullptr, V, err, s));
  HeadArgs a{};
  a.normed = (const bf16*)normed; a.ldh = ldh; a.W = (const bf16*)lm_w;
  a.labels = labels; a.n = n; a.n_dev = nullptr; a.D = D; a.V = V; a.stats = stats; a.ntn = ntn;
  a.tgt_logit = tl; a.lse = lse; a.loss_row = lr; a.loss_out = scal + 1; a.inv_nvalid = scal;
  a.run_m = rm; a.run_l = rl; a.alpha = al;
  a.dlog = dlog; a.vchunk = vchunk; a.dH = dH; a.gemm_cfg = -1;
  OPCK(head_fwd_bwd(a, s));
  OPCK(hipStreamSynchronize(s));
  int herr = 0;
  OPCK(hipMemcpy(&herr, err, sizeof(int), hipMemcpyDeviceToHost));
  if (herr) return fail(nullptr, "dsb_op_head: a target token id is outside [0, vocab)");
  OPCK(hipMemcpy(hsc, scal, sizeof(hsc), hipMemcpyDeviceToHost));
  if (loss) *loss = hsc[1];
  if (n_valid) *n_valid = nv;
  return 0;
}

int dsb_op_lora_tn(const void* P, int64_t ldp, const void* X, int64_t ldx, int n, int R, int C,
                   float scale, float* out0, float* out1, float* out2, int rg, int transpose_out,
                   void* stream) {
  if (C % 8 || ldx % 8 || rg <= 0 || (R + rg - 1) / rg > 3)
    return fail(nullptr, "dsb_op_lora_tn: C and ldx must be multiples of 8, at most 3 groups");
  hipStream_t s = (hipStream_t)stream;
  TmpDev tmp;
  const int ns = 8;
  float* work = tmp.alloc<float>((size_t)ns * R * C);
  if (!work) return fail(nullptr, "dsb_op_lora_tn: hipMalloc failed");
  TnArgs a{};
  a.P = (const bf16*)P; a.ldp = ldp; a.X = (const bf16*)X; a.ldx = ldx; a.R = R; a.C = C; a.n = n;
  a.n_dev = nullptr; a.work = work; a.nsplit = ns; a.outs[0] = out0; a.outs[1] = out1;
  a.outs[2] = out2; a.rg = rg; a.transpose_out = transpose_out; a.scale = scale;
  OPCK(lora_tn(a, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_lora_skinny(const void* X, int64_t ldx, const void* B, int64_t ldb, int n, int R, int K,
                       void* Z, int64_t ldz, void* stream) {
  if (K % 8 || ldx % 8 || ldb % 8) return fail(nullptr, "dsb_op_lora_skinny: K, ldx, ldb must be multiples of 8");
  hipStream_t s = (hipStream_t)stream;
  SkinnyArgs a{(const bf16*)X, ldx, (const bf16*)B, ldb, R, K, (bf16*)Z, ldz, n, nullptr};
  // the K split the cycle takes for short token ranges, partials in a buffer
  // allocated for the call
  TmpDev tmp;
  a.part_elems = 8L * n * R;
  if (lora_skinny_split(a) > 1) {
    a.part = tmp.alloc<float>((size_t)a.part_elems);
    if (!a.part) return fail(nullptr, "dsb_op_lora_skinny: hipMalloc failed");
  }
  OPCK(lora_skinny(a, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

}  // extern "C"

namespace {
// Validates a dsb_op_lora_dual request and fills the kernel arguments; the
// partial-sum workspace of pass i is laid out at work_off[i] floats.
int dual_setup(const dsb_dual_pass* passes, int count, int n, int n_alloc, int r,
               const int* n_dev, DualArgs* a, long* work_elems, const char* who) {
  if (!passes || count < 1 || count > 3 || n < 0 || n_alloc < n || n_alloc < 1) {
    set_error("%s: 1 to 3 passes, 0 <= n <= n_alloc", who);
    return -1;
  }
  const int C0 = passes[0].C;
  int ncb = 0;
  for (int i = 0; i < count; ++i) ncb += (passes[i].C + 511) / 512;
  const int ns = std::max(1, std::min(256 / std::max(ncb, 1), n_alloc / 64));
  long off = 0;
  for (int i = 0; i < count; ++i) {
    const dsb_dual_pass& p = passes[i];
    if (!lora_dual_supported(r, r, p.C) || p.ldg % 8 || p.ldbt % 8 || p.ldg < p.C ||
        p.ldbt < p.C || p.ldz < r || p.ldgz < r || !p.G || !p.Z || !p.BT || !p.gZ || !p.gB ||
        !aligned16(p.G, p.Z, p.BT)) {
      set_error("%s: r must be 16 or 32; C, ldg, ldbt multiples of 8 (>= C), ldz and ldgz >= r, "
                "G/Z/BT 16-byte aligned", who);
      return -1;
    }
    DualArgs& x = a[i];
    x = DualArgs{};
    x.X = (const bf16*)p.G; x.ldx = p.ldg; x.P = (const bf16*)p.Z; x.ldp = p.ldz;
    x.W = (const bf16*)p.BT; x.ldw = p.ldbt; x.R1 = r; x.R2 = r; x.C = p.C;
    x.n = n; x.n_dev = n_dev; x.n_alloc = n_alloc; x.nsplit = ns;
    x.Y = (bf16*)p.gZ; x.ldy = p.ldgz; x.out = p.gB; x.scale = p.scale;
    x.transpose_out = p.transpose_out;
    x.work = reinterpret_cast<float*>(off);  // offset; rebased by the caller
    off += (long)((p.C + 511) / 512) * n_alloc * r + (long)ns * p.C * r;
  }
  (void)C0;
  *work_elems = off;
  return 0;
}
}  // namespace

extern "C" {

}  // extern "C"

// ---- the allocation-free variant of dsb_op_lora_dual
//
// Its partial-sum workspace is this file-scope device array. Each GPU the
// library runs on holds its own copy (64 MiB) until the process ends; host
// code never uses the array's name as an address (on the host it is only a
// stand-in): the device address is looked up once per device with
// hipGetSymbolAddress and kept in scratch_dev.
namespace {
constexpr long kScratchFloats = 16L << 20;  // 64 MiB
constexpr int kMaxDevices = 64;
__device__ __align__(256) float scratch[kScratchFloats];
float* scratch_dev[kMaxDevices] = {};
std::mutex scratch_mu;

// This device's scratch address, looked up on its first use (with the device
// current); null with the error set if the lookup fails.
float* scratch_for_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("dsb_op_lora_dual_noalloc: no current HIP device (or device index >= %d)",
              kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    // The first call on a device may come while a stream of this thread is
    // being captured into a graph: the lookup is not a stream operation, and
    // relaxed mode lets it run under any capture mode.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || !p) {
      set_error("dsb_op_lora_dual_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                dev, hipGetErrorString(e));
      return nullptr;
    }
    scratch_dev[dev] = static_cast<float*>(p);
  }
  return scratch_dev[dev];
}
}  // namespace

extern "C" {

int dsb_op_lora_dual_noalloc(const dsb_dual_pass* passes, int count, int n, int n_alloc, int r,
                             void* stream) {
  DualArgs a[3];
  long elems = 0;
  if (dual_setup(passes, count, n, n_alloc, r, nullptr, a, &elems,
                 "dsb_op_lora_dual_noalloc"))
    return -1;
  if (elems > kScratchFloats)
    return fail(nullptr, "dsb_op_lora_dual_noalloc: the partial sums of this request need more "
                         "than the 64 MiB scratch array (fewer rows or columns per call)");
  float* work = scratch_for_current_device();
  if (!work) return -1;
  if (n == 0) return 0;
  // every partial is written before the reductions read it: nothing to clear
  for (int i = 0; i < count; ++i) a[i].work = work + reinterpret_cast<long>(a[i].work);
  OPCK(lora_dual(a, count, (hipStream_t)stream));
  return 0;
}

int dsb_op_lora_dual(const dsb_dual_pass* passes, int count, int n, int n_alloc, int r,
                     void* stream) {
  DualArgs a[3];
  long elems = 0;
  if (dual_setup(passes, count, n, n_alloc, r, nullptr, a, &elems, "dsb_op_lora_dual"))
    return -1;
  if (n == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  TmpDev tmp;
  float* work = tmp.alloc<float>((size_t)elems);
  int* nd = tmp.alloc<int>(1);
  if (!work || !nd) return fail(nullptr, "dsb_op_lora_dual: hipMalloc failed");
  OPCK(hipMemcpy(nd, &n, sizeof(int), hipMemcpyHostToDevice));
  for (int i = 0; i < count; ++i) {
    a[i].work = work + reinterpret_cast<long>(a[i].work);
    a[i].n_dev = nd;
    a[i].n = n_alloc;  // grid sized for the capacity, live rows from the device
  }
  OPCK(lora_dual(a, count, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

int dsb_op_clip_adamw(float* const* w, float* const* g, float* const* m, float* const* v,
                      const int32_t* numel, const int32_t* group, int ntensors, int ngroups,
                      float lr, float beta1, float beta2, float eps, float wd, int64_t step,
                      float max_norm, int do_clip, void* stream) {
  if (ntensors <= 0 || ngroups <= 0 || step < 1) return fail(nullptr, "dsb_op_clip_adamw: bad sizes");
  std::vector<OptTensor> T;
  std::vector<int2> chunks, lchunks(ngroups, int2{0, 0});
  int prev = -1;
  for (int i = 0; i < ntensors; ++i) {
    if (group[i] < prev || group[i] >= ngroups)
      return fail(nullptr, "dsb_op_clip_adamw: groups must be non-decreasing and < ngroups");
    if (group[i] != prev) {
      for (int gidx = prev + 1; gidx <= group[i]; ++gidx) lchunks[gidx] = int2{(int)chunks.size(), 0};
      prev = group[i];
    }
    T.push_back(OptTensor{w[i], g[i], m[i], v[i], numel[i], group[i]});
    for (int st = 0; st < numel[i]; st += 4096) chunks.push_back(int2{i, st});
    lchunks[group[i]].y = (int)chunks.size() - lchunks[group[i]].x;
  }
  for (int gidx = prev + 1; gidx < ngroups; ++gidx) lchunks[gidx] = int2{(int)chunks.size(), 0};
  hipStream_t s = (hipStream_t)stream;
  TmpDev tmp;
  OptTensor* dT = tmp.alloc<OptTensor>(T.size());
  int2* dc = tmp.alloc<int2>(chunks.size() + 1);
  int2* dl = tmp.alloc<int2>(lchunks.size());
  float* part = tmp.alloc<float>(chunks.size() + 1);
  float* sq = tmp.alloc<float>(ngroups);
  OptHyper* hp = tmp.alloc<OptHyper>(1);
  if (!dT || !dc || !dl || !part || !sq || !hp) return fail(nullptr, "dsb_op_clip_adamw: hipMalloc failed");
  OptHyper hh{lr, beta1, beta2, eps, wd, (float)(1.0 - pow((double)beta1, (double)step)),
              (float)(1.0 - pow((double)beta2, (double)step)), max_norm};
  OPCK(hipMemcpy(dT, T.data(), T.size() * sizeof(OptTensor), hipMemcpyHostToDevice));
  if (!chunks.empty())
    OPCK(hipMemcpy(dc, chunks.data(), chunks.size() * sizeof(int2), hipMemcpyHostToDevice));
  OPCK(hipMemcpy(dl, lchunks.data(), lchunks.size() * sizeof(int2), hipMemcpyHostToDevice));
  OPCK(hipMemcpy(hp, &hh, sizeof(hh), hipMemcpyHostToDevice));
  OPCK(hipMemset(sq, 0, ngroups * sizeof(float)));
  OPCK(clip_adamw(dT, dc, (int)chunks.size(), dl, ngroups, part, sq, hp, do_clip, s));
  OPCK(hipStreamSynchronize(s));
  return 0;
}

}  // extern "C"
