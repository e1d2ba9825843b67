// Per-layer gradient clipping + AdamW over all LoRA masters, multi-tensor.
//
// Semantics:
//   clip: deltaserve-plugin/deltaserve/bwd_services/common/trainer.py:624-636
//     (torch.nn.utils.clip_grad_norm_(layer's LoRA grads, max_norm=1.0) per
//     layer; restated at common/tp.py:249-258): total = sqrt(sum g²) over the
//     layer, coef = min(1, max_norm / (total + 1e-6)), grads scaled in place.
//   AdamW: trainer.py:252-254, :668 (torch.optim.AdamW, betas (0.9, 0.999),
//     eps 1e-8, decoupled weight decay):
//       w -= lr·wd·w; m = β1·m + (1-β1)·g; v = β2·v + (1-β2)·g²
//       w -= (lr / bc1) · m / (sqrt(v) / sqrt(bc2) + eps),  bc_i = 1 - β_i^t
//
// Tensors are cut into 4096-element chunks; a layer's chunks are contiguous,
// so its squared norm is a fixed-order sum of chunk partials (deterministic).
#include "kernels.h"

namespace dsb {

namespace {
constexpr int OPT_CHUNK = 4096;
}

__global__ __launch_bounds__(256) void sumsq_kernel(const OptTensor* __restrict__ T,
                                                    const int2* __restrict__ chunks,
                                                    float* __restrict__ partial) {
  __shared__ float red[4];
  const int2 ck = chunks[blockIdx.x];
  const OptTensor t = T[ck.x];
  const int end = min(t.numel, ck.y + OPT_CHUNK);
  float s = 0.f;
  for (int i = ck.y + threadIdx.x; i < end; i += 256) {
    const float g = t.g[i];
    s += g * g;
  }
  s = block_sum<256>(s, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = s;
}

__global__ __launch_bounds__(64) void layer_sq_kernel(const int2* __restrict__ layer_chunks,
                                                      const float* __restrict__ partial,
                                                      float* __restrict__ sq) {
  const int2 lc = layer_chunks[blockIdx.x];
  float s = 0.f;
  for (int i = threadIdx.x; i < lc.y; i += 64) s += partial[lc.x + i];
  s = wave_sum(s);
  if (threadIdx.x == 0) sq[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void adamw_kernel(const OptTensor* __restrict__ T,
                                                    const int2* __restrict__ chunks,
                                                    const float* __restrict__ sq,
                                                    const OptHyper* __restrict__ hp,
                                                    int do_clip) {
  const int2 ck = chunks[blockIdx.x];
  const OptTensor t = T[ck.x];
  const OptHyper h = *hp;
  float coef = 1.f;
  if (do_clip) coef = fminf(1.f, h.max_norm / (sqrtf(sq[t.layer]) + 1e-6f));
  const float step_size = h.lr / h.bc1;
  const float bc2s = sqrtf(h.bc2);
  const int end = min(t.numel, ck.y + OPT_CHUNK);
  for (int i = ck.y + threadIdx.x; i < end; i += 256) {
    float g = t.g[i];
    if (do_clip) {
      g *= coef;
      t.g[i] = g;
    }
    float w = t.w[i];
    w -= h.lr * h.wd * w;
    const float m = h.beta1 * t.m[i] + (1.f - h.beta1) * g;
    const float v = h.beta2 * t.v[i] + (1.f - h.beta2) * g * g;
    t.m[i] = m;
    t.v[i] = v;
    w -= step_size * m / (sqrtf(v) / bc2s + h.eps);
    t.w[i] = w;
  }
}

hipError_t clip_adamw(const OptTensor* tensors_dev, const int2* chunks_dev, int nchunks,
                      const int2* layer_chunks_dev, int nlayers, float* partial,
                      float* sq_layer, const OptHyper* hyper_dev, int do_clip, hipStream_t s) {
  if (nchunks <= 0) return hipSuccess;
  if (do_clip) {
    hipLaunchKernelGGL(sumsq_kernel, dim3(nchunks), dim3(256), 0, s, tensors_dev, chunks_dev,
                       partial);
    hipLaunchKernelGGL(layer_sq_kernel, dim3(nlayers), dim3(64), 0, s, layer_chunks_dev,
                       partial, sq_layer);
  }
  hipLaunchKernelGGL(adamw_kernel, dim3(nchunks), dim3(256), 0, s, tensors_dev, chunks_dev,
                     sq_layer, hyper_dev, do_clip);
  return hipGetLastError();
}

}  // namespace dsb
