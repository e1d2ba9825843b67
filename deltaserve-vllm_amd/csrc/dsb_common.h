// Shared device helpers for the DeltaServe LoRA-SFT backward on gfx950 (MI355X).
//
// Storage types: bf16 activations/weights (bit-compatible with torch.bfloat16),
// fp32 LoRA masters, grads, optimizer moments and softmax statistics.
// Matrix products use v_mfma_f32_32x32x16_bf16 (fp32 accumulate).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsb {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

#define DSB_DEV __device__ __forceinline__

DSB_DEV float bf2f(bf16 x) { return (float)x; }
DSB_DEV bf16 f2bf(float x) { return (bf16)x; }  // round-to-nearest-even

// One 32x32x16 bf16 MFMA. Output layout (per lane l, acc index r):
//   column j = l % 32, row i = 8*(r/4) + 4*(l/32) + (r%4).
// Operand layout: lane l supplies row/col (l % 32) and the 8 K-values of
// half (l / 32); the same (half, element) -> k map is used for both operands.
DSB_DEV f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

DSB_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
DSB_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Block-wide sum for blockDim.x == NT (multiple of 64). `red` holds NT/64 floats.
template <int NT>
DSB_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) t += red[i];
  __syncthreads();
  return t;
}

DSB_DEV u32x4 ldg128(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
DSB_DEV void stg128(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

DSB_DEV void unpack8(u32x4 v, float f[8]) {
  const bf16x8 b = __builtin_bit_cast(bf16x8, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)b[i];
}
DSB_DEV u32x4 pack8(const float f[8]) {
  bf16x8 b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (bf16)f[i];
  return __builtin_bit_cast(u32x4, b);
}

}  // namespace dsb

// Host-side error plumbing shared by the C-ABI translation units.
#define DSB_HIP_CHECK(expr)                                                   \
  do {                                                                        \
    hipError_t _e = (expr);                                                   \
    if (_e != hipSuccess) {                                                   \
      ::dsb::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                       __FILE__, __LINE__);                                   \
      return -1;                                                              \
    }                                                                         \
  } while (0)

namespace dsb {
void set_error(const char* fmt, ...);
const char* get_error();
}  // namespace dsb
