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

// One 16x16x32 bf16 MFMA. Lane l supplies row l%16 of each operand with the
// 8 K-values 8·(l/16) .. +7; the result lane l holds Y-row l%16 against
// X-rows 4·(l/16) + i, i = 0..3 (mfma16(X, Y)).
DSB_DEV f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
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
// A non-temporal 16-byte load: for data an epilogue reads once, so the
// bursts of a whole round of tiles do not evict the operand panels the next
// tiles read from L2 (the SwiGLU backward: 885 -> 815 µs per C3 launch).
DSB_DEV u32x4 ldg128_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
DSB_DEV void stg128(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// σ(x) = 1/(1 + e^(−x)) with the hardware reciprocal (1 ulp) in place of an
// IEEE division (a dozen instructions per element in the SwiGLU epilogues);
// e^(−x) = inf for x → −inf gives 0, and 0 for x → +inf gives 1.
DSB_DEV float sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

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

// ---- direct-to-LDS loads (shared by the GEMM and attention pipelines)

// The direct-to-LDS loads and the waits on them are issued as inline asm:
// the compiler's wait-count pass then neither tracks them nor inserts its own
// conservative vmcnt(0) before fragment reads (it loses track of which LDS
// stage a pending load targets across the loop back edge). Correctness rests
// on the explicit vmcnt waits below plus the barrier; the "memory" clobbers
// keep the compiler from moving LDS accesses across them. No compiler-visible
// global loads are outstanding while the ring runs.
template <int N>
DSB_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait for every outstanding LDS access (and scalar memory load) of the wave.
DSB_DEV void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier without a memory fence (a fence would wait for every
// outstanding load, including the prefetched stages); the empty asm statements
// keep the compiler from moving memory accesses across it.
DSB_DEV void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// buffer_load_dwordx4 ... lds: 64 lanes × 16 B land at lds_addr + 16·lane.
// M0 holds the LDS address (saved and restored around the load: M0 is a
// reserved register the compiler assumes preserved); one wait state
// separates the M0 write from the load.
DSB_DEV void lds_dma16(u32x4 rsrc, int voff, unsigned lds_addr) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(lds_addr)
      : "memory");
}

// Buffer descriptor (gfx9): base, stride 0, num_records bytes, raw dword access.
DSB_DEV u32x4 make_rsrc(const void* base, int bytes) {
  const unsigned long a = (unsigned long)base;
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((unsigned)a);
  r[1] = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane((unsigned)bytes);
  r[3] = 0x00020000u;
  return r;
}

// 1 KB of zeros in device memory (static device storage starts zeroed and
// nothing writes it). A buffer load whose every lane falls outside its
// descriptor never reaches memory and can complete ahead of loads issued
// before it, which breaks a wait that counts outstanding loads
// (s_waitcnt vmcnt(N), N > 0); such loads read this page instead
// (64 lanes × 16 B), so the loads of a pipelined loop complete in order.
static __device__ __align__(256) bf16 zero_page[512];
DSB_DEV u32x4 zero_rsrc() { return make_rsrc(zero_page, (int)sizeof(zero_page)); }
// Buffer descriptor for plain (register-destination) buffer loads: same
// fields as make_rsrc; loads at or beyond `bytes` return zeros.
DSB_DEV __amdgpu_buffer_rsrc_t make_brsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
// 16 bytes per lane at byte offset `off` of the descriptor's range.
DSB_DEV u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

typedef __attribute__((address_space(3))) bf16 lds_bf16;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
DSB_DEV unsigned lds_addr(bf16* p) {
  return __builtin_amdgcn_readfirstlane((unsigned)(unsigned long)(lds_bf16*)p);
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
