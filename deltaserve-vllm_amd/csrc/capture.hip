// The forward-side half of the activation handoff: the serving step's save of
// the finetuning rows into the activation store the backward reads.
//
// Semantics: deltaserve-plugin/deltaserve/ft_save_op.py:72-93 (the
// graph-capturable save op) and accumulate.py:324-343 (arm_op_step):
//   rows = x.index_select(0, src) (+ r.index_select(0, src)),  in x's dtype
//   buf.index_copy_(0, dst, rows.to(buf.dtype))
// with src/dst persistent int64 index tensors of a fixed length (max_saved):
// the first n entries gather the step's FT rows into buffer rows
// offset .. offset+n-1, the rest point at row 0 and the scratch row
// buf[max_saved]. The scratch row is never read by the backward (every
// consumer slices [:n]); this kernel skips those slots instead of writing
// them, which also removes their memory traffic. The final save point's
// input ids go through the same index pair (accumulate.py:598-622).
//
// Slots whose source row lies outside x (or the id vector) are skipped too:
// the gather never reads out of bounds.
//
// Both kernels take a fixed row count and read the indices from device
// memory, so a captured graph replays them with fresh indices each step.
#include "kernels.h"

namespace dsb {

namespace {
template <int T>
DSB_DEV float load_as_float(const void* p, long i);
template <>
DSB_DEV float load_as_float<DSB_DT_BF16>(const void* p, long i) {
  return (float)reinterpret_cast<const bf16*>(p)[i];
}
template <>
DSB_DEV float load_as_float<DSB_DT_F16>(const void* p, long i) {
  return (float)reinterpret_cast<const _Float16*>(p)[i];
}
template <>
DSB_DEV float load_as_float<DSB_DT_F32>(const void* p, long i) {
  return reinterpret_cast<const float*>(p)[i];
}
// round to the input dtype (the reference adds in x's dtype)
template <int T>
DSB_DEV float round_to(float v);
template <>
DSB_DEV float round_to<DSB_DT_BF16>(float v) { return (float)(bf16)v; }
template <>
DSB_DEV float round_to<DSB_DT_F16>(float v) { return (float)(_Float16)v; }
template <>
DSB_DEV float round_to<DSB_DT_F32>(float v) { return v; }
}  // namespace

// One block per index slot; the block's threads cover the row's width.
template <int T>
__global__ __launch_bounds__(256) void save_rows_kernel(const void* __restrict__ x, long ldx,
                                                        const void* __restrict__ r, long ldr,
                                                        long x_rows,
                                                        const int64_t* __restrict__ src,
                                                        const int64_t* __restrict__ dst, int width,
                                                        bf16* __restrict__ buf, long ldbuf,
                                                        long buf_rows) {
  const long d = dst[blockIdx.x];
  if (d < 0 || d >= buf_rows - 1) return;  // the scratch row (and out of range): skipped
  const long s = src[blockIdx.x];
  if (s < 0 || s >= x_rows) return;  // a source row outside x: skipped
  const long xo = s * ldx, ro = s * ldr, bo = d * ldbuf;
  if (T == DSB_DT_BF16 && !r && (width & 7) == 0 && ((ldx | ldbuf) & 7) == 0 &&
      (((unsigned long)x | (unsigned long)buf) & 15) == 0) {
    // plain bf16 copy: 16 bytes per lane
    const bf16* xs = reinterpret_cast<const bf16*>(x) + xo;
    for (int c = threadIdx.x * 8; c < width; c += 256 * 8)
      stg128(buf + bo + c, ldg128(xs + c));
    return;
  }
  for (int c = threadIdx.x; c < width; c += 256) {
    float v = load_as_float<T>(x, xo + c);
    if (r) v = round_to<T>(v + load_as_float<T>(r, ro + c));
    buf[bo + c] = (bf16)v;
  }
}

__global__ __launch_bounds__(256) void save_ids_kernel(const int64_t* __restrict__ ids,
                                                       long ids_len,
                                                       const int64_t* __restrict__ src,
                                                       const int64_t* __restrict__ dst, int count,
                                                       int64_t* __restrict__ out, long out_len) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const long d = dst[i];
  const long s = src[i];
  if (d < 0 || d >= out_len || s < 0 || s >= ids_len) return;
  out[d] = ids[s];
}

hipError_t save_rows(const void* x, long ldx, const void* r, long ldr, long x_rows, int dtype,
                     const int64_t* src, const int64_t* dst, int count, int width, bf16* buf,
                     long ldbuf, long buf_rows, hipStream_t s) {
  if (count <= 0 || width <= 0) return hipSuccess;
  switch (dtype) {
    case DSB_DT_BF16:
      hipLaunchKernelGGL(save_rows_kernel<DSB_DT_BF16>, dim3(count), dim3(256), 0, s, x, ldx, r,
                         ldr, x_rows, src, dst, width, buf, ldbuf, buf_rows);
      break;
    case DSB_DT_F16:
      hipLaunchKernelGGL(save_rows_kernel<DSB_DT_F16>, dim3(count), dim3(256), 0, s, x, ldx, r, ldr,
                         x_rows, src, dst, width, buf, ldbuf, buf_rows);
      break;
    case DSB_DT_F32:
      hipLaunchKernelGGL(save_rows_kernel<DSB_DT_F32>, dim3(count), dim3(256), 0, s, x, ldx, r, ldr,
                         x_rows, src, dst, width, buf, ldbuf, buf_rows);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t save_ids(const int64_t* ids, long ids_len, const int64_t* src, const int64_t* dst, int count,
                    int64_t* out, long out_len, hipStream_t s) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(save_ids_kernel, dim3((count + 255) / 256), dim3(256), 0, s, ids, ids_len, src,
                     dst, count, out, out_len);
  return hipGetLastError();
}

}  // namespace dsb
