// LoRA factor plumbing:
//  * lora_cast: per-cycle fp32 master → bf16 operand copies in the layouts the
//    NT GEMM consumes (A, Aᵀ, s·B into block-diagonal K-concat slabs, (s·B)ᵀ).
//    The reference casts the masters inline per call (ops.py:103-146:
//    `A.to(xin.dtype)`, `B.to(xin.dtype)`); here one multi-tensor launch does it.
//  * lora_skinny: the rank-r products that keep the token dimension,
//      Z = X·Aᵀ (ops.py:141) and gZ = G·(s·B) (ops.py:142), [n, R] bf16 out.
//  * lora_tn: the rank-r weight gradients that reduce over tokens,
//      gA = gZᵀ·X   (ops.py:143, grad_A = grad_Z.t() @ xin)
//      gB = s·Gᵀ·Z  (ops.py:144, grad_B = scaling * (gy.t() @ Z))
//
// Both rank-r products are HBM-bound (they stream an [n, width] activation
// once for a few flops per byte). Each streams its activation through a ring
// of LDS stages filled by direct-to-LDS loads (the tile layout of tile256.h)
// so that tens of KB per CU are in flight, and multiplies with 16×16×32
// MFMAs; the TN reduction over tokens reads both operands transposed from
// LDS with ds_read_b64_tr_b16.
#include <algorithm>

#include "kernels.h"
#include "tile256.h"

namespace dsb {

__global__ __launch_bounds__(256) void lora_cast_kernel(const CastJob* __restrict__ jobs,
                                                        const int2* __restrict__ chunks) {
  const int2 ck = chunks[blockIdx.x];
  const CastJob j = jobs[ck.x];
  const long tot = (long)j.rows * j.cols;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const long idx = (long)ck.y + threadIdx.x + e * 256;
    if (idx >= tot) break;
    const int r = (int)(idx / j.cols), c = (int)(idx % j.cols);
    float v = j.src[(long)r * j.ld_src + c] * j.scale;
    // clamp like torch.clamp: NaN stays NaN (comparisons with NaN are false)
    if (j.clamp > 0.f) v = v > j.clamp ? j.clamp : (v < -j.clamp ? -j.clamp : v);
    const long d = j.transpose ? (long)c * j.ld_dst + r : (long)r * j.ld_dst + c;
    j.dst[d] = (bf16)v;
  }
}

hipError_t lora_cast(const CastJob* jobs_dev, const int2* chunks_dev, int nchunks,
                     hipStream_t s) {
  if (nchunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(lora_cast_kernel, dim3(nchunks), dim3(256), 0, s, jobs_dev, chunks_dev);
  return hipGetLastError();
}

// ------------------------------------------------------------------ skinny NT
// Z[t, j] = sum_k X[t, k]·B[j, k]. Block: 16·TT tokens (TT = 1 for short
// rows, so more blocks share each CU and hide each other's ramp-up; TT = 2
// for long ones); the X chunk [16·TT × 128] and the B chunk [16·RB × 128]
// stream through a direct-to-LDS ring of up to 96 KB (up to 8 stages; one
// barrier per chunk); wave w multiplies columns 32w .. 32w+31 of each chunk
// with 16×16×32 MFMAs (TT token tiles × RB rank tiles) and the four waves'
// partial sums are added through LDS at the end. With a K split (grid.z > 1)
// block z takes the z-th run of 128-column chunks and stores its fp32 sums
// to a.part[z][t][j]; lora_skinny_reduce_kernel adds the slices in order.
template <int TT, int RB>
__global__ __launch_bounds__(256, 2) void lora_skinny_kernel(SkinnyArgs a) {
  constexpr int TR = 16 * TT;  // tokens per block
  constexpr int XT = TR * 128, BT = 16 * RB * 128, SE = XT + BT;
  constexpr int NS = (48 * 1024) / SE < 8 ? (48 * 1024) / SE : 8;  // SE elements = 2·SE bytes
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int t0 = blockIdx.x * TR;
  if (t0 >= N) return;
  __shared__ __attribute__((aligned(16))) bf16 smem[NS * SE];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rows = min(N - t0, TR);
  const bf16* X0 = a.X + (long)t0 * a.ldx;
  const int nc = (a.K + 127) / 128;
  // this block's chunks [cb, ce) (all of them unless K is split over grid.z)
  const int nz = (int)gridDim.z;
  const int cpk = nz == 1 ? nc : (nc + nz - 1) / nz;
  const int cb = min(nc, (int)blockIdx.z * cpk), ce = min(nc, cb + cpk);
  // ranks j0 .. j0 + Rg - 1 of this block (groups of 64 on grid.y)
  const int j0 = blockIdx.y * 64, Rg = min(a.R - j0, 64);
  const bf16* Bg = a.B + (long)j0 * a.ldb;
  // Chunk loads (the tile layout of tile256.h), set up once per block: one
  // descriptor per operand over its rows, the lane's offsets; per chunk only
  // the column advance, the lane's column test (past K: zeros) and, for a
  // load with no valid row or column, the zero page (so every load touches
  // memory and the ring's counted waits hold).
  const u32x4 zs = zero_rsrc();
  const u32x4 rx = make_rsrc(X0, (int)(((long)(rows - 1) * a.ldx + a.K) * 2));
  const u32x4 rb = make_rsrc(Bg, Rg > 0 ? (int)(((long)(Rg - 1) * a.ldb + a.K) * 2) : 0);
  const int lr4 = 4 * w + (lane >> 4);                  // load 0's row; load i adds 16·i
  const int lcol = ((lane & 15) ^ aswz(lr4)) << 3;      // aswz(r) depends on r % 16 only
  const int xl = (int)(((long)lr4 * a.ldx + lcol) * 2), bl = (int)(((long)lr4 * a.ldb + lcol) * 2);
  const unsigned lds0 = lds_addr(smem);
  auto issue = [&](int c, int slot) {
    const int k0 = c * 128;
    const bool kin = c < ce;            // uniform (ce <= nc: the chunk starts inside K)
    const bool cin = k0 + lcol < a.K;   // the lane's chunk
    const unsigned d = lds0 + (unsigned)(slot * SE * 2);
#pragma unroll
    for (int i = 0; i < TR / 16; ++i) {
      const bool live = kin && 4 * (4 * i + w) < rows;
      const int v = cin ? xl + (int)((long)16 * i * a.ldx * 2) + k0 * 2 : 0x7ff00000;
      lds_dma16(live ? rx : zs, live ? v : lane * 16, d + (unsigned)((4 * (4 * i + w)) * 256));
    }
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const bool live = kin && 4 * (4 * i + w) < Rg;
      const int v = cin ? bl + (int)((long)16 * i * a.ldb * 2) + k0 * 2 : 0x7ff00000;
      lds_dma16(live ? rb : zs, live ? v : lane * 16,
                d + (unsigned)((XT + (4 * (4 * i + w)) * 128) * 2));
    }
  };
  constexpr int LPS = TT + RB;  // loads per lane per stage
  f32x4 acc[TT][RB];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < RB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // fragment offsets (bytes): row l%16 of a 16-row tile, columns 32w + 8(l/16)
  const int fr = lane & 15, fc = 32 * w + 8 * (lane >> 4);
  const int off = toff(fr, fc) * 2;  // tiles start at multiples of 16 rows: f(r) = f(l%16)

#pragma unroll
  for (int c = 0; c < NS - 1; ++c) issue(cb + c, c);
  for (int c = cb; c < ce; ++c) {
    const int i = c - cb;        // ring position
    wait_vm<(NS - 2) * LPS>();  // own loads of chunk c landed (c+1 .. c+NS-2 may fly)
    lds_barrier();               // chunk c visible; the slot of chunk c-1 is free
    issue(c + NS - 1, (i + NS - 1) % NS);
    const char* st = reinterpret_cast<const char*>(smem + (i % NS) * SE);
    bf16x8 xf[TT], bfr[RB];
#pragma unroll
    for (int i = 0; i < TT; ++i) xf[i] = *reinterpret_cast<const bf16x8*>(st + off + i * 16 * 256);
#pragma unroll
    for (int j = 0; j < RB; ++j)
      bfr[j] = *reinterpret_cast<const bf16x8*>(st + XT * 2 + off + j * 16 * 256);
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int j = 0; j < RB; ++j) acc[i][j] = mfma16(bfr[j], xf[i], acc[i][j]);
  }
  wait_vm<0>();
  __syncthreads();
  // acc[i][j]: token 16i + l%16, ranks 16j + 4(l/16) + 0..3 → per-wave partials
  float* red = reinterpret_cast<float*>(smem);  // [4][TR][16·RB + 4]
  constexpr int RP = 16 * RB + 4;
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < RB; ++j)
      *reinterpret_cast<f32x4*>(red + (w * TR + 16 * i + (lane & 15)) * RP + 16 * j +
                                4 * (lane >> 4)) = acc[i][j];
  __syncthreads();
  for (int idx = threadIdx.x; idx < TR * 16 * RB; idx += 256) {
    const int tt = idx / (16 * RB), jj = idx % (16 * RB);
    if (tt >= rows || jj >= Rg) continue;
    const float v = red[tt * RP + jj] + red[(TR + tt) * RP + jj] + red[(2 * TR + tt) * RP + jj] +
                    red[(3 * TR + tt) * RP + jj];
    if (a.part)
      a.part[((long)blockIdx.z * a.n + t0 + tt) * a.R + j0 + jj] = v;
    else
      a.Z[(long)(t0 + tt) * a.ldz + j0 + jj] = (bf16)v;
  }
}

// Z[t, j] = bf16(sum over the K slices z, in order, of part[z][t][j]), live rows.
__global__ __launch_bounds__(256) void lora_skinny_reduce_kernel(SkinnyArgs a, int ks) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)N * a.R) return;
  const int t = (int)(idx / a.R), j = (int)(idx % a.R);
  const long plane = (long)a.n * a.R;
  float v = 0.f;
  for (int z = 0; z < ks; ++z) v += a.part[z * plane + idx];
  a.Z[(long)t * a.ldz + j] = (bf16)v;
}

template <int TT>
static hipError_t launch_skinny(const SkinnyArgs& a, int ks, hipStream_t s) {
  const dim3 grid((a.n + 16 * TT - 1) / (16 * TT), (a.R + 63) / 64, ks);
  switch ((std::min(a.R, 64) + 15) / 16) {
    case 1: hipLaunchKernelGGL((lora_skinny_kernel<TT, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((lora_skinny_kernel<TT, 2>), grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((lora_skinny_kernel<TT, 3>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((lora_skinny_kernel<TT, 4>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static int skinny_tt(const SkinnyArgs& a) { return a.K <= 8192 && a.R <= 16 ? 1 : 2; }

int lora_skinny_split(const SkinnyArgs& a) {
  if (a.part_elems <= 0 || a.R <= 0 || a.n <= 0) return 1;
  const int tr = 16 * skinny_tt(a);
  const long blocks = (long)((a.n + tr - 1) / tr) * ((a.R + 63) / 64);
  const int nc = (a.K + 127) / 128;
  // only long rows gain: with fewer than 32 chunks (4096 columns) per block
  // the second launch costs more than the slices save (C1: 2.5 → 3.3 ms per
  // cycle); then about one round of the 256 CUs, at least 8 chunks per slice
  if (blocks >= 128 || nc < 32) return 1;
  int ks = std::min((int)(256 / blocks), std::min(8, nc / 8));
  while (ks > 1 && (long)ks * a.n * a.R > a.part_elems) --ks;
  return ks >= 2 ? ks : 1;
}

hipError_t lora_skinny(const SkinnyArgs& a, hipStream_t s) {
  if (a.R <= 0 || a.n <= 0) return hipSuccess;
  // short rows at one rank group of 16: 16-token blocks (twice the blocks, two
  // per CU); wider rank groups keep 32 tokens so the B chunk is shared by two
  // token tiles
  const int ks = a.part ? lora_skinny_split(a) : 1;
  SkinnyArgs b = a;
  if (ks == 1) b.part = nullptr;
  hipError_t e = skinny_tt(a) == 1 ? launch_skinny<1>(b, ks, s) : launch_skinny<2>(b, ks, s);
  if (e != hipSuccess || ks == 1) return e;
  const long tot = (long)a.n * a.R;
  hipLaunchKernelGGL(lora_skinny_reduce_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256),
                     0, s, b, ks);
  return hipGetLastError();
}

// ------------------------------------------------------------------ TN
// work[split][c][j] = sum over the split's tokens t of X[t, c]·P[t, j].
// Block: 128 columns × one token split; token chunks of 32 stream through a
// direct-to-LDS ring of up to 80 KB (two blocks per CU, 6-8 stages): X chunk
// [32 × 128] (swizzled 256-byte rows) and P chunk [32 × R] (rows of 2R bytes). Both operands reduce over tokens, so
// both are read transposed with ds_read_b64_tr_b16 (16×16×32 pattern: lane j
// of group g points at row 8g + j/4 (+4), column c0 + 4(j%4)); wave w owns
// columns 32w .. 32w+31 (2 column tiles) × RB rank tiles.
// A launch covers up to kTnBatch passes (with one token-split count):
// grid.x runs over the (column block, rank group) blocks of every pass,
// b0[i] .. b0[i+1]-1 being those of pass i (rank group g = x / cb_i, column
// block x % cb_i); the reduction covers the passes' R·C outputs in order.
template <int RB>
__global__ __launch_bounds__(256, 2) void lora_tn_partial_kernel(TnBatch b) {
  constexpr int XT = 32 * 128, PT = 32 * 16 * RB, SE = XT + PT;
  constexpr int NS = (40 * 1024) / SE < 8 ? (40 * 1024) / SE : 8;  // SE elements = 2·SE bytes
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kTnBatch; ++i)
    if (i < b.count && (int)blockIdx.x >= b.b0[i]) pi = i;  // uniform
  const TnArgs& a = b.a[pi];
  const int bx = blockIdx.x - b.b0[pi], cbs = (a.C + 127) / 128;
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  __shared__ __attribute__((aligned(16))) bf16 smem[NS * SE];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = (bx % cbs) * 128, sp = blockIdx.y;
  int per = (N + a.nsplit - 1) / a.nsplit;
  per = (per + 31) & ~31;
  const int ta = min(N, sp * per), tb = min(N, ta + per);
  const int nk = (tb - ta + 31) / 32;
  const int cv = min(a.C - c0, 128);
  // ranks j0 .. j0 + R - 1 of this block (groups of 64)
  const int j0 = (bx / cbs) * 64, R = min(a.R - j0, 64);
  const bf16* Pg = a.P + j0;
  // P chunk loads: 32 rows × R ranks = 4·RB loads of 1 KB; wave w issues the
  // ones with index ≡ w (mod 4), so waves 0 .. RB-1 issue one each per stage.
  const bool pw = w < RB;
  // Chunk loads, set up once per block as in lora_dual: descriptors over the
  // block's rows [ta, tb) of X (columns c0 .. c0+cv) and of P, lane offsets;
  // per chunk only the row advance and, for a load with no valid row, the
  // zero page.
  const u32x4 zs = zero_rsrc();
  const u32x4 rx = make_rsrc(tb > ta ? a.X + (long)ta * a.ldx + c0 : a.X,
                             tb > ta ? (int)(((long)(tb - ta - 1) * a.ldx + cv) * 2) : 0);
  int xl[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 4 * (4 * i + w) + (lane >> 4);
    const int col = ((lane & 15) ^ aswz(r)) << 3;
    xl[i] = col < cv ? (int)(((long)r * a.ldx + col) * 2) : 0x7ff00000;
  }
  const int per_row = R / 8, prow = (w * 64 + lane) / per_row, pch = (w * 64 + lane) % per_row;
  const u32x4 rp = make_rsrc(tb > ta ? Pg + (long)ta * a.ldp : Pg,
                             tb > ta ? (int)(((long)(tb - ta - 1) * a.ldp + R) * 2) : 0);
  const int po0 = prow < 32 ? (int)(((long)prow * a.ldp + pch * 8) * 2) : 0x7ff00000;
  const unsigned lds0 = lds_addr(smem);
  auto issue = [&](int k, int slot) {
    const int rv = max(min(tb - ta - k * 32, 32), 0);  // valid rows of the chunk (uniform)
    const int xk = (int)((long)k * 32 * a.ldx * 2), pk = (int)((long)k * 32 * a.ldp * 2);
    const unsigned d = lds0 + (unsigned)(slot * SE * 2);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = 4 * (4 * i + w);
      const bool live = r0 < rv && cv > 0;
      lds_dma16(live ? rx : zs, live ? xl[i] + xk : lane * 16, d + (unsigned)(r0 * 256));
    }
    if (pw) {
      // P rows of R ranks: lane l of load w covers row (64w + l) / (R/8),
      // ranks 8·((64w + l) % (R/8))
      const bool live = w * 64 / per_row < rv;  // the wave's first row is valid
      lds_dma16(live ? rp : zs, live ? po0 + pk : lane * 16, d + (unsigned)((XT + w * 512) * 2));
    }
  };
  f32x4 acc[2][RB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < RB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // transposed-read addresses (bytes): X tile row 8g + j/4 (+4), column 32w + 16i + 4(j%4);
  // P tile row 8g + j/4 (+4), rank 16j' + 4(j%4) at a row pitch of 2R bytes
  const int g = lane >> 4, jl = lane & 15;
  const int xr = 8 * g + (jl >> 2);
  int xo[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) xo[i][h] = toff(xr + 4 * h, 32 * w + 16 * i + 4 * (jl & 3)) * 2;
  const int po = (xr * R + 4 * (jl & 3)) * 2;

  for (int k = 0; k < NS - 1; ++k) issue(k, k);
  for (int k = 0; k < nk; ++k) {
    if (pw) wait_vm<(NS - 2) * 3>(); else wait_vm<(NS - 2) * 2>();
    lds_barrier();
    issue(k + NS - 1, (k + NS - 1) % NS);
    const char* st = reinterpret_cast<const char*>(smem + (k % NS) * SE);
    bf16x8 xf[2], pf[RB];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(st + xo[i][0]));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(st + xo[i][1]));
      xf[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const char* pp = st + XT * 2 + po + j * 32;
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)pp);
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(pp + 4 * R * 2));
      pf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < RB; ++j) acc[i][j] = mfma16(pf[j], xf[i], acc[i][j]);
  }
  wait_vm<0>();
  // acc[i][j]: column c0 + 32w + 16i + l%16, ranks 16j + 4(l/16) + 0..3
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int col = c0 + 32 * w + 16 * i + (lane & 15);
    if (col >= a.C) continue;
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int jr = 16 * j + 4 * (lane >> 4);
      float* o = a.work + ((long)sp * a.C + col) * a.R + j0 + jr;
      if (jr + 3 < R) {
        *reinterpret_cast<f32x4*>(o) = acc[i][j];
      } else {
        for (int e = 0; e < 4 && jr + e < R; ++e) o[e] = acc[i][j][e];
      }
    }
  }
}

__global__ __launch_bounds__(256) void lora_tn_reduce_kernel(TnBatch b) {
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= b.r0[b.count]) return;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kTnBatch; ++i)
    if (i < b.count && idx >= b.r0[i]) pi = i;
  const TnArgs& a = b.a[pi];
  idx -= b.r0[pi];
  const int c = (int)(idx / a.R), j = (int)(idx % a.R);
  float s = 0.f;
#pragma unroll 8
  for (int sp = 0; sp < a.nsplit; ++sp) s += a.work[((long)sp * a.C + c) * a.R + j];
  s *= a.scale;
  const int grp = j / a.rg, jj = j % a.rg, rv = a.rv > 0 ? a.rv : a.rg;
  float* o = a.outs[grp];
  if (o == nullptr || jj >= rv) return;  // an untrained member; a padded rank row
  if (a.transpose_out)
    o[(long)c * rv + jj] = s;
  else
    o[(long)jj * a.C + c] = s;
}

hipError_t lora_tn_batch(const TnArgs* a, int count, hipStream_t s) {
  if (count < 1 || count > kTnBatch) return hipErrorInvalidValue;
  TnBatch b{};
  b.b0[0] = 0;
  b.r0[0] = 0;
  int rb = 1, n = 0;
  for (int i = 0; i < count; ++i) {
    const TnArgs& x = a[i];
    if (x.R <= 0 || x.C <= 0 || x.nsplit != a[0].nsplit) return hipErrorInvalidValue;
    b.a[n] = x;
    b.b0[n + 1] = b.b0[n] + ((x.C + 127) / 128) * ((x.R + 63) / 64);
    b.r0[n + 1] = b.r0[n] + (long)x.R * x.C;
    rb = std::max(rb, (std::min(x.R, 64) + 15) / 16);
    ++n;
  }
  b.count = n;
  for (int i = n; i < kTnBatch; ++i) {
    b.b0[i + 1] = b.b0[n];
    b.r0[i + 1] = b.r0[n];
  }
  const dim3 grid(b.b0[n], a[0].nsplit);
  switch (rb) {
    case 1: hipLaunchKernelGGL(lora_tn_partial_kernel<1>, grid, dim3(256), 0, s, b); break;
    case 2: hipLaunchKernelGGL(lora_tn_partial_kernel<2>, grid, dim3(256), 0, s, b); break;
    case 3: hipLaunchKernelGGL(lora_tn_partial_kernel<3>, grid, dim3(256), 0, s, b); break;
    case 4: hipLaunchKernelGGL(lora_tn_partial_kernel<4>, grid, dim3(256), 0, s, b); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long tot = b.r0[n];
  hipLaunchKernelGGL(lora_tn_reduce_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0,
                     s, b);
  return hipGetLastError();
}

hipError_t lora_tn(const TnArgs& a, hipStream_t s) {
  if (a.R <= 0 || a.C <= 0) return hipSuccess;
  return lora_tn_batch(&a, 1, s);
}

// ------------------------------------------------------------------ dual
// One pass over X = G [n, C] for both rank-r products that read it.
// Block: 512 columns (four 128-column tiles, tile q at the wave-q slot of the
// chunk) × one token split; 32-token chunks of X and P stream through a
// 4-stage direct-to-LDS ring (one barrier per chunk).
//  * TN (grad_B): wave w owns tile w (8 column tiles of 16) and accumulates
//    Pᵀ·X over the split's tokens with transposed LDS reads, as lora_tn does;
//    the fp32 partials go to workT[split][c][j].
//  * skinny (grad_Z): the chunk's two 16-token tiles go to two waves in turn
//    (token tile tt of chunk k to wave (2k + tt) % 4), each multiplying its
//    16 rows × 512 columns with the W fragments it holds in registers; the
//    fp32 partial over the block's columns goes to workY[cb][t][j].
// Two small kernels reduce the partials in a fixed order (deterministic).
// A launch covers up to 3 passes (adapters sharing ranks and token splits):
// grid.x runs over the column blocks of all of them, cb0[i] .. cb0[i+1]-1
// being those of pass i; the reductions likewise cover the passes' index
// ranges r0[i] .. r0[i+1]-1 in order.
struct DualBatch {
  DualArgs a[3];
  int count;
  int cb0[4];
  long r0[4];
};

template <int RB1, int RB2>
__global__ __launch_bounds__(256, 1) void lora_dual_kernel(DualBatch b) {
  constexpr int R1 = 16 * RB1, R2 = 16 * RB2;
  const int pi = blockIdx.x >= b.cb0[2] ? 2 : (blockIdx.x >= b.cb0[1] ? 1 : 0);  // uniform
  const DualArgs& a = b.a[pi];
  constexpr int XT = 32 * 512, PT = 32 * R1, SE = XT + PT, NS = 4;
  constexpr int LPS = 8;  // X loads per lane per chunk (+1 P load on waves < RB1)
  __shared__ __attribute__((aligned(16))) bf16 smem[NS * SE];
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cb = blockIdx.x - b.cb0[pi], c0 = cb * 512, sp = blockIdx.y;
  int per = (N + a.nsplit - 1) / a.nsplit;
  per = (per + 31) & ~31;
  const int ta = min(N, sp * per), tb = min(N, ta + per);
  const int nk = (tb - ta + 31) / 32;

  // W fragments for the block's 512 columns: k-step ks covers columns
  // c0 + 32ks .. +31; lane l holds W row 16j + l%16, columns + 8(l/16) .. +7
  bf16x8 wf[16][RB2];
  {
    const __amdgpu_buffer_rsrc_t wr =
        make_brsrc(a.W, (int)(((long)(R2 - 1) * a.ldw + a.C) * 2));
#pragma unroll
    for (int ks = 0; ks < 16; ++ks)
#pragma unroll
      for (int j = 0; j < RB2; ++j) {
        const int row = 16 * j + (lane & 15), col = c0 + 32 * ks + 8 * (lane >> 4);
        const int off = col < a.C ? (int)(((long)row * a.ldw + col) * 2) : 0x7ff00000;
        // a load with no column in range is not issued (it would complete
        // out of order with the compiler-counted loads before it)
        wf[ks][j] = c0 + 32 * ks < a.C ? __builtin_bit_cast(bf16x8, buf_load16(wr, off))
                                       : bf16x8{};
      }
  }
  const bool pw = w < RB1;
  // Chunk loads. Everything but the chunk's row offset is set up once per
  // block: one descriptor over the block's rows [ta, tb) and columns
  // [c0, c0 + 512) ∩ [0, C) (rows past tb fall outside it and load zeros),
  // the lanes' byte offsets of the 8 tile loads (load 2q + i: sub-tile q,
  // tile rows 4·(4i + w) + lane/16, chunk (lane%16) ^ f(row), as in
  // tile256.h) and of the P load. A load with no valid row or column reads
  // the zero page instead, so every load touches memory and the ring's loads
  // complete in issue order. (Computing all of this per chunk made the issue
  // of a chunk's loads take longer than streaming it.)
  const u32x4 zs = zero_rsrc();
  const int cvb = min(a.C - c0, 512);
  const u32x4 rx = make_rsrc(tb > ta ? a.X + (long)ta * a.ldx + c0 : a.X,
                             tb > ta ? (int)(((long)(tb - ta - 1) * a.ldx + cvb) * 2) : 0);
  int xl[8];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = 4 * (4 * i + w) + (lane >> 4);
      const int col = 128 * q + (((lane & 15) ^ aswz(r)) << 3);
      xl[2 * q + i] = col < cvb ? (int)(((long)r * a.ldx + col) * 2) : 0x7ff00000;
    }
  const int per_row = R1 / 8, prow = (w * 64 + lane) / per_row, pch = (w * 64 + lane) % per_row;
  const u32x4 rp = make_rsrc(tb > ta ? a.P + (long)ta * a.ldp : a.P,
                             tb > ta ? (int)(((long)(tb - ta - 1) * a.ldp + R1) * 2) : 0);
  const int po0 = prow < 32 ? (int)(((long)prow * a.ldp + pch * 8) * 2) : 0x7ff00000;
  const unsigned lds0 = lds_addr(smem);
  auto issue = [&](int k, int slot) {
    const int rv = max(min(tb - ta - k * 32, 32), 0);  // valid rows of the chunk (uniform)
    const int xk = (int)((long)k * 32 * a.ldx * 2), pk = (int)((long)k * 32 * a.ldp * 2);
    const unsigned d = lds0 + (unsigned)(slot * SE * 2);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r0 = 4 * (4 * i + w);
        const bool live = r0 < rv && 128 * q < cvb;
        lds_dma16(live ? rx : zs, live ? xl[2 * q + i] + xk : lane * 16,
                  d + (unsigned)((q * 32 * 128 + r0 * 128) * 2));
      }
    if (pw) {
      // P rows of R1 ranks: lane l of load w covers row (64w + l) / (R1/8),
      // ranks 8·((64w + l) % (R1/8))
      const bool live = w * 64 / per_row < rv;  // the wave's first row is valid
      lds_dma16(live ? rp : zs, live ? po0 + pk : lane * 16,
                d + (unsigned)((XT + w * 512) * 2));
    }
  };
  f32x4 accT[8][RB1];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < RB1; ++j) accT[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // transposed-read byte offsets (TN): X tile w, row 8g + j/4 (+4), column
  // 16i + 4(j%4); P row 8g + j/4 (+4), rank 4(j%4) at a row pitch of 2·R1 bytes
  const int g = lane >> 4, jl = lane & 15;
  const int xr = 8 * g + (jl >> 2);
  int xo[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) xo[i][h] = (w * 32 * 128 + toff(xr + 4 * h, 16 * i + 4 * (jl & 3))) * 2;
  const int po = (xr * R1 + 4 * (jl & 3)) * 2;
  // row-fragment byte offsets (skinny): row l%16 of a 16-row tile, columns 32kk + 8(l/16)
  int xs[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) xs[kk] = toff(lane & 15, 32 * kk + 8 * (lane >> 4)) * 2;
  const int ncb = (a.C + 511) / 512;
  float* workY = a.work;
  float* workT = a.work + (long)ncb * a.n_alloc * R2;

#pragma unroll
  for (int k = 0; k < NS - 1; ++k) issue(k, k);
  // Skinny partials of chunk j are stored by the waves with (w - 2j) % 4 < 2
  // (RB2 buffer stores each; rows past tb fall outside the descriptor). The
  // ring wait counts the loads of chunks k+1 .. k+NS-2 only: loads complete in
  // issue order (none is wholly out of bounds), so it holds whatever order
  // the stores complete in; a store still pending only makes it wait longer.
  const __amdgpu_buffer_rsrc_t yr =
      make_brsrc(workY + (long)cb * a.n_alloc * R2, tb * R2 * 4);
  for (int k = 0; k < nk; ++k) {
    if (pw) wait_vm<(NS - 2) * (LPS + 1)>();
    else wait_vm<(NS - 2) * LPS>();
    lds_barrier();  // chunk k visible; the slot of chunk k-1 is free
    issue(k + NS - 1, (k + NS - 1) % NS);
    const char* st = reinterpret_cast<const char*>(smem + (k % NS) * SE);
    bf16x8 pf[RB1];
#pragma unroll
    for (int j = 0; j < RB1; ++j) {
      const char* pp = st + XT * 2 + po + j * 32;
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)pp);
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(pp + 4 * R1 * 2));
      pf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(st + xo[i][0]));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(st + xo[i][1]));
      const bf16x8 xf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int j = 0; j < RB1; ++j) accT[i][j] = mfma16(pf[j], xf, accT[i][j]);
    }
    const int tt = (w - 2 * k) & 3;  // uniform
    if (tt < 2) {
      f32x4 ay[RB2];
#pragma unroll
      for (int j = 0; j < RB2; ++j) ay[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16x8 xf =
              *reinterpret_cast<const bf16x8*>(st + q * 32 * 128 * 2 + tt * 16 * 256 + xs[kk]);
#pragma unroll
          for (int j = 0; j < RB2; ++j) ay[j] = mfma16(wf[4 * q + kk][j], xf, ay[j]);
        }
      // ay[j]: token 16tt + l%16 of the chunk, ranks 16j + 4(l/16) .. +3
      const int t = ta + 32 * k + 16 * tt + (lane & 15);
#pragma unroll
      for (int j = 0; j < RB2; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ay[j]), yr,
                                               (t * R2 + 16 * j + 4 * (lane >> 4)) * 4, 0, 0);
    }
  }
  wait_vm<0>();
  // accT[i][j]: column c0 + 128w + 16i + l%16, ranks 16j + 4(l/16) .. +3
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int col = c0 + 128 * w + 16 * i + (lane & 15);
    if (col >= a.C) continue;
#pragma unroll
    for (int j = 0; j < RB1; ++j)
      *reinterpret_cast<f32x4*>(workT + ((long)sp * a.C + col) * R1 + 16 * j + 4 * (lane >> 4)) =
          accT[i][j];
  }
}

// Both reductions of lora_dual in one launch, each in a fixed order
// (deterministic). A thread handles 4 consecutive j with 16-byte partial loads;
// the first n_alloc·R2/4 threads of an entry give Y[t, j..j+3] = bf16(sum over
// the column blocks of the skinny partials) for live tokens t, the next
// C·R1/4 give out[c, j..j+3] = scale · (sum over the token splits of the TN
// partials).
__global__ __launch_bounds__(256) void lora_dual_reduce_kernel(DualBatch b) {
  long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= b.r0[b.count]) return;
  const int pi = idx >= b.r0[2] ? 2 : (idx >= b.r0[1] ? 1 : 0);
  const DualArgs& a = b.a[pi];
  idx -= b.r0[pi];
  const long ny = (long)a.n_alloc * a.R2;
  const int ncb = (a.C + 511) / 512;
  if (idx < ny / 4) {
    int N = a.n;
    if (a.n_dev) N = min(N, *a.n_dev);
    const int t = (int)(idx / (a.R2 / 4)), j = 4 * (int)(idx % (a.R2 / 4));
    if (t >= N) return;
    const float* w = a.work + (long)t * a.R2 + j;
    // partials loaded 8 at a time (loads in flight together), summed in order
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < ncb; c0 += 8) {
      f32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < ncb) v[i] = *reinterpret_cast<const f32x4*>(w + (long)(c0 + i) * ny);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < ncb) s += v[i];
    }
    bf16* y = a.Y + (long)t * a.ldy + j;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = (bf16)s[e];
    return;
  }
  const long k = idx - ny / 4;
  if (k >= (long)a.R1 * a.C / 4) return;
  const int c = (int)(k / (a.R1 / 4)), j = 4 * (int)(k % (a.R1 / 4));
  const float* wt = a.work + ny * ncb + (long)c * a.R1 + j;
  const long sstride = (long)a.C * a.R1;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int sp0 = 0; sp0 < a.nsplit; sp0 += 8) {
    f32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (sp0 + i < a.nsplit) v[i] = *reinterpret_cast<const f32x4*>(wt + (sp0 + i) * sstride);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (sp0 + i < a.nsplit) s += v[i];
  }
  const int rv = a.rv > 0 ? a.rv : a.R1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (j + e >= rv) continue;  // a padded rank row
    if (a.transpose_out)
      a.out[(long)c * rv + j + e] = s[e] * a.scale;
    else
      a.out[(long)(j + e) * a.C + c] = s[e] * a.scale;
  }
}

bool lora_dual_supported(int R1, int R2, int C) {
  return (R1 == 16 || R1 == 32) && (R2 == 16 || R2 == 32) && C % 8 == 0 && C > 0;
}

hipError_t lora_dual(const DualArgs* a, int count, hipStream_t s) {
  if (count < 1 || count > 3) return hipErrorInvalidValue;
  if (a[0].n <= 0) return hipSuccess;
  DualBatch b{};
  b.count = count;
  b.cb0[0] = 0;
  b.r0[0] = 0;
  for (int i = 0; i < count; ++i) {
    const DualArgs& x = a[i];
    if (!lora_dual_supported(x.R1, x.R2, x.C) || x.n > x.n_alloc || x.nsplit < 1 ||
        x.R1 != a[0].R1 || x.R2 != a[0].R2 || x.nsplit != a[0].nsplit || x.n != a[0].n)
      return hipErrorInvalidValue;
    b.a[i] = x;
    b.cb0[i + 1] = b.cb0[i] + (x.C + 511) / 512;
    b.r0[i + 1] = b.r0[i] + ((long)x.n_alloc * x.R2 + (long)x.R1 * x.C) / 4;
  }
  for (int i = count; i < 3; ++i) {
    b.cb0[i + 1] = b.cb0[count];
    b.r0[i + 1] = b.r0[count];
  }
  const dim3 grid(b.cb0[count], a[0].nsplit);
  const int k = (a[0].R1 / 16 - 1) * 2 + (a[0].R2 / 16 - 1);
  switch (k) {
    case 0: hipLaunchKernelGGL((lora_dual_kernel<1, 1>), grid, dim3(256), 0, s, b); break;
    case 1: hipLaunchKernelGGL((lora_dual_kernel<1, 2>), grid, dim3(256), 0, s, b); break;
    case 2: hipLaunchKernelGGL((lora_dual_kernel<2, 1>), grid, dim3(256), 0, s, b); break;
    default: hipLaunchKernelGGL((lora_dual_kernel<2, 2>), grid, dim3(256), 0, s, b); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long tot = b.r0[count];
  hipLaunchKernelGGL(lora_dual_reduce_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0,
                     s, b);
  return hipGetLastError();
}

}  // namespace dsb
