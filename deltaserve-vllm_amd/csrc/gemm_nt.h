// bf16 "NT" GEMM for gfx950: C[M,N] = A[M,K1]·B[N,K1]ᵀ (+ A2[M,K2]·B2[N,K2]ᵀ)
// with a pluggable epilogue.
//
// Every dense contraction of the backward is phrased in this one form (both
// operands K-contiguous): forward recompute uses the frozen weight [out,in] as
// is, the dX products use the transposed copy made once at bind time, and the
// LoRA factor rides along as a second K segment (K-concatenation), so
// y = x·Wᵀ + (x·Aᵀ)·(s·B)ᵀ is one kernel with K = in + r.
//
// Main loop. BK = 64: each K tile is a 128-byte run of every operand row,
// fetched by direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds; 8 lanes
// cover one row, so every request is a whole 128-byte line) into one of two
// LDS stages. Each wave owns a (BM/WM)×(BN/WN) sub-tile of
// v_mfma_f32_16x16x32_bf16 accumulators, tied to their AGPRs by inline-asm
// MFMAs (with the builtin the compiler gave each MFMA's result registers
// other than its accumulator's and moved every accumulator back at the end
// of each iteration: 400 moves per K step). A K step is two 32-deep slices:
// the first half of slice 0's MFMAs carries the fragment reads of slice 1
// (one after each MFMA); then every wave's reads of stage kt have returned
// and its loads of stage kt+1 have landed, so one barrier publishes stage
// kt+1 and frees stage kt's slot; the rest of the step's MFMAs carry the
// loads of stage kt+2 into that slot (one after every other MFMA) and, in
// slice 1, the reads of slice 0 of stage kt+1. Loads get about one step of
// latency budget. Past the end of K the loads zero-fill the slot without
// touching memory, so the waits are constants.
//
// LDS layout per stage and operand: rows of 128 B (64 bf16) as eight 16-byte
// chunks; chunk c of row r sits in slot c ^ f(r), f(r) = ((r>>1)&7) ^ ((r&1)<<2),
// which makes the 16-row fragment reads (one chunk of 16 consecutive rows per
// quarter-wave) conflict-free. The loads write LDS linearly (lane i of a load
// lands at byte 16·i of its 1 KB segment = 8 rows), so the swizzle is applied
// on the global side: the lane filling slot s of row r fetches chunk s ^ f(r).
// Out-of-range rows (past M or N) and chunks past K are fetched from an offset
// outside the buffer descriptor and land as zeros.
//
// Block ids are remapped so each XCD (round-robin dispatch over 8 XCDs) gets a
// contiguous run of tiles, grouped 4 deep along M for L2 reuse.
#pragma once

#include <algorithm>
#include <type_traits>

#include "dsb_common.h"

namespace dsb {

struct GemmProblem {
  const bf16* A;
  long lda;
  const bf16* B;
  long ldb;
  const bf16* A2;  // optional second K segment (LoRA); K2 = 0 disables
  long lda2;
  const bf16* B2;
  long ldb2;
  int M, N, K1, K2;
  const int* M_dev;  // optional device-resident row count (min with M)
  // Gated-unit layout (0 = off): B (and B2) hold 2·glu_half rows, gate rows
  // then up rows. The tile's output columns are fed so that each wave's
  // first TN/2 columns are gate features f .. f+TN/2-1 and its last TN/2 the
  // up features of the same f, so an epilogue sees both halves of a feature
  // (EpiGLU). N = 2·glu_half; glu_half a multiple of BN/2.
  int glu_half = 0;
  // Split K (launch_gemm_split): block row z of the grid's y dimension
  // computes K tiles [z·kc, (z+1)·kc) of the K1+K2 range and stores its fp32
  // partial to part + z·M·N (row stride N) instead of running the epilogue;
  // gemm_split_reduce then sums the partials in order and applies it.
  float* part = nullptr;
  // Tail launch (launch_gemm_tail): the launch's block x takes tile
  // tile0 + x of the problem's tile order; with tpart set, a block stores its
  // fp32 partial as one BM × BN tile (row stride BN) at
  // tpart + (blockIdx.y · gridDim.x + blockIdx.x) · BM · BN instead of running
  // the epilogue.
  int tile0 = 0;
  float* tpart = nullptr;
  // B (and B2) stored [K, N] row-major (element (n, k) at B[k·ldb + n]): the
  // frozen weights in their native [out, in] layout as the operand of the dX
  // products, and the LoRA A factors [r, in] as their second segment, so no
  // transposed copy of either is needed.
  int b_kn = 0;
  // rows of a [K, N] B's first segment that exist (0: K1); rows from here to
  // K1 load as zeros (the LM head's last vocabulary chunk runs K to a
  // multiple of 8 past the vocabulary)
  int kb_rows = 0;
};

DSB_DEV void tile_map(int bid, int nbm, int nbn, int& pm, int& pn) {
  const int total = nbm * nbn;
  int lid = bid;
  if ((total & 7) == 0) lid = (bid & 7) * (total >> 3) + (bid >> 3);
  // 4 M-blocks per group (each XCD's 32 concurrent tiles span 4 M × 8 N
  // blocks): measured best of 2, 4, 6, 8, 16 on the C3 cycle
  constexpr int GM = 4;
  const int per_group = GM * nbn;
  const int gid = lid / per_group;
  const int first_m = gid * GM;
  const int gsz = min(nbm - first_m, GM);
  const int r = lid - gid * per_group;
  pm = first_m + r % gsz;
  pn = r / gsz;
}

// acc += A-fragment × B-fragment with the accumulator tied to its four AGPRs.
// Operands: lane l supplies row l%16 of its 16-row block with K-values
// 8·(l/16) .. +7 of the slice; lane l then holds output row l%16 of the
// A block against columns 4·(l/16) .. +3 of the B block (mfma16 with the B
// fragment first). The compiler cannot see the MFMA's latency through the
// asm: a kernel waits before reading the accumulators (mfma_drain).
DSB_DEV void mfma16_acc(f32x4& acc, bf16x8 b, bf16x8 a) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(b), "v"(a));
}
// Wait states covering the last MFMA's result (4 passes) before the
// accumulators are read.
DSB_DEV void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// buffer_load_dwordx4 ... lds with M0 set and not restored: the GEMM kernels
// issue no other instruction that reads M0 (checked on their assembly), so
// the save/restore around each load is not needed. In the main loop the M0
// write (set_m0) goes before the MFMA that precedes its load (dma16_m0), which
// covers the wait state between them; elsewhere lds_dma16_m0 does both.
// (clang warns on every use that M0 is reserved; the warning is silenced for
// these two helpers only.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
DSB_DEV void set_m0(unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %0" ::"s"(lds_addr) : "memory", "m0");
}
DSB_DEV void dma16_m0(u32x4 rsrc, int voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc) : "memory");
}
DSB_DEV void lds_dma16_m0(u32x4 rsrc, int voff, unsigned lds_addr) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(lds_addr)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// Writes 32-row block b (rows 32b .. 32b+31 of the wave tile) of the
// accumulators, row-major at `buf` (row pitch PITCH floats): acc[2b + h][fn]
// of lane l is row 16h + l%16, columns 16fn + 4(l/16) .. +3.
template <int FM, int FN, int PITCH>
DSB_DEV void stage32(const f32x4 (&acc)[FM][FN], int b, float* buf, int lane) {
  const int l16 = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
      *reinterpret_cast<f32x4*>(buf + (16 * h + l16) * PITCH + fn * 16 + 4 * lq) = acc[2 * b + h][fn];
}

// Visit the wave's accumulator tile as runs of 8 consecutive output columns
// of one row (n a multiple of 8), staged through the wave's own LDS region
// (32 rows × TN fp32, row pitch TN + 4 floats) one 32-row block at a time,
// so TN/8 consecutive lanes cover one row and every global access of the
// epilogue is a 16- or 32-byte row-contiguous transfer. Needs
// 32·(TN + 4)·4 bytes of LDS per wave at `smem`; wave-local (a wave's LDS
// accesses complete in order), so no barrier beyond the one before the
// epilogue.
template <int FM, int FN, class F>
DSB_DEV void for_each_row8(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane,
                           int wave, void* smem, F&& f) {
  constexpr int TN = FN * 16, PITCH = TN + 4, CG = TN / 8, RPI = 64 / CG;
  static_assert(64 % CG == 0 && FM % 2 == 0, "row groups");
  float* buf = reinterpret_cast<float*>(smem) + wave * 32 * PITCH;
  const int rsub = lane / CG, cg = lane % CG;
#pragma unroll
  for (int b = 0; b < FM / 2; ++b) {
    if (mw + b * 32 >= M) break;  // uniform: the rest of the wave tile is past M
    stage32<FM, FN, PITCH>(acc, b, buf, lane);
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
      const int row = it * RPI + rsub;
      const f32x4 x = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8);
      const f32x4 y = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8 + 4);
      float v[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
      const int m = mw + b * 32 + row;
      if (m < M) f(m, nw + cg * 8, v);
    }
  }
}

// for_each_row8 for epilogues that also read global memory per output chunk
// (a residual, or the fp32 output they accumulate into): `load(m, n)` issues
// that read for the chunk (row m, columns n .. n+7) and `f(m, n, v, x)` gets
// its result x. The reads of the 32-row block two ahead are issued before
// the current block is staged and stored, three blocks in registers, so their
// latency is spent under the epilogue's other work instead of stalling every
// row (reading them in `f` left one global-load latency per 4 rows; one block
// ahead left the SwiGLU backward 13 µs slower per launch at C3).
template <int FM, int FN, class L, class F>
DSB_DEV void for_each_row8_pf(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane,
                              int wave, void* smem, L&& load, F&& f) {
  constexpr int TN = FN * 16, PITCH = TN + 4, CG = TN / 8, RPI = 64 / CG, IT = 32 / RPI;
  static_assert(64 % CG == 0 && FM % 2 == 0, "row groups");
  using T = decltype(load(0, 0));
  float* buf = reinterpret_cast<float*>(smem) + wave * 32 * PITCH;
  const int rsub = lane / CG, cg = lane % CG;
  // loads run PD blocks ahead of their use (three blocks spill at 256 × 256)
  constexpr int PD = 2;
  T pf[PD + 1][IT];
  auto issue = [&](int b, T (&dst)[IT]) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int m = mw + b * 32 + it * RPI + rsub;
      dst[it] = m < M ? load(m, nw + cg * 8) : T{};
    }
  };
#pragma unroll
  for (int b = 0; b < PD && b < FM / 2; ++b)
    if (mw + b * 32 < M) issue(b, pf[b]);
#pragma unroll
  for (int b = 0; b < FM / 2; ++b) {
    if (mw + b * 32 >= M) break;  // uniform: the rest of the wave tile is past M
    if (b + PD < FM / 2 && mw + (b + PD) * 32 < M) issue(b + PD, pf[(b + PD) % (PD + 1)]);
    stage32<FM, FN, PITCH>(acc, b, buf, lane);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int row = it * RPI + rsub;
      const f32x4 x = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8);
      const f32x4 y = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8 + 4);
      float v[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
      const int m = mw + b * 32 + row;
      if (m < M) f(m, nw + cg * 8, v, pf[b % (PD + 1)][it]);
    }
  }
}

// for_each_row8_pf for a wave tile whose rows are all below M and whose
// columns the caller has checked: no per-row or per-block tests, so the
// code between the loads and their use is straight-line and the compiler's
// memory-counter waits count exactly how many loads and stores were issued
// after the one a chunk needs. (With the tests, each row's loads and stores
// sit behind an exec-mask branch and the compiler, unable to count across
// them, waits for every outstanding access before each row of the first two
// blocks, the previous row's stores included.)
template <int FM, int FN, class L, class F>
DSB_DEV void for_each_row8_pf_full(const f32x4 (&acc)[FM][FN], int mw, int nw, int lane,
                                   int wave, void* smem, L&& load, F&& f) {
  constexpr int TN = FN * 16, PITCH = TN + 4, CG = TN / 8, RPI = 64 / CG, IT = 32 / RPI;
  static_assert(64 % CG == 0 && FM % 2 == 0, "row groups");
  using T = decltype(load(0, 0));
  float* buf = reinterpret_cast<float*>(smem) + wave * 32 * PITCH;
  const int rsub = lane / CG, cg = lane % CG, n = nw + cg * 8;
  constexpr int PD = 2;
  T pf[PD + 1][IT];
#pragma unroll
  for (int b = 0; b < PD && b < FM / 2; ++b)
#pragma unroll
    for (int it = 0; it < IT; ++it) pf[b][it] = load(mw + b * 32 + it * RPI + rsub, n);
#pragma unroll
  for (int b = 0; b < FM / 2; ++b) {
    if (b + PD < FM / 2) {
#pragma unroll
      for (int it = 0; it < IT; ++it)
        pf[(b + PD) % (PD + 1)][it] = load(mw + (b + PD) * 32 + it * RPI + rsub, n);
    }
    stage32<FM, FN, PITCH>(acc, b, buf, lane);
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int row = it * RPI + rsub;
      const f32x4 x = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8);
      const f32x4 y = *reinterpret_cast<const f32x4*>(buf + row * PITCH + cg * 8 + 4);
      float v[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
      f(mw + b * 32 + row, n, v, pf[b % (PD + 1)][it]);
    }
  }
}

// 8 values to bf16 at p[0 .. min(8, lim)); 16-byte store when whole and aligned.
// The 16-byte store is non-temporal: the outputs of a whole wave of tiles land
// at once, and streaming them keeps them from evicting the A/B panels the
// next tiles read from L2.
DSB_DEV void store8_bf16(bf16* p, const float* v, int lim) {
  if (lim >= 8 && ((unsigned long)p & 15) == 0) {
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (bf16)v[i];
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), reinterpret_cast<u32x4*>(p));
  } else {
    for (int i = 0; i < 8 && i < lim; ++i) p[i] = (bf16)v[i];
  }
}
// v[i] += bf16 r[i] for i < min(8, lim)
DSB_DEV void add8_bf16(float* v, const bf16* r, int lim) {
  if (lim >= 8 && ((unsigned long)r & 15) == 0) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(r);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] += (float)x[i];
  } else {
    for (int i = 0; i < 8 && i < lim; ++i) v[i] += (float)r[i];
  }
}

// Slot of 16-byte chunk c of LDS row r (rows of 128 B = 8 chunks): c ^ f(r).
// Any 8 consecutive rows (one 128-byte bank window per row) and any 16
// consecutive rows (256-byte windows, rows r and r^1 in different halves)
// hit distinct banks for a fixed logical chunk.
DSB_DEV int lds_swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

// The fp32 partial-sum epilogue of a split-K block (defined below), named
// through a dependent type so the kernel template can use it before then.
struct EpiF32;
struct EpiBF16;
struct EpiSwiGLUBwd;
template <class E>
struct SplitPart {
  using type = EpiF32;
  static constexpr bool enabled = std::is_same<E, EpiBF16>::value ||
                                  std::is_same<E, EpiF32>::value ||
                                  std::is_same<E, EpiSwiGLUBwd>::value;
};

// Swizzle of a [K, N]-layout B stage (rows of BN·2 bytes = CPR 16-byte
// chunks): chunk c of row k sits in slot c ^ fkn(k). A transposed B fragment
// read covers, per 16-lane group g, rows 8g + 0..3 (+4) at two adjacent
// chunks; fkn spreads those 4 rows over 8 distinct chunk pairs and separates
// groups 2h and 2h+1 (bit 3), so a 16- or 32-lane phase is conflict-free.
template <int CPR>
DSB_DEV int fkn(int k) {
  return ((2 * (k & 3)) ^ (((k >> 3) & 1) << 3)) & (CPR - 1);
}

template <int BM, int BN, int WM, int WN, class Epi, bool KN = false>
__global__ __launch_bounds__(WM* WN * 64)
__attribute__((amdgpu_waves_per_eu(WM* WN / 4, WM* WN / 4))) void gemm_nt_kernel(GemmProblem p, Epi epi) {
  constexpr int BK = 64;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  // direct-to-LDS loads per lane per stage: one load = 64 lanes × 16 B = 8 rows
  constexpr int IA = BM / (8 * NW), IB = BN / (8 * NW), IAB = IA + IB;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be 32-aligned");
  static_assert(IA >= 1 && IB >= 1 && BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "loader split");
  static_assert(NW % 2 == 0, "row-block parity is the wave's");
  static_assert(IAB < 64, "vmcnt range");
  // LDS: two A slots, then three B slots (elements). A K tile is loaded one
  // step ahead of its use, the B tile two: B is the operand every XCD fetches
  // (A's row panels are the XCD's own), so its loads miss L2 more often and
  // get the longer lead.
  constexpr int SA = BM * BK, SB = BN * BK;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * SA + 3 * SB];

  int M = p.M;
  if (p.M_dev) M = min(M, *p.M_dev);
  const int nbm = (p.M + BM - 1) / BM, nbn = (p.N + BN - 1) / BN;
  int pm, pn;
  tile_map(blockIdx.x + p.tile0, nbm, nbn, pm, pn);
  const int m0 = pm * BM, n0 = pn * BN;
  if (m0 >= M) return;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int nk1 = (p.K1 + BK - 1) / BK;
  const int nk2 = p.K2 > 0 ? (p.K2 + BK - 1) / BK : 0;
  const int nk = nk1 + nk2;
  // this block's K tiles (all of them unless K is split over the grid's y)
  const int kc = (nk + (int)gridDim.y - 1) / (int)gridDim.y;
  const int kt0 = min(nk, (int)blockIdx.y * kc), kt1 = min(nk, kt0 + kc);

  // Loader geometry: lane fills slot (lane & 7) of row (lane >> 3) of its
  // 8-row block; block b = wave + j·NW starts at row 8b, whose bit 3 is the
  // wave's parity (NW even), so the fetched chunk is the same for every load.
  const int lrow = lane >> 3;
  const int lch = (lane & 7) ^ lds_swz(lrow + 8 * (wave & 1));
  const int rowsA = min(M - m0, BM), rowsB = min(p.N - n0, BN);
  // One descriptor per operand and K segment, over the tile's rows that
  // exist: rows past M (N) and chunks past K (offset OR-ed with OOB) fall
  // outside it and load as zeros, and nothing outside the operand is read.
  auto rsrc = [](const bf16* base, long ld, int rows, int K) {
    const int bytes = rows > 0 && K > 0 ? (int)((((long)(rows - 1) * ld) + K) * 2) : 0;
    return make_rsrc(base, bytes);
  };
  const int K2 = nk2 ? p.K2 : 0;
  const bool glu = p.glu_half > 0;
  // B rows of the tile: rows n0 .. n0+BN-1, or for the gated layout the
  // gate/up row runs of the tile's BN/2 features (descriptor over all rows)
  const long bbase = glu ? 0 : n0;
  const int brows = glu ? p.N : rowsB;
  const u32x4 dA1 = rsrc(p.A + (long)m0 * p.lda, p.lda, rowsA, p.K1);
  const u32x4 dA2 = rsrc(nk2 ? p.A2 + (long)m0 * p.lda2 : p.A, p.lda2, rowsA, K2);
  const u32x4 dB1 = rsrc(p.B + bbase * p.ldb, p.ldb, brows, p.K1);
  const u32x4 dB2 = rsrc(nk2 ? p.B2 + bbase * p.ldb2 : p.B, p.ldb2, brows, K2);
  // [K, N] B: one descriptor per K tile, over the tile's rows that exist
  // (k0 .. min(k0 + BK, K) - 1) × the tile's live columns. The row advance
  // is in the descriptor's base rather than in the load's scalar offset,
  // which the hardware's range check does not include: rows past K fall
  // outside the descriptor by their lane offset alone. Columns past N are
  // forced out by their (constant) lane offset.
  const int kbr1 = p.kb_rows > 0 ? min(p.kb_rows, p.K1) : p.K1;
  auto kn_rsrc = [&](bool s1, int k0) {
    const int rows = min((s1 ? kbr1 : K2) - k0, BK);
    if (rows <= 0) return make_rsrc(p.B, 0);
    const long ld = s1 ? p.ldb : p.ldb2;
    return make_rsrc((s1 ? p.B : p.B2) + n0 + (long)k0 * ld,
                     (int)(((long)(rows - 1) * ld + rowsB) * 2));
  };
  // lane byte offset of its first row; A load j adds j·8·NW rows, B load j
  // starts at row brow0(j) of the descriptor (uniform)
  const int rw = 8 * wave + lrow;
  const int voA1 = (rw * (int)p.lda + lch * 8) * 2, voB1 = (lrow * (int)p.ldb + lch * 8) * 2;
  const int voA2 = (rw * (int)p.lda2 + lch * 8) * 2, voB2 = (lrow * (int)p.ldb2 + lch * 8) * 2;
  const int stA1 = 16 * NW * (int)p.lda;  // bytes per 8·NW rows
  const int stA2 = 16 * NW * (int)p.lda2;
  auto brow0 = [&](int jb) {
    const int r = 8 * (wave + jb * NW);  // LDS row of the block
    if (!glu) return r;
    constexpr int HF = TN / 2;                // features per wave column
    const int wcol = r / TN, c = r % TN;      // wave column, column within it
    const int f = pn * (BN / 2) + wcol * HF + (c % HF);
    return c < HF ? f : p.glu_half + f;
  };
  int boff1[IB], boff2[IB];
#pragma unroll
  for (int jb = 0; jb < IB; ++jb) {
    boff1[jb] = brow0(jb) * (int)p.ldb * 2;
    boff2[jb] = brow0(jb) * (int)p.ldb2 * 2;
  }
  // OR-ed into the offset of chunks past K: beyond any descriptor, loads zero
  constexpr int OOB = 0x7ff00000;
  // [K, N] B loads: load jb of this wave fills LDS rows RPL·(wave + jb·NW)
  // .. +RPL-1 of the stage (rows of BN·2 bytes, CPR chunks each); lane l
  // fills slot l % CPR of row l / CPR with chunk slot ^ fkn(row)
  constexpr int CPR = BN / 8, RPL = 64 / CPR;
  int vkn1[KN ? IB : 1], vkn2[KN ? IB : 1];
  if constexpr (KN) {
#pragma unroll
    for (int jb = 0; jb < IB; ++jb) {
      const int r = RPL * (wave + jb * NW) + lane / CPR;
      const int c = (lane % CPR) ^ fkn<CPR>(r);
      const int out = n0 + 8 * c < p.N ? 0 : OOB;
      vkn1[jb] = (r * (int)p.ldb + 8 * c) * 2 | out;
      vkn2[jb] = (r * (int)p.ldb2 + 8 * c) * 2 | out;
    }
  }
  const unsigned lds0 = lds_addr(smem);

  // Loads of K tile kt into stage slot `slot`, issued one at a time by
  // issue_one(j) so they can be spread over a run of MFMAs. Tiles past the
  // end (kt >= nk) fall past K of the second segment and fill the slot with
  // zeros without touching memory.
  // A fill of K tile ktA into A slot sa and of K tile ktB into B slot sb;
  // dstB is biased by −SA elements, so B row offsets keep the SA of the
  // fragment-read layout (brow, btr).
  struct Fill {
    u32x4 dA, dB;
    int voA, voB, stA;
    bool s1B;
    unsigned dstA, dstB;
  };
  auto a_slot = [&](int sa) { return lds0 + (unsigned)(sa * SA * 2) + (unsigned)(8 * wave * BK * 2); };
  auto b_slot = [&](int sb) {
    return lds0 + (unsigned)((SA + sb * SB) * 2) + (unsigned)(8 * wave * BK * 2);
  };
  auto make_fill = [&](int ktA, int sa, int ktB, int sb) {
    Fill f;
    {
      const bool s1 = ktA < nk1;
      const int k0 = s1 ? ktA * BK : (ktA - nk1) * BK;
      const int kb = (k0 * 2) | ((k0 + lch * 8 < (s1 ? p.K1 : K2)) ? 0 : OOB);
      f.dA = s1 ? dA1 : dA2;
      f.voA = (s1 ? voA1 : voA2) + kb;
      f.stA = s1 ? stA1 : stA2;
    }
    {
      const bool s1 = ktB < nk1;
      const int k0 = s1 ? ktB * BK : (ktB - nk1) * BK;
      const int kb = (k0 * 2) | ((k0 + lch * 8 < (s1 ? p.K1 : K2)) ? 0 : OOB);
      if constexpr (KN)
        f.dB = kn_rsrc(s1, k0);
      else
        f.dB = s1 ? dB1 : dB2;
      f.voB = (s1 ? voB1 : voB2) + kb;
      f.s1B = s1;
    }
    f.dstA = a_slot(sa);
    f.dstB = b_slot(sb);
    return f;
  };
  auto issue_one = [&](const Fill& f, int j) {
    if (j < IA) {
      lds_dma16_m0(f.dA, f.voA + j * f.stA, f.dstA + j * 8 * NW * BK * 2);
    } else if constexpr (KN) {
      set_m0(f.dstB + (SA + (j - IA) * 8 * NW * BK) * 2);
      asm volatile("s_nop 0" ::: "memory");
      dma16_m0(f.dB, f.s1B ? vkn1[j - IA] : vkn2[j - IA]);
    } else {
      lds_dma16_m0(f.dB, f.voB + (f.s1B ? boff1[j - IA] : boff2[j - IA]),
                   f.dstB + (SA + (j - IA) * 8 * NW * BK) * 2);
    }
  };
  // the same load split around an MFMA: M0 before it, the load after it
  auto pre_one = [&](const Fill& f, int j) {
    set_m0(j < IA ? f.dstA + j * 8 * NW * BK * 2 : f.dstB + (SA + (j - IA) * 8 * NW * BK) * 2);
  };
  auto go_one = [&](const Fill& f, int j) {
    if (j < IA)
      dma16_m0(f.dA, f.voA + j * f.stA);
    else if constexpr (KN)
      dma16_m0(f.dB, f.s1B ? vkn1[j - IA] : vkn2[j - IA]);
    else
      dma16_m0(f.dB, f.voB + (f.s1B ? boff1[j - IA] : boff2[j - IA]));
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  const int l16 = lane & 15, lq = lane >> 4;
  // Fragment rows are 16 apart, so the swizzle depends on l16 only. Slice s
  // of the stage (K 32s .. 32s+31) is chunk 4s + lq of the lane's row.
  const int g = lds_swz(l16);
  const int arow = (wm * TM + l16) * BK, brow = SA + (wn * TN + l16) * BK;
  bf16x8 af[2][FM], bfr[2][KN ? 1 : FN];
  // [K, N] B fragments as their two 4-deep halves, each read on its own
  bf16x4 bkn[2][KN ? FN : 1][2];
  // [K, N] B fragment fn of slice s: two transposed 8-byte reads. Lane j of
  // 16-lane group q points at row 32s + 8q + j/4 (then 4 rows on), columns
  // 16fn + 4(j%4) .. +3 of the wave's tile; ds_read_b64_tr_b16 hands lane j
  // the element j%4 of the pieces of lanes 4k + j/4, i.e. column j at the
  // group's 4 rows, which is the MFMA's K order. fkn(row) depends on
  // row % 16 only, the same for both reads.
  int btr[KN ? FN : 1];
  if constexpr (KN) {
    const int rq = 8 * lq + l16 / 4;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int c = (wn * TN + fn * 16 + 4 * (l16 & 3)) / 8;
      btr[fn] = (SA + rq * BN + ((c ^ fkn<CPR>(rq)) << 3) + 4 * (l16 & 1)) * 2;
    }
  }
  // Read i of slice s into buffer `buf`: A fragment i (i < FM), else B
  // fragment i - FM, or with a [K, N] B half (i - FM) % 2 of B fragment
  // (i - FM) / 2 (one LDS instruction per read, so a read fits between two
  // MFMAs).
  // ba: the A slot; bb: the B slot's base less SA elements (brow and btr
  // include SA)
  auto read_one = [&](const bf16* ba, const bf16* bb, int s, int buf, int i) {
    const int ch = ((4 * s + lq) ^ g) << 3;
    if (i < FM) {
      af[buf][i] = *reinterpret_cast<const bf16x8*>(ba + arow + ch + i * 16 * BK);
    } else if constexpr (KN) {
      const int fn = (i - FM) >> 1, h = (i - FM) & 1;
      const char* t = reinterpret_cast<const char*>(bb) + btr[fn] + 32 * s * BN * 2 + h * 4 * BN * 2;
      bkn[buf][fn][h] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)t);
    } else {
      bfr[buf][i - FM] = *reinterpret_cast<const bf16x8*>(bb + brow + ch + (i - FM) * 16 * BK);
    }
  };
  auto a_base = [&](int sa) { return (const bf16*)smem + sa * SA; };
  auto b_base = [&](int sb) { return (const bf16*)smem + SA + sb * SB; };
  constexpr int NM = FM * FN, NR = FM + (KN ? 2 : 1) * FN, H1 = IAB / 2;
  auto bfrag = [&](int buf, int fn) {
    if constexpr (KN)
      return __builtin_shufflevector(bkn[buf][fn][0], bkn[buf][fn][1], 0, 1, 2, 3, 4, 5, 6, 7);
    else
      return bfr[buf][fn];
  };
  // MFMAs t0 .. t1-1 of the slice held in `buf`, with other instructions
  // between them: first the fragment reads 0 .. nr-1 of slice ns of the
  // stage at nb (into buffer nbuf), one after each MFMA, then loads
  // j0 .. j0+nj-1 of f, one after every third MFMA (its M0 write before that
  // MFMA). A wave issues at most one instruction every few cycles, so a burst
  // of other instructions between MFMAs would leave the matrix pipe idle
  // (loads after every MFMA, or every other one, measured slower).
  auto mma = [&](int buf, int t0, int t1, const bf16* nba, const bf16* nbb, int ns, int nbuf,
                 int nr, const Fill& f, int j0, int nj) {
    int r = 0, j = 0;
#pragma unroll
    for (int t = t0; t < t1; ++t) {
      const int fm = t / FN, fn = t % FN;
      const bool ld = r >= nr && j < nj && t % 3 == 2;
      if (ld) {
        __builtin_amdgcn_sched_barrier(0);
        pre_one(f, j0 + j);
        __builtin_amdgcn_sched_barrier(0);
      }
      mfma16_acc(acc[fm][fn], bfrag(buf, fn), af[buf][fm]);
      if (r < nr) {
        __builtin_amdgcn_sched_barrier(0);
        read_one(nba, nbb, ns, nbuf, r++);
        __builtin_amdgcn_sched_barrier(0);
      } else if (ld) {
        __builtin_amdgcn_sched_barrier(0);
        go_one(f, j0 + j++);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int rr = 0; rr < NR; ++rr)
      if (rr >= r && rr < nr) read_one(nba, nbb, ns, nbuf, rr);
#pragma unroll
    for (int jj = 0; jj < IAB; ++jj)
      if (jj >= j && jj < nj) issue_one(f, j0 + jj);
  };
  // Loads of K tiles ktA, ktB (both < nk1, first segment): the descriptors
  // and row offsets are the loop-invariant ones of segment 1.
  auto make_fill1 = [&](int ktA, int sa, int ktB, int sb) {
    Fill f;
    const int k0a = ktA * BK, k0b = ktB * BK;
    f.dA = dA1;
    if constexpr (KN)
      f.dB = kn_rsrc(true, k0b);
    else
      f.dB = dB1;
    f.voA = voA1 + ((k0a * 2) | ((k0a + lch * 8 < p.K1) ? 0 : OOB));
    f.voB = voB1 + ((k0b * 2) | ((k0b + lch * 8 < p.K1) ? 0 : OOB));
    f.stA = stA1;
    f.s1B = true;
    f.dstA = a_slot(sa);
    f.dstB = b_slot(sb);
    return f;
  };

  // Prologue: tile kt0 loaded and published, slice 0 of it read, and in
  // flight, in this order: A and B of tile kt0+1, then B of tile kt0+2.
  {
    const Fill f = make_fill(kt0, 0, kt0, 0);
#pragma unroll
    for (int j = 0; j < IAB; ++j) issue_one(f, j);
  }
  wait_vm<0>();
  lds_barrier();
#pragma unroll
  for (int i = 0; i < NR; ++i) read_one(a_base(0), b_base(0), 0, 0, i);
  {
    const Fill f = make_fill(kt0 + 1, 1, kt0 + 1, 1);
#pragma unroll
    for (int j = 0; j < IAB; ++j) issue_one(f, j);
    const Fill fb = make_fill(kt0 + 1, 1, kt0 + 2, 2);
#pragma unroll
    for (int j = IA; j < IAB; ++j) issue_one(fb, j);
  }

  // Step kt computes on A slot (kt−kt0)&1 and B slot (kt−kt0)%3 (fragments of
  // slice 0 already in buffer 0). Its mid-step wait leaves in flight only the
  // B loads of tile kt+2 (issued last, in the step before): A and B of tile
  // kt+1 have landed. After that barrier its slots are free, and it issues A
  // of tile kt+2 and then B of tile kt+3 into them.
  auto step = [&](int kt, auto&& mk) {
    const int ca = (kt - kt0) & 1, cb = (kt - kt0) % 3;
    const bf16* ba = a_base(ca);
    const bf16* bb = b_base(cb);
    const Fill next = mk(kt + 2, ca, kt + 3, cb);
    __builtin_amdgcn_sched_barrier(0);
    mma(0, 0, NM / 2, ba, bb, 1, 1, NR, next, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    wait_vm<IB>();
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    mma(0, NM / 2, NM, ba, bb, 1, 1, 0, next, 0, H1);
    __builtin_amdgcn_sched_barrier(0);
    mma(1, 0, NM, a_base(ca ^ 1), b_base(cb == 2 ? 0 : cb + 1), 0, 0, NR, next, H1, IAB - H1);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Steps whose prefetches (A tile kt+2, B tile kt+3) stay in segment 1 use
  // the invariant segment-1 fill; the last few steps select the segment per
  // tile. (Tiles past this block's range that the last steps prefetch are
  // other blocks' tiles or zero fills past K: loaded, never multiplied.)
  const int nfast = max(kt0, min(kt1, nk1 - 3));
  int kt = kt0;
  for (; kt < nfast; ++kt) step(kt, make_fill1);
  for (; kt < kt1; ++kt) step(kt, make_fill);
  mfma_drain();
  // the last step's loads land before the epilogue reuses the LDS
  wait_vm<0>();
  lds_barrier();

  if constexpr (SplitPart<Epi>::enabled) {
    if (p.part) {
      const typename SplitPart<Epi>::type ep{p.part + (long)blockIdx.y * p.M * p.N, (long)p.N,
                                             p.N, 0};
      ep.template run<FM, FN, WM, WN>(acc, m0 + wm * TM, n0 + wn * TN, M, lane, wave,
                                      (void*)smem);
      return;
    }
    if (p.tpart) {
      // tile-local partial: base shifted so that global (m, n) lands at
      // (m − m0)·BN + (n − n0) of the block's tile
      const long blk = (long)blockIdx.y * gridDim.x + blockIdx.x;
      const typename SplitPart<Epi>::type ep{
          p.tpart + blk * (BM * BN) - ((long)m0 * BN + n0), (long)BN, p.N, 0};
      ep.template run<FM, FN, WM, WN>(acc, m0 + wm * TM, n0 + wn * TN, M, lane, wave,
                                      (void*)smem);
      return;
    }
  }
  {
    epi.template run<FM, FN, WM, WN>(acc, m0 + wm * TM, n0 + wn * TN, M, lane, wave,
                                     (void*)smem);
  }
}

// ---------------------------------------------------------------- epilogues

// C = acc (+ R), bf16 out. R (optional) is a bf16 residual of the same shape.
struct EpiBF16 {
  bf16* C;
  long ldc;
  int N;
  const bf16* R;
  long ldr;
  // the epilogue of one 8-column chunk (split-K reduction)
  DSB_DEV void apply8(int m, int n, float* v) const {
    const int lim = N - n;
    if (lim <= 0) return;
    if (R) add8_bf16(v, R + (long)m * ldr + n, lim);
    store8_bf16(C + (long)m * ldc + n, v, lim);
  }
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    if (!R) {
      for_each_row8(acc, mw, nw, M, lane, wave, smem, [&](int m, int n, float* v) {
        const int lim = N - n;
        if (lim <= 0) return;
        store8_bf16(C + (long)m * ldc + n, v, lim);
      });
      return;
    }
    if (mw + FM * 16 <= M && nw + FN * 16 <= N && ldr % 8 == 0 && ldc % 8 == 0 &&
        ((((unsigned long)R) | ((unsigned long)C)) & 15) == 0) {
      // every chunk whole and aligned
      for_each_row8_pf_full(
          acc, mw, nw, lane, wave, smem,
          [&](int m, int n) { return ldg128_nt(R + (long)m * ldr + n); },
          [&](int m, int n, float* v, const u32x4& r) {
            float rf[8];
            unpack8(r, rf);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] += rf[i];
            __builtin_nontemporal_store(pack8(v), reinterpret_cast<u32x4*>(C + (long)m * ldc + n));
          });
      return;
    }
    // residual rows read ahead (whole aligned chunks; others read in place)
    auto whole = [&](int m, int n) {
      return N - n >= 8 && (((unsigned long)(R + (long)m * ldr + n)) & 15) == 0;
    };
    for_each_row8_pf(
        acc, mw, nw, M, lane, wave, smem,
        [&](int m, int n) { return whole(m, n) ? ldg128_nt(R + (long)m * ldr + n) : u32x4{}; },
        [&](int m, int n, float* v, const u32x4& r) {
          const int lim = N - n;
          if (lim <= 0) return;
          if (whole(m, n)) {
            float rf[8];
            unpack8(r, rf);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] += rf[i];
          } else {
            add8_bf16(v, R + (long)m * ldr + n, lim);
          }
          store8_bf16(C + (long)m * ldc + n, v, lim);
        });
  }
};

// Gated unit (GemmProblem::glu_half = I): the wave's first TN/2 columns are
// gate features f .. f+TN/2-1, the last TN/2 the up features of the same f.
// Writes gate and up (bf16, as EpiBF16 would: GU[m, f] and GU[m, I + f]) and,
// when H is set, H[m, f] = bf16(silu(gate)·up) from the bf16-rounded halves.
struct EpiGLU {
  bf16* GU;
  long ldgu;
  bf16* H;
  long ldh;
  int I;
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    constexpr int TN = FN * 16, HF = TN / 2, PITCH = TN + 4, CG = HF / 8, RPI = 64 / CG;
    static_assert(FN % 2 == 0 && FM % 2 == 0 && 64 % CG == 0, "gate/up halves of the wave tile");
    float* buf = reinterpret_cast<float*>(smem) + wave * 32 * PITCH;
    const int rsub = lane / CG, cg = lane % CG;
    // nw = n0 + wn·TN is the tile's output column base; the features start at
    // (n0 / BN)·(BN / 2) + wn·HF, i.e. nw / 2
    const int f0 = nw / 2;
#pragma unroll
    for (int bk = 0; bk < FM / 2; ++bk) {
      if (mw + bk * 32 >= M) break;
      stage32<FM, FN, PITCH>(acc, bk, buf, lane);
#pragma unroll
      for (int it = 0; it < 32 / RPI; ++it) {
        const int row = it * RPI + rsub;
        const int m = mw + bk * 32 + row;
        const float* gp = buf + row * PITCH + cg * 8;
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(gp);
        const f32x4 g1 = *reinterpret_cast<const f32x4*>(gp + 4);
        const f32x4 u0 = *reinterpret_cast<const f32x4*>(gp + HF);
        const f32x4 u1 = *reinterpret_cast<const f32x4*>(gp + HF + 4);
        if (m >= M) continue;
        float gv[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
        float uv[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
        const int f = f0 + cg * 8;
        const u32x4 gb = pack8(gv), ub = pack8(uv);
        stg128(GU + (long)m * ldgu + f, gb);
        stg128(GU + (long)m * ldgu + I + f, ub);
        if (H) {
          float gr[8], ur[8], o[8];
          unpack8(gb, gr);
          unpack8(ub, ur);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = gr[e] * sigmoid(gr[e]) * ur[e];
          stg128(H + (long)m * ldh + f, pack8(o));
        }
      }
    }
  }
};

// SwiGLU backward in the epilogue of the product whose output is the gradient
// wrt h = silu(gate)·up (ffn.py:40-45; the GEMM's N is I): from the bf16
// rounding of each output value and the bf16 gate and up features GU[m, f],
// GU[m, I + f] it writes d_gate to G[m, f] and d_up to G[m, I + f] (bf16),
// so the [n, I] gradient itself never reaches memory. The gradient is rounded
// to bf16 first, as the reference's bf16 matmul output is. I, ldgu, ldg
// multiples of 8 and GU, G 16-byte aligned (whole 8-feature chunks).
struct EpiSwiGLUBwd {
  const bf16* GU;
  long ldgu;
  bf16* G;
  long ldg;
  int I;
  struct Chunk {
    u32x4 g, u;
  };
  DSB_DEV Chunk load(int m, int n) const {
    const bf16* p = GU + (long)m * ldgu + n;
    return Chunk{ldg128_nt(p), ldg128_nt(p + I)};
  }
  DSB_DEV void finish(int m, int n, const float* v, const Chunk& c) const {
    float d[8], g[8], u[8], og[8], ou[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = (float)(bf16)v[i];
    unpack8(c.g, g);
    unpack8(c.u, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float sg = sigmoid(g[e]);  // σ(gate)
      og[e] = d[e] * u[e] * (sg * (1.f + g[e] * (1.f - sg)));
      ou[e] = d[e] * (g[e] * sg);
    }
    // streamed past the caches, as store8_bf16 does
    bf16* o = G + (long)m * ldg + n;
    __builtin_nontemporal_store(pack8(og), reinterpret_cast<u32x4*>(o));
    __builtin_nontemporal_store(pack8(ou), reinterpret_cast<u32x4*>(o + I));
  }
  // the epilogue of one 8-column chunk (split-K reduction)
  DSB_DEV void apply8(int m, int n, float* v) const {
    if (n < I) finish(m, n, v, load(m, n));
  }
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    if (mw + FM * 16 <= M && nw + FN * 16 <= I) {
      for_each_row8_pf_full(
          acc, mw, nw, lane, wave, smem, [&](int m, int n) { return load(m, n); },
          [&](int m, int n, float* v, const Chunk& c) { finish(m, n, v, c); });
      return;
    }
    for_each_row8_pf(
        acc, mw, nw, M, lane, wave, smem,
        [&](int m, int n) { return n < I ? load(m, n) : Chunk{}; },
        [&](int m, int n, float* v, const Chunk& c) {
          if (n < I) finish(m, n, v, c);
        });
  }
};

// C (+)= acc, fp32 out.
struct EpiF32 {
  float* C;
  long ldc;
  int N;
  int accumulate;
  // accumulate with a per-row factor on what C holds: C = C·rowscale[m] + acc
  // (the LM head's dH across vocabulary chunks, rescaled to the row's running
  // softmax reference); null: factor 1
  const float* rowscale = nullptr;
  DSB_DEV void apply8(int m, int n, const float* v) const {
    const int lim = N - n;
    float* c = C + (long)m * ldc + n;
    const float sc = rowscale ? rowscale[m] : 1.f;
    for (int i = 0; i < 8 && i < lim; ++i) c[i] = accumulate ? c[i] * sc + v[i] : v[i];
  }
  template <int FM, int FN, int WM, int WN>
  DSB_DEV void run(const f32x4 (&acc)[FM][FN], int mw, int nw, int M, int lane, int wave,
                   void* smem) const {
    auto whole = [&](int m, int n) {
      return N - n >= 8 && (((unsigned long)(C + (long)m * ldc + n)) & 15) == 0;
    };
    if (!accumulate) {
      for_each_row8(acc, mw, nw, M, lane, wave, smem, [&](int m, int n, float* v) {
        const int lim = N - n;
        if (lim <= 0) return;
        float* c = C + (long)m * ldc + n;
        if (whole(m, n)) {
          *reinterpret_cast<f32x4*>(c) = f32x4{v[0], v[1], v[2], v[3]};
          *reinterpret_cast<f32x4*>(c + 4) = f32x4{v[4], v[5], v[6], v[7]};
        } else {
          for (int i = 0; i < 8 && i < lim; ++i) c[i] = v[i];
        }
      });
      return;
    }
    // the fp32 values accumulated into, read ahead as for a residual
    struct F8 {
      f32x4 a, b;
    };
    if (mw + FM * 16 <= M && nw + FN * 16 <= N && ldc % 4 == 0 &&
        (((unsigned long)C) & 15) == 0) {
      // every chunk whole and aligned; the row factor read with the chunk
      // (the pointer test outside the walk keeps its body branch-free)
      struct F8s {
        f32x4 a, b;
        float s;
      };
      auto walk = [&](auto scaled) {
        for_each_row8_pf_full(
            acc, mw, nw, lane, wave, smem,
            [&](int m, int n) {
              const float* c = C + (long)m * ldc + n;
              return F8s{*reinterpret_cast<const f32x4*>(c),
                         *reinterpret_cast<const f32x4*>(c + 4),
                         decltype(scaled)::value ? rowscale[m] : 1.f};
            },
            [&](int m, int n, float* v, const F8s& x) {
              float* c = C + (long)m * ldc + n;
              *reinterpret_cast<f32x4*>(c) = f32x4{v[0], v[1], v[2], v[3]} + x.a * x.s;
              *reinterpret_cast<f32x4*>(c + 4) = f32x4{v[4], v[5], v[6], v[7]} + x.b * x.s;
            });
      };
      if (rowscale)
        walk(std::true_type{});
      else
        walk(std::false_type{});
      return;
    }
    for_each_row8_pf(
        acc, mw, nw, M, lane, wave, smem,
        [&](int m, int n) {
          if (!whole(m, n)) return F8{};
          const float* c = C + (long)m * ldc + n;
          return F8{*reinterpret_cast<const f32x4*>(c), *reinterpret_cast<const f32x4*>(c + 4)};
        },
        [&](int m, int n, float* v, const F8& x) {
          const int lim = N - n;
          if (lim <= 0) return;
          float* c = C + (long)m * ldc + n;
          const float sc = rowscale ? rowscale[m] : 1.f;
          if (whole(m, n)) {
            *reinterpret_cast<f32x4*>(c) = f32x4{v[0], v[1], v[2], v[3]} + x.a * sc;
            *reinterpret_cast<f32x4*>(c + 4) = f32x4{v[4], v[5], v[6], v[7]} + x.b * sc;
          } else {
            for (int i = 0; i < 8 && i < lim; ++i) c[i] = c[i] * sc + v[i];
          }
        });
  }
};

// Tile configurations. Big: 256×256, 4 waves of 128×128 (256 accumulators per
// lane). Mid: 128×128, 4 waves of 64×64. Skinny: 64×64, 4 waves of 32×32.
enum GemmCfg { GEMM_BIG = 0, GEMM_MID = 1, GEMM_SKINNY = 2 };

// Sum of the split-K partials of p (in split order, so the result does not
// depend on scheduling) through epi.apply8, 8 columns per thread, live rows
// only. N must be a multiple of 8.
template <class Epi>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(GemmProblem p, int ks, Epi epi) {
  int M = p.M;
  if (p.M_dev) M = min(M, *p.M_dev);
  const int n8 = p.N / 8;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  const int m = (int)(idx / n8), n = (int)(idx % n8) * 8;
  if (m >= M) return;
  const long plane = (long)p.M * p.N;
  const float* src = p.part + (long)m * p.N + n;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < ks; ++z) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(src + z * plane);
    const f32x4 b = *reinterpret_cast<const f32x4*>(src + z * plane + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] += a[i];
      v[4 + i] += b[i];
    }
  }
  epi.apply8(m, n, v);
}

template <int BM, int BN, int WM, int WN, class Epi>
hipError_t launch_gemm_cfg(const GemmProblem& p, const Epi& e, hipStream_t s, int ks = 1) {
  const int nbm = (p.M + BM - 1) / BM, nbn = (p.N + BN - 1) / BN;
  if (nbm == 0 || nbn == 0) return hipSuccess;
  const dim3 grid(nbm * nbn, ks);
  if (p.b_kn)
    hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, WM, WN, Epi, true>), grid, dim3(WM * WN * 64), 0,
                       s, p, e);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, WM, WN, Epi, false>), grid, dim3(WM * WN * 64),
                       0, s, p, e);
  return hipGetLastError();
}

inline GemmCfg pick_gemm_cfg(int M, int N) {
  if (N <= 64) return GEMM_SKINNY;
  const long big_tiles = (long)((M + 255) / 256) * ((N + 255) / 256);
  if (big_tiles >= 192) return GEMM_BIG;
  // One 256-row block (a serving-size cycle): the product streams its
  // weights, and 128-wide tiles only fetch each weight panel twice (once per
  // 128-row half); from 64 tiles up the 256-wide tile streams faster (M = 256,
  // K = 5120: N = 17408 97 µs against 120, N = 34816 140 against 227).
  if (M <= 256 && big_tiles >= 64) return GEMM_BIG;
  return GEMM_MID;
}

template <class Epi>
hipError_t launch_gemm(const GemmProblem& p, const Epi& e, hipStream_t s, int cfg = -1) {
  if (cfg < 0) cfg = pick_gemm_cfg(p.M, p.N);
  if constexpr (std::is_same<Epi, EpiGLU>::value) {
    // the gated layout needs two 32-column fragments per wave half
    if (cfg == GEMM_BIG && p.glu_half % 128 == 0) return launch_gemm_cfg<256, 256, 2, 2>(p, e, s);
    if (p.glu_half % 64 != 0) return hipErrorInvalidValue;
    return launch_gemm_cfg<128, 128, 2, 2>(p, e, s);
  } else {
    switch (cfg) {
      case GEMM_BIG: return launch_gemm_cfg<256, 256, 2, 2>(p, e, s);
      case GEMM_MID: return launch_gemm_cfg<128, 128, 2, 2>(p, e, s);
      default: return launch_gemm_cfg<64, 64, 2, 2>(p, e, s);
    }
  }
}

// K split over the grid's y dimension for problems with too few 256×256
// tiles to fill the chip: `ks` blocks per tile each store the fp32 partial
// of a slice of K to p.part ([ks, M, N]), then one reduction launch sums them
// and applies the epilogue (those with apply8: EpiBF16, EpiF32, EpiSwiGLUBwd);
// N a multiple of 8.
// Splits so the tiles × splits blocks fit one round of the 256 CUs (a second,
// partly filled round costs more than it spreads), at least 4 K tiles each;
// 1 when the problem has more than 128 tiles (the fp32 partials' traffic
// would buy no more parallelism).
// The split's tile: 128 × 128 for one 256-row block over K ≤ 8192 when those
// tiles stay within 128 (a serving-size cycle's K = 5120–7168 products: the
// smaller tiles need fewer K slices to fill the CUs, so less partial traffic;
// M = 256, N = 5120, K = 5120: 32 µs against 37), else 256 × 256.
inline int gemm_split_tile(int M, int N, int K) {
  const long mid = (long)((M + 127) / 128) * ((N + 127) / 128);
  return M <= 256 && K <= 8192 && mid <= 128 ? 128 : 256;
}
inline int gemm_split_count(int M, int N, int K) {
  const int t = gemm_split_tile(M, N, K);
  const long tiles = (long)((M + t - 1) / t) * ((N + t - 1) / t);
  const int nk = (K + 63) / 64;
  if (tiles > 128 || N % 8 != 0 || nk < 8) return 1;
  const int ks = std::min((int)(256 / tiles), std::min(8, nk / 4));
  return ks >= 2 ? ks : 1;
}
template <class Epi>
hipError_t launch_gemm_split(const GemmProblem& p, const Epi& e, int ks, hipStream_t s) {
  static_assert(SplitPart<Epi>::enabled, "split-K epilogues");
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (!p.part || p.N % 8 != 0 || ks < 2) return hipErrorInvalidValue;
  const hipError_t e0 = gemm_split_tile(p.M, p.N, p.K1 + p.K2) == 128
                           ? launch_gemm_cfg<128, 128, 2, 2>(p, e, s, ks)
                           : launch_gemm_cfg<256, 256, 2, 2>(p, e, s, ks);
  if (e0 != hipSuccess) return e0;
  const long n = (long)p.M * (p.N / 8);
  hipLaunchKernelGGL(gemm_split_reduce_kernel<Epi>, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, s, p, ks, e);
  return hipGetLastError();
}

// Sum of the tail launch's tile-local partials (launch_gemm_tail) in split
// order through epi.apply8: 32 blocks per tail tile, one 8-column chunk of
// the 256 × 256 tile per thread; live rows and columns only.
template <class Epi>
__global__ __launch_bounds__(256) void gemm_tail_reduce_kernel(GemmProblem p, int ks, int ntail,
                                                               Epi epi) {
  int M = p.M;
  if (p.M_dev) M = min(M, *p.M_dev);
  const int t = blockIdx.x >> 5;                            // tail tile
  const int c = ((blockIdx.x & 31) << 8) + threadIdx.x;     // chunk within the tile
  const int row = c >> 5, col = (c & 31) << 3;
  const int nbm = (p.M + 255) / 256, nbn = (p.N + 255) / 256;
  int pm, pn;
  tile_map(p.tile0 + t, nbm, nbn, pm, pn);
  const int m = pm * 256 + row, n = pn * 256 + col;
  if (m >= M || n >= p.N) return;
  const float* src = p.tpart + (long)t * 65536 + row * 256 + col;
  const long plane = (long)ntail * 65536;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < ks; ++z) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(src + z * plane);
    const f32x4 b = *reinterpret_cast<const f32x4*>(src + z * plane + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] += a[i];
      v[4 + i] += b[i];
    }
  }
  epi.apply8(m, n, v);
}

// Wave-quantisation tail: a problem whose 256 × 256 tiles fill whole rounds
// of the ncu CUs plus a partial one of `tail` ≤ ncu/2 tiles. The full rounds
// run as one launch; the tail tiles then split K over ks blocks each
// (ks·tail ≤ ncu, at least 16 K tiles per block: with fewer, the partial
// stores and the reduction cost more than the idle CUs), store fp32 tile
// partials, and a reduction applies the epilogue, so the last round takes
// about 1/ks of a tile's time instead of a whole one. Returns ks (1: no tail
// split) and the tail tile count.
inline int gemm_tail_split(int M, int N, int K, int ncu, int* tail) {
  const long tiles = (long)((M + 255) / 256) * ((N + 255) / 256);
  const int nk = (K + 63) / 64;
  *tail = ncu > 0 ? (int)(tiles % ncu) : 0;
  if (ncu <= 0 || ncu % 8 || tiles <= ncu || *tail == 0 || N % 8 != 0 || nk < 8) return 1;
  const int ks = std::min(ncu / *tail, std::min(8, nk / 16));
  return ks >= 2 ? ks : 1;
}
// tpart holds ks · tail · 65536 floats.
template <class Epi>
hipError_t launch_gemm_tail(const GemmProblem& p, const Epi& e, int ks, int tail, float* tpart,
                            hipStream_t s) {
  static_assert(SplitPart<Epi>::enabled, "tail-split epilogues");
  const int nbm = (p.M + 255) / 256, nbn = (p.N + 255) / 256;
  const int full = nbm * nbn - tail;
  // full is a whole number of rounds of a CU count that is a multiple of 8,
  // so the tail launch's block x lands on the XCD that tile_map assumes
  if (!tpart || tail <= 0 || full <= 0 || full % 8 || ks < 2 || p.N % 8 || p.part)
    return hipErrorInvalidValue;
  const dim3 blk(256);
  if (p.b_kn)
    hipLaunchKernelGGL((gemm_nt_kernel<256, 256, 2, 2, Epi, true>), dim3(full), blk, 0, s, p, e);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<256, 256, 2, 2, Epi, false>), dim3(full), blk, 0, s, p, e);
  GemmProblem q = p;
  q.tile0 = full;
  q.tpart = tpart;
  if (p.b_kn)
    hipLaunchKernelGGL((gemm_nt_kernel<256, 256, 2, 2, Epi, true>), dim3(tail, ks), blk, 0, s, q,
                       e);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<256, 256, 2, 2, Epi, false>), dim3(tail, ks), blk, 0, s,
                       q, e);
  hipLaunchKernelGGL(gemm_tail_reduce_kernel<Epi>, dim3(tail * 32), dim3(256), 0, s, q, ks, tail,
                     e);
  return hipGetLastError();
}

}  // namespace dsb
