// 128-column bf16 LDS tiles (256-byte rows) shared by the attention and LoRA
// kernels: the row swizzle, direct-to-LDS tile loads, and the per-lane
// offsets of 32×32×16 row / transposed fragment reads.
#pragma once

#include "dsb_common.h"

namespace dsb {

// Chunk swizzle of a 256-byte tile row (r mod 16 → XOR mask over 16 chunks):
// conflict-free for 16- and 32-row × 16-byte fragment reads and for the
// transposed 8-byte reads (ds_read_b64_tr_b16, both the 32×32×16 and the
// 16×16×32 operand patterns), under both 128-byte and 256-byte bank windows.
// ds_read_b64_tr_b16 returns, to lane i of each 16-lane group, element i%4 of
// the 4-element pieces fetched by lanes 4k + i/4 of that group (k = 0..3).
DSB_DEV int aswz(int r) {
  return ((r & 1) << 2) ^ ((r & 2) ? 10 : 0) ^ ((r >> 2) & 1) ^ (r & 8);
}
// element offset of column `col` (multiple of 4) of row r in a swizzled tile
DSB_DEV int toff(int r, int col) {
  return r * 128 + ((((col >> 3) ^ aswz(r)) << 3) | (col & 7));
}

// Per-lane byte offsets of the fragment reads inside a tile, computed once
// per kernel (f is linear over GF(2), f(r0 + r) = f(r) for 16 | r0, and
// f(r + 8) = f(r) ^ 8):
//   row fragment kk (row l%32, chunk 2·kk + l/32):
//     (l%32)·256 + ((2kk ^ x) << 4),  x = (l/32) ^ f(l%32)
//   transposed fragment (df, hi) over the chunk at row 0 (rows rl, rl + 8;
//   rl = 4(g/2) + j/4; chunk 4·df + c, c = 2(g&1) + (j&3)/2; half j&1):
//     (rl + 8hi)·256 + 8(j&1) + (((4df ^ 8hi) ^ y) << 4),  y = c ^ f(rl)
// Row blocks of 32 rows (row fragments) and 16-row chunks (transposed) add
// compile-time multiples of 256 B, folded into the instruction offset.
struct FragOffs {
  int row[8];
  int tr[4][2];
  DSB_DEV explicit FragOffs(int lane) {
    const int lr = lane & 31, lh = lane >> 5;
    const int x = lh ^ aswz(lr);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) row[kk] = lr * 256 + (((2 * kk) ^ x) << 4);
    const int g = lane >> 4, j = lane & 15;
    const int rl = 4 * (g >> 1) + (j >> 2);
    const int y = (2 * (g & 1) + ((j & 3) >> 1)) ^ aswz(rl);
#pragma unroll
    for (int df = 0; df < 4; ++df)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
        tr[df][hi] = (rl + 8 * hi) * 256 + 8 * (j & 1) + ((((4 * df) ^ (8 * hi)) ^ y) << 4);
  }
};

// Row fragment: lane l gets columns 16·kk + 8·(l/32) .. +7 of row r0 + l%32.
DSB_DEV bf16x8 row_frag(const char* t, const FragOffs& fo, int r0, int kk) {
  return *reinterpret_cast<const bf16x8*>(t + fo.row[kk] + r0 * 256);
}
// Transposed fragment over the 16-row chunk at row `base` for columns 32·df .. +31.
DSB_DEV bf16x8 tr_frag(const char* t, const FragOffs& fo, int base, int df) {
  const bf16x4 lo =
      __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + fo.tr[df][0] + base * 256));
  const bf16x4 hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(t + fo.tr[df][1] + base * 256));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

DSB_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }  // v_exp_f32; x <= 8 here

// Direct-to-LDS tile fills (attention.hip SeqTiles, the LoRA kernels' chunk
// loads) write this layout with 256 threads: load i of wave w covers tile
// rows 4·(4i + w) .. +3, lane l filling slot l%16 of row 4·(4i + w) + l/16
// with chunk (l%16) ^ aswz(row) (aswz(r) depends only on r % 16, so all
// loads of a lane fetch the same chunk). Descriptors and lane offsets are set
// up once per block and only the row or column advance changes per load:
// building them per load costs more issue time than the load itself.

}  // namespace dsb
