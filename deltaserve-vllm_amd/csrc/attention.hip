// Packed varlen causal GQA attention on gfx950 MFMA, head_dim 128 or 64:
// forward recompute (ctx, optional fp32 ctx copy, row log-sum-exp) and the
// FA2-style backward: a dsum = rowsum(dO∘O) pass, then two passes that do
// not depend on each other (the cycle runs them concurrently): dQ (forward
// and dQ blocks: 4 waves of 32 queries sharing one kv head, see q_block) and
// dK/dV (one block per 128 keys of one kv head, summing its q-head group in
// registers, no atomics). Softmax statistics, P and dS stay fp32 in
// registers; P and dS are rounded to bf16 only as MFMA operands.
//
// head_dim 64 runs the head_dim-128 kernels on heads zero-padded to 128 inside
// the loads (dims past a.hd load as zeros, so they add nothing to Q·Kᵀ, dO·Vᵀ
// or dsum, and come out of P·V, dS·K, dSᵀ·Q and Pᵀ·dO as zeros that the
// stores skip), scaled by a.scale = 1/sqrt(head_dim).
//
// Semantics: deltaserve-plugin/deltaserve/bwd_services/common/attention.py
//   attn_forward_core   :20-45   (scale 1/sqrt(Hd), causal mask, fp32 softmax)
//   attn_backward_core  :48-112  (dS = P∘(dP − rowsum(dP∘P)), GQA group sums)
// rowsum(dP∘P) is computed as rowsum(dO∘O) with O from the forward: in the
// backward cycle as ctx + bf16(O − ctx), the bf16 rounding residual the
// forward writes next to ctx (about 16 significant bits, half the bytes of an
// fp32 copy); at op level as the fp32 copy the caller passes, else the bf16 ctx.
// The reference fills masked scores with −1e9 before the softmax; exp of that
// underflows to exactly 0, so skipping masked pairs is the same arithmetic.
//
// Data movement. The streamed operand (K and V in the forward and dQ passes,
// Q and dO in the dK/dV pass) moves in 64-row × 128-column tiles through a
// two-stage LDS ring filled by direct-to-LDS loads, one tile pair ahead of
// the MFMAs; rows past the sequence end load as zeros. Tiles keep their
// natural [row][dim] layout (rows of 256 B, 16-byte chunk c of row r stored
// in slot c ^ f(r)). Products that reduce over the streamed rows need that
// operand transposed; it is read with ds_read_b64_tr_b16, which returns, to
// lane i of each 16-lane group, element i%4 of the 4-element pieces fetched
// by lanes 4k + i/4 (k = 0..3). Pointing lane j of group g at row
// base + 4·(g/2) + j/4, column d0 + 16·(g%2) + 4·(j%4) therefore hands lane l
// rows base + 4·(l/32) + k of column d0 + l%32: the MFMA operand for 8 rows
// {base + 4·(l/32) + 0..3, base + 8 + 4·(l/32) + 0..3}, which is exactly the
// row set a 32×32 accumulator fragment holds for its 16-row chunk, so P and
// dS feed the next product straight from registers.
//
// MFMA convention (mfma32(X, Y)): lane l supplies row l%32 of X and of Y with
// 8 K-values each; the result lane l holds Y-row l%32 against X-rows
// 8(r/4) + 4(l/32) + r%4, r = 0..15.
#include "kernels.h"
#include "tile256.h"

namespace dsb {

namespace {
constexpr int HD = 128;             // head width the kernels compute on
constexpr int TR = 64;             // rows per streamed tile
constexpr int TILE = TR * HD;      // elements per tile (16 KB)
constexpr float kLog2e = 1.4426950408889634f;
// OR-ed into the lane offset of a chunk past the head width: beyond any
// descriptor (num_records < 2^31), so it loads zeros
constexpr unsigned kPastHead = 0x80000000u;

// Direct-to-LDS loads of one sequence's 64-row × 128-column tiles of a
// [rows, ld] operand, set up once per block: one descriptor over the
// sequence's rows (rows from L on fall outside it and load zeros; the
// kernels wait for all their loads at once, so the loads' completion order
// does not matter) and the lane's byte offset. The tile layout is the one
// row_frag / tr_frag read (tile256.h: chunk c of row r in slot c ^ aswz(r)).
// The four loads a wave issues per tile (tile rows 4·(4i + w) + lane/16,
// i = 0..3) share the lane's chunk, since aswz(r) depends only on r modulo
// 16, so load i is the lane's first offset plus 16·i rows. Setting up a
// descriptor and lane offsets per load (a lane-to-scalar move for every
// descriptor word) made the loads' issue a large share of each tile step.
struct SeqTiles {
  u32x4 rs;
  unsigned off0;  // bytes: row 4w + lane/16, the lane's chunk (| kPastHead past hd)
  int ldb;        // row stride in bytes
  DSB_DEV SeqTiles(const bf16* mat, long ld, int st, int L, int wave, int lane, int hd) {
    rs = make_rsrc(mat + (long)st * ld, (int)((long)max(L, 0) * ld * 2));
    const int r = 4 * wave + (lane >> 4);
    const int c = (lane & 15) ^ aswz(r);
    off0 = (unsigned)(((long)r * ld + (c << 3)) * 2) | (8 * c < hd ? 0u : kPastHead);
    ldb = (int)(ld * 2);
  }
  // tile rows t0 .. t0+63, columns col0 .. col0+127, to the tile at LDS byte
  // address `tile`
  DSB_DEV void load(int t0, int col0, unsigned tile, int wave) const {
    const unsigned base = (unsigned)(t0 * ldb + col0 * 2);
#pragma unroll
    for (int i = 0; i < TR / 16; ++i)
      lds_dma16(rs, (int)(off0 + base + (unsigned)(16 * i * ldb)),
                tile + (unsigned)((4 * (4 * i + wave)) * 256));
  }
};

// Ring prologue of the K/V stream (forward and dQ passes): key tiles 0 and 1
// (when there are two) go to the two stages at once, so the second tile's
// latency runs beside the first's instead of after it. The loop then issues
// tile t+1 at step t from t = 1 on, into the stage tile t−1 has freed. At the
// short sequences of a packed cycle most blocks stream only a few tiles, so
// the prologue's exposed latency is a large share of a block.
DSB_DEV void load_first_two(const SeqTiles& tk, const SeqTiles& tv, int nt, int col0,
                            unsigned lds0, int wave) {
  tk.load(0, col0, lds0, wave);
  tv.load(0, col0, lds0 + TILE * 2, wave);
  if (nt > 1) {
    tk.load(TR, col0, lds0 + 2 * TILE * 2, wave);
    tv.load(TR, col0, lds0 + 3 * TILE * 2, wave);
  }
}

// Row fragments of one global row (lane's row, 8 × 16 columns) straight to
// registers; columns from hd on (and rows that are not ok) are zeros.
DSB_DEV void load_row_frags(const bf16* base, long ld, long row, int col0, bool ok, int lh,
                            int hd, bf16x8 (&f)[8]) {
  const bf16* p = base + (ok ? row * ld + col0 : 0L);
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    f[kk] = kk * 16 < hd ? *reinterpret_cast<const bf16x8*>(p + kk * 16 + lh * 8) : bf16x8{};
    if (!ok) f[kk] = bf16x8{};
  }
}

// An empty volatile asm in a wave-uniform branch: the compiler may not
// execute it speculatively, so the branch stays a branch instead of being
// flattened into selects that every tile would pay for (the masks below).
DSB_DEV void keep_branch() { asm volatile(""); }

// An empty volatile asm that takes x as an operand: x is computed before it,
// and volatile asm statements keep their order, so a value pinned between two
// inline-asm MFMAs is computed there. Without it the compiler sinks softmax
// arithmetic whose results are only used later past the following branch,
// out of the MFMA phase it was interleaved with.
DSB_DEV void pin(float& x) { asm volatile("" : "+v"(x)); }

// Query-side block layout (forward and dQ passes). A 128-row tile of the
// table holds 4 subtiles of 32 queries; with G = Hq / Hkv q-heads per kv
// head its 4·G (subtile, head) pairs are taken subtile-major, heaviest
// subtile first, one per wave and four per block: G blocks per tile and kv
// head (grid x = tiles·G, y = kv heads). The waves of a block share the kv
// head's K/V stream; for G = 4 they also share the subtile, so all four
// attend the same keys and none idles at the block's barriers while another
// finishes its diagonal tiles.
struct QBlock {
  int st, L;   // sequence start row and length
  int q0, h;   // the wave's first query row (in the sequence) and q-head
  int nt;      // key tiles the block streams
  int nt_w;    // key tiles the wave attends (0 if it has no query)
  bool empty;  // no wave of the block has a query (block-uniform)
};
// Workgroups go to the 8 XCDs round robin by linear id. The kernels take
// their (tile index, kv head) from the linear id with the kv head varying
// fastest (grid.y = Hkv): with 8 kv heads every XCD, and its L2, serves one
// kv head, whose streamed tiles (K/V in the forward and dQ passes, its
// q-heads' Q/dO in the dK/dV pass) its blocks share, and consecutive tile
// indices (the heaviest-first order) still start first.
struct XcdPos {
  int x, kvh;
};
DSB_DEV XcdPos xcd_pos(int hkv) {
  const int lin = (int)(blockIdx.x + gridDim.x * blockIdx.y);
  return XcdPos{lin / hkv, lin % hkv};
}

DSB_DEV QBlock q_block(const AttnArgs& a, int w) {
  const int G = a.Hq / a.Hkv;
  const XcdPos xp = xcd_pos(a.Hkv);
  const int tile = xp.x / G, b = xp.x - tile * G;
  QBlock r{};
  r.empty = tile >= *a.ntiles_dev;
  if (r.empty) return r;
  const int4 tl = a.tiles[tile];
  r.st = tl.x;
  r.L = tl.y;
  const int p = 4 * b + w;
  r.q0 = tl.z + 32 * (3 - p / G);
  r.h = xp.kvh * G + p % G;
  r.empty = tl.z + 32 * (3 - (4 * b + 3) / G) >= r.L;  // the block's lightest subtile
  const int q_end = min(r.L, tl.z + 32 * (4 - (4 * b) / G));
  r.nt = (q_end + TR - 1) / TR;
  r.nt_w = r.q0 < r.L ? min(r.nt, (r.q0 + 31) / TR + 1) : 0;
  return r;
}

// acc += mfma(a, b) with the accumulator held in AGPRs (inline asm): the
// dK/dV pass keeps its 128 long-lived accumulators there, while this
// translation unit is compiled with MFMA results in VGPRs
// (-amdgpu-mfma-vgpr-form), so the S/dP scores the softmax reads need no
// AGPR-to-VGPR copies. The leading s_nop gives the VALU writes of a and b
// (the bf16 packs of P and dS) their wait states before the MFMA reads them;
// accumulations into one register tuple are at least 8 MFMAs apart.
DSB_DEV void mfma32_acc(f32x16& acc, bf16x8 a, bf16x8 b) {
  asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Store a wave's 32 rows × 128 columns, held in the 32×32 accumulator layout
// (lane l: row l%32, columns 32·d4 + 8·(e/4) + 4·(l/32) + e%4 of acc[d4][e]),
// as bf16(scale·x) through the wave's LDS region `buf` (32 rows at a pitch of
// kRowPitch elements): the lanes write their pieces there, then read back 16
// contiguous bytes each and store whole 256-byte rows, four rows per store
// instruction (storing the 8-byte pieces directly scatters every instruction
// over 32 rows). Rows r >= nvalid and columns from ncol on are not stored.
// With `res`, the bf16 rounding residual bf16(x − bf16(x)) goes to res (same
// row stride) after.
constexpr int kRowPitch = 136;  // 272 bytes: rows 16 apart share LDS banks, at most 2-way
DSB_DEV void store_rows32(const f32x16 (&acc)[4], float scale, bf16* buf, bf16* out, long ld,
                          int nvalid, int ncol, int lane, bf16* res = nullptr) {
  const int lr = lane & 31, lh = lane >> 5;
  for (int pass = 0; pass < (res ? 2 : 1); ++pass) {
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float x = acc[d4][4 * g + t] * scale;
          const bf16 b = (bf16)x;
          v[t] = pass == 0 ? b : (bf16)(x - (float)b);
        }
        *reinterpret_cast<bf16x4*>(buf + lr * kRowPitch + d4 * 32 + 8 * g + 4 * lh) = v;
      }
    bf16* dst = pass == 0 ? out : res;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = lane + 64 * i, r = c >> 4, col = (c & 15) * 8;
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(buf + r * kRowPitch + col);
      if (r < nvalid && col < ncol) *reinterpret_cast<bf16x8*>(dst + (long)r * ld + col) = v;
    }
  }
}

DSB_DEV bf16x8 pack_chunk(const f32x16& s, int c) {
  bf16x8 b;
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = (bf16)s[8 * c + e];
  return b;
}
}  // namespace

// ---------------------------------------------------------------- forward
// Block: 4 waves × 32 queries (q_block layout) of one kv head's q-heads;
// streams the kv head's K/V tiles. LDS: 2 stages × (K tile + V tile) = 64 KB
// → 2 blocks per CU.
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(AttnArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, lh = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const QBlock qb = q_block(a, w);
  if (qb.empty) return;
  const int kvh = qb.h / (a.Hq / a.Hkv), h = qb.h, st = qb.st, L = qb.L;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * 2 * TILE];
  const int qpos = qb.q0 + lr;
  const bool qok = qpos < L;

  const int hd = a.hd;
  bf16x8 qf[8];
  load_row_frags(a.q, a.ldq, st + qpos, h * hd, qok, lh, hd, qf);

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_i = -INFINITY, l_i = 0.f;
  const float sl2 = a.scale * kLog2e;
  const int nt = qb.nt;

  const FragOffs fo(lane);
  const SeqTiles tk(a.k, a.ldk, st, L, w, lane, hd), tv(a.v, a.ldv, st, L, w, lane, hd);
  const unsigned lds0 = lds_addr(smem);
  load_first_two(tk, tv, qb.nt, kvh * hd, lds0, w);
  // The wave computes the tiles with a key at or before its last query
  // (t < nt_w); after those it only takes part in the block's loads and
  // barriers. Two loops, so the compute loop has no skip path (a skip path
  // makes the compiler copy the accumulators on every iteration).
  const int nt_w = qb.nt_w;
  auto advance = [&](int t) {
    wait_vm<0>();
    lds_barrier();  // tile t landed for every wave; stage (t+1)&1 is free
    if (t >= 1 && t + 1 < nt) {  // tiles 0 and 1 came with the prologue
      const unsigned nxt = lds0 + (unsigned)(((t + 1) & 1) * 2 * TILE * 2);
      tk.load((t + 1) * TR, kvh * hd, nxt, w);
      tv.load((t + 1) * TR, kvh * hd, nxt + TILE * 2, w);
    }
  };
  for (int t = 0; t < nt_w; ++t) {
    const int k0 = t * TR;
    const char* sK = reinterpret_cast<const char*>(smem + (t & 1) * 2 * TILE);
    const char* sV = sK + TILE * 2;
    advance(t);

    // S = Q·Kᵀ for the two 32-key halves, their MFMA chains alternating
    // (step i: half i%2, dim chunk i/2); each K fragment read runs four steps
    // ahead of its MFMA (sched_barrier pins the order) so LDS latency hides
    // under the MFMAs.
    f32x16 s[2] = {};
    {
      bf16x8 kfr[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) kfr[i] = row_frag(sK, fo, (i & 1) * 32, i >> 1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        if (i + 4 < 16) kfr[i + 4] = row_frag(sK, fo, ((i + 4) & 1) * 32, (i + 4) >> 1);
        __builtin_amdgcn_sched_barrier(0);
        s[i & 1] = mfma32(kfr[i], qf[i >> 1], s[i & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // scores stay unscaled until the exponent: max(s)·c = max(s·c) for c > 0,
    // and exp2(s·c − m) is one fma + exp
    // causal / length mask, only on tiles that reach past this wave's first
    // query or past the sequence end (wave-uniform)
    if (k0 + TR - 1 > qb.q0 || k0 + TR > L) {
      keep_branch();
      const int lim = min(qpos, L - 1) - k0 - 4 * lh;  // key offset limit of this lane's rows
#pragma unroll
      for (int kf = 0; kf < 2; ++kf)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kf * 32 + 8 * (r >> 2) + (r & 3) > lim) s[kf][r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kf][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * sl2;
    // Lazy rescale: the running max m_i only moves when some row's tile max
    // exceeds it by more than 8 (log2 units); otherwise p = exp2(s − m_i) <= 256,
    // exact after the final 1/l normalisation.
    if (__any(mx > m_i + 8.f)) {
      const float m_new = fmaxf(m_i, mx);
      const float alpha = m_i == -INFINITY ? 0.f : fast_exp2(m_i - m_new);
      l_i *= alpha;
#pragma unroll
      for (int df = 0; df < 4; ++df)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[df][r] *= alpha;
      m_i = m_new;
    }
    const float m_use = m_i == -INFINITY ? 0.f : m_i;
    float rs4[4] = {0.f, 0.f, 0.f, 0.f};  // four partial sums: no serial add chain
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(s[kf][r], sl2, -m_use));
        s[kf][r] = p;
        rs4[r & 3] += p;
      }
    float rs = (rs4[0] + rs4[1]) + (rs4[2] + rs4[3]);
    rs += __shfl_xor(rs, 32, 64);
    l_i += rs;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      bf16x8 vfr[4];
#pragma unroll
      for (int df = 0; df < 4; ++df) vfr[df] = tr_frag(sV, fo, kc * 16, df);
      const bf16x8 pb = pack_chunk(s[kc >> 1], kc & 1);
#pragma unroll
      for (int df = 0; df < 4; ++df) o[df] = mfma32(vfr[df], pb, o[df]);
    }
  }
  for (int t = nt_w; t < nt; ++t) advance(t);

  if (!a.o32) {
    // ctx and its rounding residual as whole rows through the stages, which
    // every wave is done reading
    __syncthreads();
    if (nt_w > 0) {
      const long r0 = (long)(st + qb.q0) * a.ldc + h * hd;
      store_rows32(o, 1.f / l_i, smem + w * 32 * kRowPitch, a.ctx + r0, a.ldc, L - qb.q0, hd,
                   lane,
                   a.ores ? a.ores + r0 : nullptr);
    }
    if (qok && lh == 0) a.lse[(long)h * a.ld_stat + st + qpos] = m_i + log2f(l_i);
    return;
  }
  if (qok) {
    const float inv_l = 1.f / l_i;
    const long row = st + qpos;
#pragma unroll
    for (int df = 0; df < 4; ++df)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dim = df * 32 + 8 * g + 4 * lh;
        if (dim >= hd) continue;
        bf16x4 ob;
        f32x4 of;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          of[t] = o[df][4 * g + t] * inv_l;
          ob[t] = (bf16)of[t];
        }
        *reinterpret_cast<bf16x4*>(a.ctx + row * a.ldc + h * hd + dim) = ob;
        if (a.o32) *reinterpret_cast<f32x4*>(a.o32 + row * a.ldo32 + h * hd + dim) = of;
        if (a.ores) {
          bf16x4 rb;
#pragma unroll
          for (int t = 0; t < 4; ++t) rb[t] = (bf16)(of[t] - (float)ob[t]);
          *reinterpret_cast<bf16x4*>(a.ores + row * a.ldc + h * hd + dim) = rb;
        }
      }
    if (lh == 0) a.lse[(long)h * a.ld_stat + row] = m_i + log2f(l_i);
  }
}

// ---------------------------------------------------------------- dsum
// dsum[h, row] = rowsum(dO∘O) over head h's dims, for every live row and
// q-head: O is ctx + its rounding residual (or the fp32 copy when the forward
// wrote one, else the bf16 ctx). A thread takes 8 dims of two rows (its six
// 16-byte loads issued before any use); the hd/8 threads of a (row, head) are
// consecutive lanes and reduce by shuffles. The dQ and dK/dV passes read it,
// so they do not depend on each other.
constexpr int kDsumRows = 2;
__global__ __launch_bounds__(256) void attn_dsum_kernel(AttnArgs a) {
  const int n = a.n_dev ? min(a.n, *a.n_dev) : a.n;
  const int per_row = a.Hq * a.hd / 8, gw = a.hd / 8;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const long m0 = g / per_row * kDsumRows;
  // a (row, head) group's lanes share m0, so groups leave whole
  if (m0 >= n) return;
  const int d0 = (int)(g % per_row) * 8;
  float acc[kDsumRows];
  if (a.o32) {
#pragma unroll
    for (int i = 0; i < kDsumRows; ++i) {
      const long m = min(m0 + i, (long)n - 1);
      float dv[8];
      unpack8(ldg128(a.dout + m * a.lddo + d0), dv);
      const f32x4 o0 = *reinterpret_cast<const f32x4*>(a.o32 + m * a.ldo32 + d0);
      const f32x4 o1 = *reinterpret_cast<const f32x4*>(a.o32 + m * a.ldo32 + d0 + 4);
      acc[i] = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i] += dv[e] * o0[e] + dv[4 + e] * o1[e];
    }
  } else {
    u32x4 xd[kDsumRows], xc[kDsumRows], xr[kDsumRows];
#pragma unroll
    for (int i = 0; i < kDsumRows; ++i) {
      const long m = min(m0 + i, (long)n - 1);  // a last odd row repeats, unstored
      xd[i] = ldg128(a.dout + m * a.lddo + d0);
      xc[i] = ldg128(a.ctx + m * a.ldc + d0);
      xr[i] = a.ores ? ldg128(a.ores + m * a.ldc + d0) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < kDsumRows; ++i) {
      float dv[8], ov[8], rv[8];
      unpack8(xd[i], dv);
      unpack8(xc[i], ov);
      unpack8(xr[i], rv);
      acc[i] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[i] += dv[e] * (ov[e] + rv[e]);
    }
  }
#pragma unroll
  for (int i = 0; i < kDsumRows; ++i) {
    float v = acc[i];
    for (int o = 1; o < gw; o <<= 1) v += __shfl_xor(v, o, 64);
    if (d0 % a.hd == 0 && m0 + i < n) a.dsum[(long)(d0 / a.hd) * a.ld_stat + m0 + i] = v;
  }
}

// ---------------------------------------------------------------- dQ
// Block: 4 waves × 32 queries (q_block layout) of one kv head's q-heads;
// streams the kv head's K/V tiles. dQ = scale · dS·K.
__global__ __launch_bounds__(256, 2) void attn_dq_kernel(AttnArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, lh = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const QBlock qb = q_block(a, w);
  if (qb.empty) return;
  const int kvh = qb.h / (a.Hq / a.Hkv), h = qb.h, st = qb.st, L = qb.L;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * 2 * TILE];
  const int qpos = qb.q0 + lr;
  const bool qok = qpos < L;

  const int hd = a.hd;
  bf16x8 qf[8], df_[8];
  load_row_frags(a.q, a.ldq, st + qpos, h * hd, qok, lh, hd, qf);
  load_row_frags(a.dout, a.lddo, st + qpos, h * hd, qok, lh, hd, df_);
  const float lse2 = qok ? a.lse[(long)h * a.ld_stat + st + qpos] : 0.f;
  const float dsum = qok ? a.dsum[(long)h * a.ld_stat + st + qpos] : 0.f;
  const FragOffs fo(lane);
  const SeqTiles tk(a.k, a.ldk, st, L, w, lane, hd), tv(a.v, a.ldv, st, L, w, lane, hd);
  const unsigned lds0 = lds_addr(smem);
  load_first_two(tk, tv, qb.nt, kvh * hd, lds0, w);

  f32x16 dq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  const float sl2 = a.scale * kLog2e;
  const int nt = qb.nt;

  // The wave computes the tiles with a key at or before its last query
  // (t < nt_w); after those it only takes part in the block's loads and
  // barriers. Two loops, so the compute loop has no skip path (a skip path
  // makes the compiler copy the accumulators on every iteration).
  const int nt_w = qb.nt_w;
  auto advance = [&](int t) {
    wait_vm<0>();
    lds_barrier();  // tile t landed for every wave; stage (t+1)&1 is free
    if (t >= 1 && t + 1 < nt) {  // tiles 0 and 1 came with the prologue
      const unsigned nxt = lds0 + (unsigned)(((t + 1) & 1) * 2 * TILE * 2);
      tk.load((t + 1) * TR, kvh * hd, nxt, w);
      tv.load((t + 1) * TR, kvh * hd, nxt + TILE * 2, w);
    }
  };
  for (int t = 0; t < nt_w; ++t) {
    const int k0 = t * TR;
    const char* sK = reinterpret_cast<const char*>(smem + (t & 1) * 2 * TILE);
    const char* sV = sK + TILE * 2;
    advance(t);

    // S = Q·Kᵀ and dP = dO·Vᵀ per 32-key half; the K and V fragment reads
    // run two dim chunks ahead of their MFMAs (sched_barrier pins the order).
    f32x16 s[2] = {}, dp[2] = {};
#pragma unroll
    for (int kf = 0; kf < 2; ++kf) {
      bf16x8 kfr[8], vfr[8];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        kfr[kk] = row_frag(sK, fo, kf * 32, kk);
        vfr[kk] = row_frag(sV, fo, kf * 32, kk);
      }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        __builtin_amdgcn_sched_barrier(0);
        if (kk + 2 < 8) {
          kfr[kk + 2] = row_frag(sK, fo, kf * 32, kk + 2);
          vfr[kk + 2] = row_frag(sV, fo, kf * 32, kk + 2);
        }
        __builtin_amdgcn_sched_barrier(0);
        s[kf] = mfma32(kfr[kk], qf[kk], s[kf]);
        dp[kf] = mfma32(vfr[kk], df_[kk], dp[kf]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // P = exp2(S·scale·log2e − lse); dS = P∘(dP − dsum); masked pairs give 0
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kf][r] = fast_exp2(s[kf][r] * sl2 - lse2);
    if (k0 + TR - 1 > qb.q0 || k0 + TR > L) {
      keep_branch();
      const int lim = min(qpos, L - 1) - k0 - 4 * lh;
#pragma unroll
      for (int kf = 0; kf < 2; ++kf)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kf * 32 + 8 * (r >> 2) + (r & 3) > lim) s[kf][r] = 0.f;
    }
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kf][r] *= dp[kf][r] - dsum;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      bf16x8 kt[4];
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4) kt[d4] = tr_frag(sK, fo, kc * 16, d4);
      const bf16x8 sb = pack_chunk(s[kc >> 1], kc & 1);
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4) dq[d4] = mfma32(kt[d4], sb, dq[d4]);
    }
  }
  for (int t = nt_w; t < nt; ++t) advance(t);

  // every wave is past its last tile read: the stages take the staged rows
  __syncthreads();
  if (nt_w > 0)
    store_rows32(dq, a.scale, smem + w * 32 * kRowPitch, a.dq + (long)(st + qb.q0) * a.lddq + h * hd,
                 a.lddq, L - qb.q0, hd, lane);
}

// ---------------------------------------------------------------- dK / dV
// Block: 128 keys (4 waves × 32) of kv-head kvh; streams Q/dO tiles of every
// q head of the group over the queries at or after the block's first key.
// LDS: 2 stages × (Q tile + dO tile + lse/dsum rows) ≈ 65 KB.
__global__ __launch_bounds__(256, 1) void attn_dkdv_kernel(AttnArgs a) {
  const XcdPos xp = xcd_pos(a.Hkv);
  const int tile = xp.x;
  if (tile >= *a.ntiles_dev) return;
  const int kvh = xp.kvh, G = a.Hq / a.Hkv;
  const int4 tl = a.tiles_k[tile];
  const int st = tl.x, L = tl.y, k0 = tl.z;
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * 2 * TILE];
  __shared__ float sLD[2][2][TR];  // [stage][lse | dsum][row]
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, lh = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int key = k0 + w * 32 + lr;
  const bool kok = key < L;
  const int wk_first = k0 + w * 32;  // wave-uniform

  const int hd = a.hd;
  bf16x8 kf_[8], vf_[8];
  load_row_frags(a.k, a.ldk, st + key, kvh * hd, kok, lh, hd, kf_);
  load_row_frags(a.v, a.ldv, st + key, kvh * hd, kok, lh, hd, vf_);

  f32x16 dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[i][r] = 0.f; dv[i][r] = 0.f; }
  const float sl2 = a.scale * kLog2e;
  const FragOffs fo(lane);

  // (head, q tile) pairs flattened into one pipelined sequence; with a head
  // split (grid.z > 1) this block takes q-heads h_lo .. h_lo + hc - 1 of the
  // group and stores fp32 partial sums (dkdv_head_sum_kernel adds them)
  const int hs = (int)gridDim.z, gph = (G + hs - 1) / hs;
  const int h_lo = min(G, (int)blockIdx.z * gph), hc = min(G, h_lo + gph) - h_lo;
  const int qt0 = k0 / TR;                 // first q tile that can see these keys
  const int nq = (L + TR - 1) / TR - qt0;  // q tiles per head
  const int nit = hc * nq;
  // lse/dsum rows of pair `it` (threads < 64): loaded into registers one pair
  // ahead and stored to LDS at the end of the previous pair, so the compiler's
  // wait on these loads never drains the tile loads issued before them.
  float nl = 0.f, nd = 0.f;
  auto load_ld = [&](int it) {
    const int hq = kvh * G + h_lo + it / nq;
    const int q0 = (qt0 + it % nq) * TR;
    const bool ok = tid < TR && q0 + tid < L;
    nl = ok ? a.lse[(long)hq * a.ld_stat + st + q0 + tid] : 0.f;
    nd = ok ? a.dsum[(long)hq * a.ld_stat + st + q0 + tid] : 0.f;
  };
  const SeqTiles tq(a.q, a.ldq, st, L, w, lane, hd), to(a.dout, a.lddo, st, L, w, lane, hd);
  const unsigned lds0 = lds_addr(smem);
  auto stage = [&](int it, int sidx) {
    const int hq = kvh * G + h_lo + it / nq;
    const int q0 = (qt0 + it % nq) * TR;
    const unsigned d = lds0 + (unsigned)(sidx * 2 * TILE * 2);
    tq.load(q0, hq * hd, d, w);
    to.load(q0, hq * hd, d + TILE * 2, w);
  };
  if (nit > 0) {
    // the first two pairs' tiles (and the second pair's lse/dsum rows, kept
    // in nl/nd for the end of pair 0) are requested before the wait on the
    // first pair's lse/dsum rows, so the K/V rows, those rows and both pairs'
    // tiles arrive in one latency; the loop issues pair it+1 from it = 1 on
    load_ld(0);
    const float nl0 = nl, nd0 = nd;
    stage(0, 0);
    if (nit > 1) {
      load_ld(1);
      stage(1, 1);
    }
    if (tid < TR) {
      sLD[0][0][tid] = nl0;
      sLD[0][1][tid] = nd0;
    }
  }
  for (int it = 0; it < nit; ++it) {
    const int sidx = it & 1;
    const int q0 = (qt0 + it % nq) * TR;
    const bf16* sQ = smem + sidx * 2 * TILE;
    const bf16* sO = sQ + TILE;
    wait_vm<0>();
    __syncthreads();  // pair `it` (tiles and lse/dsum rows) visible; the other stage is free
    if (it >= 1 && it + 1 < nit) {
      load_ld(it + 1);
      stage(it + 1, sidx ^ 1);
    }
    // Every wave computes every pair: a wave whose keys all come after the
    // tile's queries gets an all-masked tile (zero contributions). Skipping it
    // would not shorten the block, whose waves meet at the next barrier, and
    // a skip path makes the compiler copy the accumulators each iteration.
    //
    // The tile's two 32-query halves run as a software pipeline of four MFMA
    // phases, so the softmax arithmetic of one half (VALU) issues between the
    // MFMAs of the next phase instead of idling the matrix pipe:
    //   A: S/dP of half 0
    //   B: S/dP of half 1   + P, dS of half 0 (one element per MFMA)
    //   C: dV/dK of half 0  + P, dS of half 1
    //   D: dV/dK of half 1
    // sched_barrier pins each (MFMA + companions) group in place.
    {
      const char* cQ = reinterpret_cast<const char*>(sQ);
      const char* cO = reinterpret_cast<const char*>(sO);
      // Mask (tiles at the diagonal or the sequence end, wave-uniform test):
      // query q pairs with the lane's key iff key <= q < L and key < L. With
      // q = q0 + 4·lh + off, off the compile-time qf·32 + 8(r/4) + r%4, that is
      // lo <= off < hi. Masked scores become −inf, so P and dS = P∘(dP − D)
      // come out 0.
      const bool masked = q0 < wk_first + 31 || q0 + TR > L || wk_first + 31 >= L;
      const int base = q0 + 4 * lh;
      const int lo = key - base;
      const int hi = kok ? L - base : lo;
      {
        // lane: key row; element r of half qf: query qf·32 + 8(r/4) + 4·lh + r%4
        f32x16 s0 = {}, d0 = {}, s1 = {}, d1 = {};
        // lse (log2) and dsum of the lane's queries, one group of 4 elements
        // ahead of its use
        f32x4 l4[2], g4[2];
        auto stats = [&](int qf, int r4, int slot) {
          const int qi = qf * 32 + 8 * r4 + 4 * lh;
          l4[slot] = *reinterpret_cast<const f32x4*>(&sLD[sidx][0][qi]);
          g4[slot] = *reinterpret_cast<const f32x4*>(&sLD[sidx][1][qi]);
        };
        float pv[8], ds[8];          // P and dS of the 16-query chunk in flight
        bf16x8 pb[2][2], sb[2][2];   // [half][16-query chunk] MFMA operands
        // P and dS of element r of half qf from its scores sc and dP values dd;
        // after the chunk's eighth element, its bf16 operands
        auto soft = [&](const f32x16& sc, const f32x16& dd, int qf, int r) {
          if ((r & 3) == 0 && (r >> 2) + 1 < 4) stats(qf, (r >> 2) + 1, ((r >> 2) + 1) & 1);
          else if ((r & 3) == 0 && qf == 0) stats(1, 0, 0);
          const float x = sc[r];
          const int sl = (r >> 2) & 1, e = r & 3;
          const float pp = fast_exp2(x * sl2 - l4[sl][e]);
          pv[r & 7] = pp;
          ds[r & 7] = pp * (dd[r] - g4[sl][e]);
          pin(pv[r & 7]);
          pin(ds[r & 7]);
          if ((r & 7) == 7) {
            bf16x8 a, b;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              a[k] = (bf16)pv[k];
              b[k] = (bf16)ds[k];
            }
            pb[qf][r >> 3] = a;
            sb[qf][r >> 3] = b;
          }
        };
        bf16x8 qf_[8], of_[8];
        // Phase A: S/dP of half 0, fragment reads two chunks ahead; the last
        // two steps read the first chunks of half 1
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          qf_[kk] = row_frag(cQ, fo, 0, kk);
          of_[kk] = row_frag(cO, fo, 0, kk);
        }
        stats(0, 0, 0);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          __builtin_amdgcn_sched_barrier(0);
          const int nk = (kk + 2) & 7, nr = kk + 2 < 8 ? 0 : 32;
          qf_[nk] = row_frag(cQ, fo, nr, nk);
          of_[nk] = row_frag(cO, fo, nr, nk);
          __builtin_amdgcn_sched_barrier(0);
          s0 = mfma32(qf_[kk], kf_[kk], s0);
          d0 = mfma32(of_[kk], vf_[kk], d0);
        }
        __builtin_amdgcn_sched_barrier(0);
        auto mask = [&](f32x16& sc, int qf) {
          if (masked) {
            keep_branch();
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int off = qf * 32 + 8 * (r >> 2) + (r & 3);
              if (off < lo || off >= hi) sc[r] = -INFINITY;
            }
          }
        };
        mask(s0, 0);
        __builtin_amdgcn_sched_barrier(0);
        // Phase B: S/dP of half 1; P, dS of half 0 one element after each MFMA
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          __builtin_amdgcn_sched_barrier(0);
          if (kk + 2 < 8) {
            qf_[kk + 2] = row_frag(cQ, fo, 32, kk + 2);
            of_[kk + 2] = row_frag(cO, fo, 32, kk + 2);
          }
          s1 = mfma32(qf_[kk], kf_[kk], s1);
          soft(s0, d0, 0, 2 * kk);
          __builtin_amdgcn_sched_barrier(0);
          d1 = mfma32(of_[kk], vf_[kk], d1);
          soft(s0, d0, 0, 2 * kk + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_sched_barrier(0);
        mask(s1, 1);
        __builtin_amdgcn_sched_barrier(0);
        // Phase C: dV += Pᵀ·dO and dK += dSᵀ·Q of half 0 over its two 16-query
        // chunks (transposed reads one block ahead); P, dS of half 1 between
        bf16x8 ot[2], qt[2];
        ot[0] = tr_frag(cO, fo, 0, 0);
        qt[0] = tr_frag(cQ, fo, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = i >> 2, d4 = i & 3;
          __builtin_amdgcn_sched_barrier(0);
          if (i + 1 < 8) {
            const int c1 = (i + 1) >> 2, e1 = (i + 1) & 3;
            ot[(i + 1) & 1] = tr_frag(cO, fo, c1 * 16, e1);
            qt[(i + 1) & 1] = tr_frag(cQ, fo, c1 * 16, e1);
          } else {
            ot[0] = tr_frag(cO, fo, 32, 0);
            qt[0] = tr_frag(cQ, fo, 32, 0);
          }
          mfma32_acc(dv[d4], ot[i & 1], pb[0][c]);
          soft(s1, d1, 1, 2 * i);
          __builtin_amdgcn_sched_barrier(0);
          mfma32_acc(dk[d4], qt[i & 1], sb[0][c]);
          soft(s1, d1, 1, 2 * i + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        // Phase D: dV/dK of half 1
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = i >> 2, d4 = i & 3;
          __builtin_amdgcn_sched_barrier(0);
          if (i + 1 < 8) {
            const int c1 = (i + 1) >> 2, e1 = (i + 1) & 3;
            ot[(i + 1) & 1] = tr_frag(cO, fo, 32 + c1 * 16, e1);
            qt[(i + 1) & 1] = tr_frag(cQ, fo, 32 + c1 * 16, e1);
          }
          __builtin_amdgcn_sched_barrier(0);
          mfma32_acc(dv[d4], ot[i & 1], pb[1][c]);
          mfma32_acc(dk[d4], qt[i & 1], sb[1][c]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (it + 1 < nit && tid < TR) {
      sLD[sidx ^ 1][0][tid] = nl;
      sLD[sidx ^ 1][1][tid] = nd;
    }
  }

  // the last accumulating MFMAs (inline asm, unseen by the compiler's hazard
  // checks) complete before their AGPRs are read
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  if (hs > 1) {
    // fp32 partials: kv_part[z][row][m·KV + kvh·128 + dim], m = 0 dK, 1 dV;
    // the lane holds key row `key`, dims d4·32 + 8g + 4·lh .. +3
    if (kok) {
      const long KV = (long)a.Hkv * hd;
      float* pr = a.kv_part + ((long)blockIdx.z * a.n + st + key) * 2 * KV + kvh * hd + 4 * lh;
      const float ks = a.scale;
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (d4 * 32 + 8 * g >= hd) continue;
          const f32x4 k4 = {dk[d4][4 * g] * ks, dk[d4][4 * g + 1] * ks, dk[d4][4 * g + 2] * ks,
                            dk[d4][4 * g + 3] * ks};
          const f32x4 v4 = {dv[d4][4 * g], dv[d4][4 * g + 1], dv[d4][4 * g + 2], dv[d4][4 * g + 3]};
          *reinterpret_cast<f32x4*>(pr + d4 * 32 + 8 * g) = k4;
          *reinterpret_cast<f32x4*>(pr + KV + d4 * 32 + 8 * g) = v4;
        }
    }
    return;
  }
  // dK and dV as whole rows through the stages, which every wave is done
  // reading
  __syncthreads();
  if (wk_first < L) {
    bf16* buf = smem + w * 32 * kRowPitch;
    const long row0 = st + wk_first;
    store_rows32(dk, a.scale, buf, a.dk + row0 * a.lddk + kvh * hd, a.lddk, L - wk_first, hd,
                 lane);
    store_rows32(dv, 1.f, buf, a.dv + row0 * a.lddv + kvh * hd, a.lddv, L - wk_first, hd, lane);
  }
}

// dK, dV = bf16(sum over the head split's slices z, in order, of the fp32
// partials), four columns per thread, live rows only.
__global__ __launch_bounds__(256) void dkdv_head_sum_kernel(AttnArgs a, int hs) {
  int N = a.n;
  if (a.n_dev) N = min(N, *a.n_dev);
  const long KV = (long)a.Hkv * a.hd, c4 = 2 * KV / 4;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)N * c4) return;
  const long row = idx / c4, col = (idx % c4) * 4;
  const float* src = a.kv_part + row * 2 * KV + col;
  const long plane = (long)a.n * 2 * KV;
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < hs; ++z) v += *reinterpret_cast<const f32x4*>(src + z * plane);
  bf16x4 b;
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = (bf16)v[i];
  bf16* dst = col < KV ? a.dk + row * a.lddk + col : a.dv + row * a.lddv + (col - KV);
  *reinterpret_cast<bf16x4*>(dst) = b;
}

hipError_t attn_fwd(const AttnArgs& a, hipStream_t s) {
  if (a.max_tiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(a.max_tiles * (a.Hq / a.Hkv), a.Hkv), dim3(256), 0, s,
                     a);
  return hipGetLastError();
}

int attn_dkdv_head_split(const AttnArgs& a) {
  const int G = a.Hkv > 0 ? a.Hq / a.Hkv : 1;
  if (G < 2 || a.n <= 0 || a.n > 1024) return 1;
  return (long)G * a.n * 2 * a.Hkv * a.hd <= a.kv_part_elems ? G : 1;
}

hipError_t attn_bwd_dkdv(const AttnArgs& a, hipStream_t s) {
  if (a.max_tiles <= 0) return hipSuccess;
  // Short cycles (at most 1024 tokens) give the pass a block per key tile
  // and kv head, far fewer than the CUs; each block then takes one q-head
  // of its group and a second launch adds the heads' fp32 partials in order.
  const int hs = a.kv_part ? attn_dkdv_head_split(a) : 1;
  hipLaunchKernelGGL(attn_dkdv_kernel, dim3(a.max_tiles, a.Hkv, hs), dim3(256), 0, s, a);
  if (hs == 1) return hipGetLastError();
  const long tot = (long)a.n * (2L * a.Hkv * a.hd / 4);
  hipLaunchKernelGGL(dkdv_head_sum_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s,
                     a, hs);
  return hipGetLastError();
}

hipError_t attn_bwd_dq(const AttnArgs& a, hipStream_t s) {
  if (a.max_tiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_dq_kernel, dim3(a.max_tiles * (a.Hq / a.Hkv), a.Hkv), dim3(256), 0, s,
                     a);
  return hipGetLastError();
}

hipError_t attn_dsum(const AttnArgs& a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const long threads = (long)(a.n + kDsumRows - 1) / kDsumRows * (a.Hq * a.hd / 8);
  hipLaunchKernelGGL(attn_dsum_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                     a);
  return hipGetLastError();
}

// dsum first (both passes read it); the dQ and dK/dV passes are independent.
hipError_t attn_bwd(const AttnArgs& a, hipStream_t s) {
  hipError_t e;
  if ((e = attn_dsum(a, s)) != hipSuccess) return e;
  if ((e = attn_bwd_dq(a, s)) != hipSuccess) return e;
  return attn_bwd_dkdv(a, s);
}

}  // namespace dsb
