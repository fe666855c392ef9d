// Per-example squared gradient norms of linear layers via the Gram identity
//   ||G_i^T A_i||_F^2 = <A_i A_i^T, G_i G_i^T>
// (no per-example gradient is ever formed), with an upper bound on the
// rounding error of the result, so that the clip factor can be taken from
// sqnorm + sqerr >= ||G_i^T A_i||^2 (the error model is in common.h).  The
// T x T Gram matrices are split into 128 x 128 tiles.  A dense work item
// stages, per 32-deep K step, the rows of two 128-row blocks p and q of both
// operands and computes from them the (p, q) tile of both A A^T and G G^T
// (waves 0..3, the same 64 x 64 block of both tiles each, so the element-wise
// inner product in fp64 needs no data exchange) and one diagonal tile that
// needs no other rows (waves 4..7; see dense_item).  Pairs with p < q count
// twice (both Gram matrices are symmetric).  Each tile writes a record to the
// workspace -- the inner product, the squared off-diagonal entries of both
// tiles and, on diagonal tiles, row weights from the diagonal entries -- and
// gram_finish_kernel folds an example's records in a fixed order into sqnorm
// and sqerr, so results are deterministic.
//
// Items are placed so that all items of one example run on one XCD (hardware
// dispatch is round-robin over the 8 XCDs): they re-read the example's rows
// from that XCD's L2 instead of from HBM.  The K loop hides LDS latency with
// two fragment sets: every group of four MFMAs runs while the next group's
// fragments are read, the barrier sits before a step's last group (which
// overlaps the next step's first reads), and the loop body has no branch
// around the accumulators (operands ordered so that din <= dout: the loop is
// the "both Gram matrices" body for A's K range, then a "G G^T only" body
// that stages G's tiles alone).  The grouped (MoE) kernel runs items of one
// tile pair on 4 waves.
#include <atomic>
#include <mutex>

#include <algorithm>

#include "clip_block.h"
#include "common.h"
#include "lds_stage.h"

// Workspace of dpc_gram_sqnorms_noalloc: one copy per device, resolved to a
// device address once per device (hipGetSymbolAddress) and used through that
// address only; the records of a call are written in full before they are
// read, so nothing in it needs clearing between calls.
static __device__ __align__(256) uint8_t scratch[DPC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kGramTile = 128;  // rows of a T-tile
constexpr int kGramThreads = 256;
constexpr int kGK = 32;                              // reduction depth per K step
constexpr int kGTileBytes = kGramTile * kGK * 2;     // 8 KiB per staged tile
constexpr int kGStageBytes = 4 * kGTileBytes;        // A_p, A_q, G_p, G_q
constexpr int kXcds = 8;
// A 16-byte chunk whose columns lie outside the row is given an offset past
// the buffer's range, which the hardware reads as zero.
constexpr int kGramOutOfRange = 0x7ff00000;

// Byte offset of 16-byte chunk c (4 per 64-byte row) of row r in a staged
// tile.  A fragment read (16 lanes = 16 consecutive rows, one chunk) and a
// staging write (16 lanes = 4 rows x 4 chunks) both touch 16 distinct 16-byte
// bank groups of the 64 four-byte banks.
__device__ __forceinline__ int gtile_off(int r, int c) {
  return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
}

__device__ __forceinline__ void pair_from_index(int pair, int* p, int* q) {
  int qq = 0;
  while ((qq + 1) * (qq + 2) / 2 <= pair) ++qq;
  *q = qq;
  *p = pair - qq * (qq + 1) / 2;
}

__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  double total = 0.0;
  if (threadIdx.x == 0) {
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) total += red[i];
  }
  return total;
}

// Record words 0..6 of a Gram tile, summed over the waves that computed it
// -- waves 4 h .. 4 h + 3 of the workgroup for h = w / 4 -- in a fixed order
// (lanes by shuffle tree, then waves), written to `rec` (if not null) with the
// gammas and the row count: see DPC_GRAM_REC_WORDS.  red: kRecStat doubles of
// LDS per wave.
constexpr int kRecStat = 7;
__device__ __forceinline__ void write_gram_record(double (&v)[kRecStat], double* red,
                                                  double* rec, double gA, double gQ, int T) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < kRecStat; ++k)
    for (int off = 32; off > 0; off >>= 1) v[k] += __shfl_down(v[k], off, 64);
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kRecStat; ++k) red[w * kRecStat + k] = v[k];
  }
  __syncthreads();
  const int t = threadIdx.x & 255, w0 = (w >> 2) * 4;
  if (rec == nullptr) return;
  if (t < kRecStat) {
    double total = 0.0;
    for (int i = 0; i < 4; ++i) total += red[(w0 + i) * kRecStat + t];
    rec[t] = total;
  } else if (t < DPC_GRAM_REC_WORDS) {
    rec[t] = t == 7 ? gA : t == 8 ? gQ : t == 9 ? (double)T : 0.0;
  }
}

// Adds a computed Gram entry pair (a of P, g of Q) to the record statistics;
// `on_diag` marks an entry with s == t, whose row weights (ws, vs) enter
// words 3..6 instead of the off-diagonal sums.
__device__ __forceinline__ void gram_entry_stats(double a, double g, bool on_diag, double gA,
                                                 double etaA, double gQ, double etaQ,
                                                 double slack, double (&v)[kRecStat]) {
  v[0] += a * g;
  if (on_diag) {
    const double ws = dpc_row_bound(a, gA, etaA, slack);
    const double vs = dpc_row_bound(g, gQ, etaQ, slack);
    v[3] += ws * ws * fabs(g);
    v[4] += vs * vs * fabs(a);
    v[5] += ws * ws;
    v[6] += vs * vs;
  } else {
    v[1] += a * a;
    v[2] += g * g;
  }
}

// Linear workgroup id -> logical (example, pair) index so that each XCD
// receives a contiguous range of logical indices.  `padded` is the grid size
// (a multiple of kXcds); returns -1 for padding workgroups.
__device__ __forceinline__ int xcd_logical_block(int padded, int nblocks) {
  const int b = blockIdx.x;
  const int per = padded / kXcds;
  const int l = (b % kXcds) * per + b / kXcds;
  return l < nblocks ? l : -1;
}

// One staged operand tile (rows row0 .. row0 + 127 of X [T, d], a 32-deep K
// step: 512 16-byte chunks): the workgroup's threads each move kC chunks,
// chunk id q = tid + (512 / kC) j -> row q >> 2, chunk q & 3.
template <int kC>
struct GramOperand {
  __amdgpu_buffer_rsrc_t rsrc;
  int row_bytes;   // d * 2
  int voff[kC];    // byte offset of the thread's chunks at K step 0
  int col[kC];     // first column of the chunks
  int d;
};

template <int kC>
__device__ __forceinline__ GramOperand<kC> make_operand(const uint16_t* X, int T, int d,
                                                        int row0) {
  GramOperand<kC> o;
  o.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(X), (short)0, T * d * 2,
                                             0x00020000);
  o.row_bytes = d * 2;
  o.d = d;
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int q = threadIdx.x + (512 / kC) * j;
    o.col[j] = (q & 3) * 8;
    o.voff[j] = (row0 + (q >> 2)) * o.row_bytes + o.col[j] * 2;
  }
  return o;
}

template <int kC>
__device__ __forceinline__ void load_operand(const GramOperand<kC>& o, int step, u32x4_t r[kC]) {
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int k = step * kGK + o.col[j];
    const int bad = k < o.d ? 0 : kGramOutOfRange;
    r[j] = __builtin_amdgcn_raw_buffer_load_b128(o.rsrc, (o.voff[j] + step * kGK * 2) | bad, 0, 0);
  }
}

template <int kC>
__device__ __forceinline__ void store_operand(uint8_t* tile, const u32x4_t r[kC]) {
#pragma unroll
  for (int j = 0; j < kC; ++j) {
    const int q = threadIdx.x + (512 / kC) * j;
    *reinterpret_cast<u32x4_t*>(tile + gtile_off(q >> 2, q & 3)) = r[j];
  }
}

// Fragments of the 16-deep sub-step kk of a staged K step for this wave's
// 64 x 64 block: a = X_p rows wr*64 + i*32 .., b = X_q rows wc*64 + j*32 ...
struct GramFrags {
  bf16x8_t a[2], b[2];
};

__device__ __forceinline__ void gram_read(const uint8_t* tp, const uint8_t* tq, int kk,
                                          GramFrags& f) {
  const int lane = threadIdx.x & 63, w = (threadIdx.x >> 6) & 3;
  const int wr = w >> 1, wc = w & 1;
  const int c = kk * 2 + (lane >> 5);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    f.a[i] = *reinterpret_cast<const bf16x8_t*>(tp + gtile_off(wr * 64 + i * 32 + (lane & 31), c));
    f.b[i] = *reinterpret_cast<const bf16x8_t*>(tq + gtile_off(wc * 64 + i * 32 + (lane & 31), c));
  }
}

// acc[i][j] += a[i] . b[j].  Rows past the segment's end read as zero, so
// the blocks they fill add nothing (their MFMAs are not skipped: a branch
// per block would put the accumulators behind control flow).
__device__ __forceinline__ void gram_mma(const GramFrags& f, f32x16_t acc[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Grouped mode: the work-item table (see gram_grouped_mfma_bf16_kernel) and
// the operands and widths of up to kMaxGramProblems problems.
constexpr int kMaxGramProblems = 64;

struct GramItems {
  const int32_t* items;  // [n_items][4]
  const int64_t* a_ptrs;
  const int64_t* g_ptrs;
  int din[kMaxGramProblems];
  int dout[kMaxGramProblems];
};

// Dense mode: the work items of an example.  An off-diagonal item (p, q)
// stages the rows of blocks p and q of both operands, which is all that the
// diagonal tiles (p, p) and (q, q) need as well, so an item also computes one
// diagonal tile from the same staged data: (b, b + 1) carries (b, b), and
// (0, nt - 1) carries (nt - 1, nt - 1) -- every diagonal tile once when nt >=
// 3.  So an example is nt (nt - 1) / 2 items of equal staging (nt = 2: (0, 1)
// carrying (0, 0), and (1, 1); nt = 1: (0, 0)), and the memory traffic of the
// diagonal tiles disappears.
DPC_HOST_DEVICE int dense_items_per_example(int nt) {
  return nt >= 3 ? nt * (nt - 1) / 2 : nt;
}

// Pair index of the j-th off-diagonal pair (p < q) of an example.
__device__ __forceinline__ int offdiag_pair(int j) {
  int q = 1;
  while (j >= q) {
    j -= q;
    ++q;
  }
  return q * (q + 1) / 2 + j;
}

// Item i of an example: its pair (p, q) and carried diagonal block c (-1:
// none).
__device__ __forceinline__ void dense_item(int i, int nt, int* p, int* q, int* c) {
  if (nt == 1) {
    *p = *q = 0;
    *c = -1;
    return;
  }
  if (nt == 2) {
    *p = i;
    *q = 1;
    *c = i == 0 ? 0 : -1;
    return;
  }
  pair_from_index(offdiag_pair(i), p, q);
  *c = (*q == *p + 1) ? *p : ((*p == 0 && *q == nt - 1) ? *q : -1);
}

// One work item: tiles (p, q) of A A^T and G G^T (waves 0..3, a 64 x 64 block
// each), and with kWaves = 8 the diagonal tiles (c, c) (waves 4..7; c = p
// when the item carries none, whose results are not recorded).  rec_pq /
// rec_c: the records to write (rec_c null: none).
template <int kWaves>
__device__ __forceinline__ void gram_body(const uint16_t* Xa, const uint16_t* Xg, int T, int din,
                                          int dout, int p, int q, int c, double* rec_pq,
                                          double* rec_c, uint8_t* lds, double* red) {
  constexpr int kC = 512 / (kWaves * 64);  // staged chunks per thread and tile
  const bool diag = (p == q);
  // <A A^T, G G^T> is symmetric in A and G: order them so that din <= dout;
  // the K loop then has one shape (both Gram matrices, then G G^T alone).
  if (din > dout) {
    const uint16_t* t = Xa;
    Xa = Xg;
    Xg = t;
    const int d = din;
    din = dout;
    dout = d;
  }

  const GramOperand<kC> ap = make_operand<kC>(Xa, T, din, p * kGramTile);
  const GramOperand<kC> aq = make_operand<kC>(Xa, T, din, q * kGramTile);
  const GramOperand<kC> gp = make_operand<kC>(Xg, T, dout, p * kGramTile);
  const GramOperand<kC> gq = make_operand<kC>(Xg, T, dout, q * kGramTile);
  const int nka = ceil_div(din, kGK), nkg = ceil_div(dout, kGK);

  f32x16_t pa[2][2], pg[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) pa[i][j] = pg[i][j] = f32x16_t{};

  // Registers hold the next K step of the four operands (the q operands are
  // not loaded on diagonal pairs).  Past an operand's K range the loads read
  // zeros, so every path issues the same loads.
  // Two register sets alternate by step parity: step s stores set (s + 1) & 1,
  // which holds step s + 1, into the other stage and reloads it with step
  // s + 3, so every load has two steps to land.
  struct Regs {
    u32x4_t ap[kC], aq[kC], gp[kC], gq[kC];
  };
  Regs R[2];
  auto load_a = [&](int step, Regs& r) __attribute__((always_inline)) {
    load_operand<kC>(ap, step, r.ap);
    if (!diag) load_operand<kC>(aq, step, r.aq);
  };
  auto load_g = [&](int step, Regs& r) __attribute__((always_inline)) {
    load_operand<kC>(gp, step, r.gp);
    if (!diag) load_operand<kC>(gq, step, r.gq);
  };
  auto store_a = [&](uint8_t* stage, const Regs& r) __attribute__((always_inline)) {
    store_operand<kC>(stage, r.ap);
    if (!diag) store_operand<kC>(stage + kGTileBytes, r.aq);
  };
  auto store_g = [&](uint8_t* stage, const Regs& r) __attribute__((always_inline)) {
    store_operand<kC>(stage + 2 * kGTileBytes, r.gp);
    if (!diag) store_operand<kC>(stage + 3 * kGTileBytes, r.gq);
  };

  load_a(0, R[0]);
  load_g(0, R[0]);
  store_a(lds, R[0]);
  store_g(lds, R[0]);
  load_a(1, R[1]);
  load_g(1, R[1]);
  load_a(2, R[0]);
  load_g(2, R[0]);
  __syncthreads();
  // A K step is four groups of MFMAs on the current stage -- A sub-steps 0
  // and 1, then G sub-steps 0 and 1 -- and each group's fragments are read
  // before the previous group's MFMAs (two fragment sets, fx and fy), so the
  // LDS latency overlaps MFMA work.  A's step s + 1 is stored into the other
  // stage (and its registers reloaded with step s + 2) after A's MFMAs, G's
  // after G's; each load is in flight for a whole step.  The barrier before
  // the last group completes the other stage, so the next step's first
  // fragments are read from it while that group's MFMAs run.  (Every wave's
  // reads of the current stage are done at the barrier -- it waits for the
  // wave's LDS operations -- so the next step may overwrite it.)
  // Waves 0..3 read the tiles of blocks p and q, waves 4..7 those of block c
  // for both operands of the product (the offsets are wave-uniform).
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool second = w >= 4;
  const int off_p = (second && c == q && !diag) ? kGTileBytes : 0;
  const int off_q = second ? off_p : (diag ? 0 : kGTileBytes);
  auto stage_ptrs = [&](const uint8_t* st, const uint8_t** tap, const uint8_t** taq,
                        const uint8_t** tgp, const uint8_t** tgq) __attribute__((always_inline)) {
    *tap = st + off_p;
    *taq = st + off_q;
    *tgp = st + 2 * kGTileBytes + off_p;
    *tgq = st + 2 * kGTileBytes + off_q;
  };
  GramFrags fx, fy;
  {
    const uint8_t *tap, *taq, *tgp, *tgq;
    stage_ptrs(lds, &tap, &taq, &tgp, &tgq);
    gram_read(tap, taq, 0, fx);
  }
  // Steps inside A's K range (nka <= nkg): on entry fx holds (in flight) A's
  // sub-step 0 fragments of the current stage.
  auto step_ag = [&](int s, Regs& rn) __attribute__((always_inline)) {
    const uint8_t* cur = lds + (s & 1) * kGStageBytes;
    uint8_t* nxt = lds + ((s + 1) & 1) * kGStageBytes;
    const uint8_t *cap, *caq, *cgp, *cgq, *nap, *naq, *ngp, *ngq;
    stage_ptrs(cur, &cap, &caq, &cgp, &cgq);
    stage_ptrs(nxt, &nap, &naq, &ngp, &ngq);
    gram_read(cap, caq, 1, fy);
    gram_mma(fx, pa);
    store_a(nxt, rn);
    load_a(s + 3, rn);
    __builtin_amdgcn_sched_barrier(0);
    gram_read(cgp, cgq, 0, fx);
    gram_mma(fy, pa);
    gram_read(cgp, cgq, 1, fy);
    gram_mma(fx, pg);
    store_g(nxt, rn);
    load_g(s + 3, rn);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    // The next step's first fragments: A's sub-step 0, or G's past A's range.
    if (s + 1 < nka) gram_read(nap, naq, 0, fx);
    else gram_read(ngp, ngq, 0, fx);
    gram_mma(fy, pg);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Steps past A's K range: on entry fx holds G's sub-step 0 fragments.  A's
  // tiles are neither loaded nor staged any more (only G's are read).
  auto step_g = [&](int s, Regs& rn) __attribute__((always_inline)) {
    const uint8_t* cur = lds + (s & 1) * kGStageBytes;
    uint8_t* nxt = lds + ((s + 1) & 1) * kGStageBytes;
    const uint8_t *cap, *caq, *cgp, *cgq, *nap, *naq, *ngp, *ngq;
    stage_ptrs(cur, &cap, &caq, &cgp, &cgq);
    stage_ptrs(nxt, &nap, &naq, &ngp, &ngq);
    gram_read(cgp, cgq, 1, fy);
    gram_mma(fx, pg);
    __builtin_amdgcn_sched_barrier(0);
    store_g(nxt, rn);
    load_g(s + 3, rn);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    gram_read(ngp, ngq, 0, fx);
    gram_mma(fy, pg);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Step s uses register set (s + 1) & 1; the loops are unrolled by two so
  // that the set is a compile-time choice.
  int s = 0;
  for (; s + 1 < nka; s += 2) {
    step_ag(s, R[1]);
    step_ag(s + 1, R[0]);
  }
  if (s < nka) {
    step_ag(s, R[1]);
    ++s;
    if (s < nkg) {
      step_g(s, R[0]);
      ++s;
    }
  }
  for (; s + 1 < nkg; s += 2) {
    step_g(s, R[1]);
    step_g(s + 1, R[0]);
  }
  if (s < nkg) step_g(s, R[1]);

  // The tile records.  Both tiles of a wave share the MFMA output layout, so
  // the element-wise product needs no knowledge of which (s, t) a register
  // holds; a diagonal entry (s == t) sits in a wave on its tile's diagonal
  // (diagonal tile, block row == block column), block i == j, at the
  // accumulator r with (r >> 2) * 8 + 4 (lane >> 5) + (r & 3) == lane & 31 --
  // one per block and lane.  After the swap above, pa is the Gram matrix of
  // the narrower operand.
  {
    const int lane = threadIdx.x & 63, wl = w & 3;
    const bool tile_diag = second || diag;
    const bool diag_wave = tile_diag && (wl >> 1) == (wl & 1);
    double st[kRecStat] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    float da[2] = {0.0f, 0.0f}, dg[2] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const double a = pa[i][j][r], g = pg[i][j][r];
          st[0] += a * g;
          const bool on_diag = i == j && diag_wave &&
                               ((r >> 2) * 8 + 4 * (lane >> 5) + (r & 3)) == (lane & 31);
          st[1] += on_diag ? 0.0 : a * a;
          st[2] += on_diag ? 0.0 : g * g;
          if (i == j) {
            da[i] = on_diag ? pa[i][j][r] : da[i];
            dg[i] = on_diag ? pg[i][j][r] : dg[i];
          }
        }
    if (!tile_diag) st[0] *= 2.0;  // exact: the off-diagonal pair counts twice
    const double gA = dpc_chain_gamma((double)nka * kGK, DPC_GRAM_U_MFMA);
    const double gQ = dpc_chain_gamma((double)nkg * kGK, DPC_GRAM_U_MFMA);
    if (diag_wave) {
      const double etaA = (double)nka * kGK * 0x1.0p-125, etaQ = (double)nkg * kGK * 0x1.0p-125;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const double ws = dpc_row_bound(da[i], gA, etaA, DPC_GRAM_ROW_SLACK_MFMA);
        const double vs = dpc_row_bound(dg[i], gQ, etaQ, DPC_GRAM_ROW_SLACK_MFMA);
        st[3] += ws * ws * fabs((double)dg[i]);
        st[4] += vs * vs * fabs((double)da[i]);
        st[5] += ws * ws;
        st[6] += vs * vs;
      }
    }
    write_gram_record(st, red, second ? rec_c : rec_pq, gA, gQ, T);
  }
}

// Dense mode: item l (after the XCD remap: each XCD takes a contiguous range
// of items, so an example's items share its L2) is item l % items of example
// l / items; 8 waves, the second four on the carried diagonal tile.
__global__ void __launch_bounds__(512, 1)
gram_mfma_bf16_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ G, int T,
                      int din, int dout, int npairs, int items, int nblocks,
                      double* __restrict__ records) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kGStageBytes];
  __shared__ double red[kRecStat * 8];
  const int l = xcd_logical_block(gridDim.x, nblocks);
  if (l < 0) return;  // padding workgroup: exits before any barrier
  const int ex = l / items;
  int p, q, c;
  dense_item(l % items, ceil_div(T, kGramTile), &p, &q, &c);
  double* rec = records + (size_t)ex * npairs * DPC_GRAM_REC_WORDS;
  gram_body<8>(A + (size_t)ex * T * din, G + (size_t)ex * T * dout, T, din, dout, p, q,
               c < 0 ? p : c, rec + (size_t)(q * (q + 1) / 2 + p) * DPC_GRAM_REC_WORDS,
               c < 0 ? nullptr : rec + (size_t)(c * (c + 3) / 2) * DPC_GRAM_REC_WORDS, lds, red);
}

// ---------------------------------------------------------------------------
// Dense split mode (bf16, an even number nt of 128-row blocks): a work item
// computes Gram tiles of ONE operand (A's K loop runs over din, G's over
// dout; with din != dout the two items of a set differ in length, and the
// dispatcher packs the short ones between the long ones).  The upper triangle of an
// example's T x T Gram matrix is cut into (nt / 2)^2 tile sets:
//   * nt / 2 diagonal sets: tiles (t, t), (t, t + 1), (t + 1, t + 1), t even
//     -- the rows of blocks t and t + 1 (8 row blocks of 32), and of the
//     diagonal tiles only the 32 x 32 blocks on or above the diagonal: 36
//     blocks;
//   * off-diagonal sets: tiles (t, q) and (t + 1, q), t even, q >= t + 2 --
//     the rows of blocks t, t + 1 and q: 32 blocks;
// and each set is computed twice, for A and for G, by two workgroups (items
// 2 j and 2 j + 1 of the example).  A workgroup stages one operand's rows (16
// or 24 KiB per 32-deep K step instead of 32, by DMA into four LDS stages)
// and holds at most 5 blocks per
// wave, the 8 waves' blocks balanced over the 4 SIMDs (9 or 8 per SIMD), so
// B (nt / 2)^2 x 2 items of nearly equal cost cover the chip (256 at B = 32,
// T = 512).  The two workgroups of a set meet through the workspace: each
// publishes its accumulators, then takes an atomic ticket; the one with the
// second ticket reads its partner's accumulators and writes the set's tile
// records -- the paired kernel's records, from the same fp32 Gram entries (a
// block above a diagonal tile's diagonal stands for itself and its mirror,
// which the MFMA computes to the same bits).  No workgroup waits for
// another.  (Letting only the first publish and the second wait for it
// measured the same.)
// ---------------------------------------------------------------------------
constexpr int kSplitWaves = 8;
template <int P>
struct StageIdx {
  static constexpr int value = P;
};
constexpr int kSplitMaxBlocks = 5;
constexpr int kSplitWaveBytes = kSplitMaxBlocks * 16 * 64 * 4;  // 20 KiB of accumulators
constexpr int kSplitSetBytes = kSplitWaves * kSplitWaveBytes;   // 160 KiB per set

DPC_HOST_DEVICE int split_sets_per_example(int nt) { return (nt / 2) * (nt / 2); }

// Tile set j of an example: *t, and *q = -1 for a diagonal set.
__device__ __forceinline__ void split_set(int j, int nt, int* t, int* q) {
  if (j < nt / 2) {
    *t = 2 * j;
    *q = -1;
    return;
  }
  j -= nt / 2;
  int tt = 0;
  while (j >= nt - tt - 2) {
    j -= nt - tt - 2;
    tt += 2;
  }
  *t = tt;
  *q = tt + 2 + j;
}

// The blocks of wave w, as row-block indices f[0..3] of the set's staged rows
// (0..7: blocks t, t + 1; 8..11: block q) and a kind:
//   kMacro      blocks (f0, f2), (f0, f3), (f1, f2), (f1, f3)
//   kExtraRows  those and (f0, f1)
//   kExtraCols  those and (f2, f3)
//   kDiag4      blocks (fk, fk), k = 0..3
// Diagonal set: the six 2 x 2 blocks above the diagonal of the 8 x 8 block
// grid go to waves 0..5, its four (2 i, 2 i + 1) blocks to waves 0..3 and its
// diagonal blocks to waves 6, 7 -- so SIMD s (waves s and s + 4) holds 9
// blocks.  Off-diagonal set: wave w holds rows 2 (w / 2), + 1 by columns 8 + 2
// (w % 2), + 1.
enum SplitKind { kMacro = 0, kExtraRows = 1, kExtraCols = 2, kDiag4 = 3 };

__device__ __forceinline__ int split_role(bool diag_set, int w, int f[4]) {
  if (!diag_set) {
    f[0] = 2 * (w >> 1);
    f[1] = f[0] + 1;
    f[2] = 8 + 2 * (w & 1);
    f[3] = f[2] + 1;
    return kMacro;
  }
  static constexpr int kF[8][4] = {{0, 1, 2, 3}, {2, 3, 4, 5}, {4, 5, 6, 7}, {2, 3, 6, 7},
                                   {0, 1, 4, 5}, {0, 1, 6, 7}, {0, 1, 2, 3}, {4, 5, 6, 7}};
  static constexpr int kKind[8] = {kExtraRows, kExtraRows, kExtraRows, kExtraCols,
                                   kMacro,     kMacro,     kDiag4,     kDiag4};
#pragma unroll
  for (int k = 0; k < 4; ++k) f[k] = kF[w][k];
  return kKind[w];
}

template <int kKind>
struct SplitShape {
  static constexpr int kBlocks = (kKind == kExtraRows || kKind == kExtraCols) ? 5 : 4;
  // Operand slots of block b: rows from slot row(b), columns from col(b).
  static __device__ __forceinline__ int row(int b) {
    if (kKind == kDiag4) return b;
    if (b == 4) return kKind == kExtraRows ? 0 : 2;
    return b >> 1;
  }
  static __device__ __forceinline__ int col(int b) {
    if (kKind == kDiag4) return b;
    if (b == 4) return kKind == kExtraRows ? 1 : 3;
    return 2 + (b & 1);
  }
};

// Tile-set record statistics of one block: its tile (0: (t, t) or (t, q);
// 1: (t, t + 1) or (t + 1, q); 2: (t + 1, t + 1)), its weight (2 for a block
// above a diagonal tile's diagonal: it stands for its mirror too) and whether
// it holds diagonal entries.
__device__ __forceinline__ void split_block_tile(bool diag_set, int rb, int cb, int* tile,
                                                 double* weight, bool* diag_block) {
  if (diag_set) {
    *tile = rb < 4 ? (cb < 4 ? 0 : 1) : 2;
    *weight = (*tile != 1 && rb < cb) ? 2.0 : 1.0;
    *diag_block = rb == cb;
  } else {
    *tile = rb < 4 ? 0 : 1;
    *weight = 1.0;
    *diag_block = false;
  }
}

// The exchange between the two items of a split tile set (or grouped
// segment): word 1 + op of the set holds item op's XCD + 1 from the kernel's
// start; the publisher adds kSplitReady once its accumulators are stored.
constexpr int kSplitReady = 0x100;
constexpr int kSplitSpinMax = 1 << 22;  // polls of ~64 cycles each: ~0.1 s

// Publisher (one thread, after the workgroup's stores completed).
__device__ __forceinline__ void split_publish(int32_t* set_words, int op, int my_xcc) {
  const int partner =
      __hip_atomic_load(&set_words[1 + (op ^ 1)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 0xff;
  if (partner != my_xcc + 1) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __hip_atomic_store(&set_words[1 + op], (my_xcc + 1) | kSplitReady, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Reader (one thread): waits for the partner's ready bit; flags[1] = the
// partner sits on this XCD, flags[2] = the wait gave up.
__device__ __forceinline__ void split_await(int32_t* set_words, int op, int my_xcc, int* flags) {
  int v = 0, spins = 0;
  for (;;) {
    v = __hip_atomic_load(&set_words[1 + (op ^ 1)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((v & kSplitReady) || ++spins >= kSplitSpinMax) break;
    __builtin_amdgcn_s_sleep(1);
  }
  flags[1] = (v & 0xff) == my_xcc + 1;
  flags[2] = (v & kSplitReady) == 0;
}

template <int kKind, bool diag_set>
__device__ __forceinline__ void split_item(const uint16_t* X, int T, int d, int din, int dout,
                                           int t, int q, const int f[4], int op, int slot,
                                           double* rec_ex, int32_t* tickets,
                                           float* __restrict__ xbuf, uint8_t* lds, double* red,
                                           int* ticket_lds, int my_xcc) {
  typedef SplitShape<kKind> S;
  constexpr int kB = S::kBlocks;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int ntr = diag_set ? 2 : 3;  // staged 128-row blocks
  const int tr_row0[3] = {t * kGramTile, (t + 1) * kGramTile, (diag_set ? t : q) * kGramTile};
  // 64-deep K steps over 128-byte row segments, three stages of three
  // 16 KiB tiles: the staging of the grouped split kernel (gsplit_item).
  constexpr int kSK = 64;
  constexpr int kTile = kGramTile * kSK * 2;
  constexpr int kStage = 3 * kTile;
  constexpr int kInst = 2 * ntr;

  // Staging by DMA: wave w moves rows 16 w .. 16 w + 15 of each staged
  // block per K step (two 1 KiB buffer_load ... lds, 8 rows each); lane i
  // the 16 bytes of row 16 w + 8 h + i / 8 that belong at physical chunk i % 8.
  const u32x4_t words = rsrc_words(X, (uint32_t)(T * d * 2));
  const int lc0 = (lane & 7) ^ ((lane >> 4) & 7), lc1 = (lane & 7) ^ ((4 + (lane >> 4)) & 7);
  int dvoff0[3], dvoff1[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    dvoff0[j] = (tr_row0[j] + 16 * w + (lane >> 3)) * d * 2 + lc0 * 16;
    dvoff1[j] = (tr_row0[j] + 16 * w + 8 + (lane >> 3)) * d * 2 + lc1 * 16;
  }
  auto dma = [&](uint8_t* stage, int step) __attribute__((always_inline)) {
    const int bad0 = step * kSK + lc0 * 8 < d ? 0 : kGramOutOfRange;
    const int bad1 = step * kSK + lc1 * 8 < d ? 0 : kGramOutOfRange;
    const uint32_t base = lds_addr(stage) + w * 2048;
#pragma unroll
    for (int j = 0; j < ntr; ++j) {
      dma16(words, base + j * kTile, dvoff0[j] | bad0, step * kSK * 2);
      dma16(words, base + j * kTile + 1024, dvoff1[j] | bad1, step * kSK * 2);
    }
  };
  // Fragment of row block f[k] at 16-deep sub-step kk: lane l reads row l % 32
  // of the block, chunk 2 kk + l / 32 (the 32x32x16 operand layout); row r's
  // chunk c sits at r * 128 + ((c ^ ((r >> 1) & 7)) << 4), so sub-step kk's
  // offset is sub-step 0's XOR 32 kk.
  int foff[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = (f[k] & 3) * 32 + (lane & 31);
    foff[k] = (f[k] >> 2) * kTile + r * 128 + (((lane >> 5) ^ ((r >> 1) & 7)) << 4);
  }
  struct Frags {
    bf16x8_t v[4];
  };
  auto read = [&](const uint8_t* stage, int kk, Frags& fr) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      fr.v[k] = *reinterpret_cast<const bf16x8_t*>(stage + (foff[k] ^ (32 * kk)));
  };
  f32x16_t acc[kB];
#pragma unroll
  for (int b = 0; b < kB; ++b) acc[b] = f32x16_t{};
  auto mma = [&](const Frags& fr) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < kB; ++b)
      acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr.v[S::row(b)], fr.v[S::col(b)], acc[b],
                                                       0, 0, 0);
  };

  // The K loop: three stages; the DMAs of step s + 3 go into step s's stage
  // right after the barrier of step s, which waits for step s + 1's.  Each
  // step is four 16-deep sub-steps whose fragments are read during the
  // previous sub-step's MFMAs; the barrier sits before the last group, which
  // runs while the next stage's first fragments are read.
  const int nk = ceil_div(d, kSK);
  uint8_t* const ring[3] = {lds, lds + kStage, lds + 2 * kStage};
  dma(ring[0], 0);
  dma(ring[1], 1);
  dma(ring[2], 2);
  DPC_WAIT_VMCNT(2 * kInst);
  __syncthreads();
  Frags fx, fy;
  read(ring[0], 0, fx);
  auto step = [&](auto P, int s) __attribute__((always_inline)) {
    constexpr int p = decltype(P)::value;
    uint8_t* cur = ring[p];
    const uint8_t* nxt = ring[(p + 1) % 3];
    read(cur, 1, fy);
    mma(fx);
    __builtin_amdgcn_sched_barrier(0);
    read(cur, 2, fx);
    mma(fy);
    __builtin_amdgcn_sched_barrier(0);
    read(cur, 3, fy);
    mma(fx);
    __builtin_amdgcn_sched_barrier(0);
    DPC_WAIT_VMCNT(kInst);  // step s + 1 has landed
    __syncthreads();
    dma(cur, s + 3);
    read(nxt, 0, fx);
    mma(fy);
    __builtin_amdgcn_sched_barrier(0);
  };
  int s = 0;
  for (; s + 3 <= nk; s += 3) {
    step(StageIdx<0>(), s);
    step(StageIdx<1>(), s + 1);
    step(StageIdx<2>(), s + 2);
  }
  if (s < nk) step(StageIdx<0>(), s);
  if (s + 1 < nk) step(StageIdx<1>(), s + 1);
  DPC_WAIT_VMCNT(0);

  // Meet the set's other workgroup.  Each takes an atomic ticket as soon as
  // its K loop is done.  The first publishes its accumulators (1 KiB per
  // store instruction), waits for the stores to complete and sets the ready
  // bit of its word (tickets[3 slot + 1 + op], which holds its XCD + 1 from
  // the kernel's start); the second, which writes the records, reads the
  // partner's accumulators once that bit is set -- in practice at once: the
  // partner took its ticket earlier and only has its stores left.  Where the
  // data meets depends on the XCDs of the two workgroups: on one XCD its L2
  // cache holds the stores and the reader only drops stale lines from its
  // CU's L1; otherwise (or when the partner's XCD is not known yet) the
  // publisher's flag carries a device-scope release and the reader's wait a
  // device-scope acquire, which write the stores back past the writer's L2
  // and drop the reader's stale L2 lines.  The wait is bounded: past
  // kSplitSpinMax polls (never seen) the records are written as NaN, which
  // makes the examples' norms non-finite, so they take the non-finite path.
  // (The waves of a diagonal set run different instantiations of this
  // function: the ticket goes through the kernel's LDS words.)
  float4* base = reinterpret_cast<float4*>(xbuf) + (size_t)slot * (2 * kSplitSetBytes / 16);
  float4* mine = base + (size_t)op * (kSplitSetBytes / 16) + (size_t)w * (kSplitWaveBytes / 16);
  const float4* theirs =
      base + (size_t)(op ^ 1) * (kSplitSetBytes / 16) + (size_t)w * (kSplitWaveBytes / 16);
  __syncthreads();
  if (tid == 0)
    ticket_lds[0] = __hip_atomic_fetch_add(&tickets[3 * slot], 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (ticket_lds[0] == 0) {
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        mine[(b * 4 + r4) * 64 + lane] = make_float4(acc[b][4 * r4], acc[b][4 * r4 + 1],
                                                     acc[b][4 * r4 + 2], acc[b][4 * r4 + 3]);
    DPC_WAIT_VMCNT(0);
    __syncthreads();
    if (tid == 0) split_publish(tickets + 3 * slot, op, my_xcc);
    return;
  }
  if (tid == 0) split_await(tickets + 3 * slot, op, my_xcc, ticket_lds);
  __syncthreads();
  if (ticket_lds[1])
    asm volatile("buffer_inv sc0" ::: "memory");  // drop stale lines from this CU's L1
  else
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const bool timed_out = ticket_lds[2] != 0;

  // Statistics per tile of the set (the paired kernel's record words; A's
  // Gram is P, G's is Q, each with the gamma of its own chain -- the bound is
  // symmetric in the two), block by block: the partner's block is read, the
  // block's words are summed over the lanes (shuffle tree) and added into
  // this wave's LDS slot of its tile; then the slots are summed over the
  // waves in order.
  const int nka = ceil_div(din, kGK), nkg = ceil_div(dout, kGK);
  const double gA = dpc_chain_gamma((double)nka * kGK, DPC_GRAM_U_MFMA);
  const double gQ = dpc_chain_gamma((double)nkg * kGK, DPC_GRAM_U_MFMA);
  const double etaA = (double)nka * kGK * 0x1.0p-125, etaQ = (double)nkg * kGK * 0x1.0p-125;
  const double invA = dpc_row_inv(gA), invQ = dpc_row_inv(gQ);
  if (lane < 3 * kRecStat) red[((lane / kRecStat) * kSplitWaves + w) * kRecStat + lane % kRecStat] = 0.0;
  // All of the partner's blocks are requested before any is used.
  f32x16_t others[kB];
#pragma unroll
  for (int b = 0; b < kB; ++b)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const float4 x = theirs[(b * 4 + r4) * 64 + lane];
      others[b][4 * r4] = x.x;
      others[b][4 * r4 + 1] = x.y;
      others[b][4 * r4 + 2] = x.z;
      others[b][4 * r4 + 3] = x.w;
    }
  // Each lane sums its blocks' words per tile (blocks in order); the lanes
  // are then summed once per tile the wave touches, and only the words its
  // blocks can make non-zero (row weights: the diagonal blocks of kDiag4
  // waves only), so a wave runs at most 7 cross-lane sums instead of 7 per
  // block.
  constexpr int kWords = kKind == kDiag4 ? kRecStat : 3;
  double tv[3][kWords];
  bool touched[3] = {false, false, false};
#pragma unroll
  for (int u = 0; u < 3; ++u)
#pragma unroll
    for (int k = 0; k < kWords; ++k) tv[u][k] = 0.0;
#pragma unroll
  for (int b = 0; b < kB; ++b) {
    const f32x16_t& other = others[b];
    int tile;
    double wgt;
    bool dblk;
    split_block_tile(diag_set, f[S::row(b)], f[S::col(b)], &tile, &wgt, &dblk);
    double v[kRecStat] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    float da = 0.0f, dg = 0.0f;
    bool has_diag = false;
    // x: this item's operand, y: the partner's; the sums of squares are
    // swapped into place (v[1]: A's, v[2]: G's) after the block.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const double x = acc[b][r], y = other[r];
      v[0] += x * y;
      // Only kDiag4 waves hold diagonal blocks (the other kinds pair distinct
      // row blocks): for them the test folds away at compile time.
      const bool on_diag = kKind == kDiag4 && dblk &&
                           ((r >> 2) * 8 + 4 * (lane >> 5) + (r & 3)) == (lane & 31);
      v[1] += on_diag ? 0.0 : x * x;
      v[2] += on_diag ? 0.0 : y * y;
      da = on_diag ? acc[b][r] : da;
      dg = on_diag ? other[r] : dg;
      has_diag = has_diag || on_diag;
    }
    if (op != 0) {
      const double t = v[1];
      v[1] = v[2];
      v[2] = t;
      const float d = da;
      da = dg;
      dg = d;
    }
    if (has_diag) {
      const double ws = dpc_row_bound_inv(da, invA, etaA, DPC_GRAM_ROW_SLACK_MFMA);
      const double vs = dpc_row_bound_inv(dg, invQ, etaQ, DPC_GRAM_ROW_SLACK_MFMA);
      v[3] = ws * ws * fabs((double)dg);
      v[4] = vs * vs * fabs((double)da);
      v[5] = ws * ws;
      v[6] = vs * vs;
    }
    // Weight 2 (exact) for a block that stands for its mirror as well.
    v[0] *= wgt;
    v[1] *= wgt;
    v[2] *= wgt;
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const bool mine = tile == u;
      touched[u] = touched[u] || mine;
#pragma unroll
      for (int k = 0; k < kWords; ++k) tv[u][k] = mine ? tv[u][k] + v[k] : tv[u][k];
    }
  }
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    if (!touched[u]) continue;  // wave-uniform
#pragma unroll
    for (int k = 0; k < kWords; ++k) {
      const double x = wave_sum_lane63_f64(tv[u][k]);
      if (lane == 63) red[(u * kSplitWaves + w) * kRecStat + k] = x;
    }
  }
  __syncthreads();

  // Records.
  const int ntiles = diag_set ? 3 : 2;
  int pair[3];
  if (diag_set) {
    pair[0] = t * (t + 3) / 2;
    pair[1] = (t + 1) * (t + 2) / 2 + t;
    pair[2] = (t + 1) * (t + 4) / 2;
  } else {
    pair[0] = q * (q + 1) / 2 + t;
    pair[1] = q * (q + 1) / 2 + t + 1;
    pair[2] = 0;
  }
  if (tid < 3 * DPC_GRAM_REC_WORDS) {
    const int u = tid / DPC_GRAM_REC_WORDS, k = tid % DPC_GRAM_REC_WORDS;
    if (u < ntiles) {
      double val;
      if (k < kRecStat) {
        val = 0.0;
        for (int i = 0; i < kSplitWaves; ++i) val += red[(u * kSplitWaves + i) * kRecStat + k];
        // The off-diagonal tile of the pair counts twice (exact).
        const bool offdiag = !diag_set || u == 1;
        if (k == 0 && offdiag) val *= 2.0;
      } else {
        val = k == 7 ? gA : k == 8 ? gQ : k == 9 ? (double)T : 0.0;
      }
      // A device-scope store: written through to memory, where another XCD's
      // workgroup (the launch's tail) reads it without a writeback of this
      // XCD's L2.
      if (timed_out && k < kRecStat) val = __builtin_nan("");
      __hip_atomic_store(&rec_ex[(size_t)pair[u] * DPC_GRAM_REC_WORDS + k], val, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Dense split mode: item l (after the XCD remap: an example's items, and
// the two items of each set, share an XCD) is operand l % 2 of set (l / 2) %
// nsets of example l / (2 nsets).
// The layers of a split launch (up to kSplitMaxLayers, one T and B): layer
// L's operands and widths, and `region`, the index of its share of the
// records, tickets and exchange area.
constexpr int kSplitMaxLayers = 8;
struct SplitLayers {
  const uint16_t* A[kSplitMaxLayers];
  const uint16_t* G[kSplitMaxLayers];
  int din[kSplitMaxLayers], dout[kSplitMaxLayers], region[kSplitMaxLayers];
  int n;
  int round;  // several layers: the CUs of an XCD (0: layer after layer)
};

// Several layers: the item at position lx of an XCD's range.  The items fall
// into classes (layer, operand) of bpx * nsets items, each with its
// operand's K loop.  An XCD's workgroups go to its CUs in launch order, one
// per free CU, and a workgroup that finds no free CU holds back the launch's
// later ones on every XCD; so the classes run in decreasing order of K (ties:
// layer, then operand), which makes every round of `round` consecutive
// positions items of one length (no CU waits behind another's long item),
// in serpentine rounds (odd rounds reversed) so that the CUs' sums even out
// where a class ends inside a round.
__device__ __forceinline__ void split_multi_item(const SplitLayers& lay, int nsets, int bpx,
                                                 int per_xcd, int lx, int* L, int* ex_local,
                                                 int* set, int* op) {
  const int W = lay.round;
  const int r = lx / W, slot = lx - r * W;
  const bool full = (r + 1) * W <= per_xcd;
  const int rank = ((r & 1) && full) ? r * W + (W - 1 - slot) : lx;
  const int per_cls = bpx * nsets;
  const int c = rank / per_cls, j = rank - c * per_cls;
  int cls = 0;
  for (int k = 0; k < 2 * lay.n; ++k) {
    const int kk = (k & 1) ? lay.dout[k >> 1] : lay.din[k >> 1];
    int pos = 0;
    for (int m = 0; m < 2 * lay.n; ++m) {
      const int km = (m & 1) ? lay.dout[m >> 1] : lay.din[m >> 1];
      pos += (km > kk || (km == kk && m < k)) ? 1 : 0;
    }
    if (pos == c) cls = k;
  }
  *L = cls >> 1;
  *op = cls & 1;
  *ex_local = j / nsets;
  *set = j - (j / nsets) * nsets;
}

// The clip factors folded into a split launch (dpc_gram_clip_factors).  Each
// tile set's record writer (the item with the second ticket) clears the
// set's ticket words and counts the set into its example's counter; the
// last set of an example folds the example's records into sqnorm / sqerr
// (as gram_finish_kernel does: the same bits) while other items still run,
// and counts the example into `done`; the last example's finisher computes
// the clip factors and plans of all examples from them (clip_factors_block:
// the same bits as clip_factors_kernel).  Every counter is back at zero when
// the launch ends, for the next one.  done == nullptr: no tail (the caller
// launches the finish).
struct SplitTail {
  int32_t* done;     // [1]
  int32_t* ex_done;  // [B]: sets (of all layers) written per example
  double* sqnorm;
  double* sqerr;
  ClipJob job;
};

__device__ __forceinline__ double gram_bound_wave(const double* rec, int nt, double* sum);

// Largest batch whose flags the tail keeps in the staging LDS (4 bytes per
// example).
constexpr int kSplitTailMaxB = 1024;

// Device-scope loads of n words into LDS by the whole workgroup, eight per
// thread in flight (the data may come from other XCDs: no cache is trusted).
template <typename T>
__device__ __forceinline__ void load_agent_to_lds(const T* __restrict__ src, T* dst, int n) {
  constexpr int kU = 8;
  for (int i0 = 0; i0 < n; i0 += kU * (int)blockDim.x) {
    T v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = i0 + u * (int)blockDim.x + (int)threadIdx.x;
      v[u] = i < n ? __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : T(0);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = i0 + u * (int)blockDim.x + (int)threadIdx.x;
      if (i < n) dst[i] = v[u];
    }
  }
}

// Called by every item after its part of the set (`writer`: this item wrote
// the set's records; its partner has taken its ticket).  Counters advance
// only after the data they announce has completed at the memory side
// (device-scope stores and a wait), so no cache writeback is needed.  The
// example's last set folds its records, computes the example's clip
// factors (clip_example_eval: the same bits as the whole-batch pass), leaves
// the example's flag bits in its set counter; the last example's finisher
// builds the plans and counts from every example's flags and clears the
// counters.  Barriers that only hand LDS words between waves order LDS
// alone (dpc_lds_barrier), so the output stores are never waited for.
__device__ void split_tail(const SplitTail& tail, const double* __restrict__ records,
                           int32_t* set_tickets, bool writer, int ex, int B, int nt, int nsets,
                           int nlayers, uint8_t* lds, int* flag) {
  if (!writer) return;
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 3) set_tickets[tid] = 0;  // both items of the set are past them
  DPC_WAIT_VMCNT(0);                  // this wave's record stores have completed
  __syncthreads();
  if (tid == 0)
    flag[0] = __hip_atomic_fetch_add(&tail.ex_done[ex], 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == nsets * nlayers - 1;
  dpc_lds_barrier();
  if (!flag[0]) return;
  // The example's last set: fold its records (every layer's).
  const size_t np = (size_t)nt * (nt + 1) / 2;
  const int ex_words = (int)(np * DPC_GRAM_REC_WORDS);
  double* rec_lds = reinterpret_cast<double*>(lds);
  for (int L = 0; L < nlayers; ++L)
    load_agent_to_lds(records + ((size_t)L * B + ex) * ex_words, rec_lds + L * ex_words,
                      ex_words);
  dpc_lds_barrier();
  if (tid < 64) {
    double v = 0.0, ev = 0.0;
    for (int L = 0; L < nlayers; ++L) {
      double sm;
      const double e = gram_bound_wave(rec_lds + L * ex_words, nt, &sm);
      v = L == 0 ? sm : v + sm;
      ev = L == 0 ? e : ev + e;
    }
    if (lane == 0) {
      const ClipExample e = clip_example_eval(v, ev, tail.sqerr != nullptr, B, tail.job);
      // The flags replace the example's set count; they are at memory before
      // the example is counted.
      __hip_atomic_store(&tail.ex_done[ex], e.flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      DPC_WAIT_VMCNT(0);
      flag[0] = __hip_atomic_fetch_add(tail.done, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == B - 1;
      // The outputs are read after the launch only: stored last, not waited for.
      tail.sqnorm[ex] = v;
      if (tail.sqerr) tail.sqerr[ex] = ev;
      clip_example_store(e, ex, B, tail.job);
    }
  }
  dpc_lds_barrier();
  if (!flag[0]) return;
  // The last example: the plans and counts of all of them (wave 0).
  if (tid == 0) *tail.done = 0;
  int* fl = reinterpret_cast<int*>(lds);
  load_agent_to_lds(tail.ex_done, fl, B);
  dpc_lds_barrier();
  for (int i = tid; i < B; i += (int)blockDim.x) tail.ex_done[i] = 0;
  if (tid < 64) {
    ClipLists st = {};
    clip_compact_wave(fl, B, 0, B, tail.job, st);
    clip_finish_wave(st, B, tail.job);
  }
}

__global__ void __launch_bounds__(512, 1)
gram_split_bf16_kernel(const SplitLayers lay, int B, int T, int npairs, int nsets, int nblocks,
                       double* __restrict__ records, int32_t* __restrict__ tickets,
                       float* __restrict__ xbuf, const SplitTail tail) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * 3 * kGramTile * 64 * 2];
  __shared__ double red[3 * kSplitWaves * kRecStat];
  __shared__ int ticket_lds[3];
  const int l0 = xcd_logical_block(gridDim.x, nblocks);
  if (l0 < 0) return;  // padding workgroup: exits before any barrier
  // Several layers (B % 8 == 0): every XCD's range holds, layer after layer,
  // the items of B / 8 examples of each layer, so the XCDs get equal work.
  int L = 0, l = l0;
  if (lay.n > 1) {
    const int per_xcd = nblocks / kXcds, bpx = B / kXcds, per_lx = bpx * 2 * nsets;
    const int x = l0 / per_xcd, lx = l0 - x * per_xcd;
    if (lay.round > 0) {
      int e, st, o;
      split_multi_item(lay, nsets, bpx, per_xcd, lx, &L, &e, &st, &o);
      l = ((x * bpx + e) * nsets + st) * 2 + o;
    } else {
      L = lx / per_lx;
      const int r = lx - L * per_lx;
      l = (x * bpx + r / (2 * nsets)) * 2 * nsets + r % (2 * nsets);
    }
  }
  L = __builtin_amdgcn_readfirstlane(L);
  l = __builtin_amdgcn_readfirstlane(l);
  const uint16_t* A = lay.A[L];
  const uint16_t* G = lay.G[L];
  const int din = lay.din[L], dout = lay.dout[L];
  const double* all_records = records;
  {
    const size_t reg = (size_t)lay.region[L];
    records += reg * B * npairs * DPC_GRAM_REC_WORDS;
    tickets += reg * 3 * nsets * B;
    xbuf += reg * B * nsets * (2 * kSplitSetBytes / 4);
  }
  const int op = l & 1, set = (l >> 1) % nsets, ex = (l >> 1) / nsets;
  const int nt = ceil_div(T, kGramTile);
  int t, q;
  split_set(set, nt, &t, &q);
  const bool diag_set = q < 0;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int f[4];
  const int kind = split_role(diag_set, w, f);
  const int d = op == 0 ? din : dout;
  const uint16_t* X = (op == 0 ? A + (size_t)ex * T * din : G + (size_t)ex * T * dout);
  double* rec_ex = records + (size_t)ex * npairs * DPC_GRAM_REC_WORDS;
  const int slot = (l >> 1);
  // This workgroup's XCD, published for the partner (tickets[3 slot + 1 +
  // op] = xcc + 1; 0 until published).
  int xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  xcc &= 0xf;
  if (threadIdx.x == 0)
    __hip_atomic_store(&tickets[3 * slot + 1 + op], xcc + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  if (!diag_set) {
    split_item<kMacro, false>(X, T, d, din, dout, t, q, f, op, slot, rec_ex, tickets, xbuf, lds, red,
                              ticket_lds, xcc);
  } else {
    switch (kind) {
      case kMacro:
        split_item<kMacro, true>(X, T, d, din, dout, t, q, f, op, slot, rec_ex, tickets, xbuf, lds,
                                 red, ticket_lds, xcc);
        break;
      case kExtraRows:
        split_item<kExtraRows, true>(X, T, d, din, dout, t, q, f, op, slot, rec_ex, tickets, xbuf,
                                     lds, red, ticket_lds, xcc);
        break;
      case kExtraCols:
        split_item<kExtraCols, true>(X, T, d, din, dout, t, q, f, op, slot, rec_ex, tickets, xbuf,
                                     lds, red, ticket_lds, xcc);
        break;
      default:
        split_item<kDiag4, true>(X, T, d, din, dout, t, q, f, op, slot, rec_ex, tickets, xbuf, lds,
                                 red, ticket_lds, xcc);
        break;
    }
  }
  if (tail.done)
    split_tail(tail, all_records, tickets + 3 * slot, ticket_lds[0] != 0, ex, B, nt, nsets, lay.n,
               lds, ticket_lds);
}

__global__ void __launch_bounds__(kGramThreads) fill_zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Grouped mode: work item l is (problem << 16 | pair, first row, rows, slot)
// -- the tile pair `pair` of the rows-long segment starting at `first row` of
// problem `problem`'s operands (a_ptrs / g_ptrs, widths din[problem] /
// dout[problem]); rows past the segment read as zero; the result goes to
// partial[slot].  4 waves; two workgroups fit on a CU (64 KiB of LDS, <= 256
// registers per lane at 2 waves per SIMD).
__global__ void __launch_bounds__(256, 2)
gram_grouped_mfma_bf16_kernel(GramItems work, int nblocks, double* __restrict__ records) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kGStageBytes];
  __shared__ double red[kRecStat * 4];
  const int l = xcd_logical_block(gridDim.x, nblocks);
  if (l < 0) return;  // padding workgroup: exits before any barrier
  const int32_t* it = work.items + 4 * (size_t)l;
  if (it[0] < 0) return;  // empty item: exits before any barrier
  const int problem = it[0] >> 16, row0 = it[1];
  const int din = work.din[problem], dout = work.dout[problem];
  int p, q;
  pair_from_index(it[0] & 0xffff, &p, &q);
  gram_body<4>(reinterpret_cast<const uint16_t*>(work.a_ptrs[problem]) + (size_t)row0 * din,
               reinterpret_cast<const uint16_t*>(work.g_ptrs[problem]) + (size_t)row0 * dout,
               it[2], din, dout, p, q, p, records + (size_t)it[3] * DPC_GRAM_REC_WORDS, nullptr,
               lds, red);
}

// ---------------------------------------------------------------------------
// Grouped split mode (bf16 MFMA path, segments of 1 .. 320 rows, the common
// case of mixture-of-experts layers: a top-2-of-8 expert sees ~T / 4 rows of
// each example).  The dense split kernel's design over one segment: a work
// item computes the upper triangle of ONE operand's segment Gram matrix, and
// the segment's two items (A and G) meet through the workspace as a tile set
// does.  A segment's rows are cut into 32-row units (rows past its end read
// as zero): up to 8 units are the dense kernel's diagonal set (36 blocks of
// 32 x 32 over 8 waves); a ninth and a tenth unit (rows 256 .. 319) add their
// columns' 9 and 10 blocks through fragment slots 4 and 5 (45 or 55 blocks:
// 11-12 or 13-14 per SIMD, at most 7 per wave).  Each item stages its
// segment's rows once per K step (16 or 20 KiB), so the launch reads every
// operand row from memory exactly once:
// the grouped Gram is bound by HBM (config 5: 1.375 GB of operands for
// 1.77e11 FLOP).  Records are the pair kernel's, per 128-row tile pair of the
// segment (3 tiles at most), so segment_finish_kernel folds both kinds.
// ---------------------------------------------------------------------------
constexpr int kGsMaxRows = 320;
constexpr int kGsMaxBlocks = 7;
constexpr int kGsWaveBytes = kGsMaxBlocks * 16 * 64 * 4;  // 28 KiB of accumulators
constexpr int kGsSetBytes = kSplitWaves * kGsWaveBytes;   // 224 KiB per operand
constexpr int kGsMaxPairs = 6;
constexpr int kGsSlots = 6;

// Modes by the segment's 32-row units: M = 8 (up to 256 rows), 9 (288), 10
// (320).  Wave w's fragment slots 0..3 hold units lo, lo + 1, hi, hi + 1
// (the dense diagonal set's roles); slots 4 and 5 hold units 8 and 9.
DPC_HOST_DEVICE constexpr int gs_unit(int w, int s) {
  // lo = {0, 2, 4, 2, 0, 0, 0, 4}[w], hi = {2, 4, 6, 6, 4, 6, 2, 6}[w], as
  // 3-bit fields (no array: every use folds to a constant).
  return s >= 4 ? 4 + s : (int)(((s < 2 ? 0x800510u : 0xCB4DA2u) >> (3 * w)) & 7u) + (s & 1);
}
// Blocks of wave w, as (row slot, column slot):
//   base  waves 0..2: (0,2) (0,3) (1,2) (1,3) (0,1); wave 3: the four and
//         (2,3); waves 4, 5: the four; waves 6, 7: (0,0) (1,1) (2,2) (3,3);
//   M>=9  unit 8's column: wave 3 (4,4); 4: (0,4) (1,4); 5, 6: (2,4) (3,4);
//         7: (0,4) (1,4);
//   M=10  unit 9's column: waves 0..2 (0,5) (1,5); 3: (2,5); 4: (4,5);
//         5: (3,5); 6: (5,5).
// Blocks per SIMD (waves s and s + 4): 9 | 11 or 12 | 13 or 14.
DPC_HOST_DEVICE constexpr int gs_nbase(int w) { return w < 4 ? 5 : 4; }
DPC_HOST_DEVICE constexpr int gs_n9(int w) { return w < 3 ? 0 : (w == 3 ? 1 : 2); }
DPC_HOST_DEVICE constexpr int gs_n10(int w) { return w < 3 ? 2 : (w == 7 ? 0 : 1); }
DPC_HOST_DEVICE constexpr int gs_nblocks(int M, int w) {
  return gs_nbase(w) + (M >= 9 ? gs_n9(w) : 0) + (M >= 10 ? gs_n10(w) : 0);
}
// Packed (row slot << 4 | column slot) of block b.
DPC_HOST_DEVICE constexpr int gs_block(int M, int w, int b) {
  if (b < gs_nbase(w)) {
    if (w >= 6) return b << 4 | b;
    if (b < 4) return (b >> 1) << 4 | (2 + (b & 1));
    return w < 3 ? (0 << 4 | 1) : (2 << 4 | 3);
  }
  const int j9 = b - gs_nbase(w);
  if (M >= 9 && j9 < gs_n9(w)) {
    if (w == 3) return 4 << 4 | 4;
    return ((w == 5 || w == 6) ? 2 + j9 : j9) << 4 | 4;
  }
  const int j = j9 - (M >= 9 ? gs_n9(w) : 0);
  if (w < 3) return j << 4 | 5;
  return (w == 3 ? 2 : w == 4 ? 4 : w == 5 ? 3 : 5) << 4 | 5;
}
DPC_HOST_DEVICE constexpr int gs_row_slot(int M, int w, int b) { return gs_block(M, w, b) >> 4; }
DPC_HOST_DEVICE constexpr int gs_col_slot(int M, int w, int b) { return gs_block(M, w, b) & 15; }
DPC_HOST_DEVICE constexpr bool gs_uses_slot(int M, int w, int s) {
  for (int b = 0; b < gs_nblocks(M, w); ++b)
    if (gs_row_slot(M, w, b) == s || gs_col_slot(M, w, b) == s) return true;
  return false;
}
// The 128-row tile pair (p <= q) of block b, as a record index q (q + 1) / 2 + p.
DPC_HOST_DEVICE constexpr int gs_pair(int M, int w, int b) {
  const int p = gs_unit(w, gs_row_slot(M, w, b)) >> 2, q = gs_unit(w, gs_col_slot(M, w, b)) >> 2;
  return q * (q + 1) / 2 + p;
}
DPC_HOST_DEVICE constexpr bool gs_has_diag(int M, int w) {
  for (int b = 0; b < gs_nblocks(M, w); ++b)
    if (gs_unit(w, gs_row_slot(M, w, b)) == gs_unit(w, gs_col_slot(M, w, b))) return true;
  return false;
}
// The wave's distinct tile pairs in order of first appearance: block b's
// index among them, their number, and the pair of index l.
DPC_HOST_DEVICE constexpr int gs_local(int M, int w, int b) {
  int n = 0;
  for (int i = 0; i < b; ++i) {
    bool seen = false;
    for (int j = 0; j < i; ++j) seen = seen || gs_pair(M, w, j) == gs_pair(M, w, i);
    if (!seen) {
      if (gs_pair(M, w, i) == gs_pair(M, w, b)) return n;
      ++n;
    }
  }
  return n;
}
DPC_HOST_DEVICE constexpr int gs_nlocal(int M, int w) {
  int n = 0;
  for (int b = 0; b < gs_nblocks(M, w); ++b)
    n = gs_local(M, w, b) + 1 > n ? gs_local(M, w, b) + 1 : n;
  return n;
}
DPC_HOST_DEVICE constexpr int gs_local_pair(int M, int w, int l) {
  for (int b = 0; b < gs_nblocks(M, w); ++b)
    if (gs_local(M, w, b) == l) return gs_pair(M, w, b);
  return 0;
}

template <int W, int M>
__device__ __forceinline__ void gsplit_item(const uint16_t* X, int n, int d, int din, int dout,
                                            int op, int set, double* rec, int32_t* tickets,
                                            float* __restrict__ xbuf, uint8_t* lds, double* red,
                                            int* ticket_lds, int my_xcc) {
  constexpr int kB = gs_nblocks(M, W);
  // 128-row tiles this wave feeds: tile 2 holds units 8 (rows 0..31) and 9.
  constexpr int kDma = W < (M - 8) * 2 ? 3 : 2;
  constexpr int kWords = gs_has_diag(M, W) ? kRecStat : 3;
  const int tid = threadIdx.x, lane = tid & 63;

  // 64-deep K steps: each staged row is a whole 128-byte segment of the
  // operand row (with 32-deep steps the memory system fetched 64 bytes from
  // every row per step and sustained ~4.3 TB/s).  A staged 128-row tile is
  // 16 KiB: row r's 16-byte chunk c at r * 128 + ((c ^ ((r >> 1) & 7)) << 4),
  // so that a fragment read (16 consecutive rows, one chunk) and a DMA write
  // (8 rows x 8 chunks) each touch 16 distinct 16-byte bank groups.  Three
  // stages of three tiles (144 KiB): the DMAs of step s + 3 go into step s's
  // stage after the barrier of step s, which waits for step s + 1's.
  constexpr int kSK = 64;                     // reduction depth per K step
  constexpr int kTile = kGramTile * kSK * 2;  // 16 KiB
  constexpr int kStage = 3 * kTile;
  constexpr int kInst = 2 * kDma;             // two 8-row DMAs per tile fed

  // Staging by DMA: wave W moves rows 16 W .. 16 W + 15 of each tile it feeds
  // (two 1 KiB buffer_load ... lds, 8 rows each); lane i the 16 bytes of row
  // 16 W + 8 h + i / 8 that belong at physical chunk i % 8.  Rows at or past
  // the segment's end are past the buffer range and read as zero.
  const u32x4_t words = rsrc_words(X, (uint32_t)(n * d * 2));
  auto lchunk_of = [&](int h) { return (lane & 7) ^ ((4 * h + (lane >> 4)) & 7); };
  const int lc0 = lchunk_of(0), lc1 = lchunk_of(1);
  const int voff0 = (16 * W + (lane >> 3)) * d * 2 + lc0 * 16;
  const int voff1 = (16 * W + 8 + (lane >> 3)) * d * 2 + lc1 * 16;
  auto dma = [&](uint8_t* stage, int step) __attribute__((always_inline)) {
    const int bad0 = step * kSK + lc0 * 8 < d ? 0 : kGramOutOfRange;
    const int bad1 = step * kSK + lc1 * 8 < d ? 0 : kGramOutOfRange;
    const uint32_t base = lds_addr(stage) + W * 2048;
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      dma16(words, base + j * kTile, (voff0 + j * kGramTile * d * 2) | bad0, step * kSK * 2);
      dma16(words, base + j * kTile + 1024, (voff1 + j * kGramTile * d * 2) | bad1,
            step * kSK * 2);
    }
  };
  // Fragment of slot s at 16-deep sub-step kk: lane l reads row l % 32 of
  // the slot's unit, chunk 2 kk + l / 32; sub-step kk's offset is sub-step
  // 0's XOR 32 kk.
  int foff[kGsSlots];
#pragma unroll
  for (int s = 0; s < kGsSlots; ++s) {
    const int u = gs_unit(W, s);
    const int r = (u & 3) * 32 + (lane & 31);
    foff[s] = (u >> 2) * kTile + r * 128 + (((lane >> 5) ^ ((r >> 1) & 7)) << 4);
  }
  struct Frags {
    bf16x8_t v[kGsSlots];
  };
  auto read = [&](const uint8_t* stage, int kk, Frags& fr) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < kGsSlots; ++s)
      if (gs_uses_slot(M, W, s))
        fr.v[s] = *reinterpret_cast<const bf16x8_t*>(stage + (foff[s] ^ (32 * kk)));
  };
  f32x16_t acc[kB];
#pragma unroll
  for (int b = 0; b < kB; ++b) acc[b] = f32x16_t{};
  auto mma = [&](const Frags& fr) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < kB; ++b)
      acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr.v[gs_row_slot(M, W, b)],
                                                       fr.v[gs_col_slot(M, W, b)], acc[b], 0, 0, 0);
  };

  // Each step: four sub-steps of MFMAs, the fragments of the next read during
  // the current one's; the barrier sits before the last group, whose MFMAs
  // run while the next stage's first fragments are read.
  const int nk = ceil_div(d, kSK);
  uint8_t* const ring[3] = {lds, lds + kStage, lds + 2 * kStage};
  dma(ring[0], 0);
  dma(ring[1], 1);
  dma(ring[2], 2);
  DPC_WAIT_VMCNT(2 * kInst);  // step 0 has landed
  __syncthreads();
  Frags fx, fy;
  read(ring[0], 0, fx);
  auto step = [&](auto P, int s) __attribute__((always_inline)) {
    constexpr int p = decltype(P)::value;
    uint8_t* cur = ring[p];
    const uint8_t* nxt = ring[(p + 1) % 3];
    read(cur, 1, fy);
    mma(fx);
    __builtin_amdgcn_sched_barrier(0);
    read(cur, 2, fx);
    mma(fy);
    __builtin_amdgcn_sched_barrier(0);
    read(cur, 3, fy);
    mma(fx);
    __builtin_amdgcn_sched_barrier(0);
    DPC_WAIT_VMCNT(kInst);  // step s + 1 has landed
    __syncthreads();
    dma(cur, s + 3);
    read(nxt, 0, fx);
    mma(fy);
    __builtin_amdgcn_sched_barrier(0);
  };
  int s = 0;
  for (; s + 3 <= nk; s += 3) {
    step(StageIdx<0>(), s);
    step(StageIdx<1>(), s + 1);
    step(StageIdx<2>(), s + 2);
  }
  if (s < nk) step(StageIdx<0>(), s);
  if (s + 1 < nk) step(StageIdx<1>(), s + 1);
  DPC_WAIT_VMCNT(0);

  // Meet the segment's other item as split_item meets its partner: the
  // first to finish publishes its accumulators and sets its ready bit, the
  // second reads them and writes the segment's records.
  float4* base = reinterpret_cast<float4*>(xbuf) + (size_t)set * (2 * kGsSetBytes / 16);
  float4* mine = base + (size_t)op * (kGsSetBytes / 16) + (size_t)W * (kGsWaveBytes / 16);
  const float4* theirs =
      base + (size_t)(op ^ 1) * (kGsSetBytes / 16) + (size_t)W * (kGsWaveBytes / 16);
  __syncthreads();
  if (tid == 0)
    ticket_lds[0] = __hip_atomic_fetch_add(&tickets[3 * set], 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (ticket_lds[0] == 0) {
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        mine[(b * 4 + r4) * 64 + lane] = make_float4(acc[b][4 * r4], acc[b][4 * r4 + 1],
                                                     acc[b][4 * r4 + 2], acc[b][4 * r4 + 3]);
    DPC_WAIT_VMCNT(0);
    __syncthreads();
    if (tid == 0) split_publish(tickets + 3 * set, op, my_xcc);
    return;
  }
  // The records phase reads this item's blocks back from its own area as well
  // (a rolled loop over the blocks cannot index the accumulator registers).
#pragma unroll
  for (int b = 0; b < kB; ++b)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      mine[(b * 4 + r4) * 64 + lane] = make_float4(acc[b][4 * r4], acc[b][4 * r4 + 1],
                                                   acc[b][4 * r4 + 2], acc[b][4 * r4 + 3]);
  if (tid == 0) split_await(tickets + 3 * set, op, my_xcc, ticket_lds);
  DPC_WAIT_VMCNT(0);
  __syncthreads();
  if (ticket_lds[1])
    asm volatile("buffer_inv sc0" ::: "memory");  // drop stale lines from this CU's L1
  else
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const bool timed_out = ticket_lds[2] != 0;

  const int nka = ceil_div(din, kGK), nkg = ceil_div(dout, kGK);
  const double gA = dpc_chain_gamma((double)nka * kGK, DPC_GRAM_U_MFMA);
  const double gQ = dpc_chain_gamma((double)nkg * kGK, DPC_GRAM_U_MFMA);
  // The statistics are taken with x = this item's entries and y = the
  // partner's, and the words of the two roles are swapped at the end when
  // this item holds G (op 1): the A role's row weights come from A's chain.
  const int kx = op == 0 ? nka : nkg, ky = op == 0 ? nkg : nka;
  const double etaX = (double)kx * kGK * 0x1.0p-125, etaY = (double)ky * kGK * 0x1.0p-125;
  const double invX = dpc_row_inv(op == 0 ? gA : gQ), invY = dpc_row_inv(op == 0 ? gQ : gA);
  if (lane < kGsMaxPairs * kRecStat)
    red[((lane / kRecStat) * kSplitWaves + W) * kRecStat + lane % kRecStat] = 0.0;
  // Both items' blocks are read back from the exchange area, one block
  // ahead of their use: the accumulators are dead after their publication,
  // and six blocks of both operands would not fit the registers at once.
  auto load_block = [&](const float4* src, int b) __attribute__((always_inline)) {
    f32x16_t o;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const float4 x = src[(b * 4 + r4) * 64 + lane];
      o[4 * r4] = x.x;
      o[4 * r4 + 1] = x.y;
      o[4 * r4 + 2] = x.z;
      o[4 * r4 + 3] = x.w;
    }
    return o;
  };
  // Lane-local sums per tile pair (blocks in order), then one cross-lane sum
  // per pair the wave touches and word its blocks can make non-zero.
  // Words: 0 sum x y, 1 / 2 off-diagonal x^2 / y^2, 3 wx^2 |y_ss|,
  // 4 wy^2 |x_ss|, 5 wx^2, 6 wy^2.
  constexpr int kLocal = gs_nlocal(M, W);
  double tv[kLocal][kWords];
#pragma unroll
  for (int u = 0; u < kLocal; ++u)
#pragma unroll
    for (int k = 0; k < kWords; ++k) tv[u][k] = 0.0;
  // A rolled loop over the blocks: unrolled, the compiler hoists the reads
  // and fp64 conversions of all blocks and runs out of registers.
  f32x16_t next_x = load_block(mine, 0), next_y = load_block(theirs, 0);
#pragma unroll 1
  for (int b = 0; b < kB; ++b) {
    const f32x16_t x16 = next_x, y16 = next_y;
    if (b + 1 < kB) {
      next_x = load_block(mine, b + 1);
      next_y = load_block(theirs, b + 1);
    }
    const int ru = gs_unit(W, gs_row_slot(M, W, b)), cu = gs_unit(W, gs_col_slot(M, W, b));
    const bool dblk = ru == cu;
    // Weight 2 (exact) for a block above a diagonal tile's diagonal: it
    // stands for its mirror as well.
    const double wgt = ((ru >> 2) == (cu >> 2) && ru < cu) ? 2.0 : 1.0;
    double v[kRecStat] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    float dx = 0.0f, dy = 0.0f;
    bool has_diag = false;
    // Four entries at a time (the scheduler would otherwise convert all 32
    // of the block to fp64 first and run out of registers).
#pragma unroll
    for (int r0 = 0; r0 < 16; r0 += 4) {
#pragma unroll
      for (int r = r0; r < r0 + 4; ++r) {
        const double x = x16[r], y = y16[r];
        v[0] += x * y;
        const bool on_diag = dblk && ((r >> 2) * 8 + 4 * (lane >> 5) + (r & 3)) == (lane & 31);
        v[1] += on_diag ? 0.0 : x * x;
        v[2] += on_diag ? 0.0 : y * y;
        dx = on_diag ? x16[r] : dx;
        dy = on_diag ? y16[r] : dy;
        has_diag = has_diag || on_diag;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (kWords == kRecStat && has_diag) {
      const double wx = dpc_row_bound_inv(dx, invX, etaX, DPC_GRAM_ROW_SLACK_MFMA);
      const double wy = dpc_row_bound_inv(dy, invY, etaY, DPC_GRAM_ROW_SLACK_MFMA);
      v[3] = wx * wx * fabs((double)dy);
      v[4] = wy * wy * fabs((double)dx);
      v[5] = wx * wx;
      v[6] = wy * wy;
    }
    v[0] *= wgt;
    v[1] *= wgt;
    v[2] *= wgt;
#pragma unroll
    for (int u = 0; u < kLocal; ++u) {
      const bool mine = gs_local(M, W, b) == u;
#pragma unroll
      for (int k = 0; k < kWords; ++k) tv[u][k] = mine ? tv[u][k] + v[k] : tv[u][k];
    }
  }
#pragma unroll
  for (int u = 0; u < kLocal; ++u) {
    const int pair = gs_local_pair(M, W, u);
    if (op == 1) {  // this item holds G: y is A
      double t = tv[u][1];
      tv[u][1] = tv[u][2];
      tv[u][2] = t;
      if (kWords == kRecStat) {
        t = tv[u][3];
        tv[u][3] = tv[u][4];
        tv[u][4] = t;
        t = tv[u][5];
        tv[u][5] = tv[u][6];
        tv[u][6] = t;
      }
    }
#pragma unroll
    for (int k = 0; k < kWords; ++k) {
      const double x = wave_sum_lane63_f64(tv[u][k]);
      if (lane == 63) red[(pair * kSplitWaves + W) * kRecStat + k] = x;
    }
  }
  __syncthreads();

  // Records of the segment's tile pairs (nt = 1..3 tiles of 128 rows).
  const int nt = ceil_div(n, kGramTile), npairs = nt * (nt + 1) / 2;
  if (tid < npairs * DPC_GRAM_REC_WORDS) {
    const int u = tid / DPC_GRAM_REC_WORDS, k = tid % DPC_GRAM_REC_WORDS;
    double val;
    if (k < kRecStat) {
      val = 0.0;
      for (int i = 0; i < kSplitWaves; ++i) val += red[(u * kSplitWaves + i) * kRecStat + k];
      // The off-diagonal tile pairs (0, 1), (0, 2), (1, 2) count twice (exact).
      const bool offdiag = u == 1 || u == 3 || u == 4;
      if (k == 0 && offdiag) val *= 2.0;
    } else {
      val = k == 7 ? gA : k == 8 ? gQ : k == 9 ? (double)n : 0.0;
    }
    if (timed_out && k < kRecStat) val = __builtin_nan("");
    rec[(size_t)u * DPC_GRAM_REC_WORDS + k] = val;
  }
}

// Grouped split launch: item l is (problem | op << 8 | set << 9, first row,
// rows, record slot) -- operand op of the rows-long segment starting at
// `first row` of problem `problem`, whose records start at `record slot`; the
// segment's two items share tickets[3 set ..] and their exchange area.  Items
// of a segment sit on one XCD (the host's placement), padding items are -1.
__global__ void __launch_bounds__(512, 1)
gram_gsplit_bf16_kernel(GramItems work, int nblocks, double* __restrict__ records,
                        int32_t* __restrict__ tickets, float* __restrict__ xbuf) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * 3 * kGramTile * 64 * 2];
  __shared__ double red[kGsMaxPairs * kSplitWaves * kRecStat];
  __shared__ int ticket_lds[3];
  const int l = xcd_logical_block(gridDim.x, nblocks);
  if (l < 0) return;  // padding workgroup: exits before any barrier
  const int32_t* it = work.items + 4 * (size_t)l;
  const int w0 = __builtin_amdgcn_readfirstlane(it[0]);
  if (w0 < 0) return;  // empty item: exits before any barrier
  const int problem = w0 & 0xff, op = (w0 >> 8) & 1, set = w0 >> 9;
  const int row0 = __builtin_amdgcn_readfirstlane(it[1]);
  const int n = __builtin_amdgcn_readfirstlane(it[2]);
  const int slot = __builtin_amdgcn_readfirstlane(it[3]);
  const int din = work.din[problem], dout = work.dout[problem];
  const int d = op == 0 ? din : dout;
  const uint16_t* X =
      reinterpret_cast<const uint16_t*>(op == 0 ? work.a_ptrs[problem] : work.g_ptrs[problem]) +
      (size_t)row0 * d;
  double* rec = records + (size_t)slot * DPC_GRAM_REC_WORDS;
  int xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  xcc &= 0xf;
  if (threadIdx.x == 0)
    __hip_atomic_store(&tickets[3 * set + 1 + op], xcc + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int units = ceil_div(n, 32);
#define DPC_GS_CASE(Wc)                                                                        \
  case Wc:                                                                                     \
    if (units <= 8)                                                                            \
      gsplit_item<Wc, 8>(X, n, d, din, dout, op, set, rec, tickets, xbuf, lds, red, ticket_lds, \
                         xcc);                                                                 \
    else if (units == 9)                                                                       \
      gsplit_item<Wc, 9>(X, n, d, din, dout, op, set, rec, tickets, xbuf, lds, red, ticket_lds, \
                         xcc);                                                                 \
    else                                                                                       \
      gsplit_item<Wc, 10>(X, n, d, din, dout, op, set, rec, tickets, xbuf, lds, red,           \
                          ticket_lds, xcc);                                                    \
    break;
  switch (w) {
    DPC_GS_CASE(0)
    DPC_GS_CASE(1)
    DPC_GS_CASE(2)
    DPC_GS_CASE(3)
    DPC_GS_CASE(4)
    DPC_GS_CASE(5)
    DPC_GS_CASE(6)
    default:
      DPC_GS_CASE(7)
  }
#undef DPC_GS_CASE
}

// Generic path (float32 inputs, or bf16 with d % 8 != 0): 64 x 64 tiles,
// fp64 FMA with a 4 x 4 register block per thread (products of fp32 values
// are exact in fp64, so the Gram entries carry only fp64 summation error).
constexpr int kGenTile = 64;
constexpr int kGenK = 16;

template <typename In>
__device__ __forceinline__ float load_as_f32(const In* p);
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const uint16_t* p) {
  return bf16_bits_to_f32(*p);
}

template <typename In>
__device__ void gram_tile_generic(const In* __restrict__ X, int T, int d, int p, int q,
                                  float (*sp)[kGenTile + 1], float (*sq)[kGenTile + 1],
                                  double acc[4][4]) {
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
  for (int k0 = 0; k0 < d; k0 += kGenK) {
    for (int e = tid; e < kGenTile * kGenK; e += kGramThreads) {
      int r = e / kGenK, k = e % kGenK;
      int rp = p * kGenTile + r, rq = q * kGenTile + r, kk = k0 + k;
      sp[k][r] = (rp < T && kk < d) ? load_as_f32(X + (size_t)rp * d + kk) : 0.f;
      sq[k][r] = (rq < T && kk < d) ? load_as_f32(X + (size_t)rq * d + kk) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kGenK; ++k) {
      double a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = sp[k][tr * 4 + i];
        b[i] = sq[k][tc * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
}

// Record statistics of one 64 x 64 generic sub-tile (p, q): thread (tr, tc)
// holds rows tr * 4 + i, columns tc * 4 + j, so the diagonal entries of a
// diagonal sub-tile are those with tr == tc and i == j.
__device__ __forceinline__ void generic_tile_stats(const double pa[4][4], const double pg[4][4],
                                                   bool diag_tile, double gA, double gQ,
                                                   double (&st)[kRecStat]) {
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      gram_entry_stats(pa[i][j], pg[i][j], diag_tile && tr == tc && i == j, gA, 0.0, gQ, 0.0,
                       0.0, st);
}

template <typename In>
__global__ void __launch_bounds__(kGramThreads)
gram_generic_kernel(const In* __restrict__ A, const In* __restrict__ G, int T, int din, int dout,
                    int npairs, double* __restrict__ records) {
  __shared__ float sp[kGenK][kGenTile + 1];
  __shared__ float sq[kGenK][kGenTile + 1];
  __shared__ double red[kRecStat * (kGramThreads / 64)];
  const int pair = blockIdx.x, ex = blockIdx.y;
  int p, q;
  pair_from_index(pair, &p, &q);
  double pa[4][4], pg[4][4];
  gram_tile_generic<In>(A + (size_t)ex * T * din, T, din, p, q, sp, sq, pa);
  gram_tile_generic<In>(G + (size_t)ex * T * dout, T, dout, p, q, sp, sq, pg);
  const double gA = dpc_chain_gamma((double)ceil_div(din, kGenK) * kGenK, DPC_GRAM_U_FP64);
  const double gQ = dpc_chain_gamma((double)ceil_div(dout, kGenK) * kGenK, DPC_GRAM_U_FP64);
  double st[kRecStat] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  generic_tile_stats(pa, pg, p == q, gA, gQ, st);
  if (p != q) st[0] *= 2.0;
  write_gram_record(st, red, records + ((size_t)ex * npairs + pair) * DPC_GRAM_REC_WORDS, gA, gQ,
                    T);
}

// Grouped generic path: one 128-row tile pair (P, Q) as its four 64-row
// sub-tile pairs; the record statistics of the sub-tiles add up to the pair's.
template <typename In>
__global__ void __launch_bounds__(kGramThreads)
gram_grouped_generic_kernel(GramItems work, double* __restrict__ records) {
  __shared__ float sp[kGenK][kGenTile + 1];
  __shared__ float sq[kGenK][kGenTile + 1];
  __shared__ double red[kRecStat * (kGramThreads / 64)];
  const int l = blockIdx.x;
  const int32_t* it = work.items + 4 * (size_t)l;
  if (it[0] < 0) return;  // empty item
  const int problem = it[0] >> 16, row0 = it[1], rows = it[2], slot = it[3];
  int P, Q;
  pair_from_index(it[0] & 0xffff, &P, &Q);
  const int din = work.din[problem], dout = work.dout[problem];
  const In* Xa = reinterpret_cast<const In*>(work.a_ptrs[problem]) + (size_t)row0 * din;
  const In* Xg = reinterpret_cast<const In*>(work.g_ptrs[problem]) + (size_t)row0 * dout;
  const double gA = dpc_chain_gamma((double)ceil_div(din, kGenK) * kGenK, DPC_GRAM_U_FP64);
  const double gQ = dpc_chain_gamma((double)ceil_div(dout, kGenK) * kGenK, DPC_GRAM_U_FP64);
  double st[kRecStat] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  for (int sub = 0; sub < 4; ++sub) {
    const int p = 2 * P + (sub >> 1), q = 2 * Q + (sub & 1);
    double pa[4][4], pg[4][4];
    gram_tile_generic<In>(Xa, rows, din, p, q, sp, sq, pa);
    gram_tile_generic<In>(Xg, rows, dout, p, q, sp, sq, pg);
    generic_tile_stats(pa, pg, p == q, gA, gQ, st);
  }
  if (P != Q) st[0] *= 2.0;
  write_gram_record(st, red, records + (size_t)slot * DPC_GRAM_REC_WORDS, gA, gQ, rows);
}

// dpc_gram_bound's fold of an example's nt (nt + 1) / 2 records by one wave:
// lane j takes pairs j, j + 64, ..., and the five partial sums are added by
// DPP row moves in a fixed order (wave_sum_all_f64: every lane gets the
// totals), so the result does not depend on timing; it differs from the serial fold only in the
// order of its fp64 additions of non-negative terms, which the bound's final
// 1 + 2^-40 covers.  Returns the bound; *sum = the inner products' sum.
__device__ __forceinline__ double gram_bound_wave(const double* rec, int nt, double* sum) {
  const int lane = threadIdx.x & 63;
  const int np = nt * (nt + 1) / 2;
  double v[5] = {0.0, 0.0, 0.0, 0.0, 0.0};  // sum, X, Y, W2, V2
  for (int j = lane; j < np; j += 64) {
    int p, q;
    pair_from_index(j, &p, &q);
    const double* r = rec + (size_t)j * DPC_GRAM_REC_WORDS;
    v[0] += r[0];
    if (p == q) {
      v[1] += r[3] + r[5] * sqrt(r[2]);
      v[2] += r[4] + r[6] * sqrt(r[1]);
      v[3] += r[5];
      v[4] += r[6];
    } else {
      const double* dp = rec + (size_t)(p * (p + 3) / 2) * DPC_GRAM_REC_WORDS;
      const double* dq = rec + (size_t)(q * (q + 3) / 2) * DPC_GRAM_REC_WORDS;
      v[1] += 2.0 * sqrt(dp[5] * dq[5] * r[2]);
      v[2] += 2.0 * sqrt(dp[6] * dq[6] * r[1]);
    }
  }
#pragma unroll
  for (int k = 0; k < 5; ++k) v[k] = wave_sum_all_f64(v[k]);
  *sum = v[0];
  const double gA = rec[7], gQ = rec[8], T = rec[9];
  const double g64 = (T * T + 256.0) * 0x1.0p-52;
  const double err =
      gA * v[1] + gQ * v[2] + (gA * gQ + g64 * (1.0 + gA) * (1.0 + gQ)) * v[3] * v[4];
  return err * (1.0 + 0x1.0p-40);
}

// Dense finish, one wave per example: sqnorm[b] (+)= the fold of example b's
// record inner products (+ the bias term), sqerr[b] (+)= its error bound (+
// the bias term's).  bias (nullable): [B] squared norms then [B] error
// bounds.
__global__ void __launch_bounds__(kGramThreads)
gram_finish_kernel(const double* __restrict__ records, int B, int nt, int nlayers,
                   int accumulate, const double* __restrict__ bias, double* __restrict__ sqnorm,
                   double* __restrict__ sqerr) {
  const int b = blockIdx.x * (kGramThreads / 64) + (int)(threadIdx.x >> 6);
  if (b >= B) return;
  const size_t np = (size_t)nt * (nt + 1) / 2;
  // Layers' records one after the other (B examples each), added in layer
  // order as consecutive accumulating calls would.
  double v = 0.0, ev = 0.0;
  for (int L = 0; L < nlayers; ++L) {
    double s;
    const double e = gram_bound_wave(
        records + ((size_t)L * B + (size_t)b) * np * DPC_GRAM_REC_WORDS, nt, &s);
    const bool first = L == 0 && !accumulate;
    v = first ? s : (L == 0 ? sqnorm[b] : v) + s;
    ev = first ? e : (L == 0 && sqerr ? sqerr[b] : ev) + e;
  }
  if ((threadIdx.x & 63) != 0) return;
  if (bias) v = v + bias[b];
  sqnorm[b] = v;
  if (sqerr) {
    if (bias) ev = ev + bias[B + b];
    sqerr[b] = ev;
  }
}

// Grouped finish, one wave per segment: seg_sq[v] / seg_err[v] (nullable)
// from segment v's records (slots item_start[v] .. item_start[v + 1] - 1, in
// pair order).
__global__ void __launch_bounds__(kGramThreads)
segment_finish_kernel(const double* __restrict__ records, const int32_t* __restrict__ item_start,
                      int S, double* __restrict__ seg_sq, double* __restrict__ seg_err) {
  const int v = blockIdx.x * (kGramThreads / 64) + (int)(threadIdx.x >> 6);
  if (v >= S) return;
  const int first = item_start[v], np = item_start[v + 1] - first;
  double s = 0.0, e = 0.0;
  if (np > 0) {
    int nt = 0;
    while ((nt + 1) * (nt + 2) / 2 <= np) ++nt;
    e = gram_bound_wave(records + (size_t)first * DPC_GRAM_REC_WORDS, nt, &s);
  }
  if ((threadIdx.x & 63) != 0) return;
  seg_sq[v] = s;
  if (seg_err) seg_err[v] = e;
}

// ||sum_t G_i[t]||^2 for a bias: one workgroup per example, columns strided
// over threads, column sums in fp32 (as the reference's per-example bias
// gradient, and in the order bias_partial_kernel sums them, so the value
// measured is the value summed), squares summed in fp64.  out[ex] = the
// squared norm, out[B + ex] = its error bound: the fp64 sum of exact squares
// and the fp32 product scale * column of the clipped sum, 2^-21 relative.
template <typename In>
__global__ void __launch_bounds__(kGramThreads)
bias_sqnorm_kernel(const In* __restrict__ G, int B, int T, int dout, double* __restrict__ out) {
  __shared__ double red[kGramThreads / 64];
  const int ex = blockIdx.x;
  const In* g = G + (size_t)ex * T * dout;
  double s = 0.0;
  for (int m = threadIdx.x; m < dout; m += blockDim.x) {
    float col = 0.f;
    for (int t = 0; t < T; ++t) col += load_as_f32(g + (size_t)t * dout + m);
    s += (double)col * (double)col;
  }
  double total = block_sum_f64(s, red);
  if (threadIdx.x == 0) {
    out[ex] = total;
    out[B + ex] = total * 0x1.0p-21;
  }
}

// Flat inputs: ||a||^2 ||g||^2 (+ ||g||^2 with a bias), each a fp64 sum of
// exact squares; the error bound is (din + dout + 512) 2^-50 relative (the
// fp64 sums, the product and the bias addition).
template <typename In>
__global__ void __launch_bounds__(kGramThreads)
flat_sqnorm_kernel(const In* __restrict__ a, const In* __restrict__ g, int din, int dout,
                   int with_bias, int accumulate, double* __restrict__ sqnorm,
                   double* __restrict__ sqerr) {
  __shared__ double red[kGramThreads / 64];
  const int ex = blockIdx.x;
  double sa = 0.0, sg = 0.0;
  for (int k = threadIdx.x; k < din; k += blockDim.x) {
    double v = (double)load_as_f32(a + (size_t)ex * din + k);
    sa += v * v;
  }
  double ta = block_sum_f64(sa, red);
  for (int k = threadIdx.x; k < dout; k += blockDim.x) {
    double v = (double)load_as_f32(g + (size_t)ex * dout + k);
    sg += v * v;
  }
  double tg = block_sum_f64(sg, red);
  if (threadIdx.x == 0) {
    double v = ta * tg + (with_bias ? tg : 0.0);
    sqnorm[ex] = accumulate ? sqnorm[ex] + v : v;
    if (sqerr) {
      const double e = fabs(v) * ((double)din + (double)dout + 512.0) * 0x1.0p-50;
      sqerr[ex] = accumulate ? sqerr[ex] + e : e;
    }
  }
}

__global__ void __launch_bounds__(kGramThreads)
row_sum_f64_kernel(const double* __restrict__ x, int B, int n, int accumulate,
                   double* __restrict__ out) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  double s = 0.0;
  for (int j = 0; j < n; ++j) s += x[(size_t)b * n + j];
  out[b] = accumulate ? out[b] + s : s;
}

}  // namespace

namespace {
// Workspace of dpc_gram_sqnorms: the tile records (sized for the generic
// path's 64-row tiles, which bound the MFMA paths' counts) and the bias
// terms; when T spans an even number of 128-row blocks, then the split
// mode's tickets (a counter and the two items' XCDs per tile set) and
// accumulator exchange area (both operands' accumulators of every set), each
// 256-byte aligned.
size_t gram_records_bytes(int B, int T) {
  const int nt = ceil_div(T, kGenTile);
  const size_t npairs = (size_t)nt * (nt + 1) / 2;
  return (npairs * (size_t)B * DPC_GRAM_REC_WORDS + 2 * (size_t)B) * sizeof(double);
}
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
bool split_shape(int T) { return ceil_div(T, kGramTile) % 2 == 0; }
size_t split_tickets_bytes(int B, int T) {
  return align256((size_t)3 * B * split_sets_per_example(ceil_div(T, kGramTile)) * sizeof(int32_t));
}
}  // namespace

extern "C" size_t dpc_gram_workspace_bytes(int B, int T) {
  if (B <= 0 || T <= 0) return 0;
  size_t n = align256(gram_records_bytes(B, T));
  if (split_shape(T))
    n += split_tickets_bytes(B, T) +
         (size_t)B * split_sets_per_example(ceil_div(T, kGramTile)) * 2 * kSplitSetBytes;
  return n;
}

extern "C" int dpc_gram_sqnorms(const void* A, const void* G, int B, int T, int din, int dout,
                                int dtype, int with_bias, int accumulate, double* sqnorm,
                                double* sqerr, void* ws, size_t ws_bytes, void* stream) {
  if (B < 0 || T <= 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!A || !G || !sqnorm || !ws) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  if (ws_bytes < dpc_gram_workspace_bytes(B, T)) return DPC_ENOSPC;
  hipStream_t s = (hipStream_t)stream;
  double* records = (double*)ws;
  int nt;
  // Buffer offsets are 32-bit: one example's rows (plus a tile of padding)
  // must stay below 2 GiB for the MFMA path.
  const size_t dmax = (size_t)(din > dout ? din : dout);
  const bool fits = ((size_t)T + kGramTile) * dmax * 2 < ((size_t)1 << 31);
  const bool mfma = dtype == DPC_BF16 && din % 8 == 0 && dout % 8 == 0 && fits;
  if (mfma && split_shape(T)) {
    // One operand per work item; the tickets start at zero.
    nt = ceil_div(T, kGramTile);
    const int npairs = nt * (nt + 1) / 2;
    const int nsets = split_sets_per_example(nt);
    const int nblocks = 2 * nsets * B;
    const int padded = ceil_div(nblocks, kXcds) * kXcds;
    uint8_t* base = (uint8_t*)ws + align256(gram_records_bytes(B, T));
    int32_t* tickets = (int32_t*)base;
    float* xbuf = (float*)(base + split_tickets_bytes(B, T));
    hipLaunchKernelGGL(fill_zero_i32_kernel, dim3(ceil_div(3 * nsets * B, kGramThreads)),
                       dim3(kGramThreads), 0, s, tickets, 3 * nsets * B);
    SplitLayers lay;
    lay.n = 1;
    lay.round = 0;
    for (int i = 0; i < kSplitMaxLayers; ++i) {
      lay.A[i] = (const uint16_t*)A;
      lay.G[i] = (const uint16_t*)G;
      lay.din[i] = din;
      lay.dout[i] = dout;
      lay.region[i] = 0;
    }
    hipLaunchKernelGGL(gram_split_bf16_kernel, dim3(padded), dim3(512), 0, s, lay, B, T, npairs,
                       nsets, nblocks, records, tickets, xbuf, SplitTail{});
  } else if (mfma) {
    nt = ceil_div(T, kGramTile);
    const int npairs = nt * (nt + 1) / 2;
    const int items = dense_items_per_example(nt);
    const int nblocks = items * B;
    const int padded = ceil_div(nblocks, kXcds) * kXcds;
    hipLaunchKernelGGL(gram_mfma_bf16_kernel, dim3(padded), dim3(512), 0, s, (const uint16_t*)A,
                       (const uint16_t*)G, T, din, dout, npairs, items, nblocks, records);
  } else {
    nt = ceil_div(T, kGenTile);
    const int npairs = nt * (nt + 1) / 2;
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(gram_generic_kernel<uint16_t>, dim3(npairs, B), dim3(kGramThreads), 0,
                         s, (const uint16_t*)A, (const uint16_t*)G, T, din, dout, npairs,
                         records);
    } else {
      hipLaunchKernelGGL(gram_generic_kernel<float>, dim3(npairs, B), dim3(kGramThreads), 0, s,
                         (const float*)A, (const float*)G, T, din, dout, npairs, records);
    }
  }
  DPC_HIP_CHECK(hipGetLastError());
  double* bias = nullptr;
  if (with_bias) {
    const size_t np = (size_t)nt * (nt + 1) / 2;
    bias = records + np * (size_t)B * DPC_GRAM_REC_WORDS;
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(bias_sqnorm_kernel<uint16_t>, dim3(B), dim3(kGramThreads), 0, s,
                         (const uint16_t*)G, B, T, dout, bias);
    } else {
      hipLaunchKernelGGL(bias_sqnorm_kernel<float>, dim3(B), dim3(kGramThreads), 0, s,
                         (const float*)G, B, T, dout, bias);
    }
    DPC_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(gram_finish_kernel, dim3(ceil_div(B, kGramThreads / 64)), dim3(kGramThreads), 0,
                     s, (const double*)records, B, nt, 1, accumulate, (const double*)bias, sqnorm,
                     sqerr);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

// Workspace of dpc_grouped_gram_sqnorms: the records, the split kernel's
// tickets (3 per set) and its accumulator exchange (two operands per set).
static size_t gs_ticket_offset(int n_records) {
  return ((size_t)n_records * DPC_GRAM_REC_WORDS * sizeof(double) + 255) & ~(size_t)255;
}
static size_t gs_xbuf_offset(int n_records, int n_sets) {
  return (gs_ticket_offset(n_records) + (size_t)n_sets * 3 * sizeof(int32_t) + 255) &
         ~(size_t)255;
}

extern "C" size_t dpc_grouped_gram_workspace_bytes(int n_records, int n_sets) {
  if (n_records < 0 || n_sets < 0) return 0;
  return gs_xbuf_offset(n_records, n_sets) + (size_t)n_sets * 2 * kGsSetBytes;
}

extern "C" int dpc_grouped_gram_sqnorms(const int64_t* a_ptrs, const int64_t* g_ptrs,
                                        const int32_t* dims, int n_problems, int dtype,
                                        const int32_t* items, int n_items, int max_rows,
                                        const int32_t* set_items, int n_set_items, int n_sets,
                                        int n_records, const int32_t* seg_item_start, int S,
                                        double* seg_sq,
                                        double* seg_err, void* ws, size_t ws_bytes,
                                        void* stream) {
  if (n_problems < 1 || !dims || n_items < 0 || S < 0 || max_rows < 0 || n_set_items < 0 ||
      n_sets < 0 || n_records < 0)
    return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (n_problems > kMaxGramProblems) return DPC_ENOTSUP;
  if (S == 0) return DPC_OK;
  if (!seg_item_start || !seg_sq || (n_items > 0 && (!a_ptrs || !g_ptrs || !items || !ws)) ||
      (n_set_items > 0 && (!a_ptrs || !g_ptrs || !set_items || !ws || n_sets < 1)) ||
      (n_sets >= (1 << 22)))
    return DPC_EINVAL;
  GramItems work;
  work.items = items;
  work.a_ptrs = a_ptrs;
  work.g_ptrs = g_ptrs;
  bool aligned = true;
  int dmax = 0;
  for (int p = 0; p < kMaxGramProblems; ++p) {
    work.din[p] = p < n_problems ? dims[2 * p] : 0;
    work.dout[p] = p < n_problems ? dims[2 * p + 1] : 0;
    if (p >= n_problems) continue;
    if (work.din[p] <= 0 || work.dout[p] <= 0) return DPC_EINVAL;
    aligned = aligned && work.din[p] % 8 == 0 && work.dout[p] % 8 == 0;
    dmax = max(dmax, max(work.din[p], work.dout[p]));
  }
  // The split kernel takes bf16 segments of at most kGsMaxRows rows, whose
  // byte range fits its 32-bit buffer offsets.
  if (n_set_items > 0 &&
      (dtype != DPC_BF16 || !aligned || (size_t)kGsMaxRows * (size_t)dmax * 2 >= ((size_t)1 << 31)))
    return DPC_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  double* records = (double*)ws;
  if (n_set_items > 0) {
    if (ws_bytes < dpc_grouped_gram_workspace_bytes(n_records, n_sets)) return DPC_ENOSPC;
    int32_t* tickets = (int32_t*)((uint8_t*)ws + gs_ticket_offset(n_records));
    float* xbuf = (float*)((uint8_t*)ws + gs_xbuf_offset(n_records, n_sets));
    hipLaunchKernelGGL(fill_zero_i32_kernel, dim3(ceil_div(3 * n_sets, kGramThreads)),
                       dim3(kGramThreads), 0, s, tickets, 3 * n_sets);
    GramItems sw = work;
    sw.items = set_items;
    const int padded = ceil_div(n_set_items, kXcds) * kXcds;
    hipLaunchKernelGGL(gram_gsplit_bf16_kernel, dim3(padded), dim3(512), 0, s, sw, n_set_items,
                       records, tickets, xbuf);
    DPC_HIP_CHECK(hipGetLastError());
  } else if (ws_bytes < (size_t)n_records * DPC_GRAM_REC_WORDS * sizeof(double)) {
    return DPC_ENOSPC;
  }
  if (n_items > 0) {
    const bool fits = ((size_t)max_rows + kGramTile) * (size_t)dmax * 2 < ((size_t)1 << 31);
    if (dtype == DPC_BF16 && aligned && fits) {
      const int padded = ceil_div(n_items, kXcds) * kXcds;
      hipLaunchKernelGGL(gram_grouped_mfma_bf16_kernel, dim3(padded), dim3(256), 0, s, work,
                         n_items, records);
    } else if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(gram_grouped_generic_kernel<uint16_t>, dim3(n_items), dim3(kGramThreads),
                         0, s, work, records);
    } else {
      hipLaunchKernelGGL(gram_grouped_generic_kernel<float>, dim3(n_items), dim3(kGramThreads), 0,
                         s, work, records);
    }
    DPC_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(segment_finish_kernel, dim3(ceil_div(S, kGramThreads / 64)), dim3(kGramThreads),
                     0,
                     s, (const double*)records, seg_item_start, S, seg_sq, seg_err);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_flat_sqnorms(const void* a, const void* g, int B, int din, int dout,
                                int dtype, int with_bias, int accumulate, double* sqnorm,
                                double* sqerr, void* stream) {
  if (B < 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!a || !g || !sqnorm) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DPC_BF16) {
    hipLaunchKernelGGL(flat_sqnorm_kernel<uint16_t>, dim3(B), dim3(kGramThreads), 0, s,
                       (const uint16_t*)a, (const uint16_t*)g, din, dout, with_bias, accumulate,
                       sqnorm, sqerr);
  } else if (dtype == DPC_F32) {
    hipLaunchKernelGGL(flat_sqnorm_kernel<float>, dim3(B), dim3(kGramThreads), 0, s,
                       (const float*)a, (const float*)g, din, dout, with_bias, accumulate,
                       sqnorm, sqerr);
  } else {
    return DPC_EINVAL;
  }
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_row_sum_f64(const double* x, int B, int n, int accumulate, double* out,
                               void* stream) {
  if (B < 0 || n < 0 || (B > 0 && (!x || !out))) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  hipLaunchKernelGGL(row_sum_f64_kernel, dim3(ceil_div(B, kGramThreads)), dim3(kGramThreads), 0,
                     (hipStream_t)stream, x, B, n, accumulate, out);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

namespace {
// Compute units per XCD of the current device (cached per device; 32 on
// MI355X: 256 CUs in 8 XCDs).
int cus_per_xcd() {
  static std::atomic<int> cached[64];  // 0: not read yet (threads may race to fill it)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 32;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < kXcds)
      cus = 32 * kXcds;
    v = cus / kXcds;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Address of this device's `scratch`, looked up on the device's first call.
void* scratch_on_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    dpc_record_error(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    dpc_record_error(hipErrorInvalidDevice);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
      dpc_record_error(e);
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int dpc_gram_sqnorms_noalloc(const void* A, const void* G, int B, int T, int din,
                                        int dout, int dtype, int with_bias, int accumulate,
                                        double* sqnorm, double* sqerr, void* stream) {
  if (B < 0 || T <= 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  const size_t need = dpc_gram_workspace_bytes(B, T);
  if (need > (size_t)DPC_NOALLOC_SCRATCH_BYTES) return DPC_ENOSPC;
  void* ws = scratch_on_current_device();
  if (!ws) return DPC_EHIP;
  return dpc_gram_sqnorms(A, G, B, T, din, dout, dtype, with_bias, accumulate, sqnorm, sqerr, ws,
                          (size_t)DPC_NOALLOC_SCRATCH_BYTES, stream);
}

namespace {
// The split-mode shape of dpc_gram_sqnorms_multi: bf16, T an even number of
// 128-row blocks, B a multiple of 8, every layer on the MFMA path.
bool split_multi_shape(int n, const int* din, const int* dout, int B, int T, int dtype) {
  if (n < 2 || n > kSplitMaxLayers || dtype != DPC_BF16 || B % kXcds != 0 || !split_shape(T))
    return false;
  for (int i = 0; i < n; ++i) {
    const size_t dmax = (size_t)(din[i] > dout[i] ? din[i] : dout[i]);
    if (din[i] % 8 != 0 || dout[i] % 8 != 0 || ((size_t)T + kGramTile) * dmax * 2 >= ((size_t)1 << 31))
      return false;
  }
  return true;
}
size_t split_multi_bytes(int n, int B, int T) {
  const int nt = ceil_div(T, kGramTile);
  const size_t npairs = (size_t)nt * (nt + 1) / 2, nsets = split_sets_per_example(nt);
  return align256((size_t)n * B * npairs * DPC_GRAM_REC_WORDS * sizeof(double)) +
         align256((size_t)n * 3 * nsets * B * sizeof(int32_t)) +
         (size_t)n * B * nsets * 2 * kSplitSetBytes;
}
}  // namespace

extern "C" size_t dpc_gram_sqnorms_multi_workspace_bytes(int n, const int* din, const int* dout,
                                                        int B, int T, int dtype) {
  if (n <= 0 || B <= 0 || T <= 0 || !din || !dout) return 0;
  const size_t one = dpc_gram_workspace_bytes(B, T);
  if (!split_multi_shape(n, din, dout, B, T, dtype)) return one;
  const size_t multi = split_multi_bytes(n, B, T);
  return multi > one ? multi : one;
}

extern "C" int dpc_gram_sqnorms_multi(int n, const void* const* A, const void* const* G,
                                      const int* din, const int* dout, int B, int T, int dtype,
                                      int accumulate, double* sqnorm, double* sqerr, void* ws,
                                      size_t ws_bytes, void* stream) {
  if (n < 0 || B < 0 || T <= 0) return DPC_EINVAL;
  if (n == 0 || B == 0) return DPC_OK;
  if (!A || !G || !din || !dout || !sqnorm || !ws) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  for (int i = 0; i < n; ++i)
    if (!A[i] || !G[i] || din[i] <= 0 || dout[i] <= 0) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  if (ws_bytes < dpc_gram_sqnorms_multi_workspace_bytes(n, din, dout, B, T, dtype))
    return DPC_ENOSPC;
  if (!split_multi_shape(n, din, dout, B, T, dtype)) {
    // Layer by layer, each accumulating into the previous layers' sums.
    for (int i = 0; i < n; ++i) {
      const int r = dpc_gram_sqnorms(A[i], G[i], B, T, din[i], dout[i], dtype, 0,
                                     i == 0 ? accumulate : 1, sqnorm, sqerr, ws, ws_bytes, stream);
      if (r != DPC_OK) return r;
    }
    return DPC_OK;
  }
  hipStream_t s = (hipStream_t)stream;
  const int nt = ceil_div(T, kGramTile);
  const int npairs = nt * (nt + 1) / 2;
  const int nsets = split_sets_per_example(nt);
  const int nblocks = n * 2 * nsets * B;  // a multiple of 8: B is
  uint8_t* base = (uint8_t*)ws;
  double* records = (double*)base;
  base += align256((size_t)n * B * npairs * DPC_GRAM_REC_WORDS * sizeof(double));
  int32_t* tickets = (int32_t*)base;
  base += align256((size_t)n * 3 * nsets * B * sizeof(int32_t));
  float* xbuf = (float*)base;
  // Table order: the layers with the longest K loops first (within each
  // XCD's range they run first, the short ones fill the end); region = the
  // caller's index, so the finish adds the layers in the caller's order.
  int order[kSplitMaxLayers];
  for (int i = 0; i < n; ++i) order[i] = i;
  std::stable_sort(order, order + n, [&](int a, int b) {
    return (long long)din[a] + dout[a] > (long long)din[b] + dout[b];
  });
  SplitLayers lay;
  lay.n = n;
  lay.round = cus_per_xcd();
  for (int k = 0; k < kSplitMaxLayers; ++k) {
    const int i = order[k < n ? k : 0];
    lay.A[k] = (const uint16_t*)A[i];
    lay.G[k] = (const uint16_t*)G[i];
    lay.din[k] = din[i];
    lay.dout[k] = dout[i];
    lay.region[k] = i;
  }
  const int nticket = n * 3 * nsets * B;
  hipLaunchKernelGGL(fill_zero_i32_kernel, dim3(ceil_div(nticket, kGramThreads)),
                     dim3(kGramThreads), 0, s, tickets, nticket);
  hipLaunchKernelGGL(gram_split_bf16_kernel, dim3(nblocks), dim3(512), 0, s, lay, B, T, npairs,
                     nsets, nblocks, records, tickets, xbuf, SplitTail{});
  DPC_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(gram_finish_kernel, dim3(ceil_div(B, kGramThreads / 64)), dim3(kGramThreads), 0,
                     s, (const double*)records, B, nt, n, accumulate, (const double*)nullptr,
                     sqnorm, sqerr);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

namespace {
bool gram_clip_one_launch(int B, int T, int din, int dout, int dtype, int with_bias) {
  const size_t dmax = (size_t)(din > dout ? din : dout);
  // The tail's LDS holds one example's records, then B flag words.
  const size_t nt = (size_t)ceil_div(T, kGramTile), np = nt * (nt + 1) / 2;
  const size_t lds_doubles = (size_t)(4 * 3 * kGTileBytes) / sizeof(double);
  return dtype == DPC_BF16 && !with_bias && din % 8 == 0 && dout % 8 == 0 && split_shape(T) &&
         B <= kSplitTailMaxB && ((size_t)T + kGramTile) * dmax * 2 < ((size_t)1 << 31) &&
         np * DPC_GRAM_REC_WORDS <= lds_doubles && (size_t)B <= 2 * lds_doubles;
}
}  // namespace

extern "C" size_t dpc_gram_clip_workspace_bytes(int B, int T) {
  return dpc_gram_workspace_bytes(B, T);
}

extern "C" size_t dpc_gram_clip_counter_bytes(int B, int T) {
  if (B <= 0 || T <= 0) return 0;
  const int nsets = split_shape(T) ? split_sets_per_example(ceil_div(T, kGramTile)) : 0;
  // The split kernel's tickets, one counter per example, the example counter.
  return (size_t)(3 * (size_t)B * nsets + (size_t)B + 1) * sizeof(int32_t);
}

extern "C" int dpc_gram_clip_factors(const void* A, const void* G, int B, int T, int din,
                                     int dout, int dtype, int with_bias, double C, int kind,
                                     double gamma, const double* guard_rel,
                                     const double* guard_abs, const int* guard_mult, int n_guards,
                                     float count_threshold, double* sqnorm, double* sqerr,
                                     float* scale, double* scale64, float* norms_out,
                                     int* nclipped, void* plan, int* nonfinite, void* ws,
                                     size_t ws_bytes, int32_t* counters, size_t counter_bytes,
                                     void* stream) {
  if (B < 0 || T <= 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!A || !G || !sqnorm || !ws) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  if (ws_bytes < dpc_gram_clip_workspace_bytes(B, T)) return DPC_ENOSPC;
  ClipJob job;
  int r = clip_job_from_args(C, kind, gamma, guard_rel, guard_abs, guard_mult, n_guards,
                             count_threshold, scale, scale64, norms_out, nclipped, plan, nonfinite,
                             &job);
  if (r != DPC_OK) return r;
  if (!gram_clip_one_launch(B, T, din, dout, dtype, with_bias)) {
    // The norms and the clip factors as separate launches (the counters
    // are not used).
    r = dpc_gram_sqnorms(A, G, B, T, din, dout, dtype, with_bias, 0, sqnorm, sqerr, ws, ws_bytes,
                         stream);
    if (r != DPC_OK) return r;
    return dpc_clip_factors(sqnorm, sqerr, B, C, kind, gamma, guard_rel, guard_abs, guard_mult,
                            n_guards, count_threshold, scale, scale64, norms_out, nclipped, plan,
                            nonfinite, stream);
  }
  if (!counters) return DPC_EINVAL;
  if (counter_bytes < dpc_gram_clip_counter_bytes(B, T)) return DPC_ENOSPC;
  hipStream_t s = (hipStream_t)stream;
  const int nt = ceil_div(T, kGramTile);
  const int npairs = nt * (nt + 1) / 2;
  const int nsets = split_sets_per_example(nt);
  const int nblocks = 2 * nsets * B;
  const int padded = ceil_div(nblocks, kXcds) * kXcds;
  uint8_t* base = (uint8_t*)ws;
  double* records = (double*)base;
  // The exchange area where dpc_gram_sqnorms keeps it (after the records
  // and its own ticket words, unused here).
  float* xbuf = (float*)(base + align256(gram_records_bytes(B, T)) + split_tickets_bytes(B, T));
  const int n_tickets = 3 * nsets * B;
  SplitLayers lay;
  lay.n = 1;
  lay.round = 0;
  for (int i = 0; i < kSplitMaxLayers; ++i) {
    lay.A[i] = (const uint16_t*)A;
    lay.G[i] = (const uint16_t*)G;
    lay.din[i] = din;
    lay.dout[i] = dout;
    lay.region[i] = 0;
  }
  SplitTail tail;
  tail.ex_done = counters + n_tickets;
  tail.done = tail.ex_done + B;
  tail.sqnorm = sqnorm;
  tail.sqerr = sqerr;
  tail.job = job;
  hipLaunchKernelGGL(gram_split_bf16_kernel, dim3(padded), dim3(512), 0, s, lay, B, T, npairs,
                     nsets, nblocks, records, counters, xbuf, tail);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
