// Per-example squared gradient norms of linear layers via the Gram identity
//   ||G_i^T A_i||_F^2 = <A_i A_i^T, G_i G_i^T>
// (no per-example gradient is ever formed).  The T x T Gram matrices are
// split into 128 x 128 tiles; a workgroup owns one (example, tile pair p <= q).
// Its 8 waves form two groups of 4: group 0 computes the (p, q) tile of
// A A^T while group 1 computes the same tile of G G^T, concurrently, with
// bf16 MFMA and fp32 accumulators (each wave 64 x 64 of the tile).  Group 1
// then hands its tile to group 0 through LDS for the element-wise inner
// product in fp64.  Pairs with p < q count twice (both Gram matrices are
// symmetric).  One fp64 partial per (example, pair) lands in the workspace;
// dpc_row_sum_f64 folds them into sqnorm in a fixed order, so results are
// deterministic.
//
// Workgroups are placed so that all pairs of one example run on one XCD
// (hardware dispatch is round-robin over the 8 XCDs): the pairs re-read the
// example's tiles from that XCD's L2 instead of from HBM.
#include "common.h"

namespace {

constexpr int kGramTile = 128;  // rows of a T-tile
constexpr int kGramK = 64;      // reduction depth staged per LDS buffer
constexpr int kGramThreads = 256;
constexpr int kGramGroupThreads = 256;                   // one group = 4 waves
constexpr int kGramMfmaThreads = 2 * kGramGroupThreads;  // A group + G group
constexpr int kTileBytes = kGramTile * kGramK * 2;       // 16 KiB per staged tile
constexpr int kStageBytes = 2 * kTileBytes;              // p tile + q tile
constexpr int kGroupBytes = 2 * kStageBytes;             // two stages
constexpr int kXcds = 8;

// Byte offset of 16-byte chunk `c` of row `r` in a [rows][64] bf16 LDS tile.
// The XOR swizzle spreads both the row-chunk writes and the MFMA fragment
// reads (32 consecutive rows, one chunk) over all 32 banks.
__device__ __forceinline__ int lds_off(int r, int c) {
  return r * 128 + ((c ^ ((r ^ (r >> 3)) & 7)) << 4);
}

__device__ __forceinline__ void pair_from_index(int pair, int* p, int* q) {
  int qq = 0;
  while ((qq + 1) * (qq + 2) / 2 <= pair) ++qq;
  *q = qq;
  *p = pair - qq * (qq + 1) / 2;
}

// Load 128 rows x 64 columns (bf16) starting at (row0, k0) of X [T, d]:
// four 16-byte chunks per group thread, zero outside [T) x [d).
__device__ __forceinline__ void gram_load(const uint16_t* __restrict__ X, int T, int d, int row0,
                                          int k0, int gt, u32x4_t regs[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int q = gt + kGramGroupThreads * j;
    int r = q >> 3, c = q & 7;
    int row = row0 + r, col = k0 + c * 8;
    if (row < T && col < d) {
      regs[j] = *reinterpret_cast<const u32x4_t*>(X + (size_t)row * d + col);
    } else {
      regs[j] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
}

__device__ __forceinline__ void gram_store(uint8_t* tile, int gt, const u32x4_t regs[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int q = gt + kGramGroupThreads * j;
    *reinterpret_cast<u32x4_t*>(tile + lds_off(q >> 3, q & 7)) = regs[j];
  }
}

// acc[bi][bj] += X[p rows] X[q rows]^T over one staged 64-deep slab; wave wg
// of the group owns rows wr * 64.. of p and wr * 64.. of q.
__device__ __forceinline__ void gram_mma(const uint8_t* lp, const uint8_t* lq, int wg,
                                         f32x16_t acc[2][2]) {
  const int lane = threadIdx.x & 63;
  const int wr = wg >> 1, wc = wg & 1;
#pragma unroll
  for (int kk = 0; kk < kGramK / 16; ++kk) {
    const int c = kk * 2 + (lane >> 5);
    bf16x8_t a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a[i] = *reinterpret_cast<const bf16x8_t*>(lp + lds_off(wr * 64 + i * 32 + (lane & 31), c));
      b[i] = *reinterpret_cast<const bf16x8_t*>(lq + lds_off(wc * 64 + i * 32 + (lane & 31), c));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
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

// Linear workgroup id -> logical (example, pair) index so that each XCD
// receives a contiguous range of logical indices.  `padded` is the grid size
// (a multiple of kXcds); returns -1 for padding workgroups.
__device__ __forceinline__ int xcd_logical_block(int padded, int nblocks) {
  const int b = blockIdx.x;
  const int per = padded / kXcds;
  const int l = (b % kXcds) * per + b / kXcds;
  return l < nblocks ? l : -1;
}

__global__ void __launch_bounds__(kGramMfmaThreads, 1)
gram_mfma_bf16_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ G, int T,
                      int din, int dout, int npairs, int nblocks, double* __restrict__ partial) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kGroupBytes];
  __shared__ double red[kGramMfmaThreads / 64];
  const int l = xcd_logical_block(gridDim.x, nblocks);
  if (l < 0) return;  // padding workgroup: exits before any barrier
  const int ex = l / npairs, pair = l % npairs;
  int p, q;
  pair_from_index(pair, &p, &q);
  const bool diag = (p == q);

  const int group = threadIdx.x / kGramGroupThreads;
  const int gt = threadIdx.x % kGramGroupThreads;
  const int wg = gt >> 6;
  const int d = group ? dout : din;
  const uint16_t* X = group ? G + (size_t)ex * T * dout : A + (size_t)ex * T * din;
  uint8_t* mine = lds + group * kGroupBytes;
  const int nk_mine = ceil_div(d, kGramK);
  const int nk = max(ceil_div(din, kGramK), ceil_div(dout, kGramK));

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16_t{};

  // Register double buffer: step s + 1 is in flight while step s is multiplied
  // and step s + 2 is requested.
  u32x4_t rp0[4], rq0[4], rp1[4], rq1[4];
  auto load = [&](int step, u32x4_t* rp, u32x4_t* rq) {
    gram_load(X, T, d, p * kGramTile, step * kGramK, gt, rp);
    if (!diag) gram_load(X, T, d, q * kGramTile, step * kGramK, gt, rq);
  };
  auto store = [&](int stage, const u32x4_t* rp, const u32x4_t* rq) {
    uint8_t* st = mine + stage * kStageBytes;
    gram_store(st, gt, rp);
    if (!diag) gram_store(st + kTileBytes, gt, rq);
  };
  auto body = [&](int s, u32x4_t* rp_next, u32x4_t* rq_next, u32x4_t* rp_free,
                  u32x4_t* rq_free) {
    // rp_next/rq_next hold step s + 1; rp_free/rq_free receive step s + 2.
    if (s + 2 < nk_mine) load(s + 2, rp_free, rq_free);
    if (s < nk_mine) {
      const uint8_t* st = mine + (s & 1) * kStageBytes;
      gram_mma(st, diag ? st : st + kTileBytes, wg, acc);
    }
    if (s + 1 < nk_mine) store((s + 1) & 1, rp_next, rq_next);
    __syncthreads();
  };

  if (nk_mine > 0) load(0, rp0, rq0);
  if (nk_mine > 1) load(1, rp1, rq1);
  if (nk_mine > 0) store(0, rp0, rq0);
  __syncthreads();
  int s = 0;
  for (; s + 1 < nk; s += 2) {
    body(s, rp1, rq1, rp0, rq0);
    body(s + 1, rp0, rq0, rp1, rq1);
  }
  if (s < nk) body(s, rp1, rq1, rp0, rq0);

  // Group 1 hands its G G^T tile to group 0 through LDS (same fragment order,
  // element e of thread gt at float index e * 256 + gt).
  float* xfer = reinterpret_cast<float*>(lds);
  if (group == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) xfer[((i * 2 + j) * 16 + r) * kGramGroupThreads + gt] = acc[i][j][r];
  }
  __syncthreads();
  double sum = 0.0;
  if (group == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sum += (double)acc[i][j][r] *
                 (double)xfer[((i * 2 + j) * 16 + r) * kGramGroupThreads + gt];
  }
  double total = block_sum_f64(sum, red);
  if (threadIdx.x == 0) {
    partial[(size_t)ex * npairs + pair] = diag ? total : 2.0 * total;
  }
}

// Generic path (float32 inputs, or bf16 with d % 8 != 0): 64 x 64 tiles,
// FMA on fp32 with a 4 x 4 register block per thread.
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
                                  float acc[4][4]) {
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
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
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = sp[k][tr * 4 + i];
        b[i] = sq[k][tc * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
}

template <typename In>
__global__ void __launch_bounds__(kGramThreads)
gram_generic_kernel(const In* __restrict__ A, const In* __restrict__ G, int T, int din, int dout,
                    int npairs, double* __restrict__ partial) {
  __shared__ float sp[kGenK][kGenTile + 1];
  __shared__ float sq[kGenK][kGenTile + 1];
  __shared__ double red[kGramThreads / 64];
  const int pair = blockIdx.x, ex = blockIdx.y;
  int p, q;
  pair_from_index(pair, &p, &q);
  float pa[4][4], pg[4][4];
  gram_tile_generic<In>(A + (size_t)ex * T * din, T, din, p, q, sp, sq, pa);
  gram_tile_generic<In>(G + (size_t)ex * T * dout, T, dout, p, q, sp, sq, pg);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += (double)pa[i][j] * (double)pg[i][j];
  double total = block_sum_f64(s, red);
  if (threadIdx.x == 0) partial[(size_t)ex * npairs + pair] = (p == q) ? total : 2.0 * total;
}

// ||sum_t G_i[t]||^2 for a bias: one workgroup per example, columns strided
// over threads, column sums in fp32 (as the reference's per-example bias
// gradient), squares summed in fp64.
template <typename In>
__global__ void __launch_bounds__(kGramThreads)
bias_sqnorm_kernel(const In* __restrict__ G, int T, int dout, double* __restrict__ out) {
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
  if (threadIdx.x == 0) out[ex] = total;
}

template <typename In>
__global__ void __launch_bounds__(kGramThreads)
flat_sqnorm_kernel(const In* __restrict__ a, const In* __restrict__ g, int din, int dout,
                   int with_bias, int accumulate, double* __restrict__ sqnorm) {
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

extern "C" size_t dpc_gram_workspace_bytes(int B, int T) {
  if (B <= 0 || T <= 0) return 0;
  // Tile counts for the generic path (64-row tiles) bound the MFMA path's.
  int nt = ceil_div(T, kGenTile);
  size_t npairs = (size_t)nt * (nt + 1) / 2;
  return (npairs * (size_t)B + (size_t)B) * sizeof(double);
}

extern "C" int dpc_gram_sqnorms(const void* A, const void* G, int B, int T, int din, int dout,
                                int dtype, int with_bias, int accumulate, double* sqnorm,
                                void* ws, size_t ws_bytes, void* stream) {
  if (B < 0 || T <= 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!A || !G || !sqnorm || !ws) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  if (ws_bytes < dpc_gram_workspace_bytes(B, T)) return DPC_ENOSPC;
  hipStream_t s = (hipStream_t)stream;
  double* partial = (double*)ws;
  int npairs;
  const bool mfma = dtype == DPC_BF16 && din % 8 == 0 && dout % 8 == 0;
  if (mfma) {
    int nt = ceil_div(T, kGramTile);
    npairs = nt * (nt + 1) / 2;
    const int nblocks = npairs * B;
    const int padded = ceil_div(nblocks, kXcds) * kXcds;
    hipLaunchKernelGGL(gram_mfma_bf16_kernel, dim3(padded), dim3(kGramMfmaThreads), 0, s,
                       (const uint16_t*)A, (const uint16_t*)G, T, din, dout, npairs, nblocks,
                       partial);
  } else {
    int nt = ceil_div(T, kGenTile);
    npairs = nt * (nt + 1) / 2;
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(gram_generic_kernel<uint16_t>, dim3(npairs, B), dim3(kGramThreads), 0,
                         s, (const uint16_t*)A, (const uint16_t*)G, T, din, dout, npairs,
                         partial);
    } else {
      hipLaunchKernelGGL(gram_generic_kernel<float>, dim3(npairs, B), dim3(kGramThreads), 0, s,
                         (const float*)A, (const float*)G, T, din, dout, npairs, partial);
    }
  }
  DPC_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(row_sum_f64_kernel, dim3(ceil_div(B, kGramThreads)), dim3(kGramThreads), 0,
                     s, partial, B, npairs, accumulate, sqnorm);
  DPC_HIP_CHECK(hipGetLastError());
  if (with_bias) {
    double* bias_sq = partial + (size_t)npairs * B;
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(bias_sqnorm_kernel<uint16_t>, dim3(B), dim3(kGramThreads), 0, s,
                         (const uint16_t*)G, T, dout, bias_sq);
    } else {
      hipLaunchKernelGGL(bias_sqnorm_kernel<float>, dim3(B), dim3(kGramThreads), 0, s,
                         (const float*)G, T, dout, bias_sq);
    }
    DPC_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(row_sum_f64_kernel, dim3(ceil_div(B, kGramThreads)), dim3(kGramThreads),
                       0, s, bias_sq, B, 1, 1, sqnorm);
    DPC_HIP_CHECK(hipGetLastError());
  }
  return DPC_OK;
}

extern "C" int dpc_flat_sqnorms(const void* a, const void* g, int B, int din, int dout,
                                int dtype, int with_bias, int accumulate, double* sqnorm,
                                void* stream) {
  if (B < 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!a || !g || !sqnorm) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DPC_BF16) {
    hipLaunchKernelGGL(flat_sqnorm_kernel<uint16_t>, dim3(B), dim3(kGramThreads), 0, s,
                       (const uint16_t*)a, (const uint16_t*)g, din, dout, with_bias, accumulate,
                       sqnorm);
  } else if (dtype == DPC_F32) {
    hipLaunchKernelGGL(flat_sqnorm_kernel<float>, dim3(B), dim3(kGramThreads), 0, s,
                       (const float*)a, (const float*)g, din, dout, with_bias, accumulate,
                       sqnorm);
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
