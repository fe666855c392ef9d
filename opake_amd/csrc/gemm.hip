// Clipped batch sum of a linear layer's per-example weight gradients,
//   out[m, n] = sum_i scale[i] * sum_t G[i, t, m] * A[i, t, n],
// as one GEMM over K = B * T with the normalisation and the Gaussian noise
// fused into the epilogue.
//
// Fast path (bf16, T % 64 == 0, din % 8 == 0, dout % 8 == 0):
//   * 256 x 256 output tile per workgroup, 4 waves of 128 x 128, bf16 MFMA
//     32x32x16 with fp32 accumulators (16 blocks per wave);
//   * operands are stored m- (n-) contiguous in HBM; each thread loads an
//     8 (k) x 8 (m) block with 16-byte loads, transposes it in registers and
//     writes 8 k-contiguous rows into an XOR-swizzled LDS tile, so the MFMA
//     fragment reads are single 16-byte LDS loads without bank conflicts;
//   * two LDS stages (128 KiB), one barrier per 64-deep K step, the next
//     step's global loads in flight during the current step's MFMAs;
//   * a K step never straddles two examples, so the per-example scale is one
//     scalar per step: it multiplies the G operand in fp32 during the
//     register transpose and the product is rounded to bf16 once
//     (v_cvt_pk_bf16_f32, round-to-nearest-even) -- the same single rounding
//     of a scaled value that the reference applies when it stores a scaled
//     bf16 per-example gradient.  The accumulators never leave the AGPRs.
//     Examples with scale 0 are skipped through the clip plan, so their data
//     (including any NaN/Inf) is never read;
//   * workgroup ids are remapped so that each of the 8 XCDs owns a compact
//     block of output tiles and re-reads operand tiles from its own L2.
#include "common.h"
#include "plan.h"

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 64, kThreads = 256;

// LDS layout of one 256-row operand tile for a 64-deep K step.  A 16-byte
// chunk holds 8 consecutive k of one row; chunk kb (0..7) of row r lives at
//   (kb >> 1) * kSlice + (kb & 1) * kHalf + 16 * (r + (r >> 3)).
// MFMA fragment reads (32 consecutive rows, one chunk) are then contiguous
// 16-byte runs, and fragment (i, kk) sits at a constant offset from a
// per-lane base; the transposed writes (rows 8 apart across lanes) land
// 144 bytes apart, which spreads 8 lanes over all 32 banks.
constexpr int kHalf = (kBM + kBM / 8) * 16;      // 4608 bytes
constexpr int kSlice = 2 * kHalf;                // 16 k per slice
constexpr int kOperandBytes = 4 * kSlice;        // 36 KiB
constexpr int kStageBytes = 2 * kOperandBytes;   // G tile + A tile

__device__ __forceinline__ int row_off(int r) { return 16 * (r + (r >> 3)); }

struct Epilogue {
  int M, N;
  float nb;
  int apply_nb;
  int noise_mode;
  const float* noise;
  uint64_t seed;
  uint32_t leaf;
  float sigma;
  int out_bf16;
  void* out;
};

#pragma clang fp contract(off)
// to_out(v); optional to_out(v / nb); optional to_out(v + sigma * z).
__device__ __forceinline__ float finish_value(float v, const Epilogue& ep, float z) {
  const bool bf = ep.out_bf16 != 0;
  if (bf) v = round_to_bf16(v);
  if (ep.apply_nb) {
    v = v / ep.nb;
    if (bf) v = round_to_bf16(v);
  }
  if (ep.sigma != 0.0f) {
    float t = ep.sigma * z;
    v = v + t;
    if (bf) v = round_to_bf16(v);
  }
  return v;
}
#pragma clang fp contract(on)

__device__ __forceinline__ void store_value(const Epilogue& ep, size_t idx, float v) {
  if (ep.out_bf16) {
    reinterpret_cast<uint16_t*>(ep.out)[idx] = f32_to_bf16_bits(v);
  } else {
    reinterpret_cast<float*>(ep.out)[idx] = v;
  }
}

// Writes rows m and m + 1 (m even) of column n from two accumulator values.
__device__ __forceinline__ void emit_pair(const Epilogue& ep, int m, int n, float v0, float v1) {
  if (n >= ep.N || m >= ep.M) return;
  float z0 = 0.0f, z1 = 0.0f;
  if (ep.sigma != 0.0f) {
    if (ep.noise_mode == DPC_NOISE_PHILOX) {
      philox_normal_pair(ep.seed, ep.leaf, (uint64_t)(m >> 1) * (uint64_t)ep.N + (uint64_t)n,
                         &z0, &z1);
    } else {
      z0 = ep.noise[(size_t)m * ep.N + n];
      if (m + 1 < ep.M) z1 = ep.noise[(size_t)(m + 1) * ep.N + n];
    }
  }
  store_value(ep, (size_t)m * ep.N + n, finish_value(v0, ep, z0));
  if (m + 1 < ep.M) store_value(ep, (size_t)(m + 1) * ep.N + n, finish_value(v1, ep, z1));
}

// 8 rows (k) x 8 columns of bf16 at byte offset `off` -> regs[k]; the row
// stride enters as a scalar offset.  A chunk outside the matrix columns is
// given an offset past the buffer's range, which the hardware reads as zero.
constexpr int kOutOfRange = 0x7ff00000;

__device__ __forceinline__ void load_block(__amdgpu_buffer_rsrc_t rsrc, int off, int row_bytes,
                                           u32x4_t regs[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    regs[r] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, r * row_bytes, 0);
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// The same transpose with every element multiplied by `s` in fp32 and
// rounded to bf16 (RNE) on the way.
__device__ __forceinline__ void store_block_t_scaled(uint8_t* tile, int mb, int kb,
                                                     const u32x4_t in[8], float s) {
  uint8_t* base = tile + (kb >> 1) * kSlice + (kb & 1) * kHalf + row_off(mb * 8);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = j >> 1;
    u32x4_t o;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t x = in[2 * t][c], y = in[2 * t + 1][c];
      uint32_t xb = (j & 1) ? (x & 0xffff0000u) : (x << 16);
      uint32_t yb = (j & 1) ? (y & 0xffff0000u) : (y << 16);
      f32x2_t v = {__builtin_bit_cast(float, xb) * s, __builtin_bit_cast(float, yb) * s};
      o[t] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    }
    *reinterpret_cast<u32x4_t*>(base + 16 * j) = o;
  }
}

// Transpose the 8 x 8 bf16 block in registers and store row j (operand row
// mb * 8 + j, k-chunk kb) of the LDS tile.
__device__ __forceinline__ void store_block_t(uint8_t* tile, int mb, int kb, const u32x4_t in[8]) {
  uint8_t* base = tile + (kb >> 1) * kSlice + (kb & 1) * kHalf + row_off(mb * 8);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = j >> 1;
    u32x4_t o;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t x = in[2 * t][c], y = in[2 * t + 1][c];
      o[t] = (j & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
    }
    *reinterpret_cast<u32x4_t*>(base + 16 * j) = o;
  }
}

// One 64-deep K step of MFMAs over the staged G and A tiles.
__device__ __forceinline__ void mma_stage(const uint8_t* tg, const uint8_t* ta,
                                          f32x16_t acc[4][4]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  const uint8_t* ga = tg + (lane >> 5) * kHalf + row_off(wm * 128 + (lane & 31));
  const uint8_t* aa = ta + (lane >> 5) * kHalf + row_off(wn * 128 + (lane & 31));
#pragma unroll
  for (int kk = 0; kk < kBK / 16; ++kk) {
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = *reinterpret_cast<const bf16x8_t*>(ga + kk * kSlice + i * row_off(32));
      b[i] = *reinterpret_cast<const bf16x8_t*>(aa + kk * kSlice + i * row_off(32));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// blockIdx -> (tile_m, tile_n): contiguous id ranges per XCD (hardware
// dispatch is round-robin over the 8 XCDs), then GROUP_M-ordered tiles so a
// group of tile rows shares the activation tiles.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int* tm, int* tn) {
  const int ntiles = tiles_m * tiles_n;
  int lin = blockIdx.x;
  if (ntiles % 8 == 0) lin = (lin % 8) * (ntiles / 8) + lin / 8;
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = lin % per_group;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

struct FastArgs {
  const uint16_t* A;  // [B * T, N]
  const uint16_t* G;  // [B * T, M]
  int T, B;
  const void* plan;
  const float* scale;
  Epilogue ep;
};

__global__ void __launch_bounds__(kThreads, 1) clipped_sum_bf16_kernel(FastArgs args) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStageBytes];
  static_assert(128 * (kBN + 4) * 4 <= 2 * kStageBytes, "epilogue tile fits");
  const int M = args.ep.M, N = args.ep.N, T = args.T;
  int tm, tn;
  tile_coords(ceil_div(M, kBM), ceil_div(N, kBN), &tm, &tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int mb = tid & 31, kb = tid >> 5;
  const bool g_ok = m0 + mb * 8 < M, a_ok = n0 + mb * 8 < N;

  ClipPlanView plan = clip_plan_view(const_cast<void*>(args.plan), args.B);
  const int nactive = *plan.nactive;
  const int spe = T / kBK;
  const int nsteps = nactive * spe;

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  if (nsteps > 0) {
    const int total_rows = args.B * T;
    __amdgpu_buffer_rsrc_t g_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(args.G), (short)0, total_rows * M * 2, 0x00020000);
    __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(args.A), (short)0, total_rows * N * 2, 0x00020000);
    const int g_col = (m0 + mb * 8) * 2, a_col = (n0 + mb * 8) * 2;
    const int g_bad = g_ok ? 0 : kOutOfRange, a_bad = a_ok ? 0 : kOutOfRange;
    u32x4_t rg[8], ra[8];
    int slot = 0, kt = 0;
    int ex = plan.active[0];
    int row = ex * T + kb * 8;
    load_block(g_rsrc, (row * M * 2 + g_col) | g_bad, M * 2, rg);
    load_block(a_rsrc, (row * N * 2 + a_col) | a_bad, N * 2, ra);
    store_block_t_scaled(lds, mb, kb, rg, args.scale[ex]);
    store_block_t(lds + kOperandBytes, mb, kb, ra);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
      uint8_t* cur = lds + (s & 1) * kStageBytes;
      uint8_t* nxt = lds + ((s + 1) & 1) * kStageBytes;
      int nslot = slot, nkt = kt + 1;
      if (nkt == spe) {
        nkt = 0;
        ++nslot;
      }
      const bool more = s + 1 < nsteps;
      float nscale = 0.0f;
      if (more) {
        const int nex = plan.active[nslot];
        nscale = args.scale[nex];
        const int nrow = nex * T + nkt * kBK + kb * 8;
        load_block(g_rsrc, (nrow * M * 2 + g_col) | g_bad, M * 2, rg);
        load_block(a_rsrc, (nrow * N * 2 + a_col) | a_bad, N * 2, ra);
      }
      mma_stage(cur, cur + kOperandBytes, acc);
      if (more) {
        store_block_t_scaled(nxt, mb, kb, rg, nscale);
        store_block_t(nxt + kOperandBytes, mb, kb, ra);
      }
      __syncthreads();
      slot = nslot;
      kt = nkt;
    }
  }

  // Epilogue: the 256 x 256 fp32 tile goes through LDS in two halves of 128
  // rows (128 KiB + padding fits in the 160 KiB LDS), then each thread owns one
  // column and walks its rows in even/odd pairs: coalesced stores, and one
  // Philox block per pair in a rolled loop (no per-element code expansion).
  const int wm = w >> 1, wn = w & 1;
  float* tile = reinterpret_cast<float*>(lds);
  constexpr int kLd = kBN + 4;
  for (int half = 0; half < 2; ++half) {
    if (wm == half) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ml = i * 32 + (r >> 2) * 8 + 4 * (lane >> 5) + (r & 3);
            const int nl = wn * 128 + j * 32 + (lane & 31);
            tile[ml * kLd + nl] = acc[i][j][r];
          }
    }
    __syncthreads();
    const int n = n0 + tid;
#pragma unroll 2
    for (int ml = 0; ml < 128; ml += 2) {
      emit_pair(args.ep, m0 + half * 128 + ml, n, tile[ml * kLd + tid], tile[(ml + 1) * kLd + tid]);
    }
    __syncthreads();
  }
}

// Generic path: any T, float32 or bf16 operands, scale applied to the G
// operand in fp32; 64 x 64 tiles with a 4 x 4 FMA block per thread.
constexpr int kGT = 64, kGK = 16;

template <typename In>
__device__ __forceinline__ float to_f32(In v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_bits_to_f32(v); }

template <typename In>
__global__ void __launch_bounds__(kThreads)
clipped_sum_generic_kernel(const In* __restrict__ A, const In* __restrict__ G,
                           const float* __restrict__ scale, int B, int T, Epilogue ep) {
  __shared__ float sg[kGK][kGT + 1];
  __shared__ float sa[kGK][kGT + 1];
  const int M = ep.M, N = ep.N;
  const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long long K = (long long)B * T;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (long long k0 = 0; k0 < K; k0 += kGK) {
    for (int e = tid; e < kGK * kGT; e += kThreads) {
      const int k = e / kGT, col = e % kGT;
      const long long kk = k0 + k;
      float gv = 0.f, av = 0.f;
      if (kk < K) {
        const float s = scale[kk / T];
        if (s > 0.0f) {
          if (m0 + col < M) gv = s * to_f32<In>(G[kk * M + m0 + col]);
          if (n0 + col < N) av = to_f32<In>(A[kk * N + n0 + col]);
        }
      }
      sg[k][col] = gv;
      sa[k][col] = av;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kGK; ++k) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = sg[k][tr * 4 + i];
        b[i] = sa[k][tc * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + tc * 4 + j;
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      emit_pair(ep, m0 + tr * 4 + i, n, acc[i][j], acc[i + 1][j]);
    }
  }
}

// Bias: partial[split][m] = sum over examples e of the split of
// scale[e] * sum_t G[e, t, m]; the finishing kernel adds the splits in order.
constexpr int kBiasSplits = 32;

template <typename In>
__global__ void __launch_bounds__(kThreads)
bias_partial_kernel(const In* __restrict__ G, const float* __restrict__ scale, int B, int T, int M,
                    int nsplit, float* __restrict__ partial) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  const int split = blockIdx.y;
  if (m >= M) return;
  const int per = ceil_div(B, nsplit);
  const int e0 = split * per, e1 = min(B, e0 + per);
  float acc = 0.f;
  for (int e = e0; e < e1; ++e) {
    const float s = scale[e];
    if (!(s > 0.0f)) continue;
    float col = 0.f;
    for (int t = 0; t < T; ++t) col += to_f32<In>(G[((size_t)e * T + t) * M + m]);
    acc += s * col;
  }
  partial[(size_t)split * M + m] = acc;
}

__global__ void __launch_bounds__(kThreads)
bias_finish_kernel(const float* __restrict__ partial, int nsplit, Epilogue ep) {
  // Rows are handled in even/odd pairs so the Philox pairing matches the
  // [M, 1] view of the bias leaf.
  const int m = 2 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (m >= ep.M) return;
  float v0 = 0.f, v1 = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    v0 += partial[(size_t)s * ep.M + m];
    if (m + 1 < ep.M) v1 += partial[(size_t)s * ep.M + m + 1];
  }
  emit_pair(ep, m, 0, v0, v1);
}

}  // namespace

extern "C" size_t dpc_clipped_sum_workspace_bytes(int B, int T, int din, int dout, int dtype) {
  (void)B;
  (void)T;
  (void)din;
  (void)dtype;
  if (dout <= 0) return 0;
  return (size_t)kBiasSplits * (size_t)dout * sizeof(float);
}

extern "C" int dpc_clipped_sum(const void* A, const void* G, const float* scale, const void* plan,
                               int B, int T, int din, int dout, int dtype, double normalize_by,
                               int noise_mode, const float* noise, const float* bias_noise,
                               uint64_t seed, uint32_t leaf_id, uint32_t bias_leaf_id,
                               double sigma, int out_dtype,
                               void* out, int with_bias, void* bias_out, void* ws,
                               size_t ws_bytes, void* stream) {
  if (B < 0 || T <= 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (out_dtype != DPC_F32 && out_dtype != DPC_BF16) return DPC_EINVAL;
  if (!(normalize_by > 0.0)) return DPC_EINVAL;
  if (noise_mode < DPC_NOISE_NONE || noise_mode > DPC_NOISE_PHILOX) return DPC_EINVAL;
  if (!out || (B > 0 && (!A || !G || !scale))) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  if (!(sigma >= 0.0)) return DPC_EINVAL;
  if (sigma != 0.0 && noise_mode == DPC_NOISE_NONE) return DPC_EINVAL;
  if (sigma != 0.0 && noise_mode == DPC_NOISE_INJECTED && (!noise || (with_bias && !bias_noise)))
    return DPC_EINVAL;
  if (with_bias && (!bias_out || !ws || ws_bytes < dpc_clipped_sum_workspace_bytes(B, T, din, dout, dtype)))
    return with_bias && !bias_out ? DPC_EINVAL : DPC_ENOSPC;
  hipStream_t s = (hipStream_t)stream;

  Epilogue ep;
  ep.M = dout;
  ep.N = din;
  ep.nb = (float)normalize_by;
  ep.apply_nb = normalize_by != 1.0;
  ep.noise_mode = sigma != 0.0 ? noise_mode : DPC_NOISE_NONE;
  ep.noise = noise;
  ep.seed = seed;
  ep.leaf = leaf_id;
  ep.sigma = (float)sigma;
  ep.out_bf16 = out_dtype == DPC_BF16;
  ep.out = out;

  // Buffer offsets are 32-bit: each operand must stay below 2 GiB.
  const size_t rows = (size_t)B * (size_t)T;
  const bool small = rows * (size_t)(din > dout ? din : dout) * 2 < ((size_t)1 << 31);
  const bool fast = dtype == DPC_BF16 && T % kBK == 0 && din % 8 == 0 && dout % 8 == 0 &&
                    plan != nullptr && B > 0 && small;
  if (fast) {
    FastArgs args;
    args.A = (const uint16_t*)A;
    args.G = (const uint16_t*)G;
    args.T = T;
    args.B = B;
    args.plan = plan;
    args.scale = scale;
    args.ep = ep;
    const int ntiles = ceil_div(dout, kBM) * ceil_div(din, kBN);
    hipLaunchKernelGGL(clipped_sum_bf16_kernel, dim3(ntiles), dim3(kThreads), 0, s, args);
  } else {
    dim3 grid(ceil_div(din, kGT), ceil_div(dout, kGT));
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(clipped_sum_generic_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                         (const uint16_t*)A, (const uint16_t*)G, scale, B, T, ep);
    } else {
      hipLaunchKernelGGL(clipped_sum_generic_kernel<float>, grid, dim3(kThreads), 0, s,
                         (const float*)A, (const float*)G, scale, B, T, ep);
    }
  }
  DPC_HIP_CHECK(hipGetLastError());

  if (with_bias) {
    const int nsplit = B > 0 ? min(B, kBiasSplits) : 1;
    float* partial = (float*)ws;
    dim3 grid(ceil_div(dout, kThreads), nsplit);
    if (B > 0) {
      if (dtype == DPC_BF16) {
        hipLaunchKernelGGL(bias_partial_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                           (const uint16_t*)G, scale, B, T, dout, nsplit, partial);
      } else {
        hipLaunchKernelGGL(bias_partial_kernel<float>, grid, dim3(kThreads), 0, s,
                           (const float*)G, scale, B, T, dout, nsplit, partial);
      }
      DPC_HIP_CHECK(hipGetLastError());
    }
    Epilogue eb = ep;
    eb.M = dout;
    eb.N = 1;
    eb.noise = bias_noise;
    eb.leaf = bias_leaf_id;
    eb.out = bias_out;
    hipLaunchKernelGGL(bias_finish_kernel, dim3(ceil_div(ceil_div(dout, 2), kThreads)),
                       dim3(kThreads), 0, s, (const float*)partial, B > 0 ? nsplit : 0, eb);
    DPC_HIP_CHECK(hipGetLastError());
  }
  return DPC_OK;
}
