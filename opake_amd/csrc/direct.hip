// Per-example weight gradients of linear layers with a narrow side (LoRA
// adapters: rank r <= 32 on one side),
//   out[b, m, n] = sum_t G[b, t, m] * A[b, t, n]      (out is [B, dout, din]),
// materialised in fp32: for such layers the per-example gradient is small and
// cheaper to form (2 T din dout FLOP) than its Gram norm (T^2 (din + dout)).
//
// One operand is wide (W columns), the other narrow (ns <= 32 columns).  Both
// kernels keep, per thread, 4 adjacent wide columns x NS narrow columns of
// fp32 sums; the chunk's narrow rows sit in LDS, where every lane of a wave
// reads the same words (a broadcast).  Memory bound: the wide operand is read
// once.
//
// bf16 with W % 4 == 0 (narrow_wide_bf16_kernel): a workgroup of 8 waves owns
// 256 wide columns of one example and a chunk of its tokens, split between the
// waves.  Each lane keeps 8 token pairs of 8-byte loads in flight (a register
// ring, loads past the wave's range read zeros, so the loop has no branch
// around them), about 64 KiB per CU; tokens go in pairs through
// v_dot2_f32_bf16.  The waves' sums are added in wave order through LDS, so a
// chunk needs no more splits than it takes to fill the CUs: wide layers write
// the result directly, narrow-wide ones a few fp32 partials.
//
// Other inputs (narrow_partial_kernel, narrow_partial_bf16_kernel): a
// workgroup of 4 waves owns 1024 wide columns and a chunk of <= 256 tokens,
// one load per thread and token.
//
// Token chunks write fp32 partial sums, added in chunk order by a second
// kernel that also lays out (and rounds) the result.
#include <algorithm>
#include <vector>

#include "common.h"
#include "lds_stage.h"

namespace {

constexpr int kDirThreads = 256;
constexpr int kWidePerThread = 4;
constexpr int kWidePerBlock = kDirThreads * kWidePerThread;
constexpr int kMaxNarrow = 32;
constexpr int kMaxChunk = 256;  // tokens per chunk (LDS: kMaxChunk * 32 floats)
constexpr int kUnroll = 4;

template <typename In>
__device__ __forceinline__ float dir_f32(In v);
template <>
__device__ __forceinline__ float dir_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float dir_f32<uint16_t>(uint16_t v) { return bf16_bits_to_f32(v); }

// Four wide values of row `row` starting at column w0 (w0 + 3 < nw, w0 % 4 == 0
// and nw % 4 == 0: one aligned load), else element by element with zeros.
template <typename In>
__device__ __forceinline__ void load_wide4(const In* row, int w0, int nw, bool vec, float x[4]);

template <>
__device__ __forceinline__ void load_wide4<uint16_t>(const uint16_t* row, int w0, int nw, bool vec,
                                                     float x[4]) {
  if (vec) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + w0);
    x[0] = __builtin_bit_cast(float, v.x << 16);
    x[1] = __builtin_bit_cast(float, v.x & 0xffff0000u);
    x[2] = __builtin_bit_cast(float, v.y << 16);
    x[3] = __builtin_bit_cast(float, v.y & 0xffff0000u);
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = (w0 + j < nw) ? bf16_bits_to_f32(row[w0 + j]) : 0.f;
}

template <>
__device__ __forceinline__ void load_wide4<float>(const float* row, int w0, int nw, bool vec,
                                                  float x[4]) {
  if (vec) {
    const float4 v = *reinterpret_cast<const float4*>(row + w0);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = (w0 + j < nw) ? row[w0 + j] : 0.f;
}

// partial[split][b][s][w] = sum over tokens t of chunk `split` of
// narrow[b, t, s] * wide[b, t, w].
template <typename In, int NS>
__global__ void __launch_bounds__(kDirThreads)
narrow_partial_kernel(const In* __restrict__ wide, const In* __restrict__ narrow, int B, int T,
                      int nw, int ns, int chunk, float* __restrict__ partial) {
  __shared__ float nl[kMaxChunk * NS];
  const int b = blockIdx.y, split = blockIdx.z;
  const int w0 = blockIdx.x * kWidePerBlock + threadIdx.x * kWidePerThread;
  const int t0 = split * chunk, t1 = min(T, t0 + chunk), n = max(t1 - t0, 0);
  // Narrow rows of the chunk -> LDS (fp32, zero past ns).
  for (int i = threadIdx.x; i < n * NS; i += kDirThreads) {
    const int t = i / NS, s = i % NS;
    nl[i] = s < ns ? dir_f32<In>(narrow[((size_t)b * T + t0 + t) * ns + s]) : 0.f;
  }
  __syncthreads();
  float acc[NS][kWidePerThread];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int j = 0; j < kWidePerThread; ++j) acc[s][j] = 0.f;
  const bool vec = (nw % 4 == 0) && (w0 + 3 < nw);
  const In* wbase = wide + ((size_t)b * T + t0) * nw;
  int t = 0;
  for (; t + kUnroll <= n; t += kUnroll) {
    float x[kUnroll][4];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load_wide4<In>(wbase + (size_t)(t + u) * nw, w0, nw, vec, x[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float v = nl[(t + u) * NS + s];
#pragma unroll
        for (int j = 0; j < kWidePerThread; ++j) acc[s][j] = fmaf(v, x[u][j], acc[s][j]);
      }
  }
  for (; t < n; ++t) {
    float x[4];
    load_wide4<In>(wbase + (size_t)t * nw, w0, nw, vec, x);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float v = nl[t * NS + s];
#pragma unroll
      for (int j = 0; j < kWidePerThread; ++j) acc[s][j] = fmaf(v, x[j], acc[s][j]);
    }
  }
  if (w0 >= nw) return;
  float* out = partial + (((size_t)split * B + b) * ns) * nw;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (s < ns) {
#pragma unroll
      for (int j = 0; j < kWidePerThread; ++j)
        if (w0 + j < nw) out[(size_t)s * nw + w0 + j] = acc[s][j];
    }
  }
}

// bf16 inputs: tokens go in pairs through v_dot2_f32_bf16 (two products
// and the fp32 sum per instruction, half the VALU work of fp32 FMAs).  The
// chunk's narrow rows are staged in LDS as (t, t + 1) bf16 pairs per narrow
// column; the wide rows t and t + 1 are re-paired per column with byte
// permutes.  A missing last token of an odd chunk is zero.
typedef __bf16 dir_bf16x2_t __attribute__((ext_vector_type(2)));

template <int NS>
__global__ void __launch_bounds__(kDirThreads)
narrow_partial_bf16_kernel(const uint16_t* __restrict__ wide, const uint16_t* __restrict__ narrow,
                           int B, int T, int nw, int ns, int chunk, float* __restrict__ partial) {
  __shared__ uint32_t nl2[(kMaxChunk / 2) * NS];
  const int b = blockIdx.y, split = blockIdx.z;
  const int w0 = blockIdx.x * kWidePerBlock + threadIdx.x * kWidePerThread;
  const int t0 = split * chunk, t1 = min(T, t0 + chunk), n = max(t1 - t0, 0);
  const int npairs = (n + 1) / 2;
  for (int i = threadIdx.x; i < npairs * NS; i += kDirThreads) {
    const int tp = i / NS, s = i % NS;
    uint32_t lo = 0, hi = 0;
    if (s < ns) {
      lo = narrow[((size_t)b * T + t0 + 2 * tp) * ns + s];
      if (2 * tp + 1 < n) hi = narrow[((size_t)b * T + t0 + 2 * tp + 1) * ns + s];
    }
    nl2[i] = lo | (hi << 16);
  }
  __syncthreads();
  float acc[NS][kWidePerThread];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int j = 0; j < kWidePerThread; ++j) acc[s][j] = 0.f;
  const bool vec = (nw % 4 == 0) && (w0 + 3 < nw);
  const uint16_t* wbase = wide + ((size_t)b * T + t0) * nw;
  auto load4 = [&](int t, uint2* v) __attribute__((always_inline)) {
    if (t >= n) {
      *v = make_uint2(0u, 0u);
    } else if (vec) {
      *v = *reinterpret_cast<const uint2*>(wbase + (size_t)t * nw + w0);
    } else {
      uint32_t e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = (w0 + j < nw) ? wbase[(size_t)t * nw + w0 + j] : 0u;
      *v = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
    }
  };
  constexpr int kPairUnroll = 2;
  for (int tp = 0; tp < npairs; tp += kPairUnroll) {
    uint2 r[kPairUnroll][2];
#pragma unroll
    for (int u = 0; u < kPairUnroll; ++u) {
      load4(2 * (tp + u), &r[u][0]);
      load4(2 * (tp + u) + 1, &r[u][1]);
    }
#pragma unroll
    for (int u = 0; u < kPairUnroll; ++u) {
      if (tp + u >= npairs) break;
      // Column j of rows (t, t + 1) as one bf16 pair.
      uint32_t wp[4];
      wp[0] = __builtin_amdgcn_perm(r[u][1].x, r[u][0].x, 0x05040100u);
      wp[1] = __builtin_amdgcn_perm(r[u][1].x, r[u][0].x, 0x07060302u);
      wp[2] = __builtin_amdgcn_perm(r[u][1].y, r[u][0].y, 0x05040100u);
      wp[3] = __builtin_amdgcn_perm(r[u][1].y, r[u][0].y, 0x07060302u);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const dir_bf16x2_t v = __builtin_bit_cast(dir_bf16x2_t, nl2[(tp + u) * NS + s]);
#pragma unroll
        for (int j = 0; j < kWidePerThread; ++j)
          acc[s][j] = __builtin_amdgcn_fdot2_f32_bf16(
              v, __builtin_bit_cast(dir_bf16x2_t, wp[j]), acc[s][j], false);
      }
    }
  }
  if (w0 >= nw) return;
  float* out = partial + (((size_t)split * B + b) * ns) * nw;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (s < ns) {
#pragma unroll
      for (int j = 0; j < kWidePerThread; ++j)
        if (w0 + j < nw) out[(size_t)s * nw + w0 + j] = acc[s][j];
    }
  }
}

// out[b] = sum of the splits, in split order, written as [dout, din]: narrow
// side G gives out[b][s][w], narrow side A gives out[b][w][s].
__global__ void __launch_bounds__(kDirThreads)
narrow_finish_kernel(const float* __restrict__ partial, int splits, int B, int nw, int ns,
                     int narrow_is_g, int out_bf16, void* __restrict__ out) {
  const size_t per = (size_t)ns * nw;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)B * per) return;
  const size_t b = idx / per, r = idx % per;
  const size_t s = r / nw, w = r % nw;
  float v = 0.f;
  for (int k = 0; k < splits; ++k) v += partial[((size_t)k * B + b) * per + r];
  const size_t o = b * per + (narrow_is_g ? s * nw + w : w * ns + s);
  if (out_bf16) {
    reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16_bits(v);
  } else {
    reinterpret_cast<float*>(out)[o] = v;
  }
}

typedef uint32_t dir_u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t dir_u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kNwWaves = 8;
constexpr int kNwThreads = kNwWaves * 64;
constexpr int kNwCols = 64 * kWidePerThread;   // wide columns per workgroup
constexpr int kNwDepth = 8;                    // token pairs in flight per lane
constexpr int kNwLdsWords = 16384;             // 64 KiB: narrow pairs, then the wave sums
constexpr int kNwOutOfRange = 0x7ff00000;      // a buffer offset past any range: reads zero

// out[b, s, w] (narrow side G) or out[b, w, s] (narrow side A) over the
// tokens of chunk `split`; with splits > 1 the fp32 partial
// partial[split][b][s][w] instead.  Requires nw % 4 == 0, T * nw * 2 <
// kNwOutOfRange and chunk <= 2 * kNwLdsWords / NS.
template <int NS>
__global__ void __launch_bounds__(kNwThreads)
narrow_wide_bf16_kernel(const uint16_t* __restrict__ wide, const uint16_t* __restrict__ narrow,
                        int B, int T, int nw, int ns, int chunk, int splits, int narrow_is_g,
                        int out_bf16, float* __restrict__ partial, void* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[kNwLdsWords];
  const int b = blockIdx.y, split = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches below
  const int col0 = blockIdx.x * kNwCols;
  const int w0 = col0 + lane * kWidePerThread;
  const int t0 = split * chunk, n = max(min(T, t0 + chunk) - t0, 0);
  const int npairs = (n + 1) >> 1;
  const int per_wave = (npairs + kNwWaves - 1) / kNwWaves;
  const int p0 = min(w * per_wave, npairs), p1 = min(p0 + per_wave, npairs);

  // Token pair p (chunk-relative) of this lane's 4 columns; pairs past the
  // wave's range, the odd last token and columns past nw read zeros.
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(wide + (size_t)b * T * nw), (short)0, T * nw * 2, 0x00020000);
  const int col_bad = (w0 < nw) ? 0 : kNwOutOfRange;
  auto issue = [&](int p, dir_u32x2_t* r) __attribute__((always_inline)) {
    const int bad0 = (p < p1) ? col_bad : kNwOutOfRange;
    const int bad1 = (p < p1 && 2 * p + 1 < n) ? col_bad : kNwOutOfRange;
    const int off = ((t0 + 2 * p) * nw + w0) * 2;
    r[0] = __builtin_amdgcn_raw_buffer_load_b64(rsrc, off | bad0, 0, 0);
    r[1] = __builtin_amdgcn_raw_buffer_load_b64(rsrc, (off + nw * 2) | bad1, 0, 0);
  };
  dir_u32x2_t ring[kNwDepth][2];
#pragma unroll
  for (int u = 0; u < kNwDepth; ++u) issue(p0 + u, ring[u]);

  // The chunk's narrow rows as (t, t + 1) bf16 pairs: lds[p * NS + s].
  const uint16_t* nb = narrow + ((size_t)b * T + t0) * ns;
  for (int i = tid; i < npairs * NS; i += kNwThreads) {
    const int p = i / NS, s = i % NS;
    uint32_t lo = 0, hi = 0;
    if (s < ns) {
      lo = nb[(size_t)(2 * p) * ns + s];
      if (2 * p + 1 < n) hi = nb[(size_t)(2 * p + 1) * ns + s];
    }
    lds[i] = lo | (hi << 16);
  }
  __syncthreads();

  float acc[NS][kWidePerThread];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int j = 0; j < kWidePerThread; ++j) acc[s][j] = 0.f;
  for (int p = p0; p < p1; p += kNwDepth) {
#pragma unroll
    for (int u = 0; u < kNwDepth; ++u) {
      // Column j of rows (t, t + 1) as one bf16 pair.
      const dir_u32x2_t r0 = ring[u][0], r1 = ring[u][1];
      uint32_t wp[4];
      wp[0] = __builtin_amdgcn_perm(r1.x, r0.x, 0x05040100u);
      wp[1] = __builtin_amdgcn_perm(r1.x, r0.x, 0x07060302u);
      wp[2] = __builtin_amdgcn_perm(r1.y, r0.y, 0x05040100u);
      wp[3] = __builtin_amdgcn_perm(r1.y, r0.y, 0x07060302u);
      issue(p + u + kNwDepth, ring[u]);
      if (p + u < p1) {
        const uint32_t* np = lds + (p + u) * NS;
#pragma unroll
        for (int g = 0; g < NS / 4; ++g) {
          const dir_u32x4_t q = *reinterpret_cast<const dir_u32x4_t*>(np + 4 * g);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            // Through a scalar: clang's __builtin_bit_cast of a vector
            // element lvalue (q[k]) reads element 0 for every k.
            const uint32_t qk = q[k];
#pragma unroll
            for (int j = 0; j < kWidePerThread; ++j)
              acc[4 * g + k][j] = __builtin_amdgcn_fdot2_f32_bf16(
                  __builtin_bit_cast(dir_bf16x2_t, qk), __builtin_bit_cast(dir_bf16x2_t, wp[j]),
                  acc[4 * g + k][j], false);
          }
        }
      }
    }
  }

  // Wave sums, added in wave order, kRound accumulators per lane at a time:
  // wave w's accumulator k of lane l at red[(w * kRound + k) * 64 + l].
  constexpr int kRound = kNwLdsWords / (kNwWaves * 64);
  constexpr int kAcc = NS * kWidePerThread;
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int f0 = 0; f0 < kAcc; f0 += kRound) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kRound; ++k)
      red[(w * kRound + k) * 64 + lane] = acc[(f0 + k) / kWidePerThread][(f0 + k) % kWidePerThread];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRound * 64 / kNwThreads; ++i) {
      const int e = tid + i * kNwThreads;
      const int k = e >> 6, l = e & 63;
      float v = 0.f;
#pragma unroll
      for (int ww = 0; ww < kNwWaves; ++ww) v += red[(ww * kRound + k) * 64 + l];
      const int f = f0 + k, s = f / kWidePerThread;
      const int col = col0 + l * kWidePerThread + f % kWidePerThread;
      if (s >= ns || col >= nw) continue;
      if (splits > 1) {
        partial[(((size_t)split * B + b) * ns + s) * nw + col] = v;
      } else {
        const size_t o = narrow_is_g ? ((size_t)b * ns + s) * nw + col : ((size_t)b * nw + col) * ns + s;
        if (out_bf16) {
          reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16_bits(v);
        } else {
          reinterpret_cast<float*>(out)[o] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA kernel (bf16, nw % 8 == 0, ns even): out[s, w] = sum_t N[t, s] W[t, w]
// is a GEMM of M = ns (<= 32), N = nw, K = the chunk's tokens, run on the
// 16x16x32 bf16 MFMA with fp32 accumulators.  A workgroup of 8 waves owns 256
// wide columns of one example; each 64-token step stages the wide tile (64
// rows of 512 bytes in the swizzled layout of tile_off, by 16-byte DMA) and
// the narrow rows (64 rows of NS bf16, by 4-byte DMA; columns past ns and
// rows past T read zeros) into one of four LDS stages, three steps ahead.
// Wave w owns wide columns 32 w .. 32 w + 31: per step it reads 2 x 2 wide
// and 2 x NS / 16 narrow fragments through ds_read_b64_tr_b16 and runs
// 4 NS / 16 MFMAs.  Each product of two bf16 is exact in fp32, as in the
// other kernels; only the summation order differs.
// ---------------------------------------------------------------------------
constexpr int kNmWaves = 8;
constexpr int kNmThreads = kNmWaves * 64;
constexpr int kNmCols = 256;                                   // wide columns per workgroup
constexpr int kNmK = 64;                                       // tokens per step
constexpr int kNmStages = 4;
constexpr int kNmWideBytes = kNmK * kTileRowBytes;             // 32 KiB
constexpr int kNmWideDma = kNmWideBytes / (kNmWaves * 1024);   // 16-byte DMAs per lane and step

// One problem of a grouped launch: up to kNmMaxSlots layers that share the
// wide operand (the LoRA A factors of the projections fed by one activation),
// each with its own narrow operand (narrow[k], ns[k] columns), written as
// out_k[b, s, w] (narrow side G) or out_k[b, w, s] (narrow side A) over the
// tokens [split * chunk, min(T, (split + 1) * chunk)) -- to out[k] when
// splits == 1, else as the fp32 partial partial[k][split][b][s][w].
// Workgroups wg_start .. wg_start + col_tiles * B * splits - 1 of the launch
// take it, column tile fastest.  Requires chunk % 64 == 0, nw % 8 == 0, every
// ns[k] even and <= NS, and (T + 64) * nw * 2 < kNwOutOfRange.
constexpr int kNmMaxProblems = 24;
constexpr int kNmMaxSlots = 3;
struct NmProblem {
  const uint16_t* wide;
  const uint16_t* narrow[kNmMaxSlots];
  void* out[kNmMaxSlots];
  float* partial[kNmMaxSlots];
  int ns[kNmMaxSlots];
  int nslots, nw, narrow_is_g;
  int col_tiles, splits, chunk;
  int wg_start;
};
// Passed by value (kernel arguments): no table upload per launch.
struct NmTable {
  NmProblem p[kNmMaxProblems];
  int n, B, T, out_bf16;
};

// kSlots narrow operands per problem (NS = 16: 3, NS = 32: 1); the LDS stage
// holds the wide tile and kSlots narrow tiles.  Every wave issues the DMAs of
// all kSlots tiles (an absent one reads zeros, from an empty range, without
// memory traffic), so the memory-counter waits are compile-time constants;
// the MFMAs and stores of absent slots are skipped.
template <int NS, int kSlots>
__global__ void __launch_bounds__(kNmThreads, 1)
narrow_wide_mfma_kernel(const NmTable tab) {
  constexpr int kRowN = NS * 2;                                 // bytes of a narrow row in LDS
  constexpr int kNarrowBytes = kNmK * kRowN;                    // 2 or 4 KiB per slot
  constexpr int kNarrowDma = kNarrowBytes / (kNmWaves * 256);   // 4-byte DMAs per lane, slot, step
  constexpr int kDma = kNmWideDma + kSlots * kNarrowDma;
  constexpr int kStage = kNmWideBytes + kSlots * kNarrowBytes;
  constexpr int kMB = NS / 16;                                  // 16-row blocks of narrow columns
  static_assert(kNarrowDma * kNmWaves * 256 == kNarrowBytes, "narrow tile split");
  static_assert(kSlots <= kNmMaxSlots && kNmStages * kStage <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kNmStages * kStage];
  const int lin = blockIdx.x;
  int pi = 0;
  for (int i = 1; i < tab.n; ++i)
    if (lin >= tab.p[i].wg_start) pi = i;
  const NmProblem& P = tab.p[pi];
  const int B = tab.B, T = tab.T;
  const int nw = P.nw, chunk = P.chunk, splits = P.splits, nslots = P.nslots;
  const int local = lin - P.wg_start;
  const int ct = local % P.col_tiles, rest = local / P.col_tiles;
  const int b = rest % B, split = rest / B;
  const uint16_t* wide = P.wide;
  const int col0 = ct * kNmCols;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t0 = split * chunk;
  const int n = max(min(T, t0 + chunk) - t0, 0);
  const int nsteps = (n + kNmK - 1) / kNmK;

  // Example b's operands; a transfer at or past the example's end (rows >= T)
  // reads zeros, and so does every transfer of an absent slot (size 0).
  const u32x4_t wrsrc = rsrc_words(wide + (size_t)b * T * nw, (uint32_t)T * nw * 2);
  u32x4_t nrsrc[kSlots];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int kk = k < nslots ? k : 0;
    nrsrc[k] = rsrc_words(P.narrow[kk] + (size_t)b * T * P.ns[kk],
                          k < nslots ? (uint32_t)T * P.ns[kk] * 2 : 0u);
  }
  // Wide: wave w's transfer j fills the 1 KiB of tile rows 2 w + 16 j and the
  // next, lane i the 16 bytes at i * 16 -- row 2 w + 16 j + i / 32, physical
  // slot i % 32, which holds the 8 columns from tile_slot_col(row, i % 32).
  // A chunk past nw reads the row's last 8 columns instead: they feed only
  // output columns that are never stored.
  const int drow = 2 * w + (lane >> 5);
  const int dcol = min(col0 + tile_slot_col(drow, lane & 31), nw - 8);
  const uint32_t wvoff = (uint32_t)((t0 + drow) * nw + dcol) * 2u;
  const uint32_t wstep = (uint32_t)kNmK * nw * 2u, wrow16 = 16u * nw * 2u;
  // Narrow slot k: wave w's transfer i fills the 256 bytes at (w * kNarrowDma
  // + i) * 256 of the slot's tile, lane l the dword at + 4 l: row r, physical
  // dword p.  With 64-byte rows (NS = 32) the two 32-byte halves are swapped
  // in rows with bit 2 set, so that a fragment read is free of bank conflicts.
  uint32_t nvoff[kSlots][kNarrowDma], nstep[kSlots];
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const int ns = k < nslots ? P.ns[k] : 0;
    nstep[k] = (uint32_t)kNmK * ns * 2u;
#pragma unroll
    for (int i = 0; i < kNarrowDma; ++i) {
      const int byte = (w * kNarrowDma + i) * 256 + 4 * lane;
      const int r = byte / kRowN, p = (byte % kRowN) / 4;
      const int d = (NS == 32) ? p ^ (((r >> 2) & 1) << 3) : p;
      nvoff[k][i] = (2 * d < ns) ? (uint32_t)((t0 + r) * ns + 2 * d) * 2u : (uint32_t)kNwOutOfRange;
    }
  }
  const uint32_t lds0 = lds_addr(lds);
  auto dma_step = [&](int stage, int step) __attribute__((always_inline)) {
    const uint32_t base = lds0 + stage * kStage;
    const uint32_t wv = wvoff + (uint32_t)step * wstep;
#pragma unroll
    for (int j = 0; j < kNmWideDma; ++j)
      dma16(wrsrc, base + (w + kNmWaves * j) * 1024, (int)(wv + j * wrow16), 0);
#pragma unroll
    for (int k = 0; k < kSlots; ++k)
#pragma unroll
      for (int i = 0; i < kNarrowDma; ++i) {
        const uint32_t v = nvoff[k][i] + (uint32_t)step * nstep[k];
        dma4(nrsrc[k], base + kNmWideBytes + k * kNarrowBytes + (w * kNarrowDma + i) * 256, (int)v,
             0);
      }
  };

  // Fragment offsets (sub-step 0, half 0): wide column blocks 32 w and
  // 32 w + 16 (the latter is the former XOR 32, tile_off), narrow row blocks
  // 16 mb of slot k at + k * kNarrowBytes; half 1 is 16 rows further,
  // sub-step 1 32 rows.
  const int boff = frag16_off(32 * w, 0, lane);
  int aoff[kMB];
  {
    const int q = lane >> 4, L = lane & 15;
    const int k = 4 * q + (L >> 2);
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      const int dw = 8 * mb + 2 * (L & 3);
      aoff[mb] = kNmWideBytes + k * kRowN + 4 * ((NS == 32) ? dw ^ ((q & 1) << 3) : dw);
    }
  }
  f32x4_t acc[kSlots][kMB][2];
#pragma unroll
  for (int k = 0; k < kSlots; ++k)
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[k][mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int stage) __attribute__((always_inline)) {
    const uint8_t* st = lds + stage * kStage;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8_t bf[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int o = (boff ^ (32 * nb)) + kk * 32 * kTileRowBytes;
        bf[nb] = join_frag(read_tr(st, o), read_tr(st, o + 16 * kTileRowBytes));
      }
#pragma unroll
      for (int k = 0; k < kSlots; ++k) {
        if (k > 0 && k >= nslots) break;
        bf16x8_t af[kMB];
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          const int o = aoff[mb] + k * kNarrowBytes + kk * 32 * kRowN;
          af[mb] = join_frag(read_tr(st, o), read_tr(st, o + 16 * kRowN));
        }
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
            acc[k][mb][nb] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mb], bf[nb], acc[k][mb][nb], 0, 0, 0);
      }
    }
  };

  // Step s waits for its own transfers (those of the next two steps may be in
  // flight); after the barrier every wave is done with stage (s + 3) % 4,
  // which takes the transfers of step s + 3.
#pragma unroll
  for (int p = 0; p < kNmStages - 1; ++p)
    if (p < nsteps) dma_step(p, p);
  auto iteration = [&](int s, int stage) __attribute__((always_inline)) {
    const int ahead = nsteps - 1 - s;
    if (ahead >= 2) {
      DPC_WAIT_VMCNT(2 * kDma);
    } else if (ahead == 1) {
      DPC_WAIT_VMCNT(kDma);
    } else {
      DPC_WAIT_VMCNT(0);
    }
    __syncthreads();
    if (s + kNmStages - 1 < nsteps) dma_step((stage + kNmStages - 1) % kNmStages, s + kNmStages - 1);
    compute(stage);
  };
  for (int s = 0; s < nsteps; s += kNmStages) {
    iteration(s, 0);
    if (s + 1 < nsteps) iteration(s + 1, 1);
    if (s + 2 < nsteps) iteration(s + 2, 2);
    if (s + 3 < nsteps) iteration(s + 3, 3);
  }

  // Lane l holds out_k[16 mb + 4 (l / 16) + e][32 w + 16 nb + l % 16].
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    if (k > 0 && k >= nslots) break;
    const int ns = P.ns[k];
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int col = col0 + 32 * w + 16 * nb + (lane & 15);
        if (col >= nw) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int s = 16 * mb + 4 * (lane >> 4) + e;
          if (s >= ns) continue;
          const float v = acc[k][mb][nb][e];
          if (splits > 1) {
            P.partial[k][(((size_t)split * B + b) * ns + s) * nw + col] = v;
          } else {
            const size_t o =
                P.narrow_is_g ? ((size_t)b * ns + s) * nw + col : ((size_t)b * nw + col) * ns + s;
            if (tab.out_bf16) {
              reinterpret_cast<uint16_t*>(P.out[k])[o] = f32_to_bf16_bits(v);
            } else {
              reinterpret_cast<float*>(P.out[k])[o] = v;
            }
          }
        }
      }
  }
}

bool narrow_mfma_ok(int T, int nw, int ns) {
  return nw % 8 == 0 && ns % 2 == 0 && ns > 0 && ns <= kMaxNarrow &&
         (long long)(T + kNmK) * nw * 2 < kNwOutOfRange;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// One problem of dpc_per_example_grads(_grouped): out [B, dout, din].
struct NmDesc {
  const void* A;
  const void* G;
  void* out;
  int din, dout;
};

// Problems of one MFMA launch entry: d[slot[0 .. n)) share the wide operand
// (same pointer, width and side), so one pass over it serves all of them.
struct NmGroup {
  int slot[kNmMaxSlots];
  int n;
};

inline bool nm_narrow_is_g(const NmDesc& q) { return q.dout <= q.din; }
inline const void* nm_wide(const NmDesc& q) { return nm_narrow_is_g(q) ? q.A : q.G; }
inline int nm_nw(const NmDesc& q) { return nm_narrow_is_g(q) ? q.din : q.dout; }
inline int nm_ns(const NmDesc& q) { return nm_narrow_is_g(q) ? q.dout : q.din; }

// The table of one MFMA launch over the groups g[0 .. m) (m <=
// kNmMaxProblems, all with narrow widths in one NS class): token chunks of a
// multiple of 64 tokens, as many splits of every group as it takes for the
// launch to have a workgroup for every CU; a split problem's partials at ws +
// its offset (ws may be null to size them).  Returns the launch's workgroups;
// *ws_bytes receives the partials' bytes.
int nm_table(NmTable& tab, const NmDesc* d, const NmGroup* g, int m, int B, int T, int out_bf16,
             char* ws, size_t* ws_bytes) {
  long long base = 0;
  for (int i = 0; i < m; ++i) base += (long long)ceil_div(nm_nw(d[g[i].slot[0]]), kNmCols) * B;
  const int want = (int)std::max<long long>(1, (256 + base - 1) / base);
  const int chunk = ceil_div(ceil_div(T, want), kNmK) * kNmK;
  const int splits = ceil_div(T, chunk);
  size_t off = 0;
  long long wg = 0;
  for (int i = 0; i < m; ++i) {
    const NmDesc& q0 = d[g[i].slot[0]];
    NmProblem& P = tab.p[i];
    P.narrow_is_g = nm_narrow_is_g(q0);
    P.nw = nm_nw(q0);
    P.wide = (const uint16_t*)nm_wide(q0);
    P.nslots = g[i].n;
    for (int k = 0; k < kNmMaxSlots; ++k) {
      const NmDesc& q = d[g[i].slot[k < g[i].n ? k : 0]];
      P.ns[k] = nm_ns(q);
      P.narrow[k] = (const uint16_t*)(P.narrow_is_g ? q.G : q.A);
      P.out[k] = q.out;
      P.partial[k] = nullptr;
      if (k < g[i].n && splits > 1) {
        P.partial[k] = ws ? (float*)(ws + off) : nullptr;
        off = align256(off + (size_t)splits * B * P.ns[k] * P.nw * sizeof(float));
      }
    }
    P.col_tiles = ceil_div(P.nw, kNmCols);
    P.splits = splits;
    P.chunk = chunk;
    P.wg_start = (int)wg;
    wg += (long long)P.col_tiles * B * splits;
  }
  tab.n = m;
  tab.B = B;
  tab.T = T;
  tab.out_bf16 = out_bf16;
  *ws_bytes = off;
  return wg > 0x7fffffffLL ? -1 : (int)wg;
}

// The MFMA launches of the eligible problems d[idx[0 .. m)): problems of
// narrow width <= 16 that share a wide operand are merged, up to kNmMaxSlots
// to a group; one launch per NS class and run of up to kNmMaxProblems groups,
// each followed by the finish kernels of its split problems (so launches
// reuse the workspace).  With launch false only sizes the workspace, without
// the operand pointers (so without the grouping): a bound on every launch's
// partials -- a problem's token splits grow as its launch's workgroup count
// shrinks, and that count is at least the problem's own column tiles times
// B, so the sum of the problems' partials at that many splits covers any
// launch (for a single problem it is exact).
int nm_run(const NmDesc* d, const int* idx, int m, int B, int T, int out_bf16, void* ws,
           size_t ws_bytes, hipStream_t s, bool launch, size_t* ws_need) {
  size_t need = 0;
  if (!launch) {
    for (int i = 0; i < m; ++i) {
      const NmDesc& q = d[idx[i]];
      const int own = ceil_div(nm_nw(q), kNmCols) * B;
      const int want = std::max(1, ceil_div(256, own));
      const int splits = ceil_div(T, ceil_div(ceil_div(T, want), kNmK) * kNmK);
      if (splits > 1) need = align256(need + (size_t)splits * B * nm_ns(q) * nm_nw(q) * sizeof(float));
    }
    *ws_need = need;
    return DPC_OK;
  }
  for (int cls = 0; cls < 2; ++cls) {
    const int max_slots = cls == 0 ? kNmMaxSlots : 1;
    std::vector<NmGroup> groups;
    for (int i = 0; i < m; ++i) {
      const NmDesc& q = d[idx[i]];
      if ((nm_ns(q) > 16) != (cls == 1)) continue;
      bool merged = false;
      for (NmGroup& grp : groups) {
        const NmDesc& q0 = d[grp.slot[0]];
        if (grp.n < max_slots && nm_wide(q0) == nm_wide(q) && nm_nw(q0) == nm_nw(q) &&
            nm_narrow_is_g(q0) == nm_narrow_is_g(q)) {
          grp.slot[grp.n++] = idx[i];
          merged = true;
          break;
        }
      }
      if (!merged) groups.push_back(NmGroup{{idx[i], idx[i], idx[i]}, 1});
    }
    for (size_t g0 = 0; g0 < groups.size(); g0 += kNmMaxProblems) {
      const int k = (int)std::min<size_t>(kNmMaxProblems, groups.size() - g0);
      NmTable tab;
      size_t part = 0;
      const int wgs = nm_table(tab, d, groups.data() + g0, k, B, T, out_bf16, (char*)ws, &part);
      if (wgs < 0) return DPC_ENOTSUP;
      need = std::max(need, part);
      if (!launch || wgs == 0) continue;
      if (part > ws_bytes || (part > 0 && !ws)) return DPC_ENOSPC;
      if (cls == 0) {
        hipLaunchKernelGGL((narrow_wide_mfma_kernel<16, kNmMaxSlots>), dim3(wgs), dim3(kNmThreads),
                           0, s, tab);
      } else {
        hipLaunchKernelGGL((narrow_wide_mfma_kernel<32, 1>), dim3(wgs), dim3(kNmThreads), 0, s,
                           tab);
      }
      DPC_HIP_CHECK(hipGetLastError());
      for (int j = 0; j < k; ++j) {
        const NmProblem& P = tab.p[j];
        if (P.splits <= 1) continue;
        for (int sl = 0; sl < P.nslots; ++sl) {
          const size_t total = (size_t)B * P.ns[sl] * P.nw;
          hipLaunchKernelGGL(narrow_finish_kernel,
                             dim3((unsigned)((total + kDirThreads - 1) / kDirThreads)),
                             dim3(kDirThreads), 0, s, (const float*)P.partial[sl], P.splits, B,
                             P.nw, P.ns[sl], P.narrow_is_g, out_bf16, P.out[sl]);
          DPC_HIP_CHECK(hipGetLastError());
        }
      }
    }
  }
  *ws_need = need;
  return DPC_OK;
}

bool narrow_wide_ok(int T, int nw, int ns) {
  return nw % 4 == 0 && ns <= kMaxNarrow && (long long)T * nw * 2 < kNwOutOfRange;
}

// Token chunks of narrow_wide_bf16_kernel: enough workgroups for every CU,
// chunks of an even length that fits the LDS.
int narrow_wide_splits(int B, int T, int nw, int ns, int* chunk_out) {
  const int blocks = ceil_div(nw, kNwCols) * B;
  const int max_chunk = 2 * kNwLdsWords / (ns <= 16 ? 16 : 32);
  int splits = max(ceil_div(256, blocks), ceil_div(T, max_chunk));
  int chunk = ceil_div(T, max(1, splits));
  chunk += chunk & 1;
  *chunk_out = chunk;
  return ceil_div(T, chunk);
}

int narrow_splits(int B, int T, int nw) {
  const int blocks = ceil_div(nw, kWidePerBlock) * B;
  int splits = max(1, ceil_div(512, blocks));
  splits = max(splits, ceil_div(T, kMaxChunk));
  return min(splits, T);
}

}  // namespace

extern "C" size_t dpc_per_example_grads_workspace_bytes(int B, int T, int din, int dout) {
  if (B <= 0 || T <= 0 || din <= 0 || dout <= 0) return 0;
  const int ns = din < dout ? din : dout, nw = din < dout ? dout : din;
  if (ns > kMaxNarrow) return 0;
  // The largest of the paths' needs (the query does not know the dtype).
  size_t bytes = (size_t)narrow_splits(B, T, nw) * B * ns * nw * sizeof(float);
  if (narrow_wide_ok(T, nw, ns)) {
    int chunk;
    const int splits = narrow_wide_splits(B, T, nw, ns, &chunk);
    if (splits > 1) bytes = max(bytes, (size_t)splits * B * ns * nw * sizeof(float));
  }
  if (narrow_mfma_ok(T, nw, ns)) {
    const NmDesc d{nullptr, nullptr, nullptr, din, dout};
    const int idx = 0;
    size_t need = 0;
    if (nm_run(&d, &idx, 1, B, T, 0, nullptr, 0, nullptr, false, &need) == DPC_OK)
      bytes = max(bytes, need);
  }
  return bytes;
}

extern "C" int dpc_per_example_grads(const void* A, const void* G, int B, int T, int din,
                                     int dout, int dtype, void* out, int out_dtype, void* ws,
                                     size_t ws_bytes, void* stream) {
  if (B < 0 || T <= 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (out_dtype != DPC_F32 && out_dtype != DPC_BF16) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!A || !G || !out) return DPC_EINVAL;
  const bool narrow_is_g = dout <= din;
  const int ns = narrow_is_g ? dout : din, nw = narrow_is_g ? din : dout;
  if (ns > kMaxNarrow || B > 65535) return DPC_ENOTSUP;
  if (!ws || ws_bytes < dpc_per_example_grads_workspace_bytes(B, T, din, dout)) return DPC_ENOSPC;
  hipStream_t s = (hipStream_t)stream;
  const void* wide = narrow_is_g ? A : G;
  const void* narrow = narrow_is_g ? G : A;
  if (dtype == DPC_BF16 && narrow_mfma_ok(T, nw, ns)) {
    const NmDesc d{A, G, out, din, dout};
    const int idx = 0;
    size_t need = 0;
    return nm_run(&d, &idx, 1, B, T, (int)(out_dtype == DPC_BF16), ws, ws_bytes, s, true, &need);
  }
  if (dtype == DPC_BF16 && narrow_wide_ok(T, nw, ns)) {
    int chunk;
    const int splits = narrow_wide_splits(B, T, nw, ns, &chunk);
    if (splits > 65535) return DPC_ENOTSUP;
    dim3 grid(ceil_div(nw, kNwCols), B, splits);
    auto wp = (const uint16_t*)wide;
    auto np = (const uint16_t*)narrow;
    const int ob = (int)(out_dtype == DPC_BF16);
    if (ns <= 16) {
      hipLaunchKernelGGL(narrow_wide_bf16_kernel<16>, grid, dim3(kNwThreads), 0, s, wp, np, B, T,
                         nw, ns, chunk, splits, (int)narrow_is_g, ob, (float*)ws, out);
    } else {
      hipLaunchKernelGGL(narrow_wide_bf16_kernel<32>, grid, dim3(kNwThreads), 0, s, wp, np, B, T,
                         nw, ns, chunk, splits, (int)narrow_is_g, ob, (float*)ws, out);
    }
    DPC_HIP_CHECK(hipGetLastError());
    if (splits > 1) {
      const size_t total = (size_t)B * ns * nw;
      hipLaunchKernelGGL(narrow_finish_kernel,
                         dim3((unsigned)((total + kDirThreads - 1) / kDirThreads)), dim3(kDirThreads),
                         0, s, (const float*)ws, splits, B, nw, ns, (int)narrow_is_g, ob, out);
      DPC_HIP_CHECK(hipGetLastError());
    }
    return DPC_OK;
  }
  const int splits = narrow_splits(B, T, nw);
  if (splits > 65535) return DPC_ENOTSUP;
  const int chunk = ceil_div(T, splits);
  float* partial = (float*)ws;
  if (chunk > kMaxChunk) return DPC_ENOTSUP;
  dim3 grid(ceil_div(nw, kWidePerBlock), B, splits);
  const bool small = ns <= 16;
  if (dtype == DPC_BF16) {
    auto wp = (const uint16_t*)wide;
    auto np = (const uint16_t*)narrow;
    if (small) {
      hipLaunchKernelGGL(narrow_partial_bf16_kernel<16>, grid, dim3(kDirThreads), 0, s, wp, np, B,
                         T, nw, ns, chunk, partial);
    } else {
      hipLaunchKernelGGL(narrow_partial_bf16_kernel<32>, grid, dim3(kDirThreads), 0, s, wp, np, B,
                         T, nw, ns, chunk, partial);
    }
  } else {
    auto wp = (const float*)wide;
    auto np = (const float*)narrow;
    if (small) {
      hipLaunchKernelGGL((narrow_partial_kernel<float, 16>), grid, dim3(kDirThreads), 0, s, wp, np,
                         B, T, nw, ns, chunk, partial);
    } else {
      hipLaunchKernelGGL((narrow_partial_kernel<float, 32>), grid, dim3(kDirThreads), 0, s, wp, np,
                         B, T, nw, ns, chunk, partial);
    }
  }
  DPC_HIP_CHECK(hipGetLastError());
  const size_t total = (size_t)B * ns * nw;
  hipLaunchKernelGGL(narrow_finish_kernel, dim3((unsigned)((total + kDirThreads - 1) / kDirThreads)),
                     dim3(kDirThreads), 0, s, (const float*)partial, splits, B, nw, ns,
                     (int)narrow_is_g, (int)(out_dtype == DPC_BF16), out);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

// Problems for the MFMA kernel (bf16 operands, eligible widths) and the others.
static int grouped_split(int n, const int* din, const int* dout, int T, int dtype, int* mfma,
                         int* other, int* n_mfma, int* n_other) {
  *n_mfma = *n_other = 0;
  for (int i = 0; i < n; ++i) {
    if (din[i] <= 0 || dout[i] <= 0) return DPC_EINVAL;
    const int ns = std::min(din[i], dout[i]), nw = std::max(din[i], dout[i]);
    if (ns > kMaxNarrow) return DPC_ENOTSUP;
    if (dtype == DPC_BF16 && narrow_mfma_ok(T, nw, ns)) {
      mfma[(*n_mfma)++] = i;
    } else {
      other[(*n_other)++] = i;
    }
  }
  return DPC_OK;
}

extern "C" size_t dpc_per_example_grads_grouped_workspace_bytes(int n, const int* din,
                                                                const int* dout, int B, int T,
                                                                int dtype) {
  if (n <= 0 || B <= 0 || T <= 0 || !din || !dout) return 0;
  std::vector<int> mfma(n), other(n);
  int nm = 0, no = 0;
  if (grouped_split(n, din, dout, T, dtype, mfma.data(), other.data(), &nm, &no) != DPC_OK) return 0;
  size_t bytes = 0;
  for (int i = 0; i < no; ++i)
    bytes = std::max(bytes, dpc_per_example_grads_workspace_bytes(B, T, din[other[i]], dout[other[i]]));
  if (nm > 0) {
    std::vector<NmDesc> d(n);
    for (int i = 0; i < n; ++i) d[i] = NmDesc{nullptr, nullptr, nullptr, din[i], dout[i]};
    size_t need = 0;
    if (nm_run(d.data(), mfma.data(), nm, B, T, 0, nullptr, 0, nullptr, false, &need) == DPC_OK)
      bytes = std::max(bytes, need);
  }
  return bytes;
}

extern "C" int dpc_per_example_grads_grouped(int n, const void* const* A, const void* const* G,
                                             void* const* out, const int* din, const int* dout,
                                             int B, int T, int dtype, int out_dtype, void* ws,
                                             size_t ws_bytes, void* stream) {
  if (n < 0 || B < 0 || T <= 0) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (out_dtype != DPC_F32 && out_dtype != DPC_BF16) return DPC_EINVAL;
  if (n == 0 || B == 0) return DPC_OK;
  if (!A || !G || !out || !din || !dout) return DPC_EINVAL;
  for (int i = 0; i < n; ++i)
    if (!A[i] || !G[i] || !out[i]) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  std::vector<int> mfma(n), other(n);
  int nm = 0, no = 0;
  const int rc = grouped_split(n, din, dout, T, dtype, mfma.data(), other.data(), &nm, &no);
  if (rc != DPC_OK) return rc;
  if (!ws || ws_bytes < dpc_per_example_grads_grouped_workspace_bytes(n, din, dout, B, T, dtype))
    return DPC_ENOSPC;
  if (nm > 0) {
    std::vector<NmDesc> d(n);
    for (int i = 0; i < n; ++i) d[i] = NmDesc{A[i], G[i], out[i], din[i], dout[i]};
    size_t need = 0;
    const int r = nm_run(d.data(), mfma.data(), nm, B, T, (int)(out_dtype == DPC_BF16), ws,
                         ws_bytes, (hipStream_t)stream, true, &need);
    if (r != DPC_OK) return r;
  }
  for (int i = 0; i < no; ++i) {
    const int j = other[i];
    const int r = dpc_per_example_grads(A[j], G[j], B, T, din[j], dout[j], dtype, out[j],
                                        out_dtype, ws, ws_bytes, stream);
    if (r != DPC_OK) return r;
  }
  return DPC_OK;
}
