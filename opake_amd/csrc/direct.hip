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
#include "common.h"

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
  // The larger of the two paths' needs (the query does not know the dtype).
  size_t bytes = (size_t)narrow_splits(B, T, nw) * B * ns * nw * sizeof(float);
  if (narrow_wide_ok(T, nw, ns)) {
    int chunk;
    const int splits = narrow_wide_splits(B, T, nw, ns, &chunk);
    if (splits > 1) bytes = max(bytes, (size_t)splits * B * ns * nw * sizeof(float));
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
