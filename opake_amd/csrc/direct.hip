// Per-example weight gradients of linear layers with a narrow side (LoRA
// adapters: rank r <= 32 on one side),
//   out[b, m, n] = sum_t G[b, t, m] * A[b, t, n]      (out is [B, dout, din]),
// materialised in fp32: for such layers the per-example gradient is small and
// cheaper to form (2 T din dout FLOP) than its Gram norm (T^2 (din + dout)).
//
// One operand is wide (W columns), the other narrow (ns <= 32 columns).  A
// workgroup owns 1024 wide columns of one example and a chunk of the tokens;
// each thread keeps 4 adjacent wide columns x NS narrow columns of fp32 sums.
// The chunk's narrow rows are staged once in LDS as fp32 (every lane of a
// wave then reads the same word: a broadcast); the wide values come with one
// 8-byte load per thread and token, four tokens in flight at a time.  Token
// chunks write fp32 partial sums, added in chunk order by a second kernel
// that also lays out (and rounds) the result.  Memory bound: the wide operand
// is read once.
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
  return (size_t)narrow_splits(B, T, nw) * B * ns * nw * sizeof(float);
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
  const int splits = narrow_splits(B, T, nw);
  if (splits > 65535) return DPC_ENOTSUP;
  if (!ws || ws_bytes < dpc_per_example_grads_workspace_bytes(B, T, din, dout)) return DPC_ENOSPC;
  const int chunk = ceil_div(T, splits);
  hipStream_t s = (hipStream_t)stream;
  float* partial = (float*)ws;
  if (chunk > kMaxChunk) return DPC_ENOTSUP;
  dim3 grid(ceil_div(nw, kWidePerBlock), B, splits);
  const void* wide = narrow_is_g ? A : G;
  const void* narrow = narrow_is_g ? G : A;
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
