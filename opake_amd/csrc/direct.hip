// Per-example weight gradients of linear layers with a narrow side (LoRA
// adapters: rank r <= 32 on one side),
//   out[b, m, n] = sum_t G[b, t, m] * A[b, t, n]      (out is [B, dout, din]),
// materialised in fp32: for such layers the per-example gradient is small and
// cheaper to form (2 T din dout FLOP) than its Gram norm (T^2 (din + dout)).
//
// One operand is wide (W columns), the other narrow (ns <= 32 columns).  A
// workgroup owns 512 wide columns of one example and a chunk of the tokens;
// each thread keeps 2 wide columns x ns narrow columns of fp32 sums, reads
// its two wide values per token with one 4-byte load and the token's narrow
// row -- the same for the whole workgroup -- through scalar loads.  Token
// chunks write fp32 partial sums, added in chunk order by a second kernel
// that also lays out (and rounds) the result.  Memory bound: the wide
// operand is read once.
#include "common.h"

namespace {

constexpr int kDirThreads = 256;
constexpr int kWidePerThread = 2;
constexpr int kWidePerBlock = kDirThreads * kWidePerThread;
constexpr int kMaxNarrow = 32;

template <typename In>
__device__ __forceinline__ float dir_f32(In v);
template <>
__device__ __forceinline__ float dir_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float dir_f32<uint16_t>(uint16_t v) { return bf16_bits_to_f32(v); }

// partial[split][b][s][w] = sum over tokens t of chunk `split` of
// narrow[b, t, s] * wide[b, t, w].
template <typename In>
__global__ void __launch_bounds__(kDirThreads)
narrow_partial_kernel(const In* __restrict__ wide, const In* __restrict__ narrow, int B, int T,
                      int nw, int ns, int chunk, float* __restrict__ partial) {
  const int b = blockIdx.y, split = blockIdx.z;
  const int w0 = blockIdx.x * kWidePerBlock + threadIdx.x * kWidePerThread;
  const int t0 = split * chunk, t1 = min(T, t0 + chunk);
  float acc[kMaxNarrow][kWidePerThread];
#pragma unroll
  for (int s = 0; s < kMaxNarrow; ++s)
#pragma unroll
    for (int j = 0; j < kWidePerThread; ++j) acc[s][j] = 0.f;
  const bool both = w0 + 1 < nw;
  const bool one = w0 < nw;
  for (int t = t0; t < t1; ++t) {
    const In* wrow = wide + ((size_t)b * T + t) * nw;
    float x0 = 0.f, x1 = 0.f;
    if (both) {
      x0 = dir_f32<In>(wrow[w0]);
      x1 = dir_f32<In>(wrow[w0 + 1]);
    } else if (one) {
      x0 = dir_f32<In>(wrow[w0]);
    }
    const In* nrow = narrow + ((size_t)b * T + t) * ns;
#pragma unroll
    for (int s = 0; s < kMaxNarrow; ++s) {
      if (s < ns) {
        const float v = dir_f32<In>(nrow[s]);
        acc[s][0] = fmaf(v, x0, acc[s][0]);
        acc[s][1] = fmaf(v, x1, acc[s][1]);
      }
    }
  }
  if (!one) return;
  float* out = partial + (((size_t)split * B + b) * ns) * nw;
#pragma unroll
  for (int s = 0; s < kMaxNarrow; ++s) {
    if (s < ns) {
      out[(size_t)s * nw + w0] = acc[s][0];
      if (both) out[(size_t)s * nw + w0 + 1] = acc[s][1];
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
  int splits = ceil_div(1024, blocks);
  splits = min(splits, max(1, T / 64));
  return max(splits, 1);
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
  dim3 grid(ceil_div(nw, kWidePerBlock), B, splits);
  const void* wide = narrow_is_g ? A : G;
  const void* narrow = narrow_is_g ? G : A;
  if (dtype == DPC_BF16) {
    hipLaunchKernelGGL(narrow_partial_kernel<uint16_t>, grid, dim3(kDirThreads), 0, s,
                       (const uint16_t*)wide, (const uint16_t*)narrow, B, T, nw, ns, chunk,
                       partial);
  } else {
    hipLaunchKernelGGL(narrow_partial_kernel<float>, grid, dim3(kDirThreads), 0, s,
                       (const float*)wide, (const float*)narrow, B, T, nw, ns, chunk, partial);
  }
  DPC_HIP_CHECK(hipGetLastError());
  const size_t total = (size_t)B * ns * nw;
  hipLaunchKernelGGL(narrow_finish_kernel, dim3((unsigned)((total + kDirThreads - 1) / kDirThreads)),
                     dim3(kDirThreads), 0, s, (const float*)partial, splits, B, nw, ns,
                     (int)narrow_is_g, (int)(out_dtype == DPC_BF16), out);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
