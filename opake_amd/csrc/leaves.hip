// Materialised-leaf clip-and-sum: stacked per-example values [B, n_l] of many
// leaves, handled by a fixed number of launches whatever the leaf count
// (multi-tensor apply through a device pointer table and a tile table).
//
// Semantics follow the reference's streaming path (packages/opake-engine/src/
// opake/api/engine/clipping/_streaming.py:39-185 with _pytree.py:160-314):
//   norm pass : sanitise (NaN/Inf -> 0), square in fp32, sum in fp64 per
//               2048-element tile, tiles summed per leaf;
//   apply pass: stored = to_dtype(float(x) * scale[b]) with bf16 results that
//               rounded up into the subnormal range zeroed; summed over the
//               batch in fp32 in order b = 0..B-1; optionally the second
//               moment, to_dtype(stored^2) summed the same way.
#include "common.h"

namespace {

constexpr int kTile = 2048;
constexpr int kThreads = 256;
constexpr int kPerThread = kTile / kThreads;  // 8

template <bool kBf16>
__device__ __forceinline__ float load_elem(int64_t base, int64_t idx) {
  if (kBf16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
  return reinterpret_cast<const float*>(base)[idx];
}

__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  double total = 0.0;
  if (threadIdx.x == 0)
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) total += red[i];
  return total;
}

__device__ __forceinline__ float block_sum_f32(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float total = 0.f;
  if (threadIdx.x == 0)
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) total += red[i];
  return total;
}

#pragma clang fp contract(off)
template <bool kBf16>
__global__ void __launch_bounds__(kThreads)
tile_sq_kernel(const int64_t* __restrict__ ptrs, const int64_t* __restrict__ sizes,
               const int32_t* __restrict__ tile_leaf, const int32_t* __restrict__ tile_local,
               int n_tiles, double* __restrict__ partial) {
  __shared__ double red[kThreads / 64];
  const int t = blockIdx.x, b = blockIdx.y;
  const int leaf = tile_leaf[t];
  const int64_t n = sizes[leaf];
  const int64_t base = ptrs[leaf];
  const int64_t off0 = (int64_t)tile_local[t] * kTile;
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t off = off0 + threadIdx.x + (int64_t)j * kThreads;
    if (off < n) {
      float x = finite_or_zero(load_elem<kBf16>(base, (int64_t)b * n + off));
      float sq = x * x;
      s += (double)sq;
    }
  }
  double total = block_sum_f64(s, red);
  if (threadIdx.x == 0) partial[(size_t)b * n_tiles + t] = total;
}
#pragma clang fp contract(on)

// leaf_sq[b, leaf_col[l]] = sum of leaf l's tile partials (fixed order).
__global__ void __launch_bounds__(kThreads)
leaf_sum_kernel(const double* __restrict__ partial, const int64_t* __restrict__ tile_start,
                const int32_t* __restrict__ leaf_col, int n_tiles, double* __restrict__ leaf_sq,
                int stride) {
  __shared__ double red[kThreads / 64];
  const int l = blockIdx.x, b = blockIdx.y;
  const int64_t t0 = tile_start[l], t1 = tile_start[l + 1];
  double s = 0.0;
  for (int64_t t = t0 + threadIdx.x; t < t1; t += blockDim.x) s += partial[(size_t)b * n_tiles + t];
  double total = block_sum_f64(s, red);
  if (threadIdx.x == 0) leaf_sq[(size_t)b * stride + leaf_col[l]] = total;
}

#pragma clang fp contract(off)
template <bool kBf16, bool kOutBf16>
__global__ void __launch_bounds__(kThreads)
apply_sum_kernel(const int64_t* __restrict__ ptrs, const int64_t* __restrict__ sizes,
                 const int32_t* __restrict__ tile_leaf, const int32_t* __restrict__ tile_local,
                 const int64_t* __restrict__ out_offs, int n_tiles, int B,
                 const float* __restrict__ scale, const int32_t* __restrict__ leaf_scale_row,
                 void* __restrict__ out, void* __restrict__ out_sq, float* __restrict__ post_sq) {
  __shared__ float red[kThreads / 64];
  const int t = blockIdx.x;
  const int leaf = tile_leaf[t];
  const int64_t n = sizes[leaf];
  const int64_t base = ptrs[leaf];
  const int64_t off0 = (int64_t)tile_local[t] * kTile;
  const float smallest_normal = 1.17549435e-38f;  // bf16 shares float32's exponent range
  float acc[kPerThread], acc2[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) acc[j] = acc2[j] = 0.f;
  const float* srow = scale + (size_t)(leaf_scale_row ? leaf_scale_row[leaf] : 0) * B;
  for (int b = 0; b < B; ++b) {
    const float s = srow[b];
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
      const int64_t off = off0 + threadIdx.x + (int64_t)j * kThreads;
      if (off < n) {
        float x = finite_or_zero(load_elem<kBf16>(base, (int64_t)b * n + off));
        float prod = x * s;
        float stored = prod;
        if (kBf16) {
          stored = round_to_bf16(prod);
          float sa = fabsf(stored);
          if (sa <= smallest_normal && sa > fabsf(prod)) stored = 0.f;
        }
        acc[j] = acc[j] + stored;
        if (out_sq) {
          // Second moment: the stored value squared in its dtype, then summed.
          float s2 = stored * stored;
          if (kBf16) s2 = round_to_bf16(s2);
          acc2[j] = acc2[j] + s2;
        }
        if (post_sq) sq = sq + stored * stored;
      }
    }
    if (post_sq) {
      float total = block_sum_f32(sq, red);
      if (threadIdx.x == 0) post_sq[(size_t)b * n_tiles + t] = total;
    }
  }
  const int64_t obase = out_offs[leaf];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int64_t off = off0 + threadIdx.x + (int64_t)j * kThreads;
    if (off < n) {
      if (kOutBf16) {
        reinterpret_cast<uint16_t*>(out)[obase + off] = f32_to_bf16_bits(acc[j]);
        if (out_sq) reinterpret_cast<uint16_t*>(out_sq)[obase + off] = f32_to_bf16_bits(acc2[j]);
      } else {
        reinterpret_cast<float*>(out)[obase + off] = acc[j];
        if (out_sq) reinterpret_cast<float*>(out_sq)[obase + off] = acc2[j];
      }
    }
  }
}
#pragma clang fp contract(on)

// out[g * B + b] = sum over columns j with col_group[j] == g of x[b, j], in
// column order (fp64): the reference's per-group accumulation in leaf order.
__global__ void __launch_bounds__(kThreads)
group_sum_kernel(const double* __restrict__ x, int B, int n, int stride,
                 const int32_t* __restrict__ col_group, int n_groups, double* __restrict__ out) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * n_groups) return;
  const int g = idx / B, b = idx % B;
  double s = 0.0;
  for (int j = 0; j < n; ++j) {
    if (col_group[j] == g) s += x[(size_t)b * stride + j];
  }
  out[(size_t)g * B + b] = s;
}

}  // namespace

extern "C" int dpc_group_sum_f64(const double* x, int B, int n, int stride,
                                 const int32_t* col_group, int n_groups, double* out,
                                 void* stream) {
  if (B < 0 || n < 0 || stride < n || n_groups < 1) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!out || (n > 0 && (!x || !col_group))) return DPC_EINVAL;
  const int total = B * n_groups;
  hipLaunchKernelGGL(group_sum_kernel, dim3(ceil_div(total, kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, x, B, n, stride, col_group, n_groups, out);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_leaves_sqnorm(const int64_t* ptrs, const int64_t* sizes,
                                 const int32_t* tile_leaf, const int32_t* tile_local,
                                 const int64_t* tile_start, const int32_t* leaf_col,
                                 int n_leaves, int n_tiles, int B, int dtype, double* partial,
                                 double* leaf_sq, int leaf_sq_stride, void* stream) {
  if (n_leaves < 0 || n_tiles < 0 || B < 0 || leaf_sq_stride < n_leaves) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (B == 0 || n_leaves == 0) return DPC_OK;
  if (!ptrs || !sizes || !tile_leaf || !tile_local || !tile_start || !leaf_col || !partial ||
      !leaf_sq)
    return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  hipStream_t s = (hipStream_t)stream;
  if (n_tiles > 0) {
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(tile_sq_kernel<true>, dim3(n_tiles, B), dim3(kThreads), 0, s, ptrs,
                         sizes, tile_leaf, tile_local, n_tiles, partial);
    } else {
      hipLaunchKernelGGL(tile_sq_kernel<false>, dim3(n_tiles, B), dim3(kThreads), 0, s, ptrs,
                         sizes, tile_leaf, tile_local, n_tiles, partial);
    }
    DPC_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(leaf_sum_kernel, dim3(n_leaves, B), dim3(kThreads), 0, s,
                     (const double*)partial, tile_start, leaf_col, n_tiles, leaf_sq,
                     leaf_sq_stride);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_leaves_apply(const int64_t* ptrs, const int64_t* sizes,
                                const int32_t* tile_leaf, const int32_t* tile_local,
                                const int64_t* out_offs, int n_tiles, int B, int dtype,
                                const float* scale, const int32_t* leaf_scale_row, void* out,
                                void* out_sq, int out_dtype, float* post_sq, void* stream) {
  if (n_tiles < 0 || B < 0) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (out_dtype != DPC_F32 && out_dtype != dtype) return DPC_EINVAL;
  if (n_tiles == 0) return DPC_OK;
  if (!ptrs || !sizes || !tile_leaf || !tile_local || !out_offs || !out || (B > 0 && !scale))
    return DPC_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DPC_BF16 && out_dtype == DPC_BF16) {
    hipLaunchKernelGGL((apply_sum_kernel<true, true>), dim3(n_tiles), dim3(kThreads), 0, s, ptrs,
                       sizes, tile_leaf, tile_local, out_offs, n_tiles, B, scale, leaf_scale_row, out, out_sq,
                       post_sq);
  } else if (dtype == DPC_BF16) {
    hipLaunchKernelGGL((apply_sum_kernel<true, false>), dim3(n_tiles), dim3(kThreads), 0, s,
                       ptrs, sizes, tile_leaf, tile_local, out_offs, n_tiles, B, scale,
                       leaf_scale_row, out, out_sq, post_sq);
  } else {
    hipLaunchKernelGGL((apply_sum_kernel<false, false>), dim3(n_tiles), dim3(kThreads), 0, s,
                       ptrs, sizes, tile_leaf, tile_local, out_offs, n_tiles, B, scale,
                       leaf_scale_row, out, out_sq, post_sq);
  }
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
