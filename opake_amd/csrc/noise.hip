// Gaussian noise on one leaf, out of place:
//   y = to_dtype(float(x) + (float)sigma * z)
// with z injected (float32, same shape) or drawn from the Philox stream of
// (seed, leaf) under the [rows, cols] view described in common.h.  Each thread
// produces one even/odd row pair of one column, so consecutive threads touch
// consecutive columns.  Wide leaves (kRowBlocks) give each workgroup 256
// columns of one row pair, so the row pair comes from one workgroup-uniform
// division; other leaves split a flat thread index per lane (in 32 bits when
// the leaf's pair count allows, a 64-bit division costing about as much as
// the rest of the thread's work).
#include <algorithm>

#include "common.h"

namespace {

constexpr int kNoiseThreads = 256;

#pragma clang fp contract(off)
template <bool kBf16>
__device__ __forceinline__ float add_scaled(float x, float sigma, float z) {
  float t = sigma * z;
  float v = x + t;
  return kBf16 ? round_to_bf16(v) : v;
}
#pragma clang fp contract(on)

template <bool kBf16, bool kRowBlocks>
__global__ void __launch_bounds__(kNoiseThreads)
add_noise_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t rows, int64_t cols,
                 float sigma, int mode, const float* __restrict__ noise, uint64_t seed,
                 uint32_t leaf, uint32_t col_blocks) {
  const int64_t pairs = (rows + 1) >> 1;
  int64_t pr, c;
  if (kRowBlocks) {
    const uint32_t b = blockIdx.x;
    const uint32_t p = b / col_blocks;
    pr = p;
    c = (int64_t)(b - p * col_blocks) * kNoiseThreads + threadIdx.x;
    if (c >= cols) return;
  } else {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t work = pairs * cols;
    if (t >= work) return;
    if (work <= 0xffffffffLL) {
      const uint32_t q = (uint32_t)t / (uint32_t)cols;
      pr = q;
      c = (uint32_t)t - q * (uint32_t)cols;
    } else {
      pr = t / cols;
      c = t - pr * cols;
    }
  }
  const int64_t t = pr * cols + c;  // Philox block of (row pair, column)
  const int64_t r0 = pr * 2;
  float z0, z1;
  if (mode == DPC_NOISE_PHILOX) {
    philox_normal_pair(seed, leaf, (uint64_t)t, &z0, &z1);
  } else {
    z0 = noise[r0 * cols + c];
    z1 = (r0 + 1 < rows) ? noise[(r0 + 1) * cols + c] : 0.0f;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t r = r0 + h;
    if (r >= rows) break;
    const int64_t idx = r * cols + c;
    const float z = h ? z1 : z0;
    if (kBf16) {
      float xv = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[idx]);
      reinterpret_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(add_scaled<true>(xv, sigma, z));
    } else {
      float xv = reinterpret_cast<const float*>(x)[idx];
      reinterpret_cast<float*>(y)[idx] = add_scaled<false>(xv, sigma, z);
    }
  }
}

// Wide leaves with an even column count and 8-byte aligned operands: each
// thread takes columns c, c + 1 (c even) of one row pair -- 4- or 8-byte
// loads and stores, two independent Philox blocks -- and each workgroup 512
// columns of one row pair.  Same Philox blocks as add_noise_kernel.
template <bool kBf16>
__global__ void __launch_bounds__(kNoiseThreads)
add_noise_pairs_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t rows,
                       int64_t cols, float sigma, int mode, const float* __restrict__ noise,
                       uint64_t seed, uint32_t leaf, uint32_t col_blocks) {
  const uint32_t b = blockIdx.x;
  const uint32_t p = b / col_blocks;
  const int64_t c = (int64_t)(b - p * col_blocks) * (2 * kNoiseThreads) + 2 * threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = 2 * (int64_t)p;
  float z[2][2];  // z[row h][column k]
  if (mode == DPC_NOISE_PHILOX) {
    const uint64_t blk = (uint64_t)p * (uint64_t)cols + (uint64_t)c;
    philox_normal_pair(seed, leaf, blk, &z[0][0], &z[1][0]);
    philox_normal_pair(seed, leaf, blk + 1, &z[0][1], &z[1][1]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float2 v = {0.0f, 0.0f};
      if (r0 + h < rows) v = *reinterpret_cast<const float2*>(noise + (r0 + h) * cols + c);
      z[h][0] = v.x;
      z[h][1] = v.y;
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t r = r0 + h;
    if (r >= rows) break;
    const int64_t idx = r * cols + c;
    if (kBf16) {
      const uint32_t xv = *reinterpret_cast<const uint32_t*>(
          reinterpret_cast<const uint16_t*>(x) + idx);
      const float a = add_scaled<true>(bf16_bits_to_f32((uint16_t)(xv & 0xffffu)), sigma, z[h][0]);
      const float d = add_scaled<true>(bf16_bits_to_f32((uint16_t)(xv >> 16)), sigma, z[h][1]);
      *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(y) + idx) =
          f32x2_to_bf16x2_bits(a, d);
    } else {
      const float2 xv = *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(x) + idx);
      float2 out;
      out.x = add_scaled<false>(xv.x, sigma, z[h][0]);
      out.y = add_scaled<false>(xv.y, sigma, z[h][1]);
      *reinterpret_cast<float2*>(reinterpret_cast<float*>(y) + idx) = out;
    }
  }
}

// Philox noise on up to kLeafMax leaves in one launch, by value (no table
// upload): leaf i takes workgroups block_start[i] .. block_start[i + 1] - 1,
// one (row pair, column) per thread as in add_noise_kernel (the same Philox
// blocks, so each leaf gets exactly dpc_add_noise's values); a leaf with sigma
// 0 is copied.  y may equal x (each element is read, then written, by one
// thread).
constexpr int kLeafMax = 32;
struct NoiseLeaf {
  const void* x;
  void* y;
  int64_t rows, cols;
  float sigma;
  uint32_t leaf;
  uint32_t block_start;
};
struct NoiseLeafTable {
  NoiseLeaf l[kLeafMax];
  int n;
  uint64_t seed;
};

template <bool kBf16>
__global__ void __launch_bounds__(kNoiseThreads) add_noise_leaves_kernel(const NoiseLeafTable tab) {
  const uint32_t blk = blockIdx.x;
  int li = 0;
  for (int i = 1; i < tab.n; ++i)
    if (blk >= tab.l[i].block_start) li = i;
  const NoiseLeaf& L = tab.l[li];
  const int64_t rows = L.rows, cols = L.cols;
  const int64_t work = ((rows + 1) >> 1) * cols;
  const int64_t t = (int64_t)(blk - L.block_start) * kNoiseThreads + threadIdx.x;
  if (t >= work) return;
  int64_t pr, c;
  if (work <= 0xffffffffLL) {
    const uint32_t q = (uint32_t)t / (uint32_t)cols;
    pr = q;
    c = (uint32_t)t - q * (uint32_t)cols;
  } else {
    pr = t / cols;
    c = t - pr * cols;
  }
  float z0 = 0.0f, z1 = 0.0f;
  if (L.sigma != 0.0f) philox_normal_pair(tab.seed, L.leaf, (uint64_t)t, &z0, &z1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t r = 2 * pr + h;
    if (r >= rows) break;
    const int64_t idx = r * cols + c;
    const float z = h ? z1 : z0;
    if (kBf16) {
      const uint16_t xv = reinterpret_cast<const uint16_t*>(L.x)[idx];
      reinterpret_cast<uint16_t*>(L.y)[idx] =
          L.sigma != 0.0f ? f32_to_bf16_bits(add_scaled<true>(bf16_bits_to_f32(xv), L.sigma, z))
                          : xv;
    } else {
      const float xv = reinterpret_cast<const float*>(L.x)[idx];
      reinterpret_cast<float*>(L.y)[idx] =
          L.sigma != 0.0f ? add_scaled<false>(xv, L.sigma, z) : xv;
    }
  }
}

// Any leaf dtype and any compute dtype cd (_gaussian.py:188-204 with
// compute_dtype): per element,
//   c = to_cd(x), z = draw (injected: a cd value; device stream: the float
//   normal rounded to cd), t = to_cd(sigma_op * z), y = to_dtype(to_cd(c + t))
// with sigma_op = (float)sigma for cd of 16 or 32 bits (torch multiplies a
// tensor by a Python scalar in float there) and sigma itself for float64;
// to_cd of a 16-bit cd rounds through float32, as torch's float arithmetic
// for 16-bit tensors does.  One (row pair, column) per thread, the same
// Philox blocks as add_noise_kernel; a grid-stride loop covers any size.
#pragma clang fp contract(off)
__global__ void __launch_bounds__(kNoiseThreads)
add_noise_generic_kernel(const void* __restrict__ x, void* __restrict__ y, int64_t rows,
                         int64_t cols, int dtype, int cd, double sigma, int mode,
                         const void* __restrict__ noise, uint64_t seed, uint32_t leaf) {
  const int64_t work = ((rows + 1) >> 1) * cols;
  const double sig = cd == DPC_F64 ? sigma : (double)(float)sigma;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < work;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t pr = t / cols, c = t - pr * cols;
    float z32[2] = {0.0f, 0.0f};
    if (mode == DPC_NOISE_PHILOX) philox_normal_pair(seed, leaf, (uint64_t)t, &z32[0], &z32[1]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t r = 2 * pr + h;
      if (r >= rows) break;
      const int64_t idx = r * cols + c;
      const double z = mode == DPC_NOISE_PHILOX ? round_to_dtype((double)z32[h], cd)
                                                : load_as_f64(noise, idx, cd);
      const double cx = round_to_dtype(load_as_f64(x, idx, dtype), cd);
      const double term = round_to_dtype(sig * z, cd);
      const double v = round_to_dtype(cx + term, cd);
      store_from_f64(y, idx, round_to_dtype(v, dtype), dtype);
    }
  }
}
#pragma clang fp contract(on)

__global__ void philox_kat_kernel(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                  uint32_t k1, int n, uint32_t* __restrict__ out) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  Philox4 r = philox4x32_10(c0 + (uint32_t)j, c1, c2, c3, k0, k1);
#pragma unroll
  for (int w = 0; w < 4; ++w) out[4 * j + w] = r.v[w];
}

}  // namespace

extern "C" int dpc_add_noise(const void* x, void* y, int64_t rows, int64_t cols, int dtype,
                             double sigma, int noise_mode, const float* noise, uint64_t seed,
                             uint32_t leaf_id, void* stream) {
  if (rows < 0 || cols < 0 || !(sigma >= 0.0)) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (rows == 0 || cols == 0) return DPC_OK;
  if (!x || !y) return DPC_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const size_t esize = dtype == DPC_BF16 ? 2 : 4;
  if (sigma == 0.0) {
    if (x != y) {
      DPC_HIP_CHECK(hipMemcpyAsync(y, x, (size_t)rows * cols * esize, hipMemcpyDeviceToDevice, s));
    }
    return DPC_OK;
  }
  if (noise_mode != DPC_NOISE_INJECTED && noise_mode != DPC_NOISE_PHILOX) return DPC_EINVAL;
  if (noise_mode == DPC_NOISE_INJECTED && !noise) return DPC_EINVAL;
  const int64_t pairs = (rows + 1) >> 1;
  const int64_t col_blocks = (cols + kNoiseThreads - 1) / kNoiseThreads;
  // Row blocks when at most 1/8 of their lanes idle (or none do).
  const bool row_blocks = cols % kNoiseThreads == 0 || cols >= 8 * kNoiseThreads;
  const int64_t blocks = row_blocks ? pairs * col_blocks
                                    : (pairs * cols + kNoiseThreads - 1) / kNoiseThreads;
  if (blocks > 0x7fffffffLL) return DPC_ENOTSUP;
  const dim3 grid((unsigned)blocks), block(kNoiseThreads);
  const float sg = (float)sigma;
  const uint32_t cb = (uint32_t)col_blocks;
  const uintptr_t align = (uintptr_t)x | (uintptr_t)y |
                          (uintptr_t)(noise_mode == DPC_NOISE_INJECTED ? noise : nullptr);
  if (row_blocks && cols % 2 == 0 && align % 8 == 0) {
    const int64_t pair_blocks = pairs * ((cols + 2 * kNoiseThreads - 1) / (2 * kNoiseThreads));
    const uint32_t pcb = (uint32_t)((cols + 2 * kNoiseThreads - 1) / (2 * kNoiseThreads));
    const dim3 pgrid((unsigned)pair_blocks);
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(add_noise_pairs_kernel<true>, pgrid, block, 0, s, x, y, rows, cols, sg,
                         noise_mode, noise, seed, leaf_id, pcb);
    } else {
      hipLaunchKernelGGL(add_noise_pairs_kernel<false>, pgrid, block, 0, s, x, y, rows, cols, sg,
                         noise_mode, noise, seed, leaf_id, pcb);
    }
  } else if (dtype == DPC_BF16) {
    if (row_blocks) {
      hipLaunchKernelGGL((add_noise_kernel<true, true>), grid, block, 0, s, x, y, rows, cols, sg,
                         noise_mode, noise, seed, leaf_id, cb);
    } else {
      hipLaunchKernelGGL((add_noise_kernel<true, false>), grid, block, 0, s, x, y, rows, cols, sg,
                         noise_mode, noise, seed, leaf_id, cb);
    }
  } else {
    if (row_blocks) {
      hipLaunchKernelGGL((add_noise_kernel<false, true>), grid, block, 0, s, x, y, rows, cols, sg,
                         noise_mode, noise, seed, leaf_id, cb);
    } else {
      hipLaunchKernelGGL((add_noise_kernel<false, false>), grid, block, 0, s, x, y, rows, cols,
                         sg, noise_mode, noise, seed, leaf_id, cb);
    }
  }
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                 uint32_t k1, int n, uint32_t* out, void* stream) {
  if (n < 0 || (n > 0 && !out)) return DPC_EINVAL;
  if (n == 0) return DPC_OK;
  hipLaunchKernelGGL(philox_kat_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, (hipStream_t)stream,
                     c0, c1, c2, c3, k0, k1, n, out);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_add_noise_leaves(int n, const void* const* x, void* const* y,
                                    const int64_t* rows, const int64_t* cols, const double* sigma,
                                    const uint32_t* leaf_ids, int dtype, uint64_t seed,
                                    void* stream) {
  if (n < 0) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (n == 0) return DPC_OK;
  if (!x || !y || !rows || !cols || !sigma || !leaf_ids) return DPC_EINVAL;
  for (int i = 0; i < n; ++i) {
    if (rows[i] < 0 || cols[i] < 0 || !(sigma[i] >= 0.0)) return DPC_EINVAL;
    if (rows[i] > 0 && cols[i] > 0 && (!x[i] || !y[i])) return DPC_EINVAL;
  }
  hipStream_t s = (hipStream_t)stream;
  NoiseLeafTable tab;
  tab.seed = seed;
  int k = 0;
  uint64_t blocks = 0;
  for (int i = 0; i <= n; ++i) {
    if (i < n && rows[i] > 0 && cols[i] > 0) {
      const uint64_t b = (uint64_t)((((rows[i] + 1) >> 1) * cols[i] + kNoiseThreads - 1) /
                                    kNoiseThreads);
      if (b > 0x7fffffffULL) return DPC_ENOTSUP;
      if (k == kLeafMax || blocks + b > 0x7fffffffULL) {
        tab.n = k;
        if (dtype == DPC_BF16) {
          hipLaunchKernelGGL(add_noise_leaves_kernel<true>, dim3((unsigned)blocks),
                             dim3(kNoiseThreads), 0, s, tab);
        } else {
          hipLaunchKernelGGL(add_noise_leaves_kernel<false>, dim3((unsigned)blocks),
                             dim3(kNoiseThreads), 0, s, tab);
        }
        DPC_HIP_CHECK(hipGetLastError());
        k = 0;
        blocks = 0;
      }
      tab.l[k] = NoiseLeaf{x[i], y[i], rows[i], cols[i], (float)sigma[i], leaf_ids[i],
                           (uint32_t)blocks};
      blocks += b;
      ++k;
    }
    if (i == n && k > 0) {
      tab.n = k;
      if (dtype == DPC_BF16) {
        hipLaunchKernelGGL(add_noise_leaves_kernel<true>, dim3((unsigned)blocks),
                           dim3(kNoiseThreads), 0, s, tab);
      } else {
        hipLaunchKernelGGL(add_noise_leaves_kernel<false>, dim3((unsigned)blocks),
                           dim3(kNoiseThreads), 0, s, tab);
      }
      DPC_HIP_CHECK(hipGetLastError());
    }
  }
  return DPC_OK;
}

extern "C" int dpc_add_noise_ex(const void* x, void* y, int64_t rows, int64_t cols, int dtype,
                                int compute_dtype, double sigma, int noise_mode,
                                const void* noise, uint64_t seed, uint32_t leaf_id,
                                void* stream) {
  if (rows < 0 || cols < 0 || !(sigma >= 0.0)) return DPC_EINVAL;
  if (!known_dtype(dtype) || !known_dtype(compute_dtype)) return DPC_EINVAL;
  if (rows == 0 || cols == 0) return DPC_OK;
  if (!x || !y) return DPC_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (sigma == 0.0) {
    if (x != y) {
      DPC_HIP_CHECK(hipMemcpyAsync(y, x, (size_t)rows * cols * dtype_bytes(dtype),
                                   hipMemcpyDeviceToDevice, s));
    }
    return DPC_OK;
  }
  if (noise_mode != DPC_NOISE_INJECTED && noise_mode != DPC_NOISE_PHILOX) return DPC_EINVAL;
  if (noise_mode == DPC_NOISE_INJECTED && !noise) return DPC_EINVAL;
  const int64_t work = ((rows + 1) >> 1) * cols;
  const int64_t blocks = std::min<int64_t>((work + kNoiseThreads - 1) / kNoiseThreads, 1 << 20);
  hipLaunchKernelGGL(add_noise_generic_kernel, dim3((unsigned)blocks), dim3(kNoiseThreads), 0, s,
                     x, y, rows, cols, dtype, compute_dtype, sigma, noise_mode, noise, seed,
                     leaf_id);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
