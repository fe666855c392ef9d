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
#include <tuple>

#include "common.h"

namespace {

constexpr int kTile = 2048;
constexpr int kThreads = 256;

template <bool kBf16>
__device__ __forceinline__ float load_elem(int64_t base, int64_t idx) {
  const void* p = reinterpret_cast<const void*>(base);
  if (kBf16) return bf16_bits_to_f32(global_ptr<const uint16_t>(p)[idx]);
  return global_ptr<const float>(p)[idx];
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


// Element e of example b of leaf `base` (n elements per example).
template <bool kBf16>
__device__ __forceinline__ float elem_f32(int64_t base, int64_t idx) {
  return finite_or_zero(load_elem<kBf16>(base, idx));
}

// The 8 (bf16) or 4 (fp32) values of a 16-byte chunk, widened to fp32.
// (Each word goes through a scalar: clang's __builtin_bit_cast of a vector
// element lvalue, c[k], reads element 0 for every k.)
template <bool kBf16>
__device__ __forceinline__ void chunk_f32(u32x4_t c, float* v) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t w = c[k];
    if constexpr (kBf16) {
      v[2 * k] = __builtin_bit_cast(float, w << 16);
      v[2 * k + 1] = __builtin_bit_cast(float, w & 0xffff0000u);
    } else {
      v[k] = __builtin_bit_cast(float, w);
    }
  }
}

__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
  return v;  // lane 0
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
  return v;  // lane 0
}

// A tile can be read with 16-byte loads when it is whole and every row of
// its leaf starts 16-byte aligned.
__device__ __forceinline__ bool tile_vectorizable(int64_t base, int64_t n, int64_t off0,
                                                  int elem_bytes) {
  return (base & 15) == 0 && ((n * elem_bytes) & 15) == 0 && off0 + kTile <= n;
}

// Norm pass: one wave per (example b, tile t) unit, unit u = b * n_tiles + t
// (consecutive waves read consecutive tiles of one example).  A whole,
// aligned tile is read as 16-byte chunks, chunk j * 64 + lane for lane
// `lane` (each load instruction of the wave covers 1 KiB contiguous); each
// value is sanitised, squared in fp32 (rounded), widened and added in fp64,
// and the wave's fp64 partials are folded by a fixed shuffle tree.  The
// order of the fp64 additions inside a tile is fixed, so results are
// deterministic.  kSqBf16 (bf16 leaves, the reference's explicit
// compute_dtype=bfloat16): each square is rounded to bf16, as x * x in bf16
// is, before the fp64 sum.
#pragma clang fp contract(off)
template <bool kSqBf16>
__device__ __forceinline__ float square_in(float x) {
  const float sq = x * x;
  return kSqBf16 ? round_to_bf16(sq) : sq;
}

template <bool kBf16, bool kSqBf16 = false>
__global__ void __launch_bounds__(kThreads)
tile_sq_kernel(const int64_t* __restrict__ ptrs, const int64_t* __restrict__ sizes,
               const int32_t* __restrict__ tile_leaf, const int32_t* __restrict__ tile_local,
               int n_tiles, long long units, double* __restrict__ partial) {
  constexpr int kElemBytes = kBf16 ? 2 : 4;
  constexpr int kPerChunk = 16 / kElemBytes;
  constexpr int kChunks = kTile / kPerChunk / 64;  // per lane: 4 (bf16) or 8 (fp32)
  const long long u = (long long)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (u >= units) return;  // whole waves exit; the kernel has no barrier
  const int lane = threadIdx.x & 63;
  const int b = (int)(u / n_tiles), t = (int)(u % n_tiles);
  const int leaf = tile_leaf[t];
  const int64_t n = sizes[leaf];
  const int64_t base = ptrs[leaf];
  const int64_t off0 = (int64_t)tile_local[t] * kTile;
  double s = 0.0;
  if (tile_vectorizable(base, n, off0, kElemBytes)) {
    const auto* row = global_ptr<const u32x4_t>(
        reinterpret_cast<const void*>(base + ((int64_t)b * n + off0) * kElemBytes));
    u32x4_t c[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; ++j) c[j] = __builtin_nontemporal_load(row + j * 64 + lane);
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      float v[kPerChunk];
      chunk_f32<kBf16>(c[j], v);
#pragma unroll
      for (int k = 0; k < kPerChunk; ++k) {
        const float x = finite_or_zero(v[k]);
        const float sq = square_in<kSqBf16>(x);
        s += (double)sq;
      }
    }
  } else {
    for (int e = lane; e < kTile; e += 64) {
      const int64_t off = off0 + e;
      if (off < n) {
        const float x = elem_f32<kBf16>(base, (int64_t)b * n + off);
        const float sq = square_in<kSqBf16>(x);
        s += (double)sq;
      }
    }
  }
  s = wave_sum_f64(s);
  if (lane == 0) partial[(size_t)b * n_tiles + t] = s;
}
#pragma clang fp contract(on)

// Norm pass for any storage dtype and any square dtype (the reference's
// reduction dtype: x.to(sq_dtype) * itself, _pytree.py:284-314), one element
// per lane step: sanitised in the storage dtype, converted, squared and
// rounded to sq_dtype, widened and added in fp64.  Same units, partials and
// fixed fold as tile_sq_kernel; used for the combinations it does not take.
#pragma clang fp contract(off)
__global__ void __launch_bounds__(kThreads)
tile_sq_generic_kernel(const int64_t* __restrict__ ptrs, const int64_t* __restrict__ sizes,
                       const int32_t* __restrict__ tile_leaf, const int32_t* __restrict__ tile_local,
                       int n_tiles, long long units, int dtype, int sq_dtype,
                       double* __restrict__ partial) {
  const long long u = (long long)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (u >= units) return;
  const int lane = threadIdx.x & 63;
  const int b = (int)(u / n_tiles), t = (int)(u % n_tiles);
  const int leaf = tile_leaf[t];
  const int64_t n = sizes[leaf];
  const void* base = reinterpret_cast<const void*>(ptrs[leaf]);
  const int64_t off0 = (int64_t)tile_local[t] * kTile;
  double s = 0.0;
  for (int e = lane; e < kTile; e += 64) {
    const int64_t off = off0 + e;
    if (off < n) {
      const double x = finite_or_zero_f64(load_as_f64(base, (int64_t)b * n + off, dtype));
      const double v = round_to_dtype(x, sq_dtype);
      s += round_to_dtype(v * v, sq_dtype);
    }
  }
  s = wave_sum_f64(s);
  if (lane == 0) partial[(size_t)b * n_tiles + t] = s;
}
#pragma clang fp contract(on)

// leaf_sq[b, leaf_col[l]] = sum of leaf l's tile partials.  1024 threads;
// thread i keeps eight running sums, of the tiles t0 + i + 8192 j + 1024 r
// (r = 0..7), so eight loads are in flight (one round trip covers a leaf of
// up to 8192 tiles, 16.8M elements); the sums are then folded in a fixed
// order (pairwise over r, then the block tree): deterministic.
constexpr int kLeafSumThreads = 1024;

__global__ void __launch_bounds__(kLeafSumThreads)
leaf_sum_kernel(const double* __restrict__ partial, const int64_t* __restrict__ tile_start,
                const int32_t* __restrict__ leaf_col, int n_tiles, double* __restrict__ leaf_sq,
                int stride) {
  __shared__ double red[kLeafSumThreads / 64];
  const int l = blockIdx.x, b = blockIdx.y;
  const int64_t t0 = tile_start[l], t1 = tile_start[l + 1];
  const double* row = partial + (size_t)b * n_tiles;
  double s[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) s[r] = 0.0;
  for (int64_t t = t0 + threadIdx.x; t < t1; t += 8 * kLeafSumThreads) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t tt = t + r * kLeafSumThreads;
      if (tt < t1) s[r] += row[tt];
    }
  }
  const double v = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
  double total = block_sum_f64(v, red);
  if (threadIdx.x == 0) leaf_sq[(size_t)b * stride + leaf_col[l]] = total;
}

// stored = to_dtype(x * s), bf16 results that rounded up into the subnormal
// range zeroed (bf16 shares float32's exponent range).
template <bool kBf16>
__device__ __forceinline__ float store_round(float x, float s) {
  const float prod = x * s;
  if (!kBf16) return prod;
  const float stored = round_to_bf16(prod);
  const float sa = fabsf(stored);
  return (sa <= 1.17549435e-38f && sa > fabsf(prod)) ? 0.f : stored;
}

// Apply pass: one workgroup per tile; thread i owns the 8 consecutive
// elements 8 i .. 8 i + 7 of the tile and walks the batch in order b = 0 ..
// B - 1, loading kApplyUnroll examples ahead (one 16-byte chunk per example for
// bf16, two for fp32), so each element's fp32 sum runs in example order.
// With post_sq, each wave's sum of stored^2 over its 512 elements of example
// b goes to post_sq[b, 4 t + wave] (a fixed shuffle tree over the thread
// sums, each in element order).  Eight examples ahead rather than four:
// 206 vs 217 us for a [32, 4096 x 4096] bf16 leaf (sixteen: 212 us).
constexpr int kApplyUnroll = 8;

#pragma clang fp contract(off)
template <bool kBf16, bool kOutBf16, bool kSecond, bool kPostSq>
__global__ void __launch_bounds__(kThreads)
apply_sum_kernel(const int64_t* __restrict__ ptrs, const int64_t* __restrict__ sizes,
                 const int32_t* __restrict__ tile_leaf, const int32_t* __restrict__ tile_local,
                 const int64_t* __restrict__ out_offs, int n_tiles, int B,
                 const float* __restrict__ scale, const int32_t* __restrict__ leaf_scale_row,
                 void* __restrict__ out, void* __restrict__ out_sq, float* __restrict__ post_sq) {
  constexpr int kElemBytes = kBf16 ? 2 : 4;
  constexpr int kLoads = kBf16 ? 1 : 2;  // 16-byte chunks per thread per example
  const int t = blockIdx.x;
  const int leaf = tile_leaf[t];
  const int64_t n = sizes[leaf];
  const int64_t base = ptrs[leaf];
  const int64_t off0 = (int64_t)tile_local[t] * kTile;
  const int e0 = 8 * threadIdx.x;  // first element of this thread in the tile
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float acc[8], acc2[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = acc2[k] = 0.f;
  const float* srow = scale + (size_t)(leaf_scale_row ? leaf_scale_row[leaf] : 0) * B;
  auto add_example = [&](int b, const float* x) __attribute__((always_inline)) {
    const float sc = srow[b];
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float stored = store_round<kBf16>(finite_or_zero(x[k]), sc);
      acc[k] = acc[k] + stored;
      if (kSecond) {
        float s2 = stored * stored;
        if (kBf16) s2 = round_to_bf16(s2);
        acc2[k] = acc2[k] + s2;
      }
      if (kPostSq) sq = sq + stored * stored;
    }
    if (kPostSq) {
      sq = wave_sum_f32(sq);
      if (lane == 0) post_sq[(size_t)b * (4 * n_tiles) + 4 * t + w] = sq;
    }
  };
  if (tile_vectorizable(base, n, off0, kElemBytes)) {
    const int64_t stride = n * kElemBytes;  // bytes between examples
    const char* p = reinterpret_cast<const char*>(base) + (off0 + e0) * kElemBytes;
    int b = 0;
    for (; b + kApplyUnroll <= B; b += kApplyUnroll) {
      u32x4_t c[kApplyUnroll][kLoads];
#pragma unroll
      for (int r = 0; r < kApplyUnroll; ++r)
#pragma unroll
        for (int h = 0; h < kLoads; ++h)
          c[r][h] = __builtin_nontemporal_load(
              global_ptr<const u32x4_t>(p + (int64_t)(b + r) * stride) + h);
#pragma unroll
      for (int r = 0; r < kApplyUnroll; ++r) {
        float x[8];
        if (kBf16) {
          chunk_f32<true>(c[r][0], x);
        } else {
          chunk_f32<false>(c[r][0], x);
          chunk_f32<false>(c[r][1], x + 4);
        }
        add_example(b + r, x);
      }
    }
    for (; b < B; ++b) {
      float x[8];
      const auto* q = global_ptr<const u32x4_t>(p + (int64_t)b * stride);
      if (kBf16) {
        chunk_f32<true>(q[0], x);
      } else {
        chunk_f32<false>(q[0], x);
        chunk_f32<false>(q[1], x + 4);
      }
      add_example(b, x);
    }
  } else {
    for (int b = 0; b < B; ++b) {
      float x[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int64_t off = off0 + e0 + k;
        x[k] = off < n ? load_elem<kBf16>(base, (int64_t)b * n + off) : 0.f;
      }
      add_example(b, x);
    }
  }
  const int64_t obase = out_offs[leaf];
  constexpr int kOutBytes = kOutBf16 ? 2 : 4;
  const int64_t o = obase + off0 + e0;
  if (off0 + e0 + 8 <= n && ((o * kOutBytes) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
      (!kSecond || (reinterpret_cast<uintptr_t>(out_sq) & 15) == 0)) {
    if (kOutBf16) {
      u32x4_t v, v2;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[k] = f32x2_to_bf16x2_bits(acc[2 * k], acc[2 * k + 1]);
        v2[k] = f32x2_to_bf16x2_bits(acc2[2 * k], acc2[2 * k + 1]);
      }
      *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(out) + o) = v;
      if (kSecond) *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(out_sq) + o) = v2;
    } else {
      float4* q = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + o);
      q[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      q[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
      if (kSecond) {
        float4* q2 = reinterpret_cast<float4*>(reinterpret_cast<float*>(out_sq) + o);
        q2[0] = make_float4(acc2[0], acc2[1], acc2[2], acc2[3]);
        q2[1] = make_float4(acc2[4], acc2[5], acc2[6], acc2[7]);
      }
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t off = off0 + e0 + k;
    if (off < n) {
      if (kOutBf16) {
        reinterpret_cast<uint16_t*>(out)[obase + off] = f32_to_bf16_bits(acc[k]);
        if (kSecond) reinterpret_cast<uint16_t*>(out_sq)[obase + off] = f32_to_bf16_bits(acc2[k]);
      } else {
        reinterpret_cast<float*>(out)[obase + off] = acc[k];
        if (kSecond) reinterpret_cast<float*>(out_sq)[obase + off] = acc2[k];
      }
    }
  }
}
#pragma clang fp contract(on)

// Apply pass for any storage dtype S, multiply dtype M = promote(S, compute
// dtype), accumulation dtype A and output dtype O (_pytree.py:160-204 and
// _clipped_fun.py:112-132): per element x of example b,
//   prod   = to_M(to_M(sanitise(x)) * scale_M[b])
//   stored = to_S(prod), zeroed if it rounded up into S's subnormal range
//   sum   += to_A(stored)          (in float for A of 16 or 32 bits, in
//                                   double for A = float64: torch's
//                                   accumulation types)
//   out    = to_O(to_A(sum))
// in example order b = 0 .. B - 1.  scale_M is row r of `scale32` (already
// rounded to M, for M of at most 32 bits) or of `scale64` (M = float64).
// The second moment sums to_A(to_S(stored * stored)) the same way; post_sq
// gets, per example and wave, the fp64 sum of stored^2 over the wave's
// elements.  Layout as apply_sum_kernel: a workgroup per tile, thread i
// owns elements 8 i .. 8 i + 7.
#pragma clang fp contract(off)
__global__ void __launch_bounds__(kThreads)
apply_sum_generic_kernel(const int64_t* __restrict__ ptrs, const int64_t* __restrict__ sizes,
                         const int32_t* __restrict__ tile_leaf,
                         const int32_t* __restrict__ tile_local,
                         const int64_t* __restrict__ out_offs, int n_tiles, int B, int dtype,
                         int mult, int acc, int out_dtype, const float* __restrict__ scale32,
                         const double* __restrict__ scale64,
                         const int32_t* __restrict__ leaf_scale_row, void* __restrict__ out,
                         void* __restrict__ out_sq, double* __restrict__ post_sq) {
  const int t = blockIdx.x;
  const int leaf = tile_leaf[t];
  const int64_t n = sizes[leaf];
  const void* base = reinterpret_cast<const void*>(ptrs[leaf]);
  const int64_t off0 = (int64_t)tile_local[t] * kTile;
  const int e0 = 8 * threadIdx.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool wide = acc == DPC_F64;
  const double tiny = smallest_normal_of(dtype);
  const size_t row = (size_t)(leaf_scale_row ? leaf_scale_row[leaf] : 0) * B;
  double sum[8], sum2[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) sum[k] = sum2[k] = 0.0;
  for (int b = 0; b < B; ++b) {
    const double sc = mult == DPC_F64 ? scale64[row + b] : (double)scale32[row + b];
    double sq = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t off = off0 + e0 + k;
      if (off >= n) continue;
      const double x = finite_or_zero_f64(load_as_f64(base, (int64_t)b * n + off, dtype));
      const double prod = round_to_dtype(x * sc, mult);
      double stored = round_to_dtype(prod, dtype);
      if (fabs(stored) <= tiny && fabs(stored) > fabs(prod)) stored = 0.0;
      const double a = round_to_dtype(stored, acc);
      sum[k] = wide ? sum[k] + a : (double)((float)sum[k] + (float)a);
      if (out_sq) {
        const double a2 = round_to_dtype(round_to_dtype(stored * stored, dtype), acc);
        sum2[k] = wide ? sum2[k] + a2 : (double)((float)sum2[k] + (float)a2);
      }
      sq += stored * stored;
    }
    if (post_sq) {
      sq = wave_sum_f64(sq);
      if (lane == 0) post_sq[(size_t)b * (4 * n_tiles) + 4 * t + w] = sq;
    }
  }
  const int64_t obase = out_offs[leaf];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t off = off0 + e0 + k;
    if (off >= n) continue;
    store_from_f64(out, obase + off, round_to_dtype(round_to_dtype(sum[k], acc), out_dtype),
                   out_dtype);
    if (out_sq)
      store_from_f64(out_sq, obase + off,
                     round_to_dtype(round_to_dtype(sum2[k], acc), out_dtype), out_dtype);
  }
}
#pragma clang fp contract(on)

// out[g * B + b] = sum over columns j with col_group[j] == g of x[b, j], in
// column order (fp64): the reference's per-group accumulation in leaf order.
__global__ void __launch_bounds__(kThreads)
group_sum_kernel(const double* __restrict__ x, int B, int n, int stride, int col_stride,
                 const int32_t* __restrict__ col_group, int n_groups, double* __restrict__ out,
                 int accumulate) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * n_groups) return;
  const int g = idx / B, b = idx % B;
  double s = 0.0;
  for (int j = 0; j < n; ++j) {
    if (col_group[j] == g) s += x[(size_t)b * stride + (size_t)j * col_stride];
  }
  double* o = out + (size_t)g * B + b;
  *o = accumulate ? *o + s : s;
}

template <bool kBf16, bool kOutBf16, typename... Args>
void launch_apply(hipStream_t s, bool second, bool postsq, Args... args) {
  const dim3 grid((unsigned)std::get<5>(std::make_tuple(args...))), block(kThreads);
  if (second && postsq)
    hipLaunchKernelGGL((apply_sum_kernel<kBf16, kOutBf16, true, true>), grid, block, 0, s, args...);
  else if (second)
    hipLaunchKernelGGL((apply_sum_kernel<kBf16, kOutBf16, true, false>), grid, block, 0, s, args...);
  else if (postsq)
    hipLaunchKernelGGL((apply_sum_kernel<kBf16, kOutBf16, false, true>), grid, block, 0, s, args...);
  else
    hipLaunchKernelGGL((apply_sum_kernel<kBf16, kOutBf16, false, false>), grid, block, 0, s, args...);
}

}  // namespace

extern "C" int dpc_group_sum_f64(const double* x, int B, int n, int stride, int col_stride,
                                 const int32_t* col_group, int n_groups, double* out,
                                 int accumulate, void* stream) {
  if (B < 0 || n < 0 || stride < 1 || col_stride < 1 || n_groups < 1) return DPC_EINVAL;
  // x is [B, n] with rows `stride` apart and columns `col_stride` apart: one
  // of the two must step over the whole other dimension.
  const bool row_major = (int64_t)stride >= (int64_t)n * col_stride;
  const bool col_major = (int64_t)col_stride >= (int64_t)B * stride;
  if (!row_major && !col_major) return DPC_EINVAL;
  if (B == 0) return DPC_OK;
  if (!out || (n > 0 && (!x || !col_group))) return DPC_EINVAL;
  const int total = B * n_groups;
  hipLaunchKernelGGL(group_sum_kernel, dim3(ceil_div(total, kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, x, B, n, stride, col_stride, col_group, n_groups, out,
                     accumulate);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_leaves_sqnorm(const int64_t* ptrs, const int64_t* sizes,
                                 const int32_t* tile_leaf, const int32_t* tile_local,
                                 const int64_t* tile_start, const int32_t* leaf_col,
                                 int n_leaves, int n_tiles, int B, int dtype,
                                 int square_dtype, double* partial, double* leaf_sq,
                                 int leaf_sq_stride, void* stream) {
  if (n_leaves < 0 || n_tiles < 0 || B < 0 || leaf_sq_stride < n_leaves) return DPC_EINVAL;
  if (!known_dtype(dtype) || !known_dtype(square_dtype)) return DPC_EINVAL;
  if (B == 0 || n_leaves == 0) return DPC_OK;
  if (!ptrs || !sizes || !tile_leaf || !tile_local || !tile_start || !leaf_col || !partial ||
      !leaf_sq)
    return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  hipStream_t s = (hipStream_t)stream;
  if (n_tiles > 0) {
    const long long units = (long long)n_tiles * B;
    const long long blocks = (units + kThreads / 64 - 1) / (kThreads / 64);
    if (blocks > 0x7fffffffLL) return DPC_ENOTSUP;
    if (dtype == DPC_BF16 && square_dtype == DPC_BF16) {
      hipLaunchKernelGGL((tile_sq_kernel<true, true>), dim3((unsigned)blocks), dim3(kThreads), 0,
                         s, ptrs, sizes, tile_leaf, tile_local, n_tiles, units, partial);
    } else if (dtype == DPC_BF16 && square_dtype == DPC_F32) {
      hipLaunchKernelGGL(tile_sq_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                         ptrs, sizes, tile_leaf, tile_local, n_tiles, units, partial);
    } else if (dtype == DPC_F32 && square_dtype == DPC_F32) {
      hipLaunchKernelGGL(tile_sq_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                         ptrs, sizes, tile_leaf, tile_local, n_tiles, units, partial);
    } else {
      hipLaunchKernelGGL(tile_sq_generic_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                         ptrs, sizes, tile_leaf, tile_local, n_tiles, units, dtype, square_dtype,
                         partial);
    }
    DPC_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(leaf_sum_kernel, dim3(n_leaves, B), dim3(kLeafSumThreads), 0, s,
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
    launch_apply<true, true>(s, out_sq != nullptr, post_sq != nullptr, ptrs, sizes, tile_leaf,
                             tile_local, out_offs, n_tiles, B, scale, leaf_scale_row, out, out_sq,
                             post_sq);
  } else if (dtype == DPC_BF16) {
    launch_apply<true, false>(s, out_sq != nullptr, post_sq != nullptr, ptrs, sizes, tile_leaf,
                              tile_local, out_offs, n_tiles, B, scale, leaf_scale_row, out, out_sq,
                              post_sq);
  } else {
    launch_apply<false, false>(s, out_sq != nullptr, post_sq != nullptr, ptrs, sizes, tile_leaf,
                               tile_local, out_offs, n_tiles, B, scale, leaf_scale_row, out,
                               out_sq, post_sq);
  }
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_leaves_apply_ex(const int64_t* ptrs, const int64_t* sizes,
                                   const int32_t* tile_leaf, const int32_t* tile_local,
                                   const int64_t* out_offs, int n_tiles, int B, int dtype,
                                   int mult_dtype, int acc_dtype, const float* scale,
                                   const double* scale64, const int32_t* leaf_scale_row,
                                   void* out, void* out_sq, int out_dtype, double* post_sq,
                                   void* stream) {
  if (n_tiles < 0 || B < 0) return DPC_EINVAL;
  if (!known_dtype(dtype) || !known_dtype(mult_dtype) || !known_dtype(acc_dtype) ||
      !known_dtype(out_dtype))
    return DPC_EINVAL;
  // The multiply dtype is promote(storage, compute): never narrower than storage.
  if (dtype_bytes(mult_dtype) < dtype_bytes(dtype) ||
      (dtype_bytes(mult_dtype) == 2 && mult_dtype != dtype))
    return DPC_EINVAL;
  if (n_tiles == 0) return DPC_OK;
  if (!ptrs || !sizes || !tile_leaf || !tile_local || !out_offs || !out) return DPC_EINVAL;
  if (B > 0 && (mult_dtype == DPC_F64 ? !scale64 : !scale)) return DPC_EINVAL;
  hipLaunchKernelGGL(apply_sum_generic_kernel, dim3(n_tiles), dim3(kThreads), 0,
                     (hipStream_t)stream, ptrs, sizes, tile_leaf, tile_local, out_offs, n_tiles, B,
                     dtype, mult_dtype, acc_dtype, out_dtype, scale, scale64, leaf_scale_row, out,
                     out_sq, post_sq);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

namespace {
// out[e, :, k] = x[e, :, k] if column k of matrix e holds only finite values,
// else 0 (every row): the operands whose product G'^T A' is the reference's
// sanitised per-example gradient of a linear layer (nan_to_num of G^T A,
// _streaming.py:73,151: a non-finite A[t, k] makes column k of G^T A
// non-finite, a non-finite G[t, m] row m).  One thread per column: a pass to
// test it, a pass to copy it; consecutive threads read consecutive columns.
__global__ void __launch_bounds__(kThreads)
sanitize_columns_kernel(const void* __restrict__ x, void* __restrict__ out, int T, int d,
                        int dtype) {
  const int k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= d) return;
  const int64_t base = (int64_t)blockIdx.y * T * d + k;
  bool finite = true;
  for (int t = 0; t < T; ++t) finite = finite && isfinite(load_as_f64(x, base + (int64_t)t * d, dtype));
  for (int t = 0; t < T; ++t) {
    const int64_t i = base + (int64_t)t * d;
    store_from_f64(out, i, finite ? load_as_f64(x, i, dtype) : 0.0, dtype);
  }
}
}  // namespace

extern "C" int dpc_sanitize_columns(const void* x, void* out, int n, int T, int d, int dtype,
                                    void* stream) {
  if (n < 0 || T < 0 || d < 0 || !known_dtype(dtype)) return DPC_EINVAL;
  if (n == 0 || T == 0 || d == 0) return DPC_OK;
  if (!x || !out || n > 65535) return DPC_EINVAL;
  hipLaunchKernelGGL(sanitize_columns_kernel, dim3(ceil_div(d, kThreads), n), dim3(kThreads), 0,
                     (hipStream_t)stream, x, out, T, d, dtype);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}
