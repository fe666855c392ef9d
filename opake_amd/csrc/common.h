// Shared device/host helpers for the DP clip-and-aggregate kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "opake_amd.h"

#define DPC_HOST_DEVICE __host__ __device__ __forceinline__
#define DPC_DEVICE __device__ __forceinline__

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// A pointer to global memory as such: a pointer loaded from a device table
// has the generic address space, and accesses through it become flat
// instructions, which also count as LDS operations (so a later barrier waits
// for them to complete).
template <typename T>
DPC_DEVICE __attribute__((address_space(1))) T* global_ptr(const void* p) {
  return (__attribute__((address_space(1))) T*)(const_cast<void*>(p));
}

// vmcnt(N) with the other counters left alone (gfx9 s_waitcnt encoding):
// the wait for a wave's direct-to-LDS transfers (buffer_load ... lds), which
// the compiler does not track.
#define DPC_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | (n))

// A workgroup barrier that orders LDS only.  __syncthreads() is a release /
// acquire on all memory: after global stores it waits for them to complete
// (vmcnt(0), a memory round trip).  This one waits for the wave's LDS
// operations alone, for barriers that only hand LDS words between waves.
DPC_DEVICE void dpc_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------
// bfloat16 <-> float.  bf16 is the upper half of an IEEE binary32; the
// narrowing conversion rounds to nearest-even and keeps NaN a NaN.
// ---------------------------------------------------------------------------
DPC_HOST_DEVICE float bf16_bits_to_f32(uint16_t b) {
  union { uint32_t u; float f; } v;
  v.u = (uint32_t)b << 16;
  return v.f;
}

// On the host, branch-free (a select, not a divergent branch around the NaN
// case).  On the device, the hardware conversion (v_cvt_pk_bf16_f32), which
// returns the same bits for every one of the 2^32 inputs, NaNs included
// (checked exhaustively on the device against the host formula).
DPC_HOST_DEVICE uint16_t f32_to_bf16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  // Opaque, so that a float64 -> float32 -> bf16 chain is not folded into one
  // float64 -> bf16 conversion (one rounding where torch rounds twice).
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
  union { uint32_t u; float f; } v;
  v.f = f;
  const uint32_t u = v.u;
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet_nan = (u >> 16) | 0x0040u;
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? quiet_nan : rounded);
#endif
}

// Round a float to the nearest bf16 and widen it back (one rounding).
DPC_HOST_DEVICE float round_to_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// f32_to_bf16_bits of a and b, packed (a in the low half): on the device one
// conversion of the pair.
DPC_HOST_DEVICE uint32_t f32x2_to_bf16x2_bits(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef float f2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
  asm("" : "+v"(a), "+v"(b));  // opaque, as in f32_to_bf16_bits
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{a, b}, b2_t));
#else
  return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
#endif
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC'11).  Counter (c0..c3), key (k0, k1); ten rounds of the
// 4x32 S-box with multipliers 0xD2511F53 / 0xCD9E8D57 and Weyl key increments
// 0x9E3779B9 / 0xBB67AE85.
// ---------------------------------------------------------------------------
struct Philox4 {
  uint32_t v[4];
};

DPC_HOST_DEVICE void philox_mulhilo(uint32_t a, uint32_t b, uint32_t* hi, uint32_t* lo) {
  uint64_t p = (uint64_t)a * (uint64_t)b;
  *hi = (uint32_t)(p >> 32);
  *lo = (uint32_t)p;
}

// a ^ b ^ c; on the device one v_bitop3_b32 (gfx950's three-input bitwise
// operation, truth table 0x96 = odd parity), where the compiler emits two
// XORs.  The builtin (not inline asm) lets a uniform operand -- the Philox
// round key -- stay in its scalar register instead of being copied to a
// vector register for every use.
DPC_HOST_DEVICE uint32_t xor3_u32(uint32_t a, uint32_t b, uint32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
#else
  return a ^ b ^ c;
#endif
}

DPC_HOST_DEVICE Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                      uint32_t k0, uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    uint32_t hi0, lo0, hi1, lo1;
    philox_mulhilo(M0, c0, &hi0, &lo0);
    philox_mulhilo(M1, c2, &hi1, &lo1);
    uint32_t n0 = xor3_u32(hi1, c1, k0);
    uint32_t n1 = lo1;
    uint32_t n2 = xor3_u32(hi0, c3, k1);
    uint32_t n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += W0;
    k1 += W1;
  }
  Philox4 r;
  r.v[0] = c0; r.v[1] = c1; r.v[2] = c2; r.v[3] = c3;
  return r;
}

// Device-stream standard normals.  A leaf is viewed as a matrix
// [rows, cols] (rows = size of dim 0, cols = numel / rows; 1-D leaves are
// [n, 1]).  Element (r, c) takes normal (r & 1) of the Box-Muller pair drawn
// from Philox block ((r >> 1) * cols + c, leaf):
//   u1 = (k + 1/2) 2^-53 with k the top 53 bits of (w0 << 32 | w1)  (in (0,1))
//   u2 = (w2 + 1/2) 2^-32
//   radius = sqrt(-2 ln u1), angle = 2 pi u2,
//   z0 = radius cos(angle), z1 = radius sin(angle).
// The 53-bit u1 keeps the tail out to |z| = 8.57 (a 24-bit uniform would cut
// it at 5.9).  Evaluation is in float except for the argument reduction of
// u1: u1 = 2^e m with m in [sqrt(1/2), sqrt(2)) (exact, in double), then
// ln u1 = e ln 2 + log1p(f), f = m - 1, with log1p(f) = 2 atanh(f / (2 + f))
// from its odd Taylor series to the s^11 term (|s| <= 0.1716, truncation
// below 2e-9 relative), so ln u1 keeps its relative accuracy as u1 -> 1; the
// angle uses the hardware sine and cosine, whose argument is in revolutions
// (the reciprocal of 2 + f and the square root are the 1-ulp hardware ones).
// Against the same formulas in double precision the normals differ by less
// than 1e-6.  The function of (seed, leaf, r, c) does not depend on how a
// kernel tiles the leaf, so every kernel that writes a leaf draws the same
// stream.
// ln(x 2^escale) for x 2^escale in (0, 1): the exact power-of-two scale goes
// to the exponent frexp returns, so it costs no float64 operation.
DPC_DEVICE float ln_unit_interval(double x, int escale) {
  int e;
  double m = frexp(x, &e);  // m in [0.5, 1)
  e += escale;
  if (m < 0.70710678118654752) {
    m *= 2.0;
    e -= 1;
  }
  const float f = (float)(m - 1.0);
  const float s = f * __builtin_amdgcn_rcpf(2.0f + f);  // 1-ulp reciprocal, 2 + f in [1.7, 2.5]
  const float s2 = s * s;
  float p = 1.0f / 11.0f;
  p = fmaf(p, s2, 1.0f / 9.0f);
  p = fmaf(p, s2, 1.0f / 7.0f);
  p = fmaf(p, s2, 1.0f / 5.0f);
  p = fmaf(p, s2, 1.0f / 3.0f);
  p = fmaf(p, s2, 1.0f);
  return fmaf((float)e, 0.693147180559945309f, 2.0f * s * p);
}

DPC_DEVICE void philox_normal_pair(uint64_t seed, uint32_t leaf, uint64_t block, float* z0,
                                   float* z1) {
  Philox4 w = philox4x32_10((uint32_t)block, (uint32_t)(block >> 32), leaf, 0u,
                            (uint32_t)seed, (uint32_t)(seed >> 32));
  uint64_t bits = ((uint64_t)w.v[0] << 32) | (uint64_t)w.v[1];
  // u1 = x1 2^-53 and u2 = x2 2^-32 with x1 = k + 1/2, x2 = w2 + 1/2 in
  // double; the power-of-two scales are exact (u2 >= 2^-33 is a normal
  // float, so scaling after the rounding to float gives the same float).
  // k = bits >> 11 as hi 2^32 + lo (21 + 32 bits): lo + 1/2 and hi 2^32 are
  // exact, so the fused multiply-add rounds k + 1/2 once, as (double)k + 0.5.
  const double x1 = fma((double)(uint32_t)(bits >> 43), 0x1.0p32,
                        (double)(uint32_t)(bits >> 11) + 0.5);
  const float u2 = (float)((double)w.v[2] + 0.5) * 0x1.0p-32f;
  // -2 ln u1 >= 2.2e-16 (u1 <= 1 - 2^-54): a normal float, so the 1-ulp
  // hardware square root needs no scaling.
  float radius = __builtin_amdgcn_sqrtf(-2.0f * ln_unit_interval(x1, -53));
  *z0 = radius * __builtin_amdgcn_cosf(u2);
  *z1 = radius * __builtin_amdgcn_sinf(u2);
}

// Sanitise a float like torch.nan_to_num(nan=0, posinf=0, neginf=0).
DPC_HOST_DEVICE float finite_or_zero(float x) {
  union { uint32_t u; float f; } v;
  v.f = x;
  return ((v.u & 0x7f800000u) == 0x7f800000u) ? 0.0f : x;
}

DPC_HOST_DEVICE int ceil_div(int a, int b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// The four element types of the materialised-leaf and noise passes, carried
// as double.  Conversions follow torch's: to float16 / bfloat16 from a wider
// type goes through float32 (c10's Half(float) / BFloat16(float)), each step
// rounding to nearest even, overflow to infinity and subnormals kept.
// ---------------------------------------------------------------------------
DPC_DEVICE double load_as_f64(const void* base, int64_t idx, int dtype) {
  switch (dtype) {
    case DPC_BF16:
      return (double)bf16_bits_to_f32(global_ptr<const uint16_t>(base)[idx]);
    case DPC_F16:
      return (double)(float)global_ptr<const _Float16>(base)[idx];
    case DPC_F64:
      return global_ptr<const double>(base)[idx];
    default:
      return (double)global_ptr<const float>(base)[idx];
  }
}

// x as read from another lane by the DPP lane move kCtrl (both 32-bit halves
// from the same lane); lanes of rows outside kRowMask get 0.0.
template <int kCtrl, int kRowMask>
DPC_DEVICE double dpp_f64(double x) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, kCtrl, kRowMask, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), kCtrl, kRowMask, 0xf,
                                             false);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

// Sum of v over the 64 lanes of a wave, in a fixed order, by DPP lane moves
// (no LDS round trips): pairs, quads, half rows, rows (every lane of a row
// then holds the row's sum), then row 1 += row 0 and row 3 += row 2, then
// rows 2, 3 += row 1.  The total is in lane 63.  Every lane must be active.
DPC_DEVICE double wave_sum_lane63_f64(double v) {
  v += dpp_f64<0xB1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f64<0x4E, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f64<0x141, 0xf>(v);  // row_half_mirror
  v += dpp_f64<0x140, 0xf>(v);  // row_mirror
  v += dpp_f64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// The same total, in every lane (read from lane 63).
DPC_DEVICE double wave_sum_all_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, wave_sum_lane63_f64(v));
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), 63);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// A float the compiler must take as given: without it, a float64 -> float32
// -> float16 chain is folded into one float64 -> float16 conversion, which
// rounds once where torch rounds twice.
DPC_DEVICE float opaque_f32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// float -> float16 -> float, rounding to nearest even (v_cvt_f16_f32).
DPC_DEVICE float round_to_f16(float f) { return (float)(_Float16)opaque_f32(f); }

// v rounded to `dtype` (and widened back).
DPC_DEVICE double round_to_dtype(double v, int dtype) {
  switch (dtype) {
    case DPC_BF16:
      return (double)round_to_bf16((float)v);
    case DPC_F16:
      return (double)round_to_f16((float)v);
    case DPC_F64:
      return v;
    default:
      return (double)(float)v;
  }
}

// Stores v, which must already be a value of `dtype` (round_to_dtype).
DPC_DEVICE void store_from_f64(void* base, int64_t idx, double v, int dtype) {
  switch (dtype) {
    case DPC_BF16:
      global_ptr<uint16_t>(base)[idx] = f32_to_bf16_bits((float)v);
      break;
    case DPC_F16:
      global_ptr<_Float16>(base)[idx] = (_Float16)opaque_f32((float)v);
      break;
    case DPC_F64:
      global_ptr<double>(base)[idx] = v;
      break;
    default:
      global_ptr<float>(base)[idx] = (float)v;
  }
}

DPC_HOST_DEVICE int dtype_bytes(int dtype) {
  return dtype == DPC_F64 ? 8 : (dtype == DPC_F32 ? 4 : 2);
}

DPC_HOST_DEVICE bool known_dtype(int dtype) {
  return dtype == DPC_F32 || dtype == DPC_BF16 || dtype == DPC_F16 || dtype == DPC_F64;
}

// Smallest positive normal value of `dtype` (torch.finfo(dtype).smallest_normal).
DPC_HOST_DEVICE double smallest_normal_of(int dtype) {
  switch (dtype) {
    case DPC_F16:
      return 6.103515625e-05;  // 2^-14
    case DPC_F64:
      return 2.2250738585072014e-308;  // 2^-1022
    default:
      return 1.1754943508222875e-38;  // 2^-126
  }
}

// torch.nan_to_num(x, nan=0, posinf=0, neginf=0) of a value held as double.
DPC_HOST_DEVICE double finite_or_zero_f64(double x) { return isfinite(x) ? x : 0.0; }

// ---------------------------------------------------------------------------
// Error model of the Gram-norm kernels (the bound that makes the ghost clip
// sound: the clip factor is taken from sqnorm + sqerr >= ||G_i^T A_i||^2).
//
// A Gram entry P_st = sum_k a_sk a_tk (n products, zero-padded to the K step)
// is accumulated in a chain of fp32 MFMA instructions, each adding 16 exact
// bf16 products to the accumulator.  Model: one instruction returns its 17
// addends' sum with an error of at most 17 * 2^-23 * (sum of their
// magnitudes) -- this covers round-to-nearest, truncation, and an aligned
// fused addition that drops bits below the largest addend's ulp -- and each
// product or partial below the fp32 normal range may be flushed (an absolute
// error of at most 2^-126 each).  Then
//   |P^_st - P_st| <= gamma(n) sum_k |a_sk a_tk| + eta(n)
//                  <= gamma(n) ||a_s|| ||a_t|| + eta(n)       (Cauchy-Schwarz)
// with gamma(n) = g / (1 - g), g = (18/16) n u (u = 2^-23, one extra addend
// of slack), eta(n) = n 2^-125.  Since eta(n) <= gamma(n) 2^-102,
//   gamma ||a_s|| ||a_t|| + eta <= gamma (||a_s|| + c)(||a_t|| + c),  c = 2^-51,
// so the row weights w_s = ||a_s|| + c carry the absolute term.  The generic
// (FMA) Gram kernels accumulate in fp64: products of fp32 values are exact
// there and never underflow, so the same form holds with u = 2^-52, eta = c = 0.
// Row norms come from the computed diagonal: P^_ss >= (1 - gamma) P_ss - eta.
// ---------------------------------------------------------------------------
#define DPC_GRAM_U_MFMA 0x1.0p-23
#define DPC_GRAM_U_FP64 0x1.0p-52
#define DPC_GRAM_ROW_SLACK_MFMA 0x1.0p-51

DPC_HOST_DEVICE double dpc_chain_gamma(double n, double u) {
  const double g = 1.125 * n * u;
  if (!(g < 0.5)) return __builtin_inf();  // no useful bound: the clip factor becomes 0
  return g / (1.0 - g) * (1.0 + 0x1.0p-40);
}

// Upper bound of ||a_s|| + slack from a computed diagonal Gram entry;
// dpc_row_bound_inv takes the chain's factor dpc_row_inv(gamma) computed once
// (the same bits).
DPC_HOST_DEVICE double dpc_row_inv(double gamma) { return (1.0 + 0x1.0p-50) / (1.0 - gamma); }
DPC_HOST_DEVICE double dpc_row_bound_inv(double diag, double inv, double eta, double slack) {
  return sqrt((fabs(diag) + eta) * inv) * (1.0 + 0x1.0p-50) + slack;
}
DPC_HOST_DEVICE double dpc_row_bound(double diag, double gamma, double eta, double slack) {
  return dpc_row_bound_inv(diag, dpc_row_inv(gamma), eta, slack);
}

// Per-tile record of a Gram work item (float64, kGramRecWords words):
//   [0] inner  <P^, Q^> over the tile (x2 for an off-diagonal pair)
//   [1] FP     sum of P^_st^2 over the tile's entries with s != t
//   [2] FQ     sum of Q^_st^2 over the same entries
//   [3] XD     sum_s w_s^2 |Q^_ss|   } diagonal pairs only (0 otherwise);
//   [4] YD     sum_s v_s^2 |P^_ss|   } w_s / v_s: row weights of the P / Q
//   [5] W2     sum_s w_s^2           } operands over the block's rows
//   [6] V2     sum_s v_s^2           }
//   [7] gamma of P's chain, [8] gamma of Q's chain, [9] rows of the example
//       or segment (T), [10..11] zero.
// P is the Gram matrix of the narrower operand (d_lo), Q of the wider one.
#define DPC_GRAM_REC_WORDS 12

// Per-example bound from the records of one example / segment (nt row
// blocks, pair index q (q + 1) / 2 + p for p <= q, records rec[pair]), folded
// by the finish kernels (gram.hip: gram_bound_wave); see the model above:
//   |S - ||g||^2| <= gA X + gQ Y + (gA gQ + g64 (1 + gA)(1 + gQ)) W2 V2
//   X = sum_p XD_p + sum_p W2_p ||Q^_pp,off||_F + 2 sum_{p<q} ||w_p|| ||w_q|| ||Q^_pq||_F
//   Y likewise with V2 and P^,  g64 = (T^2 + 256) 2^-52 for the fp64 sums,
// inflated by 1 + 2^-40 for the fold's own rounding.

// Remembers the last failing HIP status of the calling thread (abi.hip).
void dpc_record_error(hipError_t e);

#define DPC_HIP_CHECK(expr)          \
  do {                               \
    hipError_t _e = (expr);          \
    if (_e != hipSuccess) {          \
      dpc_record_error(_e);          \
      return DPC_EHIP;               \
    }                                \
  } while (0)
