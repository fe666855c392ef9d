// Clipped batch sum of a linear layer's per-example weight gradients,
//   out[m, n] = sum_i scale[i] * sum_t G[i, t, m] * A[i, t, n],
// as one GEMM over K = B * T with the normalisation and the Gaussian noise
// fused into the epilogue.
//
// Fast path (bf16, T % 64 == 0, din % 8 == 0, dout % 8 == 0):
//   * 256 x 256 output tile per workgroup, 8 waves (2 per SIMD) of 128 x 64,
//     bf16 MFMA 16x16x32 with fp32 accumulators (32 blocks per wave);
//   * both operands are m- (n-) contiguous in HBM and are staged into LDS in
//     that natural [k][m] layout (64-byte blocks XOR-swizzled by the k row),
//     straight from HBM (buffer_load ... lds).  The MFMA fragments, which
//     need 8 consecutive k per lane, come out of LDS through the gfx950
//     transposing read ds_read_b64_tr_b16 (two per fragment), so no data is
//     transposed in registers; all LDS accesses are free of bank conflicts;
//   * a K step is 64 deep and never straddles two examples, so the
//     per-example scale is one scalar per step.  Dense mode applies it to the
//     fp32 accumulators: they hold the partial sum divided by the current
//     example's scale and are multiplied by scale_prev / scale_next where the
//     example changes (the clip plan lists first the examples for which this
//     stays far inside fp32, see plan.h; the others are summed after the
//     loop).  Grouped mode does the same for a problem whose scales all lie
//     in [2^-16, 2^16] (checked per workgroup: the grouped launch is two
//     launches, one per case, and a workgroup returns at once from the one
//     that does not match its problem).  Other grouped problems, and the
//     plan's other examples, stage G through registers, multiplied by the
//     power of two of the step's scale s = m 2^e (m in [1, 2)), which is
//     exact, and apply the mantissa m to the accumulators in the same way
//     (they hold the partial sum divided by the current m, rescaled by
//     m_prev / m_next where it changes).  So no operand is ever rounded:
//     each example's contribution is the fp32 sum of the exact products of
//     the given bf16 values, times its scale.
//     Examples with scale 0 are skipped through the clip plan, so their data
//     (including any NaN/Inf) is never read;
//   * two LDS stages (128 KiB), one barrier per K step; the A DMAs of step
//     s + 2 are issued right after the barrier of step s, the moment the
//     stage is free, dense mode's G DMAs of step s + 2 at the start of step
//     s + 1 (grouped mode: the scale + store of G's step s + 1 is
//     interleaved, chunk by chunk, with the MFMAs of step s, and each
//     chunk's registers are refilled with step s + 2 right after its store).
//     In dense mode a chunk whose columns lie past the matrix reads the
//     row's last 8 columns (they feed only outputs that are not stored), so
//     every transfer is in range and a lane's DMA offsets are fixed;
//   * workgroup ids are remapped so that each of the 8 XCDs owns a compact
//     block of output tiles and re-reads operand tiles from its own L2.
#include <atomic>
#include <type_traits>

#include "common.h"
#include "lds_stage.h"
#include "plan.h"

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 64, kThreads = 256;
constexpr int kFastWaves = 8;

// LDS layout of one operand tile for a 64-deep K step: 64 rows (k) of 256
// bf16 in the swizzled layout of tile_off.
constexpr int kRowBytes = kTileRowBytes;
constexpr int kOperandBytes = kBK * kRowBytes;   // 32 KiB
constexpr int kStageBytes = 2 * kOperandBytes;   // G tile + A tile


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
    global_ptr<uint16_t>(ep.out)[idx] = f32_to_bf16_bits(v);
  } else {
    global_ptr<float>(ep.out)[idx] = v;
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
      z0 = global_ptr<const float>(ep.noise)[(size_t)m * ep.N + n];
      if (m + 1 < ep.M) z1 = global_ptr<const float>(ep.noise)[(size_t)(m + 1) * ep.N + n];
    }
  }
  store_value(ep, (size_t)m * ep.N + n, finish_value(v0, ep, z0));
  if (m + 1 < ep.M) store_value(ep, (size_t)(m + 1) * ep.N + n, finish_value(v1, ep, z1));
}

// Rows m, m + 1 (m even) of columns n, n + 1 (n even, N even): v[r][c].
// Each row's two values go out in one 4-byte (bf16) or 8-byte (fp32) store.
__device__ __forceinline__ void emit_quad(const Epilogue& ep, int m, int n, const float v[2][2]) {
  if (n >= ep.N || m >= ep.M) return;
  float z[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  if (ep.sigma != 0.0f) {
    if (ep.noise_mode == DPC_NOISE_PHILOX) {
      const uint64_t blk = (uint64_t)(m >> 1) * (uint64_t)ep.N + (uint64_t)n;
      philox_normal_pair(ep.seed, ep.leaf, blk, &z[0][0], &z[1][0]);
      philox_normal_pair(ep.seed, ep.leaf, blk + 1, &z[0][1], &z[1][1]);
    } else {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if (m + r < ep.M) {
          const f32x2_t zz = *global_ptr<const f32x2_t>(ep.noise + (size_t)(m + r) * ep.N + n);
          z[r][0] = zz.x;
          z[r][1] = zz.y;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (m + r >= ep.M) break;
    const float a = finish_value(v[r][0], ep, z[r][0]);
    const float b = finish_value(v[r][1], ep, z[r][1]);
    const size_t idx = (size_t)(m + r) * ep.N + n;
    if (ep.out_bf16) {
      const uint32_t packed = f32x2_to_bf16x2_bits(a, b);
      *global_ptr<uint32_t>(reinterpret_cast<uint16_t*>(ep.out) + idx) = packed;
    } else {
      *global_ptr<f32x2_t>(reinterpret_cast<float*>(ep.out) + idx) = f32x2_t{a, b};
    }
  }
}

#pragma clang fp contract(off)
// finish_value with the epilogue's workgroup-uniform choices fixed at compile
// time (bf16 output, / normalize_by, noise added): the tile epilogues pick
// one variant per slice, so that their loops run no branch per value.
template <bool kBf, bool kNb, bool kNoise>
__device__ __forceinline__ float finish_value_t(float v, const Epilogue& ep, float z) {
  if (kBf) v = round_to_bf16(v);
  if (kNb) {
    v = v / ep.nb;
    if (kBf) v = round_to_bf16(v);
  }
  if (kNoise) {
    float t = ep.sigma * z;
    v = v + t;
    if (kBf) v = round_to_bf16(v);
  }
  return v;
}
#pragma clang fp contract(on)

// emit_quad with the choices of finish_value_t (kNoise: sigma != 0).
template <bool kBf, bool kNb, bool kNoise>
__device__ __forceinline__ void emit_quad_t(const Epilogue& ep, int m, int n, const float v[2][2]) {
  if (n >= ep.N || m >= ep.M) return;
  float z[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  if (kNoise) {
    if (ep.noise_mode == DPC_NOISE_PHILOX) {
      const uint64_t blk = (uint64_t)(m >> 1) * (uint64_t)ep.N + (uint64_t)n;
      philox_normal_pair(ep.seed, ep.leaf, blk, &z[0][0], &z[1][0]);
      philox_normal_pair(ep.seed, ep.leaf, blk + 1, &z[0][1], &z[1][1]);
    } else {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if (m + r < ep.M) {
          const f32x2_t zz = *global_ptr<const f32x2_t>(ep.noise + (size_t)(m + r) * ep.N + n);
          z[r][0] = zz.x;
          z[r][1] = zz.y;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (m + r >= ep.M) break;
    const float a = finish_value_t<kBf, kNb, kNoise>(v[r][0], ep, z[r][0]);
    const float b = finish_value_t<kBf, kNb, kNoise>(v[r][1], ep, z[r][1]);
    const size_t idx = (size_t)(m + r) * ep.N + n;
    if (kBf) {
      const uint32_t packed = f32x2_to_bf16x2_bits(a, b);
      *global_ptr<uint32_t>(reinterpret_cast<uint16_t*>(ep.out) + idx) = packed;
    } else {
      *global_ptr<f32x2_t>(reinterpret_cast<float*>(ep.out) + idx) = f32x2_t{a, b};
    }
  }
}

// Calls f(bf16 out, / normalize_by, noise) with the epilogue's choices as
// compile-time constants.
template <typename F>
__device__ __forceinline__ void with_epilogue_choices(const Epilogue& ep, F&& f) {
  using T = std::true_type;
  using Fa = std::false_type;
  const bool bf = ep.out_bf16 != 0, nb = ep.apply_nb != 0, nz = ep.sigma != 0.0f;
  if (bf) {
    if (nb) {
      if (nz) f(T(), T(), T()); else f(T(), T(), Fa());
    } else {
      if (nz) f(T(), Fa(), T()); else f(T(), Fa(), Fa());
    }
  } else {
    if (nb) {
      if (nz) f(Fa(), T(), T()); else f(Fa(), T(), Fa());
    } else {
      if (nz) f(Fa(), Fa(), T()); else f(Fa(), Fa(), Fa());
    }
  }
}

// A 16-byte chunk outside the matrix columns is given an offset past the
// buffer's range, which the hardware reads as zero.
constexpr int kOutOfRange = 0x7ff00000;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// A positive finite scale s = m 2^e with m in [1, 2): the mantissa m and the
// power of two 2^e (both exact; 2^e is subnormal below 2^-126).
__device__ __forceinline__ float scale_mantissa(float s) {
  int e;
  return 2.0f * frexpf(s, &e);
}
__device__ __forceinline__ float scale_pow2(float s) {
  int e;
  (void)frexpf(s, &e);
  return ldexpf(1.0f, e - 1);
}

// 8 bf16 multiplied by `s` in fp32, rounded to bf16 (RNE) once; exact when s
// is a power of two (barring results below the normal range).
__device__ __forceinline__ u32x4_t scale_chunk(u32x4_t x, float s) {
  u32x4_t o;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    f32x2_t v = {__builtin_bit_cast(float, x[t] << 16) * s,
                 __builtin_bit_cast(float, x[t] & 0xffff0000u) * s};
    o[t] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
  return o;
}


// Linear workgroup id -> (tile_m, tile_n) in GROUP_M order, so a group of
// tile rows shares the activation tiles.
__device__ __forceinline__ void tile_coords(int lin, int tiles_m, int tiles_n, int* tm, int* tn) {
  constexpr int kGroupM = 4;
  const int per_group = kGroupM * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = lin % per_group;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

// Hardware dispatch is round-robin over the 8 XCDs: give each XCD a
// contiguous range of linear ids, so it re-reads operand tiles from its own L2.
__device__ __forceinline__ int xcd_linear_id(int nblocks) {
  const int b = blockIdx.x;
  return (nblocks % 8 == 0) ? (b % 8) * (nblocks / 8) + b / 8 : b;
}

// Grouped mode: E independent problems of one shape (dout x din), e.g. the
// same layer of E experts.  Problem e reads rows of A_e / G_e (rows[e] rows
// each) in 64-row K steps taken from a step table: entry (row0, seg << 7 |
// valid) covers rows row0 .. row0 + valid - 1 of segment seg, whose clip
// scale is seg_scale[seg]; rows past `valid` read as zero.  Problem e's steps
// are entries step_start[e] .. step_start[e + 1] - 1.
struct GroupedTables {
  const int64_t* a_ptrs;
  const int64_t* g_ptrs;
  const int32_t* rows;
  const int32_t* steps;
  const int32_t* step_start;
  const float* seg_scale;
  const int64_t* out_ptrs;
  const int64_t* noise_ptrs;  // nullable
  const uint32_t* leaf_ids;
  const float* sigmas;
  int E;
};

// Dense multi-layer mode: layers that share the examples, the clip plan and
// the scales (one clipping group) in one launch -- layer p takes workgroups
// tile_start .. tile_start + its tiles - 1, with its own operands, shape,
// output and noise leaf.
constexpr int kMaxDense = 8;
struct DenseProblem {
  const uint16_t* A;  // [B * T, N]
  const uint16_t* G;  // [B * T, M]
  void* out;
  const float* noise;  // injected noise [M, N] (or null)
  int M, N, tile_start;
  uint32_t leaf;
  float sigma;
  int pad;
};

struct FastArgs {
  const uint16_t* A;  // [B * T, N] (dense mode)
  const uint16_t* G;  // [B * T, M]
  int T, B;
  const void* plan;
  const float* scale;
  Epilogue ep;
  GroupedTables grp;
  // Dense split-K: workgroup (split, tile) takes steps
  // [split * n / splits, (split + 1) * n / splits) of the n steps and, for
  // splits > 1, writes its raw fp32 tile to partial[split] ([M][N]); the
  // reduce kernel adds the splits in order and applies the epilogue.
  int splits;
  float* partial;
  // Dense multi-layer mode when nprob > 0 (splits is then 1; A, G and the
  // per-layer fields of ep are taken from dp).
  int nprob;
  DenseProblem dp[kMaxDense];
};

// LDS of the fast kernel: each stage's G tile and A tile in an array of its
// own (after the K loop they hold slices of the output tile).  Operands
// filled by DMA (buffer_load ... lds) sit in distinct objects so that the
// compiler sees that a DMA into one stage does not alias the reads of the
// other, and inserts no memory-counter wait before them.
constexpr int kEpiPassRows = 32;
constexpr int kEpiLd = kBN + 4;
constexpr int kG0Bytes = (kOperandBytes > kEpiPassRows * kEpiLd * 4) ? kOperandBytes
                                                                      : kEpiPassRows * kEpiLd * 4;



// The LDS arrays of the fast kernel, at namespace scope: every instantiation
// of the tile body in one kernel uses the same four arrays.
__shared__ __attribute__((aligned(16))) uint8_t lds_g0[kG0Bytes];
__shared__ __attribute__((aligned(16))) uint8_t lds_g1[kOperandBytes];
__shared__ __attribute__((aligned(16))) uint8_t lds_a0[kOperandBytes];
__shared__ __attribute__((aligned(16))) uint8_t lds_a1[kOperandBytes];

// The body of the fast kernel for one 256 x 256 output tile: kWaves = 8
// waves (2 per SIMD) of 128 x 64, each made of 8 x 4 blocks of 16 x 16
// (16x16x32 MFMA, fp32 accumulators).  (The 16x16x32 instruction sustains a
// higher clock than 32x32x16 on the same data, and 8 waves measure faster
// than 4 waves of 128 x 128 whose 256 accumulators per lane leave too few
// registers for the pipeline.)
template <bool kGrouped, bool kGdma, int kWaves, bool kHalfDma = false>
__device__ __forceinline__ void clipped_sum_tile(const FastArgs& args) {
  constexpr int kT = kWaves * 64;           // threads
  constexpr int kWavesN = kWaves / 2;       // waves along the tile columns
  constexpr int kWC = kBN / kWavesN;        // columns of a wave tile
  constexpr int kRB = 8;                    // 16-row accumulator blocks of a wave tile
  constexpr int kCB = kWC / 16;             // 16-column accumulator blocks
  typedef f32x4_t Acc;
  constexpr int kRowsPerPass = kT / 32;     // G rows staged per pass of all threads
  constexpr int kGC = kBK / kRowsPerPass;   // G chunks per thread per K step
  constexpr int kGCSub = kGC / 4;           // ... stored per phase
  constexpr int kDma = 32 / kWaves;         // 1 KiB A transfers per wave per K step
  // kHalfDma's DMA waves step kWaves rows per instruction: the same swizzle
  // (row & 7) for every instruction needs kWaves % 8 == 0.
  static_assert(!kHalfDma || (!kGrouped && kWaves % 8 == 0), "half-wave DMAs: dense, 8k waves");
  int M = args.ep.M, N = args.ep.N;
  const int T = args.T;
  int lin = xcd_linear_id(gridDim.x);
  Epilogue ep = args.ep;
  const uint16_t* Abase = args.A;
  const uint16_t* Gbase = args.G;
  if constexpr (!kGrouped) {
    if (args.nprob > 0) {
      // The layer of this workgroup (uniform, in scalar registers).
      int p = 0;
      for (int i = 1; i < args.nprob; ++i)
        if (lin >= args.dp[i].tile_start) p = i;
      p = __builtin_amdgcn_readfirstlane(p);
      const DenseProblem& P = args.dp[p];
      lin -= P.tile_start;
      M = P.M;
      N = P.N;
      Abase = P.A;
      Gbase = P.G;
      ep.M = M;
      ep.N = N;
      ep.out = P.out;
      ep.noise = P.noise;
      ep.leaf = P.leaf;
      ep.sigma = P.sigma;
    }
  }
  const int tiles_m = ceil_div(M, kBM), tiles_n = ceil_div(N, kBN);
  int grp = 0, split = 0;
  // The quotients are workgroup-uniform, but the compiler's integer division
  // leaves them in vector registers: read them into scalar ones.
  if (kGrouped) {
    grp = __builtin_amdgcn_readfirstlane(lin / (tiles_m * tiles_n));
    lin -= grp * tiles_m * tiles_n;
  } else if (args.splits > 1) {
    split = __builtin_amdgcn_readfirstlane(lin / (tiles_m * tiles_n));
    lin -= split * tiles_m * tiles_n;
  }
  int tm, tn;
  tile_coords(lin, tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  // The wave index is uniform: read it into a scalar register, so that the
  // LDS destinations of the DMAs (which go through M0) are scalar too.
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / kWavesN, wn = w % kWavesN;  // wave tile: rows wm * 128, columns wn * kWC

  int total_rows, nsteps, step0 = 0, nactive = 0, nfast = 0, step_base = 0;
  const int spe = T / kBK;
  ClipPlanView plan = clip_plan_view(const_cast<void*>(args.plan), args.B);
  if (kGrouped) {
    // Table entries of the (uniform) problem, read into scalar registers: the
    // compiler loads them into vector registers, and a buffer resource built
    // from those would make every DMA a loop over the distinct values.
    auto uniform64 = [](int64_t v) __attribute__((always_inline)) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
      return (int64_t)(((uint64_t)hi << 32) | lo);
    };
    Abase = reinterpret_cast<const uint16_t*>(uniform64(args.grp.a_ptrs[grp]));
    Gbase = reinterpret_cast<const uint16_t*>(uniform64(args.grp.g_ptrs[grp]));
    total_rows = __builtin_amdgcn_readfirstlane(args.grp.rows[grp]);
    step0 = args.grp.step_start[grp];
    nsteps = args.grp.step_start[grp + 1] - step0;
    ep.out = reinterpret_cast<void*>(args.grp.out_ptrs[grp]);
    if (args.grp.noise_ptrs) ep.noise = reinterpret_cast<const float*>(args.grp.noise_ptrs[grp]);
    ep.leaf = args.grp.leaf_ids[grp];
    ep.sigma = ep.noise_mode == DPC_NOISE_NONE ? 0.0f : args.grp.sigmas[grp];
    // Rows past a step's `valid` are fetched out of range (zero in the G tile);
    // the A tile starts from zeros so that whatever such a fetch leaves in LDS
    // is finite.
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    for (int i = tid * 16; i < kOperandBytes; i += kT * 16) {
      *reinterpret_cast<u32x4_t*>(lds_a0 + i) = zero;
      *reinterpret_cast<u32x4_t*>(lds_a1 + i) = zero;
      if constexpr (kGdma) {
        *reinterpret_cast<u32x4_t*>(lds_g0 + i) = zero;
        *reinterpret_cast<u32x4_t*>(lds_g1 + i) = zero;
      }
    }
    __syncthreads();
  } else {
    nactive = *plan.nactive;
    nfast = *plan.nfast;
    const long long all = (long long)nfast * spe;
    step_base = (int)(all * split / args.splits);
    nsteps = (int)(all * (split + 1) / args.splits) - step_base;
    total_rows = args.B * T;
  }

  Acc acc[kRB][kCB];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int j = 0; j < kCB; ++j) acc[i][j] = Acc{};

  // Dense mode: split 0 also runs the plan's slow slots (see below).
  const bool any_slow = !kGrouped && split == 0 && nactive > nfast;
  if (nsteps > 0 || any_slow) {
    __amdgpu_buffer_rsrc_t g_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Gbase), (short)0, total_rows * M * 2, 0x00020000);
    __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Abase), (short)0, total_rows * N * 2, 0x00020000);

    // The clip plan, 64 entries at a time in registers: lane l holds slot
    // base + l (dense: example index and scale; grouped: the step's first
    // row, segment/valid word and scale).  A step reads its slot with
    // v_readlane, so the K loop issues no memory operations besides the
    // operand loads.
    int plan_base = -64, plan_ex = 0, plan_pack = 0;
    float plan_sc = 0.0f;
    auto refill_plan = [&](int slot) __attribute__((always_inline)) {
      plan_base = slot & ~63;
      const int sl = plan_base + lane;
      if (kGrouped) {
        const bool in = sl < nsteps;
        plan_ex = in ? args.grp.steps[2 * (step0 + sl)] : 0;
        plan_pack = in ? args.grp.steps[2 * (step0 + sl) + 1] : 0;
        plan_sc = in ? args.grp.seg_scale[plan_pack >> 7] : 0.0f;
      } else {
        // Only the fast list's slots (the front nfast entries) are walked
        // here; the entries between it and the slow list at the back are
        // not written by the plan builder, so neither they nor the scales
        // they would index are read.
        plan_ex = sl < nfast ? plan.active[sl] : 0;
        plan_sc = sl < nfast ? args.scale[plan_ex] : 0.0f;
      }
    };
    // Dense: step t covers rows [active[t / spe] * T + (t % spe) * 64, +64).
    // Grouped: step t is table entry step0 + t.
    auto step_row0 = [&](int t, float* sc, int* valid) __attribute__((always_inline)) {
      t += step_base;  // dense split-K: this workgroup's first step
      const int slot = kGrouped ? t : t / spe;
      if (slot - plan_base >= 64) {
        refill_plan(slot);
        DPC_WAIT_VMCNT(0);  // keep the loop's memory-counter accounting exact
      }
      const int ex = __builtin_amdgcn_readlane(plan_ex, slot - plan_base);
      *sc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                          __builtin_bit_cast(int, plan_sc), slot - plan_base));
      if (kGrouped) {
        *valid = __builtin_amdgcn_readlane(plan_pack, slot - plan_base) & 127;
        return ex;
      }
      *valid = kBK;
      return ex * T + (t % spe) * kBK;
    };

    // G staging: chunk j (< kGC) of this thread is tile row r0 + kRowsPerPass j,
    // columns col .. col + 8; columns outside the matrix read as zero.  That
    // row has the same swizzle as row r0 (kRowsPerPass is a multiple of 8), so
    // chunk j is st_off + j * kRowsPerPass rows.
    const int r0 = tid >> 5, col = (tid & 31) * 8;
    const int st_off = tile_off(r0, col);
    const int g_voff = (m0 + col) * 2;
    const int g_bad = (m0 + col < M) ? 0 : kOutOfRange;
    u32x4_t g[kGC];
    auto load_chunk = [&](int row0, int valid, int j) __attribute__((always_inline)) {
      const int row = row0 + r0;
      const int bad = (kGrouped && r0 + kRowsPerPass * j >= valid) ? kOutOfRange : g_bad;
      g[j] = __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, (row * M * 2 + g_voff) | bad,
                                                   j * kRowsPerPass * M * 2, 0);
    };
    auto store_chunk = [&](uint8_t* gstage, int j, float sc) __attribute__((always_inline)) {
      *reinterpret_cast<u32x4_t*>(gstage + st_off + j * kRowsPerPass * kRowBytes) =
          scale_chunk(g[j], sc);
    };
    // A goes straight from memory into LDS (buffer_load ... lds): wave w's
    // instruction j fills the 1 KiB of tile rows 2 w + 2 kWaves j and the
    // next, lane i the 16 bytes at i * 16 -- row 2 w + 2 kWaves j + i / 32,
    // physical 16-byte slot i % 32, which holds the 8 logical columns from
    // tile_slot_col(row, i % 32).  The swizzle depends on row & 7, which is
    // the same for every j, so a lane has one column offset per operand and
    // instruction j only adds the uniform 2 kWaves j rows.
    // Grouped mode: rows past the step's `valid` and chunks whose columns lie
    // past the matrix are given an out-of-range offset (read as zero).  Dense
    // mode: every row is valid, and a chunk past the matrix reads the row's
    // last 8 columns instead -- they feed only output rows (columns) that are
    // never stored -- so every transfer is in range, the per-lane offset is
    // fixed, and the row offset of the step and instruction is the uniform
    // soffset.
    const int dma_row = 2 * w + (lane >> 5);  // + 2 kWaves j
    const int dma_col = tile_slot_col(dma_row, lane & 31);
    const int dma_voff = dma_row * N * 2 + (kGrouped ? n0 + dma_col : min(n0 + dma_col, N - 8)) * 2;
    const int dma_bad = (kGrouped && n0 + dma_col >= N) ? kOutOfRange : 0;
    // Dense mode with kHalfDma: the first half of the waves issues all the
    // transfers, as if the workgroup had kWaves / 2 waves (wave w's
    // instruction j fills tile rows 2 w + kWaves j and the next: the same
    // swizzle, row & 7, for every j), so the other half never stalls issuing
    // one.  Measured faster for launches of one round of workgroups (config
    // 2: GEMM 6 us less) and slower for four rounds (config 3: +1%), so the
    // host picks it by the number of rounds.
    auto dma_a = [&](uint8_t* astage, int row0, int valid) __attribute__((always_inline)) {
      if constexpr (kGrouped) {
#pragma unroll
        for (int j = 0; j < kDma; ++j) {
          auto* dst = (__attribute__((address_space(3))) void*)((lds_u8_t*)astage +
                                                                 (w + kWaves * j) * 1024);
          const int rows = row0 + 2 * kWaves * j;
          const int bad = dma_row >= valid - 2 * kWaves * j ? kOutOfRange : dma_bad;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, dst, 16, (rows * N * 2 + dma_voff) | bad,
                                                   0, 0, 0);
        }
      } else if constexpr (kHalfDma) {
        if (w < kWaves / 2) {
#pragma unroll
          for (int j = 0; j < 2 * kDma; ++j) {
            auto* dst = (__attribute__((address_space(3))) void*)((lds_u8_t*)astage +
                                                                   (w + kWaves / 2 * j) * 1024);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, dst, 16, dma_voff,
                                                     (row0 + kWaves * j) * N * 2, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kDma; ++j) {
          auto* dst = (__attribute__((address_space(3))) void*)((lds_u8_t*)astage +
                                                                 (w + kWaves * j) * 1024);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, dst, 16, dma_voff,
                                                   (row0 + 2 * kWaves * j) * N * 2, 0, 0);
        }
      }
    };
    // kGdma (dense mode, and grouped problems whose scales the accumulators
    // can carry): G goes into LDS by DMA too, in the same layout as A (its
    // scale is applied to the accumulators); grouped rows past `valid` and
    // columns past M read as zero, as for A.
    const int gdma_voff =
        dma_row * M * 2 + (kGrouped ? m0 + dma_col : min(m0 + dma_col, M - 8)) * 2;
    const int gdma_bad = (kGrouped && m0 + dma_col >= M) ? kOutOfRange : 0;
    auto dma_g = [&](uint8_t* gstage, int row0, int valid) __attribute__((always_inline)) {
      if constexpr (kGrouped) {
#pragma unroll
        for (int j = 0; j < kDma; ++j) {
          auto* dst = (__attribute__((address_space(3))) void*)((lds_u8_t*)gstage +
                                                                 (w + kWaves * j) * 1024);
          const int rows = row0 + 2 * kWaves * j;
          const int bad = dma_row >= valid - 2 * kWaves * j ? kOutOfRange : gdma_bad;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(g_rsrc, dst, 16,
                                                   (rows * M * 2 + gdma_voff) | bad, 0, 0, 0);
        }
      } else if constexpr (kHalfDma) {
        if (w < kWaves / 2) {
#pragma unroll
          for (int j = 0; j < 2 * kDma; ++j) {
            auto* dst = (__attribute__((address_space(3))) void*)((lds_u8_t*)gstage +
                                                                   (w + kWaves / 2 * j) * 1024);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(g_rsrc, dst, 16, gdma_voff,
                                                     (row0 + kWaves * j) * M * 2, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kDma; ++j) {
          auto* dst = (__attribute__((address_space(3))) void*)((lds_u8_t*)gstage +
                                                                 (w + kWaves * j) * 1024);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(g_rsrc, dst, 16, gdma_voff,
                                                   (row0 + 2 * kWaves * j) * M * 2, 0, 0);
        }
      }
    };

    // 16x16x32 blocks: a K step is two 32-deep sub-steps kk, each run as two
    // phases ih of 16 MFMAs -- G block rows 4 ih .. 4 ih + 3 of the wave tile
    // against its kCB A block columns.  G fragments are read per phase, A
    // fragments per sub-step.  Block rows 2 r and 2 r + 1 are the two halves
    // of a 64-byte LDS block, so the per-lane offsets are kept for even block
    // rows (columns) only; the odd one's is that offset XOR 32 (whether a
    // lane's halves are swapped depends on its row).
    // The second half of a fragment (h = 1) is 16 rows further, with the
    // same (k & 7): 16 * kRowBytes bytes.
    int g16off[4], a16off[kCB / 2];
#pragma unroll
    for (int r = 0; r < 4; ++r) g16off[r] = frag16_off(wm * 128 + r * 32, 0, lane);
#pragma unroll
    for (int r = 0; r < kCB / 2; ++r) a16off[r] = frag16_off(wn * kWC + r * 32, 0, lane);
    struct G16 {
      bf16x8_t f[4];
    };
    struct A16 {
      bf16x8_t f[kCB];
    };
    auto read_g16 = [&](const uint8_t* gstage, int kk, int ih, G16& f) __attribute__((always_inline)) {
      const int kofs = kk * 32 * kRowBytes;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int bi = 4 * ih + i, o = (g16off[bi >> 1] ^ (32 * (bi & 1))) + kofs;
        f.f[i] = join_frag(read_tr(gstage, o), read_tr(gstage, o + 16 * kRowBytes));
      }
    };
    auto read_a16 = [&](const uint8_t* astage, int kk, A16& f) __attribute__((always_inline)) {
      const int kofs = kk * 32 * kRowBytes;
#pragma unroll
      for (int j = 0; j < kCB; ++j) {
        const int o = (a16off[j >> 1] ^ (32 * (j & 1))) + kofs;
        f.f[j] = join_frag(read_tr(astage, o), read_tr(astage, o + 16 * kRowBytes));
      }
    };
    auto mma16 = [&](const G16& g, const A16& a, int ih) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kCB; ++j)
          acc[4 * ih + i][j] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(g.f[i], a.f[j], acc[4 * ih + i][j], 0, 0, 0);
    };

    // One K step on stage (gcur, acur); the A DMAs of step s + 1 into anxt
    // were issued during step s - 1.  A step is four phases (two 32-deep
    // sub-steps of two phases each).  On entry the fragments of phase 0 are
    // in flight.
    //   * Phase 0: dense mode issues the G DMAs of step s + 1 into gnxt.
    //   * Phases 0..2: the MFMAs of phase p run while the fragments of phase
    //     p + 1 are read; grouped mode: G chunks of step s + 1 go from the
    //     registers (scaled) into the other stage, and their registers are
    //     refilled with step s + 2, so each load is in flight for a whole
    //     step.
    //   * Barrier: the other stage is complete (its DMAs have landed, every G
    //     store is done), and this stage's last fragments are in registers.
    //   * Phase 3: the A DMAs of step s + 2 go into this stage (no wave reads
    //     it any more), and the phase's MFMAs run while the fragments of phase
    //     0 of step s + 1 are read from the other stage.
    // So the MFMAs of every phase, across step boundaries too, overlap the
    // reads of the next, an A DMA has a step and a quarter to land and a G
    // DMA three quarters, and the barrier is the only place a wave waits for
    // the others.  (Issuing both operands' DMAs together after the barrier
    // measured 4% slower.)  With 8 waves the sched_group_barriers interleave
    // each phase's MFMAs with the reads of the next (the scheduler would
    // otherwise bunch them); with the sched_barriers they also keep each G
    // chunk's store and reload inside its phase.  Before the barrier only
    // the kGC G loads may still be outstanding.  Past the last step the DMAs, stores and loads repeat the
    // last step's (in-range) rows into a stage no one reads: every path
    // issues the same memory operations, which keeps the counter waits exact.
    float sc_next = 0.0f;
    int row_next = 0, valid_next = kBK, valid_cur = kBK;
    // Phases 0 and 2 read 8 fragment halves (4 G fragments), phases 1 and 3
    // 16 (4 G and 4 A fragments), under 16 MFMAs each.
    auto interleave = [&](int phase) __attribute__((always_inline)) {
      if constexpr (kWaves == 8) {
#define DPC_SG(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
        // 0x008 MFMA, 0x100 LDS read, 0x002 VALU.
        if (phase & 1) {
#pragma unroll
          for (int g = 0; g < 16; ++g) {
            DPC_SG(0x008, 1); DPC_SG(0x100, 1); DPC_SG(0x002, 2);
          }
        } else {
#pragma unroll
          for (int g = 0; g < 8; ++g) {
            DPC_SG(0x008, 1); DPC_SG(0x100, 1); DPC_SG(0x002, 2);
            DPC_SG(0x008, 1); DPC_SG(0x002, 1);
          }
        }
      }
    };
    // LDS writes and global loads of the G chunks staged in a sub-step.
    auto order_stores = [&](int chunks) __attribute__((always_inline)) {
      if constexpr (kWaves == 8) {
        if (chunks == 1) {
          DPC_SG(0x200, 1); DPC_SG(0x020, 1);
        } else {
          DPC_SG(0x200, 2); DPC_SG(0x020, 2);
        }
#undef DPC_SG
      }
    };
    G16 gf0, gf1;
    A16 af0, af1;
    // The accumulators hold the partial sum divided by the accumulator factor
    // of the step whose MFMAs run (sc_cur): dense mode, the example's scale;
    // grouped mode, the mantissa of the segment's scale (its power of two
    // multiplies G).  When the next step's factor differs they are multiplied
    // by sc_cur / sc_next.
    float sc_cur = 0.0f;
    auto acc_factor = [&](float sc) __attribute__((always_inline)) {
      return kGdma ? sc : scale_mantissa(sc);
    };
    auto rescale = [&](float r) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < kRB; ++i)
#pragma unroll
        for (int j = 0; j < kCB; ++j) acc[i][j] *= r;
    };
    auto k_step = [&](int s, uint8_t* gcur, uint8_t* acur, uint8_t* gnxt,
                      uint8_t* anxt) __attribute__((always_inline)) {
      const float sc_s1 = acc_factor(sc_next);  // accumulator factor of step s + 1
      const float g_next = kGdma ? 1.0f : scale_pow2(sc_next);  // G factor of step s + 1
      float sc_after;
      int valid2;
      const int row2 = step_row0(min(s + 2, nsteps - 1), &sc_after, &valid2);
      // Grouped mode: a segment's last step may hold fewer than 64 rows; the
      // MFMAs of a 32-row sub-step past them (all zeros) are skipped.
      const int vcur = kGrouped ? valid_cur : kBK;
      auto stage_g = [&](int kk) __attribute__((always_inline)) {
        if constexpr (!kGdma) {
#pragma unroll
          for (int c = 0; c < kGCSub; ++c) store_chunk(gnxt, kk * kGCSub + c, g_next);
#pragma unroll
          for (int c = 0; c < kGCSub; ++c) load_chunk(row2, valid2, kk * kGCSub + c);
        }
      };
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kGdma) dma_g(gnxt, row_next, valid_next);
      read_g16(gcur, 0, 1, gf1);
      mma16(gf0, af0, 0);
      stage_g(0);
      interleave(0);
      order_stores(1);
      __builtin_amdgcn_sched_barrier(0);
      read_g16(gcur, 1, 0, gf0);
      read_a16(acur, 1, af1);
      mma16(gf1, af0, 1);
      stage_g(1);
      interleave(1);
      order_stores(1);
      __builtin_amdgcn_sched_barrier(0);
      read_g16(gcur, 1, 1, gf1);
      if (vcur > 32) mma16(gf0, af1, 0);
      stage_g(2);
      stage_g(3);
      interleave(2);
      order_stores(2);
      __builtin_amdgcn_sched_barrier(0);
      sc_next = sc_after;
      row_next = row2;
      valid_cur = valid_next;
      valid_next = valid2;
      DPC_WAIT_VMCNT(kGdma ? 0 : kGC);
      __syncthreads();
      // Every wave has read this stage for the last time: the A DMAs of step
      // s + 2 go into it now, a quarter step before the next step starts.
      dma_a(acur, row_next, valid_next);
      read_g16(gnxt, 0, 0, gf0);
      read_a16(anxt, 0, af0);
      if (vcur > 32) mma16(gf1, af1, 1);
      interleave(3);
      __builtin_amdgcn_sched_barrier(0);
      if (s + 1 < nsteps && sc_s1 != sc_cur) {
        rescale(sc_cur / sc_s1);
        sc_cur = sc_s1;
      }
    };

    uint8_t* g0 = lds_g0;
    uint8_t* g1 = lds_g1;
    if (nsteps > 0) {
      // Prologue: step 0 into stage 0 (A by DMA; G by DMA in dense mode, else
      // through registers, scaled), step 1's A DMAs, in grouped mode step 1 of
      // G into the registers (dense mode: step 0's phase 0 issues step 1's G
      // DMAs); the fragments of step 0's first sub-step.
      int valid0;
      int row0 = step_row0(0, &sc_next, &valid0);
      valid_cur = valid0;
      sc_cur = acc_factor(sc_next);
      dma_a(lds_a0, row0, valid0);
      if constexpr (!kGdma) {
        const float g0f = scale_pow2(sc_next);
#pragma unroll
        for (int j = 0; j < kGC; ++j) load_chunk(row0, valid0, j);
#pragma unroll
        for (int j = 0; j < kGC; ++j) store_chunk(g0, j, g0f);
      } else {
        dma_g(g0, row0, valid0);
      }
      row_next = step_row0(min(1, nsteps - 1), &sc_next, &valid_next);
      dma_a(lds_a1, row_next, valid_next);
      if constexpr (!kGdma) {
#pragma unroll
        for (int j = 0; j < kGC; ++j) load_chunk(row_next, valid_next, j);
      }
      // Step 0's transfers have landed (step 1's DMAs and G loads may not;
      // with kHalfDma a DMA wave has 2 kDma of step 1's in flight, the
      // others none).
      if constexpr (kHalfDma) {
        DPC_WAIT_VMCNT(2 * kDma);
      } else {
        DPC_WAIT_VMCNT(kGdma ? kDma : kDma + kGC);
      }
      __syncthreads();
      read_g16(g0, 0, 0, gf0);
      read_a16(lds_a0, 0, af0);
      int s = 0;
      for (; s + 1 < nsteps; s += 2) {
        k_step(s, g0, lds_a0, g1, lds_a1);
        k_step(s + 1, g1, lds_a1, g0, lds_a0);
      }
      if (s < nsteps) k_step(s, g0, lds_a0, g1, lds_a1);
      rescale(sc_cur);
      DPC_WAIT_VMCNT(0);
      __syncthreads();
    }
    // Dense mode, examples whose scale the accumulators cannot be divided by
    // (the plan's back list; split 0 takes them), one unpipelined K step at a
    // time: G is multiplied by the power of two of the scale (exact) and the
    // accumulators carry the mantissa, as in grouped mode (after the loop
    // above they hold the finished sum, factor 1).
    if constexpr (!kGrouped) {
      const int nslow = split == 0 ? (nactive - nfast) * spe : 0;
      float m_cur = 1.0f;
      for (int t = 0; t < nslow; ++t) {
        const int ex = plan.active[args.B - 1 - t / spe];
        const float sc = args.scale[ex];
        const float m = scale_mantissa(sc);
        if (m != m_cur) {
          rescale(m_cur / m);
          m_cur = m;
        }
        const int rs = ex * T + (t % spe) * kBK;
        dma_a(lds_a0, rs, kBK);
#pragma unroll
        for (int j = 0; j < kGC; ++j) load_chunk(rs, kBK, j);
        const float p2 = scale_pow2(sc);
#pragma unroll
        for (int j = 0; j < kGC; ++j) store_chunk(g0, j, p2);
        DPC_WAIT_VMCNT(0);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          read_a16(lds_a0, kk, af0);
          read_g16(g0, kk, 0, gf0);
          mma16(gf0, af0, 0);
          read_g16(g0, kk, 1, gf0);
          mma16(gf0, af0, 1);
        }
        __syncthreads();
      }
      if (m_cur != 1.0f) rescale(m_cur);
    }
  }

  // Two epilogues: the grouped kernels write the tile in two 128-row halves,
  // which frees half the accumulators before any store; the dense kernel,
  // whose back list leaves no registers to spare, keeps eight 32-row slices
  // (the halves would spill in its K loop).
  if constexpr (kGrouped) {
    // Epilogue: the 256 x 256 fp32 tile goes through LDS in two halves of 128
    // rows -- half h holds block rows 4h .. 4h + 3 of both wave rows (tile
    // rows 64 h .. 64 h + 63 and 128 + 64 h ..), one 32-row quarter in each of
    // the four LDS arrays, columns XOR-swizzled by 16-float groups so that the
    // four row groups of a 16x16 block's write land on distinct banks.  After
    // half 0 those accumulators are dead in every wave, and half 1 has more
    // registers.  Each thread owns a pair of adjacent columns and 32 rows of a
    // half, walked in even/odd row pairs: coalesced 4- or 8-byte stores, one
    // Philox block per (row pair, column).  (Staging 32-row slices, and
    // writing each lane's accumulators straight out without LDS, measured
    // slower.)
    static_assert(kT == 512 && kRB == 8, "two 128-row halves of 512 threads");
    auto quarter = [&](int qi) __attribute__((always_inline)) {
      return qi == 0 ? lds_g0 : qi == 1 ? lds_g1 : qi == 2 ? lds_a0 : lds_a1;
    };
    auto tile_off_epi = [](int row, int col) __attribute__((always_inline)) {
      return row * kBN + (col ^ (((row >> 2) & 3) << 4));
    };
    const int eq = tid >> 7;  // emission quarter
    const int cl = 2 * (tid & 127);
    auto half = [&](auto H) __attribute__((always_inline)) {
      constexpr int h = decltype(H)::value;
      // Block row 4 h + ib (ib < 4) of wave row wm goes to quarter 2 wm + ib / 2,
      // rows 16 (ib % 2) + 4 (lane / 16) + r.
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        float* q = reinterpret_cast<float*>(quarter(2 * wm + (ib >> 1)));
#pragma unroll
        for (int j = 0; j < kCB; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int ml = 16 * (ib & 1) + 4 * (lane >> 4) + r;
            const int nl = wn * kWC + j * 16 + (lane & 15);
            q[tile_off_epi(ml, nl)] = acc[4 * h + ib][j][r];
          }
      }
      __syncthreads();
      // Quarter eq: tile rows (eq < 2 ? 0 : 128) + 64 h + 32 (eq & 1) + 0 .. 31.
      const float* qr = reinterpret_cast<const float*>(quarter(eq));
      const int mbase = m0 + (eq < 2 ? 0 : 128) + 64 * h + 32 * (eq & 1);
      const int n = n0 + cl;
      if (!kGrouped && args.splits > 1) {
        // Split-K: the raw fp32 tile; the reduce kernel finishes it.
        auto* part = global_ptr<float>(args.partial + (size_t)split * M * N);
#pragma unroll 4
        for (int ml = 0; ml < 32; ++ml) {
          const int m = mbase + ml;
          if (m < M && n < N)
            *reinterpret_cast<__attribute__((address_space(1))) f32x2_t*>(part + (size_t)m * N + n) =
                *reinterpret_cast<const f32x2_t*>(qr + tile_off_epi(ml, cl));
        }
      } else {
          with_epilogue_choices(ep, [&](auto BF, auto NB, auto NZ) __attribute__((always_inline)) {
#pragma unroll 2
          for (int ml = 0; ml < 32; ml += 2) {
            const float2 t0 = *reinterpret_cast<const float2*>(qr + tile_off_epi(ml, cl));
            const float2 t1 = *reinterpret_cast<const float2*>(qr + tile_off_epi(ml + 1, cl));
            const float v[2][2] = {{t0.x, t0.y}, {t1.x, t1.y}};
            emit_quad_t<decltype(BF)::value, decltype(NB)::value, decltype(NZ)::value>(
                ep, mbase + ml, n, v);
          }
        });
      }
      __syncthreads();
    };
    half(std::integral_constant<int, 0>());
    half(std::integral_constant<int, 1>());
  } else {
    // Epilogue: the 256 x 256 fp32 tile goes through LDS in eight slices of 32
    // rows; each thread owns a pair of adjacent columns and 32 / (kT / 128) of
    // the slice's rows, walked in even/odd row pairs: coalesced 4- or 8-byte
    // stores, and one Philox block per (row pair, column) in a rolled loop.
    // The usual choices (bf16 output, no / normalize_by, noise added) have a
    // copy of their own with no branch per value; the others take the general
    // one.
    float* tile = reinterpret_cast<float*>(lds_g0);
    constexpr int kEpiRows = kEpiPassRows / (kT / 128);
    auto epilogue = [&](auto Usual) __attribute__((always_inline)) {
      // Unrolled: the accumulator blocks are selected by compile-time indices
      // (a runtime index would move them to scratch memory).
#pragma unroll
      for (int e = 0; e < kBM / kEpiPassRows; ++e) {
        if (wm == (e >> 2)) {
          // 16x16 block (i, j): lane l holds rows 4 (l / 16) + r of column l % 16.
#pragma unroll
          for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
            for (int j = 0; j < kCB; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int ml = 16 * i2 + 4 * (lane >> 4) + r;
                const int nl = wn * kWC + j * 16 + (lane & 15);
                tile[ml * kEpiLd + nl] = acc[2 * (e & 3) + i2][j][r];
              }
        }
        __syncthreads();
        const int cl = 2 * (tid & 127);
        const int rr = (tid >> 7) * kEpiRows;
        if (!decltype(Usual)::value && !kGrouped && args.splits > 1) {
          // Split-K: the raw fp32 tile; the reduce kernel finishes it.
          auto* part = global_ptr<float>(args.partial + (size_t)split * M * N);
#pragma unroll 2
          for (int ml = rr; ml < rr + kEpiRows; ++ml) {
            const int m = m0 + e * kEpiPassRows + ml, n = n0 + cl;
            if (m < M && n < N)
              *reinterpret_cast<__attribute__((address_space(1))) f32x2_t*>(part + (size_t)m * N +
                                                                          n) =
                  *reinterpret_cast<const f32x2_t*>(tile + ml * kEpiLd + cl);
          }
        } else {
#pragma unroll 2
          for (int ml = rr; ml < rr + kEpiRows; ml += 2) {
            const float2 t0 = *reinterpret_cast<const float2*>(tile + ml * kEpiLd + cl);
            const float2 t1 = *reinterpret_cast<const float2*>(tile + (ml + 1) * kEpiLd + cl);
            const float v[2][2] = {{t0.x, t0.y}, {t1.x, t1.y}};
            if constexpr (decltype(Usual)::value)
              emit_quad_t<true, false, true>(ep, m0 + e * kEpiPassRows + ml, n0 + cl, v);
            else
              emit_quad(ep, m0 + e * kEpiPassRows + ml, n0 + cl, v);
          }
        }
        __syncthreads();
      }
    };
    if ((kGrouped || args.splits == 1) && ep.out_bf16 && !ep.apply_nb && ep.sigma != 0.0f)
      epilogue(std::true_type());
    else
      epilogue(std::false_type());
  }
}

// 8 waves (2 per SIMD) measure faster than the 4-wave 128 x 128 layout on
// both the dense and the grouped workloads.  (Launch bounds must not depend on
// a template parameter: the host stub of such a kernel is not emitted.)
// Grouped mode: whether the scales of this workgroup's problem let the
// accumulators carry them (every step's scale in [2^-16, 2^16], so the
// accumulators never hold more than 2^16 times the sum computed so far):
// then G goes in by DMA (kGdma), else through registers.  Called by every
// thread; the result is workgroup-uniform.
__device__ __forceinline__ bool grouped_scales_fit(const FastArgs& args) {
  const int tiles = ceil_div(args.ep.M, kBM) * ceil_div(args.ep.N, kBN);
  const int grp = xcd_linear_id(gridDim.x) / tiles;
  const int s0 = args.grp.step_start[grp], s1 = args.grp.step_start[grp + 1];
  int fit = 1;
  for (int i = s0 + (int)threadIdx.x; i < s1; i += (int)blockDim.x) {
    const float sc = args.grp.seg_scale[args.grp.steps[2 * i + 1] >> 7];
    fit &= (sc >= 0x1.0p-16f && sc <= 0x1.0p16f) ? 1 : 0;
  }
  return __syncthreads_and(fit) != 0;
}

// Dense mode: G by DMA.  Grouped mode: one launch in which each workgroup
// takes the body that matches its problem's scales (both bodies share the
// LDS arrays).
template <bool kGrouped, bool kHalfDma = false>
__global__ void __launch_bounds__(kFastWaves * 64, 1) clipped_sum_bf16_kernel(FastArgs args) {
  if constexpr (kGrouped) {
    if (grouped_scales_fit(args))
      clipped_sum_tile<true, true, kFastWaves>(args);
    else
      clipped_sum_tile<true, false, kFastWaves>(args);
  } else {
    clipped_sum_tile<false, true, kFastWaves, kHalfDma>(args);
  }
}

// Compute units of the current device (cached per device; 256 if unknown).
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Dense launches of at most one workgroup per compute unit take the
// half-wave DMA body (see clipped_sum_tile).
template <bool kGrouped>
void launch_fast(dim3 grid, hipStream_t s, const FastArgs& args) {
  if (!kGrouped && (int)grid.x <= device_cus())
    hipLaunchKernelGGL((clipped_sum_bf16_kernel<false, true>), grid, dim3(kFastWaves * 64), 0, s,
                       args);
  else
    hipLaunchKernelGGL((clipped_sum_bf16_kernel<kGrouped>), grid, dim3(kFastWaves * 64), 0, s,
                       args);
}

// Split-K finish: out = epilogue(sum over splits of partial[split], in
// order).  One thread per (row pair, column pair); M and N are even.
__global__ void __launch_bounds__(kThreads)
split_reduce_kernel(const float* __restrict__ partial, int splits, Epilogue ep) {
  const int half_n = ep.N / 2;
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long long)(ep.M / 2) * half_n) return;
  const int m = 2 * (int)(idx / half_n), n = 2 * (int)(idx % half_n);
  const size_t plane = (size_t)ep.M * ep.N;
  float v[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
  for (int sp = 0; sp < splits; ++sp) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float2 t = *reinterpret_cast<const float2*>(partial + sp * plane +
                                                        (size_t)(m + r) * ep.N + n);
      v[r][0] += t.x;
      v[r][1] += t.y;
    }
  }
  emit_quad(ep, m, n, v);
}

// Split-K factor of a dense fast-path launch: launches of fewer than 192
// output tiles (on 256 CUs) take their K steps in up to 8 slices so that the
// grid fills the chip; the slices' fp32 tiles go through a workspace.
int fast_splits(int B, int T, int din, int dout) {
  const int ntiles = ceil_div(dout, kBM) * ceil_div(din, kBN);
  if (ntiles >= 192) return 1;
  int splits = 1;
  const long long steps = (long long)B * (T / kBK);
  while (splits < 8 && ntiles * splits * 2 <= 256 && steps >= 8LL * splits * 2) splits *= 2;
  return splits;
}

#undef DPC_WAIT_VMCNT

// Generic path: any T, float32 or bf16 operands; 64 x 64 tiles with a 4 x 4
// FMA block per thread.  K is walked in chunks of at most 16 rows that never
// straddle two examples: G is staged multiplied by the power of two of its
// example's scale (exact) and the accumulators carry the mantissa (they hold
// the partial sum divided by the current mantissa, rescaled where it
// changes), so no operand is rounded; examples with scale 0 are skipped.
constexpr int kGT = 64, kGK = 16;

template <typename In>
__device__ __forceinline__ float to_f32(In v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_bits_to_f32(v); }

// Stages rows [k0, k0 + rows) (rows <= kGK; the rest zero) of G and A for
// the 64 x 64 tile (m0, n0), then adds their products to acc.  G is
// multiplied by p2 -- or, with kRowScale (one token per example: row k is
// example k), by row k's own scale, and rows with scale 0 are not read.
template <typename In, bool kRowScale>
__device__ __forceinline__ void generic_chunk(const In* __restrict__ A, const In* __restrict__ G,
                                              long long k0, int rows, float p2,
                                              const float* __restrict__ scale, int M, int N,
                                              int m0, int n0, float (*sg)[kGT + 1],
                                              float (*sa)[kGT + 1], float acc[4][4]) {
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  for (int e = tid; e < kGK * kGT; e += kThreads) {
    const int k = e / kGT, col = e % kGT;
    float gv = 0.f, av = 0.f;
    const float sk = kRowScale ? (k < rows ? scale[k0 + k] : 0.0f) : p2;
    if (k < rows && (!kRowScale || sk > 0.0f)) {
      const long long kk = k0 + k;
      if (m0 + col < M) gv = sk * to_f32<In>(G[kk * M + m0 + col]);
      if (n0 + col < N) av = to_f32<In>(A[kk * N + n0 + col]);
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

__device__ __forceinline__ void generic_rescale(float acc[4][4], float r) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] *= r;
}

// Split-K (splits > 1, M and N even): workgroup z sums the K range
// [z * per, (z + 1) * per) and writes its raw fp32 tile to partial[z]
// ([M][N]); split_reduce_kernel adds the splits in order and applies the
// epilogue.
template <typename In>
__global__ void __launch_bounds__(kThreads)
clipped_sum_generic_kernel(const In* __restrict__ A, const In* __restrict__ G,
                           const float* __restrict__ scale, int B, int T, Epilogue ep,
                           int splits, long long per, float* __restrict__ partial) {
  __shared__ float sg[kGK][kGT + 1];
  __shared__ float sa[kGK][kGT + 1];
  const int M = ep.M, N = ep.N;
  const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long long K = (long long)B * T;
  const long long kb = (long long)blockIdx.z * per;
  const long long ke = kb + per < K ? kb + per : K;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  float m_cur = 1.0f;
  if (T == 1) {
    // One token per example: the example's gradient is the outer product
    // g a^T, so rounding s g in fp32 changes its norm by at most the
    // relative rounding of the scaled multiply that the guard already
    // covers (as for a materialised gradient); kGK examples per chunk.
    for (long long k0 = kb; k0 < ke; k0 += kGK) {
      const long long k1 = k0 + kGK < ke ? k0 + kGK : ke;
      generic_chunk<In, true>(A, G, k0, (int)(k1 - k0), 1.0f, scale, M, N, m0, n0, sg, sa, acc);
    }
  }
  for (long long k0 = T == 1 ? ke : kb; k0 < ke;) {
    const long long ex = k0 / T, ex_end = (ex + 1) * T;
    const float s = scale[ex];  // uniform over the workgroup
    if (!(s > 0.0f)) {
      k0 = ex_end < ke ? ex_end : ke;
      continue;
    }
    long long k1 = k0 + kGK;
    k1 = k1 < ke ? k1 : ke;
    k1 = k1 < ex_end ? k1 : ex_end;
    const float m = scale_mantissa(s);
    if (m != m_cur) {
      generic_rescale(acc, m_cur / m);
      m_cur = m;
    }
    generic_chunk<In, false>(A, G, k0, (int)(k1 - k0), scale_pow2(s), nullptr, M, N, m0, n0, sg, sa,
                             acc);
    k0 = k1;
  }
  generic_rescale(acc, m_cur);
  if (splits > 1) {
    float* part = partial + (size_t)blockIdx.z * M * N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = m0 + tr * 4 + i, n = n0 + tc * 4 + j;
        if (m < M && n < N) part[(size_t)m * N + n] = acc[i][j];
      }
    return;
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

// Split-K factor of the generic kernel: enough workgroups for the CUs
// (512), K slices of at least 64 rows, M and N even (split_reduce_kernel
// works on 2 x 2 blocks).
int generic_splits(int B, int T, int din, int dout) {
  if (din % 2 != 0 || dout % 2 != 0) return 1;
  const long long tiles = (long long)ceil_div(din, kGT) * ceil_div(dout, kGT);
  const long long K = (long long)B * T;
  long long splits = (512 + tiles - 1) / tiles;
  splits = splits < K / 64 ? splits : K / 64;
  return (int)(splits < 1 ? 1 : (splits > 32 ? 32 : splits));
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

// Grouped generic path (float32, or bf16 of any shape): problem blockIdx.z,
// 64 x 64 output tiles, the steps of the problem walked in chunks of 16
// rows, G times the power of two of the step's segment scale and the
// mantissa on the accumulators (as in clipped_sum_generic_kernel).
template <typename In>
__global__ void __launch_bounds__(kThreads)
grouped_generic_kernel(GroupedTables grp, Epilogue ep0) {
  __shared__ float sg[kGK][kGT + 1];
  __shared__ float sa[kGK][kGT + 1];
  const int e = blockIdx.z;
  Epilogue ep = ep0;
  ep.out = reinterpret_cast<void*>(grp.out_ptrs[e]);
  if (grp.noise_ptrs) ep.noise = reinterpret_cast<const float*>(grp.noise_ptrs[e]);
  ep.leaf = grp.leaf_ids[e];
  ep.sigma = ep.noise_mode == DPC_NOISE_NONE ? 0.0f : grp.sigmas[e];
  const In* A = reinterpret_cast<const In*>(grp.a_ptrs[e]);
  const In* G = reinterpret_cast<const In*>(grp.g_ptrs[e]);
  const int M = ep.M, N = ep.N;
  const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  float m_cur = 1.0f;
  const int s0 = grp.step_start[e], s1 = grp.step_start[e + 1];
  for (int st = s0; st < s1; ++st) {
    const int row0 = grp.steps[2 * st];
    const int pack = grp.steps[2 * st + 1];
    const int valid = pack & 127;
    const float sc = grp.seg_scale[pack >> 7];  // > 0: the plan lists no other segment
    const float m = scale_mantissa(sc);
    if (m != m_cur) {
      generic_rescale(acc, m_cur / m);
      m_cur = m;
    }
    const float p2 = scale_pow2(sc);
    for (int k0 = 0; k0 < valid; k0 += kGK)
      generic_chunk<In, false>(A, G, (long long)row0 + k0, min(kGK, valid - k0), p2, nullptr, M, N,
                               m0, n0, sg, sa, acc);
  }
  generic_rescale(acc, m_cur);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + tc * 4 + j;
#pragma unroll
    for (int i = 0; i < 4; i += 2) emit_pair(ep, m0 + tr * 4 + i, n, acc[i][j], acc[i + 1][j]);
  }
}

// Step table of the grouped clipped sum: segments with a positive scale, in
// segment order, cut into 64-row steps; group e's steps start at
// step_start[e] (segments must be sorted by group).
constexpr int kPlanThreads = 256;
constexpr int kMaxPlanGroups = 4096;

__global__ void __launch_bounds__(kPlanThreads)
segment_plan_kernel(const int32_t* __restrict__ seg_row0, const int32_t* __restrict__ seg_len,
                    const int32_t* __restrict__ seg_group, const float* __restrict__ seg_scale,
                    int S, int E, int max_steps, int32_t* __restrict__ steps,
                    int32_t* __restrict__ step_start) {
  __shared__ int gcount[kMaxPlanGroups];
  __shared__ int wave_total[kPlanThreads / 64];
  __shared__ int base;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int g = tid; g < E; g += kPlanThreads) gcount[g] = 0;
  if (tid == 0) base = 0;
  __syncthreads();
  for (int start = 0; start < S; start += kPlanThreads) {
    const int v = start + tid;
    int cnt = 0;
    if (v < S && seg_scale[v] > 0.0f && seg_len[v] > 0) cnt = ceil_div(seg_len[v], kBK);
    int incl = cnt;
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    if (lane == 63) wave_total[w] = incl;
    __syncthreads();
    int pos = base + incl - cnt;
    for (int u = 0; u < w; ++u) pos += wave_total[u];
    for (int j = 0; j < cnt; ++j) {
      const int idx = pos + j;
      if (idx < max_steps) {
        steps[2 * idx] = seg_row0[v] + j * kBK;
        steps[2 * idx + 1] = (v << 7) | min(kBK, seg_len[v] - j * kBK);
      }
    }
    if (cnt > 0) atomicAdd(&gcount[min(max(seg_group[v], 0), E - 1)], cnt);
    __syncthreads();
    if (tid == 0) {
      int total = 0;
      for (int u = 0; u < kPlanThreads / 64; ++u) total += wave_total[u];
      base += total;
    }
    __syncthreads();
  }
  if (tid == 0) {
    int acc = 0;
    for (int g = 0; g < E; ++g) {
      step_start[g] = min(acc, max_steps);
      acc += gcount[g];
    }
    step_start[E] = min(acc, max_steps);
  }
}

}  // namespace

extern "C" int dpc_segment_plan(const int32_t* seg_row0, const int32_t* seg_len,
                                const int32_t* seg_group, const float* seg_scale, int S, int E,
                                int max_steps, int32_t* steps, int32_t* step_start, void* stream) {
  if (S < 0 || E < 1 || max_steps < 0) return DPC_EINVAL;
  if (E > kMaxPlanGroups || S >= (1 << 24)) return DPC_ENOTSUP;
  if (!step_start || (S > 0 && (!seg_row0 || !seg_len || !seg_group || !seg_scale)) ||
      (max_steps > 0 && !steps))
    return DPC_EINVAL;
  hipLaunchKernelGGL(segment_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream,
                     seg_row0, seg_len, seg_group, seg_scale, S, E, max_steps, steps, step_start);
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

extern "C" int dpc_grouped_clipped_sum(const int64_t* a_ptrs, const int64_t* g_ptrs,
                                       const int32_t* rows, int max_rows, int E, int din, int dout,
                                       int dtype, const int32_t* steps, const int32_t* step_start,
                                       const float* seg_scale, double normalize_by, int noise_mode,
                                       const int64_t* noise_ptrs, uint64_t seed,
                                       const uint32_t* leaf_ids, const float* sigmas,
                                       int out_dtype, const int64_t* out_ptrs, void* stream) {
  if (E < 0 || max_rows < 0 || din <= 0 || dout <= 0) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (out_dtype != DPC_F32 && out_dtype != DPC_BF16) return DPC_EINVAL;
  if (!(normalize_by > 0.0)) return DPC_EINVAL;
  if (noise_mode < DPC_NOISE_NONE || noise_mode > DPC_NOISE_PHILOX) return DPC_EINVAL;
  if (E == 0) return DPC_OK;
  if (!a_ptrs || !g_ptrs || !rows || !step_start || !seg_scale || !leaf_ids || !sigmas ||
      !out_ptrs || !steps)
    return DPC_EINVAL;
  if (noise_mode == DPC_NOISE_INJECTED && !noise_ptrs) return DPC_EINVAL;
  if (E > 65535) return DPC_ENOTSUP;
  hipStream_t s = (hipStream_t)stream;
  Epilogue ep;
  ep.M = dout;
  ep.N = din;
  ep.nb = (float)normalize_by;
  ep.apply_nb = normalize_by != 1.0;
  ep.noise_mode = noise_mode;
  ep.noise = nullptr;
  ep.seed = seed;
  ep.leaf = 0;
  ep.sigma = 0.0f;
  ep.out_bf16 = out_dtype == DPC_BF16;
  ep.out = nullptr;
  GroupedTables grp;
  grp.a_ptrs = a_ptrs;
  grp.g_ptrs = g_ptrs;
  grp.rows = rows;
  grp.steps = steps;
  grp.step_start = step_start;
  grp.seg_scale = seg_scale;
  grp.out_ptrs = out_ptrs;
  grp.noise_ptrs = noise_mode == DPC_NOISE_INJECTED ? noise_ptrs : nullptr;
  grp.leaf_ids = leaf_ids;
  grp.sigmas = sigmas;
  grp.E = E;
  // Buffer offsets are 32-bit, and a row past a step's end is fetched at an
  // offset >= kOutOfRange: each problem's operands must stay below that.
  const size_t dmax = (size_t)(din > dout ? din : dout);
  const bool fits = (size_t)max_rows * dmax * 2 < (size_t)kOutOfRange;
  const bool fast = dtype == DPC_BF16 && din % 8 == 0 && dout % 8 == 0 && fits;
  if (fast) {
    FastArgs args;
    args.A = nullptr;
    args.G = nullptr;
    args.nprob = 0;
    args.T = 0;
    args.B = 0;
    args.plan = nullptr;
    args.scale = nullptr;
    args.ep = ep;
    args.grp = grp;
    args.splits = 1;
    args.partial = nullptr;
    const long long ntiles = (long long)ceil_div(dout, kBM) * ceil_div(din, kBN) * E;
    if (ntiles > 0x7fffffff) return DPC_ENOTSUP;
    launch_fast<true>(dim3((unsigned)ntiles), s, args);
  } else {
    dim3 grid(ceil_div(din, kGT), ceil_div(dout, kGT), E);
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(grouped_generic_kernel<uint16_t>, grid, dim3(kThreads), 0, s, grp, ep);
    } else {
      hipLaunchKernelGGL(grouped_generic_kernel<float>, grid, dim3(kThreads), 0, s, grp, ep);
    }
  }
  DPC_HIP_CHECK(hipGetLastError());
  return DPC_OK;
}

namespace {
// Workspace layout: the bias split partials (kBiasSplits x dout floats), then,
// 256-byte aligned, the split-K tiles of a dense fast-path launch.
size_t bias_ws_bytes(int dout) {
  return ((size_t)kBiasSplits * (size_t)dout * sizeof(float) + 255) & ~(size_t)255;
}
bool fast_shape(int B, int T, int din, int dout, int dtype) {
  const size_t rows = (size_t)B * (size_t)T;
  const bool small = rows * (size_t)(din > dout ? din : dout) * 2 < ((size_t)1 << 31);
  return dtype == DPC_BF16 && T % kBK == 0 && din % 8 == 0 && dout % 8 == 0 && B > 0 && small;
}
}  // namespace

extern "C" size_t dpc_clipped_sum_workspace_bytes(int B, int T, int din, int dout, int dtype) {
  if (dout <= 0 || din <= 0 || T <= 0 || B < 0) return 0;
  size_t bytes = bias_ws_bytes(dout);
  const int splits = fast_shape(B, T, din, dout, dtype) ? fast_splits(B, T, din, dout)
                                                       : generic_splits(B, T, din, dout);
  if (splits > 1) bytes += (size_t)splits * (size_t)dout * (size_t)din * sizeof(float);
  return bytes;
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
  if (with_bias && (!bias_out || !ws || ws_bytes < bias_ws_bytes(dout)))
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
  const bool fast = fast_shape(B, T, din, dout, dtype) && plan != nullptr;
  if (fast) {
    FastArgs args;
    args.A = (const uint16_t*)A;
    args.G = (const uint16_t*)G;
    args.nprob = 0;
    args.T = T;
    args.B = B;
    args.plan = plan;
    args.scale = scale;
    args.ep = ep;
    // Split-K only with a workspace that holds the slices (else one pass).
    int splits = fast_splits(B, T, din, dout);
    const size_t need = bias_ws_bytes(dout) + (size_t)splits * dout * (size_t)din * sizeof(float);
    if (splits > 1 && (!ws || ws_bytes < need)) splits = 1;
    args.splits = splits;
    args.partial = splits > 1 ? (float*)((uint8_t*)ws + bias_ws_bytes(dout)) : nullptr;
    const int ntiles = ceil_div(dout, kBM) * ceil_div(din, kBN);
    launch_fast<false>(dim3(ntiles * splits), s, args);
    if (splits > 1) {
      DPC_HIP_CHECK(hipGetLastError());
      const long long quads = (long long)(dout / 2) * (din / 2);
      hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((quads + kThreads - 1) / kThreads)),
                         dim3(kThreads), 0, s, (const float*)args.partial, splits, ep);
    }
  } else {
    int splits = generic_splits(B, T, din, dout);
    const size_t need = bias_ws_bytes(dout) + (size_t)splits * dout * (size_t)din * sizeof(float);
    if (splits > 1 && (!ws || ws_bytes < need)) splits = 1;
    const long long K = (long long)B * T;
    const long long per = ((K + splits - 1) / splits + kGK - 1) / kGK * kGK;
    float* partial = splits > 1 ? (float*)((uint8_t*)ws + bias_ws_bytes(dout)) : nullptr;
    dim3 grid(ceil_div(din, kGT), ceil_div(dout, kGT), splits);
    if (dtype == DPC_BF16) {
      hipLaunchKernelGGL(clipped_sum_generic_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                         (const uint16_t*)A, (const uint16_t*)G, scale, B, T, ep, splits, per,
                         partial);
    } else {
      hipLaunchKernelGGL(clipped_sum_generic_kernel<float>, grid, dim3(kThreads), 0, s,
                         (const float*)A, (const float*)G, scale, B, T, ep, splits, per, partial);
    }
    if (splits > 1) {
      DPC_HIP_CHECK(hipGetLastError());
      const long long pairs = (long long)(dout / 2) * (din / 2);
      hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((pairs + kThreads - 1) / kThreads)),
                         dim3(kThreads), 0, s, (const float*)partial, splits, ep);
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

extern "C" int dpc_clipped_sum_multi(int n, const void* const* A, const void* const* G,
                                     const int* din, const int* dout, const float* scale,
                                     const void* plan, int B, int T, int dtype,
                                     double normalize_by, int noise_mode,
                                     const float* const* noise, uint64_t seed,
                                     const uint32_t* leaf_ids, const double* sigmas,
                                     int out_dtype, void* const* out, void* stream) {
  if (n < 0 || B < 0 || T <= 0) return DPC_EINVAL;
  if (n == 0) return DPC_OK;
  if (!A || !G || !din || !dout || !out || !sigmas) return DPC_EINVAL;
  if (dtype != DPC_F32 && dtype != DPC_BF16) return DPC_EINVAL;
  if (out_dtype != DPC_F32 && out_dtype != DPC_BF16) return DPC_EINVAL;
  if (!(normalize_by > 0.0)) return DPC_EINVAL;
  if (noise_mode < DPC_NOISE_NONE || noise_mode > DPC_NOISE_PHILOX) return DPC_EINVAL;
  if (B > 65535) return DPC_ENOTSUP;
  bool fast = plan != nullptr && B > 0;
  for (int i = 0; i < n; ++i) {
    if (din[i] <= 0 || dout[i] <= 0 || !out[i]) return DPC_EINVAL;
    if (B > 0 && (!A[i] || !G[i] || !scale)) return DPC_EINVAL;
    if (!(sigmas[i] >= 0.0)) return DPC_EINVAL;
    if (sigmas[i] != 0.0 && noise_mode == DPC_NOISE_NONE) return DPC_EINVAL;
    if (sigmas[i] != 0.0 && noise_mode == DPC_NOISE_INJECTED && (!noise || !noise[i]))
      return DPC_EINVAL;
    fast = fast && fast_shape(B, T, din[i], dout[i], dtype);
  }
  hipStream_t s = (hipStream_t)stream;
  if (!fast) {
    // Layer by layer, each exactly as its own call without a workspace.
    for (int i = 0; i < n; ++i) {
      const int r = dpc_clipped_sum(A[i], G[i], scale, plan, B, T, din[i], dout[i], dtype,
                                    normalize_by, noise_mode, noise ? noise[i] : nullptr, nullptr,
                                    seed, leaf_ids ? leaf_ids[i] : 0u, 0u, sigmas[i], out_dtype,
                                    out[i], 0, nullptr, nullptr, 0, stream);
      if (r != DPC_OK) return r;
    }
    return DPC_OK;
  }
  for (int i0 = 0; i0 < n; i0 += kMaxDense) {
    const int m = n - i0 < kMaxDense ? n - i0 : kMaxDense;
    FastArgs args;
    args.A = nullptr;
    args.G = nullptr;
    args.T = T;
    args.B = B;
    args.plan = plan;
    args.scale = scale;
    args.splits = 1;
    args.partial = nullptr;
    args.nprob = m;
    Epilogue& ep = args.ep;
    ep.M = 0;
    ep.N = 0;
    ep.nb = (float)normalize_by;
    ep.apply_nb = normalize_by != 1.0;
    ep.noise_mode = noise_mode;
    ep.noise = nullptr;
    ep.seed = seed;
    ep.leaf = 0;
    ep.sigma = 0.0f;
    ep.out_bf16 = out_dtype == DPC_BF16;
    ep.out = nullptr;
    long long tiles = 0;
    for (int k = 0; k < m; ++k) {
      const int i = i0 + k;
      DenseProblem& P = args.dp[k];
      P.A = (const uint16_t*)A[i];
      P.G = (const uint16_t*)G[i];
      P.out = out[i];
      P.noise = sigmas[i] != 0.0 && noise_mode == DPC_NOISE_INJECTED ? noise[i] : nullptr;
      P.M = dout[i];
      P.N = din[i];
      P.tile_start = (int)tiles;
      P.leaf = leaf_ids ? leaf_ids[i] : 0u;
      P.sigma = noise_mode == DPC_NOISE_NONE ? 0.0f : (float)sigmas[i];
      P.pad = 0;
      tiles += (long long)ceil_div(dout[i], kBM) * ceil_div(din[i], kBN);
    }
    if (tiles > 0x7fffffffLL) return DPC_ENOTSUP;
    launch_fast<false>(dim3((unsigned)tiles), s, args);
    DPC_HIP_CHECK(hipGetLastError());
  }
  return DPC_OK;
}
