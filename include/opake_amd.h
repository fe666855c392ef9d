/*
 * opake_amd — C ABI of the MI355X (gfx950) DP-SGD clip -> sum -> noise step.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers owned by the caller (inputs are
 *     borrowed and never written, outputs are written in full);
 *   - work is enqueued asynchronously on `stream` (a hipStream_t passed as
 *     void*; NULL is the default stream); nothing blocks the host;
 *   - the library allocates no device memory: scratch comes in through the
 *     `ws` / `ws_bytes` pair, sized with the matching *_workspace_bytes query;
 *   - the return value is DPC_OK or a negative status:
 *       DPC_EINVAL  bad shape, dtype, pointer or argument,
 *       DPC_ENOTSUP a valid call this build does not implement,
 *       DPC_ENOSPC  workspace too small,
 *       DPC_EHIP    the HIP runtime reported an error at launch.
 *   - tensors are dense row-major; `dtype` values are enum dpc_dtype.
 *
 * Reference interfaces named below are files of JetBrains-Research/opake.
 */
#ifndef OPAKE_AMD_H
#define OPAKE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DPC_OK 0
#define DPC_EINVAL (-22)
#define DPC_ENOTSUP (-95)
#define DPC_ENOSPC (-28)
#define DPC_EHIP (-1000)

/* Element types.  Most entry points take DPC_F32 / DPC_BF16 operands; the
 * materialised-leaf passes, the clip-factor guards and dpc_add_noise_ex also
 * take DPC_F16 and DPC_F64. */
enum dpc_dtype { DPC_F32 = 0, DPC_BF16 = 1, DPC_F16 = 2, DPC_F64 = 3 };
enum dpc_scale_kind { DPC_SCALE_FIXED = 0, DPC_SCALE_AUTO_S = 1 };
enum dpc_noise_mode { DPC_NOISE_NONE = 0, DPC_NOISE_INJECTED = 1, DPC_NOISE_PHILOX = 2 };

/* Library ABI version (major * 100 + minor). */
int dpc_version(void);

/* Last HIP error string recorded by a failing call on this thread. */
const char* dpc_last_error(void);

/* Timing events recorded without the system-scope fence (HIP's
 * hipEventDisableSystemFence): the timing hooks of the clipping entry points
 * and of bench.py use them to time launches without adding cache writeback
 * and invalidation around them (no reference counterpart: measurement
 * plumbing of this build).  create -> record on a stream (any number of
 * times) -> elapsed_ms between two recorded events once both completed ->
 * destroy. */
int dpc_timing_event_create(void** event);
int dpc_timing_event_record(void* event, void* stream);
int dpc_timing_event_elapsed_ms(void* start, void* end, float* ms);
int dpc_timing_event_destroy(void* event);

/* Writes n 32-bit words from HOST memory `host_words` to device memory `dst`
 * with kernels that carry the words as arguments: no host buffer has to
 * outlive the call, so it may be recorded into a HIP graph.  Used for the
 * small index and pointer tables the other entry points take (no reference
 * counterpart: plumbing of this build). */
int dpc_write_words(void* dst, const uint32_t* host_words, int n, void* stream);

/* ------------------------------------------------------------------------
 * Per-example squared gradient norms of linear layers (ghost / Gram norm).
 *
 * Replaces the norm pass over materialised per-example weight gradients:
 * `vmap(grad)` in packages/opake-engine/src/opake/api/engine/clipping/
 * _clipped_grad.py:278-296 followed by the per-leaf sum of squares of
 * _streaming.py:70-82 (`_leaf_sq_sum`, _pytree.py:286-314).  For a layer
 * with inputs A_i [T, din] and output gradients G_i [T, dout] the
 * per-example weight gradient is G_i^T A_i, and
 *     ||G_i^T A_i||_F^2 = <A_i A_i^T, G_i G_i^T>.
 *
 * dpc_gram_sqnorms: A [B, T, din], G [B, T, dout] in `dtype`.  Adds (or, if
 * accumulate == 0, writes) ||G_i^T A_i||^2 to sqnorm[i] (float64, [B]), and
 * an upper bound of its rounding error to sqerr[i] (float64, [B]; nullable),
 * so that sqnorm[i] + sqerr[i] >= ||G_i^T A_i||^2 exactly for the given
 * values -- the `abs_out` guard term: <A A^T, G G^T> cancels, so its error
 * scales with the magnitudes of the Gram entries, not with the result.  The
 * bound covers the Gram matrices' accumulation chains (fp32 MFMA: any
 * rounding or truncation of at most one fp32 ulp per addend of an MFMA
 * instruction, and flushed subnormals; generic path: fp64) and the fp64
 * inner product.  A layer bias adds ||sum_t G_i[t]||^2 (and its bound) when
 * with_bias != 0.  Examples whose A_i or G_i hold NaN/Inf produce a
 * non-finite value (their clip factor becomes 0).
 * -------------------------------------------------------------------------*/
size_t dpc_gram_workspace_bytes(int B, int T);
int dpc_gram_sqnorms(const void* A, const void* G, int B, int T, int din, int dout, int dtype,
                     int with_bias, int accumulate, double* sqnorm, double* sqerr, void* ws,
                     size_t ws_bytes, void* stream);

/* dpc_gram_sqnorms over several bias-free layers of one example batch (the
 * per-layer norm loop of _streaming.py:70-82 over the layers of a model):
 * layer i adds exactly what dpc_gram_sqnorms(A[i], G[i], B, T, din[i],
 * dout[i], dtype, 0, i == 0 ? accumulate : 1, ...) would, in layer order.
 * With bf16 operands, T an even number of 128-row blocks, B a multiple of 8
 * and up to 8 layers, all layers share one launch (the work items of every
 * layer spread over all XCDs); otherwise the layers run one by one.  ws:
 * dpc_gram_sqnorms_multi_workspace_bytes. */
size_t dpc_gram_sqnorms_multi_workspace_bytes(int n, const int* din, const int* dout, int B,
                                              int T, int dtype);
int dpc_gram_sqnorms_multi(int n, const void* const* A, const void* const* G, const int* din,
                           const int* dout, int B, int T, int dtype, int accumulate,
                           double* sqnorm, double* sqerr, void* ws, size_t ws_bytes,
                           void* stream);

/* dpc_gram_sqnorms_noalloc: no counterpart in the reference.  The same
 * computation as dpc_gram_sqnorms with no workspace argument and no
 * allocation, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * workspace is a static device array of DPC_NOALLOC_SCRATCH_BYTES per device,
 * held until the process ends.  Calls needing more
 * (dpc_gram_workspace_bytes(B, T) > DPC_NOALLOC_SCRATCH_BYTES) return
 * DPC_ENOSPC.  Every call on a device shares that device's array, so calls
 * that overlap on one device (other streams, other threads) race. */
#define DPC_NOALLOC_SCRATCH_BYTES (48u << 20)
int dpc_gram_sqnorms_noalloc(const void* A, const void* G, int B, int T, int din, int dout,
                             int dtype, int with_bias, int accumulate, double* sqnorm,
                             double* sqerr, void* stream);

/* Flat inputs (T == 1): a [B, din], g [B, dout];
 * sqnorm[i] (+)= ||a_i||^2 ||g_i||^2 (+ ||g_i||^2 with a bias), sqerr[i] (+)=
 * its error bound (nullable). */
int dpc_flat_sqnorms(const void* a, const void* g, int B, int din, int dout, int dtype,
                     int with_bias, int accumulate, double* sqnorm, double* sqerr, void* stream);

/* ------------------------------------------------------------------------
 * Clip factors from squared norms.
 *
 * Replaces the ratio and scale computation of _streaming.py:84-108 and
 * _pytree.py:111-157 (`_guard_scale` / `_finalize_scale`), evaluated in
 * float64, from an upper bound of the norm when sqerr (nullable, the bound of
 * dpc_gram_sqnorms) is given:
 *   norm   = sqrt(max(sqnorm[i], 0))               (the estimate, reported)
 *   up     = sqrt(max(sqnorm[i] + sqerr[i], 0))    (sqerr NULL: up = norm)
 *   ratio  = max(C, 0) / up                        (kind FIXED)
 *          = max(C, 0) / (up + gamma)              (kind AUTO_S)
 *   s      = ratio * guard_rel[g] - guard_abs[g]
 *   s      = min(1, s)                             (FIXED only)
 *   s      = isfinite(s) ? max(s, 0) : 0
 *   scale[g * B + i] = s.to(guard_mult[g]) as float, for each guard g
 *                    (the reference's scale.to(multiply dtype),
 *                    _pytree.py:160-187: DPC_F32 / DPC_F64 (float)s,
 *                    DPC_BF16 / DPC_F16 (float)s rounded to nearest even
 *                    in that type, as torch converts a float64 through
 *                    float32)
 *   scale64[g * B + i] = s for DPC_F64 guards, (double)scale[g * B + i]
 *                    otherwise (nullable; the float64 multiply of float64
 *                    leaves)
 * norms_out[i] = (float)norm; *nclipped = #{i : (float)norm > count_threshold}
 * (the reference's strict `norms > clipping_norm`, _clipped_fun.py:348-396);
 * *nonfinite (nullable; written with system scope, so it may point to pinned
 * host memory that the host reads once the call has completed) = #{i :
 * sqnorm[i] or sqerr[i] not finite} -- the examples whose operands held
 * NaN / Inf, which the ghost paths then clip from their sanitised
 * per-example gradients (_streaming.py:73,151).
 * guard_rel / guard_abs / guard_mult (nullable: all DPC_F32) are HOST arrays of
 * n_guards (1..4) values, one per storage dtype.  sqnorm and all outputs are device pointers.
 * Any output pointer may be NULL.  `plan` (nullable, device memory of
 * n_guards * dpc_clip_plan_bytes(B) bytes) receives one plan per guard: the
 * examples whose guard-g scale is positive, those the bf16 GEMM may apply to
 * its accumulators first (2^-64 <= scale <= 2^32 and B * C <= 2^55), then the
 * others, each list in increasing order; the clipped-sum GEMM walks only
 * these.
 * -------------------------------------------------------------------------*/
size_t dpc_clip_plan_bytes(int B);
int dpc_clip_factors(const double* sqnorm, const double* sqerr, int B, double C, int kind,
                     double gamma, const double* guard_rel, const double* guard_abs,
                     const int* guard_mult, int n_guards, float count_threshold, float* scale,
                     double* scale64, float* norms_out, int* nclipped, void* plan,
                     int* nonfinite, void* stream);

/* dpc_clip_factors_groups: dpc_clip_factors for n_groups clipping groups in
 * one launch -- the per-group clip of _streaming.py:84-108 with each group's
 * own bound (_pytree.py:345-352) -- bit for bit n_groups calls of
 * dpc_clip_factors, group g with C[g] and count_threshold[g] (HOST arrays of
 * n_groups values), sqnorm + g * B and sqerr + g * B, and its outputs at
 * scale / scale64 + g * n_guards * B, norms_out + g * B, nclipped + g,
 * plan + g * n_guards * dpc_clip_plan_bytes(B) bytes and nonfinite + g. */
int dpc_clip_factors_groups(const double* sqnorm, const double* sqerr, int n_groups, int B,
                            const double* C, int kind, double gamma, const double* guard_rel,
                            const double* guard_abs, const int* guard_mult, int n_guards,
                            const float* count_threshold, float* scale, double* scale64,
                            float* norms_out, int* nclipped, void* plan, int* nonfinite,
                            void* stream);

/* dpc_gram_clip_factors: the norm pass and the clip factors of one linear
 * layer -- _streaming.py:70-108 for a layer whose per-example gradients are
 * never formed -- exactly
 *   dpc_gram_sqnorms(A, G, B, T, din, dout, dtype, with_bias, 0, sqnorm,
 *                    sqerr, ...) then
 *   dpc_clip_factors(sqnorm, sqerr, B, C, kind, gamma, guard_rel, guard_abs,
 *                    guard_mult, n_guards, count_threshold, scale, scale64,
 *                    norms_out, nclipped, plan, stream)
 * (the same bits), in ONE launch when the split Gram kernel applies (bf16,
 * T an even number of 128-row blocks, din and dout multiples of 8, no bias,
 * B <= 2048): its last work item folds the records and computes the clip
 * factors.  ws: dpc_gram_clip_workspace_bytes(B, T) bytes of scratch (any
 * content).  counters: dpc_gram_clip_counter_bytes(B, T) bytes that must be
 * zero before the first call on them; every call leaves them zero again, so
 * one zero-filled buffer (as large as the largest call needs) serves call
 * after call of any shape on one stream -- calls that overlap on one
 * counter buffer race; the separate-launch shapes do not touch it.  sqnorm
 * is required. */
size_t dpc_gram_clip_workspace_bytes(int B, int T);
size_t dpc_gram_clip_counter_bytes(int B, int T);
int dpc_gram_clip_factors(const void* A, const void* G, int B, int T, int din, int dout,
                          int dtype, int with_bias, double C, int kind, double gamma,
                          const double* guard_rel, const double* guard_abs, const int* guard_mult,
                          int n_guards, float count_threshold, double* sqnorm, double* sqerr,
                          float* scale, double* scale64, float* norms_out, int* nclipped,
                          void* plan, int* nonfinite, void* ws, size_t ws_bytes,
                          int32_t* counters, size_t counter_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Clipped batch sum of a linear layer with the noise epilogue fused.
 *
 * Replaces the apply pass of _streaming.py:137-167 (scale, store, batch sum
 * via `reduce_leaf`), the `x / normalize_by` of _clipped_fun.py:880-883 and
 * the per-leaf Gaussian draw + add of packages/opake-dpsgd/src/opake/api/
 * dpsgd/noise/_gaussian.py:188-229:
 *   acc[m, n] = sum_i scale[i] * sum_t G[i, t, m] * A[i, t, n]   (fp32)
 *   v = to_out(acc); if normalize_by != 1: v = to_out(float(v) / normalize_by)
 *   if sigma != 0: v = to_out(float(v) + (float)sigma * z[m, n])
 *   out[m, n] = v             (out is [dout, din], dtype out_dtype)
 * z comes from `noise` (float32 [dout, din], mode INJECTED; bit-exact with a
 * host-drawn tensor) or from the Philox stream (mode PHILOX) keyed by
 * (seed, leaf_id).  `plan` is the dpc_clip_factors plan built from the same
 * `scale` (nullable: the generic kernel then scans every example).  On the
 * bf16 MFMA path (T % 64 == 0, din and dout multiples of 8) the products of
 * the given bf16 values are summed in fp32 and each example's scale is
 * applied to the fp32 accumulators (the plan's first list); examples of the
 * plan's second list have G multiplied by the power of two of their scale
 * (exact) and the mantissa applied to the accumulators.  With
 * with_bias, bias_out[m] = same recipe over
 * sum_i scale[i] * sum_t G[i, t, m], its noise keyed by (seed, bias_leaf_id)
 * under the [dout, 1] view.  ws (dpc_clipped_sum_workspace_bytes) holds the
 * bias partials and, on the MFMA path for layers of fewer than 192 256 x 256
 * output tiles, the fp32 K-slices of a split-K launch (summed in a fixed
 * order); with a smaller ws (or none, without bias) the launch is one pass.
 * -------------------------------------------------------------------------*/
size_t dpc_clipped_sum_workspace_bytes(int B, int T, int din, int dout, int dtype);
int dpc_clipped_sum(const void* A, const void* G, const float* scale, const void* plan, int B,
                    int T, int din, int dout, int dtype, double normalize_by, int noise_mode,
                    const float* noise, const float* bias_noise, uint64_t seed, uint32_t leaf_id,
                    uint32_t bias_leaf_id, double sigma, int out_dtype, void* out, int with_bias,
                    void* bias_out, void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------------
 * dpc_clipped_sum over several bias-free linear layers of one clipping group
 * (the same examples, scale and plan): the reference's apply pass visits the
 * leaves one by one (_streaming.py:137-167, with the per-leaf noise of
 * _gaussian.py:188-229); here layer i gets exactly
 *   dpc_clipped_sum(A[i], G[i], scale, plan, B, T, din[i], dout[i], dtype,
 *                   normalize_by, noise_mode, noise ? noise[i] : NULL, NULL,
 *                   seed, leaf_ids ? leaf_ids[i] : 0, 0, sigmas[i], out_dtype,
 *                   out[i], 0, NULL, NULL, 0, stream)
 * (one pass, no split-K), and when every layer takes the bf16 MFMA path the
 * layers share launches (up to 8 layers each): the output tiles of all of
 * them fill the chip together instead of one layer at a time.
 * -------------------------------------------------------------------------*/
int dpc_clipped_sum_multi(int n, const void* const* A, const void* const* G, const int* din,
                          const int* dout, const float* scale, const void* plan, int B, int T,
                          int dtype, double normalize_by, int noise_mode,
                          const float* const* noise, uint64_t seed, const uint32_t* leaf_ids,
                          const double* sigmas, int out_dtype, void* const* out, void* stream);

/* ------------------------------------------------------------------------
 * Gaussian noise on an arbitrary leaf (out-of-place).
 *
 * Replaces `_sample` of _gaussian.py:188-204:
 *   y = to_dtype(float(x) + (float)sigma * z),   z as in dpc_clipped_sum.
 * The leaf is viewed as [rows, cols] for the Philox stream (rows = size of
 * dim 0, cols = numel / rows).  sigma == 0 copies x.
 * -------------------------------------------------------------------------*/
int dpc_add_noise(const void* x, void* y, int64_t rows, int64_t cols, int dtype, double sigma,
                  int noise_mode, const float* noise, uint64_t seed, uint32_t leaf_id,
                  void* stream);

/* dpc_add_noise_ex: `_sample` of _gaussian.py:188-204 for any leaf dtype
 * and any compute_dtype cd (each of DPC_F16 / DPC_BF16 / DPC_F32 / DPC_F64):
 *   y = to_dtype(to_cd(to_cd(x) + to_cd(sigma_op * z)))
 * with sigma_op = (float)sigma for cd of 16 or 32 bits (torch's Python-scalar
 * multiply of such a tensor) and sigma itself for DPC_F64, and to_cd of a
 * 16-bit cd through float32 (torch's float arithmetic for 16-bit tensors).
 * z: injected (`noise`, cd values shaped like x: the reference's
 * torch.randn(shape, dtype=compute_dtype) on its CPU generator) or the
 * Philox stream of dpc_add_noise rounded to cd.  sigma == 0 copies x. */
int dpc_add_noise_ex(const void* x, void* y, int64_t rows, int64_t cols, int dtype,
                     int compute_dtype, double sigma, int noise_mode, const void* noise,
                     uint64_t seed, uint32_t leaf_id, void* stream);

/* The Philox-stream noise of n leaves of one dtype in as few launches as
 * possible (one per 32 leaves), for the many small leaves of a step (LoRA
 * adapters): leaf i gets exactly dpc_add_noise(x[i], y[i], rows[i], cols[i],
 * dtype, sigma[i], DPC_NOISE_PHILOX, NULL, seed, leaf_ids[i]).  The arrays
 * are host memory; y[i] may equal x[i] (in place).  Same reference
 * interface as dpc_add_noise (_gaussian.py:188-204, one call per leaf of
 * the pytree). */
int dpc_add_noise_leaves(int n, const void* const* x, void* const* y, const int64_t* rows,
                         const int64_t* cols, const double* sigma, const uint32_t* leaf_ids,
                         int dtype, uint64_t seed, void* stream);

/* Known-answer hook: n Philox4x32-10 blocks for counters (c0 + j, c1, c2, c3),
 * key (k0, k1), written as out[4 j + w]. */
int dpc_philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                      uint32_t k1, int n, uint32_t* out, void* stream);

/* ------------------------------------------------------------------------
 * Materialised-leaf clip-and-sum (multi-tensor apply).
 *
 * The HIP counterpart of the fused backend seam
 * (_kernel_backend.py:9-17, registered like patches/__init__.py:106-117;
 * kernels of packages/opake-patches/src/opake/api/patches/kernels/
 * _clip_sum.py:74-152).  Leaves are stacked per-example values
 * [B, n_l] of one storage dtype; `ptrs` (device int64 [L]) holds their
 * addresses, `sizes` (device int64 [L]) their per-example element counts.
 * The tile table (tile_leaf / tile_local, device int32 [n_tiles]) splits each
 * leaf into 2048-element tiles.
 *
 * dpc_leaves_sqnorm: partial[b, t] = float64 sum over tile t of example b of
 *   to_sq(v * v), v = to_sq(sanitise(x)), sq = square_dtype (the reference's
 *   reduction dtype, _pytree.py:84-108,286-314: float32 by default, float64
 *   for float64 leaves, or an explicit compute_dtype; any of the four
 *   dtypes, leaves of any of them), then leaf_sq[b, leaf_col[l]] = sum of
 *   leaf l's tiles (tile_start [L + 1]).
 * dpc_leaves_apply: out[off_l + j] = sum_b stored(b, l, j) in fp32, where
 *   stored = to_dtype(float(sanitise(x)) * scale[row_l * B + b]) with bf16
 *   subnormals that rounded up zeroed (_pytree.py:160-204); row_l =
 *   leaf_scale_row[l] (device int32 [L]; NULL: every leaf uses row 0 -- the
 *   per-group clipping of _streaming.py:63-104 gives each group its row);
 *   out_sq (nullable, same layout and dtype as out) = sum_b to_dtype(stored^2),
 *   the second moment of _streaming.py:167-172; post_sq (nullable, float32
 *   [B, 4 * n_tiles]): post_sq[b, 4 t + q] = sum of stored^2 over quarter q
 *   (elements 512 q .. 512 q + 511) of tile t, so a row sums to ||stored_b||^2.
 *   out_dtype is the storage dtype or float32.
 * -------------------------------------------------------------------------*/
int dpc_leaves_sqnorm(const int64_t* ptrs, const int64_t* sizes, const int32_t* tile_leaf,
                      const int32_t* tile_local, const int64_t* tile_start,
                      const int32_t* leaf_col, int n_leaves, int n_tiles, int B, int dtype,
                      int square_dtype, double* partial, double* leaf_sq, int leaf_sq_stride,
                      void* stream);
int dpc_leaves_apply(const int64_t* ptrs, const int64_t* sizes, const int32_t* tile_leaf,
                     const int32_t* tile_local, const int64_t* out_offs, int n_tiles, int B,
                     int dtype, const float* scale, const int32_t* leaf_scale_row, void* out,
                     void* out_sq, int out_dtype, float* post_sq, void* stream);
/* dpc_leaves_apply_ex: the apply pass for every dtype combination of
 * _pytree.py:160-204 with _clipped_fun.py:112-132 -- storage dtype S
 * (`dtype`), multiply dtype M = promote(S, compute dtype) (`mult_dtype`),
 * batch-sum dtype A (`acc_dtype`: the compute dtype, float32 for 16-bit
 * storage, else S) and output dtype O (`out_dtype`), each any of the four:
 *   prod = to_M(sanitise(x) * scale_M[b]), stored = to_S(prod) (zeroed if it
 *   rounded up into S's subnormal range), out = to_O(to_A(sum_b to_A(stored)))
 *   with the sum in float32 (A of 16 or 32 bits) or float64 (A = float64), in
 *   example order.  scale_M is row leaf_scale_row[l] of `scale` (float32,
 *   already converted to M) or, for M = float64, of `scale64` (float64).
 *   out_sq (nullable): the same sum of to_S(stored^2); post_sq (nullable,
 *   float64 [B, 4 * n_tiles]) as in dpc_leaves_apply. */
int dpc_leaves_apply_ex(const int64_t* ptrs, const int64_t* sizes, const int32_t* tile_leaf,
                        const int32_t* tile_local, const int64_t* out_offs, int n_tiles, int B,
                        int dtype, int mult_dtype, int acc_dtype, const float* scale,
                        const double* scale64, const int32_t* leaf_scale_row, void* out,
                        void* out_sq, int out_dtype, double* post_sq, void* stream);

/* dpc_sanitize_columns: out[e, :, k] = x[e, :, k] when column k of matrix e
 * (n matrices [T, d], any of the four dtypes) holds only finite values, else
 * zeros.  With A and G sanitised this way, G'^T A' is exactly the
 * reference's sanitised per-example gradient of a linear layer
 * (nan_to_num of G^T A, _streaming.py:73,151): a non-finite A[t, k] makes
 * column k of G^T A non-finite, a non-finite G[t, m] row m.  The ghost
 * paths clip the examples whose Gram norm is not finite from these. */
int dpc_sanitize_columns(const void* x, void* out, int n, int T, int d, int dtype, void* stream);

/* Per-group sums of per-leaf squared norms: s = the sum of
 * x[b * stride + j * col_stride] over the columns j with col_group[j] == g,
 * in column order (from 0.0), and out[g * B + b] (float64) = s, or
 * out[g * B + b] + s with `accumulate` -- the per-group accumulation in leaf
 * order of packages/opake-engine/src/opake/api/engine/clipping/
 * _streaming.py:71-80 (_accumulate_group_value, _pytree.py:345-352).  x is
 * [B, n] row-major (col_stride 1, stride >= n) or column-major (stride 1,
 * col_stride >= B); other layouts are DPC_EINVAL. */
int dpc_group_sum_f64(const double* x, int B, int n, int stride, int col_stride,
                      const int32_t* col_group, int n_groups, double* out, int accumulate,
                      void* stream);

/* ------------------------------------------------------------------------
 * Grouped (segmented) linear layers: E problems of one shape, e.g. the same
 * projection of E mixture-of-experts experts.  Problem e has operands A_e
 * [rows_e, din] and G_e [rows_e, dout] (addresses in the device int64 tables
 * a_ptrs / g_ptrs) whose rows are cut into segments, each segment the rows
 * of one example -- the reference's "virtual experts" b * E + e of
 * packages/opake-patches/src/opake/api/patches/kernels/fused_moe.py:20-27,
 * whose per-sample weight gradient out[g] = A_g^T B_g over the segment's rows
 * (_grouped_AtB, fused_moe.py:54-113) is never formed here.
 *
 * dpc_grouped_gram_sqnorms: seg_sq[v] = ||G_v^T A_v||^2 for every segment v
 *   (float64, written), the per-sample norms of the virtual experts that
 *   _streaming.py:70-82 would take of the materialised gradients, and
 *   seg_err[v] (nullable) its error bound as in dpc_gram_sqnorms.  Problems
 *   may differ in shape: `dims` is a HOST int32 array [n_problems][2] of
 *   (din, dout), n_problems <= 64.  `items` (device int32 [n_items][4])
 *   lists (problem << 16 | pair, first row, rows, slot) for every 128-row
 *   tile pair p <= q (pair = q (q + 1) / 2 + p) of every segment, in any
 *   order; an item whose first field is negative is skipped (padding).  With
 *   n_items a multiple of 8, item l runs on XCD l / (n_items / 8).  slot is
 *   the item's index in segment-major order, and seg_item_start (device int32
 *   [S + 1]) gives each segment's slot range.  max_rows bounds every
 *   segment's rows.
 *   set_items (device int32 [n_set_items][4], nullable when n_set_items is 0;
 *   bf16 operands with din and dout multiples of 8 only) lists segments of 1
 *   to 320 rows computed by the grouped split kernel instead: two items per
 *   segment, (problem | op << 8 | set << 9, first row, rows, first slot), op
 *   0 for A and 1 for G, set in 0 .. n_sets - 1 naming the segment's pair of
 *   items, first slot = seg_item_start of the segment (the kernel writes all
 *   of its tile-pair records); the two items of a set must lie in the same
 *   eighth of the table (one XCD), -1 items are padding.  `items` then lists
 *   only the other segments' tile pairs.
 *   n_records = seg_item_start[S] (one 12-float64 record per tile pair of
 *   every segment); ws: dpc_grouped_gram_workspace_bytes(n_records, n_sets)
 *   bytes.
 * dpc_segment_plan: the step table of dpc_grouped_clipped_sum.  Segment v
 *   (rows seg_row0[v] .. + seg_len[v] of problem seg_group[v]; segments sorted
 *   by problem) contributes ceil(seg_len / 64) steps (row0, v << 7 | rows)
 *   when seg_scale[v] > 0; step_start[e] (device int32 [E + 1]) is problem
 *   e's first step.  max_steps bounds the table (int32 [2 * max_steps]).
 * dpc_grouped_clipped_sum: for each problem e, the dpc_clipped_sum recipe
 *   over its segments, segment v scaled by seg_scale[v]:
 *     acc[m, n] = sum_v seg_scale[v] * sum_{t in v} G_e[t, m] * A_e[t, n]
 *   written to out_ptrs[e] ([dout, din], out_dtype) with / normalize_by and
 *   noise sigmas[e] * z (z from noise_ptrs[e] or Philox (seed, leaf_ids[e])).
 *   On the bf16 MFMA path G is multiplied by the power of two of its
 *   segment's scale (exact) and the mantissa is applied to the fp32
 *   accumulators.
 *   rows (device int32 [E]) bounds each problem's operand rows; max_rows
 *   bounds rows.  Segments with scale 0 are never read.
 * -------------------------------------------------------------------------*/
size_t dpc_grouped_gram_workspace_bytes(int n_records, int n_sets);
int dpc_grouped_gram_sqnorms(const int64_t* a_ptrs, const int64_t* g_ptrs, const int32_t* dims,
                             int n_problems, int dtype, const int32_t* items, int n_items,
                             int max_rows, const int32_t* set_items, int n_set_items, int n_sets,
                             int n_records, const int32_t* seg_item_start, int S, double* seg_sq,
                             double* seg_err, void* ws, size_t ws_bytes, void* stream);
int dpc_segment_plan(const int32_t* seg_row0, const int32_t* seg_len, const int32_t* seg_group,
                     const float* seg_scale, int S, int E, int max_steps, int32_t* steps,
                     int32_t* step_start, void* stream);
int dpc_grouped_clipped_sum(const int64_t* a_ptrs, const int64_t* g_ptrs, const int32_t* rows,
                            int max_rows, int E, int din, int dout, int dtype,
                            const int32_t* steps, const int32_t* step_start,
                            const float* seg_scale, double normalize_by, int noise_mode,
                            const int64_t* noise_ptrs, uint64_t seed, const uint32_t* leaf_ids,
                            const float* sigmas, int out_dtype, const int64_t* out_ptrs,
                            void* stream);

/* ------------------------------------------------------------------------
 * Per-example weight gradients of a narrow linear layer (LoRA adapters).
 *
 * Replaces the per-sample adapter gradients of packages/opake-patches/src/
 * opake/api/patches/kernels/lora.py:687-701 (`_per_sample_lora_adapter_grads`:
 * dA = X^T (G B^T) s, dB = (X A)^T G s per example) and, generally, the
 * vmap(grad) materialisation (_clipped_grad.py:278-296) of a linear layer
 * whose din or dout is at most 32:
 *   out[b, m, n] = sum_t G[b, t, m] * A[b, t, n]   (fp32 sums; out [B, dout, din]
 *   in out_dtype, rounded once).
 * A [B, T, din], G [B, T, dout] in `dtype`.  The gradients are then clipped as
 * materialised leaves (dpc_leaves_sqnorm / dpc_leaves_apply).  Wider layers:
 * DPC_ENOTSUP (use the Gram path).  ws: dpc_per_example_grads_workspace_bytes.
 * -------------------------------------------------------------------------*/
size_t dpc_per_example_grads_workspace_bytes(int B, int T, int din, int dout);
int dpc_per_example_grads(const void* A, const void* G, int B, int T, int din, int dout,
                          int dtype, void* out, int out_dtype, void* ws, size_t ws_bytes,
                          void* stream);

/* The per-example gradients of n such layers that share B and T (the
 * adapters of a block, lora.py:687-701 once per adapter) in as few launches
 * as possible: problem i is dpc_per_example_grads(A[i], G[i], B, T, din[i],
 * dout[i], dtype, out[i], out_dtype, ...), its result the same up to the
 * order of the fp32 token sums (bf16 layers whose wide side is a multiple of
 * 8 and narrow side even share MFMA launches of up to 32 problems; the
 * others run one by one).  The arrays are host memory.  ws:
 * dpc_per_example_grads_grouped_workspace_bytes. */
size_t dpc_per_example_grads_grouped_workspace_bytes(int n, const int* din, const int* dout,
                                                     int B, int T, int dtype);
int dpc_per_example_grads_grouped(int n, const void* const* A, const void* const* G,
                                  void* const* out, const int* din, const int* dout, int B, int T,
                                  int dtype, int out_dtype, void* ws, size_t ws_bytes,
                                  void* stream);

/* Row sums: out[b] (+)= sum_j x[b, j] (float64), used to fold per-leaf
 * squared norms into per-example totals in a fixed order. */
int dpc_row_sum_f64(const double* x, int B, int n, int accumulate, double* out, void* stream);

/* Measurement helper with no counterpart in the reference (used by bench.py
 * to put the roofline in context): `grid` workgroups of 8 waves run `iters`
 * rounds of 8 independent 32x32x16 bf16 MFMAs on operands taken from
 * `operands` (device, grid * 512 * 128 bytes of caller-chosen bf16 bits);
 * out (device float32, grid * 512) keeps the results live.  Timing the
 * launch gives the bf16 MFMA throughput the chip sustains on such data:
 * 2 * 32 * 32 * 16 * 8 * iters FLOP per wave. */
int dpc_calib_mfma_bf16(const void* operands, int grid, int iters, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OPAKE_AMD_H */
