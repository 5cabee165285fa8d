/*
 * hses.h -- C ABI of the MI355X-native EggRoll hot path (libhses.so).
 *
 * Each entry point replaces one function of the reference's Rust surface
 * (hyperscalees-noiser / hyperscalees-kernels / the oxide launch layer);
 * the reference function is cited next to it (paths relative to the
 * reference repository root).  Conventions:
 *   - every call returns an hses_status; on failure hses_last_error() holds a
 *     message (thread-local).  Arguments are validated before any launch, so
 *     a rejected call has no side effect;
 *   - pointers named d_* are device pointers the caller owns; nothing is
 *     allocated per call except where a function says so;
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream); all
 *     work is enqueued on it asynchronously, as the oxide launch layer
 *     enqueues on the cubecl stream (burn_impl/hyperscalees/src/oxide.rs:105-146);
 *   - results do not depend on the launch configuration.
 */
#ifndef HSES_H
#define HSES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    HSES_OK = 0,
    HSES_ERR_INVALID_ARG = 1,
    HSES_ERR_UNSUPPORTED = 2,
    HSES_ERR_HIP = 3,
    HSES_ERR_INTERNAL = 4
} hses_status;

/* Spike/activation storage formats. */
typedef enum {
    HSES_FMT_F32 = 0,  /* 0.0f / 1.0f, the reference's layout                  */
    HSES_FMT_BF16 = 1, /* 0 / 1 as bfloat16                                      */
    HSES_FMT_U8 = 2,   /* 0 / 1 bytes                                            */
    HSES_FMT_BITS = 3  /* bit-packed: a row is ceil(width/64) uint64 words, bit  */
                       /* c%64 of word c/64 is column c; pad bits are zero       */
} hses_fmt;

/* Arithmetic of the perturbed matrix products. */
typedef enum {
    HSES_MATH_F32 = 0,  /* fp32 MFMA, fp32 operands                              */
    HSES_MATH_BF16 = 1, /* bf16 MFMA (operands rounded to bf16), fp32 accumulate */
    HSES_MATH_F32X = 2  /* fp16 MFMA on split operands (each fp32 operand as an  */
                        /* fp16 high + low part, 3 products), fp32 accumulate:  */
                        /* fp32-accurate; the *_pre_x forwards only             */
} hses_math;

/* Solver kinds (burn_impl/hyperscalees-noiser/src/noiser.rs:43-92). */
typedef enum { HSES_SGD = 0, HSES_ADAM = 1, HSES_ADAMW = 2 } hses_solver;

/* Reward kinds of fitness_from_logits_reward (burn_impl/hyperscalees-envs/src/snn_mnist.rs:175-201). */
typedef enum { HSES_REWARD_LOGLIK = 0, HSES_REWARD_BINARY = 1 } hses_reward;

/* Elementwise activations a forward can apply to its output (the op that follows a
 * Linear / Tmm in the models: tanh and sigmoid of TimeMixing's low-rank branches,
 * llm.rs:388-410, relu^2 of ChannelMixing, llm.rs:206). */
typedef enum {
    HSES_ACT_NONE = 0,
    HSES_ACT_TANH = 1,
    HSES_ACT_SIGMOID = 2, /* 1 / (1 + exp(-y)) */
    HSES_ACT_RELU_SQ = 3  /* max(y, 0)^2 */
} hses_act;

/* ---- runtime ---------------------------------------------------------- */

/* Initialise device `device`: builds (once per process) the Box-Muller
 * correction tables and the row-start jump tables of every row length
 * 1..256, and uploads them.  Must be called for a device before any other
 * entry point launches on it (those return HSES_ERR_INVALID_ARG otherwise);
 * it is the only call that allocates device memory, so no launch entry point
 * allocates or copies behind the caller's stream. */
int hses_init(int device);
/* Copies the last error message of this thread into buf (NUL-terminated). */
int hses_last_error(char *buf, size_t len);
const char *hses_version(void);
/* Statistics of the Box-Muller correction tables of the current device:
 * out[0]=#logf exceptions, out[1]=#cosf exceptions. */
int hses_bm_stats(uint32_t out[2]);

/* ---- noise stream ---------------------------------------------------- */

/* noise_seed (burn_impl/hyperscalees-noiser/src/noiser.rs:495-506).  Host only. */
uint64_t hses_noise_seed(uint64_t key, int32_t true_epoch, int32_t true_thread);

/* Exhaustive evaluation of the device Box-Muller halves for unit indices
 * [k_lo, k_lo+n): d_log[i] = logf(max(k*2^-24,1e-9)), d_radius[i] =
 * sqrtf(-2*d_log[i]), d_cos[i] = cosf(TAU*k*2^-24) (noiser.rs:470-477).
 * Any output may be NULL.  Test entry point. */
int hses_bm_eval(uint32_t k_lo, uint32_t n, float *d_log, float *d_radius, float *d_cos,
                 void *stream);

/* batched_lora_noise (burn_impl/hyperscalees-noiser/src/eggroll.rs:116-227):
 * member i has thread id tids[i] (device array) or, if d_tids is NULL,
 * tid_lo + i.  Writes A (n,a,r) = sign*base_sigma*normals rows [b,a+b) and
 * B (n,b,r) = normals rows [0,b) of the member's stream, bit-exact. */
int hses_lora_factors(float base_sigma, uint64_t key, int32_t rank, int32_t epoch,
                      int32_t noise_reuse, int32_t tid_lo, const int32_t *d_tids, int32_t n,
                      int32_t a, int32_t b, float *d_A, float *d_B, void *stream);

/* get_nonlora_update_params (eggroll.rs:312-324) for n members:
 * d_out (n, a, b) = sign*base_sigma*normals, bit-exact. */
int hses_nonlora_noise(float base_sigma, uint64_t key, int32_t epoch, int32_t noise_reuse,
                       int32_t tid_lo, const int32_t *d_tids, int32_t n, int32_t a, int32_t b,
                       float *d_out, void *stream);

/* get_noisy_standard_impl (eggroll.rs:480-503) for the dense (PARAM-class)
 * parameters of n members: d_out (n, a, b) = param + sign*sigma*normals of
 * each member's stream (noiser sigma, not divided by sqrt(rank)), bit-exact.
 * The clean path (iterinfo None) and freeze_nonlora are the caller's copy of
 * param. */
int hses_noisy_standard(const float *d_param, int32_t a, int32_t b, uint64_t key, float sigma,
                        int32_t epoch, int32_t noise_reuse, int32_t tid_lo, const int32_t *d_tids,
                        int32_t n, float *d_out, void *stream);

/* _simple_full_update + _do_update for a dense parameter (eggroll.rs:331-350,
 * 384-404): d_grad (a, b) = scale * sum_m f[m] * sign_m*sigma*normals_m over
 * members m in [0, n) with thread ids tid_lo+m (do_updates: scale =
 * -sqrt(N)/N).  Each member's f32 term is accumulated in double over a fixed
 * split of the pairs and reduced in a fixed order (deterministic, no
 * atomics).  accumulate != 0 adds into d_grad.  a*b <= 524288.  d_work must
 * hold hses_full_update_workspace(a, b, n) bytes. */
size_t hses_full_update_workspace(int32_t a, int32_t b, int32_t n);
int hses_full_update(const float *d_f, int32_t n, int32_t tid_lo, uint64_t key, float sigma,
                     int32_t epoch, int32_t noise_reuse, int32_t a, int32_t b, float scale,
                     int32_t accumulate, float *d_grad, void *d_work, size_t work_bytes,
                     void *stream);

/* ---- spiking kernels ------------------------------------------------- */

/* poisson_encode_fused (burn_impl/hyperscalees-kernels/src/poisson_encode_fused_oxide.rs:61-106,
 * host wrapper burn_impl/hyperscalees/src/oxide.rs:573-625) for any T >= 1:
 * spike[t][row][col] = u_t < p[row][col], u from the per-element xorshift32
 * stream.  p rows are p_stride floats apart; output rows are out_stride
 * elements apart (words for HSES_FMT_BITS); time planes are rows*out_stride
 * apart.  If d_rows is not NULL, output row i encodes input row d_rows[i]
 * (the batch gather train_img.select(0, idx) of accumulate_train.rs:726-735);
 * an index outside [0, p_rows) encodes as an all-zero row.  Without d_rows,
 * p_rows must be >= rows.  The stream index is always the output position
 * i*in_dim + col. */
int hses_poisson_encode(const float *d_p, int64_t p_rows, const int32_t *d_rows, int64_t rows,
                        int32_t in_dim,
                        int64_t p_stride, int32_t T, uint32_t s0, uint32_t s1, uint32_t s2,
                        uint32_t s3, void *d_out, int32_t fmt, int64_t out_stride, void *stream);

/* hses_poisson_encode with the time-plane stride given: spike (t, row) at
 * t*out_plane + row*out_stride.  Besides the time-major layout above
 * (out_plane >= rows*out_stride) it takes the time-inner layout, each row's T
 * entries adjacent (out_plane >= the row's units, out_stride >= T*out_plane):
 * a member's rows then lie contiguous, the layout the fused forward of the
 * next layer reads fastest (hses_perturbed_linear_lif_pre).  The same
 * streams and spikes as hses_poisson_encode (poisson_encode_fused_oxide.rs:35-106);
 * only where they are stored differs. */
int hses_poisson_encode_planes(const float *d_p, int64_t p_rows, const int32_t *d_rows,
                               int64_t rows, int32_t in_dim, int64_t p_stride, int32_t T,
                               uint32_t s0, uint32_t s1, uint32_t s2, uint32_t s3, void *d_out,
                               int32_t fmt, int64_t out_stride, int64_t out_plane, void *stream);

/* Prepared pools: the batch gather + poisson_encode_fused of the training loop
 * (accumulate_train.rs:726-735: train_img.select(0, idx), then
 * poisson_encode_fused_oxide.rs:61-106) for a pool that stays fixed across
 * steps.  hses_poisson_pool_prepare classifies each of the pool's pool_rows
 * rows of in_dim probabilities (row stride p_stride floats) once: the exact
 * threshold K(p) of every element that can fire, compacted per row, into
 * d_pool (pool_bytes >= hses_poisson_pool_bytes(pool_rows, in_dim), 16-byte
 * aligned; 0 for unsupported sizes: in_dim > 2048).
 * hses_poisson_encode_pool then writes, for output row i, the bit-packed
 * spikes of pool row d_rows[i] (or row i with d_rows NULL; an index outside
 * [0, pool_rows) encodes as an all-zero row) at t*out_plane + i*out_stride
 * words: the same streams, seeds and spikes as hses_poisson_encode_planes with
 * HSES_FMT_BITS on the pool's probabilities, for T a power of two <= 32. */
size_t hses_poisson_pool_bytes(int64_t pool_rows, int32_t in_dim);
int hses_poisson_pool_prepare(const float *d_p, int64_t pool_rows, int32_t in_dim,
                              int64_t p_stride, void *d_pool, size_t pool_bytes, void *stream);
int hses_poisson_encode_pool(const void *d_pool, size_t pool_bytes, int64_t pool_rows,
                             int32_t in_dim, const int32_t *d_rows, int64_t rows, int32_t T,
                             uint32_t s0, uint32_t s1, uint32_t s2, uint32_t s3, uint64_t *d_out,
                             int64_t out_stride, int64_t out_plane, void *stream);

/* Mean firing rate over time (snn.rs:274, spikes.mean_dim(0)):
 * d_rate[row][c] = (number of spikes of (row, c) over T) / T, spikes in `fmt`
 * with row stride spk_stride (units) and time planes rows*spk_stride apart. */
int hses_spike_rate(const void *d_spikes, int32_t fmt, int64_t spk_stride, int32_t T,
                    int64_t rows, int32_t h, float *d_rate, void *stream);

/* run_lif (burn_impl/hyperscalees-models/src/snn.rs:53-97) / lif_fused
 * (burn_impl/hyperscalees-kernels/src/lif_fused_oxide.rs:37-70, host oxide.rs:489-543):
 * cur (T, rows, h) fp32 with row stride cur_stride; v0 (rows, h) or NULL (zeros);
 * spikes (T, rows, h) in `fmt` with row stride spk_stride; optional final
 * membrane d_v_out (rows, h) with row stride h. */
int hses_lif_scan(const float *d_cur, const float *d_v0, int32_t T, int64_t rows, int32_t h,
                  int64_t cur_stride, float tau_m, float v_th, void *d_spikes, int32_t fmt,
                  int64_t spk_stride, float *d_v_out, void *stream);

/* ---- perturbed forward ----------------------------------------------- */

/* Batched EggRoll do_mm (eggroll.rs:419-446; batched form snn.rs:665-685):
 * for member m (thread id tid_lo+m) and each of its `rows_per_member` rows,
 *     y = x W^T + (x B_m) A_m^T,   (A_m, B_m) = get_lora_update_params(...)
 * generated in-kernel.  x is (n*rows_per_member, b) in x_fmt (F32, BF16 or
 * BITS) with row stride x_stride (elements, or words for BITS); W (a, b)
 * fp32 row-major; y (n*rows_per_member, a) fp32 with row stride y_stride.
 * Member m's rows are rows [m*rows_per_member, (m+1)*rows_per_member); for
 * time-major activations (T, M, b) pass rows_per_member = slots and
 * n_time = T with plane strides x_plane / y_plane (row s of member m at time
 * t is at t*plane + (m*slots + s)*stride).  Time-major planes (plane >=
 * M*stride) and the time-inner layout (each row's T entries adjacent:
 * plane >= a row, stride >= T*plane) are both accepted, for x, y and spikes.
 * sigma=0 or rank=0 gives the clean x W^T.
 * d_work must hold hses_perturbed_linear_workspace(...) bytes (a bf16 copy of W
 * and, for large ranks, one per-workgroup staging slot for a pair's B factor;
 * the (n, b, r) factor tensor itself is never materialised).  Large ranks
 * (r a multiple of 16, r <= 128, a <= 128) need math = HSES_MATH_BF16.  With
 * math = HSES_MATH_BF16 and small ranks (members per 128-row tile x rank <= 16)
 * the wide-output kernel runs when the workspace holds its bf16 copy of W and x
 * rows are 16-byte aligned; otherwise the small-rank kernel (no workspace). */
size_t hses_perturbed_linear_workspace(int32_t a, int32_t b, int32_t rank, int32_t n,
                                       int32_t rows_per_member, int32_t n_time, int32_t math);
int hses_perturbed_linear(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                          int32_t n_time, const float *d_W, int32_t a, int32_t b,
                          uint64_t key, int32_t rank, float sigma, int32_t epoch,
                          int32_t noise_reuse, int32_t tid_lo, int32_t n, int32_t rows_per_member,
                          float *d_y, int64_t y_stride, int64_t y_plane, int32_t math,
                          void *d_work, size_t work_bytes, void *stream);

/* EggRoll::do_Tmm / do_Tmm_impl (burn_impl/hyperscalees-noiser/src/eggroll.rs:450-477):
 *     y_m = x_m W + sign_m * (sigma/sqrt(rank)) * (x_m A_m) B_m^T
 * for a parameter W of shape (a, b), fp32 row-major: x (n*rows_per_member, a), y (.., b).
 * A_m (a, r) and B_m (b, r) are the same factors as for do_mm on this (a, b) parameter
 * (one stream: B rows, then A rows), regenerated in-kernel.  Arguments, layouts, strides
 * and the workspace rule are those of hses_perturbed_linear with x rows of width a and
 * y rows of width b; large ranks need b <= 128 (the pair kernels' output width). */
size_t hses_perturbed_linear_t_workspace(int32_t a, int32_t b, int32_t rank, int32_t n,
                                         int32_t rows_per_member, int32_t n_time, int32_t math);
int hses_perturbed_linear_t(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                            int32_t n_time, const float *d_W, int32_t a, int32_t b,
                            uint64_t key, int32_t rank, float sigma, int32_t epoch,
                            int32_t noise_reuse, int32_t tid_lo, int32_t n,
                            int32_t rows_per_member, float *d_y, int64_t y_stride, int64_t y_plane,
                            int32_t math, void *d_work, size_t work_bytes, void *stream);

/* hses_perturbed_linear (transposed = 0) or hses_perturbed_linear_t (transposed = 1)
 * followed by the activation `act` (hses_act) on every output: a Linear / Tmm and the
 * elementwise op after it (llm.rs:206, 388-410), fused into the forward's epilogue by the
 * wide-output kernel and applied in place after it otherwise.  y_fmt HSES_FMT_F32, or
 * HSES_FMT_BF16 (rounded to nearest even; for an output only a bf16-math forward reads,
 * which rounds the same way) when the wide-output kernel serves the call
 * (HSES_ERR_UNSUPPORTED otherwise).  Workspace as for the unfused entry point of the same
 * orientation. */
int hses_perturbed_linear_act(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                              int32_t n_time, const float *d_W, int32_t a, int32_t b,
                              uint64_t key, int32_t rank, float sigma, int32_t epoch,
                              int32_t noise_reuse, int32_t tid_lo, int32_t n,
                              int32_t rows_per_member, void *d_y, int64_t y_stride,
                              int64_t y_plane, int32_t math, int32_t transposed, int32_t act,
                              int32_t y_fmt, void *d_work, size_t work_bytes, void *stream);

/* Perturbed forward fused with the LIF layer that consumes it
 * (forward_batched_lora_half_with_lif, snn.rs:544-595: lora_linear_batched
 * then run_lif, snn.rs:53-97; kernel lif_fused_oxide.rs:37-70).  The currents
 * are exactly those hses_perturbed_linear computes for the same arguments
 * (bf16 math) and never reach memory: every (member, slot, output) series over
 * n_time steps is run through hses_lif_scan's update from v0 = 0, giving
 *   d_spikes (n_time, n*rows_per_member, ceil(a/64)) bit-packed words with row
 *            stride spk_stride and time planes spk_plane apart, or NULL;
 *   d_rate   (n*rows_per_member, a) spike count / n_time with row stride
 *            rate_stride (snn.rs:274, mean over time), or NULL.
 * x must be bit-packed (HSES_FMT_BITS); n_time a power of two <= 64; rank a
 * multiple of 16 <= 128, a <= 128, sigma != 0.  d_work as for
 * hses_perturbed_linear (same workspace size query). */
int hses_perturbed_linear_lif(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                              int32_t n_time, const float *d_W, int32_t a, int32_t b,
                              uint64_t key, int32_t rank, float sigma, int32_t epoch,
                              int32_t noise_reuse, int32_t tid_lo, int32_t n,
                              int32_t rows_per_member, float tau_m, float v_th,
                              uint64_t *d_spikes, int64_t spk_stride, int64_t spk_plane,
                              float *d_rate, int64_t rate_stride, void *d_work,
                              size_t work_bytes, void *stream);

/* ---- factor record -------------------------------------------------------
 * The update of a parameter needs the same per-member factors as its forward:
 * the reference draws them for the forward (do_mm, eggroll.rs:419-446) and again
 * as materialised (n, a, r) / (n, b, r) tensors for the update
 * (get_lora_update_params / batched_lora_noise inside _simple_lora_update,
 * eggroll.rs:353-404).  A factor record keeps the normals the forward draws so
 * the update reads them instead: one block per antithetic pair p of the
 * members [tid_lo, tid_lo + n) (pairs tid_lo / 2 .. (tid_lo + n - 1) / 2), the
 * raw normal of stream row j (B rows [0, b), then A rows) and rank c at
 *   rec[((p - tid_lo / 2) * rank + c) * (a + b) + j]   (fp32, before any scale).
 * Rank a multiple of 16 in [32, 128], sigma != 0, do_mm only. */

/* Bytes of the record of members [tid_lo, tid_lo + n) of an (a, b) parameter. */
size_t hses_factor_record_bytes(int32_t a, int32_t b, int32_t rank, int32_t tid_lo, int32_t n);

/* hses_perturbed_linear (bf16 math, a <= 128: the pair kernels) that also
 * writes the factor record of its members to d_rec (rec_bytes >=
 * hses_factor_record_bytes).  y is identical to hses_perturbed_linear's. */
int hses_perturbed_linear_rec(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                              int32_t n_time, const float *d_W, int32_t a, int32_t b,
                              uint64_t key, int32_t rank, float sigma, int32_t epoch,
                              int32_t noise_reuse, int32_t tid_lo, int32_t n,
                              int32_t rows_per_member, float *d_y, int64_t y_stride,
                              int64_t y_plane, int32_t math, void *d_work, size_t work_bytes,
                              float *d_rec, size_t rec_bytes, void *stream);

/* hses_perturbed_linear_lif that also writes the factor record of its members;
 * spikes and rates are identical to hses_perturbed_linear_lif's. */
int hses_perturbed_linear_lif_rec(const void *d_x, int32_t x_fmt, int64_t x_stride,
                                  int64_t x_plane, int32_t n_time, const float *d_W, int32_t a,
                                  int32_t b, uint64_t key, int32_t rank, float sigma,
                                  int32_t epoch, int32_t noise_reuse, int32_t tid_lo, int32_t n,
                                  int32_t rows_per_member, float tau_m, float v_th,
                                  uint64_t *d_spikes, int64_t spk_stride, int64_t spk_plane,
                                  float *d_rate, int64_t rate_stride, void *d_work,
                                  size_t work_bytes, float *d_rec, size_t rec_bytes,
                                  void *stream);

/* ---- factors drawn ahead ---------------------------------------------------
 * The same forwards with the draw split off (get_lora_update_params /
 * batched_lora_noise, eggroll.rs:116-227, as consumed by do_mm
 * eggroll.rs:419-446 and lora_linear_batched snn.rs:665-685): hses_pair_factors
 * draws every pair's factors of members [tid_lo, tid_lo + n) into the factor
 * record and a bf16 operand image of the scaled B factors (pair-major, rank
 * rows padded to a multiple of 64 inputs); the *_pre forwards read both and
 * draw nothing.  Outputs equal the *_rec forwards' bit for bit.  The draw is
 * its own launch, so a caller can run it on another stream or ahead of the
 * forward (it depends on the key, epoch and members only, not on W or x).
 * do_mm only; rank a multiple of 16 in [32, 128], sigma != 0, a <= 128. */

/* Bytes of the operand image of members [tid_lo, tid_lo + n). */
size_t hses_pair_image_bytes(int32_t a, int32_t b, int32_t rank, int32_t tid_lo, int32_t n);

int hses_pair_factors(uint64_t key, int32_t rank, float sigma, int32_t epoch,
                      int32_t noise_reuse, int32_t tid_lo, int32_t n, int32_t a, int32_t b,
                      float *d_rec, size_t rec_bytes, uint16_t *d_img, size_t img_bytes,
                      void *stream);

/* hses_perturbed_linear_rec's y from a record and image written by
 * hses_pair_factors with the same (a, b, rank, sigma, tid_lo, n). */
int hses_perturbed_linear_pre(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                              int32_t n_time, const float *d_W, int32_t a, int32_t b,
                              int32_t rank, float sigma, int32_t tid_lo, int32_t n,
                              int32_t rows_per_member, float *d_y, int64_t y_stride,
                              int64_t y_plane, void *d_work, size_t work_bytes,
                              const float *d_rec, size_t rec_bytes, const uint16_t *d_img,
                              size_t img_bytes, void *stream);

/* hses_perturbed_linear_lif_rec's spikes and rates from a record and image
 * written by hses_pair_factors (n_time <= 16, b <= 1024). */
int hses_perturbed_linear_lif_pre(const void *d_x, int32_t x_fmt, int64_t x_stride,
                                  int64_t x_plane, int32_t n_time, const float *d_W, int32_t a,
                                  int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
                                  int32_t rows_per_member, float tau_m, float v_th,
                                  uint64_t *d_spikes, int64_t spk_stride, int64_t spk_plane,
                                  float *d_rate, int64_t rate_stride, void *d_work,
                                  size_t work_bytes, const float *d_rec, size_t rec_bytes,
                                  const uint16_t *d_img, size_t img_bytes, void *stream);

/* ---- fp32-accurate forwards (HSES_MATH_F32X) -------------------------------
 * The *_pre forwards with every operand held to fp32 accuracy: the same
 * perturbed product x W^T + sign_m (x B_m) A_m^T that snn.rs:665-685
 * (lora_linear_batched) and eggroll.rs:419-446 (do_mm) compute in fp32, on
 * fp16 MFMAs.  Each fp32 operand v is split into an fp16 high part and the
 * fp16 rounding of v - high (v to about 2^-22 of v); x is 0/1 spikes (exact).
 * x W^T takes x W_hi + x W_lo, x B_m takes x B_hi + x B_lo, and its product
 * with A takes (xB)_hi A_hi + (xB)_lo A_hi + (xB)_hi A_lo, all accumulated in
 * fp32, so the currents carry fp32 rounding, not bf16's: the spikes differ
 * from an fp32 evaluation only where a membrane potential lies within fp32
 * summation error of the threshold.  hses_pair_factors_x draws the factors
 * into the record and the split operand image; hses_pair_image_x builds the
 * image from a record written by hses_pair_factors or a *_rec forward.  The
 * *_pre_x forwards take it in place of the bf16 image.
 * Bit-packed x (x_fmt BITS), do_mm, a <= 128, rank a multiple of 16 in
 * [32, 128], b <= 896; workspace as hses_perturbed_linear_workspace with
 * math = HSES_MATH_F32X (or HSES_MATH_BF16: the same size).  None of these
 * has a counterpart in the reference's bf16-free path; they are its fp32
 * arithmetic on this hardware's fp16 matrix cores. */

/* Bytes of the split operand image of members [tid_lo, tid_lo + n). */
size_t hses_pair_image_x_bytes(int32_t a, int32_t b, int32_t rank, int32_t tid_lo, int32_t n);

/* hses_pair_factors with the split operand image in place of the bf16 one:
 * the same record, and the image hses_pair_image_x derives from it.  (Both
 * draws take d_img = NULL with img_bytes = 0 to write the record alone, the
 * input of hses_member_weights.) */
int hses_pair_factors_x(uint64_t key, int32_t rank, float sigma, int32_t epoch,
                        int32_t noise_reuse, int32_t tid_lo, int32_t n, int32_t a, int32_t b,
                        float *d_rec, size_t rec_bytes, uint16_t *d_img, size_t img_bytes,
                        void *stream);

/* The split operand image from a factor record (same a, b, rank, sigma,
 * tid_lo, n as the draw that wrote it). */
int hses_pair_image_x(int32_t a, int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
                      const float *d_rec, size_t rec_bytes, uint16_t *d_img, size_t img_bytes,
                      void *stream);

/* hses_perturbed_linear_pre at fp32 accuracy (d_img from hses_pair_image_x). */
int hses_perturbed_linear_pre_x(const void *d_x, int32_t x_fmt, int64_t x_stride,
                                int64_t x_plane, int32_t n_time, const float *d_W, int32_t a,
                                int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
                                int32_t rows_per_member, float *d_y, int64_t y_stride,
                                int64_t y_plane, void *d_work, size_t work_bytes,
                                const float *d_rec, size_t rec_bytes, const uint16_t *d_img,
                                size_t img_bytes, void *stream);

/* hses_perturbed_linear_lif_pre at fp32 accuracy (d_img from
 * hses_pair_image_x): the LIF of snn.rs:53-97 on fp32-accurate currents. */
int hses_perturbed_linear_lif_pre_x(const void *d_x, int32_t x_fmt, int64_t x_stride,
                                    int64_t x_plane, int32_t n_time, const float *d_W, int32_t a,
                                    int32_t b, int32_t rank, float sigma, int32_t tid_lo,
                                    int32_t n, int32_t rows_per_member, float tau_m, float v_th,
                                    uint64_t *d_spikes, int64_t spk_stride, int64_t spk_plane,
                                    float *d_rate, int64_t rate_stride, void *d_work,
                                    size_t work_bytes, const float *d_rec, size_t rec_bytes,
                                    const uint16_t *d_img, size_t img_bytes, void *stream);

/* hses_perturbed_linear_lif_pre_x that leaves each output row's spike count
 * over the n_time steps as bit planes instead of spikes or rates: row
 * (member m, sample s) holds P = log2(n_time) + 1 planes of ceil(a/64) words
 * at d_counts + (m * rows_per_member + s) * counts_stride, bit c of plane p
 * being bit p of neuron c's count.  rate = sum_p 2^p plane_p / n_time, so the
 * readout of the rate (snn.rs:274-280) is sum_p (2^p / n_time) (plane_p W^T +
 * (plane_p B) A^T): a bit-packed product over P rows per sample.  n_time a
 * power of two <= 16, counts_stride >= P * ceil(a/64). */
int hses_perturbed_linear_lif_counts_pre_x(
    const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane, int32_t n_time,
    const float *d_W, int32_t a, int32_t b, int32_t rank, float sigma, int32_t tid_lo, int32_t n,
    int32_t rows_per_member, float tau_m, float v_th, uint64_t *d_counts, int64_t counts_stride,
    void *d_work, size_t work_bytes, const float *d_rec, size_t rec_bytes, const uint16_t *d_img,
    size_t img_bytes, void *stream);

/* The readout (snn.rs:274-280: logits = rate W^T through do_mm,
 * eggroll.rs:419-446) on the count planes of
 * hses_perturbed_linear_lif_counts_pre_x / hses_perturbed_linear_lif_mw: for
 * every row of members [tid_lo, tid_lo + n), with rate = sum_p 2^p plane_p /
 * n_time,
 *     d_y row = rate (W + sign_m (sigma / sqrt(rank)) A_m B_m^T)^T,
 * A_m, B_m read from the factor record of the (a, b) layer (written by
 * hses_pair_factors or hses_pair_factors_x, with or without an image).  Each
 * pair's member weights are formed in fp32 in LDS and the rows' counts are
 * decoded from the planes, so nothing is materialised: the reference's
 * factored product reassociated (a no-counterpart form for narrow readouts).
 * a <= 32, b <= 128, rows_per_member <= 128, n_time a power of two <= 16,
 * rank a multiple of 16 in [32, 128], sigma != 0; counts_stride (uint64
 * words between rows) >= P * ceil(b/64), P = log2(n_time) + 1. */
int hses_perturbed_readout_counts(const uint64_t *d_counts, int64_t counts_stride,
                                  int32_t n_time, const float *d_W, int32_t a, int32_t b,
                                  int32_t rank, float sigma, int32_t tid_lo, int32_t n,
                                  int32_t rows_per_member, const float *d_rec, size_t rec_bytes,
                                  float *d_y, int64_t y_stride, void *stream);

/* ---- member weights ------------------------------------------------------
 * The same perturbed product formed per member instead of factored: with R
 * rows per member, y_m = x (W + sign_m (sigma / sqrt(r)) A_m B_m^T)^T costs
 * a b r per pair plus R b a per member, against R b (a + r) + R r a for
 * x W^T + sign_m (x B_m) A_m^T (snn.rs:665-685, eggroll.rs:419-446); at the
 * SNN's R = samples x T = 1024 and a = r = 128 about half.
 * hses_member_weights forms every member's W_m from the factor record (a
 * record written by hses_pair_factors with d_img = NULL, by either image
 * form, or by a *_rec forward): with math = HSES_MATH_BF16 W_m in bf16,
 * a x ceil(b/64)*64 per member, zero past b, stored chunk-major
 * ([b/64 chunk][a][64 inputs]); with HSES_MATH_F32X the fp16 high and low
 * parts of 1024 W_m, each of that shape (the product A_m B_m^T
 * is taken on split operands in both, so only W_m's final rounding differs).
 * The forwards read them: bit-packed x, rows per member (n_time x
 * rows_per_member) a multiple of 256, a <= 128, b <= 1024 (b > 64 with
 * HSES_MATH_BF16); the LIF form
 * takes any of spikes, rates or spike-count planes (the layout of
 * hses_perturbed_linear_lif_counts_pre_x; rates and counts exclusive).
 * None of these has a counterpart in the reference; they are its forward
 * reassociated for this hardware. */
size_t hses_member_weights_bytes(int32_t a, int32_t b, int32_t n, int32_t math);

int hses_member_weights(const float *d_W, int32_t a, int32_t b, int32_t rank, float sigma,
                        int32_t tid_lo, int32_t n, const float *d_rec, size_t rec_bytes,
                        int32_t math, uint16_t *d_wm, size_t wm_bytes, void *stream);

int hses_perturbed_linear_mw(const void *d_x, int32_t x_fmt, int64_t x_stride, int64_t x_plane,
                             int32_t n_time, int32_t a, int32_t b, int32_t tid_lo, int32_t n,
                             int32_t rows_per_member, int32_t math, const uint16_t *d_wm,
                             size_t wm_bytes, float *d_y, int64_t y_stride, int64_t y_plane,
                             void *stream);

int hses_perturbed_linear_lif_mw(const void *d_x, int32_t x_fmt, int64_t x_stride,
                                 int64_t x_plane, int32_t n_time, int32_t a, int32_t b,
                                 int32_t tid_lo, int32_t n, int32_t rows_per_member, float tau_m,
                                 float v_th, int32_t math, const uint16_t *d_wm, size_t wm_bytes,
                                 uint64_t *d_spikes, int64_t spk_stride, int64_t spk_plane,
                                 float *d_rate, int64_t rate_stride, uint64_t *d_counts,
                                 int64_t counts_stride, void *stream);

/* ---- ES update ------------------------------------------------------- */

/* EggRoll ES gradient of one MM parameter (eggroll.rs:353-404 _simple_lora_update +
 * _do_update; chunked form eggroll.rs:579-702; pair einsum eggroll.rs:778-915):
 *     d_grad (a, b) = scale * sum_m f[m] * A_m B_m^T
 * over members m in [0, n) with thread ids tid_lo+m, factors regenerated
 * in-kernel.  do_updates uses scale = -sqrt(N)/N (N = population size).
 * Deterministic: a fixed split-K partition and a fixed-order second-stage
 * reduction, no atomics.  accumulate != 0 adds into d_grad (the K-chunk
 * loop of accumulated_update) instead of overwriting it.  d_work must hold
 * hses_es_update_workspace(...) bytes. */
size_t hses_es_update_workspace(int32_t a, int32_t b, int32_t rank, int32_t n);
int hses_es_update(const float *d_f, int32_t n, int32_t tid_lo, uint64_t key, int32_t rank,
                   float sigma, int32_t epoch, int32_t noise_reuse, int32_t a, int32_t b,
                   float scale, int32_t accumulate, float *d_grad, void *d_work,
                   size_t work_bytes, void *stream);
/* No counterpart in the reference: hses_es_update for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and result (to fp32 rounding: the split count
 * may be lower) without the workspace: the split-K partials live in a fixed
 * 32 MiB device array of the library, one per GPU, kept until the process
 * ends.  Rejects a * b > (32 MiB - 16) / 4 elements with HSES_ERR_INVALID_ARG.
 * Calls share the array, so calls that overlap on one GPU race. */
int hses_es_update_noalloc(const float *d_f, int32_t n, int32_t tid_lo, uint64_t key,
                           int32_t rank, float sigma, int32_t epoch, int32_t noise_reuse,
                           int32_t a, int32_t b, float scale, int32_t accumulate, float *d_grad,
                           void *stream);

/* hses_es_update (same reference functions) of members [tid_lo, tid_lo + n)
 * reading their normals from the factor record a *_rec forward over the same
 * tid_lo and n wrote (rank >= 32): the same result, bit for bit, without
 * drawing the normals again.  Workspace: hses_es_update_workspace. */
int hses_es_update_rec(const float *d_f, int32_t n, int32_t tid_lo, const float *d_rec,
                       size_t rec_bytes, int32_t rank, float sigma, int32_t a, int32_t b,
                       float scale, int32_t accumulate, float *d_grad, void *d_work,
                       size_t work_bytes, void *stream);

/* ---- fitness, z-score, solver ----------------------------------------- */

/* fitness_from_logits_reward(Loglik) (burn_impl/hyperscalees-envs/src/snn_mnist.rs:180-201)
 * averaged over each member's rows: d_fit[m] = mean_s log_softmax(logits[m*rows+s])[label]. */
int hses_member_loglik(const float *d_logits, int32_t classes, const int32_t *d_labels,
                       int32_t n, int32_t rows_per_member, float *d_fit, void *stream);

/* fitness_from_logits_reward (snn_mnist.rs:180-201) with either reward, averaged over
 * each member's rows: Loglik log_softmax(row)[label]; Binary 1.0 when the first maximal
 * class (argmax) is the label, else 0.0.  d_correct (optional) is incremented by the
 * number of rows whose argmax is the label: the train-accuracy counter of the K-chunk
 * driver (accumulate_train.rs:847-849). */
int hses_member_fitness(const float *d_logits, int32_t classes, const int32_t *d_labels,
                        int32_t n, int32_t rows_per_member, int32_t reward, float *d_fit,
                        unsigned long long *d_correct, void *stream);

/* The K-chunk driver's raw-fitness sums (accumulate_train.rs:843-846): d_moments[0] and
 * d_moments[1] receive sum(raw) and sum(raw^2) of this chunk in double, overwritten
 * (accumulate 0, first chunk) or added to (accumulate 1).  One block; deterministic. */
int hses_fitness_moments(const float *d_raw, int32_t n, double *d_moments, int32_t accumulate,
                         void *stream);

/* combine_affine_grads (eggroll.rs:902-915) with the driver's global mean and std
 * (accumulate_train.rs:940-944) read from d_moments over `batch` members:
 * mean = S1/batch, var = max(S2/batch - mean^2, 0), std = sqrt(var + 1e-5),
 * d_out = (d_grad_acc - d_ones_acc*mean) * (-1/(std*sqrt(batch))).  d_ones_acc may be
 * NULL (an all-zero ones sum); d_out may alias d_grad_acc.  No host synchronisation. */
int hses_combine_affine(const float *d_grad_acc, const float *d_ones_acc, const double *d_moments,
                        int32_t batch, int64_t len, float *d_out, void *stream);

/* ---- RWKV-7 components (burn_impl/hyperscalees-models/src/llm.rs) ------ */

/* layer_norm / LayerNorm::forward (llm.rs:42-83): each of `rows` rows of C floats,
 * y = (x - mean) / sqrt(E[x^2] - mean^2 + eps) * w + b.  y may alias x. */
int hses_layer_norm(const float *d_x, int64_t rows, int32_t C, const float *d_w, const float *d_b,
                    float eps, float *d_y, void *stream);
/* GroupNorm::forward (llm.rs:97-150): x (n, C, L) (L = 1 for the rank-2 form),
 * G groups of C/G channels x L positions; y = w[c] * (x - mean) / sqrt(var + eps) + b[c]. */
int hses_group_norm(const float *d_x, int64_t n, int32_t C, int32_t L, int32_t G,
                    const float *d_w, const float *d_b, float eps, float *d_y, void *stream);
/* The token shift of TimeMixing / ChannelMixing (llm.rs:200-205, 360-381) with n_mix
 * mixing vectors: sx = [state, x[:-1]] (0 where new_starts) - x; out[m] = x + sx * mix[m].
 * x (nseq, T, C); state (nseq, C); new_starts (nseq, T) bytes or NULL; mix (n_mix, C);
 * out (n_mix, nseq, T, C) in out_fmt: HSES_FMT_F32, or HSES_FMT_BF16 (each value rounded to
 * nearest even, what a bf16-math forward does to its input). */
int hses_token_shift_mix(const float *d_x, const float *d_state, const uint8_t *d_new_starts,
                         const float *d_mix, int32_t n_mix, int64_t nseq, int32_t T, int32_t C,
                         void *d_out, int32_t out_fmt, void *stream);
/* ChannelMixing's activation (llm.rs:206): x = relu(x)^2 in place. */
int hses_relu_sq(float *d_x, int64_t n, void *stream);
/* rwkv7_inner_loop (llm.rs:235-300) for nseq independent sequences: r, w, k, v, a, b
 * (nseq, T, H, S) with w the raw decay (exp(-exp(w)) is applied here); s_in (nseq, H, S, S);
 * new_starts (nseq, T) bytes or NULL (a set byte zeroes the state before that step);
 * out (nseq, T, H, S); s_out (nseq, H, S, S) = the state after the last step t < length
 * (s_in when length == 0).  S = 16, 32 or 64; s_out must not alias s_in.  s_in NULL starts
 * from the zero state; s_out NULL does not store the final state (both, also for
 * hses_tm_wkv_post and hses_tm_fused). */
int hses_rwkv7_wkv(const float *d_r, const float *d_w, const float *d_k, const float *d_v,
                   const float *d_a, const float *d_b, const float *d_s_in,
                   const uint8_t *d_new_starts, int64_t nseq, int32_t T, int32_t H, int32_t S,
                   int32_t length, float *d_out, float *d_s_out, void *stream);

/* hses_rwkv7_wkv followed by the rest of TimeMixing's per-head algebra (llm.rs:455-470):
 * out = (GroupNorm_head(wkv; ln_w, ln_b, eps) + (sum_s r k r_k) v) * g, formed exactly as
 * hses_group_norm (G = H, L = 1) and hses_tm_post form it (bit-identical to that chain),
 * without writing the recurrence output.  g (nseq, T, H*S); ln_w, ln_b, r_k (H*S); out in
 * out_fmt (HSES_FMT_F32, or HSES_FMT_BF16 rounded to nearest even for a bf16-math output
 * projection) must not alias r, k or v. */
int hses_tm_wkv_post(const float *d_r, const float *d_w, const float *d_k, const float *d_v,
                     const float *d_a, const float *d_b, const float *d_s_in,
                     const uint8_t *d_new_starts, int64_t nseq, int32_t T, int32_t H, int32_t S,
                     int32_t length, const float *d_g, const float *d_ln_w, const float *d_ln_b,
                     float eps, const float *d_r_k, void *d_out, int32_t out_fmt, float *d_s_out,
                     void *stream);

/* hses_tm_gates_kk followed by hses_tm_wkv_post in one kernel (llm.rs:388-470), equal to
 * that chain bit for bit: from TimeMixing's raw projections r, k, v (nseq, T, H*S), the decay
 * branch's w2 output w2o, the rate branch's a2 output a2o and (after the first layer) the value
 * branch's v2 output v2o with v_first (else NULL), the gates, kk normalisation and k update are
 * formed per step inside the recurrence; w2o, k, v and the rest are only read. */
int hses_tm_fused(const float *d_r, const float *d_w2o, const float *d_k, const float *d_v,
                  const float *d_a2o, const float *d_v2o, const float *d_v_first, const float *d_w0,
                  const float *d_a0, const float *d_v0, const float *d_k_k, const float *d_k_a,
                  const float *d_s_in, const uint8_t *d_new_starts, int64_t nseq, int32_t T,
                  int32_t H, int32_t S, int32_t length, const float *d_g, const float *d_ln_w,
                  const float *d_ln_b, float eps, const float *d_r_k, void *d_out, int32_t out_fmt,
                  float *d_s_out, void *stream);

/* TimeMixing (llm.rs:348-480) pieces around the projections and the recurrence:
 * hses_rwkv_act: x = tanh(x) (kind 0) or sigmoid(x) (kind 1) in place (the low-rank branches);
 * hses_tm_gates (llm.rs:388-408), per element of (rows, C): w2o <- -softplus(-(w0 + w2o)) - 0.5,
 *   a2o <- sigmoid(a0 + a2o), and when v2o != NULL v <- v + (v_first - v) * sigmoid(v0 + v2o);
 * hses_tm_kk (llm.rs:414-426) per (row, head): kk = k k_k / max(||k k_k||, 1e-12), a_i = -kk,
 *   b_i = kk a, k <- k (k_a (a - 1) + 1);
 * hses_tm_post (llm.rs:455-470) per (row, head): gn <- (gn + (sum_s r k r_k) v) g.
 * Head size S <= 64; C = H * S. */
int hses_rwkv_act(float *d_x, int64_t n, int32_t kind, void *stream);
int hses_tm_gates(float *d_w2o, float *d_a2o, const float *d_v2o, float *d_v, const float *d_v_first,
                  const float *d_w0, const float *d_a0, const float *d_v0, int64_t rows, int32_t C,
                  void *stream);
int hses_tm_kk(float *d_k, const float *d_k_k, const float *d_k_a, const float *d_a, int64_t rows,
               int32_t H, int32_t S, float *d_ai, float *d_bi, void *stream);
int hses_tm_post(float *d_gn, const float *d_r, const float *d_k, const float *d_v, const float *d_g,
                 const float *d_r_k, int64_t rows, int32_t H, int32_t S, void *stream);
/* hses_tm_gates then hses_tm_kk in one pass (llm.rs:388-426), equal to the two calls bit for
 * bit; the in-context rate a stays in registers (a2o is only read). */
int hses_tm_gates_kk(float *d_w2o, const float *d_a2o, const float *d_v2o, float *d_v,
                     const float *d_v_first, const float *d_w0, const float *d_a0, const float *d_v0,
                     float *d_k, const float *d_k_k, const float *d_k_a, int64_t rows, int32_t H,
                     int32_t S, float *d_ai, float *d_bi, void *stream);

/* The RWKV-7 LM around the blocks (src/hyperscalees/models/llm/rwkv7.py:189-253):
 * hses_embed_layer_norm: y[i] = LayerNorm(emb[tokens[i]]) with ln0's w, b (embed and
 *   the ln0 of forward_seq; a token outside [0, V) gives a row of NaN);
 * hses_add_layer_norm: x += delta in place, then y = LayerNorm(x) (a block's residual
 *   add and the ln2 / next ln1 / ln_out that reads it); y must not alias x or delta.
 * LayerNorm as hses_layer_norm. */
int hses_embed_layer_norm(const int32_t *d_tokens, int64_t rows, const float *d_emb, int32_t V,
                          int32_t C, const float *d_w, const float *d_b, float eps, float *d_y,
                          void *stream);
int hses_add_layer_norm(float *d_x, const float *d_delta, int64_t rows, int32_t C,
                        const float *d_w, const float *d_b, float eps, float *d_y, void *stream);
/* A block's residual add, the LayerNorm that reads it and the next module's token shift
 * in one pass (rwkv7.py:240-249 around llm.rs:66-83, 200-205, 360-381): x (nseq, T, C) +=
 * delta (delta NULL: x only read), y = LayerNorm(x) with w, b, then out[m] = y + ([state,
 * y[:-1]] (0 where new_starts) - y) * mix[m] for the n_mix mixing vectors, (n_mix, nseq, T, C)
 * in out_fmt (HSES_FMT_F32 or HSES_FMT_BF16); state (nseq, C) the previous token's y;
 * y_last (nseq, C) or NULL receives y at row length - 1 (the next shift state).  The values
 * of hses_add_layer_norm followed by hses_token_shift_mix, bit for bit (without delta, of
 * hses_add_layer_norm with a zero delta), without y in memory.  Returns
 * HSES_ERR_UNSUPPORTED unless C is 256, 512 or 1024, n_mix is 1 or 6 and every buffer is
 * 16-byte aligned (callers then run the two steps). */
int hses_add_ln_shift(float *d_x, const float *d_delta, int64_t nseq, int32_t T, int32_t C,
                      const float *d_w, const float *d_b, float eps, const float *d_state,
                      const uint8_t *d_new_starts, const float *d_mix, int32_t n_mix, void *d_out,
                      int32_t out_fmt, float *d_y_last, int32_t length, void *stream);

/* ---- data path (host only: no device, no stream) ---------------------- */

/* read_idx_images (burn_impl/hyperscalees-envs/src/snn_mnist.rs:57-88): an IDX images
 * buffer, plain or gzip (leading 1f 8b), into pixels / 255 as f32, image-major.
 * *n_images and *pixels (rows * cols) are always set; out (may be NULL: sizes only)
 * must hold out_cap >= n_images * pixels floats.  Bad magic, a short payload, sizes
 * beyond 2^30 elements or a corrupt gzip stream return HSES_ERR_INVALID_ARG. */
int hses_read_idx_images(const uint8_t *data, size_t len, float *out, int64_t out_cap,
                         int64_t *n_images, int64_t *pixels);
/* read_idx_labels (snn_mnist.rs:90-112): an IDX labels buffer (plain or gzip) into
 * raw bytes; *n_labels always set, out (may be NULL) must hold out_cap >= n_labels. */
int hses_read_idx_labels(const uint8_t *data, size_t len, uint8_t *out, int64_t out_cap,
                         int64_t *n_labels);
/* shuffled_indices (burn_impl/hyperscalees/src/bin/accumulate_train.rs:157-174): the first
 * `count` entries of a partial Fisher-Yates shuffle of [0, n) driven by xorshift64
 * (13, 7, 17) from (seed ^ 0x9E3779B97F4A7C15) | 1, each draw multiplied by
 * 0x2545F4914F6CDD1D and reduced mod (n - i).  Requires 0 <= count <= n. */
int hses_shuffled_indices(int64_t n, int64_t count, uint64_t seed, int64_t *out);

/* convert_fitnesses (eggroll.rs:967-992): global (group_size 0) or per-group
 * z-score with the global std.  d_stats (optional) receives {mean, std}. */
int hses_convert_fitnesses(const float *d_raw, int32_t n, int32_t group_size, float *d_out,
                           float *d_stats, void *stream);

/* Solver::update for one parameter (noiser.rs:155-225).  step_t is the
 * already-incremented global step.  m, v are updated in place (ignored for SGD). */
int hses_solver_step(int32_t kind, float lr, float beta1, float beta2, float eps, float wd,
                     int32_t step_t, float *d_param, const float *d_grad, float *d_m, float *d_v,
                     int64_t len, void *stream);
/* The same step on the gradient multiplied by the device scalar *d_gscale
 * (NULL: 1): Solver::TrustRegion (noiser.rs:215-222) with the factor of
 * hses_clip_global_norm. */
int hses_solver_step_scaled(int32_t kind, float lr, float beta1, float beta2, float eps, float wd,
                            int32_t step_t, float *d_param, const float *d_grad, float *d_m,
                            float *d_v, int64_t len, const float *d_gscale, void *stream);

/* clip_grads_global_norm (noiser.rs:231-244), the factor only: over the n
 * gradient tensors h_grads[i] (device pointers in a host array) of h_lens[i]
 * floats, ||g|| = sqrt(sum_i sum g^2) and *d_scale = max_norm / ||g|| when
 * ||g|| > max_norm and ||g|| > 0, else 1.  Each tensor's sum of squares is a
 * fixed-order double reduction (f32 squares) rounded to f32; the tensors'
 * sums are added in f32 in order.  d_work holds 64 * n doubles. */
int hses_clip_global_norm(const float *const *h_grads, const int64_t *h_lens, int32_t n,
                          float max_norm, double *d_work, float *d_scale, void *stream);

/* ---- spiking self-attention transformer (C4) -------------------------- */
/* The model of src/hyperscalees/models/snn_self_attention_heads.py batched over
 * a population: member m owns rows [m R, (m+1) R) of every (rows, C) plane
 * (R = tokens per member); per-member scalars (thresholds, beta, gains) are
 * device arrays of n floats.  Its perturbed projections are
 * hses_perturbed_linear calls (one per MM leaf, heads written into column
 * blocks through y_stride); its Parameter leaves are perturbed with
 * hses_noisy_standard. */

/* jax.nn.softplus (the models' positive-threshold map, snn_self_attention_heads.py:43-44):
 * y = max(x, 0) + log1p(exp(-|x|)). */
int hses_softplus(const float *d_x, int64_t n, float *d_y, void *stream);

/* The input encoders (_rate, snn_self_attention_heads.py:33-40, 168-175):
 * X = (rate(cq) + rate(ck) + rate(cv)) / 3 + pos, rate = mean over T of the LIF
 * spikes (snn_attention.py:41-61, v0 = 0) of the time-major (T, M, d)
 * projection currents with member m's threshold th_*[m].  pos is (R, d)
 * (pos_per_member 0) or (M, d). */
int hses_sa_encode(const float *d_cq, const float *d_ck, const float *d_cv, int32_t T, int64_t M,
                   int32_t d, int32_t rows_per_member, const float *d_th_q, const float *d_th_k,
                   const float *d_th_v, float tau_m, const float *d_pos, int32_t pos_per_member,
                   float *d_X, void *stream);

/* The attention of multihead_attention_once (snn_self_attention_heads.py:47-73)
 * for every member and head: head h of a row is columns [h hd, (h+1) hd) of q, k,
 * v and out ((n R, ld) fp32); A = row_softmax_lif(beta[m] (Q K^T))
 * (snn_self_attention.py:45-80: n_iter LIF steps of the key neurons on
 * h / (max |h| + 1e-6) - g_inh * sum(count), p = count / (sum count + 1e-6),
 * threshold vth[m]), out = A V.  R <= 64, hd <= 64. */
int hses_sa_attention(const float *d_q, const float *d_k, const float *d_v, int32_t ld, int64_t n,
                      int32_t R, int32_t H, int32_t hd, const float *d_beta, const float *d_vth,
                      float g_inh, float tau_m, int32_t n_iter, float *d_out, void *stream);

/* ffn_once's lif_single (snn_self_attention_heads.py:79-83): per row,
 * act = (c / max(max |c|, 1e-6) >= vth[m]) as 0/1 fp32. */
int hses_sa_ffn_spike(const float *d_c, int64_t M, int32_t d, int32_t rows_per_member,
                      const float *d_vth, float *d_act, void *stream);

/* x += y (the blocks' residual adds, snn_self_attention_heads.py:186-187). */
int hses_add_inplace(float *d_x, const float *d_y, int64_t n, void *stream);

/* jnp.mean(X, axis=0) per member (snn_self_attention_heads.py:189):
 * out (n, d) = sum of the member's R rows / R, in row order. */
int hses_sa_pool(const float *d_X, int64_t n, int32_t R, int32_t d, float *d_out, void *stream);

/* y[r, :] *= s[r] (logits * out_gain per member, snn_self_attention_heads.py:191-192). */
int hses_scale_rows(float *d_y, int64_t rows, int32_t cols, const float *d_s, void *stream);

#ifdef __cplusplus
}
#endif
#endif
