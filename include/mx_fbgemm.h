/*
 * mx_fbgemm.h -- C-ABI of the MI355X (gfx950) kernels behind the
 * torch.ops.fbgemm.* drop-in operators.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * passed as `void*`.  Scratch memory is sized by a *_workspace_bytes() query
 * and handed in by the caller.  One exception: an eager (not graph-captured)
 * TBE backward keeps its radix sort's digit counters (about 2 MiB) in a
 * region of the current device and stream that the call's last kernel
 * leaves zeroed for the next call, allocated by the stream's first such
 * call and kept until the process ends (at most 64 streams per device);
 * under capture, past those 64 streams, or if that allocation fails, the
 * counters live in the workspace and one more kernel clears them.  Nothing
 * else allocates.  All calls are
 * asynchronous on `stream` and never synchronise the host.  They return
 * MX_OK (0) or a negative status; mx_last_error() then holds a
 * thread-local message.
 *
 * Which interface each function replaces.  The reference snapshot
 * (/root/reference) ships no FBGEMM code; its plugin boundary is a
 * torch.ops.load_library()'d .so whose static initializer registers the
 * device implementation under the upstream project's own interface
 * (reference: packages/torchcodec-xpu/src/torchcodec_xpu/__init__.py:25-56,
 * XpuDeviceInterface.cpp:33-35).  For this path the upstream interface is
 * the `fbgemm` dispatcher namespace of fbgemm_gpu; the op each function
 * serves is named in its comment (upstream fbgemm_gpu, recalled names, no
 * line numbers available offline).
 */
#ifndef MX_FBGEMM_H
#define MX_FBGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
#define MX_OK 0
#define MX_EINVAL (-1)       /* bad argument (shape, size, enum)             */
#define MX_EHIP (-2)         /* a HIP runtime call failed                    */
#define MX_EUNSUPPORTED (-3) /* valid request this build does not implement  */
#define MX_EWORKSPACE (-4)   /* workspace missing or smaller than required   */

/* ---- enums shared with the host layer ----------------------------------
 * Element types of dense/jagged tensors (own numbering). */
#define MX_DTYPE_F32 0
#define MX_DTYPE_F16 1
#define MX_DTYPE_BF16 2
#define MX_DTYPE_F64 3

/* fbgemm_gpu SparseType values (weights_tys / output_dtype). */
#define MX_SPARSE_FP32 0
#define MX_SPARSE_FP16 1
#define MX_SPARSE_INT8 2
#define MX_SPARSE_INT4 3
#define MX_SPARSE_INT2 4
#define MX_SPARSE_BF16 5
#define MX_SPARSE_FP8 6

/* fbgemm_gpu PoolingMode values. */
#define MX_POOL_SUM 0
#define MX_POOL_MEAN 1
#define MX_POOL_NONE 2

/* fbgemm_gpu BoundsCheckMode values. */
#define MX_BOUNDS_FATAL 0
#define MX_BOUNDS_WARNING 1
#define MX_BOUNDS_IGNORE 2
#define MX_BOUNDS_NONE 3

/* Maximum number of jagged dimensions the jagged kernels accept. */
#define MX_MAX_JAGGED_DIM 4

/* Library version (major*10000 + minor*100 + patch).  MX_FBGEMM_VERSION is
 * the version this header describes; a caller compares it with mx_version()
 * before binding.  0.2.0: mx_tbe_backward_rowwise_adagrad(_vbe) take their
 * stochastic-rounding state as `const mx_rng_state*` where 0.1.0 took a
 * `uint64_t seed` at the same position, and mx_set_status_mailbox takes
 * MX_STATUS_WORDS words where 0.1.0 took one (not binary compatible).
 * 0.3.0: eager TBE backward calls keep their sort counters in a per-stream
 * region (see above); mx_test_force_workspace_counters added.  0.4.0:
 * mx_nbit_forward takes max_float8_D, fp8_exponent_bits and
 * fp8_exponent_bias after row_alignment (FP8 tables; not binary compatible);
 * mx_float_to_hfp8 and mx_hfp8_to_float added; output_dtype MX_SPARSE_BF16
 * accepted.  0.5.0: the PoolingMode NONE (sequence) entry points added:
 * mx_tbe_forward_nobag, mx_tbe_backward_rowwise_adagrad_nobag,
 * mx_tbe_transpose_embedding_input_nobag, mx_nbit_forward_nobag and their
 * workspace queries, mx_cumsum, mx_permute_2d_lengths, mx_permute_2d_data
 * with mx_cumsum_workspace_bytes, mx_offsets_range, mx_expand_into_jagged_permute
 * and mx_jagged_dense_elementwise_mul (all earlier ones unchanged). */
#define MX_FBGEMM_VERSION 500
int mx_version(void);

/* Thread-local text of the last failing call on this thread ("" if none). */
const char* mx_last_error(void);

/* ---- look-back failures (no fbgemm counterpart) --------------------------
 * The radix sort and the prefix scans of the TBE backward and of
 * transpose_embedding_input wait, tile by tile, for the counts of earlier
 * tiles (decoupled look-back).  Every such wait is bounded; one that runs
 * out (never expected: the tile waited on was scheduled earlier and
 * publishes without waiting) makes the call leave its outputs -- the run
 * layout, the weight and momentum update -- unwritten, and stores 1 into
 * word MX_STATUS_LOOKBACK of the host-visible status words registered here
 * for the current device.
 * mx_nbit_forward stores 1 into word MX_STATUS_NBIT_TABLE when a table of the
 * call cannot be served -- its type byte names no type the call's max_*_D
 * arguments launch, it is an INT4 table of odd D or an INT2 table of D not a
 * multiple of 4, or its rows do not start at 4-byte boundaries (its
 * weights_offsets entry or its row stride after row_alignment is not a
 * multiple of 4) -- after writing that table's output columns as zeros.
 * host_words points at MX_STATUS_WORDS words of pinned host memory owned by
 * the caller, which reads and clears them; NULL unregisters.  Kernels
 * launched before a registration (or captured in a graph before it) do not
 * see it. */
#define MX_STATUS_LOOKBACK 0
#define MX_STATUS_NBIT_TABLE 1
#define MX_STATUS_WORDS 2
int mx_set_status_mailbox(unsigned int* host_words);

/* Test hook: while enabled, every look-back wait of later calls gives up at
 * once (failure-handling tests; every kernel still exits normally). */
int mx_test_force_lookback_giveup(int enable);

/* Test hook: while enabled, the radix sort of later calls keeps its
 * look-back counts in 64-bit words, the form used for sorts of 2^30 keys or
 * more, whatever the key count (lets tests cover that form at small sizes). */
int mx_test_force_wide_sort_words(int enable);

/* Test hook: while enabled, eager TBE backward calls keep their sort counters
 * in the caller's workspace and clear them with one more kernel, as calls
 * under graph capture always do, instead of using the stream's zeroed
 * counter region (lets tests compare the two forms). */
int mx_test_force_workspace_counters(int enable);

/* ---- jagged tensor ops ------------------------------------------------- */

/* Serves fbgemm::jagged_to_padded_dense_forward (and the forward of
 * fbgemm::jagged_to_padded_dense).
 *   values   [total_L, inner] elements of `elem_bytes` bytes each
 *   offsets  num_jagged_dim device arrays (host array of device pointers),
 *            int32 (offset_bytes 4) or int64 (offset_bytes 8); level 0
 *            bounds the B = offsets_numel[0]-1 outer rows, level k bounds
 *            the rows of level k-1
 *   offsets_numel  host array: entries in each offsets array
 *   max_lengths    host array: padded length of each jagged dimension
 *   out      [B, max_lengths[0], ..., max_lengths[k-1], inner]
 *   pad_bits the padding value's bit pattern in the element type
 * Positions past a row's length get the padding value; rows longer than
 * max_length are truncated.  Pure data movement: bit-exact. */
int mx_jagged_to_padded_dense(const void* values, int64_t elem_bytes, int64_t inner,
                              int32_t num_jagged_dim, const void* const* offsets,
                              int32_t offset_bytes, const int64_t* offsets_numel,
                              const int64_t* max_lengths, uint64_t pad_bits, void* out,
                              void* stream);

/* Serves fbgemm::dense_to_jagged_forward (and fbgemm::dense_to_jagged).
 *   dense    [B, max_lengths..., inner]
 *   out      [total_L, inner]: row i takes dense at its jagged coordinate;
 *            rows whose coordinate falls outside max_lengths, or past the
 *            last offset, are written as zero bits. */
int mx_dense_to_jagged(const void* dense, int64_t elem_bytes, int64_t inner,
                       int32_t num_jagged_dim, const void* const* offsets, int32_t offset_bytes,
                       const int64_t* offsets_numel, const int64_t* max_lengths, int64_t total_L,
                       void* out, void* stream);

/* Serves fbgemm::jagged_dense_elementwise_add_jagged_output.
 *   out[i] = x[i] + y[coordinate(i)] in the element type's arithmetic
 *   (f16/bf16 computed in fp32 and rounded to nearest even); where the
 *   coordinate lies outside y, out[i] = x[i] + 0. */
int mx_jagged_dense_elementwise_add(const void* x_values, const void* y_dense, int32_t dtype,
                                    int64_t inner, int32_t num_jagged_dim,
                                    const void* const* offsets, int32_t offset_bytes,
                                    const int64_t* offsets_numel, const int64_t* max_lengths,
                                    int64_t total_L, void* out, void* stream);

/* Serves fbgemm::jagged_dense_elementwise_mul: out[i] = x[i] * y[coordinate(i)]
 * in the element type's arithmetic (f16/bf16 computed in fp32 and rounded to
 * nearest even); where the coordinate lies outside y, out[i] = x[i] * 0. */
int mx_jagged_dense_elementwise_mul(const void* x_values, const void* y_dense, int32_t dtype,
                                    int64_t inner, int32_t num_jagged_dim,
                                    const void* const* offsets, int32_t offset_bytes,
                                    const int64_t* offsets_numel, const int64_t* max_lengths,
                                    int64_t total_L, void* out, void* stream);

/* ---- TBE training forward ---------------------------------------------- */

/* Serves fbgemm::split_embedding_codegen_forward_unweighted_cuda /
 * _weighted_cuda (the forward of the split_embedding_codegen_lookup_*
 * autograd functions), DEVICE placement, fp32 or fp16 weights.
 *   weights         all tables back to back, fp32 (weights_ty MX_SPARSE_FP32)
 *                   or fp16 (MX_SPARSE_FP16; widened to fp32 per element)
 *   weights_offsets int64 [T] element offset of each table
 *   D_offsets       int32 [T+1]; every D_t a multiple of 4, max_D <= 1024
 *   indices         [N] int32 (index_bytes 4) or int64 (8)
 *   offsets         [T*B+1], same integer type as indices, t-major bags
 *   indice_weights  fp32 [N] or NULL
 *   out             [B, total_D] fp32 (out_dtype MX_SPARSE_FP32) or fp16
 * SUM: per column, rows are added in index order starting from +0.0.
 * MEAN: the sum times (1.0f / L); empty bags give 0. */
int mx_tbe_forward(const void* weights, int32_t weights_ty, const int64_t* weights_offsets,
                   const int32_t* D_offsets, int32_t T, int64_t B, int32_t max_D,
                   const void* indices, const void* offsets, int32_t index_bytes,
                   int32_t pooling_mode, const float* indice_weights, void* out,
                   int32_t out_dtype, int64_t total_D, void* stream);

/* ---- variable batch size per feature (VBE) ------------------------------- */

/* Serves fbgemm::generate_vbe_metadata.  Feature (table) t has B[t][r]
 * samples on rank r (R ranks).  Bags are flattened feature-major and, within
 * a feature, rank-major: bag(t, b) = B_offsets[t] + b with
 * b = B_offsets_rank_per_feature[t*(R+1) + r] + b_r.  The pooled output is one
 * flat buffer, rank-major then feature-major; the (r, t) block starts at
 * output_offsets_feature_rank[r*T + t].  Writes, per bag,
 *   row_output_offsets[bag] = output_offsets_feature_rank[r*T + t] + b_r * D
 *   b_t_map[bag]            = (t << info_B_num_bits) | b
 * with D = D_offsets[t+1] - D_offsets[t], or fixed_D when fixed_D > 0.
 *   B_offsets [T+1] int32, B_offsets_rank_per_feature [T][R+1] int32,
 *   output_offsets_feature_rank [R*T+1] int64, total_B = B_offsets[T]. */
int mx_generate_vbe_metadata(const int32_t* B_offsets, const int32_t* B_offsets_rank_per_feature,
                             const int64_t* output_offsets_feature_rank,
                             const int32_t* D_offsets, int32_t fixed_D, int32_t T, int32_t R,
                             int32_t info_B_num_bits, int64_t total_B,
                             int64_t* row_output_offsets, int32_t* b_t_map, void* stream);

/* Serves fbgemm::split_embedding_codegen_forward_{unweighted,weighted}_vbe_cuda:
 * mx_tbe_forward over total_B flattened bags (offsets [total_B+1]); bag i is
 * table t, sample b of b_t_map[i] and its pooled row is written at
 * out + vbe_row_output_offsets[i] (out is the flat VBE output). */
int mx_tbe_forward_vbe(const void* weights, int32_t weights_ty, const int64_t* weights_offsets,
                       const int32_t* D_offsets, int32_t T, int64_t total_B, int32_t max_D,
                       const void* indices, const void* offsets, int32_t index_bytes,
                       int32_t pooling_mode, const float* indice_weights,
                       const int64_t* vbe_row_output_offsets, const int32_t* vbe_b_t_map,
                       int32_t info_B_num_bits, void* out, int32_t out_dtype, void* stream);

/* Serves fbgemm::split_embedding_nobag_codegen_forward_unweighted_cuda (the
 * PoolingMode NONE forward of the lookup function): every table has width D
 * (a multiple of 4, at most 1024) and position l of bag (t, b) writes its own
 * row, out[l, :] = W_t[indices[l], :] (fp16 weights widened to fp32, then
 * the output type: fp32, or fp16 rounded to nearest even).
 *   out     [N, D]; positions outside every bag (before offsets[0], from
 *           offsets[T*B] on) are written as zeros. */
int mx_tbe_forward_nobag(const void* weights, int32_t weights_ty, const int64_t* weights_offsets,
                         int32_t T, int64_t B, int32_t D, const void* indices,
                         const void* offsets, int32_t index_bytes, int64_t N, void* out,
                         int32_t out_dtype, void* stream);

/* ---- TBE backward: transpose (sort) and fused exact rowwise Adagrad ----- */

/* Number of info bits used for the bag index b in an info word
 * ((t << info_B_num_bits) | b); returns -1 if T and B do not fit 32 bits. */
int32_t mx_tbe_info_B_num_bits(int32_t T, int64_t B);

/* Workspace needed by mx_tbe_transpose_embedding_input (N lookups). */
size_t mx_tbe_transpose_workspace_bytes(int64_t N, int32_t total_hash_size_bits);

/* Serves fbgemm::transpose_embedding_input (linearize_index + stable radix
 * sort of pairs + run-length encode + complete cumsum).
 *   linear_indices[l]      = hash_size_cumsum[t] + indices[l]
 *   infos (sorted)         = (t << info_B_num_bits) | b
 *   sorted_linear_indices  keys stably sorted on their low
 *                          total_hash_size_bits bits
 *   run / run_lengths      unique keys and their counts, num_runs of them
 *   cumulative_run_lengths [num_runs+1] exclusive cumsum of run_lengths
 * Run arrays are sized N (cumulative_run_lengths N+1) and read as the
 * complete cumsum of the zero-padded run lengths: past num_runs every
 * run_lengths entry is 0 and every cumulative_run_lengths entry N; run keys
 * past num_runs are left as they were (num_runs stays on the device).
 * Integer work: bit-exact. */
int mx_tbe_transpose_embedding_input(
    const int64_t* hash_size_cumsum, int32_t T, int64_t B, int32_t total_hash_size_bits,
    int32_t info_B_num_bits, const void* indices, const void* offsets, int32_t index_bytes,
    int64_t N, int64_t* linear_indices, int64_t* sorted_linear_indices, int32_t* infos_sorted,
    int64_t* sorted_linear_indices_run, int32_t* run_lengths, int32_t* num_runs,
    int32_t* cumulative_run_lengths, void* workspace, size_t workspace_bytes, void* stream);

/* VBE variant of mx_tbe_transpose_embedding_input (fbgemm's vbe_b_t_map
 * argument): total_B flattened bags, each bag's info word taken from
 * vbe_b_t_map; workspace from mx_tbe_transpose_workspace_bytes. */
int mx_tbe_transpose_embedding_input_vbe(
    const int64_t* hash_size_cumsum, int32_t T, int64_t total_B, const int32_t* vbe_b_t_map,
    int32_t total_hash_size_bits, int32_t info_B_num_bits, const void* indices,
    const void* offsets, int32_t index_bytes, int64_t N, int64_t* linear_indices,
    int64_t* sorted_linear_indices, int32_t* infos_sorted, int64_t* sorted_linear_indices_run,
    int32_t* run_lengths, int32_t* num_runs, int32_t* cumulative_run_lengths, void* workspace,
    size_t workspace_bytes, void* stream);

/* Workspace needed by mx_tbe_transpose_embedding_input_nobag. */
size_t mx_tbe_transpose_nobag_workspace_bytes(int64_t N, int32_t T, int32_t total_hash_size_bits);

/* Serves fbgemm::transpose_embedding_input with nobag = true (sequence
 * lookups): as mx_tbe_transpose_embedding_input, except that each position
 * is its own occurrence and its info is int64, l * T + t (l the position, t
 * its table).  Needs offsets[0] = 0 and offsets[T*B] = N, as upstream. */
int mx_tbe_transpose_embedding_input_nobag(
    const int64_t* hash_size_cumsum, int32_t T, int64_t B, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    int64_t* linear_indices, int64_t* sorted_linear_indices, int64_t* infos_sorted,
    int64_t* sorted_linear_indices_run, int32_t* run_lengths, int32_t* num_runs,
    int32_t* cumulative_run_lengths, void* workspace, size_t workspace_bytes, void* stream);

/* Random state of a stochastic-rounding update, in the shape of torch's
 * Philox state: eager calls pass the seed and offset as values; a call made
 * under graph capture passes device pointers that the kernel reads when it
 * runs (offset = *offset_dev + offset), so every replay draws new bits. */
typedef struct mx_rng_state {
  uint64_t seed;
  uint64_t offset;
  const int64_t* seed_dev;    /* non-NULL: the seed is read from here */
  const int64_t* offset_dev;  /* non-NULL: the offset is *offset_dev + offset */
} mx_rng_state;

/* Workspace needed by mx_tbe_backward_rowwise_adagrad(_vbe). */
size_t mx_tbe_backward_workspace_bytes(int64_t N, int32_t total_hash_size_bits, int32_t max_D);

/* Serves fbgemm::split_embedding_backward_codegen_rowwise_adagrad_{unweighted,
 * weighted}_exact_cuda (the backward of
 * split_embedding_codegen_lookup_rowwise_adagrad_function).
 * For each distinct (t, i) touched by the batch:
 *   g      = sum over its occurrences (sorted order) of grad_output[b, D_t slice],
 *            each term scaled by 1.0f/L of its bag (MEAN) and then by its
 *            per-sample weight (indice_weights [N], weighted lookups; NULL otherwise)
 *   s      = g + weight_decay * w (mode 1, L2) or g
 *   h     += (sum_d s_d^2) / D_t
 *   m      = learning_rate / (sqrtf(h) + eps)
 *   c      = 1 (mode 0), 1 - m*weight_decay (mode 1), 1 - learning_rate*weight_decay (mode 2)
 *   w      = fmaf(-m, g, c * w)
 * weights (fp32, or fp16 with weights_ty MX_SPARSE_FP16: w read as fp32, the
 * new value rounded to fp16 -- to nearest even, or stochastically when
 * stochastic_rounding != 0: |w| plus a uniform random amount below fp16's
 * last place, then truncated, the random bits a hash of (rng, element); rng
 * may be NULL when stochastic_rounding is 0)
 * and momentum1 (fp32 [E_t] per table at momentum1_offsets[t]) are updated
 * in place; no atomics, deterministic for a given random state.  Every
 * kernel of the call runs on `stream` (also under graph capture). */
int mx_tbe_backward_rowwise_adagrad(
    void* weights, int32_t weights_ty, const int64_t* weights_offsets, const int32_t* D_offsets,
    int32_t T, int64_t B, int32_t max_D, const int64_t* hash_size_cumsum, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    int32_t pooling_mode, const float* indice_weights, const float* grad_output, int64_t total_D,
    float* momentum1, const int64_t* momentum1_offsets, float learning_rate, float eps,
    float weight_decay, int32_t weight_decay_mode, int32_t stochastic_rounding,
    const mx_rng_state* rng, void* workspace, size_t workspace_bytes, void* stream);

/* Serves fbgemm::split_embedding_backward_codegen_rowwise_adagrad_{unweighted,
 * weighted}_exact_vbe_cuda: mx_tbe_backward_rowwise_adagrad over total_B
 * flattened bags (B_offsets [T+1], vbe_row_output_offsets and vbe_b_t_map
 * [total_B] from mx_generate_vbe_metadata, b < max_B); grad_output is the flat
 * VBE gradient, the row of bag (t, b) at vbe_row_output_offsets[B_offsets[t] + b]. */
int mx_tbe_backward_rowwise_adagrad_vbe(
    void* weights, int32_t weights_ty, const int64_t* weights_offsets, const int32_t* D_offsets,
    int32_t T, int64_t max_B, int32_t max_D, const int64_t* hash_size_cumsum,
    int32_t total_hash_size_bits, const void* indices, const void* offsets, int32_t index_bytes,
    int64_t N, int32_t pooling_mode, const float* indice_weights, const float* grad_output,
    int64_t total_B, const int32_t* B_offsets, const int64_t* vbe_row_output_offsets,
    const int32_t* vbe_b_t_map, int32_t info_B_num_bits, float* momentum1,
    const int64_t* momentum1_offsets, float learning_rate, float eps, float weight_decay,
    int32_t weight_decay_mode, int32_t stochastic_rounding, const mx_rng_state* rng,
    void* workspace, size_t workspace_bytes, void* stream);

/* Workspace needed by mx_tbe_backward_rowwise_adagrad_nobag. */
size_t mx_tbe_backward_nobag_workspace_bytes(int64_t N, int32_t T, int32_t total_hash_size_bits,
                                             int32_t D);

/* Serves fbgemm::split_embedding_nobag_backward_codegen_rowwise_adagrad_
 * unweighted_exact_cuda (the PoolingMode NONE backward): every table has
 * width D and grad_output is [N, D], row l the gradient of position l.  For
 * each distinct (t, i): g = the sum of its positions' gradient rows in sorted
 * (position) order, then the update of mx_tbe_backward_rowwise_adagrad.
 * Needs offsets[0] = 0 and offsets[T*B] = N, as upstream. */
int mx_tbe_backward_rowwise_adagrad_nobag(
    void* weights, int32_t weights_ty, const int64_t* weights_offsets, int32_t T, int64_t B,
    int32_t D, const int64_t* hash_size_cumsum, int32_t total_hash_size_bits,
    const void* indices, const void* offsets, int32_t index_bytes, int64_t N,
    const float* grad_output, float* momentum1, const int64_t* momentum1_offsets,
    float learning_rate, float eps, float weight_decay, int32_t weight_decay_mode,
    int32_t stochastic_rounding, const mx_rng_state* rng, void* workspace,
    size_t workspace_bytes, void* stream);

/* Serves fbgemm::split_embedding_codegen_grad_indice_weights_cuda: the gradient
 * of a weighted lookup's per-sample weights,
 *   grad_indice_weights[l] = sum_d grad_output[b, D_off[t] + d] * W_t[indices[l], d]
 * (MEAN: times 1.0f/L), 0 for tables with feature_requires_grad[t] == 0
 * (feature_requires_grad may be NULL: every table); weights fp32 or fp16
 * (weights_ty) as in mx_tbe_forward. */
int mx_tbe_grad_indice_weights(const float* grad_output, int64_t total_D, const void* weights,
                               int32_t weights_ty, const int64_t* weights_offsets,
                               const int32_t* D_offsets, int32_t T, int64_t B, int32_t max_D,
                               const void* indices,
                               const void* offsets, int32_t index_bytes, int32_t pooling_mode,
                               const int32_t* feature_requires_grad, float* grad_indice_weights,
                               void* stream);

/* VBE variant of mx_tbe_grad_indice_weights (fbgemm's
 * split_embedding_codegen_grad_indice_weights_vbe_cuda): grad_output is the
 * flat VBE gradient, bag i reads its row at vbe_row_output_offsets[i]. */
int mx_tbe_grad_indice_weights_vbe(
    const float* grad_output, const void* weights, int32_t weights_ty,
    const int64_t* weights_offsets, const int32_t* D_offsets, int32_t T, int64_t total_B,
    int32_t max_D, const void* indices, const void* offsets, int32_t index_bytes,
    int32_t pooling_mode, const int64_t* vbe_row_output_offsets, const int32_t* vbe_b_t_map,
    int32_t info_B_num_bits, const int32_t* feature_requires_grad, float* grad_indice_weights,
    void* stream);

/* ---- index validation ---------------------------------------------------- */

/* Serves fbgemm::bounds_check_indices (the check callers run before a TBE
 * lookup).  indices [N] and offsets [T*B+1] share one integer type and are
 * repaired in place:
 *   - offsets become o'[i] = max_{j<=i} clamp(o[j], 0, N) (in range and
 *     non-decreasing, so bags never overlap);
 *   - every index of bag (t, b), positions [o'[t*B+b], o'[t*B+b+1]),
 *     outside [0, rows_per_table[t]) becomes 0;
 *   - each repaired entry adds one to *warning (device int64).
 * mode FATAL only counts (nothing is repaired; the caller raises on a
 * non-zero count), WARNING and IGNORE repair and count, NONE does nothing.
 * Workspace: mx_bounds_check_workspace_bytes(T, B). */
size_t mx_bounds_check_workspace_bytes(int32_t T, int64_t B);
int mx_bounds_check_indices(const int64_t* rows_per_table, int32_t T, int64_t B, void* indices,
                            void* offsets, int32_t index_bytes, int64_t N, int32_t mode,
                            int64_t* warning, void* workspace, size_t workspace_bytes,
                            void* stream);

/* No counterpart in the reference or in fbgemm_gpu: mx_bounds_check_indices
 * for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, semantics and
 * results, without the workspace: the scratch (at most 1024 per-tile offset
 * maxima, 4 KiB) is a static device array of the library, one per device,
 * held until the process ends.  Every batch fits it (tiles widen with the
 * batch, at most 1024 of them); a scratch need above 4 KiB would return
 * MX_EWORKSPACE instead of running.  Calls that overlap on one device
 * (two streams, or two threads, at once) share that array and race; calls
 * in stream order do not.  Nothing is allocated. */
int mx_bounds_check_indices_noalloc(const int64_t* rows_per_table, int32_t T, int64_t B,
                                    void* indices, void* offsets, int32_t index_bytes, int64_t N,
                                    int32_t mode, int64_t* warning, void* stream);

/* VBE variant (fbgemm's B_offsets argument): total_B bags, bag i of table t
 * for B_offsets[t] <= i < B_offsets[t+1]; workspace from
 * mx_bounds_check_workspace_bytes_vbe(total_B). */
size_t mx_bounds_check_workspace_bytes_vbe(int64_t total_B);
int mx_bounds_check_indices_vbe(const int64_t* rows_per_table, int32_t T, int64_t total_B,
                                const int32_t* B_offsets, void* indices, void* offsets,
                                int32_t index_bytes, int64_t N, int32_t mode, int64_t* warning,
                                void* workspace, size_t workspace_bytes, void* stream);

/* ---- rowwise quantization codecs ---------------------------------------- */

/* Serve fbgemm::FloatToFused8BitRowwiseQuantized / HalfToFused8BitRowwiseQuantized
 * and fbgemm::Fused8BitRowwiseQuantizedToFloat / ...ToHalf.
 * Fused 8-bit row: D codes, fp32 scale, fp32 bias (D + 8 bytes);
 * scale = (max - min) / 255, bias = min, q = rint((x - min) * 255 / (max - min + 1e-8));
 * dequantized value = fma(q, scale, bias).  in/out dtype: MX_DTYPE_F32 or F16. */
int mx_quantize_fused8bit_rowwise(const void* in, int32_t in_dtype, int64_t rows, int64_t D,
                                  uint8_t* out, void* stream);
int mx_dequantize_fused8bit_rowwise(const uint8_t* in, int64_t rows, int64_t D, void* out,
                                    int32_t out_dtype, void* stream);

/* Serve fbgemm::FloatToFusedNBitRowwiseQuantizedSBHalf / HalfTo... and
 * fbgemm::FusedNBitRowwiseQuantizedSBHalfToFloat / ...ToHalf (bit_rate 2, 4, 8).
 * Row: ceil(D*bit_rate/8) code bytes (element 0 in the lowest bits), fp16
 * scale, fp16 bias; bias = half(min), scale = half((max - bias) / (2^b - 1))
 * (1 for a zero range or an underflowing scale), q = clamp(rint((x - bias) *
 * (1/scale)), 0, 2^b - 1); dequantized value = fma(q, scale, bias). */
int mx_quantize_fused_nbit_rowwise(const void* in, int32_t in_dtype, int64_t rows, int64_t D,
                                   int32_t bit_rate, uint8_t* out, void* stream);
int mx_dequantize_fused_nbit_rowwise(const uint8_t* in, int64_t rows, int64_t D,
                                     int32_t bit_rate, void* out, int32_t out_dtype,
                                     void* stream);

/* Serve fbgemm::FloatToHFP8Quantized and fbgemm::HFP8QuantizedToFloat: fp32
 * <-> hfp8 codes, one byte per element (sign, ebits exponent bits, 7 - ebits
 * mantissa bits, bias exponent_bias, subnormals at exponent field 0; FBGEMM's
 * FloatToFloat8_ref / Float8ToFloat_ref).  Encoding clamps |x| to max_pos
 * (and to the largest code), then rounds to the nearest code, ties to even;
 * NaN encodes as the clamp.  1 <= ebits <= 7, 0 <= exponent_bias <= 120. */
int mx_float_to_hfp8(const float* in, int64_t n, int32_t ebits, int32_t exponent_bias,
                     float max_pos, uint8_t* out, void* stream);
int mx_hfp8_to_float(const uint8_t* in, int64_t n, int32_t ebits, int32_t exponent_bias,
                     float* out, void* stream);

/* ---- sparse-feature helpers ------------------------------------------------ */

/* Workspace needed by mx_cumsum over n elements of elem_bytes (4 or 8). */
size_t mx_cumsum_workspace_bytes(int64_t n, int32_t elem_bytes);

/* Serves fbgemm::asynchronous_exclusive_cumsum (kind 0), asynchronous_
 * inclusive_cumsum (1) and asynchronous_complete_cumsum (2: n + 1 outputs,
 * out[0] = 0; with rows > 1, x is [rows, n] and each row gets its own n + 1).
 * int32 or int64 (elem_bytes 4 or 8) in and out, two's complement
 * wrap-around; exact.  rows > 1 needs kind 2 and no workspace. */
int mx_cumsum(const void* in, int32_t elem_bytes, int64_t rows, int64_t n, int32_t kind,
              void* out, void* workspace, size_t workspace_bytes, void* stream);

/* fbgemm::permute_2D_sparse_data, step 1: permuted_lengths [T_out, B] with
 * row f = lengths row permute[f] (int32 permute; a feature outside [0, T)
 * gets zero lengths).  lengths int32 or int64 (length_bytes). */
int mx_permute_2d_lengths(const int32_t* permute, int64_t T_out, const void* lengths,
                          int32_t length_bytes, int32_t T, int64_t B, void* permuted_lengths,
                          void* stream);

/* fbgemm::permute_2D_sparse_data, step 2: bag (f, b) of the output, at
 * output_offsets[f*B + b] (the complete cumsum of the permuted lengths), is a
 * copy of the input bag (permute[f], b) at input_offsets[permute[f]*B + b]
 * (the complete cumsum of the lengths); weights (fp32, may be NULL) travel
 * with their indices.  in_len = the number of indices (and weights), out_len
 * = output_offsets[T_out*B]; lengths that disagree with either stop the copy
 * of their bag at the array's end. */
int mx_permute_2d_data(const int32_t* permute, int64_t T_out, int32_t T, int64_t B,
                       const void* input_offsets, const void* output_offsets,
                       int32_t offset_bytes, const void* indices, int32_t index_bytes,
                       int64_t in_len, const float* weights, int64_t out_len,
                       void* permuted_indices, float* permuted_weights, void* stream);

/* Serves fbgemm::offsets_range: out[j] = j - offsets[i] for j in segment i =
 * [offsets[i], offsets[i + 1]) (the last segment ends at range_size); out
 * [range_size], int32 or int64 like offsets. */
int mx_offsets_range(const void* offsets, int32_t index_bytes, int64_t nseg, int64_t range_size,
                     void* out, void* stream);

/* Serves fbgemm::expand_into_jagged_permute: for output feature t,
 * out[output_offsets[t] + j] = input_offsets[permute[t]] + j, j below its
 * length (output_offsets[t+1] - output_offsets[t]; output_size for the last
 * when output_offsets has T entries). */
int mx_expand_into_jagged_permute(const int32_t* permute, int64_t T, const void* input_offsets,
                                  int64_t input_numel, const void* output_offsets,
                                  int64_t output_numel, int32_t index_bytes, int64_t output_size,
                                  void* out, void* stream);

/* ---- TBE nbit inference forward ---------------------------------------- */

/* Padded size in bytes of one row of a table of type `ty` and dim D:
 * round_up(unpadded, row_alignment) with unpadded FP32 4D, FP16 2D,
 * INT8 D+4, INT4 D/2+4, INT2 D/4+4; -1 for an unknown type. */
int64_t mx_nbit_row_bytes(int32_t ty, int32_t D, int32_t row_alignment);

/* Serves fbgemm::int_nbit_split_embedding_codegen_lookup_function, DEVICE
 * placement.
 *   dev_weights     uint8, row (t, i) at weights_offsets[t] + i*row_bytes(t)
 *   weights_tys     uint8 [T] SparseType per table
 *   D_offsets       int32 [T+1]
 *   max_*_D         the host-side maxima the upstream op receives; a type
 *                   whose max is 0 is not launched
 *   INT8/INT4/INT2 rows begin with fp16 scale then fp16 bias; INT4 holds
 *   the even element in the low nibble.  value = scale*q + bias (fp32).
 *   Codes fill whole bytes: every INT4 table's D is even and every INT2
 *   table's D a multiple of 4 (checked on the maxima; EINVAL otherwise).
 *   FP8 rows are D hfp8 codes (sign, fp8_exponent_bits exponent bits,
 *   7 - fp8_exponent_bits mantissa bits, bias fp8_exponent_bias, subnormals
 *   at exponent field 0; fbgemm's Float8ToFloat_ref); max_float8_D > 0 needs
 *   1 <= fp8_exponent_bits <= 7 and 0 <= fp8_exponent_bias <= 120.
 *   output_dtype    MX_SPARSE_FP32, MX_SPARSE_FP16 (round to nearest even) or
 *                   MX_SPARSE_BF16 (to nearest, ties away from zero, as
 *                   FBGEMM's CPU kernels write bf16)
 *   out             [B, total_D] */
int mx_nbit_forward(const uint8_t* dev_weights, const int64_t* weights_offsets,
                    const uint8_t* weights_tys, const int32_t* D_offsets, int32_t T, int64_t B,
                    int32_t max_int2_D, int32_t max_int4_D, int32_t max_int8_D,
                    int32_t max_float16_D, int32_t max_float32_D, const void* indices,
                    const void* offsets, int32_t index_bytes, int32_t pooling_mode,
                    const float* indice_weights, int32_t output_dtype, int32_t row_alignment,
                    int32_t max_float8_D, int32_t fp8_exponent_bits, int32_t fp8_exponent_bias,
                    void* out, int64_t total_D, void* stream);

/* Serves fbgemm::int_nbit_split_embedding_codegen_lookup_function with
 * pooling_mode MX_POOL_NONE (fbgemm's int_nbit_split_embedding_nobag_codegen_
 * forward_unweighted_cuda): D is the largest max_*_D and position l of bag
 * (t, b) writes its own dequantized row, out[l, :], out [N, D].  An
 * INT8/INT4/INT2 element is fmaf(scale, q, bias); FP32, FP16 and FP8 elements
 * are the stored values; then the output type of mx_nbit_forward.  A table
 * whose D is not D, or that mx_nbit_forward could not serve, has its
 * positions written as zeros and is reported in MX_STATUS_NBIT_TABLE;
 * positions outside every bag are written as zeros. */
int mx_nbit_forward_nobag(const uint8_t* dev_weights, const int64_t* weights_offsets,
                          const uint8_t* weights_tys, const int32_t* D_offsets, int32_t T,
                          int64_t B, int32_t max_int2_D, int32_t max_int4_D, int32_t max_int8_D,
                          int32_t max_float16_D, int32_t max_float32_D, const void* indices,
                          const void* offsets, int32_t index_bytes, int64_t N,
                          int32_t output_dtype, int32_t row_alignment, int32_t max_float8_D,
                          int32_t fp8_exponent_bits, int32_t fp8_exponent_bias, void* out,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MX_FBGEMM_H */
