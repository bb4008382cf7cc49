/*
 * C ABI of the MI355X (gfx950) packed-weight matrix-vector library,
 * libqmv_hip.so.
 *
 * Only plain C types cross this boundary: pointers, sizes, and the
 * QmvTensorView descriptor below. A HIP stream is passed as void* (a
 * hipStream_t; NULL selects the calling thread's own stream for host-pointer
 * calls and the legacy default stream for device calls).
 *
 * Every function that returns int returns 1 on success and 0 on failure,
 * like the reference's packed matvec (src/quantized_matvec.h:26-31). On
 * failure qmv_last_error() returns a message for the calling thread. Output
 * buffers are left untouched when validation fails; after a failed device
 * operation their contents are unspecified.
 *
 * Thread safety: all entry points may be called concurrently from several
 * host threads on the same registered weights (the reference's sessions do
 * this, include/engine_api.h:10-17). A host-pointer call checks a context (a
 * HIP stream with its staging buffers and split-K workspace) out of a
 * per-device pool for its duration; any thread may use any context, so a
 * session may move between OS threads from call to call.
 */
#ifndef QMV_HIP_H
#define QMV_HIP_H

#include <stdint.h>
#include "qmv_formats.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Borrowed descriptor of one packed 2-D GGUF tensor. Field for field the same
 * layout and meaning as the reference's GgufQuantizedTensorView
 * (src/gguf_reader.h:31-40): dimensions[0] = columns (K), dimensions[1] =
 * rows (N); data is a host pointer with byte alignment only.
 */
typedef struct QmvTensorView {
    const unsigned char *data;
    uint32_t ggml_type;
    uint32_t dimension_count;
    uint64_t dimensions[4];
    uint64_t element_count;
    uint64_t block_elements;
    uint64_t block_bytes;
    uint64_t block_count;
} QmvTensorView;

/* ---- Drop-in host-pointer entry points -------------------------------- */

/*
 * output[N] = W[N,K] * input[K]. Replaces quantized_tensor_matvec_f32
 * (src/quantized_matvec.h:32-38, src/quantized_matvec.cpp:86-162). Same
 * argument rules: input_count == dimensions[0], output_count ==
 * dimensions[1], type in {Q5_0, Q8_0, Q4_K, Q6_K}, consistent block layout.
 * The packed tensor is uploaded to HBM on first use and cached (keyed by data
 * pointer, type and shape, guarded by a content fingerprint: every byte of
 * tensors up to 64 KiB, 64 sampled words of larger ones); input and output are
 * host buffers. The packed bytes must not change while they are cached: after
 * editing them in place, or before freeing them, call qmv_release_tensor.
 */
int qmv_tensor_matvec_f32(const QmvTensorView *matrix, const float *input,
                          int input_count, float *output, int output_count);

/*
 * outputs[B,N] = inputs[B,K] * W^T for token-major batches. Replaces
 * quantized_tensor_matmul_f32 (src/quantized_matvec.h:43-50,
 * src/quantized_matvec.cpp:164-224). batch_count must be positive; each
 * pass over the weights serves up to QMV_MAX_BATCH positions (on the
 * matrix cores).
 */
int qmv_tensor_matmul_f32(const QmvTensorView *matrix, const float *inputs,
                          int input_count, int batch_count, float *outputs,
                          int output_count);

#define QMV_MAX_BATCH 32

/*
 * Upload a packed tensor now (at model load) instead of on first use. No
 * reference counterpart: the reference reads weights straight from its mmap
 * (src/gguf_reader.cpp:695-697). Registration alone does not size the
 * staging or the split-K workspace of the host-pointer calls;
 * qmv_reserve_calls does.
 */
int qmv_register_tensor(const QmvTensorView *matrix);

/*
 * Register the tensor and pre-size, for host-pointer matvec/matmul calls on
 * it with 1..max_batch positions, everything those calls would otherwise
 * allocate on first use: the input and output staging (pinned and device) and
 * the split-K workspace, in every context of the current device's pool (one
 * is created if the pool has none). Called for every weight from the engine's
 * state initialisation (inference_state_init), it makes the reference's
 * contracts hold on whatever OS thread later runs the session: a forward pass
 * allocates nothing after init (include/engine.h:84-85) and the matvec itself
 * allocates nothing (src/quantized_matvec.h:24). The first reservation closes
 * the pool: from then on a host-pointer call that finds every context in use
 * waits for one to be returned instead of creating another. A larger batch
 * than reserved, or a later change of the launch tuning, may allocate again.
 */
int qmv_reserve_calls(const QmvTensorView *matrix, int max_batch);

/*
 * Declare how many host-pointer calls may run at once on the current device
 * (the engine's number of concurrent sessions, server/pool.go:150): the pool
 * gets at least `count` contexts (1..1024), each sized like every
 * qmv_reserve_calls so far and later, and is closed as above. Call it at
 * state initialisation, before or after the qmv_reserve_calls calls. No
 * reference counterpart (the reference opens an OpenMP team per call,
 * src/quantized_matvec.cpp:152).
 */
int qmv_reserve_contexts(int count);

/*
 * Number of device allocations, pinned host allocations and stream
 * creations the library has made in this process (a test and diagnostic
 * counter for the contract above).
 */
unsigned long long qmv_allocation_count(void);

/*
 * Drop the device copies of every tensor whose host data pointer is data
 * (call before the reference's gguf_close, src/gguf_reader.h:136-137).
 * Returns the number of tensors released.
 */
int qmv_release_tensor(const unsigned char *data);
void qmv_release_all(void);

/*
 * Decode rows [first_row, first_row + row_count) of a packed tensor on the
 * GPU into output[row_count, K] (host memory). Bit-identical to the
 * reference's per-block decoders q8_0/q5_0/q4_k/q6_k_dequantize_block
 * (src/quantization.cpp:54-67,161-184,380-409,588-615) applied row by row.
 */
int qmv_dequantize_rows_f32(const QmvTensorView *matrix, int first_row,
                            int row_count, float *output);

/*
 * Greedy argmax of host logits computed on the GPU. Same contract as
 * sampler_greedy_sample (src/sampler.cpp:29-51): largest value, lowest id
 * on exact ties, and failure (return 0, *token_id = -1) on any NaN/Inf or
 * invalid argument.
 */
int qmv_greedy_sample_f32(const float *logits, int vocab_size, int *token_id);

/* ---- Device-resident entry points ------------------------------------- */

/* Opaque handle to a tensor resident in HBM in the tiled device layout. */
typedef struct QmvDeviceTensor *qmv_device_tensor;

/*
 * Upload a packed host tensor into a new device tensor (validated like the
 * matvec). The handle is independent of the host cache above and of the host
 * data, which may be freed afterwards.
 */
int qmv_device_tensor_create(const QmvTensorView *matrix,
                             qmv_device_tensor *out_tensor);
void qmv_device_tensor_destroy(qmv_device_tensor tensor);

/* Shape and storage of a device tensor; any output pointer may be NULL.
 * device_bytes counts every device copy: the tiled layout, plus the GGUF
 * bytes that small Q4_K tensors keep for the row-major single-position
 * kernel. */
int qmv_device_tensor_info(qmv_device_tensor tensor, int *rows, int *columns,
                           uint32_t *ggml_type, uint64_t *packed_bytes,
                           uint64_t *device_bytes);

/*
 * d_outputs[B,N] = d_inputs[B,K] * W^T with device pointers, enqueued on
 * stream without host synchronisation (1 <= batch_count <= QMV_MAX_BATCH).
 * Batches of 9 to 32 positions (prefill chunks larger than the reference's
 * 8, src/qwen2_internal.h:7) read the weights once, on the matrix cores.
 */
int qmv_device_matvec_f32(qmv_device_tensor tensor, const float *d_inputs,
                          int batch_count, float *d_outputs, void *stream);

/*
 * Several device tensors with the same column count and one shared input
 * (q/k/v, or gate/up, of one layer) in a single launch. d_outputs[i] receives
 * tensors[i]'s rows. count <= QMV_MAX_GROUP.
 */
#define QMV_MAX_GROUP 8
int qmv_device_matvec_group_f32(const qmv_device_tensor *tensors, int count,
                                const float *d_inputs, int batch_count,
                                float *const *d_outputs, void *stream);

/*
 * qmv_device_matvec_group_f32 without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The split-K workspace is a fixed array in device memory of
 * QMV_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends: arrival
 * counters in its first QMV_NOALLOC_COUNTER_BYTES (one 128-byte line per
 * tile whose K is split, so at most 4096 such tiles per launch) and partial
 * sums in the rest (31.5 MiB, 8,257,536 floats). A call whose
 * launches would need more is rejected (return 0, nothing launched); the
 * decode and prefill shapes of a 7B model fit (for example a 151936 x 3584
 * vocabulary projection for one position: 455,808 floats, or one 18944 x
 * 3584 projection for 32 positions: 4,243,456 floats); the vocabulary
 * projection for 8 positions (8.5 M floats) does not. The
 * counters are cleared by a fill kernel before each launch (no memset node).
 * All calls on one GPU share its array: calls that overlap in time on one
 * GPU (other streams, other threads) race and must be serialised by the
 * caller. Results are bit-identical to qmv_device_matvec_group_f32.
 */
#define QMV_NOALLOC_SCRATCH_BYTES (32u << 20)
#define QMV_NOALLOC_COUNTER_BYTES (512u << 10)
int qmv_device_matvec_group_noalloc_f32(const qmv_device_tensor *tensors,
                                        int count, const float *d_inputs,
                                        int batch_count,
                                        float *const *d_outputs, void *stream);

/*
 * Grouped matvec with an addend fused into the store: for each tensor i,
 * d_outputs[i][b*N_i + r] = (W_i x_b)[r] + d_addends[i][b*addend_strides[i] + r]
 * (the fp32 sum of the row result and the addend, as the reference's separate
 * tensor_add_f32, src/tensor.cpp:5-23, computes it). addend_strides[i] = 0
 * adds one vector to every position: the q/k/v biases of
 * qwen2_layer_project / _project_batch (src/qwen2_architecture.cpp:714-733,
 * 763-807). addend_strides[i] = N_i with d_addends[i] == d_outputs[i] adds
 * the residual in place: x += W h after the attention output and FFN down
 * projections (src/qwen2_architecture.cpp:1363-1374, 1450-1463). A null
 * d_addends[i] stores the plain product. Other overlaps of an addend with an
 * output are rejected. Stride otherwise >= N_i.
 */
int qmv_device_matvec_add_group_f32(const qmv_device_tensor *tensors, int count,
                                    const float *d_inputs, int batch_count,
                                    const float *const *d_addends,
                                    const int *addend_strides,
                                    float *const *d_outputs, void *stream);

/*
 * FFN gate and up projections of one shared input fused with SwiGLU:
 * d_outputs[b*N + r] = up_b[r] * silu(gate_b[r]), silu(g) = g / (1 + exp(-g)),
 * the element rule of transformer_swiglu_f32 (src/transformer_ops.cpp:163-
 * 176) applied to the two projections (src/qwen2_architecture.cpp:1399-1434).
 * One launch; neither projection is stored. gate and up share type, shape
 * and device.
 */
int qmv_device_matvec_swiglu_f32(qmv_device_tensor gate, qmv_device_tensor up,
                                 const float *d_inputs, int batch_count,
                                 float *d_outputs, void *stream);

/*
 * RMSNorm of the input fused with the grouped projection that consumes it:
 * the attention and FFN norms of the reference's decode step
 * (tensor_rms_norm_f32, src/tensor.cpp:99-136, called before the q/k/v and
 * the gate/up projections, src/qwen2_architecture.cpp:1241-1260, 1376-1397)
 * followed by qmv_device_matvec_add_group_f32 / qmv_device_matvec_swiglu_f32
 * on the normalised vector. No reference counterpart as one call; it replaces
 * that pair of calls. For each position b,
 *   h_b = (x_b / sqrt(mean(x_b^2) + epsilon)) * d_norm_weight
 * and the outputs are those of the plain entry points on h. With one
 * position and Q4_K tensors whose rows hold at most 16 super-blocks (a
 * Qwen2.5 hidden size), the norm runs inside the row-major projection
 * launch: every workgroup normalises the whole input in LDS, so no h is
 * written and one launch is saved. Otherwise a norm launch writes h to
 * d_normed (batch_count x K floats, clear of the input, the weights and the
 * outputs) and the projection reads it; after the call the contents of
 * d_normed are unspecified. Results are within the row tolerance of the
 * reference's norm followed by its matvec either way. Argument rules: those
 * of qmv_device_rms_norm_f32 (epsilon <= 0 fails) and of the plain entry
 * point; d_addends may be NULL for plain stores.
 */
int qmv_device_rms_norm_matvec_add_group_f32(const qmv_device_tensor *tensors,
                                             int count, const float *d_input,
                                             const float *d_norm_weight,
                                             float epsilon, int batch_count,
                                             const float *const *d_addends,
                                             const int *addend_strides,
                                             float *const *d_outputs,
                                             float *d_normed, void *stream);
int qmv_device_rms_norm_matvec_swiglu_f32(qmv_device_tensor gate,
                                          qmv_device_tensor up,
                                          const float *d_input,
                                          const float *d_norm_weight,
                                          float epsilon, int batch_count,
                                          float *d_output, float *d_normed,
                                          void *stream);

/*
 * Vocabulary projection fused with greedy sampling: d_logits[N] = W x for one
 * position, and in the same launch d_result[0] = the greedy token (largest
 * logit, lowest id on ties) or -1, d_result[1] = 1 if every logit was finite,
 * else 0 (the contract of src/sampler.cpp:29-51, whose caller runs after the
 * output projection, src/qwen2_architecture.cpp:1504-1523). The token is the
 * argmax of exactly the logits written.
 */
int qmv_device_matvec_argmax_f32(qmv_device_tensor tensor, const float *d_input,
                                 float *d_logits, int *d_result, void *stream);

/*
 * Embedding lookup: d_output[i, K] = row d_token_ids[i] of the tensor decoded
 * to fp32 (i < count <= 65535), bit-identical to the reference's per-row
 * decode qwen2_decode_quantized_embedding_row (src/qwen2_architecture.cpp:
 * 375-456) for each id. The ids are read on the device (for example the token
 * just written by qmv_device_matvec_argmax_f32), so an id outside [0, N)
 * cannot be rejected before the launch: its output row is filled with NaN,
 * and if d_status is not NULL, d_status[0] is set to 1 when every id was in
 * range and to 0 otherwise, so the caller can fail the step as the reference
 * does for an out-of-range token (src/qwen2_architecture.cpp:384-393).
 */
int qmv_device_embed_rows_f32(qmv_device_tensor tensor, const int *d_token_ids,
                              int count, float *d_output, int *d_status,
                              void *stream);

/* Device decode of rows into d_output[row_count, K] (see qmv_dequantize_rows_f32). */
int qmv_device_dequantize_f32(qmv_device_tensor tensor, int first_row,
                              int row_count, float *d_output, void *stream);

/*
 * RMSNorm of batch_count device vectors of length elements each:
 * d_output[b*L + i] = (x[i] / sqrt(mean(x^2) + epsilon)) * d_weight[i] with
 * x = d_input + b*L, the contract of tensor_rms_norm_f32 (src/tensor.cpp:
 * 99-136; the decode step's attention and FFN norms, src/qwen2_architecture.
 * cpp:1241-1260, 1376-1397, and the output norm). Same argument rules: null
 * pointers, length <= 0 or epsilon <= 0 fail. The sum of squares is taken
 * in a fixed parallel order, so it differs from the reference's sequential
 * sum in the last bits (well inside 2e-5 relative). d_output may be d_input
 * itself; other overlaps fail.
 */
int qmv_device_rms_norm_f32(const float *d_input, const float *d_weight,
                            int length, int batch_count, float epsilon,
                            float *d_output, void *stream);

/*
 * Greedy argmax over device logits. Writes d_result[0] = token id (or -1)
 * and d_result[1] = 1 if every logit was finite, else 0.
 */
int qmv_device_greedy_argmax_f32(const float *d_logits, int vocab_size,
                                 int *d_result, void *stream);

/* ---- Library state ------------------------------------------------------ */

/* Message describing the calling thread's most recent failure ("" if none). */
const char *qmv_last_error(void);

/* Select the HIP device used by later calls from any thread (default 0). */
int qmv_set_device(int ordinal);

/* Number of HIP devices visible to the process (0 when none or no driver). */
int qmv_device_count(void);

/*
 * Launch-plan tuning (process-wide; 0 keeps the automatic choice for any
 * argument). A launch gives each workgroup one 64-row tile and a contiguous
 * range of K-units, processed by waves_per_group waves of units_per_wave
 * units each (default: 1 unit and 4 waves; for single-position launches 6
 * waves over rows of 32 or more K-units, 5 over more than 16384 units in all,
 * 2 over 2049..16384 units, and one wave per unit with no K split over rows
 * of at most 8 units in launches of at most 2048 units; batches run half
 * units, except on the matrix cores over rows of 32 or more units); a tile's
 * K is split across workgroups as far as that requires, and the last split to
 * finish adds the partials in split order.
 * target_waves, if set, instead grows the units per wave until about that
 * many waves cover the launch. Q4_K and Q6_K batches of at least
 * mfma_min_batch positions (default 7 for Q4_K, 8 for Q6_K; a value above
 * QMV_MAX_BATCH turns it off, and then batches run in launches of 8 on the
 * VALU path) run on the matrix cores, and so do Q5_0 launches of 5 to 8
 * positions and Q8_0 launches of 4 to 8 (QMV_Q5_MFMA_MIN_BATCH /
 * QMV_Q8_MFMA_MIN_BATCH in the environment; 0 turns them off). Defaults may also come from the
 * QMV_TARGET_WAVES / QMV_UNITS_PER_WAVE / QMV_WAVES_PER_GROUP /
 * QMV_MFMA_MIN_BATCH environment variables. While target_waves,
 * units_per_wave or waves_per_group is set, single-position Q4_K launches use
 * the tiled plan too (not the row-major kernel). Any setting stays within the row
 * tolerance: the plan only changes the summation order, and a given plan
 * always sums in the same order.
 */
void qmv_set_launch_tuning(int target_waves, int units_per_wave,
                           int waves_per_group, int mfma_min_batch);

/*
 * Row-major kernels for single-position Q4_K and Q6_K launches
 * (process-wide; no reference counterpart). A Q4_K tensor with at most 128
 * super-blocks per row whose tiled layout holds at most 2048 (64-row tile,
 * 256-weight unit) pairs, or of any size with at most 16 super-blocks per
 * row, keeps its GGUF bytes on the device as well while enable != 0 (the
 * default), and a Q6_K tensor with 17 to 128 super-blocks per row keeps a
 * row-major copy in chunks of 16 super-blocks (210 bytes per super-block,
 * rows padded to 16 bytes); their single-position launches read those (for
 * a Qwen2.5-7B-shaped model: q, k, v, o, gate and up, 92.9 MB per layer,
 * and down, 55.7 MB: 4.16 GB in all, +100% over the packed weights, 2.9% of
 * one GPU's HBM). enable = 0 stops both for launches planned and tensors
 * uploaded afterwards: memory-bound callers set it before loading the
 * weights. rows (1, 2 or 4; other values: 2) is how many rows each 64-lane
 * row segment of the Q4_K kernel takes in launches of at most 2048 pairs
 * (larger launches take 4, or 2 with the fused SwiGLU). QMV_ROWDOT=0 /
 * QMV_ROWDOT_ROWS in the environment set the same at start-up, and
 * QMV_ROWDOT_Q6K=0 keeps Q6_K tensors tiled only. Results stay within the
 * row tolerance either way.
 */
void qmv_set_rowmajor(int enable, int rows);

/*
 * Test hook for failure propagation (the role of the reference's link-time
 * block-dot stubs, tests/quantized_matvec_failure_test.cpp:16-38): while
 * armed, the next `count` host-pointer matvec/matmul calls fail after their
 * kernel ran and before results are copied out. count = 0 disarms.
 */
void qmv_debug_fail_next_calls(int count);

#ifdef __cplusplus
}
#endif

#endif
