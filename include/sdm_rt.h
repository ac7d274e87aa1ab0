/* sdm_rt.h -- C ABI of the run-time SDM mixer core for AMD MI355X (gfx950).
 *
 * The reference exposes this path only as a PyTorch module, RunTimeSdm
 * (experiments/track4/sdmllm/track4_onesdm_models.py:151-300); it has no FFI.  These entry points replace the
 * part of RunTimeSdm.forward that lies between the input projections and the output map:
 *   - product-key addressing of the write keys and read queries, softmax weights and write gate
 *     (pk_address, track4_onesdm_models.py:134-148; RunTimeSdm.prepare, :195-213),
 *   - the faded write and causal read of the per-head memory (RunTimeSdm._chunk / forward, :215-274),
 *   - the mean read and the per-head output norm (RunTimeSdm.finish, :243-246, without the wo map).
 * The projections (wk, wq, wv, wg) and the output map wo stay dense GEMMs in the caller.
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller.  The library allocates no device memory; scratch
 *     space is the caller's workspace of sdm_rt_workspace_bytes() bytes.
 *   - Activations are row-major with one row per token, row index n = b * T + t.  In a row, head h of the
 *     write keys / read queries occupies elements [h * addr_dim, (h + 1) * addr_dim), head h of the values and of
 *     the output occupies [h * head_dim, (h + 1) * head_dim) and the gate logit of head h is element h.
 *     Row strides are in elements.  Parameters are float32 and contiguous.
 *   - Every call is asynchronous on the given stream (a hipStream_t passed as void*; NULL is the null stream)
 *     and returns 0 on success or a negative status; sdm_rt_last_error() then describes the failure (a
 *     thread-local string).  Arguments are validated before anything is launched.
 *   - Calls keep their state in the caller's buffers and workspace, with three exceptions: the scratch array of
 *     sdm_rt_forward_noalloc (one per device, shared by every call of that entry point), the wait limit of
 *     sdm_rt_set_wait_limit and the threshold of sdm_rt_set_crowded_threshold (one each per process).
 *   - Concurrency: the forward's scan runs the column groups of one (batch row, head) slab on different compute
 *     units, and each waits (a bounded spin) for the others' partial sums of the out-norm.  Calls on different
 *     streams with different workspaces compute the same results, provided the groups of a slab can be resident
 *     together; when another kernel fills the GPU so that they cannot, a wait can give up.  A wait that gives up
 *     leaves the read-outs of its chunk NaN and records a time-out that sdm_rt_status() reports
 *     (SDM_RT_ETIMEOUT); it never hangs.
 */
#ifndef SDM_RT_H
#define SDM_RT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { SDM_RT_F32 = 0, SDM_RT_BF16 = 1 } sdm_rt_dtype;

enum {
  SDM_RT_OK = 0,
  SDM_RT_EINVAL = -1,     /* bad dimension, pointer, stride or alignment */
  SDM_RT_ENOSPACE = -2,   /* workspace too small */
  SDM_RT_EUNSUPPORTED = -3, /* a shape outside what the kernels are built for */
  SDM_RT_ELAUNCH = -4,    /* a HIP launch failed */
  SDM_RT_ETIMEOUT = -5    /* a forward's wait for the other column groups of a slab gave up (sdm_rt_status) */
};

/* Layer shape and options: the RunTimeSdm constructor arguments that reach the core
 * (track4_onesdm_models.py:154-156). */
typedef struct {
  int32_t batch;        /* B */
  int32_t seq_len;      /* T */
  int32_t heads;        /* H */
  int32_t head_dim;     /* dh = d / H, a multiple of 8 */
  int32_t addr_dim;     /* d_a, even: two halves of d_a / 2 */
  int32_t n_sub;        /* sub-keys per half; M = n_sub^2 locations per head */
  int32_t top_k;        /* k: c1 = min(k, n_sub) per half, kk = min(k, c1^2) picks */
  int32_t read_mean;    /* 1: r = num / (den + read_eps) (read_mode 'mean'); 0: r = num ('sum') */
  int32_t out_norm;     /* 1: r * rsqrt(mean(r^2) + out_norm_eps) * onorm_w */
  int32_t write_gate;   /* 1: write weights times sigmoid(gate logit + gate bias) */
  float read_eps;       /* 1e-3 by default */
  float out_norm_eps;   /* 1e-2 by default */
} sdm_rt_dims;

/* Per-layer parameters (float32, device). */
typedef struct {
  const float* keys1;     /* [H][n_sub][d_a/2], raw (unit-normalised inside) */
  const float* keys2;     /* [H][n_sub][d_a/2] */
  const float* addr_b;    /* [H][d_a] added to every key and query; may be NULL (zero) */
  const float* log_scale; /* [H]; softmax temperature is exp(log_scale) */
  const float* decay;     /* [H] per-head fade lambda in [0, 1] (RunTimeSdm.decay(), :192-193); not read by
                           * sdm_rt_address (may be NULL there) */
  const float* onorm_w;   /* [H][dh]; read only when out_norm */
  const float* gate_bias; /* [H] bias of the gate projection; may be NULL (zero) */
  const void* key_pieces; /* the bfloat16 scoring's sub-key pieces, prepared by sdm_rt_prepare_key_pieces from these
                           * keys1, keys2 and addr_b for the same heads, addr_dim and n_sub (and prepared again
                           * after any of them changes), or NULL: the scoring then derives them itself */
  size_t key_pieces_bytes; /* the size of that buffer; pieces smaller than sdm_rt_key_pieces_bytes(dims) of a call
                            * are not read (the scoring derives them instead) */
} sdm_rt_params;

/* No reference counterpart: the unit normalisation of the sub-keys (F.normalize of keys1/keys2,
 * track4_onesdm_models.py:137-140), their three-term bfloat16 split and their dot products with addr_b, which every
 * bfloat16 scoring of an address set otherwise recomputes, prepared once per parameter version into a caller-owned
 * buffer of sdm_rt_key_pieces_bytes(dims) bytes (0: the shape's scoring does not use them).  The same values the
 * scoring derives, so the same picks.  params->key_pieces is ignored here. */
size_t sdm_rt_key_pieces_bytes(const sdm_rt_dims* dims);
int sdm_rt_prepare_key_pieces(const sdm_rt_dims* dims, const sdm_rt_params* params, void* out, size_t out_bytes,
                              void* stream);

/* Bytes of workspace sdm_rt_forward needs for these dimensions (0 on invalid dims): the chunk plans (33 KB per
 * 64 positions of one head at k <= 8) and their sizes, the scan's progress counters and status word and, with
 * out_norm and more than one column group per head, the out-norm's partial sums (512 bytes per 64 positions of a
 * head and group). */
size_t sdm_rt_workspace_bytes(const sdm_rt_dims* dims);

/* With the write gate, sdm_rt_forward (and sdm_rt_forward_noalloc, in its scratch) leaves in its workspace a copy
 * of the gate logits it read, [B*T][H] in the input dtype, from this byte offset; it stays there until the
 * workspace is next used.  0 without the write gate or on invalid dims.  No reference counterpart: it lets a caller
 * keep RunTimeSdm.last_gate's logits (track4_onesdm_models.py:205, 212) without a copy of its own. */
size_t sdm_rt_gate_copy_offset(const sdm_rt_dims* dims);

/* Row pitch (entries per token and head) of the pick arrays sdm_rt_address writes: kk rounded up to 8. */
int32_t sdm_rt_pick_pitch(const sdm_rt_dims* dims);

/* Product-key addressing of one address set.  Replaces pk_address (track4_onesdm_models.py:134-148) plus the
 * softmax weights and gate of RunTimeSdm.prepare (:203-207).
 *   z            [B*T rows] of H * d_a addresses (before addr_b, which is added here), dtype in_dtype
 *   gate_logits  [B*T rows] of H gate logits (before gate_bias) or NULL: weights are then not gated
 *   slot_out     [B][H][T][pitch] int32 slot ids, the kk picks in descending score order, ties to the lower
 *                index (pad entries -1)
 *   score_out    same layout, float32 scores (v1 + v2) / 2; may be NULL
 *   weight_out   same layout, float32 softmax(exp(log_scale) * score) (times the gate); may be NULL
 *   workspace    not used by the addressing alone (may be NULL) */
int sdm_rt_address(const sdm_rt_dims* dims, const sdm_rt_params* params,
                   const void* z, int64_t z_row_stride,
                   const void* gate_logits, int64_t gate_row_stride,
                   sdm_rt_dtype in_dtype,
                   int32_t* slot_out, float* score_out, float* weight_out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* The SDM core of RunTimeSdm.forward (track4_onesdm_models.py:195-274 between the projections and wo, with
 * finish :243-246 minus wo).
 *   kz, qz       [B*T rows] write keys / read queries (H * d_a each, before addr_b), dtype in_dtype
 *   v            [B*T rows] values (H * dh), dtype in_dtype
 *   gate_logits  [B*T rows] gate logits (H, before gate_bias), dtype in_dtype; may be NULL when write_gate is 0
 *   *_row_stride    element stride between consecutive rows of each input (they may be column slices of one
 *                fused projection output)
 *   reset        [B*T rows] uint8 or NULL: 1 empties the memory before that position reads (a BOS, the reset
 *                masks of forward(x, reset), :229-233); NULL for none
 *   r_out        [B*T rows] of H * dh read-outs, dtype out_dtype, row stride out_row_stride
 *   state_in_mem / state_in_cnt    [B][H][M][dh] / [B][H][M] float32 state to start from, or both NULL to
 *                start from an empty memory (the reference always starts empty, :257-258)
 *   state_out_mem / state_out_cnt  where to write the state after the last position, or NULL (the
 *                reference's last_state side effect, :273) */
int sdm_rt_forward(const sdm_rt_dims* dims, const sdm_rt_params* params,
                   const void* kz, int64_t kz_row_stride, const void* qz, int64_t qz_row_stride,
                   const void* v, int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                   sdm_rt_dtype in_dtype, const uint8_t* reset,
                   void* r_out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                   const float* state_in_mem, const float* state_in_cnt,
                   float* state_out_mem, float* state_out_cnt,
                   void* workspace, size_t workspace_bytes, void* stream);

/* sdm_rt_forward without a workspace argument: the same kernels run on a scratch array that the library holds on
 * each device it runs on (a fixed sdm_rt_noalloc_scratch_bytes() = 128 MiB, kept until the process ends), so the
 * call allocates no device memory.  It has no counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops).  A call whose workspace (sdm_rt_workspace_bytes) exceeds the
 * scratch returns SDM_RT_ENOSPACE without launching anything.  All calls on one device share its scratch: calls that
 * overlap on one device (on different streams, or from different threads) race and must be serialised by the
 * caller.  Arguments as sdm_rt_forward. */
size_t sdm_rt_noalloc_scratch_bytes(void);
int sdm_rt_forward_noalloc(const sdm_rt_dims* dims, const sdm_rt_params* params,
                           const void* kz, int64_t kz_row_stride, const void* qz, int64_t qz_row_stride,
                           const void* v, int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                           sdm_rt_dtype in_dtype, const uint8_t* reset,
                           void* r_out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                           const float* state_in_mem, const float* state_in_cnt,
                           float* state_out_mem, float* state_out_cnt, void* stream);

/* Status of the last sdm_rt_forward (or, with workspace NULL, sdm_rt_forward_noalloc on the current device) that
 * used this workspace with these dims: synchronises the stream, then returns SDM_RT_OK, or SDM_RT_ETIMEOUT when one
 * of the scan's bounded waits gave up (the read-outs of that chunk are then NaN).  No reference counterpart: the
 * reference's forward runs on one stream of dense tensor ops and has no such wait. */
int sdm_rt_status(const sdm_rt_dims* dims, const void* workspace, void* stream);

/* Polls a forward's wait makes before it gives up, for the whole process: polls < 0 restores the default (2^20,
 * about a second), 0 makes every wait give up at once without looking at the partner's sum (for tests of the
 * error path: every kernel still runs to its end).  No reference counterpart. */
void sdm_rt_set_wait_limit(int64_t polls);

/* The forward's pick scan runs a (batch row, head) slab whose chunks crowd (a chunk's plan has a variable part of
 * more than `bytes` bytes: many positions write the same slots) with its owners' write sums ahead of the barrier
 * that ends a chunk's reads; the results are the same bits either way, only the time differs.  For the whole
 * process: bytes < 0 restores the default (4,096, the part staged in LDS), a large value keeps every slab on the
 * plain chunk step.  No reference counterpart. */
void sdm_rt_set_crowded_threshold(int32_t bytes);

/* Bytes of workspace sdm_rt_decode_step needs (the picks of one token per stream; 0 on invalid dims). */
size_t sdm_rt_decode_workspace_bytes(const sdm_rt_dims* dims);

/* One decode step: one token for each of B = dims->batch streams (dims->seq_len must be 1), with the recurrence of
 * RunTimeSdm.forward_sequential (track4_onesdm_models.py:276-300): optional reset, read, then faded write.  The
 * reference keeps no state across calls (it only exposes last_state, :299); this entry point carries it.  Shapes
 * whose addressing runs on the matrix cores (addr_dim 16, 32 or 64 and n_sub <= 32) take one kernel launch.
 *   kz, qz, v, gate_logits   one row per stream, as in sdm_rt_forward
 *   reset        [B] uint8 or NULL: 1 empties that stream's memory before it reads (a BOS, :287-289)
 *   state_mem    [B][H][M][dh] float32, state_cnt [B][H][M] float32, state_scale [B][H] float32, read and
 *                updated in place: the true memory is state_scale * state_mem and the true counts
 *                state_scale * state_cnt.  A new stream starts from mem = cnt = 0, scale = 1; a state from
 *                sdm_rt_forward (state_out_*) continues with scale = 1.  Keeping the scale apart makes the fade
 *                O(1) per step: the cost of a step does not grow with the position (the slab is rescaled once
 *                when the scale falls below 2^-60).
 *   state_last   [B][H][pitch] int32 (pitch = sdm_rt_pick_pitch(dims)) or NULL, updated in place: the slots of
 *                the last step's writes where that step left nothing else (decay 0), else -2 in entry 0.  With it
 *                a head of decay 0 zeroes only those rows instead of its whole slab.  A new stream starts with
 *                every entry -1 (an empty slab), a state from sdm_rt_forward with -2 (unknown).
 *   r_out        one row per stream of H * dh read-outs (after the mean read and the output norm, before wo),
 *                dtype out_dtype */
int sdm_rt_decode_step(const sdm_rt_dims* dims, const sdm_rt_params* params,
                       const void* kz, int64_t kz_row_stride, const void* qz, int64_t qz_row_stride,
                       const void* v, int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                       sdm_rt_dtype in_dtype, const uint8_t* reset,
                       float* state_mem, float* state_cnt, float* state_scale, int32_t* state_last,
                       void* r_out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* The weighted read of the picked rows of per-head value tables: TrainedSdm.forward's embedding_bag
 * (track4_onesdm_models.py:448-455), out[n][h*dh + c] = sum_j weight[b][h][t][j] * values[h][slot[b][h][t][j]][c]
 * over the kk picks of token n = b*T + t, summed in float32 in pick order.
 *   slots, weights  [B][H][T][pitch] as sdm_rt_address writes them (pitch = sdm_rt_pick_pitch(dims))
 *   values          [H][M][dh] (M = n_sub^2, dh = dims->head_dim, a multiple of 4 of any size), dtype values_dtype
 *   out             [B*T rows] of H * dh, dtype out_dtype, row stride out_row_stride (elements) */
int sdm_rt_table_read(const sdm_rt_dims* dims, const int32_t* slots, const float* weights,
                      const void* values, sdm_rt_dtype values_dtype,
                      void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype, void* stream);

/* TrainedSdm's read for a few tokens in one launch (a decode step): the query map q = hx Wq^T, the addressing of q
 * and the weighted read of the picked rows, each as its own entry point computes it (sdm_rt_gemm_rows for the map,
 * sdm_rt_address, sdm_rt_table_read), so the three calls and this one give the same bits.  No single counterpart in
 * the reference: it is TrainedSdm.forward's F.linear, pk_address and embedding_bag (track4_onesdm_models.py:438-455)
 * for at most 256 tokens.  All arrays bfloat16 except the picks.
 *   hx       [B*T rows] of d (the layer width, a multiple of 64), row stride hx_row_stride
 *   wq       [H * addr_dim][d] (addr_dim 32 or 64), row stride wq_row_stride
 *   values   [H][M][head_dim] (head_dim a multiple of 8 up to 1,024), rows contiguous
 *   q_out    [B*T rows] of H * addr_dim, or NULL
 *   slot_out, score_out, weight_out   [B][H][T][pitch] as sdm_rt_address writes them (score_out, weight_out may be
 *            NULL)
 *   out      [B*T rows] of H * head_dim
 * hx, wq, values and out rows 16-byte aligned; params: keys, addr_b, log_scale (no fade, no gate). */
int sdm_rt_table_step(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* hx, int64_t hx_row_stride,
                      int32_t d, const void* wq, int64_t wq_row_stride, const void* values, void* q_out,
                      int64_t q_row_stride, int32_t* slot_out, float* score_out, float* weight_out, void* out,
                      int64_t out_row_stride, void* stream);

/* sdm_rt_table_step with the residual add and TrainedSdm's input norm folded in front: the stage before the table
 * layer left y, OneSdmLM adds it to the residual stream x (x = x + layer(x), track4_onesdm_models.py:540-547) and the
 * table layer normalises the sum (TrainedSdm.norm, :441; RMSNorm, track4_sdmllm_models.py:69-71).  Here
 * sum_out = x + y (bfloat16) and hx = rms_norm(sum_out, norm_w, norm_eps) (bfloat16, kept on chip) feed the table
 * step; bit for bit sdm_rt_add_rms_norm followed by sdm_rt_table_step, in one launch.  x, y and sum_out are [B*T rows]
 * of d = 768 with the given row strides, 16-byte aligned; norm_w [d] float32, 16-byte aligned.  sum_out may be x
 * (in place) when the table has one head.  hx_out [B*T rows] of d receives hx, or NULL.  The other arguments as
 * sdm_rt_table_step's. */
int sdm_rt_table_step_residual(const sdm_rt_dims* dims, const sdm_rt_params* params, const void* x,
                               int64_t x_row_stride, const void* y, int64_t y_row_stride, const float* norm_w,
                               float norm_eps, void* sum_out, int64_t sum_row_stride, void* hx_out,
                               int64_t hx_row_stride, int32_t d, const void* wq, int64_t wq_row_stride,
                               const void* values, void* q_out, int64_t q_row_stride, int32_t* slot_out,
                               float* score_out, float* weight_out, void* out, int64_t out_row_stride, void* stream);

/* The input norm of RunTimeSdm (RMSNorm, experiments/track4/sdmllm/track4_sdmllm_models.py:63-71) with the
 * reference's rounding: out = cast_out(cast_in(x * rsqrt(mean(x^2) + eps)) * w), the mean and product in float32,
 * cast_in rounding to the input dtype and cast_out to out_dtype.
 *   x    [rows] of d values, dtype in_dtype, row stride x_row_stride (elements)
 *   w    [d] float32
 *   out  [rows] of d values, dtype out_dtype, row stride out_row_stride */
int sdm_rt_rms_norm(const void* x, int64_t x_row_stride, sdm_rt_dtype in_dtype, int64_t rows, int32_t d,
                    const float* w, float eps, void* out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                    void* stream);

/* The residual add before an RMSNorm, fused with it (OneSdmLM.residual, track4_onesdm_models.py:540-546:
 * x = x + layer(x), then the next layer's RMSNorm, track4_sdmllm_models.py:63-71): sum = cast_in(x + y), written to
 * sum_out (it may be x itself), and out = the RMSNorm of sum as sdm_rt_rms_norm computes it.
 *   x, y     [rows] of d values, dtype in_dtype, row strides in elements
 *   sum_out  [rows] of d values, dtype in_dtype
 *   out      [rows] of d values, dtype out_dtype */
int sdm_rt_add_rms_norm(const void* x, int64_t x_row_stride, const void* y, int64_t y_row_stride,
                        sdm_rt_dtype in_dtype, int64_t rows, int32_t d, const float* w, float eps,
                        void* sum_out, int64_t sum_row_stride, void* out, int64_t out_row_stride,
                        sdm_rt_dtype out_dtype, void* stream);

/* SwiGLU's gate (track4_sdmllm_models.py:89-97: silu(gate(x)) * up(x)) on the output of one fused [gate | up]
 * projection: out[r][c] = cast(cast(silu(g)) * u), g = gate_up[r][c], u = gate_up[r][f + c], silu(g) =
 * g / (1 + exp(-g)) in float32, each product rounded as torch rounds it.
 *   gate_up  [rows] of 2 f values, dtype, row stride >= 2 f;  out  [rows] of f values, dtype; f a multiple of 8 */
int sdm_rt_silu_mul(const void* gate_up, int64_t gate_up_row_stride, sdm_rt_dtype dtype, int64_t rows, int32_t f,
                    void* out, int64_t out_row_stride, void* stream);

/* y = x W^T (+ bias) for a few rows of x (bfloat16 in and out, float32 sums, bias added before the one rounding):
 * a decode step's dense maps, F.linear / matmul in the reference (RunTimeSdm's wk, wq, wv, wg and wo,
 * track4_onesdm_models.py:199-207, :247; TrainedSdm's wq and wo, :443-455) when x holds one token per stream.
 *   x  [rows][k] bf16, row stride >= k;  W  [n][k] bf16 (a Linear's weight), row stride >= k;  bias  [n] bf16 or NULL;
 *   y  [rows][n] bf16, row stride >= n.  n a multiple of 32, k a positive multiple of 64, x and W rows 16-byte
 *   aligned.  Every workgroup takes 32 columns (and 16, 32 or 64 rows) and splits k over four waves, whose sums are
 *   added in a fixed order (deterministic, and the same bits for every tiling). */
int sdm_rt_gemm_rows(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, const void* bias,
                     void* y, int64_t y_row_stride, int64_t rows, int32_t n, int32_t k, void* stream);

/* sdm_rt_gemm_rows with the residual add and the next layer's input norm folded in front: the stage before left y,
 * OneSdmLM adds it to the residual stream (x = x + layer(x), track4_onesdm_models.py:540-547) and the next mixer
 * normalises the sum before its projections (RunTimeSdm.prepare's norm and maps, :197-206; RMSNorm,
 * track4_sdmllm_models.py:69-71).  Here sum_out = x + y (bf16) and out = rms_norm(sum_out, norm_w, norm_eps) W^T
 * (+ bias), bit for bit sdm_rt_add_rms_norm (bf16 in and out) followed by sdm_rt_gemm_rows, in one launch: each
 * workgroup normalises its rows (16 or 32) on chip.
 *   x, y, sum_out  [rows][k] bf16, row strides >= k;  norm_w  [k] float32;  W, bias, out  as sdm_rt_gemm_rows
 * k = 768, n a positive multiple of 32, at most 256 tiles of 64 rows x 32 columns (a decode step's map; larger
 * calls return SDM_RT_EUNSUPPORTED).  x, y, sum_out and W rows and norm_w 16-byte aligned; sum_out and out must not
 * alias x, y or each other (every workgroup reads x and y while the first column's write the sums). */
int sdm_rt_gemm_rows_residual(const void* x, int64_t x_row_stride, const void* y, int64_t y_row_stride,
                              const float* norm_w, float norm_eps, void* sum_out, int64_t sum_row_stride,
                              const void* w, int64_t w_row_stride, const void* bias, void* out,
                              int64_t out_row_stride, int64_t rows, int32_t n, int32_t k, void* stream);

/* sdm_rt_gemm_rows with the embedding gather and the first layer's input norm folded in front: OneSdmLM embeds the
 * tokens (x = emb(idx), track4_onesdm_models.py:534-535) and the first mixer normalises them before its projections
 * (RunTimeSdm.prepare, :197-206).  Here x_out[r] = table[tokens[r]] (the residual stream, an exact copy) and
 * out = rms_norm(x_out, norm_w, norm_eps) W^T (+ bias), bit for bit the gather followed by sdm_rt_rms_norm (bf16 in
 * and out) and sdm_rt_gemm_rows, in one launch.
 *   tokens  [rows] int64, each in [0, vocab) (a token outside is clamped into it: the host does not read them);
 *   table  [vocab][k] bf16;  x_out  [rows][k] bf16;  norm_w  [k] float32;  W, bias, out  as sdm_rt_gemm_rows
 * k = 768, n a positive multiple of 32, at most 256 tiles of 64 rows x 32 columns (larger calls return
 * SDM_RT_EUNSUPPORTED).  table, x_out and W rows and norm_w 16-byte aligned; x_out and out must not alias the table
 * or each other. */
int sdm_rt_gemm_rows_embed(const int64_t* tokens, const void* table, int64_t table_row_stride, int64_t vocab,
                           const float* norm_w, float norm_eps, void* x_out, int64_t x_row_stride, const void* w,
                           int64_t w_row_stride, const void* bias, void* out, int64_t out_row_stride, int64_t rows,
                           int32_t n, int32_t k, void* stream);

/* ---- training: forward with saved tensors, and the backward ------------------------------------------------
 * The reference trains RunTimeSdm through torch autograd of its chunked dense forward (RunTimeSdm.forward under
 * torch.utils.checkpoint, track4_onesdm_models.py:259-268).  These two entry points replace that autograd for the
 * part between the projections and wo: sdm_rt_forward_train computes what sdm_rt_forward computes and keeps what the
 * backward needs; sdm_rt_backward returns the gradients of the inputs and core parameters for a gradient dy of r_out.
 * The picks are held fixed (topk and the slot ids carry no gradient, as in autograd).  The memory starts empty (no
 * state input) and the state is not returned. */

/* What the forward keeps for the backward (caller-owned device buffers; pitch = sdm_rt_pick_pitch(dims)). */
typedef struct {
  int32_t* slots_w;   /* [B][H][T][pitch] write picks, as sdm_rt_address writes them */
  float* weights_w;   /*   their weights (softmax times the gate) */
  float* scores_w;    /*   their scores */
  int32_t* slots_r;   /* [B][H][T][pitch] read picks */
  float* weights_r;
  float* scores_r;
  float* read;        /* [B*T rows] of H * dh float32: the read before the output norm (num / (den + read_eps), or
                       * num with read_mean 0) */
  float* den;         /* [B*T][H] float32 read denominators; needed only with read_mean */
} sdm_rt_saved;

/* Gradients written by sdm_rt_backward (overwritten, not accumulated; float32 device buffers). */
typedef struct {
  float* d_kz;                 /* [B*T rows] of H * d_a: d loss / d kz (rows as kz, before addr_b) */
  int64_t d_kz_row_stride;
  float* d_qz;                 /* d loss / d qz */
  int64_t d_qz_row_stride;
  float* d_v;                  /* [B*T rows] of H * dh */
  int64_t d_v_row_stride;
  float* d_gate_logits;        /* [B*T rows] of H; required when write_gate */
  int64_t d_gate_row_stride;
  float* d_keys1;              /* [H][n_sub][d_a/2] raw sub-key gradients, or NULL (then d_keys2 NULL too) */
  float* d_keys2;
  float* d_addr_b;             /* [H][d_a] or NULL */
  float* d_log_scale;          /* [H] or NULL */
  float* d_onorm_w;            /* [H][dh] or NULL (written only with out_norm) */
  float* d_gate_bias;          /* [H] or NULL (0 without the gate) */
  float* d_log_decay;          /* [H] or NULL: lambda * d loss / d lambda, the gradient with respect to log lambda
                                * (finite at lambda = 0); d decay_logit = d_log_decay * (1 - lambda) */
} sdm_rt_grads;

/* sdm_rt_forward (no state input or output) that also fills *saved.  Workspace: sdm_rt_workspace_bytes(dims). */
int sdm_rt_forward_train(const sdm_rt_dims* dims, const sdm_rt_params* params,
                         const void* kz, int64_t kz_row_stride, const void* qz, int64_t qz_row_stride,
                         const void* v, int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                         sdm_rt_dtype in_dtype, const uint8_t* reset,
                         void* r_out, int64_t out_row_stride, sdm_rt_dtype out_dtype,
                         const sdm_rt_saved* saved, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace sdm_rt_backward needs (0 on invalid dims or a shape the backward does not cover). */
size_t sdm_rt_backward_workspace_bytes(const sdm_rt_dims* dims);

/* The backward of sdm_rt_forward_train: the same inputs (kz, qz, v, gate_logits, reset, params), its *saved, and dy,
 * the gradient of r_out ([B*T rows] of H * dh, dtype dy_dtype).  Writes *grads.  The sums over tokens run in a fixed
 * order, so the result is deterministic. */
int sdm_rt_backward(const sdm_rt_dims* dims, const sdm_rt_params* params,
                    const void* kz, int64_t kz_row_stride, const void* qz, int64_t qz_row_stride,
                    const void* v, int64_t v_row_stride, const void* gate_logits, int64_t gate_row_stride,
                    sdm_rt_dtype in_dtype, const uint8_t* reset, const sdm_rt_saved* saved,
                    const void* dy, int64_t dy_row_stride, sdm_rt_dtype dy_dtype,
                    const sdm_rt_grads* grads, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace sdm_rt_table_backward needs (0 on invalid dims or a shape it does not cover). */
size_t sdm_rt_table_backward_workspace_bytes(const sdm_rt_dims* dims);

/* The backward of TrainedSdm's table layer between the query map and wo (track4_onesdm_models.py:438-455: pk_address
 * of the query, softmax(exp(log_scale) * score), the embedding_bag read of the value tables), for picks held fixed:
 *   q            [B*T rows] of H * d_a queries the picks came from (dtype in_dtype; no address bias)
 *   slots, weights, scores   [B][H][T][pitch] as sdm_rt_address wrote them for q
 *   values       [H][M][dh] value tables (dtype values_dtype); dims->head_dim = dh
 *   dy           [B*T rows] of H * dh: the gradient of the read (sdm_rt_table_read's out), dtype dy_dtype
 * writes d_q (float32 rows), d_values ([H][M][dh] float32, overwritten; each row summed over its picks in pick order:
 * the picks are sorted by slot with a stable radix sort), d_keys1 / d_keys2 (both or neither) and d_log_scale ([H] or
 * NULL).  Every sum runs in a fixed order, so the result is deterministic. */
int sdm_rt_table_backward(const sdm_rt_dims* dims, const sdm_rt_params* params,
                          const void* q, int64_t q_row_stride, sdm_rt_dtype in_dtype,
                          const int32_t* slots, const float* weights, const float* scores,
                          const void* values, sdm_rt_dtype values_dtype,
                          const void* dy, int64_t dy_row_stride, sdm_rt_dtype dy_dtype,
                          float* d_q, int64_t d_q_row_stride, float* d_values,
                          float* d_keys1, float* d_keys2, float* d_log_scale,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Description of the last failure on the calling thread ("" if none). */
const char* sdm_rt_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* SDM_RT_H */
