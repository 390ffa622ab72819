/*
 * wc_abi.h -- C ABI of libwide_hip.so, the gfx950 (MI355X) kernels behind the
 * N-first wide-primitive forward path of wide_compiler.
 *
 * The reference (WideCompiler, pure PyTorch) has no FFI: every entry point
 * below replaces one or more PyTorch library calls made by a reference
 * primitive.  Each declaration cites the reference call site it replaces
 * (paths relative to the reference repository root).
 *
 * Conventions
 *   - All pointers are device pointers unless stated otherwise.  The library
 *     never allocates or frees device memory and keeps no pointer after a call
 *     returns.
 *   - `stream` is a hipStream_t passed as void* (NULL = legacy default stream).
 *     Every launch is asynchronous on that stream; no host synchronisation.
 *   - Strides are in ELEMENTS unless the name ends in `_bytes`.
 *   - Return value: 0 = success; < 0 = argument / shape / dtype error detected
 *     on the host before any launch (nothing was launched); > 0 = a hipError_t
 *     reported by the runtime at launch.  wc_last_error() returns a
 *     thread-local message describing the last non-zero status.
 *   - Functions are stateless and re-entrant; concurrent calls on different
 *     streams are safe.
 */
#ifndef WC_ABI_H
#define WC_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WC_ABI_VERSION 5

/* element types */
enum {
  WC_F32 = 0,
  WC_BF16 = 1,
  WC_F16 = 2
};

/* status codes (negative: host-side argument errors) */
enum {
  WC_OK = 0,
  WC_ERR_NULL = -1,      /* required pointer is NULL */
  WC_ERR_SHAPE = -2,     /* inconsistent or unsupported sizes */
  WC_ERR_DTYPE = -3,     /* unsupported element type */
  WC_ERR_ALIGN = -4,     /* pointer / stride alignment the kernel requires */
  WC_ERR_LIMIT = -5,     /* size beyond what the kernel supports */
  WC_ERR_ARG = -6        /* any other invalid argument */
};

/* epilogue activations */
enum {
  WC_ACT_NONE = 0,
  WC_ACT_RELU = 1
};

/* recurrent cell kinds */
enum {
  WC_CELL_GRU = 0,
  WC_CELL_LSTM = 1
};

/* ABI version compiled into the library (== WC_ABI_VERSION). */
int32_t wc_abi_version(void);

/* Thread-local text of the last error returned on this thread ("" if none). */
const char* wc_last_error(void);

/* Number of HIP devices visible (0 without a GPU); never launches work. */
int32_t wc_device_count(void);

/*
 * pack_inputs -- replaces torch.stack(inputs, dim=1) + view
 * (wide_compiler/core/ensemble_util.py:44-60, alias api.pack api.py:310-316).
 *   dst[r, i, :] = src_i[r, :]  for r < rows, i < n,
 * where source i row r starts at srcs[i] + r * src_row_stride_bytes[i] and
 * holds row_bytes contiguous bytes; dst is contiguous [rows, n, row_bytes].
 * `srcs` and `src_row_stride_bytes` are HOST arrays of length n holding
 * device addresses / byte strides.  Bit-exact byte copy.
 */
int32_t wc_pack_rows(const void* const* srcs, const int64_t* src_row_stride_bytes,
                     int64_t n, int64_t rows, int64_t row_bytes,
                     void* dst, void* stream);

/*
 * Boundary transpose -- replaces the N-first <-> channel-packed reshapes of
 * TracedWideModel.forward (wide_compiler/core/traced_wide.py:463-469 in,
 * 527-532 out) and the permute(...).contiguous() copies of the conv / norm
 * primitives (wide_conv2d.py:179,192-194; wide_batchnorm_2d.py:63,69-71).
 *   dst[j, i, :] = src[i, j, :]   i < d0, j < d1,
 * src element (i, j) starts at src + i*src_stride0_bytes + j*src_stride1_bytes
 * and holds inner_bytes contiguous bytes; dst is contiguous [d1, d0, inner].
 * Bit-exact byte copy.
 */
int32_t wc_swap01(const void* src, int64_t d0, int64_t d1,
                  int64_t src_stride0_bytes, int64_t src_stride1_bytes,
                  int64_t inner_bytes, void* dst, void* stream);

/*
 * Embedding gather -- replaces weight[:, x] / F.embedding
 * (wide_compiler/core/primitives/wide_embedding.py:93-131).
 *   out[i, r, :] = weight[i, ids[r], :]           (ids_shared != 0, ids [rows])
 *   out[i, r, :] = weight[i, ids[i*rows + r], :]  (ids_shared == 0, ids [n, rows])
 * weight is contiguous [n, vocab, dim] of `dtype`; ids are int64; out is
 * contiguous [n, rows, dim].  An id outside [0, vocab) reads nothing, writes a
 * zero row and, if err_flag != NULL, stores 1 into *err_flag (device int32).
 * Bit-exact copy.
 */
int32_t wc_embedding_gather(const void* weight, int64_t n, int64_t vocab, int64_t dim,
                            int32_t dtype, const int64_t* ids, int64_t rows,
                            int32_t ids_shared, void* out, int32_t* err_flag,
                            void* stream);

/*
 * LayerNorm over the last dim with per-model affine -- replaces the manual
 * mean / var(unbiased=False) / normalise / affine sequence of
 * WideLayerNorm.forward (wide_compiler/core/primitives/wide_layernorm.py:48-67).
 *   x, y: [n, rows_per_model, dim] (row stride x_row_stride / y_row_stride,
 *         model stride x_model_stride / y_model_stride, unit inner stride)
 *   gamma, beta: [n, dim] contiguous of `param_dtype` (beta may be NULL)
 *   y = (x - mean) / sqrt(var + eps) * gamma + beta, statistics in fp32.
 */
int32_t wc_layernorm(const void* x, int64_t x_model_stride, int64_t x_row_stride,
                     const void* gamma, const void* beta,
                     void* y, int64_t y_model_stride, int64_t y_row_stride,
                     int64_t n, int64_t rows_per_model, int64_t dim, float eps,
                     int32_t dtype, int32_t param_dtype, void* stream);

/*
 * Embedding gather followed by LayerNorm, in one pass -- replaces WideEmbedding.forward
 * (wide_compiler/core/primitives/wide_embedding.py:93-131) feeding WideLayerNorm.forward
 * (wide_compiler/core/primitives/wide_layernorm.py:48-67) when the embedding's output goes
 * only to the LayerNorm:
 *   out[i, r, :] = LayerNorm_i(weight[i, id, :]),  id = ids[r] (ids_shared != 0, ids [rows])
 *                                                  or ids[i*rows + r] (ids_shared == 0, ids [n, rows])
 * weight contiguous [n, vocab, dim] of `dtype`; gamma, beta [n, dim] of `param_dtype` (beta may
 * be NULL); out contiguous [n, rows, dim].  An id outside [0, vocab) normalises a zero row (the
 * row wc_embedding_gather writes for it) and stores 1 into *err_flag when err_flag != NULL.
 * The output equals wc_embedding_gather followed by wc_layernorm bit for bit.  Rows must be
 * 16-byte vectors (dim a multiple of 16 / element size, at most 256 vectors) with 16-byte aligned
 * weight, gamma, beta and out; otherwise WC_ERR_LIMIT and nothing is launched.
 */
int32_t wc_embedding_layernorm(const void* weight, int64_t n, int64_t vocab, int64_t dim,
                               const int64_t* ids, int64_t rows, int32_t ids_shared,
                               const void* gamma, const void* beta, float eps, int32_t dtype,
                               int32_t param_dtype, void* out, int32_t* err_flag, void* stream);

/*
 * Eval-mode BatchNorm per (model, channel) on N-first [n, b, c, hw] --
 * replaces permute + nn.BatchNorm2d(N*C) (eval) + permute().contiguous()
 * (wide_compiler/core/primitives/wide_batchnorm_2d.py:53-71).
 *   y = (x - running_mean) / sqrt(running_var + eps) * weight + bias
 * with the per-channel parameters at index (i*c + ch), computed in fp32.
 * x strides (x_stride_n, x_stride_b) for the first two dims; the [c, hw]
 * block of each (i, b) is contiguous.  y is contiguous [n, b, c, hw].
 * weight / bias may be NULL (affine=False); act = WC_ACT_NONE or WC_ACT_RELU.
 */
int32_t wc_bn_eval(const void* x, int64_t x_stride_n, int64_t x_stride_b,
                   const void* weight, const void* bias,
                   const void* running_mean, const void* running_var, float eps,
                   void* y, int64_t n, int64_t b, int64_t c, int64_t hw,
                   int32_t dtype, int32_t param_dtype, int32_t act, void* stream);

/*
 * GroupNorm / InstanceNorm on N-first activations -- replaces the channel-packed
 * nn.GroupNorm(N*G, N*C) of WideGroupNorm.forward (wide_compiler/core/primitives/
 * wide_groupnorm.py:89-117) and nn.InstanceNorm1d/2d(N*C) of WideInstanceNorm1d/2d
 * .forward (wide_instancenorm.py:82-101, 213-232) together with the permutes and
 * .contiguous() around them.  x, y contiguous [n, b, c, s] (s = product of the
 * spatial dims); c % groups == 0 (instance norm: groups = c).  Each (model i,
 * batch row, group) normalises its (c / groups) * s elements with the biased
 * variance, in fp32:
 *   y = (x - mean) / sqrt(var + eps) * weight[i*c + ch] + bias[i*c + ch]
 * weight and bias both NULL when not affine; act = WC_ACT_NONE or WC_ACT_RELU.
 */
int32_t wc_group_norm(const void* x, void* y, int64_t n, int64_t b, int64_t c, int64_t s,
                      int64_t groups, const void* weight, const void* bias, float eps,
                      int32_t dtype, int32_t param_dtype, int32_t act, void* stream);

/*
 * Recurrent layer forward (single layer, unidirectional) -- replaces the fused
 * input projection einsum + T-step Python loop of
 *   WideGRU._forward_fused  (wide_compiler/core/primitives/wide_gru.py:148-213)
 *   WideLSTM._forward_fused (wide_compiler/core/primitives/wide_lstm.py:158-234)
 * Gate order: GRU (r, z, n); LSTM (i, f, g, o) -- the torch.nn order.
 */
typedef struct wc_rnn_args {
  int32_t cell;              /* WC_CELL_GRU or WC_CELL_LSTM */
  int32_t dtype;             /* element type of x, weights, h, out */
  int64_t n, batch, steps, input_size, hidden;
  const void* x;             /* [n, batch, steps, input_size] with strides below */
  int64_t x_stride_n, x_stride_b, x_stride_t;   /* unit stride over input_size */
  const void* w_ih;          /* [n, G, input_size] contiguous, G = 3H (GRU) / 4H (LSTM) */
  const void* w_hh;          /* [n, G, hidden] contiguous */
  const void* b_ih;          /* [n, G] or NULL */
  const void* b_hh;          /* [n, G] or NULL */
  const void* h0;            /* [n, batch, hidden] contiguous or NULL (zeros) */
  const void* c0;            /* LSTM only: [n, batch, hidden] or NULL (zeros) */
  void* out;                 /* [n, batch, steps, hidden] contiguous */
  void* h_n;                 /* [n, batch, hidden] contiguous (may be NULL) */
  void* c_n;                 /* LSTM only: [n, batch, hidden] (may be NULL) */
  void* workspace;           /* device scratch of >= wc_rnn_workspace_bytes(args) bytes,
                                16-byte aligned; holds the fp32 input projection */
  int64_t workspace_bytes;
  void* status;              /* optional caller-owned int32 device word: the partitioned
                                LSTM sets it to 1 when a bounded cross-workgroup wait gives
                                up, and the library never clears it (so it also collects
                                the verdicts of graph replays until the caller reads and
                                clears it).  NULL: the workspace's own status word
                                (wc_rnn_status_offset), zeroed by every input projection. */
} wc_rnn_args;

/* Bytes of workspace wc_rnn_forward needs for these sizes on the current device.
 * Partitioned plan (see wc_rnn_recurrence), with U = n * ceil(batch / 16) units: 16-bit
 * input projection n*batch*steps*G*2 + fp32 bias n*G*4 (+ GRU: fp32 b_hn n*hidden*4) +
 * exchange slots U*2*16*hidden*4 + step counters U*128 + a status word, each rounded up
 * to 256 bytes.  Otherwise: fp32 input projection n*batch*steps*G*4 + fp32 cell state
 * n*batch*hidden*4. */
int64_t wc_rnn_workspace_bytes(const wc_rnn_args* args);

/* Byte offset in the workspace of the int32 status word of the partitioned plan, or
 * -1 when these sizes use another plan.  wc_rnn_input_projection zeroes
 * it; the recurrence sets it to 1 if a cross-workgroup wait timed out, in which
 * case out / h_n / c_n are invalid. */
int64_t wc_rnn_status_offset(const wc_rnn_args* args);

/* Poll rounds after which a wait of the partitioned LSTM gives up, for launches made
 * from now on (process-wide; a launch captured into a graph keeps the value it was
 * captured with).  0 gives up at the first wait without polling, so every workgroup
 * leaves at once and the status word is set; a negative value restores the default
 * (2^21 rounds of >= ~0.5 us).  Returns the previous value.  No counterpart in the
 * reference (its recurrence has no cross-workgroup waits): a test hook for the
 * give-up path. */
int32_t wc_rnn_set_spin_limit(int32_t polls);

/* Runs wc_rnn_input_projection, then wc_rnn_recurrence. */
int32_t wc_rnn_forward(const wc_rnn_args* args, void* stream);

/* Phase 1: gates_x = x W_ih^T + b_ih for all steps (grouped MFMA GEMM, fp32
 * accumulate) into the workspace as fp32 [n, batch*steps, G] -- the einsum
 * before the reference's time loop (wide_gru.py:168-170, wide_lstm.py:190-193).
 * Partitioned plan: gates_x = x W_ih^T + (b_ih + b_hh) rounded once to the element type
 * (GRU: gate n takes b_ih alone; its b_hh is kept in fp32 for the recurrence), and the
 * plan's step counters and status word are zeroed. */
int32_t wc_rnn_input_projection(const wc_rnn_args* args, void* stream);

/* Phase 2: the time loop (wide_gru.py:181-211, wide_lstm.py:205-232) reading
 * gates_x from the workspace that phase 1 filled; x and w_ih are not read.
 *  - One model's W_hh fits a workgroup's registers: one persistent launch, one
 *    workgroup per (model, batch row).
 *  - Partitioned plan (LSTM or GRU, bf16 or fp16, hidden 256 / 384 / 512, 16-byte
 *    aligned w_hh / h0 / c0 / out / h_n / c_n): hidden/128 workgroups per unit of
 *    (model, 16 batch rows), one per compute unit, that keep the model's W_hh and the
 *    state on-chip for all steps and exchange h_t through device-coherent memory; a
 *    cooperative launch per (compute units / (hidden/128)) units (ordinary launches
 *    under stream capture).
 *  - Otherwise one launch per step (an MFMA gate GEMM fused with the cell update;
 *    hidden % 32 == 0). */
int32_t wc_rnn_recurrence(const wc_rnn_args* args, void* stream);

/*
 * wc_rnn_forward without a caller-provided workspace: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid allocation).  The workspace is a file-scope
 * device array of wc_rnn_noalloc_scratch_bytes() bytes (64 MiB), one per device,
 * held from the first call on a device until the process ends; args->workspace and
 * args->workspace_bytes are ignored.  Sizes whose wc_rnn_workspace_bytes exceeds it
 * return WC_ERR_LIMIT.  The call allocates and frees nothing.  All calls on one device
 * share its array: calls that overlap in time on one device race.
 */
int64_t wc_rnn_noalloc_scratch_bytes(void);
int32_t wc_rnn_forward_noalloc(const wc_rnn_args* args, void* stream);

/*
 * Grouped GEMM with fused epilogue -- replaces torch.einsum('noi,nbi->nbo')
 * + bias of WideLinear._forward_einsum (wide_compiler/core/primitives/
 * wide_linear.py:161-171), the projection einsums of WideAttention
 * (wide_attention.py:199-213, 234-236) and the recurrent input projections
 * (wide_gru.py:168-170, wide_lstm.py:190-193):
 *   C[i, m, o] = act( sum_k A[i, m, k] * W[i, o, k] + bias[i, o] + R[i, m, o] )
 * Row m of A (and of C / R) lives at  i*stride_n + (m / rows_inner)*stride_outer
 * + (m % rows_inner)*stride_inner; the K (resp. O) dimension is contiguous.
 * W is [n, o, k] with row stride k and model stride w_stride_n.
 * dtype in {WC_F32, WC_BF16, WC_F16} (fp32 accumulation on MFMA); out_dtype is
 * WC_F32 or dtype; bias_dtype is WC_F32 or dtype; bias and residual may be NULL.
 */
typedef struct wc_gemm_args {
  int32_t dtype, out_dtype, bias_dtype, act;
  int64_t n, m, o, k;
  const void* a;
  int64_t a_stride_n, a_stride_outer, a_stride_inner, a_rows_inner;
  const void* w;
  int64_t w_stride_n;
  const void* bias;
  int64_t bias_stride_n;
  const void* residual;
  int64_t r_stride_n, r_stride_outer, r_stride_inner;   /* rows as C */
  void* c;
  int64_t c_stride_n, c_stride_outer, c_stride_inner, c_rows_inner;
} wc_gemm_args;

int32_t wc_grouped_gemm(const wc_gemm_args* args, void* stream);

/*
 * Two chained WideLinear stages in one launch -- replaces, for a traced
 * Linear -> [ReLU] -> Linear chain, the two einsum + bias calls of
 * WideLinear._forward_einsum (wide_compiler/core/primitives/wide_linear.py:
 * 150-173) and the F.relu FunctionalOp between them that TracedWideModel runs
 * (wide_compiler/core/traced_wide.py:174-211, 471-514):
 *   h[i][m] = act1(x[i][m] W1[i]^T + b1[i]),  y[i][m] = act2(h[i][m] W2[i]^T + b2[i])
 * with h rounded to `dtype` (as the first stage would store it) but never
 * written to memory.  x / y rows use the two-level addressing of
 * wc_gemm_args (row m = (m / rows_inner) * stride_outer + (m % rows_inner) *
 * stride_inner within model i's block at stride_n).  W1 [n, hidden, in],
 * W2 [n, out, hidden] contiguous; biases [n, hidden] / [n, out] or NULL; all of
 * one element type.  Sizes must satisfy wc_mlp2_supported.
 */
typedef struct wc_mlp2_args {
  int32_t dtype, act1, act2;
  int64_t n, m, in_features, hidden, out_features;
  const void* x;
  int64_t x_stride_n, x_stride_outer, x_stride_inner, x_rows_inner;
  const void* w1;
  const void* b1;
  const void* w2;
  const void* b2;
  void* y;
  int64_t y_stride_n, y_stride_outer, y_stride_inner, y_rows_inner;
} wc_mlp2_args;

/* 1 if wc_mlp2 handles these sizes, else 0: in and hidden multiples of 32
 * (fp32) or 64 (bf16), out a multiple of 16, hidden and out at most 256, and
 * 32 rows of x and h plus W1 and W2 of one model within 160 KB of LDS. */
int32_t wc_mlp2_supported(int32_t dtype, int64_t in_features, int64_t hidden, int64_t out_features);

int32_t wc_mlp2(const wc_mlp2_args* args, void* stream);

/*
 * Convolution weights packed for wc_conv2d: out[i, co, r, s, c] = w[i*c_out + co, c, r, s]
 * for c < c_in and 0 for c_in <= c < Ci32 (c_in rounded up to 32).  w is the grouped
 * filter bank [n*c_out, c_in, kh, kw] of WideConv2d.grouped_conv / WideConv1d.op
 * (wide_conv2d.py:149-158, wide_conv1d.py:85-94).  out holds
 * wc_conv_packed_weight_elems(...) elements of `dtype`, 16-byte aligned (-1 for sizes that
 * are negative, a non-positive c_in / kh / kw, or a count that does not fit in int64).
 */
int32_t wc_conv_pack_weights(const void* w, int64_t n, int64_t c_out, int64_t c_in, int64_t kh,
                             int64_t kw, int32_t dtype, void* out, void* stream);
int64_t wc_conv_packed_weight_elems(int64_t n, int64_t c_out, int64_t c_in, int64_t kh, int64_t kw);

/*
 * Grouped 2-D convolution (1-D as h = 1) with fused epilogue -- replaces the
 * permute/reshape + grouped nn.Conv2d / nn.Conv1d + permute().contiguous() of
 * WideConv2d.forward (wide_conv2d.py:176-194) and WideConv1d.forward
 * (wide_conv1d.py:125-141), and, when a BatchNorm / add / ReLU stage follows,
 * WideBatchNorm2d.forward (wide_batchnorm_2d.py:60-71) and the traced add / relu
 * stages (traced_wide.py:174-211):
 *   y = act( BN(conv(x, W) + bias) + residual )
 * x: [n, batch, c_in, h, w] where each (i, b) block [c_in, h, w] is contiguous
 * (strides x_stride_n, x_stride_b); y and residual likewise with [c_out, h_out, w_out]
 * blocks.  BN is eval-mode (y = (v - mean) / sqrt(var + eps) * weight + bias),
 * applied when bn_mean != NULL.  Parameters are [n*c_out] of param_dtype.
 * dtype in {WC_F32, WC_BF16, WC_F16}; fp32 accumulation on MFMA (fp16: the general
 * packed-weight kernel).
 */
typedef struct wc_conv_args {
  int32_t dtype, param_dtype, act;
  int64_t n, batch, c_in, c_out, h, w, kh, kw;
  int64_t stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, h_out, w_out;
  const void* x;
  int64_t x_stride_n, x_stride_b;
  const void* packed_weight;   /* from wc_conv_pack_weights */
  const void* bias;
  const void* bn_weight;
  const void* bn_bias;
  const void* bn_mean;
  const void* bn_var;
  float bn_eps;
  const void* residual;
  int64_t r_stride_n, r_stride_b;
  void* y;
  int64_t y_stride_n, y_stride_b;
  const void* weight;          /* the grouped filter bank [n*c_out, c_in, kh, kw] itself (contiguous,
                                  16-byte aligned), read when packed_weight is NULL: allowed when
                                  wc_conv2d_direct_weights returns 1 */
} wc_conv_args;

int32_t wc_conv2d(const wc_conv_args* args, void* stream);

/* Part of the replacement of self.grouped_conv(x) (wide_compiler/core/primitives/
 * wide_conv2d.py:169-194), which reads grouped_conv.weight on every call: 1 when wc_conv2d
 * runs these sizes from args->weight directly (packed_weight NULL) -- the resident-weight
 * kernel (bf16 'same' convolution, stride 1, C_in 32 or 64, C_out a multiple of 64, the
 * input widths it is built for) stages the module's filter bank in its own layout, so no
 * packing pass precedes it; 0 otherwise (wc_conv_pack_weights, then wc_conv2d). */
int32_t wc_conv2d_direct_weights(const wc_conv_args* args);

/*
 * Grouped 3-D convolution -- replaces the permute/reshape + grouped nn.Conv3d +
 * permute().contiguous() of WideConv3d.forward (wide_compiler/core/primitives/
 * wide_conv3d.py:102-124):
 *   y = act(conv3d(x, W) + bias)
 * x: [n, batch, c_in, d, h, w] with each (i, b) block [c_in, d, h, w] contiguous
 * (strides x_stride_n, x_stride_b); y likewise with [c_out, d_out, h_out, w_out]
 * blocks.  packed_weight from wc_conv_pack_weights(w, n, c_out, c_in, kd * kh, kw, ...)
 * on the grouped filter bank [n*c_out, c_in, kd, kh, kw]; bias [n*c_out] of
 * param_dtype or NULL.  dtype in {WC_F32, WC_BF16, WC_F16}; fp32 accumulation on MFMA.
 */
typedef struct wc_conv3d_args {
  int32_t dtype, param_dtype, act;
  int64_t n, batch, c_in, c_out, d, h, w, kd, kh, kw;
  int64_t stride_d, stride_h, stride_w, pad_d, pad_h, pad_w, dil_d, dil_h, dil_w, d_out, h_out, w_out;
  const void* x;
  int64_t x_stride_n, x_stride_b;
  const void* packed_weight;
  const void* bias;
  void* y;
  int64_t y_stride_n, y_stride_b;
} wc_conv3d_args;

int32_t wc_conv3d(const wc_conv3d_args* args, void* stream);

/*
 * Fused multi-head attention core -- replaces the view/permute/reshape to
 * [N*B, H, T, Dh], F.scaled_dot_product_attention and the permute back of
 * WideAttention._forward_fused (wide_compiler/core/primitives/wide_attention.py:
 * 215-231):  O = softmax(Q K^T * scale [+ causal mask]) V  per (n*b, head).
 * Q/K/V/O rows live at base + nb*stride_nb + s*stride_s + head*head_dim, i.e. the
 * [N*B, S, heads*head_dim] layout of the projection outputs, read in place.
 * dtype WC_F32, WC_BF16 or WC_F16; fp32 softmax / accumulation.  Any head_dim >= 1 up to 256
 * (16-bit types) or 128 (fp32), else WC_ERR_LIMIT; pointers aligned to the element size (else
 * WC_ERR_ALIGN).  Other head dims than 16/32/64/128 are zero-padded to the next of 16/32/64/96/
 * 128/256, and past 128 take one launch per 128 output columns.  16-byte aligned rows whose head
 * spans whole 16-byte pieces load 16-byte vectors; other rows load element by element (~2x slower).
 */
typedef struct wc_attn_args {
  int32_t dtype, causal;
  int64_t nb, heads, sq, skv, head_dim;
  float scale;
  const void* q;
  int64_t q_stride_nb, q_stride_s;
  const void* k;
  int64_t k_stride_nb, k_stride_s;
  const void* v;
  int64_t v_stride_nb, v_stride_s;
  void* o;
  int64_t o_stride_nb, o_stride_s;
  const void* mask;            /* optional additive fp32 mask (NULL = none; not with causal):
                                  element (nb, head, query, key) at mask + nb*mask_stride_nb +
                                  head*mask_stride_head + query*mask_stride_q + key, added to the
                                  scaled score (a boolean mask: 0 / -inf).  Strides may be 0
                                  (broadcast).  A query row whose keys are all -inf gets zeros. */
  int64_t mask_stride_nb, mask_stride_head, mask_stride_q;
} wc_attn_args;

int32_t wc_attention(const wc_attn_args* args, void* stream);

/*
 * Self-attention core with the Q and K|V projections fused in -- replaces the Q, K and V
 * einsums and bias adds, the head reshapes and F.scaled_dot_product_attention of
 * WideAttention._forward_fused (wide_compiler/core/primitives/wide_attention.py:197-231)
 * when query, key and value are one tensor x:
 *   O = softmax((x Wq^T + bq) (x Wk^T + bk)^T * scale [+ causal mask]) (x Wv^T + bv)
 * per (model, batch row, head), with Wk, Wv = kv_weight rows [0, D), [D, 2D) and bk, bv the
 * matching halves of kv_bias.  The output projection stays a grouped GEMM (wc_grouped_gemm).
 * x row t of (model n, batch row b) at x + n*x_stride_n + b*x_stride_b + t*x_stride_s (D
 * contiguous elements); O row at o + (n*B + b)*o_stride_nb + t*o_stride_s.  Weights and
 * biases have contiguous rows.  Supported (else WC_ERR_LIMIT, nothing launched): dtype
 * WC_BF16, head_dim = d_model / heads = 32, 1 <= s <= 512, d_model <= 768; no mask.  Q, K, V
 * are rounded to bf16 after the fp32 bias add, as the unfused path's GEMMs round them.
 */
typedef struct wc_self_attn_args {
  int32_t dtype, causal;
  int64_t n, b, s, d_model, heads;
  float scale;
  const void* x;
  int64_t x_stride_n, x_stride_b, x_stride_s;
  const void* q_weight;        /* [N][D][D] */
  int64_t q_weight_stride_n;
  const void* kv_weight;       /* [N][2D][D] */
  int64_t kv_weight_stride_n;
  const void* q_bias;          /* [N][D] or NULL */
  int64_t q_bias_stride_n;
  const void* kv_bias;         /* [N][2D] or NULL */
  int64_t kv_bias_stride_n;
  void* o;
  int64_t o_stride_nb, o_stride_s;
} wc_self_attn_args;

int32_t wc_self_attention(const wc_self_attn_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WC_ABI_H */
