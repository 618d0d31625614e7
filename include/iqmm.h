/*
 * iqmm.h — C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * Drop-in for the quantized ops ironmlx's Rust `mlx` crate calls through
 * mlx-sys/mlx-c.  Every entry point mirrors the mlx-c call it replaces:
 *
 *   iqmm_quantized_matmul  <- mlx_quantized_matmul  (mlx/src/ops.rs:695-727,
 *                                                    FFI call at ops.rs:713-724)
 *   iqmm_dequantize        <- mlx_dequantize        (mlx/src/ops.rs:653-686,
 *                                                    FFI call at ops.rs:673-683)
 *   iqmm_gather_qmm        <- mlx_gather_qmm        (not bound by ironmlx today;
 *                                                    replaces the per-expert loop
 *                                                    in mlx/src/nn/moe.rs:84-170)
 *   iqmm_quantize          <- mlx_quantize          (not bound by ironmlx; makes
 *                                                    the packed inputs)
 *   iqmm_quantized_swiglu  <- gate/up quantized_matmul + silu * up
 *                             (mlx/src/nn/mlp.rs:27-33)
 *   iqmm_gather_qmm_swiglu <- the same per expert (mlx/src/nn/moe.rs:10-33)
 *   iqmm_dequantize_rows   <- dequantize + take_axis (mlx/src/nn/embedding.rs:62-72)
 *   iqmm_moe_route / _sort / _combine
 *                          <- the router, token lists and weighted sum of
 *                             mlx/src/nn/moe.rs:67-168
 *   iqmm_last_error        <- the thread-local message mlx's error handler
 *                             stores (mlx/src/error.rs:17-55)
 *
 * Conventions (same as mlx-c):
 *   - return 0 on success, non-zero on failure; the message is then
 *     available from iqmm_last_error() on the calling thread;
 *   - an absent array (biases, indices) is a zeroed iqmm_array
 *     (data == NULL, ndim == 0), like a zeroed mlx_array (ops.rs:663-666);
 *   - group_size / bits are optionals (iqmm_optional_int == mlx_optional_int,
 *     ops.rs:633-644); mode is a NUL-terminated string:
 *     "affine" | "mxfp4" | "mxfp8" | "nvfp4".
 *
 * Memory: every `data` pointer is device memory on the current HIP device,
 * C-contiguous, row-major.  Results are written into caller-allocated
 * buffers: call once with res->data == NULL to have the library fill in
 * res->shape / res->ndim / res->dtype (nothing is launched), allocate, and
 * call again.  With res->data != NULL the described shape and dtype must equal
 * the inferred ones.  Inputs are never modified or freed.  Work is enqueued on
 * `stream` (a hipStream_t; NULL = the null stream) and is complete after the
 * stream is synchronised, as after mlx's `eval` (mlx/src/array.rs:111-113).
 * Scratch memory: the fp32 partial sums of a split-K GEMM (few output tiles,
 * M > 64), the gate_up product of a fused SwiGLU outside its fused kernels,
 * the expert segment offsets of a sorted grouped gather_qmm, the per-block
 * bucket counts of iqmm_moe_sort and the widened codes of a 2 / 3 / 5 / 6-bit
 * weight at M > 64 (N K / 2 or N K bytes) live in per-stream workspaces: one
 * grow-only buffer per (device, stream, use), taken from the stream-ordered
 * pool (hipMallocAsync on `stream`) and kept until the process ends, so HIP
 * graphs captured on a stream keep valid pointers and hold kernel nodes only.
 * Nothing is allocated while `stream` is capturing: a call whose workspace
 * would have to grow then fails with a message saying so.  Size the
 * workspaces before capture by running the same calls once on the capture
 * stream, or with iqmm_workspace_reserve.  Calls are re-entrant across
 * streams; calls on one stream execute in order and share its workspaces, so
 * a graph must not be replayed concurrently with other library work on the
 * stream it was captured on, nor with another graph captured on that stream.
 */
#ifndef IQMM_H
#define IQMM_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IQMM_MAX_NDIM 8

/* element types (subset of mlx_dtype that the quantized path uses) */
typedef enum iqmm_dtype {
  IQMM_FLOAT32 = 0,
  IQMM_FLOAT16 = 1,
  IQMM_BFLOAT16 = 2,
  IQMM_UINT32 = 3,
  IQMM_UINT8 = 4,
  IQMM_INT32 = 5,
  IQMM_INT64 = 6
} iqmm_dtype;

/* == mlx_optional_int (mlx/src/ops.rs:633-644) */
typedef struct iqmm_optional_int {
  int value;
  bool has_value;
} iqmm_optional_int;

/* == mlx_optional_dtype (mlx/src/ops.rs:668-671) */
typedef struct iqmm_optional_dtype {
  iqmm_dtype value;
  bool has_value;
} iqmm_optional_dtype;

/* array view: device pointer + shape + dtype (stands in for mlx_array) */
typedef struct iqmm_array {
  void* data;
  int64_t shape[IQMM_MAX_NDIM];
  int32_t ndim;
  int32_t dtype; /* iqmm_dtype */
} iqmm_array;

typedef void* iqmm_stream; /* hipStream_t */

/*
 * out = x @ dequantize(w, scales, biases)^T   (transpose = true)
 * out = x @ dequantize(w, scales, biases)     (transpose = false)
 * Replaces mlx_quantized_matmul (mlx/src/ops.rs:695-727).
 *   x       [..., M, K]  float32 | float16 | bfloat16
 *   w       [..., N, K*bits/32] uint32 (transpose) or [..., K, N*bits/32]
 *   scales  [..., N, K/gs] (affine: x's dtype; fp modes: uint8)
 *   biases  same as scales for affine; absent for mxfp4/mxfp8/nvfp4
 *   out     broadcast(x batch, w batch) + [M, N], x's dtype
 * Defaults: affine gs=64 bits=4; mxfp4 32/4; mxfp8 32/8; nvfp4 16/4.
 * Affine supports bits in {2,3,4,5,6,8} and gs in {32,64,128}.
 */
int iqmm_quantized_matmul(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                          iqmm_array biases, bool transpose, iqmm_optional_int group_size,
                          iqmm_optional_int bits, const char* mode, iqmm_stream stream);

/*
 * Unpack and rescale w to floating point.  Replaces mlx_dequantize
 * (mlx/src/ops.rs:653-686).  Output [..., rows, K] in `dtype` when given,
 * else the scales' dtype (affine) or bfloat16 (fp modes).  Bit-exact:
 * affine w = round(fp32(fp32(s*q) + b)); fp modes w = round(elem * scale).
 */
int iqmm_dequantize(iqmm_array* res, iqmm_array w, iqmm_array scales, iqmm_array biases,
                    iqmm_optional_int group_size, iqmm_optional_int bits, const char* mode,
                    iqmm_optional_dtype dtype, iqmm_stream stream);

/*
 * Indexed batched quantized matmul (MoE experts).  Replaces mlx_gather_qmm,
 * i.e. the host loop of mlx/src/nn/moe.rs:84-170 over the stacked expert
 * tensors built in mlx/src/model/qwen35.rs:653-775.
 *   x            [..., M, K]            (batch B_x = prod of leading dims)
 *   w            [..., N, K*bits/32]    (batch B_w, typically [E, N, Kp])
 *   lhs_indices  integer array into x's flattened batch (absent: arange)
 *   rhs_indices  integer array into w's flattened batch (absent: arange)
 *   out          broadcast(lhs.shape, rhs.shape) + [M, N]
 *   out[i] = x[lhs[i]] @ dequantize(w[rhs[i]])^T
 * sorted_indices = true promises rhs_indices (flattened) is non-decreasing;
 * the library then runs one grouped pass per expert.
 */
int iqmm_gather_qmm(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                    iqmm_array biases, iqmm_array lhs_indices, iqmm_array rhs_indices,
                    bool transpose, iqmm_optional_int group_size, iqmm_optional_int bits,
                    const char* mode, bool sorted_indices, iqmm_stream stream);

/*
 * Quantize w [..., rows, K] (float32/float16/bfloat16) along its last axis.
 * Replaces mlx_quantize.  res_w: uint32 [..., rows, K*bits/32];
 * res_scales: [..., rows, K/gs] in w's dtype (affine) or uint8 (fp modes);
 * res_biases: affine only (pass NULL for fp modes).
 */
int iqmm_quantize(iqmm_array* res_w, iqmm_array* res_scales, iqmm_array* res_biases,
                  iqmm_array w, iqmm_optional_int group_size, iqmm_optional_int bits,
                  const char* mode, iqmm_stream stream);

/*
 * Fused SwiGLU over a gate_up weight: w [..., 2I, K*bits/32] holds the gate
 * rows [0, I) then the up rows [I, 2I) (the fused `gate_up_proj` layout of
 * mlx/src/model/qwen35.rs:653-658; a Llama gate_proj / up_proj pair stacked
 * along rows).  out [..., M, I] = silu(x @ gate^T) * (x @ up^T), rounded as
 * the unfused composition of mlx/src/nn/mlp.rs:27-33 rounds it (gate and up
 * stored in x's dtype, then sigmoid, the silu product and the up product each
 * rounded).  Replaces the gate / up quantized_matmul pair plus silu and
 * multiply in MLP::forward_with_stream (mlx/src/nn/mlp.rs:27-33).  transpose
 * is implied (true); other arguments as iqmm_quantized_matmul.
 */
int iqmm_quantized_swiglu(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                          iqmm_array biases, iqmm_optional_int group_size, iqmm_optional_int bits,
                          const char* mode, iqmm_stream stream);

/*
 * gather_qmm over stacked gate_up experts w [E, 2I, K*bits/32] followed by
 * the SwiGLU of iqmm_quantized_swiglu: out [..., M, I].  Replaces the gate /
 * up products and silu * up of each Expert (mlx/src/nn/moe.rs:10-33) inside
 * the per-expert loop of mlx/src/nn/moe.rs:117-143.  Index arguments as
 * iqmm_gather_qmm.
 */
int iqmm_gather_qmm_swiglu(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                           iqmm_array biases, iqmm_array lhs_indices, iqmm_array rhs_indices,
                           iqmm_optional_int group_size, iqmm_optional_int bits, const char* mode,
                           bool sorted_indices, iqmm_stream stream);

/*
 * Row gather of a quantized table: out[i, :] = dequantize(w)[indices[i], :]
 * without dequantizing the table.  Replaces dequantize + take_axis in
 * QuantizedEmbedding::forward (mlx/src/nn/embedding.rs:62-72).
 *   w [rows, K*bits/32], scales / biases [rows, K/gs] as iqmm_dequantize
 *   indices: integer array of any shape; negative values count from the end
 *   out indices.shape + [K], dtype as iqmm_dequantize (bit-identical rows)
 * Indices outside [-rows, rows) give NaN rows.
 */
int iqmm_dequantize_rows(iqmm_array* res, iqmm_array w, iqmm_array scales, iqmm_array biases,
                         iqmm_array indices, iqmm_optional_int group_size, iqmm_optional_int bits,
                         const char* mode, iqmm_optional_dtype dtype, iqmm_stream stream);

/*
 * MoE router on the device: softmax over the experts of each token, top-k,
 * optional normalisation.  Replaces mlx/src/nn/moe.rs:67-82 and the host
 * read-back of :86-90.
 *   logits       [T, E] float32 | float16 | bfloat16
 *   res_scores   [T, k] float32: the selected probabilities (stored in the
 *                logits' dtype, as MLX's softmax output is) or, with
 *                norm_topk_prob, p / sum(p of the k) rounded to that dtype
 *   res_experts  [T, k] int32: experts by descending probability, ties to the
 *                lower index (a stable argsort of -p, as moe.rs:72-73)
 * 1 <= k <= min(E, 32), E <= 2048.
 */
int iqmm_moe_route(iqmm_array* res_scores, iqmm_array* res_experts, iqmm_array logits, int k,
                   bool norm_topk_prob, iqmm_stream stream);

/*
 * Stable sort of the (token, slot) rows of a routing by expert, producing the
 * sorted_indices form of iqmm_gather_qmm.  Replaces the per-expert token lists
 * of mlx/src/nn/moe.rs:92-104.
 *   experts          [T, k] int32 (n = T*k rows, row r = t*k + slot)
 *   res_tokens       [n] int32: token of each sorted row (gather_qmm lhs_indices)
 *   res_sorted       [n] int32: expert of each sorted row (rhs_indices);
 *                    ids outside [0, num_experts) sort last
 *   res_inverse      [n] int32: sorted position of row r
 *   res_offsets      [num_experts + 1] int32: first sorted row of each expert,
 *                    offsets[num_experts] = number of valid rows (may be a
 *                    NULL pointer to skip)
 * n <= 32768.
 */
int iqmm_moe_sort(iqmm_array* res_tokens, iqmm_array* res_sorted, iqmm_array* res_inverse,
                  iqmm_array* res_offsets, iqmm_array experts, int num_experts, iqmm_stream stream);

/*
 * iqmm_moe_sort with no allocation: the same arguments, results and limits,
 * bit-identical output.  No counterpart in the reference or mlx-c; it is for
 * callers that cannot allocate device memory (code under HIP graph capture on
 * a stream whose workspaces were never sized, tight serving loops, harnesses
 * that forbid hipMalloc).  The counting sort's (bucket, block) counts,
 * (num_experts + 1) * ceil(n / 256) int32, live in one fixed per-device array
 * of 15872 int32 (62 KiB, held until the process ends); a routing that needs
 * more takes the one-workgroup bitonic sort, which uses no scratch, and
 * n > 32768 is rejected as by iqmm_moe_sort.  Calls on one GPU share that
 * array: two calls that overlap in time on one GPU (different streams, or
 * graphs replayed concurrently) race on it.
 */
int iqmm_moe_sort_noalloc(iqmm_array* res_tokens, iqmm_array* res_sorted, iqmm_array* res_inverse,
                          iqmm_array* res_offsets, iqmm_array experts, int num_experts,
                          iqmm_stream stream);

/*
 * Weighted combine of expert outputs: out[t, :] = sum over the k slots of t,
 * in ascending expert order, of float32(y[inverse[t*k + slot], :]) * score,
 * accumulated sequentially in float32 as mlx/src/nn/moe.rs:146-168 does.
 *   y        [n, D] (or [n, 1, D]) float32 | float16 | bfloat16 expert rows in
 *            any order (sorted by iqmm_moe_sort, or one row per (token, slot))
 *   inverse  [T, k] or [n] int32: the row of y of each (token, slot)
 *            (iqmm_moe_sort's inverse, or 0 .. n-1 for unsorted rows)
 *   experts  [T, k] int32, scores [T, k] float32 from iqmm_moe_route
 *   res      [T, D] float32
 * Slots whose expert is outside [0, num_experts) are skipped, as the
 * reference skips them (moe.rs:99); a token with none gets a zero row.
 */
int iqmm_moe_combine(iqmm_array* res, iqmm_array y, iqmm_array inverse, iqmm_array experts,
                     iqmm_array scores, int num_experts, iqmm_stream stream);

/*
 * One token's routed experts in two launches: the routing of
 * iqmm_moe_route, the fused gate_up SwiGLU of each routed expert
 * (iqmm_gather_qmm_swiglu over the token's k rows) and the down projections
 * with the ordered weighted combine of iqmm_moe_combine.  Replaces, for a
 * single decode token, the per-expert loop of mlx/src/nn/moe.rs:55-183
 * (route :67-82, experts :92-143, combine :146-168); mlx-c has no fused
 * counterpart, so a binding calls it where the block would otherwise run
 * route + gather + gather + combine for T = 1.
 *   logits           [1, E] (or [E]) float32 | float16 | bfloat16
 *   x                [1, H] bfloat16 | float16
 *   gate_up_*        [E, 2I, H/8] uint32, scales / biases [E, 2I, H/gs] in x's
 *                    dtype (gate rows first, as stacked by the checkpoint)
 *   down_*           [E, D, I/8] uint32, scales / biases [E, D, I/gs]
 *   res              [1, D] float32
 * Affine 4-bit only; E <= 512, 1 <= k <= min(E, 32), H in [32, 8192] and
 * I in [32, 2048] multiples of 32 and of the group size (32, 64 or 128).
 * Uses a per-stream workspace of k * I * 2 + 256 bytes (sized beforehand for
 * graph capture, as the other calls' workspaces).
 */
int iqmm_moe_token(iqmm_array* res, iqmm_array logits, iqmm_array x, iqmm_array gate_up_w,
                   iqmm_array gate_up_scales, iqmm_array gate_up_biases, iqmm_array down_w,
                   iqmm_array down_scales, iqmm_array down_biases, int k, bool norm_topk_prob,
                   int group_size, int bits, iqmm_stream stream);

/* Message of the last failed call on this thread ("" if none). */
const char* iqmm_last_error(void);

/*
 * Grow every workspace of `stream` (on the current device) to at least
 * `bytes`, outside graph capture, so that later captured calls on that stream
 * need no allocation.  No counterpart in mlx-c (MLX allocates per array); it
 * is for callers that capture the library's calls into HIP graphs.
 */
int iqmm_workspace_reserve(iqmm_stream stream, size_t bytes);

/* Library version string, e.g. "iqmm 0.1 gfx950". */
const char* iqmm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* IQMM_H */
