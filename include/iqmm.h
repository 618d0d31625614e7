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
 * The library's only device allocation is the fp32 partial-sum workspace of a
 * split-K GEMM (few output tiles, M > 64), taken with hipMallocAsync and
 * released with hipFreeAsync on `stream`, so it is stream-ordered and may be
 * captured in a HIP graph.  Calls are re-entrant; calls on one stream execute
 * in order.
 */
#ifndef IQMM_H
#define IQMM_H

#include <stdbool.h>
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

/* Message of the last failed call on this thread ("" if none). */
const char* iqmm_last_error(void);

/* Library version string, e.g. "iqmm 0.1 gfx950". */
const char* iqmm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* IQMM_H */
