// launch.h — host-side launch interface between the C-ABI dispatcher
// (api.hip) and the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace iqmm {

// One quantized-matmul problem: out[b] = x[xb(b)] (M x K) . W[wb(b)]^T (or W).
struct QmmArgs {
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;  // biases (affine) or nullptr
  void* out;
  int M, N, K;
  int gs, bits, mode, xdt;
  bool transpose;
  int64_t x_mat;  // elements per x matrix (M*K)
  int64_t w_mat;  // uint32 words per w matrix
  int64_t s_mat;  // scale entries per w matrix
  int64_t nbatch;
  BatchMap bm;
  hipStream_t stream;
  // fused SwiGLU (qmv_q4 only): w holds 2N rows, gate [0, N) and up [N, 2N);
  // out[:, n] = silu(x . gate_n) * (x . up_n)
  int glu;
};

// Dequantize / quantize problems over `rows` rows of K values.
struct ConvArgs {
  const uint32_t* w;  // packed (dequantize input)
  const void* s;
  const void* b;
  void* out;          // dequantize output
  const void* src;    // quantize input
  uint32_t* wq;       // quantize outputs
  void* sq;
  void* bq;
  int64_t rows;       // rows produced (dequantize) or quantized
  int K, gs, bits, mode, sdt, odt;
  hipStream_t stream;
  const void* idx;    // dequantize row gather: table row of each output row, or nullptr
  int idx_dt;         // I32 / U32 / I64
  int64_t table_rows; // rows of the packed table (index bound)
};

hipError_t launch_qmv(const QmmArgs& a);        // transpose=true, small M, VALU
hipError_t launch_qmv_q4_m1(const QmmArgs& a);  // 4-bit affine M=1 decode fast path
bool qmv_q4_m1_supported(const QmmArgs& a);
hipError_t launch_qmv_q8_m1(const QmmArgs& a);  // 8-bit affine / mxfp8 M=1 decode path
bool qmv_q8_m1_supported(const QmmArgs& a);
hipError_t launch_qmv_lb_m1(const QmmArgs& a);  // affine 2 / 3 / 6-bit M=1 decode path
bool qmv_lb_m1_supported(const QmmArgs& a);
hipError_t launch_qvm(const QmmArgs& a);        // transpose=false, small M, VALU
hipError_t launch_qmm_mfma(const QmmArgs& a);   // bf16/fp16 MFMA tiles, any M
bool qmm_mfma_supported(const QmmArgs& a);
hipError_t launch_qmm_gemm(const QmmArgs& a);   // 256x256 prefill GEMM
hipError_t launch_qmm_skinny(const QmmArgs& a); // decode widths 2 <= M <= 64
bool qmm_skinny_supported(const QmmArgs& a);
// factored affine 4-bit MFMA kernel for decode widths (x rows <= 4 m tiles, <= 32)
hipError_t launch_qmm_skinny_fac(const QmmArgs& a);
bool qmm_skinny_fac_supported(const QmmArgs& a);
// affine 4-bit decode widths (M <= 32) on MFMA, scales read once per wave range
hipError_t launch_qmm_decode(const QmmArgs& a);
bool qmm_decode_supported(const QmmArgs& a);
// grouped gather_qmm with the decode kernel's factored arithmetic (affine 4-bit)
hipError_t launch_gather_decode(const QmmArgs& a, int64_t nflat, int64_t E, const int64_t* off);
bool gather_decode_supported(const QmmArgs& a);
hipError_t launch_gather_stream(const QmmArgs& a, int64_t nflat, int64_t E);  // finds its own row segments
bool gather_stream_supported(const QmmArgs& a);
// sorted-expert grouped gather_qmm: nflat batch elements, E experts
hipError_t launch_gather_sorted(const QmmArgs& a, int64_t nflat, int64_t E);
bool gather_sorted_supported(const QmmArgs& a);
// with glu: the weight holds 2N rows per expert, out[., n] = silu(gate_n) * up_n
bool gather_sorted_glu_supported(const QmmArgs& a);
bool qmm_gemm_supported(const QmmArgs& a);
hipError_t launch_dequantize(const ConvArgs& a);
hipError_t launch_quantize(const ConvArgs& a);
// float16 / bfloat16 -> float32 copy (mixed-dtype calls)
hipError_t launch_cast_f32(const void* src, int sdt, float* dst, int64_t n, hipStream_t st);
// SwiGLU over a [rows, 2N] product (gate | up halves) -> [rows, N]
hipError_t launch_swiglu_rows(const void* gu, void* out, int64_t rows, int64_t n, int dt,
                              hipStream_t st);
// MoE routing: softmax / top-k, the stable sort by expert, the weighted combine
hipError_t launch_moe_route(const void* logits, int dt, float* scores, int32_t* experts, int T, int E, int k,
                            bool norm, hipStream_t st);
hipError_t launch_moe_sort(const int32_t* experts, int n, int k, int E, int32_t* tokens, int32_t* sorted,
                           int32_t* inverse, int32_t* offsets, hipStream_t st);
// the same sort with its bucket counts in a fixed per-device array (allocates nothing)
hipError_t launch_moe_sort_noalloc(const int32_t* experts, int n, int k, int E, int32_t* tokens, int32_t* sorted,
                                   int32_t* inverse, int32_t* offsets, hipStream_t st);
// decode widths on wide matrices, streaming tile-blocks per CU (qmm_stream.hip)
bool qmm_stream_supported(const QmmArgs& a);
hipError_t launch_qmm_stream(const QmmArgs& a);
// one token's MoE experts (route + fused gate_up SwiGLU + down + combine),
// affine 4-bit (moe.hip)
bool moe_token_supported(int E, int k, int H, int I, int D, int gs);
hipError_t launch_moe_token(const void* logits, int lt, const void* x, int xt, const uint32_t* gw, const void* gsc,
                            const void* gbi, const uint32_t* dw, const void* dsc, const void* dbi, int E, int k,
                            bool norm, int H, int I, int D, int gs, float* out, hipStream_t st);
hipError_t launch_moe_combine(const void* y, int dt, const int32_t* inverse, const int32_t* experts,
                              const float* scores, float* out, int T, int k, int64_t D, int E, int64_t n,
                              hipStream_t st);
// Scratch of one call: the (device, stream, slot) buffer, grown outside
// capture; during capture a request larger than the buffer fails with
// hipErrorStreamCaptureUnsupported (nothing is allocated inside a graph).
enum WsSlot : int { WS_SPLITK = 0, WS_GLU = 1, WS_OFFSETS = 2, WS_SORT = 3, WS_CONV = 4, WS_MOE = 5, WS_CODES = 6, WS_NSLOTS = 7 };
hipError_t workspace_get(hipStream_t st, int slot, size_t bytes, void** p);
// grow every slot of the stream to at least `bytes` (outside capture)
hipError_t workspace_reserve(hipStream_t st, size_t bytes);

}  // namespace iqmm
