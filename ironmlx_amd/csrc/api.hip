// api.hip — the C ABI (include/iqmm.h): argument validation, shape inference
// and kernel dispatch.
//
// Validation mirrors what mlx-c's quantized ops reject so that callers see the
// same failures the Rust wrappers turn into Error::Mlx (mlx/src/error.rs:27-35):
// unknown mode, unsupported bits / group size, dtype mismatches, shapes whose
// packed width does not match K, scales of the wrong shape, missing or
// unexpected biases, and batch shapes that do not broadcast.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/iqmm.h"
#include "launch.h"

namespace iqmm {
namespace {

thread_local std::string g_last_error;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return 1;
}

int hip_fail(const char* op, hipError_t e) {
  if (e == hipErrorStreamCaptureUnsupported)
    return fail("[%s] the stream's workspace is too small for this call during graph capture (nothing is "
                "allocated while capturing): run the same call once on this stream before capturing, or "
                "call iqmm_workspace_reserve on it.", op);
  return fail("[%s] HIP error: %s", op, hipGetErrorString(e));
}

bool present(const iqmm_array& a) { return a.data != nullptr || a.ndim > 0; }

bool is_float(int dt) { return dt == IQMM_FLOAT32 || dt == IQMM_FLOAT16 || dt == IQMM_BFLOAT16; }
bool is_index(int dt) { return dt == IQMM_INT32 || dt == IQMM_UINT32 || dt == IQMM_INT64; }

const char* dt_name(int dt) {
  switch (dt) {
    case IQMM_FLOAT32: return "float32";
    case IQMM_FLOAT16: return "float16";
    case IQMM_BFLOAT16: return "bfloat16";
    case IQMM_UINT32: return "uint32";
    case IQMM_UINT8: return "uint8";
    case IQMM_INT32: return "int32";
    case IQMM_INT64: return "int64";
  }
  return "unknown";
}

int64_t numel(const iqmm_array& a) {
  int64_t n = 1;
  for (int i = 0; i < a.ndim; ++i) n *= a.shape[i];
  return n;
}

std::string shape_str(const iqmm_array& a) {
  std::string s = "(";
  for (int i = 0; i < a.ndim; ++i) {
    s += std::to_string(a.shape[i]);
    if (i + 1 < a.ndim) s += ",";
  }
  return s + ")";
}

struct QParams {
  int mode, gs, bits;
};

// mode string + optionals -> resolved (mode, gs, bits); MLX's defaults per mode
int resolve(const char* op, const char* mode, iqmm_optional_int group_size, iqmm_optional_int bits,
            QParams& q) {
  if (!mode) mode = "affine";
  int dgs, dbits;
  if (!strcmp(mode, "affine")) { q.mode = AFFINE; dgs = 64; dbits = 4; }
  else if (!strcmp(mode, "mxfp4")) { q.mode = MXFP4; dgs = 32; dbits = 4; }
  else if (!strcmp(mode, "mxfp8")) { q.mode = MXFP8; dgs = 32; dbits = 8; }
  else if (!strcmp(mode, "nvfp4")) { q.mode = NVFP4; dgs = 16; dbits = 4; }
  else return fail("[%s] Invalid quantization mode '%s'.", op, mode);
  q.gs = group_size.has_value ? group_size.value : dgs;
  q.bits = bits.has_value ? bits.value : dbits;
  if (q.mode == AFFINE) {
    if (q.gs != 32 && q.gs != 64 && q.gs != 128)
      return fail("[%s] The requested group size %d is not supported. The supported group sizes are 32, 64, and 128.", op, q.gs);
    if (q.bits != 2 && q.bits != 3 && q.bits != 4 && q.bits != 5 && q.bits != 6 && q.bits != 8)
      return fail("[%s] The requested number of bits %d is not supported. The supported bits are 2, 3, 4, 5, 6 and 8.", op, q.bits);
  } else {
    if (q.gs != dgs)
      return fail("[%s] Quantization mode '%s' requires group_size %d (got %d).", op, mode, dgs, q.gs);
    if (q.bits != dbits)
      return fail("[%s] Quantization mode '%s' requires bits %d (got %d).", op, mode, dbits, q.bits);
  }
  return 0;
}

// scales / biases checks shared by every op; rows_shape = w.shape[:-1]
int check_scales(const char* op, const QParams& q, const iqmm_array& w, const iqmm_array& s,
                 const iqmm_array& b, int64_t groups_last, int* sdt_out) {
  if (!present(s) || s.ndim != w.ndim)
    return fail("[%s] scales must have the same number of dimensions as w (%d), got %s.", op, w.ndim, shape_str(s).c_str());
  for (int i = 0; i + 1 < w.ndim; ++i)
    if (s.shape[i] != w.shape[i])
      return fail("[%s] Shape of scales %s does not match w %s.", op, shape_str(s).c_str(), shape_str(w).c_str());
  if (s.shape[s.ndim - 1] != groups_last)
    return fail("[%s] scales last dimension %lld does not match the expected number of groups %lld.", op,
                (long long)s.shape[s.ndim - 1], (long long)groups_last);
  if (q.mode == AFFINE) {
    if (!is_float(s.dtype)) return fail("[%s] affine scales must be floating point, got %s.", op, dt_name(s.dtype));
    if (!present(b)) return fail("[%s] Biases must be provided for affine quantization.", op);
    if (b.dtype != s.dtype || b.ndim != s.ndim)
      return fail("[%s] biases must have the same shape and dtype as scales.", op);
    for (int i = 0; i < s.ndim; ++i)
      if (b.shape[i] != s.shape[i]) return fail("[%s] biases must have the same shape and dtype as scales.", op);
  } else {
    if (s.dtype != IQMM_UINT8) return fail("[%s] Scales for mode with fp elements must be uint8, got %s.", op, dt_name(s.dtype));
    if (present(b)) return fail("[%s] Biases must not be provided for quantization mode other than affine.", op);
  }
  *sdt_out = s.dtype;
  return 0;
}

// right-aligned broadcast of two batch shapes; strides are in matrices
int broadcast2(const char* op, const int64_t* a, int na, const int64_t* b, int nb, BatchMap& bm,
               std::vector<int64_t>& out_shape) {
  const int nd = na > nb ? na : nb;
  if (nd > 8) return fail("[%s] too many batch dimensions (%d).", op, nd);
  out_shape.assign(nd, 1);
  int64_t sa = 1, sb = 1;
  std::vector<int64_t> sta(nd, 0), stb(nd, 0);
  for (int d = nd - 1; d >= 0; --d) {
    const int ia = d - (nd - na), ib = d - (nd - nb);
    const int64_t da = ia >= 0 ? a[ia] : 1, db = ib >= 0 ? b[ib] : 1;
    if (da != db && da != 1 && db != 1)
      return fail("[%s] Shapes cannot be broadcast: batch dims do not match.", op);
    out_shape[d] = da == 1 ? db : da;
    sta[d] = da == 1 ? 0 : sa;
    stb[d] = db == 1 ? 0 : sb;
    sa *= da;
    sb *= db;
  }
  bm.ndim = nd;
  for (int d = 0; d < nd; ++d) {
    bm.shape[d] = out_shape[d];
    bm.xs[d] = sta[d];
    bm.ws[d] = stb[d];
  }
  return 0;
}

int set_or_check_res(const char* op, iqmm_array* res, const std::vector<int64_t>& shape, int dtype,
                     bool* query) {
  if (!res) return fail("[%s] result pointer is null.", op);
  if ((int)shape.size() > IQMM_MAX_NDIM) return fail("[%s] result has too many dimensions.", op);
  if (res->data == nullptr) {
    res->ndim = static_cast<int32_t>(shape.size());
    for (size_t i = 0; i < shape.size(); ++i) res->shape[i] = shape[i];
    res->dtype = dtype;
    *query = true;
    return 0;
  }
  *query = false;
  bool okk = res->ndim == (int)shape.size() && res->dtype == dtype;
  for (size_t i = 0; okk && i < shape.size(); ++i) okk = res->shape[i] == shape[i];
  if (!okk) {
    std::string want = "(";
    for (size_t i = 0; i < shape.size(); ++i) want += std::to_string(shape[i]) + (i + 1 < shape.size() ? "," : "");
    want += ")";
    return fail("[%s] result buffer is %s %s but the op produces %s %s.", op, shape_str(*res).c_str(),
                dt_name(res->dtype), want.c_str(), dt_name(dtype));
  }
  return 0;
}

__global__ void fill_kernel(uint16_t* p16, float* p32, int64_t n, uint16_t v16, float v32) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) {
    if (p16) p16[i] = v16;
    else p32[i] = v32;
  }
}

hipError_t fill_zero(void* p, int dt, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int64_t nb = (n + 255) / 256;
  hipLaunchKernelGGL(fill_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, st,
                     dt == IQMM_FLOAT32 ? nullptr : static_cast<uint16_t*>(p),
                     dt == IQMM_FLOAT32 ? static_cast<float*>(p) : nullptr, n, uint16_t(0), 0.f);
  return hipGetLastError();
}

// choose the kernel family for one problem
hipError_t run_qmm(QmmArgs& a) {
  // M = 2 / 3 on wide matrices: the streaming MFMA kernel is ahead of the
  // multi-row GEMV (K = 4096: N = 14336, M = 2 / 3: 13.1 / 17.1 -> 10.9 /
  // 10.9 us; N = 6144, M = 3: 8.6 -> 7.2 us; not at N = 6144, M = 2)
  if (a.M >= 2 && a.M <= 3 && (a.M == 3 || a.N >= 10240) && qmm_stream_supported(a)) return launch_qmm_stream(a);
  if (qmv_q4_m1_supported(a)) return launch_qmv_q4_m1(a);
  if (qmv_q8_m1_supported(a)) return launch_qmv_q8_m1(a);
  if (qmv_lb_m1_supported(a)) return launch_qmv_lb_m1(a);
  // decode widths on the MFMA decode kernel; M = 2 / 3 only for long K, where
  // the split-K skinny kernel is slow (N = 4096, K = 14336, M = 2: 20.4 us ->
  // the decode kernel's ~14 us at M = 4), while at K = 4096 it stays ahead
  if (a.M >= 4 && qmm_stream_supported(a)) return launch_qmm_stream(a);
  if ((a.M >= 4 || a.K >= 8192) && qmm_decode_supported(a)) return launch_qmm_decode(a);
  if (a.nbatch <= 65535 && qmm_skinny_fac_supported(a)) return launch_qmm_skinny_fac(a);
  if (a.M >= 2 && a.M <= 64 && a.nbatch * ((a.M + 31) / 32) <= 65535 && qmm_skinny_supported(a))
    return launch_qmm_skinny(a);
  if (a.M > 64 && a.nbatch <= 65535 && qmm_gemm_supported(a)) return launch_qmm_gemm(a);
  const bool small_m = a.M <= 8;
  if (!small_m && qmm_mfma_supported(a)) return launch_qmm_mfma(a);
  return a.transpose ? launch_qmv(a) : launch_qvm(a);
}

int elt_size(int dt) { return dt == IQMM_FLOAT32 ? 4 : 2; }

// Fused SwiGLU over a gate_up weight of 2I rows (a.N = I outputs): the M = 1
// GEMV reduces each gate row and its up row in one wave, and the factored
// decode kernel (M <= 32) pairs a gate tile with its up tile in one
// workgroup; both apply the SwiGLU in their epilogue.  Every other shape
// computes the [.., M, 2I] product
// into a stream-ordered workspace with the regular kernels (`product`) and
// then runs the elementwise SwiGLU over it (the product lives in the
// stream's GLU workspace, workspace.hip).
template <class F>
hipError_t run_glu(QmmArgs& a, bool try_fused, F&& product) {
  a.glu = 1;
  if (try_fused && qmv_q4_m1_supported(a)) return launch_qmv_q4_m1(a);
  // (M = 2 / 3 at 2 x 14336 rows: 22.1 -> 19.3 us against the decode kernel)
  if (try_fused && a.M >= 2 && qmm_stream_supported(a)) return launch_qmm_stream(a);
  if (try_fused && a.M >= 2 && qmm_decode_supported(a)) return launch_qmm_decode(a);
  if (try_fused && a.nbatch <= 65535 && qmm_skinny_fac_supported(a)) return launch_qmm_skinny_fac(a);
  a.glu = 0;
  const int64_t I = a.N, rows = a.nbatch * a.M;
  void* out = a.out;
  void* ws = nullptr;
  hipError_t e = workspace_get(a.stream, WS_GLU, static_cast<size_t>(rows) * 2 * I * elt_size(a.xdt), &ws);
  if (e != hipSuccess) return e;
  a.N = static_cast<int>(2 * I);
  a.out = ws;
  e = product(a);
  if (e == hipSuccess) e = launch_swiglu_rows(ws, out, rows, I, a.xdt, a.stream);
  a.N = static_cast<int>(I);
  a.out = out;
  return e;
}

// common core of quantized_matmul / gather_qmm once batch mapping is known
int qmm_common(const char* op, iqmm_array* res, const iqmm_array& x, const iqmm_array& w,
               const iqmm_array& s, const iqmm_array& b, bool transpose, const QParams& q,
               int64_t& M, int64_t& N, int64_t& K, int* sdt) {
  if (!present(x) || x.ndim < 1) return fail("[%s] x must have at least one dimension.", op);
  if (!is_float(x.dtype)) return fail("[%s] Only real floating types are supported but x.dtype() == %s.", op, dt_name(x.dtype));
  if (!present(w) || w.ndim < 2) return fail("[%s] The quantized weight should be at least 2D but received %s.", op, shape_str(w).c_str());
  if (w.dtype != IQMM_UINT32) return fail("[%s] The weight matrix should be uint32 but received %s.", op, dt_name(w.dtype));
  K = x.shape[x.ndim - 1];
  M = x.ndim >= 2 ? x.shape[x.ndim - 2] : 1;
  const int64_t wlast = w.shape[w.ndim - 1], wrows = w.shape[w.ndim - 2];
  if ((wlast * 32) % q.bits != 0)
    return fail("[%s] packed width %lld is not a whole number of %d-bit codes.", op, (long long)wlast, q.bits);
  const int64_t unpacked = wlast * 32 / q.bits;
  if (transpose) {
    if (unpacked != K)
      return fail("[%s] Last dimension of first input with shape (..., %lld) must be equal to the unpacked last dimension of the quantized weight (%lld).",
                  op, (long long)K, (long long)unpacked);
    N = wrows;
    if (K % q.gs != 0) return fail("[%s] K=%lld is not divisible by group_size %d.", op, (long long)K, q.gs);
    if (check_scales(op, q, w, s, b, K / q.gs, sdt)) return 1;
  } else {
    if (wrows != K)
      return fail("[%s] Last dimension of first input with shape (..., %lld) must be equal to the second-to-last dimension of the weight (%lld).",
                  op, (long long)K, (long long)wrows);
    N = unpacked;
    if (N % q.gs != 0) return fail("[%s] N=%lld is not divisible by group_size %d.", op, (long long)N, q.gs);
    if (check_scales(op, q, w, s, b, N / q.gs, sdt)) return 1;
    if (N % 32 != 0) return fail("[%s] transpose=false requires the output width (%lld) to be a multiple of 32.", op, (long long)N);
  }
  if (K % 32 != 0) return fail("[%s] The reduction dimension K=%lld must be a multiple of 32.", op, (long long)K);
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL) return fail("[%s] dimension too large.", op);
  (void)res;
  return 0;
}

int moe_sort_entry(const char* op, bool noalloc, iqmm_array* res_tokens, iqmm_array* res_sorted,
                   iqmm_array* res_inverse, iqmm_array* res_offsets, iqmm_array experts, int num_experts,
                   iqmm_stream stream) {
  g_last_error.clear();
  if (!present(experts) || experts.ndim != 2 || experts.dtype != IQMM_INT32)
    return fail("[%s] experts must be a 2D int32 array [tokens, k], got %s %s.", op, shape_str(experts).c_str(),
                dt_name(experts.dtype));
  if (num_experts < 1 || num_experts > 65535) return fail("[%s] num_experts must be in [1, 65535], got %d.", op, num_experts);
  const int64_t n = numel(experts), k = experts.shape[1];
  if (n > 32768) return fail("[%s] at most 32768 (token, slot) rows are sorted in one call, got %lld.", op, (long long)n);
  const std::vector<int64_t> shp = {n}, oshp = {static_cast<int64_t>(num_experts) + 1};
  bool q1, q2, q3, q4 = false;
  if (set_or_check_res(op, res_tokens, shp, IQMM_INT32, &q1)) return 1;
  if (set_or_check_res(op, res_sorted, shp, IQMM_INT32, &q2)) return 1;
  if (set_or_check_res(op, res_inverse, shp, IQMM_INT32, &q3)) return 1;
  if (res_offsets && set_or_check_res(op, res_offsets, oshp, IQMM_INT32, &q4)) return 1;
  if (q1 || q2 || q3 || q4) {
    if (!(q1 && q2 && q3 && (!res_offsets || q4))) return fail("[%s] either all result buffers are allocated or none.", op);
    return 0;
  }
  if (n == 0) {
    if (!res_offsets) return 0;
    // int32 zeros have the bits of float32 zeros; a fill kernel (not a
    // memset node) keeps the call capturable in a HIP graph
    hipError_t e = fill_zero(res_offsets->data, IQMM_FLOAT32, static_cast<int64_t>(num_experts) + 1,
                             static_cast<hipStream_t>(stream));
    return e == hipSuccess ? 0 : hip_fail(op, e);
  }
  hipError_t e = (noalloc ? launch_moe_sort_noalloc : launch_moe_sort)(
      static_cast<const int32_t*>(experts.data), static_cast<int>(n), static_cast<int>(k), num_experts,
      static_cast<int32_t*>(res_tokens->data), static_cast<int32_t*>(res_sorted->data),
      static_cast<int32_t*>(res_inverse->data), res_offsets ? static_cast<int32_t*>(res_offsets->data) : nullptr,
      static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : hip_fail(op, e);
}

}  // namespace
}  // namespace iqmm

using namespace iqmm;

extern "C" {

const char* iqmm_last_error(void) { return g_last_error.c_str(); }

const char* iqmm_version(void) { return "iqmm 0.1 gfx950"; }

int iqmm_workspace_reserve(iqmm_stream stream, size_t bytes) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs);
  if (e != hipSuccess) return hip_fail("workspace_reserve", e);
  if (cs != hipStreamCaptureStatusNone)
    return fail("[workspace_reserve] the stream is capturing; reserve before capture.");
  e = workspace_reserve(static_cast<hipStream_t>(stream), bytes);
  return e != hipSuccess ? hip_fail("workspace_reserve", e) : 0;
}

}  // extern "C"

namespace iqmm {
namespace {
// MLX promotes x, scales and biases to one type before the product
// (result_type of x and scales, then the biases'): equal types stay, float32
// wins, and float16 with bfloat16 gives float32.  Every mixed affine call
// therefore computes in float32: x and / or the scales and biases are copied
// to float32 (exact) into the stream's conversion workspace.
int result_dtype(const QParams& q, int xdt, int sdt) {
  return (q.mode == AFFINE && sdt != xdt) ? IQMM_FLOAT32 : xdt;
}

hipError_t promote_inputs(QmmArgs& a, const iqmm_array& x, const iqmm_array& s, const iqmm_array& b, int sdt) {
  if (a.mode != AFFINE || sdt == x.dtype) return hipSuccess;
  const int64_t nx = x.dtype == IQMM_FLOAT32 ? 0 : numel(x), ns = sdt == IQMM_FLOAT32 ? 0 : numel(s);
  auto up = [](int64_t n) { return (n * 4 + 255) / 256 * 256; };
  void* ws = nullptr;
  hipError_t e = workspace_get(a.stream, WS_CONV, static_cast<size_t>(up(nx) + 2 * up(ns)), &ws);
  if (e != hipSuccess) return e;
  char* p = static_cast<char*>(ws);
  if (nx) {
    e = launch_cast_f32(x.data, x.dtype, reinterpret_cast<float*>(p), nx, a.stream);
    if (e != hipSuccess) return e;
    a.x = p;
    p += up(nx);
  }
  if (ns) {
    e = launch_cast_f32(s.data, sdt, reinterpret_cast<float*>(p), ns, a.stream);
    if (e != hipSuccess) return e;
    a.s = p;
    e = launch_cast_f32(b.data, sdt, reinterpret_cast<float*>(p + up(ns)), ns, a.stream);
    if (e != hipSuccess) return e;
    a.b = p + up(ns);
  }
  a.xdt = IQMM_FLOAT32;
  return hipSuccess;
}

// quantized_matmul, and with glu its fused SwiGLU form (N = 2I weight rows -> I outputs)
int qmm_entry(const char* op, iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
              iqmm_array biases, bool transpose, iqmm_optional_int group_size,
              iqmm_optional_int bits, const char* mode, iqmm_stream stream, bool glu) {
  g_last_error.clear();
  QParams q;
  if (resolve(op, mode, group_size, bits, q)) return 1;
  int64_t M, N, K;
  int sdt;
  if (qmm_common(op, res, x, w, scales, biases, transpose, q, M, N, K, &sdt)) return 1;
  const int64_t Nw = N;  // weight rows
  if (glu) {
    if (N % 2 != 0)
      return fail("[%s] the fused gate_up weight must have an even number of rows (gate then up), got %lld.", op,
                  (long long)N);
    N /= 2;
  }

  QmmArgs a{};
  const int xb_nd = x.ndim >= 2 ? x.ndim - 2 : 0, wb_nd = w.ndim - 2;
  std::vector<int64_t> out_shape, bshape;
  if (wb_nd == 0) {
    // unbatched weight: every leading dim of x folds into M
    int64_t Mf = 1;
    for (int i = 0; i + 1 < x.ndim; ++i) Mf *= x.shape[i];
    for (int i = 0; i + 1 < x.ndim; ++i) out_shape.push_back(x.shape[i]);
    out_shape.push_back(N);
    a.M = static_cast<int>(Mf);
    if (Mf > 0x7fffffffLL) return fail("[%s] too many rows.", op);
    a.nbatch = 1;
    a.bm.ndim = 0;
  } else {
    if (broadcast2(op, x.shape, xb_nd, w.shape, wb_nd, a.bm, bshape)) return 1;
    out_shape = bshape;
    if (x.ndim >= 2) out_shape.push_back(M);
    out_shape.push_back(N);
    a.M = static_cast<int>(M);
    a.nbatch = 1;
    for (auto d : bshape) a.nbatch *= d;
  }
  const int odt = result_dtype(q, x.dtype, sdt);
  bool query;
  if (set_or_check_res(op, res, out_shape, odt, &query)) return 1;
  if (query) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t out_n = numel(*res);
  if (out_n == 0) return 0;
  if (K == 0) {
    hipError_t e = fill_zero(res->data, odt, out_n, st);
    return e == hipSuccess ? 0 : hip_fail(op, e);
  }
  a.x = x.data; a.w = static_cast<const uint32_t*>(w.data); a.s = scales.data; a.b = biases.data;
  a.out = res->data;
  a.N = static_cast<int>(N); a.K = static_cast<int>(K);
  a.gs = q.gs; a.bits = q.bits; a.mode = q.mode; a.xdt = x.dtype; a.transpose = transpose;
  a.x_mat = M * K;
  a.w_mat = w.shape[w.ndim - 2] * w.shape[w.ndim - 1];
  a.s_mat = scales.shape[scales.ndim - 2] * scales.shape[scales.ndim - 1];
  int64_t nxm = 1, nwm = 1;
  for (int i = 0; i < xb_nd; ++i) nxm *= x.shape[i];
  for (int i = 0; i < wb_nd; ++i) nwm *= w.shape[i];
  a.bm.nx = nxm; a.bm.nw = nwm; a.bm.lhs = nullptr; a.bm.rhs = nullptr;
  a.stream = st;
  (void)Nw;
  hipError_t e = promote_inputs(a, x, scales, biases, sdt);
  if (e != hipSuccess) return hip_fail(op, e);
  e = glu ? run_glu(a, true, [](QmmArgs& p) { return run_qmm(p); }) : run_qmm(a);
  return e == hipSuccess ? 0 : hip_fail(op, e);
}
}  // namespace
}  // namespace iqmm

extern "C" {

int iqmm_quantized_matmul(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                          iqmm_array biases, bool transpose, iqmm_optional_int group_size,
                          iqmm_optional_int bits, const char* mode, iqmm_stream stream) {
  return qmm_entry("quantized_matmul", res, x, w, scales, biases, transpose, group_size, bits, mode, stream,
                   false);
}

int iqmm_quantized_swiglu(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                          iqmm_array biases, iqmm_optional_int group_size, iqmm_optional_int bits,
                          const char* mode, iqmm_stream stream) {
  return qmm_entry("quantized_swiglu", res, x, w, scales, biases, true, group_size, bits, mode, stream, true);
}

}  // extern "C"

namespace iqmm {
namespace {
// gather_qmm, and with glu its fused SwiGLU form over stacked gate_up experts
int gather_entry(const char* op, iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                 iqmm_array biases, iqmm_array lhs, iqmm_array rhs, bool transpose,
                 iqmm_optional_int group_size, iqmm_optional_int bits, const char* mode,
                 bool sorted_indices, iqmm_stream stream, bool glu) {
  g_last_error.clear();
  QParams q;
  if (resolve(op, mode, group_size, bits, q)) return 1;
  if (!present(x) || x.ndim < 2) return fail("[%s] x must have at least two dimensions.", op);
  int64_t M, N, K;
  int sdt;
  if (qmm_common(op, res, x, w, scales, biases, transpose, q, M, N, K, &sdt)) return 1;
  if (glu) {
    if (N % 2 != 0)
      return fail("[%s] the fused gate_up weight must have an even number of rows (gate then up), got %lld.", op,
                  (long long)N);
    N /= 2;
  }
  const int xb_nd = x.ndim - 2, wb_nd = w.ndim - 2;
  QmmArgs a{};
  // index arrays: absent -> arange over the operand's batch, shaped like it
  const int64_t* lshape = present(lhs) ? lhs.shape : x.shape;
  const int lnd = present(lhs) ? lhs.ndim : xb_nd;
  const int64_t* rshape = present(rhs) ? rhs.shape : w.shape;
  const int rnd = present(rhs) ? rhs.ndim : wb_nd;
  if (present(lhs) && !is_index(lhs.dtype)) return fail("[%s] lhs_indices must be integers, got %s.", op, dt_name(lhs.dtype));
  if (present(rhs) && !is_index(rhs.dtype)) return fail("[%s] rhs_indices must be integers, got %s.", op, dt_name(rhs.dtype));
  std::vector<int64_t> bshape;
  if (broadcast2(op, lshape, lnd, rshape, rnd, a.bm, bshape)) return 1;
  std::vector<int64_t> out_shape = bshape;
  out_shape.push_back(M);
  out_shape.push_back(N);
  const int odt = result_dtype(q, x.dtype, sdt);
  bool query;
  if (set_or_check_res(op, res, out_shape, odt, &query)) return 1;
  if (query) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t out_n = numel(*res);
  if (out_n == 0) return 0;
  if (K == 0) {
    hipError_t e = fill_zero(res->data, odt, out_n, st);
    return e == hipSuccess ? 0 : hip_fail(op, e);
  }
  a.x = x.data; a.w = static_cast<const uint32_t*>(w.data); a.s = scales.data; a.b = biases.data;
  a.out = res->data;
  a.M = static_cast<int>(M); a.N = static_cast<int>(N); a.K = static_cast<int>(K);
  a.gs = q.gs; a.bits = q.bits; a.mode = q.mode; a.xdt = x.dtype; a.transpose = transpose;
  a.x_mat = M * K;
  a.w_mat = w.shape[w.ndim - 2] * w.shape[w.ndim - 1];
  a.s_mat = scales.shape[scales.ndim - 2] * scales.shape[scales.ndim - 1];
  a.nbatch = 1;
  for (auto d : bshape) a.nbatch *= d;
  int64_t nxm = 1, nwm = 1;
  for (int i = 0; i < xb_nd; ++i) nxm *= x.shape[i];
  for (int i = 0; i < wb_nd; ++i) nwm *= w.shape[i];
  a.bm.nx = nxm; a.bm.nw = nwm;
  a.bm.lhs = present(lhs) ? lhs.data : nullptr;
  a.bm.rhs = present(rhs) ? rhs.data : nullptr;
  a.bm.lhs_dt = lhs.dtype; a.bm.rhs_dt = rhs.dtype;
  a.stream = st;
  {
    const hipError_t pe = promote_inputs(a, x, scales, biases, sdt);
    if (pe != hipSuccess) return hip_fail(op, pe);
  }
  // sorted form: rhs (and lhs, or x's batch when lhs is absent) enumerate the
  // output batch one-to-one, so expert segments are contiguous in it
  const bool one_to_one = present(rhs) && numel(rhs) == a.nbatch &&
                          (present(lhs) ? numel(lhs) == a.nbatch : nxm == a.nbatch);
  // Sorted rows go to the grouped kernel (each expert's weights read once for
  // all of its rows), except where the M = 1 GEMV applies and experts hold at
  // most one row on average: there the per-row GEMV is as fast (T = 8 of a
  // 256-expert top-8 routing: gate projection 11.9 against 12.6 us; at T = 64
  // the grouped kernel takes 41.5 against 54.2 us).  The fused SwiGLU follows
  // the same choice.
  const int64_t rows_per_expert = a.nbatch * a.M / (nwm > 0 ? nwm : 1);
  QmmArgs probe = a;
  probe.N = glu ? 2 * a.N : a.N;
  const bool gemv_ok = qmv_q4_m1_supported(probe);
  // The grouped kernel's SwiGLU epilogue (affine 4-bit) is faster than the
  // per-row fused GEMV from 512 rows on (T = 64 of a 256-expert top-8 expert
  // block: 189 against 194 us).
  const bool glu_grouped = glu && a.nbatch * a.M >= 512 && gather_sorted_glu_supported(a);
  const bool grouped = sorted_indices && one_to_one && nwm + 1 <= 65535 && gather_sorted_supported(a) &&
                       (glu_grouped || !(gemv_ok && rows_per_expert <= 1));
  auto product = [&](QmmArgs& p) { return grouped ? launch_gather_sorted(p, p.nbatch, nwm) : run_qmm(p); };
  hipError_t e;
  if (glu && grouped && gather_sorted_glu_supported(a)) {
    // SwiGLU in the grouped kernel's epilogue
    a.glu = 1;
    e = launch_gather_sorted(a, a.nbatch, nwm);
  } else {
    e = glu ? run_glu(a, !grouped, product) : product(a);
  }
  return e == hipSuccess ? 0 : hip_fail(op, e);
}
}  // namespace
}  // namespace iqmm

extern "C" {

int iqmm_gather_qmm(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                    iqmm_array biases, iqmm_array lhs, iqmm_array rhs, bool transpose,
                    iqmm_optional_int group_size, iqmm_optional_int bits, const char* mode,
                    bool sorted_indices, iqmm_stream stream) {
  return gather_entry("gather_qmm", res, x, w, scales, biases, lhs, rhs, transpose, group_size, bits, mode,
                      sorted_indices, stream, false);
}

int iqmm_gather_qmm_swiglu(iqmm_array* res, iqmm_array x, iqmm_array w, iqmm_array scales,
                           iqmm_array biases, iqmm_array lhs, iqmm_array rhs,
                           iqmm_optional_int group_size, iqmm_optional_int bits, const char* mode,
                           bool sorted_indices, iqmm_stream stream) {
  return gather_entry("gather_qmm_swiglu", res, x, w, scales, biases, lhs, rhs, true, group_size, bits, mode,
                      sorted_indices, stream, true);
}

}  // extern "C"

namespace iqmm {
namespace {
// dequantize, and with an index array the row gather of an embedding table
int deq_entry(const char* op, iqmm_array* res, iqmm_array w, iqmm_array scales, iqmm_array biases,
              const iqmm_array* idx, iqmm_optional_int group_size, iqmm_optional_int bits,
              const char* mode, iqmm_optional_dtype dtype, iqmm_stream stream) {
  g_last_error.clear();
  QParams q;
  if (resolve(op, mode, group_size, bits, q)) return 1;
  if (!present(w) || w.ndim < 2) return fail("[%s] The matrix to be dequantized must have at least 2 dimensions but it has only %d.", op, w.ndim);
  if (w.dtype != IQMM_UINT32) return fail("[%s] The matrix should be given as a uint32 but received %s.", op, dt_name(w.dtype));
  const int64_t wlast = w.shape[w.ndim - 1];
  if ((wlast * 32) % q.bits != 0) return fail("[%s] packed width %lld is not a whole number of %d-bit codes.", op, (long long)wlast, q.bits);
  const int64_t K = wlast * 32 / q.bits;
  if (K % q.gs != 0) return fail("[%s] The unpacked width %lld is not divisible by group_size %d.", op, (long long)K, q.gs);
  int sdt;
  if (check_scales(op, q, w, scales, biases, K / q.gs, &sdt)) return 1;
  int odt = q.mode == AFFINE ? sdt : IQMM_BFLOAT16;
  if (dtype.has_value) {
    if (!is_float(dtype.value)) return fail("[%s] Output dtype must be a floating type, got %s.", op, dt_name(dtype.value));
    odt = dtype.value;
  }
  std::vector<int64_t> out_shape(w.shape, w.shape + w.ndim);
  out_shape.back() = K;
  if (idx) {
    if (w.ndim != 2) return fail("[%s] the quantized table must be 2D [rows, K*bits/32], got %s.", op, shape_str(w).c_str());
    if (!present(*idx) || !is_index(idx->dtype))
      return fail("[%s] indices must be an integer array, got %s.", op, present(*idx) ? dt_name(idx->dtype) : "none");
    out_shape.assign(idx->shape, idx->shape + idx->ndim);
    out_shape.push_back(K);
  }
  bool query;
  if (set_or_check_res(op, res, out_shape, odt, &query)) return 1;
  if (query) return 0;
  ConvArgs a{};
  a.w = static_cast<const uint32_t*>(w.data); a.s = scales.data; a.b = biases.data; a.out = res->data;
  a.rows = numel(w) / (wlast > 0 ? wlast : 1);
  if (idx) {
    a.table_rows = a.rows;
    a.rows = numel(*idx);
    a.idx = idx->data;
    a.idx_dt = idx->dtype;
    if (a.rows == 0) return 0;
  }
  if (wlast == 0) return 0;
  if (K > 0x7fffffffLL) return fail("[%s] row too long.", op);
  a.K = static_cast<int>(K); a.gs = q.gs; a.bits = q.bits; a.mode = q.mode; a.sdt = sdt; a.odt = odt;
  a.stream = static_cast<hipStream_t>(stream);
  hipError_t e = launch_dequantize(a);
  return e == hipSuccess ? 0 : hip_fail(op, e);
}
}  // namespace
}  // namespace iqmm

extern "C" {

int iqmm_dequantize(iqmm_array* res, iqmm_array w, iqmm_array scales, iqmm_array biases,
                    iqmm_optional_int group_size, iqmm_optional_int bits, const char* mode,
                    iqmm_optional_dtype dtype, iqmm_stream stream) {
  return deq_entry("dequantize", res, w, scales, biases, nullptr, group_size, bits, mode, dtype, stream);
}

int iqmm_dequantize_rows(iqmm_array* res, iqmm_array w, iqmm_array scales, iqmm_array biases,
                         iqmm_array indices, iqmm_optional_int group_size, iqmm_optional_int bits,
                         const char* mode, iqmm_optional_dtype dtype, iqmm_stream stream) {
  return deq_entry("dequantize_rows", res, w, scales, biases, &indices, group_size, bits, mode, dtype, stream);
}

int iqmm_quantize(iqmm_array* res_w, iqmm_array* res_scales, iqmm_array* res_biases,
                  iqmm_array w, iqmm_optional_int group_size, iqmm_optional_int bits,
                  const char* mode, iqmm_stream stream) {
  const char* op = "quantize";
  g_last_error.clear();
  QParams q;
  if (resolve(op, mode, group_size, bits, q)) return 1;
  if (!present(w) || w.ndim < 2) return fail("[%s] The matrix to be quantized must have at least 2 dimensions but it has only %d.", op, w.ndim);
  if (!is_float(w.dtype)) return fail("[%s] Only real floating types can be quantized but w has type %s.", op, dt_name(w.dtype));
  const int64_t K = w.shape[w.ndim - 1];
  if (K % q.gs != 0)
    return fail("[%s] The last dimension of the matrix needs to be divisible by the quantization group size %d. However the provided matrix has shape %s", op, q.gs, shape_str(w).c_str());
  if ((K * q.bits) % 32 != 0) return fail("[%s] K*bits must be a multiple of 32.", op);
  std::vector<int64_t> wq_shape(w.shape, w.shape + w.ndim), s_shape(w.shape, w.shape + w.ndim);
  wq_shape.back() = K * q.bits / 32;
  s_shape.back() = K / q.gs;
  const int sdt = q.mode == AFFINE ? w.dtype : IQMM_UINT8;
  bool q1, q2, q3 = true;
  if (set_or_check_res(op, res_w, wq_shape, IQMM_UINT32, &q1)) return 1;
  if (set_or_check_res(op, res_scales, s_shape, sdt, &q2)) return 1;
  if (q.mode == AFFINE) {
    if (set_or_check_res(op, res_biases, s_shape, sdt, &q3)) return 1;
  } else if (res_biases) {
    res_biases->ndim = 0;
    res_biases->data = nullptr;
  }
  if (q1 || q2 || (q.mode == AFFINE && q3)) {
    if (!(q1 && q2 && (q.mode != AFFINE || q3)))
      return fail("[%s] either all result buffers are allocated or none.", op);
    return 0;
  }
  ConvArgs a{};
  a.src = w.data; a.wq = static_cast<uint32_t*>(res_w->data); a.sq = res_scales->data;
  a.bq = q.mode == AFFINE ? res_biases->data : nullptr;
  a.rows = K > 0 ? numel(w) / K : 0;
  if (K > 0x7fffffffLL) return fail("[%s] row too long.", op);
  a.K = static_cast<int>(K); a.gs = q.gs; a.bits = q.bits; a.mode = q.mode; a.sdt = w.dtype;
  a.stream = static_cast<hipStream_t>(stream);
  hipError_t e = launch_quantize(a);
  return e == hipSuccess ? 0 : hip_fail(op, e);
}


int iqmm_moe_route(iqmm_array* res_scores, iqmm_array* res_experts, iqmm_array logits, int k,
                   bool norm_topk_prob, iqmm_stream stream) {
  const char* op = "moe_route";
  g_last_error.clear();
  if (!present(logits) || logits.ndim != 2) return fail("[%s] logits must be 2D [tokens, experts], got %s.", op, shape_str(logits).c_str());
  if (!is_float(logits.dtype)) return fail("[%s] logits must be floating point, got %s.", op, dt_name(logits.dtype));
  const int64_t T = logits.shape[0], E = logits.shape[1];
  if (E < 1 || E > 2048) return fail("[%s] the number of experts must be in [1, 2048], got %lld.", op, (long long)E);
  if (k < 1 || k > 32 || k > E) return fail("[%s] k must be in [1, min(experts, 32)], got %d.", op, k);
  if (T > 0x7fffffffLL / 4) return fail("[%s] too many tokens.", op);
  const std::vector<int64_t> shp = {T, k};
  bool q1, q2;
  if (set_or_check_res(op, res_scores, shp, IQMM_FLOAT32, &q1)) return 1;
  if (set_or_check_res(op, res_experts, shp, IQMM_INT32, &q2)) return 1;
  if (q1 || q2) {
    if (!(q1 && q2)) return fail("[%s] either all result buffers are allocated or none.", op);
    return 0;
  }
  hipError_t e = launch_moe_route(logits.data, logits.dtype, static_cast<float*>(res_scores->data),
                                  static_cast<int32_t*>(res_experts->data), static_cast<int>(T), static_cast<int>(E), k,
                                  norm_topk_prob, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : hip_fail(op, e);
}

int iqmm_moe_sort(iqmm_array* res_tokens, iqmm_array* res_sorted, iqmm_array* res_inverse,
                  iqmm_array* res_offsets, iqmm_array experts, int num_experts, iqmm_stream stream) {
  return moe_sort_entry("moe_sort", false, res_tokens, res_sorted, res_inverse, res_offsets, experts,
                        num_experts, stream);
}

int iqmm_moe_sort_noalloc(iqmm_array* res_tokens, iqmm_array* res_sorted, iqmm_array* res_inverse,
                          iqmm_array* res_offsets, iqmm_array experts, int num_experts, iqmm_stream stream) {
  return moe_sort_entry("moe_sort_noalloc", true, res_tokens, res_sorted, res_inverse, res_offsets, experts,
                        num_experts, stream);
}

int iqmm_moe_combine(iqmm_array* res, iqmm_array y, iqmm_array inverse, iqmm_array experts,
                     iqmm_array scores, int num_experts, iqmm_stream stream) {
  const char* op = "moe_combine";
  g_last_error.clear();
  if (!present(experts) || experts.ndim != 2 || experts.dtype != IQMM_INT32)
    return fail("[%s] experts must be a 2D int32 array [tokens, k].", op);
  const int64_t T = experts.shape[0], k = experts.shape[1];
  if (k > 32) return fail("[%s] at most 32 experts per token, got %lld.", op, (long long)k);
  if (!present(scores) || scores.dtype != IQMM_FLOAT32 || numel(scores) != T * k)
    return fail("[%s] scores must be float32 with the experts' %lld entries.", op, (long long)(T * k));
  if (!present(inverse) || inverse.dtype != IQMM_INT32 || numel(inverse) != T * k)
    return fail("[%s] inverse must be int32 with the experts' %lld entries.", op, (long long)(T * k));
  if (!present(y) || y.ndim < 2 || !is_float(y.dtype)) return fail("[%s] y must be a floating array [rows, D].", op);
  const int64_t D = y.shape[y.ndim - 1];
  const int64_t n = D > 0 ? numel(y) / D : 0;
  if (T > 0x7fffffffLL) return fail("[%s] too many tokens.", op);
  const std::vector<int64_t> shp = {T, D};
  bool q;
  if (set_or_check_res(op, res, shp, IQMM_FLOAT32, &q)) return 1;
  if (q) return 0;
  hipError_t e = launch_moe_combine(y.data, y.dtype, static_cast<const int32_t*>(inverse.data),
                                    static_cast<const int32_t*>(experts.data), static_cast<const float*>(scores.data),
                                    static_cast<float*>(res->data), static_cast<int>(T), static_cast<int>(k), D,
                                    num_experts, n, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : hip_fail(op, e);
}


int iqmm_moe_token(iqmm_array* res, iqmm_array logits, iqmm_array x, iqmm_array gate_up_w,
                   iqmm_array gate_up_scales, iqmm_array gate_up_biases, iqmm_array down_w,
                   iqmm_array down_scales, iqmm_array down_biases, int k, bool norm_topk_prob,
                   int group_size, int bits, iqmm_stream stream) {
  const char* op = "moe_token";
  g_last_error.clear();
  if (!present(logits) || !is_float(logits.dtype)) return fail("[%s] logits must be a floating array [1, experts].", op);
  const int64_t E = numel(logits);
  if (logits.ndim < 1 || logits.shape[logits.ndim - 1] != E)
    return fail("[%s] logits must hold one token's [experts] row, got %s.", op, shape_str(logits).c_str());
  if (!present(x) || (x.dtype != IQMM_BFLOAT16 && x.dtype != IQMM_FLOAT16))
    return fail("[%s] x must be bfloat16 or float16.", op);
  const int64_t H = numel(x);
  if (x.ndim < 1 || x.shape[x.ndim - 1] != H) return fail("[%s] x must hold one token's row, got %s.", op, shape_str(x).c_str());
  if (bits != 4) return fail("[%s] only 4-bit affine experts are supported, got bits=%d.", op, bits);
  auto check3 = [&](const iqmm_array& a, int dt, int64_t d0, int64_t d1, int64_t d2, const char* what) {
    if (!present(a) || a.ndim != 3 || a.dtype != dt || a.shape[0] != d0 || a.shape[1] != d1 || a.shape[2] != d2)
      return fail("[%s] %s must be %s [%lld, %lld, %lld], got %s %s.", op, what, dt_name(dt), (long long)d0,
                  (long long)d1, (long long)d2, dt_name(a.dtype), shape_str(a).c_str());
    return 0;
  };
  if (!present(gate_up_w) || gate_up_w.ndim != 3) return fail("[%s] gate_up weight must be 3D [experts, 2I, H/8].", op);
  if (!present(down_w) || down_w.ndim != 3) return fail("[%s] down weight must be 3D [experts, D, I/8].", op);
  const int64_t I2 = gate_up_w.shape[1], D = down_w.shape[1], I = I2 / 2;
  if (I2 % 2 != 0) return fail("[%s] gate_up must stack 2I rows (gate rows first), got %lld.", op, (long long)I2);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail("[%s] group_size must be 32, 64 or 128, got %d.", op, group_size);
  if (H % group_size != 0 || I % group_size != 0) return fail("[%s] H and I must be multiples of the group size.", op);
  if (check3(gate_up_w, IQMM_UINT32, E, I2, H / 8, "gate_up weight") ||
      check3(gate_up_scales, x.dtype, E, I2, H / group_size, "gate_up scales") ||
      check3(gate_up_biases, x.dtype, E, I2, H / group_size, "gate_up biases") ||
      check3(down_w, IQMM_UINT32, E, D, I / 8, "down weight") ||
      check3(down_scales, x.dtype, E, D, I / group_size, "down scales") ||
      check3(down_biases, x.dtype, E, D, I / group_size, "down biases"))
    return 1;
  if (E > 0x7fffffffLL || H > 0x7fffffffLL || I > 0x7fffffffLL || D > 0x7fffffffLL ||
      !moe_token_supported(static_cast<int>(E), k, static_cast<int>(H), static_cast<int>(I), static_cast<int>(D), group_size))
    return fail("[%s] unsupported shape: experts <= 512, 1 <= k <= min(experts, 32), H in [32, 8192] and I in "
                "[32, 2048] multiples of 32 (got E=%lld k=%d H=%lld I=%lld).", op, (long long)E, k, (long long)H, (long long)I);
  const std::vector<int64_t> shp = {1, D};
  bool q;
  if (set_or_check_res(op, res, shp, IQMM_FLOAT32, &q)) return 1;
  if (q) return 0;
  hipError_t e = launch_moe_token(logits.data, logits.dtype, x.data, x.dtype, static_cast<const uint32_t*>(gate_up_w.data),
                                  gate_up_scales.data, gate_up_biases.data, static_cast<const uint32_t*>(down_w.data),
                                  down_scales.data, down_biases.data, static_cast<int>(E), k, norm_topk_prob,
                                  static_cast<int>(H), static_cast<int>(I), static_cast<int>(D), group_size,
                                  static_cast<float*>(res->data), static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : hip_fail(op, e);
}

}  // extern "C"
