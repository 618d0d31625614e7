// moe.hip — the MoE routing around gather_qmm, on the device.
//
// route   (mlx/src/nn/moe.rs:67-82): per token, softmax over the experts in
//         fp32 with the probabilities stored in the logits' dtype, the k
//         largest by a stable descending order (ties to the lower expert id,
//         as a stable argsort of -p), and optionally p / sum(p of the k), each
//         result rounded to the logits' dtype.  One wave per token.
// sort    (mlx/src/nn/moe.rs:92-104): the (token, slot) rows ordered by
//         expert, rows of one expert kept in (token, slot) order.  One
//         workgroup bitonic-sorts unique 32-bit keys expert * n + row in LDS.
// combine (mlx/src/nn/moe.rs:146-168): per token, the expert rows times
//         their scores summed in fp32 in ascending expert order, the first
//         product taken as is and each further one added, as the reference's
//         row_sum chain does.
#include <atomic>
#include <mutex>

#include "launch.h"

namespace iqmm {

#pragma clang fp contract(off)

namespace {

// Value of the partner lane in step `st` of an all-reduce over the wave:
// quad xor 1, quad xor 2 (DPP quad_perm), 7 - i within 8 (row_half_mirror),
// 15 - i within 16 (row_mirror), the other row of a 32-lane half
// (v_permlane16_swap) and the other half (v_permlane32_swap).  Every step
// pairs lanes symmetrically, so an order-independent reduction (max, argmax
// on distinct keys) leaves the same result in every lane; no LDS traffic.
template <int ST>
__device__ __forceinline__ uint32_t wave_partner(uint32_t x) {
  if constexpr (ST == 0) return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);
  else if constexpr (ST == 1) return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);
  else if constexpr (ST == 2) return __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);
  else if constexpr (ST == 3) return __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false);
  else if constexpr (ST == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return ((threadIdx.x >> 4) & 1) ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return ((threadIdx.x >> 5) & 1) ? r[0] : r[1];
  }
}

template <int ST>
__device__ __forceinline__ void argmax_step(float& bv, int& bi) {
  const float ov = __uint_as_float(wave_partner<ST>(__float_as_uint(bv)));
  const int oi = static_cast<int>(wave_partner<ST>(static_cast<uint32_t>(bi)));
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// wave-wide (largest value, then lowest index), identical in every lane
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
  argmax_step<0>(bv, bi);
  argmax_step<1>(bv, bi);
  argmax_step<2>(bv, bi);
  argmax_step<3>(bv, bi);
  argmax_step<4>(bv, bi);
  argmax_step<5>(bv, bi);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __uint_as_float(wave_partner<0>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(wave_partner<1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(wave_partner<2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(wave_partner<3>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(wave_partner<4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(wave_partner<5>(__float_as_uint(v))));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// PL = probabilities per lane (E <= 64 * PL)
template <int DT, int PL>
__global__ __launch_bounds__(256) void moe_route_kernel(const typename Store<DT>::T* logits, float* scores,
                                                        int32_t* experts, int T, int E, int k, int norm) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // wave-uniform
  const typename Store<DT>::T* row = logits + static_cast<int64_t>(t) * E;
  float p[PL];
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? to_f<DT>(row[e]) : -__builtin_inff();
    m = fmaxf(m, p[j]);
  }
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? iq_expf(p[j] - m) : 0.f;
    s += p[j];
  }
  s = wave_sum(s);
  // probabilities in the logits' dtype; -1 marks padding and taken entries
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int e = lane + 64 * j;
    p[j] = e < E ? to_f<DT>(from_f<DT>(p[j] / s)) : -1.f;
  }
  float mine = 0.f;  // lane i keeps slot i's probability / expert
  int myexp = 0;
  float tot = 0.f;
  for (int i = 0; i < k; ++i) {
    // lane-local best: largest p, then lowest expert id
    float bv = -1.f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int e = lane + 64 * j;
      if (p[j] > bv) { bv = p[j]; bi = e; }  // ascending e within a lane: ties keep the first
    }
    wave_argmax(bv, bi);
    if ((bi & 63) == lane) {
#pragma unroll
      for (int j = 0; j < PL; ++j)
        if (lane + 64 * j == bi) p[j] = -1.f;
    }
    if (lane == i) { mine = bv; myexp = bi; }
    tot += bv;  // slot order, fp32
  }
  if (lane < k) {
    float v = mine;
    if (norm) {
      const float den = to_f<DT>(from_f<DT>(tot));
      v = to_f<DT>(from_f<DT>(mine / den));
    }
    // no candidate left (NaN logits): an invalid expert that combine skips
    scores[static_cast<int64_t>(t) * k + lane] = mine >= 0.f ? v : __builtin_nanf("");
    experts[static_cast<int64_t>(t) * k + lane] = mine >= 0.f ? myexp : -1;
  }
}

// one workgroup; np = power of two >= n; keys expert' * n + row, where
// expert' = expert for ids in [0, E) and E otherwise (sorted last)
__global__ __launch_bounds__(1024) void moe_sort_kernel(const int32_t* experts, int n, int k, int E, int np,
                                                        int32_t* tokens, int32_t* sorted, int32_t* inverse,
                                                        int32_t* offsets) {
  extern __shared__ uint32_t keys[];
  const int tid = threadIdx.x;
  for (int i = tid; i < np; i += 1024) {
    uint32_t key = 0xffffffffu;
    if (i < n) {
      const int e = experts[i];
      const uint32_t ee = (e >= 0 && e < E) ? static_cast<uint32_t>(e) : static_cast<uint32_t>(E);
      key = ee * static_cast<uint32_t>(n) + static_cast<uint32_t>(i);
    }
    keys[i] = key;
  }
  // A pass with stride <= 64 pairs elements inside 128-element windows that
  // one wave owns (pairs i = 64 w .. 64 w + 63, and i + 1024 j), so it needs a
  // workgroup barrier only after a pass (or the load) that crossed windows.
  bool cross = true;
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (cross || stride >= 128) {
        __syncthreads();
      } else {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
      }
      cross = stride >= 128;
      for (int i = tid; i < (np >> 1); i += 1024) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool asc = (lo & size) == 0;
        const uint32_t a = keys[lo], b = keys[hi];
        if ((a > b) == asc) { keys[lo] = b; keys[hi] = a; }
      }
    }
  }
  __syncthreads();
  const uint32_t un = static_cast<uint32_t>(n);
  for (int i = tid; i <= n; i += 1024) {
    const int ei = i < n ? static_cast<int>(keys[i] / un) : E + 1;
    if (i < n) {
      const int r = static_cast<int>(keys[i] % un);
      tokens[i] = r / k;
      sorted[i] = experts[r];
      inverse[r] = i;
    }
    if (offsets) {
      const int ep = i > 0 ? static_cast<int>(keys[i - 1] / un) : -1;
      for (int e = ep + 1; e <= min(ei, E); ++e) offsets[e] = i;
    }
  }
}

// Stable counting sort over blocks of 256 rows (bucket = expert for ids in
// [0, E), E otherwise), the same order as the key sort above.
// moe_count_kernel: per-block bucket counts, stored expert-major
// hist[bucket * nb + block].  moe_scatter_kernel: every block scans the whole
// histogram in LDS (an exclusive prefix in expert-major order gives the first
// position of each (bucket, block)), ranks its rows among the earlier rows of
// the block with the same bucket, and writes them; block 0 writes the offsets.
constexpr int SORT_BLOCK = 256;

__global__ __launch_bounds__(SORT_BLOCK) void moe_count_kernel(const int32_t* experts, int n, int E, int nb,
                                                               int32_t* hist) {
  extern __shared__ int32_t h[];  // E + 1 counts
  const int tid = threadIdx.x;
  for (int e = tid; e <= E; e += SORT_BLOCK) h[e] = 0;
  __syncthreads();
  const int i = blockIdx.x * SORT_BLOCK + tid;
  if (i < n) {
    const int e = experts[i];
    atomicAdd(&h[(e >= 0 && e < E) ? e : E], 1);
  }
  __syncthreads();
  for (int e = tid; e <= E; e += SORT_BLOCK) hist[static_cast<int64_t>(e) * nb + blockIdx.x] = h[e];
}

__global__ __launch_bounds__(SORT_BLOCK) void moe_scatter_kernel(const int32_t* experts, int n, int k, int E, int nb,
                                                                 const int32_t* hist, int32_t* tokens, int32_t* sorted,
                                                                 int32_t* inverse, int32_t* offsets) {
  extern __shared__ int32_t s[];  // L prefix entries, SORT_BLOCK partials, SORT_BLOCK buckets
  const int L = (E + 1) * nb;
  int32_t* part = s + L;
  int32_t* kb = part + SORT_BLOCK;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int j = tid; j < L; j += SORT_BLOCK) s[j] = hist[j];
  const int i = blockIdx.x * SORT_BLOCK + tid;
  int bucket = -1;
  if (i < n) {
    const int e = experts[i];
    bucket = (e >= 0 && e < E) ? e : E;
  }
  kb[tid] = bucket;
  __syncthreads();
  // exclusive prefix of s: each thread a contiguous segment, then the segment sums
  const int per = (L + SORT_BLOCK - 1) / SORT_BLOCK;
  const int lo = min(tid * per, L), hi = min(lo + per, L);
  int sum = 0;
  for (int j = lo; j < hi; ++j) {
    const int v = s[j];
    s[j] = sum;
    sum += v;
  }
  // inclusive scan of the segment sums: within each wave, then across waves
  int inc = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) part[wave] = inc;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += part[w];
  const int add = base + inc - sum;  // exclusive prefix of this segment
  for (int j = lo; j < hi; ++j) s[j] += add;
  // stable rank among the earlier rows of this block with the same bucket
  int rank = 0;
  for (int j = 0; j < tid; ++j) rank += kb[j] == bucket ? 1 : 0;
  __syncthreads();
  if (i < n) {
    const int pos = s[bucket * nb + blockIdx.x] + rank;
    tokens[pos] = i / k;
    sorted[pos] = experts[i];
    inverse[i] = pos;
  }
  if (blockIdx.x == 0 && offsets != nullptr)
    for (int e = tid; e <= E; e += SORT_BLOCK) offsets[e] = s[e * nb];
}

// out[t, d] = sum over t's valid slots in ascending expert order of
// float(y[pos, d]) * score.  One workgroup per token: the k slots are ranked
// once (in LDS), then each thread runs the ordered sum for its column
// (blockIdx.y picks 256 columns).  Rows may be in any order in y (sorted by
// expert, or one row per (token, slot) when the sort is skipped).
template <int DT>
__global__ __launch_bounds__(256) void moe_combine_kernel(const typename Store<DT>::T* y, const int32_t* inverse,
                                                          const int32_t* experts, const float* scores, float* out,
                                                          int T, int k, int64_t D, int E, int64_t n) {
  __shared__ int64_t rowoff[32];
  __shared__ float wt[32];
  __shared__ int nvalid;
  const int tid = threadIdx.x;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    const int64_t base = static_cast<int64_t>(t) * k;
    if (tid == 0) nvalid = 0;
    __syncthreads();
    if (tid < k) {
      const int pos = inverse[base + tid];
      const int e = experts[base + tid];
      const bool ok = pos >= 0 && pos < n && e >= 0 && e < E;
      // rank among the valid slots by expert id, then row position, then slot
      // (distinct ranks; for sorted rows the position order is the expert order)
      int rank = 0;
      for (int j = 0; j < k; ++j) {
        const int pj = inverse[base + j], ej = experts[base + j];
        const bool okj = pj >= 0 && pj < n && ej >= 0 && ej < E;
        const bool before = ej < e || (ej == e && (pj < pos || (pj == pos && j < tid)));
        rank += (okj && before) ? 1 : 0;
      }
      if (ok) {
        rowoff[rank] = static_cast<int64_t>(pos) * D;
        wt[rank] = scores[base + tid];
        atomicAdd(&nvalid, 1);
      }
    }
    __syncthreads();
    const int nv = nvalid;
    const int64_t d = static_cast<int64_t>(blockIdx.y) * 256 + tid;
    if (d < D) {
      float acc = 0.f;
      for (int i0 = 0; i0 < nv; i0 += 8) {
        // the loads of up to 8 rows are issued before the ordered adds
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = i0 + j < nv ? to_f<DT>(y[rowoff[i0 + j] + d]) : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (i0 + j < nv) {
            const float p = v[j] * wt[i0 + j];
            acc = i0 + j == 0 ? p : acc + p;
          }
        }
      }
      out[static_cast<int64_t>(t) * D + d] = acc;
    }
    __syncthreads();
  }
}

template <int DT>
hipError_t route_pl(const void* logits, float* scores, int32_t* experts, int T, int E, int k, bool norm,
                    hipStream_t st) {
  using S = typename Store<DT>::T;
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  const S* lg = static_cast<const S*>(logits);
  const int pl = (E + 63) / 64;
#define IQMM_R(P) \
  hipLaunchKernelGGL((moe_route_kernel<DT, P>), grid, dim3(256), 0, st, lg, scores, experts, T, E, k, norm ? 1 : 0)
  if (pl <= 1) IQMM_R(1);
  else if (pl <= 2) IQMM_R(2);
  else if (pl <= 4) IQMM_R(4);
  else if (pl <= 8) IQMM_R(8);
  else if (pl <= 16) IQMM_R(16);
  else IQMM_R(32);
#undef IQMM_R
  return hipGetLastError();
}

}  // namespace

hipError_t launch_moe_route(const void* logits, int dt, float* scores, int32_t* experts, int T, int E, int k,
                            bool norm, hipStream_t st) {
  if (T == 0) return hipSuccess;
  switch (dt) {
    case F32: return route_pl<F32>(logits, scores, experts, T, E, k, norm, st);
    case F16: return route_pl<F16>(logits, scores, experts, T, E, k, norm, st);
    case BF16: return route_pl<BF16>(logits, scores, experts, T, E, k, norm, st);
  }
  return hipErrorInvalidValue;
}

namespace {

// Fixed scratch of iqmm_moe_sort_noalloc: the (bucket, block) counts of the
// counting sort, SORT_HIST_MAX int32 (62 KiB) per device, held until the
// process ends.  Host code never passes `scratch` itself to a kernel: it is a
// host-side stand-in; the device address comes from hipGetSymbolAddress,
// once per device (sort_scratch).  Every call on a device shares the array.
constexpr int SORT_HIST_MAX = 16384 - 2 * SORT_BLOCK;
static __device__ __align__(256) int32_t scratch[SORT_HIST_MAX];

constexpr int kMaxDevices = 64;

hipError_t sort_scratch(int32_t** out) {
  static std::mutex mu;
  static int32_t* ptr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if (ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = ptr[dev];
  return hipSuccess;
}

// hist: the counting sort's (bucket, block) counts, or nullptr to take them
// from the stream's workspace
hipError_t moe_sort_impl(const int32_t* experts, int n, int k, int E, int32_t* tokens, int32_t* sorted,
                         int32_t* inverse, int32_t* offsets, hipStream_t st, int32_t* hist) {
  // counting sort when the (bucket, block) histogram fits one workgroup's LDS
  // with its partials: 64 KiB
  const int nb = (n + SORT_BLOCK - 1) / SORT_BLOCK;
  const int64_t L = (static_cast<int64_t>(E) + 1) * nb;
  if (n > 0 && L <= SORT_HIST_MAX) {
    hipError_t e = hipSuccess;
    if (hist == nullptr) {
      void* ws = nullptr;
      e = workspace_get(st, WS_SORT, static_cast<size_t>(L) * 4, &ws);
      if (e != hipSuccess) return e;
      hist = static_cast<int32_t*>(ws);
    }
    hipLaunchKernelGGL(moe_count_kernel, dim3(nb), dim3(SORT_BLOCK), static_cast<size_t>(E + 1) * 4, st, experts, n,
                       E, nb, hist);
    e = hipGetLastError();
    if (e == hipSuccess) {
      hipLaunchKernelGGL(moe_scatter_kernel, dim3(nb), dim3(SORT_BLOCK),
                         static_cast<size_t>(L + 2 * SORT_BLOCK) * 4, st, experts, n, k, E, nb, hist, tokens, sorted,
                         inverse, offsets);
      e = hipGetLastError();
    }
    return e;
  }
  int np = 2;
  while (np < n) np <<= 1;
  const size_t lds = static_cast<size_t>(np) * 4;
  if (lds > 65536) {
    static std::atomic<uint64_t> done{0};  // attribute raised once per device id < 64
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 64;
    const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
    if (!bit || !(done.load(std::memory_order_acquire) & bit)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(moe_sort_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 131072);
      if (e != hipSuccess) return e;
      if (bit) done.fetch_or(bit, std::memory_order_release);
    }
  }
  hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(1024), lds, st, experts, n, k, E, np, tokens, sorted, inverse,
                     offsets);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_moe_sort(const int32_t* experts, int n, int k, int E, int32_t* tokens, int32_t* sorted,
                           int32_t* inverse, int32_t* offsets, hipStream_t st) {
  return moe_sort_impl(experts, n, k, E, tokens, sorted, inverse, offsets, st, nullptr);
}

hipError_t launch_moe_sort_noalloc(const int32_t* experts, int n, int k, int E, int32_t* tokens, int32_t* sorted,
                                   int32_t* inverse, int32_t* offsets, hipStream_t st) {
  // the counts are fully overwritten by moe_count_kernel: nothing to clear
  int32_t* hist = nullptr;
  const hipError_t e = sort_scratch(&hist);
  if (e != hipSuccess) return e;
  return moe_sort_impl(experts, n, k, E, tokens, sorted, inverse, offsets, st, hist);
}

hipError_t launch_moe_combine(const void* y, int dt, const int32_t* inverse, const int32_t* experts,
                              const float* scores, float* out, int T, int k, int64_t D, int E, int64_t n,
                              hipStream_t st) {
  if (T == 0 || D == 0) return hipSuccess;
  if ((D + 255) / 256 > 65535) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(T < 1048576 ? T : 1048576), static_cast<unsigned>((D + 255) / 256));
  switch (dt) {
    case F32:
      hipLaunchKernelGGL(moe_combine_kernel<F32>, grid, dim3(256), 0, st, static_cast<const float*>(y), inverse,
                         experts, scores, out, T, k, D, E, n);
      break;
    case F16:
      hipLaunchKernelGGL(moe_combine_kernel<F16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(y), inverse,
                         experts, scores, out, T, k, D, E, n);
      break;
    case BF16:
      hipLaunchKernelGGL(moe_combine_kernel<BF16>, grid, dim3(256), 0, st, static_cast<const uint16_t*>(y), inverse,
                         experts, scores, out, T, k, D, E, n);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace iqmm
