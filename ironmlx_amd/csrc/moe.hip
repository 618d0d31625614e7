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
#include "gemv_common.h"

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

__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
  v = max(v, wave_partner<0>(v));
  v = max(v, wave_partner<1>(v));
  v = max(v, wave_partner<2>(v));
  v = max(v, wave_partner<3>(v));
  v = max(v, wave_partner<4>(v));
  v = max(v, wave_partner<5>(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One token's routing by one wave (PL probabilities per lane, E <= 64 PL):
// lane i < k receives slot i's score (as stored: rounded to the logits' dtype,
// normalised when `norm`) and expert, or NaN / -1 when no candidate is left
// (NaN logits).
template <int DT, int PL>
__device__ __forceinline__ void route_token(const typename Store<DT>::T* row, int E, int k, int norm, float& score,
                                            int& expert) {
  const int lane = threadIdx.x & 63;
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
  if constexpr (DT != F32) {
    // 16-bit probabilities: one 32-bit key per candidate, (p bits) << 16 |
    // (0xFFFF - e), orders by p (non-negative: its bits order as unsigned),
    // then by the lower expert id; 0 marks padding, NaN and taken entries, so
    // each slot is one unsigned max over the wave
    uint32_t key[PL];
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int e = lane + 64 * j;
      key[j] = p[j] >= 0.f ? (static_cast<uint32_t>(from_f<DT>(p[j])) << 16) | static_cast<uint32_t>(0xFFFF - e) : 0u;
    }
    for (int i = 0; i < k; ++i) {
      uint32_t best = key[0];
#pragma unroll
      for (int j = 1; j < PL; ++j) best = best > key[j] ? best : key[j];
      best = wave_umax(best);
#pragma unroll
      for (int j = 0; j < PL; ++j) key[j] = key[j] == best ? 0u : key[j];
      const float bv = best ? to_f<DT>(static_cast<typename Store<DT>::T>(best >> 16)) : -1.f;
      const int bi = best ? 0xFFFF - static_cast<int>(best & 0xFFFFu) : 0x7fffffff;
      if (lane == i) { mine = bv; myexp = bi; }
      tot += bv;  // slot order, fp32
    }
  } else {
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
  }
  float v = mine;
  if (norm) {
    const float den = to_f<DT>(from_f<DT>(tot));
    v = to_f<DT>(from_f<DT>(mine / den));
  }
  // no candidate left (NaN logits): an invalid expert that combine skips
  score = mine >= 0.f ? v : __builtin_nanf("");
  expert = mine >= 0.f ? myexp : -1;
}

template <int DT, int PL>
__global__ __launch_bounds__(256) void moe_route_kernel(const typename Store<DT>::T* logits, float* scores,
                                                        int32_t* experts, int T, int E, int k, int norm) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // wave-uniform
  float sc;
  int ex;
  route_token<DT, PL>(logits + static_cast<int64_t>(t) * E, E, k, norm, sc, ex);
  if (lane < k) {
    scores[static_cast<int64_t>(t) * k + lane] = sc;
    experts[static_cast<int64_t>(t) * k + lane] = ex;
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
// VEC > 1: each thread takes VEC consecutive columns (one 16-byte load per
// row, D % VEC == 0), so a token's rows are read in full 16-byte pieces and
// the ranking is paid once per 256 VEC columns.
template <int DT, int VEC = 1>
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
    if constexpr (VEC > 1) {
      using S = typename Store<DT>::T;
      const int64_t d0 = (static_cast<int64_t>(blockIdx.y) * 256 + tid) * VEC;
      if (d0 < D) {
        float acc[VEC];
#pragma unroll
        for (int c = 0; c < VEC; ++c) acc[c] = 0.f;
        for (int i0 = 0; i0 < nv; i0 += 4) {
          // the loads of up to 4 rows are issued before the ordered adds
          uint4 v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[j] = i0 + j < nv ? *reinterpret_cast<const uint4*>(y + rowoff[i0 + j] + d0) : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (i0 + j < nv) {
              const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
              for (int c = 0; c < VEC; ++c) {
                float e;
                if constexpr (sizeof(S) == 4) e = __uint_as_float(w4[c]);
                else e = to_f<DT>(static_cast<S>(w4[c / 2] >> (16 * (c & 1))));
                const float p = e * wt[i0 + j];
                acc[c] = i0 + j == 0 ? p : acc[c] + p;
              }
            }
          }
        }
        float* o = out + static_cast<int64_t>(t) * D + d0;
#pragma unroll
        for (int c = 0; c < VEC; c += 4)
          *reinterpret_cast<float4*>(o + c) = make_float4(acc[c], acc[c + 1], acc[c + 2], acc[c + 3]);
      }
      __syncthreads();
      continue;
    }
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


// ---------------------------------------------------------------------------
// One token's MoE experts (T = 1 decode, mlx/src/nn/moe.rs:55-183 for a single
// row): routing, the fused gate_up SwiGLU of the k routed experts and their
// down projections with the ordered weighted combine, in two launches instead
// of route + gather + gather + combine.  Affine 4-bit experts, x in the
// scales' 16-bit type.
struct TokArgs {
  const void* logits;  // [E], dtype LT
  const char* x;       // [H]
  const uint32_t* gw;  // gate_up codes [E, 2I, H / 8]
  const uint16_t* gs;  // gate_up scales / biases [E, 2I, H / gs]
  const uint16_t* gb;
  const uint32_t* dw;  // down codes [E, D, I / 8]
  const uint16_t* ds;  // down scales / biases [E, D, I / gs]
  const uint16_t* db;
  uint16_t* h;         // [k, I] SwiGLU rows (workspace)
  float* scores;       // [k] (workspace)
  int32_t* experts;    // [k] (workspace)
  float* out;          // [D]
  int E, k, norm, H, I, D, gshift;
};

// Kernel 1: grid (ceil(I / 2), k), one wave each.  Every wave routes the
// token (ALU work on 64 lanes instead of a launch of its own), takes slot
// blockIdx.y's expert and reduces its gate rows o0, o0 + 1 and up rows
// I + o0, I + o0 + 1 as the M = 1 GEMV does (lane l owns chunks l, l + 64,
// ...), writing h[slot, o] = silu(gate) * up.
template <int LT, int PL, int XT, int CPL>
__global__ __launch_bounds__(64) void moe_token_glu_kernel(TokArgs a) {
  using XS = uint16_t;
  const int lane = threadIdx.x;
  const int slot = blockIdx.y;
  float sc;
  int ex;
  route_token<LT, PL>(static_cast<const typename Store<LT>::T*>(a.logits), a.E, a.k, a.norm, sc, ex);
  const int e = __shfl(ex, slot, 64);
  if (blockIdx.x == 0 && slot == 0 && lane < a.k) {
    a.scores[lane] = sc;
    a.experts[lane] = ex;
  }
  const int I = a.I, H = a.H, C = H >> 5;
  const int o0 = blockIdx.x * 2;
  XS* h = a.h + static_cast<int64_t>(slot) * I;
  if (e < 0) return;  // the combine skips the slot
  const int64_t wrow = H >> 1, srow = H >> a.gshift;
  uint32_t P[CPL][16];
  float xs[CPL];
  int cidx[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    cidx[j] = min(lane + 64 * j, C - 1);
    const u32x4_t* xc = reinterpret_cast<const u32x4_t*>(a.x + static_cast<int64_t>(cidx[j]) * 64);
    uint32_t X[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t v = xc[i];
      X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
    }
    make_pairs<XT>(X, P[j], xs[j]);
    if (lane + 64 * j >= C) xs[j] = 0.f;
  }
  float red[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int o = min(o0 + (r & 1), I - 1);
    const int64_t row = static_cast<int64_t>(e) * 2 * I + (r < 2 ? o : I + o);
    const char* wr = reinterpret_cast<const char*>(a.gw) + row * wrow;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const u32x4_t wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wr + cidx[j] * 16));
      const int64_t g = row * srow + ((cidx[j] << 5) >> a.gshift);
      const float s = to_f<XT>(a.gs[g]), b = to_f<XT>(a.gb[g]);
      float d = chunk_dot<XT>(wv, P[j]);
      if (lane + 64 * j >= C) d = 0.f;
      acc = fmaf(s, fmaf(-Magic<XT>::c, xs[j], d), fmaf(b, xs[j], acc));
    }
    red[r] = dpp_sum_to_lane63(acc);
  }
  if (lane == 63) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (o0 + i < I) h[o0 + i] = swiglu_out<XT>(red[i], red[2 + i]);
  }
}

// 16-lane sum (a row of the wave), left in every lane of the row
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

// Kernel 2: grid ceil(D / TOK_RB), TOK_RB output columns per workgroup of
// ceil(k / 4) waves.  The valid slots are ranked by (expert, slot) -- the
// combine's order for rows in (token, slot) order -- and each 16-lane row of
// wave w reduces the down row of the slot of rank 4 w + row (chunks c,
// c + 16, ... of I / 32), so every slot's loads are in flight at once.  Each
// product is rounded to the 16-bit type (the down gather's output), then the
// column's ordered sum of score * y runs in fp32 as moe_combine_kernel's does.
constexpr int TOK_RB = 4;
template <int XT, int CPLD>
__global__ __launch_bounds__(512) void moe_token_down_kernel(TokArgs a) {
  __shared__ int order[32];
  __shared__ float wt[32];
  __shared__ float ys[TOK_RB][32];
  __shared__ int nv_s;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int k = a.k, E = a.E, I = a.I, D = a.D, CI = I >> 5;
  const int n0 = blockIdx.x * TOK_RB;
  if (wave == 0) {
    bool ok = false;
    if (lane < k) {
      const int ex = a.experts[lane];
      ok = ex >= 0 && ex < E;
      int rank = 0;
      for (int j = 0; j < k; ++j) {
        const int ej = a.experts[j];
        const bool okj = ej >= 0 && ej < E;
        rank += (okj && (ej < ex || (ej == ex && j < lane))) ? 1 : 0;
      }
      if (ok) {
        order[rank] = lane;
        wt[rank] = a.scores[lane];
      }
    }
    const int nv = __popcll(__ballot(ok));
    if (lane == 0) nv_s = nv;
  }
  __syncthreads();
  const int nv = nv_s;
  const int g = lane >> 4, c = lane & 15;
  const int64_t wrow = I >> 1, srow = I >> a.gshift;
  if (4 * wave < nv) {  // wave-uniform
    const int r = min(4 * wave + g, nv - 1);
    const int slot = order[r];
    const int e = a.experts[slot];
    const char* hb = reinterpret_cast<const char*>(a.h + static_cast<int64_t>(slot) * I);
    uint32_t P[CPLD][16];
    float xs[CPLD];
    int cidx[CPLD];
#pragma unroll
    for (int j = 0; j < CPLD; ++j) {
      cidx[j] = min(c + 16 * j, CI - 1);
      const u32x4_t* xc = reinterpret_cast<const u32x4_t*>(hb + static_cast<int64_t>(cidx[j]) * 64);
      uint32_t X[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4_t v = xc[i];
        X[4 * i] = v.x; X[4 * i + 1] = v.y; X[4 * i + 2] = v.z; X[4 * i + 3] = v.w;
      }
      make_pairs<XT>(X, P[j], xs[j]);
      if (c + 16 * j >= CI) xs[j] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < TOK_RB; ++i) {
      const int64_t row = static_cast<int64_t>(e) * D + min(n0 + i, D - 1);
      const char* wr = reinterpret_cast<const char*>(a.dw) + row * wrow;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < CPLD; ++j) {
        const u32x4_t wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wr + cidx[j] * 16));
        const int64_t gi = row * srow + ((cidx[j] << 5) >> a.gshift);
        const float s = to_f<XT>(a.ds[gi]), b = to_f<XT>(a.db[gi]);
        float d = chunk_dot<XT>(wv, P[j]);
        if (c + 16 * j >= CI) d = 0.f;
        acc = fmaf(s, fmaf(-Magic<XT>::c, xs[j], d), fmaf(b, xs[j], acc));
      }
      acc = row16_sum(acc);
      if (c == 0 && 4 * wave + g < nv) ys[i][4 * wave + g] = to_f<XT>(from_f<XT>(acc));
    }
  }
  __syncthreads();
  if (t < TOK_RB && n0 + t < D) {
    float acc = 0.f;
    for (int r = 0; r < nv; ++r) {
      const float p = ys[t][r] * wt[r];
      acc = r == 0 ? p : acc + p;
    }
    a.out[n0 + t] = acc;
  }
}

template <int LT, int PL, int XT>
hipError_t token_glu_cpl(const TokArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((a.I + 1) / 2), static_cast<unsigned>(a.k));
  switch (((a.H >> 5) + 63) / 64) {
    case 1: hipLaunchKernelGGL((moe_token_glu_kernel<LT, PL, XT, 1>), grid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((moe_token_glu_kernel<LT, PL, XT, 2>), grid, dim3(64), 0, st, a); break;
    case 3: hipLaunchKernelGGL((moe_token_glu_kernel<LT, PL, XT, 3>), grid, dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((moe_token_glu_kernel<LT, PL, XT, 4>), grid, dim3(64), 0, st, a); break;
  }
  return hipGetLastError();
}

template <int LT, int XT>
hipError_t token_glu_pl(const TokArgs& a, hipStream_t st) {
  const int pl = (a.E + 63) / 64;
  if (pl <= 1) return token_glu_cpl<LT, 1, XT>(a, st);
  if (pl <= 2) return token_glu_cpl<LT, 2, XT>(a, st);
  if (pl <= 4) return token_glu_cpl<LT, 4, XT>(a, st);
  return token_glu_cpl<LT, 8, XT>(a, st);
}

template <int XT>
hipError_t token_run(const TokArgs& a, int lt, hipStream_t st) {
  hipError_t e = lt == F32 ? token_glu_pl<F32, XT>(a, st)
                           : lt == F16 ? token_glu_pl<F16, XT>(a, st) : token_glu_pl<BF16, XT>(a, st);
  if (e != hipSuccess) return e;
  const dim3 grid(static_cast<unsigned>((a.D + TOK_RB - 1) / TOK_RB));
  const dim3 block(64 * ((a.k + 3) / 4));
  switch (((a.I >> 5) + 15) / 16) {
    case 1: hipLaunchKernelGGL((moe_token_down_kernel<XT, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((moe_token_down_kernel<XT, 2>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((moe_token_down_kernel<XT, 3>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((moe_token_down_kernel<XT, 4>), grid, block, 0, st, a); break;
  }
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
  // 16-byte column pieces when every row starts 16-byte aligned (256-expert
  // top-8 block, D = 2048: T = 512 block 199 -> 194 us, T = 1 18.7 -> 18.0 us)
  const int vec = dt == F32 ? 4 : 8;
  if (D % vec == 0 && (reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out)) % 16 == 0) {
    const dim3 gv(grid.x, static_cast<unsigned>((D / vec + 255) / 256));
    switch (dt) {
      case F32:
        hipLaunchKernelGGL((moe_combine_kernel<F32, 4>), gv, dim3(256), 0, st, static_cast<const float*>(y), inverse,
                           experts, scores, out, T, k, D, E, n);
        return hipGetLastError();
      case F16:
        hipLaunchKernelGGL((moe_combine_kernel<F16, 8>), gv, dim3(256), 0, st, static_cast<const uint16_t*>(y),
                           inverse, experts, scores, out, T, k, D, E, n);
        return hipGetLastError();
      case BF16:
        hipLaunchKernelGGL((moe_combine_kernel<BF16, 8>), gv, dim3(256), 0, st, static_cast<const uint16_t*>(y),
                           inverse, experts, scores, out, T, k, D, E, n);
        return hipGetLastError();
      default:
        return hipErrorInvalidValue;
    }
  }
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


bool moe_token_supported(int E, int k, int H, int I, int D, int gs) {
  return E >= 1 && E <= 512 && k >= 1 && k <= 32 && k <= E && H % 32 == 0 && H >= 32 && H <= 8192 && I % 32 == 0 &&
         I >= 32 && I <= 2048 && D >= 1 && (gs == 32 || gs == 64 || gs == 128);
}

hipError_t launch_moe_token(const void* logits, int lt, const void* x, int xt, const uint32_t* gw, const void* gsc,
                            const void* gbi, const uint32_t* dw, const void* dsc, const void* dbi, int E, int k,
                            bool norm, int H, int I, int D, int gs, float* out, hipStream_t st) {
  if (!moe_token_supported(E, k, H, I, D, gs) || (xt != BF16 && xt != F16)) return hipErrorInvalidValue;
  // workspace: h [k, I] (16-bit), then scores [k] and experts [k] (128 B each)
  const size_t hbytes = (static_cast<size_t>(k) * I * 2 + 255) / 256 * 256;
  void* ws = nullptr;
  hipError_t e = workspace_get(st, WS_MOE, hbytes + 2 * 128, &ws);
  if (e != hipSuccess) return e;
  TokArgs a;
  a.logits = logits;
  a.x = static_cast<const char*>(x);
  a.gw = gw;
  a.gs = static_cast<const uint16_t*>(gsc);
  a.gb = static_cast<const uint16_t*>(gbi);
  a.dw = dw;
  a.ds = static_cast<const uint16_t*>(dsc);
  a.db = static_cast<const uint16_t*>(dbi);
  a.h = static_cast<uint16_t*>(ws);
  a.scores = reinterpret_cast<float*>(static_cast<char*>(ws) + hbytes);
  a.experts = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + hbytes + 128);
  a.out = out;
  a.E = E;
  a.k = k;
  a.norm = norm ? 1 : 0;
  a.H = H;
  a.I = I;
  a.D = D;
  a.gshift = __builtin_ctz(gs);
  return xt == BF16 ? token_run<BF16>(a, lt, st) : token_run<F16>(a, lt, st);
}

}  // namespace iqmm
