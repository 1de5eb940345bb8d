// Token permutation kernels: scatter of token rows into expert-major packed
// rows, gather-sum back into token rows (optionally weighted), their
// backward passes, and the chunk reorder.
//
// All kernels are token-major: block t reads the k row ids of token t once
// (LDS broadcast) and moves whole rows with 16-byte vector accesses, so each
// source row is read once and each destination row written once. Row ids
// outside [0, M) are skipped, never dereferenced.
#include "common.h"

namespace {

constexpr int kMaxTopk = 64;

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

template <int VB>
struct Vec;
template <>
struct Vec<16> { typedef uint4 type; };
template <>
struct Vec<8> { typedef uint2 type; };
template <>
struct Vec<4> { typedef uint32_t type; };
template <>
struct Vec<2> { typedef uint16_t type; };

// packed[rows[t, j]] = tokens[t] (raw bytes, any dtype).
template <int VB>
__global__ __launch_bounds__(1024) void permute_scatter_kernel(
    const char* __restrict__ tokens, int64_t row_bytes, int K, const int32_t* __restrict__ rows,
    char* __restrict__ packed, int64_t M) {
  typedef typename Vec<VB>::type V;
  __shared__ int rs[kMaxTopk];
  const int64_t t = blockIdx.x;
  if (threadIdx.x < K) rs[threadIdx.x] = rows[t * K + threadIdx.x];
  __syncthreads();
  const int64_t nv = row_bytes / VB;
  const V* src = reinterpret_cast<const V*>(tokens + t * row_bytes);
  for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) {
    const V x = src[v];
    for (int j = 0; j < K; ++j) {
      const int r = rs[j];
      if (r >= 0 && r < M) reinterpret_cast<V*>(packed + (int64_t)r * row_bytes)[v] = x;
    }
  }
}

// Sort the token's (row, weight, expert) triples by ascending row in LDS.
__device__ __forceinline__ void sort_rows(int* rs, float* ws, int* es, int K) {
  if (threadIdx.x == 0) {
    for (int a = 1; a < K; ++a) {
      const int r = rs[a];
      const float w = ws[a];
      const int e = es[a];
      int b = a - 1;
      while (b >= 0 && rs[b] > r) {
        rs[b + 1] = rs[b];
        ws[b + 1] = ws[b];
        es[b + 1] = es[b];
        --b;
      }
      rs[b + 1] = r;
      ws[b + 1] = w;
      es[b + 1] = e;
    }
  }
  __syncthreads();
}

// out[t] = sum over the token's rows in ascending row order, fp32
// accumulation, one final rounding. With probs, each row is first
// multiplied by its weight and rounded to the promoted dtype `prod_dt`.
template <class TT, int V>
__global__ __launch_bounds__(256) void unpermute_gather_kernel(
    const typename TT::storage* __restrict__ packed, int64_t H, int K,
    const int32_t* __restrict__ rows, const int64_t* __restrict__ experts,
    const void* __restrict__ probs, int pdt, int E, int prod_dt,
    typename TT::storage* __restrict__ out, int64_t M) {
  typedef typename TT::storage St;
  __shared__ int rs[kMaxTopk];
  __shared__ float ws[kMaxTopk];
  __shared__ int es[kMaxTopk];
  const int64_t t = blockIdx.x;
  if (threadIdx.x < K) {
    const int j = threadIdx.x;
    rs[j] = rows[t * K + j];
    int64_t e = experts != nullptr ? experts[t * K + j] : 0;
    es[j] = (int)e;
    ws[j] = (probs != nullptr && e >= 0 && e < E) ? load_as_f32(probs, pdt, t * E + e) : 1.0f;
  }
  __syncthreads();
  sort_rows(rs, ws, es, K);
  const int64_t nv = H / V;
  for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) {
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
    for (int j = 0; j < K; ++j) {
      const int r = rs[j];
      if (r < 0 || r >= M) continue;
      St x[V];
      __builtin_memcpy(x, packed + (int64_t)r * H + v * V, sizeof(x));
      if (probs != nullptr) {
        const float w = ws[j];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] += round_to(TT::to_f32(x[i]) * w, prod_dt);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] += TT::to_f32(x[i]);
      }
    }
    St y[V];
#pragma unroll
    for (int i = 0; i < V; ++i) y[i] = TT::from_f32(round_to(acc[i], prod_dt));
    __builtin_memcpy(out + t * H + v * V, y, sizeof(y));
  }
}

// Same sum for top-k <= KMAX (small): every thread reads the token's row ids
// (uniform loads), sorts them in registers, issues all K row loads of its NS
// 16-byte column slices (v and v + blockDim.x) before adding, and
// accumulates in ascending row order. No block barrier, no LDS. NS = 2 needs
// the row's slice count to be a multiple of 2 * blockDim.x (the launch
// checks it). Row ids outside [0, M) contribute nothing (adding +0 to a sum
// that starts at +0 leaves it unchanged, so skipping and adding zero agree
// bitwise).
template <int DT>
__device__ __forceinline__ float rnd_dt(float v) {
  if constexpr (DT == TT_BF16) return bf16_to_f32(f32_to_bf16(v));
  else if constexpr (DT == TT_F16) return f16_to_f32(f32_to_f16(v));
  else return v;
}
template <int PD>
__device__ __forceinline__ float load_w(const void* p, int64_t i) {
  if constexpr (PD == TT_F32) return static_cast<const float*>(p)[i];
  else if constexpr (PD == TT_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

constexpr int kNoProbs = -1;

template <class TT, int XD, int PD, int V, int KMAX, int NS>
__global__ __launch_bounds__(1024) void unpermute_small_kernel(
    const typename TT::storage* __restrict__ packed, int64_t H, int K,
    const int32_t* __restrict__ rows, const int64_t* __restrict__ experts,
    const void* __restrict__ probs, int E, typename TT::storage* __restrict__ out, int64_t M) {
  typedef typename TT::storage St;
  constexpr int PR = (PD == kNoProbs || PD == XD) ? XD : TT_F32;
  const int64_t t = blockIdx.x;
  int rs[KMAX], es[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    rs[j] = 0x7fffffff;
    es[j] = -1;
    if (j < K) {
      const int r = rows[t * K + j];
      rs[j] = (r >= 0 && r < M) ? r : 0x7fffffff;
      if constexpr (PD != kNoProbs) {
        const int64_t e = experts[t * K + j];
        es[j] = (e >= 0 && e < E) ? (int)e : -1;
      }
    }
  }
  // Insertion sort by row (K <= KMAX <= 8), carrying the expert ids; the
  // weights are gathered after the sort, alongside the rows, so the row
  // loads do not wait for them.
#pragma unroll
  for (int a = 1; a < KMAX; ++a)
#pragma unroll
    for (int b = a; b > 0; --b) {
      const bool sw = rs[b - 1] > rs[b];
      const int r0 = rs[b - 1], r1 = rs[b];
      const int e0 = es[b - 1], e1 = es[b];
      rs[b - 1] = sw ? r1 : r0;
      rs[b] = sw ? r0 : r1;
      es[b - 1] = sw ? e1 : e0;
      es[b] = sw ? e0 : e1;
    }
  // Weights also loaded unconditionally (a token's own row of probs, column
  // 0 for an invalid expert) so that the loads are not serialized.
  float ws[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    ws[j] = 1.0f;
    if constexpr (PD != kNoProbs) {
      const float w = load_w<PD>(probs, t * E + (es[j] >= 0 ? es[j] : 0));
      ws[j] = es[j] >= 0 ? w : 1.0f;
    }
  }
  const int64_t nv = H / V;
  if (M == 0) {  // no rows: every term is zero
    St y[V];
#pragma unroll
    for (int i = 0; i < V; ++i) y[i] = TT::from_f32(0.0f);
    for (int64_t v = threadIdx.x; v < nv; v += blockDim.x)
      __builtin_memcpy(out + t * H + v * V, y, sizeof(y));
    return;
  }
  // Rows are loaded unconditionally (an invalid row reads row 0 and counts
  // as zero): a load under a per-row branch would be waited for before the
  // next one is issued. Each packed row is read once: streaming loads. Two
  // slices per thread keep 2 K loads in flight per thread (Qwen shape, 128
  // threads: 2-3 % faster than one slice at 256 threads; four slices at 64
  // threads lose occupancy and run 1.5x slower).
  for (int64_t v = threadIdx.x; v < nv; v += NS * (int64_t)blockDim.x) {
    St x[NS][KMAX][V];
#pragma unroll
    for (int u = 0; u < NS; ++u)
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        const int64_t r = rs[j] != 0x7fffffff ? rs[j] : 0;
        load_stream<sizeof(x[u][j])>(x[u][j], packed + r * H + (v + u * (int64_t)blockDim.x) * V);
      }
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      float acc[V];
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = 0.f;
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        const bool ok = rs[j] != 0x7fffffff;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const float xv = ok ? TT::to_f32(x[u][j][i]) : 0.0f;
          if constexpr (PD != kNoProbs) acc[i] += rnd_dt<PR>(xv * ws[j]);
          else acc[i] += xv;
        }
      }
      St y[V];
#pragma unroll
      for (int i = 0; i < V; ++i) y[i] = TT::from_f32(rnd_dt<PR>(acc[i]));
      // Streaming store: measured in the layer step, the token rows written
      // this way leave the caches to the kernels that follow (Qwen unpermute
      // 69 -> 72 % of HBM bandwidth, and the step faster).
      store_stream<sizeof(y)>(out + t * H + (v + u * (int64_t)blockDim.x) * V, y);
    }
  }
}

// Weighted-unpermute backward. grad_packed[r_j] = cast(grad_out[t] * w_j);
// grad_probs[t, e_j] = sum_h grad_out[t, h] * packed[r_j, h]; zeros elsewhere.
template <class TT, int V, int KMAX>
__global__ __launch_bounds__(256) void unpermute_bwd_kernel(
    const typename TT::storage* __restrict__ gout, const typename TT::storage* __restrict__ packed,
    int64_t H, int K, const int32_t* __restrict__ rows, const int64_t* __restrict__ experts,
    const void* __restrict__ probs, int pdt, int E, typename TT::storage* __restrict__ gpacked,
    void* __restrict__ gprobs, int64_t M) {
  typedef typename TT::storage St;
  __shared__ int rs[KMAX];
  __shared__ float ws[KMAX];
  __shared__ int es[KMAX];
  __shared__ float part[KMAX][256 / TT_WAVE];
  const int64_t t = blockIdx.x;
  if (threadIdx.x < K) {
    const int j = threadIdx.x;
    rs[j] = rows[t * K + j];
    const int64_t e = experts[t * K + j];
    es[j] = (e >= 0 && e < E) ? (int)e : -1;
    ws[j] = es[j] >= 0 ? load_as_f32(probs, pdt, t * E + e) : 0.f;
  }
  __syncthreads();
  float dot[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) dot[j] = 0.f;
  const int64_t nv = H / V;
  for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) {
    St g[V];
    __builtin_memcpy(g, gout + t * H + v * V, sizeof(g));
    float gf[V];
#pragma unroll
    for (int i = 0; i < V; ++i) gf[i] = TT::to_f32(g[i]);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j >= K) break;
      const int r = rs[j];
      if (r < 0 || r >= M) continue;
      St x[V], o[V];
      __builtin_memcpy(x, packed + (int64_t)r * H + v * V, sizeof(x));
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        o[i] = TT::from_f32(gf[i] * ws[j]);
        d += gf[i] * TT::to_f32(x[i]);
      }
      dot[j] += d;
      __builtin_memcpy(gpacked + (int64_t)r * H + v * V, o, sizeof(o));
    }
  }
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= K) break;
    const float s = wave_sum(dot[j]);
    if (lane_id() == 0) part[j][wave] = s;
  }
  __syncthreads();
  const int nw = blockDim.x / TT_WAVE;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float v = 0.f;
    for (int j = 0; j < K; ++j)
      if (es[j] == e) {
        v = 0.f;
        for (int w = 0; w < nw; ++w) v += part[j][w];
      }
    store_from_f32(gprobs, pdt, t * E + e, v);
  }
}

// grad_dense[t, e] = grad_packed[r_j] where e == experts[t, j], else 0. One
// wave per token: the wave zeroes a private LDS row of E values, the token's
// k lanes drop their gradients into it, and the row is written out whole.
__global__ __launch_bounds__(256) void packed_probs_bwd_kernel(
    const void* __restrict__ gpacked, int dt, int64_t T, int K, int E,
    const int32_t* __restrict__ rows, const int64_t* __restrict__ experts,
    void* __restrict__ gdense, int64_t M) {
  extern __shared__ float prow[];  // [4][E]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t >= T) return;  // whole wave; no block barrier below
  float* row = prow + (int64_t)wave * E;
  for (int e = lane; e < E; e += TT_WAVE) row[e] = 0.f;
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the zeros land before the values
  __builtin_amdgcn_wave_barrier();
  for (int j = lane; j < K; j += TT_WAVE) {
    const int64_t e = experts[t * K + j];
    const int r = rows[t * K + j];
    if (e >= 0 && e < E && r >= 0 && r < M) row[e] = load_as_f32(gpacked, dt, r);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  for (int e = lane; e < E; e += TT_WAVE) store_from_f32(gdense, dt, t * E + e, row[e]);
}

// Chunk reorder: block (i, y) copies rows y, y + gridDim.y, ... of the i-th
// output chunk, which is input chunk sorted[i].
template <int VB>
__global__ __launch_bounds__(256) void sort_chunks_kernel(
    const char* __restrict__ in, int64_t row_bytes, const int64_t* __restrict__ sizes,
    const int64_t* __restrict__ sorted, int C, const char* __restrict__ probs, int pbytes,
    char* __restrict__ out, char* __restrict__ oprobs, int64_t rows) {
  typedef typename Vec<VB>::type V;
  __shared__ int64_t red[2][256 / TT_WAVE];
  const int i = blockIdx.x;
  const int64_t c = sorted[i];
  if (c < 0 || c >= C) return;  // uniform for the block
  int64_t so = 0, ss = 0;
  for (int q = threadIdx.x; q < C; q += blockDim.x) {
    const int64_t n = sizes[q];
    if (q < c) ss += n;
  }
  for (int q = threadIdx.x; q < i; q += blockDim.x) {
    const int64_t cq = sorted[q];
    if (cq >= 0 && cq < C) so += sizes[cq];
  }
  for (int off = 32; off > 0; off >>= 1) {
    so += __shfl_xor(so, off, TT_WAVE);
    ss += __shfl_xor(ss, off, TT_WAVE);
  }
  if (lane_id() == 0) {
    red[0][threadIdx.x >> 6] = so;
    red[1][threadIdx.x >> 6] = ss;
  }
  __syncthreads();
  int64_t out_start = 0, src_start = 0;
  for (int w = 0; w < (int)(blockDim.x / TT_WAVE); ++w) {
    out_start += red[0][w];
    src_start += red[1][w];
  }
  const int64_t n = sizes[c];
  const int64_t nv = row_bytes / VB;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) {
    const int64_t src = src_start + r, dst = out_start + r;
    if (src >= rows || dst >= rows) break;
    const V* a = reinterpret_cast<const V*>(in + src * row_bytes);
    V* b = reinterpret_cast<V*>(out + dst * row_bytes);
    for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) b[v] = a[v];
    if (probs != nullptr && threadIdx.x == 0) {
      if (pbytes == 4)
        reinterpret_cast<uint32_t*>(oprobs)[dst] = reinterpret_cast<const uint32_t*>(probs)[src];
      else
        reinterpret_cast<uint16_t*>(oprobs)[dst] = reinterpret_cast<const uint16_t*>(probs)[src];
    }
  }
}

int pick_vb(const void* a, const void* b, int64_t row_bytes) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       static_cast<uintptr_t>(row_bytes);
  if (al % 16 == 0) return 16;
  if (al % 8 == 0) return 8;
  if (al % 4 == 0) return 4;
  return 2;
}

unsigned block_for(int64_t nv) {
  if (nv <= 64) return 64;
  if (nv <= 128) return 128;
  return 256;
}

bool float_dtype(int d) { return d == TT_F32 || d == TT_BF16 || d == TT_F16; }

template <class TT, int XD>
int launch_unpermute(const void* packed, int64_t T, int64_t H, int K, const int32_t* rows,
                     const int64_t* experts, const void* probs, int pdt, int E, int prod_dt,
                     void* out, int64_t M, hipStream_t s) {
  typedef typename TT::storage St;
  const int esz = sizeof(St);
  const uintptr_t al = reinterpret_cast<uintptr_t>(packed) | reinterpret_cast<uintptr_t>(out) |
                       static_cast<uintptr_t>(H * esz);
  const St* p = static_cast<const St*>(packed);
  St* o = static_cast<St*>(out);
  if (al % 16 == 0 && K <= 8) {
    constexpr int V = 16 / sizeof(St);
    const int64_t nvb = H / V;
    const dim3 grid((unsigned)T);
    // Two 16-byte column slices per thread when they split the row exactly
    // over 64-1024 threads (H 2048 bf16: 128 threads; 4096: 256; 7168: 448),
    // else one slice per thread, so that every thread issues all of its row
    // loads at once.
    if (nvb % 128 == 0 && nvb / 2 <= 1024) {
      const dim3 blk((unsigned)(nvb / 2));
      if (probs == nullptr) {
        if (K <= 2)
          hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, kNoProbs, V, 2, 2>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
        else
          hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, kNoProbs, V, 8, 2>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
      } else if (pdt == TT_F32) {
        if (K <= 2)
          hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_F32, V, 2, 2>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
        else
          hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_F32, V, 8, 2>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
      } else if (pdt == TT_BF16) {
        hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_BF16, V, 8, 2>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
      } else {
        hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_F16, V, 8, 2>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
      }
      return tt_check_launch("unpermute_gather");
    }
    const unsigned nthr =
        nvb <= 256 ? block_for(nvb) : (unsigned)(nvb <= 1024 ? ((nvb + 63) / 64) * 64 : 1024);
    const dim3 blk(nthr);
    if (probs == nullptr) {
      if (K <= 2)
        hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, kNoProbs, V, 2, 1>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
      else
        hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, kNoProbs, V, 8, 1>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
    } else if (pdt == TT_F32) {
      if (K <= 2)
        hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_F32, V, 2, 1>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
      else
        hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_F32, V, 8, 1>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
    } else if (pdt == TT_BF16) {
      hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_BF16, V, 8, 1>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
    } else {
      hipLaunchKernelGGL((unpermute_small_kernel<TT, XD, TT_F16, V, 8, 1>), grid, blk, 0, s, p, H, K, rows, experts, probs, E, o, M);
    }
  } else if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    hipLaunchKernelGGL((unpermute_gather_kernel<TT, V>), dim3(T), dim3(block_for(H / V)), 0, s, p,
                       H, K, rows, experts, probs, pdt, E, prod_dt, o, M);
  } else {
    hipLaunchKernelGGL((unpermute_gather_kernel<TT, 1>), dim3(T), dim3(block_for(H)), 0, s, p, H,
                       K, rows, experts, probs, pdt, E, prod_dt, o, M);
  }
  return tt_check_launch("unpermute_gather");
}

template <class TT, int KMAX>
int launch_unpermute_bwd_k(const void* gout, const void* packed, int64_t T, int64_t H, int K,
                           const int32_t* rows, const int64_t* experts, const void* probs,
                           int pdt, int E, void* gpacked, void* gprobs, int64_t M,
                           hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(gout) | reinterpret_cast<uintptr_t>(packed) |
                       reinterpret_cast<uintptr_t>(gpacked) |
                       static_cast<uintptr_t>(H * sizeof(St));
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    hipLaunchKernelGGL((unpermute_bwd_kernel<TT, V, KMAX>), dim3(T), dim3(256), 0, s,
                       static_cast<const St*>(gout), static_cast<const St*>(packed), H, K, rows,
                       experts, probs, pdt, E, static_cast<St*>(gpacked), gprobs, M);
  } else {
    hipLaunchKernelGGL((unpermute_bwd_kernel<TT, 1, KMAX>), dim3(T), dim3(256), 0, s,
                       static_cast<const St*>(gout), static_cast<const St*>(packed), H, K, rows,
                       experts, probs, pdt, E, static_cast<St*>(gpacked), gprobs, M);
  }
  return tt_check_launch("unpermute_gather_bwd");
}

template <class TT>
int launch_unpermute_bwd(const void* gout, const void* packed, int64_t T, int64_t H, int K,
                         const int32_t* rows, const int64_t* experts, const void* probs, int pdt,
                         int E, void* gpacked, void* gprobs, int64_t M, hipStream_t s) {
  if (K <= 2)
    return launch_unpermute_bwd_k<TT, 2>(gout, packed, T, H, K, rows, experts, probs, pdt, E,
                                         gpacked, gprobs, M, s);
  if (K <= 8)
    return launch_unpermute_bwd_k<TT, 8>(gout, packed, T, H, K, rows, experts, probs, pdt, E,
                                         gpacked, gprobs, M, s);
  return launch_unpermute_bwd_k<TT, 64>(gout, packed, T, H, K, rows, experts, probs, pdt, E,
                                        gpacked, gprobs, M, s);
}

}  // namespace

extern "C" int tt_permute_scatter(const void* tokens, int dtype, int64_t num_tokens,
                                  int64_t hidden, int32_t topk, const int32_t* row_indices,
                                  void* packed, void* stream) {
  TT_REQUIRE(float_dtype(dtype), "permute: unsupported dtype %d", dtype);
  TT_REQUIRE(topk >= 1 && topk <= kMaxTopk, "permute: topk must be in [1, 64]");
  TT_REQUIRE(num_tokens >= 0 && hidden >= 0, "permute: negative sizes");
  TT_REQUIRE(num_tokens <= 0x7fffffff, "permute: too many tokens");
  if (num_tokens == 0 || hidden == 0) return TT_OK;
  const int64_t row_bytes = hidden * tt_elem_size(dtype);
  const int64_t M = num_tokens * topk;
  hipStream_t s = S(stream);
  const int vb = pick_vb(tokens, packed, row_bytes);
  const dim3 grid((unsigned)num_tokens);
  // One thread per vector of the row (up to 1024): each thread loads once and
  // stores k times (DeepSeek-V3's 7168-wide rows: 66 -> 80 % of HBM bandwidth).
  const int64_t nvb = row_bytes / vb;
  const unsigned blk =
      nvb <= 256 ? block_for(nvb) : (unsigned)(nvb <= 1024 ? ((nvb + 63) / 64) * 64 : 1024);
  const char* a = static_cast<const char*>(tokens);
  char* b = static_cast<char*>(packed);
  switch (vb) {
    case 16: hipLaunchKernelGGL(permute_scatter_kernel<16>, grid, dim3(blk), 0, s, a, row_bytes, topk, row_indices, b, M); break;
    case 8: hipLaunchKernelGGL(permute_scatter_kernel<8>, grid, dim3(blk), 0, s, a, row_bytes, topk, row_indices, b, M); break;
    case 4: hipLaunchKernelGGL(permute_scatter_kernel<4>, grid, dim3(blk), 0, s, a, row_bytes, topk, row_indices, b, M); break;
    default: hipLaunchKernelGGL(permute_scatter_kernel<2>, grid, dim3(blk), 0, s, a, row_bytes, topk, row_indices, b, M); break;
  }
  return tt_check_launch("permute_scatter");
}

extern "C" int tt_unpermute_gather(const void* packed, int dtype, int64_t num_tokens,
                                   int64_t hidden, int32_t topk, const int32_t* row_indices,
                                   const int64_t* expert_indices, const void* probs,
                                   int probs_dtype, int32_t num_experts, void* out, void* stream) {
  TT_REQUIRE(float_dtype(dtype), "unpermute: unsupported dtype %d", dtype);
  TT_REQUIRE(topk >= 1 && topk <= kMaxTopk, "unpermute: topk must be in [1, 64]");
  TT_REQUIRE(num_tokens >= 0 && num_tokens <= 0x7fffffff && hidden >= 0, "unpermute: bad sizes");
  if (probs != nullptr) {
    TT_REQUIRE(float_dtype(probs_dtype), "unpermute: unsupported probs dtype %d", probs_dtype);
    TT_REQUIRE(expert_indices != nullptr && num_experts >= 1, "unpermute: weights need expert ids");
  }
  if (num_tokens == 0 || hidden == 0) return TT_OK;
  const int prod_dt = probs != nullptr ? tt_promote(dtype, probs_dtype) : dtype;
  const int64_t M = num_tokens * topk;
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_unpermute<BF16T, TT_BF16>(packed, num_tokens, hidden, topk, row_indices, expert_indices, probs, probs_dtype, num_experts, prod_dt, out, M, s);
    case TT_F16: return launch_unpermute<F16T, TT_F16>(packed, num_tokens, hidden, topk, row_indices, expert_indices, probs, probs_dtype, num_experts, prod_dt, out, M, s);
    default: return launch_unpermute<F32T, TT_F32>(packed, num_tokens, hidden, topk, row_indices, expert_indices, probs, probs_dtype, num_experts, prod_dt, out, M, s);
  }
}

extern "C" int tt_unpermute_gather_bwd(const void* grad_out, const void* packed, int dtype,
                                       int64_t num_tokens, int64_t hidden, int32_t topk,
                                       const int32_t* row_indices, const int64_t* expert_indices,
                                       const void* probs, int probs_dtype, int32_t num_experts,
                                       void* grad_packed, void* grad_probs, void* stream) {
  TT_REQUIRE(float_dtype(dtype) && float_dtype(probs_dtype), "unpermute_bwd: unsupported dtype");
  TT_REQUIRE(topk >= 1 && topk <= kMaxTopk, "unpermute_bwd: topk must be in [1, 64]");
  TT_REQUIRE(probs != nullptr && grad_probs != nullptr && expert_indices != nullptr,
             "unpermute_bwd: the weighted backward needs probs, expert ids and grad_probs");
  TT_REQUIRE(num_tokens >= 0 && num_tokens <= 0x7fffffff && hidden >= 0 && num_experts >= 1,
             "unpermute_bwd: bad sizes");
  if (num_tokens == 0) return TT_OK;
  const int64_t M = num_tokens * topk;
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_unpermute_bwd<BF16T>(grad_out, packed, num_tokens, hidden, topk, row_indices, expert_indices, probs, probs_dtype, num_experts, grad_packed, grad_probs, M, s);
    case TT_F16: return launch_unpermute_bwd<F16T>(grad_out, packed, num_tokens, hidden, topk, row_indices, expert_indices, probs, probs_dtype, num_experts, grad_packed, grad_probs, M, s);
    default: return launch_unpermute_bwd<F32T>(grad_out, packed, num_tokens, hidden, topk, row_indices, expert_indices, probs, probs_dtype, num_experts, grad_packed, grad_probs, M, s);
  }
}

extern "C" int tt_packed_probs_bwd(const void* grad_packed_probs, int dtype, int64_t num_tokens,
                                   int32_t topk, int32_t num_experts, const int32_t* row_indices,
                                   const int64_t* expert_indices, void* grad_probs_dense,
                                   void* stream) {
  TT_REQUIRE(float_dtype(dtype), "packed_probs_bwd: unsupported dtype %d", dtype);
  TT_REQUIRE(topk >= 1 && topk <= kMaxTopk && num_experts >= 1 && num_tokens >= 0,
             "packed_probs_bwd: bad sizes");
  const int64_t n = num_tokens * num_experts;
  if (n == 0) return TT_OK;
  const size_t lds = (size_t)4 * num_experts * sizeof(float);
  TT_REQUIRE(lds <= 64 * 1024, "packed_probs_bwd: too many experts (%d)", num_experts);
  hipLaunchKernelGGL(packed_probs_bwd_kernel, dim3((unsigned)((num_tokens + 3) / 4)), dim3(256),
                     lds, S(stream), grad_packed_probs, dtype, num_tokens, topk, num_experts,
                     row_indices, expert_indices, grad_probs_dense, num_tokens * topk);
  return tt_check_launch("packed_probs_bwd");
}

extern "C" int tt_sort_chunks(const void* input, int dtype, int64_t rows, int64_t hidden,
                              const int64_t* split_sizes, const int64_t* sorted_idxs,
                              int32_t num_chunks, const void* probs, int probs_dtype,
                              void* output, void* out_probs, void* stream) {
  TT_REQUIRE(float_dtype(dtype), "sort_chunks: unsupported dtype %d", dtype);
  TT_REQUIRE(num_chunks >= 0 && num_chunks <= 4096, "sort_chunks: num_chunks must be <= 4096");
  TT_REQUIRE(rows >= 0 && hidden >= 0, "sort_chunks: bad sizes");
  if (probs != nullptr && out_probs != nullptr)
    TT_REQUIRE(float_dtype(probs_dtype), "sort_chunks: unsupported probs dtype");
  if (rows == 0 || num_chunks == 0) return TT_OK;
  const int64_t row_bytes = hidden * tt_elem_size(dtype);
  const int vb = pick_vb(input, output, row_bytes);
  const dim3 grid((unsigned)num_chunks, 16);
  const char* pr = (out_probs != nullptr) ? static_cast<const char*>(probs) : nullptr;
  const int pb = tt_elem_size(probs_dtype);
  const char* a = static_cast<const char*>(input);
  char* b = static_cast<char*>(output);
  char* op = static_cast<char*>(out_probs);
  hipStream_t s = S(stream);
  switch (vb) {
    case 16: hipLaunchKernelGGL(sort_chunks_kernel<16>, grid, dim3(256), 0, s, a, row_bytes, split_sizes, sorted_idxs, num_chunks, pr, pb, b, op, rows); break;
    case 8: hipLaunchKernelGGL(sort_chunks_kernel<8>, grid, dim3(256), 0, s, a, row_bytes, split_sizes, sorted_idxs, num_chunks, pr, pb, b, op, rows); break;
    case 4: hipLaunchKernelGGL(sort_chunks_kernel<4>, grid, dim3(256), 0, s, a, row_bytes, split_sizes, sorted_idxs, num_chunks, pr, pb, b, op, rows); break;
    default: hipLaunchKernelGGL(sort_chunks_kernel<2>, grid, dim3(256), 0, s, a, row_bytes, split_sizes, sorted_idxs, num_chunks, pr, pb, b, op, rows); break;
  }
  return tt_check_launch("sort_chunks");
}
