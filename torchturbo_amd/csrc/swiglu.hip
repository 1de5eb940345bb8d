// SwiGLU with the expert probability weighting, forward and backward.
//
// x [rows, 2F] = [gate | up]. Forward (rounding points as PyTorch on the
// reference path):
//   s = round(silu(gate));  a = round(s * up);  out = round(a * p)
// where the last product is formed in the promoted dtype of (x, p).
// Backward (autograd of the same expression):
//   g  = grad_out (as fp32);         da = round_x(g * p)
//   dp = sum_f g * a  (per row)      ds = round(da * up);  dup = round(da * s)
//   dgate = round(ds * sigmoid(gate) * (1 + gate * (1 - sigmoid(gate))))
// Elementwise passes are HBM-bound; rows are handled by one wave each so the
// per-row probability gradient is a wave reduction.
#include <math.h>

#include "common.h"

namespace {

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

template <class TT, int V>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(
    const typename TT::storage* __restrict__ x, int64_t rows, int64_t F,
    const void* __restrict__ probs, int pdt, int prod_dt, int xdt,
    typename TT::storage* __restrict__ out) {
  typedef typename TT::storage St;
  const int64_t nv = F / V;
  const int64_t total = rows * nv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / nv;
    const int64_t v = i - r * nv;
    St g[V], u[V], o[V];
    __builtin_memcpy(g, x + r * 2 * F + v * V, sizeof(g));
    __builtin_memcpy(u, x + r * 2 * F + F + v * V, sizeof(u));
    const float p = probs != nullptr ? load_as_f32(probs, pdt, r) : 1.0f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float s = round_to(silu_f(TT::to_f32(g[k])), xdt);
      float a = round_to(s * TT::to_f32(u[k]), xdt);
      if (probs != nullptr) a = round_to(a * p, prod_dt);
      o[k] = TT::from_f32(a);
    }
    __builtin_memcpy(out + r * F + v * V, o, sizeof(o));
  }
}

template <class TT, int V>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(
    const typename TT::storage* __restrict__ x, int64_t rows, int64_t F,
    const void* __restrict__ probs, int pdt, int prod_dt, int xdt,
    const typename TT::storage* __restrict__ gout, typename TT::storage* __restrict__ gx,
    void* __restrict__ gprobs) {
  typedef typename TT::storage St;
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x / TT_WAVE) + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole wave
  const int lane = lane_id();
  const float p = probs != nullptr ? load_as_f32(probs, pdt, r) : 1.0f;
  float dp = 0.f;
  const int64_t nv = F / V;
  for (int64_t v = lane; v < nv; v += TT_WAVE) {
    St g[V], u[V], d[V], og[V], ou[V];
    __builtin_memcpy(g, x + r * 2 * F + v * V, sizeof(g));
    __builtin_memcpy(u, x + r * 2 * F + F + v * V, sizeof(u));
    __builtin_memcpy(d, gout + r * F + v * V, sizeof(d));
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float gf = TT::to_f32(g[k]);
      const float uf = TT::to_f32(u[k]);
      const float den = 1.0f + expf(-gf);
      const float sig = 1.0f / den;
      const float s = round_to(gf / den, xdt);
      float da;
      if (probs != nullptr) {
        const float gd = TT::to_f32(d[k]);
        const float a = round_to(s * uf, xdt);
        dp += round_to(gd * a, prod_dt);
        da = round_to(gd * p, xdt);
      } else {
        da = TT::to_f32(d[k]);
      }
      const float ds = round_to(da * uf, xdt);
      ou[k] = TT::from_f32(da * s);
      og[k] = TT::from_f32(ds * (sig * (1.0f + gf * (1.0f - sig))));
    }
    __builtin_memcpy(gx + r * 2 * F + v * V, og, sizeof(og));
    __builtin_memcpy(gx + r * 2 * F + F + v * V, ou, sizeof(ou));
  }
  if (gprobs != nullptr) {
    dp = wave_sum(dp);
    if (lane == 0) store_from_f32(gprobs, pdt, r, dp);
  }
}

bool float_dtype(int d) { return d == TT_F32 || d == TT_BF16 || d == TT_F16; }

template <class TT>
int launch_fwd(const void* x, int64_t rows, int64_t F, const void* probs, int pdt, int prod_dt,
               int xdt, void* out, hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       static_cast<uintptr_t>(F * sizeof(St));
  const St* xp = static_cast<const St*>(x);
  St* op = static_cast<St*>(out);
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    const int64_t total = rows * (F / V);
    const unsigned grid = (unsigned)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
    hipLaunchKernelGGL((swiglu_fwd_kernel<TT, V>), dim3(grid), dim3(256), 0, s, xp, rows, F,
                       probs, pdt, prod_dt, xdt, op);
  } else {
    const int64_t total = rows * F;
    const unsigned grid = (unsigned)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
    hipLaunchKernelGGL((swiglu_fwd_kernel<TT, 1>), dim3(grid), dim3(256), 0, s, xp, rows, F,
                       probs, pdt, prod_dt, xdt, op);
  }
  return tt_check_launch("swiglu_fwd");
}

template <class TT>
int launch_bwd(const void* x, int64_t rows, int64_t F, const void* probs, int pdt, int prod_dt,
               int xdt, const void* gout, void* gx, void* gprobs, hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gout) |
                       reinterpret_cast<uintptr_t>(gx) | static_cast<uintptr_t>(F * sizeof(St));
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    hipLaunchKernelGGL((swiglu_bwd_kernel<TT, V>), grid, dim3(256), 0, s, static_cast<const St*>(x),
                       rows, F, probs, pdt, prod_dt, xdt, static_cast<const St*>(gout),
                       static_cast<St*>(gx), gprobs);
  } else {
    hipLaunchKernelGGL((swiglu_bwd_kernel<TT, 1>), grid, dim3(256), 0, s, static_cast<const St*>(x),
                       rows, F, probs, pdt, prod_dt, xdt, static_cast<const St*>(gout),
                       static_cast<St*>(gx), gprobs);
  }
  return tt_check_launch("swiglu_bwd");
}

}  // namespace

extern "C" int tt_swiglu_fwd(const void* x, int dtype, int64_t rows, int64_t ffn,
                             const void* probs, int probs_dtype, void* out, void* stream) {
  TT_REQUIRE(float_dtype(dtype), "swiglu: unsupported dtype %d", dtype);
  TT_REQUIRE(rows >= 0 && ffn >= 0, "swiglu: negative sizes");
  if (probs != nullptr) TT_REQUIRE(float_dtype(probs_dtype), "swiglu: unsupported probs dtype");
  if (rows == 0 || ffn == 0) return TT_OK;
  const int prod_dt = probs != nullptr ? tt_promote(dtype, probs_dtype) : dtype;
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_fwd<BF16T>(x, rows, ffn, probs, probs_dtype, prod_dt, dtype, out, s);
    case TT_F16: return launch_fwd<F16T>(x, rows, ffn, probs, probs_dtype, prod_dt, dtype, out, s);
    default: return launch_fwd<F32T>(x, rows, ffn, probs, probs_dtype, prod_dt, dtype, out, s);
  }
}

extern "C" int tt_swiglu_bwd(const void* x, int dtype, int64_t rows, int64_t ffn,
                             const void* probs, int probs_dtype, const void* grad_out,
                             void* grad_x, void* grad_probs, void* stream) {
  TT_REQUIRE(float_dtype(dtype), "swiglu_bwd: unsupported dtype %d", dtype);
  TT_REQUIRE(rows >= 0 && ffn >= 0, "swiglu_bwd: negative sizes");
  if (probs != nullptr) TT_REQUIRE(float_dtype(probs_dtype), "swiglu_bwd: unsupported probs dtype");
  if (grad_probs != nullptr) TT_REQUIRE(probs != nullptr, "swiglu_bwd: grad_probs needs probs");
  if (rows == 0) return TT_OK;
  const int prod_dt = probs != nullptr ? tt_promote(dtype, probs_dtype) : dtype;
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_bwd<BF16T>(x, rows, ffn, probs, probs_dtype, prod_dt, dtype, grad_out, grad_x, grad_probs, s);
    case TT_F16: return launch_bwd<F16T>(x, rows, ffn, probs, probs_dtype, prod_dt, dtype, grad_out, grad_x, grad_probs, s);
    default: return launch_bwd<F32T>(x, rows, ffn, probs, probs_dtype, prod_dt, dtype, grad_out, grad_x, grad_probs, s);
  }
}
