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
//
// Layout: a row is handled by L lanes (a power of two chosen so that the
// row's 16-byte vectors divide evenly), 64 / L rows per wave; the per-row
// probability gradient is a reduction over those L lanes. All dtype choices
// are template parameters, so the element loop is branch-free. For 16-bit
// data the sigmoid uses the hardware exp2 and reciprocal (a few ulp in fp32,
// far below the 16-bit rounding that follows); fp32 data keeps expf and a
// correctly rounded division.
#include <math.h>

#include "common.h"

namespace {

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int NO_PROBS = -1;

template <class TT>
struct Traits;
template <>
struct Traits<BF16T> { static constexpr int code = TT_BF16; };
template <>
struct Traits<F16T> { static constexpr int code = TT_F16; };
template <>
struct Traits<F32T> { static constexpr int code = TT_F32; };

template <int DT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (DT == TT_BF16) return bf16_to_f32(f32_to_bf16(v));
  else if constexpr (DT == TT_F16) return f16_to_f32(f32_to_f16(v));
  else return v;
}

template <int PD>
__device__ __forceinline__ float load_prob(const void* p, int64_t r) {
  if constexpr (PD == TT_F32) return static_cast<const float*>(p)[r];
  else if constexpr (PD == TT_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[r]);
  else if constexpr (PD == TT_F16) return f16_to_f32(static_cast<const uint16_t*>(p)[r]);
  else return 1.0f;
}

template <int PD>
__device__ __forceinline__ void store_prob(void* p, int64_t r, float v) {
  if constexpr (PD == TT_F32) static_cast<float*>(p)[r] = v;
  else if constexpr (PD == TT_BF16) static_cast<uint16_t*>(p)[r] = f32_to_bf16(v);
  else if constexpr (PD == TT_F16) static_cast<uint16_t*>(p)[r] = f32_to_f16(v);
}

// sigmoid(g) and silu(g) = g / (1 + exp(-g)).
template <class TT>
__device__ __forceinline__ void sig_silu(float g, float& sig, float& silu) {
  if constexpr (Traits<TT>::code == TT_F32) {
    const float den = 1.0f + expf(-g);
    sig = 1.0f / den;
    silu = g / den;
  } else {
    sig = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
    silu = g * sig;
  }
}

constexpr int promote(int a, int b) { return (b == NO_PROBS || a == b) ? a : TT_F32; }

// A row of nv vectors is split into nseg segments of seg vectors (the last
// shorter), each taken by L lanes: long rows then spread over several waves
// instead of one wave walking the whole row.
// SEG: the split launch (nseg > 1); whole rows otherwise.
template <class TT, int PD, int V, bool SEG>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const typename TT::storage* __restrict__ x,
                                                         int64_t rows, int64_t F,
                                                         const void* __restrict__ probs, int L,
                                                         int nseg, int64_t seg,
                                                         typename TT::storage* __restrict__ out) {
  typedef typename TT::storage St;
  constexpr int XD = Traits<TT>::code, PR = promote(XD, PD);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t vr = ((int64_t)blockIdx.x * 4 + wave) * (64 / L) + lane / L;
  const int64_t nv = F / V;
  int64_t r = vr, v0 = 0, v1 = nv;
  if constexpr (SEG) {
    if (vr >= rows * nseg) return;
    r = (int64_t)((uint64_t)vr / (uint32_t)nseg);
    v0 = (vr - r * nseg) * seg;
    v1 = v0 + seg < nv ? v0 + seg : nv;
  } else {
    if (vr >= rows) return;
  }
  const float p = load_prob<PD>(probs, r);
  const St* xr = x + r * 2 * F;
  St* orow = out + r * F;
  for (int64_t v = v0 + (lane & (L - 1)); v < v1; v += L) {
    St g[V], u[V], o[V];
    // Streaming loads (each input element is read once); the output keeps
    // plain stores, which measured faster here than streaming ones.
    load_stream<sizeof(g)>(g, xr + v * V);
    load_stream<sizeof(u)>(u, xr + F + v * V);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      float sig, si;
      sig_silu<TT>(TT::to_f32(g[k]), sig, si);
      float a = rnd<XD>(rnd<XD>(si) * TT::to_f32(u[k]));
      if constexpr (PD != NO_PROBS) a = rnd<PR>(a * p);
      o[k] = TT::from_f32(a);
    }
    __builtin_memcpy(orow + v * V, o, sizeof(o));
  }
}

// SEG: one block per row, wave w taking vectors [w seg, (w + 1) seg) with all
// 64 lanes (L = 64), the four waves' probability-gradient partials summed
// in wave order; whole rows per lane group otherwise.
template <class TT, int PD, int V, bool GP, bool SEG>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(
    const typename TT::storage* __restrict__ x, int64_t rows, int64_t F,
    const void* __restrict__ probs, int L, int64_t seg,
    const typename TT::storage* __restrict__ gout, typename TT::storage* __restrict__ gx,
    void* __restrict__ gprobs) {
  typedef typename TT::storage St;
  constexpr int XD = Traits<TT>::code, PR = promote(XD, PD);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = SEG ? (int64_t)blockIdx.x : ((int64_t)blockIdx.x * 4 + wave) * (64 / L) + lane / L;
  const bool live = r < rows;  // idle lanes still join the row reduction
  const float p = live ? load_prob<PD>(probs, r) : 0.f;
  float dp = 0.f;
  const int64_t nv = live ? F / V : 0;
  const St* xr = x + r * 2 * F;
  const St* gr = gout + r * F;
  St* dxr = gx + r * 2 * F;
  const int64_t v0 = SEG ? wave * seg : 0;
  const int64_t v1 = SEG ? (v0 + seg < nv ? v0 + seg : nv) : nv;
  for (int64_t v = v0 + (lane & (L - 1)); v < v1; v += L) {
    St g[V], u[V], d[V], og[V], ou[V];
    // Streaming loads and stores: every element is touched once.
    load_stream<sizeof(g)>(g, xr + v * V);
    load_stream<sizeof(u)>(u, xr + F + v * V);
    load_stream<sizeof(d)>(d, gr + v * V);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float gf = TT::to_f32(g[k]);
      const float uf = TT::to_f32(u[k]);
      float sig, si;
      sig_silu<TT>(gf, sig, si);
      const float s = rnd<XD>(si);
      float da;
      if constexpr (PD != NO_PROBS) {
        const float gd = TT::to_f32(d[k]);
        if constexpr (GP) dp += rnd<PR>(gd * rnd<XD>(s * uf));
        da = rnd<XD>(gd * p);
      } else {
        da = TT::to_f32(d[k]);
      }
      const float ds = rnd<XD>(da * uf);
      ou[k] = TT::from_f32(da * s);
      og[k] = TT::from_f32(ds * (sig * (1.0f + gf * (1.0f - sig))));
    }
    store_stream<sizeof(og)>(dxr + v * V, og);
    store_stream<sizeof(ou)>(dxr + F + v * V, ou);
  }
  if constexpr (GP) {
    for (int off = L / 2; off > 0; off >>= 1) dp += __shfl_xor(dp, off, TT_WAVE);
    if constexpr (SEG) {
      __shared__ float part[4];
      if (lane == 0) part[wave] = dp;
      __syncthreads();
      if (threadIdx.x == 0 && live)
        store_prob<PD>(gprobs, r, ((part[0] + part[1]) + part[2]) + part[3]);
    } else {
      if (live && (lane & (L - 1)) == 0) store_prob<PD>(gprobs, r, dp);
    }
  }
}

// ---------------------------------------------------------------------------
// Gated activation with a cap (the reference's gated_activation op,
// src/torchturbo/ops/providers/native/gated_activation.py:15-44) and the
// probability weighting. act is SiLU or GELU (erf form); mode 0: no cap,
//   a = round(round(act(gate)) * up)                      (16-bit rounding points)
// mode 1 (cap before): a = round(act(min(gate, L)) * clamp(up, -L, L))   (fp32)
// mode 2 (cap after):  a = round(min(act(gate), L) * clamp(up, -L, L))   (fp32)
// then out = round(a * p) as in swiglu. Caps keep NaN (x > L ? L : x), and
// their backward passes the gradient where the input lies inside the
// (inclusive) bounds, as torch.clamp's does.
// ---------------------------------------------------------------------------
enum { ACT_SILU = 0, ACT_GELU = 1 };

// act(g) and its derivative.
template <class TT>
__device__ __forceinline__ void act_eval(int act, float g, float& val, float& der) {
  if (act == ACT_SILU) {
    float sig, si;
    sig_silu<TT>(g, sig, si);
    val = si;
    der = sig * (1.0f + g * (1.0f - sig));
  } else {
    const float cdf = 0.5f * (1.0f + erff(g * 0.70710678118654752f));
    const float pdf = expf(-0.5f * g * g) * 0.39894228040143268f;
    val = g * cdf;
    der = cdf + g * pdf;
  }
}

__device__ __forceinline__ float cap_hi(float x, float lim) { return x > lim ? lim : x; }
__device__ __forceinline__ float cap_both(float x, float lim) {
  return x < -lim ? -lim : (x > lim ? lim : x);
}

template <class TT, int PD, int V>
__global__ __launch_bounds__(256) void gated_fwd_kernel(const typename TT::storage* __restrict__ x,
                                                        int64_t rows, int64_t F,
                                                        const void* __restrict__ probs, int L,
                                                        int act, int mode, float lim,
                                                        typename TT::storage* __restrict__ out) {
  typedef typename TT::storage St;
  constexpr int XD = Traits<TT>::code, PR = promote(XD, PD);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = ((int64_t)blockIdx.x * 4 + wave) * (64 / L) + lane / L;
  if (r >= rows) return;
  const float p = load_prob<PD>(probs, r);
  const St* xr = x + r * 2 * F;
  St* orow = out + r * F;
  const int64_t nv = F / V;
  for (int64_t v = lane & (L - 1); v < nv; v += L) {
    St g[V], u[V], o[V];
    load_stream<sizeof(g)>(g, xr + v * V);
    load_stream<sizeof(u)>(u, xr + F + v * V);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float gf = TT::to_f32(g[k]), uf = TT::to_f32(u[k]);
      float av, der, a;
      if (mode == 0) {
        act_eval<TT>(act, gf, av, der);
        a = rnd<XD>(rnd<XD>(av) * uf);
      } else {
        act_eval<TT>(act, mode == 1 ? cap_hi(gf, lim) : gf, av, der);
        if (mode == 2) av = cap_hi(av, lim);
        a = rnd<XD>(av * cap_both(uf, lim));
      }
      if constexpr (PD != NO_PROBS) a = rnd<PR>(a * p);
      o[k] = TT::from_f32(a);
    }
    __builtin_memcpy(orow + v * V, o, sizeof(o));
  }
}

template <class TT, int PD, int V, bool GP>
__global__ __launch_bounds__(256) void gated_bwd_kernel(
    const typename TT::storage* __restrict__ x, int64_t rows, int64_t F,
    const void* __restrict__ probs, int L, int act, int mode, float lim,
    const typename TT::storage* __restrict__ gout, typename TT::storage* __restrict__ gx,
    void* __restrict__ gprobs) {
  typedef typename TT::storage St;
  constexpr int XD = Traits<TT>::code, PR = promote(XD, PD);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = ((int64_t)blockIdx.x * 4 + wave) * (64 / L) + lane / L;
  const bool live = r < rows;  // idle lanes still join the row reduction
  const float p = live ? load_prob<PD>(probs, r) : 0.f;
  float dp = 0.f;
  const int64_t nv = live ? F / V : 0;
  const St* xr = x + r * 2 * F;
  const St* gr = gout + r * F;
  St* dxr = gx + r * 2 * F;
  for (int64_t v = lane & (L - 1); v < nv; v += L) {
    St g[V], u[V], d[V], og[V], ou[V];
    load_stream<sizeof(g)>(g, xr + v * V);
    load_stream<sizeof(u)>(u, xr + F + v * V);
    load_stream<sizeof(d)>(d, gr + v * V);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float gf = TT::to_f32(g[k]), uf = TT::to_f32(u[k]);
      const float gd = TT::to_f32(d[k]);
      const float da = PD != NO_PROBS ? rnd<XD>(gd * p) : gd;
      float av, der, a, dg, du;
      if (mode == 0) {
        act_eval<TT>(act, gf, av, der);
        const float sv = rnd<XD>(av);
        a = rnd<XD>(sv * uf);
        du = da * sv;
        dg = rnd<XD>(da * uf) * der;
      } else {
        const float uc = cap_both(uf, lim);
        const bool u_in = uf >= -lim && uf <= lim;
        if (mode == 1) {
          act_eval<TT>(act, cap_hi(gf, lim), av, der);
          dg = gf <= lim ? da * uc * der : 0.f;
        } else {
          act_eval<TT>(act, gf, av, der);
          const bool a_in = av <= lim;
          av = cap_hi(av, lim);
          dg = a_in ? da * uc * der : 0.f;
        }
        a = rnd<XD>(av * uc);
        du = u_in ? da * av : 0.f;
      }
      if constexpr (PD != NO_PROBS && GP) dp += rnd<PR>(gd * a);
      og[k] = TT::from_f32(dg);
      ou[k] = TT::from_f32(du);
    }
    store_stream<sizeof(og)>(dxr + v * V, og);
    store_stream<sizeof(ou)>(dxr + F + v * V, ou);
  }
  if constexpr (GP) {
    for (int off = L / 2; off > 0; off >>= 1) dp += __shfl_xor(dp, off, TT_WAVE);
    if (live && (lane & (L - 1)) == 0) store_prob<PD>(gprobs, r, dp);
  }
}

bool float_dtype(int d) { return d == TT_F32 || d == TT_BF16 || d == TT_F16; }

// Lanes per row: the largest power of two <= 64 that leaves at most an
// eighth of its lane slots idle over the row's vectors; failing that, the
// one that wastes the fewest (larger on ties), at least 8 once the row has
// 8 vectors. Fewer lanes per row put more rows, each its own stream of
// DRAM pages, under one load, and one lane per row (the fewest-waste choice
// for an odd vector count) spreads every load over 64 rows and runs about
// 30x slower.
int lanes_per_row(int64_t nv) {
  const int lmin = nv >= 8 ? 8 : 1;
  for (int L = 64; L >= lmin; L >>= 1)
    if ((((nv + L - 1) / L) * L - nv) * 8 <= nv) return L;
  int best = 1;
  int64_t best_waste = -1;
  for (int L = 64; L >= lmin; L >>= 1) {
    const int64_t waste = ((nv + L - 1) / L) * L - nv;
    if (best_waste < 0 || waste < best_waste) {
      best = L;
      best_waste = waste;
    }
  }
  return best;
}

template <class TT, int PD>
int launch_fwd_p(const void* x, int64_t rows, int64_t F, const void* probs, void* out,
                 hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       static_cast<uintptr_t>(F * sizeof(St));
  const St* xp = static_cast<const St*>(x);
  St* op = static_cast<St*>(out);
  // Rows of more than 256 vectors go out in segments of a multiple of 64
  // vectors, at most 256 (four loads per lane).
  auto split = [](int64_t nv, int& nseg, int64_t& seg) {
    nseg = nv > 256 ? (int)((nv + 255) / 256) : 1;
    seg = nseg > 1 ? (((nv + nseg - 1) / nseg + 63) / 64) * 64 : nv;
  };
  int nseg;
  int64_t seg;
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    split(F / V, nseg, seg);
    const int L = lanes_per_row(seg);
    const dim3 grid((unsigned)((rows * nseg + 4 * (64 / L) - 1) / (4 * (64 / L))));
    if (nseg > 1)
      hipLaunchKernelGGL((swiglu_fwd_kernel<TT, PD, V, true>), grid, dim3(256), 0, s, xp, rows,
                         F, probs, L, nseg, seg, op);
    else
      hipLaunchKernelGGL((swiglu_fwd_kernel<TT, PD, V, false>), grid, dim3(256), 0, s, xp, rows,
                         F, probs, L, nseg, seg, op);
  } else {
    split(F, nseg, seg);
    const int L = lanes_per_row(seg);
    const dim3 grid((unsigned)((rows * nseg + 4 * (64 / L) - 1) / (4 * (64 / L))));
    if (nseg > 1)
      hipLaunchKernelGGL((swiglu_fwd_kernel<TT, PD, 1, true>), grid, dim3(256), 0, s, xp, rows,
                         F, probs, L, nseg, seg, op);
    else
      hipLaunchKernelGGL((swiglu_fwd_kernel<TT, PD, 1, false>), grid, dim3(256), 0, s, xp, rows,
                         F, probs, L, nseg, seg, op);
  }
  return tt_check_launch("swiglu_fwd");
}

template <class TT, int PD, bool GP>
int launch_bwd_p(const void* x, int64_t rows, int64_t F, const void* probs, const void* gout,
                 void* gx, void* gprobs, hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gout) |
                       reinterpret_cast<uintptr_t>(gx) | static_cast<uintptr_t>(F * sizeof(St));
  const St* xp = static_cast<const St*>(x);
  const St* gp = static_cast<const St*>(gout);
  St* dxp = static_cast<St*>(gx);
  // Rows of more than 256 vectors: one block per row, four segments of a
  // multiple of 64 vectors.
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    const int64_t nv = F / V;
    if (nv > 256) {
      const int64_t seg = (((nv + 3) / 4 + 63) / 64) * 64;
      hipLaunchKernelGGL((swiglu_bwd_kernel<TT, PD, V, GP, true>), dim3((unsigned)rows),
                         dim3(256), 0, s, xp, rows, F, probs, 64, seg, gp, dxp, gprobs);
    } else {
      const int L = lanes_per_row(nv);
      const int64_t rpb = 4 * (64 / L);
      hipLaunchKernelGGL((swiglu_bwd_kernel<TT, PD, V, GP, false>),
                         dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, s, xp, rows, F,
                         probs, L, nv, gp, dxp, gprobs);
    }
  } else {
    const int L = lanes_per_row(F);
    const int64_t rpb = 4 * (64 / L);
    hipLaunchKernelGGL((swiglu_bwd_kernel<TT, PD, 1, GP, false>),
                       dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, s, xp, rows, F,
                       probs, L, F, gp, dxp, gprobs);
  }
  return tt_check_launch("swiglu_bwd");
}

template <class TT>
int launch_fwd(const void* x, int64_t rows, int64_t F, const void* probs, int pdt, void* out,
               hipStream_t s) {
  if (probs == nullptr) return launch_fwd_p<TT, NO_PROBS>(x, rows, F, probs, out, s);
  switch (pdt) {
    case TT_F32: return launch_fwd_p<TT, TT_F32>(x, rows, F, probs, out, s);
    case TT_BF16: return launch_fwd_p<TT, TT_BF16>(x, rows, F, probs, out, s);
    default: return launch_fwd_p<TT, TT_F16>(x, rows, F, probs, out, s);
  }
}

template <class TT, int PD>
int launch_bwd_g(const void* x, int64_t rows, int64_t F, const void* probs, const void* gout,
                 void* gx, void* gprobs, hipStream_t s) {
  if (gprobs != nullptr) return launch_bwd_p<TT, PD, true>(x, rows, F, probs, gout, gx, gprobs, s);
  return launch_bwd_p<TT, PD, false>(x, rows, F, probs, gout, gx, gprobs, s);
}

template <class TT>
int launch_bwd(const void* x, int64_t rows, int64_t F, const void* probs, int pdt,
               const void* gout, void* gx, void* gprobs, hipStream_t s) {
  if (probs == nullptr)
    return launch_bwd_p<TT, NO_PROBS, false>(x, rows, F, probs, gout, gx, gprobs, s);
  switch (pdt) {
    case TT_F32: return launch_bwd_g<TT, TT_F32>(x, rows, F, probs, gout, gx, gprobs, s);
    case TT_BF16: return launch_bwd_g<TT, TT_BF16>(x, rows, F, probs, gout, gx, gprobs, s);
    default: return launch_bwd_g<TT, TT_F16>(x, rows, F, probs, gout, gx, gprobs, s);
  }
}

struct GatedArgs {
  int act, mode;
  float lim;
};

template <class TT, int PD>
int launch_gated_fwd_p(const void* x, int64_t rows, int64_t F, const void* probs, GatedArgs ga,
                       void* out, hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       static_cast<uintptr_t>(F * sizeof(St));
  const St* xp = static_cast<const St*>(x);
  St* op = static_cast<St*>(out);
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    const int L = lanes_per_row(F / V);
    const int64_t rpb = 4 * (64 / L);
    hipLaunchKernelGGL((gated_fwd_kernel<TT, PD, V>), dim3((unsigned)((rows + rpb - 1) / rpb)),
                       dim3(256), 0, s, xp, rows, F, probs, L, ga.act, ga.mode, ga.lim, op);
  } else {
    const int L = lanes_per_row(F);
    const int64_t rpb = 4 * (64 / L);
    hipLaunchKernelGGL((gated_fwd_kernel<TT, PD, 1>), dim3((unsigned)((rows + rpb - 1) / rpb)),
                       dim3(256), 0, s, xp, rows, F, probs, L, ga.act, ga.mode, ga.lim, op);
  }
  return tt_check_launch("gated_activation_fwd");
}

template <class TT, int PD, bool GP>
int launch_gated_bwd_p(const void* x, int64_t rows, int64_t F, const void* probs, GatedArgs ga,
                       const void* gout, void* gx, void* gprobs, hipStream_t s) {
  typedef typename TT::storage St;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gout) |
                       reinterpret_cast<uintptr_t>(gx) | static_cast<uintptr_t>(F * sizeof(St));
  const St* xp = static_cast<const St*>(x);
  const St* gp = static_cast<const St*>(gout);
  St* dxp = static_cast<St*>(gx);
  if (al % 16 == 0) {
    constexpr int V = 16 / sizeof(St);
    const int L = lanes_per_row(F / V);
    const int64_t rpb = 4 * (64 / L);
    hipLaunchKernelGGL((gated_bwd_kernel<TT, PD, V, GP>),
                       dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, s, xp, rows, F,
                       probs, L, ga.act, ga.mode, ga.lim, gp, dxp, gprobs);
  } else {
    const int L = lanes_per_row(F);
    const int64_t rpb = 4 * (64 / L);
    hipLaunchKernelGGL((gated_bwd_kernel<TT, PD, 1, GP>),
                       dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, s, xp, rows, F,
                       probs, L, ga.act, ga.mode, ga.lim, gp, dxp, gprobs);
  }
  return tt_check_launch("gated_activation_bwd");
}

template <class TT>
int launch_gated_fwd(const void* x, int64_t rows, int64_t F, const void* probs, int pdt,
                     GatedArgs ga, void* out, hipStream_t s) {
  if (probs == nullptr) return launch_gated_fwd_p<TT, NO_PROBS>(x, rows, F, probs, ga, out, s);
  switch (pdt) {
    case TT_F32: return launch_gated_fwd_p<TT, TT_F32>(x, rows, F, probs, ga, out, s);
    case TT_BF16: return launch_gated_fwd_p<TT, TT_BF16>(x, rows, F, probs, ga, out, s);
    default: return launch_gated_fwd_p<TT, TT_F16>(x, rows, F, probs, ga, out, s);
  }
}

template <class TT, int PD>
int launch_gated_bwd_g(const void* x, int64_t rows, int64_t F, const void* probs, GatedArgs ga,
                       const void* gout, void* gx, void* gprobs, hipStream_t s) {
  if (gprobs != nullptr)
    return launch_gated_bwd_p<TT, PD, true>(x, rows, F, probs, ga, gout, gx, gprobs, s);
  return launch_gated_bwd_p<TT, PD, false>(x, rows, F, probs, ga, gout, gx, gprobs, s);
}

template <class TT>
int launch_gated_bwd(const void* x, int64_t rows, int64_t F, const void* probs, int pdt,
                     GatedArgs ga, const void* gout, void* gx, void* gprobs, hipStream_t s) {
  if (probs == nullptr)
    return launch_gated_bwd_p<TT, NO_PROBS, false>(x, rows, F, probs, ga, gout, gx, gprobs, s);
  switch (pdt) {
    case TT_F32: return launch_gated_bwd_g<TT, TT_F32>(x, rows, F, probs, ga, gout, gx, gprobs, s);
    case TT_BF16: return launch_gated_bwd_g<TT, TT_BF16>(x, rows, F, probs, ga, gout, gx, gprobs, s);
    default: return launch_gated_bwd_g<TT, TT_F16>(x, rows, F, probs, ga, gout, gx, gprobs, s);
  }
}

int gated_checks(int dtype, int64_t rows, int64_t ffn, int act, float limit, const void* probs,
                 int probs_dtype) {
  TT_REQUIRE(float_dtype(dtype), "gated_activation: unsupported dtype %d", dtype);
  TT_REQUIRE(rows >= 0 && ffn >= 0, "gated_activation: negative sizes");
  TT_REQUIRE(act == ACT_SILU || act == ACT_GELU,
             "gated_activation only supports F.silu and F.gelu (act code %d)", act);
  TT_REQUIRE(limit >= 0.0f, "limit must be non-negative.");
  if (probs != nullptr)
    TT_REQUIRE(float_dtype(probs_dtype), "gated_activation: unsupported probs dtype");
  return TT_OK;
}

}  // namespace

extern "C" int tt_swiglu_fwd(const void* x, int dtype, int64_t rows, int64_t ffn,
                             const void* probs, int probs_dtype, void* out, void* stream) {
  TT_REQUIRE(float_dtype(dtype), "swiglu: unsupported dtype %d", dtype);
  TT_REQUIRE(rows >= 0 && ffn >= 0, "swiglu: negative sizes");
  if (probs != nullptr) TT_REQUIRE(float_dtype(probs_dtype), "swiglu: unsupported probs dtype");
  if (rows == 0 || ffn == 0) return TT_OK;
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_fwd<BF16T>(x, rows, ffn, probs, probs_dtype, out, s);
    case TT_F16: return launch_fwd<F16T>(x, rows, ffn, probs, probs_dtype, out, s);
    default: return launch_fwd<F32T>(x, rows, ffn, probs, probs_dtype, out, s);
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
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_bwd<BF16T>(x, rows, ffn, probs, probs_dtype, grad_out, grad_x, grad_probs, s);
    case TT_F16: return launch_bwd<F16T>(x, rows, ffn, probs, probs_dtype, grad_out, grad_x, grad_probs, s);
    default: return launch_bwd<F32T>(x, rows, ffn, probs, probs_dtype, grad_out, grad_x, grad_probs, s);
  }
}

extern "C" int tt_gated_act_fwd(const void* x, int dtype, int64_t rows, int64_t ffn, int act,
                                float limit, int clamp_after, const void* probs,
                                int probs_dtype, void* out, void* stream) {
  const int rc = gated_checks(dtype, rows, ffn, act, limit, probs, probs_dtype);
  if (rc != TT_OK) return rc;
  if (rows == 0 || ffn == 0) return TT_OK;
  const GatedArgs ga{act, limit == 0.0f ? 0 : (clamp_after ? 2 : 1), limit};
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_gated_fwd<BF16T>(x, rows, ffn, probs, probs_dtype, ga, out, s);
    case TT_F16: return launch_gated_fwd<F16T>(x, rows, ffn, probs, probs_dtype, ga, out, s);
    default: return launch_gated_fwd<F32T>(x, rows, ffn, probs, probs_dtype, ga, out, s);
  }
}

extern "C" int tt_gated_act_bwd(const void* x, int dtype, int64_t rows, int64_t ffn, int act,
                                float limit, int clamp_after, const void* probs,
                                int probs_dtype, const void* grad_out, void* grad_x,
                                void* grad_probs, void* stream) {
  const int rc = gated_checks(dtype, rows, ffn, act, limit, probs, probs_dtype);
  if (rc != TT_OK) return rc;
  if (grad_probs != nullptr)
    TT_REQUIRE(probs != nullptr, "gated_activation_bwd: grad_probs needs probs");
  if (rows == 0) return TT_OK;
  const GatedArgs ga{act, limit == 0.0f ? 0 : (clamp_after ? 2 : 1), limit};
  hipStream_t s = S(stream);
  switch (dtype) {
    case TT_BF16: return launch_gated_bwd<BF16T>(x, rows, ffn, probs, probs_dtype, ga, grad_out, grad_x, grad_probs, s);
    case TT_F16: return launch_gated_bwd<F16T>(x, rows, ffn, probs, probs_dtype, ga, grad_out, grad_x, grad_probs, s);
    default: return launch_gated_bwd<F32T>(x, rows, ffn, probs, probs_dtype, ga, grad_out, grad_x, grad_probs, s);
  }
}
