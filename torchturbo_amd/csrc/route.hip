// Router top-k (fwd/bwd) and the deterministic routing index (counting sort).
//
// Router: one wave64 per token. Lane l owns the EPL consecutive experts
// [l*EPL, (l+1)*EPL); top-k is k rounds of a wave arg-max (larger score
// first, lower expert id on equal scores): a register (DPP) maximum of the
// lanes' best remaining keys and a ballot for the lowest lane holding it.
// Group-limited selection uses segmented shuffles over the lanes of a group.
//
// Routing index: packed rows are ordered by expert, then token. Three kernels:
//   hist  : per 256-token block, per-expert counts  -> bc[E][nb]
//   scan  : per expert, exclusive scan over blocks   -> bc (in place), totals
//   rank  : per block, expert base + wave prefix + in-wave ballot rank
// The in-wave rank of a lane for expert e is popcount(ballot(lane has e) &
// lanes below it), so the order is the token order and is reproducible.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"

namespace {

constexpr int kRouterWaves = 4;  // tokens per 256-thread block

// KT: the type selection keys are compared in: fp32, or fp64 for fp64
// logits (whose plain-softmax top-k compares the fp64 logits themselves).
template <typename KT>
struct Cand {
  KT sel;      // selection key (score, or score + bias)
  int idx;     // expert id
  float sc;    // score the probability is computed from
  float lg;    // logit (fp32)
};

template <typename KT>
__device__ __forceinline__ bool better(KT v, int i, KT bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Wave-wide arg-max (segment of `width` lanes when width < 64).
template <typename KT>
__device__ __forceinline__ Cand<KT> cand_reduce(Cand<KT> c, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) {
    Cand<KT> o;
    o.sel = __shfl_xor(c.sel, off, TT_WAVE);
    o.idx = __shfl_xor(c.idx, off, TT_WAVE);
    o.sc = __shfl_xor(c.sc, off, TT_WAVE);
    o.lg = __shfl_xor(c.lg, off, TT_WAVE);
    if (better(o.sel, o.idx, c.sel, c.idx)) c = o;
  }
  return c;
}

// Wave-wide maximum in registers (DPP): butterflies within quads, half rows
// and rows, then the row broadcasts carry the running maximum into lane 63,
// which is read back as a uniform value. Exact (max), NaN-free inputs.
#define TT_DPP_FMAX(v, ctrl, rmask)                                                          \
  fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), \
                                                       ctrl, rmask, 0xf, false)))
__device__ __forceinline__ float wave_max_uniform(float v) {
  v = TT_DPP_FMAX(v, 0xb1, 0xf);   // quad_perm [1, 0, 3, 2]
  v = TT_DPP_FMAX(v, 0x4e, 0xf);   // quad_perm [2, 3, 0, 1]
  v = TT_DPP_FMAX(v, 0x141, 0xf);  // row_half_mirror
  v = TT_DPP_FMAX(v, 0x140, 0xf);  // row_mirror
  v = TT_DPP_FMAX(v, 0x142, 0xa);  // row_bcast15 into rows 1 and 3
  v = TT_DPP_FMAX(v, 0x143, 0xc);  // row_bcast31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// The same for fp64 keys: a butterfly of shuffles, then lane 0's value.
__device__ __forceinline__ double wave_max_uniform(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmax(v, __shfl_xor(v, off, TT_WAVE));
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readfirstlane((int)b);
  const int hi = __builtin_amdgcn_readfirstlane((int)(b >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float softplus_f(float x) {
  // PyTorch softplus with beta = 1, threshold = 20.
  return x > 20.0f ? x : log1pf(expf(x));
}

// Top-k routing of token t by one wave from its logits (fp32 values of the
// logits dtype ldt; lane l holds experts l*EPL .. l*EPL + EPL - 1, -inf past
// E): scores, selection, probabilities, and the outputs of row t.
// kl: the logits as selection keys (the fp64 logits for KT = double, lg
// otherwise).
template <int EPL, typename KT = float>
__device__ __forceinline__ void route_row(
    int lane, int64_t t, const float (&lg)[EPL], const KT (&kl)[EPL], const bool (&valid)[EPL],
    int ldt, int E, int K, int score_fn, int pre_softmax, const float* __restrict__ bias, int G,
    int GK, float scaling, const int64_t* __restrict__ fixed, void* __restrict__ probs,
    uint8_t* __restrict__ rmap, int64_t* __restrict__ top_idx) {
  const float NEG = -INFINITY;
  const KT KNEG = -INFINITY;
  float sc[EPL];
  KT sel[EPL];

  // Scores.
  if (score_fn == TT_SCORE_SOFTMAX) {
    if (pre_softmax) {
      float mx = NEG;
#pragma unroll
      for (int i = 0; i < EPL; ++i) mx = fmaxf(mx, lg[i]);
      mx = wave_max(mx);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        sc[i] = valid[i] ? expf(lg[i] - mx) : 0.f;
        s += sc[i];
      }
      s = wave_sum(s);
#pragma unroll
      for (int i = 0; i < EPL; ++i) sc[i] = sc[i] / s;
    } else {
#pragma unroll
      for (int i = 0; i < EPL; ++i) sc[i] = lg[i];
    }
  } else if (score_fn == TT_SCORE_SIGMOID) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) sc[i] = valid[i] ? sigmoid_f(lg[i]) : 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < EPL; ++i) sc[i] = valid[i] ? sqrtf(softplus_f(lg[i])) : 0.f;
  }
  const bool raw = score_fn == TT_SCORE_SOFTMAX && !pre_softmax;  // keys: the logits
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane * EPL + i;
    float v = sc[i];
    if (bias != nullptr && valid[i] && !raw) v = v + bias[e];  // fp32 sum
    sel[i] = valid[i] ? (raw ? kl[i] : (KT)v) : KNEG;
  }

  bool taken[EPL];
  int slot[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    taken[i] = false;
    slot[i] = 0;
  }
  Cand<KT> mine;  // lane j < K holds the j-th selected expert
  mine.sel = KNEG;
  mine.idx = 0;
  mine.sc = 0.f;
  mine.lg = 0.f;

  if (fixed != nullptr) {
    // Token-id hash routing: ids are given; fetch their scores from owners.
    int want = lane < K ? (int)fixed[t * K + lane] : -1;
    if (want >= E) want = -1;
    const int owner = want >= 0 ? want / EPL : 0;
    const int part = want >= 0 ? want % EPL : 0;
    float wsc = 0.f, wlg = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const float a = __shfl(sc[i], owner, TT_WAVE);
      const float b = __shfl(lg[i], owner, TT_WAVE);
      if (i == part) {
        wsc = a;
        wlg = b;
      }
    }
    if (lane < K) {
      mine.idx = want < 0 ? 0 : want;
      mine.sc = wsc;
      mine.lg = wlg;
      mine.sel = 0.f;
    }
    for (int j = 0; j < K; ++j) {
      const int id = __shfl(want, j, TT_WAVE);
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (id == lane * EPL + i) {
          taken[i] = true;
          slot[i] = j;
        }
    }
  } else {
    if (GK > 0) {
      // Group-limited: group score = sum of the top (K / GK) scores of the
      // group; keep the GK best groups; mask the rest.
      const int gs = E / G;        // experts per group
      const int width = gs / EPL;  // lanes per group (power of two, checked)
      const int m = K / GK;
      bool used[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) used[i] = false;
      KT gscore = 0;
      for (int r = 0; r < m; ++r) {
        Cand<KT> c;
        c.sel = KNEG;
        c.idx = 0x7fffffff;
        c.sc = 0.f;
        c.lg = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (!used[i] && better(sel[i], lane * EPL + i, c.sel, c.idx)) {
            c.sel = sel[i];
            c.idx = lane * EPL + i;
          }
        c = cand_reduce(c, width);
        gscore = gscore + c.sel;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (c.idx == lane * EPL + i) used[i] = true;
      }
      const int group = (lane * EPL) / gs;
      const bool lane_live = lane * EPL < E;
      bool keep = false;
      KT gkey = lane_live ? gscore : KNEG;
      for (int r = 0; r < GK; ++r) {
        Cand<KT> c;
        c.sel = keep ? KNEG : gkey;
        c.idx = lane_live ? group : 0x7fffffff;
        c.sc = 0.f;
        c.lg = 0.f;
        c = cand_reduce(c, TT_WAVE);
        if (c.idx == group) keep = true;
      }
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (!keep) sel[i] = KNEG;
    }
    // k rounds of a wave arg-max. Each lane keeps its head: its best
    // remaining expert (largest key, lowest id on equal keys). A round takes
    // the wave maximum of the heads, the lowest lane holding it (ballot) and
    // that lane's head — larger key first, lower expert id on equal keys, as
    // a comparison of (key, id) pairs would. Only the winning lane advances.
    KT hv = KNEG;
    float hsc = 0.f, hlg = 0.f;
    int hi = -1;
    auto head = [&]() {
      hv = KNEG;
      hi = -1;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (valid[i] && !taken[i] && (hi < 0 || sel[i] > hv)) {
          hv = sel[i];
          hi = i;
        }
      hsc = 0.f;
      hlg = 0.f;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (i == hi) {
          hsc = sc[i];
          hlg = lg[i];
        }
    };
    head();
    for (int j = 0; j < K; ++j) {
      const KT m = wave_max_uniform(hi >= 0 ? hv : KNEG);
      const uint64_t owners = __ballot(hi >= 0 && hv == m);
      // K <= E valid experts, so some lane still has a head (owners is empty
      // only for NaN keys: lane 0 then reports its head, or -1).
      const int w = __builtin_amdgcn_readfirstlane(owners ? (int)__builtin_ctzll(owners) : 0);
      const int wi = __builtin_amdgcn_readlane(hi, w);
      const float wsc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hsc), w));
      const float wlg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hlg), w));
      if (lane == j) {
        mine.sel = m;
        mine.idx = w * EPL + wi;
        mine.sc = wsc;
        mine.lg = wlg;
      }
      if (lane == w) {
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (i == hi) {
            taken[i] = true;
            slot[i] = j;
          }
        head();
      }
    }
  }

  // Probabilities of the K selected experts (lanes 0..K-1), in fp32.
  const bool active = lane < K;
  float p;
  if (score_fn == TT_SCORE_SOFTMAX && !pre_softmax) {
    const float mx = wave_max_uniform(active ? mine.lg : NEG);
    const float ex = active ? expf(mine.lg - mx) : 0.f;
    const float s = wave_sum(ex);
    p = ex / s;
  } else if (score_fn == TT_SCORE_SOFTMAX) {
    p = mine.sc;
  } else {
    const float s = wave_sum(active ? mine.sc : 0.f);
    p = K > 1 ? mine.sc / (s + 1e-20f) : mine.sc;
  }
  if (scaling != 0.f) p = p * scaling;
  p = round_to(p, ldt);

  if (active) top_idx[t * K + lane] = mine.idx;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const float v = __shfl(p, slot[i], TT_WAVE);
    if (valid[i]) {
      const int64_t o = t * E + lane * EPL + i;
      store_from_f32(probs, ldt, o, taken[i] ? v : 0.f);
      rmap[o] = taken[i] ? 1 : 0;
    }
  }
}

template <int EPL, typename KT>
__global__ __launch_bounds__(256) void router_fwd_kernel(
    const void* __restrict__ logits, int ldt, int64_t T, int E, int K, int score_fn,
    int pre_softmax, const float* __restrict__ bias, int G, int GK, float scaling,
    const int64_t* __restrict__ fixed, void* __restrict__ probs, uint8_t* __restrict__ rmap,
    int64_t* __restrict__ top_idx) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave; no block-level synchronisation below
  float lg[EPL];
  KT kl[EPL];
  bool valid[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane * EPL + i;
    valid[i] = e < E;
    if constexpr (std::is_same<KT, double>::value) {
      kl[i] = valid[i] ? static_cast<const double*>(logits)[t * E + e] : -INFINITY;
      lg[i] = (float)kl[i];
    } else {
      lg[i] = valid[i] ? load_as_f32(logits, ldt, t * E + e) : -INFINITY;
      kl[i] = lg[i];
    }
  }
  route_row<EPL, KT>(lane, t, lg, kl, valid, ldt, E, K, score_fn, pre_softmax, bias, G, GK,
                     scaling, fixed, probs, rmap, top_idx);
}

template <int EPL>
__global__ __launch_bounds__(256) void router_bwd_kernel(
    const void* __restrict__ logits, int ldt, int64_t T, int E, int K, int score_fn,
    int pre_softmax, float scaling, const int64_t* __restrict__ top_idx,
    const void* __restrict__ grad, void* __restrict__ grad_logits) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const float NEG = -INFINITY;
  const bool active = lane < K;
  int id = active ? (int)top_idx[t * K + lane] : 0;
  if (id < 0 || id >= E) id = 0;
  // d(probs) of the selected experts, as the fp32 gradient of the scaled probs.
  float d = active ? load_as_f32(grad, ldt, t * E + id) : 0.f;
  if (scaling != 0.f) d = d * scaling;
  const float lgj = active ? load_as_f32(logits, ldt, t * E + id) : 0.f;

  float out[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) out[i] = 0.f;

  if (score_fn == TT_SCORE_SOFTMAX && pre_softmax) {
    float lg[EPL], s[EPL], dv[EPL];
    float mx = NEG;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane * EPL + i;
      lg[i] = e < E ? load_as_f32(logits, ldt, t * E + e) : NEG;
      mx = fmaxf(mx, lg[i]);
      dv[i] = 0.f;
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      s[i] = (lane * EPL + i) < E ? expf(lg[i] - mx) : 0.f;
      sum += s[i];
    }
    sum = wave_sum(sum);
    for (int j = 0; j < K; ++j) {
      const int e = __shfl(id, j, TT_WAVE);
      const float g = __shfl(d, j, TT_WAVE);
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (e == lane * EPL + i) dv[i] = g;
    }
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      s[i] = s[i] / sum;
      dot += s[i] * dv[i];
    }
    dot = wave_sum(dot);
#pragma unroll
    for (int i = 0; i < EPL; ++i) out[i] = s[i] * (dv[i] - dot);
  } else {
    float g;  // gradient w.r.t. the selected logit
    if (score_fn == TT_SCORE_SOFTMAX) {
      const float mx = wave_max(active ? lgj : NEG);
      const float ex = active ? expf(lgj - mx) : 0.f;
      const float p = ex / wave_sum(ex);
      const float dot = wave_sum(active ? p * d : 0.f);
      g = p * (d - dot);
    } else {
      float s, dsdx;
      if (score_fn == TT_SCORE_SIGMOID) {
        s = sigmoid_f(lgj);
        dsdx = (1.0f - s) * s;
      } else {
        const float sp = softplus_f(lgj);
        s = sqrtf(sp);
        const float dsp = lgj > 20.0f ? 1.0f : sigmoid_f(lgj);
        dsdx = dsp / (2.0f * s);
      }
      float ds = d;
      if (K > 1) {
        const float den = wave_sum(active ? s : 0.f) + 1e-20f;
        const float dden = wave_sum(active ? -d * s / (den * den) : 0.f);
        ds = d / den + dden;
      }
      g = ds * dsdx;
    }
    for (int j = 0; j < K; ++j) {
      const int e = __shfl(id, j, TT_WAVE);
      const float gj = __shfl(g, j, TT_WAVE);
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (e == lane * EPL + i) out[i] = gj;
    }
  }
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane * EPL + i;
    if (e < E) store_from_f32(grad_logits, ldt, t * E + e, out[i]);
  }
}

// ---------------------------------------------------------------------------
// Router loss statistics: what the load-balancing (aux) loss and the z-loss
// need from the [T, E] logits, in one pass (models/modules/moe/moe_utils.py:
// 15-70, router.py:164-270).
//   prob_sum[e] = sum over valid tokens of the bias-free score s_t[e]
//                 (softmax in fp32; sigmoid or sqrt(softplus) divided by
//                 their sum + 1e-20);
//   counts[e]   = valid tokens whose top-k of s_t (larger first, lower id on
//                 equal scores) holds e;
//   z_sum       = sum over valid tokens of r(lse_t^2), r the rounding to
//                 the logits dtype, lse_t formed as torch.logsumexp forms it
//                 in that dtype (the reference's logsumexp and square run in
//                 the logits dtype).
// Each wave walks tokens wave, wave + W, ... of a grid whose size depends on
// T only; per-block partial rows are summed in block order by a one-block
// kernel, so the results are reproducible.
// ---------------------------------------------------------------------------
constexpr int kLossWaves = 4;
constexpr int kLossMaxBlocks = 512;
constexpr int kLossTokensPerWave = 2;  // at least; large batches hit the block cap

int loss_blocks(int64_t T) {
  const int64_t per = (int64_t)kLossWaves * kLossTokensPerWave;
  const int64_t nb = (T + per - 1) / per;
  return (int)(nb < 1 ? 1 : (nb > kLossMaxBlocks ? kLossMaxBlocks : nb));
}

// log-sum-exp of a token's logits as PyTorch forms it: fp32 logits
// max + log(sum exp(x - max)); bf16 / f16 logits run every step in that
// dtype (max, x - max, exp, sum, log, + max each rounded), which is what
// torch.logsumexp does for them. se is the fp32 sum of exp(x - mx). fp64
// logits take the fp32 form (the z-loss to fp32 precision, not fp64).
template <int EPL>
__device__ __forceinline__ float lse_like_torch(const float (&lg)[EPL], const bool (&valid)[EPL],
                                                float mx, float se, int ldt) {
  if (ldt == TT_F32 || ldt == TT_F64) return mx + logf(se);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    if (valid[i]) s += round_to(expf(round_to(lg[i] - mx, ldt)), ldt);
  s = round_to(wave_sum(s), ldt);
  return round_to(round_to(logf(s), ldt) + mx, ldt);
}

template <int EPL>
__global__ __launch_bounds__(256) void router_loss_fwd_kernel(
    const void* __restrict__ logits, int ldt, int64_t T, int E, int K, int score_fn,
    const uint8_t* __restrict__ pad, int want_aux, int want_z, float* __restrict__ part_p,
    int* __restrict__ part_c, float* __restrict__ part_z) {
  extern __shared__ __align__(16) float lsm[];  // [4][E] prob sums, [4][E] counts, [4] z
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const float NEG = -INFINITY;
  float ps[EPL];
  int cn[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    ps[i] = 0.f;
    cn[i] = 0;
  }
  float zs = 0.f;
  const int64_t stride = (int64_t)gridDim.x * kLossWaves;
  for (int64_t t = (int64_t)blockIdx.x * kLossWaves + wave; t < T; t += stride) {
    if (pad != nullptr && pad[t] != 0) continue;  // wave-uniform
    float lg[EPL], ex[EPL];
    bool valid[EPL];
    float mx = NEG;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane * EPL + i;
      valid[i] = e < E;
      lg[i] = valid[i] ? load_as_f32(logits, ldt, t * E + e) : NEG;
      mx = fmaxf(mx, lg[i]);
    }
    mx = wave_max_uniform(mx);
    float se = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      ex[i] = valid[i] ? expf(lg[i] - mx) : 0.f;
      se += ex[i];
    }
    se = wave_sum(se);
    if (want_z) {
      const float lse = lse_like_torch(lg, valid, mx, se, ldt);
      zs += round_to(lse * lse, ldt);
    }
    if (!want_aux) continue;
    float sc[EPL];
    if (score_fn == TT_SCORE_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) sc[i] = ex[i] / se;
    } else {
      float den = 0.f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        sc[i] = !valid[i] ? 0.f
                : score_fn == TT_SCORE_SIGMOID ? sigmoid_f(lg[i])
                                               : sqrtf(softplus_f(lg[i]));
        den += sc[i];
      }
      den = wave_sum(den) + 1e-20f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) sc[i] = sc[i] / den;
    }
    // Top-k of the scores: k rounds of the wave arg-max of the lanes' heads
    // (best remaining expert of each lane), as in router_fwd_kernel.
    bool taken[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) taken[i] = false;
    float hv = NEG;
    int hi = -1;
    auto head = [&]() {
      hv = NEG;
      hi = -1;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (valid[i] && !taken[i] && (hi < 0 || sc[i] > hv)) {
          hv = sc[i];
          hi = i;
        }
    };
    head();
    for (int j = 0; j < K; ++j) {
      const float m = wave_max_uniform(hi >= 0 ? hv : NEG);
      const uint64_t owners = __ballot(hi >= 0 && hv == m);
      const int w = __builtin_amdgcn_readfirstlane(owners ? (int)__builtin_ctzll(owners) : 0);
      if (lane == w) {
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          if (i == hi) taken[i] = true;
        head();
      }
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      ps[i] += sc[i];
      cn[i] += taken[i] ? 1 : 0;
    }
  }
  // Combine the block's four waves in wave order.
  float* sp = lsm;
  int* scn = reinterpret_cast<int*>(lsm + kLossWaves * E);
  float* sz = lsm + 2 * kLossWaves * E;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane * EPL + i;
    if (e < E) {
      sp[wave * E + e] = ps[i];
      scn[wave * E + e] = cn[i];
    }
  }
  if (lane == 0) sz[wave] = zs;
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float p = 0.f;
    int c = 0;
    for (int w = 0; w < kLossWaves; ++w) {
      p += sp[w * E + e];
      c += scn[w * E + e];
    }
    part_p[(int64_t)blockIdx.x * E + e] = p;
    part_c[(int64_t)blockIdx.x * E + e] = c;
  }
  if (threadIdx.x == 0) {
    float z = 0.f;
    for (int w = 0; w < kLossWaves; ++w) z += sz[w];
    part_z[blockIdx.x] = z;
  }
}

// One wave per expert (block e < E) and one for z (block E): lane l sums the
// partial rows l, l + 64, ... in order, then a butterfly adds the lanes, so
// the result does not depend on scheduling.
__global__ __launch_bounds__(64) void router_loss_reduce_kernel(
    const float* __restrict__ part_p, const int* __restrict__ part_c,
    const float* __restrict__ part_z, int nb, int E, float* __restrict__ prob_sum,
    int64_t* __restrict__ counts, float* __restrict__ z_sum) {
  const int lane = threadIdx.x;
  const int e = blockIdx.x;
  if (e < E) {
    if (prob_sum == nullptr) return;
    float p = 0.f;
    int c = 0;
    for (int b = lane; b < nb; b += TT_WAVE) {
      p += part_p[(int64_t)b * E + e];
      c += part_c[(int64_t)b * E + e];
    }
    p = wave_sum(p);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, TT_WAVE);
    if (lane == 0) {
      prob_sum[e] = p;
      counts[e] = c;
    }
  } else if (z_sum != nullptr) {
    float z = 0.f;
    for (int b = lane; b < nb; b += TT_WAVE) z += part_z[b];
    z = wave_sum(z);
    if (lane == 0) *z_sum = z;
  }
}

// d logits of  sum_e g_p[e] * prob_sum[e] + g_z * z_sum  (one wave per token;
// padding tokens get zeros). Softmax scores: s * (g - <s, g>); normalised
// sigmoid / sqrt(softplus) r / (sum r + 1e-20): dr = g / D - <g, r> / D^2,
// then r' = r (1 - r) or softplus' / (2 r); z: g_z * 2 r(lse) * softmax.
// For bf16 / f16 logits the two terms follow the reference's autograd in
// that dtype: the aux term is the fp32 score gradient rounded once (the
// backward of the cast to fp32); the z term rounds where PyTorch's bf16 ops
// do: g = r(g_z), square: r(g * 2 lse), logsumexp: r(g' * r(exp(r(x - lse))))
// (moe_utils.py:61-70); the sum of the two is rounded as autograd's add.
template <int EPL>
__global__ __launch_bounds__(256) void router_loss_bwd_kernel(
    const void* __restrict__ logits, int ldt, int64_t T, int E, int score_fn,
    const uint8_t* __restrict__ pad, const float* __restrict__ g_p, const float* __restrict__ g_z,
    void* __restrict__ grad_logits) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= T) return;
  const float NEG = -INFINITY;
  float out[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) out[i] = 0.f;
  if (pad == nullptr || pad[t] == 0) {
    float lg[EPL], ex[EPL];
    bool valid[EPL];
    float mx = NEG;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane * EPL + i;
      valid[i] = e < E;
      lg[i] = valid[i] ? load_as_f32(logits, ldt, t * E + e) : NEG;
      mx = fmaxf(mx, lg[i]);
    }
    mx = wave_max_uniform(mx);
    float se = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      ex[i] = valid[i] ? expf(lg[i] - mx) : 0.f;
      se += ex[i];
    }
    se = wave_sum(se);
    const bool low = ldt != TT_F32 && ldt != TT_F64;
    float zt[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) zt[i] = 0.f;
    if (g_z != nullptr) {
      const float lse = lse_like_torch(lg, valid, mx, se, ldt);
      if (low) {
        const float gl = round_to(round_to(*g_z, ldt) * (2.f * lse), ldt);
#pragma unroll
        for (int i = 0; i < EPL; ++i)
          zt[i] = valid[i] ? round_to(gl * round_to(expf(round_to(lg[i] - lse, ldt)), ldt), ldt)
                           : 0.f;
      } else {
        const float f = *g_z * 2.f * lse;
#pragma unroll
        for (int i = 0; i < EPL; ++i) zt[i] = f * (ex[i] / se);
      }
    }
    if (g_p != nullptr) {
      float g[EPL];
#pragma unroll
      for (int i = 0; i < EPL; ++i) g[i] = valid[i] ? g_p[lane * EPL + i] : 0.f;
      if (score_fn == TT_SCORE_SOFTMAX) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) dot += (ex[i] / se) * g[i];
        dot = wave_sum(dot);
#pragma unroll
        for (int i = 0; i < EPL; ++i) out[i] += (ex[i] / se) * (g[i] - dot);
      } else {
        float r[EPL];
        float den = 0.f, dot = 0.f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          r[i] = !valid[i] ? 0.f
                 : score_fn == TT_SCORE_SIGMOID ? sigmoid_f(lg[i])
                                                : sqrtf(softplus_f(lg[i]));
          den += r[i];
          dot += g[i] * r[i];
        }
        den = wave_sum(den) + 1e-20f;
        dot = wave_sum(dot);
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
          if (!valid[i]) continue;
          const float dr = g[i] / den - dot / (den * den);
          float d;
          if (score_fn == TT_SCORE_SIGMOID) {
            d = r[i] * (1.0f - r[i]);
          } else {
            const float dsp = lg[i] > 20.0f ? 1.0f : sigmoid_f(lg[i]);
            d = r[i] > 0.f ? dsp / (2.0f * r[i]) : 0.f;
          }
          out[i] += dr * d;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i) out[i] = (low ? round_to(out[i], ldt) : out[i]) + zt[i];
  }
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane * EPL + i;
    if (e < E) store_from_f32(grad_logits, ldt, t * E + e, out[i]);
  }
}

// ---------------------------------------------------------------------------
// Routing index.
// ---------------------------------------------------------------------------
constexpr int kIdxBlock = 256;  // tokens per block

// Slot j of token t is accepted when its id lies in [0, E) and no earlier
// slot of the token holds the same id; rejected slots get row -1 (skipped by
// every later kernel) and are counted, so a caller can detect bad routing.
__device__ __forceinline__ bool route_slot_ok(const int64_t* __restrict__ ids_t, int j,
                                              int64_t e, int E) {
  if (e < 0 || e >= E) return false;
  for (int i = 0; i < j; ++i)
    if (ids_t[i] == e) return false;
  return true;
}

// Per-block expert histograms (bc[e * nb + block]) and per-block counts of
// rejected slots (bad[block]); every entry is written, so nothing needs
// clearing between calls.
__global__ __launch_bounds__(kIdxBlock) void route_hist_kernel(
    const int64_t* __restrict__ ids, int64_t T, int K, int E, int nb, int* __restrict__ bc,
    int* __restrict__ bad) {
  extern __shared__ int hist[];
  __shared__ int nbad;
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  if (threadIdx.x == 0) nbad = 0;
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * kIdxBlock + threadIdx.x;
  if (t < T) {
    const int64_t* ids_t = ids + t * K;
    int rejected = 0;
    for (int j = 0; j < K; ++j) {
      const int64_t e = ids_t[j];
      if (route_slot_ok(ids_t, j, e, E)) atomicAdd(&hist[e], 1);
      else ++rejected;
    }
    if (rejected) atomicAdd(&nbad, rejected);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) bc[(int64_t)e * nb + blockIdx.x] = hist[e];
  if (threadIdx.x == 0) bad[blockIdx.x] = nbad;
}

// One wave per expert: exclusive scan of its per-block counts, in place.
// Block 0 also adds the per-block rejected counts (fixed lane order) into
// *bad_total.
__global__ __launch_bounds__(64) void route_scan_kernel(int* __restrict__ bc, int nb, int E,
                                                        int* __restrict__ totals,
                                                        int64_t* __restrict__ counts,
                                                        const int* __restrict__ bad,
                                                        int* __restrict__ bad_total) {
  const int e = blockIdx.x;
  const int lane = threadIdx.x;
  int* col = bc + (int64_t)e * nb;
  int running = 0;
  for (int base = 0; base < nb; base += TT_WAVE) {
    const int i = base + lane;
    const int c = i < nb ? col[i] : 0;
    int incl = c;
#pragma unroll
    for (int off = 1; off < TT_WAVE; off <<= 1) {
      const int o = __shfl_up(incl, off, TT_WAVE);
      if (lane >= off) incl += o;
    }
    if (i < nb) col[i] = running + incl - c;
    running += __shfl(incl, TT_WAVE - 1, TT_WAVE);
  }
  if (lane == 0) {
    totals[e] = running;
    counts[e] = running;
  }
  if (e == 0) {
    int sum = 0;
    for (int i = lane; i < nb; i += TT_WAVE) sum += bad[i];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, TT_WAVE);
    if (lane == 0) *bad_total = sum;
  }
}

// Experts up to which the rank kernel keeps a 64-bit lane mask per expert
// and wave in LDS (4 * E * 8 bytes); beyond, it ballots once per expert.
constexpr int kMaskExperts = 1024;

template <int KMAX, bool MASKS>
__global__ __launch_bounds__(kIdxBlock) void route_rank_kernel(
    const int64_t* __restrict__ ids, int64_t T, int K, int E, int nb, const int* __restrict__ bc,
    const int* __restrict__ totals, const void* __restrict__ probs, int pbytes,
    int32_t* __restrict__ rows_out, int32_t* __restrict__ token_of_row,
    void* __restrict__ packed_probs) {
  extern __shared__ __align__(16) int smem[];
  int* start = smem;           // [E]   first packed row of each expert
  int* wbase = smem + E;       // [4][E] per-wave base row of each expert
  // [4][E] lane masks (MASKS), 8-byte aligned after the two int arrays.
  uint64_t* wmask = reinterpret_cast<uint64_t*>(smem + 5 * E + (E & 1));
  __shared__ int wsum[kIdxBlock / TT_WAVE];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  // Exclusive scan of the expert totals (each thread owns a run of experts).
  const int per = (E + kIdxBlock - 1) / kIdxBlock;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) local += totals[e];
  }
  int incl = local;
#pragma unroll
  for (int off = 1; off < TT_WAVE; off <<= 1) {
    const int o = __shfl_up(incl, off, TT_WAVE);
    if (lane >= off) incl += o;
  }
  if (lane == TT_WAVE - 1) wsum[wave] = incl;
  for (int e = tid; e < 4 * E; e += kIdxBlock) wbase[e] = 0;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += wsum[w];
  int run = before + incl - local;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      start[e] = run;
      run += totals[e];
    }
  }

  // Per-wave counts of this block.
  const int64_t t = (int64_t)blockIdx.x * kIdxBlock + tid;
  int my[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    my[j] = -1;
    if (j < K && t < T) {
      const int64_t e = ids[t * K + j];
      my[j] = (e >= 0 && e < E) ? (int)e : -1;
    }
  }
  // A repeated id keeps its first slot only (as the histogram counted it).
#pragma unroll
  for (int j = 1; j < KMAX; ++j)
#pragma unroll
    for (int i = 0; i < j; ++i)
      if (my[j] >= 0 && my[i] == my[j]) my[j] = -1;
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
    if (my[j] >= 0) atomicAdd(&wbase[wave * E + my[j]], 1);
  __syncthreads();
  // Turn per-wave counts into per-wave base rows.
  for (int e = tid; e < E; e += kIdxBlock) {
    int base = start[e] + bc[(int64_t)e * nb + blockIdx.x];
    for (int w = 0; w < kIdxBlock / TT_WAVE; ++w) {
      const int c = wbase[w * E + e];
      wbase[w * E + e] = base;
      base += c;
    }
  }
  __syncthreads();

  // In-wave stable rank of lane l for expert e: popcount of the lanes below
  // l holding e (a token selects an expert at most once).
  int row[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) row[j] = -1;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (TT_WAVE - lane));
  if constexpr (MASKS) {
    // Lane masks per expert: every lane ORs its bit into the masks of its
    // experts (order-free, so deterministic), then reads them back. LDS
    // operations of one wave complete in order; the waits make it explicit.
    uint64_t* wm = wmask + (int64_t)wave * E;
    for (int e = lane; e < E; e += TT_WAVE) wm[e] = 0ull;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (my[j] >= 0) atomicOr(reinterpret_cast<unsigned long long*>(&wm[my[j]]), 1ull << lane);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (my[j] >= 0) row[j] = wbase[wave * E + my[j]] + __popcll(wm[my[j]] & below);
  }
  for (int e = 0; !MASKS && e < E; ++e) {
    int slot = -1;
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (my[j] == e) slot = j;
    const uint64_t mask = __ballot(slot >= 0);
    if (mask == 0) continue;  // uniform across the wave
    if (slot >= 0) {
      const int r = wbase[wave * E + e] + __popcll(mask & below);
#pragma unroll
      for (int j = 0; j < KMAX; ++j)
        if (j == slot) row[j] = r;
    }
  }
  if (t < T) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j >= K) break;
      const int r = row[j];
      rows_out[t * K + j] = r;
      if (r >= 0) {
        token_of_row[r] = (int32_t)t;
        if (probs != nullptr && packed_probs != nullptr) {
          const int64_t src = t * E + my[j];
          if (pbytes == 4)
            static_cast<uint32_t*>(packed_probs)[r] = static_cast<const uint32_t*>(probs)[src];
          else
            static_cast<uint16_t*>(packed_probs)[r] = static_cast<const uint16_t*>(probs)[src];
        }
      }
    }
  }
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

template <int EPL>
void launch_router_fwd(dim3 g, hipStream_t s, const void* logits, int ldt, int64_t T, int E, int K,
                       int sf, int pre, const float* bias, int G, int GK, float scale,
                       const int64_t* fixed, void* probs, uint8_t* rmap, int64_t* top) {
  if (ldt == TT_F64)
    hipLaunchKernelGGL((router_fwd_kernel<EPL, double>), g, dim3(256), 0, s, logits, ldt, T, E, K,
                       sf, pre, bias, G, GK, scale, fixed, probs, rmap, top);
  else
    hipLaunchKernelGGL((router_fwd_kernel<EPL, float>), g, dim3(256), 0, s, logits, ldt, T, E, K,
                       sf, pre, bias, G, GK, scale, fixed, probs, rmap, top);
}

template <int EPL>
void launch_router_bwd(dim3 g, hipStream_t s, const void* logits, int ldt, int64_t T, int E, int K,
                       int sf, int pre, float scale, const int64_t* top, const void* grad,
                       void* gl) {
  hipLaunchKernelGGL(router_bwd_kernel<EPL>, g, dim3(256), 0, s, logits, ldt, T, E, K, sf, pre,
                     scale, top, grad, gl);
}

// ---------------------------------------------------------------------------
// Gating linear fused with the top-k (models/modules/moe/router.py:25-58, then
// utils.py:127-230): logits = x W^T for a tile of 64 tokens and all E experts
// on MFMA (16-bit operands, fp32 accumulation), rounded to the logits dtype,
// written out, and routed from LDS by route_row (one wave per token). With
// 16-bit x and W the reference's fp32 router (x.float() @ W.float().T) forms
// the same exact products; only the order of the fp32 sum differs.
// Operand rows (64 tokens, then E experts) stream HBM -> LDS by buffer DMA in
// 64-deep chunks, 128-byte rows, chunk c of row r in slot c ^ ((r >> 1) & 7);
// rows past T come back as zeros from the resource bound. Template P = DMA
// instructions per wave per chunk = (64 + E) / 32, so E = 32 P - 64.
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(4))) int gi32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 gbf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 gf16x8;
typedef __attribute__((ext_vector_type(16))) float gf32x16;
typedef __attribute__((ext_vector_type(4))) unsigned gu32x4;
typedef __attribute__((address_space(3))) char glds_char;
typedef __attribute__((address_space(3))) gu32x4 glds_u32x4;

constexpr int kGateRow = 128;  // bytes of one row of a 64-deep chunk

#define RG_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 0xF) | ((((n) >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8))

__device__ __forceinline__ gi32x4 rg_rsrc(const void* base, int64_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t n = bytes <= 0 ? 0u : (bytes < 0xFFFFFFF0ll ? (uint32_t)bytes : 0xFFFFFFF0u);
  gi32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(b >> 32) & 0xFFFFu));
  r.z = __builtin_amdgcn_readfirstlane((int)n);
  r.w = 0x00020000;
  return r;
}

// One 16-byte load per lane into LDS at lds_addr + 16 * lane (lds_addr -> M0).
__device__ __forceinline__ void rg_dma16(uint32_t voff, gi32x4 rsrc, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory");
}

__device__ __forceinline__ uint32_t rg_swz(int r, int c) {
  return (uint32_t)(r * kGateRow + ((c ^ ((r >> 1) & 7)) << 4));
}

template <int ET>
__device__ __forceinline__ gf32x16 rg_mma(const uint4& a, const uint4& b, const gf32x16& c);
template <>
__device__ __forceinline__ gf32x16 rg_mma<TT_BF16>(const uint4& a, const uint4& b,
                                                   const gf32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gbf16x8, a),
                                                  __builtin_bit_cast(gbf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ gf32x16 rg_mma<TT_F16>(const uint4& a, const uint4& b,
                                                  const gf32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(gf16x8, a),
                                                 __builtin_bit_cast(gf16x8, b), c, 0, 0, 0);
}

// N 32-expert tiles (E = 32 N), TOK tokens per block (64, or 32 when 64-token
// blocks would leave compute units idle).
template <int N, int TOK>
struct GateShape {
  static constexpr int E = 32 * N;                              // experts
  static constexpr int NT = N;                                  // 32-expert tiles
  static constexpr int MT = TOK / 32;                           // 32-token tiles
  static constexpr int WAVES = 16;                              // waves per block
  static constexpr int TPW = (MT * NT + WAVES - 1) / WAVES;     // 32x32 output tiles per wave
  static constexpr int NI = (TOK + E) / 8;                      // DMA loads per chunk (8 rows)
  static constexpr int PW = (NI + WAVES - 1) / WAVES;           // ... per wave (rest: dummy)
  static constexpr int SB = (TOK + E) * kGateRow;               // stage bytes
  static constexpr int NS = 4 * SB + 1024 <= 128 * 1024 ? 4 : 3;  // stages in the ring
  static constexpr int LS = E + 4;                              // logits tile row stride (floats)
  static constexpr int EPL = E <= 64 ? 1 : (E <= 128 ? 2 : 4);
  static constexpr int RING = NS * SB + 1024;                   // + a dummy DMA target
  static constexpr int LDS = RING > TOK * LS * 4 ? RING : TOK * LS * 4;
};

// 16 waves: the GEMM gives each wave one or two 32x32 (token, expert) tiles;
// the selection then routes TOK / 16 tokens per wave.
template <int ET, int N, int TOK>
__global__ __launch_bounds__(1024) void router_gate_fwd_kernel(
    const char* __restrict__ x, const char* __restrict__ w, int64_t T, int H, int ldt, int K,
    int score_fn, int pre_softmax, const float* __restrict__ bias, int G, int GK, float scaling,
    const int64_t* __restrict__ fixed, void* __restrict__ logits, void* __restrict__ probs,
    uint8_t* __restrict__ rmap, int64_t* __restrict__ top_idx) {
  typedef GateShape<N, TOK> S;
  constexpr int E = S::E, NS = S::NS, SB = S::SB, EPL = S::EPL, PW = S::PW, MT = S::MT;
  extern __shared__ __align__(16) char gsm[];
  glds_char* const lds = (glds_char*)gsm;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t t0 = (int64_t)blockIdx.x * TOK;
  const int nch = H / 64;
  const int64_t nrow = T - t0 < TOK ? T - t0 : TOK;
  const gi32x4 rx = rg_rsrc(x + t0 * H * 2, nrow * H * 2);
  const gi32x4 rw = rg_rsrc(w, (int64_t)E * H * 2);

  // This wave's PW loads of chunk kc: load g = PW wave + q fills stage rows
  // 8 g .. 8 g + 7. Loads past the NI of a chunk, and chunks past the end,
  // read a zero-size resource (loads g >= NI into the dummy slot), so every
  // wave always has PW loads per chunk in flight and the counts below hold.
  auto issue = [&](int kc, int stage) {
#pragma unroll
    for (int q = 0; q < PW; ++q) {
      const int g = wave * PW + q;
      const bool real = g < S::NI;
      const bool isx = 8 * g < TOK;
      const int r = 8 * g + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int orow = isx ? r : r - TOK;
      const uint32_t off = (uint32_t)(((int64_t)orow * H + (int64_t)kc * 64 + c * 8) * 2);
      const bool live = real && kc < nch;
      gi32x4 rs;
      rs.x = __builtin_amdgcn_readfirstlane(isx ? rx.x : rw.x);
      rs.y = __builtin_amdgcn_readfirstlane(isx ? rx.y : rw.y);
      rs.z = __builtin_amdgcn_readfirstlane(live ? (isx ? rx.z : rw.z) : 0);
      rs.w = 0x00020000;
      const uint32_t dst = real ? (uint32_t)(stage * SB + 8 * g * kGateRow) : (uint32_t)(NS * SB);
      rg_dma16(live ? off : 0u, rs, lds0 + dst);
    }
  };

  gf32x16 acc[S::TPW];
#pragma unroll
  for (int i = 0; i < S::TPW; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s, s);
  for (int kc = 0; kc < nch; ++kc) {
    RG_WAIT_VMCNT((NS - 2) * PW);  // this wave's part of chunk kc has landed
    __syncthreads();               // everyone's part has; stage (kc - 1) % NS is free
    issue(kc + NS - 1, (kc + NS - 1) % NS);
    glds_char* const st = lds + (kc % NS) * SB;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = 2 * s + (lane >> 5);
#pragma unroll
      for (int i = 0; i < S::TPW; ++i) {
        const int tile = wave + S::WAVES * i;  // token tile tile % MT, expert tile tile / MT
        if (tile < MT * S::NT) {
          const uint4 a = __builtin_bit_cast(uint4, *reinterpret_cast<const glds_u32x4*>(
                                                        st + rg_swz(32 * (tile % MT) + (lane & 31), c)));
          const uint4 b = __builtin_bit_cast(
              uint4, *reinterpret_cast<const glds_u32x4*>(
                         st + rg_swz(TOK + 32 * (tile / MT) + (lane & 31), c)));
          acc[i] = rg_mma<ET>(b, a, acc[i]);
        }
      }
    }
  }
  RG_WAIT_VMCNT(0);
  __syncthreads();

  // Logits tile in LDS (fp32 values of the logits dtype). Lane l holds token
  // row 32 m + l % 32, experts 32 j + 8 q + 4 (l / 32) + 0..3 in acc[4 q ..].
  float* const L = reinterpret_cast<float*>(gsm);
#pragma unroll
  for (int i = 0; i < S::TPW; ++i) {
    const int tile = wave + S::WAVES * i;
    if (tile >= MT * S::NT) continue;
    const int row = 32 * (tile % MT) + (lane & 31);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = 32 * (tile / MT) + 8 * q + 4 * (lane >> 5);
      float4 v;
      v.x = round_to(acc[i][4 * q + 0], ldt);
      v.y = round_to(acc[i][4 * q + 1], ldt);
      v.z = round_to(acc[i][4 * q + 2], ldt);
      v.w = round_to(acc[i][4 * q + 3], ldt);
      *reinterpret_cast<float4*>(L + row * S::LS + col) = v;
    }
  }
  __syncthreads();
  for (int idx = tid; idx < TOK * E; idx += 64 * S::WAVES) {
    const int row = idx / E, col = idx % E;
    if (row < nrow) store_from_f32(logits, ldt, (t0 + row) * E + col, L[row * S::LS + col]);
  }
  constexpr int RPW = TOK / S::WAVES;  // tokens routed per wave
  for (int rr = 0; rr < RPW; ++rr) {
    const int row = wave * RPW + rr;
    if (row >= nrow) break;  // wave-uniform; no block synchronisation follows
    float lg[EPL];
    bool valid[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane * EPL + i;
      valid[i] = e < E;
      lg[i] = valid[i] ? L[row * S::LS + e] : -INFINITY;
    }
    route_row<EPL>(lane, t0 + row, lg, lg, valid, ldt, E, K, score_fn, pre_softmax, bias, G, GK,
                   scaling, fixed, probs, rmap, top_idx);
  }
}

template <int ET, int N, int TOK>
int launch_gate_t(const void* x, const void* w, int64_t T, int H, int ldt, int K, int sf, int pre,
                  const float* bias, int G, int GK, float scale, const int64_t* fixed,
                  void* logits, void* probs, uint8_t* rmap, int64_t* top, hipStream_t s) {
  typedef GateShape<N, TOK> S;
  static_assert(S::LDS <= 160 * 1024, "gate tile exceeds LDS");
  static bool allowed = false;  // the attribute belongs to the kernel, for every device
  if (!allowed) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&router_gate_fwd_kernel<ET, N, TOK>),
        hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      tt_set_error("router_gate: hipFuncSetAttribute(%d bytes): %s", S::LDS,
                   hipGetErrorString(e));
      return TT_ERR_HIP;
    }
    allowed = true;
  }
  const dim3 grid((unsigned)((T + TOK - 1) / TOK));
  hipLaunchKernelGGL((router_gate_fwd_kernel<ET, N, TOK>), grid, dim3(64 * S::WAVES), S::LDS, s,
                     static_cast<const char*>(x), static_cast<const char*>(w), T, H, ldt, K, sf,
                     pre, bias, G, GK, scale, fixed, logits, probs, rmap, top);
  return tt_check_launch("router_gate_fwd");
}

// Compute units of the current device, cached per device.
int gate_cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// 64 tokens per block, or 32 when 64-token blocks would not cover the device.
template <int ET, int N>
int launch_gate(const void* x, const void* w, int64_t T, int H, int ldt, int K, int sf, int pre,
                const float* bias, int G, int GK, float scale, const int64_t* fixed, void* logits,
                void* probs, uint8_t* rmap, int64_t* top, hipStream_t s) {
  if ((T + 63) / 64 < gate_cu_count())
    return launch_gate_t<ET, N, 32>(x, w, T, H, ldt, K, sf, pre, bias, G, GK, scale, fixed,
                                    logits, probs, rmap, top, s);
  return launch_gate_t<ET, N, 64>(x, w, T, H, ldt, K, sf, pre, bias, G, GK, scale, fixed, logits,
                                  probs, rmap, top, s);
}

int epl_for(int E) {
  const int need = (E + TT_WAVE - 1) / TT_WAVE;
  int epl = 1;
  while (epl < need) epl <<= 1;
  return epl;
}

bool float_dtype(int d) { return d == TT_F32 || d == TT_BF16 || d == TT_F16; }
// Logits dtypes of the top-k router and its losses (fp64: moe_router_dtype "fp64").
bool logits_dtype_ok(int d) { return float_dtype(d) || d == TT_F64; }

}  // namespace

extern "C" int tt_router_topk_fwd(const void* logits, int logits_dtype, int64_t num_tokens,
                                  int32_t num_experts, int32_t topk, int32_t score_function,
                                  int32_t pre_softmax, const float* expert_bias,
                                  int32_t num_groups, int32_t group_topk, float scaling_factor,
                                  const int64_t* fixed_indices, void* probs,
                                  uint8_t* routing_map, int64_t* top_indices, void* stream) {
  TT_REQUIRE(logits_dtype_ok(logits_dtype), "router: unsupported logits dtype %d", logits_dtype);
  TT_REQUIRE(num_tokens >= 0, "router: negative token count");
  TT_REQUIRE(num_experts >= 1 && num_experts <= 1024, "router: num_experts must be in [1, 1024]");
  TT_REQUIRE(topk >= 1 && topk <= 64 && topk <= num_experts, "router: topk must be in [1, min(64, E)]");
  TT_REQUIRE(score_function >= 0 && score_function <= 2, "router: bad score function");
  const int epl = epl_for(num_experts);
  if (group_topk > 0 && fixed_indices == nullptr) {
    TT_REQUIRE(num_groups > 0 && num_experts % num_groups == 0,
               "router: num_experts must be divisible by num_groups");
    TT_REQUIRE(group_topk <= num_groups && topk % group_topk == 0,
               "router: topk must be divisible by group_topk <= num_groups");
    const int gs = num_experts / num_groups;
    const int width = gs / epl;
    TT_REQUIRE(gs % epl == 0 && width >= 1 && (width & (width - 1)) == 0 && TT_WAVE % width == 0,
               "router: group size %d does not map onto whole lanes (%d experts per lane)", gs, epl);
    TT_REQUIRE(topk / group_topk <= gs, "router: topk / group_topk exceeds the group size");
    TT_REQUIRE(topk <= group_topk * gs, "router: topk exceeds the experts of the kept groups");
  }
  if (num_tokens == 0) return TT_OK;
  const dim3 grid((unsigned)((num_tokens + kRouterWaves - 1) / kRouterWaves));
  const int gk = fixed_indices ? 0 : group_topk;
  switch (epl) {
#define TT_CASE(N)                                                                               \
  case N:                                                                                        \
    launch_router_fwd<N>(grid, S(stream), logits, logits_dtype, num_tokens, num_experts, topk,   \
                         score_function, pre_softmax, expert_bias, num_groups, gk,              \
                         scaling_factor, fixed_indices, probs, routing_map, top_indices);        \
    break;
    TT_CASE(1) TT_CASE(2) TT_CASE(4) TT_CASE(8) TT_CASE(16)
#undef TT_CASE
    default:
      tt_set_error("router: unsupported expert count");
      return TT_ERR_UNSUPPORTED;
  }
  return tt_check_launch("router_fwd");
}

extern "C" int tt_router_topk_bwd(const void* logits, int logits_dtype, int64_t num_tokens,
                                  int32_t num_experts, int32_t topk, int32_t score_function,
                                  int32_t pre_softmax, float scaling_factor,
                                  const int64_t* top_indices, const void* grad_probs,
                                  void* grad_logits, void* stream) {
  TT_REQUIRE(logits_dtype_ok(logits_dtype), "router_bwd: unsupported logits dtype %d", logits_dtype);
  TT_REQUIRE(num_experts >= 1 && num_experts <= 1024, "router_bwd: num_experts must be in [1, 1024]");
  TT_REQUIRE(topk >= 1 && topk <= 64 && topk <= num_experts, "router_bwd: bad topk");
  TT_REQUIRE(score_function >= 0 && score_function <= 2, "router_bwd: bad score function");
  if (num_tokens == 0) return TT_OK;
  const dim3 grid((unsigned)((num_tokens + kRouterWaves - 1) / kRouterWaves));
  switch (epl_for(num_experts)) {
#define TT_CASE(N)                                                                            \
  case N:                                                                                     \
    launch_router_bwd<N>(grid, S(stream), logits, logits_dtype, num_tokens, num_experts, topk, \
                         score_function, pre_softmax, scaling_factor, top_indices, grad_probs, \
                         grad_logits);                                                        \
    break;
    TT_CASE(1) TT_CASE(2) TT_CASE(4) TT_CASE(8) TT_CASE(16)
#undef TT_CASE
    default:
      tt_set_error("router_bwd: unsupported expert count");
      return TT_ERR_UNSUPPORTED;
  }
  return tt_check_launch("router_bwd");
}

// Workspace: bc [nb * E] | totals [E] | bad [nb] | bad_total [1], int32.
extern "C" size_t tt_route_index_workspace(int64_t num_tokens, int32_t num_experts) {
  const int64_t nb = (num_tokens + kIdxBlock - 1) / kIdxBlock;
  return (size_t)(nb * num_experts + num_experts + nb + 1) * sizeof(int) + 256;
}

extern "C" size_t tt_route_index_rejected_offset(int64_t num_tokens, int32_t num_experts) {
  const int64_t nb = (num_tokens + kIdxBlock - 1) / kIdxBlock;
  return (size_t)(nb * num_experts + num_experts + nb) * sizeof(int);
}

namespace {

int route_index_args(int64_t num_tokens, int32_t topk, int32_t num_experts,
                     const void* probs_dense, void* packed_probs, int probs_dtype) {
  TT_REQUIRE(num_tokens >= 0 && num_tokens * (int64_t)topk < (1ll << 31),
             "route_index: T * k must fit in int32");
  TT_REQUIRE(num_experts >= 1 && num_experts <= 2048, "route_index: num_experts must be in [1, 2048]");
  TT_REQUIRE(topk >= 1 && topk <= 64, "route_index: topk must be in [1, 64]");
  if (probs_dense != nullptr && packed_probs != nullptr)
    TT_REQUIRE(float_dtype(probs_dtype), "route_index: unsupported probs dtype %d", probs_dtype);
  return TT_OK;
}

// The three routing-index kernels over a scratch area laid out as the
// workspace of tt_route_index (bc | totals | bad); the rejected-slot count
// goes to bad_total.
int route_index_run(const int64_t* expert_indices, int64_t num_tokens, int32_t topk,
                    int32_t num_experts, const void* probs_dense, int probs_dtype,
                    int32_t* row_indices, int32_t* token_of_row, void* packed_probs,
                    int64_t* tokens_per_expert, int* area, int* bad_total, hipStream_t s) {
  const int nb = (int)((num_tokens + kIdxBlock - 1) / kIdxBlock);
  int* bc = area;
  int* totals = bc + (int64_t)nb * num_experts;
  int* bad = totals + num_experts;
  if (num_tokens == 0) {
    // Counts are all zero; a one-wave scan over zero blocks writes them.
    hipLaunchKernelGGL(route_scan_kernel, dim3(num_experts), dim3(64), 0, s, bc, 0, num_experts,
                       totals, tokens_per_expert, bad, bad_total);
    return tt_check_launch("route_scan");
  }
  hipLaunchKernelGGL(route_hist_kernel, dim3(nb), dim3(kIdxBlock), num_experts * sizeof(int), s,
                     expert_indices, num_tokens, topk, num_experts, nb, bc, bad);
  hipLaunchKernelGGL(route_scan_kernel, dim3(num_experts), dim3(64), 0, s, bc, nb, num_experts,
                     totals, tokens_per_expert, bad, bad_total);
  const bool masks = num_experts <= kMaskExperts;
  const size_t lds = (size_t)5 * num_experts * sizeof(int) +
                     (masks ? (size_t)(num_experts & 1) * 4 + (size_t)4 * num_experts * 8 : 0);
  TT_REQUIRE(lds <= 160 * 1024 - 64, "route_index: too many experts for LDS");
  const int pbytes = tt_elem_size(probs_dtype);
  const void* pd = (packed_probs != nullptr) ? probs_dense : nullptr;
#define TT_RANK(KM)                                                                              \
  do {                                                                                           \
    if (masks)                                                                                   \
      hipLaunchKernelGGL((route_rank_kernel<KM, true>), dim3(nb), dim3(kIdxBlock), lds, s,       \
                         expert_indices, num_tokens, topk, num_experts, nb, bc, totals, pd,      \
                         pbytes, row_indices, token_of_row, packed_probs);                       \
    else                                                                                         \
      hipLaunchKernelGGL((route_rank_kernel<KM, false>), dim3(nb), dim3(kIdxBlock), lds, s,      \
                         expert_indices, num_tokens, topk, num_experts, nb, bc, totals, pd,      \
                         pbytes, row_indices, token_of_row, packed_probs);                       \
  } while (0)
  if (topk <= 2) TT_RANK(2);
  else if (topk <= 4) TT_RANK(4);
  else if (topk <= 8) TT_RANK(8);
  else if (topk <= 16) TT_RANK(16);
  else TT_RANK(64);
#undef TT_RANK
  return tt_check_launch("route_rank");
}

}  // namespace

extern "C" int tt_route_index(const int64_t* expert_indices, int64_t num_tokens, int32_t topk,
                              int32_t num_experts, const void* probs_dense, int probs_dtype,
                              int32_t* row_indices, int32_t* token_of_row, void* packed_probs,
                              int64_t* tokens_per_expert, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const int rc = route_index_args(num_tokens, topk, num_experts, probs_dense, packed_probs,
                                  probs_dtype);
  if (rc != TT_OK) return rc;
  TT_REQUIRE(workspace_bytes >= tt_route_index_workspace(num_tokens, num_experts),
             "route_index: workspace too small");
  int* area = static_cast<int*>(workspace);
  int* bad_total = reinterpret_cast<int*>(
      static_cast<char*>(workspace) + tt_route_index_rejected_offset(num_tokens, num_experts));
  return route_index_run(expert_indices, num_tokens, topk, num_experts, probs_dense, probs_dtype,
                         row_indices, token_of_row, packed_probs, tokens_per_expert, area,
                         bad_total, S(stream));
}

extern "C" size_t tt_router_loss_workspace(int64_t num_tokens, int32_t num_experts) {
  const int64_t nb = loss_blocks(num_tokens);
  return (size_t)(nb * num_experts * 2 + nb) * 4 + 256;
}

extern "C" int tt_router_loss_fwd(const void* logits, int logits_dtype, int64_t num_tokens,
                                  int32_t num_experts, int32_t topk, int32_t score_function,
                                  const uint8_t* padding_mask, float* prob_sum,
                                  int64_t* tokens_per_expert, float* z_sum, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  TT_REQUIRE(logits_dtype_ok(logits_dtype), "router_loss: unsupported logits dtype %d",
             logits_dtype);
  TT_REQUIRE(num_tokens >= 0, "router_loss: negative token count");
  TT_REQUIRE(num_experts >= 1 && num_experts <= 1024,
             "router_loss: num_experts must be in [1, 1024]");
  TT_REQUIRE(score_function >= 0 && score_function <= 2, "router_loss: bad score function");
  TT_REQUIRE((prob_sum == nullptr) == (tokens_per_expert == nullptr),
             "router_loss: prob_sum and tokens_per_expert go together");
  if (prob_sum != nullptr)
    TT_REQUIRE(topk >= 1 && topk <= num_experts, "router_loss: topk must be in [1, E]");
  TT_REQUIRE(workspace_bytes >= tt_router_loss_workspace(num_tokens, num_experts),
             "router_loss: workspace too small");
  if (prob_sum == nullptr && z_sum == nullptr) return TT_OK;
  hipStream_t s = S(stream);
  const int nb = loss_blocks(num_tokens);
  float* part_p = static_cast<float*>(workspace);
  int* part_c = reinterpret_cast<int*>(part_p + (int64_t)nb * num_experts);
  float* part_z = reinterpret_cast<float*>(part_c + (int64_t)nb * num_experts);
  int used = 0;
  if (num_tokens > 0) {
    const size_t lds = (size_t)(2 * kLossWaves * num_experts + kLossWaves) * 4;
    const int aux = prob_sum != nullptr, zz = z_sum != nullptr;
    switch (epl_for(num_experts)) {
#define TT_CASE(N)                                                                             \
  case N:                                                                                      \
    hipLaunchKernelGGL(router_loss_fwd_kernel<N>, dim3(nb), dim3(256), lds, s, logits,         \
                       logits_dtype, num_tokens, num_experts, topk, score_function,            \
                       padding_mask, aux, zz, part_p, part_c, part_z);                         \
    break;
      TT_CASE(1) TT_CASE(2) TT_CASE(4) TT_CASE(8) TT_CASE(16)
#undef TT_CASE
      default:
        tt_set_error("router_loss: unsupported expert count");
        return TT_ERR_UNSUPPORTED;
    }
    used = nb;
  }
  hipLaunchKernelGGL(router_loss_reduce_kernel, dim3(num_experts + 1), dim3(64), 0, s, part_p,
                     part_c, part_z, used, num_experts, prob_sum, tokens_per_expert, z_sum);
  return tt_check_launch("router_loss_fwd");
}

extern "C" int tt_router_loss_bwd(const void* logits, int logits_dtype, int64_t num_tokens,
                                  int32_t num_experts, int32_t score_function,
                                  const uint8_t* padding_mask, const float* grad_prob_sum,
                                  const float* grad_z_sum, void* grad_logits, void* stream) {
  TT_REQUIRE(logits_dtype_ok(logits_dtype), "router_loss_bwd: unsupported logits dtype %d",
             logits_dtype);
  TT_REQUIRE(num_tokens >= 0, "router_loss_bwd: negative token count");
  TT_REQUIRE(num_experts >= 1 && num_experts <= 1024,
             "router_loss_bwd: num_experts must be in [1, 1024]");
  TT_REQUIRE(score_function >= 0 && score_function <= 2, "router_loss_bwd: bad score function");
  if (num_tokens == 0) return TT_OK;
  const dim3 grid((unsigned)((num_tokens + kRouterWaves - 1) / kRouterWaves));
  switch (epl_for(num_experts)) {
#define TT_CASE(N)                                                                               \
  case N:                                                                                        \
    hipLaunchKernelGGL(router_loss_bwd_kernel<N>, grid, dim3(256), 0, S(stream), logits,         \
                       logits_dtype, num_tokens, num_experts, score_function, padding_mask,      \
                       grad_prob_sum, grad_z_sum, grad_logits);                                  \
    break;
    TT_CASE(1) TT_CASE(2) TT_CASE(4) TT_CASE(8) TT_CASE(16)
#undef TT_CASE
    default:
      tt_set_error("router_loss_bwd: unsupported expert count");
      return TT_ERR_UNSUPPORTED;
  }
  return tt_check_launch("router_loss_bwd");
}

extern "C" int tt_router_gate_fwd(const void* x, const void* weight, int in_dtype,
                                  int64_t num_tokens, int64_t hidden, int32_t num_experts,
                                  int logits_dtype, int32_t topk, int32_t score_function,
                                  int32_t pre_softmax, const float* expert_bias,
                                  int32_t num_groups, int32_t group_topk, float scaling_factor,
                                  const int64_t* fixed_indices, void* logits, void* probs,
                                  uint8_t* routing_map, int64_t* top_indices, void* stream) {
  TT_REQUIRE(in_dtype == TT_BF16 || in_dtype == TT_F16,
             "router_gate: input and weight must be bf16 or f16 (got dtype %d)", in_dtype);
  TT_REQUIRE(logits_dtype == TT_F32 || logits_dtype == in_dtype,
             "router_gate: logits dtype must be f32 or the input dtype");
  TT_REQUIRE(num_tokens >= 0, "router_gate: negative token count");
  TT_REQUIRE(hidden >= 64 && hidden % 64 == 0 && hidden <= (1 << 24),
             "router_gate: hidden size must be a positive multiple of 64");
  TT_REQUIRE(num_experts >= 32 && num_experts <= 256 && num_experts % 32 == 0,
             "router_gate: num_experts must be a multiple of 32 in [32, 256]");
  TT_REQUIRE(topk >= 1 && topk <= 64 && topk <= num_experts, "router_gate: bad topk");
  TT_REQUIRE(score_function >= 0 && score_function <= 2, "router_gate: bad score function");
  TT_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) & 15) == 0,
             "router_gate: x and weight must be 16-byte aligned");
  const int epl = epl_for(num_experts);
  if (group_topk > 0 && fixed_indices == nullptr) {
    TT_REQUIRE(num_groups > 0 && num_experts % num_groups == 0,
               "router_gate: num_experts must be divisible by num_groups");
    TT_REQUIRE(group_topk <= num_groups && topk % group_topk == 0,
               "router_gate: topk must be divisible by group_topk <= num_groups");
    const int gs = num_experts / num_groups;
    const int width = gs / epl;
    TT_REQUIRE(gs % epl == 0 && width >= 1 && (width & (width - 1)) == 0 && TT_WAVE % width == 0,
               "router_gate: group size %d does not map onto whole lanes (%d experts per lane)",
               gs, epl);
    TT_REQUIRE(topk / group_topk <= gs, "router_gate: topk / group_topk exceeds the group size");
    TT_REQUIRE(topk <= group_topk * gs, "router_gate: topk exceeds the experts of the kept groups");
  }
  if (num_tokens == 0) return TT_OK;
  const int gk = fixed_indices ? 0 : group_topk;
  const int H = (int)hidden;
  const int NE = num_experts / 32;
#define TT_GATE_N(ET, NN)                                                                       \
  case NN:                                                                                     \
    return launch_gate<ET, NN>(x, weight, num_tokens, H, logits_dtype, topk, score_function,   \
                               pre_softmax, expert_bias, num_groups, gk, scaling_factor,       \
                               fixed_indices, logits, probs, routing_map, top_indices,         \
                               S(stream));
#define TT_GATE(ET)                                                                            \
  switch (NE) {                                                                                \
    TT_GATE_N(ET, 1) TT_GATE_N(ET, 2) TT_GATE_N(ET, 3) TT_GATE_N(ET, 4)                        \
    TT_GATE_N(ET, 5) TT_GATE_N(ET, 6) TT_GATE_N(ET, 7) default: TT_GATE_N(ET, 8)               \
  }
  if (in_dtype == TT_BF16) {
    TT_GATE(TT_BF16)
  } else {
    TT_GATE(TT_F16)
  }
#undef TT_GATE_N
#undef TT_GATE
}

// ---------------------------------------------------------------------------
// Routing index without a caller workspace.
// ---------------------------------------------------------------------------
// The per-block histograms, expert totals and rejected-slot counts of
// tt_route_index_noalloc live in this fixed array instead of a workspace:
// one copy per GPU, held until the process ends. Every kernel writes each
// entry it later reads, so nothing needs clearing between calls. All calls
// on one GPU share the array: calls that overlap on a GPU (other streams or
// host threads) race.
constexpr size_t kRouteScratchBytes = 1u << 20;
static __device__ __align__(256) unsigned char scratch[kRouteScratchBytes];

namespace {

constexpr int kScratchDevices = 64;
void* g_scratch_ptr[kScratchDevices];
hipError_t g_scratch_err[kScratchDevices];
std::once_flag g_scratch_once[kScratchDevices];

// Device address of the current GPU's copy of `scratch`, looked up once per
// device with that device current. In host code the array's name only stands
// for the symbol; kernels get this address.
int route_scratch(void** out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) {
    tt_set_error("route_index_noalloc: hipGetDevice: %s", hipGetErrorString(ge));
    return TT_ERR_HIP;
  }
  TT_REQUIRE(dev >= 0 && dev < kScratchDevices, "route_index_noalloc: device %d unsupported", dev);
  std::call_once(g_scratch_once[dev], [dev]() {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = p;
  });
  if (g_scratch_err[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr) {
    tt_set_error("route_index_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                 hipGetErrorString(g_scratch_err[dev]));
    return TT_ERR_HIP;
  }
  *out = g_scratch_ptr[dev];
  return TT_OK;
}

}  // namespace

extern "C" int tt_route_index_noalloc(const int64_t* expert_indices, int64_t num_tokens,
                                      int32_t topk, int32_t num_experts, const void* probs_dense,
                                      int probs_dtype, int32_t* row_indices,
                                      int32_t* token_of_row, void* packed_probs,
                                      int64_t* tokens_per_expert, int32_t* rejected,
                                      void* stream) {
  const int rc = route_index_args(num_tokens, topk, num_experts, probs_dense, packed_probs,
                                  probs_dtype);
  if (rc != TT_OK) return rc;
  const size_t need = tt_route_index_workspace(num_tokens, num_experts);
  TT_REQUIRE(need <= kRouteScratchBytes,
             "route_index_noalloc: %lld tokens over %d experts need %zu bytes of scratch, "
             "more than the fixed %zu; use tt_route_index with a workspace",
             (long long)num_tokens, num_experts, need, kRouteScratchBytes);
  void* area = nullptr;
  const int rs = route_scratch(&area);
  if (rs != TT_OK) return rs;
  int* bad_total = rejected != nullptr
                       ? reinterpret_cast<int*>(rejected)
                       : reinterpret_cast<int*>(static_cast<char*>(area) +
                                                tt_route_index_rejected_offset(num_tokens,
                                                                               num_experts));
  return route_index_run(expert_indices, num_tokens, topk, num_experts, probs_dense, probs_dtype,
                         row_indices, token_of_row, packed_probs, tokens_per_expert,
                         static_cast<int*>(area), bad_total, S(stream));
}
