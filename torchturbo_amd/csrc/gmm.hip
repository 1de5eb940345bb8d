// Grouped GEMM over variable-length expert segments (gfx950 MFMA).
//
// Problem per expert e (rows s_e .. s_e + n_e of the packed activations):
//   fwd   : y_e  = x_e  @ W_e        (W_e [K, N], or [N, K] with trans_b)
//   dgrad : dx_e = dy_e @ W_e^T      (W_e^T when trans_b)
//   wgrad : dW_e = x_e^T @ dy_e      (dy_e^T @ x_e when trans_b)
// All three are C[i, j] = sum_k A(i, k) B(k, j) with each operand either
// K-major (k contiguous) or MN-major (i or j contiguous). MFMA
// v_mfma_f32_32x32x16 wants, per lane, 8 consecutive k of one row (A) or one
// column (B), so LDS always holds both tiles as [row][k] (k contiguous,
// padded). K-major tiles are copied with 16-byte loads; MN-major tiles are
// loaded as 8x8 micro-tiles (eight 16-byte loads along the contiguous dim)
// and transposed in registers with byte permutes before the LDS store.
// FP8 e4m3 weights are decoded and multiplied by their 128x128 block scale
// while staging, giving exactly bf16(f32(q) * f32(scale)).
//
// Tile schedule: fwd/dgrad blocks walk (expert, m-tile, n-tile) slots whose
// count is only known on the device; every block derives its slot from the
// per-expert counts (a block-wide scan in LDS) and blocks past the last slot
// exit. Block ids are remapped so that consecutive slots run on the same XCD
// (sharing its L2), which keeps an expert's weights in one L2.
#include "common.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;

enum { MODE_FWD = 0, MODE_DGRAD = 1, MODE_WGRAD = 2 };

template <int ET>
struct Mma;
template <>
struct Mma<TT_BF16> {
  static __device__ __forceinline__ f32x16 run(const uint4& a, const uint4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t out(float f) { return f32_to_bf16(f); }
};
template <>
struct Mma<TT_F16> {
  static __device__ __forceinline__ f32x16 run(const uint4& a, const uint4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t out(float f) { return f32_to_f16(f); }
};

template <int BM_, int BN_, int BK_, int WGM_, int WGN_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_;
  static constexpr int NT = 64 * WGM * WGN;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int LDK = BK + 8;  // padded LDS row (elements)
  // K-major staging: 16-byte chunks per thread.
  static constexpr int KCH_A = BM * BK / 8 / NT;
  static constexpr int KCH_B = BN * BK / 8 / NT;
  // MN-major staging: 8x8 micro-tiles per thread.
  static constexpr int MT_A = (BM / 8) * (BK / 8) / NT;
  static constexpr int MT_B = (BN / 8) * (BK / 8) / NT;
  static_assert(BM % (32 * WGM) == 0 && BN % (32 * WGN) == 0, "wave tile");
  static_assert(BK % 16 == 0, "BK");
  static_assert(KCH_A * NT * 8 == BM * BK && KCH_B * NT * 8 == BN * BK, "k-major split");
  static_assert(MT_A * NT * 64 == BM * BK && MT_B * NT * 64 == BN * BK, "mn-major split");
};

// 8x8 transpose of 16-bit elements: in[r] holds row r (8 elements), out[c]
// holds column c.
__device__ __forceinline__ void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
  const uint32_t* s = reinterpret_cast<const uint32_t*>(in);
  uint32_t* d = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int w = c >> 1;  // source dword within each row
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      d[c * 4 + q] = __builtin_amdgcn_perm(s[(2 * q + 1) * 4 + w], s[(2 * q) * 4 + w], sel);
  }
}

// One e4m3fn byte -> fp32 (exact). Via the f16 bit pattern: e4m3 shares the
// 3-bit mantissa and its exponent bias differs by 8, so (byte & 0x7f) << 7
// reinterpreted as f16 equals |value| * 2^-8, subnormals included.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint16_t h = static_cast<uint16_t>(((b & 0x80u) << 8) | ((b & 0x7fu) << 7));
  const float v = f16_to_f32(h) * 256.0f;
  return ((b & 0x7fu) == 0x7fu) ? __builtin_nanf("") : v;
}

// Four e4m3 bytes of `w` times `scale`, rounded to bf16, packed in two dwords.
__device__ __forceinline__ uint2 dequant4(uint32_t w, float scale) {
  uint2 r;
  r.x = static_cast<uint32_t>(f32_to_bf16(e4m3_to_f32(w & 0xffu) * scale)) |
        (static_cast<uint32_t>(f32_to_bf16(e4m3_to_f32((w >> 8) & 0xffu) * scale)) << 16);
  r.y = static_cast<uint32_t>(f32_to_bf16(e4m3_to_f32((w >> 16) & 0xffu) * scale)) |
        (static_cast<uint32_t>(f32_to_bf16(e4m3_to_f32(w >> 24) * scale)) << 16);
  return r;
}

__device__ __forceinline__ int xcd_remap(int b, int nb) {
  const int q = nb / 8, r = nb % 8;
  const int xcd = b % 8, pos = b / 8;
  return xcd < r ? xcd * (q + 1) + pos : r * (q + 1) + (xcd - r) * q + pos;
}

// Block-wide exclusive scans over the E expert counts: row starts and
// m-tile starts. Writes E + 1 entries of each into LDS.
template <int NT>
__device__ void scan_counts(const int64_t* __restrict__ counts, int E, int BM,
                            int64_t* row_start, int* tile_start) {
  __shared__ int64_t wrow[NT / 64];
  __shared__ int wtile[NT / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (E + NT - 1) / NT;
  int64_t r = 0;
  int tl = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      const int64_t c = counts[e];
      r += c;
      tl += (int)((c + BM - 1) / BM);
    }
  }
  int64_t ri = r;
  int ti = tl;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t o = __shfl_up(ri, off, 64);
    const int ot = __shfl_up(ti, off, 64);
    if (lane >= off) {
      ri += o;
      ti += ot;
    }
  }
  if (lane == 63) {
    wrow[wave] = ri;
    wtile[wave] = ti;
  }
  __syncthreads();
  int64_t rb = 0;
  int tb = 0;
  for (int w = 0; w < wave; ++w) {
    rb += wrow[w];
    tb += wtile[w];
  }
  rb += ri - r;
  tb += ti - tl;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) {
      row_start[e] = rb;
      tile_start[e] = tb;
      const int64_t c = counts[e];
      rb += c;
      tb += (int)((c + BM - 1) / BM);
    }
  }
  if (tid == NT - 1) {
    row_start[E] = rb;
    tile_start[E] = tb;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <class C, int MODE, bool TRANS_B, bool FP8, int ET>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(1, 2))) void gmm_kernel(
    const char* __restrict__ p0, const char* __restrict__ p1, const char* __restrict__ scale,
    int scale_dt, char* __restrict__ out, int64_t M, int64_t K, int64_t N, int E,
    const int64_t* __restrict__ counts, int tiles_i, int tiles_j) {
  // Operand layouts for this mode.
  constexpr bool A_K = MODE != MODE_WGRAD;
  constexpr bool B_K = (MODE == MODE_FWD) ? TRANS_B : (MODE == MODE_DGRAD ? !TRANS_B : false);
  constexpr int ESZ = 2;

  extern __shared__ __align__(16) char smem[];
  uint16_t* lds_a = reinterpret_cast<uint16_t*>(smem);
  uint16_t* lds_b = lds_a + C::BM * C::LDK;
  int64_t* row_start = reinterpret_cast<int64_t*>(lds_b + C::BN * C::LDK);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);

  const int tid = threadIdx.x;
  const int lb = xcd_remap(blockIdx.x, gridDim.x);

  int e, it, jt;
  if constexpr (MODE == MODE_WGRAD) {
    scan_counts<C::NT>(counts, E, C::BM, row_start, tile_start);
    e = lb / (tiles_i * tiles_j);
    const int rem = lb % (tiles_i * tiles_j);
    it = rem / tiles_j;
    jt = rem % tiles_j;
    if (e >= E) return;
  } else {
    scan_counts<C::NT>(counts, E, C::BM, row_start, tile_start);
    const int slot = lb / tiles_j;
    jt = lb % tiles_j;
    if (slot >= tile_start[E]) return;
    // binary search: last e with tile_start[e] <= slot
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile_start[mid] <= slot) lo = mid; else hi = mid - 1;
    }
    e = lo;
    it = slot - tile_start[e];
  }
  const int64_t seg0 = row_start[e];
  const int64_t nrows = row_start[e + 1] - seg0;

  // Per-mode problem description.
  const char* abase;
  const char* bbase;
  int64_t lda, ldb, I, J, R;
  char* cbase;
  int64_t ldc;
  if constexpr (MODE == MODE_FWD) {
    abase = p0 + seg0 * K * ESZ; lda = K;
    I = nrows; J = N; R = K;
    if constexpr (FP8) { bbase = p1 + (int64_t)e * N * K; ldb = K; }
    else { bbase = p1 + (int64_t)e * K * N * ESZ; ldb = TRANS_B ? K : N; }
    cbase = out + seg0 * N * ESZ; ldc = N;
  } else if constexpr (MODE == MODE_DGRAD) {
    abase = p0 + seg0 * N * ESZ; lda = N;
    I = nrows; J = K; R = N;
    if constexpr (FP8) { bbase = p1 + (int64_t)e * N * K; ldb = K; }
    else { bbase = p1 + (int64_t)e * K * N * ESZ; ldb = TRANS_B ? K : N; }
    cbase = out + seg0 * K * ESZ; ldc = K;
  } else {
    R = nrows;
    if constexpr (!TRANS_B) {
      abase = p0 + seg0 * K * ESZ; lda = K;  // x
      bbase = p1 + seg0 * N * ESZ; ldb = N;  // dy
      I = K; J = N;
    } else {
      abase = p1 + seg0 * N * ESZ; lda = N;  // dy
      bbase = p0 + seg0 * K * ESZ; ldb = K;  // x
      I = N; J = K;
    }
    cbase = out + (int64_t)e * K * N * ESZ; ldc = J;
  }
  const int64_t i0 = (int64_t)it * C::BM, j0 = (int64_t)jt * C::BN;
  // Last loadable A row relative to the segment (fwd/dgrad).
  const int64_t a_clamp = M - 1 - seg0;
  const int64_t a_rows = (MODE == MODE_WGRAD) ? I : nrows;
  const int64_t b_clamp = B_K ? (J - 1) : -1;

  // FP8 block scales of this expert.
  const char* sbase = nullptr;
  int64_t sld = 0;
  if constexpr (FP8) {
    sld = (K + 127) / 128;
    sbase = scale + (int64_t)e * ((N + 127) / 128) * sld * (scale_dt == TT_F32 ? 4 : 2);
  }

  f32x16 acc[C::FM][C::FN];
#pragma unroll
  for (int mi = 0; mi < C::FM; ++mi)
#pragma unroll
    for (int ni = 0; ni < C::FN; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

  const int nkt = (int)((R + C::BK - 1) / C::BK);
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int lr = lane & 31, lg = lane >> 5;

  // Register-staged operands for the next k-tile.
  constexpr int CA = A_K ? C::KCH_A : C::MT_A;
  constexpr int CB = B_K ? C::KCH_B : C::MT_B;
  uint4 ra[A_K ? CA : CA * 8];
  uint4 rb[B_K ? CB : CB * 8];
  // FP8 operands keep 8 raw bytes per 8 elements (k-major) or per 8x8 tile row.
  uint2 rb8[B_K ? CB : CB * 8];

  auto load_a = [&](int kt) {
    const int64_t k0 = (int64_t)kt * C::BK;
    if constexpr (A_K) {
      constexpr int KC = C::BK / 8;
#pragma unroll
      for (int q = 0; q < CA; ++q) {
        const int c = tid + C::NT * q;
        const int r = c / KC, kc = c % KC;
        // Rows past the segment belong to later experts (or are clamped to
        // the last row); their products only reach rows that are not stored.
        int64_t gr = i0 + r;
        if (gr > a_clamp) gr = a_clamp;
        const int64_t gk = k0 + kc * 8;
        ra[q] = gk < R ? *reinterpret_cast<const uint4*>(abase + (gr * lda + gk) * ESZ)
                       : make_uint4(0, 0, 0, 0);
      }
    } else {
      constexpr int RG = C::BM / 8;
#pragma unroll
      for (int q = 0; q < CA; ++q) {
        const int m = tid + C::NT * q;
        const int rg = m % RG, kg = m / RG;
        const int64_t gr = i0 + rg * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int64_t gk = k0 + kg * 8 + kk;
          const bool ok = gr < a_rows && gk < R;
          ra[q * 8 + kk] = ok ? *reinterpret_cast<const uint4*>(abase + (gk * lda + gr) * ESZ)
                              : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };

  auto load_b = [&](int kt) {
    const int64_t k0 = (int64_t)kt * C::BK;
    if constexpr (B_K) {
      constexpr int KC = C::BK / 8;
#pragma unroll
      for (int q = 0; q < CB; ++q) {
        const int c = tid + C::NT * q;
        const int r = c / KC, kc = c % KC;
        int64_t gj = j0 + r;
        if (gj > b_clamp) gj = b_clamp;
        const int64_t gk = k0 + kc * 8;
        const bool ok = gk < R;
        if constexpr (FP8) {
          rb8[q] = ok ? *reinterpret_cast<const uint2*>(bbase + gj * ldb + gk) : make_uint2(0, 0);
        } else {
          rb[q] = ok ? *reinterpret_cast<const uint4*>(bbase + (gj * ldb + gk) * ESZ)
                     : make_uint4(0, 0, 0, 0);
        }
      }
    } else {
      constexpr int RG = C::BN / 8;
#pragma unroll
      for (int q = 0; q < CB; ++q) {
        const int m = tid + C::NT * q;
        const int rg = m % RG, kg = m / RG;
        const int64_t gj = j0 + rg * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int64_t gk = k0 + kg * 8 + kk;
          const bool ok = gj < J && gk < R;
          if constexpr (FP8) {
            rb8[q * 8 + kk] = ok ? *reinterpret_cast<const uint2*>(bbase + gk * ldb + gj)
                                 : make_uint2(0, 0);
          } else {
            rb[q * 8 + kk] = ok ? *reinterpret_cast<const uint4*>(bbase + (gk * ldb + gj) * ESZ)
                                : make_uint4(0, 0, 0, 0);
          }
        }
      }
    }
  };

  auto scale_at = [&](int64_t n_out, int64_t k_in) -> float {
    const int64_t si = (n_out >> 7) * sld + (k_in >> 7);
    return scale_dt == TT_F32 ? reinterpret_cast<const float*>(sbase)[si]
                              : bf16_to_f32(reinterpret_cast<const uint16_t*>(sbase)[si]);
  };

  auto store_a = [&]() {
    if constexpr (A_K) {
      constexpr int KC = C::BK / 8;
#pragma unroll
      for (int q = 0; q < CA; ++q) {
        const int c = tid + C::NT * q;
        const int r = c / KC, kc = c % KC;
        *reinterpret_cast<uint4*>(lds_a + r * C::LDK + kc * 8) = ra[q];
      }
    } else {
      constexpr int RG = C::BM / 8;
#pragma unroll
      for (int q = 0; q < CA; ++q) {
        const int m = tid + C::NT * q;
        const int rg = m % RG, kg = m / RG;
        uint4 in[8], t[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) in[kk] = ra[q * 8 + kk];
        transpose8x8(in, t);
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
          *reinterpret_cast<uint4*>(lds_a + (rg * 8 + rr) * C::LDK + kg * 8) = t[rr];
      }
    }
  };

  auto store_b = [&](int kt) {
    const int64_t k0 = (int64_t)kt * C::BK;
    if constexpr (B_K) {
      constexpr int KC = C::BK / 8;
#pragma unroll
      for (int q = 0; q < CB; ++q) {
        const int c = tid + C::NT * q;
        const int r = c / KC, kc = c % KC;
        uint4 val;
        if constexpr (FP8) {
          int64_t gj = j0 + r;
          if (gj > b_clamp) gj = b_clamp;
          const float s = scale_at(gj, k0 + kc * 8);  // weight [out = j][in = k]
          const uint2 lo = dequant4(rb8[q].x, s), hi = dequant4(rb8[q].y, s);
          val = make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else {
          val = rb[q];
        }
        *reinterpret_cast<uint4*>(lds_b + r * C::LDK + kc * 8) = val;
      }
    } else {
      constexpr int RG = C::BN / 8;
#pragma unroll
      for (int q = 0; q < CB; ++q) {
        const int m = tid + C::NT * q;
        const int rg = m % RG, kg = m / RG;
        uint4 in[8], t[8];
        if constexpr (FP8) {
          // weight [out = k][in = j]: the 8 rows are 8 consecutive k, one
          // 128-block in k and one in j (both 8-aligned).
          const int64_t jj = (j0 + rg * 8 < J) ? j0 + rg * 8 : J - 1;  // tiles past J
          const float s = scale_at(k0 + kg * 8, jj);
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) {
            const uint2 lo = dequant4(rb8[q * 8 + kk].x, s), hi = dequant4(rb8[q * 8 + kk].y, s);
            in[kk] = make_uint4(lo.x, lo.y, hi.x, hi.y);
          }
        } else {
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) in[kk] = rb[q * 8 + kk];
        }
        transpose8x8(in, t);
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
          *reinterpret_cast<uint4*>(lds_b + (rg * 8 + rr) * C::LDK + kg * 8) = t[rr];
      }
    }
  };

  if (nkt > 0) {
    load_a(0);
    load_b(0);
  }
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();
    store_a();
    store_b(kt);
    __syncthreads();
    if (kt + 1 < nkt) {
      load_a(kt + 1);
      load_b(kt + 1);
    }
#pragma unroll
    for (int s = 0; s < C::BK / 16; ++s) {
      uint4 fa[C::FM], fb[C::FN];
#pragma unroll
      for (int mi = 0; mi < C::FM; ++mi)
        fa[mi] = *reinterpret_cast<const uint4*>(lds_a + (wm * C::WTM + mi * 32 + lr) * C::LDK +
                                                 s * 16 + lg * 8);
#pragma unroll
      for (int ni = 0; ni < C::FN; ++ni)
        fb[ni] = *reinterpret_cast<const uint4*>(lds_b + (wn * C::WTN + ni * 32 + lr) * C::LDK +
                                                 s * 16 + lg * 8);
#pragma unroll
      for (int mi = 0; mi < C::FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < C::FN; ++ni) acc[mi][ni] = Mma<ET>::run(fa[mi], fb[ni], acc[mi][ni]);
    }
  }

  // Epilogue: D[i][j] of a 32x32 block sits in lane (j + 32 * ((i / 4) % 2)),
  // register (i % 4) + 4 * (i / 8).
  uint16_t* c16 = reinterpret_cast<uint16_t*>(cbase);
#pragma unroll
  for (int mi = 0; mi < C::FM; ++mi)
#pragma unroll
    for (int ni = 0; ni < C::FN; ++ni) {
      const int64_t gj = j0 + wn * C::WTN + ni * 32 + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t gi = i0 + wm * C::WTM + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
        if (gi < I && gj < J) c16[gi * ldc + gj] = Mma<ET>::out(acc[mi][ni][r]);
      }
    }
}

// ---------------------------------------------------------------------------
// fp32 path (toy shapes and fp32 models): 64x64 tiles, 4x4 outputs per thread.
// ---------------------------------------------------------------------------
template <int MODE, bool TRANS_B>
__global__ __launch_bounds__(256) void gmm_f32_kernel(const float* __restrict__ p0,
                                                      const float* __restrict__ p1,
                                                      float* __restrict__ out, int64_t M,
                                                      int64_t K, int64_t N, int E,
                                                      const int64_t* __restrict__ counts,
                                                      int tiles_i, int tiles_j) {
  constexpr int BT = 64, BKF = 16;
  __shared__ float sa[BKF][BT + 4];
  __shared__ float sb[BKF][BT + 4];
  extern __shared__ __align__(16) char smem[];
  int64_t* row_start = reinterpret_cast<int64_t*>(smem);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);
  scan_counts<256>(counts, E, BT, row_start, tile_start);
  int e, it, jt;
  if constexpr (MODE == MODE_WGRAD) {
    e = blockIdx.x / (tiles_i * tiles_j);
    const int rem = blockIdx.x % (tiles_i * tiles_j);
    it = rem / tiles_j;
    jt = rem % tiles_j;
    if (e >= E) return;
  } else {
    const int slot = blockIdx.x / tiles_j;
    jt = blockIdx.x % tiles_j;
    if (slot >= tile_start[E]) return;
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile_start[mid] <= slot) lo = mid; else hi = mid - 1;
    }
    e = lo;
    it = slot - tile_start[e];
  }
  const int64_t seg0 = row_start[e], nrows = row_start[e + 1] - seg0;
  // element accessors A(i, k), B(k, j)
  const float* A;
  const float* B;
  int64_t I, J, R;
  float* Cp;
  bool a_k, b_k;
  int64_t lda, ldb;
  if constexpr (MODE == MODE_FWD) {
    A = p0 + seg0 * K; lda = K; a_k = true;
    B = p1 + (int64_t)e * K * N; ldb = TRANS_B ? K : N; b_k = TRANS_B;
    I = nrows; J = N; R = K; Cp = out + seg0 * N;
  } else if constexpr (MODE == MODE_DGRAD) {
    A = p0 + seg0 * N; lda = N; a_k = true;
    B = p1 + (int64_t)e * K * N; ldb = TRANS_B ? K : N; b_k = !TRANS_B;
    I = nrows; J = K; R = N; Cp = out + seg0 * K;
  } else {
    R = nrows; a_k = false; b_k = false;
    if constexpr (!TRANS_B) { A = p0 + seg0 * K; lda = K; B = p1 + seg0 * N; ldb = N; I = K; J = N; }
    else { A = p1 + seg0 * N; lda = N; B = p0 + seg0 * K; ldb = K; I = N; J = K; }
    Cp = out + (int64_t)e * K * N;
  }
  const int64_t i0 = (int64_t)it * BT, j0 = (int64_t)jt * BT;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < R; k0 += BKF) {
    for (int q = threadIdx.x; q < BKF * BT; q += 256) {
      const int kk = q / BT, rr = q % BT;
      const int64_t gk = k0 + kk, gi = i0 + rr, gj = j0 + rr;
      sa[kk][rr] = (gk < R && gi < I) ? (a_k ? A[gi * lda + gk] : A[gk * lda + gi]) : 0.f;
      sb[kk][rr] = (gk < R && gj < J) ? (b_k ? B[gj * ldb + gk] : B[gk * ldb + gj]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BKF; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        av[u] = sa[kk][ty * 4 + u];
        bv[u] = sb[kk][tx * 4 + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] += av[u] * bv[v];
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t gi = i0 + ty * 4 + u, gj = j0 + tx * 4 + v;
      if (gi < I && gj < J) Cp[gi * J + gj] = acc[u][v];
    }
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

typedef Cfg<256, 256, 64, 2, 2> Big;

template <class C>
size_t lds_bytes(int E) {
  return (size_t)(C::BM + C::BN) * C::LDK * 2 + (size_t)(E + 1) * (sizeof(int64_t) + sizeof(int)) + 64;
}

template <class C, int MODE, bool TB, bool FP8, int ET>
int launch_mfma(const void* p0, const void* p1, const void* scale, int sdt, void* out, int64_t M,
                int64_t K, int64_t N, int E, const int64_t* counts, hipStream_t s) {
  int ti, tj;
  int64_t nblk;
  if (MODE == MODE_WGRAD) {
    const int64_t I = TB ? N : K, J = TB ? K : N;
    ti = (int)((I + C::BM - 1) / C::BM);
    tj = (int)((J + C::BN - 1) / C::BN);
    nblk = (int64_t)E * ti * tj;
  } else {
    const int64_t J = MODE == MODE_FWD ? N : K;
    tj = (int)((J + C::BN - 1) / C::BN);
    ti = 0;
    nblk = ((M + C::BM - 1) / C::BM + E) * (int64_t)tj;
  }
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  const size_t lds = lds_bytes<C>(E);
  TT_REQUIRE(lds <= 160 * 1024, "gmm: too many experts for the LDS tile schedule");
  // Dynamic LDS above 64 KiB must be allowed per kernel; raise the limit to
  // what this launch needs (kept per instantiation, only ever increased).
  static size_t lds_allowed = 64 * 1024;
  if (lds > lds_allowed) {
    const hipError_t err = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gmm_kernel<C, MODE, TB, FP8, ET>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) {
      (void)hipGetLastError();  // do not leave the error for the next launch check
      tt_set_error("gmm: hipFuncSetAttribute(%zu bytes): %s", lds, hipGetErrorString(err));
      return TT_ERR_HIP;
    }
    lds_allowed = lds;
  }
  hipLaunchKernelGGL((gmm_kernel<C, MODE, TB, FP8, ET>), dim3((unsigned)nblk), dim3(C::NT), lds, s,
                     static_cast<const char*>(p0), static_cast<const char*>(p1),
                     static_cast<const char*>(scale), sdt, static_cast<char*>(out), M, K, N, E,
                     counts, ti, tj);
  return tt_check_launch("gmm");
}

template <int MODE, bool TB>
int launch_f32(const void* p0, const void* p1, void* out, int64_t M, int64_t K, int64_t N, int E,
               const int64_t* counts, hipStream_t s) {
  constexpr int BT = 64;
  int ti, tj;
  int64_t nblk;
  if (MODE == MODE_WGRAD) {
    const int64_t I = TB ? N : K, J = TB ? K : N;
    ti = (int)((I + BT - 1) / BT);
    tj = (int)((J + BT - 1) / BT);
    nblk = (int64_t)E * ti * tj;
  } else {
    const int64_t J = MODE == MODE_FWD ? N : K;
    tj = (int)((J + BT - 1) / BT);
    ti = 0;
    nblk = ((M + BT - 1) / BT + E) * (int64_t)tj;
  }
  if (nblk == 0) return TT_OK;
  const size_t lds = (size_t)(E + 1) * (sizeof(int64_t) + sizeof(int)) + 64;
  hipLaunchKernelGGL((gmm_f32_kernel<MODE, TB>), dim3((unsigned)nblk), dim3(256), lds, s,
                     static_cast<const float*>(p0), static_cast<const float*>(p1),
                     static_cast<float*>(out), M, K, N, E, counts, ti, tj);
  return tt_check_launch("gmm_f32");
}

template <int MODE>
int dispatch(const void* p0, const void* p1, int dtype, int64_t m, int64_t k, int64_t n, int E,
             int tb, const int64_t* counts, void* out, void* stream) {
  TT_REQUIRE(m >= 0 && k >= 0 && n >= 0, "gmm: negative sizes");
  TT_REQUIRE(E >= 1 && E <= 4096, "gmm: num_experts must be in [1, 4096]");
  hipStream_t s = S(stream);
  if (dtype == TT_F32) {
    if (tb) return launch_f32<MODE, true>(p0, p1, out, m, k, n, E, counts, s);
    return launch_f32<MODE, false>(p0, p1, out, m, k, n, E, counts, s);
  }
  TT_REQUIRE(dtype == TT_BF16 || dtype == TT_F16, "gmm: unsupported dtype %d", dtype);
  TT_REQUIRE(k % 8 == 0 && n % 8 == 0, "gmm: K and N must be multiples of 8 (got %lld, %lld)",
             (long long)k, (long long)n);
  TT_REQUIRE(((reinterpret_cast<uintptr_t>(p0) | reinterpret_cast<uintptr_t>(p1) |
               reinterpret_cast<uintptr_t>(out)) & 15) == 0,
             "gmm: operands must be 16-byte aligned");
  if (dtype == TT_BF16) {
    if (tb) return launch_mfma<Big, MODE, true, false, TT_BF16>(p0, p1, nullptr, 0, out, m, k, n, E, counts, s);
    return launch_mfma<Big, MODE, false, false, TT_BF16>(p0, p1, nullptr, 0, out, m, k, n, E, counts, s);
  }
  if (tb) return launch_mfma<Big, MODE, true, false, TT_F16>(p0, p1, nullptr, 0, out, m, k, n, E, counts, s);
  return launch_mfma<Big, MODE, false, false, TT_F16>(p0, p1, nullptr, 0, out, m, k, n, E, counts, s);
}

}  // namespace

extern "C" int tt_gmm_fwd(const void* x, const void* w, int dtype, int64_t m, int64_t k,
                          int64_t n, int32_t num_experts, int32_t trans_b, const int64_t* counts,
                          void* y, void* stream) {
  return dispatch<MODE_FWD>(x, w, dtype, m, k, n, num_experts, trans_b, counts, y, stream);
}

extern "C" int tt_gmm_dgrad(const void* dy, const void* w, int dtype, int64_t m, int64_t k,
                            int64_t n, int32_t num_experts, int32_t trans_b,
                            const int64_t* counts, void* dx, void* stream) {
  return dispatch<MODE_DGRAD>(dy, w, dtype, m, k, n, num_experts, trans_b, counts, dx, stream);
}

extern "C" int tt_gmm_wgrad(const void* x, const void* dy, int dtype, int64_t m, int64_t k,
                            int64_t n, int32_t num_experts, int32_t trans_b,
                            const int64_t* counts, void* dw, void* stream) {
  return dispatch<MODE_WGRAD>(x, dy, dtype, m, k, n, num_experts, trans_b, counts, dw, stream);
}

static int fp8_checks(const void* a, const uint8_t* qw, const void* out, int sdt, int64_t m,
                      int64_t k, int64_t n, int E) {
  TT_REQUIRE(m >= 0 && k >= 0 && n >= 0, "gmm_fp8: negative sizes");
  TT_REQUIRE(E >= 1 && E <= 4096, "gmm_fp8: num_experts must be in [1, 4096]");
  TT_REQUIRE(sdt == TT_BF16 || sdt == TT_F32, "gmm_fp8: scales must be bf16 or f32");
  TT_REQUIRE(k % 16 == 0 && n % 16 == 0, "gmm_fp8: K and N must be multiples of 16");
  TT_REQUIRE(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(qw) |
               reinterpret_cast<uintptr_t>(out)) & 15) == 0,
             "gmm_fp8: operands must be 16-byte aligned");
  return TT_OK;
}

extern "C" int tt_gmm_fp8_fwd(const void* x, const uint8_t* qw, const void* scale,
                              int scale_dtype, int64_t m, int64_t k, int64_t n,
                              int32_t num_experts, const int64_t* counts, void* y, void* stream) {
  const int rc = fp8_checks(x, qw, y, scale_dtype, m, k, n, num_experts);
  if (rc != TT_OK) return rc;
  return launch_mfma<Big, MODE_FWD, true, true, TT_BF16>(x, qw, scale, scale_dtype, y, m, k, n,
                                                         num_experts, counts, S(stream));
}

extern "C" int tt_gmm_fp8_dgrad(const void* dy, const uint8_t* qw, const void* scale,
                                int scale_dtype, int64_t m, int64_t k, int64_t n,
                                int32_t num_experts, const int64_t* counts, void* dx,
                                void* stream) {
  const int rc = fp8_checks(dy, qw, dx, scale_dtype, m, k, n, num_experts);
  if (rc != TT_OK) return rc;
  return launch_mfma<Big, MODE_DGRAD, true, true, TT_BF16>(dy, qw, scale, scale_dtype, dx, m, k, n,
                                                           num_experts, counts, S(stream));
}
