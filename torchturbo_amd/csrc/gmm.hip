// Grouped GEMM over variable-length expert segments (gfx950 MFMA).
//
// Problem per expert e (rows s_e .. s_e + n_e of the packed activations):
//   fwd   : y_e  = x_e  @ W_e        (W_e [K, N], or [N, K] with trans_b)
//   dgrad : dx_e = dy_e @ W_e^T      (W_e^T when trans_b)
//   wgrad : dW_e = x_e^T @ dy_e      (dy_e^T @ x_e when trans_b)
// All three are C[i, j] = sum_k A(i, k) B(k, j) with each operand either
// K-major (k contiguous) or MN-major (i or j contiguous). v_mfma_f32_32x32x16
// takes, per lane, 8 consecutive k of one row (A) or one column (B).
//
// Two kernels share the tile schedule:
//
// * gmm_dma_kernel (bf16/f16): 256x256x32 block tiles, 8 waves of 128x64,
//   four LDS stages filled by direct global->LDS loads (global_load_lds,
//   16 bytes per lane, no register round trip), three k-tiles in flight.
//   K-major tiles are stored [row][k] with the 16-byte chunks of a row
//   XOR-swizzled, read with ds_read_b128. MN-major tiles are stored in their
//   natural [k][row] order (swizzled) and read with the gfx950 transposing
//   LDS load ds_read_b64_tr_b16, which hands each lane four consecutive k of
//   one column: no register transpose. Out-of-range chunks load from a zero
//   line, so no lane ever reads outside its operand.
// * gmm_reg_kernel: 256x256x64 tiles through registers and two LDS stages,
//   8x8 register transposes for MN-major operands. Used for FP8 weights: the
//   e4m3 bytes are decoded and multiplied by their 128x128 block scale while
//   staging, giving exactly bf16(f32(q) * f32(scale)).
//
// Tile schedule: fwd/dgrad blocks walk (expert, m-tile, n-tile) slots whose
// count is only known on the device; every block derives its slot from the
// per-expert counts (a block-wide scan in LDS) and blocks past the last slot
// exit. fwd/dgrad block ids are remapped so that consecutive slots (sharing an
// A panel and an expert's weights) run on one XCD and its L2. wgrad blocks
// take experts longest-first and are left in hardware round-robin order, so
// the tiles of a heavily loaded expert spread over all XCDs.
#include "common.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) char lds_char;

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

// What one block computes: C[i0 .., j0 ..] of expert e, with operand bases
// and leading dimensions (elements). Byte pointers; ESZ is the activation
// element size, WSZ the weight element size (1 for FP8).
struct TileDesc {
  const char* a;
  const char* b;
  char* c;
  int64_t lda, ldb, ldc;
  int64_t I, J, R;  // output rows / columns, reduction length
  int64_t i0, j0;   // tile origin
  int64_t seg0, nrows;
  int e;
};

template <int NT, int BM, int BN, int MODE, bool TRANS_B, int ESZ, int WSZ>
__device__ bool describe_tile(const char* p0, const char* p1, char* out, int64_t K, int64_t N,
                              int E, const int64_t* __restrict__ counts, int tiles_i, int tiles_j,
                              int64_t* row_start, int* tile_start, TileDesc& t) {
  scan_counts<NT>(counts, E, BM, row_start, tile_start);
  int e, it, jt;
  if constexpr (MODE == MODE_WGRAD) {
    // Experts are taken longest first (rank by row count, ties by id) so the
    // long reductions of heavily loaded experts start early.
    __shared__ int lpt_expert;
    const int lb = blockIdx.x;
    const int rank = lb / (tiles_i * tiles_j);
    const int rem = lb % (tiles_i * tiles_j);
    it = rem / tiles_j;
    jt = rem % tiles_j;
    if (rank >= E) return false;
    for (int x = threadIdx.x; x < E; x += NT) {
      const int64_t cx = row_start[x + 1] - row_start[x];
      int r = 0;
      for (int y = 0; y < E; ++y) {
        const int64_t cy = row_start[y + 1] - row_start[y];
        r += (cy > cx) || (cy == cx && y < x);
      }
      if (r == rank) lpt_expert = x;
    }
    __syncthreads();
    e = lpt_expert;
  } else {
    const int lb = xcd_remap(blockIdx.x, gridDim.x);
    const int slot = lb / tiles_j;
    jt = lb % tiles_j;
    if (slot >= tile_start[E]) return false;
    int lo = 0, hi = E - 1;  // last e with tile_start[e] <= slot
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile_start[mid] <= slot) lo = mid; else hi = mid - 1;
    }
    e = lo;
    it = slot - tile_start[e];
  }
  t.e = e;
  t.seg0 = row_start[e];
  t.nrows = row_start[e + 1] - t.seg0;
  if constexpr (MODE == MODE_FWD) {
    t.a = p0 + t.seg0 * K * ESZ; t.lda = K;
    t.b = p1 + (int64_t)e * K * N * WSZ; t.ldb = TRANS_B ? K : N;
    t.I = t.nrows; t.J = N; t.R = K;
    t.c = out + t.seg0 * N * ESZ; t.ldc = N;
  } else if constexpr (MODE == MODE_DGRAD) {
    t.a = p0 + t.seg0 * N * ESZ; t.lda = N;
    t.b = p1 + (int64_t)e * K * N * WSZ; t.ldb = TRANS_B ? K : N;
    t.I = t.nrows; t.J = K; t.R = N;
    t.c = out + t.seg0 * K * ESZ; t.ldc = K;
  } else {
    t.R = t.nrows;
    if constexpr (!TRANS_B) {
      t.a = p0 + t.seg0 * K * ESZ; t.lda = K;  // x
      t.b = p1 + t.seg0 * N * ESZ; t.ldb = N;  // dy
      t.I = K; t.J = N;
    } else {
      t.a = p1 + t.seg0 * N * ESZ; t.lda = N;  // dy
      t.b = p0 + t.seg0 * K * ESZ; t.ldb = K;  // x
      t.I = N; t.J = K;
    }
    t.c = out + (int64_t)e * K * N * ESZ; t.ldc = t.J;
  }
  t.i0 = (int64_t)it * BM;
  t.j0 = (int64_t)jt * BN;
  return true;
}

// Operand layouts per mode: A is K-major except in wgrad; B is K-major for
// fwd with trans_b and dgrad without.
template <int MODE, bool TRANS_B>
struct Layout {
  static constexpr bool A_K = MODE != MODE_WGRAD;
  static constexpr bool B_K = (MODE == MODE_FWD) ? TRANS_B : (MODE == MODE_DGRAD ? !TRANS_B : false);
};

// Epilogue for a 128x64 wave tile of 32x32 MFMA blocks. D[i][j] of a block
// sits in lane (j + 32 * ((i / 4) % 2)), register (i % 4) + 4 * (i / 8).
// Neighbouring lanes swap one value so each lane stores two adjacent
// columns of one row with a single 4-byte store.
template <int ET, int FM, int FN>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[FM][FN], const TileDesc& t,
                                           int64_t ri, int64_t cj, int lane) {
  const int lr = lane & 31, lg = lane >> 5;
  const bool odd = lr & 1;
#pragma unroll
  for (int mi = 0; mi < FM; ++mi)
#pragma unroll
    for (int ni = 0; ni < FN; ++ni) {
      const int64_t gj = cj + ni * 32 + (lr & ~1);
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float send = odd ? acc[mi][ni][r] : acc[mi][ni][r + 1];
        const float recv = __shfl_xor(send, 1, TT_WAVE);
        const float lo = odd ? recv : acc[mi][ni][r];
        const float hi = odd ? acc[mi][ni][r + 1] : recv;
        const int64_t gi = ri + mi * 32 + 8 * (r >> 2) + 4 * lg + (r & 3) + (odd ? 1 : 0);
        if (gi < t.I && gj < t.J) {
          const uint32_t packed = static_cast<uint32_t>(Mma<ET>::out(lo)) |
                                  (static_cast<uint32_t>(Mma<ET>::out(hi)) << 16);
          *reinterpret_cast<uint32_t*>(t.c + (gi * t.ldc + gj) * 2) = packed;
        }
      }
    }
}

// ===========================================================================
// DMA-pipelined kernel (bf16 / f16).
// ===========================================================================
constexpr int DM_BM = 256, DM_BN = 256, DM_BK = 32, DM_ST = 4, DM_NT = 512;
constexpr int DM_TILE = DM_BM * DM_BK * 2;  // bytes of one operand tile (16 KiB)
constexpr int DM_STAGE = 2 * DM_TILE;       // A tile then B tile

// Source of out-of-range chunks: one zero line (read only).
__device__ __align__(64) uint4 g_zero_line[4];

// One 16-byte global->LDS load per lane into lds_dst + 16 * lane (lds_dst is
// wave-uniform; it goes to M0). Issued as inline assembly so the compiler
// does not drain every outstanding DMA before each LDS read: completion of a
// stage is awaited explicitly (TT_WAIT_VMCNT) before the barrier that
// publishes it. Vector-memory results return in order, so the compiler's own
// vmcnt waits for its loads stay sufficient. Nothing else in these kernels
// uses M0.
__device__ __forceinline__ void dma16(const void* src, char* lds_dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char*)lds_dst)));  // LDS offset
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(m0), "v"(src)
               : "memory");
}

// Where each lane's four 16-byte DMA chunks of a k-tile come from. Built
// once per block; per k-tile only the byte step and the k bound change, so a
// single small set of registers stays live in the main loop.
struct DmaPlan {
  const char* src[4];  // chunk addresses at k-tile 0
  int koff[4];         // k of the chunk relative to the k-tile start
  bool ok[4];          // row / column inside the operand
  int64_t step;        // bytes from one k-tile to the next
  int dst;             // byte offset of the operand tile within a stage
};

// K-major tile: rows [row0, row0 + 256) x k [k0, k0 + 32); element (r, k)
// at base + (r * ld + k) * 2. LDS row r occupies 64 bytes; its 16-byte chunk
// c (k = 8c .. 8c + 7) sits in slot c ^ ((r >> 2) & 3), which keeps the
// MFMA-operand reads (32 rows, one chunk) free of bank conflicts. A wave
// writes 1 KiB (16 rows) per instruction, lane l to slot l & 3 of row l >> 2.
__device__ __forceinline__ DmaPlan plan_kmajor(const char* base, int64_t ld, int64_t row0,
                                               int64_t rows_valid, int dst, int wv, int lane) {
  DmaPlan p;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int u = wv * 4 + q;
    const int r = 16 * u + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    const int64_t gr = row0 + r;
    p.ok[q] = gr < rows_valid;
    p.koff[q] = 8 * c;
    p.src[q] = base + (gr * ld + 8 * c) * 2;
  }
  p.step = (int64_t)DM_BK * 2;
  p.dst = dst;
  return p;
}

// MN-major tile: k rows [k0, k0 + 32) x columns [col0, col0 + 256); element
// (k, c) at base + (k * ld + c) * 2. LDS k-row kr occupies 512 bytes; its
// 16-byte chunk c (columns 8c .. 8c + 7) sits in slot c ^ (4 * (kr & 3)). A
// wave writes two k-rows per instruction.
__device__ __forceinline__ DmaPlan plan_mnmajor(const char* base, int64_t ld, int64_t col0,
                                                int64_t cols_valid, int dst, int wv, int lane) {
  DmaPlan p;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int u = wv * 4 + q;
    const int kr = 2 * u + (lane >> 5);
    const int c = (lane & 31) ^ (4 * (kr & 3));
    const int64_t gc = col0 + 8 * c;
    p.ok[q] = gc < cols_valid;
    p.koff[q] = kr;
    p.src[q] = base + (kr * ld + gc) * 2;
  }
  p.step = (int64_t)DM_BK * ld * 2;
  p.dst = dst;
  return p;
}

// Issue the lane's four chunks of k-tile kt into a stage; chunks outside the
// operand (or past the reduction length) load from the zero line.
__device__ __forceinline__ void dma_issue(const DmaPlan& p, char* stage, int kt, int64_t kvalid,
                                          int wv) {
  const int64_t k0 = (int64_t)kt * DM_BK;
  const int64_t off = (int64_t)kt * p.step;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const void* src = (p.ok[q] && k0 + p.koff[q] < kvalid)
                          ? static_cast<const void*>(p.src[q] + off)
                          : static_cast<const void*>(g_zero_line);
    dma16(src, stage + p.dst + (wv * 4 + q) * 1024);
  }
}

// MFMA operand from a K-major tile: rows r0 .. r0 + 31, k-step s (16 k).
__device__ __forceinline__ uint4 frag_k(const char* tile, int r0, int s, int lane) {
  const int r = r0 + (lane & 31);
  const int c = 2 * s + (lane >> 5);
  return *reinterpret_cast<const uint4*>(tile + r * 64 + ((c ^ ((r >> 2) & 3)) << 4));
}

// MFMA operand from an MN-major tile: columns c0 .. c0 + 31, k-step s. Two
// transposing reads: within each 16-lane group, source lane i reads k-row
// k + i / 4, columns col + 4 * (i % 4) .. + 3, and lane i receives column
// col + i at the four k-rows.
__device__ __forceinline__ uint4 frag_mn(const char* tile, int c0, int s, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int col = c0 + 16 * (g & 1) + 4 * (i & 3);
  const int chunk = col >> 3, within = (col & 7) * 2;
  uint4 out;
  uint32_t* o = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kr = 16 * s + 8 * (g >> 1) + 4 * h + (i >> 2);
    const char* p = tile + kr * 512 + ((chunk ^ (4 * (kr & 3))) << 4) + within;
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p);  // generic -> LDS
    const uint2 w = __builtin_bit_cast(uint2, v);
    o[2 * h] = w.x;
    o[2 * h + 1] = w.y;
  }
  return out;
}

// s_waitcnt with only vmcnt = n (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14,
// expcnt and lgkmcnt left at their maxima).
#define TT_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 0xF) | ((((n) >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8))

template <int MODE, bool TRANS_B, int ET>
__global__ __launch_bounds__(DM_NT) void gmm_dma_kernel(const char* __restrict__ p0,
                                                        const char* __restrict__ p1,
                                                        char* __restrict__ out, int64_t M,
                                                        int64_t K, int64_t N, int E,
                                                        const int64_t* __restrict__ counts,
                                                        int tiles_i, int tiles_j) {
  typedef Layout<MODE, TRANS_B> Lay;
  constexpr int WGN = 4, WTM = 128, WTN = 64, FM = WTM / 32, FN = WTN / 32;
  // One static LDS array per stage and a k-loop unrolled by the stage count:
  // every DMA and every read then names a fixed array, so the compiler can
  // tell that loads in flight to one stage do not alias reads of another and
  // need not drain the DMA queue before reading.
  __shared__ __align__(16) char stage0[DM_STAGE];
  __shared__ __align__(16) char stage1[DM_STAGE];
  __shared__ __align__(16) char stage2[DM_STAGE];
  __shared__ __align__(16) char stage3[DM_STAGE];
  extern __shared__ __align__(16) char smem[];  // expert schedule
  int64_t* row_start = reinterpret_cast<int64_t*>(smem);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);

  TileDesc t;
  if (!describe_tile<DM_NT, DM_BM, DM_BN, MODE, TRANS_B, 2, 2>(p0, p1, out, K, N, E, counts,
                                                                 tiles_i, tiles_j, row_start,
                                                                 tile_start, t))
    return;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WGN, wn = wave % WGN;
  const bool a_role = wave < 4;  // waves 0-3 stream A, waves 4-7 stream B
  const int wv = wave & 3;
  const int nkt = (int)((t.R + DM_BK - 1) / DM_BK);
  // A rows past the segment (fwd/dgrad) read as zeros.
  const int64_t a_rows = Lay::A_K ? t.nrows : t.I;

  DmaPlan plan;
  if (a_role) {
    plan = Lay::A_K ? plan_kmajor(t.a, t.lda, t.i0, a_rows, 0, wv, lane)
                    : plan_mnmajor(t.a, t.lda, t.i0, t.I, 0, wv, lane);
  } else {
    plan = Lay::B_K ? plan_kmajor(t.b, t.ldb, t.j0, t.J, DM_TILE, wv, lane)
                    : plan_mnmajor(t.b, t.ldb, t.j0, t.J, DM_TILE, wv, lane);
  }
  auto issue = [&](char* stg, int kt) { dma_issue(plan, stg, kt, t.R, wv); };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int mi = 0; mi < FM; ++mi)
#pragma unroll
    for (int ni = 0; ni < FN; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

  // The operand reads of both k-steps of the tile are issued before its
  // MFMAs, so the second step's LDS latency hides under the first step's
  // MFMAs (the compiler alone loads each fragment just before its use).
  constexpr int KS = DM_BK / 16;
  static_assert(KS == 2, "two k-steps per tile");
  auto load_frags = [&](const char* stg, int s, uint4 (&fa)[FM], uint4 (&fb)[FN]) {
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
      fa[mi] = Lay::A_K ? frag_k(stg, wm * WTM + mi * 32, s, lane)
                        : frag_mn(stg, wm * WTM + mi * 32, s, lane);
#pragma unroll
    for (int ni = 0; ni < FN; ++ni)
      fb[ni] = Lay::B_K ? frag_k(stg + DM_TILE, wn * WTN + ni * 32, s, lane)
                        : frag_mn(stg + DM_TILE, wn * WTN + ni * 32, s, lane);
  };
  auto mfmas = [&](const uint4 (&fa)[FM], const uint4 (&fb)[FN]) {
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
      for (int ni = 0; ni < FN; ++ni) acc[mi][ni] = Mma<ET>::run(fa[mi], fb[ni], acc[mi][ni]);
  };
  auto compute = [&](const char* stg) {
    uint4 fa0[FM], fb0[FN], fa1[FM], fb1[FN];
    load_frags(stg, 0, fa0, fb0);
    load_frags(stg, 1, fa1, fb1);
    mfmas(fa0, fb0);
    mfmas(fa1, fb1);
  };

  // Pipeline: tiles kt+1 .. kt+3 are in flight while tile kt is multiplied.
  // Each wave waits for its own loads of tile kt (vmcnt), then the barrier
  // makes every wave's loads visible and retires all reads of tile kt-1,
  // whose stage then receives tile kt+3. One barrier per k-tile.
  auto step = [&](int kt, char* cur, char* refill) {
    const int last = (kt + DM_ST - 2 < nkt - 1) ? kt + DM_ST - 2 : nkt - 1;
    const int ahead = last - kt;  // tiles issued after kt: 0, 1 or 2
    if (ahead >= 2) TT_WAIT_VMCNT(8);
    else if (ahead == 1) TT_WAIT_VMCNT(4);
    else TT_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    if (kt + DM_ST - 1 < nkt) issue(refill, kt + DM_ST - 1);
    compute(cur);
  };
  if (nkt > 0) issue(stage0, 0);
  if (nkt > 1) issue(stage1, 1);
  if (nkt > 2) issue(stage2, 2);
  for (int kt = 0; kt < nkt; kt += DM_ST) {
    step(kt, stage0, stage3);
    if (kt + 1 < nkt) step(kt + 1, stage1, stage0);
    if (kt + 2 < nkt) step(kt + 2, stage2, stage1);
    if (kt + 3 < nkt) step(kt + 3, stage3, stage2);
  }
  store_tile<ET, FM, FN>(acc, t, t.i0 + wm * WTM, t.j0 + wn * WTN, lane);
}

// ===========================================================================
// Register-staged kernel (FP8 weights).
// ===========================================================================
constexpr int RG_BM = 256, RG_BN = 256, RG_BK = 64, RG_NT = 512;
constexpr int RG_LDK = RG_BK + 8;                 // padded LDS row (elements)
constexpr int RG_STAGE = (RG_BM + RG_BN) * RG_LDK;  // elements of one stage

template <int MODE, bool TRANS_B, bool FP8, int ET>
__global__ __launch_bounds__(RG_NT) void gmm_reg_kernel(
    const char* __restrict__ p0, const char* __restrict__ p1, const char* __restrict__ scale,
    int scale_dt, char* __restrict__ out, int64_t M, int64_t K, int64_t N, int E,
    const int64_t* __restrict__ counts, int tiles_i, int tiles_j) {
  typedef Layout<MODE, TRANS_B> Lay;
  constexpr bool A_K = Lay::A_K, B_K = Lay::B_K;
  constexpr int ESZ = 2;
  constexpr int WGN = 4, WTM = 128, WTN = 64, FM = WTM / 32, FN = WTN / 32;

  extern __shared__ __align__(16) char smem[];
  uint16_t* lds = reinterpret_cast<uint16_t*>(smem);
  int64_t* row_start = reinterpret_cast<int64_t*>(lds + 2 * RG_STAGE);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);

  TileDesc t;
  if (!describe_tile<RG_NT, RG_BM, RG_BN, MODE, TRANS_B, ESZ, FP8 ? 1 : 2>(
          p0, p1, out, K, N, E, counts, tiles_i, tiles_j, row_start, tile_start, t))
    return;
  const char* abase = t.a;
  const char* bbase = t.b;
  const int64_t lda = t.lda, ldb = t.ldb, I = t.I, J = t.J, R = t.R, i0 = t.i0, j0 = t.j0;
  // Last loadable A row relative to the segment (fwd/dgrad).
  const int64_t a_clamp = M - 1 - t.seg0;
  const int64_t a_rows = (MODE == MODE_WGRAD) ? I : t.nrows;
  const int64_t b_clamp = B_K ? (J - 1) : -1;

  // FP8 block scales of this expert.
  const char* sbase = nullptr;
  int64_t sld = 0;
  if constexpr (FP8) {
    sld = (K + 127) / 128;
    sbase = scale + (int64_t)t.e * ((N + 127) / 128) * sld * (scale_dt == TT_F32 ? 4 : 2);
  }

  f32x16 acc[FM][FN];
#pragma unroll
  for (int mi = 0; mi < FM; ++mi)
#pragma unroll
    for (int ni = 0; ni < FN; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

  const int tid = threadIdx.x;
  const int nkt = (int)((R + RG_BK - 1) / RG_BK);
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WGN, wn = wave % WGN;
  const int lr = lane & 31, lg = lane >> 5;

  // Staging: the first half of the block moves the A tile, the second half
  // the B tile (wave-uniform split); each thread holds eight 16-byte slots:
  // eight K-major chunks or one 8x8 MN-major micro-tile.
  constexpr int SH = RG_NT / 2;
  static_assert(RG_BM * RG_BK / 8 == 8 * SH && RG_BN * RG_BK / 8 == 8 * SH, "staging split");
  const bool stage_a = tid < SH;
  const int st = stage_a ? tid : tid - SH;
  constexpr int KC = RG_BK / 8;
  uint4 rs[8];
  uint2 rs8[8];  // raw e4m3 bytes of the B tile (FP8 weights)

  auto scale_at = [&](int64_t n_out, int64_t k_in) -> float {
    const int64_t si = (n_out >> 7) * sld + (k_in >> 7);
    return scale_dt == TT_F32 ? reinterpret_cast<const float*>(sbase)[si]
                              : bf16_to_f32(reinterpret_cast<const uint16_t*>(sbase)[si]);
  };

  auto load_stage = [&](int kt) {
    const int64_t k0 = (int64_t)kt * RG_BK;
    if (stage_a) {
      if constexpr (A_K) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int c = st + SH * q;
          const int r = c / KC, kc = c % KC;
          // Rows past the segment belong to later experts (or are clamped to
          // the last row); their products only reach rows that are not stored.
          int64_t gr = i0 + r;
          if (gr > a_clamp) gr = a_clamp;
          const int64_t gk = k0 + kc * 8;
          rs[q] = gk < R ? *reinterpret_cast<const uint4*>(abase + (gr * lda + gk) * ESZ)
                         : make_uint4(0, 0, 0, 0);
        }
      } else {
        const int kg = st % KC, rg = st / KC;  // lanes walk k: conflict-free LDS rows
        const int64_t gr = i0 + rg * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int64_t gk = k0 + kg * 8 + kk;
          const bool ok = gr < a_rows && gk < R;
          rs[kk] = ok ? *reinterpret_cast<const uint4*>(abase + (gk * lda + gr) * ESZ)
                      : make_uint4(0, 0, 0, 0);
        }
      }
    } else {
      if constexpr (B_K) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int c = st + SH * q;
          const int r = c / KC, kc = c % KC;
          int64_t gj = j0 + r;
          if (gj > b_clamp) gj = b_clamp;
          const int64_t gk = k0 + kc * 8;
          const bool ok = gk < R;
          if constexpr (FP8)
            rs8[q] = ok ? *reinterpret_cast<const uint2*>(bbase + gj * ldb + gk) : make_uint2(0, 0);
          else
            rs[q] = ok ? *reinterpret_cast<const uint4*>(bbase + (gj * ldb + gk) * ESZ)
                       : make_uint4(0, 0, 0, 0);
        }
      } else {
        const int kg = st % KC, rg = st / KC;
        const int64_t gj = j0 + rg * 8;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int64_t gk = k0 + kg * 8 + kk;
          const bool ok = gj < J && gk < R;
          if constexpr (FP8)
            rs8[kk] = ok ? *reinterpret_cast<const uint2*>(bbase + gk * ldb + gj) : make_uint2(0, 0);
          else
            rs[kk] = ok ? *reinterpret_cast<const uint4*>(bbase + (gk * ldb + gj) * ESZ)
                        : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };

  auto store_stage = [&](int kt, uint16_t* stage) {
    const int64_t k0 = (int64_t)kt * RG_BK;
    if (stage_a) {
      if constexpr (A_K) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int c = st + SH * q;
          const int r = c / KC, kc = c % KC;
          *reinterpret_cast<uint4*>(stage + r * RG_LDK + kc * 8) = rs[q];
        }
      } else {
        const int kg = st % KC, rg = st / KC;
        uint4 tr[8];
        transpose8x8(rs, tr);
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
          *reinterpret_cast<uint4*>(stage + (rg * 8 + rr) * RG_LDK + kg * 8) = tr[rr];
      }
    } else {
      uint16_t* lb = stage + RG_BM * RG_LDK;
      if constexpr (B_K) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int c = st + SH * q;
          const int r = c / KC, kc = c % KC;
          uint4 val;
          if constexpr (FP8) {
            int64_t gj = j0 + r;
            if (gj > b_clamp) gj = b_clamp;
            const float s = scale_at(gj, k0 + kc * 8);  // weight [out = j][in = k]
            const uint2 lo = dequant4(rs8[q].x, s), hi = dequant4(rs8[q].y, s);
            val = make_uint4(lo.x, lo.y, hi.x, hi.y);
          } else {
            val = rs[q];
          }
          *reinterpret_cast<uint4*>(lb + r * RG_LDK + kc * 8) = val;
        }
      } else {
        const int kg = st % KC, rg = st / KC;
        uint4 tr[8];
        if constexpr (FP8) {
          // weight [out = k][in = j]: the 8 rows are 8 consecutive k inside one
          // 128-block of k, and 8 consecutive j inside one 128-block of j.
          const int64_t jj = (j0 + rg * 8 < J) ? j0 + rg * 8 : J - 1;  // tiles past J
          const float s = scale_at(k0 + kg * 8, jj);
          uint4 in[8];
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) {
            const uint2 lo = dequant4(rs8[kk].x, s), hi = dequant4(rs8[kk].y, s);
            in[kk] = make_uint4(lo.x, lo.y, hi.x, hi.y);
          }
          transpose8x8(in, tr);
        } else {
          transpose8x8(rs, tr);
        }
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
          *reinterpret_cast<uint4*>(lb + (rg * 8 + rr) * RG_LDK + kg * 8) = tr[rr];
      }
    }
  };

  // Pipeline: global loads of tile k+1 are in flight while tile k is
  // multiplied out of one LDS stage; they land in the other stage afterwards.
  // One barrier per k-tile.
  if (nkt > 0) {
    load_stage(0);
    store_stage(0, lds);
  }
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const uint16_t* cur = lds + (kt & 1) * RG_STAGE;
    if (kt + 1 < nkt) load_stage(kt + 1);
    const uint16_t* la = cur + (wm * WTM + lr) * RG_LDK + lg * 8;
    const uint16_t* lbp = cur + RG_BM * RG_LDK + (wn * WTN + lr) * RG_LDK + lg * 8;
#pragma unroll
    for (int s = 0; s < RG_BK / 16; ++s) {
      uint4 fa[FM], fb[FN];
#pragma unroll
      for (int mi = 0; mi < FM; ++mi)
        fa[mi] = *reinterpret_cast<const uint4*>(la + mi * 32 * RG_LDK + s * 16);
#pragma unroll
      for (int ni = 0; ni < FN; ++ni)
        fb[ni] = *reinterpret_cast<const uint4*>(lbp + ni * 32 * RG_LDK + s * 16);
#pragma unroll
      for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni) acc[mi][ni] = Mma<ET>::run(fa[mi], fb[ni], acc[mi][ni]);
    }
    if (kt + 1 < nkt) store_stage(kt + 1, lds + ((kt + 1) & 1) * RG_STAGE);
    __syncthreads();
  }
  store_tile<ET, FM, FN>(acc, t, i0 + wm * WTM, j0 + wn * WTN, lane);
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
  TileDesc t;
  if (!describe_tile<256, BT, BT, MODE, TRANS_B, 4, 4>(
          reinterpret_cast<const char*>(p0), reinterpret_cast<const char*>(p1),
          reinterpret_cast<char*>(out), K, N, E, counts, tiles_i, tiles_j, row_start,
          tile_start, t))
    return;
  typedef Layout<MODE, TRANS_B> Lay;
  const float* A = reinterpret_cast<const float*>(t.a);
  const float* B = reinterpret_cast<const float*>(t.b);
  float* Cp = reinterpret_cast<float*>(t.c);
  const int64_t I = t.I, J = t.J, R = t.R, lda = t.lda, ldb = t.ldb;
  const int64_t i0 = t.i0, j0 = t.j0;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < R; k0 += BKF) {
    for (int q = threadIdx.x; q < BKF * BT; q += 256) {
      const int kk = q / BT, rr = q % BT;
      const int64_t gk = k0 + kk, gi = i0 + rr, gj = j0 + rr;
      sa[kk][rr] = (gk < R && gi < I) ? (Lay::A_K ? A[gi * lda + gk] : A[gk * lda + gi]) : 0.f;
      sb[kk][rr] = (gk < R && gj < J) ? (Lay::B_K ? B[gj * ldb + gk] : B[gk * ldb + gj]) : 0.f;
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
      if (gi < I && gj < J) Cp[gi * t.ldc + gj] = acc[u][v];
    }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

size_t schedule_bytes(int E) { return (size_t)(E + 1) * (sizeof(int64_t) + sizeof(int)) + 64; }

// Grid of a grouped launch: fwd/dgrad use an upper bound on the number of
// (m-tile, n-tile) slots (each expert adds at most one partial m-tile);
// wgrad uses E x tiles_i x tiles_j.
int64_t grid_blocks(int MODE, bool tb, int64_t M, int64_t K, int64_t N, int E, int BM, int BN,
                    int& ti, int& tj) {
  if (MODE == MODE_WGRAD) {
    const int64_t I = tb ? N : K, J = tb ? K : N;
    ti = (int)((I + BM - 1) / BM);
    tj = (int)((J + BN - 1) / BN);
    return (int64_t)E * ti * tj;
  }
  const int64_t J = MODE == MODE_FWD ? N : K;
  tj = (int)((J + BN - 1) / BN);
  ti = 0;
  return ((M + BM - 1) / BM + E) * (int64_t)tj;
}

// Dynamic LDS above 64 KiB must be allowed per kernel; raise the limit to
// what a launch needs (kept per kernel, only ever increased).
template <typename F>
int allow_lds(F* kernel, size_t lds, size_t& allowed) {
  if (lds <= allowed) return TT_OK;
  const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (err != hipSuccess) {
    (void)hipGetLastError();  // do not leave the error for the next launch check
    tt_set_error("gmm: hipFuncSetAttribute(%zu bytes): %s", lds, hipGetErrorString(err));
    return TT_ERR_HIP;
  }
  allowed = lds;
  return TT_OK;
}

template <int MODE, bool TB, int ET>
int launch_dma(const void* p0, const void* p1, void* out, int64_t M, int64_t K, int64_t N, int E,
               const int64_t* counts, hipStream_t s) {
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE, TB, M, K, N, E, DM_BM, DM_BN, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  const size_t lds = schedule_bytes(E);  // the stages are static LDS
  TT_REQUIRE(lds + (size_t)DM_ST * DM_STAGE <= 160 * 1024,
             "gmm: too many experts for the LDS tile schedule");
  static size_t allowed = 64 * 1024;
  const int rc = allow_lds(&gmm_dma_kernel<MODE, TB, ET>, lds, allowed);
  if (rc != TT_OK) return rc;
  hipLaunchKernelGGL((gmm_dma_kernel<MODE, TB, ET>), dim3((unsigned)nblk), dim3(DM_NT), lds, s,
                     static_cast<const char*>(p0), static_cast<const char*>(p1),
                     static_cast<char*>(out), M, K, N, E, counts, ti, tj);
  return tt_check_launch("gmm");
}

template <int MODE, bool TB, bool FP8, int ET>
int launch_reg(const void* p0, const void* p1, const void* scale, int sdt, void* out, int64_t M,
               int64_t K, int64_t N, int E, const int64_t* counts, hipStream_t s) {
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE, TB, M, K, N, E, RG_BM, RG_BN, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  const size_t lds = (size_t)2 * RG_STAGE * 2 + schedule_bytes(E);
  TT_REQUIRE(lds <= 160 * 1024, "gmm: too many experts for the LDS tile schedule");
  static size_t allowed = 64 * 1024;
  const int rc = allow_lds(&gmm_reg_kernel<MODE, TB, FP8, ET>, lds, allowed);
  if (rc != TT_OK) return rc;
  hipLaunchKernelGGL((gmm_reg_kernel<MODE, TB, FP8, ET>), dim3((unsigned)nblk), dim3(RG_NT), lds,
                     s, static_cast<const char*>(p0), static_cast<const char*>(p1),
                     static_cast<const char*>(scale), sdt, static_cast<char*>(out), M, K, N, E,
                     counts, ti, tj);
  return tt_check_launch("gmm");
}

template <int MODE, bool TB>
int launch_f32(const void* p0, const void* p1, void* out, int64_t M, int64_t K, int64_t N, int E,
               const int64_t* counts, hipStream_t s) {
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE, TB, M, K, N, E, 64, 64, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  hipLaunchKernelGGL((gmm_f32_kernel<MODE, TB>), dim3((unsigned)nblk), dim3(256),
                     schedule_bytes(E), s, static_cast<const float*>(p0),
                     static_cast<const float*>(p1), static_cast<float*>(out), M, K, N, E, counts,
                     ti, tj);
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
    if (tb) return launch_dma<MODE, true, TT_BF16>(p0, p1, out, m, k, n, E, counts, s);
    return launch_dma<MODE, false, TT_BF16>(p0, p1, out, m, k, n, E, counts, s);
  }
  if (tb) return launch_dma<MODE, true, TT_F16>(p0, p1, out, m, k, n, E, counts, s);
  return launch_dma<MODE, false, TT_F16>(p0, p1, out, m, k, n, E, counts, s);
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
  return launch_reg<MODE_FWD, true, true, TT_BF16>(x, qw, scale, scale_dtype, y, m, k, n,
                                                   num_experts, counts, S(stream));
}

extern "C" int tt_gmm_fp8_dgrad(const void* dy, const uint8_t* qw, const void* scale,
                                int scale_dtype, int64_t m, int64_t k, int64_t n,
                                int32_t num_experts, const int64_t* counts, void* dx,
                                void* stream) {
  const int rc = fp8_checks(dy, qw, dx, scale_dtype, m, k, n, num_experts);
  if (rc != TT_OK) return rc;
  return launch_reg<MODE_DGRAD, true, true, TT_BF16>(dy, qw, scale, scale_dtype, dx, m, k, n,
                                                     num_experts, counts, S(stream));
}
