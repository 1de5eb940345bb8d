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
// The kernels share the tile schedule:
//
// * gmm_mfma_kernel (bf16/f16): 256x256x32 block tiles, 4 waves of 128x128
//   (one wave per SIMD, 256 accumulator registers). Operands stream into
//   four LDS stages with buffer loads that write LDS directly (16 bytes per
//   lane, no register round trip); three k-tiles are in flight. Each buffer
//   resource spans exactly its operand, so the hardware returns zeros past
//   an expert's rows or reduction length and no lane reads outside its
//   operand. K-major tiles are read with XOR-swizzled ds_read_b128;
//   MN-major tiles keep their natural [k][row] order and are read with the
//   gfx950 transposing load ds_read_b64_tr_b16 (no register transpose).
//   MFMAs, fragment reads of the next k-step and DMA issue are interleaved
//   one per slot; a chunk's offset is fixed and the k-tile's advance lives in
//   the buffer resource (scalar registers), so a load needs no vector
//   instruction. With rows gathered through a row map, every wave loads a
//   quarter of both operand tiles and turns its rows into offsets after the
//   k-tile barrier. The epilogue converts to 16 bits in hardware and stores
//   through LDS as full 256-byte rows. Serves wgrad with long expert
//   reductions over fewer than 512 output tiles per expert (its three
//   k-tiles in flight stream two activation operands fastest), the gathering
//   weight gradients, and short fwd/dgrad reductions.
// * gmm_p64_kernel (bf16/f16 fwd/dgrad with a reduction longer than 64, and
//   wgrad with few rows per expert): persistent, one block per CU; fwd/dgrad
//   blocks walk a strided list of output tiles (launches of at most four
//   n-tiles and twelve rounds: a cost-sorted list within each XCD, computed
//   at start by lpt_schedule), wgrad blocks take tickets
//   from per-XCD queues over the experts' tiles, longest expert first, and
//   claim the next ticket two or three k-tiles before the current tile ends.
//   256x256x64 tiles through two 64 KiB LDS stages, so K-major rows are
//   whole 128-byte lines. Loads as in gmm_mfma_kernel: fixed chunk offsets,
//   the k-tile in the buffer resource. The k-tiles of consecutive tiles form one stream
//   (the next tile's first loads overlap the current tile's last k-tile and
//   epilogue); the epilogue stages through a private 4 KiB of LDS per wave
//   and stores with buffer stores whose resource ends at the expert's last
//   row. fwd/dgrad tiles of at most 64 rows leave that stream for a
//   weight-streaming pipeline of their own (two weight k-tiles in flight
//   while a third is multiplied), and an expert of at most 64 rows takes its
//   tiles two per schedule slot.
// * gmm_q8_kernel (fwd/dgrad with e4m3 weights and 128x128 block scales,
//   every launch whose reduction is longer than one 64-deep k-tile):
//   persistent like gmm_p64_kernel, 128x512x64 tiles (the four waves share
//   the tile's 128 rows and take 128 columns each, so an expert's rows are
//   padded to 128 only). The weight tile stays e4m3 in LDS; each wave reads
//   its own fragments as e4m3 bytes (plain 8-byte reads of K-major rows in
//   fwd, the transposing 8-bit read ds_read_b64_tr_b8 of N-major rows in
//   dgrad) and dequantises them in registers between its MFMAs, exactly
//   bf16(f32(q) * f32(scale)) with one scale per wave and k-tile. Loads use
//   fixed chunk offsets with the k-tile in the buffer resource, so the
//   k-loop's vector instructions are almost all the dequantisation.
// * gmm_fp8_kernel (FP8 fwd/dgrad with a reduction of one k-tile): the
//   256x256x32 tiles of gmm_mfma_kernel; the weight tile arrives in LDS as
//   e4m3 bytes and each wave decodes its own rows in hardware, multiplies by
//   the block scale and rounds to bf16 into one of three rotating bf16
//   tiles, overlapped with the previous k-tile's MFMAs.
// * gmm_f32_kernel (fp32 operands): 64x64 tiles on fp32 MFMAs
//   (v_mfma_f32_32x32x2_f32).
//
// Tile schedule: fwd/dgrad blocks walk (expert, m-tile, n-tile) slots (two
// n-tiles per slot for an expert of at most 64 rows) whose
// count is only known on the device; every block derives its slot from the
// per-expert counts (a block-wide scan in LDS) and blocks past the last slot
// exit. fwd/dgrad block ids are remapped so that consecutive slots (sharing an
// A panel and an expert's weights) run on one XCD and its L2. wgrad blocks
// take experts longest-first; each expert's tiles go to one pair of XCDs
// (one-tile-per-block kernel, whose blocks read the launch's ranking from
// wgrad_rank_kernel) or to every XCD as rectangles (persistent kernel), so
// that the XCDs share its activation panels in L2.
#include "common.h"

#include <atomic>
#include <type_traits>

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
};
template <>
struct Mma<TT_F16> {
  static __device__ __forceinline__ f32x16 run(const uint4& a, const uint4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ int xcd_remap(int b, int nb) {
  const int q = nb / 8, r = nb % 8;
  const int xcd = b % 8, pos = b / 8;
  return xcd < r ? xcd * (q + 1) + pos : r * (q + 1) + (xcd - r) * q + pos;
}

// Block-wide exclusive scans over the E expert counts: row starts and
// m-tile starts. Writes E + 1 entries of each into LDS.
// tile_start[e]: prefix of the experts' m-tile counts ceil(rows / BM); with
// thin_tj > 0 (the persistent fwd / dgrad kernel), of their schedule slots
// instead: ceil(rows / BM) * thin_tj tiles, or for an expert of at most 64
// rows ceil(thin_tj / 2) slots of two thin tiles each.
template <int NT>
__device__ void scan_counts(const int64_t* __restrict__ counts, int E, int BM,
                            int64_t* row_start, int* tile_start, int thin_tj = 0) {
  auto slots = [&](int64_t c) -> int {
    if (thin_tj == 0) return (int)((c + BM - 1) / BM);
    if (c > 0 && c <= 64) return (thin_tj + 1) / 2;
    return (int)((c + BM - 1) / BM) * thin_tj;
  };
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
      tl += slots(c);
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
      tb += slots(c);
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
  int nsub;  // persistent fwd / dgrad: thin tiles in this slot (0: one ordinary tile)
};

// A block-uniform 64-bit value (read from LDS) into scalar registers.
__device__ __forceinline__ int64_t rfl64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Weight-gradient tiles of one block per tile (gmm_mfma_kernel): each
// expert's output tiles go to one pair of XCDs, half of its tile grid to
// each, so an XCD's blocks re-read an expert's activation panels from L2
// instead of all eight XCDs reading them from memory (per expert, half the
// panels that the eight-XCD rectangles read: Qwen fc1 20 instead of 40, fc2
// 14 instead of 32; 14 and 11 are the minimum). Returns how the grid splits:
// 1 along its rows (tile rows i), 2 along its columns, 0 when neither count
// is even (then every XCD takes a rectangle of every expert).
__host__ __device__ inline int wgrad_pair_split(int tiles_i, int tiles_j) {
  const bool ei = tiles_i % 2 == 0, ej = tiles_j % 2 == 0;
  if (ei && (!ej || tiles_i / 2 + tiles_j <= tiles_i + tiles_j / 2)) return 1;
  return ej ? 2 : 0;
}

// Weight-gradient launches own one of WQ_SLOTS slots of per-process device
// state (slots rotate between launches): the persistent kernel's ticket
// counters, or the one-tile-per-block kernel's expert ranking.
constexpr int WQ_SLOTS = 64;

// Expert ranking of a one-tile-per-block weight-gradient launch, computed once
// per launch by wgrad_rank_kernel on the launch stream: entry r of the slot is
// the expert of rank r, longest first (row count descending, ties by id), with
// its first row and row count. Without it every block would scan the counts
// and rank all experts itself, about 9.5k cycles per block against 4.5-4.8k
// for a median k-loop of Qwen3-30B-A3B's gathered weight gradients (stamped
// per block: 12.6 % of the CUs' time).
struct WgradRank {
  int64_t seg0;
  int32_t nrows;
  int32_t e;
};
constexpr int WR_MAX_E = 4096;
__device__ WgradRank g_wgrad_rank[WQ_SLOTS * WR_MAX_E];

// One thread per expert (grid ceil(E / 256)); every block reads all the
// counts into LDS and each thread makes one pass over them: its rank (the
// experts ahead of it) and its first row (the rows of the experts before it).
// Counts sum to at most M < 2^31 rows (the launchers' 32-bit offset limits),
// so they compare as int; the first row is summed in 64 bits.
__global__ __launch_bounds__(256) void wgrad_rank_kernel(const int64_t* __restrict__ counts, int E,
                                                         int slot) {
  __shared__ int cnt[WR_MAX_E];
  for (int y = threadIdx.x; y < E; y += 256) cnt[y] = (int)counts[y];
  __syncthreads();
  const int x = blockIdx.x * 256 + threadIdx.x;
  if (x >= E) return;
  const int cx = cnt[x];
  int r = 0;
  int64_t start = 0;
#pragma unroll 8
  for (int y = 0; y < E; ++y) {
    const int cy = cnt[y];
    r += (cy > cx) | ((cy == cx) & (y < x));
    start += y < x ? cy : 0;
  }
  g_wgrad_rank[slot * WR_MAX_E + r] = WgradRank{start, cx, x};
}

// PAIRS: weight-gradient tiles on XCD pairs (wgrad_pair_split); the launch
// must then size the grid as 8 ceil(E / 8) x tiles_i x tiles_j.
// RSLOT (weight gradients): slot of the launch's expert ranking
// (wgrad_rank_kernel), or -1 to scan and rank in the block.
template <int NT, int BM, int BN, int MODE, bool TRANS_B, int ESZ, int WSZ, bool PAIRS = false>
__device__ bool describe_tile(const char* p0, const char* p1, char* out, int64_t K, int64_t N,
                              int E, const int64_t* __restrict__ counts, int tiles_i, int tiles_j,
                              int64_t* row_start, int* tile_start, TileDesc& t, int rslot = -1) {
  const bool ranked = MODE == MODE_WGRAD && rslot >= 0;
  if (!ranked) scan_counts<NT>(counts, E, BM, row_start, tile_start);
  int e, it, jt;
  int64_t seg0 = 0, nrows = 0;
  if constexpr (MODE == MODE_WGRAD) {
    // Experts are taken longest first (rank by row count, ties by id) so the
    // long reductions of heavily loaded experts start early.
    __shared__ int lpt_expert;
    const int lb = blockIdx.x;
    const int per = tiles_i * tiles_j;
    int rank = lb / per;
    const int rem = lb % per;
    const int split = PAIRS ? wgrad_pair_split(tiles_i, tiles_j) : 0;
    // Block b runs on XCD b % 8. XCD pair p = (b % 8) / 2 takes the experts of
    // ranks 8m + p and 8m + 7 - p (longest first, a snake over the four
    // pairs, so the pairs' loads even out), and XCD 2p + h the half h of each
    // one's tile grid, in row order: the pair's blocks of one expert run
    // together and share its panels in their XCD's L2. The grid holds
    // 8 ceil(E / 8) x per blocks; ranks past the last expert exit.
    int h = 0, w = 0, c = 0;
    if (split != 0) {
      const int x = lb % 8, j = lb / 8, pr = x >> 1, hf = x & 1;
      const int half = per / 2;
      const int k = j / half, t = j % half;
      rank = 8 * (k >> 1) + ((k & 1) ? 7 - pr : pr);
      if (split == 1) {
        it = hf * (tiles_i / 2) + t / tiles_j;
        jt = t % tiles_j;
      } else {
        it = t / (tiles_j / 2);
        jt = hf * (tiles_j / 2) + t % (tiles_j / 2);
      }
    } else if (per % 8 == 0) {
      int best = 1 << 30;
      for (int a = 1; a <= 8; a <<= 1) {
        const int cc = 8 / a;
        if (tiles_i % a || tiles_j % cc) continue;
        const int hh = tiles_i / a, ww = tiles_j / cc;
        if (hh + ww < best) { best = hh + ww; h = hh; w = ww; c = cc; }
      }
    }
    if (split != 0) {
      // (it, jt) set above
    } else if (h > 0) {
      const int x = rem % 8, j = rem / 8;
      it = (x / c) * h + j / w;
      jt = (x % c) * w + j % w;
    } else {
      it = rem / tiles_j;
      jt = rem % tiles_j;
    }
    if (rank >= E) return false;
    if (ranked) {
      // One scalar load: the ranking was written by the kernel before this
      // one on the launch stream.
      const WgradRank w = g_wgrad_rank[rslot * WR_MAX_E + rank];
      e = w.e;
      seg0 = w.seg0;
      nrows = w.nrows;
    } else {
      // Rank of every expert, its comparisons split over NT / E threads per
      // expert and summed with LDS atomics; int32 counts after the schedule.
      int* cnt = tile_start + E + 1;
      int* rnk = cnt + E;
      for (int x = threadIdx.x; x < E; x += NT) {
        cnt[x] = (int)(row_start[x + 1] - row_start[x]);
        rnk[x] = 0;
      }
      __syncthreads();
      const int parts = E >= NT ? 1 : NT / E;
      for (int idx = threadIdx.x; idx < E * parts; idx += NT) {
        const int x = idx % E, part = idx / E;
        const int y0 = part * E / parts, y1 = (part + 1) * E / parts;
        const int cx = cnt[x];
        int r = 0;
#pragma unroll 8
        for (int y = y0; y < y1; ++y) {
          const int cy = cnt[y];
          r += (cy > cx) | ((cy == cx) & (y < x));
        }
        atomicAdd(&rnk[x], r);
      }
      __syncthreads();
      for (int x = threadIdx.x; x < E; x += NT)
        if (rnk[x] == rank) lpt_expert = x;
      __syncthreads();
      e = lpt_expert;
      seg0 = row_start[e];
      nrows = row_start[e + 1] - seg0;
    }
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
    seg0 = row_start[e];
    nrows = row_start[e + 1] - seg0;
  }
  // Block-uniform (some of it was read from LDS): scalar registers, so that
  // resources and loop bounds derived from it stay scalar.
  t.e = __builtin_amdgcn_readfirstlane(e);
  t.seg0 = rfl64(seg0);
  t.nrows = rfl64(nrows);
  it = __builtin_amdgcn_readfirstlane(it);
  jt = __builtin_amdgcn_readfirstlane(jt);
  e = t.e;
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

// ===========================================================================
// MFMA kernel (bf16 / f16): 256x256x32 block tiles, 4 waves of 128x128.
// ===========================================================================
constexpr int DM_BM = 256, DM_BN = 256, DM_BK = 32, DM_ST = 4, DM_NT = 256;
constexpr int DM_TILE = DM_BM * DM_BK * 2;  // bytes of one operand tile (16 KiB)
constexpr int DM_STAGE = 2 * DM_TILE;       // A tile then B tile
constexpr uint32_t DM_OOB = 0xFFFFFFF0u;    // buffer offset past any resource
// Gathered A rows: the offset of a row past an expert's end, past any gathered
// source (sources are smaller than 2 GiB) with room for the chunk and k-tile
// offsets added to it.
constexpr uint32_t GA_NOROW = 0x80000000u;

typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

// Buffer resource over [base, base + bytes): offsets at or past `bytes` read
// as zeros. Word 3 is the raw 32-bit data format of the gfx9 family.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, int64_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t n = bytes <= 0 ? 0u : (bytes < (int64_t)DM_OOB ? (uint32_t)bytes : DM_OOB);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(b >> 32) & 0xFFFFu));
  r.z = __builtin_amdgcn_readfirstlane((int)n);
  r.w = 0x00020000;
  return r;
}

// One 16-byte buffer load per lane straight into LDS at lds_addr + 16 * lane
// (lds_addr is wave-uniform and goes to M0). Inline assembly, so that the
// compiler does not drain outstanding loads before every LDS read:
// completion of a stage is awaited explicitly (TT_WAIT_VMCNT) before the
// barrier that publishes it. Nothing else in these kernels uses M0.
// The resource moved `adv` bytes along (scalar arithmetic): an offset from
// the new base is in range exactly when the same offset plus adv was before,
// and nothing is once adv passes the end.
__device__ __forceinline__ i32x4 advance_rsrc(i32x4 r, uint32_t adv) {
  const uint64_t b = (((uint64_t)(uint32_t)r.y << 32) | (uint32_t)r.x) + adv;  // stride 0
  i32x4 o;
  o.x = (int)(uint32_t)b;
  o.y = (int)(uint32_t)(b >> 32);
  // records - adv, or 0 on a borrow (SCC), in scalar instructions: the
  // compiler's saturating subtract is a vector one.
  uint32_t n;
  asm("s_sub_u32 %0, %1, %2\n\ts_cselect_b32 %0, 0, %0" : "=s"(n) : "s"(r.z), "s"(adv) : "scc");
  o.z = (int)n;
  o.w = r.w;
  return o;
}

__device__ __forceinline__ void dma16(uint32_t voff, i32x4 rsrc, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory");
}

// One dword per lane into LDS at m0 + 4 lane (row indices of a gathered operand).
__device__ __forceinline__ void dma4(uint32_t voff, i32x4 rsrc, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr_of(lds_char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// s_waitcnt with only vmcnt = n (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14,
// expcnt and lgkmcnt left at their maxima).
#define TT_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 0xF) | ((((n) >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8))

// LDS operand tiles.
// * K-major (k contiguous in memory): LDS row r (64 bytes = 32 k) holds tile
//   row r, its 16-byte chunk c in slot c ^ ((r >> 2) & 3). An MFMA operand
//   (32 rows, 8 k per lane) is one conflict-free ds_read_b128.
// * MN-major (rows/columns contiguous in memory): LDS k-row kr (512 bytes)
//   holds 256 columns, chunk c (columns 8c .. 8c + 7) in slot
//   c ^ (4 * (kr & 3)). An operand is two gfx950 transposing reads
//   (ds_read_b64_tr_b16): within each 16-lane group source lane i reads
//   k-row k + i / 4, columns col + 4 * (i % 4) .. + 3, and lane i receives
//   column col + i at the four k-rows. No register transpose is needed.
// DMA: a wave fills 1 KiB per instruction, lane l at +16 l: K-major rows
// 16u .. 16u + 15 (lane l -> row 16u + l / 4, slot l & 3); MN-major k-rows
// 2u, 2u + 1 (lane l -> k-row 2u + l / 32, slot l & 31).

// Fragment read offsets within an operand tile. K-major: rows r0 + lane % 32
// at k-step s (further 32-row blocks add 2048 bytes).
__device__ __forceinline__ uint32_t fragk_base(int r0, int s, int lane) {
  const int r = r0 + (lane & 31);
  const int c = 2 * s + (lane >> 5);
  return (uint32_t)(r * 64 + ((c ^ ((r >> 2) & 3)) << 4));
}
// MN-major: columns c0 .. c0 + 31; the second read is at +2048 and k-step s
// adds 8192.
__device__ __forceinline__ uint32_t fragmn_base(int c0, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int col = c0 + 16 * (g & 1) + 4 * (i & 3);
  const int kr = 8 * (g >> 1) + (i >> 2);
  return (uint32_t)(kr * 512 + (((col >> 3) ^ (4 * (kr & 3))) << 4) + (col & 7) * 2);
}

__device__ __forceinline__ uint4 read_k(lds_char* tile, uint32_t off) {
  return __builtin_bit_cast(uint4, *reinterpret_cast<const lds_u32x4*>(tile + off));
}
__device__ __forceinline__ uint4 read_mn(lds_char* tile, uint32_t off) {
  const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + off));
  const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + off + 2048));
  const uint2 w0 = __builtin_bit_cast(uint2, v0), w1 = __builtin_bit_cast(uint2, v1);
  return uint4{w0.x, w0.y, w1.x, w1.y};
}

// Four fp32 values -> four 16-bit values (hardware round to nearest even).
template <int ET>
__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
  if constexpr (ET == TT_BF16) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
    const bf16x2 lo = {(__bf16)a, (__bf16)b}, hi = {(__bf16)c, (__bf16)d};
    return uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
  } else {
    typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
    const f16x2 lo = {(_Float16)a, (_Float16)b}, hi = {(_Float16)c, (_Float16)d};
    return uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
  }
}

// Epilogue through LDS. The accumulators hold C^T blocks (the MFMA operands
// are swapped): block (mi, ni) register 4g + e of lane l is
// C[ri + 32 mi + l % 32][cj + 32 ni + 8 g + 4 (l / 32) + e]. Each wave writes
// its 128x128 tile row-major into its own 32 KiB of LDS (16-byte chunks
// XOR-swizzled by row), then stores four full 256-byte rows per instruction.
// Column chunks never straddle the edge (J % 8 == 0).
template <int ET>
__device__ __forceinline__ void store_wave_tile(const f32x16 (&acc)[4][4], const TileDesc& t,
                                                int64_t ri, int64_t cj, int lane,
                                                lds_char* region) {
  const int r_l = lane & 31, h = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = 32 * mi + r_l;
        const int chunk = 4 * ni + g;
        const uint2 v = pack4<ET>(acc[mi][ni][4 * g], acc[mi][ni][4 * g + 1],
                                  acc[mi][ni][4 * g + 2], acc[mi][ni][4 * g + 3]);
        *reinterpret_cast<lds_u32x2*>(region + r * 256 + ((chunk ^ (r & 15)) << 4) + 8 * h) =
            u32x2{v.x, v.y};
      }
  // Row segments leave through a buffer resource that ends at the expert's
  // last row (stores past it are dropped; columns past the output width get
  // an offset past the resource), eight reads ahead of their stores, with
  // the streaming cache policy (the output does not stay in L2).
  const int64_t rows = t.I - ri;
  const int64_t obytes = rows > 0 ? rows * t.ldc * 2 - cj * 2 : 0;
  const uint32_t nrec = obytes < (int64_t)DM_OOB ? (uint32_t)obytes : DM_OOB;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(t.c + (ri * t.ldc + cj) * 2), (short)0, (int)nrec, 0x00020000);
  const int c = lane & 15;
  const bool col_ok = cj + 8 * c < t.J;
  const uint32_t row_bytes = (uint32_t)(t.ldc * 2);
#pragma unroll
  for (int q0 = 0; q0 < 32; q0 += 8) {
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * (q0 + j) + (lane >> 4);
      v[j] = read_k(region, (uint32_t)(r * 256 + ((c ^ (r & 15)) << 4)));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * (q0 + j) + (lane >> 4);
      const uint32_t off = col_ok ? (uint32_t)r * row_bytes + (uint32_t)(16 * c) : DM_OOB;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[j]), rs, (int)off, 0, 2);
    }
  }
}

// One block computes a 256x256 tile of one expert; wave w owns the 128x128
// quarter (w / 2, w % 2). Operands stream through four LDS stages (32 KiB
// each: A tile, B tile) with buffer loads straight into LDS; waves 0-1 load
// A, waves 2-3 load B, 8 chunks of 16 bytes per lane per k-tile. Each buffer
// resource covers exactly the operand (this expert's activation rows, or
// this expert's weights), so rows past the expert's end and reduction rows
// past its length read as zeros in hardware; column overhang inside the
// operand only feeds output rows/columns that are never stored. The
// reduction tail of a K-major operand whose length is not a multiple of 32
// (KMASK) is masked explicitly.
// GX (weight gradients): 0, or 1 / 2 when the rows of x (p0) / dy (p1) are
// gathered, row r of the expert-packed order being row grow[r] of that
// operand's source ([gsrc_rows, K] / [gsrc_rows, N]).
template <int MODE, bool TRANS_B, int ET, bool KMASK, int GX = 0>
__global__ __launch_bounds__(DM_NT) void gmm_mfma_kernel(const char* __restrict__ p0,
                                                         const char* __restrict__ p1,
                                                         char* __restrict__ out, int64_t M,
                                                         int64_t K, int64_t N, int E,
                                                         const int64_t* __restrict__ counts,
                                                         int tiles_i, int tiles_j,
                                                         const int32_t* __restrict__ grow,
                                                         int64_t gsrc_rows, int rslot) {
  typedef Layout<MODE, TRANS_B> Lay;
  constexpr int WT = 128, FM = 4, FN = 4;
  constexpr bool GATH = GX != 0;
  static_assert(!GATH || (MODE == MODE_WGRAD && !KMASK), "gathered rows: weight gradients only");
  // Gathered operand: per wave, two groups of eight k-tiles of source row
  // indices, 64 each (lane i of a group: k-tile i / 8, k-row
  // 8 wave + 2 (i % 4) + i / 4 % 2, so a lane's four rows of a k-tile are one
  // 16-byte read).
  __shared__ __align__(16) int gidx[GATH ? 4 * 2 * 64 : 4];
  // One static LDS array per stage and a k-loop unrolled by the stage count:
  // every address is then a compile-time stage base plus a lane offset.
  __shared__ __align__(16) char stage0[DM_STAGE];
  __shared__ __align__(16) char stage1[DM_STAGE];
  __shared__ __align__(16) char stage2[DM_STAGE];
  __shared__ __align__(16) char stage3[DM_STAGE];
  extern __shared__ __align__(16) char smem[];  // expert schedule
  int64_t* row_start = reinterpret_cast<int64_t*>(smem);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);

  TileDesc t;
  if (!describe_tile<DM_NT, DM_BM, DM_BN, MODE, TRANS_B, 2, 2, true>(p0, p1, out, K, N, E, counts,
                                                                 tiles_i, tiles_j, row_start,
                                                                 tile_start, t, rslot))
    return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nkt = (int)((t.R + DM_BK - 1) / DM_BK);
  // Operand tiles are loaded in 16 units each (K-major: 16 rows; MN-major: a
  // pair of k-rows), one 1 KiB chunk per unit. Packed operands: waves 0-1
  // load A and waves 2-3 B, eight units each (chunk q: unit 8 (wave % 2) + q).
  // With a gathered operand every wave loads a quarter of each tile instead
  // (chunks q = 0..3: units 4 wave + q of A, q = 4..7: the same units of B),
  // so the gathered operand's offset work falls on all four waves alike: with
  // A on two waves and B on the other two, the two loading the gathered
  // operand were about 250 cycles per k-tile slower and the others waited for
  // them (gathered Qwen weight gradients 2-3 % faster this way); packed
  // operands keep one operand per wave (2 % faster on Qwen's fc1).
  // GO: the gathered operand (0 A, 1 B; x is A unless TRANS_B).
  constexpr int GO = ((GX == 1) != TRANS_B) ? 0 : 1;
  auto chunk_op = [&](int q) { return GATH ? (q >> 2) : (wave < 2 ? 0 : 1); };
  auto chunk_unit = [&](int q) { return GATH ? 4 * wave + (q & 3) : 8 * (wave & 1) + q; };
  const int64_t ldo[2] = {t.lda, t.ldb};
  const int64_t orow[2] = {t.i0, t.j0};
  const int64_t abytes = (Lay::A_K ? t.nrows : t.R) * t.lda * 2;
  const int64_t bbytes = (MODE == MODE_WGRAD) ? t.R * t.ldb * 2 : K * N * 2;
  // Per operand: its buffer resource (the whole source for the gathered one)
  // and the per-k-tile advance; per chunk: the byte offset at k-tile 0.
  i32x4 rs[2];
  rs[0] = (GATH && GO == 0) ? make_rsrc(GX == 1 ? p0 : p1, gsrc_rows * t.lda * 2)
                            : make_rsrc(t.a, abytes);
  rs[1] = (GATH && GO == 1) ? make_rsrc(GX == 1 ? p0 : p1, gsrc_rows * t.ldb * 2)
                            : make_rsrc(t.b, bbytes);
  uint32_t kst[2];
  kst[0] = Lay::A_K ? (uint32_t)(DM_BK * 2) : (uint32_t)(DM_BK * t.lda * 2);
  kst[1] = Lay::B_K ? (uint32_t)(DM_BK * 2) : (uint32_t)(DM_BK * t.ldb * 2);
  uint32_t voff[8];
  int kof[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int op = chunk_op(q), u = chunk_unit(q);
    const int64_t ld = ldo[op];
    if (op == 0 ? Lay::A_K : Lay::B_K) {
      const int c = (lane & 3) ^ ((lane >> 4) & 3);  // (row >> 2) & 3 == (lane >> 4) & 3
      const int64_t r = orow[op] + 16 * u + (lane >> 2);
      voff[q] = (uint32_t)((r * ld + 8 * c) * 2);
      kof[q] = 8 * c;
    } else {
      const int kr = 2 * u + (lane >> 5);
      const int c = (lane & 31) ^ (4 * (kr & 3));
      voff[q] = (uint32_t)((kr * ld + orow[op] + 8 * c) * 2);
      kof[q] = kr;
    }
  }
  const int kvalid = (int)t.R;

  // Gathered operand: the k-tile's source rows come through the LDS index
  // ring (a group of eight k-tiles per dword DMA, issued five k-tiles ahead
  // of its first use so the pipeline's waits cover it). A step reads the rows
  // of the k-tile it will load at the end of its first half, so the LDS reads
  // are in flight across the wait and barrier, and turns them into offsets
  // after the barrier (reading them where the loads go out, or just before
  // them, was 4-16 % slower): each chunk's offset is its source row's plus
  // the lane's column chunk (two, by k-row parity). Reduction rows past the
  // expert's end read as zeros.
  // gof: the chunks' offsets; fixed (the k-tile's advance is in the resource)
  // except for the gathered operand's chunks, set per k-tile.
  uint32_t grow_v[4], gof[8], gcol[2];
#pragma unroll
  for (int q = 0; q < 8; ++q) gof[q] = voff[q];
  const uint32_t ld2 = (uint32_t)(ldo[GO] * 2);
  const i32x4 irsrc = make_rsrc(grow, GATH ? M * 4 : 0);
  if constexpr (GATH) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int c = (lane & 31) ^ (4 * ((2 * p + (lane >> 5)) & 3));
      gcol[p] = (uint32_t)((orow[GO] + 8 * c) * 2);
    }
  }
  auto issue_idx = [&](int grp) {
    const int j = lane >> 3, h = (lane >> 2) & 1, q = lane & 3;
    const int64_t row = (int64_t)(8 * grp + j) * DM_BK + 8 * wave + 2 * q + h;
    dma4((uint32_t)((t.seg0 + row) * 4), irsrc,
         lds_addr_of((lds_char*)gidx) + (uint32_t)((wave * 2 + (grp & 1)) * 256));
  };
  const uint32_t gsrc = (uint32_t)gsrc_rows;
  // An entry outside [0, gsrc_rows) (a negative one reads as a large
  // unsigned value) becomes gsrc_rows: its offset lies past the source's
  // resource, so it reads a row of zeros (the launch bounds
  // (gsrc_rows + 1) * ld * 2 below 4 GiB, so the offset does not wrap, and
  // gsrc_rows and ld * 2 below 2^24, so the product takes the 24-bit
  // multiply-add). Only an expert's last k-tile has rows past its end.
  auto offsets = [&](int kk) {  // byte offsets of k-tile kk's gathered chunks from their rows
    if ((kk + 1) * DM_BK <= kvalid) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        gof[4 * GO + q] = (uint32_t)__umul24(min(grow_v[q], gsrc), ld2) + gcol[q & 1];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = kk * DM_BK + 8 * wave + 2 * q + (lane >> 5);
        gof[4 * GO + q] = row < kvalid
                              ? (uint32_t)__umul24(min(grow_v[q], gsrc), ld2) + gcol[q & 1]
                              : DM_OOB;
      }
    }
  };
  auto read_rows = [&](int kk) {  // source rows of k-tile kk's four gathered chunks
    lds_char* const ring = (lds_char*)gidx + (wave * 2 + ((kk >> 3) & 1)) * 256;
    const uint32_t at = (uint32_t)(((kk & 7) * 8 + (lane >> 5) * 4) * 4);
    const uint4 i0 = read_k(ring, at);
    grow_v[0] = i0.x; grow_v[1] = i0.y; grow_v[2] = i0.z; grow_v[3] = i0.w;
  };

  // The resources of k-tile kt's loads: each advanced by kt k-tiles (the
  // chunk offsets stay fixed, so a load needs no vector arithmetic), except
  // the gathered operand's (the whole source: its offsets are absolute).
  struct Rs2 {
    i32x4 r[2];
  };
  auto tile_rsrc = [&](int kt) -> Rs2 {
    Rs2 o;
    o.r[0] = (GATH && GO == 0) ? rs[0] : advance_rsrc(rs[0], (uint32_t)kt * kst[0]);
    o.r[1] = (GATH && GO == 1) ? rs[1] : advance_rsrc(rs[1], (uint32_t)kt * kst[1]);
    return o;
  };
  // Chunk q of k-tile kt into stage `stg` through rr = tile_rsrc(kt).
  auto issue_one = [&](lds_char* stg, const Rs2& rr, int kt, int q) {
    const int op = chunk_op(q);
    uint32_t off = gof[q];
    if constexpr (KMASK) {
      if ((op == 0 ? Lay::A_K : Lay::B_K) && kt * DM_BK + kof[q] >= kvalid) off = DM_OOB;
    }
    dma16(off, op == 0 ? rr.r[0] : rr.r[1],
          lds_addr_of(stg) + (op == 0 ? 0u : (uint32_t)DM_TILE) +
              (uint32_t)chunk_unit(q) * 1024u);
  };
  auto issue = [&](lds_char* stg, int kt) {
    const Rs2 rr = tile_rsrc(kt);
#pragma unroll
    for (int q = 0; q < 8; ++q) issue_one(stg, rr, kt, q);
  };

  // Fragment read offsets (K-major: per k-step; MN-major: per 32-wide block).
  uint32_t a_off[2], b_off[2], a_mn[FM], b_mn[FN];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    a_off[s] = fragk_base(wm * WT, s, lane);
    b_off[s] = fragk_base(wn * WT, s, lane) + DM_TILE;
  }
#pragma unroll
  for (int mi = 0; mi < FM; ++mi) a_mn[mi] = fragmn_base(wm * WT + mi * 32, lane);
#pragma unroll
  for (int ni = 0; ni < FN; ++ni) b_mn[ni] = fragmn_base(wn * WT + ni * 32, lane) + DM_TILE;

  f32x16 acc[FM][FN];  // set by the first k-step (a zero accumulator operand)

  // Current fragment offsets, made opaque once per half step (an empty asm on
  // the originals, no copies) so that the compiler keeps one register per
  // offset instead of one per stage. Copying them into fresh registers
  // instead cost 8 moves per half step: 1-2 % of the weight gradients.
  uint32_t ao[2], bo[2], am[FM], bm[FN];
  auto refresh = [&]() {
    if constexpr (Lay::A_K) asm volatile("" : "+v"(a_off[0]), "+v"(a_off[1]));
    else asm volatile("" : "+v"(a_mn[0]), "+v"(a_mn[1]), "+v"(a_mn[2]), "+v"(a_mn[3]));
    if constexpr (Lay::B_K) asm volatile("" : "+v"(b_off[0]), "+v"(b_off[1]));
    else asm volatile("" : "+v"(b_mn[0]), "+v"(b_mn[1]), "+v"(b_mn[2]), "+v"(b_mn[3]));
    ao[0] = a_off[0]; ao[1] = a_off[1]; bo[0] = b_off[0]; bo[1] = b_off[1];
#pragma unroll
    for (int i = 0; i < FM; ++i) am[i] = a_mn[i];
#pragma unroll
    for (int i = 0; i < FN; ++i) bm[i] = b_mn[i];
  };
  // Fragment unit i (0..FM-1: A block i, FM..: B block i - FM) of k-step s.
  auto frag = [&](lds_char* stg, int s, int i, uint4 (&fa)[FM], uint4 (&fb)[FN]) {
    if (i < FM)
      fa[i] = Lay::A_K ? read_k(stg, ao[s] + i * 2048) : read_mn(stg, am[i] + s * 8192);
    else
      fb[i - FM] = Lay::B_K ? read_k(stg, bo[s] + (i - FM) * 2048)
                            : read_mn(stg, bm[i - FM] + s * 8192);
  };
  // Operands swapped: the accumulator holds C^T blocks, so each lane owns one
  // output row and four consecutive columns per register group.
  auto mfma = [&](int i, const uint4 (&fa)[FM], const uint4 (&fb)[FN], bool fresh = false) {
    const f32x16 zero = {};
    acc[i / FN][i % FN] = Mma<ET>::run(fb[i % FN], fa[i / FN], fresh ? zero : acc[i / FN][i % FN]);
  };

  lds_char* const s0 = (lds_char*)stage0;
  lds_char* const s1 = (lds_char*)stage1;
  lds_char* const s2 = (lds_char*)stage2;
  lds_char* const s3 = (lds_char*)stage3;
  uint4 a0[FM], b0[FN], a1[FM], b1[FN];
  // Tile kt: multiply k-step 0 (a0/b0) while reading k-step 1; wait for tile
  // kt+1 (tile kt+2 stays in flight), barrier (every wave is past its reads
  // of tile kt-1); multiply k-step 1 while reading k-step 0 of tile kt+1 and
  // refilling the stage of tile kt-1 with tile kt+3. One MFMA, one fragment
  // read and one DMA chunk per slot, in this order (sched_barrier pins it).
  // Loads past the last tile fall outside the resource (zeros) and land in
  // stages that are never read again.
  auto step = [&](int kt, lds_char* cur, lds_char* nxt, lds_char* refill, auto first_c) {
    refresh();
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
      mfma(i, a0, b0, decltype(first_c)::value);
      if (i < FM + FN) frag(cur, 1, i, a1, b1);
      if constexpr (GATH) {
        if (i == FM * FN - 1) read_rows(kt + 3);  // in flight across the wait
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    TT_WAIT_VMCNT(8);
    __builtin_amdgcn_s_barrier();
    // Nothing moves above the barrier: the gathered rows' clamps would wait
    // there for the ring reads that are meant to be in flight across it.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (GATH) {
      // Indices of k-tiles kt + 5 .. kt + 12 go out before this step's loads,
      // so the next step's wait covers them before step kt + 2 reads them
      // (groups 0 and 1 went out before the prologue).
      if ((kt & 7) == 3 && kt > 3) issue_idx((kt + 5) >> 3);
      offsets(kt + 3);
    }
    refresh();
    const Rs2 rr = tile_rsrc(kt + 3);
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
      mfma(i, a1, b1);
      if (i < FM + FN) frag(nxt, 0, i, a0, b0);
      if ((i & 1) == 0) issue_one(refill, rr, kt + 3, i >> 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if constexpr (GATH) {
    issue_idx(0);
    issue_idx(1);
    TT_WAIT_VMCNT(0);
  }
  auto issue_first = [&](lds_char* stg, int kk) {
    if constexpr (GATH) {
      read_rows(kk);
      offsets(kk);
    }
    issue(stg, kk);
  };
  issue_first(s0, 0);
  issue_first(s1, 1);
  issue_first(s2, 2);
  TT_WAIT_VMCNT(16);
  __builtin_amdgcn_s_barrier();
  refresh();
#pragma unroll
  for (int i = 0; i < FM + FN; ++i) frag(s0, 0, i, a0, b0);
  // The first k-tile starts the accumulators (a zero operand in its first
  // k-step); the loop continues with the same stage rotation.
  const std::false_type more{};
  step(0, s0, s1, s3, std::true_type{});
  if (1 < nkt) step(1, s1, s2, s0, more);
  if (2 < nkt) step(2, s2, s3, s1, more);
  if (3 < nkt) step(3, s3, s0, s2, more);
  for (int kt = DM_ST; kt < nkt; kt += DM_ST) {
    step(kt, s0, s1, s3, more);
    if (kt + 1 < nkt) step(kt + 1, s1, s2, s0, more);
    if (kt + 2 < nkt) step(kt + 2, s2, s3, s1, more);
    if (kt + 3 < nkt) step(kt + 3, s3, s0, s2, more);
  }
  TT_WAIT_VMCNT(0);  // every DMA has landed before the stages are reused
  __syncthreads();   // every wave is past its last fragment read
  lds_char* const region = wave == 0 ? s0 : wave == 1 ? s1 : wave == 2 ? s2 : s3;
  store_wave_tile<ET>(acc, t, t.i0 + wm * WT, t.j0 + wn * WT, lane, region);
}

// Barrier that also publishes this wave's LDS stores and retires its LDS
// reads: wait for them, then s_barrier; the memory clobber keeps the
// compiler from moving LDS accesses across it. Loads in flight (vmcnt) are
// not waited for.
#define TT_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// Output tile L (fwd / dgrad) from the schedule in LDS.
template <int MODE, bool TRANS_B, int ESZ>
__device__ __forceinline__ void tile_at(int L, const char* p0, const char* p1, char* out,
                                        int64_t K, int64_t N, int E, int tiles_j,
                                        const int64_t* row_start, const int* tile_start,
                                        TileDesc& t) {
  const int slot = L;
  // Last e with tile_start[e] <= slot (tile_start, the experts' schedule-slot
  // prefix, is non-decreasing and tile_start[0] = 0): the wave's 64 lanes
  // test 64 evenly spaced candidates of the range at once, and the count of
  // lanes that pass narrows the range to one stride (one LDS round trip per
  // 64-fold narrowing).
  const int lane = __lane_id();
  int lo = 0, span = E;
  while (span > 1) {
    const int stride = (span + 63) >> 6;
    const bool ok = lane * stride < span && tile_start[lo + lane * stride] <= slot;
    const int c = __popcll(__ballot(ok)) - 1;
    lo += c * stride;
    span = min(stride, span - c * stride);
  }
  // Schedule values are uniform: keep them (and all that derives from them)
  // in scalar registers.
  const int e = __builtin_amdgcn_readfirstlane(lo);
  t.e = e;
  t.seg0 = rfl64(row_start[e]);
  t.nrows = rfl64(row_start[e + 1]) - t.seg0;
  const int ts_e = __builtin_amdgcn_readfirstlane(tile_start[e]);
  if constexpr (MODE == MODE_FWD) {
    t.a = p0 + t.seg0 * K * ESZ; t.lda = K;
    t.b = p1 + (int64_t)e * K * N * ESZ; t.ldb = TRANS_B ? K : N;
    t.I = t.nrows; t.J = N; t.R = K;
    t.c = out + t.seg0 * N * ESZ; t.ldc = N;
  } else {
    t.a = p0 + t.seg0 * N * ESZ; t.lda = N;
    t.b = p1 + (int64_t)e * K * N * ESZ; t.ldb = TRANS_B ? K : N;
    t.I = t.nrows; t.J = K; t.R = N;
    t.c = out + t.seg0 * K * ESZ; t.ldc = K;
  }
  const int local = slot - ts_e;
  if (t.nrows > 0 && t.nrows <= 64) {  // two thin tiles per slot
    t.i0 = 0;
    t.j0 = (int64_t)(2 * local) * DM_BN;
    t.nsub = min(2, tiles_j - 2 * local);
  } else {
    t.i0 = (int64_t)(local / tiles_j) * DM_BM;
    t.j0 = (int64_t)(local % tiles_j) * DM_BN;
    t.nsub = 0;
  }
}

// ===========================================================================
// Persistent MFMA kernel (fwd / dgrad, bf16 / f16): one block per CU walks a
// strided list of 256x256 output tiles and streams their 64-deep k-tiles as
// one sequence through two LDS stages, so a tile's first k-tiles are already
// loading while the previous tile finishes and its epilogue runs; the
// expert schedule is built once per block. Tile L of a launch (slot-major,
// n-tile minor) goes to block position L % G, positions XCD-grouped, so the
// CUs of one XCD work on consecutive tiles (shared A panels and weights).
// ===========================================================================
// 256x256x64 tiles, two 64 KiB LDS stages (A 32 KiB, B 32 KiB). K-major rows
// are 128 bytes per k-tile, so every load covers whole 128-byte lines.
constexpr int P_BK = 64;
constexpr int P_OPND = 256 * P_BK * 2;  // one operand tile (32 KiB)
constexpr int P_STAGE = 2 * P_OPND;     // A then B
constexpr int P_EPI = 4096;             // epilogue staging per wave
// wgrad takes the persistent kernel when the mean rows per expert are at most
// this (a handful of 64-deep k-tiles per output tile).
constexpr int64_t P_WGRAD_ROWS = 512;
// ... or experts of at least this many 256x256 output tiles.
constexpr int P_WGRAD_TILES = 512;

// K-major 64-deep tile: LDS row r (128 bytes) holds tile row r, its 16-byte
// chunk c in slot c ^ ((r >> 1) & 7): any 16 consecutive rows then cover the
// 16 distinct 16-byte bank groups of a 256-byte bank line, so a fragment
// read (one chunk of 32 rows per half-wave) is free of bank conflicts.
// Fragment for k-step s (0..3): rows r0 + lane % 32, chunk 2 s + lane / 32;
// further 32-row blocks add 4096.
__device__ __forceinline__ uint32_t fragk64(int r0, int s, int lane) {
  const int r = r0 + (lane & 31);
  const int c = 2 * s + (lane >> 5);
  return (uint32_t)(r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
}

// Epilogue of the 64-deep kernel: the wave's 128x128 tile in 8 rounds of
// 32 rows x 64 columns through its private 4 KiB of LDS (row r at 128 r,
// 16-byte chunk c in slot c ^ ((r >> 1) & 7)), stored as 128-byte row segments with
// buffer stores. The store resource ends at the expert's last row, so
// stores to rows past it are dropped by the hardware; columns past the
// output width are given an offset past the resource. AUX is the stores'
// cache policy: 2 (streaming, the lines do not stay in L2 to evict operand
// panels). Weight gradients: 5 % faster on DeepSeek-V3's write-bound
// launches. Activations (fwd / dgrad outputs, 384-512 MiB on Qwen, far more
// than L2 holds, so the next kernel reads them from memory either way): the
// Qwen layer step 0.4 % faster than with the default policy. The wave's
// 32-row block mi starts ROWSTEP * mi rows below ri; only its first NMI
// blocks are stored (the others lie past the expert's rows).
template <int ET, int AUX, int ROWSTEP, int NMI>
__device__ __forceinline__ void store_wave_tile_p64(const f32x16 (&acc)[4][4], const TileDesc& t,
                                                    int64_t ri, int64_t cj, lds_char* region) {
  // Lane index computed here (volatile, so neither it nor what derives from
  // it is hoisted into registers that stay live across the k-loop).
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  // The accumulator reads below are inline assembly, which the compiler's
  // hazard padding does not cover: wait out the MFMA write-to-read latency.
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  const int64_t rows = t.I - ri;
  const int64_t obytes = rows > 0 ? rows * t.ldc * 2 - cj * 2 : 0;
  const uint32_t nrec = obytes < (int64_t)DM_OOB ? (uint32_t)obytes : DM_OOB;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(t.c + (ri * t.ldc + cj) * 2), (short)0, (int)nrec, 0x00020000);
  const uint32_t row_bytes = (uint32_t)(t.ldc * 2);
  const int r_l = lane & 31, h = lane >> 5;
  const int rr = lane >> 3, ch = lane & 7;
  // Per-lane offsets, the same in every round: the eight 8-byte pieces this
  // lane writes (row r_l, chunk c), the four rows 8 q + rr it reads back
  // (chunk ch) and where they go in the output.
  uint32_t wof[8], rof[4], sof[4];
#pragma unroll
  for (int c = 0; c < 8; ++c) wof[c] = (uint32_t)(r_l * 128 + ((c ^ ((r_l >> 1) & 7)) << 4) + 8 * h);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = 8 * q + rr;
    rof[q] = (uint32_t)(r * 128 + ((ch ^ ((r >> 1) & 7)) << 4));
    sof[q] = (uint32_t)r * row_bytes + (uint32_t)(16 * ch);
  }
  const bool col_ok[2] = {cj + 8 * ch < t.J, cj + 64 + 8 * ch < t.J};
  // Round rd = (mi, nh): the wave's 32 x 64 piece through the region. The
  // rows read back in round rd are stored after round rd + 1 has been
  // written, so the LDS read latency hides behind that work (LDS accesses of
  // one wave complete in order, so the writes never overtake the reads).
  uint4 back[4];
#pragma unroll
  for (int rd = 0; rd <= 2 * NMI; ++rd) {
    if (rd < 2 * NMI) {
      const int mi = rd >> 1, nh = rd & 1;
#pragma unroll
      for (int nn = 0; nn < 2; ++nn)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ni = 2 * nh + nn;
          // Accumulators are read out of the AGPRs four at a time, where they
          // are converted (a bulk copy would need the whole register file).
          float x0, x1, x2, x3;
          asm volatile("v_accvgpr_read_b32 %0, %4\n\tv_accvgpr_read_b32 %1, %5\n\t"
                       "v_accvgpr_read_b32 %2, %6\n\tv_accvgpr_read_b32 %3, %7"
                       : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3)
                       : "a"(acc[mi][ni][4 * g]), "a"(acc[mi][ni][4 * g + 1]),
                         "a"(acc[mi][ni][4 * g + 2]), "a"(acc[mi][ni][4 * g + 3]));
          const uint2 v = pack4<ET>(x0, x1, x2, x3);
          *reinterpret_cast<lds_u32x2*>(region + wof[4 * nn + g]) = u32x2{v.x, v.y};
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (rd > 0) {
      const int mi = (rd - 1) >> 1, nh = (rd - 1) & 1;
      const uint32_t base = (uint32_t)(ROWSTEP * mi) * row_bytes + (uint32_t)(128 * nh);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t off = col_ok[nh] ? sof[q] + base : DM_OOB;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, back[q]), rs, (int)off,
                                               0, AUX);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (rd < 2 * NMI) {
#pragma unroll
      for (int q = 0; q < 4; ++q) back[q] = read_k(region, rof[q]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Weight-gradient work queues of the persistent kernel. A launch owns one
// slot (slots rotate between launches); the slot holds one ticket counter per
// tile class (the blocks of one XCD), zeroed by wgrad_queue_reset_kernel on
// the launch stream just before the launch. Blocks take tickets with atomic
// adds and leave once a ticket passes the end of their class's list; no block
// ever waits for another.
constexpr int WQ_CLASSES = 8, WQ_STRIDE = 16;
__device__ int g_wgrad_queue[WQ_SLOTS * WQ_STRIDE];

__global__ void wgrad_queue_reset_kernel(int slot) {
  if (threadIdx.x < WQ_STRIDE) g_wgrad_queue[slot * WQ_STRIDE + threadIdx.x] = 0;
}

// Expert ranks, longest first (ties by id): ranked[r] = expert of rank r.
// cnt and rnk are E ints of scratch each.
template <int NT>
__device__ void rank_experts(const int64_t* row_start, int E, int* cnt, int* rnk, int* ranked) {
  for (int x = threadIdx.x; x < E; x += NT) {
    cnt[x] = (int)(row_start[x + 1] - row_start[x]);
    rnk[x] = 0;
  }
  __syncthreads();
  const int parts = E >= NT ? 1 : NT / E;
  for (int idx = threadIdx.x; idx < E * parts; idx += NT) {
    const int x = idx % E, part = idx / E;
    const int y0 = part * E / parts, y1 = (part + 1) * E / parts;
    const int cx = cnt[x];
    int r = 0;
    for (int y = y0; y < y1; ++y) {
      const int cy = cnt[y];
      r += (cy > cx) | ((cy == cx) & (y < x));
    }
    atomicAdd(&rnk[x], r);
  }
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += NT) ranked[rnk[x]] = x;
  __syncthreads();
}

// An expert's wgrad tile grid (tiles_i x tiles_j) split into 8 equal
// rectangles (a x c of them, h x w tiles each) when it can be: tile rem then
// lies in rectangle rem % 8, so the tiles of one class (rem = x + 8 j) share
// h + w activation panels. Otherwise tiles go in row order.
struct WgradRect {
  int h, w, c;
};
__device__ __forceinline__ WgradRect wgrad_rect(int tiles_i, int tiles_j) {
  WgradRect r{0, 0, 0};
  if ((tiles_i * tiles_j) % 8 == 0) {
    int best = 1 << 30;
    for (int a = 1; a <= 8; a <<= 1) {
      const int cc = 8 / a;
      if (tiles_i % a || tiles_j % cc) continue;
      const int hh = tiles_i / a, ww = tiles_j / cc;
      if (hh + ww < best) { best = hh + ww; r.h = hh; r.w = ww; r.c = cc; }
    }
  }
  return r;
}

// Tile of ticket q in class cls (cx tiles per expert): expert of rank q / cx,
// its tile rem = cls + nx * (q % cx). Returns the tile's k-tile count (at
// least two: the pipeline prefetches two k-tiles ahead; an expert without rows
// runs two k-tiles of zeros and stores a zero gradient).
template <bool TRANS_B>
__device__ __forceinline__ int wgrad_tile_at(int q, int cls, int nx, int cx, const WgradRect& rc,
                                             int tiles_j, const char* p0, const char* p1,
                                             char* out, int64_t K, int64_t N,
                                             const int64_t* row_start, const int* ranked,
                                             TileDesc& t) {
  const int e = __builtin_amdgcn_readfirstlane(ranked[q / cx]);
  const int rem = cls + nx * (q % cx);
  int it, jt;
  if (rc.h > 0) {
    const int x = rem % 8, j = rem / 8;
    it = (x / rc.c) * rc.h + j / rc.w;
    jt = (x % rc.c) * rc.w + j % rc.w;
  } else {
    it = rem / tiles_j;
    jt = rem % tiles_j;
  }
  t.e = e;
  t.seg0 = rfl64(row_start[e]);
  t.nrows = rfl64(row_start[e + 1]) - t.seg0;
  t.R = t.nrows;
  if constexpr (!TRANS_B) {
    t.a = p0 + t.seg0 * K * 2; t.lda = K;  // x
    t.b = p1 + t.seg0 * N * 2; t.ldb = N;  // dy
    t.I = K; t.J = N;
  } else {
    t.a = p1 + t.seg0 * N * 2; t.lda = N;  // dy
    t.b = p0 + t.seg0 * K * 2; t.ldb = K;  // x
    t.I = N; t.J = K;
  }
  t.c = out + (int64_t)e * K * N * 2; t.ldc = t.J;
  t.i0 = (int64_t)it * DM_BM;
  t.j0 = (int64_t)jt * DM_BN;
  const int nkt = (int)((t.R + P_BK - 1) / P_BK);
  return nkt > 2 ? nkt : 2;
}

// Cost-sorted schedule for fwd / dgrad launches of at most LPT_MAX_TJ n-tiles per
// m-tile, whose slots differ most in cost (a slot of two thin tiles costs
// about 1.2 full tiles, a single thin tile 0.6). The static schedule hands
// every XCD its consecutive positions round by round; here each round's slots
// of an XCD, heaviest first, go to that XCD's blocks least loaded so far, so
// the same slots still run on the same XCD in the same round (shared operand
// panels in its L2). Qwen3-30B-A3B's gathered fc2 data gradient (three n-tiles,
// seven rounds): 424 -> 407 us with the assignment computed here (410 -> 379 us
// with a table computed on the host). Launches with six or more n-tiles gained
// 0-1 % from the host table and keep the static order; so do launches of many
// rounds, where the assignment costs more (one round of slot decoding and
// ranking each) and the last partial round weighs less: the varlen stress
// layer's fc2 data gradient (27 rounds) took 1589 against 1543 us.
constexpr int LPT_MAX_TJ = 4;
constexpr int LPT_MAX_ROUNDS = 12;

// Cost of schedule slot s in twentieths of a full tile: 20 full, 17 a partial
// m-tile of more than 128 rows, 13 of at most 128 rows, 12 per thin tile.
__device__ int lpt_cost(int s, int E, int tiles_j, const int64_t* row_start,
                        const int* tile_start) {
  int lo = 0, hi = E - 1;  // last e with tile_start[e] <= s
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile_start[mid] <= s) lo = mid; else hi = mid - 1;
  }
  const int64_t rows = row_start[lo + 1] - row_start[lo];
  const int local = s - tile_start[lo];
  if (rows > 0 && rows <= 64) return 12 * min(2, tiles_j - 2 * local);
  const int64_t left = rows - (int64_t)(local / tiles_j) * DM_BM;
  return left >= DM_BM ? 20 : (left <= 128 ? 13 : 17);
}

// Wave 0 computes the assignment of this block's XCD (lane l = the XCD's
// block l, positions x Q + l with Q = G / 8) and keeps this block's slots in
// `slots`; every thread gets the block's slot count. Per round: slots ranked
// by cost (descending, then position) with one ballot per cost value, blocks
// ranked by load (ascending, then index); block of load rank i takes the slot
// of cost rank i. Each slot goes to exactly one block: both ranks are
// permutations.
__device__ int lpt_schedule(int total, int G, int E, int tiles_j, const int64_t* row_start,
                            const int* tile_start, int* slots, int* tmp, int* tmpc,
                            int* nout) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    const int Q = G >> 3, base = (int)(blockIdx.x & 7) * Q, me = (int)(blockIdx.x >> 3);
    const uint64_t below = l == 0 ? 0ull : (~0ull >> (64 - l));
    const int rounds = (total + G - 1) / G;
    int acc = 0, mine = 0;
    for (int k = 0; k < rounds; ++k) {
      const int s = k * G + base + l;
      const bool valid = l < Q && s < total;
      const int c = valid ? lpt_cost(s, E, tiles_j, row_start, tile_start) : 0;
      const uint64_t m24 = __ballot(valid && c == 24), m20 = __ballot(valid && c == 20);
      const uint64_t m17 = __ballot(valid && c == 17), m13 = __ballot(valid && c == 13);
      const uint64_t m12 = __ballot(valid && c == 12);
      uint64_t heavier = 0, same = m12;
      if (c == 24) { same = m24; }
      else if (c == 20) { heavier = m24; same = m20; }
      else if (c == 17) { heavier = m24 | m20; same = m17; }
      else if (c == 13) { heavier = m24 | m20 | m17; same = m13; }
      else { heavier = m24 | m20 | m17 | m13; }
      const int rc = __popcll(heavier) + __popcll(same & below);
      const int nvalid = __popcll(m24 | m20 | m17 | m13 | m12);
      int ra = 0;
      for (int m = 0; m < Q; ++m) {
        const int am = __builtin_amdgcn_readlane(acc, m);
        ra += (am < acc) || (am == acc && m < l);
      }
      if (valid) {
        tmp[rc] = s;
        tmpc[rc] = c;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (l < Q && ra < nvalid) {
        acc += tmpc[ra];
        if (l == me) slots[mine++] = tmp[ra];
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    if (l == me) *nout = mine;
  }
  __syncthreads();
  return *nout;
}

// GA (fwd / dgrad): the A rows are gathered, row r of the packed order being
// row arow[r] of p0 ([asrc_rows, lda]); see gather_rows below.
template <int MODE, bool TRANS_B, int ET, bool KMASK, bool GA = false>
__global__ __launch_bounds__(DM_NT) void gmm_p64_kernel(const char* __restrict__ p0,
                                                        const char* __restrict__ p1,
                                                        char* __restrict__ out, int64_t M,
                                                        int64_t K, int64_t N, int E,
                                                        const int64_t* __restrict__ counts,
                                                        int tiles_i, int tiles_j, int qslot,
                                                        const int32_t* __restrict__ arow,
                                                        int64_t asrc_rows) {
  constexpr bool WG = MODE == MODE_WGRAD;
  static_assert(!(WG && KMASK), "wgrad reduces over rows (no K-major tail)");
  static_assert(!(GA && (WG || KMASK)), "gathered A rows: fwd / dgrad without a K-major tail");
  typedef Layout<MODE, TRANS_B> Lay;
  constexpr int WT = 128, FM = 4, FN = 4;
  __shared__ __align__(16) char lds_raw[2 * P_STAGE];
  __shared__ __align__(16) char epi_raw[4 * P_EPI];
  __shared__ int ticket_slot[2];
  extern __shared__ __align__(16) char smem[];  // expert schedule
  int64_t* row_start = reinterpret_cast<int64_t*>(smem);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);
  scan_counts<DM_NT>(counts, E, DM_BM, row_start, tile_start, WG ? 0 : tiles_j);

  const int G = gridDim.x;
  // fwd / dgrad: block position pos walks tiles pos, pos + G, ... (XCD-grouped
  // positions). wgrad: class cls = blockIdx % nx takes tickets from its queue.
  int pos = 0, ntiles = 0, total = 0;
  int nx = 1, cls = 0, cx = 1;
  int* queue = nullptr;
  int* ranked = nullptr;
  WgradRect rect{0, 0, 0};
  int q0 = 0;
  __shared__ int lpt_slots[LPT_MAX_ROUNDS], lpt_tmp[64], lpt_tmpc[64], lpt_n;
  bool lpt = false;
  if constexpr (!WG) {
    pos = xcd_remap(blockIdx.x, G);
    total = tile_start[E];  // schedule slots
    lpt = tiles_j <= LPT_MAX_TJ && (G & 7) == 0 && G <= 512 &&
          (total + G - 1) / G <= LPT_MAX_ROUNDS;
    if (lpt) {
      ntiles = lpt_schedule(total, G, E, tiles_j, row_start, tile_start, lpt_slots, lpt_tmp,
                            lpt_tmpc, &lpt_n);
      if (ntiles == 0) return;
    } else {
      if (pos >= total) return;
      ntiles = (total - pos + G - 1) / G;
    }
  } else {
    int* cnt = tile_start + E + 1;
    ranked = cnt + 2 * E;
    rank_experts<DM_NT>(row_start, E, cnt, cnt + E, ranked);
    nx = G >= WQ_CLASSES ? WQ_CLASSES : 1;
    cls = blockIdx.x % nx;
    const int per = tiles_i * tiles_j;
    cx = (per - cls + nx - 1) / nx;
    total = E * cx;
    if (cx == 0) return;
    rect = wgrad_rect(tiles_i, tiles_j);
    queue = g_wgrad_queue + qslot * WQ_STRIDE + cls;
    if (threadIdx.x == 0) ticket_slot[0] = atomicAdd(queue, 1);
    __syncthreads();
    q0 = ticket_slot[0];
    if (q0 >= total) return;
  }
  // Schedule slot of the block's n-th tile (fwd / dgrad).
  auto slot_of = [&](int n) -> int {
    return lpt ? __builtin_amdgcn_readfirstlane(lpt_slots[n]) : pos + n * G;
  };
  const int64_t R = MODE == MODE_FWD ? K : N;  // fwd / dgrad reduction length
  int nkt_c = (int)((R + P_BK - 1) / P_BK);     // >= 2 (host check)
  int nkt_n = nkt_c;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t lda = WG ? (TRANS_B ? N : K) : (MODE == MODE_FWD ? K : N);
  const int64_t ldb = WG ? (TRANS_B ? K : N) : (TRANS_B ? K : N);

  // Loads: every wave brings 8 KiB of A (chunks 0-7) and 8 KiB of B (8-15)
  // per k-tile, 1 KiB per instruction. K-major: rows 64 w + 8 q + lane / 8,
  // slot lane % 8; MN-major: k-rows 16 w + 2 q + lane / 32, slot lane % 32.
  // Offsets are relative to the tile origin (the resource base). The slot
  // swizzle alternates between even and odd chunks q, so each parity has a
  // base offset of its own and chunk q adds a uniform (q / 2) * qstep.
  uint32_t vbase[2], vodd[2], qstep[2], kstep[2];
  int kof = 0, kof_odd = 0;
#pragma unroll
  for (int op = 0; op < 2; ++op) {
    const bool kmaj = op == 0 ? Lay::A_K : Lay::B_K;
    const int64_t ld = op == 0 ? lda : ldb;
    if (kmaj) {
      // Row 64 w + 8 q + lane / 8: (row >> 1) & 7 = lane / 16 + 4 (q & 1).
      const int r = 64 * wave + (lane >> 3);
      const int c = (lane & 7) ^ (lane >> 4);
      const int c1 = c ^ 4;
      vbase[op] = (uint32_t)(((int64_t)r * ld + 8 * c) * 2);
      vodd[op] = (uint32_t)(((int64_t)(r + 8) * ld + 8 * c1) * 2);
      qstep[op] = (uint32_t)(16 * ld * 2);  // per pair of chunks
      kstep[op] = P_BK * 2;
      kof = 8 * c;
      kof_odd = 8 * c1;
    } else {
      const int kr = 16 * wave + (lane >> 5);
      const int c = (lane & 31) ^ (4 * (kr & 3));
      const int c1 = (lane & 31) ^ (4 * ((kr + 2) & 3));
      vbase[op] = (uint32_t)(((int64_t)kr * ld + 8 * c) * 2);
      vodd[op] = (uint32_t)(((int64_t)(kr + 2) * ld + 8 * c1) * 2);
      qstep[op] = (uint32_t)(4 * ld * 2);  // per pair of chunks
      kstep[op] = (uint32_t)(P_BK * ld * 2);
    }
  }

  // Each chunk's offset from the tile origin, fixed for the launch; the
  // k-tile moves the buffer resource (scalar arithmetic) instead.
  uint32_t choff[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int op = q < 8 ? 0 : 1, qq = q & 7;
    choff[q] = ((qq & 1) ? vodd[op] : vbase[op]) + (uint32_t)(qq >> 1) * qstep[op];
  }
  const uint32_t ks_a = (uint32_t)__builtin_amdgcn_readfirstlane((int)kstep[0]);
  const uint32_t ks_b = (uint32_t)__builtin_amdgcn_readfirstlane((int)kstep[1]);
  // Resources based at the tile origin. fwd / dgrad: A is K-major (the
  // expert's rows), B the expert's weights. wgrad: both operands are
  // MN-major over the expert's rows, so reduction rows past the expert's
  // end read as zeros.
  auto rsrc_a = [&](const TileDesc& t, bool valid) -> i32x4 {
    if constexpr (GA) return make_rsrc(p0, asrc_rows * lda * 2);  // the whole source
    if (!valid) return make_rsrc(p0, 0);
    if constexpr (WG) return make_rsrc(t.a + t.i0 * 2, t.R * t.lda * 2 - t.i0 * 2);
    const int64_t toff = t.i0 * t.lda * 2;
    return make_rsrc(t.a + toff, t.nrows * t.lda * 2 - toff);
  };
  auto rsrc_b = [&](const TileDesc& t, bool valid) -> i32x4 {
    if (!valid) return make_rsrc(p0, 0);
    if constexpr (WG) return make_rsrc(t.b + t.j0 * 2, t.R * t.ldb * 2 - t.j0 * 2);
    const int64_t toff = Lay::B_K ? t.j0 * t.ldb * 2 : t.j0 * 2;
    return make_rsrc(t.b + toff, K * N * 2 - toff);
  };

  // wgrad claims the next tile's ticket two or three k-tiles before the end
  // of the current one (late enough to keep the assignment greedy, early
  // enough to prefetch the next tile's first k-tiles): the ticket is taken at
  // k-tile claim_kt, published at k-tile nkt_c - 2 and decoded right after
  // that k-tile's barrier, before its loads of the next tile.
  TileDesc tc, tn;
  bool has_next;
  if constexpr (WG) {
    nkt_c = wgrad_tile_at<TRANS_B>(q0, cls, nx, cx, rect, tiles_j, p0, p1, out, K, N, row_start,
                                   ranked, tc);
    has_next = false;  // known at k-tile nkt_c - 2
  } else {
    tile_at<MODE, TRANS_B, 2>(slot_of(0), p0, p1, out, K, N, E, tiles_j, row_start, tile_start,
                              tc);
    has_next = ntiles > 1;
    if (has_next)
      tile_at<MODE, TRANS_B, 2>(slot_of(1), p0, p1, out, K, N, E, tiles_j, row_start, tile_start,
                                tn);
  }
  // GA: the source row of each of the lane's eight A rows of a tile (K-major
  // rows 64 wave + lane / 8 + 8 q), loaded when the tile is decoded; rows past
  // the expert's end get GA_NOROW. gather_offsets turns them into byte offsets
  // after a wait that the k-loop makes anyway (the first k-tile's), so the
  // index loads never stall the loop.
  uint32_t ro_cur[8], ro_nxt[8];
  auto gather_rows = [&](const TileDesc& t, bool valid, uint32_t (&ro)[8]) {
    if (!valid) {
#pragma unroll
      for (int q = 0; q < 8; ++q) ro[q] = GA_NOROW;
      return;
    }
    const int64_t r0 = t.i0 + 64 * wave + (lane >> 3);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int64_t row = r0 + 8 * q;
      const int64_t at = t.seg0 + row;
      const uint32_t v = (uint32_t)arow[at < M ? at : M - 1];
      // An entry outside [0, asrc_rows) (a negative id reads as a large
      // unsigned value) reads a row of zeros, like a row past the expert.
      ro[q] = row < t.nrows && v < (uint32_t)asrc_rows ? v : GA_NOROW;
    }
  };
  // Byte offsets of the lane's A chunks in the source (row and k-chunk).
  auto gather_offsets = [&](uint32_t (&ro)[8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      ro[q] = ro[q] == GA_NOROW ? GA_NOROW
                                : ro[q] * (uint32_t)(lda * 2) + (uint32_t)(2 * ((q & 1) ? kof_odd : kof));
  };
  if constexpr (GA) {
    gather_rows(tc, true, ro_cur);
    gather_rows(tn, has_next, ro_nxt);  // converted in the first k-tile
    TT_WAIT_VMCNT(0);
    gather_offsets(ro_cur);
  }
  i32x4 ra_cur = rsrc_a(tc, true), rb_cur = rsrc_b(tc, true);
  i32x4 ra_nxt = rsrc_a(tn, has_next), rb_nxt = rsrc_b(tn, has_next);
  const int kvalid = (int)R;
  int pending = 0;  // wgrad: ticket of the next tile (thread 0)
  int n = 0;        // tiles finished

  // Chunk q (0-7 A, 8-15 B) of k-tile k of the current or next tile.
  auto issue_one = [&](lds_char* stg, int k, bool nxt, int q) {
    const bool is_a = q < 8;
    const int op = is_a ? 0 : 1;
    const bool kmaj = is_a ? Lay::A_K : Lay::B_K;
    const int qq = q & 7;
    uint32_t off = choff[q];
    if constexpr (GA) {
      if (is_a) off = nxt ? ro_nxt[qq] : ro_cur[qq];  // the row's source offset and k-chunk
    }
    if constexpr (KMASK) {
      if (kmaj && k * P_BK + ((qq & 1) ? kof_odd : kof) >= kvalid) off = DM_OOB;
    }
    const i32x4 rs = advance_rsrc(is_a ? (nxt ? ra_nxt : ra_cur) : (nxt ? rb_nxt : rb_cur),
                                  (uint32_t)k * (is_a ? ks_a : ks_b));
    dma16(off, rs, lds_addr_of(stg) + (is_a ? 0u : (uint32_t)P_OPND) +
                       (uint32_t)(8 * wave + (q & 7)) * 1024u);
  };

  // A fragments. wgrad (MN-major A): wave row wm owns tile rows 128 wm ..
  // 128 wm + 127, 32-row block mi at +32 mi. fwd / dgrad (K-major A): the
  // blocks of the two wave rows interleave, wave row wm owning tile rows
  // 64 mi + 32 wm .. + 31, so the rows an expert's last (partial) tile holds
  // spread evenly over both wave rows and the blocks past them can be skipped.
  constexpr uint32_t A_MI = WG ? 4096u : 8192u;  // LDS bytes between a wave's A blocks
  constexpr int EPI_ROWS = WG ? 32 : 64;         // output rows between a wave's blocks
  const int a_row0 = WG ? wm * WT : 32 * wm;
  uint32_t a_k[4], b_k[4], a_mn[FM], b_mn[FN];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a_k[s] = fragk64(a_row0, s, lane);
    b_k[s] = fragk64(wn * WT, s, lane) + P_OPND;
  }
#pragma unroll
  for (int mi = 0; mi < FM; ++mi) a_mn[mi] = fragmn_base(wm * WT + mi * 32, lane);
#pragma unroll
  for (int ni = 0; ni < FN; ++ni) b_mn[ni] = fragmn_base(wn * WT + ni * 32, lane) + P_OPND;

  uint32_t ao, bo, am[FM], bm[FN];
  // Offsets for k-step s, made opaque per use (an empty asm on the originals,
  // no copies: one register each). Copies into fresh registers cost about 20
  // moves per k-tile: 1-3 % of the forward GEMMs.
  auto refresh = [&](int s) {
    if constexpr (Lay::A_K) asm volatile("" : "+v"(a_k[s]));
    else asm volatile("" : "+v"(a_mn[0]), "+v"(a_mn[1]), "+v"(a_mn[2]), "+v"(a_mn[3]));
    if constexpr (Lay::B_K) asm volatile("" : "+v"(b_k[s]));
    else asm volatile("" : "+v"(b_mn[0]), "+v"(b_mn[1]), "+v"(b_mn[2]), "+v"(b_mn[3]));
    ao = a_k[s]; bo = b_k[s];
#pragma unroll
    for (int i = 0; i < FM; ++i) am[i] = a_mn[i];
#pragma unroll
    for (int i = 0; i < FN; ++i) bm[i] = b_mn[i];
  };
  // Fragment i of k-step s for a tile whose waves multiply MV of their four
  // 32-row blocks: A blocks 0 .. MV - 1, then the four B blocks.
  auto frag = [&](auto mv_c, lds_char* stg, int s, int i, uint4 (&fa)[FM], uint4 (&fb)[FN]) {
    constexpr int MV = decltype(mv_c)::value;
    if (i < MV)
      fa[i] = Lay::A_K ? read_k(stg, ao + i * A_MI) : read_mn(stg, am[i] + s * 8192);
    else
      fb[i - MV] = Lay::B_K ? read_k(stg, bo + (i - MV) * 4096)
                            : read_mn(stg, bm[i - MV] + s * 8192);
  };
  // fresh: the block's first product of a tile (the accumulator starts at zero)
  auto mfma = [&](f32x16 (&acc)[FM][FN], int i, const uint4 (&fa)[FM], const uint4 (&fb)[FN],
                  bool fresh = false) {
    const f32x16 zero = {};
    acc[i / FN][i % FN] = Mma<ET>::run(fb[i % FN], fa[i / FN], fresh ? zero : acc[i / FN][i % FN]);
  };

  lds_char* const lds = (lds_char*)lds_raw;
  auto stage = [&](int g) { return lds + (g & 1) * P_STAGE; };
  uint4 a0[FM], b0[FN], a1[FM], b1[FN];

  // One k-tile of a tile whose waves multiply MV (4, 2 or 1) of their 32-row
  // blocks, NM = 4 MV MFMAs per k-step: k-steps 0-2 multiply while reading
  // the next k-step's fragments (and k-step 0 loads the B half of k-tile
  // kt + 1 into the other stage, spread over the MFMA slots); then wait for
  // k-tile kt + 1 (the only loads in flight), barrier (every wave is past its
  // reads of this stage), and k-step 3 multiplies while reading k-step 0 of
  // k-tile kt + 1 and loading the A half of k-tile kt + 2 into this stage.
  // Issuing a k-tile's 16 loads in one k-step backs up the vector memory
  // path and stalls the MFMAs behind it; the B half in k-step 0 alone (not
  // spread over k-steps 0 and 1) gives its loads one more k-step to land
  // before the wait: Qwen3-30B-A3B's four launches 0.5-2.5 % faster (one
  // level), Mixtral's 1.4-2.6 %, the varlen stress layer's up to 1.5 %
  // slower. The loads are the same in every variant: rows past an expert's
  // end read as zeros without memory traffic.
  auto step = [&](f32x16 (&acc)[FM][FN], int kt, int g, auto first_c, auto mv_c) {
    constexpr bool LAST = false;
    constexpr bool FIRST = decltype(first_c)::value;
    constexpr int MV = decltype(mv_c)::value;
    constexpr int NM = MV * FN;       // MFMAs per k-step
    constexpr int NF = MV + FN;       // fragment reads per k-step
    lds_char* const cur = stage(g);
    lds_char* const nxt = stage(g + 1);
    const int k1 = kt + 1, k2 = kt + 2;
    const bool to_next1 = k1 >= nkt_c, to_next2 = k2 >= nkt_c;
    const int kr1 = to_next1 ? k1 - nkt_c : k1;
    const int kr2 = to_next2 ? k2 - nkt_c : k2;
    if constexpr (WG) {
      const int claim_kt = nkt_c > 3 ? nkt_c - 3 : 0;
      if (kt == claim_kt && threadIdx.x == 0) pending = atomicAdd(queue, 1);
    }
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      refresh(s + 1);
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        if (s & 1) mfma(acc, i, a1, b1); else mfma(acc, i, a0, b0, FIRST && s == 0);
        if (i < NF) {
          if (s & 1) frag(mv_c, cur, s + 1, i, a0, b0); else frag(mv_c, cur, s + 1, i, a1, b1);
        }
        if (s == 0) {
          if constexpr (NM >= 8) {
            if (i % (NM / 8) == (NM / 8 > 1 ? 1 : 0))
              issue_one(nxt, kr1, to_next1, 8 + i / (NM / 8));
          } else {
            issue_one(nxt, kr1, to_next1, 8 + 2 * i);
            issue_one(nxt, kr1, to_next1, 9 + 2 * i);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = NM; i < NF; ++i) {  // one MFMA per wave row: a read left over
        if (s & 1) frag(mv_c, cur, s + 1, i, a0, b0); else frag(mv_c, cur, s + 1, i, a1, b1);
      }
    }
    TT_WAIT_VMCNT(0);
    if constexpr (GA) {
      if (FIRST) gather_offsets(ro_nxt);  // the next tile's rows have arrived
    }
    if constexpr (WG) {
      // The claimed ticket has returned (the wait above covers it); the
      // barrier publishes it, and the next tile is decoded before this
      // k-tile's loads of it.
      if (kt == nkt_c - 2 && threadIdx.x == 0) ticket_slot[n & 1] = pending;
    }
    TT_LDS_BARRIER();
    if constexpr (WG) {
      if (kt == nkt_c - 2) {
        const int q = ticket_slot[n & 1];
        has_next = q < total;
        if (has_next)
          nkt_n = wgrad_tile_at<TRANS_B>(q, cls, nx, cx, rect, tiles_j, p0, p1, out, K, N,
                                         row_start, ranked, tn);
        ra_nxt = rsrc_a(tn, has_next);
        rb_nxt = rsrc_b(tn, has_next);
      }
    }
    refresh(0);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      mfma(acc, i, a1, b1);
      if (!LAST && i < NF) frag(mv_c, nxt, 0, i, a0, b0);
      if constexpr (NM >= 8) {
        if (i % (NM / 8) == (NM / 8 - 1)) issue_one(cur, kr2, to_next2, i / (NM / 8));
      } else {
        issue_one(cur, kr2, to_next2, 2 * i);
        issue_one(cur, kr2, to_next2, 2 * i + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = NM; i < NF; ++i)
      if (!LAST) frag(mv_c, nxt, 0, i, a0, b0);
  };

  // Start of the streamed pipeline (the first tile, and a tile after a thin
  // one): k-tile 0 whole and the A half of k-tile 1 (its B half goes out in
  // the first step), then k-step 0's fragments.
  auto prologue = [&]() {
#pragma unroll
    for (int q = 0; q < 16; ++q) issue_one(stage(0), 0, false, q);
#pragma unroll
    for (int q = 0; q < 8; ++q) issue_one(stage(1), 1, false, q);
    TT_WAIT_VMCNT(8);
    __builtin_amdgcn_s_barrier();
    refresh(0);
#pragma unroll
    for (int i = 0; i < FM + FN; ++i)
      frag(std::integral_constant<int, FM>{}, stage(0), 0, i, a0, b0);
  };

  lds_char* const epi = (lds_char*)epi_raw + wave * P_EPI;
  // One output tile with MV blocks per wave: its k-tiles, then the epilogue
  // (rounds of the wave's blocks that hold rows).
  // The accumulators are local to a tile (and to its variant), so nothing
  // carries them from one tile, or variant, to the next.
  auto run_tile = [&](auto mv_c, int& g) {
    constexpr int MV = decltype(mv_c)::value;
    f32x16 acc[FM][FN];  // set by the first k-step; blocks mi >= MV are never read
    step(acc, 0, g, std::true_type{}, mv_c);
    ++g;
    for (int kt = 1; kt < nkt_c; ++kt, ++g) step(acc, kt, g, std::false_type{}, mv_c);
    __builtin_amdgcn_sched_barrier(0);
    store_wave_tile_p64<ET, 2, EPI_ROWS, MV>(acc, tc, tc.i0 + a_row0, tc.j0 + wn * WT, epi);
  };
  // Thin tiles (fwd / dgrad, at most 64 rows: one 32-row block per wave row)
  // stream a whole weight panel for a quarter of a tile's MFMAs, so the
  // weight loads in flight set their time. They run a pipeline of their own
  // with two weight k-tiles in flight while a third is multiplied (one in
  // the streamed pipeline): the weights in a ring of three 32 KiB slots and
  // the 64 activation rows in a ring of three 8 KiB slots, both in the stage
  // memory; one barrier per k-tile, fragment reads one k-step ahead of the
  // MFMAs. The streamed pipeline stops before such a tile (what it
  // prefetched for it is discarded) and restarts after it. An expert of at
  // most 64 rows takes its thin tiles two per schedule slot (each costs
  // about 0.6 of a full tile), so the static schedule stays balanced.
  constexpr bool THIN = !WG;
  constexpr uint32_t THIN_A = 3 * P_OPND;  // activation ring after the weight ring
  auto thin_tile = [&]() {
    TT_WAIT_VMCNT(0);  // the previous loads and stores have landed
    TT_LDS_BARRIER();  // and every wave is past its reads of the stage memory
    // Activation chunks c = 2 wave, 2 wave + 1 of the tile: rows 8 c + lane / 8.
    uint32_t tro[2];
    if constexpr (GA) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int64_t row = tc.i0 + 8 * (2 * wave + p) + (lane >> 3);
        const int64_t at = tc.seg0 + row;
        const uint32_t v = (uint32_t)arow[at < M ? at : M - 1];
        tro[p] = row < tc.nrows && v < (uint32_t)asrc_rows ? v * (uint32_t)(lda * 2) : GA_NOROW;
      }
    }
    auto thin_b = [&](int k) {  // weight k-tile k into ring slot k % 3
      const uint32_t slot = lds_addr_of(lds) + (uint32_t)(k % 3) * P_OPND;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        uint32_t vb = (q & 1) ? vodd[1] : vbase[1];
        asm volatile("" : "+v"(vb));
        uint32_t off = vb + ((uint32_t)(q >> 1) * qstep[1] + (uint32_t)k * kstep[1]);
        if constexpr (KMASK) {
          if (Lay::B_K && k * P_BK + ((q & 1) ? kof_odd : kof) >= kvalid) off = DM_OOB;
        }
        dma16(off, rb_cur, slot + (uint32_t)(8 * wave + q) * 1024u);
      }
    };
    auto thin_a = [&](int k) {  // activation k-tile k (64 rows) into ring slot k % 3
      const uint32_t slot = lds_addr_of(lds) + THIN_A + (uint32_t)(k % 3) * 8192u;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int c = 2 * wave + p;
        uint32_t off;
        if constexpr (GA) {
          off = tro[p] + (uint32_t)(2 * ((c & 1) ? kof_odd : kof)) + (uint32_t)k * kstep[0];
        } else {
          // wave 0's chunk c: this wave's chunk offsets less its 64-row origin
          off = ((c & 1) ? vodd[0] : vbase[0]) - (uint32_t)(64 * wave * lda * 2) +
                (uint32_t)(c >> 1) * qstep[0] + (uint32_t)k * kstep[0];
        }
        if constexpr (KMASK) {
          if (k * P_BK + ((c & 1) ? kof_odd : kof) >= kvalid) off = DM_OOB;
        }
        dma16(off, ra_cur, slot + (uint32_t)c * 1024u);
      }
    };
    f32x16 acc[FM][FN];  // block row 0 only
    uint4 ta[2], tb[2][FN];
    const f32x16 zero = {};
    auto thin_frags = [&](lds_char* sa, lds_char* sb, int s, int buf) {
      refresh(s);
      ta[buf] = read_k(sa, ao);
#pragma unroll
      for (int ni = 0; ni < FN; ++ni)
        tb[buf][ni] = Lay::B_K ? read_k(sb, bo - P_OPND + ni * 4096)
                               : read_mn(sb, bm[ni] - P_OPND + s * 8192);
    };
    thin_a(0);
    thin_b(0);
    thin_a(1);
    thin_b(1);
    for (int kt = 0; kt < nkt_c; ++kt) {
      // k-tile kt in (k-tile kt + 1 stays in flight), and every wave is past
      // k-tile kt - 1, whose slots the loads of k-tile kt + 2 refill.
      TT_WAIT_VMCNT(10);
      TT_LDS_BARRIER();
      thin_a(kt + 2);
      thin_b(kt + 2);
      lds_char* const sa = lds + THIN_A + (kt % 3) * 8192;
      lds_char* const sb = lds + (kt % 3) * P_OPND;
      thin_frags(sa, sb, 0, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s < 3) thin_frags(sa, sb, s + 1, (s + 1) & 1);
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
          acc[0][ni] = Mma<ET>::run(tb[s & 1][ni], ta[s & 1],
                                    (kt == 0 && s == 0) ? zero : acc[0][ni]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    store_wave_tile_p64<ET, 2, EPI_ROWS, 1>(acc, tc, tc.i0 + a_row0, tc.j0 + wn * WT, epi);
  };

  int g = 0;
  bool pro = true;  // the streamed pipeline has to start (prologue)
  for (;;) {
    // Blocks of 32 rows that hold rows of the expert, per wave row (the
    // interleaved blocks of a tile with b of them: ceil(b / 2)).
    int mv = 4;
    if constexpr (!WG) {
      const int64_t left = tc.nrows - tc.i0;
      const int nb32 = left >= DM_BM ? 8 : (int)((left + 31) / 32);
      mv = nb32 <= 2 ? 1 : (nb32 <= 4 ? 2 : 4);
    }
    if (THIN && mv == 1) {
      if constexpr (GA) {
        TT_WAIT_VMCNT(0);
        gather_offsets(ro_nxt);  // the next tile's rows, loaded at the last switch
      }
      const int nsub = tc.nsub > 0 ? tc.nsub : 1;
      for (int u = 0; u < nsub; ++u) {
        if (u > 0) {
          tc.j0 += DM_BN;
          rb_cur = rsrc_b(tc, true);
        }
        thin_tile();
      }
      pro = true;
    } else {
      if (pro) {
        // A thin tile's last loads have landed and every wave is past its
        // reads of the rings before the stages refill.
        TT_WAIT_VMCNT(0);
        TT_LDS_BARRIER();
        g = 0;
        prologue();
        pro = false;
      }
      if (mv == 4) run_tile(std::integral_constant<int, 4>{}, g);
      else if (mv == 2) run_tile(std::integral_constant<int, 2>{}, g);
      else run_tile(std::integral_constant<int, 1>{}, g);
    }
    if (!has_next) break;
    tc = tn;
    nkt_c = nkt_n;
    ra_cur = ra_nxt;
    rb_cur = rb_nxt;
    if constexpr (GA) {
#pragma unroll
      for (int q = 0; q < 8; ++q) ro_cur[q] = ro_nxt[q];
    }
    if constexpr (!WG) {
      has_next = n + 2 < ntiles;
      if (has_next)
        tile_at<MODE, TRANS_B, 2>(slot_of(n + 2), p0, p1, out, K, N, E, tiles_j, row_start,
                                  tile_start, tn);
      if constexpr (GA) gather_rows(tn, has_next, ro_nxt);
      ra_nxt = rsrc_a(tn, has_next);
      rb_nxt = rsrc_b(tn, has_next);
    } else {
      has_next = false;  // decided during the next tile
      ra_nxt = rsrc_a(tn, false);
      rb_nxt = rsrc_b(tn, false);
    }
    ++n;
    // The last k-step of the finished tile read the next tile's first
    // fragments. A tile with fewer row blocks than the next tile's variant
    // did not read the extra A blocks: read every fragment again when the
    // variants may differ.
    if (!pro) {
      refresh(0);
#pragma unroll
      for (int i = 0; i < FM + FN; ++i)
        frag(std::integral_constant<int, FM>{}, stage(g), 0, i, a0, b0);
    }
  }
  TT_WAIT_VMCNT(0);  // loads issued past the last tile land before the block exits
}

// ===========================================================================
// FP8-weight MFMA kernel (fwd / dgrad): e4m3 weights [E, N, K] with 128x128
// block scales, bf16 activations. The same 256x256x32 tiles and 4 waves as
// gmm_mfma_kernel; here every wave loads a quarter of the A tile and a
// quarter of the e4m3 B tile, then dequantises its own B rows into a bf16 B
// tile: bf16(f32(q) * f32(scale)) with the hardware e4m3 -> f32 conversion
// (exact) and round-to-nearest-even, i.e. the rule of the reference's
// offline dequantiser. The MFMA part then reads bf16 fragments as usual.
// ===========================================================================
constexpr int F8_STAGE = DM_TILE + DM_TILE / 2;  // A (bf16) + B (e4m3) of one k-tile
constexpr int F8_BUF = DM_TILE;                  // one dequantised B tile
constexpr int F8_LDS = 4 * F8_STAGE + 3 * F8_BUF;

typedef __attribute__((ext_vector_type(2))) float f32x2;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// Four e4m3 bytes -> four bf16 (two dwords), each bf16(f32(q) * s).
__device__ __forceinline__ uint2 deq4(uint32_t q, float s) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)q, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)q, true);
  const bf16x2_t a = {(__bf16)(lo.x * s), (__bf16)(lo.y * s)};
  const bf16x2_t b = {(__bf16)(hi.x * s), (__bf16)(hi.y * s)};
  return uint2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
}

template <int MODE, bool KMASK>
__global__ __launch_bounds__(DM_NT) void gmm_fp8_kernel(const char* __restrict__ p0,
                                                        const char* __restrict__ qw,
                                                        const char* __restrict__ scale, int sdt,
                                                        char* __restrict__ out, int64_t M,
                                                        int64_t K, int64_t N, int E,
                                                        const int64_t* __restrict__ counts,
                                                        int tiles_i, int tiles_j) {
  static_assert(MODE != MODE_WGRAD, "weights are the B operand");
  typedef Layout<MODE, true> Lay;  // B: K-major for fwd, MN-major for dgrad
  constexpr int WT = 128, FM = 4, FN = 4;
  __shared__ __align__(16) char lds_raw[F8_LDS];
  extern __shared__ __align__(16) char smem[];  // expert schedule, then scales
  int64_t* row_start = reinterpret_cast<int64_t*>(smem);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);

  TileDesc t;
  if (!describe_tile<DM_NT, DM_BM, DM_BN, MODE, true, 2, 1>(p0, qw, out, K, N, E, counts, tiles_i,
                                                             tiles_j, row_start, tile_start, t))
    return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int nkt = (int)((t.R + DM_BK - 1) / DM_BK);
  lds_char* const lds = (lds_char*)lds_raw;
  lds_char* const bufs = lds + 4 * F8_STAGE;

  // Block scales this tile needs, as f32 in LDS: fwd, scale rows of the two
  // 128-column blocks of the tile, all k-blocks; dgrad, the two 128-column
  // (k') blocks, all n-blocks. sc[b * nsc + i], b = block within the tile.
  const int64_t sld = (K + 127) / 128, snb = (N + 127) / 128;
  const int nsc = (int)(MODE == MODE_FWD ? sld : snb);
  float* sc = reinterpret_cast<float*>(tile_start + E + 1 + 2 * E);
  {
    const int64_t eoff = (int64_t)t.e * snb * sld;
    const int64_t b0 = t.j0 / 128;  // first 128-block of the tile's columns
    for (int idx = threadIdx.x; idx < 2 * nsc; idx += DM_NT) {
      const int b = idx / nsc, i = idx % nsc;
      const int64_t blk = b0 + b;
      int64_t off;
      if (MODE == MODE_FWD) off = eoff + (blk < snb ? blk : snb - 1) * sld + i;   // [n-block][k-block]
      else off = eoff + (int64_t)i * sld + (blk < sld ? blk : sld - 1);            // [n-block][k'-block]
      sc[idx] = sdt == TT_F32 ? reinterpret_cast<const float*>(scale)[off]
                              : bf16_to_f32(reinterpret_cast<const uint16_t*>(scale)[off]);
    }
    __syncthreads();
  }

  // ---- DMA plan: A rows 64w .. 64w + 63 (4 chunks), B e4m3 quarter (2).
  const i32x4 rsa = make_rsrc(t.a, t.nrows * t.lda * 2);
  const i32x4 rsb = make_rsrc(t.b, N * K);
  uint32_t va[4], vb[2];
  int kofa;
  const int ca = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t r = t.i0 + 64 * wave + 16 * q + (lane >> 2);
    va[q] = (uint32_t)((r * t.lda + 8 * ca) * 2);
  }
  kofa = 8 * ca;
  uint32_t kstep_b;
  int kofb;
  if constexpr (MODE == MODE_FWD) {
    // e4m3 rows j (K bytes each): chunk u covers rows 64w + 32u .. + 31,
    // lane l -> row + l / 2, bytes 16 (l & 1) .. + 15 of the k-tile.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t r = t.j0 + 64 * wave + 32 * u + (lane >> 1);
      vb[u] = (uint32_t)(r * K + 16 * (lane & 1));
    }
    kstep_b = DM_BK;
    kofb = 16 * (lane & 1);
  } else {
    // e4m3 k-rows n: chunk u covers k-rows 8w + 4u .. + 3, lane l -> k-row
    // + l / 16, columns 16 (l % 16) .. + 15.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kr = 8 * wave + 4 * u + (lane >> 4);
      vb[u] = (uint32_t)(kr * K + t.j0 + 16 * (lane & 15));
    }
    kstep_b = (uint32_t)(DM_BK * K);
    kofb = 0;
  }
  const int kvalid = (int)t.R;
  auto issue_one = [&](lds_char* stg, int kt, int q) {
    if (q < 4) {
      uint32_t off = va[q] + (uint32_t)kt * (DM_BK * 2);
      if (KMASK && kt * DM_BK + kofa >= kvalid) off = DM_OOB;
      dma16(off, rsa, lds_addr_of(stg) + (uint32_t)(4 * wave + q) * 1024u);
    } else {
      uint32_t off = vb[q - 4] + (uint32_t)kt * kstep_b;
      if (MODE == MODE_FWD && KMASK && kt * DM_BK + kofb >= kvalid) off = DM_OOB;
      dma16(off, rsb, lds_addr_of(stg) + DM_TILE + (uint32_t)(2 * wave + q - 4) * 1024u);
    }
  };

  // ---- Dequantisation of this wave's e4m3 rows of k-tile kt (stage `stg`)
  // into the bf16 B tile `buf`, in 8 parts of 4 values per lane.
  uint4 raw[2];
  float dsc;
  auto deq_read = [&](lds_char* stg, int kt) {
    if constexpr (MODE == MODE_FWD) {
      dsc = sc[(wave >> 1) * nsc + min((kt * DM_BK) / 128, nsc - 1)];
    } else {
      dsc = sc[((lane & 7) >> 2) * nsc + min((kt * DM_BK) / 128, nsc - 1)];
    }
    if constexpr (MODE == MODE_FWD) {
      const uint32_t o = (uint32_t)DM_TILE + (uint32_t)(64 * wave + lane) * 32u;
      raw[0] = read_k(stg, o);
      raw[1] = read_k(stg, o + 16);
    } else {
      const uint32_t o = (uint32_t)DM_TILE + (uint32_t)(8 * wave + (lane >> 3)) * 256u +
                         (uint32_t)(lane & 7) * 32u;
      raw[0] = read_k(stg, o);
      raw[1] = read_k(stg, o + 16);
    }
  };
  uint2 cvt[8];
  auto deq_part = [&](int part) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(raw);
    cvt[part] = deq4(w[part], dsc);
  };
  auto deq_write = [&](lds_char* buf, int half) {
    // 16 values = 2 x 16 bytes per half.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c16 = 2 * half + i;  // 8-value chunk of this lane's 32 values
      const uint4 v = uint4{cvt[2 * c16].x, cvt[2 * c16].y, cvt[2 * c16 + 1].x, cvt[2 * c16 + 1].y};
      uint32_t o;
      if constexpr (MODE == MODE_FWD) {
        const int r = 64 * wave + lane;  // B row j, K-major: 64 bytes, chunk c16
        o = (uint32_t)(r * 64 + ((c16 ^ ((r >> 2) & 3)) << 4));
      } else {
        const int kr = 8 * wave + (lane >> 3);
        const int ch = 4 * (lane & 7) + c16;  // 8-column chunk
        o = (uint32_t)(kr * 512 + ((ch ^ (4 * (kr & 3))) << 4));
      }
      *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(buf + o) =
          u32x4{v.x, v.y, v.z, v.w};
    }
  };

  // ---- Fragments.
  uint32_t a_off[2], b_off[2], b_mn[FN];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    a_off[s] = fragk_base(wm * WT, s, lane);
    b_off[s] = fragk_base(wn * WT, s, lane);
  }
#pragma unroll
  for (int ni = 0; ni < FN; ++ni) b_mn[ni] = fragmn_base(wn * WT + ni * 32, lane);
  uint32_t ao[2], bo[2], bm[FN];
  auto refresh = [&]() {
    ao[0] = a_off[0]; ao[1] = a_off[1]; bo[0] = b_off[0]; bo[1] = b_off[1];
#pragma unroll
    for (int i = 0; i < FN; ++i) bm[i] = b_mn[i];
    asm volatile("" : "+v"(ao[0]), "+v"(ao[1]));
    if constexpr (Lay::B_K) asm volatile("" : "+v"(bo[0]), "+v"(bo[1]));
    else asm volatile("" : "+v"(bm[0]), "+v"(bm[1]), "+v"(bm[2]), "+v"(bm[3]));
  };
  auto frag = [&](lds_char* stg, lds_char* buf, int s, int i, uint4 (&fa)[FM], uint4 (&fb)[FN]) {
    if (i < FM)
      fa[i] = read_k(stg, ao[s] + i * 2048);
    else
      fb[i - FM] = Lay::B_K ? read_k(buf, bo[s] + (i - FM) * 2048)
                            : read_mn(buf, bm[i - FM] + s * 8192);
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int mi = 0; mi < FM; ++mi)
#pragma unroll
    for (int ni = 0; ni < FN; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;
  auto mfma = [&](int i, const uint4 (&fa)[FM], const uint4 (&fb)[FN]) {
    acc[i / FN][i % FN] = Mma<TT_BF16>::run(fb[i % FN], fa[i / FN], acc[i / FN][i % FN]);
  };

  lds_char* const s0 = lds;
  lds_char* const s1 = lds + F8_STAGE;
  lds_char* const s2 = lds + 2 * F8_STAGE;
  lds_char* const s3 = lds + 3 * F8_STAGE;
  auto buf_of = [&](int kt) { return bufs + (kt % 3) * F8_BUF; };
  uint4 a0[FM], b0[FN], a1[FM], b1[FN];

  // k-tile kt: wait for this wave's loads of k-tile kt+1; multiply k-step 0
  // while reading k-step 1 and dequantising this wave's rows of k-tile kt+1;
  // barrier (k-tile kt+1 complete in LDS, A and bf16 B); multiply k-step 1
  // while reading k-step 0 of k-tile kt+1 and loading k-tile kt+3 into the
  // stage of k-tile kt-1. Three bf16 B tiles rotate, so a tile is rewritten
  // only after every wave has finished the k-tile before.
  auto step = [&](int kt, lds_char* cur, lds_char* nxt, lds_char* refill) {
    lds_char* const bc = buf_of(kt);
    lds_char* const bn = buf_of(kt + 1);
    TT_WAIT_VMCNT(6);
    refresh();
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
      mfma(i, a0, b0);
      if (i < FM + FN) frag(cur, bc, 1, i, a1, b1);
      if (i == 1) deq_read(nxt, kt + 1);
      if (i >= 4 && i < 12) deq_part(i - 4);
      if (i == 8) deq_write(bn, 0);
      if (i == 12) deq_write(bn, 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    TT_LDS_BARRIER();
    refresh();
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
      mfma(i, a1, b1);
      if (i < FM + FN) frag(nxt, bn, 0, i, a0, b0);
      if (i < 6) issue_one(refill, kt + 3, i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

#pragma unroll
  for (int q = 0; q < 6; ++q) issue_one(s0, 0, q);
#pragma unroll
  for (int q = 0; q < 6; ++q) issue_one(s1, 1, q);
#pragma unroll
  for (int q = 0; q < 6; ++q) issue_one(s2, 2, q);
  TT_WAIT_VMCNT(12);  // this wave's loads of k-tile 0
  deq_read(s0, 0);
#pragma unroll
  for (int part = 0; part < 8; ++part) deq_part(part);
  deq_write(buf_of(0), 0);
  deq_write(buf_of(0), 1);
  TT_LDS_BARRIER();
  refresh();
#pragma unroll
  for (int i = 0; i < FM + FN; ++i) frag(s0, buf_of(0), 0, i, a0, b0);
  for (int kt = 0; kt < nkt; kt += DM_ST) {
    step(kt, s0, s1, s3);
    if (kt + 1 < nkt) step(kt + 1, s1, s2, s0);
    if (kt + 2 < nkt) step(kt + 2, s2, s3, s1);
    if (kt + 3 < nkt) step(kt + 3, s3, s0, s2);
  }
  TT_WAIT_VMCNT(0);
  __syncthreads();
  store_wave_tile<TT_BF16>(acc, t, t.i0 + wm * WT, t.j0 + wn * WT, lane, lds + wave * 32768);
}

// ---------------------------------------------------------------------------
// fp32 path (toy shapes and fp32 models): 64x64 tiles, 4x4 outputs per thread.
// ---------------------------------------------------------------------------
// ===========================================================================
// Persistent FP8-weight kernel (fwd / dgrad): e4m3 weights [E, N, K] with
// 128x128 block scales, bf16 activations, 128x512x64 output tiles. The four
// waves share the tile's 128 rows and take 128 columns each, so an expert's
// rows are padded to a multiple of 128 only; per 64-deep k-tile the block
// loads 16 KiB of activations and 32 KiB of e4m3 weights (the bytes of a
// 256x256 tile with bf16 A and e4m3 B). The weights stay e4m3 in LDS: each
// wave reads its own B fragments as e4m3 bytes (plain 8-byte reads of
// K-major rows in fwd; gfx950 transposing 8-bit reads of N-major rows in
// dgrad) and dequantises them in registers, bf16(f32(q) * f32(scale)) with
// the hardware e4m3 -> f32 decode and round-to-nearest-even. A wave's 128
// columns lie in one 128-column scale block, so it needs one scale per
// k-tile, read from a private LDS row filled at the tile switch (prefetched
// into a register one tile ahead). Otherwise the persistent schedule and the
// two-stage pipeline are those of gmm_p64_kernel.
// ===========================================================================
constexpr int Q_BM = 128, Q_BN = 512, Q_BK = 64;
constexpr int Q_A = Q_BM * Q_BK * 2;  // A tile, bf16 (16 KiB)
constexpr int Q_B = Q_BN * Q_BK;      // B tile, e4m3 (32 KiB)
constexpr int Q_STAGE = Q_A + Q_B;
constexpr int Q_SMAX = 128;           // scale blocks along the reduction

// Output tile L of the 128x512 schedule (slot-major, n-tile minor).
template <int MODE>
__device__ __forceinline__ void q8_tile_at(int L, const char* p0, const char* qw, char* out,
                                           int64_t K, int64_t N, int E, int tiles_j,
                                           const int64_t* row_start, const int* tile_start,
                                           TileDesc& t) {
  const int slot = L / tiles_j, jt = L % tiles_j;
  int lo = 0, hi = E - 1;  // last e with tile_start[e] <= slot
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile_start[mid] <= slot) lo = mid; else hi = mid - 1;
  }
  const int e = __builtin_amdgcn_readfirstlane(lo);
  t.e = e;
  t.seg0 = rfl64(row_start[e]);
  t.nrows = rfl64(row_start[e + 1]) - t.seg0;
  const int ts_e = __builtin_amdgcn_readfirstlane(tile_start[e]);
  t.b = qw + (int64_t)e * N * K;
  if constexpr (MODE == MODE_FWD) {
    t.a = p0 + t.seg0 * K * 2; t.lda = K;
    t.I = t.nrows; t.J = N; t.R = K;
    t.c = out + t.seg0 * N * 2; t.ldc = N;
  } else {
    t.a = p0 + t.seg0 * N * 2; t.lda = N;
    t.I = t.nrows; t.J = K; t.R = N;
    t.c = out + t.seg0 * K * 2; t.ldc = K;
  }
  t.ldb = K;
  t.i0 = (int64_t)(slot - ts_e) * Q_BM;
  t.j0 = (int64_t)jt * Q_BN;
}

// Eight e4m3 bytes (k order) -> one bf16 B fragment.
__device__ __forceinline__ uint4 deq8(uint2 q, float s) {
  const uint2 lo = deq4(q.x, s), hi = deq4(q.y, s);
  return uint4{lo.x, lo.y, hi.x, hi.y};
}

template <int MODE, bool KMASK>
__global__ __launch_bounds__(DM_NT) void gmm_q8_kernel(const char* __restrict__ p0,
                                                       const char* __restrict__ qw,
                                                       const char* __restrict__ scale, int sdt,
                                                       char* __restrict__ out, int64_t M,
                                                       int64_t K, int64_t N, int E,
                                                       const int64_t* __restrict__ counts,
                                                       int tiles_j) {
  static_assert(MODE != MODE_WGRAD, "weights are the B operand");
  constexpr int FM = 4, FN = 4;
  __shared__ __align__(16) char lds_raw[2 * Q_STAGE];
  __shared__ __align__(16) char epi_raw[4 * P_EPI];
  __shared__ float sc_raw[4 * Q_SMAX];
  extern __shared__ __align__(16) char smem[];  // expert schedule
  int64_t* row_start = reinterpret_cast<int64_t*>(smem);
  int* tile_start = reinterpret_cast<int*>(row_start + E + 1);
  scan_counts<DM_NT>(counts, E, Q_BM, row_start, tile_start);

  const int G = gridDim.x;
  const int pos = xcd_remap(blockIdx.x, G);
  const int total = tile_start[E] * tiles_j;
  if (pos >= total) return;
  const int ntiles = (total - pos + G - 1) / G;
  const int64_t R = MODE == MODE_FWD ? K : N;  // reduction length
  const int nkt = (int)((R + Q_BK - 1) / Q_BK);  // >= 2 (host check)
  const int64_t snb = (N + 127) / 128, skb = (K + 127) / 128;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t lda = MODE == MODE_FWD ? K : N;

  // ---- Loads (offsets relative to the tile origin, the resource base).
  // A (K-major, 128 rows of 128 bytes per k-tile): chunk q (0-3) of wave w
  // covers rows 32 w + 8 q + lane / 8, LDS slot lane % 8 holding k-chunk
  // slot ^ ((row >> 1) & 7); the swizzle alternates with q's parity.
  // B fwd (K-major e4m3, 512 rows of 64 bytes): chunk q (0-7) of wave w
  // covers rows 128 w + 16 q + lane / 4, slot lane % 4 holding k-chunk
  // slot ^ ((row >> 2) & 3) = (lane % 4) ^ (lane / 16 % 4).
  // B dgrad (N-major e4m3, 64 k-rows of 512 bytes): chunk q of wave w covers
  // k-rows 16 w + 2 q + lane / 32, slot lane % 32 holding column chunk
  // slot ^ ((k-row % 8) << 1); the swizzle repeats every four chunks.
  uint32_t a_even, a_odd, b_base[4];
  int a_kof_even, a_kof_odd, b_kof = 0;
  {
    const int r = 32 * wave + (lane >> 3);
    const int c = (lane & 7) ^ (lane >> 4);
    const int c1 = c ^ 4;
    a_even = (uint32_t)(((int64_t)r * lda + 8 * c) * 2);
    a_odd = (uint32_t)(((int64_t)(r + 8) * lda + 8 * c1) * 2);
    a_kof_even = 8 * c;
    a_kof_odd = 8 * c1;
  }
  if constexpr (MODE == MODE_FWD) {
    const int j = 128 * wave + (lane >> 2);
    const int c = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
    for (int h = 0; h < 4; ++h) b_base[h] = (uint32_t)((int64_t)j * K + 16 * c);
    b_kof = 16 * c;
  } else {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int kr = 16 * wave + 2 * h + (lane >> 5);  // chunk q = 4 q' + h
      const int c = (lane & 31) ^ ((kr & 7) << 1);
      b_base[h] = (uint32_t)((int64_t)kr * K + 16 * c);
    }
  }
  const uint32_t a_qstep = (uint32_t)(16 * lda * 2);  // A: per pair of chunks
  // B: per chunk (fwd, 16 rows) or per four chunks (dgrad, 8 k-rows).
  const uint32_t b_qstep = MODE == MODE_FWD ? (uint32_t)(16 * K) : (uint32_t)(8 * K);
  const uint32_t b_kstep = MODE == MODE_FWD ? (uint32_t)Q_BK : (uint32_t)(Q_BK * K);
  // Each chunk's offset from the tile origin, fixed for the launch: a load
  // needs no vector arithmetic; the k-tile moves the buffer resource instead
  // (scalar arithmetic, range checks unchanged).
  uint32_t a_chunk[4], b_chunk[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) a_chunk[q] = ((q & 1) ? a_odd : a_even) + (uint32_t)(q >> 1) * a_qstep;
#pragma unroll
  for (int qb = 0; qb < 8; ++qb)
    b_chunk[qb] = (MODE == MODE_FWD ? b_base[0] : b_base[qb & 3]) +
                  (uint32_t)(MODE == MODE_FWD ? qb : qb >> 2) * b_qstep;

  auto rsrc_a = [&](const TileDesc& t, bool valid) -> i32x4 {
    if (!valid) return make_rsrc(p0, 0);
    const int64_t toff = t.i0 * t.lda * 2;
    return make_rsrc(t.a + toff, t.nrows * t.lda * 2 - toff);
  };
  auto rsrc_b = [&](const TileDesc& t, bool valid) -> i32x4 {
    if (!valid) return make_rsrc(p0, 0);
    const int64_t toff = MODE == MODE_FWD ? t.j0 * K : t.j0;
    return make_rsrc(t.b + toff, N * K - toff);
  };

  TileDesc tc, tn;
  q8_tile_at<MODE>(pos, p0, qw, out, K, N, E, tiles_j, row_start, tile_start, tc);
  bool has_next = ntiles > 1;
  if (has_next) q8_tile_at<MODE>(pos + G, p0, qw, out, K, N, E, tiles_j, row_start, tile_start, tn);
  i32x4 ra_cur = rsrc_a(tc, true), rb_cur = rsrc_b(tc, true);
  i32x4 ra_nxt = rsrc_a(tn, has_next), rb_nxt = rsrc_b(tn, has_next);
  const int kvalid = (int)R;

  // Scales of this wave's 128-column block along the reduction: fwd,
  // scale[e][(j0 + 128 w) / 128][kb]; dgrad, scale[e][nb][(j0 + 128 w) / 128].
  const int nsc = (int)(MODE == MODE_FWD ? skb : snb);
  auto load_scales = [&](const TileDesc& t, float (&v)[2]) {
    const int64_t colblk = (t.j0 + 128 * wave) / 128;
    const int64_t cb = MODE == MODE_FWD ? (colblk < snb ? colblk : snb - 1)
                                        : (colblk < skb ? colblk : skb - 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = lane + 64 * h;
      v[h] = 1.0f;
      if (i < nsc) {
        const int64_t off = (int64_t)t.e * snb * skb +
                            (MODE == MODE_FWD ? cb * skb + i : (int64_t)i * skb + cb);
        v[h] = sdt == TT_F32 ? reinterpret_cast<const float*>(scale)[off]
                             : bf16_to_f32(reinterpret_cast<const uint16_t*>(scale)[off]);
      }
    }
  };
  float* const sc_w = sc_raw + wave * Q_SMAX;
  float sv_next[2];
  {
    float v[2];
    load_scales(tc, v);
    sc_w[lane] = v[0];
    sc_w[lane + 64] = v[1];
  }
  if (has_next) load_scales(tn, sv_next);

  // Chunk q (0-3 A, 4-11 B) of k-tile k of the current or next tile.
  auto issue_one = [&](lds_char* stg, int k, bool nxt, int q) {
    uint32_t off, dst;
    i32x4 rs;
    if (q < 4) {
      off = a_chunk[q];
      if constexpr (KMASK) {
        if (k * Q_BK + ((q & 1) ? a_kof_odd : a_kof_even) >= kvalid) off = DM_OOB;
      }
      rs = advance_rsrc(nxt ? ra_nxt : ra_cur, (uint32_t)k * (Q_BK * 2));
      dst = (uint32_t)(4 * wave + q) * 1024u;
    } else {
      const int qb = q - 4;
      off = b_chunk[qb];
      if constexpr (KMASK && MODE == MODE_FWD) {
        if (k * Q_BK + b_kof >= kvalid) off = DM_OOB;
      }
      rs = advance_rsrc(nxt ? rb_nxt : rb_cur, (uint32_t)k * b_kstep);
      dst = (uint32_t)Q_A + (uint32_t)(8 * wave + qb) * 1024u;
    }
    dma16(off, rs, lds_addr_of(stg) + dst);
  };

  // Fragment offsets. A: rows 32 mi + lane % 32 (fragk64). B fwd: row
  // 128 w + 32 ni + lane % 32, bytes 16 s + 8 (lane / 32) of its 64, chunk
  // swizzled by (lane / 4) % 4; ni adds 2048. B dgrad: 16-lane group g,
  // index i: k-row 16 s + 8 (g / 2) + i / 2, columns 128 w + 32 ni +
  // 16 (g % 2) + 8 (i % 2); ni adds 64 (two chunks; the row swizzle only
  // touches chunk bits 1-3, so it commutes with +2 chunks when ni is even,
  // and the swizzled chunk of block ni is computed per ni below).
  uint32_t a_k[4], b_f[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a_k[s] = fragk64(0, s, lane);
    if constexpr (MODE == MODE_FWD) {
      const int f = (lane >> 2) & 3;
      b_f[s] = (uint32_t)Q_A + (uint32_t)(128 * wave + (lane & 31)) * 64u +
               (uint32_t)((s ^ f) << 4) + 8u * (uint32_t)(lane >> 5);
    } else {
      const int g = lane >> 4, i = lane & 15;
      const int kr = 16 * s + 8 * (g >> 1) + (i >> 1);
      b_f[s] = (uint32_t)Q_A + (uint32_t)kr * 512u + 8u * (uint32_t)(i & 1);
    }
  }
  // dgrad: physical chunk of column chunk c at k-row kr is c ^ ((kr % 8) << 1);
  // per fragment (s, ni) the lane's logical chunk is 8 w + 2 ni + g % 2.
  auto b_off = [&](int s, int ni) -> uint32_t {
    if constexpr (MODE == MODE_FWD) {
      return b_f[s] + (uint32_t)ni * 2048u;
    } else {
      const int g = lane >> 4, i = lane & 15;
      const int c = 8 * wave + 2 * ni + (g & 1);
      const int p = c ^ (((i >> 1) & 7) << 1);
      return b_f[s] + (uint32_t)p * 16u;
    }
  };

  f32x16 acc[FM][FN];
  uint32_t ao, bo[FN];
  uint32_t b_d[FN];  // dgrad: B fragment offsets of k-step 0
#pragma unroll
  for (int i = 0; i < FN; ++i) b_d[i] = MODE == MODE_FWD ? 0u : b_off(0, i);
  auto refresh = [&](int s) {
    asm volatile("" : "+v"(a_k[s]));
    ao = a_k[s];
    if constexpr (MODE == MODE_FWD) {
      // One opaque register per k-step; the column blocks are immediate offsets.
      asm volatile("" : "+v"(b_f[s]));
#pragma unroll
      for (int i = 0; i < FN; ++i) bo[i] = b_off(s, i);
    } else {
      // b_off(s, ni) = b_off(0, ni) + 8192 s: four opaque registers for the
      // column blocks, the k-step an immediate offset.
      asm volatile("" : "+v"(b_d[0]), "+v"(b_d[1]), "+v"(b_d[2]), "+v"(b_d[3]));
#pragma unroll
      for (int i = 0; i < FN; ++i) bo[i] = b_d[i] + (uint32_t)s * 8192u;
    }
  };
  auto read_b8 = [&](lds_char* stg, uint32_t off) -> uint2 {
    if constexpr (MODE == MODE_FWD) {
      return __builtin_bit_cast(uint2, *reinterpret_cast<const lds_u32x2*>(stg + off));
    } else {
      typedef __attribute__((ext_vector_type(2))) int i32x2_t;
      typedef __attribute__((address_space(3))) i32x2_t lds_i32x2;
      const i32x2_t v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(stg + off));
      return __builtin_bit_cast(uint2, v);
    }
  };
  // Fragment unit i (0-3 A block i, 4-7 raw B block i - 4) of the current k-step.
  auto frag = [&](lds_char* stg, int i, uint4 (&fa)[FM], uint2 (&rb)[FN]) {
    if (i < FM) fa[i] = read_k(stg, ao + i * 4096);
    else rb[i - FM] = read_b8(stg, bo[i - FM]);
  };
  auto mfma = [&](int i, const uint4 (&fa)[FM], const uint4 (&fb)[FN]) {
    acc[i / FN][i % FN] = Mma<TT_BF16>::run(fb[i % FN], fa[i / FN], acc[i / FN][i % FN]);
  };
  // Dequantisation part h (0-7): half h % 2 of raw B fragment h / 2.
  auto deq_half = [&](int h, const uint2 (&rb)[FN], uint4 (&fb)[FN], float sc) {
    const int u = h >> 1;
    if (h & 1) {
      const uint2 v = deq4(rb[u].y, sc);
      fb[u].z = v.x;
      fb[u].w = v.y;
    } else {
      const uint2 v = deq4(rb[u].x, sc);
      fb[u].x = v.x;
      fb[u].y = v.y;
    }
  };

  lds_char* const lds = (lds_char*)lds_raw;
  auto stage = [&](int g) { return lds + (g & 1) * Q_STAGE; };
  uint4 a0[FM], b0[FN], a1[FM], b1[FN];
  uint2 r0[FN], r1[FN];
  float s_cur = 1.0f;  // scale of the k-tile being read

  // One k-tile, as in gmm_p64_kernel but with the operands' load slots
  // swapped: k-steps 0-2 multiply while reading (and dequantising) the next
  // k-step, k-steps 0-1 also load the A tile of k-tile kt + 1 into the other
  // stage (one load every eighth slot); wait for k-tile kt + 1, barrier;
  // k-step 3 multiplies while reading k-step 0 of k-tile kt + 1 and loading
  // the e4m3 B tile of k-tile kt + 2 into this stage (one load every other
  // slot). The weights, which stream from HBM once per tile, so get about four
  // k-steps of latency cover and the activations (mostly L2 hits) one or two
  // (fwd / dgrad 2-4 % faster than the other way round on DeepSeek-V3).
  // Raw e4m3 fragments are read in slots 0-7 and dequantised in slots 8-15.
  auto step = [&](int kt, int g, auto last_c) {
    constexpr bool LAST = decltype(last_c)::value;
    lds_char* const cur = stage(g);
    lds_char* const nxt = stage(g + 1);
    const int k1 = kt + 1, k2 = kt + 2;
    const bool to_next1 = k1 >= nkt, to_next2 = k2 >= nkt;
    const int kr1 = to_next1 ? k1 - nkt : k1;
    const int kr2 = to_next2 ? k2 - nkt : k2;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      refresh(s + 1);
#pragma unroll
      for (int i = 0; i < FM * FN; ++i) {
        if (s & 1) mfma(i, a1, b1); else mfma(i, a0, b0);
        if (i < FM + FN) {
          if (s & 1) frag(cur, i, a0, r0); else frag(cur, i, a1, r1);
        } else {
          if (s & 1) deq_half(i - 8, r0, b0, s_cur); else deq_half(i - 8, r1, b1, s_cur);
        }
        if (s <= 1 && (i & 7) == 1) issue_one(nxt, kr1, to_next1, 2 * s + (i >> 3));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    TT_WAIT_VMCNT(0);
    TT_LDS_BARRIER();
    // Scale of the k-tile whose k-step 0 is read next (the next k-tile, or the
    // next tile's first, whose scales replace this wave's row after the
    // epilogue).
    const float s_next = LAST ? 1.0f : sc_w[(kt + 1) >> 1];
    refresh(0);
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
      mfma(i, a1, b1);
      if (!LAST && i < FM + FN) frag(nxt, i, a0, r0);
      if (!LAST && i >= FM + FN) deq_half(i - 8, r0, b0, s_next);
      if ((i & 1) == 1) issue_one(cur, kr2, to_next2, 4 + (i >> 1));
      __builtin_amdgcn_sched_barrier(0);
    }
    s_cur = s_next;
  };

  // k-tile 0 whole and the B part of k-tile 1.
#pragma unroll
  for (int q = 0; q < 12; ++q) issue_one(stage(0), 0, false, q);
#pragma unroll
  for (int q = 4; q < 12; ++q) issue_one(stage(1), 1, false, q);
  TT_WAIT_VMCNT(8);
  __builtin_amdgcn_s_barrier();

  lds_char* const epi = (lds_char*)epi_raw + wave * P_EPI;
  int g = 0;
  for (int n = 0;;) {
    // k-step 0 of the tile's first k-tile.
    s_cur = sc_w[0];
    refresh(0);
#pragma unroll
    for (int i = 0; i < FM + FN; ++i) frag(stage(g), i, a0, r0);
#pragma unroll
    for (int u = 0; u < FN; ++u) b0[u] = deq8(r0[u], s_cur);
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
      for (int ni = 0; ni < FN; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;
    for (int kt = 0; kt < nkt - 1; ++kt, ++g) step(kt, g, std::false_type{});
    step(nkt - 1, g, std::true_type{});
    ++g;
    __builtin_amdgcn_sched_barrier(0);
    store_wave_tile_p64<TT_BF16, 2, 32, 4>(acc, tc, tc.i0, tc.j0 + 128 * wave, epi);
    if (++n == ntiles) break;
    tc = tn;
    ra_cur = ra_nxt;
    rb_cur = rb_nxt;
    sc_w[lane] = sv_next[0];
    sc_w[lane + 64] = sv_next[1];
    has_next = n + 1 < ntiles;
    if (has_next) {
      q8_tile_at<MODE>(pos + (n + 1) * G, p0, qw, out, K, N, E, tiles_j, row_start, tile_start,
                       tn);
      load_scales(tn, sv_next);
    }
    ra_nxt = rsrc_a(tn, has_next);
    rb_nxt = rsrc_b(tn, has_next);
  }
  TT_WAIT_VMCNT(0);  // loads issued past the last tile land before the block exits
}

// fp32 operands (the toy configuration, fp32 LoRA adapters): 64x64 output
// tiles, each wave one 32x32 block on v_mfma_f32_32x32x2_f32 (full fp32
// products and sums, fp32 accumulation). A 16-deep k-tile is staged in LDS as
// [k][row] and [k][col]; MFMA step s takes k = s (lanes 0-31) and k = s + 8
// (lanes 32-63). B goes in as the first operand, so each lane ends with one
// output row and four consecutive columns per group (16-byte stores).
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;  // the wave's 32x32 block
  const int l32 = lane & 31, h = lane >> 5;
  f32x16 acc = {};
  for (int64_t k0 = 0; k0 < R; k0 += BKF) {
    for (int q = threadIdx.x; q < BKF * BT; q += 256) {
      const int kk = q / BT, rr = q % BT;
      const int64_t gk = k0 + kk, gi = i0 + rr, gj = j0 + rr;
      sa[kk][rr] = (gk < R && gi < I) ? (Lay::A_K ? A[gi * lda + gk] : A[gk * lda + gi]) : 0.f;
      sb[kk][rr] = (gk < R && gj < J) ? (Lay::B_K ? B[gj * ldb + gk] : B[gk * ldb + gj]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < BKF / 2; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(sb[s + 8 * h][wc + l32], sa[s + 8 * h][wr + l32],
                                                 acc, 0, 0, 0);
    __syncthreads();
  }
  const int64_t gi = i0 + wr + l32;
  if (gi >= I) return;
  float* row = Cp + gi * t.ldc;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t gj = j0 + wc + 8 * g + 4 * h;
    if (gj + 3 < J && ((t.ldc | gj) & 3) == 0) {
      *reinterpret_cast<float4*>(row + gj) = float4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2],
                                                    acc[4 * g + 3]};
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (gj + v < J) row[gj + v] = acc[4 * g + v];
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Expert schedule in dynamic LDS: row starts (int64), m-tile starts (int),
// and for the weight-gradient ranking int32 counts and ranks.
size_t schedule_bytes(int E) {
  return (size_t)(E + 1) * (sizeof(int64_t) + sizeof(int)) + (size_t)E * 2 * sizeof(int) + 64;
}

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

// Slot of the next weight-gradient launch (either kernel), in turn over all
// launches of the process.
int next_wgrad_slot() {
  static std::atomic<unsigned> next{0};
  return (int)(next.fetch_add(1, std::memory_order_relaxed) % WQ_SLOTS);
}

template <int MODE, bool TB, int ET, bool KMASK, int GX = 0>
int launch_mfma_k(const void* p0, const void* p1, void* out, int64_t M, int64_t K, int64_t N,
                  int E, const int64_t* counts, hipStream_t s, int64_t nblk, int ti, int tj,
                  const int32_t* grow = nullptr, int64_t gsrc_rows = 0) {
  // Weight gradients on XCD pairs: eight blocks per group of eight expert
  // ranks and tile (see describe_tile).
  if (MODE == MODE_WGRAD && wgrad_pair_split(ti, tj) != 0)
    nblk = 8 * (int64_t)((E + 7) / 8) * ti * tj;
  // Weight gradients: the expert ranking once per launch, into a slot of its
  // own, on the launch stream; the blocks then need no schedule in LDS.
  int rslot = -1;
  if (MODE == MODE_WGRAD && E <= WR_MAX_E) {
    rslot = next_wgrad_slot();
    hipLaunchKernelGGL(wgrad_rank_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, s,
                       counts, E, rslot);
    const int rr = tt_check_launch("gmm");
    if (rr != TT_OK) return rr;
  }
  const size_t lds = rslot >= 0 ? 0 : schedule_bytes(E);  // the stages are static LDS
  static size_t allowed = 64 * 1024;
  const int rc = allow_lds(&gmm_mfma_kernel<MODE, TB, ET, KMASK, GX>, lds, allowed);
  if (rc != TT_OK) return rc;
  hipLaunchKernelGGL((gmm_mfma_kernel<MODE, TB, ET, KMASK, GX>), dim3((unsigned)nblk),
                     dim3(DM_NT), lds, s, static_cast<const char*>(p0),
                     static_cast<const char*>(p1), static_cast<char*>(out), M, K, N, E, counts,
                     ti, tj, grow, gsrc_rows, rslot);
  return tt_check_launch("gmm");
}

// Compute units of the current device (the persistent kernel's grid), cached
// per device.
int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Dynamic LDS of the persistent kernel: the expert schedule plus the expert
// ranking of wgrad.
size_t p64_schedule_bytes(int E) { return schedule_bytes(E) + (size_t)E * sizeof(int); }
// All LDS of the persistent kernel: stages, epilogue staging, the dynamic
// schedule and about 1 KiB of small static arrays (tickets, scan partials,
// the cost-sorted schedule's slot lists).
size_t p64_lds_bytes(int E) { return p64_schedule_bytes(E) + 2 * P_STAGE + 4 * P_EPI + 1024; }

// Weight gradients (ti x tj output tiles per expert) run on the persistent
// kernel for short reductions (few rows per expert on average, known without
// the counts), and for experts of at least P_WGRAD_TILES output tiles: it
// spreads an expert's tiles over the eight XCDs in rectangles that share
// operand panels and overlaps each tile's epilogue with the next tile's
// loads, while the one-tile-per-block kernel keeps an expert's tiles on one
// pair of XCDs, which pays for smaller tile grids. Measured on packed
// operands with the layers' own routing, launches alternated (bit-identical
// either way), persistent against one tile per block: Mixtral fc1 (1792
// tiles per expert) 3519 against 3650 us, fc2 (896) 1676 against 1663 us;
// Qwen3-30B-A3B fc1 (48) 860 against 842 us, fc2 (24) 516 against 443 us;
// the varlen stress layer's fc1 (48) 3276 against 2974 us.
bool wgrad_persistent(int64_t M, int64_t K, int64_t N, int E, int ti, int tj) {
  const int64_t ld = K > N ? K : N;
  return (M <= (int64_t)E * P_WGRAD_ROWS || (int64_t)ti * tj >= P_WGRAD_TILES) &&
         p64_lds_bytes(E) <= 160 * 1024 &&
         (M + 2 * P_BK) * ld * 2 < (int64_t)DM_OOB;
}

template <int MODE, bool TB, int ET, bool KMASK, bool GA = false>
int launch_p64_k(const void* p0, const void* p1, void* out, int64_t M, int64_t K, int64_t N,
                 int E, const int64_t* counts, hipStream_t s, int64_t nblk, int ti, int tj,
                 const int32_t* arow = nullptr, int64_t asrc_rows = 0) {
  const size_t lds = p64_schedule_bytes(E);  // stages and epilogue staging are static LDS
  static size_t allowed = 64 * 1024;
  const int rc = allow_lds(&gmm_p64_kernel<MODE, TB, ET, KMASK, GA>, lds, allowed);
  if (rc != TT_OK) return rc;
  int slot = 0;
  if constexpr (MODE == MODE_WGRAD) {
    // A queue slot of its own for this launch, zeroed on the launch stream.
    slot = next_wgrad_slot();
    hipLaunchKernelGGL(wgrad_queue_reset_kernel, dim3(1), dim3(64), 0, s, slot);
    const int rq = tt_check_launch("gmm");
    if (rq != TT_OK) return rq;
  }
  const int64_t cus = cu_count();
  const int64_t grid = nblk < cus ? nblk : cus;
  hipLaunchKernelGGL((gmm_p64_kernel<MODE, TB, ET, KMASK, GA>), dim3((unsigned)grid),
                     dim3(DM_NT), lds, s, static_cast<const char*>(p0),
                     static_cast<const char*>(p1), static_cast<char*>(out), M, K, N, E, counts,
                     ti, tj, slot, arow, asrc_rows);
  return tt_check_launch("gmm");
}

template <int MODE, bool TB, int ET>
int launch_mfma(const void* p0, const void* p1, void* out, int64_t M, int64_t K, int64_t N,
                int E, const int64_t* counts, hipStream_t s) {
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE, TB, M, K, N, E, DM_BM, DM_BN, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  TT_REQUIRE(schedule_bytes(E) + (size_t)DM_ST * DM_STAGE <= 160 * 1024,
             "gmm: too many experts for the LDS tile schedule");
  // Operands are addressed through 32-bit buffer offsets: every activation
  // matrix (plus a tile of overhang) and every expert weight must stay below
  // 4 GiB.
  const int64_t ld = K > N ? K : N;
  TT_REQUIRE((M + DM_BM) * ld * 2 < (int64_t)DM_OOB && K * N * 2 < (int64_t)DM_OOB,
             "gmm: operands of 4 GiB or more are not supported (M=%lld K=%lld N=%lld)",
             (long long)M, (long long)K, (long long)N);
  const int64_t R = MODE == MODE_FWD ? K : N;  // reduction length of fwd / dgrad
  const bool p64_lds = p64_lds_bytes(E) <= 160 * 1024;
  if constexpr (MODE != MODE_WGRAD) {
    // The persistent kernel needs two k-tiles per output tile, its LDS
    // (stages, epilogue staging, schedule) and 32-bit offsets for loads that
    // run up to two k-tiles past the reduction end.
    if (R > P_BK && p64_lds && (R + 2 * P_BK) * ld * 2 < (int64_t)DM_OOB) {
      if (R % P_BK)
        return launch_p64_k<MODE, TB, ET, true>(p0, p1, out, M, K, N, E, counts, s, nblk, ti,
                                                tj);
      return launch_p64_k<MODE, TB, ET, false>(p0, p1, out, M, K, N, E, counts, s, nblk, ti,
                                               tj);
    }
  } else {
    // The persistent kernel for short reductions and large tile grids (see
    // wgrad_persistent), the four-stage one-tile-per-block kernel otherwise.
    // wgrad reduces over each expert's rows (at most M; the loads run up to
    // two k-tiles past an expert's end).
    if (wgrad_persistent(M, K, N, E, ti, tj))
      return launch_p64_k<MODE, TB, ET, false>(p0, p1, out, M, K, N, E, counts, s, nblk, ti, tj);
  }
  if (MODE != MODE_WGRAD && R % DM_BK)
    return launch_mfma_k<MODE, TB, ET, true>(p0, p1, out, M, K, N, E, counts, s, nblk, ti, tj);
  return launch_mfma_k<MODE, TB, ET, false>(p0, p1, out, M, K, N, E, counts, s, nblk, ti, tj);
}

// Shape limits of the gathering launches, shared by the launchers and
// tt_gmm_gather_supported: nullptr when the problem is taken, else what
// rules it out.
const char* gather_limit(int MODE, int64_t src_rows, int64_t M, int64_t K, int64_t N, int E) {
  const int64_t R = MODE == MODE_FWD ? K : N;  // reduction length = source row length
  const int64_t J = MODE == MODE_FWD ? N : K;  // output width
  if (!(R > P_BK && R % P_BK == 0))
    return "the reduction length must be a multiple of 64 above 64";
  if (p64_lds_bytes(E) > 160 * 1024)
    return "too many experts for the LDS tile schedule";
  if (!(src_rows >= 1 && (src_rows * R + 4 * P_BK) * 2 < (int64_t)GA_NOROW))
    return "the source must hold at least one row and less than 2 GiB";
  if (!((M + DM_BM) * J * 2 < (int64_t)DM_OOB && K * N * 2 < (int64_t)DM_OOB &&
        (R + 2 * P_BK) * J * 2 < (int64_t)DM_OOB))
    return "operands of 4 GiB or more are not supported";
  return nullptr;
}
// GX: 1 when the rows of x are gathered, 2 for the rows of dy.
const char* wgrad_gather_limit(int GX, int64_t src_rows, int64_t M, int64_t K, int64_t N, int E) {
  if (!(M > (int64_t)E * P_WGRAD_ROWS))
    return "weight gradients with gathered rows need more than 512 rows per expert on average";
  if (schedule_bytes(E) + (size_t)DM_ST * DM_STAGE + 1024 > 160 * 1024)
    return "too many experts for the LDS tile schedule";
  const int64_t ld = K > N ? K : N;
  if (!((M + DM_BM) * ld * 2 < (int64_t)DM_OOB && K * N * 2 < (int64_t)DM_OOB &&
        M * 4 < (int64_t)DM_OOB))
    return "operands of 4 GiB or more are not supported";
  const int64_t gld = GX == 1 ? K : N;
  if (!(src_rows >= 1 && (src_rows + 1) * gld * 2 < (int64_t)DM_OOB))
    return "the source must hold at least one row and less than 4 GiB";
  if (!(src_rows < (1 << 24) && gld * 2 < (1 << 24)))
    return "the source must hold fewer than 2^24 rows of fewer than 2^23 elements";
  return nullptr;
}

// fwd / dgrad with gathered A rows (persistent kernel only): A row r is row
// arow[r] of src ([src_rows, R], R the reduction length).
template <int MODE, bool TB, int ET>
int launch_gather(const void* src, int64_t src_rows, const int32_t* arow, const void* w, void* out,
                  int64_t M, int64_t K, int64_t N, int E, const int64_t* counts, hipStream_t s) {
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE, TB, M, K, N, E, DM_BM, DM_BN, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  const char* why = gather_limit(MODE, src_rows, M, K, N, E);
  TT_REQUIRE(why == nullptr, "gmm gather: %s (M=%lld K=%lld N=%lld E=%d, %lld source rows)", why,
             (long long)M, (long long)K, (long long)N, E, (long long)src_rows);
  return launch_p64_k<MODE, TB, ET, false, true>(src, w, out, M, K, N, E, counts, s, nblk, ti, tj,
                                                 arow, src_rows);
}

// Weight gradients with the rows of x (GX 1) or dy (GX 2) gathered from a
// source of src_rows rows; the long-reduction kernel only (more than 512 rows
// per expert on average), where the layer's packed copies would be read.
template <bool TB, int ET, int GX>
int launch_wgrad_gather(const void* x, const void* dy, int64_t src_rows, const int32_t* grow,
                        void* dw, int64_t M, int64_t K, int64_t N, int E, const int64_t* counts,
                        hipStream_t s) {
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE_WGRAD, TB, M, K, N, E, DM_BM, DM_BN, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm: grid too large");
  const char* why = wgrad_gather_limit(GX, src_rows, M, K, N, E);
  TT_REQUIRE(why == nullptr, "gmm gather: %s (M=%lld K=%lld N=%lld E=%d, %lld source rows)", why,
             (long long)M, (long long)K, (long long)N, E, (long long)src_rows);
  return launch_mfma_k<MODE_WGRAD, TB, ET, false, GX>(x, dy, dw, M, K, N, E, counts, s, nblk, ti,
                                                      tj, grow, src_rows);
}

template <int MODE, bool KMASK>
int launch_fp8_k(const void* p0, const uint8_t* qw, const void* scale, int sdt, void* out,
                 int64_t M, int64_t K, int64_t N, int E, const int64_t* counts, hipStream_t s,
                 int64_t nblk, int ti, int tj, size_t lds) {
  static size_t allowed = 64 * 1024;
  const int rc = allow_lds(&gmm_fp8_kernel<MODE, KMASK>, lds, allowed);
  if (rc != TT_OK) return rc;
  hipLaunchKernelGGL((gmm_fp8_kernel<MODE, KMASK>), dim3((unsigned)nblk), dim3(DM_NT), lds, s,
                     static_cast<const char*>(p0), reinterpret_cast<const char*>(qw),
                     static_cast<const char*>(scale), sdt, static_cast<char*>(out), M, K, N, E,
                     counts, ti, tj);
  return tt_check_launch("gmm_fp8");
}

template <int MODE, bool KMASK>
int launch_q8_k(const void* p0, const uint8_t* qw, const void* scale, int sdt, void* out,
                int64_t M, int64_t K, int64_t N, int E, const int64_t* counts, hipStream_t s,
                int64_t nblk, int tj) {
  const size_t lds = schedule_bytes(E);  // stages, staging and scale rows are static LDS
  static size_t allowed = 64 * 1024;
  const int rc = allow_lds(&gmm_q8_kernel<MODE, KMASK>, lds, allowed);
  if (rc != TT_OK) return rc;
  const int64_t cus = cu_count();
  const int64_t grid = nblk < cus ? nblk : cus;
  hipLaunchKernelGGL((gmm_q8_kernel<MODE, KMASK>), dim3((unsigned)grid), dim3(DM_NT), lds, s,
                     static_cast<const char*>(p0), reinterpret_cast<const char*>(qw),
                     static_cast<const char*>(scale), sdt, static_cast<char*>(out), M, K, N, E,
                     counts, tj);
  return tt_check_launch("gmm_fp8");
}

template <int MODE>
int launch_fp8(const void* p0, const uint8_t* qw, const void* scale, int sdt, void* out, int64_t M,
               int64_t K, int64_t N, int E, const int64_t* counts, hipStream_t s) {
  {
    // The persistent 128x512 kernel: a reduction of at least two 64-deep
    // k-tiles, at most Q_SMAX scale blocks along it, its LDS, and 32-bit
    // offsets for loads that run up to two k-tiles past the reduction end.
    const int64_t R = MODE == MODE_FWD ? K : N;
    const int64_t J = MODE == MODE_FWD ? N : K;
    const int64_t lda = MODE == MODE_FWD ? K : N;
    const int tjq = (int)((J + Q_BN - 1) / Q_BN);
    const int64_t nq = ((M + Q_BM - 1) / Q_BM + E) * (int64_t)tjq;
    if (nq == 0) return TT_OK;
    if (R > Q_BK && (R + 127) / 128 <= Q_SMAX &&
        schedule_bytes(E) + 2 * Q_STAGE + 4 * P_EPI + 4 * Q_SMAX * sizeof(float) + 64 <=
            160 * 1024 &&
        nq < 0x7fffffff && (M + Q_BM) * lda * 2 < (int64_t)DM_OOB &&
        (N + 2 * Q_BK + Q_BN) * K < (int64_t)DM_OOB) {
      if (R % Q_BK)
        return launch_q8_k<MODE, true>(p0, qw, scale, sdt, out, M, K, N, E, counts, s, nq, tjq);
      return launch_q8_k<MODE, false>(p0, qw, scale, sdt, out, M, K, N, E, counts, s, nq, tjq);
    }
  }
  int ti, tj;
  const int64_t nblk = grid_blocks(MODE, true, M, K, N, E, DM_BM, DM_BN, ti, tj);
  if (nblk == 0) return TT_OK;
  TT_REQUIRE(nblk < 0x7fffffff, "gmm_fp8: grid too large");
  // Dynamic LDS: the expert schedule, then the f32 block scales of the two
  // 128-column blocks of a tile.
  const int64_t nsc = MODE == MODE_FWD ? (K + 127) / 128 : (N + 127) / 128;
  const size_t lds = schedule_bytes(E) + (size_t)(2 * nsc) * sizeof(float);
  TT_REQUIRE(lds + (size_t)F8_LDS + 64 <= 160 * 1024,
             "gmm_fp8: too many experts or scale blocks for LDS (E=%d, blocks=%lld)", E,
             (long long)nsc);
  const int64_t ld = K > N ? K : N;
  TT_REQUIRE((M + DM_BM) * ld * 2 < (int64_t)DM_OOB && (N + DM_BN) * K < (int64_t)DM_OOB,
             "gmm_fp8: operands of 4 GiB or more are not supported (M=%lld K=%lld N=%lld)",
             (long long)M, (long long)K, (long long)N);
  const int64_t R = MODE == MODE_FWD ? K : N;
  if (R % DM_BK)
    return launch_fp8_k<MODE, true>(p0, qw, scale, sdt, out, M, K, N, E, counts, s, nblk, ti, tj,
                                    lds);
  return launch_fp8_k<MODE, false>(p0, qw, scale, sdt, out, M, K, N, E, counts, s, nblk, ti, tj,
                                   lds);
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
    if (tb) return launch_mfma<MODE, true, TT_BF16>(p0, p1, out, m, k, n, E, counts, s);
    return launch_mfma<MODE, false, TT_BF16>(p0, p1, out, m, k, n, E, counts, s);
  }
  if (tb) return launch_mfma<MODE, true, TT_F16>(p0, p1, out, m, k, n, E, counts, s);
  return launch_mfma<MODE, false, TT_F16>(p0, p1, out, m, k, n, E, counts, s);
}

template <int MODE>
int dispatch_gather(const void* src, int64_t src_rows, const int32_t* arow, const void* w,
                    int dtype, int64_t m, int64_t k, int64_t n, int E, int tb,
                    const int64_t* counts, void* out, void* stream) {
  TT_REQUIRE(m >= 0 && k >= 0 && n >= 0, "gmm: negative sizes");
  TT_REQUIRE(E >= 1 && E <= 4096, "gmm: num_experts must be in [1, 4096]");
  TT_REQUIRE(dtype == TT_BF16 || dtype == TT_F16, "gmm gather: unsupported dtype %d", dtype);
  TT_REQUIRE(k % 8 == 0 && n % 8 == 0, "gmm: K and N must be multiples of 8 (got %lld, %lld)",
             (long long)k, (long long)n);
  TT_REQUIRE(((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(w) |
               reinterpret_cast<uintptr_t>(out)) & 15) == 0,
             "gmm: operands must be 16-byte aligned");
  TT_REQUIRE(m == 0 || arow != nullptr, "gmm gather: row map required");
  hipStream_t s = S(stream);
  auto go = [&](auto tb_c, auto et_c) {
    return launch_gather<MODE, decltype(tb_c)::value, decltype(et_c)::value>(
        src, src_rows, arow, w, out, m, k, n, E, counts, s);
  };
  using BF = std::integral_constant<int, TT_BF16>;
  using HF = std::integral_constant<int, TT_F16>;
  if (dtype == TT_BF16) return tb ? go(std::true_type{}, BF{}) : go(std::false_type{}, BF{});
  return tb ? go(std::true_type{}, HF{}) : go(std::false_type{}, HF{});
}

int dispatch_wgrad_gather(const void* x, int64_t x_src_rows, const int32_t* x_rows,
                          const void* dy, int64_t dy_src_rows, const int32_t* dy_rows, int dtype,
                          int64_t m, int64_t k, int64_t n, int E, int tb, const int64_t* counts,
                          void* dw, void* stream) {
  TT_REQUIRE(m >= 0 && k >= 0 && n >= 0, "gmm: negative sizes");
  TT_REQUIRE(E >= 1 && E <= 4096, "gmm: num_experts must be in [1, 4096]");
  TT_REQUIRE(dtype == TT_BF16 || dtype == TT_F16, "gmm gather: unsupported dtype %d", dtype);
  TT_REQUIRE(k % 8 == 0 && n % 8 == 0, "gmm: K and N must be multiples of 8 (got %lld, %lld)",
             (long long)k, (long long)n);
  TT_REQUIRE((x_rows != nullptr) != (dy_rows != nullptr),
             "gmm gather: exactly one of the two row maps must be given");
  TT_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy) |
               reinterpret_cast<uintptr_t>(dw)) & 15) == 0,
             "gmm: operands must be 16-byte aligned");
  hipStream_t s = S(stream);
  const int32_t* rows = x_rows ? x_rows : dy_rows;
  const int64_t src = x_rows ? x_src_rows : dy_src_rows;
  auto go = [&](auto tb_c, auto et_c, auto gx_c) {
    return launch_wgrad_gather<decltype(tb_c)::value, decltype(et_c)::value,
                               decltype(gx_c)::value>(x, dy, src, rows, dw, m, k, n, E, counts,
                                                      s);
  };
  using BF = std::integral_constant<int, TT_BF16>;
  using HF = std::integral_constant<int, TT_F16>;
  using GXX = std::integral_constant<int, 1>;
  using GDY = std::integral_constant<int, 2>;
  if (dtype == TT_BF16) {
    if (x_rows) return tb ? go(std::true_type{}, BF{}, GXX{}) : go(std::false_type{}, BF{}, GXX{});
    return tb ? go(std::true_type{}, BF{}, GDY{}) : go(std::false_type{}, BF{}, GDY{});
  }
  if (x_rows) return tb ? go(std::true_type{}, HF{}, GXX{}) : go(std::false_type{}, HF{}, GXX{});
  return tb ? go(std::true_type{}, HF{}, GDY{}) : go(std::false_type{}, HF{}, GDY{});
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
  return launch_fp8<MODE_FWD>(x, qw, scale, scale_dtype, y, m, k, n, num_experts, counts,
                             S(stream));
}

extern "C" int tt_gmm_fp8_dgrad(const void* dy, const uint8_t* qw, const void* scale,
                                int scale_dtype, int64_t m, int64_t k, int64_t n,
                                int32_t num_experts, const int64_t* counts, void* dx,
                                void* stream) {
  const int rc = fp8_checks(dy, qw, dx, scale_dtype, m, k, n, num_experts);
  if (rc != TT_OK) return rc;
  return launch_fp8<MODE_DGRAD>(dy, qw, scale, scale_dtype, dx, m, k, n, num_experts, counts,
                               S(stream));
}

extern "C" int tt_gmm_gather_supported(int32_t op, int dtype, int64_t src_rows, int64_t m,
                                       int64_t k, int64_t n, int32_t num_experts) {
  if ((dtype != TT_BF16 && dtype != TT_F16) || m < 0 || k <= 0 || n <= 0 || k % 8 || n % 8 ||
      num_experts < 1 || num_experts > 4096)
    return 0;
  switch (op) {
    case 0: return gather_limit(MODE_FWD, src_rows, m, k, n, num_experts) == nullptr;
    case 1: return gather_limit(MODE_DGRAD, src_rows, m, k, n, num_experts) == nullptr;
    case 2: return wgrad_gather_limit(1, src_rows, m, k, n, num_experts) == nullptr;
    case 3: return wgrad_gather_limit(2, src_rows, m, k, n, num_experts) == nullptr;
    default: return 0;
  }
}

extern "C" int tt_gmm_wgrad_persistent(int dtype, int64_t m, int64_t k, int64_t n,
                                       int32_t num_experts, int32_t trans_b) {
  if ((dtype != TT_BF16 && dtype != TT_F16) || m < 0 || k <= 0 || n <= 0 || num_experts < 1 ||
      num_experts > 4096)
    return 0;
  int ti, tj;
  grid_blocks(MODE_WGRAD, trans_b != 0, m, k, n, num_experts, DM_BM, DM_BN, ti, tj);
  return wgrad_persistent(m, k, n, num_experts, ti, tj) ? 1 : 0;
}

extern "C" int tt_gmm_fwd_gather(const void* x_src, int64_t src_rows, const int32_t* src_of_row,
                                 const void* w, int dtype, int64_t m, int64_t k, int64_t n,
                                 int32_t num_experts, int32_t trans_b, const int64_t* counts,
                                 void* y, void* stream) {
  return dispatch_gather<MODE_FWD>(x_src, src_rows, src_of_row, w, dtype, m, k, n, num_experts,
                                   trans_b, counts, y, stream);
}

extern "C" int tt_gmm_dgrad_gather(const void* dy_src, int64_t src_rows,
                                   const int32_t* src_of_row, const void* w, int dtype, int64_t m,
                                   int64_t k, int64_t n, int32_t num_experts, int32_t trans_b,
                                   const int64_t* counts, void* dx, void* stream) {
  return dispatch_gather<MODE_DGRAD>(dy_src, src_rows, src_of_row, w, dtype, m, k, n,
                                     num_experts, trans_b, counts, dx, stream);
}

extern "C" int tt_gmm_wgrad_gather(const void* x, int64_t x_src_rows, const int32_t* x_src_of_row,
                                   const void* dy, int64_t dy_src_rows,
                                   const int32_t* dy_src_of_row, int dtype, int64_t m, int64_t k,
                                   int64_t n, int32_t num_experts, int32_t trans_b,
                                   const int64_t* counts, void* dw, void* stream) {
  return dispatch_wgrad_gather(x, x_src_rows, x_src_of_row, dy, dy_src_rows, dy_src_of_row, dtype,
                               m, k, n, num_experts, trans_b, counts, dw, stream);
}
