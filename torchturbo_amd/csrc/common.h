// Shared helpers for the MoE expert-path kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/torchturbo_moe.h"

#define TT_WAVE 64

// ---------------------------------------------------------------------------
// Scalar conversions. bf16 is handled as raw uint16_t bits so rounding is
// explicit: round-to-nearest-even, NaN kept quiet, as PyTorch's CPU cast.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// Load element i of a tensor of runtime dtype as fp32 (fp64 rounds to
// nearest, as a cast to fp32 does).
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case TT_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case TT_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case TT_F64: return (float)static_cast<const double*>(p)[i];
    default: return static_cast<const float*>(p)[i];
  }
}

// Round an fp32 value to `dtype` and return it as fp32 again.
__device__ __forceinline__ float round_to(float v, int dtype) {
  switch (dtype) {
    case TT_BF16: return bf16_to_f32(f32_to_bf16(v));
    case TT_F16: return f16_to_f32(f32_to_f16(v));
    default: return v;
  }
}

__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case TT_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); break;
    case TT_F16: static_cast<uint16_t*>(p)[i] = f32_to_f16(v); break;
    case TT_F64: static_cast<double*>(p)[i] = (double)v; break;
    default: static_cast<float*>(p)[i] = v; break;
  }
}

// Element-type traits for the 2-byte / 4-byte data-movement kernels.
struct BF16T {
  typedef uint16_t storage;
  static __device__ __forceinline__ float to_f32(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f32(float v) { return f32_to_bf16(v); }
};
struct F16T {
  typedef uint16_t storage;
  static __device__ __forceinline__ float to_f32(uint16_t v) { return f16_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f32(float v) { return f32_to_f16(v); }
};
struct F32T {
  typedef float storage;
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
};

// PyTorch type promotion between two floating dtypes of this ABI.
static inline int tt_promote(int a, int b) {
  if (a == b) return a;
  return TT_F32;  // bf16 x f16 -> f32 as well
}

static inline int tt_elem_size(int dtype) {
  switch (dtype) {
    case TT_F64: return 8;
    case TT_F32: return 4;
    case TT_BF16: case TT_F16: return 2;
    case TT_F8E4M3: return 1;
    default: return 0;
  }
}

// ---------------------------------------------------------------------------
// Wave-level primitives.
// ---------------------------------------------------------------------------
// Streaming accesses of NB bytes (2, 4, 8 or 16) with the nontemporal hint,
// for data that a kernel touches exactly once.
template <int NB>
struct StreamVec;
template <>
struct StreamVec<16> { typedef __attribute__((ext_vector_type(4))) unsigned type; };
template <>
struct StreamVec<8> { typedef __attribute__((ext_vector_type(2))) unsigned type; };
template <>
struct StreamVec<4> { typedef unsigned type; };
template <>
struct StreamVec<2> { typedef unsigned short type; };

template <int NB>
__device__ __forceinline__ void load_stream(void* dst, const void* src) {
  typedef typename StreamVec<NB>::type V;
  const V v = __builtin_nontemporal_load(reinterpret_cast<const V*>(src));
  __builtin_memcpy(dst, &v, NB);
}
template <int NB>
__device__ __forceinline__ void store_stream(void* dst, const void* src) {
  typedef typename StreamVec<NB>::type V;
  V v;
  __builtin_memcpy(&v, src, NB);
  __builtin_nontemporal_store(v, reinterpret_cast<V*>(dst));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, TT_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, TT_WAVE));
  return v;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (TT_WAVE - 1); }

// Error reporting shared by every entry point of the library.
void tt_set_error(const char* fmt, ...);
int tt_check_launch(const char* what);

#define TT_REQUIRE(cond, ...)               \
  do {                                      \
    if (!(cond)) {                          \
      tt_set_error(__VA_ARGS__);            \
      return TT_ERR_INVALID;                \
    }                                       \
  } while (0)
