// Shared helpers for the gfx950 kernels behind include/tai_kernels.h.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/tai_kernels.h"

namespace tai {

// ----------------------------------------------------------------------------- errors
void set_error(const char* fmt, ...);

#define TAI_CHECK_ARG(cond, ...)                         \
  do {                                                   \
    if (!(cond)) {                                       \
      ::tai::set_error(__VA_ARGS__);                     \
      return TAI_ERR_INVALID;                            \
    }                                                    \
  } while (0)

#define TAI_UNSUPPORTED(cond, ...)                       \
  do {                                                   \
    if (cond) {                                          \
      ::tai::set_error(__VA_ARGS__);                     \
      return TAI_ERR_UNSUPPORTED;                        \
    }                                                    \
  } while (0)

// Checks the launch that was just enqueued.
int launch_status(const char* what);

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ----------------------------------------------------------------------------- numerics
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// 16-byte global load with the non-temporal policy (`nt`), for data a kernel reads once: the
// finalize gather and the dynamic quantiser read 8-14% faster with it.
typedef unsigned tai_u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt_u4(const void* p) {
  const tai_u32x4_t v = __builtin_nontemporal_load(static_cast<const tai_u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN), the rounding torch uses.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t v) {
  return __half2float(__ushort_as_half(v));
}
// fp32 -> fp16, round to nearest even, from a value already rounded to fp32: the empty asm keeps
// the compiler from fusing the multiply that produced f into the conversion (v_fma_mix*_f16 rounds
// once, to fp16, where the op rounds to fp32 first)
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  asm("" : "+v"(f));
  return __half_as_ushort(__float2half_rn(f));
}

// Load element i of a floating tensor given its dtype code as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case TAI_DT_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case TAI_DT_FP16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case TAI_DT_INT32: return static_cast<float>(static_cast<const int32_t*>(p)[i]);
    default: return static_cast<const float*>(p)[i];
  }
}

__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case TAI_DT_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); break;
    case TAI_DT_FP16: static_cast<uint16_t*>(p)[i] = f32_to_f16(v); break;
    default: static_cast<float*>(p)[i] = v; break;
  }
}

// ----------------------------------------------------------------------------- wave ops
constexpr int kWave = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Max over the whole block (blockDim.x a multiple of 64, at most 1024). `red` holds 16 floats.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < nw; ++i) r = fmaxf(r, red[i]);
  return r;
}

// 64-bit integer max / min (HIP's max/min templates promote mixed int / int64 arguments to double).
__host__ __device__ __forceinline__ int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }
__host__ __device__ __forceinline__ int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }

// Inclusive scan over the block (blockDim.x a multiple of 64, at most 1024) of one value per
// thread, combining with + (MAX = false) or max (MAX = true). `red` holds 16 values; every thread
// of the block must call it.
template <bool MAX, class T>
__device__ __forceinline__ T block_incl_scan(T x, T* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T u = __shfl_up(x, o, kWave);
    if (lane >= o) x = MAX ? (u > x ? u : x) : x + u;
  }
  __syncthreads();
  if (lane == 63) red[w] = x;
  __syncthreads();
  if (w > 0) {
    T pre = red[0];
    for (int i = 1; i < w; ++i) pre = MAX ? (red[i] > pre ? red[i] : pre) : pre + red[i];
    x = MAX ? (pre > x ? pre : x) : x + pre;
  }
  (void)nw;
  return x;
}

__device__ __forceinline__ int64_t load_index(const void* p, int dtype, int64_t i) {
  return dtype == TAI_DT_INT64 ? static_cast<const int64_t*>(p)[i]
                               : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

// Byte-wise select of v_perm_b32: byte i of the result is byte sel[i] of {hi:lo}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

}  // namespace tai
