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
// 16 bytes with the non-temporal policy, through a global-address-space pointer (the policy bit is
// only set on global loads)
__device__ __forceinline__ int4 load_nt_i4(const void* p) {
  typedef int gv4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(1))) const gv4 ggv4;
  const gv4 v = __builtin_nontemporal_load(reinterpret_cast<ggv4*>(reinterpret_cast<uintptr_t>(p)));
  return make_int4(v.x, v.y, v.z, v.w);
}

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

// rint(v / scale) saturated to [-128, 127], bit for bit what the IEEE fp32 divide gives, with
// inv = rcp(scale) computed once per row. v * inv is within 2 ulp of v / scale, so below |q| = 2^8
// it lies within 1e-4 of the exact quotient: unless it lands that close to a half-integer (where the
// two could round apart) or is not finite, it rounds to the same integer. Those rare cases take the
// exact divide, behind a wave-uniform branch so the other waves skip it. scale == 0 gives 0.
__device__ __forceinline__ int8_t quant_i8(float v, float scale, float inv) {
  float p = v * inv;
  const float f = p - floorf(p);
  const bool exact = !(fabsf(f - 0.5f) > 1e-4f);
  if (__builtin_expect(__any(exact), 0)) {
    if (exact) p = v / scale;
  }
  const float q = fminf(fmaxf(rintf(p), -128.0f), 127.0f);
  return scale == 0.0f ? int8_t(0) : static_cast<int8_t>(static_cast<int>(q));
}

__device__ __forceinline__ float rcp_f32(float x) { return __builtin_amdgcn_rcpf(x); }

// silu(a) = a / (1 + exp(-a)) from the hardware exp2 and reciprocal: exp(-a) = exp2(-a * log2(e)),
// within a few ulp for the |a| that matter (the product's rounding grows with |a|, and past |a| ~ 20
// the term is 0 or a itself), the divide within 1 ulp. Every SwiGLU path (dequant_swiglu_quant and the
// fused grouped-GEMM epilogue) uses this one definition, so they agree bit for bit.
__device__ __forceinline__ float silu_f32(float a) {
  return a * rcp_f32(1.0f + __builtin_amdgcn_exp2f(a * -1.4426950408889634f));
}

__device__ __forceinline__ int64_t wave_incl_scan_i64(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t t = __shfl_up(v, o, kWave);
    if (lane >= o) v += t;
  }
  return v;
}

// Group of `row` from per-group row counts (int32 or int64), found by one wave on its own (no
// workgroup barrier): each lane sums a run of 4 counts, a wave scan of the run totals finds the run
// that holds the row, and that run's lane walks it. Returns -1 for a row past the total.
template <class T>
__device__ __forceinline__ int64_t group_of_row_wave_t(const T* counts, int64_t ng, int64_t row, int64_t& gbeg,
                                                      int64_t& gend) {
  constexpr int R = 4;
  const int lane = threadIdx.x & (kWave - 1);
  const bool vec = (reinterpret_cast<uintptr_t>(counts) & 15) == 0;
  int64_t carry = 0;
  for (int64_t base = 0; base < ng; base += kWave * R) {
    const int64_t g0 = base + static_cast<int64_t>(lane) * R;
    int64_t c[R];
    if (vec && g0 + R <= ng) {
      if constexpr (sizeof(T) == 8) {
        const longlong2 a = reinterpret_cast<const longlong2*>(counts + g0)[0];
        const longlong2 b = reinterpret_cast<const longlong2*>(counts + g0)[1];
        c[0] = a.x; c[1] = a.y; c[2] = b.x; c[3] = b.y;
      } else {
        const int4 a = *reinterpret_cast<const int4*>(counts + g0);
        c[0] = a.x; c[1] = a.y; c[2] = a.z; c[3] = a.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i) c[i] = g0 + i < ng ? static_cast<int64_t>(counts[g0 + i]) : 0;
    }
    const int64_t tot = c[0] + c[1] + c[2] + c[3];
    const int64_t incl = wave_incl_scan_i64(tot, lane) + carry;
    const uint64_t hit = __ballot(row >= incl - tot && row < incl);
    if (hit) {
      const int j = __ffsll(static_cast<unsigned long long>(hit)) - 1;
      int64_t found = -1, e = incl - tot, fb = 0, fe = 0;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if (found < 0 && row >= e && row < e + c[i]) {
          found = g0 + i;
          fb = e;
          fe = e + c[i];
        }
        e += c[i];
      }
      gbeg = __shfl(fb, j, kWave);
      gend = __shfl(fe, j, kWave);
      return __shfl(found, j, kWave);
    }
    carry = __shfl(incl, kWave - 1, kWave);
    if (carry > row) break;
  }
  return -1;
}

// As above for a counts array of torch dtype `dt` (int32 or int64); [gbeg, gend) receives the
// group's rows. A counts pointer that is not 16-byte aligned takes element loads for every run.
__device__ __forceinline__ int64_t group_of_row_wave(const void* counts, int dt, int64_t ng, int64_t row,
                                                    int64_t& gbeg, int64_t& gend) {
  if (dt == TAI_DT_INT64) return group_of_row_wave_t(static_cast<const int64_t*>(counts), ng, row, gbeg, gend);
  return group_of_row_wave_t(static_cast<const int32_t*>(counts), ng, row, gbeg, gend);
}
__device__ __forceinline__ int64_t group_of_row_wave(const void* counts, int dt, int64_t ng, int64_t row) {
  int64_t b, e;
  return group_of_row_wave(counts, dt, ng, row, b, e);
}

// Byte-wise select of v_perm_b32: byte i of the result is byte sel[i] of {hi:lo}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

}  // namespace tai
