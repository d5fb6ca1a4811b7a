// Per-row int8 quantisers: npu_dynamic_quant and npu_dequant_swiglu_quant.
//
// Both are HBM-bound: one read of the input row, one write of the int8 row and a scale.
// A row lives in registers between the max-reduction and the quantising pass, so every
// input byte is read from HBM exactly once. Row -> workgroup mapping:
//   narrow rows (<= 4096 elements): one wave per row, 4 rows per 256-thread workgroup;
//   wide rows: one 256-thread workgroup per row.
// Arithmetic order (fixed so results are bit-reproducible against the CPU oracle):
//   xs = x * smooth;  scale = amax(|xs|) / 127;  y = clamp(rint(xs / scale), -128, 127)
// with IEEE fp32 division; an all-zero row gives scale 0 and y 0.
#include "common.h"

namespace tai {
namespace {

constexpr int kVec = 8;  // elements per vector load

template <int DT>
struct Vec8 {  // loads 8 elements as fp32 (non-temporal: the quantiser reads its input once)
  static __device__ __forceinline__ void load(const void* base, int64_t idx, float (&v)[kVec]) {
    if constexpr (DT == TAI_DT_FP32) {
      const float* p = static_cast<const float*>(base) + idx;
      const uint4 a = load_nt_u4(p), b = load_nt_u4(p + 4);
      v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
      v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
    } else {
      uint4 r = load_nt_u4(static_cast<const uint16_t*>(base) + idx);
      uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
        if constexpr (DT == TAI_DT_BF16) {
          v[2 * i] = bf16_to_f32(lo);
          v[2 * i + 1] = bf16_to_f32(hi);
        } else {
          v[2 * i] = f16_to_f32(lo);
          v[2 * i + 1] = f16_to_f32(hi);
        }
      }
    }
  }
};

// rint(v / scale) saturated to int8 (the IEEE divide's result; see quant_i8)
__device__ __forceinline__ int8_t quant1(float v, float scale) { return quant_i8(v, scale, rcp_f32(scale)); }

__device__ __forceinline__ uint2 pack8(const float (&v)[kVec], float scale) {
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < kVec; ++i) {
    uint32_t b = static_cast<uint8_t>(quant1(v[i], scale));
    w[i >> 2] |= b << (8 * (i & 3));
  }
  return make_uint2(w[0], w[1]);
}

// Smallest g with row < ends[g] (ends ascending, cumulative). Rows past the end use the last group.
__device__ __forceinline__ int64_t group_of_row_cumsum(const void* ends, int dt, int64_t n, int64_t row) {
  int64_t lo = 0, hi = n - 1;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (row < load_index(ends, dt, mid)) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// ----------------------------------------------------------------------------- dynamic quant
// TPR threads per row (64 or 256); NV vectors of 8 per thread held in registers.
template <int DT, int TPR, int NV>
__global__ __launch_bounds__(256) void dynamic_quant_kernel(
    const void* __restrict__ x, int64_t rows, int64_t cols, const float* __restrict__ smooth,
    const void* __restrict__ gidx, int gidx_dt, int64_t ngroups, int8_t* __restrict__ y,
    float* __restrict__ scale_out) {
  constexpr int RPB = 256 / TPR;
  __shared__ float red[RPB][TPR / 64];
  const int sub = threadIdx.x / TPR;
  const int lane = threadIdx.x % TPR;
  // Rows are taken last to first: an input just written front to back by the previous kernel (the
  // routing gather) has its last rows still in the memory-side cache, so they are read first.
  const int64_t row = static_cast<int64_t>(gridDim.x - 1 - blockIdx.x) * RPB + sub;
  const bool active = row < rows;
  const int64_t nvec = cols / kVec;

  const float* sm = nullptr;
  if (smooth != nullptr && active) {
    int64_t g = (gidx != nullptr) ? group_of_row_cumsum(gidx, gidx_dt, ngroups, row) : 0;
    sm = smooth + g * cols;
  }

  float v[NV][kVec];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t vi = lane + static_cast<int64_t>(i) * TPR;
    if (active && vi < nvec) {
      Vec8<DT>::load(x, row * cols + vi * kVec, v[i]);
      if (sm != nullptr) {
        const float4* sp = reinterpret_cast<const float4*>(sm + vi * kVec);
        float4 a = sp[0], b = sp[1];
        v[i][0] *= a.x; v[i][1] *= a.y; v[i][2] *= a.z; v[i][3] *= a.w;
        v[i][4] *= b.x; v[i][5] *= b.y; v[i][6] *= b.z; v[i][7] *= b.w;
      }
#pragma unroll
      for (int j = 0; j < kVec; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
    }
  }
  amax = wave_max(amax);
  if constexpr (TPR > 64) {
    if ((lane & 63) == 0) red[sub][lane >> 6] = amax;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TPR / 64; ++i) amax = fmaxf(amax, red[sub][i]);
  }
  if (!active) return;
  const float scale = amax / 127.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t vi = lane + static_cast<int64_t>(i) * TPR;
    if (vi < nvec) *reinterpret_cast<uint2*>(y + row * cols + vi * kVec) = pack8(v[i], scale);
  }
  if (lane == 0) scale_out[row] = scale;
}

// Any shape / alignment: one workgroup per row, two passes over global memory.
__global__ __launch_bounds__(256) void dynamic_quant_generic_kernel(
    const void* __restrict__ x, int dt, int64_t rows, int64_t cols, const float* __restrict__ smooth,
    const void* __restrict__ gidx, int gidx_dt, int64_t ngroups, int8_t* __restrict__ y,
    float* __restrict__ scale_out) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const float* sm = nullptr;
  if (smooth != nullptr) {
    int64_t g = (gidx != nullptr) ? group_of_row_cumsum(gidx, gidx_dt, ngroups, row) : 0;
    sm = smooth + g * cols;
  }
  float amax = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    float v = load_as_f32(x, dt, row * cols + c);
    if (sm) v *= sm[c];
    amax = fmaxf(amax, fabsf(v));
  }
  amax = block_max(amax, red);
  const float scale = amax / 127.0f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    float v = load_as_f32(x, dt, row * cols + c);
    if (sm) v *= sm[c];
    y[row * cols + c] = quant1(v, scale);
  }
  if (threadIdx.x == 0) scale_out[row] = scale;
}

template <int DT>
int launch_dynamic_quant(const void* x, int64_t rows, int64_t cols, const float* smooth,
                         const void* gidx, int gidx_dt, int64_t ng, int8_t* y, float* scale,
                         hipStream_t st) {
  const bool aligned = (cols % kVec) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 &&
                       (reinterpret_cast<uintptr_t>(y) % 8) == 0 &&
                       (smooth == nullptr || (reinterpret_cast<uintptr_t>(smooth) % 16) == 0);
  const int64_t nvec = cols / kVec;
  // Few rows (decode-sized batches) leave most CUs idle at one wave per row: give each row 256 threads.
  const bool few_rows = rows <= 1024 && nvec > 64;
  if (aligned && nvec <= 64 * 8 && !few_rows) {
    dim3 grid(static_cast<unsigned>(cdiv(rows, 4)));
    if (nvec <= 64 * 2)
      dynamic_quant_kernel<DT, 64, 2><<<grid, 256, 0, st>>>(x, rows, cols, smooth, gidx, gidx_dt, ng, y, scale);
    else if (nvec <= 64 * 4)
      dynamic_quant_kernel<DT, 64, 4><<<grid, 256, 0, st>>>(x, rows, cols, smooth, gidx, gidx_dt, ng, y, scale);
    else
      dynamic_quant_kernel<DT, 64, 8><<<grid, 256, 0, st>>>(x, rows, cols, smooth, gidx, gidx_dt, ng, y, scale);
  } else if (aligned && nvec <= 256 * 8) {
    dim3 grid(static_cast<unsigned>(rows));
    if (nvec <= 256 * 4)
      dynamic_quant_kernel<DT, 256, 4><<<grid, 256, 0, st>>>(x, rows, cols, smooth, gidx, gidx_dt, ng, y, scale);
    else
      dynamic_quant_kernel<DT, 256, 8><<<grid, 256, 0, st>>>(x, rows, cols, smooth, gidx, gidx_dt, ng, y, scale);
  } else {
    dynamic_quant_generic_kernel<<<dim3(static_cast<unsigned>(rows)), 256, 0, st>>>(
        x, DT, rows, cols, smooth, gidx, gidx_dt, ng, y, scale);
  }
  return launch_status("tai_dynamic_quant");
}

// ----------------------------------------------------------------------------- dequant-swiglu-quant
struct DsqArgs {
  const int32_t* x;
  int64_t rows, n;  // x is [rows, 2n]
  const float* ws;
  const float* as;
  const void* bias;
  int bias_dt;
  const float* qs;
  const void* gidx;
  int gidx_dt;
  int64_t ngroups;
  int left;
  int8_t* y;
  float* scale;
  // static mode (quant_mode 0): y = clamp(rint(h * quant_scale + quant_offset)); scale output 0
  const float* qo;
  int stat;
  // swiglu_mode 1 (generic kernel only): output column j pairs input columns 2j and 2j + 1
  int swi_mode;
  float clamp_limit, glu_alpha, glu_bias;
};

// int8 of one SwiGLU output v (already multiplied by quant_scale): dynamic, rint(v / scale) with
// inv = rcp(scale); static, rint(v + offset)
__device__ __forceinline__ int8_t dsq_out(const DsqArgs& a, float v, float scale, float inv, const float* qo, int64_t j) {
  if (a.stat) {
    const float q = __fadd_rn(v, qo ? qo[j] : 0.0f);
    return static_cast<int8_t>(static_cast<int>(fminf(fmaxf(rintf(q), -128.0f), 127.0f)));
  }
  return quant_i8(v, scale, inv);
}

__device__ __forceinline__ float silu(float a) { return silu_f32(a); }

#ifndef TAI_DSQ_NT
#define TAI_DSQ_NT 1
#endif
#ifndef TAI_DSQ_RPB
#define TAI_DSQ_RPB 2
#endif
// RPB consecutive rows per workgroup of TPB threads; each thread owns NV groups of 4 output columns
// of every row. All rows' int32 loads go out first, then each wave finds the rows' groups on its own
// (a row usually shares its predecessor's group, which is then reused), so the per-row cost of the
// group lookup and of the workgroup reduction is shared by RPB rows.
template <int NV, int TPB = 256, int RPB = 1>
__global__ __launch_bounds__(TPB) void dsq_kernel(DsqArgs a) {
  __shared__ float red[RPB][TPB / 64];
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPB;
  const int tid = threadIdx.x;
  const int64_t n = a.n, n2 = 2 * a.n;
  const int64_t ng4 = n / 4;
  // The rows' int32 values do not depend on their groups: their loads go out before the lookups.
  int4 xa[RPB][NV], xb[RPB][NV];
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    const int32_t* xr = a.x + (row0 + r < a.rows ? row0 + r : row0) * n2;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = tid + static_cast<int64_t>(i) * TPB;
      if (c < ng4) {
#if TAI_DSQ_NT
        xa[r][i] = load_nt_i4(xr + 4 * c);  // each int32 input is read once
        xb[r][i] = load_nt_i4(xr + n + 4 * c);
#else
        xa[r][i] = *reinterpret_cast<const int4*>(xr + 4 * c);
        xb[r][i] = *reinterpret_cast<const int4*>(xr + n + 4 * c);
#endif
      }
    }
  }
  int64_t grp[RPB];
  {
    int64_t g = -1, gbeg = 0, gend = 0;  // last group found and its row range
#pragma unroll
    for (int r = 0; r < RPB; ++r) {
      const int64_t row = row0 + r;
      if (a.gidx == nullptr) {
        grp[r] = 0;
      } else if (g >= 0 && row >= gbeg && row < gend) {
        grp[r] = g;
      } else {
        g = group_of_row_wave(a.gidx, a.gidx_dt, a.ngroups, row, gbeg, gend);
        grp[r] = g;
      }
    }
  }
  float v[RPB][NV][4];
  float amax[RPB];
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    amax[r] = 0.0f;
    const int64_t g = grp[r];
    if (g < 0) {  // row past the grouped rows (or past the end): y 0, scale 0
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[r][i][e] = 0.0f;
      continue;
    }
    const int64_t row = row0 + r;
    const float* ws = a.ws ? a.ws + g * n2 : nullptr;
    const float* qs = a.qs ? a.qs + g * n : nullptr;
    const float act = a.as ? a.as[row < a.rows ? row : 0] : 1.0f;
    const int32_t* bi = (a.bias && a.bias_dt == TAI_DT_INT32) ? static_cast<const int32_t*>(a.bias) + g * n2 : nullptr;
    const float* bf = (a.bias && a.bias_dt == TAI_DT_FP32) ? static_cast<const float*>(a.bias) + g * n2 : nullptr;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = tid + static_cast<int64_t>(i) * TPB;
      if (c < ng4) {
        const int64_t j = 4 * c;
        int ia[4] = {xa[r][i].x, xa[r][i].y, xa[r][i].z, xa[r][i].w};
        int ib[4] = {xb[r][i].x, xb[r][i].y, xb[r][i].z, xb[r][i].w};
        if (bi) {
          int4 ba = *reinterpret_cast<const int4*>(bi + j), bb = *reinterpret_cast<const int4*>(bi + n + j);
          ia[0] += ba.x; ia[1] += ba.y; ia[2] += ba.z; ia[3] += ba.w;
          ib[0] += bb.x; ib[1] += bb.y; ib[2] += bb.z; ib[3] += bb.w;
        }
        float wa[4] = {1.f, 1.f, 1.f, 1.f}, wb[4] = {1.f, 1.f, 1.f, 1.f};
        if (ws) {
          float4 p = *reinterpret_cast<const float4*>(ws + j), q = *reinterpret_cast<const float4*>(ws + n + j);
          wa[0] = p.x; wa[1] = p.y; wa[2] = p.z; wa[3] = p.w;
          wb[0] = q.x; wb[1] = q.y; wb[2] = q.z; wb[3] = q.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float da = static_cast<float>(ia[e]) * wa[e];
          float db = static_cast<float>(ib[e]) * wb[e];
          if (a.as) { da *= act; db *= act; }
          if (bf) { da += bf[j + e]; db += bf[n + j + e]; }
          float rv = a.left ? silu(da) * db : da * silu(db);
          if (qs) rv *= qs[j + e];
          v[r][i][e] = rv;
          amax[r] = fmaxf(amax[r], fabsf(rv));
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    const float m = wave_max(amax[r]);
    if ((tid & 63) == 0) red[r][tid >> 6] = m;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    const int64_t row = row0 + r;
    if (row >= a.rows) break;
    float m = red[r][0];
#pragma unroll
    for (int q = 1; q < TPB / 64; ++q) m = fmaxf(m, red[r][q]);
    const float scale = a.stat ? 0.0f : m / 127.0f, inv = rcp_f32(scale);
    const float* qo = (a.stat && a.qo && grp[r] >= 0) ? a.qo + grp[r] * n : nullptr;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = tid + static_cast<int64_t>(i) * TPB;
      if (c < ng4) {
        uint32_t w = 0;
        if (grp[r] >= 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w |= static_cast<uint32_t>(static_cast<uint8_t>(dsq_out(a, v[r][i][e], scale, inv, qo, 4 * c + e))) << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(a.y + row * n + 4 * c) = w;
      }
    }
    if (tid == 0) a.scale[row] = scale;
  }
}

// Any n: two passes over global memory.
__global__ __launch_bounds__(256) void dsq_generic_kernel(DsqArgs a) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int64_t n = a.n, n2 = 2 * a.n;
  int64_t g = 0;
  if (a.gidx != nullptr) g = group_of_row_wave(a.gidx, a.gidx_dt, a.ngroups, row);
  if (g < 0) {
    for (int64_t c = threadIdx.x; c < n; c += blockDim.x) a.y[row * n + c] = 0;
    if (threadIdx.x == 0) a.scale[row] = 0.0f;
    return;
  }
  const float* ws = a.ws ? a.ws + g * n2 : nullptr;
  const float* qs = a.qs ? a.qs + g * n : nullptr;
  const int32_t* bi = (a.bias && a.bias_dt == TAI_DT_INT32) ? static_cast<const int32_t*>(a.bias) + g * n2 : nullptr;
  const float* bf = (a.bias && a.bias_dt == TAI_DT_FP32) ? static_cast<const float*>(a.bias) + g * n2 : nullptr;
  const float act = a.as ? a.as[row] : 1.0f;
  // dequantised input column c (before the activation)
  auto pre = [&](int64_t c) {
    int xv = a.x[row * n2 + c];
    if (bi) xv += bi[c];
    float d = static_cast<float>(xv) * (ws ? ws[c] : 1.0f);
    if (a.as) d *= act;
    if (bf) d += bf[c];
    return d;
  };
  auto value = [&](int64_t j) {
    if (a.swi_mode == 1) {
      // the clamped SwiGLU of odd-even blocked columns: the activated column (even with activate_left,
      // else odd) clamped above, the linear one on both sides;
      // h = g * sigmoid(glu_alpha * g) * (l + glu_bias)
      const float ev = pre(2 * j), od = pre(2 * j + 1);
      const float g = fminf(a.left ? ev : od, a.clamp_limit);
      const float l = fminf(fmaxf(a.left ? od : ev, -a.clamp_limit), a.clamp_limit);
      const float sg = rcp_f32(1.0f + __builtin_amdgcn_exp2f((a.glu_alpha * g) * -1.4426950408889634f));
      float r = (g * sg) * (l + a.glu_bias);
      if (qs) r *= qs[j];
      return r;
    }
    int xa = a.x[row * n2 + j], xb = a.x[row * n2 + n + j];
    if (bi) { xa += bi[j]; xb += bi[n + j]; }
    float da = static_cast<float>(xa) * (ws ? ws[j] : 1.0f);
    float db = static_cast<float>(xb) * (ws ? ws[n + j] : 1.0f);
    if (a.as) { da *= act; db *= act; }
    if (bf) { da += bf[j]; db += bf[n + j]; }
    float r = a.left ? silu(da) * db : da * silu(db);
    if (qs) r *= qs[j];
    return r;
  };
  float amax = 0.0f;
  for (int64_t j = threadIdx.x; j < n; j += blockDim.x) amax = fmaxf(amax, fabsf(value(j)));
  amax = block_max(amax, red);
  const float scale = a.stat ? 0.0f : amax / 127.0f, inv = rcp_f32(scale);
  const float* qo = (a.stat && a.qo) ? a.qo + g * n : nullptr;
  for (int64_t j = threadIdx.x; j < n; j += blockDim.x) a.y[row * n + j] = dsq_out(a, value(j), scale, inv, qo, j);
  if (threadIdx.x == 0) a.scale[row] = scale;
}

// ----------------------------------------------------------------------------- dynamic quant v2
// Symmetric with a custom range (dst_type_max), per-tensor, and asymmetric quantisation. Three
// passes: each row's max and min of the smoothed input -> (per-tensor) one workgroup folds the row
// statistics -> each row is quantised with its own or the tensor's scale and offset:
//   symmetric:  scale = max(|max|, |min|) / q,      y = clamp(rint(xs / scale), -128, 127), offset 0
//   asymmetric: hi = max(max, 0), lo = min(min, 0), scale = (hi - lo) / 255,
//               offset = -128 - lo / scale,         y = clamp(rint(xs / scale + offset), -128, 127)
// (q = dst_type_max, or 127 when it is 0; fp32 arithmetic in that order; a zero range gives scale 0,
// offset 0 and y 0).
struct Dq2Args {
  const void* x;
  int dt;
  int64_t rows, cols;
  const float* smooth;
  const void* gidx;
  int gidx_dt;
  int64_t ngroups;
  int symmetric, per_tensor;
  float qmax;
  float* smax;  // [rows] row maxima (then the tensor's at [0] when per_tensor)
  float* smin;  // [rows] row minima
  int8_t* y;
  float* scale;
  float* offset;  // asymmetric only
};

__device__ __forceinline__ float dq2_value(const Dq2Args& a, const float* sm, int64_t row, int64_t c) {
  const float v = load_as_f32(a.x, a.dt, row * a.cols + c);
  return sm ? v * sm[c] : v;
}

__device__ __forceinline__ const float* dq2_smooth(const Dq2Args& a, int64_t row) {
  if (a.smooth == nullptr) return nullptr;
  const int64_t g = a.gidx != nullptr ? group_of_row_cumsum(a.gidx, a.gidx_dt, a.ngroups, row) : 0;
  return a.smooth + g * a.cols;
}

__global__ __launch_bounds__(256) void dq2_stats_kernel(Dq2Args a) {
  __shared__ float red[2][4];
  const int64_t row = blockIdx.x;
  const float* sm = dq2_smooth(a, row);
  float mx = -INFINITY, mn = INFINITY;
  for (int64_t c = threadIdx.x; c < a.cols; c += 256) {
    const float v = dq2_value(a, sm, row, c);
    mx = fmaxf(mx, v);
    mn = fminf(mn, v);
  }
  mx = wave_max(mx);
  mn = -wave_max(-mn);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { red[0][w] = mx; red[1][w] = mn; }
  __syncthreads();
  if (threadIdx.x == 0) {
    a.smax[row] = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    a.smin[row] = fminf(fminf(red[1][0], red[1][1]), fminf(red[1][2], red[1][3]));
  }
}

__global__ __launch_bounds__(1024) void dq2_fold_kernel(Dq2Args a) {
  __shared__ float red[2][16];
  float mx = -INFINITY, mn = INFINITY;
  for (int64_t r = threadIdx.x; r < a.rows; r += 1024) {
    mx = fmaxf(mx, a.smax[r]);
    mn = fminf(mn, a.smin[r]);
  }
  mx = wave_max(mx);
  mn = -wave_max(-mn);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { red[0][w] = mx; red[1][w] = mn; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 16; ++i) { mx = fmaxf(mx, red[0][i]); mn = fminf(mn, red[1][i]); }
    mx = fmaxf(mx, red[0][0]);
    mn = fminf(mn, red[1][0]);
    a.smax[0] = mx;
    a.smin[0] = mn;
  }
}

__global__ __launch_bounds__(256) void dq2_apply_kernel(Dq2Args a) {
  const int64_t row = blockIdx.x;
  const int64_t srow = a.per_tensor ? 0 : row;
  const float mx = a.smax[srow], mn = a.smin[srow];
  float sc, off = 0.0f;
  if (a.symmetric) {
    sc = fmaxf(fabsf(mx), fabsf(mn)) / a.qmax;
  } else {
    const float hi = fmaxf(mx, 0.0f), lo = fminf(mn, 0.0f);
    sc = (hi - lo) / 255.0f;
    off = sc == 0.0f ? 0.0f : -128.0f - lo / sc;
  }
  const float* sm = dq2_smooth(a, row);
  for (int64_t c = threadIdx.x; c < a.cols; c += 256) {
    const float v = dq2_value(a, sm, row, c);
    float q = 0.0f;
    if (sc != 0.0f) q = fminf(fmaxf(rintf(a.symmetric ? v / sc : v / sc + off), -128.0f), 127.0f);
    a.y[row * a.cols + c] = static_cast<int8_t>(static_cast<int>(q));
  }
  if (threadIdx.x == 0 && (!a.per_tensor || row == 0)) {
    a.scale[a.per_tensor ? 0 : row] = sc;
    if (a.offset) a.offset[a.per_tensor ? 0 : row] = off;
  }
}

}  // namespace
}  // namespace tai

using namespace tai;

namespace tai {
namespace {
// Static per-tensor / per-group quantisation of rows: y = clamp(rint(x * scale + offset), -128, 127),
// the product and the sum each rounded once. The row's group is row / group_rows (group_rows > 0),
// found in the cumulative group ends (group_ends), or 0; scale / offset hold one value or one per
// column for each group (scale_groups 1: shared by all groups). One thread per element.
struct StaticQuantArgs {
  const void* x;
  int dt;
  int64_t rows, cols;
  const float* scale;
  const float* offset;
  int64_t scale_groups;
  int per_col;
  const void* ends;
  int ends_dt;
  int64_t ngroups;
  int64_t group_rows;
  int8_t* y;
};

__global__ __launch_bounds__(256) void static_quant_kernel(StaticQuantArgs a) {
  const int64_t total = a.rows * a.cols;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / a.cols, c = i % a.cols;
    int64_t g = 0;
    if (a.group_rows > 0) g = r / a.group_rows;
    else if (a.ends) g = group_of_row_cumsum(a.ends, a.ends_dt, a.ngroups, r);
    if (a.scale_groups == 1) g = 0;
    const int64_t si = g * (a.per_col ? a.cols : 1) + (a.per_col ? c : 0);
    float v;
    if (a.dt == TAI_DT_FP32) v = static_cast<const float*>(a.x)[i];
    else if (a.dt == TAI_DT_BF16) v = bf16_to_f32(static_cast<const uint16_t*>(a.x)[i]);
    else v = f16_to_f32(static_cast<const uint16_t*>(a.x)[i]);
    const float q = __fadd_rn(__fmul_rn(v, a.scale[si]), a.offset ? a.offset[si] : 0.0f);
    a.y[i] = static_cast<int8_t>(static_cast<int>(fminf(fmaxf(rintf(q), -128.0f), 127.0f)));
  }
}
}  // namespace
}  // namespace tai

extern "C" int tai_static_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, const float* scale,
                                     const float* offset, int64_t scale_groups, int per_col, const void* group_ends,
                                     int group_ends_dtype, int64_t num_groups, int64_t group_rows, int8_t* y,
                                     void* stream) {
  using namespace tai;
  TAI_CHECK_ARG(rows >= 0 && cols >= 0 && scale_groups >= 1 && (per_col == 0 || per_col == 1),
                "tai_static_quant_rows: bad sizes");
  TAI_CHECK_ARG(x_dtype == TAI_DT_BF16 || x_dtype == TAI_DT_FP16 || x_dtype == TAI_DT_FP32,
                "tai_static_quant_rows: x must be bf16, fp16 or fp32");
  TAI_CHECK_ARG(scale_groups == 1 || group_rows > 0 || (group_ends && num_groups == scale_groups),
                "tai_static_quant_rows: per-group scales need group_rows or group_ends of scale_groups entries");
  TAI_CHECK_ARG(group_ends == nullptr || group_ends_dtype == TAI_DT_INT64 || group_ends_dtype == TAI_DT_INT32,
                "tai_static_quant_rows: group_ends must be int32 or int64");
  if (rows == 0 || cols == 0) return TAI_OK;
  TAI_CHECK_ARG(x && scale && y, "tai_static_quant_rows: null pointer");
  StaticQuantArgs a{x, x_dtype, rows, cols, scale, offset, scale_groups, per_col, group_ends, group_ends_dtype,
                    num_groups, group_rows, y};
  const int64_t blocks = std::min<int64_t>(cdiv(rows * cols, 256), 65536);
  static_quant_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("tai_static_quant_rows");
}

extern "C" int tai_dynamic_quant(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                 const float* smooth_scales, const void* group_index,
                                 int group_index_dtype, int64_t num_groups, int8_t* y, float* scale,
                                 void* stream) {
  TAI_CHECK_ARG(rows >= 0 && cols >= 0, "tai_dynamic_quant: negative size");
  if (rows == 0) return TAI_OK;
  TAI_CHECK_ARG(x && y && scale, "tai_dynamic_quant: null pointer");
  TAI_CHECK_ARG(rows < (1ll << 31), "tai_dynamic_quant: rows must be < 2^31");
  TAI_CHECK_ARG(group_index == nullptr || (smooth_scales != nullptr && num_groups > 0),
                "tai_dynamic_quant: group_index needs smooth_scales with num_groups > 0");
  TAI_CHECK_ARG(group_index == nullptr || group_index_dtype == TAI_DT_INT32 || group_index_dtype == TAI_DT_INT64,
                "tai_dynamic_quant: group_index must be int32 or int64");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case TAI_DT_BF16: return launch_dynamic_quant<TAI_DT_BF16>(x, rows, cols, smooth_scales, group_index, group_index_dtype, num_groups, y, scale, st);
    case TAI_DT_FP16: return launch_dynamic_quant<TAI_DT_FP16>(x, rows, cols, smooth_scales, group_index, group_index_dtype, num_groups, y, scale, st);
    case TAI_DT_FP32: return launch_dynamic_quant<TAI_DT_FP32>(x, rows, cols, smooth_scales, group_index, group_index_dtype, num_groups, y, scale, st);
    default: set_error("tai_dynamic_quant: x dtype %d not supported (bf16, fp16, fp32)", x_dtype); return TAI_ERR_INVALID;
  }
}

extern "C" int tai_dequant_swiglu_quant(const int32_t* x, int64_t rows, int64_t n2,
                                        const float* weight_scale, const float* activation_scale,
                                        const void* bias, int bias_dtype, const float* quant_scale,
                                        const void* group_index, int group_index_dtype,
                                        int64_t num_groups, int activate_left, int8_t* y,
                                        float* scale, void* stream) {
  return tai_dequant_swiglu_quant_static(x, rows, n2, weight_scale, activation_scale, bias, bias_dtype, quant_scale,
                                         nullptr, group_index, group_index_dtype, num_groups, activate_left, 1, y,
                                         scale, stream);
}

namespace tai {
namespace {
int dsq_run(const int32_t* x, int64_t rows, int64_t n2, const float* weight_scale, const float* activation_scale,
            const void* bias, int bias_dtype, const float* quant_scale, const float* quant_offset,
            const void* group_index, int group_index_dtype, int64_t num_groups, int activate_left, int quant_mode,
            int8_t* y, float* scale, void* stream, int swi_mode, float clamp_limit, float glu_alpha, float glu_bias) {
  TAI_CHECK_ARG(quant_mode == 0 || quant_mode == 1, "tai_dequant_swiglu_quant: quant_mode must be 0 (static) or 1 "
                "(dynamic)");
  TAI_CHECK_ARG(quant_mode == 0 || quant_offset == nullptr, "tai_dequant_swiglu_quant: quant_offset applies to the "
                "static mode");
  TAI_CHECK_ARG(quant_mode == 1 || quant_scale != nullptr, "tai_dequant_swiglu_quant: the static mode needs quant_scale");
  TAI_CHECK_ARG(rows >= 0 && n2 >= 0 && n2 % 2 == 0, "tai_dequant_swiglu_quant: last dim must be even");
  if (rows == 0) return TAI_OK;
  TAI_CHECK_ARG(x && y && scale, "tai_dequant_swiglu_quant: null pointer");
  TAI_CHECK_ARG(rows < (1ll << 31), "tai_dequant_swiglu_quant: rows must be < 2^31");
  TAI_CHECK_ARG(bias == nullptr || bias_dtype == TAI_DT_INT32 || bias_dtype == TAI_DT_FP32,
                "tai_dequant_swiglu_quant: bias must be int32 or fp32");
  TAI_CHECK_ARG(group_index == nullptr || num_groups > 0, "tai_dequant_swiglu_quant: empty group_index");
  TAI_CHECK_ARG(group_index == nullptr || group_index_dtype == TAI_DT_INT32 || group_index_dtype == TAI_DT_INT64,
                "tai_dequant_swiglu_quant: group_index must be int32 or int64");
  DsqArgs a{x, rows, n2 / 2, weight_scale, activation_scale, bias, bias_dtype, quant_scale,
            group_index, group_index_dtype, group_index ? num_groups : 1, activate_left, y, scale, quant_offset,
            quant_mode == 0 ? 1 : 0, swi_mode, clamp_limit, glu_alpha, glu_bias};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (swi_mode == 1) {
    dsq_generic_kernel<<<dim3(static_cast<unsigned>(rows)), 256, 0, st>>>(a);
    return launch_status("tai_dequant_swiglu_quant_clamped");
  }
  const int64_t n = n2 / 2;
  auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  const bool aligned = n % 4 == 0 && al(x) && al(weight_scale) && al(bias) && (reinterpret_cast<uintptr_t>(y) % 4) == 0;
  const int64_t ng4 = n / 4;
  dim3 grid(static_cast<unsigned>(rows));
  // Few rows (decode-sized batches): 1024 threads per row spread the SwiGLU arithmetic over more SIMDs.
  if (aligned && rows <= 512 && ng4 > 512 && ng4 <= 1024 * 2) {
    if (ng4 <= 1024) dsq_kernel<1, 1024><<<grid, 1024, 0, st>>>(a);
    else dsq_kernel<2, 1024><<<grid, 1024, 0, st>>>(a);
  } else if (aligned && ng4 <= 256 * 2) {
    dsq_kernel<2, 256, TAI_DSQ_RPB><<<dim3(static_cast<unsigned>(cdiv(rows, TAI_DSQ_RPB))), 256, 0, st>>>(a);
  }
  else if (aligned && ng4 <= 256 * 4) dsq_kernel<4><<<grid, 256, 0, st>>>(a);
  else if (aligned && ng4 <= 256 * 8) dsq_kernel<8><<<grid, 256, 0, st>>>(a);
  else dsq_generic_kernel<<<grid, 256, 0, st>>>(a);
  return launch_status("tai_dequant_swiglu_quant");
}
}  // namespace
}  // namespace tai

extern "C" int tai_dequant_swiglu_quant_static(const int32_t* x, int64_t rows, int64_t n2,
                                               const float* weight_scale, const float* activation_scale,
                                               const void* bias, int bias_dtype, const float* quant_scale,
                                               const float* quant_offset, const void* group_index,
                                               int group_index_dtype, int64_t num_groups, int activate_left,
                                               int quant_mode, int8_t* y, float* scale, void* stream) {
  return dsq_run(x, rows, n2, weight_scale, activation_scale, bias, bias_dtype, quant_scale, quant_offset, group_index,
                 group_index_dtype, num_groups, activate_left, quant_mode, y, scale, stream, 0, 0.0f, 0.0f, 0.0f);
}

extern "C" int tai_dequant_swiglu_quant_clamped(const int32_t* x, int64_t rows, int64_t n2,
                                                const float* weight_scale, const float* activation_scale,
                                                const void* bias, int bias_dtype, const float* quant_scale,
                                                const float* quant_offset, const void* group_index,
                                                int group_index_dtype, int64_t num_groups, int activate_left,
                                                int quant_mode, float clamp_limit, float glu_alpha, float glu_bias,
                                                int8_t* y, float* scale, void* stream) {
  return dsq_run(x, rows, n2, weight_scale, activation_scale, bias, bias_dtype, quant_scale, quant_offset, group_index,
                 group_index_dtype, num_groups, activate_left, quant_mode, y, scale, stream, 1, clamp_limit, glu_alpha,
                 glu_bias);
}

extern "C" size_t tai_dynamic_quant_v2_workspace_size(int64_t rows) {
  return rows > 0 ? static_cast<size_t>(2 * rows) * sizeof(float) + 256 : 256;
}

extern "C" int tai_dynamic_quant_v2(const void* x, int x_dtype, int64_t rows, int64_t cols, const float* smooth_scales,
                                    const void* group_index, int group_index_dtype, int64_t num_groups, int symmetric,
                                    int per_tensor, float dst_type_max, int8_t* y, float* scale, float* offset,
                                    void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(rows >= 0 && cols >= 0, "tai_dynamic_quant_v2: negative size");
  TAI_CHECK_ARG(x_dtype == TAI_DT_BF16 || x_dtype == TAI_DT_FP16 || x_dtype == TAI_DT_FP32,
                "tai_dynamic_quant_v2: x dtype %d not supported (bf16, fp16, fp32)", x_dtype);
  TAI_CHECK_ARG(dst_type_max >= 0.0f && dst_type_max <= 127.0f, "tai_dynamic_quant_v2: dst_type_max must be in [0, 127]");
  TAI_UNSUPPORTED(!symmetric && dst_type_max != 0.0f, "tai_dynamic_quant_v2: dst_type_max applies to the symmetric mode only");
  TAI_CHECK_ARG(group_index == nullptr || (smooth_scales != nullptr && num_groups > 0),
                "tai_dynamic_quant_v2: group_index needs smooth_scales with num_groups > 0");
  TAI_CHECK_ARG(group_index == nullptr || group_index_dtype == TAI_DT_INT32 || group_index_dtype == TAI_DT_INT64,
                "tai_dynamic_quant_v2: group_index must be int32 or int64");
  if (rows == 0) return TAI_OK;
  TAI_CHECK_ARG(x && y && scale && (symmetric || offset), "tai_dynamic_quant_v2: null pointer");
  TAI_CHECK_ARG(rows < (1ll << 31), "tai_dynamic_quant_v2: rows must be < 2^31");
  const size_t need = tai_dynamic_quant_v2_workspace_size(rows);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_dynamic_quant_v2: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  float* smax = static_cast<float*>(workspace);
  Dq2Args a{x, x_dtype, rows, cols, smooth_scales, group_index, group_index_dtype, group_index ? num_groups : 1,
            symmetric ? 1 : 0, per_tensor ? 1 : 0, dst_type_max > 0.0f ? dst_type_max : 127.0f, smax, smax + rows, y,
            scale, symmetric ? nullptr : offset};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
  dq2_stats_kernel<<<grid, 256, 0, st>>>(a);
  if (per_tensor) dq2_fold_kernel<<<1, 1024, 0, st>>>(a);
  dq2_apply_kernel<<<grid, 256, 0, st>>>(a);
  return launch_status("tai_dynamic_quant_v2");
}

// ----------------------------------------------------------------------------- npu_swiglu
// y = silu(a) * b with a, b the two halves of x along one dimension, viewed as [outer, 2 * n, inner]:
// a = x[o, j, i], b = x[o, n + j, i] for j < n; fp32 arithmetic, one rounding to the output dtype.
namespace tai {
namespace {
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ x, int dt, int64_t outer, int64_t n,
                                                     int64_t inner, void* __restrict__ y) {
  const int64_t total = outer * n * inner;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t i = idx % inner, j = (idx / inner) % n, o = idx / (inner * n);
    const int64_t xa = (o * 2 * n + j) * inner + i;
    const float a = load_as_f32(x, dt, xa), b = load_as_f32(x, dt, xa + n * inner);
    store_from_f32(y, dt, idx, silu_f32(a) * b);
  }
}
}  // namespace
}  // namespace tai

extern "C" int tai_swiglu(const void* x, int dtype, int64_t outer, int64_t n, int64_t inner, void* y, void* stream) {
  TAI_CHECK_ARG(dtype == TAI_DT_BF16 || dtype == TAI_DT_FP16 || dtype == TAI_DT_FP32,
                "tai_swiglu: dtype %d not supported (bf16, fp16, fp32)", dtype);
  TAI_CHECK_ARG(outer >= 0 && n >= 0 && inner >= 0, "tai_swiglu: negative size");
  const int64_t total = outer * n * inner;
  if (total == 0) return TAI_OK;
  TAI_CHECK_ARG(x && y, "tai_swiglu: null pointer");
  const int64_t blocks = cdiv(total, 256) < 65536 ? cdiv(total, 256) : 65536;
  swiglu_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(x, dtype, outer, n,
                                                                                                   inner, y);
  return launch_status("tai_swiglu");
}

