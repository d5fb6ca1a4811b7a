// RMS-norm family and KV-cache writers: npu_add_rms_norm, npu_add_rms_norm_dynamic_quant,
// npu_scatter_pa_kv_cache and npu_kv_rmsnorm_rope_cache.
//
// All four are HBM-bound row operations. A row (or a token's cache row) lives in registers
// between its reduction and its outputs, so each input byte is read once and each output
// byte written once.
// Arithmetic order (fixed so results reproduce the CPU oracle):
//   x = float(x1) + float(x2);  rstd = 1 / sqrt(sum(x*x) / n + eps)  (IEEE divide and sqrt);
//   y = (x * rstd) * gamma [+ beta], rounded to the input dtype;
//   the fused quant quantises that rounded y exactly as npu_dynamic_quant would, so replacing
//   add_rms_norm + dynamic_quant by the fused op changes no output;
//   interleaved RoPE: xd = (x[0::2], x[1::2]); out = xd * cos + rotate_half(xd) * sin.
#include "common.h"

namespace tai {
namespace {

constexpr int kVec = 8;

// 8 consecutive elements of a bf16 / fp16 / fp32 tensor as fp32.
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t idx, float (&v)[kVec]) {
  if constexpr (DT == TAI_DT_FP32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + idx);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
      v[2 * i] = DT == TAI_DT_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      v[2 * i + 1] = DT == TAI_DT_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  }
}

// Rounds to the storage dtype and back (the value a consumer of the stored tensor sees).
template <int DT>
__device__ __forceinline__ float round_dt(float f) {
  if constexpr (DT == TAI_DT_BF16) return bf16_to_f32(f32_to_bf16(f));
  else if constexpr (DT == TAI_DT_FP16) return f16_to_f32(f32_to_f16(f));
  else return f;
}

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t idx, const float (&v)[kVec]) {
  if constexpr (DT == TAI_DT_FP32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + idx);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = DT == TAI_DT_BF16 ? f32_to_bf16(v[2 * i]) : f32_to_f16(v[2 * i]);
      const uint32_t hi = DT == TAI_DT_BF16 ? f32_to_bf16(v[2 * i + 1]) : f32_to_f16(v[2 * i + 1]);
      w[i] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + idx) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// 8 consecutive fp32 values (16-byte aligned), or 1.0 when p is null.
__device__ __forceinline__ void load8_f32_or_one(const float* p, int64_t idx, float (&v)[kVec]) {
  if (!p) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) v[j] = 1.0f;
    return;
  }
  const float4 a = reinterpret_cast<const float4*>(p + idx)[0], b = reinterpret_cast<const float4*>(p + idx)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// rint(v / scale) saturated to int8 (the IEEE divide's result; see quant_i8)
__device__ __forceinline__ int8_t quant1(float v, float scale) { return quant_i8(v, scale, rcp_f32(scale)); }

__device__ __forceinline__ uint2 pack8(const float (&v)[kVec], float scale) {
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < kVec; ++i) w[i >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(quant1(v[i], scale))) << (8 * (i & 3));
  return make_uint2(w[0], w[1]);
}

// Sum / max over the TPR threads of one row (TPR = 64: one wave; 256: the whole workgroup).
template <int TPR>
__device__ __forceinline__ float row_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (TPR > 64) {
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = 0.0f;
#pragma unroll
    for (int i = 0; i < TPR / 64; ++i) v += red[i];
  }
  return v;
}
template <int TPR>
__device__ __forceinline__ float row_max(float v, float* red) {
  v = wave_max(v);
  if constexpr (TPR > 64) {
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int i = 1; i < TPR / 64; ++i) v = fmaxf(v, red[i]);
  }
  return v;
}

struct NormArgs {
  const void* x1;
  const void* x2;
  const void* gamma;
  const void* beta;     // quant variant only (may be null)
  const float* smooth1;  // quant variant only (may be null)
  const float* smooth2;
  int64_t rows, cols;
  float eps;
  void* y;         // add_rms_norm: normalised output (input dtype)
  float* rstd;     // add_rms_norm: [rows]
  void* x_out;     // x1 + x2 in the input dtype (may be null)
  int8_t* y1;      // quant variant
  int8_t* y2;      // quant variant, second smooth scale (may be null)
  float* scale1;
  float* scale2;
};

// ----------------------------------------------------------------------------- add_rms_norm (+ quant)
// One row per TPR threads, NV vectors of 8 per thread held in registers. QUANT selects the
// fused dynamic-quant outputs instead of y / rstd.
template <int DT, int TPR, int NV, bool QUANT>
__global__ __launch_bounds__(TPR) void add_rms_norm_kernel(NormArgs a) {
  __shared__ float red[TPR / 64];
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t nvec = a.cols / kVec;
  const int64_t base = row * a.cols;
  float x[NV][kVec];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t vi = lane + static_cast<int64_t>(i) * TPR;
    if (vi < nvec) {
      float b[kVec];
      load8<DT>(a.x1, base + vi * kVec, x[i]);
      load8<DT>(a.x2, base + vi * kVec, b);
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        x[i][j] = x[i][j] + b[j];
        ss += x[i][j] * x[i][j];
      }
      if (a.x_out) {
        store8<DT>(a.x_out, base + vi * kVec, x[i]);
      }
    }
  }
  ss = row_sum<TPR>(ss, red);
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(a.cols) + a.eps);
  float amax1 = 0.0f, amax2 = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t vi = lane + static_cast<int64_t>(i) * TPR;
    if (vi < nvec) {
      float g[kVec];
      load8<DT>(a.gamma, vi * kVec, g);
      float bt[kVec] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (QUANT && a.beta) load8<DT>(a.beta, vi * kVec, bt);
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        float v = (x[i][j] * rstd) * g[j];
        if (QUANT && a.beta) v = v + bt[j];
        x[i][j] = round_dt<DT>(v);
      }
      if constexpr (!QUANT) {
        store8<DT>(a.y, base + vi * kVec, x[i]);
      } else {
        float sm[kVec];
        load8_f32_or_one(a.smooth1, vi * kVec, sm);
#pragma unroll
        for (int j = 0; j < kVec; ++j) amax1 = fmaxf(amax1, fabsf(x[i][j] * sm[j]));
        if (a.y2) {
          load8_f32_or_one(a.smooth2, vi * kVec, sm);
#pragma unroll
          for (int j = 0; j < kVec; ++j) amax2 = fmaxf(amax2, fabsf(x[i][j] * sm[j]));
        }
      }
    }
  }
  if constexpr (!QUANT) {
    if (lane == 0 && a.rstd) a.rstd[row] = rstd;
  } else {
    amax1 = row_max<TPR>(amax1, red);
    if (a.y2) amax2 = row_max<TPR>(amax2, red);
    const float sc1 = amax1 / 127.0f, sc2 = amax2 / 127.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t vi = lane + static_cast<int64_t>(i) * TPR;
      if (vi < nvec) {
        float sm[kVec], q[kVec];
        load8_f32_or_one(a.smooth1, vi * kVec, sm);
#pragma unroll
        for (int j = 0; j < kVec; ++j) q[j] = x[i][j] * sm[j];
        *reinterpret_cast<uint2*>(a.y1 + base + vi * kVec) = pack8(q, sc1);
        if (a.y2) {
          load8_f32_or_one(a.smooth2, vi * kVec, sm);
#pragma unroll
          for (int j = 0; j < kVec; ++j) q[j] = x[i][j] * sm[j];
          *reinterpret_cast<uint2*>(a.y2 + base + vi * kVec) = pack8(q, sc2);
        }
      }
    }
    if (lane == 0) {
      a.scale1[row] = sc1;
      if (a.y2) a.scale2[row] = sc2;
    }
  }
}

// Any width (cols % 8 != 0 or wider than the register-resident variants): one workgroup of 256
// threads per row, reading x1 and x2 twice.
template <bool QUANT>
__global__ __launch_bounds__(256) void add_rms_norm_generic_kernel(NormArgs a, int dt) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x, base = row * a.cols;
  float ss = 0.0f;
  for (int64_t c = threadIdx.x; c < a.cols; c += 256) {
    const float v = load_as_f32(a.x1, dt, base + c) + load_as_f32(a.x2, dt, base + c);
    ss += v * v;
    if (a.x_out) store_from_f32(a.x_out, dt, base + c, v);
  }
  ss = row_sum<256>(ss, red);
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(a.cols) + a.eps);
  auto yval = [&](int64_t c) {
    const float v = load_as_f32(a.x1, dt, base + c) + load_as_f32(a.x2, dt, base + c);
    float y = (v * rstd) * load_as_f32(a.gamma, dt, c);
    if (QUANT && a.beta) y = y + load_as_f32(a.beta, dt, c);
    // round to the input dtype through a store / load of one element
    float r = y;
    if (dt == TAI_DT_BF16) r = bf16_to_f32(f32_to_bf16(y));
    else if (dt == TAI_DT_FP16) r = f16_to_f32(f32_to_f16(y));
    return r;
  };
  if constexpr (!QUANT) {
    for (int64_t c = threadIdx.x; c < a.cols; c += 256) store_from_f32(a.y, dt, base + c, yval(c));
    if (threadIdx.x == 0 && a.rstd) a.rstd[row] = rstd;
  } else {
    float m1 = 0.0f, m2 = 0.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += 256) {
      const float y = yval(c);
      m1 = fmaxf(m1, fabsf(a.smooth1 ? y * a.smooth1[c] : y));
      if (a.y2) m2 = fmaxf(m2, fabsf(a.smooth2 ? y * a.smooth2[c] : y));
    }
    m1 = row_max<256>(m1, red);
    if (a.y2) m2 = row_max<256>(m2, red);
    const float sc1 = m1 / 127.0f, sc2 = m2 / 127.0f;
    for (int64_t c = threadIdx.x; c < a.cols; c += 256) {
      const float y = yval(c);
      a.y1[base + c] = quant1(a.smooth1 ? y * a.smooth1[c] : y, sc1);
      if (a.y2) a.y2[base + c] = quant1(a.smooth2 ? y * a.smooth2[c] : y, sc2);
    }
    if (threadIdx.x == 0) {
      a.scale1[row] = sc1;
      if (a.y2) a.scale2[row] = sc2;
    }
  }
}

template <int DT, bool QUANT>
void launch_norm(const NormArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.rows));
  const int64_t nvec = a.cols / kVec;
  if (nvec <= 64 * 4) add_rms_norm_kernel<DT, 64, 4, QUANT><<<grid, 64, 0, st>>>(a);
  else if (nvec <= 256 * 2) add_rms_norm_kernel<DT, 256, 2, QUANT><<<grid, 256, 0, st>>>(a);
  else add_rms_norm_kernel<DT, 256, 4, QUANT><<<grid, 256, 0, st>>>(a);
}

template <bool QUANT>
int run_norm(const NormArgs& a, int dt, hipStream_t st, const char* what) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  const bool vec = a.cols % kVec == 0 && a.cols / kVec <= 256 * 4 && al(a.x1) && al(a.x2) && al(a.gamma) &&
                   (!a.beta || al(a.beta)) && (!a.x_out || al(a.x_out)) && (QUANT || al(a.y)) &&
                   (!QUANT || (al(a.y1) && (!a.y2 || al(a.y2)) && (!a.smooth1 || al(a.smooth1)) &&
                               (!a.smooth2 || al(a.smooth2))));
  if (!vec) {
    add_rms_norm_generic_kernel<QUANT><<<dim3(static_cast<unsigned>(a.rows)), 256, 0, st>>>(a, dt);
  } else if (dt == TAI_DT_BF16) {
    launch_norm<TAI_DT_BF16, QUANT>(a, st);
  } else if (dt == TAI_DT_FP16) {
    launch_norm<TAI_DT_FP16, QUANT>(a, st);
  } else {
    launch_norm<TAI_DT_FP32, QUANT>(a, st);
  }
  return launch_status(what);
}

// ----------------------------------------------------------------------------- scatter_pa_kv_cache
// One wave per token: its key row and its value row go to the cache slot slot_mapping[t]
// (negative slots are skipped). Norm layout: the cache row of a slot is contiguous. PA_NZ
// layout ([blocks, row_bytes / 32, block_size, 32 bytes]): 32-byte pieces of the row are
// block_size * 32 bytes apart.
__global__ __launch_bounds__(64) void scatter_kv_kernel(const char* __restrict__ key, const char* __restrict__ value,
                                                        char* __restrict__ kc, char* __restrict__ vc,
                                                        const void* __restrict__ slots, int slot_dt, int64_t t_n,
                                                        int64_t kbytes, int64_t vbytes, int64_t bs, int64_t nslots,
                                                        int nz) {
  const int64_t t = blockIdx.x;
  const int64_t slot = load_index(slots, slot_dt, t);
  if (slot < 0 || slot >= nslots) return;
  const int64_t blk = slot / bs, off = slot % bs;
  auto copy = [&](const char* src, char* dst_base, int64_t rb) {
    for (int64_t p = threadIdx.x; p < rb / 16; p += 64) {
      int64_t d;
      if (nz) {
        const int64_t byte = p * 16, piece = byte / 32;
        d = ((blk * (rb / 32) + piece) * bs + off) * 32 + (byte % 32);
      } else {
        d = slot * rb + p * 16;
      }
      *reinterpret_cast<uint4*>(dst_base + d) = *reinterpret_cast<const uint4*>(src + t * rb + p * 16);
    }
  };
  copy(key, kc, kbytes);
  copy(value, vc, vbytes);
}

// ----------------------------------------------------------------------------- kv_rmsnorm_rope_cache
struct KvArgs {
  const void* kv;     // [tokens, dc + dr]
  const void* gamma;  // [dc]
  const void* cos;    // [tokens, dr]
  const void* sin;
  const int64_t* index;  // [tokens]: cache row (PA: slot; Norm: position in the batch's cache rows)
  int64_t tokens, seq;   // seq: tokens per batch (Norm mode: batch = token / seq)
  int dc, dr;
  float eps;
  void* k_cache;   // rows of dr (kv dtype, or int8 with k_scale)
  void* ckv_cache; // rows of dc (kv dtype, or int8)
  int64_t cache_rows;      // rows in each cache (bounds check)
  int64_t norm_rows;       // Norm mode: cache rows per batch (0 for PA)
  int k_int8, ckv_int8;
  const float* k_scale;    // static per-channel quant of k_rope: [dr]
  const float* k_offset;
  const float* ckv_scale;  // static per-channel quant of c_kv: [dc]
  const float* ckv_offset;
  float* ckv_token_scale;  // per-token quant of c_kv: [cache_rows], written at the token's row
  void* k_rope_out;        // [tokens, dr] (may be null)
  void* c_kv_out;          // [tokens, dc] (may be null)
};

__device__ __forceinline__ int8_t quant_static(float v, float scale, float offset) {
  const float q = fminf(fmaxf(rintf(v * scale + offset), -128.0f), 127.0f);
  return static_cast<int8_t>(static_cast<int>(q));
}

// One wave per token; the latent row (dc <= 64 * 8 * NV) stays in registers.
template <int DT, int NV>
__global__ __launch_bounds__(64) void kv_rmsnorm_rope_kernel(KvArgs a) {
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t idx = a.index[t];
  const int64_t row = a.norm_rows > 0 ? (t / a.seq) * a.norm_rows + idx : idx;
  const bool write = idx >= 0 && row < a.cache_rows && (a.norm_rows == 0 || idx < a.norm_rows);
  const int64_t w = a.dc + a.dr;
  const int nvec = a.dc / kVec;
  // --- latent: RMS norm
  float c[NV][kVec];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = lane + 64 * i;
    if (vi < nvec) {
      load8<DT>(a.kv, t * w + vi * kVec, c[i]);
#pragma unroll
      for (int j = 0; j < kVec; ++j) ss += c[i][j] * c[i][j];
    }
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(a.dc) + a.eps);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = lane + 64 * i;
    if (vi < nvec) {
      float g[kVec];
      load8<DT>(a.gamma, vi * kVec, g);
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        c[i][j] = round_dt<DT>((c[i][j] * rstd) * g[j]);
        amax = fmaxf(amax, fabsf(c[i][j]));
      }
      if (a.c_kv_out) store8<DT>(a.c_kv_out, t * a.dc + vi * kVec, c[i]);
    }
  }
  if (a.ckv_int8 && a.ckv_token_scale) amax = wave_max(amax);
  const float tok_scale = amax / 127.0f;
  if (write) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = lane + 64 * i;
      if (vi < nvec) {
        if (!a.ckv_int8) {
          store8<DT>(a.ckv_cache, row * a.dc + vi * kVec, c[i]);
        } else if (a.ckv_token_scale) {
          *reinterpret_cast<uint2*>(static_cast<int8_t*>(a.ckv_cache) + row * a.dc + vi * kVec) = pack8(c[i], tok_scale);
        } else {
          uint32_t wd[2] = {0, 0};
#pragma unroll
          for (int j = 0; j < kVec; ++j) {
            const int col = vi * kVec + j;
            const int8_t q = quant_static(c[i][j], a.ckv_scale[col], a.ckv_offset ? a.ckv_offset[col] : 0.0f);
            wd[j >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(q)) << (8 * (j & 3));
          }
          *reinterpret_cast<uint2*>(static_cast<int8_t*>(a.ckv_cache) + row * a.dc + vi * kVec) = make_uint2(wd[0], wd[1]);
        }
      }
    }
    if (a.ckv_int8 && a.ckv_token_scale && lane == 0) a.ckv_token_scale[row] = tok_scale;
  }
  // --- rope part: lane i < dr/2 produces output dims i and i + dr/2 from the pair (2i, 2i + 1)
  const int h = a.dr / 2;
  if (lane < h) {
    const int64_t rb = t * w + a.dc;
    const float xe = load_as_f32(a.kv, DT, rb + 2 * lane), xo = load_as_f32(a.kv, DT, rb + 2 * lane + 1);
    const float c0 = load_as_f32(a.cos, DT, t * a.dr + lane), c1 = load_as_f32(a.cos, DT, t * a.dr + lane + h);
    const float s0 = load_as_f32(a.sin, DT, t * a.dr + lane), s1 = load_as_f32(a.sin, DT, t * a.dr + lane + h);
    const float o0 = round_dt<DT>(xe * c0 - xo * s0);
    const float o1 = round_dt<DT>(xo * c1 + xe * s1);
    if (a.k_rope_out) {
      store_from_f32(a.k_rope_out, DT, t * a.dr + lane, o0);
      store_from_f32(a.k_rope_out, DT, t * a.dr + lane + h, o1);
    }
    if (write) {
      if (!a.k_int8) {
        store_from_f32(a.k_cache, DT, row * a.dr + lane, o0);
        store_from_f32(a.k_cache, DT, row * a.dr + lane + h, o1);
      } else {
        int8_t* kq = static_cast<int8_t*>(a.k_cache) + row * a.dr;
        kq[lane] = quant_static(o0, a.k_scale[lane], a.k_offset ? a.k_offset[lane] : 0.0f);
        kq[lane + h] = quant_static(o1, a.k_scale[lane + h], a.k_offset ? a.k_offset[lane + h] : 0.0f);
      }
    }
  }
}

template <int DT>
void launch_kv(const KvArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(a.tokens));
  const int nvec = a.dc / kVec;
  if (nvec <= 64) kv_rmsnorm_rope_kernel<DT, 1><<<grid, 64, 0, st>>>(a);
  else if (nvec <= 128) kv_rmsnorm_rope_kernel<DT, 2><<<grid, 64, 0, st>>>(a);
  else kv_rmsnorm_rope_kernel<DT, 4><<<grid, 64, 0, st>>>(a);
}

bool is_float_dt(int dt) { return dt == TAI_DT_BF16 || dt == TAI_DT_FP16 || dt == TAI_DT_FP32; }

}  // namespace
}  // namespace tai

using namespace tai;

extern "C" int tai_add_rms_norm(const void* x1, const void* x2, const void* gamma, int dtype, int64_t rows,
                                int64_t cols, float epsilon, void* y, float* rstd, void* x_out, void* stream) {
  TAI_CHECK_ARG(is_float_dt(dtype), "tai_add_rms_norm: dtype %d not supported (bf16, fp16, fp32)", dtype);
  TAI_CHECK_ARG(rows >= 0 && cols >= 1, "tai_add_rms_norm: bad sizes");
  if (rows == 0) return TAI_OK;
  TAI_CHECK_ARG(x1 && x2 && gamma && y, "tai_add_rms_norm: null pointer");
  NormArgs a{};
  a.x1 = x1; a.x2 = x2; a.gamma = gamma; a.rows = rows; a.cols = cols; a.eps = epsilon;
  a.y = y; a.rstd = rstd; a.x_out = x_out;
  return run_norm<false>(a, dtype, static_cast<hipStream_t>(stream), "tai_add_rms_norm");
}

extern "C" int tai_add_rms_norm_dynamic_quant(const void* x1, const void* x2, const void* gamma, const void* beta,
                                              const float* smooth_scale1, const float* smooth_scale2, int dtype,
                                              int64_t rows, int64_t cols, float epsilon, int8_t* y1, int8_t* y2,
                                              void* x_out, float* scale1, float* scale2, void* stream) {
  TAI_CHECK_ARG(is_float_dt(dtype), "tai_add_rms_norm_dynamic_quant: dtype %d not supported (bf16, fp16, fp32)",
                dtype);
  TAI_CHECK_ARG(rows >= 0 && cols >= 1, "tai_add_rms_norm_dynamic_quant: bad sizes");
  TAI_CHECK_ARG(!y2 || scale2, "tai_add_rms_norm_dynamic_quant: y2 needs scale2");
  if (rows == 0) return TAI_OK;
  TAI_CHECK_ARG(x1 && x2 && gamma && y1 && scale1, "tai_add_rms_norm_dynamic_quant: null pointer");
  NormArgs a{};
  a.x1 = x1; a.x2 = x2; a.gamma = gamma; a.beta = beta; a.smooth1 = smooth_scale1; a.smooth2 = smooth_scale2;
  a.rows = rows; a.cols = cols; a.eps = epsilon; a.x_out = x_out; a.y1 = y1; a.y2 = y2; a.scale1 = scale1;
  a.scale2 = scale2;
  return run_norm<true>(a, dtype, static_cast<hipStream_t>(stream), "tai_add_rms_norm_dynamic_quant");
}

extern "C" int tai_scatter_pa_kv_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                                       const void* slot_mapping, int slot_dtype, int64_t tokens, int64_t key_row_bytes,
                                       int64_t value_row_bytes, int64_t num_blocks, int64_t block_size,
                                       int cache_mode, void* stream) {
  TAI_CHECK_ARG(tokens >= 0 && num_blocks >= 0 && block_size >= 1, "tai_scatter_pa_kv_cache: bad sizes");
  TAI_CHECK_ARG(slot_dtype == TAI_DT_INT32 || slot_dtype == TAI_DT_INT64,
                "tai_scatter_pa_kv_cache: slot_mapping must be int32 or int64");
  TAI_CHECK_ARG(cache_mode == TAI_CACHE_NORM || cache_mode == TAI_CACHE_PA_NZ,
                "tai_scatter_pa_kv_cache: cache_mode must be Norm or PA_NZ");
  const int64_t gran = cache_mode == TAI_CACHE_PA_NZ ? 32 : 16;
  TAI_CHECK_ARG(key_row_bytes % gran == 0 && value_row_bytes % gran == 0,
                "tai_scatter_pa_kv_cache: cache rows must be multiples of %lld bytes", static_cast<long long>(gran));
  if (tokens == 0) return TAI_OK;
  TAI_CHECK_ARG(key && value && key_cache && value_cache && slot_mapping, "tai_scatter_pa_kv_cache: null pointer");
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  TAI_CHECK_ARG(al(key) && al(value) && al(key_cache) && al(value_cache),
                "tai_scatter_pa_kv_cache: tensors must be 16-byte aligned");
  scatter_kv_kernel<<<dim3(static_cast<unsigned>(tokens)), 64, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const char*>(key), static_cast<const char*>(value), static_cast<char*>(key_cache),
      static_cast<char*>(value_cache), slot_mapping, slot_dtype, tokens, key_row_bytes, value_row_bytes, block_size,
      num_blocks * block_size, cache_mode == TAI_CACHE_PA_NZ);
  return launch_status("tai_scatter_pa_kv_cache");
}

extern "C" int tai_kv_rmsnorm_rope_cache(const void* kv, const void* gamma, const void* cos, const void* sin,
                                         const int64_t* index, int dtype, int64_t tokens, int64_t seq, int dc, int dr,
                                         float epsilon, void* k_cache, int k_cache_dtype, void* ckv_cache,
                                         int ckv_cache_dtype, int64_t cache_rows, int64_t norm_rows,
                                         const float* k_rope_scale, const float* k_rope_offset,
                                         const float* c_kv_scale, const float* c_kv_offset, float* c_kv_token_scale,
                                         void* k_rope_out, void* c_kv_out, void* stream) {
  TAI_CHECK_ARG(is_float_dt(dtype), "tai_kv_rmsnorm_rope_cache: kv dtype %d not supported", dtype);
  TAI_CHECK_ARG(dc >= 8 && dc % 8 == 0 && dc <= 2048, "tai_kv_rmsnorm_rope_cache: latent width %d (multiple of 8, <= 2048)", dc);
  TAI_CHECK_ARG(dr >= 2 && dr % 2 == 0 && dr <= 128, "tai_kv_rmsnorm_rope_cache: rope width %d (even, <= 128)", dr);
  TAI_CHECK_ARG(tokens >= 0 && seq >= 1 && cache_rows >= 0 && norm_rows >= 0, "tai_kv_rmsnorm_rope_cache: bad sizes");
  TAI_CHECK_ARG(k_cache_dtype == dtype || k_cache_dtype == TAI_DT_INT8,
                "tai_kv_rmsnorm_rope_cache: k_cache must have the kv dtype or int8");
  TAI_CHECK_ARG(ckv_cache_dtype == dtype || ckv_cache_dtype == TAI_DT_INT8,
                "tai_kv_rmsnorm_rope_cache: ckv_cache must have the kv dtype or int8");
  TAI_CHECK_ARG(k_cache_dtype != TAI_DT_INT8 || k_rope_scale, "tai_kv_rmsnorm_rope_cache: int8 k_cache needs k_rope_scale");
  TAI_CHECK_ARG(ckv_cache_dtype != TAI_DT_INT8 || (c_kv_scale != nullptr) != (c_kv_token_scale != nullptr),
                "tai_kv_rmsnorm_rope_cache: int8 ckv_cache needs exactly one of a per-channel c_kv_scale or a "
                "per-token scale cache");
  if (tokens == 0) return TAI_OK;
  TAI_CHECK_ARG(kv && gamma && cos && sin && index && k_cache && ckv_cache, "tai_kv_rmsnorm_rope_cache: null pointer");
  auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  const int es = dtype == TAI_DT_FP32 ? 4 : 2;
  TAI_CHECK_ARG(al(kv) && al(gamma) && al(ckv_cache) && al(c_kv_out) && ((dc + dr) * es) % 16 == 0,
                "tai_kv_rmsnorm_rope_cache: kv rows, gamma and the latent cache must be 16-byte aligned");
  KvArgs a{};
  a.kv = kv; a.gamma = gamma; a.cos = cos; a.sin = sin; a.index = index; a.tokens = tokens; a.seq = seq;
  a.dc = dc; a.dr = dr; a.eps = epsilon; a.k_cache = k_cache; a.ckv_cache = ckv_cache; a.cache_rows = cache_rows;
  a.norm_rows = norm_rows; a.k_int8 = k_cache_dtype == TAI_DT_INT8; a.ckv_int8 = ckv_cache_dtype == TAI_DT_INT8;
  a.k_scale = k_rope_scale; a.k_offset = k_rope_offset; a.ckv_scale = c_kv_scale; a.ckv_offset = c_kv_offset;
  a.ckv_token_scale = c_kv_token_scale; a.k_rope_out = k_rope_out; a.c_kv_out = c_kv_out;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == TAI_DT_BF16) launch_kv<TAI_DT_BF16>(a, st);
  else if (dtype == TAI_DT_FP16) launch_kv<TAI_DT_FP16>(a, st);
  else launch_kv<TAI_DT_FP32>(a, st);
  return launch_status("tai_kv_rmsnorm_rope_cache");
}
