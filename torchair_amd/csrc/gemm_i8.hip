// W8A8 GEMMs: npu_quant_matmul and npu_grouped_matmul (int8 x int8 -> exact int32).
//
// Tiling: 256 threads = 2x2 waves; a workgroup computes a BM x BN tile, each wave a
// (BM/2) x (BN/2) sub-tile made of 32x32 v_mfma_i32_32x32x32_i8 tiles. K advances in
// steps of BK=64 bytes through two LDS buffers (one barrier per step): the next step's
// global loads are issued before the current step's MFMAs.
// LDS holds both operands K-contiguous ([row][BK+16], the +16 byte pad makes the 16-byte
// fragment reads of 16 consecutive rows hit 64 distinct banks). A [K,N] (N-contiguous)
// weight is transposed in registers with v_perm_b32 on its way into LDS; a [N,K] weight
// is copied as is.
// Grouped GEMM: a one-workgroup prologue turns the device-resident group_list into a
// table of (group, row range) tiles, so the launch geometry depends only on host-known
// sizes and the call can be captured into a hipGraph. Rows past the last group are zeroed.
// Linear workgroup ids are remapped so that each XCD (ids dispatched round-robin over 8
// XCDs) receives a contiguous range of tiles: tiles that share activation rows and weight
// columns meet in the same L2.
#include "common.h"

namespace tai {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;
constexpr int kPad = 16;
constexpr int kLdk = kBK + kPad;  // LDS row stride in bytes
constexpr int kXcds = 8;

struct GemmArgs {
  const int8_t* a;
  const int8_t* b;
  int64_t m, k, n;
  int64_t b_group_stride;  // elements between consecutive groups of b
  const float* scale;
  int64_t scale_len;        // 1 or n (per group)
  int64_t scale_group_stride;
  const float* pts;
  const void* bias;
  int bias_dt;
  int64_t bias_group_stride;
  int out_dt;
  void* out;
  const int4* tile_map;  // grouped: (group, row_begin, row_end, kind); kind -1 unused, -2 zero-fill
  int64_t m_slots;
  int64_t n_tiles;
};

__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nb) {
  const int64_t xcd = b % kXcds, idx = b / kXcds;
  const int64_t per = nb / kXcds, rem = nb % kXcds;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// 4x4 byte transpose: in[r] holds bytes (r,0..3); out[c] holds bytes (0..3,c).
__device__ __forceinline__ void transpose4x4(const uint32_t (&in)[4], uint32_t (&out)[4]) {
  const uint32_t lo01 = perm_b32(in[1], in[0], 0x05010400u);
  const uint32_t hi01 = perm_b32(in[1], in[0], 0x07030602u);
  const uint32_t lo23 = perm_b32(in[3], in[2], 0x05010400u);
  const uint32_t hi23 = perm_b32(in[3], in[2], 0x07030602u);
  out[0] = perm_b32(lo23, lo01, 0x05040100u);
  out[1] = perm_b32(lo23, lo01, 0x07060302u);
  out[2] = perm_b32(hi23, hi01, 0x05040100u);
  out[3] = perm_b32(hi23, hi01, 0x07060302u);
}

template <int BM, int BN, int LAYOUT>
struct Tile {
  static constexpr int kAChunks = BM * kBK / 16 / 256;  // 16-byte chunks of A per thread
  static constexpr int kBChunksNK = BN * kBK / 16 / 256;
  static constexpr int kNG = BN / 4;                    // KN: 4-column groups
  static constexpr int kKR = kBK * kNG / 256;           // KN: k rows per thread
  static_assert(kAChunks >= 1 && kBChunksNK >= 1, "tile too small");
  static_assert(kKR % 4 == 0, "KN loader needs a multiple of 4 rows per thread");

  uint4 ra[kAChunks];
  uint4 rbn[LAYOUT == TAI_LAYOUT_NK ? kBChunksNK : 1];
  uint32_t rbk[LAYOUT == TAI_LAYOUT_KN ? kKR : 1];

  __device__ __forceinline__ void load(const GemmArgs& g, const int8_t* bgrp, int row0, int rows, int64_t n0,
                                       int64_t k0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAChunks; ++i) {
      const int c = tid + i * 256, r = c >> 2, kc = c & 3;
      const int64_t kk = k0 + kc * 16;
      ra[i] = (r < rows && kk < g.k) ? *reinterpret_cast<const uint4*>(g.a + (row0 + r) * g.k + kk)
                                     : make_uint4(0, 0, 0, 0);
    }
    if constexpr (LAYOUT == TAI_LAYOUT_NK) {
#pragma unroll
      for (int i = 0; i < kBChunksNK; ++i) {
        const int c = tid + i * 256, r = c >> 2, kc = c & 3;
        const int64_t kk = k0 + kc * 16, nn = n0 + r;
        rbn[i] = (nn < g.n && kk < g.k) ? *reinterpret_cast<const uint4*>(bgrp + nn * g.k + kk)
                                        : make_uint4(0, 0, 0, 0);
      }
    } else {
      const int ng = tid % kNG, kg = tid / kNG;
      const int64_t nn = n0 + 4 * ng;
#pragma unroll
      for (int r = 0; r < kKR; ++r) {
        const int64_t kk = k0 + kg * kKR + r;
        rbk[r] = (nn < g.n && kk < g.k) ? *reinterpret_cast<const uint32_t*>(bgrp + kk * g.n + nn) : 0u;
      }
    }
  }

  __device__ __forceinline__ void store(int8_t* as, int8_t* bs) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAChunks; ++i) {
      const int c = tid + i * 256, r = c >> 2, kc = c & 3;
      *reinterpret_cast<uint4*>(as + r * kLdk + kc * 16) = ra[i];
    }
    if constexpr (LAYOUT == TAI_LAYOUT_NK) {
#pragma unroll
      for (int i = 0; i < kBChunksNK; ++i) {
        const int c = tid + i * 256, r = c >> 2, kc = c & 3;
        *reinterpret_cast<uint4*>(bs + r * kLdk + kc * 16) = rbn[i];
      }
    } else {
      const int ng = tid % kNG, kg = tid / kNG;
      uint32_t cols[kKR / 4][4];
#pragma unroll
      for (int q = 0; q < kKR / 4; ++q) {
        const uint32_t in[4] = {rbk[4 * q], rbk[4 * q + 1], rbk[4 * q + 2], rbk[4 * q + 3]};
        transpose4x4(in, cols[q]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        int8_t* dst = bs + (4 * ng + c) * kLdk + kg * kKR;
        if constexpr (kKR == 8) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(cols[0][c], cols[1][c]);
        } else {
#pragma unroll
          for (int q = 0; q < kKR / 4; ++q) *reinterpret_cast<uint32_t*>(dst + 4 * q) = cols[q][c];
        }
      }
    }
  }
};

__device__ __forceinline__ float epilogue_value(const GemmArgs& g, int e, int64_t row, int64_t col, int32_t acc,
                                                const float* bias_f) {
  float v = static_cast<float>(acc);
  if (g.scale) v = v * g.scale[e * g.scale_group_stride + (g.scale_len == 1 ? 0 : col)];
  if (g.pts) v = v * g.pts[row];
  if (bias_f) v = v + bias_f[col];
  return v;
}

template <int BM, int BN, int LAYOUT>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) int8_t s_a[2][BM * kLdk];
  __shared__ __attribute__((aligned(16))) int8_t s_b[2][BN * kLdk];
  constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;

  const int64_t nb = g.m_slots * g.n_tiles;
  const int64_t L = xcd_remap(blockIdx.x, nb);
  const int64_t slot = L / g.n_tiles, nt = L % g.n_tiles;
  const int64_t n0 = nt * BN;
  int e = 0, row0, row1;
  if (g.tile_map) {
    const int4 t = g.tile_map[slot];
    if (t.x == -1) return;
    row0 = t.y;
    row1 = t.z;
    if (t.x == -2) {  // rows past the grouped total
      for (int idx = threadIdx.x; idx < (row1 - row0) * BN; idx += 256) {
        const int64_t r = row0 + idx / BN, c = n0 + idx % BN;
        if (c < g.n) {
          if (g.out_dt == TAI_DT_INT32) static_cast<int32_t*>(g.out)[r * g.n + c] = 0;
          else store_from_f32(g.out, g.out_dt, r * g.n + c, 0.0f);
        }
      }
      return;
    }
    e = t.x;
  } else {
    row0 = static_cast<int>(slot * BM);
    row1 = static_cast<int>(min<int64_t>(g.m, row0 + BM));
  }
  const int rows = row1 - row0;
  const int8_t* bgrp = g.b + static_cast<int64_t>(e) * g.b_group_stride;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  Tile<BM, BN, LAYOUT> tile;
  const int64_t nk = cdiv(g.k, kBK);
  tile.load(g, bgrp, row0, rows, n0, 0);
  tile.store(s_a[0], s_b[0]);
  __syncthreads();

  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) tile.load(g, bgrp, row0, rows, n0, (kt + 1) * kBK);
    const int8_t* as = s_a[buf];
    const int8_t* bs = s_b[buf];
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      v4i fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const v4i*>(as + (wm * WM + i * 32 + (lane & 31)) * kLdk + kk * 32 + (lane >> 5) * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *reinterpret_cast<const v4i*>(bs + (wn * WN + j * 32 + (lane & 31)) * kLdk + kk * 32 + (lane >> 5) * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) tile.store(s_a[buf ^ 1], s_b[buf ^ 1]);
    __syncthreads();
  }

  // Epilogue. C layout of a 32x32 tile: lane holds column lane%32, rows 8*(r/4) + 4*(lane/32) + r%4.
  const int32_t* bias_i = (g.bias && g.bias_dt == TAI_DT_INT32)
                              ? static_cast<const int32_t*>(g.bias) + e * g.bias_group_stride : nullptr;
  const float* bias_f = (g.bias && g.bias_dt == TAI_DT_FP32)
                            ? static_cast<const float*>(g.bias) + e * g.bias_group_stride : nullptr;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * WN + j * 32 + (lane & 31);
    if (col >= g.n) continue;
    const int32_t bcol = bias_i ? bias_i[col] : 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = wm * WM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (lr >= rows) continue;
        const int64_t row = row0 + lr;
        const int32_t v = acc[i][j][r] + bcol;
        if (g.out_dt == TAI_DT_INT32) static_cast<int32_t*>(g.out)[row * g.n + col] = v;
        else store_from_f32(g.out, g.out_dt, row * g.n + col, epilogue_value(g, e, row, col, v, bias_f));
      }
    }
  }
}

// Any shape or alignment: one thread per output element.
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(GemmArgs g, int layout, const int32_t* row_group) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= g.m * g.n) return;
  const int64_t row = idx / g.n, col = idx % g.n;
  const int e = row_group ? row_group[row] : 0;
  if (e < 0) {
    if (g.out_dt == TAI_DT_INT32) static_cast<int32_t*>(g.out)[idx] = 0;
    else store_from_f32(g.out, g.out_dt, idx, 0.0f);
    return;
  }
  const int8_t* bgrp = g.b + static_cast<int64_t>(e) * g.b_group_stride;
  int32_t acc = 0;
  for (int64_t kk = 0; kk < g.k; ++kk) {
    const int32_t bv = layout == TAI_LAYOUT_NK ? bgrp[col * g.k + kk] : bgrp[kk * g.n + col];
    acc += static_cast<int32_t>(g.a[row * g.k + kk]) * bv;
  }
  if (g.bias && g.bias_dt == TAI_DT_INT32) acc += static_cast<const int32_t*>(g.bias)[e * g.bias_group_stride + col];
  const float* bias_f = (g.bias && g.bias_dt == TAI_DT_FP32)
                            ? static_cast<const float*>(g.bias) + e * g.bias_group_stride : nullptr;
  if (g.out_dt == TAI_DT_INT32) static_cast<int32_t*>(g.out)[idx] = acc;
  else store_from_f32(g.out, g.out_dt, idx, epilogue_value(g, e, row, col, acc, bias_f));
}

// ----------------------------------------------------------------------------- grouped prologue
// Builds the tile table for row tiles of height bm, plus a row->group map for the generic path.
__global__ __launch_bounds__(1024) void group_tiles_kernel(const int64_t* __restrict__ gl, int64_t ng, int list_type,
                                                          int64_t m, int bm, int4* __restrict__ map, int64_t slots,
                                                          int32_t* __restrict__ row_group) {
  extern __shared__ int64_t sh[];  // begin[ng], end[ng], tile_prefix[ng + 1]
  int64_t* beg = sh;
  int64_t* end = sh + ng;
  int64_t* tp = sh + 2 * ng;
  if (threadIdx.x == 0) {
    int64_t run = 0, tiles = 0;
    for (int64_t e = 0; e < ng; ++e) {
      int64_t b = run, en;
      if (list_type == 1) en = run + max<int64_t>(gl[e], 0);
      else en = max<int64_t>(gl[e], run);
      b = min<int64_t>(b, m);
      en = min<int64_t>(en, m);
      beg[e] = b;
      end[e] = en;
      tp[e] = tiles;
      tiles += (en - b + bm - 1) / bm;
      run = en;
    }
    tp[ng] = tiles;
  }
  __syncthreads();
  const int64_t real = tp[ng];
  const int64_t covered = ng > 0 ? end[ng - 1] : 0;
  const int64_t zero_tiles = (m - covered + bm - 1) / bm;
  for (int64_t s = threadIdx.x; s < slots; s += blockDim.x) {
    int4 t = make_int4(-1, 0, 0, 0);
    if (s < real) {
      int64_t lo = 0, hi = ng - 1;  // last e with tp[e] <= s
      while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (tp[mid] <= s) lo = mid; else hi = mid - 1;
      }
      const int64_t r0 = beg[lo] + (s - tp[lo]) * bm;
      t = make_int4(static_cast<int>(lo), static_cast<int>(r0), static_cast<int>(min<int64_t>(r0 + bm, end[lo])), 0);
    } else if (s < real + zero_tiles) {
      const int64_t r0 = covered + (s - real) * bm;
      t = make_int4(-2, static_cast<int>(r0), static_cast<int>(min<int64_t>(r0 + bm, m)), 0);
    }
    map[s] = t;
  }
  if (row_group) {
    for (int64_t r = threadIdx.x; r < m; r += blockDim.x) {
      int64_t lo = 0, hi = ng;  // first e with end[e] > r
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (end[mid] > r) hi = mid; else lo = mid + 1;
      }
      row_group[r] = (lo < ng && r >= beg[lo]) ? static_cast<int32_t>(lo) : -1;
    }
  }
}

bool fast_path_ok(const GemmArgs& g, int layout) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  if (g.k % 16 != 0 || !al(g.a) || !al(g.b)) return false;
  if (layout == TAI_LAYOUT_KN && g.n % 4 != 0) return false;
  if (layout == TAI_LAYOUT_KN && (g.b_group_stride % 16) != 0) return false;
  return g.m < (1ll << 31) && g.n < (1ll << 31);
}

template <int BM, int BN>
void launch_tile(const GemmArgs& g, int layout, hipStream_t st) {
  const int64_t nb = g.m_slots * g.n_tiles;
  if (layout == TAI_LAYOUT_NK) gemm_i8_kernel<BM, BN, TAI_LAYOUT_NK><<<dim3(static_cast<unsigned>(nb)), 256, 0, st>>>(g);
  else gemm_i8_kernel<BM, BN, TAI_LAYOUT_KN><<<dim3(static_cast<unsigned>(nb)), 256, 0, st>>>(g);
}

constexpr int kGroupedBM = 128;
constexpr int kMinBM = 32;  // workspace is sized for the smallest row tile any variant uses

size_t grouped_map_slots(int64_t m, int64_t ng, int bm) { return static_cast<size_t>(2 * cdiv(m, bm) + ng); }

}  // namespace
}  // namespace tai

using namespace tai;

extern "C" int tai_quant_matmul(const int8_t* x1, const int8_t* x2, int64_t m, int64_t k, int64_t n, int x2_layout,
                                const float* scale, int64_t scale_len, const float* pertoken_scale, const void* bias,
                                int bias_dtype, int out_dtype, void* out, void* stream) {
  TAI_CHECK_ARG(m >= 0 && k >= 0 && n >= 0, "tai_quant_matmul: negative size");
  TAI_CHECK_ARG(x2_layout == TAI_LAYOUT_KN || x2_layout == TAI_LAYOUT_NK, "tai_quant_matmul: x2_layout");
  TAI_CHECK_ARG(out_dtype == TAI_DT_INT32 || out_dtype == TAI_DT_BF16 || out_dtype == TAI_DT_FP16 ||
                    out_dtype == TAI_DT_FP32,
                "tai_quant_matmul: output dtype %d not supported (int32, bf16, fp16, fp32)", out_dtype);
  TAI_CHECK_ARG(out_dtype == TAI_DT_INT32 || scale != nullptr, "tai_quant_matmul: floating output needs scale");
  TAI_CHECK_ARG(scale == nullptr || scale_len == 1 || scale_len == n, "tai_quant_matmul: scale must have 1 or n entries");
  TAI_CHECK_ARG(bias == nullptr || bias_dtype == TAI_DT_INT32 || bias_dtype == TAI_DT_FP32,
                "tai_quant_matmul: bias must be int32 or fp32");
  TAI_CHECK_ARG(!(out_dtype == TAI_DT_INT32 && bias && bias_dtype != TAI_DT_INT32),
                "tai_quant_matmul: int32 output takes an int32 bias only");
  if (m == 0 || n == 0) return TAI_OK;
  TAI_CHECK_ARG(x1 && x2 && out, "tai_quant_matmul: null pointer");
  GemmArgs g{x1, x2, m, k, n, 0, scale, scale_len, 0, pertoken_scale, bias, bias_dtype, 0, out_dtype, out,
             nullptr, 0, 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!fast_path_ok(g, x2_layout)) {
    gemm_i8_generic_kernel<<<dim3(static_cast<unsigned>(cdiv(m * n, 256))), 256, 0, st>>>(g, x2_layout, nullptr);
    return launch_status("tai_quant_matmul");
  }
  // Small M leaves most CUs idle with 128-wide tiles; use narrower N tiles there.
  const bool narrow = cdiv(m, 128) * cdiv(n, 128) < 512;
  if (narrow) {
    g.m_slots = cdiv(m, 128);
    g.n_tiles = cdiv(n, 64);
    launch_tile<128, 64>(g, x2_layout, st);
  } else {
    g.m_slots = cdiv(m, 128);
    g.n_tiles = cdiv(n, 128);
    launch_tile<128, 128>(g, x2_layout, st);
  }
  return launch_status("tai_quant_matmul");
}

extern "C" size_t tai_grouped_matmul_workspace_size(int64_t m, int64_t n, int64_t num_groups) {
  (void)n;
  return sizeof(int4) * grouped_map_slots(m, num_groups, kMinBM) + sizeof(int32_t) * static_cast<size_t>(m) + 256;
}

extern "C" int tai_grouped_matmul(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                                  int64_t num_groups, int w_layout, const int64_t* group_list, int group_list_type,
                                  const float* scale, const float* per_token_scale, const void* bias, int bias_dtype,
                                  int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(m >= 0 && k >= 0 && n >= 0 && num_groups >= 1, "tai_grouped_matmul: bad sizes");
  TAI_CHECK_ARG(num_groups <= 2048, "tai_grouped_matmul: at most 2048 groups");
  TAI_CHECK_ARG(w_layout == TAI_LAYOUT_KN || w_layout == TAI_LAYOUT_NK, "tai_grouped_matmul: w_layout");
  TAI_CHECK_ARG(group_list_type == 0 || group_list_type == 1, "tai_grouped_matmul: group_list_type must be 0 or 1");
  TAI_CHECK_ARG(out_dtype == TAI_DT_INT32 || out_dtype == TAI_DT_BF16 || out_dtype == TAI_DT_FP16 ||
                    out_dtype == TAI_DT_FP32,
                "tai_grouped_matmul: output dtype %d not supported (int32, bf16, fp16, fp32)", out_dtype);
  TAI_CHECK_ARG(out_dtype == TAI_DT_INT32 || scale != nullptr, "tai_grouped_matmul: floating output needs scale");
  TAI_CHECK_ARG(bias == nullptr || bias_dtype == TAI_DT_INT32 || bias_dtype == TAI_DT_FP32,
                "tai_grouped_matmul: bias must be int32 or fp32");
  TAI_CHECK_ARG(group_list != nullptr, "tai_grouped_matmul: group_list is required");
  if (m == 0 || n == 0) return TAI_OK;
  TAI_CHECK_ARG(x && weight && out, "tai_grouped_matmul: null pointer");
  TAI_CHECK_ARG(m < (1ll << 31), "tai_grouped_matmul: m must be < 2^31");
  const size_t need = tai_grouped_matmul_workspace_size(m, n, num_groups);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_grouped_matmul: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int bm = kGroupedBM;
  const int64_t slots = static_cast<int64_t>(grouped_map_slots(m, num_groups, bm));
  int4* map = static_cast<int4*>(workspace);
  int32_t* row_group = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                                  sizeof(int4) * grouped_map_slots(m, num_groups, kMinBM));
  GemmArgs g{x, weight, m, k, n, k * n, scale, n, n, per_token_scale, bias, bias_dtype, n, out_dtype, out,
             map, slots, cdiv(n, 128)};
  const bool fast = fast_path_ok(g, w_layout);
  group_tiles_kernel<<<1, 1024, sizeof(int64_t) * (3 * num_groups + 1), st>>>(group_list, num_groups, group_list_type, m,
                                                                              bm, map, slots,
                                                                              fast ? nullptr : row_group);
  if (!fast) {
    gemm_i8_generic_kernel<<<dim3(static_cast<unsigned>(cdiv(m * n, 256))), 256, 0, st>>>(g, w_layout, row_group);
    return launch_status("tai_grouped_matmul");
  }
  launch_tile<128, 128>(g, w_layout, st);
  return launch_status("tai_grouped_matmul");
}
