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
#include <mutex>
#include <type_traits>

#include "common.h"

namespace tai {
namespace {
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

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
  // grouped: per row-tile slot (group, group_row_begin, group_row_end, index of the slot within its
  // group); group -1 marks an unused slot and -2 a zero-fill slot (then y, z are the slot's rows)
  const int4* tile_map;
  int64_t m_slots;
  int64_t n_tiles;
  const int64_t* live_slots;  // grouped: slots in use (real + zero-fill tiles), written by the prologue
  float* h;          // SwiGLU epilogue: silu(gate) * up, fp32 [m, n / 2]
  float* amax_part;  // SwiGLU epilogue: per-row max |h| of each 64-output-column part, [m, n / 128]
  // split-K (dense, int32 partials): k_split slices of k_per K stages each; slice s writes its raw
  // accumulators to out + s * m * n
  int64_t k_split;
  int64_t k_per;
  // SwiGLU epilogue: the weight is stored with gate and up interleaved in 64-column blocks (block 2t
  // holds gate columns 64t .. 64t + 63, block 2t + 1 the matching up columns), so a tile's columns
  // are contiguous in the weight rows
  int swi_packed;
  // grouped gather: row r of the product reads row a_rows[r] of a (clamped to [0, a_src_rows)); NULL
  // reads row r
  const int32_t* a_rows;
  int64_t a_src_rows;
};

// Row of a that product row r reads.
__device__ __forceinline__ int64_t a_row(const GemmArgs& g, int64_t r) {
  if (g.a_rows == nullptr) return r;
  const int64_t s = g.a_rows[r];
  return s < 0 ? 0 : (s < g.a_src_rows ? s : g.a_src_rows - 1);
}

// Output code of the fused SwiGLU epilogue (npu_grouped_matmul_swiglu_quant_v2).
constexpr int kOutSwiglu = 100;

// Weight column of tile column tc in a tile starting at n0. With the SwiGLU epilogue each
// 128-column slab of the tile holds 64 gate columns and the 64 up columns (+ n / 2) that pair
// with them, so every lane holds gate and up of the same output element in registers; the
// tile's n0 / 2 is its first output column.
template <bool SWI>
__device__ __forceinline__ int64_t weight_col(const GemmArgs& g, int64_t n0, int tc) {
  if constexpr (!SWI) {
    return n0 + tc;
  } else {
    if (g.swi_packed) return n0 + tc;
    const int w = tc & 127;
    return (w < 64 ? 0 : g.n / 2) + n0 / 2 + 64 * (tc >> 7) + (w & 63);
  }
}

__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nb) {
  const int64_t xcd = b % kXcds, idx = b / kXcds;
  const int64_t per = nb / kXcds, rem = nb % kXcds;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Linear tile id of workgroup b, or -1 when it has nothing to do. Grouped launches size the grid
// for the worst case of the device-resident group list; only the first `live` tile ids carry work,
// and each XCD takes an equal contiguous share of them (a plain remap of the whole grid would give
// the XCDs holding the upper ids nothing but empty slots).
__device__ __forceinline__ int64_t tile_id(const GemmArgs& g, int64_t b) {
  const int64_t nb = g.m_slots * g.n_tiles * (g.k_split > 1 ? g.k_split : 1);  // the launch's grid
  if (!g.live_slots) return b < nb ? xcd_remap(b, nb) : -1;
  const int64_t live = *g.live_slots * g.n_tiles;
  const int64_t xcd = b % kXcds, idx = b / kXcds;
  const int64_t per = live / kXcds, rem = live % kXcds;
  if (idx >= per + (xcd < rem ? 1 : 0)) return -1;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Grouped launches: linear tile id L -> (group, rows, column tile). The row tiles of one group that
// share a column tile are consecutive in L, so within an XCD they run together and read each weight
// slice from HBM once (the slice is then served from that XCD's L2 to the group's other row tiles).
// Returns the group, -1 (nothing to do) or -2 (zero-fill rows past the grouped total).
__device__ __forceinline__ int grouped_tile(const GemmArgs& g, int64_t L, int bm, int& row0, int& row1, int64_t& nt,
                                            int64_t& rt_out) {
  const int64_t s0 = L / g.n_tiles;
  const int4 t = g.tile_map[s0];
  rt_out = 1;
  if (t.x < 0) {
    row0 = t.y;
    row1 = t.z;
    nt = L % g.n_tiles;
    return t.x;
  }
  const int64_t first = s0 - t.w;
  const int64_t rt = (static_cast<int64_t>(t.z) - t.y + bm - 1) / bm;
  rt_out = rt;
  const int64_t off = L - first * g.n_tiles;
  nt = off / rt;
  row0 = t.y + static_cast<int>(off % rt) * bm;
  row1 = row0 + bm < t.z ? row0 + bm : t.z;
  return t.x;
}

// Mixed tiles (grouped [K, N] weights, n % 512 == 0). The slot table is built for 128-row tiles and
// each slot stands for n_tiles units of 128 x 512 outputs. A group with rt >= 2 row slots runs its
// first 2 * (rt / 2) slots as 256-row tiles of 256 columns (the same number of units), so each of its
// weight slices is read by half as many row tiles; an odd last slot stays a 128 x 512 tile. Tall
// tiles that share a 256-column slice are consecutive in L, as in grouped_tile.
__device__ __forceinline__ int grouped_tile_mixed(const GemmArgs& g, int64_t L, int& row0, int& row1, int64_t& nt,
                                                  int64_t& rt_out, bool& tall) {
  const int64_t s0 = L / g.n_tiles;
  const int4 t = g.tile_map[s0];
  tall = false;
  rt_out = 1;
  if (t.x < 0) {
    row0 = t.y;
    row1 = t.z;
    nt = L % g.n_tiles;
    return t.x;
  }
  const int64_t first = s0 - t.w;
  const int64_t rt = (static_cast<int64_t>(t.z) - t.y + 127) / 128;
  const int64_t pairs = rt / 2;
  const int64_t off = L - first * g.n_tiles;
  if (off < pairs * 2 * g.n_tiles) {
    tall = true;
    nt = off / pairs;
    row0 = t.y + static_cast<int>(off % pairs) * 256;
    row1 = row0 + 256 < t.z ? row0 + 256 : t.z;
  } else {
    nt = off - pairs * 2 * g.n_tiles;
    row0 = t.y + static_cast<int>(pairs) * 256;
    row1 = t.z;
  }
  rt_out = pairs + (rt & 1);  // row tiles that read this tile's weight columns
  return t.x;
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
      ra[i] = (r < rows && kk < g.k) ? *reinterpret_cast<const uint4*>(g.a + a_row(g, row0 + r) * g.k + kk)
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

  const int64_t L = tile_id(g, blockIdx.x);
  if (L < 0) return;
  int64_t nt = L % g.n_tiles;
  int e = 0, row0, row1;
  if (g.tile_map) {
    int64_t rt;
    e = grouped_tile(g, L, BM, row0, row1, nt, rt);
  }
  const int64_t n0 = nt * BN;
  if (g.tile_map) {
    if (e == -1) return;
    if (e == -2) {  // rows past the grouped total
      for (int idx = threadIdx.x; idx < (row1 - row0) * BN; idx += 256) {
        const int64_t r = row0 + idx / BN, c = n0 + idx % BN;
        if (c < g.n) {
          if (g.out_dt == TAI_DT_INT32) static_cast<int32_t*>(g.out)[r * g.n + c] = 0;
          else store_from_f32(g.out, g.out_dt, r * g.n + c, 0.0f);
        }
      }
      return;
    }
  } else {
    const int64_t slot = L / g.n_tiles;
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
  const int8_t* arow = g.a + a_row(g, row) * g.k;
  int32_t acc = 0;
  for (int64_t kk = 0; kk < g.k; ++kk) {
    const int32_t bv = layout == TAI_LAYOUT_NK ? bgrp[col * g.k + kk] : bgrp[kk * g.n + col];
    acc += static_cast<int32_t>(arow[kk]) * bv;
  }
  if (g.bias && g.bias_dt == TAI_DT_INT32) acc += static_cast<const int32_t*>(g.bias)[e * g.bias_group_stride + col];
  const float* bias_f = (g.bias && g.bias_dt == TAI_DT_FP32)
                            ? static_cast<const float*>(g.bias) + e * g.bias_group_stride : nullptr;
  if (g.out_dt == TAI_DT_INT32) static_cast<int32_t*>(g.out)[idx] = acc;
  else store_from_f32(g.out, g.out_dt, idx, epilogue_value(g, e, row, col, acc, bias_f));
}

// ----------------------------------------------------------------------------- grouped prologue
// Builds the tile table for row tiles of height bm, plus a row->group map for the generic path.
// One workgroup of 1024 threads, groups 2t and 2t + 1 per thread (ng <= 2048): group ends are a
// prefix sum of the counts (list type 1) or a running max of the cumulative ends (type 0), both
// clamped to m; tile offsets are a prefix sum of the per-group tile counts.
__global__ __launch_bounds__(1024) void group_tiles_kernel(const int64_t* __restrict__ gl, int64_t ng, int list_type,
                                                          int64_t m, int bm, int4* __restrict__ map, int64_t slots,
                                                          int64_t* __restrict__ live, int32_t* __restrict__ row_group) {
  extern __shared__ int64_t sh[];  // begin[ng], end[ng], tile_prefix[ng + 1]
  __shared__ int64_t red[16];
  int64_t* beg = sh;
  int64_t* end = sh + ng;
  int64_t* tp = sh + 2 * ng;
  const int64_t e0 = 2 * static_cast<int64_t>(threadIdx.x), e1 = e0 + 1;
  const int64_t g0 = e0 < ng ? gl[e0] : 0, g1 = e1 < ng ? gl[e1] : 0;
  int64_t end0, end1, beg0;
  if (list_type == 1) {
    const int64_t c0 = imax64(g0, 0), c1 = imax64(g1, 0);
    const int64_t incl = block_incl_scan<false>(c0 + c1, red);
    beg0 = incl - c0 - c1;
    end0 = beg0 + c0;
    end1 = incl;
  } else {
    __shared__ int64_t incl_sh[1024];
    const int64_t incl = block_incl_scan<true>(imax64(imax64(g0, g1), 0), red);
    incl_sh[threadIdx.x] = incl;
    __syncthreads();
    beg0 = threadIdx.x ? incl_sh[threadIdx.x - 1] : 0;  // running max before this thread's pair
    end0 = max<int64_t>(beg0, g0);
    end1 = max<int64_t>(end0, g1);
  }
  beg0 = min<int64_t>(beg0, m);
  end0 = min<int64_t>(end0, m);
  end1 = min<int64_t>(end1, m);
  const int64_t t0 = e0 < ng ? (end0 - beg0 + bm - 1) / bm : 0;
  const int64_t t1 = e1 < ng ? (end1 - end0 + bm - 1) / bm : 0;
  const int64_t tincl = block_incl_scan<false>(t0 + t1, red);
  if (e0 < ng) { beg[e0] = beg0; end[e0] = end0; tp[e0] = tincl - t0 - t1; }
  if (e1 < ng) { beg[e1] = end0; end[e1] = end1; tp[e1] = tincl - t1; }
  if (threadIdx.x == blockDim.x - 1) tp[ng] = tincl;
  __syncthreads();
  const int64_t real = tp[ng];
  const int64_t covered = ng > 0 ? end[ng - 1] : 0;
  const int64_t zero_tiles = (m - covered + bm - 1) / bm;
  if (threadIdx.x == 0) *live = real + zero_tiles;
  // each group writes its own slots (a thread per group, one store per row tile), then the zero-fill
  // and unused slots follow
  for (int64_t e = threadIdx.x; e < ng; e += blockDim.x) {
    const int64_t nt = (end[e] - beg[e] + bm - 1) / bm;
    for (int64_t j = 0; j < nt; ++j)
      map[tp[e] + j] = make_int4(static_cast<int>(e), static_cast<int>(beg[e]), static_cast<int>(end[e]),
                                 static_cast<int>(j));
  }
  for (int64_t s = real + threadIdx.x; s < slots; s += blockDim.x) {
    int4 t = make_int4(-1, 0, 0, 0);
    if (s < real + zero_tiles) {
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


// ----------------------------------------------------------------------------- big-tile kernel
// Workgroup = WM x WN waves of 64x128 (2x4 MFMA tiles, 128 int32 accumulators per lane), tile
// BM = 64*WM rows by BN = 128*WN columns. K advances 64 bytes per stage through a ring of S LDS
// stages filled by global_load_lds_dwordx4 (global -> LDS without registers); S-1 stages are in
// flight while one is multiplied. The 2x2 configuration (128x256, 72 KB of LDS) runs two
// workgroups per CU, so one workgroup's barrier wait overlaps the other's MFMAs.
// LDS layouts (each 16-byte chunk placed by the lane that loads it, so swizzles cost nothing):
//   A and an [N,K] weight: [rows][64 B]; chunk c of row r stored at chunk c ^ ((r >> 2) & 3)
//     -> 16-byte fragment reads of 16 consecutive rows cover the 64 banks once.
//   a [K,N] weight: [64 k rows][BN B]; chunk c of row r stored at chunk c ^ 2(r & 7); fragments
//     are read with ds_read_b64_tr_b8 (in each 16-lane group source lane L addresses
//     B[k0 + L/2][n0 + 8*(L&1)] and output lane j receives B[k0..k0+7][n0 + j]). The two 16-lane
//     groups of a 32-lane LDS pass read chunks c and c + 1 of the same 8 rows; the even XOR keeps
//     them on disjoint banks (an XOR by r & 7 maps both onto the same 32 banks).
// Requires K % 64 == 0 (stage loads cannot zero-fill a K tail). Rows and columns past the end of
// the tile are loaded from clamped addresses and never stored.
template <int WM, int WN, int BK, int STAGES>
struct BigCfg {
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kBM = 64 * WM, kBN = 128 * WN, kBK = BK;
  static constexpr int kStage = (kBM + kBN) * BK;
  static constexpr int kStages = STAGES;
  static constexpr int kLds = kStage * kStages;
  static constexpr int kCpr = BK / 16;                    // 16-byte chunks per A / NK-B row
  static constexpr int kRowShift = BK == 128 ? 1 : 2;      // rows per 256-byte bank cycle = 1 << shift
  static constexpr int kALoads = kBM * BK / 1024 / (WM * WN);  // 1 KB load instructions per wave per stage
  static constexpr int kBLoads = kBN * BK / 1024 / (WM * WN);
  static constexpr int kLoads = kALoads + kBLoads;
  static_assert(kALoads * WM * WN * 1024 == kBM * BK && kBLoads * WM * WN * 1024 == kBN * BK, "load split");
  static_assert(kBN >= 256, "the [K,N] swizzle spans 16 chunks of a weight row");
};

#ifndef TAI_GEMM_B_NT
#define TAI_GEMM_B_NT 1
#endif
#ifndef TAI_SPLIT_ISSUE
#define TAI_SPLIT_ISSUE 1
#endif
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;

// s_waitcnt with only vmcnt limited (expcnt / lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Two ds_read_b64_tr_b8 into one 16-byte fragment (bytes 0-7 from `lo`, 8-15 from `hi`),
// issued as inline asm: the builtin makes the compiler drain the in-flight global->LDS ring
// before the read. The caller waits with lgkm_wait before using the result.
__device__ __forceinline__ v4i ds_read_tr8_pair(const int8_t* lo, const int8_t* hi) {
  v2i a, b;
  const uint32_t alo = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const int8_t*)lo));
  const uint32_t ahi = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const int8_t*)hi));
  asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(a) : "v"(alo));
  asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(b) : "v"(ahi));
  return v4i{a[0], a[1], b[0], b[1]};
}

// 16-byte LDS read as inline asm (counted by lgkm_wait like the transposing reads).
__device__ __forceinline__ v4i ds_read_b128(const int8_t* p) {
  v4i r;
  const uint32_t a = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const int8_t*)p));
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
  return r;
}

// Waits until at most N LDS operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt is four bits");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}

// The loads of one stage: PART 0 issues all of them, PART 1 the first half and PART 2 the rest (a
// stage's loads are split so that the workgroup's waves do not all queue in the address unit at
// the same moment after a barrier).
template <int LAYOUT, class C, bool SWI = false, int PART = 0, int BPOL = 0>
__device__ __forceinline__ void big_issue_stage(const GemmArgs& g, const int8_t* bgrp, const int64_t* aoff,
                                                int64_t n0, int64_t k0, int8_t* stage, int w, int lane) {
  constexpr int BK = C::kBK, CPR = C::kCpr, RPI = 1024 / BK;  // rows per 1 KB instruction
  constexpr int kFirst = (C::kLoads + 1) / 2;
  constexpr int j0 = PART == 2 ? kFirst : 0, j1 = PART == 1 ? kFirst : C::kLoads;
#pragma unroll
  for (int i = 0; i < C::kALoads; ++i) {
    if (i < j0 || i >= j1) continue;
    const int q = C::kALoads * w + i;
    const int row = RPI * q + lane / CPR;
    const int c = (lane % CPR) ^ ((row >> C::kRowShift) & (CPR - 1));
    const int8_t* src = g.a + aoff[i] + k0 + 16 * c;
    __builtin_amdgcn_global_load_lds((gbl_void*)src, (lds_void*)(stage + q * 1024), 16, 0, 0);
  }
  int8_t* bst = stage + C::kBM * BK;
#pragma unroll
  for (int i = 0; i < C::kBLoads; ++i) {
    if (C::kALoads + i < j0 || C::kALoads + i >= j1) continue;
    const int q = C::kBLoads * w + i;
    const int8_t* src;
    if constexpr (LAYOUT == TAI_LAYOUT_NK) {
      const int row = RPI * q + lane / CPR;
      const int c = (lane % CPR) ^ ((row >> C::kRowShift) & (CPR - 1));
      const int64_t wc = weight_col<SWI>(g, n0, row);
      const int64_t nn = wc < g.n ? wc : g.n - 1;
      src = bgrp + nn * g.k + k0 + 16 * c;
    } else {
      constexpr int CPN = C::kBN / 16;  // chunks per k row
      const int kr = (1024 / C::kBN) * q + lane / CPN;
      const int c = (lane % CPN) ^ ((kr & 7) << 1);
      const int64_t wc = weight_col<SWI>(g, n0, 16 * c);
      const int64_t nn = wc < g.n ? wc : g.n - 16;
      src = bgrp + (k0 + kr) * g.n + nn;
    }
    __builtin_amdgcn_global_load_lds((gbl_void*)src, (lds_void*)(bst + q * 1024), 16, 0, BPOL);
  }
}

// SwiGLU epilogue of npu_grouped_matmul_swiglu_quant_v2 (the arithmetic of npu_dequant_swiglu_quant
// with activate_left): d = (float(acc) * weight_scale[col]) * x_scale[row]; h = silu(d_gate) * d_up.
// Writes h (fp32) and, per row, the max |h| over each wave's 64 output columns (part index
// (first output column) / 64); a second kernel turns them into the per-row int8 quantisation.
// Accumulator blocks j = 0, 1 hold gate columns and j = 2, 3 the matching up columns (weight_col).
// h leaves through a wave-private LDS region as 16-byte non-temporal stores along the rows.
template <class C>
__device__ __forceinline__ void swiglu_epilogue(const GemmArgs& g, const v16i (&acc)[2][4], int e, int row0, int rows,
                                                int64_t n0, int w, int lane, int8_t* smem) {
#pragma clang fp contract(off)
  constexpr int WN = C::kBN / 128;
  const int wm = w / WN, wn = w % WN;
  const int64_t n2 = g.n / 2;
  const int64_t oc0 = n0 / 2 + 64 * wn;  // this wave's first output column
  const float* ws = g.scale + e * g.scale_group_stride;
  float wg[2], wu[2];  // weight scales of this lane's gate / up columns
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t oc = oc0 + 32 * j + (lane & 31);
    wg[j] = ws[oc];
    wu[j] = ws[oc + n2];
  }
  // one x_scale per lane (row wm * 64 + lane), handed to the lanes that need it by a cross-lane read
  const float my_xs = g.pts[row0 + min(wm * 64 + lane, rows - 1)];
  constexpr int RB = 64 * 4 + 16;  // LDS row bytes of a 16-row slice (64 fp32 + pad)
  static_assert(8 * 16 * RB <= C::kLds, "epilogue staging must fit in the ring");
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave is past the ring
  char* wreg = reinterpret_cast<char*>(smem) + w * (16 * RB);
  float rmax[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const int r = 8 * hh + rr;
        const int sl = 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);  // row within the 16-row slice
        const float xs = __shfl(my_xs, i * 32 + 16 * hh + sl, 64);
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float dg = (static_cast<float>(acc[i][j][r]) * wg[j]) * xs;
          const float du = (static_cast<float>(acc[i][j + 2][r]) * wu[j]) * xs;
          const float hv = silu_f32(dg) * du;
          *reinterpret_cast<float*>(wreg + sl * RB + (32 * j + (lane & 31)) * 4) = hv;
          m = fmaxf(m, fabsf(hv));
        }
        rmax[i][r] = m;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int sl = 4 * q + (lane >> 4);
        const int lr = wm * 64 + i * 32 + 16 * hh + sl;
        const v4i v = *reinterpret_cast<const v4i*>(wreg + sl * RB + 16 * (lane & 15));
        if (lr < rows) {
          typedef __attribute__((address_space(1))) v4i gv4i;
          float* dst = g.h + static_cast<int64_t>(row0 + lr) * n2 + oc0 + 4 * (lane & 15);
          __builtin_nontemporal_store(v, (gv4i*)(reinterpret_cast<uintptr_t>(dst)));
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // region reused by the next slice
    }
  // Max over the 32 lanes that share a row (lanes of one half-wave hold one row's columns), as a
  // reduce-scatter: at the step with lane offset o each lane keeps half of its live row values and
  // sends the partner the other half, so 16 + 8 + 4 + 2 + 1 shuffles leave lane l (of its half)
  // with the max of row value l (i = l / 16, r = l % 16).
  float v[32];
#pragma unroll
  for (int t = 0; t < 32; ++t) v[t] = rmax[t >> 4][t & 15];
  const int l32 = lane & 31;
  auto halve = [&](auto half) {  // one step: 2 * H live values -> H, lane offset H
    constexpr int H = decltype(half)::value;
    const bool up = (l32 & H) != 0;
#pragma unroll
    for (int t = 0; t < H; ++t) {
      const float keep = up ? v[t + H] : v[t];
      const float send = up ? v[t] : v[t + H];
      v[t] = fmaxf(keep, __shfl_xor(send, H, 64));
    }
  };
  halve(std::integral_constant<int, 16>());
  halve(std::integral_constant<int, 8>());
  halve(std::integral_constant<int, 4>());
  halve(std::integral_constant<int, 2>());
  halve(std::integral_constant<int, 1>());
  const int i = l32 >> 4, r = l32 & 15;
  const int lr = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  if (lr < rows) g.amax_part[static_cast<int64_t>(row0 + lr) * (g.n / 128) + oc0 / 64] = v[0];
}

// One tile of the big-tile kernel: rows [row0, row1) of group e (dense: e = 0), column tile nt,
// linear tile id L (split-K slice); row_tiles = row tiles of the group that share this tile's
// weight slice. e = -1: nothing to do, e = -2: zero-fill rows past the grouped total.
template <int LAYOUT, int OUT, class C>
__device__ __forceinline__ void big_tile(const GemmArgs& g, int8_t* smem, int64_t L, int e, int row0, int row1,
                                         int64_t nt, int64_t row_tiles) {
  constexpr int WN = C::kBN / 128;
  constexpr int kBigBK = C::kBK;
  const int64_t n0 = nt * C::kBN;
  if (g.tile_map) {
    if (e == -1) return;
    if (e == -2) {
      if constexpr (OUT == kOutSwiglu) {  // rows past the grouped total: h = 0, partial max 0
        const int64_t n2 = g.n / 2, o0 = n0 / 2;
        for (int idx = threadIdx.x; idx < (row1 - row0) * (C::kBN / 2); idx += C::kThreads) {
          const int64_t r = row0 + idx / (C::kBN / 2), c = o0 + idx % (C::kBN / 2);
          if (c < n2) g.h[r * n2 + c] = 0.0f;
        }
        for (int idx = threadIdx.x; idx < (row1 - row0) * WN; idx += C::kThreads)  // the tile's 64-column parts
          g.amax_part[(row0 + idx / WN) * (g.n / 128) + o0 / 64 + idx % WN] = 0.0f;
      } else {
        for (int idx = threadIdx.x; idx < (row1 - row0) * C::kBN; idx += C::kThreads) {
          const int64_t r = row0 + idx / C::kBN, c = n0 + idx % C::kBN;
          if (c < g.n) {
            if constexpr (OUT == TAI_DT_INT32) static_cast<int32_t*>(g.out)[r * g.n + c] = 0;
            else store_from_f32(g.out, OUT, r * g.n + c, 0.0f);
          }
        }
      }
      return;
    }
  }
  const int rows = row1 - row0;
  const int8_t* bgrp = g.b + static_cast<int64_t>(e) * g.b_group_stride;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = w / WN, wn = w % WN;
  // source row offsets of this lane's A loads (rows past the tile re-read its last row; their sums
  // are never stored), fixed for the whole tile; a gathered product reads them first, ahead of the
  // epilogue operands, so no wait for them drains anything issued later
  int64_t aoff[C::kALoads];
#pragma unroll
  for (int i = 0; i < C::kALoads; ++i) {
    const int row = (1024 / C::kBK) * (C::kALoads * w + i) + lane / C::kCpr;
    const int rr = row < rows ? row : (rows > 0 ? rows - 1 : 0);
    aoff[i] = a_row(g, row0 + rr) * g.k;
  }
  const int act_m = max(0, min(2, (rows - wm * 64 + 31) / 32));
  const int64_t ncols = g.n - n0 - wn * 128;
  const int act_n = ncols <= 0 ? 0 : (ncols >= 128 ? 4 : static_cast<int>((ncols + 31) / 32));

  v16i acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // K range of this workgroup (split-K slices a dense launch; otherwise the whole of K)
  int64_t kbeg = 0, nk = g.k / kBigBK;
  void* gout = g.out;
  if (g.k_split > 1) {
    const int64_t ks = L / (g.m_slots * g.n_tiles);
    if (ks >= g.k_split) return;
    kbeg = ks * g.k_per;
    nk = nk - kbeg < g.k_per ? nk - kbeg : g.k_per;
    gout = static_cast<int32_t*>(g.out) + ks * g.m * g.n;
  }
  // Epilogue operands of a full-width wave tile are loaded before the main loop, and ahead of the
  // ring's first stages (whose waits count loads in issue order), so their latency is hidden: the
  // per-column scales and biases, and one per-token scale per lane (the wave's row wm * 64 + lane),
  // handed to the lanes that need it by a cross-lane read.
  const int32_t* bias_i = (g.bias && g.bias_dt == TAI_DT_INT32)
                              ? static_cast<const int32_t*>(g.bias) + e * g.bias_group_stride : nullptr;
  const float* bias_f = (g.bias && g.bias_dt == TAI_DT_FP32)
                            ? static_cast<const float*>(g.bias) + e * g.bias_group_stride : nullptr;
  const float* scl = g.scale ? g.scale + e * g.scale_group_stride : nullptr;
  const int64_t wcol0 = n0 + wn * 128;
  const bool full_width = wcol0 + 128 <= g.n;
  float my_pt = 1.0f;
  int32_t bcol[4];
  float sc[4], bf[4];
  if constexpr (OUT != kOutSwiglu) {
    if (OUT != TAI_DT_INT32 && g.pts && full_width) my_pt = g.pts[row0 + min(wm * 64 + lane, rows - 1)];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = wcol0 + j * 32 + (lane & 31);
      bcol[j] = (bias_i && full_width) ? bias_i[col] : 0;
      sc[j] = (scl && full_width) ? scl[g.scale_len == 1 ? 0 : col] : 1.0f;
      bf[j] = (bias_f && full_width) ? bias_f[col] : -0.0f;
    }
  }
  const int64_t kb0 = kbeg * kBigBK;

  const int arow = wm * 64 + (lane & 31);            // + 32 i
  const int brow = wn * 128 + (lane & 31);           // + 32 j (NK)
  const int l16 = lane & 15;
  const int bk_lane = (lane >> 5) * 16 + (l16 >> 1);  // KN: k row within the 32-row kk block (+ 8)
  const int bc_lane = wn * 128 + ((lane >> 4) & 1) * 16 + (l16 & 1) * 8;  // KN: byte column (+ 32 j)

  // Fragment reads are inline asm so that the waits below count them exactly (LDS reads complete in
  // issue order): the reads for step kk + 1 are issued before the MFMAs of step kk.
  auto load_a = [&](const int8_t* st, int kk, int i) {
    const int r = arow + 32 * i;
    const int c = (2 * kk + (lane >> 5)) ^ ((r >> C::kRowShift) & (C::kCpr - 1));
    return ds_read_b128(st + r * kBigBK + 16 * c);
  };
  auto load_b = [&](const int8_t* bs, int kk, int j) -> v4i {
    if constexpr (LAYOUT == TAI_LAYOUT_NK) {
      const int r = brow + 32 * j;
      const int c = (2 * kk + (lane >> 5)) ^ ((r >> C::kRowShift) & (C::kCpr - 1));
      return ds_read_b128(bs + r * kBigBK + 16 * c);
    } else {
      const int col = bc_lane + 32 * j;
      const int k_lo = kk * 32 + bk_lane, k_hi = k_lo + 8;
      const int8_t* plo = bs + k_lo * C::kBN + 16 * ((col >> 4) ^ ((k_lo & 7) << 1)) + (col & 15);
      const int8_t* phi = bs + k_hi * C::kBN + 16 * ((col >> 4) ^ ((k_hi & 7) << 1)) + (col & 15);
      return ds_read_tr8_pair(plo, phi);
    }
  };
  constexpr int KK = kBigBK / 32;  // MFMA steps per stage
  static_assert(KK % 2 == 0, "fragment double buffer alternates within a stage");
  // Stage kt has landed in this wave's view once only the stages issued after it remain in flight.
  auto wait_stage = [&](int64_t kt) {
    const int64_t after = nk - 1 - kt < C::kStages - 2 ? nk - 1 - kt : C::kStages - 2;
    if constexpr (C::kStages == 2) {
      wait_vmcnt<0>();
    } else {
      if (after >= C::kStages - 2) wait_vmcnt<C::kLoads * (C::kStages - 2)>();
      else if (after == 2) wait_vmcnt<C::kLoads * 2>();
      else if (after == 1) wait_vmcnt<C::kLoads>();
      else wait_vmcnt<0>();
    }
  };
  // Main loop for waves with NI live 32-row halves (NI = 0: the wave only takes part in the ring).
  // Per stage kt: steps 0 .. KK-2 prefetch the next step's fragments and multiply the current ones;
  // the last step waits for stage kt + 1, passes the workgroup barrier (after it no wave reads slot
  // kt, whose fragments are in registers), refills slot kt with stage kt + S, prefetches the first
  // fragments of stage kt + 1, then multiplies.
  constexpr bool kSplit = TAI_SPLIT_ISSUE != 0 && C::kStages > 2;  // needs two stages in flight
  auto main_loop = [&](auto ni, auto bpol) {
    constexpr int NI = decltype(ni)::value;
    constexpr int BP = decltype(bpol)::value;
#pragma unroll
    for (int s = 0; s < C::kStages - 1; ++s)
      if (s < nk)
        big_issue_stage<LAYOUT, C, OUT == kOutSwiglu, 0, BP>(g, bgrp, aoff, n0, kb0 + s * kBigBK, smem + s * C::kStage,
                                                             w, lane);
    constexpr int NF = NI == 0 ? 0 : NI + (LAYOUT == TAI_LAYOUT_KN ? 8 : 4);  // LDS reads per step
    v4i fa[2][NI > 0 ? NI : 1], fb[2][4];
    auto fetch = [&](int buf, const int8_t* st, int kk) {
      if constexpr (NI > 0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) fa[buf][i] = load_a(st, kk, i);
#pragma unroll
        for (int j = 0; j < 4; ++j) fb[buf][j] = load_b(st + C::kBM * kBigBK, kk, j);
      }
    };
    auto ready = [&](int buf) {  // orders the uses of buffer buf after the preceding wait
      if constexpr (NI > 0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) asm volatile("" : "+v"(fa[buf][i]));
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(fb[buf][j]));
      }
    };
    auto mfma = [&](int buf) {
      if constexpr (NI > 0) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[buf][i], fb[buf][j], acc[i][j], 0, 0, 0);
      }
    };
    wait_stage(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (C::kStages - 1 < nk)
      big_issue_stage<LAYOUT, C, OUT == kOutSwiglu, 0, BP>(g, bgrp, aoff, n0, kb0 + (C::kStages - 1) * kBigBK,
                                 smem + (C::kStages - 1) * C::kStage, w, lane);
    fetch(0, smem, 0);
    for (int64_t kt = 0; kt < nk; ++kt) {
      const int8_t* st = smem + (static_cast<int>(kt) % C::kStages) * C::kStage;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int cur = kk & 1;
        if (kk + 1 < KK) {
          fetch(cur ^ 1, st, kk + 1);
          lgkm_wait<NF>();
        } else {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (kt + 1 < nk) {
            wait_stage(kt + 1);
            asm volatile("s_barrier" ::: "memory");
            // stage kt + S into the slot just freed: its first half now, the rest after the next
            // stage's first MFMA step (every load is still issued before the next stage wait)
            if (kt + C::kStages < nk)
              big_issue_stage<LAYOUT, C, OUT == kOutSwiglu, kSplit ? 1 : 0, BP>(
                  g, bgrp, aoff, n0, kb0 + (kt + C::kStages) * kBigBK,
                  smem + (static_cast<int>(kt) % C::kStages) * C::kStage, w, lane);
            fetch(cur ^ 1, smem + ((static_cast<int>(kt) + 1) % C::kStages) * C::kStage, 0);
          }
        }
        ready(cur);
        mfma(cur);
        if constexpr (kSplit) {
          if (kk == 0 && kt >= 1 && kt - 1 + C::kStages < nk)
            big_issue_stage<LAYOUT, C, OUT == kOutSwiglu, 2, BP>(g, bgrp, aoff, n0, kb0 + (kt - 1 + C::kStages) * kBigBK,
                                                           smem + ((static_cast<int>(kt) - 1) % C::kStages) * C::kStage,
                                                           w, lane);
        }
        __builtin_amdgcn_sched_barrier(0);  // the next step's waits stay behind these MFMAs
      }
    }
  };
  // Waves whose 64 rows are all past the group end skip the MFMAs; waves with at most 32 live rows
  // skip those of the upper 32 (wave-uniform branches).
  // A group with a single row tile reads each weight byte once: its weight loads stream with the
  // non-temporal policy. Groups with several row tiles share their weight slices through L2.
  auto dispatch = [&](auto bpol) {
    if (act_m > 1) main_loop(std::integral_constant<int, 2>(), bpol);
    else if (act_m == 1) main_loop(std::integral_constant<int, 1>(), bpol);
    else main_loop(std::integral_constant<int, 0>(), bpol);
  };
  if (TAI_GEMM_B_NT && row_tiles == 1) dispatch(std::integral_constant<int, 2>());
  else dispatch(std::integral_constant<int, 0>());

  if constexpr (OUT == kOutSwiglu) {
    swiglu_epilogue<C>(g, acc, e, row0, rows, n0, w, lane, smem);
    return;
  }
  // Epilogue, specialised on the output dtype so the accumulators stay in registers.
  // value of accumulator (i, j, r) as fp32 after the scales and fp32 bias; absent operands hold
  // their neutral values (1.0, 1.0, -0.0: x * 1 and x + (-0) are x for every x, signed zeros
  // included), so no per-element selects are needed
  auto out_f32 = [&](int32_t v, float sc, float bf, float pt) -> float {
    return (static_cast<float>(v) * sc) * pt + bf;
  };
  // value of accumulator (i, j, r) in the output type, as raw bits (pt: the row's per-token scale)
  auto out_bits = [&](int32_t v, float sc, float bf, float pt) -> uint32_t {
    if constexpr (OUT == TAI_DT_INT32) {
      return static_cast<uint32_t>(v);
    } else {
      const float f = out_f32(v, sc, bf, pt);
      if constexpr (OUT == TAI_DT_BF16) return f32_to_bf16(f);
      else if constexpr (OUT == TAI_DT_FP16) return f32_to_f16(f);
      else return __float_as_uint(f);
    }
  };
  if (full_width) {
    // Full-width wave tile: 16-row slices go through a wave-private LDS region (the ring is free
    // once every wave is past its last stage) and leave as 16-byte stores along the rows, instead
    // of one 2- or 4-byte store per element.
    constexpr int ES = (OUT == TAI_DT_BF16 || OUT == TAI_DT_FP16) ? 2 : 4;
    constexpr int RB = 128 * ES + 16;  // LDS row bytes (padding moves the second lane half's row)
    static_assert(8 * 16 * RB <= C::kLds, "epilogue staging must fit in the ring");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    char* wreg = reinterpret_cast<char*>(smem) + w * (16 * RB);
    const bool nt_out = g.tile_map != nullptr;
    constexpr int LPR = 128 * ES / 16;  // lanes per row when reading 16 bytes each
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // accumulator rows of this slice: r = 8h .. 8h+7, local row 8((r&7)>>2) + 4(lane>>5) + (r&3)
        float pt[8];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
          pt[rr] = __shfl(my_pt, i * 32 + 16 * h + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3), 64);
        if constexpr (OUT == TAI_DT_BF16) {
          // Two rows of a lane pair (columns c, c + 1) become one bf16x2 word per lane: the even
          // lane takes row r's pair, the odd lane row r + 1's; one DPP swap, one
          // v_cvt_pk_bf16_f32 (round to nearest even) and one 4-byte LDS write per two outputs.
          const bool odd = lane & 1;
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rr = 0; rr < 8; rr += 2) {
              const int r = 8 * h + rr;
              const float f0 = out_f32(acc[i][j][r] + bcol[j], sc[j], bf[j], pt[rr]);
              const float f1 = out_f32(acc[i][j][r + 1] + bcol[j], sc[j], bf[j], pt[rr + 1]);
              const float send = odd ? f0 : f1;
              const float recv =
                  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0xB1, 0xF, 0xF, false));
              bf16x2_t pk = __builtin_convertvector((f32x2_t){odd ? recv : f0, odd ? f1 : recv}, bf16x2_t);
              const int sl = 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3) + (odd ? 1 : 0);
              char* dst = wreg + sl * RB + (j * 32 + (lane & 30)) * ES;
              *reinterpret_cast<uint32_t*>(dst) = __builtin_bit_cast(uint32_t, pk);
            }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
              const int r = 8 * h + rr;
              const int sl = 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
              const uint32_t bits = out_bits(acc[i][j][r] + bcol[j], sc[j], bf[j], pt[rr]);
              char* dst = wreg + sl * RB + (j * 32 + (lane & 31)) * ES;
              if constexpr (ES == 2) *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(bits);
              else *reinterpret_cast<uint32_t*>(dst) = bits;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int q = 0; q < 16 / (64 / LPR); ++q) {
          const int sl = q * (64 / LPR) + lane / LPR;
          const int lr = wm * 64 + i * 32 + 16 * h + sl;
          const uint4 v = *reinterpret_cast<const uint4*>(wreg + sl * RB + 16 * (lane % LPR));
          if (lr < rows) {
            tai_u32x4_t* dst = reinterpret_cast<tai_u32x4_t*>(static_cast<char*>(gout) +
                                                              (static_cast<int64_t>(row0 + lr) * g.n + wcol0) * ES +
                                                              16 * (lane % LPR));
            // grouped launches write rows that the next op streams once: non-temporal stores (down
            // projection -2%, the config-4 GEMM + quant + GEMM + finalize chain -0.7%); split-K
            // partials, re-read at once by the reduction, and dense outputs keep the default policy
            if (nt_out) {
              // a compiler-visible store (an inline-asm store hid its data registers from the
              // hazard recognizer, which then let the next VALU overwrite them too early)
              const v4i d{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
              typedef __attribute__((address_space(1))) v4i gv4i;
              __builtin_nontemporal_store(d, (gv4i*)(reinterpret_cast<uintptr_t>(dst)));
            } else {
              *dst = tai_u32x4_t{v.x, v.y, v.z, v.w};
            }
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // region reused by the next slice
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t col = n0 + wn * 128 + j * 32 + (lane & 31);
    const bool colok = j < act_n && col < g.n;
    const int64_t ccol = colok ? col : 0;
    const int32_t bcol = bias_i ? bias_i[ccol] : 0;
    const float sc = scl ? scl[g.scale_len == 1 ? 0 : ccol] : 1.0f;
    const float bf = bias_f ? bias_f[ccol] : -0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lr = wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (colok && lr < rows) {
          const int64_t idx = static_cast<int64_t>(row0 + lr) * g.n + col;
          const uint32_t bits = out_bits(acc[i][j][r] + bcol, sc, bf, g.pts ? g.pts[row0 + lr] : 1.0f);
          if constexpr (OUT == TAI_DT_BF16 || OUT == TAI_DT_FP16) static_cast<uint16_t*>(gout)[idx] = static_cast<uint16_t>(bits);
          else static_cast<uint32_t*>(gout)[idx] = bits;
        }
      }
    }
  }
}

template <int LAYOUT, int OUT, class C>
__global__ __launch_bounds__(C::kThreads, 2) void gemm_i8_big_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const int64_t L = tile_id(g, blockIdx.x);
  if (L < 0) return;
  int64_t nt, row_tiles = 0;
  int e = 0, row0, row1;
  if (g.tile_map) {
    e = grouped_tile(g, L, C::kBM, row0, row1, nt, row_tiles);
  } else {  // dense: groups of 8 row tiles walk the column tiles together (A and B reuse in L2)
    constexpr int64_t GM = 8;
    const int64_t per_group = GM * g.n_tiles;
    const int64_t Lt = g.k_split > 1 ? L % (g.m_slots * g.n_tiles) : L;  // split-K: slice = L / tiles
    const int64_t first = (Lt / per_group) * GM;
    const int64_t gsize = g.m_slots - first < GM ? g.m_slots - first : GM;
    const int64_t in = Lt % per_group;
    const int64_t slot = first + in % gsize;
    nt = in / gsize;
    row0 = static_cast<int>(slot * C::kBM);
    row1 = row0 + C::kBM < g.m ? row0 + C::kBM : static_cast<int>(g.m);
  }
  big_tile<LAYOUT, OUT, C>(g, smem, L, e, row0, row1, nt, row_tiles);
}

// Tile configurations used by the host (8 waves of 64 x 128, 256 x 256 tiles):
//   dense: 128-byte K stages, two stages (128 KB of LDS): the 8192^3 GEMM is MFMA/LDS bound and
//     fewer, larger stages halve the barriers;
//   grouped: 64-byte K stages, four stages: MoE expert GEMMs stream their weights from HBM, and
//     three stages in flight instead of one cut the gate_up time by ~6%. [K, N] weights use
//     128 x 512 tiles (2 x 4 waves, 160 KB): equal on gate_up, 9% faster on the down projection
//     (N = 7168); [N, K] weights keep 256 x 256.
// Measured and rejected on the MoE gate_up and 8192^3 shapes: 128 x 256 tiles (4 waves, 3-4
// stages), and a 4-wave kernel with 128 x 128 wave tiles and software-pipelined fragment reads;
// with one wave per SIMD the per-stage barrier and LDS reads cost more than the halved LDS
// traffic saves.
#ifndef TAI_BIG_SEL
#define TAI_BIG_SEL BigCfg<4, 2, 128, 2>
#endif
#ifndef TAI_GRP_SEL
#define TAI_GRP_SEL BigCfg<4, 2, 64, 4>
#endif
#ifndef TAI_GRP_KN_SEL
#define TAI_GRP_KN_SEL BigCfg<2, 4, 64, 4>
#endif
using BigSel = TAI_BIG_SEL;
using GrpSel = TAI_GRP_SEL;      // grouped, [N, K] weights
using GrpKnSel = TAI_GRP_KN_SEL;  // grouped, [K, N] weights
constexpr int kBigBK = BigSel::kBK;
constexpr int kBigBM = BigSel::kBM, kBigBN = BigSel::kBN;

template <class C, int LAYOUT, int OUT>
constexpr auto cfg_kernel() {
  return &gemm_i8_big_kernel<LAYOUT, OUT, C>;
}

template <class C, int LAYOUT, int OUT>
bool set_cfg_lds() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(cfg_kernel<C, LAYOUT, OUT>()),
                             hipFuncAttributeMaxDynamicSharedMemorySize, C::kLds) == hipSuccess;
}

// True when the device lets one workgroup hold configuration C's LDS (attributes set once).
template <class C>
bool cfg_available() {
  // evaluated once (a function-local static initialiser is thread-safe)
  static const bool cached = [] {
    int dev = 0, lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) {
      (void)hipGetLastError();
      lds = 0;
    }
    bool ok = lds >= C::kLds;
    if (ok) {
      ok = set_cfg_lds<C, TAI_LAYOUT_KN, TAI_DT_INT32>() && set_cfg_lds<C, TAI_LAYOUT_KN, TAI_DT_BF16>() &&
           set_cfg_lds<C, TAI_LAYOUT_KN, TAI_DT_FP16>() && set_cfg_lds<C, TAI_LAYOUT_KN, TAI_DT_FP32>() &&
           set_cfg_lds<C, TAI_LAYOUT_NK, TAI_DT_INT32>() && set_cfg_lds<C, TAI_LAYOUT_NK, TAI_DT_BF16>() &&
           set_cfg_lds<C, TAI_LAYOUT_NK, TAI_DT_FP16>() && set_cfg_lds<C, TAI_LAYOUT_NK, TAI_DT_FP32>() &&
           set_cfg_lds<C, TAI_LAYOUT_KN, kOutSwiglu>() && set_cfg_lds<C, TAI_LAYOUT_NK, kOutSwiglu>();
      (void)hipGetLastError();
    }
    return ok;
  }();
  return cached;
}

// Grouped [K, N] weights with mixed tiles (grouped_tile_mixed): 128 x 512 (GrpKnSel) or 256 x 256.
#ifndef TAI_MIX_TALL
#define TAI_MIX_TALL BigCfg<4, 2, 64, 4>
#endif
using MixTall = TAI_MIX_TALL;
#ifndef TAI_MIXED
#define TAI_MIXED 1
#endif
template <int OUT>
__global__ __launch_bounds__(GrpKnSel::kThreads, 2) void gemm_i8_mixed_kernel(GemmArgs g) {
  static_assert(GrpKnSel::kThreads == MixTall::kThreads && GrpKnSel::kBN == 512 && MixTall::kBM == 256,
                "mixed tiles: both shapes cover 128 x 512 outputs with one workgroup size");
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  const int64_t L = tile_id(g, blockIdx.x);
  if (L < 0) return;
  int64_t nt, row_tiles;
  int row0, row1;
  bool tall;
  const int e = grouped_tile_mixed(g, L, row0, row1, nt, row_tiles, tall);
  if (tall) big_tile<TAI_LAYOUT_KN, OUT, MixTall>(g, smem, L, e, row0, row1, nt, row_tiles);
  else big_tile<TAI_LAYOUT_KN, OUT, GrpKnSel>(g, smem, L, e, row0, row1, nt, row_tiles);
}

bool mixed_available() {
  static const bool ok = [] {
    if (!cfg_available<GrpKnSel>()) return false;
    constexpr int lds = GrpKnSel::kLds > MixTall::kLds ? GrpKnSel::kLds : MixTall::kLds;
    auto set = [](const void* f) {
      return hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess;
    };
    const bool r = set(reinterpret_cast<const void*>(&gemm_i8_mixed_kernel<TAI_DT_INT32>)) &&
                   set(reinterpret_cast<const void*>(&gemm_i8_mixed_kernel<TAI_DT_BF16>)) &&
                   set(reinterpret_cast<const void*>(&gemm_i8_mixed_kernel<TAI_DT_FP16>)) &&
                   set(reinterpret_cast<const void*>(&gemm_i8_mixed_kernel<TAI_DT_FP32>)) &&
                   set(reinterpret_cast<const void*>(&gemm_i8_mixed_kernel<kOutSwiglu>));
    (void)hipGetLastError();
    return r;
  }();
  return ok;
}

void launch_mixed(const GemmArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.m_slots * g.n_tiles));
  constexpr int T = GrpKnSel::kThreads;
  constexpr size_t L = GrpKnSel::kLds > MixTall::kLds ? GrpKnSel::kLds : MixTall::kLds;
  switch (g.out_dt) {
    case TAI_DT_INT32: gemm_i8_mixed_kernel<TAI_DT_INT32><<<grid, T, L, st>>>(g); break;
    case TAI_DT_BF16: gemm_i8_mixed_kernel<TAI_DT_BF16><<<grid, T, L, st>>>(g); break;
    case TAI_DT_FP16: gemm_i8_mixed_kernel<TAI_DT_FP16><<<grid, T, L, st>>>(g); break;
    case kOutSwiglu: gemm_i8_mixed_kernel<kOutSwiglu><<<grid, T, L, st>>>(g); break;
    default: gemm_i8_mixed_kernel<TAI_DT_FP32><<<grid, T, L, st>>>(g); break;
  }
}

template <class C, int LAYOUT>
void launch_cfg_layout(const GemmArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.m_slots * g.n_tiles));
  constexpr int T = C::kThreads;
  constexpr size_t L = C::kLds;
  switch (g.out_dt) {
    case TAI_DT_INT32: cfg_kernel<C, LAYOUT, TAI_DT_INT32>()<<<grid, T, L, st>>>(g); break;
    case TAI_DT_BF16: cfg_kernel<C, LAYOUT, TAI_DT_BF16>()<<<grid, T, L, st>>>(g); break;
    case TAI_DT_FP16: cfg_kernel<C, LAYOUT, TAI_DT_FP16>()<<<grid, T, L, st>>>(g); break;
    case kOutSwiglu: cfg_kernel<C, LAYOUT, kOutSwiglu>()<<<grid, T, L, st>>>(g); break;
    default: cfg_kernel<C, LAYOUT, TAI_DT_FP32>()<<<grid, T, L, st>>>(g); break;
  }
}

template <class C>
void launch_cfg(const GemmArgs& g, int layout, hipStream_t st) {
  if (layout == TAI_LAYOUT_NK) launch_cfg_layout<C, TAI_LAYOUT_NK>(g, st);
  else launch_cfg_layout<C, TAI_LAYOUT_KN>(g, st);
}

constexpr int kGroupedBM = 128;
constexpr int kMinBM = 32;  // workspace is sized for the smallest row tile any variant uses

size_t grouped_map_slots(int64_t m, int64_t ng, int bm) { return static_cast<size_t>(2 * cdiv(m, bm) + ng); }

// Skinny dense GEMMs (m < 256, e.g. a decode-sized MLP): 128 x 256 tiles leave most CUs idle, so K
// is split into slices whose int32 partials are summed (exactly) by splitk_reduce_kernel, which also
// applies the epilogue. The partials are small enough to stay in the last-level cache.
using SkinnyCfg = BigCfg<2, 2, 64, 4>;
constexpr int64_t kSkinnyTargetWgs = 512;

struct SplitPlan {
  int64_t m_slots, n_tiles, split, per;
};

SplitPlan skinny_plan(int64_t m, int64_t k, int64_t n) {
  SplitPlan p{cdiv(m, SkinnyCfg::kBM), cdiv(n, SkinnyCfg::kBN), 1, k / SkinnyCfg::kBK};
  const int64_t tiles = p.m_slots * p.n_tiles;
  const int64_t nk = k / SkinnyCfg::kBK;
  int64_t want = cdiv(kSkinnyTargetWgs, tiles);
  want = want < 1 ? 1 : (want > nk ? nk : want);
  p.per = cdiv(nk, want);
  p.split = cdiv(nk, p.per);
  return p;
}

bool skinny_ok(int64_t m, int64_t k, int64_t n, int layout) {
  return m < 256 && k % SkinnyCfg::kBK == 0 && k >= SkinnyCfg::kBK && (layout == TAI_LAYOUT_NK || n % 16 == 0) &&
         n % 4 == 0;
}

// out = epilogue(sum of the split partials); 4 consecutive elements per thread (n % 4 == 0).
template <int OUT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const int32_t* __restrict__ part, int64_t split, GemmArgs g) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  const int64_t mn = g.m * g.n;
  if (i4 >= mn) return;
  int4 acc = *reinterpret_cast<const int4*>(part + i4);
  for (int64_t sidx = 1; sidx < split; ++sidx) {
    const int4 v = *reinterpret_cast<const int4*>(part + sidx * mn + i4);
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const int64_t row = i4 / g.n, col = i4 % g.n;
  const int32_t a4[4] = {acc.x, acc.y, acc.z, acc.w};
  const int32_t* bias_i = (g.bias && g.bias_dt == TAI_DT_INT32) ? static_cast<const int32_t*>(g.bias) : nullptr;
  const float* bias_f = (g.bias && g.bias_dt == TAI_DT_FP32) ? static_cast<const float*>(g.bias) : nullptr;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int32_t v = a4[q] + (bias_i ? bias_i[col + q] : 0);
    if constexpr (OUT == TAI_DT_INT32) static_cast<int32_t*>(g.out)[i4 + q] = v;
    else store_from_f32(g.out, OUT, i4 + q, epilogue_value(g, 0, row, col + q, v, bias_f));
  }
}

// ----------------------------------------------------------------------------- skinny kernel
// Dense GEMMs with at most 128 rows (decode-sized MLPs) use each weight byte for at most 128 rows,
// so they are bound by the weight stream. One workgroup of 4 waves (one per SIMD) owns a BN-column
// slab of the output and a contiguous range of 64-byte K stages, which its waves take round-robin:
// every wave streams its own weight and activation stages through a private 2-slot LDS ring
// (global_load_lds, so no workgroup barrier in the loop; the activations are read by every slab and
// come from L2). After the loop the four partial tiles are summed through LDS. With k_split > 1 each slab's K is also split over workgroups, whose raw int32
// partials splitk_reduce_kernel sums (it also applies the epilogue).
template <int MI, int BN>
struct SkinnyShape {
  static constexpr int kD = 2;                    // ring slots per wave (3 and 4 measured slower)
  static constexpr int kSlotB = 64 * BN;          // bytes of one weight stage
  static constexpr int kSlotA = MI * 32 * 64;     // bytes of one activation stage
  static constexpr int kSlot = kSlotB + kSlotA;
  static constexpr int kNB = kSlotB / 1024;       // 1 KB weight loads per stage
  static constexpr int kNL = kNB + 2 * MI;        // vector memory instructions per stage (weights + activations)
  static constexpr int kRowWords = BN + 8;        // partial-sum row in LDS: rows r and r + 4 land 32 banks apart
  static constexpr int kRing = 4 * kD * kSlot;
  static constexpr int kRed = 4 * MI * 32 * kRowWords * 4;
  static constexpr int kLds = kRing > kRed ? kRing : kRed;
  static_assert(kNL * (kD - 1) < 64, "vmcnt holds 6 bits");
  static_assert(BN == 32 || BN == 64, "slab width");
  static_assert(kLds <= 160 * 1024, "LDS");
};

template <int LAYOUT, int MI, int BN>
__global__ __launch_bounds__(256, 1) void gemm_i8_skinny_kernel(GemmArgs g) {
#pragma clang fp contract(off)
  using Sh = SkinnyShape<MI, BN>;
  constexpr int D = Sh::kD, NJ = BN / 32, NL = Sh::kNL;
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  // consecutive ids (the K slices and row tiles of one slab, then the next slabs) share an XCD's L2
  const int64_t L = xcd_remap(blockIdx.x, g.n_tiles * g.m_slots * g.k_split);
  const int64_t ks = L % g.k_split, rt = (L / g.k_split) % g.m_slots, slab = L / (g.k_split * g.m_slots);
  const int64_t rb = rt * MI * 32;  // first row of this row tile
  const int64_t n0 = slab * BN;
  const int64_t nk = g.k / 64;
  const int64_t kb = ks * g.k_per;
  const int64_t ke = kb + g.k_per < nk ? kb + g.k_per : nk;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ns = kb + w < ke ? static_cast<int>((ke - kb - w + 3) / 4) : 0;  // stages kb + w + 4t of this wave
  int8_t* ring = smem + w * D * Sh::kSlot;
  const int m = static_cast<int>(g.m - rb < MI * 32 ? g.m - rb : MI * 32);  // rows of this row tile

  // weight source of load q relative to the stage's first K row, and the LDS placement: lane L of a
  // load fills bytes 16L .. 16L + 15 of its 1 KB
  //   [K, N] weights: slot = [64 k][BN B]; chunk c of k row r stored at c ^ 2((r >> 2) & 1) (BN = 64)
  //   [N, K] weights: slot = [BN n][64 B]; chunk c of row r stored at c ^ ((r >> 2) & 3)
  int64_t boff[Sh::kNB];
#pragma unroll
  for (int q = 0; q < Sh::kNB; ++q) {
    if constexpr (LAYOUT == TAI_LAYOUT_KN) {
      constexpr int CPR = BN / 16, RPL = 1024 / BN;
      const int kr = RPL * q + lane / CPR;
      const int c = (lane % CPR) ^ (BN == 64 ? ((kr >> 2) & 1) << 1 : 0);
      int64_t nn = n0 + 16 * c;
      nn = nn + 16 <= g.n ? nn : g.n - 16;
      boff[q] = kr * g.n + nn;
    } else {
      const int r = 16 * q + lane / 4;
      const int c = (lane & 3) ^ ((r >> 2) & 3);
      const int64_t nn = n0 + r < g.n ? n0 + r : g.n - 1;
      boff[q] = nn * g.k + 16 * c;
    }
  }
  auto stage_k = [&](int t) -> int64_t { return (kb + w + 4 * static_cast<int64_t>(t)) * 64; };
  auto issue_b = [&](int t, int slot) {
    const int64_t k0 = stage_k(t);
    const int8_t* base = LAYOUT == TAI_LAYOUT_KN ? g.b + k0 * g.n : g.b + k0;
#pragma unroll
    for (int q = 0; q < Sh::kNB; ++q)
      __builtin_amdgcn_global_load_lds((gbl_void*)(base + boff[q]), (lds_void*)(ring + slot * Sh::kSlot + q * 1024), 16,
                                       0, 0);
  };
  // activation stage: [MI * 32 rows][64 B] after the weight stage, chunk c of row r stored at
  // c ^ ((r >> 2) & 3); rows past m re-read row m - 1 (their sums are never stored). Loaded through LDS
  // (16 rows of 64 contiguous bytes per instruction): loading the fragments straight into registers
  // (32 rows of 32 bytes per instruction) made the config-1 gate_up 17.5 instead of 12 us.
  const int8_t* asrc[2 * MI];
#pragma unroll
  for (int q = 0; q < 2 * MI; ++q) {
    const int r = 16 * q + lane / 4;
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    asrc[q] = g.a + (rb + (r < m ? r : m - 1)) * g.k + 16 * c;
  }
  auto issue_a = [&](int t, int slot) {
    const int64_t k0 = stage_k(t);
#pragma unroll
    for (int q = 0; q < 2 * MI; ++q)
      __builtin_amdgcn_global_load_lds((gbl_void*)(asrc[q] + k0),
                                       (lds_void*)(ring + slot * Sh::kSlot + Sh::kSlotB + q * 1024), 16, 0, 0);
  };
  auto read_a = [&](int slot, int h, int i) -> v4i {
    const int r = 32 * i + (lane & 31);
    const int c = (2 * h + (lane >> 5)) ^ ((r >> 2) & 3);
    return ds_read_b128(ring + slot * Sh::kSlot + Sh::kSlotB + r * 64 + 16 * c);
  };
  // weight fragment (K step h, column block j) of this lane from ring slot `slot`
  const int l16 = lane & 15;
  auto read_b = [&](int slot, int h, int j) -> v4i {
    const int8_t* st = ring + slot * Sh::kSlot;
    if constexpr (LAYOUT == TAI_LAYOUT_KN) {
      const int col = 32 * j + ((lane >> 4) & 1) * 16 + (l16 & 1) * 8;
      const int k_lo = 32 * h + (lane >> 5) * 16 + (l16 >> 1), k_hi = k_lo + 8;
      auto swz = [](int k) { return BN == 64 ? ((k >> 2) & 1) << 1 : 0; };
      return ds_read_tr8_pair(st + k_lo * BN + 16 * ((col >> 4) ^ swz(k_lo)) + (col & 15),
                              st + k_hi * BN + 16 * ((col >> 4) ^ swz(k_hi)) + (col & 15));
    } else {
      const int r = 32 * j + (lane & 31);
      const int c = (2 * h + (lane >> 5)) ^ ((r >> 2) & 3);
      return ds_read_b128(st + r * 64 + 16 * c);
    }
  };

  v16i acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // Per stage: its weight loads, then its activation loads, all global -> LDS. Loads complete in
  // issue order, so stage t has landed once only the D - 1 stages issued after it are outstanding.
  // Every iteration issues one stage (past the wave's last stage it re-reads that stage and nothing
  // consumes it), so the waits are the same constant in every iteration.
  if (ns > 0) {
    auto clamp = [&](int t) { return t < ns ? t : ns - 1; };
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue_b(clamp(d), d);
      issue_a(clamp(d), d);
    }
    for (int t0 = 0; t0 < ns; t0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int t = t0 + d;
        wait_vmcnt<(D - 1) * NL>();
        v4i fb[2][NJ], fa[2][MI];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) fb[h][j] = read_b(d, h, j);
#pragma unroll
          for (int i = 0; i < MI; ++i) fa[h][i] = read_a(d, h, i);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // the reads are asm the compiler takes as complete at issue: route their results through the
        // wait so no use is scheduled above it
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) asm volatile("" : "+v"(fb[h][j]));
#pragma unroll
          for (int i = 0; i < MI; ++i) asm volatile("" : "+v"(fa[h][i]));
        }
        issue_b(clamp(t + D), d);  // the slot's fragments are in registers: refill it
        issue_a(clamp(t + D), d);
        if (t < ns) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
              for (int j = 0; j < NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[h][i], fb[h][j], acc[i][j], 0, 0, 0);
        }
      }
    }
    wait_vmcnt<0>();  // the trailing re-reads land before the ring is reused below
  }

  // Sum the four waves' partial tiles through LDS (the ring is free once every wave is past its loop).
  __syncthreads();
  int32_t* red = reinterpret_cast<int32_t*>(smem);
  constexpr int kTileWords = MI * 32 * Sh::kRowWords;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        red[w * kTileWords + row * Sh::kRowWords + 32 * j + (lane & 31)] = acc[i][j][r];
      }
  __syncthreads();
  const bool partial = g.k_split > 1;
  const int32_t* bias_i = (g.bias && g.bias_dt == TAI_DT_INT32) ? static_cast<const int32_t*>(g.bias) : nullptr;
  const float* bias_f = (g.bias && g.bias_dt == TAI_DT_FP32) ? static_cast<const float*>(g.bias) : nullptr;
  constexpr int G4 = BN / 4;
  for (int idx = threadIdx.x; idx < MI * 32 * G4; idx += 256) {
    const int row = idx / G4, c4 = 4 * (idx % G4);
    const int64_t col = n0 + c4;
    if (row >= m || col >= g.n) continue;
    int4 s = *reinterpret_cast<const int4*>(red + row * Sh::kRowWords + c4);
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      const int4 v = *reinterpret_cast<const int4*>(red + q * kTileWords + row * Sh::kRowWords + c4);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    const int64_t o = (rb + row) * g.n + col;
    if (partial) {
      *reinterpret_cast<int4*>(static_cast<int32_t*>(g.out) + ks * g.m * g.n + o) = s;
      continue;
    }
    int32_t v[4] = {s.x, s.y, s.z, s.w};
    if (bias_i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += bias_i[col + q];
    }
    if (g.out_dt == TAI_DT_INT32) {
      *reinterpret_cast<int4*>(static_cast<int32_t*>(g.out) + o) = make_int4(v[0], v[1], v[2], v[3]);
      continue;
    }
    const float pt = g.pts ? g.pts[rb + row] : 1.0f;
    float f[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float sc = g.scale_len == 1 ? g.scale[0] : g.scale[col + q];
      f[q] = (static_cast<float>(v[q]) * sc) * pt + (bias_f ? bias_f[col + q] : -0.0f);
    }
    if (g.out_dt == TAI_DT_FP32) {
      *reinterpret_cast<float4*>(static_cast<float*>(g.out) + o) = make_float4(f[0], f[1], f[2], f[3]);
    } else {
      uint16_t hv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) hv[q] = g.out_dt == TAI_DT_BF16 ? f32_to_bf16(f[q]) : f32_to_f16(f[q]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.out) + o) =
          make_uint2(hv[0] | (static_cast<uint32_t>(hv[1]) << 16), hv[2] | (static_cast<uint32_t>(hv[3]) << 16));
    }
  }
}

// Plan of the skinny kernel: 64-column slabs when there are enough of them to fill the chip, else
// 32; K split over workgroups toward one workgroup per CU, keeping at least one stage per wave (on
// the config-1 down projection the split plus its reduction takes 15 us, one workgroup per slab 21 us).
struct SkinnyPlan {
  int bn, mi;
  int64_t slabs, row_tiles, split, per;
};

bool skinny_fit(int64_t m, int64_t k, int64_t n) {
  return m >= 1 && m <= 128 && k >= 64 && k % 64 == 0 && n >= 16 && n % 16 == 0 && n < (1ll << 31);
}

#ifndef TAI_SK_ROWTILES
#define TAI_SK_ROWTILES 1
#endif
SkinnyPlan skinny_fit_plan(int64_t m, int64_t k, int64_t n) {
  SkinnyPlan p{};
  p.bn = cdiv(n, 64) >= 128 ? 64 : 32;
  p.slabs = cdiv(n, p.bn);
  // 65..128 rows over few slabs (which would split K four ways or more): two row tiles of 64 instead,
  // so K splits half as often and the partials to sum halve (config-1 down projection 12.3 -> 10.0 us
  // with [N, K] weights; with 176 slabs, as in its gate_up, the row tiles measured slower)
  const bool split_rows = TAI_SK_ROWTILES && m > 64 && p.slabs < 128;
  p.mi = m <= 32 ? 1 : (m <= 64 || split_rows ? 2 : 4);
  p.row_tiles = cdiv(m, 32 * p.mi);
  const int64_t nk = k / 64;
  const int64_t units = p.slabs * p.row_tiles;
  int64_t want = (256 + units / 2) / units;
  const int64_t cap = nk / 4 > 1 ? nk / 4 : 1;
  want = want < 1 ? 1 : (want > cap ? cap : want);
  p.per = cdiv(nk, want);
  p.split = cdiv(nk, p.per);
  return p;
}

template <int LAYOUT, int MI, int BN>
bool skinny_launch_one(const GemmArgs& g, hipStream_t st) {
  using Sh = SkinnyShape<MI, BN>;
  static const bool ready = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_i8_skinny_kernel<LAYOUT, MI, BN>),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, Sh::kLds) == hipSuccess;
  if (!ready) return false;
  gemm_i8_skinny_kernel<LAYOUT, MI, BN>
      <<<dim3(static_cast<unsigned>(g.n_tiles * g.m_slots * g.k_split)), 256, Sh::kLds, st>>>(g);
  return true;
}

template <int LAYOUT>
bool skinny_launch_layout(const GemmArgs& g, const SkinnyPlan& p, hipStream_t st) {
  if (p.bn == 64) {
    if (p.mi == 1) return skinny_launch_one<LAYOUT, 1, 64>(g, st);
    if (p.mi == 2) return skinny_launch_one<LAYOUT, 2, 64>(g, st);
    return skinny_launch_one<LAYOUT, 4, 64>(g, st);
  }
  if (p.mi == 1) return skinny_launch_one<LAYOUT, 1, 32>(g, st);
  if (p.mi == 2) return skinny_launch_one<LAYOUT, 2, 32>(g, st);
  return skinny_launch_one<LAYOUT, 4, 32>(g, st);
}

bool skinny_launch(const GemmArgs& g, int layout, const SkinnyPlan& p, hipStream_t st) {
  return layout == TAI_LAYOUT_NK ? skinny_launch_layout<TAI_LAYOUT_NK>(g, p, st)
                                 : skinny_launch_layout<TAI_LAYOUT_KN>(g, p, st);
}

// [K, N] -> [N, K] byte transpose through LDS, 64 x 256 tiles (K % 64 == 0, N % 256 == 0). Large dense
// GEMMs with a [K, N] weight run on the transposed copy: the [N, K] kernel reads its B fragments with
// plain 16-byte LDS reads instead of transposing ones and holds a higher clock (8192^3: the transpose
// moves 128 MB, ~25 us, and the GEMM gains more than that).
__global__ __launch_bounds__(256) void transpose_i8_kernel(const int8_t* __restrict__ b, int64_t k, int64_t n,
                                                          int8_t* __restrict__ bt) {
  __shared__ uint32_t tile[64][65];  // 64 k rows of 256 bytes (64 words), one word of padding
  const int64_t tiles_n = n / 256;
  const int64_t k0 = (blockIdx.x / tiles_n) * 64, n0 = (blockIdx.x % tiles_n) * 256;
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // 16-byte chunks, 16 per k row
    const int c = t + 256 * i, r = c >> 4, c16 = c & 15;
    const uint4 v = *reinterpret_cast<const uint4*>(b + (k0 + r) * n + n0 + 16 * c16);
    tile[r][4 * c16] = v.x; tile[r][4 * c16 + 1] = v.y; tile[r][4 * c16 + 2] = v.z; tile[r][4 * c16 + 3] = v.w;
  }
  __syncthreads();
  // lane: columns 4 ng .. 4 ng + 3; wave: k rows 16 kc .. 16 kc + 15; four 4 x 4 byte transposes give
  // 16 bytes of each of the four output rows
  const int ng = t & 63, kc = t >> 6;
  uint32_t out[4][4];  // [column][k word]
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t in[4] = {tile[16 * kc + 4 * q][ng], tile[16 * kc + 4 * q + 1][ng], tile[16 * kc + 4 * q + 2][ng],
                            tile[16 * kc + 4 * q + 3][ng]};
    uint32_t tr[4];
    transpose4x4(in, tr);  // tr[c] = bytes (k 4q .. 4q + 3) of column c
#pragma unroll
    for (int c = 0; c < 4; ++c) out[c][q] = tr[c];
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
    *reinterpret_cast<uint4*>(bt + (n0 + 4 * ng + c) * k + k0 + 16 * kc) = make_uint4(out[c][0], out[c][1], out[c][2], out[c][3]);
}

// Dense [K, N]-weight GEMMs at least this tall take the transpose above (its cost is below the
// [N, K] kernel's gain from M = 4096 on).
constexpr int64_t kTransposeMinM = 4096;
bool transpose_ok(int64_t m, int64_t k, int64_t n) { return m >= kTransposeMinM && k % 64 == 0 && n % 256 == 0; }

// Second half of npu_grouped_matmul_swiglu_quant_v2: one wave per row; the row's scale is
// max|h| / 127 from the column tiles' partial maxima, y = clamp(rint(h / scale), -128, 127)
// (npu_dynamic_quant arithmetic; a zero row gives scale 0 and y 0).
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float* __restrict__ h, const float* __restrict__ part,
                                                           int64_t nparts, int64_t m, int64_t n2, int8_t* __restrict__ y,
                                                           float* __restrict__ scale) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (row >= m) return;
  float amax = 0.0f;
  for (int64_t p = lane; p < nparts; p += 64) amax = fmaxf(amax, part[row * nparts + p]);
  amax = wave_max(amax);
  const float sc = amax / 127.0f, inv = rcp_f32(sc);
  for (int64_t c = 4 * lane; c < n2; c += 256) {
    const float4 v = *reinterpret_cast<const float4*>(h + row * n2 + c);
    const float vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t word = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) word |= static_cast<uint32_t>(static_cast<uint8_t>(quant_i8(vv[q], sc, inv))) << (8 * q);
    *reinterpret_cast<uint32_t*>(y + row * n2 + c) = word;
  }
  if (lane == 0) scale[row] = sc;
}

}  // namespace
}  // namespace tai

using namespace tai;

static size_t quant_matmul_ws_base(int64_t m, int64_t k, int64_t n) {
  if (m <= 0 || n <= 0) return 0;
  if (transpose_ok(m, k, n)) return static_cast<size_t>(k) * static_cast<size_t>(n) + 256;  // [N, K] copy of x2
  if (skinny_fit(m, k, n)) {
    const SkinnyPlan p = skinny_fit_plan(m, k, n);
    return p.split > 1 ? static_cast<size_t>(p.split) * static_cast<size_t>(m) * static_cast<size_t>(n) * 4 + 256 : 0;
  }
  if (!skinny_ok(m, k, n, TAI_LAYOUT_NK)) return 0;
  const SplitPlan p = skinny_plan(m, k, n);
  return p.split > 1 ? static_cast<size_t>(p.split) * static_cast<size_t>(m) * static_cast<size_t>(n) * 4 + 256 : 0;
}

// int8 output: y = clamp(rint(f + offset[n]), -128, 127) of the fp32 result f (fp32 add, then round
// half to even); 4 elements per thread.
__global__ __launch_bounds__(256) void requant_i8_kernel(const float* __restrict__ f, const float* __restrict__ offset,
                                                         int64_t offset_len, int64_t m, int64_t n, int8_t* __restrict__ y) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= m * n) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (i + q >= m * n) break;
    const int64_t col = (i + q) % n;
    float v = f[i + q];
    if (offset) v = v + offset[offset_len == 1 ? 0 : col];
    y[i + q] = static_cast<int8_t>(static_cast<int>(fminf(fmaxf(rintf(v), -128.0f), 127.0f)));
  }
}

static int quant_matmul_impl(const int8_t* x1, const int8_t* x2, int64_t m, int64_t k, int64_t n, int x2_layout,
                             const float* scale, int64_t scale_len, const float* pertoken_scale, const void* bias,
                             int bias_dtype, int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream);

extern "C" size_t tai_quant_matmul_workspace_size(int64_t m, int64_t k, int64_t n, int out_dtype) {
  const size_t base = (quant_matmul_ws_base(m, k, n) + 255) / 256 * 256;
  if (out_dtype != TAI_DT_INT8 || m <= 0 || n <= 0) return quant_matmul_ws_base(m, k, n);
  return base + static_cast<size_t>(m) * static_cast<size_t>(n) * sizeof(float) + 256;
}

extern "C" int tai_transpose_kn_to_nk(const int8_t* b, int64_t k, int64_t n, int8_t* out, void* stream) {
  TAI_CHECK_ARG(k >= 0 && n >= 0, "tai_transpose_kn_to_nk: negative size");
  TAI_UNSUPPORTED(k % 64 != 0 || n % 256 != 0, "tai_transpose_kn_to_nk: needs k %% 64 == 0 and n %% 256 == 0");
  if (k == 0 || n == 0) return TAI_OK;
  TAI_CHECK_ARG(b && out, "tai_transpose_kn_to_nk: null pointer");
  transpose_i8_kernel<<<dim3(static_cast<unsigned>((k / 64) * (n / 256))), 256, 0, static_cast<hipStream_t>(stream)>>>(
      b, k, n, out);
  return launch_status("tai_transpose_kn_to_nk");
}

// [rows, n] int8 -> the same rows with 64-column blocks reordered: output block 2t is input block t
// (a gate block), output block 2t + 1 is input block n / 128 + t (the matching up block). One thread
// per 16 bytes.
__global__ __launch_bounds__(256) void swiglu_pack_kernel(const int8_t* __restrict__ src, int64_t rows, int64_t n,
                                                          int8_t* __restrict__ dst) {
  const int64_t per_row = n / 16;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * per_row) return;
  const int64_t r = i / per_row, c = (i % per_row) * 16;  // output column
  const int64_t blk = c / 64, j = c % 64;
  const int64_t sc = (blk & 1 ? n / 2 : 0) + 64 * (blk >> 1) + j;
  *reinterpret_cast<uint4*>(dst + r * n + c) = *reinterpret_cast<const uint4*>(src + r * n + sc);
}

extern "C" int tai_swiglu_pack_kn(const int8_t* w, int64_t rows, int64_t n, int8_t* out, void* stream) {
  TAI_CHECK_ARG(rows >= 0 && n >= 0, "tai_swiglu_pack_kn: negative size");
  TAI_CHECK_ARG(n % 128 == 0, "tai_swiglu_pack_kn: n must be a multiple of 128");
  if (rows == 0 || n == 0) return TAI_OK;
  TAI_CHECK_ARG(w && out && w != out, "tai_swiglu_pack_kn: null or aliased pointer");
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  TAI_CHECK_ARG(al(w) && al(out), "tai_swiglu_pack_kn: 16-byte aligned pointers");
  const int64_t threads = rows * (n / 16);
  swiglu_pack_kernel<<<dim3(static_cast<unsigned>(cdiv(threads, 256))), 256, 0, static_cast<hipStream_t>(stream)>>>(
      w, rows, n, out);
  return launch_status("tai_swiglu_pack_kn");
}

extern "C" int tai_quant_matmul_prepack_wanted(int64_t m, int64_t k, int64_t n) {
  // tall products (the [N, K] big kernel) and decode-sized ones (the skinny kernel streams each
  // weight row's K range contiguously from [N, K] storage instead of 32- or 64-byte pieces of every
  // [K, N] row: config-1 gate_up 12.4 -> 10.7 us)
  const bool tiles = k % 64 == 0 && n % 256 == 0;
  return (transpose_ok(m, k, n) || (tiles && skinny_fit(m, k, n))) ? 1 : 0;
}

extern "C" int tai_quant_matmul(const int8_t* x1, const int8_t* x2, int64_t m, int64_t k, int64_t n, int x2_layout,
                                const float* scale, int64_t scale_len, const float* offset, int64_t offset_len,
                                const float* pertoken_scale, const void* bias, int bias_dtype, int out_dtype, void* out,
                                void* workspace, size_t ws_bytes, void* stream) {
  if (out_dtype != TAI_DT_INT8) {
    TAI_CHECK_ARG(offset == nullptr, "tai_quant_matmul: offset applies to int8 output only");
    return quant_matmul_impl(x1, x2, m, k, n, x2_layout, scale, scale_len, pertoken_scale, bias, bias_dtype, out_dtype,
                             out, workspace, ws_bytes, stream);
  }
  TAI_CHECK_ARG(m >= 0 && k >= 0 && n >= 0, "tai_quant_matmul: negative size");
  TAI_CHECK_ARG(scale != nullptr, "tai_quant_matmul: int8 output needs scale");
  TAI_CHECK_ARG(offset == nullptr || offset_len == 1 || offset_len == n, "tai_quant_matmul: offset must have 1 or n "
                "entries");
  TAI_CHECK_ARG(bias == nullptr || bias_dtype == TAI_DT_INT32, "tai_quant_matmul: int8 output takes an int32 bias only");
  if (m == 0 || n == 0) return TAI_OK;
  const size_t base = (quant_matmul_ws_base(m, k, n) + 255) / 256 * 256;
  const size_t need = tai_quant_matmul_workspace_size(m, k, n, out_dtype);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_quant_matmul: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  float* f = reinterpret_cast<float*>(static_cast<char*>(workspace) + base);
  const int rc = quant_matmul_impl(x1, x2, m, k, n, x2_layout, scale, scale_len, pertoken_scale, bias, bias_dtype,
                                   TAI_DT_FP32, f, workspace, base, stream);
  if (rc != TAI_OK) return rc;
  requant_i8_kernel<<<dim3(static_cast<unsigned>(cdiv(m * n, 1024))), 256, 0, static_cast<hipStream_t>(stream)>>>(
      f, offset, offset_len, m, n, static_cast<int8_t*>(out));
  return launch_status("tai_quant_matmul");
}

static int quant_matmul_impl(const int8_t* x1, const int8_t* x2, int64_t m, int64_t k, int64_t n, int x2_layout,
                             const float* scale, int64_t scale_len, const float* pertoken_scale, const void* bias,
                             int bias_dtype, int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream) {
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
  if (skinny_fit(m, k, n)) {
    const SkinnyPlan p = skinny_fit_plan(m, k, n);
    g.n_tiles = p.slabs;
    g.m_slots = p.row_tiles;
    g.k_split = p.split;
    g.k_per = p.per;
    if (p.split == 1) {
      if (!skinny_launch(g, x2_layout, p, st)) return launch_status("tai_quant_matmul (skinny LDS attribute)");
      return launch_status("tai_quant_matmul");
    }
    const size_t need = quant_matmul_ws_base(m, k, n);
    if (workspace == nullptr || ws_bytes < need) {
      set_error("tai_quant_matmul: workspace of %zu bytes, need %zu", ws_bytes, need);
      return TAI_ERR_WORKSPACE;
    }
    GemmArgs gp = g;  // partial pass: raw int32 slices into the workspace
    gp.out = workspace;
    if (!skinny_launch(gp, x2_layout, p, st)) return launch_status("tai_quant_matmul (skinny LDS attribute)");
    const dim3 rgrid(static_cast<unsigned>(cdiv(m * n, 1024)));
    const int32_t* part = static_cast<const int32_t*>(workspace);
    switch (out_dtype) {
      case TAI_DT_INT32: splitk_reduce_kernel<TAI_DT_INT32><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
      case TAI_DT_BF16: splitk_reduce_kernel<TAI_DT_BF16><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
      case TAI_DT_FP16: splitk_reduce_kernel<TAI_DT_FP16><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
      default: splitk_reduce_kernel<TAI_DT_FP32><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
    }
    return launch_status("tai_quant_matmul");
  }
  if (skinny_ok(m, k, n, x2_layout) && cfg_available<SkinnyCfg>()) {
    const SplitPlan p = skinny_plan(m, k, n);
    g.m_slots = p.m_slots;
    g.n_tiles = p.n_tiles;
    if (p.split == 1) {
      launch_cfg<SkinnyCfg>(g, x2_layout, st);
      return launch_status("tai_quant_matmul");
    }
    const size_t need = quant_matmul_ws_base(m, k, n);
    if (workspace == nullptr || ws_bytes < need) {
      set_error("tai_quant_matmul: workspace of %zu bytes, need %zu", ws_bytes, need);
      return TAI_ERR_WORKSPACE;
    }
    GemmArgs gp = g;  // partial pass: raw int32 slices into the workspace
    gp.scale = nullptr;
    gp.pts = nullptr;
    gp.bias = nullptr;
    gp.out_dt = TAI_DT_INT32;
    gp.out = workspace;
    gp.k_split = p.split;
    gp.k_per = p.per;
    const dim3 grid(static_cast<unsigned>(p.m_slots * p.n_tiles * p.split));
    if (x2_layout == TAI_LAYOUT_NK)
      cfg_kernel<SkinnyCfg, TAI_LAYOUT_NK, TAI_DT_INT32>()<<<grid, SkinnyCfg::kThreads, SkinnyCfg::kLds, st>>>(gp);
    else
      cfg_kernel<SkinnyCfg, TAI_LAYOUT_KN, TAI_DT_INT32>()<<<grid, SkinnyCfg::kThreads, SkinnyCfg::kLds, st>>>(gp);
    const dim3 rgrid(static_cast<unsigned>(cdiv(m * n, 1024)));
    const int32_t* part = static_cast<const int32_t*>(workspace);
    switch (out_dtype) {
      case TAI_DT_INT32: splitk_reduce_kernel<TAI_DT_INT32><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
      case TAI_DT_BF16: splitk_reduce_kernel<TAI_DT_BF16><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
      case TAI_DT_FP16: splitk_reduce_kernel<TAI_DT_FP16><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
      default: splitk_reduce_kernel<TAI_DT_FP32><<<rgrid, 256, 0, st>>>(part, p.split, g); break;
    }
    return launch_status("tai_quant_matmul");
  }
  if (m >= 256 && k % kBigBK == 0 && (x2_layout == TAI_LAYOUT_NK || n % 16 == 0) && cfg_available<BigSel>()) {
    g.m_slots = cdiv(m, kBigBM);
    g.n_tiles = cdiv(n, kBigBN);
    if (x2_layout == TAI_LAYOUT_KN && transpose_ok(m, k, n) && workspace != nullptr &&
        ws_bytes >= static_cast<size_t>(k) * static_cast<size_t>(n) &&
        (reinterpret_cast<uintptr_t>(workspace) % 16) == 0) {
      int8_t* bt = static_cast<int8_t*>(workspace);
      transpose_i8_kernel<<<dim3(static_cast<unsigned>((k / 64) * (n / 256))), 256, 0, st>>>(x2, k, n, bt);
      g.b = bt;
      launch_cfg<BigSel>(g, TAI_LAYOUT_NK, st);
      return launch_status("tai_quant_matmul");
    }
    launch_cfg<BigSel>(g, x2_layout, st);
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

static int grouped_matmul_impl(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                               int64_t num_groups, int w_layout, const int64_t* group_list, int group_list_type,
                               const float* scale, const float* per_token_scale, const void* bias, int bias_dtype,
                               int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream,
                               const int32_t* a_rows = nullptr, int64_t a_src_rows = 0);

extern "C" size_t tai_grouped_matmul_workspace_size(int64_t m, int64_t n, int64_t num_groups) {
  (void)n;
  // [live slot count, padded to 256 B][tile map][row -> group map]
  return 256 + sizeof(int4) * grouped_map_slots(m, num_groups, kMinBM) + sizeof(int32_t) * static_cast<size_t>(m) + 256;
}

extern "C" int tai_grouped_matmul(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                                  int64_t num_groups, int w_layout, const int64_t* group_list, int group_list_type,
                                  const float* scale, const float* per_token_scale, const void* bias, int bias_dtype,
                                  int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream) {
  return grouped_matmul_impl(x, weight, m, k, n, num_groups, w_layout, group_list, group_list_type, scale,
                             per_token_scale, bias, bias_dtype, out_dtype, out, workspace, ws_bytes, stream);
}

extern "C" int tai_grouped_matmul_gather(const int8_t* x, int64_t x_rows, const int32_t* a_rows,
                                         const int8_t* weight, int64_t m, int64_t k, int64_t n, int64_t num_groups,
                                         int w_layout, const int64_t* group_list, int group_list_type,
                                         const float* scale, const float* per_token_scale, const void* bias,
                                         int bias_dtype, int out_dtype, void* out, void* workspace, size_t ws_bytes,
                                         void* stream) {
  TAI_CHECK_ARG(x_rows >= 0, "tai_grouped_matmul_gather: x_rows must be >= 0");
  if (m > 0 && n > 0) TAI_CHECK_ARG(a_rows && x_rows > 0, "tai_grouped_matmul_gather: a_rows and x rows are required");
  return grouped_matmul_impl(x, weight, m, k, n, num_groups, w_layout, group_list, group_list_type, scale,
                             per_token_scale, bias, bias_dtype, out_dtype, out, workspace, ws_bytes, stream, a_rows,
                             x_rows);
}

// ----------------------------------------------------------------------------- no-allocation variant
// The grouped GEMM's scratch (tile table, live count, row -> group map) lives in a file-scope device
// array instead of a caller workspace. Each device holds its own copy; its address is looked up once
// per device with hipGetSymbolAddress and only that address reaches the kernels. Calls on one device
// share the array, so calls that overlap on one device race; every call rewrites what it reads (the
// prologue writes the whole table and count), so nothing has to start at zero.
constexpr size_t kNoAllocScratchBytes = size_t(1) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Address of this device's copy of `scratch` (looked up on the device's first call).
void* device_scratch(int* err_dev) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    *err_dev = dev;
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (g_scratch_err[dev] != hipSuccess) (void)hipGetLastError();
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
  });
  *err_dev = dev;
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" size_t tai_grouped_matmul_noalloc_max_scratch(void) { return kNoAllocScratchBytes; }

extern "C" int tai_grouped_matmul_noalloc(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                                          int64_t num_groups, int w_layout, const int64_t* group_list,
                                          int group_list_type, const float* scale, const float* per_token_scale,
                                          const void* bias, int bias_dtype, int out_dtype, void* out, void* stream) {
  TAI_CHECK_ARG(m >= 0 && n >= 0 && num_groups >= 1 && num_groups <= 2048, "tai_grouped_matmul_noalloc: bad sizes");
  const size_t need = tai_grouped_matmul_workspace_size(m, n, num_groups);
  if (need > kNoAllocScratchBytes) {
    set_error("tai_grouped_matmul_noalloc: %lld rows and %lld groups need %zu bytes of scratch; the no-allocation "
              "entry point holds %zu (use tai_grouped_matmul with a workspace)",
              static_cast<long long>(m), static_cast<long long>(num_groups), need, kNoAllocScratchBytes);
    return TAI_ERR_INVALID;
  }
  int dev = -1;
  void* ws = device_scratch(&dev);
  if (ws == nullptr) {
    set_error("tai_grouped_matmul_noalloc: no scratch address for device %d (%s)", dev,
              (dev >= 0 && dev < kMaxDevices) ? hipGetErrorString(g_scratch_err[dev]) : "no current device");
    return TAI_ERR_LAUNCH;
  }
  return grouped_matmul_impl(x, weight, m, k, n, num_groups, w_layout, group_list, group_list_type, scale,
                             per_token_scale, bias, bias_dtype, out_dtype, out, ws, kNoAllocScratchBytes, stream);
}

static int grouped_matmul_impl(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                               int64_t num_groups, int w_layout, const int64_t* group_list, int group_list_type,
                               const float* scale, const float* per_token_scale, const void* bias, int bias_dtype,
                               int out_dtype, void* out, void* workspace, size_t ws_bytes, void* stream,
                               const int32_t* a_rows, int64_t a_src_rows) {
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
  const bool kn = w_layout == TAI_LAYOUT_KN;
  const bool big = kn ? (k % GrpKnSel::kBK == 0 && n % 16 == 0 && cfg_available<GrpKnSel>())
                      : (k % GrpSel::kBK == 0 && cfg_available<GrpSel>());
  const int bm = big ? (kn ? GrpKnSel::kBM : GrpSel::kBM) : kGroupedBM;
  const int bn = big ? (kn ? GrpKnSel::kBN : GrpSel::kBN) : 128;
  const int64_t slots = static_cast<int64_t>(grouped_map_slots(m, num_groups, bm));
  int64_t* live = static_cast<int64_t*>(workspace);
  int4* map = reinterpret_cast<int4*>(static_cast<char*>(workspace) + 256);
  int32_t* row_group = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + 256 +
                                                  sizeof(int4) * grouped_map_slots(m, num_groups, kMinBM));
  GemmArgs g{x, weight, m, k, n, k * n, scale, n, n, per_token_scale, bias, bias_dtype, n, out_dtype, out,
             map, slots, cdiv(n, bn), live};
  g.a_rows = a_rows;
  g.a_src_rows = a_src_rows;
  const bool fast = fast_path_ok(g, w_layout);
  group_tiles_kernel<<<1, 1024, sizeof(int64_t) * (3 * num_groups + 1), st>>>(group_list, num_groups, group_list_type, m,
                                                                              bm, map, slots, live,
                                                                              fast ? nullptr : row_group);
  if (!fast) {
    gemm_i8_generic_kernel<<<dim3(static_cast<unsigned>(cdiv(m * n, 256))), 256, 0, st>>>(g, w_layout, row_group);
    return launch_status("tai_grouped_matmul");
  }
  if (big && kn && TAI_MIXED && n % GrpKnSel::kBN == 0 && mixed_available()) launch_mixed(g, st);
  else if (big && kn) launch_cfg<GrpKnSel>(g, w_layout, st);
  else if (big) launch_cfg<GrpSel>(g, w_layout, st);
  else launch_tile<128, 128>(g, w_layout, st);
  return launch_status("tai_grouped_matmul");
}

// Workspace of the fused op: the grouped tile table, then h [m, n / 2] fp32 and the per-tile row maxima.
static size_t swiglu_ws_parts(int64_t m, int64_t n, int64_t num_groups, size_t* h_off, size_t* part_off) {
  const size_t base = (tai_grouped_matmul_workspace_size(m, n, num_groups) + 255) / 256 * 256;
  const size_t hb = (static_cast<size_t>(m) * static_cast<size_t>(n / 2) * sizeof(float) + 255) / 256 * 256;
  const int64_t max_tiles = cdiv(n / 2, 64);  // the narrowest tile covers 64 output columns
  if (h_off) *h_off = base;
  if (part_off) *part_off = base + hb;
  return base + hb + static_cast<size_t>(m) * static_cast<size_t>(max_tiles) * sizeof(float) + 256;
}

extern "C" size_t tai_grouped_matmul_swiglu_quant_workspace_size(int64_t m, int64_t n, int64_t num_groups) {
  return swiglu_ws_parts(m, n, num_groups, nullptr, nullptr);
}

static int swiglu_quant_impl(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                             int64_t num_groups, int w_layout, const int64_t* group_list, int group_list_type,
                             const float* weight_scale, const float* x_scale, int8_t* y, float* y_scale,
                             void* workspace, size_t ws_bytes, void* stream, const int32_t* a_rows,
                             int64_t a_src_rows);

extern "C" int tai_grouped_matmul_swiglu_quant(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                                               int64_t num_groups, int w_layout, const int64_t* group_list,
                                               int group_list_type, const float* weight_scale, const float* x_scale,
                                               int8_t* y, float* y_scale, void* workspace, size_t ws_bytes,
                                               void* stream) {
  return swiglu_quant_impl(x, weight, m, k, n, num_groups, w_layout, group_list, group_list_type, weight_scale,
                           x_scale, y, y_scale, workspace, ws_bytes, stream, nullptr, 0);
}

extern "C" int tai_grouped_matmul_swiglu_quant_gather(const int8_t* x, int64_t x_rows, const int32_t* a_rows,
                                                      const int8_t* weight, int64_t m, int64_t k, int64_t n,
                                                      int64_t num_groups, int w_layout, const int64_t* group_list,
                                                      int group_list_type, const float* weight_scale,
                                                      const float* x_scale, int8_t* y, float* y_scale,
                                                      void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(x_rows >= 0, "tai_grouped_matmul_swiglu_quant_gather: x_rows must be >= 0");
  if (m > 0) TAI_CHECK_ARG(a_rows && x_rows > 0, "tai_grouped_matmul_swiglu_quant_gather: a_rows and x rows are required");
  return swiglu_quant_impl(x, weight, m, k, n, num_groups, w_layout, group_list, group_list_type, weight_scale,
                           x_scale, y, y_scale, workspace, ws_bytes, stream, a_rows, x_rows);
}

static int swiglu_quant_impl(const int8_t* x, const int8_t* weight, int64_t m, int64_t k, int64_t n,
                             int64_t num_groups, int w_layout, const int64_t* group_list, int group_list_type,
                             const float* weight_scale, const float* x_scale, int8_t* y, float* y_scale,
                             void* workspace, size_t ws_bytes, void* stream, const int32_t* a_rows,
                             int64_t a_src_rows) {
  TAI_CHECK_ARG(m >= 0 && k >= 0 && n >= 2 && num_groups >= 1, "tai_grouped_matmul_swiglu_quant: bad sizes");
  TAI_CHECK_ARG(num_groups <= 2048, "tai_grouped_matmul_swiglu_quant: at most 2048 groups");
  TAI_CHECK_ARG(w_layout == TAI_LAYOUT_KN || w_layout == TAI_LAYOUT_NK || w_layout == TAI_LAYOUT_KN_SWIGLU,
                "tai_grouped_matmul_swiglu_quant: w_layout");
  const bool packed = w_layout == TAI_LAYOUT_KN_SWIGLU;
  if (packed) w_layout = TAI_LAYOUT_KN;
  TAI_CHECK_ARG(group_list_type == 0 || group_list_type == 1, "tai_grouped_matmul_swiglu_quant: group_list_type");
  TAI_CHECK_ARG(group_list && weight_scale && x_scale, "tai_grouped_matmul_swiglu_quant: group_list, weight_scale and "
                "x_scale are required");
  if (m == 0) return TAI_OK;
  TAI_CHECK_ARG(x && weight && y && y_scale, "tai_grouped_matmul_swiglu_quant: null pointer");
  TAI_CHECK_ARG(m < (1ll << 31), "tai_grouped_matmul_swiglu_quant: m must be < 2^31");
  const bool kn = w_layout == TAI_LAYOUT_KN;
  const int bk = kn ? GrpKnSel::kBK : GrpSel::kBK;
  const int bn = kn ? GrpKnSel::kBN : GrpSel::kBN;
  const bool avail = kn ? cfg_available<GrpKnSel>() : cfg_available<GrpSel>();
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  TAI_UNSUPPORTED(!avail || k % bk != 0 || (n / 2) % (bn / 2) != 0 || !al(x) || !al(weight),
                  "tai_grouped_matmul_swiglu_quant: needs k %% %d == 0, (n / 2) %% %d == 0 and 16-byte aligned "
                  "operands", bk, bn / 2);
  size_t h_off = 0, part_off = 0;
  const size_t need = swiglu_ws_parts(m, n, num_groups, &h_off, &part_off);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_grouped_matmul_swiglu_quant: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int bm = kn ? GrpKnSel::kBM : GrpSel::kBM;
  const int64_t slots = static_cast<int64_t>(grouped_map_slots(m, num_groups, bm));
  char* wsp = static_cast<char*>(workspace);
  int64_t* live = reinterpret_cast<int64_t*>(wsp);
  int4* map = reinterpret_cast<int4*>(wsp + 256);
  float* h = reinterpret_cast<float*>(wsp + h_off);
  float* part = reinterpret_cast<float*>(wsp + part_off);
  const int64_t n_tiles = (n / 2) / (bn / 2);
  GemmArgs g{x, weight, m, k, n, k * n, weight_scale, n, n, x_scale, nullptr, 0, n, kOutSwiglu, nullptr,
             map, slots, n_tiles, live, h, part};
  g.swi_packed = packed ? 1 : 0;
  g.a_rows = a_rows;
  g.a_src_rows = a_src_rows;
  group_tiles_kernel<<<1, 1024, sizeof(int64_t) * (3 * num_groups + 1), st>>>(group_list, num_groups, group_list_type,
                                                                              m, bm, map, slots, live, nullptr);
  if (kn && TAI_MIXED && n % GrpKnSel::kBN == 0 && mixed_available()) launch_mixed(g, st);
  else if (kn) launch_cfg<GrpKnSel>(g, w_layout, st);
  else launch_cfg<GrpSel>(g, w_layout, st);
  swiglu_quant_kernel<<<dim3(static_cast<unsigned>(cdiv(m, 4))), 256, 0, st>>>(h, part, n / 128, m, n / 2, y, y_scale);
  return launch_status("tai_grouped_matmul_swiglu_quant");
}
