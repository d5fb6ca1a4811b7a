// MoE routing on one GPU: npu_moe_gating_top_k, npu_moe_init_routing(_v2) and
// npu_moe_finalize_routing - the single-GPU share of expert dispatch/combine.
//
// gating_top_k : one wave per token row; scores staged in LDS for the group scores, then the
//                iterative arg-max over registers with wave shuffles. Sigmoid/softmax are
//                evaluated in fp64 and rounded once to fp32 so the expert choice is reproducible.
// init_routing : stable counting sort of the t*k routing slots by expert, in four launches
//                (chunk histograms -> per-expert scan -> in-chunk ranks -> row gather).
//                Every kernel writes all of its outputs, so no memset is needed and the
//                sequence may be captured into a hipGraph.
// finalize     : one workgroup per token row, fp32 accumulation of the k weighted rows.
#include "common.h"

namespace tai {
namespace {

// ============================================================================ gating top-k
constexpr int kMaxExperts = 1024;
constexpr int kMaxGroups = 64;

struct GateArgs {
  const void* x;
  int x_dt;
  int64_t t, e;
  int k;
  const void* bias;
  int bias_dt;
  int k_group, group_count, group_select_mode, norm_type, out_flag;
  float rsf, eps;
  void* y;
  int32_t* idx;
  float* out;
};

// Larger (value, lower index) wins.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// 4 waves per workgroup, one row per wave.
__global__ __launch_bounds__(256) void gating_topk_kernel(GateArgs a) {
  __shared__ float s_sc[4][kMaxExperts];   // normalised scores s
  __shared__ float s_sb[4][kMaxExperts];   // selection scores s + bias
  __shared__ float s_gs[4][kMaxGroups];    // group scores
  __shared__ int s_keep[4][kMaxGroups];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + w;
  const bool valid = row < a.t;
  const int E = static_cast<int>(a.e);
  float* sc = s_sc[w];
  float* sb = s_sb[w];

  if (valid) {
    if (a.norm_type == 1) {
      for (int j = lane; j < E; j += 64) {
        double xv = static_cast<double>(load_as_f32(a.x, a.x_dt, row * E + j));
        sc[j] = static_cast<float>(1.0 / (1.0 + exp(-xv)));
      }
    } else {
      float m = -INFINITY;
      for (int j = lane; j < E; j += 64) m = fmaxf(m, load_as_f32(a.x, a.x_dt, row * E + j));
      m = wave_max(m);
      double sum = 0.0;
      for (int j = lane; j < E; j += 64) sum += exp(static_cast<double>(load_as_f32(a.x, a.x_dt, row * E + j)) - m);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
      for (int j = lane; j < E; j += 64) {
        double ev = exp(static_cast<double>(load_as_f32(a.x, a.x_dt, row * E + j)) - m);
        sc[j] = static_cast<float>(ev / sum);
      }
    }
    for (int j = lane; j < E; j += 64) {
      float v = sc[j];
      if (a.bias) v = v + load_as_f32(a.bias, a.bias_dt, j);
      sb[j] = v;
    }
  }
  __syncthreads();

  const int G = a.group_count;
  const int gsz = E / G;
  if (G > 1) {
    if (valid) {
      for (int g = lane; g < G; g += 64) {
        float b1 = -INFINITY, b2 = -INFINITY;
        for (int j = g * gsz; j < (g + 1) * gsz; ++j) {
          float v = sb[j];
          if (v > b1) { b2 = b1; b1 = v; } else if (v > b2) { b2 = v; }
        }
        s_gs[w][g] = (a.group_select_mode == 1 && gsz > 1) ? b1 + b2 : b1;
      }
    }
    __syncthreads();
    if (valid) {
      for (int g = lane; g < G; g += 64) {
        const float v = s_gs[w][g];
        int rank = 0;
        for (int h = 0; h < G; ++h) rank += better(s_gs[w][h], h, v, g) ? 1 : 0;
        s_keep[w][g] = rank < a.k_group;
      }
    }
    __syncthreads();
    if (valid) {
      for (int j = lane; j < E; j += 64)
        if (!s_keep[w][j / gsz]) sb[j] = -INFINITY;
    }
    __syncthreads();
  }

  // k rounds of arg-max: larger score wins, equal scores go to the lower expert id. The selection
  // scores stay in registers (lane holds experts lane + 64q), so a round is a local scan and one
  // wave reduction, with no LDS traffic and no barrier; lane r keeps the id chosen in round r.
  if (!valid) return;
  constexpr int kNV = kMaxExperts / 64;
  const int nq = (E + 63) / 64;
  float v[kNV];
#pragma unroll
  for (int q = 0; q < kNV; ++q) v[q] = (q < nq && lane + 64 * q < E) ? sb[lane + 64 * q] : -INFINITY;
  int my_sel = 0;
  for (int r = 0; r < a.k; ++r) {
    float bv = -INFINITY;
    int bi = kMaxExperts;
#pragma unroll
    for (int q = 0; q < kNV; ++q)
      if (q < nq && better(v[q], lane + 64 * q, bv, bi)) { bv = v[q]; bi = lane + 64 * q; }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(bv, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    bi = __builtin_amdgcn_readfirstlane(bi);
#pragma unroll
    for (int q = 0; q < kNV; ++q)
      if (lane + 64 * q == bi) v[q] = -INFINITY;
    if (lane == r) my_sel = bi;
  }
  const float myw = lane < a.k ? sc[my_sel] : 0.0f;
  float wsum = 0.0f;
  for (int r = 0; r < a.k; ++r) wsum = wsum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myw), r));
  if (lane < a.k) {
    float wv = myw;
    if (a.norm_type == 1) wv = wv / (wsum + a.eps);
    wv = wv * a.rsf;
    store_from_f32(a.y, a.x_dt, row * a.k + lane, wv);
    a.idx[row * a.k + lane] = my_sel;
  }
  if (a.out_flag && a.out)
    for (int j = lane; j < E; j += 64) a.out[row * E + j] = sc[j];
}

// The common DeepSeek-V3 shape (256 experts, sigmoid scores, no groups or 8 groups of 32) with every
// score in registers: lane l holds experts l + 64 q, q = 0..3, so expert group 2 q + (l >= 32) is one
// half-wave of slice q and its top-2 sum comes from butterfly merges of per-lane top-2 pairs, with no
// LDS and no workgroup barrier. Same arithmetic and tie rules as gating_topk_kernel, so the same result.
__global__ __launch_bounds__(256) void gating_topk_256_kernel(GateArgs a) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (row >= a.t) return;
  float sc[4], v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = lane + 64 * q;
    const double xv = static_cast<double>(load_as_f32(a.x, a.x_dt, row * 256 + j));
    sc[q] = static_cast<float>(1.0 / (1.0 + exp(-xv)));
    v[q] = a.bias ? sc[q] + load_as_f32(a.bias, a.bias_dt, j) : sc[q];
  }
  if (a.group_count == 8) {
    // top-2 of each half-wave (32 experts of one group), merged pairwise: (t1, t2) keep the largest
    // and second largest values counted with multiplicity
    float gsc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float t1 = v[q], t2 = -INFINITY;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) {
        const float u1 = __shfl_xor(t1, o, 64), u2 = __shfl_xor(t2, o, 64);
        const float n1 = fmaxf(t1, u1);
        t2 = fmaxf(fminf(t1, u1), fmaxf(t2, u2));
        t1 = n1;
      }
      gsc[q] = a.group_select_mode == 1 ? t1 + t2 : t1;
    }
    float gs[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gs[2 * q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gsc[q]), 0));
      gs[2 * q + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gsc[q]), 32));
    }
    bool keep[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      int rank = 0;
#pragma unroll
      for (int hh = 0; hh < 8; ++hh) rank += better(gs[hh], hh, gs[g], g) ? 1 : 0;
      keep[g] = rank < a.k_group;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool kept = lane < 32 ? keep[2 * q] : keep[2 * q + 1];
      if (!kept) v[q] = -INFINITY;
    }
  }
  int my_sel = 0;
  for (int r = 0; r < a.k; ++r) {
    float bv = -INFINITY;
    int bi = kMaxExperts;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (better(v[q], lane + 64 * q, bv, bi)) { bv = v[q]; bi = lane + 64 * q; }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(bv, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    bi = __builtin_amdgcn_readfirstlane(bi);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (lane + 64 * q == bi) v[q] = -INFINITY;
    if (lane == r) my_sel = bi;
  }
  // the normalised score of this lane's selected expert, from the lane that holds it
  const int sq = my_sel >> 6, sl = my_sel & 63;
  float s0 = __shfl(sc[0], sl, 64), s1 = __shfl(sc[1], sl, 64), s2 = __shfl(sc[2], sl, 64), s3 = __shfl(sc[3], sl, 64);
  const float picked = sq == 0 ? s0 : (sq == 1 ? s1 : (sq == 2 ? s2 : s3));
  const float myw = lane < a.k ? picked : 0.0f;
  float wsum = 0.0f;
  for (int r = 0; r < a.k; ++r) wsum = wsum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myw), r));
  if (lane < a.k) {
    float wv = myw;
    wv = wv / (wsum + a.eps);
    wv = wv * a.rsf;
    store_from_f32(a.y, a.x_dt, row * a.k + lane, wv);
    a.idx[row * a.k + lane] = my_sel;
  }
  if (a.out_flag && a.out) {
#pragma unroll
    for (int q = 0; q < 4; ++q) a.out[row * 256 + lane + 64 * q] = sc[q];
  }
}

// ============================================================================ init routing
constexpr int kChunk = 256;  // routing slots per chunk (one per thread)

struct RouteWs {
  int32_t* hist;      // [bins][chunks]: counts, then exclusive destination offsets
  int32_t* dst2src;   // [n] source slot of each destination row
  int32_t* total;     // [1] rows that fall in the expert range
  int32_t* bintot;    // [bins] rows per expert
};

__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

inline RouteWs carve_route_ws(void* ws, int64_t n, int64_t bins) {
  const int64_t chunks = cdiv(n, kChunk);
  char* p = static_cast<char*>(ws);
  RouteWs r;
  r.hist = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * bins * chunks);
  r.dst2src = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * n);
  r.total = reinterpret_cast<int32_t*>(p);
  p += 256;
  r.bintot = reinterpret_cast<int32_t*>(p);
  return r;
}

inline size_t route_ws_bytes(int64_t n, int64_t bins) {
  const int64_t chunks = cdiv(n, kChunk);
  return align256(sizeof(int32_t) * bins * chunks) + align256(sizeof(int32_t) * n) + 256 +
         align256(sizeof(int32_t) * bins);
}

// K1: per-chunk histogram over experts in [e0, e0 + bins).
__global__ __launch_bounds__(kChunk) void route_hist_kernel(const int32_t* __restrict__ eidx, int64_t n,
                                                            int e0, int bins, int32_t* __restrict__ hist) {
  extern __shared__ int32_t h[];
  const int64_t chunks = gridDim.x;
  for (int b = threadIdx.x; b < bins; b += blockDim.x) h[b] = 0;
  __syncthreads();
  const int64_t p = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
  if (p < n) {
    const int e = eidx[p] - e0;
    if (e >= 0 && e < bins) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < bins; b += blockDim.x) hist[static_cast<int64_t>(b) * chunks + blockIdx.x] = h[b];
}

// K2: one wave per expert. Turns the expert's row of chunk counts into exclusive in-expert offsets
// (lanes walk the chunks, 64 at a time, all loads of a row issued before the scan) and writes the
// expert's total. The cross-expert base is added by K3, so no single-workgroup pass sits on the
// critical path.
__global__ __launch_bounds__(64) void route_bin_scan_kernel(int32_t* __restrict__ hist, int64_t chunks,
                                                            int32_t* __restrict__ bintot) {
  const int lane = threadIdx.x;
  int32_t* hb = hist + static_cast<int64_t>(blockIdx.x) * chunks;
  int32_t carry = 0;
  for (int64_t c0 = 0; c0 < chunks; c0 += 256) {
    int32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = c0 + 64 * j + lane;
      v[j] = c < chunks ? hb[c] : 0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t c = c0 + 64 * j + lane;
      int32_t x = v[j];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t u = __shfl_up(x, o, 64);
        if (lane >= o) x += u;
      }
      if (c < chunks) hb[c] = carry + x - v[j];
      carry += __shfl(x, 63, 64);
    }
  }
  if (lane == 0) bintot[blockIdx.x] = carry;
}

// K3: stable in-chunk rank -> destination row of every slot.
// mode 0 (v2, row_idx_type 0): row_idx[p] = dst or -1.
// mode 1 (v2, row_idx_type 1): row_idx[dst] = p (tail filled by the gather kernel).
// mode 2 (legacy): row_idx[legacy_row[p]] = dst; eout[dst] = expert.
__global__ __launch_bounds__(kChunk) void route_place_kernel(const int32_t* __restrict__ eidx, int64_t n, int e0,
                                                             int bins, const int32_t* __restrict__ hist,
                                                             const int32_t* __restrict__ bintot,
                                                             int64_t* __restrict__ tokens, int tokens_cumsum,
                                                             int32_t* __restrict__ total,
                                                             int32_t* __restrict__ dst2src, int mode,
                                                             int32_t* __restrict__ row_idx,
                                                             const int32_t* __restrict__ legacy_row,
                                                             int32_t* __restrict__ eout) {
  __shared__ __align__(16) int32_t se[kChunk];
  __shared__ int32_t base[1024];
  __shared__ int32_t red[kChunk / 64];
  const int64_t chunks = gridDim.x;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
  int e = -1;
  if (p < n) {
    e = eidx[p] - e0;
    if (e < 0 || e >= bins) e = -1;
  }
  se[threadIdx.x] = e;
  // Exclusive scan of the per-expert totals (bins <= 1024: four per thread, in expert order).
  int32_t t4[4], s4 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = 4 * static_cast<int>(threadIdx.x) + j;
    t4[j] = b < bins ? bintot[b] : 0;
    s4 += t4[j];
  }
  const int32_t incl = block_incl_scan<false>(s4, red);
  int32_t run = incl - s4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b = 4 * static_cast<int>(threadIdx.x) + j;
    if (b < bins) {
      base[b] = run;
      if (blockIdx.x == 0 && tokens) tokens[b] = tokens_cumsum ? static_cast<int64_t>(run + t4[j]) : t4[j];
    }
    run += t4[j];
  }
  if (blockIdx.x == 0 && threadIdx.x == kChunk - 1) *total = incl;
  __syncthreads();
  if (p >= n) return;
  if (e < 0) {
    if (mode == 0) row_idx[p] = -1;
    return;
  }
  // Stable rank among the chunk's earlier slots of the same expert.
  int rank = 0;
  const int me = static_cast<int>(threadIdx.x);
  int i = 0;
  for (; i + 4 <= me; i += 4) {
    const int4 q = *reinterpret_cast<const int4*>(se + i);
    rank += (q.x == e) + (q.y == e) + (q.z == e) + (q.w == e);
  }
  for (; i < me; ++i) rank += (se[i] == e);
  const int32_t dst = base[e] + hist[static_cast<int64_t>(e) * chunks + blockIdx.x] + rank;
  dst2src[dst] = static_cast<int32_t>(p);
  if (mode == 0) row_idx[p] = dst;
  else if (mode == 1) row_idx[dst] = static_cast<int32_t>(p);
  else {
    row_idx[legacy_row[p]] = dst;
    eout[dst] = e + e0;
  }
}

// K4: expanded_x[i] = x[src(i) / k] (legacy: x[legacy_row[src] % t]); one wave per row.
__global__ __launch_bounds__(256) void route_gather_kernel(const void* __restrict__ x, int64_t row_bytes, int64_t t, int k,
                                                           const int32_t* __restrict__ dst2src, const int32_t* __restrict__ total,
                                                           int64_t active_rows, int64_t n, void* __restrict__ ex,
                                                           const float* __restrict__ scale, float* __restrict__ escale,
                                                           int tail_mode, int32_t* __restrict__ row_idx,
                                                           const int32_t* __restrict__ legacy_row) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (i >= n) return;
  const int32_t valid = *total;
  if (tail_mode == 1 && i >= valid && lane == 0) row_idx[i] = -1;
  if (i >= active_rows) return;
  char* dst = static_cast<char*>(ex) + i * row_bytes;
  if (i >= valid) {  // rows past the routed total are zero
    if ((row_bytes & 15) == 0) {
      for (int64_t o = lane * 16; o < row_bytes; o += 64 * 16) *reinterpret_cast<uint4*>(dst + o) = make_uint4(0, 0, 0, 0);
    } else {
      for (int64_t o = lane; o < row_bytes; o += 64) dst[o] = 0;
    }
    if (escale && lane == 0) escale[i] = 0.0f;
    return;
  }
  const int32_t p = dst2src[i];
  const int64_t src_row = legacy_row ? static_cast<int64_t>(legacy_row[p]) % t : p / k;
  const char* src = static_cast<const char*>(x) + src_row * row_bytes;
  if ((row_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(ex)) & 15) == 0) {
    // Four 16-byte loads in flight per lane before their stores.
    for (int64_t o = lane * 16; o < row_bytes; o += 4 * 64 * 16) {
      uint4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (o + j * 1024 < row_bytes) v[j] = *reinterpret_cast<const uint4*>(src + o + j * 1024);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (o + j * 1024 < row_bytes) *reinterpret_cast<uint4*>(dst + o + j * 1024) = v[j];
    }
  } else {
    for (int64_t o = lane; o < row_bytes; o += 64) dst[o] = src[o];
  }
  if (escale && lane == 0) escale[i] = scale[src_row];
}

// K4 without the copy: a_rows[i] = the token row of expanded row i (0 past the routed total), for a
// GEMM that gathers its rows itself; the scale is gathered as by route_gather_kernel.
__global__ __launch_bounds__(256) void route_rows_kernel(int k, const int32_t* __restrict__ dst2src,
                                                         const int32_t* __restrict__ total, int64_t active_rows,
                                                         int64_t n, int32_t* __restrict__ a_rows,
                                                         const float* __restrict__ scale, float* __restrict__ escale,
                                                         int tail_mode, int32_t* __restrict__ row_idx) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t valid = *total;
  if (tail_mode == 1 && i >= valid) row_idx[i] = -1;
  if (i >= active_rows) return;
  const int32_t src = i < valid ? dst2src[i] / k : 0;
  a_rows[i] = src;
  if (escale) escale[i] = i < valid ? scale[src] : 0.0f;
}

// ---------------------------------------------------------------------------- drop-pad routing
// npu_moe_init_routing_v2 with drop_pad_mode 1: expert e (of the range) owns rows [e * cap, (e + 1) * cap)
// of expanded_x; a slot's rank among its expert's slots (the dropless order: stable by slot) places it
// at e * cap + rank, and slots of rank >= cap are dropped (row index -1). Rows no slot fills are zero.
__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = v;
}

// dropless destination of slot p (row_idx[p], from route_place_kernel mode 0) -> padded position;
// one thread per slot; the per-expert bases are the exclusive scan of the expert totals (bins <= 1024)
__global__ __launch_bounds__(1024) void route_droppad_kernel(const int32_t* __restrict__ eidx, int64_t n, int e0,
                                                             int bins, const int32_t* __restrict__ bintot, int64_t cap,
                                                             int32_t* __restrict__ row_idx,
                                                             int32_t* __restrict__ pad2src) {
  __shared__ int32_t base[1024];
  __shared__ int32_t red[16];
  const int b = threadIdx.x;
  const int32_t v = b < bins ? bintot[b] : 0;
  const int32_t incl = block_incl_scan<false>(v, red);
  if (b < bins) base[b] = incl - v;
  __syncthreads();
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * 1024 + threadIdx.x; p < n; p += static_cast<int64_t>(gridDim.x) * 1024) {
    const int32_t d = row_idx[p];
    if (d < 0) continue;
    const int e = eidx[p] - e0;
    const int64_t rank = d - base[e];
    if (rank < cap) {
      const int64_t q = static_cast<int64_t>(e) * cap + rank;
      row_idx[p] = static_cast<int32_t>(q);
      pad2src[q] = static_cast<int32_t>(p);
    } else {
      row_idx[p] = -1;
    }
  }
}

// expanded_x[q] = x[pad2src[q] / k] or zeros; one wave per padded row
__global__ __launch_bounds__(256) void route_pad_gather_kernel(const void* __restrict__ x, int64_t row_bytes, int k,
                                                               const int32_t* __restrict__ pad2src, int64_t rows,
                                                               void* __restrict__ ex, const float* __restrict__ scale,
                                                               float* __restrict__ escale) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (q >= rows) return;
  const int32_t p = pad2src[q];
  char* dst = static_cast<char*>(ex) + q * row_bytes;
  const char* src = p >= 0 ? static_cast<const char*>(x) + static_cast<int64_t>(p / k) * row_bytes : nullptr;
  for (int64_t o = lane; o < row_bytes; o += 64) dst[o] = src ? src[o] : char(0);
  if (escale && lane == 0) escale[q] = p >= 0 ? scale[p / k] : 0.0f;
}

__global__ __launch_bounds__(1024) void route_zero_tokens_kernel(int64_t* __restrict__ tokens, int bins) {
  for (int b = threadIdx.x; b < bins; b += 1024) tokens[b] = 0;
}

// ============================================================================ finalize
struct FinArgs {
  const void* ex;
  int dt;
  int64_t t, h;
  int k;
  const void* skip1;
  const void* skip2;
  const void* bias;
  const void* scales;
  int scales_dt;
  const int32_t* s2d;
  const int32_t* expert;
  int mode;
  void* y;
};

template <bool NT = false>
__device__ __forceinline__ void load8_bf16(const void* base, int64_t off, float (&v)[8]) {
  const uint16_t* p = static_cast<const uint16_t*>(base) + off;
  uint4 r = NT ? load_nt_u4(p) : *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
    v[2 * i + 1] = bf16_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

// bf16 rows, h % 8 == 0: 16-byte loads.
__global__ __launch_bounds__(256) void finalize_bf16_kernel(FinArgs a) {
  const int64_t t = blockIdx.x;
  __shared__ int32_t s_dst[64];
  __shared__ int32_t s_exp[64];
  __shared__ float s_w[64];
  if (threadIdx.x < a.k) {
    const int j = threadIdx.x;
    const int64_t p = a.mode == 0 ? static_cast<int64_t>(j) * a.t + t : t * a.k + j;
    s_dst[j] = a.s2d[p];
    s_exp[j] = a.expert ? a.expert[t * a.k + j] : 0;
    s_w[j] = a.scales ? load_as_f32(a.scales, a.scales_dt, t * a.k + j) : 1.0f;
  }
  __syncthreads();
  const int64_t h8 = a.h / 8;
  for (int64_t c = threadIdx.x; c < h8; c += blockDim.x) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float v[8];
    if (a.skip1) {
      load8_bf16(a.skip1, t * a.h + 8 * c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = v[e];
    }
    if (a.skip2) {
      load8_bf16(a.skip2, t * a.h + 8 * c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] + v[e];
    }
    for (int j = 0; j < a.k; ++j) {
      const int32_t d = s_dst[j];
      if (d < 0) continue;
      load8_bf16<true>(a.ex, static_cast<int64_t>(d) * a.h + 8 * c, v);  // each expanded row is read once
      if (a.bias) {
        float b[8];
        load8_bf16(a.bias, static_cast<int64_t>(s_exp[j]) * a.h + 8 * c, b);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = v[e] + b[e];
      }
      const float wgt = s_w[j];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] + wgt * v[e];
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = static_cast<uint32_t>(f32_to_bf16(acc[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(acc[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.y) + t * a.h + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ __launch_bounds__(256) void finalize_generic_kernel(FinArgs a) {
  const int64_t t = blockIdx.x;
  for (int64_t c = threadIdx.x; c < a.h; c += blockDim.x) {
    float acc = 0.0f;
    if (a.skip1) acc = load_as_f32(a.skip1, a.dt, t * a.h + c);
    if (a.skip2) acc = acc + load_as_f32(a.skip2, a.dt, t * a.h + c);
    for (int j = 0; j < a.k; ++j) {
      const int64_t p = a.mode == 0 ? static_cast<int64_t>(j) * a.t + t : t * a.k + j;
      const int32_t d = a.s2d[p];
      if (d < 0) continue;
      float v = load_as_f32(a.ex, a.dt, static_cast<int64_t>(d) * a.h + c);
      if (a.bias) v = v + load_as_f32(a.bias, a.dt, static_cast<int64_t>(a.expert[t * a.k + j]) * a.h + c);
      const float wgt = a.scales ? load_as_f32(a.scales, a.scales_dt, t * a.k + j) : 1.0f;
      acc = acc + wgt * v;
    }
    store_from_f32(a.y, a.dt, t * a.h + c, acc);
  }
}

}  // namespace
}  // namespace tai

using namespace tai;

extern "C" int tai_moe_gating_top_k(const void* x, int x_dtype, int64_t t, int64_t e, int k,
                                    const void* bias, int bias_dtype, int k_group, int group_count,
                                    int group_select_mode, int renorm, int norm_type, int out_flag,
                                    float routed_scaling_factor, float eps, void* y,
                                    int32_t* expert_idx, float* out, void* stream) {
  TAI_CHECK_ARG(t >= 0 && e > 0 && e <= kMaxExperts, "tai_moe_gating_top_k: expert count must be in [1, %d]", kMaxExperts);
  TAI_CHECK_ARG(k > 0 && k <= e && k <= 32, "tai_moe_gating_top_k: k must be in [1, min(E, 32)]");
  TAI_CHECK_ARG(group_count >= 1 && group_count <= kMaxGroups && e % group_count == 0,
                "tai_moe_gating_top_k: group_count must divide E and be <= %d", kMaxGroups);
  TAI_CHECK_ARG(k_group >= 1 && k_group <= group_count, "tai_moe_gating_top_k: k_group must be in [1, group_count]");
  TAI_CHECK_ARG(k <= k_group * (e / group_count), "tai_moe_gating_top_k: k exceeds the experts in the kept groups");
  TAI_CHECK_ARG(group_select_mode == 0 || group_select_mode == 1, "tai_moe_gating_top_k: group_select_mode must be 0 or 1");
  TAI_CHECK_ARG(norm_type == 0 || norm_type == 1, "tai_moe_gating_top_k: norm_type must be 0 (softmax) or 1 (sigmoid)");
  TAI_UNSUPPORTED(renorm != 0, "tai_moe_gating_top_k: only renorm=0 (norm before top-k) is supported");
  TAI_CHECK_ARG(x_dtype == TAI_DT_FP32 || x_dtype == TAI_DT_BF16 || x_dtype == TAI_DT_FP16, "tai_moe_gating_top_k: x dtype");
  if (t == 0) return TAI_OK;
  TAI_CHECK_ARG(x && y && expert_idx, "tai_moe_gating_top_k: null pointer");
  GateArgs a{x, x_dtype, t, e, k, bias, bias_dtype, k_group, group_count, group_select_mode, norm_type,
             out_flag, routed_scaling_factor, eps, y, expert_idx, out};
  const bool fast = e == 256 && norm_type == 1 && (group_count == 1 || group_count == 8);
  if (fast)
    gating_topk_256_kernel<<<dim3(static_cast<unsigned>(cdiv(t, 4))), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  else
    gating_topk_kernel<<<dim3(static_cast<unsigned>(cdiv(t, 4))), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("tai_moe_gating_top_k");
}

extern "C" size_t tai_moe_init_routing_workspace_size(int64_t t, int k, int64_t num_experts) {
  return route_ws_bytes(t * k, num_experts);
}

namespace tai {
static int run_routing(const void* x, int elem_bytes, int64_t t, int64_t h, const int32_t* eidx, int k,
                       int e0, int bins, int64_t active_rows, int mode, int32_t* row_idx,
                       const int32_t* legacy_row, int32_t* eout, int64_t* tokens, int tokens_cumsum,
                       const float* scale, float* escale, void* ex, void* ws, size_t ws_bytes,
                       hipStream_t st, const char* name, int32_t* a_rows = nullptr) {
  const int64_t n = t * k;
  TAI_CHECK_ARG(n < (1ll << 31), "%s: t*k must be < 2^31", name);
  TAI_CHECK_ARG(bins >= 1 && bins <= 1024, "%s: expert range must hold 1..1024 experts", name);
  if (ws_bytes < route_ws_bytes(n, bins) || ws == nullptr) {
    set_error("%s: workspace of %zu bytes, need %zu", name, ws_bytes, route_ws_bytes(n, bins));
    return TAI_ERR_WORKSPACE;
  }
  RouteWs w = carve_route_ws(ws, n, bins);
  const int64_t chunks = cdiv(n, kChunk);
  TAI_CHECK_ARG(chunks < (1ll << 31), "%s: too many slots", name);
  if (n == 0) return TAI_OK;
  route_hist_kernel<<<dim3(static_cast<unsigned>(chunks)), kChunk, sizeof(int32_t) * bins, st>>>(eidx, n, e0, bins, w.hist);
  route_bin_scan_kernel<<<dim3(static_cast<unsigned>(bins)), 64, 0, st>>>(w.hist, chunks, w.bintot);
  route_place_kernel<<<dim3(static_cast<unsigned>(chunks)), kChunk, 0, st>>>(eidx, n, e0, bins, w.hist, w.bintot,
                                                                          tokens, tokens_cumsum, w.total, w.dst2src,
                                                                          mode, row_idx, legacy_row, eout);
  const int tail_mode = (mode == 1) ? 1 : 0;
  if (a_rows) {
    route_rows_kernel<<<dim3(static_cast<unsigned>(cdiv(n, 256))), 256, 0, st>>>(
        k, w.dst2src, w.total, active_rows, n, a_rows, scale, escale, tail_mode, row_idx);
    return launch_status(name);
  }
  route_gather_kernel<<<dim3(static_cast<unsigned>(cdiv(n, 4))), 256, 0, st>>>(
      x, static_cast<int64_t>(elem_bytes) * h, t, k, w.dst2src, w.total, active_rows, n, ex, scale, escale,
      tail_mode, row_idx, legacy_row);
  return launch_status(name);
}
}  // namespace tai

extern "C" int tai_moe_init_routing_v2(const void* x, int elem_bytes, int64_t t, int64_t h,
                                       const int32_t* expert_idx, int k, const float* scale,
                                       int64_t active_rows, int expert_start, int expert_end,
                                       int expert_tokens_num_type, int row_idx_type, void* expanded_x,
                                       int32_t* expanded_row_idx, int64_t* expert_tokens,
                                       float* expanded_scale, void* workspace, size_t ws_bytes,
                                       void* stream) {
  TAI_CHECK_ARG(t >= 0 && h >= 0 && k > 0, "tai_moe_init_routing_v2: bad sizes");
  TAI_CHECK_ARG(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4, "tai_moe_init_routing_v2: elem_bytes");
  TAI_CHECK_ARG(expert_start >= 0 && expert_end > expert_start, "tai_moe_init_routing_v2: expert range");
  TAI_CHECK_ARG(row_idx_type == 0 || row_idx_type == 1, "tai_moe_init_routing_v2: row_idx_type must be 0 or 1");
  TAI_CHECK_ARG(expert_tokens_num_type == 0 || expert_tokens_num_type == 1,
                "tai_moe_init_routing_v2: expert_tokens_num_type must be 0 (cumsum) or 1 (count)");
  TAI_CHECK_ARG(active_rows >= 0 && active_rows <= t * k, "tai_moe_init_routing_v2: active rows");
  TAI_CHECK_ARG(scale == nullptr || expanded_scale != nullptr, "tai_moe_init_routing_v2: expanded_scale missing");
  return run_routing(x, elem_bytes, t, h, expert_idx, k, expert_start, expert_end - expert_start, active_rows,
                     row_idx_type, expanded_row_idx, nullptr, nullptr, expert_tokens, expert_tokens_num_type == 0,
                     scale, expanded_scale, expanded_x, workspace, ws_bytes, static_cast<hipStream_t>(stream),
                     "tai_moe_init_routing_v2");
}

extern "C" int tai_moe_init_routing_v2_rows(int64_t t, const int32_t* expert_idx, int k, const float* scale,
                                            int64_t active_rows, int expert_start, int expert_end,
                                            int expert_tokens_num_type, int row_idx_type, int32_t* a_rows,
                                            int32_t* expanded_row_idx, int64_t* expert_tokens,
                                            float* expanded_scale, void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(t >= 0 && k > 0, "tai_moe_init_routing_v2_rows: bad sizes");
  TAI_CHECK_ARG(expert_start >= 0 && expert_end > expert_start, "tai_moe_init_routing_v2_rows: expert range");
  TAI_CHECK_ARG(row_idx_type == 0 || row_idx_type == 1, "tai_moe_init_routing_v2_rows: row_idx_type must be 0 or 1");
  TAI_CHECK_ARG(expert_tokens_num_type == 0 || expert_tokens_num_type == 1,
                "tai_moe_init_routing_v2_rows: expert_tokens_num_type must be 0 (cumsum) or 1 (count)");
  TAI_CHECK_ARG(active_rows >= 0 && active_rows <= t * k, "tai_moe_init_routing_v2_rows: active rows");
  TAI_CHECK_ARG(scale == nullptr || expanded_scale != nullptr, "tai_moe_init_routing_v2_rows: expanded_scale missing");
  TAI_CHECK_ARG(t == 0 || a_rows != nullptr, "tai_moe_init_routing_v2_rows: a_rows is required");
  return run_routing(nullptr, 1, t, 0, expert_idx, k, expert_start, expert_end - expert_start, active_rows,
                     row_idx_type, expanded_row_idx, nullptr, nullptr, expert_tokens, expert_tokens_num_type == 0,
                     scale, expanded_scale, nullptr, workspace, ws_bytes, static_cast<hipStream_t>(stream),
                     "tai_moe_init_routing_v2_rows", a_rows);
}

extern "C" size_t tai_moe_init_routing_v2_droppad_workspace_size(int64_t t, int k, int64_t num_experts,
                                                                 int64_t capacity) {
  return route_ws_bytes(t * k, num_experts) + align256(sizeof(int32_t) * num_experts * capacity);
}

extern "C" int tai_moe_init_routing_v2_droppad(const void* x, int elem_bytes, int64_t t, int64_t h,
                                               const int32_t* expert_idx, int k, const float* scale,
                                               int64_t capacity, int expert_start, int expert_end,
                                               int expert_tokens_num_type, void* expanded_x,
                                               int32_t* expanded_row_idx, int64_t* expert_tokens,
                                               float* expanded_scale, void* workspace, size_t ws_bytes,
                                               void* stream) {
  const char* name = "tai_moe_init_routing_v2_droppad";
  TAI_CHECK_ARG(t >= 0 && h >= 0 && k > 0 && capacity > 0, "%s: bad sizes (capacity must be > 0)", name);
  TAI_CHECK_ARG(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4, "%s: elem_bytes", name);
  TAI_CHECK_ARG(expert_start >= 0 && expert_end > expert_start && expert_end - expert_start <= 1024,
                "%s: expert range must hold 1..1024 experts", name);
  TAI_CHECK_ARG(expert_tokens_num_type == 0 || expert_tokens_num_type == 1,
                "%s: expert_tokens_num_type must be 0 (cumsum) or 1 (count)", name);
  TAI_CHECK_ARG(scale == nullptr || expanded_scale != nullptr, "%s: expanded_scale missing", name);
  const int bins = expert_end - expert_start;
  const int64_t rows = static_cast<int64_t>(bins) * capacity;
  TAI_CHECK_ARG(rows < (1ll << 31), "%s: experts * capacity must be < 2^31", name);
  const size_t need = tai_moe_init_routing_v2_droppad_workspace_size(t, k, bins, capacity);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("%s: workspace of %zu bytes, need %zu", name, ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = t * k;
  TAI_CHECK_ARG(n < (1ll << 31), "%s: t*k must be < 2^31", name);
  const size_t rws = route_ws_bytes(n, bins);
  int32_t* pad2src = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + rws);
  fill_i32_kernel<<<dim3(static_cast<unsigned>(std::min<int64_t>(cdiv(rows, 256), 4096))), 256, 0, st>>>(pad2src, rows, -1);
  if (n > 0) {
    RouteWs w = carve_route_ws(workspace, n, bins);
    const int64_t chunks = cdiv(n, kChunk);
    route_hist_kernel<<<dim3(static_cast<unsigned>(chunks)), kChunk, sizeof(int32_t) * bins, st>>>(expert_idx, n,
                                                                                                 expert_start, bins,
                                                                                                 w.hist);
    route_bin_scan_kernel<<<dim3(static_cast<unsigned>(bins)), 64, 0, st>>>(w.hist, chunks, w.bintot);
    route_place_kernel<<<dim3(static_cast<unsigned>(chunks)), kChunk, 0, st>>>(
        expert_idx, n, expert_start, bins, w.hist, w.bintot, expert_tokens, expert_tokens_num_type == 0, w.total,
        w.dst2src, 0, expanded_row_idx, nullptr, nullptr);
    route_droppad_kernel<<<dim3(static_cast<unsigned>(std::min<int64_t>(cdiv(n, 1024), 1024))), 1024, 0, st>>>(
        expert_idx, n, expert_start, bins, w.bintot, capacity, expanded_row_idx, pad2src);
  } else if (expert_tokens) {
    // no slots: every expert count (and cumsum) is 0
    route_zero_tokens_kernel<<<1, 1024, 0, st>>>(expert_tokens, bins);
  }
  if (rows > 0 && h > 0)
    route_pad_gather_kernel<<<dim3(static_cast<unsigned>(cdiv(rows, 4))), 256, 0, st>>>(
        x, static_cast<int64_t>(elem_bytes) * h, k, pad2src, rows, expanded_x, scale, expanded_scale);
  return launch_status(name);
}

extern "C" int tai_moe_init_routing(const void* x, int elem_bytes, int64_t t, int64_t h,
                                    const int32_t* row_idx, const int32_t* expert_idx, int k,
                                    int64_t num_experts, int64_t active_rows, void* expanded_x,
                                    int32_t* expanded_row_idx, int32_t* expanded_expert_idx,
                                    void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(t >= 0 && h >= 0 && k > 0, "tai_moe_init_routing: bad sizes");
  TAI_CHECK_ARG(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4, "tai_moe_init_routing: elem_bytes");
  TAI_CHECK_ARG(active_rows >= 0 && active_rows <= t * k, "tai_moe_init_routing: active rows");
  TAI_CHECK_ARG(row_idx && expanded_row_idx && expanded_expert_idx, "tai_moe_init_routing: null pointer");
  return run_routing(x, elem_bytes, t, h, expert_idx, k, 0, static_cast<int>(num_experts), active_rows, 2,
                     expanded_row_idx, row_idx, expanded_expert_idx, nullptr, 0, nullptr, nullptr, expanded_x,
                     workspace, ws_bytes, static_cast<hipStream_t>(stream), "tai_moe_init_routing");
}

extern "C" int tai_moe_finalize_routing(const void* expanded, int dtype, int64_t t, int64_t h, int k,
                                        const void* skip1, const void* skip2, const void* bias,
                                        const void* scales, int scales_dtype, const int32_t* src_to_dst,
                                        const int32_t* expert_for_source_row, int drop_pad_mode, void* y,
                                        void* stream) {
  TAI_CHECK_ARG(t >= 0 && h >= 0 && k > 0 && k <= 64, "tai_moe_finalize_routing: k must be in [1, 64]");
  TAI_UNSUPPORTED(drop_pad_mode != 0 && drop_pad_mode != 2,
                  "tai_moe_finalize_routing: drop_pad_mode %d (drop-pad) not supported; use 0 or 2", drop_pad_mode);
  TAI_CHECK_ARG(dtype == TAI_DT_BF16 || dtype == TAI_DT_FP16 || dtype == TAI_DT_FP32, "tai_moe_finalize_routing: dtype");
  TAI_CHECK_ARG(bias == nullptr || expert_for_source_row != nullptr,
                "tai_moe_finalize_routing: bias needs expert_for_source_row");
  if (t == 0 || h == 0) return TAI_OK;
  TAI_CHECK_ARG(expanded && src_to_dst && y, "tai_moe_finalize_routing: null pointer");
  FinArgs a{expanded, dtype, t, h, k, skip1, skip2, bias, scales, scales_dtype, src_to_dst, expert_for_source_row,
            drop_pad_mode == 0 ? 0 : 2, y};
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % 16) == 0; };
  if (dtype == TAI_DT_BF16 && h % 8 == 0 && al(expanded) && al(skip1) && al(skip2) && al(bias) && al(y))
    finalize_bf16_kernel<<<dim3(static_cast<unsigned>(t)), 256, 0, st>>>(a);
  else
    finalize_generic_kernel<<<dim3(static_cast<unsigned>(t)), 256, 0, st>>>(a);
  return launch_status("tai_moe_finalize_routing");
}

// ============================================================================ grouped_matmul_finalize_routing
// The W8A8 grouped GEMM writes its dequantised rows (fp32, so the combine adds no rounding of its
// own) to a scratch buffer; each output token
// then gathers the rows r with row_index[r] == token, in ascending r, as
//   y[token] = sum_r logit[r] * row[r]  (+ shared_input_weight * shared_input[token - offset]).
// The token -> rows lists come from a histogram, a scan and an atomic placement; the gather
// sorts each list, so the fp32 sum has a fixed order and the result is reproducible.
namespace tai {
namespace {

constexpr int kGfrMaxRows = 1024;  // rows one token may gather

__global__ __launch_bounds__(256) void gfr_fill_kernel(int32_t* __restrict__ p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = 0;
}

__global__ __launch_bounds__(256) void gfr_hist_kernel(const void* __restrict__ row_index, int idx_dt, int64_t m,
                                                       int64_t bs, int32_t* __restrict__ counts) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= m) return;
  const int64_t t = row_index ? load_index(row_index, idx_dt, r) : r;
  if (t >= 0 && t < bs) atomicAdd(&counts[t], 1);
}

// One workgroup: exclusive offsets of the per-token counts, 1024 tokens per pass.
__global__ __launch_bounds__(1024) void gfr_scan_kernel(const int32_t* __restrict__ counts, int64_t bs,
                                                        int32_t* __restrict__ offs) {
  __shared__ int32_t red[16];
  __shared__ int32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int64_t b0 = 0; b0 < bs; b0 += 1024) {
    const int64_t i = b0 + threadIdx.x;
    const int32_t v = i < bs ? counts[i] : 0;
    const int32_t incl = block_incl_scan<false>(v, red);
    const int32_t base = carry;
    if (i < bs) offs[i] = base + incl - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry = base + incl;
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void gfr_place_kernel(const void* __restrict__ row_index, int idx_dt, int64_t m,
                                                        int64_t bs, const int32_t* __restrict__ offs,
                                                        int32_t* __restrict__ cursor, int32_t* __restrict__ list) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= m) return;
  const int64_t t = row_index ? load_index(row_index, idx_dt, r) : r;
  if (t >= 0 && t < bs) list[offs[t] + atomicAdd(&cursor[t], 1)] = static_cast<int32_t>(r);
}

struct GfrArgs {
  const float* rows;     // [m, n] fp32 dequantised GEMM rows
  const float* logit;    // [m] or null (1)
  const int32_t* counts;
  const int32_t* offs;
  const int32_t* list;
  const uint16_t* shared;  // [shared_rows, n] bf16 or null
  int64_t shared_rows, shared_offset;
  float shared_weight;
  int64_t n;
  float* y;  // [bs, n] fp32
};

// One workgroup per output token.
__global__ __launch_bounds__(256) void gfr_gather_kernel(GfrArgs a) {
  __shared__ int32_t s_in[kGfrMaxRows];
  __shared__ int32_t s_sorted[kGfrMaxRows];
  __shared__ float s_w[kGfrMaxRows];
  const int64_t t = blockIdx.x;
  const int cnt = a.counts[t];
  float* yrow = a.y + t * a.n;
  if (cnt > kGfrMaxRows) {  // outside the supported range: make it loud
    for (int64_t c = threadIdx.x; c < a.n; c += 256) yrow[c] = __builtin_nanf("");
    return;
  }
  const int32_t* lst = a.list + a.offs[t];
  for (int i = threadIdx.x; i < cnt; i += 256) s_in[i] = lst[i];
  __syncthreads();
  for (int i = threadIdx.x; i < cnt; i += 256) {  // rank sort: rows are distinct
    const int32_t v = s_in[i];
    int rank = 0;
    for (int j = 0; j < cnt; ++j) rank += s_in[j] < v;
    s_sorted[rank] = v;
    s_w[rank] = a.logit ? a.logit[v] : 1.0f;
  }
  __syncthreads();
  const bool sh = a.shared && t >= a.shared_offset && t < a.shared_offset + a.shared_rows;
  const int64_t n8 = a.n / 8;
  for (int64_t c = threadIdx.x; c < n8; c += 256) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < cnt; ++i) {
      const float4* src = reinterpret_cast<const float4*>(a.rows + static_cast<int64_t>(s_sorted[i]) * a.n + 8 * c);
      const float4 lo = src[0], hi = src[1];
      const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      const float wgt = s_w[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] + wgt * v[e];
    }
    if (sh) {
      float v[8];
      load8_bf16(a.shared, (t - a.shared_offset) * a.n + 8 * c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = acc[e] + a.shared_weight * v[e];
    }
    float4* dst = reinterpret_cast<float4*>(yrow + 8 * c);
    dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

}  // namespace
}  // namespace tai

static size_t gfr_parts(int64_t m, int64_t n, int64_t num_groups, int64_t bs, size_t* rows_off, size_t* idx_off) {
  const size_t base = align256(tai_grouped_matmul_workspace_size(m, n, num_groups));
  const size_t rows = align256(static_cast<size_t>(m) * static_cast<size_t>(n) * sizeof(float));
  if (rows_off) *rows_off = base;
  if (idx_off) *idx_off = base + rows;
  return base + rows + align256(sizeof(int32_t) * (3 * static_cast<size_t>(bs) + static_cast<size_t>(m))) + 256;
}

extern "C" size_t tai_grouped_matmul_finalize_routing_workspace_size(int64_t m, int64_t n, int64_t num_groups,
                                                                     int64_t output_bs) {
  return gfr_parts(m, n, num_groups, output_bs, nullptr, nullptr);
}

extern "C" int tai_grouped_matmul_finalize_routing(const int8_t* x, const int8_t* weight, int64_t m, int64_t k,
                                                   int64_t n, int64_t num_groups, int w_layout,
                                                   const int64_t* group_list, int group_list_type, const float* scale,
                                                   const float* pertoken_scale, const float* bias, const float* logit,
                                                   const void* row_index, int row_index_dtype, const void* shared_input,
                                                   int64_t shared_rows, float shared_input_weight,
                                                   int64_t shared_input_offset, int64_t output_bs, float* y,
                                                   void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(m >= 0 && n >= 1 && output_bs >= 0 && shared_rows >= 0, "tai_grouped_matmul_finalize_routing: bad sizes");
  TAI_CHECK_ARG(n % 8 == 0, "tai_grouped_matmul_finalize_routing: n must be a multiple of 8");
  TAI_CHECK_ARG(scale != nullptr, "tai_grouped_matmul_finalize_routing: scale is required");
  TAI_CHECK_ARG(row_index == nullptr || row_index_dtype == TAI_DT_INT32 || row_index_dtype == TAI_DT_INT64,
                "tai_grouped_matmul_finalize_routing: row_index must be int32 or int64");
  TAI_CHECK_ARG(shared_input == nullptr || (shared_input_offset >= 0 && shared_input_offset + shared_rows <= output_bs),
                "tai_grouped_matmul_finalize_routing: shared_input rows must lie inside the output");
  TAI_CHECK_ARG(m < (1ll << 31), "tai_grouped_matmul_finalize_routing: m must be < 2^31");
  if (output_bs == 0) return TAI_OK;
  TAI_CHECK_ARG(y != nullptr, "tai_grouped_matmul_finalize_routing: null output");
  size_t rows_off = 0, idx_off = 0;
  const size_t need = gfr_parts(m, n, num_groups, output_bs, &rows_off, &idx_off);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_grouped_matmul_finalize_routing: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* wsp = static_cast<char*>(workspace);
  float* rows = reinterpret_cast<float*>(wsp + rows_off);
  int32_t* counts = reinterpret_cast<int32_t*>(wsp + idx_off);
  int32_t* cursor = counts + output_bs;
  int32_t* offs = cursor + output_bs;
  int32_t* list = offs + output_bs;
  if (m > 0) {
    const int rc = tai_grouped_matmul(x, weight, m, k, n, num_groups, w_layout, group_list, group_list_type, scale,
                                      pertoken_scale, bias, bias ? TAI_DT_FP32 : TAI_DT_NONE, TAI_DT_FP32, rows,
                                      workspace, rows_off, stream);
    if (rc != TAI_OK) return rc;
  }
  gfr_fill_kernel<<<dim3(static_cast<unsigned>(cdiv(2 * output_bs, 256) < 1024 ? cdiv(2 * output_bs, 256) : 1024)), 256, 0,
                    st>>>(counts, 2 * output_bs);
  if (m > 0) {
    const dim3 grid(static_cast<unsigned>(cdiv(m, 256)));
    gfr_hist_kernel<<<grid, 256, 0, st>>>(row_index, row_index_dtype, m, output_bs, counts);
    gfr_scan_kernel<<<1, 1024, 0, st>>>(counts, output_bs, offs);
    gfr_place_kernel<<<grid, 256, 0, st>>>(row_index, row_index_dtype, m, output_bs, offs, cursor, list);
  } else {
    gfr_scan_kernel<<<1, 1024, 0, st>>>(counts, output_bs, offs);
  }
  GfrArgs a{rows, logit, counts, offs, list, static_cast<const uint16_t*>(shared_input), shared_rows,
            shared_input_offset, shared_input_weight, n, y};
  gfr_gather_kernel<<<dim3(static_cast<unsigned>(output_bs)), 256, 0, st>>>(a);
  return launch_status("tai_grouped_matmul_finalize_routing");
}

// ----------------------------------------------------------------------------- compute_expert_tokens
// out[e] = the number of entries of the ascending `sorted` that are <= e (the end of expert e's rows),
// one binary search per expert.
namespace tai {
namespace {
__global__ __launch_bounds__(256) void expert_tokens_kernel(const int32_t* __restrict__ sorted, int64_t n,
                                                            int64_t num_experts, int32_t* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= num_experts) return;
  int64_t lo = 0, hi = n;  // first index with sorted[index] > e
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (static_cast<int64_t>(sorted[mid]) <= e) lo = mid + 1; else hi = mid;
  }
  out[e] = static_cast<int32_t>(lo);
}
}  // namespace
}  // namespace tai

extern "C" int tai_moe_compute_expert_tokens(const int32_t* sorted_experts, int64_t n, int64_t num_experts,
                                             int32_t* out, void* stream) {
  TAI_CHECK_ARG(n >= 0 && n < (1ll << 31), "tai_moe_compute_expert_tokens: n must be in [0, 2^31)");
  TAI_CHECK_ARG(num_experts > 0 && num_experts < 2147483647ll,
                "tai_moe_compute_expert_tokens: num_experts must be in (0, 2^31 - 1)");
  TAI_CHECK_ARG(out && (n == 0 || sorted_experts), "tai_moe_compute_expert_tokens: null pointer");
  tai::expert_tokens_kernel<<<dim3(static_cast<unsigned>(cdiv(num_experts, 256))), 256, 0,
                              static_cast<hipStream_t>(stream)>>>(sorted_experts, n, num_experts, out);
  return launch_status("tai_moe_compute_expert_tokens");
}

