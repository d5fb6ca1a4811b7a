// npu_fused_infer_attention_score kernels: paged GQA decode, dense (causal) prefill and
// MLA absorbed decode over an int8 latent cache.
#include "common.h"

#include <algorithm>
#include <utility>

namespace tai {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// The 16-bit element of query, key, value and output: bf16 (F16 = false) or fp16 (F16 = true). The
// score and P.V MFMAs take that type on both operands, so P is rounded to it too.
template <bool F16>
struct Half;
template <>
struct Half<false> {
  using v8 = bf16x8;
  using v2 = bf16x2_t;
  static __device__ __forceinline__ f32x4 mfma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t bits(float f) { return f32_to_bf16(f); }
  static __device__ __forceinline__ v2 pack(float a, float b) { return __builtin_convertvector((f32x2_t){a, b}, v2); }
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) { return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false); }
  static constexpr float kSlack = 64.0f;  // log2 headroom of P above the fast pass's reference max
};
template <>
struct Half<true> {
  using v8 = f16x8;
  using v2 = f16x2_t;
  static __device__ __forceinline__ f32x4 mfma16(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t bits(float f) { return f32_to_f16(f); }
  static __device__ __forceinline__ v2 pack(float a, float b) { return __builtin_convertvector((f32x2_t){a, b}, v2); }
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
  static constexpr float kSlack = 8.0f;  // P <= 2^8 keeps it well inside fp16's 65504
};

__device__ __forceinline__ uint16_t bf16_bits(float f) { return f32_to_bf16(f); }

// ============================================================================ paged GQA decode
// Work: the batch's 32-token steps are cut into equal contiguous ranges; each (range, kv head) is
// one wave, which runs a segment per sequence its range touches. Per 32-token step:
//   the step's K and V rows go global -> LDS (global_load_lds, whole 256-byte rows per 16 lanes)
//   through a ring, one step ahead of their use; S^T = K Q^T with v_mfma_f32_16x16x32_bf16
//   (rows = 16 tokens, columns = the G query heads of this kv head padded to 16). S^T leaves each
//   lane with four tokens of one head, so the online softmax needs two cross-lane reductions,
//   and P^T is already the B operand of O^T = V^T P^T; V is read transposed with
//   ds_read_b64_tr_b16.
// Each segment writes an unnormalised partial (O, running max, running sum); a second kernel
// merges the partials of each (b, head) and writes bf16 output and the logsumexp.
#ifndef TAI_DECODE_VSTAGES
#define TAI_DECODE_VSTAGES 2
#endif
constexpr int kStep = 32;
// Cache policy of loads that stream data read once (the `nt` bit of gfx950's global loads). On the
// paged decode the K/V stream went from 5.07 to 5.89 TB/s with it (config 2, C-ABI harness), and
// the MLA cache stream gained 3%. The prefill's K/V tiles, which several workgroups read, lose
// 8-11% with it, and so do the GEMM operands.
constexpr int kCpolNt = 2;
constexpr int kVStages = TAI_DECODE_VSTAGES;  // K/V ring stages of one step each

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t sb, ss, sh;  // cache strides (elements): block, slot, head
  const int32_t* bt;
  int64_t max_blocks;
  const int64_t* lens;
  int64_t b;
  int hq, hkv, g;
  int bs;
  float scale_log2;  // softmax scale * log2(e)
  int nranges;     // step ranges of a launch (one wave per range and kv head)
  int64_t* steps;  // [0] = balance units of the batch, [1 + b] = units before sequence b
  const float* sink;  // NULL or [hq] fp32: learnable_sink logits, joined to each row's max and sum by the merge
  const float* vsc;   // NULL or [hkv * D] fp32: per-channel value scales the merge applies (int8 caches)
  float* part_o;   // [slot, hkv, 16, D], slot = range + sequence
  float* part_ml;  // [slot, hkv, 16, 2]
};

// A sequence length read on the device, clamped to [0, cap]: a length past the cache extent the
// block table can address (max_blocks * block_size) would otherwise index past the sequence's
// block-table row into other sequences' blocks.
__device__ __forceinline__ int64_t clamp_len(int64_t v, int64_t cap) { return v < 0 ? 0 : (v > cap ? cap : v); }
template <class A>
__device__ __forceinline__ int64_t kv_len(const A& a, int64_t b) { return clamp_len(a.lens[b], a.max_blocks * a.bs); }

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int64_t wave_incl_scan64(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <int D>
struct DecodeTile {
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kCpr = kRowBytes / 16;                 // 16-byte chunks per row
  static constexpr int kRsh = kRowBytes >= 256 ? 0 : 1;       // rows per 256-byte bank cycle = 1 << kRsh
  static constexpr int kXm = (kCpr < 16 ? kCpr : 16) - 1;     // swizzle mask
  static constexpr int kStage = kStep * kRowBytes;            // bytes of one V step
  static constexpr int kLoads = kStage / 1024;                // 1 KB global_load_lds per step
  static constexpr int kRpi = 1024 / kRowBytes;               // rows per load instruction
  __device__ static __forceinline__ int off(int row, int c) { return row * kRowBytes + 16 * (c ^ ((row >> kRsh) & kXm)); }
};

typedef __attribute__((address_space(3))) char lds_char_t;

__device__ __forceinline__ int64_t dec_steps(int64_t len) { return len > 0 ? (len + kStep - 1) / kStep : 0; }
// Balance units of a sequence: its steps plus kDecSegCost for the start of a segment (Q load, ring
// fill, partial store), so a range that starts a sequence gets that much less streaming.
#ifndef TAI_DEC_SEG_COST
#define TAI_DEC_SEG_COST 2
#endif
constexpr int kDecSegCost = TAI_DEC_SEG_COST;
__device__ __forceinline__ int64_t dec_units(int64_t len) { return len > 0 ? dec_steps(len) + kDecSegCost : 0; }

// One segment: tokens [t_begin, t_end) of sequence b for kv head kvh, written as the partial of
// the given slot.
template <int D, bool F16>
__device__ __forceinline__ void decode_segment(const DecodeArgs& a, lds_char_t* s_kv, int64_t b, int kvh, int64_t t_begin,
                                               int64_t t_end, int64_t slot) {
  using T = DecodeTile<D>;
  using H = Half<F16>;
  using hv8 = typename H::v8;
  const int lane = threadIdx.x;
  const int hcol = lane & 15, kg = lane >> 4;
  const int64_t unit = slot * a.hkv + kvh;
  float* po = a.part_o + unit * 16 * D;
  float* pml = a.part_ml + unit * 32;

  // Q^T fragments (B operand): head = hcol (padded to 16), d slots 32m + 8kg .. +8
  hv8 qf[D / 32];
  {
    const bool valid = hcol < a.g;
    const uint16_t* qh = a.q + (b * a.hq + kvh * a.g + (valid ? hcol : 0)) * D;
#pragma unroll
    for (int m = 0; m < D / 32; ++m)
      qf[m] = __builtin_bit_cast(hv8, valid ? *reinterpret_cast<const uint4*>(qh + 32 * m + 8 * kg) : make_uint4(0, 0, 0, 0));
  }
  f32x4 acc[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) acc[t] = f32x4{0, 0, 0, 0};
  float m_run = -INFINITY, l_run = 0.0f;

  const uint16_t* kbase = a.k + static_cast<int64_t>(kvh) * a.sh;
  const uint16_t* vbase = a.v + static_cast<int64_t>(kvh) * a.sh;
  const int32_t* btrow = a.bt + b * a.max_blocks;
  // A window of 64 block-table entries, one per lane, broadcast with ds_bpermute; it moves on (a
  // rare, draining load) when a step lies past it. Offsets inside the segment are 32-bit; a
  // power-of-two bs divides by shifting.
  const int bs = a.bs;
  const int bs_shift = (bs & (bs - 1)) == 0 ? __builtin_ctz(bs) : -1;
  const int64_t pg0 = t_begin / bs;
  const int off0 = static_cast<int>(t_begin - pg0 * bs);  // slot of the segment's first token
  int wb = 0;                                              // window base (pages after pg0)
  auto load_window = [&]() {
    const int64_t pg = pg0 + wb + lane;
    return pg < a.max_blocks ? btrow[pg] : 0;
  };
  int my_page = load_window();
  // A step never straddles a page (bs % 32 == 0 and steps start at multiples of 32), so one
  // lookup per step gives the element offset of the step's first token.
  auto step_base = [&](int s) -> int64_t {
    const int x = s * kStep + off0;
    const int pi = bs_shift >= 0 ? (x >> bs_shift) : x / bs;
    if (pi - wb >= 64) {
      wb = pi;
      my_page = load_window();
    }
    const int slot_in_page = x - pi * bs;
    return static_cast<int64_t>(__shfl(my_page, pi - wb, 64)) * a.sb + static_cast<int64_t>(slot_in_page) * a.ss;
  };
  const int n_local = static_cast<int>(t_end - t_begin);

  const int nsteps = static_cast<int>((t_end - t_begin + kStep - 1) / kStep);
  // K and V rows of a step both go global -> LDS ([K tile][V tile] per ring stage).
  auto issue_kv = [&](int s) __attribute__((always_inline)) {
    lds_char_t* st = s_kv + (s % kVStages) * 2 * T::kStage;
    const int64_t sbase = step_base(s);
    const int last = n_local - 1 - s * kStep;
#pragma unroll
    for (int q = 0; q < T::kLoads; ++q) {
      const int row = q * T::kRpi + lane / T::kCpr;
      const int c = (lane % T::kCpr) ^ ((row >> T::kRsh) & T::kXm);
      const int64_t o = sbase + static_cast<int64_t>(min(row, last)) * a.ss + 8 * c;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(kbase + o),
                                       (__attribute__((address_space(3))) void*)(st + q * 1024), 16, 0, kCpolNt);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(vbase + o),
                                       (__attribute__((address_space(3))) void*)(st + T::kStage + q * 1024), 16, 0, kCpolNt);
    }
  };
  constexpr int kAhead = kVStages - 1;
#pragma unroll
  for (int i = 0; i < kAhead; ++i)
    if (i < nsteps) issue_kv(i);
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_kv));
  for (int s = 0; s < nsteps; ++s) {
    if (s + kAhead < nsteps) issue_kv(s + kAhead);
    {
      const int after = min(kAhead, nsteps - 1 - s);  // steps issued after this one
      if (after >= 2) __builtin_amdgcn_s_waitcnt(((4 * T::kLoads) & 0xF) | (((4 * T::kLoads) >> 4) << 14) | 0x70 | 0xF00);
      else if (after == 1) __builtin_amdgcn_s_waitcnt(((2 * T::kLoads) & 0xF) | (((2 * T::kLoads) >> 4) << 14) | 0x70 | 0xF00);
      else __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);
    }
    const int64_t t0 = t_begin + static_cast<int64_t>(s) * kStep;
    const uint32_t kst = lds0 + (s % kVStages) * 2 * T::kStage;
    const uint32_t vst = kst + T::kStage;
    v4i_t kcur[2][D / 32];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int m = 0; m < D / 32; ++m)
        asm volatile("ds_read_b128 %0, %1" : "=v"(kcur[tb][m]) : "v"(kst + T::off(16 * tb + hcol, 4 * m + kg)));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int m = 0; m < D / 32; ++m) asm volatile("" : "+v"(kcur[tb][m]));
    // ---- S^T = K Q^T for two 16-token blocks: lane holds tokens 16tb + 4kg + r of head hcol
    f32x4 sc[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      sc[tb] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int m = 0; m < D / 32; ++m)
        sc[tb] = H::mfma16(__builtin_bit_cast(hv8, kcur[tb][m]), qf[m], sc[tb]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = t0 + 16 * tb + 4 * kg + r < t_end;
        const float v = ok ? sc[tb][r] * a.scale_log2 : -INFINITY;
        sc[tb][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);  // finite: every step holds at least one valid token
    const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float rs = 0.0f;
    hv8 pf;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const float e0 = __builtin_amdgcn_exp2f(sc[tb][r] - m_new);
        const float e1 = __builtin_amdgcn_exp2f(sc[tb][r + 1] - m_new);
        rs += e0 + e1;
        const typename H::v2 pk = H::pack(e0, e1);
        pf[4 * tb + r] = pk[0];
        pf[4 * tb + r + 1] = pk[1];
      }
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) acc[t] *= alpha;
    // ---- O^T += V^T P^T: k slots 8kg + e are tokens 4kg + e (e < 4) and 16 + 4kg + e - 4;
    //      each half is one ds_read_b64_tr_b16 (source lane j reads V[k0 + j/4][nb + 4(j&3)],
    //      lane j receives V[k0 .. k0+3][nb + j]).
    const int j = lane & 15;
    v2i_t lo[D / 16], hi[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      const int nb = 16 * t + 4 * (j & 3);
      const int r_lo = 4 * kg + (j >> 2), r_hi = r_lo + 16;
      asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(lo[t]) : "v"(vst + T::off(r_lo, nb >> 3) + 2 * (nb & 7)));
      asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(hi[t]) : "v"(vst + T::off(r_hi, nb >> 3) + 2 * (nb & 7)));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int t = 0; t < D / 16; ++t) asm volatile("" : "+v"(lo[t]), "+v"(hi[t]));
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      const v4i_t vv = v4i_t{lo[t][0], lo[t][1], hi[t][0], hi[t][1]};
      acc[t] = H::mfma16(__builtin_bit_cast(hv8, vv), pf, acc[t]);
    }
  }
  // ---- partial out: head hcol, d = 16t + 4kg + r
  if (hcol < a.g) {
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
      *reinterpret_cast<f32x4*>(po + hcol * D + 16 * t + 4 * kg) = acc[t];
    if (kg == 0) {
      pml[2 * hcol] = m_run;
      pml[2 * hcol + 1] = l_run;
    }
  }
}


// Balanced launch: the batch's 32-token steps (sequence major) are cut into a.nranges equal
// contiguous ranges, and each range is run by hkv single-wave workgroups, one per kv head, launched
// next to each other (the cache rows of a token hold all its kv heads, so they are read at about
// the same time). A wave runs one segment per sequence its range touches. The first wave also
// records the step prefix the merge uses to find a sequence's partials.
template <int D, bool F16>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1)))
void paged_decode_kernel(DecodeArgs a) {
  using T = DecodeTile<D>;
  __shared__ __attribute__((aligned(16))) char s_kv[kVStages * 2 * T::kStage];  // [stage][K, V]
  const int lane = threadIdx.x;
  const int kvh = static_cast<int>(blockIdx.x % a.hkv);
  const int64_t r = blockIdx.x / a.hkv;
  const int64_t nb = a.b, R = a.nranges;
  int64_t mine = 0;
  for (int64_t c = lane; c < nb; c += 64) mine += dec_units(kv_len(a, c));
  const int64_t S = uniform64(wave_sum64(mine));
  if (blockIdx.x == 0) {
    int64_t carry = 0;
    for (int64_t c = 0; c < nb; c += 64) {
      const int64_t i = c + lane;
      const int64_t n = i < nb ? dec_units(kv_len(a, i)) : 0;
      const int64_t incl = wave_incl_scan64(n, lane) + carry;
      if (i < nb) a.steps[1 + i] = incl - n;
      carry = __shfl(incl, 63, 64);
    }
    if (lane == 0) a.steps[0] = S;
  }
  const int64_t g0 = r * S / R, g1 = (r + 1) * S / R;
  if (g0 >= g1) return;
  // the range's first sequence b (steps before it: pb) and step x = g0 inside the batch
  int64_t x = g0, b = 0, pb = 0;
  {
    int64_t carry = 0;
    for (int64_t c = 0; c < nb; c += 64) {
      const int64_t i = c + lane;
      const int64_t n = i < nb ? dec_units(kv_len(a, i)) : 0;
      const int64_t incl = wave_incl_scan64(n, lane) + carry;
      const uint64_t hit = __ballot(i < nb && n > 0 && incl - n <= x && x < incl);
      if (hit) {
        const int j = __ffsll(static_cast<unsigned long long>(hit)) - 1;
        b = c + j;
        pb = __shfl(incl - n, j, 64);
        break;
      }
      carry = __shfl(incl, 63, 64);
    }
  }
  b = uniform64(b);
  pb = uniform64(pb);
  for (int64_t g = g0; g < g1;) {
    const int64_t len = kv_len(a, b);
    const int64_t n = dec_units(len);
    const int64_t seg = min(g1 - g, pb + n - x);
    // units [u0, u1) of this sequence; the first kDecSegCost carry no tokens
    const int64_t u0 = x - pb, u1 = u0 + seg;
    const int64_t s0 = max<int64_t>(u0, kDecSegCost) - kDecSegCost, s1 = max<int64_t>(u1, kDecSegCost) - kDecSegCost;
    if (s1 > s0)
      decode_segment<D, F16>(a, (lds_char_t*)s_kv, b, kvh, s0 * kStep, min(len, s1 * kStep), r + b);
    g += seg;
    x += seg;
    if (x == pb + n) {  // on to the next non-empty sequence
      pb += n;
      do {
        ++b;
      } while (g < g1 && b < nb && dec_units(kv_len(a, b)) == 0);
    }
  }
}

// Merge the partials of (b, q head) pairs: one wave per head, four per workgroup, each lane owning
// D / 64 consecutive d. The partials are those of the ranges that cover the sequence's steps
// (ranges with no steps wrote nothing). A partial's statistics are wave-uniform loads and its O
// values do not depend on them, so all loads of a partial go out together.
template <int D, bool F16>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a, uint16_t* out, float* lse) {
  constexpr int E = D / 64;  // outputs per lane
  const int lane = threadIdx.x & 63;
  const int64_t bh = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (bh >= a.b * a.hq) return;
  const int h = static_cast<int>(bh % a.hq);
  const int64_t b = bh / a.hq;
  const int kvh = h / a.g, hi = h % a.g;
  // the length and the step prefix are loaded together (the prefix is valid for every b)
  const int64_t len = kv_len(a, b), S = a.steps[0], x0 = a.steps[1 + b], R = a.nranges;
  const int64_t n = dec_steps(len);
  uint16_t* o = out + (b * a.hq + h) * D + E * lane;
  // the sink logit in log2 units (-inf: none)
  const float sv = a.sink ? a.sink[h] * kLog2e : -INFINITY;
  if (n == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0;
    // with no keys the sink alone makes the denominator: lse = the sink logit
    if (lse && lane == 0) lse[b * a.hq + h] = sv != -INFINITY ? sv * kLn2 : -INFINITY;
    return;
  }
  // the sequence's units are [x0, x1); its tokens start kDecSegCost units in
  const int64_t xs = x0 + kDecSegCost, x1 = xs + n;
  const int64_t r_first = ((xs + 1) * R - 1) / S, r_last = (x1 * R - 1) / S;
  const int ns = static_cast<int>(r_last - r_first + 1);
  const int64_t row0 = ((r_first + b) * a.hkv + kvh) * 16 + hi;  // partial s: row0 + s * hkv * 16
  const int64_t rstep = static_cast<int64_t>(a.hkv) * 16;
  auto live = [&](int s) {
    const int64_t r = r_first + s;
    return (r + 1) * S / R > r * S / R;
  };
  // one pass with a running maximum: every partial's loads are independent of the others
  float M = -INFINITY, den = 0.0f, num[E];
#pragma unroll
  for (int e = 0; e < E; ++e) num[e] = 0.0f;
#pragma unroll 4
  for (int s = 0; s < ns; ++s) {
    const int64_t row = row0 + rstep * s;
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = a.part_o[row * D + E * lane + e];
    const float m = a.part_ml[row * 2], l = a.part_ml[row * 2 + 1];
    if (!live(s)) continue;
    const float m_new = fmaxf(M, m);
    const float c = exp2f(M - m_new), w = exp2f(m - m_new);  // M = -inf at first: c = 0
    den = den * c + w * l;
#pragma unroll
    for (int e = 0; e < E; ++e) num[e] = num[e] * c + w * v[e];
    M = m_new;
  }
  if (sv != -INFINITY) {
    // the sink joins the denominator only: it rescales the row like one more partial with no value
    const float m_new = fmaxf(M, sv);
    const float c = exp2f(M - m_new);
    den = den * c + exp2f(sv - m_new);
#pragma unroll
    for (int e = 0; e < E; ++e) num[e] *= c;
    M = m_new;
  }
  if (a.vsc) {
#pragma unroll
    for (int e = 0; e < E; ++e) num[e] *= a.vsc[kvh * D + E * lane + e];
  }
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = Half<F16>::bits(den > 0.0f ? num[e] / den : 0.0f);
  if (lse && lane == 0) lse[b * a.hq + h] = den > 0.0f ? (M + log2f(den)) * kLn2 : -INFINITY;
}

// Ranges per launch: about 1024 single-wave workgroups (four per CU: the 32 KB ring puts two in
// each 80 KB half of a CU's LDS).
inline int decode_ranges(int hkv) { return static_cast<int>(cdiv(1024, hkv)); }

// Workspace: [step prefix int64 x (b + 1), padded to 256 B][part_o][part_ml]
struct DecWs {
  size_t part_o, part_ml, total;
};
DecWs dec_ws(int64_t b, int hkv, int d) {
  const int64_t slots = decode_ranges(hkv) + b;
  DecWs w;
  w.part_o = (static_cast<size_t>(b + 1) * sizeof(int64_t) + 255) / 256 * 256;
  w.part_ml = w.part_o + static_cast<size_t>(slots) * hkv * 16 * d * sizeof(float);
  w.total = w.part_ml + static_cast<size_t>(slots) * hkv * 32 * sizeof(float);
  return w;
}



// ============================================================================ dense prefill
// Work item: (batch b, kv head, 8 "wave units"); a wave unit is (query head, 32 query rows), and the
// units of (b, kv head) run query-tile major, so an item is two 32-query tiles of 4 heads when
// Hq / Hkv = 4. The 8 waves of an item share the kv head: K/V tiles of 64 tokens are staged once in
// LDS and used by all of them. Two waves per SIMD: one wave's softmax (VALU) runs while the other's
// MFMAs do (a lone wave issues a VALU instruction only every ~8 cycles).
// Per wave, S^T = K Q^T with v_mfma_f32_32x32x16_bf16 puts one query per lane (column), so the
// online-softmax rescale of O^T is a per-lane scalar and P^T leaves the S^T registers already in
// the B-operand layout of O^T = V^T P^T.
// K/V tiles go through a four-slot ring filled with global_load_lds (16 bytes per lane, no
// register round trip): two tiles are in flight while one is used. LDS rows are the tile's token
// rows with 16-byte chunks XOR-swizzled by row, so the K fragment reads (32 rows, same chunk) and
// the transposing V reads (ds_read_b64_tr_b16: 4 rows x 32 bytes per 16 lanes) are free of bank
// conflicts.
// Persistent workgroups (one per CU) take items from per-XCD work queues, heaviest items first.
constexpr int kPQ = 32;       // query rows per wave
constexpr int kPWaves = 8;    // waves (units) per item
constexpr int kPKV = 64;      // kv tokens per LDS tile
constexpr int kPStages = 4;
constexpr int kPfQueues = 8;  // one work queue per XCD

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  float* lse;
  int64_t qs[3], ks[3], vs[3], os[3];  // element strides (batch, pos, head)
  const int64_t* lq;
  const int64_t* lkv;
  int64_t b;
  int64_t s_q, s_kv;
  int64_t kv_cap;  // longest kv length the inputs hold: s_kv, or max_blocks * block_size when paged
  int hq, hkv, g;
  // Visible kv positions of query i (both clamped to [0, len_kv)): -pre <= j - i - off <= next, with
  // off = len_kv - len_q (bottom-right origin) or 0 (top-left origin). A causal mask is next = 0.
  int origin_rd;
  int64_t pre, next;
  // Paged K/V (bt != null): token t of sequence b at block bt[b * bt_stride + t / bs], slot t % bs;
  // element (block, slot, head) at block * kblk (vblk) + slot * ks[1] (vs[1]) + head * ks[2] (vs[2]).
  const int32_t* bt;
  int64_t bt_stride;
  int bs;
  int64_t kblk, vblk;
  float scale_log2;    // |scale| * log2(e), > 0
  int neg_scale;       // the scale is negative: Q is negated on load
  int n_qt;            // query tiles per sequence
  int units_per_bk;    // n_qt * g
  int blocks_per_bk;   // items per (b, kv head)
  int64_t n_items;     // B * Hkv * blocks_per_bk work items
  int n_queues;        // work queues (one per XCD)
  int* queue;          // [kPfQueues] next-item counters, then the rescaling list's length and cursor
  int* flags;          // [n_items]: 1 = on the rescaling list
  int32_t* redo;       // [n_items] rescaling list
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void gbl_void_t;

// 4-byte load of a wave-uniform address through the scalar cache (counted by lgkmcnt, waited for here).
__device__ __forceinline__ int64_t sload_i32(const int32_t* p) {
  // uniform64 widens each 32-bit half unsigned: the builtin returns int, and OR-ing that into a 64-bit
  // value directly would sign-extend the low half
  const uint64_t u = static_cast<uint64_t>(uniform64(static_cast<int64_t>(reinterpret_cast<uint64_t>(p))));
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(u) : "memory");
  return v;
}

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p));
}

template <int D>
struct PrefillTile {
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kCpr = kRowBytes / 16;          // 16-byte chunks per token row
  static constexpr int kRsh = D == 128 ? 0 : 1;        // rows per 256-byte bank cycle = 1 << kRsh
  static constexpr int kTile = kPKV * kRowBytes;       // bytes of one K (or V) tile
  static constexpr int kRpi = 1024 / kRowBytes;        // token rows per 1 KB load instruction
  static constexpr int kLoadsPerWave = kTile / 1024 / kPWaves;
  static constexpr int kLoadsPerTile = 2 * kLoadsPerWave;  // K and V instructions per wave per tile
  static constexpr int kLds = kPStages * 2 * kTile;
  static_assert(kLoadsPerWave * kPWaves * 1024 == kTile, "load split");
  // XOR key of a row's 16-byte chunks. Over any 16 aligned rows it is a permutation (the K fragment
  // reads: 16 rows at one chunk hit 16 distinct 16-byte bank groups), and over 4 aligned rows of
  // one 256-byte bank line it takes 4 values that differ above the low two bits (the transposing V
  // reads: 4 rows x 4 consecutive chunks hit 16 distinct bank groups). Rows 16 apart share the key.
  __device__ static __forceinline__ int swz(int row) {
    return D == 128 ? (((row & 3) << 2) | ((row >> 2) & 3)) : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
  }
  // LDS byte offset of (row, 16-byte chunk c) within a tile
  __device__ static __forceinline__ int off(int row, int c) { return row * kRowBytes + 16 * (c ^ swz(row)); }
};

template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, so i can feed immediates
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// With two waves per SIMD a wave has 256 registers; keeping every operand and accumulator in VGPRs
// (no AGPR use in the kernel) lets the compiler use all 256 of them as VGPRs.
// LDS fragment reads with an immediate offset (inline asm, so the explicit waits count them exactly)
template <int IMM>
__device__ __forceinline__ void pf_read_b128(uint4& d, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(IMM));
}
template <int IMM>
__device__ __forceinline__ void pf_read_tr16(v2i_t& d, uint32_t addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(IMM));
}

// Counters and flags start at zero: a fill kernel clears them before the passes (a memset node
// in a captured graph is avoided on purpose).
__global__ void prefill_queue_reset(int* queue, int* flags, int64_t n_items) {
  if (blockIdx.x == 0 && threadIdx.x < kPfQueues + 2) queue[threadIdx.x] = 0;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n_items; i += gridDim.x * 256) flags[i] = 0;
}

template <int D, bool RESCALE, bool F16>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, int64_t blk, char* smem, int64_t nbk, int lane,
                                             int w, int col, int grp);

// The fast pass (RESCALE = false) takes every item; the rescaling pass takes the items the fast
// pass put on its list (none, on ordinary data: its workgroups read an empty list and exit).
// Queue x hands out items x, x + 8, x + 16, ... of the heaviest-first list (item i: query tiles
// blocks_per_bk - 1 - i / (B * Hkv) of (b, kv head) = i % (B * Hkv)). Taking items as CUs free up
// keeps the CUs busy to the end (with one workgroup per CU, the hardware dispatcher's fixed order
// leaves a CU idle behind another CU's long workgroup). When B * Hkv is a multiple of 8 a queue
// holds the items of the (b, kv head) pairs whose K/V then stays in one XCD's L2.
template <int D, bool RESCALE, bool F16>
__global__ __launch_bounds__(64 * kPWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];  // [stage][K, V]
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, grp = lane >> 5;
  const int64_t nbk = a.b * a.hkv;
  __shared__ int64_t s_item;
  const int q_id = static_cast<int>(blockIdx.x % a.n_queues);
  for (;;) {
    if (tid == 0) {
      if constexpr (RESCALE) {
        const int i = atomicAdd(a.queue + kPfQueues + 1, 1);
        s_item = i < *reinterpret_cast<volatile int*>(a.queue + kPfQueues) ? a.redo[i] : a.n_items;
      } else {
        s_item = static_cast<int64_t>(atomicAdd(a.queue + q_id, 1)) * a.n_queues + q_id;
      }
    }
    __syncthreads();  // also: every wave is done with the previous item's LDS tiles
    const uint64_t it_u = static_cast<uint64_t>(s_item);
    const int64_t blk = uniform64(static_cast<int64_t>(it_u));
    __syncthreads();
    if (blk >= a.n_items) break;
    prefill_item<D, RESCALE, F16>(a, blk, smem, nbk, lane, w, col, grp);
  }
}

template <int D, bool RESCALE, bool F16>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, int64_t blk, char* smem, int64_t nbk, int lane,
                                             int w, int col, int grp) {
  using T = PrefillTile<D>;
  using H = Half<F16>;
  using hv8 = typename H::v8;
  constexpr float kSlack = H::kSlack;
  const int jb = a.blocks_per_bk - 1 - static_cast<int>(blk / nbk);  // heaviest query tiles first
  const int64_t bk = blk % nbk;
  const int kvh = static_cast<int>(bk % a.hkv);
  const int64_t b = bk / a.hkv;
  const int unit = jb * kPWaves + w;
  const bool unit_ok = unit < a.units_per_bk;
  const int qt = unit_ok ? unit / a.g : 0;
  const int head = kvh * a.g + (unit_ok ? unit % a.g : 0);
  const int64_t Lq = a.lq ? clamp_len(a.lq[b], a.s_q) : a.s_q;
  const int64_t Lkv = a.lkv ? clamp_len(a.lkv[b], a.kv_cap) : a.s_kv;
  const int64_t off = a.origin_rd ? Lkv - Lq : 0;
  const int64_t q0 = static_cast<int64_t>(qt) * kPQ;
  const int64_t myq = q0 + col;
  // kv range [lo_of(q), hi_of(q)) that query q sees (empty when lo >= hi)
  auto hi_of = [&](int64_t q) -> int64_t { return imin64(Lkv, q + off + a.next + 1); };
  auto lo_of = [&](int64_t q) -> int64_t { return imax64(0, q + off - a.pre); };

  // kv extent of this wave and of the whole item (uniform across the workgroup)
  const bool wave_live = unit_ok && q0 < Lq;
  const int64_t wave_kv = wave_live ? imax64(0, hi_of(min<int64_t>(q0 + kPQ, Lq) - 1)) : 0;
  const int64_t wave_lo = wave_live ? imin64(lo_of(q0), wave_kv) : 0;
  int64_t blk_kv = 0, blk_lo = 0;
  {
    const int last_unit = min(jb * kPWaves + kPWaves - 1, a.units_per_bk - 1);
    const int qt_lo = (jb * kPWaves) / a.g;   // units are qtile-major: the first unit has the smallest tile
    const int qt_hi = last_unit / a.g;        // and the last unit the largest
    const int64_t qlast = min<int64_t>(static_cast<int64_t>(qt_hi) * kPQ + kPQ, Lq) - 1;
    // an item whose query tiles all lie past this sequence's length has no live wave: it loads
    // nothing (its tiles exist because the item list is sized for the longest sequence)
    const bool live = qlast >= 0 && static_cast<int64_t>(qt_lo) * kPQ < Lq;
    blk_kv = live ? imax64(0, hi_of(qlast)) : 0;
    blk_lo = live ? imin64(lo_of(static_cast<int64_t>(qt_lo) * kPQ), blk_kv) : 0;
  }
  // the item streams whole 64-token tiles from the one holding blk_lo
  const int64_t kv0 = (blk_lo / kPKV) * kPKV;

  // Q^T fragments (B operand): query myq, d slots 16 kd + 8 grp .. +8. With a negative scale Q is
  // negated (exact in bf16), so the kernel always works with a positive scale and takes the row
  // maximum of the raw scores.
  hv8 qf[D / 16];
  {
    const uint32_t qsign = a.neg_scale ? 0x80008000u : 0u;
    const bool ok = wave_live && myq < Lq;
    const uint16_t* qp = a.q + b * a.qs[0] + (ok ? myq : 0) * a.qs[1] + head * a.qs[2];
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) {
      uint4 u = ok ? *reinterpret_cast<const uint4*>(qp + 16 * kd + 8 * grp) : make_uint4(0, 0, 0, 0);
      u.x ^= qsign; u.y ^= qsign; u.z ^= qsign; u.w ^= qsign;
      qf[kd] = __builtin_bit_cast(hv8, u);
    }
  }
  f32x16 acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  // kv tokens the lane's query sees, relative to the item's first tile
  const int64_t qend = hi_of(myq) - kv0, qbeg = lo_of(myq) - kv0;

  // LDS byte offsets (within a stage) of this lane's fragment reads. Rows 32 further (the second
  // 32-token half of K) or 16 further (the next 16-token block of V) keep the row's swizzle, so
  // they are immediate offsets.
  const int h16 = lane >> 4, j16 = lane & 15;
  uint32_t koff[D / 16];
#pragma unroll
  for (int kd = 0; kd < D / 16; ++kd) koff[kd] = T::off(col, 2 * kd + grp);
  // V: k slots of lane group grp in 16-token block kb are tokens 16kb + 4grp + {0..3} (lo read) and
  // 16kb + 8 + 4grp + {0..3} (hi read), the S^T row order: in each ds_read_b64_tr_b16 source lane
  // j16 addresses V[k0 + j16/4][nb + 4 (j16 & 3)] and lane j16 receives V[k0 .. k0+3][nb + j16],
  // nb = 32dt + 16 (h16 & 1)
  uint32_t voff[2][D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    const int nb = 32 * dt + 16 * (h16 & 1) + 4 * (j16 & 3);
    const int r_lo = 4 * grp + (j16 >> 2);
    voff[0][dt] = T::kTile + T::off(r_lo, nb >> 3) + 2 * (nb & 7);
    voff[1][dt] = T::kTile + T::off(r_lo + 8, nb >> 3) + 2 * (nb & 7);
  }
  const uint32_t smem_base = lds_u32(smem);

  // global_load_lds of tile [t0, t0 + 64) into stage s; rows past the end load the last row
  // (finite values; their scores are masked, so they add nothing)
  const uint16_t* kbase = a.k + (a.bt ? 0 : b * a.ks[0]) + kvh * a.ks[2];
  const uint16_t* vbase = a.v + (a.bt ? 0 : b * a.vs[0]) + kvh * a.vs[2];
  const int32_t* btrow = a.bt ? a.bt + b * a.bt_stride : nullptr;
  // Each lane's rows of a tile and their chunk offsets do not change from tile to tile: a dense tile
  // that lies wholly before len_kv costs one scalar product and one add per load.
  // (the host keeps 64 rows of either stride below 2^31 elements)
  uint32_t lk_off[T::kLoadsPerWave], lv_off[T::kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < T::kLoadsPerWave; ++i) {
    const int q = w * T::kLoadsPerWave + i;
    const int row = q * T::kRpi + lane / T::kCpr;
    const int c = (lane % T::kCpr) ^ T::swz(row);
    lk_off[i] = static_cast<uint32_t>(row * a.ks[1] + 8 * c);
    lv_off[i] = static_cast<uint32_t>(row * a.vs[1] + 8 * c);
  }
  auto issue_tile = [&](int64_t t0, int s) {
    char* kst = smem + s * 2 * T::kTile;
    if (!btrow && t0 + kPKV <= Lkv) {
      const uint16_t* kt = kbase + t0 * a.ks[1];
      const uint16_t* vt = vbase + t0 * a.vs[1];
#pragma unroll
      for (int i = 0; i < T::kLoadsPerWave; ++i) {
        const int q = w * T::kLoadsPerWave + i;
        __builtin_amdgcn_global_load_lds((gbl_void_t*)(kt + lk_off[i]), (lds_void_t*)(kst + q * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((gbl_void_t*)(vt + lv_off[i]), (lds_void_t*)(kst + T::kTile + q * 1024), 16, 0, 0);
      }
      return;
    }
    // paged: a 64-token tile spans at most two blocks (bs >= 32); their ids come through the scalar
    // cache, so the wait for them does not drain the ring's outstanding vector loads. Token positions
    // stay below 2^31, so block arithmetic is 32-bit.
    int first_blk = 0;
    int64_t pid0 = 0, pid1 = 0;
    if (btrow) {
      first_blk = static_cast<int>(t0) / a.bs;
      const int last_blk = static_cast<int>(min<int64_t>(t0 + kPKV - 1, Lkv - 1)) / a.bs;
      pid0 = sload_i32(btrow + first_blk);
      pid1 = last_blk > first_blk ? sload_i32(btrow + last_blk) : pid0;
    }
#pragma unroll
    for (int i = 0; i < T::kLoadsPerWave; ++i) {
      const int q = w * T::kLoadsPerWave + i;
      const int row = q * T::kRpi + lane / T::kCpr;
      const int c = (lane % T::kCpr) ^ T::swz(row);
      const int tok = static_cast<int>(min<int64_t>(t0 + row, Lkv - 1));  // rows past the end load the last row
      int64_t koff = static_cast<int64_t>(tok) * a.ks[1], voff = static_cast<int64_t>(tok) * a.vs[1];
      if (btrow) {
        const int blkn = tok / a.bs, slot = tok - blkn * a.bs;
        const int64_t pid = blkn == first_blk ? pid0 : pid1;
        koff = pid * a.kblk + static_cast<int64_t>(slot) * a.ks[1];
        voff = pid * a.vblk + static_cast<int64_t>(slot) * a.vs[1];
      }
      __builtin_amdgcn_global_load_lds((gbl_void_t*)(kbase + koff + 8 * c), (lds_void_t*)(kst + q * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((gbl_void_t*)(vbase + voff + 8 * c), (lds_void_t*)(kst + T::kTile + q * 1024), 16, 0, 0);
    }
  };

  const int ntiles = static_cast<int>(cdiv(blk_kv - kv0, static_cast<int64_t>(kPKV)));
  // Ring of kPStages = 4 slots, tile u in slot u % 4. publish(u) waits for this wave's loads of tile
  // u and passes the workgroup barrier, after which every wave's part of tile u is in LDS; the tile
  // issued next goes into the slot of tile u - 2, whose last reads every wave has passed by then.
  int issued = 0;
  auto issue_next = [&] {
    if (issued < ntiles) issue_tile(kv0 + static_cast<int64_t>(issued) * kPKV, issued % kPStages);
    ++issued;
  };
  auto publish = [&](int u) {
    const int after = min(issued, ntiles) - 1 - u;  // tiles issued after u (loads complete in order)
    if (after >= 2) __builtin_amdgcn_s_waitcnt(((2 * T::kLoadsPerTile) & 0xF) | (((2 * T::kLoadsPerTile) >> 4) << 14) | 0x70 | 0xF00);
    else if (after == 1) __builtin_amdgcn_s_waitcnt((T::kLoadsPerTile & 0xF) | ((T::kLoadsPerTile >> 4) << 14) | 0x70 | 0xF00);
    else __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  static_assert(kPStages == 4, "the ring protocol below assumes four slots");
  static_assert(2 * T::kLoadsPerTile < 64, "vmcnt range");
  const typename H::v2 ones = H::pack(1.0f, 1.0f);

  // S^T of 32-token step n (tokens 32n .. 32n + 31) from the slot of its tile, raw (unscaled).
  auto s_mfma = [&](int n, f32x16& sd) {
    const uint32_t kb0 = smem_base + static_cast<uint32_t>((n >> 1) % kPStages) * 2 * T::kTile +
                         static_cast<uint32_t>(n & 1) * 32 * T::kRowBytes;
    hv8 kf[D / 16];
    static_for<D / 16>([&](auto kdc) {
      constexpr int kd = decltype(kdc)::value;
      uint4 raw;
      pf_read_b128<0>(raw, kb0 + koff[kd]);
      kf[kd] = __builtin_bit_cast(hv8, raw);
    });
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // the fragments pass through empty asm after the wait, so no use is scheduled before it
#pragma unroll
    for (int kd = 0; kd < D / 16; ++kd) asm volatile("" : "+v"(kf[kd]));
    sd = H::mfma32(kf[0], qf[0], f32x16{});
#pragma unroll
    for (int kd = 1; kd < D / 16; ++kd) sd = H::mfma32(kf[kd], qf[kd], sd);
  };
  // Steps whose every token every query of the wave sees need no mask: tokens (relative to kv0) in
  // [clean_lo, clean_hi), bounded by the last live query's first token and the first query's end.
  const int64_t clean_lo = wave_live ? lo_of(min<int64_t>(q0 + kPQ, Lq) - 1) - kv0 : 0;
  const int64_t clean_hi = wave_live ? hi_of(q0) - kv0 : 0;
  auto clean = [&](int n) { return 32 * static_cast<int64_t>(n) >= clean_lo && 32 * static_cast<int64_t>(n) + 32 <= clean_hi; };
  // masked scores of step n become -inf (branch-free: the compares run in the shadow of MFMAs)
  auto mask = [&](int n, f32x16& sd) {
    const int beg = static_cast<int>(imin64(32, imax64(0, qbeg - 32 * static_cast<int64_t>(n))));
    const int lim = static_cast<int>(imin64(32, imax64(beg, qend - 32 * static_cast<int64_t>(n))));
    const uint32_t span = static_cast<uint32_t>(lim - beg);  // token t is visible when t - beg < span (unsigned)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 8 * (r >> 2) + 4 * grp + (r & 3);
      sd[r] = static_cast<uint32_t>(t - beg) < span ? sd[r] : -INFINITY;
    }
  };
  // maximum (log2 domain) of a step's scores for this lane's query
  auto row_max = [&](const f32x16& sd) -> float {
    float m = sd[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) m = fmaxf(m, sd[r]);
    return fmaxf(m, __shfl_xor(m, 32, 64)) * a.scale_log2;
  };
  // P of a step (16 scores of this lane's query) into two bf16 B fragments; returns this lane's part
  // of the row sum (the other lane of the query, lane ^ 32, holds the rest: the two are added once,
  // after the last tile)
  auto softmax = [&](const f32x16& sc, hv8 (&pf)[2]) -> float {
    const float neg_m = (m_run == -INFINITY) ? 0.0f : -m_run;
    float rs[2] = {0.0f, 0.0f};
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[8 * kb2 + j], a.scale_log2, neg_m));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[8 * kb2 + j + 1], a.scale_log2, neg_m));
        const typename H::v2 pk = H::pack(e0, e1);
        pf[kb2][j] = pk[0];
        pf[kb2][j + 1] = pk[1];
        rs[kb2] = H::dot2(pk, ones, rs[kb2]);
      }
    return rs[0] + rs[1];
  };
  // V^T fragments of 16-token block kb (0..3) of the tile in slot `slot`
  auto v_read = [&](int slot, auto kbc, v2i_t (&lo)[D / 32], v2i_t (&hi)[D / 32]) {
    constexpr int kb = decltype(kbc)::value;
    const uint32_t vb = smem_base + static_cast<uint32_t>(slot) * 2 * T::kTile;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      pf_read_tr16<kb * 16 * T::kRowBytes>(lo[dt], vb + voff[0][dt]);
      pf_read_tr16<kb * 16 * T::kRowBytes>(hi[dt], vb + voff[1][dt]);
    }
  };
  auto pv_mfma = [&](v2i_t (&lo)[D / 32], v2i_t (&hi)[D / 32], const hv8& p) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) asm volatile("" : "+v"(lo[dt]), "+v"(hi[dt]));
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const hv8 vv = __builtin_bit_cast(hv8, (v4i_t{lo[dt][0], lo[dt][1], hi[dt][0], hi[dt][1]}));
      acc[dt] = H::mfma32(vv, p, acc[dt]);
    }
  };

  // One 64-token tile at a time. The fast pass (RESCALE = false) keeps the reference max of each
  // query at the max of the first tile it sees: a wave whose tile max rises above it by more than
  // kSlack (2^64 of headroom in P, l and O^T for bf16, 2^8 for fp16) puts the item on the rescaling pass's list and stops
  // computing (it still takes its part in the ring); the rescaling pass redoes the whole item,
  // raising the reference max (and rescaling O^T and l) whenever a tile's max exceeds it by more
  // than kSlack. Keeping the rescale out of the fast pass keeps the O^T accumulators in place.
  bool dead = false;
  // this wave's 32-token steps (relative to kv0): [step_lo, step_hi)
  const int step_hi = static_cast<int>(cdiv(imax64(0, wave_kv - kv0), 32));
  const int step_lo = static_cast<int>(imax64(0, wave_lo - kv0) / 32);
  constexpr int kVReads = 2 * (D / 32);  // ds_read_b64_tr_b16 per 16-token block
  // the ring is filled two tiles ahead (three measured slower)
  for (int i = 0; i < kPStages - 2; ++i) issue_next();
  // (the loop sits in a lambda: that placement measured 4% faster than the same loop inline)
  auto tile_loop = [&] {
    for (int it = 0; it < ntiles; ++it) {
      publish(it);
      issue_next();
      // a tile's first step runs (masked) whenever its second one is live
      if (2 * it >= step_hi || 2 * it + 1 < step_lo || dead) continue;
      const int slot = it % kPStages;
      const bool second = 2 * it + 1 < step_hi;
      // both steps' score MFMAs go out before the first mask, so the second step's K reads and MFMAs
      // overlap the wait for the first step's scores
      f32x16 s0, s1;
      s_mfma(2 * it, s0);
      if (second) s_mfma(2 * it + 1, s1);
      if (!clean(2 * it)) mask(2 * it, s0);
      if (second && !clean(2 * it + 1)) mask(2 * it + 1, s1);
      // The fast pass takes a step's maximum only while some query of the wave has no reference max
      // yet; afterwards a row sum above 2^kSlack (which any score more than kSlack above the reference
      // max produces) sends the item to the rescaling pass before the step's P V.
      const bool need_max = RESCALE || __any(m_run == -INFINITY);
      if (need_max) {
        float mx = row_max(s0);
        if (second) mx = fmaxf(mx, row_max(s1));
        if constexpr (RESCALE) {
          if (__any(mx > m_run + kSlack)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
  #pragma unroll
            for (int i = 0; i < D / 32; ++i)
  #pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;
            m_run = m_new;
          }
        } else {
          if (__any(m_run != -INFINITY && mx > m_run + kSlack)) {
            dead = true;
            if (lane == 0 && atomicExch(a.flags + blk, 1) == 0) a.redo[atomicAdd(a.queue + kPfQueues, 1)] = static_cast<int32_t>(blk);
            continue;
          }
          if (m_run == -INFINITY) m_run = mx;  // a query that has seen nothing so far: O^T and l are zero
        }
      }
      // half of 2^kSlack: a lane holds half of its query's scores, so a row sum past 2^kSlack puts one
      // of its two halves past this
      constexpr float kSlackHalf = F16 ? 128.0f : 9223372036854775808.0f;
      static_assert(kSlack == (F16 ? 8.0f : 64.0f), "kSlackHalf follows kSlack");
      auto overflow = [&](float rs) {  // fast pass, reference max fixed: does P leave its headroom?
        if (RESCALE || need_max || !__any(rs > kSlackHalf)) return false;
        dead = true;
        if (lane == 0 && atomicExch(a.flags + blk, 1) == 0) a.redo[atomicAdd(a.queue + kPfQueues, 1)] = static_cast<int32_t>(blk);
        return true;
      };
      // V^T fragments of a step's two 16-token blocks are read before its softmax, which hides their LDS
      // latency; the reads of the first block are complete once only the second block's remain
      // (LDS reads complete in order)
      hv8 pf[2];
      v2i_t lo[2][D / 32], hi[2][D / 32];
      v_read(slot, std::integral_constant<int, 0>(), lo[0], hi[0]);
      v_read(slot, std::integral_constant<int, 1>(), lo[1], hi[1]);
      const float rs0 = softmax(s0, pf);
      if (overflow(rs0)) continue;  // the next publish waits for the outstanding reads
      l_run += rs0;
      asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(kVReads) : "memory");
      pv_mfma(lo[0], hi[0], pf[0]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      pv_mfma(lo[1], hi[1], pf[1]);
      if (second) {
        v_read(slot, std::integral_constant<int, 2>(), lo[0], hi[0]);
        v_read(slot, std::integral_constant<int, 3>(), lo[1], hi[1]);
        const float rs1 = softmax(s1, pf);
        if (overflow(rs1)) continue;
        l_run += rs1;
        asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(kVReads) : "memory");
        pv_mfma(lo[0], hi[0], pf[0]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        pv_mfma(lo[1], hi[1], pf[1]);
      }
    }
  };
  tile_loop();
  if (dead) return;
  l_run += __shfl_xor(l_run, 32, 64);  // the two halves of each query's row sum
  if (!unit_ok || myq >= a.s_q) return;
  // ---- write O (lane = query col, d = 32dt + 8(r/4) + 4grp + r%4) and lse
  const bool live = wave_live && myq < Lq && l_run > 0.0f;
  const float inv = live ? 1.0f / l_run : 0.0f;
  uint16_t* op = a.out + b * a.os[0] + myq * a.os[1] + head * a.os[2];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d = 32 * dt + 8 * r4 + 4 * grp;
      uint32_t lo = static_cast<uint32_t>(H::bits(acc[dt][4 * r4] * inv)) |
                    (static_cast<uint32_t>(H::bits(acc[dt][4 * r4 + 1] * inv)) << 16);
      uint32_t hi = static_cast<uint32_t>(H::bits(acc[dt][4 * r4 + 2] * inv)) |
                    (static_cast<uint32_t>(H::bits(acc[dt][4 * r4 + 3] * inv)) << 16);
      *reinterpret_cast<uint2*>(op + d) = make_uint2(lo, hi);
    }
  if (a.lse && grp == 0)
    a.lse[(b * a.hq + head) * a.s_q + myq] = live ? (m_run + log2f(l_run)) * kLn2 : -INFINITY;
}

// ============================================================================ MLA absorbed decode
// Work: (sequence b, split of kMlaChunk tokens, group of 128 query heads) -> one workgroup of four
// waves, one per SIMD; wave w owns heads 32w .. 32w + 31 of the group. All heads of the group share
// one latent tile, so each latent row is fetched and converted once per group. A lane holds Q^T of
// its head (576 bf16, the B operand of S^T: 144 VGPRs) and that head's O^T (512 fp32: 256
// accumulators, which the allocator places in AGPRs).
// Per 32-token step s (one workgroup barrier):
//   - raw rows (int8 latent 512 B, bf16 rope key 128 B, fp32 scale) go global -> LDS with
//     global_load_lds through a four-stage ring, three steps ahead of their use;
//   - the workgroup converts step s + 1 into the other half of a double-buffered bf16 tile (the
//     int8 latent -> bf16 conversion is exact; rope rows and scales are copied alongside) while
//     step s is computed from the first;
//   - S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (rows = 32 tokens, columns = 32 heads); nope and
//     rope parts accumulate apart so the per-token scale multiplies only the first:
//     S = (q_nope . int8) * scale + q_rope . k_rope;
//   - O^T += C^T P'^T with P' = P * scale, so the MFMAs see the unscaled integers. A lane's S^T
//     values are the tokens 8i + 4h + r (h = lane / 32) of its head; the PV MFMAs order their k
//     slots the same way, so P'^T comes straight from the S^T registers and C^T is read in that
//     order with ds_read_b64_tr_b16.
// LDS accesses are inline asm with explicit waits (the compiler would otherwise drain the ring's
// outstanding global -> LDS loads before each access). The step loop is unrolled twice so that
// the tile of a step is an immediate offset.
constexpr int kMlaStep = 32;
constexpr int kMlaWaves = 4;
constexpr int kMlaHeads = 128;  // heads per workgroup (32 per wave)
constexpr int kMlaRing = 4;
constexpr int kMlaKB = 2;           // K fragments per pipelined batch
constexpr int kMlaVB = 4;           // V fragments per pipelined batch (two reads each)
constexpr float kMlaSlack = 8.0f;   // log2-domain headroom of the lazily raised softmax max
constexpr float kMlaHeadroom = 64.0f;  // log2-domain headroom of the fast pass's fixed reference
constexpr int kMlaWgs = 256;         // workgroups of a launch (one per CU of an MI355X)

struct MlaArgs {
  const uint16_t* qn;
  const uint16_t* qr;
  const int8_t* ckv;
  const float* cs;
  const uint16_t* kr;
  const int32_t* bt;
  int64_t max_blocks;
  const int64_t* lens;
  int64_t b;
  int hq, bs, hgroups;
  float scale_log2;
  // Partials: slot hg * (kMlaWgs + b_count) + w + b holds workgroup w's part of sequence b for head
  // group hg (w + b is unique: the workgroups covering one sequence are consecutive, and so are
  // the sequences one workgroup covers).
  uint16_t* part_o;  // [slots, kMlaHeads, DN] bf16, each partial divided by its own running sum
  float* part_ml;  // [slots, kMlaHeads, 2]
  int32_t* flags;  // [slots, kMlaWaves]: 1 = that wave's heads need the rescaling pass
  int32_t* wgflags;  // [kMlaWgs, kMlaWaves]: 1 = some segment of that workgroup's wave was flagged
  int64_t* steps;  // [0] = 32-token steps of all sequences S, [1 + b] = steps before sequence b
};

// Raw ring stage: [latent 32 x 512 B][rope 32 x 128 B][one 256 B scale slot per wave].
// bf16 tile: [latent 32 x 1 KB][rope 32 x 128 B][scale 32 x 4 B].
// Latent chunk c of tile row r sits at chunk c ^ X(r), X(r) = ((r & 3) << 2) | ((r >> 2) & 3): 16
// rows at one chunk hit 16 distinct 16-byte bank groups (the K reads, 16 lanes a pass), and 4
// consecutive rows x 4 chunks hit all 16 (the transposing V reads, 32 lanes a pass: X(r) >> 2
// differs over the 4 rows, so chunk sets {0..3} ^ X(r) are disjoint). X only moves the low four
// bits, so chunk 16q + c' is 256 q bytes past chunk c' ^ X(r), and X(r + 16) = X(r). Rope chunk c of row r (raw and tile) sits at c ^ ((r >> 1) & 7).
constexpr int kMlaLatBytes = kMlaStep * 512;
constexpr int kMlaRopeOff = kMlaLatBytes;
constexpr int kMlaScaleOff = kMlaRopeOff + kMlaStep * 128;
constexpr int kMlaRaw = kMlaScaleOff + kMlaWaves * 256;
constexpr int kMlaTRope = kMlaStep * 1024;
constexpr int kMlaTScale = kMlaTRope + kMlaStep * 128;
constexpr int kMlaTile = kMlaTScale + kMlaStep * 4;
constexpr int kMlaLds = kMlaRing * kMlaRaw + 2 * kMlaTile;
static_assert(kMlaLds <= 160 * 1024, "LDS budget");

__device__ __forceinline__ int mla_x(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }


template <int IMM>
__device__ __forceinline__ void lds_read_b128(v4i_t& d, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(IMM));
}
template <int IMM>
__device__ __forceinline__ void lds_read_b64(v2i_t& d, uint32_t addr) {
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(IMM));
}
template <int IMM>
__device__ __forceinline__ void lds_read_tr16(v2i_t& d, uint32_t addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(IMM));
}
template <int IMM>
__device__ __forceinline__ void lds_write_b128(uint32_t addr, const v4i_t& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(addr), "v"(v), "n"(IMM) : "memory");
}
// O^T += A B with the accumulator pinned to AGPRs. The compiler does not see the MFMA's latency:
// code that reads the accumulator with VALU ops must first wait it out (mfma_drain).
// The leading s_nop covers a VALU write of an operand just before (the compiler does not track
// hazards into inline asm).
__device__ __forceinline__ void mfma_agpr(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The same with the accumulator pinned to VGPRs (S^T, which VALU code reads): before a VALU read of
// the result, mfma_vgpr_wait() covers the latency of the last MFMA (16 passes).
__device__ __forceinline__ void mfma_vgpr(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_vgpr_zero(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b));
}
// The nops are tied to the accumulator (a read-write operand), so no instruction that reads it can
// be scheduled above them.
__device__ __forceinline__ void mfma_vgpr_wait(f32x16& acc) { asm volatile("s_nop 15\n\ts_nop 7" : "+v"(acc)::"memory"); }

// Longer than the worst-case latency of one 32x32x16 MFMA (16 passes). Every accumulator passes
// through an empty asm after the nops, so no read of one can be scheduled above them.
template <int N>
__device__ __forceinline__ void mfma_drain(f32x16 (&acc)[N]) {
  asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+a"(acc[i]));
}
template <int N>
__device__ __forceinline__ void lds_wait() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}

// One segment: tokens [t_begin, t_end) of sequence b for head group hg, partial written to slot
// `slot` (rows of kMlaHeads heads). Every wave of the workgroup runs it with the same arguments.
template <int DN, int DR, bool RESCALE>
__device__ __forceinline__ void mla_segment(const MlaArgs& a, char* smem, bool& ov_seen, int hg, int64_t b, int64_t t_begin,
                                            int64_t t_end, int64_t slot) {
  static_assert(DN == 512 && DR == 64, "MLA shape");
  constexpr int NQ = (DN + DR) / 16;  // Q^T fragments: 32 nope + 4 rope
  constexpr int NN = DN / 16;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, h = lane >> 5;
  const int hl = 32 * w + col;  // head within the group
  const int head = hg * kMlaHeads + hl;
  const bool head_ok = head < a.hq;
  const int64_t pbase = slot * kMlaHeads;
  // Q^T fragments (B operand): column = this lane's head, k slots = d 16m + 8h .. +8
  bf16x8 qf[NQ];
  {
    const int hh = head_ok ? head : 0;
    const uint16_t* qnp = a.qn + (b * a.hq + hh) * DN;
    const uint16_t* qrp = a.qr + (b * a.hq + hh) * DR;
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
      const int d = 16 * m + 8 * h;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (head_ok) v = m < NN ? *reinterpret_cast<const uint4*>(qnp + d) : *reinterpret_cast<const uint4*>(qrp + d - DN);
      qf[m] = as_bf16x8(v);
    }
  }
  // O^T accumulators, defined (as zeros) by an MFMA so that they live in AGPRs from the start
  // (The rescaling pass uses compiler-scheduled MFMAs throughout: it spills, and the compiler
  // cannot see the hazards of inline-asm MFMAs around its spill code.)
  f32x16 acc[DN / 32];
  if constexpr (RESCALE) {
#pragma unroll
    for (int dt = 0; dt < DN / 32; ++dt) acc[dt] = f32x16{};
  } else {
    const bf16x8 z = as_bf16x8(make_uint4(0, 0, 0, 0));
#pragma unroll
    for (int dt = 0; dt < DN / 32; ++dt) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(acc[dt]) : "v"(z));
  }
  float m_run = -INFINITY, l_run = 0.0f;

  // A step lies inside one page (bs % 32 == 0, segments start at multiples of 32 tokens). The page
  // ids of the segment are held one per lane, 64 at a time (a window is reloaded when a step leaves
  // it); a step's id is a lane broadcast.
  const int32_t* btrow = a.bt + b * a.max_blocks;
  const int bs = a.bs;
  const int n_local = static_cast<int>(t_end - t_begin);
  const int nsteps = (n_local + kMlaStep - 1) / kMlaStep;
  const int64_t pg_first = t_begin / bs, pg_last = (t_end - 1) / bs;
  int64_t win = pg_first;  // first page of the window
  int my_page = lane <= pg_last - win ? btrow[win + lane] : 0;
  // issue cursor: page (relative to the window) and slot of the next step to load; the steps are
  // issued in order, so the cursor advances by one step per issue (no division per step)
  int cur_pg = 0, cur_slot = static_cast<int>(t_begin - pg_first * bs);

  // Every wave issues the same number of global_load_lds per step, so one vmcnt fits all: four
  // latent instructions (2 rows of 512 B each), one rope instruction (8 rows of 128 B) and one
  // scale instruction into the wave's own 256 B slot (slot 0 is the one read).
  constexpr int kRawLoads = 6;
  // The step's cache row base is wave-uniform (scalar); per lane only a 32-bit offset is formed.
  // The lane-dependent row numbers are recomputed from an opaque copy of the lane id at every
  // step: hoisted out of the loop they would be spilled, and a scratch reload waits on vmcnt,
  // which would drain the ring.
  auto issue_raw = [&](int s) __attribute__((always_inline)) {
    char* st = smem + (s % kMlaRing) * kMlaRaw;
    if (cur_pg == 64) {  // rare: segments longer than 64 pages
      win += 64;
      cur_pg = 0;
      my_page = lane <= pg_last - win ? btrow[win + lane] : 0;
      __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);  // here, so that the common path waits for nothing
    }
    const int page = __builtin_amdgcn_readfirstlane(__shfl(my_page, cur_pg, 64));
    const int64_t tok0 = static_cast<int64_t>(page) * bs + cur_slot;  // cache row of the step
    cur_slot += kMlaStep;
    if (cur_slot == bs) { cur_slot = 0; ++cur_pg; }
    const int last = n_local - 1 - s * kMlaStep;
    int ln;
    asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
    const int8_t* lat = a.ckv + tok0 * DN;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = 4 * w + i;
      const int row = 2 * q + (ln >> 5);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(lat + min(row, last) * DN + 16 * (ln & 31)),
                                       (__attribute__((address_space(3))) void*)(st + q * 1024), 16, 0, kCpolNt);
    }
    {
      const int row = 8 * w + (ln >> 3);
      const int c = (ln & 7) ^ ((row >> 1) & 7);
      const uint16_t* src = a.kr + tok0 * DR + min(row, last) * DR + 8 * c;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(st + kMlaRopeOff + w * 1024), 16, 0, kCpolNt);
    }
    {
      const float* src = a.cs + tok0 + min(ln & 31, last);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(st + kMlaScaleOff + w * 256), 4, 0, kCpolNt);
    }
  };

  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)smem));
  const uint32_t tiles = lds0 + kMlaRing * kMlaRaw;
  // Raw step s -> bf16 tile t. Latent: 2048 units of 8 bytes, eight per thread: unit u is row
  // 8w + u, 8-byte source unit (= bf16 chunk) lane, so each 32-lane read pass covers 256 contiguous
  // bytes of one raw row. Rope rows and scales are copied as they are (16 bytes per thread; scales
  // by threads 0-7).
  auto convert = [&](int s, auto t_c) __attribute__((always_inline)) {
    constexpr int T = decltype(t_c)::value * kMlaTile;
    const uint32_t raw = lds0 + (s % kMlaRing) * kMlaRaw;
    v2i_t r[8];
    v4i_t rope, scl;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int row = 8 * w + u;
      asm volatile("ds_read_b64 %0, %1" : "=v"(r[u]) : "v"(raw + row * 512 + 8 * lane));
    }
    lds_read_b128<kMlaRopeOff>(rope, raw + 16 * tid);
    lds_read_b128<kMlaScaleOff>(scl, raw + 16 * (tid & 7));
    lds_wait<0>();
#pragma unroll
    for (int u = 0; u < 8; ++u) asm volatile("" : "+v"(r[u]));
    asm volatile("" : "+v"(rope), "+v"(scl));
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int row = 8 * w + u;
      const int c = lane;
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t wv = static_cast<uint32_t>(r[u][q]);
        const float f0 = static_cast<float>(static_cast<int8_t>(wv & 0xff));
        const float f1 = static_cast<float>(static_cast<int8_t>((wv >> 8) & 0xff));
        const float f2 = static_cast<float>(static_cast<int8_t>((wv >> 16) & 0xff));
        const float f3 = static_cast<float>(static_cast<int8_t>(wv >> 24));
        o[2 * q] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
        o[2 * q + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xffff0000u);
      }
      lds_write_b128<T>(tiles + row * 1024 + 16 * (c ^ mla_x(row)),
                        v4i_t{static_cast<int>(o[0]), static_cast<int>(o[1]), static_cast<int>(o[2]), static_cast<int>(o[3])});
    }
    lds_write_b128<T>(tiles + kMlaTRope + 16 * tid, rope);
    if (tid < 8) lds_write_b128<T>(tiles + kMlaTScale + 16 * tid, scl);
  };

  // Per-lane LDS bases (tile 0; tile 1 is kMlaTile further, an immediate).
  //   K (nope) fragment m: row col, chunk 2m + h -> kb(m & 7) + 256 (m >> 3).
  //   Rope fragment q: row col, chunk 2q + h of the 128-byte rope row -> rb(q).
  //   C^T fragment (dt, kk): lane group g = lane / 16, j = lane % 16; the two transposing reads
  //   address rows 16kk + 4h + j / 4 (+ 8) at bf16 column 32dt + 16(g & 1) + 4(j & 3)
  //   -> vb(half, dt & 3) + 256 (dt >> 2) + 16384 kk.
  // Each family of bases is one row base plus a per-lane XOR pattern: chunk (2q + h) ^ X equals
  // 2q ^ (h ^ X), so the address of fragment q is base + (pattern ^ 32q) (one v_xad per read).
  const uint32_t k_row = tiles + col * 1024, k_pat = 16 * (h ^ mla_x(col));
  const uint32_t r_row = tiles + kMlaTRope + col * 128, r_pat = 16 * (h ^ ((col >> 1) & 7));
  uint32_t v_row[2], v_pat[2];
  {
    const int g = lane >> 4, j = lane & 15;
    const int cp = 2 * (g & 1) + ((j >> 1) & 1);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int row = 4 * h + (j >> 2) + 8 * half;
      v_row[half] = tiles + row * 1024 + 8 * (j & 1);
      v_pat[half] = 16 * (cp ^ mla_x(row));
    }
  }
  auto kb = [&](int q) -> uint32_t { return k_row + (k_pat ^ (32u * q)); };
  auto rb = [&](int q) -> uint32_t { return r_row + (r_pat ^ (32u * q)); };
  auto vb = [&](int half, int q) -> uint32_t { return v_row[half] + (v_pat[half] ^ (64u * q)); };

  f32x16 sn;      // S^T of the current step (then the log2-domain logits)
  f32x4 cs[4];    // per-token scales of the lane's tokens
  float mx = 0.0f;
  // front: ring wait, the barrier, the next step's conversion, S^T and the step's max
  auto front = [&](int s, auto t_c) __attribute__((always_inline)) {
    constexpr int T = decltype(t_c)::value * kMlaTile;
    // raw(s + 1) must have landed (for the conversion); raw(s + 2) may stay in flight
    if (s + 2 < nsteps) __builtin_amdgcn_s_waitcnt(kRawLoads | 0x70 | 0xF00);
    else __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);
    // every wave's raw(s + 1) has landed, tile s is converted, and every wave is done with step
    // s - 1 (its tile and raw slot are free)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (s + 3 < nsteps) issue_raw(s + 3);
    if (s + 1 < nsteps) convert(s + 1, std::integral_constant<int, 1 - decltype(t_c)::value>{});
    // ---- per-token scales of this lane's tokens 8i + 4h + r
    static_for<4>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      lds_read_b128<T + 32 * i>(*reinterpret_cast<v4i_t*>(&cs[i]), tiles + kMlaTScale + 16 * h);
    });
    lds_wait<0>();
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(cs[i]));
    // ---- S^T: 36 fragments in batches of kMlaKB, the next batch in flight; S^T = (K_nope Q_nope^T)
    //      * scale + K_rope Q_rope^T, the rope MFMAs accumulating onto the scaled nope part
    constexpr int NKB = NQ / kMlaKB;
    static_assert(NQ % kMlaKB == 0, "K batches");
    v4i_t kf[2][kMlaKB];
    auto kread = [&](auto f_c, v4i_t& d) __attribute__((always_inline)) {
      constexpr int m = decltype(f_c)::value;
      if constexpr (m < NN) lds_read_b128<T + 256 * (m >> 3)>(d, kb(m & 7));
      else lds_read_b128<T>(d, rb(m - NN));
    };
    static_for<kMlaKB>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      kread(std::integral_constant<int, i>{}, kf[0][i]);
    });
    static_for<NKB>([&](auto bi_c) {
      constexpr int bi = decltype(bi_c)::value, cur = bi & 1;
      if constexpr (bi + 1 < NKB) {
        static_for<kMlaKB>([&](auto i_c) {
          constexpr int i = decltype(i_c)::value;
          kread(std::integral_constant<int, (bi + 1) * kMlaKB + i>{}, kf[cur ^ 1][i]);
        });
        lds_wait<kMlaKB>();
      } else {
        lds_wait<0>();
      }
      static_for<kMlaKB>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value, m = bi * kMlaKB + i;
        asm volatile("" : "+v"(kf[cur][i]));
        const bf16x8 kv = __builtin_bit_cast(bf16x8, kf[cur][i]);
        if constexpr (m == NN) {  // nope part complete: scale it, then add the rope part
          if constexpr (!RESCALE) mfma_vgpr_wait(sn);
#pragma unroll
          for (int e = 0; e < 16; ++e) sn[e] *= cs[e >> 2][e & 3];
        }
        if constexpr (RESCALE) {
          sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kv, qf[m], m == 0 ? f32x16{} : sn, 0, 0, 0);
        } else {
          if constexpr (m == 0) mfma_vgpr_zero(sn, kv, qf[m]);
          else mfma_vgpr(sn, kv, qf[m]);
        }
      });
    });
    // ---- logits
    if constexpr (!RESCALE) mfma_vgpr_wait(sn);
    const int64_t t0 = t_begin + static_cast<int64_t>(s) * kMlaStep;
    mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (t0 + 8 * i + 4 * h + r < t_end) ? sn[4 * i + r] * a.scale_log2 : -INFINITY;
        sn[4 * i + r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // finite: every step holds a valid token
  };
  // Online softmax with a lazily raised reference max: m_run moves (and O^T is rescaled) only
  // when the step's max exceeds it by more than kMlaSlack in the log2 domain, so
  // P' <= 2^kMlaSlack * scale between raises; the result is the same. Code that rescales O^T in
  // place makes the register allocator spill (it moves the AGPR accumulators through VGPRs), so
  // only the rescaling pass carries it.
  auto need_raise = [&]() __attribute__((always_inline)) { return __any(mx > m_run + kMlaSlack); };
  auto rescale = [&]() __attribute__((always_inline)) {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    mfma_drain(acc);
#pragma unroll
    for (int dt = 0; dt < DN / 32; ++dt) acc[dt] *= alpha;
    m_run = m_new;
  };
  // back: P' = exp2(S - m) * scale, l, and O^T += C^T P'^T
  auto back = [&](auto t_c) __attribute__((always_inline)) {
    constexpr int T = decltype(t_c)::value * kMlaTile;
    bf16x8 pf[2];
    float rs = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = __builtin_amdgcn_exp2f(sn[e] - m_run);
      rs += p;
      pf[e >> 3][e & 7] = static_cast<__bf16>(p * cs[e >> 2][e & 3]);
    }
    rs += __shfl_xor(rs, 32, 64);
    l_run += rs;
    // ---- O^T += C^T P'^T: fragment f = 16 kk + dt, batches of kMlaVB
    constexpr int NVF = 2 * (DN / 32), NVB = NVF / kMlaVB;
    v2i_t vlo[2][kMlaVB], vhi[2][kMlaVB];
    auto vread = [&](auto f_c, v2i_t& lo, v2i_t& hi) __attribute__((always_inline)) {
      constexpr int f = decltype(f_c)::value, kk = f / (DN / 32), dt = f % (DN / 32);
      lds_read_tr16<T + 256 * (dt >> 2) + 16384 * kk>(lo, vb(0, dt & 3));
      lds_read_tr16<T + 256 * (dt >> 2) + 16384 * kk>(hi, vb(1, dt & 3));
    };
    static_for<kMlaVB>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      vread(std::integral_constant<int, i>{}, vlo[0][i], vhi[0][i]);
    });
    static_for<NVB>([&](auto bi_c) {
      constexpr int bi = decltype(bi_c)::value, cur = bi & 1;
      if constexpr (bi + 1 < NVB) {
        static_for<kMlaVB>([&](auto i_c) {
          constexpr int i = decltype(i_c)::value;
          vread(std::integral_constant<int, (bi + 1) * kMlaVB + i>{}, vlo[cur ^ 1][i], vhi[cur ^ 1][i]);
        });
        lds_wait<2 * kMlaVB>();
      } else {
        lds_wait<0>();
      }
      static_for<kMlaVB>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value, f = bi * kMlaVB + i, kk = f / (DN / 32), dt = f % (DN / 32);
        asm volatile("" : "+v"(vlo[cur][i]), "+v"(vhi[cur][i]));
        const bf16x8 vv = __builtin_bit_cast(bf16x8, v4i_t{vlo[cur][i][0], vlo[cur][i][1], vhi[cur][i][0], vhi[cur][i][1]});
        if constexpr (RESCALE) acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv, pf[kk], acc[dt], 0, 0, 0);
        else mfma_agpr(acc[dt], vv, pf[kk]);
      });
    });
  };

  // prologue: three raw steps in flight, step 0 converted into tile 0 (the first step's barrier
  // publishes it)
  // every wave is done with the previous segment's ring and tiles
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  issue_raw(0);
  if (nsteps > 1) issue_raw(1);
  if (nsteps > 2) issue_raw(2);
  if (nsteps > 2) __builtin_amdgcn_s_waitcnt((2 * kRawLoads) | 0x70 | 0xF00);
  else if (nsteps > 1) __builtin_amdgcn_s_waitcnt(kRawLoads | 0x70 | 0xF00);
  else __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  convert(0, std::integral_constant<int, 0>{});
  const std::integral_constant<int, 0> t0c;
  const std::integral_constant<int, 1> t1c;
  // The fast pass (RESCALE = false) keeps the first step's max as the reference for the whole
  // split and never touches O^T in between: P' <= 2^kMlaHeadroom * scale keeps O^T and l far from
  // fp32 overflow (2048 tokens x 127 x 2^64). A split whose logits rise further is flagged and
  // redone by the rescaling pass, which raises the reference as above.
  bool overflow = false;
  auto settle = [&]() __attribute__((always_inline)) {
    if constexpr (RESCALE) {
      if (need_raise()) rescale();
    } else {
      if (m_run == -INFINITY) m_run = mx;  // first step: O^T and l are still zero
      else overflow = overflow || (mx > m_run + kMlaHeadroom);
    }
  };
  for (int s = 0; s < nsteps; s += 2) {
    front(s, t0c);
    settle();
    back(t0c);
    if (s + 1 < nsteps) {
      front(s + 1, t1c);
      settle();
      back(t1c);
    }
  }
  if constexpr (!RESCALE) {
    const bool any_ov = __any(overflow);
    if (lane == 0) a.flags[slot * kMlaWaves + w] = any_ov ? 1 : 0;
    ov_seen = ov_seen || any_ov;
  }
  if (!head_ok) return;
  if constexpr (!RESCALE) mfma_drain(acc);
  // ---- partial: O^T[d = 32dt + 8i + 4h + r][head] / l, as bf16 (the merge weighs it by l again); half
  //      the bytes of fp32 for the partial's write and the merge's read, at most one bf16 rounding
  //      of a convex combination's terms
  uint16_t* po = a.part_o + (pbase + hl) * DN;
  const float inv_l = 1.0f / l_run;
#pragma unroll
  for (int dt = 0; dt < DN / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2_t p0 = __builtin_convertvector((f32x2_t){acc[dt][4 * i] * inv_l, acc[dt][4 * i + 1] * inv_l}, bf16x2_t);
      const bf16x2_t p1 = __builtin_convertvector((f32x2_t){acc[dt][4 * i + 2] * inv_l, acc[dt][4 * i + 3] * inv_l}, bf16x2_t);
      *reinterpret_cast<uint2*>(po + 32 * dt + 8 * i + 4 * h) =
          make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
    }
  if (h == 0) {
    a.part_ml[(pbase + hl) * 2] = m_run;
    a.part_ml[(pbase + hl) * 2 + 1] = l_run;
  }
}

__device__ __forceinline__ int64_t mla_steps(int64_t len) { return len > 0 ? (len + kMlaStep - 1) / kMlaStep : 0; }

// The kMlaWgs workgroups of a launch split all 32-token steps (head group major, then sequence)
// into equal contiguous ranges, so every CU gets the same work whatever the lengths; a workgroup
// runs one segment per sequence its range touches. Workgroup 0 of the fast pass also records the
// step prefix the merge uses to find a sequence's partials.
template <int DN, int DR, bool RESCALE>
__global__ __launch_bounds__(64 * kMlaWaves) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mla_decode_kernel(MlaArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int lane = threadIdx.x & 63;
  const int64_t nb = a.b;
  const int64_t wg = blockIdx.x;
  int32_t* wgflag = a.wgflags + wg * kMlaWaves + (threadIdx.x >> 6);
  if constexpr (RESCALE) {  // nothing flagged in this workgroup's range: done
    const int4 f = *reinterpret_cast<const int4*>(a.wgflags + wg * kMlaWaves);
    if ((f.x | f.y | f.z | f.w) == 0) return;
  }
  bool ov_seen = false;
  int64_t mine = 0;
  for (int64_t c = lane; c < nb; c += 64) mine += mla_steps(kv_len(a, c));
  const int64_t S = uniform64(wave_sum64(mine));
  const int64_t W = S * a.hgroups;
  if (!RESCALE && wg == 0 && threadIdx.x < 64) {
    int64_t carry = 0;
    for (int64_t c = 0; c < nb; c += 64) {
      const int64_t i = c + lane;
      const int64_t n = i < nb ? mla_steps(kv_len(a, i)) : 0;
      const int64_t incl = wave_incl_scan64(n, lane) + carry;
      if (i < nb) a.steps[1 + i] = incl - n;
      carry = __shfl(incl, 63, 64);
    }
    if (lane == 0) a.steps[0] = S;
  }
  const int64_t g0 = wg * W / kMlaWgs, g1 = (wg + 1) * W / kMlaWgs;
  if (g0 >= g1) {
    if (!RESCALE && lane == 0) *wgflag = 0;
    return;
  }
  // the range's first sequence: head group g0 / S, step x = g0 % S inside it
  int hg = static_cast<int>(g0 / S);
  int64_t x = g0 % S, b = 0, pb = 0;
  {
    int64_t carry = 0;
    for (int64_t c = 0; c < nb; c += 64) {
      const int64_t i = c + lane;
      const int64_t n = i < nb ? mla_steps(kv_len(a, i)) : 0;
      const int64_t incl = wave_incl_scan64(n, lane) + carry;
      const uint64_t hit = __ballot(i < nb && n > 0 && incl - n <= x && x < incl);
      if (hit) {
        const int j = __ffsll(static_cast<unsigned long long>(hit)) - 1;
        b = c + j;
        pb = __shfl(incl - n, j, 64);
        break;
      }
      carry = __shfl(incl, 63, 64);
    }
  }
  b = uniform64(b);
  pb = uniform64(pb);
  for (int64_t g = g0; g < g1;) {
    const int64_t len = kv_len(a, b);
    const int64_t n = mla_steps(len);
    const int64_t seg = min(g1 - g, pb + n - x);
    const int64_t t_begin = (x - pb) * kMlaStep;
    const int64_t slot = hg * (kMlaWgs + nb) + wg + b;
    bool run = true;
    if constexpr (RESCALE) {
      const int32_t* f = a.flags + slot * kMlaWaves;
      run = (f[0] | f[1] | f[2] | f[3]) != 0;
    }
    if (run) mla_segment<DN, DR, RESCALE>(a, smem, ov_seen, hg, b, t_begin, min(len, t_begin + seg * kMlaStep), slot);
    g += seg;
    x += seg;
    if (x == pb + n) {  // on to the next non-empty sequence (the next head group after the last)
      pb += n;
      do {
        if (++b == nb) { b = 0; pb = 0; x = 0; ++hg; }
      } while (g < g1 && mla_steps(kv_len(a, b)) == 0);
    }
  }
  if (!RESCALE && lane == 0) *wgflag = ov_seen ? 1 : 0;
}

// Merge the partials of a sequence's heads: one wave per pair of heads (each lane owns 8
// consecutive d of both), four waves per workgroup. The partials are those of the workgroups whose
// step ranges cover the sequence. The statistics of both heads of a partial are one 16-byte load
// (uniform across the wave), and every partial's O values are loaded before the weights that
// scale them are known, so a wave waits on few dependent round trips.
constexpr int kMlaCombineHeads = 8;  // heads per combine workgroup (2 per wave)
template <int DN>
__global__ __launch_bounds__(256) void mla_combine_kernel(MlaArgs a, uint16_t* out, float* lse) {
  static_assert(DN == 512, "one lane holds 8 of the 512 latent dims");
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t per_b = (a.hq + kMlaCombineHeads - 1) / kMlaCombineHeads;
  const int64_t b = blockIdx.x / per_b;
  const int h0 = static_cast<int>(blockIdx.x % per_b) * kMlaCombineHeads + 2 * wv;
  if (h0 >= a.hq) return;
  const bool two = h0 + 1 < a.hq;
  const int64_t n = mla_steps(kv_len(a, b));
  uint4* o0 = reinterpret_cast<uint4*>(out + (b * a.hq + h0) * DN) + lane;
  uint4* o1 = reinterpret_cast<uint4*>(out + (b * a.hq + h0 + 1) * DN) + lane;
  if (n == 0) {
    *o0 = make_uint4(0, 0, 0, 0);
    if (two) *o1 = make_uint4(0, 0, 0, 0);
    if (lse && lane < (two ? 2 : 1)) lse[b * a.hq + h0 + lane] = -INFINITY;
    return;
  }
  const int64_t S = a.steps[0], W = S * a.hgroups;
  const int hg = h0 / kMlaHeads, hl = h0 % kMlaHeads;  // h0 is even, so both heads share hg
  const int64_t x0 = hg * S + a.steps[1 + b], x1 = x0 + n;
  const int64_t w_first = ((x0 + 1) * kMlaWgs - 1) / W, w_last = (x1 * kMlaWgs - 1) / W;
  const int ns = static_cast<int>(w_last - w_first + 1);
  const int64_t row0 = (hg * (kMlaWgs + a.b) + w_first + b) * kMlaHeads + hl;  // partial s: row0 + s * kMlaHeads
  const float* ml = a.part_ml + row0 * 2;
  const uint16_t* po = a.part_o + row0 * DN + 8 * lane;
  // With fewer steps than workgroups some ranges are empty; those workgroups wrote nothing.
  auto live = [&](int s) {
    const int64_t w = w_first + s;
    return (w + 1) * W / kMlaWgs > w * W / kMlaWgs;
  };
  float M0 = -INFINITY, M1 = -INFINITY;
  for (int s = 0; s < ns; ++s) {
    if (!live(s)) continue;
    const float4 st = *reinterpret_cast<const float4*>(ml + 2 * kMlaHeads * s);
    M0 = fmaxf(M0, st.x);
    M1 = fmaxf(M1, st.z);
  }
  float den0 = 0.0f, den1 = 0.0f, num0[8], num1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) num0[i] = num1[i] = 0.0f;
  for (int s = 0; s < ns; ++s) {
    const uint16_t* p = po + static_cast<int64_t>(kMlaHeads) * DN * s;
    const uint4 a8 = load_nt_u4(p), b8 = load_nt_u4(p + DN);  // each partial is read once
    if (!live(s)) continue;
    const float4 st = *reinterpret_cast<const float4*>(ml + 2 * kMlaHeads * s);
    const float w0 = exp2f(st.x - M0) * st.y, w1 = exp2f(st.z - M1) * st.w;  // weight x running sum
    den0 += w0;
    den1 += w1;
    float v0[8], v1[8];
    const uint32_t aw[4] = {a8.x, a8.y, a8.z, a8.w}, bw[4] = {b8.x, b8.y, b8.z, b8.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v0[2 * i] = __uint_as_float(aw[i] << 16);
      v0[2 * i + 1] = __uint_as_float(aw[i] & 0xffff0000u);
      v1[2 * i] = __uint_as_float(bw[i] << 16);
      v1[2 * i + 1] = __uint_as_float(bw[i] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      num0[i] += w0 * v0[i];
      num1[i] += w1 * v1[i];
    }
  }
  auto pack = [](const float (&v)[8], float den) {
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[i] = static_cast<uint32_t>(f32_to_bf16(den > 0.0f ? v[2 * i] / den : 0.0f)) |
             (static_cast<uint32_t>(f32_to_bf16(den > 0.0f ? v[2 * i + 1] / den : 0.0f)) << 16);
    return make_uint4(r[0], r[1], r[2], r[3]);
  };
  *o0 = pack(num0, den0);
  if (two) *o1 = pack(num1, den1);
  if (lse && lane == 0) {
    lse[b * a.hq + h0] = den0 > 0.0f ? (M0 + log2f(den0)) * kLn2 : -INFINITY;
    if (two) lse[b * a.hq + h0 + 1] = den1 > 0.0f ? (M1 + log2f(den1)) * kLn2 : -INFINITY;
  }
}

// Workspace: [step prefix int64 x (b + 1), padded to 256 B][part_o][part_ml][flags][workgroup flags]
struct MlaWs {
  size_t steps, part_o, part_ml, flags, wgflags, total;
};
MlaWs mla_ws(int64_t b, int hq, int dn) {
  const int64_t slots = ((hq + kMlaHeads - 1) / kMlaHeads) * (kMlaWgs + b);
  MlaWs w;
  w.steps = 0;
  w.part_o = (static_cast<size_t>(b + 1) * sizeof(int64_t) + 255) / 256 * 256;
  w.part_ml = w.part_o + (static_cast<size_t>(slots) * kMlaHeads * dn * sizeof(uint16_t) + 255) / 256 * 256;
  w.flags = w.part_ml + static_cast<size_t>(slots) * kMlaHeads * 2 * sizeof(float);
  w.wgflags = (w.flags + static_cast<size_t>(slots) * kMlaWaves * sizeof(int32_t) + 15) / 16 * 16;
  w.total = w.wgflags + static_cast<size_t>(kMlaWgs) * kMlaWaves * sizeof(int32_t);
  return w;
}
}  // namespace
}  // namespace tai

using namespace tai;

extern "C" size_t tai_fia_paged_decode_workspace_size(int64_t b, int hq, int d, int64_t max_blocks, int block_size) {
  (void)max_blocks;
  (void)block_size;
  // the largest over the kv head counts hq allows
  size_t need = 0;
  for (int hkv = 1; hkv <= hq; ++hkv)
    if (hq % hkv == 0) need = std::max(need, dec_ws(b, hkv, d).total);
  return need;
}

namespace {
// int8 pages -> 16-bit pages (the int8 values themselves, exact in bf16 and fp16): page p of sequence
// s, for the pages its length covers, goes to staging page s * max_blocks + p, and bt2 maps it there.
// One workgroup per (page, sequence); 8 bytes per thread step.
__global__ __launch_bounds__(256) void kv8_widen_kernel(const int8_t* __restrict__ k, const int8_t* __restrict__ v,
                                                        int64_t sb, int64_t ss, int64_t sh, const int32_t* bt,
                                                        int64_t max_blocks, const int64_t* lens, int bs, int hkv, int d,
                                                        bool f16, uint16_t* kw, uint16_t* vw, int32_t* bt2) {
  const int64_t page = blockIdx.x, seq = blockIdx.y;
  const int64_t idx = seq * max_blocks + page;
  if (threadIdx.x == 0) bt2[idx] = static_cast<int32_t>(idx);
  const int64_t len = imax64(0, imin64(lens[seq], max_blocks * bs));
  if (page * bs >= len) return;
  const int64_t blk = bt[idx];
  const int cpr = d / 8;  // 8-byte chunks per (slot, head) row
  const int n = bs * hkv * cpr;
  for (int c = threadIdx.x; c < n; c += 256) {
    const int row = c / cpr, ch = c - row * cpr;
    const int slot = row / hkv, head = row - slot * hkv;
    const int64_t src = blk * sb + slot * ss + head * sh + 8 * ch;
    const int64_t dst = (idx * bs + slot) * static_cast<int64_t>(hkv) * d + static_cast<int64_t>(head) * d + 8 * ch;
    const uint2 ku = *reinterpret_cast<const uint2*>(k + src);
    const uint2 vu = *reinterpret_cast<const uint2*>(v + src);
    uint32_t ko[4], vo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t kwd = q < 2 ? ku.x : ku.y, vwd = q < 2 ? vu.x : vu.y;
      const int sh0 = 16 * (q & 1);
      auto cvt = [&](uint32_t wd, int s) {
        const float x = static_cast<float>(static_cast<int8_t>((wd >> s) & 0xffu));
        return static_cast<uint32_t>(f16 ? f32_to_f16(x) : f32_to_bf16(x));
      };
      ko[q] = cvt(kwd, sh0) | (cvt(kwd, sh0 + 8) << 16);
      vo[q] = cvt(vwd, sh0) | (cvt(vwd, sh0 + 8) << 16);
    }
    *reinterpret_cast<uint4*>(kw + dst) = make_uint4(ko[0], ko[1], ko[2], ko[3]);
    *reinterpret_cast<uint4*>(vw + dst) = make_uint4(vo[0], vo[1], vo[2], vo[3]);
  }
}

// q * key scale per channel, rounded to the query's dtype: q.(k * sc) = (q * sc).k
__global__ __launch_bounds__(256) void q_scale_kernel(const uint16_t* q, const float* ksc, int64_t n, int hq, int hkv,
                                                      int d, bool f16, uint16_t* q2) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int dd = static_cast<int>(i % d);
  const int h = static_cast<int>((i / d) % hq);
  const float x = (f16 ? f16_to_f32(q[i]) : bf16_to_f32(q[i])) * ksc[(h / (hq / hkv)) * d + dd];
  q2[i] = f16 ? f32_to_f16(x) : f32_to_bf16(x);
}

int paged_decode(const void* q, const void* k_cache, const void* v_cache, int64_t stride_block, int64_t stride_slot,
                 int64_t stride_head, const int32_t* block_table, int64_t max_blocks, const int64_t* seq_lens_kv,
                 int64_t b, int hq, int hkv, int d, int dtype, int block_size, float scale, const float* sink,
                 const float* vsc, void* out, float* lse, void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(b >= 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "tai_fia_paged_decode: heads must be a multiple of kv heads");
  TAI_UNSUPPORTED(dtype != TAI_DT_BF16 && dtype != TAI_DT_FP16, "tai_fia_paged_decode: dtype %d not supported (bf16, "
                  "fp16)", dtype);
  TAI_UNSUPPORTED(hq / hkv > 16, "tai_fia_paged_decode: at most 16 query heads per kv head (got %d)", hq / hkv);
  TAI_UNSUPPORTED(d != 64 && d != 128 && d != 256, "tai_fia_paged_decode: head_dim %d not supported (64/128/256)", d);
  TAI_UNSUPPORTED(block_size <= 0 || block_size % kStep != 0, "tai_fia_paged_decode: block_size must be a multiple of %d", kStep);
  TAI_CHECK_ARG((stride_slot % 8) == 0 && (stride_head % 8) == 0 && (stride_block % 8) == 0,
                "tai_fia_paged_decode: cache strides must keep 16-byte alignment");
  if (b == 0) return TAI_OK;
  TAI_CHECK_ARG(q && k_cache && v_cache && block_table && seq_lens_kv && out, "tai_fia_paged_decode: null pointer");
  const DecWs wl = dec_ws(b, hkv, d);
  if (workspace == nullptr || ws_bytes < wl.total) {
    set_error("tai_fia_paged_decode: workspace of %zu bytes, need %zu", ws_bytes, wl.total);
    return TAI_ERR_WORKSPACE;
  }
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k_cache);
  a.v = static_cast<const uint16_t*>(v_cache);
  a.sb = stride_block; a.ss = stride_slot; a.sh = stride_head;
  a.bt = block_table; a.max_blocks = max_blocks; a.lens = seq_lens_kv;
  a.b = b; a.hq = hq; a.hkv = hkv; a.g = hq / hkv; a.bs = block_size;
  a.scale_log2 = scale * kLog2e;
  a.nranges = decode_ranges(hkv);
  a.steps = static_cast<int64_t*>(workspace);
  a.part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.part_o);
  a.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.part_ml);
  a.sink = sink;
  a.vsc = vsc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.nranges) * hkv));
  const dim3 cgrid(static_cast<unsigned>(cdiv(b * hq, 4)));
  uint16_t* o = static_cast<uint16_t*>(out);
  auto launch = [&](auto f16c) {
    constexpr bool F16 = decltype(f16c)::value;
    switch (d) {
      case 64:
        paged_decode_kernel<64, F16><<<grid, 64, 0, st>>>(a);
        decode_combine_kernel<64, F16><<<cgrid, 256, 0, st>>>(a, o, lse);
        break;
      case 128:
        paged_decode_kernel<128, F16><<<grid, 64, 0, st>>>(a);
        decode_combine_kernel<128, F16><<<cgrid, 256, 0, st>>>(a, o, lse);
        break;
      default:
        paged_decode_kernel<256, F16><<<grid, 64, 0, st>>>(a);
        decode_combine_kernel<256, F16><<<cgrid, 256, 0, st>>>(a, o, lse);
        break;
    }
  };
  if (dtype == TAI_DT_FP16) launch(std::true_type());
  else launch(std::false_type());
  return launch_status("tai_fia_paged_decode");
}
}  // namespace

extern "C" int tai_fia_paged_decode(const void* q, const void* k_cache, const void* v_cache, int64_t stride_block,
                                    int64_t stride_slot, int64_t stride_head, const int32_t* block_table,
                                    int64_t max_blocks, const int64_t* seq_lens_kv, int64_t b, int hq, int hkv, int d,
                                    int dtype, int block_size, float scale, void* out, float* lse, void* workspace,
                                    size_t ws_bytes, void* stream) {
  return paged_decode(q, k_cache, v_cache, stride_block, stride_slot, stride_head, block_table, max_blocks,
                      seq_lens_kv, b, hq, hkv, d, dtype, block_size, scale, nullptr, nullptr, out, lse, workspace,
                      ws_bytes, stream);
}

extern "C" int tai_fia_paged_decode_sink(const void* q, const void* k_cache, const void* v_cache,
                                         int64_t stride_block, int64_t stride_slot, int64_t stride_head,
                                         const int32_t* block_table, int64_t max_blocks, const int64_t* seq_lens_kv,
                                         int64_t b, int hq, int hkv, int d, int dtype, int block_size, float scale,
                                         const float* sink, void* out, float* lse, void* workspace, size_t ws_bytes,
                                         void* stream) {
  TAI_CHECK_ARG(sink != nullptr, "tai_fia_paged_decode_sink: null sink");
  return paged_decode(q, k_cache, v_cache, stride_block, stride_slot, stride_head, block_table, max_blocks,
                      seq_lens_kv, b, hq, hkv, d, dtype, block_size, scale, sink, nullptr, out, lse, workspace,
                      ws_bytes, stream);
}

namespace {
// int8 decode workspace: [decode workspace][k staging][v staging][bt2][q2], each 256-byte aligned
struct Kv8Ws {
  size_t kst, vst, bt2, q2, total;
};
Kv8Ws kv8_ws(int64_t b, int hq, int hkv, int d, int64_t max_blocks, int bs) {
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  Kv8Ws w;
  const size_t st = static_cast<size_t>(b) * max_blocks * bs * hkv * d * 2;
  w.kst = up(dec_ws(b, hkv, d).total);
  w.vst = w.kst + up(st);
  w.bt2 = w.vst + up(st);
  w.q2 = w.bt2 + up(static_cast<size_t>(b) * max_blocks * 4);
  w.total = w.q2 + up(static_cast<size_t>(b) * hq * d * 2);
  return w;
}
}  // namespace

extern "C" size_t tai_fia_paged_decode_kv8_workspace_size(int64_t b, int hq, int hkv, int d, int64_t max_blocks,
                                                         int block_size) {
  if (b <= 0 || hq <= 0 || hkv <= 0 || d <= 0 || max_blocks <= 0 || block_size <= 0) return 256;
  return kv8_ws(b, hq, hkv, d, max_blocks, block_size).total;
}

extern "C" int tai_fia_paged_decode_kv8(const void* q, const int8_t* k_cache, const int8_t* v_cache,
                                        int64_t stride_block, int64_t stride_slot, int64_t stride_head,
                                        const int32_t* block_table, int64_t max_blocks, const int64_t* seq_lens_kv,
                                        int64_t b, int hq, int hkv, int d, int dtype, int block_size, float scale,
                                        const float* k_scale, const float* v_scale, void* out, float* lse,
                                        void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(b >= 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && max_blocks > 0,
                "tai_fia_paged_decode_kv8: bad sizes or head counts");
  TAI_UNSUPPORTED(dtype != TAI_DT_BF16 && dtype != TAI_DT_FP16, "tai_fia_paged_decode_kv8: dtype %d not supported "
                  "(bf16, fp16)", dtype);
  TAI_UNSUPPORTED(d != 64 && d != 128 && d != 256, "tai_fia_paged_decode_kv8: head_dim %d not supported (64/128/256)", d);
  TAI_UNSUPPORTED(block_size <= 0 || block_size % kStep != 0, "tai_fia_paged_decode_kv8: block_size must be a "
                  "multiple of %d", kStep);
  TAI_CHECK_ARG((stride_slot % 8) == 0 && (stride_head % 8) == 0 && (stride_block % 8) == 0 &&
                    (reinterpret_cast<uintptr_t>(k_cache) % 8) == 0 && (reinterpret_cast<uintptr_t>(v_cache) % 8) == 0,
                "tai_fia_paged_decode_kv8: int8 cache rows must be 8-byte aligned");
  if (b == 0) return TAI_OK;
  TAI_CHECK_ARG(q && k_cache && v_cache && block_table && seq_lens_kv && out && k_scale && v_scale,
                "tai_fia_paged_decode_kv8: null pointer");
  const Kv8Ws w = kv8_ws(b, hq, hkv, d, max_blocks, block_size);
  if (workspace == nullptr || ws_bytes < w.total) {
    set_error("tai_fia_paged_decode_kv8: workspace of %zu bytes, need %zu", ws_bytes, w.total);
    return TAI_ERR_WORKSPACE;
  }
  TAI_CHECK_ARG(max_blocks <= 65535 && b <= 65535 && b * max_blocks < (int64_t(1) << 31),
                "tai_fia_paged_decode_kv8: at most 65535 sequences and 65535 pages per sequence");
  char* ws = static_cast<char*>(workspace);
  uint16_t* kst = reinterpret_cast<uint16_t*>(ws + w.kst);
  uint16_t* vst = reinterpret_cast<uint16_t*>(ws + w.vst);
  int32_t* bt2 = reinterpret_cast<int32_t*>(ws + w.bt2);
  uint16_t* q2 = reinterpret_cast<uint16_t*>(ws + w.q2);
  const bool f16 = dtype == TAI_DT_FP16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  kv8_widen_kernel<<<dim3(static_cast<unsigned>(max_blocks), static_cast<unsigned>(b)), 256, 0, st>>>(
      k_cache, v_cache, stride_block, stride_slot, stride_head, block_table, max_blocks, seq_lens_kv, block_size, hkv,
      d, f16, kst, vst, bt2);
  const int64_t nq = b * hq * d;
  q_scale_kernel<<<dim3(static_cast<unsigned>(cdiv(nq, 256))), 256, 0, st>>>(static_cast<const uint16_t*>(q), k_scale,
                                                                              nq, hq, hkv, d, f16, q2);
  if (launch_status("tai_fia_paged_decode_kv8") != TAI_OK) return TAI_ERR_LAUNCH;
  const int64_t sslot = static_cast<int64_t>(hkv) * d;
  return paged_decode(q2, kst, vst, sslot * block_size, sslot, d, bt2, max_blocks, seq_lens_kv, b, hq, hkv, d, dtype,
                      block_size, scale, nullptr, v_scale, out, lse, workspace, w.kst, stream);
}

extern "C" size_t tai_fia_prefill_workspace_size(int64_t b, int64_t s_q, int hq, int hkv) {
  if (b <= 0 || s_q <= 0 || hq <= 0 || hkv <= 0) return 256;
  const int64_t n_items = b * hkv * cdiv(cdiv(s_q, kPQ) * (hq / hkv), kPWaves);
  return static_cast<size_t>(256 + 8 * n_items + 256);
}

extern "C" int tai_fia_prefill(const void* q, const void* k, const void* v, int64_t b, int64_t s_q, int64_t s_kv, int hq,
                               int hkv, int d, int dtype, const int64_t* q_strides, const int64_t* k_strides,
                               const int64_t* v_strides, const int64_t* out_strides, const int64_t* seq_lens_q,
                               const int64_t* seq_lens_kv, int mask_origin, int64_t pre_tokens, int64_t next_tokens,
                               const int32_t* block_table, int64_t max_blocks, int block_size, int64_t k_block_stride,
                               int64_t v_block_stride, float scale, void* out, float* lse, void* workspace,
                               size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(b >= 0 && s_q >= 0 && s_kv >= 0, "tai_fia_prefill: negative size");
  TAI_CHECK_ARG(hq > 0 && hkv > 0 && hq % hkv == 0, "tai_fia_prefill: heads must be a multiple of kv heads");
  TAI_CHECK_ARG(mask_origin == 0 || mask_origin == 1, "tai_fia_prefill: mask_origin must be 0 (top-left) or 1 "
                "(bottom-right)");
  TAI_UNSUPPORTED(d != 64 && d != 128, "tai_fia_prefill: head_dim %d not supported (64, 128)", d);
  TAI_UNSUPPORTED(dtype != TAI_DT_BF16 && dtype != TAI_DT_FP16, "tai_fia_prefill: dtype %d not supported (bf16, fp16)",
                  dtype);
  TAI_CHECK_ARG(q_strides && k_strides && v_strides && out_strides, "tai_fia_prefill: null strides");
  for (int i = 0; i < 3; ++i)
    TAI_CHECK_ARG(q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 && out_strides[i] % 4 == 0,
                  "tai_fia_prefill: strides must keep 16-byte rows");
  TAI_UNSUPPORTED(64 * std::max(std::abs(k_strides[1]), std::abs(v_strides[1])) >= (int64_t(1) << 31) ||
                      s_kv >= (int64_t(1) << 31),
                  "tai_fia_prefill: kv positions and 64 token rows of K/V must stay below 2^31 elements");
  if (block_table) {
    TAI_CHECK_ARG(seq_lens_kv != nullptr && max_blocks > 0, "tai_fia_prefill: paged K/V need seq_lens_kv and "
                  "max_blocks > 0");
    TAI_UNSUPPORTED(block_size < 32 || block_size % 32 != 0, "tai_fia_prefill: paged block_size %d must be a "
                    "multiple of 32", block_size);
    TAI_CHECK_ARG(k_block_stride % 8 == 0 && v_block_stride % 8 == 0, "tai_fia_prefill: block strides must keep "
                  "16-byte rows");
  }
  if (b == 0 || s_q == 0) return TAI_OK;
  TAI_CHECK_ARG(q && k && v && out, "tai_fia_prefill: null pointer");
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  for (int i = 0; i < 3; ++i) { a.qs[i] = q_strides[i]; a.ks[i] = k_strides[i]; a.vs[i] = v_strides[i]; a.os[i] = out_strides[i]; }
  a.lq = seq_lens_q; a.lkv = seq_lens_kv; a.b = b; a.s_q = s_q; a.s_kv = s_kv;
  a.kv_cap = block_table ? max_blocks * block_size : s_kv;
  a.hq = hq; a.hkv = hkv; a.g = hq / hkv;
  // pre / next beyond 2^40 tokens are no bound (keeps the kernel's position arithmetic in range)
  constexpr int64_t kNoBound = int64_t(1) << 40;
  a.origin_rd = mask_origin;
  a.pre = pre_tokens < kNoBound ? pre_tokens : kNoBound;
  a.next = next_tokens < kNoBound ? next_tokens : kNoBound;
  a.pre = a.pre > -kNoBound ? a.pre : -kNoBound;
  a.next = a.next > -kNoBound ? a.next : -kNoBound;
  a.bt = block_table;
  a.bt_stride = max_blocks;
  a.bs = block_size;
  a.kblk = k_block_stride;
  a.vblk = v_block_stride;
  // the kernel works with a positive scale (a negative one negates Q); a zero scale makes every score
  // zero, which the smallest normal scale reproduces up to rounding far below bf16 resolution
  a.neg_scale = scale < 0.0f;
  a.scale_log2 = fmaxf(fabsf(scale) * kLog2e, 1.17549435e-38f);
  a.n_qt = static_cast<int>(cdiv(s_q, kPQ));
  a.units_per_bk = a.n_qt * a.g;
  a.blocks_per_bk = static_cast<int>(cdiv(a.units_per_bk, kPWaves));
  // the four-slot ring needs more LDS than a workgroup gets by default (set once per process)
  static const bool lds_ok = [] {
    auto set = [](const void* f, int bytes) {
      return hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
    };
    const bool ok = set(reinterpret_cast<const void*>(&prefill_kernel<64, false, false>), PrefillTile<64>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<64, true, false>), PrefillTile<64>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<128, false, false>), PrefillTile<128>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<128, true, false>), PrefillTile<128>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<64, false, true>), PrefillTile<64>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<64, true, true>), PrefillTile<64>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<128, false, true>), PrefillTile<128>::kLds) &&
                    set(reinterpret_cast<const void*>(&prefill_kernel<128, true, true>), PrefillTile<128>::kLds);
    (void)hipGetLastError();
    return ok;
  }();
  if (!lds_ok) {
    set_error("tai_fia_prefill: the device cannot give a workgroup %d bytes of LDS", PrefillTile<128>::kLds);
    return TAI_ERR_LAUNCH;
  }
  a.n_items = b * hkv * a.blocks_per_bk;
  const size_t need = tai_fia_prefill_workspace_size(b, s_q, hq, hkv);
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_fia_prefill: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  static const int n_cu = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    return n > 0 ? n : 256;
  }();
  a.n_queues = n_cu < kPfQueues ? n_cu : kPfQueues;
  a.queue = static_cast<int*>(workspace);
  a.flags = a.queue + 64;
  a.redo = a.flags + a.n_items;
  hipStream_t st = static_cast<hipStream_t>(stream);
  prefill_queue_reset<<<static_cast<unsigned>(std::min<int64_t>(64, cdiv(a.n_items, 256))), 256, 0, st>>>(a.queue, a.flags, a.n_items);
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(n_cu, a.n_items)));
  auto launch = [&](auto f16c) {
    constexpr bool F16 = decltype(f16c)::value;
    if (d == 64) {
      prefill_kernel<64, false, F16><<<grid, 64 * kPWaves, PrefillTile<64>::kLds, st>>>(a);
      prefill_kernel<64, true, F16><<<grid, 64 * kPWaves, PrefillTile<64>::kLds, st>>>(a);
    } else {
      prefill_kernel<128, false, F16><<<grid, 64 * kPWaves, PrefillTile<128>::kLds, st>>>(a);
      prefill_kernel<128, true, F16><<<grid, 64 * kPWaves, PrefillTile<128>::kLds, st>>>(a);
    }
  };
  if (dtype == TAI_DT_FP16) launch(std::true_type());
  else launch(std::false_type());
  return launch_status("tai_fia_prefill");
}

extern "C" size_t tai_fia_mla_decode_workspace_size(int64_t b, int hq, int dn, int64_t max_blocks, int block_size) {
  (void)max_blocks;
  (void)block_size;
  return mla_ws(b, hq, dn).total + 256;
}

extern "C" int tai_fia_mla_decode(const void* q_nope, const void* q_rope, const int8_t* ckv_cache, const float* ckv_scale,
                                  const void* krope_cache, const int32_t* block_table, int64_t max_blocks,
                                  const int64_t* seq_lens_kv, int64_t b, int hq, int dn, int dr, int block_size,
                                  float scale, void* out, float* lse, void* workspace, size_t ws_bytes, void* stream) {
  TAI_CHECK_ARG(b >= 0 && hq > 0, "tai_fia_mla_decode: bad sizes");
  TAI_UNSUPPORTED(dn != 512 || dr != 64, "tai_fia_mla_decode: only kv_lora_rank 512 with rope dim 64 is supported");
  TAI_UNSUPPORTED(block_size <= 0 || block_size % kMlaStep != 0, "tai_fia_mla_decode: block_size must be a multiple of %d",
                  kMlaStep);
  if (b == 0) return TAI_OK;
  TAI_CHECK_ARG(q_nope && q_rope && ckv_cache && ckv_scale && krope_cache && block_table && seq_lens_kv && out,
                "tai_fia_mla_decode: null pointer");
  const MlaWs lay = mla_ws(b, hq, dn);
  const size_t need = lay.total;
  if (workspace == nullptr || ws_bytes < need) {
    set_error("tai_fia_mla_decode: workspace of %zu bytes, need %zu", ws_bytes, need);
    return TAI_ERR_WORKSPACE;
  }
  MlaArgs a;
  a.qn = static_cast<const uint16_t*>(q_nope);
  a.qr = static_cast<const uint16_t*>(q_rope);
  a.ckv = ckv_cache; a.cs = ckv_scale; a.kr = static_cast<const uint16_t*>(krope_cache);
  a.bt = block_table; a.max_blocks = max_blocks; a.lens = seq_lens_kv; a.b = b; a.hq = hq; a.bs = block_size;
  a.hgroups = static_cast<int>(cdiv(hq, kMlaHeads)); a.scale_log2 = scale * kLog2e;
  char* ws = static_cast<char*>(workspace);
  a.steps = reinterpret_cast<int64_t*>(ws + lay.steps);
  a.part_o = reinterpret_cast<uint16_t*>(ws + lay.part_o);
  a.part_ml = reinterpret_cast<float*>(ws + lay.part_ml);
  a.flags = reinterpret_cast<int32_t*>(ws + lay.flags);
  a.wgflags = reinterpret_cast<int32_t*>(ws + lay.wgflags);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the LDS attribute is set once per process; a function-local static initialiser runs exactly
  // once even when several host threads reach it together
  static const bool lds_ok = [] {
    const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&mla_decode_kernel<512, 64, false>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kMlaLds) == hipSuccess &&
                    hipFuncSetAttribute(reinterpret_cast<const void*>(&mla_decode_kernel<512, 64, true>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kMlaLds) == hipSuccess;
    (void)hipGetLastError();
    return ok;
  }();
  if (!lds_ok) {
    set_error("tai_fia_mla_decode: the device cannot give a workgroup %d bytes of LDS", kMlaLds);
    return TAI_ERR_LAUNCH;
  }
  // fast pass, then the rescaling pass over the segments the fast pass flagged (it skips the others)
  const dim3 grid(kMlaWgs);
  mla_decode_kernel<512, 64, false><<<grid, 64 * kMlaWaves, kMlaLds, st>>>(a);
  mla_decode_kernel<512, 64, true><<<grid, 64 * kMlaWaves, kMlaLds, st>>>(a);
  const int64_t combine_wgs = b * ((hq + kMlaCombineHeads - 1) / kMlaCombineHeads);
  mla_combine_kernel<512><<<dim3(static_cast<unsigned>(combine_wgs)), 256, 0, st>>>(a, static_cast<uint16_t*>(out), lse);
  return launch_status("tai_fia_mla_decode");
}
