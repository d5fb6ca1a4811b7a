// npu_fused_infer_attention_score, general path: an explicit attention mask, a bf16 / fp16 MLA
// latent, head dims the tiled kernels do not take, int8 key / value caches with their antiquant
// scales and offsets, and int8 attention_out. One wave per (sequence, query head, query
// row); a 64-token chunk of keys puts one token on each lane (its score is a dot product against the
// query, held in LDS as fp32), the chunk's softmax statistics are wave reductions, and the value rows
// are accumulated with the lane owning value dims lane, lane + 64, ... Every product and sum is fp32.
#include <type_traits>

#include "common.h"

namespace tai {
namespace {

constexpr int kGenWaves = 4;
constexpr int kGenMaxDk = 640;   // query/key dims (k1 + k2)
constexpr int kGenMaxDv = 512;   // value dims
constexpr int kGenDvPerLane = kGenMaxDv / 64;

__device__ __forceinline__ float half_to_f32(uint16_t v, bool f16) { return f16 ? f16_to_f32(v) : bf16_to_f32(v); }

struct GenArgs {
  tai_fia_general_args a;
  bool f16;
  int parts;  // waves per (sequence, head, row): 1, 2 or 4, each taking every parts-th key chunk
};

// Index of an antiquant scale: per channel (mode 0, channel c), per token (mode 1, (b, t)) or per
// cache slot (mode 2, paged caches: block_table[b][t / bs] * bs + t % bs, the MLA latent scale layout)
__device__ __forceinline__ int64_t antiquant_index(const tai_fia_general_args& a, int64_t mode, int64_t b, int64_t t,
                                                   int64_t c) {
  if (mode == 0) return c;
  if (mode == 1) return b * a.tok_stride + t;
  return static_cast<int64_t>(a.block_table[b * a.max_blocks + t / a.block_size]) * a.block_size + t % a.block_size;
}

// (x + offset) * scale of an int8 key / value element
__device__ __forceinline__ float antiquant(float x, const float* sc, const float* of, int64_t i) {
  return (x + (of ? of[i] : 0.0f)) * sc[i];
}

__device__ __forceinline__ int64_t gen_row(const tai_fia_general_args& a, const int64_t* st, int64_t b, int64_t tok, int kvh) {
  if (a.block_table) {
    int64_t tb, tr;  // tok / block_size, tok % block_size (32-bit division when both fit)
    if (tok < (int64_t(1) << 31) && a.block_size < (int64_t(1) << 31)) {
      const uint32_t t32 = static_cast<uint32_t>(tok), bs32 = static_cast<uint32_t>(a.block_size);
      tb = t32 / bs32;
      tr = t32 - static_cast<uint32_t>(tb) * bs32;
    } else {
      tb = tok / a.block_size;
      tr = tok % a.block_size;
    }
    const int64_t blk = a.block_table[b * a.max_blocks + tb];
    return blk * st[0] + tr * st[1] + kvh * st[2];
  }
  return b * st[0] + tok * st[1] + kvh * st[2];
}

// NE: value dims per lane (dv <= 64 * NE)
// lane src's 64-bit value, as two 32-bit shuffles
__device__ __forceinline__ int64_t shfl64(int64_t v, int src) {
  const uint32_t lo = static_cast<uint32_t>(__shfl(static_cast<int>(v & 0xffffffff), src, 64));
  const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(v >> 32), src, 64));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <bool KV8, int NE>
__global__ __launch_bounds__(64 * kGenWaves) void fia_general_kernel(GenArgs ga) {
  const tai_fia_general_args& a = ga.a;
  const bool f16 = ga.f16;
  __shared__ float qs[kGenWaves][kGenMaxDk];
  __shared__ float part_ml[kGenWaves][2];
  __shared__ float part_o[kGenWaves][kGenMaxDv];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // parts waves share one item; wave `part` takes key chunks part, part + parts, ... and the
  // group's first wave merges their softmax states through LDS
  const int parts = ga.parts, part = w % parts;
  // (b, h, i), i fastest; the launch's last workgroup may hold waves past the end, which run item 0
  // with no keys through the barriers and write nothing
  // workgroups are dealt to the 8 XCDs in turn: renumber them so each XCD runs a contiguous range of
  // items (a GQA group's heads, which read the same keys and values, then share one L2)
  const uint32_t nblk = gridDim.x, xcd = blockIdx.x % 8u, per = nblk / 8u;
  const uint32_t blk = xcd * per + min(xcd, nblk % 8u) + blockIdx.x / 8u;
  const int64_t item0 = static_cast<int64_t>(blk) * (kGenWaves / parts) + w / parts;
  const bool in_range = item0 < (a.q_cum ? 1 : a.b) * a.hq * a.s_q;
  const int64_t item = in_range ? item0 : 0;
  // (qb, qt): the batch and row that address query, out and lse; (b, i): the sequence and the
  // query's position in it. Batched layouts: qb = b, qt = i. Packed: qb = 0, qt = the packed row,
  // and its sequence is found in q_cum (rows past the last end have lq = 0: zeros and lse -inf).
  int64_t i = item % a.s_q, h = (item / a.s_q) % a.hq, b = item / (a.s_q * a.hq);
  const int64_t qt = i, qb = a.q_cum ? 0 : b;
  int64_t lq, kv_base = 0;
  if (a.q_cum) {
    int64_t lo = 0, hi = a.b;  // the first sequence whose end lies past qt
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (a.q_cum[mid] > qt) hi = mid; else lo = mid + 1;
    }
    if (lo < a.b) {
      const int64_t end = imin64(a.q_cum[lo], a.s_q);
      const int64_t start = lo ? imax64(0, imin64(a.q_cum[lo - 1], end)) : 0;
      b = lo;
      i = qt - start;
      lq = end - start;
    } else {
      b = 0;
      i = 0;
      lq = 0;
    }
  } else {
    lq = a.seq_lens_q ? imax64(0, imin64(a.seq_lens_q[b], a.s_q)) : a.s_q;
  }
  const int kvh = static_cast<int>(h / (a.hq / a.hkv));
  // lengths read on the device are clamped to what the inputs hold (s_q; s_kv, or the blocks a
  // block-table row can address)
  int64_t kv_cap = a.block_table ? a.max_blocks * a.block_size : a.s_kv;
  // per-token antiquant scales hold tok_stride positions per sequence
  if (KV8 && (a.k_quant_mode == 1 || a.v_quant_mode == 1)) kv_cap = imin64(kv_cap, a.tok_stride);
  int64_t lk_own;
  if (a.kv_cum) {
    const int64_t end = imax64(0, imin64(a.kv_cum[b], a.s_kv));
    kv_base = b ? imax64(0, imin64(a.kv_cum[b - 1], end)) : 0;
    lk_own = end - kv_base;
  } else {
    lk_own = a.seq_lens_kv ? imax64(0, imin64(a.seq_lens_kv[b], kv_cap)) : a.s_kv;
  }
  // a shared prefix precedes every sequence's own keys: positions [0, lp) read the prefix tensors
  const int64_t lp = a.k_prefix ? imax64(0, imin64(a.prefix_len[0], a.prefix_cap)) : 0;
  const int64_t lk = lp + lk_own;
  // own key j of the sequence is row kv_base + j (packed) of batch b
  const int64_t kb = kv_base - lp;
  const int64_t o_off = qb * a.out_strides[0] + qt * a.out_strides[1] + h * a.out_strides[2];
  const int dk = a.dk1 + a.dk2;
  const bool qq = KV8 && a.q_dtype == TAI_DT_INT8;
  // per-channel int8 keys / values with no shared prefix fold their antiquant into the query / output
  const bool fold_k = KV8 && !qq && a.k_quant_mode == 0 && !a.k_prefix;
  const bool fold_v = KV8 && !qq && a.v_quant_mode == 0 && !a.v_prefix;
  float k_bias = 0.0f;
  // the query as fp32 in this wave's LDS row
  {
    const uint16_t* q1 = static_cast<const uint16_t*>(a.q1) + qb * a.q1_strides[0] + qt * a.q1_strides[1] + h * a.q1_strides[2];
    const uint16_t* q2 = a.q2 ? static_cast<const uint16_t*>(a.q2) + qb * a.q2_strides[0] + qt * a.q2_strides[1] +
                                    h * a.q2_strides[2]
                              : nullptr;
    if (KV8 && a.q_dtype == TAI_DT_INT8) {
      const int8_t* q8 = static_cast<const int8_t*>(a.q1) + qb * a.q1_strides[0] + qt * a.q1_strides[1] +
                         h * a.q1_strides[2];
      for (int d = lane; d < dk; d += 64) qs[w][d] = static_cast<float>(q8[d]);
    } else if (fold_k) {
      // per-channel int8 keys: q.((k + off) * sc) = (q * sc).k + sum(q * sc * off), the scale folded
      // into the query once per row
      float kb = 0.0f;
      for (int d = lane; d < dk; d += 64) {
        float x = d < a.dk1 ? half_to_f32(q1[d], f16) : half_to_f32(q2[d - a.dk1], f16);
        if (d < a.dk1) {
          const int64_t c = static_cast<int64_t>(kvh) * a.dk1 + d;
          x *= a.k_scale[c];
          if (a.k_offset) kb += x * a.k_offset[c];
        }
        qs[w][d] = x;
      }
      k_bias = wave_sum(kb);
    } else {
      for (int d = lane; d < dk; d += 64) qs[w][d] = d < a.dk1 ? half_to_f32(q1[d], f16) : half_to_f32(q2[d - a.dk1], f16);
    }
  }
  __syncthreads();  // (each wave reads only its own row; the barrier orders the LDS writes)
  // visible kv range of query i
  const int64_t off = a.mask_origin ? lk - lq : 0;
  const int64_t hi = in_range && i < lq ? imin64(lk, i + off + a.next_tokens + 1) : 0;
  const int64_t lo = imax64(0, i + off - a.pre_tokens);
  float m = -INFINITY, l = 0.0f;
  float o[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) o[e] = 0.0f;
  const uint16_t* k1 = static_cast<const uint16_t*>(a.k1);
  const uint16_t* k2 = static_cast<const uint16_t*>(a.k2);
  const uint16_t* vv = static_cast<const uint16_t*>(a.v);
  if (qq) {
    // int8 query, key and value: two passes over the visible keys, the first for the row max and sum,
    // the second quantising P against the final max (so the result does not depend on the chunking) and
    // accumulating P8.V exactly in int32. Each score's q.k sum is of integer products below 2^24 in
    // magnitude, exact in fp32 in any order.
    auto score = [&](int64_t j, bool& valid) -> float {
      valid = j < hi;
      if (valid && a.mask) valid = a.mask[b * a.mask_strides[0] + i * a.mask_strides[1] + j * a.mask_strides[2]] == 0;
      if (!valid) return -INFINITY;
      const int8_t* kr = static_cast<const int8_t*>(a.k1) + gen_row(a, a.k1_strides, b, j + kb, kvh);
      float acc = 0.0f;
      for (int d = 0; d < a.dk1; d += 8) {
        const uint2 u = *reinterpret_cast<const uint2*>(kr + d);
        const uint32_t wd[2] = {u.x, u.y};
#pragma unroll
        for (int q = 0; q < 8; ++q)
          acc += static_cast<float>(static_cast<int8_t>((wd[q >> 2] >> (8 * (q & 3))) & 0xffu)) * qs[w][d + q];
      }
      return __fmul_rn(__fmul_rn(acc, a.deq_scale1[0]), a.scale);
    };
    for (int64_t t0 = lo; t0 < hi; t0 += 64) {
      bool valid;
      const float s = score(t0 + lane, valid);
      const float mc = wave_max(s);
      if (mc == -INFINITY) continue;
      const float m_new = fmaxf(m, mc);
      l = l * (m == -INFINITY ? 0.0f : expf(m - m_new)) + wave_sum(valid ? expf(s - m_new) : 0.0f);
      m = m_new;
    }
    int32_t oi[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) oi[e] = 0;
    const float qs1 = a.quant_scale1[0];
    for (int64_t t0 = lo; t0 < hi && m != -INFINITY; t0 += 64) {
      bool valid;
      const float s = score(t0 + lane, valid);
      const int p8 = valid ? static_cast<int>(fminf(fmaxf(rintf(__fmul_rn(expf(s - m), qs1)), 0.0f), 127.0f)) : 0;
      const int64_t nj = imin64(64, hi - t0);
      const int64_t vrow = t0 + lane < hi ? gen_row(a, a.v_strides, b, t0 + lane + kb, kvh) : 0;
      for (int jj = 0; jj < nj; ++jj) {
        const int pj = __shfl(p8, jj, 64);
        if (pj == 0) continue;  // masked or rounded to zero (wave-uniform)
        const int8_t* vr = static_cast<const int8_t*>(a.v) + shfl64(vrow, jj);
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          const int d = lane + 64 * e;
          if (d < a.dv) oi[e] += pj * static_cast<int32_t>(vr[d]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < NE; ++e) o[e] = __fmul_rn(static_cast<float>(oi[e]), a.deq_scale2[0]);
  } else
  for (int64_t t0 = lo + 64 * part; t0 < hi; t0 += 64 * parts) {
    const int64_t j = t0 + lane;
    bool valid = j < hi;
    // this lane's token's value row, handed to every lane of the P V loop by shuffles
    const int64_t vrow = j < hi && j >= lp ? gen_row(a, a.v_strides, b, j + kb, kvh) : 0;
    if (valid && a.mask) valid = a.mask[b * a.mask_strides[0] + i * a.mask_strides[1] + j * a.mask_strides[2]] == 0;
    float s = -INFINITY;
    if (valid) {
      float acc = 0.0f;
      // int8 own keys (shared-prefix rows, j < lp, stay in the query's dtype)
      if (KV8 && j >= lp) {
        const int8_t* kr = static_cast<const int8_t*>(a.k1) + gen_row(a, a.k1_strides, b, j + kb, kvh);
        for (int d0 = 0; d0 < a.dk1; d0 += 64) {
          // 64 dims at a time: the eight 8-byte loads go out before their products
          uint2 uu[8];
#pragma unroll
          for (int g = 0; g < 8; ++g)
            uu[g] = d0 + 8 * g < a.dk1 ? *reinterpret_cast<const uint2*>(kr + d0 + 8 * g) : make_uint2(0, 0);
#pragma unroll
          for (int g = 0; g < 8; ++g) {
            const int d = d0 + 8 * g;
            if (d >= a.dk1) continue;
            const uint32_t wd[2] = {uu[g].x, uu[g].y};
            if (fold_k) {
#pragma unroll
              for (int q = 0; q < 8; ++q)
                acc += static_cast<float>(static_cast<int8_t>((wd[q >> 2] >> (8 * (q & 3))) & 0xffu)) * qs[w][d + q];
            } else {
#pragma unroll
              for (int q = 0; q < 8; ++q) {
                const float x = static_cast<float>(static_cast<int8_t>((wd[q >> 2] >> (8 * (q & 3))) & 0xffu));
                acc += antiquant(x, a.k_scale, a.k_offset,
                                 antiquant_index(a, a.k_quant_mode, b, j - lp,
                                                 static_cast<int64_t>(kvh) * a.dk1 + d + q)) *
                       qs[w][d + q];
              }
            }
          }
        }
        acc += k_bias;
      } else {
        const uint16_t* kr = j < lp ? static_cast<const uint16_t*>(a.k_prefix) + j * a.k_prefix_strides[0] +
                                          kvh * a.k_prefix_strides[1]
                                    : k1 + gen_row(a, a.k1_strides, b, j + kb, kvh);
        // 64 dims at a time: the eight 16-byte loads go out before their products
        for (int d0 = 0; d0 < a.dk1; d0 += 64) {
          uint4 u[8];
#pragma unroll
          for (int g = 0; g < 8; ++g)
            u[g] = d0 + 8 * g < a.dk1 ? *reinterpret_cast<const uint4*>(kr + d0 + 8 * g) : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int g = 0; g < 8; ++g) {
            if (d0 + 8 * g < a.dk1) {
              const int d = d0 + 8 * g;
              const uint32_t wd[4] = {u[g].x, u[g].y, u[g].z, u[g].w};
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                acc += half_to_f32(static_cast<uint16_t>(wd[q] & 0xffffu), f16) * qs[w][d + 2 * q];
                acc += half_to_f32(static_cast<uint16_t>(wd[q] >> 16), f16) * qs[w][d + 2 * q + 1];
              }
            }
          }
        }
      }
      if (a.dk2) {
        const uint16_t* kr2 = k2 + gen_row(a, a.k2_strides, b, j + kb, kvh);
        for (int d = 0; d < a.dk2; ++d) acc += half_to_f32(kr2[d], f16) * qs[w][a.dk1 + d];
      }
      s = acc * a.scale;
      if (a.pse)
        s += half_to_f32(static_cast<const uint16_t*>(a.pse)[b * a.pse_strides[0] + h * a.pse_strides[1] +
                                                              i * a.pse_strides[2] + j * a.pse_strides[3]],
                         f16);
    }
    const float mc = wave_max(s);
    if (mc == -INFINITY) continue;  // nothing visible in this chunk
    const float m_new = fmaxf(m, mc);
    const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
    const float p = valid ? expf(s - m_new) : 0.0f;
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int e = 0; e < NE; ++e) o[e] *= alpha;
    // P V, eight tokens at a time: the eight value rows' loads go out together before their products
    // (one token at a time, each load waited out its own latency). Every token below nj lies inside
    // the sequence, so its row is read even when its P is zero (a masked token adds 0 * v, no change).
    const int nj = static_cast<int>(imin64(64, hi - t0));
    constexpr int kU = 8;
    for (int jj = 0; jj < nj; jj += kU) {
      float pv[kU];
      float val[kU][NE];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const bool in = jj + u < nj;
        const int src = in ? jj + u : 0;
        pv[u] = __shfl(p, src, 64);
        const int64_t t = t0 + src;
        const int64_t vr_off = shfl64(vrow, src);
        if (KV8 && t >= lp) {
          const int8_t* vr = static_cast<const int8_t*>(a.v) + vr_off;
#pragma unroll
          for (int e = 0; e < NE; ++e) {
            const int d = lane + 64 * e;
            val[u][e] = d >= a.dv ? 0.0f
                        : fold_v ? static_cast<float>(vr[d])
                                 : antiquant(static_cast<float>(vr[d]), a.v_scale, a.v_offset,
                                             antiquant_index(a, a.v_quant_mode, b, t - lp,
                                                             static_cast<int64_t>(kvh) * a.dv + d));
          }
        } else {
          const uint16_t* vr = t < lp ? static_cast<const uint16_t*>(a.v_prefix) + t * a.v_prefix_strides[0] +
                                            kvh * a.v_prefix_strides[1]
                                      : vv + vr_off;
#pragma unroll
          for (int e = 0; e < NE; ++e) {
            const int d = lane + 64 * e;
            val[u][e] = d < a.dv ? half_to_f32(vr[d], f16) : 0.0f;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (jj + u < nj) {
#pragma unroll
          for (int e = 0; e < NE; ++e) o[e] += pv[u] * val[u][e];
        }
      }
    }
    m = m_new;
  }
  if (parts > 1) {
    if (lane == 0) {
      part_ml[w][0] = m;
      part_ml[w][1] = l;
    }
#pragma unroll
    for (int e = 0; e < NE; ++e) part_o[w][lane + 64 * e] = o[e];
    __syncthreads();
    if (part == 0) {
      float mm = -INFINITY;
      for (int p = 0; p < parts; ++p) mm = fmaxf(mm, part_ml[w + p][0]);
      l = 0.0f;
#pragma unroll
      for (int e = 0; e < NE; ++e) o[e] = 0.0f;
      for (int p = 0; p < parts; ++p) {
        const float mp = part_ml[w + p][0];
        const float f = mp == -INFINITY ? 0.0f : expf(mp - mm);
        l += part_ml[w + p][1] * f;
#pragma unroll
        for (int e = 0; e < NE; ++e) o[e] += part_o[w + p][lane + 64 * e] * f;
      }
      m = mm;
    }
  }
  if (!in_range || part != 0) return;
  if (fold_v) {
    // sum p (v + off) sc = (sum p v + off l) sc, per value channel
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int d = lane + 64 * e;
      if (d < a.dv) {
        const int64_t c = static_cast<int64_t>(kvh) * a.dv + d;
        o[e] = (o[e] + (a.v_offset ? a.v_offset[c] * l : 0.0f)) * a.v_scale[c];
      }
    }
  }
  if (a.sink && i < lq && a.sink[h] != -INFINITY) {
    // the sink joins the denominator: the reference max and the sum take it in, O gains nothing
    const float sv = a.sink[h];
    const float m2 = fmaxf(m, sv);
    const float alpha = m == -INFINITY ? 0.0f : expf(m - m2);
#pragma unroll
    for (int e = 0; e < NE; ++e) o[e] *= alpha;
    l = l * alpha + expf(sv - m2);
    m = m2;
  }
  const bool live = i < lq && l > 0.0f;
  const float inv = live ? 1.0f / l : 0.0f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const int d = lane + 64 * e;
    if (d < a.dv) {
      const float r = o[e] * inv;
      if (a.out_dtype == TAI_DT_INT8) {
        // quant_scale2 / quant_offset2: rint(o * scale + offset) saturated to int8
        const int64_t c = a.out_scale_len == 1 ? 0 : h * a.dv + d;
        const float y = __fadd_rn(__fmul_rn(r, a.out_scale[c]), a.out_offset ? a.out_offset[c] : 0.0f);
        static_cast<int8_t*>(a.out)[o_off + d] = static_cast<int8_t>(static_cast<int>(fminf(fmaxf(rintf(y), -128.0f), 127.0f)));
      } else {
        static_cast<uint16_t*>(a.out)[o_off + d] = f16 ? f32_to_f16(r) : f32_to_bf16(r);
      }
    }
  }
  if (a.lse && lane == 0)
    a.lse[a.q_cum ? qt * a.hq + h : (b * a.hq + h) * a.s_q + i] = live ? m + logf(l) : -INFINITY;
}

}  // namespace
}  // namespace tai

using namespace tai;

extern "C" size_t tai_fia_general_args_size(void) { return sizeof(tai_fia_general_args); }

extern "C" int tai_fia_general(const tai_fia_general_args* args, void* stream) {
  TAI_CHECK_ARG(args != nullptr, "tai_fia_general: null arguments");
  const tai_fia_general_args& a = *args;
  TAI_CHECK_ARG(a.dtype == TAI_DT_BF16 || a.dtype == TAI_DT_FP16, "tai_fia_general: dtype %d not supported (bf16, fp16)",
                a.dtype);
  TAI_CHECK_ARG(a.b >= 0 && a.s_q >= 0 && a.s_kv >= 0 && a.hq > 0 && a.hkv > 0 && a.hq % a.hkv == 0,
                "tai_fia_general: bad sizes or head counts");
  TAI_CHECK_ARG(a.dk1 > 0 && a.dk1 % 8 == 0 && a.dk2 >= 0 && a.dk1 + a.dk2 <= kGenMaxDk && a.dv > 0 && a.dv <= kGenMaxDv,
                "tai_fia_general: key dims (%d + %d) must be a multiple of 8 and at most %d in all, value dims at most %d",
                a.dk1, a.dk2, kGenMaxDk, kGenMaxDv);
  TAI_CHECK_ARG(a.dk2 == 0 || (a.q2 && a.k2), "tai_fia_general: a second key part needs q2 and k2");
  TAI_CHECK_ARG(a.mask_origin == 0 || a.mask_origin == 1, "tai_fia_general: mask_origin must be 0 or 1");
  TAI_CHECK_ARG(a.block_table == nullptr || (a.block_size > 0 && a.max_blocks > 0 && a.seq_lens_kv),
                "tai_fia_general: paged K/V need block_size, max_blocks and seq_lens_kv");
  if (a.b == 0 || a.s_q == 0) return TAI_OK;
  TAI_CHECK_ARG(a.q1 && a.k1 && a.v && a.out, "tai_fia_general: null pointer");
  const bool kv8 = a.kv_dtype == TAI_DT_INT8;
  TAI_CHECK_ARG(a.kv_dtype == 0 || kv8, "tai_fia_general: kv_dtype %lld not supported (0 or int8)",
                static_cast<long long>(a.kv_dtype));
  TAI_CHECK_ARG(a.out_dtype == 0 || a.out_dtype == TAI_DT_INT8, "tai_fia_general: out_dtype %lld not supported (0 or "
                "int8)", static_cast<long long>(a.out_dtype));
  const bool qq = a.q_dtype == TAI_DT_INT8;
  TAI_CHECK_ARG(a.q_dtype == 0 || qq, "tai_fia_general: q_dtype %lld not supported (0 or int8)",
                static_cast<long long>(a.q_dtype));
  TAI_CHECK_ARG(!qq || (kv8 && a.deq_scale1 && a.quant_scale1 && a.deq_scale2 && !a.k_scale && !a.v_scale &&
                        a.dk2 == 0 && !a.k_prefix && !a.pse && !a.sink),
                "tai_fia_general: an int8 query needs int8 key / value without antiquant scales, the three "
                "scales, one key part, no shared prefix, pse or sink");
  TAI_CHECK_ARG(a.kv_cum == nullptr || (a.q_cum && !a.block_table),
                "tai_fia_general: packed keys (kv_cum) go with packed queries (q_cum) and dense keys");
  TAI_CHECK_ARG(a.kv_cum == nullptr || !kv8 || (a.k_quant_mode == 0 && a.v_quant_mode == 0),
                "tai_fia_general: packed int8 keys take per-channel antiquant scales");
  if (kv8) {
    TAI_CHECK_ARG(qq || (a.k_scale && a.v_scale), "tai_fia_general: int8 key / value need k_scale and v_scale");
    TAI_CHECK_ARG(a.k_quant_mode >= 0 && a.k_quant_mode <= 2 && a.v_quant_mode >= 0 && a.v_quant_mode <= 2,
                  "tai_fia_general: antiquant modes must be 0 (per channel), 1 (per token) or 2 (per cache slot)");
    TAI_CHECK_ARG((a.k_quant_mode != 2 && a.v_quant_mode != 2) || a.block_table,
                  "tai_fia_general: per-slot antiquant scales need a paged cache");
    TAI_CHECK_ARG((a.k_quant_mode != 1 && a.v_quant_mode != 1) || a.tok_stride > 0,
                  "tai_fia_general: per-token scales need tok_stride > 0");
  }
  TAI_CHECK_ARG(a.k_prefix == nullptr || (a.v_prefix && a.prefix_len && a.dk2 == 0),
                "tai_fia_general: a shared prefix needs v_prefix and prefix_len and one key part");
  TAI_CHECK_ARG(a.k_prefix == nullptr || ((reinterpret_cast<uintptr_t>(a.k_prefix) % 16) == 0 &&
                                          a.k_prefix_strides[0] % 8 == 0 && a.k_prefix_strides[1] % 8 == 0),
                "tai_fia_general: shared-prefix key rows must be 16-byte aligned");
  if (a.out_dtype == TAI_DT_INT8)
    TAI_CHECK_ARG(a.out_scale && (a.out_scale_len == 1 || a.out_scale_len == a.hq * a.dv),
                  "tai_fia_general: int8 out needs out_scale of 1 or hq * dv entries");
  const int kalign = kv8 ? 8 : 16, kel = 8;
  TAI_CHECK_ARG((reinterpret_cast<uintptr_t>(a.k1) % kalign) == 0 && a.k1_strides[0] % kel == 0 &&
                    a.k1_strides[1] % kel == 0 && a.k1_strides[2] % kel == 0,
                "tai_fia_general: key rows must be %d-byte aligned", kalign);
  GenArgs ga{a, a.dtype == TAI_DT_FP16, 1};
  // pre / next at or beyond 2^40 tokens are no bound
  constexpr int64_t kNoBound = int64_t(1) << 40;
  ga.a.pre_tokens = imin64(imax64(a.pre_tokens, -kNoBound), kNoBound);
  ga.a.next_tokens = imin64(imax64(a.next_tokens, -kNoBound), kNoBound);
  const int64_t items = (a.q_cum ? 1 : a.b) * a.hq * a.s_q;
  // few items over long key ranges: split each item's keys over 2 or 4 waves (the int8-query
  // path's two passes need the whole row's max first and keep one wave per item)
  const int64_t kv_span = (a.block_table ? a.max_blocks * a.block_size : a.s_kv) + (a.k_prefix ? a.prefix_cap : 0);
  if (!qq && kv_span >= 256) ga.parts = items <= 4096 ? 4 : items <= 16384 ? 2 : 1;
  const dim3 grid(static_cast<unsigned>(cdiv(items, kGenWaves / ga.parts)));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](auto ne) {
    constexpr int NE = decltype(ne)::value;
    if (kv8) fia_general_kernel<true, NE><<<grid, 64 * kGenWaves, 0, st>>>(ga);
    else fia_general_kernel<false, NE><<<grid, 64 * kGenWaves, 0, st>>>(ga);
  };
  if (a.dv <= 128) launch(std::integral_constant<int, 2>{});
  else if (a.dv <= 256) launch(std::integral_constant<int, 4>{});
  else launch(std::integral_constant<int, kGenDvPerLane>{});
  return launch_status("tai_fia_general");
}
