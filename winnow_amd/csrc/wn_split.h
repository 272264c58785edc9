// The vector-ALU page scan (decode_split_kernel) and its row loaders, shared by the
// source files that instantiate it: decode.hip for the width pairs the library
// tunes, decode_split_any128.hip and decode_split_any64.hip for every other pair of
// supported widths.
#pragma once

#include "wn_decode.h"

namespace wn {
namespace {

constexpr int kBlock = 256;  // 4 waves

// The bytes holding codes [8*g, 8*g+8) of a row: exactly BW bytes at byte
// offset g*BW, loaded with the widest accesses their alignment allows.
template <int BW>
__device__ __forceinline__ void load_group(const uint8_t* p, uint32_t (&v)[2]) {
  if constexpr (BW == 8) {
    uint2 x = *reinterpret_cast<const uint2*>(p);
    v[0] = x.x;
    v[1] = x.y;
  } else if constexpr (BW == 4) {
    v[0] = *reinterpret_cast<const uint32_t*>(p);
    v[1] = 0;
  } else if constexpr (BW == 2) {
    v[0] = *reinterpret_cast<const uint16_t*>(p);
    v[1] = 0;
  } else if constexpr (BW == 6) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    v[0] = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
    v[1] = h[2];
  } else if constexpr (BW == 3) {
    v[0] = uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16);
    v[1] = 0;
  } else {  // 5
    v[0] = uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24);
    v[1] = p[4];
  }
}

// A whole packed row (NB bytes, NB even) into registers, with the widest accesses
// its alignment allows (rows start at multiples of NB from an 8-byte aligned base).
template <int NB>
__device__ __forceinline__ void load_row(const uint8_t* p, uint32_t (&w)[(NB + 3) / 4]) {
  static_assert(NB % 2 == 0, "packed rows of head_dim >= 16 are whole 16-bit pieces");
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      uint4 x = reinterpret_cast<const uint4*>(p)[i];
      w[4 * i] = x.x;
      w[4 * i + 1] = x.y;
      w[4 * i + 2] = x.z;
      w[4 * i + 3] = x.w;
    }
  } else if constexpr (NB % 8 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) {
      uint2 x = reinterpret_cast<const uint2*>(p)[i];
      w[2 * i] = x.x;
      w[2 * i + 1] = x.y;
    }
  } else if constexpr (NB % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 4; ++i) w[i] = reinterpret_cast<const uint32_t*>(p)[i];
  } else {  // 6 or 10 bytes (head_dim 16 at 3 or 5 bits): 16-bit pieces
#pragma unroll
    for (int i = 0; i < (NB + 3) / 4; ++i) w[i] = 0;
#pragma unroll
    for (int i = 0; i < NB / 2; ++i) w[i >> 1] |= uint32_t(reinterpret_cast<const uint16_t*>(p)[i]) << (16 * (i & 1));
  }
}

template <int D, int BWK, int BWV, int NREP>
__global__ __launch_bounds__(kBlock) void decode_split_kernel(DecodeArgs a) {
  constexpr int NBK = D * BWK / 8;
  constexpr int NBV = D * BWV / 8;
  constexpr int G = D / 8;     // lanes per token row in the value phase (8 dims each)
  constexpr int TPS = 64 / G;  // token rows per value step
  constexpr int LK = 1 << BWK, LV = 1 << BWV;

  __shared__ float cbk[LK];
  __shared__ float cbv[LV];
  __shared__ float pw[4][64][NREP];  // p * n_V per token of the wave's chunk
  __shared__ int pidl[4][64];        // page id per token of the chunk
  __shared__ float red_m[4][NREP], red_l[4][NREP];
  __shared__ float red_acc[4][NREP][D];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int S = 1 << a.log2S;
  const int L = a.seq_lens[b];
  const int n_pages = (L + S - 1) >> a.log2S;
  const int page_lo = split * a.pages_per_split;
  if (page_lo >= n_pages) return;  // block-uniform: this split is past the sequence
  const int page_hi = min(page_lo + a.pages_per_split, n_pages);
  const int t_lo = page_lo << a.log2S;
  const int t_hi = min(page_hi << a.log2S, L);

  if (split == 0 && tid == 0)
    a.unit_meta[b * a.Hkv + kvh] =
        make_int2((b * a.Hkv + kvh) * a.num_splits, (n_pages + a.pages_per_split - 1) / a.pages_per_split);
  const int kvp = kvh / a.kvdiv;  // the kv head whose pages this (virtual) head reads
  for (int i = tid; i < LK; i += kBlock) cbk[i] = a.cb_k[i];
  for (int i = tid; i < LV; i += kBlock) cbv[i] = a.cb_v[i];
  __syncthreads();

  const float* __restrict__ qp = a.q_rot + (int64_t(b) * a.Hkv + kvh) * NREP * D;
  const int32_t* __restrict__ trow = a.table + b * a.tsb;
  const uint8_t* kbase = a.k_pages + kvp * a.ksh;
  const uint8_t* vbase = a.v_pages + kvp * a.vsh;
  const uint16_t* knb = a.k_norms + kvp * a.knh;
  const uint16_t* vnb = a.v_norms + kvp * a.vnh;

  float m[NREP], l[NREP], acc[NREP][8];
#pragma unroll
  for (int h = 0; h < NREP; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
  }
  const int tsub = lane / G, dg = lane % G;

  for (int c0 = t_lo + w * 64; c0 < t_hi; c0 += 4 * 64) {
    // ---- score phase: lane = token
    const int t = c0 + lane;
    const bool valid = t < t_hi;
    int pid = 0;
    float nv = 0.f;
    float s[NREP];
    if (valid) {
      pid = trow[t >> a.log2S];
      const int slot = t & (S - 1);
      uint32_t kw[(NBK + 3) / 4];
      load_row<NBK>(kbase + pid * a.ksp + slot * NBK, kw);
      const float nk = f16_to_f32(knb[pid * a.knp + slot]);
      nv = f16_to_f32(vnb[pid * a.vnp + slot]);
#pragma unroll
      for (int h = 0; h < NREP; ++h) s[h] = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const float c = cbk[code_at<BWK>(kw, d)];
#pragma unroll
        for (int h = 0; h < NREP; ++h) s[h] = fmaf(qp[h * D + d], c, s[h]);
      }
#pragma unroll
      for (int h = 0; h < NREP; ++h) s[h] *= nk;
    } else {
#pragma unroll
      for (int h = 0; h < NREP; ++h) s[h] = -INFINITY;
    }

    wave_lds_sync();  // the previous chunk's value phase has read pw / pidl
    float alpha[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      const float mn = fmaxf(m[h], wave_max(s[h]));  // finite: lane 0 of a chunk is valid
      alpha[h] = expf(m[h] - mn);                     // 0 on the first chunk (m = -inf)
      const float p = valid ? expf(s[h] - mn) : 0.f;
      l[h] = l[h] * alpha[h] + wave_sum(p);
      m[h] = mn;
      pw[w][lane][h] = p * nv;
    }
    pidl[w][lane] = pid;
    wave_lds_sync();

    // ---- value phase: G lanes per token row, 8 dims per lane
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= alpha[h];
#pragma unroll 2
    for (int j = 0; j < 64 / TPS; ++j) {
      const int tl = j * TPS + tsub;
      const int tt = c0 + tl;
      if (tt < t_hi) {
        const int pv = pidl[w][tl];
        uint32_t vb[2];
        load_group<BWV>(vbase + pv * a.vsp + (tt & (S - 1)) * NBV + dg * BWV, vb);
        float wv[NREP];
#pragma unroll
        for (int h = 0; h < NREP; ++h) wv[h] = pw[w][tl][h];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float c = cbv[code_at<BWV>(vb, i)];
#pragma unroll
          for (int h = 0; h < NREP; ++h) acc[h][i] = fmaf(wv[h], c, acc[h][i]);
        }
      }
    }
  }

  // Token subgroups of a wave share m: plain sums.
#pragma unroll
  for (int o = G; o < 64; o <<= 1)
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] += __shfl_xor(acc[h][i], o, 64);
  if (lane < G) {
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) red_acc[w][h][dg * 8 + i] = acc[h][i];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      red_m[w][h] = m[h];
      red_l[w][h] = l[h];
    }
  }
  __syncthreads();

  // Max-stable merge of the four waves; a wave that saw no chunk has m = -inf.
  const int64_t row0 = ((int64_t(b) * a.Hkv + kvh) * a.num_splits + split) * a.n_rep;
  for (int e = tid; e < a.n_rep * D; e += kBlock) {
    const int h = e / D, d = e % D;
    float M = red_m[0][h];
#pragma unroll
    for (int ww = 1; ww < 4; ++ww) M = fmaxf(M, red_m[ww][h]);
    float af = 0.f, lf = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float mw = red_m[ww][h];
      if (mw != -INFINITY) {
        const float sc = expf(mw - M);
        af = fmaf(sc, red_acc[ww][h][d], af);
        lf = fmaf(sc, red_l[ww][h], lf);
      }
    }
    a.part_acc[(row0 + h) * D + d] = af;
    if (d == 0) {
      a.part_ml[2 * (row0 + h)] = M;
      a.part_ml[2 * (row0 + h) + 1] = lf;
    }
  }
}

template <int D, int BWK, int BWV>
SplitFn pick_nrep(int nrep) {
  switch (nrep) {
    case 1: return decode_split_kernel<D, BWK, BWV, 1>;
    case 2: return decode_split_kernel<D, BWK, BWV, 2>;
    case 4: return decode_split_kernel<D, BWK, BWV, 4>;
    case 8: return decode_split_kernel<D, BWK, BWV, 8>;
    case 16: return decode_split_kernel<D, BWK, BWV, 16>;
  }
  return nullptr;
}

}  // namespace
}  // namespace wn
