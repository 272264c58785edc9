// Fused prefill attention over paged packed K/V for gfx950: Q > 1 queries per
// sequence under the offset causal mask, head_dim 128, 4 and 6-bit K and V.
//
// Replaces the reference's Q > 1 route, _reconstruct_sdpa
// (turboquant_kv/packed_backend.py:211-226, reached at :278-280), which writes each
// history back to HBM dequantized and then runs SDPA. Here the pages are read in
// their packed form and the history is never expanded: the algebra is the
// compressed-domain one of the decode (turboquant_kv/packed_attention.py:260-334)
// with a query block per wave, and the mask is the reference's: query i of a
// sequence of length L (the cache already holds the Q new tokens) sees keys
// j <= L - Q + i (packed_attention.py:198-206); a query that sees no key gives 0.
//
// Three launches on the caller's stream:
//   1. pf_rotate_kernel  q_rot = scale log2(e) q Pi_K^T, one row per (sequence, kv
//                        head, r) with r = qi n_rep + h (query qi, head h of the
//                        group), rows padded to kRowPad per kv head with zeros;
//   2. pf_scan_kernel    one wave per (sequence, kv head, column block, split): the
//                        block's 16 NCT query rows against the split's share of the
//                        64-token chunks the block can see, on
//                        v_mfma_f32_16x16x32_f16 with single fp16 operands (11
//                        significant bits, rounded to nearest) and fp32 accumulation;
//                        writes an (acc, m, l) partial per row;
//   3. pf_merge_kernel   per row, the max-stable merge of its splits, 1/l, Pi_V, cast.
//
// The scan, per 64-token chunk (lane 16g + c):
//   scores  S[token, row] with A = K table entries (row c of tile t = token 16t + c,
//           k-slots of group g in K-step s = dims 32g + 8s + 0..7: quarter g of the
//           token's packed row, four pair lookups) and B = q' (column c = query row c
//           of column tile ct, the same dims). One A operand feeds NCT MFMAs. Output
//           lane (g, c) register i holds token 16t + 4g + i of column c.
//   softmax per column (query row), log2 units, lazy reference maximum (moves only
//           when a score exceeds it by more than kPfRescale): the column maximum is
//           the lane's sixteen scores, then two cross-lane steps over g.
//   values  O[dim, row] with A = V table entries (row c of M-tile mt = dim 8c + mt;
//           k-slots of group g in K-step ks = tokens 32ks + 4g + 0..3 and 32ks + 16 +
//           4g + 0..3, the token pairs' codes merged into pair indices) and B = the
//           fp16 p n_V 2^-gs of the same tokens, which are this lane's own score
//           registers: P never leaves the registers. Output lane (g, c) register i of
//           M-tile mt holds dim 32g + 8i + mt of column c.
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "wn_common.h"
#include "wn_tables.h"

namespace wn {
namespace {

constexpr float kPfRescale = 8.0f;
constexpr int kRowPad = 64;    // q_rot rows per (sequence, kv head) are a multiple of this
constexpr int kRotRows = 32;   // rows per work-group of the rotate and merge kernels

struct PrefillArgs {
  const float* q_rot;  // (B*Hkv*nrp, 128)
  const uint8_t* k_pages;
  const uint8_t* v_pages;
  const uint16_t* k_norms;
  const uint16_t* v_norms;
  const float* cb_k;
  const float* cb_v;
  const int32_t* table;
  const int32_t* seq_lens;
  float* part_acc;  // (items * 16 NCT, 128), item = ((b*Hkv + kvh)*nsplit + s)*ncb + cb
  float* part_ml;   // (items * 16 NCT, 2): maximum (log2 units), sum
  int64_t ksp, ksh, vsp, vsh;  // page strides, bytes
  int64_t knp, knh, vnp, vnh;  // norm strides, elements
  int64_t tsb;                 // page-table row stride, elements
  int B, Hkv, n_rep, Q, nrp, ncb, nsplit, log2S;
};

// The four 16-token tiles of chunk [c0, c0+64): page ids (wave-uniform) and in-page
// slots. A tile's 16 tokens share a page (16 | c0 and S >= 16); its page-table column
// is clamped to col_hi, the range's last page (tokens past the range are read from
// real pages and masked).
struct PfTiles {
  uint32_t pid[4];
  uint32_t slot[4];
};

__device__ __forceinline__ PfTiles pf_tiles(const PrefillArgs& a, const int32_t* trow, int c0, int col_hi) {
  PfTiles o;
  const int smask = (1 << a.log2S) - 1;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int t0 = c0 + 16 * t;
    // the page table is not written while the scan runs: const_view keeps these
    // wave-uniform reads scalar loads (the pacing word's LDS store would otherwise
    // make the compiler read them with vector loads and wait on them)
    o.pid[t] = uint32_t(__builtin_amdgcn_readfirstlane(const_view(trow)[min(t0 >> a.log2S, col_hi)]));
    o.slot[t] = uint32_t(t0 & smask);
  }
  return o;
}

// K rows: tile t, quarter g of token c0 + 16t + c (words [t BWK, t BWK + BWK)).
template <int BWK>
struct PfK {
  uint32_t w[4 * BWK];
};
// V rows: token (t, i) = c0 + 16t + 4g + i, codes of dims 8c .. 8c+7 (6-bit: the raw
// 8-byte window from 6c rounded down to 4), VW words each.
template <int BWV>
struct PfV {
  static constexpr int VW = BWV == 4 ? 1 : 2;
  uint32_t w[16 * VW];
};
// fp16 norms of tokens (t, i): half i & 1 of word 2t + (i >> 1).
struct PfN {
  uint32_t nk[8], nv[8];
};

template <int BWK>
__device__ __forceinline__ void pf_load_k(const PrefillArgs& a, const PfTiles& tl, int kvh, int lane, PfK<BWK>& o) {
  constexpr int NBK = 16 * BWK;
  const int g = lane >> 4, c = lane & 15;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint8_t* kp = a.k_pages + uint64_t(tl.pid[t]) * uint64_t(a.ksp) + uint64_t(kvh) * uint64_t(a.ksh) +
                        (tl.slot[t] + uint32_t(c)) * uint32_t(NBK) + uint32_t(4 * BWK * g);
    if constexpr (BWK == 4) {
      const uint4 x = *reinterpret_cast<const uint4*>(kp);
      o.w[4 * t] = x.x;
      o.w[4 * t + 1] = x.y;
      o.w[4 * t + 2] = x.z;
      o.w[4 * t + 3] = x.w;
    } else {
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const uint2 x = reinterpret_cast<const uint2*>(kp)[j];
        o.w[6 * t + 2 * j] = x.x;
        o.w[6 * t + 2 * j + 1] = x.y;
      }
    }
  }
}

template <int BWV>
__device__ __forceinline__ void pf_load_v(const PrefillArgs& a, const PfTiles& tl, int kvh, int lane, PfV<BWV>& o) {
  constexpr int NBV = 16 * BWV, VW = PfV<BWV>::VW;
  const int g = lane >> 4, c = lane & 15;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint8_t* vb = a.v_pages + uint64_t(tl.pid[t]) * uint64_t(a.vsp) + uint64_t(kvh) * uint64_t(a.vsh) +
                        (tl.slot[t] + uint32_t(4 * g)) * uint32_t(NBV);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (BWV == 4) {
        o.w[4 * t + i] = *reinterpret_cast<const uint32_t*>(vb + i * NBV + 4 * c);
      } else {
        uint2 x;
        __builtin_memcpy(&x, __builtin_assume_aligned(vb + i * NBV + ((6 * c) & ~3), 4), 8);
        o.w[VW * (4 * t + i)] = x.x;
        o.w[VW * (4 * t + i) + 1] = x.y;
      }
    }
  }
}

__device__ __forceinline__ void pf_load_n(const PrefillArgs& a, const PfTiles& tl, int kvh, int lane, PfN& o) {
  const int g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t ns = tl.slot[t] + uint32_t(4 * g);
    const uint2 nk = *reinterpret_cast<const uint2*>(a.k_norms + uint64_t(tl.pid[t]) * uint64_t(a.knp) +
                                                     uint64_t(kvh) * uint64_t(a.knh) + ns);
    const uint2 nv = *reinterpret_cast<const uint2*>(a.v_norms + uint64_t(tl.pid[t]) * uint64_t(a.vnp) +
                                                     uint64_t(kvh) * uint64_t(a.vnh) + ns);
    o.nk[2 * t] = nk.x;
    o.nk[2 * t + 1] = nk.y;
    o.nv[2 * t] = nv.x;
    o.nv[2 * t + 1] = nv.y;
  }
}

__device__ __forceinline__ float half_at(const uint32_t* w, int k) {
  return f16_to_f32(uint16_t(w[k >> 1] >> (16 * (k & 1))));
}

// The V rows' token pairs (2p, 2p+1) rewritten in place so that one word per (pair,
// dim parity) holds the pair indices: 4-bit, the byte of dims (2j, 2j+1) becomes
// (first token's code of dim 2j, second's) in the first word and the same for dim
// 2j+1 in the second; 6-bit, the raw windows are moved down to the codes and the pair
// becomes (Ce, Co), Ce holding the first token's even-numbered codes with the second's
// shifted up one field into the gaps, Co the same for the odd ones (pair index of dim
// m: the 12 bits of Ce (m even) or Co (m odd) from bit 6 m).
template <int BWV>
__device__ __forceinline__ void pf_merge_pairs(PfV<BWV>& o, int lane) {
  if constexpr (BWV == 4) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t wa = o.w[2 * p], wb = o.w[2 * p + 1];
      o.w[2 * p] = bitsel(0x0F0F0F0Fu, wa, wb << 4);
      o.w[2 * p + 1] = bitsel(0x0F0F0F0Fu, wa >> 4, wb);
    }
  } else {
    constexpr uint64_t E = 0x03F03F03F03Full;    // fields 0, 2, 4, 6 of 6 bits
    constexpr uint64_t O = ~E & 0xFFFFFFFFFFFFull;  // fields 1, 3, 5, 7
    const uint32_t sh = 16u * uint32_t(lane & 1);
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      uint32_t* x = o.w + 2 * (2 * p);
      uint32_t* y = o.w + 2 * (2 * p + 1);
      const uint64_t a = (uint64_t(x[1]) << 32 | x[0]) >> sh;
      const uint64_t b = (uint64_t(y[1]) << 32 | y[0]) >> sh;
      const uint64_t bs = b << 6;
      const uint64_t ce = (a & E) | (bs & ~E);
      const uint64_t co = (a & O) | (bs & ~O);
      x[0] = uint32_t(ce);
      x[1] = uint32_t(ce >> 32);
      y[0] = uint32_t(co);
      y[1] = uint32_t(co >> 32);
    }
  }
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

template <int NCT>
struct PfState {
  f32x4 acc[NCT][8];  // acc[ct][mt] register i: dim 32g + 8i + mt of column c, scaled by 2^(8-gs)
  float m[NCT];       // reference maximum of column c (log2 units; -inf before its first key)
  float l[NCT];       // sum of 2^(s - m) over this lane's tokens
  int lim[NCT];       // last visible token of column c (padding rows: no limit)
  int gs;             // value scale shift (wave-uniform)
};

constexpr int kPfLookahead = 4;  // K-steps of table reads in flight ahead of their MFMA

// Scores of the chunk: d[ct][t] register i = token 16t + 4g + i of column c, before
// the n_K 2^-(e+8) scale. Step k = 4s + t (K-step s of tile t); one A operand (four
// pair lookups) feeds NCT MFMAs.
template <int BWK, int NCT>
__device__ __forceinline__ void pf_scores(const PfK<BWK>& K, TabTf<BWK>& cbk, const h8 (&qb)[NCT][4],
                                          f32x4 (&d)[NCT][4]) {
  constexpr int LA = kPfLookahead;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int t = 0; t < 4; ++t) d[ct][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // the four entries of a step land in one 4-register operand (no moves to assemble it)
  u32x4 e[LA + 1];
  auto look = [&](auto kc, u32x4& o) {
    constexpr int k = decltype(kc)::value, s = k >> 2, t = k & 3;
    o[0] = piece_pair_tf<BWK, 4 * s>(K.w + t * BWK, cbk);
    o[1] = piece_pair_tf<BWK, 4 * s + 1>(K.w + t * BWK, cbk);
    o[2] = piece_pair_tf<BWK, 4 * s + 2>(K.w + t * BWK, cbk);
    o[3] = piece_pair_tf<BWK, 4 * s + 3>(K.w + t * BWK, cbk);
  };
  // the schedule is pinned step by step (sched_barrier): left free, the compiler
  // hoists every table read to the top and runs out of registers
  static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 16>([&](auto kc) {
    constexpr int k = decltype(kc)::value, s = k >> 2, t = k & 3, j = k % (LA + 1);
    if constexpr (k + LA < 16) {
      look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
    const h8 av = __builtin_bit_cast(h8, e[j]);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) d[ct][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qb[ct][s], d[ct][t], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Online softmax of the chunk per column, p n_V 2^-gs into the value B operands:
// K-step ks of column tile ct takes tokens (2ks, i) at k-slots i and (2ks + 1, i) at
// k-slots 4 + i, this lane's own score registers. Score register i of tile t is token
// c0 + 16t + 4g + i, or with TILED (the shared-tile scan's order) c0 + 32(t >> 1) +
// 8g + 4(t & 1) + i; norms word 2t + (i >> 1) holds its n_K, n_V either way. full:
// every token of the chunk is visible to every column (no masks); else a token of
// column c is visible when it is <= min(lim[c], t_hi - 1).
template <int NCT, bool TILED = false>
__device__ __forceinline__ void pf_softmax(const f32x4 (&d)[NCT][4], const PfN& N, float sc, int c0, int t_hi,
                                           bool full, int lane, PfState<NCT>& st, h8 (&pb)[NCT][2]) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const int g = lane >> 4;
  // value scale: every n_V < 2^(7 + gs), so 2^kPfRescale n_V 2^-gs < 2^15 in fp16.
  // Norms are non-negative fp16, which order as their bit patterns: a packed u16 max.
  uint32_t nvm = N.nv[0];
#pragma unroll
  for (int w = 1; w < 8; ++w) nvm = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(
                                        __builtin_bit_cast(u16x2, nvm), __builtin_bit_cast(u16x2, N.nv[w])));
  const float nvmax = fmaxf(half_at(&nvm, 0), half_at(&nvm, 1));
  if (__any(nvmax >= ldexpf(1.f, 7 + st.gs))) {  // wave-uniform, rare
    int ge;
    frexpf(wave_max(nvmax), &ge);
    const int gs_need = max(0, ge - 7);
    const float f = ldexpf(1.f, st.gs - gs_need);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) st.acc[ct][mt] *= f;
    st.gs = gs_need;
  }
  // n_V 2^-gs of tokens (k, k+1), k even, as an fp16 pair (the stored pair, scaled exactly)
  const _Float16 vsc = _Float16(ldexpf(1.f, -st.gs));
  h2 nv2[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) nv2[w] = __builtin_bit_cast(h2, N.nv[w]) * h2{vsc, vsc};
  float nks[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) nks[k] = half_at(N.nk, k) * sc;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    // u = s - m0 with m0 the reference maximum (0 before the column's first key)
    const bool fresh = st.m[ct] == -INFINITY;
    const float m0 = fresh ? 0.f : st.m[ct];
    // token (t, i) visible: its offset from the lane's base is <= lim
    const int lim = min(st.lim[ct], t_hi - 1) - (c0 + (TILED ? 8 : 4) * g);
    float u[16], umax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = fmaf(d[ct][t][i], nks[4 * t + i], -m0);
        const int off = TILED ? 32 * (t >> 1) + 4 * (t & 1) + i : 16 * t + i;
        u[4 * t + i] = (full || off <= lim) ? x : -INFINITY;
        umax = fmaxf(umax, u[4 * t + i]);
      }
    umax = fmaxf(umax, __shfl_xor(umax, 16, 64));
    umax = fmaxf(umax, __shfl_xor(umax, 32, 64));
    // the reference moves to the chunk's maximum when a score exceeds it by more than
    // kPfRescale, and on the column's first key
    const bool move = umax > kPfRescale || (fresh && umax > -INFINITY);
    if (__any(move)) {  // wave-uniform
      const float shift = move ? umax : 0.f;
      const float alpha = move ? (fresh ? 0.f : __builtin_amdgcn_exp2f(-umax)) : 1.f;
      st.m[ct] = move ? m0 + umax : st.m[ct];
      st.l[ct] *= alpha;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) st.acc[ct][mt] *= alpha;
#pragma unroll
      for (int k = 0; k < 16; ++k) u[k] -= shift;
    }
    // p (fp32, into l) and p n_V 2^-gs: p rounded to fp16, times the fp16 norm pair
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = 8 * ks + 2 * j;
        const float p0 = __builtin_amdgcn_exp2f(u[k]), p1 = __builtin_amdgcn_exp2f(u[k + 1]);  // 0 if masked
        st.l[ct] += p0 + p1;
        v[j] = __builtin_bit_cast(uint32_t, h2{_Float16(p0), _Float16(p1)} * nv2[k >> 1]);
      }
      pb[ct][ks] = __builtin_bit_cast(h8, v);
    }
  }
}

// Entry of the 4-bit pair in byte J of x: the address 4 lane | byte << 8 | slot << 16
// formed by one byte permute of x and the table register (a fresh register per read,
// where entry_tf rewrites the shared one in place).
template <int J>
__device__ __forceinline__ uint32_t entry_perm(const TabTf<4>& tab, uint32_t x) {
  const uint32_t addr = __builtin_amdgcn_perm(x, tab.r[0], 0x03020000u | uint32_t(4 + J) << 8);
  return *reinterpret_cast<const uint32_t*>(tab.lds + addr);
}

// Values of the chunk: step k = 8ks + mt; pair q of K-step ks = tokens (8ks + 2q,
// 8ks + 2q + 1) of the V rows, merged by pf_merge_pairs.
template <int BWV, int NCT>
__device__ __forceinline__ void pf_values(const PfV<BWV>& V, TabTf<BWV>& cbv, const h8 (&pb)[NCT][2],
                                          PfState<NCT>& st) {
  constexpr int LA = kPfLookahead, VW = PfV<BWV>::VW;
  u32x4 e[LA + 1];
  auto look = [&](auto kc, u32x4& o) {
    constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t* w = V.w + VW * (8 * ks + 2 * q + (mt & 1));
      if constexpr (BWV == 4) o[q] = entry_perm<(mt >> 1)>(cbv, w[0]);
      else o[q] = pair_entry_tf(cbv, pair_offset<6, 6 * mt, 2>(w));
    }
  };
  static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 16>([&](auto kc) {
    constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7, j = k % (LA + 1);
    if constexpr (k + LA < 16) {
      look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
    const h8 av = __builtin_bit_cast(h8, e[j]);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
      st.acc[ct][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb[ct][ks], st.acc[ct][mt], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Writes the (acc, m, l) partial of each column (query row) of the block: lane (g, c)
// writes dims 32g .. 32g+31 of row 16 ct + c.
template <int NCT>
__device__ __forceinline__ void pf_write(const PrefillArgs& a, PfState<NCT>& st, int64_t row0, int lane) {
  const int g = lane >> 4, c = lane & 15;
  const float f = ldexpf(1.f, st.gs - 8);
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    float l = st.l[ct];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int64_t row = row0 + 16 * ct + c;
    float* dst = a.part_acc + row * 128 + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(dst + 8 * i) = make_float4(st.acc[ct][0][i] * f, st.acc[ct][1][i] * f,
                                                            st.acc[ct][2][i] * f, st.acc[ct][3][i] * f);
      *reinterpret_cast<float4*>(dst + 8 * i + 4) = make_float4(st.acc[ct][4][i] * f, st.acc[ct][5][i] * f,
                                                                st.acc[ct][6][i] * f, st.acc[ct][7][i] * f);
    }
    if (g == 0) *reinterpret_cast<float2*>(a.part_ml + 2 * row) = make_float2(st.m[ct], l);
  }
}

// pf_write for the shared-tile scan, whose value M-tile mt row c is dim 16 mt + c:
// lane (g, c) writes dims 16 mt + 4g .. +3 of row 16 ct + c.
template <int NCT>
__device__ __forceinline__ void pf_write_tiled(const PrefillArgs& a, PfState<NCT>& st, int64_t row0, int lane) {
  const int g = lane >> 4, c = lane & 15;
  const float f = ldexpf(1.f, st.gs - 8);
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    float l = st.l[ct];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int64_t row = row0 + 16 * ct + c;
    float* dst = a.part_acc + row * 128 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) *reinterpret_cast<f32x4*>(dst + 16 * mt) = st.acc[ct][mt] * f;
    if (g == 0) *reinterpret_cast<float2*>(a.part_ml + 2 * row) = make_float2(st.m[ct], l);
  }
}

// Logical index of work-group p of n when groups go to the 8 XCDs round robin: XCD x
// holds groups x, x+8, ...; they become a contiguous run of logical indices, so the
// waves of neighbouring items (the column blocks of one split) share an XCD's L2.
__device__ __forceinline__ int pf_xcd_major(int p, int n) {
  const int q = n >> 3, r = n & 7, x = p & 7, s = p >> 3;
  return x * q + min(x, r) + s;
}

template <int BWK, int BWV>
struct PfLds {
  static constexpr bool k4 = BWK == 4, v4 = BWV == 4;
  static constexpr int k_off = k4 && !v4 ? kTfTableBytes : 0;
  static constexpr int v_off = v4 ? kTfTableBytes : k4 ? 0 : tf_table_bytes<BWK>();
  static constexpr int pace = k_off + tf_table_bytes<BWK>() > v_off + tf_table_bytes<BWV>()
                                  ? k_off + tf_table_bytes<BWK>()
                                  : v_off + tf_table_bytes<BWV>();  // one word per wave (Pace)
  static constexpr int total = pace + 4 * 8;
  static_assert(total <= 160 * 1024, "LDS of a work-group exceeds 160 KB");
};

template <int BWK, int BWV, int NCT, int WPB>
__global__ __launch_bounds__(64 * WPB) void pf_scan_kernel(PrefillArgs a) {
  using Lay = PfLds<BWK, BWV>;
  // the two waves of a SIMD are paced (Pace) except at 6/6, the one width pair that
  // ran slower paced (config 3 at Q 16: 335-337 -> 338-349 us; config 2: 423-430 ->
  // 284-285 us, and 4/6 at config 5: 609 -> 602 us; unpaced, 6/4 spills)
  constexpr bool kPace = BWK == 4 || BWV == 4;
  __shared__ __align__(16) char lds[Lay::total];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  stage_table_tf<BWK, 64 * WPB>(a.cb_k, lds + Lay::k_off, tid);
  stage_table_tf<BWV, 64 * WPB>(a.cb_v, lds + Lay::v_off, tid);
  const Pace pace = make_pace<WPB>(reinterpret_cast<uint32_t*>(lds + Lay::pace), wig);
  __syncthreads();  // the only block-wide barrier: waves run independently from here
  const int64_t w = int64_t(pf_xcd_major(blockIdx.x, gridDim.x)) * WPB + wig;
  const int64_t items = int64_t(a.B) * a.Hkv * a.nsplit * a.ncb;
  if (w >= items) return;
  const int cb = int(w % a.ncb);
  int64_t u = w / a.ncb;
  const int s = int(u % a.nsplit);
  u /= a.nsplit;
  const int kvh = int(u % a.Hkv);
  const int b = int(u / a.Hkv);
  constexpr int NR = 16 * NCT;
  const int64_t row0 = w * NR;

  PfState<NCT> st;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) st.acc[ct][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m[ct] = -INFINITY;
    st.l[ct] = 0.f;
  }
  st.gs = 0;

  // visible tokens of the block: query qi sees keys j <= L - Q + qi
  const int L = const_view(a.seq_lens)[b];  // a scalar load (const_view)
  const int rows = a.n_rep * a.Q;
  const int r_first = cb * NR, r_last = min(r_first + NR, rows) - 1;
  int T = r_first < rows ? min(L, L - a.Q + r_last / a.n_rep + 1) : 0;
  T = max(T, 0);
  const int nch = (T + 63) >> 6;
  const int ch_lo = int(int64_t(nch) * s / a.nsplit), ch_hi = int(int64_t(nch) * (s + 1) / a.nsplit);
  if (ch_lo < ch_hi) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int r = r_first + 16 * ct + c;
      st.lim[ct] = r < rows ? L - a.Q + r / a.n_rep : INT32_MAX;  // padding rows: no mask (never written)
    }
    // every column of the block sees at least tokens <= lim_min
    const int lim_min = L - a.Q + r_first / a.n_rep;
    const int t_lo = 64 * ch_lo, t_hi = min(64 * ch_hi, T);
    const int col_hi = (t_hi - 1) >> a.log2S;
    const int32_t* trow = a.table + int64_t(b) * a.tsb;

    // B operands of the scores: column c of tile ct = row r_first + 16 ct + c, K-step
    // s = dims 32g + 8s + 0..7 of q' = q_rot 2^e, rounded to nearest (e per wave:
    // |q'| < 2^15)
    float qv[NCT][32];
    float amax = 0.f;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const float4* qp = reinterpret_cast<const float4*>(
          a.q_rot + ((int64_t(b) * a.Hkv + kvh) * a.nrp + r_first + 16 * ct + c) * 128 + 32 * g);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 x = qp[k];
        qv[ct][4 * k] = x.x;
        qv[ct][4 * k + 1] = x.y;
        qv[ct][4 * k + 2] = x.z;
        qv[ct][4 * k + 3] = x.w;
      }
#pragma unroll
      for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(qv[ct][k]));
    }
    int qe;
    frexpf(wave_max(amax), &qe);
    const int e = 15 - qe;
    const float sc = ldexpf(1.f, -(e + 8));
    h8 qb[NCT][4];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j) qb[ct][k][j] = _Float16(ldexpf(qv[ct][8 * k + j], e));

    TabTf<BWK> cbk = make_tab_tf<BWK>(lds, Lay::k_off, lane);
    TabTf<BWV> cbv = make_tab_tf<BWV>(lds, Lay::v_off, lane);
    // one buffer each for the K rows, the V rows and the norms: the next chunk's K rows
    // load once the scores have read this chunk's, its norms after the softmax, its V
    // rows after the values, each about two thirds of a chunk ahead of its use
    PfK<BWK> K;
    PfV<BWV> V;
    PfN N;
    {
      const PfTiles tl = pf_tiles(a, trow, t_lo, col_hi);
      pf_load_k<BWK>(a, tl, kvh, lane, K);
      pf_load_n(a, tl, kvh, lane, N);
      pf_load_v<BWV>(a, tl, kvh, lane, V);
    }
    const int n = ch_hi - ch_lo;
    for (int ch = 0; ch < n; ++ch) {
      const int c0 = t_lo + 64 * ch;
      const uint32_t left = uint32_t(n - ch);
      uint32_t partner_left = 0;
      if constexpr (kPace) {
        pace.publish(left);
        partner_left = pace.partner_left();
      }
      // the next chunk's tiles (the last chunk's again on the last step: its loads are
      // issued on every step, so each step's waits count the same loads)
      const PfTiles nx = pf_tiles(a, trow, min(c0 + 64, t_lo + 64 * (n - 1)), col_hi);
      const bool full = c0 + 63 <= lim_min && c0 + 64 <= t_hi;
      f32x4 d[NCT][4];
      pf_scores<BWK, NCT>(K, cbk, qb, d);
      pf_load_k<BWK>(a, nx, kvh, lane, K);
      h8 pb[NCT][2];
      pf_softmax<NCT>(d, N, sc, c0, t_hi, full, lane, st, pb);
      pf_load_n(a, nx, kvh, lane, N);
      pf_merge_pairs<BWV>(V, lane);
      pf_values<BWV, NCT>(V, cbv, pb, st);
      pf_load_v<BWV>(a, nx, kvh, lane, V);
      if constexpr (kPace) pace_step(left, partner_left);
    }
    if constexpr (kPace) pace.publish(0);
  }
  pf_write<NCT>(a, st, row0, lane);
}

// ---------------------------------------------------------------- shared-tile scan
//
// For query blocks of many rows per kv head (n_rep Q >= 8 blocks of 16 NCT rows) the
// eight waves of a work-group take eight neighbouring blocks of the same (sequence,
// kv head, split) and share the chunk's dequantization: all threads turn the chunk's
// packed K and V rows into fp16 tiles in LDS (each code looked up once per work-group
// instead of once per wave), one barrier per chunk, and each wave reads its MFMA A
// operands from the tiles with one 16-byte LDS read per step. Scores, softmax and
// values are those of the per-wave scan with one change of token order: row c of
// score tile t is token tile_row(t, c), so that the 8 k-slots of lane group g in value
// K-step ks (score tiles 2ks and 2ks + 1, registers 0..3) are the consecutive tokens
// 32ks + 8g .. +7, which one read of the transposed V tile returns.
//
//   K tile   [64 tokens][128 dims] fp16, rows of 272 bytes, the 16-byte column
//            quads of rows 16..31 and 48..63 swapped by XOR 4 (the 16 rows that 16
//            lanes read together fall in 16 different bank quads)
//   V tile   [128 dims][64 tokens] fp16 (transposed), rows of 144 bytes
//   norms    n_K, n_V of the 64 tokens, fp16
// Two sets (chunk n is read from set n & 1 while chunk n + 1 is written to the other);
// the codebooks sit beside them as plain pair tables of fp16 pairs (4-bit: 256
// entries, 6-bit: 4096).

constexpr int kKRow = 272;                       // bytes per K tile row (256 + 16)
constexpr int kVRow = 144;                       // bytes per V tile row (128 + 16)
constexpr int kKTile = 64 * kKRow;               // 17,408
constexpr int kVTile = 128 * kVRow;              // 18,432
constexpr int kTileSet = kKTile + kVTile + 256;  // + 64 K and 64 V norms

// Dequantization tables of the shared-tile scan: the 4-bit pair table replicated once
// per lane of a half-wave (entry i of copy r at word 32 i + r, 32 KB), so that a wave's
// reads fall in distinct banks but for lanes l and l + 32; the 6-bit pair table plain
// (4,096 entries, 16 KB).
template <int BW>
constexpr int plain_tf_bytes() { return BW == 4 ? 256 * 32 * 4 : 4 << (2 * BW); }

// Byte offset of 16-byte column quad q of K tile row r.
__device__ __forceinline__ uint32_t ktile_off(int r, int q) { return uint32_t(r * kKRow + ((q ^ ((r & 16) >> 2)) << 4)); }

// Token of row c of score tile t (see above).
__device__ __forceinline__ int tile_row(int t, int c) { return 32 * (t >> 1) + 8 * (c >> 2) + 4 * (t & 1) + (c & 3); }

// Stages a pair table of fp16 pairs: entry i = (H(2^8 c[i mod 2^BW]), H(2^8 c[i >> BW])).
template <int BW, int NTHR>
__device__ __forceinline__ void stage_plain_tf(const float* cb, char* dst, int tid) {
  uint32_t* t = reinterpret_cast<uint32_t*>(dst);
  if constexpr (BW == 4) {
    for_strided<256 * 32, NTHR>(tid, [&](int i) { t[i] = tf_word(cb[(i >> 5) & 15] * kCbScale, cb[i >> 9] * kCbScale); });
  } else {
    for_strided<(1 << (2 * BW)), NTHR>(
        tid, [&](int i) { t[i] = tf_word(cb[i & ((1 << BW) - 1)] * kCbScale, cb[i >> BW] * kCbScale); });
  }
}

// Entry idx; lane_off = 4 (lane % 32), the lane's copy of a replicated 4-bit table.
template <int BW>
__device__ __forceinline__ uint32_t plain_entry(const char* tab, uint32_t idx, uint32_t lane_off) {
  if constexpr (BW == 4) return *reinterpret_cast<const uint32_t*>(tab + ((idx << 7) | lane_off));
  else return *reinterpret_cast<const uint32_t*>(tab + (idx << 2));
}

// The raw bytes one thread dequantizes per chunk, loaded a chunk ahead.
// K items (token, 8-dim group dg), dg fastest: 1024 / (64 WPB) per thread.
// V items (token pair tp, 8-dim group dg), tp fastest: 512 / (64 WPB) per thread.
// Norms: threads 0..31 take K norms of tokens 2i, 2i+1; threads 32..63 the V norms.
template <int BWK, int BWV, int WPB>
struct PfRaw {
  static constexpr int NK = 1024 / (64 * WPB), NV = 512 / (64 * WPB);
  static constexpr int KW = BWK == 4 ? 1 : 2, VW = BWV == 4 ? 1 : 2;
  uint32_t k[NK][KW];
  uint32_t v[NV][2][VW];
  uint32_t n;
};

template <int BWK, int BWV, int WPB>
__device__ __forceinline__ void pf_raw_load(const PrefillArgs& a, const int32_t* trow, int kvh, int c0, int col_hi,
                                            int tid, PfRaw<BWK, BWV, WPB>& o) {
  using R = PfRaw<BWK, BWV, WPB>;
  const int smask = (1 << a.log2S) - 1;
  auto row_of = [&](const uint8_t* base, int64_t sp, int64_t sh, int nb, int tok) {
    const int t = c0 + tok;
    const uint32_t pid = uint32_t(trow[min(t >> a.log2S, col_hi)]);
    return base + uint64_t(pid) * uint64_t(sp) + uint64_t(kvh) * uint64_t(sh) + uint32_t(t & smask) * uint32_t(nb);
  };
#pragma unroll
  for (int j = 0; j < R::NK; ++j) {
    const int it = tid + 64 * WPB * j, tok = it >> 4, dg = it & 15;
    const uint8_t* p = row_of(a.k_pages, a.ksp, a.ksh, 16 * BWK, tok);
    if constexpr (BWK == 4) {
      o.k[j][0] = *reinterpret_cast<const uint32_t*>(p + 4 * dg);
    } else {
      uint2 x;
      __builtin_memcpy(&x, __builtin_assume_aligned(p + ((6 * dg) & ~3), 4), 8);
      o.k[j][0] = x.x;
      o.k[j][1] = x.y;
    }
  }
#pragma unroll
  for (int j = 0; j < R::NV; ++j) {
    const int it = tid + 64 * WPB * j, tp = it & 31, dg = it >> 5;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint8_t* p = row_of(a.v_pages, a.vsp, a.vsh, 16 * BWV, 2 * tp + h);
      if constexpr (BWV == 4) {
        o.v[j][h][0] = *reinterpret_cast<const uint32_t*>(p + 4 * dg);
      } else {
        uint2 x;
        __builtin_memcpy(&x, __builtin_assume_aligned(p + ((6 * dg) & ~3), 4), 8);
        o.v[j][h][0] = x.x;
        o.v[j][h][1] = x.y;
      }
    }
  }
  if (tid < 64) {
    const int tok = 2 * (tid & 31);
    const int t = c0 + tok;
    const uint32_t pid = uint32_t(trow[min(t >> a.log2S, col_hi)]);
    const uint16_t* nb = tid < 32 ? a.k_norms + uint64_t(pid) * uint64_t(a.knp) + uint64_t(kvh) * uint64_t(a.knh)
                                  : a.v_norms + uint64_t(pid) * uint64_t(a.vnp) + uint64_t(kvh) * uint64_t(a.vnh);
    o.n = *reinterpret_cast<const uint32_t*>(nb + (t & smask));
  }
}

// Dequantizes the raw bytes into tile set `set`.
template <int BWK, int BWV, int WPB>
__device__ __forceinline__ void pf_raw_store(const PfRaw<BWK, BWV, WPB>& r, const char* tabk, const char* tabv,
                                             char* set, int tid) {
  using R = PfRaw<BWK, BWV, WPB>;
  const uint32_t lo = uint32_t(tid & 31) << 2;
#pragma unroll
  for (int j = 0; j < R::NK; ++j) {
    const int it = tid + 64 * WPB * j, tok = it >> 4, dg = it & 15;
    u32x4 e;
    if constexpr (BWK == 4) {
      const uint32_t w = r.k[j][0];
#pragma unroll
      for (int p = 0; p < 4; ++p) e[p] = plain_entry<4>(tabk, (w >> (8 * p)) & 0xFFu, lo);
    } else {
      const uint32_t sh = 16u * uint32_t(dg & 1);
      const uint64_t x = (uint64_t(r.k[j][1]) << 32 | r.k[j][0]) >> sh;
#pragma unroll
      for (int p = 0; p < 4; ++p) e[p] = plain_entry<6>(tabk, uint32_t(x >> (12 * p)) & 0xFFFu, lo);
    }
    *reinterpret_cast<u32x4*>(set + ktile_off(tok, dg)) = e;
  }
  char* vt = set + kKTile;
#pragma unroll
  for (int j = 0; j < R::NV; ++j) {
    const int it = tid + 64 * WPB * j, tp = it & 31, dg = it >> 5;
    // pair index of dim 8dg + m: (code of token 2tp, code of token 2tp + 1)
    uint32_t idx[8];
    if constexpr (BWV == 4) {
      const uint32_t wa = r.v[j][0][0], wb = r.v[j][1][0];
      const uint32_t xe = bitsel(0x0F0F0F0Fu, wa, wb << 4), xo = bitsel(0x0F0F0F0Fu, wa >> 4, wb);
#pragma unroll
      for (int m = 0; m < 8; ++m) idx[m] = ((m & 1 ? xo : xe) >> (8 * (m >> 1))) & 0xFFu;
    } else {
      const uint32_t sh = 16u * uint32_t(dg & 1);
      const uint64_t xa = (uint64_t(r.v[j][0][1]) << 32 | r.v[j][0][0]) >> sh;
      const uint64_t xb = (uint64_t(r.v[j][1][1]) << 32 | r.v[j][1][0]) >> sh;
#pragma unroll
      for (int m = 0; m < 8; ++m) idx[m] = uint32_t((xa >> (6 * m)) & 63u) | uint32_t((xb >> (6 * m)) & 63u) << 6;
    }
#pragma unroll
    for (int m = 0; m < 8; ++m)
      *reinterpret_cast<uint32_t*>(vt + (8 * dg + m) * kVRow + 4 * tp) = plain_entry<BWV>(tabv, idx[m], lo);
  }
  if (tid < 64) *reinterpret_cast<uint32_t*>(set + kKTile + kVTile + 128 * (tid >> 5) + 4 * (tid & 31)) = r.n;
}

template <int BWK, int BWV, int WPB>
struct PfTileLds {
  static constexpr int tabk = 0, tabv = plain_tf_bytes<BWK>();
  static constexpr int sets = tabv + plain_tf_bytes<BWV>();
  static constexpr int total = sets + 2 * kTileSet;
  static_assert(sets % 16 == 0 && kTileSet % 16 == 0, "tile sets 16-byte aligned");
  static_assert(total <= 160 * 1024, "LDS of a work-group exceeds 160 KB");
};

template <int BWK, int BWV, int NCT, int WPB>
__global__ __launch_bounds__(64 * WPB) void pf_tile_kernel(PrefillArgs a) {
  using Lay = PfTileLds<BWK, BWV, WPB>;
  constexpr int NR = 16 * NCT, LA = kPfLookahead;
  __shared__ __align__(16) char lds[Lay::total];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  stage_plain_tf<BWK, 64 * WPB>(a.cb_k, lds + Lay::tabk, tid);
  stage_plain_tf<BWV, 64 * WPB>(a.cb_v, lds + Lay::tabv, tid);
  // work-group unit: (sequence, kv head, split, column group of WPB blocks)
  const int ncg = (a.ncb + WPB - 1) / WPB;
  const int64_t unit = pf_xcd_major(blockIdx.x, gridDim.x);
  const int cg = int(unit % ncg);
  int64_t u = unit / ncg;
  const int s = int(u % a.nsplit);
  u /= a.nsplit;
  const int kvh = int(u % a.Hkv);
  const int b = int(u / a.Hkv);
  const bool unit_live = b < a.B;  // grid rounding
  const int cb = cg * WPB + wig;
  const bool wave_live = unit_live && cb < a.ncb;

  PfState<NCT> st;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) st.acc[ct][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m[ct] = -INFINITY;
    st.l[ct] = 0.f;
  }
  st.gs = 0;
  const int L = unit_live ? const_view(a.seq_lens)[b] : 0;
  const int rows = a.n_rep * a.Q;
  // the group's chunks: those its last row sees (the other rows mask what they must not see)
  const int g_first = cg * WPB * NR, g_last = min(g_first + WPB * NR, rows) - 1;
  const int T = max(0, g_first < rows ? min(L, L - a.Q + g_last / a.n_rep + 1) : 0);
  const int nch = (T + 63) >> 6;
  const int ch_lo = int(int64_t(nch) * s / a.nsplit), ch_hi = int(int64_t(nch) * (s + 1) / a.nsplit);
  const int n = ch_hi - ch_lo;  // work-group uniform
  const int r_first = cb * NR;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int r = r_first + 16 * ct + c;
    st.lim[ct] = r < rows ? L - a.Q + r / a.n_rep : INT32_MAX;
  }
  const int lim_min = L - a.Q + min(r_first, rows - 1) / a.n_rep;

  // B operands of the scores (as in pf_scan_kernel); a wave past the last block keeps
  // zeros. The rows are read twice (the maximum, then the conversion) rather than held
  // as floats meanwhile.
  h8 qb[NCT][4];
  float sc = 1.f;
  {
    auto qrow = [&](int ct) {
      const int64_t row = (int64_t(b) * a.Hkv + kvh) * a.nrp + min(r_first + 16 * ct + c, a.nrp - 1);
      return reinterpret_cast<const float4*>(a.q_rot + row * 128 + 32 * g);
    };
    float amax = 0.f;
    if (wave_live) {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float4 x = qrow(ct)[k];
          amax = fmaxf(amax, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
        }
    }
    int qe;
    frexpf(wave_max(amax), &qe);
    const int e = 15 - qe;
    sc = ldexpf(1.f, -(e + 8));
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 x0 = wave_live ? qrow(ct)[2 * k] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 x1 = wave_live ? qrow(ct)[2 * k + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) qb[ct][k][j] = _Float16(ldexpf(v[j], e));
      }
  }

  if (n > 0) {
    const int t_lo = 64 * ch_lo, t_hi = min(64 * ch_hi, T);
    const int col_hi = (t_hi - 1) >> a.log2S;
    const int32_t* trow = a.table + int64_t(b) * a.tsb;
    const char* tabk = lds + Lay::tabk;
    const char* tabv = lds + Lay::tabv;
    PfRaw<BWK, BWV, WPB> raw;
    pf_raw_load<BWK, BWV, WPB>(a, trow, kvh, t_lo, col_hi, tid, raw);
    __syncthreads();  // the tables are staged
    pf_raw_store<BWK, BWV, WPB>(raw, tabk, tabv, lds + Lay::sets, tid);
    if (n > 1) pf_raw_load<BWK, BWV, WPB>(a, trow, kvh, t_lo + 64, col_hi, tid, raw);
    // this lane's score A rows (token tile_row(t, c)) and value A row (dim 16 mt + c)
    uint32_t krow[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) krow[t] = uint32_t(tile_row(t, c));
    for (int ch = 0; ch < n; ++ch) {
      __syncthreads();  // chunk ch is in set ch & 1; set (ch + 1) & 1 is free
      const char* cur = lds + Lay::sets + (ch & 1) * kTileSet;
      if (ch + 1 < n) {
        pf_raw_store<BWK, BWV, WPB>(raw, tabk, tabv, lds + Lay::sets + ((ch + 1) & 1) * kTileSet, tid);
        if (ch + 2 < n) pf_raw_load<BWK, BWV, WPB>(a, trow, kvh, t_lo + 64 * (ch + 2), col_hi, tid, raw);
      }
      if (!wave_live) continue;
      const int c0 = t_lo + 64 * ch;
      const bool full = c0 + 63 <= lim_min && c0 + 64 <= t_hi;
      // scores: step k = 4s + t, A = 8 dims 32g + 8s .. of token tile_row(t, c)
      f32x4 d[NCT][4];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int t = 0; t < 4; ++t) d[ct][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      {
        h8 e[LA + 1];
        auto look = [&](auto kc, h8& o) {
          constexpr int k = decltype(kc)::value, s4 = k >> 2, t = k & 3;
          o = *reinterpret_cast<const h8*>(cur + ktile_off(int(krow[t]), 4 * g + s4));
        };
        static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, 16>([&](auto kc) {
          constexpr int k = decltype(kc)::value, s4 = k >> 2, t = k & 3, j = k % (LA + 1);
          if constexpr (k + LA < 16) {
            look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
            __builtin_amdgcn_sched_barrier(0);
          }
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
            d[ct][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(e[j], qb[ct][s4], d[ct][t], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        });
      }
      // norms of this lane's score registers: tile t register i = token tile_row(t, 4g + i),
      // i.e. tokens 32ks + 8g + 4h + i for t = 2ks + h: two 16-byte reads per side
      PfN nrm;
      {
        const uint4* nk = reinterpret_cast<const uint4*>(cur + kKTile + kVTile);
        const uint4* nv = reinterpret_cast<const uint4*>(cur + kKTile + kVTile + 128);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint4 x = nk[4 * ks + g], y = nv[4 * ks + g];
          nrm.nk[4 * ks] = x.x;
          nrm.nk[4 * ks + 1] = x.y;
          nrm.nk[4 * ks + 2] = x.z;
          nrm.nk[4 * ks + 3] = x.w;
          nrm.nv[4 * ks] = y.x;
          nrm.nv[4 * ks + 1] = y.y;
          nrm.nv[4 * ks + 2] = y.z;
          nrm.nv[4 * ks + 3] = y.w;
        }
      }
      h8 pb[NCT][2];
      pf_softmax<NCT, true>(d, nrm, sc, c0, t_hi, full, lane, st, pb);
      // values: step k = 8ks + mt, A = tokens 32ks + 8g .. +7 of dim 16 mt + c
      {
        h8 e[LA + 1];
        auto look = [&](auto kc, h8& o) {
          constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7;
          o = *reinterpret_cast<const h8*>(cur + kKTile + (16 * mt + c) * kVRow + 16 * (4 * ks + g));
        };
        static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, 16>([&](auto kc) {
          constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7, j = k % (LA + 1);
          if constexpr (k + LA < 16) {
            look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
            __builtin_amdgcn_sched_barrier(0);
          }
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
            st.acc[ct][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(e[j], pb[ct][ks], st.acc[ct][mt], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        });
      }
    }
  }
  if (wave_live) pf_write_tiled<NCT>(a, st, ((((int64_t(b) * a.Hkv + kvh) * a.nsplit + s) * a.ncb + cb) * NR), lane);
}

// ---------------------------------------------------------------- rotate and merge
//
// Both are a kRotRows-row tile times a 128 x 128 rotation per work-group: the matrix
// M^T ([j][k], 132-float rows) and the rows ([r][k], 132-float rows) in LDS, thread t
// making rows RT (t >> 4) .. and columns (t & 15) + 16 jj, jj = 0..7, from 16-byte
// reads along k (the 16 lanes of a column group read 16 different M^T rows whose 4-bank
// spans do not overlap; lanes sharing rows read the same addresses).

constexpr int kRotStride = 132;  // floats per LDS row (16-byte aligned, bank-skewed)

struct PfRotArgs {
  const void* q;
  int64_t qsb, qsh, qsq;  // element strides of q (B, Hq, Q, D)
  const float* pi;
  float* q_rot;
  float scale;
  int Hkv, n_rep, Q, nrp, q_dtype;
};

// y[r][jj] = sum_k x[rb + r][k] mt[(t & 15) + 16 jj][k], rb = RT (t >> 4).
constexpr int RT = kRotRows / 16;  // rows per thread
__device__ __forceinline__ void rows_times_t(const float* x, const float* mt, int tid, float (&y)[RT][8]) {
  const int rb = RT * (tid >> 4), jc = tid & 15;
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) y[r][jj] = 0.f;
#pragma unroll 2
  for (int k = 0; k < 128; k += 4) {
    float4 xv[RT], mv[8];
#pragma unroll
    for (int r = 0; r < RT; ++r) xv[r] = *reinterpret_cast<const float4*>(x + (rb + r) * kRotStride + k);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) mv[jj] = *reinterpret_cast<const float4*>(mt + (jc + 16 * jj) * kRotStride + k);
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        y[r][jj] = fmaf(xv[r].x, mv[jj].x, y[r][jj]);
        y[r][jj] = fmaf(xv[r].y, mv[jj].y, y[r][jj]);
        y[r][jj] = fmaf(xv[r].z, mv[jj].z, y[r][jj]);
        y[r][jj] = fmaf(xv[r].w, mv[jj].w, y[r][jj]);
      }
  }
}

// q_rot rows (sequence blockIdx.z, kv head blockIdx.y, rows kRotRows blockIdx.x ..):
// scale * q Pi_K^T, zero for rows past n_rep Q. Pi_K is [j][k] already: its rows are
// staged as they are, with coalesced 16-byte loads.
__global__ __launch_bounds__(256) void pf_rotate_kernel(PfRotArgs a) {
  __shared__ __align__(16) float mt[128 * kRotStride];
  __shared__ __align__(16) float x[kRotRows * kRotStride];
  const int tid = threadIdx.x, kvh = blockIdx.y, b = blockIdx.z, r0 = blockIdx.x * kRotRows;
  for_strided<128 * 32, 256>(tid, [&](int i) {
    const int j = i >> 5, k4 = 4 * (i & 31);
    *reinterpret_cast<float4*>(mt + j * kRotStride + k4) = reinterpret_cast<const float4*>(a.pi)[i];
  });
  const int rows = a.n_rep * a.Q;
  for_strided<kRotRows * 128, 256>(tid, [&](int i) {
    const int rr = i >> 7, k = i & 127, r = r0 + rr;
    float v = 0.f;
    if (r < rows) {
      const int qi = r / a.n_rep, h = kvh * a.n_rep + r % a.n_rep;
      v = load_elem(a.q, b * a.qsb + h * a.qsh + qi * a.qsq + k, a.q_dtype);
    }
    x[rr * kRotStride + k] = v;
  });
  __syncthreads();
  float y[RT][8];
  rows_times_t(x, mt, tid, y);
  const int rb = RT * (tid >> 4), jc = tid & 15;
  float* out = a.q_rot + ((int64_t(b) * a.Hkv + kvh) * a.nrp + r0) * 128;
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) out[(rb + r) * 128 + jc + 16 * jj] = y[r][jj] * a.scale;
}

struct PfMergeArgs {
  const float* part_acc;
  const float* part_ml;
  const float* pi_v;
  void* out;  // (B, Hq, Q, D) contiguous
  int out_dtype, Hkv, n_rep, Q, nrp, ncb, nsplit, nr;  // nr: rows per column block
};

// y[r][j] = sum_k xt[k][rb + r] m[k][jb + j] for the kRotRows rows of a work-group:
// xt = the rows transposed ([k][r]), m = M as it is stored ([k][j]); thread t makes
// rows 4 (t / 32) .. +3 (RT2 of them) and columns 4 (t % 32) .. +3.
constexpr int RT2 = kRotRows / 8;
__device__ __forceinline__ void rows_times_n(const float* xt, const float* m, int tid, float (&y)[RT2][4]) {
  const int rb = RT2 * (tid >> 5), jb = 4 * (tid & 31);
#pragma unroll
  for (int r = 0; r < RT2; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) y[r][j] = 0.f;
#pragma unroll 4
  for (int k = 0; k < 128; ++k) {
    float xa[RT2];
#pragma unroll
    for (int r = 0; r < RT2; r += 4) {
      const float4 xv = *reinterpret_cast<const float4*>(xt + k * kRotRows + rb + r);
      xa[r] = xv.x;
      xa[r + 1] = xv.y;
      xa[r + 2] = xv.z;
      xa[r + 3] = xv.w;
    }
    const float4 mv = *reinterpret_cast<const float4*>(m + k * 128 + jb);
#pragma unroll
    for (int r = 0; r < RT2; ++r) {
      y[r][0] = fmaf(xa[r], mv.x, y[r][0]);
      y[r][1] = fmaf(xa[r], mv.y, y[r][1]);
      y[r][2] = fmaf(xa[r], mv.z, y[r][2]);
      y[r][3] = fmaf(xa[r], mv.w, y[r][3]);
    }
  }
}

// Rows (sequence blockIdx.z, kv head blockIdx.y, rows kRotRows blockIdx.x ..): the
// max-stable merge of each row's split partials (weights 2^(m_s - max m)), 1 / l,
// then Pi_V ([k][j], staged as stored) and the cast; rows that saw no key are 0
// (packed_attention.py:206). The splits' maxima are read in one pass and their
// weighted rows in a second, so neither pass chains a load behind another.
__global__ __launch_bounds__(256) void pf_merge_kernel(PfMergeArgs a) {
  __shared__ __align__(16) float pv[128 * 128];
  __shared__ __align__(16) float xt[128 * kRotRows];
  const int tid = threadIdx.x, kvh = blockIdx.y, b = blockIdx.z, r0 = blockIdx.x * kRotRows;
  for_strided<128 * 128 / 4, 256>(
      tid, [&](int i) { reinterpret_cast<float4*>(pv)[i] = reinterpret_cast<const float4*>(a.pi_v)[i]; });
  {
    // thread: row rr = tid / TPR, dims DPT (tid % TPR) .. (TPR threads per row)
    constexpr int TPR = 256 / kRotRows, DPT = 128 / TPR;
    const int rr = tid / TPR, d0 = DPT * (tid % TPR), r = r0 + rr;
    const int cb = r / a.nr, ri = r % a.nr;
    const int64_t row0 = (((int64_t(b) * a.Hkv + kvh) * a.nsplit) * a.ncb + cb) * a.nr + ri;
    const int64_t srow = int64_t(a.ncb) * a.nr;  // rows between a row's consecutive splits
    float M = -INFINITY;
#pragma unroll 8
    for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.part_ml[2 * (row0 + s * srow)]);
    float den = 0.f, num[DPT];
#pragma unroll
    for (int k = 0; k < DPT; ++k) num[k] = 0.f;
    if (M != -INFINITY) {
#pragma unroll 4
      for (int s = 0; s < a.nsplit; ++s) {
        const int64_t row = row0 + s * srow;
        const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + 2 * row);
        const float w = __builtin_amdgcn_exp2f(ml.x - M);  // 0 for a split without keys (m = -inf)
        den = fmaf(w, ml.y, den);
        const float4* src = reinterpret_cast<const float4*>(a.part_acc + row * 128 + d0);
#pragma unroll
        for (int k = 0; k < DPT / 4; ++k) {
          const float4 v = src[k];
          num[4 * k] = fmaf(w, v.x, num[4 * k]);
          num[4 * k + 1] = fmaf(w, v.y, num[4 * k + 1]);
          num[4 * k + 2] = fmaf(w, v.z, num[4 * k + 2]);
          num[4 * k + 3] = fmaf(w, v.w, num[4 * k + 3]);
        }
      }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
    for (int k = 0; k < DPT; ++k) xt[(d0 + k) * kRotRows + rr] = num[k] * inv;
  }
  __syncthreads();
  float y[RT2][4];
  rows_times_n(xt, pv, tid, y);
  const int rb = RT2 * (tid >> 5), jb = 4 * (tid & 31);
  const int rows = a.n_rep * a.Q, Hq = a.Hkv * a.n_rep;
#pragma unroll
  for (int r = 0; r < RT2; ++r) {
    const int rg = r0 + rb + r;
    if (rg >= rows) continue;
    const int qi = rg / a.n_rep, h = kvh * a.n_rep + rg % a.n_rep;
    const int64_t o = ((int64_t(b) * Hq + h) * a.Q + qi) * 128 + jb;
#pragma unroll
    for (int j = 0; j < 4; ++j) store_elem(a.out, o + j, a.out_dtype, y[r][j]);
  }
}

// ---------------------------------------------------------------- host side

using PfScanFn = void (*)(PrefillArgs);

struct PfKernel {
  PfScanFn fn = nullptr;   // per-wave scan (few query blocks per kv head)
  PfScanFn tile = nullptr;  // shared-tile scan (work-groups of tile_wpb blocks)
  int wpb = 0, nct = 0, tile_wpb = 0;
};

template <int BWK, int BWV>
PfKernel pf_kernel() {
  // four column tiles (64 query rows) per wave: one K or V lookup feeds four MFMAs;
  // the accumulators take 128 registers, so one wave per SIMD
  constexpr int NCT = 2, WPB = 8;
  return PfKernel{pf_scan_kernel<BWK, BWV, NCT, WPB>, pf_tile_kernel<BWK, BWV, NCT, 8>, WPB, NCT, 8};
}

PfKernel pick_prefill(int bw_k, int bw_v) {
  if (bw_k == 4 && bw_v == 4) return pf_kernel<4, 4>();
  if (bw_k == 6 && bw_v == 6) return pf_kernel<6, 6>();
  if (bw_k == 4 && bw_v == 6) return pf_kernel<4, 6>();
  if (bw_k == 6 && bw_v == 4) return pf_kernel<6, 4>();
  return PfKernel{};
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int pf_nrp(int n_rep, int Q) { return int((int64_t(n_rep) * Q + kRowPad - 1) / kRowPad * kRowPad); }

struct PfLayout {
  int64_t qrot, acc, ml, total;
};

PfLayout pf_layout(int B, int Hq, int Hkv, int Q, int num_splits) {
  PfLayout l;
  const int64_t rows = int64_t(B) * Hkv * pf_nrp(Hq / Hkv, Q);
  l.qrot = 0;
  l.acc = align256(rows * 128 * 4);
  l.ml = l.acc + align256(rows * num_splits * 128 * 4);
  l.total = l.ml + align256(rows * num_splits * 2 * 4);
  return l;
}

// Resident work-groups of `fn` (wpb waves each) on the current device.
int resident_groups_pf(PfScanFn fn, int wpb) {
  static std::mutex mu;
  static std::map<std::pair<int, PfScanFn>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({dev, fn});
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn), 64 * wpb, 0) !=
          hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int w = per_cu * cus;
  cache[{dev, fn}] = w;
  return w;
}

// The shared-tile scan serves shapes with at least tile_wpb query blocks per kv head.
bool use_tile(const PfKernel& k, int n_rep, int Q) { return pf_nrp(n_rep, Q) / (16 * k.nct) >= k.tile_wpb; }

}  // namespace
}  // namespace wn

extern "C" int wn_prefill_plan(int B, int Hq, int Hkv, int Q, int D, int S, int bw_k, int bw_v, int max_len,
                               int* num_splits) {
  using namespace wn;
  clear_error();
  WN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Q > 0 && max_len >= 0 && num_splits, WN_E_INVALID,
             "wn_prefill_plan: bad sizes B=%d Hq=%d Hkv=%d Q=%d max_len=%d", B, Hq, Hkv, Q, max_len);
  const PfKernel k = pick_prefill(bw_k, bw_v);
  WN_REQUIRE(D == 128 && S >= 16 && is_pow2(S) && k.fn, WN_E_UNSUPPORTED,
             "wn_prefill_plan: (D=%d, S=%d, bw_k=%d, bw_v=%d) not compiled", D, S, bw_k, bw_v);
  // about two work-groups per resident slot over the (sequence, kv head, column block
  // or group of blocks) units, each split keeping at least four chunks of the longest
  // history
  const bool tile = use_tile(k, Hq / Hkv, Q);
  const int wpb = tile ? k.tile_wpb : k.wpb;
  const int w = resident_groups_pf(tile ? k.tile : k.fn, wpb);
  WN_REQUIRE(w > 0, WN_E_LAUNCH, "wn_prefill_plan: cannot query the device occupancy");
  const int ncb = pf_nrp(Hq / Hkv, Q) / (16 * k.nct);
  const int64_t units = int64_t(B > 0 ? B : 1) * Hkv * (tile ? (ncb + wpb - 1) / wpb : ncb);
  int64_t ns = (2 * int64_t(tile ? w : w * wpb) + units - 1) / units;
  const int64_t chunks = (int64_t(max_len) + 63) / 64;
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, chunks / 4));
  *num_splits = int(std::max<int64_t>(1, std::min<int64_t>(ns, 256)));
  return WN_OK;
}

extern "C" int64_t wn_prefill_workspace_bytes(int B, int Hq, int Hkv, int Q, int D, int num_splits) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Q <= 0 || D != 128 || num_splits <= 0) return -1;
  return wn::pf_layout(B, Hq, Hkv, Q, num_splits).total;
}

extern "C" int wn_prefill_attention(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_q,
    const float* pi_k, const float* pi_v, const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b, const int32_t* seq_lens,
    void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int Q, int D, int S, int bw_k, int bw_v,
    float scale, int num_splits, void* stream, void* ev_begin, void* ev_end) {
  using namespace wn;
  clear_error();
  WN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Q > 0, WN_E_INVALID,
             "prefill: need B>=0, Q>0, Hq%%Hkv==0 (B=%d Hq=%d Hkv=%d Q=%d)", B, Hq, Hkv, Q);
  const PfKernel k = pick_prefill(bw_k, bw_v);
  WN_REQUIRE(D == 128 && k.fn, WN_E_UNSUPPORTED, "prefill: (D=%d, bw_k=%d, bw_v=%d) not compiled", D, bw_k, bw_v);
  WN_REQUIRE(is_pow2(S) && S >= 16, WN_E_INVALID, "prefill: page size %d is not a power of two >= 16", S);
  WN_REQUIRE(q_dtype >= WN_F32 && q_dtype <= WN_BF16 && out_dtype >= WN_F32 && out_dtype <= WN_BF16,
             WN_E_INVALID, "prefill: dtype codes %d/%d", q_dtype, out_dtype);
  WN_REQUIRE(num_splits > 0 && num_splits <= 4096, WN_E_INVALID, "prefill: num_splits %d", num_splits);
  const int n_rep = Hq / Hkv;
  WN_REQUIRE(int64_t(n_rep) * Q <= (int64_t(1) << 24), WN_E_INVALID, "prefill: n_rep * Q too large");
  if (B == 0) return WN_OK;
  WN_REQUIRE(q && pi_k && pi_v && codebook_k && codebook_v && k_pages && v_pages && k_norms && v_norms &&
                 page_table && seq_lens && out,
             WN_E_INVALID, "prefill: null operand");
  const int nbk = D * bw_k / 8, nbv = D * bw_v / 8;
  WN_REQUIRE(aligned(k_pages, 8) && k_stride_p % 8 == 0 && k_stride_h % 8 == 0 &&
                 (bw_k != 4 || (aligned(k_pages, 16) && k_stride_p % 16 == 0 && k_stride_h % 16 == 0)),
             WN_E_INVALID, "prefill: K pages need 16 (4-bit) or 8-byte aligned base and strides");
  WN_REQUIRE(aligned(v_pages, 4) && v_stride_p % 4 == 0 && v_stride_h % 4 == 0, WN_E_INVALID,
             "prefill: V pages need 4-byte aligned base and strides");
  WN_REQUIRE(k_stride_h >= int64_t(S) * nbk && v_stride_h >= int64_t(S) * nbv && k_stride_p >= 0 &&
                 v_stride_p >= 0,
             WN_E_INVALID, "prefill: head stride smaller than one (S, NB) page block");
  // the scan reads four norms of a token quad with one 8-byte load
  WN_REQUIRE(aligned(k_norms, 8) && aligned(v_norms, 8) && kn_stride_p % 4 == 0 && kn_stride_h % 4 == 0 &&
                 vn_stride_p % 4 == 0 && vn_stride_h % 4 == 0 && kn_stride_p >= 0 && kn_stride_h >= 0 &&
                 vn_stride_p >= 0 && vn_stride_h >= 0,
             WN_E_INVALID, "prefill: norm bases 8-byte aligned and strides multiples of 4 elements");
  WN_REQUIRE(aligned(pi_v, 16) && aligned(out, 4), WN_E_INVALID, "prefill: Pi_V 16-byte aligned");
  const PfLayout lay = pf_layout(B, Hq, Hkv, Q, num_splits);
  WN_REQUIRE(workspace && workspace_bytes >= lay.total && aligned(workspace, 256), WN_E_WORKSPACE,
             "prefill: workspace needs %lld bytes, 256-aligned (got %lld)", (long long)lay.total,
             (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nrp = pf_nrp(n_rep, Q);
  const int nr = 16 * k.nct, ncb = nrp / nr;

  PfRotArgs ra{q, q_stride_b, q_stride_h, q_stride_q, pi_k, reinterpret_cast<float*>(ws + lay.qrot),
               float(double(scale) * 1.4426950408889634), Hkv, n_rep, Q, nrp, q_dtype};
  hipLaunchKernelGGL(pf_rotate_kernel, dim3(nrp / kRotRows, Hkv, B), dim3(256), 0, st, ra);

  PrefillArgs pa;
  pa.q_rot = ra.q_rot;
  pa.k_pages = k_pages;
  pa.v_pages = v_pages;
  pa.k_norms = k_norms;
  pa.v_norms = v_norms;
  pa.cb_k = codebook_k;
  pa.cb_v = codebook_v;
  pa.table = page_table;
  pa.seq_lens = seq_lens;
  pa.part_acc = reinterpret_cast<float*>(ws + lay.acc);
  pa.part_ml = reinterpret_cast<float*>(ws + lay.ml);
  pa.ksp = k_stride_p;
  pa.ksh = k_stride_h;
  pa.vsp = v_stride_p;
  pa.vsh = v_stride_h;
  pa.knp = kn_stride_p;
  pa.knh = kn_stride_h;
  pa.vnp = vn_stride_p;
  pa.vnh = vn_stride_h;
  pa.tsb = table_stride_b;
  pa.B = B;
  pa.Hkv = Hkv;
  pa.n_rep = n_rep;
  pa.Q = Q;
  pa.nrp = nrp;
  pa.ncb = ncb;
  pa.nsplit = num_splits;
  pa.log2S = ilog2(S);
  const bool tile = use_tile(k, n_rep, Q);
  const int64_t groups = tile ? int64_t(B) * Hkv * num_splits * ((ncb + k.tile_wpb - 1) / k.tile_wpb)
                              : (int64_t(B) * Hkv * num_splits * ncb + k.wpb - 1) / k.wpb;
  WN_REQUIRE(groups < (int64_t(1) << 31), WN_E_INVALID, "prefill: grid too large");
  if (ev_begin) hipEventRecord(static_cast<hipEvent_t>(ev_begin), st);
  if (tile) hipLaunchKernelGGL(k.tile, dim3(unsigned(groups)), dim3(64 * k.tile_wpb), 0, st, pa);
  else hipLaunchKernelGGL(k.fn, dim3(unsigned(groups)), dim3(64 * k.wpb), 0, st, pa);
  if (ev_end) hipEventRecord(static_cast<hipEvent_t>(ev_end), st);

  PfMergeArgs ma{pa.part_acc, pa.part_ml, pi_v, out, out_dtype, Hkv, n_rep, Q, nrp, ncb, num_splits, nr};
  hipLaunchKernelGGL(pf_merge_kernel, dim3(nrp / kRotRows, Hkv, B), dim3(256), 0, st, ma);
  return check_launch("wn_prefill_attention");
}
