// Dense (unquantized) paged decode attention for gfx950: the matched baseline of the
// packed decode (dense_decode_attention, turboquant_kv/packed_attention_triton.py:190-201,
// the DENSE branch of its kernel :101-127). It runs on the packed decode's work plan:
// the same rotate-q launch (no rotation: q_rot = scale * log2(e) * q), the same
// balanced persistent waves over 64-token chunks, the same (acc, m, l) partials and
// the same merge (no output rotation). Only the page scan differs.
//
// Pages are (P, Hkv, S, D) bf16 or fp16 with D 64 or 128, each (page, kv head) block
// S contiguous rows of 2D bytes. A wave walks its tokens in 16-token tiles, one page slice each:
//
//   scores  lane l loads row l % 16 of the tile, bytes (D/2)G .. (D/2)(G+1) - 1
//           (G = l / 16), of K and of V: 16 rows x 2D bytes contiguous per tile.
//           s^T = K q^T runs on v_mfma_f32_16x16x32_{bf16,f16}: A = K with the
//           reduction order over the D dims permuted so that lane group G covers dims
//           (D/4)G .. (D/4)(G+1) - 1 (k-step s: (D/4)G + 8s .. +8, 16 bytes the lane
//           loaded), B = q^T with the same order, query heads padded to 16. q is a hi + lo pair in the page's
//           16-bit type (K is exact in it), so scores carry fp32 accuracy. Lane l ends
//           with the scores of head l % 16 for tokens 4G .. 4G+3.
//   softmax per head in log2 units with a lazy maximum (it moves, rescaling the
//           accumulators, only when a score exceeds it by more than kRescale).
//   values  those four probabilities are, as they stand, the A operand of
//           v_mfma_f32_16x16x16 (P: head x token); V goes through a per-wave LDS tile
//           so that lane l reads V[4G .. 4G+3][16T + l % 16] for output tile T. P is a
//           hi + lo pair as well; V is exact. acc[T] lane l = O[head 4G+j][dim 16T + l%16].
#include "wn_decode.h"

namespace wn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kDenseWpb = 4;           // independent waves per work-group
// Bytes per row of a wave's V tile: 2D + 8, so that rows 4 apart start 8 banks apart
// (the transposed reads are conflict free for D = 64 and 128), and of the tile.
template <int D>
constexpr int vrow() { return 2 * D + 8; }
template <int D>
constexpr int vtile() { return 16 * vrow<D>(); }
constexpr float kDenseRescale = 8.0f;  // log2 units

// Two values in the page's 16-bit type (round to nearest even), low half first.
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (F16) return uint32_t(f32_to_f16(a)) | (uint32_t(f32_to_f16(b)) << 16);
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <bool F16>
__device__ __forceinline__ float lo16(uint32_t w) {
  if constexpr (F16) return f16_to_f32(uint16_t(w & 0xffffu));
  else return __builtin_bit_cast(float, w << 16);
}
template <bool F16>
__device__ __forceinline__ float hi16(uint32_t w) {
  if constexpr (F16) return f16_to_f32(uint16_t(w >> 16));
  else return __builtin_bit_cast(float, w & 0xffff0000u);
}
// x = hi + lo: hi the rounded pair, lo the rounded remainders.
template <bool F16>
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack2<F16>(a, b);
  lo = pack2<F16>(a - lo16<F16>(hi), b - hi16<F16>(hi));
}

template <bool F16>
__device__ __forceinline__ f32x4 mma32(const uint4& a, const uint4& b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(s16x8, a), __builtin_bit_cast(s16x8, b), c, 0,
                                                    0, 0);
}
template <bool F16>
__device__ __forceinline__ f32x4 mma16(const uint2& a, const uint2& b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
}

template <int NT>
struct DenseState {
  f32x4 acc[NT];  // acc[T][j] = O[head 4G + j][dim 16T + l % 16]
  float m;       // running maximum of head l % 16 (equal in its four lanes), log2 units
  float l;       // this lane's share of head l % 16's sum
};

// Scans tokens [t_lo, t_hi) of (sequence b, kv head kvh), t_lo a multiple of 16, and
// writes one partial at row prow. Lane group g covers dims (D/4)g .. (D/4)g + D/4 - 1:
// NS = D/32 k-steps of 8 dims, NT = D/16 output tiles.
template <bool F16, int D>
__device__ __forceinline__ void dense_range(const DecodeArgs& a, int b, int kvh, int t_lo, int t_hi, int64_t prow,
                                            int lane, char* vt) {
  constexpr int NS = D / 32, NT = D / 16, LB = D / 2, VR = vrow<D>();
  const int h = lane & 15, g = lane >> 4;
  // B operand of the scores: q^T rows (D/4)g + 8s .. +8 of head h, hi and lo
  uint4 qh[NS], ql[NS];
  {
    const bool live = h < a.n_rep;
    const float* qp = a.q_rot + ((int64_t(b) * a.Hkv + kvh) * a.qrows + (live ? h : 0)) * D + (D / 4) * g;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = live ? qp[8 * s + 2 * e] : 0.f, x1 = live ? qp[8 * s + 2 * e + 1] : 0.f;
        split2<F16>(x0, x1, hw[e], lw[e]);
      }
      qh[s] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      ql[s] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
  }
  const int smask = (1 << a.log2S) - 1;
  const int32_t* trow = a.table + b * a.tsb;
  const uint8_t* kb = a.k_pages + (kvh / a.kvdiv) * a.ksh + LB * g;  // virtual kv head -> its kv head
  const uint8_t* vb = a.v_pages + (kvh / a.kvdiv) * a.vsh + LB * g;
  const int nsub = (t_hi - t_lo + 15) >> 4;
  // page of tile u (clamped to the last tile, which is then read again)
  auto pid_of = [&](int u) { return trow[(t_lo + 16 * min(u, nsub - 1)) >> a.log2S]; };
  // row h of tile u (tokens past t_hi are rows of the same page, masked later)
  auto load = [&](int u, int pid, uint4 (&k)[NS], uint4 (&v)[NS]) {
    const int64_t slot = (t_lo + 16 * min(u, nsub - 1) + h) & smask;
    const uint4* kp = reinterpret_cast<const uint4*>(kb + pid * a.ksp + slot * (2 * D));
    const uint4* vp = reinterpret_cast<const uint4*>(vb + pid * a.vsp + slot * (2 * D));
#pragma unroll
    for (int i = 0; i < NS; ++i) k[i] = kp[i];
#pragma unroll
    for (int i = 0; i < NS; ++i) v[i] = vp[i];
  };

  DenseState<NT> st;
#pragma unroll
  for (int t = 0; t < NT; ++t) st.acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;

  auto compute = [&](int u, const uint4 (&k)[NS], const uint4 (&v)[NS]) {
    const int c0 = t_lo + 16 * u;
    // V rows into the tile (the previous tile's reads are done first)
    wave_lds_sync();
    {
      char* row = vt + h * VR + LB * g;
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        *reinterpret_cast<uint2*>(row + 16 * i) = make_uint2(v[i].x, v[i].y);
        *reinterpret_cast<uint2*>(row + 16 * i + 8) = make_uint2(v[i].z, v[i].w);
      }
    }
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      sc = mma32<F16>(k[s], qh[s], sc);
      sc = mma32<F16>(k[s], ql[s], sc);
    }
    float sv[4];
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sv[j] = c0 + 4 * g + j < t_hi ? sc[j] : -INFINITY;
      mloc = fmaxf(mloc, sv[j]);
    }
    if (__any(st.m == -INFINITY || mloc > st.m + kDenseRescale)) {  // wave-uniform
      float mh = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
      mh = fmaxf(mh, __shfl_xor(mh, 32, 64));
      const float m_new = fmaxf(st.m, mh);
      // 0 on the first tile (m = -inf); m_new is finite: the tile's first token is valid
      const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
      st.m = m_new;
      st.l *= alpha;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float aj = __shfl(alpha, 4 * g + j, 64);  // lane 4g + j holds head 4g + j
#pragma unroll
        for (int t = 0; t < NT; ++t) st.acc[t][j] *= aj;
      }
    }
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[j] = __builtin_amdgcn_exp2f(sv[j] - st.m);  // 0 for masked tokens
      st.l += p[j];
    }
    uint32_t ph0, pl0, ph1, pl1;
    split2<F16>(p[0], p[1], ph0, pl0);
    split2<F16>(p[2], p[3], ph1, pl1);
    const uint2 ph = make_uint2(ph0, ph1), pl = make_uint2(pl0, pl1);
    wave_lds_sync();  // the tile is written
    const uint16_t* col = reinterpret_cast<const uint16_t*>(vt + 4 * g * VR) + h;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint16_t* c = col + 16 * t;
      const uint2 vbk = make_uint2(uint32_t(c[0]) | (uint32_t(c[VR / 2]) << 16),
                                   uint32_t(c[VR]) | (uint32_t(c[3 * VR / 2]) << 16));
      st.acc[t] = mma16<F16>(ph, vbk, st.acc[t]);
      st.acc[t] = mma16<F16>(pl, vbk, st.acc[t]);
    }
  };

  // Two tile buffers alternate; the next tile loads while this one computes, page
  // ids one tile further ahead.
  uint4 ka[NS], va[NS], kn[NS], vn[NS];
  load(0, pid_of(0), ka, va);
  int pid1 = pid_of(1);
  for (int u = 0; u < nsub; u += 2) {
    const int pid2 = pid_of(u + 2);
    load(u + 1, pid1, kn, vn);
    compute(u, ka, va);
    if (u + 1 >= nsub) break;
    const int pid3 = pid_of(u + 3);
    load(u + 2, pid2, ka, va);
    compute(u + 1, kn, vn);
    pid1 = pid3;
  }

  // partial: head h's sum over its four lanes; acc rows heads 4g + j
  float lsum = st.l + __shfl_xor(st.l, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  const int64_t row0 = prow * a.n_rep;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int head = 4 * g + j;
    if (head < a.n_rep) {
      float* dst = a.part_acc + (row0 + head) * D + h;
#pragma unroll
      for (int t = 0; t < NT; ++t) dst[16 * t] = st.acc[t][j];
    }
  }
  if (g == 0 && h < a.n_rep) {
    a.part_ml[2 * (row0 + h)] = st.m;
    a.part_ml[2 * (row0 + h) + 1] = lsum;
  }
}

// Logical index of work-group p of n when groups go to the 8 XCDs round robin.
__device__ __forceinline__ int dense_xcd_major(int p, int n) {
  const int q = n >> 3, r = n & 7, x = p & 7, s = p >> 3;
  return x * q + min(x, r) + s;
}

// The packed row scan's work list (decode_rows.hip): fixed splits, one (split, kv
// head, sequence) per wave; or balanced, the waves sharing the flattened
// (sequence, kv head, 64-token chunk) space equally, one partial per (sequence, kv
// head) a wave touches, at row w + b*Hkv + kvh, and unit_meta for the merge.
template <bool F16, int D>
__global__ __launch_bounds__(64 * kDenseWpb) void dense_scan_kernel(DecodeArgs a) {
  __shared__ __align__(16) char lds[kDenseWpb * vtile<D>()];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t w = int64_t(dense_xcd_major(blockIdx.x, gridDim.x)) * kDenseWpb + wig;
  char* vt = lds + wig * vtile<D>();

  int b, kvh, t_lo, t_hi;
  int64_t prow;
  int64_t s = 0, e = 0;
  const int32_t* pre = a.chunk_prefix;
  if (!a.balanced) {
    if (w >= int64_t(a.num_splits) * a.Hkv * a.B) return;
    const int split = int(w % a.num_splits);
    kvh = int((w / a.num_splits) % a.Hkv);
    b = int(w / (int64_t(a.num_splits) * a.Hkv));
    const int L = a.seq_lens[b];
    const int S = 1 << a.log2S;
    const int n_pages = (L + S - 1) >> a.log2S;
    const int page_lo = split * a.pages_per_split;
    if (page_lo >= n_pages) return;
    const int page_hi = min(page_lo + a.pages_per_split, n_pages);
    t_lo = page_lo << a.log2S;
    t_hi = min(page_hi << a.log2S, L);
    prow = (int64_t(b) * a.Hkv + kvh) * a.num_splits + split;
    if (split == 0 && lane == 0)
      a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), (n_pages + a.pages_per_split - 1) / a.pages_per_split);
  } else {
    const int64_t C = int64_t(a.Hkv) * pre[a.B];
    const int64_t Wp = min(int64_t(a.num_splits), C);
    if (w >= Wp) return;
    s = C * w / Wp;
    e = C * (w + 1) / Wp;
    int lo = 0, hi = a.B;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (int64_t(a.Hkv) * pre[mid] <= s) lo = mid;
      else hi = mid;
    }
    b = lo;
    kvh = t_lo = t_hi = 0;
    prow = 0;
  }
  while (true) {
    int nb = 0, c_hi = 0;
    if (a.balanced) {
      nb = pre[b + 1] - pre[b];
      while (nb == 0) {
        ++b;
        nb = pre[b + 1] - pre[b];
      }
      const int64_t base = int64_t(a.Hkv) * pre[b];
      kvh = int((s - base) / nb);
      const int c_lo = int((s - base) % nb);
      c_hi = int(min(int64_t(nb), c_lo + (e - s)));
      t_lo = 64 * c_lo;
      t_hi = min(64 * c_hi, a.seq_lens[b]);
      prow = w + int64_t(b) * a.Hkv + kvh;
      if (c_lo == 0 && lane == 0) {
        const int64_t C = int64_t(a.Hkv) * pre[a.B];
        const int64_t Wp = min(int64_t(a.num_splits), C);
        const int64_t U1 = base + int64_t(kvh + 1) * nb;
        const int64_t wl = (U1 * Wp + C - 1) / C - 1;
        a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), int(wl - w + 1));
      }
      s += c_hi - c_lo;
    }
    dense_range<F16, D>(a, b, kvh, t_lo, t_hi, prow, lane, vt);
    if (!a.balanced || s >= e) break;
    if (kvh + 1 == a.Hkv && c_hi == nb) ++b;
  }
}

// The vector-ALU dense scan: fp32 pages (K and V are not exact in a 16-bit MFMA
// type) at every head_dim, and bf16/fp16 pages at the head dims the MFMA scan does
// not take (16, 32, 256). One work-group of four waves per (split, kv head,
// sequence) on fixed splits, as the packed pages' vector-ALU scan: score phase lane =
// token (its K row read 4 elements at a time, NREP heads), online softmax per head in
// log2 units, value phase D/8 lanes per token row (8 dims each), then the max-stable
// merge of the four waves into one (acc, m, l) partial. Virtual kv head h reads the
// pages of kv head h / kvdiv.
constexpr int kF32Block = 256;

// Elements 4 i .. 4 i + 3 of a page row of dtype DT (WN_F32, WN_F16, WN_BF16).
template <int DT>
__device__ __forceinline__ float4 row4(const uint8_t* row, int i) {
  if constexpr (DT == WN_F32) {
    return reinterpret_cast<const float4*>(row)[i];
  } else {
    const uint2 x = reinterpret_cast<const uint2*>(row)[i];
    auto cv = [](uint32_t h) { return DT == WN_BF16 ? bf16_to_f32(uint16_t(h)) : f16_to_f32(uint16_t(h)); };
    return make_float4(cv(x.x & 0xffffu), cv(x.x >> 16), cv(x.y & 0xffffu), cv(x.y >> 16));
  }
}

template <int D, int NREP, int DT>
__global__ __launch_bounds__(kF32Block) void dense_valu_kernel(DecodeArgs a) {
  constexpr int ESZ = DT == WN_F32 ? 4 : 2;  // bytes per element
  constexpr int G = D / 8;     // lanes per token row in the value phase
  constexpr int TPS = 64 / G;  // token rows per value step
  __shared__ float pw[4][64][NREP];
  __shared__ int pidl[4][64];
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
  const int kvp = kvh / a.kvdiv;
  const float* __restrict__ qp = a.q_rot + (int64_t(b) * a.Hkv + kvh) * a.qrows * D;
  const int32_t* __restrict__ trow = a.table + b * a.tsb;
  const uint8_t* kbase = a.k_pages + kvp * a.ksh;
  const uint8_t* vbase = a.v_pages + kvp * a.vsh;

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
    const int t = c0 + lane;
    const bool valid = t < t_hi;
    int pid = 0;
    float s[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) s[h] = 0.f;
    if (valid) {
      pid = trow[t >> a.log2S];
      const uint8_t* kr = kbase + pid * a.ksp + int64_t(t & (S - 1)) * D * ESZ;
#pragma unroll 4
      for (int d4 = 0; d4 < D / 4; ++d4) {
        const float4 k = row4<DT>(kr, d4);
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
          const float4 qv = reinterpret_cast<const float4*>(qp + h * D)[d4];
          s[h] = fmaf(qv.x, k.x, fmaf(qv.y, k.y, fmaf(qv.z, k.z, fmaf(qv.w, k.w, s[h]))));
        }
      }
    } else {
#pragma unroll
      for (int h = 0; h < NREP; ++h) s[h] = -INFINITY;
    }
    wave_lds_sync();  // the previous chunk's value phase has read pw / pidl
    float alpha[NREP];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      const float mn = fmaxf(m[h], wave_max(s[h]));  // finite: lane 0 of a chunk is valid
      alpha[h] = __builtin_amdgcn_exp2f(m[h] - mn);   // 0 on the first chunk (m = -inf)
      const float pr = valid ? __builtin_amdgcn_exp2f(s[h] - mn) : 0.f;
      l[h] = l[h] * alpha[h] + wave_sum(pr);
      m[h] = mn;
      pw[w][lane][h] = pr;
    }
    pidl[w][lane] = pid;
    wave_lds_sync();
#pragma unroll
    for (int h = 0; h < NREP; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= alpha[h];
#pragma unroll 2
    for (int j = 0; j < 64 / TPS; ++j) {
      const int tl = j * TPS + tsub;
      const int tt = c0 + tl;
      if (tt < t_hi) {
        const uint8_t* vr = vbase + pidl[w][tl] * a.vsp + int64_t(tt & (S - 1)) * D * ESZ + dg * 8 * ESZ;
        const float4 v0 = row4<DT>(vr, 0), v1 = row4<DT>(vr, 1);
        const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
          const float wv = pw[w][tl][h];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(wv, vv[i], acc[h][i]);
        }
      }
    }
  }
  // token subgroups of a wave share m: plain sums
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
  // max-stable merge of the four waves; a wave that saw no chunk has m = -inf
  const int64_t row0 = ((int64_t(b) * a.Hkv + kvh) * a.num_splits + split) * a.n_rep;
  for (int e = tid; e < a.n_rep * D; e += kF32Block) {
    const int h = e / D, d = e % D;
    float M = red_m[0][h];
#pragma unroll
    for (int ww = 1; ww < 4; ++ww) M = fmaxf(M, red_m[ww][h]);
    float af = 0.f, lf = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float mw = red_m[ww][h];
      if (mw != -INFINITY) {
        const float sc = __builtin_amdgcn_exp2f(mw - M);
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

template <int D, int DT>
SplitFn pick_valu_nrep(int nrep) {
  switch (nrep) {
    case 1: return dense_valu_kernel<D, 1, DT>;
    case 2: return dense_valu_kernel<D, 2, DT>;
    case 4: return dense_valu_kernel<D, 4, DT>;
    case 8: return dense_valu_kernel<D, 8, DT>;
    case 16: return dense_valu_kernel<D, 16, DT>;
  }
  return nullptr;
}

// fp32 pages at every head_dim; bf16/fp16 only where the MFMA scan does not run
template <int D>
SplitFn pick_valu_dtype(int page_dtype, int nrep) {
  if (page_dtype == WN_F32) return pick_valu_nrep<D, WN_F32>(nrep);
  if constexpr (D != 64 && D != 128) {
    if (page_dtype == WN_BF16) return pick_valu_nrep<D, WN_BF16>(nrep);
    if (page_dtype == WN_F16) return pick_valu_nrep<D, WN_F16>(nrep);
  }
  return nullptr;
}

}  // namespace

SplitKernel pick_dense_valu_scan(int page_dtype, int D, int nrep) {
  SplitKernel k;
  switch (D) {
    case 16: k.fn = pick_valu_dtype<16>(page_dtype, nrep); break;
    case 32: k.fn = pick_valu_dtype<32>(page_dtype, nrep); break;
    case 64: k.fn = pick_valu_dtype<64>(page_dtype, nrep); break;
    case 128: k.fn = pick_valu_dtype<128>(page_dtype, nrep); break;
    case 256: k.fn = pick_valu_dtype<256>(page_dtype, nrep); break;
  }
  if (!k.fn) return SplitKernel{};
  k.block = kF32Block;
  k.nrep = nrep;
  k.log2_units = true;
  return k;
}

SplitKernel pick_dense_scan(int page_dtype, int D) {
  SplitKernel k;
  if (D == 128 && page_dtype == WN_BF16) k.fn = dense_scan_kernel<false, 128>;
  else if (D == 128 && page_dtype == WN_F16) k.fn = dense_scan_kernel<true, 128>;
  else if (D == 64 && page_dtype == WN_BF16) k.fn = dense_scan_kernel<false, 64>;
  else if (D == 64 && page_dtype == WN_F16) k.fn = dense_scan_kernel<true, 64>;
  else return SplitKernel{};
  k.block = 64 * kDenseWpb;
  k.wpb = kDenseWpb;
  k.nrep = 16;
  k.log2_units = true;
  k.rows = true;
  return k;
}

}  // namespace wn
