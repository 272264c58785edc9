// Fused TurboQuant dequantization for gfx950: unpack, codebook gather, the 128x128
// inverse rotation and the norm rescale, written once in the output type
// (turboquant_kv/kernel.py:33-75, csrc/tq_dequant.cu:125-173, and the paged history
// gather of packed_backend.py:192-208).
//
//   out[r, j] = (sum_d c[code(r, d)] Pi[d, j]) * n[r]
//
// The rotation is a (rows x 128) x (128 x 128) product on the matrix cores. fp32
// MFMA would make it compute-bound (2 * 128 FLOP per output byte pair), so every
// operand x is carried as a bf16 pair hi + lo (hi = x rounded, lo = x - hi rounded)
// and the product as hi*hi + hi*lo + lo*hi with v_mfma_f32_16x16x32_bf16 (lo*lo is
// below 2^-16 of the product; the output is rounded to bf16 anyway). The fast mode
// (the reference's allow_tf32) uses one fp16 product instead: 2^-11 per term, the
// class of tf32's 10-bit mantissa.
//
// A persistent work-group of four waves stages Pi^T as bf16 hi and lo planes in LDS
// once; each wave then takes passes of 64 rows (four 16-row tiles; the fast mode 32,
// two tiles) and computes the
// transposed product out^T = Pi^T y^T, so that a lane ends with four consecutive
// output dims of one row:
// The reduction order over the 128 input dims is permuted so that lane group
// G = l/16 covers dims 32G .. 32G+31 over the four k-steps (k-step s: dims
// 32G + 8s .. +8): a lane's codes are then one contiguous 4*bw-byte load per row.
//   A  (output-dim tile t, k-step s): lane l holds Pi[32G + 8s .. +8][n] for the dim n
//      of Pi^T row 16t + l % 16,
//      one 16-byte LDS read from the transposed plane (padded rows, conflict free);
//   B  (row tile, k-step s): lane l holds the codebook values of row l % 16 at dims
//      32G + 8s .. +8, looked up from a byte-indexed pair table for 4-bit codes
//      (one entry = hi or lo of the two codes of a byte) or per code;
//   D  lane l holds four output dims of row l % 16 per tile; the Pi^T rows are
//      ordered so that tiles 2a and 2a+1 give it dims 32a + 8(l/16) .. +7, and the
//      norm rescale and the cast happen on the way out, eight values per 16-byte store.
#include "wn_common.h"

namespace wn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kDqD = 128;
// Waves per work-group: the accurate mode runs one work-group of eight per CU (two
// waves per SIMD, paced: Pace); the fast mode, at four waves per SIMD, four.
template <bool FAST>
constexpr int dq_waves() { return FAST ? 4 : 8; }
constexpr int kDqTU = 2;  // output tiles per MFMA group
constexpr int kPiRow = 136;  // bf16 per row of a Pi^T plane: 128 + 8 pad (272 B rows)

struct DqArgs {
  const uint8_t* packed;
  const uint16_t* norms;  // fp16
  const float* pi;        // (D, D) fp32
  const float* cb;        // 2^bw fp32 centroids
  void* out;              // (N, D), row r at r * D
  int64_t N;              // rows (< 2^31, checked on the host)
  int64_t L;              // rows per plane (plane = r / L, position t = r % L)
  uint32_t lm;            // r / L = (h + ((r - h) >> ls1)) >> ls2, h = umulhi(r, lm)
  int ls1, ls2;
  int64_t plane_rows;     // strided mode: rows between consecutive planes in `packed`/`norms`
  const int32_t* table;   // paged mode (not null): page of position t is table[t >> log2S]
  int log2S;
  int64_t psp, psh;       // paged: packed page / plane strides, bytes
  int64_t nsp, nsh;       // paged: norm page / plane strides, elements
};

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return uint32_t(f32_to_f16(a)) | (uint32_t(f32_to_f16(b)) << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Plane and position of row r, clamped to a valid row (the caller masks the stores).
// The plane index is a multiply-high by the host's magic number for L (exact for every
// 32-bit r; Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, Figure 4.1).
__device__ __forceinline__ void row_pos(const DqArgs& a, int64_t r, uint32_t& plane, uint32_t& t) {
  const uint32_t r32 = uint32_t(r < a.N ? r : a.N - 1);
  const uint32_t h = __umulhi(r32, a.lm);
  plane = (h + ((r32 - h) >> a.ls1)) >> a.ls2;
  t = r32 - plane * uint32_t(a.L);
}

// Paged mode: the page holding row r.
__device__ __forceinline__ int32_t row_page(const DqArgs& a, int64_t r) {
  uint32_t plane, t;
  row_pos(a, r, plane, t);
  return a.table[t >> a.log2S];
}

// Codes and norm of row r; in paged mode `page` is row_page(a, r).
template <int NB, bool PAGED>
__device__ __forceinline__ void row_src(const DqArgs& a, int64_t r, int32_t page, const uint8_t*& p,
                                        const uint16_t*& n) {
  uint32_t plane, t;
  row_pos(a, r, plane, t);
  if constexpr (PAGED) {
    const int64_t slot = t & ((1u << a.log2S) - 1u);
    p = a.packed + page * a.psp + plane * a.psh + slot * NB;
    n = a.norms + page * a.nsp + plane * a.nsh + slot;
  } else {
    const int64_t src = int64_t(plane) * a.plane_rows + t;
    p = a.packed + src * NB;
    n = a.norms + src;
  }
}

// The 4*BW bytes (BW words) holding codes 32g..32g+31 of a row, LSB-first. Rows are
// 16*BW bytes and 16-byte aligned (checked on the host), so the words are aligned.
template <int BW>
__device__ __forceinline__ void load_codes32(const uint8_t* row, int g, uint32_t (&w)[BW]) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(row + 4 * BW * g);
  if constexpr (BW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < BW / 4; ++i) {
      const uint4 x = reinterpret_cast<const uint4*>(p)[i];
      w[4 * i] = x.x;
      w[4 * i + 1] = x.y;
      w[4 * i + 2] = x.z;
      w[4 * i + 3] = x.w;
    }
  } else if constexpr (BW % 2 == 0) {
#pragma unroll
    for (int i = 0; i < BW / 2; ++i) {
      const uint2 x = reinterpret_cast<const uint2*>(p)[i];
      w[2 * i] = x.x;
      w[2 * i + 1] = x.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < BW; ++i) w[i] = p[i];
  }
}

// Codes 8s..8s+7 of the 32 in w (k-step s) as two little-endian words: their
// 8*BW bits starting at bit 8*BW*s.
template <int BW>
__device__ __forceinline__ void step_codes(const uint32_t (&w)[BW], int s, uint32_t (&c)[2]) {
  const int bit = 8 * BW * s, wi = bit >> 5, sh = bit & 31;
  uint32_t lo = w[wi] >> sh;
  if (sh && wi + 1 < BW) lo |= w[wi + 1] << (32 - sh);
  uint32_t hi = 0;
  if (BW > 4) {
    const int b2 = bit + 32, w2 = b2 >> 5, s2 = b2 & 31;
    if (w2 < BW) {
      hi = w[w2] >> s2;
      if (s2 && w2 + 1 < BW) hi |= w[w2 + 1] << (32 - s2);
    }
  }
  c[0] = lo;
  c[1] = hi;
}

// Codebook of BW-bit codes in LDS as bf16 hi / lo: for 4-bit a pair table (entry b
// = the two codes of byte b, low nibble in the low half), else one 16-bit entry per
// code.
template <int BW>
struct DqTab {
  static constexpr int kEntries = BW == 4 ? 256 : (1 << BW);
  uint32_t hi[BW == 4 ? 256 : (1 << BW) / 2 + 1];
  uint32_t lo[BW == 4 ? 256 : (1 << BW) / 2 + 1];
};

// Fast mode: hi holds fp16 values and lo is unused.
template <int BW, bool FAST>
__device__ __forceinline__ void stage_dq_tab(const float* cb, DqTab<BW>& t, int tid) {
  auto put = [&](int i, float x0, float x1) {
    if constexpr (FAST) {
      t.hi[i] = pack_f16(x0, x1);
    } else {
      const uint32_t h = pack_bf16(x0, x1);
      t.hi[i] = h;
      t.lo[i] = pack_bf16(x0 - bf16_lo(h), x1 - bf16_hi(h));
    }
  };
  if constexpr (BW == 4) {
    for (int b = tid; b < 256; b += dq_waves<FAST>() * 64) put(b, cb[b & 15], cb[b >> 4]);
  } else {
    constexpr int L = 1 << BW;
    for (int i = tid; i < (L + 1) / 2; i += dq_waves<FAST>() * 64) put(i, cb[2 * i], 2 * i + 1 < L ? cb[2 * i + 1] : 0.f);
  }
}

// 16-bit entry of code c in a per-code table.
__device__ __forceinline__ uint32_t half_of(const uint32_t* t, uint32_t c) {
  const uint32_t w = t[c >> 1];
  return (c & 1u) ? (w >> 16) : (w & 0xffffu);
}

// MFMA operands of 8 codes (little-endian words w): hi and lo of their values.
template <int BW, bool FAST>
__device__ __forceinline__ void codes_to_a(const uint32_t (&w)[2], const DqTab<BW>& t, s16x8& ah, s16x8& al) {
  uint32_t h[4], l[4];
  if constexpr (BW == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t b = (w[0] >> (8 * j)) & 0xffu;
      h[j] = t.hi[b];
      l[j] = FAST ? 0u : t.lo[b];
    }
  } else {
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int bit = j * BW, wi = bit >> 5, sh = bit & 31;
      uint32_t x = w[wi] >> sh;
      if (sh + BW > 32) x |= w[wi + 1] << (32 - sh);
      c[j] = x & ((1u << BW) - 1u);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[j] = half_of(t.hi, c[2 * j]) | (half_of(t.hi, c[2 * j + 1]) << 16);
      l[j] = FAST ? 0u : half_of(t.lo, c[2 * j]) | (half_of(t.lo, c[2 * j + 1]) << 16);
    }
  }
  ah = __builtin_bit_cast(s16x8, make_uint4(h[0], h[1], h[2], h[3]));
  al = __builtin_bit_cast(s16x8, make_uint4(l[0], l[1], l[2], l[3]));
}

// Eight consecutive output elements at index i (a multiple of 8) in one 16-byte
// store (two for fp32). The 16-bit outputs are written once and never read back
// by this kernel, so their stores are nontemporal (streamed past the caches): the
// write-bound fast mode measured 104 -> 88 us (4-bit) and 108 -> 96 us (6-bit) per
// 1M vectors, the compute-bound accurate mode unchanged.
template <int OUT>
__device__ __forceinline__ void store8(void* out, int64_t i, f32x4 u, f32x4 v) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (OUT == WN_F32) {
    float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + i);
    o[0] = make_float4(u[0], u[1], u[2], u[3]);
    o[1] = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (OUT == WN_BF16) {
    const u32x4 w = {pack_bf16(u[0], u[1]), pack_bf16(u[2], u[3]), pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + i));
  } else {
    const u32x4 w = {pack_f16(u[0], u[1]), pack_f16(u[2], u[3]), pack_f16(v[0], v[1]), pack_f16(v[2], v[3])};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + i));
  }
}

// LDS row of output dim d in the Pi^T planes. Row 16t + 4g + j of output tile t
// lands in lane group g, element j; placing dim d = 32a + 8g + 4b + j at tile 2a + b
// gives lane group g the dims 32a + 8g .. +7 of each a: four 16-byte stores per row,
// the four lane groups of a row covering 64 contiguous bytes per store.
__device__ __forceinline__ int pit_row(int d) {
  return (d & ~31) | (((d >> 2) & 1) << 4) | (((d >> 3) & 3) << 2) | (d & 3);
}

template <int BW, bool FAST, int OUT, bool PAGED>
__global__ __launch_bounds__(dq_waves<FAST>() * 64) __attribute__((amdgpu_waves_per_eu(2))) void tq_dequant_kernel(
    DqArgs a) {
  constexpr int kDqWaves = dq_waves<FAST>();
  constexpr int D = kDqD, NB = D * BW / 8, PLANES = FAST ? 1 : 2;
  // 16-row tiles per pass: each Pi^T operand read from LDS feeds RT MFMAs; four in the
  // accurate mode (half the LDS reads per row), two in the fast mode, whose registers
  // keep it at four waves per SIMD
  constexpr int RT = FAST ? 2 : 3, kRows = 16 * RT;
  __shared__ __align__(16) uint16_t pit[PLANES][D * kPiRow];  // Pi^T: bf16 hi and lo, or fp16
  __shared__ DqTab<BW> tab;
  __shared__ uint32_t pace_words[8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Pi^T planes: pit[h][pit_row(n) * kPiRow + k] = split(Pi[k][n])
  for_strided<D * D / 2, kDqWaves * 64>(tid, [&](int i) {
    const int k = i / (D / 2), n2 = 2 * (i % (D / 2));  // two columns of row k
    const float2 x = *reinterpret_cast<const float2*>(a.pi + k * D + n2);
    const int m = pit_row(n2);  // n2 even: dims n2, n2 + 1 sit in rows m, m + 1
    if constexpr (FAST) {
      const uint32_t h = pack_f16(x.x, x.y);
      pit[0][m * kPiRow + k] = uint16_t(h & 0xffffu);
      pit[0][(m + 1) * kPiRow + k] = uint16_t(h >> 16);
    } else {
      const uint32_t h = pack_bf16(x.x, x.y);
      const uint32_t l = pack_bf16(x.x - bf16_lo(h), x.y - bf16_hi(h));
      pit[0][m * kPiRow + k] = uint16_t(h & 0xffffu);
      pit[0][(m + 1) * kPiRow + k] = uint16_t(h >> 16);
      pit[PLANES - 1][m * kPiRow + k] = uint16_t(l & 0xffffu);
      pit[PLANES - 1][(m + 1) * kPiRow + k] = uint16_t(l >> 16);
    }
  });
  stage_dq_tab<BW, FAST>(a.cb, tab, tid);
  // the accurate mode paces the two waves of a SIMD (Pace); the fast mode's four
  // waves per SIMD come from two work-groups and are not paced
  const Pace pace = make_pace<8>(pace_words, __builtin_amdgcn_readfirstlane(wave) & 7);
  __syncthreads();

  const int g = lane >> 4, c16 = lane & 15;
  const int64_t passes = (a.N + kRows - 1) / kRows, stride = int64_t(gridDim.x) * kDqWaves;
  // Loads and stores share one in-order counter (vmcnt), so a wait for a load also
  // waits for every store issued before it. The pipeline is laid out so that no wait
  // covers the stores of the pass just finished:
  //  - two code buffers alternate (no register copies, which the compiler would make
  //    wait for the loads that fill them), the next pass's codes are loaded before
  //    this pass's stores, and paged mode loads page ids one more pass ahead;
  //  - the first pass is peeled, so that the loop is entered, like its back edge,
  //    with stores after the last loads;
  //  - no store is conditional: rows past N read row N - 1 (every load is in
  //    bounds) and store to row N - 1, the same bits that row's own lane writes
  //    (equal inputs, equal MFMA column), so no path skips the stores.
  auto page_ids = [&](int64_t pass, int32_t (&pg)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) pg[rt] = PAGED ? row_page(a, pass * kRows + 16 * rt + c16) : 0;
  };
  // codes 32g .. 32g+31 of row r0 + 16 rt + c16 and that row's norm
  auto load_pass = [&](int64_t pass, const int32_t (&pg)[RT], uint32_t (&cw)[RT][BW], uint32_t (&nh)[RT]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const uint8_t* p;
      const uint16_t* n;
      row_src<NB, PAGED>(a, pass * kRows + 16 * rt + c16, pg[rt], p, n);
      load_codes32<BW>(p, g, cw[rt]);
      nh[rt] = *n;
    }
  };
  auto compute_pass = [&](const uint32_t (&cw)[RT][BW], f32x4 (&acc)[RT][8]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // keeps the scheduler from hoisting the LDS reads of later k-steps (register
      // pressure past two waves per SIMD)
      __builtin_amdgcn_sched_barrier(0);
      s16x8 yh[RT], yl[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        uint32_t cs[2];
        step_codes<BW>(cw[rt], s, cs);
        codes_to_a<BW, FAST>(cs, tab, yh[rt], yl[rt]);
      }
      // kDqTU output tiles at a time, each product type over all of them before the
      // next, so that the three updates of an accumulator are 2 * kDqTU MFMAs apart
#pragma unroll
      for (int t0 = 0; t0 < 8; t0 += kDqTU) {
        s16x8 ph[kDqTU], pl[kDqTU];
#pragma unroll
        for (int u = 0; u < kDqTU; ++u) {
          const int off = (16 * (t0 + u) + c16) * kPiRow + 32 * g + 8 * s;
          ph[u] = *reinterpret_cast<const s16x8*>(&pit[0][off]);
          if constexpr (!FAST) pl[u] = *reinterpret_cast<const s16x8*>(&pit[PLANES - 1][off]);
        }
        if constexpr (FAST) {
#pragma unroll
          for (int u = 0; u < kDqTU; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
              acc[rt][t0 + u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  __builtin_bit_cast(f16x8, ph[u]), __builtin_bit_cast(f16x8, yh[rt]), acc[rt][t0 + u], 0, 0, 0);
        } else {
#pragma unroll
          for (int u = 0; u < kDqTU; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
              acc[rt][t0 + u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph[u], yh[rt], acc[rt][t0 + u], 0, 0, 0);
#pragma unroll
          for (int u = 0; u < kDqTU; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
              acc[rt][t0 + u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl[u], yh[rt], acc[rt][t0 + u], 0, 0, 0);
#pragma unroll
          for (int u = 0; u < kDqTU; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
              acc[rt][t0 + u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph[u], yl[rt], acc[rt][t0 + u], 0, 0, 0);
        }
      }
    }
  };
  auto store_pass = [&](int64_t pass, const uint32_t (&nh)[RT], const f32x4 (&acc)[RT][8]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      int64_t row = pass * kRows + 16 * rt + c16;
      row = row < a.N ? row : a.N - 1;
      const float nv = f16_to_f32(uint16_t(nh[rt]));
#pragma unroll
      for (int c = 0; c < 4; ++c)
        store8<OUT>(a.out, row * D + 32 * c + 8 * g, acc[rt][2 * c] * nv, acc[rt][2 * c + 1] * nv);
    }
  };
  // the wave's passes still to do, this one included (pacing of the two waves of a SIMD)
  int64_t pass = int64_t(blockIdx.x) * kDqWaves + wave;
  uint32_t left = pass < passes ? uint32_t((passes - pass + stride - 1) / stride) : 0u;
  // One pass: page ids two passes ahead, codes of the next pass, then this pass.
  auto half = [&](int64_t pass, const uint32_t (&cur)[RT][BW], const uint32_t (&ncur)[RT], uint32_t (&nxt)[RT][BW],
                  uint32_t (&nnxt)[RT], const int32_t (&pg_nxt)[RT], int32_t (&pg_after)[RT]) {
    uint32_t partner_left = 0;
    if constexpr (!FAST) {
      pace.publish(left);
      partner_left = pace.partner_left();
    }
    page_ids(pass + 2 * stride, pg_after);
    load_pass(pass + stride, pg_nxt, nxt, nnxt);
    f32x4 acc[RT][8];
    compute_pass(cur, acc);
    store_pass(pass, ncur, acc);
    if constexpr (!FAST) pace_step(left, partner_left);
    --left;
  };

  if (pass >= passes) return;
  uint32_t b0[RT][BW], b1[RT][BW];
  uint32_t n0[RT], n1[RT];  // fp16 bits, one register each (a packed pair would wait for both loads)
  int32_t pa[RT], pb[RT];
  page_ids(pass, pa);
  load_pass(pass, pa, b0, n0);
  page_ids(pass + stride, pb);
  half(pass, b0, n0, b1, n1, pb, pa);
  pass += stride;
  // here b1 holds this pass's codes and pa the pages of the pass after it
  while (pass < passes) {
    half(pass, b1, n1, b0, n0, pa, pb);
    pass += stride;
    if (pass >= passes) break;
    half(pass, b0, n0, b1, n1, pb, pa);
    pass += stride;
  }
  if constexpr (!FAST) pace.publish(0);
}

using DqFn = void (*)(DqArgs);

template <bool FAST, int OUT, bool PAGED>
DqFn pick_dq(int bw) {
  switch (bw) {
    case 2: return tq_dequant_kernel<2, FAST, OUT, PAGED>;
    case 3: return tq_dequant_kernel<3, FAST, OUT, PAGED>;
    case 4: return tq_dequant_kernel<4, FAST, OUT, PAGED>;
    case 5: return tq_dequant_kernel<5, FAST, OUT, PAGED>;
    case 6: return tq_dequant_kernel<6, FAST, OUT, PAGED>;
    case 8: return tq_dequant_kernel<8, FAST, OUT, PAGED>;
  }
  return nullptr;
}

template <int OUT>
DqFn pick_dq_out(int bw, int fast, bool paged) {
  if (paged) return fast ? pick_dq<true, OUT, true>(bw) : pick_dq<false, OUT, true>(bw);
  return fast ? pick_dq<true, OUT, false>(bw) : pick_dq<false, OUT, false>(bw);
}

// Magic number of r / L for every r < 2^32 (Granlund and Montgomery, Figure 4.1).
void set_plane_divisor(DqArgs& a) {
  const uint64_t d = uint64_t(a.L);
  int l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  a.lm = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  a.ls1 = l < 1 ? l : 1;
  a.ls2 = l > 1 ? l - 1 : 0;
}

int launch_dq(DqArgs& a, int bw, int fast, int out_dtype, hipStream_t st, const char* what) {
  if (a.N == 0) return WN_OK;
  WN_REQUIRE(a.N < (int64_t(1) << 31) && a.L < (int64_t(1) << 31), WN_E_INVALID, "%s: %lld rows (2^31 max)", what,
             (long long)a.N);
  set_plane_divisor(a);
  const bool paged = a.table != nullptr;
  const DqFn fn = out_dtype == WN_F32    ? pick_dq_out<WN_F32>(bw, fast, paged)
                  : out_dtype == WN_BF16 ? pick_dq_out<WN_BF16>(bw, fast, paged)
                                         : pick_dq_out<WN_F16>(bw, fast, paged);
  WN_REQUIRE(fn, WN_E_UNSUPPORTED, "%s: bit width %d not compiled", what, bw);
  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (cus <= 0) cus = 256;
  const int waves = fast ? dq_waves<true>() : dq_waves<false>();
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, waves * 64, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int64_t rows = fast ? 32 : 48;  // rows per pass (16 * RT of the kernel)
  const int64_t want = (a.N + rows * waves - 1) / (rows * waves);
  const int64_t grid = want < int64_t(per_cu) * cus ? want : int64_t(per_cu) * cus;
  hipLaunchKernelGGL(fn, dim3(unsigned(grid)), dim3(waves * 64), 0, st, a);
  return check_launch(what);
}

}  // namespace
}  // namespace wn

using namespace wn;

extern "C" int wn_tq_dequant(const uint8_t* packed, const uint16_t* norms, int64_t planes, int64_t L,
                             int64_t plane_rows, const float* centroids, const float* pi, int bw, int D, void* out,
                             int out_dtype, int fast, void* stream) {
  clear_error();
  WN_REQUIRE(D == kDqD, WN_E_UNSUPPORTED, "wn_tq_dequant: head_dim %d (128 only)", D);
  WN_REQUIRE(planes >= 0 && L >= 0 && plane_rows >= L, WN_E_INVALID,
             "wn_tq_dequant: bad sizes planes=%lld L=%lld plane_rows=%lld", (long long)planes, (long long)L,
             (long long)plane_rows);
  WN_REQUIRE(out_dtype == WN_F32 || out_dtype == WN_BF16 || out_dtype == WN_F16, WN_E_INVALID,
             "wn_tq_dequant: output dtype %d", out_dtype);
  if (planes == 0 || L == 0) return WN_OK;
  WN_REQUIRE(packed && norms && centroids && pi && out, WN_E_INVALID, "wn_tq_dequant: null pointer");
  WN_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
             WN_E_INVALID, "wn_tq_dequant: packed and out must be 16-byte aligned");
  DqArgs a{};
  a.packed = packed;
  a.norms = norms;
  a.pi = pi;
  a.cb = centroids;
  a.out = out;
  a.N = planes * L;
  a.L = L;
  a.plane_rows = plane_rows;
  a.table = nullptr;
  return launch_dq(a, bw, fast, out_dtype, static_cast<hipStream_t>(stream), "wn_tq_dequant");
}

extern "C" int wn_dequantize_history(const uint8_t* pages, int64_t page_stride, int64_t head_stride,
                                     const uint16_t* norms, int64_t norm_page_stride, int64_t norm_head_stride,
                                     const int32_t* table_row, int L, int Hkv, int S, const float* centroids,
                                     const float* pi, int bw, int D, void* out, int out_dtype, int fast,
                                     void* stream) {
  clear_error();
  WN_REQUIRE(D == kDqD, WN_E_UNSUPPORTED, "wn_dequantize_history: head_dim %d (128 only)", D);
  WN_REQUIRE(L >= 0 && Hkv > 0 && S > 0 && (S & (S - 1)) == 0, WN_E_INVALID,
             "wn_dequantize_history: bad sizes L=%d Hkv=%d S=%d", L, Hkv, S);
  WN_REQUIRE(out_dtype == WN_F32 || out_dtype == WN_BF16 || out_dtype == WN_F16, WN_E_INVALID,
             "wn_dequantize_history: output dtype %d", out_dtype);
  if (L == 0) return WN_OK;
  WN_REQUIRE(pages && norms && table_row && centroids && pi && out, WN_E_INVALID,
             "wn_dequantize_history: null pointer");
  WN_REQUIRE(reinterpret_cast<uintptr_t>(pages) % 16 == 0 && page_stride % 16 == 0 && head_stride % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(out) % 16 == 0,
             WN_E_INVALID, "wn_dequantize_history: pages, their strides and out must be 16-byte aligned");
  DqArgs a{};
  a.packed = pages;
  a.norms = norms;
  a.pi = pi;
  a.cb = centroids;
  a.out = out;
  a.N = int64_t(Hkv) * L;
  a.L = L;
  a.plane_rows = L;
  a.table = table_row;
  a.log2S = ilog2(S);
  a.psp = page_stride;
  a.psh = head_stride;
  a.nsp = norm_page_stride;
  a.nsh = norm_head_stride;
  return launch_dq(a, bw, fast, out_dtype, static_cast<hipStream_t>(stream), "wn_dequantize_history");
}
