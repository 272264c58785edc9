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
// below 2^-16 of the product; the output is rounded to bf16 anyway).
//
// A persistent work-group of four waves stages Pi^T as bf16 hi and lo planes in LDS
// once; each wave then takes passes of 32 rows (two 16-row tiles) and computes the
// transposed product out^T = Pi^T y^T, so that a lane ends with four consecutive
// output dims of one row:
//   A  (output-dim tile t, k-step s): lane l holds Pi[32s + 8(l/16) .. +8][16t + l % 16],
//      one 16-byte LDS read from the transposed plane (padded rows, conflict free);
//   B  (row tile, k-step s): lane l holds the codebook values of row l % 16 at dims
//      32s + 8(l/16) .. +8, looked up from a byte-indexed pair table for 4-bit codes
//      (one entry = hi or lo of the two codes of a byte) or per code;
//   D  lane l holds output dims 16t + 4(l/16) .. +3 of row l % 16; the norm rescale
//      and the cast happen on the way out, four values in one 8- or 16-byte store.
#include "wn_common.h"

namespace wn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kDqD = 128;
constexpr int kDqWaves = 4;
constexpr int kPiRow = 136;  // bf16 per row of a Pi^T plane: 128 + 8 pad (272 B rows)

struct DqArgs {
  const uint8_t* packed;
  const uint16_t* norms;  // fp16
  const float* pi;        // (D, D) fp32
  const float* cb;        // 2^bw fp32 centroids
  void* out;              // (N, D), row r at r * D
  int64_t N;              // rows
  int64_t L;              // rows per plane (plane = r / L, position t = r % L)
  int64_t plane_rows;     // strided mode: rows between consecutive planes in `packed`/`norms`
  const int32_t* table;   // paged mode (not null): page of position t is table[t >> log2S]
  int log2S;
  int64_t psp, psh;       // paged: packed page / plane strides, bytes
  int64_t nsp, nsh;       // paged: norm page / plane strides, elements
  int out_dtype;
};

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Source of row r (clamped to a valid row; the caller masks the stores).
template <int NB>
__device__ __forceinline__ void row_src(const DqArgs& a, int64_t r, const uint8_t*& p, const uint16_t*& n) {
  r = r < a.N ? r : a.N - 1;
  const int64_t plane = r / a.L, t = r - plane * a.L;
  if (a.table) {
    const int64_t page = a.table[t >> a.log2S];
    const int64_t slot = t & ((int64_t(1) << a.log2S) - 1);
    p = a.packed + page * a.psp + plane * a.psh + slot * NB;
    n = a.norms + page * a.nsp + plane * a.nsh + slot;
  } else {
    const int64_t src = plane * a.plane_rows + t;
    p = a.packed + src * NB;
    n = a.norms + src;
  }
}

// The BW bytes holding codes 8q..8q+7 of a row (LSB-first), as little-endian words.
template <int BW>
__device__ __forceinline__ void load_codes8(const uint8_t* row, int q, uint32_t (&w)[2]) {
  const uint8_t* p = row + BW * q;
  if constexpr (BW == 4) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
    w[1] = 0;
  } else if constexpr (BW == 8) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    w[0] = x.x;
    w[1] = x.y;
  } else if constexpr (BW == 2) {
    w[0] = *reinterpret_cast<const uint16_t*>(p);
    w[1] = 0;
  } else {  // 3, 5, 6: byte-aligned groups of BW bytes
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < BW; ++i) {
      const uint32_t b = p[i];
      if (i < 4) w0 |= b << (8 * i);
      else w1 |= b << (8 * (i - 4));
    }
    w[0] = w0;
    w[1] = w1;
  }
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

template <int BW>
__device__ __forceinline__ void stage_dq_tab(const float* cb, DqTab<BW>& t, int tid) {
  if constexpr (BW == 4) {
    for (int b = tid; b < 256; b += kDqWaves * 64) {
      const float x0 = cb[b & 15], x1 = cb[b >> 4];
      const uint32_t h = pack_bf16(x0, x1);
      t.hi[b] = h;
      t.lo[b] = pack_bf16(x0 - bf16_lo(h), x1 - bf16_hi(h));
    }
  } else {
    constexpr int L = 1 << BW;
    for (int i = tid; i < (L + 1) / 2; i += kDqWaves * 64) {
      const float x0 = cb[2 * i], x1 = 2 * i + 1 < L ? cb[2 * i + 1] : 0.f;
      const uint32_t h = pack_bf16(x0, x1);
      t.hi[i] = h;
      t.lo[i] = pack_bf16(x0 - bf16_lo(h), x1 - bf16_hi(h));
    }
  }
}

// 16-bit entry of code c in a per-code table.
__device__ __forceinline__ uint32_t half_of(const uint32_t* t, uint32_t c) {
  const uint32_t w = t[c >> 1];
  return (c & 1u) ? (w >> 16) : (w & 0xffffu);
}

// MFMA operands of 8 codes (little-endian words w): hi and lo bf16 of their values.
template <int BW>
__device__ __forceinline__ void codes_to_a(const uint32_t (&w)[2], const DqTab<BW>& t, s16x8& ah, s16x8& al) {
  uint32_t h[4], l[4];
  if constexpr (BW == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t b = (w[0] >> (8 * j)) & 0xffu;
      h[j] = t.hi[b];
      l[j] = t.lo[b];
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
      l[j] = half_of(t.lo, c[2 * j]) | (half_of(t.lo, c[2 * j + 1]) << 16);
    }
  }
  ah = __builtin_bit_cast(s16x8, make_uint4(h[0], h[1], h[2], h[3]));
  al = __builtin_bit_cast(s16x8, make_uint4(l[0], l[1], l[2], l[3]));
}

// Four consecutive output elements at index i (a multiple of 4) in one store.
__device__ __forceinline__ void store4(void* out, int64_t i, int dtype, f32x4 v) {
  if (dtype == WN_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (dtype == WN_BF16) {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + i) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
  } else {
    const uint32_t lo = uint32_t(f32_to_f16(v[0])) | (uint32_t(f32_to_f16(v[1])) << 16);
    const uint32_t hi = uint32_t(f32_to_f16(v[2])) | (uint32_t(f32_to_f16(v[3])) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + i) = make_uint2(lo, hi);
  }
}

template <int BW>
__global__ __launch_bounds__(kDqWaves * 64) void tq_dequant_kernel(DqArgs a) {
  constexpr int D = kDqD, NB = D * BW / 8;
  __shared__ __align__(16) uint16_t pit[2][D * kPiRow];  // Pi^T, bf16 hi and lo planes
  __shared__ DqTab<BW> tab;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Pi^T planes: pit[h][n * kPiRow + k] = split(Pi[k][n])
  for (int i = tid; i < D * D / 2; i += kDqWaves * 64) {
    const int k = i / (D / 2), n2 = 2 * (i % (D / 2));  // two columns of row k
    const float2 x = *reinterpret_cast<const float2*>(a.pi + k * D + n2);
    const uint32_t h = pack_bf16(x.x, x.y);
    const uint32_t l = pack_bf16(x.x - bf16_lo(h), x.y - bf16_hi(h));
    pit[0][n2 * kPiRow + k] = uint16_t(h & 0xffffu);
    pit[0][(n2 + 1) * kPiRow + k] = uint16_t(h >> 16);
    pit[1][n2 * kPiRow + k] = uint16_t(l & 0xffffu);
    pit[1][(n2 + 1) * kPiRow + k] = uint16_t(l >> 16);
  }
  stage_dq_tab<BW>(a.cb, tab, tid);
  __syncthreads();

  const int g = lane >> 4, c16 = lane & 15;
  const int64_t passes = (a.N + 31) / 32;
  for (int64_t pass = int64_t(blockIdx.x) * kDqWaves + wave; pass < passes;
       pass += int64_t(gridDim.x) * kDqWaves) {
    const int64_t r0 = pass * 32;
    // codes of row r0 + 16 rt + c16 (this lane's A rows) and norms of the D rows
    uint32_t cw[2][4][2];
    float nv[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const uint8_t* p;
      const uint16_t* n;
      row_src<NB>(a, r0 + 16 * rt + c16, p, n);
#pragma unroll
      for (int s = 0; s < 4; ++s) load_codes8<BW>(p, 4 * s + g, cw[rt][s]);
      nv[rt] = f16_to_f32(*n);
    }
    f32x4 acc[2][8];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s16x8 yh[2], yl[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) codes_to_a<BW>(cw[rt][s], tab, yh[rt], yl[rt]);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int off = (16 * t + c16) * kPiRow + 32 * s + 8 * g;
        const s16x8 ph = *reinterpret_cast<const s16x8*>(&pit[0][off]);
        const s16x8 pl = *reinterpret_cast<const s16x8*>(&pit[1][off]);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, yh[rt], acc[rt][t], 0, 0, 0);
          acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, yh[rt], acc[rt][t], 0, 0, 0);
          acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, yl[rt], acc[rt][t], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int64_t row = r0 + 16 * rt + c16;
      if (row < a.N) {
#pragma unroll
        for (int t = 0; t < 8; ++t) store4(a.out, row * D + 16 * t + 4 * g, a.out_dtype, acc[rt][t] * nv[rt]);
      }
    }
  }
}

using DqFn = void (*)(DqArgs);

DqFn pick_dq(int bw) {
  switch (bw) {
    case 2: return tq_dequant_kernel<2>;
    case 3: return tq_dequant_kernel<3>;
    case 4: return tq_dequant_kernel<4>;
    case 5: return tq_dequant_kernel<5>;
    case 6: return tq_dequant_kernel<6>;
    case 8: return tq_dequant_kernel<8>;
  }
  return nullptr;
}

int launch_dq(DqArgs& a, int bw, hipStream_t st, const char* what) {
  if (a.N == 0) return WN_OK;
  const DqFn fn = pick_dq(bw);
  WN_REQUIRE(fn, WN_E_UNSUPPORTED, "%s: bit width %d not compiled", what, bw);
  int dev = 0, cus = 0;
  (void)hipGetDevice(&dev);
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (cus <= 0) cus = 256;
  const int64_t want = (a.N + 32 * kDqWaves - 1) / (32 * kDqWaves);
  const int64_t grid = want < 2 * int64_t(cus) ? want : 2 * int64_t(cus);
  hipLaunchKernelGGL(fn, dim3(unsigned(grid)), dim3(kDqWaves * 64), 0, st, a);
  return check_launch(what);
}

}  // namespace
}  // namespace wn

using namespace wn;

extern "C" int wn_tq_dequant(const uint8_t* packed, const uint16_t* norms, int64_t planes, int64_t L,
                             int64_t plane_rows, const float* centroids, const float* pi, int bw, int D, void* out,
                             int out_dtype, void* stream) {
  clear_error();
  WN_REQUIRE(D == kDqD, WN_E_UNSUPPORTED, "wn_tq_dequant: head_dim %d (128 only)", D);
  WN_REQUIRE(planes >= 0 && L >= 0 && plane_rows >= L, WN_E_INVALID,
             "wn_tq_dequant: bad sizes planes=%lld L=%lld plane_rows=%lld", (long long)planes, (long long)L,
             (long long)plane_rows);
  WN_REQUIRE(out_dtype == WN_F32 || out_dtype == WN_BF16 || out_dtype == WN_F16, WN_E_INVALID,
             "wn_tq_dequant: output dtype %d", out_dtype);
  if (planes == 0 || L == 0) return WN_OK;
  WN_REQUIRE(packed && norms && centroids && pi && out, WN_E_INVALID, "wn_tq_dequant: null pointer");
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
  a.out_dtype = out_dtype;
  return launch_dq(a, bw, static_cast<hipStream_t>(stream), "wn_tq_dequant");
}

extern "C" int wn_dequantize_history(const uint8_t* pages, int64_t page_stride, int64_t head_stride,
                                     const uint16_t* norms, int64_t norm_page_stride, int64_t norm_head_stride,
                                     const int32_t* table_row, int L, int Hkv, int S, const float* centroids,
                                     const float* pi, int bw, int D, void* out, int out_dtype, void* stream) {
  clear_error();
  WN_REQUIRE(D == kDqD, WN_E_UNSUPPORTED, "wn_dequantize_history: head_dim %d (128 only)", D);
  WN_REQUIRE(L >= 0 && Hkv > 0 && S > 0 && (S & (S - 1)) == 0, WN_E_INVALID,
             "wn_dequantize_history: bad sizes L=%d Hkv=%d S=%d", L, Hkv, S);
  WN_REQUIRE(out_dtype == WN_F32 || out_dtype == WN_BF16 || out_dtype == WN_F16, WN_E_INVALID,
             "wn_dequantize_history: output dtype %d", out_dtype);
  if (L == 0) return WN_OK;
  WN_REQUIRE(pages && norms && table_row && centroids && pi && out, WN_E_INVALID,
             "wn_dequantize_history: null pointer");
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
  a.out_dtype = out_dtype;
  return launch_dq(a, bw, static_cast<hipStream_t>(stream), "wn_dequantize_history");
}
