// TurboQuant quantize / bit-pack / page scatter (the KV append path) and the
// standalone pack, unpack and dequantize ops, for gfx950.
//
// quantize (turboquant_kv/cache.py:108-115):
//   n = max(||x||_2, 1e-10);  y = (x / n) Pi^T;  code = #{boundaries < y}
// Each wave handles four vectors at once. The squared norm and the rotation are
// accumulated in float64 from exact fp32 inputs and rounded once to fp32, and
// x / n is the correctly rounded fp32 quotient, so every code is the bucket of
// the correctly rounded fp32 y; an fp32 GEMM elsewhere can differ from it only
// when its own rounding error crosses a boundary.
#include "wn_common.h"

namespace wn {
namespace {

constexpr int kQBlock = 256;                // 4 waves
constexpr int kVW = 4;                      // vectors a wave quantizes together
constexpr int kVecPerBlock = 4 * kVW;       // 16 per work-group

struct QuantSide {
  const void* x;
  int64_t sb, sh, sn;  // element strides of (B, H, n, D)
  const float* pi;
  const float* bnd;
  int bw;
  uint8_t* pages;  // scatter mode
  int64_t psp, psh;
  uint16_t* norms;
  int64_t nsp, nsh;
  uint8_t* codes_out;  // flat mode
  float* norms_out;
};

struct QuantArgs {
  QuantSide side[2];
  const int32_t* table;
  const int32_t* start_pos;
  int64_t tsb;
  int64_t total;  // vectors per side = B*H*n
  int H, n, log2S, num_pages, max_pages, x_dtype, scatter;
};

__device__ __forceinline__ uint32_t bucketize(const float* bnd, int bw, float y) {
  // #{b < y} over the 2^bw - 1 ascending boundaries (torch.bucketize, right=False).
  uint32_t pos = 0;
  for (int step = 1 << (bw - 1); step > 0; step >>= 1)
    if (bnd[pos + step - 1] < y) pos += step;
  return pos;
}

// Byte k of the LSB-first packing of `codes` (D codes of bw bits).
__device__ __forceinline__ uint8_t packed_byte(const uint8_t* codes, int k, int bw, int D) {
  const int bit0 = 8 * k;
  uint32_t v = 0;
  for (int d = bit0 / bw; d < D && d * bw < bit0 + 8; ++d) {
    const int off = d * bw - bit0;
    const uint32_t c = codes[d];
    v |= off >= 0 ? (c << off) : (c >> (-off));
  }
  return uint8_t(v & 0xffu);
}

// Each wave quantizes kVW vectors together (lane j forms output dims j, j+64 of all
// of them: 2*kVW independent float64 accumulation chains), so the 128-term dot
// products overlap instead of running one after another; sixteen vectors per
// work-group keep even a 4096-vector append spread over the whole GPU. Pi is
// staged in LDS in 16-byte rows of stride D+4 floats: the 16 lanes a 16-byte LDS
// read serves hit distinct banks.
template <int D>
__global__ __launch_bounds__(kQBlock) void quantize_kernel(QuantArgs a) {
  constexpr int LD = D + 4;
  constexpr int KPL = D / 64;  // output dims per lane
  __shared__ __align__(16) float pis[D * LD];
  __shared__ float bnd[255];
  __shared__ __align__(16) double xs[4][kVW][D];
  __shared__ uint8_t cs[4][kVW][D];

  const QuantSide& sd = a.side[blockIdx.y];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int nb = (1 << sd.bw) - 1;
  const int64_t v0 = int64_t(blockIdx.x) * kVecPerBlock;
  if (v0 >= a.total) return;
  for (int i = tid; i < D * D / 4; i += kQBlock) {
    const float4 pv = reinterpret_cast<const float4*>(sd.pi)[i];
    *reinterpret_cast<float4*>(pis + (4 * i / D) * LD + (4 * i) % D) = pv;
  }
  for (int i = tid; i < nb; i += kQBlock) bnd[i] = sd.bnd[i];
  __syncthreads();

  const int64_t vw = v0 + int64_t(w) * kVW;  // this wave's first vector
  float nrm[kVW];
#pragma unroll
  for (int t = 0; t < kVW; ++t) {
    const int64_t v = vw + t;
    nrm[t] = 1e-10f;
    if (v < a.total) {  // wave-uniform
      const int i = int(v % a.n);
      const int h = int((v / a.n) % a.H);
      const int b = int(v / (int64_t(a.n) * a.H));
      const int64_t xo = b * sd.sb + h * sd.sh + i * sd.sn;
      float xv[KPL];
      double ss = 0.0;
#pragma unroll
      for (int k = 0; k < KPL; ++k) {
        xv[k] = load_elem(sd.x, xo + lane + 64 * k, a.x_dtype);
        ss = fma(double(xv[k]), double(xv[k]), ss);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
      nrm[t] = fmaxf(float(sqrt(ss)), 1e-10f);
#pragma unroll
      for (int k = 0; k < KPL; ++k) xs[w][t][lane + 64 * k] = double(float(double(xv[k]) / double(nrm[t])));
    } else {
#pragma unroll
      for (int k = 0; k < KPL; ++k) xs[w][t][lane + 64 * k] = 0.0;
    }
  }
  wave_lds_sync();
  // y[t][k] = sum_d (x_t / n_t)[d] * Pi[lane + 64k][d], exact products, float64 sums
  double y[kVW][KPL];
#pragma unroll
  for (int t = 0; t < kVW; ++t)
#pragma unroll
    for (int k = 0; k < KPL; ++k) y[t][k] = 0.0;
#pragma unroll 2
  for (int d = 0; d < D; d += 4) {
    float4 pr[KPL];
#pragma unroll
    for (int k = 0; k < KPL; ++k) pr[k] = *reinterpret_cast<const float4*>(pis + (lane + 64 * k) * LD + d);
#pragma unroll
    for (int t = 0; t < kVW; ++t) {
      const double2 xa = *reinterpret_cast<const double2*>(&xs[w][t][d]);
      const double2 xb = *reinterpret_cast<const double2*>(&xs[w][t][d + 2]);
#pragma unroll
      for (int k = 0; k < KPL; ++k) {
        y[t][k] = fma(xa.x, double(pr[k].x), y[t][k]);
        y[t][k] = fma(xa.y, double(pr[k].y), y[t][k]);
        y[t][k] = fma(xb.x, double(pr[k].z), y[t][k]);
        y[t][k] = fma(xb.y, double(pr[k].w), y[t][k]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kVW; ++t)
#pragma unroll
    for (int k = 0; k < KPL; ++k) cs[w][t][lane + 64 * k] = uint8_t(bucketize(bnd, sd.bw, float(y[t][k])));
  wave_lds_sync();

  const int S = 1 << a.log2S;
  const int NB = D * sd.bw / 8;
#pragma unroll
  for (int t = 0; t < kVW; ++t) {
    const int64_t v = vw + t;
    if (v >= a.total) break;  // wave-uniform
    const int i = int(v % a.n);
    const int h = int((v / a.n) % a.H);
    const int b = int(v / (int64_t(a.n) * a.H));
    if (a.scatter) {
      const int pos = a.start_pos[b] + i;
      const int col = pos >> a.log2S;
      const int pid = (pos >= 0 && col < a.max_pages) ? a.table[b * a.tsb + col] : -1;
      if (pid >= 0 && pid < a.num_pages) {
        const int slot = pos & (S - 1);
        uint8_t* row = sd.pages + pid * sd.psp + h * sd.psh + int64_t(slot) * NB;
        for (int k = lane; k < NB; k += 64) row[k] = packed_byte(cs[w][t], k, sd.bw, D);
        if (lane == 0) sd.norms[pid * sd.nsp + h * sd.nsh + slot] = f32_to_f16(nrm[t]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < KPL; ++k) sd.codes_out[v * D + lane + 64 * k] = cs[w][t][lane + 64 * k];
      if (lane == 0) sd.norms_out[v] = nrm[t];
    }
  }
}

__global__ void pack_kernel(const uint8_t* codes, int64_t rows, int D, int bw, uint8_t* out) {
  const int NB = D * bw / 8;
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= rows * NB) return;
  const int64_t r = e / NB;
  out[e] = packed_byte(codes + r * D, int(e % NB), bw, D);
}

__global__ void unpack_kernel(const uint8_t* packed, int64_t rows, int D, int bw, uint8_t* out) {
  const int NB = D * bw / 8;
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= rows * D) return;
  const int64_t r = e / D;
  const int d = int(e % D);
  const uint8_t* p = packed + r * NB;
  const int bit = d * bw, byte = bit >> 3, sh = bit & 7;
  uint32_t v = uint32_t(p[byte]) >> sh;
  if (sh + bw > 8) v |= uint32_t(p[byte + 1]) << (8 - sh);
  out[e] = uint8_t(v & ((1u << bw) - 1u));
}

// out[r, j] = (sum_d c[code[r, d]] Pi[d, j]) * n[r]  (cache.py:125-131)
template <int D>
__global__ __launch_bounds__(D) void dequantize_kernel(const uint8_t* codes, const uint16_t* norms,
                                                      const float* pi, const float* cb, int bw, void* out,
                                                      int out_dtype) {
  __shared__ float y[D];
  const int64_t r = blockIdx.x;
  const int j = threadIdx.x;
  y[j] = cb[codes[r * D + j] & ((1u << bw) - 1u)];
  __syncthreads();
  float o = 0.f;
#pragma unroll 8
  for (int d = 0; d < D; ++d) o = fmaf(y[d], pi[d * D + j], o);
  store_elem(out, r * D + j, out_dtype, o * f16_to_f32(norms[r]));
}

}  // namespace
}  // namespace wn

using namespace wn;

static int launch_quantize(QuantArgs& a, int sides, int D, hipStream_t st, const char* what) {
  if (a.total == 0) return WN_OK;
  dim3 grid(unsigned((a.total + kVecPerBlock - 1) / kVecPerBlock), sides);
  if (D == 128)
    hipLaunchKernelGGL(quantize_kernel<128>, grid, dim3(kQBlock), 0, st, a);
  else
    hipLaunchKernelGGL(quantize_kernel<64>, grid, dim3(kQBlock), 0, st, a);
  return check_launch(what);
}

extern "C" int wn_append_kv(
    const void* k, int64_t ks_b, int64_t ks_h, int64_t ks_n,
    const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_n, int x_dtype,
    const float* pi_k, const float* boundaries_k, int bw_k,
    const float* pi_v, const float* boundaries_v, int bw_v,
    const int32_t* page_table, int64_t table_stride_b, const int32_t* start_pos,
    uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    int B, int Hkv, int n, int D, int S, int num_pages, int max_pages, void* stream) {
  clear_error();
  WN_REQUIRE(B >= 0 && Hkv > 0 && n >= 0 && num_pages >= 0 && max_pages >= 0, WN_E_INVALID,
             "append: bad sizes B=%d Hkv=%d n=%d", B, Hkv, n);
  WN_REQUIRE(D == 64 || D == 128, WN_E_UNSUPPORTED, "append: head_dim %d not compiled (64, 128)", D);
  WN_REQUIRE(is_pow2(S), WN_E_INVALID, "append: page size %d is not a power of two", S);
  WN_REQUIRE(x_dtype >= WN_F32 && x_dtype <= WN_BF16, WN_E_INVALID, "append: dtype code %d", x_dtype);
  WN_REQUIRE(valid_bw(bw_k) && (!v || valid_bw(bw_v)), WN_E_INVALID, "append: bit widths %d/%d", bw_k,
             bw_v);
  if (int64_t(B) * n == 0) return WN_OK;
  WN_REQUIRE(k && pi_k && boundaries_k && page_table && start_pos && k_pages && k_norms, WN_E_INVALID,
             "append: null operand");
  WN_REQUIRE(!v || (pi_v && boundaries_v && v_pages && v_norms), WN_E_INVALID, "append: null V operand");
  QuantArgs a{};
  a.side[0] = QuantSide{k, ks_b, ks_h, ks_n, pi_k, boundaries_k, bw_k, k_pages, k_stride_p, k_stride_h,
                        k_norms, kn_stride_p, kn_stride_h, nullptr, nullptr};
  if (v)
    a.side[1] = QuantSide{v, vs_b, vs_h, vs_n, pi_v, boundaries_v, bw_v, v_pages, v_stride_p, v_stride_h,
                          v_norms, vn_stride_p, vn_stride_h, nullptr, nullptr};
  a.table = page_table;
  a.start_pos = start_pos;
  a.tsb = table_stride_b;
  a.total = int64_t(B) * Hkv * n;
  a.H = Hkv;
  a.n = n;
  a.log2S = ilog2(S);
  a.num_pages = num_pages;
  a.max_pages = max_pages;
  a.x_dtype = x_dtype;
  a.scatter = 1;
  return launch_quantize(a, v ? 2 : 1, D, static_cast<hipStream_t>(stream), "wn_append_kv");
}

extern "C" int wn_quantize(const void* x, int x_dtype, int64_t rows, int64_t row_stride, const float* pi,
                           const float* boundaries, int bw, int D, uint8_t* codes, float* norms,
                           void* stream) {
  clear_error();
  WN_REQUIRE(rows >= 0, WN_E_INVALID, "quantize: rows %lld", (long long)rows);
  WN_REQUIRE(D == 64 || D == 128, WN_E_UNSUPPORTED, "quantize: head_dim %d not compiled (64, 128)", D);
  WN_REQUIRE(valid_bw(bw), WN_E_INVALID, "quantize: bit width %d", bw);
  WN_REQUIRE(x_dtype >= WN_F32 && x_dtype <= WN_BF16, WN_E_INVALID, "quantize: dtype code %d", x_dtype);
  if (rows == 0) return WN_OK;
  WN_REQUIRE(x && pi && boundaries && codes && norms, WN_E_INVALID, "quantize: null operand");
  QuantArgs a{};
  a.side[0] = QuantSide{x, row_stride, 0, 0, pi, boundaries, bw, nullptr, 0, 0, nullptr, 0, 0, codes, norms};
  a.total = rows;
  a.H = 1;
  a.n = 1;
  a.x_dtype = x_dtype;
  a.scatter = 0;
  return launch_quantize(a, 1, D, static_cast<hipStream_t>(stream), "wn_quantize");
}

extern "C" int wn_pack(const uint8_t* codes, int64_t rows, int D, int bw, uint8_t* packed, void* stream) {
  clear_error();
  WN_REQUIRE(rows >= 0 && D > 0 && valid_bw(bw) && (int64_t(D) * bw) % 8 == 0, WN_E_INVALID,
             "pack: unsupported bit width or shape (rows=%lld D=%d bw=%d)", (long long)rows, D, bw);
  const int64_t total = rows * (D * bw / 8);
  if (total == 0) return WN_OK;
  WN_REQUIRE(codes && packed, WN_E_INVALID, "pack: null operand");
  hipLaunchKernelGGL(pack_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, rows, D, bw, packed);
  return check_launch("wn_pack");
}

extern "C" int wn_unpack(const uint8_t* packed, int64_t rows, int D, int bw, uint8_t* codes, void* stream) {
  clear_error();
  WN_REQUIRE(rows >= 0 && D > 0 && valid_bw(bw) && (int64_t(D) * bw) % 8 == 0, WN_E_INVALID,
             "unpack: unsupported bit width or shape (rows=%lld D=%d bw=%d)", (long long)rows, D, bw);
  const int64_t total = rows * D;
  if (total == 0) return WN_OK;
  WN_REQUIRE(codes && packed, WN_E_INVALID, "unpack: null operand");
  hipLaunchKernelGGL(unpack_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), packed, rows, D, bw, codes);
  return check_launch("wn_unpack");
}

extern "C" int wn_dequantize(const uint8_t* codes, const uint16_t* norms, int64_t rows, const float* pi,
                             const float* centroids, int bw, int D, void* out, int out_dtype, void* stream) {
  clear_error();
  WN_REQUIRE(rows >= 0 && valid_bw(bw), WN_E_INVALID, "dequantize: rows=%lld bw=%d", (long long)rows, bw);
  WN_REQUIRE(D == 64 || D == 128, WN_E_UNSUPPORTED, "dequantize: head_dim %d not compiled (64, 128)", D);
  WN_REQUIRE(out_dtype >= WN_F32 && out_dtype <= WN_BF16, WN_E_INVALID, "dequantize: dtype %d", out_dtype);
  if (rows == 0) return WN_OK;
  WN_REQUIRE(rows < (int64_t(1) << 31), WN_E_INVALID, "dequantize: too many rows");
  WN_REQUIRE(codes && norms && pi && centroids && out, WN_E_INVALID, "dequantize: null operand");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D == 128)
    hipLaunchKernelGGL(dequantize_kernel<128>, dim3(unsigned(rows)), dim3(128), 0, st, codes, norms, pi,
                       centroids, bw, out, out_dtype);
  else
    hipLaunchKernelGGL(dequantize_kernel<64>, dim3(unsigned(rows)), dim3(64), 0, st, codes, norms, pi,
                       centroids, bw, out, out_dtype);
  return check_launch("wn_dequantize");
}
