// TurboQuant quantize / bit-pack / page scatter (the KV append path) and the
// standalone pack, unpack and dequantize ops, for gfx950.
//
// quantize (turboquant_kv/cache.py:108-115):
//   n = max(||x||_2, 1e-10);  y = (x / n) Pi^T;  code = #{boundaries < y}
// A work-group quantizes sixteen vectors (quantize_kernel on the float64 matrix
// cores at head_dim 64 and 128, quantize_any_kernel on the vector ALU at 16, 32 and
// 256). The squared norm and the rotation are
// accumulated in float64 from exact fp32 inputs and rounded once to fp32, and
// x / n is the correctly rounded fp32 quotient, so every code is the bucket of
// the correctly rounded fp32 y; an fp32 GEMM elsewhere can differ from it only
// when its own rounding error crosses a boundary.
#include "wn_common.h"

namespace wn {
namespace {

constexpr int kQBlock = 256;                // 4 waves
constexpr int kVecPerBlock = 16;            // vectors per work-group (the rows of one f64 MFMA tile)

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

// pos[k] = #{b < y[k]} over the 2^bw - 1 ascending boundaries (torch.bucketize,
// right=False), for N values at once: the N binary searches advance in lockstep, so
// each level issues N independent LDS reads instead of one dependent read per value.
template <int N>
__device__ __forceinline__ void bucketize_n(const float* bnd, int bw, const float (&y)[N], uint32_t (&pos)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) pos[k] = 0;
  for (int step = 1 << (bw - 1); step > 0; step >>= 1) {
    float b[N];
#pragma unroll
    for (int k = 0; k < N; ++k) b[k] = bnd[pos[k] + step - 1];
#pragma unroll
    for (int k = 0; k < N; ++k) pos[k] += b[k] < y[k] ? step : 0;
  }
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

// The bw bytes of eight bw-bit codes packed LSB-first, stored at p (p is aligned to
// the largest power of two dividing bw).
__device__ __forceinline__ void store_packed8(uint8_t* p, uint64_t v, int bw) {
  if (bw == 8) {
    *reinterpret_cast<uint2*>(p) = make_uint2(uint32_t(v), uint32_t(v >> 32));
  } else if (bw == 4) {
    *reinterpret_cast<uint32_t*>(p) = uint32_t(v);
  } else if (bw == 2) {
    *reinterpret_cast<uint16_t*>(p) = uint16_t(v);
  } else if (bw == 6) {
    reinterpret_cast<uint16_t*>(p)[0] = uint16_t(v);
    reinterpret_cast<uint16_t*>(p)[1] = uint16_t(v >> 16);
    reinterpret_cast<uint16_t*>(p)[2] = uint16_t(v >> 32);
  } else {
    for (int k = 0; k < bw; ++k) p[k] = uint8_t(v >> (8 * k));
  }
}

// A work-group quantizes sixteen vectors (sixteen per work-group keep even a
// 4096-vector append spread over the whole GPU), in phases that each run over all
// sixteen at once, so a small append costs a few round trips, not one per vector:
//   loads     sixteen threads per vector for x (D/16 consecutive elements each),
//             then the rows of Pi this wave's rotation needs (B operands, from L2 with
//             16-byte loads: Pi is not staged in LDS); in scatter mode threads 0-15
//             look up the start position, later the page, of vector tid.
//   norms     float64 sum of squares over each vector's sixteen threads, n =
//             max(fp32(sqrt), 1e-10), x / n rounded once to fp32 into the LDS rows xs.
//   rotation  y = (x / n) Pi^T on the float64 matrix cores (v_mfma_f64_16x16x4f64:
//             products of fp32 values are exact in float64 and the sums stay in
//             float64), rows = the sixteen vectors, columns = output dims: wave w
//             forms output dims [D/4 w, D/4 (w+1)), D/64 tiles of sixteen. K-step
//             s, slot k (= lane / 16) is input dim (D/4) k + s, so a lane's A
//             operands are D/4 consecutive floats of one xs row and its B operands
//             D/4 consecutive floats of one row of Pi. Output lane l, register i of a
//             tile is vector l/16 + 4i, column l%16.
//   codes     each y is rounded once to fp32 and bucketized into the LDS codes cs
//             (a lane's D/16 searches in lockstep).
//   stores    D/8 threads per vector each pack eight codes (bw bytes) and store
//             them; thread 0 of the vector stores its norm.
template <int D>
__global__ __launch_bounds__(kQBlock) void quantize_kernel(QuantArgs a) {
  constexpr int EPT = D / 16;  // x elements per thread in the norm phase
  constexpr int KS = D / 4;    // K-steps of the rotation (4 input dims each)
  constexpr int TPW = D / 64;  // output tiles of sixteen dims per wave
  constexpr int TPV = D / 8;   // threads per vector in the store phase
  typedef double f64x4 __attribute__((ext_vector_type(4)));
  __shared__ float bnd[255];
  __shared__ __align__(16) float xs[kVecPerBlock][D];
  __shared__ uint8_t cs[kVecPerBlock][D];
  __shared__ float nrms[kVecPerBlock];
  __shared__ int64_t rowoff[kVecPerBlock];  // byte offset of the vector's packed row (-1: skipped)
  __shared__ int64_t nrmoff[kVecPerBlock];  // element offset of its norm

  const QuantSide& sd = a.side[blockIdx.y];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int nb = (1 << sd.bw) - 1;
  const int64_t v0 = int64_t(blockIdx.x) * kVecPerBlock;
  if (v0 >= a.total) return;  // block-uniform
  // destination of vector v0 + tid (threads 0-15): its start position is loaded
  // first, its page-table entry after the norms (the two loads depend), and both are
  // used only by the stores
  const bool dst_thread = tid < kVecPerBlock && v0 + tid < a.total;
  int dst_pos = 0;
  if (dst_thread && a.scatter)
    dst_pos = a.start_pos[int((v0 + tid) / (int64_t(a.n) * a.H))] + int((v0 + tid) % a.n);
  for (int i = tid; i < nb; i += kQBlock) bnd[i] = sd.bnd[i];

  float4 pb[TPW][KS / 4];  // B operands: rows of Pi (from L2, not staged in LDS)
  // norms: vector tid / 16, elements EPT * (tid % 16) ..
  {
    const int vl = tid >> 4, part = tid & 15;
    const int64_t v = v0 + vl;
    float xv[EPT];
    if (v < a.total) {
      const int i = int(v % a.n);
      const int h = int((v / a.n) % a.H);
      const int b = int(v / (int64_t(a.n) * a.H));
      const int64_t xo = b * sd.sb + h * sd.sh + i * sd.sn + EPT * part;
#pragma unroll
      for (int k = 0; k < EPT; ++k) xv[k] = load_elem(sd.x, xo + k, a.x_dtype);
    } else {
#pragma unroll
      for (int k = 0; k < EPT; ++k) xv[k] = 0.f;
    }
    // the B operands of this wave (rows of Pi) are issued after x: loads return in
    // order, so the norms wait only for x and Pi arrives during them
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const float4* row = reinterpret_cast<const float4*>(sd.pi + int64_t(w * KS + 16 * j + (lane & 15)) * D +
                                                          KS * (lane >> 4));
#pragma unroll
      for (int q = 0; q < KS / 4; ++q) pb[j][q] = row[q];
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < EPT; ++k) ss = fma(double(xv[k]), double(xv[k]), ss);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
    const float n = fmaxf(float(sqrt(ss)), 1e-10f);
#pragma unroll
    for (int k = 0; k < EPT; ++k) xs[vl][EPT * part + k] = float(double(xv[k]) / double(n));
    if (part == 0) nrms[vl] = n;
  }
  int dst_pid = -1;
  if (dst_thread && a.scatter) {
    const int b = int((v0 + tid) / (int64_t(a.n) * a.H)), col = dst_pos >> a.log2S;
    if (dst_pos >= 0 && col < a.max_pages) dst_pid = a.table[b * a.tsb + col];
  }
  __syncthreads();  // xs, bnd, nrms

  // A operands: row lane%16 of xs, input dims KS (lane/16) .. + KS - 1
  float4 xa[KS / 4];
  {
    const float4* xr = reinterpret_cast<const float4*>(&xs[lane & 15][KS * (lane >> 4)]);
#pragma unroll
    for (int q = 0; q < KS / 4; ++q) xa[q] = xr[q];
  }
  // two accumulators per tile (even and odd K-step pairs), summed at the end: four
  // independent MFMA chains per wave at D = 128
  f64x4 acc[TPW][2];
#pragma unroll
  for (int j = 0; j < TPW; ++j) acc[j][0] = acc[j][1] = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int q = 0; q < KS / 4; ++q) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const double xe = double(e == 0 ? xa[q].x : e == 1 ? xa[q].y : e == 2 ? xa[q].z : xa[q].w);
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        const float pe = e == 0 ? pb[j][q].x : e == 1 ? pb[j][q].y : e == 2 ? pb[j][q].z : pb[j][q].w;
        acc[j][e >> 1] = __builtin_amdgcn_mfma_f64_16x16x4f64(xe, double(pe), acc[j][e >> 1], 0, 0, 0);
      }
    }
  }
  {
    float y[TPW * 4];
    uint32_t code[TPW * 4];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) y[4 * j + i] = float(acc[j][0][i] + acc[j][1][i]);
    bucketize_n(bnd, sd.bw, y, code);
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) cs[(lane >> 4) + 4 * i][w * KS + 16 * j + (lane & 15)] = uint8_t(code[4 * j + i]);
  }
  if (tid < kVecPerBlock) {
    // byte offset of the vector's packed row and element offset of its norm; -1: the
    // vector is past the end, or (scatter) its position lies outside the page table
    // or its page outside the pool (skipped without writing)
    const int64_t v = v0 + tid;
    int64_t ro = -1, no = 0;
    if (dst_thread) {
      const int h = int((v / a.n) % a.H);
      if (!a.scatter) {
        ro = v * D;
        no = v;
      } else if (dst_pid >= 0 && dst_pid < a.num_pages) {
        const int64_t slot = dst_pos & ((1 << a.log2S) - 1);
        ro = dst_pid * sd.psp + h * sd.psh + slot * (D * sd.bw / 8);
        no = dst_pid * sd.nsp + h * sd.nsh + slot;
      }
    }
    rowoff[tid] = ro;
    nrmoff[tid] = no;
  }
  __syncthreads();  // codes of all sixteen vectors, their destinations

  // stores: vector tid / TPV, codes 8 (tid % TPV) .. + 7
  if (tid < kVecPerBlock * TPV) {
    const int vl = tid / TPV, part = tid % TPV;
    const int64_t ro = rowoff[vl];
    if (ro >= 0) {
      const uint8_t* c = &cs[vl][8 * part];
      if (a.scatter) {
        uint64_t pk = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) pk |= uint64_t(c[k]) << (sd.bw * k);
        store_packed8(sd.pages + ro + int64_t(part) * sd.bw, pk, sd.bw);
        if (part == 0) sd.norms[nrmoff[vl]] = f32_to_f16(nrms[vl]);
      } else {
        uint64_t cw = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) cw |= uint64_t(c[k]) << (8 * k);
        *reinterpret_cast<uint2*>(sd.codes_out + ro + 8 * part) = make_uint2(uint32_t(cw), uint32_t(cw >> 32));
        if (part == 0) sd.norms_out[nrmoff[vl]] = nrms[vl];
      }
    }
  }
}

// The same computation for the head dims without the matrix-core kernel (16, 32,
// 256), on the vector ALU: a work-group quantizes sixteen vectors; norms as above
// (float64 sums of squares, x / n rounded once to fp32 into LDS), then thread j
// forms output dims j, j + 256, ... of every vector as float64 dot products with the
// rows of Pi (each product exact, the sum in float64, rounded once to fp32),
// bucketizes them into the LDS codes, and the store phase packs and scatters as
// quantize_kernel does.
template <int D>
__global__ __launch_bounds__(kQBlock) void quantize_any_kernel(QuantArgs a) {
  constexpr int TPV = D / 8;  // store threads per vector (eight codes each)
  __shared__ float bnd[255];
  __shared__ float xs[kVecPerBlock][D];
  __shared__ uint8_t cs[kVecPerBlock][D];
  __shared__ float nrms[kVecPerBlock];
  __shared__ double ssq[kVecPerBlock][16];
  __shared__ int64_t rowoff[kVecPerBlock];
  __shared__ int64_t nrmoff[kVecPerBlock];

  const QuantSide& sd = a.side[blockIdx.y];
  const int tid = threadIdx.x;
  const int nb = (1 << sd.bw) - 1;
  const int64_t v0 = int64_t(blockIdx.x) * kVecPerBlock;
  if (v0 >= a.total) return;  // block-uniform
  for (int i = tid; i < nb; i += kQBlock) bnd[i] = sd.bnd[i];
  // x into LDS as fp32 (zeros past the end)
  for (int e = tid; e < kVecPerBlock * D; e += kQBlock) {
    const int vl = e / D, dd = e % D;
    const int64_t v = v0 + vl;
    float x = 0.f;
    if (v < a.total) {
      const int i = int(v % a.n);
      const int h = int((v / a.n) % a.H);
      const int b = int(v / (int64_t(a.n) * a.H));
      x = load_elem(sd.x, b * sd.sb + h * sd.sh + i * sd.sn + dd, a.x_dtype);
    }
    xs[vl][dd] = x;
  }
  __syncthreads();
  // squared norms: sixteen threads per vector, D/16 elements each, float64
  {
    const int vl = tid >> 4, part = tid & 15;
    double ss = 0.0;
    for (int k = part; k < D; k += 16) ss = fma(double(xs[vl][k]), double(xs[vl][k]), ss);
    ssq[vl][part] = ss;
  }
  __syncthreads();
  if (tid < kVecPerBlock) {
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 16; ++k) ss += ssq[tid][k];
    nrms[tid] = fmaxf(float(sqrt(ss)), 1e-10f);
  }
  __syncthreads();
  for (int e = tid; e < kVecPerBlock * D; e += kQBlock) {
    const int vl = e / D, dd = e % D;
    xs[vl][dd] = float(double(xs[vl][dd]) / double(nrms[vl]));
  }
  __syncthreads();
  // rotation and codes: thread j, output dims j, j + kQBlock, ...
  for (int j = tid; j < D; j += kQBlock) {
    const float* prow = sd.pi + int64_t(j) * D;
    double y[kVecPerBlock];
#pragma unroll
    for (int v = 0; v < kVecPerBlock; ++v) y[v] = 0.0;
    for (int dd = 0; dd < D; ++dd) {
      const double pe = double(prow[dd]);
#pragma unroll
      for (int v = 0; v < kVecPerBlock; ++v) y[v] = fma(double(xs[v][dd]), pe, y[v]);
    }
    float yf[kVecPerBlock];
    uint32_t code[kVecPerBlock];
#pragma unroll
    for (int v = 0; v < kVecPerBlock; ++v) yf[v] = float(y[v]);
    bucketize_n(bnd, sd.bw, yf, code);
#pragma unroll
    for (int v = 0; v < kVecPerBlock; ++v) cs[v][j] = uint8_t(code[v]);
  }
  if (tid < kVecPerBlock) {
    const int64_t v = v0 + tid;
    int64_t ro = -1, no = 0;
    if (v < a.total) {
      const int h = int((v / a.n) % a.H);
      if (!a.scatter) {
        ro = v * D;
        no = v;
      } else {
        const int b = int(v / (int64_t(a.n) * a.H));
        const int pos = a.start_pos[b] + int(v % a.n), col = pos >> a.log2S;
        const int pid = (pos >= 0 && col < a.max_pages) ? a.table[b * a.tsb + col] : -1;
        if (pid >= 0 && pid < a.num_pages) {
          const int64_t slot = pos & ((1 << a.log2S) - 1);
          ro = pid * sd.psp + h * sd.psh + slot * (D * sd.bw / 8);
          no = pid * sd.nsp + h * sd.nsh + slot;
        }
      }
    }
    rowoff[tid] = ro;
    nrmoff[tid] = no;
  }
  __syncthreads();
  for (int e = tid; e < kVecPerBlock * TPV; e += kQBlock) {
    const int vl = e / TPV, part = e % TPV;
    const int64_t ro = rowoff[vl];
    if (ro < 0) continue;
    const uint8_t* c = &cs[vl][8 * part];
    if (a.scatter) {
      uint64_t pk = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) pk |= uint64_t(c[k]) << (sd.bw * k);
      store_packed8(sd.pages + ro + int64_t(part) * sd.bw, pk, sd.bw);
      if (part == 0) sd.norms[nrmoff[vl]] = f32_to_f16(nrms[vl]);
    } else {
      uint64_t cw = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) cw |= uint64_t(c[k]) << (8 * k);
      *reinterpret_cast<uint2*>(sd.codes_out + ro + 8 * part) = make_uint2(uint32_t(cw), uint32_t(cw >> 32));
      if (part == 0) sd.norms_out[nrmoff[vl]] = nrms[vl];
    }
  }
}

// wn_quantize at any other head_dim up to 256 (the legacy cache splits a head into
// regular and outlier channels, cache.py:185-196, so its quantizers see arbitrary
// widths): quantize_any_kernel with a run-time D and flat output only, each code
// stored as its byte, each norm as fp32.
constexpr int kRtMaxD = 256;

__global__ __launch_bounds__(kQBlock) void quantize_rt_kernel(QuantArgs a, int D) {
  __shared__ float bnd[255];
  __shared__ float xs[kVecPerBlock][kRtMaxD];
  __shared__ float nrms[kVecPerBlock];
  __shared__ double ssq[kVecPerBlock][16];
  const QuantSide& sd = a.side[0];
  const int tid = threadIdx.x;
  const int nb = (1 << sd.bw) - 1;
  const int64_t v0 = int64_t(blockIdx.x) * kVecPerBlock;
  if (v0 >= a.total) return;  // block-uniform
  for (int i = tid; i < nb; i += kQBlock) bnd[i] = sd.bnd[i];
  for (int e = tid; e < kVecPerBlock * D; e += kQBlock) {
    const int vl = e / D, dd = e % D;
    const int64_t v = v0 + vl;
    xs[vl][dd] = v < a.total ? load_elem(sd.x, v * sd.sb + dd, a.x_dtype) : 0.f;
  }
  __syncthreads();
  {
    const int vl = tid >> 4, part = tid & 15;
    double ss = 0.0;
    for (int k = part; k < D; k += 16) ss = fma(double(xs[vl][k]), double(xs[vl][k]), ss);
    ssq[vl][part] = ss;
  }
  __syncthreads();
  if (tid < kVecPerBlock) {
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 16; ++k) ss += ssq[tid][k];
    nrms[tid] = fmaxf(float(sqrt(ss)), 1e-10f);
    if (v0 + tid < a.total) sd.norms_out[v0 + tid] = nrms[tid];
  }
  __syncthreads();
  for (int e = tid; e < kVecPerBlock * D; e += kQBlock) {
    const int vl = e / D, dd = e % D;
    xs[vl][dd] = float(double(xs[vl][dd]) / double(nrms[vl]));
  }
  __syncthreads();
  for (int j = tid; j < D; j += kQBlock) {
    const float* prow = sd.pi + int64_t(j) * D;
    double y[kVecPerBlock];
#pragma unroll
    for (int v = 0; v < kVecPerBlock; ++v) y[v] = 0.0;
    for (int dd = 0; dd < D; ++dd) {
      const double pe = double(prow[dd]);
#pragma unroll
      for (int v = 0; v < kVecPerBlock; ++v) y[v] = fma(double(xs[v][dd]), pe, y[v]);
    }
    float yf[kVecPerBlock];
    uint32_t code[kVecPerBlock];
#pragma unroll
    for (int v = 0; v < kVecPerBlock; ++v) yf[v] = float(y[v]);
    bucketize_n(bnd, sd.bw, yf, code);
#pragma unroll
    for (int v = 0; v < kVecPerBlock; ++v)
      if (v0 + v < a.total) sd.codes_out[(v0 + v) * D + j] = uint8_t(code[v]);
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

// out[r, j] = (sum_d c[code[r, d]] Pi[d, j]) * n[r] at a run-time head_dim <= 256.
__global__ __launch_bounds__(kRtMaxD) void dequantize_rt_kernel(const uint8_t* codes, const uint16_t* norms,
                                                                const float* pi, const float* cb, int bw, int D,
                                                                void* out, int out_dtype) {
  __shared__ float y[kRtMaxD];
  const int64_t r = blockIdx.x;
  const int j = threadIdx.x;
  y[j] = cb[codes[r * D + j] & ((1u << bw) - 1u)];
  __syncthreads();
  float o = 0.f;
  for (int d = 0; d < D; ++d) o = fmaf(y[d], pi[d * D + j], o);
  store_elem(out, r * D + j, out_dtype, o * f16_to_f32(norms[r]));
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

static int launch_quantize(QuantArgs& a, int sides, int D, hipStream_t st, const char* what,
                           void* ev_begin = nullptr, void* ev_end = nullptr) {
  if (a.total == 0) return WN_OK;
  dim3 grid(unsigned((a.total + kVecPerBlock - 1) / kVecPerBlock), sides);
  if (ev_begin) hipEventRecord(static_cast<hipEvent_t>(ev_begin), st);
  switch (D) {
    case 16: hipLaunchKernelGGL(quantize_any_kernel<16>, grid, dim3(kQBlock), 0, st, a); break;
    case 32: hipLaunchKernelGGL(quantize_any_kernel<32>, grid, dim3(kQBlock), 0, st, a); break;
    case 64: hipLaunchKernelGGL(quantize_kernel<64>, grid, dim3(kQBlock), 0, st, a); break;
    case 128: hipLaunchKernelGGL(quantize_kernel<128>, grid, dim3(kQBlock), 0, st, a); break;
    case 256: hipLaunchKernelGGL(quantize_any_kernel<256>, grid, dim3(kQBlock), 0, st, a); break;
  }
  if (ev_end) hipEventRecord(static_cast<hipEvent_t>(ev_end), st);
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
    int B, int Hkv, int n, int D, int S, int num_pages, int max_pages,
    void* stream, void* ev_begin, void* ev_end) {
  clear_error();
  WN_REQUIRE(B >= 0 && Hkv > 0 && n >= 0 && num_pages >= 0 && max_pages >= 0, WN_E_INVALID,
             "append: bad sizes B=%d Hkv=%d n=%d", B, Hkv, n);
  WN_REQUIRE(valid_head_dim(D), WN_E_UNSUPPORTED, "append: head_dim %d not compiled (16, 32, 64, 128, 256)", D);
  WN_REQUIRE(is_pow2(S), WN_E_INVALID, "append: page size %d is not a power of two", S);
  WN_REQUIRE(x_dtype >= WN_F32 && x_dtype <= WN_BF16, WN_E_INVALID, "append: dtype code %d", x_dtype);
  WN_REQUIRE(valid_bw(bw_k) && (!v || valid_bw(bw_v)), WN_E_INVALID, "append: bit widths %d/%d", bw_k,
             bw_v);
  if (int64_t(B) * n == 0) return WN_OK;
  WN_REQUIRE(k && pi_k && boundaries_k && page_table && start_pos && k_pages && k_norms, WN_E_INVALID,
             "append: null operand");
  WN_REQUIRE(!v || (pi_v && boundaries_v && v_pages && v_norms), WN_E_INVALID, "append: null V operand");
  WN_REQUIRE(aligned(pi_k, 16) && (!v || aligned(pi_v, 16)), WN_E_INVALID,
             "append: rotations need 16-byte aligned rows (read with 16-byte loads)");
  WN_REQUIRE(aligned(k_pages, 8) && k_stride_p % 8 == 0 && k_stride_h % 8 == 0 &&
                 (!v || (aligned(v_pages, 8) && v_stride_p % 8 == 0 && v_stride_h % 8 == 0)),
             WN_E_INVALID, "append: pages need 8-byte aligned base and strides");
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
  return launch_quantize(a, v ? 2 : 1, D, static_cast<hipStream_t>(stream), "wn_append_kv", ev_begin, ev_end);
}

extern "C" int wn_quantize(const void* x, int x_dtype, int64_t rows, int64_t row_stride, const float* pi,
                           const float* boundaries, int bw, int D, uint8_t* codes, float* norms,
                           void* stream) {
  clear_error();
  WN_REQUIRE(rows >= 0, WN_E_INVALID, "quantize: rows %lld", (long long)rows);
  WN_REQUIRE(D >= 1 && D <= kRtMaxD, WN_E_UNSUPPORTED, "quantize: head_dim %d (1 .. %d)", D, kRtMaxD);
  WN_REQUIRE(valid_bw(bw), WN_E_INVALID, "quantize: bit width %d", bw);
  WN_REQUIRE(x_dtype >= WN_F32 && x_dtype <= WN_BF16, WN_E_INVALID, "quantize: dtype code %d", x_dtype);
  if (rows == 0) return WN_OK;
  WN_REQUIRE(x && pi && boundaries && codes && norms, WN_E_INVALID, "quantize: null operand");
  WN_REQUIRE(aligned(pi, 16), WN_E_INVALID, "quantize: the rotation needs 16-byte aligned rows");
  WN_REQUIRE(aligned(codes, 8), WN_E_INVALID, "quantize: codes need an 8-byte aligned base");
  QuantArgs a{};
  a.side[0] = QuantSide{x, row_stride, 0, 0, pi, boundaries, bw, nullptr, 0, 0, nullptr, 0, 0, codes, norms};
  a.total = rows;
  a.H = 1;
  a.n = 1;
  a.x_dtype = x_dtype;
  a.scatter = 0;
  if (!valid_head_dim(D)) {  // run-time head_dim: codes as bytes, any width
    hipLaunchKernelGGL(quantize_rt_kernel, dim3(unsigned((rows + kVecPerBlock - 1) / kVecPerBlock)), dim3(kQBlock), 0,
                       static_cast<hipStream_t>(stream), a, D);
    return check_launch("wn_quantize");
  }
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
  WN_REQUIRE(D >= 1 && D <= kRtMaxD, WN_E_UNSUPPORTED, "dequantize: head_dim %d (1 .. %d)", D, kRtMaxD);
  WN_REQUIRE(out_dtype >= WN_F32 && out_dtype <= WN_BF16, WN_E_INVALID, "dequantize: dtype %d", out_dtype);
  if (rows == 0) return WN_OK;
  WN_REQUIRE(rows < (int64_t(1) << 31), WN_E_INVALID, "dequantize: too many rows");
  WN_REQUIRE(codes && norms && pi && centroids && out, WN_E_INVALID, "dequantize: null operand");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
  switch (D) {
    case 16: hipLaunchKernelGGL(dequantize_kernel<16>, grid, dim3(16), 0, st, codes, norms, pi, centroids, bw, out, out_dtype); break;
    case 32: hipLaunchKernelGGL(dequantize_kernel<32>, grid, dim3(32), 0, st, codes, norms, pi, centroids, bw, out, out_dtype); break;
    case 64: hipLaunchKernelGGL(dequantize_kernel<64>, grid, dim3(64), 0, st, codes, norms, pi, centroids, bw, out, out_dtype); break;
    case 128: hipLaunchKernelGGL(dequantize_kernel<128>, grid, dim3(128), 0, st, codes, norms, pi, centroids, bw, out, out_dtype); break;
    case 256: hipLaunchKernelGGL(dequantize_kernel<256>, grid, dim3(256), 0, st, codes, norms, pi, centroids, bw, out, out_dtype); break;
    default:
      hipLaunchKernelGGL(dequantize_rt_kernel, grid, dim3(D), 0, st, codes, norms, pi, centroids, bw, D, out, out_dtype);
  }
  return check_launch("wn_dequantize");
}
