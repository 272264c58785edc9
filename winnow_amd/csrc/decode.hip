// Decode attention over paged packed K/V for gfx950 (CDNA4, wave64).
//
// Three launches per step, all on the caller's stream:
//   1. rotate_q_kernel   q_rot = scale * q Pi_K^T, padded to NREP rows per kv head;
//                        one block also writes the per-sequence chunk prefix the
//                        balanced scan partitions by
//   2. page scan         the row-per-lane matrix-core scan (decode_rows.hip) where
//                        it applies (head_dim 128, a width pair it compiles, and
//                        n_rep that 2^s virtual heads per kv head bring to <= 8),
//                        else decode_split_kernel (wn_split.h): one work-group per
//                        (split, kv head, sequence), score phase (lane = token),
//                        online softmax, value phase (16 lanes per token row),
//                        cross-wave max-stable merge into one (acc, m, l) partial
//   3. merge_kernel      per (query head, kv head, sequence): max-stable merge
//                        of its partials, 1/l, a Pi_V, cast to the output type
// Algebra follows turboquant_kv/packed_attention.py:260-334 (the schedule the
// reference kernel packed_attention_triton.py:51-159 implements).
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "wn_split.h"

namespace wn {
namespace {

struct RotArgs {
  const void* q;
  int64_t qsb, qsh;  // element strides of q (B, Hq, D)
  const float* pi_k;
  float* q_rot;
  const int32_t* seq_lens;
  int32_t* chunk_prefix;  // written by block (0, 0, 0) when not null
  int2* unit_meta;        // (B*Hkv) cleared to (0, 0): the scan fills in the groups that have keys
  float scale;
  int B, Hkv, n_rep, q_dtype;
};

// chunk_prefix[b] = sum over b' < b of ceil(L_b' / 64), b = 0..B (one 256-thread block).
__device__ void chunk_prefix_block(const int32_t* seq_lens, int B, int32_t* prefix) {
  __shared__ int part[4];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  int carry = 0;
  for (int b0 = 0; b0 < B; b0 += 256) {
    const int b = b0 + tid;
    const int n = b < B ? (seq_lens[b] + 63) >> 6 : 0;
    int x = n;  // inclusive wave scan
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) part[w] = x;
    __syncthreads();
    int off = carry;
    for (int i = 0; i < w; ++i) off += part[i];
    if (b < B) prefix[b] = off + x - n;  // exclusive
    const int tile = part[0] + part[1] + part[2] + part[3];
    __syncthreads();
    carry += tile;
  }
  if (tid == 0) prefix[B] = carry;
}

// Output-dim blocks of the rotation: quarters up to head_dim 128, 32 dims above.
constexpr int rot_blocks(int D) { return D <= 128 ? 4 : D / 32; }

// q_rot[b, kvh, h, j] = scale * sum_d q[b, kvh*n_rep + h, d] Pi_K[j, d] for output dims
// j in block blockIdx.z of rot_blocks(D) (zero rows for h >= n_rep). The block's rows
// of Pi_K are staged in LDS with a padded stride (thread j reads row j: banks j + d).
template <int D, int NREP>
__global__ __launch_bounds__(256) void rotate_q_kernel(RotArgs a) {
  constexpr int LDP = D + 1, JQ = D / rot_blocks(D);
  __shared__ float pis[JQ * LDP];
  __shared__ float qs[NREP][D];
  const int kvh = blockIdx.x, b = blockIdx.y, z = blockIdx.z, tid = threadIdx.x;
  if (a.chunk_prefix && kvh == 0 && b == 0 && z == 0) chunk_prefix_block(a.seq_lens, a.B, a.chunk_prefix);
  if (z == 0 && tid == 0) a.unit_meta[b * a.Hkv + kvh] = make_int2(0, 0);
  if (!a.pi_k) {  // no rotation (dense pages): q_rot = scale * q
    float* out = a.q_rot + (int64_t(b) * a.Hkv + kvh) * NREP * D + z * JQ;
    for (int i = tid; i < NREP * JQ; i += 256) {
      const int h = i / JQ, j = i % JQ;
      out[h * D + j] =
          h < a.n_rep ? a.scale * load_elem(a.q, b * a.qsb + int64_t(kvh * a.n_rep + h) * a.qsh + z * JQ + j, a.q_dtype)
                      : 0.f;
    }
    return;
  }
  const float4* src = reinterpret_cast<const float4*>(a.pi_k + z * JQ * D);
  for_strided<JQ * D / 4, 256>(tid, [&](int i) {
    const float4 v = src[i];
    const int r = (4 * i) / D, c = (4 * i) % D;
    float* dst = pis + r * LDP + c;
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
  });
  for_strided<NREP * D, 256>(tid, [&](int i) {
    const int h = i / D, d = i % D;
    qs[h][d] = h < a.n_rep ? load_elem(a.q, b * a.qsb + int64_t(kvh * a.n_rep + h) * a.qsh + d, a.q_dtype) : 0.f;
  });
  __syncthreads();
  float* out = a.q_rot + (int64_t(b) * a.Hkv + kvh) * NREP * D + z * JQ;
  for (int i = tid; i < NREP * JQ; i += 256) {
    const int h = i / JQ, j = i % JQ;
    const float* prow = pis + j * LDP;
    float acc = 0.f;
#pragma unroll 8
    for (int d = 0; d < D; ++d) acc = fmaf(qs[h][d], prow[d], acc);
    out[h * D + j] = acc * a.scale;
  }
}

struct MergeArgs {
  const float* part_acc;
  const float* part_ml;
  const float* pi_v;
  const int2* unit_meta;
  void* out;
  int out_dtype, Hq, Hkv, n_rep;
  int log2_units;  // partial maxima are in log2 units (weights 2^(m - M))
};

constexpr int kMergeBatch = 32;  // partial rows whose loads are in flight together

// out[b, kvh*n_rep + h, :] = (sum_s w_s acc_s / sum_s w_s l_s) Pi_V with
// w_s = exp(m_s - max m) (2^(m_s - max m) for log2-unit partials), zero when no
// key was seen (packed_attention_triton.py:137-159 plus :261).
//
// One work-group of max(D, 64) threads per (query head h, kv head, sequence); thread
// d < D owns output dim d. Up to head_dim 128 thread d first issues the loads of
// column d of Pi_V, so that they travel together with the partials' (one round trip
// for both); at 256 the column is read during the product instead. The partials are taken 64 at a time:
// lane k of each wave loads (m, l) of partial k, the wave reduces the maximum,
// and lane k forms the weight of partial k with one exponential; thread d then
// sums its dim of the acc rows against those weights (read from the lanes that
// hold them), 32 rows' loads in flight together. Output dim d is finally formed
// from the Pi_V column and the merged row in LDS.
// The partials of the group are rows r0 + s, s < n, with (r0, n) left by the scan
// in unit_meta (fixed splits: r0 = (b*Hkv + kvh)*num_splits and n the splits
// holding tokens; balanced: rows w + b*Hkv + kvh of the waves w that touched the
// group); a group without keys has n = 0 and an output row of zeros.
template <int D>
constexpr int merge_threads() { return D < 64 ? 64 : D; }

template <int D>
__global__ __launch_bounds__(merge_threads<D>()) void merge_kernel(MergeArgs a) {
  constexpr bool kPreload = D <= 128;  // Pi_V column in registers
  __shared__ float av[D];
  const int h = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63;
  const int d = min(tid, D - 1);  // threads past D (D < 64) only help the wave reductions
  float pc[kPreload ? D : 1];     // column d of Pi_V (none: no output rotation, dense pages)
  if (kPreload && a.pi_v) {
#pragma unroll
    for (int k = 0; k < D; ++k) pc[k] = a.pi_v[k * D + d];
  }
  const int2 meta = a.unit_meta[b * a.Hkv + kvh];
  const int64_t r0 = meta.x;
  const int n = meta.y;
  auto wexp = [&](float x) { return a.log2_units ? __builtin_amdgcn_exp2f(x) : expf(x); };
  const int64_t pstride = a.n_rep;  // partial rows between consecutive partials of a head
  const float* ml = a.part_ml + 2 * (r0 * pstride + h);
  const float* acc = a.part_acc + (r0 * pstride + h) * D + d;
  float M = -INFINITY, num = 0.f, den = 0.f;
  // every load of a batch is issued, clamped to the last partial; the extras weigh 0
  float xv[kMergeBatch];
  auto load_batch = [&](int first) {
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) xv[k] = acc[int64_t(min(first + k, n - 1)) * pstride * D];
  };
  for (int s0 = 0; s0 < n; s0 += 64) {
    const int cnt = min(64, n - s0);
    float mk = -INFINITY, lk = 0.f;
    if (lane < cnt) {
      const float2 x = *reinterpret_cast<const float2*>(ml + 2 * (int64_t(s0 + lane) * pstride));
      mk = x.x;
      lk = x.y;
    }
    // the first batch's acc rows travel with the (m, l) loads: they need only the range
    if (s0 == 0) load_batch(0);
    const float Mn = fmaxf(M, wave_max(mk));
    // a partial that saw no key (m = -inf) and the lanes past the batch weigh 0
    const float wk = mk == -INFINITY ? 0.f : wexp(mk - Mn);
    const float r_old = M == -INFINITY ? 0.f : wexp(M - Mn);
    den = fmaf(den, r_old, wave_sum(wk * lk));
    num *= r_old;
    M = Mn;
    for (int k0 = 0; k0 < cnt; k0 += kMergeBatch) {
      if (s0 + k0 > 0) load_batch(s0 + k0);
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k0 + k));
        num = fmaf(w, xv[k], num);
      }
    }
  }
  if (tid < D) av[d] = (n > 0 && den > 0.f) ? num / fmaxf(den, 1e-30f) : 0.f;
  __syncthreads();
  if (tid >= D) return;
  // out_j = sum_k a_k Pi_V[k, j]; (a / l) Pi_V == (a Pi_V) / l up to rounding
  float o = 0.f;
  if (a.pi_v) {
    if constexpr (kPreload) {
#pragma unroll
      for (int k = 0; k < D; ++k) o = fmaf(av[k], pc[k], o);
    } else {
#pragma unroll 16
      for (int k = 0; k < D; ++k) o = fmaf(av[k], a.pi_v[k * D + d], o);
    }
  } else {
    o = av[d];
  }
  store_elem(a.out, (int64_t(b) * a.Hq + kvh * a.n_rep + h) * D + d, a.out_dtype, o);
}

// merge_kernel<128> for four heads of one (kv head, sequence) per work-group: wave w
// merges head 4 hg + w (lane l owns dims 2l, 2l+1, loaded as pairs), then thread t
// forms output dim j = t % 128 of heads 4 hg + 2 (t / 128) + {0, 1}, reading column j
// of Pi_V inside the product for both. For batches of many (kv head, sequence)
// pairs, where merge_kernel's per-head work-groups each pull all of Pi_V (64 KB)
// through the L2, this reads it a quarter as often (config 4's shape, A/B: 11.8 ->
// 7.8 us); with few pairs it leaves CUs idle and merge_kernel is faster. Every sum
// runs in merge_kernel's order, so the outputs are the same bits.
constexpr int kMergeHeads = 4;

__global__ __launch_bounds__(64 * kMergeHeads) void merge4_kernel(MergeArgs a) {
  constexpr int D = 128;
  __shared__ float av[kMergeHeads][D];
  const int hg = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int h = kMergeHeads * hg + wave;
  const int2 meta = a.unit_meta[b * a.Hkv + kvh];
  const int64_t r0 = meta.x;
  const int n = meta.y;
  auto wexp = [&](float x) { return a.log2_units ? __builtin_amdgcn_exp2f(x) : expf(x); };
  const int64_t pstride = a.n_rep;
  if (h < a.n_rep) {  // wave-uniform
    const float* ml = a.part_ml + 2 * (r0 * pstride + h);
    const float2* acc = reinterpret_cast<const float2*>(a.part_acc + (r0 * pstride + h) * D) + lane;
    float M = -INFINITY, den = 0.f;
    float2 num = make_float2(0.f, 0.f);
    float2 xv[kMergeBatch];
    auto load_batch = [&](int first) {
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) xv[k] = acc[int64_t(min(first + k, n - 1)) * pstride * (D / 2)];
    };
    for (int s0 = 0; s0 < n; s0 += 64) {
      const int cnt = min(64, n - s0);
      float mk = -INFINITY, lk = 0.f;
      if (lane < cnt) {
        const float2 x = *reinterpret_cast<const float2*>(ml + 2 * (int64_t(s0 + lane) * pstride));
        mk = x.x;
        lk = x.y;
      }
      if (s0 == 0) load_batch(0);
      const float Mn = fmaxf(M, wave_max(mk));
      const float wk = mk == -INFINITY ? 0.f : wexp(mk - Mn);
      const float r_old = M == -INFINITY ? 0.f : wexp(M - Mn);
      den = fmaf(den, r_old, wave_sum(wk * lk));
      num.x *= r_old;
      num.y *= r_old;
      M = Mn;
      for (int k0 = 0; k0 < cnt; k0 += kMergeBatch) {
        if (s0 + k0 > 0) load_batch(s0 + k0);
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k) {
          const float wt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k0 + k));
          num.x = fmaf(wt, xv[k].x, num.x);
          num.y = fmaf(wt, xv[k].y, num.y);
        }
      }
    }
    const bool some = n > 0 && den > 0.f;
    av[wave][2 * lane] = some ? num.x / fmaxf(den, 1e-30f) : 0.f;
    av[wave][2 * lane + 1] = some ? num.y / fmaxf(den, 1e-30f) : 0.f;
  }
  __syncthreads();
  const int j = tid & (D - 1), hp = tid >> 7;
  const int ha = kMergeHeads * hg + 2 * hp;  // heads ha, ha + 1 (past n_rep: not stored)
  float o0 = 0.f, o1 = 0.f;
  if (a.pi_v) {
#pragma unroll 16
    for (int k = 0; k < D; ++k) {
      const float pv = a.pi_v[k * D + j];
      o0 = fmaf(av[2 * hp][k], pv, o0);
      o1 = fmaf(av[2 * hp + 1][k], pv, o1);
    }
  } else {
    o0 = av[2 * hp][j];
    o1 = av[2 * hp + 1][j];
  }
  const int64_t orow = int64_t(b) * a.Hq + kvh * a.n_rep;
  if (ha < a.n_rep) store_elem(a.out, (orow + ha) * D + j, a.out_dtype, o0);
  if (ha + 1 < a.n_rep) store_elem(a.out, (orow + ha + 1) * D + j, a.out_dtype, o1);
}

using MergeFn = void (*)(MergeArgs);

// The merge for head_dim D and its work-group size; grid = (n_rep, Hkv, B). At head_dim
// 128 with 512 or more work-groups of merge4_kernel, that kernel.
void launch_merge(int D, dim3 grid, hipStream_t st, const MergeArgs& ma) {
  if (D == 128) {
    const unsigned groups = (grid.x + kMergeHeads - 1) / kMergeHeads;
    if (int64_t(groups) * grid.y * grid.z >= 512) {
      hipLaunchKernelGGL(merge4_kernel, dim3(groups, grid.y, grid.z), dim3(64 * kMergeHeads), 0, st, ma);
      return;
    }
  }
  switch (D) {
    case 16: hipLaunchKernelGGL(merge_kernel<16>, grid, dim3(merge_threads<16>()), 0, st, ma); break;
    case 32: hipLaunchKernelGGL(merge_kernel<32>, grid, dim3(merge_threads<32>()), 0, st, ma); break;
    case 64: hipLaunchKernelGGL(merge_kernel<64>, grid, dim3(merge_threads<64>()), 0, st, ma); break;
    case 128: hipLaunchKernelGGL(merge_kernel<128>, grid, dim3(merge_threads<128>()), 0, st, ma); break;
    case 256: hipLaunchKernelGGL(merge_kernel<256>, grid, dim3(merge_threads<256>()), 0, st, ma); break;
  }
}

using RotFn = void (*)(RotArgs);

template <int D>
SplitFn pick_split(int bwk, int bwv, int nrep) {
  if (bwk == bwv) {
    switch (bwk) {
      case 2: return pick_nrep<D, 2, 2>(nrep);
      case 3: return pick_nrep<D, 3, 3>(nrep);
      case 4: return pick_nrep<D, 4, 4>(nrep);
      case 5: return pick_nrep<D, 5, 5>(nrep);
      case 6: return pick_nrep<D, 6, 6>(nrep);
      case 8: return pick_nrep<D, 8, 8>(nrep);
    }
    return nullptr;
  }
  if constexpr (D == 128) {
    if (bwk == 4 && bwv == 6) return pick_nrep<D, 4, 6>(nrep);
    if (bwk == 6 && bwv == 4) return pick_nrep<D, 6, 4>(nrep);
    if (bwk == 4 && bwv == 8) return pick_nrep<D, 4, 8>(nrep);
  }
  return pick_split_any(D, bwk, bwv, nrep);  // every other pair (decode_split_any*.hip)
}

template <int D>
RotFn pick_rot(int nrep) {
  switch (nrep) {
    case 1: return rotate_q_kernel<D, 1>;
    case 2: return rotate_q_kernel<D, 2>;
    case 4: return rotate_q_kernel<D, 4>;
    case 8: return rotate_q_kernel<D, 8>;
    case 16: return rotate_q_kernel<D, 16>;
  }
  return nullptr;
}

RotFn pick_rot_d(int D, int nrep) {
  switch (D) {
    case 16: return pick_rot<16>(nrep);
    case 32: return pick_rot<32>(nrep);
    case 64: return pick_rot<64>(nrep);
    case 128: return pick_rot<128>(nrep);
    case 256: return pick_rot<256>(nrep);
  }
  return nullptr;
}

int rot_blocks_d(int D) { return D <= 128 ? 4 : D / 32; }

// Page-scan kernel preference, read once from WN_DECODE_SCAN: "rows" (default)
// uses the row-per-lane matrix-core scan where it applies, "valu" always the
// vector-ALU scan. Both compute the same result; the knob exists to compare
// them on one machine.
bool rows_allowed() {
  static const bool allowed = [] {
    const char* e = getenv("WN_DECODE_SCAN");
    return !(e && !strcmp(e, "valu"));
  }();
  return allowed;
}

int pad_nrep(int n_rep) {
  int p = 1;
  while (p < n_rep) p <<= 1;
  return p;
}

// Virtual heads. A kv head with more query heads than a scan holds runs as kvdiv
// virtual kv heads of n_rep / kvdiv query heads each: q_rot rows, partial rows and
// output heads are laid out alike in both views (virtual head v of kv head k is
// v = k kvdiv + j and holds query heads v (n_rep / kvdiv) + h), and only the scan's
// page and norm addresses map a virtual head back to its kv head.
// Row scan: kvdiv = 2^s, the smallest with n_rep / 2^s <= 8 whole, or -1.
int row_shift(int n_rep) {
  for (int s = 0; (1 << s) <= n_rep; ++s)
    if (n_rep % (1 << s) == 0 && (n_rep >> s) <= 8) return s;
  return -1;
}
// Vector-ALU scan: the smallest divisor kvdiv of n_rep with n_rep / kvdiv <= 16.
int valu_groups(int n_rep) {
  for (int g = 1; g < n_rep; ++g)
    if (n_rep % g == 0 && n_rep / g <= 16) return g;
  return n_rep > 0 ? n_rep : 1;
}

// The scan wn_decode_attention runs for this shape: the row-per-lane matrix-core
// scan where it applies (head_dim 128, page size >= 16, a compiled width pair, any
// n_rep that 2^s virtual heads bring to <= 8), else the vector-ALU scan (any
// supported width pair, n_rep split into groups of <= 16).
// tf32: the TF32-class row scan where it is compiled (4 and 6-bit K and V, alike or
// mixed, on the row scan: n_rep up to 8, or up to 16 in virtual kv heads of eight),
// else the same choice as without it.
SplitKernel choose_scan(int Hq, int Hkv, int D, int S, int bw_k, int bw_v, bool tf32 = false) {
  SplitKernel sk;
  const int n_rep = Hq / Hkv;
  const int shift = row_shift(n_rep);
  if (D == 128 && shift >= 0 && S >= 16 && rows_allowed()) {
    if (tf32) sk = pick_split_rows_tf(bw_k, bw_v, n_rep >> shift);
    if (!sk.fn) sk = pick_split_rows(bw_k, bw_v, n_rep >> shift);
    if (sk.fn) {
      sk.kvshift = shift;
      sk.kvdiv = 1 << shift;
    }
  }
  if (!sk.fn) {
    const int g = valu_groups(n_rep);
    const int nrp = pad_nrep(n_rep / g);
    sk = SplitKernel{};
    sk.fn = D == 128 ? pick_split<128>(bw_k, bw_v, nrp)
            : D == 64 ? pick_split<64>(bw_k, bw_v, nrp)
                      : pick_split_any(D, bw_k, bw_v, nrp);  // 16, 32, 256: every pair there
    sk.block = kBlock;
    sk.nrep = nrp;
    sk.kvdiv = g;
  }
  return sk;
}

// Resident waves of the row scan `sk` on the current device: work-groups per CU
// x CUs x waves per work-group.
int resident_waves(const SplitKernel& sk) {
  static std::mutex mu;
  static std::map<std::pair<int, SplitFn>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({dev, sk.fn});
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(sk.fn), sk.block,
                                                   0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int w = per_cu * cus * sk.wpb;
  cache[{dev, sk.fn}] = w;
  return w;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

struct WsLayout {
  int64_t qrot, prefix, meta, acc, ml, total;
};

// Virtual heads per kv head either scan may use, and the q_rot rows per kv head it
// needs (NREP rows per virtual head, at least 4 on the matrix-core scan).
int max_virtual_heads(int n_rep) {
  const int s = row_shift(n_rep);
  return max(s >= 0 ? 1 << s : 1, valu_groups(n_rep));
}
int qrot_rows(int n_rep) {
  int rows = max(pad_nrep(n_rep), 4);
  const int s = row_shift(n_rep);
  if (s >= 0) rows = max(rows, (1 << s) * max(pad_nrep(n_rep >> s), 4));
  const int g = valu_groups(n_rep);
  return max(rows, g * pad_nrep(n_rep / g));
}

// Scratch: q_rot (B, Hkv, qrot_rows, D) fp32, chunk prefix (B+1) int32, and
// the partials, (rows * n_rep) x D for acc and x 2 for (m, l).
WsLayout ws_layout(int B, int Hq, int Hkv, int D, int pages_per_split, int num_splits) {
  WsLayout l;
  const int n_rep = Hq / Hkv;
  const int nrp = qrot_rows(n_rep);
  const int64_t rows = pages_per_split > 0 ? int64_t(B) * Hkv * num_splits : int64_t(num_splits) + int64_t(B) * Hkv;
  l.qrot = 0;
  l.prefix = align256(int64_t(B) * Hkv * nrp * D * 4);
  l.meta = l.prefix + align256(int64_t(B + 1) * 4);
  // unit_meta: one per (virtual) kv head of either scan (choose_scan)
  l.acc = l.meta + align256(int64_t(B) * Hkv * max_virtual_heads(n_rep) * 8);
  l.ml = l.acc + align256(rows * n_rep * D * 4);
  l.total = l.ml + align256(rows * n_rep * 2 * 4);
  return l;
}

}  // namespace
}  // namespace wn

// Work-groups the fixed-split plan aims for: 256 CUs x ~16 resident waves / 4
// waves per group, so every CU keeps several groups in flight while the
// per-split partials stay a few percent of the page bytes.
static constexpr int64_t kTargetGroups = 4096;

// Fixed splits for the vector-ALU scans: about kTargetGroups work-groups over the
// (sequence, virtual kv head) units, each split >= 16 pages.
static void fixed_plan(int B, int units_per_seq, int mp, int* pages_per_split, int* num_splits) {
  const int64_t units = int64_t(B > 0 ? B : 1) * units_per_seq;
  int64_t want = (kTargetGroups + units - 1) / units;
  if (want < 1) want = 1;
  if (want > mp) want = mp;
  int64_t pps = (mp + want - 1) / want;
  if (pps < 16) pps = 16;  // >= 256 tokens at S=16: all four waves of a group busy
  if (pps > mp) pps = mp;
  *pages_per_split = int(pps);
  *num_splits = int((mp + pps - 1) / pps);
}

namespace {
int decode_plan(int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages, int requested_splits,
                int* pages_per_split, int* num_splits, bool tf32) {
  using namespace wn;
  clear_error();
  WN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && max_pages >= 0, WN_E_INVALID,
             "wn_decode_plan: bad sizes B=%d Hq=%d Hkv=%d max_pages=%d", B, Hq, Hkv, max_pages);
  WN_REQUIRE(pages_per_split && num_splits, WN_E_INVALID, "wn_decode_plan: null output");
  const int mp = max_pages > 0 ? max_pages : 1;
  if (requested_splits > 0) {
    // packed_attention_triton.py:211-216: splits clamp to [1, max_pages],
    // each covering cdiv(max_pages, splits) page slots.
    const int ns = requested_splits < mp ? requested_splits : mp;
    *num_splits = ns;
    *pages_per_split = (mp + ns - 1) / ns;
    return WN_OK;
  }
  const SplitKernel sk = choose_scan(Hq, Hkv, D, S, bw_k, bw_v, tf32);
  if (sk.fn && sk.rows) {  // row scan: balanced persistent waves
    const int w = resident_waves(sk);
    WN_REQUIRE(w > 0, WN_E_LAUNCH, "wn_decode_plan: cannot query the device occupancy");
    *pages_per_split = 0;
    *num_splits = w;
    return WN_OK;
  }
  fixed_plan(B, Hkv * sk.kvdiv, mp, pages_per_split, num_splits);
  return WN_OK;
}
}  // namespace

extern "C" int wn_decode_plan(int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
                              int requested_splits, int* pages_per_split, int* num_splits) {
  return decode_plan(B, Hq, Hkv, D, S, bw_k, bw_v, max_pages, requested_splits, pages_per_split, num_splits,
                     false);
}

extern "C" int wn_decode_plan_tf32(int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
                                   int requested_splits, int* pages_per_split, int* num_splits) {
  return decode_plan(B, Hq, Hkv, D, S, bw_k, bw_v, max_pages, requested_splits, pages_per_split, num_splits,
                     true);
}

extern "C" int64_t wn_decode_workspace_bytes(int B, int Hq, int Hkv, int D, int pages_per_split, int num_splits) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || num_splits <= 0 || pages_per_split < 0) return -1;
  return wn::ws_layout(B, Hq, Hkv, D, pages_per_split, num_splits).total;
}

namespace {
// wn_decode_attention and wn_decode_attention_tf32: tf32 picks the TF32-class scan.
int decode_attention(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const float* pi_k, const float* pi_v, const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b, const int32_t* seq_lens,
    void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
    float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end, bool tf32) {
  using namespace wn;
  clear_error();
  WN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, WN_E_INVALID,
             "decode: need B>=0, Hq%%Hkv==0 (B=%d Hq=%d Hkv=%d)", B, Hq, Hkv);
  const int n_rep = Hq / Hkv;
  WN_REQUIRE(valid_head_dim(D), WN_E_UNSUPPORTED, "decode: head_dim %d not compiled (16, 32, 64, 128, 256)", D);
  WN_REQUIRE(valid_bw(bw_k) && valid_bw(bw_v), WN_E_INVALID, "decode: bit widths %d/%d", bw_k, bw_v);
  WN_REQUIRE(is_pow2(S), WN_E_INVALID, "decode: page size %d is not a power of two", S);
  WN_REQUIRE(q_dtype >= WN_F32 && q_dtype <= WN_BF16 && out_dtype >= WN_F32 && out_dtype <= WN_BF16,
             WN_E_INVALID, "decode: dtype codes %d/%d", q_dtype, out_dtype);
  const bool balanced = pages_per_split == 0;
  WN_REQUIRE(num_splits > 0 && pages_per_split >= 0 &&
                 (balanced || int64_t(pages_per_split) * num_splits >= int64_t(max_pages)),
             WN_E_INVALID, "decode: plan %d x %d does not cover %d pages", num_splits, pages_per_split,
             max_pages);
  if (B == 0) return WN_OK;
  WN_REQUIRE(q && pi_k && pi_v && codebook_k && codebook_v && k_pages && v_pages && k_norms &&
                 v_norms && page_table && seq_lens && out,
             WN_E_INVALID, "decode: null operand");
  const int nbk = D * bw_k / 8, nbv = D * bw_v / 8;
  const int row_align = (nbk % 16 == 0) ? 16 : 8;
  WN_REQUIRE(aligned(k_pages, row_align) && k_stride_p % row_align == 0 && k_stride_h % row_align == 0,
             WN_E_INVALID, "decode: K pages need %d-byte aligned base and strides", row_align);
  WN_REQUIRE(aligned(v_pages, 8) && v_stride_p % 8 == 0 && v_stride_h % 8 == 0, WN_E_INVALID,
             "decode: V pages need 8-byte aligned base and strides");
  WN_REQUIRE(k_stride_h >= int64_t(S) * nbk && v_stride_h >= int64_t(S) * nbv, WN_E_INVALID,
             "decode: head stride smaller than one (S, NB) page block");
  WN_REQUIRE(aligned(pi_k, 16) && aligned(pi_v, 4), WN_E_INVALID, "decode: rotation alignment");
  // the row scans form a norm's offset as a 32 x 32 -> 64-bit product of the page id
  // and the page stride plus a 32-bit in-page offset
  const int64_t lim = int64_t(1) << 31;
  WN_REQUIRE(kn_stride_p >= 0 && kn_stride_p < lim && vn_stride_p >= 0 && vn_stride_p < lim && kn_stride_h >= 0 &&
                 vn_stride_h >= 0 && int64_t(Hkv) * kn_stride_h + S <= lim && int64_t(Hkv) * vn_stride_h + S <= lim,
             WN_E_INVALID, "decode: norm strides of 2^31 elements or more");
  // the row scans form a page block's address as page id x page stride (32 x 32 -> 64 bits)
  WN_REQUIRE(k_stride_p >= 0 && k_stride_p < 2 * lim && v_stride_p >= 0 && v_stride_p < 2 * lim, WN_E_INVALID,
             "decode: page strides of 2^32 bytes or more");

  const SplitKernel sk = choose_scan(Hq, Hkv, D, S, bw_k, bw_v, tf32);
  RotFn rot = pick_rot_d(D, max(sk.nrep, 1));
  WN_REQUIRE(sk.fn && rot, WN_E_UNSUPPORTED, "decode: (D=%d, bw_k=%d, bw_v=%d) not compiled", D, bw_k,
             bw_v);
  WN_REQUIRE(!balanced || sk.rows, WN_E_INVALID,
             "decode: a balanced plan (pages_per_split 0) needs the row scan; ask wn_decode_plan");

  const WsLayout lay = ws_layout(B, Hq, Hkv, D, pages_per_split, num_splits);
  WN_REQUIRE(workspace && workspace_bytes >= lay.total && aligned(workspace, 256), WN_E_WORKSPACE,
             "decode: workspace needs %lld bytes, 256-aligned (got %lld)", (long long)lay.total,
             (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* prefix = balanced ? reinterpret_cast<int32_t*>(ws + lay.prefix) : nullptr;

  // the matrix-core scan keeps scores in log2 units: fold log2(e) into q_rot
  const float q_scale = sk.log2_units ? float(double(scale) * 1.4426950408889634) : scale;
  int2* meta = reinterpret_cast<int2*>(ws + lay.meta);
  // from here on the kv heads are the scan's (virtual) ones
  const int Hkv_s = Hkv * sk.kvdiv, n_rep_s = n_rep / sk.kvdiv;
  RotArgs ra{q, q_stride_b, q_stride_h, pi_k, reinterpret_cast<float*>(ws + lay.qrot), seq_lens, prefix, meta,
             q_scale, B, Hkv_s, n_rep_s, q_dtype};
  hipLaunchKernelGGL(rot, dim3(Hkv_s, B, rot_blocks_d(D)), dim3(256), 0, st, ra);

  DecodeArgs da;
  da.q_rot = ra.q_rot;
  da.k_pages = k_pages;
  da.v_pages = v_pages;
  da.k_norms = k_norms;
  da.v_norms = v_norms;
  da.cb_k = codebook_k;
  da.cb_v = codebook_v;
  da.table = page_table;
  da.seq_lens = seq_lens;
  da.part_acc = reinterpret_cast<float*>(ws + lay.acc);
  da.part_ml = reinterpret_cast<float*>(ws + lay.ml);
  da.ksp = k_stride_p;
  da.ksh = k_stride_h;
  da.vsp = v_stride_p;
  da.vsh = v_stride_h;
  da.knp = kn_stride_p;
  da.knh = kn_stride_h;
  da.vnp = vn_stride_p;
  da.vnh = vn_stride_h;
  da.tsb = table_stride_b;
  da.chunk_prefix = prefix;
  da.unit_meta = meta;
  da.B = B;
  da.Hkv = Hkv_s;
  da.n_rep = n_rep_s;
  da.log2S = ilog2(S);
  da.pages_per_split = pages_per_split;
  da.num_splits = num_splits;
  da.balanced = balanced ? 1 : 0;
  da.qrows = max(sk.nrep, 1);
  da.kvshift = sk.kvshift;
  da.kvdiv = sk.kvdiv;
  // the row scan numbers its waves across work-groups of sk.wpb waves
  const int64_t waves = balanced ? int64_t(num_splits) : int64_t(num_splits) * Hkv_s * B;
  const dim3 grid = sk.rows ? dim3(unsigned((waves + sk.wpb - 1) / sk.wpb)) : dim3(num_splits, Hkv_s, B);
  if (ev_begin) hipEventRecord(static_cast<hipEvent_t>(ev_begin), st);
  hipLaunchKernelGGL(sk.fn, grid, dim3(sk.block), 0, st, da);
  if (ev_end) hipEventRecord(static_cast<hipEvent_t>(ev_end), st);

  MergeArgs ma{da.part_acc, da.part_ml, pi_v, meta, out, out_dtype, Hq, Hkv_s, n_rep_s, sk.log2_units ? 1 : 0};
  launch_merge(D, dim3(n_rep_s, Hkv_s, B), st, ma);
  return check_launch(tf32 ? "wn_decode_attention_tf32" : "wn_decode_attention");
}
}  // namespace

#define WN_DECODE_PARAMS                                                                                       \
  const void *q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, const float *pi_k, const float *pi_v,    \
      const float *codebook_k, const float *codebook_v, const uint8_t *k_pages, int64_t k_stride_p,            \
      int64_t k_stride_h, const uint8_t *v_pages, int64_t v_stride_p, int64_t v_stride_h,                      \
      const uint16_t *k_norms, int64_t kn_stride_p, int64_t kn_stride_h, const uint16_t *v_norms,              \
      int64_t vn_stride_p, int64_t vn_stride_h, const int32_t *page_table, int64_t table_stride_b,             \
      const int32_t *seq_lens, void *out, int out_dtype, void *workspace, int64_t workspace_bytes, int B,      \
      int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages, float scale, int pages_per_split,      \
      int num_splits, void *stream, void *ev_begin, void *ev_end
#define WN_DECODE_ARGS                                                                                          \
  q, q_dtype, q_stride_b, q_stride_h, pi_k, pi_v, codebook_k, codebook_v, k_pages, k_stride_p, k_stride_h,    \
      v_pages, v_stride_p, v_stride_h, k_norms, kn_stride_p, kn_stride_h, v_norms, vn_stride_p, vn_stride_h,   \
      page_table, table_stride_b, seq_lens, out, out_dtype, workspace, workspace_bytes, B, Hq, Hkv, D, S,     \
      bw_k, bw_v, max_pages, scale, pages_per_split, num_splits, stream, ev_begin, ev_end

extern "C" int wn_decode_attention(WN_DECODE_PARAMS) { return decode_attention(WN_DECODE_ARGS, false); }

extern "C" int wn_decode_attention_tf32(WN_DECODE_PARAMS) { return decode_attention(WN_DECODE_ARGS, true); }

#undef WN_DECODE_PARAMS
#undef WN_DECODE_ARGS

// ------------------------------------------------- allocation-free decode entry

// Scratch of wn_decode_attention_noalloc: a file-scope device array, so a caller
// that cannot allocate device memory (code under graph capture, a serving loop
// that forbids it) still gets the rotated query, chunk prefix, partial ranges and
// partials somewhere. Each GPU the library runs on holds its own copy until the
// process ends. On the host the array's name is only a stand-in for its symbol:
// its device address comes from hipGetSymbolAddress, once per device, and only
// that address is ever handed to a kernel.
static constexpr int64_t kNoAllocScratchBytes = WN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on its first use there).
int current_scratch(void** addr) {
  using namespace wn;
  int dev = -1;
  WN_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices, WN_E_LAUNCH,
             "decode (no-alloc): no current device (or device %d beyond %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    WN_REQUIRE(e == hipSuccess && p, WN_E_LAUNCH, "decode (no-alloc): hipGetSymbolAddress on device %d: %s", dev,
               hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return WN_OK;
}
}  // namespace

extern "C" int wn_decode_attention_noalloc(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const float* pi_k, const float* pi_v, const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b, const int32_t* seq_lens,
    void* out, int out_dtype,
    int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
    float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end) {
  using namespace wn;
  clear_error();
  const int64_t need = wn_decode_workspace_bytes(B, Hq, Hkv, D, pages_per_split, num_splits);
  WN_REQUIRE(need <= kNoAllocScratchBytes, WN_E_WORKSPACE,
             "decode (no-alloc): B=%d Hq=%d Hkv=%d D=%d with %d splits x %d pages needs %lld bytes of scratch, "
             "more than the %lld-byte static scratch; call wn_decode_attention with a workspace",
             B, Hq, Hkv, D, num_splits, pages_per_split, (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc != WN_OK) return rc;
  // every byte of the scratch a call reads is written earlier in the same call
  // (rotate: q_rot, prefix, unit_meta reset; scan: partial rows and ranges), so
  // nothing is cleared between calls
  return wn_decode_attention(q, q_dtype, q_stride_b, q_stride_h, pi_k, pi_v, codebook_k, codebook_v, k_pages,
                             k_stride_p, k_stride_h, v_pages, v_stride_p, v_stride_h, k_norms, kn_stride_p,
                             kn_stride_h, v_norms, vn_stride_p, vn_stride_h, page_table, table_stride_b, seq_lens, out,
                             out_dtype, ws, kNoAllocScratchBytes, B, Hq, Hkv, D, S, bw_k, bw_v, max_pages, scale,
                             pages_per_split, num_splits, stream, ev_begin, ev_end);
}

// ---------------------------------------------------------------- dense pages

extern "C" int wn_dense_decode_plan(int B, int Hq, int Hkv, int D, int S, int page_dtype, int max_pages,
                                    int requested_splits, int* pages_per_split, int* num_splits) {
  using namespace wn;
  clear_error();
  WN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && max_pages >= 0, WN_E_INVALID,
             "wn_dense_decode_plan: bad sizes B=%d Hq=%d Hkv=%d max_pages=%d", B, Hq, Hkv, max_pages);
  WN_REQUIRE(pages_per_split && num_splits, WN_E_INVALID, "wn_dense_decode_plan: null output");
  (void)S;
  const int mp = max_pages > 0 ? max_pages : 1;
  if (requested_splits > 0) {  // packed_attention_triton.py:211-216, as for packed pages
    const int ns = requested_splits < mp ? requested_splits : mp;
    *num_splits = ns;
    *pages_per_split = (mp + ns - 1) / ns;
    return WN_OK;
  }
  WN_REQUIRE(valid_head_dim(D), WN_E_UNSUPPORTED, "wn_dense_decode_plan: head_dim %d (16, 32, 64, 128, 256)", D);
  if (page_dtype == WN_F32 || (D != 64 && D != 128)) {  // the vector-ALU scan runs on fixed splits
    WN_REQUIRE(page_dtype >= WN_F32 && page_dtype <= WN_BF16, WN_E_UNSUPPORTED,
               "wn_dense_decode_plan: page dtype %d (fp32, bf16 or fp16)", page_dtype);
    fixed_plan(B, Hkv * valu_groups(Hq / Hkv), mp, pages_per_split, num_splits);
    return WN_OK;
  }
  const SplitKernel sk = pick_dense_scan(page_dtype, D);
  WN_REQUIRE(sk.fn, WN_E_UNSUPPORTED, "wn_dense_decode_plan: page dtype %d (fp32, bf16 or fp16), head_dim %d (64, 128)",
             page_dtype, D);
  const int w = resident_waves(sk);
  WN_REQUIRE(w > 0, WN_E_LAUNCH, "wn_dense_decode_plan: cannot query the device occupancy");
  *pages_per_split = 0;
  *num_splits = w;
  return WN_OK;
}

extern "C" int wn_dense_decode_attention(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const void* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const void* v_pages, int64_t v_stride_p, int64_t v_stride_h, int page_dtype,
    const int32_t* page_table, int64_t table_stride_b, const int32_t* seq_lens,
    void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int D, int S, int max_pages, float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end) {
  using namespace wn;
  clear_error();
  WN_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, WN_E_INVALID,
             "dense decode: need B>=0, Hq%%Hkv==0 (B=%d Hq=%d Hkv=%d)", B, Hq, Hkv);
  const int n_rep = Hq / Hkv;
  WN_REQUIRE(valid_head_dim(D), WN_E_UNSUPPORTED, "dense decode: head_dim %d not compiled (16, 32, 64, 128, 256)",
             D);
  WN_REQUIRE(is_pow2(S) && S >= 16, WN_E_UNSUPPORTED, "dense decode: page size %d (a power of two >= 16)", S);
  WN_REQUIRE(q_dtype >= WN_F32 && q_dtype <= WN_BF16 && out_dtype >= WN_F32 && out_dtype <= WN_BF16,
             WN_E_INVALID, "dense decode: dtype codes %d/%d", q_dtype, out_dtype);
  // more than 16 query heads per kv head: virtual kv heads of n_rep / g each
  const int g = valu_groups(n_rep), Hkv_s = Hkv * g, n_rep_s = n_rep / g;
  // the MFMA scan for bf16/fp16 pages at head_dim 64 and 128, the vector-ALU scan otherwise
  const bool valu = page_dtype == WN_F32 || (D != 64 && D != 128);
  const SplitKernel sk =
      valu ? pick_dense_valu_scan(page_dtype, D, pad_nrep(n_rep_s)) : pick_dense_scan(page_dtype, D);
  WN_REQUIRE(sk.fn, WN_E_UNSUPPORTED, "dense decode: page dtype %d (fp32, bf16 or fp16)", page_dtype);
  const bool balanced = pages_per_split == 0;
  WN_REQUIRE(!balanced || sk.rows, WN_E_INVALID,
             "dense decode: fp32 pages and head_dim %d need fixed splits (pages_per_split > 0); ask "
             "wn_dense_decode_plan", D);
  WN_REQUIRE(num_splits > 0 && pages_per_split >= 0 &&
                 (balanced || int64_t(pages_per_split) * num_splits >= int64_t(max_pages)),
             WN_E_INVALID, "dense decode: plan %d x %d does not cover %d pages", num_splits, pages_per_split,
             max_pages);
  if (B == 0) return WN_OK;
  WN_REQUIRE(q && k_pages && v_pages && page_table && seq_lens && out, WN_E_INVALID, "dense decode: null operand");
  WN_REQUIRE(aligned(k_pages, 16) && aligned(v_pages, 16) && k_stride_p % 16 == 0 && k_stride_h % 16 == 0 &&
                 v_stride_p % 16 == 0 && v_stride_h % 16 == 0,
             WN_E_INVALID, "dense decode: pages need 16-byte aligned bases and strides");
  const int64_t esz = page_dtype == WN_F32 ? 4 : 2;
  WN_REQUIRE(k_stride_h >= int64_t(S) * D * esz && v_stride_h >= int64_t(S) * D * esz, WN_E_INVALID,
             "dense decode: head stride smaller than one (S, D) page block");
  RotFn rot = pick_rot_d(D, pad_nrep(n_rep_s));
  WN_REQUIRE(rot, WN_E_UNSUPPORTED, "dense decode: n_rep=%d", n_rep);

  const WsLayout lay = ws_layout(B, Hq, Hkv, D, pages_per_split, num_splits);
  WN_REQUIRE(workspace && workspace_bytes >= lay.total && aligned(workspace, 256), WN_E_WORKSPACE,
             "dense decode: workspace needs %lld bytes, 256-aligned (got %lld)", (long long)lay.total,
             (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t* prefix = balanced ? reinterpret_cast<int32_t*>(ws + lay.prefix) : nullptr;
  int2* meta = reinterpret_cast<int2*>(ws + lay.meta);
  // scores in log2 units: q_rot = scale * log2(e) * q, no rotation
  RotArgs ra{q, q_stride_b, q_stride_h, nullptr, reinterpret_cast<float*>(ws + lay.qrot), seq_lens, prefix, meta,
             float(double(scale) * 1.4426950408889634), B, Hkv_s, n_rep_s, q_dtype};
  hipLaunchKernelGGL(rot, dim3(Hkv_s, B, rot_blocks_d(D)), dim3(256), 0, st, ra);

  DecodeArgs da{};
  da.kvdiv = g;
  da.q_rot = ra.q_rot;
  da.k_pages = static_cast<const uint8_t*>(k_pages);
  da.v_pages = static_cast<const uint8_t*>(v_pages);
  da.table = page_table;
  da.seq_lens = seq_lens;
  da.part_acc = reinterpret_cast<float*>(ws + lay.acc);
  da.part_ml = reinterpret_cast<float*>(ws + lay.ml);
  da.ksp = k_stride_p;
  da.ksh = k_stride_h;
  da.vsp = v_stride_p;
  da.vsh = v_stride_h;
  da.tsb = table_stride_b;
  da.chunk_prefix = prefix;
  da.unit_meta = meta;
  da.B = B;
  da.Hkv = Hkv_s;
  da.n_rep = n_rep_s;
  da.log2S = ilog2(S);
  da.pages_per_split = pages_per_split;
  da.num_splits = num_splits;
  da.balanced = balanced ? 1 : 0;
  da.qrows = pad_nrep(n_rep_s);
  const int64_t waves = balanced ? int64_t(num_splits) : int64_t(num_splits) * Hkv_s * B;
  // the MFMA scan numbers its waves across work-groups of sk.wpb waves; the fp32 scan
  // runs one work-group per (split, virtual kv head, sequence)
  const dim3 grid = sk.rows ? dim3(unsigned((waves + sk.wpb - 1) / sk.wpb)) : dim3(num_splits, Hkv_s, B);
  if (ev_begin) hipEventRecord(static_cast<hipEvent_t>(ev_begin), st);
  hipLaunchKernelGGL(sk.fn, grid, dim3(sk.block), 0, st, da);
  if (ev_end) hipEventRecord(static_cast<hipEvent_t>(ev_end), st);

  MergeArgs ma{da.part_acc, da.part_ml, nullptr, meta, out, out_dtype, Hq, Hkv_s, n_rep_s, 1};
  launch_merge(D, dim3(n_rep_s, Hkv_s, B), st, ma);
  return check_launch("wn_dense_decode_attention");
}
