// Matrix-core page scan of the packed decode attention (head_dim 128, <= 4 query
// heads per kv head), gfx950.
//
// One work-group = two waves that share every 64-token chunk of the split; wave
// `h` decodes the codes of dims [64h, 64h+64) of K and of V.
//
// Both products run on v_mfma_f32_4x4x1_16b_f32 (16 independent 4x4x1 fp32
// blocks, exact fp32 multiply-add). Operand lanes: A[blk][i] from lane 4blk+i,
// B[blk][j] from lane 4blk+j, D[blk][i][j] in register i of lane 4blk+j; with
// CBSZ=4 every block takes A from block ABID instead.
//
//   score  A = q_rot[head i][dim k], broadcast from block ABID = k%16 of the
//          four registers that hold this wave's 256 query values;
//          B = c_K[code(token c0+lane, dim k)]
//          -> lane l, reg i : partial s(token c0+l, head i) over this wave's
//          dims. Both halves go to LDS as [head][token]; each wave reads the
//          two halves transposed and adds them in a fixed order, so both waves
//          hold the same scores in the value layout below.
//   value  A = p(token c0+4(l/4)+v, head l%4) * n_V
//          B = c_V[code(token c0+4(l/4)+v, dim 64h+16(l%4)+g)]
//          -> acc[g] lane l, reg r : head r, dim 64h+16(l%4)+g, summed over the
//          tokens of block l/4; blocks are folded once at the end.
//
// Online softmax in log2 units (q_rot carries log2 e) with a lazy reference
// maximum: a head's reference max moves (rescaling its accumulators) only when
// a score exceeds it by more than kRescale, so 2^(s - m) <= 2^kRescale and
// nothing overflows; the split merge is exact for any reference max. The
// wave-wide max reduction runs only on the first chunk and when that happens.
// Partials (m in log2 units, l, acc) go to the workspace for merge_kernel.
//
// Codebooks live in LDS (2^bw fp32 entries: the 64 lanes of a lookup read at
// most 2^bw distinct words). Page ids are fetched one chunk ahead and the packed
// rows of the next chunk are loaded while the current one is computed.
#include <utility>

#include "wn_decode.h"

namespace wn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kRescale = 8.0f;  // log2 units: p <= 2^8 before a rescale

template <int NBYTES>
struct Bytes {
  static constexpr int kWords = (NBYTES + 3) / 4;
  uint32_t w[kWords];
};

// NBYTES bytes at p into little-endian words; ALIGN is the guaranteed alignment of p.
template <int NBYTES, int ALIGN>
__device__ __forceinline__ void load_bytes(const uint8_t* p, Bytes<NBYTES>& out) {
  if constexpr (ALIGN >= 16 && NBYTES % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NBYTES / 16; ++i) {
      const uint4 x = reinterpret_cast<const uint4*>(p)[i];
      out.w[4 * i] = x.x;
      out.w[4 * i + 1] = x.y;
      out.w[4 * i + 2] = x.z;
      out.w[4 * i + 3] = x.w;
    }
  } else if constexpr (ALIGN >= 8 && NBYTES % 8 == 0) {
#pragma unroll
    for (int i = 0; i < NBYTES / 8; ++i) {
      const uint2 x = reinterpret_cast<const uint2*>(p)[i];
      out.w[2 * i] = x.x;
      out.w[2 * i + 1] = x.y;
    }
  } else if constexpr (ALIGN >= 4 && NBYTES % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NBYTES / 4; ++i) out.w[i] = reinterpret_cast<const uint32_t*>(p)[i];
  } else if constexpr (ALIGN >= 2 && NBYTES % 2 == 0) {
#pragma unroll
    for (int i = 0; i < Bytes<NBYTES>::kWords; ++i) out.w[i] = 0;
#pragma unroll
    for (int i = 0; i < NBYTES / 2; ++i)
      out.w[i / 2] |= uint32_t(reinterpret_cast<const uint16_t*>(p)[i]) << (16 * (i & 1));
  } else {
#pragma unroll
    for (int i = 0; i < Bytes<NBYTES>::kWords; ++i) out.w[i] = 0;
#pragma unroll
    for (int i = 0; i < NBYTES; ++i) out.w[i / 4] |= uint32_t(p[i]) << (8 * (i & 3));
  }
}

template <int NBYTES>
__device__ __forceinline__ void zero_bytes(Bytes<NBYTES>& out) {
#pragma unroll
  for (int i = 0; i < Bytes<NBYTES>::kWords; ++i) out.w[i] = 0;
}

constexpr int pow2_align(int x) { return (x % 16 == 0) ? 16 : (x % 8 == 0) ? 8 : (x % 4 == 0) ? 4 : (x % 2 == 0) ? 2 : 1; }

template <int BWK, int BWV>
struct ChunkRegs {
  static constexpr int KB = 8 * BWK;  // bytes of 64 K codes (this wave's half row)
  static constexpr int VB = 2 * BWV;  // bytes of 16 V codes
  Bytes<KB> k;                        // token c0 + lane, dims [64h, 64h+64)
  Bytes<VB> v[4];                     // tokens c0 + 4(l/4) + r, dims 64h + 16(l%4) + [0, 16)
  uint32_t nk[2], nv[2];              // fp16 norms of tokens c0 + 4(l/4) + [0, 4)
};

template <int BWK, int BWV>
__device__ __forceinline__ void load_chunk(const DecodeArgs& a, int kvh, int h, int lane, int c0, int t_hi,
                                           int pid, ChunkRegs<BWK, BWV>& r) {
  constexpr int NBK = 16 * BWK, NBV = 16 * BWV;
  constexpr int KB = ChunkRegs<BWK, BWV>::KB, VB = ChunkRegs<BWK, BWV>::VB;
  const int blk = lane >> 2, col = lane & 3;
  const int tb = c0 + 4 * blk;  // first token of this lane's block
  if (tb < t_hi) {              // the block's page exists; slots past t_hi are masked later
    const int S1 = (1 << a.log2S) - 1;
    const int slot = (c0 + lane) & S1;
    const int slot_b = tb & S1;
    load_bytes<KB, pow2_align(KB)>(a.k_pages + pid * a.ksp + kvh * a.ksh + slot * NBK + h * KB, r.k);
    const uint8_t* vrow = a.v_pages + pid * a.vsp + kvh * a.vsh + slot_b * NBV + h * 8 * BWV + col * VB;
#pragma unroll
    for (int i = 0; i < 4; ++i) load_bytes<VB, pow2_align(VB)>(vrow + i * NBV, r.v[i]);
    const uint2 nk = *reinterpret_cast<const uint2*>(a.k_norms + pid * a.knp + kvh * a.knh + slot_b);
    const uint2 nv = *reinterpret_cast<const uint2*>(a.v_norms + pid * a.vnp + kvh * a.vnh + slot_b);
    r.nk[0] = nk.x;
    r.nk[1] = nk.y;
    r.nv[0] = nv.x;
    r.nv[1] = nv.y;
  } else {
    zero_bytes(r.k);
#pragma unroll
    for (int i = 0; i < 4; ++i) zero_bytes(r.v[i]);
    r.nk[0] = r.nk[1] = r.nv[0] = r.nv[1] = 0;
  }
}

__device__ __forceinline__ float half_at(const uint32_t (&w)[2], int i) {
  return f16_to_f32(uint16_t(w[i >> 1] >> (16 * (i & 1))));
}

// Byte address (code * 4) of code K of a packed row held as little-endian
// words, into a 2^BW-entry fp32 LDS table. 4-bit codes take 12 ops per word of
// 8 (CSE shares the two masks): even and odd nibbles are spread to bytes
// already multiplied by 4, then v_perm_b32 isolates each byte.
template <int BW, int K, int NW>
__device__ __forceinline__ uint32_t code_addr(const uint32_t (&w)[NW]) {
  if constexpr (BW == 4) {
    constexpr int i = K >> 3, byte = (K & 7) >> 1;
    const uint32_t x = (K & 1) ? ((w[i] >> 2) & 0x3C3C3C3Cu) : ((w[i] << 2) & 0x3C3C3C3Cu);
    // v_perm_b32: byte `byte` of x into byte 0, zeros above (selector 0x0c = 0x00)
    return __builtin_amdgcn_perm(x, x, 0x0c0c0c00u | byte);
  } else {
    constexpr int bit = K * BW, wi = bit >> 5, sh = bit & 31;
    uint32_t v = w[wi] >> sh;
    if constexpr (sh + BW > 32) v |= w[wi + 1] << (32 - sh);
    return (v & ((1u << BW) - 1u)) << 2;
  }
}

__device__ __forceinline__ float lds_at(const float* tab, uint32_t byte_addr) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + byte_addr);
}

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Scores of this lane's token over the wave's 64 dims in 8 groups of 8: the
// lookups of group g+1 are issued before the 8 MFMAs of group g (A = q broadcast
// from block k%16 of qb[k/16], B = codebook value of dim 64h+k), and a
// scheduling barrier keeps the next groups from being hoisted.
template <int BWK, int NW>
__device__ __forceinline__ void score_pipelined(const uint32_t (&kw)[NW], const float* cbk, const float (&qb)[4],
                                                f32x4& s0, f32x4& s1) {
  float kv[2][8];
  auto look = [&](auto gc) {
    constexpr int g = decltype(gc)::value;
    static_for<0, 8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      kv[g & 1][j] = lds_at(cbk, code_addr<BWK, 8 * g + j>(kw));
    });
  };
  look(std::integral_constant<int, 0>{});
  static_for<0, 8>([&](auto gc) {
    constexpr int g = decltype(gc)::value;
    if constexpr (g + 1 < 8) look(std::integral_constant<int, g + 1>{});
    static_for<0, 8>([&](auto jc) {
      constexpr int j = decltype(jc)::value, k = 8 * g + j;
      if constexpr (j & 1)
        s1 = __builtin_amdgcn_mfma_f32_4x4x1f32(qb[k >> 4], kv[g & 1][j], s1, 4, k & 15, 0);
      else
        s0 = __builtin_amdgcn_mfma_f32_4x4x1f32(qb[k >> 4], kv[g & 1][j], s0, 4, k & 15, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Values: 4 tokens x 16 dims per lane, 8 groups of 8 (group G: token G/2, dims
// 8(G%2)+[0,8)), pipelined like the scores; A = p * n_V of the group's token.
template <int BWV, int NB>
__device__ __forceinline__ void value_pipelined(const Bytes<NB> (&vr)[4], const float* cbv,
                                                const float (&p)[4], f32x4 (&acc)[16]) {
  float vv[2][8];
  auto look = [&](auto gc) {
    constexpr int G = decltype(gc)::value;
    static_for<0, 8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      vv[G & 1][j] = lds_at(cbv, code_addr<BWV, 8 * (G & 1) + j>(vr[G >> 1].w));
    });
  };
  look(std::integral_constant<int, 0>{});
  static_for<0, 8>([&](auto gc) {
    constexpr int G = decltype(gc)::value;
    if constexpr (G + 1 < 8) look(std::integral_constant<int, G + 1>{});
    static_for<0, 8>([&](auto jc) {
      constexpr int j = decltype(jc)::value, d = 8 * (G & 1) + j;
      acc[d] = __builtin_amdgcn_mfma_f32_4x4x1f32(p[G >> 1], vv[G & 1][j], acc[d], 0, 0, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Sum of x over the 16 lanes with this lane's lane%4 (row_ror 4 and 8 inside
// a row of 16, then rows through ds_bpermute with precomputed addresses).
__device__ __forceinline__ float fold16(float x, int a16, int a32) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(a16, __builtin_bit_cast(int, x)));
  x += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(a32, __builtin_bit_cast(int, x)));
  return x;
}

struct WaveState {
  f32x4 acc[16];
  float m_ref;  // reference max (log2 units) of head lane%4
  float lsum;   // sum of exp2(s - m_ref) over this lane's block tokens, head lane%4
};

// One 64-token chunk. Scores are in log2 units (q_rot carries log2 e).
template <int BWK, int BWV>
__device__ __forceinline__ void process_chunk(const ChunkRegs<BWK, BWV>& cur, int c, int c0, int t_hi, int h,
                                              int lane, const float* cbk, const float* cbv,
                                              const float (&qb)[4], float (*xs)[2][4][64], WaveState& st) {
  const int blk = lane >> 2, col = lane & 3;
  // ---- partial scores of token c0+lane over this wave's 64 dims
  f32x4 sp0 = f32x4{0.f, 0.f, 0.f, 0.f}, sp1 = sp0;
  score_pipelined<BWK>(cur.k.w, cbk, qb, sp0, sp1);
  const f32x4 sp = sp0 + sp1;
  float* xw = &xs[c & 1][h][0][0];
#pragma unroll
  for (int r = 0; r < 4; ++r) xw[r * 64 + lane] = sp[r];
  __syncthreads();
  const f32x4 sfull = *reinterpret_cast<const f32x4*>(&xs[c & 1][0][col][4 * blk]) +
                      *reinterpret_cast<const f32x4*>(&xs[c & 1][1][col][4 * blk]);

  // ---- online softmax for head `col` over tokens c0 + 4blk + [0, 4)
  const int tb = c0 + 4 * blk;
  float s[4], p[4], nv[4];
  float lmax = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool ok = tb + r < t_hi;
    s[r] = ok ? sfull[r] * half_at(cur.nk, r) : -INFINITY;
    nv[r] = ok ? half_at(cur.nv, r) : 0.f;
    lmax = fmaxf(lmax, s[r]);
  }
  if (st.m_ref == -INFINITY || __any(lmax > st.m_ref + kRescale)) {
    float cmax = lmax;
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, o, 64));
    const float m_new = fmaxf(st.m_ref, cmax);
    const float alpha = __builtin_amdgcn_exp2f(st.m_ref - m_new);  // 0 on the first chunk
    st.lsum *= alpha;
    st.m_ref = m_new;
    float al[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) al[r] = __shfl(alpha, (lane & ~3) | r, 64);
#pragma unroll
    for (int g = 0; g < 16; ++g) st.acc[g] *= f32x4{al[0], al[1], al[2], al[3]};
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = __builtin_amdgcn_exp2f(s[r] - st.m_ref);  // exp2(-inf) = 0 for masked tokens
    st.lsum += p[r];
    p[r] *= nv[r];
  }

  // ---- values: 4 tokens x 16 dims per lane
  value_pipelined<BWV>(cur.v, cbv, p, st.acc);
}

template <int BWK, int BWV>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(3, 8))) void decode_mfma4_kernel(
    DecodeArgs a) {
  constexpr int D = 128;
  constexpr int LK = 1 << BWK, LV = 1 << BWV;
  __shared__ float cbk[LK];
  __shared__ float cbv[LV];
  __shared__ float xs[2][2][4][64];  // [chunk parity][half][head][token] partial scores

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, h = tid >> 6, lane = tid & 63;
  const int blk = lane >> 2, col = lane & 3;
  const int S = 1 << a.log2S;
  const int L = a.seq_lens[b];
  const int n_pages = (L + S - 1) >> a.log2S;
  const int page_lo = split * a.pages_per_split;
  if (page_lo >= n_pages) return;  // block-uniform
  const int page_hi = min(page_lo + a.pages_per_split, n_pages);
  const int t_lo = page_lo << a.log2S;
  const int t_hi = min(page_hi << a.log2S, L);
  const int n_chunks = (t_hi - t_lo + 63) >> 6;

  for (int i = tid; i < LK; i += 128) cbk[i] = a.cb_k[i];
  for (int i = tid; i < LV; i += 128) cbv[i] = a.cb_v[i];

  // register m of lane 4j+i holds q_rot[head i][64h + 16m + j]
  float qb[4];
  {
    const float* qp = a.q_rot + ((int64_t(b) * a.Hkv + kvh) * 4 + col) * D + 64 * h + blk;
#pragma unroll
    for (int m = 0; m < 4; ++m) qb[m] = qp[16 * m];
  }
  const int32_t* trow = a.table + b * a.tsb;
  __syncthreads();

  WaveState st;
#pragma unroll
  for (int g = 0; g < 16; ++g) st.acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m_ref = -INFINITY;
  st.lsum = 0.f;

  auto pid_of = [&](int c) {
    const int tb = t_lo + 64 * c + 4 * blk;
    return (c < n_chunks && tb < t_hi) ? trow[tb >> a.log2S] : 0;
  };
  // chunk c+1 loads while chunk c computes; page ids run two ahead. One masked
  // chunk body (two inlined copies of it exceed the register budget).
  ChunkRegs<BWK, BWV> cur, nxt;
  load_chunk(a, kvh, h, lane, t_lo, t_hi, pid_of(0), cur);
  int pid_next = pid_of(1);
  for (int c = 0; c < n_chunks; ++c) {
    if (c + 1 < n_chunks) load_chunk(a, kvh, h, lane, t_lo + 64 * (c + 1), t_hi, pid_next, nxt);
    pid_next = pid_of(c + 2);
    process_chunk(cur, c, t_lo + 64 * c, t_hi, h, lane, cbk, cbv, qb, xs, st);
    cur = nxt;
  }

  // ---- fold the 16 token blocks: lanes with equal lane%4 hold the same dims
  const int a16 = (lane ^ 16) << 2, a32 = (lane ^ 32) << 2;
  st.lsum = fold16(st.lsum, a16, a32);
#pragma unroll
  for (int g = 0; g < 16; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r) st.acc[g][r] = fold16(st.acc[g][r], a16, a32);

  const int64_t row0 = ((int64_t(b) * a.Hkv + kvh) * a.num_splits + split) * a.n_rep;
  if (lane < 4) {  // lane j: dims 64h + 16j + g, heads 0..3
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r < a.n_rep) {
        float* dst = a.part_acc + (row0 + r) * D + 64 * h + 16 * lane;
#pragma unroll
        for (int g = 0; g < 16; g += 4)
          *reinterpret_cast<float4*>(dst + g) =
              make_float4(st.acc[g][r], st.acc[g + 1][r], st.acc[g + 2][r], st.acc[g + 3][r]);
      }
    }
    if (h == 0 && lane < a.n_rep) {  // lane j holds m and l of head j
      a.part_ml[2 * (row0 + lane)] = st.m_ref;
      a.part_ml[2 * (row0 + lane) + 1] = st.lsum;
    }
  }

}

}  // namespace

SplitKernel pick_split_mfma(int bw_k, int bw_v) {
  SplitFn f = nullptr;
  if (bw_k == bw_v) {
    switch (bw_k) {
      case 2: f = decode_mfma4_kernel<2, 2>; break;
      case 3: f = decode_mfma4_kernel<3, 3>; break;
      case 4: f = decode_mfma4_kernel<4, 4>; break;
      case 5: f = decode_mfma4_kernel<5, 5>; break;
      case 6: f = decode_mfma4_kernel<6, 6>; break;
      case 8: f = decode_mfma4_kernel<8, 8>; break;
    }
  } else if (bw_k == 4 && bw_v == 6) {
    f = decode_mfma4_kernel<4, 6>;
  } else if (bw_k == 6 && bw_v == 4) {
    f = decode_mfma4_kernel<6, 4>;
  } else if (bw_k == 4 && bw_v == 8) {
    f = decode_mfma4_kernel<4, 8>;
  }
  SplitKernel k;
  if (f) {
    k.fn = f;
    k.block = 128;
    k.nrep = 4;
    k.log2_units = true;
  }
  return k;
}

}  // namespace wn
