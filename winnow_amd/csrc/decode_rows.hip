// Row-per-lane matrix-core page scan of the packed decode attention (head_dim 128,
// power-of-two page size >= 16, up to eight query heads per (virtual) kv head in one
// or two groups of four; the host runs an even n_rep of 10..16 as two virtual kv
// heads per kv head, kvshift), gfx950.
//
// Waves are independent of each other; the waves of a work-group only share the
// codebook tables staged in LDS. With fixed splits a wave owns a range of pages of
// one (sequence, kv head); with a balanced plan
// the resident waves split the flattened (sequence, kv head, chunk) space into
// equal shares. Either way a wave walks its tokens in 64-token chunks.
//
//   scores  lane l holds the packed K row of token c0+l. For each dim k one
//           v_mfma_f32_4x4x1_16b_f32 per group of four heads, with A = q_rot[head i][k]
//           broadcast to all 16 blocks (CBSZ=4, ABID=k%16) and B = c_K[code(token, k)],
//           gives D[block][i][j] = partial s(head i, token 4*block+j): lane l ends
//           with its own token's scores. 128 MFMAs per chunk and head group; each
//           codebook lookup feeds every group.
//   softmax per head in log2 units (q_rot carries log2 e), lane = token, with a
//           lazy reference maximum: it moves (rescaling the accumulators) only
//           when a score exceeds it by more than kRescale, so 2^(s - m) <= 2^kRescale.
//   values  p * n_V goes through a 1.3 KB LDS tile so that lanes 16G+i hold
//           p(head i, token c0+4q+G) for the 16 token quads q. Lanes 16G..16G+15
//           hold the packed V codes of dims 8p..8p+7 (p = lane%16) of that token.
//           A v_mfma_f32_4x4x1_16b_f32 with CBSZ=2 broadcasts A inside each group of
//           four blocks, so block group G accumulates token c0+4q+G into
//           acc[m] register i = (head i, dim 8p+m). 8 MFMAs per quad, 128 per chunk;
//           the four groups are folded once per split.
//
// Codebooks sit in LDS; every product is an exact fp32 multiply-add. 4-bit codes
// are looked up two at a time in a byte-indexed table of (c[lo nibble], c[hi nibble])
// pairs that is replicated once per lane of a half-wave, so that the 32 lanes LDS
// serves together always read 32 distinct bank pairs: a lookup never waits on a
// bank conflict, whatever the codes. Twelve waves per work-group (eight with two
// head groups or wider codes) share the tables.
// Page ids run two chunks ahead and the packed rows of chunk c+1 load while chunk c
// computes.
// Algebra: turboquant_kv/packed_attention.py:260-334 (the schedule of the
// reference kernel packed_attention_triton.py:51-134).
#include <utility>

#include "wn_decode.h"

namespace wn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));


constexpr float kRescale = 8.0f;
constexpr int kPStride = 20;  // floats per (head, token group) row of the p tile (16 + pad, 16-B rows)

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <int K>
__device__ __forceinline__ float comp(const float4& x) {
  if constexpr (K == 0) return x.x;
  else if constexpr (K == 1) return x.y;
  else if constexpr (K == 2) return x.z;
  else return x.w;
}

// Row of the p tile lane 16G+i reads its value-MFMA operands of head group g from:
// p(head 4g+i, token c0+4q+G) * n_V sits at row 16g + 4i + G, column q.
__device__ __forceinline__ const float4* tile_row(const float* pt, int g, int lane) {
  return reinterpret_cast<const float4*>(pt + (16 * g + (lane & 3) * 4 + (lane >> 4)) * kPStride);
}

// Byte K of x written into byte 1 of r, the other bytes of r kept: one VOP2 SDWA
// move. With r = 8*(lane % 32) | slot << 16 this is the LDS byte address of entry
// (byte K of x, lane % 32) of the replicated pair table in 64 KB slot `slot`.
template <int K>
__device__ __forceinline__ uint32_t put_byte1(uint32_t r, uint32_t x) {
  if constexpr (K == 0)
    asm("v_mov_b32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0" : "+v"(r) : "v"(x));
  else if constexpr (K == 1)
    asm("v_mov_b32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1" : "+v"(r) : "v"(x));
  else if constexpr (K == 2)
    asm("v_mov_b32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_2" : "+v"(r) : "v"(x));
  else
    asm("v_mov_b32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3" : "+v"(r) : "v"(x));
  return r;
}

constexpr int kPairTableBytes = 256 * 32 * 8;  // 256 byte values x 32 lanes x float2

// Widths read two codes per LDS access from a plain (not replicated) pair table of
// 2^(2 BW) entries: 2, 3, 5 and 6 bits (128 B to 32 KB). 4-bit codes have the
// replicated byte table; 8-bit pairs would need 512 KB.
template <int BW>
constexpr bool pair_coded() { return BW == 2 || BW == 3 || BW == 5 || BW == 6; }

// LDS bytes the codebook of BW-bit codes occupies: the replicated pair table for
// 4-bit codes, the pair table of pair_coded widths, else the plain 2^BW-entry table
// (padded to 16 bytes).
template <int BW>
constexpr int table_bytes() {
  return BW == 4 ? kPairTableBytes : pair_coded<BW>() ? (8 << (2 * BW)) : (4 << BW) < 16 ? 16 : (4 << BW);
}

// A codebook in LDS as one lane reads it.
template <int BW>
struct Tab {
  const float* t;  // plain table: lanes sharing a code share an address (LDS broadcasts)
};
template <>
struct Tab<4> {
  const char* lds;  // LDS block base; the table sits at 64 KB slot `slot` of it
  uint32_t r[4];    // address registers, one per byte position of a code word
  __device__ void init(const char* base, int slot, int lane) {
    lds = base;
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = uint32_t(8 * (lane & 31)) | (uint32_t(slot) << 16);
  }
};

// Stages a codebook into LDS at `dst` with all `nthr` threads of the work-group:
// the replicated pair table for 4-bit codes (entry (b, r) at byte 256*b + 8*r holds
// (c[b & 15], c[b >> 4])), the pair table of pair_coded widths (entry i holds
// (c[i mod 2^BW], c[i >> BW]): two consecutive codes, LSB first, read as one
// 2*BW-bit index), else the plain table.
template <int BW>
__device__ __forceinline__ void stage_table(const float* cb, char* dst, int tid, int nthr) {
  if constexpr (BW == 4) {
    float2* t = reinterpret_cast<float2*>(dst);
    for (int i = tid; i < 256 * 32; i += nthr) {
      const int b = i >> 5;
      t[i] = make_float2(cb[b & 15], cb[b >> 4]);
    }
  } else if constexpr (pair_coded<BW>()) {
    float2* t = reinterpret_cast<float2*>(dst);
    for (int i = tid; i < (1 << (2 * BW)); i += nthr) t[i] = make_float2(cb[i & ((1 << BW) - 1)], cb[i >> BW]);
  } else {
    float* t = reinterpret_cast<float*>(dst);
    for (int i = tid; i < (1 << BW); i += nthr) t[i] = cb[i];
  }
}

// Codebook values of the 8 codes starting at bit BIT0 of the word array (LSB-first,
// BW bits each) into v[0..7]: one SDWA move and one 8-byte LDS read per two 4-bit
// codes; one 2*BW-bit extract and one 8-byte read per two codes of a pair_coded
// width; 8-bit codes are read one by one from the plain table.
template <int BW, int BIT0, int NW>
__device__ __forceinline__ void lookup8(const uint32_t (&w)[NW], Tab<BW>& tab, float (&v)[8]) {
  if constexpr (BW == 4) {
    static_assert(BIT0 % 32 == 0, "4-bit groups are word aligned");
    static_for<0, 4>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      tab.r[k] = put_byte1<k>(tab.r[k], w[BIT0 / 32]);
      const float2 e = *reinterpret_cast<const float2*>(tab.lds + tab.r[k]);
      v[2 * k] = e.x;
      v[2 * k + 1] = e.y;
    });
  } else if constexpr (pair_coded<BW>()) {
    static_for<0, 4>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      constexpr int bit = BIT0 + 2 * BW * k, wi = bit >> 5, sh = bit & 31;
      uint32_t x = w[wi] >> sh;
      if constexpr (sh + 2 * BW > 32) x |= w[wi + 1] << (32 - sh);
      const float2 e = reinterpret_cast<const float2*>(tab.t)[x & ((1u << (2 * BW)) - 1u)];
      v[2 * k] = e.x;
      v[2 * k + 1] = e.y;
    });
  } else {
    static_for<0, 8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int bit = BIT0 + j * BW, wi = bit >> 5, sh = bit & 31;
      uint32_t x = w[wi] >> sh;
      if constexpr (sh + BW > 32) x |= w[wi + 1] << (32 - sh);
      v[j] = tab.t[x & ((1u << BW) - 1u)];
    });
  }
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): every vector
// memory load this wave issued has returned.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// A value every lane holds alike, moved to a scalar register.
__device__ __forceinline__ float uniform(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

__device__ __forceinline__ float half_lo(uint32_t h) { return f16_to_f32(uint16_t(h & 0xffffu)); }

// Words of the V codes one lane reads per token: BWV bytes (8 codes).
template <int BWV>
struct VWords {
  static constexpr int N = BWV <= 4 ? 1 : 2;
};

// One buffer of packed rows. As a K buffer it holds the packed K row of token
// c0 + lane (words [0, KW)) and that token's fp16 K and V norms (words KW, KW+1);
// as a V buffer, for each token quad q, the codes 8p..8p+7 of token c0 + 4q + G
// (G = lane/16, p = lane%16) at words [q*VW, q*VW + VW). A chunk's K buffer is
// refilled with the next chunk's V codes once the softmax has used the norms.
template <int BWK, int BWV>
struct RowBuf {
  static constexpr int KW = 4 * BWK;
  static constexpr int VW = VWords<BWV>::N;
  static constexpr int W = KW + 2 > 16 * VW ? KW + 2 : 16 * VW;
  uint32_t w[W];
};

// BWV bytes at p (8 codes of one lane) into little-endian words. p is aligned to
// gcd(BWV, 8)-ish: 4 and 8 are naturally aligned, 2 and 6 use 2-byte pieces.
// At 2, 4 and 8 bits one load instruction reads four whole packed rows (a
// contiguous 128, 256 or 512 bytes), so nothing of its lines is read again by
// another instruction: those loads are nontemporal (streamed past the caches),
// which measured 1.3 % faster on the 4/4-bit scan. The 6-bit pieces of a row come
// from two instructions, and 3/5-bit rows from bytes, so they keep cached loads.
template <int BWV>
__device__ __forceinline__ void load_vcodes(const uint8_t* p, bool odd_lane, uint32_t (&out)[VWords<BWV>::N]) {
  if constexpr (BWV == 4) {
    out[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
  } else if constexpr (BWV == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 x = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    out[0] = x.x;
    out[1] = x.y;
  } else if constexpr (BWV == 2) {
    out[0] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
  } else if constexpr (BWV == 6) {
    // bytes [6p, 6p+6): a 4-byte-aligned dword and a 2-byte piece, placed by lane parity
    const uint32_t d = *reinterpret_cast<const uint32_t*>(p + (odd_lane ? 2 : 0));
    const uint32_t h = *reinterpret_cast<const uint16_t*>(p + (odd_lane ? 0 : 4));
    out[0] = odd_lane ? (h | (d << 16)) : d;
    out[1] = odd_lane ? (d >> 16) : h;
  } else {  // 3 or 5 bytes, byte-aligned
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < BWV; ++i) {
      const uint32_t bv = p[i];
      if (i < 4) w0 |= bv << (8 * i);
      else w1 |= bv << (8 * (i - 4));
    }
    out[0] = w0;
    if constexpr (VWords<BWV>::N > 1) out[1] = w1;
  }
}

// Running state of NG groups of four query heads (head 4g+i is register i of group g).
template <int NG>
struct RowState {
  f32x4 acc[NG][8];  // acc[g][m] register i: head 4g+i, dim 8p+m (partial over this lane's token group)
  float m[4 * NG];   // reference maxima (wave-uniform), log2 units
  float l[4 * NG];   // sum of 2^(s - m) over this lane's tokens
};

// K side of chunk [c0, c0+64): the packed K row and both norms of token c0+lane,
// whose page is pid_lane.
template <int BWK, int BWV>
__device__ __forceinline__ void load_k(const DecodeArgs& a, int kvh, int lane, int c0, int pid_lane,
                                       RowBuf<BWK, BWV>& r) {
  constexpr int NBK = 16 * BWK, KW = RowBuf<BWK, BWV>::KW;
  const int slot = (c0 + lane) & ((1 << a.log2S) - 1);
  const uint8_t* krow = a.k_pages + int64_t(pid_lane) * a.ksp + (kvh >> a.kvshift) * a.ksh + slot * NBK;
#pragma unroll
  for (int i = 0; i < NBK / 16; ++i) {
    const uint4 x = reinterpret_cast<const uint4*>(krow)[i];
    r.w[4 * i] = x.x;
    r.w[4 * i + 1] = x.y;
    r.w[4 * i + 2] = x.z;
    r.w[4 * i + 3] = x.w;
  }
  r.w[KW] = a.k_norms[int64_t(pid_lane) * a.knp + (kvh >> a.kvshift) * a.knh + slot];
  r.w[KW + 1] = a.v_norms[int64_t(pid_lane) * a.vnp + (kvh >> a.kvshift) * a.vnh + slot];
}

// V side of chunk [c0, c0+64): for every token quad q the BWV bytes of codes
// 8p..8p+7 of token c0+4q+G (G = lane/16, p = lane%16). c0 is a multiple of 16 and
// pages hold >= 16 tokens, so the four quads of 16-token block j share the page of
// lane 16j (pid_lane is the page of token c0+lane).
template <int BWK, int BWV>
__device__ __forceinline__ void load_v(const DecodeArgs& a, int kvh, int lane, int c0, int pid_lane,
                                       RowBuf<BWK, BWV>& r) {
  constexpr int NBV = 16 * BWV, VW = RowBuf<BWK, BWV>::VW;
  const int smask = (1 << a.log2S) - 1;
  const int p = lane & 15;
  const int lane_off = (lane >> 4) * NBV + BWV * p;
  static_for<0, 4>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int pid_j = __builtin_amdgcn_readlane(pid_lane, 16 * j);
    const uint8_t* vj = a.v_pages + int64_t(pid_j) * a.vsp + (kvh >> a.kvshift) * a.vsh + ((c0 + 16 * j) & smask) * NBV + lane_off;
    static_for<0, 4>([&](auto qc) {
      constexpr int qq = decltype(qc)::value;
      uint32_t t[VW];
      load_vcodes<BWV>(vj + 4 * qq * NBV, p & 1, t);
#pragma unroll
      for (int x = 0; x < VW; ++x) r.w[(4 * j + qq) * VW + x] = t[x];
    });
  });
}

// Score lookups of dims [8g, 8g+8) of this lane's K row.
template <int BWK, int G, int NW>
__device__ __forceinline__ void score_look(const uint32_t (&k)[NW], Tab<BWK>& cbk, float (&kv)[8]) {
  lookup8<BWK, 8 * G * BWK>(k, cbk, kv);
}

// The score MFMAs of dims [8g, 8g+8), eight per head group: A = q_rot[head][k]
// broadcast from block k%16; every lookup feeds one MFMA per group.
template <int G, int NG>
__device__ __forceinline__ void score_mfma(const float (&qb)[NG][8], const float (&kv)[8], f32x4 (&s0)[NG],
                                           f32x4 (&s1)[NG]) {
  static_for<0, 8>([&](auto jc) {
    constexpr int j = decltype(jc)::value, k = 8 * G + j;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if constexpr (j & 1)
        s1[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(qb[g][k >> 4], kv[j], s1[g], 4, k & 15, 0);
      else
        s0[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(qb[g][k >> 4], kv[j], s0[g], 4, k & 15, 0);
    }
  });
}

// Value lookups of quad q (this lane's 8 dims of token c0+4q+G).
template <int BWV, int Q, int NW>
__device__ __forceinline__ void value_look(const uint32_t (&v)[NW], Tab<BWV>& cbv, float (&vv)[8]) {
  lookup8<BWV, 32 * VWords<BWV>::N * Q>(v, cbv, vv);
}

// The value MFMAs of quad q, eight per head group: A = p*n_V broadcast inside each
// group of four blocks.
template <int NG>
__device__ __forceinline__ void value_mfma(const float (&a_q)[NG], const float (&vv)[8], f32x4 (&acc)[NG][8]) {
  static_for<0, 8>([&](auto mc) {
    constexpr int mm = decltype(mc)::value;
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[g][mm] = __builtin_amdgcn_mfma_f32_4x4x1f32(a_q[g], vv[mm], acc[g][mm], 2, 0, 0);
  });
}

// Scores of the chunk's 64 tokens (lane = token, register i = head i). The
// lookups of group g+2 are issued before the MFMAs of group g, so every LDS read
// has sixteen of this wave's MFMAs to land before its value is needed; the sched
// barriers keep the compiler from sinking the reads next to their consumers.
template <int BWK, int NG, int NW>
__device__ __forceinline__ void score_phase(const uint32_t (&kc)[NW], Tab<BWK>& cbk, const float (&qb)[NG][8],
                                            f32x4 (&out)[NG]) {
  f32x4 s0[NG], s1[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) s0[g] = s1[g] = f32x4{0.f, 0.f, 0.f, 0.f};
  float kv[3][8];
  score_look<BWK, 0>(kc, cbk, kv[0]);
  score_look<BWK, 1>(kc, cbk, kv[1]);
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 16>([&](auto gc) {
    constexpr int g = decltype(gc)::value;
    if constexpr (g + 2 < 16) {
      score_look<BWK, g + 2>(kc, cbk, kv[(g + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);
    }
    score_mfma<g, NG>(qb, kv[g % 3], s0, s1);
    __builtin_amdgcn_sched_barrier(0);
  });
#pragma unroll
  for (int g = 0; g < NG; ++g) out[g] = s0[g] + s1[g];
}

// Lookups of the first two value quads, issued before the softmax so that they
// land while it runs.
template <int BWV, int NW>
__device__ __forceinline__ void value_prime(const uint32_t (&vc)[NW], Tab<BWV>& cbv, float (&vv)[3][8]) {
  value_look<BWV, 0>(vc, cbv, vv[0]);
  value_look<BWV, 1>(vc, cbv, vv[1]);
  __builtin_amdgcn_sched_barrier(0);
}

// Values of a chunk; lookups of quad q+2 are issued before the MFMAs of quad q,
// and the p * n_V operands of four quads are read from the tile two quads before
// the first of them.
template <int BWV, int NG, int NW>
__device__ __forceinline__ void value_phase(const uint32_t (&vc)[NW], Tab<BWV>& cbv, const float* pt, int lane,
                                            f32x4 (&acc)[NG][8], float (&vv)[3][8]) {
  const float4* arow[NG];
  float4 ab[NG][2];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    arow[g] = tile_row(pt, g, lane);
    ab[g][0] = arow[g][0];
  }
  static_for<0, 16>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    if constexpr ((q & 3) == 2 && q + 2 < 16) {
#pragma unroll
      for (int g = 0; g < NG; ++g) ab[g][((q >> 2) + 1) & 1] = arow[g][(q >> 2) + 1];
    }
    if constexpr (q + 2 < 16) value_look<BWV, q + 2>(vc, cbv, vv[(q + 2) % 3]);
    __builtin_amdgcn_sched_barrier(0);
    float aq[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) aq[g] = comp<q & 3>(ab[g][(q >> 2) & 1]);
    value_mfma<NG>(aq, vv[q % 3], acc);
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Online softmax of one chunk (lane = token) and the p * n_V transposition: on
// return the tile holds p(head 4g+i, token c0+4q+G) * n_V at row 16g+4i+G, column q,
// and lane 16G+i finds its value-MFMA operands of group g for quads 4j..4j+3 at
// float4 j of row 16g + 4(lane%4) + lane/16 (tile_row).
template <int NG>
__device__ __forceinline__ void softmax_phase(const f32x4 (&s)[NG], uint32_t nk_h, uint32_t nv_h, bool valid,
                                              int lane, float* pt, RowState<NG>& st) {
  constexpr int H = 4 * NG;
  const float nk = half_lo(nk_h);
  const float nv = valid ? half_lo(nv_h) : 0.f;
  float sv[H];
#pragma unroll
  for (int i = 0; i < H; ++i) sv[i] = valid ? s[i >> 2][i & 3] * nk : -INFINITY;
  bool move = st.m[0] == -INFINITY;
#pragma unroll
  for (int i = 0; i < H; ++i) move = move || __any(sv[i] > st.m[i] + kRescale);
  if (move) {  // wave-uniform
#pragma unroll
    for (int i = 0; i < H; ++i) {
      // wave-uniform: kept in a scalar register, which frees a VGPR per head
      const float m_new = uniform(fmaxf(st.m[i], wave_max(sv[i])));
      const float alpha = __builtin_amdgcn_exp2f(st.m[i] - m_new);  // 0 on the first chunk
      st.m[i] = m_new;
      st.l[i] *= alpha;
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) st.acc[i >> 2][mm][i & 3] *= alpha;
    }
  }
  float pv[H];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float p = __builtin_amdgcn_exp2f(sv[i] - st.m[i]);  // 0 for masked tokens
    st.l[i] += p;
    pv[i] = p * nv;
  }
  wave_lds_sync();  // the previous chunk's reads of the tile are done
  {
    const int G = lane & 3, q = lane >> 2;
#pragma unroll
    for (int i = 0; i < H; ++i) pt[(16 * (i >> 2) + (i & 3) * 4 + G) * kPStride + q] = pv[i];
  }
  wave_lds_sync();
}



// Folds the four token groups and the per-lane sums and writes the (acc, m, l)
// partial of each query head h < n_rep to row prow * n_rep + h.
template <int NG>
__device__ __forceinline__ void write_partial(const DecodeArgs& a, RowState<NG>& st, int64_t prow, int lane) {
  constexpr int D = 128, H = 4 * NG;
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int mm = 0; mm < 8; ++mm)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = st.acc[g][mm][i];
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        st.acc[g][mm][i] = x;
      }
#pragma unroll
  for (int i = 0; i < H; ++i) st.l[i] = wave_sum(st.l[i]);
  const int64_t row0 = prow * a.n_rep;
  if (lane < 16) {  // lane p: dims 8p..8p+7 of every head
#pragma unroll
    for (int i = 0; i < H; ++i) {
      if (i < a.n_rep) {
        const f32x4* ac = st.acc[i >> 2];
        float* dst = a.part_acc + (row0 + i) * D + 8 * lane;
        *reinterpret_cast<float4*>(dst) = make_float4(ac[0][i & 3], ac[1][i & 3], ac[2][i & 3], ac[3][i & 3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(ac[4][i & 3], ac[5][i & 3], ac[6][i & 3], ac[7][i & 3]);
      }
    }
  }
  // m and l are wave-uniform: lane 0 writes every head's (a lane-indexed pick would
  // turn the register arrays into an indexed stack object)
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < H; ++i) {
      if (i < a.n_rep) {
        a.part_ml[2 * (row0 + i)] = st.m[i];
        a.part_ml[2 * (row0 + i) + 1] = st.l[i];
      }
    }
  }
}

// Scans tokens [t_lo, t_hi) of (sequence b, kv head kvh) in 64-token chunks (t_lo a
// multiple of 16) and writes one partial at row prow. Each chunk runs score,
// softmax and values in turn; the packed codes of chunk c+1 load while chunk c
// computes and page ids run two chunks ahead.
template <int BWK, int BWV, int NG>
__device__ __forceinline__ void scan_range(const DecodeArgs& a, int b, int kvh, int t_lo, int t_hi, int64_t prow,
                                           int lane, Tab<BWK>& cbk, Tab<BWV>& cbv, float* ptile) {
  constexpr int D = 128;
  const int page_hi = (t_hi + (1 << a.log2S) - 1) >> a.log2S;
  const int n = (t_hi - t_lo + 63) >> 6;

  // register m of group g of lane 4j+i holds q_rot[head 4g+i][16m + j]
  float qb[NG][8];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const float* qp = a.q_rot + ((int64_t(b) * a.Hkv + kvh) * (4 * NG) + 4 * g + (lane & 3)) * D + (lane >> 2);
#pragma unroll
    for (int m = 0; m < 8; ++m) qb[g][m] = qp[16 * m];
  }
  const int32_t* trow = a.table + b * a.tsb;
  // page of this lane's token in chunk c (tokens past the range read its last page and are masked)
  auto pid_of = [&](int c) {
    const int col = min((t_lo + 64 * c + lane) >> a.log2S, page_hi - 1);
    return trow[col];
  };

  RowState<NG> st;
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) st.acc[g][mm] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4 * NG; ++i) {
    st.m[i] = -INFINITY;
    st.l[i] = 0.f;
  }
  using Buf = RowBuf<BWK, BWV>;
  // Chunk c with its K rows in X and its V codes in Y; Z is free. The K rows of
  // chunk c+1 load into Z at the start, its V codes into X once the softmax has
  // read the norms, so each load has about one chunk of compute to land, and
  // three buffers rotate through the roles: (X, Y, Z) -> (Z, X, Y).
  int pid_next;
  auto step = [&](int c, Buf& X, Buf& Y, Buf& Z) {
    const int c0 = t_lo + 64 * c;
    // page ids two chunks ahead, issued before the next chunk's rows, so the wait
    // for them never waits for those rows; clamped, so always a valid read
    const int pid_after = pid_of(c + 2);
    const bool more = c + 1 < n;
    if (more) load_k(a, kvh, lane, c0 + 64, pid_next, Z);
    float vv[3][8];
    f32x4 s[NG];
    score_phase<BWK, NG>(X.w, cbk, qb, s);
    value_prime<BWV>(Y.w, cbv, vv);
    softmax_phase<NG>(s, X.w[Buf::KW], X.w[Buf::KW + 1], c0 + lane < t_hi, lane, ptile, st);
    if (more) load_v(a, kvh, lane, c0 + 64, pid_next, X);
    value_phase<BWV, NG>(Y.w, cbv, ptile, lane, st.acc, vv);
    pid_next = pid_after;
  };

  Buf b0, b1, b2;
  load_k(a, kvh, lane, t_lo, pid_of(0), b0);
  load_v(a, kvh, lane, t_lo, pid_of(0), b1);
  pid_next = pid_of(1);
  // The prologue's loads land before the loop: the compiler's wait analysis then
  // sees nothing outstanding at the loop head, so no wait inside the body covers
  // a load issued for a later chunk.
  wait_vmem_all();
  for (int c = 0; c < n; c += 3) {
    step(c, b0, b1, b2);
    if (c + 1 >= n) break;
    step(c + 1, b2, b0, b1);
    if (c + 2 >= n) break;
    step(c + 2, b1, b2, b0);
  }
  write_partial(a, st, prow, lane);
}

// LDS of a work-group of WPB waves: the codebook tables (a replicated pair table
// first, at a 64 KB slot, so that its address registers need no base add), then
// one p tile per wave.
template <int BWK, int BWV, int NG, int WPB>
struct RowsLds {
  static constexpr int k_off = (BWK == 4 || BWV != 4) ? 0 : kPairTableBytes;
  static constexpr int v_off = BWV == 4 ? (BWK == 4 ? kPairTableBytes : 0) : (BWK == 4 ? kPairTableBytes
                                                                                      : table_bytes<BWK>());
  static constexpr int k_slot = k_off >> 16, v_slot = v_off >> 16;
  static constexpr int tiles = (BWK == 4 && BWV != 4) ? v_off + table_bytes<BWV>()
                               : (BWV == 4 && BWK != 4) ? k_off + table_bytes<BWK>()
                                                        : v_off + table_bytes<BWV>();
  static constexpr int tile_bytes = NG * 16 * kPStride * 4;
  static constexpr int total = tiles + WPB * tile_bytes;
  static_assert(total <= 160 * 1024, "LDS of a work-group exceeds 160 KB");
};

template <int BW>
__device__ __forceinline__ Tab<BW> make_tab(const char* lds, int off, int lane) {
  Tab<BW> t;
  if constexpr (BW == 4) t.init(lds, off >> 16, lane);
  else t.t = reinterpret_cast<const float*>(lds + off);
  return t;
}

// Logical index of work-group p of n when groups go to the 8 XCDs round robin:
// XCD x holds groups x, x+8, ...; they become a contiguous run of logical indices.
__device__ __forceinline__ int xcd_major(int p, int n) {
  const int q = n >> 3, r = n & 7, x = p & 7, s = p >> 3;
  return x * q + min(x, r) + s;
}

// Work-group of WPB independent waves sharing the codebook tables; wave w =
// blockIdx.x * WPB + wave-in-group.
// Fixed splits: wave w is unit (split, kv head, sequence) of the flattened
// num_splits x Hkv x B space and scans pages [split * pages_per_split, ...) of its
// sequence.
// Balanced (a.balanced): the W = num_splits waves share the flattened space of
// 64-token chunks ordered (sequence, kv head, chunk); wave w takes chunks
// [C w / W', C (w+1) / W') with C the total and W' = min(W, C), and writes one
// partial per (sequence, kv head) it touches, at row w + b*Hkv + kvh.
template <int BWK, int BWV, int NG, int WPB>
__global__ __launch_bounds__(64 * WPB) void decode_rows_kernel(DecodeArgs a) {
  using Lay = RowsLds<BWK, BWV, NG, WPB>;
  __shared__ __align__(16) char lds[Lay::total];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  stage_table<BWK>(a.cb_k, lds + Lay::k_off, tid, 64 * WPB);
  stage_table<BWV>(a.cb_v, lds + Lay::v_off, tid, 64 * WPB);
  __syncthreads();  // the only block-wide barrier: waves run independently from here
  // Work-groups are dealt to the eight XCDs round robin (group p on XCD p % 8); the
  // logical group index gives each XCD a contiguous stretch of the flattened work,
  // so the kv heads of a sequence run on one XCD and share the 128-byte lines that
  // hold their norms in its L2.
  const int64_t w = int64_t(xcd_major(blockIdx.x, gridDim.x)) * WPB + wig;
  float* ptile = reinterpret_cast<float*>(lds + Lay::tiles + wig * Lay::tile_bytes);

  // The work list: one (sequence, kv head, token range) for a fixed split, or the
  // units overlapping this wave's share of the flattened chunk space. One call site
  // for the scan keeps a single copy of its code.
  int b, kvh, t_lo, t_hi;
  int64_t prow;
  int64_t s = 0, e = 0;  // balanced: flattened chunks [s, e) still to do
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
    if (page_lo >= n_pages) return;  // wave-uniform: this split is past the sequence
    const int page_hi = min(page_lo + a.pages_per_split, n_pages);
    t_lo = page_lo << a.log2S;
    t_hi = min(page_hi << a.log2S, L);
    prow = (int64_t(b) * a.Hkv + kvh) * a.num_splits + split;
    if (split == 0 && lane == 0)  // the merge reads the group's partial rows from here
      a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), (n_pages + a.pages_per_split - 1) / a.pages_per_split);
  } else {
    const int64_t C = int64_t(a.Hkv) * pre[a.B];
    const int64_t Wp = min(int64_t(a.num_splits), C);
    if (w >= Wp) return;
    s = C * w / Wp;
    e = C * (w + 1) / Wp;
    // sequence holding flattened chunk s: the largest b with Hkv * pre[b] <= s
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
  Tab<BWK> cbk = make_tab<BWK>(lds, Lay::k_off, lane);
  Tab<BWV> cbv = make_tab<BWV>(lds, Lay::v_off, lane);

  while (true) {
    int nb = 0, c_hi = 0;
    if (a.balanced) {
      nb = pre[b + 1] - pre[b];
      while (nb == 0) {  // sequences without tokens own no chunks
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
        // the group's first wave: its partials are rows prow .. prow + n - 1, one per
        // wave up to the last wave starting before the group's end U1
        const int64_t C = int64_t(a.Hkv) * pre[a.B];
        const int64_t Wp = min(int64_t(a.num_splits), C);
        const int64_t U1 = base + int64_t(kvh + 1) * nb;
        const int64_t wl = (U1 * Wp + C - 1) / C - 1;
        a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), int(wl - w + 1));
      }
      s += c_hi - c_lo;
    }
    scan_range<BWK, BWV, NG>(a, b, kvh, t_lo, t_hi, prow, lane, cbk, cbv, ptile);
    if (!a.balanced || s >= e) break;
    if (kvh + 1 == a.Hkv && c_hi == nb) ++b;
  }
}

// Waves per work-group: three per SIMD where the scan fits in 168 VGPRs, else two.
template <int BWK, int BWV, int NG>
constexpr int rows_wpb() { return NG == 1 && BWK <= 4 && BWV <= 4 ? 12 : 8; }

template <int BWK, int BWV, int NG>
SplitKernel rows_kernel() {
  constexpr int wpb = rows_wpb<BWK, BWV, NG>();
  SplitKernel k;
  k.fn = decode_rows_kernel<BWK, BWV, NG, wpb>;
  k.block = 64 * wpb;
  k.wpb = wpb;
  k.nrep = 4 * NG;
  k.log2_units = true;
  k.rows = true;
  return k;
}

template <int NG>
SplitKernel rows_for(int bw_k, int bw_v) {
  if (bw_k == bw_v) {
    switch (bw_k) {
      case 2: return rows_kernel<2, 2, NG>();
      case 3: return rows_kernel<3, 3, NG>();
      case 4: return rows_kernel<4, 4, NG>();
      case 5: return rows_kernel<5, 5, NG>();
      case 6: return rows_kernel<6, 6, NG>();
      case 8: return rows_kernel<8, 8, NG>();
    }
  } else if (bw_k == 4 && bw_v == 6) {
    return rows_kernel<4, 6, NG>();
  } else if (bw_k == 6 && bw_v == 4) {
    return rows_kernel<6, 4, NG>();
  } else if (bw_k == 4 && bw_v == 8) {
    return rows_kernel<4, 8, NG>();
  }
  return SplitKernel{};
}

}  // namespace

SplitKernel pick_split_rows(int bw_k, int bw_v, int n_rep) {
  if (n_rep <= 4) return rows_for<1>(bw_k, bw_v);
  if (n_rep <= 8) return rows_for<2>(bw_k, bw_v);
  return SplitKernel{};
}

}  // namespace wn
