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
#include <cstdlib>
#include <cstring>
#include <utility>

#include "wn_decode.h"
#include "wn_tables.h"

namespace wn {
namespace {



constexpr float kRescale = 8.0f;
constexpr int kPStride = 20;  // floats per (head, token group) row of the p tile (16 + pad, 16-B rows)

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
template <int BW, int NTHR>
__device__ __forceinline__ void stage_table(const float* cb, char* dst, int tid) {
  if constexpr (BW == 4) {
    float2* t = reinterpret_cast<float2*>(dst);
    for_strided<256 * 32, NTHR>(tid, [&](int i) {
      const int b = i >> 5;
      t[i] = make_float2(cb[b & 15], cb[b >> 4]);
    });
  } else if constexpr (pair_coded<BW>()) {
    float2* t = reinterpret_cast<float2*>(dst);
    for_strided<(1 << (2 * BW)), NTHR>(tid, [&](int i) { t[i] = make_float2(cb[i & ((1 << BW) - 1)], cb[i >> BW]); });
  } else {
    float* t = reinterpret_cast<float*>(dst);
    for_strided<(1 << BW), NTHR>(tid, [&](int i) { t[i] = cb[i]; });
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
//
// RAW (5 and 6 bits only): the 8 bytes from p, which the caller has rounded down to 4
// bytes, one dwordx2 load, left unshifted; raw_shift gives the bit offset of the codes
// in them and unshift_raw moves them down (done where the words are used, so no wait
// for the load is needed right after it). The window ends at most at the end of the lane's
// 16-token page block (p + BWV <= block end and 8 bytes from the rounded-down start
// reach at most 3 bytes past p + 5).
template <int BWV>
__device__ __forceinline__ uint32_t raw_shift(int lane) { return 8u * uint32_t((BWV * (lane & 15)) & 3); }
__device__ __forceinline__ void unshift_raw(uint32_t& w0, uint32_t& w1, uint32_t sh) {
  w0 = __builtin_amdgcn_alignbit(w1, w0, sh);
  w1 >>= sh;
}

template <int BWV, bool RAW = false>
__device__ __forceinline__ void load_vcodes(const uint8_t* p, bool odd_lane, uint32_t (&out)[VWords<BWV>::N]) {
  if constexpr (RAW) {
    static_assert(BWV == 5 || BWV == 6, "raw windows are for 5 and 6-bit rows");
    // p is already rounded down to 4 bytes (load_v rounds the lane's offset)
    uint2 x;
    __builtin_memcpy(&x, __builtin_assume_aligned(p, 4), 8);
    out[0] = x.x;
    out[1] = x.y;
  } else if constexpr (BWV == 4) {
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

// A page-block address formed on the device (block_bases) as a pointer into global memory: the address space is
// stated, so loads through it stay global loads (a plain pointer rebuilt from an integer
// would make them flat loads, which also count against the LDS wait counter).
typedef __attribute__((address_space(1))) const uint8_t global_u8;
__device__ __forceinline__ const uint8_t* global_ptr(uint64_t x) {
  return (const uint8_t*)(global_u8*)(x);
}

// V side of chunk [c0, c0+64): for every token quad q the BWV bytes of codes
// 8p..8p+7 of token c0+4q+G (G = lane/16, p = lane%16). c0 is a multiple of 16 and
// pages hold >= 16 tokens, so the four quads of 16-token block j share the page of
// lane 16j (pid_lane is the page of token c0+lane).
template <int BWK, int BWV, bool RAW = false>
__device__ __forceinline__ void load_v(const DecodeArgs& a, int kvh, int lane, int c0, int pid_lane,
                                       RowBuf<BWK, BWV>& r, bool live = true, const uint64_t* ba = nullptr) {
  constexpr int NBV = 16 * BWV, VW = RowBuf<BWK, BWV>::VW;
  const int smask = (1 << a.log2S) - 1;
  const int p = lane & 15;
  // live == false (a chunk past the range, loaded only so that every path of the
  // scan loop issues the same loads): every lane reads the first bytes of the block
  // (RAW: rounded down to 4 bytes; page blocks are 8-byte aligned, so the windows are)
  const uint32_t lane_off = live ? uint32_t((lane >> 4) * NBV + BWV * p) & (RAW ? ~3u : ~0u) : 0u;
  static_for<0, 4>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const uint8_t* blk;
    if (ba) {  // the block's address, formed by block_bases
      blk = global_ptr(ba[j]);
    } else {
      const uint32_t pid_j = __builtin_amdgcn_readlane(pid_lane, 16 * j);  // a live page id, >= 0
      blk = a.v_pages + uint64_t(pid_j) * uint64_t(a.vsp) + (kvh >> a.kvshift) * a.vsh +
            uint32_t((c0 + 16 * j) & smask) * uint32_t(NBV);
    }
    const uint8_t* vj = blk + lane_off;
    static_for<0, 4>([&](auto qc) {
      constexpr int qq = decltype(qc)::value;
      uint32_t t[VW];
      load_vcodes<BWV, RAW>(vj + 4 * qq * NBV, p & 1, t);
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

// LDS of a work-group of WPB waves: the codebook tables (a replicated 4-bit pair table
// at a 64 KB slot, so that its address registers need no base add), then one p tile
// per wave.
template <int BWK, int BWV, int NG, int WPB>
struct RowsLds {
  // A 4-bit table takes a 64 KB slot of its own: its address registers carry the slot.
  // Beside a pair-coded table (2, 3, 5, 6 bits) it takes slot 1 and the pair table
  // offset 0, where its entry offsets (below 64 KB) need no base added: the read's
  // 16-bit offset field cannot hold a base of 64 KB, which would cost an add per lookup.
  static constexpr bool k4 = BWK == 4, v4 = BWV == 4;
  static constexpr int k_off = k4 ? (pair_coded<BWV>() ? kPairTableBytes : 0)
                                  : (v4 && !pair_coded<BWK>() ? kPairTableBytes : 0);
  static constexpr int v_off = v4 ? (k4 || pair_coded<BWK>() ? kPairTableBytes : 0)
                                  : (k4 ? (pair_coded<BWV>() ? 0 : kPairTableBytes) : table_bytes<BWK>());
  static constexpr int k_slot = k_off >> 16, v_slot = v_off >> 16;
  static constexpr int tiles = k_off + table_bytes<BWK>() > v_off + table_bytes<BWV>() ? k_off + table_bytes<BWK>()
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

// The work list of wave w, one scan(b, kvh, t_lo, t_hi, prow, left) call per
// (sequence, kv head, token range) it owns; left = the wave's chunks after the range.
// Fixed splits: wave w is unit (split, kv head, sequence) of the flattened
// num_splits x Hkv x B space and scans pages [split * pages_per_split, ...) of its
// sequence.
// Balanced (a.balanced), grouped (at least Hkv waves): the waves form G = W / Hkv
// groups of Hkv consecutive waves, wave w = j Hkv + h being kv head h of group j.
// The groups share the flattened space of 64-token chunks of one kv head, ordered
// (sequence, chunk), T in all: group j takes [T j / G', T (j+1) / G') with G' =
// min(G, T), and each of its waves scans that range for its own kv head. So the kv
// heads of a chunk are scanned side by side by the waves of one work-group, and the
// 128-byte lines that hold the norms of four kv heads of a page are fetched once
// for all four, whatever the sequence lengths. The wave writes one partial per
// sequence it touches, at row h (G' + B) + b + j: a unit's rows are contiguous (its
// groups are consecutive) and no two (group, sequence) pairs of one kv head share a
// row (j + b grows with either).
// Balanced over fewer waves than kv heads: the waves share the flattened space
// ordered (sequence, kv head, chunk); wave w takes chunks [C w / W', C (w+1) / W')
// with C the total and W' = min(W, C), and writes one partial per (sequence, kv
// head) it touches, at row w + b*Hkv + kvh.
// Either way the wave that scans a unit's first chunk records where the unit's
// partials start and how many there are (unit_meta), so the merge reads exactly that
// range.
// The walk is split in two: init() finds the wave's first range (the plan's lookups
// and divisions, which a kernel can run while its tables load) and run() scans the
// ranges one call site at a time (one copy of the scan's code).
struct RangeWalk {
  int b = 0, kvh = 0, t_lo = 0, t_hi = 0;
  int64_t prow = 0;
  int64_t s = 0, e = 0;  // balanced: flattened chunks [s, e) still to do
  int64_t G = 0, j = 0;  // grouped: groups with work, this wave's group
  bool grouped = false;

  // The chunk prefix and the lengths do not change while a scan runs (the rotate
  // launch writes the prefix before it): const_view makes their reads scalar loads.
  // false: the wave has no work
  __device__ __forceinline__ bool init(const DecodeArgs& a, int64_t w, int lane) {
    const auto* pre = const_view(a.chunk_prefix);
    const auto* seq_lens = const_view(a.seq_lens);
    grouped = a.balanced && a.num_splits >= a.Hkv;
    if (!a.balanced) {
      if (w >= int64_t(a.num_splits) * a.Hkv * a.B) return false;
      const int split = int(w % a.num_splits);
      kvh = int((w / a.num_splits) % a.Hkv);
      b = int(w / (int64_t(a.num_splits) * a.Hkv));
      const int L = seq_lens[b];
      const int S = 1 << a.log2S;
      const int n_pages = (L + S - 1) >> a.log2S;
      const int page_lo = split * a.pages_per_split;
      if (page_lo >= n_pages) return false;  // wave-uniform: this split is past the sequence
      const int page_hi = min(page_lo + a.pages_per_split, n_pages);
      t_lo = page_lo << a.log2S;
      t_hi = min(page_hi << a.log2S, L);
      prow = (int64_t(b) * a.Hkv + kvh) * a.num_splits + split;
      if (split == 0 && lane == 0)  // the merge reads the group's partial rows from here
        a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), (n_pages + a.pages_per_split - 1) / a.pages_per_split);
    } else {
      const int64_t T = pre[a.B];
      int64_t key;  // the flattened position to find the sequence of, in units of pre[]
      int64_t mult; // pre[] -> flattened position
      if (grouped) {
        G = min(int64_t(a.num_splits / a.Hkv), T);
        j = w / a.Hkv;
        if (j >= G) return false;
        s = T * j / G;
        e = T * (j + 1) / G;
        key = s;
        mult = 1;
        kvh = int(w % a.Hkv);
      } else {
        const int64_t C = int64_t(a.Hkv) * T;
        const int64_t Wp = min(int64_t(a.num_splits), C);
        if (w >= Wp) return false;
        s = C * w / Wp;
        e = C * (w + 1) / Wp;
        key = s;
        mult = a.Hkv;
        kvh = 0;
      }
      // sequence holding flattened chunk s: the largest b with mult * pre[b] <= s
      int lo = 0, hi = a.B;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (mult * pre[mid] <= key) lo = mid;
        else hi = mid;
      }
      b = lo;
      t_lo = t_hi = 0;
      prow = 0;
    }
    return true;
  }

  template <class Scan>
  __device__ __forceinline__ void run(const DecodeArgs& a, int64_t w, int lane, Scan&& scan) {
    const auto* pre = const_view(a.chunk_prefix);
    const auto* seq_lens = const_view(a.seq_lens);
    while (true) {
      int nb = 0, c_hi = 0;
      if (grouped) {
        nb = pre[b + 1] - pre[b];
        while (nb == 0) {  // sequences without tokens own no chunks
          ++b;
          nb = pre[b + 1] - pre[b];
        }
        const int c_lo = int(s - pre[b]);
        c_hi = int(min(int64_t(nb), c_lo + (e - s)));
        t_lo = 64 * c_lo;
        t_hi = min(64 * c_hi, seq_lens[b]);
        prow = int64_t(kvh) * (G + a.B) + b + j;
        if (c_lo == 0 && lane == 0) {
          // the unit's first group: its partials are rows prow .. prow + n - 1, one per
          // group up to the last group starting before the sequence's end pre[b + 1]
          const int64_t T = pre[a.B];
          const int64_t jl = (int64_t(pre[b + 1]) * G + T - 1) / T - 1;
          a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), int(jl - j + 1));
        }
        s += c_hi - c_lo;
      } else if (a.balanced) {
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
        t_hi = min(64 * c_hi, seq_lens[b]);
        prow = w + int64_t(b) * a.Hkv + kvh;
        if (c_lo == 0 && lane == 0) {
          // the unit's first wave: its partials are rows prow .. prow + n - 1, one per
          // wave up to the last wave starting before the unit's end U1
          const int64_t C = int64_t(a.Hkv) * pre[a.B];
          const int64_t Wp = min(int64_t(a.num_splits), C);
          const int64_t U1 = base + int64_t(kvh + 1) * nb;
          const int64_t wl = (U1 * Wp + C - 1) / C - 1;
          a.unit_meta[b * a.Hkv + kvh] = make_int2(int(prow), int(wl - w + 1));
        }
        s += c_hi - c_lo;
      }
      scan(b, kvh, t_lo, t_hi, prow, uint32_t(a.balanced ? e - s : 0));
      if (!a.balanced || s >= e) break;
      if (grouped) ++b;  // the group's range continues in the next sequence
      else if (kvh + 1 == a.Hkv && c_hi == nb) ++b;
    }
  }
};

template <class Scan>
__device__ __forceinline__ void for_each_range(const DecodeArgs& a, int64_t w, int lane, Scan&& scan) {
  RangeWalk rw;
  if (rw.init(a, w, lane)) rw.run(a, w, lane, scan);
}

// Work-group of WPB independent waves sharing the codebook tables; wave w =
// blockIdx.x * WPB + wave-in-group walks the work list of for_each_range.
template <int BWK, int BWV, int NG, int WPB>
__global__ __launch_bounds__(64 * WPB) void decode_rows_kernel(DecodeArgs a) {
  using Lay = RowsLds<BWK, BWV, NG, WPB>;
  __shared__ __align__(16) char lds[Lay::total];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  stage_table<BWK, 64 * WPB>(a.cb_k, lds + Lay::k_off, tid);
  stage_table<BWV, 64 * WPB>(a.cb_v, lds + Lay::v_off, tid);
  __syncthreads();  // the only block-wide barrier: waves run independently from here
  // Work-groups are dealt to the eight XCDs round robin (group p on XCD p % 8); the
  // logical group index gives each XCD a contiguous stretch of the flattened work,
  // so the kv heads of a sequence run on one XCD and share the 128-byte lines that
  // hold their norms in its L2.
  const int64_t w = int64_t(xcd_major(blockIdx.x, gridDim.x)) * WPB + wig;
  float* ptile = reinterpret_cast<float*>(lds + Lay::tiles + wig * Lay::tile_bytes);
  Tab<BWK> cbk = make_tab<BWK>(lds, Lay::k_off, lane);
  Tab<BWV> cbv = make_tab<BWV>(lds, Lay::v_off, lane);
  for_each_range(a, w, lane, [&](int b, int kvh, int t_lo, int t_hi, int64_t prow, uint32_t) {
    scan_range<BWK, BWV, NG>(a, b, kvh, t_lo, t_hi, prow, lane, cbk, cbv, ptile);
  });
}

// ------------------------------------------------------------------ 16-bit matrix-core scan
//
// The page scan on v_mfma_f32_16x16x32_f16 (16 times the MAC rate of the fp32 4x4x1
// MFMA on gfx950), for 2, 3, 4, 5 and 6-bit codes. Every fp32 factor x is carried as
// an fp16 pair x = H + L (H = fp16(x), L = fp16(x - H)) after an exact power-of-two
// scaling that keeps both in fp16's normal range; products of fp16 values are exact
// in the fp32 accumulators and each factor keeps 22 bits, so scores and values keep
// fp32 accuracy.
//
// A codebook table entry holds (H, L) of 2^8 c for each of its two codes,
// [H0, L0, H1, L1]; two entries loaded side by side are an 8-slot MFMA operand, and
// the other operand carries its factor twice per code ([f0, f0, f1, f1, ...]), so
// the k-slots pair each code's H and L with the same factor. Lane l = 16g + c.
//
//   scores   tile r (tokens 16r .. 16r+15 of the chunk) x 16 columns x 32 k-slots
//            per MFMA. Row c of
//            lane 16g+c is token 16r + 4(c%4) + c/4; its k-slots in K-step s are dims
//            32g + 4s .. +3, so a lane reads the 16-byte quarter g of one token row and
//            one load instruction reads a whole 16-token page block. Column c is head
//            c % NH of the group and the H (c < NH) or L (c >= NH) part of q' = q 2^e
//            (e per (sequence, kv head), |q'| < 2^15); with four heads the columns
//            8..15 are zero. 8 K-steps x 4 tiles = 32 MFMAs per chunk. Output lane
//            16g+c register i holds token 16r + 4i + g of column c.
//   softmax  the two column halves are added (row rotate by NH), the scores pass
//            through a per-wave LDS tile to lane = token, and the online softmax runs as
//            in the fp32 scan. p n_V 2^-gs goes back to the same tile as H | L << 16
//            words.
//   values   M-tile mt: row c of lane 16g+c is dim 8c + mt, so a lane needs codes
//            8c..8c+7 of each token: the V loads of the fp32 scan, unchanged. K-step ks:
//            k-slots of group g are tokens 16ks + 4j + g, j = 0..3; the codes of dim
//            8c + mt of tokens (j = 0, 1) and (2, 3) are merged into pair indices (4-bit:
//            a bit-field insert per four dims), whose entries form the A operand. B =
//            H or L of p n_V 2^-gs of the column's head for those tokens. 8 x 4 = 32 MFMAs
//            per chunk; output lane 16g+c register i holds dim 32g + 8i + mt, column c.
//   scales   scores are multiplied by 2^-(e+8) before the softmax; pv' = p n_V 2^-gs
//            with gs the smallest shift that keeps 256 max(n_V) 2^-gs < 2^15 (raised,
//            with an exact rescale of the accumulators, when a chunk needs it); the
//            partials are multiplied by 2^(gs-8) when written.

// One head group: the score tile keeps both column halves (q' H and L parts) and the
// softmax adds them as it reads (four adds per lane) instead of a row rotate and add
// on the sixteen output registers; two groups keep the rotate, for LDS room.
template <int NG>
constexpr bool kTileHalves = NG == 1;
template <int BWV>
constexpr bool kRawV = BWV == 5 || BWV == 6;  // V rows loaded as raw windows (load_vcodes)
constexpr int kTileStride = 80;     // words per head in the per-wave score / p n_V tile

// Maximum over the wave, in a scalar register, with DPP moves only (no LDS permutes):
// row reductions, then the row broadcasts into lane 63. The reduction runs on
// unsigned keys (0 is the identity, so lanes a row mask leaves out keep 0 and each
// move folds into its max as one DPP instruction).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t x) {
  return max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, ROWS, 0xf, false)));
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t x) {
  x = dpp_umax<0xb1, 0xf>(x);   // quad_perm [1,0,3,2]
  x = dpp_umax<0x4e, 0xf>(x);   // quad_perm [2,3,0,1]
  x = dpp_umax<0x141, 0xf>(x);  // row_half_mirror
  x = dpp_umax<0x140, 0xf>(x);  // row_mirror
  x = dpp_umax<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
  x = dpp_umax<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
  return uint32_t(__builtin_amdgcn_readlane(int(x), 63));
}
// Non-negative floats order as their bit patterns.
__device__ __forceinline__ float wave_max_nonneg(float x) {
  return __builtin_bit_cast(float, wave_umax(__builtin_bit_cast(uint32_t, x)));
}
// Any float but NaN: the key flips every bit of a negative value and the sign bit of
// a non-negative one, which orders keys as the floats.
__device__ __forceinline__ float wave_max_dpp(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  const uint32_t k = wave_umax(b ^ (uint32_t(int32_t(b) >> 31) | 0x80000000u));
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// Tile words read by every lane whether or not its token is valid: the empty asm uses
// each value unconditionally, so the compiler cannot sink a read into a branch on
// `valid` (it had: one exec-masked branch per head around a read and a full LDS wait,
// eight serialised round trips per chunk with two head groups).
template <int N>
__device__ __forceinline__ void read_unconditionally(float (&x)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(x[i]));
}

// H | L << 16 of x with H = fp16(x) and L = fp16(x - H), both rounded toward zero.
__device__ __forceinline__ uint32_t split_word(float x) {
  typedef __fp16 h2 __attribute__((ext_vector_type(2)));
  const h2 hi = __builtin_amdgcn_cvt_pkrtz(x, 0.f);
  const float r = x - (float)hi[0];
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, r));
}

// Table entry of two codebook values: [H(2^8 lo), L(2^8 lo), H(2^8 hi), L(2^8 hi)].
__device__ __forceinline__ uint2 split_pair(float lo, float hi) {
  return make_uint2(split_word(lo * kCbScale), split_word(hi * kCbScale));
}

// The pair tables of stage_table with 16-bit split entries (4-bit: replicated and
// byte-indexed; 2, 3, 5, 6 bits: 2^(2 BW) entries).
template <int BW>
constexpr int table16_entries() { return BW == 4 ? 256 * 32 : 1 << (2 * BW); }
// codes of entry i: 4-bit, byte i >> 5 (lane copy i & 31); else a code pair
template <int BW>
__device__ __forceinline__ int2 table16_codes(int i) {
  if constexpr (BW == 4) return make_int2((i >> 5) & 15, i >> 9);
  else return make_int2(i & ((1 << BW) - 1), i >> BW);
}
template <int BW, int NTHR>
using Table16Loads = CodePairs<table16_entries<BW>(), NTHR>;
template <int BW, int NTHR>
__device__ __forceinline__ Table16Loads<BW, NTHR> load_table16(const float* cb, int tid) {
  static_assert(BW == 4 || pair_coded<BW>(), "16-bit tables are pair tables");
  return load_code_pairs<table16_entries<BW>(), NTHR>(cb, tid, [](int i) { return table16_codes<BW>(i); });
}
template <int BW, int NTHR>
__device__ __forceinline__ void store_table16(const Table16Loads<BW, NTHR>& p, char* dst, int tid) {
  store_code_pairs(p, reinterpret_cast<uint2*>(dst), tid, [](float lo, float hi) { return split_pair(lo, hi); });
}

// Table reads in flight ahead of their MFMA in the 16-bit scan: eight steps where
// the widths leave the registers for them (2 and 4 bits, whose pieces are whole
// bytes), two with a 6-bit side (its kernels sit at 256 VGPRs; fewer reads in flight
// measured 2 % faster at config 5), else four.
template <int BWK, int BWV>
constexpr int mx_lookahead() {
  return (BWK == 2 || BWK == 4) && (BWV == 2 || BWV == 4) ? 8 : (BWK == 6 || BWV == 6) ? 2 : 4;
}

// Two table entries side by side as an 8-slot operand.
__device__ __forceinline__ h8 as_h8(uint2 a, uint2 b) { return __builtin_bit_cast(h8, u32x4{a.x, a.y, b.x, b.y}); }

// [x, x, y, y, z, z, w, w] of the halves picked by sel from four H | L words
// (sel 0x01000100: H; 0x03020302: L; 0x0c0c0c0c: zeros).
__device__ __forceinline__ h8 dup4(uint32_t x, uint32_t y, uint32_t z, uint32_t w, uint32_t sel) {
  return __builtin_bit_cast(h8, u32x4{__builtin_amdgcn_perm(x, x, sel), __builtin_amdgcn_perm(y, y, sel),
                                      __builtin_amdgcn_perm(z, z, sel), __builtin_amdgcn_perm(w, w, sel)});
}

// Table entry of the 4-bit pair held in byte K of x (SDWA address move, as lookup8).
template <int K>
__device__ __forceinline__ uint2 entry4(Tab<4>& tab, uint32_t x) {
  tab.r[K] = put_byte1<K>(tab.r[K], x);
  return *reinterpret_cast<const uint2*>(tab.lds + tab.r[K]);
}

template <int BW>
__device__ __forceinline__ uint2 pair_entry(const Tab<BW>& tab, uint32_t off) {
  return *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(tab.t) + off);
}

// Table entry of pair N (codes 2N, 2N+1) of a packed piece held as words.
template <int BW, int N>
__device__ __forceinline__ uint2 piece_pair(const uint32_t* w, Tab<BW>& tab) {
  if constexpr (BW == 4) return entry4<N & 3>(tab, w[N >> 2]);
  else return pair_entry<BW>(tab, pair_offset<BW, 2 * BW * N>(w));
}

// Pair indices of the value phase combine one dim of two tokens A and B (A's code
// low). Before the phase, each token pair's words are rewritten in place (A's slot,
// B's slot) = (Ce, Co): Ce holds A's even-numbered codes with B's codes shifted up
// one field into the gaps, Co the same for the odd ones, so the index of dim m is the
// 2 BW bits of Ce (m even) or Co (m odd) from bit BW m, and each lookup costs two
// instructions (pair_offset). RAW windows are unshifted on the way.
template <int BWK, int BWV>
__device__ __forceinline__ void merge_value_pairs(RowBuf<BWK, BWV>& V, int lane) {
  constexpr int VW = VWords<BWV>::N;
  constexpr uint64_t E = field_mask<BWV>(0), O = field_mask<BWV>(1);
  [[maybe_unused]] uint32_t sh = 0;
  if constexpr (kRawV<BWV>) sh = raw_shift<BWV>(lane);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    uint32_t* a = V.w + (2 * q) * VW;
    uint32_t* b = V.w + (2 * q + 1) * VW;
    if constexpr (VW == 1) {
      const uint32_t bs = b[0] << BWV;
      const uint32_t ce = bitsel(uint32_t(E), a[0], bs);
      b[0] = bitsel(uint32_t(O), a[0], bs);
      a[0] = ce;
    } else {
      if constexpr (kRawV<BWV>) {
        unshift_raw(a[0], a[1], sh);
        unshift_raw(b[0], b[1], sh);
      }
      const uint32_t bs0 = b[0] << BWV, bs1 = __builtin_amdgcn_alignbit(b[1], b[0], 32 - BWV);
      const uint32_t e0 = bitsel(uint32_t(E), a[0], bs0);
      const uint32_t e1 = bitsel(uint32_t(E >> 32), a[1], bs1);
      b[0] = bitsel(uint32_t(O), a[0], bs0);
      b[1] = bitsel(uint32_t(O >> 32), a[1], bs1);
      a[0] = e0;
      a[1] = e1;
    }
  }
}

// The 16-bit scan keeps its rows in RowBuf words too. As a K buffer: for each tile
// t, the 4 BWK bytes of quarter g of token 16t + 4(c%4) + c/4 (words [t*BWK, t*BWK +
// BWK)), then the fp16 K and V norms of token c0 + lane (words KW, KW+1). As a V
// buffer: the layout of the fp32 scan.

// Token (within its 16-token tile) whose scores row c of a score MFMA holds.
__device__ __forceinline__ int tile_token(int c) { return 4 * (c & 3) + (c >> 2); }

// Byte addresses of the four 16-token page blocks of the chunk that starts at token c0
// (a multiple of 16): each lane forms the address of its own token's block with two
// 64-bit multiply-adds (page id x page stride, slot x row bytes; base = the pages plus
// the kv head's offset) and the blocks' addresses are read from lanes 0, 16, 32 and 48.
// Page strides are below 2^32 bytes (checked on the host).
template <int NB>
__device__ __forceinline__ void block_bases(uint64_t base, uint32_t sp, int pid, int c0, int lane, int smask,
                                            uint64_t (&out)[4]) {
  const uint32_t slot = uint32_t((c0 + lane) & smask) & ~15u;
  const uint64_t x = base + uint64_t(uint32_t(pid)) * sp + uint64_t(slot * uint32_t(NB));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = __builtin_amdgcn_readlane(uint32_t(x), 16 * t);
    const uint32_t hi = __builtin_amdgcn_readlane(uint32_t(x >> 32), 16 * t);
    out[t] = uint64_t(hi) << 32 | lo;
  }
}

// K side of chunk [c0, c0+64) for the 16-bit scan: quarter g of the rows of the
// tile tokens (one whole 16-token page block per load instruction) and both norms of
// token c0 + lane, whose page is pid_lane.
template <int BWK, int BWV>
__device__ __forceinline__ void load_k16(const DecodeArgs& a, int kvh, int lane, int c0, int pid_lane,
                                         RowBuf<BWK, BWV>& r, bool live = true, const uint64_t* ba = nullptr) {
  constexpr int NBK = 16 * BWK, QB = 4 * BWK, QW = BWK, KW = RowBuf<BWK, BWV>::KW;
  const int smask = (1 << a.log2S) - 1;
  // the tile's 16 tokens share a page (c0 + 16t is a multiple of 16 and S >= 16): a
  // wave-uniform block base plus this lane's fixed 32-bit offset in it (0 when the
  // chunk is past the range, as in load_v)
  const uint32_t lane_off = live ? uint32_t(tile_token(lane & 15) * NBK + QB * (lane >> 4)) : 0u;
  static_for<0, 4>([&](auto rc) {
    constexpr int t = decltype(rc)::value;
    const uint8_t* blk;
    if (ba) {  // the block's address, formed by block_bases
      blk = global_ptr(ba[t]);
    } else {
      const uint32_t pid_t = __builtin_amdgcn_readlane(pid_lane, 16 * t);  // a live page id, >= 0
      blk = a.k_pages + uint64_t(pid_t) * uint64_t(a.ksp) + (kvh >> a.kvshift) * a.ksh +
            uint32_t((c0 + 16 * t) & smask) * uint32_t(NBK);
    }
    const uint8_t* q = blk + lane_off;
    if constexpr (QB == 16) {
      const uint4 x = *reinterpret_cast<const uint4*>(q);
      r.w[t * QW] = x.x;
      r.w[t * QW + 1] = x.y;
      r.w[t * QW + 2] = x.z;
      r.w[t * QW + 3] = x.w;
    } else if constexpr (QB % 8 == 0) {
#pragma unroll
      for (int i = 0; i < QB / 8; ++i) {
        const uint2 x = reinterpret_cast<const uint2*>(q)[i];
        r.w[t * QW + 2 * i] = x.x;
        r.w[t * QW + 2 * i + 1] = x.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < QB / 4; ++i) r.w[t * QW + i] = reinterpret_cast<const uint32_t*>(q)[i];
    }
  });
  // page ids are >= 0 and the norm strides below 2^31 (checked on the host): one
  // 32 x 32 -> 64-bit multiply-add per offset
  const uint32_t slot = uint32_t((c0 + lane) & smask);
  const uint32_t pid = uint32_t(pid_lane), kvr = uint32_t(kvh >> a.kvshift);
  r.w[KW] = a.k_norms[uint64_t(pid) * uint32_t(a.knp) + (kvr * uint32_t(a.knh) + slot)];
  r.w[KW + 1] = a.v_norms[uint64_t(pid) * uint32_t(a.vnp) + (kvr * uint32_t(a.vnh) + slot)];
}

template <int NG>
struct MxState {
  f32x4 acc[8];       // acc[mt] register i: dim 32g + 8i + mt of column c, scaled by 2^(8-gs)
  float m[4 * NG];    // reference maxima (wave-uniform), log2 units
  float l[4 * NG];    // sum of 2^(s - m) over this lane's tokens
  int gs;             // value scale shift (wave-uniform)
};

// Value of lane (c + NH) % 16's x added to x: the two halves of a column pair.
template <int NH>
__device__ __forceinline__ float add_half(float x) {
  // row_ror:(16 - NH): lane c of a row receives lane (c + NH) % 16
  return x + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x120 + (16 - NH), 0xf,
                                                                 0xf, true));
}

// Scores of the chunk into the tile (head h of token 16r + 4i + g at word
// h * kTileStride + 16r + 4g + i; with kTileHalves the part of q' L at word
// (h + NH) * kTileStride + ...), before the 2^-(e+8) scale.
template <int BWK, int BWV, int NG>
__device__ __forceinline__ void score_phase_mx(const RowBuf<BWK, BWV>& K, Tab<BWK>& cbk, const h8 (&qb)[8], int lane,
                                               uint32_t* pt) {
  constexpr int NH = 4 * NG, QW = BWK, LA = mx_lookahead<BWK, BWV>();
  f32x4 d[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) d[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  // step k = 4s + r: K-step s (codes 8s..8s+3 of the quarter: pairs 2s, 2s+1) of tile r
  uint2 e[LA + 1][2];
  auto look = [&](auto kc, uint2 (&o)[2]) {
    constexpr int k = decltype(kc)::value, s = k >> 2, r = k & 3;
    o[0] = piece_pair<BWK, 2 * s>(K.w + r * QW, cbk);
    o[1] = piece_pair<BWK, 2 * s + 1>(K.w + r * QW, cbk);
  };
  static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 32>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    if constexpr (k + LA < 32) {
      look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
    d[k & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(e[k % (LA + 1)][0], e[k % (LA + 1)][1]), qb[k >> 2],
                                                      d[k & 3], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  });
  const int c = lane & 15, g = lane >> 4;
  if constexpr (!kTileHalves<NG>) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) d[r][i] = add_half<NH>(d[r][i]);
  }
  wave_lds_sync();  // the previous chunk's reads of the tile are done
  if (c < (kTileHalves<NG> ? 2 * NH : NH)) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<float4*>(pt + c * kTileStride + 16 * r + 4 * g) = make_float4(d[r][0], d[r][1], d[r][2], d[r][3]);
  }
  wave_lds_sync();
}

// Online softmax of one chunk (lane = token) from the score tile; p n_V 2^-gs goes
// back to the same words as H | L << 16.
template <int NG>
__device__ __forceinline__ void softmax_phase_mx(float sc, uint32_t nk_h, uint32_t nv_h, bool valid, int lane,
                                                 uint32_t* pt, MxState<NG>& st) {
  constexpr int H = 4 * NG;
  const int off = 16 * (lane >> 4) + 4 * (lane & 3) + ((lane >> 2) & 3);  // word of token lane
  const float nk = half_lo(nk_h) * sc;
  const float nv = valid ? half_lo(nv_h) : 0.f;
  float sv[H];
  if constexpr (kTileHalves<NG>) {
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float x = __builtin_bit_cast(float, pt[i * kTileStride + off]) +
                      __builtin_bit_cast(float, pt[(i + H) * kTileStride + off]);
      sv[i] = valid ? x * nk : -INFINITY;
    }
  } else {
    float x[H];
#pragma unroll
    for (int i = 0; i < H; ++i) x[i] = __builtin_bit_cast(float, pt[i * kTileStride + off]);
    read_unconditionally(x);
#pragma unroll
    for (int i = 0; i < H; ++i) sv[i] = valid ? x[i] * nk : -INFINITY;
  }
  // value scale: 2^kRescale * max(n_V) * 2^-gs < 2^15, i.e. every n_V < 2^(7 + gs); the
  // scale only grows, so the wave's maximum is taken only when a norm reaches the limit
  if (__any(nv >= ldexpf(1.f, 7 + st.gs))) {  // wave-uniform, rare
    int ge;
    frexpf(wave_max_nonneg(nv), &ge);
    const int gs_need = max(0, ge - 7);
    const float f = ldexpf(1.f, st.gs - gs_need);
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) st.acc[mm] *= f;
    st.gs = gs_need;
  }
  // the reference maxima move when a score exceeds its head's by more than kRescale:
  // one test of the largest excess over the heads (masked tokens give -inf; the first
  // chunk, with every maximum at -inf, always moves)
  float d[H], dmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    d[i] = sv[i] - st.m[i];
    dmax = fmaxf(dmax, d[i]);
  }
  if (st.m[0] == -INFINITY || __any(dmax > kRescale)) {  // wave-uniform
    const int hc = (lane & 15) % H;  // head of this lane's accumulator column
    float alpha_c = 1.f;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float m_new = fmaxf(st.m[i], wave_max_dpp(sv[i]));
      const float alpha = __builtin_amdgcn_exp2f(st.m[i] - m_new);  // 0 on the first chunk
      st.m[i] = m_new;
      st.l[i] *= alpha;
      alpha_c = hc == i ? alpha : alpha_c;
      d[i] = sv[i] - m_new;
    }
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) st.acc[mm] *= alpha_c;
  }
  const float nvs = ldexpf(nv, -st.gs);
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float p = __builtin_amdgcn_exp2f(d[i]);  // 0 for masked tokens
    st.l[i] += p;
    pt[i * kTileStride + off] = split_word(p * nvs);
  }
  wave_lds_sync();
}

// Values of a chunk: 4 K-steps (16 tokens each) x 8 M-tiles (one dim of each lane's
// eight), one MFMA each; lookups run LA steps ahead.
template <int BWK, int BWV, int NG>
__device__ __forceinline__ void value_phase_mx(RowBuf<BWK, BWV>& V, Tab<BWV>& cbv, const uint32_t* pt, int lane,
                                               f32x4 (&acc)[8]) {
  constexpr int NH = 4 * NG, VW = VWords<BWV>::N, LA = mx_lookahead<BWK, BWV>();
  const int c = lane & 15, g = lane >> 4;
  if constexpr (BWV != 4) merge_value_pairs<BWK, BWV>(V, lane);
  const uint32_t sel = c < NH ? 0x01000100u : c < 2 * NH ? 0x03020302u : 0x0c0c0c0cu;
  const uint32_t* prow = pt + (c % NH) * kTileStride + 4 * g;
  // step k = 8ks + mt
  auto look = [&](auto kc, uint2 (&o)[2]) {
    constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7;
    if constexpr (BWV == 4) {
      // 4-bit: byte mt/2 of the merged bytes of token pairs (0,1), (2,3) of K-step ks
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const uint32_t wa = V.w[(4 * ks + 2 * p) * VW], wb = V.w[(4 * ks + 2 * p + 1) * VW];
        const uint32_t x = (mt & 1) ? (((wa >> 4) & 0x0F0F0F0Fu) | (wb & 0xF0F0F0F0u))
                                    : ((wa & 0x0F0F0F0Fu) | ((wb << 4) & 0xF0F0F0F0u));
        o[p] = entry4<(mt >> 1)>(cbv, x);
      }
    } else {
      // token pair (4 ks + 2p, 4 ks + 2p + 1), merged by merge_value_pairs: Ce in the
      // first token's slot (even dims), Co in the second's (odd dims)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        o[p] = pair_entry<BWV>(cbv, pair_offset<BWV, BWV * mt>(V.w + (4 * ks + 2 * p + (mt & 1)) * VW));
    }
  };
  // the p n_V words of K-step ks + 1 are read one K-step ahead: LDS returns a wave's
  // reads in order, so a read issued just before its use would also wait for every
  // lookup issued ahead of it
  uint4 wq = *reinterpret_cast<const uint4*>(prow);
  uint2 e[LA + 1][2];
  static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
  h8 bq;
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 32>([&](auto kc) {
    constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7;
    if constexpr (mt == 0) {
      bq = dup4(wq.x, wq.y, wq.z, wq.w, sel);
      if constexpr (ks + 1 < 4) wq = *reinterpret_cast<const uint4*>(prow + 16 * (ks + 1));
    }
    if constexpr (k + LA < 32) {
      look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(e[k % (LA + 1)][0], e[k % (LA + 1)][1]), bq, acc[mt], 0,
                                                     0, 0);
    __builtin_amdgcn_sched_barrier(0);
  });
}

// ------------------------------------------------------------------ TF32-class products
//
// allow_tf32 (packed_attention_triton.py:113, 127): both products on single fp16
// operands, 11 significant bits each (the class of TF32's 10 stored bits), accumulated
// in fp32; 4 or 6-bit K and V, one or two head groups. A table entry holds H(2^8 c) of
// two codes (4 bytes). The 4-bit table is replicated once per lane of the wave (entry
// (b, r) at byte 256 b + 4 r of a 64 KB slot), so one SDWA move forms its address as
// in the 16-bit scan and no read waits on a bank conflict; the 6-bit table holds the
// 4096 code pairs (16 KB) and is read at 4 x the 12-bit pair index. Without the L
// halves an 8-slot operand carries eight codes: the scores take 4 K-steps per tile (16
// MFMAs per chunk) and the values 2 K-steps per M-tile (16 MFMAs), half the 16-bit
// scan's matrix-core work, and the lookups read 4 bytes instead of 8.
//   scores  K-step s of tile r: k-slots of group g = dims 32g + 8s + (0..7); column
//           c < NH is H(q' head c), the other columns zero.
//   values  K-step ks: k-slots of group g = tokens 32ks + 4j + g, j = 0..7 (token quads
//           8ks + j of the V buffer); column c < NH is H(p n_V 2^-gs) of head c, read
//           from an fp16 p tile whose 8 halves per (head, ks, g) sit side by side.

static_assert(kTfTableBytes == kPairTableBytes, "the TF table takes the 64 KB slot of the 16-bit table");

constexpr int kTfLookahead = 4;  // K-steps of table reads in flight ahead of their MFMA

// fp16 p tile of a wave (after its score tile): NH heads x 64 tokens, token l of the
// chunk at half 32 (l >> 5) + 8 (l & 3) + ((l >> 2) & 7) of its head's row.
template <int NG>
constexpr int tf_ptile_offset() { return 4 * NG * kTileStride; }  // words

// LDS of a TF work-group: the two tables (a 4-bit table in a 64 KB slot of its own,
// slot 1 beside a 6-bit table, whose reads then need no base add: the read's 16-bit
// offset field holds its offsets), then a score tile and a p tile per wave.
template <int BWK, int BWV, int NG, int WPB>
struct TfLds {
  static constexpr bool k4 = BWK == 4, v4 = BWV == 4;
  static constexpr int k_off = k4 && !v4 ? kTfTableBytes : 0;
  static constexpr int v_off = v4 ? kTfTableBytes : k4 ? 0 : tf_table_bytes<BWK>();
  static constexpr int tiles = k_off + tf_table_bytes<BWK>() > v_off + tf_table_bytes<BWV>()
                                   ? k_off + tf_table_bytes<BWK>()
                                   : v_off + tf_table_bytes<BWV>();
  static constexpr int tile_bytes = (tf_ptile_offset<NG>() + 4 * NG * 64 / 2) * 4;
  static constexpr int pace = tiles + WPB * tile_bytes;  // one word per wave (Pace)
  static constexpr int total = pace + 4 * WPB;
  static_assert(tile_bytes % 16 == 0, "tiles stay 16-byte aligned");
  static_assert(total <= 160 * 1024, "LDS of a work-group exceeds 160 KB");
};

// Scores of a chunk into the score tile (head h of token 16r + 4i + g at word
// h * kTileStride + 16r + 4g + i), before the 2^-(e+8) scale.
template <int BWK, int BWV, int NG>
__device__ __forceinline__ void score_phase_tf(const RowBuf<BWK, BWV>& K, TabTf<BWK>& cbk, const h8 (&qb)[4],
                                               int lane, uint32_t* pt) {
  constexpr int NH = 4 * NG, QW = BWK, LA = kTfLookahead;
  f32x4 d[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) d[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  // step k = 4s + r: pairs 4s .. 4s+3 (dims 8s .. 8s+7) of the quarter of tile r
  uint32_t e[LA + 1][4];
  auto look = [&](auto kc, uint32_t (&o)[4]) {
    constexpr int k = decltype(kc)::value, s = k >> 2, r = k & 3;
    o[0] = piece_pair_tf<BWK, 4 * s>(K.w + r * QW, cbk);
    o[1] = piece_pair_tf<BWK, 4 * s + 1>(K.w + r * QW, cbk);
    o[2] = piece_pair_tf<BWK, 4 * s + 2>(K.w + r * QW, cbk);
    o[3] = piece_pair_tf<BWK, 4 * s + 3>(K.w + r * QW, cbk);
  };
  static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 16>([&](auto kc) {
    constexpr int k = decltype(kc)::value, j = k % (LA + 1);
    if constexpr (k + LA < 16) {
      look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
    d[k & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(h8, u32x4{e[j][0], e[j][1], e[j][2], e[j][3]}), qb[k >> 2], d[k & 3], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  });
  const int c = lane & 15, g = lane >> 4;
  wave_lds_sync();  // the previous chunk's reads of the tile are done
  if (c < NH) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<float4*>(pt + c * kTileStride + 16 * r + 4 * g) = make_float4(d[r][0], d[r][1], d[r][2], d[r][3]);
  }
  wave_lds_sync();
}

// Online softmax of one chunk (lane = token) from the score tile; H(p n_V 2^-gs) goes to
// the fp16 p tile. Maxima, the value scale and the rescales as softmax_phase_mx.
template <int NG>
__device__ __forceinline__ void softmax_phase_tf(float sc, uint32_t nk_h, uint32_t nv_h, bool valid, int lane,
                                                 uint32_t* pt, MxState<NG>& st) {
  constexpr int H = 4 * NG;
  const int off = 16 * (lane >> 4) + 4 * (lane & 3) + ((lane >> 2) & 3);  // word of token lane
  const float nk = half_lo(nk_h) * sc;
  const float nv = valid ? half_lo(nv_h) : 0.f;
  float x[H], sv[H];
#pragma unroll
  for (int i = 0; i < H; ++i) x[i] = __builtin_bit_cast(float, pt[i * kTileStride + off]);
  read_unconditionally(x);
#pragma unroll
  for (int i = 0; i < H; ++i) sv[i] = valid ? x[i] * nk : -INFINITY;
  if (__any(nv >= ldexpf(1.f, 7 + st.gs))) {  // wave-uniform, rare
    int ge;
    frexpf(wave_max_nonneg(nv), &ge);
    const int gs_need = max(0, ge - 7);
    const float f = ldexpf(1.f, st.gs - gs_need);
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) st.acc[mm] *= f;
    st.gs = gs_need;
  }
  float d[H], dmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    d[i] = sv[i] - st.m[i];
    dmax = fmaxf(dmax, d[i]);
  }
  if (st.m[0] == -INFINITY || __any(dmax > kRescale)) {  // wave-uniform
    const int hc = (lane & 15) % H;  // head of this lane's accumulator column (columns >= H hold zeros)
    float alpha_c = 1.f;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float m_new = fmaxf(st.m[i], wave_max_dpp(sv[i]));
      const float alpha = __builtin_amdgcn_exp2f(st.m[i] - m_new);  // 0 on the first chunk
      st.m[i] = m_new;
      st.l[i] *= alpha;
      alpha_c = hc == i ? alpha : alpha_c;
      d[i] = sv[i] - m_new;
    }
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) st.acc[mm] *= alpha_c;
  }
  const float nvs = ldexpf(nv, -st.gs);
  _Float16* ph = reinterpret_cast<_Float16*>(pt + tf_ptile_offset<NG>());
  const int slot = 32 * (lane >> 5) + 8 * (lane & 3) + ((lane >> 2) & 7);
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float p = __builtin_amdgcn_exp2f(d[i]);  // 0 for masked tokens
    st.l[i] += p;
    ph[64 * i + slot] = _Float16(p * nvs);
  }
  wave_lds_sync();
}

// Values of a chunk: 2 K-steps (32 tokens each) x 8 M-tiles (one dim of each lane's
// eight), one MFMA each. 4-bit V codes of token pairs (j, j+1) are merged into bytes;
// 6-bit ones into 12-bit pair indices by merge_value_pairs.
template <int BWK, int BWV, int NG>
__device__ __forceinline__ void value_phase_tf(RowBuf<BWK, BWV>& V, TabTf<BWV>& cbv, const uint32_t* pt, int lane,
                                               f32x4 (&acc)[8]) {
  constexpr int NH = 4 * NG, VW = VWords<BWV>::N, LA = kTfLookahead;
  const int c = lane & 15, g = lane >> 4;
  if constexpr (BWV != 4) merge_value_pairs<BWK, BWV>(V, lane);
  const _Float16* ph = reinterpret_cast<const _Float16*>(pt + tf_ptile_offset<NG>());
  const uint4* prow = reinterpret_cast<const uint4*>(ph + 64 * (c % NH) + 8 * g);
  const bool live = c < NH;
  // step k = 8ks + mt; pair p = tokens (8ks + 2p, 8ks + 2p + 1) of the V buffer
  auto look = [&](auto kc, uint32_t (&o)[4]) {
    constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (BWV == 4) {
        const uint32_t wa = V.w[8 * ks + 2 * p], wb = V.w[8 * ks + 2 * p + 1];
        const uint32_t x = (mt & 1) ? (((wa >> 4) & 0x0F0F0F0Fu) | (wb & 0xF0F0F0F0u))
                                    : ((wa & 0x0F0F0F0Fu) | ((wb << 4) & 0xF0F0F0F0u));
        o[p] = entry_tf<(mt >> 1)>(cbv, x);
      } else {
        // Ce in the first token's slot (even dims), Co in the second's (odd dims)
        o[p] = pair_entry_tf(cbv, pair_offset<BWV, BWV * mt, 2>(V.w + (8 * ks + 2 * p + (mt & 1)) * VW));
      }
    }
  };
  uint4 wq = prow[0];  // p halves of K-step 0; K-step 1's are read during K-step 0
  uint32_t e[LA + 1][4];
  static_for<0, LA>([&](auto kc) { look(kc, e[decltype(kc)::value]); });
  h8 bq;
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, 16>([&](auto kc) {
    constexpr int k = decltype(kc)::value, ks = k >> 3, mt = k & 7, j = k % (LA + 1);
    if constexpr (mt == 0) {
      bq = __builtin_bit_cast(h8, live ? u32x4{wq.x, wq.y, wq.z, wq.w} : u32x4{0u, 0u, 0u, 0u});
      if constexpr (ks == 0) wq = prow[4];  // 32 halves further: K-step 1
    }
    if constexpr (k + LA < 16) {
      look(std::integral_constant<int, k + LA>{}, e[(k + LA) % (LA + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, u32x4{e[j][0], e[j][1], e[j][2], e[j][3]}),
                                                     bq, acc[mt], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  });
}

// Undoes the value scale and writes the (acc, m, l) partial of each query head h <
// n_rep to row prow * n_rep + h: lane 16g + h writes dims 32g .. 32g+31 (columns hold
// whole values: no halves to add).
template <int NG>
__device__ __forceinline__ void write_partial_tf(const DecodeArgs& a, MxState<NG>& st, int64_t prow, int lane) {
  constexpr int D = 128, H = 4 * NG;
  const float f = ldexpf(1.f, st.gs - 8);
#pragma unroll
  for (int i = 0; i < H; ++i) st.l[i] = wave_sum(st.l[i]);
  const int64_t row0 = prow * a.n_rep;
  const int c = lane & 15, g = lane >> 4;
  if (c < H && c < a.n_rep) {
    float* dst = a.part_acc + (row0 + c) * D + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(dst + 8 * i) =
          make_float4(st.acc[0][i] * f, st.acc[1][i] * f, st.acc[2][i] * f, st.acc[3][i] * f);
      *reinterpret_cast<float4*>(dst + 8 * i + 4) =
          make_float4(st.acc[4][i] * f, st.acc[5][i] * f, st.acc[6][i] * f, st.acc[7][i] * f);
    }
  }
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

// Adds the column halves, undoes the value scale and writes the (acc, m, l) partial of
// each query head h < n_rep to row prow * n_rep + h: lane 16g + h writes dims
// 32g .. 32g+31.
template <int NG>
__device__ __forceinline__ void write_partial_mx(const DecodeArgs& a, MxState<NG>& st, int64_t prow, int lane) {
  constexpr int D = 128, H = 4 * NG;
  const float f = ldexpf(1.f, st.gs - 8);
#pragma unroll
  for (int mm = 0; mm < 8; ++mm)
#pragma unroll
    for (int i = 0; i < 4; ++i) st.acc[mm][i] = add_half<H>(st.acc[mm][i]) * f;
#pragma unroll
  for (int i = 0; i < H; ++i) st.l[i] = wave_sum(st.l[i]);
  const int64_t row0 = prow * a.n_rep;
  const int c = lane & 15, g = lane >> 4;
  if (c < H && c < a.n_rep) {
    float* dst = a.part_acc + (row0 + c) * D + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(dst + 8 * i) =
          make_float4(st.acc[0][i], st.acc[1][i], st.acc[2][i], st.acc[3][i]);
      *reinterpret_cast<float4*>(dst + 8 * i + 4) =
          make_float4(st.acc[4][i], st.acc[5][i], st.acc[6][i], st.acc[7][i]);
    }
  }
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

// scan_range on the 16x16x32 fp16 MFMA; TF: the TF32-class products (4 or 6-bit
// codes, TabTf tables). left_after: the wave's chunks after this range (pacing).
template <int BWK, int BWV, int NG, bool TF, class TabK, class TabV>
__device__ __forceinline__ void scan_range16(const DecodeArgs& a, int b, int kvh, int t_lo, int t_hi, int64_t prow,
                                             int lane, TabK& cbk, TabV& cbv, uint32_t* ptile, const Pace& pace,
                                             uint32_t left_after) {
  static_assert(!TF || ((BWK == 4 || BWK == 6) && (BWV == 4 || BWV == 6)), "TF32-class scan: 4 or 6-bit K and V");
  constexpr int D = 128, NH = 4 * NG;
  const int page_hi = (t_hi + (1 << a.log2S) - 1) >> a.log2S;
  const int n = (t_hi - t_lo + 63) >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int32_t* trow = a.table + b * a.tsb;
  auto pid_of = [&](int ch) {
    const int col = min((t_lo + 64 * ch + lane) >> a.log2S, page_hi - 1);
    return trow[col];
  };
  // the first two chunks' page ids are loaded together with the query below
  const int pid0 = pid_of(0), pid1 = pid_of(1);

  // B operands of the scores: column c, K-step s, k-slots of group g = dims
  // 32g + 4s + (0..3), each twice; H (c < NH) or L (c >= NH) of q' = q 2^e, zero
  // for columns past 2 NH
  float qv[32];
  float amax = 0.f;
  {
    const float4* qp = reinterpret_cast<const float4*>(
        a.q_rot + ((int64_t(b) * a.Hkv + kvh) * NH + (c % NH)) * D + 32 * g);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float4 x = qp[s];
      qv[4 * s] = x.x;
      qv[4 * s + 1] = x.y;
      qv[4 * s + 2] = x.z;
      qv[4 * s + 3] = x.w;
    }
#pragma unroll
    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(qv[k]));
  }
  int qe;
  frexpf(uniform(wave_max(amax)), &qe);
  const int e = 15 - qe;  // |q| < 2^qe, so |q 2^e| < 2^15
  const float sc = ldexpf(1.f, -(e + 8));
  h8 qb[TF ? 4 : 8];
  if constexpr (TF) {
    // K-step s: dims 32g + 8s + (0..7) of q' head c, rounded to nearest; zero past column 3
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) qb[s][j] = c < NH ? _Float16(ldexpf(qv[8 * s + j], e)) : _Float16(0.f);
  } else {
    const uint32_t qsel = c < NH ? 0x01000100u : c < 2 * NH ? 0x03020302u : 0x0c0c0c0cu;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qb[s] = dup4(split_word(ldexpf(qv[4 * s], e)), split_word(ldexpf(qv[4 * s + 1], e)),
                   split_word(ldexpf(qv[4 * s + 2], e)), split_word(ldexpf(qv[4 * s + 3], e)), qsel);
  }

  MxState<NG> st;
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) st.acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    st.m[i] = -INFINITY;
    st.l[i] = 0.f;
  }
  st.gs = 0;
  using Buf = RowBuf<BWK, BWV>;
  const int smask = (1 << a.log2S) - 1;
  const uint64_t kbase = uint64_t(a.k_pages) + uint64_t(kvh >> a.kvshift) * uint64_t(a.ksh);
  const uint64_t vbase = uint64_t(a.v_pages) + uint64_t(kvh >> a.kvshift) * uint64_t(a.vsh);
  int pid_next;
  // The next chunk's loads are issued on every step, the last one included (its
  // addresses clamped into the range's last page, all lanes on one line): with loads
  // on only some paths, the compiler's wait counts for a chunk's rows would have to
  // cover the paths that skipped them, and each step would wait for every load in
  // flight, the next chunk's V rows included, before it could start.
  auto step = [&](int ch, Buf& X, Buf& Y, Buf& Z) {
    const int c0 = t_lo + 64 * ch;
    const int pid_after = pid_of(ch + 2);
    const bool more = ch + 1 < n;
    const uint32_t left = uint32_t(n - ch) + left_after;
    pace.publish(left);
    const uint32_t partner_left = pace.partner_left();
    // addresses of the next chunk's four 16-token blocks, for its K and its V rows
    uint64_t kb[4], vb[4];
    block_bases<16 * BWK>(kbase, uint32_t(a.ksp), pid_next, c0 + 64, lane, smask, kb);
    load_k16(a, kvh, lane, c0 + 64, pid_next, Z, more, kb);
    if constexpr (TF) {
      score_phase_tf<BWK, BWV, NG>(X, cbk, qb, lane, ptile);
      softmax_phase_tf<NG>(sc, X.w[Buf::KW], X.w[Buf::KW + 1], c0 + lane < t_hi, lane, ptile, st);
    } else {
      score_phase_mx<BWK, BWV, NG>(X, cbk, qb, lane, ptile);
      softmax_phase_mx<NG>(sc, X.w[Buf::KW], X.w[Buf::KW + 1], c0 + lane < t_hi, lane, ptile, st);
    }
    block_bases<16 * BWV>(vbase, uint32_t(a.vsp), pid_next, c0 + 64, lane, smask, vb);
    load_v<BWK, BWV, kRawV<BWV>>(a, kvh, lane, c0 + 64, pid_next, X, more, vb);
    if constexpr (TF) value_phase_tf<BWK, BWV, NG>(Y, cbv, ptile, lane, st.acc);
    else value_phase_mx<BWK, BWV, NG>(Y, cbv, ptile, lane, st.acc);
    pid_next = pid_after;
    pace_step(left, partner_left);
  };

  Buf b0, b1, b2;
  load_k16(a, kvh, lane, t_lo, pid0, b0);
  load_v<BWK, BWV, kRawV<BWV>>(a, kvh, lane, t_lo, pid0, b1);
  pid_next = pid1;
  wait_vmem_all();
  // whole turns of the three buffers in a loop without early exits (a loop header
  // reached from an exit path gets its wait counts from that path), then the rest
  int ch = 0;
  for (; ch + 3 <= n; ch += 3) {
    step(ch, b0, b1, b2);
    step(ch + 1, b2, b0, b1);
    step(ch + 2, b1, b2, b0);
  }
  if (ch < n) step(ch, b0, b1, b2);
  if (ch + 1 < n) step(ch + 1, b2, b0, b1);
  if constexpr (TF) write_partial_tf<NG>(a, st, prow, lane);
  else write_partial_mx<NG>(a, st, prow, lane);
}

template <int BWK, int BWV, int NG, int WPB>
struct Rows16Lds {
  static constexpr int k_off = RowsLds<BWK, BWV, NG, WPB>::k_off;
  static constexpr int v_off = RowsLds<BWK, BWV, NG, WPB>::v_off;
  static constexpr int tiles = RowsLds<BWK, BWV, NG, WPB>::tiles;
  static constexpr int tile_bytes = (kTileHalves<NG> ? 2 : 1) * 4 * NG * kTileStride * 4;
  static constexpr int pace = tiles + WPB * tile_bytes;  // one word per wave (Pace)
  static constexpr int total = pace + 4 * WPB;
  static_assert(total <= 160 * 1024, "LDS of a work-group exceeds 160 KB");
};

template <int BWK, int BWV, int NG, int WPB>
__global__ __launch_bounds__(64 * WPB) void decode_rows16_kernel(DecodeArgs a) {
  using Lay = Rows16Lds<BWK, BWV, NG, WPB>;
  __shared__ __align__(16) char lds[Lay::total];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t w = int64_t(xcd_major(blockIdx.x, gridDim.x)) * WPB + wig;
  // the tables' codebook loads travel while the wave looks up its first range (the
  // plan's dependent scalar loads and divisions); the entries are stored after
  const auto lk = load_table16<BWK, 64 * WPB>(a.cb_k, tid);
  const auto lv = load_table16<BWV, 64 * WPB>(a.cb_v, tid);
  RangeWalk rw;
  const bool live = rw.init(a, w, lane);
  store_table16<BWK, 64 * WPB>(lk, lds + Lay::k_off, tid);
  store_table16<BWV, 64 * WPB>(lv, lds + Lay::v_off, tid);
  const Pace pace = make_pace<WPB>(reinterpret_cast<uint32_t*>(lds + Lay::pace), wig);
  __syncthreads();  // the only block-wide barrier: waves run independently from here
  uint32_t* ptile = reinterpret_cast<uint32_t*>(lds + Lay::tiles + wig * Lay::tile_bytes);
  Tab<BWK> cbk = make_tab<BWK>(lds, Lay::k_off, lane);
  Tab<BWV> cbv = make_tab<BWV>(lds, Lay::v_off, lane);
  if (live) {
    rw.run(a, w, lane, [&](int b, int kvh, int t_lo, int t_hi, int64_t prow, uint32_t left) {
      scan_range16<BWK, BWV, NG, false>(a, b, kvh, t_lo, t_hi, prow, lane, cbk, cbv, ptile, pace, left);
    });
  }
  pace.publish(0);
}

// The TF32-class row scan (allow_tf32): 4 or 6-bit K and V, one or two head groups,
// the 16-bit scan's plan and loads with TF tables (TfLds).
template <int BWK, int BWV, int NG, int WPB>
__global__ __launch_bounds__(64 * WPB) void decode_rows_tf_kernel(DecodeArgs a) {
  using Lay = TfLds<BWK, BWV, NG, WPB>;
  __shared__ __align__(16) char lds[Lay::total];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wig = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t w = int64_t(xcd_major(blockIdx.x, gridDim.x)) * WPB + wig;
  // table loads travel while the wave looks up its first range (as in decode_rows16_kernel)
  const auto lk = load_table_tf<BWK, 64 * WPB>(a.cb_k, tid);
  const auto lv = load_table_tf<BWV, 64 * WPB>(a.cb_v, tid);
  RangeWalk rw;
  const bool live = rw.init(a, w, lane);
  store_table_tf<BWK, 64 * WPB>(lk, lds + Lay::k_off, tid);
  store_table_tf<BWV, 64 * WPB>(lv, lds + Lay::v_off, tid);
  const Pace pace = make_pace<WPB>(reinterpret_cast<uint32_t*>(lds + Lay::pace), wig);
  __syncthreads();  // the only block-wide barrier: waves run independently from here
  uint32_t* ptile = reinterpret_cast<uint32_t*>(lds + Lay::tiles + wig * Lay::tile_bytes);
  TabTf<BWK> cbk = make_tab_tf<BWK>(lds, Lay::k_off, lane);
  TabTf<BWV> cbv = make_tab_tf<BWV>(lds, Lay::v_off, lane);
  if (live) {
    rw.run(a, w, lane, [&](int b, int kvh, int t_lo, int t_hi, int64_t prow, uint32_t left) {
      scan_range16<BWK, BWV, NG, true>(a, b, kvh, t_lo, t_hi, prow, lane, cbk, cbv, ptile, pace, left);
    });
  }
  pace.publish(0);
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

template <int BWK, int BWV, int NG>
SplitKernel rows16_kernel() {
  constexpr int wpb = 8;  // two waves per SIMD: the 16-bit scan needs up to 256 VGPRs
  SplitKernel k;
  k.fn = decode_rows16_kernel<BWK, BWV, NG, wpb>;
  k.block = 64 * wpb;
  k.wpb = wpb;
  k.nrep = 4 * NG;
  k.log2_units = true;
  k.rows = true;
  return k;
}

// The 16-bit scan's width pairs: pair-table widths (2, 3, 4, 5, 6 bits) alike for K
// and V, and 4/6, 6/4.
template <int NG>
SplitKernel rows16_for(int bw_k, int bw_v) {
  if (bw_k == bw_v) {
    switch (bw_k) {
      case 2: return rows16_kernel<2, 2, NG>();
      case 3: return rows16_kernel<3, 3, NG>();
      case 4: return rows16_kernel<4, 4, NG>();
      case 5: return rows16_kernel<5, 5, NG>();
      case 6: return rows16_kernel<6, 6, NG>();
    }
  } else if (bw_k == 4 && bw_v == 6) {
    return rows16_kernel<4, 6, NG>();
  } else if (bw_k == 6 && bw_v == 4) {
    return rows16_kernel<6, 4, NG>();
  }
  return SplitKernel{};
}

template <int BWK, int BWV, int NG>
SplitKernel rows_tf_kernel() {
  // the 16-bit scan's work-group: twelve waves (three per SIMD, in 167 VGPRs with one K
  // and one V buffer) measured 106.5 us at config 2 against 103.0 us for eight
  constexpr int wpb = 8;
  SplitKernel k;
  k.fn = decode_rows_tf_kernel<BWK, BWV, NG, wpb>;
  k.block = 64 * wpb;
  k.wpb = wpb;
  k.nrep = 4 * NG;
  k.log2_units = true;
  k.rows = true;
  return k;
}

// The TF32-class scan's width pairs: 4 and 6 bits, alike or mixed.
template <int NG>
SplitKernel rows_tf_for(int bw_k, int bw_v) {
  if (bw_k == 4 && bw_v == 4) return rows_tf_kernel<4, 4, NG>();
  if (bw_k == 6 && bw_v == 6) return rows_tf_kernel<6, 6, NG>();
  if (bw_k == 4 && bw_v == 6) return rows_tf_kernel<4, 6, NG>();
  if (bw_k == 6 && bw_v == 4) return rows_tf_kernel<6, 4, NG>();
  return SplitKernel{};
}

// WN_DECODE_SCAN=rows32 keeps the fp32-product row scan for every width (the two
// compute the same result to fp32 rounding; the knob exists to compare them on one
// machine). Read once.
bool rows16_allowed() {
  static const bool allowed = [] {
    const char* e = getenv("WN_DECODE_SCAN");
    return !(e && !strcmp(e, "rows32"));
  }();
  return allowed;
}

}  // namespace

SplitKernel pick_split_rows_tf(int bw_k, int bw_v, int n_rep) {
  const int ng = n_rep >= 1 && n_rep <= 4 ? 1 : n_rep >= 5 && n_rep <= 8 ? 2 : 0;
  if (ng == 0 || !rows16_allowed()) return SplitKernel{};
  return ng == 1 ? rows_tf_for<1>(bw_k, bw_v) : rows_tf_for<2>(bw_k, bw_v);
}

SplitKernel pick_split_rows(int bw_k, int bw_v, int n_rep) {
  const int ng = n_rep <= 4 ? 1 : n_rep <= 8 ? 2 : 0;
  if (ng == 0) return SplitKernel{};
  if (rows16_allowed()) {
    const SplitKernel k = ng == 1 ? rows16_for<1>(bw_k, bw_v) : rows16_for<2>(bw_k, bw_v);
    if (k.fn) return k;
  }
  return ng == 1 ? rows_for<1>(bw_k, bw_v) : rows_for<2>(bw_k, bw_v);
}

}  // namespace wn
