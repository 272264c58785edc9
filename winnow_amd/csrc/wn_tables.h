// Codebook tables in LDS and the operand helpers the matrix-core page scans share
// (decode_rows.hip: decode; prefill.hip: prefill), gfx950.
//
// A table entry holds the codebook values of two codes, scaled by 2^8. The 4-bit
// tables are indexed by a code byte and replicated once per lane, so that a lane's
// read never waits on a bank conflict; one SDWA move writes the code byte into the
// lane's address register. Wider codes read a plain table of all 2^(2 BW) code pairs
// at an offset cut out of the packed words in two instructions. The TF tables
// (single fp16 values, 4 bytes per entry) feed v_mfma_f32_16x16x32_f16 operands
// directly: two entries per 4-byte k-slot pair.
#pragma once

#include <cstdint>
#include <utility>

#include "wn_common.h"

namespace wn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr float kCbScale = 256.0f;  // codebook values scaled by 2^8 before the split

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
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

// Byte offset (2^SC x index; entries of 2^SC bytes) of the pair-table entry whose
// 2 BW-bit index starts at bit BIT of the little-endian words w: the index is cut out
// already multiplied (a shift or alignbit, then one mask), two instructions per lookup.
template <int BW, int BIT, int SC = 3>
__device__ __forceinline__ uint32_t pair_offset(const uint32_t* w) {
  constexpr uint32_t m = ((1u << (2 * BW)) - 1u) << SC;
  constexpr int s = BIT - SC;  // the index's bit 0 lands on bit SC
  if constexpr (s < 0) {
    return (w[0] << (-s)) & m;
  } else {
    constexpr int wi = s >> 5, sh = s & 31;
    if constexpr (sh + 2 * BW + SC <= 32) return (w[wi] >> sh) & m;
    else return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & m;
  }
}

template <int BW>
constexpr uint64_t field_mask(int parity) {
  uint64_t m = 0;
  for (int k = parity; k < 8; k += 2) m |= ((uint64_t(1) << BW) - 1) << (BW * k);
  return m;
}

// (a & m) | (b & ~m) in one instruction whatever the compiler knows of a's and b's bits.
__device__ __forceinline__ uint32_t bitsel(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(m), "v"(a), "v"(b));
  return r;
}

constexpr int kTfTableBytes = 256 * 64 * 4;  // 256 byte values x 64 lanes x two fp16

template <int BW>
constexpr int tf_table_bytes() { return BW == 4 ? kTfTableBytes : 4 << (2 * BW); }

// Codebook values behind the table entries one thread stages: entry i = tid + NTHR k
// (k < K) holds the values of codes (lo, hi) = codes(i). Loaded apart from the stores,
// so that a kernel can issue a table's loads, do other work while they travel (the
// row scans look up their plan), and store the entries after.
template <int N, int NTHR>
struct CodePairs {
  static constexpr int K = (N + NTHR - 1) / NTHR;
  float lo[K], hi[K];
};

template <int N, int NTHR, class Codes>
__device__ __forceinline__ CodePairs<N, NTHR> load_code_pairs(const float* cb, int tid, Codes&& codes) {
  CodePairs<N, NTHR> p;
#pragma unroll
  for (int k = 0; k < CodePairs<N, NTHR>::K; ++k) {
    const int2 c = codes(min(tid + NTHR * k, N - 1));  // entries past N: loaded clamped, not stored
    p.lo[k] = cb[c.x];
    p.hi[k] = cb[c.y];
  }
  return p;
}

template <int N, int NTHR, class T, class Entry>
__device__ __forceinline__ void store_code_pairs(const CodePairs<N, NTHR>& p, T* t, int tid, Entry&& entry) {
#pragma unroll
  for (int k = 0; k < CodePairs<N, NTHR>::K; ++k) {
    const int i = tid + NTHR * k;
    if (N % NTHR == 0 || i < N) t[i] = entry(p.lo[k], p.hi[k]);
  }
}

// Two fp16 values rounded to nearest, lo in the low half.
__device__ __forceinline__ uint32_t tf_word(float lo, float hi) {
  return uint32_t(__builtin_bit_cast(uint16_t, _Float16(lo))) | uint32_t(__builtin_bit_cast(uint16_t, _Float16(hi))) << 16;
}

// Stages a TF table: 4-bit, the replicated byte table (entry (b, r) holds
// (H(2^8 c[b & 15]), H(2^8 c[b >> 4]))); 6-bit, entry i holds (H(2^8 c[i mod 64]),
// H(2^8 c[i >> 6])), two consecutive codes read as one 12-bit index.
template <int BW>
constexpr int tf_entries() { return BW == 4 ? 256 * 64 : 1 << (2 * BW); }
// codes of TF table entry i: 4-bit, byte i >> 6 (lane copy i & 63); 6-bit, a code pair
template <int BW>
__device__ __forceinline__ int2 tf_codes(int i) {
  if constexpr (BW == 4) return make_int2((i >> 6) & 15, i >> 10);
  else return make_int2(i & 63, i >> 6);
}
template <int BW, int NTHR>
using TfLoads = CodePairs<tf_entries<BW>(), NTHR>;
template <int BW, int NTHR>
__device__ __forceinline__ TfLoads<BW, NTHR> load_table_tf(const float* cb, int tid) {
  static_assert(BW == 4 || BW == 6, "TF tables: 4 and 6-bit codes");
  return load_code_pairs<tf_entries<BW>(), NTHR>(cb, tid, [](int i) { return tf_codes<BW>(i); });
}
template <int BW, int NTHR>
__device__ __forceinline__ void store_table_tf(const TfLoads<BW, NTHR>& p, char* dst, int tid) {
  store_code_pairs(p, reinterpret_cast<uint32_t*>(dst), tid,
                   [](float lo, float hi) { return tf_word(lo * kCbScale, hi * kCbScale); });
}
template <int BW, int NTHR>
__device__ __forceinline__ void stage_table_tf(const float* cb, char* dst, int tid) {
  store_table_tf<BW, NTHR>(load_table_tf<BW, NTHR>(cb, tid), dst, tid);
}

// A TF table as one lane reads it: the 6-bit table's base; the 4-bit table's address
// registers 4 lane | slot << 16, one per byte position of a code word (the code byte
// goes to bits 8-15).
template <int BW>
struct TabTf {
  const char* t;
};
template <>
struct TabTf<4> {
  const char* lds;
  uint32_t r[4];
};

template <int BW>
__device__ __forceinline__ TabTf<BW> make_tab_tf(const char* lds, int off, int lane) {
  TabTf<BW> tab;
  if constexpr (BW == 4) {
    tab.lds = lds;
#pragma unroll
    for (int k = 0; k < 4; ++k) tab.r[k] = uint32_t(4 * lane) | (uint32_t(off >> 16) << 16);
  } else {
    tab.t = lds + off;
  }
  return tab;
}

// Entry of the 4-bit pair in byte K of x: one SDWA move, one 4-byte LDS read.
template <int K>
__device__ __forceinline__ uint32_t entry_tf(TabTf<4>& tab, uint32_t x) {
  tab.r[K] = put_byte1<K>(tab.r[K], x);
  return *reinterpret_cast<const uint32_t*>(tab.lds + tab.r[K]);
}

// Entry of the 6-bit pair table at byte offset off.
__device__ __forceinline__ uint32_t pair_entry_tf(const TabTf<6>& tab, uint32_t off) {
  return *reinterpret_cast<const uint32_t*>(tab.t + off);
}

// Entry of pair N (codes 2N, 2N+1) of a packed piece held as words.
template <int BW, int N>
__device__ __forceinline__ uint32_t piece_pair_tf(const uint32_t* w, TabTf<BW>& tab) {
  if constexpr (BW == 4) return entry_tf<N & 3>(tab, w[N >> 2]);
  else return pair_entry_tf(tab, pair_offset<BW, 2 * BW * N, 2>(w));
}

}  // namespace
}  // namespace wn
