// Shared device helpers and host error plumbing for the gfx950 TurboQuant path.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/winnow_hip.h"

namespace wn {

// ---------------------------------------------------------------- host errors
void set_error(const char* fmt, ...);
void clear_error();

#define WN_REQUIRE(cond, code, ...)         \
  do {                                      \
    if (!(cond)) {                          \
      ::wn::set_error(__VA_ARGS__);         \
      return (code);                        \
    }                                       \
  } while (0)

int check_launch(const char* what);

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}
inline bool valid_bw(int bw) { return bw == 2 || bw == 3 || bw == 4 || bw == 5 || bw == 6 || bw == 8; }
// Head dims the library compiles: the powers of two 16 .. 256 (the reference kernel
// takes any power of two >= 16, packed_attention_triton.py:160-172).
inline bool valid_head_dim(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }
inline bool aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ------------------------------------------------------------- device helpers
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, uint32_t(b) << 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {  // round to nearest even
  return __builtin_bit_cast(uint16_t, _Float16(f));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {  // round to nearest even, NaN kept quiet
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == WN_F32) return static_cast<const float*>(p)[i];
  if (dtype == WN_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float v) {
  if (dtype == WN_F32) static_cast<float*>(p)[i] = v;
  else if (dtype == WN_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
}

// Code `d` of a row held as little-endian 32-bit words, LSB-first, BW bits per
// code; codes may straddle a word. With `d` known at compile time this folds
// to one bit-field extract (or an align + mask on a straddle).
template <int BW, int NW>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[NW], int d) {
  const int bit = d * BW;
  const int wi = bit >> 5, sh = bit & 31;
  uint32_t v = w[wi] >> sh;
  if (sh + BW > 32) v |= w[wi + 1] << (32 - sh);
  return v & ((1u << BW) - 1u);
}

// A read-only view through the constant address space, for buffers no launch writes
// while it reads them (plans, lengths, prefixes): their wave-uniform reads become
// scalar loads, which wait on their own counter rather than behind the wave's vector
// loads (through a plain pointer the compiler cannot rule out a store by the kernel,
// and reads uniform values with vector loads).
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* const_view(const T* p) {
  return (const __attribute__((address_space(4))) T*)(p);
}

// f(i) for i = tid + NTHR k in [0, N), for the staging loops of a work-group's
// prologue: the trip count is known at compile time, so the loop unrolls and every
// iteration's loads are issued before the first wait (a loop on i < N waits for each
// iteration's loads in turn, a chain of cache round trips before the work starts).
template <int N, int NTHR, class F>
__device__ __forceinline__ void for_strided(int tid, F&& f) {
#pragma unroll
  for (int k = 0; k < (N + NTHR - 1) / NTHR; ++k) {
    const int i = tid + NTHR * k;
    if (N % NTHR == 0 || i < N) f(i);
  }
}

// Wave-wide (64 lanes) reductions.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Orders this wave's LDS writes before its later LDS reads (no block barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Pacing of the two waves that share a SIMD. A work-group's eight waves are dealt to
// the CU's four SIMDs in turn, so waves k and k ^ 4 share one, and its issue arbiter
// favours the older wave of the two: with equal shares of chunks, wave k ran ahead
// and wave k ^ 4 scanned the last fifth of its chunks alone, latency-bound (per-wave
// timestamps of the decode row scan at BASELINE config 2: waves 0-3 of every
// work-group ended at ~106 us, waves 4-7 at ~129 us). Each wave publishes the chunks
// it has left in an LDS word once per chunk and raises its priority while it has
// more left than its partner. No chunk moves between waves, so the results are those
// of an unpaced scan.
// The words are read and written with relaxed work-group-scope atomics: a stale
// value only delays the priority change by a chunk.
// Neither step branches in the caller's code. Every lane stores the same value (a
// store under `lane == 0` puts a divergent branch into the caller's loop), and the
// priority choice sits inside one asm statement (s_setprio takes only an immediate;
// a branch around two of them splits the loop body into blocks). Either branch made
// the compiler spill in the 6-bit prefill scan, which sits at 249-253 VGPRs.
struct Pace {
  uint32_t* mine;     // this wave's word
  uint32_t* partner;  // the word of the other wave on its SIMD
  __device__ void publish(uint32_t left) const {
    __hip_atomic_store(mine, left, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __device__ uint32_t partner_left() const {
    return __hip_atomic_load(partner, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
};

template <int WPB>
__device__ __forceinline__ Pace make_pace(uint32_t* words, int wig) {
  static_assert(WPB == 8, "pacing pairs waves k and k ^ 4: two waves per SIMD");
  const Pace p{words + wig, words + (wig ^ 4)};
  p.publish(0);  // before the work-group barrier
  return p;
}

// Priority for the next chunk: raised while this wave has more chunks left than its
// partner (a partner without work, or done, shows 0).
__device__ __forceinline__ void pace_step(uint32_t left, uint32_t partner_left) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(left), pl = __builtin_amdgcn_readfirstlane(partner_left);
  asm volatile(
      "s_cmp_lt_u32 %0, %1\n\t"
      "s_cbranch_scc0 .Lpace_low%=\n\t"
      "s_setprio 1\n\t"
      "s_branch .Lpace_done%=\n"
      ".Lpace_low%=:\n\t"
      "s_setprio 0\n"
      ".Lpace_done%=:"
      :
      : "s"(pl), "s"(l)
      : "scc");
}

}  // namespace wn
