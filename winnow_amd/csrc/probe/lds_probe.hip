// Measurement only (no counterpart in the reference): the LDS lookup rate that
// bounds the packed row scans' table reads. Their lookups are 8-byte LDS reads at
// data-dependent addresses, one per two codes (K and V: D per lane per 64-token
// chunk), into a pair table replicated once per lane of a half-wave (entry (b, r) at
// byte 256 b + 8 r, r = lane % 32), each address written by one vector instruction
// (an SDWA byte move) just before its read. The probe issues the same reads: each
// lane holds eight random entry addresses of such a table and moves every one to
// another row with one XOR before each read (reads that repeat their addresses run
// faster, so none does), eight reads in flight per wave, one three-input add per
// read, from `waves` waves on every CU, timed with HIP events.
// Built into libwinnow_probe.so (include/winnow_probe.h), not into the product library.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../../include/winnow_probe.h"

namespace {

thread_local char g_probe_error[256] = "";

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_probe_error, sizeof g_probe_error, fmt, ap);
  va_end(ap);
  return -1;
}

__global__ __launch_bounds__(1024) void lds_lookup_probe(int iters, uint32_t* sink) {
  __shared__ __align__(16) uint8_t tab[65536];
  for (int i = threadIdx.x; i < 65536 / 4; i += blockDim.x) reinterpret_cast<uint32_t*>(tab)[i] = i * 2654435761u;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  uint32_t x = (threadIdx.x * 0x9e3779b9u) ^ (blockIdx.x * 0x85ebca6bu), acc = 0;
  uint32_t a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    x = x * 1664525u + 1013904223u;
    a[k] = (((x >> 16) & 0xffu) << 8) | (8u * (lane & 31));  // entry (random byte, lane % 32)
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      a[k] ^= uint32_t(it & 1) << (8 + k);  // another row of the table every iteration
      asm volatile("" : "+v"(a[k]));
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint2 v = *reinterpret_cast<const uint2*>(tab + a[k]);
      acc = acc + v.x + v.y;
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the reads; practically never stored
}

}  // namespace

extern "C" const char* wn_probe_last_error(void) { return g_probe_error; }

extern "C" int wn_probe_lds_lookup_rate(int waves_per_cu, int iters, double* lookups_per_us_per_cu) {
  g_probe_error[0] = '\0';
  if (!(waves_per_cu >= 1 && waves_per_cu <= 16 && iters > 0 && lookups_per_us_per_cu))
    return fail("probe: waves_per_cu %d (1-16), iters %d", waves_per_cu, iters);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return fail("probe: no device");
  uint32_t* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipMalloc(&sink, 64) != hipSuccess) return fail("probe: hipMalloc");
  int rc = 0;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = fail("probe: hipEventCreate");
  } else {
    const dim3 grid(cus), block(64 * waves_per_cu);
    hipLaunchKernelGGL(lds_lookup_probe, grid, block, 0, nullptr, 64, sink);  // warm-up
    hipEventRecord(e0, nullptr);
    hipLaunchKernelGGL(lds_lookup_probe, grid, block, 0, nullptr, iters, sink);
    hipEventRecord(e1, nullptr);
    float ms = 0.f;
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.f) {
      rc = fail("probe: %s", hipGetErrorString(hipGetLastError()));
    } else {
      *lookups_per_us_per_cu = double(waves_per_cu) * iters * 8 / (double(ms) * 1e3);
    }
  }
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  hipFree(sink);
  return rc;
}
