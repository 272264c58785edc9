// Internal interface shared by the decode translation units.
#pragma once

#include "wn_common.h"

namespace wn {

struct DecodeArgs {
  const float* q_rot;  // (B, Hkv, NREP, D) fp32, rows >= n_rep are zero
  const uint8_t* k_pages;
  const uint8_t* v_pages;
  const uint16_t* k_norms;
  const uint16_t* v_norms;
  const float* cb_k;
  const float* cb_v;
  const int32_t* table;
  const int32_t* seq_lens;
  float* part_acc;  // (rows * n_rep, D): rows = B*Hkv*num_splits, or num_splits + B*Hkv balanced
  float* part_ml;   // (rows * n_rep, 2): running max (log2 units for the matrix-core scan), sum
  int64_t ksp, ksh, vsp, vsh;  // page strides, bytes
  int64_t knp, knh, vnp, vnh;  // norm strides, elements
  int64_t tsb;                 // page-table row stride, elements
  const int32_t* chunk_prefix;  // (B+1) running count of 64-token chunks per sequence (balanced)
  int2* unit_meta;              // (B*Hkv): first partial row and partial count of each (sequence, kv head)
  int B, Hkv, n_rep, log2S, pages_per_split, num_splits;
  int balanced;  // 1: persistent waves share the flattened chunk space (pages_per_split unused)
  int qrows;     // rows of q_rot per kv head
  int kvshift;   // the pages of (virtual) kv head h are those of kv head h >> kvshift (row scans)
  int kvdiv;     // the same for the vector-ALU scan: kv head h / kvdiv
};

using SplitFn = void (*)(DecodeArgs);

struct SplitKernel {
  SplitFn fn = nullptr;
  int block = 0;  // threads per work-group
  int wpb = 1;    // independent waves per work-group (row scan); grid counts waves / wpb
  int nrep = 0;   // query-head rows per kv head the kernel reads from q_rot
  bool log2_units = false;  // scores/maxima in log2 units (q_rot scaled by log2 e)
  bool rows = false;        // the row-per-lane matrix-core scan (balanced plans allowed)
  int kvshift = 0;          // row scan: each kv head runs as 2^kvshift virtual heads of n_rep >> kvshift
  int kvdiv = 1;            // virtual heads per kv head (1 << kvshift on the row scan)
};

// Row-per-lane matrix-core page scan for head_dim 128, power-of-two page sizes
// >= 16 and up to eight query heads per kv head, in one or two groups of four
// (wpb independent waves per work-group sharing the codebook tables, fixed
// splits or balanced persistent waves), or an empty SplitKernel when
// (bw_k, bw_v, n_rep) is not compiled.
SplitKernel pick_split_rows(int bw_k, int bw_v, int n_rep);

// The TF32-class row scan (single fp16 operands, fp32 accumulation; allow_tf32) for
// 4 and 6-bit K and V (alike or mixed) and up to eight query heads per kv head, or an
// empty SplitKernel.
SplitKernel pick_split_rows_tf(int bw_k, int bw_v, int n_rep);

// Dense-page scan (bf16 or fp16 pages of head_dim 64 or 128, up to 16 query heads
// per kv head, page size >= 16) on the row scan's work plan, or an empty SplitKernel
// for another page dtype or head_dim.
SplitKernel pick_dense_scan(int page_dtype, int D);

// The vector-ALU dense scan on fixed splits, for fp32 pages at every head_dim and
// for bf16/fp16 pages at the head dims the MFMA scan does not take (16, 32, 256),
// nrep query rows per (virtual) kv head (1, 2, 4, 8 or 16).
SplitKernel pick_dense_valu_scan(int page_dtype, int D, int nrep);

// The vector-ALU scan for what decode.hip does not instantiate: at head_dim 64 and
// 128 the width pairs without a tuned kernel, at 16, 32 and 256 every pair of
// supported widths; nrep query rows per kv head (1, 2, 4, 8 or 16), or nullptr.
SplitFn pick_split_any(int D, int bw_k, int bw_v, int nrep);
SplitFn pick_split_any_d256(int bw_k, int bw_v, int nrep);
SplitFn pick_split_any_d128(int bw_k, int bw_v, int nrep);
SplitFn pick_split_any_d64(int bw_k, int bw_v, int nrep);
SplitFn pick_split_any_d32(int bw_k, int bw_v, int nrep);
SplitFn pick_split_any_d16(int bw_k, int bw_v, int nrep);

}  // namespace wn
