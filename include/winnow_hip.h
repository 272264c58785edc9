/*
 * winnow_hip.h -- C ABI of the MI355X (gfx950) TurboQuant packed decode path.
 *
 * Every entry point is extern "C", takes plain device pointers, element or
 * byte strides and sizes, returns 0 on success or a negative WN_E* code, and
 * never aborts; wn_last_error() then holds a thread-local message. Nothing
 * here allocates device memory: outputs and scratch are caller-owned (query
 * the scratch size with wn_decode_workspace_bytes). Work is enqueued on the
 * hipStream_t passed as `stream` (NULL = the default stream), in order, with
 * no host synchronisation.
 *
 * Layouts (the reference's, byte for byte):
 *   pages  (P, Hkv, S, NB) uint8, NB = D*bw/8, codes LSB-first along D
 *   norms  (P, Hkv, S)     fp16 (passed as uint16 bits)
 *   page_table (B, max_pages) int32, -1 past a sequence's last page
 *   seq_lens   (B,) int32
 * The (S, NB) rows of one (page, head) are contiguous; page and head strides
 * are free, so one layer of a (layers, P, Hkv, S, NB) pool is passed as is.
 *
 * Reference interfaces replaced (paths relative to lgoyal6/winnow):
 *   wn_decode_attention      turboquant_kv/packed_attention_triton.py:180-187
 *                            (packed_decode_attention; kernels :51-159,
 *                            host launch :204-262)
 *   wn_decode_attention_tf32 the same with allow_tf32=True (tl.dot :113, :127)
 *   wn_append_kv             turboquant_kv/packed_backend.py:155-161
 *                            (PagedPackedCache.update: quantize, pack, scatter)
 *   wn_quantize              turboquant_kv/cache.py:108-115 (TurboQuantMSE.quantize)
 *   wn_pack / wn_unpack      turboquant_kv/packing.py:37-89
 *   wn_dequantize            turboquant_kv/cache.py:117-131
 *                            (TurboQuantMSE.dequantize_into)
 *   wn_tq_dequant            turboquant_kv/kernel.py:78-115, csrc/tq_dequant.cu:186-215
 *   wn_dequantize_history    turboquant_kv/packed_backend.py:192-208
 *   wn_prefill_attention     turboquant_kv/packed_backend.py:211-226
 *                            (_reconstruct_sdpa, the Q > 1 route at :278-280:
 *                            dequantize the history, then SDPA with the offset
 *                            causal mask of packed_attention.py:198-206)
 *   wn_dense_decode_attention turboquant_kv/packed_attention_triton.py:190-201
 *                            (dense_decode_attention, the matched unquantized
 *                            baseline; DENSE branch of the kernel :101-127)
 */
#ifndef WINNOW_HIP_H
#define WINNOW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WN_ABI_VERSION 9

/* element types of floating-point tensors crossing the ABI */
enum { WN_F32 = 0, WN_F16 = 1, WN_BF16 = 2 };

/* status codes */
enum {
  WN_OK = 0,
  WN_E_INVALID = -1,     /* argument outside the supported contract        */
  WN_E_UNSUPPORTED = -2, /* shape/width combination not compiled           */
  WN_E_WORKSPACE = -3,   /* workspace missing or too small                 */
  WN_E_LAUNCH = -4       /* the HIP runtime reported an error              */
};

/* ABI version of the loaded library (WN_ABI_VERSION). */
int wn_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* wn_last_error(void);

/* Split-K plan for a decode step of this shape.
 * requested_splits > 0 asks for exactly that many splits over max_pages (the
 * reference's num_splits, packed_attention_triton.py:211-216): *pages_per_split
 * = cdiv(max_pages, splits), one partial per (sequence, kv head, split).
 * requested_splits == 0 lets the library choose. Where the row-per-lane
 * matrix-core scan applies (head_dim 128, page size >= 16, widths 2-6 bits alike
 * for K and V, 4/6, 6/4 or 8/8, 4/8, and n_rep that 2^s virtual kv heads per kv
 * head bring to <= 8 query heads each) the plan is balanced: *pages_per_split = 0
 * and *num_splits = the number of resident waves on the current device, which then
 * share the flattened (sequence, kv head, 64-token chunk) space equally, ragged
 * batches included. Otherwise (any other pair of widths in {2,3,4,5,6,8}, head_dim
 * 16, 32, 64 or 256, any other n_rep, run as groups of <= 16 query heads) fixed
 * splits sized to fill the GPU. Head dims: the powers of two 16 .. 256. */
int wn_decode_plan(int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
                   int requested_splits, int* pages_per_split, int* num_splits);

/* Bytes of scratch wn_decode_attention needs for this shape and plan: the
 * rotated query, a per-sequence chunk prefix, each (sequence, kv head)'s
 * partial range (two int32), and the (acc, m, l) partials of
 * the real query heads (B*Hkv*num_splits rows for fixed splits, num_splits +
 * B*Hkv rows for a balanced plan). -1 for invalid sizes. */
int64_t wn_decode_workspace_bytes(int B, int Hq, int Hkv, int D, int pages_per_split, int num_splits);

/* Decode attention over paged packed K/V, one query token per sequence.
 *   q      (B, Hq, D) with element strides q_stride_b, q_stride_h (last dim
 *          contiguous), element type q_dtype
 *   out    (B, Hq, D) contiguous, element type out_dtype
 *   out = softmax(scale * q k_hat^T) v_hat computed in the quantizer bases:
 *   q_rot = scale * q Pi_K^T; per key s = n_K (q_rot . c_K); online softmax
 *   over pages; a = sum p n_V c_V; out = (a / l) Pi_V. Rows with no key are 0.
 *   pages_per_split / num_splits come from wn_decode_plan (pages_per_split 0
 *   = balanced plan over num_splits waves; any num_splits >= 1 is valid).
 *   Preconditions the device reads unchecked (the Python layer checks them on
 *   host copies before the call): 0 <= seq_lens[b] <= max_pages * S, and every
 *   page id a sequence reads, page_table[b, j] for j < cdiv(seq_lens[b], S), lies
 *   in [0, P) of the pages the strides address. Norm strides (elements) are >= 0
 *   with kn_stride_p, vn_stride_p < 2^31 and Hkv * head stride + S <= 2^31
 *   (WN_E_INVALID otherwise): the scans form norm offsets in 32-bit pieces. Page
 *   strides (bytes) are >= 0 and below 2^32 (WN_E_INVALID otherwise): the scans form
 *   a page block's address from page id x page stride in 32 x 32 -> 64 bits.
 *   ev_begin / ev_end (hipEvent_t or NULL) are recorded on `stream` around
 *   the split-K page-scan kernel only, for in-situ timing of that kernel. */
int wn_decode_attention(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const float* pi_k, const float* pi_v,
    const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b,
    const int32_t* seq_lens,
    void* out, int out_dtype,
    void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
    float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end);

/* wn_decode_plan for wn_decode_attention_tf32: its scan may keep more waves resident,
 * so its balanced plan may have more splits. Same arguments and results. */
int wn_decode_plan_tf32(int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
                        int requested_splits, int* pages_per_split, int* num_splits);

/* wn_decode_attention with TF32-class products: replaces the reference's
 * packed_decode_attention(..., allow_tf32=True) (packed_attention_triton.py:180-187,
 * whose kernel passes allow_tf32 to both tl.dot products, :113 and :127). For 4 and
 * 6-bit K and V (alike or mixed) on the row scan (head_dim 128, page size >= 16, n_rep
 * up to 8, or up to 16 in virtual kv heads of eight), the score and value products
 * take single fp16 operands (11 significant bits, rounded to nearest) and accumulate
 * in fp32; every other shape runs the fp32-exact scan of wn_decode_attention. Same arguments, workspace,
 * preconditions and errors as wn_decode_attention; the plan comes from
 * wn_decode_plan_tf32. */
int wn_decode_attention_tf32(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const float* pi_k, const float* pi_v,
    const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b,
    const int32_t* seq_lens,
    void* out, int out_dtype,
    void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
    float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end);

/* Allocation-free variant of wn_decode_attention. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory, not even a
 * workspace (code under HIP graph capture, serving loops that forbid
 * allocation). Same arguments, meaning and result as wn_decode_attention without
 * the workspace: the scratch is a static device array of WN_NOALLOC_SCRATCH_BYTES
 * (32 MiB) that each GPU the library runs on holds until the process ends. A
 * shape and plan whose wn_decode_workspace_bytes exceeds it is rejected with
 * WN_E_WORKSPACE before any launch. Calls on one GPU share that array, so calls
 * that overlap on one GPU (different streams, or threads) race; calls ordered on
 * one stream do not. Nothing is allocated or freed. */
#define WN_NOALLOC_SCRATCH_BYTES (32ll << 20)
int wn_decode_attention_noalloc(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const float* pi_k, const float* pi_v,
    const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b,
    const int32_t* seq_lens,
    void* out, int out_dtype,
    int B, int Hq, int Hkv, int D, int S, int bw_k, int bw_v, int max_pages,
    float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end);

/* Quantize, bit-pack and scatter n new tokens per sequence into pool pages,
 * K and V in one launch (v may be NULL to append K only).
 *   k, v       (B, Hkv, n, D) with element strides (s_b, s_h, s_n), last dim
 *              contiguous, element type x_dtype
 *   token i of sequence b lands at pos = start_pos[b] + i:
 *              page page_table[b, pos / S], slot pos % S
 *   per vector: n = max(||x||, 1e-10); y = (x / n) Pi^T; code = #{boundary < y};
 *   the packed row goes to pages, fp16(n) to norms. max_pages is the width of
 *   page_table. Callers must keep every position inside the table row and every
 *   page id it names inside [0, num_pages) (the Python layer raises otherwise);
 *   as a last guard the device skips, without writing, any vector that does not.
 *   Pi_K / Pi_V 16-byte aligned; pages 8-byte aligned with strides in multiples of
 *   8 bytes. D a power of two 16 .. 256. ev_begin / ev_end (hipEvent_t or NULL)
 *   are recorded on `stream` around the kernel (its time without the caller's
 *   host overhead). */
int wn_append_kv(
    const void* k, int64_t ks_b, int64_t ks_h, int64_t ks_n,
    const void* v, int64_t vs_b, int64_t vs_h, int64_t vs_n, int x_dtype,
    const float* pi_k, const float* boundaries_k, int bw_k,
    const float* pi_v, const float* boundaries_v, int bw_v,
    const int32_t* page_table, int64_t table_stride_b,
    const int32_t* start_pos,
    uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    int B, int Hkv, int n, int D, int S, int num_pages, int max_pages,
    void* stream, void* ev_begin, void* ev_end);

/* TurboQuantMSE.quantize on `rows` contiguous-D vectors at x + r*row_stride
 * (elements): codes (rows, D) uint8 and fp32 norms (rows,). Any D from 1 to 256, as
 * for wn_dequantize (the legacy cache's regular / outlier channel splits have
 * arbitrary widths); the powers of two 16 .. 256 run the tuned kernels. */
int wn_quantize(const void* x, int x_dtype, int64_t rows, int64_t row_stride,
                const float* pi, const float* boundaries, int bw, int D,
                uint8_t* codes, float* norms, void* stream);

/* Bit packing of contiguous (rows, D) uint8 codes <-> (rows, D*bw/8) bytes. */
int wn_pack(const uint8_t* codes, int64_t rows, int D, int bw, uint8_t* packed, void* stream);
int wn_unpack(const uint8_t* packed, int64_t rows, int D, int bw, uint8_t* codes, void* stream);

/* TurboQuantMSE.dequantize_into: out = (centroids[codes] Pi) * norm for
 * (rows, D) uint8 codes and fp16 norms; out (rows, D) contiguous of out_dtype.
 * Any D from 1 to 256. */
int wn_dequantize(const uint8_t* codes, const uint16_t* norms, int64_t rows,
                  const float* pi, const float* centroids, int bw, int D,
                  void* out, int out_dtype, void* stream);

/* Fused dequantization of packed rows, unpack + codebook gather + inverse rotation
 * + norm rescale in one pass (replaces tq_dequant, turboquant_kv/kernel.py:78-115,
 * and tq_dequant_cuda, csrc/tq_dequant.cu:186-215). planes x L rows: row (p, t)
 * reads its D*bw/8 packed bytes at packed + (p * plane_rows + t) * (D*bw/8) and its
 * fp16 norm at norms + p * plane_rows + t, so a (..., MAXLEN, NB) cache buffer
 * sliced to its first L positions needs no copy (plane_rows = MAXLEN).
 * out (planes * L, D) contiguous of out_dtype (fp32, bf16 or fp16):
 * out[r] = (centroids[codes(r)] Pi) * norm(r). fast = 0: the rotation at
 * near-fp32 accuracy (error below 2^-16 per term); fast = 1: one fp16 product
 * per term (2^-11, the reference's allow_tf32). head_dim 128; packed and out
 * 16-byte aligned. */
int wn_tq_dequant(const uint8_t* packed, const uint16_t* norms, int64_t planes, int64_t L,
                  int64_t plane_rows, const float* centroids, const float* pi, int bw, int D,
                  void* out, int out_dtype, int fast, void* stream);

/* The dequantized history of one sequence straight from pool pages (replaces the
 * gather + unpack + dequantize of packed_backend.py:192-208 dequantize_history).
 * Position t < L of kv head h reads page table_row[t / S], slot t % S, at
 * pages + page * page_stride + h * head_stride + slot * (D*bw/8) (bytes) and its
 * norm at norms + page * norm_page_stride + h * norm_head_stride + slot
 * (elements). out (Hkv, L, D) contiguous of out_dtype; fast as for
 * wn_tq_dequant. head_dim 128, S a power of two, pages, their strides and out
 * 16-byte aligned. */
int wn_dequantize_history(const uint8_t* pages, int64_t page_stride, int64_t head_stride,
                          const uint16_t* norms, int64_t norm_page_stride, int64_t norm_head_stride,
                          const int32_t* table_row, int L, int Hkv, int S,
                          const float* centroids, const float* pi, int bw, int D,
                          void* out, int out_dtype, int fast, void* stream);

/* Split count of wn_prefill_attention for this shape: about two waves per resident
 * scan slot on the current device over the (sequence, kv head, 32-row query block)
 * items, and at most a quarter of the 64-token chunks of max_len (the longest
 * sequence; any count >= 1 is valid whatever the lengths). head_dim 128, S a power
 * of two >= 16, widths 4 and 6 bits (alike or mixed); WN_E_UNSUPPORTED otherwise. */
int wn_prefill_plan(int B, int Hq, int Hkv, int Q, int D, int S, int bw_k, int bw_v, int max_len,
                    int* num_splits);

/* Bytes of scratch wn_prefill_attention needs: the rotated queries (rows n_rep * Q
 * per kv head rounded up to 64) and num_splits (acc, m, l) partials per row. -1 for
 * invalid sizes. */
int64_t wn_prefill_workspace_bytes(int B, int Hq, int Hkv, int Q, int D, int num_splits);

/* Prefill attention over paged packed K/V, Q >= 1 query tokens per sequence, read in
 * the packed form (no history is written to HBM). Replaces the reference's Q > 1
 * route _reconstruct_sdpa (packed_backend.py:211-226): query i of sequence b, whose
 * seq_lens[b] = L already counts the Q new tokens, attends to keys j <= L - Q + i
 * (packed_attention.py:198-206); a query that sees no key gives 0.
 *   q    (B, Hq, Q, D) with element strides q_stride_b, q_stride_h, q_stride_q
 *        (last dim contiguous), element type q_dtype
 *   out  (B, Hq, Q, D) contiguous, element type out_dtype
 * The algebra of wn_decode_attention, with single fp16 operands (11 significant bits,
 * rounded to nearest) in both products and fp32 accumulation: finer than the
 * reference's bf16 history and bf16 SDPA for bf16 queries. head_dim 128, S a power of
 * two >= 16, 4 and 6-bit K and V (alike or mixed; WN_E_UNSUPPORTED otherwise). K
 * pages 16-byte (4-bit) or 8-byte aligned in base and strides, V pages 4-byte; norm
 * bases 8-byte aligned, norm strides multiples of 4 elements. num_splits from
 * wn_prefill_plan (any value 1..4096 is valid); the page-id and length
 * preconditions of wn_decode_attention hold here too (unchecked on the device).
 * ev_begin / ev_end (hipEvent_t or NULL) are recorded around the scan kernel. */
int wn_prefill_attention(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_q,
    const float* pi_k, const float* pi_v,
    const float* codebook_k, const float* codebook_v,
    const uint8_t* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const uint8_t* v_pages, int64_t v_stride_p, int64_t v_stride_h,
    const uint16_t* k_norms, int64_t kn_stride_p, int64_t kn_stride_h,
    const uint16_t* v_norms, int64_t vn_stride_p, int64_t vn_stride_h,
    const int32_t* page_table, int64_t table_stride_b,
    const int32_t* seq_lens,
    void* out, int out_dtype,
    void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int Q, int D, int S, int bw_k, int bw_v,
    float scale, int num_splits,
    void* stream, void* ev_begin, void* ev_end);

/* Plan of wn_dense_decode_attention (as wn_decode_plan: requested_splits > 0 gives
 * the reference's cdiv split of max_pages; 0 lets the library choose: a balanced
 * plan of persistent waves, pages_per_split = 0, for WN_BF16 and WN_F16 pages, fixed
 * splits for WN_F32 pages). */
int wn_dense_decode_plan(int B, int Hq, int Hkv, int D, int S, int page_dtype, int max_pages,
                         int requested_splits, int* pages_per_split, int* num_splits);

/* Decode attention over unquantized paged K/V (replaces dense_decode_attention,
 * turboquant_kv/packed_attention_triton.py:190-201): pages (P, Hkv, S, D) of
 * page_dtype (bf16, fp16 or fp32), the (S, D) rows of one (page, head) contiguous,
 * strides in bytes; page_table, seq_lens, q, out, the scratch (sized by
 * wn_decode_workspace_bytes with this plan) and the events as for
 * wn_decode_attention. head_dim a power of two 16 .. 256, any n_rep (over 16:
 * virtual kv heads of <= 16 query heads), S a power of two >= 16, pages and their
 * strides 16-byte aligned. bf16 / fp16 pages at head_dim 64 and 128 run on the
 * matrix cores with fp32 accuracy (q and the probabilities as 16-bit hi + lo pairs
 * against exact 16-bit K and V); fp32 pages, and the other head dims, on a
 * vector-ALU scan that needs fixed splits (pages_per_split > 0, which
 * wn_dense_decode_plan returns for them). */
int wn_dense_decode_attention(
    const void* q, int q_dtype, int64_t q_stride_b, int64_t q_stride_h,
    const void* k_pages, int64_t k_stride_p, int64_t k_stride_h,
    const void* v_pages, int64_t v_stride_p, int64_t v_stride_h, int page_dtype,
    const int32_t* page_table, int64_t table_stride_b,
    const int32_t* seq_lens,
    void* out, int out_dtype,
    void* workspace, int64_t workspace_bytes,
    int B, int Hq, int Hkv, int D, int S, int max_pages,
    float scale, int pages_per_split, int num_splits,
    void* stream, void* ev_begin, void* ev_end);

#ifdef __cplusplus
}
#endif

#endif /* WINNOW_HIP_H */
