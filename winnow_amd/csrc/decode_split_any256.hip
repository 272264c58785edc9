// The vector-ALU page scan (wn_split.h) at head_dim 256 for every pair of supported
// widths (2, 3, 4, 5, 6, 8 bits for K and for V): this head_dim has no tuned
// kernel, and the reference kernel takes any power-of-two head_dim >= 16
// (packed_attention_triton.py:160-172) and any pair per call (:247). K widths 2-4
// here, 5-8 in decode_split_any256_hi.hip (the two compile beside each other).
#include "wn_split_any.h"

namespace wn {

SplitFn pick_split_any_d256_hi(int bw_k, int bw_v, int nrep);

SplitFn pick_split_any_d256(int bw_k, int bw_v, int nrep) {
  return bw_k <= 4 ? any_for_lo<256>(bw_k, bw_v, nrep) : pick_split_any_d256_hi(bw_k, bw_v, nrep);
}

}  // namespace wn
