// The vector-ALU page scan (wn_split.h) at head_dim 64 for every pair of supported
// widths (2, 3, 4, 5, 6, 8 bits for K and for V) that decode.hip does not
// instantiate. These pairs have no tuned kernel; the reference kernel takes any
// pair per call (packed_attention_triton.py:247). One source file per head_dim so
// that they compile beside each other.
#include "wn_split_any.h"

namespace wn {

SplitFn pick_split_any_d64(int bw_k, int bw_v, int nrep) { return any_for<64>(bw_k, bw_v, nrep); }

}  // namespace wn
