// The vector-ALU page scan (wn_split.h) at head_dim 256 for K widths 5, 6 and 8 and
// every V width (decode_split_any256.hip holds K widths 2-4).
#include "wn_split_any.h"

namespace wn {

SplitFn pick_split_any_d256_hi(int bw_k, int bw_v, int nrep) { return any_for_hi<256>(bw_k, bw_v, nrep); }

}  // namespace wn
