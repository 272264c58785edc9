// The vector-ALU page scan (wn_split.h) at head_dim 128 for every pair of supported
// widths (2, 3, 4, 5, 6, 8 bits for K and for V) that decode.hip does not
// instantiate. These pairs have no tuned kernel; the reference kernel takes any
// pair per call (packed_attention_triton.py:247). One source file per head_dim so
// that they compile beside each other.
#include "wn_split_any.h"

namespace wn {

SplitFn pick_split_any_d128(int bw_k, int bw_v, int nrep) { return any_for<128>(bw_k, bw_v, nrep); }

SplitFn pick_split_any(int D, int bw_k, int bw_v, int nrep) {
  switch (D) {
    case 16: return pick_split_any_d16(bw_k, bw_v, nrep);
    case 32: return pick_split_any_d32(bw_k, bw_v, nrep);
    case 64: return pick_split_any_d64(bw_k, bw_v, nrep);
    case 128: return pick_split_any_d128(bw_k, bw_v, nrep);
    case 256: return pick_split_any_d256(bw_k, bw_v, nrep);
  }
  return nullptr;
}

}  // namespace wn
