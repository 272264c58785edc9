// Instantiation helpers of the vector-ALU scan for what decode.hip does not
// instantiate (decode_split_any{16,32,64,128,256}.hip).
#pragma once

#include "wn_split.h"

namespace wn {
namespace {

// The pairs decode.hip's pick_split instantiates itself (head_dim 64 and 128 only).
template <int D, int BWK, int BWV>
constexpr bool tuned_pair() {
  return ((D == 64 || D == 128) && BWK == BWV) ||
         (D == 128 && ((BWK == 4 && BWV == 6) || (BWK == 6 && BWV == 4) || (BWK == 4 && BWV == 8)));
}

template <int D, int BWK, int BWV>
SplitFn any_pair(int nrep) {
  if constexpr (tuned_pair<D, BWK, BWV>()) {
    return nullptr;
  } else {
    return pick_nrep<D, BWK, BWV>(nrep);
  }
}

template <int D, int BWK>
SplitFn any_for_k(int bwv, int nrep) {
  switch (bwv) {
    case 2: return any_pair<D, BWK, 2>(nrep);
    case 3: return any_pair<D, BWK, 3>(nrep);
    case 4: return any_pair<D, BWK, 4>(nrep);
    case 5: return any_pair<D, BWK, 5>(nrep);
    case 6: return any_pair<D, BWK, 6>(nrep);
    case 8: return any_pair<D, BWK, 8>(nrep);
  }
  return nullptr;
}

// K widths 2-4 and 5-8 separately, so that a large head_dim compiles in two files.
template <int D>
SplitFn any_for_lo(int bwk, int bwv, int nrep) {
  switch (bwk) {
    case 2: return any_for_k<D, 2>(bwv, nrep);
    case 3: return any_for_k<D, 3>(bwv, nrep);
    case 4: return any_for_k<D, 4>(bwv, nrep);
  }
  return nullptr;
}
template <int D>
SplitFn any_for_hi(int bwk, int bwv, int nrep) {
  switch (bwk) {
    case 5: return any_for_k<D, 5>(bwv, nrep);
    case 6: return any_for_k<D, 6>(bwv, nrep);
    case 8: return any_for_k<D, 8>(bwv, nrep);
  }
  return nullptr;
}

template <int D>
SplitFn any_for(int bwk, int bwv, int nrep) {
  switch (bwk) {
    case 2: return any_for_k<D, 2>(bwv, nrep);
    case 3: return any_for_k<D, 3>(bwv, nrep);
    case 4: return any_for_k<D, 4>(bwv, nrep);
    case 5: return any_for_k<D, 5>(bwv, nrep);
    case 6: return any_for_k<D, 6>(bwv, nrep);
    case 8: return any_for_k<D, 8>(bwv, nrep);
  }
  return nullptr;
}

}  // namespace
}  // namespace wn
