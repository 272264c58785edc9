// Instantiation helpers of the vector-ALU scan for the width pairs decode.hip does
// not instantiate (decode_split_any128.hip, decode_split_any64.hip).
#pragma once

#include "wn_split.h"

namespace wn {
namespace {

// The pairs decode.hip's pick_split instantiates itself.
template <int D, int BWK, int BWV>
constexpr bool tuned_pair() {
  return BWK == BWV || (D == 128 && ((BWK == 4 && BWV == 6) || (BWK == 6 && BWV == 4) || (BWK == 4 && BWV == 8)));
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
