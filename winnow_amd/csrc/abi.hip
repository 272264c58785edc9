// Version, error reporting and split planning of the C ABI.
#include <cstdarg>

#include "wn_common.h"

namespace wn {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return WN_E_LAUNCH;
  }
  return WN_OK;
}

}  // namespace wn

extern "C" int wn_abi_version(void) { return WN_ABI_VERSION; }

extern "C" const char* wn_last_error(void) { return wn::g_last_error.c_str(); }

// Work-groups the automatic plan aims for: 256 CUs x ~16 resident waves / 4
// waves per group, so every CU keeps several groups in flight while the
// per-split partials stay a few percent of the page bytes.
static constexpr int64_t kTargetGroups = 4096;

extern "C" int wn_decode_plan(int B, int Hkv, int max_pages, int requested_splits,
                              int* pages_per_split, int* num_splits) {
  wn::clear_error();
  WN_REQUIRE(B >= 0 && Hkv > 0 && max_pages >= 0, WN_E_INVALID,
             "wn_decode_plan: bad sizes B=%d Hkv=%d max_pages=%d", B, Hkv, max_pages);
  WN_REQUIRE(pages_per_split && num_splits, WN_E_INVALID, "wn_decode_plan: null output");
  const int mp = max_pages > 0 ? max_pages : 1;
  if (requested_splits > 0) {
    // packed_attention_triton.py:211-216: splits clamp to [1, max_pages],
    // each covering cdiv(max_pages, splits) page slots.
    int ns = requested_splits < mp ? requested_splits : mp;
    *num_splits = ns;
    *pages_per_split = (mp + ns - 1) / ns;
    return WN_OK;
  }
  int64_t units = int64_t(B > 0 ? B : 1) * Hkv;
  int64_t want = (kTargetGroups + units - 1) / units;
  if (want < 1) want = 1;
  if (want > mp) want = mp;
  int64_t pps = (mp + want - 1) / want;
  if (pps < 16) pps = 16;  // >= 256 tokens at S=16: all four waves of a group busy
  if (pps > mp) pps = mp;
  *pages_per_split = int(pps);
  *num_splits = int((mp + pps - 1) / pps);
  return WN_OK;
}
