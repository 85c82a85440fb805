// wl_gemv_k.hip - decode GEMV codecs of the K-quants Q2_K, Q3_K and Q5_K (wl_codecs2.h),
// instantiated here and handed to gemv_run through GemvOps.
#include "wl_codecs2.h"
#include "wl_gemv_launch.h"
#include "wl_moe_launch.h"

namespace wl {

const GemvOps *gemv_ops_k(int type) {
  static constexpr GemvOps q2k = gemv_ops_of<Q2K>(), q3k = gemv_ops_of<Q3K>(), q5k = gemv_ops_of<Q5K>();
  switch (type) {
    case 10: return &q2k;
    case 11: return &q3k;
    case 13: return &q5k;
  }
  return nullptr;
}

const MoeOps *moe_ops_k(int type) {
  static constexpr MoeOps q2k = moe_ops_of<Q2K>(), q3k = moe_ops_of<Q3K>(), q5k = moe_ops_of<Q5K>();
  switch (type) {
    case 10: return &q2k;
    case 11: return &q3k;
    case 13: return &q5k;
  }
  return nullptr;
}

}  // namespace wl
