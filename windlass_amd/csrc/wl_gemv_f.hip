// wl_gemv_f.hip - decode GEMV codecs of F32, F16 and BF16 rows (wl_codecs2.h), instantiated
// here and handed to gemv_run through GemvOps.
#include "wl_codecs2.h"
#include "wl_gemv_launch.h"
#include "wl_moe_launch.h"

namespace wl {

const GemvOps *gemv_ops_f(int type) {
  static constexpr GemvOps f32 = gemv_ops_of<F32c>(), f16 = gemv_ops_of<F16c>(), bf16 = gemv_ops_of<BF16c>();
  switch (type) {
    case 0: return &f32;
    case 1: return &f16;
    case 30: return &bf16;
  }
  return nullptr;
}

const MoeOps *moe_ops_f(int type) {
  static constexpr MoeOps f32 = moe_ops_of<F32c>(), f16 = moe_ops_of<F16c>(), bf16 = moe_ops_of<BF16c>();
  switch (type) {
    case 0: return &f32;
    case 1: return &f16;
    case 30: return &bf16;
  }
  return nullptr;
}

}  // namespace wl
