// wl_gemv_k.hip - decode GEMV codecs of the formats listed at gemv_ops_k.
#include "wl_gemv_launch.h"

namespace wl {

const GemvOps *gemv_ops_k(int) { return nullptr; }

}  // namespace wl
