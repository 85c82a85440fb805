// wl_gemv_32.hip - decode GEMV codecs of the formats listed at gemv_ops_32.
#include "wl_gemv_launch.h"

namespace wl {

const GemvOps *gemv_ops_32(int) { return nullptr; }

}  // namespace wl
