// wl_gemv_f.hip - decode GEMV codecs of the formats listed at gemv_ops_f.
#include "wl_gemv_launch.h"

namespace wl {

const GemvOps *gemv_ops_f(int) { return nullptr; }

}  // namespace wl
