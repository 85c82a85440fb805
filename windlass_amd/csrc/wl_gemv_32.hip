// wl_gemv_32.hip - decode GEMV codecs of the 32-value block formats Q4_0, Q4_1, Q5_0, Q5_1 and
// IQ4_NL (wl_codecs2.h), instantiated here and handed to gemv_run through GemvOps.
#include "wl_codecs2.h"
#include "wl_gemv_launch.h"
#include "wl_moe_launch.h"

namespace wl {

const GemvOps *gemv_ops_32(int type) {
  static constexpr GemvOps q40 = gemv_ops_of<Q40>(), q41 = gemv_ops_of<Q41>(), q50 = gemv_ops_of<Q50>(),
                           q51 = gemv_ops_of<Q51>(), iq4nl = gemv_ops_of2<IQ4NL, IQ4NLR>();
  switch (type) {
    case 2: return &q40;
    case 3: return &q41;
    case 6: return &q50;
    case 7: return &q51;
    case 20: return &iq4nl;
  }
  return nullptr;
}

const MoeOps *moe_ops_32(int type) {
  static constexpr MoeOps q40 = moe_ops_of<Q40>(), q41 = moe_ops_of<Q41>(), q50 = moe_ops_of<Q50>(), q51 = moe_ops_of<Q51>(), iq4nl = moe_ops_of<IQ4NL>();
  switch (type) {
    case 2: return &q40;
    case 3: return &q41;
    case 6: return &q50;
    case 7: return &q51;
    case 20: return &iq4nl;
  }
  return nullptr;
}

}  // namespace wl
