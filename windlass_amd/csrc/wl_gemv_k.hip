// wl_gemv_k.hip - decode GEMV codecs of the K-quants Q2_K, Q3_K and Q5_K and of the I-quants
// IQ3_S and IQ2_S (wl_codecs2.h), instantiated here and handed to gemv_run through GemvOps (and
// to the MoE launches through MoeOps).
#include "wl_codecs2.h"
#include "wl_gemv_launch.h"
#include "wl_moe_launch.h"

namespace wl {

// their 4096-column chunks end inside 128-byte lines: split rows interleave their K-chunks
template <>
inline constexpr bool kInterleaved<IQ3S> = true;
template <>
inline constexpr bool kInterleaved<IQ2S> = true;

const GemvOps *gemv_ops_k(int type) {
  static constexpr GemvOps q2k = gemv_ops_of<Q2K>(), q3k = gemv_ops_of<Q3K>(), q5k = gemv_ops_of<Q5K>(),
                           iq3s = gemv_ops_of<IQ3S>(), iq2s = gemv_ops_of<IQ2S>();
  switch (type) {
    case 10: return &q2k;
    case 11: return &q3k;
    case 13: return &q5k;
    case 21: return &iq3s;
    case 22: return &iq2s;
  }
  return nullptr;
}

const MoeOps *moe_ops_k(int type) {
  static constexpr MoeOps q2k = moe_ops_of<Q2K>(), q3k = moe_ops_of<Q3K>(), q5k = moe_ops_of<Q5K>(),
                          iq3s = moe_ops_of<IQ3S>(), iq2s = moe_ops_of<IQ2S>();
  switch (type) {
    case 10: return &q2k;
    case 11: return &q3k;
    case 13: return &q5k;
    case 21: return &iq3s;
    case 22: return &iq2s;
  }
  return nullptr;
}

}  // namespace wl
