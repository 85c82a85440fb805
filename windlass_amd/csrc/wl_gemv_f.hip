// wl_gemv_f.hip - decode GEMV codecs of F32, F16 and BF16 rows (wl_codecs2.h), instantiated
// here and handed to gemv_run / moe_launch through GemvOps and MoeOps. Rows whose length is a
// multiple of 2048 take the coalesced wave-column codecs (FWide), others the 32-value runs; the
// choice depends only on the row length, so a token's bits do not depend on the batch.
#include "wl_codecs2.h"
#include "wl_gemv_launch.h"
#include "wl_moe_launch.h"

namespace wl {

template <class Wide, class Runs, int NM>
static hipError_t launch_f(GemvParams &p, int split, int num_cu, hipStream_t st) {
  return p.cols % 2048 == 0 ? launch_tm<Wide, NM>(p, split, num_cu, st) : launch_tm<Runs, NM>(p, split, num_cu, st);
}

template <class Wide, class Runs, int NM>
static hipError_t batch_f(const BatchArgs &a, int num_cu, hipStream_t st) {
  return a.cols % 2048 == 0 ? launch_batch<Wide, NM>(a, num_cu, st) : launch_batch<Runs, NM>(a, num_cu, st);
}

template <class Wide, class Runs, int NM>
static hipError_t moe_f(const MoeGemvArgs &a, int T, int max_slots, int num_cu, hipStream_t st) {
  return a.cols % 2048 == 0 ? launch_moe_tm<Wide, NM>(a, T, max_slots, num_cu, st)
                            : launch_moe_tm<Runs, NM>(a, T, max_slots, num_cu, st);
}

template <class Wide, class Runs>
constexpr GemvOps gemv_ops_float() {
  return GemvOps{{&launch_f<Wide, Runs, 1>, &launch_f<Wide, Runs, 2>}, {&batch_f<Wide, Runs, 1>, &batch_f<Wide, Runs, 2>}};
}

template <class Wide, class Runs>
constexpr MoeOps moe_ops_float() {
  return MoeOps{{&moe_f<Wide, Runs, 1>, &moe_f<Wide, Runs, 2>}};
}

const GemvOps *gemv_ops_f(int type) {
  static constexpr GemvOps f32 = gemv_ops_float<F32w, F32c>(), f16 = gemv_ops_float<F16w, F16c>(),
                           bf16 = gemv_ops_float<BF16w, BF16c>();
  switch (type) {
    case 0: return &f32;
    case 1: return &f16;
    case 30: return &bf16;
  }
  return nullptr;
}

const MoeOps *moe_ops_f(int type) {
  static constexpr MoeOps f32 = moe_ops_float<F32w, F32c>(), f16 = moe_ops_float<F16w, F16c>(),
                          bf16 = moe_ops_float<BF16w, BF16c>();
  switch (type) {
    case 0: return &f32;
    case 1: return &f16;
    case 30: return &bf16;
  }
  return nullptr;
}

}  // namespace wl
