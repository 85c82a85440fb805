// wl_moe.h - host-side interface of the routed MoE launches.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wl_intdot.h"

namespace wl {

constexpr int MOE_MAX_T = 8;   // tokens per pass (larger batches run in passes of 8)
constexpr int MOE_MAX_K = 16;  // experts per token
constexpr int MOE_MAX_PAIRS = MOE_MAX_T * MOE_MAX_K;

// Device-resident routing plan, written by plan_kernel.
struct MoePlan {
  int nslots;                              // distinct experts chosen (ExpertRuns)
  int slot_expert[MOE_MAX_PAIRS];          // ascending expert ids
  int slot_ntok[MOE_MAX_PAIRS];
  int slot_tok[MOE_MAX_PAIRS][MOE_MAX_T];  // tokens of the slot, ascending
  int slot_pair[MOE_MAX_PAIRS][MOE_MAX_T]; // their pair (hidden/out row) indices
  int tok_pair[MOE_MAX_T][MOE_MAX_K];      // pair of (token, j-th choice)
  float tok_w[MOE_MAX_T][MOE_MAX_K];
  int comb_pair[MOE_MAX_T][MOE_MAX_K];     // a token's pairs, ascending expert id
  float comb_w[MOE_MAX_T][MOE_MAX_K];
};

// Counters of the one-launch MoE (moe_fused_*), two sets used by alternate launches: a launch
// clears the set the next one uses. The flag every workgroup polls is replicated on 64 cache
// lines and the arrivals spread over 16 counters, because the device serialises atomics and
// polls on one address (about 11 ns each). `err` is sticky: a wait that ran out of patience
// (never expected; the workgroup goes on without its inputs and the host reports it).
constexpr int MOE_SYNC_REP = 64;      // replicas of the polled flag
constexpr int MOE_SYNC_SUB = 16;      // arrival counters
constexpr int MOE_SYNC_LINE = 32;     // words per 128-byte line
struct MoeSyncSet {
  unsigned arrive[MOE_SYNC_SUB * MOE_SYNC_LINE];
  unsigned top[MOE_SYNC_LINE];
  unsigned h_ready[MOE_SYNC_REP * MOE_SYNC_LINE];
};
struct MoeSync {
  MoeSyncSet set[2];
  unsigned err[MOE_SYNC_LINE];
};

struct MoeGemvArgs {
  const MoePlan *plan;
  const uint8_t *w, *w2;
  int64_t row_bytes;
  int rows, cols;
  const float *x;
  int64_t ldx;
  int x_by_pair;  // x rows indexed by pair (down) or by token (gate/up)
  float *y;
  int64_t ldy;
};

struct MoeLaunch {
  const float *logits;  // [T][ne]
  int T, ne, k, renorm;
  int gu_type, d_type;
  const uint8_t *gate, *up, *down;  // stacked expert tensors
  int64_t gu_row_bytes, d_row_bytes;
  int ff, embd;
  const float *x;  // [T][embd]
  float *out;      // [T][embd]
  // scratch
  int *sel;
  float *wts, *prob;  // [T][k], [T][k], [T][ne]
  MoePlan *plan;
  float *h;   // [pairs][ff]
  float *yd;  // [pairs][embd]
  // Transformer.IntDot: gate/up (gu_int) and down (d_int) on the integer kernels, with x
  // quantized into qx and h into qh
  int gu_int, d_int;
  QActsDev qx, qh;
  // counters of the one-launch path (zeroed once when allocated), or null for the launch chain;
  // parity: this launch's set (alternates between one-launch launches); spin: polls a bounded
  // wait makes before it gives up and sets the sticky err word
  MoeSync *sync;
  int parity;
  int spin;
};

// Polls of the one-launch MoE's bounded waits (each poll sleeps about 64 clocks).
constexpr int MOE_SPIN = 1 << 18;

bool moe_supports(int type);
hipError_t route_launch(const float *logits, int T, int n, int k, int renorm, int *sel, float *wts, float *prob,
                        hipStream_t st);
// Whether moe_launch runs m as the one launch (and so uses m.sync's set m.parity and clears
// the other set for the next one-launch launch), rather than the launch chain.
bool moe_uses_one_launch(const MoeLaunch &m);
hipError_t moe_launch(const MoeLaunch &m, int num_cu, hipStream_t st);
// Zeroes a MoeSync once after its allocation (a kernel, so it may sit in a captured stream).
hipError_t moe_sync_init(MoeSync *s, hipStream_t st);

}  // namespace wl
