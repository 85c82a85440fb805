// wl_gemm_tall.hip - prefill GEMM for prompts of hundreds of tokens over Q4_K / Q6_K rows
// (the batch branch of Transformer.MatMul, src/Transformer.cs:526-536: DecodeRow of a tile of
// weight rows, then FastMath.Block, src/FastMath.cs:216-264), on the bf16 matrix cores.
//
// A workgroup of four waves owns RM weight rows x 512 tokens of y; wave w owns all RM rows of
// tokens 128w .. 128w+127, so its accumulators (RM/32 x 4 tiles of 32 x 32) stay in AGPRs for the
// whole K range and one wave runs per SIMD. K advances in steps of 32:
//   - the RM x 32 weights of the step are decoded once per workgroup (each thread decodes 16
//     values of one row with the reference DecodeRow's fp32 operations, rounds them to bf16 and
//     writes them to LDS, double-buffered), and every wave reads the A operands of its
//     32 x 32 x 16 products from there;
//   - the tokens' B operands never pass through LDS: x is rounded to bf16 once per call into
//     fragment order (32 tokens x 32 columns = 2 x 64 lanes x 16 bytes, contiguous), so each
//     wave loads its own 8 fragments per step with 8 coalesced 1 KB reads straight into
//     registers, one step ahead.
// LDS traffic per step is the decoded tile written once and read by four waves (40 KB for
// RM = 128) against 32 MFMA per wave, and one barrier per step separates a buffer's writes
// from its reads. v_mfma_f32_32x32x16_bf16 issues at about 1.9 PFLOP/s on a whole MI355X where
// the 16 x 16 x 32 form stops at about 1.3 (measured with independent accumulator chains).
//
// Workgroups are numbered so that those sharing a K-chunk and token tile run on the same XCD
// (the dispatcher deals workgroup i to XCD i % 8), where that slice of x stays in one L2.
//
// MFMA operand layout (v_mfma_f32_32x32x16_bf16, checked on the device): lane l holds
// A[row l%32][k 8(l/32) .. +7] and B[k 8(l/32) .. +7][col l%32]; result value q of lane l is
// D[row 8(q/4) + 4(l/32) + q%4][col l%32].
#include "wl_gemm.h"

#include "wl_device.h"

#pragma clang fp contract(off)

namespace wl {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int TN = 512;        // tokens per workgroup
constexpr int TWN = 128;       // tokens per wave
constexpr int TK = 32;         // K per step
constexpr int TLDK = TK + 8;   // padded LDS row: 80 bytes, the 16-byte reads of 8 rows cover the banks once
constexpr int TMAXS = 8;       // K-chunks at most

__device__ __forceinline__ uint32_t pk2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v.x = (__bf16)a;  // round to nearest even (v_cvt_pk_bf16_f32)
  v.y = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// acc += A * B on the matrix cores with acc held in AGPRs (destination = accumulator operand).
// Through the builtin, the register allocator moves the accumulators between AGPRs and VGPRs at
// every step of the unrolled loop (about 47 copies per step). The compiler does not insert the
// wait states around inline assembly that an MFMA's accumulator needs, so every write of the
// accumulators before the first product and every read after the last one is separated from
// the products by mfma_drain(), with agpr_pin() holding the writes before it and the reads after.
__device__ __forceinline__ void mfma_acc(f32x16_t &acc, const uint4 &a, const uint4 &b) {
  const u32x4_t av = __builtin_bit_cast(u32x4_t, a), bv = __builtin_bit_cast(u32x4_t, b);
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(av), "v"(bv));
}

// The accumulator as it stands at this point of the program (an opaque use and redefinition):
// zeros cannot be materialized after it, nor reads hoisted before it.
__device__ __forceinline__ void agpr_pin(f32x16_t &acc) { asm volatile("" : "+a"(acc)); }

// 24 wait states, more than any MFMA result needs before another instruction reads it, and
// nothing scheduled across.
__device__ __forceinline__ void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// ------------------------------------------------------------------ per-format decode
// A block's 8 sub-blocks of 32 values are the 8 steps of 32 columns. Raw holds what one thread
// needs for the 4 steps of one half-block (phase PH = S / 4): its 16 values (h = which 16 of the
// 32) of each step. The decode of a step is cut into small pieces that fit between the products
// (the matrix core runs an MFMA while the wave issues about four independent VALU instructions):
// prep<S, PART> prepares step S's scale terms (PART 0) and its quants, one byte per value
// (PARTs 1..NPREP-1); value<I> is value I (0..15) in fp32 with the reference DecodeRow's
// operations.

// The quants word v, opaque to the compiler, so each value's extraction is one
// v_cvt_f32_ubyteN of the prepared word instead of a shift-and-mask of the raw bytes.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Q4_K, 144 B: d f16 | dmin f16 | scales[12] | qs[128] (src/Quants.cs:332-350). Sub-block S's
// values are the low (S even) or high (S odd) nibbles of qs[32 (S/2) .. +32].
struct TQ4K {
  static constexpr int BYTES = 144, NPREP = 3;
  struct Raw { uint4 hdr, q[2]; };
  struct Dec { float d1, nm1; uint32_t v[4]; };
  template <int PH>
  __device__ static void load(const uint8_t *blk, int h, Raw &r) {
    r.hdr = *reinterpret_cast<const uint4 *>(blk);  // blocks are 16-byte aligned
#pragma unroll
    for (int i = 0; i < 2; i++) r.q[i] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * (2 * PH + i) + 16 * h);
  }
  template <int S, int PART>
  __device__ static void prep(const Raw &r, int, Dec &o) {
    if constexpr (PART == 0) {
      const float d = half_lo(r.hdr.x), dmin = half_hi(r.hdr.x);
      const uint32_t sc[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
      auto B = [&](int i) { return (sc[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
      uint32_t scv, mv;  // get_scale_min_k4 of sub-block S (src/Quants.cs:322-330)
      if constexpr (S < 4) {
        scv = B(S) & 63;
        mv = B(S + 4) & 63;
      } else {
        scv = (B(S + 4) & 0xF) | ((B(S - 4) >> 6) << 4);
        mv = (B(S + 4) >> 4) | ((B(S) >> 6) << 4);
      }
      o.d1 = d * (float)scv;
      o.nm1 = -(dmin * (float)mv);
    } else {
      const uint4 q = r.q[(S / 2) & 1];
      const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 2 * (PART - 1); i < 2 * PART; i++) o.v[i] = opaque((qq[i] >> (4 * (S & 1))) & 0x0F0F0F0Fu);
    }
  }
  // d1 * q - m1 (src/Quants.cs:345-346) as one fma with the same bits: d1 = d * sc and m1 =
  // dmin * m are products of an fp16 and a 6-bit integer (at most 17 significant bits, exact in
  // fp32), so d1 * q (q < 16) is exact too and the reference's one rounding is the subtraction's,
  // the fma's. Non-finite scales give the same infinities and NaNs.
  template <int I>
  __device__ static float value(const Dec &o) {
    return __builtin_fmaf(o.d1, (float)((o.v[I / 4] >> (8 * (I % 4))) & 0xFF), o.nm1);
  }
};

// Q6_K, 210 B: ql[128] | qh[64] | scales int8[16] | d f16 (src/Quants.cs:372-396). Half n of the
// block (128 values) is steps 4n .. 4n+3; in step qq of a half, value l (0..31) is
// ((ql[64n + 32(qq&1) + l] >> 4(qq>>1)) & 15) | ((qh[32n + l] >> 2qq) & 3) << 4, minus 32, times
// d * scales[8n + 2qq + l/16]. Blocks sit at 2-byte alignment: every field offset used here is a
// multiple of 4, so all fields share the block's misalignment and come as aligned dword windows.
struct TQ6K {
  static constexpr int BYTES = 210, NPREP = 5;
  struct Raw { uint32_t l0[5], l1[5], qh[5], sc[3], dw, sh; };
  struct Dec { float ds; uint32_t v[4]; };
  template <int PH>
  __device__ static void load(const uint8_t *blk, int h, Raw &r) {
    gu32 *a = align4_down(blk);
    r.sh = misalign4(blk) * 8;
    const int o0 = (64 * PH + 16 * h) / 4, o1 = (64 * PH + 32 + 16 * h) / 4, oh = (128 + 32 * PH + 16 * h) / 4,
              os = (192 + 8 * PH) / 4;
    const u32x4a4_t a0 = *reinterpret_cast<gu32x4 *>(a + o0);
    const u32x4a4_t a1 = *reinterpret_cast<gu32x4 *>(a + o1);
    const u32x4a4_t ah = *reinterpret_cast<gu32x4 *>(a + oh);
    r.l0[0] = a0.x; r.l0[1] = a0.y; r.l0[2] = a0.z; r.l0[3] = a0.w; r.l0[4] = a[o0 + 4];
    r.l1[0] = a1.x; r.l1[1] = a1.y; r.l1[2] = a1.z; r.l1[3] = a1.w; r.l1[4] = a[o1 + 4];
    r.qh[0] = ah.x; r.qh[1] = ah.y; r.qh[2] = ah.z; r.qh[3] = ah.w; r.qh[4] = a[oh + 4];
    ldw12(a + os, r.sc);
    r.dw = a[208 / 4];
  }
  template <int S, int PART>
  __device__ static void prep(const Raw &r, int h, Dec &o) {
    constexpr int qq = S % 4;
    if constexpr (PART == 0) {
      const float d = r.sh ? half_hi(r.dw) : half_lo(r.dw);
      // scale byte 2qq + h of the half's 8
      const uint32_t scw = __builtin_amdgcn_alignbit(r.sc[qq / 2 + 1], r.sc[qq / 2], r.sh);
      o.ds = d * (float)(int8_t)(scw >> (16 * (qq & 1) + 8 * h));
    } else {
      constexpr int i = PART - 1;  // src/Quants.cs:381-392
      const uint32_t *ql = (qq & 1) ? r.l1 : r.l0;
      const uint32_t lw = __builtin_amdgcn_alignbit(ql[i + 1], ql[i], r.sh);
      const uint32_t hw = __builtin_amdgcn_alignbit(r.qh[i + 1], r.qh[i], r.sh);
      o.v[i] = opaque(((lw >> (4 * (qq >> 1))) & 0x0F0F0F0Fu) | (((hw >> (2 * qq)) & 0x03030303u) << 4));
    }
  }
  template <int I>
  __device__ static float value(const Dec &o) {
    return o.ds * (float)((int)((o.v[I / 4] >> (8 * (I % 4))) & 0xFF) - 32);
  }
};

// ------------------------------------------------------------------ x in fragment order
// xf fragment (j, s), j = token block of 32, s = step of 32 columns, is 2 x 64 lanes x 16 bytes at
// xf + (j * nsteps + s) * 128: half u (columns 16u .. 16u+15 of the step), lane l holds token
// 32j + l%32, columns 32s + 16u + 8(l/32) .. +7 as bf16 (round to nearest even). Tokens past T
// repeat token T - 1 (their results are never stored).
// One workgroup per (token block j, 8 steps): the 32 tokens' 256 columns come in as 1 KB rows
// (a wave reads one row's 256 floats), go through LDS as bf16, and leave as the 8 fragments
// (j, s0 .. s0+7), 16 KB contiguous in xf.
constexpr int FRAG_ROW = 64 + 2;  // uint2 per LDS row: 256 bf16 and a 16-byte pad
__global__ __launch_bounds__(256) void to_frag_kernel(const float *__restrict__ x, int T, int cols,
                                                      uint4 *__restrict__ xf) {
  __shared__ uint2 lds[32 * FRAG_ROW];
  const int nsteps = cols / TK, groups = nsteps / 8;
  const int j = blockIdx.x / groups, s0 = (blockIdx.x % groups) * 8;
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int r = 4 * k + (tid >> 6), c = tid & 63;
    const int t = min(32 * j + r, T - 1);
    const float4 v = reinterpret_cast<const float4 *>(x + (int64_t)t * cols + TK * s0)[c];
    lds[r * FRAG_ROW + c] = make_uint2(pk2(v.x, v.y), pk2(v.z, v.w));
  }
  __syncthreads();
  uint4 *o = xf + ((int64_t)j * nsteps + s0) * 128;
#pragma unroll
  for (int m = 0; m < 4; m++) {
    const int i = tid + 256 * m;  // fragment i / 128 of the 8; piece q = (i / 32) % 4, token l = i % 32
    const int f = i >> 7, q = (i >> 5) & 3, l = i & 31;
    o[i] = *reinterpret_cast<const uint4 *>(&lds[l * FRAG_ROW + 8 * f + 2 * q]);
  }
}

struct TallArgs {
  const uint8_t *w;
  int64_t row_bytes;
  int rows, cols, T;
  int kc;           // columns per K-chunk (whole blocks)
  const uint4 *xf;
  int64_t xf_bytes;
  float *y;         // y, or the chunk partials [S][T][rows] (ldy = rows)
  int64_t ldy, zstride;
  int tiles_m, tiles_n, nwg, remap;
};

typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));

// The wave's view of x: a buffer resource over xf, the byte offset of its first fragment block,
// and the per-lane offset of a fragment load.
struct XView {
  __amdgpu_buffer_rsrc_t rs;
  int base;     // bytes: first token block * nsteps * 2048
  int stride;   // bytes between token blocks: nsteps * 2048
  int vlane;    // lane * 16
};

// Fragment (token block jj of the wave, step s, half u) into registers.
__device__ __forceinline__ uint4 x_frag(const XView &xv, int jj, int s, int u) {
  const u32x4v_t v = __builtin_amdgcn_raw_buffer_load_b128(xv.rs, xv.vlane + u * 1024, xv.base + jj * xv.stride + s * 2048, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <class G, int RM>
struct TallState {
  typename G::Raw raw[2];   // by phase: raw[0] steps 0-3 of a block, raw[1] steps 4-7
  typename G::Dec dec[2];   // the decode state of steps s + 2 (dec[S & 1]) and s + 3
  uint4 b[2][4][2];         // B fragments by step parity, token block of 32, half of the step
  uint4 af[2][2][RM / 32];  // A fragments by step parity, half of the step, row tile of 32
  f32x16_t acc[RM / 32][4];
};

// What a step loads for the steps after it, issued from the product slots.
struct StepMem {
  const XView *xv;
  int s;                 // this step's index in the row
  const uint16_t *ar;    // step s + 1's A tile in LDS (with the lane's offset)
  const uint8_t *wnext;  // the next block's bytes (weights of a half-block ahead), or null
};

// Product K (0..NK-1) of a step, then the work that slot carries:
//   slots 0..7    the next step's B fragment K (x_frag), and value K of step s + 2's decode
//   slots 8..15   the next step's A fragment K - 8 (LDS), and value K
//   slots 16..23  the bf16 pairs; slot 17 a half-block's weight bytes, slot 23 the decoded values
//                 to LDS
//   slots 24..    the preparation of step s + 3's decode
// A scheduling barrier after each slot keeps this order, so every v_mfma is followed by one
// memory instruction and a few independent VALU instructions, which issue while the matrix core
// works, instead of the step opening with sixteen memory instructions and no product.
template <class G, int RM, int S, int K, bool HAS1, bool DEC2, bool DEC3, bool LAST>
__device__ __forceinline__ void step_products(TallState<G, RM> &st, int h, float (&y)[16], uint32_t (&o)[8],
                                              uint16_t *a_out, const StepMem &mem) {
  constexpr int NK = 2 * (RM / 32) * 4;
  static_assert(NK >= 24 + G::NPREP && NK >= 8 + 2 * (RM / 32), "decode and load slots");
  if constexpr (K < NK) {
    constexpr int u = K / ((RM / 32) * 4), i = (K / 4) % (RM / 32), jj = K % 4;
    mfma_acc(st.acc[i][jj], st.af[S & 1][u][i], st.b[S & 1][jj][u]);
    if constexpr (HAS1 && K < 8) st.b[(S + 1) & 1][K >> 1][K & 1] = x_frag(*mem.xv, K >> 1, mem.s + 1, K & 1);
    if constexpr (HAS1 && K >= 8 && K < 8 + 2 * (RM / 32)) {
      constexpr int un = (K - 8) / (RM / 32), in = (K - 8) % (RM / 32);
      st.af[(S + 1) & 1][un][in] = *reinterpret_cast<const uint4 *>(mem.ar + 32 * in * TLDK + 16 * un);
    }
    if constexpr (K == 17 && !LAST) {
      if constexpr (S == 1) G::template load<0>(mem.wnext, h, st.raw[0]);
      if constexpr (S == 5) G::template load<1>(mem.wnext, h, st.raw[1]);
    }
    if constexpr (DEC2 && K < 16) y[K] = G::template value<K>(st.dec[S & 1]);
    if constexpr (DEC2 && K >= 16 && K < 24) o[K - 16] = pk2(y[2 * (K - 16)], y[2 * (K - 16) + 1]);
    if constexpr (DEC2 && K == 23) {  // the decoded values of step s + 2 to LDS
      uint4 *ad = reinterpret_cast<uint4 *>(a_out);
      ad[0] = make_uint4(o[0], o[1], o[2], o[3]);
      ad[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
    if constexpr (DEC3 && K >= 24 && K < 24 + G::NPREP) {
      constexpr int S3 = (S + 3) & 7;
      G::template prep<S3, K - 24>(st.raw[S3 / 4], h, st.dec[(S + 1) & 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    step_products<G, RM, S, K + 1, HAS1, DEC2, DEC3, LAST>(st, h, y, o, a_out, mem);
  }
}

// Step S (0..7) of block blk. Going in, the step's A operands are in registers (af[S & 1]), its B
// operands are loaded or in flight (b[S & 1]), and the decode state of step s + 2 is ready
// (dec[S & 1]). Between its products the step loads the next step's B fragments and A operands
// (from LDS buffer (S + 1) & 3), loads the weight bytes
// of a half-block four steps ahead (at S = 1 and 5), decodes step s + 2 into buffer (S + 2) & 3
// and prepares step s + 3's decode; it ends at the barrier. Buffer (S + 1) & 3 was written
// during step s - 1 and made visible by the barrier that ended it; buffer (S + 2) & 3 held step
// s - 2's operands, read during step s - 3, so one barrier per step orders every LDS write
// against its reads.
// LAST: the row's last block (steps past its end are not prepared).
template <class G, int RM, int S, bool LAST>
__device__ __forceinline__ void tall_step(TallState<G, RM> &st, uint16_t (*As)[128 * TLDK], int blk,
                                          const uint8_t *wblk0, const XView &xv, int s0, int h, int aw, int ao) {
  constexpr int S1 = (S + 1) & 7, S2 = (S + 2) & 7;
  constexpr bool HAS1 = !(LAST && S == 7);  // step s + 1 exists
  constexpr bool HAS2 = !(LAST && S >= 6);  // step s + 2 exists
  constexpr bool HAS3 = !(LAST && S >= 5);  // step s + 3 exists
  StepMem mem{&xv, s0 + 8 * blk + S, As[S1 & 3] + ao, wblk0 + (blk + 1) * G::BYTES};
  float y[16];
  uint32_t o[8];
  __builtin_amdgcn_sched_barrier(0);
  step_products<G, RM, S, 0, HAS1, HAS2, HAS3, LAST>(st, h, y, o, As[S2 & 3] + aw, mem);
  if constexpr (HAS1) __syncthreads();
}

template <class G, int RM, bool LAST>
__device__ __forceinline__ void tall_block(TallState<G, RM> &st, uint16_t (*As)[128 * TLDK], int blk,
                                           const uint8_t *wblk0, const XView &xv, int s0, int h, int aw, int ao) {
  tall_step<G, RM, 0, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 1, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 2, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 3, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 4, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 5, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 6, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
  tall_step<G, RM, 7, LAST>(st, As, blk, wblk0, xv, s0, h, aw, ao);
}

template <class G, int S, int PART>
__device__ __forceinline__ void prep_all(const typename G::Raw &r, int h, typename G::Dec &d) {
  if constexpr (PART < G::NPREP) {
    G::template prep<S, PART>(r, h, d);
    prep_all<G, S, PART + 1>(r, h, d);
  }
}

template <class G, int I>
__device__ __forceinline__ void values_all(const typename G::Dec &d, float (&y)[16]) {
  if constexpr (I < 16) {
    y[I] = G::template value<I>(d);
    values_all<G, I + 1>(d, y);
  }
}

// Decodes step S of the block whose half-block bytes are in r into LDS at ad (the prologue).
template <class G, int S>
__device__ __forceinline__ void decode_step(const typename G::Raw &r, int h, uint16_t *ad) {
  typename G::Dec d;
  prep_all<G, S, 0>(r, h, d);
  float y[16];
  values_all<G, 0>(d, y);
  uint4 *a = reinterpret_cast<uint4 *>(ad);
  a[0] = make_uint4(pk2(y[0], y[1]), pk2(y[2], y[3]), pk2(y[4], y[5]), pk2(y[6], y[7]));
  a[1] = make_uint4(pk2(y[8], y[9]), pk2(y[10], y[11]), pk2(y[12], y[13]), pk2(y[14], y[15]));
}

template <class G, int RM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_tall_kernel(TallArgs p) {
  // a ring of four decoded A tiles, 128 rows each
  __shared__ __attribute__((aligned(16))) uint16_t As[4][128 * TLDK];
  const int wg = blockIdx.x;
  const int jlin = p.remap ? (wg % 8) * (p.nwg / 8) + wg / 8 : wg;
  const int mt = jlin % p.tiles_m, grp = jlin / p.tiles_m;
  const int nt = grp % p.tiles_n, chunk = grp / p.tiles_n;
  const int m0 = mt * RM, n0 = nt * TN;
  const int kb = chunk * p.kc, ke = min(p.cols, kb + p.kc);
  const int nblk = (ke - kb) / 256, nsteps = p.cols / TK;
  float *y = p.y + chunk * p.zstride;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);

  // decoder role: row tid / 2 of the tile, values 16h .. 16h+15 of each step (h = tid % 2). The
  // two lanes of a row read adjacent 16-byte pieces of its block, so a wave's weight load touches
  // 32 rows' lines instead of 64: the texture unit, which also carries every B fragment, spends
  // its time per line.
  const int ar = tid >> 1, h = tid & 1;
  const uint8_t *wblk0 = p.w + (int64_t)min(m0 + ar, p.rows - 1) * p.row_bytes + (int64_t)(kb / 256) * G::BYTES;
  const int aw = ar * TLDK + 16 * h;
  const int ao = (lane & 31) * TLDK + 8 * (lane >> 5);

  // this wave's 4 token blocks jb .. jb+3. Where they pass the last real block (jlast), the wave
  // loads the 4 blocks ending at jlast instead (valid memory; T >= 128) and stores only its own.
  const int jlast = (p.T - 1) / 32, jb = (n0 + TWN * wv) / 32;
  const int jfirst = jb + 3 > jlast ? max(0, jlast - 3) : jb;
  XView xv;
  xv.rs = __builtin_amdgcn_make_buffer_rsrc((void *)p.xf, (short)0, (int)p.xf_bytes, 0x00020000);
  xv.stride = nsteps * 2048;
  xv.base = jfirst * xv.stride;
  xv.vlane = lane * 16;
  const int s0 = kb / TK;

  TallState<G, RM> st;
#pragma unroll
  for (int i = 0; i < RM / 32; i++)
#pragma unroll
    for (int jj = 0; jj < 4; jj++)
#pragma unroll
      for (int q = 0; q < 16; q++) st.acc[i][jj][q] = 0.f;
#pragma unroll
  for (int i = 0; i < RM / 32; i++)
#pragma unroll
    for (int jj = 0; jj < 4; jj++) agpr_pin(st.acc[i][jj]);
  mfma_drain();  // the zeroed accumulators before the first product reads them

  if (nblk > 0) {
    // steps 0 and 1 decoded into buffers 0 and 1, step 2's decode prepared, step 0's operands in
    // registers
    G::template load<0>(wblk0, h, st.raw[0]);
    G::template load<1>(wblk0, h, st.raw[1]);
#pragma unroll
    for (int jj = 0; jj < 4; jj++)
#pragma unroll
      for (int u = 0; u < 2; u++) st.b[0][jj][u] = x_frag(xv, jj, s0, u);
    decode_step<G, 0>(st.raw[0], h, As[0] + aw);
    decode_step<G, 1>(st.raw[0], h, As[1] + aw);
    prep_all<G, 2, 0>(st.raw[0], h, st.dec[0]);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int i = 0; i < RM / 32; i++)
        st.af[0][u][i] = *reinterpret_cast<const uint4 *>(As[0] + ao + 32 * i * TLDK + 16 * u);
    for (int blk = 0; blk < nblk - 1; blk++) tall_block<G, RM, false>(st, As, blk, wblk0, xv, s0, h, aw, ao);
    tall_block<G, RM, true>(st, As, nblk - 1, wblk0, xv, s0, h, aw, ao);
  }
  mfma_drain();
#pragma unroll
  for (int i = 0; i < RM / 32; i++)
#pragma unroll
    for (int jj = 0; jj < 4; jj++) agpr_pin(st.acc[i][jj]);

  // value q of tile (i, jj): row 32i + 8(q/4) + 4(l/32) + q%4, token 32jj + l%32 (of the wave's 128)
#pragma unroll
  for (int jj = 0; jj < 4; jj++) {
    const int t = 32 * (jfirst + jj) + (lane & 31);
    const bool own = jfirst + jj >= jb;  // a block of this wave (jfirst + jj < jb + 4 always)
    if (t < p.T && own) {
#pragma unroll
      for (int i = 0; i < RM / 32; i++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int r0 = m0 + 32 * i + 8 * g + 4 * (lane >> 5);
          float *yp = y + (int64_t)t * p.ldy + r0;
          if (r0 + 3 < p.rows) {
            yp[0] = st.acc[i][jj][4 * g];
            yp[1] = st.acc[i][jj][4 * g + 1];
            yp[2] = st.acc[i][jj][4 * g + 2];
            yp[3] = st.acc[i][jj][4 * g + 3];
          } else {
#pragma unroll
            for (int q = 0; q < 4; q++)
              if (r0 + q < p.rows) yp[q] = st.acc[i][jj][4 * g + q];
          }
        }
    }
  }
}

// y = the S chunk partials added in chunk order. V = 4: rows, ldy and y's address are multiples of
// 4 floats, and each thread adds four adjacent outputs with 16-byte loads and stores.
template <int V>
__global__ __launch_bounds__(256) void tall_combine_kernel(const float *__restrict__ part, int S, int T, int rows,
                                                           float *__restrict__ y, int64_t ldy) {
  typedef float fv_t __attribute__((ext_vector_type(V)));
  const int64_t plane = (int64_t)T * rows / V, rv = rows / V;
  const fv_t *pv = reinterpret_cast<const fv_t *>(part);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < plane; i += (int64_t)gridDim.x * blockDim.x) {
    fv_t s = pv[i];
    for (int c = 1; c < S; c++) s += pv[c * plane + i];  // chunk order
    const int64_t t = i / rv, r = i % rv;
    *reinterpret_cast<fv_t *>(y + t * ldy + r * V) = s;
  }
}

struct TallPlan {
  int rm, tiles_m, tiles_n, S, kc;
};

TallPlan tall_plan(int rows, int cols, int T, int num_cu) {
  TallPlan pl;
  pl.tiles_n = (T + TN - 1) / TN;
  pl.rm = 128;
  pl.tiles_m = (rows + pl.rm - 1) / pl.rm;
  const int tiles = pl.tiles_m * pl.tiles_n, nblk = cols / 256;
  int S = 1;
  if (tiles * 8 < num_cu * 7) {  // fewer tiles than 7/8 of the CUs: split K in whole blocks
    S = (num_cu + tiles - 1) / tiles;
    if (S > TMAXS) S = TMAXS;
    if (S > nblk) S = nblk;
    const int per = (nblk + S - 1) / S;
    S = (nblk + per - 1) / per;
  }
  pl.S = S;
  pl.kc = (nblk + S - 1) / S * 256;
  return pl;
}

}  // namespace

// Q4_K and Q6_K prompts whose last 512-token tile is at least 3/4 full.
// Q4_K and Q6_K prompts of 128 tokens and more (a wave whose token blocks pass the last one reads
// the four blocks ending there, so four must exist). A tile of fewer than 512 tokens costs about
// a full one, and is still faster than the 256-token tiles of gemm_kernel: 28672x8192 Q4_K at 128,
// 256 and 320 tokens 226, 272 and 393 us there, 186, 192 and 195 us here.
bool gemm_tall_applies(int type, int T) { return T >= 128 && (type == 12 || type == 14); }

int64_t gemm_tall_scratch_bytes(int rows, int cols, int T, int num_cu) {
  const TallPlan pl = tall_plan(rows, cols, T, num_cu);
  const int64_t xf = (int64_t)((T + 31) / 32) * 32 * cols * 2;
  return xf + (pl.S > 1 ? (int64_t)pl.S * T * rows * 4 : 0);
}

hipError_t gemm_tall_launch(int type, const uint8_t *w, int64_t row_bytes, int rows, int cols, const float *x, int T,
                            float *y, int ldy, void *scratch, int num_cu, hipStream_t st) {
  if (rows <= 0 || T <= 0) return hipSuccess;
  if (cols <= 0 || cols % 256 || !scratch) return hipErrorInvalidValue;
  const TallPlan pl = tall_plan(rows, cols, T, num_cu);
  const int64_t nfrag = (int64_t)((T + 31) / 32) * (cols / TK) * 128;
  uint4 *xf = reinterpret_cast<uint4 *>(scratch);
  hipLaunchKernelGGL(to_frag_kernel, dim3((unsigned)((T + 31) / 32 * (cols / 256))), dim3(256), 0, st, x, T, cols, xf);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  float *part = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(scratch) + nfrag * 16);
  TallArgs a;
  a.w = w;
  a.row_bytes = row_bytes;
  a.rows = rows;
  a.cols = cols;
  a.T = T;
  a.kc = pl.kc;
  a.xf = xf;
  a.xf_bytes = nfrag * 16;
  a.tiles_m = pl.tiles_m;
  a.tiles_n = pl.tiles_n;
  a.nwg = pl.tiles_m * pl.tiles_n * pl.S;
  a.remap = a.nwg % 8 == 0;
  if (pl.S == 1) {
    a.y = y;
    a.ldy = ldy;
    a.zstride = 0;
  } else {
    a.y = part;
    a.ldy = rows;
    a.zstride = (int64_t)T * rows;
  }
  const dim3 grid((unsigned)a.nwg), block(256);
  if (type == 12) hipLaunchKernelGGL((gemm_tall_kernel<TQ4K, 128>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((gemm_tall_kernel<TQ6K, 128>), grid, block, 0, st, a);
  e = hipGetLastError();
  if (e != hipSuccess || pl.S == 1) return e;
  const bool v4 = rows % 4 == 0 && ldy % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
  int64_t gc = ((int64_t)T * rows / (v4 ? 4 : 1) + 255) / 256;
  if (gc > 8192) gc = 8192;
  if (v4)
    hipLaunchKernelGGL(tall_combine_kernel<4>, dim3((unsigned)gc), dim3(256), 0, st, part, pl.S, T, rows, y,
                       (int64_t)ldy);
  else
    hipLaunchKernelGGL(tall_combine_kernel<1>, dim3((unsigned)gc), dim3(256), 0, st, part, pl.S, T, rows, y,
                       (int64_t)ldy);
  return hipGetLastError();
}

}  // namespace wl
