// The decode-step MoE block of one TP rank on gfx950 (MI355X): HIP kernels and the C ABI.
//
// One persistent launch (grid = one 512-thread workgroup per CU) runs its stages
// separated by hand-offs: a workgroup that is done with a stage sets its own flag word
// (a device-coherent store), and a waiter reads all the flags until every one is set
// (every wait has a deadline, so a launch always ends):
//   N  RMSNorm of x (fused-norm shape only)                   wave per row
//   A  router GEMV part sums (fixed order) + activation quantization
//                                                              wave per (expert, K part) / (row, 512 cols)
//   B  routing (sigmoid, grouped top-k, weights): up to 8 rows every workgroup routes the
//      whole step itself, reading the part sums as they land; above 8 a workgroup a row
//   C  gate_up + SwiGLU of the step's union of experts and of the shared expert, dealt
//      as one list of units over the workgroups
//   D  down GEMMs (routed + shared) and the weighted combine   workgroup per tile of output rows
// The expert GEMMs run on bf16 MFMA by default (e4m3 / e2m1 codes converted to bf16 exactly;
// the sums are held to the numerics bounds); a per-call option selects the fixed-order VALU
// GEMVs (see WRows), whose output a CPU restatement reproduces bit for bit. Routing is
// computed in one fixed fp32 / fp64 order on every path and is bit-identical to the oracle.
// Hand-off data between workgroups is written and read with device-coherent (sc1) buffer
// accesses, so the flags need no L2 write-back / invalidate.
// The staged entry point runs the same stage functions as one launch each.
//
// Reference: the stages of sgl_amd_mono/deepseek_v41/gfx950/stages/moe.py
// (run_moe :1348-1418; stage_xq :181-263; stage_router :267-301; stage_route
// :305-391; load_route :394-489; stage_shared :502-563; stage_ug :770-832 and
// ug_epilogue :907-947; stage_down :950-1005; down_combine :1156-1184) and
// the fused norm of stages/seam.py:325-378. The weights are read in place in
// the checkpoint's row-major layouts (include/mkmoe.h).

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>

#include <mutex>
#include <type_traits>

#include "../../include/mkmoe.h"
#include "mkmoe_numerics.h"

// Built whole, or in parts (MKMOE_UNIT = 0 .. 7: one compiled shape's kernels and launcher;
// MKMOE_UNIT_HOST: the host code and the C ABI), so that the parts compile in parallel.
#define MKMOE_UNIT_HOST 9

namespace mkmoe {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kRowsMax = 48;   // rows a launch takes at most
constexpr int kTileMax = 32;   // output rows of a down tile, at most
// ... of a shape: a workgroup's share of H at the full grid (H / 256, a multiple of 4); with
// fewer workgroups a workgroup takes more tiles, not larger ones (the host caps them alike)
constexpr int tile_max(int h) {
  return ((h + 255) / 256 + 3) / 4 * 4 < kTileMax ? ((h + 255) / 256 + 3) / 4 * 4 : kTileMax;
}
constexpr int kFp8 = MKMOE_FMT_FP8_B128;
constexpr int kFp4 = MKMOE_FMT_MXFP4;
constexpr int kFp4Aiter = MKMOE_FMT_MXFP4_AITER;  // MXFP4 in SGLang's loaded (aiter-shuffled) layout
// e4m3 with E8M0 32 x 32 block scales (the V4.1 shared expert), fed by MXFP8 of the "vllm" rule;
// as a quantizer's format argument it selects that rule
constexpr int kFp8Mx = MKMOE_FMT_FP8_MX32;
constexpr int kScoreSigmoid = MKMOE_SCORE_SIGMOID, kScoreSqrtSoftplus = MKMOE_SCORE_SQRT_SOFTPLUS;
constexpr int kAuxDev = 16;  // sc1: device-coherent access
constexpr int kAuxNt = 2;    // nt: streamed once

// control words at the start of the workspace: the exit count, the error words; then, from
// byte kCtlFlags, a flag array per hand-off (a word per workgroup: set on arrival, clear
// between launches)
// hand-offs (flag arrays): N normed x, A router and x codes, B routing, C the gate_up, Q the
// intermediates quantized (the last)
constexpr int kCtlNorm = 0, kCtlA = 1, kCtlB = 2, kCtlC = 3, kCtlQ = 4;
constexpr int kCtlExit = 5;
constexpr int kCtlErr = 8;  // MKMOE_ERRW_WORDS error words from here
constexpr int kFlagWgs = 256;  // workgroups a persistent launch has at most
constexpr int kCtlFlags = 256;
constexpr int kCtlBytes = kCtlFlags + 5 * kFlagWgs * 4;

enum Stage { kStageNorm = 1, kStageA = 2, kStageB = 3, kStageC = 4, kStageD = 5, kStageQ = 6 };

// ---------------------------------------------------------------- timeline (diagnostic build)
// Built with MKMOE_TIMELINE, the persistent launch stamps s_memrealtime (100 MHz) into LDS at
// each phase end of each workgroup and writes the stamps out once at its end (workspace region
// 11: [workgroup][kTlSlots] u64: phase ends, then summed durations), so the stamps add no memory waits. Other builds compile the
// stamps away and leave region 11 untouched.
enum TlSlot {
  kTlStart = 0, kTlADone, kTlAArrived, kTlRouted, kTlUnion, kTlAAwaited, kTlGateUp, kTlCArrived,
  kTlCAwaited, kTlDRouted, kTlDShared, kTlEnd, kTlGuFirst, kTlGuWait, kTlDWait, kTlGuUnits,
  // a gate_up unit's parts, summed over the workgroup's units (wave 0): read out of the slot
  // and the next unit requested, the MFMAs, the partial-tile sync, the emit, the closing sync
  kTlGuFetch, kTlGuMma, kTlGuSync, kTlGuEmit, kTlGuSync2,
  // the routed down's parts (wave 0): quantizing the pick batches, the units' MFMAs
  kTlDQuant, kTlDMma,
  // local routing (thread 0): its wave's part sums all landed, the scores of the step in LDS
  kTlParts, kTlScores,
  // the workgroup's share of the quantize stage done, and the Q hand-off passed
  kTlQDone, kTlQAwaited,
  // the routed down's other parts (wave 0): a unit read out of its slot, the next unit
  // requested, the units counted; and the end of its first unit
  kTlDFetch, kTlDIssue, kTlDUnits, kTlDFirst,
  // the routed down's waits at the pick batches' first barrier (wave 0)
  kTlDBar,
  kTlSlots = 32
};
#ifdef MKMOE_TIMELINE
static __shared__ unsigned long long s_tl[kTlSlots];
__device__ __forceinline__ unsigned long long tl_now() { return __builtin_amdgcn_s_memrealtime(); }
// thread 0 stamps phase k
#define TL(k) do { if (threadIdx.x == 0) s_tl[(k)] = __builtin_amdgcn_s_memrealtime(); } while (0)
// thread 0 adds v to slot k
#define TL_ADD(k, v) do { if (threadIdx.x == 0) s_tl[(k)] += (v); } while (0)
#define TL_CLEAR() do { if (threadIdx.x < kTlSlots) s_tl[threadIdx.x] = 0ull; } while (0)
#define TL_DUMP(p) do { __syncthreads(); if (threadIdx.x < kTlSlots) ((unsigned long long*)((p).ws + (p).off[11]))[blockIdx.x * kTlSlots + threadIdx.x] = s_tl[threadIdx.x]; } while (0)
#else
__device__ __forceinline__ unsigned long long tl_now() { return 0ull; }
#define TL(k) do {} while (0)
#define TL_ADD(k, v) do {} while (0)
#define TL_CLEAR() do {} while (0)
#define TL_DUMP(p) do {} while (0)
#endif

template <int H_, int E_, int K_, int NG_, int TG_, int I_, int S_, int FMT_, int P_, bool NORM_, bool SHUF_ = false,
          int SCORE_ = kScoreSigmoid, int SFMT_ = kFp8, int IR_ = I_>
struct Cfg {
  static constexpr int SCORE = SCORE_;  // the router's score (sigmoid or V4.1's sqrt(softplus))
  // the shared expert's weights: FP8 with fp32 128 x 128 scales (its activations and
  // intermediate quantized per 128, fp32 scales), or with E8M0 32 x 32 scales (V4.1: MXFP8 of
  // the "vllm" rule)
  static constexpr int SFMT = SFMT_;
  static_assert(SFMT == kFp8 || SFMT == kFp8Mx, "shared formats");
  static constexpr int H = H_, E = E_, K = K_, NG = NG_, TG = TG_, I = I_, S = S_, FMT = FMT_,
                       P = P_;
  static constexpr bool NORM = NORM_;
  // MXFP4 routed experts in SGLang's loaded gfx950 layout (aiter's (16, 16) shuffle, w13's
  // 16-row gate/up interleave, scales in shuffle_scale order), read in place; such shapes run
  // every expert GEMM on MFMA (the VALU GEMVs read row-major rows)
  static constexpr bool SHUF = SHUF_;
  static_assert(!SHUF || FMT == kFp4, "the shuffled layout is MXFP4's");
  // a routed expert's real width when the loader pads it with zero weights to I (V4.1: the
  // rank's 576 columns padded to 640, stages/dims.py:13-46). The padding is never read: the
  // gate_up computes the real columns only, the intermediates are quantized from the real
  // columns (zeros past them), and the down loads no weight past K = IR (as the reference's
  // ug tasks and down tiles skip it, stages/moe.py:696-714,788-793,1065-1093). MFMA shapes
  // alone (the shuffled layout)
  static constexpr int IR = IR_;
  static_assert(IR == I || (SHUF && IR % 32 == 0 && IR < I), "real width: whole MX blocks");
  // launches of at least QROWS rows quantize the intermediates once (stage Q, a hand-off of
  // its own) instead of in every workgroup's down stage, and up to shared_mid_rows<C>() rows run
  // the shared expert's down inside that hand-off. Measured: 7-8 % faster at 48 rows, 1.4 to
  // 4 us faster at 8 rows (MXFP4 at I = 512 gains only with the shared down inside the
  // hand-off), 0.3-2 us slower at 1 and 2 rows (the hand-off costs more than the work it saves).
  // From 6 rows where each workgroup's own quantize of the picks costs more (FP8's group-128
  // rule, or I of 1024 and more): at 6 / 7 rows cfg 2 -1.2 / -1.1 us, cfg 5 -3.0 / -3.1, V4.1
  // TP2 -0.9 / -1.2, where cfg 3 (+1.7 / +1.2) and V4.1 TP4 (+2.3 / +2.3) lost (measured)
  static constexpr int QROWS = FMT == kFp8 || I >= 1024 ? 6 : 8;
  static constexpr int CH512 = H / 512;  // router / quantize chunks of a row
  static_assert(H % 1024 == 0 && CH512 % P == 0, "router chunks, K split over 8 waves");
  // (an MX shared expert's width may end in half a 128-K step: V4.1's 2304 / 4 = 576)
  static_assert(I % 128 == 0 && (SFMT == kFp8Mx ? S % 64 == 0 : S % 128 == 0), "widths");
  static_assert(E <= 1024 && (NG == 1 || (E % NG == 0)), "experts");
  // down-stage mid batch: picks whose quantized rows fit ~32 KB of LDS
  static constexpr int PB = 32768 / I;
  static constexpr int MQS = I + 16;  // LDS row stride of quantized mid (bank spread)
  static constexpr int SQS = S + 16;
  static constexpr int SSC = SFMT == kFp8Mx ? S / 32 : (S / 128) * 4;  // scale bytes of a shared row
  static constexpr int MSC = FMT == kFp4 ? I / 32 : I / 128;  // mid scales a pick
  // 16-row blocks of a routed down unit: MXFP4 rows of 512 K are 256 bytes, so a unit of 32 rows
  // keeps 8 KB a wave in flight (as 16 rows do at FP8, or at MXFP4 with 1024 K). At 640 K
  // (V4.1) a tile is H / 256 = 20 rows: one 32-row unit of 10 KB covers it, where 16-row units
  // took two, the second with 4 rows at a whole unit's latency
  static constexpr int DNA = FMT == kFp4 && I <= 640 ? 2 : 1;
  static constexpr int TMAX = tile_max(H);  // output rows of a down tile, at most
};

using CfgPlumbing = Cfg<1024, 16, 4, 1, 1, 512, 512, kFp8, 2, false>;
using CfgTp4Fp8 = Cfg<7168, 256, 8, 8, 4, 512, 512, kFp8, 7, false>;
using CfgTp4Fp4 = Cfg<7168, 256, 8, 8, 4, 512, 512, kFp4, 7, false>;
using CfgTp2Fp4Norm = Cfg<7168, 256, 8, 8, 4, 1024, 1024, kFp4, 7, true>;
using CfgTp4Fp4Aiter = Cfg<7168, 256, 8, 8, 4, 512, 512, kFp4, 7, false, true>;
using CfgTp2Fp4NormAiter = Cfg<7168, 256, 8, 8, 4, 1024, 1024, kFp4, 7, true, true>;
// the plumbing shape routed as V4.1 routes (sqrt(softplus) scores, one group)
using CfgPlumbingSoftplus = Cfg<1024, 16, 4, 1, 1, 512, 512, kFp8, 2, false, false, kScoreSqrtSoftplus>;
// DeepSeek-V4.1's MoE at TP4 (stages/moe_shape.py:24, stages/dims.py:13-56, check_ffn.py:13-18):
// hidden 5120, 384 experts top-6 by sqrt(softplus) over one group, routed experts MXFP4 in
// SGLang's aiter layout with the rank's 576 columns padded to 640 (zero weights), the shared
// expert's 576 columns FP8 with E8M0 32 x 32 scales
using CfgV41Tp4 = Cfg<5120, 384, 6, 1, 1, 640, 576, kFp4, 5, false, true, kScoreSqrtSoftplus, kFp8Mx, 576>;
// ... at TP2: the rank's 1152 routed and 1152 shared columns (a multiple of 128: no padding)
using CfgV41Tp2 = Cfg<5120, 384, 6, 1, 1, 1152, 1152, kFp4, 5, false, true, kScoreSqrtSoftplus, kFp8Mx>;

// the expert GEMMs of a launch on MFMA (else the VALU GEMVs)
template <class C>
__device__ __forceinline__ bool gate_on_mfma(int rows, int mfma_gate) { return C::SHUF || rows >= mfma_gate; }
template <class C>
__device__ __forceinline__ bool down_on_mfma(int rows, int mfma_down) { return C::SHUF || rows >= mfma_down; }

// ---------------------------------------------------------------- workspace layout
constexpr int kRegions = 16;

struct Layout {
  size_t off[kRegions];
  size_t size[kRegions];
  size_t total;
};

MKMOE_HD inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

MKMOE_HD inline Layout make_layout(int H, int E, int K, int I, int S, int fmt, int P, int norm,
                                   int rm, int sfmt = kFp8) {
  Layout L;
  size_t sz[kRegions];
  sz[0] = norm ? (size_t)rm * H * 2 : 0;                              // x normed, bf16
  sz[1] = (size_t)rm * H;                                             // x codes, routed rule
  sz[2] = fmt == kFp4 ? (size_t)rm * (H / 32) : (size_t)rm * (H / 128) * 4;  // its scales
  sz[3] = fmt == kFp4 ? (size_t)rm * H : 0;                           // x codes, shared rule
  sz[4] = fmt == kFp4 ? (size_t)rm * (H / 128) * 4 : 0;               // its fp32 scales
  sz[5] = (size_t)rm * E * P * 4;                                     // router part sums
  sz[6] = (size_t)rm * K * 4;                                         // ids
  sz[7] = (size_t)rm * K * 4;                                         // weights
  sz[8] = (size_t)rm * S * 2;                                         // shared mid, bf16
  sz[9] = (size_t)rm * K * I * 2;                                     // routed mid, bf16
  sz[10] = sz[5];  // the part sums as routing polls them (kPartUnset between launches)
  sz[11] = (size_t)kFlagWgs * kTlSlots * 8;  // the timeline build's stamps
  // the intermediates quantized once (stage Q), in the rows' LDS layout: the routed picks in
  // the union's order, codes [R k][I + 16] and scales (MXFP8: E8M0 [R k][I / 32]; FP8: fp32
  // [R k][I / 128]); the shared rows, codes [R][S + 16] and fp32 scales [R][S / 128]
  sz[12] = (size_t)rm * K * (I + 16);
  sz[13] = (size_t)rm * K * (fmt == kFp4 ? I / 32 : (I / 128) * 4);
  sz[14] = (size_t)rm * (S + 16);
  sz[15] = (size_t)rm * (sfmt == kFp8Mx ? S / 32 : (S / 128) * 4);
  size_t off = kCtlBytes;
  for (int i = 0; i < kRegions; ++i) {
    L.off[i] = off;
    L.size[i] = sz[i];
    off = align256(off + sz[i]);
  }
  L.total = off;
  return L;
}

struct Params {
  const uint16_t* x;
  uint16_t* out;
  int32_t* ids_out;
  float* w_out;
  const uint16_t* gate_w;
  const float* bias;
  const uint16_t* norm_w;
  const uint8_t* w13;
  const void* w13_s;
  const uint8_t* w2;
  const void* w2_s;
  const uint8_t* sgu;
  const float* sgu_s;
  const uint8_t* sw2;
  const float* sw2_s;
  uint8_t* ws;
  uint32_t ws_bytes;
  int rows;
  int rmax;
  int renorm;
  int tile_rows;
  int mfma_gate;  // launches with at least this many rows run the gate_up GEMMs on MFMA
  int mfma_down;  // ... and the down GEMMs
  int mx_scaled;       // the MXFP4 gate_up GEMMs on the scaled fp4 x fp8 MFMA (no converts)
  int mx_scaled_down;  // and the MXFP4 down GEMMs
  float scale;
  float limit;
  float eps;
  unsigned long long deadline;  // s_memrealtime ticks (100 MHz)
  int fault_stage;              // test fault injection: the stage whose wait workgroup fault_wg
  int fault_wg;                 // stalls to its deadline (0: none)
  uint32_t off[kRegions];
};

// ---------------------------------------------------------------- small device helpers
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}

// a weight of n bytes as a buffer resource; a load at an offset past n returns zeros without a
// memory access
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const void* w, uint32_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(w), (short)0, (int)n, 0x00020000);
}
constexpr uint32_t kNoLoad = 0xF0000000u;  // an offset past every weight resource
typedef int i32x4 __attribute__((ext_vector_type(4)));
// A wait for all of the wave's vector memory loads (vmcnt 0), placed as the compiler's own
// wait, so that it knows every register loaded before it is ready. Its own waits for loads
// issued before an asm wait would count the loads issued after it as well (they complete in
// order): a register loaded before a unit's wait, used after the next unit's rows are
// requested, would then wait for those rows.
__device__ __forceinline__ void wait_vm0() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 fields: vmcnt 0, expcnt 7 (none), lgkmcnt 15 (none)
  asm volatile("" ::: "memory");
}

// a weight of n bytes as the four scalar words of a buffer resource (for lds_dma16)
__device__ __forceinline__ i32x4 weight_rsrc_words(const void* w, uint32_t n) {
  const unsigned long long a = (unsigned long long)w;
  return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffffu)),
               __builtin_amdgcn_readfirstlane((int)n), 0x00020000};
}
// LDS-direct 16-byte load: lane l's 16 bytes at byte voff of the resource land at lds + 16 l
// (lds wave-uniform). One asm statement, so that the compiler's wait insertion (which waits
// for every LDS-direct load before any later access of LDS it cannot tell apart) leaves it
// in flight while the wave computes; the caller waits (vmcnt) before it reads what it wrote.
__device__ __forceinline__ void lds_dma16(i32x4 rs, void* lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(uint8_t*)lds);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen nt lds" ::"v"(voff), "s"(m0), "s"(rs)
               : "memory", "m0");
}
// the same with the default cache policy, for data that neighbouring waves read again from the
// same 128-byte lines (a streaming load lets the L2 drop the line before they come)
__device__ __forceinline__ void lds_dma16_cached(i32x4 rs, void* lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(uint8_t*)lds);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(voff), "s"(m0), "s"(rs)
               : "memory", "m0");
}

// the workspace as a buffer resource: hand-off data goes through sc1 (device-coherent) accesses
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(const Params& p) {
  return __builtin_amdgcn_make_buffer_rsrc(p.ws, (short)0, (int)p.ws_bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 dld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxDev);
}
__device__ __forceinline__ uint32_t dld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kAuxDev);
}
__device__ __forceinline__ uint32_t dld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kAuxDev);
}
__device__ __forceinline__ uint32_t dld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, kAuxDev);
}
__device__ __forceinline__ void dst128(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kAuxDev);
}
__device__ __forceinline__ void dst64(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kAuxDev);
}
__device__ __forceinline__ void dst32(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kAuxDev);
}
__device__ __forceinline__ void dst16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kAuxDev);
}
__device__ __forceinline__ void dst8(__amdgpu_buffer_rsrc_t r, uint32_t off, uint8_t v) {
  __builtin_amdgcn_raw_buffer_store_b8(v, r, off, 0, kAuxDev);
}

__device__ __forceinline__ uint32_t* ctl(const Params& p) { return (uint32_t*)p.ws; }

__device__ __forceinline__ float bf_lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return u2f(w & 0xffff0000u); }

// lane l < D receives lane l + D's value (what other lanes receive is unspecified):
// DPP row_shl within a 16-lane row; the gfx950 lane swaps across rows (second result of
// permlane16_swap(v, v): rows 0 and 2 get rows 1 and 3; of permlane32_swap(v, v): lanes
// 0-31 get lanes 32-63)
template <int D>
__device__ __forceinline__ float from_lane_above(float v) {
  const int iv = __float_as_int(v);
  if constexpr (D == 32) {
    return __int_as_float((int)__builtin_amdgcn_permlane32_swap(iv, iv, false, false)[1]);
  } else if constexpr (D == 16) {
    return __int_as_float((int)__builtin_amdgcn_permlane16_swap(iv, iv, false, false)[1]);
  } else {
    static_assert(D >= 1 && D <= 8, "row shift");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, iv, 0x100 + D, 0xF, 0xF, true));
  }
}

// halving-tree sum over groups of G lanes (G a power of two): lanes l and l + d added for
// d = G/2 .. 1; the first lane of each group ends with the group's sum
template <int G>
__device__ __forceinline__ float tree_sum(float v) {
  if constexpr (G >= 64) v = v + from_lane_above<32>(v);
  if constexpr (G >= 32) v = v + from_lane_above<16>(v);
  if constexpr (G >= 16) v = v + from_lane_above<8>(v);
  if constexpr (G >= 8) v = v + from_lane_above<4>(v);
  if constexpr (G >= 4) v = v + from_lane_above<2>(v);
  if constexpr (G >= 2) v = v + from_lane_above<1>(v);
  return v;
}

// lane l's value, uniform over the wave
__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// the halving-tree sum of the wave, in every lane
__device__ __forceinline__ float wave_sum(float v) { return lane_value(tree_sum<64>(v), 0); }
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
// max over aligned groups of G lanes (G <= 16), in every lane of the group; the inputs are
// never NaN, and a max of non-NaN values does not depend on the exchange pattern
template <int G>
__device__ __forceinline__ float group_max(float v) {
  static_assert(G >= 1 && G <= 16, "within a 16-lane row");
  if constexpr (G >= 2) { const float o = dpp_mov<0xB1>(v); v = o > v ? o : v; }   // quad_perm 1,0,3,2
  if constexpr (G >= 4) { const float o = dpp_mov<0x4E>(v); v = o > v ? o : v; }   // quad_perm 2,3,0,1
  if constexpr (G >= 8) { const float o = dpp_mov<0x141>(v); v = o > v ? o : v; }  // row_half_mirror
  if constexpr (G >= 16) { const float o = dpp_mov<0x140>(v); v = o > v ? o : v; } // row_mirror
  return v;
}

// inclusive prefix sum over the wave: shifts by 1, 2, 4, 8 within each 16-lane row (DPP
// row_shr, lanes without a source add 0), then row 15's total into rows 1 and 3
// (row_bcast:15) and lane 31's into rows 2 and 3 (row_bcast:31)
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
  return v;
}

__device__ __forceinline__ float clampf(float v, float lim) { return fminf(fmaxf(v, -lim), lim); }

// four e4m3 codes (a in the low byte) by the gfx950 convert after the clamp to +-448: for
// every finite input the convert's nearest-even code equals e4m3_encode's (the testing
// library's sweep, csrc/mkmoe_testing.hip, checks all finite fp32 on the device)
__device__ __forceinline__ float clamp448(float v) { return v > kFp8Max ? kFp8Max : (v < -kFp8Max ? -kFp8Max : v); }
__device__ __forceinline__ uint32_t e4m3_pack4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(a), clamp448(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(c), clamp448(d), w, true);
  return (uint32_t)w;
}

// 16 e4m3 weights . 16 e4m3 activations, unscaled
__device__ __forceinline__ float dot16_fp8(u32x4 w, u32x4 x) {
  float s = 0.0f;
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    auto w01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[q], false);
    auto w23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[q], true);
    auto x01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)xv[q], false);
    auto x23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)xv[q], true);
    s = fmaf(w01[0], x01[0], s);
    s = fmaf(w01[1], x01[1], s);
    s = fmaf(w23[0], x23[0], s);
    s = fmaf(w23[1], x23[1], s);
  }
  return s;
}

// byte B of weight dword wq: elements 2B (low nibble), 2B + 1 (high) against x bytes 2B, 2B + 1
template <int B>
__device__ __forceinline__ float fp4_pair(uint32_t wq, uint32_t x_lo, uint32_t x_hi, float s) {
  auto wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wq, 1.0f, B);
  auto xf = __builtin_amdgcn_cvt_pk_f32_fp8((int)(B < 2 ? x_lo : x_hi), (B & 1) != 0);
  s = fmaf(wf[0], xf[0], s);
  return fmaf(wf[1], xf[1], s);
}

// 32 e2m1 weights (16 bytes, even element in the low nibble) . 32 e4m3 activations, unscaled
__device__ __forceinline__ float dot32_fp4(u32x4 w, u32x4 xa, u32x4 xb) {
  float s = 0.0f;
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // weight dword q: elements 8q .. 8q + 7 = x dwords 2q, 2q + 1
    s = fp4_pair<0>(wv[q], xv[2 * q], xv[2 * q + 1], s);
    s = fp4_pair<1>(wv[q], xv[2 * q], xv[2 * q + 1], s);
    s = fp4_pair<2>(wv[q], xv[2 * q], xv[2 * q + 1], s);
    s = fp4_pair<3>(wv[q], xv[2 * q], xv[2 * q + 1], s);
  }
  return s;
}

// ---------------------------------------------------------------- hand-offs
// the first wait past its deadline names its stage and workgroup; a wait stalled by the test
// fault injection names its own in any case (the waits it holds up may time out first)
__device__ __forceinline__ void record_error(const Params& p, int stage, bool fault = false) {
  uint32_t* e = ctl(p) + kCtlErr;
  uint32_t prev = atomicCAS(&e[MKMOE_ERRW_CODE], 0u, (uint32_t)MKMOE_DEVERR_DEADLINE);
  if (prev == 0u || fault) {
    atomicExch(&e[MKMOE_ERRW_STAGE], (uint32_t)stage);
    atomicExch(&e[MKMOE_ERRW_BLOCK], (uint32_t)blockIdx.x);
  }
  if (fault) atomicExch(&e[MKMOE_ERRW_FAULT], 1u);
  atomicAdd(&e[MKMOE_ERRW_COUNT], 1u);
}
// test fault injection: this workgroup's wait at ``stage`` stalls to its deadline
__device__ __forceinline__ bool stalls(const Params& p, int stage) {
  return stage == p.fault_stage && (int)blockIdx.x == p.fault_wg;
}

// this workgroup is done with a stage: its sc1 stores acknowledged, then its flag set (an
// sc1 store: cheaper to see than a device-scope atomic count, by about 1 µs). Wave 1 stores
// it, so that wave 0's flag reads (await_all) do not complete behind the store (a wave's
// memory operations complete in order); await_all counts the own flag as set.
__device__ __forceinline__ void arrive(const Params& p, int which) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 64) dst32(ws_rsrc(p), kCtlFlags + (which * kFlagWgs + blockIdx.x) * 4, 1u);
}

// wait until the first ``nwg`` workgroups' flags at ``which`` are set (or the deadline
// passed; this workgroup's own flag counts as set, it has arrived): wave 0 reads all of them
// at once (a lane four); the data behind them is read with sc1 loads afterwards
__device__ __forceinline__ void await_all(const Params& p, int which, int nwg, int stage) {
  static_assert(kFlagWgs == 64 * 4, "a lane reads four flags");
  if (threadIdx.x < 64) {
    const auto rs = ws_rsrc(p);
    const int lane = threadIdx.x;
    const uint32_t off = kCtlFlags + (which * kFlagWgs + 4 * lane) * 4;
    const bool stall = stalls(p, stage);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (true) {
      const u32x4 f = dld128(rs, off);
      const int i = 4 * lane, own = blockIdx.x;
      const bool ok = (f.x != 0u || i == own || i >= nwg) && (f.y != 0u || i + 1 == own || i + 1 >= nwg) &&
                      (f.z != 0u || i + 2 == own || i + 2 >= nwg) && (f.w != 0u || i + 3 == own || i + 3 >= nwg);
      if (__ballot(!ok) == 0ull && !stall) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > p.deadline) {
        if (lane == 0) record_error(p, stage, stall);
        break;
      }
    }
  }
  __syncthreads();
}

// wait until workgroup ``wg``'s flag at ``which`` is set (or the deadline passed): wave 0 reads
// it; the data behind it is read with sc1 loads afterwards
__device__ __forceinline__ void await_one(const Params& p, int which, int wg, int stage) {
  if (threadIdx.x < 64) {
    const auto rs = ws_rsrc(p);
    const bool stall = stalls(p, stage);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (true) {
      // (one address in every lane: a uniform exit)
      const uint32_t f = __builtin_amdgcn_readfirstlane(dld32(rs, kCtlFlags + (which * kFlagWgs + wg) * 4));
      if (f != 0u && !stall) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > p.deadline) {
        if (threadIdx.x == 0) record_error(p, stage, stall);
        break;
      }
    }
  }
  __syncthreads();
}

// one look at a hand-off's flags (wave 0, before the workgroup requests anything behind it):
// how many are set (this workgroup's own counts as set), in every thread
__device__ __forceinline__ int flags_set_count(const Params& p, int which, int nwg) {
  __shared__ int s_n;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const u32x4 f = dld128(ws_rsrc(p), kCtlFlags + (which * kFlagWgs + 4 * lane) * 4);
    const int i = 4 * lane, own = blockIdx.x;
    const int n = __popcll(__ballot(i < nwg && (f.x != 0u || i == own))) +
                  __popcll(__ballot(i + 1 < nwg && (f.y != 0u || i + 1 == own))) +
                  __popcll(__ballot(i + 2 < nwg && (f.z != 0u || i + 2 == own))) +
                  __popcll(__ballot(i + 3 < nwg && (f.w != 0u || i + 3 == own)));
    if (lane == 0) s_n = n;
  }
  __syncthreads();
  return s_n;
}

// leave the launch with its flags clear for the next (graph replay safe): every workgroup
// here has passed the C hand-off (and Q, where the launch has one), so every workgroup has
// passed the earlier ones and a workgroup clears its own flags of those; the last workgroup
// out clears the C and Q flags (all have passed those waits) and the exit count
__device__ __forceinline__ void leave(const Params& p) {
  __syncthreads();
  if (threadIdx.x < 64) {
    const auto rs = ws_rsrc(p);
    const int lane = threadIdx.x;
    if (lane < kCtlC) dst32(rs, kCtlFlags + (lane * kFlagWgs + blockIdx.x) * 4, 0u);
    uint32_t n = 0;
    if (lane == 0)
      n = __hip_atomic_fetch_add(ctl(p) + kCtlExit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    n = __builtin_amdgcn_readfirstlane(n);
    if (n == gridDim.x - 1) {
      dst128(rs, kCtlFlags + (kCtlC * kFlagWgs + 4 * lane) * 4, u32x4{0u, 0u, 0u, 0u});
      dst128(rs, kCtlFlags + (kCtlQ * kFlagWgs + 4 * lane) * 4, u32x4{0u, 0u, 0u, 0u});
      if (lane == 0) __hip_atomic_store(ctl(p) + kCtlExit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// this thread's wave, as a uniform (scalar) value: it then takes no vector register, which the
// persistent launch's loops need for their operands
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
// wave units spread over workgroups first: this wave is slot b + nwg * wave
__device__ __forceinline__ int wave_slot(int b, int nwg) { return b + nwg * wave_index(); }

// ---------------------------------------------------------------- stage N: RMSNorm
// rows up to which every workgroup normalizes the rows itself as stage A reads them (each
// row's 1 / rms computed by one wave of every workgroup that needs it, in the order below:
// the same bits everywhere), so that no hand-off precedes stage A; above, stage N writes the
// normed rows and a hand-off follows
constexpr int kLocalNormMax = 16;

// 1 / rms of a row held as v[c] = the lane's 8 columns of 512-column chunk c (every lane):
// lane l sums the squares of its columns chunk by chunk in order, then the wave's sum
template <class C>
__device__ __forceinline__ float row_rstd(const Params& p, const u32x4 (&v)[C::CH512]) {
#pragma clang fp contract(off)
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < C::CH512; ++c) {
    const uint32_t w4[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float f = (j & 1) ? bf_hi(w4[j >> 1]) : bf_lo(w4[j >> 1]);
      acc = acc + f * f;
    }
  }
  float ss = wave_sum(acc);
  float mean = ss / (float)C::H;
  return 1.0f / sqrtf(mean + p.eps);
}
template <class C>
__device__ __forceinline__ void row_load(const Params& p, int r, int lane, u32x4 (&v)[C::CH512]) {
  const uint16_t* x = p.x + (size_t)r * C::H;
#pragma unroll
  for (int c = 0; c < C::CH512; ++c) v[c] = ld16(x + c * 512 + lane * 8);
}

// 8 normed bf16 from 8 of x and of the norm weight: bf16((x * rstd) * w)
__device__ __forceinline__ u32x4 norm8(u32x4 xv, u32x4 nw, float rstd) {
#pragma clang fp contract(off)
  const uint32_t w4[4] = {xv.x, xv.y, xv.z, xv.w};
  const uint32_t n4[4] = {nw.x, nw.y, nw.z, nw.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float a = bf_lo(w4[q]) * rstd, b = bf_hi(w4[q]) * rstd;
    a = a * bf_lo(n4[q]);
    b = b * bf_hi(n4[q]);
    o[q] = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

template <class C>
__device__ __forceinline__ void norm_row(const Params& p, int r, int lane) {
  u32x4 v[C::CH512];
  row_load<C>(p, r, lane, v);
  const float rstd = row_rstd<C>(p, v);
  const auto rs = ws_rsrc(p);
  const uint32_t base = p.off[0] + (uint32_t)r * C::H * 2;
#pragma unroll
  for (int c = 0; c < C::CH512; ++c)
    dst128(rs, base + (c * 512 + lane * 8) * 2, norm8(v[c], ld16(p.norm_w + c * 512 + lane * 8), rstd));
}

// every row's 1 / rms into rstd[] (a wave a row), for the rows normed locally
template <class C>
__device__ __forceinline__ void local_rstd(const Params& p, float* rstd) {
  const int lane = threadIdx.x & 63;
  for (int r = wave_index(); r < p.rows; r += kWaves) {
    u32x4 v[C::CH512];
    row_load<C>(p, r, lane, v);
    const float s = row_rstd<C>(p, v);
    if (lane == 0) rstd[r] = s;
  }
  __syncthreads();
}

template <class C>
__device__ __forceinline__ void stage_norm(const Params& p, int b, int nwg) {
  const int lane = threadIdx.x & 63, gw = wave_slot(b, nwg);
  for (int r = gw; r < p.rows; r += nwg * kWaves) norm_row<C>(p, r, lane);
}

// 8 bf16 of row r from element col: the normed rows (sc1: written by stage N, or normed
// here with the row's 1 / rms where the rows are normed locally, rstd non-null) or the input
template <class C>
__device__ __forceinline__ u32x4 x_load(const Params& p, __amdgpu_buffer_rsrc_t rs, int r, int col,
                                        const float* rstd = nullptr) {
  if constexpr (C::NORM) {
    if (rstd) return norm8(ld16(p.x + (size_t)r * C::H + col), ld16(p.norm_w + col), rstd[r]);
    return dld128(rs, p.off[0] + ((uint32_t)r * C::H + col) * 2);
  }
  return ld16(p.x + (size_t)r * C::H + col);
}

// ---------------------------------------------------------------- stage A
// the columns of one router K part for every row, staged in LDS
template <class C>
struct RouterSmem {
  static constexpr int PW = C::H / C::P;
  uint16_t x[kRowsMax * PW];
  float rstd[kRowsMax];  // the rows' 1 / rms, where stage A norms them itself
};

// router part sums of one workgroup unit: K part ``part`` of experts eb * 8 .. eb * 8 + 7
// (one a wave) for every row, in the fixed order: lane l sums its 8 columns of each
// 512-column chunk of the part in order (products rounded, then added), then the
// wave's halving tree
template <class C>
__device__ __forceinline__ void router_unit(const Params& p, RouterSmem<C>& sm, int part, int eb, int lane, int wave,
                                            const float* rstd) {
#pragma clang fp contract(off)
  constexpr int CPP = C::CH512 / C::P;
  constexpr int PW = RouterSmem<C>::PW;
  static_assert(PW == CPP * 512, "part width");
  const int e = eb * kWaves + wave;
  const auto rs = ws_rsrc(p);
  u32x4 wv[CPP];
  if (e < C::E) {
#pragma unroll
    for (int i = 0; i < CPP; ++i)
      wv[i] = ld16_nt(p.gate_w + (size_t)e * C::H + (part * CPP + i) * 512 + lane * 8);
  }
  __syncthreads();  // the previous unit is done with the tile
  const int n = p.rows * (PW / 8);
#pragma unroll 4
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const int r = i / (PW / 8), c = i % (PW / 8);
    *(u32x4*)(sm.x + r * PW + c * 8) = x_load<C>(p, rs, r, part * PW + c * 8, rstd);
  }
  __syncthreads();
  if (e >= C::E) return;
  for (int r = 0; r < p.rows; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < CPP; ++i) {
      const u32x4 xv = *(const u32x4*)(sm.x + r * PW + i * 512 + lane * 8);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
      const uint32_t ww[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc = acc + bf_lo(xw[q]) * bf_lo(ww[q]);
        acc = acc + bf_hi(xw[q]) * bf_hi(ww[q]);
      }
    }
    const float s = tree_sum<64>(acc);
    if (lane == 0) {
      const uint32_t at = (((uint32_t)r * C::P + part) * C::E + e) * 4;
      dst32(rs, p.off[5] + at, f2u(s));   // kept for inspection
      dst32(rs, p.off[10] + at, f2u(s));  // polled, cleared once routed
    }
  }
}

// quantize 512 columns of row r: group-128 fp8 (fp32 scale) and, for MXFP4
// experts, MXFP8 per 32 ("aiter" rule); rstd non-null: the columns are normed here, and
// stored as the normed rows (sc1) too
template <class C>
__device__ __forceinline__ void quant_unit(const Params& p, int r, int c, int lane, const float* rstd) {
#pragma clang fp contract(off)
  const auto rs = ws_rsrc(p);
  u32x4 xv = x_load<C>(p, rs, r, c * 512 + lane * 8, rstd);
  if (C::NORM && rstd) dst128(rs, p.off[0] + ((uint32_t)r * C::H + c * 512 + lane * 8) * 2, xv);
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
  float v[8];
  float am = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = bf_lo(xw[q]);
    v[2 * q + 1] = bf_hi(xw[q]);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) am = fabsf(v[j]) > am ? fabsf(v[j]) : am;
  const uint32_t col = (uint32_t)r * C::H + c * 512 + lane * 8;
  if constexpr (C::SFMT == kFp8Mx) {
    // the shared expert's rule: MXFP8 per 32, the "vllm" code (4 lanes a group)
    static_assert(C::FMT == kFp4, "the MX shared rule's codes in regions 3 / 4");
    const int code = vllm_code(group_max<4>(am));
    const float inv = mx_inv(code);
    const uint32_t lo = e4m3_pack4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    const uint32_t hi = e4m3_pack4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
    dst64(rs, p.off[3] + col, u32x2{lo, hi});
    if ((lane & 3) == 0) dst8(rs, p.off[4] + (uint32_t)r * (C::H / 32) + c * 16 + lane / 4, (uint8_t)code);
  } else {
    // group-128 fp8: 16 lanes a group
    float g = group_max<16>(am);
    float s = group_scale(g);
    const uint32_t lo = e4m3_pack4(v[0] / s, v[1] / s, v[2] / s, v[3] / s);
    const uint32_t hi = e4m3_pack4(v[4] / s, v[5] / s, v[6] / s, v[7] / s);
    const int rq = C::FMT == kFp4 ? 3 : 1, rsc = C::FMT == kFp4 ? 4 : 2;
    dst64(rs, p.off[rq] + col, u32x2{lo, hi});
    if ((lane & 15) == 0)
      dst32(rs, p.off[rsc] + ((uint32_t)r * (C::H / 128) + c * 4 + lane / 16) * 4, f2u(s));
  }
  if constexpr (C::FMT == kFp4) {
    float g = group_max<4>(am);
    int code = mx_code(g);
    float inv = mx_inv(code);
    const uint32_t lo = e4m3_pack4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    const uint32_t hi = e4m3_pack4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
    dst64(rs, p.off[1] + col, u32x2{lo, hi});
    if ((lane & 3) == 0)
      dst8(rs, p.off[2] + (uint32_t)r * (C::H / 32) + c * 16 + lane / 4, (uint8_t)code);
  }
}

// workgroup units: (router K part, block of 8 experts), then one unit a row to quantize
// The router's part sums are also stored into region 10, which holds kPartUnset between
// launches, so that routing can read them as they land. It is a NaN that no part sum takes: a NaN propagated from a bf16 input keeps a
// payload whose low 16 bits are zero, and a NaN the arithmetic generates is the default one.
constexpr uint32_t kPartUnset = 0xFFFFFFFFu;
// region 10's part sums of the step's rows back to kPartUnset, spread over the grid (once
// every workgroup is past its routing)
template <class C>
__device__ __forceinline__ void reset_parts(const Params& p, int b, int nwg) {
  static_assert(C::E % 4 == 0, "16-byte stores");
  const auto rs = ws_rsrc(p);
  const int chunks = p.rows * C::P * C::E / 4;
  for (int i = b * kThreads + (int)threadIdx.x; i < chunks; i += nwg * kThreads)
    dst128(rs, p.off[10] + (uint32_t)i * 16, u32x4{kPartUnset, kPartUnset, kPartUnset, kPartUnset});
}

template <class C>
__device__ __forceinline__ void stage_a(const Params& p, RouterSmem<C>& sm, int b, int nwg, bool local_norm) {
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  constexpr int EB = (C::E + kWaves - 1) / kWaves;
  constexpr int n_router = C::P * EB;
  // local_norm: the rows' 1 / rms first, in every workgroup with a unit
  const float* rstd = nullptr;
  if (C::NORM && local_norm && (b < n_router + p.rows || (n_router < nwg && n_router + p.rows > nwg))) {
    local_rstd<C>(p, sm.rstd);
    rstd = sm.rstd;
  }
  if (n_router < nwg && n_router + p.rows > nwg) {
    // more units than workgroups: a router unit each on workgroups [0, n_router) and the rows'
    // quantize on the others, several rows each (a router unit of many rows outlasts several
    // rows' quantize; dealt in turn, the first workgroups would run one of each)
    if (b < n_router) {
      router_unit<C>(p, sm, b % C::P, b / C::P, lane, wave, rstd);
    } else {
      for (int r = b - n_router; r < p.rows; r += nwg - n_router)
        for (int c = wave; c < C::CH512; c += kWaves) quant_unit<C>(p, r, c, lane, rstd);
    }
    return;
  }
  const int n = n_router + p.rows;
  for (int u = b; u < n; u += nwg) {
    if (u < n_router) {
      router_unit<C>(p, sm, u % C::P, u / C::P, lane, wave, rstd);
    } else {
      for (int c = wave; c < C::CH512; c += kWaves) quant_unit<C>(p, u - n_router, c, lane, rstd);
    }
  }
}

// ---------------------------------------------------------------- stage B: routing
// Scores and choices of kRouteRows rows at a time, in LDS
constexpr int kRouteRows = 16;
// rows up to which every workgroup routes the whole step itself (no routing hand-off). Above,
// a workgroup a row and the hand-off cost less than every workgroup's scores of all the rows:
// 8 against 16 at 12 and 16 rows, cfg 2 -2.8 / -3.4 us, cfg 3 -3.6 / -5.6, V4.1 TP4 -6.1 /
// -5.4 (its 384 sqrt(softplus) scores a row); lower, mixed, but V4.1 at TP2 gains with 4
// (-0.6 / -1.6 / -1.8 us at 5 / 6 / 8 rows: measured)
constexpr int kLocalRouteMax = 8;
template <class C>
constexpr int local_route_max() {
  return C::E > 256 && C::I >= 1024 ? 4 : kLocalRouteMax;
}

template <class C>
struct RouteSmem {
  static constexpr int NG = C::NG > 1 ? C::NG : 1;
  float sc[kRouteRows][C::E];
  float ch[kRouteRows][C::E];
  float gsum[kRouteRows][NG];  // a group's top-1 + top-2 choice
  float gv2[kRouteRows][NG];   // and its top-2 choice
  float cv[kWaves][C::E + 8];  // a wave's candidates: choice (8 past the last: -inf), id
  int ce[kWaves][C::E];
  float ss[kWaves][C::K];  // and its picks: score, id
  int se[kWaves][C::K];
};

// max over aligned groups of G lanes (G a power of two <= 64), in every lane of the group;
// inputs are never NaN. Across 16-lane rows: permlane16_swap(v, v) returns rows (0, 0, 2, 2)
// and (1, 1, 3, 3), permlane32_swap(v, v) lanes 0-31 twice and 32-63 twice
template <int G>
__device__ __forceinline__ float segment_max(float v) {
  if constexpr (G <= 16) {
    return group_max<G>(v);
  } else {
    v = group_max<16>(v);
    const int iv = __float_as_int(v);
    const auto s = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    const float a = __int_as_float((int)s[0]), c = __int_as_float((int)s[1]);
    v = a > c ? a : c;
    if constexpr (G == 64) {
      const int jv = __float_as_int(v);
      const auto t = __builtin_amdgcn_permlane32_swap(jv, jv, false, false);
      const float d = __int_as_float((int)t[0]), f = __int_as_float((int)t[1]);
      v = d > f ? d : f;
    }
    return v;
  }
}

// scores and choices of (row r0 + i, expert e) for i < n, spread over the workgroup: the
// logit sums the router's part sums in part order; choice = score + bias, and a NaN choice
// is -inf (max(sc + bias, -inf) of the reference's route, stages/moe.py:345-347); a NaN
// score weighs 0
// POLL: the part sums are read before the router's hand-off, each reread until it holds a
// value (kPartUnset marks a part sum not yet written in this launch)
// the fp32 logits (parts added in order) and scores of a thread's first NJ (row, expert) pairs
template <class C, int NJ, int MJ, int P>
__device__ __forceinline__ void sigmoids(const float (&part)[MJ][P], float (&sg)[MJ]) {
#pragma clang fp contract(off)
  float logit[NJ], out[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    logit[j] = 0.0f;
#pragma unroll
    for (int q = 0; q < P; ++q) logit[j] = logit[j] + part[j][q];
  }
  // the scores step by step together, four at a time (each value's operations in the scalar
  // order; wider, the chains' registers crowd the launch's)
  constexpr int W = NJ < 4 ? NJ : 4;
#pragma unroll
  for (int j0 = 0; j0 < NJ; j0 += W) {
    float xv[W], ov[W];
#pragma unroll
    for (int i = 0; i < W; ++i) xv[i] = j0 + i < NJ ? logit[j0 + i] : 0.0f;
    if constexpr (C::SCORE == kScoreSqrtSoftplus) sqrt_softplus_exact_n<W>(xv, ov);
    else sigmoid_exact_n<W>(xv, ov);
#pragma unroll
    for (int i = 0; i < W; ++i)
      if (j0 + i < NJ) out[j0 + i] = ov[i];
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) sg[j] = out[j];
}

template <class C, bool POLL = false>
__device__ __forceinline__ void route_scores(const Params& p, RouteSmem<C>& sm, int r0, int n) {
#pragma clang fp contract(off)
  constexpr int MJ = (kRouteRows * C::E + kThreads - 1) / kThreads;  // (row, expert) a thread
  const auto rs = ws_rsrc(p);
  const int tid = threadIdx.x;
  // the bias of the thread's experts, requested before the part sums arrive
  float bias[MJ];
#pragma unroll
  for (int j = 0; j < MJ; ++j) bias[j] = p.bias[(tid + j * kThreads) % C::E];
  // every part sum ([rows][P][E]) requested before the first is used
  float part[MJ][C::P];
  auto part_off = [&](int j, int q) {
    const int idx = tid + j * kThreads;
    const int i = idx / C::E, e = idx - i * C::E;
    return p.off[POLL ? 10 : 5] + ((uint32_t)(r0 + i) * C::P * C::E + e) * 4 + q * C::E * 4;
  };
#pragma unroll
  for (int j = 0; j < MJ; ++j) {
    const int idx = tid + j * kThreads;
#pragma unroll
    for (int q = 0; q < C::P; ++q) part[j][q] = idx < n * C::E ? u2f(dld32(rs, part_off(j, q))) : 0.0f;
  }
  if constexpr (POLL) {
    // wave-uniform: a wave polls until none of its lanes' part sums is unset, or gives up
    // at the deadline (s_memrealtime is a scalar read, the same in every lane), and then
    // records the error once (lane 0)
    const bool stall = stalls(p, kStageA);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (true) {
      bool unset = false;
#pragma unroll
      for (int j = 0; j < MJ; ++j)
#pragma unroll
        for (int q = 0; q < C::P; ++q) unset |= f2u(part[j][q]) == kPartUnset;
      if (__ballot(unset) == 0ull && !stall) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > p.deadline) {
        if ((tid & 63) == 0) record_error(p, kStageA, stall);
        break;
      }
#pragma unroll
      for (int j = 0; j < MJ; ++j)
#pragma unroll
        for (int q = 0; q < C::P; ++q)
          if (f2u(part[j][q]) == kPartUnset) part[j][q] = u2f(dld32(rs, part_off(j, q)));
    }
    TL(kTlParts);
  }
  // the thread's logits and sigmoids first, in one straight block for the live (row, expert)
  // pairs (the first nj; the rest of a block score unused zeros), so that their fp64 chains
  // overlap
  float sgv[MJ];
  const int nj = (n * C::E + kThreads - 1) / kThreads;
  if (nj <= 1) sigmoids<C, 1>(part, sgv);
  else if (nj <= 2) sigmoids<C, (MJ < 2 ? MJ : 2)>(part, sgv);
  else if (nj <= 4) sigmoids<C, (MJ < 4 ? MJ : 4)>(part, sgv);
  else if (MJ > 8 && nj <= 6) sigmoids<C, (MJ < 6 ? MJ : 6)>(part, sgv);  // 8 rows of 384 experts
  else if (MJ > 8 && nj <= 8) sigmoids<C, (MJ < 8 ? MJ : 8)>(part, sgv);
  else sigmoids<C, MJ>(part, sgv);
#pragma unroll
  for (int j = 0; j < MJ; ++j) {
    const int idx = tid + j * kThreads;
    if (idx < n * C::E) {
      const int i = idx / C::E, e = idx - i * C::E;
      const float sg = sgv[j];
      const float s = sg != sg ? 0.0f : sg;  // the weight of a NaN score is 0
      const float cv = sg + bias[j];
      const float ch = cv != cv ? -INFINITY : cv;  // and its choice -inf
      sm.sc[i][e] = s;
      sm.ch[i][e] = ch;
      if constexpr (C::NG > 1) {
        // a wave holds 64 consecutive experts of one row (E is a multiple of 64), i.e. whole
        // groups: top-1 of the group, then top-2: top-1 again when two experts hold it, else
        // the max of the others
        constexpr int GS = C::E / C::NG;
        static_assert(C::E % 64 == 0 && GS >= 2 && GS <= 64 && (64 % GS) == 0, "groups within a wave");
        const int lane = tid & 63;
        const uint64_t seg = GS == 64 ? ~0ull : (((1ull << GS) - 1ull) << ((lane / GS) * GS));
        const float m1 = segment_max<GS>(ch);
        const uint64_t eq = __ballot(ch == m1);
        const float m2 = segment_max<GS>(ch == m1 ? -INFINITY : ch);
        const float v2 = __popcll(eq & seg) >= 2 ? m1 : m2;
        if (lane % GS == 0) {
          sm.gsum[i][e / GS] = m1 + v2;
          sm.gv2[i][e / GS] = v2;
        }
      }
    }
  }
}

// one row's grouped top-k by one wave, from its scores sc and choices ch in LDS; cand is the
// wave's slice of the LDS scratch. Lane l holds experts l + 64 i. Group score = top-1 + top-2
// choice of the group; the topk_group best groups are kept (larger score, then lower group);
// the picks are the topk best experts of the kept groups (larger choice, then lower id), in
// that order, i.e. the order of a selection that takes the best remaining expert topk times.
// Every pick's choice is at least L, the smallest top-2 choice of the kept groups (those
// 2 * topk_group >= topk experts reach it), so only experts with choice >= L are ranked: each
// against all the others, in parallel. Lane k < topk returns pick k's id and weight.
template <class C>
__device__ __forceinline__ void select_row(const Params& p, const RouteSmem<C>& sm, int row, float* cv, int* ce,
                                           float* ss, int* se, int lane, int& my_id, float& my_w) {
#pragma clang fp contract(off)
  constexpr int EPL = (C::E + 63) / 64;
  const float* sc_row = sm.sc[row];
  const float* ch_row = sm.ch[row];
  float ch[EPL];
  bool alive[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    alive[i] = e < C::E;
    ch[i] = alive[i] ? ch_row[e] : -INFINITY;
  }
  float lb = -INFINITY;  // L
  if constexpr (C::NG > 1) {
    constexpr int GS = C::E / C::NG;
    // lane g < NG takes group g's score and counts the groups ranked above it
    const float mine = lane < C::NG ? sm.gsum[row][lane] : -INFINITY;
    int above = 0;
#pragma unroll
    for (int g = 0; g < C::NG; ++g) above += better(sm.gsum[row][g], g, mine, lane) ? 1 : 0;
    const uint64_t gkeep = __ballot(lane < C::NG && above < C::TG);
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      alive[i] = alive[i] && ((gkeep >> (e / GS)) & 1ull) != 0ull;
    }
    if constexpr (2 * C::TG >= C::K) {
      lb = INFINITY;
#pragma unroll
      for (int g = 0; g < C::NG; ++g) {
        const float v2 = sm.gv2[row][g];
        lb = ((gkeep >> g) & 1ull) && v2 < lb ? v2 : lb;
      }
    }
  } else if constexpr (C::E > 64) {
    // one group over more experts than lanes: L is the topk-th largest of the lanes' own
    // largest choices (topk rounds of a wave max, each taking out one lane's). At least topk
    // experts reach it, so every pick does, and only experts at L or above are ranked: about
    // topk of them, where ranking all E (each lane against every candidate in dependent chains)
    // took 42 us at E = 384
    static_assert(C::K <= 64, "picks from distinct lanes");
    float m = ch[0];
#pragma unroll
    for (int i = 1; i < EPL; ++i) m = ch[i] > m ? ch[i] : m;
#pragma unroll 1
    for (int k = 0; k < C::K; ++k) {
      lb = segment_max<64>(m);
      const uint64_t at = __ballot(m == lb);
      if (lane == (int)__ffsll((unsigned long long)at) - 1) m = -INFINITY;
    }
  }
  // candidates to LDS slots 0 .. nc - 1, in id order
  int nc = 0;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const bool cand = alive[i] && ch[i] >= lb;
    const uint64_t cm = __ballot(cand);
    if (cand) {
      const int slot = nc + (int)__popcll(cm & ((1ull << lane) - 1ull));
      cv[slot] = ch[i];
      ce[slot] = lane + 64 * i;
    }
    nc += (int)__popcll(cm);
  }
  if (lane < 8) cv[nc + lane] = -INFINITY;  // the slots a step of 8 reads past the last
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // a candidate's rank is the count of those better than it: a larger choice, or the same
  // choice at a lower slot (slots ascend with the id). Slot c + 64 t is lane c's candidate t;
  // the candidates are read 8 at a time (LDS broadcasts); the -inf past the last count for none
  float cvr[EPL];
#pragma unroll
  for (int t = 0; t < EPL; ++t) cvr[t] = 64 * t + lane < nc ? cv[64 * t + lane] : -INFINITY;
  int rank[EPL];
#pragma unroll
  for (int t = 0; t < EPL; ++t) rank[t] = 0;
  if (nc <= 64) {  // the usual case: one register of candidates
    for (int j0 = 0; j0 < nc; j0 += 8) {
      const f32x4 va = *(const f32x4*)(cv + j0);
      const f32x4 vb = *(const f32x4*)(cv + j0 + 4);
      const float vj[8] = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
#pragma unroll
      for (int k = 0; k < 8; ++k) rank[0] += (vj[k] > cvr[0]) | ((vj[k] == cvr[0]) & (j0 + k < lane)) ? 1 : 0;
    }
  } else {
    for (int j0 = 0; j0 < nc; j0 += 8) {
      const f32x4 va = *(const f32x4*)(cv + j0);
      const f32x4 vb = *(const f32x4*)(cv + j0 + 4);
      const float vj[8] = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int t = 0; t < EPL; ++t)
          rank[t] += (vj[k] > cvr[t]) | ((vj[k] == cvr[t]) & (j0 + k < 64 * t + lane)) ? 1 : 0;
    }
  }
#pragma unroll
  for (int t = 0; t < EPL; ++t) {
    const int c = 64 * t + lane;
    if (c < nc && rank[t] < C::K) {
      const int id = ce[c];
      ss[rank[t]] = sc_row[id];
      se[rank[t]] = id;
    }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // weights: the picks' scores summed in pick order
  const float mine_s = lane < C::K ? ss[lane] : 0.0f;
  my_id = lane < C::K ? min(max(se[lane], 0), C::E - 1) : 0;
  float total = 0.0f;
#pragma unroll
  for (int k = 0; k < C::K; ++k) total = total + lane_value(mine_s, k);
  float f = p.scale;
  if (p.renorm) f = p.scale / (total > 1e-20f ? total : 1e-20f);
  my_w = mine_s * f;
}

// row r's routing by one workgroup (stage B), written to the workspace and the outputs
template <class C>
__device__ __forceinline__ void route_row(const Params& p, RouteSmem<C>& sm, int r) {
  const int lane = threadIdx.x & 63;
  route_scores<C>(p, sm, r, 1);
  __syncthreads();
  if (threadIdx.x >= 64) return;
  int id;
  float w;
  select_row<C>(p, sm, 0, sm.cv[0], sm.ce[0], sm.ss[0], sm.se[0], lane, id, w);
  if (lane < C::K) {
    const auto rs = ws_rsrc(p);
    dst32(rs, p.off[6] + (r * C::K + lane) * 4, (uint32_t)id);
    dst32(rs, p.off[7] + (r * C::K + lane) * 4, f2u(w));
    if (p.ids_out) p.ids_out[r * C::K + lane] = id;
    if (p.w_out) p.w_out[r * C::K + lane] = w;
  }
}

// every row's routing in this workgroup, into LDS (ids, wts: [rows][topk]; rows_of: the rows
// that picked each expert, as bitmaps); wave w selects rows w, w + 8, ... of each kRouteRows
// chunk. One workgroup (publish) also writes the workspace copies and the outputs.
template <class C>
__device__ __forceinline__ void route_all(const Params& p, RouteSmem<C>& sm, int* ids, float* wts,
                                          uint32_t (*rows_of)[2], bool publish) {
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  const auto rs = ws_rsrc(p);
  for (int e = threadIdx.x; e < C::E; e += kThreads) rows_of[e][0] = rows_of[e][1] = 0u;
  for (int r0 = 0; r0 < p.rows; r0 += kRouteRows) {
    const int n = min(kRouteRows, p.rows - r0);
    __syncthreads();  // the previous chunk's selections are done with the LDS
    route_scores<C, true>(p, sm, r0, n);
    __syncthreads();
    TL(kTlScores);
    for (int i = wave; i < n; i += kWaves) {
      int id;
      float w;
      select_row<C>(p, sm, i, sm.cv[wave], sm.ce[wave], sm.ss[wave], sm.se[wave], lane, id, w);
      const int r = r0 + i;
      if (lane < C::K) {
        ids[r * C::K + lane] = id;
        wts[r * C::K + lane] = w;
        atomicOr(&rows_of[id][r >> 5], 1u << (r & 31));
        if (publish) {
          dst32(rs, p.off[6] + (r * C::K + lane) * 4, (uint32_t)id);
          dst32(rs, p.off[7] + (r * C::K + lane) * 4, f2u(w));
          if (p.ids_out) p.ids_out[r * C::K + lane] = id;
          if (p.w_out) p.w_out[r * C::K + lane] = w;
        }
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- VALU GEMV of weight rows
// Every expert GEMV runs in one fixed order (the oracle restates it): a row of KD
// elements is cut into 16-element (FP8) / 32-element (FP4) chunks; a chunk's unscaled
// sum runs in element order (the products are exact in fp32); it is scaled (FP8:
// d * fp32(s_w * s_x); FP4: d * 2^(e_w + e_x - 254)); chunk c goes to lane c % LPR,
// each lane sums its chunks in order, and the LPR lanes add as a halving tree.
// A unit of NR rows is streamed by one wave whose lanes split into G = 64 / LPR
// sub-groups, sub-group g taking rows g, g + G, ...
template <int FMT, int KD>
struct RowShape {
  static constexpr int CPR = FMT == kFp4 ? KD / 32 : KD / 16;  // chunks a row
  // lanes a row: 64, or the largest power of two below it that divides the chunks
  static constexpr int G = CPR % 64 == 0 ? 1 : CPR % 32 == 0 ? 2 : CPR % 16 == 0 ? 4 : 8;
  static constexpr int LPR = 64 / G;
  static constexpr int CPL = CPR / LPR;  // chunks a lane a row
  static_assert(CPR % LPR == 0, "row chunks");
};

// NR weight rows (FP8 with fp32 128 x 128 scales, or MXFP4 with E8M0 per 32) in registers:
// ``rows[r]`` is row r's first byte, ``srow[r]`` its scales (FP8: the row block's fp32
// scales, one per 128 K; FP4: the row's E8M0 bytes)
template <int FMT, int KD, int NR, bool FP8_SCALES = true>
struct WRows {
  using S = RowShape<FMT, KD>;
  static constexpr int RPG = NR / S::G;  // rows a sub-group
  static_assert(RPG * S::G == NR, "rows split over sub-groups");
  u32x4 w[RPG][S::CPL];
  float sf[RPG][S::CPL];
  int se[RPG][S::CPL];

  // row(i, w, s) sets row i's first byte and its scales (i < NR; this lane's sub-group g
  // takes rows g, g + G, ...)
  template <class RowFn>
  __device__ __forceinline__ void load(RowFn row, int lane) {
    const int g = lane / S::LPR, l = lane % S::LPR;
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
      const uint8_t* r;
      const void* sr;
      row(q * S::G + g, r, sr);
#pragma unroll
      for (int i = 0; i < S::CPL; ++i) w[q][i] = ld16_nt(r + (l + S::LPR * i) * 16);
#pragma unroll
      for (int i = 0; i < S::CPL; ++i) {
        const int c = l + S::LPR * i;
        if constexpr (FMT == kFp8) {
          if constexpr (FP8_SCALES) sf[q][i] = ((const float*)sr)[c / 8];
        } else {
          se[q][i] = ((const uint8_t*)sr)[c];
        }
      }
    }
  }

};

// silu(z) = z * sigmoid(z) with the exact fp64 sigmoid; the SwiGLU of a gate_up pair: the
// routed rule (check_ffn.py:220) or the shared rule, which rounds gate and up to bf16
// first (check_ffn.py:227-230)
__device__ __forceinline__ float silu_exact(float z) {
#pragma clang fp contract(off)
  return z * sigmoid_exact(z);
}
__device__ __forceinline__ float swiglu_routed(float g, float u, float lim) {
#pragma clang fp contract(off)
  return bf_round(silu_exact(fminf(g, lim)) * clampf(u, lim));
}
__device__ __forceinline__ float swiglu_shared(float g, float u, float lim) {
#pragma clang fp contract(off)
  return bf_round(silu_exact(bf_round(fminf(g, lim))) * bf_round(clampf(u, lim)));
}

constexpr int kTokGroup = 8;    // picks a VALU gate_up unit takes at most
constexpr int kMfmaPicks = 16;  // picks an MFMA unit takes at most (the MFMA's 16 columns)

// activation rows of a unit staged in LDS: up to kMfmaPicks rows of codes and their scales
template <class C>
struct XTile {
  static constexpr int QS = C::H + 16;  // row stride (bank spread)
  // fp32 block scales of an FP8 [2W][H] weight: (2W / 128) x (H / 128), padded to 1 KB
  static constexpr int WSC = (2 * (C::I > C::S ? C::I : C::S) / 128 * (C::H / 128) + 255) / 256 * 256;
  static constexpr int SB = (kMfmaPicks * (C::H / 32) + 1023) / 1024 * 1024;  // scale bytes, padded
  uint8_t q[kMfmaPicks * QS];
  uint8_t s[SB];  // E8M0 per 32, or fp32 per 128 (the same bytes), C::H / 32 bytes a row
  float wsc[WSC];
};

// the (at most NR) activation rows of a unit on their way to the tile: each thread's share of
// the codes (16-byte chunks) and scale words, loaded (sc1) before the unit's weights so that
// writing them to LDS waits for these loads alone
template <class C, int NR>
struct XRegs {
  static constexpr int QC = C::H / 16;  // 16-byte chunks a row
  static constexpr int NQ = (NR * QC + kThreads - 1) / kThreads;
  static constexpr int SW = C::H / 128;  // 4-byte scale words a row (fp32 per 128, or E8M0 per 32)
  static constexpr int NS = (NR * SW + kThreads - 1) / kThreads;
  static_assert(NR <= kMfmaPicks, "rows of the tile");
  static constexpr int NW = (XTile<C>::WSC + kThreads - 1) / kThreads;
  u32x4 q[NQ];
  uint32_t s[NS];
  float w[NW];
  int nw = 0;

  // the FP8 weight's block scales, (2W / 128) x (H / 128) fp32 from ws (read-only input)
  __device__ __forceinline__ void load_wscales(const float* ws, int W) {
    nw = 2 * W / 128 * (C::H / 128);
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int idx = threadIdx.x + i * kThreads;
      if (idx < nw) w[i] = ws[idx];
    }
  }

  // rows tok(r), r < np: codes at qoff + t H, scales at soff + t * SW * 4
  template <class TokFn>
  __device__ __forceinline__ void load(const Params& p, int np, uint32_t qoff, uint32_t soff, TokFn tok) {
    const auto rs = ws_rsrc(p);
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < np * QC) {
        const int r = idx / QC, c = idx % QC;
        q[i] = dld128(rs, qoff + (uint32_t)tok(r) * C::H + c * 16);
      }
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < np * SW) s[i] = dld32(rs, soff + (uint32_t)tok(idx / SW) * (SW * 4) + (idx % SW) * 4);
    }
  }

  __device__ __forceinline__ void store(XTile<C>& xt, int np) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < np * QC) *(u32x4*)(xt.q + (idx / QC) * XTile<C>::QS + (idx % QC) * 16) = q[i];
    }
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < np * SW) ((uint32_t*)xt.s)[idx] = s[i];
    }
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < nw) xt.wsc[idx] = w[i];
    }
  }
};

// gate_up of one intermediate column (rows j and W + j of a [2W][H] weight) against the np
// activation rows of an XTile: chunk-outer, pick-inner (the weights convert once a chunk);
// the per-(row, pick) arithmetic is the canonical order of WRows. -> g[p], u[p] in every lane
template <int FMT, int H>
struct GateUpCol {
  using R = WRows<FMT, H, 2, false>;
  using S = typename R::S;
  R wr;

  __device__ __forceinline__ void load(const uint8_t* w, const void* s, int W, int j, int lane) {
    wr.load(
        [&](int i, const uint8_t*& r, const void*& sr) {
          const int rid = i == 0 ? j : W + j;
          if constexpr (FMT == kFp8) {
            r = w + (size_t)rid * H;
            sr = (const float*)s + (size_t)(rid / 128) * (H / 128);
          } else {
            r = w + (size_t)rid * (H / 2);
            sr = (const uint8_t*)s + (size_t)rid * (H / 32);
          }
        },
        lane);
  }

  // NPB: the picks the code is unrolled for (np <= NPB)
  // wsc: the FP8 weight's block scales ((2W / 128) x (H / 128)); j: this column;
  // g[p], u[p] for p < np <= NPB
  template <int QS, int NPB>
  __device__ __forceinline__ void run(const uint8_t* xq, const uint8_t* xs, const float* wsc, int W, int j,
                                      int np, int lane, float* g, float* u) const {
#pragma clang fp contract(off)
    const int l = lane % S::LPR;
    float acc[R::RPG][NPB];
#pragma unroll
    for (int q = 0; q < R::RPG; ++q)
#pragma unroll
      for (int p = 0; p < NPB; ++p) acc[q][p] = 0.0f;
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) {
      const int c = l + S::LPR * i;
      if constexpr (FMT == kFp8) {
        float wf[R::RPG][16];
#pragma unroll
        for (int q = 0; q < R::RPG; ++q) {
          u32x4 wq = wr.w[q][i];
          asm volatile("" : "+v"(wq));
          const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[k], false);
            auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[k], true);
            wf[q][4 * k] = a[0];
            wf[q][4 * k + 1] = a[1];
            wf[q][4 * k + 2] = b[0];
            wf[q][4 * k + 3] = b[1];
          }
        }
#pragma unroll
        for (int p = 0; p < NPB; ++p) {
          if (p < np) {
            const u32x4 xv = *(const u32x4*)(xq + p * QS + c * 16);
            const float sx = ((const float*)xs)[p * (H / 128) + c / 8];
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
            float xf[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], false);
              auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], true);
              xf[4 * k] = a[0];
              xf[4 * k + 1] = a[1];
              xf[4 * k + 2] = b[0];
              xf[4 * k + 3] = b[1];
            }
#pragma unroll
            for (int q = 0; q < R::RPG; ++q) {
              float d = 0.0f;
#pragma unroll
              for (int k = 0; k < 16; ++k) d = fmaf(wf[q][k], xf[k], d);
              static_assert(FMT != kFp8 || S::G == 1, "FP8 gate and up rows in every lane");
              const float f = wsc[((q == 0 ? j : W + j) / 128) * (H / 128) + c / 8] * sx;
              acc[q][p] = acc[q][p] + d * f;
            }
          }
        }
      } else {
        float wf[R::RPG][32];
#pragma unroll
        for (int q = 0; q < R::RPG; ++q) {
          u32x4 wq = wr.w[q][i];
          asm volatile("" : "+v"(wq));
          const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            auto a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 0);
            auto b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 1);
            auto c2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 2);
            auto d2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 3);
            wf[q][8 * k] = a[0];
            wf[q][8 * k + 1] = a[1];
            wf[q][8 * k + 2] = b[0];
            wf[q][8 * k + 3] = b[1];
            wf[q][8 * k + 4] = c2[0];
            wf[q][8 * k + 5] = c2[1];
            wf[q][8 * k + 6] = d2[0];
            wf[q][8 * k + 7] = d2[1];
          }
        }
#pragma unroll
        for (int p = 0; p < NPB; ++p) {
          if (p < np) {
            const u32x4 xa = *(const u32x4*)(xq + p * QS + c * 32);
            const u32x4 xb = *(const u32x4*)(xq + p * QS + c * 32 + 16);
            const int ex = xs[p * (H / 32) + c];
            const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            float xf[32];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], false);
              auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], true);
              xf[4 * k] = a[0];
              xf[4 * k + 1] = a[1];
              xf[4 * k + 2] = b[0];
              xf[4 * k + 3] = b[1];
            }
#pragma unroll
            for (int q = 0; q < R::RPG; ++q) {
              float d = 0.0f;
#pragma unroll
              for (int k = 0; k < 32; ++k) d = fmaf(wf[q][k], xf[k], d);
              acc[q][p] = acc[q][p] + ldexpf(d, wr.se[q][i] + ex - 254);
            }
          }
        }
      }
    }
#pragma unroll
    for (int p = 0; p < NPB; ++p) {
      if (p < np) {
        if constexpr (S::G == 1) {
          g[p] = lane_value(tree_sum<64>(acc[0][p]), 0);
          u[p] = lane_value(tree_sum<64>(acc[1][p]), 0);
        } else {
          static_assert(S::G == 2, "gate and up on two sub-groups");
          const float t = tree_sum<32>(acc[0][p]);
          g[p] = lane_value(t, 0);
          u[p] = lane_value(t, 32);
        }
      }
    }
  }
};

// lane k (k < kTokGroup) receives a[k] of a wave-uniform array (lane writes, no indexing)
template <int K>
__device__ __forceinline__ void write_lane(float& v, float s) {
  const int u = __builtin_amdgcn_readfirstlane(__float_as_int(s));
  asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(u), "i"(K));
}
__device__ __forceinline__ float lane_pick(const float (&a)[kTokGroup]) {
  static_assert(kTokGroup == 8, "lanes written");
  float v = 0.0f;
  write_lane<0>(v, a[0]);
  write_lane<1>(v, a[1]);
  write_lane<2>(v, a[2]);
  write_lane<3>(v, a[3]);
  write_lane<4>(v, a[4]);
  write_lane<5>(v, a[5]);
  write_lane<6>(v, a[6]);
  write_lane<7>(v, a[7]);
  return v;
}

// one workgroup unit: columns [c0, c0 + cb) of a [2W][H] weight for np activation rows.
// When the unit has fewer columns than waves, its picks split over ps waves a column (each
// pick's sums are independent, so the split leaves the arithmetic as it is). Wave w takes
// the picks of part w % ps and columns c0 + w / ps, c0 + w / ps + 8 / ps, ..., one column
// in registers at a time (a wave's next column is requested as soon as its current one is
// computed). The activation rows are requested first (load_x fills an XRegs), then the
// first column, so the rows reach the tile without waiting for the weights;
// emit(p, column, g, u) runs in lane q for pick p = q0 + q
template <class C, int FMT, class WFn, class XFn, class EmitFn>
__device__ __forceinline__ void gu_unit(const Params& p, XTile<C>& xt, int np, int W, int c0, int cb, WFn weights,
                        XFn load_x, EmitFn emit) {
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  using GU = GateUpCol<FMT, C::H>;
  const uint8_t* wb;
  const void* sb;
  weights(wb, sb);
  int ps = 1;
  while (ps * 2 <= np && cb * ps < kWaves) ps *= 2;
  const int ppw = (np + ps - 1) / ps;           // picks a part
  const int q0 = (wave % ps) * ppw;             // this wave's first pick
  const int nq = max(0, min(ppw, np - q0));      // and its count
  const int cstep = kWaves / ps;
  const int end = c0 + cb;
  int col = c0 + wave / ps;
  if (nq == 0) col = end;
  XRegs<C, kTokGroup> xr;
  load_x(xr);
  if constexpr (FMT == kFp8) xr.load_wscales((const float*)sb, W);
  GU a;
  if (col < end) a.load(wb, sb, W, col, lane);
  __syncthreads();  // the previous unit is done with the tile
  xr.store(xt, np);
  __syncthreads();
  const uint8_t* xq = xt.q + q0 * XTile<C>::QS;
  const uint8_t* xs = xt.s + q0 * (C::H / 32);
  while (col < end) {
    float g[kTokGroup] = {}, u[kTokGroup] = {};
    a.template run<XTile<C>::QS, kTokGroup>(xq, xs, xt.wsc, W, col, nq, lane, g, u);
    const float gl = lane_pick(g), ul = lane_pick(u);
    if (lane < nq) emit(q0 + lane, col, gl, ul);
    col += cstep;
    if (col < end) a.load(wb, sb, W, col, lane);
  }
}

// this workgroup's share [lo, hi) of n items dealt evenly over nwg workgroups
__device__ __forceinline__ void even_share(int n, int b, int nwg, int& lo, int& hi) {
  lo = (int)((long long)n * b / nwg);
  hi = (int)((long long)n * (b + 1) / nwg);
}

// ---------------------------------------------------------------- MFMA expert GEMMs
// Launches with at least mfma_gate (gate_up) / mfma_down (down) rows run those expert GEMMs on
// v_mfma_f32_16x16x32_bf16 (the default: every row count; fewer rows run the fixed-order VALU
// GEMVs above). The weights reach the MFMA operands through LDS (LDS-direct loads of
// contiguous runs): the operand layout's own loads read 16 rows x 64 bytes a load, which
// streams at 5.1-5.3 TB/s against 6.6-6.8 TB/s for contiguous runs (load-only measurement, 57
// experts at 8 rows). The e4m3 and e2m1 codes convert to bf16
// exactly (with an E8M0 scale folded in, still exact), every bf16 x bf16 product is exact in
// fp32 and the instruction sums them like an fp32 chain (measured on gfx950: within 0.42 x
// 2^-24 x sum |products| of the exact sum). The fp8 MFMAs are not used: their sums drift by
// up to 267 x 2^-24 x sum |products|, enough to move bf16 outputs by two units in the last place.
// Lane l supplies row (A) / column (B) l % 16 and, as lane group j = l / 16, 8 of the 32 K of a
// step (A and B take the same K from the same places, so which 8 the hardware assigns them
// does not matter); C[m][n] lands in lane n + 16 (m / 4), element m % 4. Weights are the A
// operand (16 rows), picks the B operand (16 columns).
// FP8 weights: a 128-K step is four MFMAs on the raw codes (lane group j: K 16j .. 16j + 15
// and 64 + 16j .. 64 + 16j + 15 of the step, so that each 16-byte load reads 64 contiguous
// bytes of a row), then scaled by the weight's 128 x 128 block scale times the pick's
// group-128 scale as it is added to the sum. MXFP4 weights with MXFP8 activations: lane group
// j holds the step's 32-K block j and converts it with its row's and its column's E8M0 scales
// folded in, so every product is exactly scaled whichever block it came from; the four MFMAs
// accumulate across steps.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// 8 e4m3 codes (bytes of w0 then w1) times s, as bf16
__device__ __forceinline__ bf16x8 fp8x8(uint32_t w0, uint32_t w1, float s) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, s, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, s, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, s, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, s, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
// 8 e2m1 codes (the nibbles of w, low first) times s, as bf16
__device__ __forceinline__ bf16x8 fp4x8(uint32_t w, float s) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
// an E8M0 scale as a float (2^(e - 127))
__device__ __forceinline__ float e8m0(uint32_t e) { return e == 0u ? 0x1p-127f : __uint_as_float(e << 23); }
// an FP8 128-K step on MFMA: A and B 32 raw code bytes a lane each (lo then hi 16 bytes)
__device__ __forceinline__ f32x4 mma_fp8_step(u32x4 alo, u32x4 ahi, u32x4 blo, u32x4 bhi) {
  f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
  c = mfma_bf16(fp8x8(alo.x, alo.y, 1.0f), fp8x8(blo.x, blo.y, 1.0f), c);
  c = mfma_bf16(fp8x8(alo.z, alo.w, 1.0f), fp8x8(blo.z, blo.w, 1.0f), c);
  c = mfma_bf16(fp8x8(ahi.x, ahi.y, 1.0f), fp8x8(bhi.x, bhi.y, 1.0f), c);
  c = mfma_bf16(fp8x8(ahi.z, ahi.w, 1.0f), fp8x8(bhi.z, bhi.w, 1.0f), c);
  return c;
}
// an MXFP4 x MXFP8 128-K step, accumulated into c: a holds the lane's 32 e2m1 codes of its
// block (8 a word), sw its row's scale; blo / bhi the column's 32 code bytes of the same
// block, sx the column's scale
__device__ __forceinline__ f32x4 mma_fp4_step(u32x4 a, float sw, u32x4 blo, u32x4 bhi, float sx, f32x4 c) {
  c = mfma_bf16(fp4x8(a.x, sw), fp8x8(blo.x, blo.y, sx), c);
  c = mfma_bf16(fp4x8(a.y, sw), fp8x8(blo.z, blo.w, sx), c);
  c = mfma_bf16(fp4x8(a.z, sw), fp8x8(bhi.x, bhi.y, sx), c);
  c = mfma_bf16(fp4x8(a.w, sw), fp8x8(bhi.z, bhi.w, sx), c);
  return c;
}
// an MXFP4 x MXFP8 128-K step of two A operands (a0, a1: gate rows and up rows) against the
// same column codes, each of the column's four 8-K pieces converted once for both; each sum
// takes its pieces in the order of mma_fp4_step
__device__ __forceinline__ void mma_fp4_step2(u32x4 a0, float s0, u32x4 a1, float s1, u32x4 blo, u32x4 bhi, float sx,
                                              f32x4& c0, f32x4& c1) {
  const uint32_t bw[4][2] = {{blo.x, blo.y}, {blo.z, blo.w}, {bhi.x, bhi.y}, {bhi.z, bhi.w}};
  const uint32_t w0[4] = {a0.x, a0.y, a0.z, a0.w}, w1[4] = {a1.x, a1.y, a1.z, a1.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const bf16x8 b = fp8x8(bw[k][0], bw[k][1], sx);
    c0 = mfma_bf16(fp4x8(w0[k], s0), b, c0);
    c1 = mfma_bf16(fp4x8(w1[k], s1), b, c1);
  }
}

// an FP8 x MXFP8 128-K step with E8M0 32 x 32 weight scales (the V4.1 shared expert),
// accumulated into c: each lane's two 16-byte pieces (K 16 j .. and 64 + 16 j .. of the step)
// lie in 32-K blocks j / 2 and 2 + j / 2, converted with their own block's scales folded in
// (exact powers of two), so the products are exactly scaled whichever block they come from
__device__ __forceinline__ f32x4 mma_fp8mx_step(u32x4 alo, u32x4 ahi, float swl, float swh, u32x4 blo, u32x4 bhi,
                                                float sxl, float sxh, f32x4 c) {
  c = mfma_bf16(fp8x8(alo.x, alo.y, swl), fp8x8(blo.x, blo.y, sxl), c);
  c = mfma_bf16(fp8x8(alo.z, alo.w, swl), fp8x8(blo.z, blo.w, sxl), c);
  c = mfma_bf16(fp8x8(ahi.x, ahi.y, swh), fp8x8(bhi.x, bhi.y, sxh), c);
  c = mfma_bf16(fp8x8(ahi.z, ahi.w, swh), fp8x8(bhi.z, bhi.w, sxh), c);
  return c;
}

// an MXFP4 x MXFP8 128-K step on the scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4), no
// converts: A lane (m, j) holds row m's 32 e2m1 of K [32 j, 32 j + 32) (16 bytes), B lane
// (n, j) column n's e4m3 of K [16 j, 16 j + 16) then [64 + 16 j, 64 + 16 j + 16) (blo, bhi);
// each lane gives the E8M0 codes of the 32-K block j of its row (sa) and its column (sb), and
// the instruction scales every product by its block's codes (measured on gfx950 with exactly
// summable operands: this layout reproduces the exact dot). Its internal sum keeps fewer bits
// than fp32 (the known-answer test bounds it), so its launches are held to the numerics bar.
__device__ __forceinline__ f32x4 mma_fp4_scaled(u32x4 a, uint32_t sa, u32x4 blo, u32x4 bhi, uint32_t sb, f32x4 c) {
  const i32x8 av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
  const i32x8 bv = {(int)blo.x, (int)blo.y, (int)blo.z, (int)blo.w, (int)bhi.x, (int)bhi.y, (int)bhi.z, (int)bhi.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 0, 0, (int)sa, 0, (int)sb);
}

// 16 bytes a lane from a buffer straight into LDS: lane l's bytes land at lds + 16 l (lds
// the same in every lane of the wave)
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t rs, void* lds, uint32_t voff, int aux) {
  if (aux)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, kAuxDev);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// stage np activation rows into the tile: codes (qoff + t H) and scale bytes (soff + t H / 32)
// of rows t = tok(r) from the workspace, and, for an FP8 weight, its nw fp32 block scales
// (wsc, a read-only input); 1 KB LDS-direct loads spread over the waves, so no registers hold
// the rows on their way. Ends with the tile complete and visible to the workgroup.
template <class C, class TokFn>
__device__ __forceinline__ void stage_x_lds(const Params& p, XTile<C>& xt, int np, uint32_t qoff, uint32_t soff, TokFn tok,
                                            const float* wsc, int nw) {
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  const auto rs = ws_rsrc(p);
  constexpr int IPR = C::H / 1024;  // 1 KB loads a row of codes
  constexpr int RB = C::H / 32;     // scale bytes a row
  static_assert(C::H % 1024 == 0 && RB % 16 == 0, "1 KB code loads, 16-byte scale pieces");
  __syncthreads();  // the previous user of the tile is done
  for (int k = wave; k < np * IPR; k += kWaves) {
    const int r = k / IPR, i = k % IPR;
    lds_load16(rs, xt.q + r * XTile<C>::QS + i * 1024, qoff + (uint32_t)tok(r) * C::H + i * 1024 + lane * 16, 1);
  }
  const int sbytes = np * RB;
  for (int k = wave; k * 1024 < sbytes; k += kWaves) {
    const int off = k * 1024 + lane * 16;
    const bool ok = off < sbytes;  // the rest lands in the padding, from row 0
    const int r = ok ? off / RB : 0, in = ok ? off % RB : 0;
    lds_load16(rs, xt.s + k * 1024, soff + (uint32_t)tok(r) * RB + in, 1);
  }
  if (nw > 0) {
    const auto wr = __builtin_amdgcn_make_buffer_rsrc((void*)wsc, (short)0, nw * 4, 0x00020000);
    for (int k = wave; k * 256 < nw; k += kWaves) {
      const int off = k * 1024 + lane * 16;
      lds_load16(wr, (uint8_t*)xt.wsc + k * 1024, off < nw * 4 ? off : 0, 0);
    }
  }
  wait_vm0();
  __syncthreads();
}

// LDS of the gate_up stage: the VALU GEMVs' activation tile, or the MFMA units' weight slots
// (a wave's K slice of one unit: 2 H bytes) and the FP8 weight's block scales; and the waves'
// partial C tiles (gate, up)
template <class C>
struct GuSmem {
  // MXFP4: a wave's slot of its K slice's E8M0 scales of a unit (32 rows x 32 bytes)
  static constexpr int SSLOT = C::FMT == kFp4 || C::SFMT == kFp8Mx ? 1024 : 16;
  union {
    XTile<C> x;
    struct {
      uint8_t wslot[kWaves][2 * C::H];
      float wsc[XTile<C>::WSC];
      uint8_t sslot[kWaves][SSLOT];
    } m;
  };
  f32x4 red[2][kWaves][64];
};

// the rows of an MFMA gate_up unit of a [2W][H] weight, this wave's K steps (the 8 waves
// split the H / 128 steps evenly), in registers: FP8 units are 8 columns (one A operand: gate
// rows j0 .. j0 + 7 in A rows 0..7, up rows W + j0 .. in A rows 8..15), MXFP4 units 16 columns
// (A operands of gate rows j0 .. j0 + 15 and of up rows W + j0 ..): 56 registers a wave either way
template <class C, int WFMT, bool SH = false>
struct GuTile {
  static constexpr int KS = C::H / 128;
  static constexpr int SPW = KS / kWaves;
  static_assert(KS % kWaves == 0, "K steps split evenly over the waves");
  // FP8 (fp32 128 x 128 scales, or E8M0 32 x 32: MX) or MXFP4 weights
  static constexpr bool F8 = WFMT == kFp8 || WFMT == kFp8Mx;
  static constexpr int NA = F8 ? 1 : 2;   // A operands a K step
  static constexpr int NC = F8 ? 8 : 16;  // columns a unit
  static constexpr int NW = F8 ? 2 : 1;   // 16-byte words of a lane's step
  u32x4 a[NA][SPW][NW];
  // MXFP4: the E8M0 byte of the lane's row and block; MX FP8: the E8M0 bytes of the lane's
  // row's blocks of its two pieces (low byte: K 16 j .., next: 64 + 16 j ..)
  uint32_t sa[NA][SPW];

  // A unit's weight rows (FP8: gate rows j0 .. j0 + 7 then up rows W + j0 ..; MXFP4: 16 gate
  // rows then 16 up rows), this wave's K steps, go through the wave's LDS slot: LDS-direct
  // loads read them as runs of RB bytes a row (the operand layout's own loads read 64-byte
  // runs, which stream at about 5.1 against 6.6 TB/s: measured, loads alone). Chunk c (16 bytes)
  // of slot row r sits at position r * CPW + (c ^ key(r)), so that the 16 rows' reads of one
  // chunk fall in distinct banks.
  static constexpr int RW = F8 ? 16 : 32;              // slot rows
  static constexpr int RB = F8 ? SPW * 128 : SPW * 64;  // bytes a slot row
  static constexpr int CPW = RB / 16;
  static constexpr int SLOT = RW * RB;
  static_assert(SLOT == 2 * C::H && SLOT % 1024 == 0 && CPW % (F8 ? 8 : 4) == 0, "slot layout");
  static_assert(!SH || (WFMT == kFp4 && SLOT == 2 * SPW * 1024), "shuffled: a 1 KB block a row group and K step");
  // shuffled scales: the wave's K steps lie in the first three of the four 256-byte chunks (two
  // steps each) it loads from its first step's chunk (with an odd SPW the last wave's fourth
  // chunk lies past the 32-row block: the next block's bytes, or zeros past the tensor, unread)
  static_assert(!SH || (SPW + 2) / 2 <= 4, "scale chunks");
  __device__ __forceinline__ static int key(int r) { return F8 ? (r >> 1) : ((r & 15) >> 2); }
  __device__ __forceinline__ static int wrow(int W, int j0, int r) {
    return F8 ? (r < 8 ? j0 + r : W + j0 + r - 8) : (r >> 4) * W + j0 + (r & 15);
  }
  // w: the [2W][H] weight (wr: its resource words), sr: its MXFP4 scales' resource words
  // ([2W][H / 32] bytes); the unit's columns j0 .. j0 + nc - 1 (nc = NC, or NC / 2 at a
  // share's ends: the other rows are requested past the resource, so the slot holds zeros
  // there and no memory is read)
  // (part [b0, b1) of the unit's 1 KB blocks alone, and its scales with block 0: a wave can
  // spread its request over the current unit's K steps)
  static constexpr int kBlocks = SLOT / 1024;
  __device__ __forceinline__ void issue(i32x4 wr, i32x4 sr, int W, int j0, int nc, uint8_t* slot, uint8_t* sslot,
                                        int lane, int wave, int b0 = 0, int b1 = kBlocks) {
    const int s0 = wave * SPW;
    constexpr int ROWB = F8 ? C::H : C::H / 2;  // bytes a weight row
    if constexpr (SH) {
      // SGLang's layout: the column block's gate tile is row group 2 b and its up tile 2 b + 1
      // (16 rows each), stored per K step as 1 KB in the MFMA operand's lane order; slot
      // block q SPW + i takes K step s0 + i of tile q whole (lane l's 16 bytes at 16 l). The
      // scales of the 32 rows (one shuffle_scale block of H bytes) come in 256-byte chunks of
      // two K steps: the four from chunk s0 / 2 in one load
      const int b = j0 / 16;
#pragma unroll
      for (int blk = 0; blk < 2 * SPW; ++blk) {
        if (blk < b0 || blk >= b1) continue;
        const int q = blk / SPW, i = blk % SPW;
        lds_dma16(wr, slot + blk * 1024, (uint32_t)(2 * b + q) * 16 * ROWB + (s0 + i) * 1024 + lane * 16);
      }
      if (b0 == 0) lds_dma16_cached(sr, sslot, (uint32_t)b * C::H + (s0 / 2) * 256 + lane * 16);
      return;
    }
    // (MXFP4: a lane index the compiler cannot see through, so that a request spread over the
    // K steps computes each block's address where it is issued instead of holding them all,
    // which spilled 20-28 B)
    int ln = lane;
    if (WFMT == kFp4 && (b0 > 0 || b1 < kBlocks)) asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < SLOT / 1024; ++i) {
      if (i < b0 || i >= b1) continue;
      const int pos = i * 64 + ln, r = pos / CPW, c = (pos % CPW) ^ key(r);
      const bool live = (F8 ? (r & 7) : (r & 15)) < nc;
      lds_dma16(wr, slot + i * 1024, live ? (uint32_t)wrow(W, j0, r) * ROWB + s0 * (RB / SPW) + c * 16 : kNoLoad);
    }
    if (WFMT == kFp8Mx && b0 == 0) {
      // the E8M0 bytes of the wave's K steps (4 SPW from byte 4 s0) of the unit's two 32-row
      // scale blocks, gate (rows j0 / 32) then up (rows (W + j0) / 32), in one LDS-direct load:
      // lanes 0, 1 the gate row's 32 bytes from 4 s0, lanes 2, 3 the up row's, to sslot + 16 l
      static_assert(4 * SPW <= 32, "a scale row's slice in two 16-byte pieces");
      const int h = lane & 1, blk = (lane < 2 ? j0 : W + j0) / 32;
      lds_dma16_cached(sr, sslot, lane < 4 ? (uint32_t)blk * (C::H / 32) + s0 * 4 + h * 16 : kNoLoad);
    }
    if (WFMT == kFp4 && b0 == 0) {
      // the scales of the wave's K steps (4 SPW bytes a row, from byte 4 s0) in one LDS-direct
      // load: lane 2 r + h takes 16 bytes of row r from byte 16 h of its slice, to sslot + 32 r +
      // 16 h (the 32 - 4 SPW bytes past the slice are never read; past the resource the load
      // returns zeros). The 8 waves' slices of a row share its lines: cached loads
      static_assert(4 * SPW <= 32, "a row's slice in two 16-byte pieces");
      const int r = lane >> 1, h = lane & 1;
      const bool live = (r & 15) < nc;
      lds_dma16_cached(sr, sslot, live ? (uint32_t)wrow(W, j0, r) * (C::H / 32) + s0 * 4 + h * 16 : kNoLoad);
    }
  }
  __device__ __forceinline__ void fetch(const uint8_t* slot, const uint8_t* sslot, int lane, int wave) {
    const int m = lane & 15, j = lane >> 4;
    if constexpr (SH) {
      // lane (m, j)'s dword of a scale chunk holds its row's bytes of the chunk's two K steps,
      // gate and up: byte 2 (step % 2) + q
      const int s0 = wave * SPW;
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        const int st = s0 + i;
        const uint32_t dw = *(const uint32_t*)(sslot + ((st / 2 - s0 / 2) * 64 + lane) * 4);
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          a[q][i][0] = *(const u32x4*)(slot + (q * SPW + i) * 1024 + lane * 16);
          sa[q][i] = (dw >> (8 * (2 * (st & 1) + q))) & 0xffu;
        }
      }
      return;
    }
#pragma unroll
    for (int q = 0; q < NA; ++q)
#pragma unroll
      for (int i = 0; i < SPW; ++i)
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const int r = q * 16 + m;
          const int c = F8 ? i * 8 + j + 4 * w : i * 4 + j;
          a[q][i][w] = *(const u32x4*)(slot + (r * CPW + (c ^ key(r))) * 16);
        }
    if constexpr (WFMT == kFp8Mx) {
      // row m's scale row (gate rows 0..7, up rows 8..15), bytes 4 i + j / 2 and 4 i + 2 + j / 2
      const uint8_t* row = sslot + (m < 8 ? 0 : 32);
#pragma unroll
      for (int i = 0; i < SPW; ++i) sa[0][i] = row[4 * i + (j >> 1)] | ((uint32_t)row[4 * i + 2 + (j >> 1)] << 8);
    }
    if constexpr (WFMT == kFp4) {
      // byte j of dword i of row q 16 + m's slice: the E8M0 of the lane's row and block
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const u32x4 d0 = *(const u32x4*)(sslot + (q * 16 + m) * 32);
        const u32x4 d1 = *(const u32x4*)(sslot + (q * 16 + m) * 32 + 16);
        const uint32_t dw[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
        for (int i = 0; i < SPW; ++i) sa[q][i] = (dw[i] >> (8 * j)) & 0xffu;
      }
    }
  }
};

// a token group's activations for an MFMA gate_up, this wave's K steps, in registers: lane
// (n, j) holds pick n's codes of its K places (FP8: bytes 16 j .. and 64 + 16 j .. of each
// 128; MXFP8: 32 j .. 32 j + 31) and the scales. Lanes of picks past np hold pick 0's: an
// MFMA's output column n depends on column n of its B operand alone, and the columns past np
// are never emitted, so they are not zeroed
template <class C, int WFMT>
struct GuX {
  static constexpr int SPW = C::H / 128 / kWaves;
  u32x4 lo[SPW], hi[SPW];
  float sx[SPW];     // FP8: the pick's fp32 scale of the 128-block
  uint32_t ex[SPW];  // MXFP8: the E8M0 byte of the lane's 32-block; MX FP8: the step's four codes
  template <class TokFn>
  __device__ __forceinline__ void load(const Params& p, int np, uint32_t qoff, uint32_t soff, TokFn tok, int lane,
                                       int wave) {
    const int n = lane & 15, j = lane >> 4, s0 = wave * SPW;
    const bool live = n < np;
    const uint32_t t = (uint32_t)tok(live ? n : 0);
    const auto rs = ws_rsrc(p);
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const uint32_t k0 = (s0 + i) * 128;
      if constexpr (WFMT == kFp8) {
        lo[i] = dld128(rs, qoff + t * C::H + k0 + 16 * j);
        hi[i] = dld128(rs, qoff + t * C::H + k0 + 64 + 16 * j);
        sx[i] = u2f(dld32(rs, soff + (t * (C::H / 128) + s0 + i) * 4));
      } else if constexpr (WFMT == kFp8Mx) {
        // the codes as FP8's; the step's four E8M0 bytes (blocks 4 ks .. 4 ks + 3) in one dword
        lo[i] = dld128(rs, qoff + t * C::H + k0 + 16 * j);
        hi[i] = dld128(rs, qoff + t * C::H + k0 + 64 + 16 * j);
        ex[i] = dld32(rs, soff + t * (C::H / 32) + k0 / 32);
      } else {
        // the scaled MFMA takes K [16 j, 16 j + 16) and [64 + 16 j, ..); the converting path
        // the 32-K block j itself
        const uint32_t klo = p.mx_scaled ? 16 * j : 32 * j, khi = p.mx_scaled ? 64 + 16 * j : 32 * j + 16;
        lo[i] = dld128(rs, qoff + t * C::H + k0 + klo);
        hi[i] = dld128(rs, qoff + t * C::H + k0 + khi);
        ex[i] = dld8(rs, soff + t * (C::H / 32) + k0 / 32 + j);
      }
    }
  }
};

// this wave's partial C tiles of unit j0 over its K steps: t's weights against x's picks;
// wsc the FP8 weight's block scales in LDS
template <class C, int WFMT, bool SH, class StepFn>
__device__ __forceinline__ void gu_mma(const GuTile<C, WFMT, SH>& t, const GuX<C, WFMT>& x, const float* wsc, int W,
                                       int j0, int lane, int wave, bool scaled, f32x4 (&acc)[GuTile<C, WFMT, SH>::NA],
                                       StepFn after_step) {
  using T = GuTile<C, WFMT, SH>;
  const int s0 = wave * T::SPW;
#pragma unroll
  for (int q = 0; q < T::NA; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // FP8: this lane's C rows are gate rows (lanes 0..31) or up rows (lanes 32..63)
  const int sblk = ((lane < 32 ? j0 : W + j0) / 128) * (C::H / 128);
#pragma unroll
  for (int i = 0; i < T::SPW; ++i) {
    const int ks = s0 + i;
    if constexpr (WFMT == kFp8) {
      const float f = wsc[sblk + ks] * x.sx[i];
      const f32x4 c = mma_fp8_step(t.a[0][i][0], t.a[0][i][1], x.lo[i], x.hi[i]);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[0][v] = fmaf(c[v], f, acc[0][v]);
    } else if constexpr (WFMT == kFp8Mx) {
      const int jh = lane >> 5;  // (lane group j) / 2: the pieces' blocks are jh and 2 + jh
      const uint32_t sw = t.sa[0][i], xe = x.ex[i];
      acc[0] = mma_fp8mx_step(t.a[0][i][0], t.a[0][i][1], e8m0(sw & 0xffu), e8m0((sw >> 8) & 0xffu), x.lo[i], x.hi[i],
                              e8m0((xe >> (8 * jh)) & 0xffu), e8m0((xe >> (8 * (2 + jh))) & 0xffu), acc[0]);
    } else {
      static_assert(T::NA == 2, "gate and up rows");
      if (scaled) {
        acc[0] = mma_fp4_scaled(t.a[0][i][0], t.sa[0][i], x.lo[i], x.hi[i], x.ex[i], acc[0]);
        acc[1] = mma_fp4_scaled(t.a[1][i][0], t.sa[1][i], x.lo[i], x.hi[i], x.ex[i], acc[1]);
      } else {
        mma_fp4_step2(t.a[0][i][0], e8m0(t.sa[0][i]), t.a[1][i][0], e8m0(t.sa[1][i]), x.lo[i], x.hi[i],
                      e8m0(x.ex[i]), acc[0], acc[1]);
      }
    }
    after_step(i);
  }
}

// MFMA gate_up of units [lo, hi) of a [2W][H] weight whose first WR columns are real; unit u
// is token group u / (WR / NC) and its NC columns (u % (WR / NC)) * NC ... group(tg, w, s, np) gives a group's weight, scales and
// pick count, xload(tg, np, x) loads its activations into x, emit(tg, q, col, g, u) takes pick
// q's gate and up sums of a column. A wave's K slice of the next unit is requested into its
// LDS slot as soon as the current one is read out of it, so it streams while the current
// unit's MFMAs run and its partial tiles add in LDS (in wave order). An FP8 weight's block
// scales go to LDS when the group changes.
template <class C, int WFMT, bool HALF, bool SH, class GroupFn, class XFn, class EmitFn>
__device__ __forceinline__ void gu_mfma(GuSmem<C>& sm, int W, int WR, int lo_h, int hi_h, bool scaled, GroupFn group,
                                        XFn xload, EmitFn emit) {
  using T = GuTile<C, WFMT, SH>;
  if (lo_h >= hi_h) return;
  // HALF: the share is half-units [lo_h, hi_h): whole units, but at either end possibly one
  // half; else units [lo_h, hi_h)
  const int lo = HALF ? lo_h >> 1 : lo_h, hi = HALF ? (hi_h + 1) >> 1 : hi_h;
  auto half = [&](int u, int& c0, int& nc) {
    if constexpr (HALF) {
      c0 = u == lo && (lo_h & 1) ? T::NC / 2 : 0;
      nc = (u == hi - 1 && (hi_h & 1) ? T::NC / 2 : T::NC) - c0;
    } else {
      c0 = 0;
      nc = T::NC;
    }
  };
  const int tid = threadIdx.x, lane = tid & 63, wave = (int)(threadIdx.x >> 6);
  const int nb = WR / T::NC;  // units a token group
  constexpr uint32_t WB = T::F8 ? C::H : C::H / 2;  // bytes a weight row
  uint8_t* slot = sm.m.wslot[wave];
  uint8_t* sslot = sm.m.sslot[wave];
  // an MXFP4 weight's scales ([2W][H / 32] E8M0) as a resource (unused for FP8)
  auto srsc = [&](const void* sp) {
    return weight_rsrc_words(sp, WFMT == kFp4 ? 2u * W * (C::H / 32) : WFMT == kFp8Mx ? 2u * W / 32 * (C::H / 32) : 0u);
  };
  T t;
  GuX<C, WFMT> x;
  const uint8_t* wb;
  const void* sb;
  int tg_w = lo / nb, np_w;  // the group whose unit is in flight
  group(tg_w, wb, sb, np_w);
  __syncthreads();  // the LDS's previous users are done
  {
    int c0, nc;
    half(lo, c0, nc);
    t.issue(weight_rsrc_words(wb, 2u * W * WB), srsc(sb), W, (lo % nb) * T::NC + c0, nc, slot, sslot, lane, wave);
  }
  int tg_x = -1, np_x = 0;  // the group in x
  const void* sb_x = sb;
  for (int u = lo; u < hi; ++u) {
    int c0, ncu;
    half(u, c0, ncu);
    const int j0 = (u % nb) * T::NC + c0;
    const bool fresh = tg_w != tg_x;
    if (fresh) {
      xload(tg_w, np_w, x);
      tg_x = tg_w;
      np_x = np_w;
      sb_x = sb;
      if constexpr (WFMT == kFp8) {
        constexpr int nw = 2 * (C::I > C::S ? C::I : C::S) / 128 * (C::H / 128);
        const int nws = 2 * W / 128 * (C::H / 128);
        static_assert(nw <= XTile<C>::WSC, "block scales fit");
        const auto wr = __builtin_amdgcn_make_buffer_rsrc((void*)sb_x, (short)0, nws * 4, 0x00020000);
        for (int k = wave; k * 256 < nws; k += kWaves) {
          const int off = k * 1024 + lane * 16;
          lds_load16(wr, (uint8_t*)sm.m.wsc + k * 1024, off < nws * 4 ? off : 0, 0);
        }
      }
    }
    const unsigned long long tw0 = tl_now();
    wait_vm0();  // the unit's slot, the activations, the scales
    TL_ADD(kTlGuWait, tl_now() - tw0);
    TL_ADD(kTlGuUnits, 1ull);
    if (u == lo) TL(kTlGuFirst);
    if (fresh) __syncthreads();                       // every wave's block scales are in LDS
    const unsigned long long tf0 = tl_now();
    t.fetch(slot, sslot, lane, wave);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // read out of the slot
    // the next unit's request, spread over this unit's K steps (a share of its 1 KB blocks
    // after each step's MFMAs), so that the wave's loads queue behind one another less
    const bool more = u + 1 < hi;
    int c1 = 0, nc1 = 0;
    if (more) {
      const int tn = (u + 1) / nb;
      if (tn != tg_w) {
        tg_w = tn;
        group(tg_w, wb, sb, np_w);
      }
      half(u + 1, c1, nc1);
    }
    const i32x4 wr1 = weight_rsrc_words(wb, 2u * W * WB), sr1 = srsc(sb);
    const int j1 = ((u + 1) % nb) * T::NC + c1;
    const unsigned long long tf1 = tl_now();
    TL_ADD(kTlGuFetch, tf1 - tf0);
    f32x4 acc[T::NA];
    gu_mma<C, WFMT, SH>(t, x, sm.m.wsc, W, j0, lane, wave, scaled, acc, [&](int i) {
      if (more)
        t.issue(wr1, sr1, W, j1, nc1, slot, sslot, lane, wave, i * T::kBlocks / T::SPW, (i + 1) * T::kBlocks / T::SPW);
    });
#pragma unroll
    for (int q = 0; q < T::NA; ++q) sm.red[q][wave][lane] = acc[q];
    const unsigned long long tf2 = tl_now();
    TL_ADD(kTlGuMma, tf2 - tf1);
    __syncthreads();
    const unsigned long long tf3 = tl_now();
    TL_ADD(kTlGuSync, tf3 - tf2);
    if (tid < 16 * ncu) {
      // C[m][n] is element m % 4 of lane n + 16 (m / 4); FP8: up row m + 8 is 32 lanes on
      const int m = tid >> 4, n = tid & 15;
      const int L = n + 16 * (m >> 2), v = m & 3;
      const int qu = T::NA - 1, Lu = T::NA == 1 ? L + 32 : L;
      float g = 0.0f, uu = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        g = g + sm.red[0][w][L][v];
        uu = uu + sm.red[qu][w][Lu][v];
      }
      if (n < np_x) emit(tg_x, n, j0 + m, g, uu);
    }
    const unsigned long long tf4 = tl_now();
    TL_ADD(kTlGuEmit, tf4 - tf3);
    __syncthreads();
    TL_ADD(kTlGuSync2, tl_now() - tf4);
  }
}

// MFMA down: rows [hb, hb + 16 NA) of a [H][KD] weight (nv of them real), all K steps, in
// registers; mma() gives C[m][n] = row hb + 16 q + m against pick column n of an LDS mid tile,
// for each of the NA 16-row blocks q
template <int WFMT, int KD, int NA_ = 1, bool SH = false, int KR = KD>
struct DownTile {
  static constexpr int NA = NA_;  // 16-row A operands a unit
  // K past KR is a padded layout's zero weights: not loaded (the LDS takes zeros), and its
  // scales are taken as 1 (the shuffled layout)
  static_assert(KR == KD || (SH && KR % 32 == 0 && KR < KD), "a real K of whole MX blocks");
  static_assert(!SH || WFMT == kFp4, "the shuffled layout is MXFP4's");
  static constexpr bool kIsTile = true;
  // FP8 (fp32 128 x 128 scales, or E8M0 32 x 32: MX, whose K may end in half a step: the last
  // step's K 64 .. 127 are zeros) or MXFP4 weights
  static constexpr bool F8 = WFMT == kFp8 || WFMT == kFp8Mx;
  static_assert(KD % 128 == 0 || (WFMT == kFp8Mx && KD % 64 == 0), "whole (MX FP8: half) steps");
  static constexpr int KS = (KD + 127) / 128;
  static constexpr bool HALF = KD % 128 != 0;  // the last step's second half is past the row
  static constexpr int NW = F8 ? 2 : 1;  // 16-byte words of a lane's step
  // MXFP4 in SGLang's layout: a scale row's E8M0 columns, padded to a multiple of 8
  // (stages/dims.py:54-56, down_scale_cols)
  static constexpr int SC = (KD / 32 + 7) / 8 * 8;
  static constexpr int BYTES = NA * NW * 16 * 64 * KS;  // registers' bytes a unit
  // units a wave requests at once: 16 KB of codes (MXFP4 rows of 1024 K: one unit, leaving
  // registers for the conversions)
  static constexpr int kBatch =
      (WFMT == kFp4 && KS >= 8) || BYTES >= 16384 ? 1 : (16384 / BYTES > 4 ? 4 : 16384 / BYTES);
  static_assert(NA == 1 || WFMT == kFp4, "FP8 units are one 16-row block");
  u32x4 a[NA][KS][NW];
  // MXFP4: the E8M0 byte of the lane's row and block (load_scales<true>: the loaded dwords); MX
  // FP8: the lane's row block's codes of its two pieces' K blocks (low byte: 16 j .., next:
  // 64 + 16 j ..)
  uint32_t sa[NA][KS];
  float s0[KS], s1[KS];  // FP8: block scales of the lane's first and last C row
  int split;             // FP8: C elements v < split take s0, the rest s1

  // The unit through LDS. issue() requests its 16 NA rows into a wave's slot by LDS-direct
  // 16-byte loads, each load a contiguous KB of the weight (the operand layout's own loads read
  // 64-byte runs, which stream at about 5.1 against 6.6 TB/s: measured, loads alone). Chunk c
  // (16 bytes) of row r sits at slot position r * CPR + (c ^ (r % 16)), so that the 16 rows'
  // reads of one chunk fall in distinct banks. Rows past nv are requested past the resource
  // (zeros, no memory access). fetch() reads the slot into a[][] in the operand layout; the
  // scales travel in registers (load_scales, take_scales).
  static constexpr int RB = F8 ? KD : KD / 2;  // bytes a row
  static constexpr int CPR = RB / 16;         // chunks a row
  static constexpr int SLOT = 16 * NA * RB;   // bytes a unit
  // (row-major units through LDS: the swizzle needs CPR a power of two of 16 or more; the
  // shuffled layout's blocks go in whole)
  static constexpr bool kRowMajorSlot = CPR >= 16 && (CPR & (CPR - 1)) == 0 && SLOT % 1024 == 0;
  // wr: a resource over the weight from row 0 (H x RB bytes a matrix); wrow: the unit's first
  // row's byte offset in it
  __device__ __forceinline__ static void issue(__amdgpu_buffer_rsrc_t wr, uint32_t wrow, int nv, uint8_t* slot,
                                               int lane) {
    if constexpr (SH) {
      // SGLang's layout: a row's 16-byte piece j of K step ks sits in its 16-row group's 1 KB
      // block ks, at lane (row % 16) + 16 j (the unit's rows may straddle two groups). Slot
      // block q KS + ks takes the unit's rows 16 q .. of K step ks in the operand's lane
      // order, lane l's 16 bytes at 16 l
      const int m = lane & 15, j = lane >> 4;
      const uint32_t row0 = wrow / RB;
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const uint32_t row = row0 + q * 16 + m;
        const uint32_t base = (row / 16) * 16 * RB + ((row % 16) + 16 * j) * 16;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              wr, (__attribute__((address_space(3))) void*)(slot + (q * KS + ks) * 1024), 16,
              q * 16 + m < nv && ks * 128 + 32 * j < KR ? base + ks * 1024 : kNoLoad, 0, 0, kAuxNt);
      }
      return;
    }
    static_assert(SH || kRowMajorSlot, "slot layout");
#pragma unroll
    for (int i = 0; i < SLOT / 1024; ++i) {
      const int pos = i * 64 + lane;
      const int r = pos / CPR, c = (pos % CPR) ^ (r & 15);
      const uint32_t off = r < nv ? wrow + (uint32_t)r * RB + c * 16 : kNoLoad;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (__attribute__((address_space(3))) void*)(slot + i * 1024), 16,
                                               off, 0, 0, kAuxNt);
    }
  }
  __device__ __forceinline__ void fetch(const uint8_t* slot, int lane) {
    const int m = lane & 15, j = lane >> 4;
    if constexpr (SH) {
#pragma unroll
      for (int q = 0; q < NA; ++q)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) a[q][ks][0] = *(const u32x4*)(slot + (q * KS + ks) * 1024 + lane * 16);
      return;
    }
    static_assert(SH || kRowMajorSlot, "slot layout");
#pragma unroll
    for (int q = 0; q < NA; ++q)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const int c = F8 ? ks * 8 + j + 4 * w : ks * 4 + j;
          a[q][ks][w] = *(const u32x4*)(slot + ((q * 16 + m) * CPR + (c ^ m)) * 16);
        }
  }
  // the unit's scales alone (as load() sets them). FP8: the 128 x 128 block scales of the
  // lane's C rows; MXFP4: the lane's row's KD / 32 E8M0 bytes in 16-byte loads (byte j of
  // dword ks is its block's), rows past nv unit scales. RAW (MXFP4): sa keeps the loaded
  // dwords as they are and take_scales picks the lane's bytes out of them, so that nothing
  // waits for the loads here: a wave's loads complete in order, so a wait for the scales
  // would wait for the unit's weight rows requested just before them
  template <bool RAW = false>
  __device__ __forceinline__ void load_scales(const void* s, int hb, int nv, int lane) {
    const int m = lane & 15, j = lane >> 4;
    if constexpr (WFMT == kFp8) {
      const int r0 = hb + min(4 * j, nv - 1), r3 = hb + min(4 * j + 3, nv - 1);
      const float* sp = (const float*)s;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s0[ks] = sp[(r0 / 128) * (KD / 128) + ks];
        s1[ks] = sp[(r3 / 128) * (KD / 128) + ks];
      }
      split = r0 / 128 == r3 / 128 ? 4 : 128 - (hb + 4 * j) % 128;
    } else if constexpr (WFMT == kFp8Mx) {
      // E8M0 [H / 32][KD / 32]: lane (m, j) supplies A row hb + m (a unit may straddle two
      // 32-row blocks), its pieces of step ks in K blocks 4 ks + j / 2 and 4 ks + 2 + j / 2 (the
      // second past the row in a half step)
      const uint8_t* row = (const uint8_t*)s + (size_t)((hb + min(m, nv - 1)) / 32) * (KD / 32);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int b0 = 4 * ks + (j >> 1), b1 = b0 + 2;
        sa[0][ks] = row[b0] | (b1 < KD / 32 ? (uint32_t)row[b1] << 8 : 0u);
      }
    } else if constexpr (SH) {
      // shuffle_scale order (a [H][KD / 32] matrix of the expert): row h's bytes of K steps
      // 2 c and 2 c + 1, column j of each, are bytes 2 (step % 2) + (h / 16) % 2 of the dword
      // at 32-row block h / 32, chunk c (256 bytes), position 16 j + h % 16
      const uint8_t* ss = (const uint8_t*)s;
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const bool ok = q * 16 + m < nv;
        const int h = hb + (ok ? q * 16 + m : 0);
        const int a = (h >> 4) & 1;
        // chunk c (256 bytes) holds steps 2 c and 2 c + 1 (with an odd KS the last holds one);
        // a 32-row block's chunks are SC / 8 (the padded columns)
#pragma unroll
        for (int c = 0; c < (KS + 1) / 2; ++c) {
          const uint32_t dw = ok ? *(const uint32_t*)(ss + (size_t)(h / 32) * SC * 32 + c * 256 +
                                                      (16 * j + (h & 15)) * 4)
                                 : 0x7f7f7f7fu;
          if constexpr (RAW) {
            sa[q][2 * c] = dw;
          } else {
            sa[q][2 * c] = (dw >> (8 * a)) & 0xffu;
            if (2 * c + 1 < KS) sa[q][2 * c + 1] = (dw >> (8 * (2 + a))) & 0xffu;
          }
        }
      }
    } else {
      static_assert(KS % 4 == 0, "MXFP4 scales in 16-byte loads");
      const uint8_t* ss = (const uint8_t*)s;
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const bool ok = q * 16 + m < nv;
        const size_t h = (size_t)hb + (ok ? q * 16 + m : 0);
#pragma unroll
        for (int k4 = 0; k4 < KS; k4 += 4) {
          const u32x4 d = ok ? ld16(ss + h * (KD / 32) + k4 * 4) : u32x4{0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu};
          const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) sa[q][k4 + t] = RAW ? dw[t] : (dw[t] >> (8 * j)) & 0xffu;
        }
      }
    }
  }
  // the weight registers as values the compiler cannot see through: a loop over pick groups
  // converts them again each time instead of keeping the converted operands (twice the
  // registers) from the first
  __device__ __forceinline__ void opaque() {
#pragma unroll
    for (int q = 0; q < NA; ++q)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int w = 0; w < NW; ++w) asm volatile("" : "+v"(a[q][ks][w]));
  }
  // the scales o requested with load_scales<true> for the unit of first row hb, once they
  // have landed
  __device__ __forceinline__ void take_scales(const DownTile& o, int hb, int lane) {
    const int m = lane & 15, j = lane >> 4;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s0[ks] = o.s0[ks];
      s1[ks] = o.s1[ks];
    }
    if constexpr (WFMT == kFp4 && SH) {
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        const int a = ((hb + q * 16 + m) >> 4) & 1;  // rows past nv: 0x7f in every byte
#pragma unroll
        for (int c = 0; c < (KS + 1) / 2; ++c) {
          const uint32_t dw = o.sa[q][2 * c];
          sa[q][2 * c] = (dw >> (8 * a)) & 0xffu;
          if (2 * c + 1 < KS) sa[q][2 * c + 1] = (dw >> (8 * (2 + a))) & 0xffu;
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          if (ks * 128 + 96 >= KR && ks * 128 + 32 * j >= KR) sa[q][ks] = 127u;
      }
    } else if constexpr (WFMT == kFp4) {
#pragma unroll
      for (int q = 0; q < NA; ++q)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) sa[q][ks] = (o.sa[q][ks] >> (8 * j)) & 0xffu;
    } else if constexpr (WFMT == kFp8Mx) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sa[0][ks] = o.sa[0][ks];
    }
    split = o.split;
  }

  // w: row 0 of the weight; s: its scales (FP8 [H / 128][KD / 128] fp32, MXFP4 [H][KD / 32])
  __device__ __forceinline__ void load(const uint8_t* w, const void* s, int hb, int nv, int lane) {
    static_assert(NA == 1 && !SH, "register units are one row-major 16-row block");
    const int m = lane & 15, j = lane >> 4;
    const bool ok = m < nv;
    const size_t h = (size_t)hb + (ok ? m : 0);
    if constexpr (F8) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint8_t* p = w + h * KD + ks * 128 + 16 * j;
        const bool tail = HALF && ks == KS - 1;  // K 64 .. 127 of the step: past the row
        if (ok) {
          a[0][ks][0] = ld16_nt(p);
          a[0][ks][1] = tail ? u32x4{0u, 0u, 0u, 0u} : ld16_nt(p + 64);
        } else {
          a[0][ks][0] = a[0][ks][1] = u32x4{0u, 0u, 0u, 0u};
        }
      }
      load_scales(s, hb, nv, lane);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        a[0][ks][0] = ok ? ld16_nt(w + h * (KD / 2) + ks * 64 + 16 * j) : u32x4{0u, 0u, 0u, 0u};
      load_scales(s, hb, nv, lane);
    }
  }

  // C tiles (one a 16-row block) against picks [lp, lp + np) of the LDS mid rows (codes xq, row
  // stride QS; scales xs, SST bytes a row: fp32 per 128, or E8M0 per 32)
  template <int QS, int SST>
  __device__ __forceinline__ void mma(const uint8_t* xq, const uint8_t* xs, int lp, int np, int lane, bool scaled,
                                      f32x4 (&acc)[NA]) const {
    // (lanes of picks past np read pick lp's row: their output columns are never stored, and
    // an output column depends on its own B column alone)
    const int n = lane & 15, j = lane >> 4;
    const int row = lp + (n < np ? n : 0);
    const uint8_t* xr = xq + (size_t)row * QS;
#pragma unroll
    for (int q = 0; q < NA; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (WFMT == kFp8Mx) {
        const bool tail = HALF && ks == KS - 1;
        u32x4 blo = *(const u32x4*)(xr + ks * 128 + 16 * j);
        u32x4 bhi = tail ? u32x4{0u, 0u, 0u, 0u} : *(const u32x4*)(xr + ks * 128 + 64 + 16 * j);
        const int b0 = 4 * ks + (j >> 1);
        const float sxl = e8m0(xs[row * SST + b0]), sxh = tail ? 1.0f : e8m0(xs[row * SST + b0 + 2]);
        const uint32_t sw = sa[0][ks];
        acc[0] = mma_fp8mx_step(a[0][ks][0], a[0][ks][1], e8m0(sw & 0xffu), e8m0((sw >> 8) & 0xffu), blo, bhi, sxl, sxh,
                                acc[0]);
      } else if constexpr (WFMT == kFp8) {
        u32x4 blo = *(const u32x4*)(xr + ks * 128 + 16 * j), bhi = *(const u32x4*)(xr + ks * 128 + 64 + 16 * j);
        const float sx = ((const float*)(xs + row * SST))[ks];
        const f32x4 c = mma_fp8_step(a[0][ks][0], a[0][ks][1], blo, bhi);
        const float f0 = s0[ks] * sx, f1 = s1[ks] * sx;
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[0][v] = fmaf(c[v], v < split ? f0 : f1, acc[0][v]);
      } else if (scaled) {
        // the scaled MFMA's K layout for the column (see mma_fp4_scaled)
        u32x4 blo = *(const u32x4*)(xr + ks * 128 + 16 * j), bhi = *(const u32x4*)(xr + ks * 128 + 64 + 16 * j);
        const uint32_t sx = xs[row * SST + ks * 4 + j];
#pragma unroll
        for (int q = 0; q < NA; ++q) acc[q] = mma_fp4_scaled(a[q][ks][0], sa[q][ks], blo, bhi, sx, acc[q]);
      } else {
        u32x4 blo = *(const u32x4*)(xr + ks * 128 + 32 * j), bhi = *(const u32x4*)(xr + ks * 128 + 32 * j + 16);
        const float sx = e8m0(xs[row * SST + ks * 4 + j]);
        if constexpr (NA == 2) {
          mma_fp4_step2(a[0][ks][0], e8m0(sa[0][ks]), a[1][ks][0], e8m0(sa[1][ks]), blo, bhi, sx, acc[0], acc[1]);
        } else {
          acc[0] = mma_fp4_step(a[0][ks][0], e8m0(sa[0][ks]), blo, bhi, sx, acc[0]);
        }
      }
    }
  }
};

// ---------------------------------------------------------------- stage B: routing
// a workgroup per row (workgroups 0 .. R-1)
template <class C>
__device__ __forceinline__ void stage_b(const Params& p, RouteSmem<C>& sm, int b, int nwg) {
  for (int r = b; r < p.rows; r += nwg) {
    __syncthreads();  // the previous row's selection is done with the LDS
    route_row<C>(p, sm, r);
  }
}

// ---------------------------------------------------------------- the step's union (LDS)
// token groups of a step at most: the routed ones (one a pick at most), then the shared
// expert's (its rows in groups of kTokGroup)
template <class C>
constexpr int kMaxGroups = kRowsMax * C::K + kRowsMax / kTokGroup;

template <class C>
struct Union {
  uint32_t rows_of[C::E][2];  // rows (bit r) that picked expert e
  int cnt[C::E];
  int slot_of[C::E];
  int slot_e[C::E];
  int slot_start[C::E + 1];
  int tg_start[C::E + 1];          // a slot's first token group (kTokGroup picks, MFMA: kMfmaPicks)
  int tg_slot[kMaxGroups<C>];      // a routed token group's slot
  int picks[kRowsMax * C::K];
  int ids[kRowsMax * C::K];  // pick -> expert (row * topk + k)
  float wts[kRowsMax * C::K];
  int tg_cost[kMaxGroups<C> + 1];  // gate_up cost of the token groups before g, a column
  int n;
  int ntg_r;  // routed token groups: [0, ntg_r); the shared expert's: [ntg_r, ntg)
  int ntg;
};

// a gate_up column's cost in units of one pick's arithmetic: its weight loads (kColCost) plus
// one per pick. Fitted to per-workgroup gate_up times at 8 and 48 rows (FP8 and MXFP4 alike:
// 0.33-0.35 us a column + 0.17-0.19 us a column-pick, i.e. a column costs 1.9 picks)
constexpr int kColCost = 2;

// experts picked by any row (ascending id), their picks (pick = row * K + k; a slot's picks
// in row order, the same in every workgroup) and token groups. The routing comes from
// un.ids / un.wts when this workgroup routed the step itself (local), else from the workspace.
template <class C>
__device__ __forceinline__ void build_union(const Params& p, Union<C>& un, bool local) {
  static_assert(kRowsMax <= 64, "row bitmaps");
  const int tid = threadIdx.x;
  const int npk = p.rows * C::K;
  const int tgs = gate_on_mfma<C>(p.rows, p.mfma_gate) ? kMfmaPicks : kTokGroup;  // picks a token group
  const auto rs = ws_rsrc(p);
  __syncthreads();
  // one pick a thread; its expert is kept for the placement below. local: the routing left
  // the picks and the row bitmaps in LDS
  static_assert(kRowsMax * C::K <= kThreads, "a pick a thread");
  const int t = tid;
  int my_e = 0;
  if (local) {
    if (t < npk) my_e = un.ids[t];
  } else {
    for (int e = tid; e < C::E; e += kThreads) un.rows_of[e][0] = un.rows_of[e][1] = 0u;
    __syncthreads();
    if (t < npk) {
      my_e = min(max((int)dld32(rs, p.off[6] + t * 4), 0), C::E - 1);
      un.ids[t] = my_e;
      un.wts[t] = u2f(dld32(rs, p.off[7] + t * 4));
      const int r = t / C::K;
      atomicOr(&un.rows_of[my_e][r >> 5], 1u << (r & 31));
    }
    __syncthreads();
  }
  // wave 0: lane l takes experts l * EPL .. l * EPL + EPL - 1: slots, picks, token groups and
  // their gate_up costs (a group of c picks costs kColCost + c a column), prefix-summed
  if (tid < 64) {
    constexpr int EPL = (C::E + 63) / 64;
    const int e0 = tid * EPL;
    int cnt[EPL];
    int ns = 0, np = 0, ng = 0, nc = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = e0 + i;
      cnt[i] = e < C::E ? __popc(un.rows_of[e][0]) + __popc(un.rows_of[e][1]) : 0;
      const int groups = (cnt[i] + tgs - 1) / tgs;
      ns += cnt[i] > 0 ? 1 : 0;
      np += cnt[i];
      ng += groups;
      nc += groups * kColCost + cnt[i];
    }
    // exclusive prefixes over lanes
    const int is = wave_incl_scan(ns), ip = wave_incl_scan(np), ig = wave_incl_scan(ng), ic = wave_incl_scan(nc);
    int s = is - ns, pk = ip - np, gq = ig - ng, run = ic - nc;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = e0 + i;
      const int c = cnt[i];
      if (c > 0) {
        const int groups = (c + tgs - 1) / tgs;
        un.slot_of[e] = s;
        un.slot_e[s] = e;
        un.slot_start[s] = pk;
        un.tg_start[s] = gq;
        for (int q = 0; q < groups; ++q) {
          un.tg_slot[gq + q] = s;
          un.tg_cost[gq + q] = run;
          run += kColCost + min(tgs, c - q * tgs);
        }
        un.cnt[e] = pk;  // fill cursor
        s += 1;
        pk += c;
        gq += groups;
      }
    }
    if (tid == 63) {
      // then the shared expert's groups of its rows
      const int ntg = ig + (p.rows + tgs - 1) / tgs;
      un.n = is;
      un.slot_start[is] = ip;
      un.tg_start[is] = ig;
      un.ntg_r = ig;
      un.ntg = ntg;
      for (int g = ig; g < ntg; ++g) {
        un.tg_cost[g] = run;
        run += kColCost + min(tgs, p.rows - (g - ig) * tgs);
      }
      un.tg_cost[ntg] = run;
    }
  }
  __syncthreads();
  // a pick's place: its slot's start + the rows below its own that picked the same expert
  if (t < npk) {
    const int e = my_e;
    const int r = t / C::K;
    const uint32_t below0 = r >= 32 ? 0xffffffffu : (1u << r) - 1u;
    const uint32_t below1 = r >= 32 ? (1u << (r - 32)) - 1u : 0u;
    const int pos = un.cnt[e] + __popc(un.rows_of[e][0] & below0) + __popc(un.rows_of[e][1] & below1);
    un.picks[min(pos, npk - 1)] = t;
  }
  __syncthreads();
}

// ---------------------------------------------------------------- down GEMVs (8 lanes a row)
// A down unit is 8 weight rows of KD elements, one a group of 8 lanes: lane l of group g
// holds chunks l, l + 8, ... of row g (16-byte loads, so every load instruction reads eight
// 128-byte runs). The order is the fixed GEMV order with 8 lanes a row: each chunk's exact
// products summed in element order and scaled, a lane's chunks summed in order, then the
// 8 lanes' halving tree.
constexpr int kDownLanes = 8;
constexpr int kPickBlock = 4;  // picks a down unit computes per pass over its chunks

template <int FMT, int KD>
struct DownRows {
  static constexpr bool kIsTile = false;
  static constexpr int CE = FMT == kFp4 ? 32 : 16;  // elements a chunk
  static constexpr int CPR = KD / CE;
  static constexpr int CPL = CPR / kDownLanes;
  // units a wave requests at once (the VALU GEMVs run when a call asks for them: more units in
  // flight would spill the launch's registers)
  static constexpr int kBatch = 4;
  static_assert(CPR % kDownLanes == 0, "down row chunks");
  u32x4 w[CPL];
  float sf[CPL];
  int se[CPL];

  // this lane's row (w: its first byte, s: its scales: FP8 the row block's fp32 scales,
  // one per 128 K; FP4 its E8M0 bytes); ok false: the row is past the tile
  __device__ __forceinline__ void load(const uint8_t* r, const void* s, bool ok, int l) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) w[i] = ok ? ld16_nt(r + (l + kDownLanes * i) * 16) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = l + kDownLanes * i;
      if constexpr (FMT == kFp8) sf[i] = ok ? ((const float*)s)[c / 8] : 0.0f;
      else se[i] = ok ? (int)((const uint8_t*)s)[c] : 0;
    }
  }

  // acc[q] = this lane's sum for pick q < np of the LDS activation rows xq + q * QS
  // (codes) and xs + q * SST (scales: fp32 per 128, or E8M0 bytes per 32)
  template <int QS, int SST>
  __device__ __forceinline__ void dot(const uint8_t* xq, const uint8_t* xs, int np, int l,
                                      float (&acc)[kPickBlock]) const {
#pragma clang fp contract(off)
#pragma unroll
    for (int q = 0; q < kPickBlock; ++q) acc[q] = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = l + kDownLanes * i;
      u32x4 wq = w[i];
      asm volatile("" : "+v"(wq));
      const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
      if constexpr (FMT == kFp8) {
        float wf[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[k], false);
          auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)wv[k], true);
          wf[4 * k] = a[0];
          wf[4 * k + 1] = a[1];
          wf[4 * k + 2] = b[0];
          wf[4 * k + 3] = b[1];
        }
#pragma unroll
        for (int q = 0; q < kPickBlock; ++q) {
          if (q < np) {
            const u32x4 xv = *(const u32x4*)(xq + q * QS + c * 16);
            const float sx = ((const float*)(xs + q * SST))[c / 8];
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
            float d = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], false);
              auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], true);
              d = fmaf(wf[4 * k], a[0], d);
              d = fmaf(wf[4 * k + 1], a[1], d);
              d = fmaf(wf[4 * k + 2], b[0], d);
              d = fmaf(wf[4 * k + 3], b[1], d);
            }
            acc[q] = acc[q] + d * (sf[i] * sx);
          }
        }
      } else {
        float wf[32];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          auto a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 0);
          auto b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 1);
          auto c2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 2);
          auto d2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wv[k], 1.0f, 3);
          wf[8 * k] = a[0];
          wf[8 * k + 1] = a[1];
          wf[8 * k + 2] = b[0];
          wf[8 * k + 3] = b[1];
          wf[8 * k + 4] = c2[0];
          wf[8 * k + 5] = c2[1];
          wf[8 * k + 6] = d2[0];
          wf[8 * k + 7] = d2[1];
        }
#pragma unroll
        for (int q = 0; q < kPickBlock; ++q) {
          if (q < np) {
            const u32x4 xa = *(const u32x4*)(xq + q * QS + c * 32);
            const u32x4 xb = *(const u32x4*)(xq + q * QS + c * 32 + 16);
            const int ex = xs[q * SST + c];
            const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            float d = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], false);
              auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)xw[k], true);
              d = fmaf(wf[4 * k], a[0], d);
              d = fmaf(wf[4 * k + 1], a[1], d);
              d = fmaf(wf[4 * k + 2], b[0], d);
              d = fmaf(wf[4 * k + 3], b[1], d);
            }
            acc[q] = acc[q] + ldexpf(d, se[i] + ex - 254);
          }
        }
      }
    }
  }
};

// units v = wave, wave + 8, ... < n in batches of B (32 KB of an 8-row unit's weights a
// wave a batch at most): a batch's loads are issued together and computed once all have
// arrived, then the next batch is requested. (Two batches in flight per wave stream the
// down rows at half the rate: measured on this pattern, 3.1 against 6.5 TB/s.) The first
// batch may be requested ahead by the caller (first(rows)) before other work.
template <class Rows>
struct DownBatch {
  static constexpr int B = Rows::kBatch;
  Rows r[B];
  int v0;
  template <class LoadFn>
  __device__ __forceinline__ void load(int v, int n, LoadFn load_unit) {
    v0 = v;
#pragma unroll
    for (int k = 0; k < B; ++k)
      if (v + kWaves * k < n) load_unit(v + kWaves * k, r[k]);
  }
};

// run units v = wave, wave + 8, ... < n from a batch already requested for v = wave
template <class Rows, class LoadFn, class WorkFn>
__device__ __forceinline__ void down_pipeline(DownBatch<Rows>& bt, int n, LoadFn load, WorkFn work) {
  constexpr int B = DownBatch<Rows>::B;
  while (bt.v0 < n) {
#pragma unroll
    for (int k = 0; k < B; ++k)
      if (bt.v0 + kWaves * k < n) work(bt.v0 + kWaves * k, bt.r[k]);
    const int v1 = bt.v0 + kWaves * B;
    if (v1 >= n) break;
    bt.load(v1, n, load);
  }
}

// quantize bf16 rows [n][W] (workspace, sc1) into LDS codes [n][QS] and scales: group-128 fp8
// (fp32 scales) or MXFP8 (E8M0 bytes); row i of the source starts at byte ``src_row(i)``.
// A thread's chunks (8 values each) are requested NB at a time before any is
// converted, so a batch costs one trip to memory.
constexpr int kQuantBatch = 4;
// The rule by FMT, the weight format the rows feed: group-128 fp8 with fp32 scales (kFp8), MXFP8
// per 32 with the "aiter" code (kFp4) or the "vllm" code (kFp8Mx), E8M0 bytes
template <int FMT, int W, int QS, int NB = kQuantBatch, int WR = W, class RowFn>
__device__ __forceinline__ void quant_rows_lds(const Params& p, RowFn src_row, int n, uint8_t* q, void* s) {
#pragma clang fp contract(off)
  constexpr int PER = W / 8;  // 8-value chunks a row
  constexpr int RPER = WR / 8;  // ... of them real: the rest quantize zeros (nothing is read)
  // a group's chunks lie in adjacent lanes of one wave (rows hold whole groups)
  static_assert(PER % (FMT == kFp8 ? 16 : 4) == 0, "whole groups a row");
  const int tid = threadIdx.x;
  const auto rs = ws_rsrc(p);
  // a wave's lanes cover consecutive chunks so that a group's lanes are adjacent
  const int total = n * PER;
  for (int base = 0; base < total; base += NB * kThreads) {
    u32x4 xv[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int idx = base + k * kThreads + tid;
      if (idx < total && (RPER == PER || idx % PER < RPER)) xv[k] = dld128(rs, src_row(idx / PER) + (idx % PER) * 16);
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int idx = base + k * kThreads + tid;
      if (base + k * kThreads >= total) break;  // uniform: no chunk of this round is left
      const bool ok = idx < total;
      const int i = ok ? idx / PER : 0, c = ok ? idx % PER : 0;
      float v[8];
      float am = 0.0f;
      if (ok && (RPER == PER || c < RPER)) {
        const uint32_t xw[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = bf_lo(xw[j]);
          v[2 * j + 1] = bf_hi(xw[j]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) am = fabsf(v[j]) > am ? fabsf(v[j]) : am;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.0f;
      }
      if constexpr (FMT == kFp8) {
        float g = group_max<16>(am);
        float sc = group_scale(g);
        const uint32_t lo = e4m3_pack4(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
        const uint32_t hi = e4m3_pack4(v[4] / sc, v[5] / sc, v[6] / sc, v[7] / sc);
        if (ok) {
          *(u32x2*)(q + (size_t)i * QS + c * 8) = u32x2{lo, hi};
          if ((c & 15) == 0) ((float*)s)[i * (W / 128) + c / 16] = sc;
        }
      } else {
        float g = group_max<4>(am);
        int code = FMT == kFp8Mx ? vllm_code(g) : mx_code(g);
        float inv = mx_inv(code);
        const uint32_t lo = e4m3_pack4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
        const uint32_t hi = e4m3_pack4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
        if (ok) {
          *(u32x2*)(q + (size_t)i * QS + c * 8) = u32x2{lo, hi};
          if ((c & 3) == 0) ((uint8_t*)s)[i * (W / 32) + c / 4] = (uint8_t)code;
        }
      }
    }
  }
}


// quantize one bf16 row of W values (workspace byte src) into the workspace by one wave: codes
// at dq (8 bytes a chunk of 8 values), scales at ds; group-128 fp8 (fp32 scales) or MXFP8
// (E8M0 bytes), the arithmetic of quant_rows_lds
template <int FMT, int W, int WR = W>
__device__ __forceinline__ void quant_row_ws(const Params& p, uint32_t src, uint32_t dq, uint32_t ds, int lane) {
#pragma clang fp contract(off)
  constexpr int PER = W / 8;  // 8-value chunks a row
  constexpr int RPER = WR / 8;  // ... of them real: the rest quantize zeros (nothing is read)
  constexpr int CPL = (PER + 63) / 64;
  // the chunks past the row (a last round of fewer than 64) are whole groups of lanes, which
  // load and store nothing
  static_assert(PER % (FMT == kFp8 ? 16 : 4) == 0, "whole groups a row");
  const auto rs = ws_rsrc(p);
#pragma unroll 1
  for (int t = 0; t < CPL; ++t) {
    const int c = lane + 64 * t;
    const bool ok = PER % 64 == 0 || c < PER;
    const u32x4 xv = ok && (RPER == PER || c < RPER) ? dld128(rs, src + c * 16) : u32x4{0u, 0u, 0u, 0u};
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    float v[8];
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf_lo(xw[j]);
      v[2 * j + 1] = bf_hi(xw[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) am = fabsf(v[j]) > am ? fabsf(v[j]) : am;
    if constexpr (FMT == kFp8) {
      const float g = group_max<16>(am);
      const float sc = group_scale(g);
      const uint32_t lo = e4m3_pack4(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
      const uint32_t hi = e4m3_pack4(v[4] / sc, v[5] / sc, v[6] / sc, v[7] / sc);
      if (ok) dst64(rs, dq + c * 8, u32x2{lo, hi});
      if (ok && (c & 15) == 0) dst32(rs, ds + (c / 16) * 4, f2u(sc));
    } else {
      const float g = group_max<4>(am);
      const int code = FMT == kFp8Mx ? vllm_code(g) : mx_code(g);
      const float inv = mx_inv(code);
      const uint32_t lo = e4m3_pack4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
      const uint32_t hi = e4m3_pack4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
      if (ok) dst64(rs, dq + c * 8, u32x2{lo, hi});
      if (ok && (c & 3) == 0) dst8(rs, ds + c / 4, (uint8_t)code);
    }
  }
}

// workspace bytes [src, src + n) (hand-off data: device-coherent loads) into LDS at dst, by
// 16-byte LDS-direct loads, a wave a KB in turn; n and the addresses 16-byte aligned. The
// caller waits (vmcnt) and syncs before the rows are read.
__device__ __forceinline__ void ws_to_lds(const Params& p, uint32_t src, uint32_t n, uint8_t* dst) {
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  const auto rs = ws_rsrc(p);
  for (uint32_t kb = wave; kb * 1024 < n; kb += kWaves) {
    const uint32_t off = kb * 1024 + lane * 16;
    if (off < n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + kb * 1024), 16,
                                               src + off, 0, 0, kAuxDev);
  }
}

// row blocks of 8 in a down tile (rows past the tile masked)
constexpr int kRowBlocks = kTileMax / kDownLanes;

// ---------------------------------------------------------------- stage C: gate_up
// the shared expert's down GEMV for tile rows [h0, h0 + hn) of every row (VALU: units of an
// 8-row block and kPickBlock rows; MFMA: a 16-row block and 16 rows), into the tile's bf16
// results; the shared intermediate is quantized into LDS first
template <class C>
struct SharedDownSmem {
  uint8_t q[kRowsMax * C::SQS];
  float s[(kRowsMax * C::SSC + 3) / 4];  // fp32 per 128 or E8M0 per 32 (C::SSC bytes a row)
};

// the shared down's units a wave requests at once: one (MFMA: a 16-row block for every row of
// the step; a 28-row tile has two), up to two 8-row blocks (VALU)
template <class Rows>
struct Batched : Rows {
  static constexpr int kBatch = Rows::kBatch < 2 ? Rows::kBatch : (Rows::kIsTile ? 1 : 2);
};
template <class C, bool MF>
using SharedDownBatch =
    DownBatch<Batched<typename std::conditional<MF, DownTile<C::SFMT, C::S>, DownRows<kFp8, C::S>>::type>>;

// loader of the shared down's units of tile rows [h0, h0 + hn) (MFMA: unit v is the 16-row
// block v, for every row of the step; VALU: an 8-row block and kPickBlock rows)
template <class C, bool MF>
__device__ __forceinline__ auto shared_down_loader(const Params& p, int h0, int hn) {
  const int lane = threadIdx.x & 63, g = lane / kDownLanes, l = lane % kDownLanes;
  if constexpr (MF) {
    return [&p, h0, hn, lane](int v, DownTile<C::SFMT, C::S>& dt) {
      dt.load(p.sw2, p.sw2_s, h0 + v * 16, min(16, hn - v * 16), lane);
    };
  } else {
    return [&p, h0, hn, g, l](int v, DownRows<kFp8, C::S>& wr) {
      const int rb = v % kRowBlocks;
      const int h = h0 + rb * kDownLanes + g;
      wr.load(p.sw2 + (size_t)h * C::S, p.sw2_s + (size_t)(h / 128) * (C::S / 128), rb * kDownLanes + g < hn, l);
    };
  }
}
template <class C, bool MF>
__device__ __forceinline__ int shared_down_units(int R, int hn) {
  if constexpr (MF) return (hn + 15) / 16;
  else return kRowBlocks * ((R + kPickBlock - 1) / kPickBlock);
}
// the wave that takes the shared down's unit v first: wave 1 unit 0 and so on, wave 0 last (its
// unit is requested after the hand-off it polls)
__device__ __forceinline__ int shared_down_vwave() { return ((int)(threadIdx.x >> 6) + kWaves - 1) % kWaves; }


// the shared down of tile rows [h0, h0 + hn) into out[t * hn + hl] (bf16); first_ready: the
// first units of waves 1-7 are already requested into bt (shared_down_first); GQ: the step's
// rows were quantized by stage Q (launches of C::QROWS rows or more)
template <class C, bool MF, bool GQ>
__device__ __forceinline__ void shared_down_tile(const Params& p, SharedDownSmem<C>& sm, uint16_t* out, int h0, int hn,
                                                 SharedDownBatch<C, MF>& bt, bool first_ready) {
  const int lane = threadIdx.x & 63, g = lane / kDownLanes, l = lane % kDownLanes;
  const int R = p.rows;
  const int n_units = shared_down_units<C, MF>(R, hn);
  auto load = shared_down_loader<C, MF>(p, h0, hn);
  if (!first_ready || (int)(threadIdx.x >> 6) == 0) bt.load(shared_down_vwave(), n_units, load);
  __syncthreads();  // the previous user of the LDS is done
  if constexpr (GQ) {
    // the step's shared rows, quantized once (stage Q), copied in as they lie
    ws_to_lds(p, p.off[14], (uint32_t)R * C::SQS, sm.q);
    ws_to_lds(p, p.off[15], (uint32_t)R * C::SSC, (uint8_t*)sm.s);
    wait_vm0();
  } else {
    // (2 chunks a thread at once with MXFP4 routed experts: 4 spill the persistent launch there)
    quant_rows_lds<C::SFMT, C::S, C::SQS, C::FMT == kFp4 ? 2 : kQuantBatch>(
        p, [&](int i) { return p.off[8] + (uint32_t)i * C::S * 2; }, R, sm.q, sm.s);
  }
  __syncthreads();
  if constexpr (MF) {
    using DT = Batched<DownTile<C::SFMT, C::S>>;
    down_pipeline<DT>(bt, n_units, load, [&](int v, DT& dt) {
      const int n = lane & 15;
#pragma unroll 1
      for (int t0 = 0; t0 < R; t0 += kMfmaPicks) {  // the unit's rows stay in registers
        const int np = min(kMfmaPicks, R - t0);
        f32x4 acc[1];
        dt.opaque();
        dt.template mma<C::SQS, C::SSC>(sm.q, (const uint8_t*)sm.s, t0, np, lane, false, acc);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int hl = v * 16 + 4 * (lane >> 4) + k;
          if (n < np && hl < hn) out[(t0 + n) * hn + hl] = f2bf(acc[0][k]);
        }
      }
    });
  } else {
    static_assert(C::SFMT == kFp8, "the VALU GEMVs read FP8 128 x 128 shared rows");
    using DR = Batched<DownRows<kFp8, C::S>>;
    down_pipeline<DR>(bt, n_units, load, [&](int v, const DR& wr) {
      const int rb = v % kRowBlocks, pb = v / kRowBlocks;
      if (rb * kDownLanes >= hn) return;
      const int t0 = pb * kPickBlock, np = min(kPickBlock, R - t0);
      float acc[kPickBlock];
      wr.template dot<C::SQS, (C::S / 128) * 4>(sm.q + (size_t)t0 * C::SQS, (const uint8_t*)(sm.s + t0 * (C::S / 128)), np, l,
                                                acc);
      const int hl = rb * kDownLanes + g;
#pragma unroll
      for (int q = 0; q < kPickBlock; ++q) {
        const float y = tree_sum<kDownLanes>(acc[q]);
        if (q < np && l == 0 && hl < hn) out[(t0 + q) * hn + hl] = f2bf(y);
      }
    });
  }
}

// gate_up of the step's token groups, routed and shared (the shared expert's rows count as
// groups of their own after the routed ones): the (group, column) pairs dealt over the
// workgroups in equal shares of cost (a column costs kColCost + its picks); column j of group
// g belongs to the share holding its first cost unit
template <class C>
__device__ __forceinline__ void gate_up_valu(const Params& p, const Union<C>& un, XTile<C>& xt, int b, int nwg) {
  static_assert(C::S == C::I, "shared and routed columns deal alike");
  const int total = un.tg_cost[un.ntg] * C::I;
  const int lo = (int)((long long)total * b / nwg), hi = (int)((long long)total * (b + 1) / nwg);
  const auto rs = ws_rsrc(p);
  // the last group that starts at or before lo
  int gl = 0, gh = un.ntg - 1;
  while (gl < gh) {
    const int mid = (gl + gh + 1) >> 1;
    if (un.tg_cost[mid] * C::I <= lo) gl = mid; else gh = mid - 1;
  }
  for (int tgg = gl; tgg < un.ntg && un.tg_cost[tgg] * C::I < hi; ++tgg) {
    const int base = un.tg_cost[tgg] * C::I;
    const int cg = un.tg_cost[tgg + 1] - un.tg_cost[tgg];
    const int c0 = lo > base ? min((lo - base + cg - 1) / cg, C::I) : 0;
    const int c1 = hi > base ? min((hi - base + cg - 1) / cg, C::I) : 0;
    if (c1 <= c0) continue;
    if (tgg >= un.ntg_r) {
      // the shared expert (FP8) for rows t0 .. t0 + np - 1
      const int t0 = (tgg - un.ntg_r) * kTokGroup, np = min(kTokGroup, p.rows - t0);
      const uint32_t qoff = C::FMT == kFp4 ? p.off[3] : p.off[1];
      const uint32_t soff = C::FMT == kFp4 ? p.off[4] : p.off[2];
      gu_unit<C, kFp8>(
          p, xt, np, C::S, c0, c1 - c0,
          [&](const uint8_t*& w, const void*& s) {
            w = p.sgu;
            s = p.sgu_s;
          },
          [&](XRegs<C, kTokGroup>& xr) { xr.load(p, np, qoff, soff, [&](int r) { return t0 + r; }); },
          [&](int q, int col, float g, float u) {
            dst16(rs, p.off[8] + ((uint32_t)(t0 + q) * C::S + col) * 2, f2bf(swiglu_shared(g, u, p.limit)));
          });
      continue;
    }
    const int slot = un.tg_slot[tgg];
    const int e = un.slot_e[slot];
    const int j0 = un.slot_start[slot] + (tgg - un.tg_start[slot]) * kTokGroup;
    const int np = min(kTokGroup, un.slot_start[slot + 1] - j0);
    gu_unit<C, C::FMT>(
        p, xt, np, C::I, c0, c1 - c0,
        [&](const uint8_t*& w, const void*& s) {
          if constexpr (C::FMT == kFp8) {
            w = p.w13 + (size_t)e * 2 * C::I * C::H;
            s = (const float*)p.w13_s + (size_t)e * (2 * C::I / 128) * (C::H / 128);
          } else {
            w = p.w13 + (size_t)e * 2 * C::I * (C::H / 2);
            s = (const uint8_t*)p.w13_s + (size_t)e * 2 * C::I * (C::H / 32);
          }
        },
        [&](XRegs<C, kTokGroup>& xr) { xr.load(p, np, p.off[1], p.off[2], [&](int r) { return un.picks[j0 + r] / C::K; }); },
        [&](int q, int col, float g, float u) {
          const int pk = un.picks[j0 + q];
          dst16(rs, p.off[9] + ((uint32_t)pk * C::I + col) * 2, f2bf(swiglu_routed(g, u, p.limit)));
        });
  }
}

// The MFMA gate_up's deal: FP8 in half-units (a unit's first or last NC / 2 columns), so that
// shares differ by half a unit at most (with MXFP4 weights the extra bookkeeping crowds the
// registers of the gate_up loop: whole units)
template <class C>
struct GuDeal {
  static constexpr bool HALF = C::FMT == kFp8;
  static constexpr int HU = HALF ? 2 : 1;  // deal steps a unit
  // the shared expert's (16-row group, column block) units
  __device__ __forceinline__ static int shared_units(int rows) {
    return (rows + kMfmaPicks - 1) / kMfmaPicks * (C::S / GuTile<C, C::SFMT>::NC);
  }
};

// the shared expert's gate_up units [lo, hi) (deal steps) on MFMA; before_x runs once, after
// the first unit's weights are requested and before the activations are read
template <class C, class PreFn>
__device__ __forceinline__ void gate_up_shared(const Params& p, GuSmem<C>& sm, int lo, int hi, PreFn before_x) {
  const auto rs = ws_rsrc(p);
  const uint32_t qoff = C::FMT == kFp4 ? p.off[3] : p.off[1];
  const uint32_t soff = C::FMT == kFp4 ? p.off[4] : p.off[2];
  bool pre = false;
  gu_mfma<C, C::SFMT, GuDeal<C>::HALF, false>(
      sm, C::S, C::S, lo, hi, false,
      [&](int tg, const uint8_t*& w, const void*& s, int& np) {
        w = p.sgu;
        s = p.sgu_s;
        np = min(kMfmaPicks, p.rows - tg * kMfmaPicks);
      },
      [&](int tg, int np, GuX<C, C::SFMT>& x) {
        if (!pre) {
          before_x();
          pre = true;
        }
        x.load(p, np, qoff, soff, [&](int r) { return tg * kMfmaPicks + r; }, threadIdx.x & 63, (int)(threadIdx.x >> 6));
      },
      [&](int tg, int q, int col, float g, float u) {
        dst16(rs, p.off[8] + ((uint32_t)(tg * kMfmaPicks + q) * C::S + col) * 2, f2bf(swiglu_shared(g, u, p.limit)));
      });
  if (!pre) before_x();
}

#ifndef MKMOE_EARLY_SHARED
#define MKMOE_EARLY_SHARED 1
#endif
constexpr bool kEarlyShared = MKMOE_EARLY_SHARED != 0;
#ifndef MKMOE_PRE_SHARED
#define MKMOE_PRE_SHARED 1
#endif
// ... and then every workgroup's shared down before the C wait
constexpr bool kPreShared = MKMOE_PRE_SHARED != 0;
// The shared expert's gate_up units run while the step is routed, by workgroups [w0, w0 + n)
// that route nothing meanwhile, with the gate_up on MFMA: its weights stream during the
// routing, and the rest of the gate_up is dealt afterwards.
//   - up to local_route_max<C>() rows (every other workgroup routes the step itself): workgroups
//     [0, n), three quarters of the grid at most, take all k of its units between them (a
//     unit each where k <= n);
//   - above (workgroups [0, R) route a row each, then the B hand-off): workgroups [R, R + n)
//     take its first k = n units, one each; the others join the routed units' deal.
// n = 0: none (the shared units are dealt with the routed ones).
struct EarlyShared {
  int w0, n, k;
};
template <class C>
__device__ __forceinline__ EarlyShared early_shared(const Params& p, int nwg) {
  if (!kEarlyShared || !gate_on_mfma<C>(p.rows, p.mfma_gate)) return {0, 0, 0};
  const int n_sh = GuDeal<C>::shared_units(p.rows);
  if (p.rows <= local_route_max<C>()) return {0, min(n_sh, 3 * nwg / 4), n_sh};
  const int n = min(n_sh, nwg - p.rows);
  return {p.rows, n, n};
}

// the same on MFMA: the shared expert's (16-row group, column block) units, then the routed
// ones, dealt evenly as one list. es.n > 0: the list's first es.k shared units ran in the
// routing window (early_shared), and the rest is dealt over the other workgroups where their
// largest share stays the same, else over all
template <class C>
__device__ __forceinline__ void gate_up_mfma(const Params& p, const Union<C>& un, GuSmem<C>& sm, int b, int nwg,
                                             EarlyShared es = {0, 0, 0}) {
  const auto rs = ws_rsrc(p);
  const int n_sh = GuDeal<C>::shared_units(p.rows);
  const int n_rt = un.ntg_r * (C::IR / GuTile<C, C::FMT>::NC);
  constexpr bool HALF = GuDeal<C>::HALF;
  constexpr int HU = GuDeal<C>::HU;
  const int e0 = HU * es.k;                     // deal steps done in the window
  const int n = HU * (n_sh + n_rt) - e0;        // and the rest
  int lo, hi;
  if (es.n > 0) {
    const int m = (n + nwg - 1) / nwg;
    if (n <= m * (nwg - es.n)) {
      if (b >= es.w0 && b < es.w0 + es.n) lo = hi = 0;
      else even_share(n, b < es.w0 ? b : b - es.n, nwg - es.n, lo, hi);
    } else {
      even_share(n, b, nwg, lo, hi);
    }
  } else {
    even_share(n, b, nwg, lo, hi);
  }
  lo += e0;
  hi += e0;
  gate_up_shared<C>(p, sm, lo, min(hi, HU * n_sh), [] {});
  auto first = [&](int tg) {
    const int slot = un.tg_slot[tg];
    return un.slot_start[slot] + (tg - un.tg_start[slot]) * kMfmaPicks;
  };
  gu_mfma<C, C::FMT, HALF, C::SHUF>(
      sm, C::I, C::IR, max(lo, HU * n_sh) - HU * n_sh, hi - HU * n_sh, C::FMT == kFp4 && p.mx_scaled,
      [&](int tg, const uint8_t*& w, const void*& s, int& np) {
        const int slot = un.tg_slot[tg];
        const int e = un.slot_e[slot];
        np = min(kMfmaPicks, un.slot_start[slot + 1] - first(tg));
        if constexpr (C::FMT == kFp8) {
          w = p.w13 + (size_t)e * 2 * C::I * C::H;
          s = (const float*)p.w13_s + (size_t)e * (2 * C::I / 128) * (C::H / 128);
        } else {
          w = p.w13 + (size_t)e * 2 * C::I * (C::H / 2);
          s = (const uint8_t*)p.w13_s + (size_t)e * 2 * C::I * (C::H / 32);
        }
      },
      [&](int tg, int np, GuX<C, C::FMT>& x) {
        const int j0 = first(tg);
        x.load(p, np, p.off[1], p.off[2], [&](int r) { return un.picks[j0 + r] / C::K; }, threadIdx.x & 63,
               (int)(threadIdx.x >> 6));
      },
      [&](int tg, int q, int col, float g, float u) {
        const int pk = un.picks[first(tg) + q];
        dst16(rs, p.off[9] + ((uint32_t)pk * C::I + col) * 2, f2bf(swiglu_routed(g, u, p.limit)));
      });
}

// es: the shared expert's units that ran in the routing window (MFMA)
template <class C>
__device__ __forceinline__ void stage_c(const Params& p, const Union<C>& un, GuSmem<C>& sm, int b, int nwg,
                                        EarlyShared es = {0, 0, 0}) {
  if constexpr (C::SHUF) gate_up_mfma<C>(p, un, sm, b, nwg, es);  // (the VALU GEMVs read row-major rows)
  else if (gate_on_mfma<C>(p.rows, p.mfma_gate)) gate_up_mfma<C>(p, un, sm, b, nwg, es);
  else gate_up_valu<C>(p, un, sm.x, b, nwg);
}

// ---------------------------------------------------------------- stage D: shared and routed down + combine
template <class C>
struct DownSmem {
  uint16_t contrib[kRowsMax * C::K * C::TMAX];  // bf16 of a pick's down output x its weight
  union {
    struct {
      uint8_t q[C::PB * C::MQS];
      uint8_t s[C::PB * C::MSC * 4];
    };
    SharedDownSmem<C> sd;  // the shared down's quantized rows, done before the routed ones
  };
  uint16_t shv[kRowsMax * C::TMAX];  // the shared expert's bf16 results of the tile
  int claim;  // MFMA down: the pick batch's next unit to be claimed by a wave
  // MFMA down: a wave's slot of weight rows (one unit)
  uint8_t wslot[kWaves][DownTile<C::FMT, C::I, C::DNA>::SLOT] __attribute__((aligned(16)));
};

// the slots holding picks [pb0, pb0 + pbn) of the step: picks are stored slot by slot, so they
// are the slots of the batch's first and last picks (a scan of the slot starts, one dependent
// LDS read a slot, took about 2.5 us a call at 8 rows)
template <class C>
__device__ __forceinline__ void batch_slots(const Union<C>& un, int pb0, int pbn, int& s_lo, int& s_hi) {
  s_lo = __builtin_amdgcn_readfirstlane(un.slot_of[un.ids[un.picks[pb0]]]);
  s_hi = __builtin_amdgcn_readfirstlane(un.slot_of[un.ids[un.picks[pb0 + pbn - 1]]]);
}

// the routed down GEMVs of tile rows [h0, h0 + hn) for every pick, into sm.contrib
// (VALU, 8-row units of 8 lanes a row)
template <class C>
using DownRowsOf = DownRows<C::FMT, C::I>;
template <class C>
using DownTileOf = DownTile<C::FMT, C::I, C::DNA, C::SHUF, C::IR>;
// the down stage's batch of units: MFMA (MF) or VALU
// the MFMA down's unit in flight: its rows in the wave's LDS slot, its scales in nxt
template <class C>
struct LdsUnit {
  DownTileOf<C> nxt;
};
template <class C, bool MF>
using DownBatchOf = typename std::conditional<MF, LdsUnit<C>, DownBatch<DownRowsOf<C>>>::type;

// loaders of the units of tile rows [h0, h0 + hn) for slots from s_lo: VALU units (slot,
// 8-row block), MFMA units (slot, 16-row block)
template <class C>
__device__ __forceinline__ auto valu_down_loader(const Params& p, const Union<C>& un, int h0, int hn, int s_lo) {
  const int lane = threadIdx.x & 63, g = lane / kDownLanes, l = lane % kDownLanes;
  return [&p, &un, h0, hn, s_lo, g, l](int v, DownRowsOf<C>& wr) {
    const int slot = s_lo + v / kRowBlocks, rb = v % kRowBlocks;
    const int e = un.slot_e[slot];
    const int hl = rb * kDownLanes + g;
    const int h = h0 + hl;
    const size_t row = (size_t)e * C::H + h;
    if constexpr (C::FMT == kFp8)
      wr.load(p.w2 + row * C::I,
              (const float*)p.w2_s + (size_t)e * (C::H / 128) * (C::I / 128) + (size_t)(h / 128) * (C::I / 128), hl < hn,
              l);
    else
      wr.load(p.w2 + row * (C::I / 2), (const uint8_t*)p.w2_s + row * (C::I / 32), hl < hn, l);
  };
}
// request MFMA unit v (slot, 16-row block) of tile rows [h0, h0 + hn), slots from s_lo: its
// rows into the wave's LDS slot, its scales into nx
template <class C>
__device__ __forceinline__ void mfma_issue(const Params& p, const Union<C>& un, int h0, int hn, int s_lo, int v,
                                           uint8_t* slot, DownTileOf<C>& nx, int lane) {
  using DT = DownTileOf<C>;
  constexpr int UR = 16 * DT::NA;  // rows a unit
  const int nb = (hn + UR - 1) / UR;
  const int e = un.slot_e[s_lo + v / nb], rb = v % nb;
  const int hb = h0 + rb * UR, nv = min(UR, hn - rb * UR);
  static_assert((long long)C::E * C::H * DT::RB < (1ll << 31), "offsets within a 32-bit resource");
  const auto wr = weight_rsrc(p.w2, (uint32_t)(C::E * C::H * DT::RB));
  DT::issue(wr, (uint32_t)(e * C::H + hb) * DT::RB, nv, slot, lane);
  if constexpr (C::FMT == kFp8)
    nx.load_scales((const float*)p.w2_s + (size_t)e * (C::H / 128) * (C::I / 128), hb, nv, lane);
  else
    // (SGLang's layout: the flat [E H][SC] scale matrix's columns are padded to a multiple of 8)
    nx.template load_scales<true>((const uint8_t*)p.w2_s + (size_t)e * C::H * (C::SHUF ? DT::SC : C::I / 32), hb, nv,
                                  lane);
}

// picks [pb0, pb0 + pbn) of the union's order, quantized once (stage Q), into the LDS rows of
// the down stage as they lie (codes [pick][MQS], scales [pick][MSC words]); waited for here
// (a pick's scale bytes need not be a multiple of 16: I / 32 = 20 at I = 640; the copy then
// starts at the 16-byte boundary below the batch's first scale, and the batch's scales begin
// pick_batch_scales() bytes into sm.s)
template <class C>
__device__ __forceinline__ uint32_t pick_batch_scales(int pb0) {
  constexpr uint32_t SST = C::FMT == kFp4 ? C::I / 32 : (C::I / 128) * 4;
  return (uint32_t)pb0 * SST % 16;
}
template <class C>
__device__ __forceinline__ void copy_pick_batch(const Params& p, int pb0, int pbn, DownSmem<C>& sm) {
  constexpr uint32_t SST = C::FMT == kFp4 ? C::I / 32 : (C::I / 128) * 4;  // scale bytes of a pick
  static_assert(C::MQS % 16 == 0, "16-byte pieces");
  static_assert(SST % 16 == 0 || sizeof(sm.s) >= C::PB * SST + 16, "room for the aligned copy");
  ws_to_lds(p, p.off[12] + (uint32_t)pb0 * C::MQS, (uint32_t)pbn * C::MQS, sm.q);
  const uint32_t a = (uint32_t)pb0 * SST - pick_batch_scales<C>(pb0);
  ws_to_lds(p, p.off[13] + a, (uint32_t)(pb0 + pbn) * SST - a, (uint8_t*)sm.s);
  wait_vm0();
}

template <class C, bool GQ>
__device__ __forceinline__ void down_valu(const Params& p, const Union<C>& un, DownSmem<C>& sm, int h0, int hn,
                                          DownBatch<DownRowsOf<C>>& bt, bool first_ready) {
  const int lane = threadIdx.x & 63, l = lane % kDownLanes, g = lane / kDownLanes;
  const int npk = p.rows * C::K;
  using DR = DownRowsOf<C>;
  constexpr int SST = C::FMT == kFp4 ? C::I / 32 : (C::I / 128) * 4;  // scale bytes of a pick
  for (int pb0 = 0; pb0 < npk; pb0 += C::PB) {
    const int pbn = min(C::PB, npk - pb0);
    int s_lo, s_hi;
    batch_slots(un, pb0, pbn, s_lo, s_hi);
    const int n_units = (s_hi - s_lo + 1) * kRowBlocks;
    auto load = valu_down_loader<C>(p, un, h0, hn, s_lo);
    // the first batch's weights are requested before the picks' rows are copied in
    if (pb0 > 0 || !first_ready || threadIdx.x < 64) bt.load((int)(threadIdx.x >> 6), n_units, load);
    __syncthreads();  // the previous batch is done with the LDS rows
    if constexpr (GQ)
      copy_pick_batch<C>(p, pb0, pbn, sm);
    else
      quant_rows_lds<C::FMT, C::I, C::MQS, kQuantBatch, C::IR>(
          p, [&](int i) { return p.off[9] + (uint32_t)un.picks[pb0 + i] * C::I * 2; }, pbn, sm.q, sm.s);
    __syncthreads();
    down_pipeline<DR>(bt, n_units, load, [&](int v, const DR& wr) {
      const int slot = s_lo + v / kRowBlocks, rb = v % kRowBlocks;
      if (rb * kDownLanes >= hn) return;
      const int hl = rb * kDownLanes + g;
      const int j0 = max(un.slot_start[slot], pb0), j1 = min(un.slot_start[slot + 1], pb0 + pbn);
      for (int jj = j0; jj < j1; jj += kPickBlock) {
        const int np = min(kPickBlock, j1 - jj);
        const int lp = jj - pb0;
        float acc[kPickBlock];
        wr.template dot<C::MQS, SST>(sm.q + (size_t)lp * C::MQS, sm.s + (GQ ? pick_batch_scales<C>(pb0) : 0u) + lp * SST,
                                     np, l, acc);
#pragma unroll
        for (int q = 0; q < kPickBlock; ++q) {
          const float y = tree_sum<kDownLanes>(acc[q]);
          if (q < np && l == 0 && hl < hn) {
            const int pk = un.picks[jj + q];
            sm.contrib[pk * C::TMAX + hl] = f2bf(y * un.wts[pk]);
          }
        }
      }
    });
  }
}

// the same on MFMA: units (slot, 16-row block), each against its slot's picks 16 at a time. A
// wave keeps one unit in flight: once a unit's rows are read out of its LDS slot, the wave's
// next unit is requested into the slot, and the unit is computed while those rows stream in.
// Wave w's first unit of a pick batch is unit w (waves 1-7 request it before the hand-offs,
// wave 0, which polls them, only after); each next unit is claimed from an LDS counter, so a
// wave that started late takes fewer. A unit's results are the same whichever wave computes it.
template <class C, bool GQ>
__device__ __forceinline__ void down_mfma(const Params& p, const Union<C>& un, DownSmem<C>& sm, int h0, int hn,
                                          LdsUnit<C>& bt, int first_ready) {
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  const int npk = p.rows * C::K;
  using DT = DownTileOf<C>;
  constexpr int SST = C::FMT == kFp4 ? C::I / 32 : (C::I / 128) * 4;  // scale bytes of a pick
  constexpr int UR = 16 * DT::NA;  // rows a unit
  const int nb = (hn + UR - 1) / UR;
  uint8_t* slot = sm.wslot[wave];
  int s_lo, s_hi;
  batch_slots(un, 0, min(C::PB, npk), s_lo, s_hi);
  bool ahead = false;  // this wave's first unit of the batch was requested in the batch before
  for (int pb0 = 0; pb0 < npk; pb0 += C::PB) {
    const int pbn = min(C::PB, npk - pb0);
    const int n_units = (s_hi - s_lo + 1) * nb;
    // the next batch's slots: a wave's last unit of this batch requests its first unit there,
    // so that the batch change waits for no weight rows
    int nx_lo = 0, nx_hi = -1;
    if (pb0 + C::PB < npk) batch_slots(un, pb0 + C::PB, min(C::PB, npk - pb0 - C::PB), nx_lo, nx_hi);
    const int nx_units = (nx_hi - nx_lo + 1) * nb;
    if (!ahead && (pb0 > 0 || first_ready == 0 || (wave == 0 && first_ready < 2)) && wave < n_units)
      mfma_issue<C>(p, un, h0, hn, s_lo, wave, slot, bt.nxt, lane);
    ahead = false;
    const unsigned long long tb0 = tl_now();
    __syncthreads();  // the previous batch is done with the LDS rows (and its claims)
    const unsigned long long tq0 = tl_now();
    TL_ADD(kTlDBar, tq0 - tb0);
    if (threadIdx.x == 0) sm.claim = kWaves;  // units 0 .. 7 are the waves' first
    if constexpr (GQ)
      copy_pick_batch<C>(p, pb0, pbn, sm);
    else
      // the quantize requests 8 chunks a thread at once (4 where a unit's scales take more
      // registers: MXFP4, whose 8 spill there)
      quant_rows_lds<C::FMT, C::I, C::MQS, (C::FMT == kFp4 ? 1 : 2) * kQuantBatch, C::IR>(
          p, [&](int i) { return p.off[9] + (uint32_t)un.picks[pb0 + i] * C::I * 2; }, pbn, sm.q, sm.s);
    __syncthreads();
    TL_ADD(kTlDQuant, tl_now() - tq0);
    DT cur;
    for (int v = wave; v < n_units;) {
      const unsigned long long tw0 = tl_now();
      wait_vm0();  // the unit's rows are in the slot
      const unsigned long long tf0 = tl_now();
      TL_ADD(kTlDWait, tf0 - tw0);
      TL_ADD(kTlDUnits, 1ull);
      const int slot_i = s_lo + v / nb, rb = v % nb;
      cur.fetch(slot, lane);
      cur.take_scales(bt.nxt, h0 + rb * UR, lane);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // and read out of it
      const unsigned long long tf1 = tl_now();
      TL_ADD(kTlDFetch, tf1 - tf0);
      int nv = 0;
      if (lane == 0) nv = __hip_atomic_fetch_add(&sm.claim, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      nv = __builtin_amdgcn_readfirstlane(nv);
      if (nv < n_units) {
        mfma_issue<C>(p, un, h0, hn, s_lo, nv, slot, bt.nxt, lane);
      } else if (wave < nx_units) {
        mfma_issue<C>(p, un, h0, hn, nx_lo, wave, slot, bt.nxt, lane);
        ahead = true;
      }
      TL_ADD(kTlDIssue, tl_now() - tf1);
      const int j0 = max(un.slot_start[slot_i], pb0), j1 = min(un.slot_start[slot_i + 1], pb0 + pbn);
      const int n = lane & 15;
      const unsigned long long tm0 = tl_now();
      for (int jj = j0; jj < j1; jj += kMfmaPicks) {
        const int np = min(kMfmaPicks, j1 - jj);
        f32x4 acc[DT::NA];
        cur.template mma<C::MQS, SST>(sm.q, sm.s + (GQ ? pick_batch_scales<C>(pb0) : 0u), jj - pb0, np, lane,
                                      C::FMT == kFp4 && p.mx_scaled_down, acc);
        const int pk = n < np ? un.picks[jj + n] : 0;
#pragma unroll
        for (int q = 0; q < DT::NA; ++q)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int hl = rb * UR + q * 16 + 4 * (lane >> 4) + k;
            if (n < np && hl < hn) sm.contrib[pk * C::TMAX + hl] = f2bf(acc[q][k] * un.wts[pk]);
          }
      }
      TL_ADD(kTlDMma, tl_now() - tm0);
      if (pb0 == 0 && v == wave) TL(kTlDFirst);
      v = nv;
    }
    s_lo = nx_lo;
    s_hi = nx_hi;
  }
}

// request the first pick batch's first units of tile rows [h0, h0 + hn) (waves 1-7); the down
// stage goes on from them
template <class C, bool MF>
__device__ __forceinline__ void down_first(const Params& p, const Union<C>& un, DownSmem<C>& sm, int h0, int hn,
                                           DownBatchOf<C, MF>& bt, bool wave0 = false) {
  const int npk = p.rows * C::K;
  int s_lo, s_hi;
  batch_slots(un, 0, min(C::PB, npk), s_lo, s_hi);
  const int wave = (int)(threadIdx.x >> 6);
  // not wave 0, which polls the hand-off next: its flag reads would return only after
  // these weights (a wave's loads return in order); wave0: wave 0 alone, later
  if ((wave == 0) != wave0) return;
  if constexpr (MF) {
    constexpr int UR = 16 * DownTileOf<C>::NA;
    if (wave < (s_hi - s_lo + 1) * ((hn + UR - 1) / UR))
      mfma_issue<C>(p, un, h0, hn, s_lo, wave, sm.wslot[wave], bt.nxt, threadIdx.x & 63);
  } else {
    bt.load(wave, (s_hi - s_lo + 1) * kRowBlocks, valu_down_loader<C>(p, un, h0, hn, s_lo));
  }
}

// tile rows [h0, h0 + hn): the routed down GEMVs (MFMA or VALU, as MF), the shared expert's
// down (PRE: done before), then the combine; first_ready: the routed down's first units are
// already requested into bt (1: by waves 1-7, 2: by every wave)
template <class C, bool MF, bool GQ, bool PRE = false>
__device__ __forceinline__ void down_tile(const Params& p, const Union<C>& un, DownSmem<C>& sm, int h0, int hn,
                                          DownBatchOf<C, MF>& bt, int first_ready) {
  const int tid = threadIdx.x;
  const int R = p.rows;
  if constexpr (MF) down_mfma<C, GQ>(p, un, sm, h0, hn, bt, first_ready);
  else down_valu<C, GQ>(p, un, sm, h0, hn, bt, first_ready);
  TL(kTlDRouted);
  if constexpr (!PRE) {  // PRE: sm.shv holds the shared expert's results already
    SharedDownBatch<C, MF> bs;
    shared_down_tile<C, MF, GQ>(p, sm.sd, sm.shv, h0, hn, bs, false);
  }
  __syncthreads();
  TL(kTlDShared);
  // ---- combine: top-k order, bf16 at every add, then + the shared expert's bf16 result
  // (the thread index passes an empty asm, so that the loop's LDS addresses are formed here
  // rather than hoisted to the kernel's start and held, or spilled, across the stages)
  int c0 = tid;
  asm volatile("" : "+v"(c0));
  for (int idx = c0; idx < R * hn; idx += kThreads) {
    const int t = idx / hn, hl = idx % hn;
    float routed = 0.0f;
#pragma unroll
    for (int k = 0; k < C::K; ++k) {
      const int pk = t * C::K + k;
      routed = bf_round(routed + bf2f(sm.contrib[pk * C::TMAX + hl]));
    }
    p.out[(size_t)t * C::H + h0 + hl] = f2bf(routed + bf2f(sm.shv[idx]));
  }
  __syncthreads();
}

// this workgroup's tiles; first_ready: its first tile's first routed units are already
// requested; GQ: stage Q has quantized the step's intermediates
template <class C, bool MF, bool GQ, bool PRE = false>
__device__ __forceinline__ void stage_d(const Params& p, const Union<C>& un, DownSmem<C>& sm, int b, int nwg,
                                        DownBatchOf<C, MF>& bt, int first_ready) {
  const int tr = p.tile_rows;
  const int n_tiles = (C::H + tr - 1) / tr;
  if (b < n_tiles) down_tile<C, MF, GQ, PRE>(p, un, sm, b * tr, min(tr, C::H - b * tr), bt, first_ready);
  // further tiles (fewer workgroups than tiles) start from batches of their own, so that bt
  // is free once the first tile's routed down is done
  for (int tile = b + nwg; tile < n_tiles; tile += nwg) {
    DownBatchOf<C, MF> bl;
    down_tile<C, MF, GQ>(p, un, sm, tile * tr, min(tr, C::H - tile * tr), bl, 0);
  }
}

// stage Q: the step's intermediates quantized once, a wave a row (the arithmetic of the down
// stage's LDS rows): the routed picks in the union's order into regions 12 / 13 (the routed
// rule), the shared rows into 14 / 15 (group-128 FP8); the down stage copies a pick batch's
// rows into LDS as they lie, instead of every workgroup quantizing every row
template <class C>
__device__ __forceinline__ void stage_q(const Params& p, const Union<C>& un, int b, int nwg, bool shared = true) {
  constexpr uint32_t SST = C::FMT == kFp4 ? C::I / 32 : (C::I / 128) * 4;
  const int lane = threadIdx.x & 63;
  const int npk = p.rows * C::K;
  // shared: the shared expert's rows too (regions 14 / 15), after the picks
  const int n = npk + (shared ? p.rows : 0);
  for (int j = wave_slot(b, nwg); j < n; j += nwg * kWaves) {
    if (j < npk) {
      quant_row_ws<C::FMT, C::I, C::IR>(p, p.off[9] + (uint32_t)un.picks[j] * C::I * 2, p.off[12] + (uint32_t)j * C::MQS,
                                 p.off[13] + (uint32_t)j * SST, lane);
    } else {
      const int r = j - npk;
      quant_row_ws<C::SFMT, C::S>(p, p.off[8] + (uint32_t)r * C::S * 2, p.off[14] + (uint32_t)r * C::SQS,
                                  p.off[15] + (uint32_t)r * C::SSC, lane);
    }
  }
}

// launches of up to this many rows (and with stage Q) run the shared expert's down inside the
// Q hand-off; above, the shared rows' quantize and units outlast the hand-off and hold up the
// routed down. 16 where the routed down is FP8 or wide (at 24 rows cfg 2 +1.9 us, cfg 5 +2.1),
// 24 on the narrow MXFP4 and the MX shared shapes (cfg 3 -1.9, cfg 4 -1.3, V4.1 TP2 -1.1, TP4
// -0.3; at 48 rows +0.5 to +2.7: measured)
template <class C>
constexpr int shared_mid_rows() {
  return C::SFMT == kFp8Mx || (C::FMT == kFp4 && C::I <= 640) ? 24 : 16;
}

// the persistent launch past its C arrival: the down stage's first weights depend on the
// union alone, so they are requested before the wait for the other workgroups' gate_up. GQ
// (launches of C::QROWS rows or more): stage Q first. PRE: workgroups [0, nsw) ran the shared
// expert's gate_up in the routing window and set their flags at B, so the first tile's shared
// down runs before the wait (its rows quantized here). MID (with stage Q, up to
// shared_mid_rows<C>() rows): the first tile's shared down runs inside the Q hand-off, from units
// in registers, its rows quantized here. Each combination is a code path of its own, so that
// neither path's registers are allocated around the other's
template <class C, bool MF, bool GQ, bool PRE = false, bool MID = false>
__device__ __forceinline__ void wait_then_d(const Params& p, const Union<C>& un, DownSmem<C>& sm, int b, int nwg,
                                            int nsw = 0) {
  static_assert(!(MID && PRE), "one place for the shared down");
  static_assert(!MID || (MF && GQ), "the shared down inside the Q hand-off: MFMA down, stage Q");
  DownBatchOf<C, MF> bt;
  const int tr = p.tile_rows;
  const bool first = b * tr < C::H;
  // (tiles past the grid's first run the shared down after the routed one, from stage Q's rows)
  const bool more_tiles = (C::H + tr - 1) / tr > nwg;
  // from 8 rows the first units are requested across the wait only by the workgroups that
  // arrive among the first three quarters: a late one's requests would hold up its own sight
  // of the last flags (its CU's loads queue behind them), by up to 5 us at 8 rows, and the Q
  // hand-off with it. (Below 8 rows the wait is short and the look costs more than it saves.)
  const bool early = first && (p.rows < 8 || 4 * flags_set_count(p, kCtlC, nwg) < 3 * nwg);
  int ready = early ? 1 : 0;
  if (early) down_first<C, MF>(p, un, sm, b * tr, min(tr, C::H - b * tr), bt);
  if constexpr (PRE) {
    if (first) {
      await_all(p, kCtlB, nsw, kStageB);
      SharedDownBatch<C, MF> bs;
      shared_down_tile<C, MF, false>(p, sm.sd, sm.shv, b * tr, min(tr, C::H - b * tr), bs, false);
      // the shared down outlasts most of the gate_up's end spread: wave 0 requests its first
      // routed unit before its C poll too
      if constexpr (MF) {
        if (early) {
          down_first<C, MF>(p, un, sm, b * tr, min(tr, C::H - b * tr), bt, true);
          ready = 2;
        }
      }
    }
  }
  await_all(p, kCtlC, nwg, kStageC);
  TL(kTlCAwaited);
  reset_parts<C>(p, b, nwg);  // every workgroup is past its routing
  if constexpr (GQ) {
    stage_q<C>(p, un, b, nwg, !(PRE || MID) || more_tiles);
    TL(kTlQDone);
    arrive(p, kCtlQ);
  }
  if constexpr (MID) {
    // its rows need only the C hand-off (the shared intermediate); the routed first units stay
    // in flight in the waves' slots meanwhile
    if (first) {
      SharedDownBatch<C, MF> bs;
      shared_down_tile<C, MF, false>(p, sm.sd, sm.shv, b * tr, min(tr, C::H - b * tr), bs, false);
    }
  }
  if constexpr (GQ) {
    await_all(p, kCtlQ, nwg, kStageQ);
    TL(kTlQAwaited);
  }
  __syncthreads();  // the tile's readers are done before the down stage reuses its LDS
  stage_d<C, MF, GQ, PRE || MID>(p, un, sm, b, nwg, bt, ready);
}

// ---------------------------------------------------------------- kernels
// the LDS of the stages: the union lives from stage C to the end; the stage buffers share
template <class C>
union StageSmem {
  RouterSmem<C> a;
  RouteSmem<C> r;
  GuSmem<C> g;
  DownSmem<C> d;
};

template <class C>
__global__ __launch_bounds__(kThreads) void k_fused(Params p) {
  __shared__ Union<C> un;
  __shared__ StageSmem<C> sm;
  const int b = blockIdx.x, nwg = gridDim.x;
  TL_CLEAR();
  TL(kTlStart);
  // (up to kLocalNormMax rows stage A norms the rows itself: no stage N, no hand-off)
  if constexpr (C::NORM) {
    if (p.rows > kLocalNormMax) {
      stage_norm<C>(p, b, nwg);
      arrive(p, kCtlNorm);
      await_all(p, kCtlNorm, nwg, kStageNorm);
    }
  }
  stage_a<C>(p, sm.a, b, nwg, p.rows <= kLocalNormMax);
  TL(kTlADone);
  arrive(p, kCtlA);
  TL(kTlAArrived);
  const EarlyShared es = early_shared<C>(p, nwg);
  const int nsw = es.n;
  if (b >= es.w0 && b < es.w0 + es.n) {
    // the shared expert's gate_up while the others route: its weights are requested before
    // the A hand-off (the x codes) is awaited. Up to 8 rows: then its flag at B (the shared
    // intermediate stored), and the routing from the workgroup that publishes it; above: its
    // flag at B first (no row to route), and the routing hand-off after the units
    int lo, hi;
    even_share(GuDeal<C>::HU * es.k, b - es.w0, es.n, lo, hi);
    const bool local = p.rows <= local_route_max<C>();
    if (!local) arrive(p, kCtlB);
    gate_up_shared<C>(p, sm.g, lo, hi, [&] {
      await_all(p, kCtlA, nwg, kStageA);
      TL(kTlAAwaited);
    });
    if (local) {
      arrive(p, kCtlB);
      await_one(p, kCtlB, nwg - 1, kStageB);
    } else {
      await_all(p, kCtlB, nwg, kStageB);
    }
    TL(kTlRouted);
    build_union<C>(p, un, false);
    TL(kTlUnion);
  } else if (p.rows <= local_route_max<C>()) {
    // every workgroup routes the step itself, reading the router's part sums as they land:
    // no routing hand-off; the A hand-off (the x codes) is awaited before the gate_up. The
    // last workgroup publishes the routing (the workspace copies, then its flag at B) for
    // the workgroups that ran the shared gate_up meanwhile
    route_all<C>(p, sm.r, un.ids, un.wts, un.rows_of, b == nwg - 1);
    if (nsw > 0 && b == nwg - 1) arrive(p, kCtlB);
    TL(kTlRouted);
    build_union<C>(p, un, true);
    TL(kTlUnion);
    await_all(p, kCtlA, nwg, kStageA);
    TL(kTlAAwaited);
  } else {
    await_all(p, kCtlA, nwg, kStageA);
    TL(kTlAAwaited);
    stage_b<C>(p, sm.r, b, nwg);
    arrive(p, kCtlB);
    await_all(p, kCtlB, nwg, kStageB);
    TL(kTlRouted);
    build_union<C>(p, un, false);
    TL(kTlUnion);
  }
  stage_c<C>(p, un, sm.g, b, nwg, es);
  TL(kTlGateUp);
  arrive(p, kCtlC);
  TL(kTlCArrived);
  const bool gq = p.rows >= C::QROWS;
  if (C::SHUF || down_on_mfma<C>(p.rows, p.mfma_down)) {
    // the shared down before the C wait below stage Q's rows, inside the Q hand-off up to
    // shared_mid_rows<C>() rows, else after the routed down
    if (nsw > 0 && kPreShared && !gq) {
      // the shared down before the C wait (the shared intermediate was stored in the routing
      // window). (With stage Q, from 8 rows, it cost 1-4 us there against after the routed
      // down or inside the Q hand-off: measured)
      wait_then_d<C, true, false, true>(p, un, sm.d, b, nwg, nsw);
    } else if (gq && p.rows <= shared_mid_rows<C>()) {
      wait_then_d<C, true, true, false, true>(p, un, sm.d, b, nwg);
    } else if (gq) {
      wait_then_d<C, true, true>(p, un, sm.d, b, nwg);
    } else {
      wait_then_d<C, true, false>(p, un, sm.d, b, nwg);
    }
  } else if constexpr (!C::SHUF) {
    if (gq) wait_then_d<C, false, true>(p, un, sm.d, b, nwg);
    else wait_then_d<C, false, false>(p, un, sm.d, b, nwg);
  }
  TL(kTlEnd);
  TL_DUMP(p);
  leave(p);
}

template <class C>
__global__ __launch_bounds__(kThreads) void k_norm(Params p) {
  stage_norm<C>(p, blockIdx.x, gridDim.x);
}
template <class C>
__global__ __launch_bounds__(kThreads) void k_a(Params p) {
  __shared__ RouterSmem<C> sm;
  stage_a<C>(p, sm, blockIdx.x, gridDim.x, false);
}
template <class C>
__global__ __launch_bounds__(kThreads) void k_b(Params p) {
  __shared__ RouteSmem<C> sm;
  stage_b<C>(p, sm, blockIdx.x, gridDim.x);
}
template <class C>
__global__ __launch_bounds__(kThreads) void k_c(Params p) {
  __shared__ Union<C> un;
  __shared__ GuSmem<C> sm;
  reset_parts<C>(p, blockIdx.x, gridDim.x);  // the routing launch is done with them
  build_union<C>(p, un, false);
  stage_c<C>(p, un, sm, blockIdx.x, gridDim.x);
}
template <class C>
__global__ __launch_bounds__(kThreads) void k_q(Params p) {
  __shared__ Union<C> un;
  build_union<C>(p, un, false);
  if (p.rows >= C::QROWS) stage_q<C>(p, un, blockIdx.x, gridDim.x);
}
template <class C>
__global__ __launch_bounds__(kThreads) void k_d(Params p) {
  __shared__ Union<C> un;
  __shared__ DownSmem<C> sm;
  build_union<C>(p, un, false);
  const bool gq = p.rows >= C::QROWS;
  if (C::SHUF || down_on_mfma<C>(p.rows, p.mfma_down)) {
    DownBatchOf<C, true> bt;
    if (gq) stage_d<C, true, true>(p, un, sm, blockIdx.x, gridDim.x, bt, false);
    else stage_d<C, true, false>(p, un, sm, blockIdx.x, gridDim.x, bt, false);
  } else if constexpr (!C::SHUF) {
    DownBatchOf<C, false> bt;
    if (gq) stage_d<C, false, true>(p, un, sm, blockIdx.x, gridDim.x, bt, false);
    else stage_d<C, false, false>(p, un, sm, blockIdx.x, gridDim.x, bt, false);
  }
}


}  // namespace mkmoe

// ================================================================ host side
using namespace mkmoe;

namespace {

template <class C>
int launch(const Params& p, int nwg, hipStream_t st, bool staged) {
  dim3 grid(nwg), block(kThreads);
  if (!staged) {
    // the persistent grid must be resident: a workgroup a CU
    int per = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_fused<C>, kThreads, 0) != hipSuccess)
      return MKMOE_ERR_HIP;
    if (per < 1) return MKMOE_ERR_DEVICE;
    hipLaunchKernelGGL(k_fused<C>, grid, block, 0, st, p);
  } else {
    if constexpr (C::NORM) hipLaunchKernelGGL(k_norm<C>, grid, block, 0, st, p);
    hipLaunchKernelGGL(k_a<C>, grid, block, 0, st, p);
    hipLaunchKernelGGL(k_b<C>, grid, block, 0, st, p);
    hipLaunchKernelGGL(k_c<C>, grid, block, 0, st, p);
    hipLaunchKernelGGL(k_q<C>, grid, block, 0, st, p);
    hipLaunchKernelGGL(k_d<C>, grid, block, 0, st, p);
  }
  return hipGetLastError() == hipSuccess ? MKMOE_OK : MKMOE_ERR_LAUNCH;
}

}  // namespace

// A compiled shape's launcher. Built in parts (MKMOE_UNIT), each shape's kernels are a
// translation unit of their own (compiled in parallel) and the host code another.
#define MKMOE_LAUNCHER(N, C)                                                              \
  __attribute__((visibility("hidden"))) int mkmoe_launch_cfg##N(const Params& p, int nwg, \
                                                                 hipStream_t st, bool staged) { \
    return launch<C>(p, nwg, st, staged);                                                \
  }
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 0
MKMOE_LAUNCHER(0, CfgPlumbing)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 1
MKMOE_LAUNCHER(1, CfgTp4Fp8)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 2
MKMOE_LAUNCHER(2, CfgTp4Fp4)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 3
MKMOE_LAUNCHER(3, CfgTp2Fp4Norm)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 4
MKMOE_LAUNCHER(4, CfgTp4Fp4Aiter)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 5
MKMOE_LAUNCHER(5, CfgTp2Fp4NormAiter)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 6
MKMOE_LAUNCHER(6, CfgPlumbingSoftplus)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 7
MKMOE_LAUNCHER(7, CfgV41Tp4)
#endif
#if !defined(MKMOE_UNIT) || MKMOE_UNIT == 8
MKMOE_LAUNCHER(8, CfgV41Tp2)
#endif
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg0(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg1(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg2(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg3(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg4(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg5(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg6(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg7(const Params&, int, hipStream_t, bool);
__attribute__((visibility("hidden"))) int mkmoe_launch_cfg8(const Params&, int, hipStream_t, bool);

#if !defined(MKMOE_UNIT) || MKMOE_UNIT == MKMOE_UNIT_HOST
namespace {

// The workspace of mkmoe_forward_static (for callers that cannot allocate): one array per GPU,
// held until the process ends. In host code ``scratch`` names a host-side stand-in, not device
// memory: its device address comes from hipGetSymbolAddress (once per device, that device
// current) and only that address is used.
constexpr size_t kStaticWsBytes = MKMOE_STATIC_WS_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticWsBytes];

// before each mkmoe_forward_static launch: the hand-off and error words cleared, the polled
// router part sums of the call's rows unset (a fill kernel: no memset, so a capture may hold it)
__global__ void k_static_reset(uint8_t* ws, uint32_t ctl_bytes, uint32_t off10, uint32_t bytes10) {
  const uint32_t nctl = ctl_bytes / 16, n = nctl + bytes10 / 16;
  for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < n; k += gridDim.x * blockDim.x) {
    if (k < nctl)
      *(u32x4*)(ws + (size_t)k * 16) = u32x4{0u, 0u, 0u, 0u};
    else
      *(u32x4*)(ws + off10 + (size_t)(k - nctl) * 16) = u32x4{kPartUnset, kPartUnset, kPartUnset, kPartUnset};
  }
}

struct DevInfo {
  int cus = 0;
  bool ok = false;
};

std::mutex g_mu;
DevInfo g_dev[64];
void* g_scratch[64];  // scratch's device address per device

// scratch's device address on device dev (the current device)
int static_workspace(int dev, void** ws) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (dev < 0 || dev >= 64) return MKMOE_ERR_DEVICE;
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return MKMOE_ERR_HIP;
    g_scratch[dev] = ptr;
  }
  *ws = g_scratch[dev];
  return MKMOE_OK;
}
constexpr double kDeadlineDefault = 2.0;  // seconds
constexpr int kMfmaGateDefault = 1;       // gate_up and down on MFMA at every row count
constexpr int kMfmaDownDefault = 1;
constexpr int kMxScaledDefault = 1 << 30;  // the MXFP4 gate_up GEMMs convert to bf16 at every row count
// From 8 rows the MXFP4 down GEMM of the shapes with I <= 512 runs on the scaled fp4 x fp8 MFMA
// (no converts): 5-7 % faster there, and within the output bounds at every measured workload of
// those shapes (at most 8 of 344064 elements past 2e-2, Zipf routing at 48 rows). Its internal
// sum keeps fewer bits than fp32, and a K of 1024 adds twice the steps: the I = 1024 shapes land
// 37 elements past 2e-2 under Zipf routing at 48 rows, so they keep the converting path, as do
// launches below 8 rows (a TP2 row at 1 row lands 2 elements past 2e-2).
constexpr int kMxScaledDownDefault = 8;
constexpr int kMxScaledDownMaxInter = 512;

// the options of one call (NULL: the defaults; a field left 0 takes its default)
int options_of(const mkmoe_options* o, double& deadline_s, int& gate, int& down, int& scaled, int& scaled_down,
               int& fault_stage, int& fault_wg) {
  deadline_s = kDeadlineDefault;
  gate = kMfmaGateDefault;
  down = kMfmaDownDefault;
  scaled = kMxScaledDefault;
  scaled_down = 0;  // the shape's default (forward_impl)
  fault_stage = 0;
  fault_wg = 0;
  if (!o) return MKMOE_OK;
  // a stage the persistent launch waits at (kStageD has no wait), a workgroup of the grid
  const int fs = o->fault_stage;
  if (fs != 0 && fs != kStageNorm && fs != kStageA && fs != kStageB && fs != kStageC && fs != kStageQ)
    return MKMOE_ERR_ARG;
  if (o->fault_workgroup < 0 || o->fault_workgroup >= kFlagWgs) return MKMOE_ERR_ARG;
  fault_stage = fs;
  fault_wg = o->fault_workgroup;
  if (o->mxfp4_scaled_rows < 0 || o->mxfp4_scaled_down_rows < 0) return MKMOE_ERR_ARG;
  if (o->mxfp4_scaled_rows) scaled = o->mxfp4_scaled_rows;
  scaled_down = o->mxfp4_scaled_down_rows;  // 0: the shape's default (forward_impl)
  if (o->deadline_s != 0.0) {
    if (!(o->deadline_s > 0.0) || o->deadline_s > 3600.0) return MKMOE_ERR_ARG;
    deadline_s = o->deadline_s;
  }
  if (o->mfma_gate_rows < 0 || o->mfma_down_rows < 0) return MKMOE_ERR_ARG;
  if (o->mfma_gate_rows) gate = o->mfma_gate_rows;
  if (o->mfma_down_rows) down = o->mfma_down_rows;
  return MKMOE_OK;
}

int device_info(int dev, DevInfo* out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (dev < 0 || dev >= 64) return MKMOE_ERR_DEVICE;
  if (!g_dev[dev].ok) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MKMOE_ERR_HIP;
    g_dev[dev].cus = prop.multiProcessorCount;
    g_dev[dev].ok = true;
  }
  *out = g_dev[dev];
  return MKMOE_OK;
}

enum CfgId {
  kNone = -1, kIdPlumbing = 0, kIdTp4Fp8, kIdTp4Fp4, kIdTp2Fp4Norm, kIdTp4Fp4Aiter, kIdTp2Fp4NormAiter,
  kIdPlumbingSoftplus, kIdV41Tp4, kIdV41Tp2
};

template <class C>
bool shape_is(const mkmoe_shape* s) {
  return s->hidden == C::H && s->experts == C::E && s->topk == C::K && s->n_group == C::NG &&
         s->topk_group == C::TG && s->inter == C::I && s->shared_inter == C::S &&
         s->routed_fmt == (C::SHUF ? kFp4Aiter : C::FMT) && s->router_parts == C::P && (s->use_norm != 0) == C::NORM &&
         s->scoring == C::SCORE && (s->shared_fmt == 0 ? kFp8 : s->shared_fmt) == C::SFMT;
}

int cfg_id(const mkmoe_shape* s) {
  if (!s) return kNone;
  if (shape_is<CfgPlumbing>(s)) return kIdPlumbing;
  if (shape_is<CfgTp4Fp8>(s)) return kIdTp4Fp8;
  if (shape_is<CfgTp4Fp4>(s)) return kIdTp4Fp4;
  if (shape_is<CfgTp2Fp4Norm>(s)) return kIdTp2Fp4Norm;
  if (shape_is<CfgTp4Fp4Aiter>(s)) return kIdTp4Fp4Aiter;
  if (shape_is<CfgTp2Fp4NormAiter>(s)) return kIdTp2Fp4NormAiter;
  if (shape_is<CfgPlumbingSoftplus>(s)) return kIdPlumbingSoftplus;
  if (shape_is<CfgV41Tp4>(s)) return kIdV41Tp4;
  if (shape_is<CfgV41Tp2>(s)) return kIdV41Tp2;
  return kNone;
}

int check_shape(const mkmoe_shape* s) {
  if (!s) return MKMOE_ERR_NULL;
  if (cfg_id(s) == kNone) return MKMOE_ERR_SHAPE;
  if (s->max_rows < 1 || s->max_rows > kRowsMax) return MKMOE_ERR_ROWS;
  return MKMOE_OK;
}

Layout layout_of(const mkmoe_shape* s) {
  return make_layout(s->hidden, s->experts, s->topk, s->inter, s->shared_inter,
                     s->routed_fmt == kFp4Aiter ? kFp4 : s->routed_fmt,
                     s->router_parts, s->use_norm, s->max_rows, s->shared_fmt == kFp8Mx ? kFp8Mx : kFp8);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// static_ws: the workspace is this device's scratch (ws and ws_bytes are ignored)
int forward_impl(const mkmoe_shape* s, const mkmoe_weights* w, const void* x, int32_t rows,
                 void* out, int32_t* ids, float* wts, void* ws, size_t ws_bytes,
                 const mkmoe_options* opts, void* stream, bool staged, bool static_ws = false) {
  int rc = check_shape(s);
  if (rc) return rc;
  double dl;
  int mfma_gate, mfma_down, mx_scaled, mx_scaled_down, fault_stage, fault_wg;
  if ((rc = options_of(opts, dl, mfma_gate, mfma_down, mx_scaled, mx_scaled_down, fault_stage, fault_wg))) return rc;
  // the VALU GEMVs read row-major expert rows: SGLang's shuffled layout runs on MFMA alone
  if (s->routed_fmt == kFp4Aiter && (mfma_gate > 1 || mfma_down > 1)) return MKMOE_ERR_ARG;
  if (static_ws) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return MKMOE_ERR_HIP;
    if ((rc = static_workspace(cur, &ws))) return rc;
    ws_bytes = kStaticWsBytes;
  }
  if (!w || !x || !out || !ws) return MKMOE_ERR_NULL;
  if (!w->gate_w || !w->bias || !w->w13 || !w->w13_s || !w->w2 || !w->w2_s || !w->sgu ||
      !w->sgu_s || !w->sw2 || !w->sw2_s)
    return MKMOE_ERR_NULL;
  if (s->use_norm && !w->norm) return MKMOE_ERR_NULL;
  if (rows < 1 || rows > s->max_rows) return MKMOE_ERR_ROWS;
  const void* al[] = {x, out, ws, w->gate_w, w->w13, w->w2, w->sgu, w->sw2};
  for (const void* q : al)
    if (!aligned16(q)) return MKMOE_ERR_ALIGN;
  if (s->use_norm && !aligned16(w->norm)) return MKMOE_ERR_ALIGN;
  Layout L = layout_of(s);
  if (ws_bytes < L.total || L.total >= (1ull << 31)) return MKMOE_ERR_WORKSPACE;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MKMOE_ERR_HIP;
  DevInfo di;
  rc = device_info(dev, &di);
  if (rc) return rc;
  const int nwg = di.cus < kFlagWgs ? di.cus : kFlagWgs;  // the persistent grid: a workgroup a CU
  // a fault aimed past the grid would stall nothing (the launch's grid is smaller than 256 on a
  // device or partition with fewer CUs)
  if (fault_stage != 0 && fault_wg >= nwg) return MKMOE_ERR_ARG;

  Params p;
  p.x = (const uint16_t*)x;
  p.out = (uint16_t*)out;
  p.ids_out = ids;
  p.w_out = wts;
  p.gate_w = (const uint16_t*)w->gate_w;
  p.bias = (const float*)w->bias;
  p.norm_w = (const uint16_t*)w->norm;
  p.w13 = (const uint8_t*)w->w13;
  p.w13_s = w->w13_s;
  p.w2 = (const uint8_t*)w->w2;
  p.w2_s = w->w2_s;
  p.sgu = (const uint8_t*)w->sgu;
  p.sgu_s = (const float*)w->sgu_s;
  p.sw2 = (const uint8_t*)w->sw2;
  p.sw2_s = (const float*)w->sw2_s;
  p.ws = (uint8_t*)ws;
  p.ws_bytes = (uint32_t)L.total;
  p.rows = rows;
  p.rmax = s->max_rows;
  p.renorm = s->renorm;
  int tr = (s->hidden + nwg - 1) / nwg;
  tr = (tr + 3) / 4 * 4;
  if (tr > tile_max(s->hidden)) tr = tile_max(s->hidden);  // the shape's tile LDS (C::TMAX)
  p.tile_rows = tr;
  p.scale = s->routed_scale;
  p.limit = s->swiglu_limit;
  p.eps = s->norm_eps;
  p.deadline = (unsigned long long)(dl * 1e8);
  p.fault_stage = fault_stage;
  p.fault_wg = fault_wg;
  p.mfma_gate = mfma_gate;
  p.mfma_down = mfma_down;
  p.mx_scaled = rows >= mx_scaled && rows >= mfma_gate && rows >= mfma_down ? 1 : 0;
  if (mx_scaled_down == 0) mx_scaled_down = s->inter <= kMxScaledDownMaxInter ? kMxScaledDownDefault : 1 << 30;
  p.mx_scaled_down = (p.mx_scaled || rows >= mx_scaled_down) && rows >= mfma_down ? 1 : 0;
  for (int i = 0; i < kRegions; ++i) p.off[i] = (uint32_t)L.off[i];
  hipStream_t st = (hipStream_t)stream;
  if (static_ws) {
    const uint32_t bytes10 = (uint32_t)rows * s->router_parts * s->experts * 4;
    hipLaunchKernelGGL(k_static_reset, dim3(8), dim3(256), 0, st, (uint8_t*)ws, (uint32_t)kCtlBytes,
                       (uint32_t)L.off[10], bytes10);
    if (hipGetLastError() != hipSuccess) return MKMOE_ERR_LAUNCH;
  }
  switch (cfg_id(s)) {
    case kIdPlumbing: return mkmoe_launch_cfg0(p, nwg, st, staged);
    case kIdTp4Fp8: return mkmoe_launch_cfg1(p, nwg, st, staged);
    case kIdTp4Fp4: return mkmoe_launch_cfg2(p, nwg, st, staged);
    case kIdTp2Fp4Norm: return mkmoe_launch_cfg3(p, nwg, st, staged);
    case kIdTp4Fp4Aiter: return mkmoe_launch_cfg4(p, nwg, st, staged);
    case kIdTp2Fp4NormAiter: return mkmoe_launch_cfg5(p, nwg, st, staged);
    case kIdPlumbingSoftplus: return mkmoe_launch_cfg6(p, nwg, st, staged);
    case kIdV41Tp4: return mkmoe_launch_cfg7(p, nwg, st, staged);
    case kIdV41Tp2: return mkmoe_launch_cfg8(p, nwg, st, staged);
  }
  return MKMOE_ERR_SHAPE;
}

}  // namespace

extern "C" {

int mkmoe_abi_version(void) { return MKMOE_ABI_VERSION; }

int mkmoe_shape_supported(const mkmoe_shape* shape) { return check_shape(shape) == MKMOE_OK; }

int mkmoe_workspace_bytes(const mkmoe_shape* shape, size_t* bytes) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!bytes) return MKMOE_ERR_NULL;
  *bytes = layout_of(shape).total;
  return MKMOE_OK;
}

int mkmoe_workspace_region(const mkmoe_shape* shape, int32_t region, size_t* offset,
                           size_t* bytes) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!offset || !bytes) return MKMOE_ERR_NULL;
  if (region < 0 || region >= kRegions) return MKMOE_ERR_ARG;
  Layout L = layout_of(shape);
  *offset = L.off[region];
  *bytes = L.size[region];
  return MKMOE_OK;
}

int mkmoe_init_workspace(const mkmoe_shape* shape, void* ws, size_t ws_bytes, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!ws) return MKMOE_ERR_NULL;
  if (ws_bytes < layout_of(shape).total) return MKMOE_ERR_WORKSPACE;
  if (hipMemsetAsync(ws, 0, kCtlBytes, (hipStream_t)stream) != hipSuccess) return MKMOE_ERR_HIP;
  // the polled copy of the router's part sums starts unset (kPartUnset: every byte 0xFF)
  const Layout L = layout_of(shape);
  if (hipMemsetAsync((uint8_t*)ws + L.off[10], 0xFF, L.size[10], (hipStream_t)stream) != hipSuccess)
    return MKMOE_ERR_HIP;
  return MKMOE_OK;
}

int mkmoe_forward(const mkmoe_shape* shape, const mkmoe_weights* w, const void* x, int32_t rows,
                  void* out, int32_t* topk_ids, float* topk_w, void* ws, size_t ws_bytes,
                  const mkmoe_options* opts, void* stream) {
  return forward_impl(shape, w, x, rows, out, topk_ids, topk_w, ws, ws_bytes, opts, stream, false);
}

int mkmoe_forward_staged(const mkmoe_shape* shape, const mkmoe_weights* w, const void* x,
                         int32_t rows, void* out, int32_t* topk_ids, float* topk_w, void* ws,
                         size_t ws_bytes, const mkmoe_options* opts, void* stream) {
  return forward_impl(shape, w, x, rows, out, topk_ids, topk_w, ws, ws_bytes, opts, stream, true);
}

int mkmoe_forward_static(const mkmoe_shape* shape, const mkmoe_weights* w, const void* x,
                         int32_t rows, void* out, int32_t* topk_ids, float* topk_w,
                         const mkmoe_options* opts, void* stream) {
  return forward_impl(shape, w, x, rows, out, topk_ids, topk_w, nullptr, 0, opts, stream, false, true);
}

int mkmoe_read_errors(const void* ws, int32_t* words, int32_t n, void* stream) {
  if (!ws || !words) return MKMOE_ERR_NULL;
  if (n < 1 || n > MKMOE_ERRW_WORDS) return MKMOE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (hipMemcpyAsync(words, (const uint8_t*)ws + kCtlErr * 4, n * 4, hipMemcpyDeviceToHost, st) !=
      hipSuccess)
    return MKMOE_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) return MKMOE_ERR_HIP;
  return MKMOE_OK;
}

int mkmoe_clear_errors(const mkmoe_shape* shape, void* ws, size_t ws_bytes, void* stream) {
  return mkmoe_init_workspace(shape, ws, ws_bytes, stream);
}

const char* mkmoe_status_string(int status) {
  switch (status) {
    case MKMOE_OK: return "ok";
    case MKMOE_ERR_NULL: return "a required pointer is NULL";
    case MKMOE_ERR_SHAPE: return "no compiled specialisation has this MoE shape";
    case MKMOE_ERR_ROWS: return "rows out of range (1 .. max_rows, max_rows <= 48)";
    case MKMOE_ERR_ALIGN: return "a buffer is not 16-byte aligned";
    case MKMOE_ERR_WORKSPACE: return "workspace smaller than mkmoe_workspace_bytes";
    case MKMOE_ERR_LAUNCH: return "the HIP kernel launch failed";
    case MKMOE_ERR_DEVICE: return "the device cannot keep the persistent grid resident";
    case MKMOE_ERR_ARG: return "invalid argument";
    case MKMOE_ERR_HIP: return "a HIP runtime call failed";
  }
  return "unknown status";
}

}  // extern "C"

#endif  // host unit
