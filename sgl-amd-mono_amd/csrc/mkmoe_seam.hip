// The FFN seam before the MoE block (DeepSeek-V4.1's mHC hyper-connections) on gfx950 (MI355X):
// HIP kernels and the C ABI of include/mkmoe_seam.h.
//
// Two launches on the caller's stream:
//   k_seam_slice  a 256-thread workgroup per 32-column slice of the hidden width (160 at
//                 H = 5120) and group of 8 tokens. For each token at its columns: the new
//                 residual streams R (bf16, to res_out), the collapse lin = sum_h pre[h] R[h]
//                 (bf16, to the workspace), and the slice's partials of the 24 mix projections
//                 and of the sum of squares of R (to the workspace). The slice's projection
//                 weights (12 KB) go into registers first, and a slice's token groups share
//                 an XCD, so its L2 serves them after the first read.
//   k_seam_gate   a workgroup per token. Wave 0: the partials summed in groups of 8 slices,
//                 then the gate: pre and post on 8 lanes, the comb's 4 x 4 Sinkhorn rounds
//                 on 16 lanes by DPP exchanges. Wave 1: the RMSNorm of lin, the MoE block's
//                 input.
// Every value is a fixed sequence of IEEE fp32 / fp64 operations with contraction off (the
// residual's last term and the gate's affine steps are explicit fmas), and the sigmoid and
// exp are the exact fp64 ones of mkmoe_numerics.h, so a CPU restatement gives the same bits.
//
// Reference: sgl_amd_mono/deepseek_v41/gfx950/stages/seam.py (slice_row :137-158,
// slice_input :103-118, stage_slice :182-215, slice_mix :218-248, stage_gate :261-322,
// stage_norm :326-378), run at the head of the FFN launch (gfx950/layer.py:569-577). The
// reference sums the mix projection on fp32 MFMA and uses the hardware exp2 / rcp / rsq;
// here the projection is a fixed-order VALU sum (12 K multiply-adds a token and slice) and
// the reciprocals and square roots are IEEE.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "../../include/mkmoe_seam.h"
#include "mkmoe_numerics.h"

namespace mkmoe_seam {

using mkmoe::bf2f;
using mkmoe::f2bf;

constexpr int kHC = MKMOE_SEAM_HC;
constexpr int kMix = MKMOE_SEAM_MIX;
constexpr int kPart = kMix + 1;  // a slice's partials: the 24 mixes, then the sum of squares
constexpr int kCols = 32;        // columns a slice
constexpr int kGroup = 8;        // slices a gate group sums
constexpr int kThreads = 256;
constexpr int kTokMax = MKMOE_SEAM_MAX_TOKENS;
constexpr int kRStride = 36;  // LDS floats of a (token, stream) row of R: 16-byte reads, and the
                              // 4 rows a wave reads at once start on distinct banks
constexpr int kTasks = kPart * kHC;  // (projection, stream) sums of a slice
constexpr float kMixEps = 1e-20f;
constexpr float kHcEps = 1e-6f;
constexpr float kPostMult = 2.0f;
constexpr int kSinkhorn = 20;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct SeamParams {
  const uint16_t* a;
  const uint16_t* res;
  const float* post;
  const float* comb;
  const float* pre;
  const float* fn;
  const float* scale;
  const float* base;
  const uint16_t* norm_w;
  uint16_t* res_out;
  uint16_t* normed;
  float* post_out;
  float* comb_out;
  float* pre_out;
  uint16_t* lin;  // workspace: [T][H] bf16
  float* part;    // workspace: [H / kCols][T][kPart] (a slice's workgroups write whole rows)
  int T;
  float norm_eps;
};

__device__ __forceinline__ float bf_lo(uint32_t w) { return mkmoe::u2f(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return mkmoe::u2f(w & 0xffff0000u); }

// ---------------------------------------------------------------- slice launch
// grid (slices, token groups of kTokGroup): the token groups of slice s are blocks s + NS g,
// all on XCD s % 8 (NS is a multiple of 8 and blocks go round-robin over the 8 XCDs), so
// the slice's projection weights come from HBM once into that XCD's L2
constexpr int kTokGroup = 8;

template <int H>
__global__ __launch_bounds__(kThreads) void k_seam_slice(SeamParams p) {
#pragma clang fp contract(off)
  constexpr int NS = H / kCols;
  static_assert(NS % 8 == 0, "a slice's token groups on one XCD");
  __shared__ __align__(16) float rl[kTokGroup * kHC * kRStride];
  __shared__ float qs[kTokGroup * kTasks];
  const int s = blockIdx.x, c0 = s * kCols, tid = threadIdx.x;
  const int t0 = blockIdx.y * kTokGroup;
  const int nt = min(kTokGroup, p.T - t0);

  // the (projection j, stream o) task of this thread (j = 24: the sum of squares), its 32
  // weights requested first, into registers
  const int k = tid % 128, half = tid / 128;
  const int j = k / kHC, o = k % kHC;
  f32x4 f[kCols / 4];
  if (k < kTasks && j < kMix) {
    const f32x4* src = (const f32x4*)(p.fn + (size_t)j * kHC * H + (size_t)o * H + c0);
#pragma unroll
    for (int q = 0; q < kCols / 4; ++q) f[q] = src[q];
  }

  // R, res_out and lin: a thread per (token, column pair)
  if (tid < nt * (kCols / 2)) {
    const int tl = tid / (kCols / 2), cp = tid % (kCols / 2), col = c0 + 2 * cp, t = t0 + tl;
    const uint32_t av = *(const uint32_t*)(p.a + (size_t)t * H + col);
    uint32_t rv[kHC];
#pragma unroll
    for (int h = 0; h < kHC; ++h) rv[h] = *(const uint32_t*)(p.res + ((size_t)t * kHC + h) * H + col);
    float cm[kHC][kHC], po[kHC], pr[kHC];
#pragma unroll
    for (int h = 0; h < kHC; ++h) {
      po[h] = p.post[t * kHC + h];
      pr[h] = p.pre[t * kHC + h];
#pragma unroll
      for (int oo = 0; oo < kHC; ++oo) cm[h][oo] = p.comb[(t * kHC + h) * kHC + oo];
    }
    uint32_t ro[kHC] = {0u, 0u, 0u, 0u}, lo = 0u;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const float x = d ? bf_hi(av) : bf_lo(av);
      float r[kHC];
#pragma unroll
      for (int h = 0; h < kHC; ++h) r[h] = d ? bf_hi(rv[h]) : bf_lo(rv[h]);
      float lin = 0.0f;
#pragma unroll
      for (int oo = 0; oo < kHC; ++oo) {
        float v = po[oo] * x + r[0] * cm[0][oo];
        v = v + cm[1][oo] * r[1];
        v = v + cm[2][oo] * r[2];
        v = __builtin_fmaf(cm[3][oo], r[3], v);
        const uint16_t b = f2bf(v);
        const float R = bf2f(b);
        ro[oo] |= (uint32_t)b << (16 * d);
        rl[(tl * kHC + oo) * kRStride + 2 * cp + d] = R;
        lin = lin + pr[oo] * R;
      }
      lo |= (uint32_t)f2bf(lin) << (16 * d);
    }
#pragma unroll
    for (int oo = 0; oo < kHC; ++oo) *(uint32_t*)(p.res_out + ((size_t)t * kHC + oo) * H + col) = ro[oo];
    *(uint32_t*)(p.lin + (size_t)t * H + col) = lo;
  }
  __syncthreads();

  // the task's sums over the slice's 32 columns, in column order from 0, for the group's
  // tokens (split over the two halves of the workgroup)
  if (k < kTasks) {
    for (int tl = half; tl < nt; tl += 2) {
      const f32x4* rr = (const f32x4*)(rl + (tl * kHC + o) * kRStride);
      float acc = 0.0f;
      if (j < kMix) {
#pragma unroll
        for (int q = 0; q < kCols / 4; ++q) {
          const f32x4 r4 = rr[q];
          acc = acc + f[q].x * r4.x;
          acc = acc + f[q].y * r4.y;
          acc = acc + f[q].z * r4.z;
          acc = acc + f[q].w * r4.w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < kCols / 4; ++q) {
          const f32x4 r4 = rr[q];
          acc = acc + r4.x * r4.x;
          acc = acc + r4.y * r4.y;
          acc = acc + r4.z * r4.z;
          acc = acc + r4.w * r4.w;
        }
      }
      qs[tl * kTasks + k] = acc;
    }
  }
  __syncthreads();
  // the slice's partial of (token, projection): the streams added in order; the group's
  // tokens are one contiguous run of the slice's row
  if (tid < nt * kPart) {
    const int tl = tid / kPart, jj = tid % kPart;
    const float* q = qs + tl * kTasks + jj * kHC;
    p.part[((size_t)s * p.T + t0) * kPart + tid] = ((q[0] + q[1]) + q[2]) + q[3];
  }
}

// ---------------------------------------------------------------- gate and norm launch
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
// lanes 4 r + c of each 16-lane row hold a 4 x 4 matrix (row r, column c). Row sums as
// (x0 + x1) + (x2 + x3) by quad permutes; column sums as (x_r0 + x_r1) + (x_r2 + x_r3) by row
// rotations (a lane receives lane (i - n) mod 16 under row_ror:n): the partner 4 lanes up for
// rows 0 and 2, 4 lanes down for rows 1 and 3, then the one 8 lanes away. Every lane of a row
// (column) ends with the same bits, since each add is of the same two values in either order.
__device__ __forceinline__ float quad_sum(float x) {
  const float a = x + dpp<0xB1>(x);  // quad_perm 1, 0, 3, 2
  return a + dpp<0x4E>(a);           // quad_perm 2, 3, 0, 1
}
__device__ __forceinline__ float col_sum(float x, bool even_row) {
  const float up = dpp<0x12C>(x), down = dpp<0x124>(x);  // row_ror:12 (lane + 4), row_ror:4 (lane - 4)
  const float a = x + (even_row ? up : down);
  return a + dpp<0x128>(a);  // row_ror:8
}
__device__ __forceinline__ float quad_max(float x) {
  const float a = fmaxf(x, dpp<0xB1>(x));
  return fmaxf(a, dpp<0x4E>(a));
}

// lane l < d receives lane l + d's value (other lanes: unspecified)
__device__ __forceinline__ float from_above(float v, int d) { return __shfl_down(v, d, 64); }

// GATE: the gate (wave 0, after all 4 waves' group sums); NORM: the norm (wave 1 with the
// gate, else a one-wave launch)
template <int H, bool GATE, bool NORM>
__global__ __launch_bounds__(kThreads) void k_seam_gate(SeamParams p) {
#pragma clang fp contract(off)
  constexpr int NS = H / kCols;
  constexpr int NG = NS / kGroup;
  constexpr int CH = H / 512;
  constexpr int kNormWave = GATE ? 1 : 0;
  __shared__ float pl[kPart * NS];  // this token's partials, [projection][slice]
  __shared__ float red[kPart * NG];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // the norm wave's inputs, requested first: lin rows (written by the slice launch) and weights
  u32x4 xv[CH], nw[CH];
  if (NORM && wave == kNormWave) {
    const uint16_t* x = p.lin + (size_t)t * H;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      xv[c] = *(const u32x4*)(x + c * 512 + lane * 8);
      nw[c] = *(const u32x4*)(p.norm_w + c * 512 + lane * 8);
    }
  }

  // this token's 25 partials of each slice into LDS, then the group sums: 8 slices in order
  // from the first
  if (GATE) {
    for (int sl = tid; sl < NS; sl += kThreads) {
      const float* q = p.part + ((size_t)sl * p.T + t) * kPart;
      float v[kPart];
#pragma unroll
      for (int jj = 0; jj < kPart; ++jj) v[jj] = q[jj];
#pragma unroll
      for (int jj = 0; jj < kPart; ++jj) pl[jj * NS + sl] = v[jj];
    }
    __syncthreads();
    for (int i = tid; i < kPart * NG; i += kThreads) {
      const int jj = i / NG, g = i % NG;
      const float* q = pl + jj * NS + g * kGroup;
      float acc = q[0];
#pragma unroll
      for (int kk = 1; kk < kGroup; ++kk) acc = acc + q[kk];
      red[jj * NG + g] = acc;
    }
    __syncthreads();
  }

  if (GATE && wave == 0) {
    // lane l < 16: comb element (l / 4, l % 4), projection 8 + l; lanes 16 .. 23: pre and post,
    // projections 0 .. 7; lane 24 and up: the sum of squares
    const int jj = lane < 16 ? 2 * kHC + lane : (lane < kMix ? lane - 16 : kMix);
    float mix = red[jj * NG];
#pragma unroll
    for (int g = 1; g < NG; ++g) mix = mix + red[jj * NG + g];
    const float sq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mix), kMix));
    const float dn = __builtin_fmaf(sq, 1.0f / (float)(kHC * H), kMixEps);
    const float rstd = 1.0f / sqrtf(dn);
    const float v = mix * rstd;
    const int which = jj < kHC ? 0 : (jj < 2 * kHC ? 1 : 2);
    const float z = __builtin_fmaf(v, p.scale[which], p.base[jj < kMix ? jj : kMix - 1]);
    if (lane >= 16 && lane < 16 + kHC) p.pre_out[t * kHC + jj] = mkmoe::sigmoid_exact(z) + kHcEps;
    if (lane >= 16 + kHC && lane < kMix) p.post_out[t * kHC + jj - kHC] = mkmoe::sigmoid_exact(z) * kPostMult;
    const bool even_row = ((lane >> 2) & 1) == 0;
    const float m = quad_max(z);
    const float e = (float)mkmoe::exp_nonpos((double)(z - m));
    float cv = __builtin_fmaf(e, 1.0f / quad_sum(e), kHcEps);
    cv = cv * (1.0f / (col_sum(cv, even_row) + kHcEps));
    for (int it = 1; it < kSinkhorn; ++it) {
      cv = cv * (1.0f / (quad_sum(cv) + kHcEps));
      cv = cv * (1.0f / (col_sum(cv, even_row) + kHcEps));
    }
    if (lane < 16) p.comb_out[t * kHC * kHC + lane] = cv;
  } else if (NORM && wave == kNormWave) {
    // RMSNorm of lin: lane l holds the 8 values from 512 c + 8 l of each chunk c; squares summed
    // in chunk then element order, the lanes by a halving tree
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t w4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float f = (q & 1) ? bf_hi(w4[q >> 1]) : bf_lo(w4[q >> 1]);
        acc = acc + f * f;
      }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) acc = acc + from_above(acc, d);
    const float ss = __shfl(acc, 0, 64);
    const float mean = ss / (float)H;
    const float rstd = 1.0f / sqrtf(mean + p.norm_eps);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t w4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
      const uint32_t n4[4] = {nw[c].x, nw[c].y, nw[c].z, nw[c].w};
      uint32_t ov[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float lo = bf_lo(w4[q]) * rstd, hi = bf_hi(w4[q]) * rstd;
        lo = lo * bf_lo(n4[q]);
        hi = hi * bf_hi(n4[q]);
        ov[q] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
      }
      *(u32x4*)(p.normed + (size_t)t * H + c * 512 + lane * 8) = u32x4{ov[0], ov[1], ov[2], ov[3]};
    }
  }
}

// ---------------------------------------------------------------- host
constexpr int kHidden = MKMOE_SEAM_HIDDEN;
static_assert(kHidden % 512 == 0 && (kHidden / kCols) % kGroup == 0, "slices, gate groups and norm chunks");

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
inline size_t lin_bytes(int tokens) { return align256((size_t)tokens * kHidden * 2); }
inline size_t part_bytes(int tokens) { return align256((size_t)tokens * kPart * (kHidden / kCols) * 4); }
inline bool aligned(const void* q, size_t a) { return ((uintptr_t)q % a) == 0; }

}  // namespace mkmoe_seam

extern "C" int mkmoe_seam_workspace_bytes(int32_t hidden, int32_t tokens, size_t* bytes) {
  using namespace mkmoe_seam;
  if (!bytes) return MKMOE_ERR_NULL;
  if (hidden != kHidden) return MKMOE_ERR_SHAPE;
  if (tokens < 1 || tokens > kTokMax) return MKMOE_ERR_ROWS;
  *bytes = lin_bytes(tokens) + part_bytes(tokens);
  return MKMOE_OK;
}

namespace mkmoe_seam {

// the checks every entry point makes, then the kernel parameters
inline int prepare(const mkmoe_seam_io* io, void* ws, size_t ws_bytes, SeamParams* p) {
  if (!io || !ws) return MKMOE_ERR_NULL;
  const void* need[] = {io->a,        io->res,     io->post,    io->comb,     io->pre,
                        io->hc_fn,    io->hc_scale, io->hc_base, io->norm_w,  io->res_out,
                        io->normed,   io->post_out, io->comb_out, io->pre_out};
  for (const void* q : need)
    if (!q) return MKMOE_ERR_NULL;
  if (io->hidden != kHidden) return MKMOE_ERR_SHAPE;
  if (io->tokens < 1 || io->tokens > kTokMax) return MKMOE_ERR_ROWS;
  if ((io->flags & ~MKMOE_SEAM_GATE_LATER) != 0 || !(io->norm_eps >= 0.0f) || !isfinite(io->norm_eps))
    return MKMOE_ERR_ARG;
  const void* wide[] = {io->a, io->res, io->hc_fn, io->norm_w, io->res_out, io->normed, ws};
  for (const void* q : wide)
    if (!aligned(q, 16)) return MKMOE_ERR_ALIGN;
  const void* narrow[] = {io->post, io->comb, io->pre, io->hc_scale, io->hc_base, io->post_out, io->comb_out, io->pre_out};
  for (const void* q : narrow)
    if (!aligned(q, 4)) return MKMOE_ERR_ALIGN;
  if (ws_bytes < lin_bytes(io->tokens) + part_bytes(io->tokens)) return MKMOE_ERR_WORKSPACE;
  p->a = (const uint16_t*)io->a;
  p->res = (const uint16_t*)io->res;
  p->post = io->post;
  p->comb = io->comb;
  p->pre = io->pre;
  p->fn = io->hc_fn;
  p->scale = io->hc_scale;
  p->base = io->hc_base;
  p->norm_w = (const uint16_t*)io->norm_w;
  p->res_out = (uint16_t*)io->res_out;
  p->normed = (uint16_t*)io->normed;
  p->post_out = io->post_out;
  p->comb_out = io->comb_out;
  p->pre_out = io->pre_out;
  p->lin = (uint16_t*)ws;
  p->part = (float*)((char*)ws + lin_bytes(io->tokens));
  p->T = io->tokens;
  p->norm_eps = io->norm_eps;
  return MKMOE_OK;
}

}  // namespace mkmoe_seam

extern "C" int mkmoe_seam_forward(const mkmoe_seam_io* io, void* ws, size_t ws_bytes, void* stream) {
  using namespace mkmoe_seam;
  SeamParams p;
  const int rc = prepare(io, ws, ws_bytes, &p);
  if (rc != MKMOE_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int groups = (io->tokens + kTokGroup - 1) / kTokGroup;
  hipLaunchKernelGGL(k_seam_slice<kHidden>, dim3(kHidden / kCols, groups), dim3(kThreads), 0, st, p);
  if (hipGetLastError() != hipSuccess) return MKMOE_ERR_LAUNCH;
  if (io->flags & MKMOE_SEAM_GATE_LATER)
    hipLaunchKernelGGL((k_seam_gate<kHidden, false, true>), dim3(io->tokens), dim3(64), 0, st, p);
  else
    hipLaunchKernelGGL((k_seam_gate<kHidden, true, true>), dim3(io->tokens), dim3(kThreads), 0, st, p);
  if (hipGetLastError() != hipSuccess) return MKMOE_ERR_LAUNCH;
  return MKMOE_OK;
}

extern "C" int mkmoe_seam_gate(const mkmoe_seam_io* io, void* ws, size_t ws_bytes, void* stream) {
  using namespace mkmoe_seam;
  SeamParams p;
  const int rc = prepare(io, ws, ws_bytes, &p);
  if (rc != MKMOE_OK) return rc;
  if (!(io->flags & MKMOE_SEAM_GATE_LATER)) return MKMOE_ERR_ARG;
  hipLaunchKernelGGL((k_seam_gate<kHidden, true, false>), dim3(io->tokens), dim3(kThreads), 0, (hipStream_t)stream, p);
  if (hipGetLastError() != hipSuccess) return MKMOE_ERR_LAUNCH;
  return MKMOE_OK;
}
