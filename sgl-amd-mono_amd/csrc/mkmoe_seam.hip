// The FFN seam before the MoE block (DeepSeek-V4.1's mHC hyper-connections) on gfx950 (MI355X):
// HIP kernels and the C ABI of include/mkmoe_seam.h.
//
// Two launches on the caller's stream:
//   k_seam_slice  a 256-thread workgroup per 32-column slice of the hidden width (160 at
//                 H = 5120). For every token at its columns: the new residual streams R
//                 (bf16, to res_out), the collapse lin = sum_h pre[h] R[h] (bf16, to the
//                 workspace), and the slice's partials of the 24 mix projections and of the
//                 sum of squares of R (to the workspace). The slice's projection weights
//                 (12 KB) are read once, into registers, for all tokens.
//   k_seam_gate   a workgroup per token. Wave 0: the partials summed in groups of 8 slices,
//                 then the gate (pre, post and the Sinkhorn-normalised comb) on 24 lanes.
//                 Wave 1: the RMSNorm of lin, the MoE block's input.
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
  float* part;    // workspace: [T][kPart][H / kCols]
  int T;
  float norm_eps;
};

__device__ __forceinline__ float bf_lo(uint32_t w) { return mkmoe::u2f(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return mkmoe::u2f(w & 0xffff0000u); }

// ---------------------------------------------------------------- slice launch
template <int H>
__global__ __launch_bounds__(kThreads) void k_seam_slice(SeamParams p) {
#pragma clang fp contract(off)
  constexpr int NS = H / kCols;
  __shared__ __align__(16) float rl[kTokMax * kHC * kRStride];
  __shared__ float qs[kTokMax * kTasks];
  const int s = blockIdx.x, c0 = s * kCols, tid = threadIdx.x, T = p.T;

  // R, res_out and lin: a thread per (token, column pair)
  for (int i = tid; i < T * (kCols / 2); i += kThreads) {
    const int t = i / (kCols / 2), cp = i % (kCols / 2), col = c0 + 2 * cp;
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
      for (int o = 0; o < kHC; ++o) cm[h][o] = p.comb[(t * kHC + h) * kHC + o];
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
      for (int o = 0; o < kHC; ++o) {
        float v = po[o] * x + r[0] * cm[0][o];
        v = v + cm[1][o] * r[1];
        v = v + cm[2][o] * r[2];
        v = __builtin_fmaf(cm[3][o], r[3], v);
        const uint16_t b = f2bf(v);
        const float R = bf2f(b);
        ro[o] |= (uint32_t)b << (16 * d);
        rl[(t * kHC + o) * kRStride + 2 * cp + d] = R;
        lin = lin + pr[o] * R;
      }
      lo |= (uint32_t)f2bf(lin) << (16 * d);
    }
#pragma unroll
    for (int o = 0; o < kHC; ++o) *(uint32_t*)(p.res_out + ((size_t)t * kHC + o) * H + col) = ro[o];
    *(uint32_t*)(p.lin + (size_t)t * H + col) = lo;
  }

  // the (projection j, stream o) sums over the slice's 32 columns, in column order from 0:
  // task k = j * 4 + o (j = 24: the sum of squares), tokens split over the two halves of the
  // workgroup; the task's 32 weights stay in registers for every token
  const int k = tid % 128, half = tid / 128;
  const int j = k / kHC, o = k % kHC;
  f32x4 f[kCols / 4];
  if (k < kTasks && j < kMix) {
    const f32x4* src = (const f32x4*)(p.fn + (size_t)j * kHC * H + (size_t)o * H + c0);
#pragma unroll
    for (int q = 0; q < kCols / 4; ++q) f[q] = src[q];
  }
  __syncthreads();
  if (k < kTasks) {
    for (int t = half; t < T; t += 2) {
      const f32x4* rr = (const f32x4*)(rl + (t * kHC + o) * kRStride);
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
      qs[t * kTasks + k] = acc;
    }
  }
  __syncthreads();
  // the slice's partial of (token, projection): the streams added in order
  for (int i = tid; i < T * kPart; i += kThreads) {
    const int t = i / kPart, jj = i % kPart;
    const float* q = qs + t * kTasks + jj * kHC;
    p.part[((size_t)t * kPart + jj) * NS + s] = ((q[0] + q[1]) + q[2]) + q[3];
  }
}

// ---------------------------------------------------------------- gate and norm launch
// lane l < d receives lane l + d's value (other lanes: unspecified)
__device__ __forceinline__ float from_above(float v, int d) { return __shfl_down(v, d, 64); }

template <int H>
__global__ __launch_bounds__(kThreads) void k_seam_gate(SeamParams p) {
#pragma clang fp contract(off)
  constexpr int NS = H / kCols;
  constexpr int NG = NS / kGroup;
  constexpr int CH = H / 512;
  __shared__ float red[kPart * NG];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // group sums: 8 slices in order from the first
  for (int i = tid; i < kPart * NG; i += kThreads) {
    const int jj = i / NG, g = i % NG;
    const float* q = p.part + ((size_t)t * kPart + jj) * NS + g * kGroup;
    float acc = q[0];
#pragma unroll
    for (int kk = 1; kk < kGroup; ++kk) acc = acc + q[kk];
    red[jj * NG + g] = acc;
  }
  __syncthreads();

  if (wave == 0) {
    // projection j = lane (lane 24: the sum of squares): the groups in order from the first
    const int jj = lane < kPart ? lane : kPart - 1;
    float mix = red[jj * NG];
#pragma unroll
    for (int g = 1; g < NG; ++g) mix = mix + red[jj * NG + g];
    const float sq = __shfl(mix, kMix, 64);
    const float dn = __builtin_fmaf(sq, 1.0f / (float)(kHC * H), kMixEps);
    const float rstd = 1.0f / sqrtf(dn);
    const float v = mix * rstd;
    const int which = lane < kHC ? 0 : (lane < 2 * kHC ? 1 : 2);
    const float z = __builtin_fmaf(v, p.scale[which], p.base[lane < kMix ? lane : kMix - 1]);
    if (lane < kHC) p.pre_out[t * kHC + lane] = mkmoe::sigmoid_exact(z) + kHcEps;
    if (lane >= kHC && lane < 2 * kHC) p.post_out[t * kHC + lane - kHC] = mkmoe::sigmoid_exact(z) * kPostMult;
    // comb: lane 8 + 4 r + c holds element (r, c); other lanes shadow lanes 8 or 23
    const int cl = lane < 2 * kHC ? 2 * kHC : (lane >= kMix ? kMix - 1 : lane);
    const int rowl = 2 * kHC + ((cl - 2 * kHC) & ~3), coll = 2 * kHC + ((cl - 2 * kHC) & 3);
    auto rsum = [&](float x) {
      return (__shfl(x, rowl, 64) + __shfl(x, rowl + 1, 64)) + (__shfl(x, rowl + 2, 64) + __shfl(x, rowl + 3, 64));
    };
    auto csum = [&](float x) {
      return (__shfl(x, coll, 64) + __shfl(x, coll + 4, 64)) + (__shfl(x, coll + 8, 64) + __shfl(x, coll + 12, 64));
    };
    const float m = fmaxf(fmaxf(__shfl(z, rowl, 64), __shfl(z, rowl + 1, 64)),
                          fmaxf(__shfl(z, rowl + 2, 64), __shfl(z, rowl + 3, 64)));
    const float e = (float)mkmoe::exp_nonpos((double)(z - m));
    float cv = __builtin_fmaf(e, 1.0f / rsum(e), kHcEps);
    cv = cv * (1.0f / (csum(cv) + kHcEps));
    for (int it = 1; it < kSinkhorn; ++it) {
      cv = cv * (1.0f / (rsum(cv) + kHcEps));
      cv = cv * (1.0f / (csum(cv) + kHcEps));
    }
    if (lane >= 2 * kHC && lane < kMix) p.comb_out[t * kHC * kHC + lane - 2 * kHC] = cv;
  } else if (wave == 1) {
    // RMSNorm of lin: lane l holds the 8 values from 512 c + 8 l of each chunk c; squares summed
    // in chunk then element order, the lanes by a halving tree
    const uint16_t* x = p.lin + (size_t)t * H;
    u32x4 xv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) xv[c] = *(const u32x4*)(x + c * 512 + lane * 8);
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
      const u32x4 nw = *(const u32x4*)(p.norm_w + c * 512 + lane * 8);
      const uint32_t n4[4] = {nw.x, nw.y, nw.z, nw.w};
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

extern "C" int mkmoe_seam_forward(const mkmoe_seam_io* io, void* ws, size_t ws_bytes, void* stream) {
  using namespace mkmoe_seam;
  if (!io || !ws) return MKMOE_ERR_NULL;
  const void* need[] = {io->a,        io->res,     io->post,    io->comb,     io->pre,
                        io->hc_fn,    io->hc_scale, io->hc_base, io->norm_w,  io->res_out,
                        io->normed,   io->post_out, io->comb_out, io->pre_out};
  for (const void* q : need)
    if (!q) return MKMOE_ERR_NULL;
  if (io->hidden != kHidden) return MKMOE_ERR_SHAPE;
  if (io->tokens < 1 || io->tokens > kTokMax) return MKMOE_ERR_ROWS;
  if (io->reserved != 0 || !(io->norm_eps >= 0.0f) || !isfinite(io->norm_eps)) return MKMOE_ERR_ARG;
  const void* wide[] = {io->a, io->res, io->hc_fn, io->norm_w, io->res_out, io->normed, ws};
  for (const void* q : wide)
    if (!aligned(q, 16)) return MKMOE_ERR_ALIGN;
  const void* narrow[] = {io->post, io->comb, io->pre, io->hc_scale, io->hc_base, io->post_out, io->comb_out, io->pre_out};
  for (const void* q : narrow)
    if (!aligned(q, 4)) return MKMOE_ERR_ALIGN;
  if (ws_bytes < lin_bytes(io->tokens) + part_bytes(io->tokens)) return MKMOE_ERR_WORKSPACE;

  SeamParams p;
  p.a = (const uint16_t*)io->a;
  p.res = (const uint16_t*)io->res;
  p.post = io->post;
  p.comb = io->comb;
  p.pre = io->pre;
  p.fn = io->hc_fn;
  p.scale = io->hc_scale;
  p.base = io->hc_base;
  p.norm_w = (const uint16_t*)io->norm_w;
  p.res_out = (uint16_t*)io->res_out;
  p.normed = (uint16_t*)io->normed;
  p.post_out = io->post_out;
  p.comb_out = io->comb_out;
  p.pre_out = io->pre_out;
  p.lin = (uint16_t*)ws;
  p.part = (float*)((char*)ws + lin_bytes(io->tokens));
  p.T = io->tokens;
  p.norm_eps = io->norm_eps;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_seam_slice<kHidden>, dim3(kHidden / kCols), dim3(kThreads), 0, st, p);
  if (hipGetLastError() != hipSuccess) return MKMOE_ERR_LAUNCH;
  hipLaunchKernelGGL(k_seam_gate<kHidden>, dim3(io->tokens), dim3(kThreads), 0, st, p);
  if (hipGetLastError() != hipSuccess) return MKMOE_ERR_LAUNCH;
  return MKMOE_OK;
}
