// Exact arithmetic of the decode MoE block, compiled for the host and for gfx950.
//
// Everything routing depends on is a fixed sequence of IEEE operations with
// floating-point contraction off, so the device result equals the host build's
// and the CPU oracle's bit for bit:
//   - bf16 <-> fp32 (round to nearest even)
//   - e4m3 encode (clamp to +-448, round to nearest even) in integer steps
//   - MX scale codes (the "aiter" rule, reference gfx950 common/mx.py:26-37 and
//     test/kernels/deepseek_v41/check_ffn.py:87-105)
//   - sigmoid in fp64 from add / multiply / divide / rint / ldexp only, rounded
//     once to fp32 (an exp by Cody-Waite reduction and a degree-13 Taylor
//     polynomial in Estrin's order; the input clamped to [-60, 60])
//   - V4.1's sqrt(softplus): softplus in fp64 from the same exp and an atanh-series
//     log1p, rounded to fp32, then the correctly rounded fp32 sqrt
#pragma once

#include <stdint.h>
#include <string.h>
#include <math.h>

#ifndef MKMOE_HD
#define MKMOE_HD __host__ __device__
#endif

namespace mkmoe {

constexpr float kFp8Max = 448.0f;
constexpr float kAmaxFloor = 1e-10f;
constexpr float kInv448 = (float)(1.0 / 448.0);
constexpr double kSigClamp = 60.0;

MKMOE_HD inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
MKMOE_HD inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
MKMOE_HD inline float bf2f(uint16_t b) { return u2f((uint32_t)b << 16); }
// fp32 -> bf16 bits, nearest even (inputs are finite)
MKMOE_HD inline uint16_t f2bf(float f) {
  uint32_t u = f2u(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
MKMOE_HD inline float bf_round(float f) { return bf2f(f2bf(f)); }

// fp32 -> e4m3 code (OCP fn), v finite: clamped to +-448, then nearest even.
MKMOE_HD inline uint32_t e4m3_encode(float v) {
  v = v > kFp8Max ? kFp8Max : (v < -kFp8Max ? -kFp8Max : v);
  uint32_t b = f2u(v);
  uint32_t s = (b >> 24) & 0x80u;
  uint32_t a = b & 0x7fffffffu;
  uint32_t code;
  if (a < 0x3c800000u) {  // |v| < 2^-6: subnormal e4m3, m * 2^-9, m = 0..8
    float t = u2f(a) * 512.0f;  // exact
    code = (uint32_t)rintf(t);
  } else {
    // keep 3 mantissa bits, nearest even, then rebias exponent 127 -> 7
    uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (r >> 20) - (120u << 3);
  }
  return s | code;
}

// biased exponent of the smallest power of two >= v (v > 0 finite)
MKMOE_HD inline int code_ceil(float v) {
  uint32_t b = f2u(v);
  return (int)((b >> 23) & 0xffu) + ((b & 0x7fffffu) != 0u ? 1 : 0);
}
// the MXFP8 "aiter" code of a group amax: [1, 254]
MKMOE_HD inline int mx_code(float amax) {
  float a = amax > kAmaxFloor ? amax : kAmaxFloor;
  int c = code_ceil(a * kInv448);
  return c < 1 ? 1 : (c > 254 ? 254 : c);
}
// the MXFP8 "vllm" code of a group amax (vLLM's mxfp8_e4m3_quantize, the V4.1 shared expert's
// activations and intermediate: stages/moe.py:234-245, check_ffn.py:99-101): the smallest power
// of two >= fp32(max(amax, FLT_MIN) / 448) (a correctly rounded division), clamped to [0, 254]
MKMOE_HD inline int vllm_code(float amax) {
#pragma clang fp contract(off)
  const float kFltMin = 1.17549435e-38f;
  float a = amax > kFltMin ? amax : kFltMin;
  int c = code_ceil(a / kFp8Max);
  return c < 0 ? 0 : (c > 254 ? 254 : c);
}
// 2^(127 - code), exact for code in [0, 253]; code 254 gives 2^-127 (subnormal)
MKMOE_HD inline float mx_inv(int code) {
  return code <= 253 ? u2f((uint32_t)(254 - code) << 23) : u2f(0x00200000u);
}
// per-token-group fp8 scale: max(amax, 1e-10) / 448
MKMOE_HD inline float group_scale(float amax) {
#pragma clang fp contract(off)
  float a = amax > kAmaxFloor ? amax : kAmaxFloor;
  return a / kFp8Max;
}

// exp(y) for y <= 0 (fp64, IEEE steps only): n = rint(y / ln 2), r = y - n ln 2 (two-part
// ln 2), the degree-13 Taylor polynomial of exp(r) in Estrin's order (pairs c_2k + c_2k+1 r,
// then r^2, r^4 and r^8 combine them: 8 dependent steps instead of Horner's 26), times 2^n.
// The N-wide forms below run N values step by step together (each value's operations are the
// scalar form's, in its order), so that their dependent chains overlap: a compiler left to
// itself ran a thread's chains one after another
template <int N>
MKMOE_HD inline void exp_nonpos_n(const double (&y)[N], double (&out)[N]) {
#pragma clang fp contract(off)
  const double kInvLn2 = 1.4426950408889634;
  const double kLn2Hi = 0x1.62e42fee00000p-1;
  const double kLn2Lo = 0x1.a39ef35793c76p-33;
  // (the pairs are formed where they are used, so that few values live at once)
  double n[N], r[N], r2[N], r4[N], s0[N], s1[N], s2[N], u0[N], u1[N];
#pragma unroll
  for (int i = 0; i < N; ++i) n[i] = rint(y[i] * kInvLn2);
#pragma unroll
  for (int i = 0; i < N; ++i) r[i] = (y[i] - n[i] * kLn2Hi) - n[i] * kLn2Lo;
#pragma unroll
  for (int i = 0; i < N; ++i) r2[i] = r[i] * r[i];
#pragma unroll
  for (int i = 0; i < N; ++i) r4[i] = r2[i] * r2[i];
#pragma unroll
  for (int i = 0; i < N; ++i) s0[i] = (1.0 + 1.0 * r[i]) + (1.0 / 2.0 + (1.0 / 6.0) * r[i]) * r2[i];
#pragma unroll
  for (int i = 0; i < N; ++i) s1[i] = (1.0 / 24.0 + (1.0 / 120.0) * r[i]) + (1.0 / 720.0 + (1.0 / 5040.0) * r[i]) * r2[i];
#pragma unroll
  for (int i = 0; i < N; ++i)
    s2[i] = (1.0 / 40320.0 + (1.0 / 362880.0) * r[i]) + (1.0 / 3628800.0 + (1.0 / 39916800.0) * r[i]) * r2[i];
#pragma unroll
  for (int i = 0; i < N; ++i) u0[i] = s0[i] + s1[i] * r4[i];
#pragma unroll
  for (int i = 0; i < N; ++i) u1[i] = s2[i] + (1.0 / 479001600.0 + (1.0 / 6227020800.0) * r[i]) * r4[i];
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = ldexp(u0[i] + u1[i] * (r4[i] * r4[i]), (int)n[i]);
}
MKMOE_HD inline double exp_nonpos(double y) {
  const double yv[1] = {y};
  double o[1];
  exp_nonpos_n<1>(yv, o);
  return o[0];
}

// the sigmoid in fp64, rounded to fp32 once: the input clamped to [-60, 60], t = exp(-|d|),
// then 1 / (1 + t) or t / (1 + t) by the sign (one division, the numerator selected first)
template <int N>
MKMOE_HD inline void sigmoid_exact_n(const float (&x)[N], float (&out)[N]) {
#pragma clang fp contract(off)
  double d[N], y[N], t[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    d[i] = (double)x[i];
    d[i] = d[i] > kSigClamp ? kSigClamp : (d[i] < -kSigClamp ? -kSigClamp : d[i]);
    y[i] = -fabs(d[i]);
  }
  exp_nonpos_n<N>(y, t);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = (float)((d[i] >= 0.0 ? 1.0 : t[i]) / (1.0 + t[i]));
}
MKMOE_HD inline float sigmoid_exact(float x) {
  const float xv[1] = {x};
  float o[1];
  sigmoid_exact_n<1>(xv, o);
  return o[0];
}

// log(1 + t) for t in [0, 1] (fp64, IEEE steps only): t past sqrt(2) - 1 reduced to
// s = (t - 1) / 2 (log(1 + t) = ln 2 + log(1 + s)), then 2 atanh(s / (2 + s)) by its series,
// terms z^(2k+1) / (2k+1) for k = 0 .. 11, in Horner's order
template <int N>
MKMOE_HD inline void log1p_01_n(const double (&t)[N], double (&out)[N]) {
#pragma clang fp contract(off)
  const double kSqrt2M1 = 0.41421356237309503;
  const double kLn2 = 0.6931471805599453;
  double z[N], z2[N], p[N];
  bool big[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    big[i] = t[i] > kSqrt2M1;
    const double s = big[i] ? (t[i] - 1.0) * 0.5 : t[i];
    z[i] = s / (2.0 + s);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    z2[i] = z[i] * z[i];
    p[i] = 1.0 / 23.0;
  }
  const double c[11] = {1.0 / 21.0, 1.0 / 19.0, 1.0 / 17.0, 1.0 / 15.0, 1.0 / 13.0, 1.0 / 11.0,
                        1.0 / 9.0,  1.0 / 7.0,  1.0 / 5.0,  1.0 / 3.0,  1.0};
#pragma unroll
  for (int k = 0; k < 11; ++k)
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = p[i] * z2[i] + c[k];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const double lg = 2.0 * (z[i] * p[i]);
    out[i] = big[i] ? kLn2 + lg : lg;
  }
}
MKMOE_HD inline double log1p_01(double t) {
  const double tv[1] = {t};
  double o[1];
  log1p_01_n<1>(tv, o);
  return o[0];
}

// V4.1's score sqrt(softplus(x)): softplus in fp64 (x itself past 20, else
// max(x, 0) + log1p(exp(-|x|)), the input floored at -200), rounded to fp32, then the
// correctly rounded fp32 square root; NaN stays NaN (the input itself)
template <int N>
MKMOE_HD inline void sqrt_softplus_exact_n(const float (&x)[N], float (&out)[N]) {
#pragma clang fp contract(off)
  double d[N], y[N], t[N], l[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    d[i] = (double)x[i];
    d[i] = d[i] < -200.0 ? -200.0 : d[i];
    // (past 20, and for NaN, the exp is taken of a value whose result is never used)
    y[i] = d[i] > 20.0 || d[i] != d[i] ? -20.0 : -fabs(d[i]);
  }
  exp_nonpos_n<N>(y, t);
  log1p_01_n<N>(t, l);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const double sp = d[i] > 20.0 ? d[i] : (d[i] > 0.0 ? d[i] : 0.0) + l[i];
    out[i] = x[i] != x[i] ? x[i] : sqrtf((float)sp);
  }
}
MKMOE_HD inline float sqrt_softplus_exact(float x) {
  const float xv[1] = {x};
  float o[1];
  sqrt_softplus_exact_n<1>(xv, o);
  return o[0];
}

// a > b in the selection order: larger value, or equal value and lower index
MKMOE_HD inline bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// Host restatement of the grouped top-k (the device runs it on one wave).
// choice = score + bias; group score = top-1 + top-2 choice of the group; the
// topk_group best groups (ties: lower group); topk experts of those groups by
// choice (ties: lower id), in selection order; weights score * f with
// f = scale / max(sum, 1e-20) summed in selection order (renorm) or f = scale.
inline void topk_host(int E, int K, int NG, int TG, int renorm, float scale, const float* score,
                      const float* bias, int32_t* ids, float* wts) {
#pragma clang fp contract(off)
  float choice[1024];
  bool keep[1024];
  int per = E / NG;
  for (int e = 0; e < E; ++e) {
    const float c = score[e] + bias[e];
    choice[e] = c != c ? -INFINITY : c;  // a NaN choice is -inf
    keep[e] = NG <= 1;
  }
  if (NG > 1) {
    float gs[64];
    bool gsel[64];
    for (int g = 0; g < NG; ++g) {
      int b1 = -1, b2 = -1;
      for (int e = g * per; e < (g + 1) * per; ++e) {
        if (b1 < 0 || better(choice[e], e, choice[b1], b1)) {
          b2 = b1;
          b1 = e;
        } else if (b2 < 0 || better(choice[e], e, choice[b2], b2)) {
          b2 = e;
        }
      }
      gs[g] = choice[b1] + choice[b2];
      gsel[g] = false;
    }
    for (int t = 0; t < TG; ++t) {
      int best = -1;
      for (int g = 0; g < NG; ++g)
        if (!gsel[g] && (best < 0 || better(gs[g], g, gs[best], best))) best = g;
      gsel[best] = true;
      for (int e = best * per; e < (best + 1) * per; ++e) keep[e] = true;
    }
  }
  float total = 0.0f;
  for (int k = 0; k < K; ++k) {
    int best = -1;
    for (int e = 0; e < E; ++e)
      if (keep[e] && (best < 0 || better(choice[e], e, choice[best], best))) best = e;
    keep[best] = false;
    ids[k] = best;
    const float sc = score[best] != score[best] ? 0.0f : score[best];  // a NaN score weighs 0
    wts[k] = sc;
    total = total + sc;
  }
  float f = scale;
  if (renorm) f = scale / (total > 1e-20f ? total : 1e-20f);
  for (int k = 0; k < K; ++k) wts[k] = wts[k] * f;
}

}  // namespace mkmoe
