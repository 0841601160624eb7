// Test hooks of the MoE library's arithmetic, kept out of its product ABI (include/mkmoe.h):
// the hardware converts and the scaled MFMA the kernels use, each run alone, and host builds of
// the kernels' exact arithmetic, for the tests that pin them (include/mkmoe_testing.h). Built as
// libmkmoe_testing.so beside libmkmoe.so by python sgl-amd-mono_amd/build.py. No counterpart in
// the reference: its quantizers are torch's conversions (check_ffn.py:104) and it calls the
// scaled MFMA through FlyDSL (common/mx.py:60-66).
#define MKMOE_UNIT 100  // the kernel source's definitions alone: no shape's kernels, no host code
#include "mkmoe_kernels.hip"

#include "../../include/mkmoe_testing.h"

namespace mkmoe {

// one v_mfma_scale_f32_16x16x128_f8f6f4 a tile (a wave a workgroup, C = 0): A and B eight
// words a lane (an e2m1 A uses the first four), the E8M0 codes one word a lane; D four
// floats a lane (C[m][n] in lane n + 16 (m / 4), element m % 4)
template <int FA>
__global__ void k_mfma_scaled(const uint32_t* a, const uint32_t* b, const uint32_t* sa, const uint32_t* sb, float* d,
                              int tiles) {
  const int t = blockIdx.x, l = threadIdx.x;
  if (t >= tiles || l >= 64) return;
  const size_t base = (size_t)t * 64 + l;
  i32x8 av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = (int)a[base * 8 + i];
    bv[i] = (int)b[base * 8 + i];
  }
  f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
  c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, FA, 0, 0, (int)sa[base], 0, (int)sb[base]);
#pragma unroll
  for (int v = 0; v < 4; ++v) d[base * 4 + v] = c[v];
}

// every finite fp32 bit pattern of [first, first + count) through the gfx950 e4m3 convert the
// activation quantizers use (e4m3_pack4: clamp to +-448, then the convert) against
// e4m3_encode (the integer-step encoder the CPU oracle restates): the count of differing codes
// and the lowest differing pattern
__global__ void k_e4m3_sweep(uint32_t first, uint32_t count, uint32_t* bad, uint32_t* first_bad) {
  uint32_t n_bad = 0, lo_bad = 0xffffffffu;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
    const uint32_t bits = first + i;
    if ((bits & 0x7f800000u) == 0x7f800000u) continue;  // inf, NaN
    const float x = u2f(bits);
    const uint32_t hw = e4m3_pack4(x, 0.0f, 0.0f, 0.0f) & 0xffu;
    if (hw != e4m3_encode(x)) {
      ++n_bad;
      lo_bad = bits < lo_bad ? bits : lo_bad;
    }
  }
  if (n_bad) {
    atomicAdd(bad, n_bad);
    atomicMin(first_bad, lo_bad);
  }
}

// decode byte i as e4m3 (the fp8 convert the GEMVs use) and as two e2m1 (the fp4 convert)
__global__ void k_decode(const uint8_t* codes, float* fp8, float* fp4, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const uint32_t b = codes[i];
    auto f = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
    fp8[i] = f[0];
    auto g = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(b, 1.0f, 0);
    fp4[2 * i] = g[0];
    fp4[2 * i + 1] = g[1];
  }
}

}  // namespace mkmoe

using namespace mkmoe;

extern "C" {

int mkmoe_device_mfma_scaled(const void* a, const void* b, const void* sa, const void* sb, float* d,
                             int32_t fmt_a, int32_t tiles, void* stream) {
  if (!a || !b || !sa || !sb || !d) return MKMOE_ERR_NULL;
  if (tiles < 1 || (fmt_a != 0 && fmt_a != 4)) return MKMOE_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const uint32_t *pa = (const uint32_t*)a, *pb = (const uint32_t*)b, *psa = (const uint32_t*)sa,
                 *psb = (const uint32_t*)sb;
  if (fmt_a == 4)
    hipLaunchKernelGGL(k_mfma_scaled<4>, dim3(tiles), dim3(64), 0, st, pa, pb, psa, psb, d, tiles);
  else
    hipLaunchKernelGGL(k_mfma_scaled<0>, dim3(tiles), dim3(64), 0, st, pa, pb, psa, psb, d, tiles);
  return hipGetLastError() == hipSuccess ? MKMOE_OK : MKMOE_ERR_LAUNCH;
}

int mkmoe_device_decode(const uint8_t* codes, float* fp8, float* fp4, int32_t n, void* stream) {
  if (!codes || !fp8 || !fp4) return MKMOE_ERR_NULL;
  if (n < 1) return MKMOE_ERR_ARG;
  hipLaunchKernelGGL(k_decode, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, codes, fp8,
                     fp4, n);
  return hipGetLastError() == hipSuccess ? MKMOE_OK : MKMOE_ERR_LAUNCH;
}

int mkmoe_device_e4m3_sweep(uint32_t first, uint32_t count, uint32_t* bad, uint32_t* first_bad, void* stream) {
  if (!bad || !first_bad) return MKMOE_ERR_NULL;
  if (count == 0 || (uint64_t)first + count > (1ull << 32)) return MKMOE_ERR_ARG;
  hipLaunchKernelGGL(k_e4m3_sweep, dim3(2048), dim3(256), 0, (hipStream_t)stream, first, count, bad, first_bad);
  return hipGetLastError() == hipSuccess ? MKMOE_OK : MKMOE_ERR_LAUNCH;
}

void mkmoe_host_e4m3_encode(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)e4m3_encode(x[i]);
}

void mkmoe_host_sigmoid(const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = sigmoid_exact(x[i]);
}

void mkmoe_host_sqrt_softplus(const float* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = sqrt_softplus_exact(x[i]);
}

void mkmoe_host_topk(const mkmoe_shape* s, const float* scores, const float* bias, int32_t* ids,
                     float* weights) {
  topk_host(s->experts, s->topk, s->n_group, s->topk_group, s->renorm, s->routed_scale, scores,
            bias, ids, weights);
}

}  // extern "C"
