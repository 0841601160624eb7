/* The FFN seam before the MoE block, on one MI355X (gfx950): C ABI.
 *
 * DeepSeek-V4.1 keeps HC = 4 residual streams per token (mHC hyper-connections). Before
 * its MoE block, one decode step:
 *   - folds the attention's output into the streams (its post mix) while mixing them
 *     (its comb mix);
 *   - collapses the new streams into the layer input with the pre mix;
 *   - projects the new streams onto the 24 mixes of the next seam (pre 4 | post 4 |
 *     comb 16), with a Sinkhorn-normalised comb;
 *   - RMS-normalises the layer input, which is the MoE block's input.
 * This library runs that seam for one TP rank holding the all-reduced attention output,
 * as two launches on the caller's stream. It allocates nothing.
 *
 * Reference interface replaced: the seam half of DSV41MonoRunner.ffn
 * (sgl_amd_mono/deepseek_v41/gfx950/runner.py:436-500): part, residual, post_mix, res_mix
 * and pre_mix in; res_out, post_out, comb_out and pre_out out; FFNWeights.hc_ffn_fn,
 * hc_ffn_scale, hc_ffn_base and ffn_norm (runner.py:130-136). There the normed layer input
 * stays in the launch's scratch for its MoE (gfx950/layer.py:569-577); here it is an
 * output. The stages followed are gfx950/stages/seam.py:103-378.
 *
 * The attention's TP all-reduce that precedes the seam there (stage_reduce / stage_push,
 * seam.py:383-425) needs peers and is not part of this library: `a` is the reduced output.
 */
#ifndef MKMOE_SEAM_H
#define MKMOE_SEAM_H

#include <stddef.h>
#include <stdint.h>

#include "mkmoe.h" /* status codes */

#ifdef __cplusplus
extern "C" {
#endif

#define MKMOE_SEAM_HC 4          /* residual streams */
#define MKMOE_SEAM_MIX 24        /* projections: pre 4 | post 4 | comb 16 */
#define MKMOE_SEAM_HIDDEN 5120   /* the one compiled hidden width (V4.1's) */
#define MKMOE_SEAM_MAX_TOKENS 64 /* decode tokens a call takes at most */
/* mkmoe_seam_io.flags: mkmoe_seam_forward leaves the gate (post_out, comb_out, pre_out) to
 * a later mkmoe_seam_gate call, so that the next block's input (normed) is ready first */
#define MKMOE_SEAM_GATE_LATER 1

/* One call's tensors: device pointers, row-major, every bf16 and fp32 [.][hidden] array
 * 16-byte aligned, the small fp32 arrays 4-byte aligned. The mixes are those of
 * check_ffn.py:236-251: comb[t][h][o] is stream h's weight in new stream o. */
typedef struct mkmoe_seam_io {
  int32_t hidden;        /* MKMOE_SEAM_HIDDEN */
  int32_t tokens;        /* 1 .. MKMOE_SEAM_MAX_TOKENS */
  float norm_eps;        /* the RMSNorm's epsilon (the reference: 1e-20) */
  int32_t flags;         /* 0, or MKMOE_SEAM_GATE_LATER */
  const void* a;         /* [tokens][hidden] bf16: the all-reduced attention output ("part" at TP 1) */
  const void* res;       /* [tokens][4][hidden] bf16: the residual streams */
  const float* post;     /* [tokens][4]: the attention seam's post mix */
  const float* comb;     /* [tokens][4][4]: its comb (res) mix */
  const float* pre;      /* [tokens][4]: the pre mix of this layer input */
  const float* hc_fn;    /* [24][4 * hidden]: the mix projection (hc_ffn_fn) */
  const float* hc_scale; /* [3]: pre, post and comb scales (hc_ffn_scale) */
  const float* hc_base;  /* [24] (hc_ffn_base) */
  const void* norm_w;    /* [hidden] bf16 (ffn_norm) */
  void* res_out;         /* [tokens][4][hidden] bf16: the new residual streams */
  void* normed;          /* [tokens][hidden] bf16: the normed layer input (the MoE's x) */
  float* post_out;       /* [tokens][4]: the next seam's post mix (2 sigmoid) */
  float* comb_out;       /* [tokens][4][4]: its comb mix (Sinkhorn, 20 rounds) */
  float* pre_out;        /* [tokens][4]: its pre mix (sigmoid + 1e-6) */
} mkmoe_seam_io;

/* Workspace bytes a call of `tokens` tokens needs: the collapsed rows (bf16) and each
 * 32-column slice's mix partials. No state persists between calls. */
int mkmoe_seam_workspace_bytes(int32_t hidden, int32_t tokens, size_t* bytes);

/* Run the seam on `stream` (a hipStream_t; NULL: the default stream). Every argument is
 * checked on the host before anything is launched: MKMOE_ERR_NULL, MKMOE_ERR_SHAPE
 * (hidden), MKMOE_ERR_ROWS (tokens), MKMOE_ERR_ALIGN, MKMOE_ERR_WORKSPACE,
 * MKMOE_ERR_ARG (unknown flags, norm_eps not finite or negative), MKMOE_ERR_LAUNCH.
 * Graph-capture safe: two kernel launches, no allocation, no host synchronisation.
 * With MKMOE_SEAM_GATE_LATER the second launch is the norm alone. */
int mkmoe_seam_forward(const mkmoe_seam_io* io, void* ws, size_t ws_bytes, void* stream);

/* The gate of a mkmoe_seam_forward call made with MKMOE_SEAM_GATE_LATER: the same io and
 * workspace, whose mix partials must be untouched in between (stream order). One launch.
 * The reference runs its gates this late too, inside its MoE stage (gfx950/layer.py:579-586).
 * MKMOE_ERR_ARG without the flag; the other checks as mkmoe_seam_forward's. */
int mkmoe_seam_gate(const mkmoe_seam_io* io, void* ws, size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MKMOE_SEAM_H */
