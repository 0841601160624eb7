/*
 * mkmoe: the decode-step MoE block of one TP rank on one MI355X (gfx950), as a
 * C ABI. One call runs the router GEMV, grouped top-k, the routed experts'
 * gate_up GEMM, SwiGLU, the down GEMM, the shared expert and the weighted
 * combine, and writes the bf16 partial output before the TP all-reduce.
 *
 * Plain C: device pointers, sizes and a HIP stream passed as void*. No C++ or
 * torch types cross the boundary; no call allocates device memory. The caller
 * owns every buffer, including the workspace (one per concurrent stream).
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   - mkmoe_forward replaces the MoE half of the FFN launch,
 *     DSV41MonoRunner.ffn -> self.ffn_kernel(M)(...ptrs...)
 *     (sgl_amd_mono/deepseek_v41/gfx950/runner.py:436-510), whose MoE
 *     arguments are the ARGS tuple of gfx950/stages/moe.py:119-132
 *     (x, gate_w, bias, w13, w13_s, w2, w2_s, sgu, sgu_s, sw2, sw2_s, out);
 *     the launch itself is build_mono_ffn (gfx950/layer.py:601-767).
 *   - mkmoe_workspace_bytes / mkmoe_init_workspace replace the runner's
 *     per-width scratch and epoch buffers (runner.py:339-350,
 *     gfx950/layer.py:113-141, moe.py:136-163 scratch_layout).
 *   - mkmoe_read_errors / mkmoe_clear_errors replace the guard's error words
 *     (sgl_amd_mono/common/guard.py:22-32,194-210).
 *   - mkmoe_status_string replaces the RuntimeError reasons of
 *     runner.py:79-119.
 */
#ifndef MKMOE_H
#define MKMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 6: the test hooks moved to include/mkmoe_testing.h (libmkmoe_testing.so) */
#define MKMOE_ABI_VERSION 6

/* weight formats */
#define MKMOE_FMT_FP8_B128 1 /* e4m3, fp32 scale per 128 x 128 block */
#define MKMOE_FMT_MXFP4 2    /* e2m1 (2 a byte, even K low nibble), E8M0 per 32 K */
/* MXFP4 in SGLang's loaded gfx950 layout, read in place: the tensors the reference's
 * FFNWeights hold (deepseek_v41/gfx950/runner.py:139-142: aiter's (16, 16) shuffle with the
 * gate/up interleave, scales in shuffle_scale order; made by check_ffn.py:169-173) */
#define MKMOE_FMT_MXFP4_AITER 3
/* e4m3 with an E8M0 scale per 32 x 32 block, fed by MXFP8 activations of the "vllm" rule: the
 * V4.1 shared expert (deepseek_v41/gfx950/runner.py:143-146, check_ffn.py:118-121,226-231) */
#define MKMOE_FMT_FP8_MX32 4

/* router scores (mkmoe_shape.scoring) */
#define MKMOE_SCORE_SIGMOID 0       /* DeepSeek-V3: sigmoid(logit) */
#define MKMOE_SCORE_SQRT_SOFTPLUS 1 /* V4.1: sqrt(softplus(logit)) (check_ffn.py:201-206,
                                     * deepseek_v41/gfx950/stages/moe.py:304-316) */

/* status codes (negative: an error; the call enqueued nothing) */
#define MKMOE_OK 0
#define MKMOE_ERR_NULL (-1)        /* a required pointer is NULL */
#define MKMOE_ERR_SHAPE (-2)       /* no compiled specialisation has this shape */
#define MKMOE_ERR_ROWS (-3)        /* rows < 1 or rows > max_rows */
#define MKMOE_ERR_ALIGN (-4)       /* a pointer is not 16-byte aligned */
#define MKMOE_ERR_WORKSPACE (-5)   /* workspace smaller than mkmoe_workspace_bytes */
#define MKMOE_ERR_LAUNCH (-6)      /* the HIP launch failed */
#define MKMOE_ERR_DEVICE (-7)      /* the device cannot hold the persistent grid */
#define MKMOE_ERR_ARG (-8)         /* another invalid argument */
#define MKMOE_ERR_HIP (-9)         /* a HIP runtime call failed */

/* error words kept in the workspace (mkmoe_read_errors) */
#define MKMOE_ERRW_CODE 0    /* 0, or the first device error's code */
#define MKMOE_ERRW_STAGE 1   /* the stage whose wait ran past its deadline (the first to record,
                              * or, with a fault injected, the stalled wait's: the waits it
                              * holds up downstream may reach their deadlines before it) */
#define MKMOE_ERRW_BLOCK 2   /* the workgroup that saw it */
#define MKMOE_ERRW_COUNT 3   /* how many waits ran past their deadline */
#define MKMOE_ERRW_FAULT 4   /* 1: a wait stalled by mkmoe_options.fault_stage ran to its deadline */
#define MKMOE_ERRW_WORDS 8
#define MKMOE_DEVERR_DEADLINE 1

/* One TP rank's MoE block. Routing is a grouped top-k on the scores `scoring`
 * names (sigmoid, DeepSeek-V3; sqrt(softplus), V4.1): choice = score + bias;
 * groups ranked by the sum of their top two choices; topk experts chosen from
 * the topk_group best groups (n_group 1: a global top-k); weights =
 * score * routed_scale / sum (renorm) or score * routed_scale. */
typedef struct mkmoe_shape {
  int32_t hidden;        /* H */
  int32_t experts;       /* E routed experts */
  int32_t topk;          /* picks a row */
  int32_t n_group;       /* expert groups (1: no groups) */
  int32_t topk_group;    /* groups kept */
  int32_t inter;         /* a routed expert's intermediate width on this rank */
  int32_t shared_inter;  /* the shared expert's (FP8, shared_fmt) */
  int32_t routed_fmt;    /* MKMOE_FMT_* */
  int32_t router_parts;  /* router K parts, summed in order */
  int32_t renorm;        /* 1: normalise the top-k scores */
  int32_t use_norm;      /* 1: RMSNorm x first (norm weight required) */
  int32_t max_rows;      /* rows a call takes at most (<= 48) */
  float routed_scale;
  float swiglu_limit;
  float norm_eps;
  int32_t scoring;       /* MKMOE_SCORE_* (0: sigmoid; the bytes ABI 2 left reserved) */
  int32_t shared_fmt;    /* the shared expert's weights: MKMOE_FMT_FP8_B128 (0 taken as it: x
                          * and its intermediate quantized per 128 with fp32 scales) or
                          * MKMOE_FMT_FP8_MX32 (MXFP8 "vllm" rule); ABI 5 */
} mkmoe_shape;

/* Device pointers, read in place. Layouts (E experts, H hidden, I inter,
 * S shared_inter; e4m3 and e2m1 as raw bytes):
 *   gate_w bf16 [E][H]; bias fp32 [E]; norm bf16 [H] (use_norm only)
 *   FP8_B128: w13 [E][2I][H], w13_s fp32 [E][2I/128][H/128],
 *             w2 [E][H][I],   w2_s fp32 [E][H/128][I/128]
 *   MXFP4:    w13 [E][2I][H/2], w13_s E8M0 [E][2I][H/32],
 *             w2 [E][H][I/2],   w2_s E8M0 [E][H][I/32]
 *   MXFP4_AITER: the same sizes, permuted. w13's rows in 16-row groups alternating gate
 *             and up (group 2b: gate rows 16b.., group 2b+1: up rows 16b..); w13 and w2 in
 *             the (16, 16) shuffle: a 16-row group's bytes per 128-K step (64 bytes a row)
 *             as 1 KB in which byte 16 (m + 16 j) starts row m's K [32 j, 32 j + 32); the
 *             scales (w13_s in the interleaved row order) as one [rows][cols] byte matrix
 *             per tensor, byte (r, c) at ((((r/32 cols/8 + c/8) 4 + c%4) 16 + r%16) 2 +
 *             (c/4)%2) 2 + (r/16)%2 (common/mx.py:40-44). The GEMMs run on MFMA at every
 *             row count (mfma_*_rows above 1 are refused)
 *   sgu e4m3 [2S][H] (gate rows, then up rows), sgu_s fp32 [2S/128][H/128],
 *   sw2 e4m3 [H][S], sw2_s fp32 [H/128][S/128]; with shared_fmt MKMOE_FMT_FP8_MX32 the
 *   scales are E8M0 bytes, sgu_s [2S/32][H/32], sw2_s [H/32][S/32] (the V4.1 FFNWeights,
 *   gfx950/runner.py:143-146). The MXFP4_AITER w2_s holds [E H][C] bytes with C = I/32 padded
 *   to a multiple of 8 (stages/dims.py:54-56), read as the shuffle_scale order of that matrix
 * w13 holds each expert's gate rows [0, I) then its up rows [I, 2I). */
typedef struct mkmoe_weights {
  const void* gate_w;
  const void* bias;
  const void* w13;
  const void* w13_s;
  const void* w2;
  const void* w2_s;
  const void* sgu;
  const void* sgu_s;
  const void* sw2;
  const void* sw2_s;
  const void* norm;
} mkmoe_weights;

int mkmoe_abi_version(void);

/* 1 when this shape has a compiled specialisation, else 0. */
int mkmoe_shape_supported(const mkmoe_shape* shape);

/* Bytes of workspace one stream needs for calls of up to shape->max_rows rows. */
int mkmoe_workspace_bytes(const mkmoe_shape* shape, size_t* bytes);

/* Zero the workspace's hand-off words (exit count, arrival flags) and error
 * words, and mark the polled router part sums (region 10) unset (enqueued on
 * stream; not for use inside graph capture). Required once before the first
 * forward. */
int mkmoe_init_workspace(const mkmoe_shape* shape, void* ws, size_t ws_bytes, void* stream);

/* Per-call options (NULL: the defaults). No counterpart in the reference, whose
 * deadline is a build-time constant of the guard (common/guard.py:69-89) and whose
 * kernels pick their GEMM instruction per width at build time (spec.py:959-967). A
 * field left 0 takes its default. */
typedef struct mkmoe_options {
  double deadline_s;      /* device wait deadline in seconds (default 2.0, at most 3600): a
                           * wait past it records the error words and gives up, so the
                           * launch always ends */
  int32_t mfma_gate_rows; /* launches with at least this many rows run the gate_up GEMMs
                           * (routed and shared) on MFMA (default 1: always); fewer rows run
                           * the fixed-order VALU GEMVs, bit-identical to the oracle */
  int32_t mfma_down_rows; /* the same for the down GEMMs (default 1) */
  int32_t mxfp4_scaled_rows; /* MXFP4 shapes: launches with at least this many rows (and on
                              * MFMA) run both expert GEMMs on the scaled fp4 x fp8 MFMA
                              * (v_mfma_scale_f32_16x16x128_f8f6f4), with no conversion of
                              * the codes; 0: the default (never) */
  int32_t mxfp4_scaled_down_rows; /* MXFP4 shapes: the down GEMM alone on the scaled MFMA from
                                   * this many rows (and on MFMA); 0: the default, 8 on the
                                   * shapes with inter <= 512 and never on wider ones (the
                                   * reference runs its MXFP4 GEMMs on that instruction,
                                   * common/mx.py:60-66) */
  /* Test fault injection, the reference's SGLANG_AMD_MONO_FAULT_INJECT (common/guard.py:69-89:
   * a wait that stalls and times out). fault_stage 0: none; else workgroup fault_workgroup's
   * wait at that stage (the MKMOE_ERRW_STAGE codes of the persistent launch's waits: 1 norm,
   * 2 router part sums and x codes, 3 route (up to 8 rows, 4 on the 384-expert shape at
   * inter 1152: the routing published to the workgroups that run the shared expert's gate_up
   * meanwhile, and their shared intermediate
   * awaited before the shared down), 4 gate_up, 6 quantize) ignores what it waits for and runs
   * to the deadline, then records the error words with MKMOE_ERRW_FAULT set and the launch
   * goes on, as after any deadline. A stage the launch does not wait at (6 below the shape's
   * stage-Q rows, 1 without the norm or up to 16 rows, where every workgroup norms the rows
   * itself, 3 where the gate_up runs on the VALU up to 8 rows) and
   * the staged launches (no waits) stall nothing. The faulted launch's output is not valid;
   * mkmoe_clear_errors restores the workspace. */
  int32_t fault_stage;
  int32_t fault_workgroup; /* 0 .. 255, and below the launch's grid (one workgroup a CU, at
                            * most 256): MKMOE_ERR_ARG otherwise */
} mkmoe_options;

/* One MoE block for rows bf16 rows x [rows][H] -> out bf16 [rows][H] (this
 * rank's partial, before the all-reduce). topk_ids int32 [rows][topk] and
 * topk_w fp32 [rows][topk] receive the routing when not NULL. Enqueues exactly
 * one kernel on stream: no allocation, no host synchronisation, safe to
 * capture in a graph (a launch clears its own hand-off flags). Calls that may
 * overlap need distinct workspaces. opts may be NULL. */
int mkmoe_forward(const mkmoe_shape* shape, const mkmoe_weights* w, const void* x, int32_t rows,
                  void* out, int32_t* topk_ids, float* topk_w, void* ws, size_t ws_bytes,
                  const mkmoe_options* opts, void* stream);

/* The same results in one launch per stage (norm, router + quantize, route,
 * gate_up (routed and shared), the intermediates quantized, down (shared and
 * routed) + combine); for diagnosis and per-stage profiles. Stage codes (error
 * word MKMOE_ERRW_STAGE): 1 norm, 2 router, 3 route, 4 gate_up, 5 down, 6 quantize. */
int mkmoe_forward_staged(const mkmoe_shape* shape, const mkmoe_weights* w, const void* x,
                         int32_t rows, void* out, int32_t* topk_ids, float* topk_w, void* ws,
                         size_t ws_bytes, const mkmoe_options* opts, void* stream);

/* The same launch with the workspace in a static device array, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference. It
 * allocates nothing: the array (MKMOE_STATIC_WS_BYTES, 4 MiB, enough for every
 * compiled shape at 48 rows; a larger layout returns MKMOE_ERR_WORKSPACE) lives
 * in each GPU the library runs on until the process ends. Each call enqueues a
 * small fill kernel that clears the array's hand-off and error words and marks
 * the call's polled router part sums unset, then the forward kernel: two
 * launches, both safe to capture. Every call on one GPU shares that GPU's
 * array, so calls that may overlap on one GPU (other streams, other threads)
 * race and must not be issued. Its device error words are not readable
 * through the C ABI; a caller that needs them uses mkmoe_forward. */
#define MKMOE_STATIC_WS_BYTES (4u << 20)
int mkmoe_forward_static(const mkmoe_shape* shape, const mkmoe_weights* w, const void* x,
                         int32_t rows, void* out, int32_t* topk_ids, float* topk_w,
                         const mkmoe_options* opts, void* stream);

/* Copy the MKMOE_ERRW_WORDS error words to host memory (synchronises stream).
 * After a device error (MKMOE_ERRW_CODE non-zero) the launch that recorded it
 * gave up waiting, so its output is not valid and its hand-off state (arrival
 * flags, the polled router part sums) may be left half set: call
 * mkmoe_clear_errors before the next forward on that workspace. */
int mkmoe_read_errors(const void* ws, int32_t* words, int32_t n, void* stream);

/* Reset a workspace after a device error: the error words, the hand-off words
 * and the polled router part sums, as mkmoe_init_workspace does (enqueued on
 * stream; not for use inside graph capture). */
int mkmoe_clear_errors(const mkmoe_shape* shape, void* ws, size_t ws_bytes, void* stream);

/* Byte offset and size of a workspace region, for tests that read
 * intermediate results: 0 x normed (by the norm stage, or up to 16 rows by the quantize
 * of stage A, which norms the rows as it reads them), 1 x codes (routed rule), 2 x scales,
 * 3 x codes (shared rule), 4 x scales (shared rule), 5 router part sums
 * fp32 [rows][parts][E], 6 ids int32 [rows][topk], 7 weights fp32
 * [rows][topk], 8 shared intermediate bf16 [rows][S], 9 routed intermediate
 * bf16 [rows * topk][I], 10 the router part sums as routing polls them (every
 * word 0xFFFFFFFF between launches), 11 the phase stamps of a diagnostic build
 * compiled with MKMOE_TIMELINE (u64 s_memrealtime ticks [workgroup][32]; other
 * builds leave it untouched), 12 / 13 the routed intermediates quantized once
 * (from 6 rows on the FP8 shapes and at I >= 1024, else from 8: codes [rows * topk][I + 16]
 * in the union's pick order, E8M0 [..][I / 32]
 * or fp32 [..][I / 128] scales), 14 / 15 the shared intermediate quantized (above 16 rows,
 * or 24 on the MXFP4 shapes with inter <= 640 and the MX shared expert: codes [rows][S + 16],
 * fp32 scales [rows][S / 128] or E8M0 [rows][S / 32]; below, every workgroup quantizes the
 * shared rows into LDS itself). */
int mkmoe_workspace_region(const mkmoe_shape* shape, int32_t region, size_t* offset,
                           size_t* bytes);

const char* mkmoe_status_string(int status);

#ifdef __cplusplus
}
#endif
#endif /* MKMOE_H */
