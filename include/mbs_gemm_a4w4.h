/*
 * mbs_gemm_a4w4.h -- C ABI of the MI355X (gfx950) MXFP4 A4W4 GEMM library
 * (libmbs_gemm_kernel.so).  Plain pointers and sizes only; no torch, no HIP
 * types (streams are passed as void* holding a hipStream_t).
 *
 * Data contract (same bytes the reference kernel consumes, see
 * kernel/gemm_a4w4.h:5-26 of the reference):
 *   A        [M, K/2]   u8, two e2m1 codes per byte, low nibble = even k,
 *                       plain row-major.
 *   B        [N, K/2]   u8, e2m1 pairs, preshuffled with layout (16,16):
 *                       byte (n,kp) lives at
 *                       (n/16)*(K*8) + (kp/32)*512 + ((kp%32)/16)*256
 *                       + (n%16)*16 + kp%16.
 *   AScale   E8M0 u8, shuffled, >= round_up(M,32)*scaleN_pad bytes:
 *   BScale   E8M0 u8, shuffled, >= round_up(N,32)*scaleN_pad bytes;
 *                       byte (r,b) lives at
 *                       (r/32)*32*scaleN_pad + (b/8)*256 + (b%4)*64
 *                       + (r%16)*4 + ((b%8)/4)*2 + (r%32)/16.
 *   AFactor  [M] u8 or NULL, BFactor [N] u8 or NULL (both or neither):
 *                       out[m][n] *= f(AFactor[m]) * f(BFactor[n]),
 *                       f(b) = 1/(1+b/256).
 *   out      [Mpad, N]  bf16, Mpad = round_up(M,32); rows >= M untouched.
 *   scaleN_pad = round_up(ceil(K/32), 8).
 * Requirements: M >= 0, N % 16 == 0, K % 64 == 0 (the (16,16) preshuffle
 * needs K/2 % 32 == 0), all pointers device-accessible; A, B, the scales,
 * out, the workspace and a bias 16-byte aligned, the factors 4-byte aligned
 * (MBS_ERR_ARGUMENT otherwise).  Size limits (32-bit
 * buffer offsets): M*K/2 and N*K/2 below 2^31 bytes, 256*N*4 below 2^31; the
 * output itself may exceed 2^31 bytes (it is addressed per tile).  M == 0 (an empty
 * batch, e.g. an expert without tokens) validates the other arguments and
 * returns MBS_OK without launching; A, its scales and factors and out may
 * then be NULL.  The reference's launcher also reports success there
 * (kernel/gemm_a4w4.hip:1044-1146 launches a zero-size grid and does not
 * check the launch status).
 *
 * Every launch is asynchronous on `stream`; results are deterministic
 * (split-K partials are reduced in a fixed order, no atomics).
 */
#ifndef MBS_GEMM_A4W4_H_
#define MBS_GEMM_A4W4_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point. */
enum {
    MBS_OK = 0,
    MBS_ERR_ARGUMENT = 1,  /* null pointer, bad shape or padding argument   */
    MBS_ERR_WORKSPACE = 2, /* forced config needs more workspace than given */
    MBS_ERR_LAUNCH = 3,    /* the HIP launch itself failed                  */
    MBS_ERR_CONFIG = 4     /* forced config id out of range / unusable      */
};

/* Human-readable text for a status code (static storage). */
const char* mbs_status_string(int status);

/* Text of the last error raised on the calling thread ("" if none). */
const char* mbs_last_error(void);

/* MXFP4 A4W4 GEMM.  Replaces gemm_a4w4_mxfp4_launch
 * (reference kernel/gemm_a4w4.h:27-39, kernel/gemm_a4w4.hip:1044-1146) with
 * the same argument order, plus a caller-owned workspace for split-K partials
 * (`workspace` may be NULL when `workspace_bytes` is 0; size it with
 * mbs_gemm_a4w4_workspace_bytes).  Unlike the reference (which returns false
 * when factors meet its single-wave kernel) every shape accepts factors.
 * Returns MBS_OK or an error code; on error nothing is launched. */
int mbs_gemm_a4w4_launch(const uint8_t* A, const uint8_t* B, const uint8_t* AScale,
                         const uint8_t* BScale, const uint8_t* AFactor,
                         const uint8_t* BFactor, void* out, int M, int N, int K, int Mpad,
                         int scaleN_pad, void* workspace, size_t workspace_bytes,
                         void* stream);

/* mbs_gemm_a4w4_launch (config < 0) or mbs_gemm_a4w4_launch_config with an
 * affine epilogue:  out[m][n] = bf16( C[m][n] * (alpha * f(AFactor[m]) *
 * f(BFactor[n])) + bias[n] )  in fp32, bias bf16 [N] or NULL.  alpha = 1 with
 * no bias gives exactly mbs_gemm_a4w4_launch's bytes.  The bias follows
 * the aiter GEMM the reference's harness calls next to its own kernel
 * (test_gemm_a4w4.py:95-123, which passes a bias argument); the reference's
 * own launcher has neither alpha nor bias. */
int mbs_gemm_a4w4_launch_ex(int config, int splits, const uint8_t* A, const uint8_t* B,
                            const uint8_t* AScale, const uint8_t* BScale, const uint8_t* AFactor,
                            const uint8_t* BFactor, void* out, int M, int N, int K, int Mpad,
                            int scaleN_pad, float alpha, const void* bias, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Bytes of device scratch the allocation-free entry point owns per GPU. */
#define MBS_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* mbs_gemm_a4w4_launch_ex without a workspace argument, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * calls no hipMalloc/hipFree: split-K partials go to a static device array of
 * MBS_NOALLOC_SCRATCH_BYTES per GPU (looked up with hipGetSymbolAddress on the
 * first call on each device that needs it, with that device current; the
 * stream must belong to the current device).  config < 0: the heuristic plan,
 * limited to plans whose partials fit the scratch; config >= 0 with splits <= 0:
 * that config's split choice, or no split when it does not fit; an explicit
 * split count whose partials exceed the scratch returns MBS_ERR_WORKSPACE.
 * Nothing in the scratch needs to start at zero (every split writes its whole
 * partial plane before the reduce reads it).  All calls on one GPU share its
 * scratch: calls whose launches overlap on that GPU (different streams, no
 * ordering between them) race and must not be made. */
int mbs_gemm_a4w4_launch_noalloc(int config, int splits, const uint8_t* A, const uint8_t* B,
                                 const uint8_t* AScale, const uint8_t* BScale,
                                 const uint8_t* AFactor, const uint8_t* BFactor, void* out, int M,
                                 int N, int K, int Mpad, int scaleN_pad, float alpha,
                                 const void* bias, void* stream);

/* Grouped (mixture-of-experts) GEMM: E = num_groups experts share one launch.
 * Expert e owns rows [group_offsets[e], group_offsets[e+1]) of A (and of out)
 * and the e-th block of the stacked weights:
 *   B       [E][N, K/2]  each block (16,16)-preshuffled as above,
 *   BScale  [E][round_up(N,32) * scaleN_pad]  each block shuffled as above,
 *   BFactor [E][N] (or NULL with AFactor NULL);
 * A, AScale and AFactor cover all M rows as in mbs_gemm_a4w4_launch.
 * group_offsets: device int32 [E+1], group_offsets[0] = 0, non-decreasing,
 * every entry a multiple of 32 (pad each expert's token block, as MoE
 * routing usually does), group_offsets[E] <= M; it is read by the kernel,
 * not checked on the host.  Offsets outside [0, M] are clamped into it on
 * the device, so no store leaves the output; an expert whose first row is
 * not a multiple of 32 is skipped (its rows are not written: the shuffled A
 * scales come in 32-row groups).  mbs_gemm_a4w4_check_groups reports both
 * cases.  Rows past group_offsets[E] are not written.
 * config: -1 for the heuristic, else 0 <= config <
 * mbs_gemm_a4w4_grouped_num_configs(); the configurations named *_m32
 * (32x32x64-MFMA tiles) need K % 512 == 0 and return MBS_ERR_CONFIG
 * otherwise, before any launch.  Each expert's rows give the same
 * bytes as mbs_gemm_a4w4_launch on that expert alone.  No counterpart in the
 * reference (its launcher takes one weight matrix). */
int mbs_gemm_a4w4_grouped_launch(const uint8_t* A, const uint8_t* B, const uint8_t* AScale,
                                 const uint8_t* BScale, const uint8_t* AFactor,
                                 const uint8_t* BFactor, const int* group_offsets, int num_groups,
                                 void* out, int M, int N, int K, int Mpad, int scaleN_pad,
                                 int config, void* stream);
/* mbs_gemm_a4w4_grouped_launch with the affine epilogue of
 * mbs_gemm_a4w4_launch_ex: expert e's rows get
 * bf16(C * (alpha * f(a) * f(b)) + bias[e][n]); bias is bf16 [E][N] or NULL.
 * No counterpart in the reference. */
int mbs_gemm_a4w4_grouped_launch_ex(const uint8_t* A, const uint8_t* B, const uint8_t* AScale,
                                    const uint8_t* BScale, const uint8_t* AFactor,
                                    const uint8_t* BFactor, const int* group_offsets,
                                    int num_groups, void* out, int M, int N, int K, int Mpad,
                                    int scaleN_pad, float alpha, const void* bias, int config,
                                    void* stream);
/* Report on a grouped launch's device offsets (one small kernel; the
 * caller reads `status` after the stream reaches it):
 *   status[0] = non-empty experts whose first row is not a multiple of 32
 *               (the grouped kernels skip them),
 *   status[1] = entries the kernels clamp: group_offsets[0] != 0, an entry
 *               outside [0, M], or a decrease.
 * `status` is 2 device uint32 words, written (not accumulated).  No
 * counterpart in the reference. */
int mbs_gemm_a4w4_check_groups(const int* group_offsets, int num_groups, int M, uint32_t* status,
                               void* stream);
int mbs_gemm_a4w4_grouped_num_configs(void);
const char* mbs_gemm_a4w4_grouped_config_name(int config);

/* Workspace the heuristic launch of (M,N,K) wants (0 if it needs none).
 * Passing less makes mbs_gemm_a4w4_launch fall back to a no-split plan.
 * No counterpart in the reference (its launcher never splits K). */
size_t mbs_gemm_a4w4_workspace_bytes(int M, int N, int K);

/* Plan introspection and forced plans, for tests and tuning.  A plan is a
 * (kernel family, tile, split) triple; mbs_gemm_a4w4_plan_name() describes
 * the one the heuristic picks for (M,N,K).  mbs_gemm_a4w4_launch_config()
 * runs kernel configuration `config` (0 <= config < mbs_gemm_a4w4_num_configs())
 * with `splits` K-splits (0 = the heuristic's choice for that config).  The
 * configurations named *_m32 (32x32x64-MFMA tiles) run K % 512 == 0 with one
 * split only and return MBS_ERR_CONFIG otherwise, before any launch.
 * Stands in for the reference's MBS_FORCE_TILE_ENV / MBS_TILE debug switch
 * (kernel/gemm_a4w4.hip:1094-1102). */
int mbs_gemm_a4w4_num_configs(void);
const char* mbs_gemm_a4w4_config_name(int config);
int mbs_gemm_a4w4_plan_name(int M, int N, int K, char* buf, size_t buf_len);
size_t mbs_gemm_a4w4_config_workspace_bytes(int config, int splits, int M, int N, int K);
int mbs_gemm_a4w4_launch_config(int config, int splits, const uint8_t* A, const uint8_t* B,
                                const uint8_t* AScale, const uint8_t* BScale,
                                const uint8_t* AFactor, const uint8_t* BFactor, void* out,
                                int M, int N, int K, int Mpad, int scaleN_pad,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Decode GEMM from a bf16 activation in one launch:  x bf16 [M, K] (row
 * stride K, 16-byte aligned), M <= 32, is quantized to MXFP4 inside the
 * decode kernel (the rule of mbs_quantize_mxfp4_bf16, in registers; nothing
 * is written back) and multiplied by B as in mbs_gemm_a4w4_launch_ex with no
 * factors:  out[m][n] = bf16(C[m][n] * alpha + bias[n]).  The output bytes
 * equal mbs_quantize_mxfp4_bf16 (shuffled scales) followed by
 * mbs_gemm_a4w4_launch_ex on the same decode plan.  With BFactor ([N] u8, or
 * NULL) the activation is MBS-quantized instead (the rule of
 * mbs_quantize_mxfp4_mbs_bf16: each row's factor byte from its maximum over
 * all of K, derived inside the kernel) and the factor epilogue applies both
 * factors; the bytes equal mbs_quantize_mxfp4_mbs_bf16 followed by
 * mbs_gemm_a4w4_launch_ex with AFactor and BFactor.  MBS takes M <= 8 and a
 * 16-row decode configuration without K splits (MBS_ERR_ARGUMENT /
 * MBS_ERR_CONFIG otherwise) and no workspace.  config < 0 takes the
 * plan the heuristic picks among the skinny (decode) configurations, the
 * one mbs_gemm_a4w4_launch runs for these shapes; config >= 0 must name a
 * skinny configuration (MBS_ERR_CONFIG otherwise), with `splits` as in
 * mbs_gemm_a4w4_launch_config.  M > 32 returns MBS_ERR_ARGUMENT.  Split-K
 * plans use `workspace` (size it with mbs_gemm_a4w4_from_bf16_workspace_bytes
 * or, for a forced config, mbs_gemm_a4w4_config_workspace_bytes).  Replaces
 * the two launches of the reference's decode flow, aiter's per_1x32 quantizer
 * then gemm_a4w4 (test_gemm_a4w4.py:134-141, bench_one.py:19-30); the
 * reference has no fused form.  Every workgroup quantizes the rows it needs
 * itself: for M <= 8 (only the live rows' blocks) this is faster than the two
 * launches; for larger M each workgroup re-quantizes 16 or 32 rows and the
 * two launches are faster (measured at N = K = 8192 on MI355X).  With MBS
 * activations every workgroup also reads its rows over all of K for their
 * maxima first; one launch is then faster for M <= 4. */
int mbs_gemm_a4w4_from_bf16_launch(int config, int splits, const void* x, const uint8_t* B,
                                   const uint8_t* BScale, const uint8_t* BFactor, void* out, int M,
                                   int N, int K, int Mpad, int scaleN_pad, float alpha,
                                   const void* bias, void* workspace, size_t workspace_bytes,
                                   void* stream);
/* Workspace the heuristic (config < 0) bf16-activation launch wants. */
size_t mbs_gemm_a4w4_from_bf16_workspace_bytes(int M, int N, int K);

/* ---------------------------------------------------------------- formats
 * The on-device format helpers the reference takes from aiter
 * (test_gemm_a4w4.py:134-141): quantize, preshuffle, dequantize.
 */

/* bf16 [rows, K] (row stride K) -> packed e2m1 [rows, K/2] + E8M0 scales.
 * Rule: OCP MX v1.0 MXFP4 -- block exponent floor(log2 amax) - 2 (biased,
 * clamped to [0,254]; all-zero block -> 0x00), e2m1 round-to-nearest-even,
 * saturate to +-6, low nibble = even k.  `scale_shuffled` (may be NULL)
 * receives the shuffled layout of round_up(rows,32)*scaleN_pad bytes with
 * padding filled with `pad_byte`; `scale_plain` (may be NULL) receives
 * [rows, K/32].  K % 32 == 0.  Replaces aiter.get_triton_quant(per_1x32)
 * as called at test_gemm_a4w4.py:134-140 (rounding rule). */
int mbs_quantize_mxfp4_bf16(const void* x, int rows, int K, uint8_t* packed,
                            uint8_t* scale_shuffled, uint8_t* scale_plain, int pad_byte,
                            void* stream);

/* MBS quantization: as mbs_quantize_mxfp4_bf16, but each row is first
 * scaled by its MBS multiplier 1 + f/256, where the factor byte f (written
 * to factors[row]) is the top 8 mantissa bits of 6/max|row| (IEEE fp32
 * division, truncated; a zero, infinite or NaN maximum gives 0).  Passing
 * the factors of A and B to mbs_gemm_a4w4_launch undoes the multipliers
 * (f(b) = 1/(1 + b/256)).  This is the factor computation the reference
 * describes at docs/kernel_advanced.md:120-129 and consumes at
 * kernel/gemm_a4w4.h:20-22; the reference ships no kernel for it. */
int mbs_quantize_mxfp4_mbs_bf16(const void* x, int rows, int K, uint8_t* packed,
                                uint8_t* scale_shuffled, uint8_t* scale_plain, uint8_t* factors,
                                int pad_byte, void* stream);

/* Plain packed weights [N, K/2] -> (16,16)-preshuffled [N, K/2] (out of place).
 * Replaces aiter.ops.shuffle.shuffle_weight(w, layout=(16,16))
 * (test_gemm_a4w4.py:141). */
int mbs_shuffle_b(const uint8_t* w, uint8_t* out, int N, int K, void* stream);

/* Plain E8M0 [rows, K/32] -> shuffled buffer (padding = pad_byte). */
int mbs_shuffle_scales(const uint8_t* plain, uint8_t* out, int rows, int K, int pad_byte,
                       void* stream);

/* Inverse of mbs_shuffle_b: (16,16)-preshuffled [N, K/2] -> plain [N, K/2]
 * (out of place).  The inverse of aiter.ops.shuffle.shuffle_weight, which
 * the reference does not have; used to read back the on-disk weight format
 * (test_gemm_a4w4.py:141 produces it). */
int mbs_unshuffle_b(const uint8_t* in, uint8_t* w, int N, int K, void* stream);

/* Inverse of mbs_shuffle_scales on the live entries: shuffled buffer ->
 * plain [rows, K/32] (the padding is dropped).  K % 32 == 0. */
int mbs_unshuffle_scales(const uint8_t* shuffled, uint8_t* plain, int rows, int K, void* stream);

/* Format check of a shuffled scale buffer (round_up(rows,32)*scaleN_pad
 * bytes): writes counts[0] = padding entries != pad_byte (pad_byte = -1
 * skips that check) and counts[1] = live entries equal to 0xFF (E8M0 NaN).
 * `counts` is 2 device uint32 words, written (not accumulated), so it needs
 * no clearing.  One workgroup: meant for load-time validation, not the hot
 * path.  No counterpart in the reference, whose launcher reads the buffer
 * unchecked (interface/gemm_a4w4_pybind.cpp:22-44 checks no scale size). */
int mbs_check_scales(const uint8_t* shuffled, int rows, int K, int pad_byte, uint32_t* counts,
                     void* stream);

/* Packed operand + shuffled scales -> fp32 [rows, K]:
 * e2m1(code) * 2^(e-127) (e=255 -> NaN).  b_preshuffled selects the B layout
 * for `packed`.  Replaces fp4_utils.mxfp4_to_f32 * e8m0_to_f32 as used by
 * run_torch (test_gemm_a4w4.py:33-42); bit-exact by construction. */
int mbs_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale_shuffled, float* out,
                      int rows, int K, int b_preshuffled, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MBS_GEMM_A4W4_H_ */
