/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the MXFP4 A4W4 GEMM path.
 *
 * This file restates, in plain C, the arithmetic of the reference's
 * dequantize-to-fp32-then-matmul oracle and the byte layouts its kernel
 * consumes.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker; the shipped HIP path never does.
 *
 * Reference anchors (paths relative to the reference tree):
 *   - oracle op order ........ test_gemm_a4w4.py:28-44   (run_torch)
 *   - MBS factor oracle ...... test_gemm_a4w4.py:47-69   (convert_byte_to_float,
 *                                                         run_torch_mbs)
 *   - B preshuffle ........... kernel/gemm_a4w4.hip:19-22,84-95 (flatB),
 *                              analyze.txt:13-20
 *   - scale shuffle .......... kernel/gemm_a4w4.hip:23-25,97-105 (flatS),
 *                              analyze.txt:1-10
 *   - output / padding ....... kernel/gemm_a4w4.h:5-26,
 *                              interface/gemm_a4w4_pybind.cpp:46-63
 *   - e2m1 code 0x2 == +1.0 .. kernel/mfma_probe.hip:20
 *   - quantizer rule ......... BASELINE.json configs[0] (OCP MX v1.0 MXFP4:
 *                              E8M0 = floor(log2 amax) - 2 + 127, e2m1 RNE,
 *                              saturate to +-6, low nibble = even K index)
 *
 * Every function is plain scalar C so a reader can check it line by line;
 * speed only matters for the quantizer and dequantizer (they run on the
 * 8192 x 8192 bench configs) and those are simple O(n) loops.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bits */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------- element decode */

/* e2m1 magnitudes for codes 0..7 (OCP MX v1.0, table "FP4 E2M1"): exponent
 * bits 2:1 (bias 1), mantissa bit 0; code 0b001 is the subnormal 0.5.  Bit 3
 * is the sign.  mfma_probe.hip:20 pins code 0x2 == +1.0. */
static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

float oracle_e2m1_to_f32(uint8_t code)
{
    float m = kE2M1[code & 7];
    return (code & 8) ? -m : m;
}

/* E8M0: 2^(e-127); e == 255 is NaN (OCP MX v1.0); e == 0 is 2^-127, an fp32
 * subnormal (bit pattern 0x00400000).  Built from bits so no FTZ can bite. */
float oracle_e8m0_to_f32(uint8_t e)
{
    if (e == 255) return bits_f32(0x7FC00000u);
    if (e == 0) return bits_f32(0x00400000u);
    return bits_f32((uint32_t)e << 23);
}

/* -------------------------------------------------------------- quantize */

/* Round |q| (already divided by the block scale, |q| < 8) to the e2m1 grid
 * {0,.5,1,1.5,2,3,4,6} with round-to-nearest-even on the code and saturation
 * at 6.  Ties go to the even code (codes 0,2,4,6 = 0,1,2,4). */
static uint8_t e2m1_rne_mag(float q)
{
    /* grid midpoints and the codes on either side */
    if (q < 0.25f) return 0;
    if (q == 0.25f) return 0;          /* tie 0 / 0.5  -> 0 (even)   */
    if (q < 0.75f) return 1;
    if (q == 0.75f) return 2;          /* tie 0.5 / 1 -> 1 (even)    */
    if (q < 1.25f) return 2;
    if (q == 1.25f) return 2;          /* tie 1 / 1.5 -> 1           */
    if (q < 1.75f) return 3;
    if (q == 1.75f) return 4;          /* tie 1.5 / 2 -> 2           */
    if (q < 2.5f) return 4;
    if (q == 2.5f) return 4;           /* tie 2 / 3 -> 2             */
    if (q < 3.5f) return 5;
    if (q == 3.5f) return 6;           /* tie 3 / 4 -> 4             */
    if (q < 5.0f) return 6;
    if (q == 5.0f) return 6;           /* tie 4 / 6 -> 4             */
    return 7;                          /* (5, inf) -> 6, saturating  */
}

/* floor(log2(a)) for finite a > 0, exact (read from the fp32 exponent; a
 * subnormal is normalised first). */
static int floor_log2_f32(float a)
{
    uint32_t u = f32_bits(a);
    int e = (int)((u >> 23) & 0xFF);
    if (e != 0) return e - 127;
    uint32_t m = u & 0x7FFFFF; /* subnormal: value = m * 2^-149 */
    int msb = 31 - __builtin_clz(m);
    return msb - 149;
}

/* Block E8M0 byte for one 32-element block, BASELINE.json configs[0]:
 * shared exponent floor(log2(amax)) - 2, biased by 127, clamped to [0, 254].
 * An all-zero block gets 0x00 (configs[4]: "all-zero blocks ... scale 0x00").
 * A block holding a NaN gets 0xFF (NaN) and every element code 0. */
static uint8_t block_scale(const float* x, int n, int* has_nan)
{
    float amax = 0.0f;
    *has_nan = 0;
    for (int i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a != a) { *has_nan = 1; continue; }
        if (a > amax) amax = a;
    }
    if (*has_nan) return 255;
    if (amax == 0.0f) return 0;
    if (isinf(amax)) return 254;
    int e = floor_log2_f32(amax) - 2 + 127;
    if (e < 0) e = 0;
    if (e > 254) e = 254;
    return (uint8_t)e;
}

/* Quantize rows x K fp32 values (K % 32 == 0) to MXFP4: packed[r][k/2] holds
 * element k in the low nibble when k is even and
 * scales[r][k/32] the block's E8M0 byte (plain, unshuffled [rows, K/32]). */
void oracle_quantize_mxfp4(const float* x, int64_t rows, int64_t K,
                           uint8_t* packed, uint8_t* scales)
{
    const int64_t nb = K / 32;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const float* xb = x + r * K + b * 32;
            int has_nan = 0;
            uint8_t s = block_scale(xb, 32, &has_nan);
            scales[r * nb + b] = s;
            /* divide by 2^(s-127): exact (power of two), done as a multiply by
             * 2^(127-s); for s near 0 the factor 2^127 is still finite. */
            float inv = ldexpf(1.0f, 127 - (int)s);
            uint8_t codes[32];
            for (int i = 0; i < 32; ++i) {
                float v = xb[i];
                uint8_t sign = (f32_bits(v) >> 31) ? 8 : 0;
                if (has_nan || v != v) { codes[i] = 0; continue; }
                float q = fabsf(v) * inv;
                codes[i] = (uint8_t)(sign | e2m1_rne_mag(q));
            }
            uint8_t* out = packed + r * (K / 2) + b * 16;
            for (int i = 0; i < 16; ++i)
                out[i] = (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
        }
    }
}

/* --------------------------------------------------- MBS row factors ---- */

/* MBS factor byte of a row with absolute maximum amax, after
 * docs/kernel_advanced.md:120-125 of the reference: scale = 6.0 / max, and
 * the factor is the top 8 bits of scale's fp32 mantissa (fp32 division,
 * round to nearest even, then truncation).  A zero, infinite or NaN maximum
 * gives 0 (factor 1.0): 6/0 and 6/tiny overflow to +inf, whose mantissa is 0. */
uint8_t oracle_mbs_factor_byte(float amax)
{
    if (!(amax > 0.0f) || amax == INFINITY) return 0;
    volatile float s = 6.0f / amax;  /* IEEE single division */
    return (uint8_t)((f32_bits(s) >> 15) & 0xFF);
}

/* MBS quantization of rows: factor byte b per row from its absolute
 * maximum, the row multiplied by 1 + b/256 (the bits 0x3F800000 | b << 15:
 * the "1.xxxxx" of docs/kernel_advanced.md:128), then ordinary MXFP4
 * quantization.  The GEMM epilogue's f(b) = 1/(1 + b/256)
 * (test_gemm_a4w4.py:47-51) undoes the multiplier.  For bf16-valued inputs
 * the product is exact in fp32 (8 + 9 significant bits).  A row holding a
 * NaN gets factor 0. */
void oracle_quantize_mxfp4_mbs(const float* x, int64_t rows, int64_t K,
                               uint8_t* packed, uint8_t* scales, uint8_t* factors)
{
    float* row = (float*)malloc((size_t)K * sizeof(float));
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * K;
        float amax = 0.0f;
        int nan = 0;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(xr[k]);
            if (a != a) nan = 1;
            else if (a > amax) amax = a;
        }
        const uint8_t b = nan ? 0 : oracle_mbs_factor_byte(amax);
        const uint32_t mb = 0x3F800000u | ((uint32_t)b << 15);
        float m;
        memcpy(&m, &mb, 4);
        for (int64_t k = 0; k < K; ++k) row[k] = xr[k] * m;
        factors[r] = b;
        oracle_quantize_mxfp4(row, 1, K, packed + r * (K / 2), scales + r * (K / 32));
    }
    free(row);
}

/* ------------------------------------------------------------ dequantize */

/* out[r][k] = e2m1(packed nibble) * e8m0(scales[r][k/32]) in fp32 -- the
 * reference's mxfp4_to_f32(x) * e8m0_to_f32(scales.repeat_interleave(32))
 * (test_gemm_a4w4.py:33-42).  Each product is exact in fp32 (a 3-bit
 * significand times a power of two, staying >= 2^-128). */
void oracle_dequant_mxfp4(const uint8_t* packed, const uint8_t* scales,
                          int64_t rows, int64_t K, float* out)
{
    const int64_t nb = K / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t k = 0; k < K; ++k) {
            uint8_t byte = packed[r * (K / 2) + k / 2];
            uint8_t code = (k & 1) ? (byte >> 4) : (byte & 15);
            out[r * K + k] = oracle_e2m1_to_f32(code) *
                             oracle_e8m0_to_f32(scales[r * nb + k / 32]);
        }
}

/* --------------------------------------------------------------- layouts */

/* B preshuffle, layout (16,16) -- kernel/gemm_a4w4.hip:19-22 (flatB) and
 * analyze.txt:13-20: view [N/16, 16, Kp/32, 2, 16] permuted to
 * [N/16, Kp/32, 2, 16, 16].  Byte (n, kp) of the plain [N, Kp] matrix goes to
 *   (n/16)*(Kp*16) + (kp/32)*512 + ((kp%32)/16)*256 + (n%16)*16 + kp%16.
 * Needs N % 16 == 0 and Kp % 32 == 0 (K % 64 == 0). */
int64_t oracle_flat_b(int64_t n, int64_t kp, int64_t Kp)
{
    return (n / 16) * (Kp * 16) + (kp / 32) * 512 + ((kp % 32) / 16) * 256 +
           (n % 16) * 16 + (kp % 16);
}

void oracle_shuffle_b(const uint8_t* w, int64_t N, int64_t Kp, uint8_t* out)
{
    for (int64_t n = 0; n < N; ++n)
        for (int64_t kp = 0; kp < Kp; ++kp)
            out[oracle_flat_b(n, kp, Kp)] = w[n * Kp + kp];
}

void oracle_unshuffle_b(const uint8_t* in, int64_t N, int64_t Kp, uint8_t* w)
{
    for (int64_t n = 0; n < N; ++n)
        for (int64_t kp = 0; kp < Kp; ++kp)
            w[n * Kp + kp] = in[oracle_flat_b(n, kp, Kp)];
}

/* E8M0 scale shuffle -- kernel/gemm_a4w4.hip:23-25,97-105 (flatS) and
 * analyze.txt:1-10: the padded [Rpad, SNp] scale matrix viewed as
 * [Rpad/32, 2, 16, SNp/8, 2, 4] and permuted to [Rpad/32, SNp/8, 4, 16, 2, 2].
 * Byte (r, b) goes to
 *   (r/32)*32*SNp + (b/8)*256 + (b%4)*64 + (r%16)*4 + ((b%8)/4)*2 + (r%32)/16. */
int64_t oracle_flat_s(int64_t r, int64_t b, int64_t scaleN_pad)
{
    return (r / 32) * 32 * scaleN_pad + (b / 8) * 256 + (b % 4) * 64 +
           (r % 16) * 4 + ((b % 8) / 4) * 2 + (r % 32) / 16;
}

/* Scatter plain scales [rows, nb] into a shuffled buffer of
 * round_up(rows,32) * scaleN_pad bytes; padding rows/blocks get `pad`. */
void oracle_shuffle_scales(const uint8_t* s, int64_t rows, int64_t nb,
                           int64_t scaleN_pad, uint8_t pad, uint8_t* out)
{
    const int64_t rows_pad = (rows + 31) / 32 * 32;
    for (int64_t r = 0; r < rows_pad; ++r)
        for (int64_t b = 0; b < scaleN_pad; ++b) {
            uint8_t v = (r < rows && b < nb) ? s[r * nb + b] : pad;
            out[oracle_flat_s(r, b, scaleN_pad)] = v;
        }
}

void oracle_unshuffle_scales(const uint8_t* in, int64_t rows, int64_t nb,
                             int64_t scaleN_pad, uint8_t* s)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b)
            s[r * nb + b] = in[oracle_flat_s(r, b, scaleN_pad)];
}

/* ------------------------------------------------------ factor and bf16 */

/* MBS factor f(b) = 1 / (1 + b/256) exactly as test_gemm_a4w4.py:47-51 does it:
 * b fills the top 8 mantissa bits of 1.0f (0x3F800000 | b << 15), then one
 * IEEE fp32 division (correctly rounded). */
float oracle_mbs_factor(uint8_t b)
{
    volatile float one = bits_f32(0x3F800000u | ((uint32_t)b << 15));
    return 1.0f / one;
}

/* fp32 -> bf16 round-to-nearest-even (torch .to(torch.bfloat16)); NaN maps to
 * a quiet NaN with the sign kept. */
uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t u = f32_bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

/* ------------------------------------------------------------------ GEMM */

/* c[M,N] = a[M,K] . b[N,K]^T with an fp32 accumulator, k ascending.  This is
 * the textbook contraction torch.mm performs (test_gemm_a4w4.py:44); only
 * the summation order differs from a blocked BLAS, which the tests bound. */
void oracle_gemm_f32(const float* a, const float* b, int64_t M, int64_t N,
                     int64_t K, float* c)
{
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            const float* ar = a + m * K;
            const float* br = b + n * K;
            for (int64_t k = 0; k < K; ++k) acc += ar[k] * br[k];
            c[m * N + n] = acc;
        }
}

/* Epilogue of run_torch_mbs (test_gemm_a4w4.py:65-69): c * (f(a)[m] * f(b)[n])
 * with the factor product formed first, then bf16 RNE.  Null factors mean
 * plain run_torch (test_gemm_a4w4.py:44). */
void oracle_epilogue_bf16(const float* c, int64_t M, int64_t N,
                          const uint8_t* a_factor, const uint8_t* b_factor,
                          uint16_t* out)
{
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float v = c[m * N + n];
            if (a_factor && b_factor) {
                float p = oracle_mbs_factor(a_factor[m]) * oracle_mbs_factor(b_factor[n]);
                v = v * p;
            }
            out[m * N + n] = oracle_f32_to_bf16(v);
        }
}
