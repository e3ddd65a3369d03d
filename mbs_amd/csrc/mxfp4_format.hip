// On-device MXFP4 format helpers for gfx950: quantize bf16 -> packed e2m1 +
// E8M0 (plain and/or shuffled scales), preshuffle B with layout (16,16),
// shuffle scales, and dequantize back to fp32.  These replace the aiter
// helpers the reference drives its GEMM with (test_gemm_a4w4.py:134-141) and
// the dequant half of its oracle (test_gemm_a4w4.py:33-42).  All byte
// layouts are the ones the GEMM consumes (see mbs_gemm_a4w4.h).
#include "mxfp4_device.h"
#include "mbs_gemm_a4w4.h"

namespace mbs {

__device__ __forceinline__ int64_t flat_b(int64_t n, int64_t kp, int64_t Kp)
{
    return (n >> 4) * (Kp * 16) + (kp >> 5) * 512 + ((kp & 31) >> 4) * 256 + (n & 15) * 16 +
           (kp & 15);
}

__device__ __forceinline__ int64_t flat_s(int64_t r, int64_t b, int64_t snp)
{
    return (r >> 5) * 32 * snp + (b >> 3) * 256 + (b & 3) * 64 + (r & 15) * 4 +
           ((b & 7) >> 2) * 2 + ((r & 31) >> 4);
}

// floor(log2(a)) of a finite a > 0 given its fp32 bits (subnormals included).
__device__ __forceinline__ int floor_log2_bits(uint32_t u)
{
    const int e = (int)((u >> 23) & 0xFF);
    if (e != 0) return e - 127;
    return (31 - __builtin_clz(u & 0x7FFFFFu)) - 149;
}

// One thread per 32-element K-block: amax -> E8M0, then e2m1 round to
// nearest even on the code with saturation at 6.  The code of |q| is the
// number of grid midpoints it passes: ties at 0.25, 1.25, 2.5, 5 go down to
// the even code, ties at 0.75, 1.75, 3.5 go up to it.
__global__ void __launch_bounds__(256)
quantize_bf16_kernel(const uint16_t* __restrict__ x, int rows, int K, uint8_t* __restrict__ packed,
                     uint8_t* __restrict__ sshuf, uint8_t* __restrict__ splain, int snp)
{
    const int nb = K >> 5;
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= (int64_t)rows * nb) return;
    const int r = (int)(blk / nb), b = (int)(blk - (int64_t)r * nb);
    const i32x4* src = reinterpret_cast<const i32x4*>(x + (int64_t)r * K + b * 32);
    uint32_t w[16];
    for (int i = 0; i < 4; ++i) {
        const i32x4 v = src[i];
        w[4 * i + 0] = v[0];
        w[4 * i + 1] = v[1];
        w[4 * i + 2] = v[2];
        w[4 * i + 3] = v[3];
    }
    // bf16 -> fp32 bits is a 16-bit shift; track amax on the magnitude bits
    // (monotone for non-NaN values) and NaN separately.
    uint32_t amax_bits = 0;
    bool nan = false;
    for (int i = 0; i < 32; ++i) {
        const uint32_t h = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xFFFF);
        const uint32_t m = (h & 0x7FFF) << 16;
        nan |= m > 0x7F800000u;
        amax_bits = (m > amax_bits && m <= 0x7F800000u) ? m : amax_bits;
    }
    uint32_t s;
    if (nan) s = 255;
    else if (amax_bits == 0) s = 0;
    else if (amax_bits == 0x7F800000u) s = 254;
    else {
        int e = floor_log2_bits(amax_bits) - 2 + 127;
        s = (uint32_t)(e < 0 ? 0 : (e > 254 ? 254 : e));
    }
    // 2^(127 - s), s in [0, 254]: exponent field 254 - s, or the subnormal
    // 2^-127 for s == 254.
    const float inv = (s == 254) ? __uint_as_float(0x00400000u) : __uint_as_float((254u - s) << 23);
    uint32_t out[4] = {0, 0, 0, 0};
    for (int i = 0; i < 32; ++i) {
        const uint32_t h = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xFFFF);
        const float q = __uint_as_float((h & 0x7FFF) << 16) * inv;
        uint32_t c = (uint32_t)(q > 0.25f) + (uint32_t)(q >= 0.75f) + (uint32_t)(q > 1.25f) +
                     (uint32_t)(q >= 1.75f) + (uint32_t)(q > 2.5f) + (uint32_t)(q >= 3.5f) +
                     (uint32_t)(q > 5.0f);
        c |= (h >> 12) & 8u;  // sign
        if (nan) c = 0;
        out[i >> 3] |= c << (4 * (i & 7));
    }
    i32x4 o = {(int)out[0], (int)out[1], (int)out[2], (int)out[3]};
    *reinterpret_cast<i32x4*>(packed + (int64_t)r * (K >> 1) + b * 16) = o;
    if (splain) splain[(int64_t)r * nb + b] = (uint8_t)s;
    if (sshuf) sshuf[flat_s(r, b, snp)] = (uint8_t)s;
}

// Padding entries of a shuffled scale buffer (rows >= R or blocks >= nb).
__global__ void __launch_bounds__(256)
scale_pad_kernel(uint8_t* __restrict__ sshuf, int rows, int nb, int snp, uint8_t pad)
{
    const int rows_pad = (rows + 31) & ~31;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows_pad * snp) return;
    const int r = (int)(i / snp), b = (int)(i - (int64_t)r * snp);
    if (r >= rows || b >= nb) sshuf[flat_s(r, b, snp)] = pad;
}

__global__ void __launch_bounds__(256)
shuffle_scales_kernel(const uint8_t* __restrict__ plain, uint8_t* __restrict__ out, int rows,
                      int nb, int snp, uint8_t pad)
{
    const int rows_pad = (rows + 31) & ~31;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows_pad * snp) return;
    const int r = (int)(i / snp), b = (int)(i - (int64_t)r * snp);
    out[flat_s(r, b, snp)] = (r < rows && b < nb) ? plain[(int64_t)r * nb + b] : pad;
}

// 16 bytes per thread: (n, kp..kp+15) is contiguous in both layouts.
__global__ void __launch_bounds__(256)
shuffle_b_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ out, int N, int Kp)
{
    const int per_row = Kp >> 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)N * per_row) return;
    const int n = (int)(i / per_row), kp = (int)(i - (int64_t)n * per_row) * 16;
    *reinterpret_cast<i32x4*>(out + flat_b(n, kp, Kp)) =
        *reinterpret_cast<const i32x4*>(w + (int64_t)n * Kp + kp);
}

// fp32 bits of (code value) * 2^(e-127), built with integer ops so the result
// is exact whatever the float denormal mode: the code value is k/2 with k in
// {0,1,2,3,4,6,8,12}, so the product is k * 2^(e-128).
__device__ __forceinline__ uint32_t dequant_bits(uint32_t code, uint32_t e)
{
    if (e == 255) return 0x7FC00000u;
    const uint32_t sign = (code & 8u) << 28;
    const uint32_t mag = code & 7u;
    if (mag == 0) return sign;
    const uint32_t k = (mag < 4) ? mag : ((mag & 1) ? 3u : 2u) << ((mag >> 1) - 1);
    const int t = 31 - __builtin_clz(k);               // k = 2^t * {1, 1.5}
    const int E = t + (int)e - 128;                    // unbiased exponent
    if (E > 127) return sign | 0x7F800000u;            // overflow (e >= 253): inf
    if (E >= -126) return sign | ((uint32_t)(E + 127) << 23) | ((k > (1u << t)) ? 0x400000u : 0u);
    return sign | (k << ((int)e + 21));                // subnormal: k * 2^(e-128+149)
}

__global__ void __launch_bounds__(256)
dequant_kernel(const uint8_t* __restrict__ packed, const uint8_t* __restrict__ sshuf,
               float* __restrict__ out, int rows, int K, int snp, int preshuffled)
{
    const int Kp = K >> 1, per_row = Kp >> 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * per_row) return;
    const int r = (int)(i / per_row), c = (int)(i - (int64_t)r * per_row);
    const int64_t src = preshuffled ? flat_b(r, c * 16, Kp) : (int64_t)r * Kp + c * 16;
    const i32x4 v = *reinterpret_cast<const i32x4*>(packed + src);
    const uint32_t e = sshuf[flat_s(r, c, snp)];
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + (int64_t)r * K + c * 32);
    for (int q = 0; q < 4; ++q) {
        const uint32_t word = (uint32_t)v[q];
        uint32_t o[8];
        for (int j = 0; j < 8; ++j) o[j] = dequant_bits((word >> (4 * j)) & 15u, e);
        i32x4 lo = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
        i32x4 hi = {(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
        *reinterpret_cast<i32x4*>(dst + q * 8) = lo;
        *reinterpret_cast<i32x4*>(dst + q * 8 + 4) = hi;
    }
}

namespace {
int fmt_fail(const char* m)
{
    set_last_error(m);
    return MBS_ERR_ARGUMENT;
}
int scale_pad_of(int K) { return ((K + 31) / 32 + 7) / 8 * 8; }
unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }
int launched()
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(hipGetErrorString(e));
        return MBS_ERR_LAUNCH;
    }
    return MBS_OK;
}
}  // namespace

}  // namespace mbs

using namespace mbs;

extern "C" {

int mbs_quantize_mxfp4_bf16(const void* x, int rows, int K, uint8_t* packed,
                            uint8_t* scale_shuffled, uint8_t* scale_plain, int pad_byte,
                            void* stream)
{
    if (!x || !packed) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    if (pad_byte < 0 || pad_byte > 255) return fmt_fail("pad_byte must be a byte");
    (void)hipGetLastError();
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int snp = scale_pad_of(K);
    const int nb = K / 32;
    if (scale_shuffled) {
        const int64_t n = (int64_t)((rows + 31) & ~31) * snp;
        if ((rows % 32) || nb != snp)
            hipLaunchKernelGGL(scale_pad_kernel, dim3(blocks_for(n)), dim3(256), 0, s,
                               scale_shuffled, rows, nb, snp, (uint8_t)pad_byte);
    }
    hipLaunchKernelGGL(quantize_bf16_kernel, dim3(blocks_for((int64_t)rows * nb)), dim3(256), 0,
                       s, static_cast<const uint16_t*>(x), rows, K, packed, scale_shuffled,
                       scale_plain, snp);
    return launched();
}

int mbs_shuffle_b(const uint8_t* w, uint8_t* out, int N, int K, void* stream)
{
    if (!w || !out) return fmt_fail("null pointer");
    if (N < 16 || N % 16 || K < 64 || K % 64) return fmt_fail("need N % 16 == 0 and K % 64 == 0");
    if (w == out) return fmt_fail("shuffle_b is out of place");
    (void)hipGetLastError();
    hipLaunchKernelGGL(shuffle_b_kernel, dim3(blocks_for((int64_t)N * (K / 32))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), w, out, N, K / 2);
    return launched();
}

int mbs_shuffle_scales(const uint8_t* plain, uint8_t* out, int rows, int K, int pad_byte,
                       void* stream)
{
    if (!plain || !out) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    if (pad_byte < 0 || pad_byte > 255) return fmt_fail("pad_byte must be a byte");
    (void)hipGetLastError();
    const int snp = scale_pad_of(K);
    const int64_t n = (int64_t)((rows + 31) & ~31) * snp;
    hipLaunchKernelGGL(shuffle_scales_kernel, dim3(blocks_for(n)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), plain, out, rows, K / 32, snp,
                       (uint8_t)pad_byte);
    return launched();
}

int mbs_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale_shuffled, float* out, int rows,
                      int K, int b_preshuffled, void* stream)
{
    if (!packed || !scale_shuffled || !out) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    if (b_preshuffled && (rows % 16 || K % 64))
        return fmt_fail("preshuffled layout needs rows % 16 == 0 and K % 64 == 0");
    (void)hipGetLastError();
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks_for((int64_t)rows * (K / 32))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), packed, scale_shuffled, out, rows, K,
                       scale_pad_of(K), b_preshuffled);
    return launched();
}

}  // extern "C"
