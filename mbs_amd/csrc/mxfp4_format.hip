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

// The e2m1 codes of the block are produced by the gfx950 scaled conversions
// v_cvt_scalef32_pk_fp4_{f32,bf16}: code = RNE(v / scale) on the e2m1 grid
// {0, .5, 1, 1.5, 2, 3, 4, 6} with ties to the even code and saturation at
// 6, sign kept (so -0 and negative values that round to zero give code 8);
// the first source goes to the low nibble, and the last argument selects the
// destination byte.  These semantics were measured on MI355X against the
// oracle's rule for every multiple of 1/8 in [-9, 9] (all ties), +-0, +-inf,
// huge and subnormal values, under scales 2^-127 .. 2^127; only NaN differs
// (the hardware gives code 7), and NaN blocks are written as zeros here, as
// the oracle does.  With scale = 2^(s-127) this is the oracle's
// q = x * 2^(127-s) followed by its midpoint count.

// Plain quantization, four lanes per 32-element K-block: lane q of a quad
// loads elements 8q..8q+7 (16 bytes, so a wave reads 1 KiB of a row
// contiguously), the quad combines its magnitudes into the block maximum, and
// each lane converts its 8 elements into one dword of packed output
// (v_cvt_scalef32_pk_fp4_bf16 straight from the bf16 pairs).  blockIdx.x:
// group of 4 rows (threadIdx.y), blockIdx.y: group of 64 chunks.  With a
// shuffled scale buffer the grid also covers its padding (rows up to
// round_up(rows, 32), blocks up to scaleN_pad), whose entries get `pad`, so
// one launch fills the whole buffer.
__global__ void __launch_bounds__(256)
quantize_bf16_kernel(const uint16_t* __restrict__ x, int rows, int K, uint8_t* __restrict__ packed,
                     uint8_t* __restrict__ sshuf, uint8_t* __restrict__ splain, int snp, uint8_t pad)
{
    const int nc = K >> 3;                               // 16-byte chunks per row
    const int j = blockIdx.y * 64 + threadIdx.x;          // chunk in the row
    const int r = blockIdx.x * 4 + threadIdx.y;           // row (uniform per wave)
    // nc % 4 == 0 and quads are 4-aligned: whole quads take the same branch,
    // so the quad exchanges below only read active lanes.
    if (r >= rows || j >= nc) {
        const int rows_pad = (rows + 31) & ~31;
        if (sshuf && r < rows_pad && j < 4 * snp && (threadIdx.x & 3) == 0)
            sshuf[flat_s(r, j >> 2, snp)] = pad;
        return;
    }
    const i32x4 v = *reinterpret_cast<const i32x4*>(x + (int64_t)r * K + (int64_t)j * 8);
    // magnitude maximum on the 15 magnitude bits: a NaN orders above inf
    uint32_t mx = bf16x8_absmax(v);
    mx = max(mx, (uint32_t)__shfl_xor((int)mx, 1));
    mx = max(mx, (uint32_t)__shfl_xor((int)mx, 2));
    const bool nan = mx > 0x7F80u;
    const uint32_t s = e8m0_of(mx << 16, nan);
    const float sc = e8m0_value(nan ? 127 : s);
    const uint32_t o = bf16x8_to_e2m1(v, sc);
    *reinterpret_cast<uint32_t*>(packed + (int64_t)r * (K >> 1) + (int64_t)j * 4) = nan ? 0u : o;
    if ((threadIdx.x & 3) == 0) {
        const int b = j >> 2;
        if (splain) splain[(int64_t)r * (K >> 5) + b] = (uint8_t)s;
        if (sshuf) sshuf[flat_s(r, b, snp)] = (uint8_t)s;
    }
}

// MBS quantization (docs/kernel_advanced.md:120-129 of the reference): one
// workgroup per row.  The row's absolute maximum gives the factor byte b =
// the top 8 mantissa bits of 6/max (IEEE division, then truncation; a zero,
// infinite or NaN maximum gives 0); the row is then quantized block by block
// after scaling by 1 + b/256, which the GEMM's factor epilogue
// f(b) = 1/(1 + b/256) undoes.
// Longest row the MBS kernel keeps in LDS (64 KiB of bf16).
constexpr int kMbsStagedK = 32768;
// Row counts below this take 1024 threads per row.
constexpr int kMbsWideRows = 256;

// STAGED (K * 2 bytes of dynamic LDS, K <= kMbsStagedK): the first pass
// also keeps the row in LDS and the quantize pass reads it from there, so the
// row is read from memory once; otherwise the quantize pass reads it again.
// NT threads per row: 1024 for few rows (decode batches, where the row's
// latency is the kernel's time), 256 otherwise.
template <bool STAGED, int NT>
__global__ void __launch_bounds__(NT)
quantize_mbs_bf16_kernel(const uint16_t* __restrict__ x, int rows, int K, uint8_t* __restrict__ packed,
                         uint8_t* __restrict__ sshuf, uint8_t* __restrict__ splain,
                         uint8_t* __restrict__ factors, int snp, uint8_t pad)
{
    __shared__ uint32_t red[NT / 64];
    extern __shared__ __attribute__((aligned(16))) uint8_t mbs_row[];
    i32x4* srow = reinterpret_cast<i32x4*>(mbs_row);
    const int r = blockIdx.x;
    // With a shuffled scale buffer the grid spans round_up(rows, 32) rows:
    // a padding row's workgroup only writes its pad bytes; every row writes
    // its padding blocks [K/32, scaleN_pad).
    if (r >= rows) {
        for (int b = threadIdx.x; b < snp; b += NT) sshuf[flat_s(r, b, snp)] = pad;
        return;
    }
    if (sshuf)
        for (int b = (K >> 5) + threadIdx.x; b < snp; b += NT) sshuf[flat_s(r, b, snp)] = pad;
    const uint16_t* xr = x + (int64_t)r * K;
    // row maximum on the magnitude bits; a NaN maps above every number
    uint32_t amax = 0;
    for (int e = threadIdx.x * 8; e < K; e += NT * 8) {
        const i32x4 v = *reinterpret_cast<const i32x4*>(xr + e);
        if constexpr (STAGED) srow[e >> 3] = v;
        for (int i = 0; i < 8; ++i) {
            const uint32_t h = ((uint32_t)v[i >> 1] >> (16 * (i & 1))) & 0x7FFF;
            amax = h > amax ? h : amax;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)amax, off);
        amax = o > amax ? o : amax;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = red[0];
    for (int i = 1; i < NT / 64; ++i) amax = red[i] > amax ? red[i] : amax;
    const uint32_t fb = mbs_factor_byte(amax);
    const float m = __uint_as_float(0x3F800000u | (fb << 15));
    if (threadIdx.x == 0) factors[r] = (uint8_t)fb;
    // Quantize pass, four lanes per 32-element block as in the plain kernel:
    // quad k of the workgroup takes blocks k, k + NT/4, ...; lane q of the quad
    // elements 8q..8q+7 of the block.  nb blocks per row: whole quads take
    // part in an iteration or none does, so the quad exchanges read active lanes.
    const int nb = K >> 5;
    const int q = threadIdx.x & 3;
    for (int b = threadIdx.x >> 2; b < nb; b += NT / 4) {
        i32x4 v;
        if constexpr (STAGED) v = srow[(b * 32 + q * 8) >> 3];   // written before the barrier above
        else v = *reinterpret_cast<const i32x4*>(xr + b * 32 + q * 8);
        const uint32_t w[4] = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
        uint32_t mx = 0;
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = w[i] & 0x7FFF7FFFu;
            mx = max(mx, max(a & 0xFFFFu, a >> 16));
        }
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 1));
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 2));
        const bool nan = mx > 0x7F80u;
        const uint32_t s = e8m0_of(__float_as_uint(__uint_as_float(mx << 16) * m), nan);
        const float sc = e8m0_value(nan ? 127 : s);
        uint32_t o = 0;
        static_for<4>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const float lo = __uint_as_float(w[j] << 16) * m;
            const float hi = __uint_as_float(w[j] & 0xFFFF0000u) * m;
            o = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(o, lo, hi, sc, j);
        });
        *reinterpret_cast<uint32_t*>(packed + (int64_t)r * (K >> 1) + b * 16 + q * 4) = nan ? 0u : o;
        if (q == 0) {
            if (splain) splain[(int64_t)r * nb + b] = (uint8_t)s;
            if (sshuf) sshuf[flat_s(r, b, snp)] = (uint8_t)s;
        }
    }
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

// Inverse of shuffle_b_kernel: preshuffled [N, K/2] -> plain row-major.
__global__ void __launch_bounds__(256)
unshuffle_b_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ w, int N, int Kp)
{
    const int per_row = Kp >> 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)N * per_row) return;
    const int n = (int)(i / per_row), kp = (int)(i - (int64_t)n * per_row) * 16;
    *reinterpret_cast<i32x4*>(w + (int64_t)n * Kp + kp) =
        *reinterpret_cast<const i32x4*>(in + flat_b(n, kp, Kp));
}

// Inverse of shuffle_scales_kernel on the live entries: shuffled -> plain
// [rows, nb] (the padding is dropped).
__global__ void __launch_bounds__(256)
unshuffle_scales_kernel(const uint8_t* __restrict__ sshuf, uint8_t* __restrict__ plain, int rows,
                        int nb, int snp)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * nb) return;
    const int r = (int)(i / nb), b = (int)(i - (int64_t)r * nb);
    plain[i] = sshuf[flat_s(r, b, snp)];
}

// Format check of a shuffled scale buffer, one workgroup (no atomics, so the
// counts need no clearing): counts[0] = padding entries that differ from
// `pad` (pad < 0: not checked), counts[1] = live entries equal to 0xFF (the
// E8M0 NaN encoding, which turns a whole block of the product into NaN).
__global__ void __launch_bounds__(1024)
check_scales_kernel(const uint8_t* __restrict__ sshuf, int rows, int nb, int snp, int pad,
                    uint32_t* __restrict__ counts)
{
    __shared__ uint32_t part[2][16];
    const int rows_pad = (rows + 31) & ~31;
    const int64_t total = (int64_t)rows_pad * snp;
    uint32_t bad_pad = 0, nan_live = 0;
    for (int64_t i = threadIdx.x; i < total; i += 1024) {
        const int r = (int)(i / snp), b = (int)(i - (int64_t)r * snp);
        const uint32_t v = sshuf[flat_s(r, b, snp)];
        const bool live = r < rows && b < nb;
        bad_pad += (!live && pad >= 0 && v != (uint32_t)pad) ? 1u : 0u;
        nan_live += (live && v == 0xFFu) ? 1u : 0u;
    }
    for (int o = 32; o > 0; o >>= 1) {
        bad_pad += __shfl_xor(bad_pad, o);
        nan_live += __shfl_xor(nan_live, o);
    }
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        part[0][wv] = bad_pad;
        part[1][wv] = nan_live;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        uint32_t t = 0;
        for (int k = 0; k < 16; ++k) t += part[threadIdx.x][k];
        counts[threadIdx.x] = t;
    }
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
// The kernels read and write bf16 rows, packed bytes and fp32 output in
// 16-byte (packed codes of the quantizers: 4-byte) units.
bool misaligned(const void* p, uintptr_t a) { return p && reinterpret_cast<uintptr_t>(p) % a != 0; }
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
    if (misaligned(x, 16) || misaligned(packed, 4))
        return fmt_fail("x must be 16-byte and packed 4-byte aligned");
    if (K / 512 >= 65535) return fmt_fail("K too large for the quantizer grid");
    if (pad_byte < 0 || pad_byte > 255) return fmt_fail("pad_byte must be a byte");
    (void)hipGetLastError();
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int snp = scale_pad_of(K);
    // with a shuffled buffer the grid also spans its padding rows and blocks
    const int grid_rows = scale_shuffled ? ((rows + 31) & ~31) : rows;
    const int grid_chunks = scale_shuffled ? 4 * snp : K / 8;
    hipLaunchKernelGGL(quantize_bf16_kernel, dim3((grid_rows + 3) / 4, (grid_chunks + 63) / 64),
                       dim3(64, 4), 0, s, static_cast<const uint16_t*>(x), rows, K, packed,
                       scale_shuffled, scale_plain, snp, (uint8_t)pad_byte);
    return launched();
}

int mbs_quantize_mxfp4_mbs_bf16(const void* x, int rows, int K, uint8_t* packed,
                                uint8_t* scale_shuffled, uint8_t* scale_plain, uint8_t* factors,
                                int pad_byte, void* stream)
{
    if (!x || !packed || !factors) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    if (misaligned(x, 16) || misaligned(packed, 4))
        return fmt_fail("x must be 16-byte and packed 4-byte aligned");
    if (pad_byte < 0 || pad_byte > 255) return fmt_fail("pad_byte must be a byte");
    (void)hipGetLastError();
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int snp = scale_pad_of(K);
    const int grid = scale_shuffled ? ((rows + 31) & ~31) : rows;  // padding rows included
    const auto* xs = static_cast<const uint16_t*>(x);
    const uint8_t pb = (uint8_t)pad_byte;
    // Fewer rows than CUs: a row's latency is the kernel's time, so give each
    // row four times the threads.
    const bool wide = rows < kMbsWideRows;
    if (K <= kMbsStagedK) {
        if (wide)
            hipLaunchKernelGGL((quantize_mbs_bf16_kernel<true, 1024>), dim3(grid), dim3(1024), (size_t)K * 2,
                               s, xs, rows, K, packed, scale_shuffled, scale_plain, factors, snp, pb);
        else
            hipLaunchKernelGGL((quantize_mbs_bf16_kernel<true, 256>), dim3(grid), dim3(256), (size_t)K * 2,
                               s, xs, rows, K, packed, scale_shuffled, scale_plain, factors, snp, pb);
    } else if (wide) {
        hipLaunchKernelGGL((quantize_mbs_bf16_kernel<false, 1024>), dim3(grid), dim3(1024), 0, s, xs,
                           rows, K, packed, scale_shuffled, scale_plain, factors, snp, pb);
    } else {
        hipLaunchKernelGGL((quantize_mbs_bf16_kernel<false, 256>), dim3(grid), dim3(256), 0, s, xs,
                           rows, K, packed, scale_shuffled, scale_plain, factors, snp, pb);
    }
    return launched();
}

int mbs_shuffle_b(const uint8_t* w, uint8_t* out, int N, int K, void* stream)
{
    if (!w || !out) return fmt_fail("null pointer");
    if (N < 16 || N % 16 || K < 64 || K % 64) return fmt_fail("need N % 16 == 0 and K % 64 == 0");
    if (w == out) return fmt_fail("shuffle_b is out of place");
    if (misaligned(w, 16) || misaligned(out, 16)) return fmt_fail("w and out must be 16-byte aligned");
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

int mbs_unshuffle_b(const uint8_t* in, uint8_t* w, int N, int K, void* stream)
{
    if (!in || !w) return fmt_fail("null pointer");
    if (N < 16 || N % 16 || K < 64 || K % 64) return fmt_fail("need N % 16 == 0 and K % 64 == 0");
    if (in == w) return fmt_fail("unshuffle_b is out of place");
    if (misaligned(in, 16) || misaligned(w, 16)) return fmt_fail("in and w must be 16-byte aligned");
    (void)hipGetLastError();
    hipLaunchKernelGGL(unshuffle_b_kernel, dim3(blocks_for((int64_t)N * (K / 32))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), in, w, N, K / 2);
    return launched();
}

int mbs_unshuffle_scales(const uint8_t* shuffled, uint8_t* plain, int rows, int K, void* stream)
{
    if (!shuffled || !plain) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    (void)hipGetLastError();
    hipLaunchKernelGGL(unshuffle_scales_kernel, dim3(blocks_for((int64_t)rows * (K / 32))),
                       dim3(256), 0, static_cast<hipStream_t>(stream), shuffled, plain, rows,
                       K / 32, scale_pad_of(K));
    return launched();
}

int mbs_check_scales(const uint8_t* shuffled, int rows, int K, int pad_byte, uint32_t* counts,
                     void* stream)
{
    if (!shuffled || !counts) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    if (pad_byte < -1 || pad_byte > 255) return fmt_fail("pad_byte must be a byte or -1");
    (void)hipGetLastError();
    hipLaunchKernelGGL(check_scales_kernel, dim3(1), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), shuffled, rows, K / 32, scale_pad_of(K),
                       pad_byte, counts);
    return launched();
}

int mbs_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale_shuffled, float* out, int rows,
                      int K, int b_preshuffled, void* stream)
{
    if (!packed || !scale_shuffled || !out) return fmt_fail("null pointer");
    if (rows < 1 || K < 32 || K % 32) return fmt_fail("need rows >= 1 and K % 32 == 0");
    if (b_preshuffled && (rows % 16 || K % 64))
        return fmt_fail("preshuffled layout needs rows % 16 == 0 and K % 64 == 0");
    if (misaligned(packed, 16) || misaligned(out, 16))
        return fmt_fail("packed and out must be 16-byte aligned");
    (void)hipGetLastError();
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks_for((int64_t)rows * (K / 32))), dim3(256), 0,
                       static_cast<hipStream_t>(stream), packed, scale_shuffled, out, rows, K,
                       scale_pad_of(K), b_preshuffled);
    return launched();
}

}  // extern "C"
