// Device helpers shared by the gfx950 MXFP4 kernels: vector types, buffer
// resources, LDS DMA, the block-scaled fp4 MFMA, waits and barriers, the MBS
// factor table and bf16 packing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>

namespace mbs {

// Records the text mbs_last_error() returns (thread-local, host side).
void set_last_error(const char* msg);

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

#define MBS_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// Offset that is out of range for every buffer resource built here
// (num_records is always < 2^31): a load through it returns 0, a store is
// dropped.
constexpr uint32_t kOOB = 0x80000000u;

// ------------------------------------------------------- compile-time loops
template <int... Is, class F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F&& f)
{
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f)
{
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// ------------------------------------------------------- buffer resources
// Raw (stride 0) buffer over `bytes` bytes from `base`.  Word 3 = 0x00020000
// is the gfx9 raw-buffer format (32-bit data format, no swizzle); accesses at
// offsets >= bytes read as 0 / are discarded.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// 16-byte global->LDS DMA: lane i's 16 bytes at `voffset` land at
// lds + 16*i (M0 = lds).  soffset is kept 0 so the range check sees the whole
// offset.
__device__ __forceinline__ void dma16(rsrc_t r, void* lds, uint32_t voffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, MBS_LDS_PTR(lds), 16, voffset, 0, 0, 0);
}
// 4-byte global->LDS DMA: lane i's dword lands at lds + 4*i.
__device__ __forceinline__ void dma4(rsrc_t r, void* lds, uint32_t voffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, MBS_LDS_PTR(lds), 4, voffset, 0, 0, 0);
}

// Variants with a wave-uniform scalar offset: the range check covers
// voffset + soffset (checked on gfx950), so per-stage offsets and the
// out-of-range bit can live in an SGPR and cost no VALU work.
__device__ __forceinline__ void dma16s(rsrc_t r, void* lds, uint32_t voffset, uint32_t soffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, MBS_LDS_PTR(lds), 16, voffset, soffset, 0, 0);
}
__device__ __forceinline__ void dma4s(rsrc_t r, void* lds, uint32_t voffset, uint32_t soffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, MBS_LDS_PTR(lds), 4, voffset, soffset, 0, 0);
}
__device__ __forceinline__ i32x4 load16s(rsrc_t r, uint32_t voffset, uint32_t soffset)
{
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}
__device__ __forceinline__ int load4s(rsrc_t r, uint32_t voffset, uint32_t soffset)
{
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, 0);
}

__device__ __forceinline__ i32x4 load16(rsrc_t r, uint32_t voffset)
{
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0));
}
// Non-temporal 16-byte load (cache-policy bit 1, "nt" on gfx950): for data
// read exactly once, such as the weight stream of a decode GEMM.
__device__ __forceinline__ i32x4 load16nt(rsrc_t r, uint32_t voffset)
{
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 2));
}
__device__ __forceinline__ i32x2 load8(rsrc_t r, uint32_t voffset)
{
    return __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voffset, 0, 0));
}
__device__ __forceinline__ int load4(rsrc_t r, uint32_t voffset)
{
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, voffset, 0, 0);
}
__device__ __forceinline__ uint32_t load1(rsrc_t r, uint32_t voffset)
{
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, voffset, 0, 0);
}
__device__ __forceinline__ void store8(rsrc_t r, uint32_t voffset, uint32_t lo, uint32_t hi)
{
    i32x2 v = {(int)lo, (int)hi};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned, v), r, voffset, 0, 0);
}
__device__ __forceinline__ void store16(rsrc_t r, uint32_t voffset, f32x4 v)
{
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), r, voffset, 0, 0);
}
__device__ __forceinline__ f32x4 loadf4(rsrc_t r, uint32_t voffset)
{
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0));
}

// ---------------------------------------------------------- waits/barrier
// s_waitcnt vmcnt(n), leaving expcnt/lgkmcnt unconstrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0()
{
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));
}

// LDS reads written as instructions, for loops that schedule and wait for
// their LDS traffic themselves (s_waitcnt lgkmcnt counted by the caller):
// the compiler does not see them as memory accesses, so it neither waits
// for them nor makes them wait for LDS DMA it cannot prove disjoint.
// `addr` is an LDS byte address, OFF a compile-time offset (< 65536).
template <int OFF>
__device__ __forceinline__ i32x4 ds_read16(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    i32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ int ds_read4(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
    int v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
// s_waitcnt lgkmcnt(N) that also "rewrites" `reg`, so every later use of
// reg (an MFMA operand) is ordered after the wait.
template <int N, class R>
__device__ __forceinline__ void wait_lgkm_for(R& reg)
{
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(reg) : "n"(N));
}
// Orders later uses of `reg` after the preceding volatile asm (no code).
template <class R>
__device__ __forceinline__ void tie_after(R& reg)
{
    asm volatile("" : "+v"(reg));
}
// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Workgroup barrier with no implied memory fence (the fence of
// __syncthreads would force vmcnt(0) and drain the LDS DMA prefetch).  The
// "memory" clobber keeps the compiler from moving LDS accesses across it;
// callers wait on their own DMA (wait_vmcnt) before arriving.
__device__ __forceinline__ void barrier()
{
    asm volatile("s_barrier" ::: "memory");
}

// -------------------------------------------------------------- fp4 MFMA
// acc(16x16, fp32) += A(16x128 e2m1) * B(128x16 e2m1), block-scaled, with
// v_mfma_scale_f32_16x16x128_f8f6f4 (cbsz = blgp = 4: both operands fp4).
// Operand layout (both operands): lane L holds row/col (L % 16) and the
// 32-element K-block (L / 16) as 16 bytes (32 nibbles, low nibble first).
// Scale: lane L's E8M0 byte for that same (row, K-block); OPA/OPB (0..3) pick
// the byte of the 32-bit scale register (op_sel bit 0 / op_sel_hi bit 1).
// Output: acc[t] on lane L is D[(L / 16) * 4 + t][L % 16].
//
// Written as inline asm with the accumulator tied to an AGPR ("+a") so every
// MFMA accumulates in place: with the builtin the register allocator renames
// accumulators across the unrolled K loop and emits a v_accvgpr copy per MFMA.
// Because the compiler's hazard recognizer cannot see into the asm, an MFMA
// whose operands may come from a VALU instruction starts with s_nop 1: the two
// wait states gfx9 needs between a VALU write of a VGPR and an MFMA reading it.
// NOP = false is for loops where every operand comes straight from a buffer or
// LDS load (waited for with s_waitcnt), so no VALU write precedes the MFMA.
// Reading the accumulators after the last MFMA needs the wait of mfma_drain().
// First MFMA of an accumulation: C = 0 (inline constant), so the
// accumulator needs no zeroing and is only written.
template <int OPA, int OPB>
__device__ __forceinline__ void mfma_fp4_first(f32x4& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(OPA >= 0 && OPA < 4 && OPB >= 0 && OPB < 4, "op_sel byte index");
    asm("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel:[%5,%6,0] "
        "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
        : "=a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
          "n"(OPB >> 1));
}

template <int OPA, int OPB, bool NOP = true>
__device__ __forceinline__ void mfma_fp4(f32x4& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(OPA >= 0 && OPA < 4 && OPB >= 0 && OPB < 4, "op_sel byte index");
    if constexpr (NOP) {
        asm("s_nop 1\n\t"
            "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[%5,%6,0] "
            "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
            : "+a"(acc)
            : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
              "n"(OPB >> 1));
    } else {
        asm("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[%5,%6,0] "
            "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
            : "+a"(acc)
            : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
              "n"(OPB >> 1));
    }
}

// The same MFMAs preceded, in the same asm statement, by s_waitcnt
// lgkmcnt(W): for operands read from LDS with explicit ds_read instructions,
// whose completion the caller counts.  Keeping the wait inside the statement
// orders it before the MFMA without a fake register definition (which would
// make the compiler add wait states of its own); `volatile` keeps the
// statement in order with the ds_read statements it counts.
template <int OPA, int OPB, int W>
__device__ __forceinline__ void mfma_fp4_first_w(f32x4& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(W >= 0 && W < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%9)\n\t"
        "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel:[%5,%6,0] "
        "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
        : "=a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
          "n"(OPB >> 1), "n"(W));
}
template <int OPA, int OPB, int W, bool NOP>
__device__ __forceinline__ void mfma_fp4_w(f32x4& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(W >= 0 && W < 16, "lgkmcnt range");
    if constexpr (NOP) {
        asm volatile("s_waitcnt lgkmcnt(%9)\n\ts_nop 1\n\t"
            "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[%5,%6,0] "
            "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
            : "+a"(acc)
            : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
              "n"(OPB >> 1), "n"(W));
    } else {
        asm volatile("s_waitcnt lgkmcnt(%9)\n\t"
            "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[%5,%6,0] "
            "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
            : "+a"(acc)
            : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
              "n"(OPB >> 1), "n"(W));
    }
}

// The 32x32x64 form, v_mfma_scale_f32_32x32x64_f8f6f4 (fp4 A and B): lane L
// supplies row L%32 of its operand with K elements 32*(L/32)..+31 (16
// bytes) and the E8M0 scale of (row L%32, 32-K block L/32); acc[r] of lane
// L is D[8*(r/4) + 4*(L/32) + r%4][L%32] (D = src0 x src1^T, 32 x 32 fp32).
// OPA / OPB select the scale byte, as for the 16x16x128 form.  These
// operands only come from loads, LDS reads and (scales) a v_perm that an
// explicit s_nop separates from the first MFMA, so no wait states are
// added here.
template <int OPA, int OPB>
__device__ __forceinline__ void mfma32_fp4_first(f32x16& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(OPA >= 0 && OPA < 4 && OPB >= 0 && OPB < 4, "op_sel byte index");
    asm("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel:[%5,%6,0] "
        "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
        : "=a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
          "n"(OPB >> 1));
}
template <int OPA, int OPB>
__device__ __forceinline__ void mfma32_fp4(f32x16& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(OPA >= 0 && OPA < 4 && OPB >= 0 && OPB < 4, "op_sel byte index");
    asm("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[%5,%6,0] "
        "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
        : "+a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
          "n"(OPB >> 1));
}
template <int OPA, int OPB, int W>
__device__ __forceinline__ void mfma32_fp4_first_w(f32x16& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(W >= 0 && W < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%9)\n\t"
        "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, 0, %3, %4 op_sel:[%5,%6,0] "
        "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
        : "=a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
          "n"(OPB >> 1), "n"(W));
}
template <int OPA, int OPB, int W>
__device__ __forceinline__ void mfma32_fp4_w(f32x16& acc, i32x4 a, i32x4 b, int sa, int sb)
{
    static_assert(W >= 0 && W < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%9)\n\t"
        "v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[%5,%6,0] "
        "op_sel_hi:[%7,%8,0] cbsz:4 blgp:4"
        : "+a"(acc)
        : "v"(a), "v"(b), "v"(sa), "v"(sb), "n"(OPA & 1), "n"(OPB & 1), "n"(OPA >> 1),
          "n"(OPB >> 1), "n"(W));
}

// Wait states between the last MFMA writing an accumulator and any other
// instruction reading it (gfx9 requires up to ~19 for a 16-pass XDL op).
__device__ __forceinline__ void mfma_drain()
{
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

// Orders every later read of `acc` after an mfma_drain(): the empty asm
// "rewrites" the accumulator, so the AGPR->VGPR copies the compiler makes
// for its readers depend on it, and volatile asm statements keep their
// relative order.  Without it the scheduler may hoist those copies above
// the drain (it cannot see the latency of an MFMA written as inline asm)
// and read an accumulator an MFMA is still writing.
__device__ __forceinline__ void pin_after_drain(f32x4& acc)
{
    asm volatile("" : "+a"(acc));
}
__device__ __forceinline__ void pin_after_drain(f32x16& acc)
{
    asm volatile("" : "+a"(acc));
}

// ----------------------------------------------------------- MBS factor
// f(b) = 1/(1+b/256) = 256/(256+b), correctly rounded to fp32, computed at
// compile time with integer long division (no run-time division needed).
constexpr uint32_t mbs_factor_bits(int b)
{
    if (b == 0) return 0x3F800000u;
    const uint64_t d = 256u + (uint64_t)b;
    const uint64_t num = 1ull << 32;  // 256 * 2^24: the quotient is the
    uint64_t q = num / d;             // significand of a value in (0.5, 1)
    const uint64_t r = num % d;
    if (2 * r > d || (2 * r == d && (q & 1))) ++q;
    return (126u << 23) | (uint32_t)(q - (1u << 23));
}
struct FactorTable {
    uint32_t bits[256];
    constexpr FactorTable() : bits{}
    {
        for (int b = 0; b < 256; ++b) bits[b] = mbs_factor_bits(b);
    }
};

// ------------------------------------------------------------ bf16 pack
// x + y rounded on its own: never fused with the product that feeds it
// (the epilogue bias add has a defined fp32 order: multiply, round, add).
__device__ __forceinline__ float add_nc(float x, float y)
{
#pragma clang fp contract(off)
    return x + y;
}
// bf16 bits (low or high half of a dword) -> fp32, exactly.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}


// ---- MXFP4 block quantization (BASELINE configs[0] rule) ------------------
// floor(log2(a)) of a finite a > 0 given its fp32 bits (subnormals included).
__device__ __forceinline__ int floor_log2_bits(uint32_t u)
{
    const int e = (int)((u >> 23) & 0xFF);
    // (| 1 keeps clz defined for u == 0, whose result callers discard)
    const int sub = (31 - __builtin_clz((u & 0x7FFFFFu) | 1u)) - 149;
    return e != 0 ? e - 127 : sub;
}

// E8M0 scale of a block from its largest magnitude (fp32 bits, already times
// the row multiplier m) and its NaN flag: floor(log2(amax)) - 2, biased by
// 127 and clamped to [0, 254]; 0 for an all-zero block, 254 for an infinite
// maximum, 255 (NaN) when the block holds a NaN.
// (Selects, not early returns: the compiler keeps them branch-free.)
__device__ __forceinline__ uint32_t e8m0_of(uint32_t amax_m, bool nan)
{
    const int e = floor_log2_bits(amax_m) - 2 + 127;
    uint32_t s = (uint32_t)(e < 0 ? 0 : (e > 254 ? 254 : e));
    s = amax_m >= 0x7F800000u ? 254u : s;
    s = amax_m == 0 ? 0u : s;
    return nan ? 255u : s;
}

// 2^(s - 127) for s in [0, 254] as fp32: exponent field s, or the subnormal
// 2^-127 for s == 0.
__device__ __forceinline__ float e8m0_value(uint32_t s)
{
    return s == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(s << 23);
}

// Largest 15-bit magnitude (bf16 bits without the sign) of eight bf16 values
// (16 bytes); a NaN orders above inf.
__device__ __forceinline__ uint32_t bf16x8_absmax(const i32x4 v)
{
    uint32_t mx = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = (uint32_t)v[i] & 0x7FFF7FFFu;
        mx = max(mx, max(w & 0xFFFFu, w >> 16));
    }
    return mx;
}

// The same maximum over a whole 32-element block (four 16-byte pieces),
// on both 16-bit halves at once (v_pk_max_u16), folded at the end.
__device__ __forceinline__ uint32_t bf16x32_absmax(const i32x4 x[4])
{
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m = {0, 0};
    for (int i = 0; i < 4; ++i) {
        const i32x4 v = x[i];
        for (int j = 0; j < 4; ++j) {
            const uint32_t w = (uint32_t)v[j] & 0x7FFF7FFFu;
            m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w));
        }
    }
    return max((uint32_t)m[0], (uint32_t)m[1]);
}

// Eight bf16 values -> one dword of packed e2m1 (element 2j in the low
// nibble of byte j) under the block scale `sc`, with the gfx950 scaled
// conversion v_cvt_scalef32_pk_fp4_bf16: code = RNE(v / sc) on the e2m1
// grid, ties to the even code, saturating at 6, sign kept.  (Each word is
// copied to a scalar first: hipcc's __builtin_bit_cast of a vector element
// v[i] reads element 0.)
__device__ __forceinline__ uint32_t bf16x8_to_e2m1(const i32x4 v, float sc)
{
    const uint32_t w0 = (uint32_t)v[0], w1 = (uint32_t)v[1], w2 = (uint32_t)v[2], w3 = (uint32_t)v[3];
    // Each conversion writes one byte and keeps the other three; all four
    // bytes are written below, so the starting value is w0 (dead after the
    // first conversion) rather than a zero that costs a move.
    uint32_t o = w0;
    o = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(o, __builtin_bit_cast(bf16x2_t, w0), sc, 0);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(o, __builtin_bit_cast(bf16x2_t, w1), sc, 1);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(o, __builtin_bit_cast(bf16x2_t, w2), sc, 2);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(o, __builtin_bit_cast(bf16x2_t, w3), sc, 3);
    return o;
}

// One whole 32-element MXFP4 block in one lane: x[i] holds elements
// 8i..8i+7 (bf16); returns the 16 packed bytes (dword i = elements 8i..8i+7)
// and sets *s to the block's E8M0 byte.  Same rule and bytes as the
// four-lanes-per-block quantizer kernel: a block holding a NaN gets scale
// 255 and zero codes.
__device__ __forceinline__ i32x4 quantize_block32(const i32x4 x[4], uint32_t* s)
{
    const uint32_t mx = bf16x32_absmax(x);
    const bool nan = mx > 0x7F80u;
    *s = e8m0_of(mx << 16, nan);
    const float sc = e8m0_value(nan ? 127 : *s);
    // The four dwords' conversion chains are interleaved (each chain writes
    // one register byte by byte), and a NaN block is cleared with a mask:
    // written as a select, the compiler branches around the conversions.
    const uint32_t keep = nan ? 0u : ~0u;
    uint32_t w[4][4], o[4];
    for (int i = 0; i < 4; ++i) {
        const i32x4 v = x[i];
        w[i][0] = (uint32_t)v[0]; w[i][1] = (uint32_t)v[1];
        w[i][2] = (uint32_t)v[2]; w[i][3] = (uint32_t)v[3];
        o[i] = w[i][0];   // every byte is overwritten
    }
    static_for<4>([&](auto j) {
        constexpr int J = decltype(j)::value;
        for (int i = 0; i < 4; ++i)
            o[i] = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(o[i], __builtin_bit_cast(bf16x2_t, w[i][J]), sc, J);
    });
    i32x4 q;
    q[0] = (int)(o[0] & keep); q[1] = (int)(o[1] & keep);
    q[2] = (int)(o[2] & keep); q[3] = (int)(o[3] & keep);
    return q;
}

// One whole block of an MBS-scaled row in one lane: the block's elements
// times the row multiplier m = 1 + b/256 (fp32 products), quantized with the
// rule and conversion of the MBS quantizer kernel (block maximum of the bf16
// magnitudes times m for the scale, v_cvt_scalef32_pk_fp4_f32 of the scaled
// values); a block holding a NaN gets scale 255 and zero codes.
__device__ __forceinline__ i32x4 quantize_block32_mbs(const i32x4 x[4], float m, uint32_t* s)
{
    const uint32_t mx = bf16x32_absmax(x);
    const bool nan = mx > 0x7F80u;
    *s = e8m0_of(__float_as_uint(__uint_as_float(mx << 16) * m), nan);
    const float sc = e8m0_value(nan ? 127 : *s);
    const uint32_t keep = nan ? 0u : ~0u;
    i32x4 q;
    for (int i = 0; i < 4; ++i) {
        const i32x4 v = x[i];
        const uint32_t w[4] = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
        uint32_t o = w[0];   // every byte is overwritten
        static_for<4>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const float lo = __uint_as_float(w[j] << 16) * m;
            const float hi = __uint_as_float(w[j] & 0xFFFF0000u) * m;
            o = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(o, lo, hi, sc, j);
        });
        q[i] = (int)(o & keep);
    }
    return q;
}

// MBS factor byte of a row from its largest bf16 magnitude (15 bits): the top
// 8 mantissa bits of 6/max (IEEE division, then truncation); 0 for a zero,
// infinite or NaN maximum.  The row is quantized times 1 + b/256.
__device__ __forceinline__ uint32_t mbs_factor_byte(uint32_t amax)
{
    if (amax == 0 || amax >= 0x7F80) return 0;
    return (__float_as_uint(__fdiv_rn(6.0f, __uint_as_float(amax << 16))) >> 15) & 0xFF;
}

}  // namespace mbs
