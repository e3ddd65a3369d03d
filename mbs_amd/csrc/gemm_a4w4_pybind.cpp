// Torch-facing module `mbs_gemm_a4w4`: the drop-in for the reference's
// pybind entry (interface/gemm_a4w4_pybind.cpp:19-74 of the reference).
//
// gemm_a4w4(A, B, A_scale, B_scale, A_factor=None, B_factor=None) validates
// the operands, allocates the [Mpad, N] bf16 output (and any split-K
// workspace) through torch's caching allocator, and launches on the current
// HIP stream through the C ABI of libmbs_gemm_kernel.so.  It returns the
// [M, N] view of the padded output, as the reference does.  The factors are
// optional here (the reference requires them, which makes its own
// bench_one.py 4-argument call fail); omitting them means "no scaling".
//
// The format helpers (quantize, preshuffle, dequantize) are exported too, so
// a caller needs nothing beyond this module to prepare operands.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <string>

#include "mbs_gemm_a4w4.h"

namespace {

void* current_stream(const at::Tensor& t)
{
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_status(int st, const char* what)
{
    TORCH_CHECK(st == MBS_OK, what, ": ", mbs_status_string(st), " (", mbs_last_error(), ")");
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
int64_t scale_pad(int64_t K) { return round_up((K + 31) / 32, 8); }

// A contiguous byte view of t.  The kernels need 16-byte aligned operands
// (4-byte for the factor bytes); a view starting elsewhere in its storage is
// copied into a fresh (aligned) allocation instead of being refused.
at::Tensor as_bytes(const at::Tensor& t, uintptr_t align = 16)
{
    at::Tensor b = t.view(at::kByte).contiguous();
    if (reinterpret_cast<uintptr_t>(b.data_ptr()) % align) b = b.clone();
    return b;
}
at::Tensor aligned_contiguous(const at::Tensor& t)
{
    at::Tensor c = t.contiguous();
    if (reinterpret_cast<uintptr_t>(c.data_ptr()) % 16) c = c.clone();
    return c;
}

struct Operands {
    at::Tensor A, B, As, Bs, Af, Bf;
    int M = 0, N = 0, K = 0, Mpad = 0, snp = 0;
    bool factors = false;
};

Operands prepare(const at::Tensor& A, const at::Tensor& B, const at::Tensor& A_scale,
                 const at::Tensor& B_scale, const c10::optional<at::Tensor>& A_factor,
                 const c10::optional<at::Tensor>& B_factor)
{
    TORCH_CHECK(A.is_cuda() && B.is_cuda(), "gemm_a4w4: A, B must be on device");
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2, "gemm_a4w4: A, B must be 2D");
    TORCH_CHECK(A_scale.is_cuda() && B_scale.is_cuda(), "gemm_a4w4: scales must be on device");
    TORCH_CHECK(A.element_size() == 1 && B.element_size() == 1 && A_scale.element_size() == 1 &&
                    B_scale.element_size() == 1,
                "gemm_a4w4: A, B and the scales must have a 1-byte dtype");
    const auto dev = A.device();
    TORCH_CHECK(B.device() == dev && A_scale.device() == dev && B_scale.device() == dev,
                "gemm_a4w4: all operands must be on the same device");
    Operands o;
    o.A = as_bytes(A);
    o.B = as_bytes(B);
    o.As = as_bytes(A_scale);
    o.Bs = as_bytes(B_scale);
    o.M = (int)o.A.size(0);
    const int64_t Kp = o.A.size(1);
    o.K = (int)(Kp * 2);
    o.N = (int)o.B.size(0);
    TORCH_CHECK(o.B.size(1) == Kp, "gemm_a4w4: A, B must share K/2, got ", o.A.size(1), " vs ",
                o.B.size(1));
    TORCH_CHECK(o.K % 32 == 0, "gemm_a4w4: K must be a multiple of 32, got ", o.K);
    TORCH_CHECK(o.K % 64 == 0, "gemm_a4w4: K must be a multiple of 64 (the (16,16) B preshuffle "
                "groups 32 bytes of K), got ", o.K);
    TORCH_CHECK(o.N % 16 == 0, "gemm_a4w4: N must be a multiple of 16, got ", o.N);
    o.Mpad = (int)round_up(o.M, 32);
    o.snp = (int)scale_pad(o.K);
    TORCH_CHECK(o.As.numel() >= (int64_t)o.Mpad * o.snp, "gemm_a4w4: A_scale must hold at least ",
                (int64_t)o.Mpad * o.snp, " bytes (round_up(M,32) * scaleN_pad), got ",
                o.As.numel());
    TORCH_CHECK(o.Bs.numel() >= round_up(o.N, 32) * o.snp, "gemm_a4w4: B_scale must hold at least ",
                round_up(o.N, 32) * o.snp, " bytes (round_up(N,32) * scaleN_pad), got ",
                o.Bs.numel());
    const bool has_a = A_factor.has_value() && A_factor->defined();
    const bool has_b = B_factor.has_value() && B_factor->defined();
    TORCH_CHECK(has_a == has_b, "gemm_a4w4: A_factor and B_factor must be given together");
    o.factors = has_a;
    if (o.factors) {
        o.Af = as_bytes(*A_factor, 4);
        o.Bf = as_bytes(*B_factor, 4);
        TORCH_CHECK(o.Af.is_cuda() && o.Af.numel() == o.M, "gemm_a4w4: A_factor must hold M = ",
                    o.M, " bytes on device, got ", o.Af.numel());
        TORCH_CHECK(o.Bf.is_cuda() && o.Bf.numel() == o.N, "gemm_a4w4: B_factor must hold N = ",
                    o.N, " bytes on device, got ", o.Bf.numel());
        TORCH_CHECK(o.Af.device() == dev && o.Bf.device() == dev,
                    "gemm_a4w4: factors must be on the operands' device");
    }
    return o;
}

at::Tensor run(const Operands& o, int config, int splits, double alpha = 1.0,
               const c10::optional<at::Tensor>& bias = c10::nullopt)
{
    c10::DeviceGuard guard(o.A.device());
    auto out = torch::empty({o.Mpad, o.N},
                            torch::TensorOptions().dtype(torch::kBFloat16).device(o.A.device()));
    const size_t ws = config < 0 ? mbs_gemm_a4w4_workspace_bytes(o.M, o.N, o.K)
                                 : mbs_gemm_a4w4_config_workspace_bytes(config, splits, o.M, o.N, o.K);
    at::Tensor wst;
    if (ws) wst = torch::empty({(int64_t)ws}, torch::TensorOptions().dtype(torch::kByte).device(o.A.device()));
    const uint8_t* af = o.factors ? o.Af.data_ptr<uint8_t>() : nullptr;
    const uint8_t* bf = o.factors ? o.Bf.data_ptr<uint8_t>() : nullptr;
    void* s = current_stream(o.A);
    int st;
    at::Tensor bu;
    if (bias.has_value()) {
        TORCH_CHECK(bias->is_cuda() && bias->device() == o.A.device() &&
                        bias->scalar_type() == at::kBFloat16 && bias->numel() == o.N,
                    "gemm_a4w4: bias must be a bf16 device tensor of N entries");
        bu = aligned_contiguous(*bias);
    }
    if (alpha != 1.0 || bu.defined())
        st = mbs_gemm_a4w4_launch_ex(config, splits, o.A.data_ptr<uint8_t>(),
                                     o.B.data_ptr<uint8_t>(), o.As.data_ptr<uint8_t>(),
                                     o.Bs.data_ptr<uint8_t>(), af, bf, out.data_ptr(), o.M, o.N,
                                     o.K, o.Mpad, o.snp, (float)alpha,
                                     bu.defined() ? bu.data_ptr() : nullptr,
                                     ws ? wst.data_ptr() : nullptr, ws, s);
    else if (config < 0)
        st = mbs_gemm_a4w4_launch(o.A.data_ptr<uint8_t>(), o.B.data_ptr<uint8_t>(),
                                  o.As.data_ptr<uint8_t>(), o.Bs.data_ptr<uint8_t>(), af, bf,
                                  out.data_ptr(), o.M, o.N, o.K, o.Mpad, o.snp,
                                  ws ? wst.data_ptr() : nullptr, ws, s);
    else
        st = mbs_gemm_a4w4_launch_config(config, splits, o.A.data_ptr<uint8_t>(),
                                         o.B.data_ptr<uint8_t>(), o.As.data_ptr<uint8_t>(),
                                         o.Bs.data_ptr<uint8_t>(), af, bf, out.data_ptr(), o.M,
                                         o.N, o.K, o.Mpad, o.snp, ws ? wst.data_ptr() : nullptr,
                                         ws, s);
    check_status(st, "gemm_a4w4");
    return out.narrow(0, 0, o.M);
}

}  // namespace

// The reference's operator (interface/gemm_a4w4_pybind.cpp:19-64).
at::Tensor gemm_a4w4(at::Tensor A, at::Tensor B, at::Tensor A_scale, at::Tensor B_scale,
                     c10::optional<at::Tensor> A_factor, c10::optional<at::Tensor> B_factor,
                     double alpha, c10::optional<at::Tensor> bias)
{
    return run(prepare(A, B, A_scale, B_scale, A_factor, B_factor), -1, 0, alpha, bias);
}

// Same operator with a forced kernel configuration (tests, tuning).
at::Tensor gemm_a4w4_config(int64_t config, int64_t splits, at::Tensor A, at::Tensor B,
                            at::Tensor A_scale, at::Tensor B_scale,
                            c10::optional<at::Tensor> A_factor,
                            c10::optional<at::Tensor> B_factor, double alpha,
                            c10::optional<at::Tensor> bias)
{
    TORCH_CHECK(config >= 0 && config < mbs_gemm_a4w4_num_configs(), "gemm_a4w4_config: config ",
                config, " out of range [0, ", mbs_gemm_a4w4_num_configs(), ")");
    return run(prepare(A, B, A_scale, B_scale, A_factor, B_factor), (int)config, (int)splits,
               alpha, bias);
}

// bf16 [R, K] -> (packed u8 [R, K/2], scales).  shuffle=True returns the
// shuffled scale buffer viewed as [round_up(R,32), scaleN_pad]; False returns
// plain [R, K/32] scales (the two quantizer modes of test_gemm_a4w4.py:137-140).
std::tuple<at::Tensor, at::Tensor> quantize_mxfp4(at::Tensor x, bool shuffle, int64_t pad_byte)
{
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.scalar_type() == at::kBFloat16,
                "quantize_mxfp4: x must be a 2D bf16 device tensor");
    auto xc = aligned_contiguous(x);
    const int64_t R = xc.size(0), K = xc.size(1);
    TORCH_CHECK(K % 32 == 0, "quantize_mxfp4: K must be a multiple of 32");
    c10::DeviceGuard guard(x.device());
    auto opts = torch::TensorOptions().dtype(torch::kByte).device(x.device());
    auto packed = torch::empty({R, K / 2}, opts);
    at::Tensor scales = shuffle ? torch::empty({round_up(R, 32), scale_pad(K)}, opts)
                                : torch::empty({R, K / 32}, opts);
    check_status(mbs_quantize_mxfp4_bf16(xc.data_ptr(), (int)R, (int)K, packed.data_ptr<uint8_t>(),
                                         shuffle ? scales.data_ptr<uint8_t>() : nullptr,
                                         shuffle ? nullptr : scales.data_ptr<uint8_t>(),
                                         (int)pad_byte, current_stream(x)),
                 "quantize_mxfp4");
    return {packed, scales};
}

// MBS quantization: (packed, scales, factor bytes [R]) -- rows scaled by
// their MBS multipliers before quantization; pass the factors to gemm_a4w4.
std::tuple<at::Tensor, at::Tensor, at::Tensor> quantize_mxfp4_mbs(at::Tensor x, bool shuffle,
                                                                  int64_t pad_byte)
{
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.scalar_type() == at::kBFloat16,
                "quantize_mxfp4_mbs: x must be a 2D bf16 device tensor");
    auto xc = aligned_contiguous(x);
    const int64_t R = xc.size(0), K = xc.size(1);
    TORCH_CHECK(K % 32 == 0, "quantize_mxfp4_mbs: K must be a multiple of 32");
    c10::DeviceGuard guard(x.device());
    auto opts = torch::TensorOptions().dtype(torch::kByte).device(x.device());
    auto packed = torch::empty({R, K / 2}, opts);
    at::Tensor scales = shuffle ? torch::empty({round_up(R, 32), scale_pad(K)}, opts)
                                : torch::empty({R, K / 32}, opts);
    auto factors = torch::empty({R}, opts);
    check_status(mbs_quantize_mxfp4_mbs_bf16(
                     xc.data_ptr(), (int)R, (int)K, packed.data_ptr<uint8_t>(),
                     shuffle ? scales.data_ptr<uint8_t>() : nullptr,
                     shuffle ? nullptr : scales.data_ptr<uint8_t>(), factors.data_ptr<uint8_t>(),
                     (int)pad_byte, current_stream(x)),
                 "quantize_mxfp4_mbs");
    return {packed, scales, factors};
}

// Plain packed weights [N, K/2] -> (16,16)-preshuffled copy (shuffle_weight).
at::Tensor shuffle_weight(at::Tensor w)
{
    TORCH_CHECK(w.is_cuda() && w.dim() == 2 && w.element_size() == 1,
                "shuffle_weight: w must be a 2D 1-byte device tensor");
    auto wu = as_bytes(w);
    c10::DeviceGuard guard(w.device());
    auto out = torch::empty_like(wu);
    check_status(mbs_shuffle_b(wu.data_ptr<uint8_t>(), out.data_ptr<uint8_t>(), (int)wu.size(0),
                               (int)(wu.size(1) * 2), current_stream(w)),
                 "shuffle_weight");
    return out;
}

// Plain E8M0 [R, K/32] -> shuffled [round_up(R,32), scaleN_pad].
at::Tensor shuffle_scales(at::Tensor s, int64_t pad_byte)
{
    TORCH_CHECK(s.is_cuda() && s.dim() == 2 && s.element_size() == 1,
                "shuffle_scales: s must be a 2D 1-byte device tensor");
    auto su = as_bytes(s);
    const int64_t R = su.size(0), K = su.size(1) * 32;
    c10::DeviceGuard guard(s.device());
    auto out = torch::empty({round_up(R, 32), scale_pad(K)},
                            torch::TensorOptions().dtype(torch::kByte).device(s.device()));
    check_status(mbs_shuffle_scales(su.data_ptr<uint8_t>(), out.data_ptr<uint8_t>(), (int)R, (int)K,
                                    (int)pad_byte, current_stream(s)),
                 "shuffle_scales");
    return out;
}

// (16,16)-preshuffled weights [N, K/2] -> plain copy (inverse of shuffle_weight).
at::Tensor unshuffle_weight(at::Tensor b)
{
    TORCH_CHECK(b.is_cuda() && b.dim() == 2 && b.element_size() == 1,
                "unshuffle_weight: b must be a 2D 1-byte device tensor");
    auto bu = as_bytes(b);
    c10::DeviceGuard guard(b.device());
    auto out = torch::empty_like(bu);
    check_status(mbs_unshuffle_b(bu.data_ptr<uint8_t>(), out.data_ptr<uint8_t>(), (int)bu.size(0),
                                 (int)(bu.size(1) * 2), current_stream(b)),
                 "unshuffle_weight");
    return out;
}

// Shuffled E8M0 buffer of `rows` rows -> plain [rows, K/32] (inverse of shuffle_scales).
at::Tensor unshuffle_scales(at::Tensor s, int64_t rows, int64_t K)
{
    TORCH_CHECK(s.is_cuda() && s.element_size() == 1,
                "unshuffle_scales: s must be a 1-byte device tensor");
    TORCH_CHECK(rows >= 1 && K >= 32 && K % 32 == 0, "unshuffle_scales: need rows >= 1, K % 32 == 0");
    auto su = as_bytes(s);
    TORCH_CHECK(su.numel() >= round_up(rows, 32) * scale_pad(K), "unshuffle_scales: buffer too small");
    c10::DeviceGuard guard(s.device());
    auto out = torch::empty({rows, K / 32}, torch::TensorOptions().dtype(torch::kByte).device(s.device()));
    check_status(mbs_unshuffle_scales(su.data_ptr<uint8_t>(), out.data_ptr<uint8_t>(), (int)rows,
                                      (int)K, current_stream(s)),
                 "unshuffle_scales");
    return out;
}

// Format check of a shuffled scale buffer: (padding entries != pad_byte,
// live entries equal to 0xFF).  pad_byte = -1 skips the padding check.
// Synchronises the stream (load-time validation, not the hot path).
std::tuple<int64_t, int64_t> check_scales(at::Tensor s, int64_t rows, int64_t K, int64_t pad_byte)
{
    TORCH_CHECK(s.is_cuda() && s.element_size() == 1,
                "check_scales: s must be a 1-byte device tensor");
    TORCH_CHECK(rows >= 1 && K >= 32 && K % 32 == 0, "check_scales: need rows >= 1, K % 32 == 0");
    auto su = as_bytes(s);
    TORCH_CHECK(su.numel() >= round_up(rows, 32) * scale_pad(K), "check_scales: buffer too small");
    c10::DeviceGuard guard(s.device());
    auto counts = torch::empty({2}, torch::TensorOptions().dtype(torch::kInt32).device(s.device()));
    check_status(mbs_check_scales(su.data_ptr<uint8_t>(), (int)rows, (int)K, (int)pad_byte,
                                  reinterpret_cast<uint32_t*>(counts.data_ptr<int32_t>()),
                                  current_stream(s)),
                 "check_scales");
    auto h = counts.cpu();
    return {(int64_t)(uint32_t)h[0].item<int32_t>(), (int64_t)(uint32_t)h[1].item<int32_t>()};
}

// Packed operand + shuffled scales -> fp32 [R, K] (mxfp4_to_f32 * e8m0_to_f32).
at::Tensor dequant_mxfp4(at::Tensor packed, at::Tensor scale_shuffled, bool b_preshuffled)
{
    TORCH_CHECK(packed.is_cuda() && packed.dim() == 2 && packed.element_size() == 1,
                "dequant_mxfp4: packed must be a 2D 1-byte device tensor");
    TORCH_CHECK(scale_shuffled.is_cuda() && scale_shuffled.element_size() == 1,
                "dequant_mxfp4: scales must be a 1-byte device tensor");
    auto pu = as_bytes(packed);
    auto su = as_bytes(scale_shuffled);
    const int64_t R = pu.size(0), K = pu.size(1) * 2;
    TORCH_CHECK(su.numel() >= round_up(R, 32) * scale_pad(K), "dequant_mxfp4: scale buffer too small");
    c10::DeviceGuard guard(packed.device());
    auto out = torch::empty({R, K}, torch::TensorOptions().dtype(torch::kFloat32).device(packed.device()));
    check_status(mbs_dequant_mxfp4(pu.data_ptr<uint8_t>(), su.data_ptr<uint8_t>(),
                                   out.data_ptr<float>(), (int)R, (int)K, b_preshuffled ? 1 : 0,
                                   current_stream(packed)),
                 "dequant_mxfp4");
    return out;
}

// (non-empty experts starting off a 32-row boundary, clamped offsets) of a
// device offset vector of E+1 entries (mbs_gemm_a4w4_check_groups;
// synchronises the stream).
std::tuple<int64_t, int64_t> check_groups(at::Tensor group_offsets, int64_t M)
{
    TORCH_CHECK(group_offsets.is_cuda() && group_offsets.dim() == 1 && group_offsets.numel() >= 2 &&
                    group_offsets.scalar_type() == at::kInt,
                "check_groups: group_offsets must be an int32 device vector of E+1 entries");
    auto g = aligned_contiguous(group_offsets);
    c10::DeviceGuard guard(g.device());
    auto st = torch::empty({2}, torch::TensorOptions().dtype(torch::kInt32).device(g.device()));
    check_status(mbs_gemm_a4w4_check_groups(g.data_ptr<int32_t>(), (int)(g.numel() - 1), (int)M,
                                            reinterpret_cast<uint32_t*>(st.data_ptr<int32_t>()),
                                            current_stream(g)),
                 "check_groups");
    auto h = st.cpu();
    return {(int64_t)(uint32_t)h[0].item<int32_t>(), (int64_t)(uint32_t)h[1].item<int32_t>()};
}

// Grouped (MoE) GEMM: out[rows of expert e] = A[rows] @ B[e]^T (see
// mbs_gemm_a4w4_grouped_launch).  B: [E, N, K/2] or [E*N, K/2] bytes,
// B_scale: E shuffled blocks, group_offsets: int32 [E+1] (a host tensor is
// checked -- 0 first, non-decreasing multiples of 32, last <= M -- and
// copied to the device; a device tensor is used as it is, or checked on the
// device first with validate=True).
at::Tensor gemm_a4w4_grouped(at::Tensor A, at::Tensor B, at::Tensor A_scale, at::Tensor B_scale,
                             at::Tensor group_offsets, c10::optional<at::Tensor> A_factor,
                             c10::optional<at::Tensor> B_factor, int64_t config, double alpha,
                             c10::optional<at::Tensor> bias, bool validate)
{
    TORCH_CHECK(group_offsets.dim() == 1 && group_offsets.numel() >= 2 &&
                    group_offsets.scalar_type() == at::kInt,
                "gemm_a4w4_grouped: group_offsets must be an int32 vector of E+1 entries");
    const int64_t E = group_offsets.numel() - 1;
    TORCH_CHECK(A.is_cuda() && B.is_cuda() && A.dim() == 2, "gemm_a4w4_grouped: A, B on device, A 2D");
    TORCH_CHECK(B.element_size() == 1 && A.element_size() == 1, "gemm_a4w4_grouped: 1-byte A and B");
    const int64_t M = A.size(0), Kp = A.size(1), K = Kp * 2;
    TORCH_CHECK(B.numel() % (E * Kp) == 0, "gemm_a4w4_grouped: B must hold E blocks of [N, K/2]");
    const int64_t N = B.numel() / (E * Kp);
    TORCH_CHECK(B.size(-1) == Kp, "gemm_a4w4_grouped: B and A disagree on K");
    const int64_t snp = scale_pad(K), Mpad = round_up(M, 32), Npad = round_up(N, 32);
    TORCH_CHECK(A_scale.is_cuda() && B_scale.is_cuda(), "gemm_a4w4_grouped: scales must be on device");
    TORCH_CHECK(A_scale.numel() >= Mpad * snp, "gemm_a4w4_grouped: A_scale too small");
    TORCH_CHECK(B_scale.numel() >= E * Npad * snp, "gemm_a4w4_grouped: B_scale too small");
    TORCH_CHECK(A_factor.has_value() == B_factor.has_value(),
                "gemm_a4w4_grouped: A_factor and B_factor must be given together");
    at::Tensor goff = group_offsets;
    if (!goff.is_cuda()) {
        auto g = goff.contiguous();
        const int32_t* h = g.data_ptr<int32_t>();
        TORCH_CHECK(h[0] == 0, "gemm_a4w4_grouped: group_offsets[0] must be 0");
        for (int64_t e = 0; e < E; ++e)
            TORCH_CHECK(h[e + 1] >= h[e] && h[e + 1] % 32 == 0,
                        "gemm_a4w4_grouped: group_offsets must be non-decreasing multiples of 32");
        TORCH_CHECK(h[E] <= M, "gemm_a4w4_grouped: group_offsets[E] exceeds the rows of A");
        goff = g.to(A.device());
    } else {
        TORCH_CHECK(goff.device() == A.device(), "gemm_a4w4_grouped: group_offsets on another device");
        goff = aligned_contiguous(goff);
        if (validate) {
            // Device offsets are read by the kernel unchecked; on request,
            // check them on the device first (synchronises the stream).
            const auto st = check_groups(goff, M);
            TORCH_CHECK(std::get<0>(st) == 0 && std::get<1>(st) == 0, "gemm_a4w4_grouped: ",
                        std::get<0>(st), " experts start at a row that is not a multiple of 32 and ",
                        std::get<1>(st), " offsets lie outside [0, M] or decrease");
        }
    }
    c10::DeviceGuard guard(A.device());
    auto Au = as_bytes(A), Bu = as_bytes(B), Asu = as_bytes(A_scale), Bsu = as_bytes(B_scale);
    at::Tensor Af, Bf;
    if (A_factor.has_value()) {
        Af = as_bytes(*A_factor, 4);
        Bf = as_bytes(*B_factor, 4);
        TORCH_CHECK(Af.is_cuda() && Bf.is_cuda() && Af.numel() == M && Bf.numel() == E * N,
                    "gemm_a4w4_grouped: factors must be device bytes of M and E*N entries");
    }
    at::Tensor bz;
    if (bias.has_value()) {
        bz = aligned_contiguous(*bias);
        TORCH_CHECK(bz.is_cuda() && bz.device() == A.device() && bz.scalar_type() == at::kBFloat16 &&
                        bz.numel() == E * N,
                    "gemm_a4w4_grouped: bias must be a bf16 device tensor of E*N entries");
    }
    auto out = torch::empty({Mpad, N}, torch::TensorOptions().dtype(torch::kBFloat16).device(A.device()));
    check_status(mbs_gemm_a4w4_grouped_launch_ex(
                     Au.data_ptr<uint8_t>(), Bu.data_ptr<uint8_t>(), Asu.data_ptr<uint8_t>(),
                     Bsu.data_ptr<uint8_t>(), Af.defined() ? Af.data_ptr<uint8_t>() : nullptr,
                     Bf.defined() ? Bf.data_ptr<uint8_t>() : nullptr, goff.data_ptr<int32_t>(), (int)E,
                     out.data_ptr(), (int)M, (int)N, (int)K, (int)Mpad, (int)snp, (float)alpha,
                     bz.defined() ? bz.data_ptr() : nullptr, (int)config, current_stream(A)),
                 "gemm_a4w4_grouped");
    return out.narrow(0, 0, M);
}

// Decode from a bf16 activation, x bf16 [M, K]: one launch (the decode
// kernel quantizes x in registers, M <= 32) or two (quantize_mxfp4, then
// gemm_a4w4).  Either way the bytes are those of quantize_mxfp4 followed by
// gemm_a4w4 on the same plan.  one_launch: 1 forces the one-launch form, 0
// the two launches, -1 picks the faster: one launch for M <= 8 (each
// workgroup quantizes the live rows only: 7.7 / 8.3 / 9.7 us against
// 9.8 / 9.9 / 10.3 us for two launches at M = 1 / 4 / 8, N = K = 8192, cold,
// MI355X), two launches above (every workgroup re-quantizes all 16 or 32
// rows of A: at M = 16 / 32 one launch takes longer than two).  config/splits
// force a skinny configuration (one launch only; -1: the heuristic's).
// With MBS activations every workgroup first takes the rows' maxima over all
// of K: one launch for M <= 4 (9.8 / 10.3 us against 10.8 / 11.1 us for
// quantize_mxfp4_mbs + the factor GEMM at M = 1 / 4), two launches above
// (13.5 against 11.5 us at M = 8).
constexpr int64_t kOneLaunchMaxM = 8;
constexpr int64_t kOneLaunchMaxMbsM = 4;

// With B_factor the activation is MBS-quantized (quantize_mxfp4_mbs, its
// factor bytes derived in the kernel in the one-launch form, M <= 8).
at::Tensor gemm_a4w4_from_bf16(at::Tensor x, at::Tensor B, at::Tensor B_scale,
                               c10::optional<at::Tensor> B_factor, double alpha,
                               c10::optional<at::Tensor> bias, int64_t config, int64_t splits,
                               int64_t one_launch)
{
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.scalar_type() == at::kBFloat16,
                "gemm_a4w4_from_bf16: x must be a 2D bf16 device tensor");
    const bool mbs = B_factor.has_value() && B_factor->defined();
    const int64_t max_one = mbs ? 8 : 32;
    const bool one = one_launch > 0 || config >= 0 ||
                     (one_launch < 0 && x.size(0) <= (mbs ? kOneLaunchMaxMbsM : kOneLaunchMaxM));
    TORCH_CHECK(!(one && x.size(0) > max_one), "gemm_a4w4_from_bf16: the one-launch form needs M <= ",
                max_one, mbs ? " with MBS factors" : "");
    TORCH_CHECK(!(one_launch == 0 && config >= 0),
                "gemm_a4w4_from_bf16: a forced config runs the one-launch form");
    if (!one) {
        if (mbs) {
            auto q = quantize_mxfp4_mbs(x, true, 127);
            return run(prepare(std::get<0>(q), B, std::get<1>(q), B_scale, std::get<2>(q), B_factor),
                       -1, 0, alpha, bias);
        }
        auto q = quantize_mxfp4(x, true, 127);
        return run(prepare(std::get<0>(q), B, std::get<1>(q), B_scale, c10::nullopt, c10::nullopt),
                   -1, 0, alpha, bias);
    }
    TORCH_CHECK(B.is_cuda() && B.dim() == 2 && B_scale.is_cuda() && B.element_size() == 1 &&
                    B_scale.element_size() == 1,
                "gemm_a4w4_from_bf16: B and B_scale must be 1-byte device tensors, B 2D");
    TORCH_CHECK(B.device() == x.device() && B_scale.device() == x.device(),
                "gemm_a4w4_from_bf16: all operands must be on the same device");
    auto xc = aligned_contiguous(x);
    const at::Tensor Bb = as_bytes(B), Bsb = as_bytes(B_scale);
    const int64_t M = xc.size(0), K = xc.size(1), N = Bb.size(0);
    TORCH_CHECK(Bb.size(1) * 2 == K, "gemm_a4w4_from_bf16: B must be [N, K/2], got K/2 = ",
                Bb.size(1), " for K = ", K);
    TORCH_CHECK(Bsb.numel() >= round_up(N, 32) * scale_pad(K),
                "gemm_a4w4_from_bf16: B_scale must hold at least ", round_up(N, 32) * scale_pad(K),
                " bytes (round_up(N,32) * scaleN_pad), got ", Bsb.numel());
    c10::DeviceGuard guard(x.device());
    const int64_t Mpad = round_up(M, 32);
    auto out = torch::empty({Mpad, N}, torch::TensorOptions().dtype(torch::kBFloat16).device(x.device()));
    // (MBS launches use no K split and so no workspace)
    const size_t ws = mbs ? 0
                      : config < 0 ? mbs_gemm_a4w4_from_bf16_workspace_bytes((int)M, (int)N, (int)K)
                                   : mbs_gemm_a4w4_config_workspace_bytes((int)config, (int)splits,
                                                                          (int)M, (int)N, (int)K);
    at::Tensor wst;
    if (ws) wst = torch::empty({(int64_t)ws}, torch::TensorOptions().dtype(torch::kByte).device(x.device()));
    at::Tensor bu, bf;
    if (bias.has_value()) {
        TORCH_CHECK(bias->is_cuda() && bias->device() == x.device() &&
                        bias->scalar_type() == at::kBFloat16 && bias->numel() == N,
                    "gemm_a4w4_from_bf16: bias must be a bf16 device tensor of N entries");
        bu = aligned_contiguous(*bias);
    }
    if (mbs) {
        bf = as_bytes(*B_factor, 4);
        TORCH_CHECK(bf.is_cuda() && bf.device() == x.device() && bf.numel() == N,
                    "gemm_a4w4_from_bf16: B_factor must hold N = ", N, " bytes on the device");
    }
    check_status(mbs_gemm_a4w4_from_bf16_launch(
                     (int)config, (int)splits, xc.data_ptr(), Bb.data_ptr<uint8_t>(),
                     Bsb.data_ptr<uint8_t>(), mbs ? bf.data_ptr<uint8_t>() : nullptr,
                     out.data_ptr(), (int)M, (int)N, (int)K, (int)Mpad,
                     (int)scale_pad(K), (float)alpha, bu.defined() ? bu.data_ptr() : nullptr,
                     ws ? wst.data_ptr() : nullptr, ws, current_stream(x)),
                 "gemm_a4w4_from_bf16");
    return out.narrow(0, 0, M);
}

std::string plan_name(int64_t M, int64_t N, int64_t K)
{
    char buf[256];
    check_status(mbs_gemm_a4w4_plan_name((int)M, (int)N, (int)K, buf, sizeof(buf)), "plan_name");
    return buf;
}

PYBIND11_MODULE(mbs_gemm_a4w4, m)
{
    m.doc() = "MI355X (gfx950) MXFP4 A4W4 GEMM";
    m.def("gemm_a4w4", &gemm_a4w4,
          "MXFP4 A4W4 GEMM: out[M,N] = dequant(A) @ dequant(B)^T [* alpha * f(A_factor) * "
          "f(B_factor)^T] [+ bias]",
          pybind11::arg("A"), pybind11::arg("B"), pybind11::arg("A_scale"),
          pybind11::arg("B_scale"), pybind11::arg("A_factor") = pybind11::none(),
          pybind11::arg("B_factor") = pybind11::none(), pybind11::arg("alpha") = 1.0,
          pybind11::arg("bias") = pybind11::none());
    m.def("gemm_a4w4_config", &gemm_a4w4_config, "gemm_a4w4 with a forced kernel configuration",
          pybind11::arg("config"), pybind11::arg("splits"), pybind11::arg("A"), pybind11::arg("B"),
          pybind11::arg("A_scale"), pybind11::arg("B_scale"),
          pybind11::arg("A_factor") = pybind11::none(), pybind11::arg("B_factor") = pybind11::none(),
          pybind11::arg("alpha") = 1.0, pybind11::arg("bias") = pybind11::none());
    m.def("quantize_mxfp4", &quantize_mxfp4, "bf16 -> (packed e2m1, E8M0 scales)",
          pybind11::arg("x"), pybind11::arg("shuffle") = true, pybind11::arg("pad_byte") = 127);
    m.def("quantize_mxfp4_mbs", &quantize_mxfp4_mbs,
          "bf16 -> (packed e2m1, E8M0 scales, MBS factor bytes): rows scaled by 1 + f/256",
          pybind11::arg("x"), pybind11::arg("shuffle") = true, pybind11::arg("pad_byte") = 127);
    m.def("shuffle_weight", &shuffle_weight, "(16,16) preshuffle of packed weights",
          pybind11::arg("w"));
    m.def("shuffle_scales", &shuffle_scales, "plain -> shuffled E8M0 scales", pybind11::arg("s"),
          pybind11::arg("pad_byte") = 127);
    m.def("unshuffle_weight", &unshuffle_weight, "inverse of shuffle_weight", pybind11::arg("b"));
    m.def("unshuffle_scales", &unshuffle_scales, "shuffled -> plain E8M0 scales [rows, K/32]",
          pybind11::arg("s"), pybind11::arg("rows"), pybind11::arg("K"));
    m.def("check_scales", &check_scales,
          "(padding entries != pad_byte, live 0xFF entries) of a shuffled scale buffer",
          pybind11::arg("s"), pybind11::arg("rows"), pybind11::arg("K"),
          pybind11::arg("pad_byte") = 127);
    m.def("dequant_mxfp4", &dequant_mxfp4, "packed + shuffled scales -> fp32",
          pybind11::arg("packed"), pybind11::arg("scale"), pybind11::arg("b_preshuffled") = false);
    m.def("gemm_a4w4_grouped", &gemm_a4w4_grouped,
          "grouped (MoE) MXFP4 GEMM: expert e's rows of A times the e-th block of B",
          pybind11::arg("A"), pybind11::arg("B"), pybind11::arg("A_scale"),
          pybind11::arg("B_scale"), pybind11::arg("group_offsets"),
          pybind11::arg("A_factor") = pybind11::none(), pybind11::arg("B_factor") = pybind11::none(),
          pybind11::arg("config") = -1, pybind11::arg("alpha") = 1.0,
          pybind11::arg("bias") = pybind11::none(), pybind11::arg("validate") = false);
    m.def("check_groups", &check_groups,
          "(experts starting off a 32-row boundary, clamped offsets) of device group offsets",
          pybind11::arg("group_offsets"), pybind11::arg("M"));
    m.def("grouped_num_configs", []() { return mbs_gemm_a4w4_grouped_num_configs(); });
    m.def("grouped_config_name",
          [](int64_t c) { return std::string(mbs_gemm_a4w4_grouped_config_name((int)c)); });
    m.def("gemm_a4w4_from_bf16", &gemm_a4w4_from_bf16,
          "GEMM from a bf16 activation: quantize_mxfp4(x) then gemm_a4w4, in one launch "
          "for M <= 8 (or when asked, M <= 32)",
          pybind11::arg("x"), pybind11::arg("B"), pybind11::arg("B_scale"),
          pybind11::arg("B_factor") = pybind11::none(), pybind11::arg("alpha") = 1.0,
          pybind11::arg("bias") = pybind11::none(), pybind11::arg("config") = -1,
          pybind11::arg("splits") = 0, pybind11::arg("one_launch") = -1);
    m.def("plan_name", &plan_name, "kernel plan the heuristic picks for (M, N, K)");
    m.def("num_configs", []() { return mbs_gemm_a4w4_num_configs(); });
    m.def("config_name", [](int64_t c) { return std::string(mbs_gemm_a4w4_config_name((int)c)); });
    m.def("workspace_bytes", [](int64_t M, int64_t N, int64_t K) {
        return (int64_t)mbs_gemm_a4w4_workspace_bytes((int)M, (int)N, (int)K);
    });
}
