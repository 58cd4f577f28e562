// Native (C++) kernels of the most frequently called torch.ops.act_lib operators, registered for
// the CUDA (HIP) dispatch key. The operator schemas, the fake (meta) kernels and every other
// operator stay in act_lib.py / bn_lib.py; this library is loaded after them and replaces their
// Python implementations for the operators below, which the compressed layers call once or twice
// per layer and step. The behaviour is the Python implementations' (same checks, messages, output
// shapes and dtypes, same C ABI calls on the current stream): what changes is the host cost of a
// call, about 15 us through the Python implementation (dispatcher hop, argument handling, three
// Python allocations, ctypes) against a few microseconds here.
//
// Errors: bad bits raise ValueError (TORCH_CHECK_VALUE), as act_triton_kernel.py:329-330 and
// act_lib._bits_consts do; NotImplementedError where the Python implementations raise it;
// everything else RuntimeError. A device guard makes the tensors' device current for the call.
//
// Operators: quant_pack, quant_pack_tiles, dequant_unpack, dequant_unpack_tiles,
// quant_pack_triton, dequant_unpack_triton (AC/act_triton_kernel.py:336-395),
// relu_fwd_fused_pack, relu_bwd_fused_unpack (AC/modules/activations/kernel_registration.py:42-94),
// bn_train_fwd, bn_train_bwd (the compressed BatchNorm layers' one-call forward and backward).
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <cmath>
#include <cstdint>
#include <optional>
#include <tuple>

#include "dopt.h"

namespace {

using at::ScalarType;
using at::Tensor;

constexpr int kAlamSeed = 42;  // the reference operators' fixed seed (act_triton_kernel.py:339, :374)
constexpr double kEpsFused = 1e-5, kEpsPlain = 1e-7;

void check(int rc, const char* what) {
    if (rc == DOPT_OK) return;
    if (rc == DOPT_EBITS) TORCH_CHECK_VALUE(false, dopt_last_error());
    TORCH_CHECK(false, what, " failed (", rc, "): ", dopt_last_error());
}

// (values per word, words per group): act_lib._bits_consts
int64_t words_per_group(int64_t bits, int64_t group_size) {
    TORCH_CHECK_VALUE(bits == 1 || bits == 2 || bits == 4 || bits == 8, "bits must be one of (1,2,4,8). got ", bits);
    return group_size / (32 / bits);
}

int dtype_code(ScalarType t, const char* what) {
    switch (t) {
        case ScalarType::Float: return DOPT_F32;
        case ScalarType::Half: return DOPT_F16;
        case ScalarType::BFloat16: return DOPT_BF16;
        default: TORCH_CHECK(false, what, ": unsupported input dtype ", t);
    }
}

int meta_code(ScalarType t) { return t == ScalarType::Float ? DOPT_F32 : DOPT_BF16; }

void require_cuda(const Tensor& t) {
    TORCH_CHECK(t.device().is_cuda(), "act_lib operators run on HIP (cuda) tensors only");
}

// contiguous with a 16-byte aligned base (the kernels use 128-bit accesses)
Tensor aligned(const Tensor& t) {
    Tensor c = t.contiguous();
    if (reinterpret_cast<uintptr_t>(c.data_ptr()) % 16) c = c.clone();
    return c;
}

void* stream_of(const Tensor& t) {
    return at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

int flags(bool clamp, bool squash) { return (clamp ? DOPT_FLAG_CLAMP : 0) | (squash ? DOPT_FLAG_SQUASH : 0); }

// ---------------------------------------------------------------------------- quant-pack
std::tuple<Tensor, Tensor, Tensor> quant_pack_launch(const Tensor& x_in, int64_t n_groups, int64_t bits,
                                                     int64_t group_size, const int64_t* tile, bool clamp,
                                                     double clamp_alpha, bool squash, int64_t rounding,
                                                     const std::optional<Tensor>& noise_in, int64_t seed,
                                                     int64_t offset, ScalarType scale_dtype) {
    const int64_t nwords = words_per_group(bits, group_size);
    const int xc = dtype_code(x_in.scalar_type(), "quant_pack");
    TORCH_CHECK(scale_dtype == ScalarType::Float || scale_dtype == ScalarType::BFloat16,
                "quant_pack: scale dtype must be float32 or bfloat16, got ", scale_dtype);
    require_cuda(x_in);
    if (noise_in) require_cuda(*noise_in);
    const Tensor x = aligned(x_in);
    const auto opts = x.options();
    Tensor packed = at::empty({n_groups, nwords}, opts.dtype(at::kInt));
    Tensor scale = at::empty({n_groups}, opts.dtype(scale_dtype));
    Tensor xmin = at::empty({n_groups}, opts.dtype(scale_dtype));
    Tensor noise;
    const float* nz = nullptr;
    if (rounding == DOPT_ROUND_STOCH_NOISE) {
        TORCH_CHECK(noise_in.has_value(), "quant_pack: rounding=stochastic_noise needs a noise tensor");
        TORCH_CHECK(noise_in->numel() == n_groups * group_size, "quant_pack: noise has ", noise_in->numel(),
                    " values, expected ", n_groups * group_size);
        noise = aligned(noise_in->to(at::kFloat));
        nz = noise.data_ptr<float>();
    }
    check(dopt_quant_pack(x.data_ptr(), xc, n_groups, (int)group_size, (int)bits, tile, (int)rounding, nz,
                          (uint64_t)seed, (uint64_t)offset, flags(clamp, squash), (float)clamp_alpha,
                          (uint32_t*)packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), meta_code(scale_dtype),
                          stream_of(x)),
          "quant_pack");
    return {packed, scale, xmin};
}

std::tuple<Tensor, Tensor, Tensor> quant_pack(const Tensor& x, int64_t bits, int64_t group_size, bool clamp,
                                              double clamp_alpha, bool squash, int64_t rounding,
                                              const std::optional<Tensor>& noise, int64_t seed, int64_t offset,
                                              ScalarType scale_dtype) {
    TORCH_CHECK(x.dim() == 3 && x.size(2) == group_size, "quant_pack expects x of shape [N, G, ", group_size,
                "], got ", x.sizes());
    const c10::DeviceGuard guard(x.device());
    const int64_t N = x.size(0), G = x.size(1);
    auto [p, s, m] = quant_pack_launch(x, N * G, bits, group_size, nullptr, clamp, clamp_alpha, squash, rounding,
                                       noise, seed, offset, scale_dtype);
    return {p, s.view({N, G}), m.view({N, G})};
}

// [N, C, H, W] in s x s spatial tiles: (N, G = C (H/s) (W/s))
std::pair<int64_t, int64_t> tile_groups(at::IntArrayRef shape, int64_t group_size) {
    TORCH_CHECK(shape.size() == 4, "tile layout expects a 4-D [N, C, H, W] tensor, got ", shape);
    const int64_t s = (int64_t)std::llround(std::sqrt((double)group_size));
    const int64_t N = shape[0], C = shape[1], H = shape[2], W = shape[3];
    TORCH_CHECK(s * s == group_size && H % s == 0 && W % s == 0,
                "tile layout needs s*s == group_size and H, W divisible by s (group_size=", group_size, ", H=", H,
                ", W=", W, ")");
    return {N, C * (H / s) * (W / s)};
}

std::tuple<Tensor, Tensor, Tensor> quant_pack_tiles(const Tensor& x, int64_t bits, int64_t group_size, bool clamp,
                                                    double clamp_alpha, bool squash, int64_t rounding,
                                                    const std::optional<Tensor>& noise, int64_t seed,
                                                    int64_t offset, ScalarType scale_dtype) {
    const auto [N, G] = tile_groups(x.sizes(), group_size);
    const c10::DeviceGuard guard(x.device());
    const int64_t tile[4] = {x.size(0), x.size(1), x.size(2), x.size(3)};
    auto [p, s, m] = quant_pack_launch(x, N * G, bits, group_size, tile, clamp, clamp_alpha, squash, rounding,
                                       noise, seed, offset, scale_dtype);
    return {p, s.view({N, G}), m.view({N, G})};
}

// ---------------------------------------------------------------------------- dequant-unpack
Tensor dequant_launch(const Tensor& packed_in, const Tensor& scale_in, const Tensor& xmin_in, int64_t n_groups,
                      int64_t bits, int64_t group_size, const int64_t* tile, Tensor out) {
    const int64_t nwords = words_per_group(bits, group_size);
    TORCH_CHECK((scale_in.scalar_type() == ScalarType::Float || scale_in.scalar_type() == ScalarType::BFloat16) &&
                    xmin_in.scalar_type() == scale_in.scalar_type(),
                "dequant_unpack: scale and min must both be float32 or both bfloat16");
    TORCH_CHECK(scale_in.numel() == n_groups && xmin_in.numel() == n_groups, "dequant_unpack: scale and min must hold ",
                n_groups, " values, got ", scale_in.numel(), " and ", xmin_in.numel());
    TORCH_CHECK(packed_in.numel() * packed_in.element_size() == n_groups * nwords * 4, "dequant_unpack: packed holds ",
                packed_in.numel() * packed_in.element_size(), " bytes, expected ", n_groups * nwords * 4, " (",
                n_groups, " groups of ", nwords, " words)");
    require_cuda(packed_in);
    require_cuda(scale_in);
    require_cuda(xmin_in);
    const Tensor packed = aligned(packed_in), scale = scale_in.contiguous(), xmin = xmin_in.contiguous();
    check(dopt_dequant_unpack((const uint32_t*)packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(),
                              meta_code(scale.scalar_type()), n_groups, (int)group_size, (int)bits, tile,
                              out.data_ptr(), out.scalar_type() == ScalarType::Float ? DOPT_F32 : DOPT_BF16,
                              stream_of(packed)),
          "dequant_unpack");
    return out;
}

void check_out_dtype(ScalarType t, const char* what) {
    TORCH_CHECK(t == ScalarType::Float || t == ScalarType::BFloat16, what,
                ": output dtype must be float32 or bfloat16, got ", t);
}

Tensor dequant_unpack(const Tensor& packed, const Tensor& scale, const Tensor& xmin, int64_t bits,
                      int64_t group_size, ScalarType out_dtype) {
    TORCH_CHECK(scale.dim() == 2, "dequant_unpack: scale must be [N, G], got ", scale.sizes());
    const int64_t N = scale.size(0), G = scale.size(1);
    check_out_dtype(out_dtype, "dequant_unpack");
    const c10::DeviceGuard guard(packed.device());
    Tensor y = at::empty({N, G, group_size}, packed.options().dtype(out_dtype));
    return dequant_launch(packed, scale, xmin, N * G, bits, group_size, nullptr, y);
}

Tensor dequant_unpack_tiles(const Tensor& packed, const Tensor& scale, const Tensor& xmin, int64_t bits,
                            int64_t group_size, int64_t N, int64_t C, int64_t H, int64_t W, ScalarType out_dtype) {
    const int64_t shape[4] = {N, C, H, W};
    const auto [n, G] = tile_groups(at::IntArrayRef(shape, 4), group_size);
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == n && scale.size(1) == G, "dequant_unpack_tiles: scale shape ",
                scale.sizes(), " != (", n, ", ", G, ")");
    check_out_dtype(out_dtype, "dequant_unpack_tiles");
    const c10::DeviceGuard guard(packed.device());
    Tensor y = at::empty({N, C, H, W}, packed.options().dtype(out_dtype));
    return dequant_launch(packed, scale, xmin, n * G, bits, group_size, shape, y);
}

// ---------------------------------------------------------------------------- reference schemas
int64_t alam_words(int64_t bits, int64_t group_size, int64_t alam_bits) {
    const int64_t nwords = words_per_group(bits, group_size);
    TORCH_CHECK(alam_bits >= 1 && (alam_bits & (alam_bits - 1)) == 0 && nwords % alam_bits == 0,
                "avg_alam: alam_bits must be a power of two dividing group_size*bits/32 = ", nwords, ", got ",
                alam_bits);
    return nwords / alam_bits;
}

std::tuple<Tensor, Tensor, Tensor> quant_pack_triton(const Tensor& x, int64_t bits, int64_t group_size,
                                                     bool avg_alam, int64_t alam_bits, bool clamp,
                                                     double clamp_alpha) {
    TORCH_CHECK(x.dim() == 3 && x.size(2) == group_size, "quant_pack_triton expects x of shape [N, G, ", group_size,
                "], got ", x.sizes());
    const c10::DeviceGuard guard(x.device());
    const int64_t N = x.size(0), G = x.size(1);
    if (!avg_alam) {
        auto [p, s, m] = quant_pack_launch(x, N * G, bits, group_size, nullptr, clamp, clamp_alpha, true,
                                           DOPT_ROUND_NEAREST, std::nullopt, 0, 0, ScalarType::BFloat16);
        return {p, s.view({N, G}), m.view({N, G})};
    }
    const int64_t anw = alam_words(bits, group_size, alam_bits);
    const int xc = dtype_code(x.scalar_type(), "quant_pack_triton");
    require_cuda(x);
    const Tensor xc_t = x.contiguous();
    const auto opts = xc_t.options();
    Tensor packed = at::empty({N * G, anw}, opts.dtype(at::kInt));
    Tensor scale = at::empty({N * G}, opts.dtype(at::kBFloat16));
    Tensor xmin = at::empty({N * G}, opts.dtype(at::kBFloat16));
    check(dopt_alam_quant_pack(xc_t.data_ptr(), xc, N * G, (int)group_size, (int)bits, (int)alam_bits,
                               flags(clamp, true), (float)clamp_alpha, (uint32_t*)packed.data_ptr(),
                               (uint16_t*)scale.data_ptr(), (uint16_t*)xmin.data_ptr(), stream_of(xc_t)),
          "alam_quant_pack");
    return {packed, scale.view({N, G}), xmin.view({N, G})};
}

Tensor dequant_unpack_triton(const Tensor& packed, const Tensor& scale, const Tensor& xmin, int64_t bits,
                             int64_t group_size, bool avg_alam, int64_t alam_bits) {
    TORCH_CHECK(scale.dim() == 2, "dequant_unpack_triton: scale must be [N, G], got ", scale.sizes());
    const int64_t N = scale.size(0), G = scale.size(1);
    const c10::DeviceGuard guard(packed.device());
    Tensor y = at::empty({N, G, group_size}, packed.options().dtype(at::kBFloat16));
    if (!avg_alam) return dequant_launch(packed, scale, xmin, N * G, bits, group_size, nullptr, y);
    const int64_t anw = alam_words(bits, group_size, alam_bits);
    TORCH_CHECK(scale.scalar_type() == ScalarType::BFloat16 && xmin.scalar_type() == ScalarType::BFloat16,
                "dequant_unpack_triton: avg_alam takes the bf16 scale and min its quantizer writes");
    TORCH_CHECK(packed.numel() == N * G * anw, "dequant_unpack_triton: packed holds ", packed.numel(),
                " words, expected ", N * G * anw, " (", N * G, " groups of ", anw, ")");
    require_cuda(packed);
    require_cuda(scale);
    require_cuda(xmin);
    const Tensor p = packed.contiguous(), s = scale.contiguous(), m = xmin.contiguous();
    check(dopt_alam_dequant_unpack((const uint32_t*)p.data_ptr(), (const uint16_t*)s.data_ptr(),
                                   (const uint16_t*)m.data_ptr(), N * G, (int)group_size, (int)bits, (int)alam_bits,
                                   kAlamSeed, (uint16_t*)y.data_ptr(), stream_of(p)),
          "alam_dequant_unpack");
    return y;
}

// ---------------------------------------------------------------------------- ReLU layers
bool relu6_of(bool relu, bool relu6) {
    if (relu) return false;
    TORCH_CHECK(relu6, "relu ops need relu=True or relu6=True (the reference kernel has no other branch)");
    return true;
}

std::tuple<Tensor, Tensor, int64_t, int64_t> relu_fwd_fused_pack(const Tensor& x_in, bool relu, bool relu6,
                                                                 int64_t bits, int64_t group_size) {
    const int64_t nwords = words_per_group(bits, group_size);
    TORCH_CHECK(x_in.scalar_type() == ScalarType::BFloat16 || x_in.scalar_type() == ScalarType::Float,
                "relu_fwd_fused_pack: input must be bfloat16 or float32, got ", x_in.scalar_type());
    require_cuda(x_in);
    const int64_t N = x_in.size(0);
    TORCH_CHECK(N > 0 && x_in.numel() % (N * group_size) == 0, "x of shape ", x_in.sizes(),
                " does not split into [N, G, ", group_size, "] groups");
    const int64_t G = x_in.numel() / N / group_size;
    const bool r6 = relu6_of(relu, relu6);
    const c10::DeviceGuard guard(x_in.device());
    const Tensor x = aligned(x_in);
    Tensor y = at::empty_like(x);
    Tensor packed = at::empty({N * G, nwords}, x.options().dtype(at::kInt));
    check(dopt_relu_pack(x.data_ptr(), dtype_code(x.scalar_type(), "relu_fwd_fused_pack"), x.numel(), r6 ? 1 : 0,
                         (int)bits, y.data_ptr(), (uint32_t*)packed.data_ptr(), stream_of(x)),
          "relu_fwd_fused_pack");
    return {y, packed, N, G};
}

Tensor relu_bwd_fused_unpack(const Tensor& packed_in, const Tensor& dy_in, int64_t bits, int64_t N, int64_t G,
                             int64_t group_size) {
    words_per_group(bits, group_size);
    const int dyc = dtype_code(dy_in.scalar_type(), "relu_bwd_fused_unpack");
    TORCH_CHECK(dy_in.numel() == N * G * group_size, "relu_bwd_fused_unpack: dy has ", dy_in.numel(),
                " elements, expected ", N * G * group_size);
    TORCH_CHECK(packed_in.numel() * packed_in.element_size() * 8 >= dy_in.numel() * bits,
                "relu_bwd_fused_unpack: packed holds ", packed_in.numel() * packed_in.element_size(),
                " bytes, too few for ", dy_in.numel(), " ", bits, "-bit masks");
    require_cuda(packed_in);
    require_cuda(dy_in);
    const c10::DeviceGuard guard(dy_in.device());
    const Tensor packed = aligned(packed_in), dy = aligned(dy_in);
    Tensor dx = at::empty(dy.sizes(), dy.options().dtype(at::kBFloat16));
    check(dopt_relu_unpack((const uint32_t*)packed.data_ptr(), dy.data_ptr(), dyc, dy.numel(), (int)bits,
                           dx.data_ptr(), stream_of(dy)),
          "relu_bwd_fused_unpack");
    return dx;
}

// ---------------------------------------------------------------------------- BatchNorm layers
int64_t bn_group(int64_t block) {
    const int64_t g = block / 2;
    TORCH_CHECK(g >= 32 && g <= 512 && (g & (g - 1)) == 0, "BLOCK_M // 2 must be a power of two in [32, 512], got BLOCK_M=",
                block);
    return g;
}

int bn_layer_mode(int64_t kind) {
    TORCH_CHECK(kind == DOPT_BN_QUANT || kind == DOPT_BN_RELU_QUANT || kind == DOPT_BN_RELU6_QUANT,
                "BatchNorm layer operators take kind BN_QUANT, BN_RELU_QUANT or BN_RELU6_QUANT, got ", kind);
    return kind == DOPT_BN_RELU6_QUANT ? DOPT_BN_RELU_QUANT : (int)kind;
}

// forward and backward eps of the layer kinds (the operators' own: bn_lib._LAYER_EPS)
double bn_eps(int64_t kind, bool backward) {
    if (kind == DOPT_BN_QUANT) return backward ? kEpsPlain : kEpsFused;
    return kEpsFused;
}

Tensor f32(const Tensor& t) {
    if (t.scalar_type() == ScalarType::Float && t.is_contiguous()) return t;
    return t.detach().contiguous().to(at::kFloat);
}

Tensor bn_workspace(const Tensor& like, int64_t N, int64_t C, int64_t HW) {
    const int64_t n = dopt_bn_workspace_floats(N, C, HW);
    return at::empty({n > 1 ? n : 1}, like.options().dtype(at::kFloat));
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> bn_train_fwd(
    const Tensor& X, const Tensor& weight, const Tensor& bias, Tensor& running_mean_in, Tensor& running_var_in,
    double momentum, int64_t BLOCK_M, int64_t bits, int64_t kind) {
    bn_layer_mode(kind);
    const int64_t g = bn_group(BLOCK_M);
    words_per_group(bits, g);
    const bool has_rm = running_mean_in.defined() && running_mean_in.numel() > 0;
    const bool has_rv = running_var_in.defined() && running_var_in.numel() > 0;
    require_cuda(X);
    require_cuda(weight);
    require_cuda(bias);
    if (has_rm) require_cuda(running_mean_in);
    if (has_rv) require_cuda(running_var_in);
    TORCH_CHECK(X.dim() >= 2 && (X.scalar_type() == ScalarType::Float || X.scalar_type() == ScalarType::Half ||
                                 X.scalar_type() == ScalarType::BFloat16),
                "bn_train_fwd: X must be an [N, C, ...] float tensor, got ", X.sizes(), " ", X.scalar_type());
    const int64_t N = X.size(0), C = X.size(1);
    const int64_t HW = N * C != 0 ? X.numel() / (N * C) : 0;
    const int64_t M = N * HW;
    TORCH_CHECK(weight.numel() == C, "bn_train_fwd: weight must hold ", C, " values (one per channel), got ",
                weight.numel());
    TORCH_CHECK(bias.numel() == C, "bn_train_fwd: bias must hold ", C, " values (one per channel), got ", bias.numel());
    TORCH_CHECK(!has_rm || running_mean_in.numel() == C, "bn_train_fwd: running_mean must hold ", C,
                " values (one per channel), got ", running_mean_in.numel());
    TORCH_CHECK(!has_rv || running_var_in.numel() == C, "bn_train_fwd: running_var must hold ", C,
                " values (one per channel), got ", running_var_in.numel());
    const c10::DeviceGuard guard(X.device());
    const Tensor X3 = X.contiguous().view({N, C, HW});
    const bool in_kernel = (!has_rm || (running_mean_in.scalar_type() == ScalarType::Float && running_mean_in.is_contiguous())) &&
                           (!has_rv || (running_var_in.scalar_type() == ScalarType::Float && running_var_in.is_contiguous()));
    const auto opts = X3.options();
    Tensor y = at::empty({N, C, HW}, opts.dtype(at::kBFloat16));
    Tensor packed = at::empty({C, M * bits / 32}, opts.dtype(at::kInt));
    Tensor scale = at::empty({C, M / g}, opts.dtype(at::kBFloat16));
    Tensor xmin = at::empty_like(scale);
    Tensor rp = at::empty({C, kind != DOPT_BN_QUANT ? M / 32 : 0}, opts.dtype(at::kInt));
    Tensor mean = at::empty({C}, opts.dtype(at::kFloat));
    Tensor var = at::empty_like(mean);
    Tensor ws = bn_workspace(X3, N, C, HW);
    const Tensor w = f32(weight), b = f32(bias);
    float* rm = in_kernel && has_rm ? running_mean_in.data_ptr<float>() : nullptr;
    float* rv = in_kernel && has_rv ? running_var_in.data_ptr<float>() : nullptr;
    check(dopt_bn_train_forward(X3.data_ptr(), dtype_code(X3.scalar_type(), "bn_train_fwd"), N, C, HW, C * HW, HW,
                                ws.data_ptr<float>(), w.data_ptr<float>(), b.data_ptr<float>(),
                                (float)bn_eps(kind, false), (int)kind, (int)g, (int)bits, y.data_ptr(), nullptr,
                                (uint32_t*)packed.data_ptr(), rp.numel() ? (uint32_t*)rp.data_ptr() : nullptr,
                                scale.data_ptr(), xmin.data_ptr(), mean.data_ptr<float>(), var.data_ptr<float>(), rm,
                                rv, (float)momentum, stream_of(X3)),
          "bn_train_fwd");
    if (!in_kernel) {
        if (has_rm) running_mean_in.mul_(1.0 - momentum).add_(mean, momentum);
        if (has_rv) running_var_in.mul_(1.0 - momentum).add_(var, momentum);
    }
    return {y, packed, rp, scale, xmin, mean, var};
}

std::tuple<Tensor, Tensor, Tensor> bn_train_bwd(const Tensor& packed_in, const std::optional<Tensor>& relu_packed_in,
                                                const Tensor& dy, const Tensor& scale_in, const Tensor& min_in,
                                                const Tensor& weight, const Tensor& var, int64_t BLOCK_M, int64_t bits,
                                                int64_t kind) {
    const int m = bn_layer_mode(kind);
    const int64_t g = bn_group(BLOCK_M);
    words_per_group(bits, g);
    TORCH_CHECK(dy.dim() >= 2, "bn_train_bwd: dy must be [N, C, ...], got ", dy.sizes());
    require_cuda(dy);
    const int64_t N = dy.size(0), C = dy.size(1);
    const int64_t HW = N * C != 0 ? dy.numel() / (N * C) : 0;
    const int64_t M = N * HW;
    const c10::DeviceGuard guard(dy.device());
    const Tensor DY3 = dy.contiguous().view({N, C, HW});
    const Tensor p = packed_in.contiguous(), sc = scale_in.contiguous(), mn = min_in.contiguous();
    std::optional<Tensor> rp;
    if (m == DOPT_BN_RELU_QUANT && relu_packed_in.has_value()) rp = relu_packed_in->contiguous();
    const Tensor w = f32(weight), v = f32(var);
    // the kernels read the saved tensors unchecked: their sizes must match the channel layout
    TORCH_CHECK(p.numel() * p.element_size() * 8 == C * M * bits, "BatchNorm backward: packed codes hold ",
                p.numel() * p.element_size(), " bytes, expected ", C * M * bits / 8);
    TORCH_CHECK(!rp || rp->numel() * rp->element_size() * 8 >= C * M,
                "BatchNorm backward: the ReLU mask is too small for the tensor");
    TORCH_CHECK(sc.numel() == C * (M / g) && mn.numel() == C * (M / g), "BatchNorm backward: scale/min hold ",
                sc.numel(), " values, expected ", C * (M / g));
    TORCH_CHECK(w.numel() == C && v.numel() == C, "BatchNorm backward: per-channel vectors must hold ", C,
                " values, got ", w.numel(), " and ", v.numel());
    TORCH_CHECK(m != DOPT_BN_RELU_QUANT || rp.has_value(), "bn_train_bwd: the ReLU kinds need the saved ReLU mask");
    for (const Tensor* t : {&p, &sc, &mn, &w, &v}) require_cuda(*t);
    Tensor dx = at::empty({N, C, HW}, DY3.options().dtype(at::kBFloat16));
    Tensor dw = at::empty({C}, DY3.options().dtype(at::kFloat));
    Tensor db = at::empty_like(dw);
    Tensor ws = bn_workspace(DY3, N, C, HW);
    check(dopt_bn_train_backward(m, (const uint32_t*)p.data_ptr(), rp ? (const uint32_t*)rp->data_ptr() : nullptr,
                                 sc.data_ptr(), mn.data_ptr(), DY3.data_ptr(), dtype_code(DY3.scalar_type(), "bn_train_bwd"),
                                 N, C, HW, C * HW, HW, (int)g, (int)bits, ws.data_ptr<float>(), w.data_ptr<float>(),
                                 v.data_ptr<float>(), (float)bn_eps(kind, true), dw.data_ptr<float>(),
                                 db.data_ptr<float>(), dx.data_ptr(), stream_of(DY3)),
          "bn_train_bwd");
    return {dx, dw, db};
}

}  // namespace

TORCH_LIBRARY_IMPL(act_lib, CUDA, m) {
    m.impl("quant_pack", &quant_pack);
    m.impl("quant_pack_tiles", &quant_pack_tiles);
    m.impl("dequant_unpack", &dequant_unpack);
    m.impl("dequant_unpack_tiles", &dequant_unpack_tiles);
    m.impl("quant_pack_triton", &quant_pack_triton);
    m.impl("dequant_unpack_triton", &dequant_unpack_triton);
    m.impl("relu_fwd_fused_pack", &relu_fwd_fused_pack);
    m.impl("relu_bwd_fused_unpack", &relu_bwd_fused_unpack);
    m.impl("bn_train_fwd", &bn_train_fwd);
    m.impl("bn_train_bwd", &bn_train_bwd);
}
