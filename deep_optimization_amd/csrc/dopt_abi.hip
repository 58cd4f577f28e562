// extern "C" entry points of libdopt.so (declared in include/dopt.h): argument validation,
// layout set-up and dispatch to the templated gfx950 kernels. No entry point allocates,
// frees or synchronises; all work is enqueued on the caller's stream.
#include <stdarg.h>
#include <initializer_list>
#include <mutex>
#include <stdio.h>

#include "../../include/dopt.h"
#include "bn_fused.h"
#include "dequant_unpack.h"
#include "dw_gemm.h"
#include "quant_pack.h"

namespace dopt {
int launch_pack_codes(const int8_t* codes, uint32_t* out, uint64_t n_words, int bits, hipStream_t s);
int launch_unpack_codes(const uint32_t* packed, int8_t* codes, uint64_t n_words, int bits, hipStream_t s);
int launch_fp8_gemm_nt(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, float out_scale, uint16_t* C, int64_t ldc, hipStream_t s);
int launch_fp8_pack(const uint8_t* src, int64_t rows, int64_t cols, int64_t stride_r, int64_t stride_c, uint8_t* dst,
                    int64_t ld_dst, hipStream_t s);
int launch_relu_pack(const void* x, int dt, void* y, uint32_t* packed, uint64_t n, int bits, bool relu6, hipStream_t s);
int launch_relu_unpack(const uint32_t* packed, const void* dy, int dyt, void* dx, uint64_t n, int bits, hipStream_t s);
int launch_act_forward(const void* x, int dt, void* y, void* aux, uint64_t n, int act, hipStream_t s);
int launch_pact_clamp_fwd(const void* x, int dt, float alpha, void* y, int8_t* mask, uint64_t n, hipStream_t s);
int launch_pact_clamp_bwd(const int8_t* mask, const void* dy, int dyt, void* dx, uint64_t n, hipStream_t s);
const char* graph_node_counts(hipGraph_t g, int64_t* counts, int n_counts);
const char* graph_replace_memsets(hipGraph_t g, int64_t* replaced);
int launch_alam_quant_pack(const void* x, int dt, int64_t n_groups, int g, int bits, int alam, int flags,
                           float clamp_alpha, uint32_t* packed, uint16_t* scale, uint16_t* minv, hipStream_t s);
int launch_alam_dequant(const uint32_t* packed, const uint16_t* scale, const uint16_t* minv, int64_t n_groups,
                        int g, int bits, int alam, uint64_t seed, uint16_t* y, hipStream_t s);
int launch_alam_act_dequant_mul(const DequantArgs& d, int g, int bits, int dy_f32, uint64_t seed, hipStream_t s);
}  // namespace dopt

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return DOPT_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_bits(int bits) {
    if (bits != 1 && bits != 2 && bits != 4 && bits != 8)
        return fail(DOPT_EBITS, "bits must be one of (1,2,4,8). got %d", bits);
    return DOPT_OK;
}

int check_group(int g) {
    if (g < 64 || g > 1024 || (g & (g - 1)))
        return fail(DOPT_EINVAL, "group_size must be a power of two in [64, 1024], got %d", g);
    return DOPT_OK;
}

int ilog2(int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

// Validates an optional [N, C, H, W] tile descriptor and returns (tiles_w, log2 s, row).
int setup_tiles(const int64_t* t, int64_t n_groups, int g, uint32_t* tiled, uint32_t* tiles_w, uint32_t* log2s,
                uint64_t* row) {
    *tiled = 0;
    *tiles_w = 1;
    *log2s = 0;
    *row = 0;
    if (!t) return DOPT_OK;
    int s = 1;
    while (s * s < g) ++s;
    if (s * s != g)
        return fail(DOPT_EINVAL, "tile layout needs a square group size (s*s == g), got g=%d", g);
    const int64_t N = t[0], C = t[1], H = t[2], W = t[3];
    if (N < 0 || C < 0 || H <= 0 || W <= 0 || H % s || W % s)
        return fail(DOPT_EINVAL, "tile layout needs H %% %d == 0 and W %% %d == 0 (got N=%lld C=%lld H=%lld W=%lld)", s,
                    s, (long long)N, (long long)C, (long long)H, (long long)W);
    if (N * C * (H / s) * (W / s) != n_groups)
        return fail(DOPT_EINVAL, "n_groups=%lld does not match the tile layout (%lld)", (long long)n_groups,
                    (long long)(N * C * (H / s) * (W / s)));
    *tiled = 1;
    *tiles_w = (uint32_t)(W / s);
    *log2s = (uint32_t)ilog2(s);
    *row = (uint64_t)W;
    return DOPT_OK;
}

// Validates a BatchNorm geometry; fills g and whether 16-byte vector access applies.
int bn_geom(int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c, dopt::BnGeom* g) {
    if (N < 0 || C < 0 || HW < 0 || C > 65535)
        return fail(DOPT_EINVAL, "BatchNorm shape must have N, HW >= 0 and 0 <= C <= 65535, got N=%lld C=%lld HW=%lld",
                    (long long)N, (long long)C, (long long)HW);
    // the kernels' grids run the channels along x and the channel's BN_CHUNK-element chunks along y
    if (N * HW > (int64_t)65535 * dopt::BN_CHUNK)
        return fail(DOPT_EINVAL, "BatchNorm channel too large: N*HW=%lld (limit 65535 * %lld = %lld)", (long long)(N * HW),
                    (long long)dopt::BN_CHUNK, (long long)(65535 * dopt::BN_CHUNK));
    if (stride_n < 0 || stride_c < 0) return fail(DOPT_EINVAL, "BatchNorm strides must be non-negative");
    *g = dopt::BnGeom{N, C, HW, stride_n, stride_c};
    return DOPT_OK;
}

// Elements per vector access of the BatchNorm kernels: the largest of 8, 4, 2 that divides HW and
// both strides (so no access crosses a row) with every tensor (pointer, element bytes) aligned
// for it; else 1.
struct BnTensor {
    const void* p;
    int bytes;
};
int bn_width(const dopt::BnGeom& g, std::initializer_list<BnTensor> ts) {
    for (int v : {8, 4, 2}) {
        if (g.HW % v || g.stride_n % v || g.stride_c % v) continue;
        bool ok = true;
        for (const BnTensor& t : ts) {
            const uintptr_t align = (uintptr_t)(v * t.bytes < 16 ? v * t.bytes : 16);
            if (t.p && ((uintptr_t)t.p % align)) ok = false;
        }
        if (ok) return v;
    }
    return 1;
}

int bn_bytes(int dt) { return dt == DOPT_F32 ? 4 : 2; }

int bn_dtype(int dt, const char* what) {
    if (dt != DOPT_F32 && dt != DOPT_F16 && dt != DOPT_BF16)
        return fail(DOPT_EINVAL, "%s dtype must be F32, F16 or BF16, got code %d", what, dt);
    return DOPT_OK;
}

int bn_quant_checks(int mode, int64_t M, int group_size, int bits, const void* packed, const void* scale,
                    const void* minv, const void* relu_packed) {
    int rc;
    if (mode < DOPT_BN_NORM || mode > DOPT_BN_RELU6_QUANT) return fail(DOPT_EINVAL, "unknown BatchNorm mode %d", mode);
    if (mode == DOPT_BN_NORM) return DOPT_OK;
    if ((rc = check_bits(bits))) return rc;
    if (group_size < 32 || group_size > 512 || (group_size & (group_size - 1)))
        return fail(DOPT_EINVAL, "BatchNorm group_size must be a power of two in [32, 512], got %d", group_size);
    if (M % group_size)
        return fail(DOPT_EINVAL, "BatchNorm quant-pack needs N*HW %% group_size == 0 (N*HW=%lld, group_size=%d)",
                    (long long)M, group_size);
    if (!packed || !scale || !minv) return fail(DOPT_EINVAL, "null packed/scale/min pointer");
    if ((uintptr_t)packed & 7u) return fail(DOPT_EINVAL, "packed must be 8-byte aligned");
    if (mode != DOPT_BN_QUANT && !relu_packed) return fail(DOPT_EINVAL, "null relu_packed pointer");
    return DOPT_OK;
}

// log2 of avg_alam's run length A: a power of two dividing the group's code words
// group_size * bits / 32, as the reference's reshape of the codes into runs requires
// (kernel_registration.py:124-128)
int bn_alam_lg(int group_size, int bits, int alam_bits, int* lg) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    const int nwords = group_size * bits / 32;
    if (alam_bits < 1 || (alam_bits & (alam_bits - 1)) || nwords < 1 || nwords % alam_bits)
        return fail(DOPT_EINVAL, "alam_bits must be a power of two dividing group_size*bits/32 = %d, got %d", nwords,
                    alam_bits);
    int l = 0;
    while ((1 << l) < alam_bits) ++l;
    *lg = l;
    return DOPT_OK;
}

// Static per-device scratch of dopt_bn_train_forward_noalloc: the statistics kernel's workgroup
// partials, which the normalize kernel sums. Each partial slot is written before it is read in
// the same call, so nothing needs clearing between calls. In host code `scratch` is only a
// host-side handle: kernels get the device address that hipGetSymbolAddress returns for the
// current device, looked up on the entry point's first call on that device and kept for the
// life of the process (a hipDeviceReset, which frees the module and its scratch, invalidates it;
// this library is not to be used across one). That first call may come while the caller's stream
// is being captured into a graph: the lookup then runs in the relaxed capture mode, in which a
// call that is not a stream operation is allowed, and the previous mode is restored after it.
static __device__ __align__(256) float scratch[DOPT_BN_SCRATCH_FLOATS];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(DOPT_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(DOPT_EINVAL, "device index %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        const hipError_t em = hipThreadExchangeStreamCaptureMode(&mode);
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (em == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess || !p)
            return fail(DOPT_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = (float*)p;
    }
    *out = g_scratch_ptr[dev];
    return DOPT_OK;
}

int hip_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DOPT_EHIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

}  // namespace

extern "C" {

int dopt_abi_version(void) { return DOPT_ABI_VERSION; }

const char* dopt_last_error(void) { return g_err; }

int dopt_quant_pack(const void* x, int x_dtype, int64_t n_groups, int group_size, int bits, const int64_t* tile_nchw,
                    int rounding, const float* noise, uint64_t seed, uint64_t offset, int flags, float clamp_alpha,
                    uint32_t* packed, void* scale, void* minv, int meta_dtype, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0 || n_groups >= (int64_t)1 << 31)
        return fail(DOPT_EINVAL, "n_groups must be in [0, 2^31), got %lld", (long long)n_groups);
    if (x_dtype != DOPT_F32 && x_dtype != DOPT_F16 && x_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "unsupported input dtype code %d", x_dtype);
    if (meta_dtype != DOPT_F32 && meta_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "scale/min dtype must be F32 or BF16, got code %d", meta_dtype);
    if (rounding < DOPT_ROUND_NEAREST || rounding > DOPT_ROUND_STOCH_PHILOX)
        return fail(DOPT_EINVAL, "unknown rounding mode %d", rounding);
    if (flags & ~(DOPT_FLAG_CLAMP | DOPT_FLAG_SQUASH)) return fail(DOPT_EINVAL, "unknown flags 0x%x", flags);
    dopt::QuantPackArgs a{};
    if ((rc = setup_tiles(tile_nchw, n_groups, group_size, &a.tiled, &a.tiles_w, &a.log2s, &a.row))) return rc;
    if (n_groups == 0) return ok();
    if (!x || !packed || !scale || !minv) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(x) || !aligned16(packed))
        return fail(DOPT_EINVAL, "x and packed must be 16-byte aligned");
    if (rounding == DOPT_ROUND_STOCH_NOISE && (!noise || !aligned16(noise)))
        return fail(DOPT_EINVAL, "stochastic rounding with a noise tensor needs a 16-byte aligned fp32 noise pointer");
    a.x = x;
    a.noise = noise;
    a.packed = packed;
    a.scale = scale;
    a.minv = minv;
    a.n_groups = (uint32_t)n_groups;
    a.seed_lo = (uint32_t)seed;
    a.seed_hi = (uint32_t)(seed >> 32);
    a.off_lo = (uint32_t)offset;
    a.off_hi = (uint32_t)(offset >> 32);
    a.clamp_alpha = clamp_alpha;
    a.flags = (uint32_t)flags;
    a.meta_bf16 = meta_dtype == DOPT_BF16;
    hipStream_t s = (hipStream_t)stream;
    (void)hipGetLastError();
    switch (x_dtype) {
        case DOPT_F32: rc = dopt::launch_quant_pack_dt<dopt::DT_F32>(a, bits, group_size, rounding, flags ? dopt::PRE_REF : dopt::PRE_NONE, s); break;
        case DOPT_F16: rc = dopt::launch_quant_pack_dt<dopt::DT_F16>(a, bits, group_size, rounding, flags ? dopt::PRE_REF : dopt::PRE_NONE, s); break;
        default: rc = dopt::launch_quant_pack_dt<dopt::DT_BF16>(a, bits, group_size, rounding, flags ? dopt::PRE_REF : dopt::PRE_NONE, s); break;
    }
    if (rc) return fail(DOPT_EUNSUPPORTED, "no quant-pack kernel for bits=%d g=%d rounding=%d", bits, group_size, rounding);
    return hip_status("quant_pack launch");
}

int dopt_dequant_unpack(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype, int64_t n_groups,
                        int group_size, int bits, const int64_t* tile_nchw, void* y, int y_dtype, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0 || n_groups >= (int64_t)1 << 31)
        return fail(DOPT_EINVAL, "n_groups must be in [0, 2^31), got %lld", (long long)n_groups);
    if (meta_dtype != DOPT_F32 && meta_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "scale/min dtype must be F32 or BF16, got code %d", meta_dtype);
    if (y_dtype != DOPT_F32 && y_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "output dtype must be F32 or BF16, got code %d", y_dtype);
    dopt::DequantArgs a{};
    if ((rc = setup_tiles(tile_nchw, n_groups, group_size, &a.tiled, &a.tiles_w, &a.log2s, &a.row))) return rc;
    if (n_groups == 0) return ok();
    if (!packed || !scale || !minv || !y) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(y) || ((uintptr_t)packed & 7u))
        return fail(DOPT_EINVAL, "y must be 16-byte and packed 8-byte aligned");
    a.packed = packed;
    a.scale = scale;
    a.minv = minv;
    a.y = y;
    a.n_groups = (uint32_t)n_groups;
    a.meta_bf16 = meta_dtype == DOPT_BF16;
    hipStream_t s = (hipStream_t)stream;
    (void)hipGetLastError();
    if (y_dtype == DOPT_F32)
        rc = dopt::launch_dequant_unpack_dt<dopt::DT_F32>(a, bits, group_size, dopt::DY_NONE, s);
    else
        rc = dopt::launch_dequant_unpack_dt<dopt::DT_BF16>(a, bits, group_size, dopt::DY_NONE, s);
    if (rc) return fail(DOPT_EUNSUPPORTED, "no dequant kernel for bits=%d g=%d", bits, group_size);
    return hip_status("dequant_unpack launch");
}

static int check_alam(int64_t n_groups, int group_size, int bits, int alam_bits) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0 || n_groups >= (int64_t)1 << 31)
        return fail(DOPT_EINVAL, "n_groups must be in [0, 2^31), got %lld", (long long)n_groups);
    const int nw = group_size * bits / 32;
    if (alam_bits < 1 || (alam_bits & (alam_bits - 1)) || nw % alam_bits)
        return fail(DOPT_EINVAL,
                    "alam_bits must be a power of two dividing group_size*bits/32 = %d (the reference reshapes the "
                    "codes into runs of alam_bits), got %d", nw, alam_bits);
    return DOPT_OK;
}

int dopt_alam_quant_pack(const void* x, int x_dtype, int64_t n_groups, int group_size, int bits, int alam_bits,
                         int flags, float clamp_alpha, uint32_t* packed, uint16_t* scale, uint16_t* minv,
                         void* stream) {
    int rc;
    if ((rc = check_alam(n_groups, group_size, bits, alam_bits))) return rc;
    if (x_dtype != DOPT_F32 && x_dtype != DOPT_F16 && x_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "unsupported input dtype code %d", x_dtype);
    if (flags & ~(DOPT_FLAG_CLAMP | DOPT_FLAG_SQUASH)) return fail(DOPT_EINVAL, "unknown flags 0x%x", flags);
    if (n_groups == 0) return ok();
    if (!x || !packed || !scale || !minv) return fail(DOPT_EINVAL, "null pointer argument");
    if (((uintptr_t)x % (x_dtype == DOPT_F32 ? 4u : 2u)) || ((uintptr_t)packed & 3u) || ((uintptr_t)scale & 1u) ||
        ((uintptr_t)minv & 1u))
        return fail(DOPT_EINVAL, "x, packed, scale and min must be aligned to their element size");
    (void)hipGetLastError();
    dopt::launch_alam_quant_pack(x, x_dtype, n_groups, group_size, bits, alam_bits, flags, clamp_alpha, packed,
                                 scale, minv, (hipStream_t)stream);
    return hip_status("alam_quant_pack launch");
}

int dopt_alam_dequant_unpack(const uint32_t* packed, const uint16_t* scale, const uint16_t* minv, int64_t n_groups,
                             int group_size, int bits, int alam_bits, uint64_t seed, uint16_t* y, void* stream) {
    int rc;
    if ((rc = check_alam(n_groups, group_size, bits, alam_bits))) return rc;
    if (n_groups == 0) return ok();
    if (!packed || !scale || !minv || !y) return fail(DOPT_EINVAL, "null pointer argument");
    if (((uintptr_t)packed & 3u) || ((uintptr_t)scale & 1u) || ((uintptr_t)minv & 1u) || ((uintptr_t)y & 1u))
        return fail(DOPT_EINVAL, "packed, scale, min and y must be aligned to their element size");
    (void)hipGetLastError();
    dopt::launch_alam_dequant(packed, scale, minv, n_groups, group_size, bits, alam_bits, seed, y,
                              (hipStream_t)stream);
    return hip_status("alam_dequant_unpack launch");
}

int dopt_pack_codes(const int8_t* codes, int64_t n_groups, int group_size, int bits, uint32_t* packed, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0) return fail(DOPT_EINVAL, "n_groups must be >= 0");
    if (n_groups == 0) return ok();
    if (!codes || !packed) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(codes) || ((uintptr_t)packed & 3u)) return fail(DOPT_EINVAL, "codes must be 16-byte aligned");
    const uint64_t n_words = (uint64_t)n_groups * (uint64_t)(group_size * bits / 32);
    (void)hipGetLastError();
    dopt::launch_pack_codes(codes, packed, n_words, bits, (hipStream_t)stream);
    return hip_status("pack_codes launch");
}

int dopt_unpack_codes(const uint32_t* packed, int64_t n_groups, int group_size, int bits, int8_t* codes, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0) return fail(DOPT_EINVAL, "n_groups must be >= 0");
    if (n_groups == 0) return ok();
    if (!codes || !packed) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(codes) || ((uintptr_t)packed & 3u)) return fail(DOPT_EINVAL, "codes must be 16-byte aligned");
    const uint64_t n_words = (uint64_t)n_groups * (uint64_t)(group_size * bits / 32);
    (void)hipGetLastError();
    dopt::launch_unpack_codes(packed, codes, n_words, bits, (hipStream_t)stream);
    return hip_status("unpack_codes launch");
}

int dopt_fp8_gemm_nt(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                     float out_scale, void* C, int64_t ldc, void* stream) {
    if (M < 0 || N < 0 || K < 0) return fail(DOPT_EINVAL, "negative GEMM extent");
    if (M == 0 || N == 0) return ok();
    if (!C || (K > 0 && (!A || !B))) return fail(DOPT_EINVAL, "null pointer argument");
    if (K % 16)
        return fail(DOPT_EUNSUPPORTED, "fp8 GEMM needs K %% 16 == 0 (one 16-byte load per lane), got K=%lld",
                    (long long)K);
    if (lda < K || ldb < K || ldc < N || lda % 16 || ldb % 16 || (K > 0 && (!aligned16(A) || !aligned16(B))) ||
        ((uintptr_t)C & 1))
        return fail(DOPT_EINVAL,
                    "fp8 GEMM needs 16-byte aligned A and B, lda and ldb multiples of 16 and >= K, a 2-byte aligned C "
                    "and ldc >= N (got lda=%lld ldb=%lld ldc=%lld K=%lld N=%lld)",
                    (long long)lda, (long long)ldb, (long long)ldc, (long long)K, (long long)N);
    // a 256-row tile's offsets (up to 256 * lda) must stay inside the buffer range 0x7FFFFF00
    if (lda >= (1 << 23) || ldb >= (1 << 23))
        return fail(DOPT_EINVAL, "fp8 GEMM row strides must be below 2^23 bytes (32-bit tile offsets), got %lld, %lld",
                    (long long)lda, (long long)ldb);
    if ((M + 255) / 256 * ((N + 255) / 256) >= ((int64_t)1 << 31))
        return fail(DOPT_EINVAL, "fp8 GEMM output too large: %lld x %lld", (long long)M, (long long)N);
    (void)hipGetLastError();
    const int rc = dopt::launch_fp8_gemm_nt(A, B, M, N, K, lda, ldb, out_scale, (uint16_t*)C, ldc, (hipStream_t)stream);
    if (rc) return fail(DOPT_EUNSUPPORTED, "fp8 GEMM launch configuration unsupported");
    return hip_status("fp8_gemm launch");
}

int dopt_fp8_pack_kmajor(const uint8_t* src, int64_t rows, int64_t cols, int64_t stride_r, int64_t stride_c, uint8_t* dst,
                         int64_t ld_dst, void* stream) {
    if (rows < 0 || cols < 0 || stride_r < 0 || stride_c < 0)
        return fail(DOPT_EINVAL, "fp8 pack: negative extent or stride");
    if (rows == 0 || cols == 0) return ok();
    if (!src || !dst) return fail(DOPT_EINVAL, "null pointer argument");
    if (ld_dst < cols) return fail(DOPT_EINVAL, "fp8 pack: ld_dst (%lld) < cols (%lld)", (long long)ld_dst, (long long)cols);
    (void)hipGetLastError();
    if (dopt::launch_fp8_pack(src, rows, cols, stride_r, stride_c, dst, ld_dst, (hipStream_t)stream))
        return fail(DOPT_EINVAL, "fp8 pack: %lld x %lld is too large for one launch", (long long)rows, (long long)cols);
    return hip_status("fp8_pack launch");
}

int dopt_relu_pack(const void* x, int x_dtype, int64_t n, int relu6, int bits, void* y, uint32_t* packed, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if (x_dtype != DOPT_F32 && x_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "relu_pack: input dtype must be F32 or BF16, got code %d", x_dtype);
    if (n < 0 || n % 64) return fail(DOPT_EINVAL, "relu_pack: n must be a non-negative multiple of 64, got %lld", (long long)n);
    if (n == 0) return ok();
    if (!x || !y || !packed) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(x) || !aligned16(y) || !aligned16(packed)) return fail(DOPT_EINVAL, "x, y and packed must be 16-byte aligned");
    (void)hipGetLastError();
    if (dopt::launch_relu_pack(x, x_dtype, y, packed, (uint64_t)n, bits, relu6 != 0, (hipStream_t)stream))
        return fail(DOPT_EUNSUPPORTED, "no relu_pack kernel for dtype %d bits %d", x_dtype, bits);
    return hip_status("relu_pack launch");
}

int dopt_relu_unpack(const uint32_t* packed, const void* dy, int dy_dtype, int64_t n, int bits, void* dx, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if (dy_dtype != DOPT_F32 && dy_dtype != DOPT_F16 && dy_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "relu_unpack: unsupported dy dtype code %d", dy_dtype);
    if (n < 0 || n % 64) return fail(DOPT_EINVAL, "relu_unpack: n must be a non-negative multiple of 64, got %lld", (long long)n);
    if (n == 0) return ok();
    if (!packed || !dy || !dx) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(dy) || !aligned16(dx) || ((uintptr_t)packed & 7u))
        return fail(DOPT_EINVAL, "dy and dx must be 16-byte and packed 8-byte aligned");
    (void)hipGetLastError();
    if (dopt::launch_relu_unpack(packed, dy, dy_dtype, dx, (uint64_t)n, bits, (hipStream_t)stream))
        return fail(DOPT_EUNSUPPORTED, "no relu_unpack kernel for dtype %d bits %d", dy_dtype, bits);
    return hip_status("relu_unpack launch");
}

int dopt_act_forward(const void* x, int x_dtype, int64_t n, int act, void* y, void* aux, void* stream) {
    if (x_dtype != DOPT_F32 && x_dtype != DOPT_F16 && x_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "act_forward: unsupported input dtype code %d", x_dtype);
    if (act < DOPT_ACT_RELU || act > DOPT_ACT_SILU) return fail(DOPT_EINVAL, "act_forward: unknown activation %d", act);
    if (n < 0) return fail(DOPT_EINVAL, "act_forward: negative n");
    if (n == 0) return ok();
    if (!x || !y || !aux) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(x) || !aligned16(y) || !aligned16(aux)) return fail(DOPT_EINVAL, "x, y and aux must be 16-byte aligned");
    (void)hipGetLastError();
    if (dopt::launch_act_forward(x, x_dtype, y, aux, (uint64_t)n, act, (hipStream_t)stream))
        return fail(DOPT_EUNSUPPORTED, "no act_forward kernel for dtype %d act %d", x_dtype, act);
    return hip_status("act_forward launch");
}

int dopt_pact_clamp_forward(const void* x, int x_dtype, int64_t n, float alpha, void* y, int8_t* mask,
                            void* stream) {
    if (x_dtype != DOPT_F32 && x_dtype != DOPT_F16 && x_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "pact_clamp_forward: unsupported input dtype code %d", x_dtype);
    if (!(alpha > 0.0f)) return fail(DOPT_EINVAL, "pact_clamp_forward: alpha must be > 0 (not NaN), got %g", alpha);
    if (n < 0) return fail(DOPT_EINVAL, "pact_clamp_forward: negative n");
    if (n == 0) return ok();
    if (!x || !y || !mask) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(x) || !aligned16(y) || ((uintptr_t)mask & 7u))
        return fail(DOPT_EINVAL, "x and y must be 16-byte and mask 8-byte aligned");
    (void)hipGetLastError();
    if (dopt::launch_pact_clamp_fwd(x, x_dtype, alpha, y, mask, (uint64_t)n, (hipStream_t)stream))
        return fail(DOPT_EUNSUPPORTED, "no pact_clamp_forward kernel for dtype %d", x_dtype);
    return hip_status("pact_clamp_forward launch");
}

int dopt_pact_clamp_backward(const int8_t* mask, const void* dy, int dy_dtype, int64_t n, void* dx, void* stream) {
    if (dy_dtype != DOPT_F32 && dy_dtype != DOPT_F16 && dy_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "pact_clamp_backward: unsupported dy dtype code %d", dy_dtype);
    if (n < 0) return fail(DOPT_EINVAL, "pact_clamp_backward: negative n");
    if (n == 0) return ok();
    if (!mask || !dy || !dx) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(dy) || !aligned16(dx) || ((uintptr_t)mask & 7u))
        return fail(DOPT_EINVAL, "dy and dx must be 16-byte and mask 8-byte aligned");
    (void)hipGetLastError();
    if (dopt::launch_pact_clamp_bwd(mask, dy, dy_dtype, dx, (uint64_t)n, (hipStream_t)stream))
        return fail(DOPT_EUNSUPPORTED, "no pact_clamp_backward kernel for dtype %d", dy_dtype);
    return hip_status("pact_clamp_backward launch");
}

int dopt_act_quant_pack(const void* x, int x_dtype, int act, int64_t n_groups, int group_size, int bits,
                        const int64_t* tile_nchw, void* y, uint32_t* packed, void* scale, void* minv, int meta_dtype,
                        void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0 || n_groups >= (int64_t)1 << 31)
        return fail(DOPT_EINVAL, "n_groups must be in [0, 2^31), got %lld", (long long)n_groups);
    if (x_dtype != DOPT_F32 && x_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "act_quant_pack: input dtype must be F32 or BF16, got code %d", x_dtype);
    if (act != DOPT_ACT_GELU && act != DOPT_ACT_SILU)
        return fail(DOPT_EINVAL, "act_quant_pack: activation must be GELU or SILU, got %d", act);
    if (meta_dtype != DOPT_F32 && meta_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "scale/min dtype must be F32 or BF16, got code %d", meta_dtype);
    dopt::QuantPackArgs a{};
    if ((rc = setup_tiles(tile_nchw, n_groups, group_size, &a.tiled, &a.tiles_w, &a.log2s, &a.row))) return rc;
    if (n_groups == 0) return ok();
    if (!x || !y || !packed || !scale || !minv) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(x) || !aligned16(y) || !aligned16(packed)) return fail(DOPT_EINVAL, "x, y and packed must be 16-byte aligned");
    a.x = x;
    a.y = y;
    a.packed = packed;
    a.scale = scale;
    a.minv = minv;
    a.n_groups = (uint32_t)n_groups;
    a.meta_bf16 = meta_dtype == DOPT_BF16;
    const int pre = act == DOPT_ACT_GELU ? dopt::PRE_GELU : dopt::PRE_SILU;
    hipStream_t s = (hipStream_t)stream;
    (void)hipGetLastError();
    if (x_dtype == DOPT_F32)
        rc = dopt::launch_quant_pack_dt<dopt::DT_F32>(a, bits, group_size, dopt::RN_NEAREST, pre, s);
    else
        rc = dopt::launch_quant_pack_dt<dopt::DT_BF16>(a, bits, group_size, dopt::RN_NEAREST, pre, s);
    if (rc) return fail(DOPT_EUNSUPPORTED, "no act_quant_pack kernel for bits=%d g=%d act=%d", bits, group_size, act);
    return hip_status("act_quant_pack launch");
}

int dopt_act_dequant_mul(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype, int64_t n_groups,
                         int group_size, int bits, const int64_t* tile_nchw, const void* dy, int dy_dtype, void* dx,
                         void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0 || n_groups >= (int64_t)1 << 31)
        return fail(DOPT_EINVAL, "n_groups must be in [0, 2^31), got %lld", (long long)n_groups);
    if (meta_dtype != DOPT_F32 && meta_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "scale/min dtype must be F32 or BF16, got code %d", meta_dtype);
    if (dy_dtype != DOPT_F32 && dy_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "act_dequant_mul: dy dtype must be F32 or BF16, got code %d", dy_dtype);
    dopt::DequantArgs a{};
    if ((rc = setup_tiles(tile_nchw, n_groups, group_size, &a.tiled, &a.tiles_w, &a.log2s, &a.row))) return rc;
    if (n_groups == 0) return ok();
    if (!packed || !scale || !minv || !dy || !dx) return fail(DOPT_EINVAL, "null pointer argument");
    if (!aligned16(dx) || !aligned16(dy) || ((uintptr_t)packed & 7u))
        return fail(DOPT_EINVAL, "dx and dy must be 16-byte and packed 8-byte aligned");
    a.dy = dy;
    a.packed = packed;
    a.scale = scale;
    a.minv = minv;
    a.y = dx;
    a.n_groups = (uint32_t)n_groups;
    a.meta_bf16 = meta_dtype == DOPT_BF16;
    (void)hipGetLastError();
    rc = dopt::launch_dequant_unpack_dt<dopt::DT_BF16>(a, bits, group_size,
                                                       dy_dtype == DOPT_F32 ? dopt::DT_F32 : dopt::DT_BF16,
                                                       (hipStream_t)stream);
    if (rc) return fail(DOPT_EUNSUPPORTED, "no act_dequant_mul kernel for bits=%d g=%d", bits, group_size);
    return hip_status("act_dequant_mul launch");
}

int dopt_act_dequant_mul_alam(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype,
                              int64_t n_groups, int group_size, int bits, const int64_t* tile_nchw, const void* dy,
                              int dy_dtype, uint64_t seed, void* dx, void* stream) {
    int rc;
    if ((rc = check_bits(bits))) return rc;
    if ((rc = check_group(group_size))) return rc;
    if (n_groups < 0 || n_groups >= (int64_t)1 << 31)
        return fail(DOPT_EINVAL, "n_groups must be in [0, 2^31), got %lld", (long long)n_groups);
    if (meta_dtype != DOPT_F32 && meta_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "scale/min dtype must be F32 or BF16, got code %d", meta_dtype);
    if (dy_dtype != DOPT_F32 && dy_dtype != DOPT_BF16)
        return fail(DOPT_EINVAL, "act_dequant_mul_alam: dy dtype must be F32 or BF16, got code %d", dy_dtype);
    dopt::DequantArgs a{};
    if ((rc = setup_tiles(tile_nchw, n_groups, group_size, &a.tiled, &a.tiles_w, &a.log2s, &a.row))) return rc;
    if (n_groups == 0) return ok();
    if (!packed || !scale || !minv || !dy || !dx) return fail(DOPT_EINVAL, "null pointer argument");
    a.dy = dy;
    a.packed = packed;
    a.scale = scale;
    a.minv = minv;
    a.y = dx;
    a.n_groups = (uint32_t)n_groups;
    a.meta_bf16 = meta_dtype == DOPT_BF16;
    (void)hipGetLastError();
    dopt::launch_alam_act_dequant_mul(a, group_size, bits, dy_dtype == DOPT_F32, seed, (hipStream_t)stream);
    return hip_status("act_dequant_mul_alam launch");
}

int64_t dopt_bn_workspace_floats(int64_t N, int64_t C, int64_t HW) {
    if (N < 0 || C < 0 || HW < 0) return 0;
    return 2 * C * dopt::bn_nchunks(N * HW);
}

int dopt_bn_reduce(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c,
                   float* workspace, float* sum, float* sumsq, void* stream) {
    int rc;
    dopt::BnGeom g;
    if ((rc = bn_geom(N, C, HW, stride_n, stride_c, &g))) return rc;
    if ((rc = bn_dtype(x_dtype, "bn_reduce: x"))) return rc;
    if (C == 0) return ok();
    if (!sum || !sumsq || (N * HW > 0 && (!x || !workspace))) return fail(DOPT_EINVAL, "null pointer argument");
    (void)hipGetLastError();
    dopt::launch_bn_reduce(x, x_dtype, g, workspace, sum, sumsq, bn_width(g, {{x, bn_bytes(x_dtype)}}),
                           (hipStream_t)stream);
    return hip_status("bn_reduce launch");
}

static int bn_norm_quant_impl(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                              int64_t stride_c, const float* sum, const float* sumsq, const float* mean_in,
                              const float* invstd_in, int sync, const float* weight, const float* bias, float eps,
                              int mode, int group_size, int bits, int alam_lg, void* y, void* x_hat, uint32_t* packed,
                              uint32_t* relu_packed, void* scale, void* minv, float* mean_out, float* var_out,
                              void* stream) {
    int rc;
    dopt::BnGeom g;
    if ((rc = bn_geom(N, C, HW, stride_n, stride_c, &g))) return rc;
    if ((rc = bn_dtype(x_dtype, "bn_norm_quant: x"))) return rc;
    const int64_t M = N * HW;
    if ((rc = bn_quant_checks(mode, M, group_size, bits, packed, scale, minv, relu_packed))) return rc;
    if (C == 0 || M == 0) return ok();
    if (!x || !y || !weight || !bias) return fail(DOPT_EINVAL, "null x/y/weight/bias pointer");
    if (sync ? (!mean_in || !invstd_in) : (!sum || !sumsq || !mean_out || !var_out))
        return fail(DOPT_EINVAL, "null statistics pointer (sync=%d)", sync);
    if (mode == DOPT_BN_NORM && !x_hat) return fail(DOPT_EINVAL, "null x_hat pointer");
    dopt::BnFwdArgs a{};
    a.g = g;
    a.x = x;
    a.sum = sum;
    a.sumsq = sumsq;
    a.mean_in = mean_in;
    a.invstd_in = invstd_in;
    a.w = weight;
    a.b = bias;
    a.eps = eps;
    a.sync = sync != 0;
    a.y = (uint16_t*)y;
    a.xhat = (uint16_t*)x_hat;
    a.packed = packed;
    a.relu_packed = relu_packed;
    a.scale = (uint16_t*)scale;
    a.minv = (uint16_t*)minv;
    a.mean_out = mean_out;
    a.var_out = var_out;
    a.alam_lg = alam_lg;
    (void)hipGetLastError();
    dopt::launch_bn_fwd(a, x_dtype, mode, group_size, bits,
                        bn_width(g, {{x, bn_bytes(x_dtype)}, {y, 2}, {x_hat, 2}}), (hipStream_t)stream);
    return hip_status("bn_norm_quant launch");
}

int dopt_bn_norm_quant(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                       int64_t stride_c, const float* sum, const float* sumsq, const float* mean_in,
                       const float* invstd_in, int sync, const float* weight, const float* bias, float eps, int mode,
                       int group_size, int bits, void* y, void* x_hat, uint32_t* packed, uint32_t* relu_packed,
                       void* scale, void* minv, float* mean_out, float* var_out, void* stream) {
    return bn_norm_quant_impl(x, x_dtype, N, C, HW, stride_n, stride_c, sum, sumsq, mean_in, invstd_in, sync, weight,
                              bias, eps, mode, group_size, bits, 0, y, x_hat, packed, relu_packed, scale, minv,
                              mean_out, var_out, stream);
}

int dopt_bn_norm_quant_alam(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                            int64_t stride_c, const float* sum, const float* sumsq, const float* mean_in,
                            const float* invstd_in, int sync, const float* weight, const float* bias, float eps,
                            int group_size, int bits, int alam_bits, void* y, uint32_t* packed, void* scale,
                            void* minv, float* mean_out, float* var_out, void* stream) {
    int rc, lg = 0;
    if ((rc = bn_alam_lg(group_size, bits, alam_bits, &lg))) return rc;
    return bn_norm_quant_impl(x, x_dtype, N, C, HW, stride_n, stride_c, sum, sumsq, mean_in, invstd_in, sync, weight,
                              bias, eps, DOPT_BN_QUANT, group_size, bits, lg, y, nullptr, packed, nullptr, scale, minv,
                              mean_out, var_out, stream);
}

}  // extern "C"

namespace {

// dopt_bn_train_forward with the workspace either the caller's (noalloc = false) or this device's
// static scratch (noalloc = true, looked up after the arguments are validated).
int bn_train_forward_impl(bool noalloc, const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW,
                          int64_t stride_n, int64_t stride_c, float* workspace, const float* weight, const float* bias,
                          float eps, int mode, int group_size, int bits, void* y, void* x_hat, uint32_t* packed,
                          uint32_t* relu_packed, void* scale, void* minv, float* mean_out, float* var_out,
                          float* running_mean, float* running_var, float momentum, void* stream) {
    int rc;
    const char* name = noalloc ? "bn_train_forward_noalloc" : "bn_train_forward";
    dopt::BnGeom g;
    if ((rc = bn_geom(N, C, HW, stride_n, stride_c, &g))) return rc;
    if ((rc = bn_dtype(x_dtype, noalloc ? "bn_train_forward_noalloc: x" : "bn_train_forward: x"))) return rc;
    const int64_t M = N * HW;
    if ((rc = bn_quant_checks(mode, M, group_size, bits, packed, scale, minv, relu_packed))) return rc;
    if (noalloc) {
        const int64_t need = 2 * C * dopt::bn_nchunks(M);
        if (need > DOPT_BN_SCRATCH_FLOATS)
            return fail(DOPT_EINVAL,
                        "%s: N=%lld C=%lld HW=%lld needs %lld floats of scratch, more than the %d the static "
                        "scratch holds (use dopt_bn_train_forward with a workspace)",
                        name, (long long)N, (long long)C, (long long)HW, (long long)need, DOPT_BN_SCRATCH_FLOATS);
    }
    if (C == 0 || M == 0) return ok();
    if (!x || !y || !weight || !bias || !mean_out || !var_out || (!noalloc && !workspace))
        return fail(DOPT_EINVAL, "%s: null pointer argument", name);
    if (noalloc && (rc = scratch_of_current_device(&workspace))) return rc;
    if (mode == DOPT_BN_NORM && !x_hat) return fail(DOPT_EINVAL, "null x_hat pointer");
    const int vw = bn_width(g, {{x, bn_bytes(x_dtype)}, {y, 2}, {x_hat, 2}});
    (void)hipGetLastError();
    // workgroup partials only: the normalize kernel sums them itself (no finalize launch)
    dopt::launch_bn_reduce(x, x_dtype, g, workspace, nullptr, nullptr, bn_width(g, {{x, bn_bytes(x_dtype)}}),
                           (hipStream_t)stream, false);
    dopt::BnFwdArgs a{};
    a.g = g;
    a.x = x;
    a.partial = workspace;
    a.nchunks = dopt::bn_nchunks(M);
    a.w = weight;
    a.b = bias;
    a.eps = eps;
    a.sync = 0;
    a.y = (uint16_t*)y;
    a.xhat = (uint16_t*)x_hat;
    a.packed = packed;
    a.relu_packed = relu_packed;
    a.scale = (uint16_t*)scale;
    a.minv = (uint16_t*)minv;
    a.mean_out = mean_out;
    a.var_out = var_out;
    a.run_mean = running_mean;
    a.run_var = running_var;
    a.run_mom = momentum;
    a.run_keep = (float)(1.0 - (double)momentum);
    dopt::launch_bn_fwd(a, x_dtype, mode, group_size, bits, vw, (hipStream_t)stream);
    return hip_status(noalloc ? "bn_train_forward_noalloc launch" : "bn_train_forward launch");
}

}  // namespace

extern "C" {

int dopt_bn_train_forward(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                          int64_t stride_c, float* workspace, const float* weight, const float* bias, float eps,
                          int mode, int group_size, int bits, void* y, void* x_hat, uint32_t* packed,
                          uint32_t* relu_packed, void* scale, void* minv, float* mean_out, float* var_out,
                          float* running_mean, float* running_var, float momentum, void* stream) {
    return bn_train_forward_impl(false, x, x_dtype, N, C, HW, stride_n, stride_c, workspace, weight, bias, eps, mode,
                                 group_size, bits, y, x_hat, packed, relu_packed, scale, minv, mean_out, var_out,
                                 running_mean, running_var, momentum, stream);
}

int dopt_bn_train_forward_noalloc(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                                  int64_t stride_c, const float* weight, const float* bias, float eps, int mode,
                                  int group_size, int bits, void* y, void* x_hat, uint32_t* packed,
                                  uint32_t* relu_packed, void* scale, void* minv, float* mean_out, float* var_out,
                                  float* running_mean, float* running_var, float momentum, void* stream) {
    return bn_train_forward_impl(true, x, x_dtype, N, C, HW, stride_n, stride_c, nullptr, weight, bias, eps, mode,
                                 group_size, bits, y, x_hat, packed, relu_packed, scale, minv, mean_out, var_out,
                                 running_mean, running_var, momentum, stream);
}

int dopt_bn_train_backward(int mode, const uint32_t* packed, const uint32_t* relu_packed, const void* scale,
                           const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C, int64_t HW,
                           int64_t stride_n, int64_t stride_c, int group_size, int bits, float* workspace,
                           const float* weight, const float* var, float eps, float* dweight, float* dbias, void* dx,
                           void* stream) {
    int rc;
    dopt::BnGeom g;
    if ((rc = bn_geom(N, C, HW, stride_n, stride_c, &g))) return rc;
    if ((rc = bn_dtype(dy_dtype, "bn_train_backward: dy"))) return rc;
    if (mode == DOPT_BN_NORM) return fail(DOPT_EINVAL, "bn_train_backward takes the quantized modes");
    const int64_t M = N * HW;
    if ((rc = bn_quant_checks(mode, M, group_size, bits, packed, scale, minv, relu_packed))) return rc;
    if (C == 0 || M == 0) return ok();
    if (!dy || !dx || !dweight || !dbias || !weight || !var || !workspace) return fail(DOPT_EINVAL, "null pointer argument");
    dopt::BnBwdArgs a{};
    a.g = g;
    a.packed = packed;
    a.relu_packed = relu_packed;
    a.scale = (const uint16_t*)scale;
    a.minv = (const uint16_t*)minv;
    a.dy = dy;
    a.partial = workspace;
    a.nchunks = dopt::bn_nchunks(M);
    a.dw = dweight;
    a.db = dbias;
    a.dw_in = nullptr;  // the dx kernel sums the partials and writes dweight / dbias
    a.db_in = nullptr;
    a.w = weight;
    a.var = var;
    a.eps = eps;
    a.var_is_invstd = 0;
    a.dx = (uint16_t*)dx;
    (void)hipGetLastError();
    dopt::launch_bn_bwd_reduce(a, dy_dtype, mode, group_size, bits, bn_width(g, {{dy, bn_bytes(dy_dtype)}}),
                               (hipStream_t)stream, false);
    dopt::launch_bn_bwd_dx(a, dy_dtype, mode, group_size, bits, bn_width(g, {{dy, bn_bytes(dy_dtype)}, {dx, 2}}),
                           (hipStream_t)stream);
    return hip_status("bn_train_backward launch");
}

static int bn_bwd_reduce_impl(int mode, const void* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                              const void* scale, const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C,
                              int64_t HW, int64_t stride_n, int64_t stride_c, int group_size, int bits, int alam,
                              int alam_lg, float* workspace, float* dweight, float* dbias, void* stream) {
    int rc;
    dopt::BnGeom g;
    if ((rc = bn_geom(N, C, HW, stride_n, stride_c, &g))) return rc;
    if ((rc = bn_dtype(dy_dtype, "bn_bwd_reduce: dy"))) return rc;
    const int64_t M = N * HW;
    if ((rc = bn_quant_checks(mode, M, group_size, bits, packed, scale, minv, relu_packed))) return rc;
    if (C == 0) return ok();
    if (!dweight || !dbias) return fail(DOPT_EINVAL, "null dweight/dbias pointer");
    if (M > 0 && (!dy || !workspace || (mode == DOPT_BN_NORM && !x_hat)))
        return fail(DOPT_EINVAL, "null dy/workspace/x_hat pointer");
    dopt::BnBwdArgs a{};
    a.g = g;
    a.xhat = (const uint16_t*)x_hat;
    a.packed = packed;
    a.relu_packed = relu_packed;
    a.scale = (const uint16_t*)scale;
    a.minv = (const uint16_t*)minv;
    a.dy = dy;
    a.partial = workspace;
    a.dw = dweight;
    a.db = dbias;
    a.alam = alam;
    a.alam_lg = alam_lg;
    (void)hipGetLastError();
    dopt::launch_bn_bwd_reduce(a, dy_dtype, mode, group_size, bits,
                               bn_width(g, {{dy, bn_bytes(dy_dtype)}, {mode == DOPT_BN_NORM ? x_hat : nullptr, 2}}),
                               (hipStream_t)stream);
    return hip_status("bn_bwd_reduce launch");
}

int dopt_bn_bwd_reduce(int mode, const void* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                       const void* scale, const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C,
                       int64_t HW, int64_t stride_n, int64_t stride_c, int group_size, int bits, float* workspace,
                       float* dweight, float* dbias, void* stream) {
    return bn_bwd_reduce_impl(mode, x_hat, packed, relu_packed, scale, minv, dy, dy_dtype, N, C, HW, stride_n,
                              stride_c, group_size, bits, 0, 0, workspace, dweight, dbias, stream);
}

int dopt_bn_bwd_reduce_alam(const uint32_t* packed, const void* scale, const void* minv, const void* dy, int dy_dtype,
                            int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c, int group_size,
                            int bits, int alam_bits, float* workspace, float* dweight, float* dbias, void* stream) {
    int rc, lg = 0;
    if ((rc = bn_alam_lg(group_size, bits, alam_bits, &lg))) return rc;
    return bn_bwd_reduce_impl(DOPT_BN_QUANT, nullptr, packed, nullptr, scale, minv, dy, dy_dtype, N, C, HW, stride_n,
                              stride_c, group_size, bits, 1, lg, workspace, dweight, dbias, stream);
}

static int bn_bwd_dx_impl(int mode, const void* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                          const void* scale, const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C,
                          int64_t HW, int64_t stride_n, int64_t stride_c, int group_size, int bits, int alam_lg,
                          const float* dweight, const float* dbias, const float* weight, const float* var, float eps,
                          int var_is_invstd, void* dx, void* stream) {
    int rc;
    dopt::BnGeom g;
    if ((rc = bn_geom(N, C, HW, stride_n, stride_c, &g))) return rc;
    if ((rc = bn_dtype(dy_dtype, "bn_bwd_dx: dy"))) return rc;
    const int64_t M = N * HW;
    if ((rc = bn_quant_checks(mode, M, group_size, bits, packed, scale, minv, relu_packed))) return rc;
    if (C == 0 || M == 0) return ok();
    if (!dy || !dx || !dweight || !dbias || !weight || !var || (mode == DOPT_BN_NORM && !x_hat))
        return fail(DOPT_EINVAL, "null pointer argument");
    dopt::BnBwdArgs a{};
    a.g = g;
    a.xhat = (const uint16_t*)x_hat;
    a.packed = packed;
    a.relu_packed = relu_packed;
    a.scale = (const uint16_t*)scale;
    a.minv = (const uint16_t*)minv;
    a.dy = dy;
    a.dw_in = dweight;
    a.db_in = dbias;
    a.w = weight;
    a.var = var;
    a.eps = eps;
    a.var_is_invstd = var_is_invstd != 0;
    a.dx = (uint16_t*)dx;
    a.alam = alam_lg > 0;
    a.alam_lg = alam_lg;
    (void)hipGetLastError();
    dopt::launch_bn_bwd_dx(a, dy_dtype, mode, group_size, bits,
                           bn_width(g, {{dy, bn_bytes(dy_dtype)}, {dx, 2}, {mode == DOPT_BN_NORM ? x_hat : nullptr, 2}}),
                           (hipStream_t)stream);
    return hip_status("bn_bwd_dx launch");
}

int dopt_bn_bwd_dx(int mode, const void* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                   const void* scale, const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C, int64_t HW,
                   int64_t stride_n, int64_t stride_c, int group_size, int bits, const float* dweight,
                   const float* dbias, const float* weight, const float* var, float eps, int var_is_invstd, void* dx,
                   void* stream) {
    return bn_bwd_dx_impl(mode, x_hat, packed, relu_packed, scale, minv, dy, dy_dtype, N, C, HW, stride_n, stride_c,
                          group_size, bits, 0, dweight, dbias, weight, var, eps, var_is_invstd, dx, stream);
}

int dopt_bn_bwd_dx_alam(const uint32_t* packed, const void* scale, const void* minv, const void* dy, int dy_dtype,
                        int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c, int group_size,
                        int bits, int alam_bits, const float* dweight, const float* dbias, const float* weight,
                        const float* var, float eps, int var_is_invstd, void* dx, void* stream) {
    int rc, lg = 0;
    if ((rc = bn_alam_lg(group_size, bits, alam_bits, &lg))) return rc;
    return bn_bwd_dx_impl(DOPT_BN_QUANT, nullptr, packed, nullptr, scale, minv, dy, dy_dtype, N, C, HW, stride_n,
                          stride_c, group_size, bits, lg, dweight, dbias, weight, var, eps, var_is_invstd, dx, stream);
}

int64_t dopt_dw_gemm_workspace_floats(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K < 0 || M % 256 || N % 256) return 0;  // unsupported shapes need none
    return dopt::dw_workspace_floats(M, N, K);
}

int dopt_dw_gemm(const void* dy, int64_t ldd, const void* x_hat, int64_t ldx, const uint32_t* packed,
                 const void* scale, const void* minv, int group_size, int bits, int64_t M, int64_t N, int64_t K,
                 float* workspace, float* dw_f32, void* dw_bf16, float* db, void* stream) {
    int rc;
    if (M <= 0 || N <= 0 || K < 0 || M % 256 || N % 256)
        return fail(DOPT_EUNSUPPORTED, "dw_gemm needs M and N positive multiples of 256 (got M=%lld N=%lld K=%lld)",
                    (long long)M, (long long)N, (long long)K);
    if (M * N >= ((int64_t)1 << 40) || K >= ((int64_t)1 << 31))
        return fail(DOPT_EINVAL, "dw_gemm shape too large");
    if ((K > 0 && !dy) || !workspace || (!dw_f32 && !dw_bf16))
        return fail(DOPT_EINVAL, "null dy/workspace/output pointer");
    if (ldd < M || ldd % 8 || !aligned16(dy)) return fail(DOPT_EINVAL, "dy must be 16-byte aligned with ldd >= M, ldd %% 8 == 0");
    if (((uintptr_t)workspace & 15u) || (dw_f32 && ((uintptr_t)dw_f32 & 15u)) || (dw_bf16 && ((uintptr_t)dw_bf16 & 7u)))
        return fail(DOPT_EINVAL, "workspace / dw_f32 must be 16-byte and dw_bf16 8-byte aligned");
    dopt::DwArgs a{};
    a.dy = (const uint16_t*)dy;
    a.ldd = ldd;
    a.M = M;
    a.N = N;
    a.K = K;
    a.partial = workspace;
    int mode;
    if (x_hat || (K == 0 && !packed)) {
        if (ldx < N || ldx % 8 || !aligned16(x_hat))
            return fail(DOPT_EINVAL, "x_hat must be 16-byte aligned with ldx >= N, ldx %% 8 == 0");
        a.xh = (const uint16_t*)x_hat;
        a.ldx = ldx;
        mode = dopt::DW_B_BF16;
    } else {
        if ((rc = check_bits(bits))) return rc;
        if ((rc = check_group(group_size))) return rc;
        if (!packed || !scale || !minv) return fail(DOPT_EINVAL, "null packed/scale/min pointer");
        if ((uintptr_t)packed & 7u) return fail(DOPT_EINVAL, "packed must be 8-byte aligned");
        a.packed = packed;
        a.scale = (const uint16_t*)scale;
        a.minv = (const uint16_t*)minv;
        a.bits = bits;
        a.lg = ilog2(group_size);
        mode = dopt::DW_B_PACKED;
    }
    (void)hipGetLastError();
    dopt::launch_dw_gemm(a, mode, db != nullptr, dw_f32, (uint16_t*)dw_bf16, db, (hipStream_t)stream);
    return hip_status("dw_gemm launch");
}

}  // extern "C"

int dopt_graph_node_counts(void* graph, int64_t* counts, int n_counts) {
    if (!graph || (!counts && n_counts > 0) || n_counts < 0) return fail(DOPT_EINVAL, "null graph or counts");
    for (int i = 0; i < n_counts; ++i) counts[i] = 0;
    if (const char* e = dopt::graph_node_counts((hipGraph_t)graph, counts, n_counts))
        return fail(DOPT_EHIP, "graph_node_counts: %s failed", e);
    return ok();
}

int dopt_graph_replace_memsets(void* graph, int64_t* n_replaced) {
    if (!graph || !n_replaced) return fail(DOPT_EINVAL, "null graph or n_replaced");
    *n_replaced = 0;
    if (const char* e = dopt::graph_replace_memsets((hipGraph_t)graph, n_replaced))
        return fail(DOPT_EHIP, "graph_replace_memsets: %s failed after %lld replacements", e, (long long)*n_replaced);
    return ok();
}
