// Bandwidth-ceiling probe for the quant-pack kernel's byte mix: the same reads and writes with
// no arithmetic, so a benchmark can report how close the real kernel comes to what the memory
// system delivers for that mix (reads of two streams interleaved with a small write stream).
//
// Unit u = 8 elements: reads 16 bytes of x (8 bf16) and, with noise, 32 bytes of noise (8 fp32);
// with BITS > 0 writes BITS bytes of "codes" (8 codes of BITS bits) and, every 32 units (one
// 256-element group), 8 bytes of "scale/min". Consecutive lanes take consecutive units, as the
// quant-pack kernel's lanes take consecutive 16-byte pieces of a group. The bytes written are a
// hash of the bytes read: they only keep the loads alive.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "dopt_probe.h"
#include "quant_pack.h"  // the quantizer's division helpers, checked by valu kind 8

namespace dopt {
namespace {

constexpr int PROBE_THREADS = 256;

template <int BITS, bool NOISE>
__global__ __launch_bounds__(PROBE_THREADS) void stream_mix_kernel(const uint4* __restrict__ x,
                                                                   const uint4* __restrict__ noise,
                                                                   uint8_t* __restrict__ codes,
                                                                   uint32_t* __restrict__ meta, uint64_t n_units) {
    const uint64_t u = (uint64_t)blockIdx.x * PROBE_THREADS + threadIdx.x;
    if (u >= n_units) return;
    const uint4 a = x[u];
    uint32_t h = a.x ^ a.y ^ a.z ^ a.w;
    if constexpr (NOISE) {
        const uint4 b = noise[2 * u], c = noise[2 * u + 1];
        h ^= b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w;
    }
    if constexpr (BITS == 0) {
        if (h == 0x9E3779B9u) codes[0] = 1;  // practically never taken; keeps the loads
    } else {
        if constexpr (BITS == 1) codes[u] = (uint8_t)h;
        if constexpr (BITS == 2) ((uint16_t*)codes)[u] = (uint16_t)h;
        if constexpr (BITS == 4) ((uint32_t*)codes)[u] = h;
        if constexpr (BITS == 8) ((uint2*)codes)[u] = make_uint2(h, h >> 7);
        if ((u & 31) == 0) ((uint2*)meta)[u >> 5] = make_uint2(h, h >> 3);
    }
}

template <int BITS, bool NOISE>
hipError_t launch(const void* x, const void* noise, void* codes, void* meta, uint64_t n, hipStream_t s) {
    const uint64_t blocks = (n + PROBE_THREADS - 1) / PROBE_THREADS;
    hipLaunchKernelGGL((stream_mix_kernel<BITS, NOISE>), dim3((uint32_t)blocks), dim3(PROBE_THREADS), 0, s,
                       (const uint4*)x, (const uint4*)noise, (uint8_t*)codes, (uint32_t*)meta, n);
    return hipGetLastError();
}

// Issue-rate probe: every lane runs 8 independent chains of VALU_STEPS steps of one instruction
// kind and writes one value, so a launch of many waves measures the time per wave-instruction
// of that kind on a SIMD (the cost model behind the instruction-bound kernels' roofline).
constexpr int VALU_STEPS = 512;

template <int KIND>
__global__ __launch_bounds__(PROBE_THREADS) void valu_rate_kernel(float* __restrict__ out, float seed) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = seed + 0.01f * (float)(threadIdx.x + j);
    const float b = seed * 0.5f, c = seed * 0.25f;
    for (int i = 0; i < VALU_STEPS; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (KIND == 0) v[j] = __builtin_fmaf(v[j], b, c);            // v_fma_f32
            if constexpr (KIND == 1) v[j] = __builtin_amdgcn_exp2f(-v[j]);          // v_exp_f32
            if constexpr (KIND == 2) v[j] = __builtin_amdgcn_rcpf(v[j]);            // v_rcp_f32
            if constexpr (KIND == 3) {                                              // v_mad_u64_u32 + v_xor
                const uint64_t p = (uint64_t)__float_as_uint(v[j]) * 0xD2511F53u;
                v[j] = __uint_as_float((uint32_t)(p >> 32) ^ (uint32_t)p);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
    out[(uint64_t)blockIdx.x * PROBE_THREADS + threadIdx.x] = s;
}

// MFMA-stream probe in the shape of the weight-gradient GEMM's inner loop: each wave keeps a 4 x 4
// grid of 32 x 32 fp32 accumulators (256 per lane, one wave per SIMD) and per step issues the 16
// v_mfma_f32_32x32x16_bf16 acc[i][j] += A[i] B[j], with nothing else in the loop. RANDOM: the 4 + 4
// operand fragments hold pseudo-random bf16 values in (-1, 1) that differ per lane and fragment;
// otherwise every fragment is one constant. The operand data changes the sustained MFMA rate.
constexpr int MFMA_STEPS = 64;
typedef __bf16 probe_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float probe_f32x16_t __attribute__((ext_vector_type(16)));

template <bool RANDOM>
__global__ __launch_bounds__(PROBE_THREADS, 1) void mfma_rate_kernel(float* __restrict__ out) {
    probe_bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t h = (threadIdx.x * 8u + (uint32_t)e) * 2654435761u ^ (uint32_t)(i + 1) * 40503u;
            h ^= h >> 15;
            const float ra = RANDOM ? (float)(h & 0xffffu) / 32768.0f - 1.0f : 0.5f;
            const float rb = RANDOM ? (float)(h >> 16) / 32768.0f - 1.0f : 0.5f;
            a[i][e] = (__bf16)ra;
            b[i][e] = (__bf16)rb;
        }
    probe_f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    for (int st = 0; st < MFMA_STEPS; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) t += acc[i][j][0] + acc[i][j][15];
    out[(uint64_t)blockIdx.x * PROBE_THREADS + threadIdx.x] = t;
}

// The same for the FP8 GEMM's instruction, v_mfma_scale_f32_32x32x64_f8f6f4 with e4m3 operands
// and unit scales: 4 x 4 accumulators per wave, 4 + 4 fragments of 32 bytes per lane. RANDOM:
// pseudo-random e4m3 bytes (finite, |v| <= 448), otherwise one constant byte.
typedef int probe_v8i_t __attribute__((ext_vector_type(8)));

template <bool RANDOM>
__global__ __launch_bounds__(PROBE_THREADS, 1) void mfma_fp8_rate_kernel(float* __restrict__ out) {
    probe_v8i_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t h = (threadIdx.x * 8u + (uint32_t)e) * 2654435761u ^ (uint32_t)(i + 1) * 40503u;
            h ^= h >> 13;
            // clear bit 6 of each byte: exponent field <= 7 of 15, so no NaN encodings (0x7f / 0xff)
            const uint32_t ra = RANDOM ? (h & 0xbfbfbfbfu) : 0x38383838u;
            const uint32_t rb = RANDOM ? ((h * 0x9E3779B9u) & 0xbfbfbfbfu) : 0x38383838u;
            a[i][e] = (int)ra;
            b[i][e] = (int)rb;
        }
    probe_f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    for (int st = 0; st < MFMA_STEPS; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i], b[j], acc[i][j], 0, 0, 0, 0, 0, 0);
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) t += acc[i][j][0] + acc[i][j][15];
    out[(uint64_t)blockIdx.x * PROBE_THREADS + threadIdx.x] = t;
}

// The quantizer's fast exact-division helpers against the IEEE division, over every non-negative
// fp32 bit pattern (+0 .. +inf, strided over the grid): div_by_qmax<3/15/255>(x) against x / QMAX,
// div_by_qmax_rt with the divisor 2^bits - 1 known only at run time (bits = 1, 2, 4, 8, taken from
// the launch width, which the compiler cannot fold) against x / qmax, and exact_rcp(x) against
// 1 / x. Each thread writes its count of differing bit patterns.
__global__ __launch_bounds__(PROBE_THREADS) void division_check_kernel(float* __restrict__ out) {
    const uint32_t t = blockIdx.x * PROBE_THREADS + threadIdx.x, nt = gridDim.x * PROBE_THREADS;
    const int one = (int)(blockDim.x / PROBE_THREADS);  // 1
    float qm[4], rq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qm[i] = (float)((1 << (one << i)) - 1);  // 1, 3, 15, 255
        rq[i] = 1.0f / qm[i];
    }
    uint32_t bad = 0;
    for (uint32_t u = t; u <= 0x7F800000u; u += nt) {
        const float x = __uint_as_float(u);
        bad += __float_as_uint(div_by_qmax<3>(x)) != __float_as_uint(x / 3.0f);
        bad += __float_as_uint(div_by_qmax<15>(x)) != __float_as_uint(x / 15.0f);
        bad += __float_as_uint(div_by_qmax<255>(x)) != __float_as_uint(x / 255.0f);
#pragma unroll
        for (int i = 0; i < 4; ++i) bad += __float_as_uint(div_by_qmax_rt(x, qm[i], rq[i])) != __float_as_uint(x / qm[i]);
        bad += __float_as_uint(exact_rcp(x)) != __float_as_uint(1.0f / x);
    }
    out[(uint64_t)blockIdx.x * PROBE_THREADS + threadIdx.x] = (float)bad;
}

}  // namespace

// kind 0..3 (fma, exp, rcp, mad64 + xor), 4 / 5 (bf16 MFMA stream, random / constant operands),
// 6 / 7 (fp8 MFMA stream, random / constant operands), 8 (exact-division check: per-thread counts
// of mismatches, 0 expected); out holds n_blocks * 256 floats
static const char* launch_valu_rate(int kind, float* out, uint32_t n_blocks, hipStream_t s) {
    switch (kind) {
        case 8: hipLaunchKernelGGL(division_check_kernel, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out); break;
        case 6: hipLaunchKernelGGL(mfma_fp8_rate_kernel<true>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out); break;
        case 7: hipLaunchKernelGGL(mfma_fp8_rate_kernel<false>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out); break;
        case 4: hipLaunchKernelGGL(mfma_rate_kernel<true>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out); break;
        case 5: hipLaunchKernelGGL(mfma_rate_kernel<false>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out); break;
        case 0: hipLaunchKernelGGL(valu_rate_kernel<0>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out, 0.3f); break;
        case 1: hipLaunchKernelGGL(valu_rate_kernel<1>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out, 0.3f); break;
        case 2: hipLaunchKernelGGL(valu_rate_kernel<2>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out, 0.3f); break;
        case 3: hipLaunchKernelGGL(valu_rate_kernel<3>, dim3(n_blocks), dim3(PROBE_THREADS), 0, s, out, 0.3f); break;
        default: return "kind";
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? nullptr : hipGetErrorString(e);
}

// bits in {0, 1, 2, 4, 8}; 0 = reads only. Returns nullptr or the name of what failed.
static const char* launch_stream_mix(const void* x, const void* noise, void* codes, void* meta, uint64_t n_units, int bits,
                              hipStream_t s) {
    hipError_t e = hipSuccess;
#define DOPT_SM(B)                                                                               \
    case B:                                                                                      \
        e = noise ? launch<B, true>(x, noise, codes, meta, n_units, s)                           \
                  : launch<B, false>(x, noise, codes, meta, n_units, s);                          \
        break;
    switch (bits) {
        DOPT_SM(0)
        DOPT_SM(1)
        DOPT_SM(2)
        DOPT_SM(4)
        DOPT_SM(8)
        default:
            return "bits";
    }
#undef DOPT_SM
    return e == hipSuccess ? nullptr : hipGetErrorString(e);
}

}  // namespace dopt

namespace {

thread_local char g_probe_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_probe_err, sizeof(g_probe_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_probe_err[0] = '\0';
    return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

const char* dopt_probe_last_error(void) { return g_probe_err; }

int dopt_valu_probe(int kind, float* out, int64_t n_blocks, void* stream) {
    if (kind < 0 || kind > 8)
        return fail(-2,
                    "kind must be 0..8 (fma, exp, rcp, mad64+xor, bf16 MFMA random / constant, fp8 MFMA random / "
                    "constant, exact-division check), got %d", kind);
    if (n_blocks < 1 || n_blocks > 65536) return fail(-2, "n_blocks must be in [1, 65536], got %lld",
                                                      (long long)n_blocks);
    if (!out || ((uintptr_t)out & 3u)) return fail(-2, "out must be a 4-byte aligned pointer");
    (void)hipGetLastError();
    if (const char* e = dopt::launch_valu_rate(kind, out, (uint32_t)n_blocks, (hipStream_t)stream))
        return fail(-4, "valu_probe launch: %s", e);
    return ok();
}

int dopt_stream_probe(const void* x, const void* noise, void* codes, void* meta, int64_t n_units, int bits,
                      void* stream) {
    if (n_units < 0 || n_units > ((int64_t)1 << 31))  // one lane per unit; the grid stays below 2^32 lanes
        return fail(-2, "n_units must be in [0, 2^31], got %lld", (long long)n_units);
    if (bits != 0 && bits != 1 && bits != 2 && bits != 4 && bits != 8)
        return fail(-2, "bits must be 0, 1, 2, 4 or 8, got %d", bits);
    if (n_units == 0) return ok();
    if (!x || !aligned16(x) || (noise && !aligned16(noise))) return fail(-2, "x / noise must be 16-byte aligned");
    if (bits && (!codes || !meta || ((uintptr_t)codes % (uintptr_t)bits) || ((uintptr_t)meta & 7u)))
        return fail(-2, "codes must be bits-byte and meta 8-byte aligned");
    if (!bits && !codes) return fail(-2, "codes must point to at least one byte");
    (void)hipGetLastError();
    if (const char* e = dopt::launch_stream_mix(x, noise, codes, meta, (uint64_t)n_units, bits, (hipStream_t)stream))
        return fail(-4, "stream_probe launch: %s", e);
    return ok();
}

}  // extern "C"
