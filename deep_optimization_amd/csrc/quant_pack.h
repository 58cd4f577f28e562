// gfx950 quant-pack kernel: per-group min/max, 1/2/4/8-bit nearest or stochastic rounding and
// little-endian bit-packing. Semantics follow Activation_Compression/act_triton_kernel.py:53-171
// (nearest) and the stochastic form of cpp_extension/include/quant_common.h:148-156 with the
// Triton step convention; include/dopt.h documents the ABI.
//
// Work decomposition (one wavefront = 64 lanes):
//   - a lane owns "units" of UE contiguous elements (UB bytes, read as UB/16 consecutive 16-byte
//     loads); a group of G elements is CPG = G/UE units spread over LPG lanes, CPL units per lane
//     (unit c = i*LPG + li), so each load instruction covers LPG*UB contiguous bytes per group;
//   - a wave handles GPP = 64/LPG groups per pass and P passes, with every load of the wave
//     issued before any arithmetic;
//   - min/max: lane-local v_min3/v_max3, then a DPP all-reduce over the group's LPG lanes;
//   - codes go straight from registers to HBM: a unit's UE*BITS code bits are one dword (or a
//     2/4-dword vector), narrower pieces are merged across neighbouring lanes with DPP first, so
//     consecutive lanes store consecutive dwords; per-group scale/min of all GPW groups are
//     gathered into lanes 0..GPW-1 and written with one store per array.
//
// Arithmetic (the reference kernels are compiled with FMA contraction on: Triton's default
// enable_fp_fusion and nvcc's default --fmad=true, so `a * b + c` is one rounding):
//   nearest     q = trunc(fma(x - mn, inv, fp32(0.5 - 1e-6)))   act_triton_kernel.py:114, :155
//   stochastic  q = rint(fma(x - mn, inv, u) - 0.5)              quant_common.h:150-151
// Clamp and its exactness argument. For finite x in [mn, mx] with inv = 1/step finite, the exact
// product (x - mn) * inv is at most QMAX * (1 + 2^-22). Nearest rounding adds 0.5 - 1e-6 and
// Philox noise adds u <= 255.5/256, so those two forms stay below QMAX + 1/2 before the
// reference's clamp: the clamp is redundant there and v_cvt_u32_f32 (truncating, NaN -> 0) gives
// the exact code. A caller's noise tensor is different: torch.rand can return u = 1 - 2^-24, and
// fma(t, inv, u) with t * inv = QMAX then rounds to QMAX + 1 (the spacing of fp32 near QMAX + 1 is
// coarser than 2^-24), whose rint is QMAX + 1; noise-tensor rounding therefore always applies the
// reference's clamp (quant_common.h:152, one v_med3 per element). An infinite input or an
// overflowing range gives inv = 0 and a product of 0 or NaN (code 0 either way, as with the
// reference's clamp). The remaining case that needs the clamp is inv = +inf (step < 2^-128, a
// range of a few subnormals); a wave containing such a group takes the clamped path. Local
// min/max use raw v_min3/v_max3 (no NaN canonicalisation); a signalling NaN input would turn a
// lane's partial result into NaN, so a wave with a NaN partial result recomputes min/max with
// IEEE fminf/fmaxf, which ignore NaN operands.
#pragma once

#include "dopt_device.h"

namespace dopt {

// Pre-transform applied before min/max (template parameter PRE of quant_pack_kernel):
//   PRE_NONE  codes of x itself
//   PRE_REF   the reference quantizer's optional clamp(x, +-alpha) and tanh(x/0.5)*0.5 (runtime flags)
//   PRE_GELU  fused GELU layer: y = gelu(x) is written as bf16, the codes are of
//             tanh(clamp(gelu'(x), -3, 3)/0.5)*0.5 with the range floored at 1e-4
//             (AC/modules/activations/kernel_implementation.py:496-535)
//   PRE_SILU  the same for SiLU (kernel_implementation.py:225-243)
// At 1 and 2 bits the fused activations find their codes by comparing the clamped derivative d
// with the group's QMAX thresholds instead of evaluating the squash per element ("threshold
// codes"): the squash s(d) = sigmoid(4d) is increasing, so the group's min / max of s are s of
// the min / max of d, and code >= k exactly when s(d) >= s_k = fma(k - (0.5 - 1e-6), step, min),
// i.e. when d >= t_k = logit(s_k) / 4. Each lane computes the QMAX thresholds of its group once
// (v_rcp_f32 and v_log_f32 each), and an element costs QMAX compares instead of an exp, a
// reciprocal and the code arithmetic. The codes differ from the per-element form only for d within
// the thresholds' fp32 error (about 1e-7) of a boundary; scale and min are computed as before.
enum { PRE_NONE = 0, PRE_REF = 1, PRE_GELU = 2, PRE_SILU = 3 };

struct QuantPackArgs {
    const void* x;
    void* y;  // activation output (PRE_GELU / PRE_SILU): bf16, same layout as x
    const float* noise;
    uint32_t* packed;
    void* scale;
    void* minv;
    uint32_t n_groups;
    uint32_t tiled;    // 0: flat [n_groups, G]; 1: s x s spatial tiles of [N, C, H, W]
    uint32_t tiles_w;  // W / s
    uint32_t log2s;    // log2(s)
    uint64_t row;      // W (elements per image row)
    uint32_t seed_lo, seed_hi, off_lo, off_hi;
    float clamp_alpha;
    uint32_t flags;
    uint32_t meta_bf16;
};

// Philox noise layout: element idx (group-order index r*G + e) belongs to block idx / NOISE_EPC;
// the block number is the Philox counter's low 64 bits (offset in the high 64), the seed is the
// key, and element k of the block takes byte k of the 128-bit output (little-endian word order):
// u = (byte + 0.5) / 256.
constexpr int NOISE_BITS = 8;
constexpr int NOISE_EPC = 128 / NOISE_BITS;  // elements per Philox4x32-10 call

template <int DT, int BITS, int G, int RN, int UB, int LPG_, int P>
struct QuantPackCfg {
    static constexpr int BYTES = DType<DT>::bytes;
    static constexpr int UE = UB / BYTES;  // elements per unit
    static constexpr int LOADS = UB / 16;  // 16-byte loads per unit
    static constexpr int CPG = G / UE;     // units per group
    static constexpr int LPG = LPG_ ? LPG_ : (CPG < 64 ? CPG : 64);  // lanes per group
    static constexpr int CPL = CPG / LPG;  // units per lane
    static constexpr int GPP = 64 / LPG;
    static constexpr int GPW = P * GPP;    // groups per wave
    static constexpr int W = G * BITS / 32;
    static constexpr int UBITS = UE * BITS;  // code bits per unit
    static constexpr int WAVES = 4;
    static_assert(UB % 16 == 0 && UE * BYTES == UB, "unit must be whole 16-byte loads");
    static_assert(CPG * UE == G && LPG * CPL == CPG, "group must split evenly over lanes");
    static_assert(LPG >= 2 && LPG <= 64 && (LPG & (LPG - 1)) == 0, "2..64 lanes per group");
    static_assert(UBITS >= 32 || (32 / UBITS) <= LPG, "narrow units merge within a group");
    static_assert(UBITS <= 128, "a unit stores at most one 16-byte vector");
    static_assert(GPW <= 64, "scale/min gather uses one lane per group");
};

// Element index of element e0 of group r. The layout is a template parameter: evaluated at run
// time, the tile branch was if-converted into every load and store (an integer division by the
// tile count per access), about a fifth of the fused activation kernels' instructions.
template <int G, bool TILED>
__device__ __forceinline__ uint64_t group_elem_index(const QuantPackArgs& a, uint32_t r, uint32_t e0) {
    if constexpr (!TILED) return (uint64_t)r * G + e0;
    // spatial tile gather of tensor_act_reshape_utils.py:115-125: group r = band*(W/s) + tw
    // holds x[.., band's tile row * s + e/s, tw*s + e%s]
    const uint32_t band = r / a.tiles_w;
    const uint32_t tw = r - band * a.tiles_w;
    const uint32_t smask = (1u << a.log2s) - 1u;
    return (((uint64_t)band * a.row) << a.log2s) + ((uint64_t)tw << a.log2s) +
           (uint64_t)(e0 >> a.log2s) * a.row + (e0 & smask);
}

// min/max all-reduce over aligned blocks of LPG lanes; operands are NaN-free or quiet NaNs.
template <int LPG>
__device__ __forceinline__ void group_minmax(float& mn, float& mx) {
    if constexpr (LPG >= 2) {
        mn = vmin_dpp<0xB1>(mn);
        mx = vmax_dpp<0xB1>(mx);
    }
    if constexpr (LPG >= 4) {
        mn = vmin_dpp<0x4E>(mn);
        mx = vmax_dpp<0x4E>(mx);
    }
    if constexpr (LPG >= 8) {
        mn = vmin_dpp<0x141>(mn);
        mx = vmax_dpp<0x141>(mx);
    }
    if constexpr (LPG >= 16) {
        mn = vmin_dpp<0x140>(mn);
        mx = vmax_dpp<0x140>(mx);
    }
    if constexpr (LPG >= 32) swap_minmax<16>(mn, mx);
    if constexpr (LPG >= 64) swap_minmax<32>(mn, mx);
}

// v_cvt_u32_f32: truncating, saturating, NaN -> 0
__device__ __forceinline__ uint32_t cvt_u32(float f) {
    uint32_t d;
    asm("v_cvt_u32_f32 %0, %1" : "=v"(d) : "v"(f));
    return d;
}

// N codes rint(z[0..N-1]) packed little-endian at BITS bits each (N * BITS <= 32) with
// v_cvt_pk_u8_f32, which rounds to nearest even, saturates to [0, 255] and maps NaN to 0 (measured
// on MI355X), and inserts the byte into a dword in one instruction. Codes are gathered byte-wise
// first: partial word D_s holds code CPB*i + s in byte i (CPB = 8/BITS codes per byte), and the
// packed word is the OR of D_s << s*BITS. Equal to OR(cvt_u32(rint(z[k])) << k*BITS) when every
// rint(z[k]) lies in [0, 2^BITS - 1] or z[k] is NaN or in (-0.5, 0]: one instruction per code
// plus CPB - 1 shift-ORs per word, against rint + convert + shift-OR.
template <int BITS, int N>
__device__ __forceinline__ uint32_t pack_rne_codes(const float* z) {
    constexpr int CPB = 8 / BITS;
    constexpr int NB = (N + CPB - 1) / CPB;
    uint32_t acc = 0;
#pragma unroll
    for (int s = 0; s < (CPB < N ? CPB : N); ++s) {
        uint32_t d = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i)
            if (CPB * i + s < N) d = __builtin_amdgcn_cvt_pk_u8_f32(z[CPB * i + s], (uint32_t)i, d);
        acc = s == 0 ? d : (d << (s * BITS)) | acc;
    }
    return acc;
}

template <int DT, int BITS, int G, int RN, int UB, int LPG_, int P, int PRE, bool NT, bool TILED>
__global__ __launch_bounds__(256) void quant_pack_kernel(QuantPackArgs a) {
    using C = QuantPackCfg<DT, BITS, G, RN, UB, LPG_, P>;
    constexpr int UE = C::UE, LOADS = C::LOADS, CPL = C::CPL, LPG = C::LPG, GPP = C::GPP, W = C::W;
    constexpr int UBITS = C::UBITS;
    constexpr int QMAX = (1 << BITS) - 1;
    constexpr int E16 = DType<DT>::per16;  // elements per 16-byte load
    // threshold codes of the fused activations at 1 and 2 bits (see the PRE enum above)
    constexpr bool THR = (PRE == PRE_GELU || PRE == PRE_SILU) && RN == RN_NEAREST && BITS <= 2;

    const int lane = threadIdx.x & 63;
    const int slot = lane / LPG;
    const int li = lane % LPG;
    // below 2^32: n_groups < 2^31, and a grid's blocks past the end add fewer than GRID_ROW * WAVES * GPW
    const uint32_t g0 = (uint32_t)((linear_block() * C::WAVES + (threadIdx.x >> 6)) * C::GPW);
    const char* xb = (const char*)a.x;

    // ---- every load of the wave first: P*CPL units of LOADS 16-byte vectors per lane. Lanes past
    // the last group (n_groups >= 1: the launcher skips empty calls) load the last group again and
    // store nothing; the loads carry no branch, so all of them are in flight together (a load
    // under a lane mask, merged with a default value, waits for its data before the next issues)
    uint4 raw[P][CPL][LOADS];
    uint4 nz[P][CPL][RN == RN_NOISE ? UE / 4 : 1];
    #pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r0 = g0 + p * GPP + slot;
        const uint32_t r = r0 < a.n_groups ? r0 : a.n_groups - 1;
        #pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t e0 = (uint32_t)(i * LPG + li) * UE;
            #pragma unroll
            for (int l = 0; l < LOADS; ++l)
                raw[p][i][l] = ld16<NT>(xb + group_elem_index<G, TILED>(a, r, e0 + l * E16) * C::BYTES);
            if constexpr (RN == RN_NOISE) {
                #pragma unroll
                for (int k = 0; k < UE / 4; ++k) nz[p][i][k] = ld16<NT>(a.noise + (uint64_t)r * G + e0 + 4 * k);
            }
        }
    }

    const float qmaxf = (float)QMAX;
    const float half_m = 0.49999899f;  // fp32(0.5 - 1e-6) = 0x3EFFFFDE
    // threshold codes: the boundary this lane evaluates, k + 1 - (0.5 - 1e-6), k = min(lane % 4, 2)
    const float kq = (float)((lane & 3) < 2 ? (lane & 3) + 1 : 3) - half_m;
    (void)kq;
    float step_p[P], mn_p[P];

    #pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        float v[CPL][UE];
        #pragma unroll
        for (int i = 0; i < CPL; ++i)
            #pragma unroll
            for (int l = 0; l < LOADS; ++l) widen16<DT>(raw[p][i][l], &v[i][l * E16]);
        if constexpr (PRE == PRE_REF) {
            if (a.flags & FL_CLAMP) {
                // one v_med3 per element equals fminf(fmaxf(x, -alpha), alpha) for alpha >= 0,
                // NaN x included (med3 of a NaN and two numbers is their minimum, here -alpha)
                const float al = a.clamp_alpha;
                if (al >= 0.0f) {
#pragma unroll
                    for (int i = 0; i < CPL; ++i)
#pragma unroll
                        for (int k = 0; k < UE; ++k) v[i][k] = __builtin_amdgcn_fmed3f(v[i][k], -al, al);
                } else {
#pragma unroll
                    for (int i = 0; i < CPL; ++i)
#pragma unroll
                        for (int k = 0; k < UE; ++k) v[i][k] = fminf(fmaxf(v[i][k], -al), al);
                }
            }
            if (a.flags & FL_SQUASH) {
#pragma unroll
                for (int i = 0; i < CPL; ++i)
#pragma unroll
                    for (int k = 0; k < UE; ++k) v[i][k] = squash_half_tanh2(v[i][k]);
            }
        } else if constexpr (PRE == PRE_GELU || PRE == PRE_SILU) {
            // activation value (stored bf16) and its squashed derivative tanh(2 clamp(d, -3, 3)) / 2,
            // quantized as s = sigmoid(4 clamp(d, -3, 3)) = tanh(...) / 2 + 1/2: for finite x the
            // derivative is at least -0.17 (GELU; SiLU -0.1), so s >= 0.33 and s - 1/2 is exact
            // (Sterbenz), as is min - 1/2; differences of the shifted values, hence range, step
            // and codes, are those of s itself, and only the group's min is stored shifted
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const uint32_t e0 = (uint32_t)(i * LPG + li) * UE;
                float yv[UE];
#pragma unroll
                for (int k = 0; k < UE; ++k) {
                    float d;
                    if constexpr (PRE == PRE_GELU)
                        gelu_and_grad(v[i][k], yv[k], d);
                    else
                        silu_and_grad(v[i][k], yv[k], d);
                    const float dc = __builtin_amdgcn_fmed3f(d, -3.0f, 3.0f);
                    if constexpr (THR)
                        v[i][k] = dc;
                    else
                        v[i][k] = sigmoid4_fast(dc);
                }
                if (r < a.n_groups) {
#pragma unroll
                    for (int l = 0; l < LOADS; ++l) {
                        const float* o = &yv[l * E16];
                        char* yb = (char*)a.y + group_elem_index<G, TILED>(a, r, e0 + l * E16) * 2;
                        // y is streamed (non-temporal): SiLU's forward 113-114.5 -> 111 us on the ViT MLP
                        // activation, GELU's 116-118 -> 111.8-117 us over boxes
                        if constexpr (E16 == 8)
                            st16<true>(yb, make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]),
                                                      pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7])));
                        else
                            *(uint2*)yb = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
                    }
                }
            }
        }
        // lane-local min/max over the lane's CPL*UE values. Loaded (or clamped) values go
        // through raw v_min3/v_max3 (inline asm: no NaN canonicalisation of the operands). The
        // activation pre-transforms end in v_rcp_f32, whose result a VALU may read only after one
        // wait state, which the compiler enforces for its own instructions but not for inline
        // asm; their values are arithmetic results (canonical), so compiler min/max add nothing.
        // (threshold codes keep the clamped derivative, a v_med3 result: the raw forms apply)
        constexpr bool TRANS_IN = (PRE == PRE_GELU || PRE == PRE_SILU) && !THR;
        float mn = v[0][0], mx = v[0][0];
        #pragma unroll
        for (int j = 1; j + 1 < CPL * UE; j += 2) {
            const float f0 = v[j / UE][j % UE], f1 = v[(j + 1) / UE][(j + 1) % UE];
            if constexpr (TRANS_IN) {
                mn = fminf(mn, fminf(f0, f1));
                mx = fmaxf(mx, fmaxf(f0, f1));
            } else {
                mn = vmin3(mn, f0, f1);
                mx = vmax3(mx, f0, f1);
            }
        }
        // CPL*UE is even: one value is left over
        if constexpr (TRANS_IN) {
            mn = fminf(mn, v[CPL - 1][UE - 1]);
            mx = fmaxf(mx, v[CPL - 1][UE - 1]);
        } else {
            mn = vmin(mn, v[CPL - 1][UE - 1]);
            mx = vmax(mx, v[CPL - 1][UE - 1]);
        }
        if (wave_any(mn != mn || mx != mx)) {
            // a NaN partial result (signalling NaN input, or a lane of only NaNs): IEEE
            // fminf/fmaxf ignore NaN operands; a lane of only NaNs keeps NaN, which the
            // cross-lane min/max below then ignore
            mn = v[0][0];
            mx = v[0][0];
            #pragma unroll
            for (int i = 0; i < CPL; ++i)
                #pragma unroll
                for (int k = 0; k < UE; ++k) {
                    mn = fminf(mn, v[i][k]);
                    mx = fmaxf(mx, v[i][k]);
                }
            mn = __builtin_isnan(mn) ? __uint_as_float(0x7fc00000u) : mn;  // quiet
            mx = __builtin_isnan(mx) ? __uint_as_float(0x7fc00000u) : mx;
        }
        group_minmax<LPG>(mn, mx);
        if constexpr (THR) {  // min / max of the squash are the squash of the derivative's
            mn = sigmoid4_fast(mn);
            mx = sigmoid4_fast(mx);
        }
        mn = mn + 0.0f;  // store -0.0 as +0.0
        float rng = mx - mn;
        if constexpr (PRE == PRE_GELU || PRE == PRE_SILU) rng = fmaxf(rng, 1e-4f);  // kernel_implementation.py:236, :529
        const float step = rng > 0.0f ? div_by_qmax<QMAX>(rng) : 1.0f;
        const float inv = exact_rcp(step);
        step_p[p] = step;
        if constexpr (PRE == PRE_GELU || PRE == PRE_SILU)
            mn_p[p] = mn - 0.5f;
        else
            mn_p[p] = mn;
        // thresholds t_k = logit(s_k) / 4 = (ln 2 / 4) log2(s_k / (1 - s_k)); an s_k >= 1 (beyond
        // the group's max) gives +inf or NaN, which no derivative reaches
        float thr[THR ? QMAX : 1];
        if constexpr (THR && QMAX == 3 && LPG >= 4) {
            // lane k of each aligned quad (k < 3; lane 3 repeats k = 2) computes threshold k, and
            // quad_perm broadcasts hand every lane all three: one evaluation instead of three (a
            // group spans whole quads, so a quad's lanes agree on mn and step)
            const float sk = __builtin_fmaf(kq, step, mn);
            const float tk = 0.17328679513998632f * __builtin_amdgcn_logf(sk * __builtin_amdgcn_rcpf(1.0f - sk));
            thr[0] = dpp_f32<0x00>(tk);
            thr[1] = dpp_f32<0x55>(tk);
            thr[2] = dpp_f32<0xAA>(tk);
        } else if constexpr (THR) {
#pragma unroll
            for (int k = 0; k < QMAX; ++k) {
                const float sk = __builtin_fmaf((float)(k + 1) - half_m, step, mn);
                thr[k] = 0.17328679513998632f * __builtin_amdgcn_logf(sk * __builtin_amdgcn_rcpf(1.0f - sk));
            }
        }
        const bool clampq = !THR && wave_any(inv == __builtin_inff());  // threshold codes need no clamp

        // codes + store; the clamped variant runs only for waves holding a group with inv = +inf
        auto emit = [&](auto clamp_tag) {
            constexpr bool CL = decltype(clamp_tag)::value;
            #pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const uint32_t c = (uint32_t)(i * LPG + li);
                const uint32_t e0 = c * UE;
                float u[UE];
                if constexpr (RN == RN_NOISE) {
                    #pragma unroll
                    for (int k = 0; k < UE / 4; ++k) {
                        u[4 * k + 0] = __uint_as_float(nz[p][i][k].x);
                        u[4 * k + 1] = __uint_as_float(nz[p][i][k].y);
                        u[4 * k + 2] = __uint_as_float(nz[p][i][k].z);
                        u[4 * k + 3] = __uint_as_float(nz[p][i][k].w);
                    }
                } else if constexpr (RN == RN_PHILOX) {
                    // one Philox call per NOISE_EPC elements (a unit holds UE of them)
                    #pragma unroll
                    for (int b0 = 0; b0 < UE; b0 += NOISE_EPC) {
                        const uint64_t idx = (uint64_t)r * G + e0 + b0;
                        const uint64_t blk = idx / NOISE_EPC;
                        const uint4 w4 = philox4x32_10((uint32_t)blk, (uint32_t)(blk >> 32), a.off_lo, a.off_hi,
                                                       a.seed_lo, a.seed_hi);
                        const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
                        const int sub = (int)(idx % NOISE_EPC);  // 0 unless UE < NOISE_EPC
                        #pragma unroll
                        for (int k = 0; k < (UE < NOISE_EPC ? UE : NOISE_EPC); ++k) {
                            const int kk = sub + k;
                            u[b0 + k] = philox_byte_to_u(w[kk >> 2], kk & 3);
                        }
                    }
                }
                // UBITS code bits of this unit, little-endian
                constexpr int PER = UBITS >= 32 ? 32 / BITS : UE;  // codes per packed dword
                uint32_t d[UBITS >= 32 ? UBITS / 32 : 1];
                if constexpr (RN == RN_NEAREST) {
                    uint32_t q[UE];
                    #pragma unroll
                    for (int k = 0; k < UE; ++k) {
                        if constexpr (THR && BITS == 2) {
                            // the count of thresholds at or below the value, as a binary search
                            // over the three sorted thresholds (5 instructions, against 6 for
                            // three compares and their sum)
                            const bool hi = v[i][k] >= thr[1];
                            const float t = hi ? thr[2] : thr[0];
                            q[k] = (hi ? 2u : 0u) + (v[i][k] >= t ? 1u : 0u);
                        } else if constexpr (THR) {
                            q[k] = v[i][k] >= thr[0] ? 1u : 0u;
                        } else {
                            float qf = __builtin_fmaf(v[i][k] - mn, inv, half_m);
                            // NaN -> 0, as the reference's clamp
                            if constexpr (CL) qf = __builtin_amdgcn_fmed3f(qf, 0.0f, qmaxf);
                            q[k] = cvt_u32(qf);
                        }
                    }
                    #pragma unroll
                    for (int j = 0; j < (UBITS >= 32 ? UBITS / 32 : 1); ++j) {
                        uint32_t acc = 0;
                        #pragma unroll
                        for (int k = 0; k < PER; ++k) acc |= q[j * PER + k] << (k * BITS);
                        d[j] = acc;
                    }
                } else {
                    // z = fma(t, inv, u) - 0.5; the code rint(z) (clamped to [0, QMAX] where the
                    // clamp can matter: clamp and rint commute, both bounds being integers) is
                    // rounded, converted and packed by pack_rne_codes
                    float z[UE];
                    #pragma unroll
                    for (int k = 0; k < UE; ++k) {
                        z[k] = __builtin_fmaf(v[i][k] - mn, inv, u[k]) - 0.5f;
                        // NaN -> 0, as the reference's clamp; always on for a caller's noise tensor
                        if constexpr (CL || RN == RN_NOISE) z[k] = __builtin_amdgcn_fmed3f(z[k], 0.0f, qmaxf);
                    }
                    #pragma unroll
                    for (int j = 0; j < (UBITS >= 32 ? UBITS / 32 : 1); ++j) d[j] = pack_rne_codes<BITS, PER>(&z[j * PER]);
                }
                uint32_t* dst = a.packed + (uint64_t)r * W;
                const bool ok = r < a.n_groups;
                if constexpr (UBITS >= 32) {
                    constexpr int ND = UBITS / 32;
                    if (ok) {
                        if constexpr (ND == 1) dst[c] = d[0];
                        else if constexpr (ND == 2) *(uint2*)(dst + 2 * c) = make_uint2(d[0], d[1]);
                        else *(uint4*)(dst + 4 * c) = make_uint4(d[0], d[1], d[2], d[3]);
                    }
                } else {
                    // merge LPD = 32/UBITS neighbouring units (lanes li..li+LPD-1) into one dword
                    uint32_t m = d[0];
                    if constexpr (UBITS < 32) m |= dpp_u32<0xB1>(m) << UBITS;
                    if constexpr (UBITS * 2 < 32) m |= dpp_u32<0x4E>(m) << (2 * UBITS);
                    if constexpr (UBITS * 4 < 32) m |= dpp_u32<0x104>(m) << (4 * UBITS);
                    constexpr int LPD = 32 / UBITS;
                    if (ok && (li % LPD) == 0) dst[c / LPD] = m;
                }
            }
        };
        if (clampq)
            emit(std::true_type{});
        else
            emit(std::false_type{});
    }

    // ---- per-group scale / min: gather group j of the wave into lane j, one store per array
    float sv = 0.0f, mv = 0.0f;
    #pragma unroll
    for (int p = 0; p < P; ++p) {
        const int src = ((lane - p * GPP) & (GPP - 1)) * LPG;
        const float s_ = __shfl(step_p[p], src, 64);
        const float m_ = __shfl(mn_p[p], src, 64);
        if (lane >= p * GPP && lane < (p + 1) * GPP) {
            sv = s_;
            mv = m_;
        }
    }
    const uint32_t rg = g0 + lane;
    if (lane < C::GPW && rg < a.n_groups) {
        if (a.meta_bf16) {
            ((uint16_t*)a.scale)[rg] = to_bf16(sv);
            ((uint16_t*)a.minv)[rg] = to_bf16(mv);
        } else {
            ((float*)a.scale)[rg] = sv;
            ((float*)a.minv)[rg] = mv;
        }
    }
}

// host-side launcher; explicitly instantiated per element type in quant_pack_<dtype>.hip
template <int DT>
int launch_quant_pack_dt(const QuantPackArgs& a, int bits, int g, int rn, int pre, hipStream_t s);

}  // namespace dopt
