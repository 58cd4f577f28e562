// gfx950 quant-pack kernel: per-group min/max, 1/2/4/8-bit nearest or stochastic rounding and
// little-endian bit-packing. Semantics follow Activation_Compression/act_triton_kernel.py:53-171
// (nearest) and the stochastic form of cpp_extension/include/quant_common.h:148-156 with the
// Triton step convention; see include/dopt.h for the ABI.
//
// Work decomposition (one wavefront = 64 lanes):
//   - a group of G elements is E*CPG values in 16-byte chunks (E = 16/sizeof(elem));
//   - LPG consecutive lanes own one group, each lane CPL chunks: chunk c = i*LPG + li for
//     i < CPL, so every load instruction reads LPG*16 contiguous bytes per group (>= 128 B,
//     whole cache lines) and the wave's loads are 16-byte vector loads;
//   - a wave handles GPP = 64/LPG groups per pass and P passes per iteration (P*CPL 16-byte
//     loads in flight per lane), all issued before any arithmetic;
//   - min/max: lane-local, then a DPP all-reduce over the LPG lanes (no LDS);
//   - codes: each lane packs its chunk into a E*BITS-bit piece; pieces narrower than a dword are
//     merged with DPP from neighbour lanes; dwords are staged in a wave-private LDS slice and
//     written back with coalesced 128-bit stores (the wave's output block is contiguous).
#pragma once

#include "dopt_device.h"

namespace dopt {

struct QuantPackArgs {
    const void* x;
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

template <int DT, int BITS, int G, int RN>
struct QuantPackCfg {
    static constexpr int E = DType<DT>::per16;
    static constexpr int CPG = G / E;
    static constexpr int CPL = CPG >= 32 ? 4 : (CPG >= 16 ? 2 : 1);
    static constexpr int LPG = CPG / CPL;
    static constexpr int GPP = 64 / LPG;
    static constexpr int P = RN == RN_NOISE ? (CPL >= 4 ? 1 : 4 / CPL) : 8 / CPL;
    static constexpr int GPW = P * GPP;  // groups per wave iteration
    static constexpr int W = G * BITS / 32;
    static constexpr int PW = E * BITS;  // code bits per chunk
    static constexpr int DW = GPW * W;   // dwords staged per wave iteration
    static constexpr int WAVES = 4;      // waves per workgroup
    static_assert(LPG >= 4 && LPG <= 64, "group must span 4..64 lanes");
    static_assert(DW % 4 == 0, "staged block must be whole 16-byte vectors");
};

// Linear element index of element e0 of group r (flat, or the spatial tile gather of
// tensor_act_reshape_utils.py:115-125: group r = band*(W/s) + tw, element e = i*s + j).
template <int G>
__device__ __forceinline__ uint64_t group_elem_index(const QuantPackArgs& a, uint32_t r, uint32_t e0) {
    if (!a.tiled) return (uint64_t)r * G + e0;
    const uint32_t band = r / a.tiles_w;
    const uint32_t tw = r - band * a.tiles_w;
    const uint32_t smask = (1u << a.log2s) - 1u;
    return (((uint64_t)band * a.row) << a.log2s) + ((uint64_t)tw << a.log2s) +
           (uint64_t)(e0 >> a.log2s) * a.row + (e0 & smask);
}

template <int DT, int BITS, int G, int RN>
__global__ __launch_bounds__(256) void quant_pack_kernel(QuantPackArgs a) {
    using C = QuantPackCfg<DT, BITS, G, RN>;
    constexpr int E = C::E, CPL = C::CPL, LPG = C::LPG, GPP = C::GPP, P = C::P, W = C::W;
    constexpr int PW = C::PW;
    constexpr int QMAX = (1 << BITS) - 1;
    constexpr int NZ = RN == RN_NOISE ? E / 4 : 1;
    using piece_t = typename std::conditional<(PW > 32), uint64_t, uint32_t>::type;

    __shared__ uint32_t stage[C::WAVES][C::DW];

    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int slot = lane / LPG;
    const int li = lane % LPG;
    const uint32_t g0 = (blockIdx.x * C::WAVES + wv) * (uint32_t)C::GPW;
    const char* xb = (const char*)a.x;

    // ---- issue every load of this iteration first (P*CPL 16-byte loads per lane)
    uint4 raw[P][CPL];
    uint4 nz[P][CPL][NZ];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        const bool ok = r < a.n_groups;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t e0 = (uint32_t)(i * LPG + li) * E;
            raw[p][i] = make_uint4(0u, 0u, 0u, 0u);
            if (ok)
                raw[p][i] = *(const uint4*)(xb + group_elem_index<G>(a, r, e0) * DType<DT>::bytes);
            if constexpr (RN == RN_NOISE) {
#pragma unroll
                for (int k = 0; k < NZ; ++k) {
                    nz[p][i][k] = make_uint4(0u, 0u, 0u, 0u);
                    if (ok) nz[p][i][k] = *(const uint4*)(a.noise + (uint64_t)r * G + e0 + 4 * k);
                }
            }
        }
    }

    const float qmaxf = (float)QMAX;
    const float half_m = 0.49999899f;  // fp32(0.5 - 1e-6) = 0x3EFFFFDE

#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        const bool ok = r < a.n_groups;
        float v[CPL][E];
#pragma unroll
        for (int i = 0; i < CPL; ++i) widen16<DT>(raw[p][i], v[i]);
        if (a.flags & FL_CLAMP) {
#pragma unroll
            for (int i = 0; i < CPL; ++i)
#pragma unroll
                for (int k = 0; k < E; ++k) v[i][k] = fminf(fmaxf(v[i][k], -a.clamp_alpha), a.clamp_alpha);
        }
        if (a.flags & FL_SQUASH) {
#pragma unroll
            for (int i = 0; i < CPL; ++i)
#pragma unroll
                for (int k = 0; k < E; ++k) v[i][k] = tanhf(v[i][k] / 0.5f) * 0.5f;
        }
        float mn = v[0][0], mx = v[0][0];
#pragma unroll
        for (int i = 0; i < CPL; ++i)
#pragma unroll
            for (int k = 0; k < E; ++k) {
                mn = fminf(mn, v[i][k]);
                mx = fmaxf(mx, v[i][k]);
            }
        block_minmax<LPG>(mn, mx);
        mn = mn + 0.0f;  // store -0.0 as +0.0
        const float rng = mx - mn;
        const float step = rng > 0.0f ? rng / qmaxf : 1.0f;
        const float inv = 1.0f / step;
        if (li == 0 && ok) {
            if (a.meta_bf16) {
                ((uint16_t*)a.scale)[r] = to_bf16(step);
                ((uint16_t*)a.minv)[r] = to_bf16(mn);
            } else {
                ((float*)a.scale)[r] = step;
                ((float*)a.minv)[r] = mn;
            }
        }

#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t c = (uint32_t)(i * LPG + li);
            const uint32_t e0 = c * E;
            float u[E];
            if constexpr (RN == RN_NOISE) {
#pragma unroll
                for (int k = 0; k < NZ; ++k) {
                    u[4 * k + 0] = __uint_as_float(nz[p][i][k].x);
                    u[4 * k + 1] = __uint_as_float(nz[p][i][k].y);
                    u[4 * k + 2] = __uint_as_float(nz[p][i][k].z);
                    u[4 * k + 3] = __uint_as_float(nz[p][i][k].w);
                }
            } else if constexpr (RN == RN_PHILOX) {
                const uint64_t blk = ((uint64_t)r * G + e0) >> 3;
                const uint4 w4 = philox4x32_10((uint32_t)blk, (uint32_t)(blk >> 32), a.off_lo, a.off_hi,
                                               a.seed_lo, a.seed_hi);
                const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    const int kk = (int)(e0 & 7u) + k;  // E == 4 chunks use half a block
                    u[k] = philox_half_to_u((w[kk >> 1] >> ((kk & 1) * 16)) & 0xffffu);
                }
            }
            piece_t piece = 0;
#pragma unroll
            for (int k = 0; k < E; ++k) {
                float t = v[i][k] - mn;
                t = t * inv;
                float qf;
                if constexpr (RN == RN_NEAREST) {
                    qf = t + half_m;
                } else {
                    qf = t + u[k];
                    qf = qf - 0.5f;
                }
                qf = fminf(fmaxf(qf, 0.0f), qmaxf);
                const uint32_t q = RN == RN_NEAREST ? (uint32_t)qf : (uint32_t)rintf(qf);
                piece |= (piece_t)q << (k * BITS);
            }
            // merge narrow pieces from the next lanes (chunks c+1, c+2, ...) into a dword
            uint32_t d0 = (uint32_t)piece;
            if constexpr (PW < 32) d0 |= dpp_u32<0xB1>(d0) << PW;
            if constexpr (PW * 2 < 32) d0 |= dpp_u32<0x4E>(d0) << (2 * PW);
            if constexpr (PW * 4 < 32) d0 |= dpp_u32<0x104>(d0) << (4 * PW);
            const int sbase = (p * GPP + slot) * W;
            if constexpr (PW >= 32) {
                const int di = sbase + (int)(c * (PW / 32));
                stage[wv][di] = d0;
                if constexpr (PW == 64) stage[wv][di + 1] = (uint32_t)((uint64_t)piece >> 32);
            } else {
                constexpr int LPD = 32 / PW;  // lanes merged into one dword
                if ((li % LPD) == 0) stage[wv][sbase + (int)(c / LPD)] = d0;
            }
        }
    }
    __syncthreads();

    // ---- the wave's output block [g0, g0 + GPW) is contiguous: 128-bit stores
    const uint32_t ng = g0 < a.n_groups ? min((uint32_t)C::GPW, a.n_groups - g0) : 0u;
    const uint32_t valid = ng * W;
    uint32_t* dst = a.packed + (uint64_t)g0 * W;
#pragma unroll
    for (int o = lane * 4; o < C::DW; o += 256) {
        if ((uint32_t)o + 4 <= valid) {
            *(uint4*)(dst + o) = *(const uint4*)&stage[wv][o];
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if ((uint32_t)(o + k) < valid) dst[o + k] = stage[wv][o + k];
        }
    }
}

// host-side launcher; explicitly instantiated per element type in quant_pack_<dtype>.hip
template <int DT>
int launch_quant_pack_dt(const QuantPackArgs& a, int bits, int g, int rn, hipStream_t s);

}  // namespace dopt
