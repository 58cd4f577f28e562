// BatchNorm kernels for gfx950: per-channel statistics, normalize + quant-pack (plain, squashed
// or fused with ReLU / ReLU6) and the backward pair (dequant + reduce, then the input gradient).
//
// Restates Activation_Compression/modules/normalization/kernel_implementation.py (the live
// DOBatchNorm2d path) and Activation_Compression/triton_kernel/norm_act_fusion/bn_act_fusion.py
// (the BatchNorm + ReLU fusion):
//   stats     sum, sum of squares per channel (kernel_implementation.py:12-35)
//   BN_NORM   y = x_hat * w + b and x_hat, both bf16; invstd from eps (:38-91)
//   BN_QUANT  y, and x_hat squashed to 2 tanh(clamp(x_hat, -3, 3) / 2) quantized per group
//             (:94-201)
//   BN_RELU*  y = relu(x_hat * w + b) (or relu6), a 1-bit mask, x_hat quantized per group with
//             no squash and codes (x_hat - min) / scale + (0.5 - 1e-6) (bn_act_fusion.py:8-118)
//   backward  sum(dy [* mask]) and sum(dy [* mask] * x_hat') with x_hat' the dequantized codes
//             (or the bf16 x_hat), then dx = (dy - db/M - x_hat' dw/M) w invstd (bf16)
//             (kernel_implementation.py:204-481, bn_act_fusion.py:121-278)
//
// Floating-point order (the reference kernels compile with FMA contraction): mean = sum / M,
// var = max(fma(-mean, mean, sumsq / M), 0), invstd = 1 / sqrt(var + eps) (IEEE division and
// square root), x_hat = (x - mean) * invstd, y = fma(x_hat, w, b), codes trunc(fma(t - min,
// 1/scale, 0.5 - 1e-6)) (squashed modes) or trunc((x_hat - min) / scale + (0.5 - 1e-6)) (ReLU
// modes), x_hat' = fma(q, scale, min), dx = ((fma(-x_hat', dw/M, dy - db/M)) * w) * invstd.
//
// Grid: x runs over the channels and y over a channel's BN_CHUNK-element chunks, so the hardware
// dispatches the same chunk of consecutive channels together and the workgroups in flight read and
// write neighbouring [n, c, :] rows (with the chunks along x, the workgroups in flight walked one
// channel's rows, C * HW elements apart, and the forward ran at 82% of the speed it reaches this
// way: measured at bf16 [256, 256, 56, 56], ReLU mode 177 against 159 us, a copy with the same
// accesses 165 against 144 us).
//
// Mapping: a workgroup of 256 lanes covers 4 blocks of 2048 consecutive elements of one channel,
// 8 per lane per block, read and written as 8 / V row-contiguous accesses of V elements, V the
// largest of 8, 4, 2, 1 that divides HW and both strides and fits the pointers' alignment (so an
// access never crosses a row: one 16-byte access for 2-byte types at HW = 56 x 56, two 8-byte
// ones at 14 x 14, eight 2-byte ones at 7 x 7), with every block's loads issued before the first
// is used. A group of G elements spans G/8 aligned lanes (4..64), so group min/max and the
// code merge stay inside a wave. Reductions are two-stage and ordered (workgroup partials, then
// one wave per channel), so sums are deterministic and need no zeroed buffer or atomics.
#include "bn_fused.h"
#include "dopt_device.h"

namespace dopt {
namespace {

constexpr int TPB = 256;
constexpr int EPL = 8;
constexpr int64_t WG_ELEMS = TPB * EPL;
constexpr int ITER = (int)(BN_CHUNK / WG_ELEMS);  // 2048-element blocks per workgroup (loads issued together)

// Position of element e of channel c: row n = e / HW, column r = e % HW, at offset
// row + r with row = n * stride_n + c * stride_c. A lane finds its first element's position with
// one 32-bit division (e < M + BN_CHUNK < 2^32, the host checks M < 2^31) and walks from there:
// V elements to the next chunk of its 8, WG_ELEMS to its next block, each a remainder step
// below HW plus whole rows, so one conditional wrap per step.
struct RowCursor {
    int64_t row;
    uint32_t r;
};

__device__ __forceinline__ RowCursor cursor_at(const BnGeom& g, int64_t c, int64_t e) {
    const uint32_t hw = (uint32_t)g.HW, ee = (uint32_t)e;
    const uint32_t n = ee / hw;
    return {(int64_t)n * g.stride_n + c * g.stride_c, ee - n * hw};
}

// advance by dr < HW elements plus the whole rows folded into drow (= rows * stride_n)
__device__ __forceinline__ void cursor_step(RowCursor& p, const BnGeom& g, uint32_t dr, int64_t drow) {
    p.r += dr;
    p.row += drow;
    if (p.r >= (uint32_t)g.HW) {
        p.r -= (uint32_t)g.HW;
        p.row += g.stride_n;
    }
}

// cursors of the lane's ITER blocks (elements base + it * WG_ELEMS)
__device__ __forceinline__ void block_cursors(const BnGeom& g, int64_t c, int64_t base, RowCursor* cur) {
    const uint32_t hw = (uint32_t)g.HW;
    const uint32_t bq = (uint32_t)WG_ELEMS / hw, br = (uint32_t)WG_ELEMS - bq * hw;
    const int64_t brow = (int64_t)bq * g.stride_n;
    cur[0] = cursor_at(g, c, base);
#pragma unroll
    for (int it = 1; it < ITER; ++it) {
        cur[it] = cur[it - 1];
        cursor_step(cur[it], g, br, brow);
    }
}

// A block at or past M (a lane of the last workgroup) reads the channel's first block instead:
// every load stays in bounds and carries no lane-mask branch, so all of a lane's loads are in
// flight together (a masked load merged with a default value waits for its data); callers drop
// the results of such blocks (whole groups lie on one side of M).
__device__ __forceinline__ void block_or_first(const BnGeom& g, int64_t c, const RowCursor& cur, int64_t e0,
                                               int64_t M, RowCursor& p, int64_t& e) {
    const bool in = e0 < M;
    p = {in ? cur.row : c * g.stride_c, in ? cur.r : 0u};
    e = in ? e0 : 0;
}

// V consecutive elements of one row at element offset off (aligned to V elements)
template <int DT, int V>
__device__ __forceinline__ void ldv(const void* base, int64_t off, float* v) {
    const char* p = (const char*)base + off * DType<DT>::bytes;
    if constexpr (V * DType<DT>::bytes >= 16) {
#pragma unroll
        for (int h = 0; h < V * DType<DT>::bytes / 16; ++h) widen16<DT>(ld16<false>(p + 16 * h), v + h * DType<DT>::per16);
    } else if constexpr (DT == DT_F32) {
        if constexpr (V == 2) {
            const uint2 u = *(const uint2*)p;
            v[0] = __uint_as_float(u.x);
            v[1] = __uint_as_float(u.y);
        } else {
            v[0] = *(const float*)p;
        }
    } else {
        uint32_t w[2] = {0u, 0u};
        if constexpr (V == 4) {
            const uint2 u = *(const uint2*)p;
            w[0] = u.x;
            w[1] = u.y;
        } else if constexpr (V == 2) {
            w[0] = *(const uint32_t*)p;
        } else {
            w[0] = *(const uint16_t*)p;
        }
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const uint32_t b = (w[k >> 1] >> (16 * (k & 1))) & 0xffffu;
            if constexpr (DT == DT_BF16) v[k] = __uint_as_float(b << 16);
            else v[k] = (float)__builtin_bit_cast(_Float16, (uint16_t)b);
        }
    }
}

// the lane's 8 elements e0..e0+7 (cursor p at e0) as EPL / V row-contiguous loads; chunks at or
// past M read as 0 (M is a multiple of V, so a chunk is all in or all out)
template <int DT, int V>
__device__ __forceinline__ void load8(const void* base, const BnGeom& g, RowCursor p, int64_t e0, int64_t M,
                                      float* v) {
#pragma unroll
    for (int j = 0; j < EPL / V; ++j) {
        if (j) cursor_step(p, g, V, 0);
        if (V == EPL || e0 + j * V < M) {
            ldv<DT, V>(base, p.row + p.r, v + j * V);
        } else {
#pragma unroll
            for (int k = 0; k < V; ++k) v[j * V + k] = 0.0f;
        }
    }
}

// bf16 outputs are streamed (non-temporal: written once, read by another kernel much later)
template <int V>
__device__ __forceinline__ void store8_bf16(uint16_t* base, const BnGeom& g, RowCursor p, int64_t e0, int64_t M,
                                            const float* v) {
#pragma unroll
    for (int j = 0; j < EPL / V; ++j) {
        if (j) cursor_step(p, g, V, 0);
        if (V < EPL && e0 + j * V >= M) continue;
        uint16_t* q = base + p.row + p.r;
        const float* u = v + j * V;
        if constexpr (V == 8) {
            st16<true>(q, make_uint4(pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3]), pack_bf16x2(u[4], u[5]),
                                     pack_bf16x2(u[6], u[7])));
        } else if constexpr (V == 4) {
            *(uint2*)q = make_uint2(pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3]));
        } else if constexpr (V == 2) {
            *(uint32_t*)q = pack_bf16x2(u[0], u[1]);
        } else {
            *q = to_bf16(u[0]);
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// sums of a and b over the workgroup, in lane 0 of wave 0 (fixed order: waves 0..3)
__device__ __forceinline__ void block_sum2(float& a, float& b) {
    __shared__ float red[2][TPB / 64];
    a = wave_sum(a);
    b = wave_sum(b);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[0][w] = a;
        red[1][w] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        a = ((red[0][0] + red[0][1]) + red[0][2]) + red[0][3];
        b = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
    }
}

// min / max over aligned blocks of lpg lanes (lpg in 4..64, wave-uniform); raw v_min / v_max
// (the operands are computed values: numbers or quiet NaNs)
__device__ __forceinline__ void group_minmax(float& mn, float& mx, int lpg) {
    mn = vmin_dpp<0xB1>(mn);
    mx = vmax_dpp<0xB1>(mx);
    mn = vmin_dpp<0x4E>(mn);
    mx = vmax_dpp<0x4E>(mx);
    if (lpg >= 8) {
        mn = vmin_dpp<0x141>(mn);
        mx = vmax_dpp<0x141>(mx);
    }
    if (lpg >= 16) {
        mn = vmin_dpp<0x140>(mn);
        mx = vmax_dpp<0x140>(mx);
    }
    if (lpg >= 32) swap_minmax<16>(mn, mx);
    if (lpg >= 64) swap_minmax<32>(mn, mx);
}

// Writes the lane's 8 codes (bits each) into the channel bitstream at element e0: 1-bit codes
// merge over 4 lanes, 2-bit over 2, 4-bit fill one word, 8-bit two.
// (e0 < 2^32: 32-bit index arithmetic from the channel's base)
__device__ __forceinline__ void store_codes(uint32_t* chan, uint32_t e0, const int* q, int bits, bool active) {
    const int lane = threadIdx.x & 63;
    if (bits == 8) {
        const uint32_t lo = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
        const uint32_t hi = (uint32_t)q[4] | ((uint32_t)q[5] << 8) | ((uint32_t)q[6] << 16) | ((uint32_t)q[7] << 24);
        if (active) *(uint2*)(chan + e0 / 4) = make_uint2(lo, hi);
        return;
    }
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < EPL; ++k) v |= (uint32_t)q[k] << (k * bits);
    if (bits == 4) {
        if (active) chan[e0 / 8] = v;
    } else if (bits == 2) {
        v <<= 16 * (lane & 1);
        v |= dpp_u32<0xB1>(v);
        if (active && (lane & 1) == 0) chan[e0 / 16] = v;
    } else {
        v <<= 8 * (lane & 3);
        v |= dpp_u32<0xB1>(v);
        v |= dpp_u32<0x4E>(v);
        if (active && (lane & 3) == 0) chan[e0 >> 5] = v;
    }
}

// 8 mask bits of a lane -> one word over 4 lanes
__device__ __forceinline__ void store_mask(uint32_t* chan, uint32_t e0, uint32_t m8, bool active) {
    const int lane = threadIdx.x & 63;
    uint32_t v = m8 << (8 * (lane & 3));
    v |= dpp_u32<0xB1>(v);
    v |= dpp_u32<0x4E>(v);
    if (active && (lane & 3) == 0) chan[e0 >> 5] = v;
}

// the lane's 8 codes read back from the channel bitstream
// (e0 is a multiple of 8, so below 8 bits the lane's 8 * bits code bits lie in one dword and at
// 8 bits in two; both dwords are loaded at selected addresses, with no branch, then extracted)
__device__ __forceinline__ void load_codes(const uint32_t* chan, int64_t e0, int bits, int* q) {
    const bool b8 = bits == 8;
    const int64_t bit0 = e0 * bits;
    const uint32_t* p = chan + (bit0 >> 5);
    const uint32_t w0 = p[0] >> (bit0 & 31);  // bit0 & 31 == 0 at 8 bits
    const uint32_t w1 = p[b8 ? 1 : 0];
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        const uint32_t src = (b8 && k >= 4) ? w1 : w0;
        const uint32_t off = b8 ? 8u * (uint32_t)(k & 3) : (uint32_t)(k * bits);
        q[k] = (int)__builtin_amdgcn_ubfe(src, off, (uint32_t)bits);
    }
}

// avg_alam: the codes of the lane's 8 elements, element e carrying code e / A of the channel's
// stream of M / A codes (kernel_implementation.py:374-377, :455-458: each code repeated A times).
// e0 is a multiple of 8: below A = 8 the lane's 8 / A codes fill an aligned (8 / A) * bits <= 32
// bit field, from A = 8 on its 8 elements share one code, so one dword holds them.
__device__ __forceinline__ void load_codes_alam(const uint32_t* chan, uint32_t e0, int bits, int alam_lg, int* q) {
    const uint32_t c0 = e0 >> alam_lg, bit0 = c0 * (uint32_t)bits;
    const uint32_t w = chan[bit0 >> 5] >> (bit0 & 31);
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        const uint32_t off = (((e0 + (uint32_t)k) >> alam_lg) - c0) * (uint32_t)bits;
        q[k] = (int)__builtin_amdgcn_ubfe(w, off, (uint32_t)bits);
    }
}

template <bool ALAM>
__device__ __forceinline__ void lane_codes(const BnBwdArgs& a, int64_t c, int64_t e0, int64_t M, int bits, int* q) {
    if (ALAM && a.alam_lg > 0)
        load_codes_alam(a.packed + c * (((M >> a.alam_lg) * bits) >> 5), (uint32_t)e0, bits, a.alam_lg, q);
    else
        load_codes(a.packed + c * ((M * bits) >> 5), e0, bits, q);
}

// ------------------------------------------------------------------ statistics
template <int DT, int V>
__global__ __launch_bounds__(TPB) void bn_stats_kernel(const void* __restrict__ x, BnGeom g,
                                                       float* __restrict__ partial, int64_t nchunks) {
    const int64_t c = blockIdx.x, chunk = blockIdx.y;
    const int64_t M = g.N * g.HW;
    const int64_t base = chunk * BN_CHUNK + (int64_t)threadIdx.x * EPL;
    RowCursor cur[ITER];
    block_cursors(g, c, base, cur);
    float v[ITER][EPL];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        RowCursor p;
        int64_t e;
        block_or_first(g, c, cur[it], base + it * WG_ELEMS, M, p, e);
        load8<DT, V>(x, g, p, e, M, v[it]);
    }
    float s = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        if (base + it * WG_ELEMS >= M) continue;  // a stand-in block: no contribution
#pragma unroll
        for (int k = 0; k < EPL; ++k) {
            s += v[it][k];
            s2 = fmaf(v[it][k], v[it][k], s2);
        }
    }
    block_sum2(s, s2);
    if (threadIdx.x == 0) {
        partial[c * nchunks + chunk] = s;
        partial[(g.C + c) * nchunks + chunk] = s2;
    }
}

// one wave per channel: lane l sums partials l, l+64, ... in order, then the wave tree (fixed
// order, so the result is deterministic); the loads of a lane are independent and overlap
__global__ __launch_bounds__(64) void bn_finalize_kernel(const float* __restrict__ partial, int64_t C,
                                                         int64_t nchunks, float* __restrict__ out0,
                                                         float* __restrict__ out1) {
    const int64_t c = blockIdx.x;
    float a = 0.0f, b = 0.0f;
#pragma unroll 4
    for (int64_t k = threadIdx.x; k < nchunks; k += 64) {
        a += partial[c * nchunks + k];
        b += partial[(C + c) * nchunks + k];
    }
    a = wave_sum(a);
    b = wave_sum(b);
    if (threadIdx.x == 0) {
        out0[c] = a;
        out1[c] = b;
    }
}

// One channel's sum over its workgroup partials p[0..n), computed by a whole wave exactly as
// bn_finalize_kernel does (lane l adds p[l], p[l + 64], ... in order, then the same wave tree), so
// the result is bit-identical to the finalized value; every lane returns it.
__device__ __forceinline__ float partial_sum(const float* __restrict__ p, int64_t n) {
    float a = 0.0f;
#pragma unroll 4
    for (int64_t k = threadIdx.x & 63; k < n; k += 64) a += p[k];
    return wave_sum(a);
}

// per-channel mean and inverse std as the forward kernels derive them
__device__ __forceinline__ void channel_stats(const BnFwdArgs& a, int64_t c, int64_t M, float& mean, float& inv) {
    if (a.sync) {
        mean = a.mean_in[c];
        inv = a.invstd_in[c];
        return;
    }
    const float Mf = (float)M;
    float sum, sumsq;
    if (a.partial) {
        sum = partial_sum(a.partial + c * a.nchunks, a.nchunks);
        sumsq = partial_sum(a.partial + (a.g.C + c) * a.nchunks, a.nchunks);
    } else {
        sum = a.sum[c];
        sumsq = a.sumsq[c];
    }
    mean = sum / Mf;
    float var = fmaf(-mean, mean, sumsq / Mf);
    var = fmaxf(var, 0.0f);
    inv = 1.0f / sqrtf(var + a.eps);
    if (blockIdx.y == 0 && threadIdx.x == 0) {
        a.mean_out[c] = mean;
        a.var_out[c] = var;
        // the running statistics (biased variance, as the reference's layer updates them with
        // mul_(1 - momentum).add_(stat, alpha=momentum), normalization_ops.py:56-57)
        if (a.run_mean) a.run_mean[c] = fmaf(a.run_mom, mean, a.run_mean[c] * a.run_keep);
        if (a.run_var) a.run_var[c] = fmaf(a.run_mom, var, a.run_var[c] * a.run_keep);
    }
}

// ------------------------------------------------------------------ forward
// avg_alam codes of one wave's 512 consecutive elements (kernel_implementation.py:194-237): every
// run of A = 2^alam_lg elements becomes one code, the truncated mean of the run's
// qf = fma(t - min, 1/scale, 0.5 - 1e-6) (summed left to right, then times 1/A: exact, A a power
// of two), clamped to [0, QMAX] (NaN -> 0). A divides the group, so runs never straddle groups, and
// the channel's codes form one bitstream of M / A codes. Through LDS: the wave's 512 qf, its
// 512 / A codes (one byte each), then its (16 bits) / A words, each written when its elements lie
// below M. A wave's LDS operations complete in order, so its own reads see its writes.
__device__ __forceinline__ void alam_store(uint32_t* chan, uint32_t e0, uint32_t M, const float* t, float mn, float invs,
                                        float qmaxf, int bits, int alam_lg) {
    __shared__ float qs[TPB / 64][64 * EPL];
    __shared__ uint8_t cs[TPB / 64][64 * EPL];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float half_m = 0.49999899f;  // fp32(0.5 - 1e-6)
#pragma unroll
    for (int k = 0; k < EPL; ++k) qs[wave][lane * EPL + k] = fmaf(t[k] - mn, invs, half_m);
    __builtin_amdgcn_wave_barrier();
    const int A = 1 << alam_lg, ncodes = (64 * EPL) >> alam_lg;
    const float inv_a = 1.0f / (float)A;
    for (int k = lane; k < ncodes; k += 64) {
        float sum = qs[wave][k * A];
        for (int j = 1; j < A; ++j) sum = sum + qs[wave][k * A + j];
        cs[wave][k] = (uint8_t)(int)__builtin_amdgcn_fmed3f(sum * inv_a, 0.0f, qmaxf);
    }
    __builtin_amdgcn_wave_barrier();
    const int vpw = 32 / bits, nwords = (2 * EPL * bits) >> alam_lg;
    const uint32_t ew = e0 - (uint32_t)lane * EPL;  // the wave's first element
    if (lane < nwords && ew + (uint32_t)(lane * vpw * A) < M) {
        uint32_t word = 0;
        for (int j = 0; j < vpw; ++j) word |= (uint32_t)cs[wave][lane * vpw + j] << (j * bits);
        chan[(((ew >> alam_lg) * bits) >> 5) + lane] = word;
    }
    __builtin_amdgcn_wave_barrier();
}

// One 2048-element block of the forward: y (and the mask / codes / scale / min) from the lane's 8
// loaded values. Whole groups are active or not (M % group == 0), so the group's lanes agree.
//
// THR (the squashed mode at 1 and 2 bits, no ALAM): the squash t = 2 tanh(xc / 2) of the clamped
// x_hat xc is monotone, so the group's min and max of t are the squash of xc's min and max, and
// code q >= k exactly when t >= s_k = mn + (k - (0.5 - 1e-6)) step, i.e. when xc is at or above
// the threshold logit((s_k + 2) / 4) (t = 4 sigmoid(xc) - 2). The lane computes the group's
// thresholds once (v_log, v_rcp) and compares each element against them: no transcendental per
// element. The codes equal the per-element form's except where xc lies within the rounding of the
// transcendentals of a boundary.
template <int MODE, int V, bool R6, bool ALAM, bool THR = false>
__device__ __forceinline__ void fwd_block(const BnFwdArgs& a, int64_t c, RowCursor pos, int64_t e0, int64_t M,
                                          bool active, const float* v, float mean, float inv, float w, float b,
                                          int lg, int bits, float qmaxf, float rqmax) {
    static_assert(!THR || (MODE == BN_QUANT && !ALAM), "threshold codes: the squashed mode without ALAM");
    const BnGeom& g = a.g;
    float xh[EPL], y[EPL];
#pragma unroll
    for (int k = 0; k < EPL; ++k) {
        xh[k] = (v[k] - mean) * inv;
        y[k] = fmaf(xh[k], w, b);
    }
    if constexpr (MODE == BN_NORM) {
        if (active) {
            store8_bf16<V>(a.y, g, pos, e0, M, y);
            store8_bf16<V>(a.xhat, g, pos, e0, M, xh);
        }
    } else {
        uint32_t m8 = 0;
        if constexpr (MODE == BN_RELU_QUANT) {
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                const bool on = R6 ? (y[k] > 0.0f && y[k] < 6.0f) : (y[k] > 0.0f);
                m8 |= (uint32_t)on << k;
                y[k] = R6 ? __builtin_amdgcn_fmed3f(y[k], 0.0f, 6.0f) : (on ? y[k] : 0.0f);
            }
        }
        if (active) store8_bf16<V>(a.y, g, pos, e0, M, y);
        if constexpr (MODE == BN_RELU_QUANT) store_mask(a.relu_packed + c * (M >> 5), (uint32_t)e0, m8, active);

        // values quantized: the squashed x_hat (BN_QUANT) or x_hat itself (ReLU modes)
        float t[EPL];
#pragma unroll
        for (int k = 0; k < EPL; ++k) {
            if constexpr (THR) {
                t[k] = __builtin_amdgcn_fmed3f(xh[k], -3.0f, 3.0f);  // xc; squashed only at min / max
            } else if constexpr (MODE == BN_QUANT) {
                t[k] = two_tanh_half_fast(__builtin_amdgcn_fmed3f(xh[k], -3.0f, 3.0f));
            } else {
                t[k] = xh[k];
            }
        }
        // min / max of {+-inf, t[0..7]} (an all-NaN lane keeps the infinities), 3-operand forms
        float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
        for (int k = 0; k < EPL; k += 2) {
            mn = vmin3(mn, t[k], t[k + 1]);
            mx = vmax3(mx, t[k], t[k + 1]);
        }
        const int lpg = 1 << (lg - 3);  // group / EPL
        group_minmax(mn, mx, lpg);
        if constexpr (THR) {  // the infinities of an all-NaN group stay as they are
            mn = mn < 4.0f ? two_tanh_half_fast(mn) : mn;
            mx = mx > -4.0f ? two_tanh_half_fast(mx) : mx;
        }
        // step = rng / qmax and 1 / step, both rounded as the IEEE divisions round them
        const float rng = mx - mn;
        const float step = rng > 0.0f ? div_by_qmax_rt(rng, qmaxf, rqmax) : 1.0f;
        const float invs = exact_rcp(step);
        if constexpr (ALAM) {
            alam_store(a.packed + c * (((M >> a.alam_lg) * bits) >> 5), (uint32_t)e0, (uint32_t)M, t, mn, invs,
                       qmaxf, bits, a.alam_lg);
        } else {
            const float half_m = 0.49999899f;  // fp32(0.5 - 1e-6) = 0x3EFFFFDE
            int q[EPL];
            if constexpr (THR) {
                // thresholds ln(p / (1 - p)), p = (s_k + 2) / 4; an s_k past the group's max
                // (p >= 1, or any s_k of a constant group's step 1 beyond it) gives NaN or +inf,
                // which no xc reaches
                // lane j of each aligned quad (j < 3; lane 3 repeats j = 2) evaluates threshold j and
                // quad_perm broadcasts hand every lane all three (a group's G / 8 >= 4 lanes span
                // whole quads and agree on mn and step)
                const int jq = (threadIdx.x & 3) < 2 ? (threadIdx.x & 3) + 1 : 3;
                const float pk = fmaf(fmaf((float)jq - half_m, step, mn), 0.25f, 0.5f);
                const float tj = 0.6931471805599453f * __builtin_amdgcn_logf(pk * __builtin_amdgcn_rcpf(1.0f - pk));
                const float th[3] = {dpp_f32<0x00>(tj), dpp_f32<0x55>(tj), dpp_f32<0xAA>(tj)};
                if (bits == 1) {
#pragma unroll
                    for (int k = 0; k < EPL; ++k) q[k] = t[k] >= th[0] ? 1 : 0;
                } else {  // 2 bits: a binary search over the three sorted thresholds
#pragma unroll
                    for (int k = 0; k < EPL; ++k) {
                        const bool hi = t[k] >= th[1];
                        q[k] = (hi ? 2 : 0) + (t[k] >= (hi ? th[2] : th[0]) ? 1 : 0);
                    }
                }
            } else if constexpr (MODE == BN_QUANT) {
#pragma unroll
                for (int k = 0; k < EPL; ++k) {
                    const float qf = __builtin_amdgcn_fmed3f(fmaf(t[k] - mn, invs, half_m), 0.0f, qmaxf);
                    q[k] = (int)qf;
                }
            } else {
                // (t - mn) / step, correctly rounded, without a division per element: with y = 1/step
                // correctly rounded (one division per group), q0 = RN(a y) and the exact remainder
                // r = fma(-q0, step, a), RN(q0 + r y) is the correctly rounded a / step (Markstein's
                // theorem, the IA-64 division), given no overflow and a normal remainder. With
                // 2^-60 <= step < inf and a in [0, rng] the quotient lies in [0, qmax], and whenever it
                // can reach a rounding boundary of the code (q >= ~1e-7) the remainder is normal.
                // (Checked bit-for-bit against fp32 division on 4e8 random and quantizer-shaped pairs.)
                // (The test is per group; one wave-uniform branch keeps the common case free of
                // per-element lane masking.)
                const bool fastdiv = step >= 0x1p-60f && step < __builtin_huge_valf();
                if (__builtin_amdgcn_ballot_w64(!fastdiv) == 0) {
#pragma unroll
                    for (int k = 0; k < EPL; ++k) {
                        const float num = t[k] - mn;
                        const float q0 = num * invs;
                        const float quo = fmaf(fmaf(-q0, step, num), invs, q0);
                        q[k] = (int)__builtin_amdgcn_fmed3f(quo + half_m, 0.0f, qmaxf);
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < EPL; ++k) {
                        const float num = t[k] - mn;
                        float quo;
                        if (fastdiv) {
                            const float q0 = num * invs;
                            quo = fmaf(fmaf(-q0, step, num), invs, q0);
                        } else {
                            quo = num / step;
                        }
                        q[k] = (int)__builtin_amdgcn_fmed3f(quo + half_m, 0.0f, qmaxf);
                    }
                }
            }
            store_codes(a.packed + c * ((M * bits) >> 5), (uint32_t)e0, q, bits, active);
        }
        if (active && ((threadIdx.x & 63) & (lpg - 1)) == 0) {
            // the group's entry at a 32-bit byte offset from the channel's first (< 2^29)
            const int64_t g0 = c * (M >> lg);
            const uint32_t off = ((uint32_t)e0 >> lg) * 2u;
            *(uint16_t*)((char*)(a.scale + g0) + off) = to_bf16(step);
            *(uint16_t*)((char*)(a.minv + g0) + off) = to_bf16(mn);
        }
    }
}

// A workgroup covers ITER consecutive 2048-element blocks of one channel; all loads are issued
// before the first block is processed.
template <int DT, int MODE, int V, bool R6, bool ALAM = false, bool THR = false>
__global__ __launch_bounds__(TPB) void bn_fwd_kernel(BnFwdArgs a, int lg, int bits) {
    const int64_t c = blockIdx.x;
    const int64_t M = a.g.N * a.g.HW;
    const int64_t base = (int64_t)blockIdx.y * BN_CHUNK + (int64_t)threadIdx.x * EPL;
    RowCursor cur[ITER];
    block_cursors(a.g, c, base, cur);
    float v[ITER][EPL];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        RowCursor p;
        int64_t e;
        block_or_first(a.g, c, cur[it], base + it * WG_ELEMS, M, p, e);
        load8<DT, V>(a.x, a.g, p, e, M, v[it]);
    }
    // the channel's mean and inverse std: computed by wave 0 alone and passed through LDS (the
    // other waves' loads are in flight meanwhile)
    float mean, inv;
    {
        __shared__ float stat[2];
        if (threadIdx.x < 64) {
            channel_stats(a, c, M, mean, inv);
            if (threadIdx.x == 0) {
                stat[0] = mean;
                stat[1] = inv;
            }
        }
        __syncthreads();
        mean = stat[0];
        inv = stat[1];
    }
    const float w = a.w[c], b = a.b[c];
    const float qmaxf = (float)((1 << bits) - 1), rqmax = 1.0f / qmaxf;
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        const int64_t e0 = base + it * WG_ELEMS;
        fwd_block<MODE, V, R6, ALAM, THR>(a, c, cur[it], e0, M, e0 < M, v[it], mean, inv, w, b, lg, bits, qmaxf,
                                          rqmax);
    }
}

// ------------------------------------------------------------------ backward
// dy (times the ReLU mask) and x_hat' of the lane's 8 elements
template <int DYT, int MODE, int V, bool ALAM>
__device__ __forceinline__ void bwd_operands(const BnBwdArgs& a, int64_t c, RowCursor pos, int64_t e0, int64_t M,
                                             int lg, int bits, float* xh, float* dy) {
    load8<DYT, V>(a.dy, a.g, pos, e0, M, dy);
    if constexpr (MODE == BN_NORM) {
        load8<DT_BF16, V>(a.xhat, a.g, pos, e0, M, xh);
    } else {
        int q[EPL];
        lane_codes<ALAM>(a, c, e0, M, bits, q);
        const int64_t gi = c * (M >> lg) + (e0 >> lg);
        const float sc = bf16_bits_to_f32(a.scale[gi]);
        const float mn = bf16_bits_to_f32(a.minv[gi]);
#pragma unroll
        for (int k = 0; k < EPL; ++k) xh[k] = fmaf((float)q[k], sc, mn);
        if constexpr (MODE == BN_RELU_QUANT) {
            const uint32_t m = a.relu_packed[c * (M >> 5) + (e0 >> 5)] >> (e0 & 31);
#pragma unroll
            for (int k = 0; k < EPL; ++k) dy[k] = dy[k] * (float)((m >> k) & 1u);
        }
    }
}

// dy (times the ReLU mask), the codes and the group's scale / min of the lane's 8 elements
template <int DYT, int MODE, int V, bool ALAM>
__device__ __forceinline__ void bwd_codes(const BnBwdArgs& a, int64_t c, RowCursor pos, int64_t e0, int64_t M, int lg,
                                          int bits, int* q, float& sc, float& mn, float* dy) {
    load8<DYT, V>(a.dy, a.g, pos, e0, M, dy);
    lane_codes<ALAM>(a, c, e0, M, bits, q);
    const int64_t gi = c * (M >> lg) + (e0 >> lg);
    sc = bf16_bits_to_f32(a.scale[gi]);
    mn = bf16_bits_to_f32(a.minv[gi]);
    if constexpr (MODE == BN_RELU_QUANT) {
        const uint32_t m = a.relu_packed[c * (M >> 5) + (e0 >> 5)] >> (e0 & 31);
#pragma unroll
        for (int k = 0; k < EPL; ++k) dy[k] = dy[k] * (float)((m >> k) & 1u);
    }
}

// With avg_alam (ALAM) the reduce adds the reference's noise to each code before the product
// (kernel_implementation.py:377-381): q + (tl.rand(42 + b, e mod G) - 0.5), b = e / (2 G) the
// index of the reference's two-group block; the seed does not depend on the channel.
template <int DYT, int MODE, int V, bool ALAM = false>
__global__ __launch_bounds__(TPB) void bn_bwd_reduce_kernel(BnBwdArgs a, int lg, int bits, int64_t nchunks) {
    const int64_t c = blockIdx.x, chunk = blockIdx.y;
    const int64_t M = a.g.N * a.g.HW;
    const int64_t base = chunk * BN_CHUNK + (int64_t)threadIdx.x * EPL;
    RowCursor cur[ITER];
    block_cursors(a.g, c, base, cur);
    float sdy = 0.0f, sdyx = 0.0f;
    if constexpr (MODE == BN_NORM) {
        float xh[ITER][EPL], dy[ITER][EPL];
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
            const int64_t e0 = base + it * WG_ELEMS;
            RowCursor p;
            int64_t e;
            block_or_first(a.g, c, cur[it], e0, M, p, e);
            bwd_operands<DYT, MODE, V, false>(a, c, p, e, M, lg, bits, xh[it], dy[it]);
        }
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
            if (base + it * WG_ELEMS >= M) continue;
#pragma unroll
            for (int k = 0; k < EPL; ++k) {
                sdy += dy[it][k];
                sdyx = fmaf(dy[it][k], xh[it][k], sdyx);
            }
        }
    } else {
        // a lane's 8 elements of a block lie in one group, so sum(dy * x_hat') over them is
        // scale * sum(dy * q) + min * sum(dy): no dequantized value per element
        float dy[ITER][EPL];
        int q[ITER][EPL];
        float sc[ITER], mn[ITER];
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
            const int64_t e0 = base + it * WG_ELEMS;
            RowCursor p;
            int64_t e;
            block_or_first(a.g, c, cur[it], e0, M, p, e);
            bwd_codes<DYT, MODE, V, ALAM>(a, c, p, e, M, lg, bits, q[it], sc[it], mn[it], dy[it]);
        }
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
            if (base + it * WG_ELEMS >= M) continue;
            float gdy = 0.0f, gdyq = 0.0f;
            if constexpr (ALAM) {
                const uint32_t e0 = (uint32_t)(base + it * WG_ELEMS);
                const uint64_t seed = 42u + (e0 >> (lg + 1));
#pragma unroll
                for (int k = 0; k < EPL; ++k) {
                    const float u = triton_rand(seed, (e0 + (uint32_t)k) & ((1u << lg) - 1u));
                    gdy += dy[it][k];
                    gdyq = fmaf(dy[it][k], (float)q[it][k] + (u - 0.5f), gdyq);
                }
            } else {
#pragma unroll
                for (int k = 0; k < EPL; ++k) {
                    gdy += dy[it][k];
                    gdyq = fmaf(dy[it][k], (float)q[it][k], gdyq);
                }
            }
            sdy += gdy;
            sdyx = fmaf(sc[it], gdyq, fmaf(mn[it], gdy, sdyx));
        }
    }
    block_sum2(sdy, sdyx);
    if (threadIdx.x == 0) {
        a.partial[c * nchunks + chunk] = sdyx;            // -> dw
        a.partial[(a.g.C + c) * nchunks + chunk] = sdy;   // -> db
    }
}

template <int DYT, int MODE, int V, bool ALAM = false>
__global__ __launch_bounds__(TPB) void bn_bwd_dx_kernel(BnBwdArgs a, int lg, int bits) {
    const int64_t c = blockIdx.x;
    const int64_t M = a.g.N * a.g.HW;
    const int64_t base = (int64_t)blockIdx.y * BN_CHUNK + (int64_t)threadIdx.x * EPL;
    RowCursor cur[ITER];
    block_cursors(a.g, c, base, cur);
    float xh[ITER][EPL], dy[ITER][EPL];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        const int64_t e0 = base + it * WG_ELEMS;
        RowCursor p;
        int64_t e;
        block_or_first(a.g, c, cur[it], e0, M, p, e);
        bwd_operands<DYT, MODE, V, ALAM>(a, c, p, e, M, lg, bits, xh[it], dy[it]);
    }
    const float Mf = (float)M;
    float dws, dbs;
    if (a.dw_in) {
        dws = a.dw_in[c];
        dbs = a.db_in[c];
    } else {
        dws = partial_sum(a.partial + c * a.nchunks, a.nchunks);
        dbs = partial_sum(a.partial + (a.g.C + c) * a.nchunks, a.nchunks);
        if (blockIdx.y == 0 && threadIdx.x == 0) {
            a.dw[c] = dws;
            a.db[c] = dbs;
        }
    }
    const float dwm = dws / Mf, dbm = dbs / Mf;
    const float w = a.w[c];
    const float inv = a.var_is_invstd ? a.var[c] : 1.0f / sqrtf(a.var[c] + a.eps);
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        const int64_t e0 = base + it * WG_ELEMS;
        if (e0 >= M) break;
        float dx[EPL];
#pragma unroll
        for (int k = 0; k < EPL; ++k) dx[k] = (fmaf(-xh[it][k], dwm, dy[it][k] - dbm) * w) * inv;
        store8_bf16<V>(a.dx, a.g, cur[it], e0, M, dx);
    }
}

int log2i(int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

// kernel template for the vector width vw (8, 4, 2 or 1 elements per access)
#define DOPT_BN_BY_WIDTH(vw, LAUNCH) \
    do {                             \
        switch (vw) {                \
            case 8: LAUNCH(8); break; \
            case 4: LAUNCH(4); break; \
            case 2: LAUNCH(2); break; \
            default: LAUNCH(1); break; \
        }                            \
    } while (0)

template <int DT>
int fwd_dt(const BnFwdArgs& a, int mode, int group, int bits, int vw, hipStream_t s) {
    const int64_t M = a.g.N * a.g.HW;
    const int lg = mode == BN_NORM ? 3 : log2i(group);
    const dim3 grid((unsigned)a.g.C, (unsigned)bn_nchunks(M));
#define DOPT_BN_FWD(MODE_, V_) hipLaunchKernelGGL((bn_fwd_kernel<DT, MODE_, V_, false>), grid, dim3(TPB), 0, s, a, lg, bits)
#define DOPT_BN_FWD_RELU6(V_) hipLaunchKernelGGL((bn_fwd_kernel<DT, BN_RELU_QUANT, V_, true>), grid, dim3(TPB), 0, s, a, lg, bits)
#define DOPT_BN_FWD_ALAM(V_) hipLaunchKernelGGL((bn_fwd_kernel<DT, BN_QUANT, V_, false, true>), grid, dim3(TPB), 0, s, a, lg, bits)
#define DOPT_BN_FWD_THR(V_) hipLaunchKernelGGL((bn_fwd_kernel<DT, BN_QUANT, V_, false, false, true>), grid, dim3(TPB), 0, s, a, lg, bits)
#define DOPT_BN_FWD_NORM(V_) DOPT_BN_FWD(BN_NORM, V_)
#define DOPT_BN_FWD_QUANT(V_) DOPT_BN_FWD(BN_QUANT, V_)
#define DOPT_BN_FWD_RELU(V_) DOPT_BN_FWD(BN_RELU_QUANT, V_)
    if (mode == BN_NORM) DOPT_BN_BY_WIDTH(vw, DOPT_BN_FWD_NORM);
    else if (mode == BN_QUANT && a.alam_lg > 0) DOPT_BN_BY_WIDTH(vw, DOPT_BN_FWD_ALAM);
    else if (mode == BN_QUANT && bits <= 2) DOPT_BN_BY_WIDTH(vw, DOPT_BN_FWD_THR);
    else if (mode == BN_QUANT) DOPT_BN_BY_WIDTH(vw, DOPT_BN_FWD_QUANT);
    else if (mode == BN_RELU6_QUANT) DOPT_BN_BY_WIDTH(vw, DOPT_BN_FWD_RELU6);
    else DOPT_BN_BY_WIDTH(vw, DOPT_BN_FWD_RELU);
#undef DOPT_BN_FWD_THR
#undef DOPT_BN_FWD_RELU6
#undef DOPT_BN_FWD_ALAM
#undef DOPT_BN_FWD_RELU
#undef DOPT_BN_FWD_QUANT
#undef DOPT_BN_FWD_NORM
#undef DOPT_BN_FWD
    return 0;
}

template <int DYT>
int bwd_dt(const BnBwdArgs& a, int mode, int group, int bits, int vw, bool reduce, hipStream_t s, bool finalize) {
    const int64_t M = a.g.N * a.g.HW;
    const int lg = mode == BN_NORM ? 3 : log2i(group);
    const int64_t nch = bn_nchunks(M);
    const int m = mode == BN_RELU6_QUANT ? BN_RELU_QUANT : mode;
    const dim3 grid((unsigned)a.g.C, (unsigned)nch);
    if (reduce) {
#define DOPT_BN_RED(MODE_, V_) hipLaunchKernelGGL((bn_bwd_reduce_kernel<DYT, MODE_, V_>), grid, dim3(TPB), 0, s, a, lg, bits, nch)
#define DOPT_BN_RED_NORM(V_) DOPT_BN_RED(BN_NORM, V_)
#define DOPT_BN_RED_QUANT(V_) DOPT_BN_RED(BN_QUANT, V_)
#define DOPT_BN_RED_ALAM(V_) hipLaunchKernelGGL((bn_bwd_reduce_kernel<DYT, BN_QUANT, V_, true>), grid, dim3(TPB), 0, s, a, lg, bits, nch)
#define DOPT_BN_RED_RELU(V_) DOPT_BN_RED(BN_RELU_QUANT, V_)
        if (nch == 0) {
        } else if (m == BN_NORM) {
            DOPT_BN_BY_WIDTH(vw, DOPT_BN_RED_NORM);
        } else if (m == BN_QUANT && a.alam) {
            DOPT_BN_BY_WIDTH(vw, DOPT_BN_RED_ALAM);
        } else if (m == BN_QUANT) {
            DOPT_BN_BY_WIDTH(vw, DOPT_BN_RED_QUANT);
        } else {
            DOPT_BN_BY_WIDTH(vw, DOPT_BN_RED_RELU);
        }
#undef DOPT_BN_RED_RELU
#undef DOPT_BN_RED_ALAM
#undef DOPT_BN_RED_QUANT
#undef DOPT_BN_RED_NORM
#undef DOPT_BN_RED
        if (finalize)
            hipLaunchKernelGGL(bn_finalize_kernel, dim3((unsigned)a.g.C), dim3(64), 0, s, (const float*)a.partial,
                               a.g.C, nch, a.dw, a.db);
    } else {
#define DOPT_BN_DX(MODE_, V_) hipLaunchKernelGGL((bn_bwd_dx_kernel<DYT, MODE_, V_>), grid, dim3(TPB), 0, s, a, lg, bits)
#define DOPT_BN_DX_NORM(V_) DOPT_BN_DX(BN_NORM, V_)
#define DOPT_BN_DX_QUANT(V_) DOPT_BN_DX(BN_QUANT, V_)
#define DOPT_BN_DX_ALAM(V_) hipLaunchKernelGGL((bn_bwd_dx_kernel<DYT, BN_QUANT, V_, true>), grid, dim3(TPB), 0, s, a, lg, bits)
#define DOPT_BN_DX_RELU(V_) DOPT_BN_DX(BN_RELU_QUANT, V_)
        if (m == BN_NORM) DOPT_BN_BY_WIDTH(vw, DOPT_BN_DX_NORM);
        else if (m == BN_QUANT && a.alam_lg > 0) DOPT_BN_BY_WIDTH(vw, DOPT_BN_DX_ALAM);
        else if (m == BN_QUANT) DOPT_BN_BY_WIDTH(vw, DOPT_BN_DX_QUANT);
        else DOPT_BN_BY_WIDTH(vw, DOPT_BN_DX_RELU);
#undef DOPT_BN_DX_RELU
#undef DOPT_BN_DX_ALAM
#undef DOPT_BN_DX_QUANT
#undef DOPT_BN_DX_NORM
#undef DOPT_BN_DX
    }
    return 0;
}

}  // namespace

int64_t bn_nchunks(int64_t M) { return (M + BN_CHUNK - 1) / BN_CHUNK; }

int launch_bn_reduce(const void* x, int dt, const BnGeom& g, float* partial, float* sum, float* sumsq, int vw,
                     hipStream_t s, bool finalize) {
    const int64_t M = g.N * g.HW;
    const int64_t nch = bn_nchunks(M);
    const dim3 grid((unsigned)g.C, (unsigned)nch);
#define DOPT_BN_STATS(DT_, V_) hipLaunchKernelGGL((bn_stats_kernel<DT_, V_>), grid, dim3(TPB), 0, s, x, g, partial, nch)
#define DOPT_BN_STATS_F32(V_) DOPT_BN_STATS(DT_F32, V_)
#define DOPT_BN_STATS_F16(V_) DOPT_BN_STATS(DT_F16, V_)
#define DOPT_BN_STATS_BF16(V_) DOPT_BN_STATS(DT_BF16, V_)
    if (nch > 0) {
        switch (dt) {
            case DT_F32: DOPT_BN_BY_WIDTH(vw, DOPT_BN_STATS_F32); break;
            case DT_F16: DOPT_BN_BY_WIDTH(vw, DOPT_BN_STATS_F16); break;
            default: DOPT_BN_BY_WIDTH(vw, DOPT_BN_STATS_BF16); break;
        }
    }
#undef DOPT_BN_STATS_BF16
#undef DOPT_BN_STATS_F16
#undef DOPT_BN_STATS_F32
#undef DOPT_BN_STATS
    if (finalize)
        hipLaunchKernelGGL(bn_finalize_kernel, dim3((unsigned)g.C), dim3(64), 0, s, (const float*)partial, g.C, nch,
                           sum, sumsq);
    return 0;
}

int launch_bn_fwd(const BnFwdArgs& a, int dt, int mode, int group, int bits, int vw, hipStream_t s) {
    switch (dt) {
        case DT_F32: return fwd_dt<DT_F32>(a, mode, group, bits, vw, s);
        case DT_F16: return fwd_dt<DT_F16>(a, mode, group, bits, vw, s);
        default: return fwd_dt<DT_BF16>(a, mode, group, bits, vw, s);
    }
}

int launch_bn_bwd_reduce(const BnBwdArgs& a, int dyt, int mode, int group, int bits, int vw, hipStream_t s,
                         bool finalize) {
    switch (dyt) {
        case DT_F32: return bwd_dt<DT_F32>(a, mode, group, bits, vw, true, s, finalize);
        case DT_F16: return bwd_dt<DT_F16>(a, mode, group, bits, vw, true, s, finalize);
        default: return bwd_dt<DT_BF16>(a, mode, group, bits, vw, true, s, finalize);
    }
}

int launch_bn_bwd_dx(const BnBwdArgs& a, int dyt, int mode, int group, int bits, int vw, hipStream_t s) {
    switch (dyt) {
        case DT_F32: return bwd_dt<DT_F32>(a, mode, group, bits, vw, false, s, false);
        case DT_F16: return bwd_dt<DT_F16>(a, mode, group, bits, vw, false, s, false);
        default: return bwd_dt<DT_BF16>(a, mode, group, bits, vw, false, s, false);
    }
}

}  // namespace dopt
