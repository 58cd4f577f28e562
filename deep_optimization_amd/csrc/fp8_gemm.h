// FP8 (OCP e4m3) scaled GEMM on CDNA4 MFMA, NT layout (A [M,K], B [N,K], both K-contiguous):
//   C[m][n] = bf16(out_scale * sum_k A[m][k] * B[n][k]), fp32 accumulation, one rounding.
// Any M, N >= 0; K a multiple of 16 (one 16-byte load per lane); A, B rows 16-byte aligned.
//
// Three kernels share the tiling below: fp8_gemm_nt_kernel computes one tile per workgroup, and
// fp8_gemm_nt_persistent_kernel and fp8_gemm16_persistent_kernel (further down, the launcher's
// choice for an even, non-zero number of K slabs; the second on 16x16x128 MFMAs for large K) run
// one workgroup per CU over a list of tiles.
//
// Tiling: a workgroup of 4 waves (2 x 2) computes a BM x BN tile; each wave a (BM/2) x (BN/2)
// sub-tile as TM x TN blocks of v_mfma_f32_32x32x64_f8f6f4 (fp8 x fp8 -> fp32, 32 x 32 x 64 per
// instruction, 16 accumulator registers per block). At 128 x 128 per wave one 128-byte K slab
// is 32 MFMAs fed by 16 KB of LDS operand reads per wave, half the LDS bandwidth of a CU.
//
// Data movement: K advances in slabs of BK = 128 bytes, double-buffered in LDS (no padding:
// 2 * (BM + BN) * 128 bytes). Slabs go HBM/L2 -> LDS with buffer_load_dwordx4 ... lds (no
// staging registers): one instruction moves 64 lanes x 16 bytes into a contiguous 1 KB LDS
// block, i.e. 8 rows of 128 bytes (whole cache lines). The lane -> global address mapping
// applies an XOR swizzle, so 16-byte chunk c of row r lands at chunk position c ^ ((r / 2) % 8).
// gfx950's LDS serves a ds_read_b128 16 lanes at a time across 64 banks (256 bytes): an even
// and an odd row share one bank row, so the 16 consecutive rows of an operand fetch hit 16
// distinct 16-byte bank groups (measured: the plain c ^ (r % 8) swizzle left half of all LDS
// cycles in bank conflicts). The loads go through a range-checked buffer resource: a lane whose
// row lies beyond M (or N) or whose 16 bytes lie beyond K gets an offset past the resource's
// range, which the hardware turns into zeros without a memory access, so edge tiles need no
// other masking until the stores, and slabs past the end load nothing.
//
// Pipeline (one barrier per slab, placed mid-slab):
//   MFMAs of half 0 | ds_read operands of half 1 | wait LDS reads + slab k+1 loads | barrier |
//   issue loads of slab k+2 into this buffer | ds_read half 0 of slab k+1 | MFMAs of half 1
// so the global loads of the next-but-one slab and the operand reads of the next slab overlap
// the second half of the MFMAs.
//
// MFMA operand layout (fp8, 32x32x64): lane l supplies row (l % 32) of its operand and 32
// consecutive K bytes starting at 32*(l / 32); A and B use the same K mapping, so the dot
// products pair matching k. Accumulator layout: lane l holds column l % 32 and, in register v,
// row 8*(v/4) + 4*(l/32) + (v%4). The epilogue scales, rounds to bf16, transposes through LDS
// and writes 16-byte row chunks inside M x N (element stores for a ragged last chunk or an
// unaligned C).
//
// Workgroup order: the hardware hands consecutive workgroup ids to the 8 XCDs in turn, each XCD
// with its own L2. The id is remapped so that each XCD owns a contiguous range of tiles, walked
// in groups of GROUP_M tile rows, so the A rows and B columns one XCD streams stay in its L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "dopt_device.h"

namespace dopt {

typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));
typedef uint32_t v2u_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ v16f_t mfma_fp8_32x32x64(const v8i_t& a, const v8i_t& b, const v16f_t& c) {
    // cbsz = blgp = 0: both operands OCP fp8 e4m3; scale operands 0 select the unscaled MFMA.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

constexpr int GEMM_XCDS = 8;
constexpr uint32_t GEMM_OOB = 0x80000000u;    // buffer offset past the range: the load returns zeros
constexpr uint32_t GEMM_RANGE = 0x7FFFFF00u;  // num_records of the operand resources

struct Fp8GemmArgs {
    const uint8_t* A;
    const uint8_t* B;
    uint16_t* C;
    int64_t M, N, K, lda, ldb, ldc;
    float out_scale;
    uint32_t tiles_m, tiles_n;
    uint32_t vec_store;  // C 16-byte aligned with ldc % 8 == 0: whole chunks go out as 16-byte stores
};

template <int BM_, int BN_, int GROUP_M_, int SCHED_ = 1>
struct Fp8GemmCfg {
    static constexpr int BM = BM_, BN = BN_, BK = 128, GROUP_M = GROUP_M_;
    static constexpr int SCHED = SCHED_;  // 0: even MFMA/memory interleave, 1: LDS reads front-loaded
    static constexpr int THREADS = 256;
    static constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
    static constexpr int TM = WM / 32, TN = WN / 32;
    static constexpr int LA = BM / 32, LB = BN / 32;  // global_load_lds per wave per slab
    static constexpr int LDS_BYTES = 2 * (BM + BN) * BK;
    static_assert(BM == BN && (BM == 128 || BM == 256), "square 128 or 256 tiles (epilogue staging)");
    static_assert(WM * WN * 2 <= BN * BK, "a wave's bf16 tile fits one LDS array");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of one CU");
};

template <class C, bool EDGE>
__global__ __launch_bounds__(256, 1) void fp8_gemm_nt_kernel(Fp8GemmArgs p) {
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, TM = C::TM, TN = C::TN, WM = C::WM, WN = C::WN;
    const int64_t M = p.M, N = p.N, K = p.K, lda = p.lda, ldb = p.ldb, ldc = p.ldc;
    // four separate LDS objects (A and B, two buffers each): the compiler can then prove that an
    // operand read of one buffer does not alias the in-flight global_load_lds writes into the
    // other, and does not make the read wait for those loads
    __shared__ __attribute__((aligned(1024))) uint8_t sA0[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sA1[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sB0[BN * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sB1[BN * BK];

    // ---- XCD-aware tile order: XCD x receives ids x, x+8, x+16, ... (local index bid/8) and
    // owns the contiguous tile range [x*per + min(x, rem), ... + per + (x < rem)), a bijection
    const uint32_t tiles_m = p.tiles_m, tiles_n = p.tiles_n;
    const uint32_t n_tiles = tiles_m * tiles_n;
    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid % GEMM_XCDS, local = bid / GEMM_XCDS;
    const uint32_t per = n_tiles / GEMM_XCDS, rem = n_tiles % GEMM_XCDS;
    const uint32_t t = xcd * per + min(xcd, rem) + local;
    // grouped walk: GROUP_M tile rows at a time, column-major inside the group
    const uint32_t group = C::GROUP_M * tiles_n;
    const uint32_t first_m = (t / group) * C::GROUP_M;
    const uint32_t gsize = min(tiles_m - first_m, (uint32_t)C::GROUP_M);
    const uint32_t tm = first_m + (t % group) % gsize;
    const uint32_t tn = (t % group) / gsize;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)tm * BM;
    const int64_t n0 = (int64_t)tn * BN;

    // ---- global -> LDS slab loads: instruction j of wave w fills the 1 KB block (j*4 + w), rows
    // r = 8*(j*4 + w) + lane/8, chunk position lane%8 <- global chunk (lane%8) ^ ((r/2) % 8),
    // where (r/2) % 8 = (4*(w % 2) + lane/16) % 8 does not depend on j
    const int lrow8 = lane >> 3;
    const int lchunk = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.A + m0 * lda), (short)0, (int)GEMM_RANGE, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.B + n0 * ldb), (short)0, (int)GEMM_RANGE, 0x00020000);
    const int r0 = 8 * wave + lrow8;  // row of instruction j: 32 j + r0
    const int rows_a = (int)min((int64_t)BM, M - m0) - r0, rows_b = (int)min((int64_t)BN, N - n0) - r0;
    const uint32_t offa0 = (uint32_t)(r0 * lda + lchunk * 16), offb0 = (uint32_t)(r0 * ldb + lchunk * 16);
    const uint32_t stepa = (uint32_t)(32 * lda), stepb = (uint32_t)(32 * ldb);
    // EDGE = false (M, N multiples of the tile and K of BK, the common case): only the slabs past
    // K are out of range, a wave-uniform test. EDGE = true: lanes past K and rows past M (N) get
    // GEMM_OOB (selects, no branches; about 2% slower at 8192^3).
    auto issue = [&](uint8_t* sa, uint8_t* sb, int64_t k0, auto edge) __attribute__((always_inline)) {
        constexpr bool E = decltype(edge)::value;
        int la = C::BM, lb = C::BN;
        if constexpr (E) {
            const bool k_ok = k0 + lchunk * 16 < K;
            la = k_ok ? rows_a : 0;
            lb = k_ok ? rows_b : 0;
        }
        const uint32_t kk = k0 < K ? (uint32_t)k0 : GEMM_OOB;
#pragma unroll
        for (int j = 0; j < C::LA; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sa + wave * 1024 + j * 4096), 16,
                                                     !E || 32 * j < la ? offa0 + j * stepa + kk : GEMM_OOB, 0, 0,
                                                     0);
#pragma unroll
        for (int j = 0; j < C::LB; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sb + wave * 1024 + j * 4096), 16,
                                                     !E || 32 * j < lb ? offb0 + j * stepb + kk : GEMM_OOB, 0, 0,
                                                     0);
    };

    // ---- operand reads: tile i of the wave = rows base + i*32 + lane%32; K half h of the slab
    // is logical chunks 4h + 2*(lane/32) + {0, 1}, stored at chunk position c ^ ((row/2) % 8)
    const int orow = lane & 31;
    const int oc = 2 * (lane >> 5);
    const int sw = (lane >> 1) & 7;  // (row/2) % 8 of this lane's operand rows (base rows are multiples of 16)
    auto read_ops = [&](const uint8_t* sa, const uint8_t* sb, int h, v8i_t* a, v8i_t* b) __attribute__((always_inline)) {
        const uint8_t* la = sa + (WM * wm + orow) * BK;
        const uint8_t* lb = sb + (WN * wn + orow) * BK;
        const int p0 = ((4 * h + oc) ^ sw) * 16, p1 = ((4 * h + oc + 1) ^ sw) * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const uint4 x0 = *(const uint4*)(la + i * 32 * BK + p0);
            const uint4 x1 = *(const uint4*)(la + i * 32 * BK + p1);
            a[i] = v8i_t{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint4 x0 = *(const uint4*)(lb + j * 32 * BK + p0);
            const uint4 x1 = *(const uint4*)(lb + j * 32 * BK + p1);
            b[j] = v8i_t{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        }
    };

    v16f_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    v8i_t a0[TM], b0[TN], a1[TM], b1[TN];
    auto mma = [&](const v8i_t* a, const v8i_t* b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma_fp8_32x32x64(a[i], b[j], acc[i][j]);
    };
    // one slab: (sa, sb) hold slab kt, (na, nb) slab kt+1 (loads in flight), half 0 operands of
    // slab kt already in a0/b0. The body is branch-free: the last two slabs still issue a load
    // (past K: every lane out of range, so zeros into a buffer nobody reads any more) and read
    // the next buffer's half 0 (unused), so every slab is one scheduling region pair. The
    // sched_group_barrier hints interleave one MFMA with the LDS reads / global loads that run
    // beside it, so the in-order issue never parks a memory instruction behind a run of MFMAs.
    const int nk = (int)((K + BK - 1) / BK);
    auto slab = [&](int kt, uint8_t* sa, uint8_t* sb, uint8_t* na, uint8_t* nb, auto edge) __attribute__((always_inline)) {
        constexpr int NM = TM * TN;        // MFMAs per half slab
        constexpr int NR = 2 * (TM + TN);  // ds_read_b128 per half slab
        read_ops(sa, sb, 1, a1, b1);
        mma(a0, b0);
        if constexpr (C::SCHED == 0) {
#pragma unroll
            for (int q = 0; q < NM; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            }
        } else {
            // LDS reads in the first half of the region, two per MFMA, so their latency is
            // covered by the MFMAs that follow before the wait at the barrier
#pragma unroll
            for (int q = 0; q < NR / 2; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - NR / 2, 0);
        }
        // every LDS read of (sa, sb) and every load of slab kt+1 has landed, in all waves
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        issue(sa, sb, (int64_t)(kt + 2) * BK, edge);
        read_ops(na, nb, 0, a0, b0);
        mma(a1, b1);
        if constexpr (C::SCHED == 0) {
#pragma unroll
            for (int q = 0; q < NM; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            }
        } else {
            // next slab's half-0 operands first (consumed at the top of the next slab), then the
            // global loads of slab kt+2 (consumed a slab later)
#pragma unroll
            for (int q = 0; q < NR / 2; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
#pragma unroll
            for (int q = 0; q < NM - NR / 2; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
            }
        }
    };

    const std::integral_constant<bool, EDGE> edge{};
    issue(sA0, sB0, 0, edge);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    issue(sA1, sB1, (int64_t)BK, edge);
    read_ops(sA0, sB0, 0, a0, b0);
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        slab(kt, sA0, sB0, sA1, sB1, edge);
        slab(kt + 1, sA1, sB1, sA0, sB0, edge);
    }
    if (kt < nk) slab(kt, sA0, sB0, sA1, sB1, edge);
    // the trailing loads must land before LDS is reused below
    __builtin_amdgcn_s_waitcnt(0);

    // ---- epilogue: scale, round once to bf16, transpose through LDS, 16-byte row stores.
    // Wave w stages its WM x WN bf16 tile in one of the four LDS arrays (each >= WM*WN*2 bytes).
    __syncthreads();
    uint16_t* tile = (uint16_t*)(wave == 0 ? sA0 : wave == 1 ? sA1 : wave == 2 ? sB0 : sB1);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = j * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                tile[row * WN + col] = to_bf16(acc[i][j][v] * p.out_scale);
            }
        }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    constexpr int CPR = WN / 8;  // 16-byte chunks per tile row
    const int64_t row0 = m0 + WM * wm, col0 = n0 + WN * wn;
    uint16_t* cbase = p.C + row0 * ldc + col0;
#pragma unroll 4
    for (int q = lane; q < WM * CPR; q += 64) {
        const int row = q / CPR, c = q % CPR;
        if (row0 + row >= M) continue;
        const int64_t n = col0 + c * 8;
        if (p.vec_store && n + 8 <= N) {
            *(uint4*)(cbase + row * ldc + c * 8) = *(const uint4*)(tile + row * WN + c * 8);
        } else {
            for (int e = 0; e < 8 && n + e < N; ++e) cbase[row * ldc + c * 8 + e] = tile[row * WN + c * 8 + e];
        }
    }
}

template <class C>
inline int fp8_gemm_launch(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K, int64_t lda,
                           int64_t ldb, float out_scale, uint16_t* Cm, int64_t ldc, hipStream_t s) {
    Fp8GemmArgs p{A, B, Cm, M, N, K, lda, ldb, ldc, out_scale, (uint32_t)((M + C::BM - 1) / C::BM),
                  (uint32_t)((N + C::BN - 1) / C::BN), (uint32_t)(ldc % 8 == 0 && ((uintptr_t)Cm & 15) == 0)};
    const uint64_t tiles = (uint64_t)p.tiles_m * p.tiles_n;
    if (tiles == 0) return 0;
    if (M % C::BM == 0 && N % C::BN == 0 && K % C::BK == 0)
        hipLaunchKernelGGL((fp8_gemm_nt_kernel<C, false>), dim3((uint32_t)tiles), dim3(C::THREADS), 0, s, p);
    else
        hipLaunchKernelGGL((fp8_gemm_nt_kernel<C, true>), dim3((uint32_t)tiles), dim3(C::THREADS), 0, s, p);
    return 0;
}

// ---------------------------------------------------------------------------------------------
// Persistent form: one workgroup per CU walks a list of tiles, and its slab pipeline runs across
// tile boundaries. The loads of a tile's first two slabs are issued during the last two slabs of
// the previous tile, so a tile starts with its operands in LDS. The epilogue stages through an
// LDS array of its own (32 rows of a wave's tile at a time), so its C stores drain while the
// next tile's MFMAs run.
//
// Tile list: XCD x (workgroup ids x, x+8, ...) owns the contiguous tile range of the
// non-persistent kernel; its g_x workgroups take tiles first + local, first + local + g_x, ...,
// so at any time the XCD's workgroups work on neighbouring tiles of one GROUP_M group.
//
// The MFMA takes B's fragment as its first operand and A's as its second, which transposes the
// accumulator: lane l holds row i*32 + l%32 of A's tile and, in registers 4q..4q+3, the four
// consecutive columns j*32 + 8q + 4*(l/32) + {0..3}: lanes l and l + 32 hold the two 8-byte halves
// of the 16-byte chunk of columns j*32 + 8q + {0..7}. For a pair q, q + 1 one v_permlane32_swap
// per dword gives lane l the whole chunk q and lane l + 32 the whole chunk q + 1, so the staging
// rows are written with 16-byte stores (8-byte stores of the halves measured 2^20 LDS bank-conflict
// cycles per 8192^3 call; whole chunks, 16 lanes to a 256-byte bank row, none), and 16-byte row
// chunks go out with whole-row coalescing.
template <class C, bool EDGE>
__global__ __launch_bounds__(256, 1) void fp8_gemm_nt_persistent_kernel(Fp8GemmArgs p) {
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, TM = C::TM, TN = C::TN, WM = C::WM, WN = C::WN;
    constexpr int CPR = WN / 8;             // 16-byte chunks per staged row
    constexpr int ESTAGE = 32 * WN * 2;     // bytes staged per wave: 32 rows of its tile
    static_assert(CPR == 8 || CPR == 16, "staging swizzle");
    const int64_t M = p.M, N = p.N, K = p.K, lda = p.lda, ldb = p.ldb, ldc = p.ldc;
    __shared__ __attribute__((aligned(1024))) uint8_t sA0[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sA1[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sB0[BN * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sB1[BN * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sE[4 * ESTAGE];

    // ---- this workgroup's tiles
    const uint32_t tiles_m = p.tiles_m, tiles_n = p.tiles_n;
    const uint32_t n_tiles = tiles_m * tiles_n;
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t xcd = bid % GEMM_XCDS, local = bid / GEMM_XCDS;
    const uint32_t g_x = G / GEMM_XCDS + (xcd < G % GEMM_XCDS ? 1u : 0u);
    const uint32_t per = n_tiles / GEMM_XCDS, rem = n_tiles % GEMM_XCDS;
    const uint32_t first = xcd * per + min(xcd, rem), cnt = per + (xcd < rem ? 1u : 0u);
    const uint32_t my = local < cnt ? (cnt - local + g_x - 1) / g_x : 0u;
    const uint32_t nk = (uint32_t)((K + BK - 1) / BK);
    const uint32_t total = my * nk;
    if (total == 0) return;  // the same for every wave of the workgroup
    auto coords = [&](uint32_t i, uint32_t& tm, uint32_t& tn) __attribute__((always_inline)) {
        const uint32_t t = first + local + i * g_x;
        const uint32_t group = C::GROUP_M * tiles_n;
        const uint32_t first_m = (t / group) * C::GROUP_M;
        const uint32_t gsize = min(tiles_m - first_m, (uint32_t)C::GROUP_M);
        tm = first_m + (t % group) % gsize;
        tn = (t % group) / gsize;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: tile bases stay scalar
    const int wm = wave >> 1, wn = wave & 1;

    // ---- global -> LDS slab loads (lane mapping and swizzle as in fp8_gemm_nt_kernel), two slabs
    // ahead of the compute side
    const int lrow8 = lane >> 3;
    const int lchunk = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    const int r0 = 8 * wave + lrow8;
    const uint32_t offa0 = (uint32_t)(r0 * lda + lchunk * 16), offb0 = (uint32_t)(r0 * ldb + lchunk * 16);
    const uint32_t stepa = (uint32_t)(32 * lda), stepb = (uint32_t)(32 * ldb);
    // Tile it's slabs are issued from cur_t's buffer resources and tile it+1's from next_t's: slab
    // k of the compute side issues slab k+2 of the stream, which for the last two slabs of a tile
    // is slab k+2-nk of the next tile. The choice is a set of scalar selects, so a slab has no
    // branches and the next slab's operand reads stay interleaved with its MFMAs.
    struct IssueTile {
        __amdgpu_buffer_rsrc_t ra, rb;
        int rows_a, rows_b;
        bool live;
    };
    auto issue_tile = [&](uint32_t i) __attribute__((always_inline)) {
        IssueTile t;
        uint32_t tm, tn;
        t.live = i < my;
        coords(t.live ? i : my - 1, tm, tn);
        const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
        t.ra = __builtin_amdgcn_make_buffer_rsrc((void*)(p.A + m0 * lda), (short)0, (int)GEMM_RANGE, 0x00020000);
        t.rb = __builtin_amdgcn_make_buffer_rsrc((void*)(p.B + n0 * ldb), (short)0, (int)GEMM_RANGE, 0x00020000);
        t.rows_a = EDGE ? (int)min((int64_t)BM, M - m0) - r0 : BM;
        t.rows_b = EDGE ? (int)min((int64_t)BN, N - n0) - r0 : BN;
        return t;
    };
    IssueTile cur_t = issue_tile(0), next_t = issue_tile(1);
    // The lane's row/chunk offset goes in voffset, the wave-uniform row-block and K offsets in
    // soffset. A lane that must load nothing (a slab past this workgroup's last tile; with EDGE a
    // row past M or N or 16 bytes past K) gets voffset GEMM_OOB, past the resource's range.
    auto issue = [&](uint8_t* sa, uint8_t* sb, uint32_t ks) __attribute__((always_inline)) {
        const bool nxt = ks >= nk;
        const __amdgpu_buffer_rsrc_t ra = nxt ? next_t.ra : cur_t.ra;
        const __amdgpu_buffer_rsrc_t rb = nxt ? next_t.rb : cur_t.rb;
        const bool live = nxt ? next_t.live : cur_t.live;
        const int64_t k0 = (int64_t)(nxt ? ks - nk : ks) * BK;
        const uint32_t va = live ? offa0 : GEMM_OOB, vb = live ? offb0 : GEMM_OOB;
        int la = C::BM, lb = C::BN;
        if constexpr (EDGE) {
            const bool k_ok = k0 + lchunk * 16 < K;
            la = k_ok ? (nxt ? next_t.rows_a : cur_t.rows_a) : 0;
            lb = k_ok ? (nxt ? next_t.rows_b : cur_t.rows_b) : 0;
        }
#pragma unroll
        for (int j = 0; j < C::LA; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sa + wave * 1024 + j * 4096), 16,
                                                     !EDGE || 32 * j < la ? va : GEMM_OOB,
                                                     (int)(j * stepa + (uint32_t)k0), 0, 0);
#pragma unroll
        for (int j = 0; j < C::LB; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sb + wave * 1024 + j * 4096), 16,
                                                     !EDGE || 32 * j < lb ? vb : GEMM_OOB,
                                                     (int)(j * stepb + (uint32_t)k0), 0, 0);
    };

    const int orow = lane & 31;
    const int oc = 2 * (lane >> 5);
    const int sw = (lane >> 1) & 7;
    // LDS accesses use native vector types and shallow address arithmetic: a HIP uint4 access is
    // split into four dword accesses a level deeper, past the depth to which the LDS lowering
    // attaches the alias scopes that tell the compiler an operand read does not touch the buffer
    // an in-flight global -> LDS load is writing (without them it waits for those loads)
    auto read_ops = [&](const uint8_t* sa, const uint8_t* sb, int h, v8i_t* a, v8i_t* b) __attribute__((always_inline)) {
        const int ra0 = (WM * wm + orow) * BK, rb0 = (WN * wn + orow) * BK;
        const int p0 = ((4 * h + oc) ^ sw) * 16, p1 = ((4 * h + oc + 1) ^ sw) * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const v4u_t x0 = *(const v4u_t*)(sa + (ra0 + i * 32 * BK + p0));
            const v4u_t x1 = *(const v4u_t*)(sa + (ra0 + i * 32 * BK + p1));
            a[i] = __builtin_bit_cast(v8i_t, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const v4u_t x0 = *(const v4u_t*)(sb + (rb0 + j * 32 * BK + p0));
            const v4u_t x1 = *(const v4u_t*)(sb + (rb0 + j * 32 * BK + p1));
            b[j] = __builtin_bit_cast(v8i_t, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };

    v16f_t acc[TM][TN];
    auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    };
    zero_acc();
    v8i_t a0[TM], b0[TN], a1[TM], b1[TN];
    auto mma = [&](const v8i_t* a, const v8i_t* b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma_fp8_32x32x64(b[j], a[i], acc[i][j]);
    };

    // ---- epilogue of compute tile i: scale, round once to bf16, stage 32 rows of the wave's
    // tile at a time (16-byte chunk c of row r at position c ^ (r % CPR)), store row chunks
    uint8_t* stage = sE + wave * ESTAGE;
    auto epilogue = [&](uint32_t i_tile) __attribute__((always_inline)) {
        uint32_t tm, tn;
        coords(i_tile, tm, tn);
        const int64_t row0 = (int64_t)tm * BM + WM * wm, col0 = (int64_t)tn * BN + WN * wn;
        // the lane index passes through an empty asm so that the addresses below are computed
        // here, once per tile, instead of being hoisted out of the tile loop into registers
        int ln = lane;
        asm volatile("" : "+v"(ln));
        uint32_t ldc2 = (uint32_t)ldc * 2;  // row pitch of C in bytes (< GEMM_RANGE / BM on this path)
        asm volatile("" : "+s"(ldc2));
        const int er = ln & 31, h = ln >> 5;
        const int rr = ln / CPR, rc = ln % CPR;  // read side: row rr + r * (64 / CPR), chunk rc
        // whole tiles: one buffer resource per tile, the lane's offset in voffset and the row
        // block's in soffset
        const __amdgpu_buffer_rsrc_t rcs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.C + row0 * ldc + col0), (short)0, (int)GEMM_RANGE, 0x00020000);
        const uint32_t vo = (uint32_t)rr * ldc2 + (uint32_t)rc * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                // one 32 x 32 block's accumulators move to VGPRs here, not all of them at once
                v16f_t t = acc[i][j];
                asm volatile("" : "+v"(t));
#pragma unroll
                for (int q = 0; q < 4; q += 2) {
                    // own halves of chunks q and q + 1; after the swaps lane l holds chunk q and
                    // lane l + 32 chunk q + 1, both as {x[0], y[0], x[1], y[1]}
                    const uint32_t w0x = pack_bf16x2(t[4 * q] * p.out_scale, t[4 * q + 1] * p.out_scale);
                    const uint32_t w0y = pack_bf16x2(t[4 * q + 2] * p.out_scale, t[4 * q + 3] * p.out_scale);
                    const uint32_t w1x = pack_bf16x2(t[4 * q + 4] * p.out_scale, t[4 * q + 5] * p.out_scale);
                    const uint32_t w1y = pack_bf16x2(t[4 * q + 6] * p.out_scale, t[4 * q + 7] * p.out_scale);
                    const auto x = __builtin_amdgcn_permlane32_swap(w0x, w1x, false, false);
                    const auto y = __builtin_amdgcn_permlane32_swap(w0y, w1y, false, false);
                    const v4u_t chunk = {x[0], y[0], x[1], y[1]};
                    const int c = 4 * j + q + h;
                    *(v4u_t*)(stage + (er * (WN * 2) + ((c ^ (er & (CPR - 1))) * 16))) = chunk;
                }
            }
#pragma unroll
            for (int r = 0; r < 32 * CPR / 64; ++r) {
                const int row = rr + r * (64 / CPR);
                const v4u_t v = *(const v4u_t*)(stage + (row * (WN * 2) + ((rc ^ (row & (CPR - 1))) * 16)));
                const int grow = i * 32 + row;
                if constexpr (!EDGE) {
                    __builtin_amdgcn_raw_buffer_store_b128(v, rcs, vo,
                                                           (int)((uint32_t)(i * 32 + r * (64 / CPR)) * ldc2), 0);
                } else {
                    if (row0 + grow >= M) continue;
                    const int64_t n = col0 + rc * 8;
                    uint16_t* dst = p.C + (row0 + grow) * ldc + n;
                    if (p.vec_store && n + 8 <= N) {
                        *(v4u_t*)dst = v;
                    } else {
                        const uint16_t e8[8] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y,
                                                (uint16_t)(v.y >> 16), (uint16_t)v.z, (uint16_t)(v.z >> 16),
                                                (uint16_t)v.w, (uint16_t)(v.w >> 16)};
                        for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = e8[e];
                    }
                }
            }
        }
    };

    // ---- one slab of the stream: buffer PAR holds slab s, the other buffer slab s+1 (loads in
    // flight), half 0 operands of slab s in a0/b0; schedule as the even interleave of
    // fp8_gemm_nt_kernel. The LAST slab of a tile leaves the next slab's half-0 operand read to
    // after the epilogue, which then has the operand registers to itself.
    // Vector memory operations complete in issue order and vmcnt counts stores too: in the slab
    // after an epilogue the wait at the barrier is vmcnt(EPI_STORES), which covers the slab loads
    // issued before the epilogue's stores and leaves those stores in flight. That takes the
    // epilogue's exact store count: whole-chunk stores only (no EDGE instance, aligned C).
    constexpr int EPI_STORES = TM * (32 * CPR / 64);
    static_assert(EPI_STORES < 64, "vmcnt field");
    constexpr int WAIT_EPI = (EPI_STORES & 15) | ((EPI_STORES >> 4) << 14) | (7 << 4);  // lgkmcnt(0)
    auto slab = [&](uint8_t* sa, uint8_t* sb, uint8_t* na, uint8_t* nb, uint32_t k, auto last, auto epi)
                    __attribute__((always_inline)) {
        constexpr bool LAST = decltype(last)::value;
        constexpr bool AFTER_EPI = decltype(epi)::value && !EDGE;
        constexpr int NM = TM * TN;
        read_ops(sa, sb, 1, a1, b1);
        mma(a0, b0);
#pragma unroll
        for (int q = 0; q < NM; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (AFTER_EPI) __builtin_amdgcn_s_waitcnt(WAIT_EPI);
        else __builtin_amdgcn_s_waitcnt(0);
        // a bare barrier: __syncthreads' release fence would wait for the epilogue's stores; the
        // memory clobber keeps the compiler from moving memory operations across it
        asm volatile("s_barrier" ::: "memory");
        issue(sa, sb, k + 2);
        if constexpr (!LAST) read_ops(na, nb, 0, a0, b0);
        mma(a1, b1);
        if constexpr (LAST) {
#pragma unroll
            for (int q = 0; q < NM; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        } else {
#pragma unroll
            for (int q = 0; q < NM; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
    };
    using BF = std::integral_constant<bool, false>;
    using BT = std::integral_constant<bool, true>;

    issue(sA0, sB0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    issue(sA1, sB1, 1);
    read_ops(sA0, sB0, 0, a0, b0);
    // nk is even, so every tile starts in buffer 0. The first slab of each later tile follows its
    // predecessor's epilogue in straight-line code, so that the compiler's own wait bookkeeping
    // sees the stores in flight on one path only and adds no waits of its own to that slab.
    slab(sA0, sB0, sA1, sB1, 0, BF{}, BF{});
    for (uint32_t it = 0;;) {
        for (uint32_t k = 1; k + 2 < nk; k += 2) {
            slab(sA1, sB1, sA0, sB0, k, BF{}, BF{});
            slab(sA0, sB0, sA1, sB1, k + 1, BF{}, BF{});
        }
        slab(sA1, sB1, sA0, sB0, nk - 1, BT{}, BF{});
        __builtin_amdgcn_sched_barrier(0);
        epilogue(it);
        __builtin_amdgcn_sched_barrier(0);
        zero_acc();
        // the next slab's loads were covered by the last slab's wait
        read_ops(sA0, sB0, 0, a0, b0);
        if (++it == my) break;
        cur_t = next_t;
        next_t = issue_tile(it + 1);
        slab(sA0, sB0, sA1, sB1, 0, BF{}, BT{});
    }
    // the loads issued past the last slab write zeros into LDS: they land before the workgroup ends
    __builtin_amdgcn_s_waitcnt(0);
}

// ---------------------------------------------------------------------------------------------
// The same persistent kernel on v_mfma_f32_16x16x128_f8f6f4 (fp8 x fp8 -> fp32, 16 x 16 x 128 per
// instruction, half the work of the 32x32x64 form in half its cycles). On training-like operands
// the part's clock follows its power draw, and an MFMA stream of this shape draws less per flop:
// an instruction-stream probe sustains 3.96 PF/s against 3.47 for 32x32x64 on random e4m3 data
// (4.8 PF/s for both on constant data). At 8192^3 the kernel takes ~2% more cycles than
// fp8_gemm_nt_persistent_kernel and runs ~5% faster on random operands; at K = 4096 the two are
// within noise of each other, so the launcher picks this form for K >= FP8_MFMA16_MIN_K.
//
// Same tiles, tile list, LDS buffers and buffer-resource loads as fp8_gemm_nt_persistent_kernel.
// A wave's 128 x 128 tile is 8 x 8 blocks of 16 x 16; fragment i of A (and of B) is 16 rows x
// 128 K bytes, lane l supplying row l % 16 and the 32 K bytes from 32 (l / 16): two 16-byte LDS
// reads. The MFMA takes B's fragment first, so lane l holds row 16 i + l % 16 and columns
// 16 j + 4 (l / 16) + {0..3} of block (i, j). The epilogue pairs fragment rows 2i and 2i + 1:
// one v_permlane16_swap per dword gives lanes with even l / 16 the whole 16-byte chunk of row
// l % 16 and lanes with odd l / 16 that of row 16 + l % 16, so the staging rows are written with
// 16-byte stores.
typedef float v4f_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f_t mfma_fp8_16x16x128(const v8i_t& a, const v8i_t& b, const v4f_t& c) {
    // cbsz = blgp = 0: both operands OCP fp8 e4m3; scale operands 0 select the unscaled MFMA.
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

constexpr int64_t FP8_MFMA16_MIN_K = 8192;

template <class C, bool EDGE>
__global__ __launch_bounds__(256, 1) void fp8_gemm16_persistent_kernel(Fp8GemmArgs p) {
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, TM = C::TM, WM = C::WM, WN = C::WN;
    constexpr int CPR = WN / 8;             // 16-byte chunks per staged row
    constexpr int ESTAGE = 32 * WN * 2;     // bytes staged per wave: 32 rows of its tile
    static_assert(CPR == 8 || CPR == 16, "staging swizzle");
    const int64_t M = p.M, N = p.N, K = p.K, lda = p.lda, ldb = p.ldb, ldc = p.ldc;
    __shared__ __attribute__((aligned(1024))) uint8_t sA0[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sA1[BM * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sB0[BN * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sB1[BN * BK];
    __shared__ __attribute__((aligned(1024))) uint8_t sE[4 * ESTAGE];

    // ---- this workgroup's tiles
    const uint32_t tiles_m = p.tiles_m, tiles_n = p.tiles_n;
    const uint32_t n_tiles = tiles_m * tiles_n;
    const uint32_t G = gridDim.x, bid = blockIdx.x;
    const uint32_t xcd = bid % GEMM_XCDS, local = bid / GEMM_XCDS;
    const uint32_t g_x = G / GEMM_XCDS + (xcd < G % GEMM_XCDS ? 1u : 0u);
    const uint32_t per = n_tiles / GEMM_XCDS, rem = n_tiles % GEMM_XCDS;
    const uint32_t first = xcd * per + min(xcd, rem), cnt = per + (xcd < rem ? 1u : 0u);
    const uint32_t my = local < cnt ? (cnt - local + g_x - 1) / g_x : 0u;
    const uint32_t nk = (uint32_t)((K + BK - 1) / BK);
    const uint32_t total = my * nk;
    if (total == 0) return;  // the same for every wave of the workgroup
    auto coords = [&](uint32_t i, uint32_t& tm, uint32_t& tn) __attribute__((always_inline)) {
        const uint32_t t = first + local + i * g_x;
        const uint32_t group = C::GROUP_M * tiles_n;
        const uint32_t first_m = (t / group) * C::GROUP_M;
        const uint32_t gsize = min(tiles_m - first_m, (uint32_t)C::GROUP_M);
        tm = first_m + (t % group) % gsize;
        tn = (t % group) / gsize;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: tile bases stay scalar
    const int wm = wave >> 1, wn = wave & 1;

    // ---- global -> LDS slab loads (lane mapping as in fp8_gemm_nt_kernel), two slabs ahead of the
    // compute side. LDS chunk swizzle for this fragment shape: logical chunk c of row r at c ^ f(r),
    // f(r) = r3 | r1 << 1 | r2 << 2 (rn = bit n of r); for row r = 8 (4 j + wave) + lane / 8
    const int lrow8 = lane >> 3;
    const int lchunk = (lane & 7) ^ ((wave & 1) | (((lane >> 4) & 1) << 1) | (((lane >> 5) & 1) << 2));
    const int r0 = 8 * wave + lrow8;
    const uint32_t offa0 = (uint32_t)(r0 * lda + lchunk * 16), offb0 = (uint32_t)(r0 * ldb + lchunk * 16);
    const uint32_t stepa = (uint32_t)(32 * lda), stepb = (uint32_t)(32 * ldb);
    // Slab k of the compute side issues slab k+2 of the stream (for the last two slabs of a tile,
    // slab k+2-nk of the next tile), as in fp8_gemm_nt_persistent_kernel; `parts` selects the A
    // loads (1), the B loads (2) or both.
    struct IssueTile {
        __amdgpu_buffer_rsrc_t ra, rb;
        int rows_a, rows_b;
        bool live;
    };
    auto issue_tile = [&](uint32_t i) __attribute__((always_inline)) {
        IssueTile t;
        uint32_t tm, tn;
        t.live = i < my;
        coords(t.live ? i : my - 1, tm, tn);
        const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
        t.ra = __builtin_amdgcn_make_buffer_rsrc((void*)(p.A + m0 * lda), (short)0, (int)GEMM_RANGE, 0x00020000);
        t.rb = __builtin_amdgcn_make_buffer_rsrc((void*)(p.B + n0 * ldb), (short)0, (int)GEMM_RANGE, 0x00020000);
        t.rows_a = EDGE ? (int)min((int64_t)BM, M - m0) - r0 : BM;
        t.rows_b = EDGE ? (int)min((int64_t)BN, N - n0) - r0 : BN;
        return t;
    };
    IssueTile cur_t = issue_tile(0), next_t = issue_tile(1);
    auto issue = [&](uint8_t* sa, uint8_t* sb, uint32_t ks, int parts = 3) __attribute__((always_inline)) {
        const bool nxt = ks >= nk;
        const __amdgpu_buffer_rsrc_t ra = nxt ? next_t.ra : cur_t.ra;
        const __amdgpu_buffer_rsrc_t rb = nxt ? next_t.rb : cur_t.rb;
        const bool live = nxt ? next_t.live : cur_t.live;
        const int64_t k0 = (int64_t)(nxt ? ks - nk : ks) * BK;
        const uint32_t va = live ? offa0 : GEMM_OOB, vb = live ? offb0 : GEMM_OOB;
        int la = C::BM, lb = C::BN;
        if constexpr (EDGE) {
            const bool k_ok = k0 + lchunk * 16 < K;
            la = k_ok ? (nxt ? next_t.rows_a : cur_t.rows_a) : 0;
            lb = k_ok ? (nxt ? next_t.rows_b : cur_t.rows_b) : 0;
        }
        if (parts & 1)
#pragma unroll
        for (int j = 0; j < C::LA; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(sa + wave * 1024 + j * 4096), 16,
                                                     !EDGE || 32 * j < la ? va : GEMM_OOB,
                                                     (int)(j * stepa + (uint32_t)k0), 0, 0);
        if (parts & 2)
#pragma unroll
        for (int j = 0; j < C::LB; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(sb + wave * 1024 + j * 4096), 16,
                                                     !EDGE || 32 * j < lb ? vb : GEMM_OOB,
                                                     (int)(j * stepb + (uint32_t)k0), 0, 0);
    };

    // ---- operands: fragment i of A is rows WM*wm + 16 i + lane % 16, K bytes 32 (lane / 16) .. + 32
    // (logical chunks oc, oc + 1 at positions chunk ^ f(row) = chunk ^ sw; the fragment's base row
    // is a multiple of 16, so f depends on lane % 16 only)
    const int orow = lane & 15;
    const int oc = 2 * (lane >> 4);
    const int sw = ((lane >> 3) & 1) | (((lane >> 1) & 1) << 1) | (((lane >> 2) & 1) << 2);  // f(lane % 16)
    const int pa0 = (oc ^ sw) * 16, pa1 = ((oc + 1) ^ sw) * 16;
    auto read_frag = [&](const uint8_t* s, int base_row) __attribute__((always_inline)) -> v8i_t {
        const int o = (base_row + orow) * BK;
        const v4u_t x0 = *(const v4u_t*)(s + (o + pa0));
        const v4u_t x1 = *(const v4u_t*)(s + (o + pa1));
        return __builtin_bit_cast(v8i_t, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    auto read_a = [&](const uint8_t* s, int i) __attribute__((always_inline)) { return read_frag(s, WM * wm + 16 * i); };
    auto read_b = [&](const uint8_t* s, int j) __attribute__((always_inline)) { return read_frag(s, WN * wn + 16 * j); };

    constexpr int FM = WM / 16, FN = WN / 16, HM = FM / 2;
    v4f_t acc[FM][FN];
    auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
    };
    zero_acc();
    v8i_t a[FM], b[FN];

    // ---- epilogue of compute tile i: scale, round once to bf16, stage 32 rows of the wave's tile
    // at a time (16-byte chunk c of row r at position c ^ (r % CPR)), store row chunks (as in
    // fp8_gemm_nt_persistent_kernel)
    uint8_t* stage = sE + wave * ESTAGE;
    auto epilogue = [&](uint32_t i_tile) __attribute__((always_inline)) {
        uint32_t tm, tn;
        coords(i_tile, tm, tn);
        const int64_t row0 = (int64_t)tm * BM + WM * wm, col0 = (int64_t)tn * BN + WN * wn;
        // the lane index passes through an empty asm so that the addresses below are computed
        // here, once per tile, instead of being hoisted out of the tile loop into registers
        int ln = lane;
        asm volatile("" : "+v"(ln));
        uint32_t ldc2 = (uint32_t)ldc * 2;  // row pitch of C in bytes (< GEMM_RANGE / BM on this path)
        asm volatile("" : "+s"(ldc2));
        const int rr = ln / CPR, rc = ln % CPR;  // read side: row rr + r * (64 / CPR), chunk rc
        // whole tiles: one buffer resource per tile, the lane's offset in voffset and the row
        // block's in soffset
        const __amdgpu_buffer_rsrc_t rcs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.C + row0 * ldc + col0), (short)0, (int)GEMM_RANGE, 0x00020000);
        const uint32_t vo = (uint32_t)rr * ldc2 + (uint32_t)rc * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i) {  // 32-row blocks: fragment rows 2i, 2i + 1
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                // lane l holds rows 16 f + l % 16 (f = 0, 1), columns 16 j + 4 (l / 16) + {0..3}; one
                // permlane16 swap per dword gives lanes with even l / 16 the whole 16-byte chunk of
                // row l % 16 and lanes with odd l / 16 the chunk of row 16 + l % 16
                v4f_t t0 = acc[2 * i][j], t1 = acc[2 * i + 1][j];
                asm volatile("" : "+v"(t0), "+v"(t1));
                const uint32_t w0x = pack_bf16x2(t0[0] * p.out_scale, t0[1] * p.out_scale);
                const uint32_t w0y = pack_bf16x2(t0[2] * p.out_scale, t0[3] * p.out_scale);
                const uint32_t w1x = pack_bf16x2(t1[0] * p.out_scale, t1[1] * p.out_scale);
                const uint32_t w1y = pack_bf16x2(t1[2] * p.out_scale, t1[3] * p.out_scale);
                const auto x = __builtin_amdgcn_permlane16_swap(w0x, w1x, false, false);
                const auto y = __builtin_amdgcn_permlane16_swap(w0y, w1y, false, false);
                const v4u_t chunk = {x[0], y[0], x[1], y[1]};
                const int q4 = ln >> 4, srow = 16 * (q4 & 1) + (ln & 15);
                const int c = 2 * j + (q4 >> 1);
                *(v4u_t*)(stage + (srow * (WN * 2) + ((c ^ (srow & (CPR - 1))) * 16))) = chunk;
            }
#pragma unroll
            for (int r = 0; r < 32 * CPR / 64; ++r) {
                const int row = rr + r * (64 / CPR);
                const v4u_t v = *(const v4u_t*)(stage + (row * (WN * 2) + ((rc ^ (row & (CPR - 1))) * 16)));
                const int grow = i * 32 + row;
                if constexpr (!EDGE) {
                    __builtin_amdgcn_raw_buffer_store_b128(v, rcs, vo,
                                                           (int)((uint32_t)(i * 32 + r * (64 / CPR)) * ldc2), 0);
                } else {
                    if (row0 + grow >= M) continue;
                    const int64_t n = col0 + rc * 8;
                    uint16_t* dst = p.C + (row0 + grow) * ldc + n;
                    if (p.vec_store && n + 8 <= N) {
                        *(v4u_t*)dst = v;
                    } else {
                        const uint16_t e8[8] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y,
                                                (uint16_t)(v.y >> 16), (uint16_t)v.z, (uint16_t)(v.z >> 16),
                                                (uint16_t)v.w, (uint16_t)(v.w >> 16)};
                        for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = e8[e];
                    }
                }
            }
        }
    };

    // ---- one slab of the stream (sa/sb hold slab k, na/nb slab k+1), two barriers. a[0..HM) and b[]
    // hold slab k's fragments, read during slab k-1. Fragment rows 0..HM-1 run column by column:
    // after column 0 (CB columns), barrier 1, once every wave's reads of slab k's B fragments
    // are complete, gives sb to slab k+2's B loads, spread over columns 1..FN-1 together with
    // the reads of a[HM..FM) from sa. After barrier 2 (mid-slab) sa takes slab k+2's A loads,
    // spread over rows HM..FM-1, and slab k+1's fragments are read into registers whose last use
    // has passed: a[0..HM) first, b[j] after column j. (With both halves' loads issued after
    // one barrier, sixteen loads fell into a quarter of the slab's 32-cycle MFMA gaps and
    // stalled the wave: 11% more cycles than without loads, against 2% this way.) The LAST slab
    // of a tile leaves slab k+1's fragment reads to after the epilogue.
    // Vector memory operations complete in issue order and vmcnt counts stores too: at barrier 2
    // the LB B loads just issued (and after an epilogue its EPI_STORES stores, an exact count:
    // whole-chunk stores, no EDGE instance) may stay in flight; everything before them (slab
    // k+1's loads) has landed.
    constexpr int EPI_STORES = TM * (32 * CPR / 64);
    constexpr int WAIT_LGKM0 = 15 | (3 << 14) | (7 << 4);  // lgkmcnt(0); vmcnt and expcnt not waited for
    constexpr int W2 = C::LB, W2E = C::LB + EPI_STORES;
    static_assert(W2E < 64, "vmcnt field");
    constexpr int WAIT2 = (W2 & 15) | ((W2 >> 4) << 14) | (7 << 4);
    constexpr int WAIT2E = (W2E & 15) | ((W2E >> 4) << 14) | (7 << 4);
    // A slab is split at barrier 1 into its head (column 0's MFMAs) and the rest, and the slab loop
    // runs from one barrier 1 to the next: at a loop header the compiler's wait bookkeeping no
    // longer knows which operand reads are in flight and waits for all of them, which barrier 1
    // does anyway (with the header before the head, that wait held back column 0's MFMAs: ~1.5%
    // more cycles at 8192^3).
    constexpr int CB = 1;  // columns before barrier 1
    auto head = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < CB; ++j)
#pragma unroll
            for (int i = 0; i < HM; ++i) acc[i][j] = mfma_fp8_16x16x128(b[j], a[i], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto slab = [&](uint8_t* sa, uint8_t* sb, uint8_t* na, uint8_t* nb, uint32_t k, auto last, auto epi)
                    __attribute__((always_inline)) {
        constexpr bool LAST = decltype(last)::value;
        constexpr bool EPI = decltype(epi)::value;
        constexpr bool AFTER_EPI = EPI && !EDGE;
        __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);
        asm volatile("s_barrier" ::: "memory");
        issue(sa, sb, k + 2, 2);
#pragma unroll
        for (int i = HM; i < FM; ++i) a[i] = read_a(sa, i);
#pragma unroll
        for (int j = CB; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < HM; ++i) acc[i][j] = mfma_fp8_16x16x128(b[j], a[i], acc[i][j]);
        constexpr int NA = HM * (FN - CB), PER = NA / C::LB;
        // columns 1..FN-1: HM * (FN - 1) MFMAs beside LB loads and 2 (FM - HM) operand reads
        static_assert(PER >= 2, "two MFMAs per load after barrier 1");
#pragma unroll
        for (int q = 0; q < C::LB; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (PER > 2) __builtin_amdgcn_sched_group_barrier(0x008, PER - 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NA - PER * C::LB, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (AFTER_EPI) __builtin_amdgcn_s_waitcnt(WAIT2E);
        else if constexpr (EPI) __builtin_amdgcn_s_waitcnt(0);
        else __builtin_amdgcn_s_waitcnt(WAIT2);
        asm volatile("s_barrier" ::: "memory");
        issue(sa, sb, k + 2, 1);
        if constexpr (!LAST) {
#pragma unroll
            for (int i = 0; i < HM; ++i) a[i] = read_a(na, i);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int i = HM; i < FM; ++i) acc[i][j] = mfma_fp8_16x16x128(b[j], a[i], acc[i][j]);
            if constexpr (!LAST) b[j] = read_b(nb, j);
        }
        // second half: (FM - HM) * FN MFMAs beside LA loads and (not LAST) 2 (HM + FN) reads
        if constexpr (!LAST) {
#pragma unroll
            for (int q = 0; q < C::LA; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        } else {
#pragma unroll
            for (int q = 0; q < C::LA; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            }
        }
    };
    using BF = std::integral_constant<bool, false>;
    using BT = std::integral_constant<bool, true>;

    issue(sA0, sB0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    issue(sA1, sB1, 1);
#pragma unroll
    for (int i = 0; i < HM; ++i) a[i] = read_a(sA0, i);
#pragma unroll
    for (int j = 0; j < FN; ++j) b[j] = read_b(sB0, j);
    // nk is even, so every tile starts in buffer 0. The first slab of each later tile follows its
    // predecessor's epilogue in straight-line code, so that the compiler's own wait bookkeeping
    // sees the stores in flight on one path only and adds no waits of its own to that slab.
    head();
    slab(sA0, sB0, sA1, sB1, 0, BF{}, BF{});
    head();
    for (uint32_t it = 0;;) {
        for (uint32_t k = 1; k + 2 < nk; k += 2) {
            slab(sA1, sB1, sA0, sB0, k, BF{}, BF{});
            head();
            slab(sA0, sB0, sA1, sB1, k + 1, BF{}, BF{});
            head();
        }
        slab(sA1, sB1, sA0, sB0, nk - 1, BT{}, BF{});
        __builtin_amdgcn_sched_barrier(0);
        epilogue(it);
        __builtin_amdgcn_sched_barrier(0);
        zero_acc();
        // the next slab's loads were covered by the last slab's wait
#pragma unroll
        for (int i = 0; i < HM; ++i) a[i] = read_a(sA0, i);
#pragma unroll
        for (int j = 0; j < FN; ++j) b[j] = read_b(sB0, j);
        if (++it == my) break;
        cur_t = next_t;
        next_t = issue_tile(it + 1);
        head();
        slab(sA0, sB0, sA1, sB1, 0, BF{}, BT{});
        head();
    }
    // the loads issued past the last slab write zeros into LDS: they land before the workgroup ends
    __builtin_amdgcn_s_waitcnt(0);
}

// Persistent launch: min(tiles, CUs) workgroups (n_cu from the caller), the 16x16x128 form for
// K >= FP8_MFMA16_MIN_K. An odd or zero slab count (K / BK rounded up) takes the non-persistent
// kernel (which writes C = 0 for K = 0), and so does a device with fewer CUs than XCDs: the tile
// list gives every XCD with tiles at least one workgroup only when the grid has
// min(tiles, GEMM_XCDS) or more.
template <class C>
inline int fp8_gemm_persistent_launch(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K,
                                      int64_t lda, int64_t ldb, float out_scale, uint16_t* Cm, int64_t ldc,
                                      int n_cu, hipStream_t s) {
    Fp8GemmArgs p{A, B, Cm, M, N, K, lda, ldb, ldc, out_scale, (uint32_t)((M + C::BM - 1) / C::BM),
                  (uint32_t)((N + C::BN - 1) / C::BN), (uint32_t)(ldc % 8 == 0 && ((uintptr_t)Cm & 15) == 0)};
    const uint64_t tiles = (uint64_t)p.tiles_m * p.tiles_n;
    if (tiles == 0) return 0;
    const uint32_t grid = (uint32_t)(tiles < (uint64_t)n_cu ? tiles : (uint64_t)n_cu);
    const int64_t nk = (K + C::BK - 1) / C::BK;
    if (nk == 0 || nk % 2 || n_cu < GEMM_XCDS)
        return fp8_gemm_launch<C>(A, B, M, N, K, lda, ldb, out_scale, Cm, ldc, s);
    // whole tiles with aligned C store through a buffer resource: a tile's offsets must stay in range
    const bool whole =
        M % C::BM == 0 && N % C::BN == 0 && K % C::BK == 0 && p.vec_store && (int64_t)C::BM * ldc * 2 < GEMM_RANGE;
    if (K >= FP8_MFMA16_MIN_K) {
        if (whole)
            hipLaunchKernelGGL((fp8_gemm16_persistent_kernel<C, false>), dim3(grid), dim3(C::THREADS), 0, s, p);
        else
            hipLaunchKernelGGL((fp8_gemm16_persistent_kernel<C, true>), dim3(grid), dim3(C::THREADS), 0, s, p);
    } else if (whole) {
        hipLaunchKernelGGL((fp8_gemm_nt_persistent_kernel<C, false>), dim3(grid), dim3(C::THREADS), 0, s, p);
    } else {
        hipLaunchKernelGGL((fp8_gemm_nt_persistent_kernel<C, true>), dim3(grid), dim3(C::THREADS), 0, s, p);
    }
    return 0;
}

}  // namespace dopt
