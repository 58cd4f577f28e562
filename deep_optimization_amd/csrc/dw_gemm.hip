// Weight gradient of a Linear layer from its saved activation, on CDNA4 bf16 MFMA:
//   dW[m][n] = sum_k dy[k][m] * x_hat[k][n]      (M = out features, N = in features, K = tokens)
//   db[m]    = sum_k dy[k][m]                     (optional, fused)
// with x_hat either a bf16 tensor or decoded inside the kernel from the quantizer's packed codes
// (x_hat = bf16(fma(q, scale, min)), the value act_lib::dequant_unpack_triton writes), so the
// dequantized activation never goes through HBM.
//
// Both operands arrive K-outer ([K][M] and [K][N], row-major), which MFMA cannot read directly:
// a lane's MFMA operand is 8 consecutive K values of one row/column. Each K tile (64 tokens) is
// therefore staged through registers: a lane loads an 8 x 8 block (8 token rows x 16 bytes),
// transposes it with byte permutes (v_perm_b32) and writes 8 K-contiguous 16-byte chunks to LDS
// ([m][k] and [n][k], 128-byte rows, chunk c of row r at position c ^ ((r / 2) % 8) so a
// ds_read_b128 of 16 consecutive rows hits 16 distinct bank groups). For packed x the lane reads
// the 8 rows' codes (8 * bits bits per row) and their group's bf16 scale and min, and decodes
// straight into the transposed chunks.
//
// Tiling: 256 x 256 output tile per workgroup of 4 waves (2 x 2), each wave 128 x 128 as 4 x 4
// blocks of v_mfma_f32_32x32x16_bf16 (fp32 accumulators). The K range is split S ways so the
// small M x N of a weight gradient still fills the GPU; each split writes an fp32 partial tile
// and a second kernel sums the S partials in order (deterministic) into fp32 and/or bf16. K
// tiles are double-buffered: the global loads of tile k+1 are issued before the MFMAs of tile k,
// and their transpose/decode into the other LDS buffer follows them.
//
// MFMA layout (32x32x16 bf16): lane l supplies row (or column) l % 32 and 8 consecutive K values
// starting at 8 * (l / 32) of the 16; A and B use the same K mapping. Accumulator register v of
// lane l holds row 8*(v/4) + 4*(l/32) + (v%4), column l % 32.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "dopt_device.h"
#include "dw_gemm.h"

namespace dopt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 64, THREADS = 256;
constexpr int DW_XCDS = 8;
constexpr int TM = 4, TN = 4;          // 32 x 32 blocks per wave
constexpr int ROWB = BK * 2;           // LDS row pitch in bytes (64 bf16)

__device__ __forceinline__ f32x16_t mfma_bf16(const uint4& a, const uint4& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// byte offset of 16-byte chunk `ch` of LDS row `r`
__device__ __forceinline__ int lds_off(int r, int ch) { return r * ROWB + ((ch ^ ((r >> 1) & 7)) << 4); }

// one K tile's worth of a lane's producer inputs (registers between the global load and the LDS write)
struct Stage {
    uint4 a[8];      // dy rows k..k+7, 8 m values each
    uint4 b[8];      // x_hat rows (bf16 mode)
    uint32_t w[8];   // codes of 8 x 8 (packed mode; bits == 8 uses w and w2)
    uint32_t w2[8];
    uint32_t sm[8];  // bf16 scale (low) | min (high) per row (packed mode)
};

template <int MODE, int BITS>
__device__ __forceinline__ void load_stage(const DwArgs& a, Stage& s, int64_t k0, int kb, int mb, int64_t m0,
                                           int64_t n0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int64_t k = k0 + kb * 8 + j;
        const bool in = k < a.K;
        s.a[j] = in ? *(const uint4*)(a.dy + k * a.ldd + m0 + mb * 8) : make_uint4(0, 0, 0, 0);
        if constexpr (MODE == DW_B_BF16) {
            s.b[j] = in ? *(const uint4*)(a.xh + k * a.ldx + n0 + mb * 8) : make_uint4(0, 0, 0, 0);
        } else {
            // element e = k * N + n of the flat activation: codes at bit e * bits, group e >> lg
            // (e % 8 == 0, so the 8 codes of bits <= 4 lie in one word; bits == 8 takes two)
            const int64_t e = k * a.N + n0 + mb * 8;
            const int64_t bit = e * BITS;
            if (in) {
                const uint32_t* wp = a.packed + (bit >> 5);
                s.w[j] = BITS == 8 ? wp[0] : (wp[0] >> (bit & 31));
                s.w2[j] = BITS == 8 ? wp[1] : 0u;
                const int64_t gi = e >> a.lg;
                s.sm[j] = (uint32_t)a.scale[gi] | ((uint32_t)a.minv[gi] << 16);
            } else {
                s.w[j] = s.w2[j] = 0u;
                s.sm[j] = 0u;  // scale 0, min 0: rows past K decode to 0
            }
        }
    }
}

// Part p (0..3) of writing a staged K tile to LDS: columns 2p and 2p+1 of the lane's 8 x 8 A block
// (transposed) and of its B block (transposed or decoded); with DB also dy rows 2p, 2p+1 into db[].
template <int MODE, int BITS, bool DB>
__device__ __forceinline__ void write_part(const DwArgs& a, const Stage& s, char* sa, char* sb, int kb, int mb,
                                           float* db, int p) {
    if constexpr (DB) {
        // column sums of dy rows 2p, 2p+1 (dword q of a row holds columns 2q, 2q+1); fenced so the
        // scheduler does not widen every row early (register pressure)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 2 * p; j < 2 * p + 2; ++j) {
            const uint32_t* d = (const uint32_t*)&s.a[j];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                db[2 * q] += __uint_as_float(d[q] << 16);
                db[2 * q + 1] += __uint_as_float(d[q] & 0xffff0000u);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int c = 2 * p; c < 2 * p + 2; ++c) {
        const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
        uint32_t d[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t* lo = (const uint32_t*)&s.a[2 * r];
            const uint32_t* hi = (const uint32_t*)&s.a[2 * r + 1];
            d[r] = __builtin_amdgcn_perm(hi[c >> 1], lo[c >> 1], sel);
        }
        *(uint4*)(sa + lds_off(mb * 8 + c, kb)) = make_uint4(d[0], d[1], d[2], d[3]);
        if constexpr (MODE == DW_B_BF16) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t* lo = (const uint32_t*)&s.b[2 * r];
                const uint32_t* hi = (const uint32_t*)&s.b[2 * r + 1];
                d[r] = __builtin_amdgcn_perm(hi[c >> 1], lo[c >> 1], sel);
            }
            *(uint4*)(sb + lds_off(mb * 8 + c, kb)) = make_uint4(d[0], d[1], d[2], d[3]);
        } else {
            // value (row j, column c) = bf16(fma(q, scale_j, min_j)), rows 2r, 2r+1 in dword r
            constexpr uint32_t qm = (1u << BITS) - 1u;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t q = BITS == 8 ? (((c < 4 ? s.w[j] : s.w2[j]) >> (8 * (c & 3))) & 0xffu)
                                             : ((s.w[j] >> (c * BITS)) & qm);
                v[j] = fmaf((float)q, __uint_as_float(s.sm[j] << 16), __uint_as_float(s.sm[j] & 0xffff0000u));
            }
            *(uint4*)(sb + lds_off(mb * 8 + c, kb)) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                               pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
        }
    }
}

template <int MODE, int BITS, bool DB>
__device__ __forceinline__ void write_stage(const DwArgs& a, const Stage& s, char* sa, char* sb, int kb, int mb,
                                            float* db) {
#pragma unroll
    for (int p = 0; p < 4; ++p) write_part<MODE, BITS, DB>(a, s, sa, sb, kb, mb, db, p);
}

// The MFMAs of one K tile (4 steps of 16 K) from LDS buffers (ra, rb).
__device__ __forceinline__ void mma_tile(f32x16_t (&acc)[TM][TN], const char* ra, const char* rb, int wm, int wn,
                                         int lane) {
    const int orow = lane & 31, och = lane >> 5;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
        uint4 fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[i] = *(const uint4*)(ra + lds_off(wm * 128 + i * 32 + orow, 2 * kk + och));
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = *(const uint4*)(rb + lds_off(wn * 128 + j * 32 + orow, 2 * kk + och));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma_bf16(fa[i], fb[j], acc[i][j]);
    }
}

// K tiles kt0..kt1-1 of one split: the global loads of tile k+1 go out before the MFMAs of tile k
// (LDS buffer k % 2); after them the staged tile is transposed / decoded into buffer (k+1) % 2.
template <int MODE, int BITS, bool DB>
__global__ __launch_bounds__(THREADS, 1) void dw_gemm_kernel(DwArgs a) {
    __shared__ __attribute__((aligned(1024))) char sA[2][BM * ROWB];
    __shared__ __attribute__((aligned(1024))) char sB[2][BN * ROWB];

    // workgroup ids go to the 8 XCDs round-robin (id % 8). Work items are numbered
    // L = (split * tiles_m + tm) * tiles_n + tn and each XCD takes a contiguous range of L, so the
    // workgroups of one XCD share dy tiles (same split, tm) and x tiles (same split, tn) in its L2.
    const int tiles_n = (int)(a.N / BN), tiles = (int)(a.M / BM) * tiles_n;
    const int W = tiles * a.splits, per = (W + DW_XCDS - 1) / DW_XCDS;
    const int xcd = blockIdx.x % DW_XCDS, local = blockIdx.x / DW_XCDS;
    if (local >= per) return;
    const int L = xcd * per + local;
    if (L >= W) return;
    const int split = L / tiles, t = L % tiles;
    const int tm = t / tiles_n, tn = t % tiles_n;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t kt0 = (int64_t)split * a.kt_per_split;
    const int64_t kt1 = min(kt0 + a.kt_per_split, (a.K + BK - 1) / BK);
    // every workgroup of a DB launch sums its dy tile (a runtime tn == 0 test doubles the
    // kernel's live registers); the tn == 0 ones store the sums
    constexpr bool with_db = DB;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int kb = wave * 2 + (lane >> 5), mb = lane & 31;  // this lane's 8 x 8 producer block

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    float db[8] = {};

    Stage st;
    const int64_t nk = kt1 - kt0;
    if (nk > 0) {
        load_stage<MODE, BITS>(a, st, kt0 * BK, kb, mb, m0, n0);
        write_stage<MODE, BITS, with_db>(a, st, sA[0], sB[0], kb, mb, db);
    }
    __syncthreads();
    int cur = 0;
    for (int64_t k = kt0; k < kt1; ++k) {
        const bool more = k + 1 < kt1;
        if (more) load_stage<MODE, BITS>(a, st, (k + 1) * BK, kb, mb, m0, n0);
        mma_tile(acc, sA[cur], sB[cur], wm, wn, lane);
        if (more) write_stage<MODE, BITS, with_db>(a, st, sA[cur ^ 1], sB[cur ^ 1], kb, mb, db);
        __syncthreads();
        cur ^= 1;
    }

    // fp32 partial tile of this split
    float* P = a.partial + (int64_t)split * a.M * a.N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t col = n0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                P[row * a.N + col] = acc[i][j][v];
            }
        }
    if (with_db && tn == 0) {
        // per-lane sums of its 8 m columns over its k rows -> fixed-order sum over the 8 k blocks
        float* red = (float*)sA[0];
#pragma unroll
        for (int c = 0; c < 8; ++c) red[kb * BM + mb * 8 + c] = db[c];
        __syncthreads();
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) sum += red[q * BM + tid];
        a.db_partial[(int64_t)split * a.M + m0 + tid] = sum;
    }
}

// ------------------------------------------------------------------ v2: bf16 operands, no transposes
// Tiles go HBM -> LDS with global_load_lds (no registers, no VALU) in their natural [k][m] /
// [k][n] layout, through a ring of V2_STAGES stages of V2_BK tokens, V2_STAGES - 1 tiles ahead.
// The MFMA operands are read with ds_read_b64_tr_b16, whose 16-lane groups transpose a 4 x 16
// block: lane 4p+q of a group receives element q of the 8-byte reads of lanes p, p+4, p+8, p+12.
// Source lane 4u+v of group g reads row (k0 + 8*(g/2) + 4h + u), 4 columns at 16*(g%2) + 4v of the
// fragment, so MFMA lane l receives column l % 32 at 4 consecutive k; reads h = 0, 1 give its 8.
// LDS rows are 512 bytes (256 bf16); 16-byte chunk c of row r sits at position c ^ (4 * (r % 4)),
// which puts the 4 rows of a transposing read on 4 distinct 64-byte bank groups.
constexpr int V2_BK = 32;
constexpr int V2_ROWB = 512;                    // bytes per LDS row (256 bf16)
constexpr int V2_TILE = V2_BK * V2_ROWB;        // bytes of one operand tile (16 KB)

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;

__device__ __forceinline__ int v2_pos(int r, int c) { return (c ^ ((r & 3) << 2)) << 4; }

// s_waitcnt vmcnt(n) (expcnt / lgkmcnt left at their maxima: no wait on them)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 8 bf16 of one MFMA operand: column `col` of the stage tile (lane's column within the 32-wide
// fragment applied by the transpose), rows kk*16 + 8*(g/2) + {0..7}
template <int RB>  // LDS row pitch in bytes (512: 256-column tiles, 256: 128-column tiles)
__device__ __forceinline__ uint4 v2_frag(const char* tile, int kk, int col0, int lane) {
    const int g = lane >> 4, t = lane & 15, u = t >> 2, v = t & 3;
    const int colw = col0 + 16 * (g & 1) + 4 * v;  // first of the 4 columns this lane reads
    uint4 out;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r = kk * 16 + 8 * (g >> 1) + 4 * h + u;
        const char* p = tile + r * RB + v2_pos(r, colw >> 3) + ((colw & 4) << 1);
        const v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p);
        const uint32_t lo = (uint32_t)(uint16_t)x[0] | ((uint32_t)(uint16_t)x[1] << 16);
        const uint32_t hi = (uint32_t)(uint16_t)x[2] | ((uint32_t)(uint16_t)x[3] << 16);
        if (h == 0) {
            out.x = lo;
            out.y = hi;
        } else {
            out.z = lo;
            out.w = hi;
        }
    }
    return out;
}

// s_waitcnt vmcnt(n) lgkmcnt(0): this wave's loads older than the n most recent have landed and
// its LDS reads have returned
template <int N>
__device__ __forceinline__ void wait_vm_lds() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// workgroup barrier without the memory fence of __syncthreads (whose release would wait for every
// in-flight global -> LDS load); the asm's memory clobber keeps the compiler from moving memory
// operations across it, the waits before it are explicit
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// Pipeline, per 32-token slab i (stage i % 4: one LDS object for its A tile, one for its B tile):
//   operand reads of slab i, second 16 tokens | MFMAs of slab i, first 16 tokens (read one step
//   earlier) | wait: own loads of slab i+1 landed, own LDS reads returned | barrier |
//   issue loads of slab i+4 into stage i % 4 | operand reads of slab i+1, first 16 tokens |
//   MFMAs of slab i, second 16 tokens
// Three slabs stay in flight behind the one being multiplied; every step issues exactly one slab
// (indices past the split's last slab reload the last one, which nobody reads), so the wait count
// is the same in every step. Each stage's A and B tiles are separate LDS objects, so the compiler
// can tell which in-flight load an operand read depends on and waits for that one only.
//
// BITS = 0: x_hat is bf16 and its tiles arrive by DMA like dy's. BITS = 1, 2, 4: x_hat is the
// quantizer's packed codes. A slab's codes (32 rows x 256 columns x BITS bits) and, per decoding
// thread, the dwords holding its group's bf16 scale and min arrive by DMA into a ring of 4 code
// slots with the slab's dy. Each step's wait covers the loads issued two steps before, and in the
// step before a slab is multiplied every thread decodes its 32 values of it, bf16(fma(q, scale,
// min)) as dequant_unpack writes them, into the slab's B stage, beside that step's MFMAs; the
// step's barrier publishes the stage.
// Thread t decodes row t / 8, columns 32 (t % 8) .. +31: 32 consecutive elements of the flat
// activation, inside one group (g >= 64), whose codes are BITS consecutive words.
template <int BITS>
struct V2Codes {
    static constexpr int NC = BITS == 2 ? 2 : 1;             // code DMAs per thread per slab
    static constexpr int CODE_BYTES = BITS ? 1024 * BITS : 0;  // codes of one slab
    static constexpr int SLOT = BITS ? CODE_BYTES + 2048 : 16;  // + scale and min dwords (4 B per thread each)
};

// NW waves per workgroup: 4 (2 x 2, 128 x 128 per wave: 256 accumulators, one wave per SIMD) or,
// for bf16 x_hat, 8 (2 x 4, 128 x 64 per wave: 128 accumulators, two waves per SIMD, so one
// wave's MFMAs run while the other waits at the slab barrier or on its operand reads). The
// workgroup tile, the DMA ring and the order of the MFMA steps are the same either way.
// BMT: output rows per workgroup tile, 256 or (for small outputs, so fewer K splits fill the GPU
// and fewer split partials go through HBM) 128; the waves then cover 64 rows each.
template <int BITS, bool DB, int NW, int BMT>
__global__ __launch_bounds__(64 * NW, 1) void dw_gemm_v2_kernel(DwArgs a) {
    static_assert(BITS == 0 || BITS == 1 || BITS == 2 || BITS == 4, "bf16, or 1/2/4-bit codes");
    static_assert(NW == 4 || (NW == 8 && BITS == 0), "8 waves for bf16 x_hat only");
    using CS = V2Codes<BITS>;
    constexpr int WN = NW / 2;            // waves along n
    constexpr int CW = BN / WN;           // columns per wave
    constexpr int TNW = CW / 32;          // 32 x 32 blocks per wave along n
    constexpr int JJ = 16 / NW;           // 1 KB DMA blocks per wave per x_hat tile
    static_assert(BMT == 256 || BMT == 128, "tile rows");
    constexpr int RA = BMT * 2;           // bytes per LDS row of a dy tile
    constexpr int TILE_A = V2_BK * RA;    // bytes of one dy tile
    constexpr int JA = TILE_A / 1024 / NW;  // 1 KB DMA blocks per wave per dy tile
    constexpr int RPB = 1024 / RA;        // dy rows per 1 KB block
    constexpr int LPR = RA / 16;          // lanes per dy row
    constexpr int RW = BMT / 2;           // rows per wave (2 waves along m)
    constexpr int TMW = RW / 32;          // 32 x 32 blocks per wave along m
    constexpr int LD = BITS == 0 ? JA + JJ : JA + CS::NC + 2;  // DMAs per wave per slab
    __shared__ __attribute__((aligned(1024))) char sa0[TILE_A];
    __shared__ __attribute__((aligned(1024))) char sa1[TILE_A];
    __shared__ __attribute__((aligned(1024))) char sa2[TILE_A];
    __shared__ __attribute__((aligned(1024))) char sa3[TILE_A];
    __shared__ __attribute__((aligned(1024))) char sb0[V2_TILE];
    __shared__ __attribute__((aligned(1024))) char sb1[V2_TILE];
    __shared__ __attribute__((aligned(1024))) char sb2[V2_TILE];
    __shared__ __attribute__((aligned(1024))) char sb3[V2_TILE];
    __shared__ __attribute__((aligned(1024))) char sc0[CS::SLOT];
    __shared__ __attribute__((aligned(1024))) char sc1[CS::SLOT];
    __shared__ __attribute__((aligned(1024))) char sc2[CS::SLOT];
    __shared__ __attribute__((aligned(1024))) char sc3[CS::SLOT];

    const int tiles_n = (int)(a.N / BN), tiles = (int)(a.M / BMT) * tiles_n;
    const int W = tiles * a.splits, per = (W + DW_XCDS - 1) / DW_XCDS;
    const int xcd = blockIdx.x % DW_XCDS, local = blockIdx.x / DW_XCDS;
    if (local >= per) return;
    const int L = xcd * per + local;
    if (L >= W) return;
    const int split = L / tiles, t = L % tiles;
    const int tm = t / tiles_n, tn = t % tiles_n;
    const int64_t m0 = (int64_t)tm * BMT, n0 = (int64_t)tn * BN;
    const int64_t kt0 = (int64_t)split * a.kt_per_split;
    const int64_t kt1 = min(kt0 + a.kt_per_split, a.K / V2_BK);
    const int nk = (int)(kt1 - kt0);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // global -> LDS: instruction j of wave w fills 1 KB block b = NW j + w of a tile = rows 2b, 2b+1;
    // lane l -> row 2b + l/32, position l % 32 <- global chunk (l % 32) ^ (4 * (row % 4)).
    // The global address is a wave-uniform slab base plus a loop-invariant 32-bit lane offset.
    // The LDS offsets carry `opaque0`, a zero the compiler cannot see through: its wait insertion
    // checks an operand read against one recorded load per LDS object, and a read it can prove
    // disjoint from that load's bytes would otherwise wait for every load in flight.
    int opaque0;
    asm volatile("s_mov_b32 %0, 0" : "=s"(opaque0));
    // (a dy tile of 128 columns has 256-byte rows: 4 rows per block, 16 lanes per row)
    uint32_t offa[JA], offb[JJ];
#pragma unroll
    for (int j = 0; j < JA; ++j) {
        const int r = RPB * (NW * j + wave) + lane / LPR, c = (lane % LPR) ^ ((r & 3) << 2);
        offa[j] = (uint32_t)(r * a.ldd + c * 8) * 2u;
    }
#pragma unroll
    for (int j = 0; j < JJ; ++j) {
        const int r = 2 * (NW * j + wave) + (lane >> 5), c = (lane & 31) ^ ((r & 3) << 2);
        offb[j] = (uint32_t)(r * a.ldx + c * 8) * 2u;
    }
    // packed x_hat: this thread's decode row and column run, and its flat element offset in a slab
    const int br = tid >> 3, bj = tid & 7;
    const int64_t e_lane = (int64_t)br * a.N + 32 * bj;
    const uint32_t offc = (uint32_t)((e_lane >> 5) * BITS * 4);  // byte offset of its code words
    auto issue = [&](char* sa, char* sb, char* sc, int64_t kt) {
        kt = min(kt, kt1 - 1);
        const char* ga = (const char*)(a.dy + kt * V2_BK * a.ldd + m0);
        char* da = sa + opaque0;
#pragma unroll
        for (int j = 0; j < JA; ++j)
            __builtin_amdgcn_global_load_lds((gbl_void_t*)(ga + offa[j]), (lds_void_t*)(da + (NW * j + wave) * 1024),
                                             16, 0, 0);
        if constexpr (BITS == 0) {
            const char* gb = (const char*)(a.xh + kt * V2_BK * a.ldx + n0);
            char* db = sb + opaque0;
#pragma unroll
            for (int j = 0; j < JJ; ++j)
                __builtin_amdgcn_global_load_lds((gbl_void_t*)(gb + offb[j]), (lds_void_t*)(db + (NW * j + wave) * 1024),
                                                 16, 0, 0);
        } else {
            const int64_t e0 = kt * V2_BK * a.N + n0;  // a multiple of 256
            const char* gc = (const char*)a.packed + (e0 >> 5) * BITS * 4;
            char* dc = sc + opaque0;
            if constexpr (BITS == 4) {
                __builtin_amdgcn_global_load_lds((gbl_void_t*)(gc + offc), (lds_void_t*)(dc + wave * 1024), 16, 0, 0);
            } else {
#pragma unroll
                for (int d = 0; d < CS::NC; ++d)
                    __builtin_amdgcn_global_load_lds((gbl_void_t*)(gc + offc + 4 * d),
                                                     (lds_void_t*)(dc + d * 1024 + wave * 256), 4, 0, 0);
            }
            // the dwords holding this thread's group's bf16 scale and min
            const int64_t gi = (e0 + e_lane) >> a.lg;
            __builtin_amdgcn_global_load_lds((gbl_void_t*)((const char*)a.scale + (gi >> 1) * 4),
                                             (lds_void_t*)(dc + CS::CODE_BYTES + wave * 256), 4, 0, 0);
            __builtin_amdgcn_global_load_lds((gbl_void_t*)((const char*)a.minv + (gi >> 1) * 4),
                                             (lds_void_t*)(dc + CS::CODE_BYTES + 1024 + wave * 256), 4, 0, 0);
        }
    };
    // packed x_hat: slab kt's codes, scale and min from slot sc (LDS reads), then chunk c (8
    // values, one 16-byte LDS chunk) decoded into its B stage sb
    struct DecodeIn {
        uint32_t w[BITS ? BITS : 1];
        float scl, mnv;
    };
    auto decode_load = [&](const char* sc, int64_t kt) {
        DecodeIn d{};
        if constexpr (BITS != 0) {
            kt = min(kt, kt1 - 1);
            const int hi = (int)(((kt * V2_BK * a.N + n0 + e_lane) >> a.lg) & 1);
            const uint32_t sw = *(const uint32_t*)(sc + CS::CODE_BYTES + tid * 4);
            const uint32_t mw = *(const uint32_t*)(sc + CS::CODE_BYTES + 1024 + tid * 4);
            d.scl = __uint_as_float(hi ? (sw & 0xffff0000u) : (sw << 16));
            d.mnv = __uint_as_float(hi ? (mw & 0xffff0000u) : (mw << 16));
            if constexpr (BITS == 4) {
                const uint4 x = *(const uint4*)(sc + tid * 16);
                d.w[0] = x.x;
                d.w[1] = x.y;
                d.w[2] = x.z;
                d.w[3] = x.w;
            } else {
#pragma unroll
                for (int q = 0; q < BITS; ++q) d.w[q] = *(const uint32_t*)(sc + q * 1024 + tid * 4);
            }
        }
        return d;
    };
    auto decode_chunk = [&](const DecodeIn& d, char* sb, int c) {
        if constexpr (BITS != 0) {
            constexpr uint32_t qm = (1u << BITS) - 1u;
            uint32_t o[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int e = 8 * c + 2 * h;
                const uint32_t q0 = (d.w[(e * BITS) >> 5] >> ((e * BITS) & 31)) & qm;
                const uint32_t q1 = (d.w[((e + 1) * BITS) >> 5] >> (((e + 1) * BITS) & 31)) & qm;
                o[h] = pack_bf16x2(fmaf((float)q0, d.scl, d.mnv), fmaf((float)q1, d.scl, d.mnv));
            }
            *(uint4*)(sb + br * V2_ROWB + v2_pos(br, 4 * bj + c)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    };

    f32x16_t acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    // bias gradient from the dy fragments already in registers: lane l of fragment ii holds
    // column (l % 32) at 8 consecutive tokens as 4 bf16 pairs, and one v_dot2 with (1, 1) adds a
    // pair. Only the waves with wn == 0 of the workgroups with tn == 0 (one per dy tile) sum.
    float dbacc[TMW] = {};
    const bool db_wave = DB && tn == 0 && wn == 0;

    uint4 fa0[TMW], fb0[TNW], fa1[TMW], fb1[TNW];
    auto read_frags = [&](const char* sa, const char* sb, int kk, uint4* fa, uint4* fb) {
#pragma unroll
        for (int ii = 0; ii < TMW; ++ii) fa[ii] = v2_frag<RA>(sa, kk, wm * RW + ii * 32, lane);
#pragma unroll
        for (int jj = 0; jj < TNW; ++jj) fb[jj] = v2_frag<V2_ROWB>(sb, kk, wn * CW + jj * 32, lane);
    };
    // bias-gradient pairs of fragment row ii
    auto db_row = [&](const uint4* fa, int ii) {
        if (db_wave) {
            const bf16x2_t one = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
            const uint32_t w[4] = {fa[ii].x, fa[ii].y, fa[ii].z, fa[ii].w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dbacc[ii] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[q]), one, dbacc[ii], false);
        }
    };
    // the MFMAs of fragment row ii
    auto mma_row = [&](const uint4* fa, const uint4* fb, int ii) {
#pragma unroll
        for (int jj = 0; jj < TNW; ++jj) acc[ii][jj] = mfma_bf16(fa[ii], fb[jj], acc[ii][jj]);
    };
    auto mma = [&](const uint4* fa, const uint4* fb) {
#pragma unroll
        for (int ii = 0; ii < TMW; ++ii) mma_row(fa, fb, ii);
#pragma unroll
        for (int ii = 0; ii < TMW; ++ii) db_row(fa, ii);
    };
    constexpr int NM = TMW * TNW;          // MFMAs per 16 tokens
    constexpr int NR = 2 * (TMW + TNW);    // transposing reads per 16 tokens
    // step i: slab i in stage (ca, cb), its code slot cc; slab i+1 in (na, nb), its codes in slot
    // nc (packed x_hat: decoded into nb here, before the barrier that publishes it)
    auto step = [&](char* ca, char* cb, char* cc, char* na, char* nb, const char* nc, int i) {
        if constexpr (BITS == 0) {
            // the transposing reads of the slab's second half go out two per MFMA over the first
            // half of the MFMAs, so they have returned by the wait before the barrier (one per
            // MFMA left the last read's latency exposed there)
            read_frags(ca, cb, 1, fa1, fb1);
            mma(fa0, fb0);
#pragma unroll
            for (int q = 0; q < NR / 2; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two LDS reads
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NM - NR / 2, 0);  // the other MFMAs
        } else {
            // codes first (their wait then leaves the operand reads in flight), and the decode
            // of slab i+1 in four pieces between the MFMA rows, fenced so that the VALU work runs
            // beside the matrix pipe instead of before it
            const DecodeIn din = decode_load(nc, kt0 + i + 1);
            read_frags(ca, cb, 1, fa1, fb1);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (c < TMW) mma_row(fa0, fb0, c);
                __builtin_amdgcn_sched_barrier(0);
                decode_chunk(din, nb, c);
                if (c < TMW) db_row(fa0, c);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (BITS == 0)
            wait_vm_lds<2 * LD>();  // slab i+1 landed (slabs i+2, i+3 may stay in flight)
        else
            wait_vm_lds<LD>();  // slab i+2 landed (slab i+3 may stay in flight)
        barrier_only();
        issue(ca, cb, cc, kt0 + i + 4);
        read_frags(na, nb, 0, fa0, fb0);
        mma(fa1, fb1);
#pragma unroll
        for (int q = 0; q < NM; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            if (q < LD) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
        }
    };

    if (nk > 0) {
        issue(sa0, sb0, sc0, kt0);
        issue(sa1, sb1, sc1, kt0 + 1);
        issue(sa2, sb2, sc2, kt0 + 2);
        issue(sa3, sb3, sc3, kt0 + 3);
        if constexpr (BITS == 0) {
            wait_vm_lds<3 * LD>();
        } else {
            // slab 0 is decoded here, slab i+1 in step i (its loads landed by step i-1's wait)
            wait_vm_lds<2 * LD>();
            const DecodeIn din = decode_load(sc0, kt0);
#pragma unroll
            for (int c = 0; c < 4; ++c) decode_chunk(din, sb0, c);
            wait_vm_lds<2 * LD>();
        }
        barrier_only();
        read_frags(sa0, sb0, 0, fa0, fb0);
        int i = 0;
        for (; i + 4 <= nk; i += 4) {
            step(sa0, sb0, sc0, sa1, sb1, sc1, i);
            step(sa1, sb1, sc1, sa2, sb2, sc2, i + 1);
            step(sa2, sb2, sc2, sa3, sb3, sc3, i + 2);
            step(sa3, sb3, sc3, sa0, sb0, sc0, i + 3);
        }
        if (i < nk) step(sa0, sb0, sc0, sa1, sb1, sc1, i);
        if (i + 1 < nk) step(sa1, sb1, sc1, sa2, sb2, sc2, i + 1);
        if (i + 2 < nk) step(sa2, sb2, sc2, sa3, sb3, sc3, i + 2);
    }
    // the trailing (unused) loads land before the kernel ends
    __builtin_amdgcn_s_waitcnt(0);

    float* P = a.partial + (int64_t)split * a.M * a.N;
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
            const int64_t col = n0 + wn * CW + j * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = m0 + wm * RW + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                P[row * a.N + col] = acc[i][j][v];
            }
        }
    if (db_wave) {
        // lanes l and l + 32 hold the two token halves of column l % 32
#pragma unroll
        for (int ii = 0; ii < TMW; ++ii) {
            const float other = __shfl_xor(dbacc[ii], 32);
            if (lane < 32) a.db_partial[(int64_t)split * a.M + m0 + wm * RW + ii * 32 + lane] = dbacc[ii] + other;
        }
    }
}

// out[m][n] = sum of the split partials; fp32 and/or bf16; db likewise. SUB consecutive lanes
// share one 4-wide output: lane j sums splits [j*per, (j+1)*per) in order, 4 loads in flight,
// and the SUB partial sums are combined by an xor butterfly, which gives every lane the same
// value (fp32 addition is commutative) and fixes the order: the result depends on the split
// count only, never on timing. Thread t < M also sums db[t] over the splits in order.
__device__ __forceinline__ void add4(float4& s, const float4& p) {
    s.x += p.x;
    s.y += p.y;
    s.z += p.z;
    s.w += p.w;
}

template <int SUB>
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ partial, int splits, int64_t MN,
                                                        float* __restrict__ out32, uint16_t* __restrict__ out16,
                                                        const float* __restrict__ dbp, int64_t M,
                                                        float* __restrict__ db) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i = (t / SUB) * 4;
    const int j = (int)(t % SUB);
    const int per = (splits + SUB - 1) / SUB;
    const int k0 = min(j * per, splits), k1 = min(k0 + per, splits);
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);  // splits == 0 (no K) writes zeros
    if (i < MN) {
        int k = k0;
        for (; k + 3 < k1; k += 4) {
            const float4 p0 = *(const float4*)(partial + (int64_t)k * MN + i);
            const float4 p1 = *(const float4*)(partial + (int64_t)(k + 1) * MN + i);
            const float4 p2 = *(const float4*)(partial + (int64_t)(k + 2) * MN + i);
            const float4 p3 = *(const float4*)(partial + (int64_t)(k + 3) * MN + i);
            add4(s, p0);
            add4(s, p1);
            add4(s, p2);
            add4(s, p3);
        }
        for (; k < k1; ++k) add4(s, *(const float4*)(partial + (int64_t)k * MN + i));
    }
    // all lanes of the wave take part in the butterfly (SUB divides 64 and the grid is whole waves)
#pragma unroll
    for (int m = 1; m < SUB; m <<= 1) {
        s.x += __shfl_xor(s.x, m);
        s.y += __shfl_xor(s.y, m);
        s.z += __shfl_xor(s.z, m);
        s.w += __shfl_xor(s.w, m);
    }
    if (i < MN && j == 0) {
        if (out32) *(float4*)(out32 + i) = s;
        if (out16) *(uint2*)(out16 + i) = make_uint2(pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w));
    }
    if (db && t < M) {
        float d = splits > 0 ? dbp[t] : 0.0f;
        int k = 1;
        for (; k + 3 < splits; k += 4) {
            const float p0 = dbp[(int64_t)k * M + t], p1 = dbp[(int64_t)(k + 1) * M + t];
            const float p2 = dbp[(int64_t)(k + 2) * M + t], p3 = dbp[(int64_t)(k + 3) * M + t];
            d += p0;
            d += p1;
            d += p2;
            d += p3;
        }
        for (; k < splits; ++k) d += dbp[(int64_t)k * M + t];
        db[t] = d;
    }
}

// one launch of the reduce: SUB lanes per output for a wide split count (more loads in flight)
void launch_dw_reduce(const float* partial, int used, int64_t MN, float* out32, uint16_t* out16, const float* dbp,
                      int64_t M, float* db, hipStream_t st) {
    const int sub = used > 16 ? 8 : used > 8 ? 4 : used > 4 ? 2 : 1;
    const int64_t threads = std::max<int64_t>(MN / 4 * sub, M);
    const dim3 grid((unsigned)((threads + 255) / 256));
#define DOPT_RED(S_) hipLaunchKernelGGL(dw_reduce_kernel<S_>, grid, dim3(256), 0, st, partial, used, MN, out32, out16, dbp, M, db)
    if (sub == 8) DOPT_RED(8);
    else if (sub == 4) DOPT_RED(4);
    else if (sub == 2) DOPT_RED(2);
    else DOPT_RED(1);
#undef DOPT_RED
}

}  // namespace

// Output rows per workgroup of the pipelined kernel: 128 when 256 x 256 tiles would number 16 or
// fewer (the split count, and with it the fp32 split partials written and read back, halves).
int dw_tile_rows(int64_t M, int64_t N) { return (M / 256) * (N / 256) <= 16 ? 128 : 256; }

int dw_splits(int64_t M, int64_t N, int64_t K) {
    // the same for every kernel of a shape, so all of them split K at the same token boundaries
    const int64_t tiles = std::max<int64_t>((M / dw_tile_rows(M, N)) * (N / BN), 1);
    const int64_t kts = (K + BK - 1) / BK;
    // one round of at most 256 workgroups (one per CU: 128 KB of LDS each)
    int64_t s = std::max<int64_t>(256 / tiles, 1);
    s = std::min(s, kts);
    return (int)std::max<int64_t>(s, 1);
}

int64_t dw_workspace_floats(int64_t M, int64_t N, int64_t K) {
    const int s = dw_splits(M, N, K);
    return (int64_t)s * M * N + (int64_t)s * M;
}

int launch_dw_gemm(DwArgs a, int mode, bool with_db, float* out32, uint16_t* out16, float* db, hipStream_t st) {
    const int splits = dw_splits(a.M, a.N, a.K);
    // the packed codes go through the pipelined kernel for 1/2/4 bits with DMA-aligned arrays
    // (codes 16-byte, scale/min 4-byte aligned); 8-bit codes through the register-decoding kernel
    const bool v2_packed = mode == DW_B_PACKED && (a.bits == 1 || a.bits == 2 || a.bits == 4) &&
                           ((uintptr_t)a.packed & 15u) == 0 && ((uintptr_t)a.scale & 3u) == 0 &&
                           ((uintptr_t)a.minv & 3u) == 0;
    // (the pipelined kernel keeps a slab's lane offsets in 32 bits: 32 rows of either operand
    // must span less than 4 GiB)
    const bool v2_offsets = a.ldd < ((int64_t)1 << 26) && a.ldx < ((int64_t)1 << 26) && a.N < ((int64_t)1 << 26);
    if ((mode == DW_B_BF16 || v2_packed) && v2_offsets && a.K > 0 && a.K % V2_BK == 0) {
        // the transpose-free kernel: 32-token tiles, split at the same token boundaries as the
        // 64-token kernel, so both accumulate the same 16-token MFMA steps in the same order
        // (K % 32 == 0 and N % 256 == 0 make the group count K N / g even, so the scale/min dword
        // loads stay inside their arrays)
        const int64_t kts = a.K / V2_BK;
        const int64_t kts64 = (a.K + BK - 1) / BK;
        a.kt_per_split = std::max<int64_t>((kts64 + splits - 1) / splits, 1) * (BK / V2_BK);
        const int used = (int)((kts + a.kt_per_split - 1) / a.kt_per_split);
        a.splits = used;
        a.db_partial = a.partial + (int64_t)splits * a.M * a.N;
        const int bmt = dw_tile_rows(a.M, a.N);
        const int64_t W = (a.M / bmt) * (a.N / BN) * used;
        const dim3 grid((unsigned)(DW_XCDS * ((W + DW_XCDS - 1) / DW_XCDS)));
#define DOPT_DW2T(BITS_, BMT_)                                                                                     \
    do {                                                                                                           \
        if (with_db) hipLaunchKernelGGL((dw_gemm_v2_kernel<BITS_, true, 4, BMT_>), grid, dim3(256), 0, st, a);      \
        else hipLaunchKernelGGL((dw_gemm_v2_kernel<BITS_, false, 4, BMT_>), grid, dim3(256), 0, st, a);             \
    } while (0)
#define DOPT_DW2(BITS_)                          \
    do {                                         \
        if (bmt == 128) DOPT_DW2T(BITS_, 128);   \
        else DOPT_DW2T(BITS_, 256);              \
    } while (0)
        if (mode == DW_B_BF16) DOPT_DW2(0);
        else if (a.bits == 1) DOPT_DW2(1);
        else if (a.bits == 2) DOPT_DW2(2);
        else DOPT_DW2(4);
#undef DOPT_DW2
#undef DOPT_DW2T
        launch_dw_reduce(a.partial, used, a.M * a.N, out32, out16, a.db_partial, a.M, with_db ? db : nullptr, st);
        return 0;
    }
    const int64_t kts = (a.K + BK - 1) / BK;
    a.kt_per_split = std::max<int64_t>((kts + splits - 1) / splits, 1);
    const int used = kts ? (int)((kts + a.kt_per_split - 1) / a.kt_per_split) : 0;  // splits with work
    a.splits = used;
    a.db_partial = a.partial + (int64_t)splits * a.M * a.N;
    const int tiles = (int)((a.M / BM) * (a.N / BN));
    // ids: 8 XCDs x ceil(W / 8) slots; slots past W exit at once
    const int64_t W = (int64_t)tiles * used;
    const dim3 grid((unsigned)(DW_XCDS * ((W + DW_XCDS - 1) / DW_XCDS)));
    if (used > 0) {
#define DOPT_DW(MODE_, BITS_, DB_) hipLaunchKernelGGL((dw_gemm_kernel<MODE_, BITS_, DB_>), grid, dim3(THREADS), 0, st, a)
#define DOPT_DW_DB(MODE_, BITS_) \
    do { if (with_db) DOPT_DW(MODE_, BITS_, true); else DOPT_DW(MODE_, BITS_, false); } while (0)
    if (mode == DW_B_BF16) DOPT_DW_DB(DW_B_BF16, 0);
    else if (a.bits == 1) DOPT_DW_DB(DW_B_PACKED, 1);
    else if (a.bits == 2) DOPT_DW_DB(DW_B_PACKED, 2);
    else if (a.bits == 4) DOPT_DW_DB(DW_B_PACKED, 4);
    else DOPT_DW_DB(DW_B_PACKED, 8);
#undef DOPT_DW_DB
#undef DOPT_DW
    }
    launch_dw_reduce(a.partial, used, a.M * a.N, out32, out16, a.db_partial, a.M, with_db ? db : nullptr, st);
    return 0;
}

}  // namespace dopt
