// Layout conversion for the FP8 GEMM: any strided byte matrix -> K-contiguous rows.
//
// dst[r * ld_dst + c] = src[r * stride_r + c * stride_c] for r < rows, c < cols (element strides
// in bytes, any non-negative values). The GEMM (fp8_gemm.h) reads both operands K-contiguous; the
// reference's Triton_Linear (Activation_Compression/triton_kernel/linear.py:43-95) takes A [M, K]
// and B [K, N] with arbitrary strides, so B in its natural row-major [K, N] layout (stride_r =
// 1 along N, stride_c = ldb along K) is transposed here into [N, K].
//
// Two kernels:
//   - transpose (stride_r == 1): 64 x 64 byte tiles through LDS; each lane reads 16 contiguous
//     source bytes (one column c, rows r..r+15) and, after the LDS round trip, writes 16
//     contiguous destination bytes (one row r, columns c..c+15). The LDS tile is padded by 16
//     bytes per row so the column-wise writes fall in different banks.
//   - gather (anything else): one byte per lane, consecutive lanes along c.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dopt {

constexpr int TP = 64;  // tile edge (bytes)

__global__ __launch_bounds__(256) void fp8_transpose_kernel(const uint8_t* __restrict__ src, int64_t rows,
                                                            int64_t cols, int64_t stride_c, uint8_t* __restrict__ dst,
                                                            int64_t ld_dst, uint32_t row_tiles) {
    __shared__ uint8_t t[TP][TP + 16];
    const int64_t r0 = (int64_t)(blockIdx.x % row_tiles) * TP, c0 = (int64_t)(blockIdx.x / row_tiles) * TP;
    const int lane = threadIdx.x;
    // read: lane -> column c0 + lane / 4, rows r0 + 16 (lane % 4) .. +15 (contiguous in src)
    {
        const int cl = lane >> 2, rl = (lane & 3) * 16;
        const int64_t c = c0 + cl, r = r0 + rl;
        uint8_t v[16];
        if (c < cols && r + 16 <= rows && (((uintptr_t)(src + c * stride_c + r)) & 15) == 0) {
            const uint4 x = *(const uint4*)(src + c * stride_c + r);
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = (c < cols && r + i < rows) ? src[c * stride_c + r + i] : 0;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) t[rl + i][cl] = v[i];
    }
    __syncthreads();
    // write: lane -> row r0 + lane / 4, columns c0 + 16 (lane % 4) .. +15 (contiguous in dst)
    {
        const int rl = lane >> 2, cl = (lane & 3) * 16;
        const int64_t r = r0 + rl, c = c0 + cl;
        if (r >= rows) return;
        uint8_t* d = dst + r * ld_dst + c;
        if (c + 16 <= cols && (((uintptr_t)d) & 15) == 0) {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t)t[rl][cl + i] << (8 * (i & 3));
            *(uint4*)d = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int i = 0; i < 16 && c + i < cols; ++i) d[i] = t[rl][cl + i];
        }
    }
}

__global__ __launch_bounds__(256) void fp8_gather_kernel(const uint8_t* __restrict__ src, int64_t rows, int64_t cols,
                                                         int64_t stride_r, int64_t stride_c, uint8_t* __restrict__ dst,
                                                         int64_t ld_dst, uint32_t col_blocks) {
    const int64_t r = blockIdx.x / col_blocks;
    const int64_t c = (int64_t)(blockIdx.x % col_blocks) * 256 + threadIdx.x;
    if (r < rows && c < cols) dst[r * ld_dst + c] = src[r * stride_r + c * stride_c];
}

int launch_fp8_pack(const uint8_t* src, int64_t rows, int64_t cols, int64_t stride_r, int64_t stride_c, uint8_t* dst,
                    int64_t ld_dst, hipStream_t s) {
    if (rows == 0 || cols == 0) return 0;
    if (stride_r == 1) {
        const uint64_t rt = (uint64_t)((rows + TP - 1) / TP), ct = (uint64_t)((cols + TP - 1) / TP);
        if (rt * ct >= (1ull << 31)) return -1;
        hipLaunchKernelGGL(fp8_transpose_kernel, dim3((uint32_t)(rt * ct)), dim3(256), 0, s, src, rows, cols, stride_c,
                           dst, ld_dst, (uint32_t)rt);
    } else {
        const uint64_t cb = (uint64_t)((cols + 255) / 256);
        if ((uint64_t)rows * cb >= (1ull << 31)) return -1;
        hipLaunchKernelGGL(fp8_gather_kernel, dim3((uint32_t)(rows * cb)), dim3(256), 0, s, src, rows, cols, stride_r,
                           stride_c, dst, ld_dst, (uint32_t)cb);
    }
    return 0;
}

}  // namespace dopt
