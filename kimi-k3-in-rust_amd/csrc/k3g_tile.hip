/* k3g_tile.hip - repack weights from the checkpoint's row-major layouts into the tiled
 * layouts the matrix-core kernels stream.
 *
 * Why tile. A 16x16xK MFMA takes its A operand as 16 rows x K: lane L holds row L%16 and
 * the (L/16)-th quarter of the K step. Read straight from a row-major matrix, one load
 * instruction of such an operand touches 16 rows x 64 contiguous bytes, and the memory
 * pipeline then moves whole 128-byte lines in pieces; measured on MI355X that caps a
 * gate/up GEMV at ~3.7 TB/s against ~4.7 TB/s when every load instruction reads one
 * contiguous 1 KB run. The tiled layouts store each MFMA operand as that contiguous
 * 1 KB run (lane-major, 16 bytes per lane), so the streaming kernels read the weights
 * at full line granularity and hand them to the matrix cores untouched.
 *
 * MXFP4 tiled (matrix rows % 16 == 0, cols % 32 == 0; cols padded up to a multiple of
 * 512 with zero nibbles and unit scales):
 *   quad tile (row block rb of 16 rows, quad Q of 512 columns) = 4352 bytes at
 *   (rb * nQ + Q) * 4352:
 *     bytes [1024 j, 1024 j + 1024), j = 0..3: chunk j, lane L's 16 bytes at 16 L are
 *       the 32 nibbles of row 16 rb + L%16, MX block 16 Q + 4 j + L/16 (the engine's
 *       packed bytes of that block, unchanged: low nibble = even column)
 *     bytes [4096, 4352): lane L's 4 bytes at 4096 + 4 L; byte j is the E8M0 scale of
 *       chunk j's block for that lane
 *   A block whose scale byte is 255 (NaN in the OCP format; the engine's table maps it
 *   to 0, src/core/k3_ops.c:1315-1322) is stored as zero nibbles with scale 127, which
 *   contributes the same zero without a NaN ever reaching the matrix cores.
 *   An MXFP4 matrix keeps its size: rows * cols / 2 packed bytes + rows * cols / 32
 *   scales (plus the padding when cols % 512 != 0).
 *
 * bf16 tiled (rows % 16 == 0, cols % 32 == 0):
 *   chunk tile (row block rb, chunk c of 32 columns) = 1024 bytes at (rb * cols/32 + c)
 *   * 1024; lane L's 16 bytes are row 16 rb + L%16, columns 32 c + 8 (L/16) .. + 8.
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"

#define K3G_QT 4352

/* one 64-lane block per quad tile; every lane writes its 4 x 16 data bytes and its scale
 * dword */
__global__ void __launch_bounds__(64)
k_tile_mxfp4(uint8_t *dst, const uint8_t *packed, const uint8_t *scales, int rows, int cols)
{
    const int nQ = (cols + 511) / 512;
    const int tile = blockIdx.x;
    const int rb = tile / nQ, Q = tile - rb * nQ;
    const int L = threadIdx.x;
    const int row = 16 * rb + (L & 15);
    const size_t prow = (size_t)row * (cols / 2), srow = (size_t)row * (cols / 32);
    uint8_t *t = dst + (size_t)tile * K3G_QT;
    uint32_t sw = 0;
    for (int j = 0; j < 4; ++j) {
        const int b = 16 * Q + 4 * j + (L >> 4);
        uint8_t *o = t + 1024 * j + 16 * L;
        uint32_t s = 127;
        if (32 * b < cols && scales[srow + b] != 255) {
            const uint8_t *p = packed + prow + 16 * (size_t)b;
            for (int i = 0; i < 16; ++i) o[i] = p[i];
            s = scales[srow + b];
        } else {
            for (int i = 0; i < 16; ++i) o[i] = 0;
        }
        sw |= s << (8 * j);
    }
    *(uint32_t *)(t + 4096 + 4 * L) = sw;
}

__global__ void __launch_bounds__(64)
k_tile_bf16(uint16_t *dst, const uint16_t *src, int rows, int cols)
{
    const int nC = cols / 32;
    const int tile = blockIdx.x;
    const int rb = tile / nC, c = tile - rb * nC;
    const int L = threadIdx.x;
    const uint16_t *s = src + (size_t)(16 * rb + (L & 15)) * cols + 32 * c + 8 * (L >> 4);
    uint16_t *o = dst + (size_t)tile * 512 + 8 * L;
    for (int i = 0; i < 8; ++i) o[i] = s[i];
}

extern "C" size_t k3k_tiled_mxfp4_bytes(int rows, int cols)
{
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 32) return 0;
    return (size_t)(rows / 16) * ((cols + 511) / 512) * K3G_QT;
}

extern "C" size_t k3k_tiled_bf16_bytes(int rows, int cols)
{
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 32) return 0;
    return (size_t)rows * cols * 2;
}

extern "C" int k3k_tile_mxfp4(uint8_t *dst, const uint8_t *packed, const uint8_t *scales,
                              int rows, int cols, hipStream_t st)
{
    const size_t n = k3k_tiled_mxfp4_bytes(rows, cols);
    if (!n || !dst || !packed || !scales) return -1;
    const int tiles = (rows / 16) * ((cols + 511) / 512);
    hipLaunchKernelGGL(k_tile_mxfp4, dim3(tiles), dim3(64), 0, st, dst, packed, scales, rows,
                       cols);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_tile_bf16(uint16_t *dst, const uint16_t *src, int rows, int cols,
                             hipStream_t st)
{
    if (!k3k_tiled_bf16_bytes(rows, cols) || !dst || !src) return -1;
    const int tiles = (rows / 16) * (cols / 32);
    hipLaunchKernelGGL(k_tile_bf16, dim3(tiles), dim3(64), 0, st, dst, src, rows, cols);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
