// One-time repack of packed int4 banks from the reference's portable order
// (graph/quant_weights.py:147-148: uint8 [E][N][K/2], scales [E][N][K/G]) into
// the tiled order the expert kernels stream: per expert, per 16-row tile t and
// 128-column block b, one contiguous kilobyte whose 16-byte chunk l (the chunk
// lane l of a wave loads) holds bytes 64*b + 16*(l >> 4) .. +15 of row
// 16*t + (l & 15); scales [E][N/16][K/G][16].  A pure permutation: every byte
// and every scale is copied once, nothing is converted.
#include "kernels.h"

namespace dflash {
namespace {

// One thread per 16-byte chunk of the output.
__global__ __launch_bounds__(256) void tile_weights_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                           int64_t chunks, int rows, int cols) {
  const int64_t rb16 = cols / 32;              // 16-byte chunks per portable row (K/2 bytes)
  const int64_t per_tile = static_cast<int64_t>(cols / 128) * 64;
  const int64_t per_expert = static_cast<int64_t>(rows / 16) * per_tile;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < chunks;
       o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t e = o / per_expert;
    int64_t r = o - e * per_expert;
    const int64_t t = r / per_tile;
    r -= t * per_tile;
    const int64_t b = r >> 6;
    const int l = static_cast<int>(r & 63);
    const int64_t row = e * rows + t * 16 + (l & 15);
    dst[o] = src[row * rb16 + b * 4 + (l >> 4)];
  }
}

// One thread per scale element of the output.
template <typename ScaleT>
__global__ __launch_bounds__(256) void tile_scales_kernel(const ScaleT* __restrict__ src, ScaleT* __restrict__ dst,
                                                          int64_t count, int rows, int groups) {
  const int64_t per_tile = static_cast<int64_t>(groups) * 16;
  const int64_t per_expert = static_cast<int64_t>(rows / 16) * per_tile;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < count;
       o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t e = o / per_expert;
    int64_t r = o - e * per_expert;
    const int64_t t = r / per_tile;
    r -= t * per_tile;
    const int64_t g = r >> 4;
    const int c = static_cast<int>(r & 15);
    dst[o] = src[(e * rows + t * 16 + c) * groups + g];
  }
}

unsigned grid_for(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return static_cast<unsigned>(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

}  // namespace

void launch_tile_w4(const void* packed, const void* scales, bool fp32_scales, int64_t experts, int rows, int cols,
                    int group, void* packed_out, void* scales_out, hipStream_t stream) {
  const int64_t chunks = experts * rows * static_cast<int64_t>(cols) / 32;
  hipLaunchKernelGGL(tile_weights_kernel, dim3(grid_for(chunks)), dim3(256), 0, stream,
                     static_cast<const uint4*>(packed), static_cast<uint4*>(packed_out), chunks, rows, cols);
  const int groups = cols / group;
  const int64_t count = experts * rows * static_cast<int64_t>(groups);
  if (fp32_scales)
    hipLaunchKernelGGL(tile_scales_kernel<float>, dim3(grid_for(count)), dim3(256), 0, stream,
                       static_cast<const float*>(scales), static_cast<float*>(scales_out), count, rows, groups);
  else
    hipLaunchKernelGGL(tile_scales_kernel<uint16_t>, dim3(grid_for(count)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(scales_out), count, rows, groups);
}

}  // namespace dflash
