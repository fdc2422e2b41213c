// Load-time repacks of int4 banks.
//  * Portable -> tiled: from the reference's portable order (graph/quant_weights.py:147-148:
//    uint8 [E][N][K/2], scales [E][N][K/G]) into the tiled order the expert kernels stream:
//    per expert, per 16-row tile t and 128-column block b, one contiguous kilobyte whose
//    16-byte chunk l (the chunk lane l of a wave loads) holds bytes 64*b + 16*(l >> 4) .. +15
//    of row 16*t + (l & 15); scales [E][N/16][K/G][16].  A pure permutation: every byte and
//    every scale is copied once, nothing is converted.
//  * int8-carried -> packed: the original checkpoint keeps one signed int8 per int4 value
//    (target/original_quant.py:80-112, values in [-8, 7]) and fp16/fp32 group scales
//    (:113-133, finite and nonnegative); one pass packs the nibbles (value 2m low in byte
//    m) straight into the portable or the tiled order and widens the scales to fp32,
//    counting the values and scales the reader would reject.
#include "../../include/dflash_hip.h"
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

// One thread per 16-byte output chunk (32 int4 values) of the portable or tiled
// layout, from the int8-carried values; counts values outside [-8, 7] into bad[0].
__global__ __launch_bounds__(256) void from_int8_weights_kernel(const int8_t* __restrict__ src, uint4* __restrict__ dst,
                                                                int64_t chunks, int rows, int cols, int tiled,
                                                                int32_t* __restrict__ bad) {
  const int64_t rb16 = cols / 32;  // output chunks per row
  const int64_t per_tile = static_cast<int64_t>(cols / 128) * 64;
  const int64_t per_expert = static_cast<int64_t>(rows / 16) * per_tile;
  int outside = 0;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < chunks;
       o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t row, chunk;  // source row (experts stacked) and its 32-value chunk
    if (tiled) {
      const int64_t e = o / per_expert;
      int64_t r = o - e * per_expert;
      const int64_t t = r / per_tile;
      r -= t * per_tile;
      const int l = static_cast<int>(r & 63);
      row = e * rows + t * 16 + (l & 15);
      chunk = (r >> 6) * 4 + (l >> 4);
    } else {
      row = o / rb16;
      chunk = o - row * rb16;
    }
    const uint4* s = reinterpret_cast<const uint4*>(src + row * cols + chunk * 32);
    const uint4 lo = s[0], hi = s[1];
    const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    uint32_t out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // output word i: values 8i .. 8i + 7
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int v = static_cast<int8_t>((w[2 * i + j / 4] >> (8 * (j & 3))) & 0xFFu);
        outside += (v < -8 || v > 7) ? 1 : 0;
        word |= static_cast<uint32_t>(v & 15) << (4 * j);  // value 2m in the low nibble of byte m
      }
      out[i] = word;
    }
    dst[o] = make_uint4(out[0], out[1], out[2], out[3]);
  }
  if (outside) atomicAdd(bad, outside);
}

// One thread per fp32 output scale; counts negative or non-finite source scales into bad[1].
__global__ __launch_bounds__(256) void from_int8_scales_kernel(const void* __restrict__ src, int src_dtype,
                                                               float* __restrict__ dst, int64_t count, int rows,
                                                               int groups, int tiled, int32_t* __restrict__ bad) {
  const int64_t per_tile = static_cast<int64_t>(groups) * 16;
  const int64_t per_expert = static_cast<int64_t>(rows / 16) * per_tile;
  int wrong = 0;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < count;
       o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t i = o;  // source element [row][group]
    if (tiled) {
      const int64_t e = o / per_expert;
      int64_t r = o - e * per_expert;
      const int64_t t = r / per_tile;
      r -= t * per_tile;
      i = (e * rows + t * 16 + (r & 15)) * groups + (r >> 4);
    }
    float v;
    if (src_dtype == DFLASH_DTYPE_F32) v = static_cast<const float*>(src)[i];
    else if (src_dtype == DFLASH_DTYPE_F16) v = static_cast<float>(static_cast<const _Float16*>(src)[i]);
    else v = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(src)[i]) << 16);
    wrong += (v >= 0.f && v <= 3.402823466e38f) ? 0 : 1;  // NaN fails both
    dst[o] = v;
  }
  if (wrong) atomicAdd(bad + 1, wrong);
}

__global__ void clear_counts_kernel(int32_t* bad) {
  if (threadIdx.x < 2) bad[threadIdx.x] = 0;
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

void launch_from_int8(const int8_t* values, const void* scales, int scales_dtype, int64_t experts, int rows,
                      int cols, int group, bool tiled, void* packed_out, float* scales_out, int32_t* bad,
                      hipStream_t stream) {
  hipLaunchKernelGGL(clear_counts_kernel, dim3(1), dim3(64), 0, stream, bad);
  const int64_t chunks = experts * rows * static_cast<int64_t>(cols) / 32;
  hipLaunchKernelGGL(from_int8_weights_kernel, dim3(grid_for(chunks)), dim3(256), 0, stream, values,
                     static_cast<uint4*>(packed_out), chunks, rows, cols, tiled ? 1 : 0, bad);
  const int groups = cols / group;
  const int64_t count = experts * rows * static_cast<int64_t>(groups);
  hipLaunchKernelGGL(from_int8_scales_kernel, dim3(grid_for(count)), dim3(256), 0, stream, scales, scales_dtype,
                     scales_out, count, rows, groups, tiled ? 1 : 0, bad);
}

}  // namespace dflash
