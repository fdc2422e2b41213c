// W4A16 linear for the verify block's short activations and narrow outputs, where a launch is
// bound by its chain of dependent steps rather than by bytes (a 16-row projection with N <= a
// few thousand moves a few MB at most).
//
// Workgroup = 16 output columns (one 16-row weight tile), 8 waves; wave w takes k-blocks
// [w kKPW, (w + 1) kKPW) of the reduction (kKPW = K / 1024 rounded up).  Every operand of a
// wave is requested at once, straight into MFMA fragment registers:
//   * per k-block one 16-byte load per lane of the weight tile -- lane (Q, r) gets 32-column
//     quarter Q of row r (tiled: the k-block's kilobyte; portable: 16 bytes of the row) --
//     transposed across lane quarters (quarter_transpose) so that lane (Q, r) holds k-octet Q
//     of every quarter of row r, the B operand of one v_mfma_f32_16x16x32_bf16 per quarter;
//   * the group scale of the lane's column r;
//   * per 16-row tile of x and quarter one 16-byte load (row r, k-octet Q), reordered in
//     registers to the octet order the dequantisation produces (k0 k4 k1 k5 k2 k6 k3 k7).
// The dequantised weights are 136 + q (dequant8); one more MFMA per quarter with every B value
// -136 removes the offset, so acc = sum x q exactly as the MFMA rounds it.  Each k-block adds
// s * acc to the wave's sum; the eight sums meet in LDS and wave 0 adds them in wave order and
// writes bf16 (or fp32) outputs.  No LDS staging, one barrier.
//
// Reference: OriginalQuantizedWeights.linear, fused/quantization.py:154-165 (a vendor int4
// matmul over the dequantised weight q * s); semantics y = x (q s)^T as the oracle states it.
#include "kernels.h"

namespace dflash {
namespace {

constexpr int kSmallWaves = 8;
constexpr uint32_t kMinus136Pair = 0xC308C308u;  // bf16 pair (-136, -136)

// natural bf16 pairs (k0,k1)(k2,k3)(k4,k5)(k6,k7) -> (k0,k4)(k1,k5)(k2,k6)(k3,k7)
__device__ __forceinline__ uint4 octet_interleave(uint4 v) {
  uint4 o;
  o.x = (v.x & 0xFFFFu) | (v.z << 16);
  o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
  o.z = (v.y & 0xFFFFu) | (v.w << 16);
  o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
  return o;
}

template <int kRT, int kKPW>
__global__ __launch_bounds__(512) void w4_small_kernel(SmallLinearParams p) {
  __shared__ f32x4 part[kSmallWaves][kRT][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int t = blockIdx.x;  // 16-column weight tile
  const int K = p.K, N = p.N, M = p.M;
  const int nkb = K >> 7, ngd = K / p.G, gshift = p.G == 256 ? 1 : 0;
  const int kb0 = wave * kKPW, nk = min(kKPW, nkb - kb0);  // nk <= 0: a wave past K
  const uint32_t ssize = p.scale_f32 ? 4u : 2u;
  const buf_rsrc wr = make_rsrc(p.w, static_cast<uint32_t>(N) * static_cast<uint32_t>(K) / 2u);
  const buf_rsrc sr = make_rsrc(p.s, static_cast<uint32_t>(N) * static_cast<uint32_t>(ngd) * ssize);
  const buf_rsrc xr = make_rsrc(p.x, static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u);

  uint4 wv[kKPW];
  uint32_t sv[kKPW];
  uint4 xv[kKPW][kRT][4];
#pragma unroll
  for (int i = 0; i < kKPW; ++i) {
    const int kb = min(kb0 + i, nkb - 1);  // past K: the last k-block again, never used
    const uint32_t woff = p.tiled ? static_cast<uint32_t>(t * nkb + kb) * 1024u + static_cast<uint32_t>(lane) * 16u
                                  : static_cast<uint32_t>(t * 16 + lr) * static_cast<uint32_t>(K / 2) +
                                        static_cast<uint32_t>(kb * 64 + kq * 16);
    wv[i] = buf_load16(wr, woff, 0);
    const int g = kb >> gshift;
    const uint32_t sidx = p.tiled ? static_cast<uint32_t>((t * ngd + g) * 16 + lr)
                                  : static_cast<uint32_t>((t * 16 + lr) * ngd + g);
    sv[i] = p.scale_f32 ? __builtin_amdgcn_raw_buffer_load_b32(sr, static_cast<int>(sidx * 4u), 0, 0)
                        : __builtin_amdgcn_raw_buffer_load_b16(sr, static_cast<int>(sidx * 2u), 0, 0);
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      const int row = min(rt * 16 + lr, M - 1);  // rows past M repeat the last, never stored
#pragma unroll
      for (int dq = 0; dq < 4; ++dq)
        xv[i][rt][dq] = buf_load16(xr, static_cast<uint32_t>((row * K + kb * 128 + dq * 32 + kq * 8) * 2), 0);
    }
  }

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const uint4 minus136 = make_uint4(kMinus136Pair, kMinus136Pair, kMinus136Pair, kMinus136Pair);
  f32x4 tot[kRT];
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) tot[rt] = zero;
#pragma unroll
  for (int i = 0; i < kKPW; ++i) {
    if (i < nk) {
      uint32_t w[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
      quarter_transpose(w);
      const float s = p.scale_f32 ? __uint_as_float(sv[i]) : __uint_as_float(sv[i] << 16);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        f32x4 acc = zero;
#pragma unroll
        for (int dq = 0; dq < 4; ++dq) {
          const uint4 a = octet_interleave(xv[i][rt][dq]);
          acc = mfma16x16x32(a, minus136, acc);
          acc = mfma16x16x32(a, dequant8(w[dq]), acc);
        }
        tot[rt] += s * acc;
      }
    }
  }
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) part[wave][rt][lane] = tot[rt];
  __syncthreads();
  if (wave < kRT) {  // wave rt adds row tile rt over the waves, in wave order
    const int rt = wave;
    f32x4 y = part[0][rt][lane];
#pragma unroll
    for (int w = 1; w < kSmallWaves; ++w) y += part[w][rt][lane];
    const int col = t * 16 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = rt * 16 + 4 * kq + e;
      if (row < M) {
        if (p.y_f32) static_cast<float*>(p.y)[static_cast<int64_t>(row) * N + col] = y[e];
        else static_cast<uint16_t*>(p.y)[static_cast<int64_t>(row) * N + col] = f32_to_bf16(y[e]);
      }
    }
  }
}

// The streaming form for wide outputs (the LM head): persistent workgroups, each wave keeps
// its k-slice of x (16 rows) in registers for the whole launch and streams weight tiles.
// Workgroup b takes batches of kBatch tiles b, b + G, ... (8, 4 or 2 tiles: 8 weight loads per
// lane per batch at any K) so the grid reads one contiguous window of the weights at a time;
// the weights of the next batch are requested before the current one is computed.  After a
// batch each wave leaves one partial per tile in LDS (two buffers, alternating), one barrier,
// and wave c adds tile c of the batch over the waves and writes it.
template <int kKPW>
__global__ __launch_bounds__(512) void w4_small_stream_kernel(SmallLinearParams p) {
  constexpr int kBatch = 8 / kKPW;
  __shared__ f32x4 part[2][kSmallWaves][kBatch][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int K = p.K, N = p.N, M = p.M;
  const int nkb = K >> 7, ngd = K / p.G, gshift = p.G == 256 ? 1 : 0;
  const int kb0 = wave * kKPW, nk = min(kKPW, nkb - kb0);
  const int tiles = N >> 4, batches = (tiles + kBatch - 1) / kBatch;
  const uint32_t ssize = p.scale_f32 ? 4u : 2u;
  const buf_rsrc wr = make_rsrc(p.w, static_cast<uint32_t>(N) * static_cast<uint32_t>(K) / 2u);
  const buf_rsrc sr = make_rsrc(p.s, static_cast<uint32_t>(N) * static_cast<uint32_t>(ngd) * ssize);
  const buf_rsrc xr = make_rsrc(p.x, static_cast<uint32_t>(M) * static_cast<uint32_t>(K) * 2u);

  // this wave's k-slice of x, octet-interleaved, for the whole launch
  uint4 xa[kKPW][4];
  {
    const int row = min(lr, M - 1);
#pragma unroll
    for (int i = 0; i < kKPW; ++i) {
      const int kb = min(kb0 + i, nkb - 1);
#pragma unroll
      for (int dq = 0; dq < 4; ++dq)
        xa[i][dq] = buf_load16(xr, static_cast<uint32_t>((row * K + kb * 128 + dq * 32 + kq * 8) * 2), 0);
    }
  }
  // lane parts of the weight and scale offsets of tile t, k-block kb
  auto woff = [&](int t, int kb) {
    return p.tiled ? static_cast<uint32_t>(t * nkb + kb) * 1024u + static_cast<uint32_t>(lane) * 16u
                   : static_cast<uint32_t>(t * 16 + lr) * static_cast<uint32_t>(K / 2) +
                         static_cast<uint32_t>(kb * 64 + kq * 16);
  };
  auto sidx = [&](int t, int kb) {
    const int g = kb >> gshift;
    return p.tiled ? static_cast<uint32_t>((t * ngd + g) * 16 + lr) : static_cast<uint32_t>((t * 16 + lr) * ngd + g);
  };
  struct Batch {
    uint4 w[kBatch][kKPW];
    uint32_t s[kBatch][kKPW];
  };
  // tiles past N read nothing (an offset past the buffer) and are never stored
  auto issue = [&](Batch& bt, int j) {
#pragma unroll
    for (int c = 0; c < kBatch; ++c) {
      const int t = j * kBatch + c;
#pragma unroll
      for (int i = 0; i < kKPW; ++i) {
        const int kb = min(kb0 + i, nkb - 1);
        const bool live = t < tiles;
        bt.w[c][i] = buf_load16(wr, live ? woff(t, kb) : 0x80000000u, 0);
        const uint32_t so = live ? sidx(t, kb) * ssize : 0x80000000u;
        bt.s[c][i] = p.scale_f32 ? __builtin_amdgcn_raw_buffer_load_b32(sr, static_cast<int>(so), 0, 0)
                                 : __builtin_amdgcn_raw_buffer_load_b16(sr, static_cast<int>(so), 0, 0);
      }
    }
  };
  for (int i = 0; i < kKPW; ++i)
    for (int dq = 0; dq < 4; ++dq) xa[i][dq] = octet_interleave(xa[i][dq]);

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const uint4 minus136 = make_uint4(kMinus136Pair, kMinus136Pair, kMinus136Pair, kMinus136Pair);
  const int G = static_cast<int>(gridDim.x);
  Batch ring[2];
  int j = static_cast<int>(blockIdx.x);
  issue(ring[0], j);
  for (int it = 0; j < batches; ++it, j += G) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {  // ring slot u: batch j (slot it % 2, unrolled by two)
      if (u != (it & 1)) continue;
      issue(ring[u ^ 1], j + G);  // past the last batch: loads of nothing (offsets past the buffer)
      const Batch& bt = ring[u];
#pragma unroll
      for (int c = 0; c < kBatch; ++c) {
        f32x4 tot = zero;
#pragma unroll
        for (int i = 0; i < kKPW; ++i) {
          if (i < nk) {
            uint32_t w[4] = {bt.w[c][i].x, bt.w[c][i].y, bt.w[c][i].z, bt.w[c][i].w};
            quarter_transpose(w);
            const float s = p.scale_f32 ? __uint_as_float(bt.s[c][i]) : __uint_as_float(bt.s[c][i] << 16);
            f32x4 acc = zero;
#pragma unroll
            for (int dq = 0; dq < 4; ++dq) {
              acc = mfma16x16x32(xa[i][dq], minus136, acc);
              acc = mfma16x16x32(xa[i][dq], dequant8(w[dq]), acc);
            }
            tot += s * acc;
          }
        }
        part[it & 1][wave][c][lane] = tot;
      }
    }
    lds_barrier();
    // wave c: tile c of the batch, summed over the waves in wave order
    const int t = j * kBatch + wave;
    if (wave < kBatch && t < tiles) {
      f32x4 y = part[it & 1][0][wave][lane];
#pragma unroll
      for (int w = 1; w < kSmallWaves; ++w) y += part[it & 1][w][wave][lane];
      const int col = t * 16 + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * kq + e;
        if (row < M) {
          if (p.y_f32) static_cast<float*>(p.y)[static_cast<int64_t>(row) * N + col] = y[e];
          else static_cast<uint16_t*>(p.y)[static_cast<int64_t>(row) * N + col] = f32_to_bf16(y[e]);
        }
      }
    }
  }
}

}  // namespace

bool small_linear_fits(int M, int N, int K, int G) {
  return M >= 1 && M <= 32 && N >= 16 && N % 16 == 0 && (K == 512 || K == 1024 || K == 2048 || K == 4096) &&
         (G == 128 || G == 256);
}

bool small_linear_stream_fits(int M, int N, int K, int G) { return small_linear_fits(M, N, K, G) && M <= 16; }

void launch_w4_small_stream(const SmallLinearParams& p, int grid, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid)), block(kSmallWaves * 64);
  const int kpw = (p.K / 128 + kSmallWaves - 1) / kSmallWaves;
  if (kpw == 1) hipLaunchKernelGGL((w4_small_stream_kernel<1>), g, block, 0, stream, p);
  else if (kpw == 2) hipLaunchKernelGGL((w4_small_stream_kernel<2>), g, block, 0, stream, p);
  else hipLaunchKernelGGL((w4_small_stream_kernel<4>), g, block, 0, stream, p);
}

void launch_w4_small(const SmallLinearParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.N / 16)), block(kSmallWaves * 64);
  const int kpw = (p.K / 128 + kSmallWaves - 1) / kSmallWaves;  // 1, 2 or 4
#define DFLASH_SMALL(RT, KPW) hipLaunchKernelGGL((w4_small_kernel<RT, KPW>), grid, block, 0, stream, p)
  if (p.M > 16) {
    if (kpw == 1) DFLASH_SMALL(2, 1);
    else if (kpw == 2) DFLASH_SMALL(2, 2);
    else DFLASH_SMALL(2, 4);
  } else {
    if (kpw == 1) DFLASH_SMALL(1, 1);
    else if (kpw == 2) DFLASH_SMALL(1, 2);
    else DFLASH_SMALL(1, 4);
  }
#undef DFLASH_SMALL
}

}  // namespace dflash
