// Per-wave grouped W4A16 GEMM on v_mfma_f32_16x16x32_bf16: the general
// fallback for reduction lengths the streaming kernel does not split
// (any K % 512 == 0).
//
// One wave owns a 32-row strip of one weight matrix (two 16-row MFMA column
// tiles) and streams it once per pass over up to 32 of the slot's token rows.
// Packed int4 words are loaded 16 bytes per lane straight from HBM, turned
// into bf16 (136+q) in registers, multiplied on MFMA against octet-interleaved
// activations, and reduced per quantisation group with that group's scale.
// The +136 offset is removed at the end with one fp32 MFMA per 4 groups:
// tot += (-136*sum_group x) x scale.
//
// Semantics per mode (reference citations):
//   kModeLinear : y = x . dequant(W)^T, bf16 out                 (fused/quantization.py:154-165)
//   kModeGateUp : h = silu(x.Wg^T) * (x.Wu^T), gate rows first   (reference/fused_ops.py:170-171,
//                 h rounded to bf16, stored octet-interleaved      fused/quantization.py:193-195)
//   kModeDown   : y = route_weight * (h . Wd^T), fp32 out        (fused/quantization.py:196-199)
#include "kernels.h"

namespace dflash {

template <int kMode, int kMT, typename ScaleT>
__device__ __forceinline__ void w4_pass(const W4StreamParams& p, const uint8_t* __restrict__ w,
                                        const ScaleT* __restrict__ s, int seg, int M, int m0, bool shared, int row0,
                                        int row1, int strip) {
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int K = p.K, G = p.G;
  const int ngroups = K / G, spg = G >> 7, nkb = K >> 7;

  int arow[kMT];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    const int m = min(m0 + mt * 16 + lr, M - 1);
    if (kMode == kModeGateUp) arow[mt] = shared ? m : p.tok[seg + m];
    else if (kMode == kModeDown) arow[mt] = shared ? p.T * p.top_k + m : seg + m;
    else arow[mt] = m;
  }
  const uint16_t* ap[kMT];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) ap[mt] = p.act + static_cast<int64_t>(arow[mt]) * K + kq * 32;

  const int64_t row_bytes = K >> 1;
  const uint8_t* wp0 = w + static_cast<int64_t>(row0 + lr) * row_bytes + kq * 16;
  const uint8_t* wp1 = w + static_cast<int64_t>(row1 + lr) * row_bytes + kq * 16;
  const ScaleT* sp0 = s + static_cast<int64_t>(row0 + lr) * ngroups;
  const ScaleT* sp1 = s + static_cast<int64_t>(row1 + lr) * ngroups;

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 tot0[kMT], tot1[kMT], acc0[kMT], acc1[kMT];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) tot0[mt] = tot1[mt] = acc0[mt] = acc1[mt] = zero;

  for (int kb = 0; kb < nkb; kb += 4) {
    uint4 wq0[4], wq1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      wq0[u] = *reinterpret_cast<const uint4*>(wp0 + (kb + u) * 64);
      wq1[u] = *reinterpret_cast<const uint4*>(wp1 + (kb + u) * 64);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint4 a[kMT][4];
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) {
        const uint4* q = reinterpret_cast<const uint4*>(ap[mt] + (kb + u) * 128);
#pragma unroll
        for (int j = 0; j < 4; ++j) a[mt][j] = q[j];
      }
      const uint32_t w0[4] = {wq0[u].x, wq0[u].y, wq0[u].z, wq0[u].w};
      const uint32_t w1[4] = {wq1[u].x, wq1[u].y, wq1[u].z, wq1[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 b0 = dequant8(w0[j]);
        const uint4 b1 = dequant8(w1[j]);
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt) {
          acc0[mt] = mfma16x16x32(a[mt][j], b0, acc0[mt]);
          acc1[mt] = mfma16x16x32(a[mt][j], b1, acc1[mt]);
        }
      }
      if (((kb + u + 1) % spg) == 0) {
        const int g = (kb + u) / spg;
        const float sc0 = load_scale(sp0 + g), sc1 = load_scale(sp1 + g);
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt) {
          tot0[mt] += sc0 * acc0[mt];
          tot1[mt] += sc1 * acc1[mt];
          acc0[mt] = zero;
          acc1[mt] = zero;
        }
      }
    }
  }

  // remove the +136 offset: tot += sum_g (-136 * sum_{k in g} a[k]) * scale[g]
  for (int g0 = 0; g0 < ngroups; g0 += 4) {
    const int g = g0 + kq;
    const bool ok = g < ngroups;
    const float sv0 = ok ? load_scale(sp0 + g) : 0.f;
    const float sv1 = ok ? load_scale(sp1 + g) : 0.f;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
      float xv = 0.f;
      if (ok) {
        // act_neg holds neg_parts partial sums per 128-column block; a group spans spg blocks
        const int parts = spg * p.neg_parts;
        const float* src = p.act_neg + static_cast<int64_t>(arow[mt]) * nkb * p.neg_parts + g * parts;
        for (int c = 0; c < parts; ++c) xv += src[c];
      }
      tot0[mt] = mfma16x16x4f32(xv, sv0, tot0[mt]);
      tot1[mt] = mfma16x16x4f32(xv, sv1, tot1[mt]);
    }
  }

  // epilogue: lane holds rows m0 + mt*16 + 4*kq + e of columns (row0|row1) + lr
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + mt * 16 + 4 * kq + e;
      const bool valid = m < M;
      if (kMode == kModeLinear) {
        if (valid && p.out_f32) {  // fp32 output: the unrounded sums
          float* o = p.out_f32 + static_cast<int64_t>(m) * p.N;
          o[row0 + lr] = tot0[mt][e];
          o[row1 + lr] = tot1[mt][e];
        } else if (valid) {
          uint16_t* o = p.out_bf16 + static_cast<int64_t>(m) * p.N;
          o[row0 + lr] = f32_to_bf16(tot0[mt][e]);
          o[row1 + lr] = f32_to_bf16(tot1[mt][e]);
        }
      } else if (kMode == kModeGateUp) {
        const int inter = p.N >> 1;
        const int col = strip * 16 + lr;
        const uint16_t hb = f32_to_bf16(silu(tot0[mt][e]) * tot1[mt][e]);
        const int hrow = shared ? p.T * p.top_k + m : seg + m;
        if (valid) p.out_bf16[static_cast<int64_t>(hrow) * inter + octet_slot(col)] = hb;
        const float part = row16_sum(valid ? bf16_to_f32(hb) : 0.f);
        if (valid && lr == 0) p.out_part[static_cast<int64_t>(hrow) * (inter >> 4) + strip] = -kDequantOffset * part;
      } else {
        if (valid) {
          const float wgt = shared ? p.shared_gate[m] : p.slot_w[seg + m];
          const int yrow = shared ? p.T * p.top_k + m : seg + m;
          float* o = p.out_f32 + static_cast<int64_t>(yrow) * p.N;
          o[row0 + lr] = tot0[mt][e] * wgt;
          o[row1 + lr] = tot1[mt][e] * wgt;
        }
      }
    }
  }
}

template <int kMode, typename ScaleT>
__global__ __launch_bounds__(256) void w4_gemm_kernel(W4StreamParams p, int max_slots) {
  const int items_per_slot = p.N >> 5;  // gate_up: I/16 column pairs; down, linear: 32-row strips
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int slot = item / items_per_slot;
  const int strip = item - slot * items_per_slot;
  if (slot >= max_slots) return;
  const uint8_t* w;
  const ScaleT* s;
  int seg = 0, M;
  bool shared = false;
  if (kMode == kModeLinear) {
    w = p.w;
    s = static_cast<const ScaleT*>(p.s);
    M = p.M;
  } else {
    if (slot >= p.meta[0] + p.has_shared) return;
    const int4 d = p.slot_table[slot];  // expert (-1 shared), segment start, rows, first pass
    seg = d.y;
    M = d.z;
    if (d.x < 0) {
      shared = true;
      w = p.w_shared;
      s = static_cast<const ScaleT*>(p.s_shared);
    } else {
      w = p.w + d.x * p.w_stride;
      s = static_cast<const ScaleT*>(p.s) + d.x * p.s_stride;
    }
  }
  int row0, row1;
  if (kMode == kModeGateUp) {
    row0 = strip * 16;
    row1 = (p.N >> 1) + strip * 16;
  } else {
    row0 = strip * 32;
    row1 = row0 + 16;
  }
  for (int m0 = 0; m0 < M;) {
    if (M - m0 > 16) {
      w4_pass<kMode, 2, ScaleT>(p, w, s, seg, M, m0, shared, row0, row1, strip);
      m0 += 32;
    } else {
      w4_pass<kMode, 1, ScaleT>(p, w, s, seg, M, m0, shared, row0, row1, strip);
      m0 += 16;
    }
  }
}

void launch_w4_gemm(int mode, bool fp32_scales, int max_slots, const W4StreamParams& p, hipStream_t stream) {
  const int64_t items = static_cast<int64_t>(max_slots) * (p.N >> 5);
  if (items <= 0) return;
  const dim3 grid(static_cast<unsigned>((items + 3) / 4)), block(256);
#define DFLASH_W4_LAUNCH(MODE)                                                                          \
  if (fp32_scales) hipLaunchKernelGGL((w4_gemm_kernel<MODE, float>), grid, block, 0, stream, p, max_slots); \
  else hipLaunchKernelGGL((w4_gemm_kernel<MODE, uint16_t>), grid, block, 0, stream, p, max_slots);
  switch (mode) {
    case kModeLinear: DFLASH_W4_LAUNCH(kModeLinear) break;
    case kModeGateUp: DFLASH_W4_LAUNCH(kModeGateUp) break;
    default: DFLASH_W4_LAUNCH(kModeDown) break;
  }
#undef DFLASH_W4_LAUNCH
}

}  // namespace dflash
