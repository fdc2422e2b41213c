// Persistent streaming W4A16 GEMM for the verify-block path (T up to ~128).
//
// Grid = one 512-thread workgroup per CU.  The routing work table lists slots
// (hit experts, then the shared expert) and their passes (up to 16*kMT tokens
// each); a "unit" is one pass times one strip of weight rows.  Units are split
// into equal contiguous ranges, one per workgroup, so every CU streams the
// same number of weight bytes.
//
// Inside a workgroup the 8 waves split K: wave (rg, ks) handles row group rg
// and k-blocks [ks*KBPW, (ks+1)*KBPW) of 128 columns.  Per unit each wave
// loads its 16-byte slices of two 16-row weight tiles straight from HBM,
// dequantises them in registers (bf16 136+q), runs v_mfma_f32_16x16x32_bf16
// against the octet-interleaved activations, and scales per group.  The
// offset is removed by starting each k-block's MFMA chain at -136*sum(a).
// Partial tiles meet in LDS (double-buffered, one barrier per unit); wave
// ks < 4 of a row group finishes output rows 4*kq + ks of the unit.
//
// Issue economy decides the speed of this kernel: per unit a wave should
// issue little beyond its weight and scale loads, 16 dequant groups and the
// MFMAs.  Every weight or scale address is a lane-constant 32-bit offset,
// computed once, on top of a wave-uniform base that the scalar unit advances
// (the global_load saddr form); a slot descriptor is one s_load_dwordx4 per
// slot change.  Weights are prefetched kDepth-1 units ahead through kDepth
// register buffers, issued unconditionally (clamped to the last unit of the
// range) so the in-order vmcnt accounting keeps all newer buffers in flight.
//
// Modes:
//   kModeLinear : y = x . dequant(W)^T, bf16 out                 (fused/quantization.py:154-165)
//   kModeGateUp : h = silu(x.Wg^T) * (x.Wu^T), bf16, interleaved   (reference/fused_ops.py:170-171)
//   kModeDown   : y = route_weight * (h . Wd^T), fp32             (fused/quantization.py:196-199)
#include "kernels.h"

namespace dflash {
namespace {

// One unit's weights and scales for one wave, as loaded (converted when used,
// so no instruction waits on a load before the unit is computed).
template <int kKBPW, typename ScaleT>
struct WeightBuf {
  static constexpr int kScaleWords = (kKBPW * static_cast<int>(sizeof(ScaleT)) + 3) / 4;
  uint4 w[2][kKBPW];
  uint32_t s[2][kScaleWords];
};

// The wave's kKBPW group scales (group 128) of one weight row: element kb at
// src[kb * stride] (stride 1 in portable rows, 16 in the tiled layout); bf16
// pairs share one word, k-block 0 in the low half.
template <int kKBPW, typename ScaleT>
__device__ __forceinline__ void load_scales(uint32_t* dst, const ScaleT* src, int stride) {
  if constexpr (sizeof(ScaleT) == 2 && kKBPW == 2) {
    dst[0] = load_scale_bits(src) | (load_scale_bits(src + stride) << 16);
  } else if constexpr (kKBPW == 2) {
    dst[0] = load_scale_bits(src);
    dst[1] = load_scale_bits(src + stride);
  } else {
    dst[0] = load_scale_bits(src);
  }
}

template <int kKBPW, typename ScaleT>
__device__ __forceinline__ float scale_of(const uint32_t* w, int kb) {
  if constexpr (sizeof(ScaleT) == 2) return __uint_as_float(kb == 0 ? w[0] << 16 : w[0] & 0xFFFF0000u);
  else return __uint_as_float(w[kb]);
}

template <int kMT, int kKBPW>
struct ActRegs {
  uint4 a[kMT][kKBPW][4];
  float xn[kMT][kKBPW][4];
  float wgt[kMT][4];  // kModeDown: routing (or shared-gate) weight of output rows 4*kq + e
};

template <int kMT>
struct RedBuf {
  f32x4 v[2][8][2][kMT][64];  // [buffer][wave][tile][token tile][lane]
};

// Slot descriptor: expert (-1 shared), segment start, rows, first pass, end pass.
struct SlotDesc {
  int e, seg, M, pass0, pass_end;
};

template <int kMode, int kMT>
__device__ __forceinline__ SlotDesc load_slot(const W4StreamParams& p, int slot, int total_passes) {
  SlotDesc d;
  if (kMode == kModeLinear) {
    d.e = 0;
    d.seg = 0;
    d.M = p.M;
    d.pass0 = 0;
    d.pass_end = total_passes;
    return d;
  }
  const int4 v = ld_const_int4(p.slot_table, slot);
  d.e = v.x;
  d.seg = v.y;
  d.M = v.z;
  d.pass0 = v.w;
  d.pass_end = v.w + (v.z + 16 * kMT - 1) / (16 * kMT);
  return d;
}

// Activation row of slot row m (tv = token of that row for gate/up).
template <int kMode>
__device__ __forceinline__ int act_row(const W4StreamParams& p, const SlotDesc& sd, int tv, int m) {
  if (kMode == kModeGateUp) return sd.e < 0 ? m : tv;
  if (kMode == kModeDown) return sd.e < 0 ? p.T * p.top_k + m : sd.seg + m;
  return m;
}

// Activations of one pass: A operand rows (lane row lr), the -136*sum terms and
// the routing weights of output rows 4*kq+e.  Indirections first, then data.
template <int kMode, int kMT, int kKBPW>
__device__ __forceinline__ void load_act(ActRegs<kMT, kKBPW>& A, const W4StreamParams& p, const SlotDesc& sd,
                                         int m0, int ks, int lr, int kq) {
  const int K = p.K, nkb = K >> 7;
  constexpr int kParts = kMode == kModeDown ? 8 : 1;  // h: 8 partials of 16 columns per block; x: 1
  const bool shared = sd.e < 0;
  int ta[kMT], td[kMT][4];
  float wd[kMT][4];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    const int m = min(m0 + mt * 16 + lr, sd.M - 1);
    ta[mt] = kMode == kModeGateUp ? p.tok[shared ? 0 : sd.seg + m] : 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int md = min(m0 + mt * 16 + 4 * kq + e, sd.M - 1);
      td[mt][e] = kMode == kModeGateUp ? p.tok[shared ? 0 : sd.seg + md] : 0;
      wd[mt][e] = kMode == kModeDown ? (shared ? p.shared_gate[md] : p.slot_w[sd.seg + md]) : 0.f;
    }
  }
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    const int arow = act_row<kMode>(p, sd, ta[mt], min(m0 + mt * 16 + lr, sd.M - 1));
    const uint16_t* ap = p.act + static_cast<int64_t>(arow) * K + ks * kKBPW * 128 + kq * 32;
#pragma unroll
    for (int kb = 0; kb < kKBPW; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) A.a[mt][kb][j] = *reinterpret_cast<const uint4*>(ap + kb * 128 + j * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int md = min(m0 + mt * 16 + 4 * kq + e, sd.M - 1);
      const int drow = act_row<kMode>(p, sd, td[mt][e], md);
      const float* np = p.act_neg + static_cast<int64_t>(drow) * nkb * kParts + ks * kKBPW * kParts;
#pragma unroll
      for (int kb = 0; kb < kKBPW; ++kb) {
        float v = 0.f;
#pragma unroll
        for (int c = 0; c < kParts; ++c) v += np[kb * kParts + c];
        A.xn[mt][kb][e] = v;
      }
      if (kMode == kModeDown) A.wgt[mt][e] = wd[mt][e];
    }
  }
}

template <int kMT, int kKBPW, typename ScaleT>
__device__ __forceinline__ void compute_unit(const WeightBuf<kKBPW, ScaleT>& b, const ActRegs<kMT, kKBPW>& A, int rows_left,
                                             f32x4 (&out)[2][kMT][64]) {
  const int lane = lane_id();
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 tot[2][kMT];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) tot[0][mt] = tot[1][mt] = zero;
#pragma unroll
  for (int kb = 0; kb < kKBPW; ++kb) {
    f32x4 acc[2][kMT];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
      const f32x4 start = {A.xn[mt][kb][0], A.xn[mt][kb][1], A.xn[mt][kb][2], A.xn[mt][kb][3]};
      acc[0][mt] = acc[1][mt] = start;
    }
    const uint32_t w0[4] = {b.w[0][kb].x, b.w[0][kb].y, b.w[0][kb].z, b.w[0][kb].w};
    const uint32_t w1[4] = {b.w[1][kb].x, b.w[1][kb].y, b.w[1][kb].z, b.w[1][kb].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 d0 = dequant8(w0[j]);
      const uint4 d1 = dequant8(w1[j]);
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) {
        if (kMT == 1 || mt * 16 < rows_left) {
          acc[0][mt] = mfma16x16x32(A.a[mt][kb][j], d0, acc[0][mt]);
          acc[1][mt] = mfma16x16x32(A.a[mt][kb][j], d1, acc[1][mt]);
        }
      }
    }
    const float s0 = scale_of<kKBPW, ScaleT>(b.s[0], kb), s1 = scale_of<kKBPW, ScaleT>(b.s[1], kb);
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
      tot[0][mt] += s0 * acc[0][mt];
      tot[1][mt] += s1 * acc[1][mt];
    }
  }
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
    out[0][mt][lane] = tot[0][mt];
    out[1][mt][lane] = tot[1][mt];
  }
}

// Register buffers in the weight pipeline.  A unit holds 2*kKBPW 16-byte
// loads per lane; deeper pipelines keep more bytes in flight per CU, bounded
// by the VGPR budget of two waves per SIMD (the activations of kMT token
// tiles take the rest).
constexpr int stream_depth(int kbpw, int) { return kbpw == 1 ? 4 : 3; }

}  // namespace

template <int kMode, int kMT, int kKBPW, typename ScaleT>
__global__ __launch_bounds__(512) void w4_stream_kernel(W4StreamParams p) {
  __shared__ RedBuf<kMT> red;
  // the wave index is uniform: keep it (and all that derives from it) scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int nkb = p.K >> 7;                // k-blocks of 128 columns = scale groups per row
  const int S = nkb / kKBPW, RG = 8 / S;  // S in {4, 8}: one k-split wave per output phase e < 4
  const int rg = wave / S, ks = wave - rg * S;

  const int total_passes = kMode == kModeLinear ? (p.M + 16 * kMT - 1) / (16 * kMT) : ld_const(p.meta, 1);
  const int64_t total_units = static_cast<int64_t>(total_passes) * p.strips;
  const int u_begin = static_cast<int>(total_units * blockIdx.x / gridDim.x);
  const int u_end = static_cast<int>(total_units * (blockIdx.x + 1) / gridDim.x);
  if (u_begin >= u_end) return;
  // units in flight: kDepth - 1 prefetched while one is computed
  constexpr int kDepth = stream_depth(kKBPW, kMT);

  // ---- geometry: lane-constant 32-bit offsets, uniform strides
  const int64_t rb = p.K >> 1;  // packed bytes per weight row
  constexpr int kTileRows = kMode == kModeGateUp ? 16 : 32;  // weight rows of one row group per strip
  const int strip_rows = kTileRows * RG;
  const int64_t second = kMode == kModeGateUp ? (p.N >> 1) : 16;  // row distance of the second tile
  const int64_t w_second = second * rb, s_second = second * nkb;
  const int64_t w_strip = strip_rows * rb, s_strip = static_cast<int64_t>(strip_rows) * nkb;
  const int64_t w_first = rg * kTileRows * rb, s_first = static_cast<int64_t>(rg) * kTileRows * nkb;
  // lane offsets and k-block strides: portable rows, or the tiled layout's kilobyte per
  // 16-row tile and k-block (scales [tile][group][16]); tile bases agree in both
  const uint32_t wkb = p.tiled ? 1024u : 64u;
  const uint32_t wlane = p.tiled ? static_cast<uint32_t>(lane * 16 + ks * kKBPW * 1024)
                                 : static_cast<uint32_t>(lr * (p.K >> 1) + ks * kKBPW * 64 + kq * 16);
  const int skb = p.tiled ? 16 : 1;
  const uint32_t slane = static_cast<uint32_t>((p.tiled ? ks * kKBPW * 16 + lr : lr * nkb + ks * kKBPW) *
                                               static_cast<int>(sizeof(ScaleT)));

  // ---- load stream: uniform cursor and row pointers (tile 0 of the wave's row group)
  int l_u = u_begin;
  int l_P = l_u / p.strips, l_strip = l_u - l_P * p.strips;
  int l_slot = kMode == kModeLinear ? 0 : ld_const(p.pass_slot, l_P);
  SlotDesc ld = load_slot<kMode, kMT>(p, l_slot, total_passes);
  const uint8_t* l_w;  // weights of the current unit
  const uint8_t* l_s;  // scales of the current unit (bytes)
  auto slot_bases = [&](const SlotDesc& d) {
    const bool shared = kMode != kModeLinear && d.e < 0;
    const int64_t e = kMode == kModeLinear ? 0 : d.e;
    l_w = (shared ? p.w_shared : p.w + e * p.w_stride) + w_first;
    l_s = static_cast<const uint8_t*>(shared ? p.s_shared : static_cast<const void*>(static_cast<const ScaleT*>(p.s) + e * p.s_stride)) +
          s_first * static_cast<int64_t>(sizeof(ScaleT));
  };
  slot_bases(ld);
  l_w += l_strip * w_strip;
  l_s += l_strip * s_strip * static_cast<int64_t>(sizeof(ScaleT));

  auto issue = [&](WeightBuf<kKBPW, ScaleT>& b) {
#pragma unroll
    for (int kb = 0; kb < kKBPW; ++kb) {
      b.w[0][kb] = *reinterpret_cast<const uint4*>(l_w + wlane + kb * wkb);
      b.w[1][kb] = *reinterpret_cast<const uint4*>(l_w + w_second + wlane + kb * wkb);
    }
    load_scales<kKBPW, ScaleT>(b.s[0], reinterpret_cast<const ScaleT*>(l_s + slane), skb);
    load_scales<kKBPW, ScaleT>(b.s[1], reinterpret_cast<const ScaleT*>(l_s + s_second * sizeof(ScaleT) + slane), skb);
    // advance to the next unit of the range (the last one repeats: padding loads)
    if (l_u + 1 < u_end) {
      ++l_u;
      l_w += w_strip;
      l_s += s_strip * sizeof(ScaleT);
      if (++l_strip == p.strips) {
        l_strip = 0;
        ++l_P;
        if (kMode != kModeLinear && l_P == ld.pass_end) ld = load_slot<kMode, kMT>(p, ++l_slot, total_passes);
        slot_bases(ld);
      }
    }
  };

  WeightBuf<kKBPW, ScaleT> wb[kDepth];
#pragma unroll
  for (int i = 0; i + 1 < kDepth; ++i) issue(wb[i]);

  // ---- compute stream
  int c_P = u_begin / p.strips, c_strip = u_begin - c_P * p.strips;
  int c_slot = kMode == kModeLinear ? 0 : ld_const(p.pass_slot, c_P);
  SlotDesc cd = load_slot<kMode, kMT>(p, c_slot, total_passes);
  ActRegs<kMT, kKBPW> A;
  int act_pass = -1, m0 = 0, buf = 0;
  const int inter = p.N >> 1;

  auto step = [&](int u, WeightBuf<kKBPW, ScaleT>& cur, WeightBuf<kKBPW, ScaleT>& refill) {
    issue(refill);
    const bool live = u < u_end;  // workgroup-uniform; padding steps keep the pipeline shape only
    if (live) {
      if (c_P != act_pass) {
        m0 = (c_P - cd.pass0) * 16 * kMT;
        load_act<kMode, kMT, kKBPW>(A, p, cd, m0, ks, lr, kq);
        wait_vmem();
        act_pass = c_P;
      }
      compute_unit<kMT, kKBPW, ScaleT>(cur, A, cd.M - m0, red.v[buf][wave]);
    }
    lds_barrier();  // partial sums are in LDS; the prefetched units' loads stay in flight
    if (live) {
      const int colblock = c_strip * RG + rg;
      const int row0 = colblock * kTileRows;
      const bool shared = kMode != kModeLinear && cd.e < 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (e != ks) continue;
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt) {
          float v0 = 0.f, v1 = 0.f;
          for (int q = 0; q < S; ++q) {
            const f32x4 t0 = red.v[buf][rg * S + q][0][mt][lane];
            const f32x4 t1 = red.v[buf][rg * S + q][1][mt][lane];
            v0 += t0[e];
            v1 += t1[e];
          }
          const int m = m0 + mt * 16 + 4 * kq + e;
          const bool valid = m < cd.M;
          if (kMode == kModeLinear) {
            if (valid && p.out_f32) {  // fp32 output: the unrounded sums
              float* o = p.out_f32 + static_cast<int64_t>(m) * p.N + row0 + lr;
              o[0] = v0;
              o[second] = v1;
            } else if (valid) {
              uint16_t* o = p.out_bf16 + static_cast<int64_t>(m) * p.N + row0 + lr;
              o[0] = f32_to_bf16(v0);
              o[second] = f32_to_bf16(v1);
            }
          } else if (kMode == kModeGateUp) {
            const uint16_t hb = f32_to_bf16(silu(v0) * v1);
            const int hrow = shared ? p.T * p.top_k + m : cd.seg + m;
            if (valid) p.out_bf16[static_cast<int64_t>(hrow) * inter + octet_slot(row0 + lr)] = hb;
            const float part = row16_sum(valid ? bf16_to_f32(hb) : 0.f);
            if (valid && lr == 0)
              p.out_part[static_cast<int64_t>(hrow) * (inter >> 4) + colblock] = -kDequantOffset * part;
          } else {
            if (valid) {
              const float wgt = A.wgt[mt][e];
              const int yrow = shared ? p.T * p.top_k + m : cd.seg + m;
              float* o = p.out_f32 + static_cast<int64_t>(yrow) * p.N + row0 + lr;
              o[0] = v0 * wgt;
              o[second] = v1 * wgt;
            }
          }
        }
      }
      // advance the compute cursor
      if (++c_strip == p.strips) {
        c_strip = 0;
        ++c_P;
        if (kMode != kModeLinear && c_P == cd.pass_end && c_P < total_passes)
          cd = load_slot<kMode, kMT>(p, ++c_slot, total_passes);
      }
    }
    buf ^= 1;
  };

  for (int u = u_begin; u < u_end; u += kDepth) {
#pragma unroll
    for (int i = 0; i < kDepth; ++i) step(u + i, wb[i], wb[(i + kDepth - 1) % kDepth]);
  }
}

bool w4_stream_supports(int K, int G) { return (K == 512 || K == 1024 || K == 2048) && G == 128; }

int w4_stream_row_groups(int K) { return K == 512 ? 2 : 1; }

void launch_w4_stream(int mode, bool fp32_scales, int mt, int grid, const W4StreamParams& p, hipStream_t stream) {
  const int kbpw = (p.K >> 7) >= 8 ? (p.K >> 7) / 8 : 1;  // K = 512 -> 1 (4-way split), else 8-way split
  const dim3 g(static_cast<unsigned>(grid)), blk(512);
#define DFLASH_STREAM(MODE, MT, KB)                                                                         \
  do {                                                                                                      \
    if (fp32_scales) hipLaunchKernelGGL((w4_stream_kernel<MODE, MT, KB, float>), g, blk, 0, stream, p);    \
    else hipLaunchKernelGGL((w4_stream_kernel<MODE, MT, KB, uint16_t>), g, blk, 0, stream, p);             \
  } while (0)
#define DFLASH_STREAM_KB(MODE, MT)             \
  switch (kbpw) {                              \
    case 1: DFLASH_STREAM(MODE, MT, 1); break; \
    default: DFLASH_STREAM(MODE, MT, 2); break; \
  }
#define DFLASH_STREAM_MT(MODE)                 \
  if (mt == 1) { DFLASH_STREAM_KB(MODE, 1) }  \
  else { DFLASH_STREAM_KB(MODE, 2) }
  switch (mode) {
    case kModeLinear: DFLASH_STREAM_MT(kModeLinear) break;
    case kModeGateUp: DFLASH_STREAM_MT(kModeGateUp) break;
    default: DFLASH_STREAM_MT(kModeDown) break;
  }
#undef DFLASH_STREAM_MT
#undef DFLASH_STREAM_KB
#undef DFLASH_STREAM
}

}  // namespace dflash
