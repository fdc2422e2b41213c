// Wave-streaming W4A16 GEMM for small token counts (the verify block, T <= 32).
//
// Every wave streams whole weight rows on its own: a unit is one pass (up to
// 16 slot rows) times one strip of 2 x 16 weight rows over the full reduction
// length K, and the wave that loads a unit finishes it.  There is no split of K
// across waves, so no partial sums meet in LDS and the main loop has no
// barrier.  The activations live in LDS instead of registers:
//   kModeGateUp / kModeLinear : all T (or M) rows of x, octet-interleaved,
//                               their -136*sum terms and the token of every
//                               routed slot row, loaded once per workgroup;
//   kModeDown                 : the h rows of the passes the workgroup covers,
//                               in chunks that fit, with their -136*sum terms
//                               and routing weights.
// Units form one list, split into equal contiguous ranges per workgroup; the
// 8 waves of a workgroup take every 8th unit of its range.
//
// Per unit a lane loads its row's group scales with two to four 16-byte loads
// (no per-group scattered loads), then streams kNKB k-blocks: two 16-byte
// weight loads per k-block (16 rows x 64 bytes each), prefetched kDepth
// k-blocks ahead across unit boundaries.  Each k-block is dequantised in
// registers (bf16 136+q), multiplied on v_mfma_f32_16x16x32_bf16 against the
// A fragments read from LDS, started from -136*sum(a) and scaled.
//
// Semantics per mode (reference citations):
//   kModeLinear : y = x . dequant(W)^T, bf16 out                 (fused/quantization.py:154-165)
//   kModeGateUp : h = silu(x.Wg^T) * (x.Wu^T), gate rows first   (reference/fused_ops.py:170-171)
//   kModeDown   : y = route_weight * (h . Wd^T), fp32            (fused/quantization.py:196-199)
#include "kernels.h"

namespace dflash {
namespace {

constexpr int kWaveLdsA = 139264;     // activation rows (row stride 2K + 16 bytes)
constexpr int kWaveLdsNeg = 2048;     // -136*sum terms, floats
constexpr int kWaveLdsTok = 2048;     // token of every routed slot row (kModeGateUp)
constexpr int kWaveLdsWgt = 512;      // routing weights of the chunk rows (kModeDown)
constexpr int kWaveLdsPass = 64;      // pass descriptors of the workgroup's range (or down chunk)

struct WaveLds {
  uint4 a[kWaveLdsA / 16];
  float neg[kWaveLdsNeg];
  int tok[kWaveLdsTok];
  float wgt[kWaveLdsWgt];
  int4 pdesc[kWaveLdsPass];
};

template <int kNKB, typename ScaleT>
struct ScaleWords {
  static constexpr int kTile = kNKB * static_cast<int>(sizeof(ScaleT)) / 4;  // 32-bit words per tile row
};

// The kNKB group scales of one weight row (group size 128).
template <int kNKB, typename ScaleT>
__device__ __forceinline__ void load_row_scales(uint32_t* dst, const uint8_t* src) {
  constexpr int kWords = ScaleWords<kNKB, ScaleT>::kTile;
  if constexpr (kWords == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(src);
    dst[0] = v.x;
    dst[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < kWords / 4; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(src + 16 * i);
      dst[4 * i] = v.x;
      dst[4 * i + 1] = v.y;
      dst[4 * i + 2] = v.z;
      dst[4 * i + 3] = v.w;
    }
  }
}

template <typename ScaleT>
__device__ __forceinline__ float row_scale(const uint32_t* words, int kb) {
  if constexpr (sizeof(ScaleT) == 2) {
    const uint32_t w = words[kb >> 1];
    return __uint_as_float((kb & 1) ? (w & 0xFFFF0000u) : (w << 16));
  } else {
    return __uint_as_float(words[kb]);
  }
}

// Opaque to the optimiser: the value must exist in registers at this point.
__device__ __forceinline__ void pin(f32x4& v) { asm volatile("" : "+v"(v)); }

// k-block prefetch distance and units per unrolled loop iteration.  Loads run
// kDepth - 1 k-blocks ahead and may cross into later units; the scale ring
// holds one slot per unit of the iteration, enough for the computed unit and
// every unit with loads in flight, and every ring index is compile-time.
template <int kNKB>
struct WavePipe {
  static constexpr int kDepth = kNKB >= 8 ? 4 : 6;
  static constexpr int kUnits = kNKB >= 8 ? 2 : 3;
  static_assert(1 + (kDepth - 1 + kNKB - 1) / kNKB <= kUnits, "scale ring too small for the prefetch distance");
  static_assert((kUnits * kNKB) % kDepth == 0, "buffer indices must be compile-time");
};

}  // namespace

template <int kMode, int kNKB, typename ScaleT>
__global__ __launch_bounds__(512) void w4_wave_kernel(W4StreamParams p) {
  __shared__ WaveLds lds;
  using Pipe = WavePipe<kNKB>;
  constexpr int kDepth = Pipe::kDepth, kUnits = Pipe::kUnits;
  constexpr int kK = kNKB * 128;
  constexpr int kRS = kK * 2 + 16;                  // LDS row stride (bytes) of an activation row
  constexpr int kSW = ScaleWords<kNKB, ScaleT>::kTile;
  constexpr int kTileRows = kMode == kModeGateUp ? 16 : 32;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int tid = threadIdx.x;

  const int total_passes = kMode == kModeLinear ? (p.M + 15) >> 4 : ld_const(p.meta, 1);
  const int strips = p.strips;
  const int64_t total_units = static_cast<int64_t>(total_passes) * strips;
  const int ub = static_cast<int>(total_units * blockIdx.x / gridDim.x);
  const int ue = static_cast<int>(total_units * (blockIdx.x + 1) / gridDim.x);
  if (ub >= ue) return;

  const int64_t rb = kK >> 1;                                          // packed bytes per weight row
  const int64_t second = kMode == kModeGateUp ? (p.N >> 1) : 16;       // row distance of tile 1
  const uint32_t wlane = static_cast<uint32_t>(lr * rb + kq * 16);     // lane offset inside a tile
  const uint32_t slane = static_cast<uint32_t>(lr * kNKB * sizeof(ScaleT));

  // Pass descriptors come from LDS once staged (a scalar load would make the
  // next LDS wait, which shares its counter, wait for it too); only the first
  // unit of a chunk, issued before the staging barrier, reads them with s_load.
  int pd_base = 0, pd_count = 0;
  auto pass_desc = [&](int P, bool staged) -> int4 {
    if (kMode == kModeLinear) return make_int4(0, 0, p.M, P * 16);
    const int i = P - pd_base;
    if (staged && i >= 0 && i < pd_count) {
      const int4 v = lds.pdesc[i];
      return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                       __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
    }
    return ld_const_int4(p.pass_table, P);
  };

  // Down processes its range in chunks whose h rows fit in LDS; the other
  // modes keep all rows of x resident and have one chunk.
  constexpr int kChunkPasses = (kWaveLdsA / kRS) / 16;
  static_assert(kMode != kModeDown || kChunkPasses >= 1, "one pass of h rows must fit");
  const int P_first = ub / strips, P_last = (ue - 1) / strips;
  const int chunk_passes = kMode == kModeDown ? kChunkPasses : P_last - P_first + 1;

  for (int Pc = P_first; Pc <= P_last; Pc += chunk_passes) {
    const int Pc_end = min(P_last + 1, Pc + chunk_passes);
    const int cb = max(ub, Pc * strips), ce = min(ue, Pc_end * strips);
    if (Pc != P_first) __syncthreads();  // every wave is done with the previous chunk's rows

    // ---- this wave's units: cb + wave + 8 t
    const int n_mine = ce - cb > wave ? (ce - cb - wave + 7) >> 3 : 0;

    // load cursor (uniform)
    int l_t = 0, l_P = -1;
    int4 l_d = make_int4(0, 0, 0, 0);
    const uint8_t* l_w = nullptr;
    const uint8_t* l_s = nullptr;
    bool staged = false;  // pass descriptors of this chunk are in LDS
    auto load_unit_bases = [&]() {
      const int u = cb + wave + 8 * l_t;
      const int P = u / strips, strip = u - P * strips;
      if (P != l_P) {
        l_P = P;
        l_d = pass_desc(P, staged);
      }
      const bool shared = kMode != kModeLinear && l_d.x < 0;
      const int64_t e = kMode == kModeLinear ? 0 : l_d.x;
      const uint8_t* wbase = shared ? p.w_shared : p.w + e * p.w_stride;
      const uint8_t* sbase = static_cast<const uint8_t*>(shared ? p.s_shared : p.s) +
                             (shared ? 0 : e * p.s_stride * static_cast<int64_t>(sizeof(ScaleT)));
      const int64_t row0 = static_cast<int64_t>(strip) * kTileRows;
      l_w = wbase + row0 * rb;
      l_s = sbase + row0 * kNKB * static_cast<int64_t>(sizeof(ScaleT));
    };

    uint4 wbuf[kDepth][2];
    uint32_t sbuf[kUnits][2][kSW];
    // issue k-block kb of the load cursor's unit; scales ride with k-block 0
    auto issue = [&](uint4 (&dst)[2], uint32_t (&sdst)[2][kSW], int kb) {
      if (kb == 0) {
        load_row_scales<kNKB, ScaleT>(sdst[0], l_s + slane);
        load_row_scales<kNKB, ScaleT>(sdst[1], l_s + second * kNKB * sizeof(ScaleT) + slane);
      }
      dst[0] = *reinterpret_cast<const uint4*>(l_w + wlane + kb * 64);
      dst[1] = *reinterpret_cast<const uint4*>(l_w + second * rb + wlane + kb * 64);
      if (kb == kNKB - 1 && l_t + 1 < n_mine) {  // past the last unit the loads repeat it (never computed)
        ++l_t;
        load_unit_bases();
      }
    };

    // prologue: the first kDepth - 1 k-blocks, in flight while the rows are staged
    if (n_mine > 0) {
      load_unit_bases();
#pragma unroll
      for (int i = 0; i + 1 < kDepth; ++i) issue(wbuf[i], sbuf[(i / kNKB) % kUnits], i % kNKB);
    }

    // descriptors of the passes this chunk covers
    pd_base = Pc;
    pd_count = min(Pc_end - Pc, kWaveLdsPass);
    if (kMode != kModeLinear && tid < pd_count) lds.pdesc[tid] = p.pass_table[Pc + tid];

    if (kMode != kModeDown && Pc == P_first) {
      // x rows (octet-interleaved), their -136*sum terms, the token of every
      // routed slot row.  Loads are issued in batches (clamped indices), then
      // written to LDS, so a batch costs one memory latency.
      const int rows = kMode == kModeLinear ? p.M : p.T;
      const int total = rows * (kK / 8);
      const uint4* src = reinterpret_cast<const uint4*>(p.act);
      for (int c0 = 0; c0 < total; c0 += 8 * 512) {
        uint4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = src[min(c0 + i * 512 + tid, total - 1)];
        float ng[4];
        int tk[4];
        if (c0 == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ng[i] = p.act_neg[min(i * 512 + tid, rows * kNKB - 1)];
            if (kMode == kModeGateUp) tk[i] = p.tok[min(i * 512 + tid, p.T * p.top_k - 1)];
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = c0 + i * 512 + tid;
          if (c < total) {
            const int r = c / (kK / 8), cc = c - r * (kK / 8);
            lds.a[(r * kRS) / 16 + cc] = v[i];
          }
        }
        if (c0 == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (i * 512 + tid < rows * kNKB) lds.neg[i * 512 + tid] = ng[i];
            if (kMode == kModeGateUp && i * 512 + tid < p.T * p.top_k) lds.tok[i * 512 + tid] = tk[i];
          }
        }
      }
    }
    if (kMode == kModeDown) {
      // per pass of the chunk: its 16 h rows (clamped to the slot), -136*sum
      // terms (8 partials of 16 columns per k-block) and routing weights; every
      // load of the chunk is issued before the first LDS write
      const int npass = Pc_end - Pc;
      constexpr int kPer = kK / 256;  // 16-byte chunks per thread per pass (16 rows x K/8 chunks / 512)
      uint4 hv[kChunkPasses][kPer];
      float4 nu[kChunkPasses], nv[kChunkPasses];
      float wg[kChunkPasses];
      const int nr = min(tid / kNKB, 15), nkb = tid - (tid / kNKB) * kNKB;  // -136*sum term of this thread
      const int wr = min(tid, 15);
#pragma unroll
      for (int i = 0; i < kChunkPasses; ++i) {
        const int4 d = ld_const_int4(p.pass_table, Pc + min(i, npass - 1));
        const int base = d.x < 0 ? p.T * p.top_k : d.y;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int c = j * 512 + tid;
          const int r = c / (kK / 8), cc = c - r * (kK / 8);
          const int row = base + min(d.w + r, d.z - 1);
          hv[i][j] = reinterpret_cast<const uint4*>(p.act)[static_cast<int64_t>(row) * (kK / 8) + cc];
        }
        const int nrow = base + min(d.w + nr, d.z - 1);
        const float4* ns = reinterpret_cast<const float4*>(p.act_neg + (static_cast<int64_t>(nrow) * kNKB + nkb) * 8);
        nu[i] = ns[0];
        nv[i] = ns[1];
        const int m = min(d.w + wr, d.z - 1);
        wg[i] = d.x < 0 ? p.shared_gate[m] : p.slot_w[d.y + m];
      }
#pragma unroll
      for (int i = 0; i < kChunkPasses; ++i) {
        if (i < npass) {
#pragma unroll
          for (int j = 0; j < kPer; ++j) {
            const int c = j * 512 + tid;
            const int r = c / (kK / 8), cc = c - r * (kK / 8);
            lds.a[((i * 16 + r) * kRS) / 16 + cc] = hv[i][j];
          }
          if (tid < 16 * kNKB)
            lds.neg[(i * 16 + nr) * kNKB + nkb] =
                ((nu[i].x + nu[i].y) + (nu[i].z + nu[i].w)) + ((nv[i].x + nv[i].y) + (nv[i].z + nv[i].w));
          if (tid < 16) lds.wgt[i * 16 + tid] = wg[i];
        }
      }
    }
    __syncthreads();
    staged = true;
    if (n_mine == 0) continue;

    // compute state
    int c_P = -1;
    int4 c_d = make_int4(0, 0, 0, 0);
    int a_off = 0;      // LDS byte offset of this lane's A row (+ k-octet)
    int n_idx[4];       // LDS float index of the -136*sum row of output rows 4kq+e
    float wgt[4];
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 tot0 = zero, tot1 = zero;
    int strip = 0;

    for (int t0 = 0; t0 < n_mine; t0 += kUnits) {
#pragma clang loop unroll(full)
      for (int step = 0; step < kUnits * kNKB; ++step) {
        const int ui = step / kNKB, kb = step % kNKB;
        // keep the pipeline kDepth - 1 k-blocks ahead
        const int ls = step + kDepth - 1;  // step index of the load
        issue(wbuf[ls % kDepth], sbuf[(ls / kNKB) % kUnits], ls % kNKB);
        const int t = t0 + ui;
        if (t < n_mine) {
          if (kb == 0) {
            const int u = cb + wave + 8 * t;
            const int P = u / strips;
            strip = u - P * strips;
            if (P != c_P) {
              c_P = P;
              c_d = pass_desc(P, true);
            }
            const int M = c_d.z, m0 = c_d.w;
            const int ma = min(m0 + lr, M - 1);
            int arow;
            if (kMode == kModeGateUp) arow = c_d.x < 0 ? ma : lds.tok[c_d.y + ma];
            else if (kMode == kModeLinear) arow = ma;
            else arow = (P - Pc) * 16 + lr;
            a_off = arow * kRS + kq * 64;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int me = min(m0 + 4 * kq + e, M - 1);
              int nrow;
              if (kMode == kModeGateUp) nrow = c_d.x < 0 ? me : lds.tok[c_d.y + me];
              else if (kMode == kModeLinear) nrow = me;
              else nrow = (P - Pc) * 16 + 4 * kq + e;
              n_idx[e] = nrow * kNKB;
              if (kMode == kModeDown) wgt[e] = lds.wgt[nrow];
            }
            tot0 = zero;
            tot1 = zero;
          }
          // k-block kb of the unit
          const uint8_t* ab = reinterpret_cast<const uint8_t*>(lds.a) + a_off + kb * 256;
          uint4 a[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const uint4*>(ab + 16 * j);
          const f32x4 start = {lds.neg[n_idx[0] + kb], lds.neg[n_idx[1] + kb], lds.neg[n_idx[2] + kb],
                               lds.neg[n_idx[3] + kb]};
          const uint4 (&w)[2] = wbuf[step % kDepth];
          const uint32_t w0[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
          const uint32_t w1[4] = {w[1].x, w[1].y, w[1].z, w[1].w};
          f32x4 acc0 = start, acc1 = start;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc0 = mfma16x16x32(a[j], dequant8(w0[j]), acc0);
            acc1 = mfma16x16x32(a[j], dequant8(w1[j]), acc1);
          }
          const uint32_t (&sw)[2][kSW] = sbuf[ui % kUnits];
          tot0 += row_scale<ScaleT>(sw[0], kb) * acc0;
          tot1 += row_scale<ScaleT>(sw[1], kb) * acc1;
          // materialise the running sums here: left alone, the compiler sinks all
          // kNKB scale-accumulates to the unit's end and keeps every k-block's
          // MFMA result live until then
          pin(tot0);
          pin(tot1);

          if (kb == kNKB - 1) {
            // epilogue: lane holds rows m0 + 4kq + e of columns lr of both tiles
            const int M = c_d.z, m0 = c_d.w;
            const bool shared = kMode != kModeLinear && c_d.x < 0;
            const int row0 = strip * kTileRows;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int m = m0 + 4 * kq + e;
              const bool valid = m < M;
              if (kMode == kModeLinear) {
                if (valid) {
                  uint16_t* o = p.out_bf16 + static_cast<int64_t>(m) * p.N + row0 + lr;
                  o[0] = f32_to_bf16(tot0[e]);
                  o[16] = f32_to_bf16(tot1[e]);
                }
              } else if (kMode == kModeGateUp) {
                const int inter = p.N >> 1;
                const uint16_t hb = f32_to_bf16(silu(tot0[e]) * tot1[e]);
                const int hrow = shared ? p.T * p.top_k + m : c_d.y + m;
                if (valid) p.out_bf16[static_cast<int64_t>(hrow) * inter + octet_slot(row0 + lr)] = hb;
                const float part = row16_sum(valid ? bf16_to_f32(hb) : 0.f);
                if (valid && lr == 0)
                  p.out_part[static_cast<int64_t>(hrow) * (inter >> 4) + strip] = -kDequantOffset * part;
              } else {
                if (valid) {
                  const int yrow = shared ? p.T * p.top_k + m : c_d.y + m;
                  float* o = p.out_f32 + static_cast<int64_t>(yrow) * p.N + row0 + lr;
                  o[0] = tot0[e] * wgt[e];
                  o[16] = tot1[e] * wgt[e];
                }
              }
            }
          }
        }
        // keep the scheduler from hoisting later k-blocks' LDS reads and
        // dequantisation into this one (register pressure, not latency, binds)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

bool w4_wave_supports(int mode, int K, int G, int rows) {
  if (G != 128 || (K != 512 && K != 1024 && K != 2048)) return false;
  const int rs = K * 2 + 16;
  if (mode == kModeDown) return (kWaveLdsA / rs) >= 16;
  return rows > 0 && rows * rs <= kWaveLdsA && rows * (K / 128) <= kWaveLdsNeg;
}

void launch_w4_wave(int mode, bool fp32_scales, int grid, const W4StreamParams& p, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid)), blk(512);
#define DFLASH_WAVE(MODE, NKB)                                                                          \
  do {                                                                                                  \
    if (fp32_scales) hipLaunchKernelGGL((w4_wave_kernel<MODE, NKB, float>), g, blk, 0, stream, p);     \
    else hipLaunchKernelGGL((w4_wave_kernel<MODE, NKB, uint16_t>), g, blk, 0, stream, p);              \
  } while (0)
#define DFLASH_WAVE_K(MODE)                      \
  switch (p.K) {                                 \
    case 512: DFLASH_WAVE(MODE, 4); break;       \
    case 1024: DFLASH_WAVE(MODE, 8); break;      \
    default: DFLASH_WAVE(MODE, 16); break;       \
  }
  switch (mode) {
    case kModeLinear: DFLASH_WAVE_K(kModeLinear) break;
    case kModeGateUp: DFLASH_WAVE_K(kModeGateUp) break;
    default: DFLASH_WAVE_K(kModeDown) break;
  }
#undef DFLASH_WAVE_K
#undef DFLASH_WAVE
}

}  // namespace dflash
