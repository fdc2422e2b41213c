// LDS-tiled grouped W4A16 GEMM for long prefill (many rows per expert).
//
// A work tile is one pass (up to 96 rows of one slot: an expert segment or
// the shared expert) times one column tile of 512 outputs; persistent
// workgroups (one per CU, 8 waves, 64 columns each) take tiles from a queue,
// longest passes first (the routing writes the routed passes in descending
// order of 16-row subtiles).  The tiles left over after the last full round of
// the grid run in pieces, so that final round spreads over more workgroups:
// four per tile (two half-width column pieces of 8 waves x 32 columns, each
// over the first and the second half of the pass's subtiles) when they fill at
// most a quarter of the grid, else two half-width pieces when at most half.
// Per 128-column k-block of the reduction:
//   * every operand reaches LDS by direct-to-LDS buffer loads (no register
//     staging): the pass's activation rows in MFMA fragment order (1 KB
//     blocks, one per 16-row subtile and 32-k step) and their -136*sum terms,
//     two stages, one k-block ahead; each wave's own weight fragments (16
//     columns x 128 k, 16 bytes per lane) and their group scales, three
//     stages, two k-blocks ahead.  Every stage is its own LDS array.  One
//     barrier per k-block publishes the activation stage; a wave reads its
//     weight stages after counted waits of its own (the compiler's waits for
//     direct-to-LDS loads are not relied on: it can drop them across loop
//     iterations).
//   * the weights are dequantised once per wave to bf16 (136 + q), exact, with
//     8 VALU operations per 8 weights, and each dequantised word feeds one
//     v_mfma_f32_16x16x32_bf16 per 16-row subtile;
//   * the MFMAs accumulate straight into u = sum_kb' s_kb' acc_kb' / s_kb, the
//     running sum in units of the current group scale: at each k-block u is
//     rescaled by s_prev / s_kb and offset by -136*sum(a) in one FMA, so no
//     per-k-block accumulator set is held; the tile ends with tot = u * s_last.
//     Group scales are clamped to |s| >= 2^-64 (a zero group adds nothing
//     either way) so the ratios stay finite.
// The k-loop is specialised on the pass's subtile count, so a k-step is one
// straight-line block: while its MFMAs run the wave refills each subtile's A
// fragment for the next k-step right after the subtile's last MFMA and
// dequantises the next k-step's weights; the last k-step also reads and
// dequantises the next k-block's weights.
//
// Modes (reference citations):
//   kModeGateUp : h = silu(x.Wg^T) * (x.Wu^T), bf16, octet-interleaved, and its
//                 -136*sum per 128 columns for the down GEMM        (reference/fused_ops.py:170-171)
//   kModeDown   : y = route_weight * (h . Wd^T), rounded to bf16   (fused/quantization.py:196-199)
#include <type_traits>

#include "kernels.h"

namespace dflash {
namespace {

constexpr int kTileM = 96;                  // rows per pass (6 subtiles of 16)

// Per-tile times of the profiling build (DFLASH_TIMELINE, loaded only by timeline.py): per
// launch mode (gate/up, down), workgroup and its first 8 tiles, s_memrealtime ticks (100 MHz)
// at the tile's start and end and the tile's rows | pass << 16 | (order + 1) << 40 | half << 56
// (1 for a piece of a split tile; rows are the whole pass's).
#ifdef DFLASH_TIMELINE
constexpr int kTlWorkgroups = 1024, kTlTiles = 8, kWavesTl = 8;
__device__ unsigned long long g_timeline_tile[2 * kTlWorkgroups * kTlTiles * 3];
// Per launch mode, workgroup, its first 8 items and wave, in s_memtime cycles: the item's
// set-up in three parts (pass entry loaded; the barrier, which also waits for the row id
// loads and the previous item's stores; the first stage loads and weight reads), the k-loop,
// the epilogue (to the issue of its last store), and 1 (a written slot).
constexpr int kTlCycleFields = 6;
__device__ unsigned long long g_timeline_tile_cycles[2 * kTlWorkgroups * kTlTiles * kWavesTl * kTlCycleFields];
#endif
constexpr int kMaxSub = kTileM / 16;
constexpr int kWaves = 8;
constexpr int kTileN = kWaves * 64;         // output columns per tile
constexpr int kBlocks = kMaxSub * 4;        // activation fragment blocks per stage (subtile x k-step), 1 KB each
constexpr int kAStages = 2, kWStages = 3;

typedef __attribute__((address_space(3))) void* lds_ptr;

template <int N>
using Idx = std::integral_constant<int, N>;

// The stages, each a separate __shared__ array of the kernel.
struct TileLds {
  uint4* a[kAStages];       // [kBlocks][64 lanes] activation fragments
  float* neg[kAStages];     // [128] -136*sum of each row's k-block (rows past the pass repeat the last)
  uint4* w[kWStages];       // [kWaves][4 fragments][64 lanes] packed weights
  uint32_t* s[kWStages];    // [kWaves][4 fragments x 16 columns] raw scale bits
  float* wgt;               // [128] down: each pass row's routing weight (or shared-expert gate)
};

// Per-tile state shared by the subtile-count specialisations.
struct TileCtx {
  int4 d;                   // expert (-1 shared), segment start, slot rows, first row of the pass
  bool shared;
  int rows, nt;
  buf_rsrc wrs, srs, ars, nrs;  // the slot's weights and scales, activations, their -136*sum terms
  uint32_t woff[4];         // byte offset of this lane's 16 bytes of each weight fragment (k-block 0)
  uint32_t wkb;             // k-block stride of the weights: 64 (portable rows) or 1024 (tiled blocks)
  uint32_t soff;            // byte offset of the scale row this lane loads (fragment lane >> 4, column lane & 15)
  uint32_t aoff[3];         // byte offset of this lane's 16 bytes of activation blocks wave, wave + 8, wave + 16
  uint32_t noff;            // byte offset of the -136*sum terms of row 64 * wave + lane
  buf_rsrc grs;             // down: the pass rows' routing weights (or shared-expert gates)
  uint32_t goff;            // byte offset of the weight of row 64 * wave + lane
#ifdef DFLASH_TIMELINE
  unsigned long long t_start, t_ctx, t_sync;  // s_memtime at the start of the work item, its ids loaded, after its barrier
  unsigned long long* tl_cyc;  // this workgroup's and item's slots (null past the first 1024 workgroups)
#endif
};

__device__ __forceinline__ void dma16(buf_rsrc r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, static_cast<int>(voff), static_cast<int>(soff), 0, 0);
}
__device__ __forceinline__ void dma4(buf_rsrc r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 4, static_cast<int>(voff), static_cast<int>(soff), 0, 0);
}

// Workgroup barrier publishing this wave's direct-to-LDS loads older than its
// newest kPending ones.  __syncthreads() would not do: its release fence counts
// every load still headed for LDS as a pending LDS write and waits for all of
// them.  The empty asm statements keep the compiler from moving memory
// accesses across the barrier.
template <int kPending>
__device__ __forceinline__ void dma_barrier() {
  static_assert(kPending < 16, "vmcnt field");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | kPending);  // vmcnt(kPending) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait until at most kPending of this wave's memory loads are outstanding (no barrier)
template <int kPending>
__device__ __forceinline__ void dma_wait() {
  static_assert(kPending < 16, "vmcnt field");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70 | kPending);  // vmcnt(kPending)
  asm volatile("" ::: "memory");
}

// scheduling-group masks of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedValu = 0x002, kSchedMfma = 0x008, kSchedDsRead = 0x100;

// Instruction order of one k-step's scheduling region: kLead VALU operations,
// then kMfma x (1 MFMA, kValu VALU operations), with one LDS read after every
// kDsEvery MFMAs, so the VALU work issues while the MFMAs run.
template <int kLead, int kMfma, int kValu, int kDsEvery>
__device__ __forceinline__ void interleave() {
  if (kLead) __builtin_amdgcn_sched_group_barrier(kSchedValu, kLead, 0);
#pragma unroll
  for (int i = 0; i < kMfma; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedValu, kValu, 0);
    if ((i + 1) % kDsEvery == 0) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
  }
}

// NF: 16-column weight fragments per wave (4: a 512-column tile; 2: a half-width piece).
template <int kMode, typename ScaleT, int NSUB, int NF>
__device__ __forceinline__ void tile_pass(const W4StreamParams& p, const TileLds& lds, const TileCtx& c) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int nkb = p.K >> 7, gshift = p.G == 256 ? 1 : 0;
  const int inter = p.N >> 1;

  // loads of k-block kb (clamped: past the end they repeat the last k-block into a stage never read)
  auto load_a = [&](int kb, auto sa) {
    kb = min(kb, nkb - 1);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int b = wave + kWaves * i;
      if (b < NSUB * 4) dma16(c.ars, lds.a[sa] + b * 64, c.aoff[i], kb * 256);
    }
    if (wave * 64 < NSUB * 16) dma4(c.nrs, lds.neg[sa] + wave * 64, c.noff, kb * 4);
  };
  auto load_w = [&](int kb, auto sw) {
    kb = min(kb, nkb - 1);
#pragma unroll
    for (int f = 0; f < NF; ++f) dma16(c.wrs, lds.w[sw] + (wave * 4 + f) * 64, c.woff[f], kb * c.wkb);
    const int g = kb >> gshift;
    // portable: the 4 bytes at the lane's row and group (pair); tiled: the group's 16-column
    // chunk at the lane's even column (a bf16 lane takes its half below)
    dma4(c.srs, lds.s[sw] + wave * 64, c.soff,
         p.tiled ? g * 16 * static_cast<int>(sizeof(ScaleT)) : (sizeof(ScaleT) == 4 ? g * 4 : (g & ~1) * 2));
  };
  // this lane's weights and group scales of k-block kb from stage sw
  auto read_w = [&](uint4 (&wf)[NF], float (&sc)[NF], int kb, auto sw) {
    const int g = kb >> gshift;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      wf[f] = lds.w[sw][(wave * 4 + f) * 64 + lane];
      const uint32_t bits = lds.s[sw][wave * 64 + f * 16 + lr];
      const bool hi = p.tiled ? (lr & 1) : (g & 1);
      float v = sizeof(ScaleT) == 4 ? __uint_as_float(bits) : __uint_as_float((hi ? bits >> 16 : bits & 0xFFFFu) << 16);
      if (__builtin_fabsf(v) < 0x1p-64f) v = __builtin_copysignf(0x1p-64f, v);  // NaN passes through
      sc[f] = v;
    }
  };
  auto word = [](const uint4& w, int j) { return j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w; };

  // prologue: weights of k-blocks 0 and 1, activations of k-block 0 (the empty asm statements keep
  // the issue order the barrier's load count relies on)
  load_w(0, Idx<0>{});
  load_a(0, Idx<0>{});
  // down: the rows' routing weights now, for the epilogue (loaded there, each row's weight
  // would be a dependent memory round trip at the end of every tile); ahead of k-block 1's
  // weights, so that those stay the newest NF + 1 loads the waits below count on
  if (kMode == kModeDown && wave * 64 < NSUB * 16) dma4(c.grs, lds.wgt + wave * 64, c.goff, 0);
  asm volatile("" ::: "memory");
  load_w(1, Idx<1>{});

  f32x4 u[NSUB][NF];  // running sums in units of the current k-block's scale
  float s_prev[NF], s_next[NF];
  uint4 wf[NF];       // packed weights of the k-block about to run
  uint4 bc[NF];       // dequantised weights of the k-step about to run
  uint4 a[NSUB];      // activation fragments of the k-step about to run
#pragma unroll
  for (int f = 0; f < NF; ++f) s_prev[f] = 0.f;
#pragma unroll
  for (int ms = 0; ms < NSUB; ++ms)
#pragma unroll
    for (int f = 0; f < NF; ++f) u[ms][f] = f32x4{0.f, 0.f, 0.f, 0.f};
  // k-block 0's weights and scales are in once at most the NF + 1 loads of k-block 1's are
  // pending (this also waits for the activations of k-block 0, which the first k-block's
  // barrier waits for anyway); written out for the same reason as the k-loop's wait below
  dma_wait<NF + 1>();
  read_w(wf, s_next, 0, Idx<0>{});
#pragma unroll
  for (int f = 0; f < NF; ++f) bc[f] = dequant8(wf[f].x);

#ifdef DFLASH_TIMELINE
  const unsigned long long tl_loop = __builtin_amdgcn_s_memtime();
#endif
  auto step = [&](int kb, auto sa_tag, auto sw_tag) {
    constexpr int sa = decltype(sa_tag)::value, sw = decltype(sw_tag)::value;
    // the activation stage of k-block kb is complete once this wave's loads older than the
    // last NF + 1 (weights and scales of k-block kb + 1) are
    dma_barrier<NF + 1>();
    load_a(kb + 1, Idx<(sa + 1) % kAStages>{});
    asm volatile("" ::: "memory");
    load_w(kb + 2, Idx<(sw + 2) % kWStages>{});
#pragma unroll
    for (int ms = 0; ms < NSUB; ++ms) a[ms] = lds.a[sa][ms * 4 * 64 + lane];
    // u <- u * s_prev / s_kb - 136 * sum(a_kb)   (k-block 0: u = -136 * sum)
    float ratio[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      ratio[f] = s_prev[f] * __builtin_amdgcn_rcpf(s_next[f]);
      s_prev[f] = s_next[f];
    }
#pragma unroll
    for (int ms = 0; ms < NSUB; ++ms) {
      const f32x4 start = *reinterpret_cast<const f32x4*>(lds.neg[sa] + ms * 16 + 4 * kq);
#pragma unroll
      for (int f = 0; f < NF; ++f) u[ms][f] = u[ms][f] * ratio[f] + start;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int ms = 0; ms < NSUB; ++ms) {
#pragma unroll
        for (int f = 0; f < NF; ++f) u[ms][f] = mfma16x16x32(a[ms], bc[f], u[ms][f]);
        if (j < 3) a[ms] = lds.a[sa][(ms * 4 + j + 1) * 64 + lane];
      }
      if (j == 3) {
        // the weights and scales of k-block kb + 1 are in once only this step's loads (the
        // activations of kb + 1 and the weights of kb + 2) may be pending.  The wait is written
        // out: the compiler's own wait for a direct-to-LDS load is dropped here when a wait
        // ahead of the loop has already drained the counter
        dma_wait<NF + 1>();
        read_w(wf, s_next, kb + 1, Idx<(sw + 1) % kWStages>{});
      }
#pragma unroll
      for (int f = 0; f < NF; ++f) bc[f] = dequant8(word(wf[f], (j + 1) & 3));
      // k-step 0 also holds the scale ratios and the rescale (4 NF FMAs per subtile), k-step 3
      // the next k-block's weight and scale reads.  No VALU work is placed ahead of a k-step's
      // first MFMA, and each MFMA is followed by one VALU operation more than the k-step's share
      // (prefill layer 269.6 -> 261.2 us against placing the ratios first and the exact share)
      if (j == 0) interleave<0, NF * NSUB, (4 * NF * NSUB + 6 * NF) / (NF * NSUB) + 1, 2>();
      else if (j == 3) interleave<0, NF * NSUB, 4, 2>();
      else interleave<0, NF * NSUB, 3, 4>();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int kb = 0; kb < nkb; kb += 6) {  // nkb is even; stage indices repeat every 6 k-blocks
    step(kb, Idx<0>{}, Idx<0>{});
    step(kb + 1, Idx<1>{}, Idx<1>{});
    if (kb + 2 < nkb) {
      step(kb + 2, Idx<0>{}, Idx<2>{});
      step(kb + 3, Idx<1>{}, Idx<0>{});
    }
    if (kb + 4 < nkb) {
      step(kb + 4, Idx<0>{}, Idx<1>{});
      step(kb + 5, Idx<1>{}, Idx<2>{});
    }
  }
  // no load may land in LDS once the stages are reused
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#ifdef DFLASH_TIMELINE
  const unsigned long long tl_epi = __builtin_amdgcn_s_memtime();
#endif

  // epilogue: lane holds rows 16 ms + 4 kq + e of its fragments' column lr
  const int4 d = c.d;
  if (kMode == kModeGateUp) {
    // h, and -136 * sum(h) per 128 columns: a wave covers 16 H2 columns of the gate and up
    // halves (H2 = NF / 2), so 8 / H2 consecutive waves cover one 128-column block; per-wave row
    // partials meet in LDS (activation stage 0)
    constexpr int H2 = NF / 2, kWavesPerBlock = kWaves / H2;
    float* red = reinterpret_cast<float*>(lds.a[0]);  // [kWaves][kTileM]
    __syncthreads();  // every wave is done reading the activation stages
#pragma unroll
    for (int ms = 0; ms < NSUB; ++ms) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = ms * 16 + 4 * kq + e;
        const bool valid = r < c.rows;
        const int m = d.w + min(r, c.rows - 1);
        const int hrow = c.shared ? p.T * p.top_k + m : d.y + m;
        float part = 0.f;
#pragma unroll
        for (int f = 0; f < H2; ++f) {
          const int col = c.nt * kWaves * 16 * H2 + wave * 16 * H2 + f * 16 + lr;
          const uint16_t hb = f32_to_bf16(silu(u[ms][f][e] * s_prev[f]) * (u[ms][f + H2][e] * s_prev[f + H2]));
          if (valid) p.out_bf16[static_cast<int64_t>(hrow) * inter + octet_slot(col)] = hb;
          part += bf16_to_f32(hb);
        }
        part = row16_sum(part);
        if (lr == 0) red[wave * kTileM + r] = part;
      }
    }
    __syncthreads();
    if (tid < H2 * kTileM) {
      const int half = tid / kTileM, r = tid - half * kTileM;
      if (r < c.rows) {
        const float* q = red + kWavesPerBlock * half * kTileM + r;
        float sum = (q[0] + q[kTileM]) + (q[2 * kTileM] + q[3 * kTileM]);
        if (kWavesPerBlock == 8) sum += (q[4 * kTileM] + q[5 * kTileM]) + (q[6 * kTileM] + q[7 * kTileM]);
        const int m = d.w + r;
        const int hrow = c.shared ? p.T * p.top_k + m : d.y + m;
        p.out_part[static_cast<int64_t>(hrow) * (inter >> 7) + c.nt * H2 + half] = -kDequantOffset * sum;
      }
    }
  } else {
#pragma unroll
    for (int ms = 0; ms < NSUB; ++ms) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = ms * 16 + 4 * kq + e;
        if (r >= c.rows) continue;
        const int m = d.w + r;
        const int yrow = c.shared ? p.T * p.top_k + m : d.y + m;
        const float wgt = lds.wgt[r];
        // weighted, in bf16: halves the y traffic of this launch and the combine's
        uint16_t* o = reinterpret_cast<uint16_t*>(p.out_f32) + static_cast<int64_t>(yrow) * p.N +
                      c.nt * kWaves * 16 * NF + wave * 16 * NF + lr;
#pragma unroll
        for (int f = 0; f < NF; ++f) o[f * 16] = f32_to_bf16(u[ms][f][e] * s_prev[f] * wgt);
      }
    }
  }
#ifdef DFLASH_TIMELINE
  const unsigned long long tl_end = __builtin_amdgcn_s_memtime();
  if (lane == 0 && c.tl_cyc) {
    unsigned long long* slot = c.tl_cyc + wave * kTlCycleFields;
    slot[0] = c.t_ctx - c.t_start;
    slot[1] = c.t_sync - c.t_ctx;
    slot[2] = tl_loop - c.t_sync;
    slot[3] = tl_epi - tl_loop;
    slot[4] = tl_end - tl_epi;
    slot[5] = 1;
  }
#endif
}

// One work tile: pass d (expert or -1 for the shared expert, segment start, slot rows, first
// row of the pass; up to 96 rows of one slot) times column tile nt of 8 x 16 NF columns
// (gate/up: 8 x 8 NF of each half).
// rhalf: 0 for every row of the pass, 1 for its first ceil(nsub / 2) subtiles, 2 for the rest.
template <int kMode, typename ScaleT, int NF>
__device__ __forceinline__ void run_tile(const W4StreamParams& p, const TileLds& lds, int4 d, int nt, int rhalf
#ifdef DFLASH_TIMELINE
                                         , unsigned long long* tl_cyc
#endif
) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int K = p.K, nkb = K >> 7, ng = K / p.G;
  const uint32_t rb = static_cast<uint32_t>(K >> 1);
  const int inter = p.N >> 1;
  // activation rows: tokens (gate_up) or every routed slot row plus the shared expert's (down)
  const uint32_t act_rows = kMode == kModeGateUp ? p.T : p.T * p.top_k + (p.has_shared ? p.T : 0);

  // weight row of fragment f, column lc (0..15) of this wave: gate/up fragments f < NF / 2 are
  // gate rows, the rest the same columns' up rows
  constexpr int H2 = NF / 2;
  auto wrow = [&](int f, int lc) {
    return kMode == kModeGateUp ? (f / H2) * inter + nt * kWaves * 16 * H2 + wave * 16 * H2 + (f % H2) * 16 + lc
                                : nt * kWaves * 16 * NF + wave * 16 * NF + f * 16 + lc;
  };

  TileCtx c;
#ifdef DFLASH_TIMELINE
  c.t_start = __builtin_amdgcn_s_memtime();
  c.tl_cyc = tl_cyc;
#endif
  c.nt = nt;
  c.d = d;
  c.shared = c.d.x < 0;
  c.rows = min(kTileM, c.d.z - c.d.w);
  if (rhalf) {
    const int lo = 16 * ((((c.rows + 15) >> 4) + 1) >> 1);
    if (rhalf == 2) {
      c.d.w += lo;
      c.rows -= lo;
    } else {
      c.rows = min(c.rows, lo);
    }
    if (c.rows <= 0) return;  // a one-subtile pass has no second half
  }
  c.ars = make_rsrc(p.act, act_rows * static_cast<uint32_t>(K) * 2);
  c.nrs = make_rsrc(p.act_neg, act_rows * static_cast<uint32_t>(nkb) * 4);
  c.wrs = make_rsrc(c.shared ? p.w_shared : p.w + static_cast<int64_t>(c.d.x) * p.w_stride,
                    static_cast<uint32_t>(p.N) * rb);
  c.srs = make_rsrc(static_cast<const uint8_t*>(c.shared ? p.s_shared : p.s) +
                        (c.shared ? 0 : static_cast<int64_t>(c.d.x) * p.s_stride * static_cast<int64_t>(sizeof(ScaleT))),
                    static_cast<uint32_t>(p.N) * static_cast<uint32_t>(ng) * sizeof(ScaleT));
  // a fragment's 16 rows are one tile of the tiled layout (its base is the same in both layouts)
  c.wkb = p.tiled ? 1024u : 64u;
#pragma unroll
  for (int f = 0; f < NF; ++f)
    c.woff[f] = p.tiled ? static_cast<uint32_t>(wrow(f, 0)) * rb + lane * 16
                        : static_cast<uint32_t>(wrow(f, lr)) * rb + kq * 16;
  // scale lane: fragment lane / 16 (lanes past the wave's NF fragments repeat its last one)
  const int sf = min(lane >> 4, NF - 1);
  c.soff = p.tiled ? (static_cast<uint32_t>(wrow(sf, 0)) * static_cast<uint32_t>(ng) +
                      static_cast<uint32_t>(sizeof(ScaleT) == 4 ? lr : lr & ~1)) * sizeof(ScaleT)
                   : static_cast<uint32_t>(wrow(sf, lr)) * static_cast<uint32_t>(ng) * sizeof(ScaleT);

  // source row of pass row r (rows past the pass repeat its last row)
  auto src_row = [&](int r) {
    const int m = c.d.w + min(r, c.rows - 1);
    if (kMode == kModeGateUp) return c.shared ? m : p.tok[c.d.y + m];
    return c.shared ? p.T * p.top_k + m : c.d.y + m;
  };
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int b = wave + kWaves * i;  // block: subtile b / 4, k-step b % 4
    c.aoff[i] = static_cast<uint32_t>(src_row(16 * (b >> 2) + lr)) * static_cast<uint32_t>(K) * 2 +
                (4 * kq + (b & 3)) * 16;
  }
  c.noff = static_cast<uint32_t>(src_row(min(wave * 64 + lane, kTileM - 1))) * static_cast<uint32_t>(nkb) * 4;
  if (kMode == kModeDown) {
    c.grs = make_rsrc(c.shared ? p.shared_gate + c.d.w : p.slot_w + c.d.y + c.d.w, static_cast<uint32_t>(c.rows) * 4);
    c.goff = static_cast<uint32_t>(min(wave * 64 + lane, c.rows - 1)) * 4;
  }

#ifdef DFLASH_TIMELINE
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the pass entry is in
  c.t_ctx = __builtin_amdgcn_s_memtime();
#endif
  __syncthreads();  // the previous tile's readers are done with every LDS stage
#ifdef DFLASH_TIMELINE
  c.t_sync = __builtin_amdgcn_s_memtime();
#endif

  switch ((c.rows + 15) >> 4) {
    case 1: tile_pass<kMode, ScaleT, 1, NF>(p, lds, c); break;
    case 2: tile_pass<kMode, ScaleT, 2, NF>(p, lds, c); break;
    case 3: tile_pass<kMode, ScaleT, 3, NF>(p, lds, c); break;
    case 4: tile_pass<kMode, ScaleT, 4, NF>(p, lds, c); break;
    case 5: tile_pass<kMode, ScaleT, 5, NF>(p, lds, c); break;
    default: tile_pass<kMode, ScaleT, 6, NF>(p, lds, c); break;
  }
}

}  // namespace

template <int kMode, typename ScaleT>
__global__ __launch_bounds__(512) void w4_tile_kernel(W4StreamParams p) {
  // the stages, a separate LDS array each
  __shared__ uint4 a0[kBlocks * 64], a1[kBlocks * 64];
  __shared__ float n0[128], n1[128], wg[128];
  __shared__ uint4 w0[kWaves * 4 * 64], w1[kWaves * 4 * 64], w2[kWaves * 4 * 64];
  __shared__ uint32_t s0[kWaves * 64], s1[kWaves * 64], s2[kWaves * 64];
  const TileLds lds{{a0, a1}, {n0, n1}, {w0, w1, w2}, {s0, s1, s2}, wg};
  __shared__ int next_tile;
  const int ntiles = p.strips;  // column tiles per pass
  const int passes = ld_const(p.meta, 1);
  const int total = passes * ntiles;
  // heaviest tiles first: the shared expert's passes (the last passes of the table), then the
  // routed experts' in table order (descending subtile count on this path)
  const int sp = p.has_shared ? (p.T + kTileM - 1) / kTileM : 0;
  // The tiles past the grid's last full round run in pieces (4 when they fill at most a
  // quarter of the grid, 2 when at most half): work items [0, full) are whole tiles, then
  // `pieces` per remaining tile (piece q: half-width column piece q & 1, row half q >> 1 when
  // there are 4).  A row half with no rows (one-subtile pass) is an empty item.
  // (p.tile_pieces, when set, forces 1, 2 or 4: a test and measurement override)
  const int grid = static_cast<int>(gridDim.x), rest = total % grid;
  const int pieces = p.tile_pieces ? p.tile_pieces : 4 * rest <= grid ? 4 : 2 * rest <= grid ? 2 : 1;
  const int split = pieces > 1 ? rest : 0;
  const int full = total - split, items = full + pieces * split;
  // Each workgroup takes its first item by index, then asks a queue for more; every
  // workgroup that ran an item makes exactly one failing request, so the queue ends at
  // `items` and the request that returns items - 1 is the launch's last: it resets the
  // queue for the next launch.  Nothing waits on the queue.
  int* queue = const_cast<int*>(p.meta) + (kMode == kModeGateUp ? 2 : 3);
#ifdef DFLASH_TIMELINE
  int tl_n = 0;
#endif
  for (int item = blockIdx.x; item < items;) {
    const bool whole = item < full;
    const int q = whole ? 0 : (item - full) & (pieces - 1);
    const int tile = whole ? item : full + (item - full) / pieces;
    const int i = tile / ntiles;
    const int P = i < sp ? passes - sp + i : i - sp;
    const int nt = tile - i * ntiles;
    const int4 d = ld_const_int4(p.pass_table, P);
#ifdef DFLASH_TIMELINE
    unsigned long long* tl = g_timeline_tile +
        (((kMode == kModeGateUp ? 0 : 1) * kTlWorkgroups + blockIdx.x) * kTlTiles + min(tl_n, kTlTiles - 1)) * 3;
    if (threadIdx.x == 0 && blockIdx.x < kTlWorkgroups) tl[0] = __builtin_amdgcn_s_memrealtime();
#endif
#ifdef DFLASH_TIMELINE
    unsigned long long* tl_cyc = blockIdx.x < kTlWorkgroups
        ? g_timeline_tile_cycles + (((kMode == kModeGateUp ? 0 : 1) * kTlWorkgroups + blockIdx.x) * kTlTiles +
                                    min(tl_n, kTlTiles - 1)) * kWavesTl * kTlCycleFields
        : nullptr;
    if (whole) run_tile<kMode, ScaleT, 4>(p, lds, d, nt, 0, tl_cyc);
    else run_tile<kMode, ScaleT, 2>(p, lds, d, 2 * nt + (q & 1), pieces == 4 ? 1 + (q >> 1) : 0, tl_cyc);
#else
    if (whole) run_tile<kMode, ScaleT, 4>(p, lds, d, nt, 0);
    else run_tile<kMode, ScaleT, 2>(p, lds, d, 2 * nt + (q & 1), pieces == 4 ? 1 + (q >> 1) : 0);
#endif
#ifdef DFLASH_TIMELINE
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0 && blockIdx.x < kTlWorkgroups) {
      tl[1] = __builtin_amdgcn_s_memrealtime();
      tl[2] = static_cast<unsigned long long>(min(kTileM, d.z - d.w)) | (static_cast<unsigned long long>(P) << 16) |
              (static_cast<unsigned long long>(tl_n + 1) << 40) | (static_cast<unsigned long long>(whole ? 0 : 1) << 56);
    }
    ++tl_n;
#endif
    if (threadIdx.x == 0) {
      const int got = __hip_atomic_fetch_add(queue, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (got == items - 1) __hip_atomic_store(queue, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      next_tile = grid + got;
    }
    __syncthreads();
    item = next_tile;
    __syncthreads();  // every wave has read next_tile before thread 0 may write it again
  }
}

bool w4_tile_supports(int mode, int N, int K, int G) {
  if (K % 512 || (G != 128 && G != 256)) return false;
  return mode == kModeGateUp ? (N / 2) % 256 == 0 : (mode == kModeDown && N % kTileN == 0);
}

void launch_w4_tile(int mode, bool fp32_scales, int grid, const W4StreamParams& p, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid)), blk(512);
  if (mode == kModeGateUp) {
    if (fp32_scales) hipLaunchKernelGGL((w4_tile_kernel<kModeGateUp, float>), g, blk, 0, stream, p);
    else hipLaunchKernelGGL((w4_tile_kernel<kModeGateUp, uint16_t>), g, blk, 0, stream, p);
  } else {
    if (fp32_scales) hipLaunchKernelGGL((w4_tile_kernel<kModeDown, float>), g, blk, 0, stream, p);
    else hipLaunchKernelGGL((w4_tile_kernel<kModeDown, uint16_t>), g, blk, 0, stream, p);
  }
}

#ifdef DFLASH_TIMELINE
int timeline_tile_read(void* host, size_t bytes) {
  if (bytes != sizeof(g_timeline_tile)) return 1;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_timeline_tile), bytes) == hipSuccess ? 0 : 1;
}
int timeline_tile_cycles_read(void* host, size_t bytes) {
  if (bytes != sizeof(g_timeline_tile_cycles)) return 1;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_timeline_tile_cycles), bytes) == hipSuccess ? 0 : 1;
}
int timeline_tile_clear() {
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_timeline_tile)) != hipSuccess) return 1;
  if (hipMemset(ptr, 0, sizeof(g_timeline_tile)) != hipSuccess) return 1;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_timeline_tile_cycles)) != hipSuccess) return 1;
  return hipMemset(ptr, 0, sizeof(g_timeline_tile_cycles)) == hipSuccess ? 0 : 1;
}
#endif

}  // namespace dflash
