// Router logits, activation preparation, top-k routing with renormalised
// weights, the stable token-to-expert permutation, and the final combine.
//
// Routing contract (reference reference/fused_ops.py:160-164,
// graph/fused/quant_target.py:168-172): rank the fp32 logits in descending
// order, lowest expert id first among equal logits; weights are the softmax of
// the selected logits (the full-softmax denominator cancels in the renorm).
// Permutation contract (npu_moe_init_routing_v2 as documented in
// docs/reference/qwen35-moe-operators-and-quantization-analysis.md:685-707):
// flat pairs t*k+slot sorted by expert, stable, so a segment lists its tokens
// in ascending order.
//
// Besides the reference outputs the routing kernels emit the work table the
// expert GEMMs consume: the hit experts in ascending order (then the shared
// expert as one more slot) and, per slot, the first "pass" index, a pass being
// up to rows_per_pass of the slot's tokens.
#include <algorithm>
#include <utility>

#include "topk.h"

namespace dflash {

// f(integral_constant<int, I>) for every I of the sequence, in order.
template <typename F, int... I>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// ---------------------------------------------------------------------------
// Activation preparation of one row of x: octet-interleaved copy, the
// -136*sum per 128-column block, and (optionally) sigmoid(x . gate_w).
// Executed by the first 256 threads of a block.  K % 128 == 0.
__device__ __forceinline__ void prep_row(const uint16_t* __restrict__ x, int K, int row, uint16_t* __restrict__ x_il,
                                         float* __restrict__ xneg, const uint16_t* __restrict__ gate_w,
                                         float* __restrict__ gate_out) {
  __shared__ float part[4];
  const int tid = threadIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(row) * K);
  uint4* dst = reinterpret_cast<uint4*>(x_il + static_cast<int64_t>(row) * K);
  const int chunks = K >> 3;
  float gate_acc = 0.f;
  if (tid < 256) {
    for (int base = 0; base < chunks; base += 256) {
      const int c = base + tid;
      float sum = 0.f;
      if (c < chunks) {
        const uint4 v = src[c];
        uint4 o;  // natural pairs (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
        o.x = (v.x & 0xFFFFu) | (v.z << 16);
        o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
        o.z = (v.y & 0xFFFFu) | (v.w << 16);
        o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
        dst[c] = o;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t gg[4] = {0u, 0u, 0u, 0u};
        if (gate_w) {
          const uint4 g = reinterpret_cast<const uint4*>(gate_w)[c];
          gg[0] = g.x; gg[1] = g.y; gg[2] = g.z; gg[3] = g.w;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xFFFF0000u);
          sum += lo + hi;
          gate_acc += lo * __uint_as_float(gg[i] << 16) + hi * __uint_as_float(gg[i] & 0xFFFF0000u);
        }
      }
      sum = row16_sum(sum);  // 16 chunks of 8 = one 128-column block, in 16 consecutive lanes
      if (c < chunks && (c & 15) == 0) xneg[static_cast<int64_t>(row) * (K >> 7) + (c >> 4)] = -kDequantOffset * sum;
    }
  }
  if (gate_w) {
    gate_acc = wave_sum(gate_acc);
    if (lane_id() == 0 && tid < 256) part[tid >> 6] = gate_acc;
    __syncthreads();
    if (tid == 0) gate_out[row] = 1.0f / (1.0f + __expf(-((part[0] + part[1]) + (part[2] + part[3]))));
  }
}

// Rows per prep block: 2 for short inputs (more blocks in flight), 16 for long ones.
__host__ __device__ inline int prep_rows_per_block(int rows) { return rows <= 64 ? 2 : 16; }

// Activation preparation of up to 16 rows by a 512-thread block: thread half h
// handles rows r0 + 2i + h, and the loads of all its rows are issued before any
// of them is written back, so a block waits for memory once per 2048 columns.
__device__ __forceinline__ void prep_block(const uint16_t* __restrict__ x, int K, int r0, int nrows,
                                           uint16_t* __restrict__ x_il, float* __restrict__ xneg,
                                           const uint16_t* __restrict__ gate_w, float* __restrict__ gate_out) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __shared__ float part[16][4];
  const int tid = threadIdx.x, h = tid >> 8, t = tid & 255, wave = tid >> 6;
  const int chunks = K >> 3;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  float gacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) gacc[i] = 0.f;
  for (int base = 0; base < chunks; base += 256) {
    const int c = base + t;
    const u32x4 g = gate_w && c < chunks ? reinterpret_cast<const u32x4*>(gate_w)[c] : zero4;
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = r0 + min(2 * i + h, nrows - 1);
      v[i] = c < chunks ? reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(r) * K)[c] : zero4;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = r0 + 2 * i + h;
      const bool live = 2 * i + h < nrows && c < chunks;
      u32x4 o;  // natural pairs (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
      o.x = (v[i].x & 0xFFFFu) | (v[i].z << 16);
      o.y = (v[i].x >> 16) | (v[i].z & 0xFFFF0000u);
      o.z = (v[i].y & 0xFFFFu) | (v[i].w << 16);
      o.w = (v[i].y >> 16) | (v[i].w & 0xFFFF0000u);
      if (live) reinterpret_cast<u32x4*>(x_il + static_cast<int64_t>(r) * K)[c] = o;
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = __uint_as_float(v[i][q] << 16), hi = __uint_as_float(v[i][q] & 0xFFFF0000u);
        sum += lo + hi;
        gacc[i] += lo * __uint_as_float(g[q] << 16) + hi * __uint_as_float(g[q] & 0xFFFF0000u);
      }
      sum = row16_sum(sum);  // 16 chunks of 8 = one 128-column block, in 16 consecutive lanes
      if (live && (c & 15) == 0) xneg[static_cast<int64_t>(r) * (K >> 7) + (c >> 4)] = -kDequantOffset * sum;
    }
  }
  if (gate_w) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = wave_sum(gacc[i]);
      if (lane_id() == 0) part[2 * i + h][wave & 3] = s;
    }
    __syncthreads();
    if (tid < nrows) gate_out[r0 + tid] = 1.0f / (1.0f + __expf(-((part[tid][0] + part[tid][1]) + (part[tid][2] + part[tid][3]))));
  }
}

// Router logits for a 16x16 tile: fp32 [T][E] = x bf16 [T][H] . W bf16 [E][H]^T;
// 8 waves split H (H % 256 == 0) and are reduced through LDS.  Used for hidden sizes other
// than 512, 1024 and 2048, which take the whole-line tiles below.
__device__ __forceinline__ void router_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                            float* __restrict__ logits, int T, int E, int H, int t0, int e0) {
  __shared__ f32x4 red[8][64];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int lr = lane & 15, kq = lane >> 4;
  const int trow = min(t0 + lr, T - 1), erow = min(e0 + lr, E - 1);
  const int span = H >> 3;
  const uint16_t* xa = x + static_cast<int64_t>(trow) * H + wave * span + kq * 8;
  const uint16_t* wb = w + static_cast<int64_t>(erow) * H + wave * span + kq * 8;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // 8 MFMA steps per batch, all loads of a batch in flight together (span % 32 == 0)
  for (int k0 = 0; k0 < span; k0 += 256) {
    uint4 av[8], bv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = min(k0 + 32 * i, span - 32);
      av[i] = *reinterpret_cast<const uint4*>(xa + k);
      bv[i] = *reinterpret_cast<const uint4*>(wb + k);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + 32 * i < span) acc = mfma16x16x32(av[i], bv[i], acc);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 s = red[0][lane];
#pragma unroll
    for (int i = 1; i < 8; ++i) s += red[i][lane];
    const int e = e0 + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t0 + 4 * kq + i;
      if (t < T && e < E) logits[static_cast<int64_t>(t) * E + e] = s[i];
    }
  }
}

// Router logits for a 16-token x 16-expert tile, read in whole cache lines (short T at
// H in {512, 1024, 2048}): the tile's 32 rows (16 token rows of x, then 16 expert rows of W)
// in chunks of 256 columns, wave instruction j of a chunk reading 512 contiguous bytes of rows
// 4 wave + 2 j and 4 wave + 2 j + 1, every load in flight at once; each chunk passes through
// an LDS copy with XOR-swizzled 16-byte slots, wave w takes k-step w of every chunk, and the
// eight partial tiles are added through LDS in wave order.
template <int kSteps>
__device__ __forceinline__ void router_line_tile16(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                   float* __restrict__ logits, int T, int E, int t0, int e0,
                                                   uint4* stage_u4) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // a plain vector: stays in registers
  constexpr int H = kSteps * 256;
  const int wave = threadIdx.x >> 6, lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  u32x4* stage = reinterpret_cast<u32x4*>(stage_u4);
  const u32x4* src[2];
  int dst[2];  // slot of the loaded 16 bytes in the chunk's LDS copy (32 slots per row)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 4 * wave + 2 * j + (lane >> 5);  // tile row 0..31
    const uint16_t* row = r < 16 ? x + static_cast<int64_t>(min(t0 + r, T - 1)) * H
                                 : w + static_cast<int64_t>(min(e0 + r - 16, E - 1)) * H;
    src[j] = reinterpret_cast<const u32x4*>(row) + (lane & 31);
    dst[j] = r * 32 + ((lane & 31) ^ (r & 7));
  }
  u32x4 v[kSteps][2];
#pragma unroll
  for (int c = 0; c < kSteps; ++c)
#pragma unroll
    for (int j = 0; j < 2; ++j) v[c][j] = src[j][32 * c];
  // every load goes out before the first one is waited for
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int slot = 4 * wave + kq;  // k-step wave of the chunk, this lane's 8 columns
  static_for(std::make_integer_sequence<int, kSteps>{}, [&](auto ci) {
    constexpr int c = decltype(ci)::value;
#pragma unroll
    for (int j = 0; j < 2; ++j) stage[dst[j]] = v[c][j];
    lds_barrier();  // the chunk is in LDS (the later chunks' loads stay in flight)
    const u32x4 a = stage[lr * 32 + (slot ^ (lr & 7))];
    const u32x4 b = stage[(16 + lr) * 32 + (slot ^ (lr & 7))];
    acc = mfma16x16x32(__builtin_bit_cast(uint4, a), __builtin_bit_cast(uint4, b), acc);
    lds_barrier();  // every wave has read the chunk before the next one is written (or the partials)
  });
  f32x4* red = reinterpret_cast<f32x4*>(stage_u4);
  red[wave * 64 + lane] = acc;
  lds_barrier();
  if (wave == 0) {
    f32x4 sum = red[lane];
#pragma unroll
    for (int i = 1; i < 8; ++i) sum += red[i * 64 + lane];
    const int e = e0 + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t0 + 4 * kq + i;
      if (t < T && e < E) logits[static_cast<int64_t>(t) * E + e] = sum[i];
    }
  }
}

// Router logits for a 32-token x 64-expert tile (long T), read in whole cache lines.  The
// tile's 96 rows (32 token rows of x, then 64 expert rows of W) are read in chunks of 256
// columns: wave instruction q of a chunk reads 512 contiguous bytes of rows 2q and 2q + 1
// (loads that cover only half of each 128-byte line, as MFMA fragments read straight from
// memory do, stream about a third as fast per CU), and every load of the tile is in flight
// at once (kSteps chunks x 6 per lane).  Each chunk passes through LDS, row-major with its
// 16-byte slots XOR-swizzled by row & 7 so that the fragment reads are free of bank
// conflicts.  Wave w accumulates a 32 x 32 block (both token subtiles, expert subtiles
// 2 (w & 1) and 2 (w & 1) + 1) over k-steps 2 (w >> 1) and 2 (w >> 1) + 1 of every chunk, one
// fragment read per MFMA; the four waves of an expert half then add their partials through LDS
// in k-step order.
template <int kSteps>
__device__ __forceinline__ void router_line_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                 float* __restrict__ logits, int T, int E, int t0, int e0,
                                                 uint4* stage_u4) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // a plain vector: stays in registers
  constexpr int H = kSteps * 256;
  const int wave = threadIdx.x >> 6, lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  u32x4* stage = reinterpret_cast<u32x4*>(stage_u4);
  const u32x4* src[6];
  int dst[6];  // slot of the loaded 16 bytes in the chunk's LDS copy (32 slots per row)
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const int r = 2 * (6 * wave + j) + (lane >> 5);  // tile row 0..95
    const uint16_t* row = r < 32 ? x + static_cast<int64_t>(min(t0 + r, T - 1)) * H
                                 : w + static_cast<int64_t>(min(e0 + r - 32, E - 1)) * H;
    src[j] = reinterpret_cast<const u32x4*>(row) + (lane & 31);
    dst[j] = r * 32 + ((lane & 31) ^ (r & 7));
  }
  u32x4 v[kSteps][6];
#pragma unroll
  for (int c = 0; c < kSteps; ++c)
#pragma unroll
    for (int j = 0; j < 6; ++j) v[c][j] = src[j][32 * c];
  // every load goes out before the first one is waited for
  __builtin_amdgcn_sched_barrier(0);
  // wave w: expert half w & 1 (subtiles 2 (w & 1) and 2 (w & 1) + 1), k-steps 2 (w >> 1) and
  // 2 (w >> 1) + 1 of every chunk, both token subtiles
  const int eh = wave & 1, kp = wave >> 1;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i >> 1][i & 1] = f32x4{0.f, 0.f, 0.f, 0.f};
  static_for(std::make_integer_sequence<int, kSteps>{}, [&](auto ci) {
    constexpr int c = decltype(ci)::value;
#pragma unroll
    for (int j = 0; j < 6; ++j) stage[dst[j]] = v[c][j];
    lds_barrier();  // the chunk is in LDS (the later chunks' loads stay in flight)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int s = 2 * kp + h;
      u32x4 a[2], b[2];
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        const int ra = 16 * ts + lr;
        a[ts] = stage[ra * 32 + ((4 * s + kq) ^ (ra & 7))];
      }
#pragma unroll
      for (int el = 0; el < 2; ++el) {
        const int rb = 32 + 16 * (2 * eh + el) + lr;
        b[el] = stage[rb * 32 + ((4 * s + kq) ^ (rb & 7))];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i >> 1][i & 1] = mfma16x16x32(__builtin_bit_cast(uint4, a[i >> 1]), __builtin_bit_cast(uint4, b[i & 1]),
                                          acc[i >> 1][i & 1]);
    }
    lds_barrier();  // every wave has read the chunk before the next one is written (or the partials)
  });
  // partials: red[wave][subtile (ts, el)][lane]; then wave w sums subtile (w >> 2, w & 3) over the
  // four k-step pairs in order
  f32x4* red = reinterpret_cast<f32x4*>(stage_u4);
#pragma unroll
  for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * 64 + lane] = acc[i >> 1][i & 1];
  lds_barrier();
  const int ts = wave >> 2, es = wave & 3, i_sub = ts * 2 + (es & 1);
  f32x4 sum = red[(((0 << 1) | (es >> 1)) * 4 + i_sub) * 64 + lane];
#pragma unroll
  for (int q = 1; q < 4; ++q) sum += red[(((q << 1) | (es >> 1)) * 4 + i_sub) * 64 + lane];
  const int e = e0 + 16 * es + lr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + 16 * ts + 4 * kq + i;
    if (t < T && e < E) logits[static_cast<int64_t>(t) * E + e] = sum[i];
  }
}

// One launch doing the work that needs no routing: activation prep rows, zeroing
// of the multi-workgroup routing buffers, and router tiles (optional).
// block = 512.  blocks: [0, prep blocks) prep (prep_rows_per_block rows each), then
// n_zero blocks clearing zero_words 32-bit words, then n_router router tiles.  The
// short blocks go first: at long T the router tiles fill every CU for most of the
// launch (one workgroup per CU), and blocks behind them would start only at its end.
__global__ __launch_bounds__(512) void front_kernel(FrontParams p) {
  int b = blockIdx.x;
  const int per_block = prep_rows_per_block(p.prep_rows);
  const int prep_blocks = (p.prep_rows + per_block - 1) / per_block;
  if (b < prep_blocks) {
    prep_block(p.x, p.H, per_block * b, min(per_block, p.prep_rows - per_block * b), p.x_il, p.xneg, p.gate_w,
               p.gate_out);
    return;
  }
  b -= prep_blocks;
  if (b < p.n_zero) {
    for (int64_t i = static_cast<int64_t>(b) * 512 + threadIdx.x; i < p.zero_words;
         i += static_cast<int64_t>(p.n_zero) * 512)
      p.zero[i] = 0u;
    return;
  }
  b -= p.n_zero;
  __shared__ uint4 stage[96 * 32];  // whole-line router tiles: one 256-column chunk of the tile's rows
  if (p.router_big) {
    // the expert tiles of a token tile share its rows: blocks b, b + 8, ... of a group of
    // 8 token tiles take them (consecutive workgroups go to different XCDs, each with its L2)
    const int tiles_e = (p.E + 63) / 64, tiles_t = (p.T + 31) / 32;
    const int group = b / (8 * tiles_e), r = b - group * 8 * tiles_e;
    const bool whole = group * 8 + 8 <= tiles_t;
    const int tt = group * 8 + (whole ? r % 8 : r / tiles_e), te = whole ? r / 8 : r % tiles_e;
    const int t0 = tt * 32, e0 = te * 64;
    if (p.H == 512) router_line_tile<2>(p.x, p.router_w, p.logits, p.T, p.E, t0, e0, stage);
    else if (p.H == 1024) router_line_tile<4>(p.x, p.router_w, p.logits, p.T, p.E, t0, e0, stage);
    else router_line_tile<8>(p.x, p.router_w, p.logits, p.T, p.E, t0, e0, stage);
  } else {
    const int tiles_e = (p.E + 15) / 16;
    const int t0 = (b / tiles_e) * 16, e0 = (b % tiles_e) * 16;
    if (p.H == 512) router_line_tile16<2>(p.x, p.router_w, p.logits, p.T, p.E, t0, e0, stage);
    else if (p.H == 1024) router_line_tile16<4>(p.x, p.router_w, p.logits, p.T, p.E, t0, e0, stage);
    else if (p.H == 2048) router_line_tile16<8>(p.x, p.router_w, p.logits, p.T, p.E, t0, e0, stage);
    else router_tile(p.x, p.router_w, p.logits, p.T, p.E, p.H, t0, e0);
  }
}

// ---------------------------------------------------------------------------
// Single-workgroup routing for small T (route_small_fits).
// LDS slot map [E][tpad]: byte = slot+1 of token t in expert e, or 0.
__global__ __launch_bounds__(1024) void route_small_kernel(RouteParams p) {
  __shared__ int counts[kMaxExperts];
  __shared__ int wave_tot[3][16];
  __shared__ uint32_t slotmap_words[kSmallSlotBytes / 4];
  __shared__ float wts_lds[kSmallPairs];
  uint8_t* slotmap = reinterpret_cast<uint8_t*>(slotmap_words);
  const int T = p.T, E = p.E, k = p.k;
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  const int tpad = (T + 3) & ~3;
  for (int i = tid; i < kMaxExperts; i += 1024) counts[i] = 0;
  for (int i = tid; i < (E * tpad) / 4; i += 1024) slotmap_words[i] = 0u;
  __syncthreads();
  auto record = [&](int t, int id, float w) {
    if (lane < k) {
      p.ids[t * k + lane] = id;
      p.wts[t * k + lane] = w;
      wts_lds[t * k + lane] = w;
      atomicAdd(&counts[id], 1);
      slotmap[id * tpad + t] = static_cast<uint8_t>(lane + 1);
    }
  };
  if (E <= 256) {
    // tokens wave, wave + 16, ... in groups of 4: the group's logit rows are all requested
    // before the first selection, so a wave waits for one memory round trip per group
    constexpr int kGroup = 4;
    for (int t0 = wave; t0 < T; t0 += 16 * kGroup) {
      uint32_t key[kGroup][4];
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        const int t = min(t0 + 16 * g, T - 1);  // past the end: reload the last row, not recorded
        load_keys<4>(p.logits + static_cast<int64_t>(t) * E, E, key[g]);
      }
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        const int t = t0 + 16 * g;
        if (t < T) {
          int id;
          float w;
          select_keys<4>(key[g], k, &id, &w);
          record(t, id, w);
        }
      }
    }
  } else {
    for (int t = wave; t < T; t += 16) {
      int id;
      float w;
      topk_any(p.logits + static_cast<int64_t>(t) * E, E, k, &id, &w);
      record(t, id, w);
    }
  }
  __syncthreads();
  // exclusive scans over experts: segment offsets, hit index, first pass
  const int cnt = tid < E ? counts[tid] : 0;
  const int npass = passes_for(cnt, p.rows_per_pass);
  int a = cnt, b = cnt > 0 ? 1 : 0, c = npass;
  for (int o = 1; o < 64; o <<= 1) {
    const int ua = __shfl_up(a, o, 64), ub = __shfl_up(b, o, 64), uc = __shfl_up(c, o, 64);
    if (lane >= o) {
      a += ua;
      b += ub;
      c += uc;
    }
  }
  if (lane == 63) {
    wave_tot[0][wave] = a;
    wave_tot[1][wave] = b;
    wave_tot[2][wave] = c;
  }
  __syncthreads();
  int ba = 0, bb = 0, bc = 0;
  for (int i = 0; i < wave; ++i) {
    ba += wave_tot[0][i];
    bb += wave_tot[1][i];
    bc += wave_tot[2][i];
  }
  const int off = ba + a - cnt, hit_idx = bb + b - (cnt > 0 ? 1 : 0), pass0 = bc + c - npass;
  if (tid < E) {
    p.offsets[tid] = off;
    if (cnt > 0) {
      p.hit[hit_idx] = tid;
      p.pass_start[hit_idx] = pass0;
      write_slot(p.slot_table, p.pass_slot, p.pass_table, hit_idx, tid, off, cnt, pass0, p.rows_per_pass);
    }
    if (tid == E - 1) {
      const int nh = hit_idx + (cnt > 0 ? 1 : 0);
      int total = pass0 + npass;
      p.offsets[E] = off + cnt;
      p.pass_start[nh] = total;
      if (p.has_shared) {
        write_slot(p.slot_table, p.pass_slot, p.pass_table, nh, -1, 0, T, total, p.rows_per_pass);
        total += passes_for(T, p.rows_per_pass);
      }
      p.pass_start[nh + p.has_shared] = total;
      p.meta[0] = nh;
      p.meta[1] = total;
      p.meta[2] = 0;  // tile-queue counters of the prefill expert kernels
      p.meta[3] = 0;
    }
  }
  // stable ranks: expert tid walks its slot-map row (tokens ascending)
  if (tid < E && cnt > 0) {
    int pos = off;
    const uint32_t* row = slotmap_words + (tid * tpad) / 4;
    for (int q = 0; q < tpad / 4; ++q) {
      uint32_t word = row[q];
      while (word) {
        const int byte = __builtin_ctz(word) >> 3;
        const int flat = (q * 4 + byte) * k + static_cast<int>((word >> (byte * 8)) & 0xFFu) - 1;
        p.perm[pos] = flat;
        p.inv[flat] = pos;
        p.slot_w[pos] = wts_lds[flat];
        p.tok[pos] = q * 4 + byte;
        ++pos;
        word &= ~(0xFFu << (byte * 8));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Multi-workgroup routing for large T.  The counts and the slot map [E][T]
// (bytes) must be zero on entry: front_kernel or route_zero_kernel clears them.
__global__ void route_zero_kernel(uint32_t* __restrict__ words, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    words[i] = 0u;
}

// grid = ceil(T/4) + prep blocks, block = 256: one wave per token, then the prep blocks, each
// taking rows b, b + B, ... (B = prep blocks, at most kMaxPrepBlocks, so the grid's work-item
// count stays far below 2^32 at any T the routing accepts).
__global__ __launch_bounds__(256) void route_topk_kernel(RouteParams p) {
  const int topk_blocks = (p.T + 3) >> 2;
  if (static_cast<int>(blockIdx.x) >= topk_blocks) {
    const int b = static_cast<int>(blockIdx.x) - topk_blocks, nb = static_cast<int>(gridDim.x) - topk_blocks;
    for (int row = b; row < p.prep_rows; row += nb) {
      if (row != b) __syncthreads();  // the previous row's gate partials are read
      prep_row(p.prep_x, p.prep_H, row, p.prep_x_il, p.prep_xneg, p.prep_gate_w, p.prep_gate_out);
    }
    return;
  }
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = lane_id();
  if (t >= p.T) return;
  int id;
  float w;
  topk_any(p.logits + static_cast<int64_t>(t) * p.E, p.E, p.k, &id, &w);
  if (lane < p.k) {
    p.ids[static_cast<int64_t>(t) * p.k + lane] = id;
    p.wts[static_cast<int64_t>(t) * p.k + lane] = w;
    p.slotmap[static_cast<int64_t>(id) * route_slot_pitch(p.T) + t] = static_cast<uint8_t>(lane + 1);
  }
}

// Non-zero bytes of a 32-bit word.
__device__ __forceinline__ int nonzero_bytes(uint32_t x) {
  const uint32_t zero_hi = ~(((x & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | x | 0x7F7F7F7Fu);  // 0x80 per zero byte
  return 4 - __popc(zero_hi);
}

__device__ __forceinline__ int nonzero_bytes(uint4 v) {
  return nonzero_bytes(v.x) + nonzero_bytes(v.y) + nonzero_bytes(v.z) + nonzero_bytes(v.w);
}

// grid = ceil(E/4), block = 256: one wave per expert counts its tokens in the slot map.
__global__ __launch_bounds__(256) void route_count_kernel(RouteParams p) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= p.E) return;
  const int chunks = route_slot_pitch(p.T) >> 4;
  const uint4* row = reinterpret_cast<const uint4*>(p.slotmap + static_cast<int64_t>(e) * route_slot_pitch(p.T));
  int n = 0;
  for (int c = lane_id(); c < chunks; c += 64) n += nonzero_bytes(row[c]);
  n = wave_sum_int(n);
  if (lane_id() == 0) p.counts[e] = n;
}

// Buckets of the sorted pass table: an expert with c rows has c / rows_per_pass full passes and
// a last pass of the remaining rows; bucket j holds the passes of rows_per_pass / 16 - j
// 16-row subtiles.  n0: the expert's passes in bucket 0 (its full passes, and its last pass when
// that has as many subtiles); jl: the bucket of a lighter last pass, or -1.
__device__ __forceinline__ void pass_buckets(int c, int rows_per_pass, int& n0, int& jl) {
  const int full = c / rows_per_pass, sub = (c - full * rows_per_pass + 15) >> 4, top = rows_per_pass >> 4;
  n0 = full + (sub == top ? 1 : 0);
  jl = sub > 0 && sub < top ? top - sub : -1;
}

// Pairs up to which route_permute counts the experts itself (from the selected ids) and the
// count launch is skipped: each of a workgroup's 256 threads loads up to 16 x 4 ids.
constexpr int kPermuteCountPairs = 16384;

// grid = ceil(E/4), block = 256: one wave per expert writes its segment of the
// permutation.  Lane l owns a contiguous run of the expert's slot-map row, so
// an exclusive scan of the per-lane hit counts gives every token its position
// in ascending token order.  The wave's loads go out before their first use (its
// slot-map run, the counts of the experts below it, its own count), then the
// routing weights of its first two chunks' pairs in one batch; sums and scans
// are DPP reductions.  kCount (T*k <= kPermuteCountPairs): every workgroup builds
// the expert histogram of all T*k selected ids in LDS (one 16-byte load per thread
// per 1024 ids, LDS atomic adds), in place of route_count's launch.  sort_passes: the
// wave also reads the counts of the experts above it and places each of its passes at its rank
// in descending subtile order (passes of heavier buckets anywhere, then those of its own
// bucket in lower experts).
template <bool kCount>
__global__ __launch_bounds__(256) void route_permute_kernel(RouteParams p) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = lane_id();
  __shared__ int hist[kCount ? kMaxExperts : 1];
  if constexpr (kCount) {  // every thread of the workgroup takes part, live expert or not
    for (int i = threadIdx.x; i < p.E; i += 256) hist[i] = 0;
    __syncthreads();
    const int n = p.T * p.k;
    const buf_rsrc ir = make_rsrc(p.ids, static_cast<uint32_t>(n) * 4);
    uint4 v[kPermuteCountPairs / 1024];
#pragma unroll
    for (int j = 0; j < kPermuteCountPairs / 1024; ++j)
      v[j] = 4 * (threadIdx.x + 256 * j) < n ? buf_load16(ir, static_cast<uint32_t>(threadIdx.x + 256 * j) * 16, 0)
                                             : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int j = 0; j < kPermuteCountPairs / 1024; ++j) {
      const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * (threadIdx.x + 256 * j) + q < n) atomicAdd(&hist[w[q]], 1);
    }
    __syncthreads();
  }
  if (e >= p.E) return;
  // this lane's run of the slot-map row (its first two chunks in registers)
  const int pitch = route_slot_pitch(p.T);
  const int per_lane = ((pitch >> 4) + 63) >> 6;  // 16-byte chunks per lane
  const uint4* row = reinterpret_cast<const uint4*>(p.slotmap + static_cast<int64_t>(e) * pitch);
  const int c0 = lane * per_lane, c1 = min(c0 + per_lane, pitch >> 4);
  const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
  const uint4 r0 = c0 < c1 ? row[c0] : zero4, r1 = c0 + 1 < c1 ? row[c0 + 1] : zero4;
  const int cnt = kCount ? hist[e] : ld_const(p.counts, e);
  // sorted pass table: this expert's passes of the heaviest bucket (full ones, and a last pass
  // of as many subtiles), and the bucket of its lighter last pass (-1: none)
  int own0 = 0, jl = -1;
  if (p.sort_passes) pass_buckets(cnt, p.rows_per_pass, own0, jl);
  // sums over the experts below e; sorted table: the heaviest-bucket passes below e, the passes
  // in jl below e, and the passes of every expert in buckets heavier than jl
  int before = 0, nz_before = 0, pass_before = 0, pre0 = 0, prel = 0, heavier = 0;
  auto add = [&](int e2, int c) {
    if (e2 < e) {
      before += c;
      nz_before += c > 0 ? 1 : 0;
      pass_before += passes_for(c, p.rows_per_pass);
    }
    if (p.sort_passes) {
      int n0, j;
      pass_buckets(c, p.rows_per_pass, n0, j);
      if (e2 < e) {
        pre0 += n0;
        prel += j == jl ? 1 : 0;
      }
      heavier += (jl > 0 ? n0 : 0) + (j >= 0 && j < jl ? 1 : 0);
    }
  };
  const int span = p.sort_passes ? p.E : e;  // experts whose counts are read
  if constexpr (kCount) {
    for (int e2 = lane; e2 < span; e2 += 64) add(e2, hist[e2]);
  } else {
    // the resource reads 0 from span on
    const buf_rsrc cr = make_rsrc(p.counts, static_cast<uint32_t>(span) * 4);
#pragma unroll
    for (int j = 0; j < kMaxExperts / 64; ++j)
      add(lane + 64 * j,
          static_cast<int>(__float_as_uint(buf_load_f32(cr, static_cast<uint32_t>(lane + 64 * j) * 4, 0))));
  }
  before = __builtin_amdgcn_readlane(wave_inclusive_scan(before), 63);
  nz_before = __builtin_amdgcn_readlane(wave_inclusive_scan(nz_before), 63);
  pass_before = __builtin_amdgcn_readlane(wave_inclusive_scan(pass_before), 63);
  if (p.sort_passes) {
    pre0 = __builtin_amdgcn_readlane(wave_inclusive_scan(pre0), 63);
    prel = __builtin_amdgcn_readlane(wave_inclusive_scan(prel), 63);
    heavier = __builtin_amdgcn_readlane(wave_inclusive_scan(heavier), 63);
  }
  if (lane == 0) {
    p.offsets[e] = before;
    if (cnt > 0) {
      p.hit[nz_before] = e;
      p.pass_start[nz_before] = pass_before;
      if (p.sort_passes) {
        p.slot_table[nz_before] = make_int4(e, before, cnt, pass_before);
        for (int i = 0; i < own0; ++i) p.pass_table[pre0 + i] = make_int4(e, before, cnt, i * p.rows_per_pass);
        if (jl >= 0) p.pass_table[heavier + prel] = make_int4(e, before, cnt, own0 * p.rows_per_pass);
      } else {
        write_slot(p.slot_table, p.pass_slot, p.pass_table, nz_before, e, before, cnt, pass_before, p.rows_per_pass);
      }
    }
    if (e == p.E - 1) {
      const int nh = nz_before + (cnt > 0 ? 1 : 0);
      int total = pass_before + passes_for(cnt, p.rows_per_pass);
      p.offsets[p.E] = before + cnt;
      p.pass_start[nh] = total;
      if (p.has_shared) {
        write_slot(p.slot_table, p.pass_slot, p.pass_table, nh, -1, 0, p.T, total, p.rows_per_pass);
        total += passes_for(p.T, p.rows_per_pass);
      }
      p.pass_start[nh + p.has_shared] = total;
      p.meta[0] = nh;
      p.meta[1] = total;
      p.meta[2] = 0;  // tile-queue counters of the prefill expert kernels
      p.meta[3] = 0;
    }
  }
  if (cnt == 0) return;
  int mine = nonzero_bytes(r0) + nonzero_bytes(r1);
  for (int c = c0 + 2; c < c1; ++c) mine += nonzero_bytes(row[c]);
  int pos = before + wave_inclusive_scan(mine) - mine;
  // the routing weights of a chunk's pairs come in one batch of loads ahead of the writes (a
  // load inside each pair's branch would wait once per byte position); empty bytes load past
  // the end of the resource, which reads 0 without touching memory
  const buf_rsrc wr = make_rsrc(p.wts, static_cast<uint32_t>(p.T * p.k) * 4);
  auto chunk_weights = [&](const uint4& v, int c, float (&wt)[16]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int slot1 = (w[q >> 2] >> (8 * (q & 3))) & 0xFF;
      const uint32_t off = slot1 ? static_cast<uint32_t>(((16 * c + q) * p.k + slot1 - 1) * 4) : 0xFFFFFFF0u;
      wt[q] = buf_load_f32(wr, off, 0);
    }
  };
  auto chunk_write = [&](const uint4& v, int c, const float (&wt)[16]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int slot1 = (w[q >> 2] >> (8 * (q & 3))) & 0xFF;
      if (slot1) {
        const int t = 16 * c + q;
        const int flat = t * p.k + slot1 - 1;
        p.perm[pos] = flat;
        p.inv[flat] = pos;
        p.slot_w[pos] = wt[q];
        p.tok[pos] = t;
        ++pos;
      }
    }
  };
  float w0[16], w1[16];
  chunk_weights(r0, c0, w0);
  chunk_weights(r1, c0 + 1, w1);
  chunk_write(r0, c0, w0);
  chunk_write(r1, c0 + 1, w1);
  for (int c = c0 + 2; c < c1; ++c) {
    const uint4 v = row[c];
    chunk_weights(v, c, w0);
    chunk_write(v, c, w0);
  }
}
// ---------------------------------------------------------------------------
// Work table from existing segment offsets (experts-only entry) plus the
// activation prep rows.  block = 512: block 0 builds the table (E <= 1024
// experts, two per thread), blocks 1..T prepare rows.
__global__ __launch_bounds__(512) void table_prep_kernel(TableParams p) {
  if (blockIdx.x > 0) {
    prep_row(p.x, p.H, blockIdx.x - 1, p.x_il, p.xneg, p.gate_w, p.gate_out);
    return;
  }
  __shared__ int wave_tot[2][8];
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  int cnt[2], b = 0, c = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = 2 * tid + j;
    cnt[j] = e < p.E ? p.offsets[e + 1] - p.offsets[e] : 0;
    b += cnt[j] > 0 ? 1 : 0;
    c += passes_for(cnt[j], p.rows_per_pass);
  }
  int ib = b, ic = c;
  for (int o = 1; o < 64; o <<= 1) {
    const int ub = __shfl_up(ib, o, 64), uc = __shfl_up(ic, o, 64);
    if (lane >= o) {
      ib += ub;
      ic += uc;
    }
  }
  if (lane == 63) {
    wave_tot[0][wave] = ib;
    wave_tot[1][wave] = ic;
  }
  __syncthreads();
  int bb = 0, bc = 0;
  for (int i = 0; i < wave; ++i) {
    bb += wave_tot[0][i];
    bc += wave_tot[1][i];
  }
  int h = bb + ib - b, ps = bc + ic - c;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = 2 * tid + j;
    if (cnt[j] > 0) {
      p.hit[h] = e;
      p.pass_start[h] = ps;
      write_slot(p.slot_table, p.pass_slot, p.pass_table, h, e, p.offsets[e], cnt[j], ps, p.rows_per_pass);
      ++h;
    }
    ps += passes_for(cnt[j], p.rows_per_pass);
  }
  for (int i = tid; i < p.T * p.k; i += 512) {
    const int flat = p.perm[i];
    p.slot_w[i] = p.wts[flat];
    p.tok[i] = flat / p.k;
  }
  if (tid == 511) {
    int total = ps;
    p.pass_start[h] = total;
    if (p.has_shared) {
      write_slot(p.slot_table, p.pass_slot, p.pass_table, h, -1, 0, p.T, total, p.rows_per_pass);
      total += passes_for(p.T, p.rows_per_pass);
    }
    p.pass_start[h + p.has_shared] = total;
    p.meta[0] = h;
    p.meta[1] = total;
    p.meta[2] = 0;  // tile-queue counters of the prefill expert kernels
    p.meta[3] = 0;
  }
}

// ---------------------------------------------------------------------------
// Combine: out[t] = sum_slot y[inv[t*k+slot]] (+ y[T*k + t] for the shared
// expert), fp32 in slot order, one bf16 rounding.  y rows are fp32, or bf16
// (the prefill tile path, already weighted).  When wts is given the rows
// are unweighted expert outputs and each is scaled first: by wts[t*k+slot]
// (the routing weight) or gate[t] (the shared-expert sigmoid) -- the same fp32
// product the expert epilogues otherwise apply.  grid = (T, H / 512),
// block = 64: a lane owns 8 columns; the rows are read kBatch at a time, all
// loads of a batch in flight together, and added in slot order.  fp32 rows come
// from verify blocks (top-k + the shared expert: 9 rows at top-8), read in one
// batch of 16; the prefill's bf16 rows stream in batches of 8.
template <typename YT>
__global__ __launch_bounds__(64) void combine_kernel(const YT* __restrict__ y, const int32_t* __restrict__ inv, int T,
                                                     int k, int H, int has_shared, const float* __restrict__ wts,
                                                     const float* __restrict__ gate, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int c = (blockIdx.y * 64 + threadIdx.x) * 8;
  const int nrows = k + (has_shared ? 1 : 0);
  if (c < H) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    constexpr int kBatch = sizeof(YT) == 4 ? 16 : 8;
    for (int s0 = 0; s0 < nrows; s0 += kBatch) {
      float4 a[kBatch], b[kBatch];
      float w[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int s = min(s0 + i, nrows - 1);
        const int64_t row = s < k ? ld_const(inv, t * k + s) : static_cast<int64_t>(T) * k + t;
        if constexpr (sizeof(YT) == 4) {
          const float4* src = reinterpret_cast<const float4*>(y + row * H + c);
          a[i] = src[0];
          b[i] = src[1];
        } else {  // bf16 rows: 8 columns in one 16-byte load
          const uint4 v = *reinterpret_cast<const uint4*>(y + row * H + c);
          a[i] = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                             __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
          b[i] = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xFFFF0000u),
                             __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xFFFF0000u));
        }
        w[i] = wts == nullptr ? 1.f : (s < k ? ld_const(wts, t * k + s) : ld_const(gate, t));
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (s0 + i < nrows) {
          if (wts != nullptr) {
            a[i].x *= w[i]; a[i].y *= w[i]; a[i].z *= w[i]; a[i].w *= w[i];
            b[i].x *= w[i]; b[i].y *= w[i]; b[i].z *= w[i]; b[i].w *= w[i];
          }
          acc[0] += a[i].x; acc[1] += a[i].y; acc[2] += a[i].z; acc[3] += a[i].w;
          acc[4] += b[i].x; acc[5] += b[i].y; acc[6] += b[i].z; acc[7] += b[i].w;
        }
      }
    }
    uint4 o;
    o.x = f32_to_bf16(acc[0]) | (static_cast<uint32_t>(f32_to_bf16(acc[1])) << 16);
    o.y = f32_to_bf16(acc[2]) | (static_cast<uint32_t>(f32_to_bf16(acc[3])) << 16);
    o.z = f32_to_bf16(acc[4]) | (static_cast<uint32_t>(f32_to_bf16(acc[5])) << 16);
    o.w = f32_to_bf16(acc[6]) | (static_cast<uint32_t>(f32_to_bf16(acc[7])) << 16);
    *reinterpret_cast<uint4*>(out + static_cast<int64_t>(t) * H + c) = o;
  }
}

// Combine of the split-K down: a slot row's y is the sum of its partial rows (row_seg: first
// partial row and count, consecutive partials part_rps rows apart, in workgroup order), then
// weighted and added over the slots.  grid = (T, H / 256), block = 512: wave w takes slots
// w, w + 8, ... and loads up to 8 partials of a slot at once (four columns per lane), so every
// partial of the block is in flight together; the waves' weighted sums meet in LDS and wave 0
// adds them in wave order.
__global__ __launch_bounds__(512) void combine_parts_kernel(const float* __restrict__ y, const int2* __restrict__ seg,
                                                            int rps, const int32_t* __restrict__ inv, int T, int k,
                                                            int H, int has_shared, const float* __restrict__ wts,
                                                            const float* __restrict__ gate, uint16_t* __restrict__ out) {
  __shared__ float4 wave_sum[8][64];
  const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = blockIdx.y * 256 + lane * 4;
  const int nrows = k + (has_shared ? 1 : 0);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < H) {
    for (int s = wave; s < nrows; s += 8) {
      const int row = s < k ? ld_const(inv, t * k + s) : T * k + t;
      const int2 sg = seg[row];
      const float w = s < k ? ld_const(wts, t * k + s) : ld_const(gate, t);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int j0 = 0; j0 < sg.y; j0 += 8) {
        float4 a[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t r = static_cast<int64_t>(sg.x) + static_cast<int64_t>(rps) * min(j0 + j, sg.y - 1);
          a[j] = *reinterpret_cast<const float4*>(y + r * H + c);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (j0 + j < sg.y) {
            v.x += a[j].x; v.y += a[j].y; v.z += a[j].z; v.w += a[j].w;
          }
        }
      }
      acc.x += v.x * w; acc.y += v.y * w; acc.z += v.z * w; acc.w += v.w * w;
    }
  }
  wave_sum[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && c < H) {
    float4 o = wave_sum[0][lane];
    for (int i = 1; i < min(8, nrows); ++i) {
      const float4 u = wave_sum[i][lane];
      o.x += u.x; o.y += u.y; o.z += u.z; o.w += u.w;
    }
    uint2 r;
    r.x = f32_to_bf16(o.x) | (static_cast<uint32_t>(f32_to_bf16(o.y)) << 16);
    r.y = f32_to_bf16(o.z) | (static_cast<uint32_t>(f32_to_bf16(o.w)) << 16);
    *reinterpret_cast<uint2*>(out + static_cast<int64_t>(t) * H + c) = r;
  }
}

// ---------------------------------------------------------------------------
// host launchers
// 32 x 64 tiles read 384 KB each: they pay only with enough of them to fill the CUs (T=2048 at
// E=256 gives 256); below, 16 x 16 tiles spread the router rows over more workgroups
// (T=128: 128 tiles of 64 KB instead of 16 of 384 KB).
bool router_big_fits(int T, int H) { return T >= 1024 && (H == 512 || H == 1024 || H == 2048); }

int router_tiles(int T, int E, int H) {
  return router_big_fits(T, H) ? ((T + 31) / 32) * ((E + 63) / 64) : ((T + 15) / 16) * ((E + 15) / 16);
}

void launch_front(const FrontParams& p, hipStream_t stream) {
  const int per_block = prep_rows_per_block(p.prep_rows);
  const int blocks = p.n_router + (p.prep_rows + per_block - 1) / per_block + p.n_zero;
  if (blocks <= 0) return;
  hipLaunchKernelGGL(front_kernel, dim3(blocks), dim3(512), 0, stream, p);
}

// One workgroup selects 16 tokens at a time: above 32 tokens the per-token waves of the
// multi-workgroup kernels finish sooner (T=128: 40 us in one workgroup).
bool route_small_fits(int T, int E, int k) {
  return T <= 32 && static_cast<int64_t>(T) * k <= kSmallPairs &&
         static_cast<int64_t>((T + 3) & ~3) * E <= kSmallSlotBytes;
}

int64_t route_zero_words(int T, int E) {
  // counts [E rounded up to 4] followed by the slot map [E][pitch] bytes, in 32-bit words
  return ((E + 3) & ~3) + static_cast<int64_t>(E) * route_slot_pitch(T) / 4;
}

// Prep blocks of a route_topk launch: one per row up to this many (T = 2048 prefill: one each).
constexpr int kMaxPrepBlocks = 16384;

void launch_route(const RouteParams& p, bool zeroed, hipStream_t stream) {
  if (route_small_fits(p.T, p.E, p.k)) {
    hipLaunchKernelGGL(route_small_kernel, dim3(1), dim3(1024), 0, stream, p);
    return;
  }
  if (!zeroed) {
    const int64_t words = route_zero_words(p.T, p.E);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((words + 255) / 256, 1024));
    hipLaunchKernelGGL(route_zero_kernel, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<uint32_t*>(p.counts), words);
  }
  if (p.T > 0)
    hipLaunchKernelGGL(route_topk_kernel, dim3((p.T + 3) / 4 + std::min(p.prep_rows, kMaxPrepBlocks)), dim3(256), 0,
                       stream, p);
  if (static_cast<int64_t>(p.T) * p.k <= kPermuteCountPairs && reinterpret_cast<uintptr_t>(p.ids) % 16 == 0) {
    hipLaunchKernelGGL(route_permute_kernel<true>, dim3((p.E + 3) / 4), dim3(256), 0, stream, p);
    return;
  }
  hipLaunchKernelGGL(route_count_kernel, dim3((p.E + 3) / 4), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(route_permute_kernel<false>, dim3((p.E + 3) / 4), dim3(256), 0, stream, p);
}

void launch_table_prep(const TableParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(table_prep_kernel, dim3(1 + p.T), dim3(512), 0, stream, p);
}

void launch_combine(const float* y, const int32_t* inv, int T, int k, int H, int has_shared, const float* wts,
                    const float* gate, uint16_t* out, hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel<float>, dim3(T, (H + 511) / 512), dim3(64), 0, stream, y, inv, T, k, H, has_shared,
                     wts, gate, out);
}

void launch_combine_bf16(const uint16_t* y, const int32_t* inv, int T, int k, int H, int has_shared, uint16_t* out,
                         hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel<uint16_t>, dim3(T, (H + 511) / 512), dim3(64), 0, stream, y, inv, T, k, H,
                     has_shared, nullptr, nullptr, out);
}

void launch_combine_parts(const float* ypart, const int2* row_seg, int rps, const int32_t* inv, int T, int k, int H,
                          int has_shared, const float* wts, const float* gate, uint16_t* out, hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_parts_kernel, dim3(T, (H + 255) / 256), dim3(512), 0, stream, ypart, row_seg, rps, inv, T,
                     k, H, has_shared, wts, gate, out);
}

}  // namespace dflash
