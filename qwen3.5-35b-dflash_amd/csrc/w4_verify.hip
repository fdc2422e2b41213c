// Verify-block W4A16 expert GEMMs (T <= 32 tokens): the routed-MoE layer of a
// DFlash verify block in four launches (router front, gate/up, down, combine).
//
// Work decomposition.  A unit is one pass (up to 16 slot rows of an expert
// segment or of the shared expert) times one strip of 2 x 16 weight rows over
// the full reduction length K.  Units form one list (pass-major); each
// workgroup takes an equal contiguous range of it, and inside the workgroup the
// range's k-blocks (128 columns of K) are split over the 8 waves in fixed shares
// (wave_start: 7 parts for each of waves 0-3 to 5 for each of waves 4-7, which
// share their SIMDs with the older waves).  A unit whose k-blocks fall to several waves
// is finished by the wave holding its last k-block, after the others left their
// partial sums in LDS (summed in wave order: the result does not depend on
// timing).
//
// Per k-block a lane issues two 16-byte weight loads (16 rows x 64 bytes per
// tile) and one group scale (group size 128 or 256: its row's in tile 0 for
// lanes 0-31, in tile 1 for lanes 32-63, swapped across the halves before use),
// ahead of the k-block it computes.  Each k-block is
// dequantised in registers (bf16 136+q), multiplied on
// v_mfma_f32_16x16x32_bf16 against A fragments read from LDS, started from
// -136*sum(a) and scaled.
//
// Prologues and epilogues:
//   gate/up : optionally routes the block itself (top-k of the fp32 logits per
//             token, counts, scans and the stable permutation in LDS: every
//             workgroup derives the same work list, workgroup 0 also writes the
//             routing outputs and the down launch's work table), stages x,
//             its -136*sum terms and the token of every slot row in LDS; the
//             epilogue writes h = silu(g)*u in bf16 and its -136*sum per 16
//             columns.
//   down    : stages the h rows of its passes and their -136*sum partials
//             (chunks that fit in LDS), all by direct-to-LDS loads; the epilogue
//             writes the unweighted y = h . Wd^T in fp32, which the combine
//             kernel scales by the routing weights and sums over slots.
//             (Combining inside this launch would need an agent-scope release
//             per workgroup, an L2 write-back on every XCD, which measured
//             slower than one more launch.)
//   linear  : the raw x rows of a plain qlinear, converted while staged (one
//             launch per qlinear); one pass per 16 rows.  Used for outputs wider
//             than the small-block kernels take (the LM head) and for 17-32 rows
//             above N = 8192.
//   gate/up with SplitDown (opt-in, VerifyParams::fuse_down): the down GEMM of
//             the workgroup's own h columns runs in the same launch, split over K;
//             fp32 partial rows for combine_parts_kernel.
//
// Semantics per mode (reference citations):
//   kModeLinear : y = x . dequant(W)^T, bf16 out                 (fused/quantization.py:154-165)
//   kModeGateUp : h = silu(x.Wg^T) * (x.Wu^T), gate rows first   (reference/fused_ops.py:170-171)
//   kModeDown   : y = h . Wd^T, fp32 (the combine weighs it)   (fused/quantization.py:196-199)
//   routing     : top-k, renormalised softmax, stable permutation (reference/fused_ops.py:160-164,
//                                                                   fused/quantization.py:184-191)
#include <algorithm>

#include "topk.h"

namespace dflash {
namespace {

constexpr int kVWaves = 8;
constexpr int kVThreads = kVWaves * 64;
constexpr int kVDepthAll = 3;    // k-blocks per wave in flight (loads run 2 ahead, across units)
// Waves w and w + 4 share a SIMD, where the older wave w wins issue arbitration: with equal
// shares, waves 4-7 finished their k-blocks 16% later (gate/up and down alike), the tail
// running on half the waves.  Waves 0-3 take kVShareOld parts of the k-blocks to every
// kVShareYoung of waves 4-7 (4:3 measured best of 1:1, 7:6, 4:3, 11:8: -0.6 us per kernel; with
// one scale load per k-block, 7:5 against 4:3 and 3:2: T=16 layer -0.3 to -0.4 us on two boxes).
constexpr int kVShareOld = 7, kVShareYoung = 5;

// First k-block of wave w when a workgroup's range of n k-blocks is split by those shares.
__device__ __forceinline__ int wave_start(int n, int w) {
  const int cum = kVShareOld * min(w, 4) + kVShareYoung * max(w - 4, 0);
  return (n * cum) / (4 * (kVShareOld + kVShareYoung));
}
constexpr int kVStrip = 32;      // output columns per down/linear unit (and per combine strip)
constexpr int kVLds = 158 * 1024;  // one persistent workgroup per CU
// Rows of the split-K down's h copy hold I + kHPad columns: the pad (3 quarters, zero) lets a
// chunk of 4 quarters that runs past the row read zero h without a bounds select.
constexpr int kHPad = 96;


typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ void dma16(buf_rsrc r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, static_cast<int>(voff), static_cast<int>(soff), 0, 0);
}
__device__ __forceinline__ void dma4(buf_rsrc r, void* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 4, static_cast<int>(voff), static_cast<int>(soff), 0, 0);
}

// XCD id of the executing workgroup (hardware register).
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xFu;
}


// Phase timestamps of the profiling build (compiled with DFLASH_TIMELINE, loaded only by
// timeline.py; the product library has none of it): per separate gate/up (mode 1) or down
// (mode 2) launch and workgroup, 16 slots of s_memrealtime ticks (100 MHz): 0 start, 1 pass
// count known (after in-kernel routing), 2 first chunk staged, 3 the XCD id (not a time),
// 4 + w wave w's k-loop done, 12 the workgroup's partial sums exchanged, 13 end.
#ifdef DFLASH_TIMELINE
constexpr int kTlWorkgroups = 1024, kTlSlots = 16;
__device__ unsigned long long g_timeline_verify[2 * kTlWorkgroups * kTlSlots];
__device__ __forceinline__ void tl_mark(int mode, int slot, bool lane0_of_every_wave = false) {
  const bool writer = lane0_of_every_wave ? (threadIdx.x & 63) == 0 : threadIdx.x == 0;
  if ((mode == kModeGateUp || mode == kModeDown) && writer && blockIdx.x < kTlWorkgroups) {
    unsigned long long* row = g_timeline_verify + ((mode - 1) * kTlWorkgroups + blockIdx.x) * kTlSlots;
    row[slot] = __builtin_amdgcn_s_memrealtime();
    if (slot == 0) row[3] = xcc_id();
  }
}
#else
__device__ __forceinline__ void tl_mark(int, int, bool = false) {}
#endif

// Opaque to the optimiser: the value must exist in registers at this point.
__device__ __forceinline__ void pin(f32x4& v) { asm volatile("" : "+v"(v)); }

// Split-K down: the partial y rows of row r of pass P.  Workgroup b of G takes units
// [floor(U b / G), floor(U (b + 1) / G)) of the U = passes * strips unit list, so unit x lies
// in workgroup floor((G (x + 1) - 1) / U); pass P's first and last units give its first and
// last workgroups, and workgroup b writes the partial of (b, P) at row rps * (b + P) + r
// (rps: rows per segment, min(16, T)).  Returns (first partial row, partial count).
__device__ __forceinline__ int2 part_rows(const VerifyParams& vp, int P, int r, int total_passes) {
  const int64_t S = vp.g.strips, G = gridDim.x, U = static_cast<int64_t>(total_passes) * S;
  const int b0 = static_cast<int>((G * (P * S + 1) - 1) / U);
  const int b1 = static_cast<int>((G * (P + 1) * S - 1) / U);
  return make_int2(vp.part_rps * (b0 + P) + r, b1 - b0 + 1);
}

// ---------------------------------------------------------------------------
// In-kernel routing of the block (512 threads, T <= 32, E <= 1024).  Leaves
// every pass descriptor in pdesc and the token of every slot row in tok;
// returns the number of passes.  Workgroup 0 writes the routing outputs
// (ids, weights, perm, inv, offsets) and the work table the down launch reads.
__device__ __forceinline__ int route_block(const VerifyParams& vp, char* lds, int4* pdesc, int* tok) {
  const int T = vp.g.T, E = vp.E, k = vp.g.top_k;
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  const int tpad = (T + 3) & ~3;
  const int epad = (E + 3) & ~3;
  const bool out = blockIdx.x == 0;
  int* cnt = reinterpret_cast<int*>(lds + vp.lds_scratch);   // [epad]
  float* rw = reinterpret_cast<float*>(cnt + epad);          // [T*k]
  int* wtot = reinterpret_cast<int*>(rw + ((T * k + 3) & ~3));  // [3][8]
  uint32_t* map_words = reinterpret_cast<uint32_t*>(wtot + 24);  // [E][tpad] bytes
  uint8_t* map = reinterpret_cast<uint8_t*>(map_words);
  for (int i = tid; i < epad; i += kVThreads) cnt[i] = 0;
  for (int i = tid; i < (E * tpad) / 4; i += kVThreads) map_words[i] = 0u;
  __syncthreads();
  // tokens 2 * wave + {0, 1} (+ 16 for T > 16), two per wave at a time
  for (int t0 = 2 * wave; t0 < T; t0 += 2 * kVWaves) {
    const bool live_b = t0 + 1 < T;
    int id[2];
    float w[2];
    topk2_any(vp.logits + static_cast<int64_t>(t0) * E, vp.logits + static_cast<int64_t>(live_b ? t0 + 1 : t0) * E,
              live_b, E, k, id, w);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int t = t0 + r;
      if (lane < k && (r == 0 || live_b)) {
        rw[t * k + lane] = w[r];
        atomicAdd(&cnt[id[r]], 1);
        map[id[r] * tpad + t] = static_cast<uint8_t>(lane + 1);
        if (out) {
          vp.ids[t * k + lane] = id[r];
          vp.wts[t * k + lane] = w[r];
        }
      }
    }
  }
  __syncthreads();
  // exclusive scans over experts (two per thread): segment start, hit index, first pass
  int c[2], np[2], a = 0, b = 0, pc = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = 2 * tid + j;
    c[j] = e < E ? cnt[e] : 0;
    np[j] = passes_for(c[j], 16);
    a += c[j];
    b += c[j] > 0 ? 1 : 0;
    pc += np[j];
  }
  int ia = a, ib = b, ic = pc;
  for (int o = 1; o < 64; o <<= 1) {
    const int ua = __shfl_up(ia, o, 64), ub = __shfl_up(ib, o, 64), uc = __shfl_up(ic, o, 64);
    if (lane >= o) {
      ia += ua;
      ib += ub;
      ic += uc;
    }
  }
  if (lane == 63) {
    wtot[wave] = ia;
    wtot[8 + wave] = ib;
    wtot[16 + wave] = ic;
  }
  __syncthreads();
  int ba = 0, bb = 0, bc = 0, hits = 0, routed = 0;
#pragma unroll
  for (int i = 0; i < kVWaves; ++i) {
    const int va = wtot[i], vb = wtot[8 + i], vc = wtot[16 + i];
    if (i < wave) {
      ba += va;
      bb += vb;
      bc += vc;
    }
    hits += vb;
    routed += vc;
  }
  int off = ba + ia - a, pass = bc + ic - pc;
  (void)bb;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = 2 * tid + j;
    if (e < E) {
      if (out) vp.offsets[e] = off;
      for (int i = 0; i < np[j]; ++i) {
        const int4 d = make_int4(e, off, c[j], 16 * i);
        pdesc[pass + i] = d;
        if (out) vp.pass_table_out[pass + i] = d;
      }
    }
    off += c[j];
    pass += np[j];
  }
  const int shared_passes = vp.g.has_shared ? passes_for(T, 16) : 0;
  if (tid < shared_passes) {
    const int4 d = make_int4(-1, 0, T, 16 * tid);
    pdesc[routed + tid] = d;
    if (out) vp.pass_table_out[routed + tid] = d;
  }
  if (out && tid == 0) {
    vp.offsets[E] = T * k;
    vp.meta_out[0] = hits;
    vp.meta_out[1] = routed + shared_passes;
  }
  // stable ranks: the thread of expert e walks its slot-map row (tokens ascending)
  off = ba + ia - a;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int e = 2 * tid + j;
    if (c[j] > 0) {
      int pos = off;
      const uint32_t* row = map_words + (e * tpad) / 4;
      for (int q = 0; q < tpad / 4; ++q) {
        uint32_t word = row[q];
        while (word) {
          const int byte = __builtin_ctz(word) >> 3;
          const int t = q * 4 + byte;
          const int flat = t * k + static_cast<int>((word >> (byte * 8)) & 0xFFu) - 1;
          tok[pos] = t;
          if (out) {
            vp.perm[pos] = flat;
            vp.inv[flat] = pos;
            vp.slot_w_out[pos] = rw[flat];
            vp.tok_out[pos] = t;
          }
          ++pos;
          word &= ~(0xFFu << (byte * 8));
        }
      }
    }
    off += c[j];
  }
  __syncthreads();
  return routed + shared_passes;
}

// ---------------------------------------------------------------------------
// Half-wave-parallel routing of the block (E <= 256, k <= 16, T <= 32): one
// 32-lane half-wave per token (two tokens per wave, 16 per token pass), so the
// selection rounds are DPP reductions inside the half-wave with no LDS or scalar
// round trips, and all eight waves work on a 16-token block.  Its barriers order
// LDS only: the activation staging issued before it stays in flight.  Lane r of a
// half-wave holds the keys of experts kPR r .. kPR r + kPR - 1 (16-byte loads), so
// expert ids grow with the lane and, inside a lane, with the key index.  Same
// contract as route_block.
template <int kPR>
struct RowKeys {
  uint32_t key[2][kPR];  // token passes 0 and 1 (tokens 16..31)
};

// Max (kMin false) or min over the 16 lanes of a row, in every lane of the row.
template <bool kMin>
__device__ __forceinline__ uint32_t row_reduce(uint32_t v) {
  auto f = [](uint32_t a, uint32_t b) { return kMin ? (a < b ? a : b) : (a > b ? a : b); };
  v = f(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false)));   // quad_perm [1,0,3,2]
  v = f(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false)));   // quad_perm [2,3,0,1]
  v = f(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xF, 0xF, false)));  // row_half_mirror
  v = f(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xF, 0xF, false)));  // row_mirror
  return v;
}

// Max (kMin false) or min over the 32 lanes of a half-wave, in every lane of it:
// the row result, rows 1 and 3 folding in lane 15 of rows 0 and 2 (row_bcast:15;
// rows 0 and 2 keep their own), then lanes 31 and 63 broadcast.
template <bool kMin>
__device__ __forceinline__ uint32_t half_reduce(uint32_t v) {
  v = row_reduce<kMin>(v);
  const uint32_t o = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x142, 0xA, 0xF, false));
  v = kMin ? (v < o ? v : o) : (v > o ? v : o);
  const uint32_t lo = __builtin_amdgcn_readlane(v, 31), hi = __builtin_amdgcn_readlane(v, 63);
  return (threadIdx.x & 32) ? hi : lo;
}

// Largest of a lane's keys, and the lowest index holding a given key (kPR if none).
template <int kPR>
__device__ __forceinline__ uint32_t keys_max(const uint32_t (&k)[kPR]) {
  uint32_t m[kPR];
#pragma unroll
  for (int i = 0; i < kPR; ++i) m[i] = k[i];
#pragma unroll
  for (int w = 1; w < kPR; w *= 2)
#pragma unroll
    for (int i = 0; i + w < kPR; i += 2 * w) m[i] = m[i] > m[i + w] ? m[i] : m[i + w];
  return m[0];
}
template <int kPR>
__device__ __forceinline__ uint32_t keys_first(const uint32_t (&k)[kPR], uint32_t v) {
  uint32_t m[kPR];
#pragma unroll
  for (int i = 0; i < kPR; ++i) m[i] = k[i] == v ? static_cast<uint32_t>(i) : static_cast<uint32_t>(kPR);
#pragma unroll
  for (int w = 1; w < kPR; w *= 2)
#pragma unroll
    for (int i = 0; i + w < kPR; i += 2 * w) m[i] = m[i] < m[i + w] ? m[i] : m[i + w];
  return m[0];
}

__device__ __forceinline__ float row_sum_f32(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

// The keys of this lane's tokens (2 * wave + half-wave + 16 * pass); issued first
// so the caller's staging loads queue behind them.
template <int kPR>
__device__ __forceinline__ RowKeys<kPR> route_rows_load(const VerifyParams& vp) {
  const int T = vp.g.T, E = vp.E;
  const int r = threadIdx.x & 31;
  RowKeys<kPR> k;
#pragma unroll
  for (int tp = 0; tp < 2; ++tp) {
    const int t = 2 * (threadIdx.x >> 6) + ((threadIdx.x >> 5) & 1) + 16 * tp;
    float v[kPR];
    if (tp == 0 || T > 16) {
      // tokens past T repeat the last one (never recorded); the buffer resource reads 0 past E
      const buf_rsrc lr = make_rsrc(vp.logits + static_cast<int64_t>(min(t, T - 1)) * E, static_cast<uint32_t>(E) * 4);
#pragma unroll
      for (int i = 0; i < kPR; i += 4) {
        const uint4 q = buf_load16(lr, static_cast<uint32_t>((kPR * r + i) * 4), 0);
        v[i] = __uint_as_float(q.x);
        v[i + 1] = __uint_as_float(q.y);
        v[i + 2] = __uint_as_float(q.z);
        v[i + 3] = __uint_as_float(q.w);
      }
    }
#pragma unroll
    for (int i = 0; i < kPR; ++i) {
      const int e = kPR * r + i;
      // sortable keys stay below 0xFF800001; 0 marks no expert (or a taken one)
      k.key[tp][i] = (tp == 0 || T > 16) && e < E ? sortable_key(v[i]) + 1u : 0u;
    }
  }
  return k;
}

template <int kPR>
__device__ __forceinline__ int route_rows(const VerifyParams& vp, RowKeys<kPR> keys, char* lds, int4* pdesc, int* tok) {
  const int T = vp.g.T, E = vp.E, k = vp.g.top_k;
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id(), r = lane & 31;
  const int t0 = 2 * wave + (lane >> 5);  // token of pass 0; pass 1 adds 16
  const int tpad = (T + 3) & ~3;
  const bool out = blockIdx.x == 0;
  int* cnt = reinterpret_cast<int*>(lds + vp.lds_scratch);        // [256] tokens per expert, then its first slot row
  float* rw = reinterpret_cast<float*>(cnt + 256);                // [T*k] routing weight of every flat pair
  int* rid = reinterpret_cast<int*>(rw + 512);                    // [T*k] expert of every flat pair
  int* wtot = rid + 512;                                          // [3][4] wave totals: slot rows, passes, hits
  int* pfirst = wtot + 12;                                        // [256] first pass of every expert
  uint32_t* map_words = reinterpret_cast<uint32_t*>(pfirst + 256);  // [E][tpad] bytes: slot + 1, or 0
  uint8_t* map = reinterpret_cast<uint8_t*>(map_words);
  for (int i = tid; i < 256; i += kVThreads) cnt[i] = 0;
  for (int i = tid; i < (E * tpad) / 4; i += kVThreads) map_words[i] = 0u;

  // ---- k selection rounds per half-wave: largest key, lowest expert id among equal keys;
  // lane s of the half-wave keeps slot s.  Both token passes share the rounds.
  const int npass = T > 16 ? 2 : 1;
  int my_id[2] = {0, 0};
  uint32_t my_key[2] = {0, 0}, top_key[2] = {0, 0};
  if (2 * wave < T) {  // waves whose tokens are all past T stay off the VALU
    for (int s = 0; s < k; ++s) {
#pragma unroll
      for (int tp = 0; tp < 2; ++tp) {
        if (tp < npass) {
          const uint32_t rm = half_reduce<false>(keys_max<kPR>(keys.key[tp]));
          const uint32_t first = keys_first<kPR>(keys.key[tp], rm);
          // expert ids grow with the lane, so the lowest lane of the half-wave that holds rm
          // holds the lowest id among the equal keys (every half-wave has one: rm is its max)
          const uint64_t holds = __ballot(first < kPR);
          const int l0 = __builtin_ctz(static_cast<uint32_t>(holds));
          const int l1 = 32 + __builtin_ctz(static_cast<uint32_t>(holds >> 32));
          const uint32_t e0 = static_cast<uint32_t>(kPR * l0) + __builtin_amdgcn_readlane(first, l0);
          const uint32_t e1 = static_cast<uint32_t>(kPR * (l1 - 32)) + __builtin_amdgcn_readlane(first, l1);
          const uint32_t e = (threadIdx.x & 32) ? e1 : e0;
          const uint32_t ie = e - static_cast<uint32_t>(kPR * r);  // wraps past kPR unless this lane's
#pragma unroll
          for (int i = 0; i < kPR; ++i) keys.key[tp][i] = ie == static_cast<uint32_t>(i) ? 0u : keys.key[tp][i];
          if (s == 0) top_key[tp] = rm - 1u;
          if (r == s) {
            my_id[tp] = static_cast<int>(e);
            my_key[tp] = rm - 1u;
          }
        }
      }
    }
  }
  // renormalised softmax over the selected logits (the full-softmax denominator cancels);
  // the k <= 16 slots sit in the first row of the half-wave
  float w[2];
#pragma unroll
  for (int tp = 0; tp < 2; ++tp) {
    const float ex = r < k ? expf(key_to_float(my_key[tp]) - key_to_float(top_key[tp])) : 0.f;
    w[tp] = ex / row_sum_f32(ex);
  }
  lds_barrier();  // the counters are cleared
#pragma unroll
  for (int tp = 0; tp < 2; ++tp) {
    const int t = t0 + 16 * tp;
    if (t < T && r < k) {
      rw[t * k + r] = w[tp];
      rid[t * k + r] = my_id[tp];
      atomicAdd(&cnt[my_id[tp]], 1);
      map[my_id[tp] * tpad + t] = static_cast<uint8_t>(r + 1);
      if (out) {
        vp.ids[t * k + r] = my_id[tp];
        vp.wts[t * k + r] = w[tp];
      }
    }
  }
  lds_barrier();

  // ---- exclusive scans over experts (threads 0..255, one expert each): first slot row, first pass
  const int c = tid < E ? cnt[tid] : 0;
  const int np = passes_for(c, 16);
  const int ia = wave_inclusive_scan(c), ic = wave_inclusive_scan(np);
  const int wh = __builtin_popcountll(__ballot(c > 0));
  if (tid < 256 && lane == 63) {
    wtot[wave] = ia;
    wtot[4 + wave] = ic;
    wtot[8 + wave] = wh;
  }
  lds_barrier();
  int ba = 0, bc = 0, hits = 0, routed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < wave) {
      ba += wtot[i];
      bc += wtot[4 + i];
    }
    routed += wtot[4 + i];
    hits += wtot[8 + i];
  }
  const int off = ba + ia - c, p0 = bc + ic - np;
  if (tid < E) {
    pfirst[tid] = p0;
    if (out) vp.offsets[tid] = off;
    for (int i = 0; i < np; ++i) {
      const int4 d = make_int4(tid, off, c, 16 * i);
      pdesc[p0 + i] = d;
      if (out) vp.pass_table_out[p0 + i] = d;
    }
  }
  const int shared_passes = vp.g.has_shared ? passes_for(T, 16) : 0;
  if (tid < shared_passes) {
    const int4 d = make_int4(-1, 0, T, 16 * tid);
    pdesc[routed + tid] = d;
    if (out) vp.pass_table_out[routed + tid] = d;
  }
  if (out && tid == 0) {
    vp.offsets[E] = T * k;
    vp.meta_out[0] = hits;
    vp.meta_out[1] = routed + shared_passes;
  }
  const int total = routed + shared_passes;
  if (out && vp.fuse_down && vp.g.has_shared && tid < T) vp.row_seg[T * k + tid] = part_rows(vp, routed + (tid >> 4), tid & 15, total);
  lds_barrier();  // every count is read: cnt becomes each expert's first slot row
  if (tid < E) cnt[tid] = off;
  lds_barrier();
  // ---- stable permutation: pair (token tt, slot) goes to its expert's segment after the
  // expert's tokens below tt (nonzero bytes of the slot-map row before column tt)
  for (int i = tid; i < T * k; i += kVThreads) {
    const int tt = i / k;
    const int e = rid[i];
    const uint32_t* row = map_words + (e * tpad) / 4;
    int before = 0;
    for (int q = 0; q * 4 < tt; ++q) {
      uint32_t word = row[q];
      const int lim = tt - q * 4;  // columns of this word below tt (>= 1)
      if (lim < 4) word &= (1u << (8 * lim)) - 1u;
      const uint32_t zero_hi = ~(((word & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | word | 0x7F7F7F7Fu);  // 0x80 per zero byte
      before += 4 - __popc(zero_hi);
    }
    const int pos = cnt[e] + before;
    tok[pos] = tt;
    if (out) {
      if (vp.fuse_down) vp.row_seg[pos] = part_rows(vp, pfirst[e] + (before >> 4), before & 15, total);
      vp.perm[pos] = i;
      vp.inv[i] = pos;
      vp.slot_w_out[pos] = rw[i];
      vp.tok_out[pos] = tt;
    }
  }
  lds_barrier();
  return routed + shared_passes;
}

}  // namespace

// x rows (octet-interleaved) in 1 KB blocks and their -136*sum terms, by direct-to-LDS loads
template <int kMode, int kNKB>
__device__ __forceinline__ void stage_x(const VerifyParams& vp, char* lds) {
  const W4StreamParams& p = vp.g;
  constexpr int kK = kNKB * 128;
  constexpr int kRS = kK * 2 + 16;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id();
  uint8_t* lds_a = reinterpret_cast<uint8_t*>(lds + vp.lds_a);
  float* lds_neg = reinterpret_cast<float*>(lds + vp.lds_neg);
  const int rows = kMode == kModeLinear ? p.M : p.T;
  const buf_rsrc xr = make_rsrc(p.act, static_cast<uint32_t>(rows) * kK * 2);
  constexpr int kBlk = kK / 512;  // 1 KB blocks per row
  for (int i = wave; i < rows * kBlk; i += kVWaves) {
    const int r = i / kBlk, bl = i - r * kBlk;
    dma16(xr, lds_a + r * kRS + bl * 1024, static_cast<uint32_t>(lane * 16),
          static_cast<uint32_t>((r * kK + bl * 512) * 2));
  }
  const buf_rsrc nr = make_rsrc(p.act_neg, static_cast<uint32_t>(rows) * kNKB * 4);
  for (int i = wave; i * 64 < rows * kNKB; i += kVWaves)
    dma4(nr, lds_neg + i * 64, static_cast<uint32_t>(lane * 4), static_cast<uint32_t>(i * 256));
}

// Linear mode: the caller's raw bf16 x rows, converted while they are staged (the
// activation prep the other paths run as a launch of its own): every 16-byte
// octet to the octet-interleaved order of the MFMA A operand, and -136*sum per
// 128-column block (per-chunk sums in the prep kernel's order).  A thread issues
// all of its loads (at most 16) before it uses any.
template <int kNKB>
__device__ __forceinline__ void stage_x_raw(const VerifyParams& vp, char* lds) {
  const W4StreamParams& p = vp.g;
  constexpr int kK = kNKB * 128, kRS = kK * 2 + 16, kChunks = kK / 8;
  constexpr int kPer = kNKB < 16 ? kNKB : 16;  // rows * kChunks <= 512 * kPer (M <= 32, or 16 at K = 4096)
  uint8_t* lds_a = reinterpret_cast<uint8_t*>(lds + vp.lds_a);
  float* lds_neg = reinterpret_cast<float*>(lds + vp.lds_neg);
  const int total = p.M * kChunks;
  const buf_rsrc xr = make_rsrc(p.act, static_cast<uint32_t>(total) * 16);
  uint4 v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    v[j] = buf_load16(xr, static_cast<uint32_t>(threadIdx.x + kVThreads * j) * 16, 0);  // 0 past the rows
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = threadIdx.x + kVThreads * j;  // 16-lane rows hold the 16 chunks of one 128-column block
    if (i < total) {
      const int r = i / kChunks, c = i - r * kChunks;
      uint4 o;  // natural pairs (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
      o.x = (v[j].x & 0xFFFFu) | (v[j].z << 16);
      o.y = (v[j].x >> 16) | (v[j].z & 0xFFFF0000u);
      o.z = (v[j].y & 0xFFFFu) | (v[j].w << 16);
      o.w = (v[j].y >> 16) | (v[j].w & 0xFFFF0000u);
      *reinterpret_cast<uint4*>(lds_a + r * kRS + c * 16) = o;
      const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) sum += __uint_as_float(w[q] << 16) + __uint_as_float(w[q] & 0xFFFF0000u);
      sum = row16_sum(sum);
      if ((c & 15) == 0) lds_neg[r * kNKB + (c >> 4)] = -kDequantOffset * sum;
    }
  }
}

// Workgroup 0 of a gate/up launch that routed the block: the down launch's plan per
// workgroup b (its pass count and the descriptors of the first two passes of its unit
// range, 3 int4), so the down prologue needs one load before its first weights.
__device__ __forceinline__ void write_down_plan(const VerifyParams& vp, const int4* pdesc, int total) {
  if (!vp.down_plan || blockIdx.x != 0 || total <= 0) return;
  const int64_t units = static_cast<int64_t>(total) * vp.down_strips;
  for (int b = threadIdx.x; b < vp.down_grid; b += kVThreads) {
    const int ub = static_cast<int>(units * b / vp.down_grid);
    const int P0 = min(ub / vp.down_strips, total - 1), P1 = min(P0 + 1, total - 1);
    int4* o = vp.down_plan + 3 * b;
    o[0] = make_int4(total, P0, 0, 0);
    o[1] = pdesc[P0];
    o[2] = pdesc[P1];
  }
}

// Passes of the launch.  The gate/up launch routes the block here when asked
// (its x staging is issued first and stays in flight meanwhile).
template <int kMode, int kNKB>
__device__ __forceinline__ int verify_passes(const VerifyParams& vp, char* lds) {
  int* lds_tok = reinterpret_cast<int*>(lds + vp.lds_tok);
  int4* lds_pdesc = reinterpret_cast<int4*>(lds + vp.lds_pdesc);
  if (kMode == kModeGateUp && vp.route == 2) {
    if (vp.fuse_down) {  // h of the workgroup's unit range, zero outside it (the routing's barriers order this)
      uint4* h = reinterpret_cast<uint4*>(lds + vp.lds_h);
      for (int i = threadIdx.x; i < (2 * 16 * (vp.dI + kHPad) * 2) / 16; i += kVThreads) h[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (vp.E <= 128) {
      const RowKeys<4> keys = route_rows_load<4>(vp);
      stage_x<kMode, kNKB>(vp, lds);
      const int total = route_rows<4>(vp, keys, lds, lds_pdesc, lds_tok);
      write_down_plan(vp, lds_pdesc, total);
      return total;
    }
    const RowKeys<8> keys = route_rows_load<8>(vp);
    stage_x<kMode, kNKB>(vp, lds);
    const int total = route_rows<8>(vp, keys, lds, lds_pdesc, lds_tok);
    write_down_plan(vp, lds_pdesc, total);
    return total;
  }
  if (kMode == kModeGateUp && vp.route) {
    stage_x<kMode, kNKB>(vp, lds);
    const int total = route_block(vp, lds, lds_pdesc, lds_tok);
    write_down_plan(vp, lds_pdesc, total);
    return total;
  }
  if (kMode == kModeLinear) return (vp.g.M + 15) >> 4;
  if (kMode == kModeDown && vp.down_plan) return ld_const_int4(vp.down_plan, 3 * static_cast<int>(blockIdx.x)).x;
  return ld_const(vp.g.meta, 1);
}

// The streaming GEMM of one verify launch over `total_passes` passes: workgroup b takes the
// b-th of gridDim.x equal contiguous ranges of the unit list (linear mode: a strided share).
template <int kMode, int kNKB, typename ScaleT>
__device__ __forceinline__ void verify_gemm(const VerifyParams& vp, char* lds, const int total_passes) {
  const W4StreamParams& p = vp.g;
  constexpr int kK = kNKB * 128;
  constexpr int kRS = kK * 2 + 16;                  // LDS row stride (bytes) of an activation row
  constexpr int kTileRows = kMode == kModeGateUp ? 16 : 32;
  // K = 4096 linear (the attention and GDN output projections): one k-block more in flight
  // (8.95 -> 8.65 us per projection; the other instances measured best at kVDepthAll)
  constexpr int kVDepth = kMode == kModeLinear && kNKB == 32 ? kVDepthAll + 1 : kVDepthAll;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id(), lr = lane & 15, kq = lane >> 4;
  const int tid = threadIdx.x;

  uint8_t* lds_a = reinterpret_cast<uint8_t*>(lds + vp.lds_a);
  float* lds_neg = reinterpret_cast<float*>(lds + vp.lds_neg);
  int* lds_tok = reinterpret_cast<int*>(lds + vp.lds_tok);
  int4* lds_pdesc = reinterpret_cast<int4*>(lds + vp.lds_pdesc);
  float* lds_hpart = reinterpret_cast<float*>(lds + vp.lds_wgt);  // down: raw -136*sum partials of the h rows
  f32x4* lds_part = reinterpret_cast<f32x4*>(lds + vp.lds_part);  // [wave][2][64]

  const int strips = p.strips;
  const int rank = static_cast<int>(blockIdx.x), ranks = static_cast<int>(gridDim.x);
  // 32-bit unit arithmetic: every wave of the workgroup runs this prologue on the CU's one
  // scalar unit, where a 64-bit division costs ~130 instructions (the host admits only shapes
  // with passes x strips x grid < 2^32)
  const uint32_t total_units = static_cast<uint32_t>(total_passes) * static_cast<uint32_t>(strips);
  // linear mode: workgroup b runs units b, b + G, b + 2G, ... (G = grid), so at any moment the
  // workgroups stream one contiguous window of the weights (contiguous ranges per workgroup
  // leave ~2048 streams a fixed stride apart, which streamed up to 10% slower); its virtual
  // range [ub, ue) gives the first U % G workgroups one unit more
  int ub, ue;
  if (kMode == kModeLinear) {
    const int G = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
    const int q = static_cast<int>(total_units / static_cast<uint32_t>(G));
    const int r = static_cast<int>(total_units - static_cast<uint32_t>(q) * static_cast<uint32_t>(G));
    ub = b * q + min(b, r);
    ue = ub + q + (b < r ? 1 : 0);
  } else {
    ub = static_cast<int>(total_units * static_cast<uint32_t>(rank) / static_cast<uint32_t>(ranks));
    ue = static_cast<int>(total_units * static_cast<uint32_t>(rank + 1) / static_cast<uint32_t>(ranks));
  }
  // the unit that virtual unit v of this workgroup's range stands for
  auto unit_of = [&](int v) {
    return kMode == kModeLinear ? (v - ub) * static_cast<int>(gridDim.x) + static_cast<int>(blockIdx.x) : v;
  };

  const int64_t rb = kK >> 1;                                      // packed bytes per weight row
  const int64_t second = kMode == kModeGateUp ? (p.N >> 1) : 16;   // row distance of tile 1
  // lane offset inside a 16-row tile and k-block stride: portable rows, or the tiled
  // layout's contiguous kilobyte per k-block (tile bases are the same in both)
  const uint32_t wlane = p.tiled ? static_cast<uint32_t>(lane * 16) : static_cast<uint32_t>(lr * rb + kq * 16);
  const uint32_t wkb = p.tiled ? 1024u : 64u;
  // group scales: K / G per row (G = 128 or 256: k-block kb uses group kb >> gshift)
  const int gshift = p.G == 256 ? 1 : 0, ng = kNKB >> gshift;
  const int slane = p.tiled ? lr : lr * ng;  // scale elements: [tile][group][16] or [row][group]
  const int skb = p.tiled ? 16 : 1;

  const int P_first = ub / strips, P_last = ue > ub ? (ue - 1) / strips : P_first - 1;
  // down with a plan: the descriptors of the first two passes came with the pass count
  int plan_p = -2;
  int4 plan_d0 = make_int4(0, 0, 0, 0), plan_d1 = plan_d0;
  if (kMode == kModeDown && vp.down_plan) {
    const int b3 = 3 * static_cast<int>(blockIdx.x);
    plan_p = ld_const_int4(vp.down_plan, b3).y;
    plan_d0 = ld_const_int4(vp.down_plan, b3 + 1);
    plan_d1 = ld_const_int4(vp.down_plan, b3 + 2);
  }
  auto lds_desc = [&](int i) -> int4 {
    const int4 v = lds_pdesc[i];
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                     __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
  };
  // descriptor of pass P before the chunk is staged
  auto early_desc = [&](int P) -> int4 {
    return P == plan_p ? plan_d0 : P == plan_p + 1 ? plan_d1 : ld_const_int4(p.pass_table, P);
  };
  // pass descriptors: all of them after in-kernel routing, else the chunk's (staged below)
  int pd_base = 0;
  auto pass_desc = [&](int j) -> int4 {
    if (kMode == kModeLinear) return make_int4(0, 0, p.M, j * 16);
    return lds_desc(j - pd_base);
  };

  const bool chunked = kMode == kModeDown || (kMode == kModeGateUp && vp.gather);
  const int chunk_passes = chunked ? vp.chunk_passes : max(P_last - P_first + 1, 1);
  for (int Pc = P_first; Pc <= P_last; Pc += chunk_passes) {
    const int Pc_end = min(P_last + 1, Pc + chunk_passes);
    const int cb = max(ub, Pc * strips), ce = min(ue, Pc_end * strips);
    if (Pc != P_first) lds_barrier();  // every wave is done with the previous chunk's rows
    bool staged = false;  // the chunk's rows and descriptors are in LDS

    // ---- this wave's k-blocks of the chunk: [g0, g1), its share of them
    const int n = (ce - cb) * kNKB;
    const int g0 = wave_start(n, wave), g1 = wave_start(n, wave + 1);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

    // epilogue of unit ur (chunk-relative) from its complete sums
    auto finish = [&](int ur, const int4& cd, const f32x4& t0, const f32x4& t1) {
      const int u = unit_of(cb + ur);
      const int P = u / strips, strip = u - P * strips;
      const int M = cd.z, m0 = cd.w;
      const bool shared = kMode != kModeLinear && cd.x < 0;
      const int row0 = strip * kTileRows;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 4 * kq + e;
        const bool valid = m < M;
        if (kMode == kModeLinear) {
          if (valid && p.out_f32) {  // fp32 output: the unrounded sums
            float* o = p.out_f32 + static_cast<int64_t>(m) * p.N + row0 + lr;
            o[0] = t0[e];
            o[16] = t1[e];
          } else if (valid) {
            uint16_t* o = p.out_bf16 + static_cast<int64_t>(m) * p.N + row0 + lr;
            o[0] = f32_to_bf16(t0[e]);
            o[16] = f32_to_bf16(t1[e]);
          }
        } else if (kMode == kModeGateUp) {
          const int inter = p.N >> 1;
          const uint16_t hb = f32_to_bf16(silu(t0[e]) * t1[e]);
          const int hrow = shared ? p.T * p.top_k + m : cd.y + m;
          if (valid) p.out_bf16[static_cast<int64_t>(hrow) * inter + octet_slot(row0 + lr)] = hb;
          if (valid && vp.fuse_down) {  // pass slot P - P_first of the split-K down (its range spans at most two)
            uint16_t* lh = reinterpret_cast<uint16_t*>(lds + vp.lds_h);
            lh[((P - P_first) * 16 + 4 * kq + e) * (inter + kHPad) + octet_slot(row0 + lr)] = hb;
          }
          const float part = row16_sum(valid ? bf16_to_f32(hb) : 0.f);
          if (valid && lr == 0) p.out_part[static_cast<int64_t>(hrow) * (inter >> 4) + strip] = -kDequantOffset * part;
        } else {
          if (valid) {  // unweighted: the combine applies the routing weight
            const int yrow = shared ? p.T * p.top_k + m : cd.y + m;
            float* o = p.out_f32 + static_cast<int64_t>(yrow) * p.N + row0 + lr;
            o[0] = t0[e];
            o[16] = t1[e];
          }
        }
      }
    };

    f32x4 head0 = zero, head1 = zero;
    int head_unit = -1;  // chunk-relative unit this wave ends but did not begin
    {
      // load cursor: next k-block to issue and the bases of its unit
      int lg = g0, l_ur = -1;
      const uint8_t* l_w = nullptr;
      const uint8_t* l_s = nullptr;
      auto unit_bases = [&](int ur) {
        const int u = unit_of(cb + ur);
        const int P = u / strips, strip = u - P * strips;
        // before the staging barrier the descriptor comes from the work table (s_load),
        // except after in-kernel routing, whose table is only in LDS
        const int4 d = staged || (kMode == kModeGateUp && vp.route) || kMode == kModeLinear
                           ? pass_desc(P) : early_desc(P);
        const bool shared = kMode != kModeLinear && d.x < 0;
        const int64_t e = kMode == kModeLinear ? 0 : d.x;
        const uint8_t* wbase = shared ? p.w_shared : p.w + e * p.w_stride;
        const uint8_t* sbase = static_cast<const uint8_t*>(shared ? p.s_shared : p.s) +
                               (shared ? 0 : e * p.s_stride * static_cast<int64_t>(sizeof(ScaleT)));
        const int64_t row0 = static_cast<int64_t>(strip) * kTileRows;
        l_w = wbase + row0 * rb;
        l_s = sbase + row0 * ng * static_cast<int64_t>(sizeof(ScaleT));
      };
      // ring of k-blocks in flight: two 16-byte weight loads and one group scale per lane
      uint4 wbuf[kVDepth][2];
      uint32_t sbuf[kVDepth][1];
      // Loads are issued unconditionally (past the range they repeat its last k-block, never
      // computed): a load under a branch would make the compiler drain the queue at the loop edge.
      auto issue = [&](uint4 (&dst)[2], uint32_t (&sdst)[1]) {
        const int lc = max(min(lg, g1 - 1), 0);
        const int ur = lc / kNKB, kb = lc - ur * kNKB;
        if (ur != l_ur) {
          l_ur = ur;
          unit_bases(ur);
        }
        dst[0] = *reinterpret_cast<const uint4*>(l_w + wlane + kb * wkb);
        dst[1] = *reinterpret_cast<const uint4*>(l_w + second * rb + wlane + kb * wkb);
        // one scale load per lane: lanes 0-31 take tile 0's, lanes 32-63 tile 1's (the lane's
        // row either way); the compute swaps the halves
        const ScaleT* sp = reinterpret_cast<const ScaleT*>(l_s) + slane + (kb >> gshift) * skb;
        sdst[0] = load_scale_bits(lane >= 32 ? sp + second * ng : sp);
        ++lg;
      };
      // the first k-blocks go out before the activations are staged (they do not depend on them)
#pragma unroll
      for (int i = 0; i + 1 < kVDepth; ++i) issue(wbuf[i], sbuf[i]);

      // ---- stage the chunk's activation rows and descriptors
      if (kMode == kModeGateUp && vp.gather) {
        // the chunk's pass descriptors; per pass its 16 slot rows' x rows (the token of a
        // routed row from the work table, clamped to the slot like the compute indexes) and
        // their -136*sum terms, all by direct-to-LDS loads
        pd_base = Pc;
        const int npass = Pc_end - Pc;
        const buf_rsrc tr = make_rsrc(p.pass_table, static_cast<uint32_t>(total_passes) * 16);
        if (wave == 0)
          dma16(tr, lds_pdesc, static_cast<uint32_t>(min(Pc + lane, total_passes - 1) * 16), 0);
        const buf_rsrc xr = make_rsrc(p.act, static_cast<uint32_t>(p.T) * kK * 2);
        constexpr int kBlk = kK / 512;
        for (int i = wave; i < npass * 16 * kBlk; i += kVWaves) {
          const int rr = i / kBlk, bl = i - rr * kBlk;
          const int4 d = early_desc(Pc + rr / 16);
          const int m = min(d.w + (rr & 15), d.z - 1);
          const int t = d.x < 0 ? m : ld_const(p.tok, d.y + m);
          dma16(xr, lds_a + rr * kRS + bl * 1024, static_cast<uint32_t>(lane * 16),
                static_cast<uint32_t>((t * kK + bl * 512) * 2));
        }
        // 64 terms per load: 64 / kNKB rows, all of one pass (kNKB divides 16 * kNKB)
        const buf_rsrc nr = make_rsrc(p.act_neg, static_cast<uint32_t>(p.T) * kNKB * 4);
        for (int i = wave; i * 64 < npass * 16 * kNKB; i += kVWaves) {
          const int4 d = early_desc(Pc + (i * 64) / (16 * kNKB));
          const int f = 64 * i + lane, rr = f / kNKB, kb = f - rr * kNKB;
          const int m = min(d.w + (rr & 15), d.z - 1);
          const int t = d.x < 0 ? m : p.tok[d.y + m];
          dma4(nr, lds_neg + 64 * i, static_cast<uint32_t>((t * kNKB + kb) * 4), 0);
        }
      } else if (kMode == kModeGateUp || kMode == kModeLinear) {
        if (!(kMode == kModeGateUp && vp.route)) {
          // the token of every slot row and the chunk's pass descriptors (in-kernel routing
          // left both in LDS and staged x already)
          pd_base = Pc;
          if (kMode == kModeGateUp) {
            for (int i = tid; i < Pc_end - Pc; i += kVThreads) lds_pdesc[i] = p.pass_table[Pc + i];
            for (int i = tid; i < p.T * p.top_k; i += kVThreads) lds_tok[i] = p.tok[i];
          }
          if (kMode == kModeLinear) stage_x_raw<kNKB>(vp, lds);
          else stage_x<kMode, kNKB>(vp, lds);
        }
      } else {
        // down: the chunk's pass descriptors, per pass its 16 h rows (clamped to the slot) and
        // their -136*sum partials (8 per k-block, one per 16 columns), all by direct-to-LDS
        // loads so the prologue's weight loads are not waited for ahead of them
        pd_base = Pc;
        const int npass = Pc_end - Pc;
        const buf_rsrc tr = make_rsrc(p.pass_table, static_cast<uint32_t>(total_passes) * 16);
        if (wave == 0)
          dma16(tr, lds_pdesc, static_cast<uint32_t>(min(Pc + lane, total_passes - 1) * 16), 0);
        const int hrows = p.T * p.top_k + (p.has_shared ? p.T : 0);
        const buf_rsrc hr = make_rsrc(p.act, static_cast<uint32_t>(hrows) * kK * 2);
        constexpr int kBlk = kK / 512;
        for (int i = wave; i < npass * 16 * kBlk; i += kVWaves) {
          const int rr = i / kBlk, bl = i - rr * kBlk;
          const int4 d = early_desc(Pc + rr / 16);
          const int base = d.x < 0 ? p.T * p.top_k : d.y;
          const int row = base + min(d.w + (rr & 15), d.z - 1);
          dma16(hr, lds_a + rr * kRS + bl * 1024, static_cast<uint32_t>(lane * 16),
                static_cast<uint32_t>((row * kK + bl * 512) * 2));
        }
        constexpr int kPartRow = kNKB * 8;  // partials per h row
        const buf_rsrc pr = make_rsrc(p.act_neg, static_cast<uint32_t>(hrows) * kPartRow * 4);
        for (int i = wave; i < npass * 2 * kNKB; i += kVWaves) {  // 64 partials per load, 2 kNKB per pass
          const int pass = i / (2 * kNKB), j = i - pass * 2 * kNKB;
          const int4 d = early_desc(Pc + pass);
          const int base = d.x < 0 ? p.T * p.top_k : d.y;
          const int f = 64 * j + lane, rr = f / kPartRow;
          const int row = base + min(d.w + rr, d.z - 1);
          dma4(pr, lds_hpart + pass * 16 * kPartRow + 64 * j,
               static_cast<uint32_t>((row * kPartRow + f % kPartRow) * 4), 0);
        }
      }
      wait_vmem();
      __syncthreads();
      if (kMode == kModeDown) {
        // -136*sum(h) per 128 columns from its 8 partials (same order as the partial writer's readers)
        for (int i = tid; i < (Pc_end - Pc) * 16 * kNKB; i += kVThreads) {
          const float4 u = *reinterpret_cast<const float4*>(lds_hpart + 8 * i);
          const float4 v = *reinterpret_cast<const float4*>(lds_hpart + 8 * i + 4);
          lds_neg[i] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w));
        }
        __syncthreads();
      }
      staged = true;
      if (Pc == P_first) tl_mark(kMode, 2);

      // compute state of the current unit
      int c_ur = -1, P = 0, a_off = 0;
      int4 cd = make_int4(0, 0, 0, 0);
      int n_idx[4] = {0, 0, 0, 0};
      bool began = false;
      f32x4 tot0 = zero, tot1 = zero;
      for (int gs = g0; gs < g1; gs += kVDepth) {
#pragma unroll
        for (int i = 0; i < kVDepth; ++i) {
          const int g = gs + i;
          issue(wbuf[(i + kVDepth - 1) % kVDepth], sbuf[(i + kVDepth - 1) % kVDepth]);
          if (g < g1) {
            const int ur = g / kNKB, kb = g - ur * kNKB;
            if (ur != c_ur) {
              c_ur = ur;
              const int u = unit_of(cb + ur);
              P = u / strips;
              cd = pass_desc(P);
              const int M = cd.z, m0 = cd.w;
              const int ma = min(m0 + lr, M - 1);
              int arow;
              if (chunked) arow = (P - Pc) * 16 + lr;
              else if (kMode == kModeGateUp) arow = cd.x < 0 ? ma : lds_tok[cd.y + ma];
              else arow = ma;
              a_off = arow * kRS + kq * 64;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int me = min(m0 + 4 * kq + e, M - 1);
                int nrow;
                if (chunked) nrow = (P - Pc) * 16 + 4 * kq + e;
                else if (kMode == kModeGateUp) nrow = cd.x < 0 ? me : lds_tok[cd.y + me];
                else nrow = me;
                n_idx[e] = nrow * kNKB;
              }
              began = kb == 0;
              tot0 = zero;
              tot1 = zero;
            }
            const uint8_t* ab = lds_a + a_off + kb * 256;
            uint4 a[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const uint4*>(ab + 16 * j);
            const f32x4 start = {lds_neg[n_idx[0] + kb], lds_neg[n_idx[1] + kb], lds_neg[n_idx[2] + kb],
                                 lds_neg[n_idx[3] + kb]};
            const uint4 (&w)[2] = wbuf[i];
            const uint32_t w0[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
            const uint32_t w1[4] = {w[1].x, w[1].y, w[1].z, w[1].w};
            f32x4 acc0 = start, acc1 = start;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              acc0 = mfma16x16x32(a[j], dequant8(w0[j]), acc0);
              acc1 = mfma16x16x32(a[j], dequant8(w1[j]), acc1);
            }
            // lanes 32 apart share a row: the swap gives every lane tile 0's scale of its row in
            // the first word and tile 1's in the second
            const auto sw = __builtin_amdgcn_permlane32_swap(sbuf[i][0], sbuf[i][0], false, false);
            tot0 += scale_value<ScaleT>(sw[0]) * acc0;
            tot1 += scale_value<ScaleT>(sw[1]) * acc1;
            // materialise the running sums here: left alone, the compiler sinks the
            // scale-accumulates and keeps every k-block's MFMA result live
            pin(tot0);
            pin(tot1);
            if (kb == kNKB - 1) {
              if (began) {
                finish(ur, cd, tot0, tot1);
              } else {
                // this wave ends a unit others began: finish it once their partials are in
                head0 = tot0;
                head1 = tot1;
                head_unit = ur;
              }
            } else if (g == g1 - 1) {
              // the unit continues in the next wave: leave the partial sums
              lds_part[(wave * 2) * 64 + lane] = tot0;
              lds_part[(wave * 2 + 1) * 64 + lane] = tot1;
            }
          }
          // keep the scheduler from hoisting later k-blocks' LDS reads and
          // dequantisation into this one (register pressure, not latency, binds)
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    tl_mark(kMode, 4 + wave, true);
    lds_barrier();  // partial sums of split units are in LDS
    tl_mark(kMode, 12);
    if (head_unit >= 0) {
      // sum the partials of the waves before this one that share the unit, in wave order
      const int gs = head_unit * kNKB;
      int wa = wave - 1;
      while (wa > 0 && wave_start(n, wa) > gs) --wa;
      f32x4 t0 = zero, t1 = zero;
      for (int w = wa; w < wave; ++w) {
        if (wave_start(n, w) < wave_start(n, w + 1)) {
          t0 += lds_part[(w * 2) * 64 + lane];
          t1 += lds_part[(w * 2 + 1) * 64 + lane];
        }
      }
      t0 += head0;
      t1 += head1;
      finish(head_unit, pass_desc(unit_of(cb + head_unit) / strips), t0, t1);
    }
  }
}

// Raw bits of one group scale through a buffer resource (byte offsets voff + soff).
template <typename ScaleT>
__device__ __forceinline__ uint32_t buf_scale_bits(buf_rsrc r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(ScaleT) == 4)
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff), static_cast<int>(soff), 0);
  else
    return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(voff), static_cast<int>(soff), 0);
}

// Split-K down GEMM of a routing gate/up launch (VerifyParams::fuse_down): after its gate/up
// units, this workgroup holds h for its unit range in LDS -- strips [sa, sb) of at most two
// passes -- and multiplies each pass's rows by the matching K-slice of the down bank, so the
// down weights stream inside this launch and no h leaves it.  Wave w owns output tiles
// (16 rows of H) [w H / 128, (w + 1) H / 128).  Work item = four of the wave's tiles and a
// chunk of four consecutive 32-column quarters of the range: per tile one 16-byte load per
// lane (lane quarter Q: quarter c + Q, row lane % 16; in the tiled layout a tile's quarters
// lie 256 bytes apart, so each load is one contiguous kilobyte), transposed so lane l holds
// k-octet l / 16 of each quarter's row l % 16 -- the B operand of one
// v_mfma_f32_16x16x32_bf16 per quarter -- against that quarter's h fragment, shared by the
// four tiles; each quarter's product is scaled by its group scale (a chunk spans at most two
// groups).  Lanes whose quarter lies past the range load nothing (an offset past the buffer)
// and meet zero h (h is zero outside the range and in a 3-quarter pad after each row).  After
// a tile group's last chunk its sums are this workgroup's partial y rows (fp32, unweighted)
// at 16-row segment b + P; the combine adds every workgroup's partial of a row.  Items are
// large because the CU's one scalar unit serves all eight waves: per-item uniform work is
// amortised over 4 KB of weights per wave.  (Issuing the first items as soon as a wave's gate/up
// k-blocks were done, before the workgroup's partial-sum exchange, measured 7 us slower: the
// items' registers then overlapped the gate/up state.)
template <bool kTiled, typename ScaleT>
struct SplitDown {
  static constexpr int kQD = 3;  // items in flight per wave (4 16-byte loads per lane each)
  struct Cursor {
    int j, g, c, n;  // slot, tile group of the wave, chunk, items left after this one
  };
  struct Item {
    uint4 w[4];
    uint32_t sa[4], sb[4];  // the chunk's first and last group scale of each tile
  };
  const VerifyParams& vp;
  char* lds;
  int b, P0, I, H, nq, qshift, hs, nqs, qa0, qb0, qb1, nc0, nc1, nG, tile0, nI;
  int4 dsc0, dsc1;
  buf_rsrc wr0, wr1, sr0, sr1;
  uint32_t wlane, slane, tile_bytes, rowb, sgroup;
  Cursor ic, cc;
  Item ring[kQD];

  __device__ __forceinline__ SplitDown(const VerifyParams& p, char* l) : vp(p), lds(l) {}

  __device__ __forceinline__ int4 wave_desc(int P) const {
    const int4 v = reinterpret_cast<const int4*>(lds + vp.lds_pdesc)[P];
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                     __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
  }
  __device__ __forceinline__ uint32_t wtile(int t) const {
    return kTiled ? static_cast<uint32_t>(t) * tile_bytes : static_cast<uint32_t>(t) * 16u * rowb;
  }
  __device__ __forceinline__ uint32_t stile(int t) const {
    const int ngd = I / vp.dG;
    return static_cast<uint32_t>(t * ngd * 16) * static_cast<uint32_t>(sizeof(ScaleT));
  }
  // Items in order (slot, tile group, chunk); the issue and compute cursors walk them with no
  // divisions.  A cursor on the last item stays there (its loads are repeated, never computed).
  __device__ __forceinline__ void advance(Cursor& k) const {
    if (k.n == 0) return;
    --k.n;
    if (++k.c == (k.j == 0 ? nc0 : nc1)) {
      k.c = 0;
      if (++k.g == nG) {
        k.g = 0;
        k.j = 1;
      }
    }
  }
  __device__ __forceinline__ void issue(Item& it) {
    const bool j0 = ic.j == 0;
    const int q0 = (j0 ? qa0 : 0) + 4 * ic.c, qb = j0 ? qb0 : qb1;
    const buf_rsrc wr = j0 ? wr0 : wr1, sr = j0 ? sr0 : sr1;
    // lanes whose quarter is past the range read nothing (offset past the buffer: no fetch, 0)
    const uint32_t voff = q0 + (lane_id() >> 4) < qb ? wlane : 0x80000000u;
    const uint32_t qoff = static_cast<uint32_t>(q0) * (kTiled ? 256u : 16u);
    const uint32_t ga = static_cast<uint32_t>(q0 >> qshift) * sgroup;
    const uint32_t gb = static_cast<uint32_t>(min(q0 + 3, nq - 1) >> qshift) * sgroup;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int tile = tile0 + 4 * ic.g + t;
      it.w[t] = buf_load16(wr, voff, wtile(tile) + qoff);
      it.sa[t] = buf_scale_bits<ScaleT>(sr, slane, stile(tile) + ga);
      it.sb[t] = buf_scale_bits<ScaleT>(sr, slane, stile(tile) + gb);
    }
    advance(ic);
  }

  // the range [ub, ue) of units, its banks and the cursors; the first items go out
  __device__ __forceinline__ void start(const int ub, const int ue) {
    const int strips = vp.g.strips, lane = lane_id();
    b = static_cast<int>(blockIdx.x);
    I = vp.dI;
    H = vp.dH;
    nq = I >> 5;
    const int ngd = I / vp.dG;
    qshift = vp.dG == 256 ? 3 : 2;  // quarter -> group
    hs = I + kHPad;
    nqs = nq + 3;  // padded row lengths
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, kq = lane >> 4;
    P0 = ub / strips;
    const int np = (ue - 1) / strips - P0 + 1;  // 1 or 2 pass slots
    const int sa0 = ub - P0 * strips, sb0 = min(ue, (P0 + 1) * strips) - P0 * strips;
    qa0 = __builtin_amdgcn_readfirstlane(sa0 >> 1);
    qb0 = __builtin_amdgcn_readfirstlane((sb0 + 1) >> 1);
    qb1 = __builtin_amdgcn_readfirstlane(np > 1 ? (ue - (P0 + 1) * strips + 1) >> 1 : 0);  // from quarter 0
    dsc0 = wave_desc(P0);
    dsc1 = wave_desc(P0 + np - 1);
    nc0 = (qb0 - qa0 + 3) >> 2;
    nc1 = (qb1 + 3) >> 2;  // chunks of 4 quarters
    nG = H >> 9;
    tile0 = wave * 4 * nG;  // tile groups and first tile of the wave
    nI = nG * (nc0 + nc1);
    tile_bytes = static_cast<uint32_t>(I >> 7) * 1024u;
    rowb = static_cast<uint32_t>(I) / 2u;
    const uint32_t bank_bytes = static_cast<uint32_t>(H) * static_cast<uint32_t>(I) / 2u;
    auto bank_of = [&](const int4& d) {
      return d.x < 0 ? vp.dw_shared : vp.dw + static_cast<int64_t>(d.x) * vp.dw_stride;
    };
    auto scales_of = [&](const int4& d) {
      return static_cast<const ScaleT*>(d.x < 0 ? vp.ds_shared : vp.ds) +
             (d.x < 0 ? 0 : static_cast<int64_t>(d.x) * vp.ds_stride);
    };
    wr0 = make_rsrc(bank_of(dsc0), bank_bytes);
    wr1 = make_rsrc(bank_of(dsc1), bank_bytes);
    const uint32_t sbytes = static_cast<uint32_t>(H) * static_cast<uint32_t>(ngd) * sizeof(ScaleT);
    sr0 = make_rsrc(scales_of(dsc0), sbytes);
    sr1 = make_rsrc(scales_of(dsc1), sbytes);
    // lane parts of the addresses: weights (lane quarter = quarter of the chunk, lane % 16 =
    // row) and scales (the lane's row; tiled scales are [tile][group][16], portable [row][group],
    // both 16 ngd elements per tile)
    wlane = kTiled ? static_cast<uint32_t>(kq) * 256u + static_cast<uint32_t>(lr) * 16u
                   : static_cast<uint32_t>(lr) * rowb + static_cast<uint32_t>(kq) * 16u;
    slane = static_cast<uint32_t>(kTiled ? lr : lr * ngd) * sizeof(ScaleT);
    sgroup = static_cast<uint32_t>(kTiled ? 16 : 1) * static_cast<uint32_t>(sizeof(ScaleT));
    ic = Cursor{0, 0, 0, nI - 1};
    cc = ic;
#pragma unroll
    for (int i = 0; i + 1 < kQD; ++i) issue(ring[i]);
  }

  // An empty range (more workgroups than units) strictly inside pass P's units lies between
  // the pass's first and last workgroups, whose partial rows the combine adds one by one: it
  // writes zero rows.  (An empty range at a pass boundary belongs to no pass's run.)
  __device__ __forceinline__ void zero_rows(const int ub, const uint32_t U) const {
    const int strips = vp.g.strips, bb = static_cast<int>(blockIdx.x);
    const int P = ub / strips;
    if (static_cast<uint32_t>(ub) < U && ub != P * strips) {
      const int4 d = reinterpret_cast<const int4*>(lds + vp.lds_pdesc)[P];
      const int rows = min(16, d.z - d.w), quads = vp.dH >> 2;
      float4* o = reinterpret_cast<float4*>(vp.ypart + static_cast<int64_t>(vp.part_rps) * (bb + P) * vp.dH);
      for (int i = threadIdx.x; i < rows * quads; i += kVThreads) o[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }

  __device__ __forceinline__ void run(const int total_passes) {
    const uint32_t U = static_cast<uint32_t>(total_passes) * static_cast<uint32_t>(vp.g.strips);  // U G < 2^32
    const uint32_t G = gridDim.x, bb = blockIdx.x;
    const int ub = static_cast<int>(U * bb / G), ue = static_cast<int>(U * (bb + 1) / G);
    if (ue <= ub) {
      zero_rows(ub, U);
      return;
    }
    start(ub, ue);
    const int lr = lane_id() & 15, kq = lane_id() >> 4;
    const uint16_t* lh = reinterpret_cast<const uint16_t*>(lds + vp.lds_h);  // [2][16][hs]
    float* lst = reinterpret_cast<float*>(lds + vp.lds_hstart);            // [2][nqs][16]
    // every h value of the range is in LDS (the gate/up epilogues); -136 * sum per quarter and row
    lds_barrier();
    for (int i = threadIdx.x; i < 2 * nqs * 16; i += kVThreads) {
      const int r = i & 15, q = (i >> 4) % nqs, j = i / (16 * nqs);
      const uint4* src = reinterpret_cast<const uint4*>(lh + (j * 16 + r) * hs + 32 * q);
      float sum = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 v = src[c];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h2 = 0; h2 < 4; ++h2) sum += __uint_as_float(w[h2] << 16) + __uint_as_float(w[h2] & 0xFFFF0000u);
      }
      lst[(j * nqs + q) * 16 + r] = -kDequantOffset * sum;
    }
    lds_barrier();

    const uint16_t* hl = lh + lr * hs + 8 * kq;
    const float* sl = lst + 4 * kq;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 tot[4] = {zero, zero, zero, zero};
    for (int i0 = 0; i0 < nI; i0 += kQD) {
#pragma unroll
      for (int u = 0; u < kQD; ++u) {
        issue(ring[(u + kQD - 1) % kQD]);
        if (i0 + u < nI) {
          const bool j0 = cc.j == 0;
          const int q0 = (j0 ? qa0 : 0) + 4 * cc.c;
          const int ga = q0 >> qshift;
          // the chunk's h fragments and start terms, shared by the item's four tiles
          uint4 a[4];
          f32x4 st[4];
#pragma unroll
          for (int dq = 0; dq < 4; ++dq) {
            a[dq] = *reinterpret_cast<const uint4*>(hl + cc.j * 16 * hs + 32 * (q0 + dq));
            st[dq] = *reinterpret_cast<const f32x4*>(sl + (cc.j * nqs + q0 + dq) * 16);
          }
          const Item& it = ring[u];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            uint32_t w[4] = {it.w[t].x, it.w[t].y, it.w[t].z, it.w[t].w};
            quarter_transpose(w);
            const float sa = scale_value<ScaleT>(it.sa[t]), sb = scale_value<ScaleT>(it.sb[t]);
#pragma unroll
            for (int dq = 0; dq < 4; ++dq) {
              const f32x4 acc = mfma16x16x32(a[dq], dequant8(w[dq]), st[dq]);
              tot[t] += (((q0 + dq) >> qshift) == ga ? sa : sb) * acc;
            }
          }
          if (cc.c == (j0 ? nc0 : nc1) - 1) {  // the tile group's partial y rows: rows 4 kq + e of column lr
            const int4 d = j0 ? dsc0 : dsc1;
            const int64_t row0 = static_cast<int64_t>(vp.part_rps) * (b + P0 + cc.j);
            float* o = vp.ypart + row0 * H + (tile0 + 4 * cc.g) * 16 + lr;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (d.w + 4 * kq + e < d.z) {
#pragma unroll
                for (int t = 0; t < 4; ++t) o[static_cast<int64_t>(4 * kq + e) * H + 16 * t] = tot[t][e];
              }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) tot[t] = zero;
          }
          advance(cc);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
};

// gate/up with the split-K down in the same launch
template <bool kTiled, int kNKB, typename ScaleT>
__device__ __forceinline__ void gate_up_split_down(const VerifyParams& vp, char* lds, const int total_passes) {
  verify_gemm<kModeGateUp, kNKB, ScaleT>(vp, lds, total_passes);
  SplitDown<kTiled, ScaleT> down(vp, lds);
  down.run(total_passes);
}

template <int kMode, int kNKB, typename ScaleT>
__global__ __launch_bounds__(512) void w4_verify_kernel(VerifyParams vp) {
  __shared__ __attribute__((aligned(16))) char lds[kVLds];
  tl_mark(kMode, 0);
  const int total_passes = verify_passes<kMode, kNKB>(vp, lds);
  tl_mark(kMode, 1);
  if (kMode == kModeGateUp && vp.fuse_down) {
    if constexpr (kMode == kModeGateUp) {
      if (vp.g.tiled) gate_up_split_down<true, kNKB, ScaleT>(vp, lds, total_passes);
      else gate_up_split_down<false, kNKB, ScaleT>(vp, lds, total_passes);
    }
  } else {
    verify_gemm<kMode, kNKB, ScaleT>(vp, lds, total_passes);
  }
#ifdef DFLASH_TIMELINE
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  tl_mark(kMode, 13);
#endif
}

// ---------------------------------------------------------------------------
// host side
bool verify_layout(int mode, int T, int K, int N, int E, int k, int has_shared, int route, VerifyParams* vp) {
  // K = 4096 (the attention output projections) only as a plain linear: its x rows fill most of the LDS
  if (K != 512 && K != 1024 && K != 2048 && !(K == 4096 && mode == kModeLinear)) return false;
  // gate/up and down stage per chunk of passes when needed, so only linear mode bounds T
  if (T <= 0 || (mode == kModeLinear && T > 32) || k <= 0) return false;
  if (N % (mode == kModeGateUp ? 32 : kVStrip)) return false;
  const int rs = 2 * K + 16, nkb = K / 128;
  auto al = [](int v) { return (v + 15) & ~15; };
  const int part = kVWaves * 2 * 64 * 16;
  int off = 0;
  auto take = [&](int bytes) {
    const int o = off;
    off += al(bytes);
    return o;
  };
  VerifyParams& L = *vp;
  L.route = 0;
  L.gather = 0;
  // gathered gate/up (blocks above 32 tokens, or whose whole-block plan below does not fit):
  // per chunk of passes, 16 x rows each (by token) and their -136*sum terms, like down's h rows
  auto gather_layout = [&]() {
    off = 0;
    const int per_pass = 16 * rs + al(16 * nkb * 4);
    const int fixed = part + 64 * 16;
    const int cp = std::min(8, (kVLds - fixed) / per_pass);
    if (cp < 1) return false;
    L.route = 0;
    L.gather = 1;
    L.chunk_passes = cp;
    L.pd_cap = 64;
    L.a_rows = cp * 16;
    L.lds_a = take(cp * 16 * rs);
    L.lds_neg = take(cp * 16 * nkb * 4);
    L.lds_wgt = 0;
    L.lds_pdesc = take(64 * 16);
    L.lds_tok = 0;
    L.lds_part = L.lds_scratch = take(part);
    L.lds_bytes = off;
    return off <= kVLds;
  };
  if (mode == kModeGateUp && T > 32) return gather_layout();
  if (mode == kModeDown) {
    // per pass: 16 h rows, their -136*sum terms and raw partials (8 per k-block)
    const int per_pass = 16 * rs + al(16 * nkb * 4) + al(16 * nkb * 8 * 4);
    const int fixed = part + 64 * 16;  // partial sums of split units; 64 pass descriptors (one load)
    const int cp = std::min(8, (kVLds - fixed) / per_pass);
    if (cp < 1) return false;
    L.chunk_passes = cp;
    L.pd_cap = 64;
    L.a_rows = cp * 16;
    L.lds_a = take(cp * 16 * rs);
    L.lds_neg = take(cp * 16 * nkb * 4);
    L.lds_wgt = take(cp * 16 * nkb * 8 * 4);
    L.lds_pdesc = take(64 * 16);
    L.lds_tok = 0;
    L.lds_part = L.lds_scratch = take(part);
    L.lds_bytes = off;
    return off <= kVLds;
  }
  L.chunk_passes = 0;
  L.a_rows = T;
  L.lds_a = take(T * rs);
  L.lds_neg = take(((T * nkb + 63) & ~63) * 4);  // filled 64 terms per direct-to-LDS load
  L.lds_wgt = 0;
  if (mode == kModeLinear) {
    // stage_x_raw gives each thread at most 16 chunks of 8 columns: 32 rows up to K = 2048, 16 at K = 4096
    if (T * (K / 8) > kVThreads * std::min(nkb, 16)) return false;
    L.pd_cap = 0;
    L.lds_tok = L.lds_pdesc = 0;
    L.lds_part = L.lds_scratch = take(part);
    L.lds_bytes = off;
    return off <= kVLds;
  }
  const int tpasses = (T + 15) / 16;
  L.pd_cap = std::min(E, T * k) * tpasses + (has_shared ? tpasses : 0);
  L.lds_tok = take(T * k * 4);
  L.lds_pdesc = take(L.pd_cap * 16);
  const int base = off;
  const int tpad = (T + 3) & ~3;
  const int scratch = al(((E + 3) & ~3) * 4) + al(((T * k + 3) & ~3) * 4) + 96 + E * tpad;
  const int row_scratch = (256 + 512 + 512 + 12 + 256) * 4 + E * tpad;  // route_rows: counts, weights, ids, totals, first passes, map
  if (route && E <= 256 && k <= 16 && T * k <= 512 && base + std::max(part, row_scratch) <= kVLds) {
    L.route = 2;
    L.lds_part = L.lds_scratch = take(std::max(part, row_scratch));
  } else if (route && E <= 2 * kVThreads && base + std::max(part, al(scratch)) <= kVLds) {
    L.route = 1;
    L.lds_part = L.lds_scratch = take(std::max(part, scratch));
  } else {
    L.lds_part = L.lds_scratch = take(part);
  }
  L.lds_bytes = off;
  if (off <= kVLds) return true;
  return mode == kModeGateUp && gather_layout();  // whole-block plan too large: gathered chunks
}


int fused_down_lds(int I) {
  return ((2 * 16 * (I + kHPad) * 2 + 15) & ~15) + ((2 * (I / 32 + 3) * 16 * 4 + 15) & ~15);
}

bool fused_down_layout(VerifyParams* vp, int I) {
  const int off = (vp->lds_bytes + 15) & ~15;
  if (vp->route != 2 || off + fused_down_lds(I) > kVLds) return false;
  vp->lds_h = off;
  vp->lds_hstart = off + ((2 * 16 * (I + kHPad) * 2 + 15) & ~15);
  vp->lds_bytes = off + fused_down_lds(I);
  return true;
}

void launch_w4_verify(int mode, bool fp32_scales, int grid, const VerifyParams& vp, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid)), blk(kVThreads);
#define DFLASH_VERIFY(MODE, NKB)                                                                           \
  do {                                                                                                     \
    if (fp32_scales) hipLaunchKernelGGL((w4_verify_kernel<MODE, NKB, float>), g, blk, 0, stream, vp);     \
    else hipLaunchKernelGGL((w4_verify_kernel<MODE, NKB, uint16_t>), g, blk, 0, stream, vp);              \
  } while (0)
#define DFLASH_VERIFY_K(MODE)                    \
  switch (vp.g.K) {                              \
    case 512: DFLASH_VERIFY(MODE, 4); break;     \
    case 1024: DFLASH_VERIFY(MODE, 8); break;    \
    default: DFLASH_VERIFY(MODE, 16); break;     \
  }
  switch (mode) {
    case kModeLinear:
      if (vp.g.K == 4096) DFLASH_VERIFY(kModeLinear, 32);
      else DFLASH_VERIFY_K(kModeLinear)
      break;
    case kModeGateUp: DFLASH_VERIFY_K(kModeGateUp) break;
    default: DFLASH_VERIFY_K(kModeDown) break;
  }
#undef DFLASH_VERIFY_K
#undef DFLASH_VERIFY
}

#ifdef DFLASH_TIMELINE
int timeline_verify_read(void* host, size_t bytes) {
  if (bytes != sizeof(g_timeline_verify)) return 1;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_timeline_verify), bytes) == hipSuccess ? 0 : 1;
}
int timeline_verify_clear() {
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_timeline_verify)) != hipSuccess) return 1;
  return hipMemset(ptr, 0, sizeof(g_timeline_verify)) == hipSuccess ? 0 : 1;
}
#endif

}  // namespace dflash
