// Verify-block W4A16 expert GEMMs (T <= 32 tokens): the routed-MoE layer of a
// DFlash verify block in four launches (router front, gate/up, down, combine).
//
// Work decomposition.  A unit is one pass (up to 16 slot rows of an expert
// segment or of the shared expert) times one strip of 2 x 16 weight rows over
// the full reduction length K.  Units form one list (pass-major); each
// workgroup takes an equal contiguous range of it, and inside the workgroup the
// range's k-blocks (128 columns of K) are split evenly over the 8 waves at
// multiples of 4 k-blocks, so every wave streams the same number of weight
// bytes whatever the unit count.  A unit whose k-blocks fall to several waves
// is finished by the wave holding its last k-block, after the others left their
// partial sums in LDS (summed in wave order: the result does not depend on
// timing).
//
// Per k-block a lane issues two 16-byte weight loads (16 rows x 64 bytes per
// tile) and the two group scales of its rows (group size 128 or 256), ahead of
// the k-block it computes.  Each k-block is
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
//             launch per qlinear); one pass per 16 rows.
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
// kVShareYoung of waves 4-7 (4:3 measured best of 1:1, 7:6, 4:3, 11:8: -0.6 us per kernel).
constexpr int kVShareOld = 4, kVShareYoung = 3;

// First k-block of wave w when a workgroup's range of n k-blocks is split by those shares.
__device__ __forceinline__ int wave_start(int n, int w) {
  const int cum = kVShareOld * min(w, 4) + kVShareYoung * max(w - 4, 0);
  return (n * cum) / (4 * (kVShareOld + kVShareYoung));
}
constexpr int kVStrip = 32;      // output columns per down/linear unit (and per combine strip)
constexpr int kVLds = 158 * 1024;  // one persistent workgroup per CU

typedef __attribute__((address_space(3))) void* lds_ptr;

// Cache policy of a vector memory load: sc1 (device scope) makes it skip the CU's L1, so it
// reads this XCD's L2, where other CUs of the XCD left their stores.  (sc0 alone, workgroup
// scope, may still hit in L1.)
constexpr int kCacheSc1 = 16;

__device__ __forceinline__ void dma16(buf_rsrc r, void* dst, uint32_t voff, uint32_t soff, int cpol = 0) {
  if (cpol == kCacheSc1)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, static_cast<int>(voff), static_cast<int>(soff), 0,
                                             kCacheSc1);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 16, static_cast<int>(voff), static_cast<int>(soff), 0, 0);
}
__device__ __forceinline__ void dma4(buf_rsrc r, void* dst, uint32_t voff, uint32_t soff, int cpol = 0) {
  if (cpol == kCacheSc1)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 4, static_cast<int>(voff), static_cast<int>(soff), 0,
                                             kCacheSc1);
  else
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

// Polls a workgroup may spend waiting over its whole down range (~0.1-0.4 s).
constexpr int kSpinBudget = 200000;

// Count word of part-local pass j of part x, and the part's gate/up (phase 0) and down
// (phase 1) queues, its last two words: each part's words fill cache lines of their own.
__device__ __forceinline__ int32_t* ready_word(const VerifyParams& vp, int part, int j) {
  return vp.ready + part * vp.ready_stride + j;
}
__device__ __forceinline__ int32_t* queue_word(const VerifyParams& vp, int part, int phase) {
  return vp.ready + part * vp.ready_stride + vp.ready_stride - 2 + phase;
}

// The unit range of a verify_gemm call: part `part` of `parts` (pass P is part P % parts's
// local pass P / parts), its range `rank` of `ranks` contiguous ones.
struct Split {
  int part, parts, rank, ranks;
};

// Bounded wait (one thread) until each of the n count words of consecutive part-local passes
// reads `target` finished gate/up units (device-scope atomics and loads: the load skips L1,
// and the count is exact once it reads the target).  Every poll spends one of the workgroup's
// budget (returned: what is left); once it is spent the wait sets err bit 1 and returns at
// once, now and at every later call (the launch then ends with wrong down rows, never hangs).
__device__ __noinline__ int wait_ready(int32_t* words, int n, int target, int32_t* err, int budget) {
  for (int j = 0; j < n; ++j) {
    while (__hip_atomic_load(words + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (--budget < 0) {
        __hip_atomic_fetch_or(err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return budget;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return budget;
}

// Opaque to the optimiser: the value must exist in registers at this point.
__device__ __forceinline__ void pin(f32x4& v) { asm volatile("" : "+v"(v)); }

// ---------------------------------------------------------------------------
// In-kernel routing of the block (512 threads, T <= 32, E <= 1024).  Leaves
// every pass descriptor in pdesc and the token of every slot row in tok;
// returns the number of passes.  Workgroup 0 writes the routing outputs
// (ids, weights, perm, inv, offsets) and the work table the down launch reads.
__device__ int route_block(const VerifyParams& vp, char* lds, int4* pdesc, int* tok) {
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
__device__ int route_rows(const VerifyParams& vp, RowKeys<kPR> keys, char* lds, int4* pdesc, int* tok) {
  const int T = vp.g.T, E = vp.E, k = vp.g.top_k;
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id(), r = lane & 31;
  const int t0 = 2 * wave + (lane >> 5);  // token of pass 0; pass 1 adds 16
  const int tpad = (T + 3) & ~3;
  const bool out = blockIdx.x == 0;
  int* cnt = reinterpret_cast<int*>(lds + vp.lds_scratch);        // [256] tokens per expert, then its first slot row
  float* rw = reinterpret_cast<float*>(cnt + 256);                // [T*k] routing weight of every flat pair
  int* rid = reinterpret_cast<int*>(rw + 512);                    // [T*k] expert of every flat pair
  int* wtot = rid + 512;                                          // [3][4] wave totals: slot rows, passes, hits
  uint32_t* map_words = reinterpret_cast<uint32_t*>(wtot + 12);   // [E][tpad] bytes: slot + 1, or 0
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

// The streaming GEMM of one verify launch over `total_passes` passes: the units of range
// sp.rank of part sp.part (linear mode: every workgroup's strided share).
template <int kMode, int kNKB, typename ScaleT>
__device__ __forceinline__ void verify_gemm(const VerifyParams& vp, char* lds, const int total_passes,
                                            const Split sp) {
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
  // fused layer launch: part x's passes (global index P = x + 8 j) and a claimed range of
  // them; else one part, one range per workgroup.  Below, a pass index is part-local (j)
  // unless named global.
  const int parts = sp.parts, part = sp.part, rank = sp.rank, ranks = sp.ranks;
  const int local_passes = total_passes > part ? (total_passes - part + parts - 1) / parts : 0;
  auto gpass = [&](int j) { return part + parts * j; };
  const int64_t total_units = static_cast<int64_t>(local_passes) * strips;
  // linear mode: workgroup b runs units b, b + G, b + 2G, ... (G = grid), so at any moment the
  // workgroups stream one contiguous window of the weights (contiguous ranges per workgroup
  // leave ~2048 streams a fixed stride apart, which streamed up to 10% slower); its virtual
  // range [ub, ue) gives the first U % G workgroups one unit more
  int ub, ue;
  if (kMode == kModeLinear) {
    const int G = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
    const int q = static_cast<int>(total_units / G), r = static_cast<int>(total_units % G);
    ub = b * q + min(b, r);
    ue = ub + q + (b < r ? 1 : 0);
  } else {
    ub = static_cast<int>(total_units * rank / ranks);
    ue = static_cast<int>(total_units * (rank + 1) / ranks);
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
  // descriptor of global pass P before the chunk is staged: a fused launch holds every pass
  // in LDS since its routing prologue (the work table in memory is another XCD's to write)
  auto early_desc = [&](int P) -> int4 {
    if (vp.fused) return lds_desc(P);
    return P == plan_p ? plan_d0 : P == plan_p + 1 ? plan_d1 : ld_const_int4(p.pass_table, P);
  };
  // pass descriptors: all of them after in-kernel routing, else the chunk's (staged below)
  int pd_base = 0;
  auto pass_desc = [&](int j) -> int4 {
    if (kMode == kModeLinear) return make_int4(0, 0, p.M, j * 16);
    return lds_desc(vp.fused ? gpass(j) : j - pd_base);
  };

  const bool chunked = kMode == kModeDown || (kMode == kModeGateUp && vp.gather);
  int spin_budget = kSpinBudget;  // fused down: polls left to this workgroup's waits (thread 0)
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
                           ? pass_desc(P) : early_desc(gpass(P));
        const bool shared = kMode != kModeLinear && d.x < 0;
        const int64_t e = kMode == kModeLinear ? 0 : d.x;
        const uint8_t* wbase = shared ? p.w_shared : p.w + e * p.w_stride;
        const uint8_t* sbase = static_cast<const uint8_t*>(shared ? p.s_shared : p.s) +
                               (shared ? 0 : e * p.s_stride * static_cast<int64_t>(sizeof(ScaleT)));
        const int64_t row0 = static_cast<int64_t>(strip) * kTileRows;
        l_w = wbase + row0 * rb;
        l_s = sbase + row0 * ng * static_cast<int64_t>(sizeof(ScaleT));
      };
      // ring of k-blocks in flight: two 16-byte weight loads and the two group scales of the lane's rows
      uint4 wbuf[kVDepth][2];
      uint32_t sbuf[kVDepth][2];
      // Loads are issued unconditionally (past the range they repeat its last k-block, never
      // computed): a load under a branch would make the compiler drain the queue at the loop edge.
      auto issue = [&](uint4 (&dst)[2], uint32_t (&sdst)[2]) {
        const int lc = max(min(lg, g1 - 1), 0);
        const int ur = lc / kNKB, kb = lc - ur * kNKB;
        if (ur != l_ur) {
          l_ur = ur;
          unit_bases(ur);
        }
        dst[0] = *reinterpret_cast<const uint4*>(l_w + wlane + kb * wkb);
        dst[1] = *reinterpret_cast<const uint4*>(l_w + second * rb + wlane + kb * wkb);
        const ScaleT* sp = reinterpret_cast<const ScaleT*>(l_s) + slane + (kb >> gshift) * skb;
        sdst[0] = load_scale_bits(sp);
        sdst[1] = load_scale_bits(sp + second * ng);
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
        if (!vp.fused) {
          const buf_rsrc tr = make_rsrc(p.pass_table, static_cast<uint32_t>(total_passes) * 16);
          if (wave == 0)
            dma16(tr, lds_pdesc, static_cast<uint32_t>(min(Pc + lane, total_passes - 1) * 16), 0);
        } else {
          // fused launch: the chunk's h rows are written by this XCD's workgroups during this
          // launch; wait until every gate/up unit of each of its passes has been counted
          if (tid == 0)
            spin_budget = wait_ready(ready_word(vp, part, Pc), Pc_end - Pc, vp.ready_target, vp.err, spin_budget);
          __syncthreads();
        }
        // a fused launch reads h through the XCD's L2 (its writers are other CUs of this XCD)
        const int cpol = vp.fused ? kCacheSc1 : 0;
        const int hrows = p.T * p.top_k + (p.has_shared ? p.T : 0);
        const buf_rsrc hr = make_rsrc(p.act, static_cast<uint32_t>(hrows) * kK * 2);
        constexpr int kBlk = kK / 512;
        for (int i = wave; i < npass * 16 * kBlk; i += kVWaves) {
          const int rr = i / kBlk, bl = i - rr * kBlk;
          const int4 d = early_desc(gpass(Pc + rr / 16));
          const int base = d.x < 0 ? p.T * p.top_k : d.y;
          const int row = base + min(d.w + (rr & 15), d.z - 1);
          dma16(hr, lds_a + rr * kRS + bl * 1024, static_cast<uint32_t>(lane * 16),
                static_cast<uint32_t>((row * kK + bl * 512) * 2), cpol);
        }
        constexpr int kPartRow = kNKB * 8;  // partials per h row
        const buf_rsrc pr = make_rsrc(p.act_neg, static_cast<uint32_t>(hrows) * kPartRow * 4);
        for (int i = wave; i < npass * 2 * kNKB; i += kVWaves) {  // 64 partials per load, 2 kNKB per pass
          const int pass = i / (2 * kNKB), j = i - pass * 2 * kNKB;
          const int4 d = early_desc(gpass(Pc + pass));
          const int base = d.x < 0 ? p.T * p.top_k : d.y;
          const int f = 64 * j + lane, rr = f / kPartRow;
          const int row = base + min(d.w + rr, d.z - 1);
          dma4(pr, lds_hpart + pass * 16 * kPartRow + 64 * j,
               static_cast<uint32_t>((row * kPartRow + f % kPartRow) * 4), 0, cpol);
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
      if (Pc == P_first && !vp.fused) tl_mark(kMode, 2);

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
            tot0 += scale_value<ScaleT>(sbuf[i][0]) * acc0;
            tot1 += scale_value<ScaleT>(sbuf[i][1]) * acc1;
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
    if (!vp.fused) tl_mark(kMode, 4 + wave, true);
    lds_barrier();  // partial sums of split units are in LDS
    if (!vp.fused) tl_mark(kMode, 12);
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

template <int kMode, int kNKB, typename ScaleT>
__global__ __launch_bounds__(512) void w4_verify_kernel(VerifyParams vp) {
  __shared__ __attribute__((aligned(16))) char lds[kVLds];
  tl_mark(kMode, 0);
  const int total_passes = verify_passes<kMode, kNKB>(vp, lds);
  tl_mark(kMode, 1);
  verify_gemm<kMode, kNKB, ScaleT>(vp, lds, total_passes,
                                   Split{0, 1, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x)});
#ifdef DFLASH_TIMELINE
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  tl_mark(kMode, 13);
#endif
}

// After gate/up range `rank` of part `part` (the split verify_gemm made): every store of the
// workgroup has reached the XCD's L2 (stores are acknowledged there; L1 writes through), then
// each pass the range touched gets the number of its units the range finished added to its
// count, which the down ranges of the part poll.  The workgroup's LDS is free afterwards.
__device__ __forceinline__ void publish_ready(const VerifyParams& vp, int total_passes, int part, int rank,
                                              int ranks) {
  __builtin_amdgcn_s_waitcnt(0);  // this thread's h and partial stores are acknowledged by L2
  __syncthreads();
  const int strips = vp.g.strips;
  const int local_passes = total_passes > part ? (total_passes - part + kXcds - 1) / kXcds : 0;
  const int64_t total_units = static_cast<int64_t>(local_passes) * strips;
  const int ub = static_cast<int>(total_units * rank / ranks), ue = static_cast<int>(total_units * (rank + 1) / ranks);
  if (ue > ub) {
    for (int j = ub / strips + static_cast<int>(threadIdx.x); j <= (ue - 1) / strips; j += kVThreads) {
      const int n = min(ue, (j + 1) * strips) - max(ub, j * strips);
      __hip_atomic_fetch_add(ready_word(vp, part, j), n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
}

// After the workgroup's last claim came back empty (every wait of it has ended): the last
// workgroup of the grid to get here knows every range of every part finished, and returns
// all counts, queues and the done count to zero for the next launch on this workspace.
__device__ __forceinline__ void reset_ready(const VerifyParams& vp, int* lds_flag) {
  if (threadIdx.x == 0)
    *lds_flag = __hip_atomic_fetch_add(vp.done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                static_cast<int>(gridDim.x) - 1;
  __syncthreads();
  if (*lds_flag) {
    for (int i = static_cast<int>(threadIdx.x); i < kXcds * vp.ready_stride; i += kVThreads)
      __hip_atomic_store(vp.ready + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x == 0) __hip_atomic_store(vp.done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The routed-MoE layer's expert FFN in one launch: routing prologue, gate/up, then down.  Pass
// P belongs to part P % 8 in both phases, and only workgroups running on XCD P % 8 (read from
// the hardware, whatever the dispatch order) take ranges of it, so a down range waits only on
// gate/up work of its own XCD: counts and h rows meet in that XCD's L2, and nothing crosses
// XCDs inside the launch.  The combine that sums each token's slots over all XCDs stays a
// launch of its own.  Ranges are claimed from the part's queues (gate/up first, then down,
// the next claim in flight during a range), so a part's gate/up ranges all go to workgroups
// that finish them before any down range of theirs: every wait ends once each XCD runs a
// workgroup, whatever the residency, and a wait that does not end gives up after its budget.
template <int kNKBg, int kNKBd, typename ScaleT>
__global__ __launch_bounds__(512) void w4_layer_kernel(VerifyParams gu, VerifyParams dn) {
  __shared__ __attribute__((aligned(16))) char lds[kVLds];
  __shared__ int bcast;
  const int tid = threadIdx.x;
  const int part = static_cast<int>(xcc_id());
  if (part >= kXcds) {  // not an 8-XCD device: take no range (the waits of the others give up)
    if (tid == 0) __hip_atomic_fetch_or(gu.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    reset_ready(gu, &bcast);
    return;
  }
  // thread 0 claims; the value reaches the workgroup through LDS
  auto claim = [&](int phase) {
    return __hip_atomic_fetch_add(queue_word(gu, part, phase), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto share = [&](int v) {
    if (tid == 0) bcast = v;
    __syncthreads();
    const int c = bcast;
    __syncthreads();
    return c;
  };
  int next_gu = 0, next_dn = 0;
  if (tid == 0) {  // both first claims travel during the routing prologue
    next_gu = claim(0);
    next_dn = claim(1);
  }
  const int total_passes = verify_passes<kModeGateUp, kNKBg>(gu, lds);
  for (int c = share(next_gu); c < gu.chunks; c = share(next_gu)) {
    if (tid == 0) next_gu = claim(0);
    verify_gemm<kModeGateUp, kNKBg, ScaleT>(gu, lds, total_passes, Split{part, kXcds, c, gu.chunks});
    publish_ready(gu, total_passes, part, c, gu.chunks);
  }
  for (int c = share(next_dn); c < dn.chunks; c = share(next_dn)) {
    if (tid == 0) next_dn = claim(1);
    verify_gemm<kModeDown, kNKBd, ScaleT>(dn, lds, total_passes, Split{part, kXcds, c, dn.chunks});
  }
  reset_ready(gu, &bcast);
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
  const int row_scratch = (256 + 512 + 512 + 12) * 4 + E * tpad;  // route_rows: counts, weights, ids, totals, map
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

bool layer_layout(int T, int H, int I, int E, int k, int has_shared, VerifyParams* gu, VerifyParams* dn) {
  // instantiated shapes: gate/up over H in {512, 1024, 2048}, down over I in {512, 1024}
  if ((H != 512 && H != 1024 && H != 2048) || (I != 512 && I != 1024)) return false;
  if (T <= 0 || T > 32 || k <= 0 || H % kVStrip) return false;
  auto al = [](int v) { return (v + 15) & ~15; };
  const int part = kVWaves * 2 * 64 * 16;
  int off = 0;
  auto take = [&](int bytes) {
    const int o = off;
    off += al(bytes);
    return o;
  };
  // shared by both phases: every pass descriptor and the token of every slot row (routing)
  const int tpasses = (T + 15) / 16;
  const int pd_cap = std::min(E, T * k) * tpasses + (has_shared ? tpasses : 0);
  const int pdesc = take(pd_cap * 16), tok = take(T * k * 4);
  const int u0 = off;
  // gate/up phase: all T x rows, their -136*sum terms, the routing scratch / split partials
  *gu = VerifyParams{};
  const int rs_g = 2 * H + 16, nkb_g = H / 128;
  gu->a_rows = T;
  gu->pd_cap = pd_cap;
  gu->lds_pdesc = pdesc;
  gu->lds_tok = tok;
  gu->lds_a = take(T * rs_g);
  gu->lds_neg = take(((T * nkb_g + 63) & ~63) * 4);
  const int tpad = (T + 3) & ~3;
  const int row_scratch = (256 + 512 + 512 + 12) * 4 + E * tpad;
  const int scratch = al(((E + 3) & ~3) * 4) + al(((T * k + 3) & ~3) * 4) + 96 + E * tpad;
  if (E <= 256 && k <= 16 && T * k <= 512) {
    gu->route = 2;
    gu->lds_part = gu->lds_scratch = take(std::max(part, row_scratch));
  } else if (E <= 2 * kVThreads) {
    gu->route = 1;
    gu->lds_part = gu->lds_scratch = take(std::max(part, al(scratch)));
  } else {
    return false;
  }
  gu->lds_bytes = off;
  if (off > kVLds) return false;
  // down phase over the same bytes after the descriptors: chunks of h rows and their partials
  off = u0;
  *dn = VerifyParams{};
  const int rs_d = 2 * I + 16, nkb_d = I / 128;
  dn->lds_part = dn->lds_scratch = take(part);
  const int per_pass = 16 * rs_d + al(16 * nkb_d * 4) + al(16 * nkb_d * 8 * 4);
  const int cp = std::min(8, (kVLds - off) / per_pass);
  if (cp < 1) return false;
  dn->chunk_passes = cp;
  dn->pd_cap = pd_cap;
  dn->a_rows = cp * 16;
  dn->lds_pdesc = pdesc;
  dn->lds_tok = tok;
  dn->lds_a = take(cp * 16 * rs_d);
  dn->lds_neg = take(cp * 16 * nkb_d * 4);
  dn->lds_wgt = take(cp * 16 * nkb_d * 8 * 4);
  dn->lds_bytes = off;
  gu->fused = dn->fused = 1;
  return off <= kVLds;
}

void launch_w4_layer(bool fp32_scales, int grid, const VerifyParams& gu, const VerifyParams& dn, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid)), blk(kVThreads);
#define DFLASH_LAYER(NG, ND)                                                                             \
  do {                                                                                                   \
    if (fp32_scales) hipLaunchKernelGGL((w4_layer_kernel<NG, ND, float>), g, blk, 0, stream, gu, dn);   \
    else hipLaunchKernelGGL((w4_layer_kernel<NG, ND, uint16_t>), g, blk, 0, stream, gu, dn);            \
  } while (0)
#define DFLASH_LAYER_D(NG)                            \
  do {                                                \
    if (dn.g.K == 512) DFLASH_LAYER(NG, 4);           \
    else DFLASH_LAYER(NG, 8);                         \
  } while (0)
  switch (gu.g.K) {
    case 512: DFLASH_LAYER_D(4); break;
    case 1024: DFLASH_LAYER_D(8); break;
    default: DFLASH_LAYER_D(16); break;
  }
#undef DFLASH_LAYER_D
#undef DFLASH_LAYER
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
