// Top-k selection primitives shared by the routing kernels (route.hip) and the
// verify-block expert kernel that routes inside its prologue (w4_verify.hip).
//
// Routing contract (reference reference/fused_ops.py:160-164,
// graph/fused/quant_target.py:168-172): rank the fp32 logits in descending
// order, lowest expert id first among equal logits; weights are the softmax of
// the selected logits (the full-softmax denominator cancels in the renorm).
#pragma once

#include "kernels.h"

namespace dflash {

// Order-preserving uint32 of a float: -0 folded to +0, NaN ranks below -inf.
__device__ __forceinline__ uint32_t sortable_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0u;
  if ((u & 0x7FFFFFFFu) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Max of a 32-bit value over all 64 lanes, returned wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto dmax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  v = dmax(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false)));
  v = dmax(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false)));
  v = dmax(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xF, 0xF, false)));
  v = dmax(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xF, 0xF, false)));
  const uint32_t a = __builtin_amdgcn_readlane(static_cast<int>(v), 0), b = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t c = __builtin_amdgcn_readlane(static_cast<int>(v), 32), d = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return dmax(dmax(a, b), dmax(c, d));
}

// Top-k of one token's logits by one wave.  Lane l holds experts l + 64 i as
// 32-bit keys (sortable_key + 1; 0 marks padding and experts already taken).
// Each of the k rounds takes the wave-wide maximum key, then the lowest
// expert id holding it (a ballot per block of 64 ids, first set bit of the
// first non-empty block): the larger logit wins and, among equal logits, the
// lower expert id.  Lane s < k ends with (id_s, weight_s).
template <int kPer>
__device__ __forceinline__ void load_keys(const float* __restrict__ row, int E, uint32_t (&key)[kPer]) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = lane + 64 * i;
    key[i] = e < E ? sortable_key(row[e]) + 1u : 0u;  // sortable keys stay below 0xFF800001
  }
}

// The k selection rounds and the weights of wave_topk over keys already loaded (load_keys).
template <int kPer>
__device__ __forceinline__ void select_keys(uint32_t (&key)[kPer], int k, int* id_out, float* w_out) {
  const int lane = lane_id();
  int my_id = -1;
  uint32_t my_key = 0;
  for (int s = 0; s < k; ++s) {
    uint32_t m = key[0];
#pragma unroll
    for (int i = 1; i < kPer; ++i) m = m > key[i] ? m : key[i];
    m = wave_max_u32(m);
    int e = -1;
#pragma unroll
    for (int i = kPer - 1; i >= 0; --i) {  // the lowest block with a hit decides
      const uint64_t hits = __ballot(key[i] == m);
      if (hits) e = 64 * i + __builtin_ctzll(hits);
    }
    e = __builtin_amdgcn_readfirstlane(e);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (lane + 64 * i == e) key[i] = 0u;
    if (lane == s) {
      my_id = e;
      my_key = m - 1u;
    }
  }
  const float top = key_to_float(__builtin_amdgcn_readlane(static_cast<int>(my_key), 0));
  const float ex = (lane < k) ? expf(key_to_float(my_key) - top) : 0.f;
  const float total = wave_sum(ex);
  *id_out = my_id;
  *w_out = ex / total;
}

template <int kPer>
__device__ __forceinline__ void wave_topk(const float* __restrict__ row, int E, int k, int* id_out, float* w_out) {
  uint32_t key[kPer];
  load_keys<kPer>(row, E, key);
  select_keys<kPer>(key, k, id_out, w_out);
}

__device__ __forceinline__ void topk_any(const float* row, int E, int k, int* id, float* w) {
  if (E <= 64) wave_topk<1>(row, E, k, id, w);
  else if (E <= 128) wave_topk<2>(row, E, k, id, w);
  else if (E <= 256) wave_topk<4>(row, E, k, id, w);
  else if (E <= 512) wave_topk<8>(row, E, k, id, w);
  else wave_topk<16>(row, E, k, id, w);
}

// Top-k of two tokens by one wave, the two selections interleaved so that each
// round's reductions of one token fill the other's latencies (same result as
// wave_topk per token).  Row b is skipped when !live_b.
template <int kPer>
__device__ __forceinline__ void wave_topk2(const float* __restrict__ row_a, const float* __restrict__ row_b,
                                           bool live_b, int E, int k, int (&id_out)[2], float (&w_out)[2]) {
  const int lane = lane_id();
  uint32_t key[2][kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = lane + 64 * i;
    key[0][i] = e < E ? sortable_key(row_a[e]) + 1u : 0u;
    key[1][i] = e < E && live_b ? sortable_key(row_b[e]) + 1u : 0u;
  }
  int my_id[2] = {-1, -1};
  uint32_t my_key[2] = {0u, 0u};
  for (int s = 0; s < k; ++s) {
    uint32_t m[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      m[r] = key[r][0];
#pragma unroll
      for (int i = 1; i < kPer; ++i) m[r] = m[r] > key[r][i] ? m[r] : key[r][i];
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) m[r] = wave_max_u32(m[r]);
    int e[2] = {-1, -1};
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int i = kPer - 1; i >= 0; --i) {  // the lowest block with a hit decides
        const uint64_t hits = __ballot(key[r][i] == m[r]);
        if (hits) e[r] = 64 * i + __builtin_ctzll(hits);
      }
      e[r] = __builtin_amdgcn_readfirstlane(e[r]);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (lane + 64 * i == e[r]) key[r][i] = 0u;
      if (lane == s) {
        my_id[r] = e[r];
        my_key[r] = m[r] - 1u;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const float top = key_to_float(__builtin_amdgcn_readlane(static_cast<int>(my_key[r]), 0));
    const float ex = (lane < k) ? expf(key_to_float(my_key[r]) - top) : 0.f;
    const float total = wave_sum(ex);
    id_out[r] = my_id[r];
    w_out[r] = ex / total;
  }
}

__device__ __forceinline__ void topk2_any(const float* a, const float* b, bool live_b, int E, int k, int (&id)[2],
                                          float (&w)[2]) {
  if (E <= 64) wave_topk2<1>(a, b, live_b, E, k, id, w);
  else if (E <= 128) wave_topk2<2>(a, b, live_b, E, k, id, w);
  else if (E <= 256) wave_topk2<4>(a, b, live_b, E, k, id, w);
  else if (E <= 512) wave_topk2<8>(a, b, live_b, E, k, id, w);
  else wave_topk2<16>(a, b, live_b, E, k, id, w);
}

// Inclusive prefix sum over the 64 lanes (row shifts, then row broadcasts).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return v;
}

__device__ __forceinline__ int passes_for(int rows, int rows_per_pass) {
  return (rows + rows_per_pass - 1) / rows_per_pass;
}

}  // namespace dflash
