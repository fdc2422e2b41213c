// Router logits, top-k routing with renormalised weights, the stable
// token-to-expert permutation, activation preparation and the final combine.
//
// Routing contract (reference reference/fused_ops.py:160-164,
// graph/fused/quant_target.py:168-172): rank the fp32 logits in descending
// order, lowest expert id first among equal logits; weights are the softmax of
// the selected logits (the full-softmax denominator cancels in the renorm).
// Permutation contract (npu_moe_init_routing_v2 as documented in
// docs/reference/qwen35-moe-operators-and-quantization-analysis.md:685-707):
// flat pairs t*k+slot sorted by expert, stable, so a segment lists its tokens
// in ascending order.
#include "kernels.h"

namespace dflash {

// ---------------------------------------------------------------------------
// Activation preparation: octet-interleaved copy of x, -136*sum per group and
// (optionally) the shared-expert gate sigmoid(x . w_gate).
// grid = rows, block = 256.  Requires K % 8 == 0 and group % 8 == 0, group <= 512.
__global__ __launch_bounds__(256) void prep_kernel(const uint16_t* __restrict__ x, int K, int group,
                                                   uint16_t* __restrict__ x_il, float* __restrict__ xneg,
                                                   const uint16_t* __restrict__ gate_w,
                                                   float* __restrict__ gate_out) {
  const int row = blockIdx.x;
  const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(row) * K);
  uint4* dst = reinterpret_cast<uint4*>(x_il + static_cast<int64_t>(row) * K);
  const int chunks = K >> 3;
  const int per_group = group >> 3;
  float gate_acc = 0.f;
  for (int base = 0; base < chunks; base += 256) {
    const int c = base + threadIdx.x;
    float sum = 0.f;
    if (c < chunks) {
      const uint4 v = src[c];
      // natural pairs (0,1)(2,3)(4,5)(6,7) -> (0,4)(1,5)(2,6)(3,7)
      uint4 o;
      o.x = (v.x & 0xFFFFu) | (v.z << 16);
      o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
      o.z = (v.y & 0xFFFFu) | (v.w << 16);
      o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
      dst[c] = o;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      float gw[8];
      if (gate_w) {
        const uint4 g = reinterpret_cast<const uint4*>(gate_w)[c];
        const uint32_t gg[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          gw[2 * i] = __uint_as_float(gg[i] << 16);
          gw[2 * i + 1] = __uint_as_float(gg[i] & 0xFFFF0000u);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xFFFF0000u);
        sum += lo + hi;
        if (gate_w) gate_acc += lo * gw[2 * i] + hi * gw[2 * i + 1];
      }
    }
    // group sums: per_group consecutive chunks sit in consecutive lanes of one wave
    for (int o = 1; o < per_group; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if (c < chunks && (c % per_group) == 0) xneg[static_cast<int64_t>(row) * (K / group) + c / per_group] = -kDequantOffset * sum;
  }
  if (gate_w) {
    __shared__ float part[4];
    gate_acc = wave_sum(gate_acc);
    if (lane_id() == 0) part[threadIdx.x >> 6] = gate_acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      const float z = part[0] + part[1] + part[2] + part[3];
      gate_out[row] = 1.0f / (1.0f + __expf(-z));
    }
  }
}

// ---------------------------------------------------------------------------
// Router logits fp32 [T][E] = x bf16 [T][H] . W bf16 [E][H]^T on MFMA.
// grid = (ceil(T/16), ceil(E/16)), block = 512 (8 waves split H; H % 256 == 0).
__global__ __launch_bounds__(512) void router_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     float* __restrict__ logits, int T, int E, int H) {
  __shared__ f32x4 red[8][64];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int lr = lane & 15, kq = lane >> 4;
  const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
  const int trow = min(t0 + lr, T - 1), erow = min(e0 + lr, E - 1);
  const int span = H >> 3;
  const uint16_t* xa = x + static_cast<int64_t>(trow) * H + wave * span + kq * 8;
  const uint16_t* wb = w + static_cast<int64_t>(erow) * H + wave * span + kq * 8;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < span; k += 32) {
    const uint4 a = *reinterpret_cast<const uint4*>(xa + k);
    const uint4 b = *reinterpret_cast<const uint4*>(wb + k);
    acc = mfma16x16x32(a, b, acc);
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

// ---------------------------------------------------------------------------
// Top-k of one token's logits by one wave.  Lane s < k ends with (id, weight).
// Keys: order-preserving uint32 of the float (-0 folded to +0, NaN lowest),
// packed with ~id so one 64-bit max picks the larger logit, then the lower id.
__device__ __forceinline__ uint32_t sortable_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0u;  // NaN ranks last
  if ((u & 0x7FFFFFFFu) == 0u) u = 0u;             // -0 == +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int kPer>
__device__ __forceinline__ void wave_topk(const float* __restrict__ row, int E, int k, int* id_out,
                                          float* w_out) {
  const int lane = lane_id();
  uint64_t key[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = lane + 64 * i;
    key[i] = (e < E) ? ((static_cast<uint64_t>(sortable_key(row[e])) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(e)))
                     : 0ull;
  }
  int my_id = -1;
  uint32_t my_key = 0;
  for (int s = 0; s < k; ++s) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) best = key[i] > best ? key[i] : best;
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    const int e = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(best));
    if ((e & 63) == lane) {
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (lane + 64 * i == e) key[i] = 0ull;
    }
    if (lane == s) {
      my_id = e;
      my_key = static_cast<uint32_t>(best >> 32);
    }
  }
  const float top = key_to_float(__shfl(my_key, 0, 64));
  const float ex = (lane < k) ? expf(key_to_float(my_key) - top) : 0.f;
  const float total = wave_sum(ex);
  *id_out = my_id;
  *w_out = ex / total;
}

__device__ __forceinline__ void topk_any(const float* row, int E, int k, int* id, float* w) {
  if (E <= 64) wave_topk<1>(row, E, k, id, w);
  else if (E <= 128) wave_topk<2>(row, E, k, id, w);
  else if (E <= 256) wave_topk<4>(row, E, k, id, w);
  else if (E <= 512) wave_topk<8>(row, E, k, id, w);
  else wave_topk<16>(row, E, k, id, w);
}

// ---------------------------------------------------------------------------
// Single-workgroup routing for small T: top-k, counts, offsets, hit list and
// the stable permutation without leaving the workgroup.
// block = 1024; T*k <= kSmallPairs, E <= 1024, k <= 64.
__global__ __launch_bounds__(1024) void route_small_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                           int32_t* __restrict__ ids, float* __restrict__ wts,
                                                           int32_t* __restrict__ perm, int32_t* __restrict__ inv,
                                                           int32_t* __restrict__ offsets, int32_t* __restrict__ hit,
                                                           int32_t* __restrict__ meta) {
  __shared__ int counts[1024];
  __shared__ int offs[1024];
  __shared__ int wave_tot[2][16];
  __shared__ int lds_ids[kSmallPairs];
  __shared__ uint32_t bits[kSmallBitmapWords];
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  const int words = (E + 31) >> 5;
  for (int i = tid; i < 1024; i += 1024) counts[i] = 0;
  for (int i = tid; i < T * words; i += 1024) bits[i] = 0u;
  __syncthreads();
  for (int t = wave; t < T; t += 16) {
    int id;
    float w;
    topk_any(logits + static_cast<int64_t>(t) * E, E, k, &id, &w);
    if (lane < k) {
      ids[t * k + lane] = id;
      wts[t * k + lane] = w;
      lds_ids[t * k + lane] = id;
      atomicAdd(&counts[id], 1);
      atomicOr(&bits[t * words + (id >> 5)], 1u << (id & 31));
    }
  }
  __syncthreads();
  // exclusive scans over experts: token offsets and hit-list positions
  const int cnt = tid < E ? counts[tid] : 0;
  int incl = cnt, nz = cnt > 0 ? 1 : 0;
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(incl, o, 64), b = __shfl_up(nz, o, 64);
    if (lane >= o) {
      incl += a;
      nz += b;
    }
  }
  if (lane == 63) {
    wave_tot[0][wave] = incl;
    wave_tot[1][wave] = nz;
  }
  __syncthreads();
  int base = 0, nzbase = 0;
  for (int i = 0; i < wave; ++i) {
    base += wave_tot[0][i];
    nzbase += wave_tot[1][i];
  }
  const int excl = base + incl - cnt;
  const int nzexcl = nzbase + nz - (cnt > 0 ? 1 : 0);
  if (tid < E) {
    offs[tid] = excl;
    offsets[tid] = excl;
    if (cnt > 0) hit[nzexcl] = tid;
    if (tid == E - 1) {
      offsets[E] = excl + cnt;
      meta[0] = nzexcl + (cnt > 0 ? 1 : 0);
    }
  }
  __syncthreads();
  // stable ranks: expert tid walks the tokens in ascending order
  if (tid < E && cnt > 0) {
    int pos = offs[tid];
    const int wi = tid >> 5;
    const uint32_t bit = 1u << (tid & 31);
    for (int t = 0; t < T; ++t) {
      if (bits[t * words + wi] & bit) {
        int s = 0;
        while (s < k && lds_ids[t * k + s] != tid) ++s;
        if (s < k) {
          perm[pos] = t * k + s;
          inv[t * k + s] = pos;
        }
        ++pos;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Multi-workgroup routing for large T.
__global__ void route_zero_kernel(int32_t* __restrict__ counts, int E) {
  for (int i = threadIdx.x; i < E; i += blockDim.x) counts[i] = 0;
}

// grid = ceil(T/4), block = 256: one wave per token.
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                         int32_t* __restrict__ ids, float* __restrict__ wts,
                                                         int32_t* __restrict__ counts, uint32_t* __restrict__ bitmap) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = lane_id();
  if (t >= T) return;
  int id;
  float w;
  topk_any(logits + static_cast<int64_t>(t) * E, E, k, &id, &w);
  if (lane < k) {
    ids[static_cast<int64_t>(t) * k + lane] = id;
    wts[static_cast<int64_t>(t) * k + lane] = w;
    atomicAdd(&counts[id], 1);
  }
  // E <= 1024 keeps the bitmap row within 32 words: lane w builds word w.
  const int words = (E + 31) >> 5;
  uint32_t word = 0;
  for (int s = 0; s < k; ++s) {
    const int e = __shfl(id, s, 64);  // uniform loop: every lane takes part
    if ((e >> 5) == lane) word |= 1u << (e & 31);
  }
  if (lane < words) bitmap[static_cast<int64_t>(t) * words + lane] = word;
}

// grid = ceil(E/4), block = 256: one wave per expert.
__global__ __launch_bounds__(256) void route_permute_kernel(const int32_t* __restrict__ ids, const int32_t* __restrict__ counts,
                                                            const uint32_t* __restrict__ bitmap, int T, int E, int k,
                                                            int32_t* __restrict__ perm, int32_t* __restrict__ inv,
                                                            int32_t* __restrict__ offsets, int32_t* __restrict__ hit,
                                                            int32_t* __restrict__ meta) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = lane_id();
  if (e >= E) return;
  int before = 0, nz_before = 0;
  for (int i = lane; i < e; i += 64) {
    const int c = counts[i];
    before += c;
    nz_before += c > 0 ? 1 : 0;
  }
  for (int o = 1; o < 64; o <<= 1) {
    before += __shfl_xor(before, o, 64);
    nz_before += __shfl_xor(nz_before, o, 64);
  }
  const int cnt = counts[e];
  if (lane == 0) {
    offsets[e] = before;
    if (cnt > 0) hit[nz_before] = e;
    if (e == E - 1) {
      offsets[E] = before + cnt;
      meta[0] = nz_before + (cnt > 0 ? 1 : 0);
    }
  }
  if (cnt == 0) return;
  const int words = (E + 31) >> 5;
  const uint32_t bit = 1u << (e & 31);
  int running = 0;
  for (int t0 = 0; t0 < T; t0 += 64) {
    const int t = t0 + lane;
    const bool mine = t < T && (bitmap[static_cast<int64_t>(t) * words + (e >> 5)] & bit);
    const uint64_t mask = __ballot(mine);
    if (mine) {
      const int rank = running + __popcll(mask & ((1ull << lane) - 1ull));
      const int pos = before + rank;
      int s = 0;
      while (s < k && ids[static_cast<int64_t>(t) * k + s] != e) ++s;
      if (s < k) {
        perm[pos] = t * k + s;
        inv[t * k + s] = pos;
      }
    }
    running += __popcll(mask);
  }
}

// ---------------------------------------------------------------------------
// Hit list from existing segment offsets (experts with a nonempty segment, in
// ascending order).  block = 1024, E <= 1024.
__global__ __launch_bounds__(1024) void hitlist_kernel(const int32_t* __restrict__ offsets, int E,
                                                       int32_t* __restrict__ hit, int32_t* __restrict__ meta) {
  __shared__ int wave_nz[16];
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  const int nonempty = (tid < E && offsets[tid + 1] > offsets[tid]) ? 1 : 0;
  int incl = nonempty;
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(incl, o, 64);
    if (lane >= o) incl += a;
  }
  if (lane == 63) wave_nz[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < wave; ++i) base += wave_nz[i];
  if (nonempty) hit[base + incl - 1] = tid;
  if (tid == E - 1) meta[0] = base + incl;
}

// ---------------------------------------------------------------------------
// Combine: out[t] = sum_slot y[inv[t*k+slot]] (+ y[T*k + t] for the shared
// expert), fp32 in slot order, one bf16 rounding.  grid = T, block = 256.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, const int32_t* __restrict__ inv, int T,
                                                      int k, int H, int has_shared, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  for (int c = threadIdx.x * 8; c < H; c += 256 * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < k; ++s) {
      const float4* src = reinterpret_cast<const float4*>(y + static_cast<int64_t>(inv[t * k + s]) * H + c);
      const float4 a = src[0], b = src[1];
      acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
      acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
    }
    if (has_shared) {
      const float4* src = reinterpret_cast<const float4*>(y + (static_cast<int64_t>(T) * k + t) * H + c);
      const float4 a = src[0], b = src[1];
      acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
      acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
    }
    uint4 o;
    o.x = f32_to_bf16(acc[0]) | (static_cast<uint32_t>(f32_to_bf16(acc[1])) << 16);
    o.y = f32_to_bf16(acc[2]) | (static_cast<uint32_t>(f32_to_bf16(acc[3])) << 16);
    o.z = f32_to_bf16(acc[4]) | (static_cast<uint32_t>(f32_to_bf16(acc[5])) << 16);
    o.w = f32_to_bf16(acc[6]) | (static_cast<uint32_t>(f32_to_bf16(acc[7])) << 16);
    *reinterpret_cast<uint4*>(out + static_cast<int64_t>(t) * H + c) = o;
  }
}

// ---------------------------------------------------------------------------
// host launchers
void launch_prep(const uint16_t* x, int rows, int K, int group, uint16_t* x_il, float* xneg, const uint16_t* gate_w,
                 float* gate_out, hipStream_t stream) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(prep_kernel, dim3(rows), dim3(256), 0, stream, x, K, group, x_il, xneg, gate_w, gate_out);
}

void launch_router(const uint16_t* x, const uint16_t* w, float* logits, int T, int E, int H, hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(router_kernel, dim3((T + 15) / 16, (E + 15) / 16), dim3(512), 0, stream, x, w, logits, T, E, H);
}

bool route_small_fits(int T, int E, int k) {
  return static_cast<int64_t>(T) * k <= kSmallPairs && static_cast<int64_t>(T) * ((E + 31) / 32) <= kSmallBitmapWords;
}

void launch_route(const float* logits, int T, int E, int k, int32_t* ids, float* wts, int32_t* perm, int32_t* inv,
                  int32_t* offsets, int32_t* hit, int32_t* meta, int32_t* counts, uint32_t* bitmap, bool allow_small,
                  hipStream_t stream) {
  if (allow_small && route_small_fits(T, E, k)) {
    hipLaunchKernelGGL(route_small_kernel, dim3(1), dim3(1024), 0, stream, logits, T, E, k, ids, wts, perm, inv, offsets,
                       hit, meta);
    return;
  }
  hipLaunchKernelGGL(route_zero_kernel, dim3(1), dim3(256), 0, stream, counts, E);
  if (T > 0)
    hipLaunchKernelGGL(route_topk_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, logits, T, E, k, ids, wts, counts,
                       bitmap);
  hipLaunchKernelGGL(route_permute_kernel, dim3((E + 3) / 4), dim3(256), 0, stream, ids, counts, bitmap, T, E, k, perm,
                     inv, offsets, hit, meta);
}

void launch_hitlist(const int32_t* offsets, int E, int32_t* hit, int32_t* meta, hipStream_t stream) {
  hipLaunchKernelGGL(hitlist_kernel, dim3(1), dim3(1024), 0, stream, offsets, E, hit, meta);
}

void launch_combine(const float* y, const int32_t* inv, int T, int k, int H, int has_shared, uint16_t* out,
                    hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(256), 0, stream, y, inv, T, k, H, has_shared, out);
}

}  // namespace dflash
