// Kernel-side declarations shared by the kernel translation units and the C-ABI.
#pragma once

#include "common.h"

namespace dflash {

// Single-workgroup routing limits (LDS-resident ids and membership bitmap).
constexpr int kSmallPairs = 2048;        // T * k
constexpr int kSmallBitmapWords = 8192;  // T * ceil(E / 32)
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 64;

enum W4Mode : int { kModeLinear = 0, kModeGateUp = 1, kModeDown = 2 };

// One launch of the small-M grouped W4A16 GEMM.  A "slot" is a hit expert
// (or the shared expert, which follows the hit experts); a work item is one
// wave computing a 32-row strip of the slot's weight matrix for all of the
// slot's tokens.
struct W4GemmParams {
  const uint8_t* w;        // packed int4 [E][N][K/2] (or [N][K/2] for kModeLinear)
  const void* s;           // scales [E][N][K/G], bf16 or fp32
  const uint8_t* w_shared; // shared-expert packed [N][K/2] or null
  const void* s_shared;    // shared-expert scales [N][K/G]
  int64_t w_stride;        // bytes per expert
  int64_t s_stride;        // scale elements per expert
  int N, K, G;
  // activations: octet-interleaved bf16 rows of length K, and -136*sum terms
  const uint16_t* act;
  const float* act_neg;    // [rows][K/G] (kNegParts == 1) or [rows][K/16] partials
  // routing
  const int32_t* perm;     // sorted position -> flat pair t*k+slot
  const int32_t* offsets;  // [E+1]
  const int32_t* hit;      // hit experts, ascending
  const int32_t* meta;     // meta[0] = number of hit experts
  int top_k, T, has_shared;
  // outputs
  uint16_t* out_bf16;      // kModeLinear: [M][N]; kModeGateUp: h [(T*k+T)][N/2] interleaved
  float* out_part;         // kModeGateUp: [(T*k+T)][N/32] partial -136*sum(h) per 16 columns
  float* out_f32;          // kModeDown: y [(T*k+T)][N]
  const float* route_w;    // kModeDown: flat routing weights [T*k]
  const float* shared_gate;// kModeDown: sigmoid gate [T]
  int M;                   // kModeLinear rows
  int items_per_slot;
  int max_slots;
};

void launch_prep(const uint16_t* x, int rows, int K, int group, uint16_t* x_il, float* xneg, const uint16_t* gate_w,
                 float* gate_out, hipStream_t stream);
void launch_router(const uint16_t* x, const uint16_t* w, float* logits, int T, int E, int H, hipStream_t stream);
bool route_small_fits(int T, int E, int k);
void launch_route(const float* logits, int T, int E, int k, int32_t* ids, float* wts, int32_t* perm, int32_t* inv,
                  int32_t* offsets, int32_t* hit, int32_t* meta, int32_t* counts, uint32_t* bitmap, bool allow_small,
                  hipStream_t stream);
void launch_hitlist(const int32_t* offsets, int E, int32_t* hit, int32_t* meta, hipStream_t stream);
void launch_combine(const float* y, const int32_t* inv, int T, int k, int H, int has_shared, uint16_t* out,
                    hipStream_t stream);
void launch_w4_gemm(int mode, bool fp32_scales, const W4GemmParams& p, hipStream_t stream);

}  // namespace dflash
