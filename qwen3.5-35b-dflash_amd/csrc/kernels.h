// Kernel-side declarations shared by the kernel translation units and the C-ABI.
#pragma once

#include "common.h"

namespace dflash {

constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 64;
// Single-workgroup routing limits (LDS-resident slot map).
constexpr int kSmallPairs = 2048;       // T * k
constexpr int kSmallSlotBytes = 32768;  // roundup(T, 4) * E

__device__ __forceinline__ int wave_sum_int(int v) {
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Router tiles + activation prep + zeroing, in one launch (front_kernel).
struct FrontParams {
  const uint16_t* x;        // bf16 [T][H]
  const uint16_t* router_w; // bf16 [E][H]
  float* logits;            // fp32 [T][E]
  int T, E, H;
  int n_router;             // router tiles (0 when the logits are given)
  int router_big;           // 32 x 64 tiles (router_big_fits) instead of 16 x 16
  int prep_rows;            // rows of x to prepare (T, or 0: router tiles only, or the prep runs in route_topk's launch)
  uint16_t* x_il;           // octet-interleaved copy of x [T][H]
  float* xneg;              // -136 * sum per 128-column block [T][H/128]
  const uint16_t* gate_w;   // shared-expert gate vector [H] or null
  float* gate_out;          // sigmoid gate [T]
  uint32_t* zero;           // words cleared by the launch
  int64_t zero_words;
  int n_zero;               // blocks assigned to clearing
};

struct RouteParams {
  const float* logits;  // [T][E]
  int T, E, k;
  int32_t* ids;         // [T][k]
  float* wts;           // [T][k]
  int32_t* perm;        // [T*k]
  int32_t* inv;         // [T*k]
  int32_t* offsets;     // [E+1]
  int32_t* hit;         // [E] hit experts, ascending
  int32_t* pass_start;  // [E+2] first pass of each slot, then the total
  int32_t* meta;        // [0] hit experts, [1] total passes
  int32_t* counts;      // [E], followed in memory by the slot map (multi-workgroup path)
  uint8_t* slotmap;     // [E][route_slot_pitch(T)] bytes: slot + 1 of token t in expert e, or 0; 16-byte aligned
  int4* slot_table;     // [E+1] per slot: expert (-1 shared), segment start, rows, first pass
  int32_t* pass_slot;   // [T*k + T] slot of every pass
  int4* pass_table;     // [T*k + T] per pass: expert (-1 shared), segment start, slot rows, first row of the pass
  float* slot_w;        // [T*k] routing weight of every slot row (wts[perm[i]])
  int32_t* tok;         // [T*k] token of every slot row (perm[i] / k)
  int rows_per_pass;
  int has_shared;
  // prefill tile path (route_permute only): the routed experts' passes go into pass_table in
  // descending order of 16-row subtiles, the order in which the tile kernels' queue hands
  // them out (longest first); pass_slot is then not written for them
  int sort_passes;
  // activation prep by extra blocks of the route_topk launch (multi-workgroup routing only,
  // prep_rows > 0): rows of x converted as front_kernel's prep blocks would, while the routing
  // runs (no routing kernel reads them)
  const uint16_t* prep_x;
  uint16_t* prep_x_il;
  float* prep_xneg;
  const uint16_t* prep_gate_w;
  float* prep_gate_out;
  int prep_H, prep_rows;
};

struct TableParams {
  const int32_t* offsets;
  int E, T;
  int32_t* hit;
  int32_t* pass_start;
  int32_t* meta;
  int4* slot_table;
  int32_t* pass_slot;
  int4* pass_table;
  const int32_t* perm;
  const float* wts;
  float* slot_w;
  int32_t* tok;
  int k;
  int rows_per_pass, has_shared;
  // prep
  const uint16_t* x;
  int H;
  uint16_t* x_il;
  float* xneg;
  const uint16_t* gate_w;
  float* gate_out;
};

// Record slot `slot` (expert e, or -1 for the shared expert) in the work table.
__device__ __forceinline__ void write_slot(int4* slot_table, int32_t* pass_slot, int4* pass_table, int slot, int e,
                                           int seg, int rows, int pass0, int rows_per_pass) {
  slot_table[slot] = make_int4(e, seg, rows, pass0);
  const int n = (rows + rows_per_pass - 1) / rows_per_pass;
  for (int i = 0; i < n; ++i) {
    pass_slot[pass0 + i] = slot;
    pass_table[pass0 + i] = make_int4(e, seg, rows, i * rows_per_pass);
  }
}

enum W4Mode : int { kModeLinear = 0, kModeGateUp = 1, kModeDown = 2 };

// Persistent streaming W4A16 GEMM over the routing work table (w4_stream.hip).
struct W4StreamParams {
  const uint8_t* w;        // packed int4 [E][N][K/2] (or [N][K/2] for kModeLinear)
  const void* s;           // scales [E][N][K/G], bf16 or fp32
  const uint8_t* w_shared; // shared-expert packed [N][K/2] or null
  const void* s_shared;
  int64_t w_stride;        // bytes per expert
  int64_t s_stride;        // scale elements per expert
  int N, K, G;
  // activations: octet-interleaved bf16 rows of length K and their -136*sum
  // per 128-column block, given as neg_parts consecutive partial sums
  const uint16_t* act;
  const float* act_neg;
  int neg_parts;
  // work table (every input below lives in the workspace)
  const int32_t* tok;      // token of every routed slot row [T*k]
  const int32_t* meta;
  const int4* slot_table;  // per slot: expert (-1 shared), segment start, rows, first pass
  const int32_t* pass_slot;
  const int4* pass_table;  // per pass: expert (-1 shared), segment start, slot rows, first row of the pass
  int top_k, T, has_shared;
  int rows_per_pass;       // 16 * MT
  int strips;              // units per pass
  // outputs
  uint16_t* out_bf16;      // kModeLinear: [M][N]; kModeGateUp: h [(T*k+T)][N/2] interleaved
  float* out_part;         // kModeGateUp: [(T*k+T)][N/32] partial -136*sum(h) per 16 columns ([N/256] per 128 on the tile kernel)
  float* out_f32;          // kModeDown: y [(T*k+T)][N] (the tile kernel writes it as bf16);
                           // kModeLinear: when set, y [M][N] in fp32 instead of out_bf16
  const float* slot_w;     // kModeDown: routing weight of every slot row [T*k]
  const float* shared_gate;// kModeDown: sigmoid gate [T]
  int M;                   // kModeLinear rows
  int tiled;               // banks in the tiled layout (DFLASH_LAYOUT_TILED), else portable
  int tile_pieces;         // tile kernels: pieces per tile past the grid's last full round (0: by the grid)
};

// Portable -> tiled repack of a packed bank and its scales (repack.hip).
void launch_tile_w4(const void* packed, const void* scales, bool fp32_scales, int64_t experts, int rows, int cols,
                    int group, void* packed_out, void* scales_out, hipStream_t stream);
// int8-carried int4 values [experts][rows][cols] and group scales (dflash_dtype src) -> packed
// bank (portable or tiled) with fp32 scales; bad[0] / bad[1] count values outside [-8, 7] /
// negative or non-finite scales (cleared by the launch).
void launch_from_int8(const int8_t* values, const void* scales, int scales_dtype, int64_t experts, int rows,
                      int cols, int group, bool tiled, void* packed_out, float* scales_out, int32_t* bad,
                      hipStream_t stream);

void launch_front(const FrontParams& p, hipStream_t stream);
// Router tiles of a launch: 32 tokens x 64 experts when T >= 1024 and H in {512, 1024, 2048}, else 16 x 16.
bool router_big_fits(int T, int H);
int router_tiles(int T, int E, int H);
bool route_small_fits(int T, int E, int k);
// Row pitch of the multi-workgroup slot map: T rounded up to 16 bytes.
__host__ __device__ inline int route_slot_pitch(int T) { return (T + 15) & ~15; }
int64_t route_zero_words(int T, int E);
void launch_route(const RouteParams& p, bool zeroed, hipStream_t stream);
void launch_table_prep(const TableParams& p, hipStream_t stream);
// out = bf16(sum over slots of y rows): rows pre-weighted when wts is null, else weighted
// here by wts [T*k] (flat pair order) and gate [T] (shared expert).
void launch_combine(const float* y, const int32_t* inv, int T, int k, int H, int has_shared, const float* wts,
                    const float* gate, uint16_t* out, hipStream_t stream);
// The same over weighted bf16 y rows (the prefill tile path).
void launch_combine_bf16(const uint16_t* y, const int32_t* inv, int T, int k, int H, int has_shared, uint16_t* out,
                         hipStream_t stream);
// Per-wave fallback for any K % 512 == 0 (w4_gemm.hip); max_slots bounds the hit experts + shared.
void launch_w4_gemm(int mode, bool fp32_scales, int max_slots, const W4StreamParams& p, hipStream_t stream);
// K in {512, 1024, 2048} and group 128 (spill-free register budgets); K = 512 splits 4 ways with 2 row groups,
// larger K 8 ways with 1.
bool w4_stream_supports(int K, int G);
int w4_stream_row_groups(int K);
// mt: token tiles per pass (1 or 2); grid: persistent workgroups (one per CU)
void launch_w4_stream(int mode, bool fp32_scales, int mt, int grid, const W4StreamParams& p, hipStream_t stream);
// Verify-block expert kernels (w4_verify.hip), T <= 32 tokens: 16-row passes,
// group 128, K in {512, 1024, 2048}.  Each workgroup splits its contiguous
// range of units evenly over its 8 waves at k-block granularity; units split
// between waves meet in LDS.  The gate/up launch can route in its prologue, so a
// whole layer is front, gate/up, down, combine.
struct VerifyParams {
  W4StreamParams g;
  // dynamic LDS layout, byte offsets (verify_layout)
  int lds_a, lds_neg, lds_tok, lds_pdesc, lds_wgt, lds_part, lds_scratch, lds_bytes;  // lds_wgt: down's raw partials
  int pd_cap;        // pass descriptors the LDS holds
  int a_rows;        // activation rows the LDS holds (gate/up: T; linear: M; down: chunk_passes * 16)
  int chunk_passes;  // down (and gathered gate/up): passes whose activation rows are staged at once
  int gather;        // gate/up: stage per chunk only its passes' x rows, gathered by token (any T)
  // in-kernel routing (gate/up only; 1: one wave per token, 2: one 16-lane row per token):
  // fp32 logits [T][E] -> the dflash_moe_route outputs (written by workgroup 0) and the
  // work table of the down launch
  int route, E;
  const float* logits;
  int32_t* ids;
  float* wts;
  int32_t* perm;
  int32_t* inv;
  int32_t* offsets;
  int32_t* meta_out;       // [0] hit experts, [1] passes
  int4* pass_table_out;
  float* slot_w_out;
  int32_t* tok_out;
  // down plan: 3 int4 per down workgroup (pass count and first pass; the descriptors of its
  // first two passes), written by workgroup 0 of a routing gate/up launch, read by the down
  // launch (null: neither).  down_grid / down_strips: the down launch's grid and strips.
  int4* down_plan;
  int down_grid, down_strips;
  // split-K down in the gate/up launch (gate/up with in-kernel routing only): each workgroup
  // keeps the h columns of its unit range in LDS (lds_h: two pass slots x 16 rows x I, bf16
  // octet-interleaved, zero outside the range; lds_hstart: -136 * sum of each 32-column
  // quarter of each row) and multiplies them by the matching K-slice of the down bank (the
  // gate/up bank's layout and scale type), writing one fp32 partial y row per pass row into
  // ypart row 16 * (b + P) + r (workgroup b, pass P, pass row r; b + P never repeats).
  // Workgroup 0 writes row_seg: per slot row its first partial row and partial count
  // (consecutive partials 16 rows apart), which the combine sums in workgroup order.
  int fuse_down;
  const uint8_t* dw;         // down bank [E][H][I/2], shared expert's [H][I/2]
  const void* ds;
  const uint8_t* dw_shared;
  const void* ds_shared;
  int64_t dw_stride, ds_stride;  // bytes / scale elements per expert
  int dH, dI, dG;
  float* ypart;
  int2* row_seg;
  int part_rps;              // rows per partial segment: min(16, T)
  int lds_h, lds_hstart;
};
#ifdef DFLASH_TIMELINE
// Profiling build: phase timestamps of the verify and tile launches (timeline.py).
int timeline_verify_read(void* host, size_t bytes);
int timeline_verify_clear();
int timeline_tile_read(void* host, size_t bytes);
int timeline_tile_cycles_read(void* host, size_t bytes);
int timeline_tile_clear();
#endif
// LDS bytes and layout of one verify launch; false when it does not fit (the
// caller keeps the separate routing / streaming kernels then).
bool verify_layout(int mode, int T, int K, int N, int E, int k, int has_shared, int route, VerifyParams* vp);
void launch_w4_verify(int mode, bool fp32_scales, int grid, const VerifyParams& vp, hipStream_t stream);
// LDS the split-K down adds to a routing gate/up launch (two pass slots of h, quarter sums);
// fused_down_layout appends it to a gate/up layout whose block routes in the prologue with
// one 32-lane row per token, false when it does not fit.
int fused_down_lds(int I);
bool fused_down_layout(VerifyParams* vp, int I);
// out = bf16(sum over slots of w * (sum of the slot row's partial y rows)) (+ gate * shared row),
// partial rows as VerifyParams::row_seg lists them, fp32 in slot and partial order.
void launch_combine_parts(const float* ypart, const int2* row_seg, int rps, const int32_t* inv, int T, int k, int H,
                          int has_shared, const float* wts, const float* gate, uint16_t* out, hipStream_t stream);
// LDS-tiled kernel for long prefill (w4_tile.hip): 96-row passes, column tiles of 512
// (p.strips = I / 256 for gate_up, H / 512 for down), K % 512 == 0; its gate_up writes one
// -136*sum(h) per 128 columns and its down reads them that way; its down writes weighted
// y rows in bf16 (launch_combine_bf16).  Workgroups take tiles from a queue in meta[2]
// (gate/up) / meta[3] (down), zero on entry and left zero.
constexpr int kTileRowsPerPass = 96;
bool w4_tile_supports(int mode, int N, int K, int G);
void launch_w4_tile(int mode, bool fp32_scales, int grid, const W4StreamParams& p, hipStream_t stream);

// Latency-bound W4A16 linear for short blocks and narrow outputs (w4_small.hip): one workgroup
// per 16 output columns, each wave a run of 128-column k-blocks, every operand loaded straight
// into MFMA fragments up front and the waves' sums added once through LDS.
struct SmallLinearParams {
  const uint16_t* x;       // bf16 [M][K]
  const uint8_t* w;        // packed int4 [N][K/2], portable or tiled
  const void* s;           // scales [N][K/G] (tiled: [N/16][K/G][16]), bf16 or fp32
  void* y;                 // [M][N], bf16 or fp32
  int M, N, K, G;
  int tiled, scale_f32, y_f32;
};
// M <= 32, K in {512, 1024, 2048, 4096}, G in {128, 256}, N % 16 == 0
bool small_linear_fits(int M, int N, int K, int G);
void launch_w4_small(const SmallLinearParams& p, hipStream_t stream);
// its streaming form (persistent workgroups, x in registers): M <= 16
bool small_linear_stream_fits(int M, int N, int K, int G);
void launch_w4_small_stream(const SmallLinearParams& p, int grid, hipStream_t stream);

}  // namespace dflash
