/*
 * dflash_hip.h -- C ABI of the MI355X (gfx950) W4A16 qlinear / routed-MoE library.
 *
 * Plain C: pointers, sizes and status codes only.  Every entry point is
 * stream-ordered on the caller's HIP stream (passed as void*), never
 * allocates or frees device memory, never synchronises, and keeps no pointer
 * after it returns.  Scratch memory is a caller-provided workspace whose size
 * comes from the matching *_workspace_bytes() query, except for
 * dflash_moe_w4a16_noalloc, whose scratch is a static per-device array of the
 * library.  Device pointers must be 16-byte aligned.
 *
 * Weight format (reference model/qwen35_moe_dflash/graph/quant_weights.py:147-148,
 * graph/quant_plan.py:76-87,165): a logical weight W[E][N][K] is stored as
 * uint8 [E][N][K/2], signed two's-complement nibbles, k = 2j in the low nibble
 * of byte j and k = 2j+1 in the high nibble; scales are [E][N][K/G] (bf16 or
 * fp32), dequantised weight = q * scale[k / G].  Expert banks keep checkpoint
 * orientation: gate_up [E][2I][H] (gate rows first), down [E][H][I].
 *
 * Every function returns DFLASH_OK (0) or a nonzero status; the message of the
 * last failure on the calling thread is available from dflash_last_error().
 */
#ifndef DFLASH_HIP_H
#define DFLASH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFLASH_ABI_VERSION 6

enum dflash_status {
  DFLASH_OK = 0,
  DFLASH_ERR_INVALID_ARGUMENT = 1, /* null/misaligned pointer, bad size or layout */
  DFLASH_ERR_UNSUPPORTED = 2,      /* shape outside what the kernels implement */
  DFLASH_ERR_WORKSPACE = 3,        /* workspace missing or smaller than queried */
  DFLASH_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed */
};

enum dflash_dtype { DFLASH_DTYPE_BF16 = 0, DFLASH_DTYPE_F32 = 1, DFLASH_DTYPE_F16 = 2 /* source scales only */ };

/*
 * Byte order of a packed bank (same sizes either way):
 *   PORTABLE  the reference format above: packed [experts][rows][cols/2], scales
 *             [experts][rows][cols/group_size].
 *   TILED     this library's streaming order, made once by dflash_w4_to_tiled():
 *             per expert, per tile of 16 rows t and per 128-column block b, one
 *             contiguous 1 KB block whose byte 16*l + j (l = 0..63) is portable
 *             byte 64*b + 16*(l / 16) + j of row 16*t + l % 16; scales per expert
 *             [rows/16][cols/group_size][16], element [t][g][c] = portable [16*t + c][g].
 *             Every 64-lane 16-byte load of the expert kernels is then one
 *             contiguous kilobyte.  Needs rows % 16 == 0 and cols % 128 == 0.
 */
enum dflash_layout { DFLASH_LAYOUT_PORTABLE = 0, DFLASH_LAYOUT_TILED = 1 };

/* One packed int4 matrix (experts == 1) or expert bank (experts == E). */
typedef struct dflash_w4 {
  const void* packed;  /* uint8, experts * rows * cols / 2 bytes in `layout` order */
  const void* scales;  /* experts * rows * cols / group_size elements of scale_dtype, in `layout` order */
  int64_t experts;
  int64_t rows;        /* N: output features */
  int64_t cols;        /* K: input features */
  int64_t group_size;  /* 128 or 256 */
  int32_t scale_dtype; /* enum dflash_dtype */
  int32_t layout;      /* enum dflash_layout */
} dflash_w4;

/*
 * Repack a PORTABLE matrix or bank into the TILED layout (same shape fields,
 * group size and scale dtype; packed_out and scales_out are the caller's, the
 * size of src's arrays).  A one-time step at weight-load time, like the vendor
 * path's conversion to its own int4 layout (fused/quantization.py:112-115
 * expects I4ZN [K, N/8] for npu_quant_matmul); it has no counterpart in the
 * CPU reference.  Constraints: rows % 16 == 0, cols % 128 == 0.
 */
int dflash_w4_to_tiled(const dflash_w4* src, void* packed_out, void* scales_out, void* stream);

/*
 * Pack weights carried as one signed int8 per int4 value -- the original
 * checkpoint's format read by target/original_quant.py:214-272 (values int8
 * [experts][rows][cols] in [-8, 7]; group scales [experts][rows][cols/group_size]
 * in scales_dtype, fp16 or fp32 there, bf16 accepted too; a linear's trailing
 * [.., 1] axis is the same memory) -- into a bank in `layout` order with fp32 scales:
 * packed_out experts*rows*cols/2 bytes, scales_out experts*rows*cols/group_size
 * floats.  The reference packs the same values into its vendor layout instead
 * (pack_i4zn, :80-112).  invalid: two device int32 the call clears and fills with
 * the number of values outside [-8, 7] and of scales that are negative or not
 * finite (the reader's ValueError cases); they are valid once the stream reaches
 * them.  Constraints: cols % 32 == 0, group_size in {128, 256}, cols % group_size
 * == 0; TILED also rows % 16 == 0 and cols % 128 == 0.
 */
int dflash_w4_from_int8(const int8_t* values, const void* scales, int32_t scales_dtype, int64_t experts,
                        int64_t rows, int64_t cols, int64_t group_size, int32_t layout, void* packed_out,
                        float* scales_out, int32_t* invalid, void* stream);

/* ABI version of the loaded library (DFLASH_ABI_VERSION). */
int dflash_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* dflash_last_error(void);

/*
 * W4A16 quantized linear: y[m][n] = sum_k x[m][k] * q[n][k] * s[n][k/G].
 * x bf16 [m][K], y bf16 [m][N]; fp32 accumulation, one bf16 rounding.
 * Replaces the vendor QuantBatchMatmul call of
 * model/qwen35_moe_dflash/fused/quantization.py:154-165
 * (OriginalQuantizedWeights.linear; dynamic int8 activation quant is not used:
 * activations stay bf16 per specs/dflash-contract.json:104-113).
 * Constraints: N % 32 == 0, K % 512 == 0, group_size in {128, 256}.
 */
size_t dflash_qlinear_workspace_bytes(int64_t m, int64_t k, int64_t group_size);
int dflash_qlinear_w4a16(const void* x, int64_t m, const dflash_w4* weight, void* y, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * The same qlinear with y fp32 [m][N]: the fp32 sums, not rounded.  For a packed
 * router (the gate.weight key is linear_int4 in the portable plan,
 * graph/quant_plan.py:25-32), whose logits feed the top-k: the vendor path ranks
 * the QuantMatmul output (fused/quantization.py:183-184); here routing stays a
 * function of the unrounded fp32 logits, so it is bit-exact against a CPU top-k
 * of the same logits.  Same constraints and workspace as dflash_qlinear_w4a16.
 */
int dflash_qlinear_w4a16_f32(const void* x, int64_t m, const dflash_w4* weight, float* y, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Router logits, fp32 [tokens][experts] = hidden bf16 [tokens][H] . router_weight bf16 [E][H]^T,
 * accumulated in fp32 and not rounded (reference/fused_ops.py:161 computes the
 * same product; fp32 output keeps routing a function of exact logits).
 * Constraints: H % 256 == 0.
 */
int dflash_router_logits(const void* hidden, int64_t tokens, int64_t hidden_size, const void* router_weight,
                         int64_t experts, float* logits, void* stream);

/*
 * Top-k routing + stable expert permutation from fp32 logits [tokens][experts].
 * Replaces npu_moe_gating_top_k_softmax + renorm + npu_moe_init_routing_v2
 * (fused/quantization.py:184-192; reference/fused_ops.py:162-164):
 *   topk_ids     int32 [tokens][k]  experts by descending logit, lowest id on ties
 *   topk_weights fp32  [tokens][k]  softmax over the selected logits
 *   perm         int32 [tokens*k]   flat pair t*k+slot at each expert-sorted position
 *   inv_perm     int32 [tokens*k]   expert-sorted position of each flat pair
 *   expert_offsets int32 [experts+1] segment starts (tokens_per_expert = diff)
 * Constraints: experts <= 1024, 0 < k <= min(experts, 64).
 */
size_t dflash_moe_route_workspace_bytes(int64_t tokens, int64_t experts, int64_t top_k);
int dflash_moe_route(const float* logits, int64_t tokens, int64_t experts, int64_t top_k, int32_t* topk_ids,
                     float* topk_weights, int32_t* perm, int32_t* inv_perm, int32_t* expert_offsets,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Routed-MoE expert FFN over packed banks given a routing (from dflash_moe_route):
 * per expert segment, h = silu(x.Wg^T) * (x.Wu^T) (bf16), y = h.Wd^T; then
 * out[t] = sum_slot w[t][slot] * y[t][slot] (+ shared expert) in fp32, one bf16
 * rounding.  Replaces npu_grouped_matmul x2 + SiLU*up + npu_moe_finalize_routing
 * (fused/quantization.py:193-199) and the expert loop of reference/fused_ops.py:165-173.
 * The optional shared expert (shared_gate_up [2I][H], shared_down [H][I],
 * shared_gate_weight bf16 [H]) adds down(silu(gate(x))*up(x)) * sigmoid(x.w)
 * (fused/model.py:305-307); pass NULLs to leave it out.
 * Constraints: H % 512 == 0, I % 512 == 0, experts <= 1024, 0 < k <= 64.
 */
size_t dflash_moe_workspace_bytes(int64_t tokens, int64_t hidden_size, int64_t inter_size, int64_t experts,
                                  int64_t top_k, int64_t group_size, int has_shared);
int dflash_moe_experts_w4a16(const void* hidden, int64_t tokens, int64_t hidden_size, int64_t top_k,
                             const float* topk_weights, const int32_t* perm, const int32_t* inv_perm,
                             const int32_t* expert_offsets, const dflash_w4* gate_up, const dflash_w4* down,
                             const dflash_w4* shared_gate_up, const dflash_w4* shared_down,
                             const void* shared_gate_weight, void* out, void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * Whole routed-MoE layer (+ optional shared expert): router logits (from
 * router_weight bf16 [E][H], or taken as given when router_logits != NULL),
 * routing, expert FFN and combine.  The routing outputs are written to the
 * caller's arrays exactly as dflash_moe_route defines them.  Mirrors
 * OriginalQuantizedWeights.moe (fused/quantization.py:181-202) and the
 * FusedOps.moe contract (fused/ops.py:108-123) over packed banks.
 * For blocks of up to 32 tokens dflash_moe_workspace_bytes includes partial down
 * rows sized for the current device's CU count (room for the opt-in split-K down GEMM
 * inside the gate/up launch, dflash_set_split_down): query it with the call's device current.
 */
int dflash_moe_w4a16(const void* hidden, int64_t tokens, int64_t hidden_size, const float* router_logits,
                     const void* router_weight, int64_t top_k, const dflash_w4* gate_up, const dflash_w4* down,
                     const dflash_w4* shared_gate_up, const dflash_w4* shared_down, const void* shared_gate_weight,
                     void* out, float* logits_out, int32_t* topk_ids, float* topk_weights, int32_t* perm,
                     int32_t* inv_perm, int32_t* expert_offsets, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Split-K down GEMM of verify blocks (no counterpart in the reference, whose vendor path
 * runs two grouped GEMMs, fused/quantization.py:193-199).  A block of up to 32 tokens that
 * dflash_moe_w4a16 routes inside its gate/up launch, with banks of one scale dtype and H in
 * {512, 1024, 2048}, runs the down GEMM in that launch too: each workgroup multiplies
 * the h columns it produced by the matching K-slice of the down bank and writes fp32 partial
 * rows, which the combine adds in a fixed order (deterministic; the fp32 summation order
 * differs from the two-launch form).  Opt-in: dflash_set_split_down(1) turns it on
 * process-wide (off by default: on MI355X the separate down launch measured faster, 57.5
 * against 64.2 us per T=16 layer); dflash_moe_split_down returns 1 when a call of this shape runs it on
 * the current device, else 0.
 */
int dflash_set_split_down(int enable);

/*
 * Tail split of the long-prefill tile kernels (no counterpart in the reference; a test and
 * measurement override).  The tiles left over after the grid's last full round run in pieces:
 * by default 4 per tile when they fill at most a quarter of the grid, 2 when at most half,
 * else whole.  Pieces change only the fp32 summation order of h's -136*sum partials.
 * dflash_set_tile_pieces(1, 2 or 4) forces that many pieces, 0 restores the default.
 * Process-wide.
 */
int dflash_set_tile_pieces(int pieces);
int dflash_moe_split_down(int64_t tokens, int64_t hidden_size, int64_t inter_size, int64_t experts, int64_t top_k,
                          int64_t group_size, int has_shared, int32_t scale_dtype, int32_t layout);

/*
 * dflash_moe_w4a16 without a workspace: the same layer, arguments and results, with its
 * scratch in a static device array of DFLASH_NOALLOC_SCRATCH_BYTES (8 MiB) that each GPU
 * the library runs on holds until the process ends.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  It calls no allocating routine.
 * A layer whose dflash_moe_workspace_bytes() exceeds the scratch is refused with
 * DFLASH_ERR_UNSUPPORTED (at H=2048, I=512, E=256, top-8 + shared expert: up to 92 tokens).
 * All calls on one GPU share its scratch: calls that overlap on one GPU race.
 */
#define DFLASH_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int dflash_moe_w4a16_noalloc(const void* hidden, int64_t tokens, int64_t hidden_size, const float* router_logits,
                             const void* router_weight, int64_t top_k, const dflash_w4* gate_up,
                             const dflash_w4* down, const dflash_w4* shared_gate_up, const dflash_w4* shared_down,
                             const void* shared_gate_weight, void* out, float* logits_out, int32_t* topk_ids,
                             float* topk_weights, int32_t* perm, int32_t* inv_perm, int32_t* expert_offsets,
                             void* stream);

/*
 * Measurement mode (no counterpart in the reference; for benchmarks and
 * profilers that time one kernel of the layer on its own): while a stage is
 * set, dflash_moe_w4a16 and dflash_moe_experts_w4a16 validate their arguments
 * as usual but launch only that stage's kernel, which reads the routing, work
 * table and intermediate activations that an earlier full call with the same
 * arguments left in the same workspace, and writes the same intermediate
 * output again (out is not written).  On the verify path (T <= 32) the gate/up
 * kernel also routes the block in its prologue; in measurement mode it does so
 * only when the call passes router_logits (else it reads the work table).
 * Where dflash_moe_w4a16 runs the down GEMM inside the gate/up launch (a verify
 * block routed in that launch, dflash_moe_split_down), DFLASH_STAGE_EXPERTS with
 * router_logits relaunches that one kernel; GATE_UP and DOWN alone, or EXPERTS
 * without router_logits, run the separate verify gate/up and down kernels of
 * the same layer instead.
 * DFLASH_STAGE_NONE restores full calls.  Process-wide.
 */
enum dflash_stage {
  DFLASH_STAGE_NONE = 0,
  DFLASH_STAGE_GATE_UP = 1, /* grouped gate/up GEMM + SiLU*up of the expert FFN */
  DFLASH_STAGE_DOWN = 2,    /* grouped down GEMM of the expert FFN */
  DFLASH_STAGE_EXPERTS = 3  /* every expert GEMM kernel of the call (gate/up and down) */
};
int dflash_set_measure_stage(int stage);

#ifdef __cplusplus
}
#endif

#endif /* DFLASH_HIP_H */
