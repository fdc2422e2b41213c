// extern "C" entry points of libdflash_hip.so (declared in include/dflash_hip.h).
//
// Each entry validates shapes and pointers on the host, carves the caller's
// workspace, and enqueues kernels on the caller's stream.  No allocation, no
// synchronisation, no C++ exception crosses the ABI.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

#include "../../include/dflash_hip.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DFLASH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return DFLASH_OK;
}

size_t align256(size_t v) { return (v + 255u) & ~static_cast<size_t>(255u); }

struct Carver {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  }
};

int check_w4(const dflash_w4* w, const char* name, int64_t experts, int64_t rows, int64_t cols) {
  if (!w) return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": descriptor is NULL");
  if (!w->packed || !w->scales) return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": NULL packed or scales");
  if (!aligned16(w->packed)) return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": packed weights not 16-byte aligned");
  if (w->scale_dtype != DFLASH_DTYPE_BF16 && w->scale_dtype != DFLASH_DTYPE_F32)
    return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": scale_dtype must be BF16 or F32");
  const size_t sal = w->scale_dtype == DFLASH_DTYPE_F32 ? 4u : 2u;
  if (reinterpret_cast<uintptr_t>(w->scales) % sal)
    return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": scales misaligned");
  if (w->experts != experts || w->rows != rows || w->cols != cols)
    return fail(DFLASH_ERR_INVALID_ARGUMENT,
                std::string(name) + ": expected [" + std::to_string(experts) + "," + std::to_string(rows) + "," +
                    std::to_string(cols) + "], got [" + std::to_string(w->experts) + "," + std::to_string(w->rows) +
                    "," + std::to_string(w->cols) + "]");
  if (w->group_size != 128 && w->group_size != 256)
    return fail(DFLASH_ERR_UNSUPPORTED, std::string(name) + ": group_size must be 128 or 256");
  if (cols % w->group_size) return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": K not a multiple of group_size");
  if (w->layout != DFLASH_LAYOUT_PORTABLE && w->layout != DFLASH_LAYOUT_TILED)
    return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": layout must be PORTABLE or TILED");
  if (w->layout == DFLASH_LAYOUT_TILED && (rows % 16 || cols % 128))
    return fail(DFLASH_ERR_INVALID_ARGUMENT, std::string(name) + ": the tiled layout needs rows % 16 == 0 and cols % 128 == 0");
  return DFLASH_OK;
}

// The per-wave fallback kernel (w4_gemm) reads portable rows only.
int tiled_unsupported(const char* what) {
  return fail(DFLASH_ERR_UNSUPPORTED, std::string(what) +
                                          ": tiled weights are streamed by the verify, streaming and tile kernels "
                                          "only (group size 128 for T <= 32 and the streaming path); use the "
                                          "portable layout for this shape");
}

// ---------------------------------------------------------------- layouts
struct RouteLayout {
  size_t meta, hit, pass_start, slot_table, pass_slot, pass_table, slot_w, tok, counts, slotmap, total;
};

RouteLayout route_layout(int64_t T, int64_t k, int64_t E) {
  Carver c;
  RouteLayout L;
  L.meta = c.take(16);
  L.hit = c.take(4 * static_cast<size_t>(E + 1));
  L.pass_start = c.take(4 * static_cast<size_t>(E + 4));
  L.slot_table = c.take(16 * static_cast<size_t>(E + 2));
  L.pass_slot = c.take(4 * static_cast<size_t>(T * k + T + 4));  // a pass holds at least one row
  L.pass_table = c.take(16 * static_cast<size_t>(T * k + T + 4));
  L.slot_w = c.take(4 * static_cast<size_t>(T * k + 1));
  L.tok = c.take(4 * static_cast<size_t>(T * k + 1));
  // counts and the slot map are contiguous: one clearing pass covers both
  L.counts = c.off;
  L.slotmap = L.counts + 4 * static_cast<size_t>((E + 3) & ~3);
  c.take(4 * static_cast<size_t>(dflash::route_zero_words(static_cast<int>(T), static_cast<int>(E))) + 16);
  L.total = c.off;
  return L;
}

// The down plan of the verify path covers persistent grids up to this many workgroups.
constexpr int kDownPlanMaxGrid = 1024;

// Split-K down of the verify path: rows per partial segment (min(16, T)) and the partial
// y rows it may write on a grid of `grid` workgroups: rps * (grid + passes), at most
// min(E, T k) * ceil(T / 16) routed passes plus ceil(T / 16) of the shared expert.
int64_t part_rps(int64_t T) { return std::min<int64_t>(16, T); }
int64_t verify_pass_cap(int64_t T, int64_t E, int64_t k, bool shared) {
  const int64_t tp = (T + 15) / 16;
  return std::min(E, T * k) * tp + (shared ? tp : 0);
}

struct MoeLayout {
  RouteLayout route;
  size_t logits, x_il, xneg, gate, h, hpart, y, down_plan;
  size_t ypart, row_seg;  // split-K down (parts_grid > 0): partial y rows, per slot row its partials
  int parts_grid;         // the grid the partial rows cover, 0 without them
  size_t total;
};

MoeLayout moe_layout(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, bool shared, int parts_grid = 0) {
  MoeLayout L;
  L.route = route_layout(T, k, E);
  Carver c;
  c.off = L.route.total;
  const size_t rows = static_cast<size_t>(T) * k + (shared ? T : 0);
  L.logits = c.take(4 * static_cast<size_t>(T) * E);
  L.x_il = c.take(2 * static_cast<size_t>(T) * H);
  L.xneg = c.take(4 * static_cast<size_t>(T) * (H / 128));
  L.gate = c.take(4 * static_cast<size_t>(T));
  L.h = c.take(2 * rows * I);
  L.hpart = c.take(4 * rows * (I / 16));
  L.y = c.take(4 * rows * H);
  L.down_plan = c.take(48 * static_cast<size_t>(kDownPlanMaxGrid));
  L.parts_grid = parts_grid;
  L.ypart = L.row_seg = 0;
  if (parts_grid > 0) {
    const int64_t prow = part_rps(T) * (parts_grid + verify_pass_cap(T, E, k, shared));
    L.ypart = c.take(4 * static_cast<size_t>(prow) * H);
    L.row_seg = c.take(8 * rows);
  }
  L.total = c.off;
  return L;
}

template <typename T>
T* at(void* base, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

// Scratch of dflash_moe_w4a16_noalloc: one copy per device, held until the process ends.
// In host code `scratch` names a host-side stand-in, never the device memory: kernels and
// copies get the address that hipGetSymbolAddress returns for the current device.  Every
// call on a device shares that device's copy, so calls that overlap on one device race;
// each call's kernels clear what must start at zero (routing counters, slot map, tile
// queues) before using it.
constexpr size_t kScratchBytes = DFLASH_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DFLASH_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(DFLASH_ERR_UNSUPPORTED, "device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DFLASH_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DFLASH_OK;
}

// Compute units of the current device (persistent grids launch one workgroup per CU).
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

int token_tiles(int64_t T) { return T <= 16 ? 1 : 2; }

// Blocks of up to 32 tokens keep all their x rows in the verify gate/up launch's LDS (and
// may route inside it); larger ones stage x rows per chunk of passes, gathered by token.
constexpr int64_t kVerifyMaxTokens = 32;

int check_route_args(int64_t T, int64_t E, int64_t k) {
  if (T < 0) return fail(DFLASH_ERR_INVALID_ARGUMENT, "tokens must be >= 0");
  if (T > (1 << 24)) return fail(DFLASH_ERR_UNSUPPORTED, "tokens above 2^24 are not supported");
  if (E <= 0 || E > dflash::kMaxExperts) return fail(DFLASH_ERR_UNSUPPORTED, "experts must be in [1, 1024]");
  if (k <= 0 || k > E || k > dflash::kMaxTopK)
    return fail(DFLASH_ERR_INVALID_ARGUMENT, "top_k must be in (0, min(experts, 64)]");
  // routing offsets and buffer sizes (T*k*4 bytes, byte offsets of (T*k + T) rows) stay in 32 bits
  if (T * k > (int64_t(1) << 28)) return fail(DFLASH_ERR_UNSUPPORTED, "tokens * top_k above 2^28 is not supported");
  return DFLASH_OK;
}

struct MoeShapes {
  int64_t T, H, I, E, k, G, Gd;  // Gd: group size of the down bank
  bool shared;
  bool gu_f32, dn_f32;
  bool scales16;  // every scale bank 16-byte aligned (row scales load as 16-byte words)
  bool tiled;     // every bank in the tiled layout
};

// Long prefill (at least 16 rows per expert on average) runs both expert GEMMs
// on the LDS-tiled kernel, whose passes hold 96 rows.
bool moe_tile_path(const MoeShapes& S) {
  using namespace dflash;
  const int64_t rows = S.T * S.k + S.T;
  return S.T * S.k >= 16 * S.E && rows * std::max(S.H, S.I) < (int64_t(1) << 31) &&
         w4_tile_supports(kModeGateUp, static_cast<int>(2 * S.I), static_cast<int>(S.H), static_cast<int>(S.G)) &&
         w4_tile_supports(kModeDown, static_cast<int>(S.H), static_cast<int>(S.I), static_cast<int>(S.Gd));
}

bool verify_fits(const MoeShapes& S, bool route, dflash::VerifyParams* gu, dflash::VerifyParams* dn);

// Rows per pass of the work table: 16 on the verify path (T <= 32), 96 on
// the prefill tile path, else 16 per token tile of the streaming kernel.
int rows_per_pass(const MoeShapes& S) {
  dflash::VerifyParams gu, dn;
  if (verify_fits(S, false, &gu, &dn)) return 16;
  if (moe_tile_path(S)) return dflash::kTileRowsPerPass;
  return 16 * token_tiles(S.T);
}

int check_moe(const void* hidden, int64_t T, int64_t H, int64_t k, const dflash_w4* gate_up, const dflash_w4* down,
              const dflash_w4* sgu, const dflash_w4* sdn, const void* sgate, const void* out, MoeShapes* S) {
  if (!gate_up || !down) return fail(DFLASH_ERR_INVALID_ARGUMENT, "gate_up and down descriptors are required");
  const int64_t E = gate_up->experts, I2 = gate_up->rows;
  if (I2 <= 0 || I2 % 2) return fail(DFLASH_ERR_INVALID_ARGUMENT, "gate_up rows must be 2*I");
  const int64_t I = I2 / 2;
  if (int r = check_route_args(T, E, k)) return r;
  if (H <= 0 || H % 512) return fail(DFLASH_ERR_UNSUPPORTED, "hidden_size must be a positive multiple of 512");
  if (I % 512) return fail(DFLASH_ERR_UNSUPPORTED, "intermediate size must be a multiple of 512");
  if (int r = check_w4(gate_up, "gate_up", E, 2 * I, H)) return r;
  if (int r = check_w4(down, "down", E, H, I)) return r;
  const bool shared = sgu || sdn || sgate;
  if (shared) {
    if (!sgu || !sdn || !sgate)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "shared expert needs shared_gate_up, shared_down and shared_gate_weight");
    if (int r = check_w4(sgu, "shared_gate_up", 1, 2 * I, H)) return r;
    if (int r = check_w4(sdn, "shared_down", 1, H, I)) return r;
    if (sgu->group_size != gate_up->group_size || sdn->group_size != down->group_size ||
        sgu->scale_dtype != gate_up->scale_dtype || sdn->scale_dtype != down->scale_dtype ||
        sgu->layout != gate_up->layout || sdn->layout != gate_up->layout)
      return fail(DFLASH_ERR_UNSUPPORTED,
                  "shared expert must use the routed banks' group sizes, scale dtypes and layout");
    if (!aligned16(sgate)) return fail(DFLASH_ERR_INVALID_ARGUMENT, "shared_gate_weight not 16-byte aligned");
  }
  if (T > 0 && (!hidden || !out)) return fail(DFLASH_ERR_INVALID_ARGUMENT, "hidden and out are required");
  if (!aligned16(hidden) || !aligned16(out)) return fail(DFLASH_ERR_INVALID_ARGUMENT, "hidden/out not 16-byte aligned");
  const bool scales16 = aligned16(gate_up->scales) && aligned16(down->scales) &&
                        (!shared || (aligned16(sgu->scales) && aligned16(sdn->scales)));
  if (gate_up->layout != down->layout)
    return fail(DFLASH_ERR_UNSUPPORTED, "gate_up and down must share one layout");
  *S = MoeShapes{T, H, I, E, k, gate_up->group_size, down->group_size, shared,
                 gate_up->scale_dtype == DFLASH_DTYPE_F32, down->scale_dtype == DFLASH_DTYPE_F32, scales16,
                 gate_up->layout == DFLASH_LAYOUT_TILED};
  return DFLASH_OK;
}

// Stage of dflash_set_measure_stage (process-wide): when set, the MoE entry
// points launch only that stage's kernel.
std::atomic<int> g_measure{DFLASH_STAGE_NONE};

bool measuring() { return g_measure.load(std::memory_order_acquire) != DFLASH_STAGE_NONE; }
// Whether this call launches the kernel(s) of `stage` (GATE_UP, DOWN, or EXPERTS: the fused
// verify launch); measurement of EXPERTS launches every expert GEMM kernel of the call.
bool stage_on(int stage) {
  const int m = g_measure.load(std::memory_order_acquire);
  return m == DFLASH_STAGE_NONE || m == stage || m == DFLASH_STAGE_EXPERTS;
}

// One W4 GEMM over the work table: the LDS-tiled kernel for long prefill, else
// the workgroup-streaming kernel when it splits this K evenly, else the per-wave
// fallback (w4_gemm: K outside {512, 1024, 2048} or group 256).
enum class GemmPath { kTile, kStream };

// dflash_set_tile_pieces (process-wide): 0 lets the tile kernels split their last round by the
// grid, 1, 2 or 4 force that many pieces per remaining tile.
std::atomic<int> g_tile_pieces{0};

void launch_w4(int mode, bool fp32_scales, int mt, int max_slots, GemmPath path, dflash::W4StreamParams& p,
               hipStream_t stream) {
  using namespace dflash;
  if (path == GemmPath::kTile) {
    p.strips = mode == kModeGateUp ? p.N / 2 / 256 : p.N / 512;  // column tiles per pass
    p.tile_pieces = g_tile_pieces.load(std::memory_order_acquire);
    launch_w4_tile(mode, fp32_scales, cu_count(), p, stream);
    return;
  }
  const int cols = mode == kModeGateUp ? p.N / 2 / 16 : p.N / 32;  // 16-column pairs or 32-row strips
  const int rg = w4_stream_row_groups(p.K);
  if (w4_stream_supports(p.K, p.G) && cols % rg == 0) {
    p.strips = cols / rg;
    launch_w4_stream(mode, fp32_scales, mt, cu_count(), p, stream);
  } else {
    launch_w4_gemm(mode, fp32_scales, max_slots, p, stream);
  }
}

// Whether launch_w4 would run a kernel that reads the tiled layout (tile, or the
// streaming kernel when it splits this K); the per-wave fallback does not.
bool w4_path_reads_tiled(int mode, int N, int K, int G, GemmPath path) {
  using namespace dflash;
  if (path == GemmPath::kTile) return true;
  const int cols = mode == kModeGateUp ? N / 2 / 16 : N / 32;
  return w4_stream_supports(K, G) && cols % w4_stream_row_groups(K) == 0;
}

// Verify-block path (T <= 32): both expert GEMMs on w4_verify, the gate/up
// launch routing in its prologue when `route` is asked for and fits, the down
// launch running the combine.  False when the shapes need the other kernels.
bool verify_fits(const MoeShapes& S, bool route, dflash::VerifyParams* gu, dflash::VerifyParams* dn) {
  using namespace dflash;
  const auto group_ok = [](int64_t g) { return g == 128 || g == 256; };
  if (!group_ok(S.G) || !group_ok(S.Gd)) return false;
  // long prefill (at least 16 rows per expert on average) belongs to the MFMA tile kernel
  if (S.T > kVerifyMaxTokens && moe_tile_path(S)) return false;
  const int T = static_cast<int>(S.T), H = static_cast<int>(S.H), I = static_cast<int>(S.I);
  const int E = static_cast<int>(S.E), k = static_cast<int>(S.k), sh = S.shared ? 1 : 0;
  // the kernels split units (passes x strips) over the grid in 32-bit arithmetic
  const int64_t units = verify_pass_cap(S.T, S.E, S.k, S.shared) * std::max(S.I / 16, S.H / 32);
  if (units * cu_count() >= (int64_t{1} << 32)) return false;
  *gu = VerifyParams{};
  *dn = VerifyParams{};
  return verify_layout(kModeGateUp, T, H, 2 * I, E, k, sh, route ? 1 : 0, gu) &&
         verify_layout(kModeDown, T, I, H, E, k, sh, 0, dn);
}

// Routing outputs the gate/up launch writes when it routes in its prologue.
struct RouteOut {
  bool logits_given;  // the caller's logits (valid in measurement mode too)
  const float* logits;
  int32_t* ids;
  float* wts;
  int32_t* perm;
  int32_t* inv;
  int32_t* offsets;
};

// Split-K down (SplitDown in the gate/up launch): a verify block routed in the gate/up
// prologue (one 32-lane row per token), banks of one scale type, H in {512, 1024, 2048}, a
// workspace with the partial rows for this grid, and unit ranges of at most two passes.
// Appends the LDS of the down phase to gu's layout.
std::atomic<int> g_split_down{0};  // dflash_set_split_down (process-wide, opt-in)

bool fused_down_fits(const MoeShapes& S, dflash::VerifyParams* gu, const MoeLayout& L, int grid) {
  using namespace dflash;
  if (!g_split_down.load(std::memory_order_acquire)) return false;
  if (gu->route != 2 || S.gu_f32 != S.dn_f32 || L.parts_grid < grid) return false;
  if (S.H != 512 && S.H != 1024 && S.H != 2048) return false;
  const int64_t strips = S.I / 16, cap = verify_pass_cap(S.T, S.E, S.k, S.shared);
  if ((cap * strips + grid - 1) / grid > strips + 1) return false;  // a range of <= strips + 1 units spans <= 2 passes
  return fused_down_layout(gu, static_cast<int>(S.I));
}

// fuse_down: run the down GEMM inside the gate/up launch (fused_down_fits was true); not in
// measurement of GATE_UP or DOWN alone, which times the two verify launches instead.
int run_verify(const MoeShapes& S, dflash::VerifyParams gu, dflash::VerifyParams dn, bool fuse_down,
               const RouteOut& ro, const int32_t* inv, const float* wts, void* ws, const MoeLayout& L,
               const dflash_w4* gate_up, const dflash_w4* down, const dflash_w4* sgu, const dflash_w4* sdn, void* out,
               hipStream_t stream) {
  using namespace dflash;
  const int T = static_cast<int>(S.T), H = static_cast<int>(S.H), I = static_cast<int>(S.I);
  W4StreamParams p{};
  p.pass_table = at<int4>(ws, L.route.pass_table);
  p.tok = at<int32_t>(ws, L.route.tok);
  p.meta = at<int32_t>(ws, L.route.meta);
  p.top_k = static_cast<int>(S.k);
  p.T = T;
  p.has_shared = S.shared ? 1 : 0;
  p.rows_per_pass = 16;
  p.tiled = S.tiled ? 1 : 0;

  // gate_up: N = 2I rows over K = H, SiLU*up epilogue into h
  p.w = static_cast<const uint8_t*>(gate_up->packed);
  p.s = gate_up->scales;
  p.w_shared = S.shared ? static_cast<const uint8_t*>(sgu->packed) : nullptr;
  p.s_shared = S.shared ? sgu->scales : nullptr;
  p.w_stride = S.I * S.H;
  p.s_stride = 2 * S.I * (S.H / S.G);
  p.N = 2 * I;
  p.K = H;
  p.G = static_cast<int>(S.G);
  p.act = at<uint16_t>(ws, L.x_il);
  p.act_neg = at<float>(ws, L.xneg);
  p.neg_parts = 1;
  p.out_bf16 = at<uint16_t>(ws, L.h);
  p.out_part = at<float>(ws, L.hpart);
  p.strips = I / 16;
  gu.g = p;
  gu.E = static_cast<int>(S.E);
  // measurement mode routes again only from the caller's logits (valid without the front
  // launch); otherwise it times the GEMM on the work table an earlier full call left
  if (measuring() && !ro.logits_given) gu.route = 0;
  if (gu.route) {
    gu.logits = ro.logits;
    gu.ids = ro.ids;
    gu.wts = ro.wts;
    gu.perm = ro.perm;
    gu.inv = ro.inv;
    gu.offsets = ro.offsets;
    gu.meta_out = at<int32_t>(ws, L.route.meta);
    gu.pass_table_out = at<int4>(ws, L.route.pass_table);
    gu.slot_w_out = at<float>(ws, L.route.slot_w);
    gu.tok_out = at<int32_t>(ws, L.route.tok);
  }
  const int stage = g_measure.load(std::memory_order_acquire);
  const bool fused = fuse_down && gu.route && (stage == DFLASH_STAGE_NONE || stage == DFLASH_STAGE_EXPERTS);
  // the routing gate/up launch also plans the down launch's prologue (same workspace, next
  // launch) when there is one
  const int grid = cu_count();
  if (gu.route && !fused && grid <= kDownPlanMaxGrid) {
    gu.down_plan = at<int4>(ws, L.down_plan);
    gu.down_grid = grid;
    gu.down_strips = H / 32;
  }
  if (fused) {
    gu.fuse_down = 1;
    gu.dw = static_cast<const uint8_t*>(down->packed);
    gu.ds = down->scales;
    gu.dw_shared = S.shared ? static_cast<const uint8_t*>(sdn->packed) : nullptr;
    gu.ds_shared = S.shared ? sdn->scales : nullptr;
    gu.dw_stride = S.H * S.I / 2;
    gu.ds_stride = S.H * (S.I / S.Gd);
    gu.dH = H;
    gu.dI = I;
    gu.dG = static_cast<int>(S.Gd);
    gu.ypart = at<float>(ws, L.ypart);
    gu.row_seg = at<int2>(ws, L.row_seg);
    gu.part_rps = static_cast<int>(part_rps(S.T));
  } else {
    gu.fuse_down = 0;
  }
  if (stage_on(DFLASH_STAGE_GATE_UP)) launch_w4_verify(kModeGateUp, S.gu_f32, grid, gu, stream);
  if (int r = launch_status("gate_up")) return r;

  if (!fused) {
    // down: N = H rows over K = I, unweighted fp32 y (the combine applies the routing weights)
    p.w = static_cast<const uint8_t*>(down->packed);
    p.s = down->scales;
    p.w_shared = S.shared ? static_cast<const uint8_t*>(sdn->packed) : nullptr;
    p.s_shared = S.shared ? sdn->scales : nullptr;
    p.w_stride = S.H * S.I / 2;
    p.s_stride = S.H * (S.I / S.Gd);
    p.G = static_cast<int>(S.Gd);
    p.N = H;
    p.K = I;
    p.act = at<uint16_t>(ws, L.h);
    p.act_neg = at<float>(ws, L.hpart);
    p.neg_parts = 8;
    p.out_bf16 = nullptr;
    p.out_part = nullptr;
    p.out_f32 = at<float>(ws, L.y);
    p.slot_w = at<float>(ws, L.route.slot_w);
    p.shared_gate = at<float>(ws, L.gate);
    p.strips = H / 32;
    dn.g = p;
    dn.E = static_cast<int>(S.E);
    // a plan exists only when this call's gate/up launch wrote one (measurement mode timing the
    // down launch alone keeps the work table's pass count)
    dn.down_plan = gu.down_plan && stage_on(DFLASH_STAGE_GATE_UP) ? gu.down_plan : nullptr;
    if (stage_on(DFLASH_STAGE_DOWN)) launch_w4_verify(kModeDown, S.dn_f32, grid, dn, stream);
    if (int r = launch_status("down")) return r;
  }

  if (measuring()) return DFLASH_OK;
  if (fused) {
    launch_combine_parts(at<float>(ws, L.ypart), at<int2>(ws, L.row_seg), gu.part_rps, inv, T, p.top_k, H,
                         p.has_shared, wts, at<float>(ws, L.gate), static_cast<uint16_t*>(out), stream);
    return launch_status("combine");
  }
  // the verify down launch leaves y unweighted: the combine applies the routing weights
  launch_combine(at<float>(ws, L.y), inv, T, p.top_k, H, p.has_shared, wts, at<float>(ws, L.gate),
                 static_cast<uint16_t*>(out), stream);
  return launch_status("combine");
}

// gate_up -> down -> combine for a routing and work table already in place.
// Every kernel input besides x and the weight banks comes from the workspace
// (routing kernels or table_prep wrote it); inv (the caller's) feeds combine.
GemmPath moe_gemm_path(const MoeShapes& S) {
  return moe_tile_path(S) ? GemmPath::kTile : GemmPath::kStream;
}

// Tiled banks need every expert kernel of the call to read that layout; checked
// before anything is launched.
int check_tiled_moe(const MoeShapes& S, bool verify) {
  using namespace dflash;
  if (!S.tiled || verify) return DFLASH_OK;
  const GemmPath path = moe_gemm_path(S);
  const int H = static_cast<int>(S.H), I = static_cast<int>(S.I);
  if (!w4_path_reads_tiled(kModeGateUp, 2 * I, H, static_cast<int>(S.G), path) ||
      !w4_path_reads_tiled(kModeDown, H, I, static_cast<int>(S.Gd), path))
    return tiled_unsupported("moe");
  return DFLASH_OK;
}

int run_experts(const MoeShapes& S, const int32_t* inv, void* ws, const MoeLayout& L, const dflash_w4* gate_up,
                const dflash_w4* down, const dflash_w4* sgu, const dflash_w4* sdn, void* out, hipStream_t stream) {
  using namespace dflash;
  const int T = static_cast<int>(S.T), H = static_cast<int>(S.H), I = static_cast<int>(S.I);
  const int k = static_cast<int>(S.k);
  const GemmPath path = moe_gemm_path(S);
  const int mt = path == GemmPath::kStream ? token_tiles(S.T) : 1;
  const int32_t* meta = at<int32_t>(ws, L.route.meta);
  const int4* slot_table = at<int4>(ws, L.route.slot_table);
  const int32_t* pass_slot = at<int32_t>(ws, L.route.pass_slot);
  W4StreamParams p{};
  p.pass_table = at<int4>(ws, L.route.pass_table);
  p.tok = at<int32_t>(ws, L.route.tok);
  p.meta = meta;
  p.slot_table = slot_table;
  p.pass_slot = pass_slot;
  p.top_k = k;
  p.T = T;
  p.has_shared = S.shared ? 1 : 0;
  p.rows_per_pass = rows_per_pass(S);
  p.tiled = S.tiled ? 1 : 0;
  const int max_slots = static_cast<int>(std::min<int64_t>(S.E, S.T * S.k)) + p.has_shared;

  // gate_up: N = 2I rows over K = H, SiLU*up epilogue into h
  p.w = static_cast<const uint8_t*>(gate_up->packed);
  p.s = gate_up->scales;
  p.w_shared = S.shared ? static_cast<const uint8_t*>(sgu->packed) : nullptr;
  p.s_shared = S.shared ? sgu->scales : nullptr;
  p.w_stride = S.I * S.H;
  p.s_stride = 2 * S.I * (S.H / gate_up->group_size);
  p.N = 2 * I;
  p.K = H;
  p.G = static_cast<int>(gate_up->group_size);
  p.act = at<uint16_t>(ws, L.x_il);
  p.act_neg = at<float>(ws, L.xneg);
  p.neg_parts = 1;
  p.out_bf16 = at<uint16_t>(ws, L.h);
  p.out_part = at<float>(ws, L.hpart);
  if (stage_on(DFLASH_STAGE_GATE_UP)) launch_w4(kModeGateUp, S.gu_f32, mt, max_slots, path, p, stream);
  if (int r = launch_status("gate_up")) return r;

  // down: N = H rows over K = I, routing-weight epilogue into y
  p.w = static_cast<const uint8_t*>(down->packed);
  p.s = down->scales;
  p.w_shared = S.shared ? static_cast<const uint8_t*>(sdn->packed) : nullptr;
  p.s_shared = S.shared ? sdn->scales : nullptr;
  p.w_stride = S.H * S.I / 2;
  p.s_stride = S.H * (S.I / down->group_size);
  p.N = H;
  p.K = I;
  p.G = static_cast<int>(down->group_size);
  p.act = at<uint16_t>(ws, L.h);
  p.act_neg = at<float>(ws, L.hpart);
  p.neg_parts = path == GemmPath::kTile ? 1 : 8;  // the tile kernel's gate_up sums h per 128 columns
  p.out_bf16 = nullptr;
  p.out_part = nullptr;
  p.out_f32 = at<float>(ws, L.y);
  p.slot_w = at<float>(ws, L.route.slot_w);
  p.shared_gate = at<float>(ws, L.gate);
  if (stage_on(DFLASH_STAGE_DOWN)) launch_w4(kModeDown, S.dn_f32, mt, max_slots, path, p, stream);
  if (int r = launch_status("down")) return r;

  if (measuring()) return DFLASH_OK;
  if (path == GemmPath::kTile)
    launch_combine_bf16(at<uint16_t>(ws, L.y), inv, T, k, H, p.has_shared, static_cast<uint16_t*>(out), stream);
  else
    launch_combine(at<float>(ws, L.y), inv, T, k, H, p.has_shared, nullptr, nullptr, static_cast<uint16_t*>(out),
                   stream);
  return launch_status("combine");
}

dflash::RouteParams route_params(const float* logits, int64_t T, int64_t E, int64_t k, int32_t* ids, float* wts,
                                 int32_t* perm, int32_t* inv, int32_t* offsets, void* ws, const RouteLayout& L,
                                 int rows_per_pass, bool shared, bool sort_passes = false) {
  dflash::RouteParams r{};
  r.logits = logits;
  r.T = static_cast<int>(T);
  r.E = static_cast<int>(E);
  r.k = static_cast<int>(k);
  r.ids = ids;
  r.wts = wts;
  r.perm = perm;
  r.inv = inv;
  r.offsets = offsets;
  r.hit = at<int32_t>(ws, L.hit);
  r.pass_start = at<int32_t>(ws, L.pass_start);
  r.meta = at<int32_t>(ws, L.meta);
  r.counts = at<int32_t>(ws, L.counts);
  r.slotmap = at<uint8_t>(ws, L.slotmap);
  r.slot_table = at<int4>(ws, L.slot_table);
  r.pass_slot = at<int32_t>(ws, L.pass_slot);
  r.pass_table = at<int4>(ws, L.pass_table);
  r.slot_w = at<float>(ws, L.slot_w);
  r.tok = at<int32_t>(ws, L.tok);
  r.rows_per_pass = rows_per_pass;
  r.has_shared = shared ? 1 : 0;
  r.sort_passes = sort_passes ? 1 : 0;
  return r;
}

}  // namespace

extern "C" {

int dflash_abi_version(void) { return DFLASH_ABI_VERSION; }

int dflash_w4_to_tiled(const dflash_w4* src, void* packed_out, void* scales_out, void* stream) {
  try {
    if (!src) return fail(DFLASH_ERR_INVALID_ARGUMENT, "to_tiled: descriptor is NULL");
    if (src->experts <= 0 || src->rows <= 0 || src->cols <= 0)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "to_tiled: experts, rows and cols must be positive");
    if (int r = check_w4(src, "to_tiled", src->experts, src->rows, src->cols)) return r;
    if (src->layout != DFLASH_LAYOUT_PORTABLE) return fail(DFLASH_ERR_INVALID_ARGUMENT, "to_tiled: source must be PORTABLE");
    if (src->rows % 16 || src->cols % 128)
      return fail(DFLASH_ERR_UNSUPPORTED, "to_tiled: needs rows % 16 == 0 and cols % 128 == 0");
    if (src->rows > (1 << 30) || src->cols > (1 << 30))
      return fail(DFLASH_ERR_UNSUPPORTED, "to_tiled: rows and cols must stay below 2^30");
    if (!packed_out || !scales_out || !aligned16(packed_out))
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "to_tiled: outputs NULL or packed_out not 16-byte aligned");
    const size_t sal = src->scale_dtype == DFLASH_DTYPE_F32 ? 4u : 2u;
    if (reinterpret_cast<uintptr_t>(scales_out) % sal)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "to_tiled: scales_out misaligned");
    if (packed_out == src->packed || scales_out == src->scales)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "to_tiled: outputs must not alias the source");
    dflash::launch_tile_w4(src->packed, src->scales, src->scale_dtype == DFLASH_DTYPE_F32, src->experts,
                           static_cast<int>(src->rows), static_cast<int>(src->cols),
                           static_cast<int>(src->group_size), packed_out, scales_out,
                           static_cast<hipStream_t>(stream));
    return launch_status("to_tiled");
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}

int dflash_w4_from_int8(const int8_t* values, const void* scales, int32_t scales_dtype, int64_t experts,
                        int64_t rows, int64_t cols, int64_t group_size, int32_t layout, void* packed_out,
                        float* scales_out, int32_t* invalid, void* stream) {
  try {
    if (experts <= 0 || rows <= 0 || cols <= 0)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "from_int8: experts, rows and cols must be positive");
    if (group_size != 128 && group_size != 256)
      return fail(DFLASH_ERR_UNSUPPORTED, "from_int8: group_size must be 128 or 256");
    if (cols % 32 || cols % group_size)
      return fail(DFLASH_ERR_UNSUPPORTED, "from_int8: cols must be a multiple of 32 and of group_size");
    if (layout != DFLASH_LAYOUT_PORTABLE && layout != DFLASH_LAYOUT_TILED)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "from_int8: unknown layout");
    if (layout == DFLASH_LAYOUT_TILED && (rows % 16 || cols % 128))
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "from_int8: the tiled layout needs rows % 16 == 0 and cols % 128 == 0");
    if (scales_dtype != DFLASH_DTYPE_BF16 && scales_dtype != DFLASH_DTYPE_F32 && scales_dtype != DFLASH_DTYPE_F16)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "from_int8: unknown scales_dtype");
    if (!values || !scales || !packed_out || !scales_out || !invalid)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "from_int8: NULL pointer");
    if (!aligned16(values) || !aligned16(packed_out) || reinterpret_cast<uintptr_t>(scales) % 4 ||
        reinterpret_cast<uintptr_t>(scales_out) % 4 || reinterpret_cast<uintptr_t>(invalid) % 4)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "from_int8: values/packed_out need 16-byte, scales/invalid 4-byte alignment");
    if (rows > (1 << 30) || cols > (1 << 30) || experts * rows * cols > (int64_t(1) << 40))
      return fail(DFLASH_ERR_UNSUPPORTED, "from_int8: bank too large");
    dflash::launch_from_int8(values, scales, scales_dtype, experts, static_cast<int>(rows), static_cast<int>(cols),
                             static_cast<int>(group_size), layout == DFLASH_LAYOUT_TILED, packed_out, scales_out,
                             invalid, static_cast<hipStream_t>(stream));
    return launch_status("from_int8");
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}

const char* dflash_last_error(void) { return g_last_error.c_str(); }

size_t dflash_qlinear_workspace_bytes(int64_t m, int64_t k, int64_t group_size) {
  if (m < 0 || k <= 0 || group_size <= 0) return 0;
  Carver c;
  c.take(2 * static_cast<size_t>(m) * k);
  c.take(4 * static_cast<size_t>(m) * (k / 128));
  return c.off;
}

namespace {
// Both qlinear entry points: y is bf16 [m][N], or fp32 when y_f32.
// 16-row blocks (w4_small.hip): the one-round-trip kernel up to N = 8192, its streaming form
// (x kept in registers, persistent workgroups) up to N = 32768, the staging verify kernel
// above (measured per projection: N = 8192 6.5 against 7.6 us streaming; N = 9216 7.5 against
// 8.4 one-round-trip; N = 65536 16.1 against 19.1 streaming; LM head 59.7 against 69.1).
constexpr int64_t kSmallLinearMaxN = 8192;
constexpr int64_t kSmallStreamMinN = 8193, kSmallStreamMaxN = 32768;

int qlinear_impl(const void* x, int64_t m, const dflash_w4* weight, void* y, bool y_f32, void* workspace,
                 size_t workspace_bytes, void* stream) {
  try {
    if (!weight) return fail(DFLASH_ERR_INVALID_ARGUMENT, "weight descriptor is NULL");
    if (m < 0) return fail(DFLASH_ERR_INVALID_ARGUMENT, "m must be >= 0");
    if (m > (1 << 24)) return fail(DFLASH_ERR_UNSUPPORTED, "m above 2^24 is not supported");
    const int64_t N = weight->rows, K = weight->cols;
    if (int r = check_w4(weight, "weight", 1, N, K)) return r;
    if (N <= 0 || N % 32) return fail(DFLASH_ERR_UNSUPPORTED, "qlinear needs N % 32 == 0");
    if (K <= 0 || K % 512) return fail(DFLASH_ERR_UNSUPPORTED, "qlinear needs K % 512 == 0");
    if (m == 0) return DFLASH_OK;
    if (!x || !y || !aligned16(x) || !aligned16(y)) return fail(DFLASH_ERR_INVALID_ARGUMENT, "x/y NULL or not 16-byte aligned");
    const size_t need = dflash_qlinear_workspace_bytes(m, K, weight->group_size);
    if (!workspace || workspace_bytes < need || !aligned16(workspace))
      return fail(DFLASH_ERR_WORKSPACE, "qlinear workspace needs " + std::to_string(need) + " bytes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool tiled = weight->layout == DFLASH_LAYOUT_TILED;
    // narrow projections of a short block: the one-round-trip kernel (operands straight into
    // MFMA fragments, one workgroup per 16 columns); wider ones stage x once per workgroup
    const bool stream_form =
        N >= kSmallStreamMinN && N <= kSmallStreamMaxN && dflash::small_linear_stream_fits(static_cast<int>(m), static_cast<int>(N),
                                                                   static_cast<int>(K),
                                                                   static_cast<int>(weight->group_size));
    if (stream_form || (N <= kSmallLinearMaxN &&
                        dflash::small_linear_fits(static_cast<int>(m), static_cast<int>(N), static_cast<int>(K),
                                                  static_cast<int>(weight->group_size)))) {
      dflash::SmallLinearParams sp{};
      sp.x = static_cast<const uint16_t*>(x);
      sp.w = static_cast<const uint8_t*>(weight->packed);
      sp.s = weight->scales;
      sp.y = y;
      sp.M = static_cast<int>(m);
      sp.N = static_cast<int>(N);
      sp.K = static_cast<int>(K);
      sp.G = static_cast<int>(weight->group_size);
      sp.tiled = tiled ? 1 : 0;
      sp.scale_f32 = weight->scale_dtype == DFLASH_DTYPE_F32 ? 1 : 0;
      sp.y_f32 = y_f32 ? 1 : 0;
      if (stream_form) dflash::launch_w4_small_stream(sp, cu_count(), st);
      else dflash::launch_w4_small(sp, st);
      return launch_status("qlinear");
    }
    // GEMM kernel: verify (m <= 32), else the streaming kernel (or its per-wave fallback)
    dflash::VerifyParams vl{};
    // the verify kernel stages at most 16 rows of K = 4096; 17..32 rows run as two launches of it
    const int64_t vrows = K == 4096 && m > 16 && m <= 32 ? 16 : m;
    const bool verify = (weight->group_size == 128 || weight->group_size == 256) &&
                        dflash::verify_layout(dflash::kModeLinear, static_cast<int>(vrows), static_cast<int>(K),
                                              static_cast<int>(N), 1, 1, 0, 0, &vl);
    if (tiled && !verify &&
        !w4_path_reads_tiled(dflash::kModeLinear, static_cast<int>(N), static_cast<int>(K),
                             static_cast<int>(weight->group_size), GemmPath::kStream))
      return tiled_unsupported("qlinear");
    Carver c;
    uint16_t* x_il = at<uint16_t>(workspace, c.take(2 * static_cast<size_t>(m) * K));
    float* xneg = at<float>(workspace, c.take(4 * static_cast<size_t>(m) * (K / 128)));
    if (!verify) {  // the verify kernel converts the raw rows itself
      dflash::FrontParams f{};
      f.x = static_cast<const uint16_t*>(x);
      f.T = static_cast<int>(m);
      f.prep_rows = static_cast<int>(m);
      f.H = static_cast<int>(K);
      f.x_il = x_il;
      f.xneg = xneg;
      dflash::launch_front(f, st);
      if (int r = launch_status("prep")) return r;
    }
    dflash::W4StreamParams p{};
    p.w = static_cast<const uint8_t*>(weight->packed);
    p.s = weight->scales;
    p.tiled = weight->layout == DFLASH_LAYOUT_TILED ? 1 : 0;
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.G = static_cast<int>(weight->group_size);
    p.act = x_il;
    p.act_neg = xneg;
    p.neg_parts = 1;
    p.out_bf16 = y_f32 ? nullptr : static_cast<uint16_t*>(y);
    p.out_f32 = y_f32 ? static_cast<float*>(y) : nullptr;
    p.M = static_cast<int>(m);
    if (verify) {
      p.act_neg = nullptr;
      p.rows_per_pass = 16;
      p.strips = p.N / 32;
      for (int64_t r0 = 0; r0 < m; r0 += vrows) {
        p.act = static_cast<const uint16_t*>(x) + r0 * K;
        if (y_f32) p.out_f32 = static_cast<float*>(y) + r0 * N;
        else p.out_bf16 = static_cast<uint16_t*>(y) + r0 * N;
        p.M = static_cast<int>(std::min(vrows, m - r0));
        vl.g = p;
        dflash::launch_w4_verify(dflash::kModeLinear, weight->scale_dtype == DFLASH_DTYPE_F32, cu_count(), vl, st);
        if (int r = launch_status("qlinear")) return r;
      }
      return DFLASH_OK;
    }
    const int mt = token_tiles(m);
    p.rows_per_pass = 16 * mt;
    launch_w4(dflash::kModeLinear, weight->scale_dtype == DFLASH_DTYPE_F32, mt, 1, GemmPath::kStream,
              p, st);
    return launch_status("qlinear");
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}
}  // namespace

int dflash_qlinear_w4a16(const void* x, int64_t m, const dflash_w4* weight, void* y, void* workspace,
                         size_t workspace_bytes, void* stream) {
  return qlinear_impl(x, m, weight, y, false, workspace, workspace_bytes, stream);
}

int dflash_qlinear_w4a16_f32(const void* x, int64_t m, const dflash_w4* weight, float* y, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return qlinear_impl(x, m, weight, y, true, workspace, workspace_bytes, stream);
}

int dflash_router_logits(const void* hidden, int64_t tokens, int64_t hidden_size, const void* router_weight,
                         int64_t experts, float* logits, void* stream) {
  try {
    if (tokens < 0 || experts <= 0 || experts > dflash::kMaxExperts)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "router needs tokens >= 0 and experts in [1, 1024]");
    if (hidden_size <= 0 || hidden_size % 256) return fail(DFLASH_ERR_UNSUPPORTED, "router needs hidden_size % 256 == 0");
    if (tokens == 0) return DFLASH_OK;
    if (!hidden || !router_weight || !logits || !aligned16(hidden) || !aligned16(router_weight))
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "router: NULL or misaligned pointer");
    dflash::FrontParams f{};
    f.x = static_cast<const uint16_t*>(hidden);
    f.router_w = static_cast<const uint16_t*>(router_weight);
    f.logits = logits;
    f.T = static_cast<int>(tokens);
    f.E = static_cast<int>(experts);
    f.H = static_cast<int>(hidden_size);
    f.router_big = dflash::router_big_fits(f.T, f.H) ? 1 : 0;
    f.n_router = dflash::router_tiles(f.T, f.E, f.H);
    dflash::launch_front(f, static_cast<hipStream_t>(stream));
    return launch_status("router");
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}

size_t dflash_moe_route_workspace_bytes(int64_t tokens, int64_t experts, int64_t top_k) {
  if (tokens < 0 || experts <= 0 || top_k <= 0) return 0;
  return route_layout(tokens, top_k, experts).total;
}

int dflash_moe_route(const float* logits, int64_t tokens, int64_t experts, int64_t top_k, int32_t* topk_ids,
                     float* topk_weights, int32_t* perm, int32_t* inv_perm, int32_t* expert_offsets, void* workspace,
                     size_t workspace_bytes, void* stream) {
  try {
    if (int r = check_route_args(tokens, experts, top_k)) return r;
    if (!expert_offsets) return fail(DFLASH_ERR_INVALID_ARGUMENT, "expert_offsets is required");
    if (tokens > 0 && (!logits || !topk_ids || !topk_weights || !perm || !inv_perm))
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "route: NULL pointer");
    const RouteLayout L = route_layout(tokens, top_k, experts);
    if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
      return fail(DFLASH_ERR_WORKSPACE, "route workspace needs " + std::to_string(L.total) + " bytes");
    const dflash::RouteParams r = route_params(logits, tokens, experts, top_k, topk_ids, topk_weights, perm, inv_perm,
                                               expert_offsets, workspace, L, 16 * token_tiles(tokens), false);
    dflash::launch_route(r, false, static_cast<hipStream_t>(stream));
    return launch_status("route");
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}

size_t dflash_moe_workspace_bytes(int64_t tokens, int64_t hidden_size, int64_t inter_size, int64_t experts,
                                  int64_t top_k, int64_t group_size, int has_shared) {
  if (tokens < 0 || hidden_size <= 0 || inter_size <= 0 || experts <= 0 || top_k <= 0 || group_size <= 0) return 0;
  return moe_layout(tokens, hidden_size, inter_size, experts, top_k, has_shared != 0,
                    tokens <= kVerifyMaxTokens ? cu_count() : 0).total;
}

int dflash_moe_experts_w4a16(const void* hidden, int64_t tokens, int64_t hidden_size, int64_t top_k,
                             const float* topk_weights, const int32_t* perm, const int32_t* inv_perm,
                             const int32_t* expert_offsets, const dflash_w4* gate_up, const dflash_w4* down,
                             const dflash_w4* shared_gate_up, const dflash_w4* shared_down,
                             const void* shared_gate_weight, void* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  try {
    MoeShapes S;
    if (int r = check_moe(hidden, tokens, hidden_size, top_k, gate_up, down, shared_gate_up, shared_down,
                          shared_gate_weight, out, &S))
      return r;
    if (tokens == 0) return DFLASH_OK;
    if (!topk_weights || !perm || !inv_perm || !expert_offsets)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "experts: routing arrays are required");
    const MoeLayout L = moe_layout(S.T, S.H, S.I, S.E, S.k, S.shared);
    if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
      return fail(DFLASH_ERR_WORKSPACE, "moe workspace needs " + std::to_string(L.total) + " bytes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    dflash::TableParams t{};
    t.offsets = expert_offsets;
    t.E = static_cast<int>(S.E);
    t.T = static_cast<int>(S.T);
    t.hit = at<int32_t>(workspace, L.route.hit);
    t.pass_start = at<int32_t>(workspace, L.route.pass_start);
    t.meta = at<int32_t>(workspace, L.route.meta);
    t.slot_table = at<int4>(workspace, L.route.slot_table);
    t.pass_slot = at<int32_t>(workspace, L.route.pass_slot);
    t.pass_table = at<int4>(workspace, L.route.pass_table);
    t.perm = perm;
    t.wts = topk_weights;
    t.slot_w = at<float>(workspace, L.route.slot_w);
    t.tok = at<int32_t>(workspace, L.route.tok);
    t.k = static_cast<int>(S.k);
    t.rows_per_pass = rows_per_pass(S);
    t.has_shared = S.shared ? 1 : 0;
    t.x = static_cast<const uint16_t*>(hidden);
    t.H = static_cast<int>(S.H);
    t.x_il = at<uint16_t>(workspace, L.x_il);
    t.xneg = at<float>(workspace, L.xneg);
    t.gate_w = S.shared ? static_cast<const uint16_t*>(shared_gate_weight) : nullptr;
    t.gate_out = at<float>(workspace, L.gate);
    dflash::VerifyParams vgu{}, vdn{};
    const bool verify = verify_fits(S, false, &vgu, &vdn);
    if (int r = check_tiled_moe(S, verify)) return r;
    if (!measuring()) dflash::launch_table_prep(t, st);
    if (int r = launch_status("table_prep")) return r;
    if (verify)
      return run_verify(S, vgu, vdn, false, RouteOut{}, inv_perm, topk_weights, workspace, L, gate_up, down,
                        shared_gate_up, shared_down, out, st);
    return run_experts(S, inv_perm, workspace, L, gate_up, down, shared_gate_up, shared_down, out, st);
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}

// The whole layer on a caller workspace, or (static_scratch) on this device's copy of
// `scratch`, whose address is looked up only after every argument has been validated.
static int moe_w4a16_body(const void* hidden, int64_t tokens, int64_t hidden_size, const float* router_logits,
                          const void* router_weight, int64_t top_k, const dflash_w4* gate_up, const dflash_w4* down,
                          const dflash_w4* shared_gate_up, const dflash_w4* shared_down,
                          const void* shared_gate_weight, void* out, float* logits_out, int32_t* topk_ids,
                          float* topk_weights, int32_t* perm, int32_t* inv_perm, int32_t* expert_offsets,
                          void* workspace, size_t workspace_bytes, bool static_scratch, void* stream) {
  try {
    MoeShapes S;
    if (int r = check_moe(hidden, tokens, hidden_size, top_k, gate_up, down, shared_gate_up, shared_down,
                          shared_gate_weight, out, &S))
      return r;
    if (!router_logits && !router_weight)
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "either router_logits or router_weight is required");
    if (!router_logits && !aligned16(router_weight))
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "router_weight not 16-byte aligned");
    if (!expert_offsets) return fail(DFLASH_ERR_INVALID_ARGUMENT, "expert_offsets is required");
    if (tokens > 0 && (!topk_ids || !topk_weights || !perm || !inv_perm))
      return fail(DFLASH_ERR_INVALID_ARGUMENT, "routing output arrays are required");
    // a caller workspace also holds the split-K down's partial rows (sized for this device's grid)
    const MoeLayout L = moe_layout(S.T, S.H, S.I, S.E, S.k, S.shared,
                                   !static_scratch && S.T <= kVerifyMaxTokens ? cu_count() : 0);
    if (static_scratch) {
      if (L.total > kScratchBytes)
        return fail(DFLASH_ERR_UNSUPPORTED, "moe_noalloc: this layer needs " + std::to_string(L.total) +
                                                " bytes of scratch, above the static " +
                                                std::to_string(kScratchBytes) + "; use dflash_moe_w4a16");
      if (int r = scratch_on_current_device(&workspace)) return r;
      workspace_bytes = kScratchBytes;
    }
    if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
      return fail(DFLASH_ERR_WORKSPACE, "moe workspace needs " + std::to_string(L.total) + " bytes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int T = static_cast<int>(S.T), E = static_cast<int>(S.E);
    const bool small = dflash::route_small_fits(T, E, static_cast<int>(S.k));
    // the verify path routes inside its gate/up launch when the block fits there
    dflash::VerifyParams vgu{}, vdn{};
    const bool verify = tokens > 0 && verify_fits(S, small, &vgu, &vdn);
    if (int r = check_tiled_moe(S, verify)) return r;
    const bool fused = verify && fused_down_fits(S, &vgu, L, cu_count());
    float* logits = router_logits ? const_cast<float*>(router_logits)
                                  : (logits_out ? logits_out : at<float>(workspace, L.logits));
    dflash::FrontParams f{};
    f.x = static_cast<const uint16_t*>(hidden);
    f.router_w = static_cast<const uint16_t*>(router_weight);
    f.logits = logits;
    f.T = T;
    f.E = E;
    f.H = static_cast<int>(S.H);
    f.router_big = dflash::router_big_fits(T, f.H) ? 1 : 0;
    f.n_router = router_logits ? 0 : dflash::router_tiles(T, E, f.H);
    // with multi-workgroup routing the activation prep runs in the route_topk launch instead
    const bool route_launch = !(verify && vgu.route);
    const bool prep_in_route = route_launch && !small && T > 0;
    f.prep_rows = prep_in_route ? 0 : T;
    f.x_il = at<uint16_t>(workspace, L.x_il);
    f.xneg = at<float>(workspace, L.xneg);
    f.gate_w = S.shared ? static_cast<const uint16_t*>(shared_gate_weight) : nullptr;
    f.gate_out = at<float>(workspace, L.gate);
    if (!small) {
      f.zero = at<uint32_t>(workspace, L.route.counts);
      f.zero_words = dflash::route_zero_words(T, E);
      f.n_zero = static_cast<int>(std::min<int64_t>(256, (f.zero_words + 2047) / 2048));
    }
    if (!measuring()) dflash::launch_front(f, st);
    if (int r = launch_status("front")) return r;
    if (route_launch) {
      // the prefill tile kernels take the routed passes longest first
      dflash::RouteParams r = route_params(logits, S.T, S.E, S.k, topk_ids, topk_weights, perm, inv_perm,
                                                 expert_offsets, workspace, L.route, rows_per_pass(S), S.shared,
                                                 !verify && moe_gemm_path(S) == GemmPath::kTile);
      if (prep_in_route) {
        r.prep_x = f.x;
        r.prep_H = f.H;
        r.prep_rows = T;
        r.prep_x_il = f.x_il;
        r.prep_xneg = f.xneg;
        r.prep_gate_w = f.gate_w;
        r.prep_gate_out = f.gate_out;
      }
      if (!measuring()) dflash::launch_route(r, true, st);
      if (int rc = launch_status("route")) return rc;
    }
    if (tokens == 0) return DFLASH_OK;
    if (verify)
      return run_verify(S, vgu, vdn, fused,
                        RouteOut{router_logits != nullptr, logits, topk_ids, topk_weights, perm, inv_perm, expert_offsets},
                        inv_perm, topk_weights, workspace, L, gate_up, down, shared_gate_up, shared_down, out, st);
    return run_experts(S, inv_perm, workspace, L, gate_up, down, shared_gate_up, shared_down, out, st);
  } catch (...) {
    return fail(DFLASH_ERR_HIP, "unexpected host exception");
  }
}

int dflash_moe_w4a16(const void* hidden, int64_t tokens, int64_t hidden_size, const float* router_logits,
                     const void* router_weight, int64_t top_k, const dflash_w4* gate_up, const dflash_w4* down,
                     const dflash_w4* shared_gate_up, const dflash_w4* shared_down, const void* shared_gate_weight,
                     void* out, float* logits_out, int32_t* topk_ids, float* topk_weights, int32_t* perm,
                     int32_t* inv_perm, int32_t* expert_offsets, void* workspace, size_t workspace_bytes,
                     void* stream) {
  return moe_w4a16_body(hidden, tokens, hidden_size, router_logits, router_weight, top_k, gate_up, down,
                        shared_gate_up, shared_down, shared_gate_weight, out, logits_out, topk_ids, topk_weights,
                        perm, inv_perm, expert_offsets, workspace, workspace_bytes, false, stream);
}

int dflash_moe_w4a16_noalloc(const void* hidden, int64_t tokens, int64_t hidden_size, const float* router_logits,
                             const void* router_weight, int64_t top_k, const dflash_w4* gate_up,
                             const dflash_w4* down, const dflash_w4* shared_gate_up, const dflash_w4* shared_down,
                             const void* shared_gate_weight, void* out, float* logits_out, int32_t* topk_ids,
                             float* topk_weights, int32_t* perm, int32_t* inv_perm, int32_t* expert_offsets,
                             void* stream) {
  return moe_w4a16_body(hidden, tokens, hidden_size, router_logits, router_weight, top_k, gate_up, down,
                        shared_gate_up, shared_down, shared_gate_weight, out, logits_out, topk_ids, topk_weights,
                        perm, inv_perm, expert_offsets, nullptr, 0, true, stream);
}

int dflash_set_tile_pieces(int pieces) {
  if (pieces != 0 && pieces != 1 && pieces != 2 && pieces != 4)
    return fail(DFLASH_ERR_INVALID_ARGUMENT, "pieces must be 0, 1, 2 or 4");
  g_tile_pieces.store(pieces, std::memory_order_release);
  return DFLASH_OK;
}

int dflash_set_split_down(int enable) {
  if (enable != 0 && enable != 1) return fail(DFLASH_ERR_INVALID_ARGUMENT, "enable must be 0 or 1");
  g_split_down.store(enable, std::memory_order_release);
  return DFLASH_OK;
}

int dflash_moe_split_down(int64_t tokens, int64_t hidden_size, int64_t inter_size, int64_t experts, int64_t top_k,
                          int64_t group_size, int has_shared, int32_t scale_dtype, int32_t layout) {
  try {
    if (tokens <= 0 || check_route_args(tokens, experts, top_k) != DFLASH_OK) return 0;
    if (hidden_size <= 0 || hidden_size % 512 || inter_size <= 0 || inter_size % 512) return 0;
    if (group_size != 128 && group_size != 256) return 0;
    const bool f32 = scale_dtype == DFLASH_DTYPE_F32;
    const MoeShapes S{tokens, hidden_size, inter_size, experts, top_k, group_size, group_size, has_shared != 0,
                      f32, f32, true, layout == DFLASH_LAYOUT_TILED};
    const bool small = dflash::route_small_fits(static_cast<int>(tokens), static_cast<int>(experts),
                                                static_cast<int>(top_k));
    dflash::VerifyParams vgu{}, vdn{};
    if (!verify_fits(S, small, &vgu, &vdn)) return 0;
    const MoeLayout L = moe_layout(S.T, S.H, S.I, S.E, S.k, S.shared, S.T <= kVerifyMaxTokens ? cu_count() : 0);
    return fused_down_fits(S, &vgu, L, cu_count()) ? 1 : 0;
  } catch (...) {
    return 0;
  }
}

#ifdef DFLASH_TIMELINE
// Profiling build only (timeline.py; not in the product ABI): which 0 = verify launches
// (2 x 1024 x 16 ticks), 1 = tile launches (2 x 1024 x 8 x 3), 2 = the tile launches' per-wave
// cycles (2 x 1024 x 8 x 8 x 6).
int dflash_timeline_read(int which, void* host, size_t bytes) {
  return which == 0 ? dflash::timeline_verify_read(host, bytes)
       : which == 1 ? dflash::timeline_tile_read(host, bytes)
                    : dflash::timeline_tile_cycles_read(host, bytes);
}
int dflash_timeline_clear(void) { return dflash::timeline_verify_clear() | dflash::timeline_tile_clear(); }
#endif

int dflash_set_measure_stage(int stage) {
  if (stage != DFLASH_STAGE_NONE && stage != DFLASH_STAGE_GATE_UP && stage != DFLASH_STAGE_DOWN &&
      stage != DFLASH_STAGE_EXPERTS)
    return fail(DFLASH_ERR_INVALID_ARGUMENT, "unknown stage");
  g_measure.store(stage, std::memory_order_release);
  return DFLASH_OK;
}

}  // extern "C"
