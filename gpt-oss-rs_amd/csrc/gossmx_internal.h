// Internal declarations shared by the gfx950 kernels (gossmx_kernels.hip) and
// the C ABI host code (gossmx_api.hip). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace gossmx {

constexpr int kBlock = 32;      // values per MXFP4 / Q8 block (QUANT_BLOCK_SIZE)
constexpr int kRecord = 17;     // E8M0 byte + 16 packed nibble bytes per (row, block)
constexpr int kTileRows = 16;   // rows per MFMA tile (one wave)
constexpr int kWgRows = 64;     // gate_up rows (32 gate/up pairs) per 32-value block of the down input
constexpr int kChunk = 16;      // activation rows per GEMM work item (batches of more than kSmallChunk rows)
constexpr int kSmallChunk = 8;  // activation rows per work item for batches of at most 8 rows
constexpr int kHugeChunk = 32;  // activation rows per work item for batches of at least kHugeMinRows rows
constexpr int kHugeMinRows = 512;
constexpr int kChunkMax = 32;
// Small-batch GEMV (gemv_kernel): batches of at most kTinyMaxRows rows whose
// blocks per row are at most kTinyMaxBlocks (the activation image of the
// whole K range fits the work-group's LDS).
constexpr int kTinyMaxRows = 4;
constexpr int kTinyMaxBlocks = 96;
constexpr int kMaxExperts = 128;
constexpr int kMaxTopK = 8;
constexpr int kNormMaxHidden = 8192;  // hidden sizes the fused post-attention RMSNorm stages in LDS

// Device error flags (sticky until the host reads them).
constexpr int kErrNonFiniteLogits = 1;
constexpr int kErrNonFiniteInput = 2;
constexpr int kErrWorkOrder = 4;  // a kernel found the work list in an order it relies on not holding

// Resident layout v3 of one [experts][rows][blocks] MXFP4 tensor.
//  tiles = ceil(rows / 16). Per expert and tile t:
//   nibble plane: 16 * blocks * 16 bytes at t * 256 * blocks. Block group
//     q (blocks 4q .. 4q+nb-1, nb = min(4, blocks - 4q)) starts at q * 1024;
//     lane L = 16 * g + n (g = K slice 0..3, n = row in tile) owns nb * 4
//     bytes at L * nb * 4, one dword per block: packed bytes 4g..4g+3 of the
//     canonical record, i.e. codes 8g..8g+7 (low nibble = even code).
//   scale plane: 64 * ceil(blocks / 4) bytes at t * 64 * ceil(blocks / 4);
//     group q at q * 64, byte (n, j) at n * 4 + j (a partial last group is
//     padded to 4 bytes per row so every group is one aligned dword per row).
//  Padding rows (rows..16*tiles-1) hold zero codes and scale 127.
struct TiledWeights {
  uint8_t* nib = nullptr;
  uint8_t* scl = nullptr;
  size_t experts = 0, rows = 0, blocks = 0, tiles = 0;
  size_t nib_stride = 0;  // bytes per expert in the nibble plane
  size_t scl_stride = 0;  // bytes per expert in the scale plane
  // [experts][tiles]: 1 when every scale byte of the tile is in the exact
  // scaled-conversion range (see tile_flags_kernel); set after every write.
  uint8_t* fast = nullptr;
};

// Extra bytes allocated after each plane: the GEMM reads whole 4-block groups
// (and dword-granular tails) of the last tile unconditionally.
constexpr size_t kPlaneSlack = 2048;
// Extra bytes after each activation operand buffer: the GEMM's staging reads
// a last partial K step as a whole step (up to 15 blocks of 128 bytes past a
// row).
constexpr size_t kActSlack = 2048;

// Activation operand of the expert GEMM, one row per token or route:
//  actv [row][block][part 0 = primary, 1 = residual][32] f16 (the Q8 codes,
//  exact in f16), acts [row][block][2] f32 (primary scale, residual scale).
struct ActBuffers {
  _Float16* v = nullptr;
  float* s = nullptr;
};

enum GemmMode { kPlain = 0, kGateUp = 1, kDown = 2 };

// CpuExpertProjection (cpu_runner.rs:49-90): how expert inputs are prepared.
enum Projection { kProjResidualQ8 = 0, kProjQ8 = 1, kProjExactBf16 = 2 };

struct GemmArgs {
  TiledWeights w;
  int fast_ok;           // 0: never take the scaled-conversion fast path (self-test found it unsafe)
  const _Float16* actv;
  const float* acts;
  const float* bias;     // bias of expert e at bias + e * bias_expert_stride, or null
  size_t bias_expert_stride;
  int residual;          // 1 = residual-Q8 activations, 0 = Q8 (primary only)
  // work items
  int plain_expert, plain_m;          // kPlain
  const int* work;                    // [n][4] (expert, first grouped route, rows, 0)   (gate_up/down)
  const int* n_work;
  const int* route_tok;               // grouped route -> source row
  const int* route_slot;              // grouped route -> row * top_k + rank
  // outputs
  float* out; size_t out_stride;      // kPlain
  _Float16* actv_next; float* acts_next;  // kGateUp: down-projection input per grouped route
  float alpha, limit;                 // kGateUp
  const uint16_t* sig_tab;            // kGateUp: SwiGLU sigmoid per bf16 input (65,536 entries)
  uint16_t* y;                        // kDown: [m * top_k][rows] bf16
  float* trace_gu;                    // kGateUp, nullable: [m * top_k][rows] bf16-rounded gate_up by (row, rank) slot
  float* trace_sw;                    // kGateUp, nullable: [m * top_k][rows / 2] SwiGLU values by slot
  // Exact-BF16 projection: input rows (gate_up: [m][K] by source row, down:
  // [routes][K] by grouped route) and gate_up's bf16 SwiGLU output by grouped route.
  const uint16_t* xin;
  uint16_t* act_next16;
  int* err;
};

struct RouteArgs {
  const uint16_t* x;        // [m][hidden] bf16
  const uint16_t* router_w; // [experts][hidden]
  const float* router_b;    // [experts]
  const float* injected;    // [m][experts] or null
  const float* norm_w;      // [hidden] post-attention RMSNorm weight (route_kernel), or null
  float norm_eps;
  int m, hidden, experts, top_k;
  float* logits;            // [m][experts]
  int* selected;            // [m][top_k]
  float* weights;           // [m][top_k]
  ActBuffers act;           // gate_up input per token
  // How the quantization work-groups store each input block (Projection):
  // residual-Q8, Q8 (residual codes and scale zero), or the bf16 values
  // themselves (exact-BF16 after the fused RMSNorm: act.v holds [m][hidden]
  // bf16). quant = 0 launches no quantization work-groups.
  int qmode;
  int quant;
  int* err;
};

struct DispatchArgs {
  const int* selected;  // [m * top_k]
  int routes, top_k, experts;
  int* bucket_off;      // [experts + 1]
  int* route_tok;       // [routes]
  int* route_slot;      // [routes]
  int* work;            // [max_work][4] (expert, first grouped route, rows, 0): one record per item
  int* n_work;
  int chunk;            // rows per work item: kSmallChunk, kChunk or kHugeChunk (by batch size)
};

// Batches whose logits fit one work-group's LDS take the fused selection +
// dispatch kernel (one launch; no global round trip between the two).
constexpr int kSelectLds = 8448;        // m * (experts + 1) floats
constexpr int kSelectMaxRoutes = 2048;  // m * top_k
constexpr int kSelectTopK = 4;          // top_k (GPT-OSS routes to 4 experts)

// Computed router logits of small batches take one launch for the router,
// the selection and the dispatch (route_select_kernel).
constexpr int kFusedRouteRows = 4;
constexpr int kFusedRouteHidden = 4096;
// One-row batches select inside the gate_up launch up to this many experts.
constexpr int kRouteGemvExperts = kMaxExperts;

// Launchers (gossmx_kernels.hip). All are asynchronous on `stream`.
// Router logits (bf16-rounded, into a.logits) and the gate_up input
// quantization; followed by one of the two selection paths below.
hipError_t launch_route(const RouteArgs& a, hipStream_t stream);
// Batches past the fused kernel's limits: selection with per-work-group
// expert counts (cnt: ceil(m / select_rows_per_wg) x experts ints), then the
// grouping. quantize = 1 adds the gate_up input quantization (no route_kernel).
int select_rows_per_wg(int experts, int top_k);
hipError_t launch_select_count(const RouteArgs& r, int quantize, int* cnt, hipStream_t stream);
hipError_t launch_place(const DispatchArgs& a, int m, const int* cnt, hipStream_t stream);
// Work-group 0: top-k, softmax and dispatch of all rows from r.injected (bf16
// rounded here) or from the logits r.logits computed by launch_route with
// select = 0. quantize = 1 adds the gate_up input quantization work-groups
// (when no launch_route ran).
hipError_t launch_select_dispatch(const RouteArgs& r, const DispatchArgs& d, int quantize, hipStream_t stream);
// Router logits, top-k, softmax, dispatch and (r.quant) the gate_up input
// quantization of m <= kFusedRouteRows rows in one launch. `counter`: a
// device int that is 0 before the launch; the launch leaves it 0.
hipError_t launch_route_select(const RouteArgs& r, const DispatchArgs& d, int* counter, hipStream_t stream);
// chunk: rows per work item (kSmallChunk, kChunk or kHugeChunk), selecting
// the kernel's geometry; it must match the chunk the dispatch used.
// start/stop (nullable): events the launch itself records around the kernel.
hipError_t launch_gemm(GemmMode mode, const GemmArgs& a, int chunk, int grid_work, hipStream_t stream,
                       hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
hipError_t launch_tile_flags(TiledWeights w, hipStream_t stream);
// Small-batch GEMV over the work list (kGateUp, kDown) or a plain problem
// (kPlain): same arguments and outputs as launch_gemm with chunk kSmallChunk,
// for residual-Q8 activations; requires every work item (and, for kPlain, m)
// to hold at most rows_max <= kTinyMaxRows rows and blocks <= kTinyMaxBlocks.
hipError_t launch_gemv(GemmMode mode, const GemmArgs& a, int rows_max, int grid_work, hipStream_t stream,
                       hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Router logits of m <= kFusedRouteRows rows only (route_select_kernel
// without its arrival counter), and the gate_up input quantization when
// r.quant.
hipError_t launch_route_logits(const RouteArgs& r, hipStream_t stream);
// Selection, dispatch and gate_up GEMV of a one-row batch in one launch,
// after launch_route_logits with r.quant (computed router, experts <=
// kRouteGemvExperts, top_k <= 4, residual-Q8, hidden <= kTinyMaxBlocks * 32,
// no gate_up / SwiGLU traces): the outputs of launch_route_select followed by
// launch_gemv(kGateUp).
hipError_t launch_route_gemv(const RouteArgs& r, const DispatchArgs& d, const GemmArgs& g, hipStream_t stream,
                             hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Down projection + weighted combine of a one-row batch (residual-Q8, every
// work item one route, top_k <= 4, blocks <= kTinyMaxBlocks): the outputs of
// launch_gemv(kDown) followed by launch_combine with m = 1, without the y
// buffer (d.y is not written).
// out16 (nullable): the output as bf16 bits, beside or instead of out.
hipError_t launch_down_combine(const GemmArgs& d, const float* weights, int top_k, float* out, uint16_t* out16,
                               float* trace_down, const uint16_t* resid, uint16_t* next, float* unrounded,
                               hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Exact-BF16 expert projection over the work list (mode kGateUp or kDown);
// chunk <= kChunkMax.
hipError_t launch_exact(GemmMode mode, const GemmArgs& a, int grid_work, hipStream_t stream);

hipError_t launch_combine(const uint16_t* y, const float* weights, int m, int top_k, int hidden, float* out,
                          uint16_t* out16, float* trace_down, const uint16_t* resid, uint16_t* next,
                          float* unrounded, hipStream_t stream);
hipError_t launch_prep_records(const uint8_t* records, int kind, size_t m, size_t blocks, size_t row_stride,
                               ActBuffers act, int* err, hipStream_t stream);
hipError_t launch_repack(const uint8_t* src, int layout, TiledWeights w, hipStream_t stream);
hipError_t launch_generate(uint64_t seed, uint64_t stream_id, TiledWeights w, hipStream_t stream);
hipError_t launch_export(TiledWeights w, uint8_t* dst, hipStream_t stream);
hipError_t launch_fill_tiled_padding(TiledWeights w, hipStream_t stream);
hipError_t launch_clear_ints(int* p, size_t n, hipStream_t stream);

// Gathers a host-memory call's outputs into one device buffer for a single
// device-to-host copy: dst[0] = the device error flags word, then each piece's
// bytes (a multiple of 4) at its offset (a multiple of 16).
constexpr int kPackPieces = 10;
struct PackArgs {
  const int* err;
  char* dst;
  const void* src[kPackPieces];
  uint64_t off[kPackPieces];    // bytes into dst
  uint64_t words[kPackPieces];  // 4-byte words
  int pieces;
};
hipError_t launch_pack(const PackArgs& a, hipStream_t stream);
hipError_t launch_build_sigmoid_table(uint16_t* tab, hipStream_t stream);
// Self-test outputs (floats): kSelftestCodes conversion results, 256 MFMA
// results, kSelftestCodes scaled results, then kSelftestDirty x 16 results of
// the scaled conversion with the E8M0 byte in a dirty scale dword (see
// selftest_kernel).
constexpr int kSelftestCodes = 8;
constexpr int kSelftestDirty = 5 * 4 * 6;  // exponents x byte positions x neighbour patterns
// bf16 conversion cases: fixed edges (ties, NaN payloads, denormals, the
// overflow boundary) and hashed bit patterns; input k is selftest_bf16_input(k).
constexpr int kSelftestBf16 = 1024;
constexpr int kSelftestBf16Base = kSelftestCodes + 256 + kSelftestCodes + 16 * kSelftestDirty;
constexpr int kSelftestFloats = kSelftestBf16Base + kSelftestBf16;
constexpr uint32_t kBf16Edges[] = {0x00000000u, 0x80000000u, 0x3f808000u, 0x3f818000u, 0x3f808001u, 0x3f80ffffu,
                                   0x7f7f8000u, 0x7f7fffffu, 0x7f800000u, 0xff800000u, 0x7f800001u, 0x7fc00000u,
                                   0xffc00001u, 0x7fa00000u, 0xff80ffffu, 0x00008000u, 0x00018000u, 0x807fffffu,
                                   0x00400000u, 0xbf7f8000u};
constexpr int kBf16EdgeCount = (int)(sizeof(kBf16Edges) / sizeof(kBf16Edges[0]));
__host__ __device__ constexpr uint32_t selftest_bf16_input(int k) {
  return k < kBf16EdgeCount ? kBf16Edges[k] : (uint32_t)k * 0x9E3779B1u + 0x7F4A7C15u;
}
hipError_t launch_selftest(float* out, hipStream_t stream);
// Every f32 bit pattern through bf16_bits against half's rounding restated
// in software; mismatches are counted into *count (device, zeroed by the caller).
hipError_t launch_bf16_exhaustive(unsigned long long* count, hipStream_t stream);
// The model's dense bf16 projections (16-lane dot order), up to three of the
// same input in one launch: out_p[r * rows_p + o] = dot(w_p[o], x[r])
// (+ bias_p[o]) for r < m, o < rows_p; w bf16 [rows][cols], x f32 [m][cols],
// bias f32 [rows] or null. wg_begin is filled by the launchers.
struct DenseSet {
  const uint16_t* w[3];
  const float* bias[3];
  float* out[3];
  int rows[3];
  int wg_begin[4];
};
hipError_t launch_dense_proj(const DenseSet& set, int count, const float* x, int cols, int m, hipStream_t stream);
// One token through up to three projections with the whole K range of a
// work-group staged at once (cols a multiple of 8, at most 4096).
hipError_t launch_dense_gemv(const DenseSet& set, int count, const float* x, int cols, hipStream_t stream);
// after[i] = bf16(hidden[i] + bf16(proj[i])) for i < n (bf16 bits).
hipError_t launch_residual_add(const uint16_t* hidden, const float* proj, uint16_t* after, size_t n,
                               hipStream_t stream);

}  // namespace gossmx

// Hooks of the C ABI host code (gossmx_api.hip) for the host-side store
// module (gossmx_store.cpp): the last-error message, and the resident layout
// v3 image (nibble plane and scale plane, experts x stride bytes each); and
// for the dense path (gossmx_dense.cpp): a MoE layer's configuration.
struct gossmx_ctx;
struct gossmx_weights;
struct gossmx_layer;
struct gossmx_moe_config;
namespace gossmx {
int set_error(int status, const char* message);
const gossmx_moe_config* layer_config(const gossmx_layer* layer);
int context_device(const gossmx_ctx* ctx);
hipStream_t context_stream(const gossmx_ctx* ctx);
// A GPU round trip's status: GOSSMX_ERR_DEVICE or GOSSMX_ERR_OUT_OF_MEMORY
// drains the context's stream and opens the process-wide circuit breaker.
int run_time_result(gossmx_ctx* ctx, int status);
// Process-wide accounting of host<->device copies (gossmx_stats).
enum TransferDirection { kTransferUpload = 0, kTransferActivation = 1, kTransferOutput = 2 };
void count_transfer(int direction, size_t bytes);
// gossmx_weights_open_or_create's repack cache: a valid repack was found.
void count_repack_cache(bool hit);
void tiled_image_bytes(size_t experts, size_t rows, size_t blocks, size_t* nib_bytes, size_t* scl_bytes);
int tiled_image_read(gossmx_ctx* ctx, const gossmx_weights* w, uint8_t* nib, uint8_t* scl);
int tiled_image_create(gossmx_ctx* ctx, size_t experts, size_t rows, size_t blocks, const uint8_t* nib,
                       const uint8_t* scl, gossmx_weights** out);
}  // namespace gossmx
