/*
 * gossmx: MI355X (gfx950) MXFP4 mixture-of-experts block for GPT-OSS.
 *
 * C ABI of libgossmx.so. Plain pointers and sizes only. Every entry point
 * returns a gossmx_status; the message of the last failure on the calling
 * thread is available from gossmx_last_error().
 *
 * Reference interfaces replaced (paths relative to gpt-oss-rs v0.1.0):
 *   - gossmx_mxfp4_matmul       <- Kernels::mxfp4_matmul(backend, Mxfp4MatmulProblem, scratch)
 *                                  crates/gpt-oss-cpu-kernels/src/matmul.rs:398-414, problem
 *                                  constructors and validation matmul.rs:297-369
 *   - gossmx_moe_forward        <- CpuModel::moe_batch(layer, idx, inputs, capture, ...)
 *                                  crates/gpt-oss-model-runner/src/cpu_runner.rs:2794-3013
 *   - gossmx_moe_forward_residual <- the MoE half of forward_layer_batch: norm_boundary of the
 *                                  post-attention residual, moe_batch, add_residual
 *                                  (cpu_runner.rs:2519-2553, 2680-2687, 3732-3738)
 *   - gossmx_weights_open_or_create, _load_repack, _save_repack, gossmx_repack_*
 *                               <- CpuRepackCache / RepackedMxfp4, cpu_repack.rs:21-480 (container,
 *                                  cache key, lock, atomic publish) with a resident layout 3
 *   - gossmx_safetensors_find, gossmx_weights_from_safetensors
 *                               <- CpuTensorStore::open / tensor, cpu_tensor_store.rs:46-288
 *   - gossmx_weights_upload     <- CpuRepackCache::open_or_create + RepackedMxfp4::expert_view
 *                                  crates/gpt-oss-model-runner/src/cpu_repack.rs:149-216,302-318
 *                                  (the resident copy is a new GPU layout, see below)
 *   - gossmx_layer_create       <- load_layer (router/gate_up/down tensors and biases)
 *                                  crates/gpt-oss-model-runner/src/cpu_runner.rs:3526-3671
 *   - gossmx_status codes       <- KernelError variants, crates/gpt-oss-cpu-kernels/src/lib.rs:138-157,
 *                                  and the non-finite router ModelError, cpu_runner.rs:2829-2834
 *   - gossmx_profile_*          <- CpuExecutionProfiler records, cpu_profile.rs:30-51
 *   - gossmx_inject_fault       <- CpuExecutionFailurePoint test hook, cpu_runner.rs:478-483
 *   - gossmx_model_*            <- the dense CPU step around the block: CpuModel::load,
 *                                  new_sequence_state, prefill_layer_major, prepare_step/commit,
 *                                  decode (cpu_runner.rs:1115-1306, 1596-1627, 1827-1885,
 *                                  2080-2586, 1081-1113), with each MoE half on the GPU
 *   - gossmx_attention, gossmx_yarn_rope, gossmx_greedy_token
 *                               <- attention_one_staged, YarnRope (cpu_runner.rs:3840-4013),
 *                                  greedy_token (gpt-oss-bench/src/bin/cpu_parity.rs:750-762)
 *
 * Weight layouts accepted on upload (Mxfp4WeightLayout, lib.rs:70-90):
 *   GOSSMX_LAYOUT_CANONICAL_V1 : per (row, block) 17 bytes = E8M0 scale byte, then
 *                                16 bytes with code(2j) | code(2j+1) << 4.
 *   GOSSMX_LAYOUT_X8_SPLIT_V2  : complete 8-row groups of 136-byte records, rows % 8
 *                                tail canonical (lib.rs:810-851, cpu_repack.rs:437-480).
 * Resident layout (GOSSMX_LAYOUT_GPU_TILED_V3, device only): 16-row tiles; a nibble
 * plane where each 64-lane wave loads one contiguous 1 KiB segment per 4 K-blocks,
 * and a separate E8M0 scale plane. Same 17 bytes per (row, block).
 *
 * Threading: a context owns one HIP stream and is used by one thread at a time
 * (like CpuExecutionContext, cpu_runner.rs:868-876). Calls are asynchronous on that
 * stream unless they return host data; gossmx_synchronize() waits.
 *
 * Lifetimes: weights and layers do not refer to their context after creation
 * (their destroy waits for the whole device), so they may outlive it. Graphs
 * and models do: destroy them before their context.
 */
#ifndef GOSSMX_H
#define GOSSMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gossmx_status {
  GOSSMX_OK = 0,
  GOSSMX_ERR_INVALID_ARGUMENT = 1,    /* null pointer or unknown enum value */
  GOSSMX_ERR_UNSUPPORTED = 2,         /* shape this build does not handle */
  GOSSMX_ERR_INVALID_DIMENSIONS = 3,  /* KernelError::InvalidDimensions */
  GOSSMX_ERR_NON_FINITE_INPUT = 4,    /* KernelError::NonFiniteInput */
  GOSSMX_ERR_UNAVAILABLE_BACKEND = 5, /* KernelError::UnavailableMatmulBackend (no gfx950 device) */
  GOSSMX_ERR_DEVICE = 6,              /* HIP runtime error, or a kernel's internal consistency check */
  GOSSMX_ERR_OUT_OF_MEMORY = 7,
  GOSSMX_ERR_NON_FINITE_LOGITS = 8,   /* "CPU router produced non-finite logits" */
  GOSSMX_ERR_INJECTED_FAULT = 9,      /* gossmx_inject_fault test hook fired */
  GOSSMX_ERR_BAD_FILE = 10,           /* missing, unreadable or malformed file (the store's ModelError / io::Error) */
  GOSSMX_ERR_CIRCUIT_OPEN = 11        /* XeError::CircuitOpen: an earlier run-time fault opened the breaker */
} gossmx_status;

enum {
  GOSSMX_LAYOUT_CANONICAL_V1 = 1,
  GOSSMX_LAYOUT_X8_SPLIT_V2 = 2,
  GOSSMX_LAYOUT_GPU_TILED_V3 = 3
};

enum { GOSSMX_ACT_Q8 = 1, GOSSMX_ACT_RESIDUAL_Q8 = 2 };

/* Where the caller's activation/bias/output pointers live. */
enum { GOSSMX_MEM_HOST = 0, GOSSMX_MEM_DEVICE = 1 };

typedef struct gossmx_ctx gossmx_ctx;
typedef struct gossmx_weights gossmx_weights;
typedef struct gossmx_layer gossmx_layer;

/* Last failure message of the calling thread ("" when none). */
const char* gossmx_last_error(void);
/* Library/ABI version: major * 10000 + minor * 100 + patch. */
int gossmx_version(void);
/* Number of visible gfx950 devices (0 on a host without one). */
int gossmx_device_count(int* count);

/* Context: one device, one in-order HIP stream. `stream` may be NULL (the
 * context creates its own) or a caller hipStream_t (not destroyed by us).
 * Creation runs the device self-test (gossmx_selftest) and fails with
 * GOSSMX_ERR_UNSUPPORTED if a lane layout or the sigmoid table is wrong; if
 * only the scaled FP4 conversion with dirty scale operands is, the context is
 * created with the GEMM's scaled-conversion fast path off (same bits, slower). */
int gossmx_ctx_create(int device, void* stream, gossmx_ctx** out);
/* 1 when the context's GEMMs may take the scaled-conversion fast path. */
int gossmx_ctx_fast_path(const gossmx_ctx* ctx, int* enabled);
void gossmx_ctx_destroy(gossmx_ctx* ctx);
/* Replaces the context's stream (after draining the old one). Every later
 * call, including a model's steps, runs on the new stream. */
int gossmx_ctx_set_stream(gossmx_ctx* ctx, void* stream);
void* gossmx_ctx_stream(gossmx_ctx* ctx);
/* Waits for the context's stream and reads the device error flags. A
 * run-time failure found here (GOSSMX_ERR_DEVICE, GOSSMX_ERR_OUT_OF_MEMORY:
 * what a device-memory call reports only when it is waited for) opens the
 * circuit breaker, as it does inside a call. */
int gossmx_synchronize(gossmx_ctx* ctx);

/* Device memory helpers (so non-PyTorch callers can stage device buffers). */
int gossmx_malloc(gossmx_ctx* ctx, size_t bytes, void** out);
int gossmx_free(gossmx_ctx* ctx, void* ptr);
int gossmx_memcpy_h2d(gossmx_ctx* ctx, void* dst, const void* src, size_t bytes);
int gossmx_memcpy_d2h(gossmx_ctx* ctx, void* dst, const void* src, size_t bytes);

/* Resident MXFP4 weights [experts][rows][blocks] (17 B per row-block).
 * `data` is host memory in `layout` (canonical v1 or x8 v2), `len` must be
 * experts * rows * blocks * 17 bytes, each expert laid out independently as
 * RepackedMxfp4::expert_view yields it. Repacked on the device to v3. */
int gossmx_weights_upload(gossmx_ctx* ctx, const uint8_t* data, size_t len, size_t experts, size_t rows,
                          size_t blocks, int layout, gossmx_weights** out);
/* Synthetic weights generated on the device: record i = (expert*rows+row)*blocks+block
 * takes two 64-bit counter hashes h0 = H(seed, stream, 2i), h1 = H(seed, stream, 2i+1)
 * (SplitMix64 based); scale byte = 119 + (h1 >> 61) % 5, packed bytes = h0 then h1
 * little-endian. Equal to the canonical tensor a host generator of the same rule makes. */
int gossmx_weights_generate(gossmx_ctx* ctx, uint64_t seed, uint64_t stream, size_t experts, size_t rows,
                            size_t blocks, gossmx_weights** out);
/* Copy the resident weights back to host memory in layout v1 (canonical). */
int gossmx_weights_export(gossmx_ctx* ctx, const gossmx_weights* w, uint8_t* out, size_t len);
int gossmx_weights_shape(const gossmx_weights* w, size_t* experts, size_t* rows, size_t* blocks);
size_t gossmx_weights_device_bytes(const gossmx_weights* w);
void gossmx_weights_destroy(gossmx_weights* w);

/* Resident weights on disk (CpuRepackCache, crates/gpt-oss-model-runner/src/cpu_repack.rs)
 * and from SafeTensors checkpoints (CpuTensorStore, cpu_tensor_store.rs). Host file I/O.
 *
 * GOSSMX4 repack container (cpu_repack.rs:21-23, 120-130, 231-280, 400-480): the 8 bytes
 * "GOSSMX4\0", the header length (u64 LE), the JSON RepackHeader {format_version,
 * layout_version, layout_identifier, tensor_name, model_revision, source_hashes, shape
 * [experts, rows, blocks], records}, then the payload. Layouts 1 (CanonicalAdjacentV1) and
 * 2 (InterleavedSplitX8V2) carry records x 17 bytes as the reference writes them; layout 3
 * (GpuTiledV3) carries this library's resident image: the nibble plane, then the scale
 * plane, experts x stride bytes each. */
typedef struct gossmx_repack_info {
  uint32_t format_version;
  uint32_t layout_version;
  size_t experts, rows, blocks, records;
  size_t payload_offset; /* bytes from the start of the file */
  size_t payload_bytes;
} gossmx_repack_info;

/* Reads and validates a container header as RepackedMxfp4::open does (magic, header
 * length, known layout identifier and version, records = experts * rows * blocks, file
 * length = payload offset + payload bytes). No device access. tensor_name (nullable)
 * receives the header's tensor name, cut to cap - 1 bytes and NUL-terminated. */
int gossmx_repack_inspect(const char* path, gossmx_repack_info* info, char* tensor_name, size_t cap);
/* Loads a container of any of the three layouts as resident weights (layouts 1 and 2
 * through gossmx_weights_upload; layout 3 by copying the image). */
int gossmx_weights_load_repack(gossmx_ctx* ctx, const char* path, gossmx_weights** out);
/* Writes resident weights as a layout-3 container: a temporary file in the target's
 * directory, synced, renamed over the target, then the directory synced (the atomic
 * publish of open_or_create, cpu_repack.rs:190-204). */
int gossmx_weights_save_repack(gossmx_ctx* ctx, const gossmx_weights* w, const char* path, const char* tensor_name,
                               const char* model_revision, const char* const* source_hashes, size_t n_hashes);
/* SourceIdentity::cache_key (cpu_repack.rs:92-107): SHA-256 of "gpt-oss-rs-mxfp4-repack",
 * the format version 1 (u32 LE), the layout name, the layout identifier (u32 LE), the
 * model revision, each source hash, the tensor name and each dimension (u64 LE), written
 * to key as 64 lowercase hex digits and a NUL. layout is 1, 2 or 3. */
int gossmx_repack_cache_key(const char* tensor_name, const size_t shape[3], int layout, const char* model_revision,
                            const char* const* source_hashes, size_t n_hashes, char key[65]);

/* One tensor of a SafeTensors shard, with parse_shard_header's checks
 * (cpu_tensor_store.rs:176-288): dtype as spelled in the file, shape, absolute byte range. */
typedef struct gossmx_tensor_info {
  char dtype[16];
  size_t rank;
  size_t shape[8];
  size_t offset;
  size_t bytes;
} gossmx_tensor_info;
int gossmx_safetensors_find(const char* path, const char* name, gossmx_tensor_info* info);
/* Resident weights from the U8 tensors blocks_name [experts][rows][blocks][16] and
 * scales_name [experts][rows][blocks], each in exactly one of the shards (the source
 * checks of open_or_create, cpu_repack.rs:155-174). */
int gossmx_weights_from_safetensors(gossmx_ctx* ctx, const char* const* shards, size_t n_shards,
                                    const char* blocks_name, const char* scales_name, gossmx_weights** out);
/* CpuRepackCache::open_or_create (cpu_repack.rs:149-216) with layout 3: the container
 * cache_root/mxfp4/<cache key of blocks_name>/weights.repack is loaded when its header
 * matches this source; otherwise the weights come from the shards and the container is
 * published under the lock file repack.lock ("pid=<pid>"; a lock whose process is gone
 * is taken over; waits at most 120 s). */
int gossmx_weights_open_or_create(gossmx_ctx* ctx, const char* cache_root, const char* model_revision,
                                  const char* const* source_hashes, size_t n_hashes, const char* const* shards,
                                  size_t n_shards, const char* blocks_name, const char* scales_name,
                                  gossmx_weights** out);

/* Kernel boundary: C[m, n] = A[m, K] . W[expert][n, K]^T + bias[n] for n < rows,
 * written at output[i * output_stride + n]; columns rows..output_stride-1 of each
 * output row are never written. Activations are the reference's records:
 * Q8Block {f32 scale; i8 values[32]} (36 B) or ResidualQ8Block {Q8Block primary;
 * Q8Block residual} (72 B), row i at activations + i * row_stride records
 * (ResidualQ8MatrixView, lib.rs). The float accumulation per output is the
 * reference's: total = bias; per block in order total += (p * 0.5 * e8m0) * ps
 * (then the residual term), bit-identical to scalar_matmul_range
 * (matmul.rs:529-578). Validation failures return before any output write. */
typedef struct gossmx_matmul_problem {
  const gossmx_weights* weights;
  size_t expert;
  int activation_kind;     /* GOSSMX_ACT_Q8 or GOSSMX_ACT_RESIDUAL_Q8 */
  const void* activations; /* records, see above */
  size_t activations_len;  /* in records */
  size_t m;                /* activation rows */
  size_t blocks_per_row;   /* must equal the weights' blocks */
  size_t row_stride;       /* in records, >= blocks_per_row */
  const float* bias;       /* nullable, bias_len == rows */
  size_t bias_len;
  float* output;
  size_t output_len;       /* in floats, >= (m - 1) * output_stride + rows */
  size_t output_stride;    /* >= rows */
  int memory;              /* GOSSMX_MEM_HOST or GOSSMX_MEM_DEVICE for activations/bias/output */
} gossmx_matmul_problem;

int gossmx_mxfp4_matmul(gossmx_ctx* ctx, const gossmx_matmul_problem* problem);
/* The validation gossmx_mxfp4_matmul runs first, against a weights shape, with
 * no device access (Mxfp4MatmulProblem::new, matmul.rs:339-369). */
int gossmx_mxfp4_matmul_check(const gossmx_matmul_problem* problem, size_t rows, size_t blocks, size_t experts);
/* Mxfp4MatmulBackend::scratch_requirement (matmul.rs:58-93): caller-owned scratch
 * the call needs. The GPU backend keeps its own operand buffers, so a valid
 * problem gets size 0 and alignment 1 (Mxfp4ScratchRequirement::NONE, :124-129);
 * an invalid one the validation's status. No device access. */
int gossmx_mxfp4_scratch_requirement(const gossmx_matmul_problem* problem, size_t* size, size_t* alignment);

/* Process-wide circuit breaker (the Xe engine's PROCESS_XE_CIRCUIT_OPEN,
 * crates/gpt-oss-xe/src/lib.rs:605-724). A projection call (gossmx_mxfp4_matmul,
 * gossmx_moe_forward, gossmx_moe_forward_residual) that fails at run time with
 * GOSSMX_ERR_DEVICE or GOSSMX_ERR_OUT_OF_MEMORY drains its stream and opens the
 * circuit; while it is open those calls validate their arguments and then return
 * GOSSMX_ERR_CIRCUIT_OPEN without touching the device. The caller recomputes the
 * failed call once on its CPU path (cpu_runner.rs:3365-3387) and keeps using the
 * CPU until it resets the breaker. Argument, data (non-finite) and injected
 * (mode 1) failures leave it closed. */
int gossmx_circuit_is_open(void);
void gossmx_circuit_reset(void);

/* Process-wide accounting, the counters the Xe engine exports as metrics
 * (crates/gpt-oss-xe/src/lib.rs:44-49: projection_total by result,
 * transfer_bytes_total by direction, circuit_breaker, the expert cache's
 * resident bytes; record_projection_metrics :785-825; XeResidencyStats
 * :358-370). Projection calls (gossmx_mxfp4_matmul, gossmx_moe_forward,
 * gossmx_moe_forward_residual, gossmx_moe_forward_noalloc) count by their
 * return: ok; failed (GOSSMX_ERR_DEVICE, GOSSMX_ERR_OUT_OF_MEMORY,
 * GOSSMX_ERR_INJECTED_FAULT: the caller's fallback reason "execution
 * failure"); refused (GOSSMX_ERR_CIRCUIT_OPEN: the caller's fallback reason
 * "fault"); rejected (every other status: argument, shape or non-finite data).
 * A device-memory call counts when it returns; a device-side error that a
 * later gossmx_synchronize reports does not change its count. Transfer bytes
 * are the bytes the library moves between host and device (copies, or kernel
 * writes into its pinned staging): weights, router and bias uploads
 * (weights_bias_uploaded); the inputs of host-memory calls and the dense
 * model's round trips (activations); their results (output). Resident
 * bytes are the device memory held by live gossmx_weights and gossmx_layer
 * objects (planes with their padding, router and biases); contexts' scratch is
 * not included. */
typedef struct gossmx_stats {
  uint64_t projections_ok;
  uint64_t projections_failed;
  uint64_t projections_refused;
  uint64_t projections_rejected;
  uint64_t weights_bias_uploaded_bytes;
  uint64_t activation_bytes;
  uint64_t output_bytes;
  uint64_t resident_bytes;
  uint64_t resident_high_water_bytes;
  uint64_t resident_cap_bytes;        /* 0: no cap */
  uint64_t capacity_refusals;         /* creations refused by the cap */
  uint64_t repack_cache_hits;         /* gossmx_weights_open_or_create found a valid repack */
  uint64_t repack_cache_misses;       /* ... repacked from the SafeTensors shards */
  int32_t circuit_open;
  int32_t reserved;
} gossmx_stats;
int gossmx_stats_read(gossmx_stats* out);
/* Zeroes the counters and sets the high-water mark to the bytes resident now;
 * the cap and the resident bytes are kept. */
void gossmx_stats_reset(void);
/* Cap on the resident bytes (AttachConfig::max_resident_bytes,
 * crates/gpt-oss-xe/src/lib.rs:239-250; 0 removes it). Weights and layer
 * creation that would pass it fails with GOSSMX_ERR_OUT_OF_MEMORY before
 * allocating anything and counts a capacity refusal; what is already resident
 * stays, also when the new cap is below it. */
int gossmx_set_resident_cap(uint64_t bytes);

/* MoE layer (GPT-OSS): router [experts][hidden] bf16 + f32 bias, gate_up
 * [experts][2*intermediate][hidden/32] with gate/up rows interleaved even/odd
 * and f32 bias [experts][2*intermediate], down [experts][hidden][intermediate/32]
 * and f32 bias [experts][hidden]. Host arrays are copied; weights are borrowed
 * (they must outlive the layer). */
/* CpuExpertProjection (cpu_runner.rs:49-90): how the expert projections
 * prepare their inputs. RESIDUAL_Q8 (the reference's default): quantize_residual_q8
 * and two integer dots per block; Q8: quantize_q8, one dot; EXACT_BF16: the bf16
 * inputs against bf16(decode * scale) weights in 16 ordered float lanes
 * (accumulate_mxfp4_bf16_block, lib.rs:932-945; a conformance path, VALU only). */
enum { GOSSMX_PROJECTION_RESIDUAL_Q8 = 0, GOSSMX_PROJECTION_Q8 = 1, GOSSMX_PROJECTION_EXACT_BF16 = 2 };

typedef struct gossmx_moe_config {
  size_t experts;      /* num_local_experts, <= 128 */
  size_t hidden;       /* hidden_size, multiple of 32 */
  size_t intermediate; /* intermediate_size, multiple of 32 */
  size_t top_k;        /* num_experts_per_tok, 1..8 and <= experts */
  float alpha;         /* 1.702 */
  float limit;         /* swiglu_limit, 7.0 */
  int projection;      /* GOSSMX_PROJECTION_*; 0 = residual-Q8 */
} gossmx_moe_config;

int gossmx_layer_create(gossmx_ctx* ctx, const gossmx_moe_config* config, const uint16_t* router_weight_bf16,
                        const float* router_bias, const gossmx_weights* gate_up, const float* gate_up_bias,
                        const gossmx_weights* down, const float* down_bias, gossmx_layer** out);
void gossmx_layer_destroy(gossmx_layer* layer);

/* One MoE block over m rows (CpuMoeStep per row, cpu_runner.rs:569-575).
 * Required: x [m][hidden] bf16 and output [m][hidden] f32 (bf16-rounded values).
 * Optional (nullable): injected_logits [m][experts] replaces the router
 * projection output before its bf16 round trip; router_logits [m][experts];
 * selected [m][top_k]; routing_weights [m][top_k]; route_order [m*top_k] receives
 * row * top_k + rank in the grouped (expert, row, rank) order; trace_down
 * [m][top_k][hidden] receives each rank's bf16-rounded down projection,
 * trace_gate_up [m][top_k][2 * intermediate] its bf16-rounded gate_up
 * projection and trace_swiglu [m][top_k][intermediate] its SwiGLU values
 * (CpuExpertTrace, cpu_runner.rs:2970-2984). output_unrounded [m][hidden] f32
 * receives the weighted sum of the ranks before its bf16 round trip
 * (fp32_to_bf16_roundtrip, cpu_runner.rs:2991), for callers that compare
 * pre-round values; no counterpart field in CpuMoeStep. All pointers are host
 * or device memory as `memory` says. Callers that zero-initialize the struct
 * leave the trailing fields null. */
typedef struct gossmx_moe_io {
  const uint16_t* x;
  size_t m;
  const float* injected_logits;
  float* router_logits;
  uint32_t* selected;
  float* routing_weights;
  float* output;
  uint32_t* route_order;
  float* trace_down;
  int memory;
  float* trace_gate_up;
  float* trace_swiglu;
  float* output_unrounded;
} gossmx_moe_io;

int gossmx_moe_forward(gossmx_ctx* ctx, const gossmx_layer* layer, const gossmx_moe_io* io);

/* gossmx_moe_forward without allocating (no counterpart in the reference; for
 * callers that cannot allocate device memory: code under HIP-graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same outputs, bit for
 * bit. All io pointers must be device memory (GOSSMX_MEM_DEVICE). The call's
 * scratch is carved from a fixed 64 MiB device array that each device holds
 * from the first context created on it until the process ends (about 84.5 KB
 * per row at the GPT-OSS-20B shape, so batches up to about 780 rows);
 * a larger call returns GOSSMX_ERR_UNSUPPORTED before launching anything. Every
 * call on one device shares that array and it keeps the last call's contents:
 * calls that overlap on one device (other streams or contexts) race. Nothing in
 * it needs to start at zero. No profiling events are recorded. */
int gossmx_moe_forward_noalloc(gossmx_ctx* ctx, const gossmx_layer* layer, const gossmx_moe_io* io);

/* The MoE half of a decoder layer on its residual stream (forward_layer_batch,
 * cpu_runner.rs:2519-2553): io->x is after_attention [m][hidden] bf16, the
 * block runs on norm_boundary(io->x, norm_weight) (the post-attention RMSNorm,
 * Kernels::rms_norm lib.rs:699-730 with epsilon = rms_norm_eps, rounded to bf16,
 * cpu_runner.rs:2680-2687), and next_residual [m][hidden] bf16 receives
 * add_residual(io->x, output) (cpu_runner.rs:3732-3738), the next layer's
 * input. norm_weight is the layer's post_attention_norm [hidden] f32. io->output
 * may be null here; the other io fields are as in gossmx_moe_forward (router
 * outputs and injected_logits refer to the normalized rows). norm_weight and
 * next_residual are host or device memory as io->memory says; in device memory
 * io->x and norm_weight must be 16-byte aligned. hidden <= 8192. */
int gossmx_moe_forward_residual(gossmx_ctx* ctx, const gossmx_layer* layer, const gossmx_moe_io* io,
                                const float* norm_weight, float epsilon, uint16_t* next_residual);

/* Profiling with hipEvents on the context stream, in the reference's operation
 * vocabulary (CpuProfileOperation, cpu_profile.rs:30-51). Top-k, softmax and
 * the grouping are recorded as GOSSMX_OP_DISPATCH on every path (one kernel
 * when m * (experts + 1) <= 8448, m * top_k <= 2048 and top_k <= 4, two
 * kernels otherwise). GOSSMX_OP_ROUTER_ROUTING holds the router projection
 * and the input quantization only, and has no launch when the logits are
 * injected; the quantization is then recorded under GOSSMX_OP_DISPATCH. */
enum {
  GOSSMX_OP_ROUTER_ROUTING = 0,     /* RouterProjection + Routing + ResidualQ8Preparation */
  GOSSMX_OP_DISPATCH = 1,           /* stable_group_routes + bucket gather */
  GOSSMX_OP_GATE_UP = 2,            /* GateUpProjection + SwiGlu + the down input quantization */
  GOSSMX_OP_DOWN = 3,               /* DownProjection */
  GOSSMX_OP_WEIGHTING = 4,          /* ExpertWeightingAccumulation */
  GOSSMX_OP_MATMUL = 5,             /* gossmx_mxfp4_matmul kernel */
  GOSSMX_OP_POST_ATTENTION_NORM = 6, /* PostAttentionNormalization: no launch of its own; the norm runs
                                       inside ROUTER_ROUTING (computed router) or DISPATCH (injected logits) */
  GOSSMX_OP_COUNT = 7
};
typedef struct gossmx_profile_record {
  int op;
  uint64_t launches;
  double total_ms;
} gossmx_profile_record;
int gossmx_profile_enable(gossmx_ctx* ctx, int enabled);
/* Synchronizes, folds pending events into totals, writes GOSSMX_OP_COUNT records. */
int gossmx_profile_read(gossmx_ctx* ctx, gossmx_profile_record* out, size_t capacity, size_t* written);
/* Also clears the per-stage records below and their dropped count. */
int gossmx_profile_reset(gossmx_ctx* ctx);

/* Per-stage records of the profiled calls, a fixed-layout record per stage
 * like CpuExecutionProfileRecord (cpu_profile.rs:121-150): the operation, the
 * layer and phase the caller tagged, the shape, the projection role, the
 * kernel family that ran, and the timing from the stage's events. A context
 * keeps at most GOSSMX_PROFILE_CAPACITY records between resets; later stages
 * still add to the totals of gossmx_profile_read and count as dropped. */
enum {
  GOSSMX_ROLE_NONE = 0,
  GOSSMX_ROLE_ROUTER = 1,
  GOSSMX_ROLE_GATE_UP = 2,
  GOSSMX_ROLE_DOWN = 3
};
enum {
  GOSSMX_KERNEL_ROUTE = 0,          /* router / selection / grouping kernels */
  GOSSMX_KERNEL_GEMV = 1,           /* one work-group per (row block, route): few rows */
  GOSSMX_KERNEL_GEMM = 2,           /* MFMA tiles; rows_per_item tells the geometry */
  GOSSMX_KERNEL_EXACT = 3,          /* exact-BF16 expert projection */
  GOSSMX_KERNEL_COMBINE = 4         /* routing-weight accumulation */
};
enum {
  GOSSMX_PHASE_UNKNOWN = 0,
  GOSSMX_PHASE_PREFILL = 1,
  GOSSMX_PHASE_DECODE = 2
};
#define GOSSMX_PROFILE_CAPACITY 65536
typedef struct gossmx_profile_event {
  uint64_t sequence;        /* per context, from 0 after a reset */
  int32_t op;               /* GOSSMX_OP_* */
  int32_t role;             /* GOSSMX_ROLE_* */
  int32_t kernel;           /* GOSSMX_KERNEL_* */
  int32_t layer;            /* gossmx_profile_tag value; -1 untagged */
  int32_t phase;            /* GOSSMX_PHASE_* from gossmx_profile_tag */
  int32_t memory;           /* GOSSMX_MEM_HOST or GOSSMX_MEM_DEVICE */
  uint32_t m;               /* activation rows of the call */
  uint32_t n;               /* output columns of the stage (0: none) */
  uint32_t k;               /* input columns of the stage */
  uint32_t routes;          /* (row, expert) pairs of the call */
  uint32_t rows_per_item;   /* GEMM work-item rows (0 off the GEMM) */
  uint32_t reserved;
  uint64_t start_ns;        /* from the first recorded stage after a reset */
  uint64_t duration_ns;
  uint64_t scratch_bytes;   /* the context's scratch buffers at the call */
  uint64_t resident_bytes;  /* process resident bytes at the call */
} gossmx_profile_event;
/* Layer index and phase stamped on the following records (the model step sets
 * them per layer; -1 and GOSSMX_PHASE_UNKNOWN by default). */
int gossmx_profile_tag(gossmx_ctx* ctx, int layer, int phase);
/* Synchronizes, then copies up to `capacity` records (oldest first) without
 * consuming them; *available receives the count kept, *dropped those lost
 * to the cap. */
int gossmx_profile_events(gossmx_ctx* ctx, gossmx_profile_event* out, size_t capacity, size_t* written,
                          size_t* available, uint64_t* dropped);

/* HIP-graph capture of a sequence of calls on this context (no counterpart in
 * the reference; it removes the per-kernel launch gaps of a multi-layer step).
 * Between begin and end, gossmx_moe_forward / gossmx_mxfp4_matmul calls with
 * GOSSMX_MEM_DEVICE pointers are recorded, not run; host-memory calls and
 * profiling are refused, and scratch buffers must already be large enough
 * (run the same shapes once eagerly first). A graph replays on the context's
 * stream with the pointers it was recorded with, including the context's
 * scratch buffers: while a graph is alive, a later call that needs larger
 * scratch gets new buffers and the old ones stay allocated until the last graph
 * of the context is destroyed, so eager calls of any size may run between
 * replays. Replays and eager calls share the scratch, so they must not overlap
 * (both run on the context's stream, which orders them). Device-side checks
 * surface at gossmx_synchronize as usual. Destroy graphs before the context. */
typedef struct gossmx_graph gossmx_graph;
int gossmx_capture_begin(gossmx_ctx* ctx);
int gossmx_capture_end(gossmx_ctx* ctx, gossmx_graph** out);
int gossmx_graph_launch(gossmx_ctx* ctx, const gossmx_graph* graph);
void gossmx_graph_destroy(gossmx_graph* graph);

/* Test hook for the next projection call on this context (gossmx_moe_forward,
 * gossmx_moe_forward_residual, gossmx_mxfp4_matmul), after its argument checks
 * and before it launches anything (outputs untouched): armed = 1 fails it with
 * GOSSMX_ERR_INJECTED_FAULT (a model error, like CpuExecutionFailurePoint);
 * armed = 2 fails it as a device fault, GOSSMX_ERR_DEVICE, which opens the
 * circuit breaker; armed = 3 lets the call run and raises the device's
 * work-order error flag ahead of its kernels (a host-sourced copy), so the
 * failure (GOSSMX_ERR_DEVICE, breaker opened) surfaces where the flags are
 * next read: inside a host-memory call, at gossmx_synchronize after a
 * device-memory one, or in the model step that made the call; 0 disarms. */
int gossmx_inject_fault(gossmx_ctx* ctx, int armed);

/* Device self-test of what the GEMM relies on: the FP4 -> f16 conversion order,
 * the 16x16x32 MFMA operand/result layout, the scaled conversion with clean
 * and with dirty scale operands (E8M0 byte in the exponent field, the
 * neighbouring bytes in the sign and mantissa bits), and the SwiGLU sigmoid
 * table against the host expf. No counterpart in the reference;
 * GOSSMX_ERR_UNSUPPORTED with a message on any mismatch. */
int gossmx_selftest(gossmx_ctx* ctx);
/* The kernels round f32 to bf16 with gfx950's conversion instruction; this
 * runs it on all 2^32 f32 bit patterns against half 2.7.1's rounding (nearest
 * even, NaN quieted with its sign and upper payload kept) restated in integer
 * operations, and counts the differences into *mismatches (0 expected). No
 * counterpart in the reference; a diagnostic (about 0.1 s). */
int gossmx_selftest_bf16_exhaustive(gossmx_ctx* ctx, uint64_t* mismatches);

/* ---------------------------------------------------------------------------
 * The dense path around the block (crates/gpt-oss-model-runner/src/
 * cpu_runner.rs): a GPT-OSS model that computes what the reference's CPU runner
 * computes, bit for bit. Attention, RoPE, norms and the KV caches run on host
 * threads. The Q/K/V/O projections and lm_head run on the context's GPU with the
 * reference's 16-lane dot order, over copies of those matrices made in HBM by
 * gossmx_model_create (about 2.4 GB for GPT-OSS-20B, with the post-attention
 * norm weights). The MoE halves run on the GPU through
 * gossmx_moe_forward_residual (device memory, one round trip per layer with the
 * O projection). The embedding, the input and final norm weights, the sinks and
 * the MoE layers stay borrowed and must outlive the model. A model holds one
 * sequence's KV caches. */
typedef struct gossmx_model gossmx_model;

/* CpuGptOssConfig (cpu_runner.rs:252-291) and the sequence's context cap
 * (new_sequence_state, :1596-1627). */
typedef struct gossmx_model_config {
  size_t vocab;                       /* vocab_size */
  size_t hidden;                      /* hidden_size; equal to every MoE layer's hidden */
  size_t layers;                      /* num_hidden_layers */
  size_t heads;                       /* num_attention_heads */
  size_t kv_heads;                    /* num_key_value_heads; divides heads */
  size_t head_dim;                    /* even */
  size_t sliding_window;              /* KV tokens a sliding layer keeps */
  size_t context_cap;                 /* KV tokens a full layer keeps; positions stay below it */
  float rms_norm_eps;
  double rope_theta;
  int rope_yarn;                      /* rope_scaling present (YaRN): 1, absent: 0 */
  double rope_factor;
  size_t rope_original_max_positions; /* original_max_position_embeddings */
  double rope_beta_fast;              /* 32 by default */
  double rope_beta_slow;              /* 1 by default */
  int rope_truncate;
  size_t threads;                     /* host threads for the dense path; 0: all hardware threads (at most 64) */
} gossmx_model_config;

/* One decoder layer (CpuLayer, load_layer cpu_runner.rs:3526-3671). Vectors are
 * f32 (the reference loads them to f32), matrices bf16 row-major [out][in]. */
typedef struct gossmx_dense_layer {
  const float* input_norm;          /* [hidden] */
  const uint16_t* q_weight;         /* [heads * head_dim][hidden] */
  const float* q_bias;              /* [heads * head_dim] */
  const uint16_t* k_weight;         /* [kv_heads * head_dim][hidden] */
  const float* k_bias;              /* [kv_heads * head_dim] */
  const uint16_t* v_weight;         /* [kv_heads * head_dim][hidden] */
  const float* v_bias;              /* [kv_heads * head_dim] */
  const uint16_t* o_weight;         /* [hidden][heads * head_dim] */
  const float* o_bias;              /* [hidden] */
  const float* sinks;               /* [heads] */
  const float* post_attention_norm; /* [hidden] */
  int sliding;                      /* layer_types "sliding_attention" / "local_attention" */
  const gossmx_layer* moe;          /* this layer's MoE block */
} gossmx_dense_layer;

/* CpuModel::load + new_sequence_state. embedding and lm_head bf16 [vocab][hidden],
 * final_norm f32 [hidden], layers [config->layers]. */
int gossmx_model_create(gossmx_ctx* ctx, const gossmx_model_config* config, const uint16_t* embedding,
                        const float* final_norm, const uint16_t* lm_head, const gossmx_dense_layer* layers,
                        gossmx_model** out);
void gossmx_model_destroy(gossmx_model* model);
/* CpuModelRunner::reset (:1803-1807): empty caches, position 0. */
int gossmx_model_reset(gossmx_model* model);
/* CpuModelRunner::prefill_layer_major (:1827-1855): reset, then all n tokens as
 * one layer-major step (positions 0..n-1, each layer's MoE over the n rows);
 * logits [vocab] of the last token, bf16 values (:2300-2312). */
int gossmx_model_prefill(gossmx_model* model, const uint32_t* tokens, size_t n, float* logits);
/* prepare_step + commit (:2080-2333, :1081-1113) of n more tokens of the
 * sequence at its current position, as one layer-major step (a prompt chunk);
 * logits of the last one. */
int gossmx_model_append(gossmx_model* model, const uint32_t* tokens, size_t n, float* logits);
/* CpuModelRunner::decode (:1877-1885): one token at the next position. */
int gossmx_model_decode(gossmx_model* model, uint32_t token, float* logits);
/* Steps are transactional (prepare/commit, :1081-1113): on any error the caches
 * and the position are unchanged. */
int gossmx_model_position(const gossmx_model* model, size_t* position);
/* CpuKvCache::len / start_position of a layer's cache (:674-680). */
int gossmx_model_cache(const gossmx_model* model, size_t layer, size_t* len, size_t* start_position);
/* Wall time spent so far in the dense path and in the MoE calls (including
 * their host<->device copies). */
int gossmx_model_times(const gossmx_model* model, double* dense_seconds, double* moe_seconds);

/* greedy_token (crates/gpt-oss-bench/src/bin/cpu_parity.rs:750-762): the
 * largest finite logit, the lowest index on ties. */
int gossmx_greedy_token(const float* logits, size_t n, uint32_t* token);
/* YarnRope::new + apply (cpu_runner.rs:3933-4013) over values [heads][head_dim]
 * in place, for one position (uses config->head_dim and the rope fields only). */
int gossmx_yarn_rope(const gossmx_model_config* config, float* values, size_t heads, size_t position);
/* attention_one_staged (cpu_runner.rs:3840-3924) for one query [heads][head_dim]
 * over the last min(tokens, window) of `tokens` key/value rows bf16
 * [tokens][kv_heads][head_dim] (a cache of capacity `window` after `tokens`
 * appends); out [heads][head_dim] (bf16 values). */
int gossmx_attention(const float* query, const uint16_t* keys, const uint16_t* values, size_t tokens, size_t window,
                     const float* sinks, size_t heads, size_t kv_heads, size_t head_dim, float* out);

#ifdef __cplusplus
}
#endif

#endif /* GOSSMX_H */
