// C ABI of libgossmx.so (include/gossmx.h): contexts, resident weights, the
// kernel-boundary matmul and the MoE block, profiling and the fault hook.
#include "../../include/gossmx.h"
#include "gossmx_internal.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

using namespace gossmx;

namespace {

thread_local std::string g_last_error;

// Fixed scratch of gossmx_moe_forward_noalloc, for callers that cannot
// allocate: one copy per device (each device holds its own until the process
// ends). Host code never passes the array's name to a kernel or a copy: it
// is a host-side stand-in; the device address comes from hipGetSymbolAddress
// (scratch_address), taken once per device at context creation.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
int g_scratch_state[kMaxDevices] = {};  // 0: not looked up, 1: found, -1: lookup failed

// Process-wide circuit breaker of the GPU backend, the counterpart of the Xe
// engine's PROCESS_XE_CIRCUIT_OPEN (crates/gpt-oss-xe/src/lib.rs:605-724): a
// projection that fails at run time (a HIP error, or the injected device
// fault) drains its stream and opens the circuit; while it is open every
// projection call returns GOSSMX_ERR_CIRCUIT_OPEN after validating its
// arguments, so the caller recomputes once on its CPU path and stays there
// until gossmx_circuit_reset().
std::atomic<bool> g_circuit_open{false};

// Process-wide accounting (gossmx_stats_read): projection results, transfer
// bytes by direction, and the resident bytes of live weights and layers with
// their optional cap.
struct Stats {
  std::atomic<uint64_t> ok{0}, failed{0}, refused{0}, rejected{0};
  std::atomic<uint64_t> transfer[3] = {};  // TransferDirection
  std::atomic<uint64_t> resident{0}, high_water{0}, cap{0}, cap_refusals{0};
  std::atomic<uint64_t> cache_hits{0}, cache_misses{0};
};
Stats g_stats;

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(e == hipErrorOutOfMemory ? GOSSMX_ERR_OUT_OF_MEMORY : GOSSMX_ERR_DEVICE, "%s: %s", what,
              hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                   \
  do {                                        \
    hipError_t e_ = (expr);                   \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// A grow-only device buffer.
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
};

// What a profiled stage records beside its events: the stage's shape and
// kernel family, and the call it belongs to.
struct StageInfo {
  int role = GOSSMX_ROLE_NONE;
  int kernel = GOSSMX_KERNEL_ROUTE;
  uint32_t n = 0, k = 0, rows_per_item = 0;
};
struct CallInfo {
  int layer = -1, phase = GOSSMX_PHASE_UNKNOWN, memory = GOSSMX_MEM_DEVICE;
  uint32_t m = 0, routes = 0;
  uint64_t scratch_bytes = 0, resident_bytes = 0;
};

struct ProfileMark {
  int op;
  hipEvent_t start, stop;
  StageInfo stage;
  CallInfo call;
};

}  // namespace

struct gossmx_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  int* err = nullptr;  // [0]: device error flags; [1]: route_select_kernel's arrival counter (0 between launches)
  uint16_t* sig_tab = nullptr;  // SwiGLU sigmoid table (built at context creation)
  bool fast_ok = true;          // the scaled FP4 conversion passed the self-test (see run_selftest)
  bool capturing = false;
  int fault_armed = 0;          // gossmx_inject_fault mode for the next projection call
  // Instantiated graphs of this context still alive. While any is, scratch
  // buffers that must grow are retired (kept until the last graph is
  // destroyed) instead of freed: the graphs hold their addresses.
  int live_graphs = 0;
  std::vector<void*> retired;
  bool profiling = false;
  std::vector<ProfileMark> marks;
  std::vector<hipEvent_t> event_pool;
  double op_ms[GOSSMX_OP_COUNT] = {0};
  uint64_t op_launches[GOSSMX_OP_COUNT] = {0};
  // Per-stage records (gossmx_profile_events): at most
  // GOSSMX_PROFILE_CAPACITY between resets, timed from `prof_base`, the
  // first recorded stage's start event (kept out of the pool until a reset).
  std::vector<gossmx_profile_event> events;
  uint64_t events_dropped = 0, events_seq = 0;
  hipEvent_t prof_base = nullptr;
  int tag_layer = -1, tag_phase = GOSSMX_PHASE_UNKNOWN;
  CallInfo call;  // the profiled call in progress
  // Pinned host staging of the host-memory MoE calls (grow-only): the inputs
  // (one host-to-device copy), and the outputs with the error flags (coherent
  // memory the kernels write directly; one synchronization).
  char* h_in = nullptr;
  size_t in_cap = 0;
  char* h_stage = nullptr;
  size_t stage_cap = 0;
  // scratch (x: the host-memory MoE call's input pack)
  DevBuf x, logits, selected, weights, act1v, act1s, bucket, route_tok, route_slot, work, act2v, act2s, y, cnt,
      trace, trace_gu, trace_sw, rec, bias, mout, unrounded;
  template <class F>
  void each_buf(F f) {
    for (DevBuf* b : {&x, &logits, &selected, &weights, &act1v, &act1s, &bucket, &route_tok, &route_slot, &work,
                      &act2v, &act2s, &y, &cnt, &trace, &trace_gu, &trace_sw, &rec, &bias, &mout, &unrounded})
      f(*b);
  }
};

struct gossmx_weights {
  int device = 0;
  TiledWeights t;
  uint64_t resident = 0;  // bytes taken from the resident budget
};

struct gossmx_graph {
  gossmx_ctx* ctx = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int device = 0;
};

struct gossmx_layer {
  int device = 0;
  gossmx_moe_config cfg;
  const gossmx_weights* gate_up = nullptr;
  const gossmx_weights* down = nullptr;
  uint16_t* router_w = nullptr;
  float* router_b = nullptr;
  float* gate_up_bias = nullptr;
  float* down_bias = nullptr;
  uint64_t resident = 0;  // bytes taken from the resident budget
};

namespace {

int ensure(gossmx_ctx* ctx, DevBuf& b, size_t bytes) {
  if (bytes <= b.cap) return GOSSMX_OK;
  if (ctx->capturing)
    return fail(GOSSMX_ERR_UNSUPPORTED, "scratch would grow during graph capture; run the same shapes eagerly first");
  if (b.p) {
    if (ctx->live_graphs > 0) {
      ctx->retired.push_back(b.p);  // a live graph still reads and writes it
    } else {
      HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
      HIP_TRY(hipFree(b.p), "hipFree");
    }
    b.p = nullptr;
    b.cap = 0;
  }
  const size_t cap = std::max<size_t>(bytes, 256) * 5 / 4;
  HIP_TRY(hipMalloc(&b.p, cap), "hipMalloc(scratch)");
  b.cap = cap;
  return GOSSMX_OK;
}

// Grow-only pinned host staging. The stream is drained before a smaller
// buffer is freed: work of an earlier call that ended in an error may still
// read or write it. `flags`: hipHostMalloc flags (coherent staging is written
// by kernels directly).
int ensure_pinned(gossmx_ctx* ctx, char** p, size_t* cap, size_t bytes, unsigned flags = hipHostMallocDefault) {
  if (bytes <= *cap) return GOSSMX_OK;
  if (*p) {
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    HIP_TRY(hipHostFree(*p), "hipHostFree");
  }
  *p = nullptr;
  *cap = 0;
  const size_t want = std::max<size_t>(bytes, 4096) * 5 / 4;
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(p), want, flags), "pinned staging");
  *cap = want;
  return GOSSMX_OK;
}

constexpr size_t align16(size_t n) { return (n + 15) / 16 * 16; }

// A fixed block of device memory that a call's scratch is carved from
// (256-byte aligned pieces), instead of the context's grow-only buffers.
struct ScratchArena {
  char* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
};

// `bytes` of scratch for one buffer role: carved from `arena` when one is
// given (failing, before anything is launched, when it is full), else the
// context's grow-only buffer `b`.
template <class T>
int take(gossmx_ctx* ctx, ScratchArena* arena, DevBuf& b, size_t bytes, T** out) {
  if (arena) {
    const size_t off = (arena->used + 255) & ~(size_t)255;
    if (off > arena->cap || bytes > arena->cap - off)
      return fail(GOSSMX_ERR_UNSUPPORTED, "this call needs more than the %zu bytes of fixed scratch", arena->cap);
    *out = reinterpret_cast<T*>(arena->base + off);
    arena->used = off + bytes;
    return GOSSMX_OK;
  }
  if (int s = ensure(ctx, b, bytes)) return s;
  *out = static_cast<T*>(b.p);
  return GOSSMX_OK;
}

hipEvent_t take_event(gossmx_ctx* ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Brackets one launch with events when profiling is on.
struct OpScope {
  gossmx_ctx* ctx;
  int op;
  StageInfo info;
  hipEvent_t start = nullptr;
  OpScope(gossmx_ctx* c, int o, StageInfo i = {}) : ctx(c), op(o), info(i) {
    if (ctx->profiling && !ctx->capturing) {
      start = take_event(ctx);
      if (start) (void)hipEventRecord(start, ctx->stream);
    }
  }
  ~OpScope() {
    if (start) {
      hipEvent_t stop = take_event(ctx);
      if (stop) {
        (void)hipEventRecord(stop, ctx->stream);
        ctx->marks.push_back({op, start, stop, info, ctx->call});
      } else {
        ctx->event_pool.push_back(start);
      }
    }
  }
};

// A stage of exactly one kernel: the launch itself records the start and stop
// events (hipExtLaunchKernelGGL), so the interval is the kernel's execution
// alone, without the stream's launch gaps around it.
struct KernelScope {
  gossmx_ctx* ctx;
  int op;
  StageInfo info;
  hipEvent_t start = nullptr, stop = nullptr;
  KernelScope(gossmx_ctx* c, int o, StageInfo i = {}) : ctx(c), op(o), info(i) {
    if (ctx->profiling && !ctx->capturing) {
      start = take_event(ctx);
      stop = start ? take_event(ctx) : nullptr;
      if (!stop && start) {
        ctx->event_pool.push_back(start);
        start = nullptr;
      }
    }
  }
  ~KernelScope() {
    if (start) ctx->marks.push_back({op, start, stop, info, ctx->call});
  }
};

// Folds the recorded stages into the per-operation totals and the per-stage
// records (synchronizes the stream).
int fold_profile(gossmx_ctx* ctx) {
  if (ctx->marks.empty()) return GOSSMX_OK;
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (!ctx->prof_base) ctx->prof_base = ctx->marks.front().start;
  for (const ProfileMark& m : ctx->marks) {
    float ms = 0.0f, at = 0.0f;
    if (hipEventElapsedTime(&ms, m.start, m.stop) == hipSuccess) {
      ctx->op_ms[m.op] += ms;
      ctx->op_launches[m.op] += 1;
      if (ctx->events.size() < GOSSMX_PROFILE_CAPACITY) {
        if (hipEventElapsedTime(&at, ctx->prof_base, m.start) != hipSuccess) at = 0.0f;
        gossmx_profile_event ev{};
        ev.sequence = ctx->events_seq;
        ev.op = m.op;
        ev.role = m.stage.role;
        ev.kernel = m.stage.kernel;
        ev.layer = m.call.layer;
        ev.phase = m.call.phase;
        ev.memory = m.call.memory;
        ev.m = m.call.m;
        ev.n = m.stage.n;
        ev.k = m.stage.k;
        ev.routes = m.call.routes;
        ev.rows_per_item = m.stage.rows_per_item;
        ev.start_ns = (uint64_t)std::llround(std::max(0.0, (double)at * 1e6));
        ev.duration_ns = (uint64_t)std::llround(std::max(0.0, (double)ms * 1e6));
        ev.scratch_bytes = m.call.scratch_bytes;
        ev.resident_bytes = m.call.resident_bytes;
        ctx->events.push_back(ev);
      } else {
        ctx->events_dropped += 1;
      }
      ctx->events_seq += 1;
    }
    if (m.start != ctx->prof_base) ctx->event_pool.push_back(m.start);
    ctx->event_pool.push_back(m.stop);
  }
  ctx->marks.clear();
  return GOSSMX_OK;
}

// The call about to be profiled: its shape, memory and scratch, and the
// caller's layer / phase tag.
void begin_call(gossmx_ctx* ctx, size_t m, size_t routes, int memory, uint64_t scratch_bytes) {
  if (!ctx->profiling) return;
  CallInfo& c = ctx->call;
  c.layer = ctx->tag_layer;
  c.phase = ctx->tag_phase;
  c.memory = memory;
  c.m = (uint32_t)std::min<size_t>(m, UINT32_MAX);
  c.routes = (uint32_t)std::min<size_t>(routes, UINT32_MAX);
  c.scratch_bytes = scratch_bytes;
  c.resident_bytes = g_stats.resident.load(std::memory_order_relaxed);
}

uint64_t context_scratch_bytes(gossmx_ctx* ctx) {
  uint64_t total = 0;
  ctx->each_buf([&](DevBuf& b) { total += b.cap; });
  return total;
}

void raise_high_water(uint64_t v) {
  uint64_t hw = g_stats.high_water.load();
  while (v > hw && !g_stats.high_water.compare_exchange_weak(hw, v)) {
  }
}

// Takes `bytes` of the resident budget before an allocation; past the cap
// the creation fails (and counts a capacity refusal).
int reserve_resident(uint64_t bytes, const char* what) {
  const uint64_t cap = g_stats.cap.load();
  uint64_t cur = g_stats.resident.load();
  for (;;) {
    if (cap != 0 && (cur > cap || bytes > cap - cur)) {
      g_stats.cap_refusals.fetch_add(1);
      return fail(GOSSMX_ERR_OUT_OF_MEMORY, "%s of %llu bytes would pass the resident cap (%llu of %llu bytes held)",
                  what, (unsigned long long)bytes, (unsigned long long)cur, (unsigned long long)cap);
    }
    if (g_stats.resident.compare_exchange_weak(cur, cur + bytes)) break;
  }
  raise_high_water(cur + bytes);
  return GOSSMX_OK;
}

void release_resident(uint64_t bytes) { g_stats.resident.fetch_sub(bytes); }

// Counts a projection call by its result.
int count_projection(int status) {
  switch (status) {
    case GOSSMX_OK: g_stats.ok.fetch_add(1, std::memory_order_relaxed); break;
    case GOSSMX_ERR_CIRCUIT_OPEN: g_stats.refused.fetch_add(1, std::memory_order_relaxed); break;
    case GOSSMX_ERR_DEVICE:
    case GOSSMX_ERR_OUT_OF_MEMORY:
    case GOSSMX_ERR_INJECTED_FAULT: g_stats.failed.fetch_add(1, std::memory_order_relaxed); break;
    default: g_stats.rejected.fetch_add(1, std::memory_order_relaxed); break;
  }
  return status;
}

// Clears the sticky device error flags after a read that found `flags` set,
// and returns the error they name.
int device_flags_fail(gossmx_ctx* ctx, int flags) {
  HIP_TRY(launch_clear_ints(ctx->err, 1, ctx->stream), "clear error flags");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (flags & kErrWorkOrder) return fail(GOSSMX_ERR_DEVICE, "internal: work list not in the order a kernel relies on");
  if (flags & kErrNonFiniteLogits) return fail(GOSSMX_ERR_NON_FINITE_LOGITS, "router produced non-finite logits");
  return fail(GOSSMX_ERR_NON_FINITE_INPUT, "kernel input contains a non-finite value");
}

// Reads and clears the sticky device error flags (synchronizes).
int check_device_errors(gossmx_ctx* ctx) {
  int flags = 0;
  HIP_TRY(hipMemcpyAsync(&flags, ctx->err, sizeof(int), hipMemcpyDeviceToHost, ctx->stream), "read error flags");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return flags == 0 ? GOSSMX_OK : device_flags_fail(ctx, flags);
}

int set_device(int device) {
  HIP_TRY(hipSetDevice(device), "hipSetDevice");
  return GOSSMX_OK;
}

// Looks up the device address of `scratch` on `device` (which must be
// current) the first time a context is created on it.
void scratch_lookup(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_state[device] != 0) return;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  g_scratch_ptr[device] = e == hipSuccess ? ptr : nullptr;
  g_scratch_state[device] = (e == hipSuccess && ptr != nullptr) ? 1 : -1;
}

// The device address of `scratch` on `device`, or null.
void* scratch_address(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  return g_scratch_state[device] == 1 ? g_scratch_ptr[device] : nullptr;
}

// The checks every projection call makes after validating its arguments and
// before touching the device: the circuit breaker, then the fault hook.
int projection_gate(gossmx_ctx* ctx) {
  if (g_circuit_open.load(std::memory_order_acquire))
    return fail(GOSSMX_ERR_CIRCUIT_OPEN, "GPU circuit breaker is open");
  const int mode = ctx->fault_armed;
  ctx->fault_armed = 0;
  if (mode == 1) return fail(GOSSMX_ERR_INJECTED_FAULT, "injected fault before launch");
  if (mode == 2) return fail(GOSSMX_ERR_DEVICE, "injected device fault before launch");
  if (mode == 3) {
    // The call runs, and the device's work-order flag is raised ahead of its
    // kernels in stream order (a host-sourced copy, no kernel faults), so the
    // failure surfaces where the call's device flags are next read.
    static const int kRaised = kErrWorkOrder;
    HIP_TRY(hipMemcpyAsync(ctx->err, &kRaised, sizeof(int), hipMemcpyHostToDevice, ctx->stream), "raise flag");
  }
  return GOSSMX_OK;
}

// A projection's result: a run-time failure (HIP error or out of memory,
// including the injected device fault) drains the stream and opens the
// circuit (execute_projection, crates/gpt-oss-xe/src/lib.rs:680-724).
int projection_result(gossmx_ctx* ctx, int status) {
  if (status == GOSSMX_ERR_DEVICE || status == GOSSMX_ERR_OUT_OF_MEMORY) {
    if (ctx) (void)hipStreamSynchronize(ctx->stream);
    g_circuit_open.store(true, std::memory_order_release);
  }
  return status;
}

TiledWeights make_tiled(size_t experts, size_t rows, size_t blocks) {
  TiledWeights t;
  t.experts = experts;
  t.rows = rows;
  t.blocks = blocks;
  t.tiles = (rows + kTileRows - 1) / kTileRows;
  t.nib_stride = t.tiles * 256 * blocks;
  t.scl_stride = t.tiles * 64 * ((blocks + 3) / 4);
  return t;
}

int alloc_tiled(gossmx_ctx* ctx, size_t experts, size_t rows, size_t blocks, gossmx_weights** out) {
  if (!ctx || !out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context or output handle");
  if (experts == 0 || rows == 0 || blocks == 0)
    return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "invalid MXFP4 tensor shape [%zu, %zu, %zu]", experts, rows, blocks);
  if (int s = set_device(ctx->device)) return s;
  auto* w = new gossmx_weights();
  w->device = ctx->device;
  w->t = make_tiled(experts, rows, blocks);
  if (w->t.nib_stride > (size_t)INT32_MAX - kPlaneSlack || w->t.scl_stride > (size_t)INT32_MAX - kPlaneSlack) {
    delete w;
    return fail(GOSSMX_ERR_UNSUPPORTED, "expert of %zu x %zu blocks too large for this build", rows, blocks);
  }
  const size_t nib_bytes = experts * w->t.nib_stride + kPlaneSlack, scl_bytes = experts * w->t.scl_stride + kPlaneSlack,
               fast_bytes = experts * w->t.tiles;
  if (int s = reserve_resident(nib_bytes + scl_bytes + fast_bytes, "MXFP4 weights")) {
    delete w;
    return s;
  }
  w->resident = nib_bytes + scl_bytes + fast_bytes;
  hipError_t e = hipMalloc(&w->t.nib, nib_bytes);
  if (e == hipSuccess) e = hipMalloc(&w->t.scl, scl_bytes);
  if (e == hipSuccess) e = hipMalloc(&w->t.fast, fast_bytes);
  // The scale bytes of the blocks past the last one in a compact last group
  // are never stored: zero them (E8M0 2^-127), so that every byte of the
  // plane converts to finite values (gemv_kernel converts whole groups).
  if (e == hipSuccess)
    e = launch_clear_ints(reinterpret_cast<int*>(w->t.scl), (experts * w->t.scl_stride + kPlaneSlack) / 4,
                          ctx->stream);
  if (e == hipSuccess) e = launch_fill_tiled_padding(w->t, ctx->stream);
  if (e != hipSuccess) {
    if (w->t.nib) (void)hipFree(w->t.nib);
    if (w->t.scl) (void)hipFree(w->t.scl);
    if (w->t.fast) (void)hipFree(w->t.fast);
    release_resident(w->resident);
    delete w;
    return hip_fail(e, "weights allocation");
  }
  *out = w;
  return GOSSMX_OK;
}

// Mxfp4MatmulProblem::new + validate_activation_extent (matmul.rs:245-267,
// 339-369) and the view checks of Mxfp4MatrixView::new (lib.rs:774-796).
int validate_problem(const gossmx_matmul_problem* p, size_t rows, size_t blocks, size_t experts) {
  if (!p) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null problem");
  if (p->activation_kind != GOSSMX_ACT_Q8 && p->activation_kind != GOSSMX_ACT_RESIDUAL_Q8)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown activation kind %d", p->activation_kind);
  if (p->memory != GOSSMX_MEM_HOST && p->memory != GOSSMX_MEM_DEVICE)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown memory kind %d", p->memory);
  if (!p->activations || !p->output) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null activations or output");
  if (p->expert >= experts) return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "expert %zu of %zu", p->expert, experts);
  const size_t m = p->m;
  if (m == 0 || p->blocks_per_row == 0 || p->row_stride < p->blocks_per_row ||
      (m - 1) > (SIZE_MAX - p->blocks_per_row) / std::max<size_t>(p->row_stride, 1) ||
      (m - 1) * p->row_stride + p->blocks_per_row > p->activations_len)
    return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "invalid activation matrix view: rows=%zu, blocks=%zu, stride=%zu, len=%zu",
                m, p->blocks_per_row, p->row_stride, p->activations_len);
  if (p->blocks_per_row != blocks || p->output_stride < rows ||
      (m - 1) > (SIZE_MAX - rows) / std::max<size_t>(p->output_stride, 1) ||
      (m - 1) * p->output_stride + rows > p->output_len || (p->bias && p->bias_len != rows))
    return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "invalid MXFP4 matmul: M=%zu, N=%zu, K=%zu, output_stride=%zu", m, rows,
                blocks * kBlock, p->output_stride);
  // The GEMM addresses the activation operand with 32-bit byte offsets.
  if (m > (size_t)INT32_MAX / 2 || rows > (size_t)INT32_MAX / 2 ||
      m * blocks * 2 * kBlock * sizeof(_Float16) >= (size_t)INT32_MAX - kActSlack)
    return fail(GOSSMX_ERR_UNSUPPORTED, "matrix too large for this build");
  return GOSSMX_OK;
}

}  // namespace

// Hooks for the host-side modules (gossmx_store.cpp, gossmx_dense.cpp).
namespace gossmx {

int set_error(int status, const char* message) { return fail(status, "%s", message); }

const gossmx_moe_config* layer_config(const gossmx_layer* layer) { return layer ? &layer->cfg : nullptr; }
int context_device(const gossmx_ctx* ctx) { return ctx->device; }
hipStream_t context_stream(const gossmx_ctx* ctx) { return ctx->stream; }
int run_time_result(gossmx_ctx* ctx, int status) { return projection_result(ctx, status); }

void count_transfer(int direction, size_t bytes) {
  if (direction >= 0 && direction < 3) g_stats.transfer[direction].fetch_add(bytes, std::memory_order_relaxed);
}

void count_repack_cache(bool hit) { (hit ? g_stats.cache_hits : g_stats.cache_misses).fetch_add(1); }

void tiled_image_bytes(size_t experts, size_t rows, size_t blocks, size_t* nib_bytes, size_t* scl_bytes) {
  const TiledWeights t = make_tiled(experts, rows, blocks);
  *nib_bytes = experts * t.nib_stride;
  *scl_bytes = experts * t.scl_stride;
}

int tiled_image_read(gossmx_ctx* ctx, const gossmx_weights* w, uint8_t* nib, uint8_t* scl) {
  if (!ctx || !w || !nib || !scl) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (w->device != ctx->device) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "weights live on another device");
  if (int s = set_device(ctx->device)) return s;
  HIP_TRY(hipMemcpyAsync(nib, w->t.nib, w->t.experts * w->t.nib_stride, hipMemcpyDeviceToHost, ctx->stream),
          "D2H nibble plane");
  HIP_TRY(hipMemcpyAsync(scl, w->t.scl, w->t.experts * w->t.scl_stride, hipMemcpyDeviceToHost, ctx->stream),
          "D2H scale plane");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return GOSSMX_OK;
}

int tiled_image_create(gossmx_ctx* ctx, size_t experts, size_t rows, size_t blocks, const uint8_t* nib,
                       const uint8_t* scl, gossmx_weights** out) {
  gossmx_weights* w = nullptr;
  if (int s = alloc_tiled(ctx, experts, rows, blocks, &w)) return s;
  count_transfer(kTransferUpload, experts * (w->t.nib_stride + w->t.scl_stride));
  hipError_t e = hipMemcpyAsync(w->t.nib, nib, experts * w->t.nib_stride, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(w->t.scl, scl, experts * w->t.scl_stride, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = launch_tile_flags(w->t, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    gossmx_weights_destroy(w);
    return hip_fail(e, "weights image upload");
  }
  *out = w;
  return GOSSMX_OK;
}

}  // namespace gossmx

static int run_selftest(gossmx_ctx* ctx, bool* scaled_ok);

// ===========================================================================
extern "C" {

const char* gossmx_last_error(void) { return g_last_error.c_str(); }
int gossmx_version(void) { return 100; }

int gossmx_device_count(int* count) {
  if (!count) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null count");
  *count = 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return GOSSMX_OK;
  for (int d = 0; d < n; ++d) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++*count;
  }
  return GOSSMX_OK;
}

int gossmx_ctx_create(int device, void* stream, gossmx_ctx** out) {
  if (!out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null output handle");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
    return fail(GOSSMX_ERR_UNAVAILABLE_BACKEND, "no HIP device %d", device);
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(GOSSMX_ERR_UNAVAILABLE_BACKEND, "device %d is %s, this build needs gfx950", device, prop.gcnArchName);
  if (int s = set_device(device)) return s;
  scratch_lookup(device);
  auto* ctx = new gossmx_ctx();
  ctx->device = device;
  if (stream) {
    ctx->stream = static_cast<hipStream_t>(stream);
  } else {
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete ctx;
      return hip_fail(e, "hipStreamCreate");
    }
    ctx->own_stream = true;
  }
  hipError_t e = hipMalloc(&ctx->err, 16);
  if (e == hipSuccess) e = launch_clear_ints(ctx->err, 4, ctx->stream);
  if (e == hipSuccess) e = hipMalloc(&ctx->sig_tab, 65536 * sizeof(uint16_t));
  if (e == hipSuccess) e = launch_build_sigmoid_table(ctx->sig_tab, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    gossmx_ctx_destroy(ctx);
    return hip_fail(e, "context setup");
  }
  // The lane layouts and the sigmoid table must hold on this device; the
  // scaled-conversion fast path is used only if its dirty-operand cases are
  // exact (otherwise every tile takes the masked E8M0 path).
  bool scaled_ok = true;
  if (int s = run_selftest(ctx, &scaled_ok)) {
    const std::string msg = g_last_error;
    gossmx_ctx_destroy(ctx);
    return fail(s, "device self-test failed: %s", msg.c_str());
  }
  ctx->fast_ok = scaled_ok;
  g_last_error.clear();
  *out = ctx;
  return GOSSMX_OK;
}

void gossmx_ctx_destroy(gossmx_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  for (auto& m : ctx->marks) {
    (void)hipEventDestroy(m.start);
    (void)hipEventDestroy(m.stop);
  }
  for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
  if (ctx->prof_base) (void)hipEventDestroy(ctx->prof_base);
  ctx->each_buf([](DevBuf& b) {
    if (b.p) (void)hipFree(b.p);
  });
  for (void* p : ctx->retired) (void)hipFree(p);
  if (ctx->err) (void)hipFree(ctx->err);
  if (ctx->sig_tab) (void)hipFree(ctx->sig_tab);
  if (ctx->h_in) (void)hipHostFree(ctx->h_in);
  if (ctx->h_stage) (void)hipHostFree(ctx->h_stage);
  if (ctx->own_stream && ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

int gossmx_ctx_set_stream(gossmx_ctx* ctx, void* stream) {
  if (!ctx || !stream) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context or stream");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (int s = fold_profile(ctx)) return s;
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
  ctx->stream = static_cast<hipStream_t>(stream);
  ctx->own_stream = false;
  return GOSSMX_OK;
}

void* gossmx_ctx_stream(gossmx_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int gossmx_synchronize(gossmx_ctx* ctx) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (int s = set_device(ctx->device)) return s;
  // Device-memory calls report their run-time failures here, so a device
  // fault found here opens the circuit breaker as inside a call.
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return projection_result(ctx, hip_fail(e, "hipStreamSynchronize"));
  return projection_result(ctx, check_device_errors(ctx));
}

int gossmx_malloc(gossmx_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (int s = set_device(ctx->device)) return s;
  HIP_TRY(hipMalloc(out, std::max<size_t>(bytes, 1)), "hipMalloc");
  return GOSSMX_OK;
}
int gossmx_free(gossmx_ctx* ctx, void* ptr) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (!ptr) return GOSSMX_OK;
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  HIP_TRY(hipFree(ptr), "hipFree");
  return GOSSMX_OK;
}
int gossmx_memcpy_h2d(gossmx_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpy H2D");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return GOSSMX_OK;
}
int gossmx_memcpy_d2h(gossmx_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy D2H");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  return GOSSMX_OK;
}

// --- weights ---------------------------------------------------------------

int gossmx_weights_upload(gossmx_ctx* ctx, const uint8_t* data, size_t len, size_t experts, size_t rows,
                          size_t blocks, int layout, gossmx_weights** out) {
  if (!ctx || !data || !out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (layout != GOSSMX_LAYOUT_CANONICAL_V1 && layout != GOSSMX_LAYOUT_X8_SPLIT_V2)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown source layout %d", layout);
  if (experts == 0 || rows == 0 || blocks == 0 || len != experts * rows * blocks * kRecord)
    return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "invalid MXFP4 matrix view: rows=%zu, blocks=%zu, bytes=%zu", rows,
                blocks, len);
  gossmx_weights* w = nullptr;
  if (int s = alloc_tiled(ctx, experts, rows, blocks, &w)) return s;
  void* staging = nullptr;
  hipError_t e = hipMalloc(&staging, len);
  count_transfer(kTransferUpload, len);
  if (e == hipSuccess) e = hipMemcpyAsync(staging, data, len, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = launch_repack(static_cast<const uint8_t*>(staging), layout, w->t, ctx->stream);
  if (e == hipSuccess) e = launch_tile_flags(w->t, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (staging) (void)hipFree(staging);
  if (e != hipSuccess) {
    gossmx_weights_destroy(w);
    return hip_fail(e, "weights upload");
  }
  *out = w;
  return GOSSMX_OK;
}

int gossmx_weights_generate(gossmx_ctx* ctx, uint64_t seed, uint64_t stream, size_t experts, size_t rows,
                            size_t blocks, gossmx_weights** out) {
  gossmx_weights* w = nullptr;
  if (int s = alloc_tiled(ctx, experts, rows, blocks, &w)) return s;
  hipError_t e = launch_generate(seed, stream, w->t, ctx->stream);
  if (e == hipSuccess) e = launch_tile_flags(w->t, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    gossmx_weights_destroy(w);
    return hip_fail(e, "weights generate");
  }
  *out = w;
  return GOSSMX_OK;
}

int gossmx_weights_export(gossmx_ctx* ctx, const gossmx_weights* w, uint8_t* out, size_t len) {
  if (!ctx || !w || !out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  const size_t need = w->t.experts * w->t.rows * w->t.blocks * kRecord;
  if (len != need) return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "export needs %zu bytes, got %zu", need, len);
  if (int s = set_device(ctx->device)) return s;
  void* dev = nullptr;
  HIP_TRY(hipMalloc(&dev, len), "hipMalloc(export)");
  hipError_t e = launch_export(w->t, static_cast<uint8_t*>(dev), ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out, dev, len, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (e != hipSuccess) return hip_fail(e, "weights export");
  return GOSSMX_OK;
}

int gossmx_weights_shape(const gossmx_weights* w, size_t* experts, size_t* rows, size_t* blocks) {
  if (!w) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null weights");
  if (experts) *experts = w->t.experts;
  if (rows) *rows = w->t.rows;
  if (blocks) *blocks = w->t.blocks;
  return GOSSMX_OK;
}

size_t gossmx_weights_device_bytes(const gossmx_weights* w) {
  return w ? w->t.experts * (w->t.nib_stride + w->t.scl_stride) : 0;
}

void gossmx_weights_destroy(gossmx_weights* w) {
  if (!w) return;
  // Work of any stream may still read the planes; the device-wide wait does
  // not need the context, which may already be gone.
  (void)hipSetDevice(w->device);
  (void)hipDeviceSynchronize();
  if (w->t.nib) (void)hipFree(w->t.nib);
  if (w->t.scl) (void)hipFree(w->t.scl);
  if (w->t.fast) (void)hipFree(w->t.fast);
  release_resident(w->resident);
  delete w;
}

// Rows per GEMM work item for a batch of m activation rows (it selects the
// kernel geometry). Batches of at most kSmallChunk rows: every bucket is one
// work item (more work-groups, fewer sequential K steps). Batches of at least
// kHugeMinRows rows: 32-row items share each weight block's conversion.
static int gemm_chunk(size_t m) {
  if (m <= (size_t)kSmallChunk) return kSmallChunk;
  return m >= (size_t)kHugeMinRows ? kHugeChunk : kChunk;
}

// Batches of at most kTinyMaxRows rows on weights of at most kTinyMaxBlocks
// blocks per row take the small-batch GEMV (whole K range per wave in
// registers) instead of the stepped GEMM.
static bool use_gemv(size_t m, size_t blocks, bool residual) {
  return residual && m <= (size_t)kTinyMaxRows && blocks <= (size_t)kTinyMaxBlocks;
}

// --- kernel boundary ---------------------------------------------------------

int gossmx_mxfp4_matmul_check(const gossmx_matmul_problem* p, size_t rows, size_t blocks, size_t experts) {
  return validate_problem(p, rows, blocks, experts);
}

static int matmul_impl(gossmx_ctx* ctx, const gossmx_matmul_problem* p) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (!p || !p->weights) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null problem or weights");
  const TiledWeights& w = p->weights->t;
  if (int s = validate_problem(p, w.rows, w.blocks, w.experts)) return s;
  if (ctx->capturing && p->memory == GOSSMX_MEM_HOST)
    return fail(GOSSMX_ERR_UNSUPPORTED, "host-memory calls cannot be captured");
  if (p->weights->device != ctx->device) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "weights live on another device");
  if (int s = projection_gate(ctx)) return s;
  if (int s = set_device(ctx->device)) return s;
  const size_t m = p->m, rows = w.rows, B = w.blocks;
  const size_t rsz = p->activation_kind == GOSSMX_ACT_RESIDUAL_Q8 ? 72 : 36;
  const size_t rec_count = (m - 1) * p->row_stride + B;
  const uint8_t* rec = static_cast<const uint8_t*>(p->activations);
  if (p->memory == GOSSMX_MEM_HOST) {
    if (int s = ensure(ctx, ctx->rec, rec_count * rsz)) return s;
    count_transfer(kTransferActivation, rec_count * rsz);
    HIP_TRY(hipMemcpyAsync(ctx->rec.p, rec, rec_count * rsz, hipMemcpyHostToDevice, ctx->stream), "H2D activations");
    rec = static_cast<const uint8_t*>(ctx->rec.p);
  }
  if (int s = ensure(ctx, ctx->act1v, m * B * 2 * kBlock * sizeof(_Float16) + kActSlack)) return s;
  if (int s = ensure(ctx, ctx->act1s, m * B * 2 * sizeof(float) + kActSlack)) return s;
  ActBuffers act{static_cast<_Float16*>(ctx->act1v.p), static_cast<float*>(ctx->act1s.p)};
  HIP_TRY(launch_prep_records(rec, p->activation_kind, m, B, p->row_stride, act, ctx->err, ctx->stream),
          "prepare activations");
  const float* bias = p->bias;
  if (bias && p->memory == GOSSMX_MEM_HOST) {
    if (int s = ensure(ctx, ctx->bias, rows * sizeof(float))) return s;
    count_transfer(kTransferUpload, rows * sizeof(float));
    HIP_TRY(hipMemcpyAsync(ctx->bias.p, p->bias, rows * sizeof(float), hipMemcpyHostToDevice, ctx->stream), "H2D bias");
    bias = static_cast<const float*>(ctx->bias.p);
  }
  float* out = p->output;
  size_t out_stride = p->output_stride;
  if (p->memory == GOSSMX_MEM_HOST) {
    if (int s = ensure(ctx, ctx->mout, m * rows * sizeof(float))) return s;
    out = static_cast<float*>(ctx->mout.p);
    out_stride = rows;
  }
  GemmArgs g{};
  g.w = w;
  g.fast_ok = ctx->fast_ok ? 1 : 0;
  g.actv = act.v;
  g.acts = act.s;
  g.bias = bias;
  g.residual = p->activation_kind == GOSSMX_ACT_RESIDUAL_Q8 ? 1 : 0;
  g.plain_expert = (int)p->expert;
  g.plain_m = (int)m;
  g.out = out;
  g.out_stride = out_stride;
  g.err = ctx->err;
  g.bias_expert_stride = 0;  // this problem's single bias vector
  begin_call(ctx, m, m, p->memory, context_scratch_bytes(ctx));
  {
    const bool gemv = use_gemv(m, B, g.residual != 0);
    KernelScope scope(ctx, GOSSMX_OP_MATMUL,
                      {GOSSMX_ROLE_NONE, gemv ? GOSSMX_KERNEL_GEMV : GOSSMX_KERNEL_GEMM, (uint32_t)rows,
                       (uint32_t)(B * kBlock), gemv ? 0u : (uint32_t)gemm_chunk(m)});
    if (gemv) {
      HIP_TRY(launch_gemv(kPlain, g, (int)m, 1, ctx->stream, scope.start, scope.stop), "matmul launch");
    } else {
      const int chunk = gemm_chunk(m);
      HIP_TRY(launch_gemm(kPlain, g, chunk, (int)((m + chunk - 1) / chunk), ctx->stream, scope.start, scope.stop),
              "matmul launch");
    }
  }
  if (p->memory == GOSSMX_MEM_HOST) {
    count_transfer(kTransferOutput, m * rows * sizeof(float));
    HIP_TRY(hipMemcpy2DAsync(p->output, p->output_stride * sizeof(float), out, rows * sizeof(float),
                             rows * sizeof(float), m, hipMemcpyDeviceToHost, ctx->stream),
            "D2H output");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  }
  return GOSSMX_OK;
}

int gossmx_mxfp4_matmul(gossmx_ctx* ctx, const gossmx_matmul_problem* p) {
  return count_projection(projection_result(ctx, matmul_impl(ctx, p)));
}

int gossmx_mxfp4_scratch_requirement(const gossmx_matmul_problem* p, size_t* size, size_t* alignment) {
  if (!size || !alignment) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null output");
  if (!p || !p->weights) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null problem or weights");
  const TiledWeights& w = p->weights->t;
  if (int s = validate_problem(p, w.rows, w.blocks, w.experts)) return s;
  // The device keeps its own operand buffers: Mxfp4ScratchRequirement::NONE.
  *size = 0;
  *alignment = 1;
  return GOSSMX_OK;
}

int gossmx_circuit_is_open(void) { return g_circuit_open.load(std::memory_order_acquire) ? 1 : 0; }

void gossmx_circuit_reset(void) { g_circuit_open.store(false, std::memory_order_release); }

// --- MoE block -------------------------------------------------------------

int gossmx_layer_create(gossmx_ctx* ctx, const gossmx_moe_config* cfg, const uint16_t* router_weight_bf16,
                        const float* router_bias, const gossmx_weights* gate_up, const float* gate_up_bias,
                        const gossmx_weights* down, const float* down_bias, gossmx_layer** out) {
  if (!ctx || !cfg || !router_weight_bf16 || !router_bias || !gate_up || !gate_up_bias || !down || !down_bias || !out)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  const size_t E = cfg->experts, H = cfg->hidden, I = cfg->intermediate, K = cfg->top_k;
  if (E == 0 || E > (size_t)kMaxExperts || K == 0 || K > (size_t)kMaxTopK || K > E || H == 0 || I == 0 ||
      H % kBlock || I % kBlock)
    return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "invalid MoE config E=%zu H=%zu I=%zu K=%zu", E, H, I, K);
  if (cfg->projection != GOSSMX_PROJECTION_RESIDUAL_Q8 && cfg->projection != GOSSMX_PROJECTION_Q8 &&
      cfg->projection != GOSSMX_PROJECTION_EXACT_BF16)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown expert projection %d", cfg->projection);
  if (gate_up->t.experts != E || gate_up->t.rows != 2 * I || gate_up->t.blocks != H / kBlock ||
      down->t.experts != E || down->t.rows != H || down->t.blocks != I / kBlock)
    return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "expert tensors do not match [%zu, %zu, %zu] / [%zu, %zu, %zu]", E, 2 * I,
                H / kBlock, E, H, I / kBlock);
  if (int s = set_device(ctx->device)) return s;
  const uint64_t bytes = E * H * 2 + E * 4 + E * 2 * I * 4 + E * H * 4;
  if (int s = reserve_resident(bytes, "MoE layer")) return s;
  auto* L = new gossmx_layer();
  L->device = ctx->device;
  L->cfg = *cfg;
  L->gate_up = gate_up;
  L->down = down;
  L->resident = bytes;
  count_transfer(kTransferUpload, bytes);
  hipError_t e = hipMalloc(&L->router_w, E * H * 2);
  if (e == hipSuccess) e = hipMalloc(&L->router_b, E * 4);
  if (e == hipSuccess) e = hipMalloc(&L->gate_up_bias, E * 2 * I * 4);
  if (e == hipSuccess) e = hipMalloc(&L->down_bias, E * H * 4);
  if (e == hipSuccess) e = hipMemcpy(L->router_w, router_weight_bf16, E * H * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(L->router_b, router_bias, E * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(L->gate_up_bias, gate_up_bias, E * 2 * I * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(L->down_bias, down_bias, E * H * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    gossmx_layer_destroy(L);
    return hip_fail(e, "layer upload");
  }
  *out = L;
  return GOSSMX_OK;
}

void gossmx_layer_destroy(gossmx_layer* L) {
  if (!L) return;
  (void)hipSetDevice(L->device);
  (void)hipDeviceSynchronize();
  if (L->router_w) (void)hipFree(L->router_w);
  if (L->router_b) (void)hipFree(L->router_b);
  if (L->gate_up_bias) (void)hipFree(L->gate_up_bias);
  if (L->down_bias) (void)hipFree(L->down_bias);
  release_resident(L->resident);
  delete L;
}

// The MoE block; with norm_weight, also the decoder layer's post-attention
// RMSNorm in front of it (io->x is then the residual stream) and the residual
// add behind it into next_residual.
static int moe_forward_impl(gossmx_ctx* ctx, const gossmx_layer* L, const gossmx_moe_io* io,
                            const float* norm_weight, float norm_eps, uint16_t* next_residual,
                            ScratchArena* arena = nullptr) {
  const bool residual = norm_weight != nullptr;
  if (!ctx || !L || !io || !io->x || (!io->output && !residual) || (residual && !next_residual))
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (io->memory != GOSSMX_MEM_HOST && io->memory != GOSSMX_MEM_DEVICE)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown memory kind %d", io->memory);
  if (io->m == 0) return fail(GOSSMX_ERR_INVALID_DIMENSIONS, "empty MoE batch");
  if (residual && L->cfg.hidden > (size_t)kNormMaxHidden)
    return fail(GOSSMX_ERR_UNSUPPORTED, "hidden size %zu above the fused RMSNorm's %d", L->cfg.hidden,
                kNormMaxHidden);
  if (residual && io->memory == GOSSMX_MEM_DEVICE &&
      (reinterpret_cast<uintptr_t>(io->x) % 16 != 0 || reinterpret_cast<uintptr_t>(norm_weight) % 16 != 0))
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "device x and norm_weight must be 16-byte aligned");
  if (ctx->capturing && io->memory == GOSSMX_MEM_HOST)
    return fail(GOSSMX_ERR_UNSUPPORTED, "host-memory calls cannot be captured");
  const size_t m = io->m, E = L->cfg.experts, H = L->cfg.hidden, I = L->cfg.intermediate, K = L->cfg.top_k;
  const size_t R = m * K, B1 = H / kBlock, B2 = I / kBlock;
  if (m > (size_t)(INT32_MAX / 8) / std::max<size_t>(H, E) ||
      R * std::max(B1, B2) * 2 * kBlock * sizeof(_Float16) >= (size_t)INT32_MAX - kActSlack)
    return fail(GOSSMX_ERR_UNSUPPORTED, "batch too large for this build");
  if (L->device != ctx->device) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "layer lives on another device");
  if (int s = projection_gate(ctx)) return s;
  if (int s = set_device(ctx->device)) return s;
  const bool host = io->memory == GOSSMX_MEM_HOST;
  const int proj = L->cfg.projection;
  const int chunk = gemm_chunk(m);
  const size_t max_work = (R + chunk - 1) / chunk + std::min(E, R);

  // Scratch: the context's grow-only buffers, or the no-allocation entry
  // point's fixed arena. Every piece is taken here, before the first launch.
  int s = GOSSMX_OK;
  float* logits_buf = nullptr;
  int *selected = nullptr, *bucket = nullptr, *work = nullptr, *route_tok = nullptr, *route_slot = nullptr;
  float* weights = nullptr;
  ActBuffers act1, act2;
  uint16_t* ybuf = nullptr;
  if ((s = take(ctx, arena, ctx->logits, m * E * 4, &logits_buf)) || (s = take(ctx, arena, ctx->selected, R * 4, &selected)) ||
      (s = take(ctx, arena, ctx->weights, R * 4, &weights)) ||
      (s = take(ctx, arena, ctx->act1v, m * B1 * 2 * kBlock * 2 + kActSlack, &act1.v)) ||
      (s = take(ctx, arena, ctx->act1s, m * B1 * 8 + kActSlack, &act1.s)) ||
      (s = take(ctx, arena, ctx->bucket, (E + 1) * 4, &bucket)) ||
      (s = take(ctx, arena, ctx->route_tok, R * 4, &route_tok)) ||
      (s = take(ctx, arena, ctx->route_slot, R * 4, &route_slot)) ||
      (s = take(ctx, arena, ctx->work, (4 * max_work + 1) * 4, &work)) ||
      (s = take(ctx, arena, ctx->act2v, R * B2 * 2 * kBlock * 2 + kActSlack, &act2.v)) ||
      (s = take(ctx, arena, ctx->act2s, R * B2 * 8 + kActSlack, &act2.s)) ||
      (s = take(ctx, arena, ctx->y, R * H * 2, &ybuf)))
    return s;
  // Batches whose logits fit one work-group take the fused selection +
  // dispatch kernel; larger ones a selection kernel with per-work-group
  // expert counts and a placement kernel. The router projection (when the
  // logits are not injected) is a kernel in front of either.
  const bool fused = m * (E + 1) <= (size_t)kSelectLds && R <= (size_t)kSelectMaxRoutes && K <= (size_t)kSelectTopK;
  int* cnt = nullptr;
  if (!fused) {
    const size_t n_sel = (m + select_rows_per_wg((int)E, (int)K) - 1) / select_rows_per_wg((int)E, (int)K);
    if ((s = take(ctx, arena, ctx->cnt, n_sel * E * 4, &cnt))) return s;
  }
  const uint16_t* x = io->x;
  const float* injected = io->injected_logits;
  float* output = io->output;
  uint16_t* output16 = nullptr;  // host memory: the output comes back as bf16 bits
  float* trace = io->trace_down;
  float* trace_gu = io->trace_gate_up;
  float* trace_sw = io->trace_swiglu;
  float* unrounded = io->output_unrounded;
  float* logits = (!host && io->router_logits) ? io->router_logits : logits_buf;
  // Host memory: the inputs (x, injected logits, norm weight) cross in one
  // copy from pinned staging; the outputs and the error flags come back in
  // one copy of a device pack (layout below).
  const float* norm_dev = norm_weight;
  if (host) {
    const size_t x_bytes = m * H * 2, inj_bytes = injected ? m * E * 4 : 0, nw_bytes = residual ? H * 4 : 0;
    const size_t off_inj = align16(x_bytes), off_nw = off_inj + align16(inj_bytes), in_bytes = off_nw + nw_bytes;
    if ((s = ensure(ctx, ctx->x, in_bytes)) || (s = ensure_pinned(ctx, &ctx->h_in, &ctx->in_cap, in_bytes))) return s;
    std::memcpy(ctx->h_in, io->x, x_bytes);
    if (inj_bytes) std::memcpy(ctx->h_in + off_inj, io->injected_logits, inj_bytes);
    if (nw_bytes) std::memcpy(ctx->h_in + off_nw, norm_weight, nw_bytes);
    count_transfer(kTransferActivation, x_bytes + inj_bytes + nw_bytes);
    HIP_TRY(hipMemcpyAsync(ctx->x.p, ctx->h_in, in_bytes, hipMemcpyHostToDevice, ctx->stream), "H2D inputs");
    char* const in = static_cast<char*>(ctx->x.p);
    x = reinterpret_cast<const uint16_t*>(in);
    if (inj_bytes) injected = reinterpret_cast<const float*>(in + off_inj);
    if (nw_bytes) norm_dev = reinterpret_cast<const float*>(in + off_nw);
    output = nullptr;
    if (trace) {
      if ((s = ensure(ctx, ctx->trace, R * H * 4))) return s;
      trace = static_cast<float*>(ctx->trace.p);
    }
    if (trace_gu) {
      if ((s = ensure(ctx, ctx->trace_gu, R * 2 * I * 4))) return s;
      trace_gu = static_cast<float*>(ctx->trace_gu.p);
    }
    if (trace_sw) {
      if ((s = ensure(ctx, ctx->trace_sw, R * I * 4))) return s;
      trace_sw = static_cast<float*>(ctx->trace_sw.p);
    }
    if (unrounded) {
      if ((s = ensure(ctx, ctx->unrounded, m * H * 4))) return s;
      unrounded = static_cast<float*>(ctx->unrounded.p);
    }
  }
  // Post-attention RMSNorm: the block runs on the normalized rows, the
  // residual add reads the rows as given.
  const uint16_t* resid = nullptr;
  uint16_t* next = nullptr;
  const float* route_norm_w = nullptr;
  if (residual) {
    next = next_residual;
    resid = x;
    // The router kernel normalizes each row as it reads it; with injected
    // logits the selection kernels' quantization work-groups do.
    route_norm_w = norm_dev;
  }
  // The host-memory output pack, in the context's coherent pinned staging:
  // the error flags word (16 bytes), then each requested output at a 16-byte
  // boundary. The output rows are bf16 values: they cross PCIe as bf16 bits
  // (half the bytes) and are widened into the caller's f32 rows after the
  // checks. The combine writes the rows and the next residual rows there
  // directly; pack_kernel writes the flags and the rest.
  struct Piece {
    const void* src;     // device source (null: written in place)
    void* dst;           // the caller's buffer
    size_t bytes = 0;    // device bytes
    bool widen = false;  // bf16 bits widened into f32 at dst
    size_t off = 0;      // in the pack
  };
  Piece pieces[kPackPieces];
  int n_pieces = 0;
  size_t pack_bytes = 16;
  if (host) {
    const Piece want[] = {
        {nullptr, io->output, io->output ? m * H * 2 : 0, true},
        {nullptr, next_residual, residual ? m * H * 2 : 0},
        {logits, io->router_logits, io->router_logits ? m * E * 4 : 0},
        {selected, io->selected, io->selected ? R * 4 : 0},
        {weights, io->routing_weights, io->routing_weights ? R * 4 : 0},
        {route_slot, io->route_order, io->route_order ? R * 4 : 0},
        {trace, io->trace_down, io->trace_down ? R * H * 4 : 0},
        {trace_gu, io->trace_gate_up, io->trace_gate_up ? R * 2 * I * 4 : 0},
        {trace_sw, io->trace_swiglu, io->trace_swiglu ? R * I * 4 : 0},
        {unrounded, io->output_unrounded, io->output_unrounded ? m * H * 4 : 0},
    };
    static_assert(sizeof(want) / sizeof(want[0]) == kPackPieces, "pack pieces");
    for (const Piece& w : want) {
      if (!w.bytes) continue;
      pieces[n_pieces] = w;
      pieces[n_pieces++].off = pack_bytes;
      pack_bytes += align16(w.bytes);
    }
    if ((s = ensure_pinned(ctx, &ctx->h_stage, &ctx->stage_cap, pack_bytes, hipHostMallocCoherent))) return s;
    char* pack = nullptr;
    HIP_TRY(hipHostGetDevicePointer(reinterpret_cast<void**>(&pack), ctx->h_stage, 0), "hipHostGetDevicePointer");
    if (io->output) output16 = reinterpret_cast<uint16_t*>(pack + pieces[0].off);
    if (residual) next = reinterpret_cast<uint16_t*>(pack + pieces[io->output ? 1 : 0].off);
  }
  int* n_work = work + 4 * max_work;

  RouteArgs ra{};
  ra.x = x;
  ra.router_w = L->router_w;
  ra.router_b = L->router_b;
  ra.injected = injected;
  ra.norm_w = route_norm_w;
  ra.norm_eps = norm_eps;
  ra.m = (int)m;
  ra.hidden = (int)H;
  ra.experts = (int)E;
  ra.top_k = (int)K;
  ra.logits = logits;
  ra.selected = selected;
  ra.weights = weights;
  ra.act = act1;
  // Quantization work-groups: every quantized projection; the exact-BF16
  // projection reads its input rows directly, or (with the fused RMSNorm)
  // the normalized bf16 rows those work-groups store into act1.
  ra.qmode = proj;
  ra.quant = (proj != GOSSMX_PROJECTION_EXACT_BF16 || residual) ? 1 : 0;
  ra.err = ctx->err;
  DispatchArgs da{};
  da.selected = selected;
  da.routes = (int)R;
  da.top_k = (int)K;
  da.experts = (int)E;
  da.bucket_off = bucket;
  da.route_tok = route_tok;
  da.route_slot = route_slot;
  da.work = work;
  da.n_work = n_work;
  da.chunk = chunk;
  // Small batches with a computed router: router, selection and dispatch in
  // one launch (the route counter is the second int of the flags buffer).
  const bool route_fused = injected == nullptr && fused && m <= (size_t)kFusedRouteRows && H <= (size_t)kFusedRouteHidden;
  // One row (no gate_up / SwiGLU traces): a launch for the logits and the
  // input quantization, then every gate_up work-group selects for itself in
  // the gate_up launch.
  const bool route_gemv = route_fused && m == 1 && E <= (size_t)kRouteGemvExperts && K <= (size_t)kSelectTopK &&
                          proj == GOSSMX_PROJECTION_RESIDUAL_Q8 && use_gemv(m, B1, true) && !trace_gu && !trace_sw;
  begin_call(ctx, m, R, io->memory, arena ? arena->used : context_scratch_bytes(ctx));
  const StageInfo router_stage{GOSSMX_ROLE_ROUTER, GOSSMX_KERNEL_ROUTE, (uint32_t)E, (uint32_t)H, 0};
  if (route_gemv) {
    OpScope sc(ctx, GOSSMX_OP_ROUTER_ROUTING, router_stage);
    HIP_TRY(launch_route_logits(ra, ctx->stream), "router launch");
  } else if (route_fused) {
    OpScope sc(ctx, GOSSMX_OP_ROUTER_ROUTING, router_stage);
    HIP_TRY(launch_route_select(ra, da, ctx->err + 1, ctx->stream), "route/select launch");
  } else if (injected == nullptr) {
    OpScope sc(ctx, GOSSMX_OP_ROUTER_ROUTING, router_stage);
    HIP_TRY(launch_route(ra, ctx->stream), "route launch");
  }
  if (!route_fused) {
    // This stage also holds top-k, softmax and (with injected logits) the
    // gate_up input quantization.
    OpScope sc(ctx, GOSSMX_OP_DISPATCH, {GOSSMX_ROLE_NONE, GOSSMX_KERNEL_ROUTE, 0, (uint32_t)E, 0});
    const int quantize = (injected != nullptr && ra.quant) ? 1 : 0;
    if (fused) {
      HIP_TRY(launch_select_dispatch(ra, da, quantize, ctx->stream), "select/dispatch launch");
    } else {
      HIP_TRY(launch_select_count(ra, quantize, cnt, ctx->stream), "select launch");
      HIP_TRY(launch_place(da, (int)m, cnt, ctx->stream), "grouping launch");
    }
  }
  GemmArgs g{};
  g.w = L->gate_up->t;
  g.fast_ok = ctx->fast_ok ? 1 : 0;
  g.actv = act1.v;
  g.acts = act1.s;
  g.bias = L->gate_up_bias;
  g.bias_expert_stride = 2 * I;
  g.residual = proj == GOSSMX_PROJECTION_RESIDUAL_Q8 ? 1 : 0;
  g.trace_gu = trace_gu;
  g.trace_sw = trace_sw;
  g.xin = residual ? reinterpret_cast<const uint16_t*>(act1.v) : x;
  g.act_next16 = reinterpret_cast<uint16_t*>(act2.v);
  g.work = work;
  g.n_work = n_work;
  g.route_tok = da.route_tok;
  g.route_slot = da.route_slot;
  g.actv_next = act2.v;
  g.acts_next = act2.s;
  g.alpha = L->cfg.alpha;
  g.limit = L->cfg.limit;
  g.sig_tab = ctx->sig_tab;
  g.err = ctx->err;
  GemmArgs d = g;
  d.w = L->down->t;
  d.actv = g.actv_next;
  d.acts = g.acts_next;
  d.bias = L->down_bias;
  d.bias_expert_stride = H;
  d.y = ybuf;
  d.trace_gu = d.trace_sw = nullptr;
  d.xin = g.act_next16;
  // One row with at most four routes (one route per work item): the down
  // projection's work-groups also run the combine.
  const bool down_combine = proj != GOSSMX_PROJECTION_EXACT_BF16 && m == 1 && K <= 4 && use_gemv(m, B2, d.residual != 0);
  const uint32_t n_gu = (uint32_t)(2 * I), n_down = (uint32_t)H;
  if (proj == GOSSMX_PROJECTION_EXACT_BF16) {
    {
      OpScope sc(ctx, GOSSMX_OP_GATE_UP, {GOSSMX_ROLE_GATE_UP, GOSSMX_KERNEL_EXACT, n_gu, (uint32_t)H, 0});
      HIP_TRY(launch_exact(kGateUp, g, (int)max_work, ctx->stream), "exact gate_up launch");
    }
    {
      OpScope sc(ctx, GOSSMX_OP_DOWN, {GOSSMX_ROLE_DOWN, GOSSMX_KERNEL_EXACT, n_down, (uint32_t)I, 0});
      HIP_TRY(launch_exact(kDown, d, (int)max_work, ctx->stream), "exact down launch");
    }
  } else {
    {
      const bool gemv = route_gemv || use_gemv(m, B1, g.residual != 0);
      KernelScope sc(ctx, GOSSMX_OP_GATE_UP,
                     {GOSSMX_ROLE_GATE_UP, gemv ? GOSSMX_KERNEL_GEMV : GOSSMX_KERNEL_GEMM, n_gu, (uint32_t)H,
                      gemv ? 0u : (uint32_t)chunk});
      if (route_gemv)
        HIP_TRY(launch_route_gemv(ra, da, g, ctx->stream, sc.start, sc.stop), "route/gate_up launch");
      else if (use_gemv(m, B1, g.residual != 0))
        HIP_TRY(launch_gemv(kGateUp, g, (int)m, (int)max_work, ctx->stream, sc.start, sc.stop), "gate_up launch");
      else
        HIP_TRY(launch_gemm(kGateUp, g, chunk, (int)max_work, ctx->stream, sc.start, sc.stop), "gate_up launch");
    }
    {
      const bool gemv = down_combine || use_gemv(m, B2, d.residual != 0);
      KernelScope sc(ctx, GOSSMX_OP_DOWN,
                     {GOSSMX_ROLE_DOWN, gemv ? GOSSMX_KERNEL_GEMV : GOSSMX_KERNEL_GEMM, n_down, (uint32_t)I,
                      gemv ? 0u : (uint32_t)chunk});
      if (down_combine)
        HIP_TRY(launch_down_combine(d, weights, (int)K, output, output16, trace, resid, next, unrounded, ctx->stream,
                                    sc.start, sc.stop),
                "down/combine launch");
      else if (use_gemv(m, B2, d.residual != 0))
        HIP_TRY(launch_gemv(kDown, d, (int)m, (int)max_work, ctx->stream, sc.start, sc.stop), "down launch");
      else
        HIP_TRY(launch_gemm(kDown, d, chunk, (int)max_work, ctx->stream, sc.start, sc.stop), "down launch");
    }
  }
  if (!down_combine) {
    OpScope sc(ctx, GOSSMX_OP_WEIGHTING, {GOSSMX_ROLE_NONE, GOSSMX_KERNEL_COMBINE, n_down, (uint32_t)K, 0});
    HIP_TRY(launch_combine(d.y, weights, (int)m, (int)K, (int)H, output, output16, trace, resid, next, unrounded,
                           ctx->stream),
            "combine launch");
  }

  if (host) {
    // One gather into the pinned pack, one synchronization; the caller's
    // buffers are written only when the flags are clear.
    PackArgs pa{};
    pa.err = ctx->err;
    HIP_TRY(hipHostGetDevicePointer(reinterpret_cast<void**>(&pa.dst), ctx->h_stage, 0), "hipHostGetDevicePointer");
    size_t payload = 0;
    for (int i = 0; i < n_pieces; ++i) {
      payload += pieces[i].bytes;
      if (!pieces[i].src) continue;
      pa.src[pa.pieces] = pieces[i].src;
      pa.off[pa.pieces] = pieces[i].off;
      pa.words[pa.pieces++] = pieces[i].bytes / 4;
    }
    count_transfer(kTransferOutput, payload);
    HIP_TRY(launch_pack(pa, ctx->stream), "pack launch");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    const int flags = *reinterpret_cast<const int*>(ctx->h_stage);
    if (flags != 0) return device_flags_fail(ctx, flags);
    for (int i = 0; i < n_pieces; ++i) {
      const Piece& pc = pieces[i];
      if (pc.widen) {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(ctx->h_stage + pc.off);
        uint32_t* dst = static_cast<uint32_t*>(pc.dst);
        for (size_t j = 0; j < pc.bytes / 2; ++j) dst[j] = (uint32_t)src[j] << 16;
      } else {
        std::memcpy(pc.dst, ctx->h_stage + pc.off, pc.bytes);
      }
    }
  } else {
    if (io->selected)
      HIP_TRY(hipMemcpyAsync(io->selected, selected, R * 4, hipMemcpyDeviceToDevice, ctx->stream), "D2D selected");
    if (io->routing_weights)
      HIP_TRY(hipMemcpyAsync(io->routing_weights, weights, R * 4, hipMemcpyDeviceToDevice, ctx->stream), "D2D weights");
    if (io->route_order)
      HIP_TRY(hipMemcpyAsync(io->route_order, da.route_slot, R * 4, hipMemcpyDeviceToDevice, ctx->stream), "D2D order");
  }
  return GOSSMX_OK;
}

int gossmx_moe_forward(gossmx_ctx* ctx, const gossmx_layer* L, const gossmx_moe_io* io) {
  return count_projection(projection_result(ctx, moe_forward_impl(ctx, L, io, nullptr, 0.0f, nullptr)));
}

int gossmx_moe_forward_residual(gossmx_ctx* ctx, const gossmx_layer* L, const gossmx_moe_io* io,
                                const float* norm_weight, float epsilon, uint16_t* next_residual) {
  if (!norm_weight) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  return count_projection(projection_result(ctx, moe_forward_impl(ctx, L, io, norm_weight, epsilon, next_residual)));
}

static int moe_forward_noalloc_impl(gossmx_ctx* ctx, const gossmx_layer* L, const gossmx_moe_io* io) {
  if (!ctx || !L || !io) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (io->memory != GOSSMX_MEM_DEVICE)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "gossmx_moe_forward_noalloc takes device memory only");
  void* base = scratch_address(ctx->device);
  if (!base) return fail(GOSSMX_ERR_DEVICE, "no fixed scratch on device %d (symbol lookup failed)", ctx->device);
  ScratchArena arena;
  arena.base = static_cast<char*>(base);
  arena.cap = kNoAllocScratchBytes;
  // Profiling events are created on demand; a call that must not allocate
  // records none.
  const bool profiling = ctx->profiling;
  ctx->profiling = false;
  const int s = moe_forward_impl(ctx, L, io, nullptr, 0.0f, nullptr, &arena);
  ctx->profiling = profiling;
  return projection_result(ctx, s);
}

int gossmx_moe_forward_noalloc(gossmx_ctx* ctx, const gossmx_layer* L, const gossmx_moe_io* io) {
  return count_projection(moe_forward_noalloc_impl(ctx, L, io));
}

// --- profiling, fault hook, self-test -------------------------------------------

int gossmx_profile_enable(gossmx_ctx* ctx, int enabled) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  ctx->profiling = enabled != 0;
  return GOSSMX_OK;
}

int gossmx_profile_read(gossmx_ctx* ctx, gossmx_profile_record* out, size_t capacity, size_t* written) {
  if (!ctx || !out || !written) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (int s = fold_profile(ctx)) return s;
  size_t n = std::min<size_t>(capacity, GOSSMX_OP_COUNT);
  for (size_t i = 0; i < n; ++i) {
    out[i].op = (int)i;
    out[i].launches = ctx->op_launches[i];
    out[i].total_ms = ctx->op_ms[i];
  }
  *written = n;
  return GOSSMX_OK;
}

int gossmx_profile_reset(gossmx_ctx* ctx) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (int s = fold_profile(ctx)) return s;
  for (int i = 0; i < GOSSMX_OP_COUNT; ++i) {
    ctx->op_ms[i] = 0.0;
    ctx->op_launches[i] = 0;
  }
  ctx->events.clear();
  ctx->events_dropped = 0;
  ctx->events_seq = 0;
  if (ctx->prof_base) ctx->event_pool.push_back(ctx->prof_base);
  ctx->prof_base = nullptr;
  return GOSSMX_OK;
}

int gossmx_profile_tag(gossmx_ctx* ctx, int layer, int phase) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (layer < -1) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "layer tag %d below -1", layer);
  if (phase != GOSSMX_PHASE_UNKNOWN && phase != GOSSMX_PHASE_PREFILL && phase != GOSSMX_PHASE_DECODE)
    return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown phase %d", phase);
  ctx->tag_layer = layer;
  ctx->tag_phase = phase;
  return GOSSMX_OK;
}

int gossmx_profile_events(gossmx_ctx* ctx, gossmx_profile_event* out, size_t capacity, size_t* written,
                          size_t* available, uint64_t* dropped) {
  if (!ctx || !written || (capacity && !out)) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (int s = fold_profile(ctx)) return s;
  const size_t n = std::min(capacity, ctx->events.size());
  if (n) std::memcpy(out, ctx->events.data(), n * sizeof(gossmx_profile_event));
  *written = n;
  if (available) *available = ctx->events.size();
  if (dropped) *dropped = ctx->events_dropped;
  return GOSSMX_OK;
}

int gossmx_stats_read(gossmx_stats* out) {
  if (!out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null output");
  *out = gossmx_stats{};
  out->projections_ok = g_stats.ok.load();
  out->projections_failed = g_stats.failed.load();
  out->projections_refused = g_stats.refused.load();
  out->projections_rejected = g_stats.rejected.load();
  out->weights_bias_uploaded_bytes = g_stats.transfer[kTransferUpload].load();
  out->activation_bytes = g_stats.transfer[kTransferActivation].load();
  out->output_bytes = g_stats.transfer[kTransferOutput].load();
  out->resident_bytes = g_stats.resident.load();
  out->resident_high_water_bytes = g_stats.high_water.load();
  out->resident_cap_bytes = g_stats.cap.load();
  out->capacity_refusals = g_stats.cap_refusals.load();
  out->repack_cache_hits = g_stats.cache_hits.load();
  out->repack_cache_misses = g_stats.cache_misses.load();
  out->circuit_open = g_circuit_open.load() ? 1 : 0;
  return GOSSMX_OK;
}

void gossmx_stats_reset(void) {
  for (std::atomic<uint64_t>* c : {&g_stats.ok, &g_stats.failed, &g_stats.refused, &g_stats.rejected,
                                   &g_stats.transfer[0], &g_stats.transfer[1], &g_stats.transfer[2],
                                   &g_stats.cap_refusals, &g_stats.cache_hits, &g_stats.cache_misses})
    c->store(0);
  g_stats.high_water.store(g_stats.resident.load());
}

int gossmx_set_resident_cap(uint64_t bytes) {
  g_stats.cap.store(bytes);
  return GOSSMX_OK;
}

int gossmx_capture_begin(gossmx_ctx* ctx) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (ctx->capturing) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "already capturing");
  if (int s = set_device(ctx->device)) return s;
  if (int s = fold_profile(ctx)) return s;
  HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  ctx->capturing = true;
  return GOSSMX_OK;
}

int gossmx_capture_end(gossmx_ctx* ctx, gossmx_graph** out) {
  if (!ctx || !out) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (!ctx->capturing) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "not capturing");
  ctx->capturing = false;
  hipGraph_t graph = nullptr;
  HIP_TRY(hipStreamEndCapture(ctx->stream, &graph), "hipStreamEndCapture");
  auto* g = new gossmx_graph();
  g->graph = graph;
  g->device = ctx->device;
  hipError_t e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    gossmx_graph_destroy(g);
    return hip_fail(e, "hipGraphInstantiate");
  }
  g->ctx = ctx;
  ++ctx->live_graphs;
  *out = g;
  return GOSSMX_OK;
}

int gossmx_graph_launch(gossmx_ctx* ctx, const gossmx_graph* g) {
  if (!ctx || !g || !g->exec) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (ctx->capturing) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "cannot launch a graph while capturing");
  if (int s = set_device(ctx->device)) return s;
  HIP_TRY(hipGraphLaunch(g->exec, ctx->stream), "hipGraphLaunch");
  return GOSSMX_OK;
}

void gossmx_graph_destroy(gossmx_graph* g) {
  if (!g) return;
  (void)hipSetDevice(g->device);
  if (g->ctx) (void)hipStreamSynchronize(g->ctx->stream);  // no replay still reads its buffers
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  if (g->ctx && --g->ctx->live_graphs == 0) {
    for (void* p : g->ctx->retired) (void)hipFree(p);
    g->ctx->retired.clear();
  }
  delete g;
}

int gossmx_inject_fault(gossmx_ctx* ctx, int armed) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  if (armed < 0 || armed > 3) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "unknown fault mode %d", armed);
  ctx->fault_armed = armed;
  return GOSSMX_OK;
}

// Checks the lane layouts of the FP4 conversion and the 16x16x32 f16 MFMA on
// this device against what the GEMM assumes, and the device SwiGLU sigmoid
// table against the host expf. *scaled_ok reports whether the scaled
// conversion with dirty scale operands (the GEMM's fast path) gave the exact
// scaled values; the other checks fail the call.
int gossmx_selftest(gossmx_ctx* ctx);
}  // extern "C"

static int run_selftest(gossmx_ctx* ctx, bool* scaled_ok) {
  if (int s = set_device(ctx->device)) return s;
  float* dev = nullptr;
  HIP_TRY(hipMalloc(&dev, kSelftestFloats * sizeof(float)), "hipMalloc(selftest)");
  std::vector<float> host(kSelftestFloats);
  hipError_t e = launch_selftest(dev, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(host.data(), dev, kSelftestFloats * sizeof(float), hipMemcpyDeviceToHost,
                                          ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (e != hipSuccess) return hip_fail(e, "selftest");
  const float codes[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                           -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
  for (int i = 0; i < 8; ++i)
    if (host[i] != codes[i])
      return fail(GOSSMX_ERR_UNSUPPORTED, "fp4 conversion element %d is %g, expected %g", i, host[i], codes[i]);
  for (int i = 0; i < 8; ++i)
    if (host[264 + i] != codes[i] * 0.0625f)
      return fail(GOSSMX_ERR_UNSUPPORTED, "scaled fp4 conversion element %d is %g, expected %g", i, host[264 + i],
                  codes[i] * 0.0625f);
  for (int lane = 0; lane < 64; ++lane)
    for (int r = 0; r < 4; ++r) {
      const float want = (float)(10 * (4 * (lane / 16) + r) + lane % 16);
      if (host[8 + 4 * lane + r] != want)
        return fail(GOSSMX_ERR_UNSUPPORTED, "mfma lane %d reg %d is %g, expected %g", lane, r, host[8 + 4 * lane + r],
                    want);
    }
  // Dirty scale operands (selftest_kernel): every result must be the code's
  // value times 2^(e - 127), with the sign of -0.0 codes kept.
  const uint32_t dirty_exp[5] = {114, 120, 127, 133, 139};
  *scaled_ok = true;
  for (int c = 0; c < kSelftestDirty && *scaled_ok; ++c) {
    const float scale = std::ldexp(1.0f, (int)dirty_exp[c / 24] - 127);
    for (int i = 0; i < 16; ++i) {
      const float want = codes[i] * scale, got = host[272 + 16 * c + i];
      if (std::memcmp(&want, &got, 4) != 0) {
        *scaled_ok = false;
        fail(GOSSMX_ERR_UNSUPPORTED,
             "scaled fp4 conversion with a dirty scale operand (exponent %u, byte %d, case %d) gave %g for code %d, "
             "expected %g",
             dirty_exp[c / 24], (c / 6) % 4, c, got, i, want);
        break;
      }
    }
  }
  // The device's f32 -> bf16 conversion against half's rounding.
  for (int k = 0; k < kSelftestBf16; ++k) {
    const uint32_t x = selftest_bf16_input(k);
    uint16_t want;
    if ((x & 0x7fffffffu) > 0x7f800000u) want = (uint16_t)((x >> 16) | 0x40u);
    else if ((x & 0x8000u) && (x & 0x17fffu)) want = (uint16_t)((x >> 16) + 1u);
    else want = (uint16_t)(x >> 16);
    if (host[kSelftestBf16Base + k] != (float)want)
      return fail(GOSSMX_ERR_UNSUPPORTED, "bf16 conversion of %#010x gave %#06x, expected %#06x", x,
                  (unsigned)host[kSelftestBf16Base + k], want);
  }
  // The device SwiGLU sigmoid table against the host libm expf on all 65,536
  // bf16 inputs (the reference's f32::exp is the host expf).
  std::vector<uint16_t> tab(65536);
  HIP_TRY(hipMemcpyAsync(tab.data(), ctx->sig_tab, 65536 * sizeof(uint16_t), hipMemcpyDeviceToHost, ctx->stream),
          "D2H sigmoid table");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  for (uint32_t i = 0; i < 65536u; ++i) {
    uint32_t xb = i << 16;
    float x;
    std::memcpy(&x, &xb, 4);
    const float y = 1.0f / (1.0f + expf(-x));
    uint32_t yb;
    std::memcpy(&yb, &y, 4);
    uint16_t want;
    if ((yb & 0x7fffffffu) > 0x7f800000u) want = (uint16_t)((yb >> 16) | 0x40u);
    else if ((yb & 0x8000u) && (yb & 0x17fffu)) want = (uint16_t)((yb >> 16) + 1u);
    else want = (uint16_t)(yb >> 16);
    if (tab[i] != want)
      return fail(GOSSMX_ERR_UNSUPPORTED, "sigmoid table entry %#06x is %#06x, host expf gives %#06x", i, tab[i], want);
  }
  return GOSSMX_OK;
}

extern "C" {

int gossmx_selftest(gossmx_ctx* ctx) {
  if (!ctx) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null context");
  const std::string prior = g_last_error;
  bool scaled_ok = true;
  if (int s = run_selftest(ctx, &scaled_ok)) return s;
  if (!scaled_ok) return GOSSMX_ERR_UNSUPPORTED;  // message set by run_selftest
  g_last_error = prior;
  return GOSSMX_OK;
}

int gossmx_selftest_bf16_exhaustive(gossmx_ctx* ctx, uint64_t* mismatches) {
  if (!ctx || !mismatches) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (int s = set_device(ctx->device)) return s;
  unsigned long long* dev = nullptr;
  HIP_TRY(hipMalloc(&dev, sizeof(unsigned long long)), "hipMalloc(bf16 check)");
  unsigned long long n = 0;
  hipError_t e = hipMemcpyAsync(dev, &n, sizeof n, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = launch_bf16_exhaustive(dev, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(&n, dev, sizeof n, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (e != hipSuccess) return hip_fail(e, "bf16 check");
  *mismatches = n;
  return GOSSMX_OK;
}

int gossmx_ctx_fast_path(const gossmx_ctx* ctx, int* enabled) {
  if (!ctx || !enabled) return fail(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  *enabled = ctx->fast_ok ? 1 : 0;
  return GOSSMX_OK;
}

}  // extern "C"
