// The dense path around the MoE block: the rest of a GPT-OSS decoder step as
// CpuModel::prepare_step runs it (crates/gpt-oss-model-runner/src/
// cpu_runner.rs:2103-2333, forward_layer_batch :2335-2586). Norms, RoPE,
// attention and the KV cache run on the host; the projections and each
// layer's MoE half (post-attention RMSNorm, moe_batch, residual add, through
// gossmx_moe_forward_residual) on the GPU.
//
// - bf16 projections: Kernels::bf16_matvec (gpt-oss-cpu-kernels lib.rs:314-341)
//   with its 16 fixed reduction lanes, multiply then add, lanes folded 0..15
//   (scalar_bf16_dot lib.rs:1007-1029), then += bias (project_bf16[_batch]
//   cpu_runner.rs:2689-2792): dense_proj_kernel, over copies of the Q/K/V/O
//   weights and lm_head made in HBM when the model is created.
// - RMSNorm boundaries: norm_boundary (:2680-2687) over Kernels::rms_norm
//   (lib.rs:699-730, the same 16-lane sum of squares).
// - YaRN RoPE (YarnRope :3927-4013) with its bf16 boundaries.
// - Attention with learned sinks over the visible KV window
//   (attention_one_staged :3840-3924), and the KV cache of CpuKvCache
//   (:653-740): a sliding layer keeps sliding_window tokens, a full layer
//   context_cap. A step's rows are staged and committed to the caches only
//   when the whole step succeeded (PreparedCpuStep::commit, :1081-1113).
// - Residual adds (add_residual :3732-3738), the final norm, lm_head and its
//   bf16 round trip with the finiteness check (:2255-2312).
// expf, powf, cosf, sinf and log are the host C library's: the functions
// Rust's f32/f64 methods call on x86_64 Linux.

#include "../../include/gossmx.h"
#include "gossmx_internal.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

namespace {

int err(int status, const char* message) { return gossmx::set_error(status, message); }

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
// bf16::from_f32 of half 2.7.1: round to nearest even, NaN quieted.
inline uint16_t bf16_bits(float f) {
  const uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  const uint32_t round_bit = 0x8000u;
  const uint32_t up = ((u & round_bit) != 0 && (u & (3 * round_bit - 1)) != 0) ? 1u : 0u;
  return (uint16_t)((u >> 16) + up);
}
inline float bf16_f32(uint16_t b) { return u2f((uint32_t)b << 16); }
inline float bf16_round(float f) { return bf16_f32(bf16_bits(f)); }

// ---------------------------------------------------------------------------
// Worker pool: run(n, fn) calls fn(i) for every i < n on the pool's threads
// and the caller's, and returns when all calls have returned.

class Pool {
 public:
  explicit Pool(size_t threads) {
    for (size_t i = 1; i < threads; ++i) workers_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(m_);
      stop_ = true;
      ++generation_;
    }
    wake_.notify_all();
    for (auto& t : workers_) t.join();
  }
  size_t size() const { return workers_.size() + 1; }
  void run(size_t n, const std::function<void(size_t)>& fn) {
    if (workers_.empty() || n <= 1) {
      for (size_t i = 0; i < n; ++i) fn(i);
      return;
    }
    {
      std::lock_guard<std::mutex> g(m_);
      fn_ = &fn;
      n_ = n;
      next_.store(0);
      pending_ = workers_.size();
      ++generation_;
    }
    wake_.notify_all();
    work();
    std::unique_lock<std::mutex> l(m_);
    done_.wait(l, [this] { return pending_ == 0; });
  }

 private:
  void work() {
    for (size_t i; (i = next_.fetch_add(1)) < n_;) (*fn_)(i);
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> l(m_);
        wake_.wait(l, [&] { return generation_ != seen; });
        seen = generation_;
        if (stop_) return;
      }
      work();
      std::lock_guard<std::mutex> g(m_);
      if (--pending_ == 0) done_.notify_one();
    }
  }
  std::vector<std::thread> workers_;
  std::mutex m_;
  std::condition_variable wake_, done_;
  const std::function<void(size_t)>* fn_ = nullptr;
  size_t n_ = 0, pending_ = 0;
  std::atomic<size_t> next_{0};
  uint64_t generation_ = 0;
  bool stop_ = false;
};

// norm_boundary: bf16 -> f32, rms_norm, -> bf16.
void norm_boundary(const uint16_t* x, const float* w, size_t n, float eps, uint16_t* out) {
  float lanes[16] = {0};
  size_t i = 0;
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 16; ++l) {
      const float v = bf16_f32(x[i + l]);
      lanes[l] += v * v;
    }
  for (size_t l = 0; i < n; ++i, ++l) {
    const float v = bf16_f32(x[i]);
    lanes[l] += v * v;
  }
  float ss = 0.0f;
  for (int l = 0; l < 16; ++l) ss += lanes[l];
  const float inv = 1.0f / std::sqrt(ss / (float)n + eps);
  for (size_t k = 0; k < n; ++k) out[k] = bf16_bits(bf16_f32(x[k]) * inv * w[k]);
}

// ---------------------------------------------------------------------------
// YaRN RoPE (YarnRope::new / apply, cpu_runner.rs:3933-4013).

struct Rope {
  std::vector<float> inv_freq;
  float attention_scale = 1.0f;
  size_t head_dim = 0;
};

Rope make_rope(const gossmx_model_config& c) {
  Rope r;
  const size_t dim = c.head_dim;
  r.head_dim = dim;
  const float theta = (float)c.rope_theta;
  if (!c.rope_yarn) {
    for (size_t i = 0; i < dim; i += 2) r.inv_freq.push_back(1.0f / powf(theta, (float)i / (float)dim));
    return r;
  }
  const double two_pi = 6.283185307179586;
  auto correction = [&](double rotations) {
    return ((double)dim * std::log((double)c.rope_original_max_positions / (rotations * two_pi))) /
           (2.0 * std::log(c.rope_theta));
  };
  double low = correction(c.rope_beta_fast), high = correction(c.rope_beta_slow);
  if (c.rope_truncate) {
    low = std::floor(low);
    high = std::ceil(high);
  }
  low = std::max(low, 0.0);
  high = std::min(high, (double)(dim - 1));
  const double range = std::max(std::fabs(high - low), 0.001);
  for (size_t i = 0; i < dim / 2; ++i) {
    const float frequency = powf(theta, (float)(i * 2) / (float)dim);
    const float extrapolation = 1.0f / frequency;
    const float interpolation = 1.0f / ((float)c.rope_factor * frequency);
    float ramp = ((float)i - (float)low) / (float)range;
    ramp = std::min(std::max(ramp, 0.0f), 1.0f);
    r.inv_freq.push_back(interpolation * ramp + extrapolation * (1.0f - ramp));
  }
  r.attention_scale = (float)(0.1 * std::log(c.rope_factor) + 1.0);
  return r;
}

// The bf16 cosine and sine of a position depend on (position, i) only: they
// are computed once per call and shared by every head.
void rope_apply(const Rope& r, float* v, size_t heads, size_t position) {
  const size_t half = r.head_dim / 2;
  thread_local std::vector<float> table;
  table.resize(2 * half);
  for (size_t i = 0; i < half; ++i) {
    const float angle = (float)position * r.inv_freq[i];
    table[i] = bf16_round(cosf(angle) * r.attention_scale);
    table[half + i] = bf16_round(sinf(angle) * r.attention_scale);
  }
  for (size_t h = 0; h < heads; ++h) {
    float* p = v + h * r.head_dim;
    for (size_t i = 0; i < half; ++i) {
      const float cosine = table[i], sine = table[half + i];
      const float left = bf16_round(p[i]), right = bf16_round(p[half + i]);
      const float left_cosine = bf16_round(left * cosine), right_sine = bf16_round(right * sine);
      const float right_cosine = bf16_round(right * cosine), left_sine = bf16_round(left * sine);
      p[i] = bf16_round(left_cosine - right_sine);
      p[half + i] = bf16_round(right_cosine + left_sine);
    }
  }
}

// ---------------------------------------------------------------------------
// Attention for one query over `tokens` visible key/value rows, oldest first
// (attention_one_staged): bf16 QK dot, bf16 scale, softmax with the sink in
// the denominator, bf16 probabilities, f32 accumulation, bf16 output.
// key(t) / value(t) return the row of visible token t (all kv heads). Heads
// are independent: this computes heads [h_begin, h_end) of out.

template <class KeyRow, class ValueRow>
void attention(const float* q_all, size_t tokens, const KeyRow& key, const ValueRow& value, const float* sinks,
               size_t heads, size_t kv_heads, size_t head_dim, float* out, std::vector<float>& scores,
               size_t h_begin, size_t h_end) {
  const size_t groups = heads / kv_heads;
  const float scale = 1.0f / std::sqrt((float)head_dim);
  scores.resize(tokens);
  for (size_t h = h_begin; h < h_end; ++h) {
    const float* q = q_all + h * head_dim;
    const size_t kvh = h / groups;
    for (size_t t = 0; t < tokens; ++t) {
      const uint16_t* k = key(t) + kvh * head_dim;
      float dot = 0.0f;
      for (size_t d = 0; d < head_dim; ++d) dot += q[d] * bf16_f32(k[d]);
      dot = bf16_round(dot);
      scores[t] = bf16_round(dot * scale);
    }
    float maximum = sinks[h];
    for (size_t t = 0; t < tokens; ++t) maximum = std::fmax(maximum, scores[t]);
    float sum = 0.0f;
    for (size_t t = 0; t < tokens; ++t) sum += expf(scores[t] - maximum);
    const float denominator = expf(sinks[h] - maximum) + sum;
    float* o = out + h * head_dim;
    for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
    for (size_t t = 0; t < tokens; ++t) {
      const float p = bf16_round(expf(scores[t] - maximum) / denominator);
      const uint16_t* v = value(t) + kvh * head_dim;
      for (size_t d = 0; d < head_dim; ++d) o[d] += p * bf16_f32(v[d]);
    }
    for (size_t d = 0; d < head_dim; ++d) o[d] = bf16_round(o[d]);
  }
}

// Committed KV rows of one layer (CpuKvCache): the last min(positions, capacity)
// tokens, position p in slot p % capacity.
struct KvCache {
  size_t capacity = 0, width = 0, len = 0, start = 0;
  std::vector<uint16_t> k, v;
  const uint16_t* key(size_t p) const { return k.data() + (p % capacity) * width; }
  const uint16_t* value(size_t p) const { return v.data() + (p % capacity) * width; }
  void append(size_t p, const uint16_t* key_row, const uint16_t* value_row) {
    const size_t slots = std::min(p + 1, capacity);
    if (k.size() < slots * width) {
      k.resize(std::min(capacity, std::max(slots, 2 * k.size() / std::max<size_t>(width, 1))) * width);
      v.resize(k.size());
    }
    std::memcpy(k.data() + (p % capacity) * width, key_row, width * 2);
    std::memcpy(v.data() + (p % capacity) * width, value_row, width * 2);
    if (len == capacity) ++start;
    else ++len;
    if (len == 1) start = p;
  }
};

double seconds_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

int check_config(const gossmx_model_config* c) {
  if (!c) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null model config");
  if (!c->vocab || !c->hidden || !c->layers || !c->heads || !c->kv_heads || !c->head_dim || c->head_dim % 2 ||
      c->heads % c->kv_heads || !c->sliding_window || !c->context_cap)
    return err(GOSSMX_ERR_INVALID_DIMENSIONS,
               "model config needs non-zero sizes, an even head_dim and heads divisible by kv_heads");
  if (c->rope_yarn && (c->rope_factor <= 0.0 || !c->rope_original_max_positions))
    return err(GOSSMX_ERR_INVALID_DIMENSIONS, "YaRN scaling needs a positive factor and original positions");
  return GOSSMX_OK;
}

}  // namespace

// The model's device side: the projection weights and lm_head copied to HBM,
// and grow-only f32 staging for the projections' inputs and outputs (device
// buffers, and pinned host buffers for the copies).
struct DenseDevice {
  struct Layer {
    const uint16_t *q, *k, *v, *o;
    const float *qb, *kb, *vb, *ob;
    const float* post_norm;  // post_attention_norm, for the MoE call in device memory
  };
  int device = 0;
  std::vector<void*> weights;  // device allocations of the copies
  std::vector<Layer> layers;
  const uint16_t* lm_head = nullptr;
  float *d_in = nullptr, *d_out = nullptr, *h_in = nullptr, *h_out = nullptr;
  size_t in_cap = 0, out_cap = 0;  // floats
  // The residual rows around the MoE call: device hidden, after and next
  // (m x hidden bf16 each) and their pinned staging, as floats' worth of bytes.
  float *d_rows = nullptr, *h_rows = nullptr;
  size_t rows_cap = 0;
  ~DenseDevice() {
    (void)hipSetDevice(device);
    for (void* p : weights) (void)hipFree(p);
    (void)hipFree(d_in);
    (void)hipFree(d_out);
    (void)hipFree(d_rows);
    (void)hipHostFree(h_in);
    (void)hipHostFree(h_out);
    (void)hipHostFree(h_rows);
  }
};

struct gossmx_model {
  gossmx_ctx* ctx = nullptr;
  gossmx_model_config cfg{};
  const uint16_t* embedding = nullptr;
  const float* final_norm = nullptr;
  const uint16_t* lm_head = nullptr;
  std::vector<gossmx_dense_layer> layers;
  Rope rope;
  std::vector<KvCache> caches;
  size_t position = 0;
  std::unique_ptr<Pool> pool;
  DenseDevice dev;
  double dense_seconds = 0.0, moe_seconds = 0.0;
};

namespace {

int hip_err(hipError_t e, const char* what) {
  char msg[256];
  std::snprintf(msg, sizeof msg, "%s: %s", what, hipGetErrorString(e));
  return err(e == hipErrorOutOfMemory ? GOSSMX_ERR_OUT_OF_MEMORY : GOSSMX_ERR_DEVICE, msg);
}

#define DENSE_HIP(expr, what)                        \
  do {                                               \
    const hipError_t e_ = (expr);                    \
    if (e_ != hipSuccess) return hip_err(e_, what);  \
  } while (0)

// A copy of n elements of T in device memory, owned by the model.
template <class T>
int upload(DenseDevice& D, const T* src, size_t n, const T** dst) {
  void* p = nullptr;
  DENSE_HIP(hipMalloc(&p, n * sizeof(T)), "model weights allocation");
  D.weights.push_back(p);
  gossmx::count_transfer(gossmx::kTransferUpload, n * sizeof(T));
  DENSE_HIP(hipMemcpy(p, src, n * sizeof(T), hipMemcpyHostToDevice), "model weights upload");
  *dst = static_cast<const T*>(p);
  return GOSSMX_OK;
}

int grow(float** dev, float** host, size_t* cap, size_t n) {
  if (n <= *cap) return GOSSMX_OK;
  (void)hipFree(*dev);
  (void)hipHostFree(*host);
  *dev = *host = nullptr;
  *cap = 0;
  DENSE_HIP(hipMalloc(dev, n * sizeof(float)), "projection buffer");
  DENSE_HIP(hipHostMalloc(host, n * sizeof(float)), "projection staging");
  *cap = n;
  return GOSSMX_OK;
}

// One projection of the rows `in` (m x cols bf16) by w ([rows][cols] bf16 in
// HBM) + bias, into out (m x rows f32, host).
struct Projection {
  const uint16_t* w;
  const float* bias;
  size_t rows;
  float* out;
};

// Runs the projections of one input on the GPU (project_bf16_batch): one copy
// in, one launch each, one copy out, one synchronization.
int gpu_project_impl(gossmx_model* M, const uint16_t* in, size_t m, size_t cols, const Projection* p,
                     size_t count) {
  DenseDevice& D = M->dev;
  // The context's stream is read on every call: gossmx_ctx_set_stream may
  // have replaced it since the model was created.
  const hipStream_t stream = gossmx::context_stream(M->ctx);
  size_t total = 0;
  for (size_t i = 0; i < count; ++i) total += m * p[i].rows;
  DENSE_HIP(hipSetDevice(D.device), "hipSetDevice");
  if (int st = grow(&D.d_in, &D.h_in, &D.in_cap, m * cols)) return st;
  if (int st = grow(&D.d_out, &D.h_out, &D.out_cap, total)) return st;
  for (size_t i = 0; i < m * cols; ++i) D.h_in[i] = bf16_f32(in[i]);
  gossmx::count_transfer(gossmx::kTransferActivation, m * cols * sizeof(float));
  DENSE_HIP(hipMemcpyAsync(D.d_in, D.h_in, m * cols * sizeof(float), hipMemcpyHostToDevice, stream),
            "projection input copy");
  // One launch per group. One token through small matrices (Q/K/V, O):
  // work-groups stage their whole K range at once; lm_head and batches: the
  // K-chunked kernel.
  if (count > 3) return err(GOSSMX_ERR_INVALID_ARGUMENT, "internal: more than three projections in a group");
  gossmx::DenseSet set{};
  size_t off = 0;
  for (size_t i = 0; i < count; ++i) {
    set.w[i] = p[i].w;
    set.bias[i] = p[i].bias;
    set.out[i] = D.d_out + off;
    set.rows[i] = (int)p[i].rows;
    off += m * p[i].rows;
  }
  const bool whole_k = m == 1 && cols % 8 == 0 && cols <= 4096 && total <= 65536;
  DENSE_HIP(whole_k ? gossmx::launch_dense_gemv(set, (int)count, D.d_in, (int)cols, stream)
                    : gossmx::launch_dense_proj(set, (int)count, D.d_in, (int)cols, (int)m, stream),
            "projection launch");
  gossmx::count_transfer(gossmx::kTransferOutput, total * sizeof(float));
  DENSE_HIP(hipMemcpyAsync(D.h_out, D.d_out, total * sizeof(float), hipMemcpyDeviceToHost, stream),
            "projection output copy");
  DENSE_HIP(hipStreamSynchronize(stream), "projection");
  off = 0;
  for (size_t i = 0; i < count; ++i) {
    std::memcpy(p[i].out, D.h_out + off, m * p[i].rows * sizeof(float));
    off += m * p[i].rows;
  }
  return GOSSMX_OK;
}

// A run-time failure of the round trip (HIP error, out of memory) opens the
// circuit breaker, as a failed projection call does.
int gpu_project(gossmx_model* M, const uint16_t* in, size_t m, size_t cols, const Projection* p, size_t count) {
  return gossmx::run_time_result(M->ctx, gpu_project_impl(M, in, m, cols, p, count));
}

// The rest of a layer after attention, in one round trip: the O projection of
// attn (m x QW bf16), the residual add with hidden, and the MoE half
// (post-attention norm, block, residual add) in device memory; hidden
// (m x H bf16) becomes the next layer's rows. The MoE time is added to *moe.
int gpu_o_residual_moe_impl(gossmx_model* M, const gossmx_dense_layer& L, const DenseDevice::Layer& DL,
                            const uint16_t* attn, size_t m, uint16_t* hidden, double* moe) {
  DenseDevice& D = M->dev;
  const hipStream_t stream = gossmx::context_stream(M->ctx);
  const size_t H = M->cfg.hidden, QW = M->cfg.heads * M->cfg.head_dim, n = m * H;
  DENSE_HIP(hipSetDevice(D.device), "hipSetDevice");
  if (int st = grow(&D.d_in, &D.h_in, &D.in_cap, m * QW)) return st;
  if (int st = grow(&D.d_out, &D.h_out, &D.out_cap, n)) return st;
  if (int st = grow(&D.d_rows, &D.h_rows, &D.rows_cap, (3 * n + 1) / 2)) return st;
  uint16_t* d_hidden = reinterpret_cast<uint16_t*>(D.d_rows);
  uint16_t *d_after = d_hidden + n, *d_next = d_hidden + 2 * n;
  uint16_t* h_rows = reinterpret_cast<uint16_t*>(D.h_rows);
  for (size_t i = 0; i < m * QW; ++i) D.h_in[i] = bf16_f32(attn[i]);
  std::memcpy(h_rows, hidden, n * 2);
  gossmx::count_transfer(gossmx::kTransferActivation, m * QW * sizeof(float) + n * 2);
  DENSE_HIP(hipMemcpyAsync(D.d_in, D.h_in, m * QW * sizeof(float), hipMemcpyHostToDevice, stream),
            "projection input copy");
  DENSE_HIP(hipMemcpyAsync(d_hidden, h_rows, n * 2, hipMemcpyHostToDevice, stream), "residual rows copy");
  gossmx::DenseSet set{};
  set.w[0] = DL.o;
  set.bias[0] = DL.ob;
  set.out[0] = D.d_out;
  set.rows[0] = (int)H;
  const bool whole_k = m == 1 && QW % 8 == 0 && QW <= 4096;
  DENSE_HIP(whole_k ? gossmx::launch_dense_gemv(set, 1, D.d_in, (int)QW, stream)
                    : gossmx::launch_dense_proj(set, 1, D.d_in, (int)QW, (int)m, stream),
            "projection launch");
  DENSE_HIP(gossmx::launch_residual_add(d_hidden, D.d_out, d_after, n, stream), "residual add launch");
  const auto t_moe = std::chrono::steady_clock::now();
  gossmx_moe_io io{};
  io.x = d_after;
  io.m = m;
  io.memory = GOSSMX_MEM_DEVICE;
  int st = gossmx_moe_forward_residual(M->ctx, L.moe, &io, DL.post_norm, M->cfg.rms_norm_eps, d_next);
  (void)gossmx_profile_tag(M->ctx, -1, GOSSMX_PHASE_UNKNOWN);
  if (st == GOSSMX_OK) {
    // gossmx_synchronize reports the device error flags.
    gossmx::count_transfer(gossmx::kTransferOutput, n * 2);
    const hipError_t e = hipMemcpyAsync(h_rows + n, d_next, n * 2, hipMemcpyDeviceToHost, stream);
    st = e == hipSuccess ? gossmx_synchronize(M->ctx) : hip_err(e, "next rows copy");
  }
  *moe += seconds_since(t_moe);
  if (st != GOSSMX_OK) {
    (void)hipStreamSynchronize(stream);  // the staging buffers' copies end before the next step reuses them
    return st;
  }
  std::memcpy(hidden, h_rows + n, n * 2);
  return GOSSMX_OK;
}

int gpu_o_residual_moe(gossmx_model* M, const gossmx_dense_layer& L, const DenseDevice::Layer& DL,
                       const uint16_t* attn, size_t m, uint16_t* hidden, double* moe) {
  return gossmx::run_time_result(M->ctx, gpu_o_residual_moe_impl(M, L, DL, attn, m, hidden, moe));
}

// One layer-major step over m rows at positions model->position + r
// (prepare_step with every row in one sequence). Writes the last row's logits.
// The caches change only when the step succeeds.
int run_step(gossmx_model* M, const uint32_t* tokens, size_t m, float* logits) {
  const gossmx_model_config& c = M->cfg;
  const size_t H = c.hidden, QW = c.heads * c.head_dim, KW = c.kv_heads * c.head_dim;
  for (size_t r = 0; r < m; ++r)
    if (tokens[r] >= c.vocab) return err(GOSSMX_ERR_INVALID_ARGUMENT, "token id is not below vocab");
  if (M->position + m > c.context_cap)
    return err(GOSSMX_ERR_INVALID_DIMENSIONS, "the step would pass the sequence's context cap");
  const auto t_step = std::chrono::steady_clock::now();
  double moe = 0.0;
  const size_t base = M->position;
  std::vector<uint16_t> hidden(m * H), normalized(m * H), attn(m * QW);
  std::vector<float> q(m * QW), k(m * KW), v(m * KW), attn_f(m * QW), scores;
  std::vector<uint16_t> staged_k(c.layers * m * KW), staged_v(c.layers * m * KW);
  for (size_t r = 0; r < m; ++r) std::memcpy(&hidden[r * H], M->embedding + (size_t)tokens[r] * H, H * 2);
  Pool& pool = *M->pool;
  for (size_t li = 0; li < c.layers; ++li) {
    const gossmx_dense_layer& L = M->layers[li];
    const DenseDevice::Layer& DL = M->dev.layers[li];
    const KvCache& cache = M->caches[li];
    pool.run(m, [&](size_t r) { norm_boundary(&hidden[r * H], L.input_norm, H, c.rms_norm_eps, &normalized[r * H]); });
    const Projection qkv[3] = {{DL.q, DL.qb, QW, q.data()}, {DL.k, DL.kb, KW, k.data()}, {DL.v, DL.vb, KW, v.data()}};
    if (int st = gpu_project(M, normalized.data(), m, H, qkv, 3)) return st;
    uint16_t* sk = &staged_k[li * m * KW];
    uint16_t* sv = &staged_v[li * m * KW];
    // Rows are independent once staged: row r attends to the committed rows and
    // the staged rows 0..r of this step.
    pool.run(m, [&](size_t r) {
      float* qr = &q[r * QW];
      float* kr = &k[r * KW];
      for (size_t i = 0; i < QW; ++i) qr[i] = bf16_round(qr[i]);
      for (size_t i = 0; i < KW; ++i) kr[i] = bf16_round(kr[i]);
      rope_apply(M->rope, qr, c.heads, base + r);
      rope_apply(M->rope, kr, c.kv_heads, base + r);
      for (size_t i = 0; i < KW; ++i) {
        sk[r * KW + i] = bf16_bits(kr[i]);
        sv[r * KW + i] = bf16_bits(v[r * KW + i]);
      }
    });
    // Tasks of (row, block of heads): a one-row step still spreads over the
    // pool.
    const size_t head_blocks = std::min<size_t>(c.heads, m >= 16 ? 1 : (32 + m - 1) / m);
    const size_t per_block = (c.heads + head_blocks - 1) / head_blocks;
    pool.run(m * head_blocks, [&](size_t task) {
      thread_local std::vector<float> sc;
      const size_t r = task / head_blocks, hb = task % head_blocks;
      const size_t h_begin = hb * per_block, h_end = std::min(c.heads, h_begin + per_block);
      if (h_begin >= h_end) return;
      // Positions below `base` are committed (slot p % capacity of the ring),
      // the others are this step's staged rows.
      const size_t combined = cache.len + r + 1;
      const size_t visible = std::min(combined, cache.capacity);
      const size_t first = base + r + 1 - visible, cap = cache.capacity;
      const uint16_t* ck = cache.k.data();
      const uint16_t* cv = cache.v.data();
      const uint16_t* rk = sk;
      const uint16_t* rv = sv;
      auto key = [=](size_t t) -> const uint16_t* {
        const size_t p = first + t;
        return p < base ? ck + (p % cap) * KW : rk + (p - base) * KW;
      };
      auto value = [=](size_t t) -> const uint16_t* {
        const size_t p = first + t;
        return p < base ? cv + (p % cap) * KW : rv + (p - base) * KW;
      };
      float* ctx = &attn_f[r * QW];
      attention(&q[r * QW], visible, key, value, L.sinks, c.heads, c.kv_heads, c.head_dim, ctx, sc, h_begin, h_end);
      for (size_t i = h_begin * c.head_dim; i < h_end * c.head_dim; ++i) attn[r * QW + i] = bf16_bits(ctx[i]);
    });
    // O projection, residual add and the MoE half (norm_boundary(after,
    // post_attention_norm), moe_batch, add_residual) -> the next layer's rows.
    // The MoE block's profile records carry the layer and the phase.
    (void)gossmx_profile_tag(M->ctx, (int)li, base == 0 || m > 1 ? GOSSMX_PHASE_PREFILL : GOSSMX_PHASE_DECODE);
    const int st = gpu_o_residual_moe(M, L, DL, attn.data(), m, hidden.data(), &moe);
    if (st != GOSSMX_OK) return st;
  }
  // Final norm and lm_head for the last row (the only row whose logits are required).
  std::vector<uint16_t> fin(H);
  norm_boundary(&hidden[(m - 1) * H], M->final_norm, H, c.rms_norm_eps, fin.data());
  const Projection head = {M->dev.lm_head, nullptr, c.vocab, logits};
  if (int st = gpu_project(M, fin.data(), 1, H, &head, 1)) return st;
  bool finite = true;
  for (size_t i = 0; i < c.vocab; ++i) {
    logits[i] = bf16_round(logits[i]);
    finite = finite && std::isfinite(logits[i]);
  }
  if (!finite) return err(GOSSMX_ERR_NON_FINITE_LOGITS, "CPU model produced non-finite logits");
  // Commit the staged rows.
  for (size_t li = 0; li < c.layers; ++li)
    for (size_t r = 0; r < m; ++r)
      M->caches[li].append(base + r, &staged_k[(li * m + r) * KW], &staged_v[(li * m + r) * KW]);
  M->position = base + m;
  M->moe_seconds += moe;
  M->dense_seconds += seconds_since(t_step) - moe;
  return GOSSMX_OK;
}

void reset_caches(gossmx_model* M) {
  const size_t KW = M->cfg.kv_heads * M->cfg.head_dim;
  M->caches.assign(M->cfg.layers, KvCache{});
  for (size_t li = 0; li < M->cfg.layers; ++li) {
    KvCache& kv = M->caches[li];
    kv.capacity = M->layers[li].sliding ? M->cfg.sliding_window : M->cfg.context_cap;
    kv.width = KW;
  }
  M->position = 0;
}

}  // namespace

extern "C" {

int gossmx_model_create(gossmx_ctx* ctx, const gossmx_model_config* config, const uint16_t* embedding,
                        const float* final_norm, const uint16_t* lm_head, const gossmx_dense_layer* layers,
                        gossmx_model** out) {
  if (!ctx || !embedding || !final_norm || !lm_head || !layers || !out)
    return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  if (int st = check_config(config)) return st;
  for (size_t li = 0; li < config->layers; ++li) {
    const gossmx_dense_layer& L = layers[li];
    if (!L.input_norm || !L.q_weight || !L.q_bias || !L.k_weight || !L.k_bias || !L.v_weight || !L.v_bias ||
        !L.o_weight || !L.o_bias || !L.sinks || !L.post_attention_norm || !L.moe)
      return err(GOSSMX_ERR_INVALID_ARGUMENT, "null layer tensor");
    const gossmx_moe_config* mc = gossmx::layer_config(L.moe);
    if (mc->hidden != config->hidden)
      return err(GOSSMX_ERR_INVALID_DIMENSIONS, "MoE layer hidden size differs from the model's");
  }
  gossmx_model* M = new (std::nothrow) gossmx_model;
  if (!M) return err(GOSSMX_ERR_OUT_OF_MEMORY, "model allocation failed");
  M->ctx = ctx;
  M->cfg = *config;
  M->embedding = embedding;
  M->final_norm = final_norm;
  M->lm_head = lm_head;
  M->layers.assign(layers, layers + config->layers);
  M->rope = make_rope(*config);
  size_t threads = config->threads;
  if (!threads) threads = std::max(1u, std::thread::hardware_concurrency());
  M->pool.reset(new Pool(std::min<size_t>(threads, 64)));
  reset_caches(M);
  // The projection weights and lm_head go to the context's GPU.
  const size_t H = config->hidden, QW = config->heads * config->head_dim, KW = config->kv_heads * config->head_dim;
  DenseDevice& D = M->dev;
  D.device = gossmx::context_device(ctx);
  int st = hipSetDevice(D.device) == hipSuccess ? GOSSMX_OK : err(GOSSMX_ERR_DEVICE, "hipSetDevice failed");
  D.layers.resize(config->layers);
  for (size_t li = 0; li < config->layers && st == GOSSMX_OK; ++li) {
    const gossmx_dense_layer& L = layers[li];
    DenseDevice::Layer& DL = D.layers[li];
    if (!st) st = upload(D, L.q_weight, QW * H, &DL.q);
    if (!st) st = upload(D, L.k_weight, KW * H, &DL.k);
    if (!st) st = upload(D, L.v_weight, KW * H, &DL.v);
    if (!st) st = upload(D, L.o_weight, H * QW, &DL.o);
    if (!st) st = upload(D, L.q_bias, QW, &DL.qb);
    if (!st) st = upload(D, L.k_bias, KW, &DL.kb);
    if (!st) st = upload(D, L.v_bias, KW, &DL.vb);
    if (!st) st = upload(D, L.o_bias, H, &DL.ob);
    if (!st) st = upload(D, L.post_attention_norm, H, &DL.post_norm);
  }
  if (!st) st = upload(D, lm_head, config->vocab * H, &D.lm_head);
  if (st) {
    delete M;
    return st;
  }
  *out = M;
  return GOSSMX_OK;
}

void gossmx_model_destroy(gossmx_model* model) { delete model; }

int gossmx_model_reset(gossmx_model* model) {
  if (!model) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null model");
  reset_caches(model);
  return GOSSMX_OK;
}

int gossmx_model_prefill(gossmx_model* model, const uint32_t* tokens, size_t n, float* logits) {
  if (!model || !tokens || !logits) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (!n) return err(GOSSMX_ERR_INVALID_DIMENSIONS, "CPU prefill is empty");
  reset_caches(model);
  return run_step(model, tokens, n, logits);
}

int gossmx_model_append(gossmx_model* model, const uint32_t* tokens, size_t n, float* logits) {
  if (!model || !tokens || !logits) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (!n) return err(GOSSMX_ERR_INVALID_DIMENSIONS, "CPU step is empty");
  return run_step(model, tokens, n, logits);
}

int gossmx_model_decode(gossmx_model* model, uint32_t token, float* logits) {
  if (!model || !logits) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (!model->position) return err(GOSSMX_ERR_INVALID_ARGUMENT, "CPU decode requires an existing prefill cache");
  return run_step(model, &token, 1, logits);
}

int gossmx_model_position(const gossmx_model* model, size_t* position) {
  if (!model || !position) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  *position = model->position;
  return GOSSMX_OK;
}

int gossmx_model_cache(const gossmx_model* model, size_t layer, size_t* len, size_t* start_position) {
  if (!model || !len || !start_position) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (layer >= model->cfg.layers) return err(GOSSMX_ERR_INVALID_ARGUMENT, "layer index out of range");
  *len = model->caches[layer].len;
  *start_position = model->caches[layer].start;
  return GOSSMX_OK;
}

int gossmx_model_times(const gossmx_model* model, double* dense_seconds, double* moe_seconds) {
  if (!model || !dense_seconds || !moe_seconds) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  *dense_seconds = model->dense_seconds;
  *moe_seconds = model->moe_seconds;
  return GOSSMX_OK;
}

int gossmx_greedy_token(const float* logits, size_t n, uint32_t* token) {
  if (!logits || !token) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  size_t best = n;
  for (size_t i = 0; i < n; ++i)
    if (std::isfinite(logits[i]) && (best == n || logits[i] > logits[best])) best = i;
  if (best == n) return err(GOSSMX_ERR_NON_FINITE_LOGITS, "model returned no finite logits");
  *token = (uint32_t)best;
  return GOSSMX_OK;
}

int gossmx_yarn_rope(const gossmx_model_config* config, float* values, size_t heads, size_t position) {
  if (!config || !values) return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (!config->head_dim || config->head_dim % 2)
    return err(GOSSMX_ERR_INVALID_DIMENSIONS, "head_dim must be even and non-zero");
  if (config->rope_yarn && (config->rope_factor <= 0.0 || !config->rope_original_max_positions))
    return err(GOSSMX_ERR_INVALID_DIMENSIONS, "YaRN scaling needs a positive factor and original positions");
  rope_apply(make_rope(*config), values, heads, position);
  return GOSSMX_OK;
}

int gossmx_attention(const float* query, const uint16_t* keys, const uint16_t* values, size_t tokens, size_t window,
                     const float* sinks, size_t heads, size_t kv_heads, size_t head_dim, float* out) {
  if (!query || !sinks || !out || (tokens && (!keys || !values)))
    return err(GOSSMX_ERR_INVALID_ARGUMENT, "null argument");
  if (!heads || !kv_heads || heads % kv_heads || !head_dim || !window)
    return err(GOSSMX_ERR_INVALID_DIMENSIONS, "invalid CPU attention dimensions");
  const size_t visible = std::min(tokens, window), first = tokens - visible, KW = kv_heads * head_dim;
  std::vector<float> scores;
  attention(query, visible, [&](size_t t) { return keys + (first + t) * KW; },
            [&](size_t t) { return values + (first + t) * KW; }, sinks, heads, kv_heads, head_dim, out, scores, 0,
            heads);
  return GOSSMX_OK;
}

}  // extern "C"
