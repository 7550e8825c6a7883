// gfx950 kernels of the GPT-OSS MXFP4 mixture-of-experts block.
//
// Exactness contract (crates/gpt-oss-cpu-kernels and cpu_runner.rs of
// gpt-oss-rs v0.1.0): every integer FP4 x Q8 block dot is exact, and every
// float chain keeps the reference's operation order, so the outputs are
// bit-identical to the scalar CPU path. Build with -ffp-contract=off: no
// multiply-add below may be fused unless written as fma() on purpose.
//
// Expert GEMM: v_mfma_f32_16x16x32_f16 with K = 32 = one MXFP4 block. The B
// operand is the weight tile converted from FP4 by v_cvt_scalef32_pk_f16_fp4
// (E2M1 values are exact in f16); the A operand holds the Q8 codes as f16
// (exact). Each product is exact in f32 and every partial sum is a multiple of
// 0.5 below 2^15, so the MFMA returns p / 2 exactly, where p is the reference's
// doubled-LUT integer dot (lib.rs:1067-1098). The reference term
// (p * (0.5 * e8m0)) * act_scale equals ((p / 2) * e8m0) * act_scale bit for
// bit: the first product is the same real number rounded once.
#include "gossmx_internal.h"

#include <cmath>

namespace gossmx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Scalar helpers.

// bf16::from_f32 of half 2.7.1 (round to nearest even, NaN quieted), used by
// fp32_to_bf16_roundtrip, cpu_runner.rs:3740-3744.
__device__ __forceinline__ uint16_t bf16_bits(float f) {
  const uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  const uint32_t round_bit = 0x8000u;
  if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0) return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float bf16r(float f) { return bf16_to_f32(bf16_bits(f)); }

// e8m0_scale, lib.rs:957-963: 0x00 -> 2^-127, 0xff -> NaN, else 2^(s-127).
__device__ __forceinline__ float e8m0(uint32_t s) {
  return s == 0 ? __uint_as_float(0x00400000u) : (s == 0xffu ? __uint_as_float(0x7fc00000u) : __uint_as_float(s << 23));
}

// expf with the exact results of the host's glibc 2.35 expf, which is what
// Rust's f32::exp calls on x86_64 Linux (softmax cpu_runner.rs:3784-3795,
// gpt_oss_swiglu :3797-3826). Algorithm of glibc sysdeps/ieee754/flt-32/e_expf.c
// (Szabolcs Nagy, ARM optimized-routines): x * 32/ln2 split by the 0x1.8p52
// shift into k and r, a 32-entry table of 2^(i/32), and a cubic in r, all in
// double with fused multiply-adds as the FMA build of glibc evaluates it.
// Table entries: bits of 2^(i/32) rounded to double, minus i << 47.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__device__ float expf_glibc(float x) {
  const uint32_t ux = __float_as_uint(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88 (top 12 bits of 88.0f), inf or NaN
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd = fma(inv_ln2_n, xd, shift);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd -= shift;
  const double r = fma(inv_ln2_n, xd, -kd);
  const uint64_t t = kExp2Tab[ki % 32] + (ki << 47);
  const double s = __longlong_as_double((long long)t);
  const double z = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// The SwiGLU sigmoid bf16(1 / (1 + expf(-s))) of gpt_oss_swiglu
// (cpu_runner.rs:3819-3820) for every bf16 value s = bits << 16.
__device__ __forceinline__ uint16_t sigmoid_bf16(uint32_t bits) {
  const float scaled = bf16_to_f32((uint16_t)bits);
  return bf16_bits(1.0f / (1.0f + expf_glibc(-scaled)));
}

// gpt_oss_swiglu for one (gate, up) pair, cpu_runner.rs:3797-3826: gate =
// min(g, limit) (NaN-ignoring like f32::min), up = clamp(u, -limit, limit)
// (NaN kept), then bf16 after every tensor operation. The sigmoid's input is
// a bf16 value, so it is read from `sig_tab`, the 65,536 values of
// sigmoid_bf16 computed by the same code (build_sigmoid_table).
__device__ __forceinline__ float swiglu_one(float g, float u, float alpha, float limit, const uint16_t* sig_tab) {
  const float gate = fminf(g, limit);
  float up = u;
  if (up < -limit) up = -limit;
  if (up > limit) up = limit;
  const float sig = bf16_to_f32(sig_tab[bf16_bits(gate * alpha)]);
  const float glu = bf16r(gate * sig);
  const float lin = bf16r(up + 1.0f);
  return bf16r(glu * lin);
}

__global__ void build_sigmoid_table_kernel(uint16_t* tab) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 65536u) tab[i] = sigmoid_bf16(i);
}

// quantize_q8_block (lib.rs:1051-1065) for the 32 values held by a 32-lane
// half wave (lane l32 holds value l32): scale = max|v| / 127, inverse =
// 1 / scale (0 when scale is 0), q = clamp(round_half_away(v * inverse)).
// max is order-free, so the butterfly gives the reference's fold.
__device__ __forceinline__ void q8_half_wave(float v, float& q, float& scale) {
  float mx = fabsf(v);
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  scale = mx / 127.0f;
  const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
  q = fminf(fmaxf(roundf(v * inv), -127.0f), 127.0f);
}

// quantize_residual_q8 (lib.rs:382-409) of one block held by a half wave;
// writes the f16 codes and the two scales of (row, blk) into `act`.
__device__ __forceinline__ void residual_q8_store(float v, int l32, size_t row, int blocks, int blk, ActBuffers act) {
  float q, s;
  q8_half_wave(v, q, s);
  const float r = v - q * s;
  float rq, rs;
  q8_half_wave(r, rq, rs);
  _Float16* dst = act.v + ((row * blocks + blk) * 2) * kBlock;
  dst[l32] = (_Float16)q;
  dst[kBlock + l32] = (_Float16)rq;
  if (l32 == 0) {
    float2 sc;
    sc.x = s;
    sc.y = rs;
    reinterpret_cast<float2*>(act.s)[row * blocks + blk] = sc;
  }
}

// ---------------------------------------------------------------------------
// Router projection, top-k, routing softmax and the gate_up input quantization,
// one work-group per row (moe_batch routing loop, cpu_runner.rs:2808-2854).

__device__ __forceinline__ bool route_better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);  // stable_top_k order, cpu_runner.rs:3768-3778
}

__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int r = blockIdx.x;
  const int E = a.experts, H = a.hidden, K = a.top_k;
  const uint16_t* x = a.x + (size_t)r * H;
  __shared__ float s_chain[kMaxExperts * 16];
  __shared__ float s_logit[kMaxExperts];
  __shared__ int s_sel[kMaxTopK];

  if (a.injected == nullptr) {
    // scalar_bf16_dot (lib.rs:1007-1029): 16 reduction lanes, lane j sums
    // w[i] * x[i] for i = j mod 16 in increasing i, multiply then add.
    for (int c = threadIdx.x; c < E * 16; c += blockDim.x) {
      const int e = c >> 4, l = c & 15;
      const uint16_t* w = a.router_w + (size_t)e * H;
      float acc = 0.0f;
      for (int i = l; i < H; i += 16) acc = acc + bf16_to_f32(w[i]) * bf16_to_f32(x[i]);
      s_chain[c] = acc;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      float s = s_chain[e * 16];
      for (int l = 1; l < 16; ++l) s = s + s_chain[e * 16 + l];
      s_logit[e] = bf16r(s + a.router_b[e]);  // += bias (cpu_runner.rs:2781-2783), bf16 (:2829)
    }
  } else {
    for (int e = threadIdx.x; e < E; e += blockDim.x) s_logit[e] = bf16r(a.injected[(size_t)r * E + e]);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const float v = s_logit[e];
    if (!isfinite(v)) atomicOr(a.err, kErrNonFiniteLogits);
    if (a.logits) a.logits[(size_t)r * E + e] = v;
  }

  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    // Each lane owns experts lane and lane + 64; K rounds of a wave argmax.
    // NaN logits (already flagged as an error) rank as -inf so that every
    // round still returns a valid expert index.
    bool taken0 = false, taken1 = false;
    float v0 = lane < E ? s_logit[lane] : -INFINITY;
    float v1 = lane + 64 < E ? s_logit[lane + 64] : -INFINITY;
    if (isnan(v0)) v0 = -INFINITY;
    if (isnan(v1)) v1 = -INFINITY;
    for (int k = 0; k < K; ++k) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      if (lane < E && !taken0) { bv = v0; bi = lane; }
      if (lane + 64 < E && !taken1 && route_better(v1, lane + 64, bv, bi)) { bv = v1; bi = lane + 64; }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (route_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      if (bi < 0 || bi >= E) bi = 0;
      if (bi == lane) taken0 = true;
      if (bi == lane + 64) taken1 = true;
      if (lane == 0) s_sel[k] = bi;
    }
    if (lane == 0) {
      // softmax over the selected logits in rank order (cpu_runner.rs:3784-3795),
      // then bf16 (:2840-2843).
      float mx = -INFINITY;
      for (int k = 0; k < K; ++k) mx = fmaxf(mx, s_logit[s_sel[k]]);
      float ex[kMaxTopK];
      float sum = 0.0f;
      for (int k = 0; k < K; ++k) {
        ex[k] = expf_glibc(s_logit[s_sel[k]] - mx);
        sum = sum + ex[k];
      }
      for (int k = 0; k < K; ++k) {
        a.selected[(size_t)r * K + k] = s_sel[k];
        a.weights[(size_t)r * K + k] = bf16r(ex[k] / sum);
      }
    }
  }

  // quantize_residual_q8 of the row for gate_up (cpu_runner.rs:3224-3231):
  // one half wave per 32-value block.
  const int hw = threadIdx.x >> 5, l32 = threadIdx.x & 31;
  const int blocks = H / kBlock;
  for (int b = hw; b < blocks; b += blockDim.x / 32) {
    const float v = bf16_to_f32(x[b * kBlock + l32]);
    if (!isfinite(v)) atomicOr(a.err, kErrNonFiniteInput);
    residual_q8_store(v, l32, (size_t)r, blocks, b, a.act);
  }
}

// ---------------------------------------------------------------------------
// Stable grouping of routes by expert (stable_group_routes,
// cpu_runner.rs:3780-3782): route i = row * top_k + rank goes to
// bucket_off[e] + #{j < i : expert(j) == e}. One work-group of 1024 threads;
// in-wave ranks come from one ballot per expert.

__global__ __launch_bounds__(1024) void dispatch_kernel(DispatchArgs a) {
  const int E = a.experts, R = a.routes;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int s_tot[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_run[kMaxExperts];
  __shared__ int s_wcnt[16][kMaxExperts];
  for (int e = tid; e < E; e += 1024) { s_tot[e] = 0; s_run[e] = 0; }
  __syncthreads();
  for (int i = tid; i < R; i += 1024) atomicAdd(&s_tot[a.selected[i]], 1);
  __syncthreads();
  if (tid == 0) {
    // Work items: buckets of at most kSmallRows rows go to the small-bucket
    // kernel (when enabled), larger ones are cut into kChunk-row chunks.
    int acc = 0, ns = 0;
    for (int e = 0; e < E; ++e) {
      s_off[e] = acc;
      a.bucket_off[e] = acc;
      const int c = s_tot[e];
      if (a.small_enabled && c > 0 && c <= kSmallRows) {
        a.work_small[2 * ns] = e;
        a.work_small[2 * ns + 1] = 0;
        ++ns;
      }
      acc += c;
    }
    a.bucket_off[E] = acc;
    *a.n_work_small = ns;
  }
  __syncthreads();
  // Large buckets: chunks in descending row count, so the heaviest work items
  // are dispatched first and the grid's last wave is light. All chunks of an
  // expert but the last hold kChunk rows; full chunks come first (expert
  // order), then the partial last chunks by size (ties by expert).
  for (int e = tid; e < E; e += 1024) {
    const int c = s_tot[e];
    const bool large = c > 0 && !(a.small_enabled && c <= kSmallRows);
    const int full = large ? c / kChunk : 0, part = large ? c % kChunk : 0;
    int full_before = 0, full_total = 0, part_before = 0, parts = 0;
    for (int f = 0; f < E; ++f) {
      const int cf = s_tot[f];
      const bool lf = cf > 0 && !(a.small_enabled && cf <= kSmallRows);
      const int ff = lf ? cf / kChunk : 0, pf = lf ? cf % kChunk : 0;
      full_total += ff;
      if (f < e) full_before += ff;
      if (pf > 0) {
        ++parts;
        if (pf > part || (pf == part && f < e)) ++part_before;
      }
    }
    for (int i = 0; i < full; ++i) {
      a.work[2 * (full_before + i)] = e;
      a.work[2 * (full_before + i) + 1] = i * kChunk;
    }
    if (part > 0) {
      a.work[2 * (full_total + part_before)] = e;
      a.work[2 * (full_total + part_before) + 1] = full * kChunk;
    }
    if (e == 0) *a.n_work = full_total + parts;
  }
  __syncthreads();
  for (int base = 0; base < R; base += 1024) {
    const int i = base + tid;
    const int e = i < R ? a.selected[i] : -1;
    const unsigned long long lt = (1ull << lane) - 1ull;
    int rank = 0;
    for (int ee = 0; ee < E; ++ee) {
      const unsigned long long m = __ballot(e == ee);
      if (e == ee) rank = __popcll(m & lt);
      if (lane == 0) s_wcnt[wave][ee] = __popcll(m);
    }
    __syncthreads();
    if (e >= 0) {
      int pos = s_off[e] + s_run[e] + rank;
      for (int w = 0; w < wave; ++w) pos += s_wcnt[w][e];
      a.route_tok[pos] = i / a.top_k;
      a.route_slot[pos] = i;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += 1024) {
      int add = 0;
      for (int w = 0; w < 16; ++w) add += s_wcnt[w][ee];
      s_run[ee] += add;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Expert GEMM on the resident v3 layout. One work-group = kWaves waves, one
// 16-row weight tile per wave (128 rows), times one work item (<= 64
// activation rows). Each lane owns one weight row (lane % 16) and two
// activation rows per group of 8, and runs the reference's per-row float
// chain in order:
//   total = bias; for each block: total += (p * ws) * ps; total += (r * ws) * rs
// (mxfp4_residual_q8_gemv_rows lib.rs:673-696, scalar_matmul_range
// matmul.rs:529-578).
//
// Streaming: K is walked in groups of 4 blocks. Each wave keeps the weights of
// the next kPrefetch groups in flight in registers (one 16-byte load per lane
// per group, a 1 KiB contiguous segment per wave). The work item's activations
// for a group (f16 codes and scales) are staged through LDS once per
// work-group: loaded from global memory into registers one group ahead, then
// written to LDS between two barriers, so all waves share one L2 read.

__device__ __forceinline__ half8 fp4x8_to_half8(uint32_t w) {
  const half2v h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0);
  const half2v h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1);
  const half2v h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2);
  const half2v h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3);
  half8 b;
  b[0] = h0[0]; b[1] = h0[1]; b[2] = h1[0]; b[3] = h1[1];
  b[4] = h2[0]; b[5] = h2[1]; b[6] = h3[0]; b[7] = h3[1];
  return b;
}

constexpr int kWaves = 8;                  // waves per GEMM work-group
constexpr int kSlotBytes = 4 * kChunk * 2 * kBlock * 2;  // f16 codes of one K group in LDS
constexpr int kCodeDma = 4 * kChunk * 8 / (64 * kWaves);  // 16-byte DMA instructions per wave per group
static_assert(4 * kChunk * 8 == kCodeDma * 64 * kWaves, "code DMA covers a slot exactly");
static_assert(4 * kChunk * 2 <= 64 * kWaves, "one 4-byte DMA per wave covers a group's scales");
constexpr int kSclSlot = 64 * kWaves / 2;                  // float2 written by one group's scale DMA
// s_waitcnt immediate: vmcnt = kCodeDma + 1 (D(q+1)) + 2 + 2 (W(q+1), W(q+2)),
// expcnt and lgkmcnt not waited on (7, 15).
constexpr int kWaitVm = kCodeDma + 1 + 4;
constexpr int kWaitDmaGroup = (kWaitVm & 15) | ((kWaitVm >> 4) << 14) | (7 << 4) | (15 << 8);
constexpr int kGemmThreads = 64 * kWaves;  // 512
constexpr int kGemmRows = 16 * kWaves;     // weight rows per work-group
constexpr int kPrefetch = 3;               // weight groups in flight per wave

struct WeightGroup {
  uint4 v;     // one dword of nibbles per block (codes 8g..8g+7 of this lane's row)
  uint32_t s;  // E8M0 bytes of this lane's row for the group's blocks
};

// Loads of a full 4-block group q. Unconditional (no branch around a load),
// so the compiler's load counters stay exact and the prefetched groups stay
// in flight; callers clamp q to a full group of a valid tile.
__device__ __forceinline__ WeightGroup load_full_group(const uint8_t* nib, const uint8_t* scl, int q, int lane,
                                                       int nl) {
  WeightGroup g;
  g.v = *reinterpret_cast<const uint4*>(nib + (size_t)q * 1024 + lane * 16);
  g.s = *reinterpret_cast<const uint32_t*>(scl + (size_t)q * 64 + nl * 4);
  return g;
}

// Loads of the last group when K is not a multiple of 4 blocks (rem = 1..3
// blocks): dwords at lane * rem * 4 of the compact nibble group, and the
// row's (padded) scale dword. Reads past the group stay inside the
// allocation slack (kPlaneSlack).
__device__ __forceinline__ WeightGroup load_tail_group(const uint8_t* nib, const uint8_t* scl, int q, int rem,
                                                       int lane, int nl) {
  const uint32_t* gw = reinterpret_cast<const uint32_t*>(nib + (size_t)q * 1024 + lane * rem * 4);
  WeightGroup g;
  g.v = make_uint4(gw[0], gw[1], gw[2], 0u);
  g.s = *reinterpret_cast<const uint32_t*>(scl + (size_t)q * 64 + nl * 4);
  return g;
}

// E8M0 bytes whose scaled E2M1 values are exact f16 normals: 0.5 * 2^(s-127)
// >= 2^-14 and 6 * 2^(s-127) <= 65504.
constexpr uint32_t kFastScaleLo = 114, kFastScaleHi = 139;

__device__ __forceinline__ half8 fp4x8_to_half8_scaled(uint32_t w, float scale) {
  const half2v h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 0);
  const half2v h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 1);
  const half2v h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 2);
  const half2v h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 3);
  half8 b;
  b[0] = h0[0]; b[1] = h0[1]; b[2] = h1[0]; b[3] = h1[1];
  b[4] = h2[0]; b[5] = h2[1]; b[6] = h3[0]; b[7] = h3[1];
  return b;
}

// e8m0_scale without branches (lib.rs:957-963).
__device__ __forceinline__ float e8m0_select(uint32_t s) {
  const float normal = __uint_as_float(s << 23);
  const float v = s == 0u ? __uint_as_float(0x00400000u) : normal;
  return s == 0xffu ? __uint_as_float(0x7fc00000u) : v;
}

// LDS slot layout of one K group (written by DMA, read as MFMA A operands):
// for block j and token group tg, 1 KiB = [k-slice g (4)][vector i (16)][16 B]
// with vector i = 2 * (row within the group) + part (0 primary, 1 residual),
// so lane (g, i) of a wave reads the 16 bytes at lane * 16 (conflict-free).
__device__ __forceinline__ int slot_chunk(int j, int tg) { return j * (kChunk / 8) + tg; }

// One block j of the current group against NTG token groups: the MFMAs and
// the ordered chain updates. SCALED: the weight operand already carries the
// E8M0 scale (exact), so the MFMA returns (p / 2) * e8m0 and a term is
// d * act_scale; otherwise a term is (d * e8m0) * act_scale. Both are the
// reference's (p * (0.5 * e8m0)) * act_scale rounded once.
template <bool RESIDUAL, bool SCALED, int NTG>
__device__ __forceinline__ void block_update(float (&tot)[kChunk / 8][2], const char* codes, const float2* scl,
                                             const half8 bop, const float e8, const int j, const int lane,
                                             const int G) {
#pragma unroll
  for (int tg = 0; tg < NTG; ++tg) {
    const half8 aop = *reinterpret_cast<const half8*>(codes + slot_chunk(j, tg) * 1024 + lane * 16);
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, zero, 0, 0, 0);
    const float4 sc = *reinterpret_cast<const float4*>(&scl[j * kChunk + tg * 8 + 2 * G]);
    if (SCALED) {
      tot[tg][0] = tot[tg][0] + d[0] * sc.x;
      if (RESIDUAL) tot[tg][0] = tot[tg][0] + d[1] * sc.y;
      tot[tg][1] = tot[tg][1] + d[2] * sc.z;
      if (RESIDUAL) tot[tg][1] = tot[tg][1] + d[3] * sc.w;
    } else {
      tot[tg][0] = tot[tg][0] + (d[0] * e8) * sc.x;
      if (RESIDUAL) tot[tg][0] = tot[tg][0] + (d[1] * e8) * sc.y;
      tot[tg][1] = tot[tg][1] + (d[2] * e8) * sc.z;
      if (RESIDUAL) tot[tg][1] = tot[tg][1] + (d[3] * e8) * sc.w;
    }
  }
}

// All blocks of one K group for this wave's tile.
template <bool RESIDUAL, int NTG>
__device__ __forceinline__ void group_update(float (&tot)[kChunk / 8][2], const char* codes, const float2* scl,
                                             const WeightGroup cur, const int nb, const int lane, const int G) {
  const uint32_t wv[4] = {cur.v.x, cur.v.y, cur.v.z, cur.v.w};
  bool in_range = true;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t s = (cur.s >> (8 * j)) & 0xffu;
    if (j < nb) in_range = in_range && (s - kFastScaleLo) <= (kFastScaleHi - kFastScaleLo);
  }
  if (__all(in_range)) {  // wave-uniform
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nb) {
        const float e8 = __uint_as_float(((cur.s >> (8 * j)) & 0xffu) << 23);
        block_update<RESIDUAL, true, NTG>(tot, codes, scl, fp4x8_to_half8_scaled(wv[j], e8), 0.0f, j, lane, G);
      }
    }
  } else {
    // Rare: a scale outside the exact-f16 range (including the 0x00 and 0xff
    // encodings). Kept compact; same bits through the unscaled operand.
#pragma unroll 1
    for (int j = 0; j < nb; ++j) {
      const uint32_t w = j == 0 ? wv[0] : (j == 1 ? wv[1] : (j == 2 ? wv[2] : wv[3]));
      const float e8 = e8m0_select((cur.s >> (8 * j)) & 0xffu);
      block_update<RESIDUAL, false, NTG>(tot, codes, scl, fp4x8_to_half8(w), e8, j, lane, G);
    }
  }
}

// Shared GEMM epilogue: plain f32 stores, the down projection's bf16 rows,
// or gate_up's SwiGLU and down-input quantization. `s_act` is LDS scratch of
// at least count * (kGemmRows / 2 + 1) floats, free for reuse.
template <int MODE, int NT>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, const float (&tot)[NT][2], const int n_tg,
                                              const int count, const int start, const int route_base, const int row,
                                              const bool tile_ok, float* s_act) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int nl = lane & 15, G = lane >> 4;
  const int rows = (int)a.w.rows;


  if (MODE == kPlain) {
    if (tile_ok && row < rows) {
#pragma unroll
      for (int tg = 0; tg < NT; ++tg)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int c = tg * 8 + 2 * G + t;
          if (c < count) a.out[(size_t)(start + c) * a.out_stride + row] = tot[tg][t];
        }
    }
  } else if (MODE == kDown) {
    if (tile_ok && row < rows) {
#pragma unroll
      for (int tg = 0; tg < NT; ++tg)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int c = tg * 8 + 2 * G + t;
          if (c < count) {
            const int slot = a.route_slot[route_base + start + c];
            a.y[(size_t)slot * rows + row] = bf16_bits(tot[tg][t]);  // bf16 (cpu_runner.rs:2945-2947)
          }
        }
    }
  } else {
    // gate_up epilogue: bf16 (cpu_runner.rs:2905), SwiGLU over (even, odd)
    // rows (:2907-2919), then the down input's residual-Q8 blocks: the 128
    // rows of this work-group make two 32-value blocks (cpu_runner.rs:3224-3231).
    // The SwiGLU values reuse the first LDS slot as [kChunk rows][64 values].
    constexpr int kActStride = kGemmRows / 2 + 1;
    // Lane pairs (even = gate row, odd = up row) hold both values for tokens
    // t0 = 2G and t1 = 2G + 1; the even lane finishes t0 and the odd lane t1.
    const bool odd = (nl & 1) != 0;
#pragma unroll
    for (int tg = 0; tg < NT; ++tg) {
      if (tg < n_tg) {
        const float own0 = bf16r(tot[tg][0]), own1 = bf16r(tot[tg][1]);
        const float recv = __shfl_xor(odd ? own0 : own1, 1);
        const float gate = odd ? recv : own0;
        const float up = odd ? own1 : recv;
        const int c = tg * 8 + 2 * G + (odd ? 1 : 0);
        if (c < count)
          s_act[c * kActStride + wave * 8 + (nl >> 1)] = swiglu_one(gate, up, a.alpha, a.limit, a.sig_tab);
      }
    }
    __syncthreads();
    const int hw = tid >> 5, l32 = tid & 31;
    const int blocks_next = rows / kWgRows;
    constexpr int kBlocksPerWg = kGemmRows / 64;
    for (int item = hw; item < count * kBlocksPerWg; item += kGemmThreads / 32) {
      const int c = item / kBlocksPerWg, h = item % kBlocksPerWg;
      if (blockIdx.x * kBlocksPerWg + h >= blocks_next) continue;  // uniform per half wave
      const float v = s_act[c * kActStride + h * kBlock + l32];
      if (!isfinite(v)) atomicOr(a.err, kErrNonFiniteInput);
      ActBuffers nx;
      nx.v = a.actv_next;
      nx.s = a.acts_next;
      residual_q8_store(v, l32, (size_t)(route_base + start + c), blocks_next, blockIdx.x * kBlocksPerWg + h, nx);
    }
  }
}

// Loop-invariant state of the K loop.
struct KLoop {
  const uint8_t* nib;
  const uint8_t* scl;
  WeightGroup tail;
  int nq, nqf, last_full, B, wave, lane, nl, G;
  bool tile_ok;
  // DMA lane map (see gemm_kernel)
  const char* gcodes;
  const char* gscl;
  int coff[kCodeDma];  // byte offset of this lane's code piece in group 0, or -1: nothing to move
  int soff;            // same for the scale dword
};

// Issues the DMA of group qq (clamped to the last group) into one ring slot.
__device__ __forceinline__ void issue_dma(const KLoop& k, int qq_raw, char* codes, float2* scl) {
  const int qq = min(qq_raw, k.nq - 1);
  const int gstep = qq * 4 * 128;  // 4 blocks of 128 B per activation row
#pragma unroll
  for (int i = 0; i < kCodeDma; ++i) {
    const char* src = k.coff[i] >= 0 ? k.gcodes + (k.coff[i] + gstep) : k.gcodes;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(codes + (i * kWaves + k.wave) * 1024),
                                     16, 0, 0);
  }
  const char* ssrc = k.soff >= 0 ? k.gscl + (k.soff + qq * 4 * 8) : k.gscl;
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)ssrc,
                                   (__attribute__((address_space(3))) void*)((char*)scl + k.wave * 256), 4, 0, 0);
}

// The K loop for NTG token groups. Vector-memory issue order per wave, fixed
// so that one immediate wait covers every group:
//   prologue W(0) D(0) W(1) D(1) W(2); iteration q: wait(D(q)) barrier
//   D(q+2) compute(q) W(q+3).
// After D(q) come W(q+1), D(q+1), W(q+2) = kWaitVm instructions.
template <bool RESIDUAL, int NTG>
__device__ __forceinline__ void k_loop(const KLoop& k, float (&tot)[kChunk / 8][2], char* c0, char* c1, char* c2,
                                       float2* s0, float2* s1, float2* s2) {
  WeightGroup wg0, wg1, wg2;
  __builtin_amdgcn_sched_barrier(0);
  wg0 = load_full_group(k.nib, k.scl, min(0, k.last_full), k.lane, k.nl);
  __builtin_amdgcn_sched_barrier(0);
  issue_dma(k, 0, c0, s0);
  __builtin_amdgcn_sched_barrier(0);
  wg1 = load_full_group(k.nib, k.scl, min(1, k.last_full), k.lane, k.nl);
  __builtin_amdgcn_sched_barrier(0);
  issue_dma(k, 1, c1, s1);
  __builtin_amdgcn_sched_barrier(0);
  wg2 = load_full_group(k.nib, k.scl, min(2, k.last_full), k.lane, k.nl);
  __builtin_amdgcn_sched_barrier(0);
#define GOSSMX_GROUP(QV, SLOT, CODES, SCL, NCODES, NSCL)                                            \
  {                                                                                                 \
    const int q = (QV);                                                                             \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    __builtin_amdgcn_s_waitcnt(kWaitDmaGroup); /* this wave's DMA for group q has landed */        \
    __builtin_amdgcn_s_barrier();              /* ... and every other wave's; slot of q-1 is free */ \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    issue_dma(k, q + 2, NCODES, NSCL);                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    const WeightGroup cur = q < k.nqf ? SLOT : k.tail;                                              \
    if (k.tile_ok && q < k.nq)                                                                      \
      group_update<RESIDUAL, NTG>(tot, CODES, SCL, cur, min(4, k.B - 4 * q), k.lane, k.G);          \
    __builtin_amdgcn_sched_barrier(0);                                                              \
    SLOT = load_full_group(k.nib, k.scl, min(q + 3, k.last_full), k.lane, k.nl);                    \
    __builtin_amdgcn_sched_barrier(0);                                                              \
  }
  const int nq_pad = (k.nq + 2) / 3 * 3;
  for (int q0 = 0; q0 < nq_pad; q0 += 3) {
    GOSSMX_GROUP(q0, wg0, c0, s0, c2, s2)
    GOSSMX_GROUP(q0 + 1, wg1, c1, s1, c0, s0)
    GOSSMX_GROUP(q0 + 2, wg2, c2, s2, c1, s1)
  }
#undef GOSSMX_GROUP
}

template <int MODE, bool RESIDUAL>
__global__ __launch_bounds__(kGemmThreads, 4) void gemm_kernel(GemmArgs a) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int nl = lane & 15, G = lane >> 4;
  int expert, start, count, route_base = 0;
  if (MODE == kPlain) {
    expert = a.plain_expert;
    start = blockIdx.y * kChunk;
    count = min(kChunk, a.plain_m - start);
  } else {
    const int wi = blockIdx.y;
    if (wi >= *a.n_work) return;  // uniform over the work-group
    expert = a.work[2 * wi];
    start = a.work[2 * wi + 1];
    route_base = a.bucket_off[expert];
    count = min(kChunk, a.bucket_off[expert + 1] - route_base - start);
  }
  // LDS ring of three K groups, filled by global->LDS DMA two groups ahead.
  __shared__ __align__(16) char s_codes0[kSlotBytes], s_codes1[kSlotBytes], s_codes2[kSlotBytes];
  // A scale DMA writes 64 dwords per wave: kSclSlot float2 per slot, of which
  // the first 4 * kChunk ([block][row]) hold data.
  __shared__ __align__(16) float2 s_scl0[kSclSlot], s_scl1[kSclSlot], s_scl2[kSclSlot];
  __shared__ int s_row[kChunk];
  if (tid < kChunk) {
    int r = -1;
    if (tid < count) {
      if (MODE == kPlain) r = start + tid;
      else if (MODE == kGateUp) r = a.route_tok[route_base + start + tid];
      else r = route_base + start + tid;
    }
    s_row[tid] = r;
  }
  __syncthreads();

  const int rows = (int)a.w.rows, B = (int)a.w.blocks;
  const int tile = blockIdx.x * kWaves + wave;
  const int row = tile * kTileRows + nl;
  const int n_tg = (count + 7) >> 3;

  KLoop k;
  k.B = B;
  k.nq = (B + 3) >> 2;
  k.nqf = B >> 2;
  k.last_full = k.nqf > 0 ? k.nqf - 1 : 0;
  k.wave = wave;
  k.lane = lane;
  k.nl = nl;
  k.G = G;
  k.tile_ok = tile < (int)a.w.tiles;
  // Waves past the last tile read tile 0 and discard it.
  const int safe_tile = k.tile_ok ? tile : 0;
  k.nib = a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)safe_tile * 256 * B;
  k.scl = a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)safe_tile * 64 * k.nq;
  k.tail = load_tail_group(k.nib, k.scl, k.nqf, (B & 3) > 0 ? (B & 3) : 1, lane, nl);

  float b0 = 0.0f;
  if (a.bias != nullptr && k.tile_ok && row < rows) b0 = a.bias[(size_t)expert * a.bias_expert_stride + row];
  b0 = b0 + 0.0f;  // a -0.0 bias becomes +0.0, as the reference's first add does
  float tot[kChunk / 8][2];
#pragma unroll
  for (int tg = 0; tg < kChunk / 8; ++tg) { tot[tg][0] = b0; tot[tg][1] = b0; }

  // DMA lane map, the same for every group. Code instruction i of this wave
  // fills slot bytes c * 16 with c = (i * kWaves + wave) * 64 + lane, i.e.
  // block j, token group tg, k-slice g, vector v (row tg*8 + v/2, part v%2)
  // in the slot layout above; its source is piece (part, g) of the row's
  // 128-byte block record. Scale dword d = wave * 64 + lane holds half d % 2
  // of (block d / (2 kChunk), row (d / 2) % kChunk). Lanes with nothing to
  // move read the buffer base (valid memory) into slot bytes no row uses, so
  // every wave issues the same instructions. Reads of a last partial group
  // run up to 3 blocks past a row, inside the buffers' slack.
  k.gcodes = reinterpret_cast<const char*>(a.actv);
  k.gscl = reinterpret_cast<const char*>(a.acts);
#pragma unroll
  for (int i = 0; i < kCodeDma; ++i) {
    const int c = (i * kWaves + wave) * 64 + lane;
    const int j = c / (kChunk * 8), r = c % (kChunk * 8);
    const int tg = r >> 6, g = (r >> 4) & 3, v = r & 15;
    const int t = tg * 8 + (v >> 1), part = v & 1;
    k.coff[i] = t < count ? ((s_row[t] * B + j) * 8 + part * 4 + g) * 16 : -1;
  }
  {
    const int d = wave * 64 + lane;
    const int j = d / (kChunk * 2), t = (d >> 1) % kChunk;
    k.soff = (d < 4 * kChunk * 2 && t < count) ? ((s_row[t] * B + j) * 2 + (d & 1)) * 4 : -1;
  }

  switch (n_tg) {
    case 1: k_loop<RESIDUAL, 1>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2); break;
    case 2: k_loop<RESIDUAL, 2>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2); break;
    case 3: k_loop<RESIDUAL, 3>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2); break;
    case 4: k_loop<RESIDUAL, 4>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2); break;
    default: k_loop<RESIDUAL, 6>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2); break;
  }
  // Drain the trailing DMA into the ring before the LDS is reused or the
  // work-group ends.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  gemm_epilogue<MODE, kChunk / 8>(a, tot, n_tg, count, start, route_base, row, k.tile_ok,
                                  reinterpret_cast<float*>(s_codes0));
}

// ---------------------------------------------------------------------------
// Small-bucket expert GEMM: work items of at most kSmallRows (16) activation
// rows, most of the experts at decode batch 64 under Zipf routing. The item's
// activations are staged into LDS for a whole phase of K (all 90 blocks for
// <= 4 rows, 48 blocks for <= 8, 24 blocks for <= 16), so the K loop inside a
// phase has no barriers and no activation traffic: each wave streams its
// 16-row weight tile through a kSmallRing-deep register ring that continues
// across phases. Same operands, chain order and epilogue as gemm_kernel.
//
// Per-block LDS layouts (V vectors = 2 parts x token slots):
//   V = 8  (<= 4 rows):  512 B = [k-slice g][vector v < 8][16 B]; MFMA rows
//                         8..15 repeat rows 0..7 (unused results).
//   V = 16 (<= 8 rows):  1 KiB = [g][v < 16][16 B]
//   V = 32 (<= 16 rows): 2 KiB = two 1 KiB token groups of the V = 16 form.
// Scales: [block][token slot] float2, V / 2 slots per block, plus an 8-entry
// tail (lanes of unused token slots read past a block).
constexpr int kSmallRing = 3;
constexpr int kSmallCodeBytes = 48 * 1024;
constexpr int kSmallSclEntries = 384 + 8;
constexpr int kSmallStage = 6;  // 16-byte staging pieces per thread per phase (max over layouts)

template <int V>
struct SmallLayout {
  static constexpr int kNT = V <= 16 ? 1 : 2;           // MFMA token groups
  static constexpr int kBlockBytes = V * 64;            // LDS bytes per block
  static constexpr int kSlots = V / 2;                  // token slots per block
  static constexpr int kPhaseBlocks = kSmallCodeBytes / kBlockBytes;  // 96, 48, 24
  static_assert(kPhaseBlocks % 12 == 0, "phases are whole multiples of the 3-deep, 4-block ring");
  static_assert(kPhaseBlocks * kSlots + 8 <= kSmallSclEntries, "scale LDS");
  static_assert(16 * 24 * 8 <= kSmallStage * kGemmThreads, "staging pieces");
};

template <int V, bool RESIDUAL, bool SCALED>
__device__ __forceinline__ void small_block(float (&tot)[2][2], const char* codes, const float2* scl, const half8 bop,
                                            const float e8, const int jl, const int lane, const int nl,
                                            const int G) {
  using L = SmallLayout<V>;
#pragma unroll
  for (int tg = 0; tg < L::kNT; ++tg) {
    const int a_off = V == 8 ? (G * 8 + (nl & 7)) * 16 : tg * 1024 + lane * 16;
    const half8 aop = *reinterpret_cast<const half8*>(codes + jl * L::kBlockBytes + a_off);
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, zero, 0, 0, 0);
    const float4 sc = *reinterpret_cast<const float4*>(&scl[jl * L::kSlots + tg * 8 + 2 * G]);
    if (SCALED) {
      tot[tg][0] = tot[tg][0] + d[0] * sc.x;
      if (RESIDUAL) tot[tg][0] = tot[tg][0] + d[1] * sc.y;
      tot[tg][1] = tot[tg][1] + d[2] * sc.z;
      if (RESIDUAL) tot[tg][1] = tot[tg][1] + d[3] * sc.w;
    } else {
      tot[tg][0] = tot[tg][0] + (d[0] * e8) * sc.x;
      if (RESIDUAL) tot[tg][0] = tot[tg][0] + (d[1] * e8) * sc.y;
      tot[tg][1] = tot[tg][1] + (d[2] * e8) * sc.z;
      if (RESIDUAL) tot[tg][1] = tot[tg][1] + (d[3] * e8) * sc.w;
    }
  }
}

// One 4-block weight group whose first block is phase-local block jl0.
template <int V, bool RESIDUAL>
__device__ __forceinline__ void small_group(float (&tot)[2][2], const char* codes, const float2* scl,
                                            const WeightGroup cur, const int jl0, const int nb, const int lane,
                                            const int nl, const int G) {
  const uint32_t wv[4] = {cur.v.x, cur.v.y, cur.v.z, cur.v.w};
  bool in_range = true;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t s = (cur.s >> (8 * j)) & 0xffu;
    if (j < nb) in_range = in_range && (s - kFastScaleLo) <= (kFastScaleHi - kFastScaleLo);
  }
  if (__all(in_range)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nb) {
        const float e8 = __uint_as_float(((cur.s >> (8 * j)) & 0xffu) << 23);
        small_block<V, RESIDUAL, true>(tot, codes, scl, fp4x8_to_half8_scaled(wv[j], e8), 0.0f, jl0 + j, lane, nl, G);
      }
    }
  } else {
#pragma unroll 1
    for (int j = 0; j < nb; ++j) {
      const uint32_t w = j == 0 ? wv[0] : (j == 1 ? wv[1] : (j == 2 ? wv[2] : wv[3]));
      const float e8 = e8m0_select((cur.s >> (8 * j)) & 0xffu);
      small_block<V, RESIDUAL, false>(tot, codes, scl, fp4x8_to_half8(w), e8, jl0 + j, lane, nl, G);
    }
  }
}

// Stages blocks [k0, k0 + nbk) of every row into LDS (loads unconditional,
// clamped to valid indices; stores only for real pieces).
template <int V>
__device__ __forceinline__ void small_stage(char* codes, float2* scl, const uint4* gactv, const float2* gacts,
                                            const int* s_row, const int count, const int B, const int k0,
                                            const int nbk, const int tid) {
  using L = SmallLayout<V>;
  const int per_row = nbk * 8, pieces = count * per_row;
  uint4 st[kSmallStage];
#pragma unroll
  for (int i = 0; i < kSmallStage; ++i) {
    const int c = min(tid + i * kGemmThreads, pieces - 1);
    const int t = c / per_row, rem = c - t * per_row;
    st[i] = gactv[((size_t)s_row[t] * B + k0) * 8 + rem];
  }
  const int sc = min(tid, count * nbk - 1);
  const int stt = sc / nbk, stj = sc - stt * nbk;
  const float2 sv = gacts[(size_t)s_row[stt] * B + k0 + stj];
#pragma unroll
  for (int i = 0; i < kSmallStage; ++i) {
    const int c = tid + i * kGemmThreads;
    if (c < pieces) {
      const int t = c / per_row, rem = c - t * per_row;
      const int j = rem >> 3, p = rem & 7, part = p >> 2, g = p & 3;  // piece p of the block's 128-byte record
      const int off = V == 8 ? j * 512 + (g * 8 + 2 * t + part) * 16
                             : j * L::kBlockBytes + (t >> 3) * 1024 + (g * 16 + 2 * (t & 7) + part) * 16;
      *reinterpret_cast<uint4*>(codes + off) = st[i];
    }
  }
  if (tid < count * nbk) scl[stj * L::kSlots + stt] = sv;
}

template <int V, bool RESIDUAL>
__device__ __forceinline__ void small_k_loop(float (&tot)[2][2], char* codes, float2* scl, const int* s_row,
                                             const GemmArgs& a, const uint8_t* nib, const uint8_t* wscl,
                                             const int count, const int B, const int tid, const int lane,
                                             const int nl, const int G) {
  using L = SmallLayout<V>;
  const int nqf = B >> 2, last_full = nqf > 0 ? nqf - 1 : 0;
  const uint4* gactv = reinterpret_cast<const uint4*>(a.actv);
  const float2* gacts = reinterpret_cast<const float2*>(a.acts);
  const WeightGroup tail = load_tail_group(nib, wscl, nqf, (B & 3) > 0 ? (B & 3) : 1, lane, nl);
  WeightGroup r0 = load_full_group(nib, wscl, min(0, last_full), lane, nl);
  WeightGroup r1 = load_full_group(nib, wscl, min(1, last_full), lane, nl);
  WeightGroup r2 = load_full_group(nib, wscl, min(2, last_full), lane, nl);
  const int phases = (B + L::kPhaseBlocks - 1) / L::kPhaseBlocks;
  for (int ph = 0; ph < phases; ++ph) {
    const int k0 = ph * L::kPhaseBlocks, nbk = min(L::kPhaseBlocks, B - k0);
    if (ph > 0) __syncthreads();  // every wave is done with the previous phase
    small_stage<V>(codes, scl, gactv, gacts, s_row, count, B, k0, nbk, tid);
    __syncthreads();
    const int q_begin = k0 >> 2, q_end = (k0 + nbk + 3) >> 2;
#define GOSSMX_SMALL_GROUP(QQ, SLOT)                                                                   \
  {                                                                                                    \
    const int q = (QQ);                                                                                \
    if (q < q_end) {                                                                                   \
      const bool full = q < nqf;                                                                       \
      small_group<V, RESIDUAL>(tot, codes, scl, full ? SLOT : tail, 4 * q - k0, full ? 4 : (B & 3), lane, \
                               nl, G);                                                                 \
    }                                                                                                  \
    SLOT = load_full_group(nib, wscl, min(q + kSmallRing, last_full), lane, nl); /* after last use */  \
  }
    for (int q0 = q_begin; q0 < q_begin + L::kPhaseBlocks / 4; q0 += 3) {
      GOSSMX_SMALL_GROUP(q0, r0)
      GOSSMX_SMALL_GROUP(q0 + 1, r1)
      GOSSMX_SMALL_GROUP(q0 + 2, r2)
    }
#undef GOSSMX_SMALL_GROUP
  }
}

template <int MODE, bool RESIDUAL>
__global__ __launch_bounds__(kGemmThreads, 6) void gemm_small_kernel(GemmArgs a) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int nl = lane & 15, G = lane >> 4;
  const int wi = blockIdx.y;
  if (wi >= *a.n_work_small) return;  // uniform over the work-group
  const int expert = a.work_small[2 * wi];
  const int route_base = a.bucket_off[expert];
  const int count = a.bucket_off[expert + 1] - route_base;  // 1..kSmallRows
  __shared__ __align__(16) char s_codes[kSmallCodeBytes];
  __shared__ __align__(16) float2 s_scl[kSmallSclEntries];
  __shared__ int s_row[kSmallRows];
  if (tid < kSmallRows) {
    int r = -1;
    if (tid < count) r = MODE == kGateUp ? a.route_tok[route_base + tid] : route_base + tid;
    s_row[tid] = r;
  }
  __syncthreads();

  const int rows = (int)a.w.rows, B = (int)a.w.blocks;
  const int nq = (B + 3) >> 2;
  const int tile = blockIdx.x * kWaves + wave;
  const bool tile_ok = tile < (int)a.w.tiles;
  const int row = tile * kTileRows + nl;
  const int safe_tile = tile_ok ? tile : 0;
  const uint8_t* nib = a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)safe_tile * 256 * B;
  const uint8_t* wscl = a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)safe_tile * 64 * nq;

  float b0 = 0.0f;
  if (a.bias != nullptr && tile_ok && row < rows) b0 = a.bias[(size_t)expert * a.bias_expert_stride + row];
  b0 = b0 + 0.0f;  // a -0.0 bias becomes +0.0, as the reference's first add does
  float tot[2][2] = {{b0, b0}, {b0, b0}};
  if (count <= 4) small_k_loop<8, RESIDUAL>(tot, s_codes, s_scl, s_row, a, nib, wscl, count, B, tid, lane, nl, G);
  else if (count <= 8) small_k_loop<16, RESIDUAL>(tot, s_codes, s_scl, s_row, a, nib, wscl, count, B, tid, lane, nl, G);
  else small_k_loop<32, RESIDUAL>(tot, s_codes, s_scl, s_row, a, nib, wscl, count, B, tid, lane, nl, G);
  __syncthreads();  // the activation LDS is reused by the epilogue
  gemm_epilogue<MODE, 2>(a, tot, count <= 8 ? 1 : 2, count, 0, route_base, row, tile_ok,
                         reinterpret_cast<float*>(s_codes));
}

// ---------------------------------------------------------------------------
// Weighted combine by source row and rank (cpu_runner.rs:2959-2999):
// out = 0; out += y_rank * w_rank in rank order; then bf16.

__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* y, const float* w, int top_k, int hidden,
                                                     float* out, float* trace) {
  const int r = blockIdx.y;
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= hidden) return;
  float acc = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    const size_t slot = (size_t)r * top_k + k;
    const float v = bf16_to_f32(y[slot * hidden + h]);
    acc = acc + v * w[slot];
    if (trace) trace[slot * hidden + h] = v;
  }
  out[(size_t)r * hidden + h] = bf16r(acc);
}

// ---------------------------------------------------------------------------
// Reference activation records -> GEMM operand. Q8Block {f32 scale; i8[32]}
// is 36 bytes, ResidualQ8Block {primary; residual} 72 bytes (lib.rs:732-742).

__global__ __launch_bounds__(256) void prep_records_kernel(const uint8_t* rec, int kind, int m, int blocks,
                                                          size_t row_stride, ActBuffers act) {
  const int hw = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;
  const int l32 = threadIdx.x & 31;
  if (hw >= m * blocks) return;
  const int r = hw / blocks, b = hw % blocks;
  const size_t rsz = kind == 2 ? 72 : 36;
  const uint8_t* p = rec + ((size_t)r * row_stride + b) * rsz;
  const float ps = *reinterpret_cast<const float*>(p);
  const int8_t pq = (int8_t)p[4 + l32];
  float rs = 0.0f;
  int8_t rq = 0;
  if (kind == 2) {
    rs = *reinterpret_cast<const float*>(p + 36);
    rq = (int8_t)p[40 + l32];
  }
  _Float16* dst = act.v + (((size_t)r * blocks + b) * 2) * kBlock;
  dst[l32] = (_Float16)(float)pq;
  dst[kBlock + l32] = (_Float16)(float)rq;
  if (l32 == 0) {
    float2 sc;
    sc.x = ps;
    sc.y = rs;
    reinterpret_cast<float2*>(act.s)[(size_t)r * blocks + b] = sc;
  }
}

// ---------------------------------------------------------------------------
// Layout conversion into the resident v3 layout.

__device__ __forceinline__ void v3_offsets(const TiledWeights& w, size_t e, size_t row, size_t b, size_t g,
                                           size_t* nib_off, size_t* scl_off) {
  const size_t B = w.blocks, t = row / kTileRows, n = row % kTileRows, q = b / 4, j = b % 4;
  const size_t nb = B - 4 * q < 4 ? B - 4 * q : 4;
  *nib_off = e * w.nib_stride + t * 256 * B + q * 1024 + (g * 16 + n) * nb * 4 + j * 4;
  *scl_off = e * w.scl_stride + t * 64 * ((B + 3) / 4) + q * 64 + n * 4 + j;
}

// Mxfp4MatrixView::block (lib.rs:810-851) for canonical v1 and x8 v2 data of
// one expert: fills the 16 adjacent-packed bytes and the scale byte.
__device__ void view_block(const uint8_t* data, int layout, size_t rows, size_t blocks, size_t row, size_t b,
                           uint8_t packed[16], uint8_t* scale) {
  if (layout == 1) {
    const uint8_t* p = data + (row * blocks + b) * kRecord;
    *scale = p[0];
    for (int i = 0; i < 16; ++i) packed[i] = p[1 + i];
    return;
  }
  const size_t complete = rows / 8 * 8;
  if (row < complete) {
    const size_t group = row / 8, lane = row % 8;
    const uint8_t* x8 = data + (group * blocks + b) * 136;
    uint8_t split[16];
    for (int i = 0; i < 16; ++i) split[i] = x8[8 + (i / 8) * 64 + lane * 8 + i % 8];
    *scale = x8[lane];
    // mxfp4_split_to_adjacent (lib.rs:919-928): split byte i = code(i) | code(i+16) << 4.
    for (int i = 0; i < 16; ++i) {
      const int c0 = 2 * i, c1 = 2 * i + 1;
      const uint8_t lo = c0 < 16 ? (split[c0] & 0x0f) : (split[c0 - 16] >> 4);
      const uint8_t hi = c1 < 16 ? (split[c1] & 0x0f) : (split[c1 - 16] >> 4);
      packed[i] = (uint8_t)(lo | (hi << 4));
    }
    return;
  }
  const uint8_t* p = data + (rows / 8) * blocks * 136 + ((row - complete) * blocks + b) * kRecord;
  *scale = p[0];
  for (int i = 0; i < 16; ++i) packed[i] = p[1 + i];
}

__device__ __forceinline__ void store_v3(const TiledWeights& w, size_t e, size_t row, size_t b, const uint8_t packed[16],
                                         uint8_t scale) {
  for (size_t g = 0; g < 4; ++g) {
    size_t no, so;
    v3_offsets(w, e, row, b, g, &no, &so);
    const uint32_t d = (uint32_t)packed[4 * g] | ((uint32_t)packed[4 * g + 1] << 8) |
                       ((uint32_t)packed[4 * g + 2] << 16) | ((uint32_t)packed[4 * g + 3] << 24);
    *reinterpret_cast<uint32_t*>(w.nib + no) = d;
    if (g == 0) w.scl[so] = scale;
  }
}

__global__ void repack_kernel(const uint8_t* src, int layout, TiledWeights w) {
  const size_t per_expert = w.rows * w.blocks;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * per_expert) return;
  const size_t e = i / per_expert, rb = i % per_expert, row = rb / w.blocks, b = rb % w.blocks;
  uint8_t packed[16], scale;
  view_block(src + e * per_expert * kRecord, layout, w.rows, w.blocks, row, b, packed, &scale);
  store_v3(w, e, row, b, packed, scale);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t stream_hash(uint64_t seed, uint64_t stream, uint64_t index) {
  return splitmix64(splitmix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) + index);
}

__global__ void generate_kernel(uint64_t seed, uint64_t stream, TiledWeights w) {
  const size_t per_expert = w.rows * w.blocks;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * per_expert) return;
  const size_t e = i / per_expert, rb = i % per_expert, row = rb / w.blocks, b = rb % w.blocks;
  const uint64_t h0 = stream_hash(seed, stream, 2 * i), h1 = stream_hash(seed, stream, 2 * i + 1);
  uint8_t packed[16];
  for (int j = 0; j < 8; ++j) packed[j] = (uint8_t)(h0 >> (8 * j));
  for (int j = 0; j < 8; ++j) packed[8 + j] = (uint8_t)(h1 >> (8 * j));
  store_v3(w, e, row, b, packed, (uint8_t)(119 + (h1 >> 61) % 5));
}

__global__ void export_kernel(TiledWeights w, uint8_t* dst) {
  const size_t per_expert = w.rows * w.blocks;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * per_expert) return;
  const size_t e = i / per_expert, rb = i % per_expert, row = rb / w.blocks, b = rb % w.blocks;
  uint8_t* p = dst + i * kRecord;
  for (size_t g = 0; g < 4; ++g) {
    size_t no, so;
    v3_offsets(w, e, row, b, g, &no, &so);
    const uint32_t d = *reinterpret_cast<const uint32_t*>(w.nib + no);
    for (int k = 0; k < 4; ++k) p[1 + 4 * g + k] = (uint8_t)(d >> (8 * k));
    if (g == 0) p[0] = w.scl[so];
  }
}

// Padding rows of the last tile: zero codes, scale 127.
__global__ void fill_padding_kernel(TiledWeights w) {
  const size_t pad_rows = w.tiles * kTileRows - w.rows;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * pad_rows * w.blocks) return;
  const size_t e = i / (pad_rows * w.blocks), rb = i % (pad_rows * w.blocks);
  const size_t row = w.rows + rb / w.blocks, b = rb % w.blocks;
  const uint8_t zero[16] = {0};
  store_v3(w, e, row, b, zero, 127);
}

__global__ void clear_ints_kernel(int* p, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Lane-layout self-test of the two gfx950 builtins the GEMM relies on.
// out[0..7]: v_cvt_scalef32_pk_f16_fp4 of codes 0..7 (bytes 0x10 0x32 0x54 0x76).
// out[8 + 4 * lane + r]: D of a 16x16x32 f16 MFMA with A[i][k] = (k == i) and
// B[k][j] = 10 k + j, expected 10 * (4 * (lane / 16) + r) + lane % 16.
// out[264..271]: codes 0..7 converted with scale 2^-4.
__global__ void selftest_kernel(float* out) {
  const int lane = threadIdx.x;
  const half8 w = fp4x8_to_half8(0x76543210u);
  if (lane == 0)
    for (int i = 0; i < 8; ++i) out[i] = (float)w[i];
  half8 av, bv;
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * (lane >> 4) + e;
    av[e] = (_Float16)((k == (lane & 15)) ? 1.0f : 0.0f);
    bv[e] = (_Float16)(float)(10 * k + (lane & 15));
  }
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, zero, 0, 0, 0);
  for (int r = 0; r < 4; ++r) out[8 + 4 * lane + r] = d[r];
  // out[264..271]: the scaled conversion with E8M0 byte 123 (2^-4).
  const half8 ws = fp4x8_to_half8_scaled(0x76543210u, __uint_as_float(123u << 23));
  if (lane == 0)
    for (int i = 0; i < 8; ++i) out[264 + i] = (float)ws[i];
}

// ---------------------------------------------------------------------------
// Launchers.

static inline unsigned grid1d(size_t n, unsigned block) { return (unsigned)((n + block - 1) / block); }

hipError_t launch_route(const RouteArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(route_kernel, dim3(a.m), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_dispatch(const DispatchArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_gemm(GemmMode mode, const GemmArgs& a, int grid_work, hipStream_t stream) {
  const dim3 grid((unsigned)((a.w.tiles + kWaves - 1) / kWaves), (unsigned)grid_work);
  const dim3 block(kGemmThreads);
  if (a.residual) {
    switch (mode) {
      case kPlain: hipLaunchKernelGGL((gemm_kernel<kPlain, true>), grid, block, 0, stream, a); break;
      case kGateUp: hipLaunchKernelGGL((gemm_kernel<kGateUp, true>), grid, block, 0, stream, a); break;
      case kDown: hipLaunchKernelGGL((gemm_kernel<kDown, true>), grid, block, 0, stream, a); break;
    }
  } else {
    if (mode != kPlain) return hipErrorInvalidValue;  // the MoE block always runs residual-Q8
    hipLaunchKernelGGL((gemm_kernel<kPlain, false>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_small(GemmMode mode, const GemmArgs& a, int grid_work, hipStream_t stream) {
  if (!a.residual || mode == kPlain) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.w.tiles + kWaves - 1) / kWaves), (unsigned)grid_work);
  const dim3 block(kGemmThreads);
  if (mode == kGateUp) hipLaunchKernelGGL((gemm_small_kernel<kGateUp, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((gemm_small_kernel<kDown, true>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t* y, const float* weights, int m, int top_k, int hidden, float* out,
                          float* trace_down, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(grid1d(hidden, 256), m), dim3(256), 0, stream, y, weights, top_k, hidden,
                     out, trace_down);
  return hipGetLastError();
}

hipError_t launch_prep_records(const uint8_t* records, int kind, size_t m, size_t blocks, size_t row_stride,
                               ActBuffers act, int* /*err*/, hipStream_t stream) {
  hipLaunchKernelGGL(prep_records_kernel, dim3(grid1d(m * blocks * 32, 256)), dim3(256), 0, stream, records, kind,
                     (int)m, (int)blocks, row_stride, act);
  return hipGetLastError();
}

hipError_t launch_repack(const uint8_t* src, int layout, TiledWeights w, hipStream_t stream) {
  hipLaunchKernelGGL(repack_kernel, dim3(grid1d(w.experts * w.rows * w.blocks, 256)), dim3(256), 0, stream, src,
                     layout, w);
  return hipGetLastError();
}

hipError_t launch_generate(uint64_t seed, uint64_t stream_id, TiledWeights w, hipStream_t stream) {
  hipLaunchKernelGGL(generate_kernel, dim3(grid1d(w.experts * w.rows * w.blocks, 256)), dim3(256), 0, stream, seed,
                     stream_id, w);
  return hipGetLastError();
}

hipError_t launch_export(TiledWeights w, uint8_t* dst, hipStream_t stream) {
  hipLaunchKernelGGL(export_kernel, dim3(grid1d(w.experts * w.rows * w.blocks, 256)), dim3(256), 0, stream, w, dst);
  return hipGetLastError();
}

hipError_t launch_fill_tiled_padding(TiledWeights w, hipStream_t stream) {
  const size_t n = w.experts * (w.tiles * kTileRows - w.rows) * w.blocks;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_padding_kernel, dim3(grid1d(n, 256)), dim3(256), 0, stream, w);
  return hipGetLastError();
}

hipError_t launch_clear_ints(int* p, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(clear_ints_kernel, dim3(grid1d(n, 256)), dim3(256), 0, stream, p, n);
  return hipGetLastError();
}

hipError_t launch_build_sigmoid_table(uint16_t* tab, hipStream_t stream) {
  hipLaunchKernelGGL(build_sigmoid_table_kernel, dim3(256), dim3(256), 0, stream, tab);
  return hipGetLastError();
}

hipError_t launch_selftest(float* out, hipStream_t stream) {
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError();
}

}  // namespace gossmx
